"""OCP e4m3 activations for the fp8 kNN-conv path (no counterpart in the reference).

``quantize_e4m3`` runs the library's HIP quantizer (``fovi_quantize_e4m3``):
per-tensor scale ``amax * headroom / 448`` computed on the device (no host
round trip), values ``x / scale`` rounded to nearest even into a channels-last
``[B, N, C]`` e4m3 buffer. ``headroom`` (a power of two) keeps sums of up to
that many quantized values below the e4m3 maximum 448; the kNN-conv layer
passes its largest slot count rounded up to a power of two, because its fp8
kernel re-rounds each multi-neighbour slot sum to e4m3.
"""
from __future__ import annotations

import math
from typing import NamedTuple, Optional

import torch

from .. import _lib

__all__ = ["Fp8Activations", "quantize_e4m3", "headroom_for"]


class Fp8Activations(NamedTuple):
    """``data``: float8_e4m3fn ``[B, C, N]`` view of channels-last storage; ``scale``: fp32 ``[1]``
    on the same device, so that ``x ~= data.float() * scale``."""
    data: torch.Tensor
    scale: torch.Tensor

    def dequantize(self) -> torch.Tensor:
        return self.data.float() * self.scale


def headroom_for(max_count: int) -> float:
    """Smallest power of two >= max_count (>= 1)."""
    return float(2 ** max(0, math.ceil(math.log2(max(1, int(max_count))))))


def quantize_e4m3(x: torch.Tensor, headroom: float = 1.0, scale: Optional[torch.Tensor] = None) -> Fp8Activations:
    """Quantizes ``x [B, C, N]`` (fp32 or bf16, any strides) to channels-last e4m3.

    With ``scale`` (a 1-element fp32 device tensor, e.g. from calibration) the
    amax pass is skipped and that scale is used.
    """
    _lib.require_device(x)
    if x.dim() != 3:
        raise ValueError(f"quantize_e4m3: expected [B, C, N], got {tuple(x.shape)}")
    if x.dtype not in (torch.float32, torch.bfloat16):
        raise TypeError(f"quantize_e4m3: unsupported dtype {x.dtype}")
    b, c, n = x.shape
    q = torch.empty(b, n, c, dtype=torch.float8_e4m3fn, device=x.device)
    qv = q.transpose(1, 2)
    a = _lib.QuantizeArgs()
    a.x = x.data_ptr(); a.x_dtype = _lib.dtype_code(x.dtype)
    a.batch, a.channels, a.points = b, c, n
    a.x_stride[:] = list(x.stride())
    a.q = q.data_ptr(); a.q_stride[:] = list(qv.stride())
    a.headroom = float(headroom)
    work = torch.empty(2, dtype=torch.float32, device=x.device)
    if scale is not None:
        _lib.require_device(scale)
        scale = scale.to(torch.float32).reshape(1).contiguous()
        a.scale_in = scale.data_ptr()
        out_scale = scale
    else:
        a.amax_work = work[0:1].data_ptr(); a.scale_out = work[1:2].data_ptr()
        out_scale = work[1:2]
    lib = _lib.load()
    _lib.check(lib.fovi_quantize_e4m3(a, _lib.stream_handle(x.device)), "fovi_quantize_e4m3")
    return Fp8Activations(qv, out_scale)
