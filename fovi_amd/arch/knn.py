"""kNN-convolution layer, drop-in for the reference ``fovi.arch.knn.KNNConvLayer``.

Same constructor, parameters (``weight [C_out, C_in*V]``, ``bias [C_out]``,
so state dicts load unchanged) and attributes (``k``/``_k``, ``knn_indices``,
``knn_indices_pad_token``, ``ref_coords``, ``ref_grid_size``, ``local_rf``,
``in_coords``/``out_coords``) as the reference (``fovi/arch/knn.py:401-719``).

The forward is one HIP launch (``fovi_knnconv_fwd``): gather, slot sum and
GEMM fused, with neighbour lists in slot-major CSR form in HBM. Input
``[B, C_in, N_in]`` may have any strides; a channels-last view (a previous
layer's output) takes the vectorised path. The output is ``[B, C_out, N_out]``
as a transposed view of channels-last ``[B, N_out, C_out]`` storage, which is
also what the reference returns (``F.linear(...).transpose(1,2)``,
``knn.py:555``).

Compute dtype: bf16 inputs, or any input under ``torch.autocast('cuda',
dtype=torch.bfloat16)``, run the bf16 MFMA kernel with fp32 accumulation and
return bf16 (the reference's autocast behaviour); fp32 inputs run the fp32
kernel. ``Fp8Activations`` inputs (``layer.quantize_input``), or any input
when ``layer.fp8`` is set, run the e4m3 MFMA kernel (per-tensor activation
scale, per-output-channel weight scale ``amax|W[o]|/448``, fp32 accumulation,
bf16 output); the reference has no fp8 path.

Backward (autograd through ``_KnnConvFn``): the slot sums again
(``fovi_knnconv_slotsum``) for ``dW = dy^T a``, ``dy W`` as a library GEMM and
its transposed gather (``fovi_knnconv_bwd_x``, over the inverse neighbour
table, no atomics) for ``dx``; fp32 and bf16 inputs. The fp8 path has no
backward.
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn as nn
import torch.nn.functional as F
from einops import rearrange

from .. import _lib
from ..sensing.coords import SamplingCoords
from . import knn_tables as T
from .fp8 import Fp8Activations, headroom_for, quantize_e4m3

__all__ = [
    "KNNBaseLayer",
    "KNNConvLayer",
    "KNNPoolingLayer",
    "KNN_CONV_REGISTRY",
    "get_knn_conv_layer",
    "get_in_out_coords",
    "register_with_reference",
]

_KCHUNK = 64  # reduction chunk of the MFMA kernel; packed weights are padded to it

# Attributes of a sensor point set the kNN layers read (those of the reference's
# SamplingCoords, fovi/sensing/coords.py:21-66); cartesian_pad_coords (absent on the
# reference's one-point sets) and cortical_pad_coords (isotropic styles only) are optional.
_COORD_ATTRS = ("shape", "style", "cartesian", "cortical")


def _check_coords(coords, what):
    """Accepts any object with the reference ``SamplingCoords`` attributes the layers read
    (this package's ``SamplingCoords``, the reference's own, or a plain namespace)."""
    missing = [a for a in _COORD_ATTRS if not hasattr(coords, a)]
    if missing:
        raise TypeError(f"{what} lacks the SamplingCoords attributes {missing}")


def _pad_coords(coords, name="cartesian_pad_coords"):
    """The point set's pad ring in the space of ``cartesian`` or ``cortical`` (empty when it
    has none)."""
    pads = getattr(coords, name, None)
    if pads is None:
        like = coords.cartesian if name == "cartesian_pad_coords" else coords.cortical
        return torch.zeros(0, like.shape[1], dtype=like.dtype)
    return pads.cpu()


class KNNBaseLayer:
    """Neighbour search shared by kNN layers (reference ``knn.py:14-224``)."""

    def _compute_knns(self, batch_size=None):
        """(indices ``[k, N_out]``, distances ``[k, N_out]``) of the k nearest inputs per output
        (reference ``knn.py:23-152``); indices >= N_in are points of the input's pad ring.

        Log-polar sensors search the wrapped 2-D log-polar lattice without pads; isotropic
        sensors search the 3-D cortical manifold over points and pad ring
        (``sample_cortex=True``); ``sample_cortex=False`` searches the visual field over
        points and pad ring. Output batches are sized as the reference sizes them (pads
        counted, at most 5e8 pairs per batch)."""
        if self.sample_cortex == "geodesic":
            raise NotImplementedError("geodesic neighbourhoods need pygeodesic, which is not available")
        in_c, out_c = self.in_coords, self.out_coords
        pads = _pad_coords(in_c)
        n_out = out_c.shape[0]
        if batch_size is None:
            batch_size = T.default_batch(in_c.shape[0] + pads.shape[0], n_out)
        batch_size = min(batch_size, n_out)
        self.sample_coords_cart = torch.cat([in_c.cartesian.cpu(), pads], 0)
        if not self.sample_cortex:
            self.sample_coords = self.sample_coords_cart
            return self._knn_euclidean(out_c.cartesian.cpu(), batch_size)
        if in_c.style in ("image", "logpolar"):
            assert out_c.style == in_c.style
            if self._gpu_tables(in_c.shape[0]):
                idx, dist, src = T.knn_logpolar_device(in_c.cortical.cpu(), out_c.cortical.cpu(), self._k,
                                                       self.device)
            else:
                idx, dist, src = T.knn_logpolar(in_c.cortical.cpu(), out_c.cortical.cpu(), self._k, batch_size)
            self.sample_coords = src
            return idx, dist
        if in_c.cortical is None:
            raise ValueError(f"style {in_c.style!r} has no cortical coordinates: use sample_cortex=False")
        self.sample_coords = torch.cat([in_c.cortical.cpu(), _pad_coords(in_c, "cortical_pad_coords")], 0)
        return self._knn_euclidean(out_c.cortical.cpu(), batch_size)

    def _knn_euclidean(self, out_pts, batch_size):
        """``cdist`` + ``topk`` neighbours of ``out_pts`` among ``self.sample_coords``: the GPU
        scan with host-verified candidates for a CUDA layer where it applies
        (``knn_tables.knn_euclidean_device``, the host's results bit for bit), else the host."""
        if self._on_gpu() and T.knn_euclidean_device_ok(self.sample_coords, self._k) \
                and out_pts.dtype == torch.float32:
            return T.knn_euclidean_device(self.sample_coords, out_pts, self._k, self.device, batch_size)
        return T.knn_euclidean(self.sample_coords, out_pts, self._k, batch_size)

    def _on_gpu(self):
        dev = torch.device(self.device) if not isinstance(self.device, torch.device) else self.device
        return dev.type == "cuda" and torch.cuda.is_available()

    def _compute_all_distances(self):
        """Distances ``[N_in + P, N_out]`` between every input point (pad ring included) and
        every output point in one ``cdist`` call: cortical for ``sample_cortex=True``
        (isotropic sensors), visual field for ``sample_cortex=False`` (reference
        ``knn.py:155-224``, non-geodesic branches)."""
        if self.sample_cortex == "geodesic":
            raise NotImplementedError("geodesic distances need pygeodesic, which is not available")
        in_c, out_c = self.in_coords, self.out_coords
        pads = _pad_coords(in_c)
        self.sample_coords_cart = torch.cat([in_c.cartesian.cpu(), pads], 0)
        if not self.sample_cortex:
            self.sample_coords = self.sample_coords_cart
            return torch.cdist(self.sample_coords, out_c.cartesian.cpu())
        if in_c.style not in ("isotropic", "isotropic_fixn"):
            raise ValueError(f"all-pairs cortical distances need the isotropic manifold, not {in_c.style!r}")
        self.sample_coords = torch.cat([in_c.cortical.cpu(), _pad_coords(in_c, "cortical_pad_coords")], 0)
        return torch.cdist(self.sample_coords, out_c.cortical.cpu())

    def _gpu_tables(self, n_in):
        """Whether the neighbour search runs on the GPU (``knn_tables.knn_logpolar_device``, the
        host's results bit for bit): a CUDA layer where the GPU search applies."""
        return self._on_gpu() and T.knn_logpolar_device_ok(n_in, self._k)


class _KnnConvFn(torch.autograd.Function):
    """Forward ``fovi_knnconv_fwd``; backward = the slot sums again (``fovi_knnconv_slotsum``)
    and the transposed gather (``fovi_knnconv_bwd_x``) around two library GEMMs."""

    @staticmethod
    def forward(ctx, x, layer, weight, bias, activation=None):
        y = layer._launch(x, activation)
        ctx.layer, ctx.activation, ctx.has_bias = layer, activation, bias is not None
        ctx.save_for_backward(x, weight, y if activation == "relu" else None)
        return y

    @staticmethod
    def backward(ctx, dy):
        x, weight, y = ctx.saved_tensors
        layer = ctx.layer
        if ctx.activation == "relu":
            dy = dy * (y > 0)
        dx, dw = layer._backward(x, weight, dy, ctx.needs_input_grad[0], ctx.needs_input_grad[2])
        db = dy.sum(dim=(0, 2)).to(torch.float32) if ctx.has_bias and ctx.needs_input_grad[3] else None
        return dx, None, dw, db, None


class KNNConvLayer(nn.Module, KNNBaseLayer):
    """K-nearest-neighbour convolution on a sensor point cloud (HIP forward)."""

    def __init__(self, in_channels, out_channels, k, in_coords, out_coords,
                 device="cuda",
                 arch_flag="",
                 sample_cortex=True,
                 bias=False,
                 ref_frame_side_length=None,
                 batch_size=None,
                 ):
        super().__init__()
        _check_coords(in_coords, "in_coords")
        _check_coords(out_coords, "out_coords")
        self.in_channels = in_channels
        self.out_channels = out_channels
        self.in_coords = in_coords
        self.out_coords = out_coords
        self.device = device
        self.arch_flag = arch_flag
        self.sample_cortex = sample_cortex
        self.ref_frame_side_length = ref_frame_side_length
        self.batch_size = batch_size

        n_in = in_coords.shape[0]
        self.k = torch.minimum(torch.tensor(k), torch.tensor(n_in))
        self._k = int(self.k.item())

        knn_indices, knn_distances = self._compute_knns(batch_size)
        self._setup(knn_indices, knn_distances, bias)

    @classmethod
    def from_tables(cls, in_channels, out_channels, in_coords, out_coords, knn_indices, local_rf=None,
                    slots=None, device="cuda", arch_flag="", sample_cortex=True, bias=False,
                    ref_frame_side_length=None, ref_coords=None, ref_grid_size=None, batch_size=None):
        """A kernel-backed layer on neighbour and ref-slot tables computed elsewhere, such as
        a reference layer's geodesic ones (``knn.py:59-99``, pygeodesic), which this package
        does not compute.

        ``knn_indices [k, N_out]``: input indices per output point; entries >= N_in (the pad
        ring) and < 0 (the -1 padding of a partition, ``knnvit.py:194-198``) carry no input.
        The slots come as the reference's one-hot ``local_rf [N_out, k, V]`` or as indices
        ``slots [N_out, k]``. The ref grid is ``ref_coords [V, 2]`` when given, else the one
        ``compute_reference_coords`` builds from k, ``arch_flag`` and
        ``ref_frame_side_length``. Parameters are initialised as the constructor does."""
        _check_coords(in_coords, "in_coords")
        _check_coords(out_coords, "out_coords")
        knn_indices = torch.as_tensor(knn_indices).detach().cpu()
        if knn_indices.dim() != 2 or knn_indices.dtype.is_floating_point or knn_indices.dtype == torch.bool:
            raise ValueError(f"knn_indices must be an integer [k, N_out] table, got {tuple(knn_indices.shape)} "
                             f"{knn_indices.dtype}")
        knn_indices = knn_indices.to(torch.int64)
        k, n_out = knn_indices.shape
        if n_out != out_coords.shape[0]:
            raise ValueError(f"knn_indices has {n_out} columns for {out_coords.shape[0]} output points")
        n_in = in_coords.shape[0]
        n_pad = _pad_coords(in_coords).shape[0]
        if knn_indices.numel() and int(knn_indices.max()) >= n_in + max(n_pad, 1):
            raise ValueError(f"knn_indices reaches {int(knn_indices.max())}, beyond the {n_in} points and "
                             f"{n_pad} pad points of in_coords")
        self = cls.__new__(cls)
        nn.Module.__init__(self)
        self.in_channels, self.out_channels = in_channels, out_channels
        self.in_coords, self.out_coords = in_coords, out_coords
        self.device, self.arch_flag, self.sample_cortex = device, arch_flag, sample_cortex
        self.ref_frame_side_length, self.batch_size = ref_frame_side_length, batch_size
        self.k = torch.tensor(k)
        self._k = k
        if ref_coords is not None:
            ref_coords = torch.as_tensor(ref_coords).detach()
            if ref_coords.dim() != 2:
                raise ValueError(f"ref_coords must be [V, 2], got {tuple(ref_coords.shape)}")
        else:
            self.compute_reference_coords(arch_flag)
            ref_coords, ref_grid_size = self.ref_coords, self.ref_grid_size
        n_ref = ref_coords.shape[0]
        if (local_rf is None) == (slots is None):
            raise ValueError("give exactly one of local_rf (one-hot [N_out, k, V]) and slots ([N_out, k])")
        if local_rf is not None:
            rf = torch.as_tensor(local_rf).detach().cpu()
            if tuple(rf.shape) != (n_out, k, n_ref):
                raise ValueError(f"local_rf must be [N_out, k, V] = {(n_out, k, n_ref)}, got {tuple(rf.shape)}")
            if not (((rf == 0) | (rf == 1)).all() and (rf.sum(2) == 1).all()):
                raise ValueError("local_rf must be one-hot over its last axis (one ref slot per neighbour)")
            slots = rf.argmax(2)
        slots = torch.as_tensor(slots).detach().cpu().to(torch.int64)
        if tuple(slots.shape) != (n_out, k):
            raise ValueError(f"slots must be [N_out, k] = {(n_out, k)}, got {tuple(slots.shape)}")
        if slots.numel() and (int(slots.min()) < 0 or int(slots.max()) >= n_ref):
            raise ValueError(f"slots must index the {n_ref} ref points")
        self._setup(knn_indices, None, bias, param_device="cpu", slots=slots, ref_coords=ref_coords,
                    ref_grid_size=ref_grid_size)
        return self

    @classmethod
    def from_reference(cls, layer, device=None):
        """The kernel-backed twin of a reference ``KNNConvLayer`` (or patch embedding) ``layer``:
        its coords objects, neighbour table, one-hot ``local_rf``, ref grid, flags, ``weight``
        and ``bias`` (copied), and ``transposed`` where it has one (``knnvit.py:17-290``).
        This is how a layer whose tables this package cannot compute (geodesic neighbourhoods)
        runs on the kernels; ``device`` defaults to the reference layer's."""
        dev = getattr(layer, "device", "cuda") if device is None else device
        new = cls.from_tables(layer.in_channels, layer.out_channels, layer.in_coords, layer.out_coords,
                              layer.knn_indices, local_rf=layer.local_rf, device=dev,
                              arch_flag=getattr(layer, "arch_flag", ""),
                              sample_cortex=getattr(layer, "sample_cortex", True), bias=layer.bias is not None,
                              ref_frame_side_length=getattr(layer, "ref_frame_side_length", None),
                              ref_coords=layer.ref_coords, ref_grid_size=getattr(layer, "ref_grid_size", None),
                              batch_size=getattr(layer, "batch_size", None))
        if tuple(layer.weight.shape) != tuple(new.weight.shape):
            raise ValueError(f"reference weight {tuple(layer.weight.shape)} != {tuple(new.weight.shape)}")
        with torch.no_grad():
            new.weight.copy_(layer.weight.detach())
            if new.bias is not None:
                new.bias.copy_(layer.bias.detach())
        for attr in ("transposed", "knn_pad_index_token_val", "knn_pad_token_val"):
            if hasattr(layer, attr):
                setattr(new, attr, getattr(layer, attr))
        return new

    def _setup(self, knn_indices, knn_distances, bias, param_device=None, slots=None, ref_coords=None,
               ref_grid_size=None):
        """Pad tokens, ref grid, parameters (created on ``param_device``, default the layer's
        device, then moved there), ref slots and device tables of a neighbour table
        ``[k, N_out]`` whose entries >= N_in (pad ring) or < 0 (padding of a partition) carry
        no input (reference ``knn.py:445-471``). Given ``slots [N_out, k]`` (and the ref grid
        ``ref_coords [V, 2]`` they index), those are used instead of computed."""
        n_in, device = self.in_coords.shape[0], self.device
        self.knn_indices_pad_mask = (knn_indices >= n_in) | (knn_indices < 0)
        pad_token = knn_indices.clone()
        pad_token[self.knn_indices_pad_mask] = n_in
        self.knn_indices_batch_cache = pad_token

        if ref_coords is None:
            self.compute_reference_coords(self.arch_flag)
        else:
            self.ref_coords = ref_coords.to(device)
            self.ref_grid_size = (int(ref_grid_size) if ref_grid_size is not None
                                  else int(round(ref_coords.shape[0] ** 0.5)))
        n_ref = self.ref_coords.shape[0]
        pdev = device if param_device is None else param_device
        self.weight = nn.Parameter(torch.empty(self.out_channels, self.in_channels * n_ref, device=pdev))
        if bias:
            self.bias = nn.Parameter(torch.empty(self.out_channels, device=pdev))
        else:
            self.register_parameter("bias", None)
        self._init_conv_like()
        if param_device is not None:
            self.weight.data = self.weight.data.to(device)
            if self.bias is not None:
                self.bias.data = self.bias.data.to(device)

        self.slots = self.compute_local_rf_slots(knn_indices) if slots is None else slots
        self.knn_indices = knn_indices.to(device)
        self.knn_distances = None if knn_distances is None else knn_distances.to(device)
        self.knn_indices_pad_token = pad_token.to(device)
        self.knn_indices_pad_mask = self.knn_indices_pad_mask.to(device)
        self._init_tables(knn_indices, self.slots, n_in, n_ref, device)

    def _init_tables(self, knn_indices, slots, n_in, n_ref, device):
        """Device tables of the forward kernels from the kNN table ``[k, N_out]`` (indices >=
        n_in are pad tokens) and the slots ``[N_out, k]``, and the per-layer switches."""
        slot_ptr, nbr_sorted = T.csr_tables(knn_indices, slots, n_in, n_ref)
        self.register_buffer("slot_ptr", slot_ptr.to(device), persistent=False)
        self.register_buffer("nbr_sorted", nbr_sorted.to(device), persistent=False)
        tiles = T.direct_tables(knn_indices, slots, n_in, n_ref)
        self._max_span = 0
        self._zero_row = 0
        for name, t in zip(("tile_lo", "tile_span", "tile_ent", "tile_nbr", "tile_coll", "tile_coll_n"),
                           tiles[:6] if tiles is not None else (None,) * 6):
            self.register_buffer(name, None if t is None else t.to(device), persistent=False)
        if tiles is not None:
            self._max_span = int(tiles[1].max())
            self._zero_row = tiles[6]
        # tables of the wide-layer (fragment-order weight) kernel, in a slot-visit order
        # that spreads the heavy slots' collision sums over the stream
        self._direct_tables = tiles
        self._packed = {}
        order = None
        if tiles is not None:
            order = T.stream_slot_order(T.slot_stream_units(tiles), ahead=T.wide_tiles_of(tiles))
        self.set_slot_order(order)
        # tables of the fused few-channel kernel (c_in <= 8): the first geometry whose LDS fits
        self.set_few_channel_geometry(None, knn_indices, slots, n_in, n_ref, device)
        # few-channel layers: the fused kernel when its tables fit (False: the slot sums through
        # a workspace and a dense GEMM, or the single-pass kernel)
        self.few_channel_fused = True
        # few-channel layers given view-major input rows (padded_input(..., view_major=True)):
        # the view-major kernel (False: the two-pass or single-pass paths); its tables are
        # built on first use
        self.view_major_kernel = True
        self._vm = None
        # slot-sum headroom of the fp8 path: the largest neighbour count of a slot
        self._max_slot_count = int((slot_ptr & 0xFFFF).max()) if slot_ptr.numel() else 1
        # quantize every input to e4m3 and run the fp8 kernel
        self.fp8 = False
        # few-channel bf16 layers: slot sums through a workspace, then a dense GEMM
        # (False: the single fused kernel, which needs no workspace)
        self.two_pass_few_channels = True
        # input gradient as a kNN-conv forward over the inverse tables (False: a GEMM into
        # [B * N_out, V * C] and the inverse-table gather, fovi_knnconv_bwd_x)
        self.dx_by_transposed_conv = True
        # bf16 weight gradient by fovi_knnconv_dw (False: the slot sums and a library GEMM)
        self.dw_fused = True
        # its work split: output points per pair segment, images per workgroup
        self.dw_chunk = 1 << 30
        self.dw_images_per_group = 1
        # wide layers (bf16 c_in % 32 == 0 or e4m3 c_in % 64 == 0, c_out filling >= 3/4 of its
        # 256-channel tiles, tables within LDS): weights in MFMA-fragment order for the
        # 256 x 256-tile kernel (False: the row-packed kernels)
        self.mfma_weights = True

    def set_few_channel_geometry(self, geometries=None, knn_indices=None, slots=None, n_in=None, n_ref=None,
                                 device=None):
        """Tables of the fused few-channel kernel (layers with c_in <= 8) for the first of
        ``geometries`` (``(tile, threads, chunk)`` tuples; default ``knn_tables.FC_GEOMETRIES``)
        whose tile fits the LDS; none fits: the layer takes the other few-channel paths."""
        self._fc = None
        cp = 4 if self.in_channels <= 4 else (8 if self.in_channels <= 8 else None)
        if knn_indices is None:
            knn_indices, slots = self.knn_indices.cpu(), self.slots
            n_in, n_ref, device = self.in_coords.shape[0], self.ref_coords.shape[0], self.weight.device
        fc = None
        if cp is not None:
            k_pad = -(-cp * n_ref // _KCHUNK) * _KCHUNK
            for tile, threads, chunk in (T.FC_GEOMETRIES if geometries is None else geometries):
                fc = T.few_channel_tables(knn_indices, slots, n_in, n_ref, cp, k_pad, tile, threads, chunk)
                if fc is not None and T.few_channel_lds_bytes(fc, self.out_channels, cp) < (1 << 30):
                    break
                fc = None
        for name, field in (("fc_lo", "lo"), ("fc_span", "span"), ("fc_item", "item"), ("fc_comb", "comb"),
                            ("fc_comb_off", "comb_off")):
            self.register_buffer(name, None if fc is None else getattr(fc, field).to(device), persistent=False)
        if fc is not None:
            self._fc = (fc.tile, fc.zero_row, fc.pmax, fc.pairs, fc.threads, fc.chunk)

    # -- setup ---------------------------------------------------------------
    def _init_conv_like(self):
        nn.init.kaiming_normal_(self.weight)
        if self.bias is not None:
            nn.init.zeros_(self.bias)

    def compute_reference_coords(self, arch_flag):
        """Square ref grid of side ``ref_frame_side_length`` or ceil(sqrt(k)), doubled for a
        flag containing 'doubleres' (``knn.py:559-597``). Of the flags its docstring names only
        'doubleres' changes the grid there: 'fovref' and 'circref' give the square grid, here
        as in the reference."""
        if self.ref_frame_side_length is not None:
            assert not len(arch_flag), "self.ref_frame_side_length is incompatible with use of arch_flag"
            ref, side = T.reference_grid(self._k, side_length=self.ref_frame_side_length)
        else:
            ref, side = T.reference_grid(self._k, doubleres="doubleres" in arch_flag)
        self.ref_grid_size = side
        self.ref_coords = ref.to(self.device, dtype=getattr(self.in_coords, "dtype", torch.float32))

    def compute_local_rf_slots(self, knn_indices):
        """Ref slot ``[N_out, k]`` of every neighbour (reference ``knn.py:599-647``), on the CPU;
        for a CUDA layer the per-neighbour arithmetic runs on the GPU and only the points
        it flags as near a tie are recomputed here (``knn_tables.local_rf_slots_device``,
        the same slots bit for bit)."""
        ref = self.ref_coords.cpu()
        if not self.sample_cortex:
            return T.visual_rf_slots(knn_indices, self.sample_coords, ref)
        args = (knn_indices, self.sample_coords, self.sample_coords_cart, self.out_coords.cortical.cpu(),
                self.out_coords.cartesian.cpu(), ref)
        if self._on_gpu() and T.local_rf_slots_device_ok(knn_indices, self.sample_coords, ref):
            slots, self.slots_recomputed = T.local_rf_slots_device(*args, device=self.device)
            return slots
        return T.local_rf_slots(*args)

    @property
    def local_rf(self):
        """One-hot ``[N_out, k, V]`` neighbour -> ref-slot map (built on demand)."""
        return T.slots_to_one_hot(self.slots, self.ref_coords.shape[0]).to(self.weight.device)

    def compute_local_rf(self):
        return self.local_rf

    def _apply_local_rf_to_weights(self):
        weights = rearrange(self.weight, "d (c v) -> d c v", c=self.in_channels, v=self.ref_coords.shape[0])
        return torch.einsum("dcv,nkv->ncdk", weights, self.local_rf)

    # -- weights -------------------------------------------------------------
    def _packed_weight(self, dtype, c_slot=None):
        """Packed weight (slot-major, ``c_slot`` channels per slot), cached per weight version."""
        c_slot = self.in_channels if c_slot is None else c_slot
        w = self.weight
        key = (dtype, c_slot, w._version, w.data_ptr())
        hit = self._packed.get((dtype, c_slot))
        if hit is not None and hit[0] == key:
            return hit[1]
        n_ref = self.ref_coords.shape[0]
        k_pad = -(-c_slot * n_ref // _KCHUNK) * _KCHUNK
        src = w.detach().to(torch.float32).contiguous()
        out = torch.empty(self.out_channels, k_pad, dtype=dtype, device=w.device)
        w_scale = self._fp8_weight_scale(src) if dtype == torch.float8_e4m3fn else None
        lib = _lib.load()
        _lib.check(lib.fovi_knnconv_pack_weight(_lib.ptr(src), self.out_channels, self.in_channels, n_ref,
                                                _lib.ptr(out), _lib.dtype_code(dtype), k_pad, c_slot,
                                                _lib.ptr(w_scale), _lib.stream_handle(w.device)),
                   "fovi_knnconv_pack_weight")
        packed = out if w_scale is None else (out, w_scale)
        self._packed[(dtype, c_slot)] = (key, packed)
        return packed

    @staticmethod
    def _fp8_weight_scale(src):
        """Per-output-channel e4m3 weight scale amax|W[o, :]| / 448 (1 for an all-zero row),
        divided on the host: torch's device kernel divides by a scalar via its reciprocal."""
        amax = src.abs().amax(1).cpu()
        return torch.where(amax > 0, amax / 448.0, torch.ones_like(amax)).to(src.device)

    def invalidate_packed_weights(self):
        """Drops the packed copies of ``weight``. They are keyed on the parameter's version, which
        ``copy_``, optimiser steps and ``load_state_dict`` bump; an in-place change through
        ``weight.data`` does not, so call this after one."""
        self._packed = {}
        t = getattr(self, "_transposed_conv", None)
        if t is not None:
            t._weight_key = None

    def set_slot_order(self, order=None):
        """Order in which the wide-layer kernel visits the slots of a channel chunk (a
        permutation of range(V); None = 0, 1, ...). The sum over slots does not depend on it;
        the order 0, 1, ... gives results bit-identical to the row-packed kernels."""
        tiles = self._direct_tables
        wide = T.wide_tables(tiles, self._k, order) if tiles is not None else None
        self._cent_stride = self._coll_off_stride = self._heavy_stride = self._hlist_stride = 0
        self._wide_units = bool(wide.units) if wide is not None else False
        self._wide_tiles = wide.tiles if wide is not None else T.WIDE_TILES
        dev = self.weight.device
        for name, field in (("tile_src", "src"), ("tile_cent", "coll"), ("tile_coll_off", "coll_off"),
                            ("tile_heavy", "heavy"), ("tile_hlist", "hlist")):
            t = None if wide is None else getattr(wide, field)
            self.register_buffer(name, None if t is None else t.to(dev), persistent=False)
        if wide is not None:
            self._cent_stride = wide.stride
            self._coll_off_stride = int(wide.coll_off.shape[1])
            self._heavy_stride = wide.heavy_stride
            self._hlist_stride = wide.hlist_stride
        self.slot_order = None if order is None else [int(v) for v in order]
        self._slot_order_dev = None if order is None else torch.tensor(self.slot_order, dtype=torch.int32,
                                                                          device=dev)
        self._packed.pop(("mfma", torch.bfloat16), None)
        self._packed.pop(("mfma", torch.float8_e4m3fn), None)

    def _packed_weight_mfma(self, dtype=torch.bfloat16):
        """Weight in MFMA-fragment order (``fovi_knnconv_pack_weight_mfma``) for the current slot
        order, cached per weight version: bf16, or (e4m3, per-output-channel scale)."""
        w = self.weight
        key = ("mfma", dtype, w._version, w.data_ptr())
        hit = self._packed.get(("mfma", dtype))
        if hit is not None and hit[0] == key:
            return hit[1]
        n_ref = self.ref_coords.shape[0]
        lib = _lib.load()
        n = lib.fovi_knnconv_weight_mfma_elems(self.out_channels, self.in_channels, n_ref)
        if n <= 0:
            raise ValueError("fragment-order weights need in_channels % 32 == 0")
        src = w.detach().to(torch.float32).contiguous()
        out = torch.empty(n, dtype=dtype, device=w.device)
        w_scale = self._fp8_weight_scale(src) if dtype == torch.float8_e4m3fn else None
        _lib.check(lib.fovi_knnconv_pack_weight_mfma(_lib.ptr(src), self.out_channels, self.in_channels, n_ref,
                                                     _lib.ptr(out), _lib.dtype_code(dtype),
                                                     _lib.ptr(self._slot_order_dev), _lib.ptr(w_scale),
                                                     _lib.stream_handle(w.device)),
                   "fovi_knnconv_pack_weight_mfma")
        packed = out if w_scale is None else (out, w_scale)
        self._packed[("mfma", dtype)] = (key, packed)
        return packed

    def _mfma_lds_bytes(self):
        """LDS bytes of the fragment-order kernel's tile for the layer's tables
        (``knn_tables.wide_layout``)."""
        return T.wide_layout(self.ref_coords.shape[0], self._zero_row, self._coll_off_stride,
                             self._cent_stride, self._heavy_stride, self._hlist_stride)[1]

    def _mfma_column_use(self):
        """Fraction of the fragment-order kernel's 256-channel output tiles that holds real
        channels (the weight is zero-padded up to the tile)."""
        c = self.out_channels
        return c / (256 * -(-c // 256))

    def _mfma_path(self, x, dt):
        """Whether this call runs the fragment-order kernel (see ``mfma_weights``): bf16 or e4m3
        input, channel chunks of 32 (bf16) or 64 (e4m3), 16-byte channels-last input rows."""
        chunk, align = {torch.bfloat16: (32, 8), torch.float8_e4m3fn: (64, 16)}.get(dt, (0, 0))
        return (self.mfma_weights and chunk > 0 and self.in_channels % chunk == 0
                and self._mfma_lds_bytes() <= 160 * 1024
                and self.out_channels % 8 == 0 and self._mfma_column_use() >= 0.75
                and self.tile_src is not None and 0 < self._zero_row <= T.WIDE_MAX_ROWS
                and self._k <= 255 and x.stride(1) == 1 and x.stride(2) % align == 0
                and x.stride(0) % align == 0 and x.data_ptr() % 16 == 0)

    @property
    def padded_channels(self):
        """Channels per input row the few-channel bf16 kernel reads (4 or 8), or None."""
        c = self.in_channels
        return 4 if c <= 4 else (8 if c <= 8 else None)

    def padded_input(self, batch, device=None, view_major=False):
        """A zeroed buffer of input rows padded to ``padded_channels`` (bf16) and its
        ``[B, C_in, N_in]`` view: a producer (e.g. the sampler) that writes into the view
        hands this layer its preferred layout without a copy. Point-major ``[B, N_in, cp]``
        (the fused point-tile kernel), or with ``view_major`` ``[N_in, B, cp]``: the rows of
        one input point for all images adjacent (the view-major kernel)."""
        cp = self.padded_channels
        if cp is None:
            raise ValueError("padded input rows are for layers with at most 8 input channels")
        dev = device or self.weight.device
        if view_major:
            buf = torch.zeros(self.in_coords.shape[0], batch, cp, dtype=torch.bfloat16, device=dev)
            return buf, buf.permute(1, 2, 0)[:, :self.in_channels]
        buf = torch.zeros(batch, self.in_coords.shape[0], cp, dtype=torch.bfloat16, device=dev)
        return buf, buf.transpose(1, 2)[:, :self.in_channels]

    @staticmethod
    def _vm_blocks(c_out):
        """(32-column blocks per wave, blocks with padding) of the view-major kernel: as few
        channel groups as blocks of at most 6 allow (each group gathers the inputs again)."""
        nb = -(-c_out // 32)
        groups = -(-nb // 6)
        cb = next(c for c in (1, 2, 3, 4, 6) if c * groups >= nb)
        return cb, cb * groups

    def _view_major_tables(self, device):
        """The view-major kernel's round tables (``knn_tables.view_major_tables``), built once."""
        if self._vm is None or self._vm[0] != device:
            cp = self.padded_channels
            k_pad = -(-cp * self.ref_coords.shape[0] // _KCHUNK) * _KCHUNK
            vt = T.view_major_tables(self.slot_ptr.cpu(), self.nbr_sorted.cpu(), self.in_coords.shape[0],
                                     self.ref_coords.shape[0], cp, k_pad)
            self._vm = (device, vt.idx.to(device), vt.ev.to(device), vt.off.to(device), vt.j0.to(device))
        return self._vm[1:]

    def _packed_weight_vm(self, c_slot):
        """The view-major kernel's weight fragments (``knn_tables.view_major_weight``), cached
        per weight version; ``(fragments, blocks, blocks per wave)``."""
        w = self.weight
        key = ("vm", c_slot, w._version, w.data_ptr())
        hit = self._packed.get(("vm", c_slot))
        if hit is not None and hit[0] == key:
            return hit[1]
        cb, nb = self._vm_blocks(self.out_channels)
        frag = T.view_major_weight(self._packed_weight(torch.bfloat16, c_slot), cb)
        # skipped reduction steps add nothing only when every weight is finite (0 * inf is NaN)
        finite = bool(torch.isfinite(w.detach()).all())
        packed = (frag, nb, cb, finite)
        self._packed[("vm", c_slot)] = (key, packed)
        return packed

    # -- forward -------------------------------------------------------------
    def _compute_dtype(self, x):
        if x.dtype == torch.bfloat16:
            return torch.bfloat16
        if torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") == torch.bfloat16:
            return torch.bfloat16
        if x.dtype == torch.float32:
            return torch.float32
        raise TypeError(f"KNNConvLayer: unsupported input dtype {x.dtype}")

    def _launch(self, x, activation=None):
        a, y, _keep = self.launch_args(x, activation)
        lib = _lib.load()
        _lib.check(lib.fovi_knnconv_fwd(a, _lib.stream_handle(x.device)), "fovi_knnconv_fwd")
        return y.transpose(1, 2)

    def launch_args(self, x, activation=None, workspace=True):
        """The ``fovi_knnconv_args`` of a forward of ``x`` (fp32 or bf16): ``(args, y, keep)``
        with ``y`` the channels-last ``[B, N_out, C_out]`` output it writes and ``keep`` the
        tensors its pointers name (hold them until the call has run). ``workspace=False``
        leaves the few-channel path's slot-sum workspace out (``fovi_knnconv_fwd_noalloc``
        takes none)."""
        _lib.require_device(x, self.weight)
        if x.dim() != 3 or x.shape[1] != self.in_channels or x.shape[2] != self.in_coords.shape[0]:
            raise ValueError(f"KNNConvLayer: expected [B, {self.in_channels}, {self.in_coords.shape[0]}], "
                             f"got {tuple(x.shape)}")
        dt = self._compute_dtype(x)
        if x.dtype != dt:
            x = x.to(dt)
        c_slot = self.in_channels
        cp = self.padded_channels if dt == torch.bfloat16 else None
        view_major = False
        if cp is not None:
            c_slot = cp
            view_major = (x.stride(1) == 1 and x.stride(0) == cp and x.stride(2) % cp == 0
                          and x.stride(2) >= cp and x.data_ptr() % (2 * cp) == 0)
            if not view_major and not (x.stride(1) == 1 and x.stride(2) == cp and x.stride(0) % cp == 0
                                       and x.data_ptr() % (2 * cp) == 0):
                buf, view = self.padded_input(x.shape[0], x.device)
                view.copy_(x)
                x = view
        mfma = cp is None and self._mfma_path(x, dt)
        self.last_weight_layout = "mfma" if mfma else "rows"
        w = self._packed_weight_mfma() if mfma else self._packed_weight(dt, c_slot)
        bsz, n_out = x.shape[0], self.out_coords.shape[0]
        y = torch.empty(bsz, n_out, self.out_channels, dtype=dt, device=x.device)
        bias = None if self.bias is None else self.bias.detach().to(torch.float32).contiguous()
        a = _lib.KnnConvArgs()
        a.x = x.data_ptr(); a.x_dtype = _lib.dtype_code(dt)
        a.batch, a.c_in, a.n_in = bsz, self.in_channels, x.shape[2]
        a.x_stride[:] = list(x.stride())
        a.n_out, a.k, a.n_ref = n_out, self._k, self.ref_coords.shape[0]
        a.slot_ptr = self.slot_ptr.data_ptr(); a.nbr_sorted = self.nbr_sorted.data_ptr()
        a.w = w.data_ptr(); a.w_dtype = _lib.dtype_code(dt)
        a.w_layout = _lib.W_MFMA if mfma else _lib.W_ROWS
        a.c_out = self.out_channels
        a.k_pad = self.in_channels * self.ref_coords.shape[0] if mfma else w.shape[1]
        a.bias = None if bias is None else bias.data_ptr()
        a.y = y.data_ptr(); a.y_dtype = _lib.dtype_code(dt)
        a.y_stride[:] = [y.stride(0), y.stride(2), y.stride(1)]
        if activation not in (None, "relu"):
            raise ValueError(f"activation must be None or 'relu', got {activation!r}")
        a.activation = _lib.ACT_RELU if activation == "relu" else _lib.ACT_NONE
        a.w_c_slot = c_slot
        vm = None
        if view_major and self.view_major_kernel:
            frag, nb, cb, finite = self._packed_weight_vm(c_slot)
            if finite:
                vm = (self._view_major_tables(x.device), frag, nb, cb)
        if vm is not None:
            (a.vm_idx, a.vm_ev, a.vm_off, a.vm_j0), a.vm_w = [t.data_ptr() for t in vm[0]], vm[1].data_ptr()
            a.vm_nb, a.vm_cb = vm[2], vm[3]
        fused = cp is not None and self.few_channel_fused and self._fc is not None and not view_major
        if fused:
            a.fc_lo = self.fc_lo.data_ptr(); a.fc_span = self.fc_span.data_ptr()
            a.fc_item = self.fc_item.data_ptr()
            a.fc_comb = self.fc_comb.data_ptr(); a.fc_comb_off = self.fc_comb_off.data_ptr()
            a.fc_tile_points, a.fc_zero_row, a.fc_pmax, a.fc_pairs, a.fc_threads, a.fc_chunk = self._fc
        ws = None
        if cp is not None and self.two_pass_few_channels and workspace and not fused and vm is None:
            # slot-sum rows for the two-pass few-channel path (caller-owned scratch)
            ws = torch.empty(bsz * n_out * w.shape[1], dtype=torch.bfloat16, device=x.device)
            a.workspace = ws.data_ptr(); a.workspace_bytes = ws.numel() * 2
        if self.tile_lo is not None:
            a.tile_lo = self.tile_lo.data_ptr(); a.tile_span = self.tile_span.data_ptr()
            a.tile_ent = self.tile_ent.data_ptr(); a.tile_nbr = self.tile_nbr.data_ptr()
            a.tile_points = T.TILE_POINTS; a.max_span = self._max_span
            a.tile_coll = self.tile_coll.data_ptr(); a.tile_coll_n = self.tile_coll_n.data_ptr()
            a.zero_row = self._zero_row
        if mfma:
            self._set_wide_tables(a)
        return a, y, (x, w, bias, ws, vm)

    def _set_wide_tables(self, a):
        """The fragment-order kernel's tables, into the ``fovi_knnconv_args`` ``a``."""
        a.tile_src = self.tile_src.data_ptr(); a.tile_coll_off = self.tile_coll_off.data_ptr()
        a.tile_cent = self.tile_cent.data_ptr()
        a.coll_off_stride = self._coll_off_stride; a.cent_stride = self._cent_stride
        a.tile_heavy = self.tile_heavy.data_ptr(); a.tile_hlist = self.tile_hlist.data_ptr()
        a.heavy_stride = self._heavy_stride; a.hlist_stride = self._hlist_stride
        a.wide_units = int(self._wide_units)
        a.wide_tiles = int(self._wide_tiles)

    # -- backward --------------------------------------------------------------
    def _backward(self, x, weight, dy, need_x, need_w):
        """Gradients of ``y = W a(x) + b`` (a = the slot sums of the gathered inputs, columns
        c * V + v in the reference weight): ``dW = dy^T a`` and ``dx = gather^T (dy W)``. The
        GEMMs run in the input's dtype (fp32 accumulation), the gathers in fp32."""
        _lib.require_device(x, dy)
        if x.dtype not in (torch.float32, torch.bfloat16):
            raise TypeError(f"KNNConvLayer backward: input must be float32 or bfloat16, got {x.dtype}")
        bsz, c, n_in = x.shape
        n_out, v, c_out = self.out_coords.shape[0], self.ref_coords.shape[0], self.out_channels
        dt = x.dtype
        dy2 = dy.to(dt).permute(0, 2, 1).reshape(bsz * n_out, c_out)
        w_sm = weight.detach().to(dt).reshape(c_out, c, v).permute(0, 2, 1).reshape(c_out, v * c)
        lib = _lib.load()
        stream = _lib.stream_handle(x.device)
        dx = dw = None
        if need_w and self.dw_fused and self._dw_fused_ok(x, dt):
            dw = self._dw_fused(x, dy).to(weight.dtype)
        elif need_w:
            a_mat = torch.empty(bsz * n_out, v * c, dtype=dt, device=x.device)
            sa = _lib.SlotsumArgs()
            sa.x = x.data_ptr(); sa.x_dtype = _lib.dtype_code(dt); sa.a_dtype = _lib.dtype_code(dt)
            sa.batch, sa.c_in, sa.n_in = bsz, c, n_in
            sa.x_stride[:] = list(x.stride())
            sa.n_out, sa.k, sa.n_ref = n_out, self._k, v
            sa.slot_ptr = self.slot_ptr.data_ptr(); sa.nbr_sorted = self.nbr_sorted.data_ptr()
            sa.a = a_mat.data_ptr()
            _lib.check(lib.fovi_knnconv_slotsum(sa, stream), "fovi_knnconv_slotsum")
            dw_sm = dy2.t() @ a_mat                                     # [C_out, V * C]
            dw = dw_sm.reshape(c_out, v, c).permute(0, 2, 1).reshape(c_out, c * v).to(weight.dtype)
        if need_x and self.dx_by_transposed_conv:
            dx = self._transposed(x.device)(dy.to(dt), weight)
        elif need_x:
            g = (dy2 @ w_sm).contiguous()                               # [B * N_out, V * C]
            inv_ptr, inv = self._inverse_tables(x.device)
            dx = (torch.empty(bsz, n_in, c, dtype=dt, device=x.device).transpose(1, 2) if x.stride(1) == 1
                  else torch.empty(bsz, c, n_in, dtype=dt, device=x.device))
            ba = _lib.BwdXArgs()
            ba.g = g.data_ptr(); ba.g_dtype = _lib.dtype_code(dt); ba.dx_dtype = _lib.dtype_code(dt)
            ba.batch, ba.c_in, ba.n_in, ba.n_out, ba.n_ref = bsz, c, n_in, n_out, v
            ba.inv_ptr = inv_ptr.data_ptr(); ba.inv = inv.data_ptr()
            ba.dx = dx.data_ptr()
            ba.dx_stride[:] = list(dx.stride())
            _lib.check(lib.fovi_knnconv_bwd_x(ba, stream), "fovi_knnconv_bwd_x")
        return dx, dw

    def _dw_fused_ok(self, x, dt):
        """Whether ``fovi_knnconv_dw`` takes the weight gradient: bf16, channel counts multiples
        of 8, channels-last input rows 16-byte aligned."""
        return (dt == torch.bfloat16 and self.in_channels % 8 == 0 and self.out_channels % 8 == 0
                and x.stride(1) == 1 and x.stride(2) % 8 == 0 and x.stride(0) % 8 == 0
                and x.data_ptr() % 16 == 0)

    def _dw_fused(self, x, dy):
        """``dW`` (fp32, reference layout) by ``fovi_knnconv_dw``: per slot a GEMM over its
        (output, input) pairs, no slot-sum matrix; one workgroup per slot, chunk of
        ``dw_chunk`` output points and ``dw_images_per_group`` images."""
        bsz, c, n_in = x.shape
        n_out, v, c_out = self.out_coords.shape[0], self.ref_coords.shape[0], self.out_channels
        dyc = dy.to(torch.bfloat16)
        if not (dyc.stride(1) == 1 and dyc.stride(2) % 8 == 0 and dyc.stride(0) % 8 == 0
                and dyc.data_ptr() % 16 == 0):
            dyc = dyc.transpose(1, 2).contiguous().transpose(1, 2)
        pair_off, pairs = self._slot_pairs(x.device)
        lib = _lib.load()
        n_chunks = (pair_off.numel() - 1) // v
        ipg = self.dw_images_per_group
        nbytes = lib.fovi_knnconv_dw_workspace_bytes(bsz, ipg, n_chunks, c, c_out, v)
        ws = torch.empty(nbytes // 4, dtype=torch.float32, device=x.device)
        dw = torch.empty(c_out, c * v, dtype=torch.float32, device=x.device)
        a = _lib.KnnConvDwArgs()
        a.x = x.data_ptr(); a.x_stride[:] = list(x.stride())
        a.dy = dyc.data_ptr(); a.dy_stride[:] = list(dyc.stride())
        a.batch, a.c_in, a.c_out, a.n_in, a.n_out, a.n_ref = bsz, c, c_out, n_in, n_out, v
        a.pair_off = pair_off.data_ptr(); a.pairs = pairs.data_ptr()
        a.n_chunks = n_chunks
        a.images_per_group = ipg
        a.workspace = ws.data_ptr(); a.workspace_bytes = nbytes
        a.dw = dw.data_ptr()
        _lib.check(lib.fovi_knnconv_dw(a, _lib.stream_handle(x.device)), "fovi_knnconv_dw")
        return dw

    def _slot_pairs(self, device):
        """``knn_tables.slot_pairs`` of this layer, built on the first backward and kept."""
        sp = getattr(self, "_slot_pair_tables", None)
        if sp is None or sp[0].device != device:
            off, pairs = T.slot_pairs(self.slot_ptr.cpu(), self.nbr_sorted.cpu(), self.ref_coords.shape[0],
                                      chunk=self.dw_chunk, step=64)
            sp = (off.to(device), pairs.to(device))
            self._slot_pair_tables = sp
        return sp

    def _transposed(self, device):
        """The input gradient as a kNN-conv forward (``_TransposedKnnConv``), built on the first
        backward and kept."""
        t = getattr(self, "_transposed_conv", None)
        if t is None or t.weight.device != device:
            t = _TransposedKnnConv(self, device)
            # kept outside the module tree: not a submodule, parameter or state-dict entry, and
            # not found by code that walks modules() for kNN layers
            object.__setattr__(self, "_transposed_conv", t)
        return t

    def _inverse_tables(self, device):
        """Per input point, the (output, slot) pairs that read it (``knn_tables.inverse_tables``),
        built on the first backward and kept on the device."""
        inv = getattr(self, "_inv_tables", None)
        if inv is None or inv[0].device != device:
            ptr, ent = T.inverse_tables(self.slot_ptr.cpu(), self.nbr_sorted.cpu(), self.in_coords.shape[0],
                                        self.ref_coords.shape[0])
            inv = (ptr.to(device), ent.to(device))
            self._inv_tables = inv
        return inv

    # -- fp8 ----------------------------------------------------------------
    @property
    def fp8_headroom(self):
        """Power of two >= the largest slot neighbour count: the activation scale
        ``amax * headroom / 448`` keeps every slot sum of quantized values <= 448."""
        return headroom_for(self._max_slot_count)

    def quantize_input(self, x, scale=None):
        """e4m3 activations for this layer (``Fp8Activations``; channels-last)."""
        if isinstance(x, Fp8Activations):
            return x
        return quantize_e4m3(x, self.fp8_headroom, scale)

    def _launch_fp8(self, xq, activation=None):
        x, scale = xq.data, xq.scale
        _lib.require_device(x, scale, self.weight)
        if x.dtype != torch.float8_e4m3fn:
            raise TypeError(f"Fp8Activations.data must be float8_e4m3fn, got {x.dtype}")
        if x.dim() != 3 or x.shape[1] != self.in_channels or x.shape[2] != self.in_coords.shape[0]:
            raise ValueError(f"KNNConvLayer: expected [B, {self.in_channels}, {self.in_coords.shape[0]}], "
                             f"got {tuple(x.shape)}")
        if self.tile_lo is None:
            raise NotImplementedError("fp8 kNN-conv needs the tile tables (k <= 255, tile spans <= 65535)")
        mfma = self._mfma_path(x, torch.float8_e4m3fn)
        self.last_weight_layout = "mfma" if mfma else "rows"
        w, w_scale = (self._packed_weight_mfma(torch.float8_e4m3fn) if mfma
                      else self._packed_weight(torch.float8_e4m3fn))
        bsz, n_out = x.shape[0], self.out_coords.shape[0]
        y = torch.empty(bsz, n_out, self.out_channels, dtype=torch.bfloat16, device=x.device)
        bias = None if self.bias is None else self.bias.detach().to(torch.float32).contiguous()
        scale = scale.to(torch.float32).reshape(1).contiguous()
        a = _lib.KnnConvArgs()
        a.x = x.data_ptr(); a.x_dtype = _lib.F8E4M3
        a.batch, a.c_in, a.n_in = bsz, self.in_channels, x.shape[2]
        a.x_stride[:] = list(x.stride())
        a.n_out, a.k, a.n_ref = n_out, self._k, self.ref_coords.shape[0]
        a.slot_ptr = self.slot_ptr.data_ptr(); a.nbr_sorted = self.nbr_sorted.data_ptr()
        a.w = w.data_ptr(); a.w_dtype = _lib.F8E4M3
        a.w_layout = _lib.W_MFMA if mfma else _lib.W_ROWS
        a.c_out = self.out_channels
        a.k_pad = self.in_channels * self.ref_coords.shape[0] if mfma else w.shape[1]
        a.bias = None if bias is None else bias.data_ptr()
        a.w_scale = w_scale.data_ptr(); a.x_scale_dev = scale.data_ptr()
        a.y = y.data_ptr(); a.y_dtype = _lib.BF16
        a.y_stride[:] = [y.stride(0), y.stride(2), y.stride(1)]
        if activation not in (None, "relu"):
            raise ValueError(f"activation must be None or 'relu', got {activation!r}")
        a.activation = _lib.ACT_RELU if activation == "relu" else _lib.ACT_NONE
        a.w_c_slot = self.in_channels
        a.tile_lo = self.tile_lo.data_ptr(); a.tile_span = self.tile_span.data_ptr()
        a.tile_ent = self.tile_ent.data_ptr(); a.tile_nbr = self.tile_nbr.data_ptr()
        a.tile_points = T.TILE_POINTS; a.max_span = self._max_span
        a.tile_coll = self.tile_coll.data_ptr(); a.tile_coll_n = self.tile_coll_n.data_ptr()
        a.zero_row = self._zero_row
        if mfma:
            self._set_wide_tables(a)
        lib = _lib.load()
        _lib.check(lib.fovi_knnconv_fwd(a, _lib.stream_handle(x.device)), "fovi_knnconv_fwd(fp8)")
        return y.transpose(1, 2)

    def forward(self, X_l):
        if isinstance(X_l, Fp8Activations) or self.fp8:
            return self._launch_fp8(self.quantize_input(X_l))
        return _KnnConvFn.apply(X_l, self, self.weight, self.bias)

    def forward_fused(self, X_l, activation="relu"):
        """``activation(forward(X_l))`` with the activation applied in the kernel's store."""
        if isinstance(X_l, Fp8Activations) or self.fp8:
            return self._launch_fp8(self.quantize_input(X_l), activation)
        return _KnnConvFn.apply(X_l, self, self.weight, self.bias, activation)

    # -- conv2d import (reference knn.py:649-715) -------------------------------
    def _load_conv_2d_weight(self, conv_weight, conv_bias, strict=False):
        if conv_weight.shape[0] != self.out_channels:
            raise ValueError(f"Conv2d out_channels {conv_weight.shape[0]} != layer out_channels {self.out_channels}")
        if conv_weight.shape[1] != self.in_channels:
            raise ValueError(f"Conv2d in_channels {conv_weight.shape[1]} != layer in_channels {self.in_channels}")
        # conv (row, col) = (-y, x) -> ref grid (x, y)
        conv_weight = conv_weight.transpose(-1, -2).flip(-1)
        s = self.ref_grid_size
        if conv_weight.shape[2] != s or conv_weight.shape[3] != s:
            if strict:
                raise ValueError(f"Conv2d kernel size {conv_weight.shape[2]}x{conv_weight.shape[3]} != "
                                 f"ref_grid_size {s}x{s}. Set strict=False to resample the kernel.")
            conv_weight = F.interpolate(conv_weight, size=(s, s), mode="bilinear", align_corners=True)
        if conv_bias is not None and self.bias is None:
            raise ValueError("Conv2d has bias but layer does not. Recreate layer with bias=True.")
        # copy_ on the parameter itself (not .data) bumps its version, which keys the packed
        # weight caches; they are cleared as well
        with torch.no_grad():
            self.weight.copy_(conv_weight.reshape(conv_weight.shape[0], -1))
            if conv_bias is not None:
                self.bias.copy_(conv_bias.detach())
        self.invalidate_packed_weights()

    def load_conv2d_weights(self, conv2d, strict=False):
        self._load_conv_2d_weight(conv2d.weight.data.clone(), conv2d.bias, strict=strict)

    def load_conv3d_weights(self, conv3d, temporal_strategy="average", strict=False):
        w = conv3d.weight.data.clone()
        if temporal_strategy == "average":
            w = w.mean(2)
        elif temporal_strategy == "select_first":
            w = w[:, :, 0]
        else:
            raise NotImplementedError()
        self._load_conv_2d_weight(w, conv3d.bias, strict=strict)

    def __repr__(self):
        return (f"{self.__class__.__name__}(\n\tin_channels={self.in_channels}\n\tout_channels="
                f"{self.out_channels}\n\tk={self.k}\n\tn_ref={self.ref_coords.shape[0]}\n\tin_coords="
                f"{self.in_coords}\n\tout_coords={self.out_coords}\n\tsample_cortex={self.sample_cortex}\n)")


class _TransposedKnnConv(KNNConvLayer):
    """The input gradient of a ``KNNConvLayer`` as a kNN-conv forward of its own.

    ``dx[b, c, i] = sum over the (n, v) whose slot v holds i of sum_o dy[b, o, n] W[o, c V + v]``:
    a kNN-conv from the output points to the input points with the inverse neighbour table
    (``knn_tables.inverse_knn``: the lists of input i hold the outputs n that read i, in the
    slot i sits in) and the weight ``W_T[c, o V + v] = W[o, c V + v]``, so it runs the forward
    kernels (fused gather, slot sum and MFMA GEMM) with no ``[B N_out, V C]`` intermediate.
    """

    def __init__(self, layer, device):
        nn.Module.__init__(self)
        n_in, n_out = layer.in_coords.shape[0], layer.out_coords.shape[0]
        n_ref = layer.ref_coords.shape[0]
        idx, slots = T.inverse_knn(layer.slot_ptr.cpu(), layer.nbr_sorted.cpu(), n_in, n_ref)
        self.in_channels, self.out_channels = layer.out_channels, layer.in_channels
        self.in_coords, self.out_coords = layer.out_coords, layer.in_coords
        self.ref_coords = layer.ref_coords
        self._k = idx.shape[0]
        self.bias = None
        self.weight = torch.zeros(layer.in_channels, layer.out_channels * n_ref, device=device)
        self._weight_key = None
        self._init_tables(idx, slots, n_out, n_ref, device)

    def forward(self, dy, weight):
        """``dx`` of the layer for the output gradient ``dy [B, C_out, N_out]`` and the weight
        the forward ran with: ``[B, C_in, N_in]`` (a transposed view of channels-last storage),
        in ``dy``'s dtype."""
        key = (weight._version, weight.data_ptr())
        if key != self._weight_key:
            c_out, c_in_v = weight.shape
            n_ref = self.ref_coords.shape[0]
            w_t = weight.detach().reshape(c_out, c_in_v // n_ref, n_ref).permute(1, 0, 2)
            self.weight.copy_(w_t.reshape(self.weight.shape))
            self._weight_key = key
        return self._launch(dy)


def _normalize(x, dim=None):
    """Min-max normalisation (reference fovi/utils/__init__.py:126-167): (x - min) / (max - min)
    with min and max over ``dim`` (kept) or over the whole tensor."""
    if dim is not None:
        lo, hi = x.min(dim).values.unsqueeze(dim), x.max(dim).values.unsqueeze(dim)
    else:
        lo, hi = x.min(), x.max()
    return (x - lo) / (hi - lo)


class _KnnPoolFn(torch.autograd.Function):
    """Forward ``fovi_knnpool_fwd``; backward ``fovi_knnpool_bwd`` (gather over the inverse
    neighbour table, the reference's NaN masks carry no gradient)."""

    @staticmethod
    def forward(ctx, x, layer):
        ctx.layer = layer
        ctx.save_for_backward(x)
        return layer._launch(x)

    @staticmethod
    def backward(ctx, dy):
        (x,) = ctx.saved_tensors
        return ctx.layer._backward(x, dy), None


_POOL_MODES = {"max": _lib.POOL_MAX, "avg": _lib.POOL_AVG, "sum": _lib.POOL_SUM, "gaussian": _lib.POOL_GAUSSIAN}


class KNNPoolingLayer(nn.Module, KNNBaseLayer):
    """kNN pooling on a sensor point cloud (HIP forward; reference ``knn.py:272-394``).

    Same constructor, attributes and results as the reference: each output point reduces
    its k nearest input points (cortical distance) per channel by max, NaN-ignoring mean
    or sum, or a Gaussian-weighted mean; pad-token neighbours (index >= N_in) read NaN.
    The forward is ``fovi_knnpool_fwd`` (one fused gather-reduce launch, fp32 arithmetic);
    channels-last inputs give channels-last outputs (the ``[B, C, N]`` view of
    ``[B, N, C]`` storage), as the kNN-conv layers do.
    """

    def __init__(self, k, in_coords, out_coords, mode="max", device="cuda", sample_cortex=True, gauss_sigma=10,
                 batch_size=None):
        super().__init__()
        self.k = k
        self.in_coords = in_coords
        self.out_coords = out_coords
        self.device = device
        assert mode in ["max", "avg", "sum", "gaussian"]
        self.mode = mode
        self.sample_cortex = sample_cortex
        self.batch_size = batch_size
        _check_coords(in_coords, "in_coords")
        _check_coords(out_coords, "out_coords")
        self.k = torch.minimum(torch.tensor(self.k), torch.tensor(self.in_coords.shape[0]))   # knn.py:311
        self._k = int(self.k.item())
        knn_indices, knn_distances = self._compute_knns(batch_size)
        self.knn_indices = knn_indices.to(device)
        self.knn_distances = knn_distances.to(device)
        # padding mask / token (knn.py:317-321)
        self.knn_pad_token_val = self.in_coords.shape[0]
        self.knn_indices_pad_mask = self.knn_indices >= self.in_coords.shape[0]
        self.knn_indices_pad_token = self.knn_indices.clone()
        self.knn_indices_pad_token[self.knn_indices_pad_mask] = self.knn_pad_token_val
        if self.mode == "gaussian":
            self.gauss_sigma = gauss_sigma
            self.gaussian_weights = self._compute_gaussian_weights()
        # kernel tables: each output point's k neighbours (and weights) contiguous
        self.register_buffer("nbr_rows", self.knn_indices_pad_token.t().contiguous().to(torch.int32),
                             persistent=False)
        self.register_buffer("weight_rows", self.gaussian_weights.t().contiguous().to(torch.float32)
                             if self.mode == "gaussian" else None, persistent=False)

    def _compute_gaussian_weights(self):
        """exp(-d^2 / (2 sigma^2)) over the per-point min-max normalised neighbour distances,
        divided by (sum + 1e-8) per output point (reference knn.py:325-343). ``[k, N_out]``."""
        k_distances = _normalize(self.knn_distances, dim=0)
        gaussian_weights = torch.exp(-k_distances ** 2 / (2 * self.gauss_sigma ** 2))
        return gaussian_weights / (gaussian_weights.sum(dim=0, keepdim=True) + 1e-8)

    def _launch(self, x):
        _lib.require_device(x, self.nbr_rows)
        if x.dim() != 3 or x.shape[2] != self.in_coords.shape[0]:
            raise ValueError(f"KNNPoolingLayer: expected [B, C, {self.in_coords.shape[0]}], got {tuple(x.shape)}")
        if x.dtype not in (torch.float32, torch.bfloat16):
            raise TypeError(f"KNNPoolingLayer: input must be float32 or bfloat16, got {x.dtype}")
        bsz, c, n_out = x.shape[0], x.shape[1], self.out_coords.shape[0]
        # the Gaussian mode multiplies by fp32 weights: the reference's result is promoted
        dt = torch.promote_types(x.dtype, torch.float32) if self.mode == "gaussian" else x.dtype
        if x.stride(1) == 1 and c > 1:
            y = torch.empty(bsz, n_out, c, dtype=dt, device=x.device).transpose(1, 2)
        else:
            y = torch.empty(bsz, c, n_out, dtype=dt, device=x.device)
        a = _lib.KnnPoolArgs()
        a.x = x.data_ptr(); a.x_dtype = _lib.dtype_code(x.dtype); a.mode = _POOL_MODES[self.mode]
        a.batch, a.channels, a.n_in = bsz, c, x.shape[2]
        a.x_stride[:] = list(x.stride())
        a.nbr = self.nbr_rows.data_ptr()
        a.weights = self.weight_rows.data_ptr() if self.weight_rows is not None else None
        a.n_out, a.k = n_out, self._k
        a.y = y.data_ptr(); a.y_dtype = _lib.dtype_code(dt)
        a.y_stride[:] = list(y.stride())
        lib = _lib.load()
        _lib.check(lib.fovi_knnpool_fwd(a, _lib.stream_handle(x.device)), "fovi_knnpool_fwd")
        return y

    def forward(self, X_l):
        """``[B, C, N_in] -> [B, C, N_out]`` (reference knn.py:345-394)."""
        return _KnnPoolFn.apply(X_l, self)

    def _backward(self, x, dy):
        """``dx`` in ``x``'s dtype and layout (``fovi_knnpool_bwd``)."""
        _lib.require_device(x, dy)
        bsz, c, n_in = x.shape
        n_out = self.out_coords.shape[0]
        inv = getattr(self, "_inv_rows", None)
        if inv is None or inv[0].device != x.device:
            ptr, ent = T.inverse_rows(self.nbr_rows.cpu(), n_in)
            inv = (ptr.to(x.device), ent.to(x.device))
            self._inv_rows = inv
        dx = (torch.empty(bsz, n_in, c, dtype=x.dtype, device=x.device).transpose(1, 2) if x.stride(1) == 1
              else torch.empty(bsz, c, n_in, dtype=x.dtype, device=x.device))
        if dy.dtype not in (torch.float32, torch.bfloat16):
            dy = dy.float()
        state = None if self.mode == "sum" else torch.empty(bsz * n_out * c, dtype=torch.float32, device=x.device)
        a = _lib.KnnPoolBwdArgs()
        a.x = x.data_ptr(); a.x_dtype = _lib.dtype_code(x.dtype); a.mode = _POOL_MODES[self.mode]
        a.batch, a.channels, a.n_in = bsz, c, n_in
        a.x_stride[:] = list(x.stride())
        a.nbr = self.nbr_rows.data_ptr()
        a.weights = self.weight_rows.data_ptr() if self.weight_rows is not None else None
        a.n_out, a.k = n_out, self._k
        a.dy = dy.data_ptr(); a.dy_dtype = _lib.dtype_code(dy.dtype)
        a.dy_stride[:] = list(dy.stride())
        a.dx_dtype = _lib.dtype_code(dx.dtype)
        a.inv_ptr, a.inv = inv[0].data_ptr(), inv[1].data_ptr()
        a.state = None if state is None else state.data_ptr()
        a.dx = dx.data_ptr(); a.dx_stride[:] = list(dx.stride())
        lib = _lib.load()
        _lib.check(lib.fovi_knnpool_bwd(a, _lib.stream_handle(x.device)), "fovi_knnpool_bwd")
        return dx

    def __repr__(self):
        return (f"KNNPoolingLayer(\n\tmode={self.mode}\n\tk={self.k}\n\tin_coords={self.in_coords}\n"
                f"\tout_coords={self.out_coords}\n\tsample_cortex={self.sample_cortex}\n)")


def get_in_out_coords(in_res, fov, cmf_a, stride, style="isotropic", auto_match_cart_resources=1,
                      in_cart_res=None, device="cuda", in_coords=None, force_out_match_less_than=True,
                      max_out_coord_val=1):
    """Input and strided output point sets (reference ``knn.py:958-1003``)."""
    from ..sensing.coords import auto_match_num_coords
    if in_coords is None:
        if auto_match_cart_resources:
            in_res, in_cart_res = auto_match_num_coords(fov, cmf_a, in_cart_res, style, auto_match_cart_resources,
                                                        device, force_less_than=True, quiet=True)
        in_coords = SamplingCoords(fov, cmf_a, in_res, device=device, style=style)
    tmp_max = 1 if max_out_coord_val == "auto" else max_out_coord_val
    out_coords, _, out_cart_res = in_coords.get_strided_coords(
        stride, auto_match_cart_resources=auto_match_cart_resources, in_cart_res=in_cart_res,
        force_less_than=force_out_match_less_than, max_val=tmp_max)
    if max_out_coord_val == "auto":
        radii = torch.unique(out_coords.polar[:, 0])
        final = (radii[-1] + radii[-2]) / 2
        out_coords, _, out_cart_res = in_coords.get_strided_coords(
            stride, auto_match_cart_resources=auto_match_cart_resources, in_cart_res=in_cart_res,
            force_less_than=force_out_match_less_than, max_val=final)
    return in_coords, out_coords, out_cart_res


KNN_CONV_REGISTRY = {
    "default": KNNConvLayer,
}


def register_with_reference(ref_knn, name="mi355x", ref_knnalexnet=None):
    """Plugs the kernel-backed layers into an unmodified fovi checkout.

    ``ref_knn`` is the reference's ``fovi.arch.knn`` module. Registers, under ``name`` in its
    ``KNN_CONV_REGISTRY`` (``knn.py:1007-1030``, where ``KNNAlexNetBlock``,
    ``knnalexnet.py:56-57``, and ``cfg.model.conv_layer_cls``, ``architectures.py:114``, look
    layers up), a ``KNNConvLayer`` subclass that is also a subclass of the reference's
    ``KNNBaseLayer``, so ``FoviNet.list_knn_layers`` (``fovinet.py:504-514``) and the
    visualizer's ``isinstance`` filters (``visualizer.py:360,482``) find it. The layers take
    the reference's ``SamplingCoords`` as they come. With ``ref_knnalexnet`` (the
    reference's ``fovi.arch.knnalexnet``) its blocks also build the kernel-backed
    ``KNNPoolingLayer`` (``knnalexnet.py:90-101``). Returns ``(conv_cls, pool_cls)``."""
    base = ref_knn.KNNBaseLayer
    conv = type("MI355XKNNConvLayer", (KNNConvLayer, base),
                {"__module__": __name__, "__doc__": KNNConvLayer.__doc__})
    pool = type("MI355XKNNPoolingLayer", (KNNPoolingLayer, base),
                {"__module__": __name__, "__doc__": KNNPoolingLayer.__doc__})
    ref_knn.KNN_CONV_REGISTRY[name] = conv
    if ref_knnalexnet is not None:
        ref_knnalexnet.KNNPoolingLayer = pool
    return conv, pool


def get_knn_conv_layer(name: str):
    """Layer class by registry name (reference ``knn.py:1014-1030``)."""
    if name not in KNN_CONV_REGISTRY:
        raise ValueError(f"Unknown KNN conv layer: {name}. Available: {list(KNN_CONV_REGISTRY.keys())}")
    return KNN_CONV_REGISTRY[name]
