"""fovi_knnconv_fwd_noalloc: the kNN-conv forward for callers that cannot allocate (no
counterpart in the reference). It must equal fovi_knnconv_fwd with a caller workspace bit for
bit, on consecutive calls (the scratch keeps the previous call's rows), and refuse inputs whose
slot sums do not fit its 64 MiB scratch before launching anything.
"""
import ctypes as C

import numpy as np
import pytest
import torch

from fovi_amd import _lib
from fovi_amd.arch.knn import KNNConvLayer
from fovi_amd.sensing.coords import SamplingCoords

SCRATCH = 64 << 20


def _layer(res_in, res_out, k, c_in, c_out, side=None, seed=1):
    layer = KNNConvLayer(c_in, c_out, k, SamplingCoords(16, 2.78, res_in, style="logpolar"),
                         SamplingCoords(16, 2.78, res_out, style="logpolar"), device="cuda", bias=True,
                         ref_frame_side_length=side)
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        layer.weight.copy_(torch.randn(layer.weight.shape, generator=g) * (1.0 / (c_in * layer._k)) ** 0.5)
        layer.bias.copy_(torch.randn(c_out, generator=g) * 0.1)
    return layer


def _call(layer, x, entry):
    """Runs one C-ABI entry point on the layer's arguments; returns (y [B, N_out, C_out], path)."""
    a, y, keep = layer.launch_args(x, workspace=(entry == "fovi_knnconv_fwd"))
    lib = _lib.load()
    _lib.check(getattr(lib, entry)(a, _lib.stream_handle(x.device)), entry)
    torch.cuda.synchronize()
    del keep
    return y, _lib.knnconv_last_path()


@pytest.mark.gpu
def test_noalloc_equals_workspace_entry_point_on_consecutive_calls():
    """C4 patch-embedding geometry (16384 -> 256 log-polar points, k = 256, 16 x 16 ref grid,
    3 -> 384): one view's slot sums are 256 x 1024 bf16 = 512 KiB, so the 64 MiB scratch holds
    128 views. First call 300 views (three chunks), then 5 views (one chunk, smaller)."""
    from oracle import knnconv_ref
    from tests.helpers import assert_close_rel
    layer = _layer(128, 16, 256, 3, 384, side=16)
    layer.few_channel_fused = False      # the two-pass path, whose slot sums need the scratch
    g = torch.Generator().manual_seed(2)
    for n_views in (300, 5):
        x = torch.rand(n_views, 3, 16384, generator=g).bfloat16()
        _, xv = layer.padded_input(n_views)
        xv.copy_(x.cuda())
        y_ws, path_ws = _call(layer, xv, "fovi_knnconv_fwd")
        y, path = _call(layer, xv, "fovi_knnconv_fwd_noalloc")
        assert path_ws == path == "bf16 few-channel two-pass", (path_ws, path)
        assert torch.equal(y, y_ws), f"{n_views} views: noalloc differs from the workspace entry point"
    w = layer.weight.detach().cpu().bfloat16().float()
    ref = knnconv_ref.knnconv_forward(x[:2].float(), layer.knn_indices.cpu(), 16384, layer.local_rf.cpu(), w,
                                      layer.bias.detach().cpu())
    assert_close_rel(y[:2].transpose(1, 2).float().cpu(), ref, 1e-2, "noalloc vs the oracle")


@pytest.mark.gpu
def test_noalloc_paths_without_scratch_and_workspace_rejected():
    """A wide layer (C2 layer 4 geometry, 384 -> 256) takes a path with no scratch: same result
    as fovi_knnconv_fwd. A workspace argument is refused."""
    layer = _layer(16, 16, 9, 384, 256)
    x = torch.randn(3, 256, 384, generator=torch.Generator().manual_seed(3)).bfloat16().cuda().transpose(1, 2)
    y_ref, p_ref = _call(layer, x, "fovi_knnconv_fwd")
    y, p = _call(layer, x, "fovi_knnconv_fwd_noalloc")
    assert p == p_ref == "bf16 v5" and torch.equal(y, y_ref)
    a, y, keep = layer.launch_args(x)
    a.workspace, a.workspace_bytes = y.data_ptr(), 16
    assert _lib.load().fovi_knnconv_fwd_noalloc(a, _lib.stream_handle(x.device)) != 0
    assert b"takes no workspace" in _lib.load().fovi_last_error()


def test_noalloc_refuses_slot_sums_beyond_its_scratch():
    """Host-side check, before any HIP call (runs without a GPU): one image's slot sums of
    n_out x k_pad bf16 above 64 MiB are an error naming the limit. Every data pointer is NULL,
    so were the size check to pass, the null-pointer checks would still refuse the call: no
    launch can follow, on a GPU host either."""
    lib = _lib.load()
    a = _lib.KnnConvArgs()
    a.x_dtype = a.w_dtype = _lib.BF16; a.y_dtype = _lib.BF16; a.w_layout = _lib.W_ROWS
    a.batch, a.c_in, a.n_in, a.c_out = 2, 3, 1024, 64
    a.x_stride[:] = [1024 * 4, 1, 4]
    a.y_stride[:] = [1 << 20, 1, 64]
    a.w_c_slot = 4
    a.n_out, a.k, a.n_ref, a.k_pad = 1 << 16, 256, 256, 1024     # 65536 x 1024 x 2 B = 128 MiB
    assert lib.fovi_knnconv_fwd_noalloc(a, None) != 0
    msg = lib.fovi_last_error().decode()
    assert "exceed" in msg and str(SCRATCH) in msg, msg
    a.n_out = SCRATCH // (2 * 1024) + 1                            # just past the limit
    assert lib.fovi_knnconv_fwd_noalloc(a, None) != 0 and "exceed" in lib.fovi_last_error().decode()
    a.n_out = SCRATCH // (2 * 1024)                                # fits: the NULL pointers are refused
    assert lib.fovi_knnconv_fwd_noalloc(a, None) != 0 and "null pointer" in lib.fovi_last_error().decode()


@pytest.mark.gpu
def test_noalloc_calls_on_two_streams_take_the_scratch_in_call_order():
    """Two streams, no synchronisation between the calls: a long call (300 views, three chunks
    through the scratch) on stream A, then a short one (5 views) on stream B. The second waits
    for the first's last use of the scratch, so both equal the workspace entry point, and
    stream B's call completes after stream A's (without the wait the short call, enqueued on
    an idle stream, would finish first and its slot sums would overwrite A's in flight)."""
    layer = _layer(128, 16, 256, 3, 384, side=16)
    layer.few_channel_fused = False
    g = torch.Generator().manual_seed(4)
    xs, want = [], []
    for n_views in (300, 5):
        x = torch.rand(n_views, 3, 16384, generator=g).bfloat16()
        _, xv = layer.padded_input(n_views)
        xv.copy_(x.cuda())
        xs.append(xv)
        want.append(_call(layer, xv, "fovi_knnconv_fwd")[0])
    lib = _lib.load()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    done = [torch.cuda.Event(enable_timing=True) for _ in streams]
    start = torch.cuda.Event(enable_timing=True)
    outs, keep = [], []
    torch.cuda.synchronize()
    start.record(streams[0])
    streams[1].wait_event(start)
    for xv, st, ev in zip(xs, streams, done):
        with torch.cuda.stream(st):
            a, y, k = layer.launch_args(xv, workspace=False)
            _lib.check(lib.fovi_knnconv_fwd_noalloc(a, C.c_void_p(st.cuda_stream)), "fovi_knnconv_fwd_noalloc")
            ev.record(st)
        outs.append(y)
        keep.append(k)
    torch.cuda.synchronize()
    for y, w in zip(outs, want):
        assert torch.equal(y, w)
    assert start.elapsed_time(done[1]) >= start.elapsed_time(done[0])
