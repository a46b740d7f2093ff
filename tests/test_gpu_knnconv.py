"""GPU parity of the kNN-conv forward against the CPU oracle (torch restatement of knn.py:484-557).

Bar: fp32 within 1e-5 relative (L2 and max-abs/max|ref|); bf16 within 1e-2
relative against the oracle evaluated on the bf16-rounded operands.
"""
import pytest
import torch

from fovi_amd.arch.knn import KNNConvLayer
from fovi_amd.sensing.coords import SamplingCoords
from oracle import knnconv_ref
from tests.helpers import assert_close_rel

pytestmark = pytest.mark.gpu


def _layer(res_in, res_out, k, c_in, c_out, side=None, bias=False, seed=1):
    cin = SamplingCoords(16, 2.78, res_in, style="logpolar")
    cout = SamplingCoords(16, 2.78, res_out, style="logpolar")
    layer = KNNConvLayer(c_in, c_out, k, cin, cout, device="cuda", bias=bias, ref_frame_side_length=side)
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        layer.weight.copy_(torch.randn(layer.weight.shape, generator=g) * (1.0 / (c_in * layer._k)) ** 0.5)
        if bias:
            layer.bias.copy_(torch.randn(c_out, generator=g) * 0.1)
    return layer


def _oracle(layer, x, w=None):
    w = layer.weight.detach().cpu() if w is None else w
    b = None if layer.bias is None else layer.bias.detach().cpu()
    return knnconv_ref.knnconv_forward(x.float().cpu(), layer.knn_indices.cpu(), layer.in_coords.shape[0],
                                       layer.local_rf.cpu(), w, b)


def test_c1_fp32():
    """C1: 8 x 3 x 4096 fp32, k=9 on the 64x64 log-polar lattice, 3 -> 64."""
    layer = _layer(64, 64, 9, 3, 64)
    x = torch.rand(8, 3, 4096, generator=torch.Generator().manual_seed(0))
    with torch.no_grad():
        y = layer(x.cuda())
    assert y.shape == (8, 64, 4096) and y.dtype == torch.float32
    assert_close_rel(y.cpu(), _oracle(layer, x), 1e-5, "C1 fp32")


@pytest.mark.parametrize("res_in,res_out,k,c_in,c_out,side,bias", [
    (64, 32, 49, 3, 64, None, False),     # C2 layer 1 geometry
    (32, 16, 25, 64, 192, None, False),   # C2 layer 2
    (16, 16, 9, 192, 384, None, True),    # C2 layer 3
    (16, 16, 9, 384, 256, None, False),   # C2 layer 4
    (24, 12, 30, 5, 40, None, True),      # ragged: non-square k, odd channels, partial tiles
    (32, 4, 256, 3, 96, 16, True),        # patch-embed style: k=256, 16x16 ref grid
])
def test_fp32_shapes(res_in, res_out, k, c_in, c_out, side, bias):
    layer = _layer(res_in, res_out, k, c_in, c_out, side, bias)
    x = torch.randn(3, c_in, res_in * res_in, generator=torch.Generator().manual_seed(5))
    with torch.no_grad():
        y = layer(x.cuda())
    assert_close_rel(y.cpu(), _oracle(layer, x), 1e-5)


@pytest.mark.parametrize("res_in,res_out,k,c_in,c_out,side,bias,channels_last", [
    (64, 32, 49, 3, 64, None, False, False),     # C2 layer 1 (generic loader)
    (32, 16, 25, 64, 192, None, False, True),    # C2 layer 2 (vector loader)
    (32, 16, 25, 64, 192, None, False, False),   # same, channel-major input (generic loader)
    (16, 16, 9, 192, 384, None, True, True),     # C2 layer 3
    (16, 16, 9, 384, 256, None, False, True),    # C2 layer 4
    (24, 12, 30, 5, 40, None, True, False),      # ragged
    (32, 4, 256, 3, 96, 16, True, False),        # patch-embed style
])
def test_bf16_shapes(res_in, res_out, k, c_in, c_out, side, bias, channels_last):
    layer = _layer(res_in, res_out, k, c_in, c_out, side, bias)
    n_in = res_in * res_in
    x = torch.randn(3, c_in, n_in, generator=torch.Generator().manual_seed(6)).bfloat16()
    xd = x.cuda()
    if channels_last:
        xd = xd.transpose(1, 2).contiguous().transpose(1, 2)
    with torch.no_grad():
        y = layer(xd)
    assert y.dtype == torch.bfloat16
    ref = _oracle(layer, x, layer.weight.detach().cpu().bfloat16().float())
    assert_close_rel(y.float().cpu(), ref, 1e-2)


def test_autocast_bf16_casts_fp32_input():
    layer = _layer(32, 16, 25, 64, 128)
    x = torch.randn(2, 64, 1024, generator=torch.Generator().manual_seed(7))
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        y = layer(x.cuda())
    assert y.dtype == torch.bfloat16
    ref = _oracle(layer, x.bfloat16(), layer.weight.detach().cpu().bfloat16().float())
    assert_close_rel(y.float().cpu(), ref, 1e-2)


def test_output_is_channels_last_view_and_chains():
    """Output [B,C,N] is a view of [B,N,C]; feeding it to the next layer takes the vector path."""
    l1 = _layer(32, 16, 25, 64, 128, seed=2)
    l2 = _layer(16, 16, 9, 128, 64, seed=3)
    x = torch.randn(2, 64, 1024, generator=torch.Generator().manual_seed(8)).bfloat16()
    with torch.no_grad():
        h = l1(x.cuda())
        assert h.stride(1) == 1
        y = l2(torch.relu(h))
    h_ref = _oracle(l1, x, l1.weight.detach().cpu().bfloat16().float()).bfloat16()
    y_ref = _oracle(l2, torch.relu(h_ref), l2.weight.detach().cpu().bfloat16().float())
    assert_close_rel(y.float().cpu(), y_ref, 2e-2)


def test_weight_update_repacks():
    layer = _layer(16, 16, 9, 64, 64)
    x = torch.randn(1, 64, 256, generator=torch.Generator().manual_seed(9)).cuda()
    with torch.no_grad():
        y0 = layer(x)
        layer.weight.mul_(2.0)
        y1 = layer(x)
    assert_close_rel(y1.cpu(), 2 * y0.cpu(), 1e-6)


def test_gradients_flow_and_fp8_has_no_graph():
    """The layer is differentiable (values checked in test_knnconv_bwd.py); the fp8 path is
    forward only: its output carries no autograd graph."""
    layer = _layer(16, 16, 9, 64, 64, bias=True)
    x = torch.randn(1, 64, 256, device="cuda").bfloat16().requires_grad_(True)
    layer(x).float().sum().backward()
    assert x.grad.shape == x.shape and layer.weight.grad.shape == layer.weight.shape
    assert layer.bias.grad.shape == (64,)
    layer.fp8 = True
    y8 = layer(x)
    assert y8.grad_fn is None


def test_c3_large_layer_slice_and_batch_independence():
    """C3 geometry (16384 points, k=25, 256 -> 256, bf16): B=64 launch.

    Oracle on one batch row (the reference algorithm at B=64 needs ~27 GB),
    plus a size-independent property: each row of the B=64 result equals the
    B=1 launch of that row bit for bit.
    """
    layer = _layer(128, 128, 25, 256, 256, seed=11)
    g = torch.Generator().manual_seed(0)
    x = torch.randn(64, 256, 16384, generator=g).bfloat16()
    xd = x.cuda().transpose(1, 2).contiguous().transpose(1, 2)
    with torch.no_grad():
        y = layer(xd)
        for b in (0, 37, 63):
            yb = layer(xd[b:b + 1])
            assert torch.equal(y[b:b + 1], yb), f"row {b} differs from its B=1 launch"
    ref = _oracle(layer, x[:1], layer.weight.detach().cpu().bfloat16().float())
    assert_close_rel(y[:1].float().cpu(), ref, 1e-2, "C3 row 0")


@pytest.mark.parametrize("c_in,channels_last,dt", [(64, True, torch.bfloat16), (5, False, torch.bfloat16),
                                                   (8, False, torch.float32)])
def test_fused_relu_equals_relu_of_output(c_in, channels_last, dt):
    layer = _layer(32, 16, 25, c_in, 128, bias=True, seed=4)
    x = torch.randn(2, c_in, 1024, generator=torch.Generator().manual_seed(10)).to(dt).cuda()
    if channels_last:
        x = x.transpose(1, 2).contiguous().transpose(1, 2)
    with torch.no_grad():
        y = layer(x)
        yr = layer.forward_fused(x, "relu")
    assert torch.equal(yr, torch.relu(y))


def test_patch_embedding_c4_geometry():
    """C4 patch embedding: 16384 log-polar points -> 256 tokens, k=256, 16x16 ref grid, 3 -> 384, bias."""
    from fovi_amd.arch.knnvit import KNNPatchEmbedding
    pe = KNNPatchEmbedding(3, 384, 128, 16, 2.78, style="logpolar", auto_match_cart_resources=0,
                           cart_patch_size=16, patch_overlap_factor=2, new_parameterization=True, transposed=True,
                           sample_cortex=True, ref_frame_side_length=16, device="cuda", bias=True)
    assert pe._k == 256 and pe.ref_coords.shape[0] == 256 and pe.out_coords.shape[0] == 256
    g = torch.Generator().manual_seed(12)
    with torch.no_grad():
        pe.weight.copy_(torch.randn(pe.weight.shape, generator=g) * (1.0 / 768) ** 0.5)
        pe.bias.copy_(torch.randn(384, generator=g) * 0.1)
    x = torch.rand(3, 3, 16384, generator=g).bfloat16()
    with torch.no_grad():
        y = pe(x.cuda())
    assert y.shape == (3, 384, 256)
    ref = _oracle(pe, x, pe.weight.detach().cpu().bfloat16().float())
    assert_close_rel(y.float().cpu(), ref, 1e-2)
    pe.transposed = False
    with torch.no_grad():
        assert pe(x.cuda()).shape == (3, 256, 384)


def test_alexnet_chain_c2_geometry():
    """C2 network (5 layers, 64/192/384/256/256, k=49/25/9/9/9, strides 2,2,1,1,1, ReLU between)
    against the oracle chain with bf16 rounding between layers, as autocast does."""
    from fovi_amd.arch.knnalexnet import KNNAlexNet
    net = KNNAlexNet(64, 3, [64, 192, 384, 256, 256], [2, 2, 1, 1, 1], [], [49, 25, 9, 9, 9], style="logpolar",
                     norm_type="none", fov=16, cmf_a=2.78, device="cuda", final_activation=False)
    g = torch.Generator().manual_seed(13)
    with torch.no_grad():
        for blk in net.layers:
            c = blk.conv
            c.weight.copy_(torch.randn(c.weight.shape, generator=g) * (1.0 / (c.in_channels * c._k)) ** 0.5)
    x = torch.rand(2, 3, 4096, generator=g).bfloat16()
    with torch.no_grad():
        y = net(x.cuda())
    h = x
    for i, blk in enumerate(net.layers):
        c = blk.conv
        h = _oracle(c, h.float(), c.weight.detach().cpu().bfloat16().float())
        if i < 4:
            h = torch.relu(h)
        h = h.bfloat16()
    assert y.shape == (2, 256, 256)
    assert_close_rel(y.float().cpu(), h.float(), 2e-2)


@pytest.mark.parametrize("c_in,k,side,c_out", [(3, 49, None, 96), (1, 9, None, 96), (4, 25, None, 96),
                                               (6, 25, None, 96), (3, 256, 16, 96), (3, 49, None, 64),
                                               (3, 256, 16, 384), (5, 9, None, 200)])
def test_bf16_few_channels_padded_rows(c_in, k, side, c_out):
    """Few-channel layers, rows padded to 4/8 channels by the producer (no copy) or by the
    layer: the fused kernel (default), the two-pass path (slot sums through a workspace, then a
    dense GEMM) and the single-pass kernel. The fused kernel sums slots in the same order and
    runs the same MFMA sequence as the two-pass path: bit-identical."""
    from fovi_amd import _lib
    res_out = 4 if k == 256 else 16
    layer = _layer(32, res_out, k, c_in, c_out, side, bias=True, seed=7)
    x = torch.randn(3, c_in, 1024, generator=torch.Generator().manual_seed(11)).bfloat16()
    buf, view = layer.padded_input(3)
    view.copy_(x.cuda())
    buf[..., c_in:] = torch.nan          # padding channels must not leak into the result
    with torch.no_grad():
        y_view = layer(view)
        assert _lib.knnconv_last_path() == "bf16 few-channel fused"
        y_copy = layer(x.cuda())
        layer.few_channel_fused = False
        y_two = layer(view)
        assert _lib.knnconv_last_path() == "bf16 few-channel two-pass"
        layer.two_pass_few_channels = False      # single-pass kernel, no workspace
        y_one = layer(view)
        assert _lib.knnconv_last_path() == "bf16 few-channel"
    ref = _oracle(layer, x, layer.weight.detach().cpu().bfloat16().float())
    assert_close_rel(y_view.float().cpu(), ref, 1e-2)
    assert torch.equal(y_view, y_copy)
    assert torch.equal(y_view, y_two), "fused and two-pass few-channel paths differ"
    assert_close_rel(y_one.float().cpu(), ref, 1e-2)


@pytest.mark.parametrize("geom", [(64, 256, 32), (128, 512, 64), (256, 512, 64)])
def test_few_channel_fused_takes_every_geometry_the_host_accepts(geom):
    """Whenever the host builds fused tables for a geometry and output width (its mirror of the
    kernel's wave tilings and LDS layout says they fit), the library launches the fused kernel
    for them, and its output equals the two-pass path's bit for bit."""
    from fovi_amd import _lib
    x = torch.randn(2, 5, 1024, generator=torch.Generator().manual_seed(3)).bfloat16().cuda()
    accepted = 0
    for c_out in (32, 64, 96, 128, 160, 200, 256, 320, 384, 512):
        layer = _layer(32, 16, 9, 5, c_out, None, bias=True, seed=c_out)
        layer.set_few_channel_geometry([geom])
        if layer._fc is None:
            continue
        accepted += 1
        with torch.no_grad():
            y = layer(x)
            assert _lib.knnconv_last_path() == "bf16 few-channel fused", (geom, c_out)
            layer.few_channel_fused = False
            y_two = layer(x)
        assert torch.equal(y, y_two), (geom, c_out)
    assert accepted >= 6, accepted


@pytest.mark.parametrize("res_in,res_out,k,side,c_in,c_out,bsz,act", [
    (128, 16, 256, 16, 3, 384, 64, None),     # C4 patch embedding
    (128, 16, 256, 16, 3, 384, 300, None),    # a partial block of 128 images
    (64, 32, 49, None, 3, 64, 256, "relu"),   # C2 layer 1
    (32, 16, 25, None, 5, 96, 40, None),      # eight-channel rows, three 32-channel blocks
    (24, 12, 30, None, 4, 200, 33, "relu"),   # ragged: padding slots, 200 = 7 blocks (+1 zero block)
    (32, 16, 25, None, 2, 64, 40, None),      # two channels of four-channel rows (masked sums)
    (32, 16, 25, None, 1, 32, 17, "relu"),    # one channel
    (48, 12, 64, 8, 3, 96, 20, None),         # 8 x 8 ref grid: collisions on every point
])
def test_view_major_kernel_equals_the_two_pass_path(res_in, res_out, k, side, c_in, c_out, bsz, act):
    """Few-channel input written view-major (padded_input(..., view_major=True): the rows of
    one point for all images adjacent) takes the view-major kernel; its output equals the
    two-pass path on the same input and the point-major fused kernel on the same values bit for
    bit (same grouped slot sums, same MFMA order; skipped steps add +0), and two images match
    the oracle."""
    from fovi_amd import _lib
    layer = _layer(res_in, res_out, k, c_in, c_out, side, bias=True, seed=13)
    n_in = layer.in_coords.shape[0]
    x = torch.randn(bsz, c_in, n_in, generator=torch.Generator().manual_seed(14)).bfloat16()
    buf, view = layer.padded_input(bsz, view_major=True)
    assert buf.shape == (n_in, bsz, layer.padded_channels) and view.stride(0) == layer.padded_channels
    buf[..., c_in:] = torch.nan          # padding channels must not leak into the result
    view.copy_(x.cuda())
    with torch.no_grad():
        y = layer(view) if act is None else layer._launch(view, act)
        assert _lib.knnconv_last_path() == "bf16 few-channel view-major"
        layer.view_major_kernel = False
        y_two = layer(view) if act is None else layer._launch(view, act)
        assert _lib.knnconv_last_path() == "bf16 few-channel two-pass"
        _, pm = layer.padded_input(bsz)
        pm.copy_(x.cuda())
        y_pm = layer(pm) if act is None else layer._launch(pm, act)
        assert _lib.knnconv_last_path() == "bf16 few-channel fused"
    assert torch.equal(y, y_two), "view-major and two-pass paths differ"
    assert torch.equal(y, y_pm), "view-major and point-major kernels differ"
    w = layer.weight.detach().cpu().bfloat16().float()
    for b in (0, bsz - 1):
        ref = _oracle(layer, x[b:b + 1], w)
        if act == "relu":
            ref = torch.relu(ref)
        assert_close_rel(y[b:b + 1].float().cpu(), ref, 1e-2, f"image {b}")


def test_view_major_kernel_is_not_used_with_non_finite_weights():
    """A skipped reduction step adds nothing only for finite weights (0 x inf is NaN): with an
    infinite weight the layer takes the two-pass path, which multiplies every column."""
    from fovi_amd import _lib
    layer = _layer(64, 32, 49, 3, 64, None, bias=False, seed=15)
    with torch.no_grad():
        layer.weight[0, 5] = float("inf")
    _, view = layer.padded_input(4, view_major=True)
    view.copy_(torch.rand(4, 3, layer.in_coords.shape[0]).bfloat16().cuda())
    with torch.no_grad():
        layer(view)
    assert _lib.knnconv_last_path() == "bf16 few-channel two-pass"


@pytest.mark.parametrize("geom", [(64, 256, 32), (128, 512, 64)])
def test_few_channel_fused_c4_patch_embedding_geometry(geom):
    """C4 patch embedding (16384 -> 256 log-polar points, k = 256, 16 x 16 ref grid, 3 -> 384,
    bias) at 64 views: the fused kernel at each tile geometry (64 points / 256 threads / 32
    columns, two workgroups per CU; 128 / 512 / 64) equals the two-pass path bit for bit, and
    views 0 and 63 match the oracle."""
    from fovi_amd import _lib
    layer = _layer(128, 16, 256, 3, 384, 16, bias=True, seed=9)
    layer.set_few_channel_geometry([geom])
    assert layer._fc is not None and (layer._fc[0], layer._fc[4], layer._fc[5]) == geom
    x = torch.rand(64, 3, 16384, generator=torch.Generator().manual_seed(12)).bfloat16()
    _, view = layer.padded_input(64)
    view.copy_(x.cuda())
    with torch.no_grad():
        y = layer(view)
        assert _lib.knnconv_last_path() == "bf16 few-channel fused"
        layer.few_channel_fused = False
        y_two = layer(view)
    assert torch.equal(y, y_two)
    w = layer.weight.detach().cpu().bfloat16().float()
    for v in (0, 63):
        assert_close_rel(y[v:v + 1].float().cpu(), _oracle(layer, x[v:v + 1], w), 1e-2, f"view {v}")


@pytest.mark.parametrize("res_in,res_out,k,c_in,c_out,bias,act,batch", [
    (16, 16, 9, 32, 256, True, None, 3),      # one channel chunk
    (16, 16, 9, 96, 512, False, "relu", 2),   # three chunks, two channel tiles
    (24, 12, 25, 64, 256, True, None, 3),     # strided: 144 outputs (one partial point tile)
    (16, 16, 25, 64, 256, False, None, 2),    # k = 25 on a small lattice (seam-heavy tiles)
    (128, 128, 25, 256, 256, False, None, 2), # C3 geometry
    (24, 12, 25, 64, 192, True, "relu", 4),   # one 256-channel tile, 192 real channels
    (16, 16, 9, 192, 384, False, None, 3),    # C2 layer 3: two tiles, 384 real
    (32, 16, 25, 64, 192, True, "relu", 3),   # C2 layer 2: one tile reads all 1024 input rows
])
def test_fragment_order_kernel(res_in, res_out, k, c_in, c_out, bias, act, batch):
    """Wide bf16 layers take the fragment-order (256 x 256 tile) kernel; it matches the oracle
    and the row-packed kernel."""
    layer = _layer(res_in, res_out, k, c_in, c_out, bias=bias, seed=12)
    layer.mfma_weights = True
    x = torch.randn(batch, c_in, res_in * res_in, generator=torch.Generator().manual_seed(13)).bfloat16()
    xd = x.cuda().transpose(1, 2).contiguous().transpose(1, 2)
    with torch.no_grad():
        y = layer.forward_fused(xd, act) if act else layer(xd)
        assert layer.last_weight_layout == "mfma"
        layer.mfma_weights = False
        y_rows = layer.forward_fused(xd, act) if act else layer(xd)
        assert layer.last_weight_layout == "rows"
    ref = _oracle(layer, x, layer.weight.detach().cpu().bfloat16().float())
    if act:
        ref = torch.relu(ref)
    assert_close_rel(y.float().cpu(), ref, 1e-2, "fragment-order kernel vs oracle")
    assert_close_rel(y.float().cpu(), y_rows.float().cpu(), 1e-2, "fragment-order vs row-packed kernel")
    # visiting the slots in order 0, 1, ...: the same fp32 slot sums (in list order, one
    # rounding) and the same MFMA accumulation order as the row-packed kernel, bit for bit
    layer.mfma_weights = True
    layer.set_slot_order(None)
    with torch.no_grad():
        y_plain = layer.forward_fused(xd, act) if act else layer(xd)
    assert layer.last_weight_layout == "mfma"
    assert torch.equal(y_plain, y_rows), "fragment-order (plain slot order) and row-packed kernels differ"


def test_fragment_order_kernel_falls_back_when_tables_exceed_lds():
    """k = 49 (7x7 ref grid): the tile's tables do not fit the fragment-order kernel's LDS, so the
    layer keeps the row-packed kernel."""
    layer = _layer(32, 16, 49, 64, 256, seed=14)
    layer.mfma_weights = True
    x = torch.randn(2, 64, 1024, generator=torch.Generator().manual_seed(15)).bfloat16()
    xd = x.cuda().transpose(1, 2).contiguous().transpose(1, 2)
    with torch.no_grad():
        y = layer(xd)
    assert layer.last_weight_layout == "rows"
    ref = _oracle(layer, x, layer.weight.detach().cpu().bfloat16().float())
    assert_close_rel(y.float().cpu(), ref, 1e-2)


def test_wide_tables_for_another_tile_count_are_refused():
    """The wide-layer tables name collision-tile destinations for one tile count; a call that
    states another count than the kernel's rule for the table sizes is an error, before any
    launch. C3's tables (four tiles) and C2 layer 2's are both checked; the right count runs."""
    from fovi_amd import _lib
    lib = _lib.load()
    for geom in ((128, 128, 25, 256, 256), (32, 16, 25, 64, 192)):
        layer = _layer(*geom, seed=16)
        x = torch.randn(2, geom[3], geom[0] ** 2, generator=torch.Generator().manual_seed(17)).bfloat16()
        xd = x.cuda().transpose(1, 2).contiguous().transpose(1, 2)
        a, y, keep = layer.launch_args(xd)
        assert a.w_layout == _lib.W_MFMA and a.wide_tiles in (3, 4)
        good = a.wide_tiles
        a.wide_tiles = 7 - good
        assert lib.fovi_knnconv_fwd(a, _lib.stream_handle(xd.device)) != 0
        assert b"collision tiles" in lib.fovi_last_error()
        a.wide_tiles = good
        _lib.check(lib.fovi_knnconv_fwd(a, _lib.stream_handle(xd.device)), "fovi_knnconv_fwd")
        torch.cuda.synchronize()
        with torch.no_grad():
            assert torch.equal(y, layer(xd).transpose(1, 2))
        del keep


# Kernel path each benchmark geometry selects (fovi_knnconv_last_path), with the oracle check
# for the paths no other test reaches on purpose.
_SELECTION = [
    # name, (res_in, res_out, k, c_in, c_out, side), input, expected path
    ("C1 fp32", (64, 64, 9, 3, 64, None), "f32", "f32"),
    ("C1 bf16", (64, 64, 9, 3, 64, None), "bf16", "bf16 few-channel fused"),
    ("C2 layer 1", (64, 32, 49, 3, 64, None), "bf16", "bf16 few-channel fused"),
    ("C2 layer 2", (32, 16, 25, 64, 192, None), "bf16", "bf16 v5"),
    ("bf16 rows, no wide tables", (32, 16, 25, 64, 64, None), "bf16", "bf16 v4"),
    ("C2 layer 3", (16, 16, 9, 192, 384, None), "bf16", "bf16 v5"),
    ("C2 layer 4", (16, 16, 9, 384, 256, None), "bf16", "bf16 v5"),
    ("C2 layer 5", (16, 16, 9, 256, 256, None), "bf16", "bf16 v5"),
    ("C3", (128, 128, 25, 256, 256, None), "bf16", "bf16 v5"),
    ("C4 patch embedding", (128, 16, 256, 3, 384, 16), "bf16", "bf16 few-channel fused"),
    ("C5", (128, 128, 25, 256, 256, None), "fp8", "fp8 v5"),
    ("fp8, narrow output", (32, 16, 25, 64, 64, None), "fp8", "fp8 rows"),
    ("bf16 channel-major", (32, 16, 25, 64, 192, None), "bf16 channel-major", "bf16 generic"),
    ("bf16 rows, c_in % 32 != 0", (16, 16, 9, 48, 64, None), "bf16", "bf16 generic"),
    ("bf16 rows, k = 256", (32, 4, 256, 64, 96, 16), "bf16", "bf16 generic (rows)"),
    ("bf16 without tile tables", (32, 16, 25, 64, 192, None), "bf16 no tiles", "bf16 v2"),
]


@pytest.mark.parametrize("name,geom,mode,path", _SELECTION, ids=[s[0] for s in _SELECTION])
def test_kernel_selection(name, geom, mode, path):
    from fovi_amd import _lib
    res_in, res_out, k, c_in, c_out, side = geom
    layer = _layer(res_in, res_out, k, c_in, c_out, side, bias=True)
    if mode == "bf16 no tiles":
        layer.tile_lo = None            # a caller without the tile tables
        layer.mfma_weights = False
    x = torch.randn(1, c_in, res_in * res_in, generator=torch.Generator().manual_seed(21))
    xd = x.cuda()
    if mode == "f32":
        run = lambda: layer(xd)
    elif mode == "fp8":
        xq = layer.quantize_input(xd.bfloat16().transpose(1, 2).contiguous().transpose(1, 2))
        run = lambda: layer(xq)
    else:
        xd = xd.bfloat16()
        if mode != "bf16 channel-major":
            xd = xd.transpose(1, 2).contiguous().transpose(1, 2)
        run = lambda: layer(xd)
    with torch.no_grad():
        y = run()
    assert _lib.knnconv_last_path() == path, f"{name}: took {_lib.knnconv_last_path()!r}"
    if path in ("bf16 v2", "bf16 generic (rows)", "bf16 generic", "fp8 rows"):
        if path == "fp8 rows":
            return          # the row-packed e4m3 kernel: tests/test_gpu_fp8.py
        ref = _oracle(layer, x.bfloat16(), layer.weight.detach().cpu().bfloat16().float())
        assert_close_rel(y.float().cpu(), ref, 1e-2, name)
