"""kNN pooling (reference fovi/arch/knn.py:272-394): the oracle pinned on the CPU, the HIP kernel
against it on the GPU."""
import math

import numpy as np
import pytest
import torch

from fovi_amd import _lib
from fovi_amd.arch.knn import KNNPoolingLayer
from fovi_amd.sensing.coords import SamplingCoords
from oracle import knnpool_ref as P
from tests.helpers import assert_close_rel

MODES = ["max", "avg", "sum", "gaussian"]


def _tables(n_in=40, n_out=12, k=5, seed=0, pads=True):
    g = torch.Generator().manual_seed(seed)
    idx = torch.randint(0, n_in, (k, n_out), generator=g)
    if pads:
        idx[k - 1, ::3] = n_in + 2                      # pad tokens
    dist = torch.rand(k, n_out, generator=g)
    dist[0] = 0.0                                      # the nearest neighbour first, as a kNN table has it
    return idx, dist


# ------------------------------------------------------------------- CPU: oracle pinning ---
@pytest.mark.parametrize("mode", MODES)
def test_pool_oracle_matches_bruteforce_with_nans_and_pads(mode):
    idx, dist = _tables()
    x = torch.randn(2, 3, 40, generator=torch.Generator().manual_seed(1), dtype=torch.float64)
    x[0, 1, 5] = float("nan")
    x[1, :, 7] = float("nan")
    w = P.gaussian_weights(dist.double(), 10.0) if mode == "gaussian" else None
    got = P.knnpool_forward(x, idx, 40, mode, w).numpy()
    want = P.knnpool_bruteforce(x, idx, 40, mode, w)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    assert np.allclose(got[ok], want[ok], rtol=1e-12, atol=1e-12)


def test_pool_oracle_closed_forms():
    idx, _ = _tables(pads=False)
    k = idx.shape[0]
    const = torch.full((1, 2, 40), 2.5, dtype=torch.float64)
    for mode, want in (("max", 2.5), ("avg", 2.5), ("sum", 2.5 * k)):
        assert torch.allclose(P.knnpool_forward(const, idx, 40, mode), torch.full((1, 2, 12), want,
                                                                                  dtype=torch.float64))
    ramp = torch.arange(40, dtype=torch.float64).reshape(1, 1, 40)      # x[i] = i
    assert torch.equal(P.knnpool_forward(ramp, idx, 40, "max")[0, 0], idx.max(0).values.double())
    assert torch.allclose(P.knnpool_forward(ramp, idx, 40, "sum")[0, 0], idx.sum(0).double())
    # an all-pad neighbourhood: max -inf, mean NaN, sum 0
    allpad = torch.full((k, 1), 40)
    x = torch.randn(1, 1, 40, dtype=torch.float64)
    assert P.knnpool_forward(x, allpad, 40, "max").item() == -math.inf
    assert math.isnan(P.knnpool_forward(x, allpad, 40, "avg").item())
    assert P.knnpool_forward(x, allpad, 40, "sum").item() == 0.0


def test_gaussian_weights_closed_form():
    _, dist = _tables(n_out=7, k=6)
    sigma = 0.7
    w = P.gaussian_weights(dist.double(), sigma)
    for n in range(7):
        d = [dist[j, n].item() for j in range(6)]
        lo, hi = min(d), max(d)
        e = [math.exp(-((v - lo) / (hi - lo)) ** 2 / (2 * sigma ** 2)) for v in d]
        s = sum(e)
        for j in range(6):
            assert abs(w[j, n].item() - e[j] / (s + 1e-8)) < 1e-12
        assert abs(w[:, n].sum().item() - s / (s + 1e-8)) < 1e-12
        assert w[:, n].argmax().item() == int(np.argmin(d))


def test_pool_layer_attributes_and_tables():
    ci = SamplingCoords(16, 2.78, 32, style="logpolar")
    co = SamplingCoords(16, 2.78, 16, style="logpolar")
    layer = KNNPoolingLayer(9, ci, co, mode="gaussian", device="cpu", gauss_sigma=2.0)
    assert layer._k == 9 and layer.knn_indices.shape == (9, 256) and layer.knn_distances.shape == (9, 256)
    assert torch.equal(layer.nbr_rows, layer.knn_indices_pad_token.t().to(torch.int32))
    assert torch.allclose(layer.gaussian_weights, P.gaussian_weights(layer.knn_distances, 2.0))
    assert torch.equal(layer.weight_rows, layer.gaussian_weights.t().float())
    assert not layer.knn_indices_pad_mask.any()          # log-polar neighbourhoods have no pad ring
    big = KNNPoolingLayer(5000, ci, co, mode="max", device="cpu")
    assert big._k == 1024                                # k clamped to the input size (knn.py:311)


# ------------------------------------------------------------------------- GPU: kernel ---
def _pool_args(x, nbr_rows, weights, n_out, k, mode, y):
    a = _lib.KnnPoolArgs()
    a.x = x.data_ptr(); a.x_dtype = _lib.dtype_code(x.dtype); a.mode = mode
    a.batch, a.channels, a.n_in = x.shape
    a.x_stride[:] = list(x.stride())
    a.nbr = nbr_rows.data_ptr()
    a.weights = weights.data_ptr() if weights is not None else None
    a.n_out, a.k = n_out, k
    a.y = y.data_ptr(); a.y_dtype = _lib.dtype_code(y.dtype)
    a.y_stride[:] = list(y.stride())
    return a


@pytest.mark.gpu
@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("channels_last", [True, False])
@pytest.mark.parametrize("k", [9, 25])     # channels-last: k <= 16 gathers every row first, k = 25 loops
def test_knnpool_layer_vs_oracle(mode, dt, channels_last, k):
    ci = SamplingCoords(16, 2.78, 32, style="logpolar")
    co = SamplingCoords(16, 2.78, 16, style="logpolar")
    layer = KNNPoolingLayer(k, ci, co, mode=mode, device="cuda", gauss_sigma=3.0)
    x = torch.randn(3, 64, 1024, generator=torch.Generator().manual_seed(4)).to(dt)
    x[1, 5, 100:140] = float("nan")                                   # NaN features are skipped
    xd = x.cuda()
    if channels_last:
        xd = xd.transpose(1, 2).contiguous().transpose(1, 2)
    with torch.no_grad():
        y = layer(xd)
    want_dt = torch.float32 if mode == "gaussian" else dt             # the reference promotes
    assert y.dtype == want_dt and y.shape == (3, 64, 256)
    assert (y.stride(1) == 1) == channels_last
    w = layer.gaussian_weights.cpu() if mode == "gaussian" else None
    ref = P.knnpool_forward(x.float(), layer.knn_indices.cpu(), 1024, mode, w)
    got = y.float().cpu()
    assert torch.equal(torch.isnan(got), torch.isnan(ref))
    ok = ~torch.isnan(ref)
    if mode == "max":
        assert torch.equal(got[ok], ref[ok].to(dt).float())            # a max is exact
    else:
        tol = 1e-5 if want_dt == torch.float32 else 1e-2
        assert_close_rel(got[ok], ref[ok], tol, f"kNN pooling {mode}")


@pytest.mark.gpu
@pytest.mark.parametrize("mode", MODES)
def test_knnpool_pad_tokens_through_the_c_abi(mode):
    """Indices >= n_in read the reference's appended NaN column."""
    idx, dist = _tables(n_in=40, n_out=12, k=5)
    x = torch.randn(2, 8, 40, generator=torch.Generator().manual_seed(2))
    w = P.gaussian_weights(dist, 10.0) if mode == "gaussian" else None
    y = torch.empty(2, 8, 12, device="cuda")
    nbr = idx.t().contiguous().to(torch.int32).cuda()
    wr = w.t().contiguous().cuda() if w is not None else None
    xd = x.cuda()
    a = _pool_args(xd, nbr, wr, 12, 5, {"max": _lib.POOL_MAX, "avg": _lib.POOL_AVG, "sum": _lib.POOL_SUM,
                                        "gaussian": _lib.POOL_GAUSSIAN}[mode], y)
    lib = _lib.load()
    _lib.check(lib.fovi_knnpool_fwd(a, _lib.stream_handle(xd.device)), "fovi_knnpool_fwd")
    torch.cuda.synchronize()
    ref = P.knnpool_forward(x, idx, 40, mode, w)
    assert_close_rel(y.cpu(), ref, 1e-5, f"pad tokens, {mode}")


@pytest.mark.gpu
def test_alexnet_blocks_with_pooling():
    """Blocks with pooling (reference knnalexnet.py:90-127) and the output average pooling
    layer (knnalexnet.py:193-209): the pooled outputs equal the pooling layers applied to the
    block outputs, on the pooled grids."""
    from fovi_amd.arch.knnalexnet import KNNAlexNet
    net = KNNAlexNet(32, 3, [32, 64], [1, 2], [0], [9, 9], out_res=8, style="logpolar", norm_type="none",
                     cmf_a=2.78, device="cuda", auto_match_cart_resources=0)
    assert net.layers[0].pool is not None and net.layers[1].pool is None
    assert isinstance(net.layers[2], KNNPoolingLayer) and net.layers[2].mode == "avg"
    x = torch.rand(2, 3, 1024, generator=torch.Generator().manual_seed(9)).bfloat16().cuda()
    with torch.no_grad():
        h0 = net.layers[0].conv.forward_fused(x, "relu")
        p0 = net.layers[0].pool(h0)
        assert p0.shape[2] == net.layers[0].out_coords.shape[0]
        ref0 = P.knnpool_forward(h0.float().cpu(), net.layers[0].pool.knn_indices.cpu(), h0.shape[2], "max")
        assert torch.equal(p0.float().cpu(), ref0)
        y = net(x)
        h1 = net.layers[1](p0)
        ref = P.knnpool_forward(h1.float().cpu(), net.layers[2].knn_indices.cpu(), h1.shape[2], "avg")
    assert y.shape == (2, 64, net.layers[2].out_coords.shape[0])
    assert_close_rel(y.float().cpu(), ref, 1e-2, "output pooling")


@pytest.mark.gpu
@pytest.mark.parametrize("sampler,mode", [("pooling", "avg"), ("gaussian_pooling", "gaussian")])
def test_knn_grid_samplers_vs_oracle(sampler, mode):
    """RetinalTransform's kNN pooling samplers (reference samplers.py:134-259, retina.py:99-102):
    nearest samples on the dense grid, then kNN pooling onto the sensor grid."""
    from fovi_amd.sensing.retina import RetinalTransform
    from oracle import sampler_ref
    rt = RetinalTransform(16, start_res=64, fov=16, cmf_a=2.78, style="logpolar", sampler=sampler, device="cuda",
                          auto_match_cart_resources=0, res_mult=2)
    s = rt.sampler
    assert s.highres_coords.shape[0] == 4 * s.coords.shape[0] and s.k == 4 and s.pooler.mode == mode
    img = torch.rand(2, 3, 64, 64, generator=torch.Generator().manual_seed(5))
    fix_loc = torch.tensor([[0.5, 0.5], [0.4, 0.6]])
    with torch.no_grad():
        y = rt(img.cuda(), fix_loc, 64)
    dense, _ = sampler_ref.sampler_forward(img, s.sampling_grid.cpu(), fix_loc, np.array([[64, 64]] * 2),
                                           mode="nearest")
    w = s.pooler.gaussian_weights.cpu() if mode == "gaussian" else None
    ref = P.knnpool_forward(dense, s.pooler.knn_indices.cpu(), dense.shape[2], mode, w)
    assert y.shape == (2, 3, s.coords.shape[0])
    assert_close_rel(y.float().cpu(), ref, 1e-5, f"kNN grid sampler ({mode})")


# ------------------------------------------------------------------------------ backward ---
def _oracle_pool_grad(x, idx, n_in, mode, w, dy):
    xg = x.clone().requires_grad_(True)
    y = P.knnpool_forward(xg, idx, n_in, mode, w)
    y.backward(dy)
    return xg.grad


def _bruteforce_pool_grad(x, idx, n_in, mode, w, dy):
    """float64 loop form of the gradient rules: NaN features get nothing; max: the first
    position of the maximum (NaN as -inf); avg: 1 / non-NaN count; sum: 1; gaussian:
    w_j / (sum of the non-NaN weights + 1e-8)."""
    x = np.asarray(x, np.float64)
    B, C, _ = x.shape
    k, n_out = idx.shape
    dx = np.zeros_like(x)
    for b in range(B):
        for c in range(C):
            for n in range(n_out):
                vals = [x[b, c, i] if i < n_in else np.nan for i in idx[:, n].tolist()]
                ok = [not np.isnan(v) for v in vals]
                g = float(dy[b, c, n])
                if mode == "max":
                    m = [v if o else -np.inf for v, o in zip(vals, ok)]
                    j = int(np.argmax(m))                      # first occurrence
                    coef = {j: 1.0}
                elif mode == "avg":
                    cnt = sum(ok)
                    coef = {j: 1.0 / cnt for j in range(k) if ok[j]} if cnt else {}
                elif mode == "sum":
                    coef = {j: 1.0 for j in range(k) if ok[j]}
                else:
                    s = sum(float(w[j, n]) for j in range(k) if ok[j])
                    coef = {j: float(w[j, n]) / (s + 1e-8) for j in range(k) if ok[j]}
                for j, cf in coef.items():
                    i = int(idx[j, n])
                    if i < n_in and ok[j]:
                        dx[b, c, i] += cf * g
    return dx


@pytest.mark.parametrize("mode", MODES)
def test_pool_gradient_rules_match_oracle_autograd(mode):
    """The loop restatement of the gradient equals torch autograd through the oracle forward,
    with NaN features, pad tokens and (max) ties."""
    idx, dist = _tables()
    g = torch.Generator().manual_seed(3)
    x = torch.randint(0, 4, (2, 3, 40), generator=g).double()           # small integers: many ties
    x[0, 1, 5] = float("nan")
    x[1, :, 7] = float("nan")
    dy = torch.randn(2, 3, 12, generator=g, dtype=torch.float64)
    w = P.gaussian_weights(dist.double(), 10.0) if mode == "gaussian" else None
    got = _oracle_pool_grad(x, idx, 40, mode, w, dy).numpy()
    want = _bruteforce_pool_grad(x, idx, 40, mode, w, dy)
    assert np.allclose(got, want, rtol=1e-12, atol=1e-12)
    assert (got[np.isnan(x.numpy())] == 0).all()


@pytest.mark.parametrize("mode", MODES)
def test_pool_oracle_gradcheck(mode):
    idx, dist = _tables(pads=False)
    x = torch.randn(1, 2, 40, generator=torch.Generator().manual_seed(4), dtype=torch.float64,
                    requires_grad=True)
    w = P.gaussian_weights(dist.double(), 10.0) if mode == "gaussian" else None
    assert torch.autograd.gradcheck(lambda t: P.knnpool_forward(t, idx, 40, mode, w), (x,))


def test_inverse_rows_bruteforce():
    from fovi_amd.arch import knn_tables as T
    idx, _ = _tables()
    rows = idx.t().contiguous().to(torch.int32)                       # [n_out, k]
    ptr, inv = T.inverse_rows(rows, 40)
    for i in range(40):
        want = sorted(n * 5 + j for n in range(12) for j in range(5) if rows[n, j].item() == i)
        assert inv[ptr[i]:ptr[i + 1]].tolist() == want
    assert inv.numel() == int((rows < 40).sum())


@pytest.mark.gpu
@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("channels_last", [True, False])
def test_knnpool_layer_backward_vs_oracle(mode, dt, channels_last):
    ci = SamplingCoords(16, 2.78, 32, style="logpolar")
    co = SamplingCoords(16, 2.78, 16, style="logpolar")
    layer = KNNPoolingLayer(9, ci, co, mode=mode, device="cuda", gauss_sigma=3.0)
    g = torch.Generator().manual_seed(8)
    x = torch.randint(0, 6, (2, 16, 1024), generator=g).float().to(dt)   # ties for max
    x[1, 5, 100:140] = float("nan")
    dy = torch.randn(2, 16, 256, generator=g)
    xd = x.cuda()
    if channels_last:
        xd = xd.transpose(1, 2).contiguous().transpose(1, 2)
    xd.requires_grad_(True)
    y = layer(xd)
    y.backward(dy.to(y.dtype).cuda())
    assert xd.grad.dtype == dt and xd.grad.shape == x.shape
    w = layer.gaussian_weights.cpu() if mode == "gaussian" else None
    ref = _oracle_pool_grad(x.float(), layer.knn_indices.cpu(), 1024, mode, w, dy.to(y.dtype).float())
    tol = 1e-5 if dt == torch.float32 else 1e-2
    assert_close_rel(xd.grad.float().cpu(), ref, tol, f"pool backward {mode}")
    if mode in ("max", "sum"):
        # where the gradient lands is exact (the first maximum among ties, NaN features none)
        assert torch.equal(xd.grad.float().cpu() != 0, ref != 0)


@pytest.mark.gpu
@pytest.mark.parametrize("mode", MODES)
def test_knnpool_backward_pad_tokens_through_the_c_abi(mode):
    from fovi_amd.arch import knn_tables as T
    idx, dist = _tables(n_in=40, n_out=12, k=5)
    g = torch.Generator().manual_seed(9)
    x = torch.randint(0, 3, (2, 8, 40), generator=g).float()
    x[0, 2, 11] = float("nan")
    dy = torch.randn(2, 8, 12, generator=g)
    w = P.gaussian_weights(dist, 10.0) if mode == "gaussian" else None
    rows = idx.t().contiguous().to(torch.int32)
    ptr, inv = T.inverse_rows(rows, 40)
    xd, dyd, rd, pd, ivd = x.cuda(), dy.cuda(), rows.cuda(), ptr.cuda(), inv.cuda()
    wr = w.t().contiguous().cuda() if w is not None else None
    state = torch.empty(2 * 12 * 8, device="cuda")
    dx = torch.full((2, 8, 40), float("nan"), device="cuda")
    a = _lib.KnnPoolBwdArgs()
    a.x = xd.data_ptr(); a.x_dtype = _lib.dtype_code(xd.dtype)
    a.mode = {"max": _lib.POOL_MAX, "avg": _lib.POOL_AVG, "sum": _lib.POOL_SUM, "gaussian": _lib.POOL_GAUSSIAN}[mode]
    a.batch, a.channels, a.n_in = 2, 8, 40
    a.x_stride[:] = list(xd.stride())
    a.nbr = rd.data_ptr(); a.weights = wr.data_ptr() if wr is not None else None
    a.n_out, a.k = 12, 5
    a.dy = dyd.data_ptr(); a.dy_dtype = _lib.dtype_code(dyd.dtype); a.dy_stride[:] = list(dyd.stride())
    a.dx_dtype = _lib.dtype_code(dx.dtype)
    a.inv_ptr, a.inv, a.state = pd.data_ptr(), ivd.data_ptr(), state.data_ptr()
    a.dx = dx.data_ptr(); a.dx_stride[:] = list(dx.stride())
    lib = _lib.load()
    _lib.check(lib.fovi_knnpool_bwd(a, _lib.stream_handle(xd.device)), "fovi_knnpool_bwd")
    torch.cuda.synchronize()
    ref = _oracle_pool_grad(x, idx, 40, mode, w, dy)
    assert_close_rel(dx.cpu(), ref, 1e-5, f"pool backward pads {mode}")


@pytest.mark.gpu
def test_alexnet_training_step_backward():
    """A training step through KNNAlexNet (kNN-conv blocks with fused ReLU, max pooling,
    output average pooling): every parameter gets a finite gradient of the right shape, and
    the input gradient equals the one autograd forms layer by layer from the oracles."""
    from fovi_amd.arch.knnalexnet import KNNAlexNet
    net = KNNAlexNet(32, 3, [32, 64], [1, 2], [0], [9, 9], out_res=8, style="logpolar", norm_type="none",
                     cmf_a=2.78, device="cuda", auto_match_cart_resources=0)
    x = torch.rand(2, 3, 1024, generator=torch.Generator().manual_seed(11)).cuda().requires_grad_(True)
    y = net(x)
    y.float().square().sum().backward()
    for name, prm in net.named_parameters():
        assert prm.grad is not None and prm.grad.shape == prm.shape and torch.isfinite(prm.grad).all(), name
    assert x.grad.shape == x.shape and torch.isfinite(x.grad).all() and x.grad.abs().sum() > 0
