"""kNN-conv backward: the gradients of the reference forward (fovi/arch/knn.py:484-557, taken
by torch autograd in the reference) from the slot-sum and transposed-gather kernels.

CPU: the oracle's autograd gradients pinned by finite differences (gradcheck, float64) and by
the closed form dW = dy^T a (a = the brute-force slot sums); the inverse neighbour table by
brute force; the host decomposition of the backward (slot-major GEMMs, the column permutation
back to c * V + v, the inverse gather) against the oracle's autograd, with pad tokens.
GPU: the layer's backward against the oracle's autograd (fp32 1e-5, bf16 1e-2 relative),
and the two entry points through the C-ABI.
"""
import numpy as np
import pytest
import torch

from fovi_amd import _lib
from fovi_amd.arch import knn_tables as T
from oracle import knnconv_ref
from tests.helpers import assert_close_rel, layer_tables


def _synthetic(n_in=30, n_out=11, k=6, V=4, seed=0, pads=True):
    """A random neighbour table with pad tokens (index >= n_in) and its slots."""
    g = torch.Generator().manual_seed(seed)
    idx = torch.randint(0, n_in, (k, n_out), generator=g)
    if pads:
        idx[k - 1, ::2] = n_in                          # pad tokens read the zero column
        idx[k - 2, ::5] = n_in + 3
    slots = torch.randint(0, V, (n_out, k), generator=g)
    rf = T.slots_to_one_hot(slots, V)
    ptr, nbr = T.csr_tables(idx, slots, n_in, V)
    return idx, slots, rf, ptr, nbr


def _oracle_grads(x, idx, n_in, rf, w, b, dy, relu=False):
    x = x.clone().requires_grad_(True)
    w = w.clone().requires_grad_(True)
    b = b.clone().requires_grad_(True) if b is not None else None
    y = knnconv_ref.knnconv_forward(x, idx, n_in, rf, w, b)
    if relu:
        y = torch.relu(y)
    y.backward(dy)
    return x.grad, w.grad, (b.grad if b is not None else None)


def _slot_sums(x, ptr, nbr, V):
    """a[b, n, v * C + c] = sum of x[b, c, i] over the list entries i of slot v (CSR form)."""
    B, C, _ = x.shape
    n_out = ptr.shape[0]
    a = torch.zeros(B, n_out, V, C, dtype=x.dtype)
    p = ptr.numpy().astype(np.int64)
    nb = nbr.numpy()
    for n in range(n_out):
        for v in range(V):
            beg, cnt = p[n, v] >> 16, p[n, v] & 0xFFFF
            for j in range(beg, beg + cnt):
                a[:, n, v] += x[:, :, nb[n, j]]
    return a.reshape(B * n_out, V * C)


# ------------------------------------------------------------------- CPU: pinning ---
def test_oracle_gradients_match_finite_differences():
    idx, _, rf, _, _ = _synthetic(n_in=9, n_out=5, k=4, V=3)
    g = torch.Generator().manual_seed(1)
    x = torch.randn(2, 3, 9, generator=g, dtype=torch.float64, requires_grad=True)
    w = torch.randn(4, 9, generator=g, dtype=torch.float64, requires_grad=True)
    b = torch.randn(4, generator=g, dtype=torch.float64, requires_grad=True)
    assert torch.autograd.gradcheck(lambda x, w, b: knnconv_ref.knnconv_forward(x, idx, 9, rf.double(), w, b),
                                    (x, w, b))


def test_oracle_weight_gradient_closed_form():
    """dW[o, c * V + v] = sum over (b, n) of dy[b, o, n] * a[b, n, v, c] with the slot sums from
    the CSR tables (brute force), and db = dy summed over batch and points."""
    idx, slots, rf, ptr, nbr = _synthetic()
    g = torch.Generator().manual_seed(2)
    x = torch.randn(2, 5, 30, generator=g, dtype=torch.float64)
    w = torch.randn(7, 5 * 4, generator=g, dtype=torch.float64)
    b = torch.randn(7, generator=g, dtype=torch.float64)
    dy = torch.randn(2, 7, 11, generator=g, dtype=torch.float64)
    _, dw, db = _oracle_grads(x, idx, 30, rf.double(), w, b, dy)
    a = _slot_sums(x, ptr, nbr, 4).reshape(2, 11, 4, 5)
    want = torch.einsum("bon,bnvc->ocv", dy, a).reshape(7, 20)
    assert torch.allclose(dw, want, rtol=1e-12, atol=1e-12)
    assert torch.allclose(db, dy.sum((0, 2)), rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("pads", [True, False])
def test_inverse_tables_bruteforce(pads):
    idx, slots, _, ptr, nbr = _synthetic(pads=pads)
    inv_ptr, inv = T.inverse_tables(ptr, nbr, 30, 4)
    assert inv_ptr.dtype == torch.int32 and inv.dtype == torch.int32
    assert inv_ptr.shape == (31,) and inv_ptr[0] == 0 and inv_ptr[-1] == inv.shape[0]
    for i in range(30):
        want = sorted(n * 4 + slots[n, j].item() for n in range(11) for j in range(6) if idx[j, n].item() == i)
        assert inv[inv_ptr[i]:inv_ptr[i + 1]].tolist() == want
    # every real list entry appears once; pad tokens never
    assert inv.shape[0] == int((idx < 30).sum())


@pytest.mark.parametrize("relu", [False, True])
def test_decomposed_backward_matches_oracle_autograd(relu):
    """The backward as the layer runs it -- slot-major a and G = dy W_sm, dW permuted back to
    c * V + v, dx gathered over the inverse table -- restated on the CPU."""
    idx, slots, rf, ptr, nbr = _synthetic()
    n_in, n_out, V, C, C_out, B = 30, 11, 4, 5, 7, 2
    g = torch.Generator().manual_seed(3)
    x = torch.randn(B, C, n_in, generator=g, dtype=torch.float64)
    w = torch.randn(C_out, C * V, generator=g, dtype=torch.float64)
    dy = torch.randn(B, C_out, n_out, generator=g, dtype=torch.float64)
    dx_ref, dw_ref, _ = _oracle_grads(x, idx, n_in, rf.double(), w, None, dy, relu)
    if relu:
        y = knnconv_ref.knnconv_forward(x, idx, n_in, rf.double(), w)
        dy = dy * (y > 0)
    dy2 = dy.permute(0, 2, 1).reshape(B * n_out, C_out)
    a = _slot_sums(x, ptr, nbr, V)
    dw = (dy2.t() @ a).reshape(C_out, V, C).permute(0, 2, 1).reshape(C_out, C * V)
    w_sm = w.reshape(C_out, C, V).permute(0, 2, 1).reshape(C_out, V * C)
    gm = (dy2 @ w_sm).reshape(B, n_out * V, C)
    inv_ptr, inv = T.inverse_tables(ptr, nbr, n_in, V)
    dx = torch.zeros(B, C, n_in, dtype=torch.float64)
    for i in range(n_in):
        for q in range(inv_ptr[i], inv_ptr[i + 1]):
            dx[:, :, i] += gm[:, inv[q]]
    assert torch.allclose(dw, dw_ref, rtol=1e-12, atol=1e-12)
    assert torch.allclose(dx, dx_ref, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("pads", [True, False])
def test_input_gradient_is_the_transposed_conv(pads):
    """dx of the oracle's autograd = the oracle forward over the inverse kNN table
    (knn_tables.inverse_knn) with the weight W_T[c, o V + v] = W[o, c V + v]."""
    idx, slots, rf, ptr, nbr = _synthetic(pads=pads)
    n_in, n_out, V, C, C_out, B = 30, 11, 4, 5, 7, 2
    g = torch.Generator().manual_seed(4)
    x = torch.randn(B, C, n_in, generator=g, dtype=torch.float64)
    w = torch.randn(C_out, C * V, generator=g, dtype=torch.float64)
    dy = torch.randn(B, C_out, n_out, generator=g, dtype=torch.float64)
    dx_ref, _, _ = _oracle_grads(x, idx, n_in, rf.double(), w, None, dy)
    idx_t, slots_t = T.inverse_knn(ptr, nbr, n_in, V)
    assert idx_t.shape[1] == n_in and slots_t.shape == (n_in, idx_t.shape[0])
    assert idx_t.shape[0] == max(int(torch.bincount(idx[idx < n_in].flatten(), minlength=n_in).max()), 1)
    w_t = w.reshape(C_out, C, V).permute(1, 0, 2).reshape(C, C_out * V)
    dx = knnconv_ref.knnconv_forward(dy, idx_t, n_out, T.slots_to_one_hot(slots_t, V).double(), w_t)
    assert torch.allclose(dx, dx_ref, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("pads", [True, False])
@pytest.mark.parametrize("chunk", [256, 4])
def test_slot_pairs_bruteforce_and_weight_gradient(pads, chunk):
    """knn_tables.slot_pairs: segment q * V + v holds the (n, i) list entries in slot v with
    n // chunk == q, output order, padded to 32 with (-1, -1); dW from the pairs equals the
    oracle's autograd."""
    idx, slots, rf, ptr, nbr = _synthetic(pads=pads)
    off, pairs = T.slot_pairs(ptr, nbr, 4, chunk=chunk)
    n_chunks = -(-11 // chunk)
    assert off.numel() == n_chunks * 4 + 1
    assert off[0] == 0 and (off % 32 == 0).all() and pairs.numel() == 2 * off[-1]
    pr = pairs.reshape(-1, 2)
    for q in range(n_chunks):
        for v in range(4):
            want = [(n, idx[j, n].item()) for n in range(q * chunk, min(11, (q + 1) * chunk)) for j in range(6)
                    if slots[n, j].item() == v and idx[j, n].item() < 30]
            got = [tuple(t) for t in pr[off[q * 4 + v]:off[q * 4 + v + 1]].tolist()]
            real = [t for t in got if t[0] >= 0]
            assert sorted(real) == sorted(want) and [t[0] for t in real] == sorted(t[0] for t in real)
            assert all(t == (-1, -1) for t in got[len(real):]) and len(got) - len(real) < 32
    g = torch.Generator().manual_seed(6)
    x = torch.randn(2, 5, 30, generator=g, dtype=torch.float64)
    w = torch.randn(7, 20, generator=g, dtype=torch.float64)
    dy = torch.randn(2, 7, 11, generator=g, dtype=torch.float64)
    _, dw_ref, _ = _oracle_grads(x, idx, 30, rf.double(), w, None, dy)
    dw = torch.zeros(7, 5, 4, dtype=torch.float64)
    for sg in range(n_chunks * 4):
        for n, i in pr[off[sg]:off[sg + 1]].tolist():
            if n >= 0:
                dw[:, :, sg % 4] += dy[:, :, n].t() @ x[:, :, i]
    assert torch.allclose(dw.reshape(7, 20), dw_ref, rtol=1e-12, atol=1e-12)


def test_inverse_tables_of_a_layer_geometry():
    """On a real log-polar layer: counts per input point equal its occurrences in the kNN table."""
    t = layer_tables(32, 16, 25)
    inv_ptr, inv = T.inverse_tables(t["ptr"], t["nbr"], t["n_in"], t["V"])
    idx = t["idx"]
    valid = idx[idx < t["n_in"]]
    want = torch.bincount(valid.flatten(), minlength=t["n_in"])
    assert torch.equal((inv_ptr[1:] - inv_ptr[:-1]).long(), want)
    ent = inv.long()
    n, v = ent // t["V"], ent % t["V"]
    src = torch.repeat_interleave(torch.arange(t["n_in"]), want)
    # each entry (n, v) names an output whose list holds the input in slot v
    assert bool(((idx[:, n] == src) & (t["slots"][n].t() == v)).any(0).all())


# ------------------------------------------------------------------------ GPU ---
def _layer(res_in, res_out, k, c_in, c_out, bias, seed=1):
    from fovi_amd.arch.knn import KNNConvLayer
    from fovi_amd.sensing.coords import SamplingCoords
    cin = SamplingCoords(16, 2.78, res_in, style="logpolar")
    cout = SamplingCoords(16, 2.78, res_out, style="logpolar")
    layer = KNNConvLayer(c_in, c_out, k, cin, cout, device="cuda", bias=bias)
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        layer.weight.copy_(torch.randn(layer.weight.shape, generator=g) * (1.0 / (c_in * layer._k)) ** 0.5)
        if bias:
            layer.bias.copy_(torch.randn(c_out, generator=g) * 0.1)
    return layer


@pytest.mark.gpu
@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("res_in,res_out,k,c_in,c_out,bias,channels_last,relu", [
    (32, 16, 25, 64, 192, False, True, True),     # C2 layer 2 geometry, fused ReLU
    (32, 16, 25, 64, 192, True, False, False),    # channel-major input
    (24, 12, 30, 5, 40, True, False, False),      # ragged: non-square k, odd channels
    (64, 32, 49, 3, 64, False, False, True),      # C2 layer 1 (few channels)
])
@pytest.mark.parametrize("tconv", [True, False], ids=["dx_tconv+dw_fused", "dx_gather+dw_gemm"])
def test_layer_backward_vs_oracle(dt, res_in, res_out, k, c_in, c_out, bias, channels_last, relu, tconv):
    layer = _layer(res_in, res_out, k, c_in, c_out, bias)
    layer.dx_by_transposed_conv = tconv
    layer.dw_fused = tconv
    n_in = res_in * res_in
    g = torch.Generator().manual_seed(7)
    x = torch.randn(2, c_in, n_in, generator=g).to(dt)
    dy = torch.randn(2, c_out, layer.out_coords.shape[0], generator=g)
    xd = x.cuda()
    if channels_last:
        xd = xd.transpose(1, 2).contiguous().transpose(1, 2)
    xd.requires_grad_(True)
    y = layer.forward_fused(xd, "relu") if relu else layer(xd)
    y.backward(dy.to(y.dtype).cuda())
    w = layer.weight.detach().cpu()
    b = layer.bias.detach().cpu() if bias else None
    # the oracle on the operands the kernels saw (bf16-rounded input and weight for bf16)
    w_eff = w.to(dt).float()
    dy_eff = dy.to(y.dtype).float()
    if relu:
        dy_eff = dy_eff * (y.detach().float().cpu() > 0)
    dx_ref, dw_ref, db_ref = _oracle_grads(x.float(), layer.knn_indices.cpu(), n_in, layer.local_rf.cpu(),
                                           w_eff, b, dy_eff)
    tol = 1e-5 if dt == torch.float32 else 1e-2
    assert xd.grad.dtype == dt and xd.grad.shape == x.shape
    assert_close_rel(xd.grad.float().cpu(), dx_ref, tol, "dx")
    assert_close_rel(layer.weight.grad.cpu(), dw_ref, tol, "dW")
    if bias:
        assert_close_rel(layer.bias.grad.cpu(), db_ref, 1e-5 if dt == torch.float32 else 1e-2, "db")
    # the backward's helper objects stay out of the module tree and the state dict
    assert [n for n, _ in layer.named_modules()] == [""]
    assert set(layer.state_dict()) <= {"weight", "bias"}


@pytest.mark.gpu
@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_entry_points_with_pad_tokens_through_the_c_abi(dt):
    """fovi_knnconv_slotsum and fovi_knnconv_bwd_x on a synthetic table with pad tokens,
    against the CPU slot sums and inverse gather."""
    idx, slots, rf, ptr, nbr = _synthetic()
    n_in, n_out, V, C, B = 30, 11, 4, 5, 2
    g = torch.Generator().manual_seed(8)
    x = torch.randn(B, C, n_in, generator=g).to(dt)
    lib = _lib.load()
    xd = x.cuda()
    stream = _lib.stream_handle(xd.device)
    a = torch.empty(B * n_out, V * C, dtype=dt, device="cuda")
    ptr_d, nbr_d = ptr.cuda(), nbr.cuda()
    sa = _lib.SlotsumArgs()
    sa.x = xd.data_ptr(); sa.x_dtype = _lib.dtype_code(dt); sa.a_dtype = _lib.dtype_code(dt)
    sa.batch, sa.c_in, sa.n_in = B, C, n_in
    sa.x_stride[:] = list(xd.stride())
    sa.n_out, sa.k, sa.n_ref = n_out, nbr.shape[1], V
    sa.slot_ptr = ptr_d.data_ptr(); sa.nbr_sorted = nbr_d.data_ptr(); sa.a = a.data_ptr()
    _lib.check(lib.fovi_knnconv_slotsum(sa, stream), "fovi_knnconv_slotsum")
    torch.cuda.synchronize()
    want_a = _slot_sums(x.double(), ptr, nbr, V)
    assert_close_rel(a.double().cpu(), want_a, 1e-6 if dt == torch.float32 else 1e-2, "slot sums")

    gm = torch.randn(B * n_out, V * C, generator=g).to(dt)
    gd = gm.cuda()
    inv_ptr, inv = T.inverse_tables(ptr, nbr, n_in, V)
    ip_d, inv_d = inv_ptr.cuda(), inv.cuda()
    dx = torch.full((B, C, n_in), float("nan"), dtype=dt, device="cuda")
    ba = _lib.BwdXArgs()
    ba.g = gd.data_ptr(); ba.g_dtype = _lib.dtype_code(dt); ba.dx_dtype = _lib.dtype_code(dt)
    ba.batch, ba.c_in, ba.n_in, ba.n_out, ba.n_ref = B, C, n_in, n_out, V
    ba.inv_ptr = ip_d.data_ptr(); ba.inv = inv_d.data_ptr(); ba.dx = dx.data_ptr()
    ba.dx_stride[:] = list(dx.stride())
    _lib.check(lib.fovi_knnconv_bwd_x(ba, stream), "fovi_knnconv_bwd_x")
    torch.cuda.synchronize()
    gmr = gm.double().reshape(B, n_out * V, C)
    want = torch.zeros(B, C, n_in, dtype=torch.float64)
    for n in range(n_out):
        for j in range(6):
            i = idx[j, n].item()
            if i < n_in:
                want[:, :, i] += gmr[:, n * V + slots[n, j].item()]
    assert_close_rel(dx.double().cpu(), want, 1e-6 if dt == torch.float32 else 1e-2, "dx gather")


@pytest.mark.gpu
@pytest.mark.parametrize("res_in,res_out,k,c_in,c_out,batch,chunk,ipg", [
    (32, 32, 25, 256, 256, 3, 256, 3),    # C3 neighbourhood, one full tile, 4 point chunks, all images
    (32, 32, 25, 256, 256, 3, 4096, 1),   # one chunk, one image per workgroup
    (32, 16, 25, 40, 72, 2, 256, 1),      # partial tiles in both channel axes
    (16, 16, 9, 320, 264, 3, 48, 2),      # two tiles in each axis, 6 chunks (last partial), odd split
])
def test_fused_weight_gradient_vs_oracle(res_in, res_out, k, c_in, c_out, batch, chunk, ipg):
    """fovi_knnconv_dw through the C-ABI against the oracle's autograd dW (bf16 operands,
    fp32 accumulation: 1e-2 relative against the oracle on the bf16-rounded operands)."""
    layer = _layer(res_in, res_out, k, c_in, c_out, False)
    g = torch.Generator().manual_seed(12)
    x = torch.randn(batch, c_in, res_in * res_in, generator=g).bfloat16()
    dy = torch.randn(batch, c_out, layer.out_coords.shape[0], generator=g).bfloat16()
    xd = x.cuda().transpose(1, 2).contiguous().transpose(1, 2)
    dyd = dy.cuda().transpose(1, 2).contiguous().transpose(1, 2)
    v = layer.ref_coords.shape[0]
    pair_off, pairs = T.slot_pairs(layer.slot_ptr.cpu(), layer.nbr_sorted.cpu(), v, chunk=chunk)
    pair_off, pairs = pair_off.cuda(), pairs.cuda()
    n_chunks = (pair_off.numel() - 1) // v
    lib = _lib.load()
    nbytes = lib.fovi_knnconv_dw_workspace_bytes(batch, ipg, n_chunks, c_in, c_out, v)
    ws = torch.empty(nbytes // 4, device="cuda")
    dw = torch.full((c_out, c_in * v), float("nan"), device="cuda")
    a = _lib.KnnConvDwArgs()
    a.x = xd.data_ptr(); a.x_stride[:] = list(xd.stride())
    a.dy = dyd.data_ptr(); a.dy_stride[:] = list(dyd.stride())
    a.batch, a.c_in, a.c_out, a.n_in, a.n_out, a.n_ref = batch, c_in, c_out, res_in * res_in, dy.shape[2], v
    a.pair_off = pair_off.data_ptr(); a.pairs = pairs.data_ptr()
    a.n_chunks = n_chunks
    a.images_per_group = ipg
    a.workspace = ws.data_ptr(); a.workspace_bytes = nbytes
    a.dw = dw.data_ptr()
    _lib.check(lib.fovi_knnconv_dw(a, _lib.stream_handle(xd.device)), "fovi_knnconv_dw")
    torch.cuda.synchronize()
    _, dw_ref, _ = _oracle_grads(x.float(), layer.knn_indices.cpu(), res_in * res_in, layer.local_rf.cpu(),
                                 layer.weight.detach().cpu(), None, dy.float())
    assert_close_rel(dw.cpu(), dw_ref, 1e-2, "fused dW")
    # the layer's own path gives the same
    layer.dw_chunk, layer.dw_images_per_group = chunk, ipg
    assert torch.equal(layer._dw_fused(xd, dyd), dw)
