"""GPU kNN search (fovi_knn_logpolar) against the host builder (knn_tables.knn_logpolar, the
reference's knn.py:101-152 op sequence with torch's CPU topk): indices and distances bit for bit.

CPU: the selection order the kernel restates -- a size-k max-heap over the inputs in index order
that admits strictly smaller values, then heap-sorted -- equals torch's CPU topk(largest=False)
on tie-heavy data wherever k * 64 <= n (the regime the kernel serves)."""
import numpy as np
import pytest
import torch

from fovi_amd.arch import knn_tables as T
from fovi_amd.sensing.coords import SamplingCoords


def _adjust(a, hole, n, value):
    top = child = hole
    while child < (n - 1) // 2:
        child = 2 * (child + 1)
        if a[child][0] < a[child - 1][0]:
            child -= 1
        a[hole] = a[child]
        hole = child
    if n % 2 == 0 and child == (n - 2) // 2:
        child = 2 * (child + 1)
        a[hole] = a[child - 1]
        hole = child - 1
    parent = (hole - 1) // 2
    while hole > top and a[parent][0] < value[0]:
        a[hole] = a[parent]
        hole = parent
        parent = (hole - 1) // 2
    a[hole] = value


def _heap_topk(vals, k):
    a = [(float(v), j) for j, v in enumerate(vals)]
    for parent in range((k - 2) // 2, -1, -1):
        _adjust(a, parent, k, a[parent])
    for i in range(k, len(a)):
        if a[i][0] < a[0][0]:
            _adjust(a, 0, k, a[i])
    for last in range(k - 1, 0, -1):
        v = a[last]
        a[last] = a[0]
        _adjust(a, 0, last, v)
    return [j for _, j in a[:k]]


def test_heap_selection_is_torch_cpu_topk_order():
    rng = np.random.default_rng(0)
    for _ in range(120):
        n = int(rng.integers(64, 2500))
        k = int(rng.integers(1, n // 64 + 1))
        vals = rng.integers(0, int(rng.integers(2, 40)), n).astype(np.float32)
        _, ti = torch.topk(torch.from_numpy(vals), k, largest=False)
        assert ti.tolist() == _heap_topk(vals, k), (n, k)


def test_device_search_eligibility():
    assert T.knn_logpolar_device_ok(4096, 49) and T.knn_logpolar_device_ok(16384, 256)
    assert not T.knn_logpolar_device_ok(1024, 25) and not T.knn_logpolar_device_ok(1 << 20, 257)


# ------------------------------------------------------------------------------ GPU ---
@pytest.mark.gpu
@pytest.mark.parametrize("res_in,res_out,k", [(64, 64, 9), (64, 32, 49), (128, 128, 25), (128, 16, 256),
                                              (32, 16, 9), (24, 12, 7)])
def test_device_search_equals_host(res_in, res_out, k):
    ci = SamplingCoords(16, 2.78, res_in, style="logpolar")
    co = SamplingCoords(16, 2.78, res_out, style="logpolar")
    hi, hd, hs = T.knn_logpolar(ci.cortical, co.cortical, k)
    gi, gd, gs = T.knn_logpolar_device(ci.cortical, co.cortical, k, "cuda")
    assert torch.equal(gs, hs)
    assert torch.equal(gi, hi), f"indices differ at {int((gi != hi).sum())} entries"
    assert torch.equal(gd, hd)


@pytest.mark.gpu
@pytest.mark.parametrize("seed", [0, 1])
def test_device_search_tie_heavy(seed):
    """Coordinates on a coarse grid: many exactly equal distances, including at the k-th."""
    g = torch.Generator().manual_seed(seed)
    src = torch.randint(0, 9, (3000, 2), generator=g).float() / 8
    dst = torch.randint(0, 9, (700, 2), generator=g).float() / 8
    hi, hd, _ = T.knn_logpolar(src, dst, 40)
    gi, gd, _ = T.knn_logpolar_device(src, dst, 40, "cuda")
    assert torch.equal(gd, hd)
    assert torch.equal(gi, hi), f"indices differ at {int((gi != hi).sum())} entries"


@pytest.mark.gpu
def test_layer_tables_built_on_the_gpu_equal_the_host_build():
    from fovi_amd.arch.knn import KNNConvLayer
    ci = SamplingCoords(16, 2.78, 64, style="logpolar")
    co = SamplingCoords(16, 2.78, 32, style="logpolar")
    gpu = KNNConvLayer(8, 16, 49, ci, co, device="cuda")
    assert gpu._gpu_tables(ci.shape[0])
    cpu = KNNConvLayer(8, 16, 49, ci, co, device="cpu")
    assert torch.equal(gpu.knn_indices.cpu(), cpu.knn_indices)
    assert torch.equal(gpu.knn_distances.cpu(), cpu.knn_distances)
    assert torch.equal(gpu.slots, cpu.slots)
    with pytest.raises(ValueError):
        T.knn_logpolar_device(ci.cortical, co.cortical, 65, "cuda")     # 65 * 64 > 4096


# -------------------------------------------------- ref slots (fovi_local_rf_slots) ---
def _logpolar_case(res_in, res_out, k):
    ci = SamplingCoords(16, 2.78, res_in, style="logpolar")
    co = SamplingCoords(16, 2.78, res_out, style="logpolar")
    idx, _, src = T.knn_logpolar(ci.cortical, co.cortical, k)
    ref, _ = T.reference_grid(k)
    return idx, src, ci.cartesian, co.cortical, co.cartesian, ref


def test_device_slots_eligibility():
    idx = torch.zeros(25, 10, dtype=torch.long)
    assert T.local_rf_slots_device_ok(idx, torch.zeros(5, 2), torch.zeros(25, 2))
    assert T.local_rf_slots_device_ok(idx, torch.zeros(5, 3), torch.zeros(25, 2))
    assert not T.local_rf_slots_device_ok(idx, torch.zeros(5, 2, dtype=torch.float64), torch.zeros(25, 2))
    assert not T.local_rf_slots_device_ok(torch.zeros(257, 10, dtype=torch.long), torch.zeros(5, 2),
                                          torch.zeros(25, 2))


@pytest.mark.gpu
@pytest.mark.parametrize("res_in,res_out,k", [(64, 64, 9), (64, 32, 49), (32, 16, 25), (16, 8, 9),
                                              (128, 128, 25), (128, 16, 256), (24, 12, 7), (8, 4, 9)])
def test_device_slots_equal_host(res_in, res_out, k):
    """Log-polar layers of C1-C4's shapes, both cdist forms of the radius (k <= 25, k > 25) and
    of the ref distances (N_out and V on either side of 25)."""
    args = _logpolar_case(res_in, res_out, k)
    want = T.local_rf_slots(*args)
    got, redone = T.local_rf_slots_device(*args, device="cuda")
    print(f"\n{res_in}->{res_out} k={k}: {redone} of {want.shape[0]} points recomputed on the host")
    assert got.dtype == want.dtype and got.shape == want.shape
    assert torch.equal(got, want), f"slots differ at {int((got != want).sum())} entries"


@pytest.mark.gpu
def test_device_slots_with_padding_entries():
    """Entries < 0 (a partition's padding) read the last point and have radius 0."""
    idx, *rest = _logpolar_case(32, 16, 49)
    g = torch.Generator().manual_seed(5)
    idx = idx.clone()
    cut = torch.randint(20, 50, (idx.shape[1],), generator=g)
    idx[torch.arange(idx.shape[0]).unsqueeze(1) >= cut.unsqueeze(0)] = -1
    want = T.local_rf_slots(idx, *rest)
    got, _ = T.local_rf_slots_device(idx, *rest, device="cuda")
    assert torch.equal(got, want), f"slots differ at {int((got != want).sum())} entries"


@pytest.mark.gpu
@pytest.mark.parametrize("seed", [0, 1])
def test_device_slots_tie_heavy(seed):
    """Points on a coarse lattice: many neighbours fall exactly between two ref points, so the
    host recomputation has work to do."""
    g = torch.Generator().manual_seed(seed)
    src = torch.randint(0, 9, (600, 2), generator=g).float() / 8
    out = torch.randint(0, 9, (80, 2), generator=g).float() / 8
    idx, _, norm = T.knn_logpolar(src, out, 16)
    ref, _ = T.reference_grid(16)
    want = T.local_rf_slots(idx, norm, src, out, out, ref)
    got, redone = T.local_rf_slots_device(idx, norm, src, out, out, ref, device="cuda")
    assert redone > 0
    assert torch.equal(got, want), f"slots differ at {int((got != want).sum())} entries"


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["iso_16_8", "iso_24_12", "iso_16_16"])
def test_device_slots_isotropic_equal_host_build(name):
    """Isotropic layers (3-D cortical coordinates, pad-ring neighbours) built on the GPU: slots
    equal the host build's (which the CPU tests pin to the reference's tests/golden/isotropic.npz
    on the host that wrote it)."""
    from fovi_amd.arch.knn import KNNConvLayer
    r_in, r_out, k = {"iso_16_8": (16, 8, 9), "iso_24_12": (24, 12, 25), "iso_16_16": (16, 16, 9)}[name]
    ci = SamplingCoords(16, 2.78, r_in, style="isotropic")
    co = SamplingCoords(16, 2.78, r_out, style="isotropic")
    layer = KNNConvLayer(1, 1, k, ci, co, device="cuda")
    assert hasattr(layer, "slots_recomputed")
    cpu = KNNConvLayer(1, 1, k, ci, co, device="cpu")
    assert torch.equal(layer.slots, cpu.slots)


# ------------------------------------------- Euclidean search (fovi_knn_euclid_candidates) ---
def _iso_points(res):
    c = SamplingCoords(16, 2.78, res, style="isotropic")
    return torch.cat([c.cortical, c.cortical_pad_coords], 0), c.cortical


def _eu_candidates(src, dst, k):
    """The candidate scan restated on the CPU (fp32 steps as the kernel takes them)."""
    import heapq
    s32, d32 = src.numpy().astype(np.float32), dst.numpy().astype(np.float32)
    norm_max = np.float32(float(torch.linalg.vector_norm(src.double(), dim=1).max()) * (1 + 2 ** -20))
    out = []
    for n in range(d32.shape[0]):
        y = d32[n]
        yn = np.float32(0)
        for t in y:
            yn = np.float32(yn + np.float32(t * t))
        reach = np.float32(norm_max + np.float32(np.sqrt(yn)))
        m2 = np.float32(np.float32(2.0 * 2 ** -20) * reach * reach)
        diff = s32 - y
        sq = np.zeros(s32.shape[0], dtype=np.float32)
        for d in range(s32.shape[1]):
            sq = (sq + diff[:, d] * diff[:, d]).astype(np.float32)
        heap = [-float(v) for v in sq[:k]]
        heapq.heapify(heap)
        cand = list(range(k))
        for i in range(k, sq.shape[0]):
            top = np.float32(-heap[0])
            if sq[i] < np.float32(top + np.float32(m2 + np.float32(top * np.float32(2 ** -20)))):
                cand.append(i)
            if sq[i] < top:
                heapq.heapreplace(heap, -float(sq[i]))
        reach2 = (float(norm_max) + float(np.sqrt(np.float64(y) @ np.float64(y)))) ** 2
        out.append((cand, sq[cand], 4.0 * 2 ** -20 * reach2 * (1 + 2 ** -10)))
    return out


def test_candidate_distances_equal_the_chunk_cdist():
    """Distances of candidate pairs from the grouped host cdist equal the whole chunk's call,
    for chunks above and below the group size (a chunk of one output included)."""
    src, dst = _iso_points(24)
    g = torch.Generator().manual_seed(0)
    n_out = dst.shape[0]
    for step in (n_out, 200, 63, 1):
        for s in range(0, n_out, step)[:6]:
            e = min(s + step, n_out)
            owner = torch.sort(torch.randint(s, e, (400,), generator=g))[0]
            flat = torch.randint(0, src.shape[0], (400,), generator=g)
            got = T._candidate_distances(src, dst, flat, owner, s, e)
            want = torch.cdist(src, dst[s:e])[flat, owner - s]
            assert torch.equal(got, want), (step, s, int((got != want).sum()))


@pytest.mark.parametrize("case", ["iso", "ties"])
def test_euclid_candidates_and_selection_equal_host_topk(case):
    """The candidate scan (restated) keeps every input the host heap admits, and the selection
    replayed over the candidates -- with the host's distances for those _deciding picks and the
    scan's own square-rooted values for the rest -- gives the host's topk bit for bit."""
    if case == "iso":
        src, dst = _iso_points(16)
        dst = dst[::3]
        k = 9
    else:
        g = torch.Generator().manual_seed(3)
        src = torch.randint(0, 5, (1300, 3), generator=g).float() / 4
        dst = torch.randint(0, 5, (40, 3), generator=g).float() / 4
        k = 20
    hi, hd = T.knn_euclidean(src, dst, k)
    full = torch.cdist(src, dst)
    taken = total = 0
    for n, (c, sq, gap) in enumerate(_eu_candidates(src, dst, k)):
        c = torch.tensor(c)
        sq = torch.from_numpy(sq).unsqueeze(0)
        need = T._deciding(sq, torch.ones_like(sq, dtype=torch.bool), k, torch.tensor([gap]), 2 ** -18)[0]
        taken, total = taken + int(need.sum()), total + c.numel()
        # the host's distances where they can decide, the kernel's square-rooted elsewhere
        d = torch.where(need, full[c, n], sq[0].sqrt())
        order = _heap_topk(d.numpy(), k)
        assert c[order].tolist() == hi[:, n].tolist(), n
        assert torch.equal(d[order], hd[:, n])
    assert taken < total


@pytest.mark.gpu
@pytest.mark.parametrize("res_in,res_out,k,batch", [(16, 8, 9, None), (24, 12, 25, None), (16, 16, 9, None),
                                                    (64, 32, 9, None), (64, 64, 25, None), (96, 48, 49, None),
                                                    (64, 32, 9, 500), (64, 32, 9, 1001)])
def test_device_euclid_search_equals_host(res_in, res_out, k, batch):
    """Isotropic cortical points (3-D, pad ring included), the reference's default output
    batching and batchings that leave a short last chunk."""
    src, _ = _iso_points(res_in)
    _, dst = _iso_points(res_out)
    hi, hd = T.knn_euclidean(src, dst, k, batch)
    gi, gd = T.knn_euclidean_device(src, dst, k, "cuda", batch)
    assert torch.equal(gi, hi), f"indices differ at {int((gi != hi).sum())} entries"
    assert torch.equal(gd, hd)


@pytest.mark.gpu
@pytest.mark.parametrize("seed", [0, 1])
def test_device_euclid_search_tie_heavy(seed):
    g = torch.Generator().manual_seed(seed)
    src = torch.randint(0, 5, (3000, 3), generator=g).float() / 4
    dst = torch.randint(0, 5, (500, 3), generator=g).float() / 4
    hi, hd = T.knn_euclidean(src, dst, 40)
    gi, gd = T.knn_euclidean_device(src, dst, 40, "cuda")
    assert torch.equal(gd, hd)
    assert torch.equal(gi, hi), f"indices differ at {int((gi != hi).sum())} entries"


@pytest.mark.gpu
def test_device_euclid_search_visual_field():
    """2-D visual-field points (sample_cortex=False layers)."""
    ci = SamplingCoords(16, 2.78, 64, style="isotropic")
    co = SamplingCoords(16, 2.78, 32, style="isotropic")
    src = torch.cat([ci.cartesian, ci.cartesian_pad_coords], 0)
    hi, hd = T.knn_euclidean(src, co.cartesian, 9)
    gi, gd = T.knn_euclidean_device(src, co.cartesian, 9, "cuda")
    assert torch.equal(gi, hi) and torch.equal(gd, hd)


@pytest.mark.gpu
def test_isotropic_layer_built_on_the_gpu_equals_the_host_build():
    from fovi_amd.arch.knn import KNNConvLayer
    ci = SamplingCoords(16, 2.78, 64, style="isotropic")
    co = SamplingCoords(16, 2.78, 32, style="isotropic")
    gpu = KNNConvLayer(8, 16, 25, ci, co, device="cuda")
    cpu = KNNConvLayer(8, 16, 25, ci, co, device="cpu")
    assert torch.equal(gpu.knn_indices.cpu(), cpu.knn_indices)
    assert torch.equal(gpu.knn_distances.cpu(), cpu.knn_distances)
    assert torch.equal(gpu.slots, cpu.slots)
    assert torch.equal(gpu.slot_ptr.cpu(), cpu.slot_ptr.cpu())


def test_deciding_candidates():
    """The k smallest and everything within the gap of them, and every pair within the gap of
    each other (equal values included), are taken; isolated values above them are not."""
    sq = torch.tensor([[5.0, 1.0, 9.0, 3.0, 3.0, 20.0, 30.0, 30.05, 50.0, 2.05, 0.0]])
    mask = torch.ones_like(sq, dtype=torch.bool)
    mask[0, -1] = False                                   # past the row's count
    need = T._deciding(sq, mask, 2, torch.tensor([0.1]), 0.0)[0].tolist()
    #        5.0    1.0   9.0    3.0   3.0   20.0   30.0  30.05  50.0  2.05   (unused)
    assert need == [False, True, False, True, True, False, True, True, False, True, False]


def test_deciding_candidates_exact_values():
    """Host distance a function of the kernel's value: copies of one value need not be taken,
    but every copy of a value close to a distinct other value is."""
    sq = torch.tensor([[5.0, 1.0, 9.0, 3.0, 3.0, 20.0, 30.0, 30.0, 50.0, 2.05, 0.0, 30.000002, 9.0]])
    mask = torch.ones_like(sq, dtype=torch.bool)
    mask[0, 10] = False
    need = T._deciding(sq, mask, 2, torch.tensor([0.0]), 2 ** -19, exact_values=True)[0].tolist()
    assert need == [False, True, False, False, False, False, True, True, False, True, False, True, False]


@pytest.mark.gpu
@pytest.mark.parametrize("dim,k,offset", [(1, 1, 0.0), (2, 5, 0.0), (3, 16, 1000.0), (2, 64, -300.0)])
def test_device_euclid_search_edge_cases(dim, k, offset):
    """One to three dimensions, k = 1 and k = 64, and points far from the origin, where torch's
    matrix-product cdist cancels (|x|^2 + |y|^2 >> |x - y|^2): the bound on its rounding covers
    it, and the search still equals the host's bit for bit."""
    g = torch.Generator().manual_seed(dim * 100 + k)
    src = torch.rand(64 * k + 37, dim, generator=g) * 3 + offset
    dst = torch.rand(301, dim, generator=g) * 3 + offset
    hi, hd = T.knn_euclidean(src, dst, k)
    gi, gd = T.knn_euclidean_device(src, dst, k, "cuda")
    assert torch.equal(gi, hi), f"indices differ at {int((gi != hi).sum())} entries"
    assert torch.equal(gd, hd)


@pytest.mark.gpu
def test_device_slots_degenerate_neighbourhoods():
    """Neighbourhoods whose points all coincide (radius 0 everywhere: the min-max span is the
    1e-6 guard, and every step is exact on both sides) or nearly coincide (a 1e-6 jitter, which
    the normalisation magnifies), and neighbourhoods on one horizontal line: the slots equal
    the host's."""
    g = torch.Generator().manual_seed(4)
    n_src, n_out, k = 200, 40, 9
    src_c = torch.rand(n_src, 2, generator=g)
    src_c[:50] = 0.5                                   # a cluster of identical points
    src_c[150:] = 0.25 + 1e-6 * torch.rand(50, 2, generator=g)   # a nearly coincident cluster
    src_cart = torch.rand(n_src, 2, generator=g)
    src_cart[50:100, 1] = 0.25                         # points on a horizontal line
    idx = torch.stack([torch.randperm(n_src, generator=g)[:k] for _ in range(n_out)], 1)
    idx[:, :10] = torch.arange(k).unsqueeze(1)         # neighbourhoods inside the cluster
    idx[:, 10:20] = 50 + torch.arange(k).unsqueeze(1) * 3
    idx[:, 20:30] = 150 + torch.arange(k).unsqueeze(1) * 5
    out_c = torch.rand(n_out, 2, generator=g)
    out_c[:10] = 0.5
    out_cart = torch.rand(n_out, 2, generator=g)
    ref, _ = T.reference_grid(k)
    want = T.local_rf_slots(idx, src_c, src_cart, out_c, out_cart, ref)
    got, redone = T.local_rf_slots_device(idx, src_c, src_cart, out_c, out_cart, ref, device="cuda")
    print(f"\n{redone} of {n_out} points recomputed on the host")
    assert torch.equal(got, want), f"slots differ at {int((got != want).sum())} entries"
