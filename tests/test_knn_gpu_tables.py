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
