"""Host tables against vectors the reference itself computed (tests/golden/tables.npz,
written by tests/golden/make_golden.py from fovi/sensing/coords.py and
fovi/arch/knn.py). Bit-exact: sensor coordinates, kNN indices (including the
topk tie order at the angle seam, knn.py:137-146) and ref-slot assignment
(including near-equidistant argmin choices, knn.py:637-642)."""
import hashlib
import os

import numpy as np
import pytest

from tests.helpers import layer_tables

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "tables.npz")
CONFIGS = {
    "c1": (64, 64, 9, None),
    "c2_l1": (64, 32, 49, None),
    "c2_l2": (32, 16, 25, None),
    "c2_l3": (16, 16, 9, None),
    "ragged": (24, 12, 30, None),
    "c4_patch": (128, 16, 256, 16),
    "c3": (128, 128, 25, None),
}


def _digest(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


@pytest.fixture(scope="module")
def golden():
    return dict(np.load(GOLDEN, allow_pickle=False))


def _same(got, want):
    """Array or digest (a 0-d string array) comparison."""
    if want.dtype.kind == "U":
        return _digest(got) == str(want)
    return got.shape == want.shape and np.array_equal(got, want)


@pytest.mark.parametrize("name", list(CONFIGS))
def test_tables_match_reference_vectors(golden, name):
    r_in, r_out, k, side = CONFIGS[name]
    t = layer_tables(r_in, r_out, k, side=side)
    g = {key.split("__", 1)[1]: v for key, v in golden.items() if key.startswith(name + "__")}
    assert _same(t["cin"].cartesian.numpy(), g["in_cartesian"]), "input cartesian coords"
    assert _same(t["cin"].cortical.numpy(), g["in_cortical"]), "input cortical coords"
    assert _same(t["cout"].cortical.numpy(), g["out_cortical"]), "output cortical coords"
    from fovi_amd.arch import knn_tables as T
    ref, _ = T.reference_grid(t["k"], side_length=side)
    assert np.array_equal(ref.numpy(), g["ref_coords"]), "ref grid"
    idx = t["idx"].numpy().astype(np.int32)
    slots = t["slots"].numpy().astype(np.uint8)
    if "idx" in g:
        np.testing.assert_array_equal(idx, g["idx"].astype(np.int32))
        np.testing.assert_array_equal(slots, g["slots"])
    else:
        cols = g["seam_cols"]
        np.testing.assert_array_equal(idx[:, cols], g["idx_seam"].astype(np.int32))
        np.testing.assert_array_equal(slots[cols], g["slots_seam"])
    assert _digest(idx) == str(g["idx_sha256"]), "kNN indices (full array digest)"
    assert _digest(slots) == str(g["slots_sha256"]), "ref slots (full array digest)"


def test_fixture_records_torch_version(golden):
    assert str(golden["torch_version"]).startswith("2.")


@pytest.mark.parametrize("name,res", [("c1", 64), ("c2_l2", 32), ("c2_l3", 16)])
def test_sampling_grid_from_reference_cartesian(golden, name, res):
    """GridSampler.sampling_grid is the grid the reference's _prep_grid_for_grid_sample makes
    from its own sensor points (samplers.py:35-47): bit-identical (x, -y) rows."""
    import torch

    from fovi_amd.sensing.samplers import GridSampler
    from oracle import sampler_ref
    cart = torch.from_numpy(golden[f"{name}__in_cartesian"])
    s = GridSampler(16, 2.78, res, device="cpu", style="logpolar")
    assert torch.equal(s.sampling_grid, sampler_ref.grid_from_cartesian(cart))
