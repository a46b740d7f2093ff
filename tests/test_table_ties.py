"""Host tables on any host: the reference-written tables or tie flips of them.

The neighbour and ref-slot tables come from torch CPU calls (``cdist``'s matrix-product form,
``topk``'s heap selection, vector ``exp``/``atan2``/``cos``), whose last-bit rounding depends on
the CPU. On the host that wrote ``tests/golden`` the tables are bit-identical (``test_golden.py``,
``test_isotropic.py``, ``test_dinov3_adapter.py``); on another host (the GPU box's) an entry
may differ. This test shows that every difference is a tie, which the reference itself would
break the same way on that host, and not a mistake:

* a neighbour index that differs from the reference's at rank j of output n has the same
  distance there, recomputed in float64 from the coordinates (the reference's metric: the
  wrapped log-polar lattice, ``knn.py:130-141``, or Euclidean ``cdist`` over points and pad
  ring, ``knn.py:117-119,143``), within the fp32 rounding bound of that distance; rank by rank,
  so a changed member at the k-th place is a tie too;
* a ref slot that differs for the same neighbour is, in float64 (``knn.py:599-647``), a nearest
  ref point within 1e-4 of the nearest for both tables' neighbourhoods (the slot flagger's
  margin), and every slot either table holds is such a near-nearest one;
* a point of a partition that sits in another group is as near to both centres
  (``knnvit.py:164-186``);
* sensor coordinates differ by at most what one rounding of the fp32 ``exp`` that makes the
  ring radii can move them: the radius is ``exp(w) - a`` divided by ``fov / 2``, so a unit in
  the last place of ``exp(w)`` (at most ``fov / 2 + a``) shifts a small inner-ring coordinate
  by many of its own units in the last place (bound ``CART_ULPS_OF_EXP`` of those units,
  plus the point's own fp32 rounding).
Counts of differing entries are printed per config. The ``gpu``-marked copies run these same
checks in the GPU suite, on the GPU box's host.
"""
import os

import numpy as np
import pytest
import torch

from fovi_amd.arch import knn_tables as T
from fovi_amd.arch.knn import KNNConvLayer
from fovi_amd.arch.knnvit import KNNPartitioningPatchEmbedding, PartitioningPatchEmbedding
from fovi_amd.sensing.coords import SamplingCoords

GOLD_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
LP = np.load(os.path.join(GOLD_DIR, "tables.npz"))
ISO = np.load(os.path.join(GOLD_DIR, "isotropic.npz"))
DINO = np.load(os.path.join(GOLD_DIR, "dinov3.npz"))

EPS = 2.0 ** -24          # fp32 unit roundoff
SLOT_TIE = 1e-4           # the GPU slot flagger's margin between a neighbour's two nearest ref points
CART_ULPS_OF_EXP = 2      # sensor coordinates: units in the last place of exp(w) a ring radius may move

LP_LAYERS = {"c1": (64, 64, 9, None), "c2_l1": (64, 32, 49, None), "c2_l2": (32, 16, 25, None),
             "c2_l3": (16, 16, 9, None), "ragged": (24, 12, 30, None), "c4_patch": (128, 16, 256, 16),
             "c3": (128, 128, 25, None)}
ISO_LAYERS = {"iso_16_8": ("isotropic", 16, 8, 9, True), "iso_24_12": ("isotropic", 24, 12, 25, True),
              "iso_16_16": ("isotropic", 16, 16, 9, True), "vis_iso_16_8": ("isotropic", 16, 8, 9, False),
              "vis_lp_16_8": ("logpolar", 16, 8, 9, False)}
PATCH = {"part_a05": (PartitioningPatchEmbedding, 0.5, 16), "kpart_a05": (KNNPartitioningPatchEmbedding, 0.5, 16),
         "kpart_a2786": (KNNPartitioningPatchEmbedding, 2.785765, 8)}
DINO_ARGS = dict(in_channels=3, embed_dim=384, in_res=64, fov=16.0, cmf_a=2.785765, style="isotropic",
                 auto_match_cart_resources=True, in_cart_res=64, max_coord_val="auto", arch_flag="",
                 sample_cortex=True, force_patches_less_than_matched=False, ref_frame_side_length=16,
                 transposed=True, bias=True, cart_patch_size=8)

SUITES = [pytest.param("host", id="host"), pytest.param("box", id="box", marks=pytest.mark.gpu)]


def _np64(t):
    return t.detach().cpu().double().numpy()


def _lp_distances(layer):
    """[N_in, N_out] float64 wrapped log-polar distances of the search (``knn.py:110-141``):
    both point sets min-max normalised per column; the angle difference d becomes max - d where
    it passes half the range."""
    src = _np64(layer.sample_coords)
    out = _np64(layer.out_coords.cortical)
    dst = (out - out.min(0)) / (out.max(0) - out.min(0))
    d_r = np.abs(src[:, None, 0] - dst[None, :, 0])
    d_t = np.abs(src[:, None, 1] - dst[None, :, 1])
    hi, lo = src[:, 1].max(), src[:, 1].min()
    d_t = np.where(d_t > lo + (hi - lo) / 2, hi - d_t, d_t)
    return np.sqrt(d_r ** 2 + d_t ** 2), np.full_like(d_r, 8 * EPS)


def _eu_distances(src, out):
    """[N_in, N_out] float64 Euclidean distances and each one's fp32 error bound: torch's
    ``cdist`` computes |x|^2 + |y|^2 - 2 x.y in fp32 above 25 rows, a squared-distance error of
    a few units of EPS (|x|^2 + |y|^2), which the square root turns into at most
    min(delta / (2 d), sqrt(delta))."""
    d = np.sqrt(((src[:, None, :] - out[None, :, :]) ** 2).sum(-1))
    nx, ny = (src ** 2).sum(1), (out ** 2).sum(1)
    delta = 16 * EPS * (nx[:, None] + ny[None, :])
    sq = np.minimum(delta / np.maximum(2 * d, 1e-300), np.sqrt(delta))
    return d, sq + 2 * EPS * (np.sqrt(nx)[:, None] + np.sqrt(ny)[None, :])


def _distances(layer):
    if layer.in_coords.style == "logpolar" and layer.sample_cortex:
        return _lp_distances(layer)
    src = _np64(layer.sample_coords)
    out = _np64(layer.out_coords.cortical if layer.sample_cortex else layer.out_coords.cartesian)
    return _eu_distances(src, out)


def _tie_bound(d, extra):
    return 8 * EPS * d + extra


def check_index_ties(D, B, got, want, cols=None):
    """Rank by rank, a differing neighbour has the reference's neighbour's distance (float64)
    within the fp32 bound; returns the number of differing entries."""
    got = np.asarray(got, np.int64)
    want = np.asarray(want, np.int64)
    cols = np.arange(got.shape[1]) if cols is None else np.asarray(cols)
    assert got.shape == want.shape, (got.shape, want.shape)
    diff = got != want
    for j, c in zip(*np.nonzero(diff)):
        n = cols[c]
        a, b = got[j, c], want[j, c]
        da, db = D[a, n], D[b, n]
        tol = _tie_bound(max(da, db), max(B[a, n], B[b, n]))
        assert abs(da - db) <= tol, (f"output {n} rank {j}: input {a} at {da!r} vs the reference's {b} at "
                                     f"{db!r} (bound {tol:.3g})")
    return int(diff.sum())


def _local_rf64(layer, idx_col, n):
    """[k, V] float64 distances from each neighbour's local coordinate to the ref points for
    output n with neighbour list ``idx_col`` (``knn.py:612-640``): Cartesian angle, cortical
    radius (0 for -1 partition padding), min-max normalised over the neighbourhood."""
    ref = _np64(layer.ref_coords)
    idx = np.asarray(idx_col, np.int64)
    if not layer.sample_cortex:
        local = _np64(layer.sample_coords)[idx] - 0.0
    else:
        nb = _np64(layer.sample_coords)[idx]
        nb_cart = _np64(layer.sample_coords_cart)[idx]
        oc = _np64(layer.out_coords.cortical)[n]
        ocart = _np64(layer.out_coords.cartesian)[n]
        theta = np.arctan2(nb_cart[:, 1] - ocart[1], nb_cart[:, 0] - ocart[0])
        r = np.sqrt(((nb - oc) ** 2).sum(1))
        r[idx < 0] = 0
        local = np.stack([r * np.cos(theta), r * np.sin(theta)], 1)
    lo, hi = local.min(0), local.max(0)
    local = 2 * (local - lo) / (hi - lo + 1e-6) - 1
    return np.sqrt(((local[:, None, :] - ref[None, :, :]) ** 2).sum(-1))


def check_slot_ties(layer, idx_got, slots_got, idx_want, slots_want, cols=None):
    """Every slot either table holds where they differ is a nearest ref point within SLOT_TIE
    of the nearest (float64) for its own neighbourhood; where both neighbourhoods are the same
    set, the reference's slot is also near-nearest for this host's. Returns the count of
    differing (output, neighbour) slots."""
    idx_got, idx_want = np.asarray(idx_got, np.int64), np.asarray(idx_want, np.int64)
    slots_got, slots_want = np.asarray(slots_got, np.int64), np.asarray(slots_want, np.int64)
    cols = np.arange(idx_got.shape[1]) if cols is None else np.asarray(cols)
    n_diff = 0
    for c, n in enumerate(cols):
        sg = dict(zip(idx_got[:, c].tolist(), slots_got[c].tolist()))
        sw = dict(zip(idx_want[:, c].tolist(), slots_want[c].tolist()))
        if sg == sw:
            continue
        dg = _local_rf64(layer, idx_got[:, c], n)
        dw = _local_rf64(layer, idx_want[:, c], n)
        same_set = sorted(idx_got[:, c].tolist()) == sorted(idx_want[:, c].tolist())
        for j, i in enumerate(idx_got[:, c].tolist()):
            s = slots_got[c, j]
            assert dg[j, s] <= dg[j].min() + SLOT_TIE, f"output {n} input {i}: slot {s} is not a nearest ref point"
        for j, i in enumerate(idx_want[:, c].tolist()):
            s = slots_want[c, j]
            assert dw[j, s] <= dw[j].min() + SLOT_TIE, f"output {n} input {i}: reference slot {s} is not nearest"
        for j, i in enumerate(idx_got[:, c].tolist()):
            if i in sw and sw[i] != sg[i]:
                n_diff += 1
                if same_set:
                    assert dg[j, sw[i]] <= dg[j].min() + SLOT_TIE, \
                        f"output {n} input {i}: slots {sg[i]} vs the reference's {sw[i]} are not a tie"
    return n_diff


def _ulps(a, b):
    a = np.ascontiguousarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.ascontiguousarray(b, np.float32).view(np.int32).astype(np.int64)
    a = np.where(a < 0, -(a & 0x7FFFFFFF), a)
    b = np.where(b < 0, -(b & 0x7FFFFFFF), b)
    return int(np.abs(a - b).max(initial=0))


@pytest.mark.parametrize("suite", SUITES)
@pytest.mark.parametrize("name", list(LP_LAYERS))
def test_logpolar_tables_are_reference_or_ties(name, suite):
    r_in, r_out, k, side = LP_LAYERS[name]
    cin = SamplingCoords(16, 2.78, r_in, style="logpolar")
    cout = SamplingCoords(16, 2.78, r_out, style="logpolar")
    layer = KNNConvLayer(1, 1, k, cin, cout, device="cpu", ref_frame_side_length=side)
    g = {key.split("__", 1)[1]: LP[key] for key in LP.files if key.startswith(name + "__")}
    ulps = None
    if g["in_cartesian"].dtype.kind == "f":
        got_c, want_c = cin.cartesian.numpy().astype(np.float64), g["in_cartesian"].astype(np.float64)
        ulps = _ulps(got_c, want_c)
        half = 16 / 2
        tol = (CART_ULPS_OF_EXP * float(np.spacing(np.float32(half + 2.78))) / half
               + np.spacing(np.abs(want_c).astype(np.float32)).astype(np.float64))
        worst = float((np.abs(got_c - want_c) - tol).max())
        assert worst <= 0, f"cartesian coordinates beyond the exp rounding bound by {worst:.3g} ({ulps} ulps)"
    D, B = _distances(layer)
    idx, slots = layer.knn_indices.numpy(), layer.slots.numpy()
    if "idx" in g:
        cols, want_idx, want_slots = None, g["idx"], g["slots"]
    else:
        cols, want_idx, want_slots = g["seam_cols"], g["idx_seam"], g["slots_seam"]
        idx, slots = idx[:, cols], slots[cols]
    n_idx = check_index_ties(D, B, idx, want_idx, cols)
    n_slot = check_slot_ties(layer, idx, slots, want_idx, want_slots, cols)
    print(f"{name}: {n_idx} of {idx.size} indices and {n_slot} slots differ, all ties; "
          f"cartesian {ulps} ulps", flush=True)


@pytest.mark.parametrize("suite", SUITES)
@pytest.mark.parametrize("name", list(ISO_LAYERS))
def test_isotropic_and_visual_tables_are_reference_or_ties(name, suite):
    style, r_in, r_out, k, cortex = ISO_LAYERS[name]
    cin, cout = SamplingCoords(16, 2.78, r_in, style=style), SamplingCoords(16, 2.78, r_out, style=style)
    layer = KNNConvLayer(1, 1, k, cin, cout, device="cpu", sample_cortex=cortex)
    D, B = _distances(layer)
    idx, slots = layer.knn_indices.numpy(), layer.slots.numpy()
    n_idx = check_index_ties(D, B, idx, ISO[f"{name}__idx"])
    n_slot = check_slot_ties(layer, idx, slots, ISO[f"{name}__idx"], ISO[f"{name}__slots"])
    # the distances the layer keeps are the float64 ones within the bound
    d32 = layer.knn_distances.numpy().astype(np.float64)
    d64 = np.take_along_axis(D, idx, 0)
    b64 = np.take_along_axis(B, idx, 0)
    assert np.all(np.abs(d32 - d64) <= _tie_bound(d64, b64))
    print(f"{name}: {n_idx} of {idx.size} indices and {n_slot} slots differ, all ties", flush=True)


def check_partition_ties(layer, want_idx):
    """Partitioning layers: a point in another group than the reference's is as near to both
    centres (float64, within the fp32 bound)."""
    D, B = _distances(layer)
    got, want = layer.knn_indices.numpy(), np.asarray(want_idx, np.int64)
    n_in = layer.in_coords.shape[0]

    def groups(t):
        g = np.full(n_in, -1)
        r, c = np.nonzero((t >= 0) & (t < n_in))
        g[t[r, c]] = c
        return g
    gg, gw = groups(got), groups(want)
    moved = np.flatnonzero(gg != gw)
    for i in moved:
        a, b = gg[i], gw[i]
        tol = _tie_bound(max(D[i, a], D[i, b]), max(B[i, a], B[i, b]))
        assert abs(D[i, a] - D[i, b]) <= tol, f"point {i}: centres {a} and {b} are not a tie"
    return len(moved)


@pytest.mark.parametrize("suite", SUITES)
@pytest.mark.parametrize("name", list(PATCH) + ["dino_kpart", "dino_part"])
def test_patch_embedding_tables_are_reference_or_ties(name, suite):
    if name.startswith("dino"):
        cls = KNNPartitioningPatchEmbedding if name == "dino_kpart" else PartitioningPatchEmbedding
        layer, gold = cls(device="cpu", **DINO_ARGS), DINO
    else:
        cls, cmf_a, patch = PATCH[name]
        layer = cls(3, 8, 64, 16, cmf_a, in_cart_res=64, cart_patch_size=patch, device="cpu", sample_cortex=True)
        gold = ISO
    assert layer._k == int(gold[f"{name}__k"]), f"k {layer._k} vs the reference's {int(gold[f'{name}__k'])}"
    want_idx, want_slots = gold[f"{name}__idx"].astype(np.int64), gold[f"{name}__slots"].astype(np.int64)
    if isinstance(layer, PartitioningPatchEmbedding):
        n_idx = check_partition_ties(layer, want_idx)
        what = "points in another group"
    else:
        D, B = _distances(layer)
        n_idx = check_index_ties(D, B, layer.knn_indices.numpy(), want_idx)
        what = "indices"
    n_slot = check_slot_ties(layer, layer.knn_indices.numpy(), layer.slots.numpy(), want_idx, want_slots)
    print(f"{name}: {n_idx} {what} and {n_slot} slots differ, all ties", flush=True)


def test_planted_mistakes_are_caught():
    """The checks fail on what a bug would produce: a neighbour replaced by a farther one, a
    slot moved to a ref point that is not near-nearest, a point moved to a far centre."""
    name = "c2_l3"
    cin = SamplingCoords(16, 2.78, 16, style="logpolar")
    layer = KNNConvLayer(1, 1, 9, cin, cin, device="cpu")
    D, B = _distances(layer)
    idx, slots = layer.knn_indices.numpy().copy(), layer.slots.numpy().copy()
    assert check_index_ties(D, B, idx, LP[f"{name}__idx"]) >= 0
    bad = idx.copy()
    bad[4, 100] = int(np.argsort(D[:, 100])[40])          # the 41st nearest instead of a 5th
    with pytest.raises(AssertionError, match="rank 4"):
        check_index_ties(D, B, bad, LP[f"{name}__idx"])
    bad_s = slots.copy()
    bad_s[100, 0] = (bad_s[100, 0] + 4) % 9                # the centre neighbour moved off its slot
    with pytest.raises(AssertionError, match="not a nearest"):
        check_slot_ties(layer, idx, bad_s, LP[f"{name}__idx"], LP[f"{name}__slots"])
    part = PartitioningPatchEmbedding(3, 8, 64, 16, 0.5, in_cart_res=64, cart_patch_size=16, device="cpu",
                                      sample_cortex=True)
    want = ISO["part_a05__idx"].astype(np.int64).copy()
    r, c = np.nonzero(want >= 0)
    want[r[0], c[0]], want[r[-1], c[-1]] = want[r[-1], c[-1]], want[r[0], c[0]]   # swap two groups' points
    with pytest.raises(AssertionError, match="not a tie"):
        check_partition_ties(part, want)
