"""Host construction of the kNN-conv tables (neighbour indices and ref-grid slots).

Runs once per layer on the host CPU with torch, in the reference's op order so
that neighbour indices and slot ids are bit-identical to the reference's:

* log-polar neighbour search: per-column min-max normalised cortical coords,
  L1 distance per axis, angle axis wrapped to ``max - d`` when ``d`` exceeds
  the half-range, Euclidean combination, ``topk(k, largest=False)``
  (reference ``fovi/arch/knn.py:101-152``). The wrap period is the normalised
  angle range, so angle indices 0 and res-1 of one ring are at distance 0;
  this is reproduced, not corrected;
* generic cortical/cartesian neighbour search with ``torch.cdist``
  (``knn.py:116-120,143``);
* square reference grid ``linspace(-1,1,s)`` x ``linspace(-1,1,s)`` in 'ij'
  order (``knn.py:559-597``);
* slot assignment: neighbour offsets as (cortical distance, cartesian angle),
  per-neighbourhood min-max to [-1,1], nearest ref-grid point by
  ``cdist``/``argmin`` (``knn.py:599-647``).

The device-side format is a slot-major CSR list per output point
(``csr_tables``). Several neighbours often land in one slot (the reference's
one-hot einsum sums them, ``knn.py:505-526``) and many slots stay empty: on
the 128x128 log-polar lattice with k=25, 36% of slots are empty and up to 23
neighbours share a slot near the fovea, so a fixed one-index-per-slot table
cannot represent the operator.
"""
from __future__ import annotations

from typing import NamedTuple

import numpy as np
import torch

from .. import _lib

__all__ = [
    "knn_logpolar",
    "knn_euclidean",
    "reference_grid",
    "local_rf_slots",
    "slots_to_one_hot",
    "csr_tables",
    "tile_tables",
    "direct_tables",
    "TILE_POINTS",
    "few_channel_tables",
    "few_channel_lds_bytes",
]

_PAIR_BUDGET = 500_000_000  # distance-matrix elements per chunk (reference knn.py:43-49)


def default_batch(n_in, n_out):
    """Outputs per distance batch: at most ``_PAIR_BUDGET`` input-output pairs (reference
    ``knn.py:43-52``; ``n_in`` counts the pad ring)."""
    return int(np.minimum(n_out / np.maximum(0.0001, n_in * n_out / _PAIR_BUDGET), n_out))


def _chunk(n_in, n_out, batch_size):
    if batch_size is None:
        batch_size = default_batch(n_in, n_out)
    return max(1, min(batch_size, n_out))


def _minmax01(x):
    lo = x.min(dim=0)[0]
    hi = x.max(dim=0)[0]
    return (x - lo) / (hi - lo)


def _logpolar_prep(in_cortical, out_cortical):
    """Per-column min-max normalised coordinates (reference knn.py:113-114) and the angle
    wrap constants: the largest normalised angle and the half range (knn.py:135-141)."""
    src = _minmax01(in_cortical.clone())
    dst = _minmax01(out_cortical.clone())
    theta_hi = src[:, 1].max()
    theta_half = src[:, 1].min() + (theta_hi - src[:, 1].min()) / 2
    return src, dst, theta_hi, theta_half


def knn_logpolar_device_ok(n_in, k):
    """Whether ``knn_logpolar_device`` applies: the GPU search reproduces the host's tie order
    where torch's CPU topk runs its heap selection (k * 64 <= n_in), for k <= 256."""
    return 1 <= k <= 256 and k * 64 <= n_in


def _deciding(sq, mask, k, gap_abs, gap_rel, exact_values=False):
    """Candidates whose host distance can decide the selection: ``[m, cap]`` bool.

    ``sq`` holds the kernel's squared distances, each within ``gap / 4`` (``gap = gap_abs +
    gap_rel * value``, ``gap_abs`` per row) of what the host's distance squares to. A candidate
    whose value is more than ``gap`` away from every other candidate's compares with each of
    them as the host's values do, and one more than ``gap`` above the k-th smallest is not
    selected: such candidates may take any value that keeps those comparisons (the kernel's
    own, square rooted). The rest -- the k smallest and any within ``gap`` of them, and every
    pair within ``gap`` of each other -- take the host's distances. With ``exact_values`` the
    host's distance is a function of the kernel's value (its square root), so equal values
    stay equal either way and only distinct values within ``gap`` count as close (every copy
    of such a value is taken, so that equal values are treated alike)."""
    v = sq.masked_fill(~mask, float("inf"))
    sv, order = v.sort(dim=1)
    g = gap_abs.unsqueeze(1)
    kth = sv[:, k - 1:k]
    need = v <= kth + g + gap_rel * kth
    step = sv[:, 1:] - sv[:, :-1]
    close = (step <= g + gap_rel * sv[:, 1:]) & torch.isfinite(sv[:, 1:])
    if exact_values:
        close &= step > 0
    near = torch.zeros_like(need)
    near[:, 1:] |= close
    near[:, :-1] |= close
    if exact_values:
        # every copy of a value marked close: a running id of the distinct values in each row
        run = torch.zeros_like(sv, dtype=torch.long)
        run[:, 1:] = torch.cumsum(step != 0, dim=1)
        run += torch.arange(sv.shape[0], device=sv.device).unsqueeze(1) * sv.shape[1]
        marked = torch.zeros(sv.numel(), dtype=torch.bool, device=sv.device)
        marked[run[near]] = True
        near = marked[run]
    need |= torch.zeros_like(need).scatter_(1, order, near)
    return need & mask


def _device_search(run, dst, n_in, k, distances, gap_rel, max_bytes, exact_values=False):
    """Driver of the candidate-and-select GPU searches: ``(indices [k, N_out] int64, distances
    [k, N_out] fp32)`` on the CPU.

    ``run(dst_rows, cap)`` launches a candidate kernel for the output points ``dst_rows`` (a
    device tensor) with room for ``cap`` candidates per point and returns ``(cand_idx [m, cap],
    cand_n [m], cand_sq [m, cap], gap_abs [m])``; ``distances(flat, owner, sq)`` gives the host's
    distances of candidate pairs (input ``flat[j]``, output ``owner[j]``, in output then index
    order, kernel value ``sq[j]``), taken for the candidates ``_deciding`` picks; the others
    keep the square root of the kernel's value. ``fovi_knn_select`` then replays the host's
    selection. The scan emits every input below its running k-th smallest, so a point far in
    index order from the first inputs collects a few hundred: every point first gets room for
    ``max(8k, 4096)`` candidates, and any whose count exceeds that runs again with room for
    every input, so no candidate is ever dropped. Rows go in chunks of at most ``max_bytes``
    of candidate storage."""
    from .. import _lib
    n_out = dst.shape[0]
    dev = dst.device
    idx = torch.empty(k, n_out, dtype=torch.int32)
    dist = torch.empty(k, n_out, dtype=torch.float32)
    lib = _lib.load()
    stream = _lib.stream_handle(dev)

    def one(rows, cap):
        over = []
        chunk = max(1, min(rows.numel(), max_bytes // (cap * 24)))
        lanes = torch.arange(cap, device=dev)
        for a0 in range(0, rows.numel(), chunk):
            r = rows[a0:a0 + chunk]
            m = r.numel()
            contiguous = int(r[-1]) - int(r[0]) + 1 == m
            d_rows = dst[int(r[0]):int(r[0]) + m] if contiguous else dst[r.to(dev)].contiguous()
            cand_idx, cand_n, cand_sq, gap_abs = run(d_rows, cap)
            mask = lanes.unsqueeze(0) < cand_n.unsqueeze(1)
            need = _deciding(cand_sq, mask, k, gap_abs, gap_rel, exact_values)
            counts = need.sum(dim=1).cpu().numpy()
            owner = torch.from_numpy(np.repeat(r.numpy(), counts))
            cand_d = cand_sq.sqrt()
            cand_d[need] = distances(cand_idx[need].cpu().long(), owner, cand_sq[need].cpu()).to(dev)
            del cand_sq, need
            out_i = torch.empty(k, m, dtype=torch.int32, device=dev)
            out_d = torch.empty(k, m, dtype=torch.float32, device=dev)
            sa = _lib.KnnSelectArgs()
            sa.n_out, sa.k, sa.cap = m, k, cap
            sa.cand_idx, sa.cand_d, sa.cand_n = cand_idx.data_ptr(), cand_d.data_ptr(), cand_n.data_ptr()
            sa.idx, sa.dist = out_i.data_ptr(), out_d.data_ptr()
            _lib.check(lib.fovi_knn_select(sa, stream), "fovi_knn_select")
            if contiguous:
                idx[:, int(r[0]):int(r[0]) + m] = out_i.cpu()
                dist[:, int(r[0]):int(r[0]) + m] = out_d.cpu()
            else:
                idx[:, r] = out_i.cpu()
                dist[:, r] = out_d.cpu()
            over.append(r[cand_n.cpu() > cap])
        return torch.cat(over) if over else torch.zeros(0, dtype=torch.long)

    if n_out:
        over = one(torch.arange(n_out), min(n_in, max(8 * k, 4096)))
        if over.numel():
            one(over, n_in)
    return idx.long(), dist


def knn_logpolar_device(in_cortical, out_cortical, k, device, max_bytes=8 << 30):
    """``knn_logpolar`` with the O(N_in N_out) scan on the GPU: the same ``(indices [k, N_out]
    int64, distances [k, N_out] fp32, normalised input coords)``, bit for bit, on the CPU.

    ``fovi_knn_logpolar_candidates`` emits per output point the inputs the host's heap
    selection could admit, with their exact squared distances; their square roots are taken
    here with the host builder's own call (``** (1 / 2)`` on a CPU tensor, whose rounding is
    not always IEEE); ``fovi_knn_select`` replays the selection over them (``_device_search``).
    """
    from .. import _lib
    src, dst, theta_hi, theta_half = _logpolar_prep(in_cortical, out_cortical)
    n_in = src.shape[0]
    if not knn_logpolar_device_ok(n_in, k):
        raise ValueError(f"knn_logpolar_device: needs 1 <= k <= 256 and k * 64 <= n_in (k={k}, n_in={n_in})")
    s_d = src.to(device=device, dtype=torch.float32).contiguous()
    d_d = dst.to(device=device, dtype=torch.float32).contiguous()
    lib = _lib.load()
    stream = _lib.stream_handle(s_d.device)

    def run(rows, cap):
        m = rows.shape[0]
        cand_idx = torch.empty(m, cap, dtype=torch.int32, device=rows.device)
        cand_sq = torch.empty(m, cap, dtype=torch.float32, device=rows.device)
        cand_n = torch.empty(m, dtype=torch.int32, device=rows.device)
        a = _lib.KnnLogpolarArgs()
        a.src, a.dst = s_d.data_ptr(), rows.data_ptr()
        a.n_in, a.n_out, a.k = n_in, m, k
        a.theta_hi, a.theta_half = float(theta_hi), float(theta_half)
        a.cap = cap
        a.cand_idx, a.cand_sq, a.cand_n = cand_idx.data_ptr(), cand_sq.data_ptr(), cand_n.data_ptr()
        _lib.check(lib.fovi_knn_logpolar_candidates(a, stream), "fovi_knn_logpolar_candidates")
        return cand_idx, cand_n, cand_sq, torch.zeros(m, device=rows.device)

    def distances(flat, owner, sq):
        return sq ** (1 / 2)                                   # the host builder's square root

    # the squared distances are exact on both sides and the square roots differ by an ulp or
    # so: values 2^-19 apart (8 ulps of the distance) stay strictly ordered
    idx, dist = _device_search(run, d_d, n_in, k, distances, 2 ** -19, max_bytes, exact_values=True)
    return idx, dist, src


def knn_logpolar(in_cortical, out_cortical, k, batch_size=None):
    """k nearest inputs per output on the wrapped log-polar cortical lattice.

    Returns ``(indices [k, N_out] int64, distances [k, N_out] fp32,
    normalised input cortical coords [N_in, 2])``.
    """
    src, dst, theta_hi, theta_half = _logpolar_prep(in_cortical, out_cortical)
    n_out = dst.shape[0]
    idx = torch.zeros((k, n_out), dtype=torch.long)
    dist = torch.zeros((k, n_out), dtype=torch.float32)
    step = _chunk(src.shape[0], n_out, batch_size)
    for s in range(0, n_out, step):
        e = min(s + step, n_out)
        d_rho = torch.cdist(src[:, 0].unsqueeze(1), dst[s:e, 0].unsqueeze(1), p=1)
        d_theta = torch.cdist(src[:, 1].unsqueeze(1), dst[s:e, 1].unsqueeze(1), p=1)
        wrap = d_theta > theta_half
        d_theta[wrap] = theta_hi - d_theta[wrap]
        d = (d_rho ** 2 + d_theta ** 2) ** (1 / 2)
        vals, inds = torch.topk(d, k, dim=0, largest=False)
        idx[:, s:e] = inds
        dist[:, s:e] = vals
    return idx, dist, src


def knn_euclidean(in_pts, out_pts, k, batch_size=None):
    """k nearest inputs per output by plain Euclidean ``cdist`` over batches of outputs, then
    ``topk`` (reference ``knn.py:119-152``: isotropic cortical manifold or visual field, pad
    ring included in ``in_pts``)."""
    n_out = out_pts.shape[0]
    idx = torch.zeros((k, n_out), dtype=torch.long)
    dist = torch.zeros((k, n_out), dtype=torch.float32)
    step = _chunk(in_pts.shape[0], n_out, batch_size)
    for s in range(0, n_out, step):
        e = min(s + step, n_out)
        vals, inds = torch.topk(torch.cdist(in_pts, out_pts[s:e]), k, dim=0, largest=False)
        idx[:, s:e] = inds
        dist[:, s:e] = vals
    return idx, dist


def knn_euclidean_device_ok(in_pts, k):
    """Whether ``knn_euclidean_device`` applies: fp32 points of 1 to 3 dimensions, 1 <= k <= 256
    and k * 64 <= N_in (where torch's CPU topk runs the heap selection the GPU replays)."""
    return (in_pts.dtype == torch.float32 and in_pts.dim() == 2 and 1 <= in_pts.shape[1] <= 3
            and 1 <= k <= 256 and k * 64 <= in_pts.shape[0])


def _candidate_distances(in_pts, out_pts, flat, owner, s, e, group=256):
    """Host distances of candidate pairs (input ``flat[j]``, output ``owner[j]``), all owners in
    the reference chunk ``[s, e)``, equal to the entries of that chunk's ``cdist(in_pts,
    out_pts[s:e])``: a chunk of fewer than ``group`` outputs is computed whole with that call;
    otherwise each ``group`` consecutive outputs take one ``cdist`` over the union of their
    candidates (at least ``group`` rows and columns, padded with repeats): at such shapes the
    matrix-product form rounds every entry as the whole chunk's call does (a single column or a
    few rows take other BLAS paths, which round differently)."""
    out = torch.empty(flat.numel(), dtype=torch.float32)
    if flat.numel() == 0:
        return out
    if e - s < group:
        d = torch.cdist(in_pts, out_pts[s:e])
        return d[flat, owner - s]
    bounds = np.searchsorted(owner.numpy(), np.minimum(np.arange(s, e + group, group), e))
    flat_np = flat.numpy()
    seen = np.zeros(in_pts.shape[0], dtype=bool)
    where = np.empty(in_pts.shape[0], dtype=np.int64)
    for g, g0 in enumerate(range(s, e, group)):
        a, b = int(bounds[g]), int(bounds[g + 1])
        if a == b:
            continue
        seg = flat_np[a:b]
        seen[seg] = True
        rows = np.flatnonzero(seen)                      # the group's inputs, ascending
        seen[rows] = False
        where[rows] = np.arange(rows.size)
        g1 = min(g0 + group, e)
        cols = np.arange(g0, g0 + group).clip(max=g1 - 1)
        r = rows if rows.size >= group else np.concatenate([rows, np.repeat(rows[:1], group - rows.size)])
        d = torch.cdist(in_pts[torch.from_numpy(r)], out_pts[torch.from_numpy(cols)])
        out[a:b] = d[torch.from_numpy(where[seg]), owner[a:b] - g0]
    return out


def knn_euclidean_device(in_pts, out_pts, k, device, batch_size=None, max_bytes=8 << 30):
    """``knn_euclidean`` with the O(N_in N_out) scan on the GPU: the same ``(indices [k, N_out]
    int64, distances [k, N_out] fp32)``, bit for bit, on the CPU.

    ``fovi_knn_euclid_candidates`` emits per output point, in index order, every input the
    host's heap selection could admit given how far torch's matrix-product ``cdist`` can round
    from the direct distance; their distances are taken here with the host's ``cdist``
    (``_candidate_distances``, over the reference's chunks of ``batch_size`` outputs); and
    ``fovi_knn_select`` replays the selection over them (``_device_search``)."""
    from .. import _lib
    if not knn_euclidean_device_ok(in_pts, k) or out_pts.dtype != torch.float32 or \
            out_pts.shape[-1] != in_pts.shape[1]:
        raise ValueError(f"knn_euclidean_device: needs fp32 points of 1 to 3 dimensions, 1 <= k <= 256 and "
                         f"k * 64 <= n_in (k={k}, n_in={in_pts.shape[0]})")
    in_pts, out_pts = in_pts.contiguous(), out_pts.contiguous()
    if not (torch.isfinite(in_pts).all() and torch.isfinite(out_pts).all()):
        raise ValueError("knn_euclidean_device: coordinates must be finite")
    n_in, n_out, dim = in_pts.shape[0], out_pts.shape[0], in_pts.shape[1]
    s_d = in_pts.to(device)
    d_d = out_pts.to(device)
    src_norm = (torch.linalg.vector_norm(in_pts.double(), dim=1) * (1 + 2 ** -20)).to(device)
    norm_max = float(src_norm.max())
    step = _chunk(n_in, n_out, batch_size)
    lib = _lib.load()
    stream = _lib.stream_handle(s_d.device)

    def run(rows, cap):
        m = rows.shape[0]
        cand_idx = torch.empty(m, cap, dtype=torch.int32, device=rows.device)
        cand_sq = torch.empty(m, cap, dtype=torch.float32, device=rows.device)
        cand_n = torch.empty(m, dtype=torch.int32, device=rows.device)
        a = _lib.KnnEuclidArgs()
        a.src, a.dst = s_d.data_ptr(), rows.data_ptr()
        a.n_in, a.n_out, a.k, a.dim, a.src_norm_max = n_in, m, k, dim, norm_max
        a.cap, a.cand_idx, a.cand_sq, a.cand_n = cap, cand_idx.data_ptr(), cand_sq.data_ptr(), cand_n.data_ptr()
        _lib.check(lib.fovi_knn_euclid_candidates(a, stream), "fovi_knn_euclid_candidates")
        # four times the bound on the matrix-product form's difference, 2^-20 (|x| + |y|)^2, with
        # |x| the row's largest candidate: two values that far apart stay strictly ordered,
        # square roots included
        held = torch.arange(cap, device=rows.device).unsqueeze(0) < cand_n.unsqueeze(1)
        xn = src_norm[cand_idx.clamp(0, n_in - 1).long()].masked_fill(~held, 0).amax(dim=1)
        reach = xn + torch.linalg.vector_norm(rows.double(), dim=1)
        return cand_idx, cand_n, cand_sq, (4.0 * 2 ** -20 * reach * reach).float() * (1 + 2 ** -10)

    def distances(flat, owner, sq):
        out = torch.empty(flat.numel(), dtype=torch.float32)
        if flat.numel() == 0:
            return out
        for s in range((int(owner[0]) // step) * step, int(owner[-1]) + 1, step):
            e = min(s + step, n_out)
            a_, b_ = int(torch.searchsorted(owner, s)), int(torch.searchsorted(owner, e))
            out[a_:b_] = _candidate_distances(in_pts, out_pts, flat[a_:b_], owner[a_:b_], s, e)
        return out

    # the direct form's own rounding, 2^-20 of the value per candidate, four times over
    return _device_search(run, d_d, n_in, k, distances, 2 ** -18, max_bytes)


def reference_grid(k, side_length=None, doubleres=False, dtype=torch.float32):
    """Square ref grid: (coords [s*s, 2], s); slot v = i*s + j at (lin[i], lin[j])."""
    if side_length is None:
        side_length = int(torch.ceil(torch.sqrt(torch.tensor(k))).long())
        if doubleres:
            side_length *= 2
    lin = torch.linspace(-1, 1, side_length)
    grid = torch.stack(torch.meshgrid(lin, lin, indexing="ij"), -1).reshape(-1, 2)
    return grid.to(dtype=dtype), side_length


def local_rf_slots(knn_idx, src_cortical, src_cart, out_cortical, out_cart, ref_coords):
    """Ref slot id ``[N_out, k]`` (int64) of every neighbour.

    ``src_cortical`` is the (normalised) cortical point set the neighbour
    search ran on; ``out_cortical`` is the output set's own cortical coords.
    The per-output radial distance is one ``cdist`` call per output point,
    as the reference makes it, because ``cdist`` switches to its matmul
    formulation above 25 rows and the two formulations round differently.
    """
    k, n_out = knn_idx.shape
    nb = src_cortical[knn_idx]                      # [k, N_out, d]
    nb_cart = src_cart[knn_idx]                     # [k, N_out, 2]
    theta = torch.arctan2(nb_cart[:, :, 1] - out_cart[:, 1], nb_cart[:, :, 0] - out_cart[:, 0])
    radial = torch.empty(n_out, k, dtype=nb.dtype)
    for i in range(n_out):
        radial[i] = torch.cdist(out_cortical[i].unsqueeze(0), nb[:, i]).squeeze(0)
    radial = radial.t()
    radial[knn_idx < 0] = 0
    local = torch.stack([radial * torch.cos(theta), radial * torch.sin(theta)], dim=2)
    lo = local.min(dim=0, keepdim=True)[0]
    hi = local.max(dim=0, keepdim=True)[0]
    local = 2 * (local - lo) / (hi - lo + 1e-6) - 1
    nearest = torch.argmin(torch.cdist(local, ref_coords), dim=2)   # [k, N_out]
    return nearest.t().contiguous()


def local_rf_slots_rows(knn_idx, src_cortical, src_cart, out_cortical, out_cart, ref_coords, rows):
    """``local_rf_slots`` for the output points ``rows`` only: ``[len(rows), k]``, equal to
    those rows of the full computation. Every step is per output point (the per-point
    ``cdist``, ``arctan2``/``cos``/``sin`` element by element, the min-max over a point's
    neighbours) except the final ``cdist`` to the ref grid, whose formula depends on the row
    count (a matrix product above 25 rows): it runs on at least 26 rows, the subset padded
    with copies of its first row, as the full call does for more than 25 output points."""
    rows = torch.as_tensor(rows, dtype=torch.long)
    k, n_out = knn_idx.shape
    if rows.numel() == 0:
        return torch.zeros(0, k, dtype=torch.long)
    sub = knn_idx[:, rows]
    nb = src_cortical[sub]
    nb_cart = src_cart[sub]
    oc, ocart = out_cortical[rows], out_cart[rows]
    theta = torch.arctan2(nb_cart[:, :, 1] - ocart[:, 1], nb_cart[:, :, 0] - ocart[:, 0])
    m = rows.numel()
    radial = torch.empty(m, k, dtype=nb.dtype)
    for i in range(m):
        radial[i] = torch.cdist(oc[i].unsqueeze(0), nb[:, i]).squeeze(0)
    radial = radial.t()
    radial[sub < 0] = 0
    local = torch.stack([radial * torch.cos(theta), radial * torch.sin(theta)], dim=2)
    lo = local.min(dim=0, keepdim=True)[0]
    hi = local.max(dim=0, keepdim=True)[0]
    local = 2 * (local - lo) / (hi - lo + 1e-6) - 1
    pad = 0
    if n_out > 25 and m <= 25:
        pad = 26 - m
        local = torch.cat([local, local[:, :1].expand(k, pad, 2)], dim=1)
    nearest = torch.argmin(torch.cdist(local, ref_coords), dim=2)
    return nearest[:, :m].t().contiguous()


def local_rf_slots_device_ok(knn_idx, src_cortical, ref_coords):
    """Whether ``local_rf_slots_device`` applies: fp32 coordinates of 1 to 3 dimensions,
    k <= 256 neighbours, at most 65536 ref points."""
    k = knn_idx.shape[0]
    return (src_cortical.dtype == torch.float32 and ref_coords.dtype == torch.float32
            and 1 <= src_cortical.shape[1] <= 3 and 1 <= k <= 256 and 1 <= ref_coords.shape[0] <= 65536)


def local_rf_slots_device(knn_idx, src_cortical, src_cart, out_cortical, out_cart, ref_coords, device,
                          tol=1e-4):
    """``local_rf_slots`` with the per-neighbour arithmetic on the GPU: the same ``[N_out, k]``
    int64 slots, bit for bit, on the CPU, and the number of output points recomputed here.

    ``fovi_local_rf_slots`` assigns every neighbour in fp32 and flags each output point where
    some neighbour's two nearest ref points are closer than ``tol`` plus its bound on the
    kernel's difference from this host's arithmetic (its transcendental functions and the
    matrix-product ``cdist`` round differently); those points are recomputed here with
    ``local_rf_slots_rows``, the reference's own calls."""
    from .. import _lib
    if not local_rf_slots_device_ok(knn_idx, src_cortical, ref_coords):
        raise ValueError("local_rf_slots_device: needs fp32 coordinates of 1 to 3 dimensions, k <= 256, "
                         "n_ref <= 65536")
    k, n_out = knn_idx.shape
    lib = _lib.load()
    dev = torch.device(device)
    stream = _lib.stream_handle(dev)
    dim = src_cortical.shape[1]

    def put(t, cols):
        t = t.to(device=dev, dtype=torch.float32).contiguous()
        if t.dim() != 2 or t.shape[1] != cols:
            raise ValueError(f"local_rf_slots_device: coordinate rows of {cols} expected, got {tuple(t.shape)}")
        return t

    sc, scart = put(src_cortical, dim), put(src_cart, 2)
    oc, ocart = put(out_cortical, dim), put(out_cart, 2)
    # the visual-field set may be longer (log-polar layers: the pad ring follows the points)
    if scart.shape[0] < sc.shape[0] or ocart.shape[0] != n_out or oc.shape[0] != n_out:
        raise ValueError("local_rf_slots_device: point counts of the coordinate sets disagree")
    n_src = sc.shape[0]
    if knn_idx.numel() and (int(knn_idx.max()) >= n_src or int(knn_idx.min()) < -1):
        raise ValueError("local_rf_slots_device: neighbour index out of range")
    idx = knn_idx.to(device=dev, dtype=torch.int32).contiguous()
    ref = put(ref_coords, 2)
    slots = torch.empty(n_out, k, dtype=torch.int32, device=dev)
    flags = torch.empty(n_out, dtype=torch.int32, device=dev)
    a = _lib.LocalRfArgs()
    a.src_cortical, a.src_cart, a.n_src, a.dim = sc.data_ptr(), scart.data_ptr(), n_src, dim
    a.out_cortical, a.out_cart, a.n_out = oc.data_ptr(), ocart.data_ptr(), n_out
    a.knn_idx, a.k, a.ref, a.n_ref = idx.data_ptr(), k, ref.data_ptr(), ref.shape[0]
    a.tol = float(tol)
    a.slots, a.flags = slots.data_ptr(), flags.data_ptr()
    _lib.check(lib.fovi_local_rf_slots(a, stream), "fovi_local_rf_slots")
    out = slots.cpu().long()
    rows = torch.nonzero(flags.cpu(), as_tuple=True)[0]
    if rows.numel():
        out[rows] = local_rf_slots_rows(knn_idx, src_cortical, src_cart, out_cortical, out_cart, ref_coords,
                                        rows)
    return out, int(rows.numel())


def visual_rf_slots(knn_idx, src_cart, ref_coords):
    """Ref slot id ``[N_out, k]`` (int64) of every neighbour for visual-field neighbourhoods
    (``sample_cortex=False``): the neighbours' visual (x, y), min-max normalised to [-1, 1]
    per output, nearest ref point (reference ``knn.py:620-647`` without the cortical
    re-projection)."""
    local = src_cart[knn_idx]                         # [k, N_out, 2]
    lo = local.min(dim=0, keepdim=True)[0]
    hi = local.max(dim=0, keepdim=True)[0]
    local = 2 * (local - lo) / (hi - lo + 1e-6) - 1
    nearest = torch.argmin(torch.cdist(local, ref_coords), dim=2)
    return nearest.t().contiguous()


def slots_to_one_hot(slots, n_ref):
    """One-hot ``local_rf [N_out, k, V]`` fp32 (the reference's stored form)."""
    n_out, k = slots.shape
    rf = torch.zeros(n_out, k, n_ref, dtype=torch.float32)
    rf.scatter_(2, slots.unsqueeze(2), 1)
    return rf


def csr_tables(knn_idx, slots, n_in, n_ref):
    """Slot-major CSR neighbour lists, the device format of the kNN-conv kernel.

    Returns ``(slot_ptr [N_out, V] int32, nbr_sorted [N_out, k] int32)``:
    ``slot_ptr[n, v] = (begin << 16) | count`` and the inputs that land in slot
    ``v`` of output ``n`` are ``nbr_sorted[n, begin:begin+count]``, in
    neighbour (distance) order. Pad-token neighbours (``>= n_in``) contribute
    zeros in the reference and are dropped; unused tail entries are ``-1``.
    """
    k, n_out = knn_idx.shape
    if k > 0x7FFF:
        # begin << 16 must stay a non-negative int32: the kernels decode it with a signed shift
        raise ValueError(f"k={k} does not fit the CSR fields (k <= 32767)")
    idx = knn_idx.t().numpy().astype(np.int64)             # [N_out, k]
    sl = slots.numpy().astype(np.int64)
    valid = (idx >= 0) & (idx < n_in)
    key = np.where(valid, sl, n_ref)
    order = np.argsort(key, axis=1, kind="stable")
    nbr = np.take_along_axis(idx, order, axis=1)
    nbr = np.where(np.take_along_axis(valid, order, axis=1), nbr, -1).astype(np.int32)
    counts = np.zeros((n_out, n_ref + 1), dtype=np.int64)
    np.add.at(counts, (np.repeat(np.arange(n_out), k), key.reshape(-1)), 1)
    counts = counts[:, :n_ref]
    begin = np.cumsum(counts, axis=1) - counts
    ptr = ((begin << 16) | counts).astype(np.int32)
    return torch.from_numpy(ptr), torch.from_numpy(nbr)


def inverse_tables(slot_ptr, nbr_sorted, n_in, n_ref):
    """Inverse of the CSR neighbour lists, the input-gradient gather of the backward.

    For every input point i, the entries ``n * n_ref + v`` of the (output point, slot) pairs
    whose list holds i, in increasing order: ``inv[inv_ptr[i]:inv_ptr[i + 1]]``. Returns
    ``(inv_ptr [n_in + 1] int32, inv [E] int32)``.
    """
    ptr = slot_ptr.numpy().astype(np.int64)
    nbr = nbr_sorted.numpy().astype(np.int64)
    n_out = ptr.shape[0]
    cnt = ptr & 0xFFFF
    beg = ptr >> 16
    # the slot of every list position: position j of output n is in slot v when beg <= j < beg + cnt
    k = nbr.shape[1]
    slot_of = np.full((n_out, k), -1, np.int64)
    for v in range(n_ref):
        j = np.arange(k)[None, :]
        inside = (j >= beg[:, v:v + 1]) & (j < beg[:, v:v + 1] + cnt[:, v:v + 1])
        slot_of = np.where(inside, v, slot_of)
    valid = (nbr >= 0) & (nbr < n_in) & (slot_of >= 0)
    ins = nbr[valid]
    ent = (np.arange(n_out)[:, None] * n_ref + slot_of)[valid]
    order = np.lexsort((ent, ins))
    ins, ent = ins[order], ent[order]
    inv_ptr = np.zeros(n_in + 1, np.int64)
    np.add.at(inv_ptr, ins + 1, 1)
    inv_ptr = np.cumsum(inv_ptr)
    return torch.from_numpy(inv_ptr.astype(np.int32)), torch.from_numpy(ent.astype(np.int32))


def slot_pairs(slot_ptr, nbr_sorted, n_ref, chunk=256, step=32):
    """The (output, input) pairs of every slot, the reduction lists of the weight gradient,
    cut into segments of ``chunk`` consecutive output points.

    Returns ``(pair_off [n_chunks * n_ref + 1] int32, pairs [2 * pair_off[-1]] int32)``:
    segment ``q * n_ref + v`` holds slot v's pairs ``(n, i)`` with ``n // chunk == q``, in
    output order and list order within an output, padded with ``(-1, -1)`` to a multiple of
    ``step``.
    """
    ptr = slot_ptr.numpy().astype(np.int64)
    nbr = nbr_sorted.numpy().astype(np.int64)
    n_out, k = nbr.shape
    n_chunks = max(1, -(-n_out // chunk))
    cnt = ptr & 0xFFFF
    beg = ptr >> 16
    j = np.arange(k)[None, None, :]
    inside = (j >= beg[:, :, None]) & (j < (beg + cnt)[:, :, None])           # [n_out, V, k]
    n_idx, v_idx, j_idx = np.nonzero(inside)
    seg_idx = (n_idx // chunk) * n_ref + v_idx
    order = np.lexsort((j_idx, n_idx, seg_idx))
    n_idx, seg_idx, j_idx = n_idx[order], seg_idx[order], j_idx[order]
    i_idx = nbr[n_idx, j_idx]
    counts = np.bincount(seg_idx, minlength=n_chunks * n_ref)
    padded = -(-counts // step) * step
    off = np.concatenate([[0], np.cumsum(padded)])
    pairs = np.full((int(off[-1]), 2), -1, np.int64)
    pos = off[seg_idx] + (np.arange(len(seg_idx)) - np.concatenate([[0], np.cumsum(counts)])[seg_idx])
    pairs[pos, 0] = n_idx
    pairs[pos, 1] = i_idx
    return torch.from_numpy(off.astype(np.int32)), torch.from_numpy(pairs.reshape(-1).astype(np.int32))


def inverse_rows(nbr_rows, n_in):
    """Per input point, the entries ``n * k + j`` of the row-major neighbour table
    ``nbr_rows [N_out, k]`` that hold it (indices outside [0, n_in) dropped), in increasing
    order: ``(inv_ptr [n_in + 1] int32, inv [E] int32)``."""
    nbr = nbr_rows.numpy().astype(np.int64).reshape(-1)
    ent = np.arange(nbr.shape[0], dtype=np.int64)
    ok = (nbr >= 0) & (nbr < n_in)
    nbr, ent = nbr[ok], ent[ok]
    order = np.lexsort((ent, nbr))
    nbr, ent = nbr[order], ent[order]
    ptr = np.zeros(n_in + 1, np.int64)
    np.add.at(ptr, nbr + 1, 1)
    return torch.from_numpy(np.cumsum(ptr).astype(np.int32)), torch.from_numpy(ent.astype(np.int32))


def inverse_knn(slot_ptr, nbr_sorted, n_in, n_ref):
    """The kNN table of the transposed convolution (the input gradient): for every input
    point i, the output points whose lists hold i, with the slot i sits in there.

    Returns ``(idx [k', N_in] int64, slots [N_in, k'] int64)`` in the forward's table format,
    k' the largest number of lists an input point is in (at least 1); shorter columns end in
    the pad token ``N_out``, whose slot is 0.
    """
    inv_ptr, inv = inverse_tables(slot_ptr, nbr_sorted, n_in, n_ref)
    n_out = slot_ptr.shape[0]
    ptr = inv_ptr.numpy().astype(np.int64)
    ent = inv.numpy().astype(np.int64)
    deg = ptr[1:] - ptr[:-1]
    kk = max(int(deg.max()) if n_in else 0, 1)
    pos = np.arange(ent.shape[0]) - np.repeat(ptr[:-1], deg)
    row = np.repeat(np.arange(n_in), deg)
    idx = np.full((n_in, kk), n_out, np.int64)
    sl = np.zeros((n_in, kk), np.int64)
    idx[row, pos] = ent // n_ref
    sl[row, pos] = ent % n_ref
    return torch.from_numpy(np.ascontiguousarray(idx.T)), torch.from_numpy(sl)


TILE_POINTS = 256  # output points per workgroup tile of the staged-row kernel


def tile_tables(knn_idx, slots, n_in, n_ref, tile=TILE_POINTS):
    """Per-tile compact tables for the kernel that stages input rows in LDS.

    Output points are cut into tiles of ``tile`` consecutive points. The
    inputs any point of a tile reads lie in one contiguous index range
    ``[lo, lo + span)`` (on the ring-major log-polar lattice a tile of two
    rings reads about six rings), which the kernel copies into LDS. Returns
    ``(lo [T] int32, span [T] int32, ent [T*tile, V] int32,
    nbr [T*tile, k] uint16)`` where ``ent = (first << 16) | (count << 8) |
    begin`` (``first`` = the slot's first input, relative to ``lo``) and
    ``nbr`` holds input indices relative to ``lo`` in the CSR order of
    ``csr_tables``; or ``None`` when k > 255 or a span exceeds 65535.
    """
    k, n_out = knn_idx.shape
    if k > 255:
        return None
    ptr, nbr = csr_tables(knn_idx, slots, n_in, n_ref)
    ptr = ptr.numpy().astype(np.int64)
    nbr = nbr.numpy().astype(np.int64)
    n_tiles = -(-n_out // tile)
    lo = np.zeros(n_tiles, np.int64)
    span = np.zeros(n_tiles, np.int64)
    nbr_loc = np.zeros((n_tiles * tile, k), np.int64)
    ent = np.zeros((n_tiles * tile, n_ref), np.int64)
    for t in range(n_tiles):
        s, e = t * tile, min((t + 1) * tile, n_out)
        blk = nbr[s:e]
        valid = blk >= 0
        if not valid.any():
            continue
        lo[t] = blk[valid].min()
        span[t] = blk[valid].max() - lo[t] + 1
        nbr_loc[s:e] = np.where(valid, blk - lo[t], 0)
        beg = ptr[s:e] >> 16
        first = np.take_along_axis(nbr_loc[s:e], np.minimum(beg, k - 1), axis=1)
        first = np.where((ptr[s:e] & 0xFFFF) > 0, first, 0)
        ent[s:e] = (first << 16) | ((ptr[s:e] & 0xFFFF) << 8) | beg
    if span.max() > 0xFFFF:
        return None
    return (torch.from_numpy(lo.astype(np.int32)), torch.from_numpy(span.astype(np.int32)),
            torch.from_numpy(ent.astype(np.uint32).view(np.int32)), torch.from_numpy(nbr_loc.astype(np.uint16)))


def direct_tables(knn_idx, slots, n_in, n_ref, tile=TILE_POINTS):
    """Tables of the kernel that reads single-neighbour slots straight from LDS.

    Extends ``tile_tables``: the kernel keeps the staged input rows in LDS plus
    one zero row at index ``zero_row = max span``; a slot with no neighbour
    points at the zero row, a slot with one neighbour at that neighbour's row,
    and only slots with two or more neighbours are summed into a separate
    tile. Returns ``(lo, span, ent, nbr, coll, coll_n, zero_row)`` where
    ``ent [T*tile, V] int32 = (first << 16) | (count << 8) | begin`` (first =
    ``zero_row`` when count is 0), ``coll [T, V, tile] uint8`` lists, per tile
    and slot, the tile rows with count >= 2 in decreasing count order, and
    ``coll_n [T, V] int32`` their number; or ``None`` (see ``tile_tables``).
    """
    base = tile_tables(knn_idx, slots, n_in, n_ref, tile)
    if base is None:
        return None
    lo, span, ent, nbr = base
    zero_row = int(span.max())
    if zero_row >= 0xFFFF:
        return None
    e = ent.numpy().view(np.uint32).astype(np.int64)
    cnt = (e >> 8) & 0xFF
    e = np.where(cnt == 0, (zero_row << 16) | (e & 0xFFFF), e)
    n_tiles = lo.shape[0]
    coll = np.zeros((n_tiles, n_ref, tile), np.uint8)
    coll_n = np.zeros((n_tiles, n_ref), np.int32)
    c3 = cnt.reshape(n_tiles, tile, n_ref)
    for t in range(n_tiles):
        for v in range(n_ref):
            rows = np.nonzero(c3[t, :, v] >= 2)[0]
            rows = rows[np.argsort(-c3[t, rows, v], kind="stable")]
            coll[t, v, :len(rows)] = rows
            coll_n[t, v] = len(rows)
    return (lo, span, torch.from_numpy(e.astype(np.uint32).view(np.int32)), nbr,
            torch.from_numpy(coll), torch.from_numpy(coll_n), zero_row)


class FewChannelTables(NamedTuple):
    lo: torch.Tensor         # [T] int32 first staged input row of tile t
    span: torch.Tensor       # [T] int32 staged rows
    item: torch.Tensor       # [T, n_chunks, threads, pairs] int32 (uint32 pair words)
    pairs: int               # pair words per thread and chunk (FC_PAIR_COUNTS)
    tile: int                # output points per tile
    threads: int             # threads of the kernel's workgroup
    chunk: int               # reduction columns per chunk
    zero_row: int
    comb: torch.Tensor       # [total] int32 (uint32 words): per (tile, chunk) combine entries
    comb_off: torch.Tensor   # [T * n_chunks + 1] int32 block starts
    pmax: int                # most partial sums of one chunk


# Tile geometries of the fused few-channel kernel, (output points, threads, chunk columns), in
# the order a layer tries them (fastest first, measured on the C4 patch embedding and C2
# layer 1: 128 / 512 / 64 0.229 and 0.062 ms, 256 / 512 / 64 -- and 0.073 ms, 64 / 256 / 32,
# two workgroups per CU, 0.329 and 0.085 ms)
FC_GEOMETRIES = ((128, 512, 64), (256, 512, 64), (64, 256, 32))
# Waves along the tile's rows each geometry's kernel is built for, tried in this order (the
# library's FC_GEOMS); the other waves of the workgroup split the output channels
FC_WAVE_ROWS = {(64, 256, 32): (1, 2), (128, 512, 64): (2, 4), (256, 512, 64): (2, 4)}
# Slot sums of few-channel layers run over the neighbour list in groups of this many: each
# group's fp32 sum in list order from +0, the groups' sums added in order (for up to this many
# neighbours, the plain list order). The fused kernel sums the groups of one slot on different
# lanes; the two-pass slot-sum kernel uses the same order.
FC_GROUP = 8
# (sum, neighbour) pairs per thread and chunk in the fused kernel's table: the first of these
# counts whose packing fits the workgroup's threads
FC_PAIR_COUNTS = (8, 16)
FC_LAST = 1 << 29      # pair word flag: the last pair of its sum or partial sum
FC_PARTIAL = 1 << 28   # pair word flag: the run is one group of a long list (an fp32 partial sum)


def _fc_entry(row, slot, cp, chunk):
    """Index, in units of one slot entry (2 cp bytes), of (row, slot) in the fused kernel's A
    tile: rows of 2 ``chunk`` bytes whose 16-byte part q sits at part q ^ ((row >> 1) & 7)
    (128-byte rows) or q ^ g(row), g(r) = (bit1(r) ^ bit3(r)) | bit2(r) << 1 (64-byte rows)."""
    b = slot * cp * 2
    if chunk == 64:
        g = (row >> 1) & 7
    else:
        g = (((row >> 1) ^ (row >> 3)) & 1) | ((row >> 1) & 2)
    off = row * chunk * 2 + (((b >> 4) ^ g) << 4) + (b & 15)
    return off // (2 * cp)


def few_channel_tables(knn_idx, slots, n_in, n_ref, cp, k_pad, tile, threads=512, chunk=64):
    """Tables of the fused few-channel kernel (``knnconv_fewc.hip``; ``fc_*`` in the C-ABI).

    Output points are cut into tiles of ``tile`` consecutive points, each run by a workgroup of
    ``threads`` threads (a geometry of ``FC_GEOMETRIES``); a tile stages input rows ``[lo, lo +
    span)`` and a zero row ``zero_row`` (the largest span). The reduction runs in chunks of
    ``chunk`` columns, ``chunk // cp`` slots each; the kernel clears a chunk's A tile and
    writes only its non-empty (row, slot) sums. They come from (sum, neighbour) pairs,
    ``pairs`` per thread and chunk: word ``j`` of thread ``th`` in chunk ``c`` of tile ``t`` is
    ``item[t, c, th, j]`` = the neighbour's S row (bits 0-15; the zero row for an unused pair)
    | target << 16 | ``FC_PARTIAL`` | ``FC_LAST``. A sum's pairs are consecutive within one
    thread, in CSR list order (``csr_tables``); the thread adds them in fp32 from +0 and, at the
    pair flagged ``FC_LAST``, writes the sum rounded to bf16 to A entry ``target``
    (``_fc_entry``). A slot of more than ``FC_GROUP`` neighbours is one run per group of
    ``FC_GROUP`` (partial flag set) writing an fp32 partial sum to index ``target`` of the
    chunk's partial buffer, and a combine entry ``dest | m << 12 | p0 << 20`` (``dest = row *
    spc + slot``) adds its ``m`` partials ``p0 ..`` in order and writes A. Runs are packed into
    thread segments in (row, slot) order, a run that does not fit a segment's remaining pairs
    going to the next, so every thread issues ``pairs`` independent row reads; ``pairs`` is the
    first of ``FC_PAIR_COUNTS`` for which every chunk fits the threads. The segments are dealt
    round robin over the workgroup's waves. Returns ``None`` when a span does not fit 16 bits,
    or a chunk needs more segments than threads, more combine entries than threads or more
    than 4095 partials.
    """
    for pairs in FC_PAIR_COUNTS:
        ft = _few_channel_tables(knn_idx, slots, n_in, n_ref, cp, k_pad, tile, threads, chunk, pairs)
        if ft != "threads":
            return ft
    return None


def _few_channel_tables(knn_idx, slots, n_in, n_ref, cp, k_pad, tile, threads, chunk, pairs):
    """``few_channel_tables`` at ``pairs`` pair words per thread; "threads" when a chunk needs
    more segments than threads."""
    k, n_out = knn_idx.shape
    spc = chunk // cp
    n_chunks = k_pad // chunk
    per_chunk = tile * spc
    if k_pad % chunk or n_chunks * spc < n_ref or per_chunk > 4096:
        return None
    ptr, nbr = csr_tables(knn_idx, slots, n_in, n_ref)
    ptr = ptr.numpy().astype(np.int64)
    nbr = nbr.numpy().astype(np.int64)
    n_tiles = -(-n_out // tile)
    lo = np.zeros(n_tiles, np.int64)
    span = np.zeros(n_tiles, np.int64)
    for t in range(n_tiles):
        blk = nbr[t * tile:(t + 1) * tile]
        valid = blk >= 0
        if valid.any():
            lo[t] = blk[valid].min()
            span[t] = blk[valid].max() - lo[t] + 1
    zero_row = int(span.max())
    if zero_row >= 0xFFFF:
        return None
    # per (point, padded slot): count, begin
    vpad = n_chunks * spc
    cnt = np.zeros((n_tiles * tile, vpad), np.int64)
    beg = np.zeros((n_tiles * tile, vpad), np.int64)
    cnt[:n_out, :n_ref] = ptr & 0xFFFF
    beg[:n_out, :n_ref] = ptr >> 16
    nbr_pad = np.full((n_tiles * tile, k), -1, np.int64)
    nbr_pad[:n_out] = nbr
    rows_lo = np.repeat(lo, tile)[:, None]
    nbr_rel = np.where(nbr_pad >= 0, nbr_pad - rows_lo, 0)
    G, P = FC_GROUP, pairs
    n_waves = threads // 64
    item = np.full((n_tiles, n_chunks, threads, P), zero_row, np.int64)
    seg = np.arange(threads)
    seg_thread = (seg % n_waves) * 64 + seg // n_waves
    cblocks, coff = [], [0]
    pmax = 0
    for t in range(n_tiles):
        rows = slice(t * tile, (t + 1) * tile)
        nrel = nbr_rel[rows]
        for c in range(n_chunks):
            cols = slice(c * spc, (c + 1) * spc)
            cc = cnt[rows, cols].reshape(-1)            # dest = row * spc + slot
            bb = beg[rows, cols].reshape(-1)
            words = np.full((threads, P), zero_row, np.int64)
            comb = []
            n_part = 0
            th, used = 0, 0
            for d in np.nonzero(cc)[0]:
                n, b0 = int(cc[d]), int(bb[d])
                r, sl = divmod(int(d), spc)
                if n <= G:
                    runs = [(b0, n, _fc_entry(r, sl, cp, chunk), 0)]
                else:
                    m = -(-n // G)
                    if m > 0xFF:
                        return None
                    comb.append(int(d) | (m << 12) | (n_part << 20))
                    runs = [(b0 + g * G, min(G, n - g * G), n_part + g, FC_PARTIAL) for g in range(m)]
                    n_part += m
                for start, gn, target, part in runs:
                    if used + gn > P:
                        th, used = th + 1, 0
                    if th >= threads:
                        return "threads"
                    words[th, used:used + gn] = nrel[r, start:start + gn]
                    words[th, used + gn - 1] |= (target << 16) | part | FC_LAST
                    used += gn
            # thread segments dealt round robin over the waves: segment i to thread
            # (i % waves) * 64 + i // waves, so every wave builds about the same share
            item[t, c, seg_thread] = words
            if len(comb) > threads or n_part > 0xFFF:
                return None
            cblocks.append(np.asarray(comb, np.int64))
            coff.append(coff[-1] + len(comb))
            pmax = max(pmax, n_part)
    comb_all = np.concatenate(cblocks) if cblocks else np.zeros(0, np.int64)
    if len(comb_all) == 0:
        comb_all = np.zeros(1, np.int64)
    return FewChannelTables(
        torch.from_numpy(lo.astype(np.int32)), torch.from_numpy(span.astype(np.int32)),
        torch.from_numpy(item.astype(np.uint32).view(np.int32)), pairs, tile, threads, chunk, zero_row,
        torch.from_numpy(comb_all.astype(np.uint32).view(np.int32)), torch.from_numpy(np.asarray(coff, np.int32)),
        pmax)


def few_channel_lds_bytes(tables, c_out, cp):
    """LDS bytes the fused few-channel kernel needs for these tables and ``c_out`` (its
    layout: staged rows and the zero row, two A chunks, the weight chunk of ``c_out`` rounded
    up to 64 columns, the partial sums, at least the epilogue's transposition buffers), or
    ``1 << 30`` when no wave tiling of the kernel covers ``c_out`` at this geometry or the
    layout passes the workgroup's share of the CU's 160 KB (half for 256 threads, whose
    workgroups run two per CU)."""
    ntp = -(-c_out // 64) * 64
    nw = tables.threads // 64
    # the kernel's wave tilings: wm x (nw / wm) waves of rb x cb blocks of 32 x 32, cb <= 4,
    # rb * cb <= 8, wm among those the geometry is built for
    fits = []
    for wm in FC_WAVE_ROWS.get((tables.tile, tables.threads, tables.chunk), ()):
        if nw % wm or tables.tile % (32 * wm) or ntp % (32 * (nw // wm)):
            continue
        rb, cb = tables.tile // (32 * wm), ntp // (32 * (nw // wm))
        if 1 <= cb <= 4 and rb * cb <= 8:
            fits.append((rb, cb))
    if not fits:
        return 1 << 30
    rb, cb = fits[0]
    s = ((tables.zero_row + 1) * cp * 2 + 15) & ~15
    body = s + 2 * tables.tile * tables.chunk * 2 + ntp * tables.chunk * 2 + tables.pmax * cp * 4
    total = max(body, nw * rb * 32 * cb * 32 * 2)
    return total if total <= (80 if tables.threads == 256 else 160) * 1024 else 1 << 30


# The view-major few-channel kernel (input rows of one point for every image adjacent in memory,
# [N_in, B, CP]): an MFMA block's 32 rows are 32 images of one output point, so a reduction step
# of 16 columns (16 / CP slots) that is empty for the point is skipped for all of them, and each
# lane gathers its image's rows with one load per neighbour.
VM_CHUNK = 8           # rounds per event / index load of the kernel
VM_G, VM_P, VM_S = 1, 2, 4   # event flags: close a group of FC_GROUP; end of phase A; end of the step
VM_X, VM_Q = 8, 16     # step pairings (cp = 4): exchange slots 1 and 2 between the halves; half 1 phases swapped
VM_JSHIFT = 5          # the next step's index sits in bits 5-15 of a step's last event
VM_J_NONE = 0x7FF      # no next step


class ViewMajorTables(NamedTuple):
    idx: torch.Tensor    # int32 [2 * rounds]: per point, half 0's input row per round, then half 1's
    ev: torch.Tensor     # int16 [rounds]: per round, flags | next active step << 3 (at a step's end)
    off: torch.Tensor    # int32 [n_out + 1]: first round of each point (multiples of VM_CHUNK)
    j0: torch.Tensor     # int32 [n_out]: each point's first active step (-1: none)
    pad: int             # the input row a padding round names (n_in: past the rows, read as zeros)
    steps: int           # active steps over all points


def view_major_tables(slot_ptr, nbr_sorted, n_in, n_ref, cp, k_pad):
    """Tables of the view-major few-channel kernel from the CSR lists (``csr_tables``).

    Reduction step j covers columns 16 j .. 16 j + 15, i.e. slots ``16 / cp * j ..``; lane half h
    of an MFMA block holds columns 8 h .. 8 h + 7 of it when the step's MFMAs run: for cp = 4
    slots 4j + 2h and 4j + 2h + 1, for cp = 8 slot 2j + h (one phase). A point's steps with no
    neighbour in any of their slots are left out. For cp = 4 a step's four slots s0..s3 are
    summed in two phases, each pairing a slot of half 0 with one of half 1; per point and step
    the pairing with the fewest rounds is taken (ties: the first):
      (s0|s2, s1|s3): the halves sum their own slots;
      (s0|s3, s1|s2), VM_Q: half 1 puts phase A's sum in its second slot, phase B's in its first;
      (s0|s1, s2|s3), VM_X: after the step's last sum half 0's second slot (s2) and half 1's
        first (s1) change halves (v_permlane32_swap).
    For each active step and phase the kernel runs max(count of half 0's slot, count of half 1's
    slot) rounds; in round q each half adds neighbour q of its slot's list (CSR order) or, past
    its count, a padding row (+0). The sums are the two-pass path's (``slotsum_kernel``): groups
    of FC_GROUP neighbours summed in fp32 from +0 in list order, the groups' sums added in order
    (VM_G closes a group), one rounding to bf16 at the phase's end (VM_P: phase A's sum; VM_S:
    the step's last sum, then its MFMAs; a step whose phase B is empty ends on phase A's last
    round with both flags); VM_Q and VM_X ride on those events. The S event also names the next
    active step (bits VM_JSHIFT..15), whose weight fragments the kernel loads then. Each
    point's rounds are padded to a multiple of VM_CHUNK."""
    if cp not in (4, 8) or k_pad % 16:
        raise ValueError(f"view-major tables need cp in (4, 8) and k_pad % 16 == 0, got {cp}, {k_pad}")
    ptr = slot_ptr.numpy().astype(np.int64)
    nbr = nbr_sorted.numpy().astype(np.int64)
    n_out = ptr.shape[0]
    ks, spk = k_pad // 16, 16 // cp
    if ks >= VM_J_NONE:
        raise ValueError(f"k_pad={k_pad} has more reduction steps than the event word holds")
    cnt = np.zeros((n_out, ks * spk), np.int64)
    beg = np.zeros((n_out, ks * spk), np.int64)
    cnt[:, :n_ref] = ptr & 0xFFFF
    beg[:, :n_ref] = ptr >> 16
    # (phases, flags) per pairing: phase = (slot of half 0, slot of half 1)
    pairings = ((((0, 2), (1, 3)), 0), (((0, 3), (1, 2)), VM_Q), (((0, 1), (2, 3)), VM_X)) if cp == 4 \
        else ((((0, 1),), 0),)
    pad = int(n_in)
    idx_parts, ev_parts, off, j0 = [], [], [0], []
    n_steps = 0
    for t in range(n_out):
        c_t, b_t = cnt[t].reshape(ks, spk), beg[t].reshape(ks, spk)
        active = np.nonzero(c_t.sum(1))[0]
        rows = ([], [])
        evs = []
        ends = []
        for j in active:
            cost = [sum(max(int(c_t[j, a]), int(c_t[j, b])) for a, b in ph) for ph, _ in pairings]
            phases, flag = pairings[int(np.argmin(cost))]
            for pi, qs in enumerate(phases):
                m = [int(c_t[j, q]) for q in qs]
                r = max(m)
                if r == 0:
                    continue
                for hh in range(2):
                    b = int(b_t[j, qs[hh]])
                    rows[hh].extend(nbr[t, b:b + m[hh]].tolist())
                    rows[hh].extend([pad] * (r - m[hh]))
                e = [0] * r
                for q in range(FC_GROUP - 1, r - 1, FC_GROUP):
                    e[q] |= VM_G
                if cp == 4 and pi == 0:
                    e[-1] |= VM_P | flag
                evs.extend(e)
            evs[-1] |= VM_S | flag
            ends.append(len(evs) - 1)
        for i, er in enumerate(ends):
            evs[er] |= (int(active[i + 1]) if i + 1 < len(active) else VM_J_NONE) << VM_JSHIFT
        n_r = -(-len(evs) // VM_CHUNK) * VM_CHUNK
        fill = n_r - len(evs)
        idx_parts.append(np.asarray(rows[0] + [pad] * fill + rows[1] + [pad] * fill, np.int64))
        ev_parts.append(np.asarray(evs + [0] * fill, np.int64))
        off.append(off[-1] + n_r)
        j0.append(int(active[0]) if len(active) else -1)
        n_steps += len(active)
    idx = np.concatenate(idx_parts) if idx_parts else np.zeros(0, np.int64)
    ev = np.concatenate(ev_parts) if ev_parts else np.zeros(0, np.int64)
    return ViewMajorTables(torch.from_numpy(idx.astype(np.int32)),
                           torch.from_numpy(ev.astype(np.uint16).view(np.int16)),
                           torch.from_numpy(np.asarray(off, np.int32)), torch.from_numpy(np.asarray(j0, np.int32)),
                           pad, n_steps)


def view_major_weight(w_rows, cb):
    """The view-major kernel's weight: fragments ``[k_pad / 16, n_blocks, 64, 8]`` of the
    row-packed weight ``w_rows`` [c_out, k_pad] (bf16), 32-column blocks padded with zero
    columns to a multiple of ``cb`` blocks: lane l of fragment (j, b) holds columns
    16 j + 8 (l / 32) .. + 7 of row 32 b + l % 32, the MFMA B operand of step j and block b."""
    c_out, k_pad = w_rows.shape
    nb = -(-c_out // 32)
    nb = -(-nb // cb) * cb
    wp = torch.zeros(nb * 32, k_pad, dtype=w_rows.dtype, device=w_rows.device)
    wp[:c_out] = w_rows
    return wp.view(nb, 32, k_pad // 16, 2, 8).permute(2, 0, 3, 1, 4).contiguous().view(k_pad // 16, nb, 64, 8)


def _row_offset(r):
    """Byte offset in the kernel's LDS of 16-byte part 0 of staged row ``r``: rows are 64
    bytes, and part q of row r sits at ``(64 r + 16 g(r)) ^ 16 q`` with
    g(r) = (bit1(r) ^ bit3(r)) | bit2(r) << 1 (the XOR swizzle that keeps 8 or 16
    consecutive rows of one part on distinct LDS banks)."""
    r = np.asarray(r, np.int64)
    g = (((r >> 1) ^ (r >> 3)) & 1) | ((r >> 1) & 2)
    return r * 64 + (g << 4)


# Collision entries of the wide-layer kernel's stream hold at most this many
# neighbours; rows whose slot holds more ("heavy") are summed once per channel
# chunk into their own LDS rows.
STREAM_MAX_COUNT = 6
# LDS bytes of one collision tile of the wide-layer kernel (256 rows x 64 bytes)
WIDE_TILE_BYTES = 256 * 64
# collision tiles of the wide-layer kernel: four when its LDS layout with four fits
# WIDE_LDS_BYTES, else three (slot position p sums into tile p % tiles)
WIDE_TILES = 3
WIDE_TILES_MAX = 4
WIDE_LDS_BYTES = 160 * 1024
# staged rows the wide-layer kernel holds (four 16-byte pieces per thread and row, 16 per thread)
WIDE_MAX_ROWS = 1024


def wide_layout(n_ref, zero_row, coll_off_stride, cent_stride, heavy_stride, hlist_stride):
    """(collision tiles, LDS bytes) of the wide-layer kernel's tile for tables of these sizes:
    ``WIDE_TILES_MAX`` tiles when that layout fits ``WIDE_LDS_BYTES``, else ``WIDE_TILES``. The
    rule and the layout are the kernel's own, asked of the library
    (``fovi_knnconv_wide_tiles``), so the tables and the kernel cannot disagree; the forward
    refuses tables built for another count."""
    return _lib.knnconv_wide_tiles(n_ref, zero_row, coll_off_stride, cent_stride, heavy_stride, hlist_stride)


def wide_tile_count(n_ref, zero_row, coll_off_stride, cent_stride, heavy_stride, hlist_stride):
    """Collision tiles of the wide-layer kernel for these table sizes (``wide_layout``)."""
    return wide_layout(n_ref, zero_row, coll_off_stride, cent_stride, heavy_stride, hlist_stride)[0]


def wide_strides(direct):
    """Table sizes of ``wide_tables`` for ``direct`` (any slot order): ``(coll_off_stride,
    cent_stride, heavy_stride, hlist_stride)``."""
    ent = direct[2]
    n_tiles, n_ref, tile = direct[4].shape
    e3 = ent.numpy().view(np.uint32).astype(np.int64).reshape(n_tiles, tile, n_ref)
    cnt = (e3 >> 8) & 0xFF
    light = (cnt >= 2) & (cnt <= STREAM_MAX_COUNT)
    heavy = cnt > STREAM_MAX_COUNT
    stride = max(1, int(light.sum(axis=(1, 2)).max(initial=0)))
    heavy_stride = max(2, -(-int(heavy.sum(axis=(1, 2)).max(initial=0)) // 2) * 2)
    hlist_stride = max(8, -(-int(np.where(heavy, cnt, 0).sum(axis=(1, 2)).max(initial=0)) // 8) * 8)
    return -(-(n_ref + 1) // 4) * 4, stride, heavy_stride, hlist_stride


def wide_tiles_of(direct):
    """Collision tiles the wide-layer kernel uses for ``direct``'s tables."""
    return wide_tile_count(direct[4].shape[1], direct[6], *wide_strides(direct))


class WideTables(NamedTuple):
    src: torch.Tensor        # [T, V, tile] uint16
    coll: torch.Tensor       # [T, stride, 4] int32 (uint32 words)
    coll_off: torch.Tensor   # [T, V + 1 rounded up to 4] int32
    stride: int
    heavy: torch.Tensor      # [T, heavy_stride, 2] int32 (uint32 words)
    heavy_stride: int
    hlist: torch.Tensor      # [T, hlist_stride] int16 (uint16 offsets)
    hlist_stride: int
    units: bool              # row offsets in 16-byte units (True) or bytes (False)
    tiles: int               # collision tiles (slot position p sums into tile p % tiles)


def wide_tables(direct, k, order=None):
    """Tables of the wide-layer (fragment-order) kernel, derived from ``direct_tables``.

    Laid out in the kernel's LDS order (16-byte copies) and holding swizzled
    LDS offsets of rows (``_row_offset``) rather than row numbers, so the
    kernel forms every address with one XOR: byte offsets when they fit 16
    bits (up to 1023 staged rows), else 16-byte units (every row part is
    16-byte aligned; ``units``), which the kernel shifts back. The kernel's
    LDS starts with the staged rows and the zero row (``zero_row + 1`` rows of
    64 bytes), followed by ``heavy_stride`` rows of heavy sums.

    * ``src [T, V, tile] uint16``: per (slot, row) the offset of the 64-byte
      row the MFMA lanes read for that slot: the neighbour's staged row when
      the slot holds one neighbour, the zero row when it holds none, the row's
      heavy sum when it holds more than ``STREAM_MAX_COUNT``; 0xFFFF when it
      holds 2 .. ``STREAM_MAX_COUNT`` (the row's sum in a collision tile).
    * ``coll [T, stride, 4] uint32``: one 16-byte stream entry per (slot,
      collision row with 2 .. ``STREAM_MAX_COUNT`` neighbours), grouped by slot
      position and within a slot by decreasing count. Word 0: bits 0-15 the
      destination in bytes, relative to the first collision tile (tile ``p %
      tiles`` of slot position p, then the row's offset; ``tiles`` =
      ``wide_tile_count`` of the table sizes), bits 16-23 the count; words
      1-3: offsets of the staged rows of neighbours 1-6, two per word (low
      half first; the zero row past the count).
    * ``coll_off [T, V + 1 rounded up to 4] int32``: slot position p's entries
      are ``coll[t, coll_off[t, p]:coll_off[t, p + 1]]``.
    * ``heavy [T, heavy_stride, 2] uint32``: one entry per heavy (slot, row):
      word 0 bits 0-15 the offset of its heavy-sum row, bits 16-23 the count
      (0 = padding); word 1 the index of its first neighbour in ``hlist``.
    * ``hlist [T, hlist_stride] uint16``: the heavy entries' neighbour
      offsets, in list order.

    ``order`` (default: slot order) is the order in which the kernel visits
    the slots (``stream_slot_order``): the tables are laid out by position p
    in that order, slot ``order[p]``.

    Returns a ``WideTables``, or ``None`` when the kernel cannot stage the rows
    (more than 1024 staged rows) or k exceeds 255.
    """
    lo, span, ent, nbr, coll, coll_n, zero_row = direct
    if zero_row > WIDE_MAX_ROWS or k > 255:
        return None
    e = ent.numpy().view(np.uint32).astype(np.int64)          # [T*tile, V]
    n_tiles, n_ref, tile = coll.shape
    order = np.arange(n_ref) if order is None else np.asarray(order, np.int64)
    if sorted(order.tolist()) != list(range(n_ref)):
        raise ValueError("order must be a permutation of the slots")
    e3 = e.reshape(n_tiles, tile, n_ref)
    first, cnt, begin = e3 >> 16, (e3 >> 8) & 0xFF, e3 & 0xFF
    heavy_mask = cnt > STREAM_MAX_COUNT                        # [T, tile, V]
    voff, stride, heavy_stride, hlist_stride = wide_strides(direct)
    n_tiles_c = wide_tile_count(n_ref, zero_row, voff, stride, heavy_stride, hlist_stride)
    units = zero_row > 1023
    sh = 4 if units else 0                                    # offset = byte offset >> sh
    row_b = 64 >> sh
    heavy_base = (zero_row + 1) * row_b
    if heavy_base + heavy_stride * row_b >= 0xFFFF:           # 0xFFFF marks a stream-built sum
        return None
    nb = nbr.numpy().astype(np.int64).reshape(n_tiles, tile, k)
    zoff = int(_row_offset(zero_row)) >> sh

    # heavy entries: in (slot, row) order of each tile
    heavy_row = np.full((n_tiles, tile, n_ref), -1, np.int64)
    hent = []
    for t in range(n_tiles):
        rr, vv = np.nonzero(heavy_mask[t])
        ordv = np.lexsort((rr, vv))
        rr, vv = rr[ordv], vv[ordv]
        heavy_row[t, rr, vv] = np.arange(len(rr))
        hent.append((rr, vv))
    heavy = np.zeros((n_tiles, heavy_stride, 2), np.uint32)
    hlist = np.zeros((n_tiles, hlist_stride), np.uint16)
    for t in range(n_tiles):
        rr, vv = hent[t]
        pos = 0
        for h, (r, v) in enumerate(zip(rr, vv)):
            c, b0 = int(cnt[t, r, v]), int(begin[t, r, v])
            heavy[t, h, 0] = (heavy_base + row_b * h) | (c << 16)
            heavy[t, h, 1] = pos
            hlist[t, pos:pos + c] = _row_offset(nb[t, r, b0:b0 + c]) >> sh
            pos += c

    src = np.where(cnt >= 2, 0xFFFF, _row_offset(first) >> sh)
    src = np.where(heavy_mask, heavy_base + row_b * heavy_row, src).astype(np.uint16)
    src = src.transpose(0, 2, 1)[:, order].copy()              # [T, V (position), tile]

    # stream entries: collision rows of each slot with 2 .. STREAM_MAX_COUNT neighbours
    cl = coll.numpy().astype(np.int64)
    cn = coll_n.numpy().astype(np.int64)
    lists = [[None] * n_ref for _ in range(n_tiles)]
    light_n = np.zeros((n_tiles, n_ref), np.int64)
    for t in range(n_tiles):
        for q in range(n_ref):
            v = order[q]
            rows = cl[t, v, :cn[t, v]]
            rows = rows[cnt[t, rows, v] <= STREAM_MAX_COUNT]
            lists[t][q] = rows
            light_n[t, q] = len(rows)
    out = np.zeros((n_tiles, stride, 4), np.uint32)
    coll_off = np.zeros((n_tiles, voff), np.int32)
    for t in range(n_tiles):
        off = np.concatenate([[0], np.cumsum(light_n[t])])
        coll_off[t, :n_ref + 1] = off
        if off[-1] == 0:
            continue
        rows = np.concatenate(lists[t])
        pos = np.repeat(np.arange(n_ref), light_n[t])
        v = order[pos]
        c, b0 = cnt[t, rows, v], begin[t, rows, v]
        nbo = []
        for j in range(STREAM_MAX_COUNT):
            r = nb[t, rows, np.minimum(b0 + j, k - 1)]
            nbo.append(np.where(j < c, _row_offset(r) >> sh, zoff))
        n_e = off[-1]
        dst = (pos % n_tiles_c) * WIDE_TILE_BYTES + _row_offset(rows)
        out[t, :n_e, 0] = (dst | (c << 16)).astype(np.uint32)
        for w in range(3):
            out[t, :n_e, 1 + w] = (nbo[2 * w] | (nbo[2 * w + 1] << 16)).astype(np.uint32)
    return WideTables(torch.from_numpy(src), torch.from_numpy(out.view(np.int32)), torch.from_numpy(coll_off),
                      stride, torch.from_numpy(heavy.view(np.int32)), heavy_stride,
                      torch.from_numpy(hlist.view(np.int16)), hlist_stride, units, n_tiles_c)


def slot_stream_units(direct):
    """Stream demand of each (tile, slot) in the wide-layer kernel: four units (16-byte parts)
    per collision row with 2 .. ``STREAM_MAX_COUNT`` neighbours. ``[T, V] int64``."""
    ent = direct[2]
    n_tiles, n_ref, tile = direct[4].shape
    cnt = (ent.numpy().view(np.uint32).astype(np.int64) >> 8) & 0xFF
    light = (cnt >= 2) & (cnt <= STREAM_MAX_COUNT)
    return 4 * light.reshape(n_tiles, tile, n_ref).sum(axis=1)


def stream_slot_order(units_per_slot, rate=256, ahead=3, iters=600, seed=0):
    """Order in which the wide-layer kernel visits the slots of a channel chunk.

    The kernel forms collision sums as a stream that advances ``rate`` units
    per slot visit, up to ``ahead - 1`` slots ahead of the slot being
    consumed; a slot not complete at its turn is finished serially, and the
    first slot of a chunk is always built serially. ``units_per_slot [T, V]``
    is the stream demand of each (tile, slot). Heavy and light slots are
    interleaved (light first), then refined by pairwise swaps that lower the
    mean serialized work over the tiles. The sum over slots does not depend
    on the order. Returns a list of V slot indices.
    """
    units = np.asarray(units_per_slot, np.int64)
    n_tiles, n_ref = units.shape
    if n_ref <= 2:
        return list(range(n_ref))

    def cost(order):
        u = units[:, order]
        off = np.concatenate([np.zeros((n_tiles, 1), np.int64), np.cumsum(u, axis=1)], axis=1)
        bpos = off[:, 1].copy()
        serial = off[:, 1].astype(np.float64)
        for v in range(n_ref):
            need = off[:, v + 1]
            serial += np.maximum(need - bpos, 0)
            bpos = np.minimum(np.maximum(bpos, need) + rate, off[:, min(v + ahead, n_ref)])
        return float(serial.mean())

    by_load = list(np.argsort(-units.mean(axis=0), kind="stable"))
    order, lo, hi = [], 0, n_ref - 1
    while lo <= hi:
        order.append(int(by_load[hi])); hi -= 1          # light
        if lo <= hi:
            order.append(int(by_load[lo])); lo += 1      # heavy
    best = cost(order)
    rng = np.random.default_rng(seed)
    for _ in range(iters):
        a, b = rng.integers(0, n_ref, 2)
        if a == b:
            continue
        cand = order[:]
        cand[a], cand[b] = cand[b], cand[a]
        c = cost(cand)
        if c <= best:
            order, best = cand, c
    return order
