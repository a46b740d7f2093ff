"""CPU tests: host geometry/tables (closed forms, CSR format) and the oracle's own pinning."""
import numpy as np
import pytest
import torch

from fovi_amd.arch import knn_tables as T
from fovi_amd.sensing.coords import SamplingCoords, find_desired_res, logpolar_ring_radii
from oracle import knnconv_ref, sampler_ref
from tests.helpers import layer_tables


# ---------------------------------------------------------------- geometry ---
@pytest.mark.parametrize("res", [8, 16, 64])
def test_logpolar_point_set_closed_form(res):
    fov, a = 16, 2.78
    c = SamplingCoords(fov, a, res, style="logpolar")
    assert c.shape == (res * res, 2)
    # ring radii: r_i = (exp(w_i) - a) / (fov/2), w evenly spaced in log(r + a)
    w = np.linspace(np.log(a), np.log(fov / 2 + a) + (np.log(fov / 2 + a) - np.log(a)) / (res - 1), res + 1)
    r_closed = (np.exp(w) - a) / (fov / 2)
    radii = c.polar[::res, 0].double().numpy()
    assert np.allclose(radii, r_closed[:-1], atol=2e-6)
    assert abs(radii[0]) < 1e-5                   # ring 0 is degenerate (exp(log a) - a)
    ang = c.polar[:res, 1].double().numpy()
    assert np.allclose(ang, np.arange(res) * 2 * np.pi / res, atol=1e-6)
    xy = c.cartesian.double().numpy()
    rr = np.repeat(radii, res)
    aa = np.tile(ang, res)
    assert np.allclose(xy[:, 0], rr * np.cos(aa), atol=1e-6)
    assert np.allclose(xy[:, 1], rr * np.sin(aa), atol=1e-6)
    # cortical: normalised log radius per ring and normalised angle, both in [0, 1]
    cort = c.cortical.double().numpy()
    assert cort.min() == 0.0 and cort.max() == 1.0
    lr = np.log(np.hypot(xy[:, 0], xy[:, 1]) * fov / 2 + a)
    lr = (lr - lr.min()) / (lr.max() - lr.min())
    assert np.allclose(cort[:, 0], lr, atol=1e-5)
    assert np.allclose(cort[:res, 1], np.arange(res) / (res - 1), atol=1e-6)


def test_find_desired_res_logpolar():
    assert find_desired_res(16, 2.78, 64 ** 2, "logpolar", force_less_than=True, quiet=True) == (64, 4096)
    assert find_desired_res(16, 2.78, 1000, "logpolar", force_less_than=True, quiet=True) == (31, 961)
    assert find_desired_res(16, 2.78, 1000, "logpolar", force_less_than=False, quiet=True) == (32, 1024)


def test_strided_coords_are_regenerated_grids():
    c = SamplingCoords(16, 2.78, 64, style="logpolar")
    out, radii, _ = c.get_strided_coords(2)
    assert radii == 32 and out.shape == (1024, 2)
    assert torch.equal(out.cartesian, SamplingCoords(16, 2.78, 32, style="logpolar").cartesian)


def test_knn_lattice_neighbourhoods():
    """Away from the radial edges and the angle seam, k=9/25 are the 3x3/5x5 lattice squares."""
    res = 32
    t = layer_tables(res, res, 25)
    idx = t["idx"].numpy()
    for ring in range(4, res - 4):
        for ang in range(4, res - 4):
            n = ring * res + ang
            got = set(idx[:, n].tolist())
            want = {(ring + dr) * res + ang + da for dr in range(-2, 3) for da in range(-2, 3)}
            assert got == want, (ring, ang)
            assert idx[0, n] == n            # self first, distance 0
    assert torch.all(t["dist"][0] == 0)


def test_knn_seam_wraps_with_period_res_minus_one():
    """Angle indices 0 and res-1 of a ring are at distance 0 (reference knn.py:137-140)."""
    res = 16
    t = layer_tables(res, res, 9)
    d = t["dist"].numpy()
    idx = t["idx"].numpy()
    n = 6 * res + 0
    assert (n + res - 1) in idx[:, n]
    j = list(idx[:, n]).index(n + res - 1)
    assert d[j, n] == 0.0


def test_slots_self_at_centre_and_ranges():
    """Slot ids index the ref grid; an interior point (symmetric neighbourhood) maps itself to the
    centre slot, since its own offset is (0, 0) and min-max normalisation is symmetric."""
    t = layer_tables(32, 32, 9)
    slots = t["slots"].numpy()
    idx = t["idx"].numpy()
    assert slots.min() >= 0 and slots.max() < 9
    for ring in range(8, 30):
        for ang in range(2, 30):
            n = ring * 32 + ang
            j = list(idx[:, n]).index(n)
            assert slots[n, j] == 4, (ring, ang)


@pytest.mark.parametrize("res_in,res_out,k,side", [(16, 16, 9, None), (24, 12, 30, None), (32, 4, 256, 16)])
def test_csr_tables_match_one_hot(res_in, res_out, k, side):
    t = layer_tables(res_in, res_out, k, side)
    ptr, nbr = t["ptr"].numpy(), t["nbr"].numpy()
    idx, slots, V = t["idx"].numpy(), t["slots"].numpy(), t["V"]
    for n in range(t["n_out"]):
        want = {}
        for j in range(t["k"]):
            want.setdefault(slots[n, j], []).append(idx[j, n])
        for v in range(V):
            beg, cnt = int(ptr[n, v]) >> 16, int(ptr[n, v]) & 0xFFFF
            assert list(nbr[n, beg:beg + cnt]) == want.get(v, [])


def _csr_forward(x, ptr, nbr, w_ref, c_in, V):
    """The kernel's arithmetic restated in numpy (float64): packed weight + CSR slot sums."""
    B, C, _ = x.shape
    n_out = ptr.shape[0]
    wp = w_ref.reshape(w_ref.shape[0], c_in, V).transpose(0, 2, 1).reshape(w_ref.shape[0], V * c_in)
    A = np.zeros((B, n_out, V * c_in))
    for n in range(n_out):
        for v in range(V):
            beg, cnt = int(ptr[n, v]) >> 16, int(ptr[n, v]) & 0xFFFF
            for i in range(cnt):
                A[:, n, v * c_in:(v + 1) * c_in] += x[:, :, nbr[n, beg + i]]
    return np.einsum("bnk,ok->bon", A, wp)


@pytest.mark.parametrize("res_in,res_out,k,c_in,c_out,side", [(16, 16, 9, 3, 8, None), (16, 8, 25, 4, 5, None),
                                                               (24, 4, 100, 2, 3, 10)])
def test_csr_formulation_equals_oracle_and_bruteforce(res_in, res_out, k, c_in, c_out, side):
    t = layer_tables(res_in, res_out, k, side)
    g = torch.Generator().manual_seed(0)
    x = torch.randn(2, c_in, t["n_in"], generator=g, dtype=torch.float64)
    w = torch.randn(c_out, c_in * t["V"], generator=g, dtype=torch.float64)
    bias = torch.randn(c_out, generator=g, dtype=torch.float64)
    ref = knnconv_ref.knnconv_forward(x, t["idx"], t["n_in"], t["rf"].double(), w, bias)
    brute = knnconv_ref.knnconv_bruteforce(x, t["idx"], t["slots"], t["n_in"], w, bias)
    assert np.allclose(ref.numpy(), brute, rtol=1e-10, atol=1e-10)
    csr = _csr_forward(x.numpy(), t["ptr"].numpy(), t["nbr"].numpy(), w.numpy(), c_in, t["V"]) + \
        bias.numpy()[None, :, None]
    assert np.allclose(csr, brute, rtol=1e-10, atol=1e-10)


def test_oracle_weight_index_is_channel_major():
    """A weight that is 1 at column c*V + v only selects channel c of the neighbours in slot v."""
    t = layer_tables(16, 16, 9)
    c_in, V = 3, t["V"]
    x = torch.randn(1, c_in, t["n_in"], dtype=torch.float64)
    w = torch.zeros(1, c_in * V, dtype=torch.float64)
    c, v = 2, 4
    w[0, c * V + v] = 1.0
    y = knnconv_ref.knnconv_forward(x, t["idx"], t["n_in"], t["rf"].double(), w)[0, 0]
    idx, slots = t["idx"].numpy(), t["slots"].numpy()
    for n in (0, 50, 200):
        want = sum(x[0, c, idx[j, n]].item() for j in range(9) if slots[n, j] == v)
        assert abs(y[n].item() - want) < 1e-12


def test_oracle_linearity():
    t = layer_tables(16, 16, 9)
    g = torch.Generator().manual_seed(1)
    x1, x2 = (torch.randn(2, 4, t["n_in"], generator=g, dtype=torch.float64) for _ in range(2))
    w = torch.randn(6, 4 * t["V"], generator=g, dtype=torch.float64)
    f = lambda x: knnconv_ref.knnconv_forward(x, t["idx"], t["n_in"], t["rf"].double(), w)
    assert torch.allclose(f(x1 + 3 * x2), f(x1) + 3 * f(x2), atol=1e-10)


# ----------------------------------------------------------------- sampler ---
@pytest.mark.parametrize("mode", ["bilinear", "nearest"])
@pytest.mark.parametrize("pad", ["zeros", "border"])
def test_grid_sample_matches_textbook(mode, pad):
    g = torch.Generator().manual_seed(0)
    img = torch.rand(1, 3, 5, 7, generator=g, dtype=torch.float64)
    pts = torch.rand(1, 1, 40, 2, generator=g, dtype=torch.float64) * 2.6 - 1.3
    got = sampler_ref.grid_sample_views(img.float(), pts.float(), mode, pad)[0]
    want = sampler_ref.bilinear_numpy(img[0].numpy(), pts[0, 0, :, 0].float().double().numpy(),
                                      pts[0, 0, :, 1].float().double().numpy(), mode, pad)
    assert np.allclose(got.double().numpy(), want, atol=1e-5)


def test_transform_sampling_grid_closed_form():
    """The sensor centre lands on the fixation pixel; unit radius spans half the window."""
    grid = torch.tensor([[[[0.0, 0.0], [1.0, 0.0], [0.0, -1.0]]]])
    fix = torch.tensor([[0.25, 0.75]])      # (h, w)
    size = np.array([[64, 128]])            # (h, w) pixels
    g = sampler_ref.transform_sampling_grid(grid, fix, size, (256, 512))[0, 0]
    # centre: x = 0.75*512 = 384 px -> 2*384/512 - 1 = 0.5 ; y = 0.25*256 = 64 -> -0.5
    assert g[0].tolist() == [0.5, -0.5]
    # +x edge: 384 + 64 = 448 -> 0.75 ; -y edge (grid y=-1): 64 - 32 = 32 -> -0.75
    assert g[1].tolist() == [0.75, -0.5]
    assert g[2].tolist() == [0.5, -0.75]


@pytest.mark.parametrize("res_in,res_out,k", [(32, 32, 25), (32, 16, 25), (64, 32, 49), (16, 16, 9)])
def test_tile_tables_are_the_csr_lists_relative_to_tile_lo(res_in, res_out, k):
    t = layer_tables(res_in, res_out, k)
    lo, span, ent, nbr = (x.numpy().astype(np.int64) for x in
                          T.tile_tables(t["idx"], t["slots"], t["n_in"], t["V"], tile=256))
    ent = ent & 0xFFFFFFFF
    ptr, gnbr = t["ptr"].numpy(), t["nbr"].numpy()
    for n in range(t["n_out"]):
        tt = n // 256
        for v in range(t["V"]):
            cnt, beg, first = (ent[n, v] >> 8) & 0xFF, ent[n, v] & 0xFF, ent[n, v] >> 16
            assert cnt == (ptr[n, v] & 0xFFFF) and beg == (ptr[n, v] >> 16)
            if cnt:
                assert first == nbr[n, beg]
            got = nbr[n, beg:beg + cnt] + lo[tt]
            assert list(got) == list(gnbr[n, beg:beg + cnt])
            assert np.all(nbr[n, beg:beg + cnt] < span[tt])


@pytest.mark.parametrize("res_in,res_out,k", [(32, 32, 25), (64, 32, 49), (16, 16, 9)])
def test_direct_tables_lists_and_zero_row(res_in, res_out, k):
    t = layer_tables(res_in, res_out, k)
    lo, span, ent, nbr, coll, coll_n, zr = T.direct_tables(t["idx"], t["slots"], t["n_in"], t["V"])
    e = ent.numpy().view(np.uint32).astype(np.int64)
    cnt, first = (e >> 8) & 0xFF, e >> 16
    assert zr == int(span.max())
    assert np.all(first[cnt == 0] == zr)
    assert np.all(first[cnt > 0] < zr)
    coll, coll_n = coll.numpy(), coll_n.numpy()
    for tt in range(coll.shape[0]):
        for v in range(t["V"]):
            rows = coll[tt, v, :coll_n[tt, v]].astype(np.int64)
            want = np.nonzero(cnt[tt * 256:(tt + 1) * 256, v] >= 2)[0]
            assert sorted(rows.tolist()) == want.tolist()
            c = cnt[tt * 256 + rows, v]
            assert np.all(np.diff(c) <= 0)          # decreasing count order


def header_wide_lds_bytes(n_ref, zero_row, coll_off_stride, cent_stride, heavy_stride, hlist_stride, tiles):
    """The wide-layer tile's LDS bytes as include/fovi_hip.h states them (tile_cent): 64 (zero_row
    + 1 + heavy_stride) rounded up to 128, + (256 nb + 1) 64 + 512 n_ref + 4 coll_off_stride +
    16 cent_stride + 8 heavy_stride + 2 hlist_stride."""
    o = ((zero_row + 1 + heavy_stride) * 64 + 127) // 128 * 128
    return (o + (tiles * 256 + 1) * 64 + 512 * n_ref + 4 * coll_off_stride + 16 * cent_stride
            + 8 * heavy_stride + 2 * hlist_stride)


@pytest.mark.parametrize("res_in,res_out,k,permute", [(32, 32, 25, False), (64, 32, 49, False), (16, 16, 9, False),
                                                      (128, 128, 25, False), (32, 32, 25, True),
                                                      (32, 16, 25, False)])   # C2 layer 2: 1024 staged rows
def test_wide_tables_decode_to_the_csr_lists(res_in, res_out, k, permute):
    """Fragment-order kernel tables: every (slot, row) source, stream entry and heavy entry
    decodes back to the slot-major CSR lists (global input index = staged row + tile_lo)."""
    t = layer_tables(res_in, res_out, k)
    direct = T.direct_tables(t["idx"], t["slots"], t["n_in"], t["V"])
    lo, span, ent, nbr, coll, coll_n, zr = direct
    order = list(np.random.default_rng(3).permutation(t["V"])) if permute else list(range(t["V"]))
    wide = T.wide_tables(direct, t["k"], order if permute else None)
    if wide is None:                      # more rows than the kernel stages
        assert zr > T.WIDE_MAX_ROWS
        return
    # collision tiles: four exactly when the four-tile layout fits, whatever the slot order
    sizes = (t["V"], zr, wide.coll_off.shape[1], wide.stride, wide.heavy_stride, wide.hlist_stride)
    assert T.wide_strides(direct) == sizes[2:]
    big = header_wide_lds_bytes(*sizes, T.WIDE_TILES_MAX) <= T.WIDE_LDS_BYTES
    assert wide.tiles == (T.WIDE_TILES_MAX if big else T.WIDE_TILES) == T.wide_tiles_of(direct)
    src, cent, coll_off = wide.src.numpy().astype(np.int64), wide.coll.numpy().view(np.uint32), wide.coll_off.numpy()
    heavy, hlist = wide.heavy.numpy().view(np.uint32), wide.hlist.numpy().view(np.uint16)
    # byte offset -> row: 64-byte rows, swizzle bits only in bits 4-5; the tables hold staged
    # and heavy rows in bytes or 16-byte units, collision-tile destinations in bytes
    row_of_byte = {int(T._row_offset(r)): r for r in range(zr + 1)}
    assert len(row_of_byte) == zr + 1 and all(o & 15 == 0 for o in row_of_byte)
    sh = 4 if wide.units else 0
    assert wide.units == (zr > 1023)
    row_of = {o >> sh: r for o, r in row_of_byte.items()}
    heavy_base = (zr + 1) * (64 >> sh)
    ptr, gnbr = t["ptr"].numpy(), t["nbr"].numpy()
    lo = lo.numpy().astype(np.int64)
    n_tiles, V = src.shape[0], t["V"]
    assert cent.shape == (n_tiles, wide.stride, 4)
    assert heavy.shape == (n_tiles, wide.heavy_stride, 2) and wide.heavy_stride % 2 == 0
    assert hlist.shape == (n_tiles, wide.hlist_stride) and wide.hlist_stride % 8 == 0
    n_heavy = 0
    for tt in range(n_tiles):
        seen = set()
        for pos in range(V):
            v = order[pos]
            for ei in range(coll_off[tt, pos], coll_off[tt, pos + 1]):
                w0, w1, w2, w3 = (int(x) for x in cent[tt, ei])
                dst, cnt = w0 & 0xFFFF, (w0 >> 16) & 0xFF
                assert w0 >> 24 == 0
                assert dst // T.WIDE_TILE_BYTES == pos % wide.tiles
                row = row_of_byte[dst % T.WIDE_TILE_BYTES]
                n = tt * 256 + row
                assert 2 <= cnt <= T.STREAM_MAX_COUNT and cnt == (ptr[n, v] & 0xFFFF)
                beg = ptr[n, v] >> 16
                rs = [row_of[o] for o in (w1 & 0xFFFF, w1 >> 16, w2 & 0xFFFF, w2 >> 16, w3 & 0xFFFF, w3 >> 16)]
                want = list(gnbr[n, beg:beg + cnt])
                assert [r + lo[tt] for r in rs[:cnt]] == want
                assert all(r == zr for r in rs[cnt:])
                assert src[tt, pos, row] == 0xFFFF
                assert (v, row) not in seen
                seen.add((v, row))
        used = 0
        for pos in range(V):
            v = order[pos]
            for row in range(256):
                n = tt * 256 + row
                if n >= t["n_out"] or (v, row) in seen:
                    continue
                cnt = ptr[n, v] & 0xFFFF
                if cnt > T.STREAM_MAX_COUNT:       # heavy: its own row, summed once per chunk
                    h, r = divmod(int(src[tt, pos, row]) - heavy_base, 64 >> sh)
                    assert r == 0 and 0 <= h < wide.heavy_stride
                    w0, w1 = (int(x) for x in heavy[tt, h])
                    assert w0 & 0xFFFF == src[tt, pos, row] and (w0 >> 16) & 0xFF == cnt
                    beg = ptr[n, v] >> 16
                    got = [row_of[int(o)] + lo[tt] for o in hlist[tt, w1:w1 + cnt]]
                    assert got == list(gnbr[n, beg:beg + cnt])
                    used += 1
                    continue
                assert cnt <= 1
                want = gnbr[n, ptr[n, v] >> 16] - lo[tt] if cnt == 1 else zr
                assert row_of[src[tt, pos, row]] == want
        # every non-padding heavy entry is one (slot, row) of this tile
        assert used == int((((heavy[tt, :, 0] >> 16) & 0xFF) > 0).sum())
        n_heavy += used
    if (res_in, res_out, k) == (128, 128, 25):
        assert n_heavy > 0                 # the C3 lattice has slots with more than six neighbours


def test_stream_slot_order_is_a_permutation_that_lowers_serial_work():
    """The slot-visit order search returns a permutation, light slots first, and on the C3
    lattice it leaves less serialized collision work than the plain order."""
    t = layer_tables(128, 128, 25)
    direct = T.direct_tables(t["idx"], t["slots"], t["n_in"], t["V"])
    units = T.slot_stream_units(direct)
    order = T.stream_slot_order(units)
    assert sorted(order) == list(range(t["V"]))

    def serial(order, rate=256, ahead=3):
        u = units[:, order]
        off = np.concatenate([np.zeros((u.shape[0], 1), np.int64), np.cumsum(u, axis=1)], axis=1)
        bpos, tot = off[:, 1].copy(), off[:, 1].sum()
        for v in range(u.shape[1]):
            tot += np.maximum(off[:, v + 1] - bpos, 0).sum()
            bpos = np.minimum(np.maximum(bpos, off[:, v + 1]) + rate, off[:, min(v + ahead, u.shape[1])])
        return tot
    assert serial(order) < 0.5 * serial(list(range(t["V"])))


@pytest.mark.parametrize("res_in,res_out,k,side,cp,geom", [
    (128, 16, 256, 16, 4, (64, 256, 32)),     # C4 patch embedding
    (128, 16, 256, 16, 4, (128, 512, 64)),
    (64, 32, 49, None, 4, (256, 512, 64)),    # C2 layer 1
    (64, 32, 49, None, 4, (64, 256, 32)),
    (32, 16, 25, None, 8, (128, 512, 64)),    # eight-channel rows
    (32, 16, 25, None, 8, (64, 256, 32)),
    (24, 12, 30, None, 4, (128, 512, 64)),    # ragged: partial tile, padding slots in the last chunk
    (24, 12, 30, None, 4, (64, 256, 32)),
])
def test_few_channel_tables_rebuild_the_slot_sums(res_in, res_out, k, side, cp, geom):
    """Emulates the fused few-channel kernel's use of its tables in float64: the A tile starts
    cleared; every thread's FC_PAIRS pair words form runs, each a sum of at most FC_GROUP
    neighbours written at its last word (to a distinct A entry of the swizzled layout, or as a
    partial sum that a combine entry adds in order with the other groups of its slot); unused
    words read the zero row; every S row read is a staged row; every non-empty (row, slot) of a
    chunk is written exactly once, and the rebuilt A chunks equal the slot sums of the CSR
    lists."""
    import numpy as np

    from fovi_amd.arch import knn_tables as T
    t = layer_tables(res_in, res_out, k, side=side)
    V, n_in, n_out = t["V"], t["n_in"], t["n_out"]
    k_pad = -(-V * cp // 64) * 64
    tile, threads, chunk = geom
    ft = T.few_channel_tables(t["idx"], t["slots"], n_in, V, cp, k_pad, tile, threads, chunk)
    assert ft is not None and (ft.tile, ft.threads, ft.chunk) == geom
    G = T.FC_GROUP
    spc, nc = chunk // cp, k_pad // chunk
    rng = np.random.default_rng(0)
    x = rng.standard_normal((n_in, cp))
    # reference slot sums [n_out, V, cp] from the CSR lists
    ptr, nbr = t["ptr"].numpy(), t["nbr"].numpy()
    want = np.zeros((n_out, nc * spc, cp))
    for n in range(n_out):
        for v in range(V):
            b, c = ptr[n, v] >> 16, ptr[n, v] & 0xFFFF
            if c:
                want[n, v] = x[nbr[n, b:b + c]].sum(0)
    item = ft.item.numpy().view(np.uint32)
    assert item.shape == (ft.lo.shape[0], nc, threads, ft.pairs) and ft.pairs in T.FC_PAIR_COUNTS
    assert not (item >> 30).any(), "pair words use bits 0-29"
    # A entries of the swizzled 128-byte rows: one per (row, slot), all distinct
    entry_dest = {T._fc_entry(r, sl, cp, chunk): r * spc + sl for r in range(tile) for sl in range(spc)}
    assert len(entry_dest) == tile * spc and max(entry_dest) < tile * chunk * 2 // (2 * cp)
    comb = ft.comb.numpy().view(np.uint32)
    coff = ft.comb_off.numpy()
    split = 0
    for ti in range(ft.lo.shape[0]):
        lo, span = int(ft.lo[ti]), int(ft.span[ti])
        S = np.concatenate([x[lo:lo + span], np.zeros((1, cp))])[np.r_[0:span, [span] * (ft.zero_row + 1 - span)]]
        assert ft.zero_row >= span and not S[ft.zero_row].any()
        for c in range(nc):
            got = np.zeros((tile * spc, cp))
            written = np.zeros(tile * spc, bool)
            P = np.full((ft.pmax, cp), np.nan)
            for th in range(threads):
                run = []
                for word in item[ti, c, th].tolist():
                    run.append(word & 0xFFFF)
                    if not word & T.FC_LAST:
                        continue
                    target = (word >> 16) & 0xFFF
                    assert 1 <= len(run) <= G and all(0 <= r < span for r in run), run
                    val = S[run].sum(0)
                    if word & T.FC_PARTIAL:
                        assert np.isnan(P[target]).all(), "a partial sum is written twice"
                        P[target] = val
                    else:
                        dest = entry_dest[target]
                        assert not written[dest], "a (row, slot) is written twice"
                        written[dest] = True
                        got[dest] = val
                    run = []
                assert all(r == ft.zero_row for r in run), "unused pair words read the zero row"
            for cw in comb[coff[ti * nc + c]:coff[ti * nc + c + 1]]:
                dest, m, p0 = int(cw & 0xFFF), int(cw >> 12) & 0xFF, int(cw >> 20)
                assert m >= 2 and not written[dest]
                assert not np.isnan(P[p0:p0 + m]).any(), "a combined partial is never written"
                written[dest] = True
                got[dest] = P[p0:p0 + m].sum(0)
                split += 1
            got = got.reshape(tile, spc, cp)
            rows = slice(ti * tile, min((ti + 1) * tile, n_out))
            m_rows = rows.stop - rows.start
            np.testing.assert_allclose(got[:m_rows], want[rows, c * spc:(c + 1) * spc], rtol=1e-12, atol=1e-12)
            nonempty = (ptr[rows, :] & 0xFFFF)
            occ = np.zeros((m_rows, nc * spc), bool)
            occ[:, :V] = nonempty > 0
            assert (written.reshape(tile, spc)[:m_rows] == occ[:, c * spc:(c + 1) * spc]).all()
            assert not got[m_rows:].any(), "rows past n_out must be zero"
    if k == 256:
        assert split > 0, "the C4 geometry has slots of more than FC_GROUP neighbours"


def _grouped_slot_sum(rows, group):
    """fp32 slot sum of bf16-valued rows in the two-pass path's order: groups of ``group``
    summed from +0 in list order, the groups' sums added in order from +0."""
    total = np.zeros(rows.shape[1:], np.float32)
    for g0 in range(0, rows.shape[0], group):
        part = np.zeros(rows.shape[1:], np.float32)
        for r in rows[g0:g0 + group]:
            part = (part + r).astype(np.float32)
        total = (total + part).astype(np.float32)
    return total


@pytest.mark.parametrize("res_in,res_out,k,side,cp", [
    (128, 16, 256, 16, 4),     # C4 patch embedding: foveal slots of up to 121 neighbours
    (64, 32, 49, None, 4),     # C2 layer 1
    (32, 16, 25, None, 8),     # eight-channel rows: one phase per step
    (24, 12, 30, None, 4),     # ragged: padding slots in the last step
    (48, 12, 64, 8, 4),        # 8 x 8 ref grid, collisions on every point
    (40, 20, 49, None, 8),     # eight-channel rows, 49 slots
])
def test_view_major_tables_rebuild_the_slot_sums(res_in, res_out, k, side, cp):
    """Emulates the view-major kernel's rounds in fp32 for 32 images at once: per point, each
    lane half adds its round's input row (a padding row: zeros) to a group sum; the events close
    groups, end phase A (its sum rounded to bf16 into A dwords 0-1, half 1 into 2-3 under
    VM_Q) and end steps (the last sum into the rest, half 0's second and half 1's first slot
    exchanged under VM_X, then the step's columns are emitted) and name the next active step. The A
    rows rebuilt this way equal the grouped fp32 slot sums of the CSR lists rounded to bf16 bit
    for bit, skipped steps are exactly those with no neighbour, and every round's input row is
    a real row or the padding row."""
    import torch
    from fovi_amd.arch import knn_tables as T
    t = layer_tables(res_in, res_out, k, side=side)
    V, n_in, n_out = t["V"], t["n_in"], t["n_out"]
    k_pad = -(-V * cp // 64) * 64
    ks, spk = k_pad // 16, 16 // cp
    vt = T.view_major_tables(t["ptr"], t["nbr"], n_in, V, cp, k_pad)
    idx = vt.idx.numpy().astype(np.int64)
    ev = vt.ev.numpy().view(np.uint16).astype(np.int64)
    off, j0 = vt.off.numpy(), vt.j0.numpy()
    assert vt.pad == n_in and (np.diff(off) % T.VM_CHUNK == 0).all() and len(idx) == 2 * off[-1]
    rng = np.random.default_rng(1)
    B = 32
    x = torch.from_numpy(rng.standard_normal((n_in, B, cp)).astype(np.float32)).bfloat16().float().numpy()
    xpad = np.concatenate([x, np.zeros((1, B, cp), np.float32)])
    bf = lambda a: torch.from_numpy(np.ascontiguousarray(a)).bfloat16().float().numpy()
    ptr, nbr = t["ptr"].numpy(), t["nbr"].numpy()
    n_active = n_x = n_q = 0
    for p in range(n_out):
        # the grouped slot sums of the CSR lists, [k_pad / cp slots, B, cp], rounded to bf16
        want = np.zeros((ks * spk, B, cp), np.float32)
        for v in range(V):
            b, c = ptr[p, v] >> 16, ptr[p, v] & 0xFFFF
            if c:
                want[v] = bf(_grouped_slot_sum(x[nbr[p, b:b + c]], T.FC_GROUP))
        active = [j for j in range(ks) if (ptr[p, j * spk:(j + 1) * spk] & 0xFFFF).sum() > 0
                  and j * spk < V]
        assert j0[p] == (active[0] if active else -1)
        n_active += len(active)
        got = np.zeros_like(want)
        R = off[p + 1] - off[p]
        rows = [idx[2 * off[p] + h * R: 2 * off[p] + (h + 1) * R] for h in range(2)]
        assert all(((r >= 0) & (r <= n_in)).all() for r in rows)
        part = np.zeros((2, B, cp), np.float32)
        acc = np.zeros((2, B, cp), np.float32)
        a = np.zeros((2, 2, B, cp), np.float32)        # [half, dword pair (phase), image, channel]
        steps = iter(active)
        j_cur = next(steps, None)
        for q in range(R):
            e = int(ev[off[p] + q])
            if j_cur is None:
                assert e == 0 and rows[0][q] == n_in and rows[1][q] == n_in, "tail rounds are padding"
                continue
            for h in range(2):
                part[h] = (part[h] + xpad[rows[h][q]]).astype(np.float32)
            if e & 7:
                if e & (T.VM_P | T.VM_S):
                    val = (acc + part).astype(np.float32)
                    for h in range(2):
                        first = cp == 8 or (bool(e & T.VM_P) != (h == 1 and bool(e & T.VM_Q)))
                        a[h, 0 if first else 1] = bf(val[h])
                    acc[:] = 0
                else:
                    acc = (acc + part).astype(np.float32)
                part[:] = 0
                if e & T.VM_S:
                    assert j_cur is not None, "a step end past the point's active steps"
                    if e & T.VM_X:       # half 0's second slot and half 1's first change halves
                        a[0, 1], a[1, 0] = a[1, 0].copy(), a[0, 1].copy()
                        n_x += 1
                    n_q += bool(e & T.VM_Q)
                    for h in range(2):
                        if cp == 4:
                            got[4 * j_cur + 2 * h] = a[h, 0]
                            got[4 * j_cur + 2 * h + 1] = a[h, 1]
                        else:
                            got[2 * j_cur + h] = a[h, 0]
                    a[:] = 0
                    j_next = next(steps, None)
                    assert (e >> T.VM_JSHIFT) == (T.VM_J_NONE if j_next is None else j_next)
                    j_cur = j_next
        assert j_cur is None, "every active step ends"
        np.testing.assert_array_equal(got, want)
    assert n_active == vt.steps
    if cp == 4:                  # both other pairings occur
        assert n_x > 0 and n_q > 0, (n_x, n_q)
    if k == 256:
        assert (np.diff(off) > 0).all() and vt.steps < n_out * ks


@pytest.mark.parametrize("res_in,res_out,k,side", [(64, 64, 9, None), (64, 32, 49, None), (32, 16, 25, None),
                                                    (128, 16, 256, 16), (24, 12, 30, None)])
def test_local_rf_slots_of_a_subset_equal_the_full_computation(res_in, res_out, k, side):
    """The host recomputation of flagged output points (local_rf_slots_rows) equals the full
    computation's rows bit for bit, for subsets of 1, 7, 25 and 100 points."""
    import numpy as np

    from fovi_amd.arch import knn_tables as T
    t = layer_tables(res_in, res_out, k, side=side)
    src = t["cin"].cortical
    ref, _ = T.reference_grid(t["k"], side_length=side)
    full = t["slots"]
    rng = np.random.default_rng(1)
    for m in (1, 7, 25, 100):
        rows = torch.from_numpy(np.sort(rng.choice(t["n_out"], size=min(m, t["n_out"]), replace=False)))
        got = T.local_rf_slots_rows(t["idx"], src, t["cin"].cartesian, t["cout"].cortical, t["cout"].cartesian, ref,
                                    rows)
        assert torch.equal(got, full[rows]), m
