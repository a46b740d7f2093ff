// kNN-convolution forward, bf16, for wide layers (c_in % 32 == 0, weight in
// MFMA-fragment order): the kernel of the large-layer shape.
//
// GEMM view as in knnconv.hip: rows = (b, n) output points, columns = output
// channels o, reduction kk = (slot v, channel c). The gathered A matrix is
// never materialised; a workgroup owns a tile of 256 points x 256 channels:
//  * 4 waves in a 2 x 2 grid, each with a 128 x 128 accumulator tile (4 x 4
//    blocks of v_mfma_f32_32x32x16_bf16, 256 fp32 accumulators per lane), so
//    each A fragment read from LDS feeds 4 MFMAs and each weight fragment 4.
//  * The tile's input rows (one contiguous index range, six rings for a
//    two-ring tile of the log-polar lattice) are staged in LDS one 32-channel
//    chunk at a time (S); the next chunk is loaded into registers while the
//    current one is consumed. MFMA lanes read single-neighbour slots straight
//    from S (an LDS zero row serves empty slots); slots with 2 to 6
//    neighbours are summed in fp32 (one RNE rounding) into a ring of three or
//    four collision tiles, up to two or three slots ahead, as a stream over the tile's
//    collision entries that advances a fixed 256 units per iteration; the few
//    slots with more neighbours are summed once per chunk into rows of their
//    own, which the MFMA lanes read like staged rows.
//  * Weights are not staged in LDS: fovi_knnconv_pack_weight_mfma stores
//    them in the order the MFMA B operand is consumed, so each lane loads its
//    16-byte fragment with one coalesced load (1 KB per wave and fragment)
//    straight into registers, one iteration ahead. The LDS then carries only
//    A fragments, staging and collision sums.
//  * Iterations run channel chunk outer, slot inner; one barrier per
//    iteration, two more per chunk for the S refresh.
#include "knnconv_internal.h"

namespace fovi {

constexpr int V5_MT = 256;   // output points per tile
constexpr int V5_NT = 256;   // output channels per tile
constexpr int V5_ROW = 64;   // bytes of an LDS row: one reduction chunk (32 bf16 or 64 e4m3 channels)
// Collision tiles: slot position v sums into tile v % nb, so the stream runs up to nb - 1
// slots ahead of the slot the MFMAs consume; nb = 4 when that layout fits the LDS, else 3
// (the host tables encode the same rule).
constexpr int V5_NB_MIN = 3, V5_NB_MAX = 4;

constexpr int V5_STREAM_MAX = 6;   // neighbours of a stream entry; more: a heavy entry

typedef int i32x8 __attribute__((ext_vector_type(8)));        // e4m3 MFMA operand (32 bytes)
typedef uint32_t u32x8v __attribute__((ext_vector_type(8)));

// LDS byte layout of a tile. The staged rows S come first, at offset 0, then
// the heavy-sum rows, so the host tables can hold absolute LDS byte offsets
// (16 bits) of every row an MFMA lane reads.
struct V5Layout {
  int heavy_rows, acol_off, src_off, coff_off, cent_off, heavy_off, hlist_off, total;  // bytes
};

__host__ __device__ inline V5Layout v5_layout(int V, int zero_row, int coff_stride, int cent_stride,
                                              int heavy_stride, int hlist_stride, int nb) {
  V5Layout l;
  int o = (zero_row + 1) * V5_ROW;                  // staged rows + zero row
  l.heavy_rows = o; o += heavy_stride * V5_ROW;     // heavy sums, one row per heavy entry
  o = (o + 127) & ~127;
  l.acol_off = o;   o += (nb * V5_MT + 1) * V5_ROW; // nb collision tiles of 256 rows + a trash row
  l.src_off = o;    o += V * V5_MT * 2;             // per (slot, row) A source, slot-major
  l.coff_off = o;   o += coff_stride * 4;           // per-slot collision entry offsets
  l.cent_off = o;   o += cent_stride * 16;          // collision entries
  l.heavy_off = o;  o += heavy_stride * 8;          // heavy entries
  l.hlist_off = o;  o += hlist_stride * 2;          // heavy entries' neighbour offsets
  l.total = o;
  return l;
}

constexpr uint32_t V5_TILE_BYTES = V5_MT * V5_ROW;   // one collision tile

__host__ __device__ inline int v5_tiles(int V, int zero_row, int coff_stride, int cent_stride, int heavy_stride,
                                        int hlist_stride) {
  return v5_layout(V, zero_row, coff_stride, cent_stride, heavy_stride, hlist_stride, V5_NB_MAX).total <= 160 * 1024
             ? V5_NB_MAX
             : V5_NB_MIN;
}

// Byte offset of 16-byte part 0 of 64-byte row r under the swz32 XOR swizzle;
// part q of the row is at row_off(r) ^ (q << 4).
__device__ __forceinline__ uint32_t row_off(int r) {
  const int g = (((r >> 1) ^ (r >> 3)) & 1) | ((r >> 1) & 2);
  return static_cast<uint32_t>(r * 64 + (g << 4));
}

__device__ __forceinline__ u32x4 lds16(const uint8_t* smem, uint32_t off) {
  return *reinterpret_cast<const u32x4*>(smem + off);
}

// Element types. A 64-byte LDS row is one reduction chunk; collision sums
// of a 16-byte part are fp32 (adds in list order from +0) rounded once to the
// element type (bf16: RNE; e4m3: RNE, saturating).
template <bool F8> struct V5Elem;
template <> struct V5Elem<false> {
  static constexpr int CC = 32;        // channels per chunk
  static constexpr int ESZ = 2;        // bytes per element
  typedef f32x8 Sum;                   // the 8 channels of a 16-byte part
  static __device__ __forceinline__ void acc(Sum& a, u32x4 x) { a += unpack_bf16x8(x); }
  static __device__ __forceinline__ u32x4 pack(const Sum& a) {
    return u32x4{cvt_pk_bf16(a[0], a[1]), cvt_pk_bf16(a[2], a[3]), cvt_pk_bf16(a[4], a[5]), cvt_pk_bf16(a[6], a[7])};
  }
};
template <> struct V5Elem<true> {
  static constexpr int CC = 64;
  static constexpr int ESZ = 1;
  typedef f32x16 Sum;                  // the 16 channels of a 16-byte part
  static __device__ __forceinline__ void acc(Sum& a, u32x4 x) {
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(x[w]), false);
      const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(x[w]), true);
      a[4 * w] += lo[0];
      a[4 * w + 1] += lo[1];
      a[4 * w + 2] += hi[0];
      a[4 * w + 3] += hi[1];
    }
  }
  static __device__ __forceinline__ u32x4 pack(const Sum& a) {
    u32x4 out;
    // Without a NaN among the 16 sums the saturation is the v_med3 clamp alone; their sum
    // is NaN when one is (or when infinities cancel, which takes the exact path too).
    float t = a[0];
#pragma unroll
    for (int i = 1; i < 16; ++i) t += a[i];
    if (t == t) {
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float c0 = __builtin_amdgcn_fmed3f(a[4 * w], -448.0f, 448.0f);
        const float c1 = __builtin_amdgcn_fmed3f(a[4 * w + 1], -448.0f, 448.0f);
        const float c2 = __builtin_amdgcn_fmed3f(a[4 * w + 2], -448.0f, 448.0f);
        const float c3 = __builtin_amdgcn_fmed3f(a[4 * w + 3], -448.0f, 448.0f);
        // the low pair's conversion keeps its third operand's high half, which the high
        // pair's conversion then replaces: any register serves (no zero to materialise)
        const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(c0, c1, __float_as_int(c0), false));
        out[w] = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(c2, c3, static_cast<int>(lo), true));
      }
      return out;
    }
#pragma unroll
    for (int w = 0; w < 4; ++w)
      out[w] = cvt_pk_e4m3<true>(a[4 * w + 2], a[4 * w + 3],
                                 cvt_pk_e4m3<false>(a[4 * w], a[4 * w + 1], __float_as_uint(a[4 * w])));
    return out;
  }
};

// Index of the 1 KB weight fragment (iteration it, 32-column block cb,
// half ks) in the MFMA-fragment order; iteration it = chunk * n_ref + slot.
__host__ __device__ inline int64_t v5_frag(int64_t it, int64_t ncb, int64_t cb, int ks) {
  return (it * ncb + cb) * 2 + ks;
}

// SH: the tables name staged and heavy rows by byte offsets (0) or in 16-byte units (4, for
// more than 1023 staged rows); byte offset = value << SH.
template <int SV, typename OutT, bool F8, int SH>
__device__ __forceinline__ void v5_body(const KnnParams& p, int ncb, int64_t tiles_per_b, int64_t n_tiles_n,
                                        int64_t total_tiles, int64_t padded_tiles, int vec_out) {
  typedef V5Elem<F8> E;
  typedef typename E::Sum Sum;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int V = static_cast<int>(p.V);
  const int zr = p.zero_row;
  const int nb = v5_tiles(V, zr, p.coll_off_stride, p.cent_stride, p.heavy_stride, p.hlist_stride);
  const V5Layout L = v5_layout(V, zr, p.coll_off_stride, p.cent_stride, p.heavy_stride, p.hlist_stride, nb);
  const uint16_t* srcs = reinterpret_cast<const uint16_t*>(smem + L.src_off);
  const int32_t* coff = reinterpret_cast<const int32_t*>(smem + L.coff_off);
  const u32x4* cent = reinterpret_cast<const u32x4*>(smem + L.cent_off);
  const uint32_t* heavy = reinterpret_cast<const uint32_t*>(smem + L.heavy_off);
  const uint16_t* hlist = reinterpret_cast<const uint16_t*>(smem + L.hlist_off);
  const uint32_t acol = static_cast<uint32_t>(L.acol_off);
  const uint32_t trash = acol + nb * V5_TILE_BYTES;

  const int64_t tile = xcd_tile(blockIdx.x, padded_tiles);
  if (tile >= total_tiles) return;
  const int64_t mt = tile / n_tiles_n;
  const int64_t tn = tile % n_tiles_n;
  const int64_t o0 = tn * V5_NT;
  const int64_t b = mt / tiles_per_b;
  const int64_t pt = mt % tiles_per_b;
  const int64_t n0 = pt * V5_MT;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform
  const int wm = wave & 1, wn = wave >> 1;
  const int64_t lo = p.tile_lo[pt];
  const int span = static_cast<int>(min(static_cast<int64_t>(zr), p.Nin - lo));

  const char* xrows = static_cast<const char*>(p.x) + (b * p.xs0 + lo * p.xs2) * E::ESZ;
  uint32_t s_off[SV];
  uint32_t s_ok = 0;
#pragma unroll
  for (int j = 0; j < SV; ++j) {
    const int q = tid + 256 * j;
    s_ok |= static_cast<uint32_t>((q >> 2) < span) << j;
    s_off[j] = static_cast<uint32_t>((q >> 2) * p.xs2 * E::ESZ + (q & 3) * 16);
  }
  const int ncc = static_cast<int>(p.C / E::CC);
  const int nit = ncc * V;
  // this wave's weight fragments: column blocks cb0 .. cb0 + 3; the base of
  // an iteration's fragments is wave-uniform, the lane adds 16 bytes
  const int64_t cb0 = tn * (V5_NT / 32) + wn * 4;

  u32x4 rs[SV];
  auto load_s = [&](int cc) {
    const char* base = xrows + cc * V5_ROW;
#pragma unroll
    for (int j = 0; j < SV; ++j)
      rs[j] = ((s_ok >> j) & 1) ? *reinterpret_cast<const u32x4*>(base + s_off[j]) : u32x4{0u, 0u, 0u, 0u};
  };
  auto store_s = [&]() {
#pragma unroll
    for (int j = 0; j < SV; ++j) {
      const int q = tid + 256 * j;
      if ((s_ok >> j) & 1) *reinterpret_cast<u32x4*>(smem + (row_off(q >> 2) ^ ((q & 3) << 4))) = rs[j];
    }
  };
  auto load_w = [&](int it, u32x4 (&dst)[8]) {
    const u32x4* wb = reinterpret_cast<const u32x4*>(p.w) + v5_frag(it, ncb, cb0, 0) * 64;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) dst[j * 2 + ks] = wb[(j * 2 + ks) * 64 + lane];
  };

  // Prologue: the first chunk's rows and the tile's tables, all loads in
  // flight together (16-byte copies; the tables are laid out on the host in
  // this LDS order).
  load_s(0);
  {
    const int n_src = V * V5_MT * 2 / 16, n_coff = p.coll_off_stride * 4 / 16;
    const int n_ce = p.cent_stride, n_hv = p.heavy_stride * 8 / 16, n_hl = p.hlist_stride * 2 / 16;
    const u32x4* g_src = reinterpret_cast<const u32x4*>(p.tile_src + pt * V * V5_MT);
    const u32x4* g_coff = reinterpret_cast<const u32x4*>(p.tile_coll_off + pt * p.coll_off_stride);
    const u32x4* g_ce = reinterpret_cast<const u32x4*>(p.tile_cent) + pt * p.cent_stride;
    const u32x4* g_hv = reinterpret_cast<const u32x4*>(p.tile_heavy + pt * p.heavy_stride * 2);
    const u32x4* g_hl = reinterpret_cast<const u32x4*>(p.tile_hlist + pt * p.hlist_stride);
    u32x4* d_src = reinterpret_cast<u32x4*>(smem + L.src_off);
    u32x4* d_coff = reinterpret_cast<u32x4*>(smem + L.coff_off);
    u32x4* d_ce = reinterpret_cast<u32x4*>(smem + L.cent_off);
    u32x4* d_hv = reinterpret_cast<u32x4*>(smem + L.heavy_off);
    const int total = n_src + n_coff + n_ce + n_hv + n_hl;
    for (int base = 0; base < total; base += 8 * 256) {
      u32x4 t[8];
      u32x4* dst[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        int i = base + u * 256 + tid;
        dst[u] = nullptr;
        if (i < n_src) { t[u] = g_src[i]; dst[u] = d_src + i; continue; }
        i -= n_src;
        if (i < n_coff) { t[u] = g_coff[i]; dst[u] = d_coff + i; continue; }
        i -= n_coff;
        if (i < n_ce) { t[u] = g_ce[i]; dst[u] = d_ce + i; continue; }
        i -= n_ce;
        if (i < n_hv) { t[u] = g_hv[i]; dst[u] = d_hv + i; continue; }
        i -= n_hv;
        if (i < n_hl) { t[u] = g_hl[i]; dst[u] = d_hv + n_hv + i; }
      }
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (dst[u]) *dst[u] = t[u];
    }
  }
  if (tid < 4) *reinterpret_cast<u32x4*>(smem + zr * V5_ROW + tid * 16) = u32x4{0u, 0u, 0u, 0u};
  __syncthreads();
  // The A sources become final LDS offsets in 16-byte units (below 160 KB / 16): a
  // stream-built sum (0xFFFF) is row r of collision tile pos % nb, where pos is
  // the slot's position in the chunk; other rows keep their offset. The MFMA lanes
  // then address a fragment with one shift and their part's XOR.
  {
    uint16_t* s16 = reinterpret_cast<uint16_t*>(smem + L.src_off);
    for (int i = tid; i < V * V5_MT; i += 256) {
      const uint32_t e = s16[i];
      const int pos = i / V5_MT, r = i % V5_MT;
      const uint32_t off = e == 0xffffu ? acol + static_cast<uint32_t>(pos % nb) * V5_TILE_BYTES + row_off(r)
                                        : e << SH;
      s16[i] = static_cast<uint16_t>(off >> 4);
    }
  }

  // Collision sums. A unit is (entry, 16-byte part): entry = unit / 4. Its
  // first four neighbours are summed from the entry's words 1-2, neighbours 5
  // and 6 from word 3 (missing ones are the zero row).
  auto unit_sum4 = [&](const u32x4 ce, uint32_t pq) {
    Sum a = {};
    E::acc(a, lds16(smem, ((ce[1] & 0xffffu) << SH) ^ pq));
    E::acc(a, lds16(smem, ((ce[1] >> 16) << SH) ^ pq));
    E::acc(a, lds16(smem, ((ce[2] & 0xffffu) << SH) ^ pq));
    E::acc(a, lds16(smem, ((ce[2] >> 16) << SH) ^ pq));
    return a;
  };
  auto unit_sum2 = [&](const u32x4 ce, uint32_t pq) {
    Sum a = {};
    E::acc(a, lds16(smem, ((ce[1] & 0xffffu) << SH) ^ pq));
    E::acc(a, lds16(smem, ((ce[1] >> 16) << SH) ^ pq));
    return a;
  };
  auto unit_rest = [&](Sum& a, const u32x4 ce, uint32_t pq) {
    if (((ce[0] >> 16) & 0xffu) > 4) {
      E::acc(a, lds16(smem, ((ce[3] & 0xffffu) << SH) ^ pq));
      E::acc(a, lds16(smem, ((ce[3] >> 16) << SH) ^ pq));
    }
  };
  // collision tile offset of a unit (the entry holds tile and row)
  auto unit_dst = [&](const u32x4 ce, uint32_t pq) { return acol + ((ce[0] & 0xffffu) ^ pq); };
  // Heavy sums of the current chunk: one unit per (heavy entry, 16-byte part),
  // neighbours in list order, four reads in flight (the zero row past the
  // count: +0 leaves an fp32 sum that started at +0 unchanged).
  const uint32_t zoff = row_off(zr);
  auto build_heavy = [&]() {
    for (int u = tid; u < p.heavy_stride * 4; u += 256) {
      const uint32_t w0 = heavy[(u >> 2) * 2], w1 = heavy[(u >> 2) * 2 + 1];
      const int cnt = static_cast<int>((w0 >> 16) & 0xffu);
      if (cnt == 0) continue;
      const uint32_t pq = static_cast<uint32_t>(u & 3) << 4;
      Sum a = {};
      for (int j = 0; j < cnt; j += 4) {
        uint32_t r[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) r[q] = j + q < cnt ? static_cast<uint32_t>(hlist[w1 + j + q]) << SH : zoff;
#pragma unroll
        for (int q = 0; q < 4; ++q) E::acc(a, lds16(smem, r[q] ^ pq));
      }
      *reinterpret_cast<u32x4*>(smem + (((w0 & 0xffffu) << SH) ^ pq)) = E::pack(a);
    }
  };
  // units [from, to) of the tile's unit stream (the entry list in slot order,
  // four 16-byte parts per entry), complete sums; from % 4 == 0. A chunk start
  // deals its units from the last thread down, away from the heavy sums, which
  // take the first threads.
  auto build_range = [&](int from, int to, bool from_top = false) {
    for (int u = from + (from_top ? 255 - tid : tid); u < to; u += 256) {
      const u32x4 ce = cent[u >> 2];
      const uint32_t pq = static_cast<uint32_t>(u & 3) << 4;
      Sum a = unit_sum4(ce, pq);
      unit_rest(a, ce, pq);
      *reinterpret_cast<u32x4*>(smem + unit_dst(ce, pq)) = E::pack(a);
    }
  };

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  // this lane's rows of the A tile
  int rowm[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) rowm[i] = wm * 128 + i * 32 + (lane & 31);
  // the two 16-byte parts of a row this lane feeds to the MFMAs: bf16, parts
  // (lane / 32) and 2 + lane / 32 (K halves ks = 0, 1); e4m3, parts
  // 2 (lane / 32) and 2 (lane / 32) + 1 (channels 32 (lane / 32) .. + 32)
  const uint32_t qx0 = F8 ? static_cast<uint32_t>(lane >> 5) << 5 : static_cast<uint32_t>(lane >> 5) << 4;
  const uint32_t qx1 = F8 ? qx0 ^ 16u : qx0 ^ 32u;

  u32x4 wa[8], wb[8];
  load_w(0, wa);
  store_s();
  if (ncc > 1) load_s(1);
  __syncthreads();
  // Collision sums run as a stream over the tile's entry list (units in slot
  // order): every iteration takes the next 256 units (one per thread,
  // straight-line code interleaved with its MFMAs) of slots up to nb - 1 ahead
  // of the one it consumes, so heavy and light slots even out. A chunk starts
  // with its slot 0 built; a slot not yet complete when its turn comes is
  // finished first (uniform branch). Masked units write a trash row; entries
  // with more than four neighbours finish after the MFMAs.
  // stream position (units) of the end of slot position i, clamped to the tile's entries so
  // that inconsistent caller tables cannot run the stream past them
  // e4m3: the slot bounds live in two VGPRs, 16 bits each (lane l of c_lo: coff[2l] and
  // coff[2l + 1]; c_hi: the next 128), read with v_readlane at a uniform index, so the bounds
  // cost no LDS read and wait inside the MFMA block (C5 -2%; bf16 gains nothing from it). The
  // bounds fit 16 bits: 16-byte entries within 160 KB of LDS number fewer than 2^14.
  uint32_t c_lo = 0u, c_hi = 0u;
  if constexpr (F8) {
    auto ent = [&](int i) { return i <= V ? static_cast<uint32_t>(min(coff[i], p.cent_stride)) : 0u; };
    c_lo = ent(2 * lane) | (ent(2 * lane + 1) << 16);
    c_hi = ent(128 + 2 * lane) | (ent(129 + 2 * lane) << 16);
  }
  auto upos = [&](int i) {
    if constexpr (F8) {
      const uint32_t lo = __builtin_amdgcn_readlane(c_lo, (i >> 1) & 63);
      const uint32_t hi = __builtin_amdgcn_readlane(c_hi, (i >> 1) & 63);
      return static_cast<int>(4u * (((i < 128 ? lo : hi) >> ((i & 1) * 16)) & 0xffffu));
    } else {
      return 4 * min(coff[i], p.cent_stride);
    }
  };
  int bpos = upos(1);
  build_heavy();
  build_range(0, bpos, true);
  uint32_t ecur[4], enxt[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) ecur[i] = srcs[rowm[i]];
  __syncthreads();

  int v = 0, cc = 0;
  // stream bounds of the current slot, read one iteration ahead
  int need = bpos, lim = upos(min(nb, V));
  // The entry of this thread's next stream unit is read an iteration ahead (the
  // entry list is static), so the unit's row reads start with the iteration;
  // read again where the stream position moves otherwise (a catch-up, a chunk
  // start).
  const uint32_t pq = static_cast<uint32_t>(tid & 3) << 4;
  auto read_ce = [&](int at, int bound) {
    const int u = at + tid;
    u32x4 e = cent[u < bound ? (u >> 2) : 0];
    if (u >= bound) e[0] = 0;     // count 0: written to the trash row
    return e;
  };
  u32x4 ce = read_ce(bpos, lim);
  // One iteration: bc holds its weight fragments and ecur its A sources; bn and
  // enxt receive the next iteration's.
  auto step = [&](const int it, u32x4 (&bc)[8], u32x4 (&bn)[8], uint32_t (&ecur)[4],
                  uint32_t (&enxt)[4]) __attribute__((always_inline)) {
    if (bpos < need) {            // slot v incomplete: finish it
      build_range(bpos, need);
      bpos = need;
      __syncthreads();
      ce = read_ce(bpos, lim);
    }
    const bool more = it + 1 < nit;
    const int vn = v + 1 == V ? 0 : v + 1;
    const int need_n = upos(vn + 1), lim_n = upos(min(vn + nb, V));

    u32x4 af[2][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t a = ecur[i] << 4;
      af[0][i] = lds16(smem, a ^ qx0);
      af[1][i] = lds16(smem, a ^ qx1);
    }
    load_w(more ? it + 1 : it, bn);
#pragma unroll
    for (int i = 0; i < 4; ++i) enxt[i] = srcs[vn * V5_MT + rowm[i]];

    // e4m3: rows 1-2 of the unit are summed in the MFMA block, rows 3-4 after it only when a
    // unit of this wave has more than two (a uniform branch; C5 -3%: in 58% of the C5 stream's
    // 16-entry windows no entry has more than two rows). Rows are still added in list order,
    // and the skipped ones are the zero row, whose +0 leaves a sum that is never -0 unchanged:
    // the same bits either way. bf16: the adds this exposes after the MFMA block in the other
    // waves cost more than the skipped ones save (C3 +2%).
    const bool wave_full = !F8 || __builtin_amdgcn_ballot_w64(((ce[0] >> 16) & 0xffu) > 2u) != 0;
    Sum sum;
    if constexpr (F8) sum = unit_sum2(ce, pq); else sum = unit_sum4(ce, pq);

    if constexpr (F8) {
      // one 32x32x64 e4m3 MFMA per block (unit scales); lane operands: 32
      // channels = the two parts, weight fragments j * 2 + 0, 1
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const i32x8 a8 = __builtin_bit_cast(i32x8, u32x8v{af[0][i][0], af[0][i][1], af[0][i][2], af[0][i][3],
                                                            af[1][i][0], af[1][i][1], af[1][i][2], af[1][i][3]});
          const u32x4 b0 = bc[j * 2], b1 = bc[j * 2 + 1];
          const i32x8 b8 = __builtin_bit_cast(i32x8, u32x8v{b0[0], b0[1], b0[2], b0[3], b1[0], b1[1], b1[2], b1[3]});
          acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a8, b8, acc[i][j], 0, 0, 0, 127, 0, 127);
        }
    } else {
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, af[ks][i]),
                                                                __builtin_bit_cast(bf16x8, bc[j * 2 + ks]), acc[i][j],
                                                                0, 0, 0);
      // Issue order (one wave per SIMD, so the wave's own MFMAs are all that can
      // cover its LDS and memory latency): each of the first 12 MFMAs followed by
      // one LDS read (A fragments, the stream's entry and rows, the next sources),
      // the next 8 each by one weight-fragment load, then the remaining 12. The
      // scheduler's default (reads bunched next to their first use, the weight
      // loads in one burst) leaves the matrix pipe idle on every wait: C3 3.66 ->
      // 3.30 ms with this order (measured against patterns with 8-19 reads first,
      // the loads first or between the reads, pairs of either: 3.30-3.77 ms).
#pragma unroll
      for (int q = 0; q < 12; ++q) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // LDS read
      }
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
        __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);   // global load
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 12, 0);
    }

    if constexpr (F8) {
      if (wave_full) {
        E::acc(sum, lds16(smem, ((ce[2] & 0xffffu) << SH) ^ pq));
        E::acc(sum, lds16(smem, ((ce[2] >> 16) << SH) ^ pq));
        unit_rest(sum, ce, pq);
      }
    } else {
      unit_rest(sum, ce, pq);
    }
    *reinterpret_cast<u32x4*>(smem + (((ce[0] >> 16) & 0xffu) ? unit_dst(ce, pq) : trash)) = E::pack(sum);
    bpos = min(bpos + 256, lim);
    ce = read_ce(bpos, lim_n);
    __syncthreads();
    v = vn;
    need = need_n;
    lim = lim_n;
    if (v == 0) {                 // chunk boundary
      ++cc;
      if (more) {                 // every MFMA of the finished chunk is done with S
        store_s();
        __syncthreads();
        if (cc + 1 < ncc) load_s(cc + 1);
        bpos = upos(1);
        build_heavy();
        build_range(0, bpos, true);
        ce = read_ce(bpos, lim);
        __syncthreads();
      }
    }
  };
  // Two iterations per trip with the register sets swapping roles: no copies at
  // the loop latch, whose moves of the next weight fragments would wait for
  // their loads (C3 ~1% faster).
  int it = 0;
  for (; it + 1 < nit; it += 2) {
    step(it, wa, wb, ecur, enxt);
    step(it + 1, wb, wa, enxt, ecur);
  }
  if (it < nit) step(it, wa, wb, ecur, enxt);

  OutT* y = static_cast<OutT*>(p.y) + b * p.ys0;
  float bo[4], sc[4];
  const float xs = F8 ? (p.x_scale_dev ? *p.x_scale_dev : p.x_scale) : 1.0f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t o = o0 + wn * 128 + j * 32 + (lane & 31);
    bo[j] = (p.bias && o < p.Cout) ? p.bias[o] : 0.0f;
    sc[j] = F8 && o < p.Cout ? xs * p.w_scale[o] : 1.0f;
  }
  // y = acc + bias (bf16); x_scale * w_scale[o] * acc + bias (e4m3)
  auto out_val = [&](float a, int j) { return epilogue(F8 ? a * sc[j] + bo[j] : a + bo[j], p.relu); };
  if (vec_out) {
    // bf16 channels-last output: each wave transposes its 32-row blocks
    // through LDS (the collision tiles, free now) and stores 16-byte pieces,
    // four 256-byte row runs per store instruction
    uint16_t* Eo = reinterpret_cast<uint16_t*>(smem + acol) + wave * 32 * 128;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
          Eo[row * 128 + j * 32 + (lane & 31)] = f32_to_bf16_bits(out_val(acc[i][j][r], j));
        }
      __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0): this wave's LDS writes are done
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const int piece = q * 64 + lane;
        const int row = piece >> 4, part = piece & 15;
        const u32x4 val = *reinterpret_cast<const u32x4*>(&Eo[row * 128 + part * 8]);
        const int64_t n = n0 + wm * 128 + i * 32 + row;
        const int64_t o = o0 + wn * 128 + part * 8;
        if (n < p.Nout && o < p.Cout)
          *reinterpret_cast<u32x4*>(reinterpret_cast<uint16_t*>(y) + n * p.ys2 + o) = val;
      }
      __builtin_amdgcn_s_waitcnt(0xc07f);
      __builtin_amdgcn_wave_barrier();
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t o = o0 + wn * 128 + j * 32 + (lane & 31);
    if (o >= p.Cout) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t n = n0 + wm * 128 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (n < p.Nout) Elem<OutT>::store(y + o * p.ys1 + n * p.ys2, out_val(acc[i][j][r], j));
      }
  }
}

template <int SV, typename OutT, int SH = 0>
__global__ __launch_bounds__(256, 1) void knnconv_bf16_v5_kernel(KnnParams p, int ncb, int64_t tiles_per_b,
                                                                 int64_t n_tiles_n, int64_t total_tiles,
                                                                 int64_t padded_tiles, int vec_out) {
  v5_body<SV, OutT, false, SH>(p, ncb, tiles_per_b, n_tiles_n, total_tiles, padded_tiles, vec_out);
}

template <int SV, typename OutT, int SH = 0>
__global__ __launch_bounds__(256, 1) void knnconv_fp8_v5_kernel(KnnParams p, int ncb, int64_t tiles_per_b,
                                                                int64_t n_tiles_n, int64_t total_tiles,
                                                                int64_t padded_tiles, int vec_out) {
  v5_body<SV, OutT, true, SH>(p, ncb, tiles_per_b, n_tiles_n, total_tiles, padded_tiles, vec_out);
}

template <int SV, bool F8, typename OutT, int SH>
static void launch_v5_kernel(const KnnParams& p, hipStream_t s, size_t lds, dim3 grid, int ncb, int64_t tiles_per_b,
                             int64_t n_tiles_n, int64_t total, int64_t padded, int vec_out) {
  const void* fn = F8 ? reinterpret_cast<const void*>(&knnconv_fp8_v5_kernel<SV, OutT, SH>)
                      : reinterpret_cast<const void*>(&knnconv_bf16_v5_kernel<SV, OutT, SH>);
  (void)reserve_dynamic_lds(fn, lds);
  if constexpr (F8)
    hipLaunchKernelGGL((knnconv_fp8_v5_kernel<SV, OutT, SH>), grid, dim3(256), lds, s, p, ncb, tiles_per_b, n_tiles_n,
                       total, padded, vec_out);
  else
    hipLaunchKernelGGL((knnconv_bf16_v5_kernel<SV, OutT, SH>), grid, dim3(256), lds, s, p, ncb, tiles_per_b, n_tiles_n,
                       total, padded, vec_out);
}

template <int SV, bool F8, int SH = 0>
static void launch_v5_sv(const KnnParams& p, int out_t, hipStream_t s) {
  const int64_t tiles_per_b = (p.Nout + V5_MT - 1) / V5_MT;
  const int64_t n_tiles_n = (p.Cout + V5_NT - 1) / V5_NT;
  const int64_t total = p.B * tiles_per_b * n_tiles_n;
  const int64_t padded = (total + 7) / 8 * 8;
  const int ncb = static_cast<int>(n_tiles_n * (V5_NT / 32));
  const int nb = v5_tiles(static_cast<int>(p.V), p.zero_row, p.coll_off_stride, p.cent_stride, p.heavy_stride,
                          p.hlist_stride);
  const size_t lds = v5_layout(static_cast<int>(p.V), p.zero_row, p.coll_off_stride, p.cent_stride,
                               p.heavy_stride, p.hlist_stride, nb).total;
  // 16-byte channels-last bf16 stores: unit channel stride, rows and base 16-byte aligned
  const int vec_out = out_t == FOVI_BF16 && p.ys1 == 1 && p.ys2 % 8 == 0 && p.ys0 % 8 == 0 && p.Cout % 8 == 0 &&
                      reinterpret_cast<uintptr_t>(p.y) % 16 == 0;
  const dim3 grid(static_cast<unsigned>(padded));
  if (out_t == FOVI_BF16)
    launch_v5_kernel<SV, F8, uint16_t, SH>(p, s, lds, grid, ncb, tiles_per_b, n_tiles_n, total, padded, vec_out);
  else
    launch_v5_kernel<SV, F8, float, SH>(p, s, lds, grid, ncb, tiles_per_b, n_tiles_n, total, padded, 0);
}

int v5_applies(const KnnParams& p, int f8) {
  if (p.w_layout != FOVI_W_MFMA) return 0;
  if (p.C % (f8 ? V5Elem<true>::CC : V5Elem<false>::CC) != 0 || p.zero_row <= 0 || p.zero_row > 1024 ||
      !p.tile_lo || !p.tile_src || !p.tile_coll_off || !p.tile_cent || !p.tile_heavy || !p.tile_hlist || p.V > 255)
    return 0;
  if (f8 && !p.w_scale) return 0;
  if (p.coll_off_stride <= p.V || p.coll_off_stride % 4 != 0 || p.cent_stride < 1) return 0;
  if (p.heavy_stride < 2 || p.heavy_stride % 2 != 0 || p.hlist_stride < 8 || p.hlist_stride % 8 != 0) return 0;
  // 16-bit row offsets (bytes, or 16-byte units), below the 0xFFFF marker of stream-built sums
  if ((p.zero_row + 1 + p.heavy_stride) * (p.wide_units ? V5_ROW / 16 : V5_ROW) >= 0xffff) return 0;
  if ((reinterpret_cast<uintptr_t>(p.tile_src) | reinterpret_cast<uintptr_t>(p.tile_coll_off) |
       reinterpret_cast<uintptr_t>(p.tile_cent) | reinterpret_cast<uintptr_t>(p.tile_heavy) |
       reinterpret_cast<uintptr_t>(p.tile_hlist)) % 16 != 0)
    return 0;
  // channels-last rows, 16-byte aligned
  const int64_t al = f8 ? 16 : 8;
  if (p.xs1 != 1 || p.xs2 % al != 0 || p.xs0 % al != 0 || reinterpret_cast<uintptr_t>(p.x) % 16 != 0) return 0;
  if (reinterpret_cast<uintptr_t>(p.w) % 16 != 0) return 0;
  return v5_layout(static_cast<int>(p.V), p.zero_row, p.coll_off_stride, p.cent_stride, p.heavy_stride,
                   p.hlist_stride, V5_NB_MIN).total <= 160 * 1024;
}

template <bool F8>
static int launch_v5(const KnnParams& p, int out_t, hipStream_t s) {
  const int sv = (p.zero_row * 4 + 255) / 256;
  if (p.wide_units) {                 // 16-byte-unit tables: more than 1023 staged rows
    if (sv > 16) return 1;
    launch_v5_sv<16, F8, 4>(p, out_t, s);
    return 0;
  }
  if (sv <= 4) launch_v5_sv<4, F8>(p, out_t, s);
  else if (sv <= 8) launch_v5_sv<8, F8>(p, out_t, s);
  else if (sv <= 12) launch_v5_sv<12, F8>(p, out_t, s);
  else if (sv <= 16) launch_v5_sv<16, F8>(p, out_t, s);
  else return 1;
  return 0;
}

int v5_tiles_of(const KnnParams& p) {
  return v5_tiles(static_cast<int>(p.V), p.zero_row, p.coll_off_stride, p.cent_stride, p.heavy_stride,
                  p.hlist_stride);
}

int launch_knnconv_bf16_v5(const KnnParams& p, int out_t, hipStream_t s) { return launch_v5<false>(p, out_t, s); }
int launch_knnconv_fp8_v5(const KnnParams& p, int out_t, hipStream_t s) { return launch_v5<true>(p, out_t, s); }

// Fragment-order weight, 1 KB fragments f = (it * ncb + cb) * 2 + h with
// it = chunk * n_ref + p and slot v = order[p] (v = p without an order);
// lane l of fragment f holds w[o = cb * 32 + l % 32][c * n_ref + v] (zero for
// o >= c_out) for
//  * bf16 (32-channel chunks), e < 8: c % 32 = h * 16 + (l / 32) * 8 + e;
//  * e4m3 (64-channel chunks, divided by w_scale[o]), e < 16:
//    c % 64 = (l / 32) * 32 + h * 16 + e.
__global__ void pack_weight_mfma_kernel(const float* w_ref, int64_t c_out, int64_t c_in, int64_t n_ref, void* out,
                                        int64_t ncb, int64_t total, const int32_t* order, const float* w_scale) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const bool f8 = w_scale != nullptr;
  const int eb = f8 ? 4 : 3;   // log2 of elements per lane and fragment
  const int e = static_cast<int>(idx & ((1 << eb) - 1));
  const int l = static_cast<int>((idx >> eb) & 63);
  const int64_t frag = idx >> (eb + 6);
  const int h = static_cast<int>(frag & 1);
  const int64_t cb = (frag >> 1) % ncb;
  const int64_t it = (frag >> 1) / ncb;
  const int64_t pos = it % n_ref, cc = it / n_ref;
  const int64_t v = order ? order[pos] : pos;
  const int64_t o = cb * 32 + (l & 31);
  const int64_t c = f8 ? cc * 64 + (l >> 5) * 32 + h * 16 + e : cc * 32 + h * 16 + (l >> 5) * 8 + e;
  const float val = o < c_out ? w_ref[o * c_in * n_ref + c * n_ref + v] : 0.0f;
  if (f8) static_cast<uint8_t*>(out)[idx] = o < c_out ? f32_to_e4m3(val / w_scale[o]) : 0;
  else static_cast<uint16_t*>(out)[idx] = f32_to_bf16_bits(val);
}

}  // namespace fovi

extern "C" int fovi_knnconv_wide_tiles(int64_t n_ref, int32_t zero_row, int32_t coll_off_stride,
                                       int32_t cent_stride, int32_t heavy_stride, int32_t hlist_stride,
                                       int64_t* lds_bytes) {
  using namespace fovi;
  clear_error();
  // n_ref below 2^16 and sizes up to 2^20 keep the layout's 32-bit byte count below 2^28
  constexpr int64_t lim = int64_t(1) << 20;
  if (n_ref < 0 || n_ref >= (int64_t(1) << 16) || zero_row < 0 || zero_row > lim || coll_off_stride < 0 || coll_off_stride > lim ||
      cent_stride < 0 || cent_stride > lim || heavy_stride < 0 || heavy_stride > lim || hlist_stride < 0 ||
      hlist_stride > lim) {
    set_error("fovi_knnconv_wide_tiles: n_ref must lie in [0, 2^16), the other sizes in [0, 2^20]");
    return 0;
  }
  const int V = static_cast<int>(n_ref);
  const int nb = v5_tiles(V, zero_row, coll_off_stride, cent_stride, heavy_stride, hlist_stride);
  if (lds_bytes)
    *lds_bytes = static_cast<int64_t>(
        v5_layout(V, zero_row, coll_off_stride, cent_stride, heavy_stride, hlist_stride, nb).total);
  return nb;
}

extern "C" int64_t fovi_knnconv_weight_mfma_elems(int64_t c_out, int64_t c_in, int64_t n_ref) {
  using namespace fovi;
  if (c_out <= 0 || c_in <= 0 || n_ref <= 0 || c_in % 32 != 0) return -1;
  const int64_t ncb = (c_out + V5_NT - 1) / V5_NT * (V5_NT / 32);
  return c_in * n_ref * ncb * 32;
}

extern "C" int fovi_knnconv_pack_weight_mfma(const float* w_ref, int64_t c_out, int64_t c_in, int64_t n_ref,
                                             void* w_frag, int32_t out_dtype, const int32_t* slot_order,
                                             const float* w_scale, void* stream) {
  using namespace fovi;
  clear_error();
  if (!w_ref || !w_frag) { set_error("fovi_knnconv_pack_weight_mfma: null pointer"); return 1; }
  if (out_dtype != FOVI_BF16 && out_dtype != FOVI_F8E4M3) {
    set_error("fovi_knnconv_pack_weight_mfma: out_dtype must be BF16 or F8E4M3"); return 1;
  }
  if (out_dtype == FOVI_F8E4M3 && (!w_scale || c_in % 64 != 0)) {
    set_error("fovi_knnconv_pack_weight_mfma: F8E4M3 needs w_scale and c_in %% 64 == 0"); return 1;
  }
  const int64_t total = fovi_knnconv_weight_mfma_elems(c_out, c_in, n_ref);
  if (total < 0) {
    set_error("fovi_knnconv_pack_weight_mfma: bad sizes c_out=%lld c_in=%lld (multiple of 32) n_ref=%lld",
              (long long)c_out, (long long)c_in, (long long)n_ref);
    return 1;
  }
  const int64_t ncb = (c_out + V5_NT - 1) / V5_NT * (V5_NT / 32);
  hipLaunchKernelGGL(pack_weight_mfma_kernel, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), w_ref, c_out, c_in, n_ref, w_frag, ncb, total, slot_order,
                     out_dtype == FOVI_F8E4M3 ? w_scale : nullptr);
  return check_launch("fovi_knnconv_pack_weight_mfma");
}
