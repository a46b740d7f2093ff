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
//    from S (an LDS zero row serves empty slots); slots with two or more
//    neighbours are summed in fp32 (one RNE rounding) into a double-buffered
//    collision tile one iteration ahead, from per-(tile, slot) row lists.
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
constexpr int V5_CC = 32;    // channels per reduction chunk (one 64-byte LDS row)

struct V5Layout {
  int acol_off, src_off, coff_off, coll4_off, nbl_off, s_off, total;  // bytes
};

__host__ __device__ inline V5Layout v5_layout(int V, int K, int zero_row, int coff_stride, int coll4_stride) {
  V5Layout l;
  int o = 0;
  l.acol_off = o;   o += (2 * V5_MT + 1) * V5_CC * 2; // two 256 x 32 bf16 collision tiles + a trash row
  l.src_off = o;    o += V * V5_MT * 2;             // per (slot, row) source row, slot-major
  l.coff_off = o;   o += coff_stride * 4;           // per-slot collision entry offsets
  l.coll4_off = o;  o += coll4_stride * 8;          // packed collision entries
  l.nbl_off = o;    o += V5_MT * K * 2;             // neighbour lists (rows with > 4 neighbours)
  o = (o + 127) & ~127;                             // rows 128-byte aligned (fragment offsets are XORed)
  l.s_off = o;      o += (zero_row + 1) * V5_CC * 2; // staged rows + zero row
  l.total = o;
  return l;
}

// Index of the 1 KB weight fragment (iteration it, 32-column block cb,
// half ks) in the MFMA-fragment order; iteration it = chunk * n_ref + slot.
__host__ __device__ inline int64_t v5_frag(int64_t it, int64_t ncb, int64_t cb, int ks) {
  return (it * ncb + cb) * 2 + ks;
}

// Staged-row index of neighbour j (< 4) of a packed collision entry.
__device__ __forceinline__ int coll4_row(uint64_t w, int j) { return static_cast<int>((w >> (24 + 10 * j)) & 0x3ff); }

template <int SV, typename OutT>
__global__ __launch_bounds__(256, 1) void knnconv_bf16_v5_kernel(KnnParams p, int ncb, int64_t tiles_per_b,
                                                                 int64_t n_tiles_n, int64_t total_tiles,
                                                                 int64_t padded_tiles, int vec_out) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int V = static_cast<int>(p.V), K = static_cast<int>(p.K);
  const int zr = p.zero_row;
  const V5Layout L = v5_layout(V, K, zr, p.coll_off_stride, p.coll4_stride);
  uint16_t* sm16 = reinterpret_cast<uint16_t*>(smem);
  const uint16_t* srcs = reinterpret_cast<const uint16_t*>(smem + L.src_off);
  const int32_t* coff = reinterpret_cast<const int32_t*>(smem + L.coff_off);
  const uint64_t* coll4 = reinterpret_cast<const uint64_t*>(smem + L.coll4_off);
  const uint16_t* nbl = reinterpret_cast<const uint16_t*>(smem + L.nbl_off);
  const int s16 = L.s_off / 2;                    // S offset in bf16 elements
  uint16_t* S = sm16 + s16;

  const int64_t tile = xcd_tile(blockIdx.x, padded_tiles);
  if (tile >= total_tiles) return;
  const int64_t mt = tile / n_tiles_n;
  const int64_t tn = tile % n_tiles_n;
  const int64_t o0 = tn * V5_NT;
  const int64_t b = mt / tiles_per_b;
  const int64_t pt = mt % tiles_per_b;
  const int64_t n0 = pt * V5_MT;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  const int64_t lo = p.tile_lo[pt];
  const int span = static_cast<int>(min(static_cast<int64_t>(zr), p.Nin - lo));

  const char* xrows = reinterpret_cast<const char*>(static_cast<const uint16_t*>(p.x) + b * p.xs0 + lo * p.xs2);
  uint32_t s_off[SV];
  uint32_t s_ok = 0;
#pragma unroll
  for (int j = 0; j < SV; ++j) {
    const int q = tid + 256 * j;
    s_ok |= static_cast<uint32_t>((q >> 2) < span) << j;
    s_off[j] = static_cast<uint32_t>(((q >> 2) * p.xs2 + (q & 3) * 8) * 2);
  }
  const int ncc = static_cast<int>(p.C / V5_CC);
  const int nit = ncc * V;
  // this wave's weight fragments: column blocks cb0 .. cb0 + 3, lane-contiguous
  const u32x4* wq = reinterpret_cast<const u32x4*>(p.w) + lane;
  const int64_t cb0 = tn * (V5_NT / 32) + wn * 4;

  u32x4 rs[SV];
  auto load_s = [&](int cc) {
    const char* base = xrows + cc * V5_CC * 2;
#pragma unroll
    for (int j = 0; j < SV; ++j)
      rs[j] = ((s_ok >> j) & 1) ? *reinterpret_cast<const u32x4*>(base + s_off[j]) : u32x4{0u, 0u, 0u, 0u};
  };
  auto store_s = [&]() {
#pragma unroll
    for (int j = 0; j < SV; ++j) {
      const int q = tid + 256 * j;
      if ((s_ok >> j) & 1) *reinterpret_cast<u32x4*>(&S[swz32(q >> 2, q & 3)]) = rs[j];
    }
  };
  auto load_w = [&](int it, u32x4 (&dst)[8]) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) dst[j * 2 + ks] = wq[v5_frag(it, ncb, cb0 + j, ks) * 64];
  };

  // Prologue: the first chunk's rows and the tile's tables, all loads in
  // flight together (16-byte copies; the tables are laid out on the host in
  // this LDS order).
  load_s(0);
  {
    const int n_src = V * V5_MT * 2 / 16, n_coff = p.coll_off_stride * 4 / 16;
    const int n_c4 = p.coll4_stride * 8 / 16, n_nbl = V5_MT * K * 2 / 16;
    const u32x4* g_src = reinterpret_cast<const u32x4*>(p.tile_src + pt * V * V5_MT);
    const u32x4* g_coff = reinterpret_cast<const u32x4*>(p.tile_coll_off + pt * p.coll_off_stride);
    const u32x4* g_c4 = reinterpret_cast<const u32x4*>(p.tile_coll4 + pt * p.coll4_stride);
    const u32x4* g_nbl = reinterpret_cast<const u32x4*>(p.tile_nbr + n0 * p.K);
    u32x4* d_src = reinterpret_cast<u32x4*>(smem + L.src_off);
    u32x4* d_coff = reinterpret_cast<u32x4*>(smem + L.coff_off);
    u32x4* d_c4 = reinterpret_cast<u32x4*>(smem + L.coll4_off);
    u32x4* d_nbl = reinterpret_cast<u32x4*>(smem + L.nbl_off);
    const int total = n_src + n_coff + n_c4 + n_nbl;
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
        if (i < n_c4) { t[u] = g_c4[i]; dst[u] = d_c4 + i; continue; }
        i -= n_c4;
        if (i < n_nbl) { t[u] = g_nbl[i]; dst[u] = d_nbl + i; }
      }
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (dst[u]) *dst[u] = t[u];
    }
  }
  if (tid < 4) *reinterpret_cast<u32x4*>(&S[zr * V5_CC + tid * 8]) = u32x4{0u, 0u, 0u, 0u};

  // Full sums of slot v's collision rows into tile `buf` (all neighbours; used
  // at chunk boundaries and for lists longer than the in-loop straight-line part).
  auto coll_item = [&](int v, int buf, int item) {
    const uint64_t w = coll4[coff[v] + (item >> 2)];
    const int part = item & 3;
    const int row = static_cast<int>(w & 0xff), cnt = static_cast<int>((w >> 8) & 0xff);
    f32x8 acc8 = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j) acc8 += unpack_bf16x8(*reinterpret_cast<const u32x4*>(&S[swz32(coll4_row(w, j), part)]));
    const uint16_t* nb = nbl + row * K + ((w >> 16) & 0xff);
    for (int j = 4; j < cnt; ++j) acc8 += unpack_bf16x8(*reinterpret_cast<const u32x4*>(&S[swz32(nb[j], part)]));
    *reinterpret_cast<u32x4*>(&sm16[buf * V5_MT * V5_CC + swz32(row, part)]) =
        u32x4{cvt_pk_bf16(acc8[0], acc8[1]), cvt_pk_bf16(acc8[2], acc8[3]), cvt_pk_bf16(acc8[4], acc8[5]),
              cvt_pk_bf16(acc8[6], acc8[7])};
  };
  auto build_coll = [&](int v, int buf) {
    const int items = (coff[v + 1] - coff[v]) * 4;
    for (int item = tid; item < items; item += 256) coll_item(v, buf, item);
  };

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  int rowm[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) rowm[i] = wm * 128 + i * 32 + (lane & 31);

  u32x4 bcur[8], bnxt[8];
  load_w(0, bcur);
  store_s();
  if (ncc > 1) load_s(1);
  __syncthreads();
  build_coll(0, 0);
  uint32_t ecur[4], enxt[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) ecur[i] = srcs[rowm[i]];
  __syncthreads();

  // In-loop collision sums for the next iteration, written as straight-line
  // code so that they interleave with this iteration's MFMAs: each thread owns
  // items tid and tid + 256 (item = collision entry * 4 + 16-byte part) and
  // sums the entry's first four neighbours (missing ones are the zero row);
  // masked items write a trash row. Entries with more than four neighbours
  // (the head of each slot's list, which is sorted by count) finish in a
  // short loop after the MFMAs, and lists longer than 128 entries in the
  // generic loop.
  const int trash = 2 * V5_MT * V5_CC;
  int cc1 = 0, v1 = 0;
  for (int it = 0; it < nit; ++it) {
    const int cur = it & 1;
    if (++v1 == V) { v1 = 0; ++cc1; }
    const bool more = it + 1 < nit;
    const int itn = more ? it + 1 : it;
    const int vn = v1;   // slot of the next iteration (chunk boundaries build after the S refresh)
    const int c0 = coff[vn];
    const int items = (more && v1 != 0) ? (coff[vn + 1] - c0) * 4 : 0;

    int src[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      src[i] = (ecur[i] & 0x8000u) ? cur * V5_MT * V5_CC + swz32(rowm[i], 0)
                                   : s16 + swz32(static_cast<int>(ecur[i]), 0);
    bf16x8 af[2][4];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        // swz32(r, q) = swz32(r, 0) ^ (q << 3) within the row (XOR of the 16-byte part)
        af[ks][i] = *reinterpret_cast<const bf16x8*>(&sm16[src[i] ^ ((ks * 2 + (lane >> 5)) << 3)]);

    load_w(itn, bnxt);
#pragma unroll
    for (int i = 0; i < 4; ++i) enxt[i] = srcs[v1 * V5_MT + rowm[i]];

    uint64_t w_k[2];
    int part_k[2];
    f32x8 sum_k[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int item = tid + 256 * k;
      const bool valid = item < items;
      const uint64_t w = coll4[valid ? c0 + (item >> 2) : 0];
      const int part = item & 3;
      f32x8 acc8 = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc8 += unpack_bf16x8(*reinterpret_cast<const u32x4*>(&S[swz32(coll4_row(w, j), part)]));
      w_k[k] = valid ? w : 0;      // count 0: nothing left to add, written to the trash row
      part_k[k] = part;
      sum_k[k] = acc8;
    }

#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[ks][i], __builtin_bit_cast(bf16x8, bcur[j * 2 + ks]),
                                                              acc[i][j], 0, 0, 0);

#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const uint64_t w = w_k[k];
      const int cnt = static_cast<int>((w >> 8) & 0xff), row = static_cast<int>(w & 0xff);
      if (cnt > 4) {                      // neighbours 5 .. count, in order
        const uint16_t* nb = nbl + row * K + ((w >> 16) & 0xff);
        for (int j = 4; j < cnt; ++j)
          sum_k[k] += unpack_bf16x8(*reinterpret_cast<const u32x4*>(&S[swz32(nb[j], part_k[k])]));
      }
      const f32x8 a8 = sum_k[k];
      const int dst = cnt > 0 ? (cur ^ 1) * V5_MT * V5_CC + swz32(row, part_k[k]) : trash;
      *reinterpret_cast<u32x4*>(&sm16[dst]) =
          u32x4{cvt_pk_bf16(a8[0], a8[1]), cvt_pk_bf16(a8[2], a8[3]), cvt_pk_bf16(a8[4], a8[5]),
                cvt_pk_bf16(a8[6], a8[7])};
    }
    for (int item = tid + 512; item < items; item += 256) coll_item(vn, cur ^ 1, item);
    __syncthreads();
    if (more && v1 == 0) {      // chunk boundary: every MFMA of chunk cc1-1 is done with S
      store_s();
      __syncthreads();
      if (cc1 + 1 < ncc) load_s(cc1 + 1);
      build_coll(0, cur ^ 1);
      __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) ecur[i] = enxt[i];
#pragma unroll
    for (int k = 0; k < 8; ++k) bcur[k] = bnxt[k];
  }

  OutT* y = static_cast<OutT*>(p.y) + b * p.ys0;
  float bo[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t o = o0 + wn * 128 + j * 32 + (lane & 31);
    bo[j] = (p.bias && o < p.Cout) ? p.bias[o] : 0.0f;
  }
  if (vec_out) {
    // bf16 channels-last output: each wave transposes its 32-row blocks
    // through LDS (the collision tiles, free now) and stores 16-byte pieces,
    // four 256-byte row runs per store instruction
    uint16_t* E = sm16 + wave * 32 * 128;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
          E[row * 128 + j * 32 + (lane & 31)] = f32_to_bf16_bits(epilogue(acc[i][j][r] + bo[j], p.relu));
        }
      __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0): this wave's LDS writes are done
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const int piece = q * 64 + lane;
        const int row = piece >> 4, part = piece & 15;
        const u32x4 val = *reinterpret_cast<const u32x4*>(&E[row * 128 + part * 8]);
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
        if (n < p.Nout) Elem<OutT>::store(y + o * p.ys1 + n * p.ys2, epilogue(acc[i][j][r] + bo[j], p.relu));
      }
  }
}

template <int SV>
static void launch_v5_sv(const KnnParams& p, int out_t, hipStream_t s) {
  const int64_t tiles_per_b = (p.Nout + V5_MT - 1) / V5_MT;
  const int64_t n_tiles_n = (p.Cout + V5_NT - 1) / V5_NT;
  const int64_t total = p.B * tiles_per_b * n_tiles_n;
  const int64_t padded = (total + 7) / 8 * 8;
  const int ncb = static_cast<int>(n_tiles_n * (V5_NT / 32));
  const size_t lds = v5_layout(static_cast<int>(p.V), static_cast<int>(p.K), p.zero_row, p.coll_off_stride,
                               p.coll4_stride).total;
  // 16-byte channels-last bf16 stores: unit channel stride, rows and base 16-byte aligned
  const int vec_out = out_t == FOVI_BF16 && p.ys1 == 1 && p.ys2 % 8 == 0 && p.ys0 % 8 == 0 && p.Cout % 8 == 0 &&
                      reinterpret_cast<uintptr_t>(p.y) % 16 == 0;
  dim3 grid(static_cast<unsigned>(padded));
  if (out_t == FOVI_BF16) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&knnconv_bf16_v5_kernel<SV, uint16_t>),
                        hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    hipLaunchKernelGGL((knnconv_bf16_v5_kernel<SV, uint16_t>), grid, dim3(256), lds, s, p, ncb, tiles_per_b,
                       n_tiles_n, total, padded, vec_out);
  } else {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&knnconv_bf16_v5_kernel<SV, float>),
                        hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    hipLaunchKernelGGL((knnconv_bf16_v5_kernel<SV, float>), grid, dim3(256), lds, s, p, ncb, tiles_per_b,
                       n_tiles_n, total, padded, 0);
  }
}

int v5_applies(const KnnParams& p) {
  if (p.w_layout != FOVI_W_MFMA) return 0;
  if (p.C % V5_CC != 0 || p.zero_row <= 0 || p.zero_row > 1023 || !p.tile_lo || !p.tile_nbr || !p.tile_src ||
      !p.tile_coll_off || !p.tile_coll4 || p.K > 255 || p.V > 255)
    return 0;
  if (p.coll_off_stride <= p.V || p.coll_off_stride % 4 != 0 || p.coll4_stride < 2 || p.coll4_stride % 2 != 0) return 0;
  if ((reinterpret_cast<uintptr_t>(p.tile_src) | reinterpret_cast<uintptr_t>(p.tile_coll_off) |
       reinterpret_cast<uintptr_t>(p.tile_coll4) | reinterpret_cast<uintptr_t>(p.tile_nbr)) % 16 != 0)
    return 0;
  if (p.xs1 != 1 || p.xs2 % 8 != 0 || p.xs0 % 8 != 0 || reinterpret_cast<uintptr_t>(p.x) % 16 != 0) return 0;
  if (reinterpret_cast<uintptr_t>(p.w) % 16 != 0) return 0;
  return v5_layout(static_cast<int>(p.V), static_cast<int>(p.K), p.zero_row, p.coll_off_stride, p.coll4_stride)
             .total <= 160 * 1024;
}

int launch_knnconv_bf16_v5(const KnnParams& p, int out_t, hipStream_t s) {
  const int sv = (p.zero_row * 4 + 255) / 256;
  if (sv <= 4) launch_v5_sv<4>(p, out_t, s);
  else if (sv <= 8) launch_v5_sv<8>(p, out_t, s);
  else if (sv <= 12) launch_v5_sv<12>(p, out_t, s);
  else if (sv <= 16) launch_v5_sv<16>(p, out_t, s);
  else return 1;
  return 0;
}

// Fragment-order weight: fragment (it, cb, ks) holds, for lane l and e < 8,
// w[o = cb * 32 + l % 32][c * n_ref + v] with it = (c / 32) * n_ref + v and
// c % 32 = ks * 16 + (l / 32) * 8 + e (zero for o >= c_out).
__global__ void pack_weight_mfma_kernel(const float* w_ref, int64_t c_out, int64_t c_in, int64_t n_ref,
                                        uint16_t* out, int64_t ncb, int64_t total) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int e = static_cast<int>(idx & 7);
  const int l = static_cast<int>((idx >> 3) & 63);
  const int64_t frag = idx >> 9;
  const int ks = static_cast<int>(frag & 1);
  const int64_t cb = (frag >> 1) % ncb;
  const int64_t it = (frag >> 1) / ncb;
  const int64_t v = it % n_ref, cc = it / n_ref;
  const int64_t o = cb * 32 + (l & 31);
  const int64_t c = cc * V5_CC + ks * 16 + (l >> 5) * 8 + e;
  const float val = o < c_out ? w_ref[o * c_in * n_ref + c * n_ref + v] : 0.0f;
  out[idx] = f32_to_bf16_bits(val);
}

}  // namespace fovi

extern "C" int64_t fovi_knnconv_weight_mfma_elems(int64_t c_out, int64_t c_in, int64_t n_ref) {
  using namespace fovi;
  if (c_out <= 0 || c_in <= 0 || n_ref <= 0 || c_in % V5_CC != 0) return -1;
  const int64_t ncb = (c_out + V5_NT - 1) / V5_NT * (V5_NT / 32);
  return c_in * n_ref * ncb * 32;
}

extern "C" int fovi_knnconv_pack_weight_mfma(const float* w_ref, int64_t c_out, int64_t c_in, int64_t n_ref,
                                             void* w_frag, int32_t out_dtype, void* stream) {
  using namespace fovi;
  clear_error();
  if (!w_ref || !w_frag) { set_error("fovi_knnconv_pack_weight_mfma: null pointer"); return 1; }
  if (out_dtype != FOVI_BF16) { set_error("fovi_knnconv_pack_weight_mfma: only BF16 is supported"); return 1; }
  const int64_t total = fovi_knnconv_weight_mfma_elems(c_out, c_in, n_ref);
  if (total < 0) {
    set_error("fovi_knnconv_pack_weight_mfma: bad sizes c_out=%lld c_in=%lld (multiple of 32) n_ref=%lld",
              (long long)c_out, (long long)c_in, (long long)n_ref);
    return 1;
  }
  const int64_t ncb = (c_out + V5_NT - 1) / V5_NT * (V5_NT / 32);
  hipLaunchKernelGGL(pack_weight_mfma_kernel, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), w_ref, c_out, c_in, n_ref, static_cast<uint16_t*>(w_frag),
                     ncb, total);
  return check_launch("fovi_knnconv_pack_weight_mfma");
}
