// kNN-convolution forward, bf16, for layers with few input channels (c_in <= 8;
// input rows padded to CP = 4 or 8 channels): the sensor's first layer (C2
// layer 1) and the DINOv3 patch embedding (C4), fused into one pass.
//
// GEMM view: rows = (b, n) output points, columns = output channels, reduction
// = (slot v, channel c), column v * CP + c, as the row-packed weight
// (fovi_knnconv_pack_weight with c_slot = CP). A workgroup (8 waves, two per
// SIMD) owns TM consecutive output points of one image and every output
// channel (NTP, c_out rounded up to the wave tiling):
//  * The tile's input rows form one contiguous index range; they are staged
//    in LDS once (S, CP channels per row, channels >= c_in zeroed), plus a
//    zero row.
//  * The reduction runs in chunks of 64 columns (64 / CP slots). A chunk's A
//    tile [TM x 64] is cleared and its non-empty (point, slot) sums are built
//    in LDS from S by "items": up to 8 neighbours summed in fp32 in list order
//    from +0 and rounded once to bf16. A longer list (the fovea's slots hold
//    up to ~120 neighbours) is one item per group of 8, each writing its fp32
//    partial sum, and a combine entry adds the partials in order and rounds
//    once: a long list no longer serialises its wave (and the barrier after
//    the build) for its whole length. Items come from a host table, sorted by
//    neighbour count and dealt in a snake over the threads (lanes of a wave
//    hold items of similar counts); each is 8 bytes (first neighbour's S row,
//    count, destination, offset of the further neighbours in the chunk's
//    extras list, which is staged in LDS). The slot sums equal the two-pass
//    path's (slotsum_kernel, same grouped order) bit for bit.
//  * The weight chunk [NTP x 64] is staged in LDS once per workgroup and read
//    by all waves; A and weight rows are 128 bytes, 16-byte parts XOR-swizzled
//    by bits 1-3 of the row (conflict-free fragment reads).
//  * Per chunk: the MFMAs of chunk c (32x32x16 bf16, ascending K, as the
//    two-pass GEMM) and the build of chunk c + 1's A tile into the other A
//    buffer; after a barrier, chunk c + 1's long lists are combined, chunk c's
//    buffer is cleared for chunk c + 2, and the weight and extras of the next
//    chunks (loaded into registers one chunk ahead) are stored; two barriers
//    per chunk.
//  * Epilogue: bias and ReLU, each wave transposes its tile through LDS and
//    stores 16-byte pieces of channels-last rows.
#include "knnconv_internal.h"

namespace fovi {

constexpr int FC_KC = 64;          // reduction columns per chunk
constexpr int FC_ROWB = FC_KC * 2; // bytes of an A or weight row in LDS

struct FewcTables {
  const int32_t* lo;       // [n_tiles] first staged input row
  const int32_t* span;     // [n_tiles] staged rows
  const uint32_t* item;    // [n_tiles, n_chunks, TM * SPC] x 2 words
  const uint16_t* xlist;   // extras, per (tile, chunk) blocks
  const int32_t* xoff;     // [n_tiles * n_chunks + 1] block starts (uint16 units, multiples of 8)
  const uint32_t* comb;    // combine entries, per (tile, chunk) blocks
  const int32_t* comb_off; // [n_tiles * n_chunks + 1] block starts
  int zero_row;            // S row of zeros (>= every span)
  int xmax;                // largest extras block (uint16 units, multiple of 8)
  int pmax;                // most partial sums of a chunk
  int n_chunks;
};

struct FewcLayout {
  int s_off, a_off, w_off, x_off, p_off, total;
};

__host__ __device__ inline FewcLayout fewc_layout(int tm, int ntp, int cp, int zero_row, int xmax, int pmax,
                                                  int epi_bytes) {
  FewcLayout l;
  int o = 0;
  l.s_off = o; o += ((zero_row + 1) * cp * 2 + 15) & ~15;
  l.a_off = o; o += 2 * tm * FC_ROWB;
  l.w_off = o; o += ntp * FC_ROWB;
  l.x_off = o; o += (xmax * 2 + 15) & ~15;
  l.p_off = o; o += pmax * cp * 4;
  l.total = o > epi_bytes ? o : epi_bytes;
  return l;
}

// Byte offset of 16-byte part q of 128-byte row r: the part index XOR bits 1-3
// of r, so 8 consecutive rows' part q occupy 8 distinct 16-byte bank groups,
// and 16 consecutive rows all 16 groups of a 256-byte bank window.
__device__ __forceinline__ uint32_t fc_off(int r, int q) {
  return static_cast<uint32_t>(r * FC_ROWB + ((q ^ ((r >> 1) & 7)) << 4));
}

template <int CP> struct FcRow;
template <> struct FcRow<4> {
  typedef uint2 T;
  static __device__ __forceinline__ void acc(float* a, T v) {
    a[0] += __uint_as_float(v.x << 16); a[1] += __uint_as_float(v.x & 0xffff0000u);
    a[2] += __uint_as_float(v.y << 16); a[3] += __uint_as_float(v.y & 0xffff0000u);
  }
  static __device__ __forceinline__ T pack(const float* a) { return T{cvt_pk_bf16(a[0], a[1]), cvt_pk_bf16(a[2], a[3])}; }
  static __device__ __forceinline__ T mask(T v, const uint32_t* m) { return T{v.x & m[0], v.y & m[1]}; }
};
template <> struct FcRow<8> {
  typedef u32x4 T;
  static __device__ __forceinline__ void acc(float* a, T v) {
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      a[2 * w] += __uint_as_float(v[w] << 16);
      a[2 * w + 1] += __uint_as_float(v[w] & 0xffff0000u);
    }
  }
  static __device__ __forceinline__ T pack(const float* a) {
    return T{cvt_pk_bf16(a[0], a[1]), cvt_pk_bf16(a[2], a[3]), cvt_pk_bf16(a[4], a[5]), cvt_pk_bf16(a[6], a[7])};
  }
  static __device__ __forceinline__ T mask(T v, const uint32_t* m) { return T{v[0] & m[0], v[1] & m[1], v[2] & m[2], v[3] & m[3]}; }
};

// TM output points per tile, WM x (8 / WM) waves, each wave RB x CB blocks of
// 32 x 32 (rows x columns), CP channels per input row.
template <int TM, int WM, int RB, int CB, int CP, int XV>
__global__ __launch_bounds__(512, 1) void knnconv_fewc_kernel(KnnParams p, FewcTables ft, int64_t tiles_per_b,
                                                              int64_t total_tiles, int64_t padded_tiles,
                                                              int vec_out) {
  constexpr int WN = 8 / WM;
  constexpr int NTP = WN * CB * 32;
  constexpr int SPC = FC_KC / CP;            // slots per chunk
  constexpr int IT = TM * SPC / 512;         // items per thread per chunk
  constexpr int WV = NTP * (FC_ROWB / 16) / 512;   // weight pieces per thread per chunk
  static_assert(RB * 32 * WM == TM, "wave rows");
  static_assert(IT >= 1 && TM * SPC % 512 == 0, "items per thread");
  static_assert(WV >= 1 && NTP * (FC_ROWB / 16) % 512 == 0, "weight pieces per thread");
  typedef FcRow<CP> R;
  typedef typename R::T RowT;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

  const int64_t lt = xcd_tile(blockIdx.x, padded_tiles);
  if (lt >= total_tiles) return;
  const int64_t b = lt / tiles_per_b;
  const int t = static_cast<int>(lt % tiles_per_b);
  const int64_t n0 = static_cast<int64_t>(t) * TM;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave % WM, wn = wave / WM;
  const int zr = ft.zero_row;
  const FewcLayout L = fewc_layout(TM, NTP, CP, zr, ft.xmax, ft.pmax, 0);
  const int NC = ft.n_chunks;

  // Stage the tile's input rows (channels >= c_in zeroed) and the zero row.
  {
    uint32_t cm[CP / 2];
#pragma unroll
    for (int w = 0; w < CP / 2; ++w)
      cm[w] = (2 * w < p.C ? 0x0000ffffu : 0u) | (2 * w + 1 < p.C ? 0xffff0000u : 0u);
    const int lo = ft.lo[t], span = ft.span[t];
    const RowT* src = reinterpret_cast<const RowT*>(static_cast<const uint16_t*>(p.x) + b * p.xs0 +
                                                   static_cast<int64_t>(lo) * CP);
    RowT* S = reinterpret_cast<RowT*>(smem + L.s_off);
    for (int r0 = 0; r0 < span; r0 += 8 * 512) {
      RowT v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int r = r0 + u * 512 + tid;
        if (r < span) v[u] = src[r];
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int r = r0 + u * 512 + tid;
        if (r < span) S[r] = R::mask(v[u], cm);
      }
    }
    if (tid == 0) {
      RowT z;
#pragma unroll
      for (int w = 0; w < CP / 2; ++w) reinterpret_cast<uint32_t*>(&z)[w] = 0u;
      S[zr] = z;
    }
  }

  const uint2* items = reinterpret_cast<const uint2*>(ft.item) + static_cast<int64_t>(t) * NC * (TM * SPC);
  auto load_items = [&](int c, uint2 (&dst)[IT]) {
    const uint2* src = items + static_cast<int64_t>(c) * (TM * SPC);
#pragma unroll
    for (int j = 0; j < IT; ++j) dst[j] = src[j * 512 + tid];
  };
  // weight chunk c: column o's 128 bytes at w + (o * k_pad + 64 c) * 2; columns >= c_out are zero
  const uint16_t* wg = static_cast<const uint16_t*>(p.w);
  auto load_w = [&](int c, u32x4 (&dst)[WV]) {
#pragma unroll
    for (int j = 0; j < WV; ++j) {
      const int q = j * 512 + tid, o = q >> 3, part = q & 7;
      dst[j] = o < p.Cout ? *reinterpret_cast<const u32x4*>(wg + static_cast<int64_t>(o) * p.Kpad + c * FC_KC + part * 8)
                          : u32x4{0u, 0u, 0u, 0u};
    }
  };
  auto store_w = [&](const u32x4 (&src)[WV]) {
#pragma unroll
    for (int j = 0; j < WV; ++j) {
      const int q = j * 512 + tid;
      *reinterpret_cast<u32x4*>(smem + L.w_off + fc_off(q >> 3, q & 7)) = src[j];
    }
  };
  // Bounds of chunk c's extras and combine blocks (x = start and 16-byte pieces, y = start and
  // entries), read a chunk before the blocks themselves so that their loads never wait on them
  struct Meta { int xb, xn, cb, cn; };
  auto meta = [&](int c) {
    const int64_t blk = static_cast<int64_t>(t) * NC + c;
    Meta m;
    m.xb = ft.xoff[blk]; m.xn = (ft.xoff[blk + 1] - m.xb) >> 3;
    m.cb = ft.comb_off[blk]; m.cn = ft.comb_off[blk + 1] - m.cb;
    return m;
  };
  // extras of a chunk: uint16 S rows, a block of 8-entry pieces
  auto load_x = [&](const Meta& m, u32x4 (&dst)[XV], int& n16) {
    n16 = m.xn;
    const u32x4* src = reinterpret_cast<const u32x4*>(ft.xlist + m.xb);
#pragma unroll
    for (int j = 0; j < XV; ++j) {
      const int q = j * 512 + tid;
      if (q < n16) dst[j] = src[q];
    }
  };
  auto store_x = [&](const u32x4 (&src)[XV], int n16) {
#pragma unroll
    for (int j = 0; j < XV; ++j) {
      const int q = j * 512 + tid;
      if (q < n16) *reinterpret_cast<u32x4*>(smem + L.x_off + q * 16) = src[j];
    }
  };
  const RowT* S = reinterpret_cast<const RowT*>(smem + L.s_off);
  const uint16_t* X = reinterpret_cast<const uint16_t*>(smem + L.x_off);
  // A-tile address of (row, slot) dest of a chunk in buffer A
  auto a_addr = [&](uint8_t* A, int dest) {
    const int r = dest / SPC, sl = dest - r * SPC;
    const int byte = sl * CP * 2;
    return reinterpret_cast<RowT*>(A + fc_off(r, byte >> 4) + (byte & 15));
  };
  float* P = reinterpret_cast<float*>(smem + L.p_off);
  // A tile of chunk c into buffer `buf` from this thread's items; further neighbours in list
  // order (a plain loop: the compiler pipelines its index and row reads better than
  // hand-staged batches of reads, measured)
  auto build = [&](const uint2 (&it)[IT], int buf) {
    uint8_t* A = smem + L.a_off + buf * TM * FC_ROWB;
#pragma unroll
    for (int j = 0; j < IT; ++j) {
      const uint32_t w0 = it[j].x, w1 = it[j].y;
      const int count = static_cast<int>(w0 & 0xfu);
      if (count == 0) continue;            // no item in this slot: the A tile was cleared
      float a[CP];
#pragma unroll
      for (int c = 0; c < CP; ++c) a[c] = 0.0f;
      R::acc(a, S[w0 >> 16]);
      const uint16_t* xl = X + (w1 & 0xffffu);
      for (int q = 0; q < count - 1; ++q) R::acc(a, S[xl[q]]);
      const int dest = static_cast<int>(w1 >> 16);
      if (w0 & 0x8000u) {                  // one group of a long list: its fp32 partial sum
#pragma unroll
        for (int c = 0; c < CP; c += 4)
          *reinterpret_cast<f32x4*>(P + dest * CP + c) = f32x4{a[c], a[c + 1], a[c + 2], a[c + 3]};
      } else {
        *a_addr(A, dest) = R::pack(a);
      }
    }
  };
  // the long lists of a chunk: entry dest | m << 12 | p0 << 20 adds partials p0 .. p0 + m - 1
  // in order (from the first, which an fp32 sum from +0 never leaves at -0) and writes A
  auto combine = [&](uint32_t cw, int buf) {
    if (cw == 0u) return;
    uint8_t* A = smem + L.a_off + buf * TM * FC_ROWB;
    const int dest = static_cast<int>(cw & 0xfffu), m = static_cast<int>((cw >> 12) & 0xffu);
    const int p0 = static_cast<int>(cw >> 20);
    float a[CP];
#pragma unroll
    for (int c = 0; c < CP; c += 4) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(P + p0 * CP + c);
      a[c] = v[0]; a[c + 1] = v[1]; a[c + 2] = v[2]; a[c + 3] = v[3];
    }
    for (int i = 1; i < m; ++i) {
#pragma unroll
      for (int c = 0; c < CP; c += 4) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(P + (p0 + i) * CP + c);
        a[c] += v[0]; a[c + 1] += v[1]; a[c + 2] += v[2]; a[c + 3] += v[3];
      }
    }
    *a_addr(A, dest) = R::pack(a);
  };
  auto load_comb = [&](const Meta& m) -> uint32_t { return tid < m.cn ? ft.comb[m.cb + tid] : 0u; };
  // zero A buffer `buf` (TM rows of 128 bytes)
  auto clear = [&](int buf) {
    u32x4* A = reinterpret_cast<u32x4*>(smem + L.a_off + buf * TM * FC_ROWB);
#pragma unroll
    for (int j = 0; j < TM * FC_ROWB / 16 / 512; ++j) A[j * 512 + tid] = u32x4{0u, 0u, 0u, 0u};
  };

  uint2 it_a[IT], it_b[IT];
  u32x4 wreg[WV], xreg[XV];
  int xn = 0;
  const Meta m0 = meta(0);
  const Meta m1 = NC > 1 ? meta(1) : m0;
  const Meta m2 = NC > 2 ? meta(2) : m0;
  Meta mn = NC > 3 ? meta(3) : m0;          // the next chunk whose blocks are loaded (c + 3)
  load_items(0, it_a);
  if (NC > 1) load_items(1, it_b);
  uint32_t cw_a = load_comb(m0), cw_b = NC > 1 ? load_comb(m1) : 0u;
  load_w(0, wreg);
  load_x(m0, xreg, xn);
  store_w(wreg);
  store_x(xreg, xn);
  clear(0);
  clear(1);
  if (NC > 1) {
    load_w(1, wreg);
    load_x(m1, xreg, xn);
  }
  __syncthreads();
  build(it_a, 0);
  if (NC > 1) {
#pragma unroll
    for (int j = 0; j < IT; ++j) it_a[j] = it_b[j];
    if (NC > 2) load_items(2, it_b);
  }
  __syncthreads();
  combine(cw_a, 0);
  cw_a = cw_b;
  cw_b = NC > 2 ? load_comb(m2) : 0u;
  if (NC > 1) {
    store_x(xreg, xn);
    if (NC > 2) load_x(m2, xreg, xn);
  }
  __syncthreads();

  f32x16 acc[RB][CB];
#pragma unroll
  for (int i = 0; i < RB; ++i)
#pragma unroll
    for (int j = 0; j < CB; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  for (int c = 0; c < NC; ++c) {
    const uint8_t* A = smem + L.a_off + (c & 1) * TM * FC_ROWB;
#pragma unroll
    for (int ks = 0; ks < FC_KC / 16; ++ks) {
      const int q = ks * 2 + (lane >> 5);
      bf16x8 af[RB], bw[CB];
#pragma unroll
      for (int i = 0; i < RB; ++i)
        af[i] = *reinterpret_cast<const bf16x8*>(A + fc_off(wm * RB * 32 + i * 32 + (lane & 31), q));
#pragma unroll
      for (int j = 0; j < CB; ++j)
        bw[j] = *reinterpret_cast<const bf16x8*>(smem + L.w_off + fc_off(wn * CB * 32 + j * 32 + (lane & 31), q));
#pragma unroll
      for (int i = 0; i < RB; ++i)
#pragma unroll
        for (int j = 0; j < CB; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bw[j], acc[i][j], 0, 0, 0);
    }
    if (c + 1 < NC) build(it_a, (c + 1) & 1);
    __syncthreads();
    // every wave is past chunk c's fragment reads and chunk c + 1's items: finish c + 1's long
    // lists, clear c's buffer for chunk c + 2, stage the next weights and extras
    if (c + 1 < NC) combine(cw_a, (c + 1) & 1);
    if (c + 2 < NC) clear(c & 1);
    // everything this window stores was loaded a chunk ago; the next loads are issued after
    // those uses, so waiting for them never waits for a load issued here
    if (c + 1 < NC) store_w(wreg);
    if (c + 2 < NC) store_x(xreg, xn);
#pragma unroll
    for (int j = 0; j < IT; ++j) it_a[j] = it_b[j];
    cw_a = cw_b;
    cw_b = c + 3 < NC ? load_comb(mn) : 0u;
    if (c + 3 < NC) load_items(c + 3, it_b);
    if (c + 2 < NC) load_w(c + 2, wreg);
    if (c + 3 < NC) load_x(mn, xreg, xn);
    if (c + 4 < NC) mn = meta(c + 4);
    __syncthreads();
  }

  // Epilogue: y = acc + bias (ReLU optional)
  float bo[CB];
#pragma unroll
  for (int j = 0; j < CB; ++j) {
    const int64_t o = wn * CB * 32 + j * 32 + (lane & 31);
    bo[j] = (p.bias && o < p.Cout) ? p.bias[o] : 0.0f;
  }
  uint16_t* y = static_cast<uint16_t*>(p.y) + b * p.ys0;
  if (vec_out) {
    // each wave writes its RB*32 x CB*32 block into its own LDS region (the staged rows and A
    // tiles are free now: the loop ended on a barrier) and stores 16-byte pieces of rows
    constexpr int WC = CB * 32;
    uint16_t* Eo = reinterpret_cast<uint16_t*>(smem) + wave * (RB * 32 * WC);
#pragma unroll
    for (int i = 0; i < RB; ++i)
#pragma unroll
      for (int j = 0; j < CB; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
          Eo[row * WC + j * 32 + (lane & 31)] = f32_to_bf16_bits(epilogue(acc[i][j][r] + bo[j], p.relu));
        }
    __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0): this wave's LDS writes are done
    __builtin_amdgcn_wave_barrier();
    constexpr int PPR = WC / 8;           // 16-byte pieces per row
#pragma unroll
    for (int k = 0; k < RB * 32 * PPR / 64; ++k) {
      const int piece = k * 64 + lane;
      const int row = piece / PPR, part = piece - row * PPR;
      const int64_t n = n0 + wm * RB * 32 + row;
      const int64_t o = wn * WC + part * 8;
      if (n < p.Nout && o < p.Cout)
        *reinterpret_cast<u32x4*>(y + n * p.ys2 + o) = *reinterpret_cast<const u32x4*>(&Eo[row * WC + part * 8]);
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < CB; ++j) {
    const int64_t o = wn * CB * 32 + j * 32 + (lane & 31);
    if (o >= p.Cout) continue;
#pragma unroll
    for (int i = 0; i < RB; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t n = n0 + wm * RB * 32 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (n < p.Nout) Elem<uint16_t>::store(y + o * p.ys1 + n * p.ys2, epilogue(acc[i][j][r] + bo[j], p.relu));
      }
  }
}

// Tiling of a call: waves along rows, wave blocks, LDS bytes; false if none fits.
struct FewcPlan {
  int tm, wm, rb, cb, xv, lds;
};

static bool fewc_plan(const KnnParams& p, int cp, int tm, int zero_row, int xmax, int pmax, FewcPlan& pl) {
  if (tm != 128 && tm != 256) return false;
  // output columns padded to a multiple of 64 (zero weight columns, masked stores)
  const int ntp = static_cast<int>((p.Cout + 63) / 64 * 64);
  for (int wm : {2, 4}) {
    const int wn = 8 / wm;
    if (ntp % (32 * wn) != 0) continue;
    const int cb = ntp / (32 * wn), rb = tm / (32 * wm);
    if (cb < 1 || cb > 4 || rb * cb > 8) continue;
    // weight pieces and items must divide evenly over 512 threads
    if ((ntp * 8) % 512 != 0 || (tm * (FC_KC / cp)) % 512 != 0) continue;
    const int xv = (xmax / 8 + 511) / 512;
    if (xv > 4) return false;
    const int epi = 8 * rb * 32 * cb * 32 * 2;
    const FewcLayout l = fewc_layout(tm, 32 * wn * cb, cp, zero_row, xmax, pmax, epi);
    if (l.total > 160 * 1024) continue;
    pl = FewcPlan{tm, wm, rb, cb, xv < 1 ? 1 : xv, l.total};
    return true;
  }
  return false;
}

template <int TM, int WM, int RB, int CB, int CP, int XV>
static void launch_fewc_t(const KnnParams& p, const FewcTables& ft, const FewcPlan& pl, int vec_out, hipStream_t s) {
  const int64_t tiles_per_b = (p.Nout + TM - 1) / TM;
  const int64_t total = p.B * tiles_per_b;
  const int64_t padded = (total + 7) / 8 * 8;
  auto* k = &knnconv_fewc_kernel<TM, WM, RB, CB, CP, XV>;
  (void)reserve_dynamic_lds(reinterpret_cast<const void*>(k), pl.lds);
  hipLaunchKernelGGL(k, dim3(static_cast<unsigned>(padded)), dim3(512), pl.lds, s, p, ft, tiles_per_b, total, padded,
                     vec_out);
}

template <int TM, int WM, int RB, int CB, int CP>
static int launch_fewc_x(const KnnParams& p, const FewcTables& ft, const FewcPlan& pl, int vec_out, hipStream_t s) {
  switch (pl.xv) {
    case 1: launch_fewc_t<TM, WM, RB, CB, CP, 1>(p, ft, pl, vec_out, s); return 0;
    case 2: launch_fewc_t<TM, WM, RB, CB, CP, 2>(p, ft, pl, vec_out, s); return 0;
    case 3: launch_fewc_t<TM, WM, RB, CB, CP, 3>(p, ft, pl, vec_out, s); return 0;
    case 4: launch_fewc_t<TM, WM, RB, CB, CP, 4>(p, ft, pl, vec_out, s); return 0;
  }
  return 1;
}

template <int TM, int WM, int RB, int CP>
static int launch_fewc_cb(const KnnParams& p, const FewcTables& ft, const FewcPlan& pl, int vec_out, hipStream_t s) {
  switch (pl.cb) {
    case 1: return launch_fewc_x<TM, WM, RB, 1, CP>(p, ft, pl, vec_out, s);
    case 2: return launch_fewc_x<TM, WM, RB, 2, CP>(p, ft, pl, vec_out, s);
    case 3: if constexpr (RB * 3 <= 8) return launch_fewc_x<TM, WM, RB, 3, CP>(p, ft, pl, vec_out, s); break;
    case 4: if constexpr (RB * 4 <= 8) return launch_fewc_x<TM, WM, RB, 4, CP>(p, ft, pl, vec_out, s); break;
  }
  return 1;
}

template <int CP>
static int launch_fewc_cp(const KnnParams& p, const FewcTables& ft, const FewcPlan& pl, int vec_out, hipStream_t s) {
  if (pl.tm == 128 && pl.wm == 2) return launch_fewc_cb<128, 2, 2, CP>(p, ft, pl, vec_out, s);
  if (pl.tm == 128 && pl.wm == 4) return launch_fewc_cb<128, 4, 1, CP>(p, ft, pl, vec_out, s);
  if (pl.tm == 256 && pl.wm == 2) return launch_fewc_cb<256, 2, 4, CP>(p, ft, pl, vec_out, s);
  if (pl.tm == 256 && pl.wm == 4) return launch_fewc_cb<256, 4, 2, CP>(p, ft, pl, vec_out, s);
  return 1;
}

// 1 if launched, 0 if the fused kernel does not take this call (caller falls back).
int launch_knnconv_fewc(const KnnParams& p, const fovi_knnconv_args* a, int cp, hipStream_t s) {
  if (!a->fc_lo || !a->fc_span || !a->fc_item || !a->fc_xoff || !a->fc_comb || !a->fc_comb_off ||
      a->y_dtype != FOVI_BF16)
    return 0;
  if (a->fc_zero_row <= 0 || a->fc_zero_row > 0xffff || a->fc_xmax < 0 || a->fc_xmax % 8 != 0 ||
      a->fc_xmax > 0xffff || a->fc_pmax < 0 || a->fc_pmax > 0xfff || a->k_pad % FC_KC != 0 ||
      a->k_pad / cp > 4096)
    return 0;
  if (a->fc_xmax > 0 && !a->fc_xlist) return 0;
  FewcPlan pl;
  if (!fewc_plan(p, cp, a->fc_tile_points, a->fc_zero_row, a->fc_xmax, a->fc_pmax, pl)) return 0;
  FewcTables ft;
  ft.lo = a->fc_lo; ft.span = a->fc_span; ft.item = a->fc_item; ft.xlist = a->fc_xlist; ft.xoff = a->fc_xoff;
  ft.comb = a->fc_comb; ft.comb_off = a->fc_comb_off; ft.pmax = a->fc_pmax;
  ft.zero_row = a->fc_zero_row; ft.xmax = a->fc_xmax; ft.n_chunks = static_cast<int>(a->k_pad / FC_KC);
  const int vec_out = p.ys1 == 1 && p.ys2 % 8 == 0 && p.ys0 % 8 == 0 && p.Cout % 8 == 0 &&
                      reinterpret_cast<uintptr_t>(p.y) % 16 == 0;
  const int rc = cp == 4 ? launch_fewc_cp<4>(p, ft, pl, vec_out, s) : launch_fewc_cp<8>(p, ft, pl, vec_out, s);
  return rc == 0 ? 1 : 0;
}

}  // namespace fovi
