// kNN-convolution forward, bf16, for layers with few input channels (c_in <= 8;
// input rows padded to CP = 4 or 8 channels): the sensor's first layer (C2
// layer 1) and the DINOv3 patch embedding (C4), fused into one pass.
//
// GEMM view: rows = (b, n) output points, columns = output channels, reduction
// = (slot v, channel c), column v * CP + c, as the row-packed weight
// (fovi_knnconv_pack_weight with c_slot = CP). A workgroup of NT threads (256
// or 512: WM x WN waves) owns TM consecutive output points of one image and
// every output channel (NTP, c_out rounded up to the wave tiling). The host
// builds the tables for one geometry (TM, NT, KC) of FC_GEOMS; with 256 threads
// and a tile within 80 KB of LDS two workgroups share a CU.
//  * The tile's input rows form one contiguous index range; they are staged
//    in LDS once (S, CP channels per row, channels >= c_in zeroed), plus a
//    zero row, with 16-byte loads all in flight at once.
//  * The reduction runs in chunks of KC (32 or 64) columns (KC / CP slots).
//    A chunk's A tile [TM x KC] is cleared and its non-empty (point, slot)
//    sums are built in LDS from S out of (sum, neighbour) pairs: a host table
//    gives every thread NP (8 or 16) pairs per chunk, the runs of whole sums
//    packed into threads in (row, slot) order and the threads' segments dealt
//    over the waves. A thread issues its NP row reads at once (no read depends
//    on another), adds them in fp32 in list order from +0, and writes a sum,
//    rounded once to bf16, at the last pair of its run. A longer list (the
//    fovea's slots hold up to ~120 neighbours) is one run per group of 8, each
//    writing its fp32 partial sum, and a combine entry adds the partials in
//    order and rounds once. The slot sums equal the two-pass path's
//    (slotsum_kernel, same grouped order) bit for bit.
//  * The weight chunk [NTP x KC] is staged in LDS once per workgroup and read
//    by all waves; A and weight rows are 2 KC bytes, 16-byte parts
//    XOR-swizzled by low bits of the row (conflict-free fragment reads).
//  * Per chunk: the MFMAs of chunk c (32x32x16 bf16, ascending K, as the
//    two-pass GEMM) and the build of chunk c + 1's A tile into the other A
//    buffer, the two waves of a SIMD in opposite orders; after a barrier,
//    chunk c + 1's long lists are combined, chunk c's buffer is cleared for
//    chunk c + 2, and the weight of the next chunk (loaded into registers one
//    chunk ahead) is stored; two barriers per chunk.
//  * Epilogue: bias and ReLU, each wave transposes its tile through LDS and
//    stores 16-byte pieces of channels-last rows.
#include "knnconv_internal.h"

namespace fovi {

// 16-byte pieces of staged rows a thread loads at once: up to 512 threads x 16 x 16 bytes
constexpr int FC_STAGE_PIECES = 16;
constexpr uint32_t FC_LAST = 1u << 29;         // pair flag: the last pair of its run (write after it)
constexpr uint32_t FC_PARTIAL = 1u << 28;      // pair flag: the run is a group of a long list

struct FewcTables {
  const int32_t* lo;       // [n_tiles] first staged input row
  const int32_t* span;     // [n_tiles] staged rows
  const uint32_t* item;    // [n_tiles, n_chunks, NT threads, NP] pair words
  const uint32_t* comb;    // combine entries, per (tile, chunk) blocks
  const int32_t* comb_off; // [n_tiles * n_chunks + 1] block starts
  int zero_row;            // S row of zeros (>= every span)
  int pmax;                // most partial sums of a chunk
  int n_chunks;
};

struct FewcLayout {
  int s_off, a_off, w_off, p_off, total;
};

__host__ __device__ inline FewcLayout fewc_layout(int tm, int ntp, int cp, int kc, int zero_row, int pmax,
                                                  int epi_bytes) {
  FewcLayout l;
  int o = 0;
  l.s_off = o; o += ((zero_row + 1) * cp * 2 + 15) & ~15;
  l.a_off = o; o += 2 * tm * kc * 2;
  l.w_off = o; o += ntp * kc * 2;
  l.p_off = o; o += pmax * cp * 4;
  l.total = o > epi_bytes ? o : epi_bytes;
  return l;
}

// Byte offset of 16-byte part q of row r (rows of KC * 2 bytes): 128-byte rows XOR the part
// with bits 1-3 of the row, 64-byte rows with g(r) = (bit1(r) ^ bit3(r)) | bit2(r) << 1; either
// keeps 8 (and 16) consecutive rows' part q on distinct 16-byte bank groups.
template <int KC>
__device__ __forceinline__ uint32_t fc_off(int r, int q) {
  if constexpr (KC == 64) {
    return static_cast<uint32_t>(r * 128 + ((q ^ ((r >> 1) & 7)) << 4));
  } else {
    const int g = (((r >> 1) ^ (r >> 3)) & 1) | ((r >> 1) & 2);
    return static_cast<uint32_t>(r * 64 + ((q ^ g) << 4));
  }
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
  // a 16-byte piece holds two rows
  static __device__ __forceinline__ u32x4 mask_piece(u32x4 v, const uint32_t* m) {
    return u32x4{v[0] & m[0], v[1] & m[1], v[2] & m[0], v[3] & m[1]};
  }
  static __device__ __forceinline__ T piece_row(u32x4 v, int h) { return h ? T{v[2], v[3]} : T{v[0], v[1]}; }
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
  // a 16-byte piece is one row
  static __device__ __forceinline__ u32x4 mask_piece(u32x4 v, const uint32_t* m) { return mask(v, m); }
  static __device__ __forceinline__ T piece_row(u32x4 v, int) { return v; }
};

// TM output points per tile, NT threads in WM x WN waves, each wave RB x CB blocks of 32 x 32
// (rows x columns), CP channels per input row, KC reduction columns per chunk, NP (sum,
// neighbour) pairs per thread and chunk.
template <int TM, int NT, int WM, int RB, int CB, int CP, int KC, int NP>
__global__ __launch_bounds__(NT, 512 / NT) void knnconv_fewc_kernel(KnnParams p, FewcTables ft, int64_t tiles_per_b,
                                                                     int64_t total_tiles, int64_t padded_tiles,
                                                                     int vec_out, int stage16) {
  constexpr int NW = NT / 64;                       // waves
  constexpr int WN = NW / WM;
  constexpr int NTP = WN * CB * 32;
  constexpr int ROWB = KC * 2;                      // bytes of an A or weight row
  constexpr int PPR = ROWB / 16;                    // 16-byte parts of a row
  constexpr int SPC = KC / CP;                      // slots per chunk
  constexpr int WP = NTP * PPR;                     // 16-byte weight pieces per chunk
  constexpr int WV = (WP + NT - 1) / NT;            // weight pieces per thread per chunk
  constexpr int AP = TM * PPR / NT;                 // 16-byte A pieces per thread to clear a buffer
  constexpr int NQ = NP / 4;                        // 16-byte pair loads per thread and chunk
  static_assert(WM * WN == NW && RB * 32 * WM == TM, "wave grid");
  static_assert(TM * SPC <= 4096, "12-bit A entry targets");
  static_assert(AP >= 1 && TM * PPR % NT == 0, "A pieces per thread");
  static_assert(NP % 4 == 0 && (KC == 32 || KC == 64), "pairs in 16-byte loads; chunk width");
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
  const FewcLayout L = fewc_layout(TM, NTP, CP, KC, zr, ft.pmax, 0);
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
    if (stage16) {
      // 16-byte pieces of 16 / (2 CP) rows from the first row at a 16-byte boundary, all
      // loads in flight at once; a row before that boundary and a last row that does not fill
      // a piece are loaded on their own (no read past the tile's rows)
      constexpr int RPP = 8 / CP;                    // rows per piece
      const int lead = (RPP - (lo % RPP)) % RPP;
      const int n_pc = (span - lead) / RPP;
      const u32x4* pc = reinterpret_cast<const u32x4*>(src + lead);
      u32x4 v[FC_STAGE_PIECES];
#pragma unroll
      for (int u = 0; u < FC_STAGE_PIECES; ++u) {
        const int q = u * NT + tid;
        if (q < n_pc) v[u] = pc[q];
      }
      const int rest = span - lead - n_pc * RPP;      // rows after the last piece (< RPP)
      const bool has_e = tid < lead + rest;
      const int er = tid < lead ? tid : lead + n_pc * RPP + (tid - lead);
      RowT e;
      if (has_e) e = src[er];
#pragma unroll
      for (int u = 0; u < FC_STAGE_PIECES; ++u) {
        const int q = u * NT + tid;
        if (q < n_pc) {
          const u32x4 m = R::mask_piece(v[u], cm);
#pragma unroll
          for (int h = 0; h < RPP; ++h) S[lead + q * RPP + h] = R::piece_row(m, h);
        }
      }
      if (has_e) S[er] = R::mask(e, cm);
    } else {
      for (int r0 = 0; r0 < span; r0 += 8 * NT) {
        RowT v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int r = r0 + u * NT + tid;
          if (r < span) v[u] = src[r];
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int r = r0 + u * NT + tid;
          if (r < span) S[r] = R::mask(v[u], cm);
        }
      }
    }
    if (tid == 0) {
      RowT z;
#pragma unroll
      for (int w = 0; w < CP / 2; ++w) reinterpret_cast<uint32_t*>(&z)[w] = 0u;
      S[zr] = z;
    }
  }

  // this thread's NP pair words of chunk c
  const u32x4* pairs = reinterpret_cast<const u32x4*>(ft.item) + (static_cast<int64_t>(t) * NC * NT + tid) * NQ;
  auto load_items = [&](int c, u32x4 (&dst)[NQ]) {
    const u32x4* src = pairs + static_cast<int64_t>(c) * NT * NQ;
#pragma unroll
    for (int q = 0; q < NQ; ++q) dst[q] = src[q];
  };
  // weight chunk c: column o's 2 KC bytes at w + (o * k_pad + KC c) * 2; columns >= c_out are zero
  const uint16_t* wg = static_cast<const uint16_t*>(p.w);
  auto load_w = [&](int c, u32x4 (&dst)[WV]) {
#pragma unroll
    for (int j = 0; j < WV; ++j) {
      const int q = j * NT + tid, o = q / PPR, part = q % PPR;
      dst[j] = (q < WP && o < p.Cout)
                   ? *reinterpret_cast<const u32x4*>(wg + static_cast<int64_t>(o) * p.Kpad + c * KC + part * 8)
                   : u32x4{0u, 0u, 0u, 0u};
    }
  };
  auto store_w = [&](const u32x4 (&src)[WV]) {
#pragma unroll
    for (int j = 0; j < WV; ++j) {
      const int q = j * NT + tid;
      if (q < WP) *reinterpret_cast<u32x4*>(smem + L.w_off + fc_off<KC>(q / PPR, q % PPR)) = src[j];
    }
  };
  // Bounds of chunk c's combine block (start, entries), read a chunk before the block itself
  // so that its load never waits on them
  struct Meta { int cb, cn; };
  auto meta = [&](int c) {
    const int64_t blk = static_cast<int64_t>(t) * NC + c;
    Meta m;
    m.cb = ft.comb_off[blk]; m.cn = ft.comb_off[blk + 1] - m.cb;
    return m;
  };
  auto load_comb = [&](const Meta& m) -> uint32_t { return tid < m.cn ? ft.comb[m.cb + tid] : 0u; };
  const RowT* S = reinterpret_cast<const RowT*>(smem + L.s_off);
  float* P = reinterpret_cast<float*>(smem + L.p_off);
  auto a_buf = [&](int buf) { return smem + L.a_off + buf * TM * ROWB; };
  // A-tile address of (row, slot) dest of a chunk in A buffer A
  auto a_addr = [&](uint8_t* A, int dest) {
    const int r = dest / SPC, sl = dest - r * SPC;
    const int byte = sl * CP * 2;
    return reinterpret_cast<RowT*>(A + fc_off<KC>(r, byte >> 4) + (byte & 15));
  };
  // A tile of a chunk into buffer `buf` from this thread's pairs: all NP row reads first (none
  // depends on another; an unused pair reads the zero row), then the runs' fp32 sums in list
  // order from +0, each written at its last pair: rounded to bf16 into A, or a long list's
  // group as its fp32 partial sum
  auto build = [&](const u32x4 (&pw)[NQ], int buf) {
    uint8_t* A = a_buf(buf);
    uint32_t w[NP];
#pragma unroll
    for (int j = 0; j < NP; ++j) w[j] = pw[j >> 2][j & 3];
    RowT v[NP];
#pragma unroll
    for (int j = 0; j < NP; ++j) v[j] = S[w[j] & 0xffffu];
    float a[CP];
#pragma unroll
    for (int q = 0; q < CP; ++q) a[q] = 0.0f;
#pragma unroll
    for (int j = 0; j < NP; ++j) {
      R::acc(a, v[j]);
      if (w[j] & FC_LAST) {
        const uint32_t target = (w[j] >> 16) & 0xfffu;
        if (w[j] & FC_PARTIAL) {
#pragma unroll
          for (int q = 0; q < CP; q += 4)
            *reinterpret_cast<f32x4*>(P + target * CP + q) = f32x4{a[q], a[q + 1], a[q + 2], a[q + 3]};
        } else {
          *reinterpret_cast<RowT*>(A + target * sizeof(RowT)) = R::pack(a);
        }
#pragma unroll
        for (int q = 0; q < CP; ++q) a[q] = 0.0f;
      }
    }
  };
  // the long lists of a chunk: entry dest | m << 12 | p0 << 20 adds partials p0 .. p0 + m - 1
  // in order (from the first, which an fp32 sum from +0 never leaves at -0) and writes A
  auto combine = [&](uint32_t cw, int buf) {
    if (cw == 0u) return;
    const int dest = static_cast<int>(cw & 0xfffu), m = static_cast<int>((cw >> 12) & 0xffu);
    const int p0 = static_cast<int>(cw >> 20);
    float a[CP];
#pragma unroll
    for (int q = 0; q < CP; q += 4) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(P + p0 * CP + q);
      a[q] = v[0]; a[q + 1] = v[1]; a[q + 2] = v[2]; a[q + 3] = v[3];
    }
    for (int i = 1; i < m; ++i) {
#pragma unroll
      for (int q = 0; q < CP; q += 4) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(P + (p0 + i) * CP + q);
        a[q] += v[0]; a[q + 1] += v[1]; a[q + 2] += v[2]; a[q + 3] += v[3];
      }
    }
    *a_addr(a_buf(buf), dest) = R::pack(a);
  };
  // zero A buffer `buf`
  auto clear = [&](int buf) {
    u32x4* A = reinterpret_cast<u32x4*>(a_buf(buf));
#pragma unroll
    for (int j = 0; j < AP; ++j) A[j * NT + tid] = u32x4{0u, 0u, 0u, 0u};
  };

  u32x4 it_a[NQ], it_b[NQ];
  u32x4 wreg[WV];
  const Meta m0 = meta(0);
  const Meta m1 = NC > 1 ? meta(1) : m0;
  const Meta m2 = NC > 2 ? meta(2) : m0;
  Meta mn = NC > 3 ? meta(3) : m0;          // the next chunk whose combine block is loaded (c + 3)
  load_items(0, it_a);
  if (NC > 1) load_items(1, it_b);
  uint32_t cw_a = load_comb(m0), cw_b = NC > 1 ? load_comb(m1) : 0u;
  load_w(0, wreg);
  store_w(wreg);
  clear(0);
  clear(1);
  if (NC > 1) load_w(1, wreg);
  __syncthreads();
  build(it_a, 0);
  if (NC > 1) {
#pragma unroll
    for (int q = 0; q < NQ; ++q) it_a[q] = it_b[q];
    if (NC > 2) load_items(2, it_b);
  }
  __syncthreads();
  combine(cw_a, 0);
  cw_a = cw_b;
  cw_b = NC > 2 ? load_comb(m2) : 0u;
  __syncthreads();

  f32x16 acc[RB][CB];
#pragma unroll
  for (int i = 0; i < RB; ++i)
#pragma unroll
    for (int j = 0; j < CB; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
  // chunk c's MFMAs (ascending K)
  auto mfma_chunk = [&](int c) {
    const uint8_t* A = a_buf(c & 1);
#pragma unroll
    for (int ks = 0; ks < KC / 16; ++ks) {
      const int q = ks * 2 + (lane >> 5);
      bf16x8 af[RB], bw[CB];
#pragma unroll
      for (int i = 0; i < RB; ++i)
        af[i] = *reinterpret_cast<const bf16x8*>(A + fc_off<KC>(wm * RB * 32 + i * 32 + (lane & 31), q));
#pragma unroll
      for (int j = 0; j < CB; ++j)
        bw[j] = *reinterpret_cast<const bf16x8*>(smem + L.w_off + fc_off<KC>(wn * CB * 32 + j * 32 + (lane & 31), q));
#pragma unroll
      for (int i = 0; i < RB; ++i)
#pragma unroll
        for (int j = 0; j < CB; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bw[j], acc[i][j], 0, 0, 0);
    }
  };
  // The two waves of a SIMD take chunk c's MFMAs and chunk c + 1's build in opposite orders
  // (they touch different A buffers), so one wave's build issues while the other's MFMAs run.
  // With 8 waves, waves w and w + 4 share a SIMD (waves are dealt to the SIMDs in turn); with
  // 4 waves (two workgroups per CU) the other workgroup's waves are offset anyway.
  const bool build_first = NW == 8 && ((wave >> 2) & 1) != 0;
  for (int c = 0; c < NC; ++c) {
    // one copy of each job, in a two-step loop (two copies spill registers)
#pragma unroll 1
    for (int h = 0; h < 2; ++h) {
      if ((h ^ static_cast<int>(build_first)) == 0) mfma_chunk(c);
      else if (c + 1 < NC) build(it_a, (c + 1) & 1);
    }
    __syncthreads();
    // every wave is past chunk c's fragment reads and chunk c + 1's pairs: finish c + 1's long
    // lists, clear c's buffer for chunk c + 2, stage the next weights
    if (c + 1 < NC) combine(cw_a, (c + 1) & 1);
    if (c + 2 < NC) clear(c & 1);
    // everything this window stores was loaded a chunk ago; the next loads are issued after
    // those uses, so waiting for them never waits for a load issued here
    if (c + 1 < NC) store_w(wreg);
#pragma unroll
    for (int q = 0; q < NQ; ++q) it_a[q] = it_b[q];
    cw_a = cw_b;
    cw_b = c + 3 < NC ? load_comb(mn) : 0u;
    if (c + 3 < NC) load_items(c + 3, it_b);
    if (c + 2 < NC) load_w(c + 2, wreg);
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
    constexpr int PPW = WC / 8;           // 16-byte pieces per row of the wave's block
#pragma unroll
    for (int k = 0; k < RB * 32 * PPW / 64; ++k) {
      const int piece = k * 64 + lane;
      const int row = piece / PPW, part = piece - row * PPW;
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

// Geometries built (tile points, threads, chunk columns) and, as a bit mask, the waves along
// rows (1, 2, 4) each is instantiated for; the host mirror is knn_tables.FC_WAVE_ROWS.
struct FewcGeom { int tm, nt, kc, wms; };
constexpr FewcGeom FC_GEOMS[] = {{64, 256, 32, 1 | 2}, {128, 512, 64, 2 | 4}, {256, 512, 64, 2 | 4}};

// Tiling of a call: geometry, waves along rows, wave blocks, pairs per thread, LDS bytes;
// false if none fits.
struct FewcPlan {
  int tm, nt, kc, wm, rb, cb, np, lds;
};

static bool fewc_plan(const KnnParams& p, int cp, int tm, int nt, int kc, int zero_row, int pmax, int np,
                      FewcPlan& pl) {
  int wms = 0;
  for (const FewcGeom& g : FC_GEOMS)
    if (g.tm == tm && g.nt == nt && g.kc == kc) wms = g.wms;
  if (wms == 0 || (np != 8 && np != 16)) return false;
  // output columns padded to a multiple of 64 (zero weight columns, masked stores)
  const int ntp = static_cast<int>((p.Cout + 63) / 64 * 64);
  const int nw = nt / 64;
  for (int wm : {1, 2, 4}) {
    if ((wms & wm) == 0 || nw % wm != 0 || tm % (32 * wm) != 0) continue;
    const int wn = nw / wm;
    if (ntp % (32 * wn) != 0) continue;
    const int cb = ntp / (32 * wn), rb = tm / (32 * wm);
    if (cb < 1 || cb > 4 || rb < 1 || rb * cb > 8) continue;
    if (tm * (kc / cp) > 4096) continue;              // A entry targets fit 12 bits
    const int epi = nw * rb * 32 * cb * 32 * 2;
    const FewcLayout l = fewc_layout(tm, 32 * wn * cb, cp, kc, zero_row, pmax, epi);
    // two 256-thread workgroups share a CU within half of its LDS
    if (l.total > (nt == 256 ? 80 : 160) * 1024) continue;
    pl = FewcPlan{tm, nt, kc, wm, rb, cb, np, l.total};
    return true;
  }
  return false;
}

template <int TM, int NT, int WM, int RB, int CB, int CP, int KC, int NP>
static int launch_fewc_t(const KnnParams& p, const FewcTables& ft, const FewcPlan& pl, int vec_out, hipStream_t s) {
  const int64_t tiles_per_b = (p.Nout + TM - 1) / TM;
  const int64_t total = p.B * tiles_per_b;
  const int64_t padded = (total + 7) / 8 * 8;
  auto* k = &knnconv_fewc_kernel<TM, NT, WM, RB, CB, CP, KC, NP>;
  (void)reserve_dynamic_lds(reinterpret_cast<const void*>(k), pl.lds);
  // staged rows in 16-byte pieces: 16-byte aligned image rows, every span within the pieces
  const int stage16 = (reinterpret_cast<uintptr_t>(p.x) % 16 == 0 && p.xs0 % 8 == 0 &&
                       ft.zero_row <= FC_STAGE_PIECES * NT * (8 / CP)) ? 1 : 0;
  hipLaunchKernelGGL(k, dim3(static_cast<unsigned>(padded)), dim3(NT), pl.lds, s, p, ft, tiles_per_b, total, padded,
                     vec_out, stage16);
  return 0;
}

template <int TM, int NT, int WM, int RB, int CB, int CP, int KC>
static int launch_fewc_np(const KnnParams& p, const FewcTables& ft, const FewcPlan& pl, int vec_out, hipStream_t s) {
  if (pl.np == 8) return launch_fewc_t<TM, NT, WM, RB, CB, CP, KC, 8>(p, ft, pl, vec_out, s);
  if (pl.np == 16) return launch_fewc_t<TM, NT, WM, RB, CB, CP, KC, 16>(p, ft, pl, vec_out, s);
  return 1;
}

template <int TM, int NT, int WM, int CP, int KC>
static int launch_fewc_cb(const KnnParams& p, const FewcTables& ft, const FewcPlan& pl, int vec_out, hipStream_t s) {
  constexpr int RB = TM / (32 * WM);
  switch (pl.cb) {
    case 1: return launch_fewc_np<TM, NT, WM, RB, 1, CP, KC>(p, ft, pl, vec_out, s);
    case 2: if constexpr (RB * 2 <= 8) return launch_fewc_np<TM, NT, WM, RB, 2, CP, KC>(p, ft, pl, vec_out, s); break;
    case 3: if constexpr (RB * 3 <= 8) return launch_fewc_np<TM, NT, WM, RB, 3, CP, KC>(p, ft, pl, vec_out, s); break;
    case 4: if constexpr (RB * 4 <= 8) return launch_fewc_np<TM, NT, WM, RB, 4, CP, KC>(p, ft, pl, vec_out, s); break;
  }
  return 1;
}

template <int CP>
static int launch_fewc_cp(const KnnParams& p, const FewcTables& ft, const FewcPlan& pl, int vec_out, hipStream_t s) {
  if (pl.tm == 64 && pl.nt == 256 && pl.wm == 1) return launch_fewc_cb<64, 256, 1, CP, 32>(p, ft, pl, vec_out, s);
  if (pl.tm == 64 && pl.nt == 256 && pl.wm == 2) return launch_fewc_cb<64, 256, 2, CP, 32>(p, ft, pl, vec_out, s);
  if (pl.tm == 128 && pl.nt == 512 && pl.wm == 2) return launch_fewc_cb<128, 512, 2, CP, 64>(p, ft, pl, vec_out, s);
  if (pl.tm == 128 && pl.nt == 512 && pl.wm == 4) return launch_fewc_cb<128, 512, 4, CP, 64>(p, ft, pl, vec_out, s);
  if (pl.tm == 256 && pl.nt == 512 && pl.wm == 2) return launch_fewc_cb<256, 512, 2, CP, 64>(p, ft, pl, vec_out, s);
  if (pl.tm == 256 && pl.nt == 512 && pl.wm == 4) return launch_fewc_cb<256, 512, 4, CP, 64>(p, ft, pl, vec_out, s);
  return 1;
}

// 1 if launched, 0 if the fused kernel does not take this call (caller falls back).
int launch_knnconv_fewc(const KnnParams& p, const fovi_knnconv_args* a, int cp, hipStream_t s) {
  if (!a->fc_lo || !a->fc_span || !a->fc_item || !a->fc_comb || !a->fc_comb_off || a->y_dtype != FOVI_BF16 ||
      p.xs2 != cp)   // a tile stages a contiguous range of one image's rows
    return 0;
  const int kc = a->fc_chunk;
  if (a->fc_zero_row <= 0 || a->fc_zero_row > 0xffff || a->fc_pmax < 0 || a->fc_pmax > 0xfff ||
      (kc != 32 && kc != 64) || a->k_pad % kc != 0 || a->k_pad / cp > 4096 ||
      (reinterpret_cast<uintptr_t>(a->fc_item) & 15) != 0)
    return 0;
  FewcPlan pl;
  if (!fewc_plan(p, cp, a->fc_tile_points, a->fc_threads, kc, a->fc_zero_row, a->fc_pmax, a->fc_pairs, pl)) return 0;
  FewcTables ft;
  ft.lo = a->fc_lo; ft.span = a->fc_span; ft.item = a->fc_item;
  ft.comb = a->fc_comb; ft.comb_off = a->fc_comb_off; ft.pmax = a->fc_pmax;
  ft.zero_row = a->fc_zero_row; ft.n_chunks = static_cast<int>(a->k_pad / kc);
  const int vec_out = p.ys1 == 1 && p.ys2 % 8 == 0 && p.ys0 % 8 == 0 && p.Cout % 8 == 0 &&
                      reinterpret_cast<uintptr_t>(p.y) % 16 == 0;
  const int rc = cp == 4 ? launch_fewc_cp<4>(p, ft, pl, vec_out, s) : launch_fewc_cp<8>(p, ft, pl, vec_out, s);
  return rc == 0 ? 1 : 0;
}

}  // namespace fovi
