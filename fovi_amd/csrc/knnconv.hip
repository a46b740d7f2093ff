// kNN-convolution forward: fused neighbour gather -> slot sum -> GEMM.
//
// GEMM view: rows m = (b, n) output points, columns o output channels,
// reduction index kk = v * c_in + c (ref slot major). Row m's reduction
// vector is assembled on the fly from the slot-major CSR neighbour lists:
//   A[m, v*c_in + c] = sum_{i < count(n,v)} x[b, c, nbr_sorted[n, begin(n,v) + i]]
// so the [B, C, k, N] gather tensor, the one-hot einsum and its permute copies
// of the reference (fovi/arch/knn.py:484-526) are never materialised.
//
// Kernels (fovi_knnconv_fwd picks one per call; fovi_knnconv_last_path names it)
//  * knnconv_f32_kernel: fp32 operands, any strides, fp32 FMA SGEMM tiling.
//    The fp32 parity path.
//  * the wide-layer kernels (knnconv_v5.hip): fragment-order weights.
//  * knnconv_bf16_v4_kernel: channels-last rows, c_in % 32 == 0, with the
//    tile tables: input rows staged in LDS, single-neighbour slots read in
//    place; see below.
//  * knnconv_bf16_v2_kernel: channels-last rows, c_in % 32 == 0, without the
//    tile tables (k > 255, or spans past LDS): CSR lists staged in LDS.
//  * few-channel kernels (c_in <= 8, rows padded to 4 or 8 channels).
//  * knnconv_bf16_kernel: any strides and channel counts: bf16 operands, fp32 accumulate on
//    v_mfma_f32_32x32x16_bf16. 128-point x NT-channel tiles, 4 waves (2x2),
//    64-wide reduction chunks double buffered in LDS (XOR-swizzled 16-byte
//    chunks so the MFMA fragment reads are bank-conflict free), next chunk's
//    gather issued into registers before the current chunk's MFMAs.
//    VEC loader: channels-last rows and c_in % 64 == 0, one 16-byte load per
//    (row, 8 channels). Generic loader: any strides / c_in, element gathers.
#include "knnconv_internal.h"

#include <algorithm>
#include <mutex>

namespace fovi {

// ---------------------------------------------------------------------------
// fp32 path
// ---------------------------------------------------------------------------
constexpr int F32_TM = 64, F32_TN = 64, F32_TK = 16;

template <typename OutT>
__global__ __launch_bounds__(256) void knnconv_f32_kernel(KnnParams p, int64_t tiles_per_b) {
  __shared__ float As[F32_TK][F32_TM + 4];
  __shared__ float Ws[F32_TK][F32_TN + 4];
  const int tid = threadIdx.x;
  const int64_t mt = blockIdx.x;
  const int64_t b = mt / tiles_per_b;
  const int64_t n0 = (mt % tiles_per_b) * F32_TM;
  const int64_t o0 = static_cast<int64_t>(blockIdx.y) * F32_TN;
  const float* x = static_cast<const float*>(p.x) + b * p.xs0;
  const float* w = static_cast<const float*>(p.w);
  const int tm = tid & 15, tn = tid >> 4;
  float acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0.0f;
  const int64_t ktot = p.V * p.C;

  for (int64_t k0 = 0; k0 < ktot; k0 += F32_TK) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = tid + 256 * i;
      const int pl = e & 63, kk = e >> 6;
      const int64_t k = k0 + kk, n = n0 + pl;
      float a = 0.0f;
      if (k < ktot && n < p.Nout) {
        const int64_t v = k / p.C, c = k - v * p.C;
        const int32_t ent = p.slot_ptr[n * p.V + v];
        const int32_t* nb = p.nbr + n * p.K + (ent >> 16);
        const int cnt = ent & 0xffff;
        for (int j = 0; j < cnt; ++j) a += x[c * p.xs1 + static_cast<int64_t>(nb[j]) * p.xs2];
      }
      As[kk][pl] = a;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = tid + 256 * i;
      const int kk = e & 15, ol = e >> 4;
      const int64_t o = o0 + ol;
      Ws[kk][ol] = (o < p.Cout) ? w[o * p.Kpad + k0 + kk] : 0.0f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < F32_TK; ++kk) {
      float av[4], wv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) av[i] = As[kk][tm * 4 + i];
#pragma unroll
      for (int j = 0; j < 4; ++j) wv[j] = Ws[kk][tn * 4 + j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_fmaf(av[i], wv[j], acc[i][j]);
    }
    __syncthreads();
  }

  OutT* y = static_cast<OutT*>(p.y) + b * p.ys0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t n = n0 + tm * 4 + i;
    if (n >= p.Nout) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t o = o0 + tn * 4 + j;
      if (o >= p.Cout) continue;
      float r = acc[i][j];
      if (p.bias) r += p.bias[o];
      Elem<OutT>::store(y + o * p.ys1 + n * p.ys2, epilogue(r, p.relu));
    }
  }
}

// ---------------------------------------------------------------------------
// bf16 MFMA path
// ---------------------------------------------------------------------------
constexpr int MM_MT = 128;  // output points per tile
constexpr int MM_KC = 64;   // reduction chunk (bf16 elements)

struct Raw16 { uint32_t a, b, c, d; };

__device__ __forceinline__ void add_bf16x8(float (&s)[8], const Raw16& r) {
  const uint32_t u[4] = {r.a, r.b, r.c, r.d};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    s[2 * i] += __uint_as_float(u[i] << 16);
    s[2 * i + 1] += __uint_as_float(u[i] & 0xffff0000u);
  }
}

__device__ __forceinline__ Raw16 pack_bf16x8(const float (&s)[8]) {
  uint32_t u[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    u[i] = static_cast<uint32_t>(f32_to_bf16_bits(s[2 * i])) |
           (static_cast<uint32_t>(f32_to_bf16_bits(s[2 * i + 1])) << 16);
  return Raw16{u[0], u[1], u[2], u[3]};
}

// LDS offset (in bf16 elements) of 16-byte chunk `q` of row `r` in a
// [rows][64] tile: chunk index XOR (row mod 8).
__device__ __forceinline__ int swz(int r, int q) { return r * MM_KC + ((q ^ (r & 7)) << 3); }

// Gathered 8-channel vector of row n (slot v, channels c .. c+7), VEC layout.
__device__ __forceinline__ Raw16 gather_vec(const KnnParams& p, const uint16_t* xb, int64_t n, int64_t v,
                                            int64_t c) {
  Raw16 r{0u, 0u, 0u, 0u};
  if (n >= p.Nout) return r;
  const int32_t ent = p.slot_ptr[n * p.V + v];
  const int cnt = ent & 0xffff;
  if (cnt == 0) return r;
  const int32_t* nb = p.nbr + n * p.K + (ent >> 16);
  if (cnt == 1) return *reinterpret_cast<const Raw16*>(xb + static_cast<int64_t>(nb[0]) * p.xs2 + c);
  float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int j = 0; j < cnt; ++j)
    add_bf16x8(s, *reinterpret_cast<const Raw16*>(xb + static_cast<int64_t>(nb[j]) * p.xs2 + c));
  return pack_bf16x8(s);
}

// Generic layout: 8 consecutive reduction indices kk .. kk+7, element gathers.
__device__ __forceinline__ Raw16 gather_generic(const KnnParams& p, const uint16_t* xb, int64_t n,
                                                int64_t kk) {
  float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  const int64_t ktot = p.V * p.C;
  if (n < p.Nout && kk < ktot) {
    int64_t v = kk / p.C, c = kk - v * p.C;
    int32_t ent = p.slot_ptr[n * p.V + v];
    for (int e = 0; e < 8 && kk + e < ktot; ++e) {
      const int cnt = ent & 0xffff;
      const int32_t* nb = p.nbr + n * p.K + (ent >> 16);
      for (int j = 0; j < cnt; ++j)
        s[e] += bf16_bits_to_f32(xb[c * p.xs1 + static_cast<int64_t>(nb[j]) * p.xs2]);
      if (++c == p.C && kk + e + 1 < ktot) {
        c = 0;
        ++v;
        ent = p.slot_ptr[n * p.V + v];
      }
    }
  }
  return pack_bf16x8(s);
}

template <int NT, bool VEC, typename OutT>
__global__ __launch_bounds__(256, 2) void knnconv_bf16_kernel(KnnParams p, int64_t tiles_per_b,
                                                              int64_t n_tiles_n, int64_t total_tiles,
                                                              int64_t padded_tiles) {
  constexpr int A_VECS = MM_MT * MM_KC / 8 / 256;  // 16-byte vectors per thread
  constexpr int B_VECS = NT * MM_KC / 8 / 256;
  constexpr int WN = NT / 2;                       // wave tile columns
  constexpr int CB = WN / 32;                      // 32-wide column blocks per wave
  __shared__ __attribute__((aligned(16))) uint16_t As[2][MM_MT * MM_KC];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[2][NT * MM_KC];

  const int64_t tile = xcd_tile(blockIdx.x, padded_tiles);
  if (tile >= total_tiles) return;
  const int64_t mt = tile / n_tiles_n;
  const int64_t o0 = (tile % n_tiles_n) * NT;
  const int64_t b = mt / tiles_per_b;
  const int64_t n0 = (mt % tiles_per_b) * MM_MT;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  const uint16_t* xb = static_cast<const uint16_t*>(p.x) + b * p.xs0;
  const uint16_t* wp = static_cast<const uint16_t*>(p.w);
  const int64_t nk = p.Kpad / MM_KC;

  Raw16 ra[A_VECS], rb[B_VECS];
  auto load_chunk = [&](int64_t kt) {
    const int64_t k0 = kt * MM_KC;
#pragma unroll
    for (int i = 0; i < A_VECS; ++i) {
      const int q = tid + 256 * i;
      const int row = q >> 3, part = q & 7;
      if (VEC) {
        const int64_t v = k0 / p.C;
        const int64_t c = k0 - v * p.C + part * 8;
        ra[i] = gather_vec(p, xb, n0 + row, v, c);
      } else {
        ra[i] = gather_generic(p, xb, n0 + row, k0 + part * 8);
      }
    }
#pragma unroll
    for (int i = 0; i < B_VECS; ++i) {
      const int q = tid + 256 * i;
      const int row = q >> 3, part = q & 7;
      const int64_t o = o0 + row;
      rb[i] = (o < p.Cout) ? *reinterpret_cast<const Raw16*>(wp + o * p.Kpad + k0 + part * 8)
                           : Raw16{0u, 0u, 0u, 0u};
    }
  };
  auto store_chunk = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_VECS; ++i) {
      const int q = tid + 256 * i;
      *reinterpret_cast<Raw16*>(&As[buf][swz(q >> 3, q & 7)]) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < B_VECS; ++i) {
      const int q = tid + 256 * i;
      *reinterpret_cast<Raw16*>(&Bs[buf][swz(q >> 3, q & 7)]) = rb[i];
    }
  };

  f32x16 acc[2][CB];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < CB; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  load_chunk(0);
  store_chunk(0);
  __syncthreads();
  for (int64_t kt = 0; kt < nk; ++kt) {
    const int buf = static_cast<int>(kt & 1);
    if (kt + 1 < nk) load_chunk(kt + 1);
#pragma unroll
    for (int ks = 0; ks < MM_KC / 16; ++ks) {
      const int q = ks * 2 + (lane >> 5);
      bf16x8 af[2], bfr[CB];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int row = wm * 64 + i * 32 + (lane & 31);
        af[i] = *reinterpret_cast<const bf16x8*>(&As[buf][swz(row, q)]);
      }
#pragma unroll
      for (int j = 0; j < CB; ++j) {
        const int col = wn * WN + j * 32 + (lane & 31);
        bfr[j] = *reinterpret_cast<const bf16x8*>(&Bs[buf][swz(col, q)]);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < CB; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) store_chunk(buf ^ 1);
    __syncthreads();
  }

  OutT* y = static_cast<OutT*>(p.y) + b * p.ys0;
#pragma unroll
  for (int j = 0; j < CB; ++j) {
    const int64_t o = o0 + wn * WN + j * 32 + (lane & 31);
    if (o >= p.Cout) continue;
    const float bo = p.bias ? p.bias[o] : 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t n = n0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (n < p.Nout) Elem<OutT>::store(y + o * p.ys1 + n * p.ys2, epilogue(acc[i][j][r] + bo, p.relu));
      }
  }
}

// ---------------------------------------------------------------------------
// bf16 MFMA path, large tiles (channels-last input, c_in % 32 == 0)
// ---------------------------------------------------------------------------
// 256 output points x NT output channels per workgroup of 8 waves (4 along
// the points, 2 along the channels; wave tile 64 x NT/2 = 2 x NT/64 blocks of
// v_mfma_f32_32x32x16_bf16). The tile's CSR lists (slot entries and
// neighbour indices, 256 x (V + k) int32) are copied into LDS once, so the
// reduction loop issues only data loads to memory. The reduction runs over
// 32-channel chunks of one slot: the chunk's gathered A tile (256 x 32) and
// weight tile (NT x 32) are double buffered in LDS, with the next chunk's
// global loads in flight in registers while the current chunk's MFMAs run.
// LDS rows are 64 bytes (four 16-byte chunks), XOR-swizzled per row (swz32)
// so that fragment reads and tile writes are bank-conflict free.
constexpr int V2_MT = 256;

size_t v2_lds_bytes(int nt, int64_t V, int64_t K) {
  return static_cast<size_t>(2 * V2_MT * V2_CC * 2 + 2 * nt * V2_CC * 2) +
         static_cast<size_t>(V2_MT) * static_cast<size_t>(V + K) * 4;
}

template <int NT, typename OutT>
__global__ __launch_bounds__(512, 1) void knnconv_bf16_v2_kernel(KnnParams p, int64_t tiles_per_b,
                                                                 int64_t n_tiles_n, int64_t total_tiles,
                                                                 int64_t padded_tiles) {
  constexpr int WN = NT / 2;
  constexpr int CB = WN / 32;
  constexpr int B_VECS = (NT * V2_CC / 8 + 511) / 512;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint16_t* As = reinterpret_cast<uint16_t*>(smem);                 // [2][256*32]
  uint16_t* Bs = As + 2 * V2_MT * V2_CC;                            // [2][NT*32]
  int32_t* ent = reinterpret_cast<int32_t*>(Bs + 2 * NT * V2_CC);   // [256][V]
  int32_t* nbl = ent + V2_MT * p.V;                                 // [256][K]

  const int64_t tile = xcd_tile(blockIdx.x, padded_tiles);
  if (tile >= total_tiles) return;
  const int64_t mt = tile / n_tiles_n;
  const int64_t o0 = (tile % n_tiles_n) * NT;
  const int64_t b = mt / tiles_per_b;
  const int64_t n0 = (mt % tiles_per_b) * V2_MT;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 3, wn = wave >> 2;
  const int V = static_cast<int>(p.V), K = static_cast<int>(p.K);

  // stage the tile's CSR lists
  for (int i = tid; i < V2_MT * V; i += 512) {
    const int64_t n = n0 + i / V;
    ent[i] = n < p.Nout ? p.slot_ptr[n0 * p.V + i] : 0;
  }
  for (int i = tid; i < V2_MT * K; i += 512) {
    const int64_t n = n0 + i / K;
    nbl[i] = n < p.Nout ? p.nbr[n0 * p.K + i] : -1;
  }
  __syncthreads();

  const uint16_t* xb = static_cast<const uint16_t*>(p.x) + b * p.xs0;
  const uint16_t* wp = static_cast<const uint16_t*>(p.w);
  const int nc = static_cast<int>(p.C / V2_CC);     // chunks per slot
  const int nk = V * nc;
  const int part = tid & 3;
  const int row0 = tid >> 2;                         // rows row0 and row0 + 128

  Raw16 ra[2], rb[B_VECS];
  auto load_chunk = [&](int kt) {
    const int v = kt / nc;
    const int c = (kt - v * nc) * V2_CC + part * 8;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int row = row0 + 128 * i;
      const int32_t e = ent[row * V + v];
      const int cnt = e & 0xffff;
      const int32_t* nb = nbl + row * K + (e >> 16);
      Raw16 r{0u, 0u, 0u, 0u};
      if (cnt == 1) {
        r = *reinterpret_cast<const Raw16*>(xb + static_cast<int64_t>(nb[0]) * p.xs2 + c);
      } else if (cnt > 1) {
        float s8[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        for (int j = 0; j < cnt; ++j)
          add_bf16x8(s8, *reinterpret_cast<const Raw16*>(xb + static_cast<int64_t>(nb[j]) * p.xs2 + c));
        r = pack_bf16x8(s8);
      }
      ra[i] = r;
    }
    const int64_t k0 = static_cast<int64_t>(v) * p.C + (kt - v * nc) * V2_CC;
#pragma unroll
    for (int i = 0; i < B_VECS; ++i) {
      const int q = tid + 512 * i;
      const int row = q >> 2;
      const int64_t o = o0 + row;
      rb[i] = (q < NT * 4 && o < p.Cout)
                  ? *reinterpret_cast<const Raw16*>(wp + o * p.Kpad + k0 + (q & 3) * 8)
                  : Raw16{0u, 0u, 0u, 0u};
    }
  };
  auto store_chunk = [&](int buf) {
    uint16_t* a = As + buf * V2_MT * V2_CC;
    uint16_t* bsm = Bs + buf * NT * V2_CC;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int row = row0 + 128 * i;
      *reinterpret_cast<Raw16*>(&a[swz32(row, part)]) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < B_VECS; ++i) {
      const int q = tid + 512 * i;
      if (q < NT * 4) *reinterpret_cast<Raw16*>(&bsm[swz32(q >> 2, q & 3)]) = rb[i];
    }
  };

  f32x16 acc[2][CB];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < CB; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  load_chunk(0);
  store_chunk(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) load_chunk(kt + 1);
    const uint16_t* a = As + buf * V2_MT * V2_CC;
    const uint16_t* bsm = Bs + buf * NT * V2_CC;
#pragma unroll
    for (int ks = 0; ks < V2_CC / 16; ++ks) {
      const int q = ks * 2 + (lane >> 5);
      bf16x8 af[2], bfr[CB];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        af[i] = *reinterpret_cast<const bf16x8*>(&a[swz32(wm * 64 + i * 32 + (lane & 31), q)]);
#pragma unroll
      for (int j = 0; j < CB; ++j)
        bfr[j] = *reinterpret_cast<const bf16x8*>(&bsm[swz32(wn * WN + j * 32 + (lane & 31), q)]);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < CB; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) store_chunk(buf ^ 1);
    __syncthreads();
  }

  OutT* y = static_cast<OutT*>(p.y) + b * p.ys0;
#pragma unroll
  for (int j = 0; j < CB; ++j) {
    const int64_t o = o0 + wn * WN + j * 32 + (lane & 31);
    if (o >= p.Cout) continue;
    const float bo = p.bias ? p.bias[o] : 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t n = n0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (n < p.Nout) Elem<OutT>::store(y + o * p.ys1 + n * p.ys2, epilogue(acc[i][j][r] + bo, p.relu));
      }
  }
}

template <int NT>
static int launch_bf16_v2(const KnnParams& p, int out_t, hipStream_t s) {
  const int64_t tiles_per_b = (p.Nout + V2_MT - 1) / V2_MT;
  const int64_t n_tiles_n = (p.Cout + NT - 1) / NT;
  const int64_t total = p.B * tiles_per_b * n_tiles_n;
  const int64_t padded = (total + 7) / 8 * 8;
  const size_t lds = v2_lds_bytes(NT, p.V, p.K);
  dim3 grid(static_cast<unsigned>(padded));
  if (out_t == FOVI_BF16) {
    (void)reserve_dynamic_lds(reinterpret_cast<const void*>(&knnconv_bf16_v2_kernel<NT, uint16_t>), lds);
    hipLaunchKernelGGL((knnconv_bf16_v2_kernel<NT, uint16_t>), grid, dim3(512), lds, s, p, tiles_per_b,
                       n_tiles_n, total, padded);
  } else {
    (void)reserve_dynamic_lds(reinterpret_cast<const void*>(&knnconv_bf16_v2_kernel<NT, float>), lds);
    hipLaunchKernelGGL((knnconv_bf16_v2_kernel<NT, float>), grid, dim3(512), lds, s, p, tiles_per_b,
                       n_tiles_n, total, padded);
  }
  return 0;
}

// Picks the widest channel tile whose LDS footprint fits; 0 if none does.
static int v2_tile_n(const KnnParams& p) {
  const int cands[4] = {256, 192, 128, 64};
  for (int nt : cands) {
    if (nt > 64 && p.Cout <= nt / 2) continue;   // avoid tiles more than half empty
    if (v2_lds_bytes(nt, p.V, p.K) <= 160 * 1024) return nt;
  }
  return 0;
}

// ---------------------------------------------------------------------------
// Shared by the staged-row kernels below: 256-point tiles, 32-channel chunks.
// ---------------------------------------------------------------------------
constexpr int V3_MT = 256;
constexpr int V3_CC = 32;

// ---------------------------------------------------------------------------
// bf16 MFMA path reading single-neighbour slots straight from the staged rows
// ---------------------------------------------------------------------------
// Same tile, staging (S, now XOR-swizzled like the tiles) and MFMA core as
// above, but the A tile is no longer assembled for every slot: an MFMA lane
// takes its 16-byte fragment from the S row of its point's only neighbour in
// the slot, or from a zero row (index zero_row) when the slot is empty. Only
// the points of a slot with two or more neighbours (about a quarter on the
// log-polar lattice) are summed, into a small tile, driven by a per-(tile,
// slot) row list sorted by count so that lanes of a wave loop about equally.
// S may only be refreshed after the last MFMA of a channel chunk has read it,
// so the refresh (and the first slot's sums) run between two extra barriers
// once per chunk.
__device__ __forceinline__ int swz_g(int r) { return (((r >> 1) ^ (r >> 3)) & 1) | ((r >> 1) & 2); }

struct V4Layout {
  int b_off, ent_off, colln_off, coll_off, nbl_off, s_off, total;  // bytes
};

__host__ __device__ inline V4Layout v4_layout(int nt, int V, int K, int zero_row) {
  V4Layout l;
  int o = 2 * 256 * 32 * 2;                       // A: two 256 x 32 bf16 tiles
  l.b_off = o;      o += 2 * nt * 32 * 2;         // B: two NT x 32 tiles
  l.ent_off = o;    o += 256 * V * 4;             // CSR words, slot-major
  l.colln_off = o;  o += (V * 4 + 15) & ~15;      // collision row counts
  l.coll_off = o;   o += V * 256;                 // collision row lists
  l.nbl_off = o;    o += (256 * K * 2 + 15) & ~15;
  l.s_off = o;      o += (zero_row + 1) * 32 * 2; // staged rows + zero row
  l.total = o;
  return l;
}

template <int NT, int SV, typename OutT>
__global__ __launch_bounds__(512, 1) void knnconv_bf16_v4_kernel(KnnParams p, int64_t tiles_per_b,
                                                                 int64_t n_tiles_n, int64_t total_tiles,
                                                                 int64_t padded_tiles) {
  constexpr int WN = NT / 2;
  constexpr int CB = WN / 32;
  constexpr int B_VECS = (NT * V3_CC / 8 + 511) / 512;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int V = static_cast<int>(p.V), K = static_cast<int>(p.K);
  const int zr = p.zero_row;
  const V4Layout L = v4_layout(NT, V, K, zr);
  uint16_t* sm16 = reinterpret_cast<uint16_t*>(smem);
  uint16_t* Bs = sm16 + L.b_off / 2;
  uint32_t* ent = reinterpret_cast<uint32_t*>(smem + L.ent_off);
  int32_t* colln = reinterpret_cast<int32_t*>(smem + L.colln_off);
  uint8_t* coll = smem + L.coll_off;
  uint16_t* nbl = sm16 + L.nbl_off / 2;
  const int s16 = L.s_off / 2;                    // S offset in bf16 elements
  uint16_t* S = sm16 + s16;

  const int64_t tile = xcd_tile(blockIdx.x, padded_tiles);
  if (tile >= total_tiles) return;
  const int64_t mt = tile / n_tiles_n;
  const int64_t o0 = (tile % n_tiles_n) * NT;
  const int64_t b = mt / tiles_per_b;
  const int64_t pt = mt % tiles_per_b;
  const int64_t n0 = pt * V3_MT;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 3, wn = wave >> 2;
  const int64_t lo = p.tile_lo[pt];
  const int span = static_cast<int>(min(static_cast<int64_t>(zr), p.Nin - lo));

  for (int i = tid; i < V3_MT * V; i += 512) {
    const int r = i / V, v = i - r * V;
    ent[v * V3_MT + r] = p.tile_ent[n0 * p.V + i];
  }
  for (int i = tid; i < V * 64; i += 512)
    reinterpret_cast<uint32_t*>(coll)[i] = reinterpret_cast<const uint32_t*>(p.tile_coll)[pt * V * 64 + i];
  for (int i = tid; i < V; i += 512) colln[i] = p.tile_coll_n[pt * V + i];
  for (int i = tid; i < V3_MT * K; i += 512) nbl[i] = p.tile_nbr[n0 * p.K + i];
  if (tid < 4) *reinterpret_cast<u32x4*>(&S[zr * V3_CC + tid * 8]) = u32x4{0u, 0u, 0u, 0u};

  const char* xrows = reinterpret_cast<const char*>(static_cast<const uint16_t*>(p.x) + b * p.xs0 + lo * p.xs2);
  const char* wbase = reinterpret_cast<const char*>(static_cast<const uint16_t*>(p.w) + o0 * p.Kpad);
  uint32_t s_off[SV], w_off[B_VECS];
  uint32_t s_ok = 0, w_ok = 0;
#pragma unroll
  for (int j = 0; j < SV; ++j) {
    const int q = tid + 512 * j;
    s_ok |= static_cast<uint32_t>((q >> 2) < span) << j;
    s_off[j] = static_cast<uint32_t>(((q >> 2) * p.xs2 + (q & 3) * 8) * 2);
  }
#pragma unroll
  for (int i = 0; i < B_VECS; ++i) {
    const int q = tid + 512 * i;
    w_ok |= static_cast<uint32_t>(q < NT * 4 && o0 + (q >> 2) < p.Cout) << i;
    w_off[i] = static_cast<uint32_t>(((q >> 2) * p.Kpad + (q & 3) * 8) * 2);
  }
  const int ncc = static_cast<int>(p.C / V3_CC);
  const int nit = ncc * V;

  u32x4 rs[SV], rb[B_VECS];
  auto load_s = [&](int cc) {
    const char* base = xrows + cc * V3_CC * 2;
#pragma unroll
    for (int j = 0; j < SV; ++j)
      rs[j] = ((s_ok >> j) & 1) ? *reinterpret_cast<const u32x4*>(base + s_off[j]) : u32x4{0u, 0u, 0u, 0u};
  };
  auto store_s = [&]() {
#pragma unroll
    for (int j = 0; j < SV; ++j) {
      const int q = tid + 512 * j;
      if ((s_ok >> j) & 1) *reinterpret_cast<u32x4*>(&S[swz32(q >> 2, q & 3)]) = rs[j];
    }
  };
  auto load_w = [&](int cc, int v) {
    const char* base = wbase + (static_cast<int64_t>(v) * p.C + cc * V3_CC) * 2;
#pragma unroll
    for (int i = 0; i < B_VECS; ++i)
      rb[i] = ((w_ok >> i) & 1) ? *reinterpret_cast<const u32x4*>(base + w_off[i]) : u32x4{0u, 0u, 0u, 0u};
  };
  auto store_w = [&](int buf) {
    uint16_t* bsm = Bs + buf * NT * V3_CC;
#pragma unroll
    for (int i = 0; i < B_VECS; ++i) {
      const int q = tid + 512 * i;
      if (q < NT * 4) *reinterpret_cast<u32x4*>(&bsm[swz32(q >> 2, q & 3)]) = rb[i];
    }
  };
  // sums of the slots with two or more neighbours into A tile `buf`
  auto build_coll = [&](int v, int buf) {
    const int items = colln[v] * 4;
    uint16_t* a = sm16 + buf * V3_MT * V3_CC;
    for (int item = tid; item < items; item += 512) {
      const int row = coll[v * V3_MT + (item >> 2)];
      const int part = item & 3;
      const uint32_t e = ent[v * V3_MT + row];
      const int cnt = (e >> 8) & 0xff;
      const uint16_t* nb = nbl + row * K + (e & 0xff);
      // groups of four neighbours: independent index reads, then independent
      // row reads; missing neighbours read the zero row (adding exact zeros)
      f32x8 acc8 = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      for (int j0 = 0; j0 < cnt; j0 += 4) {
        const int r0 = j0 == 0 ? static_cast<int>(e >> 16) : nb[j0];
        const int r1 = j0 + 1 < cnt ? nb[j0 + 1] : zr;
        const int r2 = j0 + 2 < cnt ? nb[j0 + 2] : zr;
        const int r3 = j0 + 3 < cnt ? nb[j0 + 3] : zr;
        const u32x4 x0 = *reinterpret_cast<const u32x4*>(&S[swz32(r0, part)]);
        const u32x4 x1 = *reinterpret_cast<const u32x4*>(&S[swz32(r1, part)]);
        const u32x4 x2 = *reinterpret_cast<const u32x4*>(&S[swz32(r2, part)]);
        const u32x4 x3 = *reinterpret_cast<const u32x4*>(&S[swz32(r3, part)]);
        acc8 += unpack_bf16x8(x0);
        acc8 += unpack_bf16x8(x1);
        acc8 += unpack_bf16x8(x2);
        acc8 += unpack_bf16x8(x3);
      }
      *reinterpret_cast<u32x4*>(&a[swz32(row, part)]) =
          u32x4{cvt_pk_bf16(acc8[0], acc8[1]), cvt_pk_bf16(acc8[2], acc8[3]), cvt_pk_bf16(acc8[4], acc8[5]),
                cvt_pk_bf16(acc8[6], acc8[7])};
    }
  };

  f32x16 acc[2][CB];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < CB; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  int rowm[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) rowm[i] = wm * 64 + i * 32 + (lane & 31);

  load_s(0);
  load_w(0, 0);
  store_s();
  store_w(0);
  if (ncc > 1) load_s(1);
  __syncthreads();
  build_coll(0, 0);
  uint32_t ecur[2], enxt[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) ecur[i] = ent[rowm[i]];
  __syncthreads();

  int cc1 = 0, v1 = 0;
  for (int it = 0; it < nit; ++it) {
    const int cur = it & 1;
    if (++v1 == V) { v1 = 0; ++cc1; }
    const bool more = it + 1 < nit;
    if (more) {
      load_w(cc1, v1);
#pragma unroll
      for (int i = 0; i < 2; ++i) enxt[i] = ent[v1 * V3_MT + rowm[i]];
      if (v1 != 0) build_coll(v1, cur ^ 1);
    }
    int a_base[2], s_row[2];
    bool from_a[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      from_a[i] = ((ecur[i] >> 8) & 0xff) >= 2;
      s_row[i] = static_cast<int>(ecur[i] >> 16);
      a_base[i] = cur * V3_MT * V3_CC;
    }
    const uint16_t* bsm = Bs + cur * NT * V3_CC;
#pragma unroll
    for (int ks = 0; ks < V3_CC / 16; ++ks) {
      const int q = ks * 2 + (lane >> 5);
      bf16x8 af[2], bfr[CB];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int off = from_a[i] ? a_base[i] + swz32(rowm[i], q) : s16 + swz32(s_row[i], q);
        af[i] = *reinterpret_cast<const bf16x8*>(&sm16[off]);
      }
#pragma unroll
      for (int j = 0; j < CB; ++j)
        bfr[j] = *reinterpret_cast<const bf16x8*>(&bsm[swz32(wn * WN + j * 32 + (lane & 31), q)]);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < CB; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
    }
    if (more) store_w(cur ^ 1);
    __syncthreads();
    if (more && v1 == 0) {      // chunk boundary: every MFMA of chunk cc1-1 is done with S
      store_s();
      __syncthreads();
      if (cc1 + 1 < ncc) load_s(cc1 + 1);
      build_coll(0, cur ^ 1);
      __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) ecur[i] = enxt[i];
  }

  OutT* y = static_cast<OutT*>(p.y) + b * p.ys0;
#pragma unroll
  for (int j = 0; j < CB; ++j) {
    const int64_t o = o0 + wn * WN + j * 32 + (lane & 31);
    if (o >= p.Cout) continue;
    const float bo = p.bias ? p.bias[o] : 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t n = n0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (n < p.Nout) Elem<OutT>::store(y + o * p.ys1 + n * p.ys2, epilogue(acc[i][j][r] + bo, p.relu));
      }
  }
}

template <int NT, int SV>
static void launch_bf16_v4_sv(const KnnParams& p, int out_t, hipStream_t s) {
  const int64_t tiles_per_b = (p.Nout + V3_MT - 1) / V3_MT;
  const int64_t n_tiles_n = (p.Cout + NT - 1) / NT;
  const int64_t total = p.B * tiles_per_b * n_tiles_n;
  const int64_t padded = (total + 7) / 8 * 8;
  const size_t lds = v4_layout(NT, static_cast<int>(p.V), static_cast<int>(p.K), p.zero_row).total;
  dim3 grid(static_cast<unsigned>(padded));
  if (out_t == FOVI_BF16) {
    (void)reserve_dynamic_lds(reinterpret_cast<const void*>(&knnconv_bf16_v4_kernel<NT, SV, uint16_t>), lds);
    hipLaunchKernelGGL((knnconv_bf16_v4_kernel<NT, SV, uint16_t>), grid, dim3(512), lds, s, p, tiles_per_b,
                       n_tiles_n, total, padded);
  } else {
    (void)reserve_dynamic_lds(reinterpret_cast<const void*>(&knnconv_bf16_v4_kernel<NT, SV, float>), lds);
    hipLaunchKernelGGL((knnconv_bf16_v4_kernel<NT, SV, float>), grid, dim3(512), lds, s, p, tiles_per_b,
                       n_tiles_n, total, padded);
  }
}

template <int NT>
static bool launch_bf16_v4(const KnnParams& p, int out_t, hipStream_t s) {
  const int sv = (p.zero_row * 4 + 511) / 512;
  if (sv <= 2) launch_bf16_v4_sv<NT, 2>(p, out_t, s);
  else if (sv <= 4) launch_bf16_v4_sv<NT, 4>(p, out_t, s);
  else if (sv <= 6) launch_bf16_v4_sv<NT, 6>(p, out_t, s);
  else if (sv <= 8) launch_bf16_v4_sv<NT, 8>(p, out_t, s);
  else return false;
  return true;
}

static int v4_tile_n(const KnnParams& p) {
  if (p.zero_row <= 0 || p.zero_row > 1024 || !p.tile_coll || !p.tile_coll_n) return 0;
  return pick_tile_n(p.Cout, [&](int nt) {
    return v4_layout(nt, static_cast<int>(p.V), static_cast<int>(p.K), p.zero_row).total <= 160 * 1024;
  });
}

// ---------------------------------------------------------------------------
// bf16 MFMA path for few input channels (c_in <= CP, CP = 4 or 8)
// ---------------------------------------------------------------------------
// Input rows are channels-last and padded to CP channels (8 or 16 bytes), so
// one load fetches a neighbour's whole feature vector; the packed weight has
// CP channels per slot (zeros beyond c_in), and a 32-wide reduction chunk is
// 32 / CP slots. Each thread assembles the slot sums of (point, slot) items
// from the CSR lists (fp32 sums, one RNE rounding) into the chunk's A tile;
// channels >= c_in of the input rows are masked to zero. Tile shape and MFMA
// core are those of the large-channel kernels.
template <int CP> struct RowVec;
template <> struct RowVec<4> { typedef uint32_t __attribute__((ext_vector_type(2))) T; };
template <> struct RowVec<8> { typedef u32x4 T; };

template <int NT, int CP, typename OutT>
__global__ __launch_bounds__(512, 1) void knnconv_bf16_smallc_kernel(KnnParams p, int64_t tiles_per_b,
                                                                     int64_t n_tiles_n, int64_t total_tiles,
                                                                     int64_t padded_tiles) {
  typedef typename RowVec<CP>::T RowT;
  constexpr int NW = CP / 2;               // 32-bit words per row
  constexpr int SPC = 32 / CP;             // slots per chunk
  constexpr int ITEMS = V3_MT * SPC / 512; // (point, slot) items per thread
  constexpr int WN = NT / 2;
  constexpr int CB = WN / 32;
  constexpr int B_VECS = (NT * V3_CC / 8 + 511) / 512;
  __shared__ __attribute__((aligned(16))) uint16_t As[2][V3_MT * V3_CC];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[2][NT * V3_CC];

  const int64_t tile = xcd_tile(blockIdx.x, padded_tiles);
  if (tile >= total_tiles) return;
  const int64_t mt = tile / n_tiles_n;
  const int64_t o0 = (tile % n_tiles_n) * NT;
  const int64_t b = mt / tiles_per_b;
  const int64_t n0 = (mt % tiles_per_b) * V3_MT;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 3, wn = wave >> 2;
  const uint16_t* xb = static_cast<const uint16_t*>(p.x) + b * p.xs0;
  const char* wbase = reinterpret_cast<const char*>(static_cast<const uint16_t*>(p.w) + o0 * p.Kpad);
  const int nk = static_cast<int>((p.V * CP + V3_CC - 1) / V3_CC);
  // mask of the real channels within a padded row
  uint32_t cmask[NW];
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    const int c0 = 2 * w;
    cmask[w] = (c0 < p.C ? 0x0000ffffu : 0u) | (c0 + 1 < p.C ? 0xffff0000u : 0u);
  }

  RowT ra[ITEMS];
  u32x4 rb[B_VECS];
  // All of a thread's (point, slot) items advance together through their
  // neighbour lists in groups of four: the index loads of a group are issued
  // together, then the row loads, so a list of length c costs about
  // 2 * ceil(c / 4) memory round trips instead of 2 * c.
  auto gather = [&](int kt) {
    int cnt[ITEMS];
    const int32_t* nb[ITEMS];
    int most = 0;
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      const int item = tid + 512 * i;
      const int row = item / SPC, sl = item - row * SPC;
      const int64_t n = n0 + row;
      const int64_t v = static_cast<int64_t>(kt) * SPC + sl;
      int32_t e = 0;
      if (n < p.Nout && v < p.V) e = p.slot_ptr[n * p.V + v];
      cnt[i] = e & 0xffff;
      nb[i] = p.nbr + n * p.K + (e >> 16);
      most = max(most, cnt[i]);
    }
    float acc[ITEMS][CP];
#pragma unroll
    for (int i = 0; i < ITEMS; ++i)
#pragma unroll
      for (int c = 0; c < CP; ++c) acc[i][c] = 0.0f;
    for (int j0 = 0; j0 < most; j0 += 4) {
      int idx[ITEMS][4];
#pragma unroll
      for (int i = 0; i < ITEMS; ++i)
#pragma unroll
        for (int u = 0; u < 4; ++u) idx[i][u] = (j0 + u < cnt[i]) ? nb[i][j0 + u] : -1;
      RowT r[ITEMS][4];
#pragma unroll
      for (int i = 0; i < ITEMS; ++i)
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          RowT z;
#pragma unroll
          for (int w = 0; w < NW; ++w) z[w] = 0u;
          r[i][u] = idx[i][u] >= 0 ? *reinterpret_cast<const RowT*>(xb + static_cast<int64_t>(idx[i][u]) * p.xs2) : z;
        }
#pragma unroll
      for (int i = 0; i < ITEMS; ++i)
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
          for (int w = 0; w < NW; ++w) {
            const uint32_t bits = r[i][u][w] & cmask[w];
            acc[i][2 * w] += __uint_as_float(bits << 16);
            acc[i][2 * w + 1] += __uint_as_float(bits & 0xffff0000u);
          }
    }
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      RowT out;
#pragma unroll
      for (int w = 0; w < NW; ++w) out[w] = cvt_pk_bf16(acc[i][2 * w], acc[i][2 * w + 1]);
      ra[i] = out;
    }
  };
  auto store_a = [&](int buf) {
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      const int item = tid + 512 * i;
      const int row = item / SPC, sl = item - row * SPC;
      const int byte = sl * CP * 2;                 // byte offset in the 64-byte row
      const int q = byte >> 4;
      uint16_t* dst = &As[buf][swz32(row, q) + ((byte & 15) >> 1)];
      *reinterpret_cast<RowT*>(dst) = ra[i];
    }
  };
  auto load_w = [&](int kt) {
    const char* base = wbase + static_cast<int64_t>(kt) * V3_CC * 2;
#pragma unroll
    for (int i = 0; i < B_VECS; ++i) {
      const int q = tid + 512 * i;
      const bool ok = q < NT * 4 && o0 + (q >> 2) < p.Cout;
      rb[i] = ok ? *reinterpret_cast<const u32x4*>(base + ((q >> 2) * p.Kpad + (q & 3) * 8) * 2)
                 : u32x4{0u, 0u, 0u, 0u};
    }
  };
  auto store_w = [&](int buf) {
#pragma unroll
    for (int i = 0; i < B_VECS; ++i) {
      const int q = tid + 512 * i;
      if (q < NT * 4) *reinterpret_cast<u32x4*>(&Bs[buf][swz32(q >> 2, q & 3)]) = rb[i];
    }
  };

  f32x16 acc[2][CB];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < CB; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  gather(0);
  load_w(0);
  store_a(0);
  store_w(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < nk;
    if (more) {
      gather(kt + 1);
      load_w(kt + 1);
    }
#pragma unroll
    for (int ks = 0; ks < V3_CC / 16; ++ks) {
      const int q = ks * 2 + (lane >> 5);
      bf16x8 af[2], bfr[CB];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        af[i] = *reinterpret_cast<const bf16x8*>(&As[cur][swz32(wm * 64 + i * 32 + (lane & 31), q)]);
#pragma unroll
      for (int j = 0; j < CB; ++j)
        bfr[j] = *reinterpret_cast<const bf16x8*>(&Bs[cur][swz32(wn * WN + j * 32 + (lane & 31), q)]);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < CB; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
    }
    if (more) {
      store_a(cur ^ 1);
      store_w(cur ^ 1);
    }
    __syncthreads();
  }

  OutT* y = static_cast<OutT*>(p.y) + b * p.ys0;
#pragma unroll
  for (int j = 0; j < CB; ++j) {
    const int64_t o = o0 + wn * WN + j * 32 + (lane & 31);
    if (o >= p.Cout) continue;
    const float bo = p.bias ? p.bias[o] : 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t n = n0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (n < p.Nout) Elem<OutT>::store(y + o * p.ys1 + n * p.ys2, epilogue(acc[i][j][r] + bo, p.relu));
      }
  }
}

template <int NT, int CP>
static void launch_bf16_smallc(const KnnParams& p, int out_t, hipStream_t s) {
  const int64_t tiles_per_b = (p.Nout + V3_MT - 1) / V3_MT;
  const int64_t n_tiles_n = (p.Cout + NT - 1) / NT;
  const int64_t total = p.B * tiles_per_b * n_tiles_n;
  const int64_t padded = (total + 7) / 8 * 8;
  dim3 grid(static_cast<unsigned>(padded));
  if (out_t == FOVI_BF16)
    hipLaunchKernelGGL((knnconv_bf16_smallc_kernel<NT, CP, uint16_t>), grid, dim3(512), 0, s, p, tiles_per_b,
                       n_tiles_n, total, padded);
  else
    hipLaunchKernelGGL((knnconv_bf16_smallc_kernel<NT, CP, float>), grid, dim3(512), 0, s, p, tiles_per_b,
                       n_tiles_n, total, padded);
}

template <int CP>
static void launch_bf16_smallc_nt(const KnnParams& p, int out_t, hipStream_t s) {
  if (p.Cout % 256 == 0) launch_bf16_smallc<256, CP>(p, out_t, s);
  else if (p.Cout % 192 == 0) launch_bf16_smallc<192, CP>(p, out_t, s);
  else if (p.Cout > 64) launch_bf16_smallc<128, CP>(p, out_t, s);
  else launch_bf16_smallc<64, CP>(p, out_t, s);
}

// ---------------------------------------------------------------------------
// Few-channel layers with many slots, two passes through a workspace
// ---------------------------------------------------------------------------
// Pass 1 (slotsum_kernel): one wave per output point, each lane owning every 64th
// slot. A lane issues its slots' table entries together, then the first
// neighbour index of each, then those neighbours' rows (three rounds of
// independent loads instead of a dependent chain per slot); neighbours after
// the first, rare at one neighbour per slot on average, follow in list order.
// The lane writes the point's slot-major reduction row A[b, n, v * CP + c] in
// bf16 (fp32 sums, one RNE rounding; in list order from +0 over groups of
// FC_GROUP neighbours, the groups' sums added in order, as the fused kernel
// sums them), zero padded to k_pad. Few registers, many waves in flight: the neighbour-list latency is
// hidden by occupancy, which the MFMA kernels (one 8-wave workgroup per CU)
// cannot do. Pass 2 (dense_gemm_kernel): the MFMA tile core of the kernels
// above with A rows read contiguously from the workspace.
template <int CP>
__global__ __launch_bounds__(256) void slotsum_kernel(KnnParams p, uint16_t* A, int64_t rows) {
  typedef typename RowVec<CP>::T RowT;
  constexpr int NW = CP / 2;
  constexpr int SL = 4;                       // slots per lane per round
  const int lane = threadIdx.x & 63;
  // XCD-aware order: each XCD sums a contiguous range of rows (whole images), so an image's
  // rows are fetched into one L2 only (the grid is padded to a multiple of 8 blocks)
  const int64_t m = xcd_tile(blockIdx.x, gridDim.x) * 4 + (threadIdx.x >> 6);   // output row (b, n)
  if (m >= rows) return;
  const int64_t b = m / p.Nout, n = m - b * p.Nout;
  const uint16_t* xb = static_cast<const uint16_t*>(p.x) + b * p.xs0;
  const int32_t* nbn = p.nbr + n * p.K;
  uint16_t* arow = A + m * p.Kpad;
  uint32_t cmask[NW];
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    const int c0 = 2 * w;
    cmask[w] = (c0 < p.C ? 0x0000ffffu : 0u) | (c0 + 1 < p.C ? 0xffff0000u : 0u);
  }
  auto add_row = [&](float* acc, const RowT& r) {
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const uint32_t bits = r[w] & cmask[w];
      acc[2 * w] += __uint_as_float(bits << 16);
      acc[2 * w + 1] += __uint_as_float(bits & 0xffff0000u);
    }
  };
  RowT zero;
#pragma unroll
  for (int w = 0; w < NW; ++w) zero[w] = 0u;
  const int64_t nslots = p.Kpad / CP;
  for (int64_t v0 = 0; v0 < nslots; v0 += 64 * SL) {
    int32_t e[SL];
#pragma unroll
    for (int s = 0; s < SL; ++s) {
      const int64_t v = v0 + lane + 64 * s;
      e[s] = v < p.V ? p.slot_ptr[n * p.V + v] : 0;          // padding slots: no neighbour
    }
    int idx[SL];
#pragma unroll
    for (int s = 0; s < SL; ++s) idx[s] = (e[s] & 0xffff) ? nbn[e[s] >> 16] : -1;
    RowT r[SL];
#pragma unroll
    for (int s = 0; s < SL; ++s)
      r[s] = idx[s] >= 0 ? *reinterpret_cast<const RowT*>(xb + static_cast<int64_t>(idx[s]) * p.xs2) : zero;
    float acc[SL][CP];
#pragma unroll
    for (int s = 0; s < SL; ++s) {
#pragma unroll
      for (int c = 0; c < CP; ++c) acc[s][c] = 0.0f;
      add_row(acc[s], r[s]);
    }
    // neighbours [from, to) of a slot's list added to sum in list order, four reads in flight
    auto add_range = [&](float* sum, const int32_t* nb, int from, int to) {
      for (int j0 = from; j0 < to; j0 += 4) {
        int id4[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) id4[u] = j0 + u < to ? nb[j0 + u] : -1;
        RowT r4[4];
#pragma unroll
        for (int u = 0; u < 4; ++u)
          r4[u] = id4[u] >= 0 ? *reinterpret_cast<const RowT*>(xb + static_cast<int64_t>(id4[u]) * p.xs2) : zero;
#pragma unroll
        for (int u = 0; u < 4; ++u) add_row(sum, r4[u]);
      }
    };
#pragma unroll
    for (int s = 0; s < SL; ++s) {
      const int cnt = e[s] & 0xffff;
      const int32_t* nb = nbn + (e[s] >> 16);
      // the first group of FC_GROUP (the first neighbour is in already), then each further
      // group summed from +0 and added in order: the fused kernel's order
      add_range(acc[s], nb, 1, cnt < FC_GROUP ? cnt : FC_GROUP);
      for (int g0 = FC_GROUP; g0 < cnt; g0 += FC_GROUP) {
        float part[CP];
#pragma unroll
        for (int c = 0; c < CP; ++c) part[c] = 0.0f;
        add_range(part, nb, g0, cnt < g0 + FC_GROUP ? cnt : g0 + FC_GROUP);
#pragma unroll
        for (int c = 0; c < CP; ++c) acc[s][c] += part[c];
      }
    }
#pragma unroll
    for (int s = 0; s < SL; ++s) {
      const int64_t v = v0 + lane + 64 * s;
      if (v < nslots) {
        RowT out;
#pragma unroll
        for (int w = 0; w < NW; ++w) out[w] = cvt_pk_bf16(acc[s][2 * w], acc[s][2 * w + 1]);
        *reinterpret_cast<RowT*>(arow + v * CP) = out;
      }
    }
  }
}

// Y[b, n, o] = sum_k A[(b, n), k] * W[o, k] (+ bias, activation), A in the workspace.
template <int NT, typename OutT>
__global__ __launch_bounds__(512, 1) void dense_gemm_kernel(KnnParams p, const uint16_t* A, int64_t tiles_per_b,
                                                            int64_t n_tiles_n, int64_t total_tiles,
                                                            int64_t padded_tiles) {
  constexpr int WN = NT / 2;
  constexpr int CB = WN / 32;
  constexpr int B_VECS = (NT * V3_CC / 8 + 511) / 512;
  __shared__ __attribute__((aligned(16))) uint16_t As[2][V3_MT * V3_CC];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[2][NT * V3_CC];
  const int64_t tile = xcd_tile(blockIdx.x, padded_tiles);
  if (tile >= total_tiles) return;
  const int64_t mt = tile / n_tiles_n;
  const int64_t o0 = (tile % n_tiles_n) * NT;
  const int64_t b = mt / tiles_per_b;
  const int64_t n0 = (mt % tiles_per_b) * V3_MT;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 3, wn = wave >> 2;
  const uint16_t* ab = A + (b * p.Nout + n0) * p.Kpad;
  const char* wbase = reinterpret_cast<const char*>(static_cast<const uint16_t*>(p.w) + o0 * p.Kpad);
  const int nk = static_cast<int>(p.Kpad / V3_CC);
  u32x4 ra[2], rb[B_VECS];
  auto load = [&](int kt) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int q = tid + 512 * i;
      const int row = q >> 2;
      ra[i] = n0 + row < p.Nout
                  ? *reinterpret_cast<const u32x4*>(ab + static_cast<int64_t>(row) * p.Kpad + kt * V3_CC + (q & 3) * 8)
                  : u32x4{0u, 0u, 0u, 0u};
    }
    const char* base = wbase + static_cast<int64_t>(kt) * V3_CC * 2;
#pragma unroll
    for (int i = 0; i < B_VECS; ++i) {
      const int q = tid + 512 * i;
      const bool ok = q < NT * 4 && o0 + (q >> 2) < p.Cout;
      rb[i] = ok ? *reinterpret_cast<const u32x4*>(base + ((q >> 2) * p.Kpad + (q & 3) * 8) * 2)
                 : u32x4{0u, 0u, 0u, 0u};
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int q = tid + 512 * i;
      *reinterpret_cast<u32x4*>(&As[buf][swz32(q >> 2, q & 3)]) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < B_VECS; ++i) {
      const int q = tid + 512 * i;
      if (q < NT * 4) *reinterpret_cast<u32x4*>(&Bs[buf][swz32(q >> 2, q & 3)]) = rb[i];
    }
  };
  f32x16 acc[2][CB];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < CB; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
  load(0);
  store(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < nk;
    if (more) load(kt + 1);
#pragma unroll
    for (int ks = 0; ks < V3_CC / 16; ++ks) {
      const int q = ks * 2 + (lane >> 5);
      bf16x8 af[2], bfr[CB];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        af[i] = *reinterpret_cast<const bf16x8*>(&As[cur][swz32(wm * 64 + i * 32 + (lane & 31), q)]);
#pragma unroll
      for (int j = 0; j < CB; ++j)
        bfr[j] = *reinterpret_cast<const bf16x8*>(&Bs[cur][swz32(wn * WN + j * 32 + (lane & 31), q)]);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < CB; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
    }
    if (more) store(cur ^ 1);
    __syncthreads();
  }
  OutT* y = static_cast<OutT*>(p.y) + b * p.ys0;
#pragma unroll
  for (int j = 0; j < CB; ++j) {
    const int64_t o = o0 + wn * WN + j * 32 + (lane & 31);
    if (o >= p.Cout) continue;
    const float bo = p.bias ? p.bias[o] : 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t n = n0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (n < p.Nout) Elem<OutT>::store(y + o * p.ys1 + n * p.ys2, epilogue(acc[i][j][r] + bo, p.relu));
      }
  }
}

template <int NT>
static void launch_dense(const KnnParams& p, const uint16_t* A, int out_t, hipStream_t s) {
  const int64_t tiles_per_b = (p.Nout + V3_MT - 1) / V3_MT;
  const int64_t n_tiles_n = (p.Cout + NT - 1) / NT;
  const int64_t total = p.B * tiles_per_b * n_tiles_n;
  const int64_t padded = (total + 7) / 8 * 8;
  dim3 grid(static_cast<unsigned>(padded));
  if (out_t == FOVI_BF16)
    hipLaunchKernelGGL((dense_gemm_kernel<NT, uint16_t>), grid, dim3(512), 0, s, p, A, tiles_per_b, n_tiles_n,
                       total, padded);
  else
    hipLaunchKernelGGL((dense_gemm_kernel<NT, float>), grid, dim3(512), 0, s, p, A, tiles_per_b, n_tiles_n,
                       total, padded);
}

static int launch_two_pass(const KnnParams& p, int cp, uint16_t* A, int out_t, hipStream_t s) {
  const int64_t rows = p.B * p.Nout;
  dim3 g1(static_cast<unsigned>(((rows + 3) / 4 + 7) / 8 * 8));
  if (cp == 4) hipLaunchKernelGGL((slotsum_kernel<4>), g1, dim3(256), 0, s, p, A, rows);
  else hipLaunchKernelGGL((slotsum_kernel<8>), g1, dim3(256), 0, s, p, A, rows);
  if (check_launch("fovi_knnconv_fwd(slot sums)")) return 1;
  if (p.Cout % 256 == 0) launch_dense<256>(p, A, out_t, s);
  else if (p.Cout % 192 == 0) launch_dense<192>(p, A, out_t, s);
  else if (p.Cout > 64) launch_dense<128>(p, A, out_t, s);
  else launch_dense<64>(p, A, out_t, s);
  return check_launch("fovi_knnconv_fwd(dense gemm)");
}

template <int NT, bool VEC>
static void launch_bf16(const KnnParams& p, int out_t, hipStream_t s) {
  const int64_t tiles_per_b = (p.Nout + MM_MT - 1) / MM_MT;
  const int64_t n_tiles_n = (p.Cout + NT - 1) / NT;
  const int64_t total = p.B * tiles_per_b * n_tiles_n;
  const int64_t padded = (total + 7) / 8 * 8;
  dim3 grid(static_cast<unsigned>(padded));
  if (out_t == FOVI_BF16)
    hipLaunchKernelGGL((knnconv_bf16_kernel<NT, VEC, uint16_t>), grid, dim3(256), 0, s, p, tiles_per_b,
                       n_tiles_n, total, padded);
  else
    hipLaunchKernelGGL((knnconv_bf16_kernel<NT, VEC, float>), grid, dim3(256), 0, s, p, tiles_per_b,
                       n_tiles_n, total, padded);
}

// ---------------------------------------------------------------------------
// weight packing
// ---------------------------------------------------------------------------
__global__ void pack_weight_kernel(const float* w_ref, int64_t c_out, int64_t c_in, int64_t n_ref,
                                   void* out, int dtype, int64_t k_pad, int64_t c_slot, const float* w_scale) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= c_out * k_pad) return;
  const int64_t o = idx / k_pad, kk = idx - o * k_pad;
  const int64_t v = kk / c_slot, c = kk - v * c_slot;
  const float val = (v < n_ref && c < c_in) ? w_ref[o * c_in * n_ref + c * n_ref + v] : 0.0f;
  if (dtype == FOVI_F32) static_cast<float*>(out)[idx] = val;
  else if (dtype == FOVI_BF16) static_cast<uint16_t*>(out)[idx] = f32_to_bf16_bits(val);
  else static_cast<uint8_t*>(out)[idx] = f32_to_e4m3(val / w_scale[o]);
}

}  // namespace fovi

extern "C" int fovi_knnconv_pack_weight(const float* w_ref, int64_t c_out, int64_t c_in, int64_t n_ref,
                                        void* w_packed, int32_t out_dtype, int64_t k_pad, int64_t c_slot,
                                        const float* w_scale, void* stream) {
  using namespace fovi;
  clear_error();
  if (!w_ref || !w_packed) { set_error("fovi_knnconv_pack_weight: null pointer"); return 1; }
  if (c_slot == 0) c_slot = c_in;
  if (c_out <= 0 || c_in <= 0 || n_ref <= 0 || c_slot < c_in || k_pad < c_slot * n_ref || k_pad % MM_KC != 0) {
    set_error("fovi_knnconv_pack_weight: bad sizes c_out=%lld c_in=%lld n_ref=%lld k_pad=%lld c_slot=%lld",
              (long long)c_out, (long long)c_in, (long long)n_ref, (long long)k_pad, (long long)c_slot);
    return 1;
  }
  if (out_dtype != FOVI_F32 && out_dtype != FOVI_BF16 && out_dtype != FOVI_F8E4M3) {
    set_error("fovi_knnconv_pack_weight: bad dtype %d", out_dtype); return 1;
  }
  if (out_dtype == FOVI_F8E4M3 && !w_scale) { set_error("fovi_knnconv_pack_weight: fp8 needs w_scale"); return 1; }
  const int64_t n = c_out * k_pad;
  hipLaunchKernelGGL(pack_weight_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), w_ref, c_out, c_in, n_ref, w_packed, out_dtype, k_pad,
                     c_slot, w_scale);
  return check_launch("fovi_knnconv_pack_weight");
}

namespace fovi {

// The few-channel bf16 path: a weight packed with w_c_slot = 4 or 8 >= c_in channels per slot and
// input rows padded to w_c_slot channels: point-major (rows of one image adjacent, x_stride[2] ==
// w_c_slot) or view-major (rows of one point for all images adjacent, x_stride[0] == w_c_slot).
static bool few_channel_rows(const fovi_knnconv_args* a) {
  const int64_t cp = a->w_c_slot;
  return a->x_dtype == FOVI_BF16 && a->w_dtype == FOVI_BF16 && a->w_layout == FOVI_W_ROWS &&
         (cp == 4 || cp == 8) && cp >= a->c_in && a->x_stride[1] == 1 && a->x_stride[0] % cp == 0 &&
         a->x_stride[2] % cp == 0 && (a->x_stride[2] == cp || a->x_stride[0] == cp) &&
         reinterpret_cast<uintptr_t>(a->x) % (2 * cp) == 0;
}

}  // namespace fovi

extern "C" int fovi_knnconv_fwd(const fovi_knnconv_args* a, void* stream) {
  using namespace fovi;
  clear_error();
  note_path("");
  if (!a) { set_error("fovi_knnconv_fwd: null args"); return 1; }
  if (!a->x || !a->slot_ptr || !a->nbr_sorted || !a->w || !a->y) {
    set_error("fovi_knnconv_fwd: null pointer argument"); return 1;
  }
  if (a->batch <= 0 || a->c_in <= 0 || a->n_in <= 0 || a->n_out <= 0 || a->k <= 0 || a->n_ref <= 0 ||
      a->c_out <= 0) {
    set_error("fovi_knnconv_fwd: bad sizes"); return 1;
  }
  // slot_ptr entries are begin << 16 | count in an int32 decoded with a signed shift: begin < 2^15
  if (a->k > 32767) { set_error("fovi_knnconv_fwd: k=%lld exceeds 32767", (long long)a->k); return 1; }
  if (a->w_layout == FOVI_W_ROWS && a->k_pad % MM_KC != 0) {
    set_error("fovi_knnconv_fwd: k_pad=%lld must be a multiple of 64 >= c_in*n_ref=%lld",
              (long long)a->k_pad, (long long)(a->c_in * a->n_ref));
    return 1;
  }
  if (a->y_dtype != FOVI_F32 && a->y_dtype != FOVI_BF16) { set_error("fovi_knnconv_fwd: bad y dtype"); return 1; }
  KnnParams p;
  p.x = a->x; p.B = a->batch; p.C = a->c_in; p.Nin = a->n_in;
  p.xs0 = a->x_stride[0]; p.xs1 = a->x_stride[1]; p.xs2 = a->x_stride[2];
  p.Nout = a->n_out; p.K = a->k; p.V = a->n_ref; p.slot_ptr = a->slot_ptr; p.nbr = a->nbr_sorted;
  p.w = a->w; p.Cout = a->c_out; p.Kpad = a->k_pad; p.bias = a->bias; p.w_scale = a->w_scale;
  p.x_scale = a->x_scale; p.x_scale_dev = a->x_scale_dev; p.y = a->y; p.ys0 = a->y_stride[0]; p.ys1 = a->y_stride[1]; p.ys2 = a->y_stride[2];
  p.tile_lo = a->tile_lo; p.tile_ent = a->tile_ent; p.tile_nbr = a->tile_nbr; p.max_span = a->max_span;
  p.tile_coll = a->tile_coll; p.tile_coll_n = a->tile_coll_n; p.zero_row = a->zero_row;
  if (a->activation != FOVI_ACT_NONE && a->activation != FOVI_ACT_RELU) {
    set_error("fovi_knnconv_fwd: bad activation %d", a->activation); return 1;
  }
  p.relu = a->activation == FOVI_ACT_RELU;
  p.w_layout = a->w_layout;
  p.tile_src = a->tile_src; p.tile_coll_off = a->tile_coll_off; p.tile_cent = a->tile_cent;
  p.coll_off_stride = a->coll_off_stride; p.cent_stride = a->cent_stride;
  p.tile_heavy = a->tile_heavy; p.tile_hlist = a->tile_hlist;
  p.heavy_stride = a->heavy_stride; p.hlist_stride = a->hlist_stride;
  p.wide_units = a->wide_units ? 1 : 0;
  p.w_c_slot = a->w_c_slot > 0 ? a->w_c_slot : static_cast<int>(a->c_in);
  if (p.w_c_slot < p.C || a->k_pad < p.w_c_slot * p.V) {
    set_error("fovi_knnconv_fwd: w_c_slot=%d must be >= c_in and k_pad >= w_c_slot * n_ref", p.w_c_slot);
    return 1;
  }
  if (a->tile_lo && (a->tile_points != V3_MT || !a->tile_span || a->max_span <= 0)) {
    set_error("fovi_knnconv_fwd: tile tables need tile_points=%d, tile_span and max_span > 0", V3_MT);
    return 1;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);

  if (a->w_layout != FOVI_W_ROWS) {
    const int f8 = a->x_dtype == FOVI_F8E4M3 && a->w_dtype == FOVI_F8E4M3;
    if (a->w_layout != FOVI_W_MFMA || !(f8 || (a->x_dtype == FOVI_BF16 && a->w_dtype == FOVI_BF16)) ||
        p.w_c_slot != p.C) {
      set_error("fovi_knnconv_fwd: w_layout=%d needs BF16 or F8E4M3 input and weight", a->w_layout);
      return 1;
    }
    if (!v5_applies(p, f8)) {
      set_error("fovi_knnconv_fwd: fragment-order weights need c_in %% %d == 0, channels-last 16-byte input "
                "rows, the wide-layer tables within 160 KB of LDS (zero_row <= 1024)%s", f8 ? 64 : 32,
                f8 ? " and w_scale" : "");
      return 1;
    }
    const int nb = v5_tiles_of(p);
    if (a->wide_tiles != nb) {
      set_error("fovi_knnconv_fwd: the wide-layer tables were built for %d collision tiles; the kernel uses %d "
                "for their sizes (fovi_knnconv_wide_tiles)", a->wide_tiles, nb);
      return 1;
    }
    if ((f8 ? launch_knnconv_fp8_v5(p, a->y_dtype, s) : launch_knnconv_bf16_v5(p, a->y_dtype, s)) != 0) {
      set_error("fovi_knnconv_fwd: tile span too large for the fragment-order kernel");
      return 1;
    }
    note_path(f8 ? "fp8 v5" : "bf16 v5");
    return check_launch(f8 ? "fovi_knnconv_fwd(fp8 v5)" : "fovi_knnconv_fwd(bf16 v5)");
  }

  if (a->x_dtype == FOVI_F32 && a->w_dtype == FOVI_F32) {
    const int64_t tiles_per_b = (p.Nout + F32_TM - 1) / F32_TM;
    const int64_t mt = p.B * tiles_per_b;
    const int64_t nt = (p.Cout + F32_TN - 1) / F32_TN;
    if (mt > 0x7fffffff || nt > 65535) { set_error("fovi_knnconv_fwd: grid too large"); return 1; }
    dim3 grid(static_cast<unsigned>(mt), static_cast<unsigned>(nt));
    if (a->y_dtype == FOVI_F32)
      hipLaunchKernelGGL((knnconv_f32_kernel<float>), grid, dim3(256), 0, s, p, tiles_per_b);
    else
      hipLaunchKernelGGL((knnconv_f32_kernel<uint16_t>), grid, dim3(256), 0, s, p, tiles_per_b);
    note_path("f32");
    return check_launch("fovi_knnconv_fwd(f32)");
  }
  if (a->x_dtype == FOVI_F8E4M3 && a->w_dtype == FOVI_F8E4M3) {
    if (p.w_c_slot != p.C) { set_error("fovi_knnconv_fwd(fp8): w_c_slot must equal c_in"); return 1; }
    note_path("fp8 rows");
    return launch_knnconv_fp8(p, a->y_dtype, s);
  }
  if (a->x_dtype == FOVI_BF16 && a->w_dtype == FOVI_BF16 && (p.w_c_slot != p.C || few_channel_rows(a))) {
    // packed weight with padded slots: only the few-channel kernels read it
    const int cp = p.w_c_slot;
    if (few_channel_rows(a)) {
      if (launch_knnconv_fewc_vm(p, a, cp, s)) {
        note_path("bf16 few-channel view-major");
        return check_launch("fovi_knnconv_fwd(bf16 few-channel view-major)");
      }
      if (launch_knnconv_fewc(p, a, cp, s)) {
        note_path("bf16 few-channel fused");
        return check_launch("fovi_knnconv_fwd(bf16 few-channel fused)");
      }
      const uint64_t need = static_cast<uint64_t>(p.B) * static_cast<uint64_t>(p.Nout) *
                            static_cast<uint64_t>(p.Kpad) * 2u;
      if (a->workspace && static_cast<uint64_t>(a->workspace_bytes) >= need &&
          reinterpret_cast<uintptr_t>(a->workspace) % 16 == 0)
      {
        note_path("bf16 few-channel two-pass");
        return launch_two_pass(p, cp, static_cast<uint16_t*>(a->workspace), a->y_dtype, s);
      }
      if (cp == 4) launch_bf16_smallc_nt<4>(p, a->y_dtype, s);
      else launch_bf16_smallc_nt<8>(p, a->y_dtype, s);
      note_path("bf16 few-channel");
      return check_launch("fovi_knnconv_fwd(bf16 small-c)");
    }
    set_error("fovi_knnconv_fwd: w_c_slot=%d needs input rows padded to it (point- or view-major)", cp);
    return 1;
  }
  if (p.w_c_slot != p.C) {
    set_error("fovi_knnconv_fwd: w_c_slot != c_in is only supported for bf16"); return 1;
  }
  if (a->x_dtype == FOVI_BF16 && a->w_dtype == FOVI_BF16) {
    const uintptr_t xa = reinterpret_cast<uintptr_t>(a->x);
    const bool rows16 = p.xs1 == 1 && p.xs2 % 8 == 0 && p.xs0 % 8 == 0 && (xa % 16) == 0;
    if (rows16 && p.C % V3_CC == 0 && a->tile_lo && a->tile_ent && a->tile_nbr &&
        a->tile_points == V3_MT && p.K <= 255 && p.V <= 255) {
      const int nt4 = v4_tile_n(p);
      bool ok4 = false;
      if (nt4 == 256) ok4 = launch_bf16_v4<256>(p, a->y_dtype, s);
      else if (nt4 == 192) ok4 = launch_bf16_v4<192>(p, a->y_dtype, s);
      else if (nt4 == 128) ok4 = launch_bf16_v4<128>(p, a->y_dtype, s);
      else if (nt4 == 64) ok4 = launch_bf16_v4<64>(p, a->y_dtype, s);
      if (ok4) {
        note_path("bf16 v4");
        return check_launch("fovi_knnconv_fwd(bf16 v4)");
      }
    }
    if (rows16 && p.C % V2_CC == 0) {
      const int nt = v2_tile_n(p);
      int rc = -1;
      if (nt == 256) rc = launch_bf16_v2<256>(p, a->y_dtype, s);
      else if (nt == 192) rc = launch_bf16_v2<192>(p, a->y_dtype, s);
      else if (nt == 128) rc = launch_bf16_v2<128>(p, a->y_dtype, s);
      else if (nt == 64) rc = launch_bf16_v2<64>(p, a->y_dtype, s);
      if (rc == 0) {
        note_path("bf16 v2");
        return check_launch("fovi_knnconv_fwd(bf16 v2)");
      }
    }
    const bool vec = rows16 && p.C % MM_KC == 0;
    const bool wide = p.Cout % 128 == 0;
    if (vec && wide) launch_bf16<128, true>(p, a->y_dtype, s);
    else if (vec) launch_bf16<64, true>(p, a->y_dtype, s);
    else if (wide) launch_bf16<128, false>(p, a->y_dtype, s);
    else launch_bf16<64, false>(p, a->y_dtype, s);
    note_path(vec ? "bf16 generic (rows)" : "bf16 generic");
    return check_launch("fovi_knnconv_fwd(bf16)");
  }
  set_error("fovi_knnconv_fwd: unsupported dtypes x=%d w=%d", a->x_dtype, a->w_dtype);
  return 1;
}

// ---------------------------------------------------------------------------
// fovi_knnconv_fwd_noalloc: the forward with the library's static scratch
// ---------------------------------------------------------------------------
namespace fovi {

// Slot-sum rows of the few-channel two-pass path for callers that cannot allocate. One copy per
// GPU (a file-scope __device__ array lives in every device's copy of the code object), held
// until the process ends. Host code names it only through the per-device address below.
constexpr int64_t kNoAllocScratchBytes = int64_t(64) << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
// Held for a whole call: one call at a time reads and orders the per-device state below.
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxDevices];
// Recorded on a call's stream after its last use of the scratch; the next call's stream waits
// for it, so calls on different streams of one GPU take the scratch in host call order.
static hipEvent_t g_scratch_done[kMaxDevices];
static bool g_scratch_recorded[kMaxDevices];

// Per-device set-up, once per device with that device current (the caller holds the mutex):
// the device address of `scratch` and the ordering event. Returns the device index, or -1.
static int scratch_setup() {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    set_error("fovi_knnconv_fwd_noalloc: no current device (%s)", hipGetErrorString(e));
    return -1;
  }
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
      set_error("fovi_knnconv_fwd_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                hipGetErrorString(e));
      return -1;
    }
    hipEvent_t ev = nullptr;
    e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    if (e != hipSuccess) {
      set_error("fovi_knnconv_fwd_noalloc: hipEventCreateWithFlags failed on device %d: %s", dev,
                hipGetErrorString(e));
      return -1;
    }
    g_scratch_done[dev] = ev;
    g_scratch_ptr[dev] = ptr;
  }
  return dev;
}

}  // namespace fovi

extern "C" int fovi_knnconv_fwd_noalloc(const fovi_knnconv_args* a, void* stream) {
  using namespace fovi;
  clear_error();
  note_path("");
  if (!a) { set_error("fovi_knnconv_fwd_noalloc: null args"); return 1; }
  if (a->workspace || a->workspace_bytes) {
    set_error("fovi_knnconv_fwd_noalloc: takes no workspace (its scratch is the library's own)");
    return 1;
  }
  if (!few_channel_rows(a)) return fovi_knnconv_fwd(a, stream);   // a path without scratch
  if (a->batch <= 0 || a->n_out <= 0 || a->k_pad <= 0) { set_error("fovi_knnconv_fwd_noalloc: bad sizes"); return 1; }
  // one image's slot-sum rows must fit the scratch; images are then taken in chunks that fit
  const int64_t per_image = a->n_out * a->k_pad * 2;
  if (a->n_out > kNoAllocScratchBytes || a->k_pad > kNoAllocScratchBytes || per_image > kNoAllocScratchBytes) {
    set_error("fovi_knnconv_fwd_noalloc: one image's slot sums (n_out=%lld x k_pad=%lld bf16 = %lld bytes) "
              "exceed the %lld-byte scratch", (long long)a->n_out, (long long)a->k_pad, (long long)per_image,
              (long long)kNoAllocScratchBytes);
    return 1;
  }
  if (!a->x || !a->y) { set_error("fovi_knnconv_fwd_noalloc: null pointer argument"); return 1; }
  if (a->y_dtype != FOVI_F32 && a->y_dtype != FOVI_BF16) {
    set_error("fovi_knnconv_fwd_noalloc: bad y dtype"); return 1;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  const int dev = scratch_setup();
  if (dev < 0) return 1;
  hipStream_t s = static_cast<hipStream_t>(stream);
  // Under stream capture the caller's graph orders the calls; otherwise wait for the previous
  // call's use of the scratch (a no-op on its own stream) and record this one's.
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  hipError_t e = hipStreamIsCapturing(s, &cap);
  if (e != hipSuccess) {
    set_error("fovi_knnconv_fwd_noalloc: hipStreamIsCapturing failed: %s", hipGetErrorString(e));
    return 1;
  }
  const bool order = cap == hipStreamCaptureStatusNone;
  if (order && g_scratch_recorded[dev]) {
    e = hipStreamWaitEvent(s, g_scratch_done[dev], 0);
    if (e != hipSuccess) {
      set_error("fovi_knnconv_fwd_noalloc: hipStreamWaitEvent failed: %s", hipGetErrorString(e));
      return 1;
    }
  }
  const int64_t chunk = kNoAllocScratchBytes / per_image;
  const int64_t y_esize = a->y_dtype == FOVI_F32 ? 4 : 2;
  fovi_knnconv_args b = *a;
  int rc = 0;
  for (int64_t b0 = 0; b0 < a->batch && rc == 0; b0 += chunk) {
    b.batch = std::min(chunk, a->batch - b0);
    b.x = static_cast<const char*>(a->x) + b0 * a->x_stride[0] * 2;
    b.y = static_cast<char*>(a->y) + b0 * a->y_stride[0] * y_esize;
    b.workspace = g_scratch_ptr[dev];
    b.workspace_bytes = kNoAllocScratchBytes;
    rc = fovi_knnconv_fwd(&b, stream);
  }
  if (order) {
    // recorded after whatever was enqueued, also after a failed chunk, so the next call waits for it
    e = hipEventRecord(g_scratch_done[dev], s);
    if (e != hipSuccess) {
      if (rc == 0) set_error("fovi_knnconv_fwd_noalloc: hipEventRecord failed: %s", hipGetErrorString(e));
      g_scratch_recorded[dev] = false;
      return 1;
    }
    g_scratch_recorded[dev] = true;
  }
  return rc;
}
