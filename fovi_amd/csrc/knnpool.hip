// kNN pooling forward (KNNPoolingLayer.forward, fovi/arch/knn.py:345-394).
//
// An HBM-bound gather: every output point reads its k neighbours' feature
// rows and reduces them per channel in fp32 (max, NaN-ignoring mean or sum,
// or a Gaussian-weighted mean renormalised over the non-NaN neighbours),
// rounding once to the output type. Pad-token indices (>= n_in) read NaN,
// as the reference's appended NaN column does.
//  * Channels-last rows (the layout the kNN-conv kernels produce): one
//    thread per (batch row, output point, 16-byte channel group), so the
//    threads of a point read each neighbour row with contiguous 16-byte
//    loads and store 16-byte output pieces; consecutive points share
//    neighbours, and each XCD takes a contiguous range of batch rows, so
//    the rows are fetched into one L2.
//  * Any other strides: one thread per (batch row, output point, channel).
#include "common.h"

namespace fovi {

struct PoolParams {
  const void* x;
  int64_t B, C, Nin, Nout, K;
  int64_t xs0, xs1, xs2;
  const int32_t* nbr;
  const float* w;
  void* y;
  int64_t ys0, ys1, ys2;
  int mode;
};

// Per-channel reduction state of one output value.
struct PoolAcc {
  float a, b;   // max: running max | mean/sum: sum, count | gaussian: sum of weights, sum of x * w
};

__device__ __forceinline__ void pool_init(PoolAcc& s, int mode) {
  s.a = mode == FOVI_POOL_MAX ? -__builtin_inff() : 0.0f;
  s.b = 0.0f;
}

// pass 0 of the Gaussian mode sums the weights of the non-NaN features
__device__ __forceinline__ void pool_add(PoolAcc& s, int mode, float v, float w) {
  const bool nan = v != v;
  switch (mode) {
    case FOVI_POOL_MAX: s.a = fmaxf(s.a, nan ? -__builtin_inff() : v); break;
    case FOVI_POOL_AVG: if (!nan) { s.a += v; s.b += 1.0f; } break;
    case FOVI_POOL_SUM: if (!nan) s.a += v; break;
    default: if (!nan) s.a += w; break;
  }
}

// pass 1 of the Gaussian mode: x * (w / (S + 1e-8)) over the non-NaN features
__device__ __forceinline__ void pool_add_weighted(PoolAcc& s, float v, float w) {
  if (v == v) s.b += v * (w / (s.a + 1e-8f));
}

__device__ __forceinline__ float pool_result(const PoolAcc& s, int mode) {
  switch (mode) {
    case FOVI_POOL_AVG: return s.a / s.b;   // 0 / 0 = NaN when every feature is NaN
    case FOVI_POOL_GAUSSIAN: return s.b;
    default: return s.a;
  }
}

template <typename T> struct Vec16;
template <> struct Vec16<float> {
  static constexpr int N = 4;
  static __device__ __forceinline__ void unpack(uint4 a, float (&v)[4]) {
    v[0] = __uint_as_float(a.x); v[1] = __uint_as_float(a.y);
    v[2] = __uint_as_float(a.z); v[3] = __uint_as_float(a.w);
  }
  static __device__ __forceinline__ void load(const float* p, float (&v)[4]) {
    unpack(*reinterpret_cast<const uint4*>(p), v);
  }
};
template <> struct Vec16<uint16_t> {
  static constexpr int N = 8;
  static __device__ __forceinline__ void unpack(uint4 a, float (&v)[8]) {
    const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(w[i] << 16);
      v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
  static __device__ __forceinline__ void load(const uint16_t* p, float (&v)[8]) {
    unpack(*reinterpret_cast<const uint4*>(p), v);
  }
};

// NV consecutive output channels (unit channel stride, aligned row): 16-byte stores
template <typename OutT, int NV> struct Vec16Out;
template <int NV> struct Vec16Out<uint16_t, NV> {
  static __device__ __forceinline__ void store(uint16_t* y, const float (&o)[NV]) {
#pragma unroll
    for (int q = 0; q < NV / 8; ++q) {
      uint4 w;
      w.x = cvt_pk(o[8 * q], o[8 * q + 1]); w.y = cvt_pk(o[8 * q + 2], o[8 * q + 3]);
      w.z = cvt_pk(o[8 * q + 4], o[8 * q + 5]); w.w = cvt_pk(o[8 * q + 6], o[8 * q + 7]);
      *reinterpret_cast<uint4*>(y + 8 * q) = w;
    }
  }
  static __device__ __forceinline__ uint32_t cvt_pk(float a, float b) {
    return static_cast<uint32_t>(f32_to_bf16_bits(a)) | (static_cast<uint32_t>(f32_to_bf16_bits(b)) << 16);
  }
};
template <int NV> struct Vec16Out<float, NV> {
  static __device__ __forceinline__ void store(float* y, const float (&o)[NV]) {
#pragma unroll
    for (int q = 0; q < NV / 4; ++q) *reinterpret_cast<f32x4*>(y + 4 * q) = f32x4{o[4 * q], o[4 * q + 1], o[4 * q + 2], o[4 * q + 3]};
  }
};

// channels-last rows: thread = (batch row, output point, channel group of 16
// bytes); blocks in XCD-aware order; 32-bit index arithmetic (checked on the host)
template <typename InT, typename OutT>
__global__ __launch_bounds__(256) void knnpool_rows_kernel(PoolParams p, uint32_t groups, int vec_out,
                                                           uint32_t blocks_per_b, int64_t total_blocks,
                                                           int64_t padded_blocks) {
  constexpr int NV = Vec16<InT>::N;
  // each XCD (and its L2) takes a contiguous range of batch rows
  const int64_t tile = xcd_tile(blockIdx.x, padded_blocks);
  if (tile >= total_blocks) return;
  const uint32_t t = static_cast<uint32_t>(tile % blocks_per_b) * 256u + threadIdx.x;
  if (t >= static_cast<uint32_t>(p.Nout) * groups) return;
  const uint32_t g = t % groups, n = t / groups;
  const int64_t b = tile / blocks_per_b;
  const InT* xb = static_cast<const InT*>(p.x) + b * p.xs0 + g * NV;
  const int32_t* nb = p.nbr + static_cast<int64_t>(n) * p.K;
  const float* wn = p.w ? p.w + static_cast<int64_t>(n) * p.K : nullptr;
  PoolAcc s[NV];
#pragma unroll
  for (int c = 0; c < NV; ++c) pool_init(s[c], p.mode);
  const int passes = p.mode == FOVI_POOL_GAUSSIAN ? 2 : 1;
  for (int pass = 0; pass < passes; ++pass) {
    for (int64_t j = 0; j < p.K; ++j) {
      const int64_t idx = nb[j];
      const float w = wn ? wn[j] : 0.0f;
      float v[NV];
      if (idx >= 0 && idx < p.Nin) {
        Vec16<InT>::load(xb + idx * p.xs2, v);
      } else {
#pragma unroll
        for (int c = 0; c < NV; ++c) v[c] = __builtin_nanf("");
      }
#pragma unroll
      for (int c = 0; c < NV; ++c) {
        if (pass == 0) pool_add(s[c], p.mode, v[c], w);
        else pool_add_weighted(s[c], v[c], w);
      }
    }
  }
  OutT* yo = static_cast<OutT*>(p.y) + b * p.ys0 + static_cast<int64_t>(n) * p.ys2 + g * NV * p.ys1;
  float o[NV];
#pragma unroll
  for (int c = 0; c < NV; ++c) o[c] = pool_result(s[c], p.mode);
  if (vec_out) {
    Vec16Out<OutT, NV>::store(yo, o);
  } else {
#pragma unroll
    for (int c = 0; c < NV; ++c) Elem<OutT>::store(yo + c * p.ys1, o[c]);
  }
}

// Channels-last rows, lists of at most POOL_KF neighbours, one reduction mode: the thread
// reads all its indices, then issues all its row loads (a pad token or a list slot past k
// reads row 0, discarded), then reduces in list order, branch-free: two memory latencies per
// thread instead of two per neighbour. The reduction is the one above: a NaN feature adds +0,
// which leaves a sum that started at +0 unchanged (such a sum is never -0).
constexpr int POOL_KF = 16;

template <typename InT, typename OutT, int MODE>
__global__ __launch_bounds__(256) void knnpool_rows_kf_kernel(PoolParams p, uint32_t groups, int vec_out,
                                                              uint32_t blocks_per_b, int64_t total_blocks,
                                                              int64_t padded_blocks) {
  constexpr int NV = Vec16<InT>::N;
  const int64_t tile = xcd_tile(blockIdx.x, padded_blocks);
  if (tile >= total_blocks) return;
  const uint32_t t = static_cast<uint32_t>(tile % blocks_per_b) * 256u + threadIdx.x;
  if (t >= static_cast<uint32_t>(p.Nout) * groups) return;
  const uint32_t g = t % groups, n = t / groups;
  const int64_t b = tile / blocks_per_b;
  const InT* xb = static_cast<const InT*>(p.x) + b * p.xs0 + g * NV;
  const int K = static_cast<int>(p.K);
  const int32_t* nb = p.nbr + static_cast<int64_t>(n) * K;
  const float* wn = MODE == FOVI_POOL_GAUSSIAN ? p.w + static_cast<int64_t>(n) * K : nullptr;
  const int32_t nin = static_cast<int32_t>(p.Nin);
  int32_t idx[POOL_KF];
  float w[POOL_KF];
#pragma unroll
  for (int j = 0; j < POOL_KF; ++j) {
    idx[j] = j < K ? nb[j] : -1;
    w[j] = MODE == FOVI_POOL_GAUSSIAN && j < K ? wn[j] : 0.0f;
  }
  uint4 raw[POOL_KF];
#pragma unroll
  for (int j = 0; j < POOL_KF; ++j) {
    const bool ok = idx[j] >= 0 && idx[j] < nin;
    if (j < K) raw[j] = *reinterpret_cast<const uint4*>(xb + static_cast<int64_t>(ok ? idx[j] : 0) * p.xs2);
  }
  float a[NV], c[NV];
#pragma unroll
  for (int q = 0; q < NV; ++q) {
    a[q] = MODE == FOVI_POOL_MAX ? -__builtin_inff() : 0.0f;
    c[q] = 0.0f;
  }
#pragma unroll
  for (int j = 0; j < POOL_KF; ++j) {
    if (j < K) {
      const bool ok = idx[j] >= 0 && idx[j] < nin;
      float v[NV];
      Vec16<InT>::unpack(raw[j], v);
#pragma unroll
      for (int q = 0; q < NV; ++q) {
        const bool use = ok && v[q] == v[q];
        if (MODE == FOVI_POOL_MAX) a[q] = fmaxf(a[q], use ? v[q] : -__builtin_inff());
        else if (MODE == FOVI_POOL_GAUSSIAN) a[q] += use ? w[j] : 0.0f;
        else a[q] += use ? v[q] : 0.0f;
        if (MODE == FOVI_POOL_AVG) c[q] += use ? 1.0f : 0.0f;
      }
    }
  }
  if (MODE == FOVI_POOL_GAUSSIAN) {
#pragma unroll
    for (int j = 0; j < POOL_KF; ++j) {
      if (j < K) {
        const bool ok = idx[j] >= 0 && idx[j] < nin;
        float v[NV];
        Vec16<InT>::unpack(raw[j], v);
#pragma unroll
        for (int q = 0; q < NV; ++q) {
          const float t = v[q] * (w[j] / (a[q] + 1e-8f));
          c[q] += ok && v[q] == v[q] ? t : 0.0f;
        }
      }
    }
  }
  OutT* yo = static_cast<OutT*>(p.y) + b * p.ys0 + static_cast<int64_t>(n) * p.ys2 + g * NV * p.ys1;
  float o[NV];
#pragma unroll
  for (int q = 0; q < NV; ++q) {
    PoolAcc s{a[q], c[q]};
    o[q] = pool_result(s, MODE);
  }
  if (vec_out) {
    Vec16Out<OutT, NV>::store(yo, o);
  } else {
#pragma unroll
    for (int q = 0; q < NV; ++q) Elem<OutT>::store(yo + q * p.ys1, o[q]);
  }
}

// any strides: thread = (b, n, c)
template <typename InT, typename OutT>
__global__ __launch_bounds__(256) void knnpool_any_kernel(PoolParams p, int64_t total) {
  for (int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; t < total;
       t += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t c = t % p.C;
    const int64_t n = (t / p.C) % p.Nout;
    const int64_t b = t / (p.C * p.Nout);
    const InT* xb = static_cast<const InT*>(p.x) + b * p.xs0 + c * p.xs1;
    const int32_t* nb = p.nbr + n * p.K;
    const float* wn = p.w ? p.w + n * p.K : nullptr;
    PoolAcc s;
    pool_init(s, p.mode);
    const int passes = p.mode == FOVI_POOL_GAUSSIAN ? 2 : 1;
    for (int pass = 0; pass < passes; ++pass)
      for (int64_t j = 0; j < p.K; ++j) {
        const int64_t idx = nb[j];
        const float v = idx >= 0 && idx < p.Nin ? Elem<InT>::load(xb + idx * p.xs2) : __builtin_nanf("");
        const float w = wn ? wn[j] : 0.0f;
        if (pass == 0) pool_add(s, p.mode, v, w);
        else pool_add_weighted(s, v, w);
      }
    Elem<OutT>::store(static_cast<OutT*>(p.y) + b * p.ys0 + c * p.ys1 + n * p.ys2, pool_result(s, p.mode));
  }
}

template <typename InT, typename OutT>
static void launch_pool(const PoolParams& p, hipStream_t s) {
  constexpr int NV = Vec16<InT>::N;
  const bool rows = p.xs1 == 1 && p.C % NV == 0 && p.xs2 % NV == 0 && p.xs0 % NV == 0 &&
                    reinterpret_cast<uintptr_t>(p.x) % 16 == 0;
  const int64_t groups = p.C / NV;
  const int64_t pts = p.Nout * groups;
  const int64_t blocks_per_b = (pts + 255) / 256;
  const int64_t total_blocks = blocks_per_b * p.B;
  const int64_t padded = (total_blocks + 7) / 8 * 8;
  if (rows && pts <= 0x7fffffffLL && padded <= 0x7fffffffLL) {
    const dim3 grid(static_cast<unsigned>(padded));
    // whole channel groups to unit-stride, 16-byte aligned output rows
    const int vec_out = p.ys1 == 1 && (p.ys2 * sizeof(OutT)) % 16 == 0 && (p.ys0 * sizeof(OutT)) % 16 == 0 &&
                        (NV * sizeof(OutT)) % 16 == 0 && reinterpret_cast<uintptr_t>(p.y) % 16 == 0;
    if (p.K <= POOL_KF) {
      const auto args = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, grid, dim3(256), 0, s, p, static_cast<uint32_t>(groups), vec_out,
                           static_cast<uint32_t>(blocks_per_b), total_blocks, padded);
      };
      switch (p.mode) {
        case FOVI_POOL_MAX: args(knnpool_rows_kf_kernel<InT, OutT, FOVI_POOL_MAX>); break;
        case FOVI_POOL_AVG: args(knnpool_rows_kf_kernel<InT, OutT, FOVI_POOL_AVG>); break;
        case FOVI_POOL_SUM: args(knnpool_rows_kf_kernel<InT, OutT, FOVI_POOL_SUM>); break;
        default: args(knnpool_rows_kf_kernel<InT, OutT, FOVI_POOL_GAUSSIAN>); break;
      }
      return;
    }
    hipLaunchKernelGGL((knnpool_rows_kernel<InT, OutT>), grid, dim3(256), 0, s, p, static_cast<uint32_t>(groups),
                       vec_out, static_cast<uint32_t>(blocks_per_b), total_blocks, padded);
    return;
  }
  const int64_t total = p.B * p.Nout * p.C;
  const int64_t blocks = std::min<int64_t>((total + 255) / 256, 256 * 64);
  hipLaunchKernelGGL((knnpool_any_kernel<InT, OutT>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, p,
                     total);
}

}  // namespace fovi

extern "C" int fovi_knnpool_fwd(const fovi_knnpool_args* a, void* stream) {
  using namespace fovi;
  clear_error();
  if (!a || !a->x || !a->nbr || !a->y) { set_error("fovi_knnpool_fwd: null pointer"); return 1; }
  if (a->mode < FOVI_POOL_MAX || a->mode > FOVI_POOL_GAUSSIAN) {
    set_error("fovi_knnpool_fwd: bad mode %d", a->mode); return 1;
  }
  if (a->mode == FOVI_POOL_GAUSSIAN && !a->weights) {
    set_error("fovi_knnpool_fwd: the Gaussian mode needs weights"); return 1;
  }
  if ((a->x_dtype != FOVI_F32 && a->x_dtype != FOVI_BF16) || (a->y_dtype != FOVI_F32 && a->y_dtype != FOVI_BF16)) {
    set_error("fovi_knnpool_fwd: x and y must be F32 or BF16"); return 1;
  }
  if (a->batch < 0 || a->channels < 0 || a->n_in < 0 || a->n_out < 0 || a->k < 1) {
    set_error("fovi_knnpool_fwd: bad sizes (k must be >= 1)"); return 1;
  }
  if (a->batch * a->channels * a->n_out == 0) return 0;
  PoolParams p;
  p.x = a->x; p.B = a->batch; p.C = a->channels; p.Nin = a->n_in; p.Nout = a->n_out; p.K = a->k;
  p.xs0 = a->x_stride[0]; p.xs1 = a->x_stride[1]; p.xs2 = a->x_stride[2];
  p.nbr = a->nbr; p.w = a->mode == FOVI_POOL_GAUSSIAN ? a->weights : nullptr;
  p.y = a->y; p.ys0 = a->y_stride[0]; p.ys1 = a->y_stride[1]; p.ys2 = a->y_stride[2];
  p.mode = a->mode;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (a->x_dtype == FOVI_F32) {
    if (a->y_dtype == FOVI_F32) launch_pool<float, float>(p, s);
    else launch_pool<float, uint16_t>(p, s);
  } else {
    if (a->y_dtype == FOVI_F32) launch_pool<uint16_t, float>(p, s);
    else launch_pool<uint16_t, uint16_t>(p, s);
  }
  return check_launch("fovi_knnpool_fwd");
}

// ----------------------------------------------------------------------------------- backward
// The gradient autograd forms through the reference forward (gather, the NaN handling of each
// mode, the reduction): dx[b, c, i] = sum over the (n, j) whose j-th neighbour is input i of
// coef * dy[b, c, n], and 0 where x[b, c, i] is NaN (the reference masks those features):
//   max:      coef = 1 for the first neighbour position holding the maximum (torch.max over a
//             dim returns the first one), NaN features reading as -inf;
//   avg:      coef = 1 / (number of non-NaN features of (b, c, n));
//   sum:      coef = 1;
//   gaussian: coef = w[n, j] / (sum of the non-NaN features' weights + 1e-8).
// Two passes: the per-output state (argmax position, count, or weight sum + 1e-8) into an fp32
// workspace [b, n, c], then one thread per input element summing over its inverse list.

namespace fovi {
namespace {

struct PoolBwdParams {
  const void* x;
  int64_t B, C, Nin, Nout, K;
  int64_t xs0, xs1, xs2;
  const int32_t* nbr;
  const float* w;
  const void* dy;
  int64_t ds0, ds1, ds2;
  const int32_t* inv_ptr;
  const int32_t* inv;
  float* state;
  void* dx;
  int64_t gs0, gs1, gs2;
  int mode;
};

template <typename InT>
__global__ __launch_bounds__(256) void knnpool_bwd_state_kernel(PoolBwdParams p, int64_t total) {
  for (int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; t < total;
       t += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t c = t % p.C;
    const int64_t n = (t / p.C) % p.Nout;
    const int64_t b = t / (p.C * p.Nout);
    const InT* xb = static_cast<const InT*>(p.x) + b * p.xs0 + c * p.xs1;
    const int32_t* nb = p.nbr + n * p.K;
    float best = -__builtin_inff(), sum = 0.0f;
    int64_t arg = 0;
    for (int64_t j = 0; j < p.K; ++j) {
      const int64_t idx = nb[j];
      const float v = idx >= 0 && idx < p.Nin ? Elem<InT>::load(xb + idx * p.xs2) : __builtin_nanf("");
      const bool nan = v != v;
      if (p.mode == FOVI_POOL_MAX) {
        const float m = nan ? -__builtin_inff() : v;
        if (j == 0 || m > best) { best = m; arg = j; }      // first position of the maximum
      } else if (!nan) {
        sum += p.mode == FOVI_POOL_GAUSSIAN ? p.w[n * p.K + j] : 1.0f;
      }
    }
    p.state[(b * p.Nout + n) * p.C + c] =
        p.mode == FOVI_POOL_MAX ? static_cast<float>(arg) : (p.mode == FOVI_POOL_GAUSSIAN ? sum + 1e-8f : sum);
  }
}

template <typename InT, typename GT, typename DT>
__global__ __launch_bounds__(256) void knnpool_bwd_dx_kernel(PoolBwdParams p, int64_t total) {
  for (int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; t < total;
       t += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t c = t % p.C;
    const int64_t i = (t / p.C) % p.Nin;
    const int64_t b = t / (p.C * p.Nin);
    const float xv = Elem<InT>::load(static_cast<const InT*>(p.x) + b * p.xs0 + c * p.xs1 + i * p.xs2);
    float acc = 0.0f;
    if (xv == xv) {
      const GT* dyb = static_cast<const GT*>(p.dy) + b * p.ds0 + c * p.ds1;
      for (int32_t q = p.inv_ptr[i]; q < p.inv_ptr[i + 1]; ++q) {
        const int64_t e = p.inv[q];
        const int64_t n = e / p.K, j = e - n * p.K;
        const float g = Elem<GT>::load(dyb + n * p.ds2);
        const float st = p.mode == FOVI_POOL_SUM ? 1.0f : p.state[(b * p.Nout + n) * p.C + c];
        switch (p.mode) {
          case FOVI_POOL_MAX: if (st == static_cast<float>(j)) acc += g; break;
          case FOVI_POOL_AVG: acc += g / st; break;
          case FOVI_POOL_SUM: acc += g; break;
          default: acc += g * (p.w[e] / st); break;
        }
      }
    }
    Elem<DT>::store(static_cast<DT*>(p.dx) + b * p.gs0 + c * p.gs1 + i * p.gs2, acc);
  }
}

template <typename InT, typename GT>
static void launch_pool_bwd(const PoolBwdParams& p, bool dx_f32, hipStream_t s) {
  const int64_t n1 = p.B * p.Nout * p.C, n2 = p.B * p.Nin * p.C;
  auto grid = [](int64_t n) { return dim3(static_cast<unsigned>(std::min<int64_t>((n + 255) / 256, 256 * 64))); };
  if (p.mode != FOVI_POOL_SUM && n1 > 0)
    hipLaunchKernelGGL((knnpool_bwd_state_kernel<InT>), grid(n1), dim3(256), 0, s, p, n1);
  if (n2 == 0) return;
  if (dx_f32) hipLaunchKernelGGL((knnpool_bwd_dx_kernel<InT, GT, float>), grid(n2), dim3(256), 0, s, p, n2);
  else hipLaunchKernelGGL((knnpool_bwd_dx_kernel<InT, GT, uint16_t>), grid(n2), dim3(256), 0, s, p, n2);
}

}  // namespace
}  // namespace fovi

extern "C" int fovi_knnpool_bwd(const fovi_knnpool_bwd_args* a, void* stream) {
  using namespace fovi;
  clear_error();
  if (!a || !a->x || !a->nbr || !a->dy || !a->inv_ptr || !a->inv || !a->dx) {
    set_error("fovi_knnpool_bwd: null pointer"); return 1;
  }
  if (a->mode < FOVI_POOL_MAX || a->mode > FOVI_POOL_GAUSSIAN) {
    set_error("fovi_knnpool_bwd: bad mode %d", a->mode); return 1;
  }
  if (a->mode == FOVI_POOL_GAUSSIAN && !a->weights) {
    set_error("fovi_knnpool_bwd: the Gaussian mode needs weights"); return 1;
  }
  if (a->mode != FOVI_POOL_SUM && !a->state) {
    set_error("fovi_knnpool_bwd: this mode needs the state workspace"); return 1;
  }
  const auto okd = [](int d) { return d == FOVI_F32 || d == FOVI_BF16; };
  if (!okd(a->x_dtype) || !okd(a->dy_dtype) || !okd(a->dx_dtype)) {
    set_error("fovi_knnpool_bwd: x, dy and dx must be F32 or BF16"); return 1;
  }
  if (a->batch < 0 || a->channels < 0 || a->n_in < 0 || a->n_out < 0 || a->k < 1) {
    set_error("fovi_knnpool_bwd: bad sizes (k must be >= 1)"); return 1;
  }
  PoolBwdParams p;
  p.x = a->x; p.B = a->batch; p.C = a->channels; p.Nin = a->n_in; p.Nout = a->n_out; p.K = a->k;
  p.xs0 = a->x_stride[0]; p.xs1 = a->x_stride[1]; p.xs2 = a->x_stride[2];
  p.nbr = a->nbr; p.w = a->weights;
  p.dy = a->dy; p.ds0 = a->dy_stride[0]; p.ds1 = a->dy_stride[1]; p.ds2 = a->dy_stride[2];
  p.inv_ptr = a->inv_ptr; p.inv = a->inv; p.state = a->state;
  p.dx = a->dx; p.gs0 = a->dx_stride[0]; p.gs1 = a->dx_stride[1]; p.gs2 = a->dx_stride[2];
  p.mode = a->mode;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool dx32 = a->dx_dtype == FOVI_F32;
  if (a->x_dtype == FOVI_F32) {
    if (a->dy_dtype == FOVI_F32) launch_pool_bwd<float, float>(p, dx32, s);
    else launch_pool_bwd<float, uint16_t>(p, dx32, s);
  } else {
    if (a->dy_dtype == FOVI_F32) launch_pool_bwd<uint16_t, float>(p, dx32, s);
    else launch_pool_bwd<uint16_t, uint16_t>(p, dx32, s);
  }
  return check_launch("fovi_knnpool_bwd");
}
