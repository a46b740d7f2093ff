// Per-tensor OCP e4m3 activation quantization for the fp8 kNN-conv path.
//
// Three launches on the caller's stream, all HBM-bound elementwise work:
//   1. clear the one-float amax accumulator (a fill kernel, no memset node);
//   2. amax: each thread folds 8 elements at a time, a wave reduces with
//      shuffles, one atomic max per wave on the float's bit pattern (|x| >= 0 orders
//      like an unsigned integer);
//   3. quantize: scale = amax * headroom / 448 (1 when amax is 0), q = e4m3(x /
//      scale) with v_cvt_pk_fp8_f32 (round to nearest even, saturating);
//      block 0 stores the scale.
// Dense layouts (x and q with identical strides that cover a contiguous
// range) take a flat 8-elements-per-thread path; anything else walks the
// [batch, channel, point] view element by element.
#include "common.h"
#include "knnconv_internal.h"

namespace fovi {

struct QuantParams {
  const void* x;
  int64_t B, C, N;
  int64_t xs0, xs1, xs2;
  uint8_t* q;
  int64_t qs0, qs1, qs2;
  float headroom;
  const float* scale_in;
  float* scale_out;
  float* amax;
  int64_t total;     // B * C * N
  int dense;         // x and q share strides covering [0, total)
};

template <typename T>
__device__ __forceinline__ void load8(const T* src, float (&v)[8]);
template <>
__device__ __forceinline__ void load8<float>(const float* src, float (&v)[8]) {
  const f32x4 a = *reinterpret_cast<const f32x4*>(src);
  const f32x4 b = *reinterpret_cast<const f32x4*>(src + 4);
#pragma unroll
  for (int i = 0; i < 4; ++i) { v[i] = a[i]; v[4 + i] = b[i]; }
}
template <>
__device__ __forceinline__ void load8<uint16_t>(const uint16_t* src, float (&v)[8]) {
  const u32x4 a = *reinterpret_cast<const u32x4*>(src);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = __uint_as_float(a[i] << 16);
    v[2 * i + 1] = __uint_as_float(a[i] & 0xffff0000u);
  }
}

__device__ __forceinline__ int64_t x_offset(const QuantParams& p, int64_t i) {
  const int64_t n = i % p.N, bc = i / p.N, c = bc % p.C, b = bc / p.C;
  return b * p.xs0 + c * p.xs1 + n * p.xs2;
}
__device__ __forceinline__ int64_t q_offset(const QuantParams& p, int64_t i) {
  const int64_t n = i % p.N, bc = i / p.N, c = bc % p.C, b = bc / p.C;
  return b * p.qs0 + c * p.qs1 + n * p.qs2;
}

__global__ void clear_amax_kernel(float* amax) { *amax = 0.0f; }

template <typename T>
__global__ __launch_bounds__(256) void amax_kernel(QuantParams p) {
  const T* x = static_cast<const T*>(p.x);
  const int64_t step = static_cast<int64_t>(gridDim.x) * 256;
  const int64_t first = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  float m = 0.0f;
  bool nan = false;
  if (p.dense) {
    const int64_t n8 = p.total / 8;
    int64_t i = first;
    // four 8-element pieces per trip, their loads in flight together (one load per trip
    // left the kernel latency-bound at ~2.2 TB/s); the max does not depend on the order
    for (; i + 3 * step < n8; i += 4 * step) {
      float v[4][8];
#pragma unroll
      for (int u = 0; u < 4; ++u) load8<T>(x + (i + u * step) * 8, v[u]);
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          m = fmaxf(m, fabsf(v[u][k]));
          nan |= v[u][k] != v[u][k];
        }
    }
    for (; i < n8; i += step) {
      float v[8];
      load8<T>(x + i * 8, v);
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        m = fmaxf(m, fabsf(v[k]));
        nan |= v[k] != v[k];
      }
    }
    for (int64_t i = n8 * 8 + first; i < p.total; i += step) {
      const float v = Elem<T>::load(x + i);
      m = fmaxf(m, fabsf(v));
      nan |= v != v;
    }
  } else {
    for (int64_t i = first; i < p.total; i += step) {
      const float v = Elem<T>::load(x + x_offset(p, i));
      m = fmaxf(m, fabsf(v));
      nan |= v != v;
    }
  }
  // a NaN anywhere makes the result NaN, as torch's amax does; its bit
  // pattern is above every finite |x|, so the unsigned max carries it
  uint32_t bits = nan ? 0x7fc00000u : __float_as_uint(m);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1)
    bits = max(bits, static_cast<uint32_t>(__shfl_xor(static_cast<int>(bits), off)));
  // one atomic per block: the atomics of every wave on one address serialize in its L2 channel
  __shared__ uint32_t wave_max[4];
  if ((threadIdx.x & 63) == 0) wave_max[threadIdx.x >> 6] = bits;
  __syncthreads();
  if (threadIdx.x == 0)
    atomicMax(reinterpret_cast<unsigned int*>(p.amax),
              max(max(wave_max[0], wave_max[1]), max(wave_max[2], wave_max[3])));
}

__device__ __forceinline__ float quant_scale(const QuantParams& p) {
  if (p.scale_in) return *p.scale_in;
  const float a = *p.amax;
  return a == 0.0f ? 1.0f : a * p.headroom / 448.0f;
}

template <typename T>
__global__ __launch_bounds__(256) void quantize_kernel(QuantParams p) {
  const T* x = static_cast<const T*>(p.x);
  const float s = quant_scale(p);
  if (blockIdx.x == 0 && threadIdx.x == 0 && p.scale_out) *p.scale_out = s;
  if (p.dense) {
    const int64_t n8 = p.total / 8;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n8;
         i += static_cast<int64_t>(gridDim.x) * 256) {
      float v[8];
      load8<T>(x + i * 8, v);
      uint32_t w0 = cvt_pk_e4m3<false>(v[0] / s, v[1] / s, 0u);
      w0 = cvt_pk_e4m3<true>(v[2] / s, v[3] / s, w0);
      uint32_t w1 = cvt_pk_e4m3<false>(v[4] / s, v[5] / s, 0u);
      w1 = cvt_pk_e4m3<true>(v[6] / s, v[7] / s, w1);
      *reinterpret_cast<uint2*>(p.q + i * 8) = make_uint2(w0, w1);
    }
    for (int64_t i = n8 * 8 + static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < p.total;
         i += static_cast<int64_t>(gridDim.x) * 256)
      p.q[i] = f32_to_e4m3(Elem<T>::load(x + i) / s);
  } else {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < p.total;
         i += static_cast<int64_t>(gridDim.x) * 256)
      p.q[q_offset(p, i)] = f32_to_e4m3(Elem<T>::load(x + x_offset(p, i)) / s);
  }
}

// x and q use the same strides and those strides tile [0, total) exactly
// (some permutation of a packed [B, C, N] layout).
static bool dense_same_layout(const fovi_quantize_args* a) {
  for (int i = 0; i < 3; ++i)
    if (a->x_stride[i] != a->q_stride[i]) return false;
  const int64_t ext[3] = {a->batch, a->channels, a->points};
  int order[3] = {0, 1, 2};
  for (int i = 0; i < 3; ++i)
    for (int j = i + 1; j < 3; ++j)
      if (a->x_stride[order[j]] < a->x_stride[order[i]]) { const int t = order[i]; order[i] = order[j]; order[j] = t; }
  int64_t expect = 1;
  for (int i = 0; i < 3; ++i) {
    if (ext[order[i]] > 1 && a->x_stride[order[i]] != expect) return false;
    expect *= ext[order[i]];
  }
  return true;
}

}  // namespace fovi

using namespace fovi;

extern "C" int fovi_quantize_e4m3(const fovi_quantize_args* a, void* stream) {
  clear_error();
  if (!a || !a->x || !a->q) { set_error("fovi_quantize_e4m3: null argument"); return 1; }
  if (a->x_dtype != FOVI_F32 && a->x_dtype != FOVI_BF16) {
    set_error("fovi_quantize_e4m3: x_dtype must be F32 or BF16"); return 1;
  }
  if (a->batch < 0 || a->channels < 0 || a->points < 0) { set_error("fovi_quantize_e4m3: negative size"); return 1; }
  if (!a->scale_in && (!a->amax_work || !a->scale_out)) {
    set_error("fovi_quantize_e4m3: amax_work and scale_out are required without scale_in"); return 1;
  }
  if (!(a->headroom >= 1.0f) || a->headroom > 65536.0f) {
    set_error("fovi_quantize_e4m3: headroom must be in [1, 65536]"); return 1;
  }
  QuantParams p;
  p.x = a->x; p.B = a->batch; p.C = a->channels; p.N = a->points;
  p.xs0 = a->x_stride[0]; p.xs1 = a->x_stride[1]; p.xs2 = a->x_stride[2];
  p.q = a->q; p.qs0 = a->q_stride[0]; p.qs1 = a->q_stride[1]; p.qs2 = a->q_stride[2];
  p.headroom = a->headroom; p.scale_in = a->scale_in; p.scale_out = a->scale_out; p.amax = a->amax_work;
  p.total = p.B * p.C * p.N;
  const int esz = a->x_dtype == FOVI_F32 ? 4 : 2;
  p.dense = dense_same_layout(a) && reinterpret_cast<uintptr_t>(a->x) % (8 * esz) == 0 &&
            reinterpret_cast<uintptr_t>(a->q) % 8 == 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (p.total == 0) {
    if (!a->scale_in) {
      hipLaunchKernelGGL(clear_amax_kernel, dim3(1), dim3(1), 0, s, p.amax);
      hipLaunchKernelGGL((quantize_kernel<float>), dim3(1), dim3(256), 0, s, p);
    }
    return check_launch("fovi_quantize_e4m3");
  }
  const int64_t work = p.dense ? (p.total + 7) / 8 : p.total;
  const unsigned blocks = static_cast<unsigned>(std::min<int64_t>((work + 255) / 256, 256 * 16));
  if (!a->scale_in) {
    // at most 1024 blocks (four per CU), so 1024 atomics at most land on the one address
    const unsigned ablocks = std::min(blocks, 1024u);
    hipLaunchKernelGGL(clear_amax_kernel, dim3(1), dim3(1), 0, s, p.amax);
    if (a->x_dtype == FOVI_F32) hipLaunchKernelGGL((amax_kernel<float>), dim3(ablocks), dim3(256), 0, s, p);
    else hipLaunchKernelGGL((amax_kernel<uint16_t>), dim3(ablocks), dim3(256), 0, s, p);
  }
  if (a->x_dtype == FOVI_F32) hipLaunchKernelGGL((quantize_kernel<float>), dim3(blocks), dim3(256), 0, s, p);
  else hipLaunchKernelGGL((quantize_kernel<uint16_t>), dim3(blocks), dim3(256), 0, s, p);
  return check_launch("fovi_quantize_e4m3");
}
