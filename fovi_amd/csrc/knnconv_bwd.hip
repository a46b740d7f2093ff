// kNN-conv backward: the two gather kernels around its two GEMMs.
//
// The forward contracts y = W a with a[(b, n), (v, c)] the slot sums of the
// gathered inputs. Its gradients are dW = dy^T a (the slot sums again) and
// dx = the transpose of the gather applied to g = dy W: every input i sums
// the g entries of the (output, slot) pairs that read it. Both gathers are
// HBM-bound; the GEMMs between them are plain library GEMMs.
//  * fovi_knnconv_slotsum: thread = (row, slot, 16-byte channel group) for
//    channels-last inputs (one contiguous row load per neighbour, one
//    16-byte store), else (row, slot, channel).
//  * fovi_knnconv_bwd_x: thread = (batch row, input point, 16-byte channel
//    group of g) walking the input's inverse list (no atomics, a fixed sum
//    order), else (batch row, input point, channel).
#include "common.h"

namespace fovi {

struct SlotsumParams {
  const void* x;
  int64_t B, C, Nin, Nout, K, V;
  int64_t xs0, xs1, xs2;
  const int32_t* slot_ptr;
  const int32_t* nbr;
  void* a;
};

struct BwdXParams {
  const void* g;
  int64_t B, C, Nin, Nout, V;
  const int32_t* inv_ptr;
  const int32_t* inv;
  void* dx;
  int64_t ds0, ds1, ds2;
};

// 16 bytes of T as floats
template <typename T> struct Chunk16;
template <> struct Chunk16<float> {
  static constexpr int N = 4;
  static __device__ __forceinline__ void add(const float* p, float (&acc)[4]) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] += a[i];
  }
  static __device__ __forceinline__ void store(float* p, const float (&v)[4]) {
    *reinterpret_cast<f32x4*>(p) = f32x4{v[0], v[1], v[2], v[3]};
  }
};
template <> struct Chunk16<uint16_t> {
  static constexpr int N = 8;
  static __device__ __forceinline__ void add(const uint16_t* p, float (&acc)[8]) {
    const uint4 a = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc[2 * i] += __uint_as_float(w[i] << 16);
      acc[2 * i + 1] += __uint_as_float(w[i] & 0xffff0000u);
    }
  }
  static __device__ __forceinline__ void store(uint16_t* p, const float (&v)[8]) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = static_cast<uint32_t>(f32_to_bf16_bits(v[2 * i])) |
             (static_cast<uint32_t>(f32_to_bf16_bits(v[2 * i + 1])) << 16);
    *reinterpret_cast<uint4*>(p) = uint4{w[0], w[1], w[2], w[3]};
  }
};

// channels-last x and an output type of the same element size: 16-byte chunks
template <typename T>
__global__ __launch_bounds__(256) void slotsum_rows_kernel(SlotsumParams p, int64_t total) {
  constexpr int NV = Chunk16<T>::N;
  const int64_t G = p.C / NV;
  for (int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; t < total;
       t += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t g = t % G;
    const int64_t v = (t / G) % p.V;
    const int64_t m = t / (G * p.V);
    const int64_t b = m / p.Nout, n = m - b * p.Nout;
    const int32_t e = p.slot_ptr[n * p.V + v];
    const int cnt = e & 0xffff;
    const int32_t* nb = p.nbr + n * p.K + (e >> 16);
    const T* xb = static_cast<const T*>(p.x) + b * p.xs0 + g * NV;
    float acc[NV];
#pragma unroll
    for (int c = 0; c < NV; ++c) acc[c] = 0.0f;
    for (int j = 0; j < cnt; ++j) {
      const int64_t i = nb[j];
      if (i >= 0 && i < p.Nin) Chunk16<T>::add(xb + i * p.xs2, acc);
    }
    Chunk16<T>::store(static_cast<T*>(p.a) + m * p.V * p.C + v * p.C + g * NV, acc);
  }
}

template <typename InT, typename OutT>
__global__ __launch_bounds__(256) void slotsum_any_kernel(SlotsumParams p, int64_t total) {
  for (int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; t < total;
       t += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t c = t % p.C;
    const int64_t v = (t / p.C) % p.V;
    const int64_t m = t / (p.C * p.V);
    const int64_t b = m / p.Nout, n = m - b * p.Nout;
    const int32_t e = p.slot_ptr[n * p.V + v];
    const int cnt = e & 0xffff;
    const int32_t* nb = p.nbr + n * p.K + (e >> 16);
    const InT* xb = static_cast<const InT*>(p.x) + b * p.xs0 + c * p.xs1;
    float acc = 0.0f;
    for (int j = 0; j < cnt; ++j) {
      const int64_t i = nb[j];
      if (i >= 0 && i < p.Nin) acc += Elem<InT>::load(xb + i * p.xs2);
    }
    Elem<OutT>::store(static_cast<OutT*>(p.a) + m * p.V * p.C + v * p.C + c, acc);
  }
}

// g rows in 16-byte chunks (c_in a multiple of the chunk)
template <typename GT, typename DT>
__global__ __launch_bounds__(256) void bwd_x_rows_kernel(BwdXParams p, int64_t total, int vec_out) {
  constexpr int NV = Chunk16<GT>::N;
  const int64_t G = p.C / NV;
  for (int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; t < total;
       t += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t gi = t % G;
    const int64_t i = (t / G) % p.Nin;
    const int64_t b = t / (G * p.Nin);
    const GT* gb = static_cast<const GT*>(p.g) + b * p.Nout * p.V * p.C + gi * NV;
    float acc[NV];
#pragma unroll
    for (int c = 0; c < NV; ++c) acc[c] = 0.0f;
    for (int32_t q = p.inv_ptr[i], q1 = p.inv_ptr[i + 1]; q < q1; ++q) {
      const int64_t e = p.inv[q];                 // n * V + v: row n, column block v
      Chunk16<GT>::add(gb + (e / p.V) * p.V * p.C + (e % p.V) * p.C, acc);
    }
    DT* d = static_cast<DT*>(p.dx) + b * p.ds0 + i * p.ds2 + gi * NV * p.ds1;
    if constexpr (sizeof(DT) == sizeof(GT)) {
      if (vec_out) {
        Chunk16<DT>::store(d, acc);
        continue;
      }
    }
#pragma unroll
    for (int c = 0; c < NV; ++c) Elem<DT>::store(d + c * p.ds1, acc[c]);
  }
}

template <typename GT, typename DT>
__global__ __launch_bounds__(256) void bwd_x_any_kernel(BwdXParams p, int64_t total) {
  for (int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; t < total;
       t += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t c = t % p.C;
    const int64_t i = (t / p.C) % p.Nin;
    const int64_t b = t / (p.C * p.Nin);
    const GT* gb = static_cast<const GT*>(p.g) + b * p.Nout * p.V * p.C + c;
    float acc = 0.0f;
    for (int32_t q = p.inv_ptr[i], q1 = p.inv_ptr[i + 1]; q < q1; ++q) {
      const int64_t e = p.inv[q];
      acc += Elem<GT>::load(gb + (e / p.V) * p.V * p.C + (e % p.V) * p.C);
    }
    Elem<DT>::store(static_cast<DT*>(p.dx) + b * p.ds0 + c * p.ds1 + i * p.ds2, acc);
  }
}

static unsigned grid_for(int64_t total) {
  return static_cast<unsigned>(std::min<int64_t>((total + 255) / 256, 256 * 64));
}

template <typename InT, typename OutT>
static void launch_slotsum(const SlotsumParams& p, hipStream_t s) {
  constexpr int NV = Chunk16<InT>::N;
  const bool rows = sizeof(InT) == sizeof(OutT) && p.xs1 == 1 && p.C % NV == 0 && p.xs2 % NV == 0 &&
                    p.xs0 % NV == 0 && reinterpret_cast<uintptr_t>(p.x) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(p.a) % 16 == 0;
  if (rows) {
    const int64_t total = p.B * p.Nout * p.V * (p.C / NV);
    hipLaunchKernelGGL((slotsum_rows_kernel<InT>), dim3(grid_for(total)), dim3(256), 0, s, p, total);
  } else {
    const int64_t total = p.B * p.Nout * p.V * p.C;
    hipLaunchKernelGGL((slotsum_any_kernel<InT, OutT>), dim3(grid_for(total)), dim3(256), 0, s, p, total);
  }
}

template <typename GT, typename DT>
static void launch_bwd_x(const BwdXParams& p, hipStream_t s) {
  constexpr int NV = Chunk16<GT>::N;
  if (p.C % NV == 0 && reinterpret_cast<uintptr_t>(p.g) % 16 == 0) {
    const int vec_out = sizeof(DT) == sizeof(GT) && p.ds1 == 1 && p.ds2 % NV == 0 && p.ds0 % NV == 0 &&
                        reinterpret_cast<uintptr_t>(p.dx) % 16 == 0;
    const int64_t total = p.B * p.Nin * (p.C / NV);
    hipLaunchKernelGGL((bwd_x_rows_kernel<GT, DT>), dim3(grid_for(total)), dim3(256), 0, s, p, total, vec_out);
  } else {
    const int64_t total = p.B * p.Nin * p.C;
    hipLaunchKernelGGL((bwd_x_any_kernel<GT, DT>), dim3(grid_for(total)), dim3(256), 0, s, p, total);
  }
}

static bool ok_dtype(int d) { return d == FOVI_F32 || d == FOVI_BF16; }

}  // namespace fovi

extern "C" int fovi_knnconv_slotsum(const fovi_knnconv_slotsum_args* a, void* stream) {
  using namespace fovi;
  clear_error();
  if (!a || !a->x || !a->slot_ptr || !a->nbr_sorted || !a->a) {
    set_error("fovi_knnconv_slotsum: null pointer"); return 1;
  }
  if (!ok_dtype(a->x_dtype) || !ok_dtype(a->a_dtype)) {
    set_error("fovi_knnconv_slotsum: x and a must be F32 or BF16"); return 1;
  }
  if (a->batch < 0 || a->c_in < 1 || a->n_in < 0 || a->n_out < 0 || a->k < 1 || a->n_ref < 1) {
    set_error("fovi_knnconv_slotsum: bad sizes"); return 1;
  }
  // slot_ptr entries are begin << 16 | count in an int32 decoded with a signed shift: begin < 2^15
  if (a->k > 32767) { set_error("fovi_knnconv_slotsum: k=%lld exceeds 32767", (long long)a->k); return 1; }
  if (a->batch * a->n_out == 0) return 0;
  SlotsumParams p;
  p.x = a->x; p.B = a->batch; p.C = a->c_in; p.Nin = a->n_in; p.Nout = a->n_out; p.K = a->k; p.V = a->n_ref;
  p.xs0 = a->x_stride[0]; p.xs1 = a->x_stride[1]; p.xs2 = a->x_stride[2];
  p.slot_ptr = a->slot_ptr; p.nbr = a->nbr_sorted; p.a = a->a;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (a->x_dtype == FOVI_F32) {
    if (a->a_dtype == FOVI_F32) launch_slotsum<float, float>(p, s);
    else launch_slotsum<float, uint16_t>(p, s);
  } else {
    if (a->a_dtype == FOVI_F32) launch_slotsum<uint16_t, float>(p, s);
    else launch_slotsum<uint16_t, uint16_t>(p, s);
  }
  return check_launch("fovi_knnconv_slotsum");
}

extern "C" int fovi_knnconv_bwd_x(const fovi_knnconv_bwd_x_args* a, void* stream) {
  using namespace fovi;
  clear_error();
  if (!a || !a->g || !a->inv_ptr || !a->inv || !a->dx) { set_error("fovi_knnconv_bwd_x: null pointer"); return 1; }
  if (!ok_dtype(a->g_dtype) || !ok_dtype(a->dx_dtype)) {
    set_error("fovi_knnconv_bwd_x: g and dx must be F32 or BF16"); return 1;
  }
  if (a->batch < 0 || a->c_in < 1 || a->n_in < 0 || a->n_out < 0 || a->n_ref < 1) {
    set_error("fovi_knnconv_bwd_x: bad sizes"); return 1;
  }
  if (a->batch * a->n_in == 0) return 0;
  BwdXParams p;
  p.g = a->g; p.B = a->batch; p.C = a->c_in; p.Nin = a->n_in; p.Nout = a->n_out; p.V = a->n_ref;
  p.inv_ptr = a->inv_ptr; p.inv = a->inv; p.dx = a->dx;
  p.ds0 = a->dx_stride[0]; p.ds1 = a->dx_stride[1]; p.ds2 = a->dx_stride[2];
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (a->g_dtype == FOVI_F32) {
    if (a->dx_dtype == FOVI_F32) launch_bwd_x<float, float>(p, s);
    else launch_bwd_x<float, uint16_t>(p, s);
  } else {
    if (a->dx_dtype == FOVI_F32) launch_bwd_x<uint16_t, float>(p, s);
    else launch_bwd_x<uint16_t, uint16_t>(p, s);
  }
  return check_launch("fovi_knnconv_bwd_x");
}
