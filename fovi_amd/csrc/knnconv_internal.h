// Internal declarations shared by the kNN-conv translation units.
#pragma once

#include "common.h"

namespace fovi {

// Few-channel slot sums (the fused kernel and the two-pass slot-sum kernel) run over a slot's
// neighbour list in groups of FC_GROUP: each group's fp32 sum in list order from +0, the
// groups' sums added in order (for up to FC_GROUP neighbours, the plain list order).
constexpr int FC_GROUP = 8;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct KnnParams {
  const void* x;
  int64_t B, C, Nin;
  int64_t xs0, xs1, xs2;
  int64_t Nout, K, V;
  const int32_t* slot_ptr;
  const int32_t* nbr;
  const void* w;
  int64_t Cout, Kpad;
  const float* bias;
  const float* w_scale;
  float x_scale;
  const float* x_scale_dev;
  void* y;
  int64_t ys0, ys1, ys2;
  const int32_t* tile_lo;
  const uint32_t* tile_ent;
  const uint16_t* tile_nbr;
  int max_span;
  const uint8_t* tile_coll;
  const int32_t* tile_coll_n;
  int zero_row;
  int relu;
  int w_c_slot;
  int w_layout;   // FOVI_W_ROWS or FOVI_W_MFMA
  const uint16_t* tile_src;
  const int32_t* tile_coll_off;
  const uint32_t* tile_cent;
  int coll_off_stride;
  int cent_stride;
  const uint32_t* tile_heavy;
  const uint16_t* tile_hlist;
  int heavy_stride;
  int hlist_stride;
  int wide_units;   // wide-layer tables in 16-byte units (1) or bytes (0)
};

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
typedef float f32x8 __attribute__((ext_vector_type(8)));

// Eight bf16 values (one 16-byte row part) widened to fp32.
__device__ __forceinline__ f32x8 unpack_bf16x8(u32x4 r) {
  f32x8 f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(r[i] << 16);
    f[2 * i + 1] = __uint_as_float(r[i] & 0xffff0000u);
  }
  return f;
}

// Two floats -> packed bf16 pair, round to nearest even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t cvt_pk_bf16(float a, float b) {
  const f32x2 v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2v));
}

// Output transform: optional ReLU fused into the store (the activation that
// follows the conv in the reference blocks when no norm sits between them).
__device__ __forceinline__ float epilogue(float v, int relu) { return relu ? fmaxf(v, 0.0f) : v; }

constexpr int V2_CC = 32;   // bf16 elements per 64-byte LDS row

// XOR pattern g(r) = (bit1(r) ^ bit3(r)) | bit2(r) << 1 keeps any 8 consecutive
// rows of one chunk in distinct 16-byte slots of a 128-byte window and any 16
// consecutive rows in distinct slots of a 256-byte window, so 16-byte reads
// are conflict-free whether the LDS serves 8 or 16 lanes per cycle.
__device__ __forceinline__ int swz32(int r, int q) {
  const int g = (((r >> 1) ^ (r >> 3)) & 1) | ((r >> 1) & 2);
  return r * V2_CC + ((q ^ g) << 3);
}

// Two floats -> two OCP fp8 e4m3 bytes (v_cvt_pk_fp8_f32, round to nearest
// even) written into byte pair `hi` (0: bytes 0-1, 1: bytes 2-3) of `old`.
// Finite inputs are clamped to +-448 first, so out-of-range values saturate;
// NaN stays NaN.
__device__ __forceinline__ float sat_e4m3(float f) {
  // v_med3_f32 clamps finite values and infinities (it returns a bound for NaN, so NaN is
  // selected back): three instructions, where fminf(fmaxf()) also canonicalises its input
  const float c = __builtin_amdgcn_fmed3f(f, -448.0f, 448.0f);
  return f == f ? c : f;
}
template <bool HI>
__device__ __forceinline__ uint32_t cvt_pk_e4m3(float a, float b, uint32_t old) {
  return static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(sat_e4m3(a), sat_e4m3(b), static_cast<int>(old), HI));
}
__device__ __forceinline__ uint8_t f32_to_e4m3(float f) {
  return static_cast<uint8_t>(cvt_pk_e4m3<false>(f, 0.0f, 0u) & 0xffu);
}

// Channel-tile width: the widest candidate that divides c_out and fits the
// LDS budget (no wasted MFMA columns); otherwise the widest that fits.
template <typename Fits>
static int pick_tile_n(int64_t cout, Fits fits) {
  const int cands[4] = {256, 192, 128, 64};
  for (int nt : cands)
    if (cout % nt == 0 && fits(nt)) return nt;
  for (int nt : cands) {
    if (nt > 64 && cout <= nt / 2) continue;
    if (fits(nt)) return nt;
  }
  return 0;
}

int launch_knnconv_fp8(const KnnParams& p, int out_t, hipStream_t s);
// The fused few-channel kernel (knnconv_fewc.hip): 1 if it took the call, 0 if its tables are
// absent or the tiling does not fit (the caller falls back).
int launch_knnconv_fewc(const KnnParams& p, const fovi_knnconv_args* a, int cp, hipStream_t s);
// 1 if launched, 0 if the view-major few-channel kernel does not take this call.
int launch_knnconv_fewc_vm(const KnnParams& p, const fovi_knnconv_args* a, int cp, hipStream_t s);
// 1 if the fragment-order kernel takes this call (see knnconv_v5.hip; f8:
// e4m3 input and weight), 0 if not.
int v5_applies(const KnnParams& p, int f8);
// The collision-tile count the fragment-order kernel uses for p's table sizes (4 when that tile
// layout fits 160 KB of LDS, else 3): the tables must have been built for it.
int v5_tiles_of(const KnnParams& p);
int launch_knnconv_bf16_v5(const KnnParams& p, int out_t, hipStream_t s);
int launch_knnconv_fp8_v5(const KnnParams& p, int out_t, hipStream_t s);

}  // namespace fovi
