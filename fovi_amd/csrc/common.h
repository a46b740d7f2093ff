// Internal helpers shared by the gfx950 kernels of libfovi_hip.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>
#include <string>

#include "fovi_hip.h"

namespace fovi {

// Thread-local message for fovi_last_error().
void set_error(const char* fmt, ...);
void clear_error();

// Returns 0, or records the HIP error of the last launch and returns 1.
int check_launch(const char* what);

// hipFuncSetAttribute(MaxDynamicSharedMemorySize) for `kernel` on the current device, called
// only when `bytes` exceeds what an earlier call reserved (a runtime call per launch costs host
// time that small layers notice).
hipError_t reserve_dynamic_lds(const void* kernel, size_t bytes);

// Records (thread-local) the kernel path fovi_knnconv_fwd took; `name` must be
// a string literal. Read back by fovi_knnconv_last_path().
void note_path(const char* name);

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// float -> bf16 bits, round to nearest even (NaN stays NaN): one
// v_cvt_pk_bf16_f32 on gfx950.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

template <typename T> struct Elem;
template <> struct Elem<float> {
  static __device__ __forceinline__ float load(const float* p) { return *p; }
  static __device__ __forceinline__ void store(float* p, float v) { *p = v; }
};
template <> struct Elem<uint16_t> {  // bf16 stored as raw bits
  static __device__ __forceinline__ float load(const uint16_t* p) { return bf16_bits_to_f32(*p); }
  static __device__ __forceinline__ void store(uint16_t* p, float v) { *p = f32_to_bf16_bits(v); }
};

// Blocks are dispatched round-robin over the 8 XCDs of an MI355X; this maps
// the hardware block id to a logical tile id so that each XCD (and its L2)
// works on one contiguous range of tiles. `padded` = 8 * ceil(total / 8).
__device__ __forceinline__ int64_t xcd_tile(int64_t bid, int64_t padded) {
  const int64_t per = padded >> 3;
  return (bid & 7) * per + (bid >> 3);
}

}  // namespace fovi
