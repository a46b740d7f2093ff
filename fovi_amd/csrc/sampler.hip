// Foveated sampler: fixation transform + grid-sample, one launch for all views.
//
// One thread per (view, sensor point); channels are looped inside the thread
// so the fixation transform and tap coordinates are computed once per point.
// Consecutive threads are consecutive sensor points (consecutive angles on a
// log-polar ring), so output stores along the point axis are coalesced and
// neighbouring threads read neighbouring pixels.
//
// Arithmetic follows the reference bit for bit where it is defined:
//  * fixation transform (fovi/sensing/coords.py:624-640): fp32
//    x*half + c*W, then 2*x/W - 1, each op rounded (built with
//    -ffp-contract=off, so no fused multiply-add);
//  * grid_sample (align_corners=False) in the rounding of the CPU kernel of
//    torch.nn.functional.grid_sample, which is the oracle: unnormalisation as
//    one fused multiply-add fma(g + 1, size/2, -0.5); 'border' clips to
//    [0, size-1]; 'nearest' rounds half to even; bilinear weights
//    (1-dy)(1-dx), (1-dy)dx, dy(1-dx), dy*dx from floor() and the fractional
//    parts, blended as the chain fma(se, fma(sw, fma(ne, nw*v_nw)));
//    out-of-image taps contribute zero. This matches that kernel bit for bit
//    (checked on 20000 random points at a non-power-of-two size).
#include <type_traits>

#include "common.h"

namespace fovi {

struct SamplerParams {
  const void* img;
  int64_t n_img, C, H, W;
  int64_t is0, is1, is2, is3;
  const float* grid;
  int64_t N;
  const float* fix_loc;
  const double* fix_half;
  int wide;
  const int32_t* view_image;
  void* out;
  int64_t os0, os1, os2;
  float* grid_out;
  int64_t ring_len;
};

// Two horizontally adjacent pixels (cx, cx + 1) of one row with one load.
// Only used when 0 <= cx and the loaded words stay inside the row (checked
// by the caller): bf16 reads the 4-byte-aligned words covering cx and cx + 1
// (8 bytes at the even pixel at or below cx), fp32 reads the 8 bytes at cx.
template <typename T> struct PixelPair;
template <> struct PixelPair<uint16_t> {
  typedef uint32_t u32x2a4 __attribute__((ext_vector_type(2), aligned(4)));
  // row is 4-byte aligned (checked on the host); pairs need cx & ~1 + 4 <= W
  template <typename Off>
  static __device__ __forceinline__ bool fits(Off cx, Off W) { return cx >= 0 && (cx & ~Off(1)) + 4 <= W; }
  template <typename Off>
  static __device__ __forceinline__ void load(const uint16_t* row, Off cx, float& a, float& b) {
    const u32x2a4 w = *reinterpret_cast<const u32x2a4*>(row + (cx & ~Off(1)));
    const uint32_t lo = (cx & 1) ? (w[0] >> 16) | (w[1] << 16) : w[0];
    a = __uint_as_float(lo << 16);
    b = __uint_as_float(lo & 0xffff0000u);
  }
};
template <> struct PixelPair<float> {
  typedef float f32x2a4 __attribute__((ext_vector_type(2), aligned(4)));
  template <typename Off>
  static __device__ __forceinline__ bool fits(Off cx, Off W) { return cx >= 0 && cx + 1 < W; }
  template <typename Off>
  static __device__ __forceinline__ void load(const float* row, Off cx, float& a, float& b) {
    const f32x2a4 w = *reinterpret_cast<const f32x2a4*>(row + cx);
    a = w[0];
    b = w[1];
  }
};

// Sampling set-up of one (view, sensor point): fixation transform, tap
// coordinates and weights; value() then samples one channel plane.
template <typename InT, int MODE, int PAD, bool PAIRS, typename Off = int64_t>
struct Taps {
  bool inb, y0, y1, pair;
  bool b_nw, b_ne, b_sw, b_se;
  Off off, o_nw, o_ne, o_sw, o_se;
  Off cx, px;
  float w_nw, w_ne, w_sw, w_se;

  __device__ __forceinline__ Taps(const SamplerParams& p, int64_t v, int64_t pt) {
    // (v, pt) index the small per-view / per-point tables
    const float W = static_cast<float>(p.W);
    const float H = static_cast<float>(p.H);
    const float g0 = p.grid[2 * pt];
    const float g1 = p.grid[2 * pt + 1];
    const double half_h = p.fix_half[2 * v];
    const double half_w = p.fix_half[2 * v + 1];
    float x, y;
    if (p.wide) {
      x = static_cast<float>(static_cast<double>(g0) * half_w);
      y = static_cast<float>(static_cast<double>(g1) * half_h);
    } else {
      x = g0 * static_cast<float>(half_w);
      y = g1 * static_cast<float>(half_h);
    }
    const float centre_h = p.fix_loc[2 * v] * H;
    const float centre_w = p.fix_loc[2 * v + 1] * W;
    x = x + centre_w;
    y = y + centre_h;
    const float gx = (2.0f * x) / W - 1.0f;
    const float gy = (2.0f * y) / H - 1.0f;
    if (p.grid_out) {
      p.grid_out[(v * p.N + pt) * 2] = gx;
      p.grid_out[(v * p.N + pt) * 2 + 1] = gy;
    }
    float ix = __builtin_fmaf(gx + 1.0f, W * 0.5f, -0.5f);
    float iy = __builtin_fmaf(gy + 1.0f, H * 0.5f, -0.5f);
    if (PAD == FOVI_PAD_BORDER) {
      ix = fminf(fmaxf(ix, 0.0f), W - 1.0f);
      iy = fminf(fmaxf(iy, 0.0f), H - 1.0f);
    }
    // Every bounds decision below is a float comparison (false for NaN), and
    // coordinates are clamped to [-1, size] before any integer conversion, so
    // infinite, NaN or huge coordinates select no tap and convert defined
    // values (they sample zeros, as the reference's grid_sample does).
    if (MODE == FOVI_NEAREST) {
      const float rx = __builtin_rintf(ix);
      const float ry = __builtin_rintf(iy);
      inb = rx >= 0.0f && rx < W && ry >= 0.0f && ry < H;
      const Off ox = static_cast<Off>(fminf(fmaxf(rx, 0.0f), W - 1.0f));
      const Off oy = static_cast<Off>(fminf(fmaxf(ry, 0.0f), H - 1.0f));
      off = inb ? oy * static_cast<Off>(p.is2) + ox * static_cast<Off>(p.is3) : 0;
      px = ox;
      return;
    }
    const float fx = floorf(ix);
    const float fy = floorf(iy);
    const float we = ix - fx;          // weight of the east column
    const float ww = 1.0f - we;
    const float ws = iy - fy;          // weight of the south row
    const float wn = 1.0f - ws;
    w_nw = wn * ww; w_ne = wn * we; w_sw = ws * ww; w_se = ws * we;
    const bool x0 = fx >= 0.0f && fx < W, x1 = fx + 1.0f >= 0.0f && fx + 1.0f < W;
    y0 = fy >= 0.0f && fy < H;
    y1 = fy + 1.0f >= 0.0f && fy + 1.0f < H;
    cx = static_cast<Off>(fminf(fmaxf(fx, -1.0f), W));
    const Off cy = static_cast<Off>(fminf(fmaxf(fy, -1.0f), H));
    const Off is2 = static_cast<Off>(p.is2), is3 = static_cast<Off>(p.is3);
    // the pair path needs both columns inside the image (float test) and, for bf16, the
    // 8-byte word pair inside the row (integer test on the clamped column)
    pair = PAIRS && x0 && x1 && PixelPair<InT>::fits(cx, static_cast<Off>(p.W));
    if (pair) {  // both columns inside the image; rows checked per row
      o_nw = y0 ? cy * is2 : 0;
      o_sw = y1 ? (cy + 1) * is2 : 0;
      return;
    }
    b_nw = y0 && x0; b_ne = y0 && x1; b_sw = y1 && x0; b_se = y1 && x1;
    o_nw = b_nw ? cy * is2 + cx * is3 : 0;
    o_ne = b_ne ? cy * is2 + (cx + 1) * is3 : 0;
    o_sw = b_sw ? (cy + 1) * is2 + cx * is3 : 0;
    o_se = b_se ? (cy + 1) * is2 + (cx + 1) * is3 : 0;
  }

  __device__ __forceinline__ float value(const InT* s) const {
    if (MODE == FOVI_NEAREST) return inb ? Elem<InT>::load(s + off) : 0.0f;
    float v_nw = 0.0f, v_ne = 0.0f, v_sw = 0.0f, v_se = 0.0f;
    if (pair) {
      if (y0) PixelPair<InT>::load(s + o_nw, cx, v_nw, v_ne);
      if (y1) PixelPair<InT>::load(s + o_sw, cx, v_sw, v_se);
    } else {
      v_nw = b_nw ? Elem<InT>::load(s + o_nw) : 0.0f;
      v_ne = b_ne ? Elem<InT>::load(s + o_ne) : 0.0f;
      v_sw = b_sw ? Elem<InT>::load(s + o_sw) : 0.0f;
      v_se = b_se ? Elem<InT>::load(s + o_se) : 0.0f;
    }
    return __builtin_fmaf(v_se, w_se, __builtin_fmaf(v_sw, w_sw, __builtin_fmaf(v_ne, w_ne, v_nw * w_nw)));
  }

  // Channels-last bf16 images (channel stride 1, pixel stride NCH = 3 or 4, image base
  // 4-byte aligned, and for NCH = 4 even image and row strides, so every pixel of a 4-channel
  // image starts at an even element): the NCH channels of the tap at element offset e with
  // one 8-byte load of the 4-byte-aligned words at or below it. Those 8 bytes hold the pixel
  // (NCH <= 4 - (e & 1)) and stay inside the row unless the pixel is the row's last and
  // starts at an even element (then NCH = 3 reads two bytes of the next pixel): there the
  // channels are loaded one by one. One load instead of NCH cuts the distinct cache lines a
  // wave's gather touches by NCH.
  template <int NCH>
  __device__ __forceinline__ static void pixel_cl(const uint16_t* s, Off e, Off x, Off W, float (&v)[4]) {
    if (NCH == 4 || (e & 1) || x + 1 < W) {
      typedef uint32_t u32x2a4 __attribute__((ext_vector_type(2), aligned(4)));
      const u32x2a4 w = *reinterpret_cast<const u32x2a4*>(s + (e & ~Off(1)));
      const uint32_t h[4] = {w[0] << 16, w[0] & 0xffff0000u, w[1] << 16, w[1] & 0xffff0000u};
      const int o = static_cast<int>(e & 1);
#pragma unroll
      for (int c = 0; c < NCH; ++c) v[c] = __uint_as_float(h[o + c]);
    } else {
#pragma unroll
      for (int c = 0; c < NCH; ++c) v[c] = bf16_bits_to_f32(s[e + c]);
    }
  }

  // The two horizontally adjacent pixels at e and e + NCH of a channels-last bf16 image with
  // one 16-byte load of the 4-byte-aligned words at or below e; the caller checks that the
  // load stays in the row (NCH = 4, or a third pixel follows).
  template <int NCH>
  __device__ __forceinline__ static void pair_cl(const uint16_t* s, Off e, float (&a)[4], float (&b)[4]) {
    typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));
    const u32x4a4 w = *reinterpret_cast<const u32x4a4*>(s + (e & ~Off(1)));
    const uint32_t h[8] = {w[0] << 16, w[0] & 0xffff0000u, w[1] << 16, w[1] & 0xffff0000u,
                           w[2] << 16, w[2] & 0xffff0000u, w[3] << 16, w[3] & 0xffff0000u};
    const int o = static_cast<int>(e & 1);
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      a[c] = __uint_as_float(h[o + c]);
      b[c] = __uint_as_float(h[o + NCH + c]);
    }
  }

  // Every channel of the sample from a channels-last bf16 image (see pixel_cl), blended in
  // the order value() blends one channel plane: the same results bit for bit.
  template <int NCH>
  __device__ __forceinline__ void values_cl(const uint16_t* s, Off W, float (&out)[4]) const {
    if (MODE == FOVI_NEAREST) {
      if (inb) pixel_cl<NCH>(s, off, px, W, out);
      else
#pragma unroll
        for (int c = 0; c < NCH; ++c) out[c] = 0.0f;
      return;
    }
    float nw[4] = {}, ne[4] = {}, sw[4] = {}, se[4] = {};
    const bool row2 = NCH == 4 || cx + 2 < W;   // a row's two taps with one load
    if (b_nw && b_ne && row2) {
      pair_cl<NCH>(s, o_nw, nw, ne);
    } else {
      if (b_nw) pixel_cl<NCH>(s, o_nw, cx, W, nw);
      if (b_ne) pixel_cl<NCH>(s, o_ne, cx + 1, W, ne);
    }
    if (b_sw && b_se && row2) {
      pair_cl<NCH>(s, o_sw, sw, se);
    } else {
      if (b_sw) pixel_cl<NCH>(s, o_sw, cx, W, sw);
      if (b_se) pixel_cl<NCH>(s, o_se, cx + 1, W, se);
    }
#pragma unroll
    for (int c = 0; c < NCH; ++c)
      out[c] = __builtin_fmaf(se[c], w_se, __builtin_fmaf(sw[c], w_sw, __builtin_fmaf(ne[c], w_ne, nw[c] * w_nw)));
  }
};

// Linear path: one thread per (view, sensor point). Blocks are numbered
// view-major (blocks_per_view blocks of 256 points per view) and mapped
// XCD-aware: each of the 8 XCDs takes one contiguous range of views, so the
// views of one image (adjacent when views are ordered image by image, as the
// fused fixation loop orders them) are sampled by one XCD and share its L2:
// at 128-byte line granularity the fixation views of an image together touch
// most of the image, which is then fetched from HBM about once.
// PAIRS: image rows are unit-stride and 4-byte aligned, so the two pixels of
// a bilinear row are fetched with one load.
template <typename InT, typename OutT, int MODE, int PAD, bool PAIRS>
__global__ __launch_bounds__(256) void sampler_kernel(SamplerParams p, int64_t blocks_per_view, int64_t total_blocks,
                                                      int64_t padded_blocks) {
  const int64_t lb = xcd_tile(blockIdx.x, padded_blocks);
  if (lb >= total_blocks) return;
  const int64_t v = lb / blocks_per_view;
  const int64_t pt = (lb - v * blocks_per_view) * 256 + threadIdx.x;
  if (pt >= p.N) return;
  const Taps<InT, MODE, PAD, PAIRS> t(p, v, pt);
  OutT* out = static_cast<OutT*>(p.out) + v * p.os0 + pt * p.os2;
  const int64_t img = p.view_image ? static_cast<int64_t>(p.view_image[v]) : v;
  if (img < 0 || img >= p.n_img) {
    for (int64_t c = 0; c < p.C; ++c) Elem<OutT>::store(out + c * p.os1, 0.0f);
    return;
  }
  const InT* src = static_cast<const InT*>(p.img) + img * p.is0;
  for (int64_t c = 0; c < p.C; ++c) Elem<OutT>::store(out + c * p.os1, t.value(src + c * p.is1));
}

// 16 bytes of consecutive samples from LDS to one unit-stride, 16-byte aligned store.
template <typename T> struct Vec16Store;
template <> struct Vec16Store<float> {
  static __device__ __forceinline__ void store(float* p, const float* v) {
    *reinterpret_cast<f32x4*>(p) = f32x4{v[0], v[1], v[2], v[3]};
  }
};
template <> struct Vec16Store<uint16_t> {
  static __device__ __forceinline__ void store(uint16_t* p, const float* v) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = static_cast<uint32_t>(f32_to_bf16_bits(v[2 * i])) |
             (static_cast<uint32_t>(f32_to_bf16_bits(v[2 * i + 1])) << 16);
    *reinterpret_cast<uint4*>(p) = uint4{w[0], w[1], w[2], w[3]};
  }
};

// Blocked path for grids of whole rings (point = ring * ring_len + angle,
// ring_len % 32 == 0, rings % 8 == 0) and at most 4 channels (NC, or 0 for a
// run-time count <= 4). A block takes 8 rings x 32 angles of one view, each
// wave 8 rings x 8 angles: on the log-polar sensor these points are
// neighbours in the image, so the lanes of one gather share cache lines
// (about 1.75x fewer distinct lines per load than a wave along one ring). The
// block's samples are staged in LDS and written back along the rings (64-byte
// runs per channel plane, 16 bytes per lane when the planes are unit-stride
// and aligned). The grid is only a processing order: every point
// of the view is sampled exactly once whatever the geometry, so results do
// not depend on it. Block indices and in-image / in-view offsets are 32-bit
// (the host checks the extents).
// CL = 3 or 4: channels-last bf16 image with NC = CL channels, each tap's channels read with
// one load (Taps::values_cl); 0: channel planes, one load per channel.
//
// The point block a workgroup samples: the blocks of view (or view group) v rotated by 13 v, so
// that the workgroups running together sample different regions of their images. Without it,
// views fixating the same place (C2's centre fixations) have every running workgroup read the
// same offsets of different images, which crowds a few memory channels (C2 view-major sampler
// 47 -> 34 us; C4 nearest / bilinear 87 / 145 -> 86 / 140 us).
__device__ __forceinline__ uint32_t rotated_block(uint32_t b, uint32_t v, uint32_t blocks_per_view) {
  return (b + (v % blocks_per_view) * 13u) % blocks_per_view;
}

template <typename InT, typename OutT, int MODE, int PAD, bool PAIRS, int NC, int CL = 0>
__global__ __launch_bounds__(256) void sampler_rings_kernel(SamplerParams p, uint32_t blocks_per_view,
                                                            uint32_t total_blocks, uint32_t padded_blocks,
                                                            int vec_out) {
  __shared__ float st[4][256];
  const uint32_t per = padded_blocks >> 3;
  const uint32_t lb = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
  if (lb >= total_blocks) return;
  const uint32_t v = lb / blocks_per_view;
  const uint32_t b = rotated_block(lb - v * blocks_per_view, v, blocks_per_view);
  const uint32_t ring_len = static_cast<uint32_t>(p.ring_len);
  const uint32_t segs = ring_len >> 5;              // 32-angle segments per ring
  const uint32_t band = b / segs;
  const uint32_t ring0 = band * 8, ang0 = (b - band * segs) * 32;
  const int tid = threadIdx.x;
  const uint32_t r_in = (tid & 63) >> 3, a_in = (tid >> 6) * 8 + (tid & 7);
  const uint32_t pt = (ring0 + r_in) * ring_len + ang0 + a_in;
  const int C = NC > 0 ? NC : static_cast<int>(p.C);
  const int64_t img = p.view_image ? static_cast<int64_t>(p.view_image[v]) : static_cast<int64_t>(v);
  const Taps<InT, MODE, PAD, PAIRS, int32_t> t(p, v, pt);
  float val[4];
  if (img >= 0 && img < p.n_img) {
    const InT* src = static_cast<const InT*>(p.img) + img * p.is0;
    if constexpr (CL > 0) {
#pragma unroll
      for (int c = 0; c < 4; ++c) val[c] = 0.0f;
      t.template values_cl<CL>(src, static_cast<int32_t>(p.W), val);
    } else {
      const int32_t is1 = static_cast<int32_t>(p.is1);
#pragma unroll
      for (int c = 0; c < 4; ++c) val[c] = c < C ? t.value(src + c * is1) : 0.0f;
    }
  } else {
#pragma unroll
    for (int c = 0; c < 4; ++c) val[c] = 0.0f;
  }
  const int li = r_in * 32 + a_in;
#pragma unroll
  for (int c = 0; c < 4; ++c)
    if (c < C) st[c][li] = val[c];
  __syncthreads();
  OutT* out = static_cast<OutT*>(p.out) + static_cast<int64_t>(v) * p.os0;
  if (vec_out) {
    // 16-byte runs: a ring's 32 angles are contiguous in a channel plane, so the block's
    // samples leave in 8 rings x C x (32 / VPL) pieces of VPL values, one store per lane
    constexpr int VPL = 16 / sizeof(OutT);
    constexpr int PPR = 32 / VPL;                   // pieces per ring
    if (tid < 8 * PPR * C) {
      const int c = tid / (8 * PPR), r = (tid / PPR) % 8, part = tid % PPR;
      const float* sv = &st[c][r * 32 + part * VPL];
      const int32_t o = static_cast<int32_t>((ring0 + r) * ring_len + ang0 + part * VPL) +
                        c * static_cast<int32_t>(p.os1);
      Vec16Store<OutT>::store(out + o, sv);
    }
    return;
  }
  const uint32_t pw = (ring0 + (tid >> 5)) * ring_len + ang0 + (tid & 31);
  const int32_t o = static_cast<int32_t>(pw) * static_cast<int32_t>(p.os2);
#pragma unroll
  for (int c = 0; c < 4; ++c)
    if (c < C) Elem<OutT>::store(out + o + c * static_cast<int32_t>(p.os1), st[c][tid]);
}

// View-major output (bf16 rows of 4 elements holding C <= 4 channels, the rows of one point for
// all views adjacent: element (v, c, n) at n * os2 + v * 4 + c), the input layout of the
// view-major few-channel kNN-conv kernel. A block samples the blocked path's 256 points (8
// rings x 32 angles) for VM_VIEWS consecutive views with the blocked path's tap code (same
// values bit for bit), one view after another, staging each sample's channels in LDS; it then
// writes each point's views as one run of VM_VIEWS rows, one row per lane. Only the C channels
// of a row are written. More views per block write longer runs but leave fewer blocks: 16
// views when that still gives 2048 blocks, else 4 (C4 nearest, 512 views of 16384 points,
// images alternating between two sets: 16 views 123 us, 8 128, 4 141; warm images 82, 92,
// 99; C2 bilinear, 256 views of 4096 points: 4 views 30 us, 8 32; warm 16 views 41).
// Nearest sampling from channel planes, in a block of VM_VIEWS valid views, takes the views
// eight at a time with branch-free code: every tap is loaded (an out-of-image tap or view
// reads the image's first element and is replaced by zero), so the eight views' loads are in
// flight together instead of one view's (C4: 119 -> 97 us, the point-major kernel's 94).
constexpr int VM_RS = 34;                      // LDS entries per ring of a view (32 + 2: banks)
constexpr int VM_VS = 8 * VM_RS + 2;           // LDS entries per view

template <typename InT, int MODE, int PAD, bool PAIRS, int NC, int CL = 0, int VM_VIEWS = 16>
__global__ __launch_bounds__(256) void sampler_rings_vm_kernel(SamplerParams p, uint32_t blocks_per_view,
                                                               uint32_t n_views, uint32_t total_blocks,
                                                               uint32_t padded_blocks) {
  typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));
  __shared__ u32x2v st[VM_VIEWS * VM_VS];
  const uint32_t per = padded_blocks >> 3;
  const uint32_t lb = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
  if (lb >= total_blocks) return;
  const uint32_t vg = lb / blocks_per_view;
  const uint32_t b = rotated_block(lb - vg * blocks_per_view, vg, blocks_per_view);
  const uint32_t ring_len = static_cast<uint32_t>(p.ring_len);
  const uint32_t segs = ring_len >> 5;
  const uint32_t band = b / segs;
  const uint32_t ring0 = band * 8, ang0 = (b - band * segs) * 32;
  const int tid = threadIdx.x;
  const uint32_t r_in = (tid & 63) >> 3, a_in = (tid >> 6) * 8 + (tid & 7);
  const uint32_t pt = (ring0 + r_in) * ring_len + ang0 + a_in;
  const int C = NC > 0 ? NC : static_cast<int>(p.C);
  auto put = [&](int vi, const float (&val)[4]) {
    st[vi * VM_VS + r_in * VM_RS + a_in] =
        u32x2v{static_cast<uint32_t>(f32_to_bf16_bits(val[0])) | (static_cast<uint32_t>(f32_to_bf16_bits(val[1])) << 16),
               static_cast<uint32_t>(f32_to_bf16_bits(val[2])) | (static_cast<uint32_t>(f32_to_bf16_bits(val[3])) << 16)};
  };
  bool batched = false;
  if constexpr (MODE == FOVI_NEAREST && CL == 0 && VM_VIEWS % 8 == 0) {
    if (vg * VM_VIEWS + VM_VIEWS <= n_views && !p.grid_out && p.n_img > 0) {
      batched = true;
      const int32_t is1 = static_cast<int32_t>(p.is1);
#pragma unroll
      for (int v0 = 0; v0 < VM_VIEWS; v0 += 8) {
        float val[8][4];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const uint32_t v = vg * VM_VIEWS + v0 + j;
          const int64_t img = p.view_image ? static_cast<int64_t>(p.view_image[v]) : static_cast<int64_t>(v);
          const bool iok = img >= 0 && img < p.n_img;
          const Taps<InT, MODE, PAD, PAIRS, int32_t> t(p, v, pt);
          const InT* src = static_cast<const InT*>(p.img) + (iok ? img : 0) * p.is0;
          const bool ok = iok && t.inb;     // t.off is 0 outside the image
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const float x = c < C ? Elem<InT>::load(src + c * is1 + t.off) : 0.0f;
            val[j][c] = ok && c < C ? x : 0.0f;
          }
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) put(v0 + j, val[j]);
      }
    }
  }
  if (!batched)
  for (int vi = 0; vi < VM_VIEWS; ++vi) {
    const uint32_t v = vg * VM_VIEWS + vi;
    float val[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (v < n_views) {
      const int64_t img = p.view_image ? static_cast<int64_t>(p.view_image[v]) : static_cast<int64_t>(v);
      const Taps<InT, MODE, PAD, PAIRS, int32_t> t(p, v, pt);
      if (img >= 0 && img < p.n_img) {
        const InT* src = static_cast<const InT*>(p.img) + img * p.is0;
        if constexpr (CL > 0) {
          t.template values_cl<CL>(src, static_cast<int32_t>(p.W), val);
        } else {
          const int32_t is1 = static_cast<int32_t>(p.is1);
#pragma unroll
          for (int c = 0; c < 4; ++c) val[c] = c < C ? t.value(src + c * is1) : 0.0f;
        }
      }
    }
#pragma unroll
    for (int c = 0; c < 4; ++c)
      if (c >= C) val[c] = 0.0f;
    put(vi, val);
  }
  __syncthreads();
  uint16_t* out = static_cast<uint16_t*>(p.out);
#pragma unroll
  for (int k = 0; k < VM_VIEWS; ++k) {
    const int q = k * 256 + tid;
    const int ln = q / VM_VIEWS, vi = q % VM_VIEWS;      // point of the block, view of the group
    const uint32_t v = vg * VM_VIEWS + vi;
    if (v < n_views) {
      const uint32_t point = (ring0 + (ln >> 5)) * ring_len + ang0 + (ln & 31);
      uint16_t* o = out + static_cast<int64_t>(point) * p.os2 + static_cast<int64_t>(v) * 4;
      const u32x2v w = st[vi * VM_VS + (ln >> 5) * VM_RS + (ln & 31)];
      // exactly channels 0 .. C - 1 of the row (a fourth element outside the view is not written)
      if (C == 4) {
        *reinterpret_cast<u32x2v*>(o) = w;
      } else {
        if (C >= 2) *reinterpret_cast<uint32_t*>(o) = w[0];
        else o[0] = static_cast<uint16_t>(w[0]);
        if (C == 3) o[2] = static_cast<uint16_t>(w[1]);
      }
    }
  }
}

// Whether the blocked path applies (see sampler_rings_kernel).
static bool rings_path(const SamplerParams& p, int64_t n_views) {
  if (!(p.ring_len > 0 && p.ring_len % 32 == 0 && p.N % (8 * p.ring_len) == 0 && p.C <= 4)) return false;
  // 32-bit block ids, in-image tap offsets and in-view output offsets
  const int64_t lim = (int64_t(1) << 31) - 1;
  if (p.is1 < 0 || p.is2 < 0 || p.is3 < 0 || p.os1 < 0 || p.os2 < 0) return false;
  const int64_t img_ext = (p.C - 1) * p.is1 + (p.H + 1) * p.is2 + (p.W + 1) * p.is3;
  const int64_t out_ext = (p.C - 1) * p.os1 + p.N * p.os2;
  return img_ext < lim && out_ext < lim && (p.N / 256) * n_views + 8 < lim;
}

// View-major bf16 output rows of 4 channels (see sampler_rings_vm_kernel): os0 == 4, os1 == 1,
// 8-byte aligned rows.
static bool vm_out(const SamplerParams& p, bool bf16_out) {
  return bf16_out && p.os0 == 4 && p.os1 == 1 && p.os2 % 4 == 0 && p.os2 >= 4 &&
         reinterpret_cast<uintptr_t>(p.out) % 8 == 0;
}

template <typename InT, int MODE, int PAD, bool PAIRS, int VMV>
static void launch_rings_vm_v(const SamplerParams& p, uint32_t bpv, int64_t n_views, hipStream_t s) {
  const uint32_t groups = static_cast<uint32_t>((n_views + VMV - 1) / VMV);
  const uint32_t total = bpv * groups, padded = (total + 7) / 8 * 8;
  const uint32_t nv = static_cast<uint32_t>(n_views);
  if constexpr (std::is_same<InT, uint16_t>::value) {
    if (p.is1 == 1 && p.is3 == p.C && (p.C == 3 || (p.C == 4 && p.is2 % 2 == 0)) && p.is0 % 2 == 0 &&
        reinterpret_cast<uintptr_t>(p.img) % 4 == 0) {
      if (p.C == 3)
        hipLaunchKernelGGL((sampler_rings_vm_kernel<InT, MODE, PAD, false, 3, 3, VMV>), dim3(padded), dim3(256), 0,
                           s, p, bpv, nv, total, padded);
      else
        hipLaunchKernelGGL((sampler_rings_vm_kernel<InT, MODE, PAD, false, 4, 4, VMV>), dim3(padded), dim3(256), 0,
                           s, p, bpv, nv, total, padded);
      return;
    }
  }
  if (p.C == 3)
    hipLaunchKernelGGL((sampler_rings_vm_kernel<InT, MODE, PAD, PAIRS, 3, 0, VMV>), dim3(padded), dim3(256), 0, s, p,
                       bpv, nv, total, padded);
  else
    hipLaunchKernelGGL((sampler_rings_vm_kernel<InT, MODE, PAD, PAIRS, 0, 0, VMV>), dim3(padded), dim3(256), 0, s, p,
                       bpv, nv, total, padded);
}

template <typename InT, int MODE, int PAD, bool PAIRS>
static void launch_rings_vm(const SamplerParams& p, uint32_t bpv, int64_t n_views, hipStream_t s) {
  if (static_cast<int64_t>(bpv) * ((n_views + 15) / 16) >= 2048)
    launch_rings_vm_v<InT, MODE, PAD, PAIRS, 16>(p, bpv, n_views, s);
  else
    launch_rings_vm_v<InT, MODE, PAD, PAIRS, 4>(p, bpv, n_views, s);
}

template <typename InT, typename OutT, int MODE, int PAD, bool PAIRS>
static void launch_rings(const SamplerParams& p, uint32_t bpv, uint32_t total, uint32_t padded, hipStream_t s) {
  if (vm_out(p, std::is_same<OutT, uint16_t>::value)) {
    launch_rings_vm<InT, MODE, PAD, PAIRS>(p, bpv, total / bpv, s);
    return;
  }
  dim3 grid(padded);
  // unit-stride channel planes with 16-byte aligned plane and view starts: whole 16-byte runs
  constexpr int64_t VPL = 16 / sizeof(OutT);
  const int vec_out = p.os2 == 1 && p.os1 % VPL == 0 && p.os0 % VPL == 0 &&
                      reinterpret_cast<uintptr_t>(p.out) % 16 == 0;
  if constexpr (std::is_same<InT, uint16_t>::value) {
    // channels-last bf16 pixels of 3 or 4 channels, 4-byte aligned image starts; 4-channel
    // pixels only at even elements (an odd one would need 5 of the 8-byte load's 4 halves)
    if (p.is1 == 1 && p.is3 == p.C && (p.C == 3 || (p.C == 4 && p.is2 % 2 == 0)) && p.is0 % 2 == 0 &&
        reinterpret_cast<uintptr_t>(p.img) % 4 == 0) {
      if (p.C == 3)
        hipLaunchKernelGGL((sampler_rings_kernel<InT, OutT, MODE, PAD, false, 3, 3>), grid, dim3(256), 0, s, p, bpv,
                           total, padded, vec_out);
      else
        hipLaunchKernelGGL((sampler_rings_kernel<InT, OutT, MODE, PAD, false, 4, 4>), grid, dim3(256), 0, s, p, bpv,
                           total, padded, vec_out);
      return;
    }
  }
  if (p.C == 3)
    hipLaunchKernelGGL((sampler_rings_kernel<InT, OutT, MODE, PAD, PAIRS, 3>), grid, dim3(256), 0, s, p, bpv, total,
                       padded, vec_out);
  else if (p.C == 1)
    hipLaunchKernelGGL((sampler_rings_kernel<InT, OutT, MODE, PAD, PAIRS, 1>), grid, dim3(256), 0, s, p, bpv, total,
                       padded, vec_out);
  else
    hipLaunchKernelGGL((sampler_rings_kernel<InT, OutT, MODE, PAD, PAIRS, 0>), grid, dim3(256), 0, s, p, bpv, total,
                       padded, vec_out);
}

template <typename InT, typename OutT, int MODE, int PAD>
static void launch_mode(const SamplerParams& p, int64_t n_views, bool pairs, hipStream_t s) {
  const int64_t bpv = (p.N + 255) / 256;
  const int64_t total = bpv * n_views;
  const int64_t padded = (total + 7) / 8 * 8;
  dim3 grid(static_cast<unsigned>(padded));
  if (rings_path(p, n_views)) {
    if (MODE == FOVI_BILINEAR && pairs)
      launch_rings<InT, OutT, MODE, PAD, true>(p, static_cast<uint32_t>(bpv), static_cast<uint32_t>(total),
                                               static_cast<uint32_t>(padded), s);
    else
      launch_rings<InT, OutT, MODE, PAD, false>(p, static_cast<uint32_t>(bpv), static_cast<uint32_t>(total),
                                                static_cast<uint32_t>(padded), s);
    return;
  }
  if (MODE == FOVI_BILINEAR && pairs)
    hipLaunchKernelGGL((sampler_kernel<InT, OutT, MODE, PAD, true>), grid, dim3(256), 0, s, p, bpv, total, padded);
  else
    hipLaunchKernelGGL((sampler_kernel<InT, OutT, MODE, PAD, false>), grid, dim3(256), 0, s, p, bpv, total, padded);
}

template <typename InT, typename OutT>
static void launch_typed(const SamplerParams& p, int mode, int pad, int64_t n_views, hipStream_t s) {
  // pixel pairs need unit-stride rows whose starts are 4-byte aligned
  const bool pairs = p.is3 == 1 && (reinterpret_cast<uintptr_t>(p.img) & 3) == 0 &&
                     (sizeof(InT) == 4 || ((p.is0 | p.is1 | p.is2) & 1) == 0);
  if (mode == FOVI_NEAREST) {
    if (pad == FOVI_PAD_ZEROS) launch_mode<InT, OutT, FOVI_NEAREST, FOVI_PAD_ZEROS>(p, n_views, pairs, s);
    else launch_mode<InT, OutT, FOVI_NEAREST, FOVI_PAD_BORDER>(p, n_views, pairs, s);
  } else {
    if (pad == FOVI_PAD_ZEROS) launch_mode<InT, OutT, FOVI_BILINEAR, FOVI_PAD_ZEROS>(p, n_views, pairs, s);
    else launch_mode<InT, OutT, FOVI_BILINEAR, FOVI_PAD_BORDER>(p, n_views, pairs, s);
  }
}

}  // namespace fovi

extern "C" int fovi_sampler_fwd(const fovi_sampler_args* a, void* stream) {
  using namespace fovi;
  clear_error();
  if (!a) { set_error("fovi_sampler_fwd: null args"); return 1; }
  if (!a->img || !a->grid || !a->fix_loc || !a->fix_half || !a->out) {
    set_error("fovi_sampler_fwd: null pointer argument"); return 1;
  }
  if (a->n_img <= 0 || a->channels <= 0 || a->height <= 0 || a->width <= 0 || a->n_points < 0 ||
      a->n_views < 0) {
    set_error("fovi_sampler_fwd: bad sizes (n_img=%lld C=%lld H=%lld W=%lld N=%lld views=%lld)",
              (long long)a->n_img, (long long)a->channels, (long long)a->height, (long long)a->width,
              (long long)a->n_points, (long long)a->n_views);
    return 1;
  }
  if ((a->n_points + 255) / 256 * a->n_views > (int64_t(1) << 31) - 8) {
    set_error("fovi_sampler_fwd: %lld views x %lld points exceed one launch", (long long)a->n_views,
              (long long)a->n_points);
    return 1;
  }
  if (!a->view_image && a->n_views > a->n_img) {
    set_error("fovi_sampler_fwd: %lld views but %lld images and no view_image map",
              (long long)a->n_views, (long long)a->n_img);
    return 1;
  }
  if (a->mode != FOVI_NEAREST && a->mode != FOVI_BILINEAR) { set_error("fovi_sampler_fwd: bad mode %d", a->mode); return 1; }
  if (a->padding != FOVI_PAD_ZEROS && a->padding != FOVI_PAD_BORDER) {
    set_error("fovi_sampler_fwd: bad padding %d", a->padding); return 1;
  }
  if (a->n_points == 0 || a->n_views == 0) return 0;
  SamplerParams p;
  p.img = a->img; p.n_img = a->n_img; p.C = a->channels; p.H = a->height; p.W = a->width;
  p.is0 = a->img_stride[0]; p.is1 = a->img_stride[1]; p.is2 = a->img_stride[2]; p.is3 = a->img_stride[3];
  p.grid = a->grid; p.N = a->n_points; p.fix_loc = a->fix_loc; p.fix_half = a->fix_half;
  p.wide = a->fix_half_wide ? 1 : 0; p.view_image = a->view_image; p.out = a->out;
  p.os0 = a->out_stride[0]; p.os1 = a->out_stride[1]; p.os2 = a->out_stride[2]; p.grid_out = a->grid_out;
  p.ring_len = a->ring_len > 0 ? a->ring_len : 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int in_t = a->img_dtype, out_t = a->out_dtype;
  if (in_t == FOVI_F32 && out_t == FOVI_F32) launch_typed<float, float>(p, a->mode, a->padding, a->n_views, s);
  else if (in_t == FOVI_F32 && out_t == FOVI_BF16) launch_typed<float, uint16_t>(p, a->mode, a->padding, a->n_views, s);
  else if (in_t == FOVI_BF16 && out_t == FOVI_F32) launch_typed<uint16_t, float>(p, a->mode, a->padding, a->n_views, s);
  else if (in_t == FOVI_BF16 && out_t == FOVI_BF16) launch_typed<uint16_t, uint16_t>(p, a->mode, a->padding, a->n_views, s);
  else { set_error("fovi_sampler_fwd: unsupported dtypes img=%d out=%d", in_t, out_t); return 1; }
  return check_launch("fovi_sampler_fwd");
}
