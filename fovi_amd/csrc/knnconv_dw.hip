// Weight gradient of the kNN convolution for gfx950, without the slot-sum matrix.
//
// dW[o, c * V + v] = sum over images b and over the (output n, input i) pairs whose
// neighbour i sits in slot v of n of dy[b, n, o] * x[b, i, c]: for every slot a GEMM whose
// reduction runs over that slot's pair list (the sum of a collision slot is linear, so its
// pairs enter one by one). The pairs come in segments (one slot, one chunk of output
// points); a workgroup owns one segment, a group of images and one 256 x 256 (o, c) tile.
// Its eight waves, two per SIMD so one wave's memory waits overlap the other's MFMAs, hold
// 128 x 64 fp32 blocks (8 blocks of v_mfma_f32_32x32x16_bf16). Workgroups are numbered
// slot-fastest and mapped XCD by XCD, so the V workgroups of a chunk share one L2.
//
// Per step of 64 pairs the workgroup loads the 64 dy rows and the 64 x rows (16-byte
// chunks, a full row per 32 lanes) into LDS in their natural [pair][channel] layout, double
// buffered one step ahead. Both MFMA operands need the pair index contiguous per lane, which
// the transposed LDS read ds_read_b64_tr_b16 delivers: within a 16-lane group, lane j
// addresses four channels of pair row k0 + j/4 and lane i receives channel i of pairs
// k0 .. k0 + 3. Rows are 576 bytes apart so those reads hit 64 distinct banks.
// Per-workgroup partial tiles go to a caller workspace; a second kernel sums them into the
// reference weight layout (column c * V + v), fp32.
#include "common.h"

namespace fovi {
namespace {

constexpr int DW_T = 256;          // o and c tile
constexpr int DW_K = 64;           // pairs per step
constexpr int DW_R = DW_K / 16;    // rows per thread and operand in a step (512 threads, 32 per row)
constexpr int DW_RS = 576;         // LDS bytes per pair row (256 bf16 + 64 bytes of bank skew)
constexpr int DW_BUF = DW_K * DW_RS;            // one operand, one step
constexpr int DW_LDS = 2 * 2 * DW_BUF;          // two operands, two steps: 147,456 bytes

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

struct DwParams {
  const uint16_t* x;
  int64_t xs0, xs2;                // x[b * xs0 + i * xs2 + c]
  const uint16_t* dy;
  int64_t ds0, ds2;                // dy[b * ds0 + n * ds2 + o]
  int64_t B, C, Cout, Nin, Nout, V;
  const int32_t* pair_off;         // [NQ * V + 1], segment q * V + v
  const int32_t* pairs;            // (n, i) per pair; n < 0 pads
  int64_t NQ, ipg, S, tiles_o, tiles_c;
  float* part;                     // [S, NQ, V, tiles_o, tiles_c, 256, 256]
};

__device__ __forceinline__ s16x4 tr_read(const uint8_t* lds_base, int byte_off) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4*)(reinterpret_cast<uintptr_t>(lds_base) + byte_off));
}

__global__ __launch_bounds__(512, 1) void knnconv_dw_kernel(DwParams p, int64_t total, int64_t padded) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int64_t L = xcd_tile(blockIdx.x, padded);
  if (L >= total) return;                       // whole workgroup: before any barrier
  const int64_t v = L % p.V;
  int64_t rest = L / p.V;
  const int64_t tc = rest % p.tiles_c;
  rest /= p.tiles_c;
  const int64_t to = rest % p.tiles_o;
  rest /= p.tiles_o;
  const int64_t q = rest % p.NQ;
  const int64_t split = rest / p.NQ;
  const int64_t o0 = to * DW_T, c0 = tc * DW_T;

  // eight waves, two per SIMD: wave (wm, wn) holds o rows wm*128 .. +127, c columns wn*64 .. +63
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, wm = wave >> 2, wn = wave & 3;
  const int64_t seg = q * p.V + v;
  const int64_t P0 = p.pair_off[seg], P1 = p.pair_off[seg + 1];
  const int64_t steps_img = (P1 - P0 + DW_K - 1) / DW_K;     // the last step's tail reads as pads
  const int64_t b_beg = split * p.ipg;
  const int64_t steps = steps_img * (min(p.B, b_beg + p.ipg) - b_beg);

  // load task: pair rows t/32 + 16r (r < DW_R), 16-byte chunk g of the row; chunks past the
  // channels load chunk 0 and pads load row 0, both masked to zero when stored
  const int g = t & 31, pr0 = t >> 5;
  const bool okc = c0 + 8 * g < p.C, oko = o0 + 8 * g < p.Cout;
  const int gd = oko ? g : 0, gc = okc ? g : 0;

  f32x16 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  int2 pe[DW_R];                                // pair entries of the step being prefetched
  u32x4v rd[DW_R], rx[DW_R];                    // rows of the step in flight
  uint32_t m = 0;                               // their live bits
  auto load_pairs = [&](int64_t st) __attribute__((always_inline)) {
    const int64_t base = P0 + DW_K * ((st < steps ? st : 0) % steps_img);
#pragma unroll
    for (int r = 0; r < DW_R; ++r) {
      const int64_t pi = base + pr0 + 16 * r;
      pe[r] = *reinterpret_cast<const int2*>(p.pairs + 2 * (pi < P1 ? pi : P1 - 1));
      if (pi >= P1) pe[r].x = -1;                 // past the segment: a pad
    }
  };
  auto load_rows = [&](int64_t st) __attribute__((always_inline)) {
    const bool on = st < steps;
    const int64_t b = b_beg + (on ? st / steps_img : 0);   // uniform: the image base stays scalar
    const uint16_t* xb = p.x + b * p.xs0 + c0;
    const uint16_t* db = p.dy + b * p.ds0 + o0;
    m = 0;
#pragma unroll
    for (int r = 0; r < DW_R; ++r) {
      const bool live = on && pe[r].x >= 0;
      const uint32_t n = live ? pe[r].x : 0, i = live ? pe[r].y : 0;
      // 32-bit element offsets within the image (the host checks they fit)
      rd[r] = *reinterpret_cast<const u32x4v*>(db + (n * static_cast<uint32_t>(p.ds2) + 8u * gd));
      rx[r] = *reinterpret_cast<const u32x4v*>(xb + (i * static_cast<uint32_t>(p.xs2) + 8u * gc));
      m |= static_cast<uint32_t>(live && oko) << r | static_cast<uint32_t>(live && okc) << (DW_R + r);
    }
  };
  auto store_rows = [&](int buf) __attribute__((always_inline)) {
    uint8_t* bd = smem + buf * 2 * DW_BUF;
    uint8_t* bx = bd + DW_BUF;
    const u32x4v z = {0, 0, 0, 0};
#pragma unroll
    for (int r = 0; r < DW_R; ++r) {
      *reinterpret_cast<u32x4v*>(bd + (pr0 + 16 * r) * DW_RS + 16 * g) = (m >> r & 1) ? rd[r] : z;
      *reinterpret_cast<u32x4v*>(bx + (pr0 + 16 * r) * DW_RS + 16 * g) = (m >> (DW_R + r) & 1) ? rx[r] : z;
    }
  };

  // this lane's transposed-read offsets: 16-lane group G supplies pair rows kb*16 + 8*(G>>1)
  // + li/4 (+4 for the second half) and channels 16*(G&1) + 4*(li%4) of each 32-block
  const int G = lane >> 4, li = lane & 15;
  const int lane_off = ((G >> 1) * 8 + (li >> 2)) * DW_RS + ((G & 1) * 16 + 4 * (li & 3)) * 2;

  if (steps > 0) {
    // prologue: step 0 into LDS buffer 0, step 1 in flight, pair entries of step 2 loading
    load_pairs(0);
    load_rows(0);
    store_rows(0);
    load_pairs(1);
    load_rows(1);
    load_pairs(2);
    __syncthreads();
    for (int64_t st = 0; st < steps; ++st) {
      const uint8_t* bd = smem + (st & 1) * 2 * DW_BUF;
      const uint8_t* bx = bd + DW_BUF;
#pragma unroll
      for (int kb = 0; kb < DW_K / 16; ++kb) {
        bf16x8 af[4], bf[2];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int off = lane_off + kb * 16 * DW_RS + (wm * 128 + i * 32) * 2;
          const s16x4 lo = tr_read(bd, off), hi = tr_read(bd, off + 4 * DW_RS);
          af[i] = __builtin_bit_cast(bf16x8, s16x8(__builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7)));
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int off = lane_off + kb * 16 * DW_RS + (wn * 64 + j * 32) * 2;
          const s16x4 lo = tr_read(bx, off), hi = tr_read(bx, off + 4 * DW_RS);
          bf[j] = __builtin_bit_cast(bf16x8, s16x8(__builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7)));
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bf[j], acc[i][j], 0, 0, 0);
      }
      if (st + 1 < steps) store_rows((st + 1) & 1);  // buffer last read in step st - 1
      load_rows(st + 2);
      load_pairs(st + 3);
      __syncthreads();
    }
  }

  float* out = p.part + (((split * p.NQ * p.V + seg) * p.tiles_o + to) * p.tiles_c + tc) * (DW_T * DW_T);
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int o = wm * 128 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        const int c = wn * 64 + j * 32 + (lane & 31);
        out[o * DW_T + c] = acc[i][j][r];
      }
}

// dW[o, c * V + v] = sum over the (image group, chunk) partial tiles (fp32); one thread per
// (v, o, c), consecutive threads along c (coalesced partial reads)
__global__ __launch_bounds__(256) void knnconv_dw_reduce_kernel(DwParams p, float* dw) {
  const int64_t total = p.V * p.Cout * p.C;
  for (int64_t q = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; q < total;
       q += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t c = q % p.C;
    const int64_t o = (q / p.C) % p.Cout;
    const int64_t v = q / (p.C * p.Cout);
    const int64_t tile = (o / DW_T) * p.tiles_c + c / DW_T;
    const int64_t in_tile = (o % DW_T) * DW_T + c % DW_T;
    const int64_t stride = p.V * p.tiles_o * p.tiles_c * (DW_T * DW_T);   // next (group, chunk)
    const float* src = p.part + (v * p.tiles_o * p.tiles_c + tile) * (DW_T * DW_T) + in_tile;
    // partials added in (group, chunk) order; four loads in flight per trip
    float sum = 0.0f;
    const int64_t n = p.S * p.NQ;
    int64_t sq = 0;
    for (; sq + 4 <= n; sq += 4) {
      float t[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) t[u] = src[(sq + u) * stride];
#pragma unroll
      for (int u = 0; u < 4; ++u) sum += t[u];
    }
    for (; sq < n; ++sq) sum += src[sq * stride];
    dw[o * p.C * p.V + c * p.V + v] = sum;
  }
}

}  // namespace
}  // namespace fovi

using namespace fovi;

extern "C" int64_t fovi_knnconv_dw_workspace_bytes(int64_t batch, int64_t images_per_group, int64_t n_chunks,
                                                   int64_t c_in, int64_t c_out, int64_t n_ref) {
  if (batch < 1 || images_per_group < 1 || n_chunks < 1 || c_in < 1 || c_out < 1 || n_ref < 1) return -1;
  const int64_t splits = (batch + images_per_group - 1) / images_per_group;
  const int64_t tiles = ((c_out + DW_T - 1) / DW_T) * ((c_in + DW_T - 1) / DW_T);
  return splits * n_chunks * n_ref * tiles * DW_T * DW_T * static_cast<int64_t>(sizeof(float));
}

extern "C" int fovi_knnconv_dw(const fovi_knnconv_dw_args* a, void* stream) {
  clear_error();
  if (!a || !a->x || !a->dy || !a->pair_off || !a->pairs || !a->workspace || !a->dw) {
    set_error("fovi_knnconv_dw: null pointer");
    return 1;
  }
  if (a->batch < 1 || a->c_in < 8 || a->c_out < 8 || a->c_in % 8 || a->c_out % 8 || a->n_in < 1 ||
      a->n_out < 1 || a->n_ref < 1 || a->n_chunks < 1 || a->images_per_group < 1 || a->n_in > INT32_MAX ||
      a->n_out > INT32_MAX) {
    set_error("fovi_knnconv_dw: bad sizes (channel counts must be multiples of 8)");
    return 1;
  }
  if (a->n_in * a->x_stride[2] + a->c_in > UINT32_MAX || a->n_out * a->dy_stride[2] + a->c_out > UINT32_MAX) {
    set_error("fovi_knnconv_dw: one image's rows must span fewer than 2^32 elements");
    return 1;
  }
  if (a->x_stride[1] != 1 || a->dy_stride[1] != 1 || a->x_stride[2] % 8 || a->x_stride[0] % 8 ||
      a->dy_stride[2] % 8 || a->dy_stride[0] % 8 || reinterpret_cast<uintptr_t>(a->x) % 16 ||
      reinterpret_cast<uintptr_t>(a->dy) % 16) {
    set_error("fovi_knnconv_dw: x and dy must be channels-last bf16 with 16-byte aligned rows");
    return 1;
  }
  const int64_t need = fovi_knnconv_dw_workspace_bytes(a->batch, a->images_per_group, a->n_chunks, a->c_in,
                                                       a->c_out, a->n_ref);
  if (a->workspace_bytes < need) {
    set_error("fovi_knnconv_dw: workspace %lld bytes, need %lld", (long long)a->workspace_bytes, (long long)need);
    return 1;
  }
  DwParams p;
  p.x = static_cast<const uint16_t*>(a->x); p.xs0 = a->x_stride[0]; p.xs2 = a->x_stride[2];
  p.dy = static_cast<const uint16_t*>(a->dy); p.ds0 = a->dy_stride[0]; p.ds2 = a->dy_stride[2];
  p.B = a->batch; p.C = a->c_in; p.Cout = a->c_out; p.Nin = a->n_in; p.Nout = a->n_out; p.V = a->n_ref;
  p.pair_off = a->pair_off; p.pairs = a->pairs;
  p.NQ = a->n_chunks; p.ipg = a->images_per_group; p.S = (p.B + p.ipg - 1) / p.ipg;
  p.tiles_o = (p.Cout + DW_T - 1) / DW_T; p.tiles_c = (p.C + DW_T - 1) / DW_T;
  p.part = static_cast<float*>(a->workspace);
  const int64_t total = p.S * p.NQ * p.V * p.tiles_o * p.tiles_c;
  const int64_t padded = (total + 7) / 8 * 8;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (reserve_dynamic_lds(reinterpret_cast<const void*>(&knnconv_dw_kernel), DW_LDS) != hipSuccess) {
    set_error("fovi_knnconv_dw: cannot reserve %d bytes of LDS", DW_LDS);
    return 1;
  }
  hipLaunchKernelGGL(knnconv_dw_kernel, dim3(static_cast<unsigned>(padded)), dim3(512), DW_LDS, s, p, total,
                     padded);
  if (check_launch("fovi_knnconv_dw")) return 1;
  const int64_t n = p.V * p.Cout * p.C;
  hipLaunchKernelGGL(knnconv_dw_reduce_kernel, dim3(static_cast<unsigned>(std::min<int64_t>((n + 255) / 256, 65536))),
                     dim3(256), 0, s, p, a->dw);
  return check_launch("fovi_knnconv_dw(reduce)");
}
