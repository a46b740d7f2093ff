// kNN-convolution forward with OCP fp8 e4m3 operands on gfx950 MFMA.
//
// Same structure as the bf16 staged-row kernel (knnconv.hip): 256-point x NT
// tiles, the tile's contiguous input rows staged in LDS, single-neighbour
// slots read straight from them, collision slots summed into a small tile.
// Differences:
//  * an LDS row is 64 fp8 channels (64 bytes), one reduction chunk, consumed
//    by one v_mfma_scale_f32_32x32x64_f8f6f4 per 32x32 block (unit scales);
//  * collision sums are formed in fp32 from the e4m3 values and rounded once
//    back to e4m3 (round to nearest even, saturating), with the hardware
//    conversions v_cvt_pk_f32_fp8 / v_cvt_pk_fp8_f32. The per-tensor input
//    scale given by the caller must leave room for the largest sum (the
//    library's Python side uses 2^r * amax / 448 with 2^r >= the layer's
//    largest slot count), so sums never saturate;
//  * y = x_scale * w_scale[o] * acc + bias[o] (x_scale from device memory when
//    x_scale_dev is given).
#include "common.h"
#include "knnconv_internal.h"

namespace fovi {

typedef int i32x8 __attribute__((ext_vector_type(8)));

// acc[0..15] += the 16 e4m3 values of one 16-byte chunk (v_cvt_pk_f32_fp8).
__device__ __forceinline__ void add_e4m3x16(float (&acc)[16], const u32x4 v) {
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(v[w]), false);
    const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(v[w]), true);
    acc[4 * w] += lo[0];
    acc[4 * w + 1] += lo[1];
    acc[4 * w + 2] += hi[0];
    acc[4 * w + 3] += hi[1];
  }
}

struct F8Layout {
  int b_off, ent_off, colln_off, coll_off, nbl_off, s_off, total;
};

__host__ __device__ inline F8Layout f8_layout(int nt, int V, int K, int zero_row) {
  F8Layout l;
  int o = 2 * 256 * 64;                          // A: two 256 x 64-byte tiles
  l.b_off = o;      o += 2 * nt * 64;            // B: two NT x 64-byte tiles
  l.ent_off = o;    o += 256 * V * 4;
  l.colln_off = o;  o += (V * 4 + 15) & ~15;
  l.coll_off = o;   o += V * 256;
  l.nbl_off = o;    o += (256 * K * 2 + 15) & ~15;
  l.s_off = o;      o += (zero_row + 1) * 64;
  l.total = o;
  return l;
}

// byte offset of 16-byte chunk q of 64-byte row r (same swizzle as the bf16 tiles)
__device__ __forceinline__ int swzb(int r, int q) { return swz32(r, q) * 2; }

template <int NT, int SV, typename OutT>
__global__ __launch_bounds__(512, 1) void knnconv_fp8_kernel(KnnParams p, int64_t tiles_per_b, int64_t n_tiles_n,
                                                             int64_t total_tiles, int64_t padded_tiles) {
  constexpr int WN = NT / 2;
  constexpr int CB = WN / 32;
  constexpr int CCE = 64;                           // channels (bytes) per chunk
  constexpr int B_VECS = (NT * 4 + 511) / 512;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int V = static_cast<int>(p.V), K = static_cast<int>(p.K);
  const int zr = p.zero_row;
  const F8Layout L = f8_layout(NT, V, K, zr);
  uint8_t* Bs = smem + L.b_off;
  uint32_t* ent = reinterpret_cast<uint32_t*>(smem + L.ent_off);
  int32_t* colln = reinterpret_cast<int32_t*>(smem + L.colln_off);
  uint8_t* coll = smem + L.coll_off;
  uint16_t* nbl = reinterpret_cast<uint16_t*>(smem + L.nbl_off);
  uint8_t* S = smem + L.s_off;

  const int64_t tile = xcd_tile(blockIdx.x, padded_tiles);
  if (tile >= total_tiles) return;
  const int64_t mt = tile / n_tiles_n;
  const int64_t o0 = (tile % n_tiles_n) * NT;
  const int64_t b = mt / tiles_per_b;
  const int64_t pt = mt % tiles_per_b;
  const int64_t n0 = pt * 256;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 3, wn = wave >> 2;
  const int64_t lo = p.tile_lo[pt];
  const int span = static_cast<int>(min(static_cast<int64_t>(zr), p.Nin - lo));

  for (int i = tid; i < 256 * V; i += 512) {
    const int r = i / V, v = i - r * V;
    ent[v * 256 + r] = p.tile_ent[n0 * p.V + i];
  }
  for (int i = tid; i < V * 64; i += 512)
    reinterpret_cast<uint32_t*>(coll)[i] = reinterpret_cast<const uint32_t*>(p.tile_coll)[pt * V * 64 + i];
  for (int i = tid; i < V; i += 512) colln[i] = p.tile_coll_n[pt * V + i];
  for (int i = tid; i < 256 * K; i += 512) nbl[i] = p.tile_nbr[n0 * p.K + i];
  if (tid < 4) *reinterpret_cast<u32x4*>(&S[zr * 64 + tid * 16]) = u32x4{0u, 0u, 0u, 0u};

  const char* xrows = static_cast<const char*>(p.x) + b * p.xs0 + lo * p.xs2;
  const char* wbase = static_cast<const char*>(p.w) + o0 * p.Kpad;
  uint32_t s_off[SV], w_off[B_VECS];
  uint32_t s_ok = 0, w_ok = 0;
#pragma unroll
  for (int j = 0; j < SV; ++j) {
    const int q = tid + 512 * j;
    s_ok |= static_cast<uint32_t>((q >> 2) < span) << j;
    s_off[j] = static_cast<uint32_t>((q >> 2) * p.xs2 + (q & 3) * 16);
  }
#pragma unroll
  for (int i = 0; i < B_VECS; ++i) {
    const int q = tid + 512 * i;
    w_ok |= static_cast<uint32_t>(q < NT * 4 && o0 + (q >> 2) < p.Cout) << i;
    w_off[i] = static_cast<uint32_t>((q >> 2) * p.Kpad + (q & 3) * 16);
  }
  const int ncc = static_cast<int>(p.C / CCE);
  const int nit = ncc * V;

  u32x4 rs[SV], rb[B_VECS];
  auto load_s = [&](int cc) {
    const char* base = xrows + cc * CCE;
#pragma unroll
    for (int j = 0; j < SV; ++j)
      rs[j] = ((s_ok >> j) & 1) ? *reinterpret_cast<const u32x4*>(base + s_off[j]) : u32x4{0u, 0u, 0u, 0u};
  };
  auto store_s = [&]() {
#pragma unroll
    for (int j = 0; j < SV; ++j) {
      const int q = tid + 512 * j;
      if ((s_ok >> j) & 1) *reinterpret_cast<u32x4*>(&S[swzb(q >> 2, q & 3)]) = rs[j];
    }
  };
  auto load_w = [&](int cc, int v) {
    const char* base = wbase + static_cast<int64_t>(v) * p.C + cc * CCE;
#pragma unroll
    for (int i = 0; i < B_VECS; ++i)
      rb[i] = ((w_ok >> i) & 1) ? *reinterpret_cast<const u32x4*>(base + w_off[i]) : u32x4{0u, 0u, 0u, 0u};
  };
  auto store_w = [&](int buf) {
    uint8_t* bsm = Bs + buf * NT * 64;
#pragma unroll
    for (int i = 0; i < B_VECS; ++i) {
      const int q = tid + 512 * i;
      if (q < NT * 4) *reinterpret_cast<u32x4*>(&bsm[swzb(q >> 2, q & 3)]) = rb[i];
    }
  };
  auto build_coll = [&](int v, int buf) {
    const int items = colln[v] * 4;
    uint8_t* a = smem + buf * 256 * 64;
    for (int item = tid; item < items; item += 512) {
      const int row = coll[v * 256 + (item >> 2)];
      const int part = item & 3;
      const uint32_t e = ent[v * 256 + row];
      const int cnt = (e >> 8) & 0xff;
      const uint16_t* nb = nbl + row * K + (e & 0xff);
      float acc16[16];
#pragma unroll
      for (int c = 0; c < 16; ++c) acc16[c] = 0.0f;
      for (int j0 = 0; j0 < cnt; j0 += 4) {
        int rr[4];
        rr[0] = j0 == 0 ? static_cast<int>(e >> 16) : nb[j0];
        rr[1] = j0 + 1 < cnt ? nb[j0 + 1] : zr;
        rr[2] = j0 + 2 < cnt ? nb[j0 + 2] : zr;
        rr[3] = j0 + 3 < cnt ? nb[j0 + 3] : zr;
        u32x4 xv[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) xv[u] = *reinterpret_cast<const u32x4*>(&S[swzb(rr[u], part)]);
#pragma unroll
        for (int u = 0; u < 4; ++u) add_e4m3x16(acc16, xv[u]);
      }
      u32x4 out;
#pragma unroll
      for (int w = 0; w < 4; ++w)
        out[w] = cvt_pk_e4m3<true>(acc16[4 * w + 2], acc16[4 * w + 3],
                                   cvt_pk_e4m3<false>(acc16[4 * w], acc16[4 * w + 1], 0u));
      *reinterpret_cast<u32x4*>(&a[swzb(row, part)]) = out;
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
  const int qa = (lane >> 5) * 2;                 // this lane's two 16-byte chunks: qa, qa + 1

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
      for (int i = 0; i < 2; ++i) enxt[i] = ent[v1 * 256 + rowm[i]];
      if (v1 != 0) build_coll(v1, cur ^ 1);
    }
    i32x8 af[2], bfr[CB];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const bool from_a = ((ecur[i] >> 8) & 0xff) >= 2;
      const int srow = static_cast<int>(ecur[i] >> 16);
      const uint8_t* base = from_a ? smem + cur * 256 * 64 : S;
      const int r = from_a ? rowm[i] : srow;
      const u32x4 lo4 = *reinterpret_cast<const u32x4*>(&base[swzb(r, qa)]);
      const u32x4 hi4 = *reinterpret_cast<const u32x4*>(&base[swzb(r, qa + 1)]);
      af[i] = i32x8{(int)lo4[0], (int)lo4[1], (int)lo4[2], (int)lo4[3], (int)hi4[0], (int)hi4[1], (int)hi4[2], (int)hi4[3]};
    }
    const uint8_t* bsm = Bs + cur * NT * 64;
#pragma unroll
    for (int j = 0; j < CB; ++j) {
      const int col = wn * WN + j * 32 + (lane & 31);
      const u32x4 lo4 = *reinterpret_cast<const u32x4*>(&bsm[swzb(col, qa)]);
      const u32x4 hi4 = *reinterpret_cast<const u32x4*>(&bsm[swzb(col, qa + 1)]);
      bfr[j] = i32x8{(int)lo4[0], (int)lo4[1], (int)lo4[2], (int)lo4[3], (int)hi4[0], (int)hi4[1], (int)hi4[2], (int)hi4[3]};
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < CB; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(af[i], bfr[j], acc[i][j], 0, 0, 0, 127, 0, 127);
    if (more) store_w(cur ^ 1);
    __syncthreads();
    if (more && v1 == 0) {
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
  const float xs = p.x_scale_dev ? *p.x_scale_dev : p.x_scale;
#pragma unroll
  for (int j = 0; j < CB; ++j) {
    const int64_t o = o0 + wn * WN + j * 32 + (lane & 31);
    if (o >= p.Cout) continue;
    const float sc = xs * p.w_scale[o];
    const float bo = p.bias ? p.bias[o] : 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t n = n0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (n < p.Nout) Elem<OutT>::store(y + o * p.ys1 + n * p.ys2, epilogue(acc[i][j][r] * sc + bo, p.relu));
      }
  }
}

template <int NT, int SV>
static void launch_fp8_sv(const KnnParams& p, int out_t, hipStream_t s) {
  const int64_t tiles_per_b = (p.Nout + 255) / 256;
  const int64_t n_tiles_n = (p.Cout + NT - 1) / NT;
  const int64_t total = p.B * tiles_per_b * n_tiles_n;
  const int64_t padded = (total + 7) / 8 * 8;
  const size_t lds = f8_layout(NT, static_cast<int>(p.V), static_cast<int>(p.K), p.zero_row).total;
  dim3 grid(static_cast<unsigned>(padded));
  if (out_t == FOVI_BF16) {
    (void)reserve_dynamic_lds(reinterpret_cast<const void*>(&knnconv_fp8_kernel<NT, SV, uint16_t>), lds);
    hipLaunchKernelGGL((knnconv_fp8_kernel<NT, SV, uint16_t>), grid, dim3(512), lds, s, p, tiles_per_b, n_tiles_n,
                       total, padded);
  } else {
    (void)reserve_dynamic_lds(reinterpret_cast<const void*>(&knnconv_fp8_kernel<NT, SV, float>), lds);
    hipLaunchKernelGGL((knnconv_fp8_kernel<NT, SV, float>), grid, dim3(512), lds, s, p, tiles_per_b, n_tiles_n,
                       total, padded);
  }
}

template <int NT>
static bool launch_fp8_nt(const KnnParams& p, int out_t, hipStream_t s) {
  const int sv = (p.zero_row * 4 + 511) / 512;
  if (sv <= 2) launch_fp8_sv<NT, 2>(p, out_t, s);
  else if (sv <= 4) launch_fp8_sv<NT, 4>(p, out_t, s);
  else if (sv <= 6) launch_fp8_sv<NT, 6>(p, out_t, s);
  else if (sv <= 8) launch_fp8_sv<NT, 8>(p, out_t, s);
  else return false;
  return true;
}

int launch_knnconv_fp8(const KnnParams& p, int out_t, hipStream_t s) {
  if (p.C % 64 != 0) { set_error("fovi_knnconv_fwd(fp8): c_in must be a multiple of 64"); return 1; }
  if (p.xs1 != 1 || p.xs2 % 16 != 0 || p.xs0 % 16 != 0 || reinterpret_cast<uintptr_t>(p.x) % 16 != 0) {
    set_error("fovi_knnconv_fwd(fp8): needs channels-last 16-byte aligned input rows"); return 1;
  }
  if (!p.tile_lo || !p.tile_coll || !p.tile_coll_n || p.zero_row <= 0 || p.zero_row > 1024 || p.K > 255 ||
      p.V > 255) {
    set_error("fovi_knnconv_fwd(fp8): needs the tile tables (k, n_ref <= 255, spans <= 1024)"); return 1;
  }
  if (!p.w_scale) { set_error("fovi_knnconv_fwd(fp8): w_scale is required"); return 1; }
  // channel tiles up to 128 wide: the 32-register fp8 operand fragments of a
  // wider tile do not fit beside its accumulators without spilling
  const int nt = pick_tile_n(p.Cout, [&](int t) {
    return t <= 128 && f8_layout(t, static_cast<int>(p.V), static_cast<int>(p.K), p.zero_row).total <= 160 * 1024;
  });
  bool ok = false;
  if (nt == 128) ok = launch_fp8_nt<128>(p, out_t, s);
  else if (nt == 64) ok = launch_fp8_nt<64>(p, out_t, s);
  if (!ok) { set_error("fovi_knnconv_fwd(fp8): tile does not fit LDS"); return 1; }
  return check_launch("fovi_knnconv_fwd(fp8)");
}

}  // namespace fovi
