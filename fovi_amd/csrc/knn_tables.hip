// kNN search on the wrapped log-polar cortical lattice for gfx950: the
// O(N_in * N_out) part of a kNN layer's table construction
// (fovi/arch/knn.py:101-152, log-polar branch), with the host builder's
// results bit for bit.
//
// The host builder takes torch's CPU square root, which is not always the
// correctly rounded one, and torch's CPU topk, whose order among equal
// distances comes from its heap selection. So the search runs in two passes
// around one host step:
//   1. knn_lp_candidates_kernel (one thread per output point): the scan in
//      input order with IEEE distances and a size-k max-heap that tracks the
//      running k-th smallest; it emits (index, squared distance) for the first
//      k inputs and every input within a small margin below that running
//      value: every input the host's heap can admit (the host's distances
//      are within an ulp of the IEEE ones, so its running k-th value is too).
//   2. the host takes the square roots of the emitted squared distances (exact
//      fp32 on both sides) with the same torch call the host builder makes.
//   3. knn_select_kernel replays the host's selection over the candidates in
//      input order: the heap steps of the C++ standard library's partial_sort
//      as libstdc++ builds it (heap select: make the heap of the first k,
//      replace the top by every later element that compares strictly smaller,
//      sifting the hole down to a leaf and the value back up; then sort the
//      heap by repeated pops), which torch's CPU topk(largest=False) runs when
//      k * 64 <= n. Inputs never emitted are never admitted by that heap, so
//      skipping them changes nothing.
// Heaps live in LDS, interleaved by thread. Uniform input loads (every lane
// reads the same point) go through the scalar cache; all stores are vector
// stores.
#include "common.h"

namespace fovi {
namespace {

constexpr int KNN_THREADS = 64;
constexpr int KNN_MAX_K = 256;
// admission margin of the candidate scan, relative: 8 ulp of fp32 at the running k-th distance
constexpr float KNN_MARGIN = 1.0f + 0x1p-20f;

struct KnnLpParams {
  const float* src;
  const float* dst;
  int64_t n_in, n_out;
  int k;
  float theta_hi, theta_half;
};

// The topk comparator for the smallest values: NaN counts as larger than any number.
__device__ __forceinline__ bool knn_less(float x, float y) {
  return (!__builtin_isnan(x) && __builtin_isnan(y)) || x < y;
}

// Sift a value into the heap [0, len) (element j at hv[j * T]) from the hole at `hole`:
// the hole moves down along the larger child to a leaf, then the value moves up.
__device__ __forceinline__ void heap_adjust(float* hv, int32_t* hi, int hole, int len, float val, int32_t idx) {
  constexpr int T = KNN_THREADS;
  const int top = hole;
  int child = hole;
  while (child < (len - 1) / 2) {
    child = 2 * (child + 1);
    if (knn_less(hv[child * T], hv[(child - 1) * T])) --child;
    hv[hole * T] = hv[child * T];
    hi[hole * T] = hi[child * T];
    hole = child;
  }
  if ((len & 1) == 0 && child == (len - 2) / 2) {
    child = 2 * (child + 1);
    hv[hole * T] = hv[(child - 1) * T];
    hi[hole * T] = hi[(child - 1) * T];
    hole = child - 1;
  }
  int parent = (hole - 1) / 2;
  while (hole > top && knn_less(hv[parent * T], val)) {
    hv[hole * T] = hv[parent * T];
    hi[hole * T] = hi[parent * T];
    hole = parent;
    parent = (hole - 1) / 2;
  }
  hv[hole * T] = val;
  hi[hole * T] = idx;
}

// Squared distance of input i to the output at (r0, t0): |drho|^2 + |dtheta|^2 with the angle
// wrap, fp32 products and sum with no contraction (the build passes -ffp-contract=off): the
// same value on the host and on the GPU.
__device__ __forceinline__ float lp_sq(const float* src, int64_t i, float r0, float t0, float theta_hi,
                                       float theta_half) {
  const float dr = fabsf(src[2 * i] - r0);
  float dt = fabsf(src[2 * i + 1] - t0);
  if (dt > theta_half) dt = theta_hi - dt;
  return dr * dr + dt * dt;
}

// Heap in LDS of the first k (value, index) pairs, made a max-heap.
__device__ __forceinline__ void heap_make(float* hv, int32_t* hi, int k) {
  constexpr int T = KNN_THREADS;
  if (k < 2) return;
  for (int parent = (k - 2) / 2;; --parent) {
    heap_adjust(hv, hi, parent, k, hv[parent * T], hi[parent * T]);
    if (parent == 0) break;
  }
}

// Pass 1: the scan in index order with IEEE distances. Emits every input the exact heap
// (whatever rounding its square roots have, within a few ulp) could admit: the first k,
// then each input whose distance is below the running k-th smallest times (1 + 2^-20).
// Emitted as (index, squared distance dr*dr + dt*dt, exact in fp32 on any device).
__global__ __launch_bounds__(KNN_THREADS) void knn_lp_candidates_kernel(KnnLpParams p, int64_t cap,
                                                                        int32_t* cand_idx, float* cand_sq,
                                                                        int32_t* cand_n) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  constexpr int T = KNN_THREADS;
  const int t = threadIdx.x;
  const int64_t n = static_cast<int64_t>(blockIdx.x) * T + t;
  if (n >= p.n_out) return;                      // no block-wide synchronisation below
  float* hv = reinterpret_cast<float*>(smem) + t;
  int32_t* hi = reinterpret_cast<int32_t*>(smem + static_cast<size_t>(p.k) * T * sizeof(float)) + t;
  const float r0 = p.dst[2 * n], t0 = p.dst[2 * n + 1];
  const int k = p.k;
  int32_t* ci = cand_idx + n * cap;
  float* cs = cand_sq + n * cap;
  int64_t m = 0;
  for (int j = 0; j < k; ++j) {
    const float sq = lp_sq(p.src, j, r0, t0, p.theta_hi, p.theta_half);
    hv[j * T] = sqrtf(sq);
    hi[j * T] = j;
    ci[m] = j;
    cs[m] = sq;
    ++m;
  }
  heap_make(hv, hi, k);
  float top = hv[0];
  for (int64_t i = k; i < p.n_in; ++i) {
    const float sq = lp_sq(p.src, i, r0, t0, p.theta_hi, p.theta_half);
    const float d = sqrtf(sq);
    if (d < top * KNN_MARGIN) {
      if (m < cap) {
        ci[m] = static_cast<int32_t>(i);
        cs[m] = sq;
      }
      ++m;
    }
    if (knn_less(d, top)) {
      heap_adjust(hv, hi, 0, k, d, static_cast<int32_t>(i));
      top = hv[0];
    }
  }
  cand_n[n] = static_cast<int32_t>(m < INT32_MAX ? m : INT32_MAX);
}

// Pass 2: the exact heap selection over the candidates (in index order) with the distances
// the host rounded, then the heap sort; outputs in the k-major layout of knn_indices.
__global__ __launch_bounds__(KNN_THREADS) void knn_select_kernel(int64_t n_out, int k, int64_t cap,
                                                                 const int32_t* cand_idx, const float* cand_d,
                                                                 const int32_t* cand_n, int32_t* idx, float* dist) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  constexpr int T = KNN_THREADS;
  const int t = threadIdx.x;
  const int64_t n = static_cast<int64_t>(blockIdx.x) * T + t;
  if (n >= n_out) return;                        // no block-wide synchronisation below
  float* hv = reinterpret_cast<float*>(smem) + t;
  int32_t* hi = reinterpret_cast<int32_t*>(smem + static_cast<size_t>(k) * T * sizeof(float)) + t;
  const int32_t* ci = cand_idx + n * cap;
  const float* cd = cand_d + n * cap;
  const int64_t m = cand_n[n] < cap ? cand_n[n] : cap;
  for (int j = 0; j < k; ++j) {
    hv[j * T] = cd[j];
    hi[j * T] = ci[j];
  }
  heap_make(hv, hi, k);
  float top = hv[0];
  for (int64_t j = k; j < m; ++j) {
    const float d = cd[j];
    if (knn_less(d, top)) {
      heap_adjust(hv, hi, 0, k, d, ci[j]);
      top = hv[0];
    }
  }
  for (int last = k - 1; last >= 1; --last) {    // sort the heap: ascending
    const float v = hv[last * T];
    const int32_t ix = hi[last * T];
    hv[last * T] = hv[0];
    hi[last * T] = hi[0];
    heap_adjust(hv, hi, 0, last, v, ix);
  }
  for (int j = 0; j < k; ++j) {
    idx[j * n_out + n] = hi[j * T];
    dist[j * n_out + n] = hv[j * T];
  }
}

// Euclidean search (fovi/arch/knn.py:119-152 for isotropic cortical and visual-field points):
// the host builder's distances are torch's CPU cdist in its matrix-product form, whose rounding
// (|x|^2 + |y|^2 - 2 x.y summed by the BLAS kernel, then clamped and square-rooted) this kernel
// does not reproduce. So the scan runs on the direct form sum (x - y)^2, accurate to a few ulps,
// and emits every input whose squared distance lies within a margin of the running k-th
// smallest: the matrix-product form differs from the exact value by at most 16 ulps of
// (|x| + |y|)^2 (five products and sums, each rounded once), so margin = 2 * 2^-20 *
// (r_src + |y|)^2 with r_src the largest |x|, plus 2^-20 of the running value for the direct
// form's own rounding. An input outside the margin has a host value at or above the host's
// running k-th smallest, which the heap never admits (it admits strictly smaller values).
// Emits (index, direct squared distance); the host takes the distances of the candidates
// that can decide the result with its own cdist.
struct KnnEuParams {
  const float* src;
  const float* dst;
  int64_t n_in, n_out;
  int k, dim;
  float src_norm_max;
};

__device__ __forceinline__ float eu_sq(const float* src, int64_t i, const float* y, int dim) {
  float s = 0.0f;
  for (int d = 0; d < dim; ++d) {
    const float t = src[i * dim + d] - y[d];
    s = s + t * t;
  }
  return s;
}

__global__ __launch_bounds__(KNN_THREADS) void knn_eu_candidates_kernel(KnnEuParams p, int64_t cap,
                                                                        int32_t* cand_idx, float* cand_sq,
                                                                        int32_t* cand_n) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  constexpr int T = KNN_THREADS;
  const int t = threadIdx.x;
  const int64_t n = static_cast<int64_t>(blockIdx.x) * T + t;
  if (n >= p.n_out) return;                      // no block-wide synchronisation below
  float* hv = reinterpret_cast<float*>(smem) + t;
  int32_t* hi = reinterpret_cast<int32_t*>(smem + static_cast<size_t>(p.k) * T * sizeof(float)) + t;
  float y[3] = {0.0f, 0.0f, 0.0f};
  float yn = 0.0f;
  for (int d = 0; d < p.dim; ++d) {
    y[d] = p.dst[n * p.dim + d];
    yn = yn + y[d] * y[d];
  }
  const float reach = p.src_norm_max + sqrtf(yn);
  const float m2 = 2.0f * 0x1p-20f * reach * reach;
  const int k = p.k;
  int32_t* ci = cand_idx + n * cap;
  float* cs = cand_sq + n * cap;
  int64_t m = 0;
  for (int j = 0; j < k; ++j) {
    const float sq = eu_sq(p.src, j, y, p.dim);
    hv[j * T] = sq;
    hi[j * T] = j;
    ci[m] = j;
    cs[m] = sq;
    ++m;
  }
  heap_make(hv, hi, k);
  float top = hv[0];
  for (int64_t i = k; i < p.n_in; ++i) {
    const float sq = eu_sq(p.src, i, y, p.dim);
    if (sq < top + (m2 + top * 0x1p-20f)) {
      if (m < cap) {
        ci[m] = static_cast<int32_t>(i);
        cs[m] = sq;
      }
      ++m;
    }
    if (knn_less(sq, top)) {
      heap_adjust(hv, hi, 0, k, sq, static_cast<int32_t>(i));
      top = hv[0];
    }
  }
  cand_n[n] = static_cast<int32_t>(m < INT32_MAX ? m : INT32_MAX);
}

static int reserve_lds(const void* kernel, size_t lds, const char* what) {
  if (lds > 64 * 1024 &&
      reserve_dynamic_lds(kernel, lds) != hipSuccess) {
    set_error("%s: cannot reserve %zu bytes of LDS", what, lds);
    return 1;
  }
  return 0;
}

// ---------------------------------------------------------------------------
// Ref-slot assignment of every neighbour (KNNConvLayer.compute_local_rf,
// fovi/arch/knn.py:599-647), one wave per output point, candidate-and-verify:
// the kernel follows the reference's formulas in fp32 and flags each output
// point where some neighbour's nearest and second-nearest ref points lie
// within `tol`; the host recomputes the flagged points with the reference's
// own torch calls (their transcendental functions and the matrix-product
// cdist round differently from these), so the combined table is the host's.
//  * angle theta = atan2(y_j - y_n, x_j - x_n) on the visual-field points;
//  * radial distance r = cdist(cortical_n, cortical_j): the direct form
//    sqrt(sum (a - b)^2), or for k > 25 the matrix-product form torch's cdist
//    switches to, sqrt(max(|a|^2 + |b|^2 - 2 a.b, 0)); r = 0 for a padding
//    index (< 0), whose coordinates are the last point's (Python indexing);
//  * local point (r cos theta, r sin theta), min-max normalised over the
//    point's neighbours to 2 (p - lo) / (hi - lo + 1e-6) - 1;
//  * the nearest ref point (first index among equals), distances in the
//    direct form, or the matrix-product form for more than 25 output points.
// ---------------------------------------------------------------------------
constexpr int RF_LANES = 64;
constexpr int RF_PER_LANE = 4;   // k <= 256

struct RfParams {
  const float* src_cort;
  const float* src_cart;
  int64_t n_src;
  int dim;
  const float* out_cort;
  const float* out_cart;
  int64_t n_out;
  const int32_t* knn;
  int k;
  const float* ref;
  int V;
  int mm_radial, mm_ref;
  float tol;
  int32_t* slots;
  int32_t* flags;
};

// Radial distance and a bound on its difference from the host's value: the
// direct form differs by a few ulps of r; the matrix-product form by a few ulps
// of the terms it sums, which near r = 0 is sqrt of that (cancellation).
__device__ __forceinline__ float rf_radial(const float* a, const float* b, int dim, int mm, float* err) {
  if (!mm) {
    float s = 0.0f;
    for (int d = 0; d < dim; ++d) {
      const float t = a[d] - b[d];
      s = s + t * t;
    }
    const float r = sqrtf(s);
    *err = r * 0x1p-20f;
    return r;
  }
  float na = 0.0f, nb = 0.0f, dot = 0.0f;
  for (int d = 0; d < dim; ++d) {
    na = na + a[d] * a[d];
    nb = nb + b[d] * b[d];
    dot = dot + (-2.0f * a[d]) * b[d];
  }
  const float r = sqrtf(fmaxf(dot + na + nb, 0.0f));
  const float e2 = (na + nb + fabsf(dot)) * 0x1p-20f;
  *err = e2 / (r + sqrtf(e2));
  return r;
}

__global__ __launch_bounds__(RF_LANES) void local_rf_slots_kernel(RfParams p) {
  const int64_t n = blockIdx.x;
  const int lane = threadIdx.x;
  float oc[3] = {0.0f, 0.0f, 0.0f};
  for (int d = 0; d < p.dim; ++d) oc[d] = p.out_cort[n * p.dim + d];
  const float ox = p.out_cart[2 * n], oy = p.out_cart[2 * n + 1];
  float lx[RF_PER_LANE], ly[RF_PER_LANE];
  float mnx = __builtin_inff(), mny = __builtin_inff(), mxx = -__builtin_inff(), mxy = -__builtin_inff();
  float emax = 0.0f;
#pragma unroll
  for (int m = 0; m < RF_PER_LANE; ++m) {
    const int i = lane + RF_LANES * m;
    lx[m] = ly[m] = 0.0f;
    if (i >= p.k) continue;
    const int32_t j = p.knn[static_cast<int64_t>(i) * p.n_out + n];
    const int64_t jj = j < 0 ? p.n_src - 1 : j;
    float sc[3] = {0.0f, 0.0f, 0.0f};
    for (int d = 0; d < p.dim; ++d) sc[d] = p.src_cort[jj * p.dim + d];
    const float th = atan2f(p.src_cart[2 * jj + 1] - oy, p.src_cart[2 * jj] - ox);
    float er = 0.0f;
    float r = rf_radial(oc, sc, p.dim, p.mm_radial, &er);
    if (j < 0) r = er = 0.0f;
    lx[m] = r * cosf(th);
    ly[m] = r * sinf(th);
    // the angle and its cosine and sine differ from the host's by a few ulps
    emax = fmaxf(emax, er + r * 0x1p-19f);
    mnx = fminf(mnx, lx[m]); mxx = fmaxf(mxx, lx[m]);
    mny = fminf(mny, ly[m]); mxy = fmaxf(mxy, ly[m]);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    mnx = fminf(mnx, __shfl_xor(mnx, off)); mxx = fmaxf(mxx, __shfl_xor(mxx, off));
    mny = fminf(mny, __shfl_xor(mny, off)); mxy = fmaxf(mxy, __shfl_xor(mxy, off));
    emax = fmaxf(emax, __shfl_xor(emax, off));
  }
  const float dx = (mxx - mnx) + 1e-6f, dy = (mxy - mny) + 1e-6f;
  // an error e in the local points moves a normalised coordinate by at most
  // 8 e / span (the point, lo and hi each move); a distance comparison sees
  // twice the sum over both axes
  const float tol = p.tol + 16.0f * emax * (1.0f / dx + 1.0f / dy);
  bool near = !(tol < 0.5f);
#pragma unroll
  for (int m = 0; m < RF_PER_LANE; ++m) {
    const int i = lane + RF_LANES * m;
    if (i >= p.k) continue;
    const float x = (2.0f * (lx[m] - mnx)) / dx - 1.0f;
    const float y = (2.0f * (ly[m] - mny)) / dy - 1.0f;
    const float xn = x * x + y * y;
    float best = __builtin_inff(), second = __builtin_inff();
    int bv = 0;
    for (int v = 0; v < p.V; ++v) {
      const float rx = p.ref[2 * v], ry = p.ref[2 * v + 1];
      float dist;
      if (p.mm_ref) {
        dist = sqrtf(fmaxf((-2.0f * x) * rx + (-2.0f * y) * ry + xn + (rx * rx + ry * ry), 0.0f));
      } else {
        const float tx = x - rx, ty = y - ry;
        dist = sqrtf(tx * tx + ty * ty);
      }
      if (dist < best) {
        second = best;
        best = dist;
        bv = v;
      } else if (dist < second) {
        second = dist;
      }
    }
    p.slots[n * p.k + i] = bv;
    near |= !(second - best > tol);
  }
  const bool any = __builtin_amdgcn_ballot_w64(near) != 0;
  if (lane == 0) p.flags[n] = any ? 1 : 0;
}

}  // namespace
}  // namespace fovi

using namespace fovi;

extern "C" int fovi_local_rf_slots(const fovi_local_rf_args* a, void* stream) {
  clear_error();
  if (!a || !a->src_cortical || !a->src_cart || !a->out_cortical || !a->out_cart || !a->knn_idx || !a->ref ||
      !a->slots || !a->flags) {
    set_error("fovi_local_rf_slots: null pointer");
    return 1;
  }
  if (a->dim < 1 || a->dim > 3 || a->k < 1 || a->k > RF_LANES * RF_PER_LANE || a->n_ref < 1 ||
      a->n_ref > 65536 || a->n_out < 0 || a->n_src < 1 || !(a->tol >= 0.0f)) {
    set_error("fovi_local_rf_slots: need 1 <= dim <= 3, 1 <= k <= %d, 1 <= n_ref <= 65536, n_src >= 1, tol >= 0 "
              "(dim=%d k=%lld n_ref=%lld)", RF_LANES * RF_PER_LANE, a->dim, (long long)a->k, (long long)a->n_ref);
    return 1;
  }
  if (a->n_out == 0) return 0;
  if (a->n_out > INT32_MAX) { set_error("fovi_local_rf_slots: n_out too large"); return 1; }
  RfParams p;
  p.src_cort = a->src_cortical; p.src_cart = a->src_cart; p.n_src = a->n_src; p.dim = a->dim;
  p.out_cort = a->out_cortical; p.out_cart = a->out_cart; p.n_out = a->n_out;
  p.knn = a->knn_idx; p.k = static_cast<int>(a->k); p.ref = a->ref; p.V = static_cast<int>(a->n_ref);
  p.mm_radial = a->k > 25; p.mm_ref = a->n_out > 25 || a->n_ref > 25; p.tol = a->tol;
  p.slots = a->slots; p.flags = a->flags;
  hipLaunchKernelGGL(local_rf_slots_kernel, dim3(static_cast<unsigned>(a->n_out)), dim3(RF_LANES), 0,
                     static_cast<hipStream_t>(stream), p);
  return check_launch("fovi_local_rf_slots");
}

static bool knn_sizes_ok(int64_t k, int64_t n_in, int64_t n_out, const char* what) {
  if (k < 1 || k > KNN_MAX_K || n_out < 0 || n_in < k * 64 || n_in > INT32_MAX) {
    set_error("%s: need 1 <= k <= %d, k * 64 <= n_in < 2^31 (k=%lld, n_in=%lld, n_out=%lld)", what, KNN_MAX_K,
              (long long)k, (long long)n_in, (long long)n_out);
    return false;
  }
  return true;
}

extern "C" int fovi_knn_logpolar_candidates(const fovi_knn_logpolar_args* a, void* stream) {
  clear_error();
  if (!a || !a->src || !a->dst || !a->cand_idx || !a->cand_sq || !a->cand_n) {
    set_error("fovi_knn_logpolar_candidates: null pointer");
    return 1;
  }
  if (!knn_sizes_ok(a->k, a->n_in, a->n_out, "fovi_knn_logpolar_candidates")) return 1;
  if (a->cap < a->k) {
    set_error("fovi_knn_logpolar_candidates: cap %lld < k %lld", (long long)a->cap, (long long)a->k);
    return 1;
  }
  if (a->n_out == 0) return 0;
  KnnLpParams p;
  p.src = a->src; p.dst = a->dst; p.n_in = a->n_in; p.n_out = a->n_out; p.k = static_cast<int>(a->k);
  p.theta_hi = a->theta_hi; p.theta_half = a->theta_half;
  const size_t lds = static_cast<size_t>(p.k) * KNN_THREADS * (sizeof(float) + sizeof(int32_t));
  if (reserve_lds(reinterpret_cast<const void*>(&knn_lp_candidates_kernel), lds, "fovi_knn_logpolar_candidates"))
    return 1;
  const unsigned blocks = static_cast<unsigned>((a->n_out + KNN_THREADS - 1) / KNN_THREADS);
  hipLaunchKernelGGL(knn_lp_candidates_kernel, dim3(blocks), dim3(KNN_THREADS), lds,
                     static_cast<hipStream_t>(stream), p, a->cap, a->cand_idx, a->cand_sq, a->cand_n);
  return check_launch("fovi_knn_logpolar_candidates");
}

extern "C" int fovi_knn_euclid_candidates(const fovi_knn_euclid_args* a, void* stream) {
  clear_error();
  if (!a || !a->src || !a->dst || !a->cand_idx || !a->cand_sq || !a->cand_n) {
    set_error("fovi_knn_euclid_candidates: null pointer");
    return 1;
  }
  if (!knn_sizes_ok(a->k, a->n_in, a->n_out, "fovi_knn_euclid_candidates")) return 1;
  if (a->dim < 1 || a->dim > 3 || !(a->src_norm_max >= 0.0f) || !__builtin_isfinite(a->src_norm_max)) {
    set_error("fovi_knn_euclid_candidates: need 1 <= dim <= 3 and a finite src_norm_max >= 0 (dim=%d)", a->dim);
    return 1;
  }
  if (a->cap < a->k) {
    set_error("fovi_knn_euclid_candidates: cap %lld < k %lld", (long long)a->cap, (long long)a->k);
    return 1;
  }
  if (a->n_out == 0) return 0;
  KnnEuParams p;
  p.src = a->src; p.dst = a->dst; p.n_in = a->n_in; p.n_out = a->n_out; p.k = static_cast<int>(a->k);
  p.dim = a->dim; p.src_norm_max = a->src_norm_max;
  const size_t lds = static_cast<size_t>(p.k) * KNN_THREADS * (sizeof(float) + sizeof(int32_t));
  if (reserve_lds(reinterpret_cast<const void*>(&knn_eu_candidates_kernel), lds, "fovi_knn_euclid_candidates"))
    return 1;
  const unsigned blocks = static_cast<unsigned>((a->n_out + KNN_THREADS - 1) / KNN_THREADS);
  hipLaunchKernelGGL(knn_eu_candidates_kernel, dim3(blocks), dim3(KNN_THREADS), lds,
                     static_cast<hipStream_t>(stream), p, a->cap, a->cand_idx, a->cand_sq, a->cand_n);
  return check_launch("fovi_knn_euclid_candidates");
}

extern "C" int fovi_knn_select(const fovi_knn_select_args* a, void* stream) {
  clear_error();
  if (!a || !a->cand_idx || !a->cand_d || !a->cand_n || !a->idx || !a->dist) {
    set_error("fovi_knn_select: null pointer");
    return 1;
  }
  if (a->k < 1 || a->k > KNN_MAX_K || a->n_out < 0 || a->cap < a->k) {
    set_error("fovi_knn_select: need 1 <= k <= %d and cap >= k (k=%lld, cap=%lld)", KNN_MAX_K, (long long)a->k,
              (long long)a->cap);
    return 1;
  }
  if (a->n_out == 0) return 0;
  const int k = static_cast<int>(a->k);
  const size_t lds = static_cast<size_t>(k) * KNN_THREADS * (sizeof(float) + sizeof(int32_t));
  if (reserve_lds(reinterpret_cast<const void*>(&knn_select_kernel), lds, "fovi_knn_select")) return 1;
  const unsigned blocks = static_cast<unsigned>((a->n_out + KNN_THREADS - 1) / KNN_THREADS);
  hipLaunchKernelGGL(knn_select_kernel, dim3(blocks), dim3(KNN_THREADS), lds, static_cast<hipStream_t>(stream),
                     a->n_out, k, a->cap, a->cand_idx, a->cand_d, a->cand_n, a->idx, a->dist);
  return check_launch("fovi_knn_select");
}
