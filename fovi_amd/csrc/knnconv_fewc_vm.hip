// kNN-convolution forward, bf16, for layers with few input channels (c_in <= 8, input rows
// padded to CP = 4 or 8 channels) whose input is view-major: the rows of one input point for
// all images are adjacent in memory ([N_in, B, CP], x_stride = (CP, 1, row stride)). The
// sampler can write this layout, and it lets the kernel skip the input staging of the
// point-major kernel (knnconv_fewc.hip): an MFMA block's 32 rows are 32 images of ONE output
// point, so
//  * a reduction step (16 columns = 16 / CP slots) in which the point has no neighbour is
//    skipped for all 32 rows (C4 patch embedding: 24 of 64 steps), and
//  * lane (image i, half h) gathers its A operand itself: one 8- or 16-byte buffer load per
//    neighbour, the 32 images of a half reading 32 adjacent rows (256 or 512 contiguous bytes).
// GEMM view: rows = (image, point), columns = output channels, reduction = (slot v, channel c)
// at column v * CP + c as in the row-packed weight. A wave owns 32 images x CB blocks of 32
// output channels of one point; a workgroup of 4 waves owns 128 images, and the grid covers
// (image block, point, channel group).
//  * The host table (knn_tables.view_major_tables) gives each point a stream of rounds. In a
//    round every lane adds one input row (its half's neighbour, or a padding row past the
//    input, which the buffer range check reads as zeros) to an fp32 group sum; events of the
//    round (uniform, read with scalar loads) close a group of FC_GROUP (added to the slot
//    sum), end phase A (the slot sum rounded once to bf16 into A operand dwords 0-1) or end the
//    step (the last sum into the remaining dwords, then CB MFMAs 32x32x16 in ascending column
//    order, and the next active step's weight fragments are loaded). With four-channel rows a
//    step's two phases pair a slot of each half; the table picks per point and step the
//    pairing with the fewest rounds (C4 patch embedding: 201 -> 168 rounds per point), and
//    the step's events say where the sums go: VM_Q, half 1 writes phase A's sum into its
//    second slot; VM_X, half 0's second slot and half 1's first change halves at the step's
//    end (v_permlane32_swap), so the MFMA operands are those of the natural pairing. The slot sums are the
//    two-pass path's (slotsum_kernel) bit for bit; a skipped step's columns are zero in its A
//    rows, whose products add +0 to an accumulator that is never -0, so the outputs equal the
//    dense GEMM's for finite weights.
//  * The input rows of the next 8 rounds are loaded while the current 8 are summed; the
//    weight fragments (the MFMA B operand, 1 KB per block and step, in fragment order) one
//    step ahead.
//  * Epilogue: bias and ReLU, a per-wave transposition through LDS, 16-byte stores of
//    channels-last output rows.
#include "knnconv_internal.h"

namespace fovi {

namespace {

constexpr uint32_t VM_G = 1u, VM_P = 2u, VM_S = 4u, VM_X = 8u, VM_Q = 16u;
constexpr uint32_t VM_JSHIFT = 5u, VM_J_NONE = 0x7FFu;
constexpr int VM_WAVES = 4;                  // waves (groups of 32 images) per workgroup
constexpr int VM_IMAGES = VM_WAVES * 32;

typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));

struct VmTables {
  const uint32_t* idx;   // per point: half 0's input row per round, then half 1's
  const uint16_t* ev;    // per point: one event word per round
  const int32_t* off;    // [n_out + 1] first round of each point (multiples of 8)
  const int32_t* j0;     // [n_out] first active step (-1: none)
  const u32x4* w;        // weight fragments ((j * nb + b) * 64 + lane)
  int nb;                // 32-column blocks in w
};

template <int CP> struct VmRow;
template <> struct VmRow<4> {
  typedef u32x2v T;
  static __device__ __forceinline__ T load(__amdgpu_buffer_rsrc_t rs, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b64(rs, off, 0, 0);
  }
  template <int NCH>
  static __device__ __forceinline__ void acc(float* a, T v) {
    a[0] += __uint_as_float(v[0] << 16); a[1] += __uint_as_float(v[0] & 0xffff0000u);
    a[2] += __uint_as_float(v[1] << 16);
    if constexpr (NCH == 4) a[3] += __uint_as_float(v[1] & 0xffff0000u);
  }
};
template <> struct VmRow<8> {
  typedef u32x4 T;
  static __device__ __forceinline__ T load(__amdgpu_buffer_rsrc_t rs, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0);
  }
  template <int NCH>
  static __device__ __forceinline__ void acc(float* a, T v) {
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      a[2 * w] += __uint_as_float(v[w] << 16);
      a[2 * w + 1] += __uint_as_float(v[w] & 0xffff0000u);
    }
  }
};

// NCH: channels summed per row; CP (channels >= c_in cleared by masks in the packed sums) or 3
// (c_in = 3 of CP = 4: the fourth channel is neither summed nor packed, its bf16 is +0)
template <int CP, int CB, int NCH>
__global__ __launch_bounds__(VM_WAVES * 64, 2) void knnconv_fewc_vm_kernel(KnnParams p, VmTables t, int n_cg,
                                                                          int64_t total, int64_t padded,
                                                                          int vec_out) {
  typedef VmRow<CP> R;
  typedef typename R::T RowT;
  constexpr int WC = CB * 32 + 8;             // LDS row of the epilogue (halfwords, padded)
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

  const int64_t lb = xcd_tile(blockIdx.x, padded);
  if (lb >= total) return;
  const int cg = static_cast<int>(lb % n_cg);
  const int64_t rest = lb / n_cg;
  const int64_t tok = rest % p.Nout;
  const int64_t vb = rest / p.Nout;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int h = lane >> 5;
  const bool h1 = h != 0;
  const int64_t v0 = vb * VM_IMAGES + wave * 32;     // the wave's first image
  if (v0 >= p.B) return;                            // no barrier follows: whole waves may leave
  const uint32_t row_bytes = static_cast<uint32_t>(p.xs2) * 2u;
  // input rows 0 .. Nin - 1; an offset at or past Nin rows reads zeros
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<void*>(p.x), static_cast<short>(0), static_cast<int>(static_cast<uint32_t>(p.Nin) * row_bytes),
      0x00020000);
  // lanes of images >= B read another row's bytes (or zeros); their outputs are not stored
  const uint32_t img_off = static_cast<uint32_t>(v0 + (lane & 31)) * (CP * 2u);

  const int r0 = t.off[tok];
  const int nch = (t.off[tok + 1] - r0) / 8;
  const uint32_t* ix = t.idx + 2 * static_cast<int64_t>(r0) + h * (nch * 8);
  const uint16_t* ev = t.ev + r0;
  const int cb0 = cg * CB;

  f32x16 acc[CB];
#pragma unroll
  for (int b = 0; b < CB; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[b][r] = 0.0f;
  u32x4 wf[CB];
  auto load_w = [&](int j) {
    const u32x4* src = t.w + (static_cast<int64_t>(j) * t.nb + cb0) * 64 + lane;
#pragma unroll
    for (int b = 0; b < CB; ++b) wf[b] = src[b * 64];
  };
  if (nch > 0) load_w(t.j0[tok]);

  float part[CP], sum[CP];
#pragma unroll
  for (int c = 0; c < CP; ++c) { part[c] = 0.0f; sum[c] = 0.0f; }
  constexpr bool MASK = NCH == CP;
  // channels >= c_in of the padded rows are cleared in the packed sums (whatever they hold:
  // the sums are per channel, so a NaN there stays in its own column)
  uint32_t cm[CP / 2];
#pragma unroll
  for (int w = 0; w < CP / 2; ++w)
    cm[w] = (2 * w < p.C ? 0x0000ffffu : 0u) | (2 * w + 1 < p.C ? 0xffff0000u : 0u);
  uint32_t a0 = 0u, a1 = 0u, a2 = 0u, a3 = 0u;      // the step's A operand dwords

  // one round: add this lane's row to the group sum, then the round's events (uniform)
  auto round = [&](const RowT& x, uint32_t e) {
    R::template acc<NCH>(part, x);
    if (e & 7u) {
      if (e & (VM_P | VM_S)) {
        // the slot sum: the groups' sums added in order (a branch on whether the phase has
        // more than one group, to use a lone group's sum as it is, cost C4 5%)
        float v[CP];
#pragma unroll
        for (int c = 0; c < NCH; ++c) { v[c] = sum[c] + part[c]; sum[c] = 0.0f; part[c] = 0.0f; }
        if constexpr (CP == 4) {
          // phase A's slot into dwords 0-1, phase B's into 2-3; in half 1 the other way round
          // under VM_Q (selects: no indexed registers)
          uint32_t lo = cvt_pk_bf16(v[0], v[1]), hi = cvt_pk_bf16(v[2], NCH == 4 ? v[3] : 0.0f);
          if constexpr (MASK) { lo &= cm[0]; hi &= cm[1]; }
          const bool first = ((e & VM_P) != 0) != (h1 && (e & VM_Q) != 0);
          a0 = first ? lo : a0; a1 = first ? hi : a1;
          a2 = first ? a2 : lo; a3 = first ? a3 : hi;
        } else {
          a0 = cvt_pk_bf16(v[0], v[1]) & cm[0]; a1 = cvt_pk_bf16(v[2], v[3]) & cm[1];
          a2 = cvt_pk_bf16(v[4], v[5]) & cm[2]; a3 = cvt_pk_bf16(v[6], v[7]) & cm[3];
        }
      } else {
        // a group of FC_GROUP closes inside the phase
#pragma unroll
        for (int c = 0; c < NCH; ++c) { sum[c] += part[c]; part[c] = 0.0f; }
      }
      if (e & VM_S) {
        if constexpr (CP == 4) {
          if (e & VM_X) {   // half 0's second slot and half 1's first change halves
            const auto s0 = __builtin_amdgcn_permlane32_swap(a0, a2, false, false);
            const auto s1 = __builtin_amdgcn_permlane32_swap(a1, a3, false, false);
            a0 = s0[0]; a2 = s0[1]; a1 = s1[0]; a3 = s1[1];
          }
        }
        const bf16x8 a = __builtin_bit_cast(bf16x8, u32x4{a0, a1, a2, a3});
#pragma unroll
        for (int b = 0; b < CB; ++b)
          acc[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, __builtin_bit_cast(bf16x8, wf[b]), acc[b], 0, 0, 0);
        a0 = a1 = a2 = a3 = 0u;
        // unconditional (the last step loads step 0's fragments again): a branch here cost
        // C4 4%
        const uint32_t jn = e >> VM_JSHIFT;
        load_w(jn != VM_J_NONE ? static_cast<int>(jn) : 0);
      }
    }
  };

  u32x4 in0 = {0u, 0u, 0u, 0u}, in1 = {0u, 0u, 0u, 0u};   // input rows of the next chunk's rounds
  auto load_idx = [&](int c) {
    const u32x4* s = reinterpret_cast<const u32x4*>(ix + c * 8);
    in0 = s[0];
    in1 = s[1];
  };
  auto issue_rows = [&](RowT (&x)[8]) {
#pragma unroll
    for (int u = 0; u < 4; ++u) x[u] = R::load(rs, __umul24(in0[u], row_bytes) + img_off);
#pragma unroll
    for (int u = 0; u < 4; ++u) x[4 + u] = R::load(rs, __umul24(in1[u], row_bytes) + img_off);
  };
  // chunk c: its rows are in cur; the next chunk's rows are issued into nxt first,
  // unconditionally where the caller knows they exist (then the compiler counts the loads in
  // flight exactly at every wait; loads in a branch make it wait for all of them)
  auto chunk = [&](int c, RowT (&cur)[8], RowT (&nxt)[8], bool inside) __attribute__((always_inline)) {
    if (inside) {
      issue_rows(nxt);
      load_idx(c + 2);
    } else if (c + 1 < nch) {
      issue_rows(nxt);
      if (c + 2 < nch) load_idx(c + 2);
    }
    const u32x4 e4 = *reinterpret_cast<const u32x4*>(ev + c * 8);
#pragma unroll
    for (int u = 0; u < 8; ++u) round(cur[u], (e4[u >> 1] >> ((u & 1) * 16)) & 0xffffu);
  };

  RowT xa[8], xb[8];
  if (nch > 0) {
    load_idx(0);
    issue_rows(xa);
    if (nch > 1) load_idx(1);
  }
  // chunk pairs whose prefetches stay inside the point's rounds, then the last ones (C4 -5%;
  // prefetching past the rounds everywhere, with out-of-range rows, cost C2 layer 1 4%)
  int c = 0;
  for (; c + 3 < nch; c += 2) {
    chunk(c, xa, xb, true);
    chunk(c + 1, xb, xa, true);
  }
  for (; c < nch; c += 2) {
    chunk(c, xa, xb, false);
    if (c + 1 < nch) chunk(c + 1, xb, xa, false);
  }

  // Epilogue: y = acc + bias (ReLU optional), channels-last rows of images v0 .. v0 + 31
  float bo[CB];
#pragma unroll
  for (int b = 0; b < CB; ++b) {
    const int64_t o = (cb0 + b) * 32 + (lane & 31);
    bo[b] = (p.bias && o < p.Cout) ? p.bias[o] : 0.0f;
  }
  uint16_t* y = static_cast<uint16_t*>(p.y) + tok * p.ys2;
  if (vec_out) {
    uint16_t* E = reinterpret_cast<uint16_t*>(smem) + wave * 32 * WC;
#pragma unroll
    for (int b = 0; b < CB; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = 8 * (r >> 2) + 4 * h + (r & 3);
        E[row * WC + b * 32 + (lane & 31)] = f32_to_bf16_bits(epilogue(acc[b][r] + bo[b], p.relu));
      }
    __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0): this wave's LDS writes are done
    __builtin_amdgcn_wave_barrier();
    constexpr int PPR = CB * 4;           // 16-byte pieces per image row
#pragma unroll
    for (int k = 0; k < 32 * PPR / 64; ++k) {
      const int piece = k * 64 + lane;
      const int row = piece / PPR, part8 = piece - row * PPR;
      const int64_t img = v0 + row;
      const int64_t o = cb0 * 32 + part8 * 8;
      if (img < p.B && o < p.Cout)
        *reinterpret_cast<u32x4*>(y + img * p.ys0 + o) = *reinterpret_cast<const u32x4*>(&E[row * WC + part8 * 8]);
    }
    return;
  }
#pragma unroll
  for (int b = 0; b < CB; ++b) {
    const int64_t o = (cb0 + b) * 32 + (lane & 31);
    if (o >= p.Cout) continue;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t img = v0 + 8 * (r >> 2) + 4 * h + (r & 3);
      if (img < p.B) Elem<uint16_t>::store(y + img * p.ys0 + o * p.ys1, epilogue(acc[b][r] + bo[b], p.relu));
    }
  }
}

template <int CP, int CB, int NCH>
int launch_vm(const KnnParams& p, const VmTables& t, int n_cg, int vec_out, hipStream_t s) {
  const int64_t n_vb = (p.B + VM_IMAGES - 1) / VM_IMAGES;
  const int64_t total = n_vb * p.Nout * n_cg;
  const int64_t padded = (total + 7) / 8 * 8;
  if (padded > 0x7fffffff) return 0;
  const size_t lds = static_cast<size_t>(VM_WAVES) * 32 * (CB * 32 + 8) * 2;
  hipLaunchKernelGGL((knnconv_fewc_vm_kernel<CP, CB, NCH>), dim3(static_cast<unsigned>(padded)), dim3(VM_WAVES * 64),
                     lds, s, p, t, n_cg, total, padded, vec_out);
  return 1;
}

template <int CP, int NCH>
int launch_vm_cb(const KnnParams& p, const VmTables& t, int cb, int n_cg, int vec_out, hipStream_t s) {
  switch (cb) {
    case 1: return launch_vm<CP, 1, NCH>(p, t, n_cg, vec_out, s);
    case 2: return launch_vm<CP, 2, NCH>(p, t, n_cg, vec_out, s);
    case 3: return launch_vm<CP, 3, NCH>(p, t, n_cg, vec_out, s);
    case 4: return launch_vm<CP, 4, NCH>(p, t, n_cg, vec_out, s);
    case 6: return launch_vm<CP, 6, NCH>(p, t, n_cg, vec_out, s);
  }
  return 0;
}

}  // namespace

// 1 if launched, 0 if the view-major kernel does not take this call (caller falls back).
int launch_knnconv_fewc_vm(const KnnParams& p, const fovi_knnconv_args* a, int cp, hipStream_t s) {
  if (!a->vm_idx || !a->vm_ev || !a->vm_off || !a->vm_j0 || !a->vm_w || a->y_dtype != FOVI_BF16) return 0;
  if (p.xs0 != cp || p.xs1 != 1 || p.xs2 % cp != 0 || p.xs2 < cp) return 0;
  const int cb = a->vm_cb;
  if ((cb != 1 && cb != 2 && cb != 3 && cb != 4 && cb != 6) || a->vm_nb <= 0 || a->vm_nb % cb != 0 ||
      a->vm_nb * 32 < p.Cout || a->k_pad % 16 != 0)
    return 0;
  // 32-bit buffer offsets: every row (and a padding row index up to n_in) times the row stride
  const uint64_t row_bytes = static_cast<uint64_t>(p.xs2) * 2u;
  if ((static_cast<uint64_t>(p.Nin) + 1) * row_bytes >= (uint64_t(1) << 31) ||
      static_cast<uint64_t>(p.B + VM_IMAGES) * cp * 2 >= (uint64_t(1) << 31) || p.Nin >= (int64_t(1) << 24) ||
      row_bytes >= (uint64_t(1) << 24))
    return 0;
  if ((reinterpret_cast<uintptr_t>(p.x) % (2 * cp)) != 0 || (reinterpret_cast<uintptr_t>(a->vm_idx) % 16) != 0 ||
      (reinterpret_cast<uintptr_t>(a->vm_ev) % 16) != 0 || (reinterpret_cast<uintptr_t>(a->vm_w) % 16) != 0)
    return 0;
  VmTables t;
  t.idx = a->vm_idx; t.ev = a->vm_ev; t.off = a->vm_off; t.j0 = a->vm_j0;
  t.w = static_cast<const u32x4*>(a->vm_w); t.nb = a->vm_nb;
  const int n_cg = a->vm_nb / cb;
  const int vec_out = p.ys1 == 1 && p.ys2 % 8 == 0 && p.ys0 % 8 == 0 && p.Cout % 8 == 0 &&
                      reinterpret_cast<uintptr_t>(p.y) % 16 == 0;
  if (cp == 8) return launch_vm_cb<8, 8>(p, t, cb, n_cg, vec_out, s);
  return p.C == 3 ? launch_vm_cb<4, 3>(p, t, cb, n_cg, vec_out, s) : launch_vm_cb<4, 4>(p, t, cb, n_cg, vec_out, s);
}

}  // namespace fovi
