/*
 * fovi_hip.h - C-ABI of the MI355X (gfx950) foveated sampler and kNN-conv forward.
 *
 * The reference (nblauch/fovi) is pure Python and exposes no FFI: its
 * plug-in boundary is the nn.Module surface of GridSampler/RetinalTransform
 * and KNNConvLayer. Each entry point below replaces the ATen call sites of one
 * stage of that surface; the Python modules in fovi_amd/ bind them with ctypes.
 *
 * Conventions
 *   - All memory is caller-owned device memory (HBM); no entry point
 *     allocates. Strides are in elements, not bytes.
 *   - Calls are asynchronous on `stream` (a hipStream_t passed as void*,
 *     NULL = default stream), stateless and reentrant.
 *   - Return 0 on success, non-zero on error; the message is in
 *     fovi_last_error() (thread-local). No C++ exception crosses the ABI.
 */
#ifndef FOVI_HIP_H
#define FOVI_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FOVI_ABI_VERSION 33

enum fovi_dtype { FOVI_F32 = 0, FOVI_BF16 = 1, FOVI_F8E4M3 = 2 };
enum fovi_interp { FOVI_NEAREST = 0, FOVI_BILINEAR = 1 };
enum fovi_padding { FOVI_PAD_ZEROS = 0, FOVI_PAD_BORDER = 1 };
enum fovi_activation { FOVI_ACT_NONE = 0, FOVI_ACT_RELU = 1 };
enum fovi_weight_layout { FOVI_W_ROWS = 0, FOVI_W_MFMA = 1 };

/* Version of this header the library was built from (FOVI_ABI_VERSION). */
int fovi_abi_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* fovi_last_error(void);

/*
 * Foveated sampler: fixation transform + grid-sample of image views onto
 * sensor points.
 *
 * Replaces GridSampler.forward (fovi/sensing/samplers.py:91-112), i.e.
 * transform_sampling_grid (fovi/sensing/coords.py:590-642) followed by
 * torch.nn.functional.grid_sample(img, grid, mode, align_corners=False)
 * (samplers.py:108), for every fixation view in one launch (the per-fixation
 * loop of fovi/sensing/policies.py:268-270 becomes the view axis).
 *
 * View v samples image view_image[v] (view v if view_image is NULL) at
 *   gx = 2 * (grid[p].x * half_w[v] + fix_loc[v].w * W) / W - 1
 *   gy = 2 * (grid[p].y * half_h[v] + fix_loc[v].h * H) / H - 1
 * evaluated in fp32 in that order (fp64 for the multiply by the half size
 * when fix_half_wide != 0, as the reference does for float fixation sizes).
 */
typedef struct fovi_sampler_args {
  const void* img;            /* image batch, dtype img_dtype (F32 or BF16) */
  int32_t img_dtype;
  int32_t reserved0;
  int64_t n_img, channels, height, width;
  int64_t img_stride[4];      /* image, channel, row, column */
  const float* grid;          /* [n_points, 2] sensor grid (x, -y) in [-1, 1] */
  int64_t n_points;
  int64_t n_views;
  const float* fix_loc;       /* [n_views, 2] (h, w) fixation centre in [0, 1] */
  const double* fix_half;     /* [n_views, 2] (h, w) half fixation size in pixels */
  int32_t fix_half_wide;      /* 0: half size is used as fp32; 1: fp64 multiply */
  int32_t ring_len;           /* processing-order hint: points per ring when the grid is
                                 ring-major (point = ring * ring_len + angle), else 0;
                                 results do not depend on it */
  const int32_t* view_image;  /* [n_views] or NULL */
  int32_t mode;               /* fovi_interp */
  int32_t padding;            /* fovi_padding */
  void* out;                  /* dtype out_dtype (F32 or BF16) */
  int32_t out_dtype;
  int32_t reserved2;
  int64_t out_stride[3];      /* view, channel, point */
  float* grid_out;            /* optional [n_views, n_points, 2] (gx, gy), or NULL */
} fovi_sampler_args;

int fovi_sampler_fwd(const fovi_sampler_args* args, void* stream);

/*
 * kNN-convolution forward.
 *
 * Replaces KNNConvLayer.forward (fovi/arch/knn.py:538-557): the zero pad
 * column + gather (_pad_and_gather_knns, knn.py:484-503), the one-hot
 * local-RF einsum (_apply_local_rf, knn.py:505-526) and F.linear with the
 * [c_out, c_in * n_ref] weight (knn.py:555) become one fused launch:
 *
 *   y[b, o, n] = bias[o] + sum_v sum_c A[b, n, v, c] * w[o, v * c_in + c]
 *   A[b, n, v, c] = sum over the neighbours j of n in ref slot v of x[b, c, j]
 *
 * Neighbour lists are slot-major CSR per output point:
 *   slot_ptr[n * n_ref + v] = (begin << 16) | count, and the input indices
 *   are nbr_sorted[n * k + begin + i], i < count (k <= 32767, so every entry
 *   is a non-negative int32).
 * The weight is the packed form made by fovi_knnconv_pack_weight: row o holds
 * the reduction axis in slot-major order (v * c_in + c), zero padded to
 * k_pad (a multiple of 64).
 *
 * x_dtype/w_dtype: F32/F32 (fp32 parity path) or BF16/BF16 (MFMA path) or
 * F8E4M3/F8E4M3 (MFMA path; y = x_scale * w_scale[o] * sum(q_x * q_w) + bias).
 * The fp8 path has no counterpart in the reference. It needs channels-last
 * input rows (x_stride[1] == 1, 16-byte aligned), c_in % 64 == 0 and the tile
 * tables. Each slot with two or more neighbours is summed in fp32 and rounded
 * once more to e4m3 (round to nearest even) before the MFMA, so the activation
 * scale must keep sums of up to max(count) quantized values below 448 (the
 * headroom argument of fovi_quantize_e4m3).
 *
 * Optional tile tables (all NULL to leave them out) select the kernel that
 * copies each tile's input rows into LDS: output points are cut into tiles
 * of tile_points (256) consecutive points; tile t reads only input points
 * tile_lo[t] .. tile_lo[t] + tile_span[t] - 1 (max_span = max tile_span);
 * tile_ent[n * n_ref + v] = (first << 16) | (count << 8) | begin and
 * tile_nbr[n * k + begin + i] = input index - tile_lo[t] (first = the i = 0
 * entry; zero_row when count is 0), same lists as the CSR tables. With
 * tile_coll / tile_coll_n also given they select the staged-row kernel for
 * channels-last bf16 input when the rows fit in LDS (k <= 255).
 * tile_coll[t * n_ref * tile_points + v * tile_points + i], i < tile_coll_n[t * n_ref + v],
 * lists the tile rows whose slot v has two or more neighbours (decreasing
 * count); zero_row (>= every tile_span) is the LDS row index standing for an
 * empty slot. With these the kernel reads single-neighbour slots straight
 * from the staged rows and only sums the listed ones.
 */
typedef struct fovi_knnconv_args {
  const void* x;
  int32_t x_dtype;
  int32_t reserved0;
  int64_t batch, c_in, n_in;
  int64_t x_stride[3];        /* batch, channel, point */
  int64_t n_out, k, n_ref;
  const int32_t* slot_ptr;    /* [n_out, n_ref] */
  const int32_t* nbr_sorted;  /* [n_out, k] */
  const void* w;              /* packed [c_out, k_pad] (FOVI_W_ROWS) or fragment order (FOVI_W_MFMA) */
  int32_t w_dtype;
  int32_t w_layout;           /* fovi_weight_layout: FOVI_W_MFMA (from fovi_knnconv_pack_weight_mfma)
                                 selects the wide-layer bf16 kernel and needs c_in % 32 == 0,
                                 channels-last 16-byte input rows and the tile tables */
  int64_t c_out, k_pad;
  const float* bias;          /* [c_out] or NULL */
  const float* w_scale;       /* [c_out] (F8E4M3 only) */
  float x_scale;              /* (F8E4M3 only) */
  int32_t reserved2;
  void* y;
  int32_t y_dtype;            /* F32 or BF16 */
  int32_t reserved3;
  int64_t y_stride[3];        /* batch, out channel, point */
  const int32_t* tile_lo;     /* [n_tiles] or NULL */
  const int32_t* tile_span;   /* [n_tiles] or NULL */
  const uint32_t* tile_ent;   /* [n_tiles * tile_points, n_ref] or NULL */
  const uint16_t* tile_nbr;   /* [n_tiles * tile_points, k] or NULL */
  int32_t tile_points;
  int32_t max_span;
  const uint8_t* tile_coll;   /* [n_tiles, n_ref, tile_points] or NULL */
  const int32_t* tile_coll_n; /* [n_tiles, n_ref] or NULL */
  int32_t zero_row;
  int32_t activation;         /* fovi_activation applied to y (after bias) */
  int32_t w_c_slot;           /* channels per slot in the packed weight (0 = c_in); 4 or 8
                                 with c_in <= w_c_slot selects the few-channel kernels, which
                                 need channels-last input rows padded to w_c_slot channels */
  int32_t reserved5;
  void* workspace;            /* optional caller-owned device scratch (16-byte aligned); with
                                 >= batch * n_out * k_pad * 2 bytes the few-channel path runs
                                 in two passes (slot sums into it, then a dense GEMM) */
  int64_t workspace_bytes;
  const float* x_scale_dev;   /* (F8E4M3 only) device copy of the activation scale, e.g. the one
                                 fovi_quantize_e4m3 writes; used instead of x_scale when non-NULL */
  /* Tables of the wide-layer kernel (w_layout = FOVI_W_MFMA), in its LDS order and in the
   * slot visit order (position p visits slot slot_order[p], see fovi_knnconv_pack_weight_mfma).
   * 64-byte rows are named by LDS offsets u(r): byte offsets off(r) (wide_units = 0), or in
   * 16-byte units off(r) / 16 (wide_units = 1, needed past 1023 staged rows): staged row r
   * (relative to tile_lo[t]) is at byte off(r) = 64 r + 16 g(r), g(r) = (bit1(r) ^ bit3(r)) |
   * bit2(r) << 1 (16-byte part q at off(r) ^ 16 q); zero_row must be at most 1024. Heavy-sum
   * row h is at byte 64 (zero_row + 1 + h). Collision-tile destinations are in bytes.
   *   tile_src[(t * n_ref + p) * tile_points + r]: the row (unit offset) the MFMA reads for
   *     position p of output row r: the neighbour's staged row (one neighbour), the zero row
   *     (none), the row's heavy sum (more than 6), or 0xFFFF (2 to 6: summed by the stream);
   *   tile_cent[(t * cent_stride + i) * 4 + 0..3], i in [tile_coll_off[t * coll_off_stride + p],
   *     tile_coll_off[t * coll_off_stride + p + 1]): one 16-byte entry per (position p, row
   *     with 2 to 6 neighbours), decreasing count within a position: word 0 = destination
   *     ((p % nb) * 16384 + off(row), bytes) | count << 16, nb = 4 collision tiles when the
   *     kernel's tile layout with four fits 160 KB (64 (zero_row + 1 + heavy_stride) rounded
   *     up to 128, + (256 nb + 1) 64 + 512 n_ref + 4 coll_off_stride + 16 cent_stride +
   *     8 heavy_stride + 2 hlist_stride bytes), else 3; words 1-3 = u() of the staged
   *     rows of neighbours 1-6 in list order, two 16-bit halves each (the zero row past the
   *     count);
   *   tile_heavy[(t * heavy_stride + h) * 2 + 0..1]: heavy entry h (more than 6 neighbours):
   *     word 0 = its heavy-sum row's unit offset | count << 16 (count 0: padding); word 1 =
   *     the index of its first neighbour in tile_hlist[t * hlist_stride ...] (u() values, in
   *     list order). */
  const uint16_t* tile_src;
  const int32_t* tile_coll_off;
  const uint32_t* tile_cent;
  int32_t coll_off_stride;    /* multiple of 4, > n_ref */
  int32_t cent_stride;        /* entries per tile, >= 1 */
  const uint32_t* tile_heavy;
  const uint16_t* tile_hlist;
  int32_t heavy_stride;       /* heavy entries per tile, even, >= 2 */
  int32_t hlist_stride;       /* multiple of 8, >= 8 */
  /* Tables of the fused few-channel kernel (the few-channel path: bf16, w_c_slot = 4 or 8 >=
   * c_in, channels-last rows padded to w_c_slot; all NULL to leave it out). Output points are
   * cut into tiles of fc_tile_points consecutive points, each run by a workgroup of fc_threads
   * threads with chunks of fc_chunk reduction columns: (64, 256, 32), (128, 512, 64) or
   * (256, 512, 64). Tile t stages input rows fc_lo[t] .. fc_lo[t] + fc_span[t] - 1 (S rows 0 ..
   * span - 1) and a zero row fc_zero_row (>= every span, < 65536). The reduction runs in
   * k_pad / fc_chunk chunks of fc_chunk / w_c_slot slots (at most 4096 slots). The kernel
   * clears chunk c's A tile and writes its non-empty (row, slot) sums from (sum, neighbour)
   * pairs: thread j of tile t reads the fc_pairs (8 or 16) words
   * fc_item[((t * n_chunks + c) * fc_threads + j) * fc_pairs ..] (16-byte aligned), each
   *   S row of the neighbour (bits 0-15; the zero row for an unused word) | target << 16
   *   (12 bits) | partial << 28 | last << 29.
   * A run of consecutive words of one thread is one sum: added in fp32 in word (list) order
   * from +0 and written at the word with the last bit, rounded once to bf16, to A entry
   * `target` (an index in units of 2 * w_c_slot bytes of the A tile, whose rows of 2 *
   * fc_chunk bytes hold the chunk's slots in order with 16-byte part q of row r at part
   * q ^ ((r >> 1) & 7) for 128-byte rows, q ^ g(r) for 64-byte rows, g(r) = (bit1(r) ^
   * bit3(r)) | bit2(r) << 1), or, with the partial bit, as its fp32 partial sum to index target
   * (below fc_pmax <= 4095) of the chunk's partial sums. A (row, slot) of up to 8 neighbours is
   * one run; a longer one is one partial run per group of 8 consecutive neighbours and one
   * combine entry. Combine entries (t, c), fc_comb[fc_comb_off[t * n_chunks + c] ..
   * fc_comb_off[t * n_chunks + c + 1]) (at most fc_threads), each destination | m << 12 | p0
   * << 20 with destination = row * (fc_chunk / w_c_slot) + slot, write to A the partials p0 ..
   * p0 + m - 1 added in order and rounded once. The slot sums (this grouped order) and the
   * MFMA order equal the two-pass path's. */
  const int32_t* fc_lo;
  const int32_t* fc_span;
  const uint32_t* fc_item;
  int32_t fc_threads;         /* threads of the kernel's workgroup the pair table is dealt to: 256 or 512 */
  int32_t fc_chunk;           /* reduction columns per chunk: 32 or 64 */
  const void* reserved7;      /* NULL */
  int32_t fc_tile_points;
  int32_t fc_zero_row;
  int32_t fc_pairs;           /* pair words per thread and chunk in fc_item: 8 or 16 */
  int32_t wide_units;         /* 1: the wide-layer tables (tile_src, tile_cent words 1-3, tile_heavy
                                 word 0, tile_hlist) name staged and heavy rows in 16-byte units
                                 (needed past 1023 staged rows); 0: in bytes */
  const uint32_t* fc_comb;    /* the fused few-channel kernel's combine entries (above) */
  const int32_t* fc_comb_off;
  int32_t fc_pmax;
  int32_t wide_tiles;         /* (w_layout = FOVI_W_MFMA) the collision-tile count nb the wide-layer
                                 tables were built for (tile_cent word 0 destinations); must equal
                                 fovi_knnconv_wide_tiles() of the table sizes, else the call fails */
  /*
   * The view-major few-channel kernel (optional; NULL vm_idx: not used). It takes bf16 input
   * whose rows of one point for all images are adjacent, x_stride = (w_c_slot, 1, row stride
   * s, a multiple of w_c_slot): element (b, c, n) at x[n * s + b * w_c_slot + c], channels
   * >= c_in zero or ignored by zero weight columns, (n_in + 1) * s * 2 < 2^31, bf16 output.
   * Reduction step j is columns 16 j .. 16 j + 15 of the row-packed weight. Per output point
   * p, rounds vm_off[p] .. vm_off[p + 1] - 1 (R of them, a multiple of 8): half h of the MFMA
   * lanes (h = 0: columns 8 h .. 8 h + 7 of a step) adds, in round q, input row
   * vm_idx[2 * vm_off[p] + h * R + q] (rows >= n_in read as zeros) to a group sum, and the
   * round's event vm_ev[vm_off[p] + q] (bit 0: add the group sum to the slot sum; bit 1: end
   * of the step's first phase, w_c_slot = 4; bit 2: end of the step; bit 3 (at a step's end):
   * half 0's second slot and half 1's first change halves; bit 4 (at phase ends): half 1 holds
   * its slots in the other order; bits 5-15 at a step's end: the point's next active step,
   * 0x7FF none) closes sums as knn_tables.view_major_tables describes; vm_j0[p] is the
   * point's first active step (-1: none). vm_w holds the weight
   * in fragment order: 16 bytes per lane at ((j * vm_nb + b) * 64 + lane) * 16, lane l
   * holding columns 16 j + 8 (l / 32) .. + 7 of output channel 32 b + l % 32 (zero past c_out);
   * vm_nb >= c_out / 32 blocks, a multiple of vm_cb (1, 2, 3, 4 or 6 blocks per wave).
   * Sums, rounding and MFMA order are the two-pass path's: outputs equal it bit for bit for
   * finite weights. Tables and weight 16-byte aligned.
   */
  const uint32_t* vm_idx;
  const uint16_t* vm_ev;
  const int32_t* vm_off;
  const int32_t* vm_j0;
  const void* vm_w;
  int32_t vm_nb;
  int32_t vm_cb;
} fovi_knnconv_args;

int fovi_knnconv_fwd(const fovi_knnconv_args* args, void* stream);

/*
 * The wide-layer kernel's LDS layout for tables of these sizes (the fields of
 * fovi_knnconv_args with the same names): returns the number of collision
 * tiles nb it uses, 4 when that layout fits 160 KB of LDS, else 3, and writes
 * the layout's LDS bytes to *lds_bytes when lds_bytes is not NULL (fits when
 * <= 160 KB). Host only, no device call; returns 0 (with an error message)
 * unless 0 <= n_ref < 2^16 and the other sizes lie in [0, 2^20]. The tables' builder takes nb from here, so builder and
 * kernel share one rule. No counterpart in the reference.
 */
int fovi_knnconv_wide_tiles(int64_t n_ref, int32_t zero_row, int32_t coll_off_stride, int32_t cent_stride,
                            int32_t heavy_stride, int32_t hlist_stride, int64_t* lds_bytes);

/*
 * fovi_knnconv_fwd for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * No counterpart in the reference, whose forward allocates its intermediates
 * (fovi/arch/knn.py:484-557).
 *
 * Runs what fovi_knnconv_fwd runs for the same arguments, except that the
 * few-channel two-pass path (bf16, a weight packed with w_c_slot = 4 or 8
 * channels per slot >= c_in, channels-last input rows padded to w_c_slot) keeps
 * its slot-sum rows in the library's own scratch instead of a caller
 * workspace: a static 64 MiB device array per GPU, held until the process
 * ends, filled and read one chunk of whole images at a time (the same kernels
 * per image, so results equal fovi_knnconv_fwd's with a workspace bit for
 * bit). The other paths use no scratch. Calls no hipMalloc or hipFree.
 *   - workspace must be NULL and workspace_bytes 0;
 *   - one image's slot sums, n_out * k_pad * 2 bytes, must fit the 64 MiB
 *     scratch, or the call fails with an error (no launch);
 *   - every call on a GPU shares that GPU's scratch. Calls are ordered in host
 *     call order: each call's stream waits for a per-device event the previous
 *     call recorded after its last use of the scratch (created with the
 *     scratch's address at the first call on a device), and calls from several
 *     threads take a lock. Calls enqueued under stream capture are not ordered
 *     this way: the caller's graph must order them, and its replays must not
 *     overlap other calls on that GPU. Each chunk's rows are written in full
 *     before they are read, so nothing needs clearing between calls.
 */
int fovi_knnconv_fwd_noalloc(const fovi_knnconv_args* args, void* stream);

/*
 * The kernel path the last successful fovi_knnconv_fwd call on this thread
 * took ("" before any, or after a failed call): "f32", "bf16 v5", "fp8 v5",
 * "fp8 rows", "bf16 v4", "bf16 v2", "bf16 few-channel view-major", "bf16 few-channel fused", "bf16 few-channel",
 * "bf16 few-channel two-pass", "bf16 generic (rows)" or "bf16 generic". Diagnostics only (no
 * counterpart in the reference, whose forward is a fixed op sequence,
 * fovi/arch/knn.py:538-557); tests use it to check which kernel a layer
 * geometry selects.
 */
const char* fovi_knnconv_last_path(void);

/*
 * Packs the reference weight layout for fovi_knnconv_fwd.
 *
 * w_ref is KNNConvLayer.weight, fp32 [c_out, c_in * n_ref] with reduction
 * index c * n_ref + v (fovi/arch/knn.py:462,524). The packed output is
 * [c_out, k_pad] with index v * c_slot + c (c_slot >= c_in channels per slot,
 * 0 = c_in; channels >= c_in are zero), zero padded, in out_dtype. For
 * F8E4M3, row o is divided by w_scale[o] and rounded to OCP e4m3 (RNE,
 * saturating to +-448).
 */
int fovi_knnconv_pack_weight(const float* w_ref, int64_t c_out, int64_t c_in, int64_t n_ref,
                             void* w_packed, int32_t out_dtype, int64_t k_pad, int64_t c_slot,
                             const float* w_scale, void* stream);

/*
 * Weight in MFMA-fragment order for the wide-layer kernels (w_layout =
 * FOVI_W_MFMA). Same source as fovi_knnconv_pack_weight (w_ref = KNNConvLayer.weight,
 * fp32 [c_out, c_in * n_ref], index c * n_ref + v, fovi/arch/knn.py:462,524);
 * the output is fovi_knnconv_weight_mfma_elems(c_out, c_in, n_ref) elements of
 * out_dtype in 1 KB fragments f = (it * ncb + cb) * 2 + h, ncb = 8 * ceil(c_out / 256),
 * it = chunk * n_ref + p. Lane l of fragment f holds w_ref[o = 32 * cb + l % 32][c * n_ref + v]
 * (zero for o >= c_out) at
 *   BF16 (32-channel chunks, c_in % 32 == 0): 8 * l + e, c % 32 = 16 * h + 8 * (l / 32) + e;
 *   F8E4M3 (64-channel chunks, c_in % 64 == 0): 16 * l + e, c % 64 = 32 * (l / 32) + 16 * h + e,
 *     the value divided by w_scale[o] and rounded to OCP e4m3 (RNE, saturating).
 * slot_order (device int32 [n_ref], or NULL for 0, 1, ...) is the order in
 * which the kernel visits the slots of a channel chunk: position p holds slot
 * v = slot_order[p]. The wide-layer tables (tile_src, tile_cent, tile_coll_off)
 * must be laid out in the same order. w_scale (device fp32 [c_out]) is read
 * for F8E4M3 only.
 */
int64_t fovi_knnconv_weight_mfma_elems(int64_t c_out, int64_t c_in, int64_t n_ref);
int fovi_knnconv_pack_weight_mfma(const float* w_ref, int64_t c_out, int64_t c_in, int64_t n_ref,
                                  void* w_frag, int32_t out_dtype, const int32_t* slot_order,
                                  const float* w_scale, void* stream);

/*
 * Per-tensor OCP e4m3 quantization of activations for the fp8 kNN-conv path
 * (no counterpart in the reference, which has no fp8 path; callers are
 * quantized inference pipelines feeding fovi_knnconv_fwd with F8E4M3 input).
 *
 *   amax  = max |x| over the [batch, channels, points] view
 *   scale = amax * headroom / 448 in fp32 (1 when amax is 0)
 *   q[b, c, n] = e4m3(x[b, c, n] / scale)   (fp32 division, round to nearest
 *                                            even, saturating to +-448)
 *
 * headroom (>= 1, a power of two) leaves room below 448 for sums of up to
 * `headroom` quantized values. scale_out[0] receives the scale (device
 * memory). With scale_in non-NULL the amax pass is skipped and *scale_in (a
 * calibrated device scale) is used; scale_out may then be NULL. amax_work is
 * one float of caller device memory, overwritten. Strides are in elements of
 * the [batch, channel, point] views of x and q.
 */
typedef struct fovi_quantize_args {
  const void* x;
  int32_t x_dtype;            /* F32 or BF16 */
  int32_t reserved0;
  int64_t batch, channels, points;
  int64_t x_stride[3];
  uint8_t* q;                 /* e4m3 bytes */
  int64_t q_stride[3];
  float headroom;
  int32_t reserved1;
  const float* scale_in;      /* optional */
  float* scale_out;
  float* amax_work;
} fovi_quantize_args;

int fovi_quantize_e4m3(const fovi_quantize_args* args, void* stream);

/*
 * kNN pooling forward: replaces KNNPoolingLayer.forward (fovi/arch/knn.py:345-394).
 *
 *   y[b, c, n] = reduce over j < k of x[b, c, nbr[n * k + j]]
 *
 * nbr is the reference's knn_indices_pad_token transposed to [n_out, k]; an
 * index >= n_in is the pad token, whose feature is NaN (knn.py:357). NaN
 * features (pad or input) are handled as the reference does:
 *   FOVI_POOL_MAX:      NaN -> -inf, then max (knn.py:371-373);
 *   FOVI_POOL_AVG:      mean over the non-NaN features (torch.nanmean; NaN when none);
 *   FOVI_POOL_SUM:      sum over the non-NaN features (torch.nansum);
 *   FOVI_POOL_GAUSSIAN: weights[n * k + j] zeroed where the feature is NaN,
 *                       divided by (their sum + 1e-8), then sum of feature x
 *                       weight over the non-NaN features (knn.py:376-389).
 * Arithmetic in fp32, one rounding to y_dtype. x and y: F32 or BF16, any
 * element strides [batch, channel, point]; the fast path is channels-last
 * rows (x_stride[1] == 1, 16-byte aligned rows).
 */
enum fovi_pool_mode { FOVI_POOL_MAX = 0, FOVI_POOL_AVG = 1, FOVI_POOL_SUM = 2, FOVI_POOL_GAUSSIAN = 3 };

typedef struct fovi_knnpool_args {
  const void* x;
  int32_t x_dtype;
  int32_t mode;               /* fovi_pool_mode */
  int64_t batch, channels, n_in;
  int64_t x_stride[3];
  const int32_t* nbr;         /* [n_out, k] */
  const float* weights;       /* [n_out, k], FOVI_POOL_GAUSSIAN only */
  int64_t n_out, k;
  void* y;
  int32_t y_dtype;
  int32_t reserved0;
  int64_t y_stride[3];
} fovi_knnpool_args;

int fovi_knnpool_fwd(const fovi_knnpool_args* args, void* stream);

/*
 * kNN pooling backward: the input gradient autograd forms through
 * KNNPoolingLayer.forward (fovi/arch/knn.py:345-394):
 *   dx[b, c, i] = sum over the (n, j) with nbr[n * k + j] == i of coef * dy[b, c, n],
 * and 0 where x[b, c, i] is NaN (the reference's NaN masks carry no gradient):
 *   FOVI_POOL_MAX:      coef = 1 at the first position j of the maximum of
 *                       (b, c, n) (NaN read as -inf), as torch.max over a dim;
 *   FOVI_POOL_AVG:      coef = 1 / (number of non-NaN features of (b, c, n));
 *   FOVI_POOL_SUM:      coef = 1;
 *   FOVI_POOL_GAUSSIAN: coef = weights[n * k + j] / (sum of the non-NaN
 *                       features' weights + 1e-8).
 * inv_ptr [n_in + 1] / inv: per input i, the entries n * k + j whose neighbour
 * is i (pad tokens excluded), any order. state: fp32 workspace
 * [batch * n_out * channels] (all modes but FOVI_POOL_SUM). fp32 sums, one
 * rounding to dx_dtype. x, dy, dx: F32 or BF16, any element strides.
 */
typedef struct fovi_knnpool_bwd_args {
  const void* x;
  int32_t x_dtype;
  int32_t mode;               /* fovi_pool_mode */
  int64_t batch, channels, n_in;
  int64_t x_stride[3];
  const int32_t* nbr;         /* [n_out, k] */
  const float* weights;       /* [n_out, k], FOVI_POOL_GAUSSIAN only */
  int64_t n_out, k;
  const void* dy;
  int32_t dy_dtype;
  int32_t dx_dtype;
  int64_t dy_stride[3];
  const int32_t* inv_ptr;     /* [n_in + 1] */
  const int32_t* inv;
  float* state;
  void* dx;
  int64_t dx_stride[3];
} fovi_knnpool_bwd_args;

int fovi_knnpool_bwd(const fovi_knnpool_bwd_args* args, void* stream);

/*
 * kNN-conv backward, the two gather kernels around its two GEMMs (the
 * gradients autograd forms through KNNConvLayer.forward, fovi/arch/knn.py:484-557;
 * the reference has no hand-written backward):
 *
 *   fovi_knnconv_slotsum: the reduction matrix of the forward,
 *     a[(b * n_out + n) * n_ref * c_in + v * c_in + c] = sum over the inputs i
 *     in slot v of output n (slot_ptr / nbr_sorted, as fovi_knnconv_args) of
 *     x[b, c, i], fp32 sums in list order rounded once to a_dtype. With it,
 *     dW (slot-major columns) = dy^T a.
 *   fovi_knnconv_bwd_x: the input gradient from g = dy W (slot-major columns),
 *     dx[b, c, i] = sum over the entries e = n * n_ref + v of input i's inverse
 *     list (inv[inv_ptr[i] .. inv_ptr[i + 1]]: every (output, slot) that reads
 *     input i) of g[(b * n_out + n) * n_ref * c_in + v * c_in + c], fp32 sums
 *     rounded once to dx_dtype.
 * x, a, g, dx: F32 or BF16; a and g dense row-major; x and dx any element
 * strides [batch, channel, point].
 */
typedef struct fovi_knnconv_slotsum_args {
  const void* x;
  int32_t x_dtype;
  int32_t a_dtype;
  int64_t batch, c_in, n_in;
  int64_t x_stride[3];
  int64_t n_out, k, n_ref;
  const int32_t* slot_ptr;    /* [n_out, n_ref] */
  const int32_t* nbr_sorted;  /* [n_out, k] */
  void* a;                    /* [batch * n_out, n_ref * c_in] */
} fovi_knnconv_slotsum_args;

int fovi_knnconv_slotsum(const fovi_knnconv_slotsum_args* args, void* stream);

typedef struct fovi_knnconv_bwd_x_args {
  const void* g;              /* [batch * n_out, n_ref * c_in] */
  int32_t g_dtype;
  int32_t dx_dtype;
  int64_t batch, c_in, n_in, n_out, n_ref;
  const int32_t* inv_ptr;     /* [n_in + 1] */
  const int32_t* inv;         /* entries n * n_ref + v */
  void* dx;
  int64_t dx_stride[3];
} fovi_knnconv_bwd_x_args;

int fovi_knnconv_bwd_x(const fovi_knnconv_bwd_x_args* args, void* stream);

/*
 * kNN search on the wrapped log-polar cortical lattice, the table of
 * KNNBaseLayer._compute_knns / _compute_euclidean_distances_batched
 * (fovi/arch/knn.py:23-57,101-152) for sample_cortex=True on log-polar
 * coordinates, in two GPU passes around one host step:
 *
 *   fovi_knn_logpolar_candidates: per output point n, the scan over the
 *     inputs in index order of the squared distance
 *       sq(i, n) = |rho_i - rho_n|^2 + dth^2, dth = |theta_i - theta_n|,
 *       replaced by theta_hi - dth when dth > theta_half,
 *     in fp32 with no contraction, on the min-max normalised coordinates
 *     (src, dst: [n, 2] rows (rho, theta)). Writes cand_idx[n * cap + j] and
 *     cand_sq[n * cap + j] for the first k inputs and every later input whose
 *     IEEE distance sqrt(sq) is below (1 + 2^-20) times the running k-th
 *     smallest, in index order, and their number to cand_n[n] (entries past
 *     cap are counted, not written: cand_n[n] > cap means the row overflowed).
 *   (host) cand_d = sqrt(cand_sq) with the host builder's own square root for
 *     the candidates that can decide the selection, any square root for the rest.
 *   fovi_knn_select: per output point, the k smallest of its candidates in
 *     the order torch's CPU topk(largest=False) returns them for k * 64 <= n_in
 *     (a size-k max-heap over the candidates in index order that admits
 *     strictly smaller values, then heap-sorted): idx [k, n_out] (k-major, as
 *     knn_indices) and dist [k, n_out]. Reads min(cand_n[n], cap) candidates.
 *
 * Needs 1 <= k <= 256, k * 64 <= n_in < 2^31 and cap >= k.
 */
typedef struct fovi_knn_logpolar_args {
  const float* src;           /* [n_in, 2] */
  const float* dst;           /* [n_out, 2] */
  int64_t n_in, n_out, k;
  float theta_hi, theta_half;
  int64_t cap;                /* candidates per output row */
  int32_t* cand_idx;          /* [n_out, cap] */
  float* cand_sq;             /* [n_out, cap] */
  int32_t* cand_n;            /* [n_out] */
} fovi_knn_logpolar_args;

int fovi_knn_logpolar_candidates(const fovi_knn_logpolar_args* args, void* stream);

/*
 * Candidate pass of the Euclidean kNN search (fovi/arch/knn.py:119-152, the
 * torch.cdist + topk branch: isotropic cortical points, visual-field points),
 * for the host builder's results bit for bit together with a host step and
 * fovi_knn_select:
 *   fovi_knn_euclid_candidates: per output point n, the scan over the inputs
 *     in index order of the direct squared distance sum_d (src_i,d - dst_n,d)^2
 *     in fp32 (src: [n_in, dim], dst: [n_out, dim]), writing cand_idx[n * cap + j]
 *     for the first k inputs and every later input whose squared distance is
 *     below the running k-th smallest plus 2^-19 (src_norm_max + |dst_n|)^2 plus
 *     2^-20 of that running value (a bound on the difference from the
 *     matrix-product form torch's cdist rounds in; src_norm_max >= every |src_i|),
 *     with that squared distance in cand_sq[n * cap + j], in index order, and
 *     their number to cand_n[n] (entries past cap are counted, not written).
 *   (host) the distances of the candidates that can decide the selection (the
 *     k smallest within the margin, and any two within the margin of each
 *     other) with the host's own cdist; the square root of cand_sq for the rest.
 *   fovi_knn_select: the heap selection over them (below).
 * Needs 1 <= k <= 256, k * 64 <= n_in < 2^31, 1 <= dim <= 3 and cap >= k.
 */
typedef struct fovi_knn_euclid_args {
  const float* src;           /* [n_in, dim] */
  const float* dst;           /* [n_out, dim] */
  int64_t n_in, n_out, k;
  int32_t dim;
  float src_norm_max;
  int64_t cap;                /* candidates per output row */
  int32_t* cand_idx;          /* [n_out, cap] */
  float* cand_sq;             /* [n_out, cap] direct squared distances */
  int32_t* cand_n;            /* [n_out] */
} fovi_knn_euclid_args;

int fovi_knn_euclid_candidates(const fovi_knn_euclid_args* args, void* stream);

typedef struct fovi_knn_select_args {
  int64_t n_out, k, cap;
  const int32_t* cand_idx;    /* [n_out, cap] */
  const float* cand_d;        /* [n_out, cap] */
  const int32_t* cand_n;      /* [n_out] */
  int32_t* idx;               /* [k, n_out] */
  float* dist;                /* [k, n_out] */
} fovi_knn_select_args;

int fovi_knn_select(const fovi_knn_select_args* args, void* stream);

/*
 * Ref slot of every neighbour, replacing the host loop of
 * KNNConvLayer.compute_local_rf (fovi/arch/knn.py:599-647, sample_cortex=True):
 * per output point n and neighbour i (j = knn_idx[i * n_out + n], k-major as
 * knn_indices; j < 0 reads point n_src - 1 and has radius 0):
 *   theta = atan2(y_j - y_n, x_j - x_n) on the visual-field points (cart),
 *   r = |cortical_n - cortical_j| (the matrix-product form torch's cdist
 *   uses for k > 25), local = (r cos theta, r sin theta), min-max normalised
 *   over the point's neighbours to 2 (p - lo) / (hi - lo + 1e-6) - 1, and
 *   slots[n * k + i] = the nearest ref point (first among equals; the
 *   matrix-product form for n_out > 25 or n_ref > 25).
 * fp32 throughout; flags[n] = 1 where, for some neighbour, the nearest and
 * second-nearest ref points lie within tol plus a bound on the kernel's
 * difference from the host's arithmetic: those points' slots must be
 * recomputed on the host (candidate and verify); flags[n] = 0 means the
 * slots equal the host's. Needs 1 <= dim <= 3, 1 <= k <= 256,
 * 1 <= n_ref <= 65536, tol >= 0.
 */
typedef struct fovi_local_rf_args {
  const float* src_cortical;  /* [n_src, dim] */
  const float* src_cart;      /* [n_src, 2] */
  int64_t n_src;
  int dim;
  const float* out_cortical;  /* [n_out, dim] */
  const float* out_cart;      /* [n_out, 2] */
  int64_t n_out;
  const int32_t* knn_idx;     /* [k, n_out] */
  int64_t k;
  const float* ref;           /* [n_ref, 2] */
  int64_t n_ref;
  float tol;
  int32_t* slots;             /* [n_out, k] */
  int32_t* flags;             /* [n_out] */
} fovi_local_rf_args;

int fovi_local_rf_slots(const fovi_local_rf_args* args, void* stream);

/*
 * Weight gradient of the kNN convolution without the slot-sum matrix (the
 * gradient autograd forms for F.linear's weight through knn.py:521-555):
 *   dw[o * c_in * n_ref + c * n_ref + v] = sum over images b and over the
 *   pairs (n, i) of slot v of dy[b, n, o] * x[b, i, c],
 * fp32 accumulation of bf16 products, fp32 output in the reference weight
 * layout. pairs holds (n, i) int32 pairs in n_chunks * n_ref segments,
 * segment q * n_ref + v at [pair_off[q * n_ref + v], pair_off[q * n_ref + v + 1])
 * holding slot v's pairs of one chunk of output points (the layer: 256
 * consecutive points per chunk, output order), optionally padded with
 * (-1, -1) entries (the layer pads to multiples of 64, the kernel's step). One workgroup takes one segment for
 * images_per_group consecutive images; the workspace holds its partial tile
 * (fovi_knnconv_dw_workspace_bytes). x and
 * dy bf16 channels-last (element strides [batch, channel, point] with channel
 * stride 1, rows 16-byte aligned); c_in and c_out multiples of 8.
 */
typedef struct fovi_knnconv_dw_args {
  const void* x;              /* bf16 [batch, c_in, n_in] (strides below) */
  int64_t x_stride[3];
  const void* dy;             /* bf16 [batch, c_out, n_out] */
  int64_t dy_stride[3];
  int64_t batch, c_in, c_out, n_in, n_out, n_ref;
  const int32_t* pair_off;    /* [n_chunks * n_ref + 1] */
  const int32_t* pairs;       /* [2 * pair_off[n_chunks * n_ref]] */
  int64_t n_chunks;
  int64_t images_per_group;
  void* workspace;
  int64_t workspace_bytes;
  float* dw;                  /* [c_out, c_in * n_ref] */
} fovi_knnconv_dw_args;

int64_t fovi_knnconv_dw_workspace_bytes(int64_t batch, int64_t images_per_group, int64_t n_chunks, int64_t c_in,
                                        int64_t c_out, int64_t n_ref);
int fovi_knnconv_dw(const fovi_knnconv_dw_args* args, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FOVI_HIP_H */
