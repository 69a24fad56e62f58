/*
 * drama3_moe.h -- C ABI of the MI355X (gfx950) packed FP8 top-8 MoE step.
 *
 * Every entry point takes raw device pointers, sizes and strides (in
 * elements) and a hipStream_t passed as `void *stream` (NULL = legacy default
 * stream).  Nothing here allocates or frees memory, synchronises the stream
 * or copies device data to the host, so every call is hipGraph-capturable.
 * Calls are re-entrant: the library keeps no mutable global state besides a
 * thread-local error message, except d3_decode_step_static, whose static
 * device scratch is shared by every call on a GPU.
 *
 * Data types:   bf16 = uint16_t bit patterns;  fp8 = uint8_t OCP e4m3fn codes;
 *               fp32 block scales = float, one per 128 x 128 weight block or
 *               per 128 contiguous activation elements.
 * Weight layout (reference src/drama3/kernels.py:290-318):
 *               w13 [E, 2I, H] fp8 rows [gate; up],  s13 [E, 2I/128, H/128]
 *               w2  [E, H, I]  fp8,                  s2  [E, H/128, I/128]
 *               The fp8 codes may instead be given in the fragment-major
 *               layout of d3_pack_expert_weights (same size, scales
 *               unchanged), selected by a weight_layout argument.
 * Device row counts: wherever `row_count` appears, a non-NULL pointer names an
 * int32 on the device holding the live number of rows (<= the host `rows`
 * capacity); rows at or beyond it are left untouched.  NULL means all `rows`.
 * Empty batches: the elementwise and dense entry points (route, quantize_rows,
 * prepare_moe_input, combine_*, add_norm, silu_mul, dense_bf16) accept
 * rows = 0 with NULL buffers, launch nothing and return D3_OK; their shape
 * arguments are still checked.
 *
 * Return value: D3_OK or a D3_ERR_* code; d3_last_error() describes the
 * failure of the last call made on the calling thread.
 */
#ifndef DRAMA3_MOE_H
#define DRAMA3_MOE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define D3_OK 0
#define D3_ERR_INVALID_ARGUMENT 1 /* shape / stride / pointer contract violated */
#define D3_ERR_UNSUPPORTED 2      /* shape outside the compiled kernel set */
#define D3_ERR_HIP 3              /* a HIP runtime call failed */

#define D3_DTYPE_BF16 0
#define D3_DTYPE_F32 1
#define D3_DTYPE_I32 2
#define D3_DTYPE_I64 3

/* Expert weight layouts accepted by the expert GEMM entry points. */
#define D3_LAYOUT_REFERENCE 0 /* w [E, N, K] row-major, as the checkpoint stores it */
#define D3_LAYOUT_FRAGMENT 1  /* fragment-major, produced by d3_pack_expert_weights */

/*
 * Self-check of the e4m3 conversion (no counterpart in the reference).
 * Every quantiser of this library converts clamped fp32 values with the
 * gfx950 instruction v_cvt_pk_fp8_f32; the reference's bytes are the
 * round-to-nearest-even e4m3fn cast (src/drama3/moe_input.py:24-27).  For
 * the fp32 bit patterns [first, first + count) (multiples of 4, inside
 * 2^32), each clamped to [-448, 448], the instruction's byte is compared with
 * the software conversion in every byte position of the packed word;
 * result[0] += mismatches, result[1] = min(result[1], first bad pattern).
 * The caller initialises result to {0, 0xffffffff}.
 */
int d3_check_e4m3_conversion(uint64_t first, uint64_t count, uint32_t *result, void *stream);

/*
 * Device self-check of the arithmetic shortcuts of the quantisers and the
 * SwiGLU requantisation (no counterpart in the reference: it shows that the
 * shortcuts give the IEEE results the reference's rule moe_input.py:24-27
 * asks for, and bounds the sigmoid of its silu (kernels.py:392-394) against
 * the float64 sigmoid).  Over the fp32 bit patterns
 * [first, first + count):
 *   kind 0: hardware bf16 rounding (v_cvt_pk_bf16_f32) against the software
 *           round-to-nearest-even (NaN patterns skipped);
 *   kind 1: hardware reciprocal + one Newton-Raphson step against 1.0f / d
 *           (patterns inside [2^-43, 2^126));
 *   kind 2: division by `scale` through its reciprocal + one residual
 *           correction against v / scale, for +v and -v (finite patterns):
 *           quotients from 2^-12 up bit for bit, all by e4m3 code;
 *   kind 3: the sigmoid 1 / (1 + exp(-g)) of the SwiGLU (hardware
 *           exponential of a split product, Newton-corrected reciprocal)
 *           against the float64 sigmoid rounded to fp32: a mismatch is more
 *           than `scale` ulps apart where the reference is normal, or a
 *           result not below 2^-125 where it is not (NaN patterns skipped);
 *   kind 4: the group scale max(m, 1e-10) / 448 through a constant
 *           reciprocal + one residual correction against the IEEE division
 *           (non-negative patterns up to +inf);
 *   kind 5: kind 3 over the bf16 inputs: g = pattern << 16 for the patterns
 *           [first, first + count) inside [0, 2^16).
 * result[0] += mismatches, result[1] = min(result[1], first bad pattern);
 * the caller initialises result to {0, 0xffffffff}.
 */
int d3_check_epilogue_arithmetic(int32_t kind, uint64_t first, uint64_t count, float scale,
                                 uint32_t *result, void *stream);

/* Version of this ABI (bumped on any signature change). */
int d3_abi_version(void);

/* Message for the last failed call on this thread ("" after success). */
const char *d3_last_error(void);

/*
 * A1  Active-slot compaction.
 * Replaces the host-side filter of live requests and slot list assembly of
 * the reference engine (src/drama3/engine.py:637-647, engine.py:136-144).
 * occupancy[num_slots] (nonzero = live) -> active_slots[0..n) ascending,
 * active_slots[n..num_slots) = -1, *count = n.  One workgroup; no padding
 * rows (the reference pads to a graph bucket with reserved slots instead).
 */
int d3_compact_slots(const uint8_t *occupancy, int32_t num_slots, int32_t *active_slots,
                     int32_t *count, void *stream);

/*
 * A3  Top-k softmax routing.
 * Replaces route() / route_kernel (src/drama3/kernels.py:360-383).
 * logits[row_index ? row_index[r] : r] (bf16 or f32, row stride in elements,
 * unit column stride) -> ids (int32 and/or int64, [rows, top_k]) and weights
 * ([rows, top_k] bf16 or f32).  Ranking key: the bf16 value of the logit,
 * ties to the lower expert index; output in descending key order; weights are
 * the fp32 softmax probabilities of the selected experts renormalised to sum
 * to one.  num_experts <= 512, top_k <= 16.  ids32 / ids64 may be NULL.
 */
int d3_route(const void *logits, int32_t logits_dtype, int64_t logits_row_stride, int32_t rows,
             int32_t num_experts, int32_t top_k, const int32_t *row_index,
             const int32_t *row_count, int32_t *ids32, int64_t *ids64, void *weights,
             int32_t weights_dtype, void *stream);

/*
 * A4  Per-128 FP8 activation quantisation.
 * Replaces Fish Speech quantize_groups(quant_kernel, x, H) as called at
 * src/drama3/kernels.py:332,732 and model.py:554 (its rule restated by
 * prepare_kernel, src/drama3/moe_input.py:24-27).
 * x[row_index ? row_index[r] : r] bf16 [rows, width] -> q fp8 [rows, width]
 * and scales f32: [rows, width/128] (scales_transposed = 0) or
 * [width/128, rows] (scales_transposed = 1).  width % 128 == 0.
 */
int d3_quantize_rows(const uint16_t *x, int64_t x_row_stride, int32_t rows, int32_t width,
                     const int32_t *row_index, const int32_t *row_count, uint8_t *q,
                     float *scales, int32_t scales_transposed, void *stream);

/*
 * A4  Fused MoE input preparation.
 * Replaces prepare_moe_input / prepare_kernel (src/drama3/moe_input.py:8-79).
 * x bf16 [rows, hidden] -> q fp8 [rows, hidden], scales f32 [hidden/128, rows]
 * (transposed layout), logits f32 [rows, num_experts] converted from the
 * router (bf16 or f32).  When row_slots != NULL (int32 or int64, one per
 * row), rows whose slot >= padding_start read router row 0.
 */
int d3_prepare_moe_input(const uint16_t *x, int64_t x_row_stride, const void *router,
                         int32_t router_dtype, int64_t router_row_stride, int32_t rows,
                         int32_t hidden, int32_t num_experts, const void *row_slots,
                         int32_t row_slots_dtype, int64_t padding_start, uint8_t *q,
                         float *scales, float *logits, void *stream);

/*
 * A5-A7  Expert histogram, padded offsets and stable route sort.
 * Replaces expert_counts_kernel, expert_offsets_kernel and
 * expert_scatter_kernel (src/drama3/kernels.py:658-699) with the buffer
 * sizing of native_moe (kernels.py:710-731).
 * ids (int32 or int64) [rows, top_k]; pairs = live rows * top_k.
 *   counts[E], starts[E] (exclusive scan of counts padded to `tile`), *total;
 *   sorted_ids[max_rows]: pair ids grouped by expert in ascending pair order,
 *     padding and every slot from *total on hold the sentinel `pairs`;
 *   expert_ids[max_rows / tile]: expert of each tile, -1 from *total/tile on;
 *   inverse[pairs] (optional, NULL to skip): sorted position of each pair;
 *   items[max_items][4] (optional): work items {expert, sorted start, routes,
 *     0} covering each expert's routes in chunks of item_rows (a multiple of
 *     tile), with *num_items.  max_items must be >= d3_max_items(...).
 *   *pairs_out (optional): the live pair count, i.e. the sentinel value.
 * One workgroup; deterministic.
 */
int d3_sort_routes(const void *ids, int32_t ids_dtype, int32_t rows, const int32_t *row_count,
                   int32_t top_k, int32_t num_experts, int32_t tile, int32_t *counts,
                   int32_t *starts, int32_t *total, int32_t *sorted_ids, int32_t *expert_ids,
                   int32_t max_rows, int32_t *inverse, int32_t item_rows, int32_t *items,
                   int32_t max_items, int32_t *num_items, int32_t *pairs_out, void *stream);

/*
 * A1 + A3 + A4 + A5-A7  Fused front end of one MoE step (one launch).
 * Replaces the engine's host-side slot filtering (src/drama3/engine.py:
 * 637-647) followed by route / quantize_groups / expert_counts_kernel /
 * expert_offsets_kernel / expert_scatter_kernel (kernels.py:360-383,
 * 658-731; moe_input.py:24-27).  Results are those of d3_compact_slots,
 * d3_route (ids int32), d3_quantize_rows (native scale layout) and
 * d3_sort_routes, bit for bit.
 * Rows: with occupancy != NULL the live slots of occupancy[num_slots] in
 * ascending order (active_slots / *count written as d3_compact_slots; rows =
 * num_slots, row_index and row_count must be NULL); otherwise rows r <
 * (row_count ? *row_count : rows) reading source row row_index ? row_index[r]
 * : r of x and logits.  Row r of ids / weights / q / scales is output row r.
 * With sorted_ids != NULL the last workgroup to finish also sorts the routes
 * (rows * top_k <= 8192, num_experts <= 256; the same outputs as
 * d3_sort_routes, ranked through per-expert bit masks of rows since the
 * router's top_k experts of a row are distinct); `ticket` is a device int32
 * that must hold 0 before the first launch and is left at 0 by every launch.
 */
int d3_moe_front(const uint8_t *occupancy, int32_t num_slots, int32_t *active_slots,
                 int32_t *count, const uint16_t *x, int64_t x_row_stride, const void *logits,
                 int32_t logits_dtype, int64_t logits_row_stride, int32_t rows,
                 const int32_t *row_index, const int32_t *row_count, int32_t hidden,
                 int32_t num_experts, int32_t top_k, int32_t *ids, void *weights,
                 int32_t weights_dtype, uint8_t *q, float *scales, int32_t tile,
                 int32_t item_rows, int32_t *counts, int32_t *starts, int32_t *total,
                 int32_t *sorted_ids, int32_t *expert_ids, int32_t max_rows, int32_t *inverse,
                 int32_t *items, int32_t max_items, int32_t *num_items, int32_t *pairs_out,
                 int32_t *ticket, void *stream);

/*
 * A5-A7  The same histogram / offsets / stable sort as d3_sort_routes, for
 * prefill-sized batches: the ranking is spread over one workgroup per 512
 * pairs (two launches) instead of one workgroup walking every pair.
 * Same arguments and outputs as d3_sort_routes (starts is required), plus a
 * caller-owned int32 scratch of d3_sort_wide_scratch_ints(rows, top_k, E)
 * ints.  With max_items >= d3_max_items_aligned(pairs, E, item_rows), and
 * when the experts with routes average at least 1.5 items (decided on the
 * device from the live histogram), the items are aligned: every expert's
 * items start at an even item index, and an expert with an odd number of
 * items is followed by one empty item {expert, start, 0, 0} (counted in
 * *num_items), so two consecutive items never mix experts' weights; the
 * grouped GEMMs skip empty items (their XCD runs of two consecutive items
 * then share one expert's weights in L2).  Replaces expert_counts_kernel / expert_offsets_kernel /
 * expert_scatter_kernel (src/drama3/kernels.py:658-699) as native_moe runs
 * them for prefill (kernels.py:710-731).
 */
int d3_sort_routes_wide(const void *ids, int32_t ids_dtype, int32_t rows, const int32_t *row_count,
                        int32_t top_k, int32_t num_experts, int32_t tile, int32_t *counts,
                        int32_t *starts, int32_t *total, int32_t *sorted_ids, int32_t *expert_ids,
                        int32_t max_rows, int32_t *inverse, int32_t item_rows, int32_t *items,
                        int32_t max_items, int32_t *num_items, int32_t *pairs_out,
                        int32_t *scratch, int64_t scratch_ints, void *stream);

/* Scratch ints d3_sort_routes_wide needs (host-side arithmetic only). */
int64_t d3_sort_wide_scratch_ints(int32_t rows, int32_t top_k, int32_t num_experts);

/* Capacity helpers for d3_sort_routes (host-side arithmetic only). */
/*
 * A7  A caller's sorted-tile layout as work items.
 * For native_moe's layout (src/drama3/kernels.py:666-699, sized at 710-731)
 * as moe_atomic.atomic_down receives it (src/drama3/moe_atomic.py:60-78):
 * sorted_ids int32 [max_tiles * tile] (pair ids, sentinel `pairs` in the
 * padding), expert_ids int32 [max_tiles] (expert of each tile), *total (a
 * multiple of tile).  Writes items int32 [max_tiles][4] = {expert_ids[t],
 * t * tile, routes of tile t below the sentinel, 0} for t < *total / tile
 * (an expert id outside [0, num_experts) gives an item of 0 routes) and
 * *num_items = *total / tile (clamped to [0, max_tiles]).  items 16-byte
 * aligned.
 */
int d3_items_from_tiles(const int32_t *sorted_ids, const int32_t *expert_ids,
                        const int32_t *total, int32_t tile, int32_t pairs, int32_t max_tiles,
                        int32_t num_experts, int32_t *items, int32_t *num_items, void *stream);

/*
 * A8  Row gather (permute) by an index list.
 * The gather of activation rows stored by pair into sorted order that the
 * reference's atomic down projection does inside its GEMM
 * (src/drama3/moe_atomic.py:38-42: X + pairs * I).  dst row r (r < *row_count,
 * or all rows when row_count is NULL) = src row index[r] when 0 <= index[r]
 * < src_rows, else zeros; rows at or beyond the count are left untouched.
 * row_bytes a multiple of 4; src / dst 4-byte aligned.
 */
int d3_gather_rows(const void *src, int64_t row_bytes, int64_t src_rows, const int32_t *index,
                   const int32_t *row_count, int32_t rows, void *dst, void *stream);

int32_t d3_max_sorted_rows(int32_t pairs, int32_t num_experts, int32_t tile);
int32_t d3_max_items(int32_t pairs, int32_t num_experts, int32_t item_rows);
/* Items capacity for d3_sort_routes_wide's aligned items: d3_max_items plus
 * one empty item per used expert (no counterpart in the reference). */
int32_t d3_max_items_aligned(int32_t pairs, int32_t num_experts, int32_t item_rows);

/*
 * A8-A11  Grouped FP8 expert GEMM over sorted routes (FC1 or FC2).
 * Replaces expert_up_kernel / expert_down_kernel (src/drama3/kernels.py:290-322)
 * and Fish fused_moe_gemm as driven by native_moe (kernels.py:734-778).
 * For every work item {e, start, n}: rows p in [start, start+n) of the
 * sorted route list contract with expert e's weight w[e] (fp8 [N, K] in
 * weight_layout, block scales ws[e] [N/128, K/128]) on MFMA tiles:
 *   out[p, j] = sum_k (w[e,j,k] ws[e,j/128,k/128]) (a[r,k] as[r,k/128])
 * accumulated in fp32, where the activation row r is
 *   mode 0 (FC1): token sorted_ids[p] / top_k of a [*, K] (gather = permute),
 *                 output bf16 at sorted position p: out_bf16[p, N];
 *   mode 1 (FC2): sorted position p of a [max_rows, K],
 *                 output fp32 at pair sorted_ids[p]: out_f32[pair, N]
 *                 (scatter = unpermute).
 * Items with <= exact_routes routes contract on bf16 MFMAs after an exact
 * FP8 -> bf16 widening (fp32-accurate sums); larger items use FP8 MFMAs,
 * whose in-instruction product alignment rounds at ~1e-4 of sum|products|.
 * Work items cover live routes only, so padding slots are never read.
 * item_rows: upper bound on the routes of one item (the sort's item_rows).
 * With item_rows <= 16 (every item one 16-route MFMA tile) each FC2
 * workgroup takes two consecutive weight tiles of its item, the second
 * streaming in while the first one's outputs are stored; otherwise one.
 * The grid is max_items x (N / row tile) / tiles per workgroup; items at or
 * beyond *num_items exit.
 * Supported: K in {256, 512, 768, 1024, 1536, 2048}; N a multiple of the
 * workgroup row tile (64 for K >= 1024, 128 for K = 512/768, 256 for K = 256).
 */
int d3_expert_gemm(int32_t mode, const uint8_t *w, const float *ws, int32_t weight_layout,
                   int32_t num_experts, int32_t n, int32_t k, const uint8_t *a, const float *a_scales,
                   const int32_t *sorted_ids, int32_t top_k, const int32_t *items,
                   const int32_t *num_items, int32_t max_items, int32_t item_rows,
                   int32_t exact_routes, uint16_t *out_bf16, float *out_f32, void *stream);

/* Weight rows per workgroup tile of d3_expert_gemm for contraction length k. */
int32_t d3_expert_tile_rows(int32_t k);

/*
 * A8-A10  Tiled grouped FC1 + SwiGLU requant for real contractions (packed
 * prefill, mixed batches).  Replaces Fish fused_moe_gemm's FC1 as driven by
 * native_moe (src/drama3/kernels.py:734-747) and silu_mul_quant
 * (kernels.py:344,748).  For every work item {e, start, n} (n <= item_rows
 * <= 128: the sort's items) the routes p in [start, start+n)
 * gather token sorted_ids[p] / top_k of q fp8 [q_rows, hidden] (scales
 * x_scales [q_rows, hidden/128]) and contract with w13[e] ([gate; up],
 * fp8 [2I, hidden] in weight_layout, block scales s13[e]); FC1 is rounded
 * to bf16, a = silu(gate) * up is requantised per 128 columns and written
 * at sorted position p: act fp8 [rows, I], act_scales [rows, I/128].
 * items holds max_items entries ({e, start, n, -}, the sort's layout); every
 * one of them may be read, those at or beyond *num_items are ignored.
 * Contraction on FP8 MFMAs with the per-K128 rescale of d3_expert_gemm's
 * FP8 path; act / act_scales equal d3_expert_gemm (mode 0, exact_routes 0)
 * followed by d3_silu_mul_quant, byte for byte.  hidden in {256, 512, 768,
 * 1024, 1536, 2048}; intermediate a multiple of 128.
 * Optional dense shared expert in the same launch (the reference's moe_parts
 * shared expert, src/drama3/model.py:503-518; shared_w13 NULL for none):
 * fp8 [2I, hidden] in weight_layout with scales shared_s13, applied to q rows
 * [0, shared_rows), its act / act_scales written at rows shared_act_row + r
 * (act then needs max sorted rows + shared_rows rows).
 */
int d3_grouped_fc1_swiglu(const uint8_t *w13, const float *s13, int32_t weight_layout,
                          int32_t num_experts, int32_t intermediate, int32_t hidden,
                          const uint8_t *q, int64_t q_rows, const float *x_scales,
                          const int32_t *sorted_ids, int32_t top_k, const int32_t *items,
                          const int32_t *num_items, int32_t max_items, int32_t item_rows,
                          const uint8_t *shared_w13, const float *shared_s13,
                          int32_t shared_rows, int32_t shared_act_row, uint8_t *act,
                          float *act_scales, void *stream);

/*
 * A11  Tiled grouped FC2 for real contractions.  Replaces Fish
 * fused_moe_gemm's FC2 as driven by native_moe (src/drama3/kernels.py:
 * 764-778) before the combine: for every work item the sorted rows
 * [start, start+n) of act fp8 [act_rows, intermediate] (act_scales
 * [act_rows, intermediate/128]) contract with w2[e] (fp8 [hidden, I]) and
 * are stored fp32 by pair sorted_ids[p]: down [pairs, hidden] (unpermute).
 * items holds max_items entries, as for d3_grouped_fc1_swiglu.
 * Equal to d3_expert_gemm mode 1 with exact_routes 0, bit for bit.
 * item_rows: upper bound on the routes of one item, <= 128.
 * intermediate in {256, 512, 768, 1024, 1536, 2048}; hidden a multiple of 256.
 * Optional dense shared expert (shared_w2 NULL for none): act rows
 * shared_act_row + r, r < shared_rows, contract with shared_w2 (fp8 [hidden,
 * I] in weight_layout, scales shared_s2) into fp32 rows shared_out_row + r
 * of down.
 */
int d3_grouped_fc2(const uint8_t *w2, const float *s2, int32_t weight_layout,
                   int32_t num_experts, int32_t hidden, int32_t intermediate, const uint8_t *act,
                   int64_t act_rows, const float *act_scales, const int32_t *sorted_ids,
                   int32_t top_k, const int32_t *items, const int32_t *num_items,
                   int32_t max_items, int32_t item_rows, const uint8_t *shared_w2,
                   const float *shared_s2, int32_t shared_rows, int32_t shared_act_row,
                   int32_t shared_out_row, float *down, void *stream);

/*
 * A5-A8 + A9 + A10  The tiled grouped FP8 FC1 without a route sort, for
 * small batches (routes of up to 8192 (row, rank) pairs): replaces the sort
 * kernels.py:658-731 + the first fused_moe_gemm (kernels.py:734-779) for
 * batches where one sort launch is a large share of the step.  Work item
 * (expert e, part j), item index i = e * parts + j with parts =
 * ceil(capacity / 128), takes e's routes of ranks [128 j, 128 j + 128) in
 * pair order, found by the workgroup in `ids` ([capacity, top_k] int32
 * routed expert ids of the rows, *row_count live).  It writes what it found
 * as a sorted route list: list_items[i] = (e, 128 i, routes, 0) int32x4,
 * the item's pairs at list_ids[128 i ..] (ascending), *list_count =
 * E * parts; and act [E * parts * 128, I] / act_scales at those positions.
 * d3_grouped_fc2 with sorted_ids = list_ids, items = list_items, num_items
 * = list_count, max_items = E * parts, item_rows = 128 then writes down by
 * pair.  The values are those of d3_grouped_fc1_swiglu / d3_grouped_fc2
 * after d3_sort_routes.  Requires capacity * top_k <= 8192.
 */
int d3_grouped_fc1_swiglu_by_pair(const uint8_t *w13, const float *s13, int32_t weight_layout,
                                  int32_t num_experts, int32_t intermediate, int32_t hidden,
                                  const uint8_t *q, int64_t q_rows, const float *x_scales,
                                  const int32_t *ids, int32_t top_k, const int32_t *row_count,
                                  int32_t capacity, uint8_t *act, float *act_scales,
                                  int32_t *list_ids, int32_t *list_items, int32_t *list_count,
                                  void *stream);

/*
 * A9/A11 weight preparation (once, at load time).
 * Counterpart of the reference's load-time re-layout of the expert weights
 * for its FlashInfer path (src/drama3/model.py:195-205: [up | gate] copies
 * and blocked_moe_weight shuffling).  w fp8 [E, N, K] (reference layout) ->
 * packed fp8, same size, fragment-major: each 16-row tile of N is stored as
 * [K/128 blocks][2 halves][64 lanes][16 bytes], where lane l holds bytes
 * [64*half + 16*(l/16), +16) of K block kb of row 16*tile + l%16.  One
 * expert-GEMM wave then reads 1 KiB of contiguous memory per load
 * instruction.  N % 16 == 0, K % 128 == 0, w and packed must not overlap.
 * The block scales keep their layout.
 */
int d3_pack_expert_weights(const uint8_t *w, int32_t num_experts, int32_t n, int32_t k,
                           uint8_t *packed, void *stream);

/*
 * A10 + A11  FC2 with the SwiGLU requantisation done in its prologue.
 * Replaces Fish silu_mul_quant (src/drama3/kernels.py:344) followed by the
 * FC2 GEMM (kernels.py:304-318).  d3_expert_gemm mode 1 (down fp32 by pair,
 * n = hidden, k = intermediate), except that each workgroup computes the
 * activation tile itself from gate_up bf16 [sorted rows, 2I] ([gate | up])
 * exactly as d3_silu_mul_quant would (same fp8 codes and scales), while its
 * weight loads are in flight; no act / act_scales buffers are read or
 * written.  Every workgroup of an item recomputes the item's activations,
 * so this suits decode-sized items (a few route tiles).
 * Supported: intermediate in {256, 512, 768, 1024}.
 */
int d3_expert_fc2_swiglu(const uint8_t *w2, const float *s2, int32_t weight_layout,
                         int32_t num_experts, int32_t hidden, int32_t intermediate,
                         const uint16_t *gate_up, const int32_t *sorted_ids, int32_t top_k,
                         const int32_t *items, const int32_t *num_items, int32_t max_items,
                         int32_t item_rows, int32_t exact_routes, float *down, void *stream);

/*
 * A8-A11  Decode expert GEMMs without a route sort.
 * Replaces expert_up_kernel / expert_down_kernel (src/drama3/kernels.py:290-318)
 * with the Fish silu_mul_quant between them (kernels.py:344) for decode
 * batches, where the reference sorts routes first (kernels.py:658-731).
 * The grid is (expert, weight row tile); each workgroup finds its expert's
 * routes in ids int32 [capacity, top_k] (rows below *row_count, or all
 * capacity rows when row_count is NULL), in ascending pair order, while its
 * weight tile streams in.  Rows are indexed by pair = row * top_k + rank:
 *   mode 0 (FC1): a = q fp8 [capacity, k], a_scales [capacity, k/128]
 *                 -> out_bf16 gate_up [capacity * top_k, n], n = 2I, k = H;
 *   mode 2 (FC2): a = gate_up bf16 [capacity * top_k, 2k]; the SwiGLU
 *                 requant of each route is computed in the prologue exactly
 *                 as d3_silu_mul_quant -> out_f32 down [capacity * top_k, n],
 *                 n = H, k = I.  With row_slots int32 [capacity] (the slot
 *                 of each row: d3_decode_route_fc1's active) down rows are
 *                 indexed by slot pair, row_slots[row] * top_k + rank, the
 *                 layout d3_decode_route_combine reads; NULL: by pair.
 *                 Mode 0 takes row_slots = NULL.
 * Values equal d3_expert_gemm's for the same pair.  Weights must be
 * fragment-major (d3_pack_expert_weights).  A workgroup of an expert with no
 * route reads half a weight tile before it knows, so this suits batches
 * whose routes cover most experts.  capacity <= 256, top_k <= 8; k in
 * {1024, 2048} (mode 0) or {256, 512, 768, 1024} (mode 2).
 */
int d3_decode_expert_gemm(int32_t mode, const uint8_t *w, const float *ws, int32_t num_experts,
                          int32_t n, int32_t k, const int32_t *ids, const int32_t *row_count,
                          const int32_t *row_slots, int32_t capacity, int32_t top_k,
                          const void *a, const float *a_scales, int32_t exact_routes,
                          uint16_t *out_bf16, float *out_f32, void *stream);

/*
 * A1-A3, A5, A8  Decode FC1 straight from the slots (no front launch).
 * Replaces, for the decode step, the slot filter (src/drama3/engine.py:637-647),
 * route_kernel's top-k (src/drama3/kernels.py:360-383), the per-128
 * quantisation (src/drama3/moe_input.py:24-27) and expert_up_kernel
 * (kernels.py:290-301) of DramaModel.routed_moe (src/drama3/model.py:520-583).
 * Each (expert, weight tile) workgroup ranks its expert in every occupied
 * slot from the logits (rank = experts with a larger routing key; a route
 * when rank < top_k), quantises the x rows of its routes while staging them,
 * and writes gate_up by pair exactly as d3_moe_front + d3_decode_expert_gemm
 * mode 0 do.  It also writes that front's ids int32 [capacity, top_k] (by
 * row), *count and active int32 [capacity] (ascending slots, -1 padded);
 * the routing weights are left to d3_decode_route_combine, and no q /
 * x_scales are stored.
 *   occupancy u8 [capacity]; x bf16 [capacity rows, x_stride];
 *   logits bf16 or f32 [capacity rows, logits_stride] (16-byte aligned rows);
 *   w / ws fragment-major W13 and its block scales; n = 2I, k = H in
 *   {1024, 2048}; capacity <= 256, top_k <= 8, E <= 256 (bf16 logits) or
 *   128 (f32).
 */
int d3_decode_route_fc1(const uint8_t *w, const float *ws, int32_t num_experts, int32_t n,
                        int32_t k, const uint8_t *occupancy, int32_t capacity, const uint16_t *x,
                        int64_t x_stride, const void *logits, int32_t logits_dtype,
                        int64_t logits_stride, int32_t top_k, int32_t exact_routes, int32_t *ids,
                        int32_t *count, int32_t *active, uint16_t *gate_up, void *stream);

/*
 * A4, A12  Weighted combine of the step started by d3_decode_route_fc1.
 * Replaces route_kernel's weights (src/drama3/kernels.py:360-383) and the
 * combine (kernels.py:319-322) for the decode step.  One workgroup per
 * (slot, 512 columns): occupied slot s, row r, gets
 * out[r] = bf16(sum_rank w[rank] * down[s * top_k + rank]) in rank order
 * (down f32 [capacity * top_k, hidden] by slot pair, as d3_decode_expert_gemm
 * mode 2 writes it with row_slots; the slot indexing lets the down rows load
 * with the logits, before the row is known), w being the front's routing
 * weights of the slot's logits rounded to weights_dtype (bf16 or f32),
 * which are also stored in weights [capacity, top_k] by row.  Same bytes
 * as d3_moe_front's weights + d3_weighted_combine.  capacity <= 256,
 * top_k <= 8, E <= 256.
 */
int d3_decode_route_combine(const uint8_t *occupancy, int32_t capacity, const void *logits,
                            int32_t logits_dtype, int64_t logits_stride, int32_t num_experts,
                            int32_t top_k, int32_t hidden, const float *down, void *weights,
                            int32_t weights_dtype, uint16_t *out, void *stream);

/*
 * A1-A12  The decode MoE step over persistent slots (three launches).
 * Replaces DramaModel.routed_moe's decode path (src/drama3/model.py:520-583:
 * the slot filter engine.py:637-647, route kernels.py:360-383, the per-128
 * quantisation moe_input.py:24-27, expert_up_kernel / silu_mul_quant /
 * expert_down_kernel and the combine kernels.py:290-322, 344) for one
 * step: d3_decode_route_fc1 (ids int32 [capacity, top_k], *count, active
 * int32 [capacity], gate_up bf16 [capacity * top_k, 2I] by pair), then
 * d3_decode_expert_gemm mode 2 with row_count = count and row_slots = active
 * (down f32 [capacity * top_k, hidden] by slot pair), then
 * d3_decode_route_combine (weights [capacity,
 * top_k] in weights_dtype, out bf16 [capacity, hidden]: row r < *count
 * belongs to slot active[r]).  Every stage's arguments are checked before
 * the first launch; the limits are those of the three entry points
 * (fragment-major weights, hidden in {1024, 2048}, intermediate in {256,
 * 512, 768, 1024}, capacity <= 256, top_k <= 8).
 */
int d3_decode_step(const uint8_t *w13, const float *s13, const uint8_t *w2, const float *s2,
                   int32_t num_experts, int32_t hidden, int32_t intermediate,
                   const uint8_t *occupancy, int32_t capacity, const uint16_t *x,
                   int64_t x_stride, const void *logits, int32_t logits_dtype,
                   int64_t logits_stride, int32_t top_k, int32_t exact_routes, int32_t *ids,
                   void *weights, int32_t weights_dtype, uint16_t *gate_up, float *down,
                   int32_t *active, int32_t *count, uint16_t *out, void *stream);

/*
 * d3_decode_step on the library's static device scratch, for callers that
 * cannot allocate device memory (code under graph capture, serving loops
 * that forbid allocation); it has no counterpart in the reference.  The
 * intermediate buffers (ids, route weights in the logits' dtype, gate_up,
 * down) live in a static device array of the library, 6 MiB + 4 KiB per
 * GPU, held by each GPU it runs on until the process ends; the caller
 * passes only inputs and outputs (active, count, out: as d3_decode_step).
 * Limits of that array: capacity * top_k <= 512 routes, 2I <= 2048,
 * hidden <= 2048; larger calls return D3_ERR_UNSUPPORTED and launch
 * nothing.  Allocates nothing (no hipMalloc / hipFree).  Every call on one
 * GPU shares the array: calls that overlap on one GPU (other streams, other
 * threads) race and must be serialised by the caller.  Results equal
 * d3_decode_step's byte for byte.
 */
int d3_decode_step_static(const uint8_t *w13, const float *s13, const uint8_t *w2,
                          const float *s2, int32_t num_experts, int32_t hidden,
                          int32_t intermediate, const uint8_t *occupancy, int32_t capacity,
                          const uint16_t *x, int64_t x_stride, const void *logits,
                          int32_t logits_dtype, int64_t logits_stride, int32_t top_k,
                          int32_t exact_routes, int32_t *active, int32_t *count, uint16_t *out,
                          void *stream);

/*
 * A10  SwiGLU + per-128 FP8 requantisation of FC1 rows.
 * Replaces Fish quantize_groups(silu_mul_quant_kernel, gate_up, I)
 * (src/drama3/kernels.py:344,748).  gate_up bf16 [rows, 2I] ([gate | up]) ->
 * a = silu(gate) * up in fp32 -> act fp8 [rows, I] + act_scales f32
 * [rows, I/128].  When sorted_ids != NULL, row p is processed only if
 * sorted_ids[p] < pairs (live routes); rows = capacity, row_count optional.
 */
int d3_silu_mul_quant(const uint16_t *gate_up, int32_t rows, int32_t intermediate,
                      const int32_t *row_count, const int32_t *sorted_ids,
                      const int32_t *pairs_dev, int32_t pairs, uint8_t *act, float *act_scales,
                      void *stream);

/*
 * A11  Weighted combine (unpermute + top-k reduction).
 * Replaces the fused combine of expert_down_kernel (src/drama3/kernels.py:319-322)
 * and native_moe's down.view(T, 8, H).sum(1) (kernels.py:779).
 * out[t, :] = bf16( sum_{r=0..top_k-1} w[t,r] * down[t*top_k + r, :] ) in
 * rank order, fp32 accumulation; w bf16 or f32 [rows, top_k].  When
 * shared != NULL (fp32 [rows, hidden]), out = bf16(out + bf16(shared)): a
 * dense shared expert added to the routed output.
 */
int d3_weighted_combine(const float *down, const void *weights, int32_t weights_dtype,
                        int32_t rows, int32_t top_k, int32_t hidden, const int32_t *row_count,
                        const float *shared, uint16_t *out, void *stream);

/*
 * A12  Routed + gated shared expert combine.
 * Replaces combine_experts (src/drama3/kernels.py:427-445) as compiled: one
 * single-rounding bf16 FMA (kernels.py:465-474),
 * out = bf16(shared * bf16(sigmoid(gate[r * gate_stride])) + routed), so this
 * followed by d3_add_norm equals d3_combine_experts_add_norm byte for byte.
 */
int d3_combine_experts(const uint16_t *routed, const uint16_t *shared, const uint16_t *gate,
                       int64_t gate_stride, int32_t rows, int32_t width, uint16_t *out,
                       void *stream);

/*
 * A12  Combine + residual update + (1 + w) RMSNorm.
 * Replaces combine_experts_add_norm and combine_experts_add_norm_inverse
 * (src/drama3/kernels.py:448-556).  Row r reads MoE row inverse[r] when
 * inverse != NULL (int64), else r.  combined is the single-rounding bf16
 * FMA shared * bf16(sigmoid(gate)) + routed; residual[r] is updated in place
 * to bf16(combined + residual[r]); out[r] = bf16(residual * rsqrt(mean(
 * residual^2) + eps) * (1 + weight)).  width <= 8192.
 */
int d3_combine_experts_add_norm(const uint16_t *routed, const uint16_t *shared,
                                const uint16_t *gate, int64_t gate_stride,
                                const int64_t *inverse, uint16_t *residual,
                                const uint16_t *weight, float eps, int32_t rows, int32_t width,
                                uint16_t *out, void *stream);

/*
 * A11 + A12  Weighted combine of the per-route rows, then combine + residual
 * + RMSNorm, in one launch.
 * Replaces native_moe's down.view(T, 8, H).sum(1) (src/drama3/kernels.py:779)
 * followed by combine_experts_add_norm(_inverse) (kernels.py:448-556).
 * Row r reads MoE row m = inverse[r] (int64) when inverse != NULL, else r;
 * routed = bf16(sum_k w[m, k] * down[m * top_k + k, :]) in rank order with
 * fp32 accumulation (exactly d3_weighted_combine's bytes), then the
 * d3_combine_experts_add_norm rule.  down f32 [MoE rows * top_k, width]
 * (16-byte aligned); w bf16 or f32 [MoE rows, top_k]; shared bf16
 * [MoE rows, width]; gate bf16 (row stride gate_stride); residual bf16
 * [rows, width] updated in place; out bf16 [rows, width].  With residual ==
 * NULL (weight and eps unused) out[r] = the combined row: the bytes of
 * d3_weighted_combine followed by d3_combine_experts.  width <= 8192.
 */
int d3_combine_routes_add_norm(const float *down, const void *route_weights,
                               int32_t weights_dtype, int32_t top_k, const uint16_t *shared,
                               const uint16_t *gate, int64_t gate_stride, const int64_t *inverse,
                               uint16_t *residual, const uint16_t *weight, float eps,
                               int32_t rows, int32_t width, uint16_t *out, void *stream);

/*
 * Residual add + RMSNorm without the MoE combine.
 * Replaces add_norm (src/drama3/kernels.py:405-424).
 */
int d3_add_norm(const uint16_t *x, uint16_t *residual, const uint16_t *weight, float eps,
                int32_t rows, int32_t width, uint16_t *out, void *stream);

/*
 * BF16 SwiGLU of a [gate | up] projection (shared expert input).
 * Replaces silu_mul (src/drama3/kernels.py:386-402).
 */
int d3_silu_mul(const uint16_t *projected, int64_t row_stride, int32_t rows, int32_t width,
                uint16_t *out, void *stream);

/*
 * A11, A12  The decode layer's epilogue in one launch.
 * Replaces route_kernel's weights (src/drama3/kernels.py:360-383), the
 * routed combine (kernels.py:319-322) and combine_experts /
 * combine_experts_add_norm (kernels.py:427-499) after a decode step whose
 * FC1 ranked the experts itself (d3_decode_route_fc1: rows = live slots,
 * down f32 [rows * top_k, width] by pair, no weights stored).  Row r: the
 * routing weights of logits row r (bf16 or f32, logits_stride) rounded to
 * weights_dtype (also stored in route_weights [rows, top_k] when non-NULL),
 * routed = bf16(sum_rank w * down[r * top_k + rank]) in rank order,
 * combined = single-rounding bf16 FMA shared * bf16(sigmoid(gate)) +
 * routed; with residual == NULL out[r] = combined, otherwise residual[r] <-
 * bf16(combined + residual[r]) and out[r] = bf16(residual * rsqrt(mean(
 * residual^2) + eps) * (1 + weight)).  Bytes equal d3_decode_route_combine
 * then d3_combine_experts (then d3_add_norm).  top_k <= 8, E <= 256,
 * width <= 2048.
 */
int d3_combine_route_logits(const float *down, const void *logits, int32_t logits_dtype,
                            int64_t logits_stride, int32_t num_experts, int32_t top_k,
                            void *route_weights, int32_t weights_dtype, const uint16_t *shared,
                            const uint16_t *gate, int64_t gate_stride, uint16_t *residual,
                            const uint16_t *weight, float eps, int32_t rows, int32_t width,
                            uint16_t *out, void *stream);

/*
 * f4  Dense bf16 GEMM of the MoE layer's projections.
 * Replaces the two bf16 linear layers around the routed experts in
 * DramaModel.moe_parts (src/drama3/model.py:495-518): the packed input
 * projection (shared gate / up rows, router, shared-expert gate;
 * model.py:230-245) with the shared expert's silu_mul (kernels.py:386-402)
 * in its epilogue, and the shared expert's down projection.
 * out[r, j] = bf16(sum_c x[r, c] w[j, c]) for r < rows, j < n, c < k, fp32
 * accumulation.  With pair_rows = P > 0, rows [0, P) of w are gate rows and
 * rows [P, 2P) the matching up rows; when act != NULL it also receives
 * act[r, c] = bf16(bf16(silu(out[r, c])) * out[r, P + c]) for c < P (the
 * bytes of d3_silu_mul on out).  x bf16 [rows, x_stride], w bf16 [n, k]
 * row-major (a torch Linear weight), out bf16 [rows, out_stride], act bf16
 * [rows, act_stride].  Up to 768 rows with k in {256, 512, 768, 1024, 1536,
 * 2048} a streaming kernel runs (n and P multiples of 16); otherwise a
 * tiled kernel (k a multiple of 64, n a multiple of 16, P a multiple of
 * 64).  x / w rows 16-byte aligned, out / act rows 8-byte; operands below
 * 2 GiB.
 */
int d3_dense_bf16(const uint16_t *x, int64_t x_stride, int32_t rows, const uint16_t *w, int32_t n,
                  int32_t k, int32_t pair_rows, uint16_t *out, int64_t out_stride, uint16_t *act,
                  int64_t act_stride, void *stream);

/*
 * A13  Ragged packed-row metadata.
 * Replaces row_metadata (src/drama3/packed_prefill.py:51-78).
 * cu_seqlens int32 [sequences + 1], sequence_slots int64 [sequences] ->
 * positions int64 [capacity], row_slots int64 [capacity] and, when frames !=
 * NULL, labels int64 [capacity, codes] (next row's frame inside the sequence,
 * else eos / 0).  frames int64 [capacity, codes].
 */
int d3_row_metadata(const int32_t *cu_seqlens, const int64_t *sequence_slots,
                    int32_t sequences, int32_t capacity, const int64_t *frames, int32_t codes,
                    int64_t eos, int64_t *positions, int64_t *row_slots, int64_t *labels,
                    void *stream);

/*
 * A13  Rows of one mixed decode + prefill step, from device data (one launch,
 * graph-capturable, no host sync).
 * Replaces the host-side row preparation of MixedGraph.prepare
 * (src/drama3/mixed_graph.py:139-179: decode slots padded with reserved
 * slots, packed prompt suffix) and the row ownership of plan_row_reuse
 * (src/drama3/row_reuse.py:46-109) whose keep / inverse lists
 * mixed_backbone feeds to the MoE and to combine_experts_add_norm_inverse
 * (src/drama3/mixed_model.py:193-198,239-242).
 * Row space: decode rows [0, decode_rows), then the prefill suffix's
 * capacity rows.
 *   occupancy u8 [num_slots] -> active_slots int32 [num_slots] (ascending,
 *     -1 padded), *count; decode_slots int64 [decode_rows]: the first
 *     min(count, decode_rows) occupied slots, then padding_start + j;
 *   boundaries int32 [prompts + 1]: prompt i is suffix rows [b[i], b[i+1])
 *     (the reference layout's boundaries, prompts = its sequences before
 *     the padding sequence); suffix rows from b[prompts] on are padding;
 *   frames int64 [capacity, codes] (the suffix's frames) or NULL: with
 *     frames and prompts >= 2, each prompt's leading rows alias the rows of
 *     the earlier prompt with the longest agreeing leading run (the
 *     reference's prefix reuse; <= 16 prompts, <= 8192 rows);
 *   keep int32 [full]: the live rows (occupied decode rows, prompt rows)
 *     that own themselves, ascending, then 0; *keep_count of them;
 *   inverse int64 [full]: the keep index of each live row's owner, 0 for
 *     padding rows.
 * The MoE runs on rows keep[0 .. keep_count) (a front row_index / device
 * row_count); combine_experts_add_norm with inverse maps its rows back.
 * Padding rows never reach the MoE (the reference computes and discards
 * them).  More occupied slots than decode_rows: *count reports them all and
 * the first decode_rows become rows.
 * With positions != NULL the same launch also writes d3_row_metadata's
 * positions / row_slots int64 [capacity] of the suffix (boundaries then hold
 * sequences + 1 entries, sequence_slots int64 [sequences], sequences >=
 * prompts; NULL skips them).
 */
int d3_mixed_rows(const uint8_t *occupancy, int32_t num_slots, int32_t decode_rows,
                  int64_t padding_start, const int32_t *boundaries, int32_t prompts,
                  int32_t capacity, const int64_t *frames, int32_t codes,
                  const int64_t *sequence_slots, int32_t sequences, int32_t *active_slots,
                  int32_t *count, int64_t *decode_slots, int32_t *keep, int32_t *keep_count,
                  int64_t *inverse, int64_t *positions, int64_t *row_slots, void *stream);

/*
 * A1  Per-slot request state gather / update.
 * Replace DeviceRequests.load / .save and their _load / _save kernels
 * (src/drama3/runtime_state.py:10-56,94-124).  State layout: last [S, 11],
 * history [S, 16], metadata [S, 4] = {position, count, limit, done}, codes
 * [S, max_frames, 10]; all int64.  slots int64 [rows].
 */
int d3_requests_load(const int64_t *last, const int64_t *history, const int64_t *metadata,
                     const int64_t *slots, int32_t rows, int64_t max_length,
                     int64_t padding_start, int64_t *frames_out, int64_t *history_out,
                     int64_t *positions_out, void *stream);
int d3_requests_save(int64_t *last, int64_t *history, int64_t *metadata, int64_t *codes,
                     const int64_t *slots, int32_t rows, const int64_t *output, int64_t eos,
                     int64_t limit, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* DRAMA3_MOE_H */
