// Standalone route sort: the block sort of route_sort.h in one 1024-thread
// workgroup, for batches whose pair count is too large for the fused front
// end and for the reference-named sort operator; and the wide sort for
// prefill-sized batches, which spreads the stable ranking over many
// workgroups (one 1024-thread workgroup walks a 29k-pair batch in 29
// dependent chunks: 56 us on MI355X).
#include "expert_tile.h"
#include "route_sort.h"
#include "status.h"

namespace d3 {
namespace {

constexpr int kSortThreads = 1024;
constexpr int kMaxSortExperts = 512;  // LDS: (4 + 16 waves) * E ints <= 40 KiB

constexpr int kSortPerThread = 8;        // row-mask sort: up to 8192 pairs
constexpr int kSortMaskCells = 4096;     // row-mask sort: E * ceil(rows / 64) <= 4096 (48 KiB)

// mask_cells > 0: try the row-mask sort first (it gives up, writing
// nothing, when a row repeats an expert; the chunked ballot sort then runs).
template <bool kI64>
__global__ __launch_bounds__(kSortThreads) void sort_routes_kernel(
    const void* __restrict__ ids, int rows, const int32_t* __restrict__ row_count, int top_k,
    int num_experts, int tile, int item_rows, int mask_cells, SortOutputs out) {
  extern __shared__ int smem[];
  const int live = live_rows(row_count, rows);
  if (mask_cells > 0 &&
      sort_rows_block<kSortThreads, kSortPerThread, kI64, false>(
          ids, live, top_k, num_experts, tile, item_rows, smem, mask_cells, out))
    return;
  __syncthreads();  // the row-mask attempt's LDS is reused
  sort_routes_block<kSortThreads, kI64>(ids, live * top_k, num_experts, tile, item_rows, smem, out);
}

// ---------------------------------------------------------------------------
// Wide sort (two launches), the same results as sort_routes_block:
//   1. wide_rank_kernel: one workgroup per chunk of kWideChunk pairs ranks
//      every pair among the chunk's pairs of its expert, in pair order
//      (per-wave ballot matching on the expert-id bits, per-wave counts in
//      LDS, a running per-expert base across sub-chunks), and writes the
//      chunk's expert histogram;
//   2. wide_place_kernel: one workgroup per chunk again, a thread per pair
//      and per expert.  Every workgroup reads all chunk histograms (thread e
//      sums its expert's column, and the part of it above its own chunk), so
//      each holds the padded expert scan and its chunk's offsets itself:
//      sorted_ids[start[e] + chunk offset + rank] = p.  The last workgroup
//      also writes the sentinel padding, expert ids, work items and totals.
//      (A single workgroup scanning the histograms between two launches, as
//      before, took 8 us of a 13 us pair at config 4.)
// Scratch: chunk histograms [chunks][E] and ranks [pairs] (int32).
// ---------------------------------------------------------------------------
constexpr int kWideThreads = 256;
constexpr int kWideChunk = 512;
constexpr int kPlaceThreads = kWideChunk;  // one pair and at most one expert per thread
static_assert(kPlaceThreads >= kMaxSortExperts, "a placement thread per expert");
constexpr int kPlaceBatch = 64;  // chunk counts a placement thread holds in registers

template <bool kI64>
__global__ __launch_bounds__(kWideThreads) void wide_rank_kernel(
    const void* __restrict__ ids, int rows, const int32_t* __restrict__ row_count, int top_k,
    int num_experts, int32_t* __restrict__ chunk_counts, int32_t* __restrict__ ranks) {
  constexpr int kWaves = kWideThreads / kWave;
  extern __shared__ int smem[];
  int* running = smem;                  // [E]
  int* wave_counts = smem + num_experts;  // [kWaves][E]
  const int pairs = live_rows(row_count, rows) * top_k;
  const int tid = threadIdx.x;
  const int wave = tid / kWave;
  const int base = blockIdx.x * kWideChunk;
  for (int e = tid; e < num_experts; e += kWideThreads) running[e] = 0;
  for (int i = tid; i < kWaves * num_experts; i += kWideThreads) wave_counts[i] = 0;
  __syncthreads();
  int bits = 0;
  while ((1 << bits) < num_experts) ++bits;
  const uint64_t below = lanemask_lt();
  // All of a chunk's ids in registers first (one memory round trip).
  constexpr int kSub = kWideChunk / kWideThreads;
  int e_of[kSub];
#pragma unroll
  for (int s = 0; s < kSub; ++s) {
    const int p = base + s * kWideThreads + tid;
    e_of[s] = p < pairs ? load_route_id<kI64>(ids, p) : -1;
  }
#pragma unroll
  for (int s = 0; s < kSub; ++s) {
    if (base + s * kWideThreads >= pairs) break;  // uniform
    const int p = base + s * kWideThreads + tid;
    const int e = e_of[s];
    const bool valid = p < pairs && e >= 0 && e < num_experts;
    uint64_t peers = __ballot(valid);
    for (int b = 0; b < bits; ++b) {
      const bool bit = valid && ((e >> b) & 1);
      const uint64_t set = __ballot(bit);
      peers &= bit ? set : ~set;
    }
    const int rank = __popcll(peers & below);
    const bool leader = valid && rank == 0;
    if (leader) wave_counts[wave * num_experts + e] = __popcll(peers);
    __syncthreads();
    if (valid) {
      int r = running[e] + rank;
      for (int w = 0; w < wave; ++w) r += wave_counts[w * num_experts + e];
      ranks[p] = r;
    } else if (p < pairs) {
      ranks[p] = -1;
    }
    __syncthreads();
    if (leader) {
      atomicAdd(&running[e], __popcll(peers));
      wave_counts[wave * num_experts + e] = 0;
    }
    __syncthreads();
  }
  for (int e = tid; e < num_experts; e += kWideThreads)
    chunk_counts[static_cast<size_t>(blockIdx.x) * num_experts + e] = running[e];
}

template <bool kI64>
__global__ __launch_bounds__(kPlaceThreads) void wide_place_kernel(
    const void* __restrict__ ids, int rows, const int32_t* __restrict__ row_count, int top_k,
    int num_experts, int tile, int item_rows, int align_items, int chunks,
    const int32_t* __restrict__ chunk_counts, const int32_t* __restrict__ ranks, SortOutputs out) {
  __shared__ int wave_totals[kPlaceThreads / kWave];
  __shared__ int counts[kMaxSortExperts];
  __shared__ int starts[kMaxSortExperts];
  __shared__ int first_item[kMaxSortExperts];
  __shared__ int base[kMaxSortExperts];  // start + this chunk's offset, per expert
  const int pairs = live_rows(row_count, rows) * top_k;
  const int tid = threadIdx.x;
  const int mine = blockIdx.x;
  // This thread's pair: its expert and rank, issued first (they do not
  // depend on the histograms).
  const int p = mine * kWideChunk + tid;
  const int e_p = p < pairs ? load_route_id<kI64>(ids, p) : -1;
  const int rank = p < pairs ? ranks[p] : -1;
  // Expert e = tid: its column of the chunk histograms, in batches read
  // branch-free (cells past the last chunk or expert read zero).
  const uint32_t cells = static_cast<uint32_t>(chunks) * num_experts;
  const BufferView count_view(chunk_counts, cells * 4);
  int total_e = 0, below = 0;
  for (int b = 0; b < chunks; b += kPlaceBatch) {
    int v[kPlaceBatch];
#pragma unroll
    for (int q = 0; q < kPlaceBatch; ++q) {
      const int c = b + q;
      v[q] = static_cast<int>(count_view.load4(
          c < chunks && tid < num_experts ? static_cast<uint32_t>(c * num_experts + tid) * 4 : kNoRow));
    }
#pragma unroll
    for (int q = 0; q < kPlaceBatch; ++q) {
      total_e += v[q];
      below += b + q < mine ? v[q] : 0;
    }
  }
  if (tid < num_experts) counts[tid] = total_e;
  __syncthreads();
  int total = 0, total_items = 0;
  expert_offsets<kPlaceThreads>(counts, num_experts, tile, item_rows, starts, first_item, wave_totals,
                                &total, &total_items);
  const int count_e = tid < num_experts ? counts[tid] : 0;
  const int items_e = (count_e + item_rows - 1) / item_rows;
  // Padding pays while the experts with routes average at least 1.5 items;
  // at about one item each, most of them would take an empty item.
  const int used = __syncthreads_count(count_e > 0);
  if (align_items && 2 * total_items >= 3 * used) {  // uniform
    // Every expert's items start on an even item (an odd count is followed
    // by one empty item), so the grouped GEMMs' XCD runs of two consecutive
    // items hold one expert's items and share its weights in that L2.
    const int padded_items = (items_e + 1) & ~1;
    const int first_aligned =
        block_inclusive_scan<kPlaceThreads>(padded_items, wave_totals, &total_items) - padded_items;
    if (tid < num_experts) first_item[tid] = first_aligned;
    if (mine == static_cast<int>(gridDim.x) - 1 && tid < num_experts && padded_items > items_e)
      out.items[first_aligned + items_e] = make_int4(tid, starts[tid], 0, 0);
  }
  if (tid < num_experts) base[tid] = starts[tid] + below;
  __syncthreads();
  if (p < pairs) {
    if (e_p < 0 || e_p >= num_experts || rank < 0) {
      if (out.inverse != nullptr) out.inverse[p] = -1;
    } else {
      const int position = base[e_p] + rank;
      out.sorted_ids[position] = p;
      if (out.inverse != nullptr) out.inverse[p] = position;
    }
  }
  if (mine == static_cast<int>(gridDim.x) - 1)
    write_sort_tail<kPlaceThreads, false>(counts, starts, first_item, num_experts, tile, item_rows, total,
                                          total_items, pairs, out);
}

}  // namespace
}  // namespace d3

using namespace d3;

extern "C" int32_t d3_max_sorted_rows(int32_t pairs, int32_t num_experts, int32_t tile) {
  if (pairs < 0 || num_experts <= 0 || tile <= 0) return -1;
  const int64_t used = pairs < num_experts ? pairs : num_experts;
  const int64_t raw = static_cast<int64_t>(pairs) + used * (tile - 1);
  return static_cast<int32_t>((raw + tile - 1) / tile * tile);
}

extern "C" int32_t d3_max_items(int32_t pairs, int32_t num_experts, int32_t item_rows) {
  if (pairs < 0 || num_experts <= 0 || item_rows <= 0) return -1;
  const int64_t used = pairs < num_experts ? pairs : num_experts;
  return static_cast<int32_t>((static_cast<int64_t>(pairs) + used * (item_rows - 1)) / item_rows);
}

extern "C" int32_t d3_max_items_aligned(int32_t pairs, int32_t num_experts, int32_t item_rows) {
  const int32_t plain = d3_max_items(pairs, num_experts, item_rows);
  if (plain < 0) return -1;
  return plain + (pairs < num_experts ? pairs : num_experts);  // one empty item per used expert at most
}

extern "C" int d3_sort_routes(const void* ids, int32_t ids_dtype, int32_t rows,
                              const int32_t* row_count, int32_t top_k, int32_t num_experts,
                              int32_t tile, int32_t* counts, int32_t* starts, int32_t* total,
                              int32_t* sorted_ids, int32_t* expert_ids, int32_t max_rows,
                              int32_t* inverse, int32_t item_rows, int32_t* items,
                              int32_t max_items, int32_t* num_items, int32_t* pairs_out,
                              void* stream) {
  D3_REQUIRE(ids && counts && starts && total && sorted_ids && expert_ids,
             "sort_routes: null pointer");
  D3_REQUIRE(ids_dtype == D3_DTYPE_I32 || ids_dtype == D3_DTYPE_I64,
             "sort_routes: ids must be int32 or int64");
  D3_REQUIRE(rows >= 0 && top_k >= 1 && top_k <= 64, "sort_routes: bad rows/top_k");
  D3_SUPPORTED(num_experts >= 1 && num_experts <= kMaxSortExperts,
               "sort_routes: num_experts %d not in [1, %d]", num_experts, kMaxSortExperts);
  D3_REQUIRE(tile >= 1 && tile <= 1024, "sort_routes: tile %d not in [1, 1024]", tile);
  const int64_t pairs = static_cast<int64_t>(rows) * top_k;
  D3_REQUIRE(pairs < (1 << 30), "sort_routes: too many pairs");
  const int32_t need = d3_max_sorted_rows(static_cast<int32_t>(pairs), num_experts, tile);
  D3_REQUIRE(max_rows >= need && max_rows % tile == 0,
             "sort_routes: max_rows %d < required %d or not a multiple of tile", max_rows, need);
  if (items != nullptr) {
    D3_REQUIRE(num_items != nullptr, "sort_routes: items need num_items");
    D3_REQUIRE(item_rows >= tile && item_rows % tile == 0,
               "sort_routes: item_rows must be a positive multiple of tile");
    const int32_t need_items = d3_max_items(static_cast<int32_t>(pairs), num_experts, item_rows);
    D3_REQUIRE(max_items >= need_items, "sort_routes: max_items %d < required %d", max_items,
               need_items);
  } else {
    item_rows = tile;
  }
  // The row-mask sort covers batches whose masks (sized for the capacity
  // rows) and pairs fit; the ballot sort everything else.
  const int64_t cells = static_cast<int64_t>(num_experts) * mask_words(rows);
  const int mask_cells =
      pairs <= kSortThreads * kSortPerThread && cells <= kSortMaskCells ? static_cast<int>(cells) : 0;
  int shared_ints = sort_shared_ints(kSortThreads, num_experts);
  if (mask_cells > 0) {
    const int mask_ints = mask_sort_shared_ints(kSortThreads, num_experts, mask_cells);
    shared_ints = mask_ints > shared_ints ? mask_ints : shared_ints;
  }
  const size_t shared = sizeof(int) * static_cast<size_t>(shared_ints);
  const SortOutputs out{counts, starts, total, sorted_ids, expert_ids, max_rows, inverse,
                        reinterpret_cast<int4*>(items), max_items, num_items, pairs_out};
  hipStream_t s = as_stream(stream);
  if (ids_dtype == D3_DTYPE_I64)
    hipLaunchKernelGGL(sort_routes_kernel<true>, dim3(1), dim3(kSortThreads), shared, s, ids,
                       rows, row_count, top_k, num_experts, tile, item_rows, mask_cells, out);
  else
    hipLaunchKernelGGL(sort_routes_kernel<false>, dim3(1), dim3(kSortThreads), shared, s, ids,
                       rows, row_count, top_k, num_experts, tile, item_rows, mask_cells, out);
  D3_LAUNCHED("sort_routes");
}

extern "C" int64_t d3_sort_wide_scratch_ints(int32_t rows, int32_t top_k, int32_t num_experts) {
  if (rows < 0 || top_k < 1 || num_experts < 1) return -1;
  const int64_t pairs = static_cast<int64_t>(rows) * top_k;
  const int64_t chunks = (pairs + kWideChunk - 1) / kWideChunk;
  return chunks * num_experts + pairs;
}

extern "C" int d3_sort_routes_wide(const void* ids, int32_t ids_dtype, int32_t rows,
                                   const int32_t* row_count, int32_t top_k, int32_t num_experts,
                                   int32_t tile, int32_t* counts, int32_t* starts, int32_t* total,
                                   int32_t* sorted_ids, int32_t* expert_ids, int32_t max_rows,
                                   int32_t* inverse, int32_t item_rows, int32_t* items,
                                   int32_t max_items, int32_t* num_items, int32_t* pairs_out,
                                   int32_t* scratch, int64_t scratch_ints, void* stream) {
  D3_REQUIRE(ids && counts && starts && total && sorted_ids && expert_ids && scratch,
             "sort_routes_wide: null pointer");
  D3_REQUIRE(ids_dtype == D3_DTYPE_I32 || ids_dtype == D3_DTYPE_I64,
             "sort_routes_wide: ids must be int32 or int64");
  D3_REQUIRE(rows >= 0 && top_k >= 1 && top_k <= 64, "sort_routes_wide: bad rows/top_k");
  D3_SUPPORTED(num_experts >= 1 && num_experts <= kMaxSortExperts,
               "sort_routes_wide: num_experts %d not in [1, %d]", num_experts, kMaxSortExperts);
  D3_REQUIRE(tile >= 1 && tile <= 1024, "sort_routes_wide: tile %d not in [1, 1024]", tile);
  const int64_t pairs = static_cast<int64_t>(rows) * top_k;
  D3_REQUIRE(pairs < (1 << 30), "sort_routes_wide: too many pairs");
  const int32_t need = d3_max_sorted_rows(static_cast<int32_t>(pairs), num_experts, tile);
  D3_REQUIRE(max_rows >= need && max_rows % tile == 0,
             "sort_routes_wide: max_rows %d < required %d or not a multiple of tile", max_rows, need);
  D3_REQUIRE(scratch_ints >= d3_sort_wide_scratch_ints(rows, top_k, num_experts),
             "sort_routes_wide: scratch of %lld ints < required %lld",
             static_cast<long long>(scratch_ints),
             static_cast<long long>(d3_sort_wide_scratch_ints(rows, top_k, num_experts)));
  if (items != nullptr) {
    D3_REQUIRE(num_items != nullptr, "sort_routes_wide: items need num_items");
    D3_REQUIRE(item_rows >= tile && item_rows % tile == 0,
               "sort_routes_wide: item_rows must be a positive multiple of tile");
    const int32_t need_items = d3_max_items(static_cast<int32_t>(pairs), num_experts, item_rows);
    D3_REQUIRE(max_items >= need_items, "sort_routes_wide: max_items %d < required %d", max_items,
               need_items);
  } else {
    item_rows = tile;
  }
  const int align_items =
      items != nullptr && max_items >= d3_max_items_aligned(static_cast<int32_t>(pairs), num_experts, item_rows);
  const int chunks = static_cast<int>((pairs + kWideChunk - 1) / kWideChunk);
  int32_t* chunk_counts = scratch;
  int32_t* ranks = scratch + static_cast<int64_t>(chunks) * num_experts;
  const SortOutputs out{counts, starts, total, sorted_ids, expert_ids, max_rows, inverse,
                        reinterpret_cast<int4*>(items), max_items, num_items, pairs_out};
  hipStream_t s = as_stream(stream);
  const size_t rank_shared = sizeof(int) * static_cast<size_t>(num_experts) * (1 + kWideThreads / kWave);
  if (chunks > 0) {
    if (ids_dtype == D3_DTYPE_I64)
      hipLaunchKernelGGL(wide_rank_kernel<true>, dim3(chunks), dim3(kWideThreads), rank_shared, s, ids,
                         rows, row_count, top_k, num_experts, chunk_counts, ranks);
    else
      hipLaunchKernelGGL(wide_rank_kernel<false>, dim3(chunks), dim3(kWideThreads), rank_shared, s, ids,
                         rows, row_count, top_k, num_experts, chunk_counts, ranks);
  }
  // At least one placement workgroup, for the outputs of an empty batch.
  const dim3 place_grid(chunks > 0 ? chunks : 1);
  if (ids_dtype == D3_DTYPE_I64)
    hipLaunchKernelGGL(wide_place_kernel<true>, place_grid, dim3(kPlaceThreads), 0, s, ids, rows, row_count,
                       top_k, num_experts, tile, item_rows, align_items, chunks, chunk_counts, ranks,
                       out);
  else
    hipLaunchKernelGGL(wide_place_kernel<false>, place_grid, dim3(kPlaceThreads), 0, s, ids, rows, row_count,
                       top_k, num_experts, tile, item_rows, align_items, chunks, chunk_counts, ranks,
                       out);
  D3_LAUNCHED("sort_routes_wide");
}
