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
// Wide sort (three launches), the same results as sort_routes_block:
//   1. wide_rank_kernel: one workgroup per chunk of kWideChunk pairs ranks
//      every pair among the chunk's pairs of its expert, in pair order
//      (per-wave ballot matching on the expert-id bits, per-wave counts in
//      LDS, a running per-expert base across sub-chunks), and writes the
//      chunk's expert histogram;
//   2. wide_scan_kernel: one workgroup turns the chunk histograms into
//      per-chunk expert offsets (exclusive scan over chunks, 1024 / E
//      threads per expert), then the padded expert scan, work items, expert
//      ids and sentinel padding;
//   3. wide_scatter_kernel: sorted_ids[starts[e] + chunk offset + rank] = p.
// Scratch: chunk histograms [chunks][E] and ranks [pairs] (int32).
// ---------------------------------------------------------------------------
constexpr int kWideThreads = 256;
constexpr int kWideChunk = 512;
constexpr int kScanRegs = 16;  // chunk counts a scan thread holds in registers

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

__global__ __launch_bounds__(kSortThreads) void wide_scan_kernel(
    int rows, const int32_t* __restrict__ row_count, int top_k, int num_experts, int tile,
    int item_rows, int chunks, int32_t* __restrict__ chunk_counts, SortOutputs out) {
  __shared__ int wave_totals[kSortThreads / kWave];
  __shared__ int partial[kSortThreads];               // [E][share] chunk-range sums
  __shared__ int expert_info[3 * kMaxSortExperts];    // count, start, first item per expert
  const int pairs = live_rows(row_count, rows) * top_k;
  const int tid = threadIdx.x;
  // Expert e is handled by `share` threads (e, j), thread j owning the
  // contiguous chunk range [c0, c1); E <= 512 gives share >= 2.
  const int share = kSortThreads / num_experts;
  const int e = tid / share;
  const int j = tid - e * share;
  const bool owner = e < num_experts;
  const int per = (chunks + share - 1) / share;
  const int c0 = j * per;
  const int c1 = min(chunks, c0 + per);
  const uint32_t cells = static_cast<uint32_t>(chunks) * num_experts;
  const BufferView count_view(chunk_counts, cells * 4);
  auto cell = [&](int c) { return owner && c < c1 ? static_cast<uint32_t>(c * num_experts + e) * 4 : kNoRow; };
  // Per expert: exclusive scan of its chunk counts over the chunks (written
  // back in place as the chunk offsets) and its count.  A thread's range is
  // read in batches of kScanRegs cells, every load of a batch issued before
  // the first use (branch-free: cells outside the range read zero through
  // the buffer bounds); ranges of at most kScanRegs chunks (up to 64k pairs
  // at E = 128, 32k at E = 256) stay in registers between the sum and the
  // write-back, longer ones are read twice.
  int v[kScanRegs];
  int sum = 0;
  for (int b = c0; b < c1; b += kScanRegs) {
#pragma unroll
    for (int q = 0; q < kScanRegs; ++q) v[q] = static_cast<int>(count_view.load4(cell(b + q)));
#pragma unroll
    for (int q = 0; q < kScanRegs; ++q) sum += v[q];
  }
  partial[tid] = sum;
  __syncthreads();
  int base = 0;
  for (int q = 0; q < j; ++q) base += partial[e * share + q];
  if (owner) {
    if (per <= kScanRegs) {
#pragma unroll
      for (int q = 0; q < kScanRegs; ++q) {
        if (c0 + q < c1) chunk_counts[static_cast<size_t>(c0 + q) * num_experts + e] = base;
        base += v[q];
      }
    } else {
      for (int b = c0; b < c1; b += kScanRegs) {
#pragma unroll
        for (int q = 0; q < kScanRegs; ++q) v[q] = static_cast<int>(count_view.load4(cell(b + q)));
#pragma unroll
        for (int q = 0; q < kScanRegs; ++q) {
          if (b + q < c1) chunk_counts[static_cast<size_t>(b + q) * num_experts + e] = base;
          base += v[q];
        }
      }
    }
  }
  int count = 0;
  if (tid < num_experts)
    for (int q = 0; q < share; ++q) count += partial[tid * share + q];
  // Padded expert scan and work items (thread e < E holds expert e).
  const int padded = (count + tile - 1) / tile * tile;
  int total = 0;
  const int start = block_inclusive_scan<kSortThreads>(padded, wave_totals, &total) - padded;
  const int my_items = (count + item_rows - 1) / item_rows;
  int total_items = 0;
  const int item_base =
      block_inclusive_scan<kSortThreads>(my_items, wave_totals, &total_items) - my_items;
  if (tid < num_experts) {
    expert_info[3 * tid] = count;
    expert_info[3 * tid + 1] = start;
    expert_info[3 * tid + 2] = item_base;
    if (out.counts != nullptr) out.counts[tid] = count;
    out.starts[tid] = start;
  }
  __syncthreads();
  // Each expert's sentinel padding, expert ids and work items, spread over
  // its `share` threads.
  if (owner) {
    const int e_count = expert_info[3 * e], e_start = expert_info[3 * e + 1];
    const int e_padded = (e_count + tile - 1) / tile * tile;
    for (int i = e_count + j; i < e_padded; i += share) out.sorted_ids[e_start + i] = pairs;
    if (out.expert_ids != nullptr)
      for (int t = j; t < e_padded / tile; t += share) out.expert_ids[e_start / tile + t] = e;
    if (out.items != nullptr) {
      const int e_items = (e_count + item_rows - 1) / item_rows, e_item_base = expert_info[3 * e + 2];
      for (int it = j; it < e_items; it += share) {
        const int routes = min(item_rows, e_count - it * item_rows);
        out.items[e_item_base + it] = make_int4(e, e_start + it * item_rows, routes, 0);
      }
    }
  }
  for (int i = total + tid; i < out.max_rows; i += kSortThreads) out.sorted_ids[i] = pairs;
  if (out.expert_ids != nullptr)
    for (int i = total / tile + tid; i < out.max_rows / tile; i += kSortThreads) out.expert_ids[i] = -1;
  if (out.items != nullptr)
    for (int i = total_items + tid; i < out.max_items; i += kSortThreads)
      out.items[i] = make_int4(-1, 0, 0, 0);
  if (tid == 0) {
    if (out.total != nullptr) *out.total = total;
    if (out.num_items != nullptr) *out.num_items = total_items;
    if (out.pairs_out != nullptr) *out.pairs_out = pairs;
  }
}

template <bool kI64>
__global__ __launch_bounds__(kWideThreads) void wide_scatter_kernel(
    const void* __restrict__ ids, int rows, const int32_t* __restrict__ row_count, int top_k,
    int num_experts, const int32_t* __restrict__ chunk_counts, const int32_t* __restrict__ ranks,
    const int32_t* __restrict__ starts, int32_t* __restrict__ sorted_ids, int32_t* __restrict__ inverse) {
  const int pairs = live_rows(row_count, rows) * top_k;
  const int p = blockIdx.x * kWideThreads + threadIdx.x;
  if (p >= pairs) return;
  const int e = load_route_id<kI64>(ids, p);
  const int rank = ranks[p];
  if (e < 0 || e >= num_experts || rank < 0) {
    if (inverse != nullptr) inverse[p] = -1;
    return;
  }
  const int position = starts[e] + chunk_counts[static_cast<size_t>(p / kWideChunk) * num_experts + e] + rank;
  sorted_ids[position] = p;
  if (inverse != nullptr) inverse[p] = position;
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
  const int chunks = static_cast<int>((pairs + kWideChunk - 1) / kWideChunk);
  int32_t* chunk_counts = scratch;
  int32_t* ranks = scratch + static_cast<int64_t>(chunks) * num_experts;
  const SortOutputs out{counts, starts, total, sorted_ids, expert_ids, max_rows, inverse,
                        reinterpret_cast<int4*>(items), max_items, num_items, pairs_out};
  hipStream_t s = as_stream(stream);
  const size_t rank_shared = sizeof(int) * static_cast<size_t>(num_experts) * (1 + kWideThreads / kWave);
  const int scatter_blocks = static_cast<int>((pairs + kWideThreads - 1) / kWideThreads);
  if (chunks > 0) {
    if (ids_dtype == D3_DTYPE_I64)
      hipLaunchKernelGGL(wide_rank_kernel<true>, dim3(chunks), dim3(kWideThreads), rank_shared, s, ids,
                         rows, row_count, top_k, num_experts, chunk_counts, ranks);
    else
      hipLaunchKernelGGL(wide_rank_kernel<false>, dim3(chunks), dim3(kWideThreads), rank_shared, s, ids,
                         rows, row_count, top_k, num_experts, chunk_counts, ranks);
  }
  hipLaunchKernelGGL(wide_scan_kernel, dim3(1), dim3(kSortThreads), 0, s, rows, row_count,
                     top_k, num_experts, tile, item_rows, chunks, chunk_counts, out);
  if (scatter_blocks > 0) {
    if (ids_dtype == D3_DTYPE_I64)
      hipLaunchKernelGGL(wide_scatter_kernel<true>, dim3(scatter_blocks), dim3(kWideThreads), 0, s, ids,
                         rows, row_count, top_k, num_experts, chunk_counts, ranks, starts, sorted_ids,
                         inverse);
    else
      hipLaunchKernelGGL(wide_scatter_kernel<false>, dim3(scatter_blocks), dim3(kWideThreads), 0, s, ids,
                         rows, row_count, top_k, num_experts, chunk_counts, ranks, starts, sorted_ids,
                         inverse);
  }
  D3_LAUNCHED("sort_routes_wide");
}
