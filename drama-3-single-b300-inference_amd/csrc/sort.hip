// Expert histogram, padded exclusive scan and stable route sort in one
// workgroup (1024 threads, 16 waves).
//
// The stable scatter needs, for every (pair p, expert e), the number of
// earlier pairs routed to e.  Each wave finds the lanes holding the same
// expert with one ballot per expert-id bit (lanes agree on every bit <=>
// same expert), so a lane's rank inside its wave is a popcount; per-wave
// counts in LDS give the rank inside the 1024-pair chunk and a running
// per-expert base carries it across chunks.  Everything is integer, so the
// result is independent of scheduling.
#include "common.h"
#include "status.h"

namespace d3 {
namespace {

constexpr int kSortThreads = 1024;
constexpr int kSortWaves = kSortThreads / kWave;
constexpr int kMaxSortExperts = 512;  // LDS: (4 + 16 waves) * E ints <= 40 KiB

template <bool kI64>
__device__ __forceinline__ int load_id(const void* ids, int p) {
  if constexpr (kI64) return static_cast<int>(static_cast<const int64_t*>(ids)[p]);
  return static_cast<const int32_t*>(ids)[p];
}

// Inclusive scan of one int per thread across the workgroup.
__device__ __forceinline__ int block_inclusive_scan(int value, int* wave_totals, int* total) {
  const int lane = lane_id();
  const int wave = threadIdx.x / kWave;
#pragma unroll
  for (int offset = 1; offset < kWave; offset <<= 1) {
    const int other = __shfl_up(value, offset);
    if (lane >= offset) value += other;
  }
  if (lane == kWave - 1) wave_totals[wave] = value;
  __syncthreads();
  int prefix = 0;
  int sum = 0;
#pragma unroll
  for (int w = 0; w < kSortWaves; ++w) {
    prefix += w < wave ? wave_totals[w] : 0;
    sum += wave_totals[w];
  }
  __syncthreads();  // wave_totals is reused by the next scan
  *total = sum;
  return value + prefix;
}

template <bool kI64>
__global__ __launch_bounds__(kSortThreads) void sort_routes_kernel(
    const void* __restrict__ ids, int rows, const int32_t* __restrict__ row_count, int top_k,
    int num_experts, int tile, int32_t* __restrict__ counts_out,
    int32_t* __restrict__ starts_out, int32_t* __restrict__ total_out,
    int32_t* __restrict__ sorted_ids, int32_t* __restrict__ expert_ids, int max_rows,
    int32_t* __restrict__ inverse, int item_rows, int4* __restrict__ items, int max_items,
    int32_t* __restrict__ num_items_out, int32_t* __restrict__ pairs_out) {
  extern __shared__ int smem[];
  int* counts = smem;                       // [E]
  int* starts = counts + num_experts;       // [E]
  int* running = starts + num_experts;      // [E]
  int* first_item = running + num_experts;  // [E]
  int* wave_counts = first_item + num_experts;  // [kSortWaves][E]
  __shared__ int wave_totals[kSortWaves];

  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = tid / kWave;
  const int pairs = live_rows(row_count, rows) * top_k;

  for (int e = tid; e < num_experts; e += kSortThreads) {
    counts[e] = 0;
    running[e] = 0;
  }
  for (int i = tid; i < kSortWaves * num_experts; i += kSortThreads) wave_counts[i] = 0;
  __syncthreads();

  // Histogram (expert_counts_kernel, kernels.py:658-663).
  for (int p = tid; p < pairs; p += kSortThreads) {
    const int e = load_id<kI64>(ids, p);
    if (e >= 0 && e < num_experts) atomicAdd(&counts[e], 1);
  }
  __syncthreads();

  // Padded exclusive scan (expert_offsets_kernel, kernels.py:666-673) and the
  // work-item offsets.  num_experts <= kSortThreads: one expert per thread.
  const int count = tid < num_experts ? counts[tid] : 0;
  const int padded = (count + tile - 1) / tile * tile;
  int total = 0;
  const int start = block_inclusive_scan(padded, wave_totals, &total) - padded;
  const int my_items = (count + item_rows - 1) / item_rows;
  int total_items = 0;
  const int item_base = block_inclusive_scan(my_items, wave_totals, &total_items) - my_items;
  if (tid < num_experts) {
    starts[tid] = start;
    first_item[tid] = item_base;
  }
  __syncthreads();

  // Stable scatter (expert_scatter_kernel, kernels.py:676-699) + inverse.
  int bits = 0;
  while ((1 << bits) < num_experts) ++bits;
  const uint64_t below = lanemask_lt();
  for (int chunk = 0; chunk < pairs; chunk += kSortThreads) {
    const int p = chunk + tid;
    int e = p < pairs ? load_id<kI64>(ids, p) : -1;
    const bool valid = e >= 0 && e < num_experts;
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
      int position = starts[e] + running[e] + rank;
      for (int w = 0; w < wave; ++w) position += wave_counts[w * num_experts + e];
      sorted_ids[position] = p;
      if (inverse != nullptr) inverse[p] = position;
    } else if (p < pairs && inverse != nullptr) {
      inverse[p] = -1;
    }
    __syncthreads();
    if (leader) {
      atomicAdd(&running[e], __popcll(peers));
      wave_counts[wave * num_experts + e] = 0;
    }
    __syncthreads();
  }

  // Padding sentinels, tile -> expert map, work items.
  for (int e = tid; e < num_experts; e += kSortThreads) {
    const int c = counts[e];
    const int s = starts[e];
    const int pad = (c + tile - 1) / tile * tile;
    for (int i = c; i < pad; ++i) sorted_ids[s + i] = pairs;
    for (int b = 0; b < pad / tile; ++b) expert_ids[s / tile + b] = e;
    counts_out[e] = c;
    starts_out[e] = s;
    if (items != nullptr) {
      const int n = (c + item_rows - 1) / item_rows;
      for (int j = 0; j < n; ++j) {
        const int routes = c - j * item_rows < item_rows ? c - j * item_rows : item_rows;
        items[first_item[e] + j] = make_int4(e, s + j * item_rows, routes, 0);
      }
    }
  }
  for (int i = total + tid; i < max_rows; i += kSortThreads) sorted_ids[i] = pairs;
  for (int i = total / tile + tid; i < max_rows / tile; i += kSortThreads) expert_ids[i] = -1;
  if (items != nullptr)
    for (int i = total_items + tid; i < max_items; i += kSortThreads)
      items[i] = make_int4(-1, 0, 0, 0);
  if (tid == 0) {
    *total_out = total;
    if (num_items_out != nullptr) *num_items_out = total_items;
    if (pairs_out != nullptr) *pairs_out = pairs;
  }
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
  const size_t shared = sizeof(int) * static_cast<size_t>(num_experts) * (4 + kSortWaves);
  hipStream_t s = as_stream(stream);
  if (ids_dtype == D3_DTYPE_I64)
    hipLaunchKernelGGL(sort_routes_kernel<true>, dim3(1), dim3(kSortThreads), shared, s, ids,
                       rows, row_count, top_k, num_experts, tile, counts, starts, total,
                       sorted_ids, expert_ids, max_rows, inverse, item_rows,
                       reinterpret_cast<int4*>(items), max_items, num_items, pairs_out);
  else
    hipLaunchKernelGGL(sort_routes_kernel<false>, dim3(1), dim3(kSortThreads), shared, s, ids,
                       rows, row_count, top_k, num_experts, tile, counts, starts, total,
                       sorted_ids, expert_ids, max_rows, inverse, item_rows,
                       reinterpret_cast<int4*>(items), max_items, num_items, pairs_out);
  D3_LAUNCHED("sort_routes");
}
