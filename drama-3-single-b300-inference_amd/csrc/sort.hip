// Standalone route sort: the block sort of route_sort.h in one 1024-thread
// workgroup, for batches whose pair count is too large for the fused front
// end (prefill) and for the reference-named sort operator.
#include "route_sort.h"
#include "status.h"

namespace d3 {
namespace {

constexpr int kSortThreads = 1024;
constexpr int kMaxSortExperts = 512;  // LDS: (4 + 16 waves) * E ints <= 40 KiB

template <bool kI64>
__global__ __launch_bounds__(kSortThreads) void sort_routes_kernel(
    const void* __restrict__ ids, int rows, const int32_t* __restrict__ row_count, int top_k,
    int num_experts, int tile, int item_rows, SortOutputs out) {
  extern __shared__ int smem[];
  const int pairs = live_rows(row_count, rows) * top_k;
  sort_routes_block<kSortThreads, kI64>(ids, pairs, num_experts, tile, item_rows, smem, out);
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
  const size_t shared = sizeof(int) * static_cast<size_t>(sort_shared_ints(kSortThreads, num_experts));
  const SortOutputs out{counts, starts, total, sorted_ids, expert_ids, max_rows, inverse,
                        reinterpret_cast<int4*>(items), max_items, num_items, pairs_out};
  hipStream_t s = as_stream(stream);
  if (ids_dtype == D3_DTYPE_I64)
    hipLaunchKernelGGL(sort_routes_kernel<true>, dim3(1), dim3(kSortThreads), shared, s, ids,
                       rows, row_count, top_k, num_experts, tile, item_rows, out);
  else
    hipLaunchKernelGGL(sort_routes_kernel<false>, dim3(1), dim3(kSortThreads), shared, s, ids,
                       rows, row_count, top_k, num_experts, tile, item_rows, out);
  D3_LAUNCHED("sort_routes");
}
