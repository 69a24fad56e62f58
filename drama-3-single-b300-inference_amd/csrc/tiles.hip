// A caller's own sorted-route layout as this library's work items.
//
// The reference's native_moe sorts routes into tiles of block_m sorted
// positions, each tile one expert's (expert_ids[t]), with the sentinel
// `pairs` in the padding at the end of an expert's last tile
// (kernels.py:666-699, 710-731), and its atomic down projection reads the
// activation rows by pair through that layout (moe_atomic.py:14-78).  These
// two small kernels let the library's FC2 run on such a layout: one turns
// the tiles into work items {expert, start, live routes, 0}, the other
// gathers rows stored by pair into sorted order.
#include "common.h"
#include "status.h"

namespace d3 {
namespace {

constexpr int kTileThreads = 256;

// One thread per tile: the live routes of a tile are its entries below the
// sentinel (they form a prefix: padding only ends an expert's segment).
__global__ __launch_bounds__(kTileThreads) void items_from_tiles_kernel(
    const int32_t* __restrict__ sorted_ids, const int32_t* __restrict__ expert_ids,
    const int32_t* __restrict__ total, int tile, int pairs, int max_tiles, int num_experts,
    int4* __restrict__ items, int32_t* __restrict__ num_items) {
  const int t = blockIdx.x * kTileThreads + threadIdx.x;
  int tiles = *total / tile;
  tiles = tiles < 0 ? 0 : (tiles > max_tiles ? max_tiles : tiles);
  if (t == 0) *num_items = tiles;
  if (t >= tiles) return;
  const int expert = expert_ids[t];
  int live = 0;
  for (int j = 0; j < tile; ++j) {
    const int id = sorted_ids[static_cast<int64_t>(t) * tile + j];
    live += (id >= 0 && id < pairs) ? 1 : 0;
  }
  // An out-of-range expert id (a layout the caller did not finish) becomes
  // an empty item instead of an out-of-bounds weight read.
  const bool valid = expert >= 0 && expert < num_experts;
  items[t] = make_int4(valid ? expert : 0, t * tile, valid ? live : 0, 0);
}

// dst row r = src row index[r] for r below the live count, zeros when the
// index is outside [0, src_rows); 16 bytes per thread when rows allow it,
// otherwise 4.
template <int kBytes>
__global__ __launch_bounds__(kTileThreads) void gather_rows_kernel(
    const uint8_t* __restrict__ src, int64_t row_bytes, int64_t src_rows,
    const int32_t* __restrict__ index, const int32_t* __restrict__ row_count, int rows,
    uint8_t* __restrict__ dst) {
  const int live = live_rows(row_count, rows);
  const int64_t per_row = row_bytes / kBytes;
  const int64_t n = static_cast<int64_t>(rows) * per_row;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kTileThreads + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * kTileThreads) {
    const int64_t r = i / per_row;
    const int64_t c = (i - r * per_row) * kBytes;
    if (r >= live) continue;
    const int64_t s = index[r];
    uint8_t* out = dst + r * row_bytes + c;
    if constexpr (kBytes == 16) {
      const int4 v = s >= 0 && s < src_rows ? *reinterpret_cast<const int4*>(src + s * row_bytes + c)
                                            : make_int4(0, 0, 0, 0);
      *reinterpret_cast<int4*>(out) = v;
    } else {
      const uint32_t v = s >= 0 && s < src_rows ? *reinterpret_cast<const uint32_t*>(src + s * row_bytes + c)
                                                : 0u;
      *reinterpret_cast<uint32_t*>(out) = v;
    }
  }
}

}  // namespace
}  // namespace d3

using namespace d3;

extern "C" int d3_items_from_tiles(const int32_t* sorted_ids, const int32_t* expert_ids,
                                   const int32_t* total, int32_t tile, int32_t pairs,
                                   int32_t max_tiles, int32_t num_experts, int32_t* items,
                                   int32_t* num_items, void* stream) {
  D3_REQUIRE(sorted_ids && expert_ids && total && items && num_items, "items_from_tiles: null pointer");
  D3_REQUIRE(tile >= 1 && tile <= 1024 && pairs >= 0 && max_tiles >= 0 && num_experts >= 1,
             "items_from_tiles: tile %d, pairs %d, max_tiles %d, E %d", tile, pairs, max_tiles,
             num_experts);
  D3_REQUIRE(reinterpret_cast<uintptr_t>(items) % 16 == 0, "items_from_tiles: items alignment");
  const int blocks = (max(max_tiles, 1) + kTileThreads - 1) / kTileThreads;
  hipLaunchKernelGGL(items_from_tiles_kernel, dim3(blocks), dim3(kTileThreads), 0, as_stream(stream),
                     sorted_ids, expert_ids, total, tile, pairs, max_tiles, num_experts,
                     reinterpret_cast<int4*>(items), num_items);
  D3_LAUNCHED("items_from_tiles");
}

extern "C" int d3_gather_rows(const void* src, int64_t row_bytes, int64_t src_rows,
                              const int32_t* index, const int32_t* row_count, int32_t rows,
                              void* dst, void* stream) {
  D3_REQUIRE(src && index && dst, "gather_rows: null pointer");
  D3_REQUIRE(row_bytes > 0 && row_bytes % 4 == 0 && src_rows >= 0 && rows >= 0,
             "gather_rows: row_bytes %lld must be a positive multiple of 4",
             static_cast<long long>(row_bytes));
  const auto s = reinterpret_cast<uintptr_t>(src), d = reinterpret_cast<uintptr_t>(dst);
  D3_REQUIRE(s % 4 == 0 && d % 4 == 0, "gather_rows: alignment");
  if (rows == 0) {
    clear_error();
    return D3_OK;
  }
  const bool wide = row_bytes % 16 == 0 && s % 16 == 0 && d % 16 == 0;
  const int64_t work = static_cast<int64_t>(rows) * (row_bytes / (wide ? 16 : 4));
  const int blocks = static_cast<int>(std::min<int64_t>((work + kTileThreads - 1) / kTileThreads, 4096));
  if (wide)
    hipLaunchKernelGGL(gather_rows_kernel<16>, dim3(blocks), dim3(kTileThreads), 0, as_stream(stream),
                       static_cast<const uint8_t*>(src), row_bytes, src_rows, index, row_count, rows,
                       static_cast<uint8_t*>(dst));
  else
    hipLaunchKernelGGL(gather_rows_kernel<4>, dim3(blocks), dim3(kTileThreads), 0, as_stream(stream),
                       static_cast<const uint8_t*>(src), row_bytes, src_rows, index, row_count, rows,
                       static_cast<uint8_t*>(dst));
  D3_LAUNCHED("gather_rows");
}
