// Front end of the MoE step: active-slot compaction, top-k routing and
// per-128 FP8 activation quantisation.
//
// All three are row-parallel integer / byte work: one wavefront per routed
// row, one workgroup per quantised row (or for the compaction), coalesced
// 16-byte loads, wave64 ballots and DPP reductions instead of LDS round trips.
#include <math.h>

#include "common.h"
#include "front_rows.h"
#include "route_sort.h"
#include "status.h"

namespace d3 {
namespace {

constexpr int kCompactThreads = 1024;

// ---------------------------------------------------------------------------
// Active-slot compaction: ballot + popcount per wave, wave offsets in LDS.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kCompactThreads) void compact_slots_kernel(
    const uint8_t* __restrict__ occupancy, int num_slots, int32_t* __restrict__ active,
    int32_t* __restrict__ count) {
  __shared__ int wave_counts[kCompactThreads / kWave];
  const int lane = lane_id();
  const int wave = threadIdx.x / kWave;
  int base = 0;
  for (int start = 0; start < num_slots; start += kCompactThreads) {
    const int slot = start + static_cast<int>(threadIdx.x);
    const bool live = slot < num_slots && occupancy[slot] != 0;
    const uint64_t mask = __ballot(live);
    if (lane == 0) wave_counts[wave] = __popcll(mask);
    __syncthreads();
    int offset = base;
    int chunk = 0;
    for (int w = 0; w < kCompactThreads / kWave; ++w) {
      offset += w < wave ? wave_counts[w] : 0;
      chunk += wave_counts[w];
    }
    if (live) active[offset + __popcll(mask & lanemask_lt())] = slot;
    base += chunk;
    __syncthreads();
  }
  for (int i = base + static_cast<int>(threadIdx.x); i < num_slots; i += kCompactThreads)
    active[i] = -1;
  if (threadIdx.x == 0) *count = base;
}

template <int NPL, bool kF32>
__global__ __launch_bounds__(kFrontThreads) void route_kernel(
    const void* __restrict__ logits, int64_t stride, int rows, int num_experts, int top_k,
    const int32_t* __restrict__ row_index, const int32_t* __restrict__ row_count,
    int32_t* __restrict__ ids32, int64_t* __restrict__ ids64, void* __restrict__ weights,
    int weights_f32) {
  const int row = (blockIdx.x * kFrontThreads + threadIdx.x) / kWave;
  if (row >= live_rows(row_count, rows)) return;  // uniform per wave
  const int source = row_index != nullptr ? row_index[row] : row;
  const char* base = static_cast<const char*>(logits) +
                     static_cast<int64_t>(source) * stride * (kF32 ? 4 : 2);
  route_row<NPL, kF32>(base, num_experts, top_k, row, ids32, ids64, weights, weights_f32);
}


template <bool kPrepare>
__global__ __launch_bounds__(kFrontThreads) void quantize_kernel(
    const uint16_t* __restrict__ x, int64_t stride, int rows, int width,
    const int32_t* __restrict__ row_index, const int32_t* __restrict__ row_count,
    uint8_t* __restrict__ q, float* __restrict__ scales, int transposed,
    // prepare_moe_input extras
    const void* __restrict__ router, int router_f32, int64_t router_stride, int num_experts,
    const void* __restrict__ row_slots, int row_slots_i64, int64_t padding_start,
    float* __restrict__ logits_out) {
  const int row = blockIdx.x;
  const int part = threadIdx.x / kWave;
  const int lane = lane_id();
  const int live = live_rows(row_count, rows);
  if (row >= live) return;
  const int source = row_index != nullptr ? row_index[row] : row;
  const int groups = width / kGroup;
  RowPart xrow;
  load_row_part(x + static_cast<int64_t>(source) * stride, width, part, xrow);
  quantize_row_part(xrow, width, part, q + static_cast<int64_t>(row) * width,
                    transposed ? scales + row : scales + static_cast<int64_t>(row) * groups,
                    transposed ? rows : 1);
  if constexpr (kPrepare) {
    if (part != 0) return;
    // Reserved padding rows reuse row 0's routing (moe_input.py:31-37).
    int router_row = row;
    if (row_slots != nullptr) {
      const int64_t slot = row_slots_i64 ? static_cast<const int64_t*>(row_slots)[row]
                                         : static_cast<const int32_t*>(row_slots)[row];
      if (slot >= padding_start) router_row = 0;
    }
    const char* src = static_cast<const char*>(router) +
                      static_cast<int64_t>(router_row) * router_stride * (router_f32 ? 4 : 2);
    for (int column = lane; column < num_experts; column += kWave) {
      const float value = router_f32 ? reinterpret_cast<const float*>(src)[column]
                                     : bf16_to_f32(reinterpret_cast<const uint16_t*>(src)[column]);
      logits_out[static_cast<int64_t>(row) * num_experts + column] = value;
    }
  }
}

// ---------------------------------------------------------------------------
// Fused front end of one MoE step: slot compaction + routing + quantisation
// (one slot / row per workgroup: wave 0 routes it, the 4 waves quantise a
// quarter each) and, in the last workgroup to finish, the route sort.  The last
// workgroup is found with an atomic ticket after the ids were published with
// coherent stores; nobody waits, so the launch cannot deadlock, and the last
// workgroup resets the ticket so the next launch (or graph replay) starts at 0.
// ---------------------------------------------------------------------------
constexpr int kMaxFrontExperts = 512;
constexpr int kMaxFusedSortExperts = kFrontThreads;  // the block sorts: one expert per thread
constexpr int kMaxFusedSortPairs = 8192;
constexpr int kFrontPerThread = kMaxFusedSortPairs / kFrontThreads;
constexpr int kFrontSortInts =
    sort_shared_ints(kFrontThreads, kMaxFusedSortExperts) >
            mask_sort_shared_ints(kFrontThreads, kMaxFusedSortExperts, kMaskWords)
        ? sort_shared_ints(kFrontThreads, kMaxFusedSortExperts)
        : mask_sort_shared_ints(kFrontThreads, kMaxFusedSortExperts, kMaskWords);

struct FrontArgs {
  const uint8_t* occupancy;
  int num_slots;
  int32_t* active;
  int32_t* count;
  const uint16_t* x;
  int64_t x_stride;
  const void* logits;
  int64_t logits_stride;
  int rows;
  const int32_t* row_index;
  const int32_t* row_count;
  int hidden;
  int num_experts;
  int top_k;
  int32_t* ids;
  void* weights;
  int weights_f32;
  uint8_t* q;
  float* scales;
  int tile;
  int item_rows;
  SortOutputs sort;
  int32_t* ticket;
};

template <int NPL, bool kF32, bool kSort>
__global__ __launch_bounds__(kFrontThreads) void moe_front_kernel(FrontArgs a) {
  __shared__ int smem[kSort ? kFrontSortInts : 1];
  __shared__ int ticket_shared;
  const int lane = lane_id();
  const int wave = threadIdx.x / kWave;
  int live;
  int row;
  bool on;
  RowPart xrow;
  RouteLogits<NPL> logits;
  if (a.occupancy != nullptr) {
    // One workgroup per slot: the slot's x row and logits are loaded first
    // (wasted when the slot is free), then every wave counts the occupied
    // slots with ballots: before this slot (= its row) and in total;
    // workgroup 0 also writes the ascending slot list.
    const int slot = blockIdx.x;
    load_row_part(a.x + static_cast<int64_t>(slot) * a.x_stride, a.hidden, wave, xrow);
    // Every wave loads the logits (only wave 0 routes): under a wave-0
    // branch their first use waits inside the branch, before the occupancy
    // loads below are issued.
    load_route_logits<NPL, kF32>(static_cast<const char*>(a.logits) +
                                     static_cast<int64_t>(slot) * a.logits_stride * (kF32 ? 4 : 2),
                                 a.num_experts, logits);
    int running = 0;
    row = 0;
    on = false;
    for (int base = 0, chunk = 0; base < a.num_slots; base += kWave, ++chunk) {
      const bool occupied = base + lane < a.num_slots && a.occupancy[base + lane] != 0;
      const uint64_t mask = __ballot(occupied);
      const int rank = __popcll(mask & lanemask_lt());
      if (slot >= base && slot < base + kWave) {
        row = running + __popcll(mask & (slot - base == 0 ? 0ull : (~0ull >> (kWave - (slot - base)))));
        on = (mask >> (slot - base)) & 1ull;
      }
      if (blockIdx.x == 0 && (chunk % (kFrontThreads / kWave)) == wave && occupied)
        a.active[running + rank] = base + lane;
      running += __popcll(mask);
    }
    live = running;
    if (blockIdx.x == 0) {
      for (int i = live + static_cast<int>(threadIdx.x); i < a.num_slots; i += kFrontThreads)
        a.active[i] = -1;
      if (threadIdx.x == 0) *a.count = live;
    }
  } else {
    row = blockIdx.x;  // one row per workgroup
    live = live_rows(a.row_count, a.rows);
    on = row < live;
    if (on) {
      const int source = a.row_index != nullptr ? a.row_index[row] : row;
      load_row_part(a.x + static_cast<int64_t>(source) * a.x_stride, a.hidden, wave, xrow);
      load_route_logits<NPL, kF32>(static_cast<const char*>(a.logits) +
                                       static_cast<int64_t>(source) * a.logits_stride * (kF32 ? 4 : 2),
                                   a.num_experts, logits);
    }
  }

  if (on) {
    // wave 0 routes the row while every wave quantises its part
    if (wave == 0)
      route_logits<NPL, kSort>(logits, a.num_experts, a.top_k, row, a.ids, nullptr, a.weights,
                               a.weights_f32);
    quantize_row_part(xrow, a.hidden, wave, a.q + static_cast<int64_t>(row) * a.hidden,
                      a.scales + static_cast<int64_t>(row) * (a.hidden / kGroup), 1);
  }

  if constexpr (kSort) {
    wait_stores();  // this workgroup's published ids are visible device-wide
    __syncthreads();
    if (threadIdx.x == 0) ticket_shared = take_ticket(a.ticket);
    __syncthreads();
    if (ticket_shared != static_cast<int>(gridDim.x) - 1) return;
    // The router's ids name distinct experts per row: the row-mask sort,
    // unless its masks exceed the LDS share (then the chunked ballot sort).
    const bool masked = a.num_experts * mask_words(live) <= kMaskWords &&
                        sort_rows_block<kFrontThreads, kFrontPerThread, false, true>(
                            a.ids, live, a.top_k, a.num_experts, a.tile, a.item_rows, smem,
                            kMaskWords, a.sort);
    if (!masked)
      sort_routes_block<kFrontThreads, false, true>(a.ids, live * a.top_k, a.num_experts, a.tile,
                                                     a.item_rows, smem, a.sort);
    if (threadIdx.x == 0) reset_ticket(a.ticket);
  }
}

inline int wave_blocks(int rows) { return (rows + kFrontThreads / kWave - 1) / (kFrontThreads / kWave); }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace d3

using namespace d3;

extern "C" int d3_compact_slots(const uint8_t* occupancy, int32_t num_slots, int32_t* active_slots,
                                int32_t* count, void* stream) {
  D3_REQUIRE(occupancy && active_slots && count, "compact_slots: null pointer");
  D3_REQUIRE(num_slots > 0 && num_slots <= (1 << 20), "compact_slots: num_slots out of range");
  hipLaunchKernelGGL(compact_slots_kernel, dim3(1), dim3(kCompactThreads), 0, as_stream(stream),
                     occupancy, num_slots, active_slots, count);
  D3_LAUNCHED("compact_slots");
}

extern "C" int d3_route(const void* logits, int32_t logits_dtype, int64_t logits_row_stride,
                        int32_t rows, int32_t num_experts, int32_t top_k,
                        const int32_t* row_index, const int32_t* row_count, int32_t* ids32,
                        int64_t* ids64, void* weights, int32_t weights_dtype, void* stream) {
  D3_REQUIRE(rows == 0 || (logits && weights), "route: null logits or weights");
  D3_REQUIRE(rows == 0 || ids32 || ids64, "route: need ids32 or ids64");
  D3_REQUIRE(logits_dtype == D3_DTYPE_BF16 || logits_dtype == D3_DTYPE_F32,
             "route: logits must be bf16 or f32");
  D3_REQUIRE(weights_dtype == D3_DTYPE_BF16 || weights_dtype == D3_DTYPE_F32,
             "route: weights must be bf16 or f32");
  D3_REQUIRE(rows >= 0, "route: negative rows");
  D3_SUPPORTED(num_experts >= 1 && num_experts <= 512, "route: num_experts %d not in [1, 512]",
               num_experts);
  D3_REQUIRE(top_k >= 1 && top_k <= 16 && top_k <= num_experts, "route: bad top_k %d", top_k);
  D3_REQUIRE(logits_row_stride >= num_experts, "route: row stride smaller than num_experts");
  if (rows == 0) {
    clear_error();
    return D3_OK;
  }
  const bool f32 = logits_dtype == D3_DTYPE_F32;
  const int wf32 = weights_dtype == D3_DTYPE_F32;
  const dim3 grid(wave_blocks(rows)), block(kFrontThreads);
  hipStream_t s = as_stream(stream);
#define D3_ROUTE_LAUNCH(NPL)                                                                   \
  if (f32)                                                                                     \
    hipLaunchKernelGGL((route_kernel<NPL, true>), grid, block, 0, s, logits, logits_row_stride, \
                       rows, num_experts, top_k, row_index, row_count, ids32, ids64, weights,  \
                       wf32);                                                                  \
  else                                                                                         \
    hipLaunchKernelGGL((route_kernel<NPL, false>), grid, block, 0, s, logits,                  \
                       logits_row_stride, rows, num_experts, top_k, row_index, row_count,      \
                       ids32, ids64, weights, wf32);
  if (num_experts <= 64) {
    D3_ROUTE_LAUNCH(1)
  } else if (num_experts <= 128) {
    D3_ROUTE_LAUNCH(2)
  } else if (num_experts <= 256) {
    D3_ROUTE_LAUNCH(4)
  } else {
    D3_ROUTE_LAUNCH(8)
  }
#undef D3_ROUTE_LAUNCH
  D3_LAUNCHED("route");
}

extern "C" int d3_quantize_rows(const uint16_t* x, int64_t x_row_stride, int32_t rows,
                                int32_t width, const int32_t* row_index,
                                const int32_t* row_count, uint8_t* q, float* scales,
                                int32_t scales_transposed, void* stream) {
  D3_REQUIRE(rows == 0 || (x && q && scales), "quantize_rows: null pointer");
  D3_REQUIRE(rows >= 0 && width > 0 && width % kGroup == 0,
             "quantize_rows: width %d must be a positive multiple of 128", width);
  D3_SUPPORTED(width <= kMaxRowChunks * 8 * kWave, "quantize_rows: width %d > 4096", width);
  D3_REQUIRE(x_row_stride >= width && x_row_stride % 8 == 0 && aligned16(x),
             "quantize_rows: x rows must be 16-byte aligned (stride %% 8 == 0)");
  D3_REQUIRE(aligned16(q), "quantize_rows: q must be 16-byte aligned");
  if (rows == 0) {
    clear_error();
    return D3_OK;
  }
  hipLaunchKernelGGL(quantize_kernel<false>, dim3(rows), dim3(kFrontThreads), 0,
                     as_stream(stream), x, x_row_stride, rows, width, row_index, row_count, q,
                     scales, scales_transposed ? 1 : 0, nullptr, 0, 0, 0, nullptr, 0, 0,
                     nullptr);
  D3_LAUNCHED("quantize_rows");
}

extern "C" int d3_prepare_moe_input(const uint16_t* x, int64_t x_row_stride, const void* router,
                                    int32_t router_dtype, int64_t router_row_stride,
                                    int32_t rows, int32_t hidden, int32_t num_experts,
                                    const void* row_slots, int32_t row_slots_dtype,
                                    int64_t padding_start, uint8_t* q, float* scales,
                                    float* logits, void* stream) {
  D3_REQUIRE(rows == 0 || (x && router && q && scales && logits), "prepare_moe_input: null pointer");
  D3_REQUIRE(rows >= 0 && hidden > 0 && hidden % kGroup == 0,
             "prepare_moe_input: hidden %d must be a positive multiple of 128", hidden);
  D3_SUPPORTED(hidden <= kMaxRowChunks * 8 * kWave, "prepare_moe_input: hidden %d > 4096", hidden);
  D3_REQUIRE(num_experts > 0 && router_row_stride >= num_experts,
             "prepare_moe_input: bad router shape");
  D3_REQUIRE(router_dtype == D3_DTYPE_BF16 || router_dtype == D3_DTYPE_F32,
             "prepare_moe_input: router must be bf16 or f32");
  D3_REQUIRE(x_row_stride >= hidden && x_row_stride % 8 == 0 && aligned16(x) && aligned16(q),
             "prepare_moe_input: x rows must be 16-byte aligned");
  if (row_slots != nullptr) {
    D3_REQUIRE(row_slots_dtype == D3_DTYPE_I32 || row_slots_dtype == D3_DTYPE_I64,
               "prepare_moe_input: row_slots must be int32 or int64");
    D3_REQUIRE(padding_start > 0, "prepare_moe_input: padding_start must be positive");
  }
  if (rows == 0) {
    clear_error();
    return D3_OK;
  }
  hipLaunchKernelGGL(quantize_kernel<true>, dim3(rows), dim3(kFrontThreads), 0,
                     as_stream(stream), x, x_row_stride, rows, hidden, nullptr, nullptr, q,
                     scales, 1, router, router_dtype == D3_DTYPE_F32 ? 1 : 0, router_row_stride,
                     num_experts, row_slots, row_slots_dtype == D3_DTYPE_I64 ? 1 : 0,
                     padding_start, logits);
  D3_LAUNCHED("prepare_moe_input");
}

extern "C" int d3_moe_front(const uint8_t* occupancy, int32_t num_slots, int32_t* active_slots,
                            int32_t* count, const uint16_t* x, int64_t x_row_stride,
                            const void* logits, int32_t logits_dtype, int64_t logits_row_stride,
                            int32_t rows, const int32_t* row_index, const int32_t* row_count,
                            int32_t hidden, int32_t num_experts, int32_t top_k, int32_t* ids,
                            void* weights, int32_t weights_dtype, uint8_t* q, float* scales,
                            int32_t tile, int32_t item_rows, int32_t* counts, int32_t* starts,
                            int32_t* total, int32_t* sorted_ids, int32_t* expert_ids,
                            int32_t max_rows, int32_t* inverse, int32_t* items,
                            int32_t max_items, int32_t* num_items, int32_t* pairs_out,
                            int32_t* ticket, void* stream) {
  D3_REQUIRE(x && logits && ids && weights && q && scales, "moe_front: null pointer");
  D3_REQUIRE(logits_dtype == D3_DTYPE_BF16 || logits_dtype == D3_DTYPE_F32,
             "moe_front: logits must be bf16 or f32");
  D3_REQUIRE(weights_dtype == D3_DTYPE_BF16 || weights_dtype == D3_DTYPE_F32,
             "moe_front: weights must be bf16 or f32");
  if (occupancy != nullptr) {
    D3_REQUIRE(active_slots && count, "moe_front: occupancy needs active_slots and count");
    D3_REQUIRE(num_slots > 0 && num_slots <= 4096, "moe_front: num_slots %d not in [1, 4096]",
               num_slots);
    D3_REQUIRE(row_index == nullptr && row_count == nullptr,
               "moe_front: occupancy excludes row_index / row_count");
    rows = num_slots;
  }
  D3_REQUIRE(rows >= 0, "moe_front: negative rows");
  D3_REQUIRE(hidden > 0 && hidden % kGroup == 0 && hidden <= kMaxRowChunks * 8 * kWave,
             "moe_front: hidden %d must be a multiple of 128 up to 4096", hidden);
  D3_REQUIRE(x_row_stride >= hidden && x_row_stride % 8 == 0 && aligned16(x) && aligned16(q),
             "moe_front: x rows must be 16-byte aligned");
  D3_SUPPORTED(num_experts >= 1 && num_experts <= kMaxFrontExperts,
               "moe_front: num_experts %d not in [1, %d]", num_experts, kMaxFrontExperts);
  D3_REQUIRE(top_k >= 1 && top_k <= 16 && top_k <= num_experts, "moe_front: bad top_k %d", top_k);
  D3_REQUIRE(logits_row_stride >= num_experts, "moe_front: logits row stride < num_experts");
  const bool sort = sorted_ids != nullptr;
  SortOutputs out{};
  if (sort) {
    D3_REQUIRE(counts && starts && total && expert_ids && ticket, "moe_front: sort outputs");
    D3_REQUIRE(tile >= 1 && tile <= 1024, "moe_front: bad tile %d", tile);
    const int64_t pairs = static_cast<int64_t>(rows) * top_k;
    D3_SUPPORTED(pairs <= kMaxFusedSortPairs,
                 "moe_front: %lld pairs exceed the fused sort (use d3_sort_routes)",
                 static_cast<long long>(pairs));
    D3_SUPPORTED(num_experts <= kMaxFusedSortExperts,
                 "moe_front: the fused sort covers up to %d experts (use d3_sort_routes)",
                 kMaxFusedSortExperts);
    const int32_t need = d3_max_sorted_rows(static_cast<int32_t>(pairs), num_experts, tile);
    D3_REQUIRE(max_rows >= need && max_rows % tile == 0, "moe_front: max_rows %d < required %d",
               max_rows, need);
    if (items != nullptr) {
      D3_REQUIRE(num_items != nullptr && item_rows >= tile && item_rows % tile == 0,
                 "moe_front: items need num_items and item_rows a multiple of tile");
      const int32_t need_items = d3_max_items(static_cast<int32_t>(pairs), num_experts, item_rows);
      D3_REQUIRE(max_items >= need_items, "moe_front: max_items %d < required %d", max_items,
                 need_items);
    } else {
      item_rows = tile;
    }
    out = SortOutputs{counts, starts, total, sorted_ids, expert_ids, max_rows, inverse,
                      reinterpret_cast<int4*>(items), max_items, num_items, pairs_out};
  }
  if (rows == 0 && !sort && occupancy == nullptr) {
    clear_error();
    return D3_OK;
  }
  const FrontArgs args{occupancy, num_slots, active_slots, count, x, x_row_stride, logits,
                       logits_row_stride, rows, row_index, row_count, hidden, num_experts, top_k,
                       ids, weights, weights_dtype == D3_DTYPE_F32 ? 1 : 0, q, scales, tile,
                       item_rows, out, ticket};
  const dim3 grid(rows > 0 ? rows : 1), block(kFrontThreads);
  hipStream_t s = as_stream(stream);
  const bool f32 = logits_dtype == D3_DTYPE_F32;
#define D3_FRONT_LAUNCH(NPL)                                                                  \
  if (f32 && sort)                                                                            \
    hipLaunchKernelGGL((moe_front_kernel<NPL, true, true>), grid, block, 0, s, args);         \
  else if (f32)                                                                               \
    hipLaunchKernelGGL((moe_front_kernel<NPL, true, false>), grid, block, 0, s, args);        \
  else if (sort)                                                                              \
    hipLaunchKernelGGL((moe_front_kernel<NPL, false, true>), grid, block, 0, s, args);        \
  else                                                                                        \
    hipLaunchKernelGGL((moe_front_kernel<NPL, false, false>), grid, block, 0, s, args);
  if (num_experts <= 64) {
    D3_FRONT_LAUNCH(1)
  } else if (num_experts <= 128) {
    D3_FRONT_LAUNCH(2)
  } else if (num_experts <= 256) {
    D3_FRONT_LAUNCH(4)
  } else {
    D3_FRONT_LAUNCH(8)
  }
#undef D3_FRONT_LAUNCH
  D3_LAUNCHED("moe_front");
}
