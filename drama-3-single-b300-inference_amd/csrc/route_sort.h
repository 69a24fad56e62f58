// Expert histogram, padded exclusive scan and stable route sort, as a
// workgroup-level device function (any multiple of 64 threads up to 1024).
//
// Semantics (reference src/drama3/kernels.py:658-731):
//   counts[e]  = #{p : ids[p] == e}
//   starts[e]  = exclusive scan of counts padded to `tile`, *total = sum
//   sorted_ids: pairs of expert e in ascending pair order at starts[e] + rank,
//               padding up to the padded end (and everything from *total on)
//               holds the sentinel `pairs`
//   expert_ids: expert of each tile, -1 from *total / tile on
// plus the unpermute map inverse[p] and work items {e, start, routes, 0}
// covering each expert's routes in chunks of item_rows.
//
// The stable scatter needs, for every pair, the number of earlier pairs of
// the same expert.  Each wave finds the lanes holding the same expert with
// one ballot per expert-id bit (lanes agree on every bit <=> same expert), so
// a lane's rank inside its wave is a popcount; per-wave counts in LDS give the
// rank inside a chunk and a running per-expert base carries it across chunks.
// Everything is integer, so the result does not depend on scheduling.
#pragma once

#include "common.h"

namespace d3 {

// LDS ints needed by sort_routes_block for `threads` threads and E experts.
constexpr int sort_shared_ints(int threads, int experts) {
  return (4 + threads / kWave) * experts + threads / kWave;
}

// kCollect: the ids were published by other workgroups (coherent loads).
template <bool kI64, bool kCollect = false>
__device__ __forceinline__ int load_route_id(const void* ids, int p) {
  if constexpr (kI64) return static_cast<int>(static_cast<const int64_t*>(ids)[p]);
  if constexpr (kCollect) return static_cast<int>(collect_u32(static_cast<const int32_t*>(ids) + p));
  return static_cast<const int32_t*>(ids)[p];
}

// Inclusive scan of one int per thread across the workgroup; *total gets the sum.
template <int THREADS>
__device__ __forceinline__ int block_inclusive_scan(int value, int* wave_totals, int* total) {
  constexpr int kWaves = THREADS / kWave;
  const int lane = lane_id();
  const int wave = threadIdx.x / kWave;
  // Wave inclusive scan on DPP moves: row_shr 1, 2, 4, 8 inside each 16-lane
  // row, then row_bcast 15 / 31 carry the row totals into the later rows.
  uint32_t v = static_cast<uint32_t>(value);
  v += dpp_move<0x111>(v, 0u);
  v += dpp_move<0x112>(v, 0u);
  v += dpp_move<0x114>(v, 0u);
  v += dpp_move<0x118>(v, 0u);
  v += dpp_move<kDppRowBcast15, 0xa>(v, 0u);
  v += dpp_move<kDppRowBcast31, 0xc>(v, 0u);
  value = static_cast<int>(v);
  if (lane == kWave - 1) wave_totals[wave] = value;
  __syncthreads();
  int prefix = 0;
  int sum = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    prefix += w < wave ? wave_totals[w] : 0;
    sum += wave_totals[w];
  }
  __syncthreads();  // wave_totals is reused by the next scan
  *total = sum;
  return value + prefix;
}

struct SortOutputs {
  int32_t* counts;      // optional
  int32_t* starts;      // optional
  int32_t* total;       // optional
  int32_t* sorted_ids;
  int32_t* expert_ids;  // optional
  int max_rows;
  int32_t* inverse;  // optional
  int4* items;       // optional
  int max_items;
  int32_t* num_items;  // optional
  int32_t* pairs_out;  // optional
  // optional: per expert {count + 1, start} as one 64-bit word at the start
  // of a 16-byte record, written last (see kPublishOut)
  int4* expert_state;
};

// Padded exclusive expert scan (starts, total) and work-item offsets
// (first_item, total_items) from counts[E] in LDS: one expert per thread
// (num_experts <= THREADS).  Synchronises; starts / first_item are readable
// by every thread on return.
template <int THREADS>
__device__ __forceinline__ void expert_offsets(const int* counts, int num_experts, int tile,
                                               int item_rows, int* starts, int* first_item,
                                               int* wave_totals, int* total, int* total_items) {
  const int tid = threadIdx.x;
  const int count = tid < num_experts ? counts[tid] : 0;
  const int padded = (count + tile - 1) / tile * tile;
  const int start = block_inclusive_scan<THREADS>(padded, wave_totals, total) - padded;
  const int my_items = (count + item_rows - 1) / item_rows;
  const int item_base = block_inclusive_scan<THREADS>(my_items, wave_totals, total_items) - my_items;
  if (tid < num_experts) {
    starts[tid] = start;
    first_item[tid] = item_base;
  }
  __syncthreads();
}

// Everything but the sorted pair ids: sentinel padding of each expert's
// tile-padded run and of the rows from *total on, expert ids per tile,
// counts / starts, work items, totals and (optional) the published per-expert
// state words.
template <int THREADS, bool kPublishOut>
__device__ void write_sort_tail(const int* counts, const int* starts, const int* first_item,
                                int num_experts, int tile, int item_rows, int total,
                                int total_items, int pairs, const SortOutputs& out) {
  const int tid = threadIdx.x;
  for (int e = tid; e < num_experts; e += THREADS) {
    const int c = counts[e];
    const int s = starts[e];
    const int pad = (c + tile - 1) / tile * tile;
    for (int i = c; i < pad; ++i) out.sorted_ids[s + i] = pairs;
    if (out.expert_ids != nullptr)
      for (int b = 0; b < pad / tile; ++b) out.expert_ids[s / tile + b] = e;
    if (out.counts != nullptr) out.counts[e] = c;
    if (out.starts != nullptr) out.starts[e] = s;
    if (out.items != nullptr) {
      const int n = (c + item_rows - 1) / item_rows;
      for (int j = 0; j < n; ++j) {
        const int routes = c - j * item_rows < item_rows ? c - j * item_rows : item_rows;
        out.items[first_item[e] + j] = make_int4(e, s + j * item_rows, routes, 0);
      }
    }
  }
  for (int i = total + tid; i < out.max_rows; i += THREADS) out.sorted_ids[i] = pairs;
  if (out.expert_ids != nullptr)
    for (int i = total / tile + tid; i < out.max_rows / tile; i += THREADS) out.expert_ids[i] = -1;
  if (out.items != nullptr)
    for (int i = total_items + tid; i < out.max_items; i += THREADS)
      out.items[i] = make_int4(-1, 0, 0, 0);
  if (tid == 0) {
    if (out.total != nullptr) *out.total = total;
    if (out.num_items != nullptr) *out.num_items = total_items;
    if (out.pairs_out != nullptr) *out.pairs_out = pairs;
  }
  if (out.expert_state != nullptr) {
    if constexpr (kPublishOut) {
      wait_stores();  // every sorted id of this thread is visible device-wide
      __syncthreads();
    }
    for (int e = tid; e < num_experts; e += THREADS)
      publish_u64(&out.expert_state[e], (static_cast<uint64_t>(static_cast<uint32_t>(starts[e])) << 32) |
                                            static_cast<uint32_t>(counts[e] + 1));
  }
}

// All THREADS threads of the workgroup must call this (it synchronises).
// num_experts <= THREADS; `smem` holds sort_shared_ints(THREADS, E) ints.
// kPublishOut: the outputs are read by other workgroups of the same launch:
// sorted ids go out with coherent stores, and each expert's state word is
// published only after every sorted id is visible, so a reader that sees
// count + 1 > 0 may read the expert's sorted ids.
template <int THREADS, bool kI64, bool kCollect = false, bool kPublishOut = false>
__device__ void sort_routes_block(const void* __restrict__ ids, int pairs, int num_experts,
                                  int tile, int item_rows, int* smem, const SortOutputs& out) {
  constexpr int kWaves = THREADS / kWave;
  int* counts = smem;                           // [E]
  int* starts = counts + num_experts;           // [E]
  int* running = starts + num_experts;          // [E]
  int* first_item = running + num_experts;      // [E]
  int* wave_counts = first_item + num_experts;  // [kWaves][E]
  int* wave_totals = wave_counts + kWaves * num_experts;  // [kWaves]

  const int tid = threadIdx.x;
  const int wave = tid / kWave;

  // Small batches (decode) read the ids once into registers and reuse them
  // for the scatter; larger ones read them again per chunk.
  constexpr int kCached = 4;
  const bool cache = pairs <= THREADS * kCached;
  int cached[kCached];
#pragma unroll
  for (int c = 0; c < kCached; ++c) {
    const int p = c * THREADS + tid;
    cached[c] = cache && p < pairs ? load_route_id<kI64, kCollect>(ids, p) : -1;
  }

  for (int e = tid; e < num_experts; e += THREADS) {
    counts[e] = 0;
    running[e] = 0;
  }
  for (int i = tid; i < kWaves * num_experts; i += THREADS) wave_counts[i] = 0;
  __syncthreads();

  // Larger batches read kBatch chunks per round trip (all loads in flight
  // before the first use), once for the histogram and once for the scatter.
  constexpr int kBatch = 8;
  auto load_batch = [&](int group, int batch[kBatch]) {
#pragma unroll
    for (int c = 0; c < kBatch; ++c) {
      const int p = group + c * THREADS + tid;
      batch[c] = p < pairs ? load_route_id<kI64, kCollect>(ids, p) : -1;
    }
  };
  int bits = 0;
  while ((1 << bits) < num_experts) ++bits;
  const uint64_t below = lanemask_lt();
  // Lanes of this wave holding the same expert as this lane (one ballot per
  // expert-id bit); invalid lanes get an empty mask.
  auto peers_of = [&](int e, bool valid) {
    uint64_t peers = __ballot(valid);
    for (int b = 0; b < bits; ++b) {
      const bool bit = valid && ((e >> b) & 1);
      const uint64_t set = __ballot(bit);
      peers &= bit ? set : ~set;
    }
    return valid ? peers : 0ull;
  };
  auto count_chunk = [&](int e) {
    if (e >= 0 && e < num_experts) atomicAdd(&counts[e], 1);
  };
  if (cache) {
#pragma unroll
    for (int c = 0; c < kCached; ++c)
      if (c * THREADS < pairs) count_chunk(cached[c]);  // uniform condition
  } else {
    for (int group = 0; group < pairs; group += THREADS * kBatch) {
      int batch[kBatch];
      load_batch(group, batch);
#pragma unroll
      for (int c = 0; c < kBatch; ++c)
        if (group + c * THREADS < pairs) count_chunk(batch[c]);  // uniform condition
    }
  }
  __syncthreads();

  int total = 0, total_items = 0;
  expert_offsets<THREADS>(counts, num_experts, tile, item_rows, starts, first_item, wave_totals,
                          &total, &total_items);

  // One chunk of THREADS pairs (all threads call it: it synchronises).
  auto scatter = [&](int chunk, int e) {
    const int p = chunk + tid;
    const bool valid = p < pairs && e >= 0 && e < num_experts;
    const uint64_t peers = peers_of(e, valid);
    const int rank = __popcll(peers & below);
    const bool leader = valid && rank == 0;
    if (leader) wave_counts[wave * num_experts + e] = __popcll(peers);
    __syncthreads();
    if (valid) {
      int position = starts[e] + running[e] + rank;
      for (int w = 0; w < wave; ++w) position += wave_counts[w * num_experts + e];
      if constexpr (kPublishOut)
        publish_u32(out.sorted_ids + position, static_cast<uint32_t>(p));
      else
        out.sorted_ids[position] = p;
      if (out.inverse != nullptr) out.inverse[p] = position;
    } else if (p < pairs && out.inverse != nullptr) {
      out.inverse[p] = -1;
    }
    __syncthreads();
    if (leader) {
      atomicAdd(&running[e], __popcll(peers));
      wave_counts[wave * num_experts + e] = 0;
    }
    __syncthreads();
  };
  if (cache) {
#pragma unroll
    for (int c = 0; c < kCached; ++c)
      if (c * THREADS < pairs) scatter(c * THREADS, cached[c]);  // uniform condition
  } else {
    for (int group = 0; group < pairs; group += THREADS * kBatch) {
      int batch[kBatch];
      load_batch(group, batch);
#pragma unroll
      for (int c = 0; c < kBatch; ++c)
        if (group + c * THREADS < pairs) scatter(group + c * THREADS, batch[c]);  // uniform
    }
  }

  write_sort_tail<THREADS, kPublishOut>(counts, starts, first_item, num_experts, tile, item_rows,
                                        total, total_items, pairs, out);
}

// ---------------------------------------------------------------------------
// Row-mask sort: the same outputs as sort_routes_block whenever no row names
// an expert twice (always so for router ids: a row's top_k experts are
// distinct).  Then expert e has at most one pair per row, its pairs in
// ascending pair order are its rows in ascending order, and the rank of pair
// (r, k) among them is the number of earlier rows that chose e: a popcount
// over a per-expert bit mask of rows (bit r % 64 of word r / 64) plus the
// expert's running count over the earlier words.  No per-chunk ballots or
// barriers: one LDS atomic OR and one popcount per pair.  The ORs detect a
// repeated expert in a row (the bit is already set); the function then
// returns false having written nothing, and the caller runs
// sort_routes_block.  Requires pairs <= THREADS * kPerThread and
// num_experts * mask_words(rows) <= max_cells.
// ---------------------------------------------------------------------------
constexpr int kMaskWords = 2048;  // mask cells of the fused front's sort (16 KiB)
__host__ __device__ constexpr int mask_words(int rows) { return (rows + 63) / 64; }
// LDS ints of sort_rows_block: masks (2 ints per cell), prefix (1), 3 per
// expert, one per wave.
constexpr int mask_sort_shared_ints(int threads, int experts, int cells) {
  return 3 * cells + 3 * experts + threads / kWave;
}

template <int THREADS, int kPerThread, bool kI64, bool kCollect>
__device__ bool sort_rows_block(const void* __restrict__ ids, int rows, int top_k,
                                int num_experts, int tile, int item_rows, int* smem,
                                int max_cells, const SortOutputs& out) {
  uint64_t* masks = reinterpret_cast<uint64_t*>(smem);  // [E][words], 8-byte aligned
  int* prefix = smem + 2 * max_cells;                    // [E][words]: rows of earlier words
  int* counts = prefix + max_cells;                      // [E]
  int* starts = counts + num_experts;                    // [E]
  int* first_item = starts + num_experts;                // [E]
  int* wave_totals = first_item + num_experts;           // [THREADS / 64]
  const int tid = threadIdx.x;
  const int pairs = rows * top_k;
  const int words = mask_words(rows);
  const int cells = num_experts * words;

  // Every loop over this thread's pairs stops at the last chunk holding a
  // pair (a uniform exit: small batches pay for the chunks they use).
  const int chunks = (pairs + THREADS - 1) / THREADS;
  int expert[kPerThread];
#pragma unroll
  for (int c = 0; c < kPerThread; ++c) {
    const int p = c * THREADS + tid;
    expert[c] = c < chunks && p < pairs ? load_route_id<kI64, kCollect>(ids, p) : -1;
  }
  for (int i = tid; i < cells; i += THREADS) masks[i] = 0;
  __syncthreads();
  // Row of pair p = p / top_k as floor((p + 0.5) * (1 / top_k)) in fp32:
  // (p + 0.5) / top_k lies at least 0.5 / top_k from an integer, and the two
  // roundings move it by at most (p + 0.5) / top_k * 2^-23, less than that
  // for p < 2^22.
  const float inv_k = 1.0f / static_cast<float>(top_k);
  auto row_of = [&](int p) { return static_cast<int>((static_cast<float>(p) + 0.5f) * inv_k); };
  bool repeated = false;
#pragma unroll
  for (int c = 0; c < kPerThread; ++c) {
    if (c >= chunks) break;
    const int e = expert[c];
    const int r = row_of(c * THREADS + tid);
    if (e >= 0 && e < num_experts) {
      const unsigned long long bit = 1ull << (r & 63);
      const unsigned long long before =
          atomicOr(reinterpret_cast<unsigned long long*>(&masks[e * words + (r >> 6)]), bit);
      repeated |= (before & bit) != 0;
    }
  }
  if (__syncthreads_or(repeated)) return false;
  for (int e = tid; e < num_experts; e += THREADS) {
    int running = 0;
    for (int w = 0; w < words; ++w) {
      prefix[e * words + w] = running;
      running += __popcll(masks[e * words + w]);
    }
    counts[e] = running;
  }
  __syncthreads();
  int total = 0, total_items = 0;
  expert_offsets<THREADS>(counts, num_experts, tile, item_rows, starts, first_item, wave_totals,
                          &total, &total_items);
#pragma unroll
  for (int c = 0; c < kPerThread; ++c) {
    if (c >= chunks) break;
    const int p = c * THREADS + tid;
    const int e = expert[c];
    if (e >= 0 && e < num_experts) {
      const int r = row_of(p);
      const int cell = e * words + (r >> 6);
      const uint64_t earlier = masks[cell] & ((1ull << (r & 63)) - 1ull);
      const int position = starts[e] + prefix[cell] + __popcll(earlier);
      out.sorted_ids[position] = p;
      if (out.inverse != nullptr) out.inverse[p] = position;
    } else if (p < pairs && out.inverse != nullptr) {
      out.inverse[p] = -1;
    }
  }
  write_sort_tail<THREADS, false>(counts, starts, first_item, num_experts, tile, item_rows, total,
                                  total_items, pairs, out);
  return true;
}

}  // namespace d3
