// Expert GEMMs of the decode step without a route sort.
//
// Decode batches are small (<= 256 rows): the routed expert ids of every row
// fit in a few KB, so each expert-GEMM workgroup can find its own expert's
// routes itself instead of waiting for a sorted route list.  The grid is
// indexed by (expert, row tile): a workgroup knows its weight tile from
// blockIdx alone and issues its first weight loads immediately, before its
// route list is known; the ids (read before the weights, so their wait does
// not include them) give the list while the weights stream.  The step then
// needs no sort: routing + quantisation (d3_moe_front without its sort),
// these two GEMMs, and the weighted combine.
//
// A route list is in ascending pair order (pair = row * top_k + rank) - the
// order of the sorted layout (kernels.py:658-731) - and intermediate rows are
// indexed by pair: gate_up [pairs, 2I] and down [pairs, H].  Every output
// value is the one the sorted chain computes for that pair (same weights
// and activation bytes, same per-element arithmetic).
//
// A workgroup whose expert receives no route exits after its first weight
// loads (those bytes are wasted): the layout suits batches whose routes
// cover most experts; sparse ones are better served by the sorted chain.
//
// The FC1 can also start from the slots themselves (MODE 1), which removes
// the front launch: slot s routes to expert e at rank c when c, the number
// of experts whose routing key beats e's in that row, is below top_k (the
// keys are unique, so this is exactly the rank the front's top-k assigns),
// and the workgroup quantises the x rows of its routes itself with the
// front's per-128 rule.  The routing weights are then computed by the
// combine (routed_combine_kernel) from the same logits with the front's
// function, so every byte matches the chain that runs the front.
#include <algorithm>
#include <mutex>

#include "common.h"
#include "expert_tile.h"
#include "front_rows.h"
#include "status.h"

namespace d3 {
namespace {

constexpr int kMaxSlots = 256;                        // rows per launch (one route per row and expert)
constexpr int kMaxIds = kMaxSlots * 8;                // ids read per workgroup (top_k <= 8)
constexpr int kIdsPerThread = kMaxIds / kGemmThreads;  // 8

struct DecodeArgs {
  const uint8_t* w;  // fragment-major weights [E, n_rows, K]
  const float* ws;   // block scales [E, n_rows / 128, K / 128]
  int n_rows;
  int capacity;  // slot rows
  int top_k;
  int exact_routes;
  // MODE 0 / 2: routed ids of every row and the live row count (front output)
  const int32_t* ids;
  const int32_t* row_count;
  // MODE 0: q rows and their scales; MODE 2: bf16 gate|up by pair
  const void* act;
  const float* act_scales;
  // MODE 1: the slots (occupancy bytes, bf16 x rows, logits) and the
  // front outputs this FC1 writes instead (ids by pair, count, slot list)
  const uint8_t* occupancy;
  const uint16_t* x;
  int64_t x_stride;  // elements
  const void* logits;
  int logits_f32;
  int64_t logits_stride;  // elements
  int num_experts;
  int32_t* ids_out;
  int32_t* count_out;
  int32_t* active_out;
  uint16_t* out_bf16;  // MODE 0 / 1: gate|up [pairs, n_rows]
  float* out_f32;      // MODE 2: down [pairs, n_rows]
  // MODE 2: the slot of every row (FC1's slot list); down rows are then
  // indexed by slot pair, row_slots[row] * top_k + rank (nullptr: by pair)
  const int32_t* row_slots;
  // Route slices per (expert, weight-tile group), set at launch: slice j of
  // an expert takes its route tiles j, j + slices, ... (1: every tile).
  int slices;
};

constexpr int kPassSlots = kGemmThreads / 4;         // MODE 1: 4 lanes per slot
constexpr int kMaxPasses = kMaxSlots / kPassSlots;  // 4: capacity 256
constexpr int kLogitChunks = 8;                      // 16-byte logit loads per lane and pass

// MODE 1 ranking: the logits of one pass of 64 slots (lane q of a slot's quad
// holds 16-byte chunks q, q + 4, ...) and the slot's own logit of this expert.
struct LogitPass {
  int4 chunk[kLogitChunks];
  uint32_t own;
};

// MODE 0: FC1, q rows of the routes' tokens x W13 -> bf16 gate|up by pair.
// MODE 1: FC1 from the slots: routing ranks from the logits, x rows
//         quantised while staged -> bf16 gate|up by pair, ids, count, slots.
// MODE 2: FC2 with the SwiGLU requant in the prologue, gate|up by pair x W2
//         -> fp32 down by pair.
// TILES weight tiles per workgroup, streamed through the registers in halves
// (TILES > 1: routes beyond the first 16 reload the weight tiles).
// PASSES (MODE 1): ranking passes of 64 slots the kernel is built for.
// kWholeFirst: the whole first weight tile is issued before the routes are
// known (batches that reach nearly every expert), instead of its first half
// (otherwise the wasted loads of experts without routes cost more).
// Launches that may split an expert's route tiles over several workgroups
// (route slices): one weight tile per workgroup, except FC1 from the slots
// at K = 2048, whose two bodies together would not fit the registers.
constexpr bool sliced_kernel(int kb, int mode, int tiles) { return tiles == 1 && !(mode == 1 && kb >= 16); }

// LDS of one decode GEMM workgroup (declared once in the kernel, shared by
// both instantiations of its body).
template <int KB, int MODE>
struct DecodeLds {
  static constexpr int kStride = KB * kGroup + 16;  // 16-byte pad: the 16 rows of a ds_read_b128 hit distinct banks
  __attribute__((aligned(16))) uint8_t b_tile[16 * kStride];
  float b_scales[16 * KB];
  int b_target[16];  // pair of each route column, -1 = none
  int route_pairs[kMaxSlots];
  int route_slots[MODE == 1 ? kMaxSlots : 1];
  int chunk_counts[kIdsPerThread * kGemmWaves];
};

// One workgroup's work: expert `expert`, weight tiles [first_tile,
// first_tile + TILES), route tiles first_route, first_route + 16 slices, ...
// kEarly: the first weights are issued before the route scan (every
// workgroup of an unsliced launch, slice 0 of a sliced one); otherwise only
// after it, once the workgroup knows it has a route tile.
template <int KB, int RT, int MODE, int TILES, int PASSES, bool kWholeFirst, bool kEarly>
__device__ __forceinline__ void decode_gemm_body(const DecodeArgs& a, DecodeLds<KB, MODE>& lds, int expert,
                                                 int first_tile, int slice, int slices) {
  const uint8_t* __restrict__ w = a.w;
  const float* __restrict__ ws = a.ws;
  const int n_rows = a.n_rows;
  const int capacity = a.capacity;
  const int top_k = a.top_k;
  const int exact_routes = a.exact_routes;
  const void* __restrict__ act = a.act;
  const float* __restrict__ act_scales = a.act_scales;
  uint16_t* __restrict__ out_bf16 = a.out_bf16;
  float* __restrict__ out_f32 = a.out_f32;
  constexpr int K = KB * kGroup;
  constexpr int kRowsPerWave = RT * 16;
  constexpr int kRowsPerGroup = kGemmWaves * kRowsPerWave;
  constexpr int kStride = DecodeLds<KB, MODE>::kStride;
  constexpr int kChunks = K / 256;
  constexpr int kFirstHalf = KB > 1 ? KB / 2 : KB;
  auto& b_tile = lds.b_tile;
  auto& b_scales = lds.b_scales;
  auto& b_target = lds.b_target;
  auto& route_pairs = lds.route_pairs;
  auto& route_slots = lds.route_slots;
  auto& chunk_counts = lds.chunk_counts;
  const int first_route = 16 * slice;  // this slice's first route tile
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
  const int row16 = lane & 15;
  const int group = lane >> 4;
  auto n0_of = [&](int tile) { return tile * kRowsPerGroup + wave * kRowsPerWave; };

  const uint8_t* wexp = w + static_cast<size_t>(expert) * n_rows * K;
  const float* wsexp = ws + static_cast<size_t>(expert) * (n_rows / kGroup) * KB;
  int32x8 a_frag[RT][KB];
  float w_scale[RT][KB];
  auto load_weights = [&](int tile, int kb0, int kb1) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
        if (kb >= kb0 && kb < kb1)
          a_frag[rt][kb] = load_packed_fragment(wexp + static_cast<size_t>(n0_of(tile) + rt * 16) * K, kb, lane);
  };
  auto load_scales = [&](int tile, int kb0 = 0, int kb1 = KB) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
        if (kb >= kb0 && kb < kb1) w_scale[rt][kb] = wsexp[((n0_of(tile) + rt * 16) / kGroup) * KB + kb];
  };

  int routes;
  if constexpr (MODE == 1) {
    // 1. Occupancy and the first 64 slots' logits, issued before any weight.
    const int elem = a.logits_f32 ? 4 : 2;
    const int chunk_columns = 16 / elem;
    const BufferView logit_view(a.logits, static_cast<uint32_t>(capacity * a.logits_stride * elem));
    const int q = threadIdx.x & 3;
    auto load_pass = [&](int p, LogitPass& lp) {
      const int s = p * kPassSlots + (static_cast<int>(threadIdx.x) >> 2);
      const bool valid = s < capacity;
      const uint32_t row_bytes = static_cast<uint32_t>(s * a.logits_stride * elem);
#pragma unroll
      for (int i = 0; i < kLogitChunks; ++i) {
        const int column = (i * 4 + q) * chunk_columns;
        lp.chunk[i] = logit_view.load16(valid && column < a.num_experts
                                            ? row_bytes + static_cast<uint32_t>(column * elem)
                                            : kNoRow);
      }
      // the dword holding this expert's logit (a bf16 logit is one half of it)
      lp.own = logit_view.load4(valid ? ((row_bytes + static_cast<uint32_t>(expert * elem)) & ~3u) : kNoRow);
    };
    const BufferView occupancy_view(a.occupancy, static_cast<uint32_t>(capacity));
    uint32_t occupied_bits[PASSES];
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
      const int s = p * kWave + lane;
      occupied_bits[p] = occupancy_view.load1(s < capacity ? static_cast<uint32_t>(s) : kNoRow);
    }
    LogitPass lp;
    load_pass(0, lp);
    __builtin_amdgcn_sched_barrier(0);
    // 2. The first half of the first weight tile streams meanwhile.
    if constexpr (kEarly) {
      load_weights(first_tile, 0, kWholeFirst ? KB : kFirstHalf);
      load_scales(first_tile, 0, kWholeFirst ? KB : kFirstHalf);
    }
    __builtin_amdgcn_sched_barrier(0);

    // 3. Occupied slots (every wave holds the masks) and this expert's rank
    //    in every live slot: the keys above its key, summed over the quad.
    uint64_t occ_mask[PASSES];
    int occ_base[PASSES];
    int live = 0;
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
      occ_mask[p] = __ballot(occupied_bits[p] != 0u);
      occ_base[p] = live;
      live += __popcll(occ_mask[p]);
    }
    // An expert has at most one route per live row: a slice whose first
    // route tile lies beyond the live rows has nothing to do (uniform).
    // (Slice 0 always goes on: one of its workgroups writes the slot list.)
    if (slice > 0 && first_route >= live) return;
    const uint32_t own_key_column = static_cast<uint32_t>(expert);
    uint64_t hits[PASSES];
    int my_pair[PASSES];
    auto rank_pass = [&](int p, const LogitPass& lp2) {
      const int bit = static_cast<int>(threadIdx.x) >> 2;  // slot - 64 p
      const int s = p * kPassSlots + bit;
      const uint32_t own_bits = elem == 4 ? lp2.own
                                : (((expert * 2) & 2) ? (lp2.own & 0xffff0000u) : (lp2.own << 16));
      const uint32_t own_key = route_key(__uint_as_float(own_bits), static_cast<int>(own_key_column));
      // Keys of columns past E must rank below every valid key: their bits
      // are set to all ones (ordered value 0; the column is above e, so
      // the tie-break field is below e's too).  Only the last chunk row can
      // hold such columns, and only when E is not a multiple of its width.
      const int row_columns = 4 * chunk_columns;
      const int chunks = (a.num_experts + row_columns - 1) / row_columns;  // uniform
      const bool ragged = a.num_experts % row_columns != 0;
      uint32_t above = 0;
#pragma unroll
      for (int i = 0; i < kLogitChunks; ++i) {
        if (i >= chunks) break;  // uniform
        uint32_t words[4] = {static_cast<uint32_t>(lp2.chunk[i].x), static_cast<uint32_t>(lp2.chunk[i].y),
                             static_cast<uint32_t>(lp2.chunk[i].z), static_cast<uint32_t>(lp2.chunk[i].w)};
        const int column0 = (i * 4 + q) * chunk_columns;
        if (ragged && i == chunks - 1) {
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            if (a.logits_f32) {
              words[k] |= column0 + k < a.num_experts ? 0u : 0xffffffffu;
            } else {
              words[k] |= column0 + 2 * k < a.num_experts ? 0u : 0x0000ffffu;
              words[k] |= column0 + 2 * k + 1 < a.num_experts ? 0u : 0xffff0000u;
            }
          }
        }
        const uint32_t tie0 = 65535u - static_cast<uint32_t>(column0);
        if (a.logits_f32) {
#pragma unroll
          for (int c = 0; c < 4; ++c) above += key_of_bits(words[c], tie0 - c) > own_key ? 1u : 0u;
        } else {
#pragma unroll
          for (int c = 0; c < 8; ++c) {
            const uint32_t bits = (c & 1) ? (words[c >> 1] & 0xffff0000u) : (words[c >> 1] << 16);
            above += key_of_bits(bits, tie0 - c) > own_key ? 1u : 0u;
          }
        }
      }
      above += dpp_move<kDppQuad1032>(above, 0u);
      above += dpp_move<kDppQuad2301>(above, 0u);
      const uint64_t mask = occ_mask[p];
      const bool occupied = s < capacity && ((mask >> bit) & 1ull);
      const int row = occ_base[p] + __popcll(mask & ((1ull << bit) - 1ull));
      const bool routed = occupied && static_cast<int>(above) < top_k;
      hits[p] = __ballot(q == 0 && routed);
      my_pair[p] = row * top_k + static_cast<int>(above);
      if (q == 0 && routed && first_tile == 0 && slice == 0) a.ids_out[my_pair[p]] = expert;
    };
    rank_pass(0, lp);
#pragma unroll
    for (int p = 1; p < PASSES; ++p) {
      hits[p] = 0ull;
      my_pair[p] = 0;
      if (p * kPassSlots < capacity) {
        load_pass(p, lp);
        rank_pass(p, lp);
      }
    }
    // The slot list and the live count (one workgroup writes them).
    if (expert == 0 && first_tile == 0 && slice == 0) {
      if (wave == 0) {
#pragma unroll
        for (int p = 0; p < PASSES; ++p)
          if ((occ_mask[p] >> lane) & 1ull)
            a.active_out[occ_base[p] + __popcll(occ_mask[p] & lanemask_lt())] = p * kWave + lane;
      }
      for (int i = live + static_cast<int>(threadIdx.x); i < capacity; i += kGemmThreads) a.active_out[i] = -1;
      if (threadIdx.x == 0) *a.count_out = live;
    }
    // 4. The route list in slot order (= ascending pair order).
    if (lane == 0) {
#pragma unroll
      for (int p = 0; p < PASSES; ++p) chunk_counts[p * kGemmWaves + wave] = __popcll(hits[p]);
    }
    __syncthreads();
    int chunk_base = 0;
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
      int base = chunk_base;
#pragma unroll
      for (int w2 = 0; w2 < kGemmWaves; ++w2) {
        const int c = chunk_counts[p * kGemmWaves + w2];
        base += w2 < wave ? c : 0;
        chunk_base += c;
      }
      if ((hits[p] >> lane) & 1ull) {
        const int r = base + __popcll(hits[p] & lanemask_lt());
        route_pairs[r] = my_pair[p];
        route_slots[r] = p * kPassSlots + (static_cast<int>(threadIdx.x) >> 2);
      }
    }
    routes = chunk_base;
  } else {
    // 1. The routed ids of every slot row (past the capacity: zeros, masked
    //    below), issued before any weight.
    const uint32_t id_bytes = static_cast<uint32_t>(capacity * top_k) * 4;
    const BufferView id_view(a.ids, id_bytes);
    uint32_t id[kIdsPerThread];
#pragma unroll
    for (int j = 0; j < kIdsPerThread; ++j) {
      const uint32_t p = static_cast<uint32_t>(j * kGemmThreads + threadIdx.x);
      id[j] = id_view.load4(p * 4 < id_bytes ? p * 4 : kNoRow);
    }
    const int rows = live_rows(a.row_count, capacity);
    if (slice > 0 && first_route >= rows) return;  // at most one route per live row (uniform)
    // 2. The first half of the first weight tile streams meanwhile.
    if constexpr (kEarly) {
      load_weights(first_tile, 0, kWholeFirst ? KB : kFirstHalf);
      load_scales(first_tile, 0, kWholeFirst ? KB : kFirstHalf);
    }
    __builtin_amdgcn_sched_barrier(0);

    // 3. This expert's route list, in ascending pair order: pair p = j * 256 +
    //    thread, so the order is (j, wave, lane).
    const int pairs = rows * top_k;
    uint64_t hits[kIdsPerThread];
#pragma unroll
    for (int j = 0; j < kIdsPerThread; ++j) {
      const int p = j * kGemmThreads + static_cast<int>(threadIdx.x);
      hits[j] = __ballot(p < pairs && static_cast<int>(id[j]) == expert);
      if (lane == 0) chunk_counts[j * kGemmWaves + wave] = __popcll(hits[j]);
    }
    __syncthreads();
    int chunk_base = 0;  // routes in chunks before chunk j
#pragma unroll
    for (int j = 0; j < kIdsPerThread; ++j) {
      int base = chunk_base;  // + blocks of earlier waves in chunk j
#pragma unroll
      for (int w2 = 0; w2 < kGemmWaves; ++w2) {
        const int c = chunk_counts[j * kGemmWaves + w2];
        base += w2 < wave ? c : 0;
        chunk_base += c;
      }
      if ((hits[j] >> lane) & 1ull)
        route_pairs[base + __popcll(hits[j] & lanemask_lt())] = j * kGemmThreads + threadIdx.x;
    }
    routes = chunk_base;
  }
  __syncthreads();
  routes = __builtin_amdgcn_readfirstlane(routes);
  // No route for this expert (or for this slice): the loads issued so far
  // are dropped.
  if (routes <= first_route) return;
  const bool exact = routes <= exact_routes;

  // 4. Staging of one route tile (16 threads per route column), branch-free.
  const int stage_col = threadIdx.x >> 4;
  const int stage_part = threadIdx.x & 15;
  int4 b_stage[MODE == 0 ? kChunks : 1];
  float b_stage_scale = 0.0f;
  int stage_pair = -1;
  uint32_t stage_slot = 0;  // MODE 2 with row_slots: the slot of the route's row
  // MODE 1: live (route column, 128-group) units packed densely as in MODE
  // 2; a unit's 16 threads hold 8 bf16 each (the front's quantisation
  // layout), so only live units are quantised.
  constexpr int kStageUnits = MODE == 1 ? (KB < 8 ? KB : 8) : 1;  // unit rows staged at once
  uint4 x_stage[kStageUnits];
  // MODE 2: live (route column, K group) units packed densely: unit
  // u = 16 p + stage_col is column u / KB, group u % KB.
  uint4 g_stage[MODE == 2 ? KB : 1], u_stage[MODE == 2 ? KB : 1];
  int live_units = 0;
  // MODE 1: unit rows [base, base + kStageUnits) of route tile stage_m0.
  int stage_m0 = 0;
  auto fetch_units = [&](int base) __attribute__((always_inline)) {
    if constexpr (MODE == 1) {
      const BufferView x_view(a.x, static_cast<uint32_t>(capacity * a.x_stride * 2));
#pragma unroll
      for (int i = 0; i < kStageUnits; ++i) {
        const int u = (base + i) * 16 + stage_col;
        const int col = u / KB;
        const bool live = u < live_units;
        const int slot = route_slots[min(stage_m0 + col, routes - 1)];
        const uint32_t offset =
            live ? static_cast<uint32_t>(slot * a.x_stride * 2 + ((u - col * KB) * kGroup + stage_part * 8) * 2)
                 : kNoRow;
        const int4 v = x_view.load16(offset);
        x_stage[i] = make_uint4(v.x, v.y, v.z, v.w);
      }
    }
  };
  // Per-128 e4m3 quantisation of the staged units: the arithmetic and lane
  // layout of quantize_row_part, so the tile holds the front's q bytes and
  // scales.
  auto quantize_units = [&](int base) __attribute__((always_inline)) {
    if constexpr (MODE == 1) {
#pragma unroll
      for (int i = 0; i < kStageUnits; ++i) {
        if ((base + i) * 16 >= live_units) break;  // uniform
        const int u = (base + i) * 16 + stage_col;
        const int col = u / KB;
        const int j = u - col * KB;
        const uint32_t words[4] = {x_stage[i].x, x_stage[i].y, x_stage[i].z, x_stage[i].w};
        float v[8];
        float amax = 0.0f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[2 * e] = __uint_as_float(words[e] << 16);
          v[2 * e + 1] = __uint_as_float(words[e] & 0xffff0000u);
          amax = fmaxf(amax, fmaxf(fabsf(v[2 * e]), fabsf(v[2 * e + 1])));
        }
        amax = segment_max<16>(amax);
        const float scale = group_scale(amax);
        const uint32_t lo = quantize_four(v, scale);
        const uint32_t hi = quantize_four(v + 4, scale);
        if (u < live_units) {
          *reinterpret_cast<uint2*>(b_tile + col * kStride + j * kGroup + stage_part * 8) = make_uint2(lo, hi);
          if (stage_part == 0) b_scales[col * KB + j] = scale;
        }
      }
    }
  };
  // MODE 1: the unit rows beyond the first kStageUnits (route tiles with
  // more than 128 / KB routes), staged and quantised after the rest.
  auto stage_rest = [&]() {
    if constexpr (MODE == 1 && kStageUnits < KB) {
      for (int base = kStageUnits; base < KB; base += kStageUnits) {
        if (base * 16 >= live_units) break;  // uniform
        fetch_units(base);
        quantize_units(base);
      }
    }
  };
  auto fetch_tile = [&](int m0) {
    const int r = m0 + stage_col;
    stage_pair = r < routes ? route_pairs[r] : -1;
    if constexpr (MODE == 1) {
      live_units = min(16, routes - m0) * KB;
      stage_m0 = m0;
      fetch_units(0);
    } else if constexpr (MODE == 0) {
      const BufferView rows_view(act, static_cast<uint32_t>(capacity) * K);
      const BufferView scale_view(act_scales, static_cast<uint32_t>(capacity) * KB * 4);
      const int token = stage_pair / top_k;
      const uint32_t offset = stage_pair >= 0 ? static_cast<uint32_t>(token) * K : kNoRow;
#pragma unroll
      for (int j = 0; j < kChunks; ++j) b_stage[j] = rows_view.load16(offset + j * 256 + stage_part * 16);
      b_stage_scale = __uint_as_float(scale_view.load4(
          stage_pair >= 0 && stage_part < KB ? static_cast<uint32_t>(token * KB + stage_part) * 4 : kNoRow));
    } else {
      // The route's slot first (read only with row_slots: an empty view
      // otherwise), so that waiting for the gate|up rows covers it.
      const BufferView slot_view(a.row_slots, a.row_slots != nullptr ? static_cast<uint32_t>(capacity) * 4 : 0u);
      stage_slot = slot_view.load4(stage_pair >= 0 ? static_cast<uint32_t>(stage_pair / top_k) * 4 : kNoRow);
      const BufferView gu_view(act, static_cast<uint32_t>(capacity * top_k) * 2 * K * 2);
      live_units = min(16, routes - m0) * KB;
#pragma unroll
      for (int p = 0; p < KB; ++p) {
        const int u = p * 16 + stage_col;
        const int col = u / KB;
        const bool live = u < live_units;
        const int pair = route_pairs[min(m0 + col, routes - 1)];
        const uint32_t offset =
            live ? static_cast<uint32_t>((pair * 2 * K + (u - col * KB) * kGroup + stage_part * 8) * 2) : kNoRow;
        const int4 gv = gu_view.load16(offset);
        const int4 uv = gu_view.load16(live ? offset + K * 2 : kNoRow);
        g_stage[p] = make_uint4(gv.x, gv.y, gv.z, gv.w);
        u_stage[p] = make_uint4(uv.x, uv.y, uv.z, uv.w);
      }
    }
  };
  auto store_tile = [&]() {
    if constexpr (MODE == 2) {
      // SwiGLU + e4m3 requant of the staged units: the function of
      // silu_mul_quant_kernel, so the tile holds that kernel's bytes.
#pragma unroll
      for (int p = 0; p < KB; ++p) {
        const int u = p * 16 + stage_col;
        if (p * 16 < live_units && u < live_units) {
          const int col = u / KB;
          const int kb = u - col * KB;
          uint2 codes;
          const float scale = swiglu_quant_group(g_stage[p], u_stage[p], &codes);
          *reinterpret_cast<uint2*>(b_tile + col * kStride + kb * kGroup + stage_part * 8) = codes;
          if (stage_part == 0) b_scales[col * KB + kb] = scale;
        }
      }
    } else if constexpr (MODE == 1) {
      quantize_units(0);
      stage_rest();
    } else {
#pragma unroll
      for (int j = 0; j < kChunks; ++j)
        *reinterpret_cast<int4*>(b_tile + stage_col * kStride + j * 256 + stage_part * 16) = b_stage[j];
      if (stage_part < KB) b_scales[stage_col * KB + stage_part] = b_stage_scale;
    }
    int target = stage_pair;
    if constexpr (MODE == 2) {
      if (a.row_slots != nullptr && stage_pair >= 0)
        target = static_cast<int>(stage_slot) * top_k + (stage_pair - (stage_pair / top_k) * top_k);
    }
    if (stage_part == 0) b_target[stage_col] = target;
  };

  // K blocks [kb0, kb1) of one weight tile against the route tile in LDS.
  auto mma_range = [&](floatx4 (&acc)[RT], int kb0, int kb1) {
    const uint8_t* brow = b_tile + row16 * kStride;
    if (exact) {
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        if (kb < kb0 || kb >= kb1) continue;
        bf16x8 b_wide[4];
        widen_fp8(load_fragment(brow, kb, group), b_wide);
        const float b_scale = b_scales[row16 * KB + kb];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          const floatx4 partial = mfma_block_bf16(a_frag[rt][kb], b_wide);
          scale_accumulate(acc[rt], partial, w_scale[rt][kb] * b_scale);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        if (kb < kb0 || kb >= kb1) continue;
        const int32x8 b_frag = load_fragment(brow, kb, group);
        const float b_scale = b_scales[row16 * KB + kb];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          const floatx4 partial = mfma_fp8(a_frag[rt][kb], b_frag);
          scale_accumulate(acc[rt], partial, w_scale[rt][kb] * b_scale);
        }
      }
    }
  };
  auto mma = [&](floatx4 (&acc)[RT]) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) acc[rt] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    mma_range(acc, 0, KB);
  };
  auto epilogue = [&](const floatx4 (&acc)[RT], int tile) {
    const int target = b_target[row16];
    if (target < 0) return;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int n = n0_of(tile) + rt * 16 + group * 4;  // rows n..n+3 of this column
      if constexpr (MODE != 2) {
        const uint32_t lo = f32_to_bf16(acc[rt][0]) | (static_cast<uint32_t>(f32_to_bf16(acc[rt][1])) << 16);
        const uint32_t hi = f32_to_bf16(acc[rt][2]) | (static_cast<uint32_t>(f32_to_bf16(acc[rt][3])) << 16);
        *reinterpret_cast<uint2*>(out_bf16 + static_cast<size_t>(target) * n_rows + n) = make_uint2(lo, hi);
      } else {
        *reinterpret_cast<float4*>(out_f32 + static_cast<size_t>(target) * n_rows + n) =
            make_float4(acc[rt][0], acc[rt][1], acc[rt][2], acc[rt][3]);
      }
    }
  };

  // 5. First route tile between the weight halves, then the tiles.
  fetch_tile(first_route);
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (!kEarly) {  // the whole tile, after the route tile's loads
    load_weights(first_tile, 0, KB);
    load_scales(first_tile, 0, KB);
  } else if constexpr (!kWholeFirst) {
    load_weights(first_tile, kFirstHalf, KB);
    load_scales(first_tile, kFirstHalf, KB);
  }
  store_tile();
  __syncthreads();
  if constexpr (TILES > 1) {
    // Weight tiles stream through the same registers in halves: once the
    // first half of tile tt has been multiplied, the first half of tile
    // tt + 1 is loaded into its registers while the second half of tile tt
    // is multiplied, and so on, so every wave keeps at least half a tile of
    // loads in flight until its last tile (memory returns are counted in
    // issue order, so each wait covers only the half it needs).  A half's
    // block scales load with its weights: loaded after the second half,
    // they would make the first half's wait cover the whole tile.
#pragma unroll
    for (int tt = 0; tt < TILES; ++tt) {
      floatx4 acc[RT];
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) acc[rt] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
      mma_range(acc, 0, kFirstHalf);
      if (tt + 1 < TILES) {
        __builtin_amdgcn_sched_barrier(0);  // the next half reuses these registers
        load_weights(first_tile + tt + 1, 0, kFirstHalf);
        load_scales(first_tile + tt + 1, 0, kFirstHalf);
      }
      mma_range(acc, kFirstHalf, KB);
      if (tt + 1 < TILES) {
        __builtin_amdgcn_sched_barrier(0);
        load_weights(first_tile + tt + 1, kFirstHalf, KB);
        load_scales(first_tile + tt + 1, kFirstHalf, KB);
      }
      epilogue(acc, first_tile + tt);
    }
    // Routes beyond the first 16 (experts busier than a route tile): each
    // further route tile walks the weight tiles again.
    for (int m0 = 16; m0 < routes; m0 += 16) {
      __syncthreads();
      fetch_tile(m0);
      store_tile();
      for (int tt = 0; tt < TILES; ++tt) {
        load_weights(first_tile + tt, 0, KB);
        load_scales(first_tile + tt);
        __syncthreads();
        floatx4 acc[RT];
        mma(acc);
        epilogue(acc, first_tile + tt);
      }
    }
  } else {
    floatx4 acc[RT];
    mma(acc);
    epilogue(acc, first_tile);
    for (int m0 = first_route + 16 * slices; m0 < routes; m0 += 16 * slices) {
      __syncthreads();  // previous route tile fully consumed
      fetch_tile(m0);
      store_tile();
      __syncthreads();
      floatx4 acc2[RT];
      mma(acc2);
      epilogue(acc2, first_tile);
    }
  }
}

template <int KB, int RT, int MODE, int TILES, int PASSES = 1, bool kWholeFirst = false>
__global__ __launch_bounds__(kGemmThreads) __attribute__((amdgpu_waves_per_eu(2))) void decode_gemm_kernel(
    DecodeArgs a) {
  __shared__ DecodeLds<KB, MODE> lds;
  constexpr int kRowsPerGroup = kGemmWaves * RT * 16;
  const int groups = a.n_rows / kRowsPerGroup / TILES;
  // Workgroup -> (expert, tile group, route slice).  Slice-major: every
  // (expert, group)'s slice 0 is dispatched first, the extra slices after;
  // the slice stride is a multiple of 8 workgroups, so the slices of one
  // (expert, group) run on one XCD (workgroup b on XCD b % 8) and share the
  // weight tile in its L2.
  const int slices = sliced_kernel(KB, MODE, TILES) && a.slices > 1 ? a.slices : 1;
  int unit = static_cast<int>(blockIdx.x), slice = 0;
  if (slices > 1) {
    const int units = a.num_experts * groups;
    const int stride = (units + 7) / 8 * 8;
    slice = unit / stride;
    unit -= slice * stride;
    if (unit >= units) return;  // padding up to the stride (uniform)
  }
  const int expert = unit / groups;
  const int first_tile = (unit % groups) * TILES;
  // Two straight-line bodies, never merged: a branch around the early loads
  // inside one body would leave the compiler unable to count outstanding
  // loads at the join.
  if constexpr (sliced_kernel(KB, MODE, TILES)) {
    if (slice > 0) {
      decode_gemm_body<KB, RT, MODE, TILES, PASSES, kWholeFirst, false>(a, lds, expert, first_tile, slice, slices);
      return;
    }
  }
  decode_gemm_body<KB, RT, MODE, TILES, PASSES, kWholeFirst, true>(a, lds, expert, first_tile, slice, slices);
}

bool aligned(const void* p, uintptr_t bytes) { return (reinterpret_cast<uintptr_t>(p) % bytes) == 0; }

constexpr int kResidentGroups = 512;

// Route slices of a one-tile-per-workgroup launch: while (expert, tile)
// workgroups fill less than one round of resident workgroups (few experts),
// each gets up to `capacity / 16` slices that take its route tiles in turn,
// so a busy expert's route tiles run side by side instead of one after
// another in one workgroup (skewed routing: a few experts with up to one
// route per slot).  Slices beyond an expert's route tiles exit after the
// route scan.
int route_slices(int units, int capacity) {
  const int most = (capacity + 15) / 16;
  const int fit = kResidentGroups / (units > 0 ? units : 1);
  return std::max(1, std::min(most, fit));
}

template <int KB, int MODE, int TILES>
void launch_tiles(int num_experts, hipStream_t s, const DecodeArgs& args) {
  const int tiles = args.n_rows / tile_rows_for(KB);
  const int units = num_experts * (tiles / TILES);
  DecodeArgs a = args;
  a.slices = sliced_kernel(KB, MODE, TILES) ? route_slices(units, a.capacity) : 1;
  const int blocks = a.slices > 1 ? (units + 7) / 8 * 8 * a.slices : units;
  const dim3 grid(blocks), block(kGemmThreads);
  if constexpr (MODE == 1) {
    if (a.capacity > kPassSlots) {
      hipLaunchKernelGGL((decode_gemm_kernel<KB, rt_for(KB), MODE, TILES, kMaxPasses>), grid, block, 0, s, a);
      return;
    }
  }
  // Several tiles per workgroup and at least four routes per expert at full
  // capacity (few experts go without routes): the whole first tile is
  // issued up front (c2: -0.7 to -1.1 us per step; at two routes per expert,
  // as for 256 experts, +2.8 us; with one tile per workgroup, as for 16
  // experts, +1.0 to +1.6 us).
  if (TILES > 1 && a.capacity * a.top_k >= 4 * num_experts)
    hipLaunchKernelGGL((decode_gemm_kernel<KB, rt_for(KB), MODE, TILES, 1, true>), grid, block, 0, s, a);
  else
    hipLaunchKernelGGL((decode_gemm_kernel<KB, rt_for(KB), MODE, TILES, 1>), grid, block, 0, s, a);
}

// Weight tiles per workgroup: enough that the whole grid is about one round
// of resident workgroups (two per CU), so each workgroup streams its tiles
// back to back instead of the GPU turning workgroups over; a divisor of the
// expert's tile count (8 for 256 experts of 16 tiles).  Experts averaging
// more than 8 routes at full capacity take one tile per workgroup (each
// further route tile would walk all of a workgroup's tiles again).
int tiles_per_group(int num_experts, int tiles, int capacity, int top_k, int mode) {
  if (capacity * top_k > 8 * num_experts) return 1;
  const int options[] = {1, 2, 4, 6, 8};
  for (int t : options)
    if ((t != 6 || mode != 2) && tiles % t == 0 && num_experts * (tiles / t) <= kResidentGroups)
      return t;
  for (int i = 4; i >= 0; --i)
    if ((options[i] != 6 || mode != 2) && tiles % options[i] == 0) return options[i];
  return 1;
}

template <int KB, int MODE>
void launch_decode(int num_experts, hipStream_t s, const DecodeArgs& a) {
  const int tiles = a.n_rows / tile_rows_for(KB);
  const int t = tiles_per_group(num_experts, tiles, a.capacity, a.top_k, MODE);
  if constexpr (MODE != 2) {
    if (t == 6) {
      launch_tiles<KB, MODE, 6>(num_experts, s, a);
      return;
    }
  }
  if (t == 8)
    launch_tiles<KB, MODE, 8>(num_experts, s, a);
  else if (t == 4)
    launch_tiles<KB, MODE, 4>(num_experts, s, a);
  else if (t == 2)
    launch_tiles<KB, MODE, 2>(num_experts, s, a);
  else
    launch_tiles<KB, MODE, 1>(num_experts, s, a);
}

// ---------------------------------------------------------------------------
// Weighted combine of the step whose FC1 routed the slots itself: one
// workgroup per (slot, 512-column slice).  The down rows of the slot's
// routes (indexed by slot pair: FC2 wrote them there from the slot list)
// are loaded first, with the logits, in one memory round trip; meanwhile wave 0 recomputes the slot's top-k
// weights from its logits with the front's function (route_top_k) and
// rounds them to the stored dtype, so the sum is the chain combine's
// (one fused multiply-add per rank, in rank order).  Slice 0 also stores
// the weights, as the front would.
// ---------------------------------------------------------------------------
constexpr int kRoutedCombineThreads = 128;
constexpr int kRoutedCombineColumns = kRoutedCombineThreads * 4;

struct RoutedCombineArgs {
  const uint8_t* occupancy;
  int capacity;
  const void* logits;
  int64_t logits_stride;  // elements
  int num_experts;
  int top_k;
  int hidden;
  const float* down;  // [pairs, hidden] by pair
  void* weights;      // [capacity, top_k] by row, bf16 or f32
  int weights_f32;
  uint16_t* out;  // [capacity, hidden] by row
};

template <int NPL, bool kF32>
__global__ __launch_bounds__(kRoutedCombineThreads) void routed_combine_kernel(RoutedCombineArgs a) {
  __shared__ float route_w[8];
  const int slices = (a.hidden + kRoutedCombineColumns - 1) / kRoutedCombineColumns;
  const int slot = blockIdx.x / slices;
  const int slice = blockIdx.x % slices;
  const int lane = lane_id();
  const int wave = static_cast<int>(threadIdx.x) / kWave;
  // The slot's logits and down rows (both indexed by slot, so issued before
  // its row is known; every wave loads the logits, so no branch makes the
  // first wait come early).  A free slot's rows are read and dropped.
  RouteLogits<NPL> logits;
  load_route_logits<NPL, kF32>(static_cast<const char*>(a.logits) +
                                     static_cast<int64_t>(slot) * a.logits_stride * (kF32 ? 4 : 2),
                                 a.num_experts, logits);
  const int column = slice * kRoutedCombineColumns + static_cast<int>(threadIdx.x) * 4;
  const bool inside = column < a.hidden;
  const BufferView down_view(a.down, static_cast<uint32_t>(a.capacity * a.top_k * a.hidden) * 4);
  float4 y[8];
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    const int4 v = down_view.load16(
        inside && r < a.top_k
            ? static_cast<uint32_t>(((slot * a.top_k + r) * a.hidden + column) * 4)
            : kNoRow);
    y[r] = make_float4(__int_as_float(v.x), __int_as_float(v.y), __int_as_float(v.z), __int_as_float(v.w));
  }
  // The slot's row: occupied slots below it (every wave counts them).
  int row = 0;
  bool on = false;
  for (int base = 0; base < a.capacity; base += kWave) {
    const bool occupied = base + lane < a.capacity && a.occupancy[base + lane] != 0;
    const uint64_t mask = __ballot(occupied);
    if (slot >= base && slot < base + kWave) {
      const int bit = slot - base;
      row += __popcll(mask & ((1ull << bit) - 1ull));
      on = (mask >> bit) & 1ull;
    } else if (slot >= base + kWave) {
      row += __popcll(mask);
    }
  }
  if (!on) return;  // uniform over the workgroup
  if (wave == 0) {
    const RouteChoice choice = route_top_k<NPL>(logits, a.num_experts, a.top_k);
    if (lane < a.top_k) {
      route_w[lane] = stored_weight(choice.weight, a.weights_f32);
      if (slice == 0) {
        const size_t index = static_cast<size_t>(row) * a.top_k + lane;
        if (a.weights_f32)
          static_cast<float*>(a.weights)[index] = choice.weight;
        else
          static_cast<uint16_t*>(a.weights)[index] = f32_to_bf16(choice.weight);
      }
    }
  }
  __syncthreads();
  float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    if (r < a.top_k) {
      const float wr = route_w[r];
      acc.x = fmaf(wr, y[r].x, acc.x);
      acc.y = fmaf(wr, y[r].y, acc.y);
      acc.z = fmaf(wr, y[r].z, acc.z);
      acc.w = fmaf(wr, y[r].w, acc.w);
    }
  }
  if (inside) *reinterpret_cast<uint2*>(a.out + static_cast<size_t>(row) * a.hidden + column) = pack_bf16x4(acc);
}

// The same combine for E <= 64 (one logit per lane): one wave per (slot,
// 256 columns), which routes the slot itself and reads each rank's weight
// from its lane (readlane): no LDS and no barrier, and twice the workgroups
// of the 512-column form.  For configs 1 and 3 (E16, H1024) 0.4-0.5 us
// faster per step; with 128 or 256 experts every slice pays for the wider
// top-8 and the 512-column form is kept.
constexpr int kWaveCombineColumns = kWave * 4;

template <bool kF32>
__global__ __launch_bounds__(kWave) void routed_combine_wave_kernel(RoutedCombineArgs a) {
  const int slices = (a.hidden + kWaveCombineColumns - 1) / kWaveCombineColumns;
  const int slot = blockIdx.x / slices;
  const int slice = blockIdx.x % slices;
  const int lane = lane_id();
  RouteLogits<1> logits;
  load_route_logits<1, kF32>(static_cast<const char*>(a.logits) +
                                 static_cast<int64_t>(slot) * a.logits_stride * (kF32 ? 4 : 2),
                             a.num_experts, logits);
  const int column = slice * kWaveCombineColumns + lane * 4;
  const bool inside = column < a.hidden;
  const BufferView down_view(a.down, static_cast<uint32_t>(a.capacity * a.top_k * a.hidden) * 4);
  float4 y[8];
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    const int4 v = down_view.load16(
        inside && r < a.top_k
            ? static_cast<uint32_t>(((slot * a.top_k + r) * a.hidden + column) * 4)
            : kNoRow);
    y[r] = make_float4(__int_as_float(v.x), __int_as_float(v.y), __int_as_float(v.z), __int_as_float(v.w));
  }
  int row = 0;
  bool on = false;
  for (int base = 0; base < a.capacity; base += kWave) {
    const bool occupied = base + lane < a.capacity && a.occupancy[base + lane] != 0;
    const uint64_t mask = __ballot(occupied);
    if (slot >= base && slot < base + kWave) {
      const int bit = slot - base;
      row += __popcll(mask & ((1ull << bit) - 1ull));
      on = (mask >> bit) & 1ull;
    } else if (slot >= base + kWave) {
      row += __popcll(mask);
    }
  }
  if (!on) return;
  const RouteChoice choice = route_top_k<1>(logits, a.num_experts, a.top_k);
  if (lane < a.top_k && slice == 0) {
    const size_t index = static_cast<size_t>(row) * a.top_k + lane;
    if (a.weights_f32)
      static_cast<float*>(a.weights)[index] = choice.weight;
    else
      static_cast<uint16_t*>(a.weights)[index] = f32_to_bf16(choice.weight);
  }
  const float mine = stored_weight(choice.weight, a.weights_f32);
  float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    if (r < a.top_k) {
      const float wr = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mine), r));
      acc.x = fmaf(wr, y[r].x, acc.x);
      acc.y = fmaf(wr, y[r].y, acc.y);
      acc.z = fmaf(wr, y[r].z, acc.z);
      acc.w = fmaf(wr, y[r].w, acc.w);
    }
  }
  if (inside) *reinterpret_cast<uint2*>(a.out + static_cast<size_t>(row) * a.hidden + column) = pack_bf16x4(acc);
}

// ---------------------------------------------------------------------------
// Entry points: each validates its arguments into a launch description
// first, so the whole-step entry points can check all three stages before
// launching any.
// ---------------------------------------------------------------------------
struct GemmLaunch {
  int mode;
  int kb;
  int num_experts;
  DecodeArgs args;
};

int check_expert_gemm(int32_t mode, const uint8_t* w, const float* ws, int32_t num_experts,
                      int32_t n, int32_t k, const int32_t* ids, const int32_t* row_count,
                      const int32_t* row_slots, int32_t capacity, int32_t top_k, const void* a,
                      const float* a_scales, int32_t exact_routes, uint16_t* out_bf16,
                      float* out_f32, GemmLaunch* launch) {
  D3_REQUIRE(mode == 0 || mode == 2, "decode_expert_gemm: mode must be 0 (FC1) or 2 (FC2 + SwiGLU)");
  D3_REQUIRE(row_slots == nullptr || mode == 2, "decode_expert_gemm: row_slots is for mode 2 (FC2)");
  D3_REQUIRE(w && ws && ids && a && (mode == 2 || a_scales), "decode_expert_gemm: null pointer");
  D3_REQUIRE(mode == 0 ? out_bf16 != nullptr : out_f32 != nullptr, "decode_expert_gemm: null output");
  D3_REQUIRE(num_experts >= 1 && n > 0 && k > 0 && n % kGroup == 0 && k % 256 == 0,
             "decode_expert_gemm: N=%d must be a multiple of 128 and K=%d of 256", n, k);
  D3_SUPPORTED(capacity >= 1 && capacity <= kMaxSlots && top_k >= 1 && top_k <= 8,
               "decode_expert_gemm: capacity %d (<= %d) x top_k %d (<= 8)", capacity, kMaxSlots,
               top_k);
  D3_REQUIRE(aligned(w, 16) && aligned(a, 16) &&
                 (mode == 0 ? aligned(out_bf16, 8) : aligned(out_f32, 16)),
             "decode_expert_gemm: alignment");
  const int kb = k / kGroup;
  D3_SUPPORTED(mode == 0 ? (kb == 8 || kb == 16) : (kb == 2 || kb == 4 || kb == 6 || kb == 8),
               "decode_expert_gemm: K=%d not in the compiled set", k);
  D3_SUPPORTED(n % tile_rows_for(kb) == 0, "decode_expert_gemm: N=%d must be a multiple of %d", n,
               tile_rows_for(kb));
  DecodeArgs args{};
  args.w = w;
  args.ws = ws;
  args.n_rows = n;
  args.capacity = capacity;
  args.top_k = top_k;
  args.exact_routes = exact_routes;
  args.num_experts = num_experts;
  args.ids = ids;
  args.row_count = row_count;
  args.act = a;
  args.act_scales = a_scales;
  args.out_bf16 = out_bf16;
  args.out_f32 = out_f32;
  args.row_slots = row_slots;
  *launch = GemmLaunch{mode, kb, num_experts, args};
  return D3_OK;
}

void launch_expert_gemm(const GemmLaunch& l, hipStream_t s) {
  if (l.mode == 0) {
    if (l.kb == 8) launch_decode<8, 0>(l.num_experts, s, l.args);
    else launch_decode<16, 0>(l.num_experts, s, l.args);
  } else if (l.mode == 1) {
    if (l.kb == 8) launch_decode<8, 1>(l.num_experts, s, l.args);
    else launch_decode<16, 1>(l.num_experts, s, l.args);
  } else {
    if (l.kb == 2) launch_decode<2, 2>(l.num_experts, s, l.args);
    else if (l.kb == 4) launch_decode<4, 2>(l.num_experts, s, l.args);
    else if (l.kb == 6) launch_decode<6, 2>(l.num_experts, s, l.args);
    else launch_decode<8, 2>(l.num_experts, s, l.args);
  }
}

int check_route_fc1(const uint8_t* w, const float* ws, int32_t num_experts, int32_t n, int32_t k,
                    const uint8_t* occupancy, int32_t capacity, const uint16_t* x, int64_t x_stride,
                    const void* logits, int32_t logits_dtype, int64_t logits_stride, int32_t top_k,
                    int32_t exact_routes, int32_t* ids, int32_t* count, int32_t* active,
                    uint16_t* gate_up, GemmLaunch* launch) {
  D3_REQUIRE(w && ws && occupancy && x && logits && ids && count && active && gate_up,
             "decode_route_fc1: null pointer");
  D3_REQUIRE(logits_dtype == D3_DTYPE_BF16 || logits_dtype == D3_DTYPE_F32,
             "decode_route_fc1: logits must be bf16 or f32");
  D3_REQUIRE(num_experts >= 1 && top_k >= 1 && top_k <= num_experts && n > 0 && k > 0 &&
                 n % kGroup == 0 && k % 256 == 0,
             "decode_route_fc1: bad shape (E=%d, top_k=%d, N=%d, K=%d)", num_experts, top_k, n, k);
  const bool f32 = logits_dtype == D3_DTYPE_F32;
  D3_SUPPORTED(capacity >= 1 && capacity <= kMaxSlots && top_k <= 8,
               "decode_route_fc1: capacity %d (<= %d) x top_k %d (<= 8)", capacity, kMaxSlots, top_k);
  D3_SUPPORTED(num_experts <= kLogitChunks * 4 * (f32 ? 4 : 8),
               "decode_route_fc1: E=%d above the %d a workgroup ranks", num_experts,
               kLogitChunks * 4 * (f32 ? 4 : 8));
  D3_REQUIRE(x_stride >= k && logits_stride >= num_experts, "decode_route_fc1: row strides");
  D3_SUPPORTED(aligned(logits, 16) && logits_stride % (f32 ? 4 : 8) == 0 && aligned(x, 16) &&
                   x_stride % 8 == 0,
               "decode_route_fc1: logits / x rows must be 16-byte aligned");
  D3_SUPPORTED(static_cast<int64_t>(capacity) * x_stride * 2 < (int64_t{1} << 31) &&
                   static_cast<int64_t>(capacity) * logits_stride * 4 < (int64_t{1} << 31),
               "decode_route_fc1: slot rows above 2 GiB");
  D3_REQUIRE(aligned(w, 16) && aligned(gate_up, 8), "decode_route_fc1: alignment");
  const int kb = k / kGroup;
  D3_SUPPORTED(kb == 8 || kb == 16, "decode_route_fc1: K=%d not in the compiled set", k);
  D3_SUPPORTED(n % tile_rows_for(kb) == 0, "decode_route_fc1: N=%d must be a multiple of %d", n,
               tile_rows_for(kb));
  DecodeArgs args{};
  args.w = w;
  args.ws = ws;
  args.n_rows = n;
  args.capacity = capacity;
  args.top_k = top_k;
  args.exact_routes = exact_routes;
  args.occupancy = occupancy;
  args.x = x;
  args.x_stride = x_stride;
  args.logits = logits;
  args.logits_f32 = f32 ? 1 : 0;
  args.logits_stride = logits_stride;
  args.num_experts = num_experts;
  args.ids_out = ids;
  args.count_out = count;
  args.active_out = active;
  args.out_bf16 = gate_up;
  *launch = GemmLaunch{1, kb, num_experts, args};
  return D3_OK;
}

struct CombineLaunch {
  bool f32;
  RoutedCombineArgs args;
};

int check_route_combine(const uint8_t* occupancy, int32_t capacity, const void* logits,
                        int32_t logits_dtype, int64_t logits_stride, int32_t num_experts,
                        int32_t top_k, int32_t hidden, const float* down, void* weights,
                        int32_t weights_dtype, uint16_t* out, CombineLaunch* launch) {
  D3_REQUIRE(occupancy && logits && down && weights && out, "decode_route_combine: null pointer");
  D3_REQUIRE(logits_dtype == D3_DTYPE_BF16 || logits_dtype == D3_DTYPE_F32,
             "decode_route_combine: logits must be bf16 or f32");
  D3_REQUIRE(weights_dtype == D3_DTYPE_BF16 || weights_dtype == D3_DTYPE_F32,
             "decode_route_combine: weights must be bf16 or f32");
  D3_REQUIRE(num_experts >= 1 && top_k >= 1 && top_k <= num_experts && hidden > 0 &&
                 hidden % 4 == 0 && logits_stride >= num_experts,
             "decode_route_combine: bad shape");
  D3_SUPPORTED(capacity >= 1 && capacity <= kMaxSlots && top_k <= 8 && num_experts <= 256,
               "decode_route_combine: capacity %d (<= %d), top_k %d (<= 8), E %d (<= 256)",
               capacity, kMaxSlots, top_k, num_experts);
  D3_REQUIRE(aligned(down, 16) && aligned(out, 8), "decode_route_combine: alignment");
  D3_SUPPORTED(static_cast<int64_t>(capacity) * top_k * hidden * 4 < (int64_t{1} << 31),
               "decode_route_combine: down rows above 2 GiB");
  *launch = CombineLaunch{logits_dtype == D3_DTYPE_F32,
                          RoutedCombineArgs{occupancy, capacity, logits, logits_stride, num_experts,
                                            top_k, hidden, down, weights,
                                            weights_dtype == D3_DTYPE_F32 ? 1 : 0, out}};
  return D3_OK;
}

void launch_route_combine(const CombineLaunch& l, hipStream_t s) {
  if (l.args.num_experts <= kWave) {
    const int wave_slices = (l.args.hidden + kWaveCombineColumns - 1) / kWaveCombineColumns;
    const dim3 grid(l.args.capacity * wave_slices), block(kWave);
    if (l.f32)
      hipLaunchKernelGGL((routed_combine_wave_kernel<true>), grid, block, 0, s, l.args);
    else
      hipLaunchKernelGGL((routed_combine_wave_kernel<false>), grid, block, 0, s, l.args);
    return;
  }
  const int slices = (l.args.hidden + kRoutedCombineColumns - 1) / kRoutedCombineColumns;
  const dim3 grid(l.args.capacity * slices), block(kRoutedCombineThreads);
#define D3_COMBINE(NPL)                                                                  \
  if (l.f32)                                                                             \
    hipLaunchKernelGGL((routed_combine_kernel<NPL, true>), grid, block, 0, s, l.args);  \
  else                                                                                   \
    hipLaunchKernelGGL((routed_combine_kernel<NPL, false>), grid, block, 0, s, l.args);
  if (l.args.num_experts <= 128) {
    D3_COMBINE(2)
  } else {
    D3_COMBINE(4)
  }
#undef D3_COMBINE
}

// The three launches of the decode step on the given intermediate buffers:
// FC1 from the slots (ids, count, active, gate_up), FC2 with the SwiGLU
// requant (down), the routed combine (weights, out).  Everything is checked
// before the first launch.
int decode_step(const uint8_t* w13, const float* s13, const uint8_t* w2, const float* s2,
                int32_t num_experts, int32_t hidden, int32_t intermediate, const uint8_t* occupancy,
                int32_t capacity, const uint16_t* x, int64_t x_stride, const void* logits,
                int32_t logits_dtype, int64_t logits_stride, int32_t top_k, int32_t exact_routes,
                int32_t* ids, void* weights, int32_t weights_dtype, uint16_t* gate_up, float* down,
                int32_t* active, int32_t* count, uint16_t* out, void* stream) {
  D3_REQUIRE(hidden > 0 && intermediate > 0, "decode_step: hidden %d, intermediate %d", hidden,
             intermediate);
  GemmLaunch fc1{}, fc2{};
  CombineLaunch combine{};
  int status = check_route_fc1(w13, s13, num_experts, 2 * intermediate, hidden, occupancy, capacity,
                               x, x_stride, logits, logits_dtype, logits_stride, top_k,
                               exact_routes, ids, count, active, gate_up, &fc1);
  if (status != D3_OK) return status;
  status = check_expert_gemm(2, w2, s2, num_experts, hidden, intermediate, ids, count, active,
                             capacity, top_k, gate_up, nullptr, exact_routes, nullptr, down, &fc2);
  if (status != D3_OK) return status;
  status = check_route_combine(occupancy, capacity, logits, logits_dtype, logits_stride, num_experts,
                               top_k, hidden, down, weights, weights_dtype, out, &combine);
  if (status != D3_OK) return status;
  hipStream_t s = as_stream(stream);
  launch_expert_gemm(fc1, s);
  launch_expert_gemm(fc2, s);
  launch_route_combine(combine, s);
  D3_LAUNCHED("decode_step");
}

// ---------------------------------------------------------------------------
// Allocation-free decode step: the intermediate buffers of decode_step live
// in one device array of this file, `scratch`, for callers that cannot
// allocate (code under graph capture, serving loops that forbid it).  Its
// layout: ids int32 [pairs], route weights [pairs] (the logits' dtype),
// gate_up bf16 [pairs, 2I], down f32 [pairs, H], pairs = capacity * top_k,
// each region at a fixed offset sized for the maximum below.  Nothing in it
// needs clearing: every buffer is written before it is read within a call
// (ids and gate_up for every live route, down for every live route, the
// weights of every live row).  The array is per GPU (each device holds its
// own copy at its own address, found with hipGetSymbolAddress with that
// device current) and every call on a GPU shares it: calls that overlap on
// one GPU race.
// ---------------------------------------------------------------------------
constexpr int kStaticPairs = 512;     // capacity * top_k (64 slots x top-8)
constexpr int kStaticGateUp = 2048;   // 2I
constexpr int kStaticHidden = 2048;   // H
constexpr size_t kScratchIds = 0;
constexpr size_t kScratchWeights = kScratchIds + size_t{kStaticPairs} * 4;
constexpr size_t kScratchGateUp = kScratchWeights + size_t{kStaticPairs} * 4;
constexpr size_t kScratchDown = kScratchGateUp + size_t{kStaticPairs} * kStaticGateUp * 2;
constexpr size_t kScratchBytes = kScratchDown + size_t{kStaticPairs} * kStaticHidden * 4;
static_assert(kScratchWeights % 256 == 0 && kScratchGateUp % 256 == 0 && kScratchDown % 256 == 0,
              "scratch regions keep 256-byte alignment");

constexpr int kMaxDevices = 64;
std::mutex g_scratch_lock;
uint8_t* g_scratch_address[kMaxDevices] = {};

}  // namespace
}  // namespace d3

// The allocation-free decode step's device scratch (6 MiB + 4 KiB per GPU).
static __device__ __align__(256) uint8_t scratch[d3::kScratchBytes];

namespace d3 {
namespace {

// Address of `scratch` on the current device, looked up once per device.
int scratch_address(uint8_t** address) {
  int device = -1;
  hipError_t status = hipGetDevice(&device);
  if (status != hipSuccess)
    return set_error(D3_ERR_HIP, "decode_step_static: hipGetDevice failed: %s", hipGetErrorString(status));
  D3_SUPPORTED(device >= 0 && device < kMaxDevices, "decode_step_static: device %d beyond %d", device,
               kMaxDevices);
  std::lock_guard<std::mutex> guard(g_scratch_lock);
  if (g_scratch_address[device] == nullptr) {
    void* p = nullptr;
    status = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (status != hipSuccess || p == nullptr)
      return set_error(D3_ERR_HIP, "decode_step_static: hipGetSymbolAddress(scratch) failed: %s",
                       hipGetErrorString(status));
    g_scratch_address[device] = static_cast<uint8_t*>(p);
  }
  *address = g_scratch_address[device];
  return D3_OK;
}

}  // namespace
}  // namespace d3

using namespace d3;

extern "C" int d3_decode_expert_gemm(int32_t mode, const uint8_t* w, const float* ws,
                                     int32_t num_experts, int32_t n, int32_t k,
                                     const int32_t* ids, const int32_t* row_count,
                                     const int32_t* row_slots, int32_t capacity, int32_t top_k,
                                     const void* a, const float* a_scales, int32_t exact_routes,
                                     uint16_t* out_bf16, float* out_f32, void* stream) {
  GemmLaunch launch{};
  const int status = check_expert_gemm(mode, w, ws, num_experts, n, k, ids, row_count, row_slots,
                                       capacity, top_k, a, a_scales, exact_routes, out_bf16, out_f32,
                                       &launch);
  if (status != D3_OK) return status;
  launch_expert_gemm(launch, as_stream(stream));
  D3_LAUNCHED("decode_expert_gemm");
}

extern "C" int d3_decode_route_fc1(const uint8_t* w, const float* ws, int32_t num_experts,
                                   int32_t n, int32_t k, const uint8_t* occupancy,
                                   int32_t capacity, const uint16_t* x, int64_t x_stride,
                                   const void* logits, int32_t logits_dtype,
                                   int64_t logits_stride, int32_t top_k, int32_t exact_routes,
                                   int32_t* ids, int32_t* count, int32_t* active,
                                   uint16_t* gate_up, void* stream) {
  GemmLaunch launch{};
  const int status = check_route_fc1(w, ws, num_experts, n, k, occupancy, capacity, x, x_stride,
                                     logits, logits_dtype, logits_stride, top_k, exact_routes, ids,
                                     count, active, gate_up, &launch);
  if (status != D3_OK) return status;
  launch_expert_gemm(launch, as_stream(stream));
  D3_LAUNCHED("decode_route_fc1");
}

extern "C" int d3_decode_route_combine(const uint8_t* occupancy, int32_t capacity,
                                       const void* logits, int32_t logits_dtype,
                                       int64_t logits_stride, int32_t num_experts, int32_t top_k,
                                       int32_t hidden, const float* down, void* weights,
                                       int32_t weights_dtype, uint16_t* out, void* stream) {
  CombineLaunch launch{};
  const int status = check_route_combine(occupancy, capacity, logits, logits_dtype, logits_stride,
                                         num_experts, top_k, hidden, down, weights, weights_dtype,
                                         out, &launch);
  if (status != D3_OK) return status;
  launch_route_combine(launch, as_stream(stream));
  D3_LAUNCHED("decode_route_combine");
}

extern "C" int d3_decode_step(const uint8_t* w13, const float* s13, const uint8_t* w2,
                              const float* s2, int32_t num_experts, int32_t hidden,
                              int32_t intermediate, const uint8_t* occupancy, int32_t capacity,
                              const uint16_t* x, int64_t x_stride, const void* logits,
                              int32_t logits_dtype, int64_t logits_stride, int32_t top_k,
                              int32_t exact_routes, int32_t* ids, void* weights,
                              int32_t weights_dtype, uint16_t* gate_up, float* down,
                              int32_t* active, int32_t* count, uint16_t* out, void* stream) {
  return decode_step(w13, s13, w2, s2, num_experts, hidden, intermediate, occupancy, capacity, x,
                     x_stride, logits, logits_dtype, logits_stride, top_k, exact_routes, ids,
                     weights, weights_dtype, gate_up, down, active, count, out, stream);
}

extern "C" int d3_decode_step_static(const uint8_t* w13, const float* s13, const uint8_t* w2,
                                     const float* s2, int32_t num_experts, int32_t hidden,
                                     int32_t intermediate, const uint8_t* occupancy,
                                     int32_t capacity, const uint16_t* x, int64_t x_stride,
                                     const void* logits, int32_t logits_dtype,
                                     int64_t logits_stride, int32_t top_k, int32_t exact_routes,
                                     int32_t* active, int32_t* count, uint16_t* out,
                                     void* stream) {
  D3_REQUIRE(capacity >= 1 && top_k >= 1 && hidden > 0 && intermediate > 0,
             "decode_step_static: capacity %d, top_k %d, hidden %d, intermediate %d", capacity,
             top_k, hidden, intermediate);
  D3_SUPPORTED(static_cast<int64_t>(capacity) * top_k <= kStaticPairs,
               "decode_step_static: capacity %d x top_k %d = %lld routes exceeds the static "
               "scratch's %d",
               capacity, top_k, static_cast<long long>(capacity) * top_k, kStaticPairs);
  D3_SUPPORTED(2 * intermediate <= kStaticGateUp && hidden <= kStaticHidden,
               "decode_step_static: intermediate %d / hidden %d exceed the static scratch's %d / %d",
               intermediate, hidden, kStaticGateUp / 2, kStaticHidden);
  uint8_t* base = nullptr;
  const int status = scratch_address(&base);
  if (status != D3_OK) return status;
  return decode_step(w13, s13, w2, s2, num_experts, hidden, intermediate, occupancy, capacity, x,
                     x_stride, logits, logits_dtype, logits_stride, top_k, exact_routes,
                     reinterpret_cast<int32_t*>(base + kScratchIds), base + kScratchWeights,
                     logits_dtype, reinterpret_cast<uint16_t*>(base + kScratchGateUp),
                     reinterpret_cast<float*>(base + kScratchDown), active, count, out, stream);
}
