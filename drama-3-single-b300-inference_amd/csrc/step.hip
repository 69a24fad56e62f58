// The whole decode MoE step in one launch: slot compaction, top-k routing,
// FP8 quantisation, route sort, FC1, SwiGLU + FP8 requantisation, FC2 and
// the weighted top-k combine (reference: DramaModel.routed_moe's decode path,
// src/drama3/model.py:520-583, with kernels.py:325-357 / 658-779).
//
// Why one launch: on MI355X the step is a 600 MB weight stream (c2) wrapped
// in latency-bound work (routing, sort, requant, combine).  As separate
// kernels, each boundary drains the GPU and the latency-bound kernels run
// with HBM idle.  Here every expert-GEMM workgroup issues its weight loads
// as soon as it starts, before it knows its routes, so the weight stream
// runs under the front end, and each piece of latency-bound work is done by
// whichever workgroup finishes the data it needs.
//
// Workgroups are tasks, in blockIdx order (S = slot capacity, T1 / T2 = FC1 /
// FC2 row tiles per expert):
//   [0, S)                       front: compaction, routing + quantisation of
//                                row blockIdx; the last of them (ticket) runs
//                                the route sort and publishes, per expert,
//                                {count + 1, start} in expert_state.
//   [S, S + E*T1)                FC1 tile t of expert e: weights, then wait for
//                                expert_state[e]; the last of the expert's T1
//                                tiles (ticket) computes the expert's SwiGLU
//                                requant and sets its act_done flag.
//   [S + E*T1, S + E*(T1+T2))    FC2 tile t of expert e: weights, then wait for
//                                act_done[e] (or count 0); per route, the last
//                                of a token's top_k contributions to the tile
//                                (ticket) writes the combined output columns.
//   last                         janitor: waits for every other workgroup to
//                                leave, then clears the per-expert state.
// (Expert tasks dispatched after the first resident wave read their expert's
// state first and, when it is ready, stage their activations while the
// weights stream, like the multi-kernel GEMM.)
// A task waits only for tasks with a smaller blockIdx, and workgroups are
// dispatched in blockIdx order, so the waits always end; each wait is also
// bounded (error word set, task skipped) so every wave exits regardless.
//
// Data handed between workgroups is written with coherent (sc1,
// write-through) stores, waited for, then signalled with an agent-scope
// atomic; readers load it with coherent loads.  MI355X's XCDs have separate
// L2s, so plain stores would stay in the writer's L2.
//
// Every counter is zero between launches: each ticket is reset by the task
// that took its last value, and the janitor clears the per-expert state and
// the exit count.  The error word is never cleared here.
#include "common.h"
#include "expert_tile.h"
#include "front_rows.h"
#include "route_sort.h"
#include "status.h"

namespace d3 {
namespace {

constexpr int kStepThreads = kGemmThreads;  // 256: four waves
static_assert(kStepThreads == kFrontThreads, "front and GEMM tasks share the block size");
constexpr int kSortTile = 16;     // sorted-layout padding (same as the multi-kernel step)
constexpr int kMaxSpins = 1 << 20;  // >= ~0.5 s of polling before a wait gives up
constexpr int kActBatch = 4;      // requant units per thread loaded before arithmetic
// Workgroups dispatched after the first resident wave (2 per CU, 256 CUs)
// expect to find the route sort done.
constexpr int kFirstWave = 512;

constexpr int kCoherent = 16;  // cache policy sc1: device-coherent access

// Buffer view whose loads are coherent across the XCDs' L2s.
struct CoherentBuffer {
  BufferView view;
  __device__ CoherentBuffer(const void* base, uint32_t bytes) : view(base, bytes) {}
  __device__ int4 load16(uint32_t offset) const { return view.load16<kCoherent>(offset); }
  __device__ uint32_t load4(uint32_t offset) const { return view.load4<kCoherent>(offset); }
};

struct StepArgs {
  const uint8_t* occupancy;
  int num_slots;
  int32_t* active;
  int32_t* count;
  const uint16_t* x;
  int64_t x_stride;
  const uint16_t* logits;
  int64_t logits_stride;
  int hidden;
  int num_experts;
  int intermediate;
  int top_k;
  const uint8_t* w13;  // fragment-major [E, 2I, H]
  const float* s13;
  const uint8_t* w2;  // fragment-major [E, H, I]
  const float* s2;
  int exact_routes;
  int32_t* ids;
  void* weights;
  int weights_f32;
  uint8_t* q;
  float* x_scales;
  int32_t* sorted_ids;
  int max_rows;
  uint16_t* gate_up;
  uint8_t* act;
  float* act_scales;
  float* down;
  uint16_t* out;
  int32_t* error;
  int32_t* front_ticket;
  int32_t* exit_count;
  int4* expert_state;  // {count + 1, start, act_done, FC1 ticket}
  int32_t* combine_tickets;  // [S, T2]
  int fc1_tiles;
  int fc2_tiles;
};

// Sync words (int32, zero between launches): error, front ticket, exit
// count, pad, expert_state[E] (4 ints each), combine tickets [S * T2].
constexpr int kSyncHeader = 4;

__device__ __forceinline__ float collect_route_weight(const void* weights, int weights_f32,
                                                      int index) {
  if (weights_f32) return __uint_as_float(collect_u32(static_cast<const float*>(weights) + index));
  const uint32_t word = collect_u32(static_cast<const uint16_t*>(weights) + (index & ~1));
  return bf16_to_f32(static_cast<uint16_t>((index & 1) ? word >> 16 : word & 0xffffu));
}

// ---------------------------------------------------------------------------
// Front task: one row (the multi-kernel moe_front_kernel, with coherent
// stores), then the route sort in the last front workgroup.
// ---------------------------------------------------------------------------
template <int NPL>
__device__ void front_task(const StepArgs& a, int row, int* smem, int* bcast) {
  const int lane = lane_id();
  const int wave = threadIdx.x / kWave;
  // Every wave scans the occupancy to find the live count and its row's
  // slot; workgroup 0 also writes the ascending slot list.
  int running = 0;
  int source = -1;
  for (int base = 0, chunk = 0; base < a.num_slots; base += kWave, ++chunk) {
    const bool on = base + lane < a.num_slots && a.occupancy[base + lane] != 0;
    const uint64_t mask = __ballot(on);
    const int rank = __popcll(mask & lanemask_lt());
    const int here = __popcll(mask);
    if (row >= running && row < running + here) {
      const uint64_t hit = __ballot(on && rank == row - running);
      source = base + __ffsll(static_cast<unsigned long long>(hit)) - 1;
    }
    if (row == 0 && (chunk % (kStepThreads / kWave)) == wave && on) a.active[running + rank] = base + lane;
    running += here;
  }
  const int live = running;
  if (row == 0) {
    for (int i = live + static_cast<int>(threadIdx.x); i < a.num_slots; i += kStepThreads) a.active[i] = -1;
    if (threadIdx.x == 0) *a.count = live;
  }
  if (row < live) {
    RowPart xrow;
    load_row_part(a.x + static_cast<int64_t>(source) * a.x_stride, a.hidden, wave, xrow);
    if (wave == 0) {
      const char* lbase = reinterpret_cast<const char*>(a.logits + static_cast<int64_t>(source) * a.logits_stride);
      route_row<NPL, false, true>(lbase, a.num_experts, a.top_k, row, a.ids, nullptr, a.weights,
                                  a.weights_f32);
    }
    quantize_row_part<true>(xrow, a.hidden, wave, a.q + static_cast<int64_t>(row) * a.hidden,
                            a.x_scales + static_cast<int64_t>(row) * (a.hidden / kGroup), 1);
  }
  wait_stores();  // this row's ids, weights and q are visible device-wide
  __syncthreads();
  if (threadIdx.x == 0) bcast[0] = take_ticket(a.front_ticket);
  __syncthreads();
  if (bcast[0] != a.num_slots - 1) return;
  SortOutputs out{};
  out.sorted_ids = a.sorted_ids;
  out.max_rows = a.max_rows;
  out.expert_state = a.expert_state;
  sort_routes_block<kStepThreads, false, true, true>(a.ids, live * a.top_k, a.num_experts,
                                                     kSortTile, kSortTile, smem, out);
  if (threadIdx.x == 0) reset_ticket(a.front_ticket);
}

// ---------------------------------------------------------------------------
// SwiGLU + requant of one expert's routes (rows [first, first + routes) of
// gate_up), by the last FC1 task of the expert: the same arithmetic as
// silu_mul_quant_kernel, so the same bytes.
// ---------------------------------------------------------------------------
template <int KB2>
__device__ void act_finish(const StepArgs& a, int4* state, int routes, int first) {
  constexpr int I = KB2 * kGroup;
  const int seg = threadIdx.x >> 4;
  const int part = threadIdx.x & 15;
  const int units = routes * KB2;
  const CoherentBuffer gate_up(a.gate_up, static_cast<uint32_t>(a.max_rows) * 2 * I * 2);
  for (int base = 0; base < units; base += 16 * kActBatch) {
    uint4 g[kActBatch], u[kActBatch];
#pragma unroll
    for (int p = 0; p < kActBatch; ++p) {
      const int unit = base + p * 16 + seg;
      if (unit < units) {
        const int col = unit / KB2;
        const uint32_t offset = static_cast<uint32_t>(((first + col) * 2 * I + (unit - col * KB2) * kGroup + part * 8) * 2);
        const int4 gv = gate_up.load16(offset);
        const int4 uv = gate_up.load16(offset + I * 2);
        g[p] = make_uint4(gv.x, gv.y, gv.z, gv.w);
        u[p] = make_uint4(uv.x, uv.y, uv.z, uv.w);
      }
    }
#pragma unroll
    for (int p = 0; p < kActBatch; ++p) {
      const int unit = base + p * 16 + seg;
      if (unit < units) {  // whole 16-lane rows agree
        const int col = unit / KB2;
        const int grp = unit - col * KB2;
        uint2 codes;
        const float scale = swiglu_quant_group(g[p], u[p], &codes);
        const size_t row = static_cast<size_t>(first + col);
        publish_u64(a.act + row * I + grp * kGroup + part * 8,
                    (static_cast<uint64_t>(codes.y) << 32) | codes.x);
        if (part == 0) publish_u32(a.act_scales + row * KB2 + grp, __float_as_uint(scale));
      }
    }
  }
  wait_stores();
  __syncthreads();
  if (threadIdx.x == 0) {
    publish_u32(&state->z, 1u);  // act_done
    reset_ticket(&state->w);
    wait_stores();  // before this workgroup's exit count
  }
}

// ---------------------------------------------------------------------------
// Expert GEMM task: one row tile of one expert against all of its routes
// (the multi-kernel expert_gemm_kernel's arithmetic, fragment-major weights).
//   kFC1: q rows of the routes' tokens x W13 -> bf16 gate|up at sorted
//         positions; FC2: act rows at sorted positions x W2 -> fp32 per pair.
// Workgroups of the first resident wave start before routing is known: they
// load their weight tile, then wait.  Later ones normally find their expert
// ready: they read its state first and issue the activation loads before
// (FC2) or between the halves of (FC1) the weight loads, so the staging
// latency hides under the weight stream as in the multi-kernel GEMM.
// ---------------------------------------------------------------------------
template <int KB, int RT, bool kFC1, int KB2, int TILES>
__device__ void expert_task(const StepArgs& a, int expert, int tile_group, uint8_t* smem, int* bcast) {
  constexpr int K = KB * kGroup;
  constexpr int kRowsPerWave = RT * 16;
  constexpr int kRowsPerGroup = kGemmWaves * kRowsPerWave;
  constexpr int kStride = K + 16;  // 16-byte pad: the 16 rows of a ds_read_b128 hit distinct banks
  constexpr int kChunks = K / 256;
  constexpr int kFirstHalf = KB > 1 ? KB / 2 : KB;
  uint8_t* b_tile = smem;
  float* b_scales = reinterpret_cast<float*>(smem + 16 * kStride);
  int* b_target = reinterpret_cast<int*>(b_scales + 16 * KB);
  int* finish = b_target + 16;  // [16 * TILES]

  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
  const int row16 = lane & 15;
  const int group = lane >> 4;
  const int n_rows = kFC1 ? 2 * a.intermediate : a.hidden;
  const int first_tile = tile_group * TILES;
  int4* state = a.expert_state + expert;

  // Weight tiles of this workgroup: TILES consecutive row tiles of the
  // expert, each held in registers in turn.
  const uint8_t* wexp = (kFC1 ? a.w13 : a.w2) + static_cast<size_t>(expert) * n_rows * K;
  const float* wsexp = (kFC1 ? a.s13 : a.s2) + static_cast<size_t>(expert) * (n_rows / kGroup) * KB;
  int32x8 a_frag[RT][KB];
  float w_scale[RT][KB];
  auto load_weights = [&](int tile, int kb0, int kb1) {
    const int n0 = tile * kRowsPerGroup + wave * kRowsPerWave;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
        if (kb >= kb0 && kb < kb1)
          a_frag[rt][kb] = load_packed_fragment(wexp + static_cast<size_t>(n0 + rt * 16) * K, kb, lane);
  };
  auto load_scales = [&](int tile) {
    const int n0 = tile * kRowsPerGroup + wave * kRowsPerWave;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) w_scale[rt][kb] = wsexp[((n0 + rt * 16) / kGroup) * KB + kb];
  };

  // Staging of one route tile: 16 threads per route column.  The loads are
  // unconditional (dead columns read past the buffer and get zeros): no
  // branch, so no register copy of a loaded value forces an early wait.
  const int stage_col = threadIdx.x >> 4;
  const int stage_part = threadIdx.x & 15;
  const uint32_t a_rows = static_cast<uint32_t>(kFC1 ? a.num_slots : a.max_rows);
  const CoherentBuffer act_rows(kFC1 ? static_cast<const void*>(a.q) : a.act, a_rows * K);
  const CoherentBuffer act_scales(kFC1 ? static_cast<const void*>(a.x_scales) : a.act_scales,
                                  a_rows * KB * 4);
  const CoherentBuffer sorted(a.sorted_ids, static_cast<uint32_t>(a.max_rows) * 4);
  int routes = 0;
  int first = 0;
  int4 b_stage[kChunks];
  float b_stage_scale = 0.0f;
  int stage_pair = 0;
  auto fetch_ids = [&](int m0) {  // pair of this thread's route column
    const int r = m0 + stage_col;
    stage_pair = static_cast<int>(sorted.load4(r < routes ? static_cast<uint32_t>(first + r) * 4 : kNoRow));
  };
  auto fetch_rows = [&](int m0) {  // activation row + scale of that column
    const int r = m0 + stage_col;
    const bool live = r < routes;
    const int a_row = kFC1 ? stage_pair / a.top_k : first + r;
    const uint32_t row_offset = live ? static_cast<uint32_t>(a_row) * K : kNoRow;
#pragma unroll
    for (int j = 0; j < kChunks; ++j) b_stage[j] = act_rows.load16(row_offset + j * 256 + stage_part * 16);
    b_stage_scale = __uint_as_float(act_scales.load4(
        live && stage_part < KB ? static_cast<uint32_t>(a_row * KB + stage_part) * 4 : kNoRow));
  };
  auto store_tile = [&](int m0) {
    const bool live = m0 + stage_col < routes;
#pragma unroll
    for (int j = 0; j < kChunks; ++j)
      *reinterpret_cast<int4*>(b_tile + stage_col * kStride + j * 256 + stage_part * 16) = b_stage[j];
    if (stage_part < KB) b_scales[stage_col * KB + stage_part] = b_stage_scale;
    if (stage_part == 0) b_target[stage_col] = live ? (kFC1 ? first + m0 + stage_col : stage_pair) : -1;
  };

  // Expert state: {count + 1, start} (0 = routing not done), act_done.
  auto ready = [&](uint64_t word, uint32_t act_done) {
    const int count1 = static_cast<int>(static_cast<uint32_t>(word));
    return count1 > 0 && (kFC1 || count1 == 1 || act_done != 0u);
  };
  // One read of the state decides the path for the whole workgroup (the
  // state may change between two reads).
  bool fast = false;
  if (blockIdx.x >= a.num_slots + kFirstWave) {
    if (threadIdx.x == 0) {
      const uint64_t word = collect_u64(state);
      const uint32_t act_done = kFC1 ? 0u : collect_u32(&state->z);
      bcast[2] = ready(word, act_done) ? static_cast<int>(static_cast<uint32_t>(word)) - 1 : -1;
      bcast[3] = static_cast<int>(word >> 32);
    }
    __syncthreads();
    const int count = __builtin_amdgcn_readfirstlane(bcast[2]);
    if (count >= 0) {
      fast = true;
      routes = count;
      first = __builtin_amdgcn_readfirstlane(bcast[3]);
    }
  }
  if (fast) {
    if (routes == 0) return;
    load_scales(first_tile);
    if constexpr (kFC1) {
      fetch_ids(0);  // before any weight: its wait does not include them
      load_weights(first_tile, 0, kFirstHalf);
      __builtin_amdgcn_sched_barrier(0);
      fetch_rows(0);
      __builtin_amdgcn_sched_barrier(0);
      load_weights(first_tile, kFirstHalf, KB);
    } else {
      fetch_ids(0);
      fetch_rows(0);
      __builtin_amdgcn_sched_barrier(0);
      load_weights(first_tile, 0, KB);
    }
    store_tile(0);
  } else {
    load_weights(first_tile, 0, KB);
    load_scales(first_tile);
    if (threadIdx.x == 0) {
      int count = 0, start = 0;
      for (int spins = 0;; ++spins) {
        const uint64_t word = collect_u64(state);
        if (ready(word, kFC1 ? 0u : collect_u32(&state->z))) {
          count = static_cast<int>(static_cast<uint32_t>(word)) - 1;
          start = static_cast<int>(word >> 32);
          break;
        }
        if (spins == kMaxSpins) {
          publish_u32(a.error, 1u);
          break;
        }
        __builtin_amdgcn_s_sleep(2);
      }
      bcast[0] = count;
      bcast[1] = start;
    }
    __syncthreads();
    routes = __builtin_amdgcn_readfirstlane(bcast[0]);
    first = __builtin_amdgcn_readfirstlane(bcast[1]);
    if (routes == 0) return;
    fetch_ids(0);
    fetch_rows(0);
    store_tile(0);
  }
  const bool exact = routes <= a.exact_routes;

  // One weight tile against the route tile in LDS.
  auto mma = [&](floatx4 (&acc)[RT]) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) acc[rt] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    const uint8_t* brow = b_tile + row16 * kStride;
    if (exact) {
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        bf16x8 b_wide[4];
        widen_fp8(load_fragment(brow, kb, group), b_wide);
        const float b_scale = b_scales[row16 * KB + kb];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          const floatx4 partial = mfma_block_bf16(a_frag[rt][kb], b_wide);
          acc[rt] += partial * (w_scale[rt][kb] * b_scale);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        const int32x8 b_frag = load_fragment(brow, kb, group);
        const float b_scale = b_scales[row16 * KB + kb];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          const floatx4 partial = mfma_fp8(a_frag[rt][kb], b_frag);
          acc[rt] += partial * (w_scale[rt][kb] * b_scale);
        }
      }
    }
  };
  auto epilogue = [&](const floatx4 (&acc)[RT], int tile) {
    const int target = b_target[row16];
    if (target < 0) return;
    const int n0 = tile * kRowsPerGroup + wave * kRowsPerWave;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int n = n0 + rt * 16 + group * 4;  // rows n..n+3 of this column
      if constexpr (kFC1) {
        const uint32_t lo = f32_to_bf16(acc[rt][0]) | (static_cast<uint32_t>(f32_to_bf16(acc[rt][1])) << 16);
        const uint32_t hi = f32_to_bf16(acc[rt][2]) | (static_cast<uint32_t>(f32_to_bf16(acc[rt][3])) << 16);
        publish_u64(a.gate_up + static_cast<size_t>(target) * n_rows + n, (static_cast<uint64_t>(hi) << 32) | lo);
      } else {
        float* dst = a.down + static_cast<size_t>(target) * n_rows + n;
        publish_u64(dst, (static_cast<uint64_t>(__float_as_uint(acc[rt][1])) << 32) | __float_as_uint(acc[rt][0]));
        publish_u64(dst + 2, (static_cast<uint64_t>(__float_as_uint(acc[rt][3])) << 32) | __float_as_uint(acc[rt][2]));
      }
    }
  };
  // FC2: for the route tile in LDS and column tiles [tile0, tile0 + count),
  // the weighted combine of each token whose last contribution this was
  // (rank order, one rounding to bf16).
  auto combine_handoff = [&](int tile0, int count) {
    wait_stores();
    __syncthreads();
    if (threadIdx.x < 16 * count) {
      const int t = b_target[threadIdx.x & 15];
      int done = -1;
      if (t >= 0) {
        const int token = t / a.top_k;
        const int index = token * a.fc2_tiles + tile0 + (threadIdx.x >> 4);
        if (take_ticket(&a.combine_tickets[index]) == a.top_k - 1) done = token;
      }
      finish[threadIdx.x] = done;
    }
    __syncthreads();
    const int seg = threadIdx.x >> 4;
    const int part = threadIdx.x & 15;
    for (int f = seg; f < 16 * count; f += 16) {
      const int token = finish[f];
      if (token < 0) continue;  // whole 16-thread segment
      const int tile = tile0 + (f >> 4);
      const int tile_n0 = tile * kRowsPerGroup;
      for (int column = tile_n0 + part * 4; column < tile_n0 + kRowsPerGroup; column += 64) {
        float4 acc4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        for (int r = 0; r < a.top_k; ++r) {
          const int index = token * a.top_k + r;
          const float w = collect_route_weight(a.weights, a.weights_f32, index);
          const float* src = a.down + static_cast<size_t>(index) * n_rows + column;
          const uint64_t lo = collect_u64(src), hi = collect_u64(src + 2);
          acc4.x = fmaf(w, __uint_as_float(static_cast<uint32_t>(lo)), acc4.x);
          acc4.y = fmaf(w, __uint_as_float(static_cast<uint32_t>(lo >> 32)), acc4.y);
          acc4.z = fmaf(w, __uint_as_float(static_cast<uint32_t>(hi)), acc4.z);
          acc4.w = fmaf(w, __uint_as_float(static_cast<uint32_t>(hi >> 32)), acc4.w);
        }
        *reinterpret_cast<uint2*>(a.out + static_cast<size_t>(token) * n_rows + column) = pack_bf16x4(acc4);
      }
      if (part == 0) reset_ticket(&a.combine_tickets[token * a.fc2_tiles + tile]);
    }
  };

  if (routes <= 16) {
    // One route tile: the weight tiles follow each other through the same
    // registers; tile tt + 1 streams in while tile tt's outputs are stored.
    __syncthreads();
#pragma unroll
    for (int tt = 0; tt < TILES; ++tt) {
      floatx4 acc[RT];
      mma(acc);
      if (tt + 1 < TILES) {
        // Not above the MFMAs: the next tile reuses this tile's registers.
        __builtin_amdgcn_sched_barrier(0);
        load_weights(first_tile + tt + 1, 0, KB);
        load_scales(first_tile + tt + 1);
      }
      epilogue(acc, first_tile + tt);
    }
    if constexpr (!kFC1) combine_handoff(first_tile, TILES);
  } else {
    // Several route tiles: each weight tile walks them, restaging each.
#pragma unroll
    for (int tt = 0; tt < TILES; ++tt) {
      if (tt > 0) {
        __builtin_amdgcn_sched_barrier(0);
        load_weights(first_tile + tt, 0, KB);
        load_scales(first_tile + tt);
      }
      for (int m0 = 0; m0 < routes; m0 += 16) {
        if (tt > 0 || m0 > 0) {
          __syncthreads();  // previous route tile fully consumed
          fetch_ids(m0);
          fetch_rows(m0);
          store_tile(m0);
        }
        __syncthreads();
        floatx4 acc[RT];
        mma(acc);
        epilogue(acc, first_tile + tt);
        if constexpr (!kFC1) combine_handoff(first_tile + tt, 1);
      }
    }
  }

  if constexpr (kFC1) {
    // The expert's last FC1 workgroup computes its SwiGLU requant.
    wait_stores();
    __syncthreads();
    if (threadIdx.x == 0) bcast[2] = take_ticket(&state->w) == a.fc1_tiles / TILES - 1 ? 1 : 0;
    __syncthreads();
    if (bcast[2]) act_finish<KB2>(a, state, routes, first);
  }
}

// The last workgroup of the grid: waits until every other workgroup has
// left, then clears the per-expert state for the next launch.
__device__ void janitor(const StepArgs& a) {
  if (threadIdx.x == 0) {
    const uint32_t others = gridDim.x - 1;
    for (int spins = 0; collect_u32(a.exit_count) != others; ++spins) {
      if (spins == kMaxSpins) {
        publish_u32(a.error, 1u);
        break;
      }
      __builtin_amdgcn_s_sleep(8);
    }
  }
  __syncthreads();
  for (int e = threadIdx.x; e < a.num_experts; e += kStepThreads) {
    publish_u64(&a.expert_state[e].x, 0ull);
    publish_u64(&a.expert_state[e].z, 0ull);
  }
  if (threadIdx.x == 0) reset_ticket(a.exit_count);
}

constexpr int kMaxTiles = 4;  // weight tiles per expert workgroup
constexpr int gemm_smem_bytes(int kb) { return 16 * (kb * kGroup + 16) + 16 * kb * 4 + 16 * 4 + 16 * kMaxTiles * 4; }
constexpr int max3(int x, int y, int z) { return x > y ? (x > z ? x : z) : (y > z ? y : z); }

template <int NPL, int KB1, int KB2, int TILES1, int TILES2>
__global__ __launch_bounds__(kStepThreads) __attribute__((amdgpu_waves_per_eu(2))) void moe_step_kernel(
    StepArgs a) {
  constexpr int kSmem = max3(gemm_smem_bytes(KB1), gemm_smem_bytes(KB2),
                             sort_shared_ints(kStepThreads, kWave * NPL) * 4);
  __shared__ __attribute__((aligned(16))) uint8_t smem[kSmem];
  __shared__ int bcast[4];
  const int b = blockIdx.x;
  if (b == static_cast<int>(gridDim.x) - 1) {
    janitor(a);
    return;
  }
  const int fc1_groups = a.fc1_tiles / TILES1;
  const int fc2_groups = a.fc2_tiles / TILES2;
  const int fc1_end = a.num_slots + a.num_experts * fc1_groups;
  if (b < a.num_slots) {
    front_task<NPL>(a, b, reinterpret_cast<int*>(smem), bcast);
  } else if (b < fc1_end) {
    const int t = b - a.num_slots;
    expert_task<KB1, rt_for(KB1), true, KB2, TILES1>(a, t / fc1_groups, t % fc1_groups, smem, bcast);
  } else {
    const int t = b - fc1_end;
    expert_task<KB2, rt_for(KB2), false, KB2, TILES2>(a, t / fc2_groups, t % fc2_groups, smem, bcast);
  }
  // Leave: every access of this workgroup to the expert state has completed
  // (loads consumed, tickets returned, act_done stores waited for), so a
  // fire-and-forget count suffices for the janitor.
  __syncthreads();
  if (threadIdx.x == 0) __hip_atomic_fetch_add(a.exit_count, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

bool aligned(const void* p, uintptr_t bytes) { return (reinterpret_cast<uintptr_t>(p) % bytes) == 0; }

// Compiled (H / 128, I / 128) pairs.
bool supported_shape(int hidden, int intermediate) {
  const int kb1 = hidden / kGroup, kb2 = intermediate / kGroup;
  return hidden % kGroup == 0 && intermediate % kGroup == 0 &&
         ((kb1 == 8 && kb2 == 2) || (kb1 == 16 && kb2 == 6) || (kb1 == 16 && kb2 == 4) ||
          (kb1 == 8 && kb2 == 4));
}

int fc2_tiles_of(int hidden, int intermediate) { return hidden / tile_rows_for(intermediate / kGroup); }

}  // namespace
}  // namespace d3

using namespace d3;

extern "C" int32_t d3_moe_step_sync_ints(int32_t num_slots, int32_t num_experts, int32_t hidden,
                                         int32_t intermediate) {
  if (num_slots < 1 || num_experts < 1 || !supported_shape(hidden, intermediate)) return -1;
  return kSyncHeader + 4 * num_experts + num_slots * fc2_tiles_of(hidden, intermediate);
}

extern "C" int d3_moe_decode_step(const uint8_t* occupancy, int32_t num_slots,
                                  int32_t* active_slots, int32_t* count, const uint16_t* x,
                                  int64_t x_row_stride, const uint16_t* logits,
                                  int64_t logits_row_stride, int32_t hidden, int32_t num_experts,
                                  int32_t intermediate, int32_t top_k, const uint8_t* w13,
                                  const float* s13, const uint8_t* w2, const float* s2,
                                  int32_t exact_routes, int32_t* ids, void* weights,
                                  int32_t weights_dtype, uint8_t* q, float* x_scales,
                                  int32_t* sorted_ids, int32_t max_rows, uint16_t* gate_up,
                                  uint8_t* act, float* act_scales, float* down, uint16_t* out,
                                  int32_t* sync, void* stream) {
  D3_REQUIRE(occupancy && active_slots && count && x && logits && w13 && s13 && w2 && s2 && ids &&
                 weights && q && x_scales && sorted_ids && gate_up && act && act_scales && down &&
                 out && sync,
             "moe_decode_step: null pointer");
  D3_REQUIRE(weights_dtype == D3_DTYPE_BF16 || weights_dtype == D3_DTYPE_F32,
             "moe_decode_step: weights must be bf16 or f32");
  D3_REQUIRE(num_slots >= 1 && num_slots <= 256, "moe_decode_step: num_slots %d not in [1, 256]",
             num_slots);
  D3_SUPPORTED(supported_shape(hidden, intermediate),
               "moe_decode_step: (hidden %d, intermediate %d) not in the compiled set", hidden,
               intermediate);
  D3_SUPPORTED(num_experts >= 1 && num_experts <= kStepThreads,
               "moe_decode_step: num_experts %d not in [1, %d]", num_experts, kStepThreads);
  D3_REQUIRE(top_k >= 1 && top_k <= 16 && top_k <= num_experts, "moe_decode_step: bad top_k %d",
             top_k);
  D3_REQUIRE(x_row_stride >= hidden && x_row_stride % 8 == 0 && logits_row_stride >= num_experts,
             "moe_decode_step: bad row strides");
  D3_REQUIRE(aligned(x, 16) && aligned(q, 16) && aligned(gate_up, 16) && aligned(act, 16) &&
                 aligned(down, 16) && aligned(out, 8) && aligned(sync, 16) && aligned(w13, 16) &&
                 aligned(w2, 16),
             "moe_decode_step: alignment");
  const int32_t need = d3_max_sorted_rows(num_slots * top_k, num_experts, kSortTile);
  D3_REQUIRE(max_rows >= need, "moe_decode_step: max_rows %d < required %d", max_rows, need);
  StepArgs args{};
  args.occupancy = occupancy;
  args.num_slots = num_slots;
  args.active = active_slots;
  args.count = count;
  args.x = x;
  args.x_stride = x_row_stride;
  args.logits = logits;
  args.logits_stride = logits_row_stride;
  args.hidden = hidden;
  args.num_experts = num_experts;
  args.intermediate = intermediate;
  args.top_k = top_k;
  args.w13 = w13;
  args.s13 = s13;
  args.w2 = w2;
  args.s2 = s2;
  args.exact_routes = exact_routes;
  args.ids = ids;
  args.weights = weights;
  args.weights_f32 = weights_dtype == D3_DTYPE_F32 ? 1 : 0;
  args.q = q;
  args.x_scales = x_scales;
  args.sorted_ids = sorted_ids;
  args.max_rows = max_rows;
  args.gate_up = gate_up;
  args.act = act;
  args.act_scales = act_scales;
  args.down = down;
  args.out = out;
  args.error = sync;
  args.front_ticket = sync + 1;
  args.exit_count = sync + 2;
  args.expert_state = reinterpret_cast<int4*>(sync + kSyncHeader);
  args.combine_tickets = sync + kSyncHeader + 4 * num_experts;
  args.fc1_tiles = 2 * intermediate / tile_rows_for(hidden / kGroup);
  args.fc2_tiles = fc2_tiles_of(hidden, intermediate);
  // Weight tiles per expert workgroup (each divides the expert's tile count).
  constexpr int kTiles1 = 2, kTiles2 = 2;
  const dim3 grid(num_slots + num_experts * (args.fc1_tiles / kTiles1 + args.fc2_tiles / kTiles2) + 1);  // + janitor
  const dim3 block(kStepThreads);
  hipStream_t s = as_stream(stream);
  const int kb1 = hidden / kGroup, kb2 = intermediate / kGroup;
#define D3_STEP_LAUNCH(NPL)                                                                     \
  if (kb1 == 8 && kb2 == 2)                                                                     \
    hipLaunchKernelGGL((moe_step_kernel<NPL, 8, 2, kTiles1, kTiles2>), grid, block, 0, s, args);                  \
  else if (kb1 == 8 && kb2 == 4)                                                                \
    hipLaunchKernelGGL((moe_step_kernel<NPL, 8, 4, kTiles1, kTiles2>), grid, block, 0, s, args);                  \
  else if (kb1 == 16 && kb2 == 4)                                                               \
    hipLaunchKernelGGL((moe_step_kernel<NPL, 16, 4, kTiles1, kTiles2>), grid, block, 0, s, args);                 \
  else                                                                                          \
    hipLaunchKernelGGL((moe_step_kernel<NPL, 16, 6, kTiles1, kTiles2>), grid, block, 0, s, args);
  if (num_experts <= 64) {
    D3_STEP_LAUNCH(1)
  } else if (num_experts <= 128) {
    D3_STEP_LAUNCH(2)
  } else {
    D3_STEP_LAUNCH(4)
  }
#undef D3_STEP_LAUNCH
  D3_LAUNCHED("moe_decode_step");
}
