// Tiled grouped FP8 expert GEMM for real contractions (packed prefill and
// mixed batches): work items of up to 128 sorted routes against 256 weight
// rows, the contraction streamed in 128-byte K blocks.
//
// Design (gfx950, wave64, MFMA 16x16x128 OCP-FP8, 4 waves per workgroup,
// two workgroups per CU):
//   * A workgroup owns (work item, weight row tile).  Each wave owns four
//     16-row weight tiles (FC1: two gate tiles and the matching two up
//     tiles) and all eight 16-route tiles of the item: 32 MFMAs per K block,
//     128 fp32 accumulators per lane; each B fragment read from LDS feeds
//     four MFMAs.
//   * Weights go straight from memory into MFMA fragments one K block ahead
//     of the MFMAs (fragment-major layout: two 1 KiB contiguous loads per
//     tile and K block; checkpoint layout: 16 rows x 64 bytes per load).
//     Activation rows (gathered by route: FC1 reads token sorted_ids /
//     top_k, FC2 the sorted row) are staged one K block ahead into a
//     two-slot LDS ring (128 routes x 144-byte rows; the 16-byte pad keeps
//     the 16 rows of each ds_read_b128 on distinct banks); their loads are
//     issued before the weights', so waiting for them never waits for the
//     weights.  The next block's loads are issued in units spread over the
//     current block's route tiles (one activation copy or one weight tile
//     per route tile): issued in one block at its top they held the wave's
//     MFMAs back while the memory pipeline drained (3 % slower per GEMM).
//     One barrier per K block.
//   * Measured per workgroup (per-workgroup timestamps, config-4 FC1): the
//     prologue (item, route ids, scales, first blocks) and the epilogue
//     cost a third of a workgroup's time; two resident workgroups per CU
//     hide them behind each other's K loop, which measured faster than
//     8-wave workgroups with deeper prefetch (one per CU).  The prologue's
//     loads are branch-free so they form one round trip per dependency.
//   * Scales as in the other expert kernels: every MFMA is exactly one K
//     block, rescaled with acc += mfma(w, a) * (w_scale * a_scale), K blocks
//     in ascending order, so the sums are bit-identical to d3_expert_gemm's
//     FP8 path.
//   * FC1 (mode 0): a workgroup covers 128 gate rows and the 128 matching up
//     rows, so each lane holds gate and up of the same columns: the epilogue
//     rounds both to bf16 (the reference's FC1 output), computes SwiGLU
//     (swiglu_values), reduces the per-(route, 128-column) amax across lanes
//     and waves and writes the e4m3 codes and scale, the bytes
//     d3_silu_mul_quant would write.  FC2 (mode 1) stores fp32 rows by pair (the unpermute),
//     each route tile passed through LDS so that every store instruction
//     writes one route's whole 1 KiB run (against sixteen 64-byte pieces
//     straight from the MFMA layout: the prefill FC2 4.5 us faster).
//   * Workgroups are grouped so that two consecutive items' tiles run on one
//     XCD together: an item's tiles share its activation rows, and an
//     expert's consecutive items its weights, in that XCD's L2.
#include "common.h"
#include "expert_tile.h"
#include "status.h"

namespace d3 {
namespace {

constexpr int kGgWaves = 4;
constexpr int kGgThreads = kGgWaves * kWave;
constexpr int kGgRoutes = 128;                     // routes per work item (MFMA N side)
constexpr int kGgPairRoutes = 64;                  // routes per work item of by-pair launches
constexpr int kGgWaveTiles = 4;                    // 16-row weight tiles per wave
constexpr int kGgRows = kGgWaves * kGgWaveTiles * 16;  // 256 weight rows per workgroup
constexpr int kGgStride = kGroup + 16;             // LDS bytes per staged route row
constexpr int kGgXcds = 8;
constexpr int kStreamOutRoutes = 16384;  // FC2 launches up to this many item routes stream their rows
// Routes found by the workgroups themselves (by-pair launches): at most this
// many (row, rank) pairs, read in chunks of one id per thread.
constexpr int kGgMaxPairChunks = 32;
constexpr int kGgMaxPairs = kGgMaxPairChunks * kGgThreads;  // 8192
static_assert(kGgMaxPairChunks * kGgWaves == 2 * kWave, "one wave scans the (chunk, wave) counts, two per lane");

// A dense shared expert folded into the routed launch: items after the
// routed ones cover its rows [128 j, 128 j + 128) with identity routes and
// its own weights.  FC1 reads q row r and writes act row pos + r; FC2 reads
// act row pos + r and writes fp32 row pair + r.
struct SharedItems {
  const uint8_t* w;  // nullptr: none
  const float* ws;
  int rows;
  int pos;
  int pair;
};

// kByPair (FC1 of small batches): no sorted route list.  A work item is
// part j (routes [64 j, 64 j + 64) in pair order) of an expert; the
// workgroup finds those routes itself in `sorted_ids`, which
// then holds the routed expert of every (row, rank) pair, the live row
// count being *num_items.  What they found is written out as a sorted
// route list of 128-route items, two parts each - item i = (expert, 128 i,
// routes), its pairs at list_ids[128 i ..] in ascending order - and FC1
// writes act rows at those positions, so the sorted FC2 launch reads them
// as it reads a route sort's.
// kStreamOut (FC2): the fp32 rows go out with non-temporal stores.
template <int KB, int MODE, bool kPacked, bool kByPair, bool kStreamOut = false>
__global__ __launch_bounds__(kGgThreads) __attribute__((amdgpu_waves_per_eu(2))) void grouped_gemm_kernel(
    const uint8_t* __restrict__ w, const float* __restrict__ ws, int n_rows, int out_cols,
    const uint8_t* __restrict__ act, uint32_t act_bytes, const float* __restrict__ act_scales,
    const int32_t* __restrict__ sorted_ids, int top_k, const int4* __restrict__ items,
    const int32_t* __restrict__ num_items, int max_items, SharedItems shared, int n_tiles, int chunk,
    int parts, int capacity, int32_t* __restrict__ list_ids, int4* __restrict__ list_items,
    int32_t* __restrict__ list_count, uint8_t* __restrict__ out_codes, float* __restrict__ out_scales,
    float* __restrict__ out_f32) {
  static_assert(!kByPair || MODE == 0, "the route lists come from FC1");
  constexpr int K = KB * kGroup;
  // Routes per work item: by-pair launches take 64 (twice the workgroups,
  // each with half the epilogue, for batches that leave most CUs idle).
  constexpr int kR = kByPair ? kGgPairRoutes : kGgRoutes;
  constexpr int kRT = kR / 16;                              // 16-route tiles per wave
  constexpr int kStage = kR * kGgStride;
  constexpr int kStaged = kR * kGroup / (16 * kGgThreads);  // 16-byte copies per thread and K block
  __shared__ __attribute__((aligned(16))) uint8_t stage[2][kStage];
  __shared__ float a_scale[KB][kR];
  __shared__ int target[kR];  // FC1: sorted position, FC2: pair; -1 = no route
  __shared__ float amax_part[MODE == 0 ? kGgWaves : 1][kR];
  __shared__ int route_pair[kByPair ? kR : 1];
  __shared__ uint64_t chunk_masks[kByPair ? kGgMaxPairChunks * kGgWaves : 1];
  __shared__ int chunk_base[kByPair ? kGgMaxPairChunks * kGgWaves + 1 : 1];

  // XCD-aware order: workgroup b runs on XCD b % 8; logical index L gives
  // each XCD runs of `chunk` = 2 n_tiles consecutive workgroups: the tiles
  // of two consecutive items, interleaved so that the two workgroups that
  // read one weight tile are dispatched back to back.
  const int b = blockIdx.x;
  const int xcd = b % kGgXcds, j = b / kGgXcds;
  const int logical = ((j / chunk) * kGgXcds + xcd) * chunk + j % chunk;
  const int within = logical % chunk;
  const int item_index = (logical / chunk) * 2 + (within & 1);
  const int tile = within >> 1;
  const bool dense = item_index >= max_items;  // a shared-expert item (uniform)
  int expert = 0, first = 0, routes = 0;
  int pj = 0, slot = 0;  // by-pair: the expert's part, and its expert-major index
  if constexpr (kByPair) {
    if (item_index >= max_items) return;
    // Part-pair-major order (parts 2 p and 2 p + 1 of every expert, then
    // the next p): the launch's first workgroups take the parts that hold
    // routes, so they start on CUs of their own.
    const int experts_n = max_items / parts;
    const int pp = item_index / (2 * experts_n), rem = item_index - pp * 2 * experts_n;
    expert = rem >> 1;
    pj = 2 * pp + (rem & 1);
    slot = expert * parts + pj;
  } else if (!dense) {
    // The item is read together with the item count (item_index <
    // max_items: in bounds) and both decide the one early exit, so both
    // loads are in flight at once: one memory round trip, not two.
    const int4 item = items[item_index];
    const int count = *num_items;
    expert = item.x;
    first = item.y;
    routes = item_index < count ? min(item.z, kR) : 0;
    if (routes <= 0) return;  // a padding item (uniform)
  } else {
    first = (item_index - max_items) * kR;
    if (first >= shared.rows) return;
    routes = min(kR, shared.rows - first);
  }

  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int row16 = lane & 15;
  const int group = lane >> 4;

  // Weight rows of this wave's tile t (16 rows each).
  const int n0 = tile * (MODE == 0 ? kGroup : kGgRows);
  auto tile_row = [&](int t) {
    if constexpr (MODE == 0)  // t = 0, 1: gate rows; t = 2, 3: the matching up rows
      return (t < 2 ? 0 : out_cols) + n0 + 32 * wave + 16 * (t & 1);
    else
      return n0 + 64 * wave + 16 * t;
  };
  const uint8_t* wexp = dense ? shared.w : w + static_cast<size_t>(expert) * n_rows * K;
  const float* wsexp = dense ? shared.ws : ws + static_cast<size_t>(expert) * (n_rows / kGroup) * KB;

  // Weight fragments through a buffer view of the expert: the lane offset
  // is one VGPR, the tile / K block offset a wave-uniform scalar.  Loads are
  // not marked non-temporal: an expert's other items read the same weights
  // from L2 shortly after (measured: 18 % less L2 fetch than with nt).
  constexpr int kNonTemporal = 0;
  const __amdgpu_buffer_rsrc_t wrsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(wexp), 0, static_cast<uint32_t>(n_rows) * K, 0x00020000);
  const uint32_t w_lane = kPacked ? lane * 16 : row16 * K + group * 16;
  int32x8 wf[2][kGgWaveTiles];
  auto load_weights = [&](int kb) {
#pragma unroll
    for (int t = 0; t < kGgWaveTiles; ++t) {
      const uint32_t base = static_cast<uint32_t>(tile_row(t)) * K;
      int32x4 lo, hi;
      if constexpr (kPacked) {
        lo = __builtin_amdgcn_raw_buffer_load_b128(wrsrc, w_lane, base + kb * 2048, kNonTemporal);
        hi = __builtin_amdgcn_raw_buffer_load_b128(wrsrc, w_lane, base + kb * 2048 + 1024, kNonTemporal);
      } else {
        lo = __builtin_amdgcn_raw_buffer_load_b128(wrsrc, w_lane, base + kb * kGroup, 0);
        hi = __builtin_amdgcn_raw_buffer_load_b128(wrsrc, w_lane, base + kb * kGroup + 64, 0);
      }
      int32x8 v;
      v[0] = lo[0]; v[1] = lo[1]; v[2] = lo[2]; v[3] = lo[3];
      v[4] = hi[0]; v[5] = hi[1]; v[6] = hi[2]; v[7] = hi[3];
      wf[kb & 1][t] = v;
    }
  };
  if constexpr (!kByPair) load_weights(0);  // depends on the item only

  if constexpr (kByPair) {
    // The expert's routes in pair order: pair p = 256 j + thread.  Each
    // wave's ballot of chunk j goes to LDS; one wave turns their counts into
    // exclusive bases (in pair order: chunk, then wave); each thread then
    // ranks only its own matches (a few of its 32 chunks).
    const int part_first = pj * kR;
    const int live_rows = min(*num_items, capacity);
    const int pairs = live_rows * top_k;
    const BufferView id_view(sorted_ids, static_cast<uint32_t>(capacity * top_k) * 4);
    const int my_wave = static_cast<int>(threadIdx.x) / kWave;
    uint32_t mine = 0;  // bit j: this thread's pair of chunk j routes to the expert
    {
      int idv[kGgMaxPairChunks];
#pragma unroll
      for (int j = 0; j < kGgMaxPairChunks; ++j) {
        const int p = j * kGgThreads + static_cast<int>(threadIdx.x);
        idv[j] = p < pairs ? static_cast<int>(id_view.load4(static_cast<uint32_t>(p) * 4)) : -1;
      }
      // The first weight block after the ids: memory returns are counted in
      // issue order, so the wait for the ids does not cover the weights.
      load_weights(0);
#pragma unroll
      for (int j = 0; j < kGgMaxPairChunks; ++j) {
        mine |= (idv[j] == expert ? 1u : 0u) << j;
        const uint64_t hits = __ballot(idv[j] == expert);
        if (lane_id() == 0) chunk_masks[j * kGgWaves + my_wave] = hits;
      }
    }
    __syncthreads();
    if (my_wave == 0) {
      // exclusive scan of the 128 (chunk, wave) counts: two per lane
      constexpr int kCells = kGgMaxPairChunks * kGgWaves;
      const int c0 = __popcll(chunk_masks[2 * lane_id()]);
      const int c1 = __popcll(chunk_masks[2 * lane_id() + 1]);
      int incl = c0 + c1;
#pragma unroll
      for (int offset = 1; offset < kWave; offset <<= 1) {
        const int up = __shfl_up(incl, offset);
        if (lane_id() >= offset) incl += up;
      }
      const int excl = incl - c0 - c1;
      chunk_base[2 * lane_id()] = excl;
      chunk_base[2 * lane_id() + 1] = excl + c0;
      if (lane_id() == kWave - 1) chunk_base[kCells] = incl;
    }
    __syncthreads();
    for (uint32_t m = mine; m != 0; m &= m - 1) {
      const int j = __builtin_ctz(m);
      const int cell = j * kGgWaves + my_wave;
      const int r = chunk_base[cell] + __popcll(chunk_masks[cell] & lanemask_lt()) - part_first;
      if (r >= 0 && r < kR) route_pair[r] = j * kGgThreads + static_cast<int>(threadIdx.x);
    }
    const int base = chunk_base[kGgMaxPairChunks * kGgWaves];
    routes = __builtin_amdgcn_readfirstlane(min(max(base - part_first, 0), kR));
    __syncthreads();
    if (tile == 0) {  // the route list (empty parts included)
      for (int r = static_cast<int>(threadIdx.x); r < routes; r += kGgThreads)
        list_ids[slot * kR + r] = route_pair[r];
      // list item = kGgRoutes / kR consecutive parts, written by the first
      constexpr int kPer = kGgRoutes / kR;
      if (threadIdx.x == 0 && pj % kPer == 0) {
        const int list_item = slot / kPer;
        const int listed = min(max(base - part_first, 0), kGgRoutes);
        list_items[list_item] = make_int4(expert, list_item * kGgRoutes, listed, 0);
        if (item_index == 0) *list_count = max_items / kPer;
      }
    }
    if (routes == 0) return;  // uniform: this part of the expert is empty
  }

  // Route rows of the item, loaded branch-free (a dead route reads the
  // item's first id and is masked afterwards): one round trip.  Shared-expert
  // items map row r of the item to token first + r.
  auto route_row = [&](int r, int id) {
    if (dense) return MODE == 0 ? first + r : shared.pos + first + r;
    return MODE == 0 ? id / top_k : first + r;
  };
  const int part = tid & 7;
  const int r0 = tid >> 3;
  int ids[kStaged];
#pragma unroll
  for (int i = 0; i < kStaged; ++i) {
    const int r = r0 + (kGgThreads / 8) * i;
    if constexpr (kByPair)
      ids[i] = route_pair[r < routes ? r : 0];
    else
      ids[i] = dense ? 0 : sorted_ids[first + (r < routes ? r : 0)];
  }
  const int rs = tid % kR;       // route of this thread's scales / target
  const int k0 = tid / kR;       // first K block of its scales
  const int id_s = kByPair ? route_pair[rs < routes ? rs : 0]
                           : (dense ? 0 : sorted_ids[first + (rs < routes ? rs : 0)]);

  // Staging: thread t copies 16 bytes (chunk t % 8 of the K block) of routes
  // t / 8 + 32 i.  Dead routes read past the buffer (zeros).
  const BufferView view(act, act_bytes);
  uint32_t src[kStaged];
#pragma unroll
  for (int i = 0; i < kStaged; ++i) {
    const int r = r0 + (kGgThreads / 8) * i;
    src[i] = r < routes ? static_cast<uint32_t>(route_row(r, ids[i])) * K + part * 16 : kNoRow;
  }
  int4 staged[kStaged];
  auto stage_load = [&](int kb) {
#pragma unroll
    for (int i = 0; i < kStaged; ++i) staged[i] = view.load16(src[i] + kb * kGroup);
  };
  auto stage_store = [&](int kb) {
#pragma unroll
    for (int i = 0; i < kStaged; ++i)
      *reinterpret_cast<int4*>(&stage[kb & 1][(r0 + (kGgThreads / 8) * i) * kGgStride + part * 16]) =
          staged[i];
  };
  stage_load(0);

  // Route targets and activation scales of the item.
  {
    constexpr int kSplit = kGgThreads / kR;  // threads per route row of scales
    const bool live = rs < routes;
    const float* srow = act_scales + static_cast<size_t>(route_row(rs, id_s)) * KB;
    float sc[(KB + kSplit - 1) / kSplit];
#pragma unroll
    for (int q = 0; q * kSplit + k0 < KB; ++q) sc[q] = srow[q * kSplit + k0];
#pragma unroll
    for (int q = 0; q * kSplit + k0 < KB; ++q) a_scale[q * kSplit + k0][rs] = live ? sc[q] : 0.0f;
    int t = MODE == 1 ? id_s : (kByPair ? slot * kR : first) + rs;
    if (dense) t = (MODE == 0 ? shared.pos : shared.pair) + first + rs;
    if (k0 == 0) target[rs] = live ? t : -1;
  }
  // Block scales of the wave's tiles for every K block (wave-uniform): FC1
  // tiles 0-1 (gate) share one 128-row block and tiles 2-3 (up) another; a
  // wave's four FC2 tiles lie in one block.
  float w_rows[2][KB];
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) {
    w_rows[0][kb] = wsexp[(tile_row(0) / kGroup) * KB + kb];
    w_rows[1][kb] = wsexp[(tile_row(2) / kGroup) * KB + kb];
  }
  stage_store(0);
  __syncthreads();

  floatx4 acc[kGgWaveTiles][kRT];
#pragma unroll
  for (int t = 0; t < kGgWaveTiles; ++t)
#pragma unroll
    for (int rt = 0; rt < kRT; ++rt) acc[t][rt] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

  // The next K block's loads in issue units (activation staging copies
  // first, so that waiting for them never waits for the weights; then one
  // weight tile, two loads, per unit), spread over the route tiles of the
  // current block so the MFMAs keep issuing while the loads go out.
  constexpr int kUnits = kStaged + kGgWaveTiles;
  auto issue_unit = [&](int kb, int u) {
    if (u < kStaged) {
      staged[u] = view.load16(src[u] + kb * kGroup);
    } else {
      const int t = u - kStaged;
      const uint32_t base = static_cast<uint32_t>(tile_row(t)) * K;
      int32x4 lo, hi;
      if constexpr (kPacked) {
        lo = __builtin_amdgcn_raw_buffer_load_b128(wrsrc, w_lane, base + kb * 2048, kNonTemporal);
        hi = __builtin_amdgcn_raw_buffer_load_b128(wrsrc, w_lane, base + kb * 2048 + 1024, kNonTemporal);
      } else {
        lo = __builtin_amdgcn_raw_buffer_load_b128(wrsrc, w_lane, base + kb * kGroup, 0);
        hi = __builtin_amdgcn_raw_buffer_load_b128(wrsrc, w_lane, base + kb * kGroup + 64, 0);
      }
      int32x8 v;
      v[0] = lo[0]; v[1] = lo[1]; v[2] = lo[2]; v[3] = lo[3];
      v[4] = hi[0]; v[5] = hi[1]; v[6] = hi[2]; v[7] = hi[3];
      wf[kb & 1][t] = v;
    }
  };
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) {
    // Keep each K block's loads in its own iteration (the unrolled loop would
    // otherwise let the scheduler hoist later blocks' loads).
    __builtin_amdgcn_sched_barrier(0);
    float wsc[kGgWaveTiles];
#pragma unroll
    for (int t = 0; t < kGgWaveTiles; ++t) wsc[t] = w_rows[t < 2 ? 0 : 1][kb];
    const uint8_t* buf = stage[kb & 1];
    // Software pipeline over the route tiles: the MFMAs of tile rt, then
    // the scale FMAs of tile rt - 1 (whose products are ready by then), so
    // at most two tiles' products are live next to the accumulators.
    floatx4 partial[2][kGgWaveTiles];
    float as_prev = 0.0f;
#pragma unroll
    for (int rt = 0; rt <= kRT; ++rt) {
      if (kb + 1 < KB) {  // units rt (and, on the last route tile, the rest)
#pragma unroll
        for (int u = 0; u < kUnits; ++u)
          if (u == rt || (rt == kRT - 1 && u >= kRT)) issue_unit(kb + 1, u);
      }
      float as = 0.0f;
      if (rt < kRT) {
        const int route = 16 * rt + row16;
        const int32x8 bfrag = load_fragment(buf + route * kGgStride, 0, group);
        as = a_scale[kb][route];
#pragma unroll
        for (int t = 0; t < kGgWaveTiles; ++t) partial[rt & 1][t] = mfma_fp8(wf[kb & 1][t], bfrag);
      }
      if (rt > 0) {
#pragma unroll
        for (int t = 0; t < kGgWaveTiles; ++t) {
          scale_accumulate(acc[t][rt - 1], partial[(rt - 1) & 1][t], wsc[t] * as_prev);
          // Materialise the sum here: the accumulators are only used under
          // the epilogue's per-route conditions, and without this the
          // compiler sinks every K block's FMAs (keeping every product live).
          asm volatile("" : "+v"(acc[t][rt - 1]));
        }
      }
      as_prev = as;
      __builtin_amdgcn_sched_barrier(0);
    }
    if (kb + 1 < KB) stage_store(kb + 1);
    __syncthreads();
  }

  if constexpr (MODE == 1) {
    // Each route tile's 16 x 256 fp32 block goes through LDS (two buffers in
    // the staging ring) so that every store writes one route's 1 KiB run.
    constexpr int kRowF = kGgRows + 4;
    static_assert(2 * 16 * kRowF * 4 <= 2 * kStage, "epilogue buffers fit the staging ring");
    float* tbuf = reinterpret_cast<float*>(&stage[0][0]);
#pragma unroll
    for (int rt = 0; rt < kRT; ++rt) {
      float* buf = tbuf + (rt & 1) * 16 * kRowF;
#pragma unroll
      for (int t = 0; t < kGgWaveTiles; ++t)
        *reinterpret_cast<floatx4*>(buf + row16 * kRowF + 64 * wave + 16 * t + 4 * group) = acc[t][rt];
      __syncthreads();
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = 4 * wave + j;
        const int pair = target[16 * rt + r];
        const floatx4 v = *reinterpret_cast<const floatx4*>(buf + r * kRowF + 4 * lane);
        if (pair >= 0) {
          float* dst = out_f32 + static_cast<size_t>(pair) * n_rows + n0 + 4 * lane;
          if constexpr (kStreamOut)
            __builtin_nontemporal_store(v, reinterpret_cast<floatx4*>(dst));
          else
            *reinterpret_cast<floatx4*>(dst) = v;
        }
      }
    }
  } else {
    // SwiGLU on the bf16-rounded FC1 outputs; lane holds gate / up columns
    // 32 wave + 16 p + 4 group + i (p < 2, i < 4) of route 16 rt + row16.
    float v[kRT][8];
#pragma unroll
    for (int rt = 0; rt < kRT; ++rt) {
      float g[8], u[8];
#pragma unroll
      for (int p = 0; p < 2; ++p)
#pragma unroll
        for (int i = 0; i < 4; i += 2) {
          const uint32_t gw = pack_bf16x2(acc[p][rt][i], acc[p][rt][i + 1]);
          const uint32_t uw = pack_bf16x2(acc[2 + p][rt][i], acc[2 + p][rt][i + 1]);
          g[4 * p + i] = bf16_lo(gw);
          g[4 * p + i + 1] = bf16_hi(gw);
          u[4 * p + i] = bf16_lo(uw);
          u[4 * p + i + 1] = bf16_hi(uw);
        }
      swiglu_values<8>(g, u, v[rt]);
      float amax = 0.0f;
#pragma unroll
      for (int k = 0; k < 8; ++k) amax = fmaxf(amax, fabsf(v[rt][k]));
      amax = fmaxf(amax, __shfl_xor(amax, 16));
      amax = fmaxf(amax, __shfl_xor(amax, 32));
      if (group == 0) amax_part[wave][16 * rt + row16] = amax;
    }
    __syncthreads();
    const int groups = out_cols / kGroup;
#pragma unroll
    for (int rt = 0; rt < kRT; ++rt) {
      const int route = 16 * rt + row16;
      const int position = target[route];
      if (position < 0) continue;
      float amax = amax_part[0][route];
#pragma unroll
      for (int q = 1; q < kGgWaves; ++q) amax = fmaxf(amax, amax_part[q][route]);
      const float scale = group_scale(amax);
      uint8_t* dst = out_codes + static_cast<size_t>(position) * out_cols + n0 + 32 * wave + 4 * group;
      *reinterpret_cast<uint32_t*>(dst) = quantize_four(&v[rt][0], scale);
      *reinterpret_cast<uint32_t*>(dst + 16) = quantize_four(&v[rt][4], scale);
      if (wave == 0 && group == 0) out_scales[static_cast<size_t>(position) * groups + tile] = scale;
    }
  }
}

struct GroupedLaunch {
  int mode;
  int layout;
  const uint8_t* w;
  const float* ws;
  int n_rows;
  int out_cols;
  const uint8_t* a;
  uint32_t a_bytes;
  const float* as;
  const int32_t* sorted_ids;
  int top_k;
  const int4* items;
  const int32_t* num_items;
  int max_items;
  int item_rows;
  SharedItems shared;
  uint8_t* codes;
  float* scales;
  float* out;
  int parts = 0;     // by-pair launches: work items per expert (0: sorted items)
  int capacity = 0;  // by-pair launches: slot rows of the ids
  int32_t* list_ids = nullptr;  // by-pair launches: the route list they write
  int4* list_items = nullptr;
  int32_t* list_count = nullptr;
};

template <int KB, int MODE>
void launch_grouped(const GroupedLaunch& g, hipStream_t s) {
  const int n_tiles = MODE == 0 ? g.out_cols / kGroup : g.n_rows / kGgRows;
  // Two consecutive items' tiles per XCD run.
  const int chunk = 2 * n_tiles;
  const int shared_items = g.shared.w ? (g.shared.rows + kGgRoutes - 1) / kGgRoutes : 0;
  const int64_t logical = (static_cast<int64_t>(g.max_items) + shared_items) * n_tiles;
  const int64_t per_round = static_cast<int64_t>(kGgXcds) * chunk;
  const int blocks = static_cast<int>((logical + per_round - 1) / per_round * per_round);
#define D3_GG_ARGS dim3(blocks), dim3(kGgThreads), 0, s, g.w, g.ws, g.n_rows, g.out_cols, g.a, \
                   g.a_bytes, g.as, g.sorted_ids, g.top_k, g.items, g.num_items, g.max_items, \
                   g.shared, n_tiles, chunk, g.parts, g.capacity, g.list_ids, g.list_items,   \
                   g.list_count, g.codes, g.scales, g.out
  if constexpr (MODE == 0) {
    if (g.parts > 0) {
      if (g.layout == D3_LAYOUT_FRAGMENT)
        hipLaunchKernelGGL((grouped_gemm_kernel<KB, MODE, true, true>), D3_GG_ARGS);
      else
        hipLaunchKernelGGL((grouped_gemm_kernel<KB, MODE, false, true>), D3_GG_ARGS);
      return;
    }
  }
  if constexpr (MODE == 1) {
    // Small batches (the mixed step's few thousand routes) write FC2's fp32
    // rows non-temporally: measured 1.4 us less per mixed step, while the
    // prefill batch (29k routes, 240 MB of rows) is 10 us slower that way.
    if ((static_cast<int64_t>(g.max_items) + shared_items) * kGgRoutes <= kStreamOutRoutes) {
      if (g.layout == D3_LAYOUT_FRAGMENT)
        hipLaunchKernelGGL((grouped_gemm_kernel<KB, MODE, true, false, true>), D3_GG_ARGS);
      else
        hipLaunchKernelGGL((grouped_gemm_kernel<KB, MODE, false, false, true>), D3_GG_ARGS);
      return;
    }
  }
  if (g.layout == D3_LAYOUT_FRAGMENT) {
    hipLaunchKernelGGL((grouped_gemm_kernel<KB, MODE, true, false>), D3_GG_ARGS);
  } else {
    hipLaunchKernelGGL((grouped_gemm_kernel<KB, MODE, false, false>), D3_GG_ARGS);
  }
#undef D3_GG_ARGS
}

template <int MODE>
int dispatch_grouped(const GroupedLaunch& g, int k, hipStream_t s) {
  switch (k / kGroup) {
    case 2: launch_grouped<2, MODE>(g, s); return D3_OK;
    case 4: launch_grouped<4, MODE>(g, s); return D3_OK;
    case 6: launch_grouped<6, MODE>(g, s); return D3_OK;
    case 8: launch_grouped<8, MODE>(g, s); return D3_OK;
    case 12: launch_grouped<12, MODE>(g, s); return D3_OK;
    case 16: launch_grouped<16, MODE>(g, s); return D3_OK;
    default:
      return set_error(D3_ERR_UNSUPPORTED, "grouped gemm: K=%d not in {256,512,768,1024,1536,2048}", k);
  }
}

bool aligned_to(const void* p, uintptr_t bytes) { return (reinterpret_cast<uintptr_t>(p) % bytes) == 0; }

int check_grouped(const GroupedLaunch& g, int num_experts, int k, int64_t a_rows, const char* name,
                  bool need_items = true) {
  D3_REQUIRE(g.w && g.ws && g.a && g.as && g.sorted_ids && (g.items || !need_items) && g.num_items,
             "%s: null pointer", name);
  D3_REQUIRE(g.layout == D3_LAYOUT_REFERENCE || g.layout == D3_LAYOUT_FRAGMENT,
             "%s: weight_layout must be D3_LAYOUT_REFERENCE or D3_LAYOUT_FRAGMENT", name);
  D3_REQUIRE(num_experts >= 1 && k > 0 && k % kGroup == 0, "%s: K=%d must be a positive multiple of 128",
             name, k);
  D3_REQUIRE(g.top_k >= 1 && g.max_items >= 0 && a_rows >= 1, "%s: bad top_k / max_items / rows", name);
  D3_REQUIRE(g.item_rows >= 1 && g.item_rows <= kGgRoutes, "%s: item_rows %d not in [1, %d]", name,
             g.item_rows, kGgRoutes);
  D3_REQUIRE(a_rows * k < (int64_t{1} << 31), "%s: activation buffer beyond 2 GiB", name);
  D3_REQUIRE(aligned_to(g.w, 16) && aligned_to(g.a, 16), "%s: operands must be 16-byte aligned", name);
  return D3_OK;
}

}  // namespace
}  // namespace d3

using namespace d3;

extern "C" int d3_grouped_fc1_swiglu(const uint8_t* w13, const float* s13, int32_t weight_layout,
                                     int32_t num_experts, int32_t intermediate, int32_t hidden,
                                     const uint8_t* q, int64_t q_rows, const float* x_scales,
                                     const int32_t* sorted_ids, int32_t top_k, const int32_t* items,
                                     const int32_t* num_items, int32_t max_items,
                                     int32_t item_rows, const uint8_t* shared_w13,
                                     const float* shared_s13, int32_t shared_rows,
                                     int32_t shared_act_row, uint8_t* act, float* act_scales,
                                     void* stream) {
  D3_REQUIRE(act && act_scales, "grouped_fc1_swiglu: null output");
  D3_REQUIRE(!shared_w13 || (shared_s13 && shared_rows >= 0 && shared_rows <= q_rows &&
                             shared_act_row >= 0 && aligned_to(shared_w13, 16)),
             "grouped_fc1_swiglu: shared expert needs scales, 0 <= rows <= q_rows, a row offset "
             "and 16-byte aligned weights");
  D3_REQUIRE(intermediate > 0 && intermediate % kGroup == 0,
             "grouped_fc1_swiglu: intermediate %d must be a multiple of 128", intermediate);
  D3_REQUIRE(aligned_to(act, 4), "grouped_fc1_swiglu: act must be 4-byte aligned");
  const GroupedLaunch g{0, weight_layout, w13, s13, 2 * intermediate, intermediate, q,
                        static_cast<uint32_t>(q_rows * hidden), x_scales, sorted_ids, top_k,
                        reinterpret_cast<const int4*>(items), num_items, max_items, item_rows,
                        SharedItems{shared_w13, shared_s13, shared_rows, shared_act_row, 0}, act,
                        act_scales, nullptr};
  int status = check_grouped(g, num_experts, hidden, q_rows, "grouped_fc1_swiglu");
  if (status != D3_OK) return status;
  if (max_items == 0 && !(shared_w13 && shared_rows > 0)) {
    clear_error();
    return D3_OK;
  }
  status = dispatch_grouped<0>(g, hidden, as_stream(stream));
  if (status != D3_OK) return status;
  D3_LAUNCHED("grouped_fc1_swiglu");
}

extern "C" int d3_grouped_fc2(const uint8_t* w2, const float* s2, int32_t weight_layout,
                              int32_t num_experts, int32_t hidden, int32_t intermediate,
                              const uint8_t* act, int64_t act_rows, const float* act_scales,
                              const int32_t* sorted_ids, int32_t top_k, const int32_t* items,
                              const int32_t* num_items, int32_t max_items, int32_t item_rows,
                              const uint8_t* shared_w2, const float* shared_s2,
                              int32_t shared_rows, int32_t shared_act_row,
                              int32_t shared_out_row, float* down, void* stream) {
  D3_REQUIRE(down != nullptr, "grouped_fc2: null output");
  D3_REQUIRE(!shared_w2 || (shared_s2 && shared_rows >= 0 && shared_act_row >= 0 &&
                            static_cast<int64_t>(shared_act_row) + shared_rows <= act_rows &&
                            shared_out_row >= 0 && aligned_to(shared_w2, 16)),
             "grouped_fc2: shared expert needs scales, its act rows inside act_rows, an output "
             "row offset and 16-byte aligned weights");
  D3_SUPPORTED(hidden > 0 && hidden % kGgRows == 0,
               "grouped_fc2: hidden %d must be a multiple of %d", hidden, kGgRows);
  D3_REQUIRE(aligned_to(down, 16), "grouped_fc2: down must be 16-byte aligned");
  const GroupedLaunch g{1, weight_layout, w2, s2, hidden, hidden, act,
                        static_cast<uint32_t>(act_rows * intermediate), act_scales, sorted_ids, top_k,
                        reinterpret_cast<const int4*>(items), num_items, max_items, item_rows,
                        SharedItems{shared_w2, shared_s2, shared_rows, shared_act_row, shared_out_row},
                        nullptr, nullptr, down};
  int status = check_grouped(g, num_experts, intermediate, act_rows, "grouped_fc2");
  if (status != D3_OK) return status;
  if (max_items == 0 && !(shared_w2 && shared_rows > 0)) {
    clear_error();
    return D3_OK;
  }
  status = dispatch_grouped<1>(g, intermediate, as_stream(stream));
  if (status != D3_OK) return status;
  D3_LAUNCHED("grouped_fc2");
}

extern "C" int d3_grouped_fc1_swiglu_by_pair(const uint8_t* w13, const float* s13,
                                             int32_t weight_layout, int32_t num_experts,
                                             int32_t intermediate, int32_t hidden,
                                             const uint8_t* q, int64_t q_rows,
                                             const float* x_scales, const int32_t* ids,
                                             int32_t top_k, const int32_t* row_count,
                                             int32_t capacity, uint8_t* act, float* act_scales,
                                             int32_t* list_ids, int32_t* list_items,
                                             int32_t* list_count, void* stream) {
  D3_REQUIRE(act && act_scales && ids && row_count && list_ids && list_items && list_count,
             "grouped_fc1_swiglu_by_pair: null pointer");
  D3_REQUIRE(intermediate > 0 && intermediate % kGroup == 0,
             "grouped_fc1_swiglu_by_pair: intermediate %d must be a multiple of 128", intermediate);
  D3_REQUIRE(capacity >= 1 && capacity <= q_rows, "grouped_fc1_swiglu_by_pair: capacity %d not in [1, %lld]",
             capacity, static_cast<long long>(q_rows));
  D3_SUPPORTED(static_cast<int64_t>(capacity) * top_k <= kGgMaxPairs,
               "grouped_fc1_swiglu_by_pair: capacity %d x top_k %d above %d routes", capacity, top_k,
               kGgMaxPairs);
  D3_REQUIRE(aligned_to(act, 4), "grouped_fc1_swiglu_by_pair: act must be 4-byte aligned");
  // work items of 64 routes, two per 128-route item of the list
  const int parts = (capacity + kGgRoutes - 1) / kGgRoutes * (kGgRoutes / kGgPairRoutes);
  GroupedLaunch g{0, weight_layout, w13, s13, 2 * intermediate, intermediate, q,
                  static_cast<uint32_t>(q_rows * hidden), x_scales, ids, top_k, nullptr, row_count,
                  num_experts * parts, kGgPairRoutes, SharedItems{nullptr, nullptr, 0, 0, 0}, act,
                  act_scales, nullptr};
  g.parts = parts;
  g.capacity = capacity;
  g.list_ids = list_ids;
  g.list_items = reinterpret_cast<int4*>(list_items);
  g.list_count = list_count;
  int status = check_grouped(g, num_experts, hidden, q_rows, "grouped_fc1_swiglu_by_pair",
                             /*need_items=*/false);
  if (status != D3_OK) return status;
  status = dispatch_grouped<0>(g, hidden, as_stream(stream));
  if (status != D3_OK) return status;
  D3_LAUNCHED("grouped_fc1_swiglu_by_pair");
}


