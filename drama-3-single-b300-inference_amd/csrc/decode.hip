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
#include "common.h"
#include "expert_tile.h"
#include "status.h"

namespace d3 {
namespace {

constexpr int kMaxSlots = 256;                        // rows per launch (one route per row and expert)
constexpr int kMaxIds = kMaxSlots * 8;                // ids read per workgroup (top_k <= 8)
constexpr int kIdsPerThread = kMaxIds / kGemmThreads;  // 8

// MODE 0: FC1, q rows of the routes' tokens x W13 -> bf16 gate|up by pair.
// MODE 2: FC2 with the SwiGLU requant in the prologue, gate|up by pair x W2
//         -> fp32 down by pair.
// TILES weight tiles per workgroup, streamed through the registers in halves
// (TILES > 1: routes beyond the first 16 reload the weight tiles).
template <int KB, int RT, int MODE, int TILES>
__global__ __launch_bounds__(kGemmThreads) __attribute__((amdgpu_waves_per_eu(2))) void decode_gemm_kernel(
    const uint8_t* __restrict__ w, const float* __restrict__ ws, int n_rows,
    const int32_t* __restrict__ ids, const int32_t* __restrict__ row_count, int capacity,
    int top_k, const void* __restrict__ act, const float* __restrict__ act_scales,
    int exact_routes, uint16_t* __restrict__ out_bf16, float* __restrict__ out_f32) {
  constexpr int K = KB * kGroup;
  constexpr int kRowsPerWave = RT * 16;
  constexpr int kRowsPerGroup = kGemmWaves * kRowsPerWave;
  constexpr int kStride = K + 16;  // 16-byte pad: the 16 rows of a ds_read_b128 hit distinct banks
  constexpr int kChunks = K / 256;
  constexpr int kFirstHalf = KB > 1 ? KB / 2 : KB;
  __shared__ __attribute__((aligned(16))) uint8_t b_tile[16 * kStride];
  __shared__ float b_scales[16 * KB];
  __shared__ int b_target[16];  // pair of each route column, -1 = none
  __shared__ int route_pairs[kMaxSlots];
  __shared__ int chunk_counts[kIdsPerThread * kGemmWaves];

  const int tiles = n_rows / kRowsPerGroup;
  const int groups = tiles / TILES;
  const int expert = blockIdx.x / groups;
  const int first_tile = (blockIdx.x % groups) * TILES;
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
  auto load_scales = [&](int tile) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) w_scale[rt][kb] = wsexp[((n0_of(tile) + rt * 16) / kGroup) * KB + kb];
  };

  // 1. The routed ids of every slot row (past the capacity: zeros, masked
  //    below), issued before any weight.
  const uint32_t id_bytes = static_cast<uint32_t>(capacity * top_k) * 4;
  const BufferView id_view(ids, id_bytes);
  uint32_t id[kIdsPerThread];
#pragma unroll
  for (int j = 0; j < kIdsPerThread; ++j) {
    const uint32_t p = static_cast<uint32_t>(j * kGemmThreads + threadIdx.x);
    id[j] = id_view.load4(p * 4 < id_bytes ? p * 4 : kNoRow);
  }
  const int rows = live_rows(row_count, capacity);
  // 2. The first half of the first weight tile streams meanwhile.
  load_weights(first_tile, 0, kFirstHalf);
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
  int routes = chunk_base;
  __syncthreads();
  routes = __builtin_amdgcn_readfirstlane(routes);
  if (routes == 0) return;  // no route for this expert: the loads issued so far are dropped
  const bool exact = routes <= exact_routes;

  // 4. Staging of one route tile (16 threads per route column), branch-free.
  const int stage_col = threadIdx.x >> 4;
  const int stage_part = threadIdx.x & 15;
  int4 b_stage[MODE == 0 ? kChunks : 1];
  float b_stage_scale = 0.0f;
  int stage_pair = -1;
  // MODE 2: live (route column, K group) units packed densely: unit
  // u = 16 p + stage_col is column u / KB, group u % KB.
  uint4 g_stage[MODE == 2 ? KB : 1], u_stage[MODE == 2 ? KB : 1];
  int live_units = 0;
  auto fetch_tile = [&](int m0) {
    const int r = m0 + stage_col;
    stage_pair = r < routes ? route_pairs[r] : -1;
    if constexpr (MODE == 0) {
      const BufferView rows_view(act, static_cast<uint32_t>(capacity) * K);
      const BufferView scale_view(act_scales, static_cast<uint32_t>(capacity) * KB * 4);
      const int token = stage_pair / top_k;
      const uint32_t offset = stage_pair >= 0 ? static_cast<uint32_t>(token) * K : kNoRow;
#pragma unroll
      for (int j = 0; j < kChunks; ++j) b_stage[j] = rows_view.load16(offset + j * 256 + stage_part * 16);
      b_stage_scale = __uint_as_float(scale_view.load4(
          stage_pair >= 0 && stage_part < KB ? static_cast<uint32_t>(token * KB + stage_part) * 4 : kNoRow));
    } else {
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
    } else {
#pragma unroll
      for (int j = 0; j < kChunks; ++j)
        *reinterpret_cast<int4*>(b_tile + stage_col * kStride + j * 256 + stage_part * 16) = b_stage[j];
      if (stage_part < KB) b_scales[stage_col * KB + stage_part] = b_stage_scale;
    }
    if (stage_part == 0) b_target[stage_col] = stage_pair;
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
          acc[rt] += partial * (w_scale[rt][kb] * b_scale);
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
          acc[rt] += partial * (w_scale[rt][kb] * b_scale);
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
      if constexpr (MODE == 0) {
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
  fetch_tile(0);
  __builtin_amdgcn_sched_barrier(0);
  load_weights(first_tile, kFirstHalf, KB);
  load_scales(first_tile);
  store_tile();
  __syncthreads();
  if constexpr (TILES > 1) {
    // Weight tiles stream through the same registers in halves: once the
    // first half of tile tt has been multiplied, the first half of tile
    // tt + 1 is loaded into its registers while the second half of tile tt
    // is multiplied, and so on, so every wave keeps at least half a tile of
    // loads in flight until its last tile (memory returns are counted in
    // issue order, so each wait covers only the half it needs).
#pragma unroll
    for (int tt = 0; tt < TILES; ++tt) {
      floatx4 acc[RT];
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) acc[rt] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
      mma_range(acc, 0, kFirstHalf);
      if (tt + 1 < TILES) {
        __builtin_amdgcn_sched_barrier(0);  // the next half reuses these registers
        load_weights(first_tile + tt + 1, 0, kFirstHalf);
      }
      mma_range(acc, kFirstHalf, KB);
      if (tt + 1 < TILES) {
        __builtin_amdgcn_sched_barrier(0);
        load_weights(first_tile + tt + 1, kFirstHalf, KB);
        load_scales(first_tile + tt + 1);
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
    for (int m0 = 16; m0 < routes; m0 += 16) {
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

bool aligned(const void* p, uintptr_t bytes) { return (reinterpret_cast<uintptr_t>(p) % bytes) == 0; }

template <int KB, int MODE, int TILES>
void launch_tiles(int num_experts, int n, hipStream_t s, const uint8_t* w, const float* ws,
                  const int32_t* ids, const int32_t* row_count, int capacity, int top_k,
                  const void* a, const float* as, int exact_routes, uint16_t* out_bf16,
                  float* out_f32) {
  const int tiles = n / tile_rows_for(KB);
  hipLaunchKernelGGL((decode_gemm_kernel<KB, rt_for(KB), MODE, TILES>),
                     dim3(num_experts * (tiles / TILES)), dim3(kGemmThreads), 0, s, w, ws, n, ids,
                     row_count, capacity, top_k, a, as, exact_routes, out_bf16, out_f32);
}

// Weight tiles per workgroup: enough that the whole grid is about one round
// of resident workgroups (two per CU), so each workgroup streams its tiles
// back to back instead of the GPU turning workgroups over; a divisor of the
// expert's tile count.  Experts averaging more than 8 routes at full
// capacity take one tile per workgroup (each further route tile would walk
// all of a workgroup's tiles again).
constexpr int kResidentGroups = 512;
int tiles_per_group(int num_experts, int tiles, int capacity, int top_k, int mode) {
  if (capacity * top_k > 8 * num_experts) return 1;
  const int options[] = {1, 2, 4, 6};
  const int limit = mode == 0 ? 6 : 4;
  for (int t : options)
    if (t <= limit && tiles % t == 0 && num_experts * (tiles / t) <= kResidentGroups) return t;
  for (int i = 3; i >= 0; --i)
    if (options[i] <= limit && tiles % options[i] == 0) return options[i];
  return 1;
}

template <int KB, int MODE>
void launch_decode(int num_experts, int n, hipStream_t s, const uint8_t* w, const float* ws,
                   const int32_t* ids, const int32_t* row_count, int capacity, int top_k,
                   const void* a, const float* as, int exact_routes, uint16_t* out_bf16,
                   float* out_f32) {
  const int tiles = n / tile_rows_for(KB);
  const int t = tiles_per_group(num_experts, tiles, capacity, top_k, MODE);
#define D3_TILES(T)                                                                             \
  launch_tiles<KB, MODE, T>(num_experts, n, s, w, ws, ids, row_count, capacity, top_k, a, as, \
                            exact_routes, out_bf16, out_f32)
  if constexpr (MODE == 0) {
    if (t == 6) { D3_TILES(6); return; }
  }
  if (t == 4) D3_TILES(4);
  else if (t == 2) D3_TILES(2);
  else D3_TILES(1);
#undef D3_TILES
}

}  // namespace
}  // namespace d3

using namespace d3;

extern "C" int d3_decode_expert_gemm(int32_t mode, const uint8_t* w, const float* ws,
                                     int32_t num_experts, int32_t n, int32_t k,
                                     const int32_t* ids, const int32_t* row_count,
                                     int32_t capacity, int32_t top_k, const void* a,
                                     const float* a_scales, int32_t exact_routes,
                                     uint16_t* out_bf16, float* out_f32, void* stream) {
  D3_REQUIRE(mode == 0 || mode == 2, "decode_expert_gemm: mode must be 0 (FC1) or 2 (FC2 + SwiGLU)");
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
  hipStream_t s = as_stream(stream);
#define D3_DECODE(KB_, MODE_)                                                                 \
  launch_decode<KB_, MODE_>(num_experts, n, s, w, ws, ids, row_count, capacity, top_k, a,    \
                            a_scales, exact_routes, out_bf16, out_f32)
  if (mode == 0) {
    if (kb == 8) D3_DECODE(8, 0); else D3_DECODE(16, 0);
  } else {
    if (kb == 2) D3_DECODE(2, 2); else if (kb == 4) D3_DECODE(4, 2); else if (kb == 6) D3_DECODE(6, 2); else D3_DECODE(8, 2);
  }
#undef D3_DECODE
  D3_LAUNCHED("decode_expert_gemm");
}
