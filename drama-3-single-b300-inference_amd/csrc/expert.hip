// Grouped FP8 expert GEMM over sorted routes, SwiGLU + FP8 requantisation,
// and the deterministic weighted combine.
//
// Expert GEMM design (gfx950, wave64, MFMA 16x16x128 OCP-FP8):
//   * A workgroup owns one work item {expert e, run of sorted routes} and a
//     tile of 4 waves x RT x 16 weight rows.  Each wave loads its RT x 16
//     weight rows for the whole contraction (K = KB x 128 bytes per row)
//     straight into registers before it touches any activation, so every
//     weight byte is read from HBM exactly once per work item and the loads
//     of all waves are in flight together.
//   * The routes are the MFMA's N dimension, 16 per tile; the workgroup walks
//     the item's routes tile by tile against the register-resident weights.
//     Decode items are a single tile (GEMV-like, bandwidth bound); prefill
//     items hold up to item_rows routes (a real contraction on the matrix
//     cores).
//   * The 128x128 weight block scale is uniform over a 16-row tile and the
//     activation scale is per route (= per MFMA column), so each 16x16x128
//     MFMA (exactly one K block) is rescaled with one fp32 multiply-add per
//     accumulator element: acc += mfma(w, a) * (w_scale * a_scale).
//   * Operand layout: lane l holds row/column l % 16 and 32 contraction bytes
//     of group g = l / 16.  Both operands use the same byte->k map (bytes
//     0-15 = k in [16g, 16g+16), bytes 16-31 = k in [64+16g, 64+16g+16)).
//     The product is invariant under any k permutation applied to both.
//   * Weights come in one of two layouts.  The reference layout [E, N, K]
//     gives each 16-byte load 64 contiguous bytes per row (16 rows per
//     instruction).  The fragment-major layout (d3_pack_expert_weights)
//     stores each 16-row tile as [K block][half][lane][16 bytes]: the two
//     loads of a fragment are each 1 KiB of contiguous memory per wave, read
//     non-temporally (every weight byte is used once).  On MI355X a pure
//     read stream of 1 KiB-contiguous non-temporal loads sustains 6.9-7.1
//     TB/s against 6.1 TB/s for the 16-row pattern.
//   * Two arithmetic paths, chosen per work item (uniform per workgroup):
//     - exact path (items with <= exact_routes routes: decode, bandwidth
//       bound): the FP8 bytes are widened to bf16 in registers (exact, e4m3
//       is a subset of bf16) and contracted with MFMA 16x16x32 bf16, whose
//       products are exact and whose accumulation has fp32 accuracy;
//     - contraction path (larger items: prefill): MFMA 16x16x128 FP8 at twice
//       the bf16 rate.  The FP8 instruction aligns the products of each
//       output element before summing with limited precision (measured on
//       MI355X: error up to ~1e-4 of sum|products|, exact when the products
//       share an exponent range), the same class of rounding as FP8 tensor
//       core GEMMs.
#include "common.h"
#include "expert_tile.h"
#include "status.h"

namespace d3 {
namespace {

template <int KB, int RT, int MODE, bool kPacked, int TILES>
__global__ __launch_bounds__(kGemmThreads) __attribute__((amdgpu_waves_per_eu(2))) void expert_gemm_kernel(
    const uint8_t* __restrict__ w, const float* __restrict__ ws, int n_rows,
    const uint8_t* __restrict__ act, const float* __restrict__ act_scales,
    const int32_t* __restrict__ sorted_ids, int top_k, const int4* __restrict__ items,
    const int32_t* __restrict__ num_items, int exact_routes, uint16_t* __restrict__ out_bf16,
    float* __restrict__ out_f32) {
  constexpr int K = KB * kGroup;
  constexpr int kRowsPerWave = RT * 16;
  constexpr int kRowsPerGroup = kGemmWaves * kRowsPerWave;
  // Activation tile: 16 routes x K bytes.  The 16-byte row pad rotates each
  // route row by 4 banks so the 16 rows of one ds_read_b128 hit distinct banks.
  constexpr int kStride = K + 16;
  __shared__ __attribute__((aligned(16))) uint8_t b_tile[16 * kStride];
  __shared__ float b_scales[16 * KB];
  __shared__ int b_target[16];  // FC1: sorted position, FC2: pair id; -1 = no route

  const int tiles = n_rows / kRowsPerGroup;
  const int groups = tiles / TILES;  // workgroups per item
  const int item_index = blockIdx.x / groups;
  const int first_tile = (blockIdx.x % groups) * TILES;
  if (item_index >= *num_items) return;
  const int4 item = items[item_index];
  const int expert = item.x;
  const int first = item.y;
  const int routes = item.z;  // every route of an item is live (no padding)
  const bool exact = routes <= exact_routes;

  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
  const int row16 = lane & 15;
  const int group = lane >> 4;
  // Rows of weight tile `tile` held by this wave: n0_of(tile) + [0, RT * 16).
  auto n0_of = [&](int tile) { return tile * kRowsPerGroup + wave * kRowsPerWave; };

  // Issue order of the first tile (memory returns are counted in issue
  // order): the first half of the weights, then the route ids (scalar loads,
  // counted apart from the vector stream) and the activation rows they name,
  // then the second half of the weights.  The staging wait then covers only
  // the first half, whose MFMAs overlap the second half's transfer (MODE 2
  // also computes the SwiGLU requantisation of the staged rows meanwhile).
  const int stage_col = threadIdx.x >> 4;   // route column staged by this thread
  const int stage_part = threadIdx.x & 15;  // 16 threads per route row
  constexpr int kChunks = K / 256;          // 16-byte chunks per thread and row
  int4 b_stage[kChunks];
  float b_stage_scale = 0.0f;
  int b_stage_target = -1;
  // MODE 2: the live (route column, K group) units of the tile, packed
  // densely: unit u = 16 p + stage_col is column u / KB, group u % KB, and
  // its 16-thread row holds 8 gate and 8 up bf16 values per thread.  Dead
  // columns are not computed (their output columns are never stored).
  uint4 g_stage[MODE == 2 ? KB : 1], u_stage[MODE == 2 ? KB : 1];
  int live_units = 0;
  auto fetch_tile = [&](int m0) {
    int pair = 0;
#pragma unroll
    for (int c = 0; c < 16; ++c) {  // uniform loads of the tile's 16 route ids
      const int id = m0 + c < routes ? sorted_ids[first + m0 + c] : 0;
      pair = stage_col == c ? id : pair;
    }
    const int r = m0 + stage_col;
    const bool live = r < routes;
    const int position = first + r;
    b_stage_target = live ? (MODE == 0 ? position : pair) : -1;
    if constexpr (MODE == 2) {
      live_units = min(16, routes - m0) * KB;
      const uint16_t* rows = reinterpret_cast<const uint16_t*>(act) +
                             static_cast<size_t>(first + m0) * (2 * K) + stage_part * 8;
#pragma unroll
      for (int p = 0; p < KB; ++p) {
        const int u = p * 16 + stage_col;
        if (p * 16 < live_units && u < live_units) {
          const int col = u / KB;
          const uint16_t* src = rows + static_cast<size_t>(col) * (2 * K) + (u - col * KB) * kGroup;
          g_stage[p] = *reinterpret_cast<const uint4*>(src);
          u_stage[p] = *reinterpret_cast<const uint4*>(src + K);
        }
      }
      return;
    }
    const size_t a_row = MODE == 0 ? static_cast<size_t>(pair / top_k) : static_cast<size_t>(position);
    const uint8_t* src = act + a_row * K;
#pragma unroll
    for (int j = 0; j < kChunks; ++j) {
      b_stage[j] = make_int4(0, 0, 0, 0);
      if (live) b_stage[j] = *reinterpret_cast<const int4*>(src + j * 256 + stage_part * 16);
    }
    b_stage_scale = (live && stage_part < KB) ? act_scales[a_row * KB + stage_part] : 0.0f;
  };
  auto store_tile = [&]() {
    if constexpr (MODE == 2) {
      // SwiGLU + e4m3 requantisation of the staged units, the same function
      // as silu_mul_quant_kernel, so the tile holds the bytes that kernel
      // would have written.  A unit's 16 threads are one DPP row.
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
    if (stage_part == 0) b_target[stage_col] = b_stage_target;
  };

  // A 16-row tile starts at the same offset in both weight layouts.
  const uint8_t* wexp = w + static_cast<size_t>(expert) * n_rows * K;
  int32x8 a_frag[RT][KB];
  auto load_weights = [&](int tile, int kb0, int kb1) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        if (kb < kb0 || kb >= kb1) continue;
        const uint8_t* rows = wexp + static_cast<size_t>(n0_of(tile) + rt * 16) * K;
        if constexpr (kPacked)
          a_frag[rt][kb] = load_packed_fragment(rows, kb, lane);
        else
          a_frag[rt][kb] = load_fragment(rows + row16 * K, kb, group);
      }
  };
  float w_scale[RT][KB];
  const float* wsexp = ws + static_cast<size_t>(expert) * (n_rows / kGroup) * KB;
  auto load_scales = [&](int tile) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) w_scale[rt][kb] = wsexp[((n0_of(tile) + rt * 16) / kGroup) * KB + kb];
  };
  constexpr int kFirstHalf = MODE == 2 ? 0 : (KB > 1 ? KB / 2 : KB);
  load_weights(first_tile, 0, kFirstHalf);
  __builtin_amdgcn_sched_barrier(0);
  // MODE 2 issues the gate / up rows before any weight (they are addressed
  // by sorted position, no route id needed), so the SwiGLU arithmetic runs
  // while the whole weight tile is in flight.
  fetch_tile(0);
  __builtin_amdgcn_sched_barrier(0);
  load_weights(first_tile, kFirstHalf, KB);
  load_scales(first_tile);

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
          scale_accumulate(acc[rt], partial, w_scale[rt][kb] * b_scale);
        }
        // Keep one K block's widened operands live at a time (the weights
        // already occupy most of the register file).
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
          scale_accumulate(acc[rt], partial, w_scale[rt][kb] * b_scale);
        }
      }
    }
  };
  auto epilogue = [&](const floatx4 (&acc)[RT], int tile) {
    const int target = b_target[row16];
    if (target >= 0) {
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        const int n = n0_of(tile) + rt * 16 + group * 4;  // rows n..n+3 of this column
        if constexpr (MODE == 0) {
          const uint32_t lo = f32_to_bf16(acc[rt][0]) | (static_cast<uint32_t>(f32_to_bf16(acc[rt][1])) << 16);
          const uint32_t hi = f32_to_bf16(acc[rt][2]) | (static_cast<uint32_t>(f32_to_bf16(acc[rt][3])) << 16);
          uint16_t* dst = out_bf16 + static_cast<size_t>(target) * n_rows + n;
          *reinterpret_cast<uint2*>(dst) = make_uint2(lo, hi);
        } else {
          float* dst = out_f32 + static_cast<size_t>(target) * n_rows + n;
          *reinterpret_cast<float4*>(dst) = make_float4(acc[rt][0], acc[rt][1], acc[rt][2], acc[rt][3]);
        }
      }
    }
  };
  // The first route tile is staged outside any loop: staged registers
  // carried around a loop back edge make the compiler wait for every
  // outstanding load (the weights included) before staging.
  store_tile();
  if constexpr (TILES > 1) {
    // Items of at most 16 routes (one route tile, a launch contract): the
    // TILES weight tiles pass through the same registers, tile tt + 1
    // streaming in while tile tt's outputs are stored.
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
  } else {
    // Route tiles of 16 against the one weight tile.
    for (int m0 = 0; m0 < routes; m0 += 16) {
      if (m0 > 0) {
        __syncthreads();  // previous route tile fully consumed
        fetch_tile(m0);
        store_tile();
      }
      __syncthreads();
      floatx4 acc[RT];
      mma(acc);
      epilogue(acc, first_tile);
    }
  }
}

// ---------------------------------------------------------------------------
// SwiGLU + per-128 requantisation: one thread per 8 columns, so a 16-lane
// DPP row is exactly one 128-column group (I / 8 threads per FC1 row, a
// multiple of 16).  The gate/up loads are issued together with the loads
// of the row count and sorted id (every row below `rows` is inside the
// buffer, live or not), so a row costs one memory latency.
// ---------------------------------------------------------------------------
constexpr int kRowThreads = 256;

__global__ __launch_bounds__(kRowThreads) void silu_mul_quant_kernel(
    const uint16_t* __restrict__ gate_up, int rows, int intermediate,
    const int32_t* __restrict__ row_count, const int32_t* __restrict__ sorted_ids,
    const int32_t* __restrict__ pairs_dev, int pairs_host, uint8_t* __restrict__ act,
    float* __restrict__ act_scales) {
  const int per_row = intermediate / 8;
  const int64_t thread = static_cast<int64_t>(blockIdx.x) * kRowThreads + threadIdx.x;
  const int row = static_cast<int>(thread / per_row);
  const int column = static_cast<int>(thread % per_row) * 8;
  if (row >= rows) return;  // whole 16-lane groups agree
  const uint16_t* gate = gate_up + static_cast<size_t>(row) * 2 * intermediate + column;
  const uint4 graw = *reinterpret_cast<const uint4*>(gate);
  const uint4 uraw = *reinterpret_cast<const uint4*>(gate + intermediate);
  if (row >= live_rows(row_count, rows)) return;
  if (sorted_ids != nullptr) {
    const int pairs = pairs_dev != nullptr ? *pairs_dev : pairs_host;
    if (sorted_ids[row] >= pairs) return;  // padding slot of the sorted layout
  }
  uint2 codes;
  const float scale = swiglu_quant_group(graw, uraw, &codes);
  *reinterpret_cast<uint2*>(act + static_cast<size_t>(row) * intermediate + column) = codes;
  if ((lane_id() & 15) == 0)
    act_scales[static_cast<size_t>(row) * (intermediate / kGroup) + column / kGroup] = scale;
}

// ---------------------------------------------------------------------------
// Weighted combine: out[t] = bf16(sum_r w[t,r] * down[t*K + r]) in rank order.
// ---------------------------------------------------------------------------
// One workgroup per (row, 512-column slice); with top_k = 8 every load of
// the slice is issued before the first FMA (combine4_fixed).

// 128 threads x 4 columns: a c2 decode step (52 rows x 2048 columns) spreads
// over 208 workgroups, so most CUs have one row slice in flight.
constexpr int kCombineThreads = 128;
constexpr int kCombineColumns = kCombineThreads * 4;

__global__ __launch_bounds__(kCombineThreads) void weighted_combine_kernel(
    const float* __restrict__ down, const void* __restrict__ weights, int weights_f32, int rows,
    int top_k, int hidden, const int32_t* __restrict__ row_count,
    const float* __restrict__ shared, uint16_t* __restrict__ out) {
  const int slices = (hidden + kCombineColumns - 1) / kCombineColumns;
  const int row = blockIdx.x / slices;
  const int column = (blockIdx.x % slices) * kCombineColumns + threadIdx.x * 4;
  if (column >= hidden) return;
  float4 acc = top_k == 8 ? combine4_fixed<8>(down, weights, weights_f32, row, hidden, column)
                          : combine4(down, weights, weights_f32, row, top_k, hidden, column);
  if (row >= live_rows(row_count, rows)) return;
  if (shared != nullptr) {
    // Dense shared expert added to the routed output, each rounded to bf16.
    const float4 s = *reinterpret_cast<const float4*>(shared + static_cast<size_t>(row) * hidden + column);
    acc.x = bf16_to_f32(f32_to_bf16(acc.x)) + bf16_to_f32(f32_to_bf16(s.x));
    acc.y = bf16_to_f32(f32_to_bf16(acc.y)) + bf16_to_f32(f32_to_bf16(s.y));
    acc.z = bf16_to_f32(f32_to_bf16(acc.z)) + bf16_to_f32(f32_to_bf16(s.z));
    acc.w = bf16_to_f32(f32_to_bf16(acc.w)) + bf16_to_f32(f32_to_bf16(s.w));
  }
  *reinterpret_cast<uint2*>(out + static_cast<size_t>(row) * hidden + column) = pack_bf16x4(acc);
}

// ---------------------------------------------------------------------------
// Reference layout -> fragment-major layout, one thread per 16-byte chunk of
// the output: chunk o = ((tile * KB + kb) * 2 + half) * 64 + lane holds
// bytes [kb*128 + 64*half + 16*(lane/16), +16) of row 16*tile + lane % 16
// (tiles run over all experts' rows: N is a multiple of 16).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void pack_weights_kernel(const uint8_t* __restrict__ w,
                                                           uint8_t* __restrict__ packed,
                                                           size_t chunks, int k) {
  const int kbs = k / kGroup;
  for (size_t o = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; o < chunks;
       o += static_cast<size_t>(gridDim.x) * 256) {
    const int lane = static_cast<int>(o % kWave);
    const int half = static_cast<int>((o / kWave) % 2);
    const size_t block = o / (2 * kWave);  // tile * KB + kb
    const int kb = static_cast<int>(block % kbs);
    const size_t row = (block / kbs) * 16 + (lane & 15);
    const size_t column = static_cast<size_t>(kb) * kGroup + 64 * half + 16 * (lane >> 4);
    *reinterpret_cast<int4*>(packed + o * 16) = *reinterpret_cast<const int4*>(w + row * k + column);
  }
}

struct GemmLaunch {
  int mode;
  int packed;  // weight layout: 0 reference [E, N, K], 1 fragment-major
  const uint8_t* w;
  const float* ws;
  int n;
  const uint8_t* a;
  const float* as;
  const int32_t* sorted_ids;
  int top_k;
  const int4* items;
  const int32_t* num_items;
  int max_items;
  int item_rows;  // upper bound on the routes of one item
  int exact_routes;
  uint16_t* out_bf16;
  float* out_f32;
};

// Weight tiles per workgroup: FC2 takes two when every item is one route
// tile and the tile count is even (the second tile streams in while the
// first one's outputs are stored, the activation staging - and for MODE 2
// the SwiGLU requant - is done once, and the two-tile kernel fits three
// workgroups per CU).  FC1 keeps one: its tiles are 128 KiB, and longer
// workgroups leave a longer partial last round (measured on c2: 65.5 us
// with two tiles against 62.5 us with one).
template <int KB, int RT, int MODE>
void launch_gemm(int tiles, hipStream_t s, const GemmLaunch& g) {
  const bool pair = MODE != 0 && tiles % 2 == 0 && g.item_rows <= 16;
  const dim3 grid(g.max_items * (pair ? tiles / 2 : tiles));
#define D3_GEMM_ARGS                                                                          \
  grid, dim3(kGemmThreads), 0, s, g.w, g.ws, g.n, g.a, g.as, g.sorted_ids, g.top_k, g.items, \
      g.num_items, g.exact_routes, g.out_bf16, g.out_f32
  if (pair) {
    if (g.packed)
      hipLaunchKernelGGL((expert_gemm_kernel<KB, RT, MODE, true, 2>), D3_GEMM_ARGS);
    else
      hipLaunchKernelGGL((expert_gemm_kernel<KB, RT, MODE, false, 2>), D3_GEMM_ARGS);
    return;
  }
  if (g.packed)
    hipLaunchKernelGGL((expert_gemm_kernel<KB, RT, MODE, true, 1>), D3_GEMM_ARGS);
  else
    hipLaunchKernelGGL((expert_gemm_kernel<KB, RT, MODE, false, 1>), D3_GEMM_ARGS);
#undef D3_GEMM_ARGS
}

// FC2 with the SwiGLU prologue stages 2 x 16 bytes of gate / up per K block
// and thread next to the weights; beyond 8 K blocks that spills.
constexpr int kMaxSwigluKB = 8;


template <int KB>
int dispatch_gemm(const GemmLaunch& g, hipStream_t s) {
  constexpr int RT = rt_for(KB);
  constexpr int rows_per_group = tile_rows_for(KB);
  D3_SUPPORTED(g.n % rows_per_group == 0, "expert_gemm: N=%d must be a multiple of %d for K=%d",
               g.n, rows_per_group, KB * kGroup);
  const int tiles = g.n / rows_per_group;
  if (g.mode == 0)
    launch_gemm<KB, RT, 0>(tiles, s, g);
  else if (g.mode == 1)
    launch_gemm<KB, RT, 1>(tiles, s, g);
  else if constexpr (KB <= kMaxSwigluKB)
    launch_gemm<KB, RT, 2>(tiles, s, g);
  else
    return set_error(D3_ERR_UNSUPPORTED, "expert_fc2_swiglu: intermediate %d > %d", KB * kGroup,
                     kMaxSwigluKB * kGroup);
  return D3_OK;
}

int run_gemm(const GemmLaunch& g, int k, hipStream_t s) {
  switch (k / kGroup) {
    case 2: return dispatch_gemm<2>(g, s);
    case 4: return dispatch_gemm<4>(g, s);
    case 6: return dispatch_gemm<6>(g, s);
    case 8: return dispatch_gemm<8>(g, s);
    case 12: return dispatch_gemm<12>(g, s);
    case 16: return dispatch_gemm<16>(g, s);
    default: return set_error(D3_ERR_UNSUPPORTED, "expert_gemm: K=%d not in the compiled set", k);
  }
}

int tile_rows(int k) {
  switch (k / kGroup) {
    case 2: return tile_rows_for(2);
    case 4: return tile_rows_for(4);
    case 6: return tile_rows_for(6);
    case 8: return tile_rows_for(8);
    case 12: return tile_rows_for(12);
    case 16: return tile_rows_for(16);
    default: return -1;
  }
}

bool aligned(const void* p, uintptr_t bytes) { return (reinterpret_cast<uintptr_t>(p) % bytes) == 0; }

int check_gemm(const GemmLaunch& g, int num_experts, int k, const char* name) {
  D3_REQUIRE(g.w && g.ws && g.a && (g.as || g.mode == 2) && g.sorted_ids && g.items && g.num_items,
             "%s: null pointer", name);
  D3_REQUIRE(g.packed == D3_LAYOUT_REFERENCE || g.packed == D3_LAYOUT_FRAGMENT,
             "%s: weight_layout must be D3_LAYOUT_REFERENCE or D3_LAYOUT_FRAGMENT", name);
  D3_REQUIRE(num_experts >= 1 && g.n > 0 && k > 0 && g.n % kGroup == 0 && k % kGroup == 0,
             "%s: N=%d, K=%d must be positive multiples of 128", name, g.n, k);
  D3_REQUIRE(g.top_k >= 1 && g.max_items >= 0, "%s: bad top_k/max_items", name);
  D3_REQUIRE(aligned(g.w, 16) && aligned(g.a, 16), "%s: operands must be 16-byte aligned", name);
  D3_SUPPORTED(k % 256 == 0 && tile_rows(k) > 0, "%s: K=%d not in the compiled set", name, k);
  return D3_OK;
}

}  // namespace
}  // namespace d3

using namespace d3;

extern "C" int32_t d3_expert_tile_rows(int32_t k) { return k % kGroup ? -1 : tile_rows(k); }

extern "C" int d3_expert_gemm(int32_t mode, const uint8_t* w, const float* ws,
                              int32_t weight_layout, int32_t num_experts, int32_t n, int32_t k,
                              const uint8_t* a, const float* a_scales,
                              const int32_t* sorted_ids, int32_t top_k, const int32_t* items,
                              const int32_t* num_items, int32_t max_items, int32_t item_rows,
                              int32_t exact_routes, uint16_t* out_bf16, float* out_f32,
                              void* stream) {
  D3_REQUIRE(mode == 0 || mode == 1, "expert_gemm: mode must be 0 (FC1) or 1 (FC2)");
  D3_REQUIRE(mode == 0 ? out_bf16 != nullptr : out_f32 != nullptr, "expert_gemm: null output");
  D3_REQUIRE(mode == 0 ? aligned(out_bf16, 8) : aligned(out_f32, 16),
             "expert_gemm: output alignment");
  D3_REQUIRE(item_rows >= 1, "expert_gemm: item_rows must be positive");
  const GemmLaunch g{mode, weight_layout, w, ws, n, a, a_scales, sorted_ids, top_k,
                     reinterpret_cast<const int4*>(items), num_items, max_items, item_rows,
                     exact_routes, out_bf16, out_f32};
  int status = check_gemm(g, num_experts, k, "expert_gemm");
  if (status != D3_OK) return status;
  if (max_items == 0) {
    clear_error();
    return D3_OK;
  }
  status = run_gemm(g, k, as_stream(stream));
  if (status != D3_OK) return status;
  D3_LAUNCHED("expert_gemm");
}

extern "C" int d3_expert_fc2_swiglu(const uint8_t* w2, const float* s2, int32_t weight_layout,
                                    int32_t num_experts, int32_t hidden, int32_t intermediate,
                                    const uint16_t* gate_up, const int32_t* sorted_ids,
                                    int32_t top_k, const int32_t* items, const int32_t* num_items,
                                    int32_t max_items, int32_t item_rows, int32_t exact_routes,
                                    float* down, void* stream) {
  D3_REQUIRE(gate_up && down, "expert_fc2_swiglu: null pointer");
  D3_REQUIRE(item_rows >= 1, "expert_fc2_swiglu: item_rows must be positive");
  D3_REQUIRE(aligned(gate_up, 16) && aligned(down, 16), "expert_fc2_swiglu: alignment");
  const GemmLaunch g{2, weight_layout, w2, s2, hidden,
                     reinterpret_cast<const uint8_t*>(gate_up), nullptr, sorted_ids, top_k,
                     reinterpret_cast<const int4*>(items), num_items, max_items, item_rows,
                     exact_routes, nullptr, down};
  int status = check_gemm(g, num_experts, intermediate, "expert_fc2_swiglu");
  if (status != D3_OK) return status;
  if (max_items == 0) {
    clear_error();
    return D3_OK;
  }
  status = run_gemm(g, intermediate, as_stream(stream));
  if (status != D3_OK) return status;
  D3_LAUNCHED("expert_fc2_swiglu");
}

extern "C" int d3_silu_mul_quant(const uint16_t* gate_up, int32_t rows, int32_t intermediate,
                                 const int32_t* row_count, const int32_t* sorted_ids,
                                 const int32_t* pairs_dev, int32_t pairs, uint8_t* act,
                                 float* act_scales, void* stream) {
  D3_REQUIRE(gate_up && act && act_scales, "silu_mul_quant: null pointer");
  D3_REQUIRE(rows >= 0 && intermediate > 0 && intermediate % kGroup == 0,
             "silu_mul_quant: intermediate %d must be a positive multiple of 128", intermediate);
  D3_REQUIRE(aligned(gate_up, 16) && aligned(act, 8), "silu_mul_quant: alignment");
  if (rows == 0) {
    clear_error();
    return D3_OK;
  }
  const int64_t threads = static_cast<int64_t>(rows) * (intermediate / 8);
  const int blocks = static_cast<int>((threads + kRowThreads - 1) / kRowThreads);
  hipLaunchKernelGGL(silu_mul_quant_kernel, dim3(blocks), dim3(kRowThreads), 0, as_stream(stream),
                     gate_up, rows, intermediate, row_count, sorted_ids, pairs_dev, pairs, act,
                     act_scales);
  D3_LAUNCHED("silu_mul_quant");
}

extern "C" int d3_weighted_combine(const float* down, const void* weights, int32_t weights_dtype,
                                   int32_t rows, int32_t top_k, int32_t hidden,
                                   const int32_t* row_count, const float* shared, uint16_t* out,
                                   void* stream) {
  D3_REQUIRE(down && weights && out, "weighted_combine: null pointer");
  D3_REQUIRE(weights_dtype == D3_DTYPE_BF16 || weights_dtype == D3_DTYPE_F32,
             "weighted_combine: weights must be bf16 or f32");
  D3_REQUIRE(rows >= 0 && top_k >= 1 && top_k <= 16 && hidden > 0 && hidden % 4 == 0,
             "weighted_combine: bad shape");
  D3_REQUIRE(aligned(down, 16) && aligned(out, 8) && (shared == nullptr || aligned(shared, 16)),
             "weighted_combine: alignment");
  if (rows == 0) {
    clear_error();
    return D3_OK;
  }
  const int slices = (hidden + kCombineColumns - 1) / kCombineColumns;
  hipLaunchKernelGGL(weighted_combine_kernel, dim3(rows * slices), dim3(kCombineThreads), 0,
                     as_stream(stream),
                     down, weights, weights_dtype == D3_DTYPE_F32 ? 1 : 0, rows, top_k, hidden,
                     row_count, shared, out);
  D3_LAUNCHED("weighted_combine");
}

extern "C" int d3_pack_expert_weights(const uint8_t* w, int32_t num_experts, int32_t n, int32_t k,
                                      uint8_t* packed, void* stream) {
  D3_REQUIRE(w && packed, "pack_expert_weights: null pointer");
  D3_REQUIRE(w != packed, "pack_expert_weights: cannot pack in place");
  D3_REQUIRE(num_experts >= 0 && n > 0 && n % 16 == 0 && k > 0 && k % kGroup == 0,
             "pack_expert_weights: N=%d must be a multiple of 16 and K=%d of 128", n, k);
  D3_REQUIRE(aligned(w, 16) && aligned(packed, 16), "pack_expert_weights: 16-byte alignment");
  const size_t chunks = static_cast<size_t>(num_experts) * n * (k / 16);
  if (chunks == 0) {
    clear_error();
    return D3_OK;
  }
  const size_t want = (chunks + 255) / 256;
  const int blocks = static_cast<int>(want < 65536 ? want : 65536);
  hipLaunchKernelGGL(pack_weights_kernel, dim3(blocks), dim3(256), 0, as_stream(stream), w, packed,
                     chunks, k);
  D3_LAUNCHED("pack_expert_weights");
}
