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
//     0-15 = k in [16g, 16g+16), bytes 16-31 = k in [64+16g, 64+16g+16)), so
//     each 16-byte load covers 64 contiguous bytes per row per instruction.
//     The product is invariant under any k permutation applied to both.
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
#include "status.h"

namespace d3 {
namespace {

typedef int int32x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

constexpr int kGemmWaves = 4;
constexpr int kGemmThreads = kGemmWaves * kWave;

__device__ __forceinline__ int32x8 load_fragment(const uint8_t* row, int kb, int group) {
  const uint8_t* p = row + kb * kGroup + group * 16;
  const int4 lo = *reinterpret_cast<const int4*>(p);
  const int4 hi = *reinterpret_cast<const int4*>(p + 64);
  int32x8 v;
  v[0] = lo.x; v[1] = lo.y; v[2] = lo.z; v[3] = lo.w;
  v[4] = hi.x; v[5] = hi.y; v[6] = hi.z; v[7] = hi.w;
  return v;
}

__device__ __forceinline__ floatx4 mfma_fp8(const int32x8& a, const int32x8& b) {
  const floatx4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
  // cbsz = blgp = 0 selects OCP E4M3 for both operands; zero scale operands
  // select the unscaled instruction.
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, zero, 0, 0, 0, 0, 0, 0);
}

// 32 e4m3 bytes -> 4 x 8 bf16, exactly (scale 1.0).  Element i of part j is
// byte 8j + i, for both operands alike.
__device__ __forceinline__ void widen_fp8(const int32x8& v, bf16x8 out[4]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const bf16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(v[2 * j], 1.0f, false);
    const bf16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(v[2 * j], 1.0f, true);
    const bf16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(v[2 * j + 1], 1.0f, false);
    const bf16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(v[2 * j + 1], 1.0f, true);
    out[j] = bf16x8{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
  }
}

// One K128 block on the exact path: four chained bf16 MFMAs.  The weight
// fragment is passed through an empty asm so the widening cannot be hoisted
// out of the route-tile loop (that would hold every K block in bf16 at once).
__device__ __forceinline__ floatx4 mfma_block_bf16(int32x8 a, const bf16x8 b[4]) {
  asm volatile("" : "+v"(a));
  bf16x8 wide[4];
  widen_fp8(a, wide);
  floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int j = 0; j < 4; ++j) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wide[j], b[j], acc, 0, 0, 0);
  return acc;
}

template <int KB, int RT, int MODE>
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
  const int item_index = blockIdx.x / tiles;
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
  const int n0 = (blockIdx.x % tiles) * kRowsPerGroup + wave * kRowsPerWave;

  // The first route tile's activation rows are fetched before the weights:
  // memory returns are counted in issue order, so staging issued behind the
  // weights would wait for all of them before the first MFMA.
  const int stage_col = threadIdx.x >> 4;   // route column staged by this thread
  const int stage_part = threadIdx.x & 15;  // 16 threads per route row
  constexpr int kChunks = K / 256;          // 16-byte chunks per thread and row
  int4 b_stage[kChunks];
  float b_stage_scale = 0.0f;
  int b_stage_target = -1;
  auto fetch_tile = [&](int m0) {
    const int r = m0 + stage_col;
    const bool live = r < routes;
    const int position = first + r;
    const int pair = live ? sorted_ids[position] : 0;
    const size_t a_row = MODE == 0 ? static_cast<size_t>(pair / top_k) : static_cast<size_t>(position);
    const uint8_t* src = act + a_row * K;
#pragma unroll
    for (int j = 0; j < kChunks; ++j) {
      b_stage[j] = make_int4(0, 0, 0, 0);
      if (live) b_stage[j] = *reinterpret_cast<const int4*>(src + j * 256 + stage_part * 16);
    }
    b_stage_scale = (live && stage_part < KB) ? act_scales[a_row * KB + stage_part] : 0.0f;
    b_stage_target = live ? (MODE == 0 ? position : pair) : -1;
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int j = 0; j < kChunks; ++j)
      *reinterpret_cast<int4*>(b_tile + stage_col * kStride + j * 256 + stage_part * 16) = b_stage[j];
    if (stage_part < KB) b_scales[stage_col * KB + stage_part] = b_stage_scale;
    if (stage_part == 0) b_target[stage_col] = b_stage_target;
  };
  fetch_tile(0);

  // Weights for the whole contraction: the bulk of the HBM stream.
  const uint8_t* wexp = w + static_cast<size_t>(expert) * n_rows * K;
  int32x8 a_frag[RT][KB];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const uint8_t* row = wexp + static_cast<size_t>(n0 + rt * 16 + row16) * K;
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) a_frag[rt][kb] = load_fragment(row, kb, group);
  }
  float w_scale[RT][KB];
  const float* wsexp = ws + static_cast<size_t>(expert) * (n_rows / kGroup) * KB;
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) w_scale[rt][kb] = wsexp[((n0 + rt * 16) / kGroup) * KB + kb];

  for (int m0 = 0; m0 < routes; m0 += 16) {
    if (m0 > 0) {
      __syncthreads();  // previous tile fully consumed
      fetch_tile(m0);
    }
    store_tile();
    __syncthreads();

    floatx4 acc[RT];
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
          acc[rt] += partial * (w_scale[rt][kb] * b_scale);
        }
      }
    }
    const int target = b_target[row16];
    if (target >= 0) {
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        const int n = n0 + rt * 16 + group * 4;  // rows n..n+3 of this column
        if constexpr (MODE == 0) {
          const uint32_t lo = f32_to_bf16(acc[rt][0]) | (static_cast<uint32_t>(f32_to_bf16(acc[rt][1])) << 16);
          const uint32_t hi = f32_to_bf16(acc[rt][2]) | (static_cast<uint32_t>(f32_to_bf16(acc[rt][3])) << 16);
          *reinterpret_cast<uint2*>(out_bf16 + static_cast<size_t>(target) * n_rows + n) =
              make_uint2(lo, hi);
        } else {
          *reinterpret_cast<float4*>(out_f32 + static_cast<size_t>(target) * n_rows + n) =
              make_float4(acc[rt][0], acc[rt][1], acc[rt][2], acc[rt][3]);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// SwiGLU + per-128 requantisation: one wave per FC1 row, 8 elements per lane.
// ---------------------------------------------------------------------------
constexpr int kRowThreads = 256;

__global__ __launch_bounds__(kRowThreads) void silu_mul_quant_kernel(
    const uint16_t* __restrict__ gate_up, int rows, int intermediate,
    const int32_t* __restrict__ row_count, const int32_t* __restrict__ sorted_ids,
    const int32_t* __restrict__ pairs_dev, int pairs_host, uint8_t* __restrict__ act,
    float* __restrict__ act_scales) {
  const int row = (blockIdx.x * kRowThreads + threadIdx.x) / kWave;
  const int lane = lane_id();
  if (row >= live_rows(row_count, rows)) return;
  if (sorted_ids != nullptr) {
    const int pairs = pairs_dev != nullptr ? *pairs_dev : pairs_host;
    if (sorted_ids[row] >= pairs) return;  // padding slot of the sorted layout
  }
  const uint16_t* gate = gate_up + static_cast<size_t>(row) * 2 * intermediate;
  const uint16_t* up = gate + intermediate;
  uint8_t* out = act + static_cast<size_t>(row) * intermediate;
  const int groups = intermediate / kGroup;
  for (int base = 0; base < intermediate; base += 8 * kWave) {
    const int column = base + lane * 8;
    const bool inside = column < intermediate;
    uint4 graw = make_uint4(0u, 0u, 0u, 0u), uraw = make_uint4(0u, 0u, 0u, 0u);
    if (inside) {
      graw = *reinterpret_cast<const uint4*>(gate + column);
      uraw = *reinterpret_cast<const uint4*>(up + column);
    }
    const uint32_t gw[4] = {graw.x, graw.y, graw.z, graw.w};
    const uint32_t uw[4] = {uraw.x, uraw.y, uraw.z, uraw.w};
    float v[8];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t gbits = (i & 1) ? (gw[i / 2] & 0xffff0000u) : (gw[i / 2] << 16);
      const uint32_t ubits = (i & 1) ? (uw[i / 2] & 0xffff0000u) : (uw[i / 2] << 16);
      const float g = __uint_as_float(gbits);
      const float u = __uint_as_float(ubits);
      const float sig = 1.0f / (1.0f + expf(-g));
      v[i] = (g * sig) * u;
      amax = fmaxf(amax, fabsf(v[i]));
    }
    amax = segment_max<16>(amax);
    const float scale = group_scale(amax);
    uint32_t lo = 0u, hi = 0u;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      lo |= quantize_one(v[i], scale) << (8 * i);
      hi |= quantize_one(v[i + 4], scale) << (8 * i);
    }
    if (inside) {
      *reinterpret_cast<uint2*>(out + column) = make_uint2(lo, hi);
      if ((lane & 15) == 0) act_scales[static_cast<size_t>(row) * groups + column / kGroup] = scale;
    }
  }
}

// ---------------------------------------------------------------------------
// Weighted combine: out[t] = bf16(sum_r w[t,r] * down[t*K + r]) in rank order.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kRowThreads) void weighted_combine_kernel(
    const float* __restrict__ down, const void* __restrict__ weights, int weights_f32, int rows,
    int top_k, int hidden, const int32_t* __restrict__ row_count,
    const float* __restrict__ shared, uint16_t* __restrict__ out) {
  const int row = blockIdx.x;
  if (row >= live_rows(row_count, rows)) return;
  float w[16];
  for (int r = 0; r < top_k; ++r) {
    const size_t index = static_cast<size_t>(row) * top_k + r;
    w[r] = weights_f32 ? static_cast<const float*>(weights)[index]
                       : bf16_to_f32(static_cast<const uint16_t*>(weights)[index]);
  }
  for (int column = threadIdx.x * 4; column < hidden; column += kRowThreads * 4) {
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int r = 0; r < top_k; ++r) {
      const float4 y = *reinterpret_cast<const float4*>(
          down + (static_cast<size_t>(row) * top_k + r) * hidden + column);
      acc.x = fmaf(w[r], y.x, acc.x);
      acc.y = fmaf(w[r], y.y, acc.y);
      acc.z = fmaf(w[r], y.z, acc.z);
      acc.w = fmaf(w[r], y.w, acc.w);
    }
    if (shared != nullptr) {
      // Dense shared expert added to the routed output, each rounded to bf16.
      const float4 s = *reinterpret_cast<const float4*>(shared + static_cast<size_t>(row) * hidden + column);
      acc.x = bf16_to_f32(f32_to_bf16(acc.x)) + bf16_to_f32(f32_to_bf16(s.x));
      acc.y = bf16_to_f32(f32_to_bf16(acc.y)) + bf16_to_f32(f32_to_bf16(s.y));
      acc.z = bf16_to_f32(f32_to_bf16(acc.z)) + bf16_to_f32(f32_to_bf16(s.z));
      acc.w = bf16_to_f32(f32_to_bf16(acc.w)) + bf16_to_f32(f32_to_bf16(s.w));
    }
    const uint32_t lo = f32_to_bf16(acc.x) | (static_cast<uint32_t>(f32_to_bf16(acc.y)) << 16);
    const uint32_t hi = f32_to_bf16(acc.z) | (static_cast<uint32_t>(f32_to_bf16(acc.w)) << 16);
    *reinterpret_cast<uint2*>(out + static_cast<size_t>(row) * hidden + column) = make_uint2(lo, hi);
  }
}

template <int KB, int RT, int MODE>
void launch_gemm(dim3 grid, hipStream_t s, const uint8_t* w, const float* ws, int n,
                 const uint8_t* a, const float* as, const int32_t* sorted_ids, int top_k,
                 const int4* items, const int32_t* num_items, int exact_routes,
                 uint16_t* out_bf16, float* out_f32) {
  hipLaunchKernelGGL((expert_gemm_kernel<KB, RT, MODE>), grid, dim3(kGemmThreads), 0, s, w, ws,
                     n, a, as, sorted_ids, top_k, items, num_items, exact_routes, out_bf16,
                     out_f32);
}

// Row tiles per wave: keep each wave's register-resident weights near 32 KiB.
constexpr int rt_for(int kb) { return kb >= 8 ? 1 : (kb >= 4 ? 2 : 4); }

template <int KB>
int dispatch_gemm(int mode, int n, dim3 items_grid, hipStream_t s, const uint8_t* w,
                  const float* ws, const uint8_t* a, const float* as, const int32_t* sorted_ids,
                  int top_k, const int4* items, const int32_t* num_items, int exact_routes,
                  uint16_t* out_bf16, float* out_f32) {
  constexpr int RT = rt_for(KB);
  constexpr int rows_per_group = kGemmWaves * RT * 16;
  D3_SUPPORTED(n % rows_per_group == 0, "expert_gemm: N=%d must be a multiple of %d for K=%d", n,
               rows_per_group, KB * kGroup);
  const dim3 grid(items_grid.x * (n / rows_per_group));
  if (mode == 0)
    launch_gemm<KB, RT, 0>(grid, s, w, ws, n, a, as, sorted_ids, top_k, items, num_items,
                           exact_routes, out_bf16, out_f32);
  else
    launch_gemm<KB, RT, 1>(grid, s, w, ws, n, a, as, sorted_ids, top_k, items, num_items,
                           exact_routes, out_bf16, out_f32);
  return D3_OK;
}

bool aligned(const void* p, uintptr_t bytes) { return (reinterpret_cast<uintptr_t>(p) % bytes) == 0; }

}  // namespace
}  // namespace d3

using namespace d3;

extern "C" int d3_expert_gemm(int32_t mode, const uint8_t* w, const float* ws, int32_t num_experts,
                              int32_t n, int32_t k, const uint8_t* a, const float* a_scales,
                              const int32_t* sorted_ids, int32_t top_k, const int32_t* items,
                              const int32_t* num_items, int32_t max_items, int32_t exact_routes,
                              uint16_t* out_bf16, float* out_f32, void* stream) {
  D3_REQUIRE(mode == 0 || mode == 1, "expert_gemm: mode must be 0 (FC1) or 1 (FC2)");
  D3_REQUIRE(w && ws && a && a_scales && sorted_ids && items && num_items,
             "expert_gemm: null pointer");
  D3_REQUIRE(mode == 0 ? out_bf16 != nullptr : out_f32 != nullptr, "expert_gemm: null output");
  D3_REQUIRE(num_experts >= 1 && n > 0 && k > 0 && n % kGroup == 0 && k % kGroup == 0,
             "expert_gemm: N=%d, K=%d must be positive multiples of 128", n, k);
  D3_REQUIRE(top_k >= 1 && max_items >= 0, "expert_gemm: bad top_k/max_items");
  D3_REQUIRE(aligned(w, 16) && aligned(a, 16), "expert_gemm: operands must be 16-byte aligned");
  D3_REQUIRE(mode == 0 ? aligned(out_bf16, 8) : aligned(out_f32, 16),
             "expert_gemm: output alignment");
  if (max_items == 0) {
    clear_error();
    return D3_OK;
  }
  hipStream_t s = as_stream(stream);
  const dim3 items_grid(max_items);
  const int4* it = reinterpret_cast<const int4*>(items);
  int status;
  switch (k / kGroup) {
#define D3_GEMM_CASE(KB)                                                                       \
  case KB:                                                                                     \
    status = dispatch_gemm<KB>(mode, n, items_grid, s, w, ws, a, a_scales, sorted_ids, top_k,  \
                               it, num_items, exact_routes, out_bf16, out_f32);                \
    break;
    D3_GEMM_CASE(2)
    D3_GEMM_CASE(4)
    D3_GEMM_CASE(6)
    D3_GEMM_CASE(8)
    D3_GEMM_CASE(12)
    D3_GEMM_CASE(16)
#undef D3_GEMM_CASE
    default:
      return set_error(D3_ERR_UNSUPPORTED, "expert_gemm: K=%d not in the compiled set", k);
  }
  if (status != D3_OK) return status;
  D3_LAUNCHED("expert_gemm");
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
  const int blocks = (rows + kRowThreads / kWave - 1) / (kRowThreads / kWave);
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
  hipLaunchKernelGGL(weighted_combine_kernel, dim3(rows), dim3(kRowThreads), 0, as_stream(stream),
                     down, weights, weights_dtype == D3_DTYPE_F32 ? 1 : 0, rows, top_k, hidden,
                     row_count, shared, out);
  D3_LAUNCHED("weighted_combine");
}
