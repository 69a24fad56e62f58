// Row-parallel pieces of the MoE front end shared by the standalone front
// kernels (front.hip) and the one-launch decode step (step.hip): top-k
// routing of one row by one wavefront, and per-128 FP8 quantisation of one
// row by the four waves of a workgroup.
#pragma once

#include <math.h>

#include "common.h"

namespace d3 {

constexpr int kFrontThreads = 256;  // 4 waves

// ---------------------------------------------------------------------------
// Routing: one wave per row, NPL logits per lane (E <= 64 * NPL).
// ---------------------------------------------------------------------------
template <bool kF32>
__device__ __forceinline__ float load_logit(const void* row, int column) {
  if constexpr (kF32) return static_cast<const float*>(row)[column];
  return bf16_to_f32(static_cast<const uint16_t*>(row)[column]);
}

// route_kernel's ranking key (kernels.py:364-368): the order-preserving
// unsigned image of the fp32 bits, truncated to its bf16 half, with
// 65535 - column below it so equal values rank the lower expert first.
__device__ __forceinline__ uint32_t route_key(float value, int column) {
  const uint32_t bits = __float_as_uint(value);
  const uint32_t ordered = bits ^ ((bits & 0x80000000u) ? 0xffffffffu : 0x80000000u);
  return (ordered & 0xffff0000u) | (65535u - static_cast<uint32_t>(column));
}

// route_key from the logit's fp32 bits (a bf16 logit: its bits in the high
// half) and the tie-break field tie = 65535 - column.
__device__ __forceinline__ uint32_t key_of_bits(uint32_t bits, uint32_t tie) {
  const uint32_t ordered = bits ^ ((bits & 0x80000000u) ? 0xffffffffu : 0x80000000u);
  return (ordered & 0xffff0000u) | tie;
}

// One row's logits, NPL per lane (column lane + 64 j; -inf past E).
template <int NPL>
struct RouteLogits {
  float values[NPL];
};

template <int NPL, bool kF32>
__device__ __forceinline__ void load_route_logits(const char* base, int num_experts,
                                                  RouteLogits<NPL>& logits) {
  const int lane = lane_id();
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    // Lanes past E load the last column and discard it: no branch around
    // the load, so all NPL loads are in flight before the first wait.
    const int column = lane + j * kWave;
    const float v = load_logit<kF32>(base, column < num_experts ? column : num_experts - 1);
    logits.values[j] = column < num_experts ? v : -INFINITY;
  }
}

// Top-k of one row (one wave) from its loaded logits (E <= 64 * NPL): lane
// k < top_k gets the rank-k expert and its normalised weight (fp32, before
// any rounding to the stored dtype); other lanes get -1 and 0.
struct RouteChoice {
  int expert;
  float weight;
};

template <int NPL>
__device__ __forceinline__ RouteChoice route_top_k(const RouteLogits<NPL>& logits, int num_experts,
                                                   int top_k) {
  const int lane = lane_id();
  float values[NPL];
  uint32_t keys[NPL];
  float row_max = -INFINITY;
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    const int column = lane + j * kWave;
    values[j] = logits.values[j];
    if (column < num_experts) {
      keys[j] = route_key(values[j], column);
      row_max = fmaxf(row_max, values[j]);
    } else {
      keys[j] = 0u;  // below every valid key (65535 - column > 0)
    }
  }
  row_max = segment_max<kWave>(row_max);
  float denominator = 0.0f;
#pragma unroll
  for (int j = 0; j < NPL; ++j) denominator += expf(values[j] - row_max);
  denominator = segment_sum<kWave>(denominator);

  // Top-k by repeated wave arg-max over unique keys; lane k keeps rank k and
  // the winner's logit (read from the owning lane, not reloaded).
  int selected = -1;
  float selected_value = 0.0f;
  for (int k = 0; k < top_k; ++k) {
    uint32_t best = 0u;
#pragma unroll
    for (int j = 0; j < NPL; ++j) best = keys[j] > best ? keys[j] : best;
    best = wave_max_u32(best);
    const int column = 65535 - static_cast<int>(best & 0xffffu);  // uniform
    float mine = values[0];
#pragma unroll
    for (int j = 1; j < NPL; ++j) mine = column / kWave == j ? values[j] : mine;
    const float value =
        __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mine), column % kWave));
#pragma unroll
    for (int j = 0; j < NPL; ++j) keys[j] = keys[j] == best ? 0u : keys[j];
    if (lane == k) {
      selected = column;
      selected_value = value;
    }
  }
  float probability = 0.0f;
  if (lane < top_k) probability = expf(selected_value - row_max) / denominator;
  const float total = segment_sum<kWave>(probability);
  return {selected, lane < top_k ? probability / total : 0.0f};
}

// The weight as read back from the stored dtype (bf16 rounding or fp32).
__device__ __forceinline__ float stored_weight(float weight, int weights_f32) {
  return weights_f32 ? weight : bf16_to_f32(f32_to_bf16(weight));
}

// Routes one row (one wave) from its loaded logits: top-k ids into
// ids[out_row * top_k + rank], weights likewise.
// kPublish: ids and weights are read by other workgroups (coherent stores).
template <int NPL, bool kPublish = false>
__device__ __forceinline__ void route_logits(const RouteLogits<NPL>& logits, int num_experts,
                                             int top_k, int64_t out_row, int32_t* ids32,
                                             int64_t* ids64, void* weights, int weights_f32) {
  const int lane = lane_id();
  const RouteChoice choice = route_top_k<NPL>(logits, num_experts, top_k);
  if (lane < top_k) {
    const int64_t out = out_row * top_k + lane;
    const int selected = choice.expert;
    const float weight = choice.weight;
    if (ids32 != nullptr) {
      if constexpr (kPublish)
        publish_u32(ids32 + out, static_cast<uint32_t>(selected));
      else
        ids32[out] = selected;
    }
    if (ids64 != nullptr) ids64[out] = selected;
    if constexpr (kPublish) {
      if (weights_f32)
        publish_u32(static_cast<float*>(weights) + out, __float_as_uint(weight));
      else
        publish_u16(static_cast<uint16_t*>(weights) + out, f32_to_bf16(weight));
    } else if (weights_f32) {
      static_cast<float*>(weights)[out] = weight;
    } else {
      static_cast<uint16_t*>(weights)[out] = f32_to_bf16(weight);
    }
  }
}

// Routes the row at `base`: load_route_logits + route_logits.
template <int NPL, bool kF32, bool kPublish = false>
__device__ __forceinline__ void route_row(const char* base, int num_experts, int top_k,
                                          int64_t out_row, int32_t* ids32, int64_t* ids64,
                                          void* weights, int weights_f32) {
  RouteLogits<NPL> logits;
  load_route_logits<NPL, kF32>(base, num_experts, logits);
  route_logits<NPL, kPublish>(logits, num_experts, top_k, out_row, ids32, ids64, weights,
                              weights_f32);
}

// ---------------------------------------------------------------------------
// Quantisation: one workgroup per row, its 4 waves splitting the row into
// 512-element chunks (8 elements per lane, 16 lanes per 128-group).
// ---------------------------------------------------------------------------
constexpr int kRowWaves = kFrontThreads / kWave;
constexpr int kMaxRowChunks = 8;  // rows up to 8 * 512 = 4096 elements
constexpr int kPartChunks = kMaxRowChunks / kRowWaves;
constexpr int kChunk = 8 * kWave;

// Chunks part, part + 4, ... of one row, loaded before any arithmetic so the
// row costs one memory latency.
struct RowPart {
  uint4 raw[kPartChunks];
};

__device__ __forceinline__ void load_row_part(const uint16_t* in, int width, int part,
                                              RowPart& row) {
  const int lane = lane_id();
#pragma unroll
  for (int i = 0; i < kPartChunks; ++i) {
    const int column = (part + i * kRowWaves) * kChunk + lane * 8;
    row.raw[i] = make_uint4(0u, 0u, 0u, 0u);
    if (column < width) row.raw[i] = *reinterpret_cast<const uint4*>(in + column);
  }
}

// Quantises the chunks loaded by load_row_part: q bytes and per-128 scales
// at scales[group * scale_stride].  kPublish: read by other workgroups of
// the same launch (coherent stores).
template <bool kPublish = false>
__device__ __forceinline__ void quantize_row_part(const RowPart& row, int width, int part,
                                                  uint8_t* out, float* scales,
                                                  int64_t scale_stride) {
  const int lane = lane_id();
  const uint4* raw = row.raw;
#pragma unroll
  for (int i = 0; i < kPartChunks; ++i) {
    const int column = (part + i * kRowWaves) * kChunk + lane * 8;
    if ((part + i * kRowWaves) * kChunk >= width) break;  // uniform
    const bool inside = column < width;  // whole 16-lane groups agree
    const uint32_t words[4] = {raw[i].x, raw[i].y, raw[i].z, raw[i].w};
    float v[8];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(words[i] << 16);
      v[2 * i + 1] = __uint_as_float(words[i] & 0xffff0000u);
      amax = fmaxf(amax, fmaxf(fabsf(v[2 * i]), fabsf(v[2 * i + 1])));
    }
    amax = segment_max<16>(amax);
    const float scale = group_scale(amax);
    const uint32_t lo = quantize_four(v, scale);
    const uint32_t hi = quantize_four(v + 4, scale);
    if (inside) {
      float* scale_out = scales + static_cast<int64_t>(column / kGroup) * scale_stride;
      if constexpr (kPublish) {
        publish_u64(out + column, (static_cast<uint64_t>(hi) << 32) | lo);
        if ((lane & 15) == 0) publish_u32(scale_out, __float_as_uint(scale));
      } else {
        *reinterpret_cast<uint2*>(out + column) = make_uint2(lo, hi);
        if ((lane & 15) == 0) *scale_out = scale;
      }
    }
  }
}

}  // namespace d3
