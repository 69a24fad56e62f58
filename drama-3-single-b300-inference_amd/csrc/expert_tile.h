// Expert-GEMM building blocks shared by the standalone expert kernels
// (expert.hip) and the one-launch decode step (step.hip): MFMA operand
// fragments of the two weight layouts, the exact (bf16-widened) and FP8 MFMA
// blocks, the SwiGLU + e4m3 requantisation of one 128-column group and the
// rank-order combine.
//
// Operand layout of the 16x16x128 MFMA block (both operands): lane l holds
// row / column l % 16 and 32 contraction bytes of group g = l / 16, bytes
// 0-15 = k in [16g, 16g+16) and bytes 16-31 = k in [64+16g, 64+16g+16).
// The product is invariant under any k permutation applied to both.
#pragma once

#include "common.h"

namespace d3 {

typedef int int32x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef int int32x4 __attribute__((ext_vector_type(4)));

constexpr int kGemmWaves = 4;
constexpr int kGemmThreads = kGemmWaves * kWave;

// Row tiles per wave: keep each wave's register-resident weights near 32 KiB.
constexpr int rt_for(int kb) { return kb >= 8 ? 1 : (kb >= 4 ? 2 : 4); }
constexpr int tile_rows_for(int kb) { return kGemmWaves * rt_for(kb) * 16; }

// Raw (untyped) buffer view: loads at or past `bytes` return zeros, so lanes
// with nothing to load take an out-of-range offset instead of a branch (a
// branch around a load leaves register copies that force an early wait on
// every outstanding load).  kPolicy: cache policy bits (16 = sc1, coherent
// across the XCDs' L2s).
constexpr uint32_t kNoRow = 0x80000000u;  // past every buffer used here
struct BufferView {
  __amdgpu_buffer_rsrc_t rsrc;
  __device__ BufferView(const void* base, uint32_t bytes)
      : rsrc(__builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000)) {}
  template <int kPolicy = 0>
  __device__ int4 load16(uint32_t offset) const {
    const int32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rsrc, offset, 0, kPolicy);
    return make_int4(v[0], v[1], v[2], v[3]);
  }
  template <int kPolicy = 0>
  __device__ uint32_t load4(uint32_t offset) const {
    return static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b32(rsrc, offset, 0, kPolicy));
  }
  __device__ uint32_t load1(uint32_t offset) const {
    return static_cast<uint32_t>(static_cast<uint8_t>(__builtin_amdgcn_raw_buffer_load_b8(rsrc, offset, 0, 0)));
  }
};

// Fragment of one row in the reference layout [N, K] (row = this lane's row).
__device__ __forceinline__ int32x8 load_fragment(const uint8_t* row, int kb, int group) {
  const uint8_t* p = row + kb * kGroup + group * 16;
  const int4 lo = *reinterpret_cast<const int4*>(p);
  const int4 hi = *reinterpret_cast<const int4*>(p + 64);
  int32x8 v;
  v[0] = lo.x; v[1] = lo.y; v[2] = lo.z; v[3] = lo.w;
  v[4] = hi.x; v[5] = hi.y; v[6] = hi.z; v[7] = hi.w;
  return v;
}

// Fragment of a 16-row tile in the fragment-major layout: the tile is
// stored as [K block][half][lane][16 bytes], so each of the two loads is
// 1 KiB of contiguous memory per wave, read non-temporally (every weight
// byte is used once).
__device__ __forceinline__ int32x8 load_packed_fragment(const uint8_t* tile, int kb, int lane) {
  const int32x4* p = reinterpret_cast<const int32x4*>(tile + kb * 2048) + lane;
  const int32x4 lo = __builtin_nontemporal_load(p);
  const int32x4 hi = __builtin_nontemporal_load(p + kWave);
  int32x8 v;
  v[0] = lo[0]; v[1] = lo[1]; v[2] = lo[2]; v[3] = lo[3];
  v[4] = hi[0]; v[5] = hi[1]; v[6] = hi[2]; v[7] = hi[3];
  return v;
}

__device__ __forceinline__ floatx4 mfma_fp8(const int32x8& a, const int32x8& b) {
  const floatx4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
  // cbsz = blgp = 0 selects OCP E4M3 for both operands; zero scale operands
  // select the unscaled instruction.
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, zero, 0, 0, 0, 0, 0, 0);
}

// acc += partial * scale with one fused multiply-add per element: the
// per-K-block rescale of every expert GEMM.  Spelled out rather than left to
// the compiler's contraction, which it may skip where the add ends up in
// another basic block than the product (two roundings instead of one): the
// expert kernels agree bit for bit only with the same rounding everywhere.
__device__ __forceinline__ void scale_accumulate(floatx4& acc, const floatx4& partial, float scale) {
  acc[0] = fmaf(partial[0], scale, acc[0]);
  acc[1] = fmaf(partial[1], scale, acc[1]);
  acc[2] = fmaf(partial[2], scale, acc[2]);
  acc[3] = fmaf(partial[3], scale, acc[3]);
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

// exp(-g) as 2^(-g log2 e) on the hardware exponential, with log2 e split
// into fp32 high and low parts (Cody and Waite's argument splitting): the
// product -g * hi is formed with its exact rounding error (one fma), the low
// part's contribution added to that error, and 2^(t + t_lo) taken as
// 2^t * (1 + t_lo ln 2).  Six instructions against the library expf's
// range reduction; measured on the device against the float64 sigmoid it
// gives the same error distribution as expf over every bf16 input (at most
// two ulps of the sigmoid, d3_check_epilogue_arithmetic kind 5).  -g is
// clamped to [-88, 88], so every step stays finite (no inf * 0 in the
// correction) and the result lies in [2^-127, 2^127]: exp(-g) itself
// would overflow from -g > 88.7 on, and 1 + exp(-g) rounds to 1 from
// -g < -16.7 on.
__device__ __forceinline__ float exp_neg(float g) {
  constexpr float kLog2eHi = 1.44269502162933349609375f;  // RN(log2 e)
  constexpr float kLog2eLo = 1.925963033500011e-08f;      // RN(log2 e - kLog2eHi)
  constexpr float kLn2 = 0.693147180559945309f;
  const float x = __builtin_amdgcn_fmed3f(-g, -88.0f, 88.0f);
  const float t = x * kLog2eHi;
  const float t_lo = fmaf(x, kLog2eLo, fmaf(x, kLog2eHi, -t));
  const float e = __builtin_amdgcn_exp2f(t);
  return fmaf(e, t_lo * kLn2, e);
}

// sigmoid(g) = 1 / (1 + exp(-g)) in fp32: exp_neg and a correctly rounded
// reciprocal (recip_rn), branch-free.  Where the true sigmoid is below
// 2^-126 (g < -87.3, d = 1 + exp(-g) >= 2^126) the result is 0 or a
// subnormal below 2^-125; no fp32 form keeps it exact there (1 + expf(-g)
// overflows from g < -88.7 on, and the reference's own silu gives 0 from
// there).  The SwiGLU requantisations quantise g * sigmoid(g) * u
// (|g * sigmoid(g)| < 2^-118 there) against a group scale of at least
// 1e-10 / 448, so they give the float64 oracle's code, a zero of the same
// sign, unless |u| exceeds 2^67.  (A wave-uniform branch to the IEEE form
// for such values cost the prefill FC1 launch 10 % even untaken: it keeps
// the N values of a call from being interleaved with the code after it.)
template <int N>
__device__ __forceinline__ void sigmoid_n(const float* g, float* sig) {
#pragma unroll
  for (int i = 0; i < N; ++i) sig[i] = recip_rn(1.0f + exp_neg(g[i]));
}
__device__ __forceinline__ float sigmoid_rn(float g) {
  float sig;
  sigmoid_n<1>(&g, &sig);
  return sig;
}

// SwiGLU of bf16-rounded gate / up pairs in fp32: a = (g * sigmoid(g)) * u,
// the arithmetic of the reference's in-repo SwiGLU (kernels.py:392-394)
// without its bf16 rounding of silu(g).  Every kernel of this build that
// requantises FC1 outputs uses these functions, so they agree bit for bit.
template <int N>
__device__ __forceinline__ void swiglu_values(const float* g, const float* u, float* a) {
  float sig[N];
  sigmoid_n<N>(g, sig);
#pragma unroll
  for (int i = 0; i < N; ++i) a[i] = (g[i] * sig[i]) * u[i];
}
__device__ __forceinline__ float swiglu_value(float g, float u) { return (g * sigmoid_rn(g)) * u; }

// The reference's bf16 SwiGLU, silu_mul (kernels.py:392-394): silu(g)
// rounded to bf16, times u; the caller rounds the product to bf16 as it
// stores it.
template <int N>
__device__ __forceinline__ void silu_mul_values(const float* g, const float* u, float* a) {
  float sig[N];
  sigmoid_n<N>(g, sig);
#pragma unroll
  for (int i = 0; i < N; ++i) a[i] = bf16_to_f32(f32_to_bf16(g[i] * sig[i])) * u[i];
}

// SwiGLU + e4m3 requantisation of one 128-column group held by 16 lanes
// (8 gate and 8 up bf16 values per lane): a = swiglu_value(g, u), scale =
// max(amax, 1e-10) / 448, codes quantize_four(a, scale) (the correctly
// rounded division by the scale, the rule of moe_input.py:24-27).  Shared by the standalone
// kernel, the FC2 prologues and the fused FC1 epilogue, so all give the
// same bytes.
__device__ __forceinline__ float swiglu_quant_group(uint4 graw, uint4 uraw, uint2* codes) {
  const uint32_t gw[4] = {graw.x, graw.y, graw.z, graw.w};
  const uint32_t uw[4] = {uraw.x, uraw.y, uraw.z, uraw.w};
  float g[8], u[8], v[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    g[i] = __uint_as_float((i & 1) ? (gw[i / 2] & 0xffff0000u) : (gw[i / 2] << 16));
    u[i] = __uint_as_float((i & 1) ? (uw[i / 2] & 0xffff0000u) : (uw[i / 2] << 16));
  }
  swiglu_values<8>(g, u, v);
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
  amax = segment_max<16>(amax);
  const float scale = group_scale(amax);
  const uint32_t lo = quantize_four(v, scale);
  const uint32_t hi = quantize_four(v + 4, scale);
  *codes = make_uint2(lo, hi);
  return scale;
}

__device__ __forceinline__ float route_weight(const void* weights, int weights_f32, size_t index) {
  return weights_f32 ? static_cast<const float*>(weights)[index]
                     : bf16_to_f32(static_cast<const uint16_t*>(weights)[index]);
}

// out[token, column .. column+3] = sum_r w[token, r] * down[token*top_k + r, ...]
// with one fused multiply-add per rank in rank order (fp32), before rounding.
// kCollect: `down` was published by other workgroups (coherent loads).
template <bool kCollect = false>
__device__ __forceinline__ float4 combine4(const float* down, const void* weights, int weights_f32,
                                           int token, int top_k, int hidden, int column) {
  float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  for (int r = 0; r < top_k; ++r) {
    const float w = route_weight(weights, weights_f32, static_cast<size_t>(token) * top_k + r);
    const float* src = down + (static_cast<size_t>(token) * top_k + r) * hidden + column;
    float4 y;
    if constexpr (kCollect) {
      const uint64_t lo = collect_u64(src), hi = collect_u64(src + 2);
      y = make_float4(__uint_as_float(static_cast<uint32_t>(lo)), __uint_as_float(static_cast<uint32_t>(lo >> 32)),
                      __uint_as_float(static_cast<uint32_t>(hi)), __uint_as_float(static_cast<uint32_t>(hi >> 32)));
    } else {
      y = *reinterpret_cast<const float4*>(src);
    }
    acc.x = fmaf(w, y.x, acc.x);
    acc.y = fmaf(w, y.y, acc.y);
    acc.z = fmaf(w, y.z, acc.z);
    acc.w = fmaf(w, y.w, acc.w);
  }
  return acc;
}

// combine4 for a compile-time top_k: every route row and weight is loaded
// before the first FMA; the same rank-order chain, so the same bits.  The
// route rows are issued first and the weights' dtype is chosen once for all
// ranks: a dtype branch per rank made each weight load wait before the next
// rank's loads were issued (one memory round trip per rank).  The route
// rows are read exactly once, with non-temporal loads, so they do not evict
// from the caches what the next launches read again.
template <int kTopK>
__device__ __forceinline__ float4 combine4_fixed(const float* down, const void* weights,
                                                 int weights_f32, int token, int hidden,
                                                 int column) {
  float4 y[kTopK];
#pragma unroll
  for (int r = 0; r < kTopK; ++r) {
    const floatx4 v = __builtin_nontemporal_load(
        reinterpret_cast<const floatx4*>(down + (static_cast<size_t>(token) * kTopK + r) * hidden + column));
    y[r] = make_float4(v[0], v[1], v[2], v[3]);
  }
  float w[kTopK];
  const size_t first = static_cast<size_t>(token) * kTopK;
  if (weights_f32) {
#pragma unroll
    for (int r = 0; r < kTopK; ++r) w[r] = static_cast<const float*>(weights)[first + r];
  } else {
    uint16_t raw[kTopK];
#pragma unroll
    for (int r = 0; r < kTopK; ++r) raw[r] = static_cast<const uint16_t*>(weights)[first + r];
#pragma unroll
    for (int r = 0; r < kTopK; ++r) w[r] = bf16_to_f32(raw[r]);
  }
  float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
  for (int r = 0; r < kTopK; ++r) {
    acc.x = fmaf(w[r], y[r].x, acc.x);
    acc.y = fmaf(w[r], y[r].y, acc.y);
    acc.z = fmaf(w[r], y[r].z, acc.z);
    acc.w = fmaf(w[r], y[r].w, acc.w);
  }
  return acc;
}

__device__ __forceinline__ uint2 pack_bf16x4(float4 v) {
  const uint32_t lo = f32_to_bf16(v.x) | (static_cast<uint32_t>(f32_to_bf16(v.y)) << 16);
  const uint32_t hi = f32_to_bf16(v.z) | (static_cast<uint32_t>(f32_to_bf16(v.w)) << 16);
  return make_uint2(lo, hi);
}

}  // namespace d3
