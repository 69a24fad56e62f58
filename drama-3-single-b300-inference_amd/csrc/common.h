// Device helpers shared by the MoE kernels (gfx950, wave64).
//
// Numeric conventions follow the reference (src/drama3/kernels.py,
// moe_input.py): bf16 activations, OCP FP8 e4m3fn ("fn": no infinities,
// max finite 448) weights and quantised activations, fp32 block scales.
// Conversions are exact bit manipulations so that quantised bytes match a
// CPU restatement bit for bit.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace d3 {

constexpr int kWave = 64;
constexpr int kGroup = 128;  // FP8 block size along every contracted dimension

// ---------------------------------------------------------------------------
// bf16
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// Round to nearest even; NaN stays a quiet NaN.  Written as a select: an
// early return for NaN compiles to a divergent branch per value.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  const uint32_t b = __float_as_uint(f);
  const uint32_t rounded = (b + 0x7fffu + ((b >> 16) & 1u)) >> 16;
  const uint32_t quiet = (b >> 16) | 0x40u;
  return static_cast<uint16_t>((b & 0x7fffffffu) > 0x7f800000u ? quiet : rounded);
}

// Two values rounded to bf16 by v_cvt_pk_bf16_f32 (round to nearest even),
// `lo` in the low half.  d3_check_epilogue_arithmetic (selftest.hip) shows
// it gives f32_to_bf16's bits for every non-NaN fp32 input in both halves.
typedef __bf16 bf16x2_hw __attribute__((ext_vector_type(2)));
typedef float floatx2_hw __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const floatx2_hw v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_hw));
}
// The two halves of a pack_bf16x2 word as fp32.
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// ---------------------------------------------------------------------------
// OCP e4m3fn
// ---------------------------------------------------------------------------
// float -> e4m3fn code, round to nearest even.  Magnitudes >= 464 and NaN
// give the NaN code 0x7f (torch's float8_e4m3fn conversion); the MoE path
// clamps to +-448 first so it never produces NaN.
__device__ __forceinline__ uint32_t f32_to_e4m3(float f) {
  const uint32_t b = __float_as_uint(f);
  const uint32_t sign = (b >> 24) & 0x80u;
  const uint32_t mag = b & 0x7fffffffu;
  uint32_t code;
  if (mag >= 0x43e80000u) {
    code = 0x7fu;
  } else if (mag < 0x3c800000u) {
    // Below the smallest normal 2^-6: value = m * 2^-9, m in [0, 8].
    // Scaling by 512 is exact; rint rounds half to even.
    code = static_cast<uint32_t>(__builtin_rintf(__uint_as_float(mag) * 512.0f));
  } else {
    uint32_t shifted = (((mag >> 23) - 120u) << 3) | ((mag >> 20) & 7u);
    const uint32_t rest = mag & 0xfffffu;
    shifted += (rest > 0x80000u) || (rest == 0x80000u && (shifted & 1u));
    code = shifted;
  }
  return code | sign;
}

__device__ __forceinline__ float e4m3_to_f32(uint32_t code) {
  const uint32_t sign = (code & 0x80u) << 24;
  const uint32_t exponent = (code >> 3) & 0xfu;
  const uint32_t mantissa = code & 7u;
  float mag;
  if (exponent == 0) {
    mag = static_cast<float>(mantissa) * (1.0f / 512.0f);
  } else if (exponent == 15 && mantissa == 7) {
    mag = __uint_as_float(0x7fc00000u);
  } else {
    mag = __uint_as_float(((exponent + 120u) << 23) | (mantissa << 20));
  }
  return __uint_as_float(__float_as_uint(mag) | sign);
}

// 1 / d rounded to nearest even for d in [2^-43, 2^126): the hardware
// reciprocal (v_rcp_f32, within one ulp) and one Newton-Raphson correction
// with the exact residual 1 - d * y (Markstein's reciprocal step).
// d3_check_epilogue_arithmetic (selftest.hip) compares it with the IEEE
// division 1.0f / d for every fp32 d in that range on the device.
__device__ __forceinline__ float recip_rn(float d) {
  const float y = __builtin_amdgcn_rcpf(d);
  const float e = fmaf(-d, y, 1.0f);
  return fmaf(e, y, y);
}

// Per-128 group quantisation rule of the reference (moe_input.py:24-27):
// scale = max(amax, 1e-10) / 448 and q = e4m3(clamp(x / scale, -448, 448)),
// with IEEE fp32 division.  The division by 448 is Markstein's division by
// a constant: q0 = m * RN(1/448), the exact residual m - 448 q0, one
// correction; three instructions instead of the general division sequence.
// m = +inf gives +inf, as the IEEE division does.
// d3_check_epilogue_arithmetic compares it with the IEEE form for every
// non-negative fp32 amax (+inf included).
__device__ __forceinline__ float group_scale(float amax) {
  constexpr float kInv448 = 1.0f / 448.0f;
  const float m = fmaxf(amax, 1e-10f);
  const float q0 = m * kInv448;
  const float r = fmaf(-q0, 448.0f, m);
  const float q = fmaf(r, kInv448, q0);
  return m == __builtin_huge_valf() ? m : q;
}

// 1.0f / scale for a group scale: every finite group scale lies in
// [RN(1e-10 / 448), FLT_MAX / 448], inside recip_rn's range; +inf gives 0.
__device__ __forceinline__ float scale_reciprocal(float scale) {
  return scale == __builtin_huge_valf() ? 0.0f : recip_rn(scale);
}

__device__ __forceinline__ uint32_t quantize_one(float x, float scale) {
  const float v = fminf(fmaxf(x / scale, -448.0f), 448.0f);
  return f32_to_e4m3(v);
}

// x / s rounded to nearest even, given inv = 1.0f / s (IEEE): q0 = x * inv,
// then one correction with the exact residual x - q0 * s (Markstein's
// division step: with inv the correctly rounded reciprocal, q0 lies within
// one ulp of x / s, the residual is exact and q0 + r * inv rounds to the
// correctly rounded quotient).  copysign keeps the sign of a zero quotient
// (x = -0).  Equal to the IEEE division for every quotient in the fp32
// normal range; below it (|x / s| < 2^-126, an e4m3 zero either way) it may
// differ in the last place.  d3_check_epilogue_arithmetic (selftest.hip)
// compares the quantised codes with quantize_one's on the device.
__device__ __forceinline__ float div_rn(float x, float s, float inv) {
  const float q0 = x * inv;
  const float r = fmaf(-q0, s, x);
  return copysignf(fmaf(r, inv, q0), x);
}

// quantize_one of four values, packed little-endian (v[0] in the low byte),
// for a scale from group_scale.  The division is div_rn with the reciprocal
// from scale_reciprocal (one per call: callers that quantise several words
// with one scale share it after inlining).  The conversion is
// v_cvt_pk_fp8_f32 (round to nearest even into OCP e4m3), which gives
// f32_to_e4m3's byte for every input in [-448, 448] in every byte position:
// d3_check_e4m3_conversion (selftest.hip) compares the two over all 2^32
// fp32 bit patterns after the clamp.
__device__ __forceinline__ uint32_t quantize_four(const float* v, float scale) {
  const float inv = scale_reciprocal(scale);
  float c[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) c[i] = fminf(fmaxf(div_rn(v[i], scale, inv), -448.0f), 448.0f);
  int word = __builtin_amdgcn_cvt_pk_fp8_f32(c[0], c[1], 0, false);
  word = __builtin_amdgcn_cvt_pk_fp8_f32(c[2], c[3], word, true);
  return static_cast<uint32_t>(word);
}

// ---------------------------------------------------------------------------
// wave64 reductions on DPP lane moves (VALU operand modifiers, no LDS
// round trip): quad_perm [1,0,3,2] and [2,3,0,1], row_half_mirror and
// row_mirror reduce each 16-lane row so that every lane of the row holds the
// result; row_bcast:15 / row_bcast:31 fold the four rows into lane 63, which
// readlane broadcasts.  Lanes not written by a DPP move receive the
// operation's identity.
// ---------------------------------------------------------------------------
constexpr int kDppQuad1032 = 0xb1;
constexpr int kDppQuad2301 = 0x4e;
constexpr int kDppRowMirror = 0x140;
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowBcast15 = 0x142;
constexpr int kDppRowBcast31 = 0x143;

template <int kCtrl, int kRowMask = 0xf>
__device__ __forceinline__ uint32_t dpp_move(uint32_t v, uint32_t identity) {
  return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(
      static_cast<int>(identity), static_cast<int>(v), kCtrl, kRowMask, 0xf, false));
}

struct MaxF32 {
  static constexpr uint32_t kIdentity = 0xff800000u;  // -inf
  __device__ static uint32_t apply(uint32_t a, uint32_t b) {
    return __float_as_uint(fmaxf(__uint_as_float(a), __uint_as_float(b)));
  }
};
struct SumF32 {
  static constexpr uint32_t kIdentity = 0u;  // +0
  __device__ static uint32_t apply(uint32_t a, uint32_t b) {
    return __float_as_uint(__uint_as_float(a) + __uint_as_float(b));
  }
};
struct MaxU32 {
  static constexpr uint32_t kIdentity = 0u;
  __device__ static uint32_t apply(uint32_t a, uint32_t b) { return a > b ? a : b; }
};
struct SumU32 {
  static constexpr uint32_t kIdentity = 0u;
  __device__ static uint32_t apply(uint32_t a, uint32_t b) { return a + b; }
};

// Every lane of each 16-lane row gets the reduction over its row.
template <class Op>
__device__ __forceinline__ uint32_t row_reduce(uint32_t v) {
  v = Op::apply(v, dpp_move<kDppQuad1032>(v, Op::kIdentity));
  v = Op::apply(v, dpp_move<kDppQuad2301>(v, Op::kIdentity));
  v = Op::apply(v, dpp_move<kDppRowHalfMirror>(v, Op::kIdentity));
  v = Op::apply(v, dpp_move<kDppRowMirror>(v, Op::kIdentity));
  return v;
}

// Every lane gets the reduction over the wave (a wave-uniform value).
template <class Op>
__device__ __forceinline__ uint32_t wave_reduce(uint32_t v) {
  v = row_reduce<Op>(v);
  v = Op::apply(v, dpp_move<kDppRowBcast15, 0xa>(v, Op::kIdentity));
  v = Op::apply(v, dpp_move<kDppRowBcast31, 0xc>(v, Op::kIdentity));
  return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), kWave - 1));
}

// Reductions over aligned segments of WIDTH lanes (16 or 64); every lane of
// a segment receives the segment's result.
template <int WIDTH>
__device__ __forceinline__ float segment_max(float v) {
  static_assert(WIDTH == 16 || WIDTH == kWave, "segments of 16 or 64 lanes");
  if constexpr (WIDTH == 16) return __uint_as_float(row_reduce<MaxF32>(__float_as_uint(v)));
  return __uint_as_float(wave_reduce<MaxF32>(__float_as_uint(v)));
}

template <int WIDTH>
__device__ __forceinline__ float segment_sum(float v) {
  static_assert(WIDTH == 16 || WIDTH == kWave, "segments of 16 or 64 lanes");
  if constexpr (WIDTH == 16) return __uint_as_float(row_reduce<SumF32>(__float_as_uint(v)));
  return __uint_as_float(wave_reduce<SumF32>(__float_as_uint(v)));
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) { return wave_reduce<MaxU32>(v); }

__device__ __forceinline__ int lane_id() { return static_cast<int>(threadIdx.x) & (kWave - 1); }

__device__ __forceinline__ uint64_t lanemask_lt() {
  const int lane = lane_id();
  return lane == 0 ? 0ull : (~0ull >> (64 - lane));
}

// ---------------------------------------------------------------------------
// Cross-workgroup hand-off without cache-wide fences.
// On gfx950 every XCD has its own L2; an agent-scope fence writes back and
// invalidates that whole L2.  Data handed from one workgroup to another is
// instead stored and loaded with agent-scope relaxed atomics (write-through /
// coherent accesses, sc1), the stores are waited for before a workgroup
// barrier, and only then is the hand-off ticket taken with an agent-scope
// atomic add.  The reader, having seen the final ticket, loads the data with
// coherent loads.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void publish_u64(void* p, uint64_t v) {
  __hip_atomic_store(static_cast<uint64_t*>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void publish_u32(void* p, uint32_t v) {
  __hip_atomic_store(static_cast<uint32_t*>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void publish_u16(void* p, uint16_t v) {
  __hip_atomic_store(static_cast<uint16_t*>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t collect_u64(const void* p) {
  return __hip_atomic_load(static_cast<const uint64_t*>(p), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t collect_u32(const void* p) {
  return __hip_atomic_load(static_cast<const uint32_t*>(p), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}
// Every store of the calling thread has completed (reached the coherent
// level for published stores) before it proceeds.
__device__ __forceinline__ void wait_stores() { __builtin_amdgcn_s_waitcnt(0); }
// Workgroup barrier ordering LDS only: global loads and stores issued before
// it stay in flight (__syncthreads also waits for every outstanding global
// access).  For kernels whose threads exchange data through LDS alone.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}
__device__ __forceinline__ int take_ticket(int32_t* ticket) {
  return __hip_atomic_fetch_add(ticket, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void reset_ticket(int32_t* ticket) {
  __hip_atomic_store(ticket, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Row count visible to graph-captured kernels: a device scalar when given,
// otherwise the host capacity.
__device__ __forceinline__ int live_rows(const int32_t* count, int capacity) {
  if (count == nullptr) return capacity;
  const int n = *count;
  return n < capacity ? (n < 0 ? 0 : n) : capacity;
}

}  // namespace d3
