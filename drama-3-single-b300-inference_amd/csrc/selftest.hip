// Device self-checks of the arithmetic every quantiser relies on.
//
// The quantisers (quantize_four in common.h: the MoE input, FC1 staging and
// the SwiGLU requantisation) convert with v_cvt_pk_fp8_f32, which rounds to
// nearest even into OCP e4m3, after clamping to [-448, 448].  Parity with
// the reference's bytes needs that conversion to give the software
// f32_to_e4m3 byte (the rule torch's float8_e4m3fn cast implements) for
// every clamped fp32 input and in every byte position of the packed word.
// This kernel compares the two over a range of fp32 bit patterns.
//
// The quantisers and the SwiGLU requantisation also take shortcuts that
// must give the IEEE results: pack_bf16x2 (hardware bf16 rounding),
// recip_rn (hardware reciprocal + one Newton-Raphson step) inside
// sigmoid_rn and for the reciprocal of every group scale, exp_neg (the
// hardware exponential of a split product) inside sigmoid_rn, div_rn
// (reciprocal of the scale + one residual correction) inside quantize_four,
// and group_scale's division by 448 (a constant reciprocal + one residual
// correction).
// check_arithmetic_kernel compares each with its IEEE / software form over a
// range of fp32 bit patterns; the sigmoid, which is not correctly rounded,
// with the float64 sigmoid rounded to fp32, within a stated number of ulps.
#include "common.h"
#include "expert_tile.h"
#include "status.h"

namespace d3 {
namespace {

constexpr int kCheckThreads = 256;

__device__ __forceinline__ float clamp448(float v) { return fminf(fmaxf(v, -448.0f), 448.0f); }

// Mismatch counting shared by the checks: per wave, per workgroup, then one
// atomic add / min into result.
__device__ void report_mismatches(uint32_t mismatches, uint32_t first_bad, uint32_t* result) {
  __shared__ uint32_t bad_count[kCheckThreads / kWave];
  __shared__ uint32_t bad_first[kCheckThreads / kWave];
  const uint32_t wave_count = wave_reduce<SumU32>(mismatches);
  uint32_t wave_first = first_bad;
#pragma unroll
  for (int offset = 32; offset >= 1; offset >>= 1)
    wave_first = min(wave_first, static_cast<uint32_t>(__shfl_xor(static_cast<int>(wave_first), offset)));
  const int wave = threadIdx.x / kWave;
  if (lane_id() == 0) {
    bad_count[wave] = wave_count;
    bad_first[wave] = wave_first;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t total = 0, least = 0xffffffffu;
#pragma unroll
    for (int w = 0; w < kCheckThreads / kWave; ++w) {
      total += bad_count[w];
      least = min(least, bad_first[w]);
    }
    if (total) {
      atomicAdd(&result[0], total);
      atomicMin(&result[1], least);
    }
  }
}

// Each thread takes groups of four consecutive patterns; each group is
// converted four times, rotated so that every pattern lands in every byte
// position of the packed word once.
__global__ __launch_bounds__(kCheckThreads) void check_e4m3_kernel(uint64_t first, uint64_t groups,
                                                                   uint32_t* __restrict__ result) {
  uint32_t mismatches = 0;
  uint32_t first_bad = 0xffffffffu;
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kCheckThreads;
  for (uint64_t g = static_cast<uint64_t>(blockIdx.x) * kCheckThreads + threadIdx.x; g < groups; g += stride) {
    const uint32_t p0 = static_cast<uint32_t>(first + 4 * g);
    float c[4];
    uint32_t want[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      c[i] = clamp448(__uint_as_float(p0 + i));
      want[i] = f32_to_e4m3(c[i]) & 0xffu;
    }
#pragma unroll
    for (int rot = 0; rot < 4; ++rot) {
      // byte position j holds pattern (j + rot) % 4
      int word = __builtin_amdgcn_cvt_pk_fp8_f32(c[rot & 3], c[(rot + 1) & 3], 0, false);
      word = __builtin_amdgcn_cvt_pk_fp8_f32(c[(rot + 2) & 3], c[(rot + 3) & 3], word, true);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int i = (j + rot) & 3;
        const uint32_t got = (static_cast<uint32_t>(word) >> (8 * j)) & 0xffu;
        if (got != want[i]) {
          ++mismatches;
          first_bad = min(first_bad, p0 + i);
        }
      }
    }
  }
  report_mismatches(mismatches, first_bad, result);
}

// kind 0: pack_bf16x2 against f32_to_bf16 (NaN patterns skipped), pattern
//   p in the low half next to p ^ 0x80000000 in the high half and the
//   other way round;
// kind 1: recip_rn(d) against 1.0f / d, d = pattern (inside [2^-43, 2^126));
// kind 2: the code and the quotient of div_rn(v, s, 1.0f / s) against
//   v / s for v = +-pattern, s = scale (quotients from 2^-12 up compared
//   bit for bit, smaller ones by their e4m3 code after the clamp);
// kind 3: sigmoid_rn(g) against RN(1 / (1 + exp(-g))) evaluated in float64,
//   g = pattern (NaN patterns skipped): more than `scale` ulps apart where
//   the reference is a normal number, or not below 2^-125 where it is not;
// kind 4: group_scale(m) against fmaxf(m, 1e-10f) / 448.0f, m = pattern
//   (non-negative patterns up to +inf);
// kind 5: kind 3 for the bf16 inputs only, g = pattern << 16 (patterns
//   below 2^16), the values every SwiGLU of this library feeds it.
__global__ __launch_bounds__(kCheckThreads) void check_arithmetic_kernel(int kind, uint64_t first, uint64_t count,
                                                                         float scale, uint32_t* __restrict__ result) {
  uint32_t mismatches = 0;
  uint32_t first_bad = 0xffffffffu;
  const float inv = 1.0f / scale;
  const uint32_t shift = kind == 5 ? 16 : 0;
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kCheckThreads;
  for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kCheckThreads + threadIdx.x; i < count; i += stride) {
    const uint32_t p = static_cast<uint32_t>(first + i) << shift;
    const float x = __uint_as_float(p);
    bool bad = false;
    if (kind == 0) {
      if ((p & 0x7fffffffu) <= 0x7f800000u) {
        const float y = __uint_as_float(p ^ 0x80000000u);
        const uint32_t a = pack_bf16x2(x, y), b = pack_bf16x2(y, x);
        const uint32_t want_x = f32_to_bf16(x), want_y = f32_to_bf16(y);
        bad = (a & 0xffffu) != want_x || (a >> 16) != want_y || (b & 0xffffu) != want_y || (b >> 16) != want_x;
      }
    } else if (kind == 1) {
      bad = __float_as_uint(recip_rn(x)) != __float_as_uint(1.0f / x);
    } else if (kind == 2) {
#pragma unroll
      for (int sign = 0; sign < 2; ++sign) {
        const float v = sign ? -x : x;
        const float want = v / scale, got = div_rn(v, scale, inv);
        const float cw = fminf(fmaxf(want, -448.0f), 448.0f), cg = fminf(fmaxf(got, -448.0f), 448.0f);
        if (fabsf(want) >= 0x1p-12f) bad |= __float_as_uint(got) != __float_as_uint(want);
        bad |= f32_to_e4m3(cw) != f32_to_e4m3(cg);
      }
    } else if (kind == 3 || kind == 5) {
      if ((p & 0x7fffffffu) <= 0x7f800000u) {
        const float want = static_cast<float>(1.0 / (1.0 + exp(-static_cast<double>(x))));
        const float got = sigmoid_rn(x);
        // both lie in [0, 1]: the bit patterns order the values
        const uint32_t a = __float_as_uint(got), b = __float_as_uint(want);
        bad = want >= 0x1p-126f ? static_cast<float>(a > b ? a - b : b - a) > scale : !(got < 0x1p-125f);
      }
    } else {
      if (p <= 0x7f800000u) bad = __float_as_uint(group_scale(x)) != __float_as_uint(fmaxf(x, 1e-10f) / 448.0f);
    }
    if (bad) {
      ++mismatches;
      first_bad = min(first_bad, p);
    }
  }
  report_mismatches(mismatches, first_bad, result);
}

}  // namespace
}  // namespace d3

using namespace d3;

extern "C" int d3_check_e4m3_conversion(uint64_t first, uint64_t count, uint32_t* result,
                                        void* stream) {
  D3_REQUIRE(result != nullptr, "check_e4m3_conversion: null result");
  D3_REQUIRE(first % 4 == 0 && count % 4 == 0 && first + count <= (uint64_t{1} << 32),
             "check_e4m3_conversion: the range must be whole groups of four patterns inside 2^32");
  if (count == 0) {
    clear_error();
    return D3_OK;
  }
  const uint64_t groups = count / 4;
  const int blocks = static_cast<int>(std::min<uint64_t>((groups + kCheckThreads - 1) / kCheckThreads, 8192));
  hipLaunchKernelGGL(check_e4m3_kernel, dim3(blocks), dim3(kCheckThreads), 0, as_stream(stream), first,
                     groups, result);
  D3_LAUNCHED("check_e4m3_conversion");
}

extern "C" int d3_check_epilogue_arithmetic(int32_t kind, uint64_t first, uint64_t count, float scale,
                                            uint32_t* result, void* stream) {
  D3_REQUIRE(result != nullptr, "check_epilogue_arithmetic: null result");
  D3_REQUIRE(kind >= 0 && kind <= 5, "check_epilogue_arithmetic: kind must be 0-5");
  D3_REQUIRE(first + count <= (uint64_t{1} << 32), "check_epilogue_arithmetic: range beyond 2^32");
  D3_REQUIRE(kind != 1 || (first >= 0x2a000000u && first + count <= 0x7e800000u),
             "check_epilogue_arithmetic: reciprocal inputs must lie in [2^-43, 2^126)");
  D3_REQUIRE(kind != 2 || (scale > 0.0f && first + count <= 0x7f800000u),
             "check_epilogue_arithmetic: division needs a positive scale and finite patterns");
  D3_REQUIRE(kind != 5 || first + count <= (uint64_t{1} << 16),
             "check_epilogue_arithmetic: bf16 sigmoid inputs are patterns below 2^16");
  D3_REQUIRE((kind != 3 && kind != 5) || scale >= 0.0f,
             "check_epilogue_arithmetic: the sigmoid's ulp bound must be non-negative");
  if (count == 0) {
    clear_error();
    return D3_OK;
  }
  const int blocks = static_cast<int>(std::min<uint64_t>((count + kCheckThreads - 1) / kCheckThreads, 8192));
  hipLaunchKernelGGL(check_arithmetic_kernel, dim3(blocks), dim3(kCheckThreads), 0, as_stream(stream), kind,
                     first, count, scale, result);
  D3_LAUNCHED("check_epilogue_arithmetic");
}
