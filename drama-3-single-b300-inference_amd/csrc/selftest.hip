// Device self-check of the e4m3 conversion every quantiser relies on.
//
// The quantisers (quantize_four in common.h: the MoE input, FC1 staging and
// the SwiGLU requantisation) convert with v_cvt_pk_fp8_f32, which rounds to
// nearest even into OCP e4m3, after clamping to [-448, 448].  Parity with
// the reference's bytes needs that conversion to give the software
// f32_to_e4m3 byte (the rule torch's float8_e4m3fn cast implements) for
// every clamped fp32 input and in every byte position of the packed word.
// This kernel compares the two over a range of fp32 bit patterns.
#include "common.h"
#include "status.h"

namespace d3 {
namespace {

constexpr int kCheckThreads = 256;

__device__ __forceinline__ float clamp448(float v) { return fminf(fmaxf(v, -448.0f), 448.0f); }

// Each thread takes groups of four consecutive patterns; each group is
// converted four times, rotated so that every pattern lands in every byte
// position of the packed word once.
__global__ __launch_bounds__(kCheckThreads) void check_e4m3_kernel(uint64_t first, uint64_t groups,
                                                                   uint32_t* __restrict__ result) {
  __shared__ uint32_t bad_count[kCheckThreads / kWave];
  __shared__ uint32_t bad_first[kCheckThreads / kWave];
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
  // per wave, then per workgroup, then one atomic each
  const uint32_t wave_count = wave_reduce<SumU32>(mismatches);
  uint32_t wave_first = first_bad;
#pragma unroll
  for (int offset = 32; offset >= 1; offset >>= 1) wave_first = min(wave_first, static_cast<uint32_t>(__shfl_xor(static_cast<int>(wave_first), offset)));
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
