// Row-wise epilogues around the routed MoE output: gated shared-expert
// combine, combine + residual + RMSNorm (direct and inverse-row), residual
// add + RMSNorm, and the bf16 SwiGLU of the shared expert input.
//
// One workgroup (256 threads) per row; 4 contiguous bf16 per thread access
// (8-byte loads).  Rounding points follow the reference kernels exactly; the
// single-rounding bf16 FMA is evaluated as an exact fp64 fma followed by one
// round-to-nearest-even to bf16.
#include <math.h>

#include "common.h"
#include "expert_tile.h"
#include "front_rows.h"
#include "status.h"

namespace d3 {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxPerThread = 32;  // width <= 8192

__device__ __forceinline__ void load4(const uint16_t* p, float v[4]) {
  const uint2 raw = *reinterpret_cast<const uint2*>(p);
  v[0] = __uint_as_float(raw.x << 16);
  v[1] = __uint_as_float(raw.x & 0xffff0000u);
  v[2] = __uint_as_float(raw.y << 16);
  v[3] = __uint_as_float(raw.y & 0xffff0000u);
}

__device__ __forceinline__ void store4(uint16_t* p, const float v[4]) {
  const uint32_t lo = f32_to_bf16(v[0]) | (static_cast<uint32_t>(f32_to_bf16(v[1])) << 16);
  const uint32_t hi = f32_to_bf16(v[2]) | (static_cast<uint32_t>(f32_to_bf16(v[3])) << 16);
  *reinterpret_cast<uint2*>(p) = make_uint2(lo, hi);
}

__device__ __forceinline__ float round_bf16(float x) { return bf16_to_f32(f32_to_bf16(x)); }

// bf16(sigmoid(fp32 gate)) (kernels.py:434-438), of the gate's bf16 bits.
__device__ __forceinline__ float gate_sigmoid_bf16(uint16_t bits) {
  const float g = bf16_to_f32(bits);
  return round_bf16(1.0f / (1.0f + expf(-g)));
}
__device__ __forceinline__ float gate_bf16(const uint16_t* gate, int64_t stride, int row) {
  return gate_sigmoid_bf16(gate[static_cast<int64_t>(row) * stride]);
}

// Single rounding of a*b + c to bf16 for bf16 operands: the fp64 fma is exact
// unless the operands differ by more than ~2^37 in magnitude.
__device__ __forceinline__ float fma_bf16(float a, float b, float c) {
  const double exact = fma(static_cast<double>(a), static_cast<double>(b), static_cast<double>(c));
  const uint64_t bits = static_cast<uint64_t>(__double_as_longlong(exact));
  const uint64_t mag = bits & 0x7fffffffffffffffull;
  if (mag == 0) return static_cast<float>(exact);
  uint64_t kept = mag >> 45;
  const uint64_t rest = mag & ((1ull << 45) - 1);
  const uint64_t half = 1ull << 44;
  kept += (rest > half) || (rest == half && (kept & 1));
  const int64_t exponent = static_cast<int64_t>(kept >> 7) - 1023 + 127;
  if (exponent <= 0 || exponent >= 255) return round_bf16(static_cast<float>(exact));
  const uint32_t out = (static_cast<uint32_t>(bits >> 63) << 31) |
                       (static_cast<uint32_t>(exponent) << 23) |
                       (static_cast<uint32_t>(kept & 0x7f) << 16);
  return __uint_as_float(out);
}

__device__ __forceinline__ float block_sum(float v, float* scratch) {
  v = segment_sum<kWave>(v);
  const int wave = threadIdx.x / kWave;
  if (lane_id() == 0) scratch[wave] = v;
  __syncthreads();
  float total = 0.0f;
#pragma unroll
  for (int w = 0; w < kThreads / kWave; ++w) total += scratch[w];
  return total;
}

// out = bf16(shared * bf16(sigmoid(gate)) + routed), rounded once: the
// reference's combine_experts (kernels.py:427-445) is written as two bf16
// roundings, but its compiled form contracts the multiply-add into one bf16
// FMA, the result the reference then keeps in its fused residual variant
// (kernels.py:465-474); with the same FMA here, this kernel followed by
// add_norm gives combine_experts_add_norm's bytes.
__global__ __launch_bounds__(kThreads) void combine_experts_kernel(
    const uint16_t* __restrict__ routed, const uint16_t* __restrict__ shared,
    const uint16_t* __restrict__ gate, int64_t gate_stride, int width,
    uint16_t* __restrict__ out) {
  const int row = blockIdx.x;
  const int64_t base = static_cast<int64_t>(row) * width;
  for (int column = threadIdx.x * 4; column < width; column += kThreads * 4) {
    float r[4], s[4], v[4];
    load4(routed + base + column, r);
    load4(shared + base + column, s);
    // the gate loads with the rows (kept in the loop by the empty asm):
    // hoisted above them, its sigmoid's wait cost a round trip of its own
    const uint16_t* gate_row = gate;
    asm volatile("" : "+s"(gate_row));
    const float g = gate_bf16(gate_row, gate_stride, row);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = fma_bf16(s[i], g, r[i]);
    store4(out + base + column, v);
  }
}

// Per-route fp32 rows of the MoE (down [rows * top_k, width], by pair) and
// their routing weights, for kMode 2.
struct RouteRows {
  const float* down;
  const void* weights;
  int weights_f32;
  int top_k;
};

// kMode 0: add_norm(x, residual); 1: combine_experts_add_norm(_inverse);
// 2: mode 1 with each routed row reduced here from the per-route rows: the
//    rank-order fp32 sum of d3_weighted_combine, rounded to bf16 as it does,
//    so the bytes equal d3_weighted_combine followed by mode 1;
// 3: mode 2 without the residual and the norm: out = the combined row, the
//    bytes of d3_weighted_combine followed by d3_combine_experts.
template <int kMode>
__global__ __launch_bounds__(kThreads) void add_norm_kernel(
    const uint16_t* __restrict__ routed, const uint16_t* __restrict__ shared,
    const uint16_t* __restrict__ gate, int64_t gate_stride, const int64_t* __restrict__ inverse,
    uint16_t* __restrict__ residual, const uint16_t* __restrict__ weight, float eps, int width,
    uint16_t* __restrict__ out, RouteRows routes) {
  __shared__ float scratch[kThreads / kWave];
  constexpr bool kNorm = kMode != 3;
  constexpr bool kRoutes = kMode >= 2;
  const int row = blockIdx.x;
  const int source = inverse != nullptr ? static_cast<int>(inverse[row]) : row;
  const int64_t src = static_cast<int64_t>(source) * width;
  const int64_t dst = static_cast<int64_t>(row) * width;
  // Every load of a column group (norm weights, residual, shared row, gate,
  // then the routed rows) is issued before the first value is used, so a
  // row costs one memory round trip: the gate's sigmoid hoisted above the
  // row loads, or the residual loaded after the routed sum, each cost one
  // more.
  float values[kMaxPerThread], norm[kMaxPerThread];
  float squares = 0.0f;
  int count = 0;
  for (int column = threadIdx.x * 4; column < width; column += kThreads * 4, count += 4) {
    float r[4], res[4], v[4], s[4];
    uint16_t gate_bits = 0;
    if constexpr (kNorm) {
      load4(weight + column, &norm[count]);
      load4(residual + dst + column, res);
    }
    if constexpr (kMode != 0) {
      load4(shared + src + column, s);
      const uint16_t* gate_row = gate;
      asm volatile("" : "+s"(gate_row));  // loaded here, not hoisted out of the loop and waited for
      gate_bits = gate_row[static_cast<int64_t>(source) * gate_stride];
    }
    if constexpr (kRoutes) {
      const float4 sum = routes.top_k == 8
                             ? combine4_fixed<8>(routes.down, routes.weights, routes.weights_f32,
                                                 source, width, column)
                             : combine4(routes.down, routes.weights, routes.weights_f32, source,
                                        routes.top_k, width, column);
      r[0] = round_bf16(sum.x);
      r[1] = round_bf16(sum.y);
      r[2] = round_bf16(sum.z);
      r[3] = round_bf16(sum.w);
    } else {
      load4(routed + src + column, r);
    }
    if constexpr (!kNorm) {
      const float g = gate_sigmoid_bf16(gate_bits);
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = fma_bf16(s[i], g, r[i]);
      store4(out + dst + column, v);
      continue;
    } else if constexpr (kMode != 0) {
      const float g = gate_sigmoid_bf16(gate_bits);
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = round_bf16(fma_bf16(s[i], g, r[i]) + res[i]);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = round_bf16(r[i] + res[i]);
    }
    store4(residual + dst + column, v);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      values[count + i] = v[i];
      squares += v[i] * v[i];
    }
  }
  if constexpr (!kNorm) return;
  const float total = block_sum(squares, scratch);
  const float inv = 1.0f / sqrtf(total / static_cast<float>(width) + eps);
  count = 0;
  for (int column = threadIdx.x * 4; column < width; column += kThreads * 4, count += 4) {
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = values[count + i] * inv * (1.0f + norm[count + i]);
    store4(out + dst + column, v);
  }
}

// The decode layer's epilogue in one launch: for row r (a live slot of a
// decode step whose FC1 ranked the experts itself, so no routing weights
// are stored yet), wave 0 routes the row's logits with the front's function
// (route_top_k) and rounds the weights to the stored dtype, while every
// thread loads its columns' eight down rows (by pair r * top_k + rank), the
// shared expert row and (kNorm) the residual row; then
//   routed   = bf16(sum_rank w[rank] * down[rank])   (rank order, fp32 FMAs)
//   combined = bf16 FMA(shared, bf16(sigmoid(gate)), routed)
// and out = combined (combine_experts), or (kNorm) residual <- bf16(combined
// + residual), out = bf16(residual * rsqrt(mean(residual^2) + eps) * (1 + w))
// (combine_experts_add_norm).  The bytes equal d3_decode_route_combine
// followed by d3_combine_experts (+ d3_add_norm): the same arithmetic in the
// same order.
struct RouteLogitArgs {
  const float* down;
  const void* logits;
  int64_t logits_stride;  // elements
  int num_experts;
  int top_k;
  void* weights;  // [rows, top_k] stored routing weights, or nullptr
  int weights_f32;
  const uint16_t* shared;
  const uint16_t* gate;
  int64_t gate_stride;
  uint16_t* residual;
  const uint16_t* norm;
  float eps;
  int width;
  uint16_t* out;
};

template <int NPL, bool kF32, bool kNorm, int kChunks>
__global__ __launch_bounds__(kThreads) void combine_route_logits_kernel(RouteLogitArgs a) {
  __shared__ float route_w[8];
  __shared__ float scratch[kThreads / kWave];
  const int row = blockIdx.x;
  const int lane = lane_id();
  const int wave = static_cast<int>(threadIdx.x) / kWave;
  const int width = a.width;
  const int64_t base = static_cast<int64_t>(row) * width;
  // without the norm, workgroup (row, slice) takes the row's columns
  // [slice * 4 * blockDim, (slice + 1) * 4 * blockDim) and recomputes the
  // row's routing
  const int span = static_cast<int>(blockDim.x) * 4;
  const int column0 = static_cast<int>(blockIdx.y) * span * kChunks;
  // Every load (logits in every wave, the gate, the route rows, shared,
  // residual and norm weights) is issued before the first value is used:
  // logits loaded under a wave-0 branch, or the gate and norm weights
  // loaded after the first use of another load, each cost a memory round
  // trip of their own.
  RouteLogits<NPL> logits;
  load_route_logits<NPL, kF32>(static_cast<const char*>(a.logits) +
                                   static_cast<int64_t>(row) * a.logits_stride * (kF32 ? 4 : 2),
                               a.num_experts, logits);
  const uint16_t gate_bits = a.gate[static_cast<int64_t>(row) * a.gate_stride];
  float4 y[kChunks][8];
  float s[kChunks][4], res[kChunks][4], norm[kChunks][4];
#pragma unroll
  for (int c = 0; c < kChunks; ++c) {
    const int column = column0 + threadIdx.x * 4 + c * span;
    const bool inside = column < width;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      y[c][r] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if (inside && r < a.top_k)
        y[c][r] = *reinterpret_cast<const float4*>(a.down + (static_cast<int64_t>(row) * a.top_k + r) * width +
                                                   column);
    }
    if (inside) {
      load4(a.shared + base + column, s[c]);
      if constexpr (kNorm) {
        load4(a.residual + base + column, res[c]);
        load4(a.norm + column, norm[c]);
      }
    }
  }
  const float g = gate_sigmoid_bf16(gate_bits);
  if (wave == 0) {
    const RouteChoice choice = route_top_k<NPL>(logits, a.num_experts, a.top_k);
    if (lane < a.top_k) {
      route_w[lane] = stored_weight(choice.weight, a.weights_f32);
      if (a.weights != nullptr && blockIdx.y == 0) {
        const int64_t index = static_cast<int64_t>(row) * a.top_k + lane;
        if (a.weights_f32)
          static_cast<float*>(a.weights)[index] = choice.weight;
        else
          static_cast<uint16_t*>(a.weights)[index] = f32_to_bf16(choice.weight);
      }
    }
  }
  __syncthreads();
  float values[kChunks][4];
  float squares = 0.0f;
#pragma unroll
  for (int c = 0; c < kChunks; ++c) {
    const int column = column0 + threadIdx.x * 4 + c * span;
    if (column >= width) continue;
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      if (r < a.top_k) {
        const float wr = route_w[r];
        acc.x = fmaf(wr, y[c][r].x, acc.x);
        acc.y = fmaf(wr, y[c][r].y, acc.y);
        acc.z = fmaf(wr, y[c][r].z, acc.z);
        acc.w = fmaf(wr, y[c][r].w, acc.w);
      }
    }
    const float routed[4] = {round_bf16(acc.x), round_bf16(acc.y), round_bf16(acc.z), round_bf16(acc.w)};
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = fma_bf16(s[c][i], g, routed[i]);
    if constexpr (kNorm) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[i] = round_bf16(v[i] + res[c][i]);
        squares += v[i] * v[i];
        values[c][i] = v[i];
      }
      store4(a.residual + base + column, v);
    } else {
      store4(a.out + base + column, v);
    }
  }
  if constexpr (kNorm) {
    const float total = block_sum(squares, scratch);
    const float inv = 1.0f / sqrtf(total / static_cast<float>(width) + a.eps);
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
      const int column = column0 + threadIdx.x * 4 + c * span;
      if (column >= width) continue;
      float v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = values[c][i] * inv * (1.0f + norm[c][i]);
      store4(a.out + base + column, v);
    }
  }
}

template <int NPL, bool kF32, bool kNorm>
void launch_route_logits(const RouteLogitArgs& a, int rows, hipStream_t s) {
  if constexpr (!kNorm) {  // 512-column slices: a decode batch's rows alone leave most CUs idle
    constexpr int kSliceThreads = 128;
    const int slices = (a.width + kSliceThreads * 4 - 1) / (kSliceThreads * 4);
    hipLaunchKernelGGL((combine_route_logits_kernel<NPL, kF32, kNorm, 1>), dim3(rows, slices),
                       dim3(kSliceThreads), 0, s, a);
  } else if (a.width <= kThreads * 4) {
    hipLaunchKernelGGL((combine_route_logits_kernel<NPL, kF32, kNorm, 1>), dim3(rows), dim3(kThreads), 0, s, a);
  } else {
    hipLaunchKernelGGL((combine_route_logits_kernel<NPL, kF32, kNorm, 2>), dim3(rows), dim3(kThreads), 0, s, a);
  }
}

template <int NPL>
void launch_route_logits(const RouteLogitArgs& a, int rows, bool f32, bool norm, hipStream_t s) {
  if (f32) {
    if (norm) launch_route_logits<NPL, true, true>(a, rows, s);
    else launch_route_logits<NPL, true, false>(a, rows, s);
  } else {
    if (norm) launch_route_logits<NPL, false, true>(a, rows, s);
    else launch_route_logits<NPL, false, false>(a, rows, s);
  }
}

// silu_mul (kernels.py:386-395): bf16(bf16(g * sigmoid(g)) * u).
__global__ __launch_bounds__(kThreads) void silu_mul_kernel(const uint16_t* __restrict__ x,
                                                            int64_t stride, int width,
                                                            uint16_t* __restrict__ out) {
  const int row = blockIdx.x;
  const uint16_t* in = x + static_cast<int64_t>(row) * stride;
  for (int column = threadIdx.x * 4; column < width; column += kThreads * 4) {
    float g[4], u[4], v[4];
    load4(in + column, g);
    load4(in + width + column, u);
    silu_mul_values<4>(g, u, v);
    store4(out + static_cast<int64_t>(row) * width + column, v);
  }
}

bool aligned8(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7u) == 0; }

}  // namespace
}  // namespace d3

using namespace d3;

extern "C" int d3_combine_experts(const uint16_t* routed, const uint16_t* shared,
                                  const uint16_t* gate, int64_t gate_stride, int32_t rows,
                                  int32_t width, uint16_t* out, void* stream) {
  D3_REQUIRE(rows == 0 || (routed && shared && gate && out), "combine_experts: null pointer");
  D3_REQUIRE(rows >= 0 && width > 0 && width % 4 == 0, "combine_experts: width %% 4 != 0");
  D3_REQUIRE(aligned8(routed) && aligned8(shared) && aligned8(out), "combine_experts: alignment");
  if (rows == 0) {
    clear_error();
    return D3_OK;
  }
  hipLaunchKernelGGL(combine_experts_kernel, dim3(rows), dim3(kThreads), 0, as_stream(stream),
                     routed, shared, gate, gate_stride, width, out);
  D3_LAUNCHED("combine_experts");
}

extern "C" int d3_combine_experts_add_norm(const uint16_t* routed, const uint16_t* shared,
                                           const uint16_t* gate, int64_t gate_stride,
                                           const int64_t* inverse, uint16_t* residual,
                                           const uint16_t* weight, float eps, int32_t rows,
                                           int32_t width, uint16_t* out, void* stream) {
  D3_REQUIRE(rows == 0 || (routed && shared && gate && residual && weight && out),
             "combine_experts_add_norm: null pointer");
  D3_REQUIRE(rows >= 0 && width > 0 && width % 4 == 0 && width <= kThreads * kMaxPerThread,
             "combine_experts_add_norm: width %d must be a multiple of 4 and <= 8192", width);
  D3_REQUIRE(aligned8(routed) && aligned8(shared) && aligned8(residual) && aligned8(out) &&
                 aligned8(weight),
             "combine_experts_add_norm: alignment");
  if (rows == 0) {
    clear_error();
    return D3_OK;
  }
  hipLaunchKernelGGL(add_norm_kernel<1>, dim3(rows), dim3(kThreads), 0, as_stream(stream), routed,
                     shared, gate, gate_stride, inverse, residual, weight, eps, width, out,
                     RouteRows{});
  D3_LAUNCHED("combine_experts_add_norm");
}

extern "C" int d3_combine_routes_add_norm(const float* down, const void* route_weights,
                                          int32_t weights_dtype, int32_t top_k,
                                          const uint16_t* shared, const uint16_t* gate,
                                          int64_t gate_stride, const int64_t* inverse,
                                          uint16_t* residual, const uint16_t* weight, float eps,
                                          int32_t rows, int32_t width, uint16_t* out,
                                          void* stream) {
  D3_REQUIRE(rows == 0 || (down && route_weights && shared && gate && out && (residual == nullptr || weight)),
             "combine_routes_add_norm: null pointer");
  D3_REQUIRE(weights_dtype == D3_DTYPE_BF16 || weights_dtype == D3_DTYPE_F32,
             "combine_routes_add_norm: weights must be bf16 or f32");
  D3_REQUIRE(top_k >= 1 && top_k <= 16, "combine_routes_add_norm: bad top_k %d", top_k);
  D3_REQUIRE(rows >= 0 && width > 0 && width % 4 == 0 && width <= kThreads * kMaxPerThread,
             "combine_routes_add_norm: width %d must be a multiple of 4 and <= 8192", width);
  D3_REQUIRE((reinterpret_cast<uintptr_t>(down) & 15u) == 0 && aligned8(shared) && aligned8(out) &&
                 (residual == nullptr || (aligned8(residual) && aligned8(weight))),
             "combine_routes_add_norm: alignment");
  if (rows == 0) {
    clear_error();
    return D3_OK;
  }
  const RouteRows routes{down, route_weights, weights_dtype == D3_DTYPE_F32 ? 1 : 0, top_k};
  if (residual == nullptr)  // combine_experts of the routed combine, no norm
    hipLaunchKernelGGL(add_norm_kernel<3>, dim3(rows), dim3(kThreads), 0, as_stream(stream),
                       nullptr, shared, gate, gate_stride, inverse, nullptr, nullptr, eps, width,
                       out, routes);
  else
    hipLaunchKernelGGL(add_norm_kernel<2>, dim3(rows), dim3(kThreads), 0, as_stream(stream),
                       nullptr, shared, gate, gate_stride, inverse, residual, weight, eps, width,
                       out, routes);
  D3_LAUNCHED("combine_routes_add_norm");
}

extern "C" int d3_add_norm(const uint16_t* x, uint16_t* residual, const uint16_t* weight, float eps,
                           int32_t rows, int32_t width, uint16_t* out, void* stream) {
  D3_REQUIRE(rows == 0 || (x && residual && weight && out), "add_norm: null pointer");
  D3_REQUIRE(rows >= 0 && width > 0 && width % 4 == 0 && width <= kThreads * kMaxPerThread,
             "add_norm: width %d must be a multiple of 4 and <= 8192", width);
  D3_REQUIRE(aligned8(x) && aligned8(residual) && aligned8(out) && aligned8(weight),
             "add_norm: alignment");
  if (rows == 0) {
    clear_error();
    return D3_OK;
  }
  hipLaunchKernelGGL(add_norm_kernel<0>, dim3(rows), dim3(kThreads), 0, as_stream(stream), x,
                     nullptr, nullptr, 0, nullptr, residual, weight, eps, width, out, RouteRows{});
  D3_LAUNCHED("add_norm");
}

extern "C" int d3_silu_mul(const uint16_t* projected, int64_t row_stride, int32_t rows,
                           int32_t width, uint16_t* out, void* stream) {
  D3_REQUIRE(rows == 0 || (projected && out), "silu_mul: null pointer");
  D3_REQUIRE(rows >= 0 && width > 0 && width % 4 == 0 && row_stride >= 2 * width &&
                 row_stride % 4 == 0,
             "silu_mul: bad shape");
  D3_REQUIRE(aligned8(projected) && aligned8(out), "silu_mul: alignment");
  if (rows == 0) {
    clear_error();
    return D3_OK;
  }
  hipLaunchKernelGGL(silu_mul_kernel, dim3(rows), dim3(kThreads), 0, as_stream(stream), projected,
                     row_stride, width, out);
  D3_LAUNCHED("silu_mul");
}

extern "C" int d3_combine_route_logits(const float* down, const void* logits, int32_t logits_dtype,
                                       int64_t logits_stride, int32_t num_experts, int32_t top_k,
                                       void* route_weights, int32_t weights_dtype,
                                       const uint16_t* shared, const uint16_t* gate,
                                       int64_t gate_stride, uint16_t* residual,
                                       const uint16_t* weight, float eps, int32_t rows,
                                       int32_t width, uint16_t* out, void* stream) {
  D3_REQUIRE(rows == 0 || (down && logits && shared && gate && out && (residual == nullptr || weight != nullptr)),
             "combine_route_logits: null pointer");
  D3_REQUIRE(logits_dtype == D3_DTYPE_BF16 || logits_dtype == D3_DTYPE_F32,
             "combine_route_logits: logits must be bf16 or f32");
  D3_REQUIRE(weights_dtype == D3_DTYPE_BF16 || weights_dtype == D3_DTYPE_F32,
             "combine_route_logits: weights must be bf16 or f32");
  D3_REQUIRE(num_experts >= 1 && top_k >= 1 && top_k <= num_experts && logits_stride >= num_experts,
             "combine_route_logits: bad routing shape (E=%d, top_k=%d)", num_experts, top_k);
  D3_SUPPORTED(top_k <= 8 && num_experts <= 256,
               "combine_route_logits: top_k %d (<= 8), E %d (<= 256)", top_k, num_experts);
  D3_REQUIRE(rows >= 0 && width > 0 && width % 4 == 0, "combine_route_logits: width %d", width);
  D3_SUPPORTED(width <= 2 * kThreads * 4, "combine_route_logits: width %d above %d", width,
               2 * kThreads * 4);
  D3_REQUIRE((reinterpret_cast<uintptr_t>(down) & 15u) == 0 && aligned8(shared) && aligned8(out) &&
                 (residual == nullptr || (aligned8(residual) && aligned8(weight))),
             "combine_route_logits: alignment");
  if (rows == 0) {
    clear_error();
    return D3_OK;
  }
  const RouteLogitArgs args{down, logits, logits_stride, num_experts, top_k, route_weights,
                            weights_dtype == D3_DTYPE_F32 ? 1 : 0, shared, gate, gate_stride,
                            residual, weight, eps, width, out};
  const bool f32 = logits_dtype == D3_DTYPE_F32, norm = residual != nullptr;
  hipStream_t s = as_stream(stream);
  if (num_experts <= 64)
    launch_route_logits<1>(args, rows, f32, norm, s);
  else if (num_experts <= 128)
    launch_route_logits<2>(args, rows, f32, norm, s);
  else
    launch_route_logits<4>(args, rows, f32, norm, s);
  D3_LAUNCHED("combine_route_logits");
}
