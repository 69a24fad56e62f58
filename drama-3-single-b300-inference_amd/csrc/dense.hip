// Dense bf16 GEMM of the MoE layer's projections: out[M, N] = x[M, K] .
// W[N, K]^T, fp32 accumulation, one bf16 rounding.  Used for the packed input projection (model.py:230-245,
// 495-501: shared gate / up rows, router, shared-expert gate), whose
// epilogue also forms the shared expert's activation silu_mul(gate, up)
// (kernels.py:386-395), and for the shared expert's down projection.
//
// Decode-sized row counts (up to 768; gfx950, wave64, mfma_f32_16x16x32_bf16):
//   * A workgroup owns two 16-row tiles of W and one 16-row tile of x, so a
//     decode-sized batch spreads over (tile pairs) x (x tiles) workgroups
//     instead of leaving most CUs idle (64 rows of x per workgroup measured
//     3.5 us slower on the reference model's layer).  K is walked in chunks
//     of 256 columns: the workgroup copies the chunk of both operands (16 x
//     rows, 32 W rows; 24 KB) into LDS with coalesced 16-byte loads (each
//     wave instruction reads 1 KB of contiguous row), the next two chunks'
//     loads in flight (registers) while the current chunk is multiplied.
//   * LDS rows are 512 bytes; the 16-byte part p of row r is stored at
//     position p ^ (r & 31), so the 16 rows an MFMA fragment read touches
//     land on distinct banks.
//   * Wave w computes weight tile w / 4 over the K quarter w % 4 of every
//     chunk; the four quarters' fp32 sums meet in LDS and are added in
//     quarter order.  (Operands loaded straight into MFMA fragments, with
//     no LDS, measured 1.7 us slower: each wave instruction then reads 16
//     row pieces of 64 bytes.)
//   * Paired tiles (the projection's first 2I rows are the shared expert's
//     gate rows then its up rows): a workgroup takes gate tile j and up tile
//     j, so it holds both halves of 16 activation columns and writes
//     act = bf16(bf16(silu(gate)) * up) from the rounded outputs, the bytes
//     of d3_silu_mul.
//
// Prefill-sized row counts (the layer's projections over thousands of packed
// rows) take a second kernel, tiled for contraction rather than for streaming
// the weights:
//   * A workgroup (4 waves, two workgroups per CU) owns a tile of 128 weight
//     rows by 128 (or 64) x rows; each wave a 64 x 64 (or 64 x 32) part of
//     it as 4 x 4 (4 x 2) blocks of mfma_f32_16x16x32_bf16, so every
//     fragment read from LDS feeds four MFMAs.
//   * K is walked in steps of 64 columns (128 bytes of a row): both operand
//     tiles are staged global -> registers -> LDS (coalesced 16-byte loads,
//     8 threads per 128-byte row; 144-byte LDS rows, the 16-byte pad putting
//     the 16 rows of each ds_read_b128 on distinct banks), the next step's
//     loads in flight while the current step is multiplied; two LDS slots,
//     one barrier per step.
//   * Paired tiles hold 64 gate rows and the matching 64 up rows, so each
//     lane holds gate and up of the same (row, column) and the epilogue
//     writes act as the small-batch kernel does.
//   * Tiles are numbered weight-tile fastest and handed to the XCDs in
//     contiguous ranges, so the tiles an XCD runs at once share their x rows
//     (and, a few rows of tiles apart, their weight rows) in that XCD's L2.
//   * Measured (per-phase timestamps of one wave): a step's 32 KB of global
//     loads per workgroup take as long to issue as the step's MFMAs; issued
//     in one block they kept the wave from issuing MFMAs meanwhile, so the
//     loads are spread among the MFMAs (one load per four MFMAs, a fixed
//     issue order set with sched_group_barrier): 7 % faster.  At 4096 x 1408
//     x 2048 the 352 tiles leave most CUs one workgroup and some two (the
//     kernel's time); tiles that divide evenly over the CUs, or a split of
//     K across workgroups, are the next step.
#include <type_traits>

#include "common.h"
#include "expert_tile.h"
#include "status.h"

namespace d3 {
namespace {

constexpr int kDenseWaves = 8;
constexpr int kDenseThreads = kDenseWaves * kWave;
constexpr int kDenseTokens = 16;   // x rows per workgroup (one token tile)
constexpr int kDenseChunk = 256;   // K columns per LDS chunk (512 bytes of a row)
constexpr int kDenseParts = kDenseChunk * 2 / 16;  // 16-byte parts per chunk row (32)
constexpr int kXLoads = kDenseTokens * kDenseParts / kDenseThreads;  // 1 per thread
constexpr int kWLoads = 32 * kDenseParts / kDenseThreads;            // 2 per thread

struct DenseArgs {
  const uint16_t* x;
  int64_t x_stride;  // elements
  int rows;
  const uint16_t* w;  // [n, k]
  int n;
  int k;
  uint16_t* out;
  int64_t out_stride;  // elements
  int pairs;           // workgroups 0 .. pairs-1 take gate tile j and up tile j
  int pair_offset;     // rows between a gate tile and its up tile (I)
  uint16_t* act;       // [rows, act_stride] silu_mul of each pair, or nullptr
  int64_t act_stride;
};

__device__ __forceinline__ bf16x8 as_bf16x8(int32x4 v) { return __builtin_bit_cast(bf16x8, v); }

// Byte offset of 16-byte part p of LDS row r (512-byte rows, XOR swizzle).
__device__ __forceinline__ int lds_part(int r, int p) { return r * 512 + ((p ^ (r & 31)) << 4); }

// CHUNKS = K / 256 (compile time, so the register sets of the chunk loop
// are indexed statically).
template <int CHUNKS>
__global__ __launch_bounds__(kDenseThreads) void dense_bf16_kernel(DenseArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t xs[2][kDenseTokens * 512];
  __shared__ __attribute__((aligned(16))) uint8_t wsm[2][32 * 512];
  __shared__ floatx4 quarter_sum[2][4][kWave];
  __shared__ floatx4 up_sum[kWave];
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int row16 = lane & 15;
  const int quarter = lane >> 4;
  const int tiles = a.n / 16;
  const int b = blockIdx.x;
  int t0, t1;
  if (b < a.pairs) {  // gate tile j and its up tile
    t0 = b;
    t1 = b + a.pair_offset / 16;
  } else {  // two consecutive tiles after the pairs (the second clamped)
    t0 = 2 * a.pairs + 2 * (b - a.pairs);
    t1 = min(t0 + 1, tiles - 1);
  }
  const bool second = t1 != t0;
  constexpr int chunks = CHUNKS;
  const BufferView w_view(a.w, static_cast<uint32_t>(static_cast<int64_t>(a.n) * a.k * 2));
  const BufferView x_view(a.x, static_cast<uint32_t>(static_cast<int64_t>(a.rows) * a.x_stride * 2));
  const int r_tile = wave >> 2;  // this wave's weight tile (0: t0, 1: t1)
  const int kq = wave & 3;       // and quarter of each chunk's K columns

  {
    const int m0 = blockIdx.y * kDenseTokens;
    // staging of chunk c: thread loads x parts q = tid + 512 i (row q / 32,
    // part q % 32) and W parts likewise (rows 0-15: tile t0, 16-31: t1);
    // the next two chunks are in flight in registers (set c % 2) while chunk
    // c is multiplied from LDS.
    constexpr int kSets = chunks < 2 ? chunks : 2;
    int4 xr[kSets][kXLoads], wr[kSets][kWLoads];
    auto load_chunk = [&](int c, int set) {
#pragma unroll
      for (int i = 0; i < kXLoads; ++i) {
        const int q = tid + kDenseThreads * i, r = q >> 5, p = q & 31;
        const int token = m0 + r;
        xr[set][i] = x_view.load16(token < a.rows ? static_cast<uint32_t>((static_cast<int64_t>(token) * a.x_stride +
                                                                             c * kDenseChunk + p * 8) * 2)
                                                  : kNoRow);
      }
#pragma unroll
      for (int i = 0; i < kWLoads; ++i) {
        const int q = tid + kDenseThreads * i, r = q >> 5, p = q & 31;
        const int row = (r < 16 ? t0 : t1) * 16 + (r & 15);
        wr[set][i] = w_view.load16(static_cast<uint32_t>((static_cast<int64_t>(row) * a.k + c * kDenseChunk + p * 8) * 2));
      }
    };
    auto store_chunk = [&](int set, int slot) {
#pragma unroll
      for (int i = 0; i < kXLoads; ++i) {
        const int q = tid + kDenseThreads * i;
        *reinterpret_cast<int4*>(&xs[slot][lds_part(q >> 5, q & 31)]) = xr[set][i];
      }
#pragma unroll
      for (int i = 0; i < kWLoads; ++i) {
        const int q = tid + kDenseThreads * i;
        *reinterpret_cast<int4*>(&wsm[slot][lds_part(q >> 5, q & 31)]) = wr[set][i];
      }
    };
#pragma unroll
    for (int c = 0; c < kSets; ++c) load_chunk(c, c);
    store_chunk(0, 0);
    __syncthreads();
    floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int c = 0; c < chunks; ++c) {
      // set c % 2 was stored; reuse it for chunk c + 2
      if (c + kSets < chunks) load_chunk(c + kSets, c % kSets);
      __builtin_amdgcn_sched_barrier(0);
      const uint8_t* xb = xs[c & 1];
      const uint8_t* wb = wsm[c & 1];
      const int xrow = row16, wrow = 16 * r_tile + row16;
#pragma unroll
      for (int s = 2 * kq; s < 2 * kq + 2; ++s) {
        const int p = 4 * s + quarter;  // k = 32 s + 8 quarter .. + 8
        const int32x4 av = *reinterpret_cast<const int32x4*>(&wb[lds_part(wrow, p)]);
        const int32x4 bv = *reinterpret_cast<const int32x4*>(&xb[lds_part(xrow, p)]);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(av), as_bf16x8(bv), acc, 0, 0, 0);
      }
      if (c + 1 < chunks) store_chunk((c + 1) % kSets, (c + 1) & 1);
      __syncthreads();
    }
    // The quarters' sums meet in LDS and the first wave of each W tile adds
    // them in quarter order; lane holds rows 16 tile + 4 quarter .. + 3 of
    // token m0 + row16.
    quarter_sum[r_tile][kq][lane] = acc;
    __syncthreads();
    const int token = m0 + row16;
    const int tile = r_tile ? t1 : t0;
    float rounded[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (kq == 0) {
      floatx4 sum = quarter_sum[r_tile][0][lane];
#pragma unroll
      for (int q = 1; q < 4; ++q) sum += quarter_sum[r_tile][q][lane];
#pragma unroll
      for (int i = 0; i < 4; ++i) rounded[i] = bf16_to_f32(f32_to_bf16(sum[i]));
      if (token < a.rows && (r_tile == 0 || second)) {
        const uint32_t lo = f32_to_bf16(sum[0]) | (static_cast<uint32_t>(f32_to_bf16(sum[1])) << 16);
        const uint32_t hi = f32_to_bf16(sum[2]) | (static_cast<uint32_t>(f32_to_bf16(sum[3])) << 16);
        *reinterpret_cast<uint2*>(a.out + static_cast<int64_t>(token) * a.out_stride + tile * 16 + 4 * quarter) =
            make_uint2(lo, hi);
      }
      if (r_tile == 1) up_sum[lane] = floatx4{rounded[0], rounded[1], rounded[2], rounded[3]};
    }
    if (b < a.pairs && a.act != nullptr) {  // uniform over the workgroup
      __syncthreads();
      if (kq == 0 && r_tile == 0 && token < a.rows) {
        const floatx4 up4 = up_sum[lane];
        const float up[4] = {up4[0], up4[1], up4[2], up4[3]};
        float v[4];
        silu_mul_values<4>(rounded, up, v);
        const uint32_t lo = f32_to_bf16(v[0]) | (static_cast<uint32_t>(f32_to_bf16(v[1])) << 16);
        const uint32_t hi = f32_to_bf16(v[2]) | (static_cast<uint32_t>(f32_to_bf16(v[3])) << 16);
        *reinterpret_cast<uint2*>(a.act + static_cast<int64_t>(token) * a.act_stride + t0 * 16 + 4 * quarter) =
            make_uint2(lo, hi);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Tiled kernel for prefill-sized row counts.
// ---------------------------------------------------------------------------
constexpr int kTiledWaves = 4;
constexpr int kTiledThreads = kTiledWaves * kWave;
constexpr int kTiledN = 128;                    // weight rows per workgroup tile
constexpr int kTiledK = 64;                     // K columns per step
constexpr int kTiledRowBytes = kTiledK * 2;     // 128 bytes of a row per step
constexpr int kTiledStride = kTiledRowBytes + 16;  // LDS bytes per staged row
constexpr int kTiledPairRows = kTiledN / 2;     // gate (and up) rows of a paired tile
constexpr int kTiledXcds = 8;
constexpr int kTiledMinRows = 769;  // fewer rows (and K in its set): the small-batch kernel

struct TiledGrid {
  int m_tiles;
  int n_tiles;
  int pair_tiles;  // tiles 0 .. pair_tiles-1 are paired (gate rows + up rows)
  int per_xcd;     // logical tiles per XCD range
};

// BM: x rows per workgroup (128 or 64).
template <int BM>
__global__ __launch_bounds__(kTiledThreads) __attribute__((amdgpu_waves_per_eu(2))) void dense_bf16_tiled_kernel(
    DenseArgs a, TiledGrid grid) {
  constexpr int kWM = BM / 2;       // x rows per wave
  constexpr int kTB = kWM / 16;     // 16-row x blocks per wave
  constexpr int kFB = 4;            // 16-row weight blocks per wave
  constexpr int kWLoads = kTiledN * (kTiledRowBytes / 16) / kTiledThreads;  // 4
  constexpr int kXLoads = BM * (kTiledRowBytes / 16) / kTiledThreads;       // 4 or 2
  __shared__ __attribute__((aligned(16))) uint8_t wsm[2][kTiledN * kTiledStride];
  __shared__ __attribute__((aligned(16))) uint8_t xsm[2][BM * kTiledStride];

  // Contiguous logical ranges per XCD (workgroup b runs on XCD b % 8).
  const int b = blockIdx.x;
  const int logical = (b % kTiledXcds) * grid.per_xcd + b / kTiledXcds;
  if (logical >= grid.m_tiles * grid.n_tiles) return;  // uniform
  const int mt = logical / grid.n_tiles;
  const int nt = logical - mt * grid.n_tiles;
  const bool paired = nt < grid.pair_tiles;
  const int m0 = mt * BM;

  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int wm = wave & 1;   // x-row half of the tile
  const int wn = wave >> 1;  // weight-row half
  const int row16 = lane & 15;
  const int quarter = lane >> 4;

  // Weight row of LDS row r of this tile (paired: 64 gate rows, then the
  // matching 64 up rows).
  auto weight_row = [&](int r) {
    if (paired) return r < kTiledPairRows ? kTiledPairRows * nt + r : a.pair_offset + kTiledPairRows * nt + r - kTiledPairRows;
    return 2 * a.pair_offset + kTiledN * (nt - grid.pair_tiles) + r;
  };
  // LDS row of this wave's weight block fb: paired waves take gate blocks
  // 0-1 and the up blocks of the same columns as 2-3.
  auto block_lds_row = [&](int fb) {
    if (paired) return (fb < 2 ? 0 : kTiledPairRows) + 32 * wn + 16 * (fb & 1);
    return 64 * wn + 16 * fb;
  };

  const BufferView w_view(a.w, static_cast<uint32_t>(static_cast<int64_t>(a.n) * a.k * 2));
  const BufferView x_view(a.x, static_cast<uint32_t>(static_cast<int64_t>(a.rows) * a.x_stride * 2));
  // Staging: thread t copies 16-byte part t % 8 of rows t / 8 + 32 i.
  const int part = tid & 7;
  const int r0 = tid >> 3;
  uint32_t w_src[kWLoads], x_src[kXLoads];
#pragma unroll
  for (int i = 0; i < kWLoads; ++i) {
    const int row = weight_row(r0 + 32 * i);
    w_src[i] = row < a.n ? static_cast<uint32_t>(row) * a.k * 2 + part * 16 : kNoRow;
  }
#pragma unroll
  for (int i = 0; i < kXLoads; ++i) {
    const int token = m0 + r0 + 32 * i;
    x_src[i] = token < a.rows ? static_cast<uint32_t>(static_cast<int64_t>(token) * a.x_stride * 2) + part * 16 : kNoRow;
  }
  // Two register sets: the loads of step k + 2 are issued while step k is
  // multiplied, and step k + 1's data (loaded one step earlier) is stored to
  // LDS after it, so every load has two steps of MFMAs to arrive.
  int4 wr[2][kWLoads], xr[2][kXLoads];
  // Steps past K (the loop runs an even number of steps) load zeros
  // through the buffer bounds, so every load and store of the loop is
  // unconditional: a branch around them would leave the compiler unable to
  // count outstanding loads, and it would then wait for all of them (the
  // ones just issued for step k + 2 included) before each LDS store.
  const int steps = a.k / kTiledK;
  auto load_step = [&](int step, auto set) {
    const uint32_t k_off = static_cast<uint32_t>(step) * kTiledRowBytes;
    const bool live = step < steps;
#pragma unroll
    for (int i = 0; i < kXLoads; ++i)
      xr[set][i] = x_view.load16(live && x_src[i] != kNoRow ? x_src[i] + k_off : kNoRow);
#pragma unroll
    for (int i = 0; i < kWLoads; ++i)
      wr[set][i] = w_view.load16(live && w_src[i] != kNoRow ? w_src[i] + k_off : kNoRow);
  };
  auto store_step = [&](auto set, int slot) {
#pragma unroll
    for (int i = 0; i < kXLoads; ++i)
      *reinterpret_cast<int4*>(&xsm[slot][(r0 + 32 * i) * kTiledStride + part * 16]) = xr[set][i];
#pragma unroll
    for (int i = 0; i < kWLoads; ++i)
      *reinterpret_cast<int4*>(&wsm[slot][(r0 + 32 * i) * kTiledStride + part * 16]) = wr[set][i];
  };

  floatx4 acc[kFB][kTB];
#pragma unroll
  for (int fb = 0; fb < kFB; ++fb)
#pragma unroll
    for (int tb = 0; tb < kTB; ++tb) acc[fb][tb] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

  auto multiply = [&](int slot) {
    const uint8_t* wb = wsm[slot];
    const uint8_t* xb = xsm[slot];
#pragma unroll
    for (int s = 0; s < 2; ++s) {  // the two 32-column slices of the step
      const int col = s * 64 + quarter * 16;
      int32x4 wf[kFB], xf[kTB];
#pragma unroll
      for (int fb = 0; fb < kFB; ++fb)
        wf[fb] = *reinterpret_cast<const int32x4*>(&wb[(block_lds_row(fb) + row16) * kTiledStride + col]);
#pragma unroll
      for (int tb = 0; tb < kTB; ++tb)
        xf[tb] = *reinterpret_cast<const int32x4*>(&xb[(kWM * wm + 16 * tb + row16) * kTiledStride + col]);
#pragma unroll
      for (int fb = 0; fb < kFB; ++fb)
#pragma unroll
        for (int tb = 0; tb < kTB; ++tb)
          acc[fb][tb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(wf[fb]), as_bf16x8(xf[tb]), acc[fb][tb], 0, 0, 0);
    }
  };
  // Step k: issue step k + 2's loads into set k % 2 (its step-k data is in
  // LDS already), multiply slot k % 2, store set (k + 1) % 2 to slot
  // (k + 1) % 2 (last read in step k - 1, before the previous barrier),
  // barrier.  With an odd step count the last step multiplies zeros.
  auto iteration = [&](int step, auto set) {
    constexpr int kSet = decltype(set)::value;
    constexpr int kOther = 1 - kSet;
    load_step(step + 2, set);
    multiply(kSet);
    store_step(std::integral_constant<int, kOther>{}, kOther);
    // Issue order: each slice's LDS reads, then its MFMAs with the next
    // steps' global loads spread among them (a wave blocked issuing loads
    // then has MFMAs of its own in flight), the LDS stores last.
    constexpr int kLoads = kWLoads + kXLoads;
    constexpr int kSliceMfma = kFB * kTB;
    constexpr int kHalf = kLoads / 2;
    constexpr int kPer = (kSliceMfma + kHalf - 1) / kHalf;
    __builtin_amdgcn_sched_group_barrier(0x100, kFB + kTB, 0);
#pragma unroll
    for (int i = 0; i < kHalf; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, kPer, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x100, kFB + kTB, 0);
#pragma unroll
    for (int i = 0; i < kLoads - kHalf; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, kPer, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 2 * kSliceMfma, 0);
    __builtin_amdgcn_sched_group_barrier(0x200, kLoads, 0);
    __syncthreads();
  };

  using Set0 = std::integral_constant<int, 0>;
  using Set1 = std::integral_constant<int, 1>;
  load_step(0, Set0{});
  load_step(1, Set1{});
  store_step(Set0{}, 0);
  __syncthreads();
  for (int step = 0; step < steps; step += 2) {
    iteration(step, Set0{});
    iteration(step + 1, Set1{});
  }

  // Lane holds output columns (weight rows) 4 quarter + i of each block for
  // x row row16 of each x block.
#pragma unroll
  for (int tb = 0; tb < kTB; ++tb) {
    const int token = m0 + kWM * wm + 16 * tb + row16;
    if (token >= a.rows) continue;
    uint16_t* out_row = a.out + static_cast<int64_t>(token) * a.out_stride;
#pragma unroll
    for (int fb = 0; fb < kFB; ++fb) {
      const int col = weight_row(block_lds_row(fb)) + 4 * quarter;
      if (col < a.n)
        *reinterpret_cast<uint2*>(out_row + col) =
            make_uint2(pack_bf16x2(acc[fb][tb][0], acc[fb][tb][1]), pack_bf16x2(acc[fb][tb][2], acc[fb][tb][3]));
    }
    if (paired && a.act != nullptr) {
#pragma unroll
      for (int fb = 0; fb < 2; ++fb) {
        float g[4], u[4], v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          g[i] = bf16_to_f32(f32_to_bf16(acc[fb][tb][i]));
          u[i] = bf16_to_f32(f32_to_bf16(acc[fb + 2][tb][i]));
        }
        silu_mul_values<4>(g, u, v);
        const int col = weight_row(block_lds_row(fb)) + 4 * quarter;  // a gate row: the act column
        *reinterpret_cast<uint2*>(a.act + static_cast<int64_t>(token) * a.act_stride + col) =
            make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
      }
    }
  }
}

bool aligned_to(const void* p, uintptr_t bytes) { return (reinterpret_cast<uintptr_t>(p) % bytes) == 0; }

}  // namespace
}  // namespace d3

using namespace d3;

extern "C" int d3_dense_bf16(const uint16_t* x, int64_t x_stride, int32_t rows, const uint16_t* w,
                             int32_t n, int32_t k, int32_t pair_rows, uint16_t* out,
                             int64_t out_stride, uint16_t* act, int64_t act_stride, void* stream) {
  D3_REQUIRE(rows == 0 || (x && w && out), "dense_bf16: null pointer");
  D3_REQUIRE(rows >= 0 && n > 0 && k > 0 && pair_rows >= 0 && 2 * pair_rows <= n,
             "dense_bf16: rows %d, N %d, K %d, pair_rows %d", rows, n, k, pair_rows);
  D3_SUPPORTED(n % 16 == 0 && pair_rows % 16 == 0, "dense_bf16: N=%d and pair_rows %d must be multiples of 16",
               n, pair_rows);
  D3_REQUIRE(x_stride >= k && out_stride >= n && (act == nullptr || act_stride >= pair_rows),
             "dense_bf16: row strides");
  D3_REQUIRE(aligned_to(x, 16) && x_stride % 8 == 0 && aligned_to(w, 16) && aligned_to(out, 8) &&
                 out_stride % 4 == 0 && (act == nullptr || (aligned_to(act, 8) && act_stride % 4 == 0)),
             "dense_bf16: x / w rows must be 16-byte aligned, out / act rows 8-byte");
  D3_SUPPORTED(static_cast<int64_t>(rows) * x_stride * 2 < (int64_t{1} << 31) &&
                   static_cast<int64_t>(n) * k * 2 < (int64_t{1} << 31),
               "dense_bf16: operands above 2 GiB");
  const int chunks = k / kDenseChunk;
  const bool small_k = k % kDenseChunk == 0 && (chunks == 1 || chunks == 2 || chunks == 3 || chunks == 4 ||
                                                 chunks == 6 || chunks == 8);
  const bool small = rows < kTiledMinRows && small_k;
  if (!small) {
    D3_SUPPORTED(k % kTiledK == 0, "dense_bf16: K=%d must be a multiple of %d above %d rows (or in {256, 512, "
                 "768, 1024, 1536, 2048})", k, kTiledK, kTiledMinRows - 1);
    D3_SUPPORTED(pair_rows % kTiledPairRows == 0,
                 "dense_bf16: pair_rows %d must be a multiple of %d above %d rows", pair_rows, kTiledPairRows,
                 kTiledMinRows - 1);
  }
  if (rows == 0) {
    clear_error();
    return D3_OK;
  }
  const int pairs = pair_rows / 16;
  const DenseArgs args{x, x_stride, rows, w, n, k, out, out_stride, pairs, pair_rows, act, act_stride};
  hipStream_t s = as_stream(stream);
  if (!small) {
    TiledGrid g{};
    g.pair_tiles = pair_rows / kTiledPairRows;
    g.n_tiles = g.pair_tiles + (n - 2 * pair_rows + kTiledN - 1) / kTiledN;
    // 128-row x tiles when they already give every CU a workgroup, else 64
    const int tiles128 = (rows + 127) / 128 * g.n_tiles;
    const bool wide = tiles128 >= 256;
    g.m_tiles = wide ? (rows + 127) / 128 : (rows + 63) / 64;
    const int total = g.m_tiles * g.n_tiles;
    g.per_xcd = (total + kTiledXcds - 1) / kTiledXcds;
    const dim3 grid(g.per_xcd * kTiledXcds), block(kTiledThreads);
    if (wide)
      hipLaunchKernelGGL(dense_bf16_tiled_kernel<128>, grid, block, 0, s, args, g);
    else
      hipLaunchKernelGGL(dense_bf16_tiled_kernel<64>, grid, block, 0, s, args, g);
    D3_LAUNCHED("dense_bf16");
  }
  const int rest = n / 16 - 2 * pairs;
  const dim3 grid(pairs + (rest + 1) / 2, (rows + kDenseTokens - 1) / kDenseTokens), block(kDenseThreads);
  switch (k / kDenseChunk) {
    case 1: hipLaunchKernelGGL(dense_bf16_kernel<1>, grid, block, 0, s, args); break;
    case 2: hipLaunchKernelGGL(dense_bf16_kernel<2>, grid, block, 0, s, args); break;
    case 3: hipLaunchKernelGGL(dense_bf16_kernel<3>, grid, block, 0, s, args); break;
    case 4: hipLaunchKernelGGL(dense_bf16_kernel<4>, grid, block, 0, s, args); break;
    case 6: hipLaunchKernelGGL(dense_bf16_kernel<6>, grid, block, 0, s, args); break;
    default: hipLaunchKernelGGL(dense_bf16_kernel<8>, grid, block, 0, s, args); break;
  }
  D3_LAUNCHED("dense_bf16");
}
