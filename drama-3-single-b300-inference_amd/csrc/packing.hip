// Ragged-batch bookkeeping around the MoE rows: packed-prefill row metadata
// (cu_seqlens -> sequence, position, slot, next-frame labels) and the
// per-slot request state gather / update of persistent decode slots.
// Integer-only, one thread per row (metadata) or one wave per row (state).
#include "common.h"
#include "status.h"

namespace d3 {
namespace {

constexpr int kThreads = 256;

__global__ __launch_bounds__(kThreads) void row_metadata_kernel(
    const int32_t* __restrict__ cu, const int64_t* __restrict__ slots, int sequences,
    int capacity, const int64_t* __restrict__ frames, int codes, int64_t eos,
    int64_t* __restrict__ positions, int64_t* __restrict__ row_slots,
    int64_t* __restrict__ labels) {
  const int row = blockIdx.x * kThreads + threadIdx.x;
  if (row >= capacity) return;
  // Sequence index: number of interior boundaries at or below the row
  // (packed_prefill.py:63-66).
  int sequence = 0;
  for (int i = 1; i < sequences; ++i) sequence += row >= cu[i];
  const int start = cu[sequence];
  const int end = cu[sequence + 1];
  positions[row] = row - start;
  row_slots[row] = slots[sequence];
  if (labels != nullptr) {
    // frames holds `capacity` rows: never read past it, even when the
    // boundaries describe more rows than the buffer has.
    const bool next = row + 1 < end && row + 1 < capacity;
    for (int c = 0; c < codes; ++c) {
      const int64_t fallback = c == 0 ? eos : 0;
      labels[static_cast<int64_t>(row) * codes + c] =
          next ? frames[static_cast<int64_t>(row + 1) * codes + c] : fallback;
    }
  }
}

constexpr int kFrame = 11;    // main token + 10 acoustic codes
constexpr int kHistory = 16;  // main-token history window

// DeviceRequests._load (runtime_state.py:10-32): one wave per row.
__global__ __launch_bounds__(kThreads) void requests_load_kernel(
    const int64_t* __restrict__ last, const int64_t* __restrict__ history,
    const int64_t* __restrict__ metadata, const int64_t* __restrict__ slots, int rows,
    int64_t max_length, int64_t padding_start, int64_t* __restrict__ frames_out,
    int64_t* __restrict__ history_out, int64_t* __restrict__ positions_out) {
  const int row = (blockIdx.x * kThreads + threadIdx.x) / kWave;
  const int lane = lane_id();
  if (row >= rows) return;
  const int64_t slot = slots[row];
  if (lane < kFrame) frames_out[static_cast<int64_t>(row) * kFrame + lane] = last[slot * kFrame + lane];
  if (lane < kHistory)
    history_out[static_cast<int64_t>(row) * kHistory + lane] = history[slot * kHistory + lane];
  if (lane == 0) {
    int64_t position = metadata[slot * 4];
    if (padding_start >= 0 && slot >= padding_start) position = 0;
    positions_out[row] = position < max_length - 1 ? position : max_length - 1;
  }
}

// DeviceRequests._save (runtime_state.py:35-56): one wave per row.
__global__ __launch_bounds__(kThreads) void requests_save_kernel(
    int64_t* __restrict__ last, int64_t* __restrict__ history, int64_t* __restrict__ metadata,
    int64_t* __restrict__ codes, const int64_t* __restrict__ slots, int rows,
    const int64_t* __restrict__ output, int64_t eos, int64_t limit_frames) {
  const int row = (blockIdx.x * kThreads + threadIdx.x) / kWave;
  const int lane = lane_id();
  if (row >= rows) return;
  const int64_t slot = slots[row];
  const int64_t* frame = output + static_cast<int64_t>(row) * kFrame;
  const int64_t main = frame[0];
  const int64_t position = metadata[slot * 4];
  int64_t count = metadata[slot * 4 + 1];
  const int64_t limit = metadata[slot * 4 + 2];
  const int64_t done = metadata[slot * 4 + 3];
  const bool append = done == 0 && main != eos && count < limit;
  // Read the shifted history before any lane overwrites it.
  const int64_t shifted = lane < kHistory - 1 ? history[slot * kHistory + lane + 1]
                                              : (lane == kHistory - 1 ? main : -1);
  if (append) {
    if (lane < kFrame) last[slot * kFrame + lane] = frame[lane];
    if (lane < kHistory) history[slot * kHistory + lane] = shifted;
    if (lane < kFrame - 1 && count < limit_frames)
      codes[(slot * limit_frames + count) * (kFrame - 1) + lane] = frame[lane + 1];
  }
  if (lane == 0) {
    count += append ? 1 : 0;
    metadata[slot * 4] = position + (append ? 1 : 0);
    metadata[slot * 4 + 1] = count;
    metadata[slot * 4 + 3] = done | (main == eos ? 1 : 0) | (count >= limit ? 1 : 0);
  }
}

}  // namespace
}  // namespace d3

using namespace d3;

extern "C" int d3_row_metadata(const int32_t* cu_seqlens, const int64_t* sequence_slots,
                               int32_t sequences, int32_t capacity, const int64_t* frames,
                               int32_t codes, int64_t eos, int64_t* positions,
                               int64_t* row_slots, int64_t* labels, void* stream) {
  D3_REQUIRE(cu_seqlens && sequence_slots && positions && row_slots, "row_metadata: null pointer");
  D3_REQUIRE(sequences >= 1 && capacity >= 0, "row_metadata: need at least one sequence");
  D3_REQUIRE(labels == nullptr || (frames != nullptr && codes >= 1),
             "row_metadata: labels need frames and codes >= 1");
  if (capacity == 0) {
    clear_error();
    return D3_OK;
  }
  hipLaunchKernelGGL(row_metadata_kernel, dim3((capacity + kThreads - 1) / kThreads),
                     dim3(kThreads), 0, as_stream(stream), cu_seqlens, sequence_slots, sequences,
                     capacity, frames, codes, eos, positions, row_slots, labels);
  D3_LAUNCHED("row_metadata");
}

extern "C" int d3_requests_load(const int64_t* last, const int64_t* history,
                                const int64_t* metadata, const int64_t* slots, int32_t rows,
                                int64_t max_length, int64_t padding_start, int64_t* frames_out,
                                int64_t* history_out, int64_t* positions_out, void* stream) {
  D3_REQUIRE(last && history && metadata && slots && frames_out && history_out && positions_out,
             "requests_load: null pointer");
  D3_REQUIRE(rows >= 0 && max_length >= 1, "requests_load: bad rows/max_length");
  if (rows == 0) {
    clear_error();
    return D3_OK;
  }
  const int blocks = (rows + kThreads / kWave - 1) / (kThreads / kWave);
  hipLaunchKernelGGL(requests_load_kernel, dim3(blocks), dim3(kThreads), 0, as_stream(stream),
                     last, history, metadata, slots, rows, max_length, padding_start, frames_out,
                     history_out, positions_out);
  D3_LAUNCHED("requests_load");
}

extern "C" int d3_requests_save(int64_t* last, int64_t* history, int64_t* metadata, int64_t* codes,
                                const int64_t* slots, int32_t rows, const int64_t* output,
                                int64_t eos, int64_t limit, void* stream) {
  D3_REQUIRE(last && history && metadata && codes && slots && output,
             "requests_save: null pointer");
  D3_REQUIRE(rows >= 0 && limit >= 1, "requests_save: bad rows/limit");
  if (rows == 0) {
    clear_error();
    return D3_OK;
  }
  const int blocks = (rows + kThreads / kWave - 1) / (kThreads / kWave);
  hipLaunchKernelGGL(requests_save_kernel, dim3(blocks), dim3(kThreads), 0, as_stream(stream),
                     last, history, metadata, codes, slots, rows, output, eos, limit);
  D3_LAUNCHED("requests_save");
}
