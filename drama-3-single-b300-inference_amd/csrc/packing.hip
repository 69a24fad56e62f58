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

// ---------------------------------------------------------------------------
// Mixed decode + prefill rows (one workgroup).  Row space: decode rows
// [0, decode_rows) then the packed prefill suffix [decode_rows, full).
// ---------------------------------------------------------------------------
constexpr int kMixedThreads = 1024;
constexpr int kMixedWaves = kMixedThreads / kWave;
constexpr int kMixedMaxRows = 8192;   // row space with prefix reuse (LDS owner table)
constexpr int kMixedMaxPrompts = 16;  // prompts compared for prefix reuse
constexpr int kMixedMaxBounds = 1025; // boundaries staged in LDS (1024 sequences)
constexpr int kMixedMaxCodes = 16;    // frame codes compared from registers
constexpr int kMixedCodeParts = 4;    // threads per (pair, row) comparison, each a quarter of the codes
constexpr int kMixedPartCodes = kMixedMaxCodes / kMixedCodeParts;
constexpr int kMixedMaxPairs = kMixedMaxPrompts * (kMixedMaxPrompts - 1) / 2;  // 120

// Exclusive rank of `flag` among the workgroup's threads (thread order) and
// the workgroup's total.  Two LDS barriers; `wave_counts` is free again on
// return.
__device__ __forceinline__ int block_rank(bool flag, int* wave_counts, int* total) {
  const int wave = threadIdx.x / kWave;
  const uint64_t mask = __ballot(flag);
  if (lane_id() == 0) wave_counts[wave] = __popcll(mask);
  lds_barrier();
  int before = 0, all = 0;
  for (int w = 0; w < kMixedWaves; ++w) {
    before += w < wave ? wave_counts[w] : 0;
    all += wave_counts[w];
  }
  lds_barrier();
  *total = all;
  return before + __popcll(mask & lanemask_lt());
}

// One mixed step's rows on the device (the host-side preparation of
// mixed_graph.py:139-179 and the prefix-reuse ownership of
// row_reuse.py:74-101, from device data so that a captured graph needs no
// host sync):
//   1. occupied slots, ascending (active / count), and the decode rows'
//      slots: the first min(count, decode_rows) occupied slots, then
//      padding_start + j for the remaining rows j;
//   2. with frames: prompt i (suffix rows [b[i], b[i+1])) aliases its first
//      L rows to the same positions of the earliest earlier prompt j with the
//      longest agreeing leading run L (every code compared); owners chain to
//      canonical rows because prompts are processed in order;
//   3. live rows (occupied decode rows, suffix rows below b[prompts]) that
//      own themselves are the MoE rows (keep, ascending; keep_count); every
//      live row reads back its owner's MoE row (inverse), other rows row 0.
// Boundaries are clamped to [0, capacity] and made non-decreasing, so every
// frame read stays inside the suffix's capacity rows.
__global__ __launch_bounds__(kMixedThreads) void mixed_rows_kernel(
    const uint8_t* __restrict__ occupancy, int num_slots, int decode_rows, int64_t padding_start,
    const int32_t* __restrict__ boundaries, int prompts, int capacity,
    const int64_t* __restrict__ frames, int codes, const int64_t* __restrict__ sequence_slots,
    int sequences, int32_t* __restrict__ active, int32_t* __restrict__ count,
    int64_t* __restrict__ decode_slots, int32_t* __restrict__ keep,
    int32_t* __restrict__ keep_count, int64_t* __restrict__ inverse,
    int64_t* __restrict__ positions, int64_t* __restrict__ row_slots) {
  __shared__ int32_t owner_of[kMixedMaxRows];  // owner row; -(rank + 1) once kept
  __shared__ int wave_counts[kMixedWaves];
  __shared__ int starts[kMixedMaxPrompts + 1];
  __shared__ int common[kMixedMaxPrompts * kMixedMaxPrompts];
  __shared__ int bounds[kMixedMaxBounds];
  __shared__ int first[kMixedMaxPairs + 1];
  __shared__ int64_t sequence_slot[kMixedMaxBounds - 1];
  const int tid = static_cast<int>(threadIdx.x);
  const int full = decode_rows + capacity;
  const bool reuse = frames != nullptr && prompts >= 2;
  // Every boundary read below goes to this LDS copy (one parallel load; a
  // loop over global boundaries pays a memory round trip per entry).  The
  // compaction's barriers order it before its first use.
  // The first 1024 slots' occupancy is loaded with the boundaries (at most
  // 1025 of them: two per thread), every load before the first use: one
  // memory round trip instead of one for each.
  const int nbounds = (prompts > sequences ? prompts : sequences) + 1;
  const int bound0 = tid < nbounds ? boundaries[tid] : 0;
  const int bound1 = tid + kMixedThreads < nbounds ? boundaries[tid + kMixedThreads] : 0;
  const uint8_t occupancy0 = tid < num_slots ? occupancy[tid] : 0;
  // the suffix sequences' slots (positions only; sequences <= 1024)
  const int64_t slot_of = positions != nullptr && tid < sequences ? sequence_slots[tid] : 0;
  if (tid < nbounds) bounds[tid] = bound0;
  if (tid + kMixedThreads < nbounds) bounds[tid + kMixedThreads] = bound1;
  if (positions != nullptr && tid < sequences) sequence_slot[tid] = slot_of;
  // Threads exchange data through LDS only (inputs are read, outputs
  // written once), so every barrier here is an LDS barrier: global loads
  // stay in flight across them.
  lds_barrier();  // bounds written

  // b[prompts] after clamping: the largest clamped boundary.
  int live_prefill = 0;
  for (int i = 0; i <= prompts; ++i) {
    const int b = bounds[i];
    const int clamped = b > capacity ? capacity : b;
    live_prefill = clamped > live_prefill ? clamped : live_prefill;
  }

  // 2a. Prefix reuse set-up from the boundaries alone: clamped, non-
  //     decreasing starts; for every pair (i, j), j < i, its comparable
  //     length common[i][j] (the shorter prompt's) and its first flat
  //     comparison index first[q].  Each thread then issues the frame loads
  //     of its first comparison unit, which stay in flight through the slot
  //     compaction below.
  const int pairs = reuse ? prompts * (prompts - 1) / 2 : 0;
  if (reuse) {
    if (tid == 0) {
      int previous = 0;
      for (int i = 0; i <= prompts; ++i) {
        int b = bounds[i];
        b = b < previous ? previous : (b > capacity ? capacity : b);
        starts[i] = b;
        previous = b;
      }
      int sum = 0;
      for (int q = 0, i = 1, base = 0; q < pairs; ++q) {
        if (q - base == i) base += i++;  // pair q = (i, q - base)
        const int j = q - base;
        const int li = starts[i + 1] - starts[i], lj = starts[j + 1] - starts[j];
        const int n = li < lj ? li : lj;
        common[i * kMixedMaxPrompts + j] = n;
        first[q] = sum;
        sum += n;
      }
      first[pairs] = sum;
    }
    lds_barrier();
  }
  const int compares = reuse ? first[pairs] : 0;
  // The pair (i, j) and row p of flat comparison f.
  auto comparison = [&](int f, int& i, int& j, int& p) {
    int q = 0;  // the pair holding f: last q with first[q] <= f
    for (int step = 64; step >= 1; step >>= 1)  // pairs <= 120 < 128
      if (q + step < pairs && first[q + step] <= f) q += step;
    int base = 0;
    i = 1;
    while (base + i <= q) base += i++;
    j = q - base;
    p = f - first[q];
  };
  // Comparison unit u = kMixedCodeParts f + part: codes part, part + 4, ...
  // of comparison f.  A thread's first unit (u = tid) is loaded here.
  const int units = compares * kMixedCodeParts;
  // (uniform; with at least one comparison, frame row 0 exists)
  const bool registered = reuse && codes <= kMixedMaxCodes && compares > 0;
  int64_t va[kMixedPartCodes], vb[kMixedPartCodes];
  int fi = 0, fj = 0, fp = 0;
  const bool preloaded = registered && tid < units;
  if (registered) {
    // Branch-free loads (a thread without a unit, or a code past `codes`,
    // reads frame row 0 / code 0 and ignores it): all of them are in
    // flight before the compaction's first barrier.
    if (preloaded) comparison(tid / kMixedCodeParts, fi, fj, fp);
    const int64_t* a = frames + (preloaded ? static_cast<int64_t>(starts[fi] + fp) * codes : 0);
    const int64_t* b = frames + (preloaded ? static_cast<int64_t>(starts[fj] + fp) * codes : 0);
#pragma unroll
    for (int m = 0; m < kMixedPartCodes; ++m) {
      const int c = tid % kMixedCodeParts + m * kMixedCodeParts;
      va[m] = a[c < codes ? c : 0];
      vb[m] = b[c < codes ? c : 0];
    }
  }

  // 1. slot compaction and decode row slots
  int occupied = 0;
  for (int start = 0; start < num_slots; start += kMixedThreads) {
    const int slot = start + tid;
    const bool live = slot < num_slots && (start == 0 ? occupancy0 : occupancy[slot]) != 0;
    int chunk;
    const int at = occupied + block_rank(live, wave_counts, &chunk);
    if (live) {
      active[at] = slot;
      if (at < decode_rows) decode_slots[at] = slot;
    }
    occupied += chunk;
  }
  for (int i = occupied + tid; i < num_slots; i += kMixedThreads) active[i] = -1;
  const int used = occupied < decode_rows ? occupied : decode_rows;
  for (int j = used + tid; j < decode_rows; j += kMixedThreads) decode_slots[j] = padding_start + j;
  if (tid == 0) *count = occupied;

  // 2b. prefix ownership: prompt i (suffix rows [b[i], b[i+1])) aliases its
  //     first L rows to the earliest earlier prompt with the longest
  //     agreeing leading run L.  Every (pair, row) comparison of all pairs
  //     at once, a quarter of its codes per thread, so the frames cost one
  //     memory round trip per 256 rows rather than one per 64 rows of each
  //     pair (and the first of them overlaps the compaction).
  if (reuse) {
    for (int r = tid; r < full; r += kMixedThreads) owner_of[r] = r;
    if (registered) {
      for (int u = tid; u < units; u += kMixedThreads) {
        const int part = u % kMixedCodeParts;
        int i, j, p;
        bool differ = false;
        if (u == tid) {
          i = fi;
          j = fj;
          p = fp;
#pragma unroll
          for (int m = 0; m < kMixedPartCodes; ++m) {
            // compared here, after the compaction (not where they were loaded)
            asm volatile("" : "+v"(va[m]), "+v"(vb[m]));
            differ |= part + m * kMixedCodeParts < codes && va[m] != vb[m];
          }
        } else {
          comparison(u / kMixedCodeParts, i, j, p);
          const int64_t* a = frames + static_cast<int64_t>(starts[i] + p) * codes;
          const int64_t* b = frames + static_cast<int64_t>(starts[j] + p) * codes;
          int64_t xa[kMixedPartCodes], xb[kMixedPartCodes];
#pragma unroll
          for (int m = 0; m < kMixedPartCodes; ++m) {
            const int c = part + m * kMixedCodeParts;
            xa[m] = a[c < codes ? c : 0];
            xb[m] = b[c < codes ? c : 0];
          }
#pragma unroll
          for (int m = 0; m < kMixedPartCodes; ++m) differ |= part + m * kMixedCodeParts < codes && xa[m] != xb[m];
        }
        if (differ) atomicMin(&common[i * kMixedMaxPrompts + j], p);
      }
    } else {
      for (int f = tid; f < compares; f += kMixedThreads) {
        int i, j, p;
        comparison(f, i, j, p);
        const int64_t* a = frames + static_cast<int64_t>(starts[i] + p) * codes;
        const int64_t* b = frames + static_cast<int64_t>(starts[j] + p) * codes;
        bool differ = false;
        for (int c = 0; c < codes; ++c) differ |= a[c] != b[c];
        if (differ) atomicMin(&common[i * kMixedMaxPrompts + j], p);
      }
    }
    lds_barrier();
    for (int i = 1; i < prompts; ++i) {
      int longest = 0, source = 0;
      for (int j = 0; j < i; ++j) {
        const int n = common[i * kMixedMaxPrompts + j];
        if (n > longest) {
          longest = n;
          source = j;
        }
      }
      for (int p = tid; p < longest; p += kMixedThreads)
        owner_of[decode_rows + starts[i] + p] = owner_of[decode_rows + starts[source] + p];
      lds_barrier();
    }
  }

  // Optional: the suffix rows' positions and slots, row_metadata_kernel's
  // rule on the raw boundaries (sequences + 1 of them).
  if (positions != nullptr) {
    for (int r = tid; r < capacity; r += kMixedThreads) {
      int sequence = 0;
      for (int i = 1; i < sequences; ++i) sequence += r >= bounds[i];
      positions[r] = r - bounds[sequence];
      row_slots[r] = sequence_slot[sequence];
    }
  }

  // 3. MoE rows and the read-back map
  int kept_total = 0;
  for (int start = 0; start < full; start += kMixedThreads) {
    const int r = start + tid;
    const bool in = r < full;
    const bool live = in && (r < decode_rows ? r < used : r - decode_rows < live_prefill);
    const int owner = reuse && in ? owner_of[r] : r;
    const bool kept = live && owner == r;
    int chunk;
    const int at = kept_total + block_rank(kept, wave_counts, &chunk);
    if (kept) {
      keep[at] = r;
      if (reuse) owner_of[r] = -(at + 1);
    }
    if (reuse) lds_barrier();
    if (in) {
      int64_t back = 0;
      if (live) {
        if (reuse) {
          const int s = owner_of[owner];
          back = s < 0 ? -(s + 1) : 0;
        } else {
          back = at;
        }
      }
      inverse[r] = back;
    }
    kept_total += chunk;
  }
  for (int i = kept_total + tid; i < full; i += kMixedThreads) keep[i] = 0;
  if (tid == 0) *keep_count = kept_total;
}

}  // namespace
}  // namespace d3

using namespace d3;

extern "C" int d3_mixed_rows(const uint8_t* occupancy, int32_t num_slots, int32_t decode_rows,
                             int64_t padding_start, const int32_t* boundaries, int32_t prompts,
                             int32_t capacity, const int64_t* frames, int32_t codes,
                             const int64_t* sequence_slots, int32_t sequences,
                             int32_t* active_slots, int32_t* count, int64_t* decode_slots,
                             int32_t* keep, int32_t* keep_count, int64_t* inverse,
                             int64_t* positions, int64_t* row_slots, void* stream) {
  D3_REQUIRE(occupancy && boundaries && active_slots && count && keep && keep_count && inverse,
             "mixed_rows: null pointer");
  D3_REQUIRE(decode_rows == 0 || decode_slots, "mixed_rows: null decode_slots");
  D3_REQUIRE(num_slots > 0 && num_slots <= (1 << 20), "mixed_rows: num_slots out of range");
  D3_REQUIRE(decode_rows >= 0 && capacity >= 0 && prompts >= 0,
             "mixed_rows: negative decode_rows, capacity or prompts");
  const int64_t full = static_cast<int64_t>(decode_rows) + capacity;
  D3_REQUIRE(full >= 1 && full <= (1 << 30), "mixed_rows: %lld rows out of range",
             static_cast<long long>(full));
  D3_REQUIRE(frames == nullptr || codes >= 1, "mixed_rows: frames need codes >= 1");
  D3_REQUIRE(positions == nullptr ||
                 (row_slots && sequence_slots && sequences >= 1 && sequences >= prompts),
             "mixed_rows: row metadata needs row_slots, sequence_slots and sequences >= prompts");
  if (positions == nullptr) sequences = 0;
  D3_SUPPORTED(prompts < kMixedMaxBounds && sequences < kMixedMaxBounds,
               "mixed_rows: %d prompts / %d sequences (max %d)", prompts, sequences,
               kMixedMaxBounds - 1);
  if (frames != nullptr && prompts >= 2) {
    D3_SUPPORTED(prompts <= kMixedMaxPrompts, "mixed_rows: prefix reuse over %d prompts (max %d)",
                 prompts, kMixedMaxPrompts);
    D3_SUPPORTED(full <= kMixedMaxRows, "mixed_rows: prefix reuse over %lld rows (max %d)",
                 static_cast<long long>(full), kMixedMaxRows);
  }
  hipLaunchKernelGGL(mixed_rows_kernel, dim3(1), dim3(kMixedThreads), 0, as_stream(stream),
                     occupancy, num_slots, decode_rows, padding_start, boundaries, prompts,
                     capacity, frames, codes, sequence_slots, sequences, active_slots, count,
                     decode_slots, keep, keep_count, inverse, positions, row_slots);
  D3_LAUNCHED("mixed_rows");
}

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
