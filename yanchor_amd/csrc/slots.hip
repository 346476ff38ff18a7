// Continuous-batch slot management on the GPU: per-step bookkeeping, cu_seqlens
// packing, stable slot selection (refill targets / compaction keep-lists) and
// multi-tensor row gather/scatter for cache compaction and refill.
//
// Replaces (runtime/model/inference_kernels.py):
//   _qwen35_decode_state_update_kernel / _update_fixed_decode_state_ 1169-1208
//   torch.nonzero(finished) refill targets                          1549
//   torch.nonzero(~finished & slot_rows >= 0) compaction keep-list   1725
// and the row ops of the fixed-memory caches (modeling_yanchor.py:540-554,
// 647-683, 723-731: batch_select_indices / batch_scatter_from), plus the
// cu_seqlens exclusive scan of packed varlen prefill.
#include "common.h"

namespace yh {
namespace {

constexpr int kScanThreads = 1024;
constexpr int kScanWaves = kScanThreads / kWave;

// Block-wide exclusive scan of one int64 per thread; returns the exclusive
// prefix and writes the block total to *total.
__device__ __forceinline__ int64_t block_exclusive_scan(int64_t x, int64_t* total) {
  __shared__ int64_t wsum[kScanWaves];
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
  int64_t incl = x;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int64_t y = __shfl_up(incl, off, kWave);
    if (lane >= off) incl += y;
  }
  if (lane == kWave - 1) wsum[wid] = incl;
  __syncthreads();
  int64_t before = 0, all = 0;
  for (int w = 0; w < kScanWaves; ++w) {
    before += w < wid ? wsum[w] : 0;
    all += wsum[w];
  }
  __syncthreads();  // wsum may be reused by the next call
  *total = all;
  return before + incl - x;
}

struct BookArgs {
  const int64_t* sampled;      // [S] (tokens [S, 1])
  int32_t* storage;            // [R, W]
  uint8_t* dense_seen;         // [S, V]
  int64_t* generated_lengths;  // [R]
  uint8_t* finished_by_eos;    // [R]
  uint8_t* finished;           // [S]
  const int64_t* slot_rows;    // [S]
  const int64_t* sink_rows;    // [S]
  const int64_t* slot_caps;    // [S]
  int64_t* row_steps;          // [S]
  int64_t* row_positions;      // [S]
  int64_t* decode_ids;         // [S] (tokens [S, 1])
  int64_t* useful_events;      // scalar
  int64_t slots, storage_rows, storage_width, seen_width, max_new;
  int64_t pad, eos0, eos1;
  int eos_count;
};

// One workgroup walks all slots (the reference runs one program); every store
// is bounds-checked against the tensor it targets.
__global__ void __launch_bounds__(kScanThreads) bookkeeping_kernel(BookArgs a) {
  int64_t useful = 0;
  for (int64_t r = threadIdx.x; r < a.slots; r += kScanThreads) {
    const int64_t sampled = a.sampled[r];
    const bool fin = a.finished[r] != 0;
    const int64_t slot_row = a.slot_rows[r];
    const bool active = !fin && slot_row >= 0;
    const int64_t step = a.row_steps[r];
    const int64_t write_row = active ? slot_row : a.sink_rows[r];
    const int64_t write_col = active ? step : a.max_new;
    const int64_t stored = active ? sampled : a.pad;
    const bool row_ok = write_row >= 0 && write_row < a.storage_rows;
    if (row_ok && write_col >= 0 && write_col < a.storage_width)
      a.storage[write_row * a.storage_width + write_col] = static_cast<int32_t>(stored);
    if (stored >= 0 && stored < a.seen_width) a.dense_seen[r * a.seen_width + stored] = 1;
    const int64_t next_step = step + (active ? 1 : 0);
    if (row_ok && active) a.generated_lengths[write_row] = next_step;
    const bool is_eos = (a.eos_count >= 1 && stored == a.eos0) || (a.eos_count >= 2 && stored == a.eos1);
    if (row_ok && active && is_eos) a.finished_by_eos[write_row] = 1;
    const bool next_fin = fin || (active && (is_eos || next_step >= a.slot_caps[r]));
    a.finished[r] = next_fin ? 1 : 0;
    a.row_steps[r] = next_step;
    a.row_positions[r] += active ? 1 : 0;
    a.decode_ids[r] = next_fin ? a.pad : stored;
    useful += active ? 1 : 0;
  }
  int64_t total = 0;
  (void)block_exclusive_scan(useful, &total);
  if (threadIdx.x == 0) *a.useful_events += total;
}

// cu[0] = 0, cu[i + 1] = lengths[0] + ... + lengths[i]
__global__ void __launch_bounds__(kScanThreads) cu_seqlens_kernel(const void* lengths, int len_i64, int32_t* cu,
                                                                  int64_t n) {
  int64_t carry = 0;
  if (threadIdx.x == 0) cu[0] = 0;
  for (int64_t base = 0; base < n; base += kScanThreads) {
    const int64_t i = base + threadIdx.x;
    int64_t x = 0;
    if (i < n) x = len_i64 ? static_cast<const int64_t*>(lengths)[i] : static_cast<const int32_t*>(lengths)[i];
    int64_t total = 0;
    const int64_t excl = block_exclusive_scan(x, &total);
    if (i < n) cu[i + 1] = static_cast<int32_t>(carry + excl + x);
    carry += total;
  }
}

// Ascending indices i with pred(i); mode 0: !finished[i] && slot_rows[i] >= 0
// (compaction keep-list), mode 1: finished[i] (refill targets).  Unused tail
// entries are -1; *count receives the number selected.
__global__ void __launch_bounds__(kScanThreads) select_slots_kernel(const uint8_t* finished, const int64_t* slot_rows,
                                                                    int mode, int64_t* out, int64_t* count,
                                                                    int64_t n) {
  int64_t carry = 0;
  for (int64_t base = 0; base < n; base += kScanThreads) {
    const int64_t i = base + threadIdx.x;
    bool take = false;
    if (i < n) take = mode == 0 ? (finished[i] == 0 && slot_rows[i] >= 0) : (finished[i] != 0);
    int64_t total = 0;
    const int64_t excl = block_exclusive_scan(take ? 1 : 0, &total);
    if (take) out[carry + excl] = i;
    carry += total;
  }
  __syncthreads();
  for (int64_t i = carry + threadIdx.x; i < n; i += kScanThreads) out[i] = -1;
  if (threadIdx.x == 0) *count = carry;
}

constexpr int kMaxCopyTensors = 32;
constexpr int kCopyThreads = 256;
constexpr int64_t kCopyChunk = 64 * 1024;  // bytes per block

struct CopyArgs {
  const char* src[kMaxCopyTensors];
  char* dst[kMaxCopyTensors];
  int64_t row_bytes[kMaxCopyTensors];
  int64_t src_rows[kMaxCopyTensors];
  int64_t dst_rows[kMaxCopyTensors];
  const int64_t* src_index;  // [n] or null (identity)
  const int64_t* dst_index;  // [n] or null (identity)
  int64_t n;
};

// grid (chunks of the widest row, n rows, tensors): dst_t[dst_index[i]] =
// src_t[src_index[i]], 16-byte copies when row and pointers allow, else bytes.
__global__ void __launch_bounds__(kCopyThreads) gather_rows_kernel(CopyArgs a) {
  const int t = blockIdx.z;
  const int64_t i = blockIdx.y;
  const int64_t rb = a.row_bytes[t];
  const int64_t off = static_cast<int64_t>(blockIdx.x) * kCopyChunk;
  if (off >= rb) return;
  const int64_t si = a.src_index ? a.src_index[i] : i;
  const int64_t di = a.dst_index ? a.dst_index[i] : i;
  if (si < 0 || si >= a.src_rows[t] || di < 0 || di >= a.dst_rows[t]) return;
  const char* s = a.src[t] + si * rb + off;
  char* d = a.dst[t] + di * rb + off;
  const int64_t len = rb - off < kCopyChunk ? rb - off : kCopyChunk;
  if (((reinterpret_cast<uintptr_t>(s) | reinterpret_cast<uintptr_t>(d) | static_cast<uintptr_t>(len)) & 15) == 0) {
    const uint4* s4 = reinterpret_cast<const uint4*>(s);
    uint4* d4 = reinterpret_cast<uint4*>(d);
    for (int64_t k = threadIdx.x; k < len / 16; k += kCopyThreads) d4[k] = s4[k];
  } else {
    for (int64_t k = threadIdx.x; k < len; k += kCopyThreads) d[k] = s[k];
  }
}

}  // namespace
}  // namespace yh

extern "C" int yh_decode_bookkeeping(const int64_t* sampled_token, int32_t* storage, uint8_t* dense_seen,
                                     int64_t* generated_lengths, uint8_t* finished_by_eos, uint8_t* finished,
                                     const int64_t* slot_rows, const int64_t* sink_rows, const int64_t* slot_caps,
                                     int64_t* row_steps, int64_t* row_positions, int64_t* decode_ids,
                                     int64_t* decode_useful_events, int64_t slots, int64_t storage_rows,
                                     int64_t storage_width, int64_t seen_width, int64_t maximum_new_tokens,
                                     int64_t pad_token_id, const int64_t* eos_token_ids, int64_t eos_count,
                                     yh_stream_t stream) {
  using namespace yh;
  YH_CHECK_ARG(sampled_token && storage && dense_seen && generated_lengths && finished_by_eos && finished &&
                   slot_rows && sink_rows && slot_caps && row_steps && row_positions && decode_ids &&
                   decode_useful_events,
               "decode_bookkeeping: null pointer");
  YH_CHECK_ARG(slots >= 0 && storage_rows >= 0 && storage_width > 0 && seen_width > 0,
               "decode_bookkeeping: bad sizes");
  YH_CHECK_ARG(eos_count >= 0 && (eos_count == 0 || eos_token_ids != nullptr), "decode_bookkeeping: bad eos list");
  if (slots == 0) return YH_OK;
  BookArgs a{sampled_token, storage, dense_seen, generated_lengths, finished_by_eos, finished, slot_rows,
             sink_rows, slot_caps, row_steps, row_positions, decode_ids, decode_useful_events, slots,
             storage_rows, storage_width, seen_width, maximum_new_tokens, pad_token_id,
             eos_count >= 1 ? eos_token_ids[0] : 0, eos_count >= 2 ? eos_token_ids[1] : 0,
             static_cast<int>(eos_count < 2 ? eos_count : 2)};
  hipLaunchKernelGGL(bookkeeping_kernel, dim3(1), dim3(kScanThreads), 0, static_cast<hipStream_t>(stream), a);
  YH_CHECK_LAUNCH("decode_bookkeeping");
  return YH_OK;
}

extern "C" int yh_cu_seqlens(const void* lengths, int lengths_dtype, int32_t* cu_seqlens, int64_t n,
                             yh_stream_t stream) {
  using namespace yh;
  YH_CHECK_ARG(cu_seqlens && n >= 0 && (n == 0 || lengths), "cu_seqlens: bad arguments");
  YH_CHECK_ARG(lengths_dtype == YH_I32 || lengths_dtype == YH_I64, "cu_seqlens: lengths must be int32 or int64");
  hipLaunchKernelGGL(cu_seqlens_kernel, dim3(1), dim3(kScanThreads), 0, static_cast<hipStream_t>(stream), lengths,
                     lengths_dtype == YH_I64 ? 1 : 0, cu_seqlens, n);
  YH_CHECK_LAUNCH("cu_seqlens");
  return YH_OK;
}

extern "C" int yh_select_slots(const uint8_t* finished, const int64_t* slot_rows, int mode, int64_t* out,
                               int64_t* count, int64_t n, yh_stream_t stream) {
  using namespace yh;
  YH_CHECK_ARG(count && n >= 0 && (n == 0 || (finished && out)), "select_slots: bad arguments");
  YH_CHECK_ARG(mode == YH_SELECT_KEEP || mode == YH_SELECT_FINISHED, "select_slots: unknown mode %d", mode);
  YH_CHECK_ARG(n == 0 || mode != YH_SELECT_KEEP || slot_rows != nullptr, "select_slots: keep mode needs slot_rows");
  hipLaunchKernelGGL(select_slots_kernel, dim3(1), dim3(kScanThreads), 0, static_cast<hipStream_t>(stream),
                     finished, slot_rows, mode, out, count, n);
  YH_CHECK_LAUNCH("select_slots");
  return YH_OK;
}

extern "C" int yh_gather_rows(int n_tensors, const void* const* src, void* const* dst, const int64_t* row_bytes,
                              const int64_t* src_rows, const int64_t* dst_rows, const int64_t* src_index,
                              const int64_t* dst_index, int64_t n, yh_stream_t stream) {
  using namespace yh;
  YH_CHECK_ARG(n_tensors >= 0 && n >= 0 && n < (1LL << 31), "gather_rows: bad sizes");
  YH_CHECK_ARG(n_tensors == 0 || (src && dst && row_bytes && src_rows && dst_rows), "gather_rows: null array");
  hipStream_t st = static_cast<hipStream_t>(stream);
  for (int t0 = 0; t0 < n_tensors; t0 += kMaxCopyTensors) {
    const int cnt = n_tensors - t0 < kMaxCopyTensors ? n_tensors - t0 : kMaxCopyTensors;
    CopyArgs a{};
    int64_t widest = 0;
    for (int t = 0; t < cnt; ++t) {
      YH_CHECK_ARG(src[t0 + t] && dst[t0 + t] && row_bytes[t0 + t] > 0, "gather_rows: tensor %d invalid", t0 + t);
      YH_CHECK_ARG(src[t0 + t] != dst[t0 + t], "gather_rows: tensor %d copies onto itself", t0 + t);
      a.src[t] = static_cast<const char*>(src[t0 + t]);
      a.dst[t] = static_cast<char*>(dst[t0 + t]);
      a.row_bytes[t] = row_bytes[t0 + t];
      a.src_rows[t] = src_rows[t0 + t];
      a.dst_rows[t] = dst_rows[t0 + t];
      widest = widest > row_bytes[t0 + t] ? widest : row_bytes[t0 + t];
    }
    a.src_index = src_index;
    a.dst_index = dst_index;
    a.n = n;
    if (n == 0) continue;
    const dim3 grid(static_cast<unsigned>((widest + kCopyChunk - 1) / kCopyChunk), static_cast<unsigned>(n), cnt);
    hipLaunchKernelGGL(gather_rows_kernel, grid, dim3(kCopyThreads), 0, st, a);
    YH_CHECK_LAUNCH("gather_rows");
  }
  return YH_OK;
}
