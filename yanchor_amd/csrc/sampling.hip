// Counter-based top-k / top-p sampling over the vocabulary, and the dense
// presence penalty.
//
// Replaces (runtime/model/inference_kernels.py):
//   counter_uniform                 24-33
//   sample_top_k_top_p_counter      35-88   (mode YH_SAMPLE_TORCH)
//   _qwen35_top20_counter_sample_kernel + torch.topk in
//   _sample_top_k_top_p_counter_triton 1119-1167 (mode YH_SAMPLE_FUSED)
//   _qwen35_dense_presence_penalty_kernel 1095-1114
//
// Top-k runs in two launches.  Phase 1: a workgroup per (row, vocabulary
// segment).  Every thread takes the maximum of its 32 elements; the k-th
// largest of the 256 maxima (each wave sorts its 64, the first k of the four
// waves are ranked) is at most the segment's k-th largest element, and only
// the k threads whose maxima reach it can hold elements that do -- at most
// 32 k, gathered in LDS and ranked by counting.  Elements are compared by the
// unique key (value, -index): larger value first, lower index on equal
// values.  bf16 rows of 16-byte runs with k <= 32 (the decode step's logits)
// take topk_wide_kernel instead: 64 elements a thread, float maxima per run,
// the same lists.  Phase 2: a workgroup per row ranks the segment lists' keys
// by counting, then draws the token.
#include "common.h"

#include <cmath>
#include <mutex>

namespace yh {
namespace {

constexpr int kTopkThreads = 256;
constexpr int kSampleThreads = 512;  // phase 2: one thread a candidate key of the row
constexpr int kMaxK = 64;
constexpr int kMaxPerThread = 64;  // elements per thread per segment

// Larger float -> larger key; -0.0 == +0.0.
__device__ __forceinline__ uint32_t okey(float x) {
  if (x == 0.f) x = 0.f;
  const uint32_t u = __float_as_uint(x);
  return (u & 0x80000000u) ? ~u : (u ^ 0x80000000u);
}
__device__ __forceinline__ float okey_inv(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k ^ 0x80000000u) : ~k);
}
__device__ __forceinline__ uint64_t ckey(float v, uint32_t idx) {
  return (static_cast<uint64_t>(okey(v)) << 32) | (0xffffffffu - idx);
}

struct TopkArgs {
  const void* scores;      // [B, V]
  const uint8_t* seen;     // [B, V] or null
  uint64_t* work;          // [B, S, k] composite keys
  int B, V, S, seg, k;
  int64_t row_stride, seen_stride;
  float penalty;
};

constexpr int kVecPerThread = 8;                           // 4-element vectors per thread
constexpr int kSegLen = kTopkThreads * 4 * kVecPerThread;  // 8192 elements per segment
constexpr int kPerThread = 4 * kVecPerThread;              // 32
static_assert(kPerThread <= kMaxPerThread, "elements per thread");
// Candidates of a segment: the elements of the at most k threads whose
// maximum reaches the threshold (the k-th largest thread maximum).
constexpr int kCandMax = kMaxK * kPerThread;  // 2048

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

template <int DT>
__device__ __forceinline__ float decode_elem(uint32_t bits) {
  if constexpr (DT == YH_F32) return __uint_as_float(bits);
  else if constexpr (DT == YH_BF16) return __uint_as_float(bits << 16);
  else return f16_to_f32(static_cast<uint16_t>(bits));
}

// A thread's 32 elements of one segment, kept as loaded (the raw words and
// seen bytes) and decoded on use, in increasing vocabulary index.  RUNS (rows
// 16-byte aligned, V a multiple of the run): 16-byte runs, element
// e = (run c, slot j) at lo + (c * 256 + tid) * E + j, through buffer
// resources bounded by the row, so runs past V read zeros (and are invalid).
// Otherwise element e at lo + e * 256 + tid, loaded one by one at a clamped
// index and invalid past V.  Every load is issued before the first is used.
template <int DT, bool RUNS> struct SegElems;

template <int DT> struct SegElems<DT, true> {
  static constexpr int ES = DT == YH_F32 ? 4 : 2, E = 16 / ES, NC = kPerThread / E;
  uint4 raw[NC];
  uint64_t sm[NC];
  int base, V;
  bool full;
  __device__ __forceinline__ void load(const char* row, const uint8_t* srow, int lo, int tid, int V_) {
    V = V_;
    full = lo + kSegLen <= V;
    base = lo + tid * E;
    const __amdgpu_buffer_rsrc_t rr = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(row), 0, V * ES, 0x00020000);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rr, (base + c * kTopkThreads * E) * ES, 0, 0);
      raw[c] = make_uint4(v.x, v.y, v.z, v.w);
    }
#pragma unroll
    for (int c = 0; c < NC; ++c) sm[c] = 0;
    if (srow) {
      const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(srow), 0, V, 0x00020000);
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int off = base + c * kTopkThreads * E;
        if constexpr (E == 8) {
          const u32x2 m = __builtin_amdgcn_raw_buffer_load_b64(sr, off, 0, 0);
          sm[c] = (static_cast<uint64_t>(m.y) << 32) | m.x;
        } else {
          sm[c] = __builtin_amdgcn_raw_buffer_load_b32(sr, off, 0, 0);
        }
      }
    }
  }
  // an opaque use of the loaded words: the second pass decodes them again
  // instead of keeping 32 keys live across the threshold search
  __device__ __forceinline__ void touch() {
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      asm volatile("" : "+v"(raw[c].x), "+v"(raw[c].y), "+v"(raw[c].z), "+v"(raw[c].w));
      uint32_t lo = static_cast<uint32_t>(sm[c]), hi = static_cast<uint32_t>(sm[c] >> 32);
      asm volatile("" : "+v"(lo), "+v"(hi));
      sm[c] = (static_cast<uint64_t>(hi) << 32) | lo;
    }
  }
  __device__ __forceinline__ bool valid(int e) const { return full || index(e) < V; }
  __device__ __forceinline__ int index(int e) const { return base + (e / E) * kTopkThreads * E + e % E; }
  __device__ __forceinline__ float value(int e, float penalty) const {
    const int c = e / E, j = e % E;
    const uint32_t w = reinterpret_cast<const uint32_t*>(&raw[c])[ES == 4 ? j : j / 2];
    const uint32_t bits = ES == 4 ? w : (w >> (16 * (j & 1))) & 0xffffu;
    const float x = decode_elem<DT>(bits);
    return ((sm[c] >> (8 * j)) & 0xffu) ? x - penalty : x;
  }
};

template <int DT> struct SegElems<DT, false> {
  static constexpr int ES = DT == YH_F32 ? 4 : 2;
  uint32_t raw[kPerThread];
  uint32_t sm;  // bit e: element e was seen
  int base, V;
  __device__ __forceinline__ void load(const char* row, const uint8_t* srow, int lo, int tid, int V_) {
    base = lo + tid;
    V = V_;
#pragma unroll
    for (int e = 0; e < kPerThread; ++e) {
      const int i = min(base + e * kTopkThreads, V - 1);
      if constexpr (ES == 4) raw[e] = *reinterpret_cast<const uint32_t*>(row + static_cast<int64_t>(i) * 4);
      else raw[e] = *reinterpret_cast<const uint16_t*>(row + static_cast<int64_t>(i) * 2);
    }
    sm = 0;
    if (srow) {
#pragma unroll
      for (int e = 0; e < kPerThread; ++e) sm |= (srow[min(base + e * kTopkThreads, V - 1)] ? 1u : 0u) << e;
    }
  }
  __device__ __forceinline__ void touch() {
#pragma unroll
    for (int e = 0; e < kPerThread; ++e) asm volatile("" : "+v"(raw[e]));
    asm volatile("" : "+v"(sm));
  }
  __device__ __forceinline__ bool valid(int e) const { return base + e * kTopkThreads < V; }
  __device__ __forceinline__ int index(int e) const { return base + e * kTopkThreads; }
  __device__ __forceinline__ float value(int e, float penalty) const {
    const float x = decode_elem<DT>(raw[e]);
    return ((sm >> e) & 1u) ? x - penalty : x;
  }
};

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m) {
  const uint32_t lo = __shfl_xor(static_cast<uint32_t>(v), m, kWave);
  const uint32_t hi = __shfl_xor(static_cast<uint32_t>(v >> 32), m, kWave);
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

// The top k of one segment, as keys sorted in descending order (0 past the
// segment's elements), into out[0 .. k).
//  1. Each thread's maximum key (the first of equal values: its elements come
//     in increasing index).
//  2. Each wave sorts its 64 maxima (bitonic network); its first k go to LDS.
//  3. The threshold is the k-th largest of those 4 k keys, i.e. the k-th
//     largest of all 256 thread maxima (0 if fewer than k threads hold an
//     element): k threads hold an element at least that large, so it does not
//     exceed the segment's k-th largest element, and only the at most k
//     threads whose maximum reaches it can hold elements that do.
//  4. Those threads put their elements at or above it in LDS (at most 32 k);
//     they are ranked by counting.
// okey with the zero made canonical by an addition (-0 + 0 = +0) and the sign
// handled by a mask, without compares: the same keys, fewer instructions.
__device__ __forceinline__ uint32_t okey_fast(float x) {
  const uint32_t u = __float_as_uint(x + 0.0f);
  return u ^ (static_cast<uint32_t>(static_cast<int32_t>(u) >> 31) | 0x80000000u);
}

template <bool CHECK, class El>
__device__ __forceinline__ void segment_topk(El& el, float penalty, int k, uint64_t* __restrict__ out,
                                             uint64_t (&wtop)[kTopkThreads / kWave][kMaxK],
                                             uint64_t* __restrict__ cand, uint64_t& thr_s, int& ncand) {
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wv = tid / kWave;
  // the value key of element e (0 past the row; real keys are nonzero),
  // decoded from the loaded words in both passes
  auto vkey = [&](int e) {
    const uint32_t kx = okey_fast(el.value(e, penalty));
    if constexpr (CHECK) return el.valid(e) ? kx : 0u;
    return kx;
  };
  // the thread's maximum key and its first position
  uint32_t mk = 0;
  int mi = 0;
#pragma unroll
  for (int e = 0; e < kPerThread; ++e) {
    const uint32_t kx = vkey(e);
    const bool gt = kx > mk;
    mi = gt ? e : mi;
    mk = gt ? kx : mk;
    // the running pair is materialised at every element: otherwise the
    // compiler defers the index selects and keeps every key live
    asm volatile("" : "+v"(mi), "+v"(mk));
  }
  const uint64_t best =
      mk != 0 ? (static_cast<uint64_t>(mk) << 32) | (0xffffffffu - static_cast<uint32_t>(el.index(mi))) : 0ull;
  uint64_t x = best;
#pragma unroll
  for (int size = 2; size <= kWave; size <<= 1)
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      const uint64_t y = shfl_xor_u64(x, stride);
      const bool keep_max = ((lane & size) == 0) == ((lane & stride) == 0);
      x = keep_max ? (x > y ? x : y) : (x < y ? x : y);
    }
  if (lane < k) wtop[wv][lane] = x;  // descending: lane j holds the wave's (j + 1)-th largest
  __syncthreads();
  if (tid < (kTopkThreads / kWave) * k) {
    const uint64_t c = wtop[tid / k][tid % k];
    int rank = 0;
    for (int w = 0; w < kTopkThreads / kWave; ++w)
      for (int j = 0; j < k; ++j) rank += wtop[w][j] > c;
    if (rank == k - 1 && c != 0) thr_s = c;  // real keys are unique: at most one thread
  }
  __syncthreads();
  const uint64_t thr = thr_s;
  el.touch();
  if (best != 0 && best >= thr) {
#pragma unroll
    for (int e = 0; e < kPerThread; ++e) {
      const uint32_t kx = vkey(e);
      const uint64_t key = (static_cast<uint64_t>(kx) << 32) | (0xffffffffu - static_cast<uint32_t>(el.index(e)));
      if (kx != 0 && key >= thr) cand[atomicAdd(&ncand, 1)] = key;
    }
  }
  __syncthreads();
  const int n = ncand;
  for (int i = tid; i < n; i += kTopkThreads) {
    const uint64_t mine = cand[i];
    int rank = 0;
    for (int j = 0; j < n; ++j) rank += cand[j] > mine;
    if (rank < k) out[rank] = mine;
  }
  for (int r = n + tid; r < k; r += kTopkThreads) out[r] = 0;  // padding: below every element
}

template <int DT, bool VEC>
__global__ void __launch_bounds__(kTopkThreads) topk_segment_kernel(TopkArgs a) {
  __shared__ uint64_t wtop[kTopkThreads / kWave][kMaxK];
  __shared__ uint64_t cand[kCandMax + 1];  // + a spare entry
  __shared__ uint64_t thr_s;
  __shared__ int ncand;
  const int seg = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const int lo = seg * kSegLen;
  if (tid == 0) {
    ncand = 0;
    thr_s = 0;
  }
  constexpr int ES = DT == YH_F32 ? 4 : 2;
  const char* row = static_cast<const char*>(a.scores) + static_cast<int64_t>(b) * a.row_stride * ES;
  const uint8_t* srow = a.seen ? a.seen + static_cast<int64_t>(b) * a.seen_stride : nullptr;
  uint64_t* out = a.work + (static_cast<int64_t>(b) * a.S + seg) * a.k;
  SegElems<DT, VEC> el;
  el.load(row, srow, lo, tid, a.V);
  if (lo + kSegLen <= a.V)  // uniform: no element past the row
    segment_topk<false>(el, a.penalty, a.k, out, wtop, cand, thr_s, ncand);
  else
    segment_topk<true>(el, a.penalty, a.k, out, wtop, cand, thr_s, ncand);
}

// ---- bf16 rows, top_k <= 32: 64 elements a thread --------------------------
// The same lists as topk_segment_kernel over 16384-element segments, with
// fewer VALU operations per element (the 8192-element kernel spends ~37 an
// element and is bound by their issue):
//  1. each thread takes the maxima of its eight 8-element runs of penalised
//     values as floats (max chains; the penalty as x - p * seen, seen 0 / 1),
//     keyed once per run; a NaN anywhere in the segment (which the float
//     maxima skip) makes the workgroup key every element instead;
//  2. the threshold t is the k-th largest of the 256 thread maxima by value
//     alone (each wave sorts its 64 keys, the first k of the four waves are
//     ranked, ties counted): k elements reach it, so every element of the
//     segment's top k does, and they lie in the threads whose maxima do;
//  3. those threads key the elements of their runs whose maxima reach t,
//     (value, -index) as in the 8192-element kernel, and the candidates are
//     ranked by counting.  When ties at t let more than kWideCandThreads
//     threads reach it, the list takes the elements above t (fewer than k
//     threads hold them) and then, if they are fewer than k, the elements
//     equal to t in index order up to k.
constexpr int kWideRuns = 8;                            // 16-byte runs (8 bf16) a thread
constexpr int kWidePer = 8 * kWideRuns;                 // 64 elements a thread
constexpr int kWideSeg = kTopkThreads * kWidePer;       // 16384 elements a segment
constexpr int kWideMaxK = 32;
constexpr int kWideCandThreads = kCandMax / kWidePer;   // 32 threads' elements fit the list
static_assert(kWideCandThreads >= kWideMaxK, "the k - 1 threads above the threshold fit the list");

// A thread's 64 bf16 elements: element e = (run c, slot j) at
// lo + (c * 256 + tid) * 8 + j, loaded through buffer resources bounded by
// the row (runs past V read zeros and are invalid).  The first pass keeps
// the loaded runs; the later passes load the runs they need again (from the
// cache), so the 48 registers of the first are free after it.
struct WideRun {
  uint4 raw;
  uint32_t sm[2];
  __device__ __forceinline__ float value(int j, float penalty) const {
    const uint32_t w = reinterpret_cast<const uint32_t*>(&raw)[j / 2];
    const float x = __uint_as_float((j & 1) ? (w & 0xffff0000u) : (w << 16));
    return ((sm[j / 4] >> (8 * (j % 4))) & 0xffu) ? x - penalty : x;
  }
  __device__ __forceinline__ uint32_t key(int j, float penalty) const { return okey_fast(value(j, penalty)); }
};

struct WideElems {
  __amdgpu_buffer_rsrc_t rr, sr;
  bool seen;
  int base, V;
  bool full;
  __device__ __forceinline__ void init(const char* row, const uint8_t* srow, int lo, int tid, int V_) {
    V = V_;
    full = lo + kWideSeg <= V;
    base = lo + tid * 8;
    seen = srow != nullptr;
    rr = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(row), 0, V * 2, 0x00020000);
    sr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(seen ? srow : nullptr), 0, seen ? V : 0, 0x00020000);
  }
  // again: an opaque offset, so the compiler loads the run anew instead of
  // keeping the first pass's registers live
  template <bool AGAIN = true>
  __device__ __forceinline__ void load(int c, WideRun& r) const {
    int off = base + c * kTopkThreads * 8;
    if constexpr (AGAIN) asm volatile("" : "+v"(off));
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rr, off * 2, 0, 0);
    r.raw = make_uint4(v.x, v.y, v.z, v.w);
    r.sm[0] = r.sm[1] = 0;
    if (seen) {
      const u32x2 m = __builtin_amdgcn_raw_buffer_load_b64(sr, off, 0, 0);
      r.sm[0] = m.x;
      r.sm[1] = m.y;
    }
  }
  // the key of one element, loaded on its own (the rare NaN pass)
  __device__ __forceinline__ uint32_t key(int c, int j, float penalty) const {
    const int i = base + c * kTopkThreads * 8 + j;
    const float x = __uint_as_float(static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b16(rr, i * 2, 0, 0)) << 16);
    const bool s = seen && __builtin_amdgcn_raw_buffer_load_b8(sr, i, 0, 0) != 0;
    return okey_fast(s ? x - penalty : x);
  }
  __device__ __forceinline__ bool run_valid(int c) const { return full || base + c * kTopkThreads * 8 < V; }
  __device__ __forceinline__ int index(int c, int j) const { return base + c * kTopkThreads * 8 + j; }
};

// Bytes of s made 0 / 1 (nonzero -> 1), without carries between bytes.
__device__ __forceinline__ uint32_t nonzero_bytes(uint32_t s) {
  return ((((s & 0x7f7f7f7fu) + 0x7f7f7f7fu) | s) >> 7) & 0x01010101u;
}

// Exclusive prefix sum of v over the workgroup in thread order; *total = the sum.
__device__ __forceinline__ int block_excl_scan(int v, int* total, int (&wsum)[kTopkThreads / kWave]) {
  const int lane = threadIdx.x & (kWave - 1), wv = threadIdx.x / kWave;
  int x = v;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int y = __shfl_up(x, off, kWave);
    if (lane >= off) x += y;
  }
  __syncthreads();  // wsum free
  if (lane == kWave - 1) wsum[wv] = x;
  __syncthreads();
  int before = 0, all = 0;
#pragma unroll
  for (int w = 0; w < kTopkThreads / kWave; ++w) {
    before += w < wv ? wsum[w] : 0;
    all += wsum[w];
  }
  *total = all;
  return before + x - v;
}

// Five workgroups a CU (20 waves): the decode batch's 1280 segments are resident at once.
template <bool CHECK>
__global__ void __launch_bounds__(kTopkThreads) __attribute__((amdgpu_waves_per_eu(5, 5)))
topk_wide_kernel(TopkArgs a) {
  __shared__ uint32_t wtop[kTopkThreads / kWave][kWideMaxK];
  __shared__ uint64_t cand[kCandMax + 1];  // + a spare entry
  __shared__ int wsum[kTopkThreads / kWave];
  __shared__ uint32_t thr_v;
  __shared__ int ncand, nthreads;
  const int seg = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const int lane = tid & (kWave - 1), wv = tid / kWave, k = a.k;
  const int lo = seg * kWideSeg;
  if (tid == 0) {
    ncand = 0;
    nthreads = 0;
    thr_v = 1;  // fewer than k real maxima: every real element is a candidate
  }
  const char* row = static_cast<const char*>(a.scores) + static_cast<int64_t>(b) * a.row_stride * 2;
  const uint8_t* srow = a.seen ? a.seen + static_cast<int64_t>(b) * a.seen_stride : nullptr;
  uint64_t* out = a.work + (static_cast<int64_t>(b) * a.S + seg) * a.k;
  WideElems el;
  el.init(row, srow, lo, tid, a.V);
  WideRun run[kWideRuns];
#pragma unroll
  for (int c = 0; c < kWideRuns; ++c) el.load<false>(c, run[c]);
  const float pen = a.penalty;

  // 1. run maxima of the penalised values (0: a run past the row); |x| bits
  // of the raw words to find a NaN
  const float np = -pen;
  uint32_t rkey[kWideRuns];
  float rmax[kWideRuns];
  u16x2 absmax = {0, 0};
#pragma unroll
  for (int c = 0; c < kWideRuns; ++c) {
    const uint32_t* w = reinterpret_cast<const uint32_t*>(&run[c].raw);
    const uint32_t s0 = nonzero_bytes(run[c].sm[0]), s1 = nonzero_bytes(run[c].sm[1]);
    float m = -INFINITY;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const uint32_t sw = d < 2 ? s0 : s1;
      const int sh = 16 * (d & 1);
      const float x0 = fmaf(np, static_cast<float>((sw >> sh) & 0xffu), __uint_as_float(w[d] << 16));
      const float x1 = fmaf(np, static_cast<float>((sw >> (sh + 8)) & 0xffu), __uint_as_float(w[d] & 0xffff0000u));
      m = fmaxf(m, fmaxf(x0, x1));
      absmax = __builtin_elementwise_max(absmax, __builtin_bit_cast(u16x2, w[d] & 0x7fff7fffu));
    }
    rmax[c] = m;
  }
  const bool nan = absmax.x > 0x7f80u || absmax.y > 0x7f80u;
  if (__syncthreads_or(nan)) {  // exact keys of every element
#pragma unroll
    for (int c = 0; c < kWideRuns; ++c) {
      uint32_t m = 0;
#pragma unroll 1
      for (int j = 0; j < 8; ++j) m = max(m, el.key(c, j, pen));  // element by element: few registers
      rkey[c] = m;
    }
  } else {
#pragma unroll
    for (int c = 0; c < kWideRuns; ++c) rkey[c] = okey_fast(rmax[c]);
  }
  uint32_t tkey = 0;
#pragma unroll
  for (int c = 0; c < kWideRuns; ++c) {
    if (CHECK && !el.run_valid(c)) rkey[c] = 0;
    tkey = max(tkey, rkey[c]);
  }

  // 2. the k-th largest thread maximum by value, ties counted
  uint32_t x = tkey;
#pragma unroll
  for (int size = 2; size <= kWave; size <<= 1)
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      const uint32_t y = __shfl_xor(x, stride, kWave);
      const bool keep_max = ((lane & size) == 0) == ((lane & stride) == 0);
      x = keep_max ? (x > y ? x : y) : (x < y ? x : y);
    }
  if (lane < k) wtop[wv][lane] = x;  // descending
  __syncthreads();
  if (tid < (kTopkThreads / kWave) * k) {
    const uint32_t c = wtop[tid / k][tid % k];
    int gt = 0, ge = 0;
    for (int w = 0; w < kTopkThreads / kWave; ++w)
      for (int j = 0; j < k; ++j) {
        const uint32_t o = wtop[w][j];
        gt += o > c;
        ge += o >= c;
      }
    if (c != 0 && gt < k && ge >= k) thr_v = c;  // every such c holds the same value
  }
  __syncthreads();
  const uint32_t thr = thr_v;
  if (tkey >= thr) atomicAdd(&nthreads, 1);
  __syncthreads();

  // 3. the candidates
  if (nthreads <= kWideCandThreads) {  // uniform
    if (tkey >= thr) {
#pragma unroll
      for (int c = 0; c < kWideRuns; ++c) {
        if (rkey[c] < thr) continue;
        WideRun r;
        el.load(c, r);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const uint32_t kx = r.key(j, pen);
          if (kx >= thr) cand[atomicAdd(&ncand, 1)] = (static_cast<uint64_t>(kx) << 32) |
                                                      (0xffffffffu - static_cast<uint32_t>(el.index(c, j)));
        }
      }
    }
  } else {
    // ties at the threshold: the elements above it (fewer than k threads
    // hold them), then those equal to it in index order until k are listed
    if (tkey > thr) {
#pragma unroll
      for (int c = 0; c < kWideRuns; ++c) {
        if (rkey[c] <= thr) continue;
        WideRun r;
        el.load(c, r);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const uint32_t kx = r.key(j, pen);
          if (kx > thr) cand[atomicAdd(&ncand, 1)] = (static_cast<uint64_t>(kx) << 32) |
                                                     (0xffffffffu - static_cast<uint32_t>(el.index(c, j)));
        }
      }
    }
    __syncthreads();
    int need = k - ncand;
#pragma unroll
    for (int c = 0; c < kWideRuns; ++c) {
      if (need <= 0) break;  // uniform
      int cnt = 0;
      WideRun r;
      if (rkey[c] >= thr) {
        el.load(c, r);
#pragma unroll
        for (int j = 0; j < 8; ++j) cnt += r.key(j, pen) == thr;
      }
      int total = 0;
      int pos = block_excl_scan(cnt, &total, wsum);
      if (cnt > 0 && pos < need) {
        const int base_slot = ncand;  // read before any thread of this run appends
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          if (r.key(j, pen) == thr && pos < need) {
            cand[base_slot + pos] = (static_cast<uint64_t>(thr) << 32) |
                                    (0xffffffffu - static_cast<uint32_t>(el.index(c, j)));
            ++pos;
          }
        }
      }
      __syncthreads();
      if (tid == 0) ncand += min(total, need);
      need -= total;
      __syncthreads();
    }
  }
  __syncthreads();
  const int n = ncand;
  for (int i = tid; i < n; i += kTopkThreads) {
    const uint64_t me = cand[i];
    int rank = 0;
    for (int j = 0; j < n; ++j) rank += cand[j] > me;
    if (rank < k) out[rank] = me;
  }
  for (int r = n + tid; r < k; r += kTopkThreads) out[r] = 0;  // padding: below every element
}

struct SampleArgs {
  const uint64_t* work;      // [B, S, k]
  const int64_t* ids;        // [B]
  const int64_t* steps;      // [B] or null (then `step` is used)
  int64_t* out;              // [B]
  float* out_values;         // [B, k] (optional) sorted top-k values before temperature
  int64_t* out_indices;      // [B, k] (optional)
  int B, S, k, mode;
  int64_t step;
  uint32_t seed, stream;
  float temperature, top_p;
};

__device__ __forceinline__ uint32_t counter_word(uint32_t id, uint32_t step, uint32_t seed, uint32_t stream) {
  const uint32_t state = id * 747796405u + step * 289133645u + seed * 277803737u + stream * 144269504u;
  const uint32_t shift = (state >> 28) + 4u;
  uint32_t w = ((state >> shift) ^ state) * 277803737u;
  return (w >> 22) ^ w;
}

// Inclusive prefix sum over the first 64 lanes of a wave (lane order).
__device__ __forceinline__ float wave_scan(float x, int lane) {
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const float y = __shfl_up(x, off, kWave);
    if (lane >= off) x += y;
  }
  return x;
}

__global__ void __launch_bounds__(kSampleThreads) sample_rows_kernel(SampleArgs a) {
  __shared__ uint64_t cand[kMaxK * 64];
  __shared__ uint64_t top[kMaxK];
  const int b = blockIdx.x, tid = threadIdx.x;
  const int n = a.S * a.k;
  const uint64_t* src = a.work + static_cast<int64_t>(b) * n;
  for (int i = tid; i < n; i += kSampleThreads) cand[i] = src[i];
  __syncthreads();
  // rank by counting: one thread a key (S k <= 64 k keys, 512 threads)
  for (int i = tid; i < n; i += kSampleThreads) {
    const uint64_t mine = cand[i];
    int rank = 0;
    for (int j = 0; j < n; ++j) rank += cand[j] > mine;
    if (rank < a.k) top[rank] = mine;
  }
  __syncthreads();
  if (tid >= kWave) return;
  const int lane = tid;
  const bool in = lane < a.k;
  const uint64_t c = in ? top[lane] : 0;
  const bool real = in && c != 0;
  const float v = real ? okey_inv(static_cast<uint32_t>(c >> 32)) : -INFINITY;
  const int64_t index = real ? static_cast<int64_t>(0xffffffffu - static_cast<uint32_t>(c & 0xffffffffu)) : 0;
  if (a.out_values && in) a.out_values[static_cast<int64_t>(b) * a.k + lane] = v;
  if (a.out_indices && in) a.out_indices[static_cast<int64_t>(b) * a.k + lane] = index;
  if (a.k == 1) {
    if (lane == 0) a.out[b] = index;
    return;
  }
  const uint32_t id = static_cast<uint32_t>(a.ids[b]);
  const uint32_t st = static_cast<uint32_t>(a.steps ? a.steps[b] : a.step);
  const uint32_t word = counter_word(id, st, a.seed, a.stream);
  const double ud = (static_cast<double>(word) + 0.5) / 4294967296.0;
  float u = static_cast<float>(ud);
  const float x = real ? v / a.temperature : -INFINITY;
  const float m = __shfl(x, 0, kWave);  // row maximum is the first candidate
  const float w = real ? expf(x - m) : 0.f;
  const float total = wave_sum(w);
  const float p = w / total;
  const float cum_p = wave_scan(p, lane);
  const bool keep = real && (cum_p - p) < a.top_p;
  int rank;
  if (a.mode == YH_SAMPLE_FUSED) {
    // _qwen35_top20_counter_sample_kernel: u unclamped, threshold = u * retained
    const float t = keep ? p : 0.f;
    const float retained = wave_sum(t);
    const float cum = wave_scan(t, lane);
    const float threshold = u * retained;
    const unsigned long long below = __ballot(in && cum < threshold);
    rank = __popcll(below);
    rank = rank < a.k - 1 ? rank : a.k - 1;
  } else {
    // top_k_top_p_distribution + sample_probabilities_counter + _sample_cdf_counter
    float t = keep ? p : 0.f;
    t = t / wave_sum(t);
    t = t / wave_sum(t);
    const float cum = wave_scan(t, lane);
    const float tot = __shfl(cum, a.k - 1, kWave);
    const float umax = 1.0f - 5.9604644775390625e-08f;  // 1 - eps/2 for float32
    u = u < umax ? u : umax;
    float threshold = u * tot;
    const float below_tot = nextafterf(tot, 0.f);
    threshold = threshold < below_tot ? threshold : below_tot;
    const unsigned long long below = __ballot(in && cum < threshold);
    rank = __popcll(below);
    rank = rank < a.k - 1 ? rank : a.k - 1;
  }
  const int64_t token = __shfl(index, rank, kWave);
  if (lane == 0) a.out[b] = token;
}

__global__ void presence_penalty_kernel(float* scores, const uint8_t* seen, int64_t n, float penalty) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) scores[i] = scores[i] - (seen[i] ? penalty : 0.f);
}

__global__ void counter_uniform_kernel(const int64_t* ids, const int64_t* steps, int64_t step, float* out,
                                       int n, uint32_t seed, uint32_t stream) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const uint32_t w = counter_word(static_cast<uint32_t>(ids[i]),
                                  static_cast<uint32_t>(steps ? steps[i] : step), seed, stream);
  const float u = static_cast<float>((static_cast<double>(w) + 0.5) / 4294967296.0);
  const float umax = 1.0f - 5.9604644775390625e-08f;
  out[i] = u < umax ? u : umax;
}

}  // namespace
}  // namespace yh

namespace yh {
namespace {

// ---- full-vocabulary sampling ------------------------------------------------
// sample_top_k_top_p_counter's branches past the top-64 path
// (inference_kernels.py:78-86): top_k <= 0 with top_p == 1 draws from the
// softmax over the whole vocabulary in vocabulary order; any other top_k
// outside [1, 64] (top_k <= 0 meaning the whole vocabulary) keeps the top k,
// truncates them at top_p in value order and draws from the rest.
//
// One workgroup per row.  Every draw is a selection "the first element, in a
// given order, whose inclusive cumulative weight reaches t": the elements are
// ordered by a 64-bit key K (descending), (value key << 32 | ~index) for value
// order (larger value first, lower index first on equal values) or ~index
// for vocabulary order.  K* is found 4 bits at a time from the top: a pass
// over the row sums the weight of the elements that share the bits fixed so
// far into 16 buckets of the next digit, and the largest digit whose
// cumulative weight (with everything above) reaches t is kept.  Weights are
// counts (for the top-k cut) or probabilities as 2^62 fixed-point integers,
// so every sum is exact and independent of summation order.  The row is
// re-read on every pass (from L2 / the Infinity Cache after the first).
constexpr int kFullThreads = 1024;
constexpr int kFullWaves = kFullThreads / kWave;
constexpr int kFan = 16;
constexpr double kMassOne = 4611686018427387904.0;  // 2^62: fixed-point probability 1

struct FullArgs {
  const void* scores;     // [B, V] rows row_stride apart
  const uint8_t* seen;    // [B, V] rows seen_stride apart, or null
  const int64_t* ids;     // [B]
  const int64_t* steps;   // [B] or null (then `step`)
  int64_t* out;           // [B]
  int64_t row_stride, seen_stride, step, top_k;
  int V, vocab_order;
  uint32_t seed, stream;
  float penalty, temperature, top_p;
};

struct FullShared {
  uint64_t part[kFullWaves][kFan];
  uint32_t cpart[kFullWaves][kFan];
  uint64_t bucket[kFan];
  uint32_t bcount[kFan];
  double dpart[kFullWaves];
  float fpart[kFullWaves];
};

__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += shfl_xor_u64(v, off);
  return v;
}
__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}
__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

// Score of element i with the presence penalty applied (before temperature).
template <int DT>
__device__ __forceinline__ float full_value(const FullArgs& a, const char* row, const uint8_t* srow, int i) {
  uint32_t bits;
  if constexpr (DT == YH_F32) bits = *reinterpret_cast<const uint32_t*>(row + static_cast<int64_t>(i) * 4);
  else bits = *reinterpret_cast<const uint16_t*>(row + static_cast<int64_t>(i) * 2);
  float x = decode_elem<DT>(bits);
  if (srow && srow[i]) x = x - a.penalty;
  return x;
}

// Selection state of one row: the candidate set is K >= lo; weights are
// masses (mass) or counts; masses need the row's tempered maximum mt and
// the candidate set's sum S of exp(x / T - mt).
struct FullRow {
  const char* row;
  const uint8_t* srow;
  uint64_t lo;
  float mt;
  double scale;  // 2^62 / S: fixed-point mass per unit of exp(x / T - mt)
};

__device__ __forceinline__ uint64_t full_key(const FullArgs& a, float x, int i) {
  return a.vocab_order ? static_cast<uint64_t>(0xffffffffu - static_cast<uint32_t>(i)) : ckey(x, static_cast<uint32_t>(i));
}

template <int DT>
__device__ __forceinline__ uint64_t full_mass(const FullArgs& a, const FullRow& r, float x) {
  const float xt = x / a.temperature;
  return static_cast<uint64_t>(static_cast<double>(expf(xt - r.mt)) * r.scale);
}

// The largest K* among candidates with W(K >= K*) >= t (t >= 1), and
// W(K >= K*) in *incl.  Bits from `top` up are fixed to `prefix` (the bits of
// ~index above bit 19, all ones for an index below 2^20).  If t exceeds the
// candidates' total weight the smallest candidate key is returned.
template <int DT, bool MASS>
__device__ uint64_t full_select(const FullArgs& a, const FullRow& r, uint64_t t, int top, uint64_t prefix,
                                uint64_t* incl, FullShared& sh) {
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wv = tid / kWave;
  uint64_t above = 0;  // weight of candidates with a key above every key of the current prefix
  for (int pos = top - 4; pos >= 0; pos -= 4) {
    if (!a.vocab_order && pos == 28) {  // ~index bits 31..20: all ones (index < 2^20)
      prefix = (prefix << 12) | 0xfffull;
      pos = 16;
    }
    uint64_t acc[kFan];
    uint32_t cnt[kFan];
#pragma unroll
    for (int c = 0; c < kFan; ++c) {
      acc[c] = 0;
      cnt[c] = 0;
    }
    for (int i = tid; i < a.V; i += kFullThreads) {
      const float x = full_value<DT>(a, r.row, r.srow, i);
      const uint64_t K = full_key(a, x, i);
      if (K < r.lo || (pos + 4 < 64 && (K >> (pos + 4)) != prefix)) continue;
      const int d = static_cast<int>((K >> pos) & 0xf);
      const uint64_t w = MASS ? full_mass<DT>(a, r, x) : 1ull;
#pragma unroll
      for (int c = 0; c < kFan; ++c) {
        acc[c] += d == c ? w : 0ull;
        cnt[c] += d == c ? 1u : 0u;
      }
    }
#pragma unroll
    for (int c = 0; c < kFan; ++c) {
      const uint64_t s = wave_sum_u64(acc[c]);
      const uint32_t n = wave_sum_u32(cnt[c]);
      if (lane == 0) {
        sh.part[wv][c] = s;
        sh.cpart[wv][c] = n;
      }
    }
    __syncthreads();
    if (tid < kFan) {
      uint64_t s = 0;
      uint32_t n = 0;
      for (int w = 0; w < kFullWaves; ++w) {
        s += sh.part[w][tid];
        n += sh.cpart[w][tid];
      }
      sh.bucket[tid] = s;
      sh.bcount[tid] = n;
    }
    __syncthreads();
    // largest digit whose cumulative weight reaches t; past the total, the
    // smallest non-empty digit
    int dsel = -1, last = 0;
    uint64_t cum = above, cum_last = above;
    for (int c = kFan - 1; c >= 0; --c) {
      if (sh.bcount[c]) {
        last = c;
        cum_last = cum;
      }
      if (cum + sh.bucket[c] >= t && sh.bcount[c]) {
        dsel = c;
        break;
      }
      cum += sh.bucket[c];
    }
    if (dsel < 0) {
      dsel = last;
      cum = cum_last;
    }
    const uint64_t w_sel = sh.bucket[dsel];
    const uint32_t n_sel = sh.bcount[dsel];
    __syncthreads();
    above = cum;
    prefix = (prefix << 4) | static_cast<uint64_t>(dsel);
    if (n_sel == 1 && pos > 0) {
      // a single element left: its key is the largest key under the prefix
      uint64_t best = 0;
      for (int i = tid; i < a.V; i += kFullThreads) {
        const float x = full_value<DT>(a, r.row, r.srow, i);
        const uint64_t K = full_key(a, x, i);
        if (K >= r.lo && (K >> pos) == prefix) best = K > best ? K : best;
      }
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) {
        const uint64_t y = shfl_xor_u64(best, off);
        best = y > best ? y : best;
      }
      if (lane == 0) sh.part[wv][0] = best;
      __syncthreads();
      uint64_t k = 0;
      for (int w = 0; w < kFullWaves; ++w) k = sh.part[w][0] > k ? sh.part[w][0] : k;
      __syncthreads();
      *incl = above + w_sel;
      return k;
    }
    if (pos == 0) {
      *incl = above + w_sel;
      return prefix;
    }
  }
  *incl = above;
  return prefix;
}

template <int DT>
__global__ void __launch_bounds__(kFullThreads) sample_full_kernel(FullArgs a) {
  __shared__ FullShared sh;
  constexpr int ES = DT == YH_F32 ? 4 : 2;
  const int64_t b = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wv = tid / kWave;
  FullRow r{static_cast<const char*>(a.scores) + b * a.row_stride * ES, a.seen ? a.seen + b * a.seen_stride : nullptr,
            0ull, 0.f, 0.0};

  // row maximum of the scores (the top of the value order; its tempered
  // value is the softmax shift torch uses, division being monotone)
  float m = -INFINITY;
  for (int i = tid; i < a.V; i += kFullThreads) m = fmaxf(m, full_value<DT>(a, r.row, r.srow, i));
  m = wave_max(m);
  if (lane == 0) sh.fpart[wv] = m;
  __syncthreads();
  m = sh.fpart[0];
  for (int w = 1; w < kFullWaves; ++w) m = fmaxf(m, sh.fpart[w]);
  __syncthreads();
  r.mt = m / a.temperature;

  uint64_t incl = 0;
  // top-k cut (1 < k < V, value order): the k-th largest key bounds the candidates
  if (!a.vocab_order && a.top_k > 1 && a.top_k < a.V)
    r.lo = full_select<DT, false>(a, r, static_cast<uint64_t>(a.top_k), 64, 0ull, &incl, sh);

  // S = sum of exp(x / T - mt) over the candidates (fixed order: per thread,
  // then the wave butterfly, then the waves in order)
  double s = 0.0;
  for (int i = tid; i < a.V; i += kFullThreads) {
    const float x = full_value<DT>(a, r.row, r.srow, i);
    if (full_key(a, x, i) >= r.lo) s += static_cast<double>(expf(x / a.temperature - r.mt));
  }
  s = wave_sum_f64(s);
  if (lane == 0) sh.dpart[wv] = s;
  __syncthreads();
  s = 0.0;
  for (int w = 0; w < kFullWaves; ++w) s += sh.dpart[w];
  __syncthreads();
  r.scale = kMassOne / s;

  // total fixed-point mass of the candidates
  uint64_t tot = 0;
  for (int i = tid; i < a.V; i += kFullThreads) {
    const float x = full_value<DT>(a, r.row, r.srow, i);
    if (full_key(a, x, i) >= r.lo) tot += full_mass<DT>(a, r, x);
  }
  tot = wave_sum_u64(tot);
  if (lane == 0) sh.part[wv][0] = tot;
  __syncthreads();
  tot = 0;
  for (int w = 0; w < kFullWaves; ++w) tot += sh.part[w][0];
  __syncthreads();

  const uint32_t id = static_cast<uint32_t>(a.ids[b]);
  const uint32_t st = static_cast<uint32_t>(a.steps ? a.steps[b] : a.step);
  float u = static_cast<float>((static_cast<double>(counter_word(id, st, a.seed, a.stream)) + 0.5) / 4294967296.0);
  const float umax = 1.0f - 5.9604644775390625e-08f;  // counter_uniform's clamp: 1 - eps/2
  u = u < umax ? u : umax;
  auto at_least = [](double x, uint64_t hi) -> uint64_t {  // ceil(x) clamped to [1, hi]
    double c = ceil(x);
    uint64_t t = c < 1.0 ? 1ull : static_cast<uint64_t>(c);
    return t > hi ? hi : t;
  };
  uint64_t key;
  if (a.vocab_order) {
    // first index whose cumulative probability reaches u * total; the index
    // bits above bit 19 are ~index's all-ones
    key = full_select<DT, true>(a, r, at_least(static_cast<double>(u) * static_cast<double>(tot), tot), 20,
                                0xfffull, &incl, sh);
  } else {
    // last kept element: the first whose inclusive mass reaches top_p (so
    // every element before it has an exclusive mass below top_p); then the
    // draw inside the kept mass
    full_select<DT, true>(a, r, at_least(static_cast<double>(a.top_p) * static_cast<double>(tot), tot), 64, 0ull,
                          &incl, sh);
    const uint64_t kept = incl;
    key = full_select<DT, true>(a, r, at_least(static_cast<double>(u) * static_cast<double>(kept), kept), 64, 0ull,
                                &incl, sh);
  }
  if (tid == 0) a.out[b] = static_cast<int64_t>(0xffffffffu - static_cast<uint32_t>(key & 0xffffffffu));
}

// Both phases of the sampler with the candidate lists in `workspace`; the
// two entry points differ only in where that memory comes from.
int topk_sample_launch(const void* scores, int dtype, int64_t row_stride, const uint8_t* seen,
                       int64_t seen_stride, float penalty, const int64_t* attempt_ids, const int64_t* steps,
                       int64_t step, uint64_t seed, uint64_t stream_id, float temperature, int64_t top_k,
                       float top_p, int mode, int64_t* tokens, float* out_values, int64_t* out_indices,
                       void* workspace, int64_t workspace_bytes, int64_t B, int64_t V, yh_stream_t stream) {
  YH_CHECK_ARG(B >= 0 && V > 0 && V <= 64LL * kSegLen, "topk_sample: V must lie in [1, %d]", 64 * kSegLen);
  YH_CHECK_ARG(dtype == YH_F32 || dtype == YH_BF16 || dtype == YH_F16, "topk_sample: unsupported dtype");
  if (top_k <= 0 || top_k > kMaxK) {
    // the full-vocabulary branches of the torch sampler: no workspace
    YH_CHECK_ARG(scores && tokens && attempt_ids, "topk_sample: null pointer");
    YH_CHECK_ARG(mode == YH_SAMPLE_TORCH, "topk_sample: top_k outside [1, %d] needs the torch-sampler mode", kMaxK);
    YH_CHECK_ARG(top_k <= V, "topk_sample: top_k exceeds the vocabulary");
    YH_CHECK_ARG(temperature > 0.f && top_p > 0.f && top_p <= 1.f,
                 "topk_sample: needs temperature > 0 and 0 < top_p <= 1");
    YH_CHECK_ARG(out_values == nullptr && out_indices == nullptr,
                 "topk_sample: the selected top-k is returned only for top_k <= %d", kMaxK);
    YH_CHECK_ARG(row_stride >= V && (seen == nullptr || seen_stride >= V), "topk_sample: bad row strides");
    if (B == 0) return YH_OK;
    FullArgs fa{scores, seen, attempt_ids, steps, tokens, row_stride, seen_stride, step, top_k, (int)V,
                (top_k <= 0 && top_p == 1.f) ? 1 : 0, static_cast<uint32_t>(seed & 0xffffffffu),
                static_cast<uint32_t>(stream_id & 0xffffffffu), penalty, temperature, top_p};
    hipStream_t st = static_cast<hipStream_t>(stream);
    const dim3 grid(static_cast<unsigned>(B));
    if (dtype == YH_F32) hipLaunchKernelGGL(sample_full_kernel<YH_F32>, grid, dim3(kFullThreads), 0, st, fa);
    else if (dtype == YH_BF16) hipLaunchKernelGGL(sample_full_kernel<YH_BF16>, grid, dim3(kFullThreads), 0, st, fa);
    else hipLaunchKernelGGL(sample_full_kernel<YH_F16>, grid, dim3(kFullThreads), 0, st, fa);
    YH_CHECK_LAUNCH("sample_full");
    return YH_OK;
  }
  YH_CHECK_ARG(scores && tokens && workspace && attempt_ids, "topk_sample: null pointer");
  YH_CHECK_ARG(top_k <= V, "topk_sample: top_k exceeds the vocabulary");
  YH_CHECK_ARG(mode == YH_SAMPLE_FUSED || mode == YH_SAMPLE_TORCH, "topk_sample: unknown mode %d", mode);
  YH_CHECK_ARG(top_k == 1 || (temperature > 0.f && top_p > 0.f && top_p <= 1.f),
               "topk_sample: needs temperature > 0 and 0 < top_p <= 1");
  YH_CHECK_ARG(row_stride >= V && (seen == nullptr || seen_stride >= V), "topk_sample: bad row strides");
  const int64_t need = yh_topk_workspace_bytes(B, V, top_k);
  YH_CHECK_ARG(workspace_bytes >= need, "topk_sample: workspace of %lld bytes needs %lld",
               (long long)workspace_bytes, (long long)need);
  YH_CHECK_ARG((reinterpret_cast<uintptr_t>(workspace) & 7) == 0, "topk_sample: workspace must be 8-byte aligned");
  if (B == 0) return YH_OK;
  int S = 0, seg = 0;
  yh_topk_segments(V, top_k, &S, &seg);
  hipStream_t st = static_cast<hipStream_t>(stream);
  TopkArgs ta{scores, seen, static_cast<uint64_t*>(workspace), (int)B, (int)V, S, seg, (int)top_k,
              row_stride, seen_stride, penalty};
  const size_t esz = dtype == YH_F32 ? 4 : 2;
  const int64_t run = 16 / static_cast<int64_t>(esz);  // elements per 16-byte load
  const bool vec = (reinterpret_cast<uintptr_t>(scores) % 16) == 0 && row_stride % run == 0 && V % run == 0 &&
                   (seen == nullptr || ((reinterpret_cast<uintptr_t>(seen) % run) == 0 && seen_stride % run == 0));
  if (dtype == YH_BF16 && vec && top_k <= kWideMaxK && std::isfinite(penalty)) {
    // bf16 runs: 16384-element segments of 64 elements a thread
    S = static_cast<int>((V + kWideSeg - 1) / kWideSeg);
    ta.S = S;
    ta.seg = kWideSeg;
    const dim3 grid(S, static_cast<unsigned>(B));
    if (V % kWideSeg == 0) hipLaunchKernelGGL(topk_wide_kernel<false>, grid, dim3(kTopkThreads), 0, st, ta);
    else hipLaunchKernelGGL(topk_wide_kernel<true>, grid, dim3(kTopkThreads), 0, st, ta);
  } else {
    const dim3 grid(S, static_cast<unsigned>(B));
    switch (dtype * 2 + (vec ? 1 : 0)) {
      case YH_F32 * 2 + 1: hipLaunchKernelGGL((topk_segment_kernel<YH_F32, true>), grid, dim3(kTopkThreads), 0, st, ta); break;
      case YH_F32 * 2: hipLaunchKernelGGL((topk_segment_kernel<YH_F32, false>), grid, dim3(kTopkThreads), 0, st, ta); break;
      case YH_BF16 * 2 + 1: hipLaunchKernelGGL((topk_segment_kernel<YH_BF16, true>), grid, dim3(kTopkThreads), 0, st, ta); break;
      case YH_BF16 * 2: hipLaunchKernelGGL((topk_segment_kernel<YH_BF16, false>), grid, dim3(kTopkThreads), 0, st, ta); break;
      case YH_F16 * 2 + 1: hipLaunchKernelGGL((topk_segment_kernel<YH_F16, true>), grid, dim3(kTopkThreads), 0, st, ta); break;
      default: hipLaunchKernelGGL((topk_segment_kernel<YH_F16, false>), grid, dim3(kTopkThreads), 0, st, ta); break;
    }
  }
  YH_CHECK_LAUNCH("topk_segment");
  SampleArgs sa{static_cast<const uint64_t*>(workspace), attempt_ids, steps, tokens, out_values, out_indices,
                (int)B, S, (int)top_k, mode, step, static_cast<uint32_t>(seed & 0xffffffffu),
                static_cast<uint32_t>(stream_id & 0xffffffffu), temperature, top_p};
  hipLaunchKernelGGL(sample_rows_kernel, dim3(static_cast<unsigned>(B)), dim3(kSampleThreads), 0, st, sa);
  YH_CHECK_LAUNCH("sample_rows");
  return YH_OK;
}

// ---- allocation-free variant -----------------------------------------------
// The candidate lists live in this file-scope array: one copy per GPU, held
// until the process ends.  Host code never passes `scratch` itself (its name
// is a host-side stand-in, not a device address): the device address comes
// from hipGetSymbolAddress, looked up once per device on that device's first
// call and kept in g_scratch_addr.  Every call on a GPU shares that GPU's
// array, so calls that overlap on one GPU (different streams, different
// host threads) race.  Nothing in it has to start at zero: phase 1 writes all
// k entries of every (row, segment) list before phase 2 reads them.
__device__ __align__(256) uint64_t scratch[YH_TOPK_STATIC_SCRATCH_BYTES / sizeof(uint64_t)];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_addr[kMaxDevices] = {};

// Device address of `scratch` on the device the stream runs on (which must
// be the current device: the symbol lookup is per current device).
int static_scratch(yh_stream_t stream, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    set_error("topk_sample_noalloc: hipGetDevice failed: %s", hipGetErrorString(e));
    return YH_ERR_HIP;
  }
  if (stream != nullptr) {
    int sdev = -1;
    e = hipStreamGetDevice(static_cast<hipStream_t>(stream), &sdev);
    if (e != hipSuccess) {
      set_error("topk_sample_noalloc: hipStreamGetDevice failed: %s", hipGetErrorString(e));
      return YH_ERR_HIP;
    }
    YH_CHECK_ARG(sdev == dev, "topk_sample_noalloc: the stream's device %d is not the current device %d", sdev,
                 dev);
  }
  YH_CHECK_ARG(dev >= 0 && dev < kMaxDevices, "topk_sample_noalloc: device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_addr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      set_error("topk_sample_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                hipGetErrorString(e));
      return YH_ERR_HIP;
    }
    g_scratch_addr[dev] = p;
  }
  *out = g_scratch_addr[dev];
  return YH_OK;
}

}  // namespace
}  // namespace yh

extern "C" int yh_topk_sample(const void* scores, int dtype, int64_t row_stride, const uint8_t* seen,
                              int64_t seen_stride, float penalty, const int64_t* attempt_ids,
                              const int64_t* steps, int64_t step, uint64_t seed, uint64_t stream_id,
                              float temperature, int64_t top_k, float top_p, int mode, int64_t* tokens,
                              float* out_values, int64_t* out_indices, void* workspace,
                              int64_t workspace_bytes, int64_t B, int64_t V, yh_stream_t stream) {
  return yh::topk_sample_launch(scores, dtype, row_stride, seen, seen_stride, penalty, attempt_ids, steps, step,
                                seed, stream_id, temperature, top_k, top_p, mode, tokens, out_values,
                                out_indices, workspace, workspace_bytes, B, V, stream);
}

extern "C" int yh_topk_sample_noalloc(const void* scores, int dtype, int64_t row_stride, const uint8_t* seen,
                                      int64_t seen_stride, float penalty, const int64_t* attempt_ids,
                                      const int64_t* steps, int64_t step, uint64_t seed, uint64_t stream_id,
                                      float temperature, int64_t top_k, float top_p, int mode, int64_t* tokens,
                                      float* out_values, int64_t* out_indices, int64_t B, int64_t V,
                                      yh_stream_t stream) {
  using namespace yh;
  YH_CHECK_ARG(B >= 0 && V > 0, "topk_sample_noalloc: bad sizes");
  const int64_t need = (top_k >= 1 && top_k <= kMaxK) ? yh_topk_workspace_bytes(B, V, top_k) : 0;
  YH_CHECK_ARG(need <= YH_TOPK_STATIC_SCRATCH_BYTES,
               "topk_sample_noalloc: B=%lld, V=%lld, top_k=%lld need %lld bytes of scratch, above the static "
               "maximum of %lld (use yh_topk_sample with a workspace)",
               (long long)B, (long long)V, (long long)top_k, (long long)need,
               (long long)YH_TOPK_STATIC_SCRATCH_BYTES);
  void* ws = nullptr;
  const int rc = static_scratch(stream, &ws);
  if (rc != YH_OK) return rc;
  return topk_sample_launch(scores, dtype, row_stride, seen, seen_stride, penalty, attempt_ids, steps, step, seed,
                            stream_id, temperature, top_k, top_p, mode, tokens, out_values, out_indices, ws,
                            YH_TOPK_STATIC_SCRATCH_BYTES, B, V, stream);
}

extern "C" void yh_topk_segments(int64_t V, int64_t top_k, int* n_segments, int* seg_len) {
  // 8192-element segments: 256 threads x 8 vectors of 4; the candidate bound
  // k * 32 <= 2048 fits the LDS list for every k <= 64.  bf16 rows with
  // k <= 32 use half as many 16384-element segments, within this workspace.
  (void)top_k;
  *n_segments = static_cast<int>((V + yh::kSegLen - 1) / yh::kSegLen);
  *seg_len = yh::kSegLen;
}

extern "C" int64_t yh_topk_workspace_bytes(int64_t B, int64_t V, int64_t top_k) {
  int S = 0, seg = 0;
  yh_topk_segments(V, top_k, &S, &seg);
  return B * S * (top_k < 1 ? 1 : top_k) * static_cast<int64_t>(sizeof(uint64_t));
}

extern "C" int yh_presence_penalty(float* scores, const uint8_t* seen, int64_t n, float penalty,
                                   yh_stream_t stream) {
  using namespace yh;
  YH_CHECK_ARG(scores && seen, "presence_penalty: null pointer");
  YH_CHECK_ARG(n >= 0, "presence_penalty: bad size");
  if (n == 0 || penalty == 0.f) return YH_OK;
  const int threads = 256;
  hipLaunchKernelGGL(presence_penalty_kernel, dim3(static_cast<unsigned>((n + threads - 1) / threads)),
                     dim3(threads), 0, static_cast<hipStream_t>(stream), scores, seen, n, penalty);
  YH_CHECK_LAUNCH("presence_penalty");
  return YH_OK;
}

extern "C" int yh_counter_uniform(const int64_t* attempt_ids, const int64_t* steps, int64_t step, uint64_t seed,
                                  uint64_t stream_id, float* out, int64_t n, yh_stream_t stream) {
  using namespace yh;
  YH_CHECK_ARG(attempt_ids && out && n >= 0 && n < (1LL << 31), "counter_uniform: bad arguments");
  if (n == 0) return YH_OK;
  const int threads = 256;
  hipLaunchKernelGGL(counter_uniform_kernel, dim3(static_cast<unsigned>((n + threads - 1) / threads)),
                     dim3(threads), 0, static_cast<hipStream_t>(stream), attempt_ids, steps, step, out, (int)n,
                     static_cast<uint32_t>(seed & 0xffffffffu), static_cast<uint32_t>(stream_id & 0xffffffffu));
  YH_CHECK_LAUNCH("counter_uniform");
  return YH_OK;
}
