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
// segment).  Every thread takes the maximum of its strided elements; the k-th
// largest of those 256 maxima is a lower bound of the segment's k-th largest
// element (k threads hold an element at least that large), so only elements at
// or above it can be in the top k -- at most k * (elements per thread) of
// them.  They are gathered in LDS and ranked by counting.  Elements are
// compared by the unique key (value, -index): larger value first, lower index
// on equal values.  Phase 2: a workgroup per row ranks the segment lists, then
// draws the token.
#include "common.h"

namespace yh {
namespace {

constexpr int kTopkThreads = 256;
constexpr int kMaxK = 64;
constexpr int kCandCap = 4096;
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

constexpr int kVecPerThread = 8;                       // 4-element vectors per thread
constexpr int kSegLen = kTopkThreads * 4 * kVecPerThread;  // 8192 elements per segment
static_assert(kVecPerThread * 4 <= kMaxPerThread, "elements per thread");

// 4 scores (with the presence penalty) starting at element i of row b.
template <int DT, bool VEC>
__device__ __forceinline__ void load_scores4(const TopkArgs& a, int64_t b, int i, float* v) {
  const int64_t off = b * a.row_stride + i;
  if constexpr (VEC) {
    if (i + 3 < a.V) {
      if constexpr (DT == YH_F32) {
        const float4 x = *reinterpret_cast<const float4*>(static_cast<const float*>(a.scores) + off);
        v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w;
      } else {
        const uint2 w = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(a.scores) + off);
        if constexpr (DT == YH_BF16) {
          v[0] = __uint_as_float(w.x << 16); v[1] = __uint_as_float(w.x & 0xffff0000u);
          v[2] = __uint_as_float(w.y << 16); v[3] = __uint_as_float(w.y & 0xffff0000u);
        } else {
          v[0] = f16_to_f32(w.x & 0xffff); v[1] = f16_to_f32(w.x >> 16);
          v[2] = f16_to_f32(w.y & 0xffff); v[3] = f16_to_f32(w.y >> 16);
        }
      }
      if (a.seen) {
        const uint32_t m = *reinterpret_cast<const uint32_t*>(a.seen + b * a.seen_stride + i);
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if ((m >> (8 * j)) & 0xffu) v[j] = v[j] - a.penalty;
      }
      return;
    }
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (i + j < a.V) {
      v[j] = Elem<DT>::ld(static_cast<const typename Elem<DT>::T*>(a.scores), off + j);
      if (a.seen && a.seen[b * a.seen_stride + i + j]) v[j] = v[j] - a.penalty;
    } else {
      v[j] = NAN;  // marks "no element"; never becomes a candidate
    }
  }
}

template <int DT, bool VEC>
__global__ void __launch_bounds__(kTopkThreads) topk_segment_kernel(TopkArgs a) {
  __shared__ uint64_t maxima[kTopkThreads];
  __shared__ uint64_t cand[kCandCap];
  __shared__ uint64_t thr_s;
  __shared__ int ncand;
  const int seg = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const int lo = seg * kSegLen;
  if (tid == 0) {
    ncand = 0;
    thr_s = 0;
  }
  // issue every load of this thread first, then build the keys
  float v[kVecPerThread][4];
#pragma unroll
  for (int c = 0; c < kVecPerThread; ++c) {
    const int i = lo + (c * kTopkThreads + tid) * 4;
    if (i < a.V) load_scores4<DT, VEC>(a, b, i, v[c]);
    else v[c][0] = v[c][1] = v[c][2] = v[c][3] = NAN;
  }
  uint64_t key[kVecPerThread][4];
  uint64_t best = 0;  // key 0 is below every real element key
#pragma unroll
  for (int c = 0; c < kVecPerThread; ++c) {
    const int i = lo + (c * kTopkThreads + tid) * 4;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool real = i + j < a.V;
      key[c][j] = real ? ckey(v[c][j], static_cast<uint32_t>(i + j)) : 0ull;
      best = key[c][j] > best ? key[c][j] : best;
    }
  }
  maxima[tid] = best;
  __syncthreads();
  // Threshold = k-th largest thread maximum.  Real keys are unique, so exactly
  // one thread has rank k-1 when at least k threads hold elements; otherwise the
  // threshold stays 0 and every element of the segment is a candidate (fewer
  // than k threads hold at most (k-1) * per-thread elements).
  if (best != 0) {
    int rank = 0;
    for (int j = 0; j < kTopkThreads; ++j) rank += maxima[j] > best;
    if (rank == a.k - 1) thr_s = best;
  }
  __syncthreads();
  const uint64_t thr = thr_s;
  if (best >= thr && best != 0) {
#pragma unroll
    for (int c = 0; c < kVecPerThread; ++c)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (key[c][j] >= thr && key[c][j] != 0) {
          const int slot = atomicAdd(&ncand, 1);
          if (slot < kCandCap) cand[slot] = key[c][j];
        }
  }
  __syncthreads();
  const int n = min(ncand, kCandCap);
  uint64_t* out = a.work + (static_cast<int64_t>(b) * a.S + seg) * a.k;
  for (int i = tid; i < n; i += kTopkThreads) {
    const uint64_t mine = cand[i];
    int rank = 0;
    for (int j = 0; j < n; ++j) rank += cand[j] > mine;
    if (rank < a.k) out[rank] = mine;
  }
  for (int r = n + tid; r < a.k; r += kTopkThreads) out[r] = 0;  // padding: below every element
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

__global__ void __launch_bounds__(kTopkThreads) sample_rows_kernel(SampleArgs a) {
  __shared__ uint64_t cand[kMaxK * 64];
  __shared__ uint64_t top[kMaxK];
  const int b = blockIdx.x, tid = threadIdx.x;
  const int n = a.S * a.k;
  const uint64_t* src = a.work + static_cast<int64_t>(b) * n;
  for (int i = tid; i < n; i += kTopkThreads) cand[i] = src[i];
  __syncthreads();
  for (int i = tid; i < n; i += kTopkThreads) {
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

extern "C" int yh_topk_sample(const void* scores, int dtype, int64_t row_stride, const uint8_t* seen,
                              int64_t seen_stride, float penalty, const int64_t* attempt_ids,
                              const int64_t* steps, int64_t step, uint64_t seed, uint64_t stream_id,
                              float temperature, int64_t top_k, float top_p, int mode, int64_t* tokens,
                              float* out_values, int64_t* out_indices, void* workspace,
                              int64_t workspace_bytes, int64_t B, int64_t V, yh_stream_t stream) {
  using namespace yh;
  YH_CHECK_ARG(scores && tokens && workspace && attempt_ids, "topk_sample: null pointer");
  YH_CHECK_ARG(B >= 0 && V > 0 && V <= 64LL * kSegLen, "topk_sample: V must lie in [1, %d]", 64 * kSegLen);
  YH_CHECK_ARG(top_k >= 1 && top_k <= kMaxK && top_k <= V, "topk_sample: top_k must lie in [1, %d]", kMaxK);
  YH_CHECK_ARG(dtype == YH_F32 || dtype == YH_BF16 || dtype == YH_F16, "topk_sample: unsupported dtype");
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
  const bool vec = (reinterpret_cast<uintptr_t>(scores) % (4 * esz)) == 0 && row_stride % 4 == 0 &&
                   (seen == nullptr || ((reinterpret_cast<uintptr_t>(seen) & 3) == 0 && seen_stride % 4 == 0));
  const dim3 grid(S, static_cast<unsigned>(B));
  switch (dtype * 2 + (vec ? 1 : 0)) {
    case YH_F32 * 2 + 1: hipLaunchKernelGGL((topk_segment_kernel<YH_F32, true>), grid, dim3(kTopkThreads), 0, st, ta); break;
    case YH_F32 * 2: hipLaunchKernelGGL((topk_segment_kernel<YH_F32, false>), grid, dim3(kTopkThreads), 0, st, ta); break;
    case YH_BF16 * 2 + 1: hipLaunchKernelGGL((topk_segment_kernel<YH_BF16, true>), grid, dim3(kTopkThreads), 0, st, ta); break;
    case YH_BF16 * 2: hipLaunchKernelGGL((topk_segment_kernel<YH_BF16, false>), grid, dim3(kTopkThreads), 0, st, ta); break;
    case YH_F16 * 2 + 1: hipLaunchKernelGGL((topk_segment_kernel<YH_F16, true>), grid, dim3(kTopkThreads), 0, st, ta); break;
    default: hipLaunchKernelGGL((topk_segment_kernel<YH_F16, false>), grid, dim3(kTopkThreads), 0, st, ta); break;
  }
  YH_CHECK_LAUNCH("topk_segment");
  SampleArgs sa{static_cast<const uint64_t*>(workspace), attempt_ids, steps, tokens, out_values, out_indices,
                (int)B, S, (int)top_k, mode, step, static_cast<uint32_t>(seed & 0xffffffffu),
                static_cast<uint32_t>(stream_id & 0xffffffffu), temperature, top_p};
  hipLaunchKernelGGL(sample_rows_kernel, dim3(static_cast<unsigned>(B)), dim3(kTopkThreads), 0, st, sa);
  YH_CHECK_LAUNCH("sample_rows");
  return YH_OK;
}

extern "C" void yh_topk_segments(int64_t V, int64_t top_k, int* n_segments, int* seg_len) {
  // fixed 8192-element segments: 256 threads x 8 vectors of 4; the candidate
  // bound k * 32 <= 2048 fits the LDS list for every k <= 64
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
