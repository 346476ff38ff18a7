// Anchor memory, prefill continuation: the block-wise Top-K scan and the
// state rewrite of IndependentGQAMemory._sequence with a state
// (modeling_yanchor.py:178-275), for prefill chunks that continue a memory
// state (the CausalLM's bounded prefill chunks, modeling_yanchor.py:981-1012;
// the vLLM / SGLang per-request prefill, vllm_yanchor.py:85-96,
// sglang_models/yanchor.py:70-83).
//
// The sequence a row sees is its old pending tokens (count of them) followed
// by its valid new tokens, cut into blocks of C.  Queries of block j read the
// memory committed before block j: the Top-K of the initial committed slots
// and every complete block before j.  The reference computes those prefixes
// with an up-sweep / down-sweep tree of merge_topk (exclusive_prefix_topk,
// modeling_yanchor.py:65-78) and merges the initial state in afterwards
// (217-219).  Top-K under one strict order is a selection of the best K of a
// union, so a left-to-right scan -- memory_{j+1} = TopK(memory_j u block_j) --
// gives the same sets in the same (rank) order, and that is what the decode
// commit does one chunk at a time.  One workgroup per (row, group) ranks the
// committed slots once (the reference merges them into every prefix, so even
// a chunk with no full block leaves them in rank order), then scans the
// blocks; every merge ranks the block's C candidates by counting and places
// them and the memory by binary search in each other's rank order.
//
// Source rows (per batch row, shared by its groups) number the candidates:
//   [0, K)          the committed slots of the state
//   [K, K + C)      the old pending slots
//   [K + C, K + C + L)  the new tokens, in order
// anchor_prefix_kernel writes, per block, the source rows of the memory in
// force (the `read_refs` of modeling_yanchor.py:248), and rewrites the scores,
// positions and pending scores of the state in place; anchor_seq_commit_kernel
// then copies the key / value rows of the final memory and of the new pending
// tokens out of the assembled sources (modeling_yanchor.py:256-274) and
// advances count / total.
#include "common.h"

namespace yh {
namespace {

constexpr int kSeqThreads = 256;
constexpr int kSeqMaxCand = 2048;  // capacity + chunk
constexpr int kSeqMaxChunk = 1024;
constexpr int kSeqPer = kSeqMaxCand / kSeqThreads;

struct PrefixArgs {
  const float* new_scores;  // [B, L, G]   valid tokens first
  const int64_t* counts;    // [B]         valid new tokens per row
  float* scores;            // [B, G, KC]  committed scores (in place)
  int32_t* pos;             // [B, G, KC]  committed positions (in place)
  float* pscores;           // [B, G, PC]  pending scores (in place)
  const int64_t* count;     // [B]
  const int64_t* total;     // [B]
  int32_t* block_refs;      // [B, NB, G, KC]
  int32_t* final_refs;      // [B, G, KC]
  int32_t* pending_refs;    // [B, G, PC]
  int L, G, KC, PC, C, NB;
};

// Rank candidates [0, n) by counting (score descending, position ascending
// with invalid last, candidate index ascending) and move the best `keep` to
// [0, keep) in rank order.  Starts and ends with a workgroup barrier.
__device__ __forceinline__ void rank_into_memory(uint64_t* ckey, float* cscore, int32_t* cpos, int32_t* cref,
                                                 int32_t* chosen, int n, int keep, int tid) {
  __syncthreads();
  for (int i = tid; i < n; i += kSeqThreads) ckey[i] = topk_key(cscore[i], cpos[i]);
  __syncthreads();
  for (int i = tid; i < n; i += kSeqThreads) {
    const uint64_t mine = ckey[i];
    int rank = 0;
    for (int m = 0; m < n; ++m) {
      const uint64_t o = ckey[m];
      rank += (o < mine) | ((o == mine) & (m < i));
    }
    if (rank < keep) chosen[rank] = i;
  }
  __syncthreads();
  float rs[kSeqPer];
  int32_t rp[kSeqPer], rr[kSeqPer];
#pragma unroll
  for (int k = 0; k < kSeqPer; ++k) {
    const int s = tid + k * kSeqThreads;
    if (s < keep) {
      const int src = chosen[s];
      rs[k] = cscore[src];
      rp[k] = cpos[src];
      rr[k] = cref[src];
    }
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < kSeqPer; ++k) {
    const int s = tid + k * kSeqThreads;
    if (s < keep) {
      cscore[s] = rs[k];
      cpos[s] = rp[k];
      cref[s] = rr[k];
    }
  }
  __syncthreads();
}

// The memory [0, KC) is in rank order.  Merge the C candidates at [KC, KC + C)
// in (the next block, in token order) and keep the best KC, in rank order:
// the same result as rank_into_memory over all KC + C (one strict order:
// key, then candidate index, so a memory entry wins a tie with a block entry
// and block entries tie in token order).  The block is ranked by counting
// (C x C), then each entry's merged rank is its place in its own list plus the
// number of the other list's entries above it (a binary search).  Starts and
// ends with a workgroup barrier.
__device__ __forceinline__ void merge_into_memory(uint64_t* ckey, float* cscore, int32_t* cpos, int32_t* cref,
                                                  int32_t* chosen, int KC, int C, int tid) {
  __syncthreads();
  for (int i = tid; i < KC + C; i += kSeqThreads) ckey[i] = topk_key(cscore[i], cpos[i]);
  __syncthreads();
  for (int i = tid; i < C; i += kSeqThreads) {  // the block in rank order: chosen[r] = its candidate
    const uint64_t mine = ckey[KC + i];
    int rank = 0;
    for (int m = 0; m < C; ++m) {
      const uint64_t o = ckey[KC + m];
      rank += (o < mine) | ((o == mine) & (m < i));
    }
    chosen[rank] = KC + i;
  }
  __syncthreads();
  // merged ranks: memory entry p is above block entries with key >= its own;
  // block entry q (in block rank order) is above memory entries with key > its own
  float rs[kSeqPer];
  int32_t rp[kSeqPer], rr[kSeqPer], rk[kSeqPer];
#pragma unroll
  for (int k = 0; k < kSeqPer; ++k) {
    const int e = tid + k * kSeqThreads;  // [0, KC): memory p = e; [KC, KC + C): block rank q = e - KC
    rk[k] = KC;                            // not kept
    if (e < KC + C) {
      int src, rank;
      if (e < KC) {
        src = e;
        const uint64_t mine = ckey[e];
        int lo = 0, hi = C;  // block entries (rank order, keys non-decreasing) with key < mine
        while (lo < hi) {
          const int mid = (lo + hi) >> 1;
          if (ckey[chosen[mid]] < mine) lo = mid + 1; else hi = mid;
        }
        rank = e + lo;
      } else {
        const int q = e - KC;
        src = chosen[q];
        const uint64_t mine = ckey[src];
        int lo = 0, hi = KC;  // memory entries (rank order) with key <= mine
        while (lo < hi) {
          const int mid = (lo + hi) >> 1;
          if (ckey[mid] <= mine) lo = mid + 1; else hi = mid;
        }
        rank = q + lo;
      }
      if (rank < KC) {
        rk[k] = rank;
        rs[k] = cscore[src];
        rp[k] = cpos[src];
        rr[k] = cref[src];
      }
    }
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < kSeqPer; ++k) {
    if (rk[k] < KC) {
      cscore[rk[k]] = rs[k];
      cpos[rk[k]] = rp[k];
      cref[rk[k]] = rr[k];
    }
  }
  __syncthreads();
}

__global__ void __launch_bounds__(kSeqThreads) anchor_prefix_kernel(PrefixArgs a) {
  __shared__ uint64_t ckey[kSeqMaxCand];
  __shared__ float cscore[kSeqMaxCand];
  __shared__ int32_t cpos[kSeqMaxCand];
  __shared__ int32_t cref[kSeqMaxCand];
  __shared__ int32_t chosen[kSeqMaxCand];
  __shared__ float opend[kSeqMaxChunk];

  const int tid = threadIdx.x;
  const int64_t bg = blockIdx.x;
  const int64_t b = bg / a.G;
  const int g = static_cast<int>(bg % a.G);
  const int KC = a.KC, C = a.C, G = a.G, N = KC + C;
  int32_t* brefs = a.block_refs + (b * a.NB * G + g) * KC;  // block j at + j * G * KC
  const int64_t old_count = a.count[b];
  if (old_count < 0 || old_count >= C) {
    // corrupt counter: the row reads nothing and its state is left untouched
    for (int j = 0; j < a.NB; ++j)
      for (int s = tid; s < KC; s += kSeqThreads) brefs[static_cast<int64_t>(j) * G * KC + s] = -1;
    return;
  }
  const int64_t n_new = min(max(a.counts[b], static_cast<int64_t>(0)), static_cast<int64_t>(a.L));
  const int64_t n_all = old_count + n_new;
  const int64_t full = n_all / C, rem = n_all - full * C;
  const int64_t base_pos = a.total[b] - old_count;
  float* scores = a.scores + bg * KC;
  int32_t* pos = a.pos + bg * KC;
  float* pscores = a.pscores + bg * a.PC;
  const float* nsc = a.new_scores + b * a.L * G + g;  // token i at nsc[i * G]

  for (int s = tid; s < KC; s += kSeqThreads) {
    const int32_t p = pos[s];
    cscore[s] = scores[s];
    cpos[s] = p >= 0 ? p : -1;
    cref[s] = p >= 0 ? s : -1;
  }
  for (int t = tid; t < old_count; t += kSeqThreads) opend[t] = pscores[t];

  // Rank the committed slots once (the merge of the initial state into an
  // empty prefix, modeling_yanchor.py:217-219): the memory is kept in rank
  // order from here on, also when no block completes.
  rank_into_memory(ckey, cscore, cpos, cref, chosen, KC, KC, tid);

  for (int j = 0; j < a.NB; ++j) {
    int32_t* out = brefs + static_cast<int64_t>(j) * G * KC;
    for (int s = tid; s < KC; s += kSeqThreads) out[s] = cref[s];
    if (j >= full) continue;  // uniform: the memory stays as it is
    // candidates: the memory [0, KC), then block j's C tokens
    for (int n = KC + tid; n < N; n += kSeqThreads) {
      const int64_t q = static_cast<int64_t>(j) * C + (n - KC);  // sequence index
      const bool old = q < old_count;
      cscore[n] = old ? opend[q] : nsc[(q - old_count) * G];
      cpos[n] = static_cast<int32_t>(base_pos + q);
      cref[n] = static_cast<int32_t>(old ? KC + q : KC + C + (q - old_count));
    }
    merge_into_memory(ckey, cscore, cpos, cref, chosen, KC, C, tid);
  }

  // the final memory, in rank order, and the tokens left pending
  int32_t* frefs = a.final_refs + bg * KC;
  for (int s = tid; s < KC; s += kSeqThreads) {
    scores[s] = cscore[s];
    pos[s] = cpos[s];
    frefs[s] = cref[s];
  }
  int32_t* prefs = a.pending_refs + bg * a.PC;
  for (int t = tid; t < a.PC; t += kSeqThreads) {
    float sc = -INFINITY;
    int32_t ref = -1;
    if (t < rem) {
      const int64_t q = full * C + t;
      const bool old = q < old_count;
      sc = old ? opend[q] : nsc[(q - old_count) * G];
      ref = static_cast<int32_t>(old ? KC + q : KC + C + (q - old_count));
    }
    pscores[t] = sc;
    prefs[t] = ref;
  }
}

struct SeqCommitArgs {
  const char* src_k;          // [B, S, G, D]
  const char* src_v;
  const int32_t* final_refs;  // [B, G, KC]
  const int32_t* pending_refs;  // [B, G, PC]
  const int64_t* counts;      // [B]
  char* keys;                 // [B, G, KC, D]
  char* values;
  char* pkeys;                // [B, G, PC, D]
  char* pvalues;
  int64_t* count;             // [B]
  int64_t* total;             // [B]
  int S, G, KC, PC, C, L;
  int64_t rowbytes;
};

// One workgroup per (row, group): the committed slots and the pending slots
// take their key / value rows from the sources (zeros where no row is
// referenced, as the masked copies of the reference).  Group 0 advances the
// row's count and total.  A corrupt count leaves the row untouched.
__global__ void __launch_bounds__(kSeqThreads) anchor_seq_commit_kernel(SeqCommitArgs a) {
  const int tid = threadIdx.x;
  const int64_t bg = blockIdx.x;
  const int64_t b = bg / a.G;
  const int g = static_cast<int>(bg % a.G);
  const int64_t old_count = a.count[b];
  if (old_count < 0 || old_count >= a.C) return;
  const int pieces = static_cast<int>(a.rowbytes / 16);
  const int64_t rows = static_cast<int64_t>(a.KC) + a.PC;
  for (int64_t idx = tid; idx < rows * pieces; idx += kSeqThreads) {
    const int64_t slot = idx / pieces;
    const int c = static_cast<int>(idx % pieces);
    int32_t ref;
    int64_t dst;
    char *dk, *dv;
    if (slot < a.KC) {
      ref = a.final_refs[bg * a.KC + slot];
      dst = (bg * a.KC + slot) * a.rowbytes;
      dk = a.keys;
      dv = a.values;
    } else {
      ref = a.pending_refs[bg * a.PC + (slot - a.KC)];
      dst = (bg * a.PC + (slot - a.KC)) * a.rowbytes;
      dk = a.pkeys;
      dv = a.pvalues;
    }
    uint4 k = make_uint4(0, 0, 0, 0), v = k;
    if (ref >= 0 && ref < a.S) {
      const int64_t src = ((b * a.S + ref) * a.G + g) * a.rowbytes;
      k = reinterpret_cast<const uint4*>(a.src_k + src)[c];
      v = reinterpret_cast<const uint4*>(a.src_v + src)[c];
    }
    reinterpret_cast<uint4*>(dk + dst)[c] = k;
    reinterpret_cast<uint4*>(dv + dst)[c] = v;
  }
  if (g == 0 && tid == 0) {
    const int64_t n = min(max(a.counts[b], static_cast<int64_t>(0)), static_cast<int64_t>(a.L));
    a.count[b] = (old_count + n) % a.C;
    a.total[b] += n;
  }
}

}  // namespace
}  // namespace yh

extern "C" int yh_anchor_prefix(const float* new_scores, const int64_t* counts, float* scores, int32_t* positions,
                                float* pending_scores, const int64_t* count, const int64_t* total,
                                int32_t* block_refs, int32_t* final_refs, int32_t* pending_refs, int64_t B, int64_t L,
                                int64_t G, int64_t capacity, int64_t pending_capacity, int64_t chunk, int64_t NB,
                                yh_stream_t stream) {
  using namespace yh;
  YH_CHECK_ARG(B >= 0 && L >= 0 && G > 0 && capacity > 0 && NB >= 0, "anchor_prefix: bad sizes");
  YH_CHECK_ARG(chunk >= 1 && chunk <= pending_capacity && chunk <= kSeqMaxChunk,
               "anchor_prefix: chunk must be in [1, min(pending capacity, %d)]", kSeqMaxChunk);
  YH_CHECK_ARG(capacity + chunk <= kSeqMaxCand, "anchor_prefix: capacity + chunk must be <= %d", kSeqMaxCand);
  YH_CHECK_ARG(NB * chunk >= L + chunk - 1, "anchor_prefix: %lld blocks of %lld cannot hold %lld pending + new tokens",
               (long long)NB, (long long)chunk, (long long)(L + chunk - 1));
  YH_CHECK_ARG(capacity + chunk + L < (1LL << 31) && B * G < (1LL << 31), "anchor_prefix: too large");
  if (B == 0) return YH_OK;
  YH_CHECK_ARG(counts && scores && positions && pending_scores && count && total && final_refs && pending_refs &&
                   (L == 0 || new_scores) && (NB == 0 || block_refs),
               "anchor_prefix: null pointer");
  PrefixArgs a{new_scores, counts, scores, positions, pending_scores, count, total, block_refs, final_refs,
               pending_refs, (int)L, (int)G, (int)capacity, (int)pending_capacity, (int)chunk, (int)NB};
  hipLaunchKernelGGL(anchor_prefix_kernel, dim3(static_cast<unsigned>(B * G)), dim3(kSeqThreads), 0,
                     static_cast<hipStream_t>(stream), a);
  YH_CHECK_LAUNCH("anchor_prefix");
  return YH_OK;
}

extern "C" int yh_anchor_sequence_commit(const void* src_keys, const void* src_values, const int32_t* final_refs,
                                         const int32_t* pending_refs, const int64_t* counts, void* keys, void* values,
                                         void* pending_keys, void* pending_values, int64_t* count, int64_t* total,
                                         int64_t B, int64_t S, int64_t L, int64_t G, int64_t capacity,
                                         int64_t pending_capacity, int64_t chunk, int64_t D, int dtype,
                                         yh_stream_t stream) {
  using namespace yh;
  YH_CHECK_ARG(B >= 0 && S >= 0 && L >= 0 && G > 0 && capacity > 0 && pending_capacity > 0 && D > 0,
               "anchor_sequence_commit: bad sizes");
  YH_CHECK_ARG(chunk >= 1 && chunk <= pending_capacity, "anchor_sequence_commit: chunk outside [1, pending capacity]");
  YH_CHECK_ARG(is_float_dtype(dtype), "anchor_sequence_commit: unsupported dtype %d", dtype);
  const int64_t rowbytes = D * (dtype == YH_F32 ? 4 : 2);
  YH_CHECK_ARG(rowbytes % 16 == 0, "anchor_sequence_commit: a row must be a multiple of 16 bytes");
  YH_CHECK_ARG(S < (1LL << 31) && B * G < (1LL << 31), "anchor_sequence_commit: too large");
  if (B == 0) return YH_OK;
  YH_CHECK_ARG(src_keys && src_values && final_refs && pending_refs && counts && keys && values && pending_keys &&
                   pending_values && count && total,
               "anchor_sequence_commit: null pointer");
  YH_CHECK_ARG(((reinterpret_cast<uintptr_t>(src_keys) | reinterpret_cast<uintptr_t>(src_values) |
                 reinterpret_cast<uintptr_t>(keys) | reinterpret_cast<uintptr_t>(values) |
                 reinterpret_cast<uintptr_t>(pending_keys) | reinterpret_cast<uintptr_t>(pending_values)) & 15) == 0,
               "anchor_sequence_commit: key/value tensors must be 16-byte aligned");
  SeqCommitArgs a{static_cast<const char*>(src_keys), static_cast<const char*>(src_values), final_refs,
                  pending_refs, counts, static_cast<char*>(keys), static_cast<char*>(values),
                  static_cast<char*>(pending_keys), static_cast<char*>(pending_values), count, total,
                  (int)S, (int)G, (int)capacity, (int)pending_capacity, (int)chunk, (int)L, rowbytes};
  hipLaunchKernelGGL(anchor_seq_commit_kernel, dim3(static_cast<unsigned>(B * G)), dim3(kSeqThreads), 0,
                     static_cast<hipStream_t>(stream), a);
  YH_CHECK_LAUNCH("anchor_sequence_commit");
  return YH_OK;
}
