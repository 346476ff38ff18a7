// Skinny bf16 projection for the decode step: out[M, N] = x[M, K] . W[N, K]^T
// with M <= 128 (one row per live slot), fp32 accumulation, bf16 output --
// torch.nn.functional.linear without bias, as every projection of the decode
// layers (modeling_yanchor.py:147-176; the Qwen3.5 GDN / attention / MLP
// projections in the transformers wheel).
//
// At M <= 128 the product is bound by streaming W once from HBM (2 bytes per
// weight, 2M FLOP per weight), with MFMA work close behind (at M = 128 the
// HBM rate needs ~40 % of the MFMA peak).  The runtime uses this kernel where
// it beats the library GEMM: output widths up to 4096 with long K, where a
// split K fills the chip.  Layout of the work:
//   * a workgroup (4 waves) owns 128 output columns and a slice of K; wave w
//     owns columns 32w .. 32w+31 (two 16-column MFMA tiles) and all M rows
//     (ceil(M/16) row tiles), so every x fragment read from LDS feeds two
//     MFMAs;
//   * W fragments go straight from HBM into registers as the B operand of
//     16x16x32 bf16 MFMA (lane: 16 contiguous bytes of one weight row), four
//     64-wide K chunks ahead of use (a register ring), so each workgroup keeps
//     64 KiB of weights in flight;
//   * x chunks (M x 64) are staged through double-buffered LDS, shared by the
//     four waves, and read as the A operand (row stride padded to 144 bytes:
//     16-byte reads of 16 different rows hit distinct banks);
//   * x chunks are loaded two chunks ahead into registers, so their L2
//     latency is hidden behind two chunks of MFMA work;
//   * with K split over S workgroups per column tile (to fill the chip when N
//     is small), each slice writes an fp32 partial tile to the
//     workspace and a second kernel sums the S partials in slice order -- a
//     fixed order, so results do not depend on scheduling.
#include <algorithm>

#include "common.h"

namespace yh {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4v __attribute__((ext_vector_type(4)));

constexpr int kLinThreads = 256;
constexpr int kNT = 128;         // output columns per workgroup (4 waves x 2 tiles of 16)
constexpr int kNQ = 64;          // N granularity accepted by the entry point
constexpr int kKC = 64;          // K per chunk
constexpr int kXPad = kKC + 8;   // LDS row stride (elements) of an x chunk
constexpr int kMaxM = 128;


struct LinArgs {
  const uint16_t* x;   // [M, K], row stride xs
  const uint16_t* w;   // [N, K]
  uint16_t* out;       // [M, N], row stride os
  float* part;         // [S, M, N] fp32 partials (S > 1)
  int64_t xs, os;
  int M, N, K, S, chunks_per_slice;
  const uint16_t* res;  // optional residual [M, N], rows rs apart: out = bf16(bf16(x . W^T) + res)
  int64_t rs;
  int silu_pairs;       // packed gate|up pairs: out[M, N/2] = bf16(bf16(silu(gate)) * up)
};

typedef unsigned int u32x4v __attribute__((ext_vector_type(4)));

// 16 bytes of a weight row, streamed past the caches' retention (each weight
// is used by exactly one workgroup).
__device__ __forceinline__ uint4 ld_w16(const uint16_t* p) {
  return __builtin_bit_cast(uint4, __builtin_nontemporal_load(reinterpret_cast<const u32x4v*>(p)));
}

// Workgroup barrier that waits only for this wave's LDS traffic.  The plain
// __syncthreads() also drains every outstanding global load (vmcnt(0)), which
// would empty the weight and x prefetch rings at every chunk.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

__device__ __forceinline__ f32x4v mfma(bf16x8_t a, bf16x8_t b, f32x4v c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Rows [0, 16 MT) x [k, k + 64) of x into registers.  Rows >= M re-read row
// M-1: output row m depends on x row m only, and rows >= M are never stored,
// so no masking (and no branch) is needed -- which also lets the compiler
// count the loads in flight.  256 threads x NV vectors of 8 elements.
template <int MT>
__device__ __forceinline__ void load_x(const LinArgs& a, int k, uint4 (&r)[MT * 16 * 8 / kLinThreads]) {
  constexpr int NV = MT * 16 * 8 / kLinThreads;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int idx = i * kLinThreads + threadIdx.x;
    const int row = idx >> 3, c8 = (idx & 7) * 8;
    r[i] = *reinterpret_cast<const uint4*>(a.x + min(row, a.M - 1) * a.xs + k + c8);
  }
}
template <int MT>
__device__ __forceinline__ void store_x(uint16_t (*buf)[kXPad], const uint4 (&r)[MT * 16 * 8 / kLinThreads]) {
  constexpr int NV = MT * 16 * 8 / kLinThreads;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int idx = i * kLinThreads + threadIdx.x;
    const int row = idx >> 3, c8 = (idx & 7) * 8;
    *reinterpret_cast<uint4*>(&buf[row][c8]) = r[i];
  }
}

constexpr int kWDepth = 4;  // K chunks of W in flight per lane

template <int MT>
struct Pipe {
  uint4 wr[kWDepth][2][2];                  // W ring: [chunk slot][column tile][k step]
  uint4 xr[2][MT * 16 * 8 / kLinThreads];   // x ring: chunk c in xr[(c - c0) % 2]
  f32x4v acc[MT][2];
};

template <int MT, int U>
__device__ __forceinline__ void load_w(Pipe<MT>& p, const uint16_t* const (&wrow)[2], int c) {
#pragma unroll
  for (int ct = 0; ct < 2; ++ct) {
    p.wr[U][ct][0] = ld_w16(wrow[ct] + c * kKC);
    p.wr[U][ct][1] = ld_w16(wrow[ct] + c * kKC + 32);
  }
}

// One K chunk c (ring slot U = (c - c0) % kWDepth): load x two chunks ahead,
// 2 steps x MT row tiles x 2 column tiles of MFMA (each A fragment read from
// LDS once and used for both column tiles), load W kWDepth chunks ahead, move
// the next x chunk to LDS.  Loads past the slice end re-read its last chunk
// (no branches).
template <int MT, int U>
__device__ __forceinline__ void chunk_step(Pipe<MT>& p, uint16_t (*xs)[MT * 16][kXPad], const LinArgs& a,
                                           const uint16_t* const (&wrow)[2], int c, int c1, int col, int quad) {
  load_x<MT>(a, min(c + 2, c1 - 1) * kKC, p.xr[U & 1]);
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const bf16x8_t b0 = __builtin_bit_cast(bf16x8_t, p.wr[U][0][s]);
    const bf16x8_t b1 = __builtin_bit_cast(bf16x8_t, p.wr[U][1][s]);
    bf16x8_t av[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t)
      av[t] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(&xs[U & 1][t * 16 + col][s * 32 + quad * 8]));
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      p.acc[t][0] = mfma(av[t], b0, p.acc[t][0]);
      p.acc[t][1] = mfma(av[t], b1, p.acc[t][1]);
    }
  }
  load_w<MT, U>(p, wrow, min(c + kWDepth, c1 - 1));
  store_x<MT>(xs[(U + 1) & 1], p.xr[(U + 1) & 1]);
  lds_barrier();
}

template <int MT>
__global__ void __launch_bounds__(kLinThreads) skinny_linear_kernel(LinArgs a) {
  static_assert(MT * 16 * 8 % kLinThreads == 0, "x chunk must split evenly over the workgroup");
  static_assert(kWDepth == 4, "the main loop is unrolled over the W ring");
  __shared__ __align__(16) uint16_t xs[2][MT * 16][kXPad];

  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int col = lane & 15, quad = lane >> 4;
  const int tile = blockIdx.x, slice = blockIdx.y;
  const int total_chunks = a.K / kKC;
  const int c0 = slice * a.chunks_per_slice;
  const int c1 = min(total_chunks, c0 + a.chunks_per_slice);
  int ncol[2];
  const uint16_t* wrow[2];
#pragma unroll
  for (int ct = 0; ct < 2; ++ct) {
    ncol[ct] = tile * kNT + w * 32 + ct * 16 + col;  // output column / weight row of this lane
    wrow[ct] = a.w + static_cast<int64_t>(min(ncol[ct], a.N - 1)) * a.K + quad * 8;
  }

  Pipe<MT> p;
#pragma unroll
  for (int t = 0; t < MT; ++t) p.acc[t][0] = p.acc[t][1] = f32x4v{0.f, 0.f, 0.f, 0.f};

  if (c0 < c1) {
    // Same issue order as a loop step (x, then W), so the wait counts the
    // compiler derives at the loop head stay those of the steady state.
    load_x<MT>(a, c0 * kKC, p.xr[0]);
    load_x<MT>(a, min(c0 + 1, c1 - 1) * kKC, p.xr[1]);
    load_w<MT, 0>(p, wrow, c0);
    load_w<MT, 1>(p, wrow, min(c0 + 1, c1 - 1));
    load_w<MT, 2>(p, wrow, min(c0 + 2, c1 - 1));
    load_w<MT, 3>(p, wrow, min(c0 + 3, c1 - 1));
    store_x<MT>(xs[0], p.xr[0]);
    lds_barrier();
    int c = c0;
    for (; c + kWDepth <= c1; c += kWDepth) {
      chunk_step<MT, 0>(p, xs, a, wrow, c, c1, col, quad);
      chunk_step<MT, 1>(p, xs, a, wrow, c + 1, c1, col, quad);
      chunk_step<MT, 2>(p, xs, a, wrow, c + 2, c1, col, quad);
      chunk_step<MT, 3>(p, xs, a, wrow, c + 3, c1, col, quad);
    }
    if (c < c1) chunk_step<MT, 0>(p, xs, a, wrow, c, c1, col, quad);
    if (c + 1 < c1) chunk_step<MT, 1>(p, xs, a, wrow, c + 1, c1, col, quad);
    if (c + 2 < c1) chunk_step<MT, 2>(p, xs, a, wrow, c + 2, c1, col, quad);
  }

  // acc[t][ct][i] = out[t*16 + quad*4 + i][ncol[ct]]
  if (a.S == 1) {
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      if (ncol[ct] >= a.N) continue;
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int m = t * 16 + quad * 4 + i;
          if (m < a.M) a.out[m * a.os + ncol[ct]] = f32_to_bf16(p.acc[t][ct][i]);
        }
    }
    return;
  }
  float* mine = a.part + static_cast<int64_t>(slice) * a.M * a.N;
#pragma unroll
  for (int ct = 0; ct < 2; ++ct) {
    if (ncol[ct] >= a.N) continue;
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = t * 16 + quad * 4 + i;
        if (m < a.M) mine[static_cast<int64_t>(m) * a.N + ncol[ct]] = p.acc[t][ct][i];
      }
  }
}

// out = bf16(sum_s part[s]) in slice order (a fixed order: results do not
// depend on scheduling); 4 columns per thread.
__global__ void __launch_bounds__(256) linear_reduce_kernel(const float* part, uint16_t* out, int64_t os, int M,
                                                            int N, int S, const uint16_t* res, int64_t rs) {
  const int64_t e = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t per_row = N / 4;
  if (e >= static_cast<int64_t>(M) * per_row) return;
  const int64_t m = e / per_row, c = (e % per_row) * 4;
  const float* p = part + m * N + c;
  const int64_t plane = static_cast<int64_t>(M) * N;
  // planes are loaded eight at a time (all in flight together), then added
  // in slice order
  float4 sum = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int s0 = 0; s0 < S; s0 += 8) {
    float4 v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (s0 + j < S) v[j] = *reinterpret_cast<const float4*>(p + (s0 + j) * plane);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (s0 + j >= S) break;
      if (s0 + j == 0) {
        sum = v[0];
      } else {
        sum.x += v[j].x;
        sum.y += v[j].y;
        sum.z += v[j].z;
        sum.w += v[j].w;
      }
    }
  }
  if (res) {  // the product is a bf16 tensor before the residual add
    const uint2 r = *reinterpret_cast<const uint2*>(res + m * rs + c);
    sum.x = bf16_to_f32(f32_to_bf16(sum.x)) + bf16_to_f32(static_cast<uint16_t>(r.x & 0xffff));
    sum.y = bf16_to_f32(f32_to_bf16(sum.y)) + bf16_to_f32(static_cast<uint16_t>(r.x >> 16));
    sum.z = bf16_to_f32(f32_to_bf16(sum.z)) + bf16_to_f32(static_cast<uint16_t>(r.y & 0xffff));
    sum.w = bf16_to_f32(f32_to_bf16(sum.w)) + bf16_to_f32(static_cast<uint16_t>(r.y >> 16));
  }
  const uint2 o = make_uint2(static_cast<uint32_t>(f32_to_bf16(sum.x)) | (static_cast<uint32_t>(f32_to_bf16(sum.y)) << 16),
                             static_cast<uint32_t>(f32_to_bf16(sum.z)) | (static_cast<uint32_t>(f32_to_bf16(sum.w)) << 16));
  *reinterpret_cast<uint2*>(out + m * os + c) = o;
}

// ---- Packed weights -----------------------------------------------------------
// The weights of the decode projections are repacked once (yh_linear_pack)
// into MFMA fragment order: for column tile T (16 output columns) and K block
// kb (32 of K) the 1 KiB B operand of one 16x16x32 MFMA is stored
// contiguously, lane l holding W[16 T + l % 16][32 kb + 8 (l / 16) .. + 8],
// and the N/16 tiles of one K block follow each other:
//   packed[((kb * N/16 + T) * 64 + l) * 8 + e] = W[16 T + l % 16][32 kb + 8 (l / 16) + e]
// A wave's weight load is then one contiguous 1 KiB (eight whole 128-byte
// lines).  From the row-major layout every load takes 64 bytes from each of 16
// rows, and the number of line misses a CU keeps in flight caps the streaming
// rate (measured on MI355X at M = 128: 3.0 -> 4.5 TB/s on a 168 MB weight).
// K blocks outermost put the blocks that every workgroup of a projection
// reads in the same phase side by side (one moving window of ~N KiB rather
// than N/16 stripes K/32 KiB apart): 30.3 -> 28.5 us for the 19456 x 2560
// MLP gate/up at M = 128, 29.9 -> 27.0 for the 16448 x 2560 GDN input.
// The projection kernels on this layout are in proj.hip.

// W [N, K] row-major -> packed fragment order; one thread per 16-byte piece.
// With pair_halves the column tiles alternate between the two row halves of W
// (tile 2j = rows 16j.., tile 2j+1 = rows N/2 + 16j..), so a wave holds a
// gate tile and its up tile.
__global__ void __launch_bounds__(256) linear_pack_kernel(const uint16_t* w, uint16_t* packed, int64_t N, int64_t K,
                                                          int pair_halves) {
  const int64_t piece = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;  // packed order
  if (piece >= N * K / 8) return;
  const int64_t l = piece & 63, blk = piece >> 6;  // blk = kb * N/16 + T
  const int64_t tiles = N / 16, T = blk % tiles, kb = blk / tiles;
  const int64_t src_tile = pair_halves ? (T & 1) * (N / 32) + (T >> 1) : T;
  const int64_t row = src_tile * 16 + (l & 15), k = kb * 32 + (l >> 4) * 8;
  reinterpret_cast<uint4*>(packed)[piece] = *reinterpret_cast<const uint4*>(w + row * K + k);
}

// Split-K factor S (a power of two, at most 8): grow S while the grid is
// under one workgroup per CU, every slice keeps >= 4 chunks, and the fp32
// partials (written and read once: 8 S M N bytes) stay under twice the weight
// bytes (2 N K).  Measured on MI355X at M = 128: S = 8 is best for N = 2560
// with K = 2560 ... 9728; large N needs no split.
int pick_split(int64_t M, int64_t N, int64_t K) {
  const int64_t tiles = (N + kNT - 1) / kNT, chunks = K / kKC;
  int64_t s = 1;
  while (s < 8 && tiles * s < 256 && chunks / (s * 2) >= 4 && (s * 2) * M <= K / 2) s *= 2;
  return static_cast<int>(s);
}

}  // namespace
}  // namespace yh

extern "C" int yh_linear_split(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N < yh::kNQ || K < yh::kKC) return 1;
  return yh::pick_split(M, N, K);
}

extern "C" int64_t yh_linear_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t split_k) {
  (void)K;
  if (split_k <= 1) return 0;
  return split_k * M * N * 4;
}

extern "C" int yh_linear(const void* x, int64_t x_stride, const void* w, void* out, int64_t out_stride, int64_t M,
                         int64_t N, int64_t K, int64_t split_k, void* workspace, int64_t workspace_bytes,
                         yh_stream_t stream) {
  using namespace yh;
  YH_CHECK_ARG(M >= 0 && M <= kMaxM, "linear: M must be in [0, %d] (got %lld)", kMaxM, (long long)M);
  YH_CHECK_ARG(N > 0 && N % kNQ == 0, "linear: N must be a positive multiple of %d", kNQ);
  YH_CHECK_ARG(K > 0 && K % kKC == 0, "linear: K must be a positive multiple of %d", kKC);
  YH_CHECK_ARG(x_stride >= K && x_stride % 8 == 0 && out_stride >= N, "linear: bad strides");
  YH_CHECK_ARG(split_k >= 1 && split_k <= K / kKC, "linear: split_k must be in [1, K/%d]", kKC);
  if (M == 0) return YH_OK;
  YH_CHECK_ARG(x && w && out, "linear: null pointer");
  YH_CHECK_ARG(((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w)) & 15) == 0,
               "linear: x and w must be 16-byte aligned");
  const int64_t need = yh_linear_workspace_bytes(M, N, K, split_k);
  YH_CHECK_ARG(split_k == 1 || (workspace && workspace_bytes >= need),
               "linear: workspace of %lld bytes required", (long long)need);
  const int64_t chunks = K / kKC;
  const int cps = static_cast<int>((chunks + split_k - 1) / split_k);
  const int S = static_cast<int>((chunks + cps - 1) / cps);  // slices that own at least one chunk
  float* part = S > 1 ? static_cast<float*>(workspace) : nullptr;
  YH_CHECK_ARG(S == 1 || (reinterpret_cast<uintptr_t>(workspace) & 15) == 0, "linear: workspace must be 16-byte aligned");
  YH_CHECK_ARG(S == 1 || out_stride % 4 == 0, "linear: split-K output rows must be 8-byte aligned");
  LinArgs a{static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(w), static_cast<uint16_t*>(out), part,
            x_stride, out_stride, (int)M, (int)N, (int)K, S, cps};
  const dim3 grid(static_cast<unsigned>((N + kNT - 1) / kNT), static_cast<unsigned>(S));
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int mt = static_cast<int>((M + 15) / 16);
  switch (mt <= 2 ? 2 : mt <= 4 ? 4 : 8) {
    case 2: hipLaunchKernelGGL(skinny_linear_kernel<2>, grid, dim3(kLinThreads), 0, st, a); break;
    case 4: hipLaunchKernelGGL(skinny_linear_kernel<4>, grid, dim3(kLinThreads), 0, st, a); break;
    default: hipLaunchKernelGGL(skinny_linear_kernel<8>, grid, dim3(kLinThreads), 0, st, a); break;
  }
  YH_CHECK_LAUNCH("linear");
  if (S > 1) {
    const int64_t quads = M * N / 4;
    hipLaunchKernelGGL(linear_reduce_kernel, dim3(static_cast<unsigned>((quads + 255) / 256)), dim3(256), 0, st,
                       part, static_cast<uint16_t*>(out), out_stride, (int)M, (int)N, S, nullptr, 0);
    YH_CHECK_LAUNCH("linear_reduce");
  }
  return YH_OK;
}

extern "C" int yh_linear_pack(const void* w, void* packed, int64_t N, int64_t K, int pair_halves,
                              yh_stream_t stream) {
  using namespace yh;
  YH_CHECK_ARG(N > 0 && N % 16 == 0 && K > 0 && K % 32 == 0, "linear_pack: N must be a multiple of 16, K of 32");
  YH_CHECK_ARG(!pair_halves || N % 32 == 0, "linear_pack: paired halves need N % 32 == 0");
  YH_CHECK_ARG(w && packed && w != packed, "linear_pack: null or aliased pointer");
  YH_CHECK_ARG(((reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(packed)) & 15) == 0,
               "linear_pack: tensors must be 16-byte aligned");
  const int64_t pieces = N * K / 8;
  YH_CHECK_ARG((pieces + 255) / 256 < (1LL << 31), "linear_pack: too large");
  hipLaunchKernelGGL(linear_pack_kernel, dim3(static_cast<unsigned>((pieces + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(w), static_cast<uint16_t*>(packed),
                     N, K, pair_halves);
  YH_CHECK_LAUNCH("linear_pack");
  return YH_OK;
}

extern "C" int yh_linear_reduce(const float* part, void* out, int64_t out_stride, int64_t M, int64_t N, int64_t S,
                                const void* residual, int64_t residual_stride, yh_stream_t stream) {
  using namespace yh;
  YH_CHECK_ARG(M >= 0 && N > 0 && N % 4 == 0 && S >= 1 && out_stride >= N && out_stride % 4 == 0,
               "linear_reduce: bad sizes");
  YH_CHECK_ARG(!residual || (residual_stride >= N && residual_stride % 4 == 0), "linear_reduce: bad residual");
  if (M == 0) return YH_OK;
  YH_CHECK_ARG(part && out, "linear_reduce: null pointer");
  // partials are read 16 bytes at a time, the output and residual 8
  YH_CHECK_ARG((reinterpret_cast<uintptr_t>(part) & 15) == 0 && (reinterpret_cast<uintptr_t>(out) & 7) == 0 &&
                   (reinterpret_cast<uintptr_t>(residual) & 7) == 0,
               "linear_reduce: part must be 16-byte aligned, out and residual 8-byte aligned");
  const int64_t quads = M * N / 4;
  hipLaunchKernelGGL(linear_reduce_kernel, dim3(static_cast<unsigned>((quads + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), part, static_cast<uint16_t*>(out), out_stride, (int)M, (int)N,
                     (int)S, static_cast<const uint16_t*>(residual), residual_stride);
  YH_CHECK_LAUNCH("linear_reduce");
  return YH_OK;
}
