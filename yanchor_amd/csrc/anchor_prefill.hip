// Anchor-memory prefill read: every query of a C-token block attends over the
// source tokens its block references (the block's prefix Top-K), with the
// zero-logit sink.  Replaces _indexed_forward / indexed_gqa
// (runtime/model/independent_memory.py:6-45) and indexed_gqa_torch / _gqa_tile
// (modeling_yanchor.py:22-42), called from IndependentGQAMemory._sequence
// (modeling_yanchor.py:249).
//
//   query       [B, NB, C, H, D]   bf16 / fp16
//   key, value  [KB, S, G, D]      KB == B, or 1 (one source shared by all rows)
//   references  [B, NB, G, CAP]    int32 / int64 index into S, -1 = none
//   out         [B, NB, C, H, D]
//
// Query head h belongs to group h / (H / G).  Per (b, block, g) the C * H/G
// query rows share one gathered set of CAP key/value rows, so the read is a
// small dense attention: S^T = K Q^T and O^T = V^T P^T on 16x16x32 MFMA, with
// an online softmax whose running max starts at 0 and denominator at 1 (the
// sink logit 0 with value 0).  As in the reference, P enters the PV product as
// a hi + lo pair of 16-bit values, so the product keeps fp32 accuracy.
//
// Workgroup = 4 waves x 16 query rows; grid (B * NB * G, ceil(C * H/G / 64)).
// Reference rows are gathered 64 at a time into LDS: K row-major (A operand
// of S^T), V transposed (A operand of O^T).  The MFMA K-index order of the PV
// product is permuted to match the lanes that hold each score, so P never
// leaves registers.
#include "common.h"

namespace yh {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4v __attribute__((ext_vector_type(4)));

constexpr int kD = 128;
constexpr int kTile = 64;        // reference rows per LDS tile
constexpr int kKPad = kD + 8;    // K row stride (elements): 272 B, conflict-free 16 B reads
constexpr int kVPad = kTile + 4; // V^T row stride (elements): 136 B, conflict-free 8 B reads

struct IdxArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const void* refs;
  uint16_t* out;
  int NB, C, H, G, S, CAP, KB, ref64;
  float scale;
  // tokens in place (yh_anchor_sequence_read): query / out [B, L, H, D]; the
  // query at block position p = nb * C + t of row b is token p - first[b]
  // (no token, no read, for p outside [first[b], first[b] + L))
  const int64_t* first;
  int L;
};

template <int DT>
struct Mfma;
template <>
struct Mfma<YH_BF16> {
  typedef bf16x8_t vec;
  static __device__ __forceinline__ f32x4v run(vec a, vec b, f32x4v c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint16_t round(float x) { return f32_to_bf16(x); }
  static __device__ __forceinline__ float widen(uint16_t h) { return bf16_to_f32(h); }
};
template <>
struct Mfma<YH_F16> {
  typedef f16x8_t vec;
  static __device__ __forceinline__ f32x4v run(vec a, vec b, f32x4v c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint16_t round(float x) { return f32_to_f16(x); }
  static __device__ __forceinline__ float widen(uint16_t h) { return f16_to_f32(h); }
};

__device__ __forceinline__ uint32_t pack2(uint16_t lo, uint16_t hi) {
  return static_cast<uint32_t>(lo) | (static_cast<uint32_t>(hi) << 16);
}

template <int DT>
__global__ void __launch_bounds__(256) indexed_gqa_kernel(IdxArgs a) {
  using M = Mfma<DT>;
  using vec = typename M::vec;
  __shared__ __align__(16) uint16_t ks[kTile][kKPad];
  __shared__ __align__(16) uint16_t vt[kD][kVPad];
  __shared__ int rs[kTile];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int R = a.H / a.G;
  const int rows = a.C * R;
  const int bg = blockIdx.x;
  const int g = bg % a.G;
  const int64_t bb = bg / a.G;          // b * NB + block
  const int64_t b = bb / a.NB;
  const int qn = lane & 15, quad = lane >> 4;
  const int m = blockIdx.y * 64 + w * 16 + qn;  // query row of this lane (as the MFMA column)
  bool mvalid = m < rows;
  int64_t qrow;
  if (a.first == nullptr) {
    qrow = mvalid ? ((bb * a.C + m % a.C) * a.H + g * R + m / a.C) : 0;
  } else {
    const int64_t tok = (bb - b * a.NB) * a.C + m % a.C - a.first[b];
    mvalid = mvalid && tok >= 0 && tok < a.L;
    qrow = mvalid ? ((b * a.L + tok) * a.H + g * R + m / a.C) : 0;
  }

  // Q^T operand (B of S^T = K Q^T): lane holds Q[m][step*32 + quad*8 + 0..7].
  vec qv[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    uint4 x = make_uint4(0, 0, 0, 0);
    if (mvalid) x = *reinterpret_cast<const uint4*>(a.q + qrow * kD + s * 32 + quad * 8);
    qv[s] = __builtin_bit_cast(vec, x);
  }

  f32x4v acc[kD / 16];
#pragma unroll
  for (int t = 0; t < kD / 16; ++t) acc[t] = f32x4v{0.f, 0.f, 0.f, 0.f};
  float mx = 0.f, den = 1.f;  // the sink: logit 0, value 0

  const int64_t kb = a.KB == 1 ? 0 : b;
  const int64_t ref_base = static_cast<int64_t>(bg) * a.CAP;
  for (int start = 0; start < a.CAP; start += kTile) {
    __syncthreads();  // previous tile fully consumed
    if (tid < kTile) {
      const int n = start + tid;
      int64_t r = -1;
      if (n < a.CAP) {
        r = a.ref64 ? static_cast<const int64_t*>(a.refs)[ref_base + n]
                    : static_cast<const int32_t*>(a.refs)[ref_base + n];
      }
      rs[tid] = (r >= 0 && r < a.S) ? static_cast<int>(r) : -1;
    }
    __syncthreads();
    const bool any = __syncthreads_or(tid < kTile && rs[tid] >= 0);
    if (!any) continue;
    // gather: 64 rows x 16 vectors of 8 elements, 4 vectors per thread
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int idx = it * 256 + tid;
      const int row = idx >> 4, c8 = (idx & 15) * 8;
      const int r = rs[row];
      uint4 kx = make_uint4(0, 0, 0, 0), vx = make_uint4(0, 0, 0, 0);
      if (r >= 0) {
        const int64_t off = ((kb * a.S + r) * a.G + g) * kD + c8;
        kx = *reinterpret_cast<const uint4*>(a.k + off);
        vx = *reinterpret_cast<const uint4*>(a.v + off);
      }
      *reinterpret_cast<uint4*>(&ks[row][c8]) = kx;
      const uint16_t* vh = reinterpret_cast<const uint16_t*>(&vx);
#pragma unroll
      for (int j = 0; j < 8; ++j) vt[c8 + j][row] = vh[j];
    }
    __syncthreads();

    // S^T tiles: rt covers refs rt*16 .. +15; lane holds refs rt*16 + quad*4 + i
    // for query column qn.
    float sc[4][4];
    float tmax = -INFINITY;
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      f32x4v c = f32x4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const vec kvv = __builtin_bit_cast(vec, *reinterpret_cast<const uint4*>(&ks[rt * 16 + qn][s * 32 + quad * 8]));
        c = M::run(kvv, qv[s], c);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const bool live = rs[rt * 16 + quad * 4 + i] >= 0;
        sc[rt][i] = live ? c[i] * a.scale : -INFINITY;
        tmax = fmaxf(tmax, sc[rt][i]);
      }
    }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float nmx = fmaxf(mx, tmax);
    const float alpha = __expf(mx - nmx);
    float psum = 0.f;
    uint16_t ph[4][4], pl[4][4];
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float p = __expf(sc[rt][i] - nmx);  // 0 for masked refs
        psum += p;
        ph[rt][i] = M::round(p);
        pl[rt][i] = M::round(p - M::widen(ph[rt][i]));
      }
    }
    psum += __shfl_xor(psum, 16, 64);
    psum += __shfl_xor(psum, 32, 64);
    den = den * alpha + psum;
    mx = nmx;
#pragma unroll
    for (int t = 0; t < kD / 16; ++t) acc[t] *= alpha;

    // O^T += V^T P^T over two 32-deep steps; K-index j of lane (quad) maps to
    // ref 32s + quad*4 + j (j < 4) and 32s + 16 + quad*4 + j-4 (j >= 4).
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const vec phv = __builtin_bit_cast(
          vec, make_uint4(pack2(ph[2 * s][0], ph[2 * s][1]), pack2(ph[2 * s][2], ph[2 * s][3]),
                          pack2(ph[2 * s + 1][0], ph[2 * s + 1][1]), pack2(ph[2 * s + 1][2], ph[2 * s + 1][3])));
      const vec plv = __builtin_bit_cast(
          vec, make_uint4(pack2(pl[2 * s][0], pl[2 * s][1]), pack2(pl[2 * s][2], pl[2 * s][3]),
                          pack2(pl[2 * s + 1][0], pl[2 * s + 1][1]), pack2(pl[2 * s + 1][2], pl[2 * s + 1][3])));
#pragma unroll
      for (int t = 0; t < kD / 16; ++t) {
        const uint16_t* row = &vt[t * 16 + qn][0];
        const uint2 lo = *reinterpret_cast<const uint2*>(row + 32 * s + quad * 4);
        const uint2 hi = *reinterpret_cast<const uint2*>(row + 32 * s + 16 + quad * 4);
        const vec vv = __builtin_bit_cast(vec, make_uint4(lo.x, lo.y, hi.x, hi.y));
        acc[t] = M::run(vv, phv, acc[t]);
        acc[t] = M::run(vv, plv, acc[t]);
      }
    }
  }

  if (!mvalid) return;
  const float inv = 1.f / den;
  uint16_t* orow = a.out + qrow * kD;
#pragma unroll
  for (int t = 0; t < kD / 16; ++t) {
    const int d0 = t * 16 + quad * 4;
    const uint2 o = make_uint2(pack2(M::round(acc[t][0] * inv), M::round(acc[t][1] * inv)),
                               pack2(M::round(acc[t][2] * inv), M::round(acc[t][3] * inv)));
    *reinterpret_cast<uint2*>(orow + d0) = o;
  }
}

}  // namespace
}  // namespace yh

namespace yh {
namespace {
int launch_indexed(const void* query, const void* key, const void* value, const void* references, int ref_dtype,
                   void* out, int64_t B, int64_t NB, int64_t C, int64_t H, int64_t G, int64_t D, int64_t KB,
                   int64_t S, int64_t CAP, const int64_t* first, int64_t L, int dtype, yh_stream_t stream,
                   const char* what) {
  YH_CHECK_ARG(B >= 0 && NB >= 0 && C > 0 && H > 0 && G > 0 && H % G == 0 && S >= 0 && CAP >= 0 && L >= 0,
               "%s: bad sizes", what);
  YH_CHECK_ARG(D == kD, "%s: head dim must be %d", what, kD);
  YH_CHECK_ARG(KB == 1 || KB == B, "%s: key batch must be 1 or B", what);
  YH_CHECK_ARG(ref_dtype == YH_I32 || ref_dtype == YH_I64, "%s: references must be int32 or int64", what);
  if (dtype != YH_BF16 && dtype != YH_F16) {
    set_error("%s: dtype must be bf16 or fp16", what);
    return YH_ERR_UNSUPPORTED;
  }
  const int64_t groups = B * NB * G;
  if (groups == 0) return YH_OK;
  YH_CHECK_ARG(query && key && value && out && (CAP == 0 || references), "%s: null pointer", what);
  YH_CHECK_ARG(((reinterpret_cast<uintptr_t>(query) | reinterpret_cast<uintptr_t>(key) |
                 reinterpret_cast<uintptr_t>(value) | reinterpret_cast<uintptr_t>(out)) & 15) == 0,
               "%s: tensors must be 16-byte aligned", what);
  YH_CHECK_ARG(groups < (1ll << 31) && C * (H / G) < (1ll << 20) && L < (1ll << 31), "%s: grid too large", what);
  IdxArgs a{static_cast<const uint16_t*>(query), static_cast<const uint16_t*>(key),
            static_cast<const uint16_t*>(value), references, static_cast<uint16_t*>(out), (int)NB, (int)C, (int)H,
            (int)G, (int)S, (int)CAP, (int)KB, ref_dtype == YH_I64 ? 1 : 0, 1.f / sqrtf(static_cast<float>(D)),
            first, (int)L};
  const dim3 grid(static_cast<unsigned>(groups), static_cast<unsigned>((C * (H / G) + 63) / 64));
  if (dtype == YH_BF16)
    hipLaunchKernelGGL(indexed_gqa_kernel<YH_BF16>, grid, dim3(256), 0, static_cast<hipStream_t>(stream), a);
  else
    hipLaunchKernelGGL(indexed_gqa_kernel<YH_F16>, grid, dim3(256), 0, static_cast<hipStream_t>(stream), a);
  YH_CHECK_LAUNCH(what);
  return YH_OK;
}
}  // namespace
}  // namespace yh

extern "C" int yh_indexed_gqa(const void* query, const void* key, const void* value, const void* references,
                              int ref_dtype, void* out, int64_t B, int64_t NB, int64_t C, int64_t H, int64_t G,
                              int64_t D, int64_t KB, int64_t S, int64_t CAP, int dtype, yh_stream_t stream) {
  return yh::launch_indexed(query, key, value, references, ref_dtype, out, B, NB, C, H, G, D, KB, S, CAP, nullptr, 0,
                            dtype, stream, "indexed_gqa");
}

extern "C" int yh_anchor_sequence_read(const void* query, const void* key, const void* value,
                                       const void* references, int ref_dtype, const int64_t* first, void* out,
                                       int64_t B, int64_t L, int64_t NB, int64_t C, int64_t H, int64_t G, int64_t D,
                                       int64_t S, int64_t CAP, int dtype, yh_stream_t stream) {
  using namespace yh;
  YH_CHECK_ARG(first != nullptr || B == 0, "anchor_sequence_read: null pointer");
  return launch_indexed(query, key, value, references, ref_dtype, out, B, NB, C, H, G, D, B, S, CAP, first, L, dtype,
                        stream, "anchor_sequence_read");
}
