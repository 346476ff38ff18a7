// Refill prefill of a packed, ragged set of prompt pieces (cu_seqlens), each
// piece continuing its sequence's caches:
//
//   conv_prefill_kernel   the GDN layer's causal conv1d + SiLU over every token
//                         of every piece, the first K-1 taps of a piece taken
//                         from the sequence's conv window (the causal-conv1d
//                         prefill call of the CUDA backend, modeling_yanchor.py:
//                         392-407; torch form wheel transformers/models/qwen3_5/
//                         modeling_qwen3_5.py:455-470).  One rounding: fp32
//                         taps in the decode prologue's order, SiLU, bf16.
//   conv_window_kernel    the conv window left behind: the last K-1 inputs of
//                         [window | piece].
//   swa_prefill_kernel    sliding-window causal attention of every query over
//                         the W keys ending at its own position (flash_swa /
//                         reference_swa, modeling_yanchor.py:412-449), the keys
//                         before the piece read from the sequence's physical
//                         ring (slot = position mod W), GQA, and the output
//                         gate read * sigmoid(gate) of Qwen3_5FixedWindowAttention
//                         (modeling_yanchor.py:871-875) in the store.
//   ring_fill_kernel      the last min(W, L) keys / values / positions of each
//                         piece into its ring slots (the chronological ring of
//                         runtime/model/inference_kernels.py:1799-1856, built
//                         in place).
//
// swa_prefill_kernel: workgroup = 4 waves x 16 query rows = 64 rows of one
// (piece, KV group): 64 / R consecutive tokens x the R query heads of the
// group, so all four waves share the key tiles.  Keys of the tile range are
// staged 64 at a time in LDS (K row-major, V transposed); S^T = K Q^T and
// O^T = V^T P^T on 16x16x32 MFMA with an online softmax; the PV product's
// K-index order is permuted to the lanes that hold each score, so P stays in
// registers (the layout of the anchor-memory block read).
#include "common.h"

namespace yh {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float silu(float x) { return x / (1.f + expf(-x)); }

// Sequence of packed token n: the last r with cu[r] <= n (cu ascending,
// empty pieces allowed).
__device__ __forceinline__ int seq_of(const int32_t* cu, int nseq, int64_t n) {
  int lo = 0, hi = nseq - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (cu[mid] <= n) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

// ---------------------------------------------------------------------------
// conv: x = proj[:, :C] of the packed tokens; window [R, 3, C] time-major
// (oldest first); w [C, 4].  y[n, c] = bf16(silu(sum_j x(t - 3 + j) w[c, j]))
// with x(u < 0) = window[r, 3 + u].
struct ConvArgs {
  const uint16_t* proj;
  int64_t P;
  const uint16_t* window;
  const uint16_t* w;
  const int32_t* cu;
  uint16_t* y;
  int64_t C;
  int nseq;
};

__global__ void __launch_bounds__(256) conv_prefill_kernel(ConvArgs a) {
  const int64_t n = blockIdx.x;
  const int64_t c = static_cast<int64_t>(blockIdx.y) * 256 + threadIdx.x;
  if (c >= a.C) return;
  const int r = seq_of(a.cu, a.nseq, n);
  const int64_t t = n - a.cu[r];
  if (t < 0 || n >= a.cu[r + 1]) return;   // a token outside every piece
  float x[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t u = t - 3 + j;
    const uint16_t h = u >= 0 ? a.proj[(n - 3 + j) * a.P + c] : a.window[(static_cast<int64_t>(r) * 3 + 3 + u) * a.C + c];
    x[j] = bf16_to_f32(h);
  }
  const uint16_t* wc = a.w + c * 4;
  float acc = x[0] * bf16_to_f32(wc[0]);
  acc = fmaf(x[1], bf16_to_f32(wc[1]), acc);
  acc = fmaf(x[2], bf16_to_f32(wc[2]), acc);
  acc = fmaf(x[3], bf16_to_f32(wc[3]), acc);
  a.y[n * a.C + c] = f32_to_bf16(silu(acc));
}

// window[r, m] <- input at relative time L - 3 + m (m = 0, 1, 2): from the
// piece, or, for pieces shorter than 3 tokens, the old window shifted.  One
// thread owns a (row, channel) and goes in ascending m, so every old entry is
// read before it is overwritten.
__global__ void __launch_bounds__(256) conv_window_kernel(ConvArgs a) {
  const int r = blockIdx.x;
  const int64_t c = static_cast<int64_t>(blockIdx.y) * 256 + threadIdx.x;
  if (c >= a.C) return;
  const int64_t s0 = a.cu[r], len = a.cu[r + 1] - s0;
  uint16_t* win = const_cast<uint16_t*>(a.window) + static_cast<int64_t>(r) * 3 * a.C;
#pragma unroll
  for (int m = 0; m < 3; ++m) {
    const int64_t u = len - 3 + m;
    win[m * a.C + c] = u >= 0 ? a.proj[(s0 + u) * a.P + c] : win[(3 + u) * a.C + c];
  }
}

// ---------------------------------------------------------------------------
constexpr int kD = 128;
constexpr int kTile = 64;
constexpr int kKPad = kD + 8;     // 272 B rows: conflict-free 16 B reads
constexpr int kVPad = kTile + 4;  // 136 B rows: conflict-free 8 B reads

struct SwaArgs {
  const uint16_t* q;      // [N, H, D]
  int64_t q_ts;
  const uint16_t* k;      // [N, G, D] normed, rotated piece keys
  int64_t k_ts;
  const uint16_t* v;      // [N, G, D] piece values
  int64_t v_ts;
  const uint16_t* ring_k; // [RB, G, W, D]
  const uint16_t* ring_v;
  const int64_t* ring_row;  // [R], -1 = no ring context
  const int64_t* start;     // [R] position of each piece's first token
  const int32_t* cu;        // [R + 1]
  const int32_t* tiles;     // [n_tiles, 2] (piece, first token)
  const uint16_t* gate;   // [N, H, D] (token / head strides) or null
  int64_t g_ts, g_hs;
  uint16_t* out;          // [N, H, D]
  int H, G, W;
  float scale;
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
__global__ void __launch_bounds__(256) swa_prefill_kernel(SwaArgs a) {
  using M = Mfma<DT>;
  using vec = typename M::vec;
  __shared__ __align__(16) uint16_t ks[kTile][kKPad];
  __shared__ __align__(16) uint16_t vt[kD][kVPad];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = blockIdx.y;
  const int r = a.tiles[2 * blockIdx.x], t0 = a.tiles[2 * blockIdx.x + 1];
  const int R = a.H / a.G, TT = kTile / R;
  const int64_t s0 = a.cu[r];
  const int len = a.cu[r + 1] - a.cu[r];
  const int64_t start = a.start[r];
  const int64_t rrow = a.ring_row[r];
  const int nctx = rrow < 0 ? 0 : static_cast<int>(start < a.W - 1 ? start : a.W - 1);
  const int qn = lane & 15, quad = lane >> 4;
  const int m = w * 16 + qn;                    // query row of this lane (the MFMA column)
  const int tok = t0 + m % TT;
  const int head = g * R + m / TT;
  const bool mvalid = tok < len;
  const int64_t qrow = s0 + (mvalid ? tok : 0);
  const int self = nctx + tok;                  // this query's own key index in [ring context | piece]

  vec qv[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    uint4 x = make_uint4(0, 0, 0, 0);
    if (mvalid) x = *reinterpret_cast<const uint4*>(a.q + qrow * a.q_ts + head * kD + s * 32 + quad * 8);
    qv[s] = __builtin_bit_cast(vec, x);
  }

  f32x4v acc[kD / 16];
#pragma unroll
  for (int t = 0; t < kD / 16; ++t) acc[t] = f32x4v{0.f, 0.f, 0.f, 0.f};
  float mx = -INFINITY, den = 0.f;

  const int last_tok = (t0 + TT < len ? t0 + TT : len) - 1;
  const int j_hi = nctx + last_tok;                        // inclusive
  const int j_lo = nctx + t0 - a.W + 1 > 0 ? nctx + t0 - a.W + 1 : 0;
  const int64_t ring_base = rrow < 0 ? 0 : (rrow * a.G + g) * a.W;
  const int64_t pos0 = start - nctx;                       // position of key index 0

  for (int j0 = j_lo; j0 <= j_hi; j0 += kTile) {
    __syncthreads();  // the previous tile is consumed
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int idx = it * 256 + tid;
      const int row = idx >> 4, c8 = (idx & 15) * 8;
      const int j = j0 + row;
      uint4 kx = make_uint4(0, 0, 0, 0), vx = make_uint4(0, 0, 0, 0);
      if (j <= j_hi) {
        if (j < nctx) {
          const int64_t off = (ring_base + (pos0 + j) % a.W) * kD + c8;
          kx = *reinterpret_cast<const uint4*>(a.ring_k + off);
          vx = *reinterpret_cast<const uint4*>(a.ring_v + off);
        } else {
          const int64_t tk = s0 + j - nctx;
          kx = *reinterpret_cast<const uint4*>(a.k + tk * a.k_ts + g * kD + c8);
          vx = *reinterpret_cast<const uint4*>(a.v + tk * a.v_ts + g * kD + c8);
        }
      }
      *reinterpret_cast<uint4*>(&ks[row][c8]) = kx;
      const uint16_t* vh = reinterpret_cast<const uint16_t*>(&vx);
#pragma unroll
      for (int e = 0; e < 8; ++e) vt[c8 + e][row] = vh[e];
    }
    __syncthreads();

    // S^T tiles: rt covers keys j0 + rt*16 .. +15; lane holds keys
    // j0 + rt*16 + quad*4 + i for query column qn
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
        const int j = j0 + rt * 16 + quad * 4 + i;
        const bool live = mvalid && j <= self && j > self - a.W;
        sc[rt][i] = live ? c[i] * a.scale : -INFINITY;
        tmax = fmaxf(tmax, sc[rt][i]);
      }
    }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float nmx = fmaxf(mx, tmax);
    const float base = nmx == -INFINITY ? 0.f : nmx;   // a row with no live key so far stays at 0
    const float alpha = __expf(mx - base);
    float psum = 0.f;
    uint16_t ph[4][4];
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float p = __expf(sc[rt][i] - base);  // 0 for masked keys
        psum += p;
        ph[rt][i] = M::round(p);
      }
    }
    psum += __shfl_xor(psum, 16, 64);
    psum += __shfl_xor(psum, 32, 64);
    den = den * alpha + psum;
    mx = nmx;
#pragma unroll
    for (int t = 0; t < kD / 16; ++t) acc[t] *= alpha;

    // O^T += V^T P^T over two 32-deep steps; K-index e of lane (quad) maps to
    // key 32s + quad*4 + e (e < 4) and 32s + 16 + quad*4 + e-4 (e >= 4)
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const vec phv = __builtin_bit_cast(
          vec, make_uint4(pack2(ph[2 * s][0], ph[2 * s][1]), pack2(ph[2 * s][2], ph[2 * s][3]),
                          pack2(ph[2 * s + 1][0], ph[2 * s + 1][1]), pack2(ph[2 * s + 1][2], ph[2 * s + 1][3])));
#pragma unroll
      for (int t = 0; t < kD / 16; ++t) {
        const uint16_t* vrow = &vt[t * 16 + qn][0];
        const uint2 lo = *reinterpret_cast<const uint2*>(vrow + 32 * s + quad * 4);
        const uint2 hi = *reinterpret_cast<const uint2*>(vrow + 32 * s + 16 + quad * 4);
        const vec vv = __builtin_bit_cast(vec, make_uint4(lo.x, lo.y, hi.x, hi.y));
        acc[t] = M::run(vv, phv, acc[t]);
      }
    }
  }

  if (!mvalid) return;
  const float inv = 1.f / den;   // den > 0: every query sees its own key
  uint16_t* orow = a.out + (qrow * a.H + head) * kD;
  const uint16_t* grow = a.gate ? a.gate + qrow * a.g_ts + head * a.g_hs : nullptr;
#pragma unroll
  for (int t = 0; t < kD / 16; ++t) {
    const int d0 = t * 16 + quad * 4;
    uint16_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o[i] = M::round(acc[t][i] * inv);
      if (grow) {   // read * sigmoid(gate), each product rounded as the torch ops round it
        const uint16_t sg = M::round(1.f / (1.f + __expf(-M::widen(grow[d0 + i]))));
        o[i] = M::round(M::widen(o[i]) * M::widen(sg));
      }
    }
    *reinterpret_cast<uint2*>(orow + d0) = make_uint2(pack2(o[0], o[1]), pack2(o[2], o[3]));
  }
}

// ---------------------------------------------------------------------------
// ring_fill: block per packed token; the last min(W, L) tokens of each piece
// write their key / value rows (all G heads, 16 B per thread) and position.
struct FillArgs {
  const uint16_t* k;
  int64_t k_ts;
  const uint16_t* v;
  int64_t v_ts;
  const int64_t* ring_row;
  const int64_t* start;
  const int32_t* cu;
  uint16_t* ring_k;
  uint16_t* ring_v;
  int32_t* ring_pos;
  int G, W, nseq;
};

__global__ void __launch_bounds__(256) ring_fill_kernel(FillArgs a) {
  const int64_t n = blockIdx.x;
  const int r = seq_of(a.cu, a.nseq, n);
  const int64_t t = n - a.cu[r], len = a.cu[r + 1] - a.cu[r];
  const int64_t rrow = a.ring_row[r];
  if (t < 0 || t >= len) return;           // a token outside every piece
  if (rrow < 0 || t < len - a.W) return;   // overwritten by a later token of the piece
  const int64_t pos = a.start[r] + t;
  const int64_t slot = pos % a.W;
  for (int e = threadIdx.x; e < a.G * (kD / 8); e += blockDim.x) {
    const int g = e / (kD / 8), c8 = (e % (kD / 8)) * 8;
    const int64_t dst = ((rrow * a.G + g) * a.W + slot) * kD + c8;
    *reinterpret_cast<uint4*>(a.ring_k + dst) = *reinterpret_cast<const uint4*>(a.k + n * a.k_ts + g * kD + c8);
    *reinterpret_cast<uint4*>(a.ring_v + dst) = *reinterpret_cast<const uint4*>(a.v + n * a.v_ts + g * kD + c8);
    if (c8 == 0) a.ring_pos[(rrow * a.G + g) * a.W + slot] = static_cast<int32_t>(pos);
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace
}  // namespace yh

extern "C" int yh_conv_prefill(const void* proj, int64_t proj_stride, void* window, const void* conv_w,
                               const int32_t* cu_seqlens, int64_t n_seqs, int64_t total_tokens, int64_t channels,
                               void* out, int dtype, yh_stream_t stream) {
  using namespace yh;
  YH_CHECK_ARG(n_seqs >= 0 && total_tokens >= 0 && channels > 0 && proj_stride >= channels,
               "conv_prefill: bad sizes");
  YH_CHECK_ARG(dtype == YH_BF16, "conv_prefill: activations must be bfloat16");
  if (n_seqs == 0) return YH_OK;
  YH_CHECK_ARG(proj && window && conv_w && cu_seqlens && (out || total_tokens == 0), "conv_prefill: null pointer");
  YH_CHECK_ARG(total_tokens < (1ll << 31) && n_seqs < (1ll << 31), "conv_prefill: sizes too large");
  hipStream_t st = static_cast<hipStream_t>(stream);
  ConvArgs c{static_cast<const uint16_t*>(proj), proj_stride, static_cast<const uint16_t*>(window),
             static_cast<const uint16_t*>(conv_w), cu_seqlens, static_cast<uint16_t*>(out), channels, (int)n_seqs};
  const unsigned cb = static_cast<unsigned>((channels + 255) / 256);
  if (total_tokens > 0) {
    hipLaunchKernelGGL(conv_prefill_kernel, dim3(static_cast<unsigned>(total_tokens), cb), dim3(256), 0, st, c);
    YH_CHECK_LAUNCH("conv_prefill");
  }
  hipLaunchKernelGGL(conv_window_kernel, dim3(static_cast<unsigned>(n_seqs), cb), dim3(256), 0, st, c);
  YH_CHECK_LAUNCH("conv_prefill window");
  return YH_OK;
}

extern "C" int yh_swa_prefill(const void* q, int64_t q_stride, const void* k, int64_t k_stride, const void* v,
                              int64_t v_stride, const void* ring_k, const void* ring_v, const int64_t* ring_rows,
                              const int64_t* starts, const int32_t* cu_seqlens, const int32_t* tiles,
                              int64_t n_tiles, const void* gate, int64_t gate_token_stride,
                              int64_t gate_head_stride, void* out, int64_t n_seqs, int64_t ring_batch, int64_t H,
                              int64_t G, int64_t D, int64_t window, int dtype, yh_stream_t stream) {
  using namespace yh;
  YH_CHECK_ARG(n_seqs >= 0 && n_tiles >= 0 && H > 0 && G > 0 && H % G == 0 && window > 0 && ring_batch >= 0,
               "swa_prefill: bad sizes");
  YH_CHECK_ARG(D == kD, "swa_prefill: head dim must be %d", kD);
  YH_CHECK_ARG(kTile % (H / G) == 0, "swa_prefill: query heads per KV head must divide %d", kTile);
  if (dtype != YH_BF16 && dtype != YH_F16) {
    set_error("swa_prefill: dtype must be bf16 or fp16");
    return YH_ERR_UNSUPPORTED;
  }
  if (n_tiles == 0) return YH_OK;
  YH_CHECK_ARG(q && k && v && out && starts && ring_rows && cu_seqlens && tiles, "swa_prefill: null pointer");
  YH_CHECK_ARG(ring_batch == 0 || (ring_k && ring_v), "swa_prefill: null ring");
  YH_CHECK_ARG(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(out) && (!ring_k || aligned16(ring_k)) &&
                   (!ring_v || aligned16(ring_v)),
               "swa_prefill: tensors must be 16-byte aligned");
  YH_CHECK_ARG(q_stride % 8 == 0 && k_stride % 8 == 0 && v_stride % 8 == 0 && q_stride >= H * D && k_stride >= G * D &&
                   v_stride >= G * D,
               "swa_prefill: token strides must hold whole heads and keep 16-byte rows");
  YH_CHECK_ARG(!gate || (gate_head_stride >= D && gate_token_stride >= H * gate_head_stride),
               "swa_prefill: bad gate strides");
  YH_CHECK_ARG(n_tiles < (1ll << 31) && G < 65536 && window < (1ll << 30), "swa_prefill: grid too large");
  SwaArgs a{static_cast<const uint16_t*>(q), q_stride, static_cast<const uint16_t*>(k), k_stride,
            static_cast<const uint16_t*>(v), v_stride, static_cast<const uint16_t*>(ring_k),
            static_cast<const uint16_t*>(ring_v), ring_rows, starts, cu_seqlens, tiles,
            static_cast<const uint16_t*>(gate), gate_token_stride, gate_head_stride, static_cast<uint16_t*>(out),
            (int)H, (int)G, (int)window, 1.f / sqrtf(static_cast<float>(D))};
  const dim3 grid(static_cast<unsigned>(n_tiles), static_cast<unsigned>(G));
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == YH_BF16)
    hipLaunchKernelGGL(swa_prefill_kernel<YH_BF16>, grid, dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL(swa_prefill_kernel<YH_F16>, grid, dim3(256), 0, st, a);
  YH_CHECK_LAUNCH("swa_prefill");
  return YH_OK;
}

extern "C" int yh_ring_fill(const void* k, int64_t k_stride, const void* v, int64_t v_stride,
                            const int64_t* ring_rows, const int64_t* starts, const int32_t* cu_seqlens,
                            int64_t n_seqs, int64_t total_tokens, void* ring_k, void* ring_v, int32_t* ring_pos,
                            int64_t G, int64_t D, int64_t window, int dtype, yh_stream_t stream) {
  using namespace yh;
  YH_CHECK_ARG(n_seqs >= 0 && total_tokens >= 0 && G > 0 && window > 0, "ring_fill: bad sizes");
  YH_CHECK_ARG(D == kD, "ring_fill: head dim must be %d", kD);
  YH_CHECK_ARG(dtype == YH_BF16 || dtype == YH_F16, "ring_fill: dtype must be bf16 or fp16");
  if (total_tokens == 0 || n_seqs == 0) return YH_OK;
  YH_CHECK_ARG(k && v && ring_rows && starts && cu_seqlens && ring_k && ring_v && ring_pos, "ring_fill: null pointer");
  YH_CHECK_ARG(aligned16(k) && aligned16(v) && aligned16(ring_k) && aligned16(ring_v) && k_stride % 8 == 0 &&
                   v_stride % 8 == 0 && k_stride >= G * D && v_stride >= G * D,
               "ring_fill: rows must be 16-byte aligned");
  YH_CHECK_ARG(total_tokens < (1ll << 31), "ring_fill: sizes too large");
  FillArgs a{static_cast<const uint16_t*>(k), k_stride, static_cast<const uint16_t*>(v), v_stride, ring_rows, starts,
             cu_seqlens, static_cast<uint16_t*>(ring_k), static_cast<uint16_t*>(ring_v), ring_pos, (int)G,
             (int)window, (int)n_seqs};
  hipLaunchKernelGGL(ring_fill_kernel, dim3(static_cast<unsigned>(total_tokens)), dim3(128), 0,
                     static_cast<hipStream_t>(stream), a);
  YH_CHECK_LAUNCH("ring_fill");
  return YH_OK;
}
