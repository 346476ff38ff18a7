// Fused decode-layer neighbours of the hot path (one launch each instead of a
// chain of elementwise kernels):
//
//   rmsnorm_kernel        Qwen3_5RMSNorm, y = x / rms(x) * (1 + w), with an
//                         optional fused residual add (the
//                         _qwen35_rmsnorm_torch_tree / fused residual RMSNorm
//                         of runtime/model/inference_kernels.py:227-271,
//                         1767-1797)
//   gdn_prep_kernel       causal conv1d decode update + SiLU, q/k/v split, and
//                         the GDN gates beta = sigmoid(b),
//                         g = -exp(A_log) softplus(a + dt_bias)
//                         (inference_kernels.py:339-376, 668-691; transformers
//                         wheel models/qwen3_5/modeling_qwen3_5.py:210-225,
//                         500-502)
//   gated_rmsnorm_kernel  Qwen3_5RMSNormGated (wheel:175-190)
//   silu_mul_kernel       silu(gate) * up (inference_kernels.py:642-666)
//   head_norm_rope_kernel per-head RMSNorm (1 + w) and rotate-half RoPE on the
//                         leading rotary dims (modeling_yanchor.py:46-49 and the
//                         Qwen3.5 attention q/k path)
//
// Every rounding point of the torch formulation is kept (bf16 where torch
// materialises a bf16 tensor), so results match it to bf16 precision.
#include "common.h"

namespace yh {
namespace {

__device__ __forceinline__ float bf(uint16_t h) { return __uint_as_float(static_cast<uint32_t>(h) << 16); }
__device__ __forceinline__ uint16_t tobf(float x) { return f32_to_bf16(x); }
__device__ __forceinline__ float silu(float x) { return x / (1.f + expf(-x)); }

// RMSNorm rows: one workgroup per row, one 8-element vector per thread
// (blockDim = D / 8 rounded up to whole waves, D <= 8192), so a row's loads
// are all issued before the first is consumed.
// s = residual ? bf16(x + residual) : x; residual_out = s;
// out = bf16(s / sqrt(mean(s^2) + eps) * (1 + w)); out2 the same with w2.
// x may instead come as S fp32 split-K partial planes of a projection (part
// [S, rows, D]; x = bf16(sum in slice order), plus an optional residual of the
// projection: x = bf16(x + res1)), so the projection's reduce needs no launch
// of its own.  The projection's residual may itself be the S2 partial planes
// of a second projection (part2, summed in slice order and rounded to bf16,
// as a separate reduce would store it).
constexpr int kNormMaxThreads = 1024;
constexpr int kNormMaxD = 8 * kNormMaxThreads;

struct NormArgs {
  const uint16_t* x;
  int64_t x_stride;
  const float* part;       // [S, rows, D] or null
  int64_t plane;
  int S;
  const uint16_t* res1;    // projection residual (with part) or null
  int64_t res1_stride;
  const uint16_t* res;     // residual stream [rows, D] or null
  uint16_t* res_out;
  const uint16_t* w;
  uint16_t* out;
  int64_t out_stride;
  const uint16_t* w2;      // optional second weight: out2 [rows, D], rows out2_stride apart
  uint16_t* out2;
  int64_t out2_stride;
  int D, plus_one;
  float eps;
  const float* part2;      // [S2, rows, D]: the projection's residual as partials, or null
  int S2;
};

// Block-wide fp32 sum (blockDim a multiple of 64, at most 1024).
__device__ __forceinline__ float block_sum(float x) {
  __shared__ float part[kNormMaxThreads / kWave];
  x = wave_sum(x);
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave, nw = blockDim.x / kWave;
  if (lane == 0) part[w] = x;
  __syncthreads();
  float t = 0.f;
  for (int i = 0; i < nw; ++i) t += part[i];
  return t;
}

__device__ __forceinline__ void set_f4(float* acc, float4 lo, float4 hi) {
  acc[0] = lo.x; acc[1] = lo.y; acc[2] = lo.z; acc[3] = lo.w;
  acc[4] = hi.x; acc[5] = hi.y; acc[6] = hi.z; acc[7] = hi.w;
}

__device__ __forceinline__ void add_f4(float* acc, float4 lo, float4 hi) {
  acc[0] += lo.x; acc[1] += lo.y; acc[2] += lo.z; acc[3] += lo.w;
  acc[4] += hi.x; acc[5] += hi.y; acc[6] += hi.z; acc[7] += hi.w;
}

// SG = partial planes loaded per round (0: x is a bf16 row); 16 planes in
// flight need the registers of at most 512 threads (D <= 4096).
template <int SG>
__global__ void __launch_bounds__(SG > 8 ? 512 : kNormMaxThreads) rmsnorm_kernel(NormArgs a) {
  const int64_t row = blockIdx.x;
  const int c = threadIdx.x, D = a.D;
  const bool on = c < D / 8;
  float v[8];
  float ss = 0.f;
  if (on) {
    uint4 xa, ra = {}, r1a = {};
    if (a.res) ra = *reinterpret_cast<const uint4*>(a.res + row * D + c * 8);
    if constexpr (SG > 0) {
      if (a.res1) r1a = *reinterpret_cast<const uint4*>(a.res1 + row * a.res1_stride + c * 8);
      const float* pp = a.part + row * D + c * 8;
      const float* pp2 = a.part2 ? a.part2 + row * D + c * 8 : pp;
      // planes 0 .. S-1 of part, then S .. S+S2-1 of part2: SG in flight,
      // each set added in its slice order
      const int T = a.S + (a.part2 ? a.S2 : 0);
      float acc[8], acc2[8];
      for (int s0 = 0; s0 < T; s0 += SG) {
        float4 lo[SG], hi[SG];
#pragma unroll
        for (int q = 0; q < SG; ++q) {
          const int vp = s0 + q;
          if (vp < T) {
            const float* src = vp < a.S ? pp + vp * a.plane : pp2 + (vp - a.S) * a.plane;
            lo[q] = *reinterpret_cast<const float4*>(src);
            hi[q] = *reinterpret_cast<const float4*>(src + 4);
          }
        }
#pragma unroll
        for (int q = 0; q < SG; ++q) {
          const int vp = s0 + q;
          if (vp >= T) break;
          if (vp == 0) set_f4(acc, lo[q], hi[q]);
          else if (vp < a.S) add_f4(acc, lo[q], hi[q]);
          else if (vp == a.S) set_f4(acc2, lo[q], hi[q]);
          else add_f4(acc2, lo[q], hi[q]);
        }
      }
      uint16_t xh[8];
      uint16_t* r1h = reinterpret_cast<uint16_t*>(&r1a);
      if (a.part2) {
#pragma unroll
        for (int j = 0; j < 8; ++j) r1h[j] = tobf(acc2[j]);
      }
      const bool add1 = a.res1 || a.part2;
#pragma unroll
      for (int j = 0; j < 8; ++j) xh[j] = add1 ? tobf(bf(tobf(acc[j])) + bf(r1h[j])) : tobf(acc[j]);
      xa = *reinterpret_cast<const uint4*>(xh);
    } else {
      xa = *reinterpret_cast<const uint4*>(a.x + row * a.x_stride + c * 8);
    }
    const uint16_t* xh = reinterpret_cast<const uint16_t*>(&xa);
    if (a.res) {
      const uint16_t* rh = reinterpret_cast<const uint16_t*>(&ra);
      uint16_t sh[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        sh[j] = tobf(bf(xh[j]) + bf(rh[j]));
        v[j] = bf(sh[j]);
      }
      if (a.res_out) *reinterpret_cast<uint4*>(a.res_out + row * D + c * 8) = *reinterpret_cast<const uint4*>(sh);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = bf(xh[j]);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) ss = fmaf(v[j], v[j], ss);
  }
  const float r = rsqrtf(block_sum(ss) / static_cast<float>(D) + a.eps);
  if (!on) return;
  const uint4 wv = *reinterpret_cast<const uint4*>(a.w + c * 8);
  const uint16_t* wh = reinterpret_cast<const uint16_t*>(&wv);
  uint16_t o[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) o[j] = tobf(v[j] * r * (a.plus_one ? 1.f + bf(wh[j]) : bf(wh[j])));
  *reinterpret_cast<uint4*>(a.out + row * a.out_stride + c * 8) = *reinterpret_cast<const uint4*>(o);
  if (a.out2) {
    const uint4 w2v = *reinterpret_cast<const uint4*>(a.w2 + c * 8);
    const uint16_t* w2h = reinterpret_cast<const uint16_t*>(&w2v);
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = tobf(v[j] * r * (a.plus_one ? 1.f + bf(w2h[j]) : bf(w2h[j])));
    *reinterpret_cast<uint4*>(a.out2 + row * a.out2_stride + c * 8) = *reinterpret_cast<const uint4*>(o);
  }
}

void launch_rmsnorm(const NormArgs& a, int64_t N, hipStream_t st) {
  const unsigned threads = static_cast<unsigned>((a.D / 8 + kWave - 1) / kWave * kWave);
  const dim3 grid(static_cast<unsigned>(N));
  const int planes = a.S + (a.part2 ? a.S2 : 0);
  if (!a.part) hipLaunchKernelGGL(rmsnorm_kernel<0>, grid, dim3(threads), 0, st, a);
  else if (planes <= 4) hipLaunchKernelGGL(rmsnorm_kernel<4>, grid, dim3(threads), 0, st, a);
  else if (planes <= 8 || threads > 512) hipLaunchKernelGGL(rmsnorm_kernel<8>, grid, dim3(threads), 0, st, a);
  else hipLaunchKernelGGL(rmsnorm_kernel<16>, grid, dim3(threads), 0, st, a);
}

// Per-step decode inputs, one workgroup per slot b (blockDim = hidden / 8
// rounded up to whole waves): h = embed[tokens[b]] (a zero row for an id
// outside [0, V)), xn = RMSNorm(h) * (1 + w), cos / sin [B, rd] of
// positions[b] * inv_freq[j % (rd / 2)] (the rotate-half layout), the SWA ring
// row b * ring_stride + positions[b] % window, and valid = !finished[b] &&
// slot_rows[b] >= 0 when both are given.
struct InputArgs {
  const int64_t* tokens;
  const int64_t* positions;
  const uint16_t* embed;
  const uint16_t* w;
  const float* inv_freq;
  const uint8_t* finished;
  const int64_t* slot_rows;
  uint16_t* h;
  uint16_t* xn;
  float* cos;
  float* sin;
  int64_t* ring_rows;
  uint8_t* valid;
  int64_t V, ring_stride, window;
  int D, rd;
  float eps;
};

__global__ void __launch_bounds__(kNormMaxThreads) decode_inputs_kernel(InputArgs a) {
  const int64_t b = blockIdx.x;
  const int c = threadIdx.x, D = a.D;
  const int64_t tok = a.tokens[b], pos = a.positions[b];
  const bool on = c < D / 8;
  float v[8];
  float ss = 0.f;
  if (on) {
    uint4 x = {};
    if (tok >= 0 && tok < a.V) x = *reinterpret_cast<const uint4*>(a.embed + tok * D + c * 8);
    *reinterpret_cast<uint4*>(a.h + b * D + c * 8) = x;
    const uint16_t* xh = reinterpret_cast<const uint16_t*>(&x);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      v[j] = bf(xh[j]);
      ss = fmaf(v[j], v[j], ss);
    }
  }
  if (c < a.rd) {
    const float ang = static_cast<float>(pos) * a.inv_freq[c % (a.rd / 2)];
    a.cos[b * a.rd + c] = cosf(ang);
    a.sin[b * a.rd + c] = sinf(ang);
  }
  if (c == 0) {
    a.ring_rows[b] = b * a.ring_stride + pos % a.window;
    if (a.valid) a.valid[b] = (a.finished[b] == 0 && a.slot_rows[b] >= 0) ? 1 : 0;
  }
  const float r = rsqrtf(block_sum(ss) / static_cast<float>(D) + a.eps);
  if (!on) return;
  const uint4 wv = *reinterpret_cast<const uint4*>(a.w + c * 8);
  const uint16_t* wh = reinterpret_cast<const uint16_t*>(&wv);
  uint16_t o[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) o[j] = tobf(v[j] * r * (1.f + bf(wh[j])));
  *reinterpret_cast<uint4*>(a.xn + b * D + c * 8) = *reinterpret_cast<const uint4*>(o);
}

// grid (B, ceil(C / 256)): channel c of row b.  proj [B, P] (row stride P)
// holds [qkv (C) | z | b (HV) | a (HV)] at offsets 0 / -- / boff / aoff.
// conv_state [B, K-1, C] (time-major), conv_w [C, K], K = 4.
struct PrepArgs {
  const uint16_t* proj;
  uint16_t* conv_state;
  const uint16_t* conv_w;
  const float* a_log;
  const float* dt_bias;
  uint16_t* q;    // [B, QK]
  uint16_t* k;    // [B, QK]
  uint16_t* v;    // [B, VV]
  float* g;       // [B, HV]
  float* beta;    // [B, HV]
  int C, QK, HV, boff, aoff;
  int64_t P;
};

__global__ void __launch_bounds__(256) gdn_prep_kernel(PrepArgs a) {
  const int64_t b = blockIdx.x;
  const int c = blockIdx.y * 256 + threadIdx.x;
  if (c < a.C) {
    uint16_t* st = a.conv_state + b * 3 * a.C;
    const float s0 = bf(st[c]), s1 = bf(st[a.C + c]), s2 = bf(st[2 * a.C + c]);
    const uint16_t xh = a.proj[b * a.P + c];
    const float x = bf(xh);
    const uint16_t* wc = a.conv_w + static_cast<int64_t>(c) * 4;
    float acc = s0 * bf(wc[0]);
    acc = fmaf(s1, bf(wc[1]), acc);
    acc = fmaf(s2, bf(wc[2]), acc);
    acc = fmaf(x, bf(wc[3]), acc);
    const uint16_t y = tobf(silu(acc));
    st[c] = st[a.C + c];
    st[a.C + c] = st[2 * a.C + c];
    st[2 * a.C + c] = xh;
    if (c < a.QK) a.q[b * a.QK + c] = y;
    else if (c < 2 * a.QK) a.k[b * a.QK + c - a.QK] = y;
    else a.v[b * (a.C - 2 * a.QK) + c - 2 * a.QK] = y;
  }
  if (blockIdx.y == 0 && threadIdx.x < a.HV) {
    const int h = threadIdx.x;
    const float bb = bf(a.proj[b * a.P + a.boff + h]);
    const float aa = bf(a.proj[b * a.P + a.aoff + h]) + a.dt_bias[h];
    const float sp = aa > 20.f ? aa : log1pf(expf(aa));
    a.beta[b * a.HV + h] = bf(tobf(1.f / (1.f + expf(-bb))));   // beta is stored in the logits' dtype (bf16)
    a.g[b * a.HV + h] = -expf(a.a_log[h]) * sp;
  }
}

// One wave per (row, head) of 128 elements: o [N, H, 128] bf16 contiguous,
// z with row stride z_stride (head h at z + row * z_stride + h * 128).
__global__ void __launch_bounds__(256) gated_rmsnorm_kernel(const uint16_t* o, const uint16_t* z, int64_t z_stride,
                                                            const uint16_t* w, uint16_t* out, int64_t NH, int H,
                                                            float eps) {
  const int64_t item = static_cast<int64_t>(blockIdx.x) * 4 + threadIdx.x / kWave;
  if (item >= NH) return;
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = item / H, h = item % H;
  const uint32_t ov = reinterpret_cast<const uint32_t*>(o + item * 128)[lane];
  const uint32_t zv = reinterpret_cast<const uint32_t*>(z + row * z_stride + h * 128)[lane];
  const uint32_t wv = reinterpret_cast<const uint32_t*>(w)[lane];
  const float o0 = bf(ov & 0xffff), o1 = bf(ov >> 16);
  const float r = rsqrtf(wave_sum(o0 * o0 + o1 * o1) / 128.f + eps);
  const float y0 = bf(tobf(bf(wv & 0xffff) * bf(tobf(o0 * r))));
  const float y1 = bf(tobf(bf(wv >> 16) * bf(tobf(o1 * r))));
  const uint32_t res = tobf(y0 * silu(bf(zv & 0xffff))) | (static_cast<uint32_t>(tobf(y1 * silu(bf(zv >> 16)))) << 16);
  reinterpret_cast<uint32_t*>(out + item * 128)[lane] = res;
}

// out[n, i] = bf16(bf16(silu(gu[n, i])) * gu[n, I + i]), gu rows of 2I
// elements `gs` apart.
__global__ void __launch_bounds__(256) silu_mul_kernel(const uint16_t* gu, int64_t gs, uint16_t* out, int64_t N,
                                                       int I) {
  const int64_t idx = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * 8;
  if (idx >= N * I) return;
  const int64_t n = idx / I, i = idx % I;
  const uint4 gv = *reinterpret_cast<const uint4*>(gu + n * gs + i);
  const uint4 uv = *reinterpret_cast<const uint4*>(gu + n * gs + I + i);
  const uint16_t* g = reinterpret_cast<const uint16_t*>(&gv);
  const uint16_t* u = reinterpret_cast<const uint16_t*>(&uv);
  uint16_t o[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) o[j] = tobf(bf(tobf(silu(bf(g[j])))) * bf(u[j]));
  *reinterpret_cast<uint4*>(out + n * I + i) = *reinterpret_cast<const uint4*>(o);
}

// One wave per (token, head) of D = 128: y = bf16(x / rms(x) * (1 + w)), then
// rotate-half RoPE on the first rd dims with cos/sin [N_tok, rd] (fp32):
// out = bf16(y * cos + rotate_half(y) * sin), the rest copied.  The output
// row of (token n, head h) is out + n * out_tok_stride + h * out_head_stride.
struct RopeArgs {
  const uint16_t* x;
  int64_t x_tok_stride, x_head_stride;
  const uint16_t* w;
  const float* cos;
  const float* sin;
  uint16_t* out;
  int64_t out_tok_stride, out_head_stride;
  const int64_t* out_tok_index;  // optional: output row of token n is out_tok_index[n] (e.g. a ring slot)
  // optional ring write of the same token: head h of v (raw) goes to v_out at
  // the output row / strides of the normed head, and pos_val[n] (int32) to
  // pos_out[orow * pos_tok_stride + h * pos_head_stride]
  const uint16_t* v;
  int64_t v_tok_stride, v_head_stride;
  uint16_t* v_out;
  int32_t* pos_out;
  const int64_t* pos_val;
  int64_t pos_tok_stride, pos_head_stride;
  int64_t NH;
  int H, rd;
  float eps;
};

__global__ void __launch_bounds__(256) head_norm_rope_kernel(RopeArgs a) {
  const int64_t item = static_cast<int64_t>(blockIdx.x) * 4 + threadIdx.x / kWave;
  if (item >= a.NH) return;
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t n = item / a.H, h = item % a.H;
  const uint32_t xv = reinterpret_cast<const uint32_t*>(a.x + n * a.x_tok_stride + h * a.x_head_stride)[lane];
  const uint32_t wv = reinterpret_cast<const uint32_t*>(a.w)[lane];
  const float x0 = bf(xv & 0xffff), x1 = bf(xv >> 16);
  const float r = rsqrtf(wave_sum(x0 * x0 + x1 * x1) / 128.f + a.eps);
  float y0 = bf(tobf(x0 * r * (1.f + bf(wv & 0xffff))));
  float y1 = bf(tobf(x1 * r * (1.f + bf(wv >> 16))));
  // rotary part: element e = 2 * lane + {0, 1}; partner e +- rd/2
  const int e0 = 2 * lane, half = a.rd / 2;
  const bool rot = e0 < a.rd;
  const int pl = e0 < half ? lane + half / 2 : lane - half / 2;  // partner lane (rd/2 is even)
  const float p0 = __shfl(y0, rot ? pl : lane, kWave), p1 = __shfl(y1, rot ? pl : lane, kWave);
  if (rot) {
    const float c0 = a.cos[n * a.rd + e0], c1 = a.cos[n * a.rd + e0 + 1];
    const float s0 = a.sin[n * a.rd + e0], s1 = a.sin[n * a.rd + e0 + 1];
    const float sg = e0 < half ? -1.f : 1.f;
    y0 = y0 * c0 + sg * p0 * s0;
    y1 = y1 * c1 + sg * p1 * s1;
  }
  const int64_t orow = a.out_tok_index ? a.out_tok_index[n] : n;
  reinterpret_cast<uint32_t*>(a.out + orow * a.out_tok_stride + h * a.out_head_stride)[lane] =
      tobf(y0) | (static_cast<uint32_t>(tobf(y1)) << 16);
  if (a.v_out) {
    const uint32_t vv = reinterpret_cast<const uint32_t*>(a.v + n * a.v_tok_stride + h * a.v_head_stride)[lane];
    reinterpret_cast<uint32_t*>(a.v_out + orow * a.out_tok_stride + h * a.out_head_stride)[lane] = vv;
  }
  if (a.pos_out && lane == 0)
    a.pos_out[orow * a.pos_tok_stride + h * a.pos_head_stride] = static_cast<int32_t>(a.pos_val[n]);
}

// The memory-read prologue of one decode token (IndependentGQAMemory.
// _query_scores, modeling_yanchor.py:167-176): from the fused projection
// [q | admission features | ...] of token b,
//   q     = RoPE(RMSNorm_(1+w)(q_h))                          bf16 [B, H, 128]
//   gate  = tanh(read_scale_h) * 2 * sigmoid(<qn_h, gw_h> / sqrt(128) + gb_h)   f32 [B, H]
//           (qn_h: the normed head before RoPE, as bf16)
//   score = silu(features) (bf16) . adm_up^T                  f32 [B, G]
// Grid (B, H/4 + 1): four heads per workgroup (a wave each); the last column
// computes the admission scores (one wave, 64 features per lane pass).
struct MemProArgs {
  const uint16_t* proj;  // [B, P] rows ps apart
  int64_t ps;
  const uint16_t* w;     // q norm weight [128]
  const float* cos;      // [B, rd]
  const float* sin;
  const float* read_scale;  // [H]
  const float* gate_w;      // [H, 128]
  const float* gate_b;      // [H]
  const float* adm_up;      // [G, A]
  uint16_t* q;              // [B, H, 128]
  float* gate;              // [B, H]
  float* scores;            // [B, G]
  int H, G, A, rd, feat_off;
  float eps;
  uint16_t* act;            // [B, act_w] rows act_s apart, or null
  int64_t act_s;
  int act_off, act_w;       // writer gate columns [act_off, act_off + act_w), up columns after them
};

__global__ void __launch_bounds__(256) memory_prologue_kernel(MemProArgs a) {
  const int64_t b = blockIdx.x;
  const int lane = threadIdx.x & (kWave - 1), wv = threadIdx.x / kWave;
  const uint16_t* row = a.proj + b * a.ps;
  if (static_cast<int>(blockIdx.y) * 4 >= a.H) {
    if (wv != 0) {
      // waves 1-3: the writer's silu(gate) * up (silu_mul_kernel's roundings)
      if (a.act == nullptr) return;
      for (int v = (wv - 1) * kWave + lane; v < a.act_w / 8; v += 3 * kWave) {
        const uint4 gv = *reinterpret_cast<const uint4*>(row + a.act_off + 8 * v);
        const uint4 uv = *reinterpret_cast<const uint4*>(row + a.act_off + a.act_w + 8 * v);
        const uint16_t* g = reinterpret_cast<const uint16_t*>(&gv);
        const uint16_t* u = reinterpret_cast<const uint16_t*>(&uv);
        uint16_t o[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] = tobf(bf(tobf(silu(bf(g[j])))) * bf(u[j]));
        *reinterpret_cast<uint4*>(a.act + b * a.act_s + 8 * v) = *reinterpret_cast<const uint4*>(o);
      }
      return;
    }
    // wave 0: admission scores, silu(features) rounded to bf16, then fp32 dots
    for (int g = 0; g < a.G; ++g) {
      float acc = 0.f;
      for (int j = lane; j < a.A; j += kWave) acc = fmaf(bf(tobf(silu(bf(row[a.feat_off + j])))), a.adm_up[g * a.A + j], acc);
      acc = wave_sum(acc);
      if (lane == 0) a.scores[b * a.G + g] = acc;
    }
    return;
  }
  const int h = blockIdx.y * 4 + wv;
  if (h >= a.H) return;
  const uint32_t xv = reinterpret_cast<const uint32_t*>(row + h * 128)[lane];
  const uint32_t wvv = reinterpret_cast<const uint32_t*>(a.w)[lane];
  const float x0 = bf(xv & 0xffff), x1 = bf(xv >> 16);
  const float r = rsqrtf(wave_sum(x0 * x0 + x1 * x1) / 128.f + a.eps);
  float y0 = bf(tobf(x0 * r * (1.f + bf(wvv & 0xffff))));
  float y1 = bf(tobf(x1 * r * (1.f + bf(wvv >> 16))));
  // read gate from the normed (unrotated) head
  const float dot = wave_sum(fmaf(y0, a.gate_w[h * 128 + 2 * lane], y1 * a.gate_w[h * 128 + 2 * lane + 1]));
  if (lane == 0) {
    const float z = dot / sqrtf(128.f) + a.gate_b[h];
    a.gate[b * a.H + h] = tanhf(a.read_scale[h]) * 2.f * (1.f / (1.f + expf(-z)));
  }
  const int e0 = 2 * lane, half = a.rd / 2;
  const bool rot = e0 < a.rd;
  const int pl = e0 < half ? lane + half / 2 : lane - half / 2;
  const float p0 = __shfl(y0, rot ? pl : lane, kWave), p1 = __shfl(y1, rot ? pl : lane, kWave);
  if (rot) {
    const float c0 = a.cos[b * a.rd + e0], c1 = a.cos[b * a.rd + e0 + 1];
    const float s0 = a.sin[b * a.rd + e0], s1 = a.sin[b * a.rd + e0 + 1];
    const float sg = e0 < half ? -1.f : 1.f;
    y0 = y0 * c0 + sg * p0 * s0;
    y1 = y1 * c1 + sg * p1 * s1;
  }
  reinterpret_cast<uint32_t*>(a.q + (b * a.H + h) * 128)[lane] = tobf(y0) | (static_cast<uint32_t>(tobf(y1)) << 16);
}

}  // namespace
}  // namespace yh

extern "C" int yh_rmsnorm(const void* x, int64_t x_stride, const void* residual, void* residual_out, const void* w,
                          void* out, int64_t out_stride, int64_t N, int64_t D, float eps, int plus_one,
                          yh_stream_t stream) {
  using namespace yh;
  YH_CHECK_ARG(w && N >= 0 && (N == 0 || (x && out)), "rmsnorm: bad arguments");
  YH_CHECK_ARG(D > 0 && D % 8 == 0 && D <= kNormMaxD, "rmsnorm: D must be a multiple of 8 up to %d", kNormMaxD);
  YH_CHECK_ARG(x_stride % 8 == 0 && out_stride % 8 == 0, "rmsnorm: strides must be multiples of 8 elements");
  YH_CHECK_ARG(((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(w) |
                 reinterpret_cast<uintptr_t>(residual) | reinterpret_cast<uintptr_t>(residual_out)) & 15) == 0,
               "rmsnorm: pointers must be 16-byte aligned");
  if (N == 0) return YH_OK;
  NormArgs a{static_cast<const uint16_t*>(x), x_stride, nullptr, 0, 0, nullptr, 0,
             static_cast<const uint16_t*>(residual), static_cast<uint16_t*>(residual_out),
             static_cast<const uint16_t*>(w), static_cast<uint16_t*>(out), out_stride, nullptr, nullptr, 0,
             (int)D, plus_one, eps, nullptr, 0};
  launch_rmsnorm(a, N, static_cast<hipStream_t>(stream));
  YH_CHECK_LAUNCH("rmsnorm");
  return YH_OK;
}

extern "C" int yh_decode_inputs(const int64_t* tokens, const int64_t* positions, const void* embed, int64_t V,
                                const void* w, const float* inv_freq, const uint8_t* finished,
                                const int64_t* slot_rows, void* h, void* xn, float* cos, float* sin,
                                int64_t* ring_rows, uint8_t* valid, int64_t B, int64_t D, int64_t rotary_dim,
                                int64_t ring_stride, int64_t window, float eps, yh_stream_t stream) {
  using namespace yh;
  YH_CHECK_ARG(B >= 0 && V > 0 && window > 0 && ring_stride >= window, "decode_inputs: bad sizes");
  YH_CHECK_ARG(D > 0 && D % 8 == 0 && D <= kNormMaxD, "decode_inputs: D must be a multiple of 8 up to %d", kNormMaxD);
  YH_CHECK_ARG(rotary_dim >= 0 && rotary_dim % 2 == 0 && rotary_dim <= (D / 8 + kWave - 1) / kWave * kWave,
               "decode_inputs: rotary dim must be even and within the workgroup");
  YH_CHECK_ARG(B == 0 || (tokens && positions && embed && w && h && xn && ring_rows &&
                          (rotary_dim == 0 || (inv_freq && cos && sin))),
               "decode_inputs: null pointer");
  YH_CHECK_ARG(!valid == !finished && !valid == !slot_rows, "decode_inputs: valid needs finished and slot_rows");
  YH_CHECK_ARG(((reinterpret_cast<uintptr_t>(embed) | reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(h) |
                 reinterpret_cast<uintptr_t>(xn)) & 15) == 0,
               "decode_inputs: embed / w / h / xn must be 16-byte aligned");
  if (B == 0) return YH_OK;
  InputArgs a{tokens, positions, static_cast<const uint16_t*>(embed), static_cast<const uint16_t*>(w), inv_freq,
              finished, slot_rows, static_cast<uint16_t*>(h), static_cast<uint16_t*>(xn), cos, sin, ring_rows, valid,
              V, ring_stride, window, (int)D, (int)rotary_dim, eps};
  const unsigned threads = static_cast<unsigned>((D / 8 + kWave - 1) / kWave * kWave);
  hipLaunchKernelGGL(decode_inputs_kernel, dim3(static_cast<unsigned>(B)), dim3(threads), 0,
                     static_cast<hipStream_t>(stream), a);
  YH_CHECK_LAUNCH("decode_inputs");
  return YH_OK;
}

extern "C" int yh_rmsnorm_partials(const float* part, int64_t S, const void* proj_residual,
                                   int64_t proj_residual_stride, const float* part2, int64_t S2,
                                   const void* residual, void* residual_out,
                                   const void* w, void* out, int64_t out_stride, int64_t N, int64_t D, float eps,
                                   int plus_one, const void* w2, void* out2, int64_t out2_stride, yh_stream_t stream) {
  using namespace yh;
  YH_CHECK_ARG(w && N >= 0 && S >= 1 && (N == 0 || (part && out)), "rmsnorm_partials: bad arguments");
  YH_CHECK_ARG(!out2 == !w2, "rmsnorm_partials: out2 and w2 come together");
  YH_CHECK_ARG(!part2 || (!proj_residual && S2 >= 1 && S + S2 <= 64),
               "rmsnorm_partials: part2 replaces proj_residual, with 1 <= S2 and S + S2 <= 64");
  YH_CHECK_ARG(D > 0 && D % 8 == 0 && D <= kNormMaxD, "rmsnorm_partials: D must be a multiple of 8 up to %d",
               kNormMaxD);
  YH_CHECK_ARG(out_stride % 8 == 0 && (!proj_residual || proj_residual_stride % 8 == 0) &&
                   (!out2 || (out2_stride >= D && out2_stride % 8 == 0)),
               "rmsnorm_partials: strides must be multiples of 8 elements (out2_stride >= D)");
  YH_CHECK_ARG(((reinterpret_cast<uintptr_t>(part) | reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(w) |
                 reinterpret_cast<uintptr_t>(proj_residual) | reinterpret_cast<uintptr_t>(residual) |
                 reinterpret_cast<uintptr_t>(residual_out) | reinterpret_cast<uintptr_t>(w2) |
                 reinterpret_cast<uintptr_t>(out2) | reinterpret_cast<uintptr_t>(part2)) & 15) == 0,
               "rmsnorm_partials: pointers must be 16-byte aligned");
  if (N == 0) return YH_OK;
  NormArgs a{nullptr, 0, part, N * D, (int)S, static_cast<const uint16_t*>(proj_residual), proj_residual_stride,
             static_cast<const uint16_t*>(residual), static_cast<uint16_t*>(residual_out),
             static_cast<const uint16_t*>(w), static_cast<uint16_t*>(out), out_stride,
             static_cast<const uint16_t*>(w2), static_cast<uint16_t*>(out2), out2_stride, (int)D, plus_one, eps,
             part2, part2 ? (int)S2 : 0};
  launch_rmsnorm(a, N, static_cast<hipStream_t>(stream));
  YH_CHECK_LAUNCH("rmsnorm_partials");
  return YH_OK;
}

extern "C" int yh_gdn_decode_prep(const void* proj, int64_t proj_stride, void* conv_state, const void* conv_w,
                                  const float* a_log, const float* dt_bias, void* q, void* k, void* v, float* g,
                                  float* beta, int64_t B, int64_t conv_dim, int64_t qk_dim, int64_t HV,
                                  int64_t b_offset, int64_t a_offset, int64_t conv_kernel, yh_stream_t stream) {
  using namespace yh;
  YH_CHECK_ARG(B == 0 || (proj && conv_state && conv_w && a_log && dt_bias && q && k && v && g && beta),
               "gdn_prep: null pointer");
  YH_CHECK_ARG(conv_kernel == 4, "gdn_prep: conv kernel must be 4");
  YH_CHECK_ARG(B >= 0 && conv_dim > 2 * qk_dim && qk_dim > 0 && HV > 0 && HV <= 256, "gdn_prep: bad sizes");
  YH_CHECK_ARG(b_offset + HV <= proj_stride && a_offset + HV <= proj_stride && conv_dim <= proj_stride,
               "gdn_prep: projection layout exceeds the row");
  if (B == 0) return YH_OK;
  PrepArgs a{static_cast<const uint16_t*>(proj), static_cast<uint16_t*>(conv_state),
             static_cast<const uint16_t*>(conv_w), a_log, dt_bias, static_cast<uint16_t*>(q),
             static_cast<uint16_t*>(k), static_cast<uint16_t*>(v), g, beta, (int)conv_dim, (int)qk_dim, (int)HV,
             (int)b_offset, (int)a_offset, proj_stride};
  hipLaunchKernelGGL(gdn_prep_kernel, dim3(static_cast<unsigned>(B), static_cast<unsigned>((conv_dim + 255) / 256)),
                     dim3(256), 0, static_cast<hipStream_t>(stream), a);
  YH_CHECK_LAUNCH("gdn_prep");
  return YH_OK;
}

extern "C" int yh_gated_rmsnorm(const void* o, const void* z, int64_t z_stride, const void* w, void* out, int64_t N,
                                int64_t H, int64_t D, float eps, yh_stream_t stream) {
  using namespace yh;
  YH_CHECK_ARG(N >= 0 && H > 0 && (N == 0 || (o && z && w && out)), "gated_rmsnorm: bad arguments");
  YH_CHECK_ARG(D == 128, "gated_rmsnorm: head dim must be 128");
  YH_CHECK_ARG(z_stride % 2 == 0 && ((reinterpret_cast<uintptr_t>(z) | reinterpret_cast<uintptr_t>(o)) & 3) == 0,
               "gated_rmsnorm: 4-byte alignment");
  if (N == 0) return YH_OK;
  const int64_t nh = N * H;
  hipLaunchKernelGGL(gated_rmsnorm_kernel, dim3(static_cast<unsigned>((nh + 3) / 4)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(o),
                     static_cast<const uint16_t*>(z), z_stride, static_cast<const uint16_t*>(w),
                     static_cast<uint16_t*>(out), nh, (int)H, eps);
  YH_CHECK_LAUNCH("gated_rmsnorm");
  return YH_OK;
}

extern "C" int yh_silu_mul(const void* gate_up, int64_t gate_up_stride, void* out, int64_t N, int64_t I,
                           yh_stream_t stream) {
  using namespace yh;
  YH_CHECK_ARG(N >= 0 && (N == 0 || (gate_up && out)) && I > 0 && I % 8 == 0, "silu_mul: I must be a positive multiple of 8");
  YH_CHECK_ARG(gate_up_stride >= 2 * I && gate_up_stride % 8 == 0 &&
                   (reinterpret_cast<uintptr_t>(gate_up) & 15) == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0,
               "silu_mul: rows must be 16-byte aligned");
  if (N == 0) return YH_OK;
  const int64_t vecs = N * I / 8;
  hipLaunchKernelGGL(silu_mul_kernel, dim3(static_cast<unsigned>((vecs + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(gate_up), gate_up_stride,
                     static_cast<uint16_t*>(out), N, (int)I);
  YH_CHECK_LAUNCH("silu_mul");
  return YH_OK;
}

static int head_norm_rope_impl(const void* x, int64_t x_tok_stride, int64_t x_head_stride, const void* w,
                               const float* cos, const float* sin, void* out, int64_t out_tok_stride,
                               int64_t out_head_stride, const int64_t* out_tok_index, const void* v,
                               int64_t v_tok_stride, int64_t v_head_stride, void* v_out, int32_t* pos_out,
                               const int64_t* pos_val, int64_t pos_tok_stride, int64_t pos_head_stride, int64_t N,
                               int64_t H, int64_t D, int64_t rotary_dim, float eps, yh_stream_t stream) {
  using namespace yh;
  YH_CHECK_ARG(N >= 0 && H > 0 && (N == 0 || (x && w && out)), "head_norm_rope: bad arguments");
  YH_CHECK_ARG(D == 128, "head_norm_rope: head dim must be 128");
  YH_CHECK_ARG(rotary_dim >= 0 && rotary_dim <= D && rotary_dim % 4 == 0, "head_norm_rope: rotary dim %lld",
               (long long)rotary_dim);
  YH_CHECK_ARG(rotary_dim == 0 || (cos && sin), "head_norm_rope: cos/sin required");
  YH_CHECK_ARG((x_tok_stride | x_head_stride | out_tok_stride | out_head_stride | v_tok_stride | v_head_stride) % 2 ==
                   0,
               "head_norm_rope: strides must be even");
  YH_CHECK_ARG(N == 0 || !v_out || v, "ring write: value source required");
  YH_CHECK_ARG(N == 0 || !pos_out || pos_val, "ring write: positions required");
  if (N == 0) return YH_OK;
  RopeArgs a{static_cast<const uint16_t*>(x), x_tok_stride, x_head_stride, static_cast<const uint16_t*>(w), cos, sin,
             static_cast<uint16_t*>(out), out_tok_stride, out_head_stride, out_tok_index,
             static_cast<const uint16_t*>(v), v_tok_stride, v_head_stride, static_cast<uint16_t*>(v_out), pos_out,
             pos_val, pos_tok_stride, pos_head_stride, N * H, (int)H, (int)rotary_dim, eps};
  hipLaunchKernelGGL(head_norm_rope_kernel, dim3(static_cast<unsigned>((N * H + 3) / 4)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), a);
  YH_CHECK_LAUNCH("head_norm_rope");
  return YH_OK;
}

extern "C" int yh_head_norm_rope(const void* x, int64_t x_tok_stride, int64_t x_head_stride, const void* w,
                                 const float* cos, const float* sin, void* out, int64_t out_tok_stride,
                                 int64_t out_head_stride, const int64_t* out_tok_index, int64_t N, int64_t H,
                                 int64_t D, int64_t rotary_dim, float eps, yh_stream_t stream) {
  return head_norm_rope_impl(x, x_tok_stride, x_head_stride, w, cos, sin, out, out_tok_stride, out_head_stride,
                             out_tok_index, nullptr, 0, 0, nullptr, nullptr, nullptr, 0, 0, N, H, D, rotary_dim, eps,
                             stream);
}

extern "C" int yh_ring_write(const void* k, int64_t k_tok_stride, int64_t k_head_stride, const void* v,
                             int64_t v_tok_stride, int64_t v_head_stride, const void* w, const float* cos,
                             const float* sin, const int64_t* rows, const int64_t* positions, void* ring_k,
                             void* ring_v, int32_t* ring_pos, int64_t N, int64_t H, int64_t window, int64_t D,
                             int64_t rotary_dim, float eps, yh_stream_t stream) {
  using namespace yh;
  YH_CHECK_ARG(window > 0 && N >= 0, "ring_write: bad sizes");
  YH_CHECK_ARG(N == 0 || (rows && positions && ring_k && ring_v && ring_pos && v), "ring_write: null pointer");
  return head_norm_rope_impl(k, k_tok_stride, k_head_stride, w, cos, sin, ring_k, D, window * D, rows, v, v_tok_stride,
                             v_head_stride, ring_v, ring_pos, positions, 1, window, N, H, D, rotary_dim, eps, stream);
}

extern "C" int yh_memory_prologue(const void* proj, int64_t proj_stride, int64_t feat_offset, const void* q_norm_w,
                                  const float* cos, const float* sin, const float* read_scale, const float* gate_w,
                                  const float* gate_b, const float* adm_up, void* q, float* gate, float* scores,
                                  int64_t B, int64_t H, int64_t D, int64_t G, int64_t A, int64_t rotary_dim, float eps,
                                  int64_t act_offset, int64_t act_width, void* act, int64_t act_stride,
                                  yh_stream_t stream) {
  using namespace yh;
  YH_CHECK_ARG(D == 128, "memory_prologue: head dim must be 128");
  YH_CHECK_ARG(!act || (act_width > 0 && act_width % 8 == 0 && act_offset % 8 == 0 && proj_stride % 8 == 0 &&
                        act_offset >= 0 && act_offset + 2 * act_width <= proj_stride && act_stride >= act_width &&
                        act_stride % 8 == 0 && (reinterpret_cast<uintptr_t>(act) & 15) == 0 &&
                        (reinterpret_cast<uintptr_t>(proj) & 15) == 0),
               "memory_prologue: the writer activation needs 16-byte aligned rows with gate and up inside proj");
  YH_CHECK_ARG(B >= 0 && H > 0 && G > 0 && A > 0 && G <= 64, "memory_prologue: bad sizes");
  YH_CHECK_ARG(rotary_dim >= 0 && rotary_dim <= D && rotary_dim % 4 == 0, "memory_prologue: rotary dim");
  YH_CHECK_ARG(feat_offset >= H * D && feat_offset + A <= proj_stride && proj_stride % 2 == 0,
               "memory_prologue: the features must follow the query in each projection row");
  if (B == 0) return YH_OK;
  YH_CHECK_ARG(proj && q_norm_w && read_scale && gate_w && gate_b && adm_up && q && gate && scores &&
                   (rotary_dim == 0 || (cos && sin)),
               "memory_prologue: null pointer");
  YH_CHECK_ARG((reinterpret_cast<uintptr_t>(proj) & 3) == 0, "memory_prologue: projection must be 4-byte aligned");
  MemProArgs a{static_cast<const uint16_t*>(proj), proj_stride, static_cast<const uint16_t*>(q_norm_w), cos, sin,
               read_scale, gate_w, gate_b, adm_up, static_cast<uint16_t*>(q), gate, scores, (int)H, (int)G, (int)A,
               (int)rotary_dim, (int)feat_offset, eps, static_cast<uint16_t*>(act), act_stride, (int)act_offset,
               (int)act_width};
  const dim3 grid(static_cast<unsigned>(B), static_cast<unsigned>((H + 3) / 4 + 1));
  hipLaunchKernelGGL(memory_prologue_kernel, grid, dim3(256), 0, static_cast<hipStream_t>(stream), a);
  YH_CHECK_LAUNCH("memory_prologue");
  return YH_OK;
}
