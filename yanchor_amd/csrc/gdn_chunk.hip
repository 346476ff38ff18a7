// Chunked varlen prefill of the gated delta rule on bf16 MFMA (gfx950).
//
// Follows torch_chunk_gated_delta_rule (transformers wheel,
// models/qwen3_5/modeling_qwen3_5.py:234-311) with chunk C = 64: per chunk,
//   G = cumsum(g);  Gamma[t][s] = exp(G_t - G_s) for s <= t
//   L = beta_t (k_t . k_s) Gamma[t][s] for s < t;  T = (I + L)^{-1}
//   U = T diag(beta) V;  W S = T diag(beta e^G) (K S)
//   v_new = U - W S
//   o = diag(e^G) Q S + (Q K^T o Gamma) v_new
//   S <- e^{G_last} S + K^T diag(e^{G_last - G}) v_new
// with q, k L2-normalised (eps 1e-6 inside rsqrt) and q scaled.
//
// Layout of the work: one workgroup (8 waves) per (sequence, value head,
// 64-wide value tile); the 128 x 64 fp32 state tile stays in MFMA
// accumulators across the sequence's chunks (value tiles of one head evolve
// independently).  Per-token L2 norms, beta and decays are diagonal factors,
// so every product with the raw q / k / v tensors runs on exact bf16 MFMA
// operands and the factors are applied in the epilogues.  Products whose
// operands are fp32 on chip (the state, T, P = K S, v_new) split each fp32
// operand into bf16 hi + lo and accumulate 2 or 3 MFMA passes (hi.hi, hi.lo,
// lo.hi), which keeps the state path near fp32 accuracy; the output-only
// product (Q K^T o Gamma) v_new and Q S use one pass.  T is inverted in fp32 on
// the VALU by 16 x 16 blocks.  Sequences are independent; `order` lets the
// caller dispatch the longest sequences first.
#include "common.h"

namespace yh {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4v __attribute__((ext_vector_type(4)));

constexpr int kC = 64;        // chunk length
constexpr int kK = 128;       // key dim
constexpr int kVT = 64;       // value tile
constexpr int kThreads = 512;
constexpr int SKR = 136;      // bf16 row stride of 128-wide matrices (padded: conflict-free 16 B reads)
constexpr int SK64 = 72;      // bf16 row stride of 64-wide matrices
constexpr int SF = 68;        // fp32 row stride of 64-wide matrices

struct ChunkArgs {
  const uint16_t* q;   // [total, H, K]
  const uint16_t* k;   // [total, H, K]
  const uint16_t* v;   // [total, HV, V]
  const void* g;       // [total, HV]
  const void* beta;    // [total, HV]
  const float* h0;     // [N, HV, K, V] or null
  float* ht;           // [N, HV, K, V]
  uint16_t* o;         // [total, HV, V]
  const int32_t* cu;   // [N + 1]
  const int32_t* order;  // [N] or null
  int n_seqs, H, HV, V;
  float scale;
  int l2, g_dt, beta_dt;
};

struct __align__(16) Smem {
  uint16_t kr[kC * SKR];   // K [t][d]
  uint16_t kt[kK * SK64];  // K^T [d][t]
  union {
    uint16_t q[kC * SKR];  // Q [t][d]
    float pt[kVT * SF];    // P^T [v][t], P = K S
  } qp;
  uint16_t vt[kVT * SK64];  // V tile ^T [v][t]
  union {
    struct {
      uint16_t hi[kVT * SKR];  // S^T [v][d], bf16 hi part
      uint16_t lo[kVT * SKR];  // S^T, bf16 lo part
    } st;
    struct {
      uint16_t vn[kVT * SK64];   // v_new^T [v][t]
      uint16_t dhi[kVT * SK64];  // (diag(d2) v_new)^T hi
      uint16_t dlo[kVT * SK64];  // (diag(d2) v_new)^T lo
    } vn;
  } sv;
  float l[kC * SF];    // L
  float t[kC * SF];    // T = (I + L)^{-1}
  float aqk[kC * SF];  // (Q K^T o Gamma) with the q / k scalings
  float x[3 * 256];    // block-inversion scratch
  float rk[kC], rqs[kC], G[kC], beta[kC], d1[kC], d2[kC], orow[kC];
  float gl;
};

__device__ __forceinline__ bf16x8_t lds8(const uint16_t* p) {
  return __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(p));
}
__device__ __forceinline__ uint32_t pack2(uint16_t a, uint16_t b) {
  return static_cast<uint32_t>(a) | (static_cast<uint32_t>(b) << 16);
}
__device__ __forceinline__ float bfv(uint16_t h) { return __uint_as_float(static_cast<uint32_t>(h) << 16); }

// 8 fp32 values (times optional per-element scales) -> bf16 hi / lo vectors.
__device__ __forceinline__ void split8(const float* x, bf16x8_t& hi, bf16x8_t& lo) {
  uint16_t h[8], l[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    h[j] = f32_to_bf16(x[j]);
    l[j] = f32_to_bf16(x[j] - bfv(h[j]));
  }
  hi = __builtin_bit_cast(bf16x8_t, make_uint4(pack2(h[0], h[1]), pack2(h[2], h[3]), pack2(h[4], h[5]), pack2(h[6], h[7])));
  lo = __builtin_bit_cast(bf16x8_t, make_uint4(pack2(l[0], l[1]), pack2(l[2], l[3]), pack2(l[4], l[5]), pack2(l[6], l[7])));
}
__device__ __forceinline__ bf16x8_t round8(const float* x) {
  uint16_t h[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) h[j] = f32_to_bf16(x[j]);
  return __builtin_bit_cast(bf16x8_t, make_uint4(pack2(h[0], h[1]), pack2(h[2], h[3]), pack2(h[4], h[5]), pack2(h[6], h[7])));
}
__device__ __forceinline__ void ld8f(const float* p, float* x) {
  const float4 a = reinterpret_cast<const float4*>(p)[0], b = reinterpret_cast<const float4*>(p)[1];
  x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w; x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
}
__device__ __forceinline__ f32x4v mfma(bf16x8_t a, bf16x8_t b, f32x4v c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// (I + L)^{-1} for strictly lower triangular L (64 x 64, fp32, LDS), by 16 x 16
// blocks: the diagonal blocks by column-parallel forward substitution (one lane
// per column, L rows read as 16-byte vectors), then the off-diagonal blocks
// level by level, T_ij = -T_ii sum_{m=j}^{i-1} L_im T_mj, one thread per
// 4 adjacent columns so T and X rows are read as vectors.
__device__ void invert_unit_lower(Smem& sm) {
  const int tid = threadIdx.x;
  if (tid < 64) {
    const int b = tid >> 4, j = tid & 15;
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float lr[16];
      ld8f(&sm.l[(16 * b + i) * SF + 16 * b], lr);
      ld8f(&sm.l[(16 * b + i) * SF + 16 * b + 8], lr + 8);
      float acc = i == j ? 1.f : 0.f;
#pragma unroll
      for (int m = 0; m < i; ++m) acc = fmaf(-lr[m], x[m], acc);
      x[i] = acc;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) sm.t[(16 * b + i) * SF + 16 * b + j] = x[i];
  } else {
    // zero the strictly upper blocks
    for (int e = tid - 64; e < 64 * 64; e += kThreads - 64) {
      const int r = e >> 6, c = e & 63;
      if ((c >> 4) > (r >> 4)) sm.t[r * SF + c] = 0.f;
    }
  }
  __syncthreads();
#pragma unroll 1
  for (int lev = 1; lev < 4; ++lev) {
    const int nb = 4 - lev;  // blocks (i, i - lev), i = lev..3; 64 threads per block
    if (tid < nb * 64) {
      const int bi = tid >> 6, r = (tid >> 2) & 15, c4 = (tid & 3) * 4;
      const int i = lev + bi, j = i - lev;
      float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
      for (int m = j; m < i; ++m) {
        float lr[16];
        ld8f(&sm.l[(16 * i + r) * SF + 16 * m], lr);
        ld8f(&sm.l[(16 * i + r) * SF + 16 * m + 8], lr + 8);
#pragma unroll
        for (int q = 0; q < 16; ++q) {
          const float4 tv = *reinterpret_cast<const float4*>(&sm.t[(16 * m + q) * SF + 16 * j + c4]);
          acc.x = fmaf(lr[q], tv.x, acc.x);
          acc.y = fmaf(lr[q], tv.y, acc.y);
          acc.z = fmaf(lr[q], tv.z, acc.z);
          acc.w = fmaf(lr[q], tv.w, acc.w);
        }
      }
      *reinterpret_cast<float4*>(&sm.x[bi * 256 + r * 16 + c4]) = acc;
    }
    __syncthreads();
    if (tid < nb * 64) {
      const int bi = tid >> 6, r = (tid >> 2) & 15, c4 = (tid & 3) * 4;
      const int i = lev + bi, j = i - lev;
      float tr[16];
      ld8f(&sm.t[(16 * i + r) * SF + 16 * i], tr);
      ld8f(&sm.t[(16 * i + r) * SF + 16 * i + 8], tr + 8);
      float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const float4 xv = *reinterpret_cast<const float4*>(&sm.x[bi * 256 + q * 16 + c4]);
        acc.x = fmaf(tr[q], xv.x, acc.x);
        acc.y = fmaf(tr[q], xv.y, acc.y);
        acc.z = fmaf(tr[q], xv.z, acc.z);
        acc.w = fmaf(tr[q], xv.w, acc.w);
      }
      *reinterpret_cast<float4*>(&sm.t[(16 * i + r) * SF + 16 * j + c4]) =
          make_float4(-acc.x, -acc.y, -acc.z, -acc.w);
    }
    __syncthreads();
  }
}

__global__ void __launch_bounds__(kThreads) gdn_chunk_kernel(ChunkArgs a) {
  __shared__ Smem sm;
  const int nvt = a.V / kVT;
  int blk = blockIdx.x;
  const int vt = blk % nvt;
  blk /= nvt;
  const int hv = blk % a.HV;
  const int sidx = blk / a.HV;
  const int n = a.order ? a.order[sidx] : sidx;
  const int hk = hv / (a.HV / a.H);
  const int64_t tb = a.cu[n], te = a.cu[n + 1];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int r16 = lane & 15, kq = (lane >> 4) * 8, rq4 = (lane >> 4) * 4;
  const int vbase = vt * kVT;

  // state tile: wave w owns rows d in [16w, 16w + 16) and the four 16-wide value tiles
  f32x4v S[4];
  const int64_t sbase = (static_cast<int64_t>(n) * a.HV + hv) * kK;
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      S[j][i] = a.h0 ? a.h0[(sbase + 16 * w + rq4 + i) * a.V + vbase + 16 * j + r16] : 0.f;

  for (int64_t c0 = tb; c0 < te; c0 += kC) {
    const int Lc = static_cast<int>(te - c0 < kC ? te - c0 : kC);
    // ---- (a) stage K, Q, V tile and gates; state -> S^T hi / lo ----
    for (int ci = tid; ci < kC * 16; ci += kThreads) {
      const int t = ci >> 4, d8 = (ci & 15) * 8;
      uint4 kw = make_uint4(0, 0, 0, 0), qw = make_uint4(0, 0, 0, 0);
      if (t < Lc) {
        const int64_t off = ((c0 + t) * a.H + hk) * kK + d8;
        kw = *reinterpret_cast<const uint4*>(a.k + off);
        qw = *reinterpret_cast<const uint4*>(a.q + off);
      }
      *reinterpret_cast<uint4*>(&sm.kr[t * SKR + d8]) = kw;
      *reinterpret_cast<uint4*>(&sm.qp.q[t * SKR + d8]) = qw;
      const uint32_t kk[4] = {kw.x, kw.y, kw.z, kw.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        sm.kt[(d8 + 2 * j) * SK64 + t] = static_cast<uint16_t>(kk[j] & 0xffff);
        sm.kt[(d8 + 2 * j + 1) * SK64 + t] = static_cast<uint16_t>(kk[j] >> 16);
      }
    }
    {
      const int t = tid >> 3, v8 = (tid & 7) * 8;
      uint4 vw = make_uint4(0, 0, 0, 0);
      if (t < Lc) vw = *reinterpret_cast<const uint4*>(a.v + ((c0 + t) * a.HV + hv) * a.V + vbase + v8);
      const uint32_t vv[4] = {vw.x, vw.y, vw.z, vw.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        sm.vt[(v8 + 2 * j) * SK64 + t] = static_cast<uint16_t>(vv[j] & 0xffff);
        sm.vt[(v8 + 2 * j + 1) * SK64 + t] = static_cast<uint16_t>(vv[j] >> 16);
      }
    }
    if (tid < kC) {
      float gg = 0.f, bb = 0.f;
      if (tid < Lc) {
        gg = load_any(a.g, (c0 + tid) * a.HV + hv, a.g_dt);
        bb = load_any(a.beta, (c0 + tid) * a.HV + hv, a.beta_dt);
      }
      sm.G[tid] = gg;
      sm.beta[tid] = bb;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int d = 16 * w + rq4 + i, vv = 16 * j + r16;
        const float x = S[j][i];
        const uint16_t h = f32_to_bf16(x);
        sm.sv.st.hi[vv * SKR + d] = h;
        sm.sv.st.lo[vv * SKR + d] = f32_to_bf16(x - bfv(h));
      }
    __syncthreads();
    // ---- per-token scalars: norms (8 lanes per token), decay scan ----
    {
      const int t = tid >> 3, p = tid & 7;
      float sk = 0.f, sq = 0.f;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float kf = bfv(sm.kr[t * SKR + 16 * p + e]);
        const float qf = bfv(sm.qp.q[t * SKR + 16 * p + e]);
        sk = fmaf(kf, kf, sk);
        sq = fmaf(qf, qf, sq);
      }
#pragma unroll
      for (int off = 1; off < 8; off <<= 1) {
        sk += __shfl_xor(sk, off, kWave);
        sq += __shfl_xor(sq, off, kWave);
      }
      if (p == 0) {
        sm.rk[t] = a.l2 ? rsqrtf(sk + 1e-6f) : 1.f;
        sm.rqs[t] = (a.l2 ? rsqrtf(sq + 1e-6f) : 1.f) * a.scale;
      }
    }
    if (w == 7) {
      float x = sm.G[lane];
#pragma unroll
      for (int off = 1; off < kWave; off <<= 1) {
        const float y = __shfl_up(x, off, kWave);
        if (lane >= off) x += y;
      }
      sm.G[lane] = x;
      if (lane == kWave - 1) sm.gl = x;
    }
    __syncthreads();
    if (tid < kC) {
      const float eg = expf(sm.G[tid]);
      sm.d1[tid] = sm.beta[tid] * eg * sm.rk[tid];
      sm.d2[tid] = sm.rk[tid] * expf(sm.gl - sm.G[tid]);
      sm.orow[tid] = eg * sm.rqs[tid];
    }
    __syncthreads();

    // ---- (c) K K^T, Q K^T, Q S, P = K S ----
    f32x4v oacc[2], pacc[2];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const int tau = 2 * w + tt, mt = tau >> 2, nt = tau & 3, m0 = 16 * mt, n0 = 16 * nt;
      f32x4v kk = {0.f, 0.f, 0.f, 0.f}, qk = {0.f, 0.f, 0.f, 0.f};
      if (nt <= mt) {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          const int k0 = 32 * ks;
          const bf16x8_t b = lds8(&sm.kr[(n0 + r16) * SKR + k0 + kq]);
          kk = mfma(lds8(&sm.kr[(m0 + r16) * SKR + k0 + kq]), b, kk);
          qk = mfma(lds8(&sm.qp.q[(m0 + r16) * SKR + k0 + kq]), b, qk);
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = m0 + rq4 + i, s = n0 + r16;
        const float dec = s <= t ? expf(sm.G[t] - sm.G[s]) : 0.f;
        sm.l[t * SF + s] = s < t ? sm.beta[t] * sm.rk[t] * sm.rk[s] * dec * kk[i] : 0.f;
        sm.aqk[t * SF + s] = s <= t ? sm.rqs[t] * sm.rk[s] * dec * qk[i] : 0.f;
      }
      f32x4v qs = {0.f, 0.f, 0.f, 0.f}, pp = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const int k0 = 32 * ks;
        const bf16x8_t sh = lds8(&sm.sv.st.hi[(n0 + r16) * SKR + k0 + kq]);
        const bf16x8_t sl = lds8(&sm.sv.st.lo[(n0 + r16) * SKR + k0 + kq]);
        const bf16x8_t ka = lds8(&sm.kr[(m0 + r16) * SKR + k0 + kq]);
        qs = mfma(lds8(&sm.qp.q[(m0 + r16) * SKR + k0 + kq]), sh, qs);
        pp = mfma(ka, sh, pp);
        pp = mfma(ka, sl, pp);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) qs[i] *= sm.orow[m0 + rq4 + i];
      oacc[tt] = qs;
      pacc[tt] = pp;
    }
    __syncthreads();  // Q and S^T are dead from here on
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const int tau = 2 * w + tt, m0 = 16 * (tau >> 2), n0 = 16 * (tau & 3);
#pragma unroll
      for (int i = 0; i < 4; ++i) sm.qp.pt[(n0 + r16) * SF + m0 + rq4 + i] = pacc[tt][i];
    }
    // ---- (e) T = (I + L)^{-1} ----
    invert_unit_lower(sm);  // ends with a barrier (also orders the P^T writes)

    // ---- (f) U = T diag(beta) V, Y = T diag(d1) P, v_new = U - Y ----
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const int tau = 2 * w + tt, mt = tau >> 2, m0 = 16 * mt, n0 = 16 * (tau & 3);
      f32x4v u = {0.f, 0.f, 0.f, 0.f}, y = {0.f, 0.f, 0.f, 0.f};
      const int ksteps = (16 * (mt + 1) + 31) / 32;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        if (ks >= ksteps) break;
        const int k0 = 32 * ks;
        float trow[8], bsc[8], dsc[8], xa[8], pv[8];
        ld8f(&sm.t[(m0 + r16) * SF + k0 + kq], trow);
        ld8f(&sm.beta[k0 + kq], bsc);
        ld8f(&sm.d1[k0 + kq], dsc);
        ld8f(&sm.qp.pt[(n0 + r16) * SF + k0 + kq], pv);
        bf16x8_t ah, al, bh, bl;
#pragma unroll
        for (int j = 0; j < 8; ++j) xa[j] = trow[j] * bsc[j];
        split8(xa, ah, al);
        const bf16x8_t vb = lds8(&sm.vt[(n0 + r16) * SK64 + k0 + kq]);
        u = mfma(ah, vb, u);
        u = mfma(al, vb, u);
#pragma unroll
        for (int j = 0; j < 8; ++j) xa[j] = trow[j] * dsc[j];
        split8(xa, ah, al);
        split8(pv, bh, bl);
        y = mfma(ah, bh, y);
        y = mfma(ah, bl, y);
        y = mfma(al, bh, y);
      }
      pacc[tt] = u - y;  // v_new tile (registers of P are free now)
    }
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const int tau = 2 * w + tt, m0 = 16 * (tau >> 2), n0 = 16 * (tau & 3);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = m0 + rq4 + i, vv = n0 + r16;
        const float x = pacc[tt][i];
        sm.sv.vn.vn[vv * SK64 + t] = f32_to_bf16(x);
        const float z = sm.d2[t] * x;
        const uint16_t zh = f32_to_bf16(z);
        sm.sv.vn.dhi[vv * SK64 + t] = zh;
        sm.sv.vn.dlo[vv * SK64 + t] = f32_to_bf16(z - bfv(zh));
      }
    }
    __syncthreads();

    // ---- (g) o += (Q K^T o Gamma) v_new; S <- e^{G_last} S + K^T diag(d2) v_new ----
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const int tau = 2 * w + tt, mt = tau >> 2, m0 = 16 * mt, n0 = 16 * (tau & 3);
      const int ksteps = (16 * (mt + 1) + 31) / 32;
      f32x4v acc = oacc[tt];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        if (ks >= ksteps) break;
        const int k0 = 32 * ks;
        float ar[8];
        ld8f(&sm.aqk[(m0 + r16) * SF + k0 + kq], ar);
        acc = mfma(round8(ar), lds8(&sm.sv.vn.vn[(n0 + r16) * SK64 + k0 + kq]), acc);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = m0 + rq4 + i;
        if (t < Lc) a.o[((c0 + t) * a.HV + hv) * a.V + vbase + n0 + r16] = f32_to_bf16(acc[i]);
      }
    }
    const float egl = expf(sm.gl);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      f32x4v s = S[j] * egl;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const int k0 = 32 * ks;
        const bf16x8_t ak = lds8(&sm.kt[(16 * w + r16) * SK64 + k0 + kq]);
        s = mfma(ak, lds8(&sm.sv.vn.dhi[(16 * j + r16) * SK64 + k0 + kq]), s);
        s = mfma(ak, lds8(&sm.sv.vn.dlo[(16 * j + r16) * SK64 + k0 + kq]), s);
      }
      S[j] = s;
    }
    __syncthreads();  // the next chunk restages every LDS buffer
  }
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i) a.ht[(sbase + 16 * w + rq4 + i) * a.V + vbase + 16 * j + r16] = S[j][i];
}

}  // namespace
}  // namespace yh

extern "C" int yh_gdn_chunk_varlen(const void* q, const void* k, const void* v, const void* g, const void* beta,
                                   const float* initial_state, float* final_state, void* o,
                                   const int32_t* cu_seqlens, const int32_t* order, int64_t n_seqs, int64_t H,
                                   int64_t HV, int64_t K, int64_t V, float scale, int use_qk_l2norm, int qkv_dtype,
                                   int g_dtype, int beta_dtype, yh_stream_t stream) {
  using namespace yh;
  YH_CHECK_ARG(q && k && v && g && beta && final_state && o && cu_seqlens, "gdn_chunk: null pointer");
  YH_CHECK_ARG(n_seqs >= 0 && H > 0 && HV > 0 && HV % H == 0, "gdn_chunk: bad sizes");
  YH_CHECK_ARG(K == 128, "gdn_chunk: K must be 128 (got %lld)", (long long)K);
  YH_CHECK_ARG(V > 0 && V % 64 == 0, "gdn_chunk: V must be a positive multiple of 64 (got %lld)", (long long)V);
  YH_CHECK_ARG(qkv_dtype == YH_BF16, "gdn_chunk: q/k/v must be bfloat16");
  YH_CHECK_ARG(is_float_dtype(g_dtype) && is_float_dtype(beta_dtype), "gdn_chunk: bad gate dtypes");
  YH_CHECK_ARG(((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v)) &
                15) == 0,
               "gdn_chunk: q/k/v must be 16-byte aligned");
  YH_CHECK_ARG(n_seqs * HV * (V / 64) < (1LL << 31), "gdn_chunk: grid too large");
  if (n_seqs == 0) return YH_OK;
  ChunkArgs a{static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k), static_cast<const uint16_t*>(v), g,
              beta, initial_state, final_state, static_cast<uint16_t*>(o), cu_seqlens, order, (int)n_seqs, (int)H,
              (int)HV, (int)V, scale, use_qk_l2norm ? 1 : 0, g_dtype, beta_dtype};
  hipLaunchKernelGGL(gdn_chunk_kernel, dim3(static_cast<unsigned>(n_seqs * HV * (V / 64))), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), a);
  YH_CHECK_LAUNCH("gdn_chunk");
  return YH_OK;
}
