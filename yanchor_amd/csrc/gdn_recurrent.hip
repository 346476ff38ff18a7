// Gated delta rule, token-recurrent form, fp32 state updated in place.
//
// Replaces the FLA fused_recurrent_gated_delta_rule launch with h0 == ht
// (runtime/model/inference_kernels.py:147-173) and follows the arithmetic of
// torch_recurrent_gated_delta_rule (transformers wheel,
// models/qwen3_5/modeling_qwen3_5.py:314-353):
//   S <- exp(g) S;  kv = S^T k;  delta = beta (v - kv);  S <- S + k delta^T;
//   o = S^T q
// with q, k optionally L2-normalised (eps 1e-6 inside rsqrt) and q scaled.
//
// Decode (T = 1) is HBM-bound on the state read-modify-write: every state
// element is read once and written once.  One workgroup owns one
// (batch row, value head, value tile) and keeps its K x VT slice of the state
// in registers for all T steps:
//   * LPR = VT/4 lanes cover one state row with 16-byte accesses, so a wave's
//     load/store instruction touches whole contiguous rows;
//   * the K rows are dealt round-robin to RG = NT/LPR row groups;
//   * the column reductions S^T k and S^T q are xor-shuffle reductions across
//     the row groups of a wave followed by one LDS exchange across waves;
//   * o = exp(g) S^T q + delta (k.q) is formed from the same pass, so the
//     updated state is never re-read.
// The state loads are issued before anything else so their HBM latency
// overlaps the q/k normalisation, and both state directions use nontemporal
// (streaming) accesses.
#include "common.h"

#include <stdlib.h>

namespace yh {
namespace {

struct GdnArgs {
  const void* q;
  const void* k;
  const void* v;
  const void* g;
  const void* beta;
  float* state;
  const int32_t* idx;
  const int32_t* cu;  // packed varlen offsets [B + 1] or null
  void* o;
  int B, T, H, HV, V;
  int64_t n_rows;
  float scale;
  int l2;
  int g_dt, beta_dt;
};

__device__ __forceinline__ float4 f4(float x) { return make_float4(x, x, x, x); }
__device__ __forceinline__ float4 fma4(float4 a, float b, float4 c) {
  return make_float4(fmaf(a.x, b, c.x), fmaf(a.y, b, c.y), fmaf(a.z, b, c.z), fmaf(a.w, b, c.w));
}

// Per-token inputs of one step, loaded ahead of use (for step 0 before the
// state loads, for step t+1 before the state update of step t).  They are kept
// as raw bits and converted only where they are used, so no wait on them is
// placed in front of the state stream.
template <int DT> struct Raw4 { using T = uint2; };
template <> struct Raw4<YH_F32> { using T = uint4; };

template <int DT>
__device__ __forceinline__ typename Raw4<DT>::T ld_raw4(const void* p, int64_t i) {
  if constexpr (DT == YH_F32) return reinterpret_cast<const uint4*>(static_cast<const float*>(p) + i)[0];
  else return reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(p) + i)[0];
}
template <int DT>
__device__ __forceinline__ float4 cvt4(const typename Raw4<DT>::T& w) {
  if constexpr (DT == YH_F32) {
    return make_float4(__uint_as_float(w.x), __uint_as_float(w.y), __uint_as_float(w.z), __uint_as_float(w.w));
  } else if constexpr (DT == YH_BF16) {
    return make_float4(__uint_as_float(w.x << 16), __uint_as_float(w.x & 0xffff0000u),
                       __uint_as_float(w.y << 16), __uint_as_float(w.y & 0xffff0000u));
  } else {
    return make_float4(f16_to_f32(w.x & 0xffff), f16_to_f32(w.x >> 16), f16_to_f32(w.y & 0xffff),
                       f16_to_f32(w.y >> 16));
  }
}
template <int DT>
__device__ __forceinline__ uint32_t ld_raw1(const void* p, int64_t i) {
  if constexpr (DT == YH_F32) return static_cast<const uint32_t*>(p)[i];
  else return static_cast<const uint16_t*>(p)[i];
}
template <int DT>
__device__ __forceinline__ float cvt1(uint32_t w) {
  if constexpr (DT == YH_F32) return __uint_as_float(w);
  else if constexpr (DT == YH_BF16) return __uint_as_float(w << 16);
  else return f16_to_f32(static_cast<uint16_t>(w));
}
__device__ __forceinline__ uint32_t ld_raw_any(const void* p, int64_t i, int dt) {
  return dt == YH_F32 ? static_cast<const uint32_t*>(p)[i] : static_cast<const uint16_t*>(p)[i];
}
__device__ __forceinline__ float cvt_any(uint32_t w, int dt) {
  return dt == YH_F32 ? __uint_as_float(w)
         : dt == YH_BF16 ? __uint_as_float(w << 16) : f16_to_f32(static_cast<uint16_t>(w));
}

template <int DT, int KPL>
struct TokIn {
  uint32_t kx[KPL], qx[KPL];  // raw q / k (normalising wave only)
  typename Raw4<DT>::T v;     // this thread's 4 value columns
  uint32_t g, beta;
};

template <int DT, int K, int KPL>
__device__ __forceinline__ void load_tok(TokIn<DT, KPL>& in, const GdnArgs& a, int64_t tok, int hk,
                                         int hv, int col0, bool norm_wave, int lane) {
  if (norm_wave) {
    const int64_t base = (tok * a.H + hk) * K;
#pragma unroll
    for (int j = 0; j < KPL; ++j) {
      in.kx[j] = ld_raw1<DT>(a.k, base + lane + j * kWave);
      in.qx[j] = ld_raw1<DT>(a.q, base + lane + j * kWave);
    }
  }
  const int64_t vh = tok * a.HV + hv;
  in.v = ld_raw4<DT>(a.v, vh * a.V + col0);
  in.g = ld_raw_any(a.g, vh, a.g_dt);
  in.beta = ld_raw_any(a.beta, vh, a.beta_dt);
}

__device__ __forceinline__ void wave_sum3(float& x, float& y, float& z) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float a = __shfl_xor(x, off, kWave), b = __shfl_xor(y, off, kWave), c = __shfl_xor(z, off, kWave);
    x += a; y += b; z += c;
  }
}

template <int DT, int K, int VT, int NT>
__global__ void __launch_bounds__(NT) gdn_recurrent_kernel(GdnArgs a) {
  constexpr int LPR = VT / 4;
  constexpr int RG = NT / LPR;
  constexpr int RPT = K / RG;
  constexpr int NW = NT / kWave;
  constexpr int KPL = K / kWave;  // q/k elements per lane in the normalising wave
  static_assert(RPT * RG == K, "row split");
  static_assert(LPR <= kWave && kWave % LPR == 0, "lanes per row");

  __shared__ float kn[2][K];
  __shared__ float qn[2][K];
  __shared__ float kq_s[2];
  __shared__ float4 red[NW][2][LPR];

  const int nvt = a.V / VT;
  const int vt = blockIdx.x % nvt;
  const int bh = blockIdx.x / nvt;
  const int hv = bh % a.HV;
  const int b = bh / a.HV;
  const int hk = hv / (a.HV / a.H);
  const int tid = threadIdx.x;
  const int lc = tid % LPR;
  const int rg = tid / LPR;
  const int lane = tid & (kWave - 1);
  const int wid = tid / kWave;
  const int col0 = vt * VT + lc * 4;
  const bool norm_wave = wid == 0;

  // tokens of row b: [t0, t0 + Tb) of the token axis
  const int64_t t0 = a.cu ? static_cast<int64_t>(a.cu[b]) : static_cast<int64_t>(b) * a.T;
  const int Tb = a.cu ? a.cu[b + 1] - a.cu[b] : a.T;
  // The token inputs do not depend on the state row: their loads go out
  // before the slot index is waited for.
  TokIn<DT, KPL> in;
  if (Tb > 0) load_tok<DT, K, KPL>(in, a, t0, hk, hv, col0, norm_wave, lane);
  int64_t srow = a.idx ? static_cast<int64_t>(a.idx[b]) : static_cast<int64_t>(b);
  if (srow < 0 || srow >= a.n_rows) {
    if (rg == 0) {
      for (int t = 0; t < Tb; ++t) {
        const int64_t tok = t0 + t;
        store4<DT>(a.o, (tok * a.HV + hv) * a.V + col0, f4(0.f));
      }
    }
    return;
  }

  float* S = a.state + (srow * a.HV + hv) * static_cast<int64_t>(K) * a.V + col0;
  float4 s[RPT];
#pragma unroll
  for (int i = 0; i < RPT; ++i)
    s[i] = ld_stream4(S + static_cast<int64_t>(rg + i * RG) * a.V);

  for (int t = 0; t < Tb; ++t) {
    const int buf = t & 1;
    const int64_t tok = t0 + t;
    if (norm_wave) {
      float ssk = 0.f, ssq = 0.f, dot = 0.f, kf[KPL], qf[KPL];
#pragma unroll
      for (int j = 0; j < KPL; ++j) {
        kf[j] = cvt1<DT>(in.kx[j]);
        qf[j] = cvt1<DT>(in.qx[j]);
        ssk = fmaf(kf[j], kf[j], ssk);
        ssq = fmaf(qf[j], qf[j], ssq);
        dot = fmaf(kf[j], qf[j], dot);
      }
      wave_sum3(ssk, ssq, dot);
      const float rk = a.l2 ? rsqrtf(ssk + 1e-6f) : 1.f;
      const float rq = (a.l2 ? rsqrtf(ssq + 1e-6f) : 1.f) * a.scale;
#pragma unroll
      for (int j = 0; j < KPL; ++j) {
        kn[buf][lane + j * kWave] = kf[j] * rk;
        qn[buf][lane + j * kWave] = qf[j] * rq;
      }
      if (lane == 0) kq_s[buf] = dot * rk * rq;
    }
    const float4 vv = cvt4<DT>(in.v);
    const float eg = expf(cvt_any(in.g, a.g_dt));
    const float bt = cvt_any(in.beta, a.beta_dt);
    __syncthreads();

    float4 pk = f4(0.f), pq = f4(0.f);
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      const int r = rg + i * RG;
      pk = fma4(s[i], kn[buf][r], pk);
      pq = fma4(s[i], qn[buf][r], pq);
    }
#pragma unroll
    for (int off = LPR; off < kWave; off <<= 1) {
      pk.x += __shfl_xor(pk.x, off, kWave);
      pk.y += __shfl_xor(pk.y, off, kWave);
      pk.z += __shfl_xor(pk.z, off, kWave);
      pk.w += __shfl_xor(pk.w, off, kWave);
      pq.x += __shfl_xor(pq.x, off, kWave);
      pq.y += __shfl_xor(pq.y, off, kWave);
      pq.z += __shfl_xor(pq.z, off, kWave);
      pq.w += __shfl_xor(pq.w, off, kWave);
    }
    if (lane < LPR) {
      red[wid][0][lc] = pk;
      red[wid][1][lc] = pq;
    }
    __syncthreads();
    float4 kv = red[0][0][lc], sq = red[0][1][lc];
#pragma unroll
    for (int w = 1; w < NW; ++w) {
      const float4 x = red[w][0][lc], y = red[w][1][lc];
      kv.x += x.x; kv.y += x.y; kv.z += x.z; kv.w += x.w;
      sq.x += y.x; sq.y += y.y; sq.z += y.z; sq.w += y.w;
    }
    const float kq = kq_s[buf];
    if (t + 1 < Tb) load_tok<DT, K, KPL>(in, a, tok + 1, hk, hv, col0, norm_wave, lane);
    float4 d;
    d.x = bt * (vv.x - eg * kv.x);
    d.y = bt * (vv.y - eg * kv.y);
    d.z = bt * (vv.z - eg * kv.z);
    d.w = bt * (vv.w - eg * kv.w);
    if (rg == 0) {
      float4 o;
      o.x = fmaf(eg, sq.x, d.x * kq);
      o.y = fmaf(eg, sq.y, d.y * kq);
      o.z = fmaf(eg, sq.z, d.z * kq);
      o.w = fmaf(eg, sq.w, d.w * kq);
      store4<DT>(a.o, (tok * a.HV + hv) * a.V + col0, o);
    }
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      const float kr = kn[buf][rg + i * RG];
      s[i].x = fmaf(s[i].x, eg, kr * d.x);
      s[i].y = fmaf(s[i].y, eg, kr * d.y);
      s[i].z = fmaf(s[i].z, eg, kr * d.z);
      s[i].w = fmaf(s[i].w, eg, kr * d.w);
    }
  }

#pragma unroll
  for (int i = 0; i < RPT; ++i)
    st_stream4(S + static_cast<int64_t>(rg + i * RG) * a.V, s[i]);
}

// ---------------------------------------------------------------------------
// Decode GDN layer core in one launch (T = 1, H == HV, K = V = 128, bf16):
// the causal-conv update + SiLU of the packed projection (gdn_prep_kernel),
// the gated delta rule (gdn_recurrent_kernel at a 128-column tile) and the
// gated RMSNorm of the output (gated_rmsnorm_kernel), with each of those
// kernels' rounding points, so the result equals the three launches bit for
// bit.  One workgroup per (row, head) owns the head's conv channels (its q,
// k and v channels are read by no other workgroup, so the conv window is
// shifted in place), its whole K x V state slice and its output row.
struct FusedArgs {
  const uint16_t* proj;      // [B, P]: qkv (C) | z (HV V) | b (HV) | a (HV)
  uint16_t* conv_state;      // [B, 3, C], oldest first
  const uint16_t* conv_w;    // [C, 4]
  const float* a_log;        // [HV]
  const float* dt_bias;      // [HV]
  void* state;               // [n_rows, HV, K, V] float32, or fp16 (H16)
  const int32_t* idx;        // [B] or null
  const uint16_t* norm_w;    // [V]
  uint16_t* y;               // [B, HV V]
  int64_t P, n_rows;
  int C, QK, HV, zoff, boff, aoff;
  float scale, eps;
  int l2;
};

__device__ __forceinline__ float bfv(uint16_t h) { return __uint_as_float(static_cast<uint32_t>(h) << 16); }
__device__ __forceinline__ float siluf(float x) { return x / (1.f + expf(-x)); }

// Conv window of channel c: loads (phase 1), output + shift (phase 2).
struct ConvIn {
  uint16_t s0, s1, s2, x;
  uint2 w;
};
__device__ __forceinline__ ConvIn conv_load(const uint16_t* st, const uint16_t* prow, const uint16_t* conv_w, int C,
                                            int c) {
  ConvIn r;
  r.s0 = st[c];
  r.s1 = st[C + c];
  r.s2 = st[2 * C + c];
  r.x = prow[c];
  r.w = *reinterpret_cast<const uint2*>(conv_w + static_cast<int64_t>(c) * 4);
  return r;
}
__device__ __forceinline__ float conv_out(const ConvIn& r) {
  float acc = bfv(r.s0) * bfv(r.w.x & 0xffff);
  acc = fmaf(bfv(r.s1), bfv(r.w.x >> 16), acc);
  acc = fmaf(bfv(r.s2), bfv(r.w.y & 0xffff), acc);
  acc = fmaf(bfv(r.x), bfv(r.w.y >> 16), acc);
  return bfv(f32_to_bf16(siluf(acc)));
}
__device__ __forceinline__ void conv_shift(uint16_t* st, int C, int c, const ConvIn& r) {
  st[c] = r.s1;
  st[C + c] = r.s2;
  st[2 * C + c] = r.x;
}

// A thread's state rows: float4 registers (float32 state), or the loaded fp16
// words (8 bytes a row), widened where they are used -- half the registers, so
// twice the workgroups fit a CU while their conv / norm chains run.
template <bool H16, int RPT> struct StateRegs {
  float4 v[RPT];
  __device__ __forceinline__ void load(int i, const void* p, int64_t e) {
    v[i] = ld_stream4(static_cast<const float*>(p) + e);
  }
  __device__ __forceinline__ float4 get(int i) const { return v[i]; }
  __device__ __forceinline__ void opaque() {}
  __device__ __forceinline__ void store(int i, void* p, int64_t e, float4 x) {
    st_stream4(static_cast<float*>(p) + e, x);
  }
};
template <int RPT> struct StateRegs<true, RPT> {
  u32x2_t v[RPT];
  __device__ __forceinline__ void load(int i, const void* p, int64_t e) {
    v[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(static_cast<const uint16_t*>(p) + e));
  }
  __device__ __forceinline__ float4 get(int i) const {
    return make_float4(f16_to_f32(v[i].x & 0xffffu), f16_to_f32(v[i].x >> 16), f16_to_f32(v[i].y & 0xffffu),
                       f16_to_f32(v[i].y >> 16));
  }
  // the words stay the only copy: the second pass widens them again
  __device__ __forceinline__ void opaque() {
#pragma unroll
    for (int i = 0; i < RPT; ++i) asm volatile("" : "+v"(v[i]));
  }
  __device__ __forceinline__ void store(int i, void* p, int64_t e, float4 x) {
    st_stream_h4(static_cast<uint16_t*>(p) + e, x);
  }
};

// H16: the state is stored as fp16 (computed in fp32, rounded once a step on
// the store), as the reference's throughput profile keeps it.
template <int K, int V, int NT, bool H16>
__global__ void __launch_bounds__(NT) gdn_decode_fused_kernel(FusedArgs a) {
  constexpr int LPR = V / 4;
  constexpr int RG = NT / LPR;
  constexpr int RPT = K / RG;
  constexpr int NW = NT / kWave;
  constexpr int KPL = K / kWave;
  constexpr int VPL = V / kWave;
  static_assert(RPT * RG == K && LPR == 32 && NW >= 2, "tile");

  __shared__ float kn[K];
  __shared__ float qn[K];
  __shared__ float vn[V];
  __shared__ float sc[3];  // k.q, exp(g), beta
  __shared__ float4 red[NW][2][LPR];

  const int hv = blockIdx.x % a.HV;
  const int64_t b = blockIdx.x / a.HV;
  const int tid = threadIdx.x;
  const int lc = tid % LPR;
  const int rg = tid / LPR;
  const int lane = tid & (kWave - 1);
  const int wid = tid / kWave;
  const int col0 = lc * 4;
  const int64_t srow = a.idx ? static_cast<int64_t>(a.idx[b]) : b;
  const bool live = srow >= 0 && srow < a.n_rows;

  const int64_t s0 = (live ? srow * a.HV + hv : 0) * static_cast<int64_t>(K) * V + col0;
  StateRegs<H16, RPT> s;
  if (live) {
#pragma unroll
    for (int i = 0; i < RPT; ++i) s.load(i, a.state, s0 + static_cast<int64_t>(rg + i * RG) * V);
  }
  const uint16_t* prow = a.proj + b * a.P;
  uint16_t* st = a.conv_state + b * 3 * a.C;
  if (wid == 0) {
    ConvIn cq[KPL], ck[KPL];
#pragma unroll
    for (int j = 0; j < KPL; ++j) {
      const int c = hv * K + lane + j * kWave;
      cq[j] = conv_load(st, prow, a.conv_w, a.C, c);
      ck[j] = conv_load(st, prow, a.conv_w, a.C, a.QK + c);
    }
    float kf[KPL], qf[KPL], ssk = 0.f, ssq = 0.f, dot = 0.f;
#pragma unroll
    for (int j = 0; j < KPL; ++j) {
      kf[j] = conv_out(ck[j]);
      qf[j] = conv_out(cq[j]);
      ssk = fmaf(kf[j], kf[j], ssk);
      ssq = fmaf(qf[j], qf[j], ssq);
      dot = fmaf(kf[j], qf[j], dot);
    }
#pragma unroll
    for (int j = 0; j < KPL; ++j) {
      const int c = hv * K + lane + j * kWave;
      conv_shift(st, a.C, c, cq[j]);
      conv_shift(st, a.C, a.QK + c, ck[j]);
    }
    wave_sum3(ssk, ssq, dot);
    const float rk = a.l2 ? rsqrtf(ssk + 1e-6f) : 1.f;
    const float rq = (a.l2 ? rsqrtf(ssq + 1e-6f) : 1.f) * a.scale;
#pragma unroll
    for (int j = 0; j < KPL; ++j) {
      kn[lane + j * kWave] = kf[j] * rk;
      qn[lane + j * kWave] = qf[j] * rq;
    }
    if (lane == 0) sc[0] = dot * rk * rq;
  } else if (wid == 1) {
    ConvIn cv[VPL];
#pragma unroll
    for (int j = 0; j < VPL; ++j) cv[j] = conv_load(st, prow, a.conv_w, a.C, 2 * a.QK + hv * V + lane + j * kWave);
    uint16_t bb = 0, aa = 0;
    if (lane == 0) {
      bb = prow[a.boff + hv];
      aa = prow[a.aoff + hv];
    }
#pragma unroll
    for (int j = 0; j < VPL; ++j) vn[lane + j * kWave] = conv_out(cv[j]);
#pragma unroll
    for (int j = 0; j < VPL; ++j) conv_shift(st, a.C, 2 * a.QK + hv * V + lane + j * kWave, cv[j]);
    if (lane == 0) {
      const float av = bfv(aa) + a.dt_bias[hv];
      const float sp = av > 20.f ? av : log1pf(expf(av));
      sc[2] = bfv(f32_to_bf16(1.f / (1.f + expf(-bfv(bb)))));   // beta is stored in the logits' dtype
      sc[1] = expf(-expf(a.a_log[hv]) * sp);
    }
  }
  __syncthreads();

  float4 o = f4(0.f);
  if (live) {
    float4 pk = f4(0.f), pq = f4(0.f);
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      const int r = rg + i * RG;
      const float4 si = s.get(i);
      pk = fma4(si, kn[r], pk);
      pq = fma4(si, qn[r], pq);
    }
    s.opaque();
#pragma unroll
    for (int off = LPR; off < kWave; off <<= 1) {
      pk.x += __shfl_xor(pk.x, off, kWave);
      pk.y += __shfl_xor(pk.y, off, kWave);
      pk.z += __shfl_xor(pk.z, off, kWave);
      pk.w += __shfl_xor(pk.w, off, kWave);
      pq.x += __shfl_xor(pq.x, off, kWave);
      pq.y += __shfl_xor(pq.y, off, kWave);
      pq.z += __shfl_xor(pq.z, off, kWave);
      pq.w += __shfl_xor(pq.w, off, kWave);
    }
    if (lane < LPR) {
      red[wid][0][lc] = pk;
      red[wid][1][lc] = pq;
    }
  }
  __syncthreads();
  if (live) {
    float4 kv = red[0][0][lc], sq = red[0][1][lc];
#pragma unroll
    for (int w = 1; w < NW; ++w) {
      const float4 x = red[w][0][lc], z = red[w][1][lc];
      kv.x += x.x; kv.y += x.y; kv.z += x.z; kv.w += x.w;
      sq.x += z.x; sq.y += z.y; sq.z += z.z; sq.w += z.w;
    }
    const float kq = sc[0], eg = sc[1], bt = sc[2];
    const float4 vv = make_float4(vn[col0], vn[col0 + 1], vn[col0 + 2], vn[col0 + 3]);
    float4 d;
    d.x = bt * (vv.x - eg * kv.x);
    d.y = bt * (vv.y - eg * kv.y);
    d.z = bt * (vv.z - eg * kv.z);
    d.w = bt * (vv.w - eg * kv.w);
    o.x = fmaf(eg, sq.x, d.x * kq);
    o.y = fmaf(eg, sq.y, d.y * kq);
    o.z = fmaf(eg, sq.z, d.z * kq);
    o.w = fmaf(eg, sq.w, d.w * kq);
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      const float kr = kn[rg + i * RG];
      float4 x = s.get(i);
      x.x = fmaf(x.x, eg, kr * d.x);
      x.y = fmaf(x.y, eg, kr * d.y);
      x.z = fmaf(x.z, eg, kr * d.z);
      x.w = fmaf(x.w, eg, kr * d.w);
      s.store(i, a.state, s0 + static_cast<int64_t>(rg + i * RG) * V, x);
    }
  }
  if (wid != 0) return;
  // Gated RMSNorm of the bf16-rounded output row (128 values over lanes 0..31,
  // 4 each).  The sum of squares follows the 64-lane xor tree of the separate
  // kernel, whose lane v holds columns 2v, 2v+1: here lane l holds its lanes
  // 2l and 2l+1, and xor offsets 32..2 become 16..1.
  const float o0 = bfv(f32_to_bf16(o.x)), o1 = bfv(f32_to_bf16(o.y));
  const float o2 = bfv(f32_to_bf16(o.z)), o3 = bfv(f32_to_bf16(o.w));
  float x0 = o0 * o0 + o1 * o1, x1 = o2 * o2 + o3 * o3;
#pragma unroll
  for (int off = LPR / 2; off > 0; off >>= 1) {
    x0 += __shfl_xor(x0, off, kWave);
    x1 += __shfl_xor(x1, off, kWave);
  }
  if (lane >= LPR) return;
  const float r = rsqrtf((x0 + x1) / static_cast<float>(V) + a.eps);
  const uint2 wv = *reinterpret_cast<const uint2*>(a.norm_w + col0);
  const uint2 zv = *reinterpret_cast<const uint2*>(prow + a.zoff + hv * V + col0);
  const float ov[4] = {o0, o1, o2, o3};
  const uint16_t wh[4] = {static_cast<uint16_t>(wv.x & 0xffff), static_cast<uint16_t>(wv.x >> 16),
                          static_cast<uint16_t>(wv.y & 0xffff), static_cast<uint16_t>(wv.y >> 16)};
  const uint16_t zh[4] = {static_cast<uint16_t>(zv.x & 0xffff), static_cast<uint16_t>(zv.x >> 16),
                          static_cast<uint16_t>(zv.y & 0xffff), static_cast<uint16_t>(zv.y >> 16)};
  uint16_t out[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float yj = bfv(f32_to_bf16(bfv(wh[j]) * bfv(f32_to_bf16(ov[j] * r))));
    out[j] = f32_to_bf16(yj * siluf(bfv(zh[j])));
  }
  *reinterpret_cast<uint2*>(a.y + (b * a.HV + hv) * V + col0) = *reinterpret_cast<const uint2*>(out);
}

template <int K, int VT, int NT>
int launch_tile(int dt, const GdnArgs& a, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>(static_cast<int64_t>(a.B) * a.HV * (a.V / VT)));
  switch (dt) {
    case YH_F32: hipLaunchKernelGGL((gdn_recurrent_kernel<YH_F32, K, VT, NT>), grid, dim3(NT), 0, st, a); break;
    case YH_BF16: hipLaunchKernelGGL((gdn_recurrent_kernel<YH_BF16, K, VT, NT>), grid, dim3(NT), 0, st, a); break;
    case YH_F16: hipLaunchKernelGGL((gdn_recurrent_kernel<YH_F16, K, VT, NT>), grid, dim3(NT), 0, st, a); break;
    default: set_error("gdn_recurrent: unsupported q/k/v dtype %d", dt); return YH_ERR_INVALID;
  }
  YH_CHECK_LAUNCH("gdn_recurrent");
  return YH_OK;
}

// Tile choice.  YH_GDN_TILE="VT:NT" overrides the default (tuning sweeps);
// it is read on every call so a process can sweep tiles.
void pick_tile(int K, int V, int64_t B, int64_t HV, int* vt, int* nt) {
  const char* e = getenv("YH_GDN_TILE");
  int x = 0, y = 0;
  if (e && sscanf(e, "%d:%d", &x, &y) == 2 && x > 0 && V % x == 0) { *vt = x; *nt = y; return; }
  // Measured on MI355X (decode, HV = 32, dk = dv = 128): 64-column tiles of
  // 256 threads are best up to ~4096 tiles (B = 64), 512 threads above.
  if (K == 128) { *vt = 64; *nt = B * HV * (V / 64) > 4096 ? 512 : 256; }
  else { *vt = 64; *nt = 128; }
}

}  // namespace
}  // namespace yh


static int gdn_recurrent_impl(const void* q, const void* k, const void* v, const void* g,
                                const void* beta, float* state, const int32_t* state_indices,
                                const int32_t* cu_seqlens, void* o, int64_t B, int64_t T, int64_t H, int64_t HV, int64_t K,
                                int64_t V, int64_t n_state_rows, float scale, int use_qk_l2norm,
                                int qkv_dtype, int g_dtype, int beta_dtype, yh_stream_t stream) {
  using namespace yh;
  YH_CHECK_ARG(q && k && v && g && beta && state && o, "gdn_recurrent: null tensor pointer");
  YH_CHECK_ARG(B >= 0 && T >= 0 && H > 0 && HV > 0, "gdn_recurrent: bad sizes B=%lld T=%lld H=%lld HV=%lld",
               (long long)B, (long long)T, (long long)H, (long long)HV);
  YH_CHECK_ARG(HV % H == 0, "gdn_recurrent: HV (%lld) must be a multiple of H (%lld)", (long long)HV, (long long)H);
  YH_CHECK_ARG(K == 64 || K == 128, "gdn_recurrent: K must be 64 or 128 (got %lld)", (long long)K);
  YH_CHECK_ARG(V == 64 || V == 128, "gdn_recurrent: V must be 64 or 128 (got %lld)", (long long)V);
  YH_CHECK_ARG(is_float_dtype(qkv_dtype) && is_float_dtype(g_dtype) && is_float_dtype(beta_dtype),
               "gdn_recurrent: unsupported dtype codes %d/%d/%d", qkv_dtype, g_dtype, beta_dtype);
  YH_CHECK_ARG(state_indices != nullptr || n_state_rows >= B,
               "gdn_recurrent: state has %lld rows for batch %lld", (long long)n_state_rows, (long long)B);
  YH_CHECK_ARG(B * HV * 2 < (1LL << 31), "gdn_recurrent: grid too large");
  {
    // the kernel moves 16-byte state vectors and 4-element q/k/v/o groups
    const uintptr_t vec = qkv_dtype == YH_F32 ? 15 : 7;
    YH_CHECK_ARG((reinterpret_cast<uintptr_t>(state) & 15) == 0, "gdn_recurrent: state must be 16-byte aligned");
    YH_CHECK_ARG((reinterpret_cast<uintptr_t>(v) & vec) == 0 && (reinterpret_cast<uintptr_t>(o) & vec) == 0,
                 "gdn_recurrent: v and o must be aligned to 4 elements");
  }
  if (B == 0 || T == 0) return YH_OK;
  GdnArgs a{q, k, v, g, beta, state, state_indices, cu_seqlens, o,
            (int)B, (int)T, (int)H, (int)HV, (int)V, n_state_rows, scale, use_qk_l2norm ? 1 : 0,
            g_dtype, beta_dtype};
  hipStream_t st = static_cast<hipStream_t>(stream);
  int vt = 0, nt = 0;
  pick_tile((int)K, (int)V, B, HV, &vt, &nt);
  if (K == 128) {
    if (vt == 128 && nt == 256) return launch_tile<128, 128, 256>(qkv_dtype, a, st);
    if (vt == 128 && nt == 512) return launch_tile<128, 128, 512>(qkv_dtype, a, st);
    if (vt == 64 && nt == 512) return launch_tile<128, 64, 512>(qkv_dtype, a, st);
    if (vt == 64 && nt == 256) return launch_tile<128, 64, 256>(qkv_dtype, a, st);
    if (vt == 64 && nt == 128) return launch_tile<128, 64, 128>(qkv_dtype, a, st);
    if (vt == 32 && nt == 128) return launch_tile<128, 32, 128>(qkv_dtype, a, st);
    if (vt == 32 && nt == 256) return launch_tile<128, 32, 256>(qkv_dtype, a, st);
    if (vt == 32 && nt == 64) return launch_tile<128, 32, 64>(qkv_dtype, a, st);
    if (vt == 16 && nt == 64) return launch_tile<128, 16, 64>(qkv_dtype, a, st);
    return launch_tile<128, 64, 256>(qkv_dtype, a, st);
  }
  if (vt == 64 && nt == 64) return launch_tile<64, 64, 64>(qkv_dtype, a, st);
  if (vt == 32 && nt == 64) return launch_tile<64, 32, 64>(qkv_dtype, a, st);
  return launch_tile<64, 64, 128>(qkv_dtype, a, st);
}

extern "C" int yh_gdn_recurrent(const void* q, const void* k, const void* v, const void* g, const void* beta,
                                float* state, const int32_t* state_indices, void* o, int64_t B, int64_t T,
                                int64_t H, int64_t HV, int64_t K, int64_t V, int64_t n_state_rows, float scale,
                                int use_qk_l2norm, int qkv_dtype, int g_dtype, int beta_dtype, yh_stream_t stream) {
  return gdn_recurrent_impl(q, k, v, g, beta, state, state_indices, nullptr, o, B, T, H, HV, K, V, n_state_rows,
                            scale, use_qk_l2norm, qkv_dtype, g_dtype, beta_dtype, stream);
}

extern "C" int yh_gdn_recurrent_varlen(const void* q, const void* k, const void* v, const void* g,
                                       const void* beta, float* state, const int32_t* state_indices,
                                       const int32_t* cu_seqlens, void* o, int64_t n_seqs, int64_t H, int64_t HV,
                                       int64_t K, int64_t V, int64_t n_state_rows, float scale, int use_qk_l2norm,
                                       int qkv_dtype, int g_dtype, int beta_dtype, yh_stream_t stream) {
  if (cu_seqlens == nullptr) {
    yh::set_error("gdn_recurrent_varlen: cu_seqlens is required");
    return YH_ERR_INVALID;
  }
  return gdn_recurrent_impl(q, k, v, g, beta, state, state_indices, cu_seqlens, o, n_seqs, 1, H, HV, K, V,
                            n_state_rows, scale, use_qk_l2norm, qkv_dtype, g_dtype, beta_dtype, stream);
}

extern "C" int yh_gdn_decode_fused(const void* proj, int64_t proj_stride, void* conv_state, const void* conv_w,
                                   const float* a_log, const float* dt_bias, void* state, int state_dtype,
                                   const int32_t* state_indices, const void* norm_w, void* y, int64_t B, int64_t H,
                                   int64_t HV, int64_t K, int64_t V, int64_t conv_dim, int64_t z_offset,
                                   int64_t b_offset, int64_t a_offset, int64_t n_state_rows, float scale,
                                   int use_qk_l2norm, float eps, yh_stream_t stream) {
  using namespace yh;
  YH_CHECK_ARG(B >= 0 && H > 0 && HV == H, "gdn_decode_fused: needs as many value heads as key heads");
  YH_CHECK_ARG(state_dtype == YH_F32 || state_dtype == YH_F16, "gdn_decode_fused: the state is float32 or fp16");
  YH_CHECK_ARG(K == 128 && V == 128, "gdn_decode_fused: needs 128-dim heads");
  YH_CHECK_ARG(conv_dim == 2 * H * K + HV * V, "gdn_decode_fused: conv_dim must be 2 H K + HV V");
  YH_CHECK_ARG(z_offset >= conv_dim && z_offset + HV * V <= proj_stride && b_offset + HV <= proj_stride &&
                   a_offset + HV <= proj_stride && b_offset >= 0 && a_offset >= 0,
               "gdn_decode_fused: projection layout exceeds the row");
  YH_CHECK_ARG(B == 0 || (proj && conv_state && conv_w && a_log && dt_bias && state && norm_w && y),
               "gdn_decode_fused: null pointer");
  YH_CHECK_ARG(state_indices != nullptr || n_state_rows >= B, "gdn_decode_fused: state has fewer rows than the batch");
  YH_CHECK_ARG(proj_stride % 4 == 0 && z_offset % 4 == 0, "gdn_decode_fused: z rows must be 8-byte aligned");
  YH_CHECK_ARG(((reinterpret_cast<uintptr_t>(state) & 15) | (reinterpret_cast<uintptr_t>(proj) & 7) |
                (reinterpret_cast<uintptr_t>(conv_w) & 7) | (reinterpret_cast<uintptr_t>(norm_w) & 7) |
                (reinterpret_cast<uintptr_t>(y) & 7)) == 0,
               "gdn_decode_fused: misaligned pointer");
  YH_CHECK_ARG(B * HV < (1LL << 31), "gdn_decode_fused: grid too large");
  if (B == 0) return YH_OK;
  FusedArgs a{static_cast<const uint16_t*>(proj), static_cast<uint16_t*>(conv_state),
              static_cast<const uint16_t*>(conv_w), a_log, dt_bias, state, state_indices,
              static_cast<const uint16_t*>(norm_w), static_cast<uint16_t*>(y), proj_stride, n_state_rows,
              (int)conv_dim, (int)(H * K), (int)HV, (int)z_offset, (int)b_offset, (int)a_offset, scale, eps,
              use_qk_l2norm ? 1 : 0};
  // 512 threads measured fastest on MI355X at B = 128 (97 us per layer against
  // 104 / 109 us for 256 / 1024 threads)
  // fp16 state: 52.5 us per layer at B = 128 (71 VGPRs, seven waves a SIMD;
  // 61 us with the state widened in registers, 88 VGPRs, for 256, 512 or
  // 1024 threads alike; 55.8 us forced to 64 VGPRs and eight waves)
  if (state_dtype == YH_F16)
    hipLaunchKernelGGL((gdn_decode_fused_kernel<128, 128, 512, true>), dim3(static_cast<unsigned>(B * HV)), dim3(512),
                       0, static_cast<hipStream_t>(stream), a);
  else
    hipLaunchKernelGGL((gdn_decode_fused_kernel<128, 128, 512, false>), dim3(static_cast<unsigned>(B * HV)),
                       dim3(512), 0, static_cast<hipStream_t>(stream), a);
  YH_CHECK_LAUNCH("gdn_decode_fused");
  return YH_OK;
}
