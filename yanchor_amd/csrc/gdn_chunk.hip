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
// T and A = Q K^T o Gamma do not depend on the state S, so the work is split
// in two kernels:
//   chunk_prep_kernel   a persistent grid over the (chunk, value head) items
//                       of all sequences: norms, decays, K K^T and Q K^T on
//                       MFMA, the fp32 inverse T (block products on MFMA).
//                       Writes the lower 16 x 16 blocks of T diag(beta) (bf16
//                       hi + lo) and A (bf16, with the q / k scalings), and the
//                       per-token scalings, to a workspace -- 15.8 KiB per
//                       chunk and head.
//   chunk_scan_kernel   one workgroup per (sequence, value head), walking the
//                       sequence's chunks with the 128 x V fp32 state in MFMA
//                       accumulators (wave w owns value columns 16w..16w+15):
//                       Q S and W S, v_new, o, and the state update, with S
//                       and v_new never leaving registers.  The chunk inputs
//                       (which do not depend on S) are double-buffered in LDS:
//                       chunk c + 1 is staged while chunk c computes, from
//                       registers loaded during chunk c - 1; one barrier per
//                       chunk.
// Per-token L2 norms, beta and decays are diagonal factors, so products with
// the raw q / k / v tensors take exact bf16 MFMA operands and the factors go
// into the epilogues or the fp32 operand.  Products whose operands are fp32 on
// chip (T, W, the state, v_new) split each fp32 operand into bf16 hi + lo and
// accumulate 2 or 3 MFMA passes (hi.hi, hi.lo, lo.hi), which keeps the state
// path near fp32 accuracy; the output-only products Q S and A v_new take one
// pass.
#include "common.h"

namespace yh {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4v __attribute__((ext_vector_type(4)));

constexpr int kC = 64;        // chunk length
constexpr int kK = 128;       // key dim
constexpr int SKR = 136;      // bf16 row stride of 128-wide matrices (padded: conflict-free 16 B reads)
constexpr int SK64 = 72;      // bf16 row stride of 64-wide matrices
constexpr int SF = 68;        // fp32 row stride of 64-wide matrices
constexpr int kScal = 196;    // per (chunk, head) scalars: orow[64], d2[64], ek[64], e^{G_last}, pad
// T diag(beta) and A are lower triangular by 16 x 16 blocks: the workspace
// holds only the 10 lower blocks (bi, bj), bj <= bi, block lblock(bi, bj),
// each 16 x 16 row-major.
constexpr int kLB = 10;
constexpr int kLBElems = kLB * 256;
__device__ __forceinline__ int lblock(int bi, int bj) { return bi * (bi + 1) / 2 + bj; }
__device__ __forceinline__ int lblock_row(int q) { return (q >= 1) + (q >= 3) + (q >= 6); }

__device__ __forceinline__ bf16x8_t lds8(const uint16_t* p) {
  return __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(p));
}
__device__ __forceinline__ uint32_t pack2(uint16_t a, uint16_t b) {
  return static_cast<uint32_t>(a) | (static_cast<uint32_t>(b) << 16);
}
__device__ __forceinline__ float bfv(uint16_t h) { return __uint_as_float(static_cast<uint32_t>(h) << 16); }

typedef float f32x8v __attribute__((ext_vector_type(8)));

// 8 fp32 values -> bf16 hi (round to nearest even) and lo = bf16(x - hi), on
// the packed hardware conversion (v_cvt_pk_bf16_f32).
__device__ __forceinline__ void split8(const float* x, bf16x8_t& hi, bf16x8_t& lo) {
  const f32x8v v = {x[0], x[1], x[2], x[3], x[4], x[5], x[6], x[7]};
  hi = __builtin_convertvector(v, bf16x8_t);
  lo = __builtin_convertvector(v - __builtin_convertvector(hi, f32x8v), bf16x8_t);
}
__device__ __forceinline__ bf16x8_t round8v(const float* x) {
  const f32x8v v = {x[0], x[1], x[2], x[3], x[4], x[5], x[6], x[7]};
  return __builtin_convertvector(v, bf16x8_t);
}
__device__ __forceinline__ void ld8f(const float* p, float* x) {
  const float4 a = reinterpret_cast<const float4*>(p)[0], b = reinterpret_cast<const float4*>(p)[1];
  x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w; x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
}
__device__ __forceinline__ f32x4v mfma(bf16x8_t a, bf16x8_t b, f32x4v c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
// Workgroup barrier that waits only for LDS traffic (__syncthreads() also
// drains every outstanding global load, which would empty the prefetch).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// ---------------------------------------------------------------------------
// Chunk table: chunk i of the packed batch starts at token table[4i], holds
// table[4i+1] tokens and belongs to sequence table[4i+2]; sequence n owns
// chunks [cstart[n], cstart[n+1]); cstart[n_seqs] is the chunk count.
constexpr int kIdxThreads = 1024;
__global__ void __launch_bounds__(kIdxThreads) chunk_index_kernel(const int32_t* cu, int n_seqs, int32_t* table,
                                                                  int32_t* cstart, int nc_max) {
  __shared__ int32_t wsum[kIdxThreads / 64];
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  int32_t carry = 0;
  for (int base = 0; base < n_seqs; base += kIdxThreads) {
    const int i = base + threadIdx.x;
    int32_t len = 0, cnt = 0;
    if (i < n_seqs) {
      len = max(cu[i + 1] - cu[i], 0);
      cnt = (len + kC - 1) / kC;
    }
    int32_t incl = cnt;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int32_t y = __shfl_up(incl, off, 64);
      if (lane >= off) incl += y;
    }
    if (lane == 63) wsum[wid] = incl;
    __syncthreads();
    int32_t before = 0, all = 0;
    for (int w = 0; w < kIdxThreads / 64; ++w) {
      before += w < wid ? wsum[w] : 0;
      all += wsum[w];
    }
    __syncthreads();
    const int32_t first = carry + before + incl - cnt;
    if (i < n_seqs) {
      cstart[i] = first;
      for (int j = 0; j < cnt && first + j < nc_max; ++j) {
        int32_t* e = table + 4 * static_cast<int64_t>(first + j);
        e[0] = cu[i] + j * kC;
        e[1] = min(kC, len - j * kC);
        e[2] = i;
        e[3] = 0;
      }
    }
    carry += all;
  }
  if (threadIdx.x == 0) cstart[n_seqs] = min(carry, nc_max);
}

// ---------------------------------------------------------------------------
struct PrepArgs {
  const uint16_t* q;     // [total, H, K]
  const uint16_t* k;
  const void* g;         // [total, HV]
  const void* beta;
  const int32_t* table;
  const int32_t* cstart;
  uint16_t* thi;         // [nc, HV, kLBElems]  T diag(beta) (lower blocks), bf16 hi
  uint16_t* tlo;         //                     bf16 lo
  uint16_t* aqk;         // [nc, HV, kLBElems]  A (lower blocks)
  float* scal;           // [nc, HV, kScal]
  int n_seqs, H, HV;
  float scale;
  int l2, g_dt, beta_dt;
};

constexpr int kPrepThreads = 256;
constexpr int kPrepGrid = 768;  // persistent prep workgroups: three per CU on 256 CUs

struct __align__(16) PrepSmem {
  union {
    uint16_t kr[kC * SKR];  // K [t][d]          (K K^T, Q K^T)
    float t[kC * SF];       // T = (I + L)^{-1}   (after the products)
  } kt0;
  union {
    uint16_t q[kC * SKR];   // Q [t][d]          (Q K^T)
    uint16_t out[kC * SK64];  // A staged for coalesced stores (after the inversion)
  } qx;
  float l[kC * SF];         // L
  float rk[kC], rqs[kC], G[kC], beta[kC];
  float G2[kC];             // G log2(e), for the decays exp2(G2_t - G2_s)
  float gl;
};

// fp32 MFMA 16x16x4: lane l supplies A[l % 16][k] and B[k][l % 16] for the
// reduction index k it is given; D is in the 16 x 16 accumulator layout (lane
// l holds D[4 (l / 16) + e][l % 16], e = 0..3).
__device__ __forceinline__ f32x4v mfma4(float a, float b, f32x4v c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
// acc += L_im T_mj (16 x 16 blocks of the fp32 LDS matrices); MFMA s gives
// lane group g the reduction index 4 s + g.
__device__ __forceinline__ void acc_lt(f32x4v& acc, const float* l, const float* t, int i, int m, int j, int r, int g) {
#pragma unroll
  for (int s = 0; s < 4; ++s)
    acc = mfma4(l[(16 * i + r) * SF + 16 * m + 4 * s + g], t[(16 * m + 4 * s + g) * SF + 16 * j + r], acc);
}
// acc += T_ab X for X in the accumulator layout: MFMA s gives lane group g the
// reduction index 4 g + s, which is element s of the lane's own X.
__device__ __forceinline__ void acc_tx(f32x4v& acc, const float* t, int a, int b, const f32x4v& x, int r, int g) {
#pragma unroll
  for (int s = 0; s < 4; ++s) acc = mfma4(t[(16 * a + r) * SF + 16 * b + 4 * g + s], x[s], acc);
}
__device__ __forceinline__ void put_block(float* t, int i, int j, const f32x4v& v, int r, int g) {
#pragma unroll
  for (int e = 0; e < 4; ++e) t[(16 * i + 4 * g + e) * SF + 16 * j + r] = -v[e];
}

// T = (I + L)^{-1} for strictly lower triangular L (64 x 64 fp32 in LDS), by
// 16 x 16 blocks (the strictly upper blocks of T are left unwritten):
//   diagonal blocks T_bb by column-parallel forward substitution (one lane per
//   column, wave 0);
//   T_10 = -T_11 L_10 T_00 and T_32 = -T_33 L_32 T_22 (waves 0, 1);
//   the lower-left 32 x 32 block -B^{-1} C A^{-1} of the 2 x 2 block inverse,
//   with Y = C A^{-1}:  T_20 = -T_22 Y_00, T_21 = -T_22 Y_01,
//   T_30 = -(T_32 Y_00 + T_33 Y_10), T_31 = -(T_32 Y_01 + T_33 Y_11)
//   (one wave each, Y recomputed where needed).
// The block products run on fp32 MFMA.
__device__ void invert_unit_lower(const float* l, float* t) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int r = lane & 15, g = lane >> 4;
  if (w == 0) {
    const int b = lane >> 4, j = lane & 15;
    float xs[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float lr[16];
      ld8f(&l[(16 * b + i) * SF + 16 * b], lr);
      ld8f(&l[(16 * b + i) * SF + 16 * b + 8], lr + 8);
      float acc = i == j ? 1.f : 0.f;
#pragma unroll
      for (int m = 0; m < i; ++m) acc = fmaf(-lr[m], xs[m], acc);
      xs[i] = acc;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) t[(16 * b + i) * SF + 16 * b + j] = xs[i];
  }
  lds_barrier();
  if (w < 2) {
    const int i = w == 0 ? 1 : 3, j = i - 1;  // T_10, T_32
    f32x4v x = {0.f, 0.f, 0.f, 0.f}, o = {0.f, 0.f, 0.f, 0.f};
    acc_lt(x, l, t, i, j, j, r, g);
    acc_tx(o, t, i, i, x, r, g);
    put_block(t, i, j, o, r, g);
  }
  lds_barrier();
  {
    const int i = 2 + (w >> 1), j = w & 1;  // w: T_20, T_21, T_30, T_31
    f32x4v y0 = {0.f, 0.f, 0.f, 0.f}, o = {0.f, 0.f, 0.f, 0.f};
    // Y_0j = L_20 T_0j + L_21 T_1j (T_01 = 0)
    if (j == 0) acc_lt(y0, l, t, 2, 0, 0, r, g);
    acc_lt(y0, l, t, 2, 1, j, r, g);
    if (i == 2) {
      acc_tx(o, t, 2, 2, y0, r, g);
    } else {
      f32x4v y1 = {0.f, 0.f, 0.f, 0.f};  // Y_1j = L_30 T_0j + L_31 T_1j
      if (j == 0) acc_lt(y1, l, t, 3, 0, 0, r, g);
      acc_lt(y1, l, t, 3, 1, j, r, g);
      acc_tx(o, t, 3, 2, y0, r, g);
      acc_tx(o, t, 3, 3, y1, r, g);
    }
    put_block(t, i, j, o, r, g);
  }
  lds_barrier();
}

// Inputs of one (chunk, head) item, held in registers from their load (one
// item ahead) to their move into LDS.
struct PrepRegs {
  uint4 k[4], q[4];
  float g, b;
};

__device__ __forceinline__ void prep_load(PrepRegs& r, const PrepArgs& a, int item) {
  const int chunk = item / a.HV, hv = item % a.HV;
  const int64_t tok0 = a.table[4 * chunk];
  const int Lc = a.table[4 * chunk + 1];
  const int hk = hv / (a.HV / a.H);
  const int tid = threadIdx.x;
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int ci = it * kPrepThreads + tid;
    const int t = ci >> 4, d8 = (ci & 15) * 8;
    const int64_t off = ((tok0 + t) * a.H + hk) * kK + d8;
    r.k[it] = t < Lc ? *reinterpret_cast<const uint4*>(a.k + off) : make_uint4(0, 0, 0, 0);
    r.q[it] = t < Lc ? *reinterpret_cast<const uint4*>(a.q + off) : make_uint4(0, 0, 0, 0);
  }
  r.g = tid < Lc ? load_any(a.g, (tok0 + tid) * a.HV + hv, a.g_dt) : 0.f;
  r.b = tid < Lc ? load_any(a.beta, (tok0 + tid) * a.HV + hv, a.beta_dt) : 0.f;
}

// The 10 lower 16 x 16 tiles (mt, nt), nt <= mt, of K K^T and Q K^T, three
// slots per wave: (mt << 4) | nt, or -1 for an empty slot.
__device__ __forceinline__ int prep_tile(int w, int slot) {
  constexpr int8_t kTiles[4][3] = {{0x00, 0x10, 0x33}, {0x11, 0x20, 0x32}, {0x21, 0x22, -1}, {0x30, 0x31, -1}};
  return kTiles[w][slot];
}

// Persistent: workgroup b takes items b, b + gridDim.x, ... of the
// (chunk, value head) list, item = chunk * HV + head, and loads the next
// item's rows while it works on the current one (so every barrier inside
// waits for LDS traffic only).
__global__ void __launch_bounds__(kPrepThreads, 3) chunk_prep_kernel(PrepArgs a) {
  __shared__ PrepSmem sm;
  const int n_items = a.cstart[a.n_seqs] * a.HV;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, kq = (lane >> 4) * 8, rq4 = (lane >> 4) * 4;
  PrepRegs cur;
  if (static_cast<int>(blockIdx.x) < n_items) prep_load(cur, a, blockIdx.x);
  for (int item = blockIdx.x; item < n_items; item += gridDim.x) {
    const int chunk = item / a.HV, hv = item % a.HV;
    const int64_t ch = static_cast<int64_t>(chunk) * a.HV + hv;  // (chunk, head) record

    // ---- stage K, Q rows (rows t >= Lc are zero) and the gates; prefetch the next item ----
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int ci = it * kPrepThreads + tid;
      const int t = ci >> 4, d8 = (ci & 15) * 8;
      *reinterpret_cast<uint4*>(&sm.kt0.kr[t * SKR + d8]) = cur.k[it];
      *reinterpret_cast<uint4*>(&sm.qx.q[t * SKR + d8]) = cur.q[it];
    }
    if (tid < kC) {
      sm.G[tid] = cur.g;
      sm.beta[tid] = cur.b;
    }
    if (item + static_cast<int>(gridDim.x) < n_items) prep_load(cur, a, item + gridDim.x);
    lds_barrier();

    // ---- norms (4 lanes per token) and the decay scan, in the same phase as
    // the products below ----
    {  // norms: 4 lanes per token
      const int t = tid >> 2, p = tid & 3;
      float sk = 0.f, sq = 0.f;
#pragma unroll
      for (int e = 0; e < 32; e += 8) {
        const uint4 kv = *reinterpret_cast<const uint4*>(&sm.kt0.kr[t * SKR + 32 * p + e]);
        const uint4 qv = *reinterpret_cast<const uint4*>(&sm.qx.q[t * SKR + 32 * p + e]);
        const uint32_t kw[4] = {kv.x, kv.y, kv.z, kv.w}, qw[4] = {qv.x, qv.y, qv.z, qv.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float k0 = __uint_as_float(kw[j] << 16), k1 = __uint_as_float(kw[j] & 0xffff0000u);
          const float q0 = __uint_as_float(qw[j] << 16), q1 = __uint_as_float(qw[j] & 0xffff0000u);
          sk = fmaf(k0, k0, fmaf(k1, k1, sk));
          sq = fmaf(q0, q0, fmaf(q1, q1, sq));
        }
      }
      sk += __shfl_xor(sk, 1, kWave);
      sq += __shfl_xor(sq, 1, kWave);
      sk += __shfl_xor(sk, 2, kWave);
      sq += __shfl_xor(sq, 2, kWave);
      if (p == 0) {
        sm.rk[t] = a.l2 ? rsqrtf(sk + 1e-6f) : 1.f;
        sm.rqs[t] = (a.l2 ? rsqrtf(sq + 1e-6f) : 1.f) * a.scale;
      }
    }
    if (w == 0) {
      float x = sm.G[lane];
#pragma unroll
      for (int off = 1; off < kWave; off <<= 1) {
        const float y = __shfl_up(x, off, kWave);
        if (lane >= off) x += y;
      }
      sm.G[lane] = x;
      sm.G2[lane] = x * 1.4426950408889634f;
      if (lane == kWave - 1) sm.gl = x;
    }
    // ---- K K^T and Q K^T on MFMA (lower tiles only); scaled after the barrier ----
    f32x4v kk[3], qk[3];
#pragma unroll
    for (int slot = 0; slot < 3; ++slot) {
      kk[slot] = qk[slot] = f32x4v{0.f, 0.f, 0.f, 0.f};
      const int code = prep_tile(w, slot);
      if (code < 0) continue;
      const int m0 = 16 * (code >> 4), n0 = 16 * (code & 15);
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const int k0 = 32 * ks;
        const bf16x8_t b = lds8(&sm.kt0.kr[(n0 + r16) * SKR + k0 + kq]);
        kk[slot] = mfma(lds8(&sm.kt0.kr[(m0 + r16) * SKR + k0 + kq]), b, kk[slot]);
        qk[slot] = mfma(lds8(&sm.qx.q[(m0 + r16) * SKR + k0 + kq]), b, qk[slot]);
      }
    }
    lds_barrier();
    if (tid < kC) {
      const float eg = expf(sm.G[tid]);
      float* sc = a.scal + ch * kScal;
      sc[tid] = eg * sm.rqs[tid];                           // output row scale of Q S
      sc[kC + tid] = sm.rk[tid] * expf(sm.gl - sm.G[tid]);  // state-update scale of v_new row t
      sc[2 * kC + tid] = eg * sm.rk[tid];                   // row scale of K S inside W S
      if (tid == 0) sc[3 * kC] = expf(sm.gl);
    }

    // ---- scale: L (strictly lower, to LDS) and A (registers) ----
    float areg[3][4];
#pragma unroll
    for (int slot = 0; slot < 3; ++slot) {
      const int code = prep_tile(w, slot);
      if (code < 0) continue;
      const int m0 = 16 * (code >> 4), n0 = 16 * (code & 15);
      // rows t = m0 + rq4 + i (four consecutive), column s = n0 + r16
      const int s = n0 + r16, t0 = m0 + rq4;
      const float4 g2t = *reinterpret_cast<const float4*>(&sm.G2[t0]);
      const float4 bt = *reinterpret_cast<const float4*>(&sm.beta[t0]);
      const float4 rkt = *reinterpret_cast<const float4*>(&sm.rk[t0]);
      const float4 rqt = *reinterpret_cast<const float4*>(&sm.rqs[t0]);
      const float g2s = sm.G2[s], rks = sm.rk[s];
      const float g2v[4] = {g2t.x, g2t.y, g2t.z, g2t.w}, bv[4] = {bt.x, bt.y, bt.z, bt.w};
      const float rkv[4] = {rkt.x, rkt.y, rkt.z, rkt.w}, rqv[4] = {rqt.x, rqt.y, rqt.z, rqt.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = t0 + i;
        const float dec = s <= t ? exp2f(g2v[i] - g2s) : 0.f;
        sm.l[t * SF + s] = s < t ? bv[i] * rkv[i] * rks * dec * kk[slot][i] : 0.f;
        areg[slot][i] = s <= t ? rqv[i] * rks * dec * qk[slot][i] : 0.f;
      }
    }
    lds_barrier();  // K and Q are dead from here on

    invert_unit_lower(sm.l, sm.kt0.t);  // ends with a barrier

    // ---- T diag(beta) (hi / lo) straight to the workspace's lower blocks
    // (8-byte pieces); A through LDS for 16-byte stores ----
    uint16_t* thi_g = a.thi + ch * kLBElems;
    uint16_t* tlo_g = a.tlo + ch * kLBElems;
#pragma unroll
    for (int it = 0; it < 4; ++it) {  // T rows: 64 x 64, 16 elements per thread
      const int e = (it * kPrepThreads + tid) * 4;
      const int t = e >> 6, s4 = e & 63;
      if ((s4 >> 4) > (t >> 4)) continue;  // strictly upper block: not stored
      const int off = lblock(t >> 4, s4 >> 4) * 256 + (t & 15) * 16 + (s4 & 15);
      const float4 tv = *reinterpret_cast<const float4*>(&sm.kt0.t[t * SF + s4]);
      const float4 bv = *reinterpret_cast<const float4*>(&sm.beta[s4]);
      const float x[4] = {tv.x * bv.x, tv.y * bv.y, tv.z * bv.z, tv.w * bv.w};
      uint16_t h[4], lo[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        h[j] = f32_to_bf16(x[j]);
        lo[j] = f32_to_bf16(x[j] - bfv(h[j]));
      }
      *reinterpret_cast<uint2*>(thi_g + off) = make_uint2(pack2(h[0], h[1]), pack2(h[2], h[3]));
      *reinterpret_cast<uint2*>(tlo_g + off) = make_uint2(pack2(lo[0], lo[1]), pack2(lo[2], lo[3]));
    }
    uint16_t* a_s = sm.qx.out;
#pragma unroll
    for (int slot = 0; slot < 3; ++slot) {
      const int code = prep_tile(w, slot);
      if (code < 0) continue;
      const int m0 = 16 * (code >> 4), n0 = 16 * (code & 15);
#pragma unroll
      for (int i = 0; i < 4; ++i) a_s[(m0 + rq4 + i) * SK64 + n0 + r16] = f32_to_bf16(areg[slot][i]);
    }
    lds_barrier();
    uint16_t* a_g = a.aqk + ch * kLBElems;
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      const int ci = it * kPrepThreads + tid;  // 512 vectors of 8, the lower blocks' stored
      const int t = ci >> 3, s8 = (ci & 7) * 8;
      if ((s8 >> 4) <= (t >> 4))
        *reinterpret_cast<uint4*>(a_g + lblock(t >> 4, s8 >> 4) * 256 + (t & 15) * 16 + (s8 & 15)) =
            *reinterpret_cast<const uint4*>(&a_s[t * SK64 + s8]);
    }
    lds_barrier();  // the next item restages K and Q over T and the A staging
  }
}

// ---------------------------------------------------------------------------
// Sequential pass.  The state is partitioned by value column: wave w holds the
// full 128 x 16 column block S[:, 16w .. 16w+15] as eight 16 x 16 accumulator
// tiles, so every product that consumes S, K S or v_new takes it as the B
// operand straight from the wave's own registers.  The MFMA reduction index
// of a 32-deep step is visited in the order the accumulator layout provides:
// element j of quad q is row 32 ks + 4 q + j (j < 4) or 32 ks + 16 + 4 q +
// j - 4 (j >= 4), and the A operands are read in that same order: rows of
// Q, K, T diag(beta) and A from column-permuted LDS rows (one 16-byte read),
// K^T and V^T by transposing reads of the row-major K and V.  Only the
// chunk inputs go through LDS: two barriers per chunk.
struct ScanArgs {
  const uint16_t* q;     // [total, H, K]
  const uint16_t* k;
  const uint16_t* v;     // [total, HV, V]
  const uint16_t* thi;
  const uint16_t* tlo;
  const uint16_t* aqk;
  const float* scal;
  const int32_t* cu;     // [N + 1]
  const int32_t* cstart;
  const int32_t* order;  // [N] or null
  const float* h0;       // [N, HV, K, V] or null
  float* ht;             // [N, HV, K, V]
  uint16_t* o;           // [total, HV, V]
  int n_seqs, H, HV;
};

template <int NW>
struct __align__(16) ScanSmem {
  uint16_t q[kC * SKR];        // Q [t][d]
  uint16_t k[kC * SKR];        // K [t][d]  (K^T operands by transposing reads)
  uint16_t v[kC * SKR];        // V [t][v]  (V^T operands by transposing reads)
  uint16_t thi[kC * SK64];     // T diag(beta) [t][s], hi
  uint16_t tlo[kC * SK64];     // lo
  uint16_t aqk[kC * SK64];     // A [t][s]
  float orow[kC], d2[kC], ek[kC];
  float egl;
};

// Inputs of one chunk that do not depend on the state, held in registers
// between their load and their move to LDS.  NW waves.
template <int NW>
struct ChunkRegs {
  static constexpr int NT = NW * 64;
  static constexpr int kRow = kC * kK / 8 / NT;        // 16-byte vectors per thread of a 64 x 128 matrix
  static constexpr int kVec = kC * 16 * NW / 8 / NT;   // ... of the 64 x V value rows (= 2)
  static constexpr int kSq = (kLB * 32 + NT - 1) / NT;  // ... of the lower blocks of a 64 x 64 matrix
  static constexpr int kSc = (3 * kC + 1 + NT - 1) / NT;
  uint4 q[kRow], k[kRow], v[kVec];
  uint4 thi[kSq], tlo[kSq], aqk[kSq];
  float scal[kSc];
};

// chunk `chunk` of a sequence starting at token `tok0` (its j-th chunk) holds
// tokens tok0 .. tok0 + Lc - 1
template <int NW>
__device__ __forceinline__ void load_chunk(ChunkRegs<NW>& r, const ScanArgs& a, int chunk, int64_t tok0, int Lc,
                                           int hv, int hk) {
  using R = ChunkRegs<NW>;
  constexpr int NT = R::NT, V = 16 * NW;
  const int tid = threadIdx.x;
  const int64_t ch = static_cast<int64_t>(chunk) * a.HV + hv;
  // Row-major pieces: 16 lanes per 128-wide token row (2 NW per V-wide row),
  // so a wave instruction covers whole lines.
#pragma unroll
  for (int it = 0; it < R::kRow; ++it) {
    const int ci = it * NT + tid, t = ci >> 4;
    const int64_t off = ((tok0 + t) * a.H + hk) * kK + (ci & 15) * 8;
    r.q[it] = t < Lc ? *reinterpret_cast<const uint4*>(a.q + off) : make_uint4(0, 0, 0, 0);
    r.k[it] = t < Lc ? *reinterpret_cast<const uint4*>(a.k + off) : make_uint4(0, 0, 0, 0);
  }
#pragma unroll
  for (int it = 0; it < R::kVec; ++it) {
    const int ci = it * NT + tid, t = ci / (2 * NW);
    r.v[it] = t < Lc ? *reinterpret_cast<const uint4*>(a.v + ((tok0 + t) * a.HV + hv) * V + (ci % (2 * NW)) * 8)
                     : make_uint4(0, 0, 0, 0);
  }
#pragma unroll
  for (int it = 0; it < R::kSq; ++it) {
    const int ci = it * NT + tid;
    const bool in = ci < kLB * 32;
    const int64_t off = ch * kLBElems + ci * 8;
    r.thi[it] = in ? *reinterpret_cast<const uint4*>(a.thi + off) : make_uint4(0, 0, 0, 0);
    r.tlo[it] = in ? *reinterpret_cast<const uint4*>(a.tlo + off) : make_uint4(0, 0, 0, 0);
    r.aqk[it] = in ? *reinterpret_cast<const uint4*>(a.aqk + off) : make_uint4(0, 0, 0, 0);
  }
#pragma unroll
  for (int it = 0; it < R::kSc; ++it) {
    const int ci = it * NT + tid;
    r.scal[it] = ci < 3 * kC + 1 ? a.scal[ch * kScal + ci] : 0.f;
  }
}

// A-operand matrices (Q, K, T diag(beta), A) are stored in LDS with their
// columns permuted within each 32-column block so that the 8 reduction
// indices of quad q for a 32-deep step -- columns 4q + 0..3 and 16 + 4q +
// 0..3 -- sit next to each other: column c (c % 4 == 0) of block b is at
// 32 b + 8 ((c / 4) % 4) + 4 ((c % 32) / 16).  One 16-byte read then gives a
// lane its operand.
__device__ __forceinline__ int pcol(int c) {
  const int b = (c & 31) >> 2;
  return (c & ~31) + 8 * (b & 3) + 4 * (b >> 2);
}
// Store 8 consecutive columns c8 .. c8 + 7 (c8 % 8 == 0) of a row.
__device__ __forceinline__ void put8p(uint16_t* row, int c8, uint4 x) {
  *reinterpret_cast<uint2*>(row + pcol(c8)) = make_uint2(x.x, x.y);
  *reinterpret_cast<uint2*>(row + pcol(c8 + 4)) = make_uint2(x.z, x.w);
}
// The operand of quad `quad` for the 32-deep step starting at column k0 of a
// column-permuted row.
__device__ __forceinline__ bf16x8_t lds8r(const uint16_t* row, int k0, int quad) {
  return lds8(row + k0 + 8 * quad);
}
// The B operand of a 32-deep step from two accumulator tiles (rows 32 ks ..
// 32 ks + 15 and 32 ks + 16 .. 32 ks + 31), as bf16 hi / lo.
__device__ __forceinline__ void pack_b(const f32x4v& t0, const f32x4v& t1, bf16x8_t& hi, bf16x8_t& lo) {
  const float x[8] = {t0[0], t0[1], t0[2], t0[3], t1[0], t1[1], t1[2], t1[3]};
  split8(x, hi, lo);
}
// Operand of a 32-deep step whose reduction index is the ROW of a row-major
// LDS matrix m (row stride SKR): lane (i = lane % 16, quad) gets column
// c0 + i at rows k0 + 4 quad + 0..3 and k0 + 16 + 4 quad + 0..3 -- the
// permuted reduction order above -- by two ds_read_b64_tr_b16.  That
// instruction transposes within each 16-lane group: lane 4m + e receives, in
// slot j, element e of the 8 bytes addressed by lane 4j + m.  So lane
// 4j + m of the group addresses row k0 (+16) + 4 quad + j, columns
// c0 + 4m .. c0 + 4m + 3.
typedef short s16x4v __attribute__((ext_vector_type(4)));
typedef short s16x8v __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) s16x4v lds_s16x4v;
template <bool PERM>  // m's columns permuted (pcol) or plain
__device__ __forceinline__ bf16x8_t lds8t(const uint16_t* m, int k0, int c0, int lane) {
  const int i = lane & 15, quad = lane >> 4;
  const int c = c0 + 4 * (i & 3);
  const uint16_t* p = m + (k0 + 4 * quad + (i >> 2)) * SKR + (PERM ? pcol(c) : c);
  const s16x4v lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4v*)(p));
  const s16x4v hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4v*)(p + 16 * SKR));
  return __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

// One chunk's inputs from registers to an LDS buffer (A operands with
// permuted columns, V row-major, the per-token scalings).
template <int NW>
__device__ __forceinline__ void stage_chunk(ScanSmem<NW>& sm, const ChunkRegs<NW>& cur) {
  using R = ChunkRegs<NW>;
  constexpr int NT = NW * 64;
  const int tid = threadIdx.x;
#pragma unroll
  for (int it = 0; it < R::kRow; ++it) {
    const int ci = it * NT + tid, o = (ci >> 4) * SKR, c8 = (ci & 15) * 8;
    put8p(&sm.q[o], c8, cur.q[it]);
    put8p(&sm.k[o], c8, cur.k[it]);
  }
#pragma unroll
  for (int it = 0; it < R::kVec; ++it) {
    const int ci = it * NT + tid;
    *reinterpret_cast<uint4*>(&sm.v[(ci / (2 * NW)) * SKR + (ci % (2 * NW)) * 8]) = cur.v[it];
  }
#pragma unroll
  for (int it = 0; it < R::kSq; ++it) {
    const int ci = it * NT + tid;
    if (ci < kLB * 32) {  // vector ci: block q = ci / 32, row (ci % 32) / 2, half ci % 2
      const int q = ci >> 5, bi = lblock_row(q), bj = q - bi * (bi + 1) / 2;
      const int o = (16 * bi + ((ci & 31) >> 1)) * SK64, c8 = 16 * bj + 8 * (ci & 1);
      put8p(&sm.thi[o], c8, cur.thi[it]);
      put8p(&sm.tlo[o], c8, cur.tlo[it]);
      put8p(&sm.aqk[o], c8, cur.aqk[it]);
    }
  }
#pragma unroll
  for (int it = 0; it < R::kSc; ++it) {
    const int ci = it * NT + tid;
    if (ci < kC) sm.orow[ci] = cur.scal[it];
    else if (ci < 2 * kC) sm.d2[ci - kC] = cur.scal[it];
    else if (ci < 3 * kC) sm.ek[ci - 2 * kC] = cur.scal[it];
    else if (ci == 3 * kC) sm.egl = cur.scal[it];
  }
}

// Two LDS buffers: chunk c computes from one while chunk c + 1 (loaded into
// registers during chunk c - 1) is staged into the other, so one barrier per
// chunk separates them.
template <int NW>
__global__ void __launch_bounds__(NW * 64) chunk_scan_kernel(ScanArgs a) {
  using R = ChunkRegs<NW>;
  __shared__ ScanSmem<NW> smb[2];
  constexpr int V = 16 * NW;
  constexpr int NT = NW * 64;
  const int hv = blockIdx.x % a.HV;
  const int sidx = blockIdx.x / a.HV;
  const int n = a.order ? a.order[sidx] : sidx;
  const int hk = hv / (a.HV / a.H);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int r16 = lane & 15, quad = lane >> 4, rq4 = quad * 4;
  const int cs = a.cstart[n], ce = a.cstart[n + 1];
  const int64_t seq0 = a.cu[n];
  const int seqlen = a.cu[n + 1] - a.cu[n];
  const int vcol = 16 * w + r16;  // this lane's value column

  // S[dt][i] = S[16 dt + 4 quad + i][vcol]
  f32x4v S[8];
  const int64_t sbase = (static_cast<int64_t>(n) * a.HV + hv) * kK;
#pragma unroll
  for (int dt = 0; dt < 8; ++dt)
#pragma unroll
    for (int i = 0; i < 4; ++i) S[dt][i] = a.h0 ? a.h0[(sbase + 16 * dt + rq4 + i) * V + vcol] : 0.f;

  // The upper blocks of T diag(beta) and A are zero and never staged: clear
  // them once in both buffers (disjoint from every staged element).
  for (int e = tid; e < 2 * 6 * 32; e += NT) {
    const int buf = e / 192, u = (e % 192) >> 5, v = e & 31;  // upper block u: (0,1) (0,2) (0,3) (1,2) (1,3) (2,3)
    const int bi = u < 3 ? 0 : (u < 5 ? 1 : 2), bj = u < 3 ? u + 1 : (u < 5 ? u - 1 : 3);
    const int o = (16 * bi + (v >> 1)) * SK64, c8 = 16 * bj + 8 * (v & 1);
    put8p(&smb[buf].thi[o], c8, make_uint4(0, 0, 0, 0));
    put8p(&smb[buf].tlo[o], c8, make_uint4(0, 0, 0, 0));
    put8p(&smb[buf].aqk[o], c8, make_uint4(0, 0, 0, 0));
  }
  R cur;
  if (cs < ce) {
    load_chunk<NW>(cur, a, cs, seq0, min(kC, seqlen), hv, hk);
    stage_chunk<NW>(smb[0], cur);
    if (cs + 1 < ce) load_chunk<NW>(cur, a, cs + 1, seq0 + kC, min(kC, seqlen - kC), hv, hk);
    lds_barrier();
  }
  for (int c = cs; c < ce; ++c) {
    const int j = c - cs;
    const int64_t tok0 = seq0 + static_cast<int64_t>(j) * kC;
    const int Lc = min(kC, seqlen - j * kC);
    ScanSmem<NW>& sm = smb[j & 1];
    // ---- Q S (1 pass) and P = K S (2 passes), four row tiles of this column block ----
    f32x4v qs[4], ps[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) qs[mt] = ps[mt] = f32x4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      bf16x8_t bh, bl;
      pack_b(S[2 * ks], S[2 * ks + 1], bh, bl);
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const int row = (16 * mt + r16) * SKR;
        const bf16x8_t aq = lds8r(&sm.q[row], 32 * ks, quad);
        const bf16x8_t ak = lds8r(&sm.k[row], 32 * ks, quad);
        qs[mt] = mfma(aq, bh, qs[mt]);
        ps[mt] = mfma(ak, bh, ps[mt]);
        ps[mt] = mfma(ak, bl, ps[mt]);
      }
    }
    // Stage chunk c + 1 into the other buffer and prefetch chunk c + 2 while
    // the products above drain.
    if (c + 1 < ce) {
      stage_chunk<NW>(smb[(j & 1) ^ 1], cur);
      if (c + 2 < ce) load_chunk<NW>(cur, a, c + 2, tok0 + 2 * kC, min(kC, seqlen - (j + 2) * kC), hv, hk);
    }
    // ---- v_new = T diag(beta) V - T diag(beta) (diag(e^G rk) P): 2 + 3 passes, T lower triangular ----
    bf16x8_t vb[2], ph[2], pl[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      vb[ks] = lds8t<false>(sm.v, 32 * ks, 16 * w, lane);
      f32x4v p0 = ps[2 * ks], p1 = ps[2 * ks + 1];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        p0[i] *= sm.ek[32 * ks + rq4 + i];
        p1[i] *= sm.ek[32 * ks + 16 + rq4 + i];
      }
      pack_b(p0, p1, ph[ks], pl[ks]);
    }
    f32x4v vn[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      f32x4v u = {0.f, 0.f, 0.f, 0.f}, y = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        if (32 * ks <= 16 * mt + 15) {
          const int row = (16 * mt + r16) * SK64;
          const bf16x8_t th = lds8r(&sm.thi[row], 32 * ks, quad);
          const bf16x8_t tl = lds8r(&sm.tlo[row], 32 * ks, quad);
          u = mfma(th, vb[ks], u);
          u = mfma(tl, vb[ks], u);
          y = mfma(th, ph[ks], y);
          y = mfma(th, pl[ks], y);
          y = mfma(tl, ph[ks], y);
        }
      }
      vn[mt] = u - y;
    }
    // ---- S <- e^{G_last} S + K^T diag(d2) v_new (2 passes); issued before the
    // output, which the next chunk does not wait for ----
    bf16x8_t zh[2], zl[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      f32x4v z0 = vn[2 * ks], z1 = vn[2 * ks + 1];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        z0[i] *= sm.d2[32 * ks + rq4 + i];
        z1[i] *= sm.d2[32 * ks + 16 + rq4 + i];
      }
      pack_b(z0, z1, zh[ks], zl[ks]);
    }
    const float egl = sm.egl;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      f32x4v s = S[dt] * egl;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const bf16x8_t ak = lds8t<true>(sm.k, 32 * ks, 16 * dt, lane);
        s = mfma(ak, zh[ks], s);
        s = mfma(ak, zl[ks], s);
      }
      S[dt] = s;
    }
    // ---- o = diag(orow) Q S + A v_new (A lower triangular, 1 pass) ----
    bf16x8_t vnb[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const float x[8] = {vn[2 * ks][0], vn[2 * ks][1], vn[2 * ks][2], vn[2 * ks][3],
                          vn[2 * ks + 1][0], vn[2 * ks + 1][1], vn[2 * ks + 1][2], vn[2 * ks + 1][3]};
      vnb[ks] = round8v(x);
    }
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      f32x4v acc = qs[mt];
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] *= sm.orow[16 * mt + rq4 + i];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
        if (32 * ks <= 16 * mt + 15) acc = mfma(lds8r(&sm.aqk[(16 * mt + r16) * SK64], 32 * ks, quad), vnb[ks], acc);
      // Column pairs (vcol, vcol ^ 1) go out as 4-byte stores: the even lane
      // stores rows 0, 1 of its quad, the odd lane rows 2, 3.
      const bool odd = r16 & 1;
      const float y0 = __shfl_xor(odd ? acc[0] : acc[2], 1, kWave);
      const float y1 = __shfl_xor(odd ? acc[1] : acc[3], 1, kWave);
      const float2 p0 = odd ? make_float2(y0, acc[2]) : make_float2(acc[0], y0);
      const float2 p1 = odd ? make_float2(y1, acc[3]) : make_float2(acc[1], y1);
      const int t0 = 16 * mt + rq4 + (odd ? 2 : 0), c0 = vcol & ~1;
      uint32_t* o0 = reinterpret_cast<uint32_t*>(a.o + ((tok0 + t0) * a.HV + hv) * V + c0);
      uint32_t* o1 = reinterpret_cast<uint32_t*>(a.o + ((tok0 + t0 + 1) * a.HV + hv) * V + c0);
      const uint32_t w0 = pack2(f32_to_bf16(p0.x), f32_to_bf16(p0.y)), w1 = pack2(f32_to_bf16(p1.x), f32_to_bf16(p1.y));
      if (Lc == kC) {  // uniform: every chunk but a sequence's last
        *o0 = w0;
        *o1 = w1;
      } else {
        if (t0 < Lc) *o0 = w0;
        if (t0 + 1 < Lc) *o1 = w1;
      }
    }
    lds_barrier();  // chunk c + 1's buffer is complete; chunk c's may be restaged
  }
#pragma unroll
  for (int dt = 0; dt < 8; ++dt)
#pragma unroll
    for (int i = 0; i < 4; ++i) a.ht[(sbase + 16 * dt + rq4 + i) * V + vcol] = S[dt][i];
}

int64_t chunk_bound(int64_t total, int64_t n_seqs) { return total / kC + n_seqs; }

struct WsLayout {
  int64_t table, cstart, thi, tlo, aqk, scal, bytes;
};
WsLayout ws_layout(int64_t total, int64_t n_seqs, int64_t HV) {
  const int64_t nc = chunk_bound(total, n_seqs);
  auto up = [](int64_t x) { return (x + 255) / 256 * 256; };
  WsLayout l;
  l.table = 0;
  l.cstart = up(nc * 16);
  l.thi = up(l.cstart + (n_seqs + 1) * 4);
  l.tlo = l.thi + up(nc * HV * kLBElems * 2);
  l.aqk = l.tlo + up(nc * HV * kLBElems * 2);
  l.scal = l.aqk + up(nc * HV * kLBElems * 2);
  l.bytes = l.scal + up(nc * HV * kScal * 4);
  return l;
}

}  // namespace
}  // namespace yh

extern "C" int64_t yh_gdn_chunk_workspace_bytes(int64_t total_tokens, int64_t n_seqs, int64_t HV, int64_t V) {
  if (total_tokens < 0 || n_seqs < 0 || HV <= 0 || V <= 0) return 0;
  return yh::ws_layout(total_tokens, n_seqs, HV).bytes;
}

extern "C" int yh_gdn_chunk_varlen(const void* q, const void* k, const void* v, const void* g, const void* beta,
                                   const float* initial_state, float* final_state, void* o,
                                   const int32_t* cu_seqlens, const int32_t* order, int64_t n_seqs,
                                   int64_t total_tokens, int64_t H, int64_t HV, int64_t K, int64_t V, float scale,
                                   int use_qk_l2norm, int qkv_dtype, int g_dtype, int beta_dtype, void* workspace,
                                   int64_t workspace_bytes, yh_stream_t stream) {
  using namespace yh;
  YH_CHECK_ARG(n_seqs >= 0 && total_tokens >= 0 && H > 0 && HV > 0 && HV % H == 0, "gdn_chunk: bad sizes");
  YH_CHECK_ARG(K == 128, "gdn_chunk: K must be 128 (got %lld)", (long long)K);
  YH_CHECK_ARG(V == 64 || V == 128, "gdn_chunk: V must be 64 or 128 (got %lld)", (long long)V);
  YH_CHECK_ARG(qkv_dtype == YH_BF16, "gdn_chunk: q/k/v must be bfloat16");
  YH_CHECK_ARG(is_float_dtype(g_dtype) && is_float_dtype(beta_dtype), "gdn_chunk: bad gate dtypes");
  if (n_seqs == 0) return YH_OK;
  YH_CHECK_ARG(q && k && v && g && beta && final_state && o && cu_seqlens && workspace, "gdn_chunk: null pointer");
  YH_CHECK_ARG(((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v) |
                 reinterpret_cast<uintptr_t>(workspace)) & 15) == 0,
               "gdn_chunk: q/k/v and the workspace must be 16-byte aligned");
  const WsLayout l = ws_layout(total_tokens, n_seqs, HV);
  YH_CHECK_ARG(workspace_bytes >= l.bytes, "gdn_chunk: workspace of %lld bytes required", (long long)l.bytes);
  const int64_t nc = chunk_bound(total_tokens, n_seqs);
  YH_CHECK_ARG(nc < (1LL << 31) && n_seqs * HV < (1LL << 31) && HV < 65536, "gdn_chunk: grid too large");
  char* ws = static_cast<char*>(workspace);
  int32_t* table = reinterpret_cast<int32_t*>(ws + l.table);
  int32_t* cstart = reinterpret_cast<int32_t*>(ws + l.cstart);
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(chunk_index_kernel, dim3(1), dim3(kIdxThreads), 0, st, cu_seqlens, (int)n_seqs, table, cstart,
                     (int)nc);
  YH_CHECK_LAUNCH("gdn_chunk_index");
  uint16_t* thi = reinterpret_cast<uint16_t*>(ws + l.thi);
  uint16_t* tlo = reinterpret_cast<uint16_t*>(ws + l.tlo);
  uint16_t* aqk = reinterpret_cast<uint16_t*>(ws + l.aqk);
  float* scal = reinterpret_cast<float*>(ws + l.scal);
  if (nc > 0) {
    PrepArgs p{static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k), g, beta, table, cstart, thi, tlo, aqk,
               scal, (int)n_seqs, (int)H, (int)HV, scale, use_qk_l2norm ? 1 : 0, g_dtype, beta_dtype};
    const int64_t items = nc * HV;  // an upper bound: the kernel reads the chunk count
    hipLaunchKernelGGL(chunk_prep_kernel, dim3(static_cast<unsigned>(items < kPrepGrid ? items : kPrepGrid)),
                       dim3(kPrepThreads), 0, st, p);
    YH_CHECK_LAUNCH("gdn_chunk_prep");
  }
  ScanArgs s{static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k), static_cast<const uint16_t*>(v), thi, tlo,
             aqk, scal, cu_seqlens, cstart, order, initial_state, final_state, static_cast<uint16_t*>(o), (int)n_seqs,
             (int)H, (int)HV};
  const dim3 grid(static_cast<unsigned>(n_seqs * HV));
  if (V == 128)
    hipLaunchKernelGGL(chunk_scan_kernel<8>, grid, dim3(512), 0, st, s);
  else
    hipLaunchKernelGGL(chunk_scan_kernel<4>, grid, dim3(256), 0, st, s);
  YH_CHECK_LAUNCH("gdn_chunk_scan");
  return YH_OK;
}
