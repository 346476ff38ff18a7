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
// T and A = Q K^T o Gamma do not depend on the state S.  One kernel,
// chunk_fused_kernel, runs one workgroup per (sequence, value head) that walks
// the sequence's chunks.  Eight scan waves hold the 128 x V fp32 state in MFMA
// accumulators (wave w owns value columns 16w..16w+15) and run the
// state-dependent products of chunk j - 1 (Q S and K S, v_new, o, the state
// update, with S and v_new never leaving registers) while four prep waves
// (with help from the scan waves where those have time to spare) prepare chunk
// j: decays, K K^T and Q K^T with the L2 norms from their diagonals, the fp32
// inverse T on MFMA block products, A, the scalings.  Only q, k, v, the gates,
// o and the states cross HBM.
// Per-token L2 norms, beta and decays are diagonal factors, so products with
// the raw q / k / v tensors take exact bf16 MFMA operands and the factors go
// into the epilogues or the fp32 operand.  Products whose operands are fp32 on
// chip (T, the state, v_new) split each fp32 operand into bf16 hi + lo and
// accumulate 2 or 3 MFMA passes (hi.hi, hi.lo, lo.hi), which keeps the state
// path near fp32 accuracy (every pass is needed: dropping any one of them
// raises the final-state error to 3e-4 .. 1e-3 on slowly decaying inputs);
// v_new is evaluated as T diag(beta) (V - diag(e^G) K S) with the difference
// formed in fp32 and split once.  The output-only products Q S and A v_new
// take one pass.
#include "common.h"

namespace yh {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4v __attribute__((ext_vector_type(4)));

constexpr int kC = 64;        // chunk length
constexpr int kK = 128;       // key dim
constexpr int SF = 68;        // fp32 row stride of 64-wide matrices
// Lower 16 x 16 tile q (0..9, row-major over the lower triangle) lies in row
// block lblock_row(q).
__device__ __forceinline__ int lblock_row(int q) { return (q >= 1) + (q >= 3) + (q >= 6); }

// T diag(beta) and A are stored in LDS with their
// columns permuted within each 32-column block so that the 8 reduction
// indices of quad q for a 32-deep step -- columns 4q + 0..3 and 16 + 4q +
// 0..3 -- sit next to each other: column c (c % 4 == 0) of block b is at
// 32 b + 8 ((c / 4) % 4) + 4 ((c % 32) / 16).  One 16-byte read then gives a
// lane its operand.
__device__ __forceinline__ int pcol(int c) {
  const int b = (c & 31) >> 2;
  return (c & ~31) + 8 * (b & 3) + 4 * (b >> 2);
}

// LDS rows are unpadded; their 16-byte pieces are XOR-swizzled by row against
// gfx950's LDS bank conflicts (measured with the bank-conflict counter and
// with timed reads on in-bounds probes):
//   V     128 wide, transposed b64 reads:                 piece p of row r at p ^ swz_kv(r)
//   Q,K   128 wide, b128 operand reads (lds_k) and, for
//         K, transposed b64 reads (lds8t_key):            piece p of row r at p ^ swz_qk(r)
//   T,A   64 wide, columns permuted, b128 row reads:      piece p of row r at p ^ ((r / 2) % 8)
// swz_qk is the XOR-linear map of r % 16 with bit images 1, 4, 10, 9: of all
// 20160 invertible linear maps, timed on both Q / K read patterns, the
// fastest for their mix -- b128 reads twice as fast as with swz_kv (which
// leaves them 2-way conflicted) and transposed reads ~13 % faster.  (A
// 16-byte row padding gives the T / A reads 2- to 4-way conflicts.)
__device__ __forceinline__ int swz_kv(int r) { return (2 * r + ((r >> 3) & 1)) & 15; }
__device__ __forceinline__ int kvpos(int r, int p) { return r * 16 + ((p ^ swz_kv(r)) & 15); }
__device__ __forceinline__ int swz_qk(int r) { return static_cast<int>((0x6723cd89feba5410ull >> (4 * (r & 15))) & 15); }
__device__ __forceinline__ int qkpos(int r, int p) { return r * 16 + ((p ^ swz_qk(r)) & 15); }
__device__ __forceinline__ int tpos(int r, int p) { return r * 8 + ((p ^ (r >> 1)) & 7); }
// T diag(beta) hi / lo of row r: rows 0-31 take the first 8 KB (hi, then lo) and
// rows 32-63 the next 8 KB, so that rows 0-31 can be written while L's rows
// 32-63 (from byte 8704 of the same storage) are still being read.
__device__ __forceinline__ int thi(int r, int p) { return tpos(r, p) + (r >= 32 ? 256 : 0); }
__device__ __forceinline__ int tlo(int r, int p) { return tpos(r, p) + (r >= 32 ? 512 : 256); }

__device__ __forceinline__ uint32_t pack2(uint16_t a, uint16_t b) {
  return static_cast<uint32_t>(a) | (static_cast<uint32_t>(b) << 16);
}
__device__ __forceinline__ float bfv(uint16_t h) { return __uint_as_float(static_cast<uint32_t>(h) << 16); }

typedef float f32x8v __attribute__((ext_vector_type(8)));

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2v __attribute__((ext_vector_type(2)));
// Two fp32 values -> packed bf16 hi (round to nearest even) and lo = bf16(x -
// hi): one packed conversion each, hi unpacked by a shift and a mask (3
// instructions a value).
__device__ __forceinline__ void split2(float x0, float x1, uint32_t& hi, uint32_t& lo) {
  hi = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2v){x0, x1}, bf16x2_t));
  const f32x2v r = {x0 - __uint_as_float(hi << 16), x1 - __uint_as_float(hi & 0xffff0000u)};
  lo = __builtin_bit_cast(uint32_t, __builtin_convertvector(r, bf16x2_t));
}
// 8 fp32 values -> bf16 hi and lo.
__device__ __forceinline__ void split8(const float* x, bf16x8_t& hi, bf16x8_t& lo) {
  uint32_t h[4], l[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) split2(x[2 * j], x[2 * j + 1], h[j], l[j]);
  hi = __builtin_bit_cast(bf16x8_t, make_uint4(h[0], h[1], h[2], h[3]));
  lo = __builtin_bit_cast(bf16x8_t, make_uint4(l[0], l[1], l[2], l[3]));
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
// drains every outstanding vector memory operation).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// s_waitcnt vmcnt(0) as a compiler builtin (gfx9 encoding: vmcnt in bits
// 3:0 and 15:14 all zero, expcnt 7 and lgkmcnt 15 -- no wait on those).  The
// compiler's wait pass sees it, so the state loads before the chunk loop count
// as complete after it and the pass places no wait at the loop head.
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// A gate element from the aligned 32-bit word that holds it (a 16-bit
// element shares its word with a neighbour; the word never leaves the
// element's page): the words are copied into LDS with the q / k rows and
// converted where they are used.
__device__ __forceinline__ float gate_value(uint32_t w, int64_t i, int dt) {
  if (dt == YH_F32) return __uint_as_float(w);
  const uint32_t h = (i & 1) ? (w >> 16) : (w & 0xffffu);
  return dt == YH_BF16 ? __uint_as_float(h << 16) : f16_to_f32(static_cast<uint16_t>(h));
}

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

typedef __attribute__((address_space(3))) void lds_void;
typedef unsigned int u32x4n __attribute__((ext_vector_type(4)));
// One copy instruction (16 or 4 bytes a lane) into LDS at `lds` (wave-uniform)
// + 16 l (4 l).  Written as inline assembly: the compiler's wait insertion
// treats a copy it can see as a write to every LDS byte and would make each
// later LDS read of the other buffer wait for it; the code waits for the copy
// itself (vmcnt, then a barrier) before any wave reads what it wrote.
// The wait for those copies, as inline assembly too, so that the compiler
// (which does not see the copies) cannot drop it.
__device__ __forceinline__ void dma_wait() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
// (The LDS offset is the low half of the flat address of an LDS object.)
// The 16-byte copies (q, k, v rows, read once) are nontemporal.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, const void* lds, int voff) {
  const unsigned m0v = __builtin_amdgcn_readfirstlane(static_cast<unsigned>(reinterpret_cast<uintptr_t>(lds)));
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen nt lds" ::"s"(m0v), "v"(voff), "s"(r)
               : "memory", "m0");
}
__device__ __forceinline__ void dma4(__amdgpu_buffer_rsrc_t r, const void* lds, int voff) {
  const unsigned m0v = __builtin_amdgcn_readfirstlane(static_cast<unsigned>(reinterpret_cast<uintptr_t>(lds)));
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dword %1, %2, 0 offen lds" ::"s"(m0v), "v"(voff), "s"(r)
               : "memory", "m0");
}
// The B operand of a 32-deep step from two accumulator tiles (rows 32 ks ..
// 32 ks + 15 and 32 ks + 16 .. 32 ks + 31), as bf16 hi / lo.
__device__ __forceinline__ void pack_b(const f32x4v& t0, const f32x4v& t1, bf16x8_t& hi, bf16x8_t& lo) {
  const float x[8] = {t0[0], t0[1], t0[2], t0[3], t1[0], t1[1], t1[2], t1[3]};
  split8(x, hi, lo);
}
// The A operand of quad `quad` for the 32-deep step ks of row r: one b128
// read of a column-permuted row (T / A at tpos) ...
__device__ __forceinline__ bf16x8_t lds_t(const uint4* m, int r, int ks, int quad) {
  return __builtin_bit_cast(bf16x8_t, m[tpos(r, 4 * ks + quad)]);
}
// ... or of a plain Q / K row (qkpos) when the reduction index is the key
// dimension.  The key dimension is relabelled so that the 8 reduction slots of
// quad `quad` in step ks are the 8 consecutive columns 32 ks + 8 quad .. + 7:
// the state register S[dt][i] of lane (quad, column) holds key row
// 32 (dt / 2) + 8 quad + 4 (dt % 2) + i, so pack_b(S[2 ks], S[2 ks + 1]) lines
// up with this read.
__device__ __forceinline__ bf16x8_t lds_k(const uint4* m, int r, int ks, int quad) {
  return __builtin_bit_cast(bf16x8_t, m[qkpos(r, 4 * ks + quad)]);
}
__device__ __forceinline__ int state_row(int dt, int quad, int i) { return 32 * (dt >> 1) + 8 * quad + 4 * (dt & 1) + i; }
// Operand of a 32-deep step whose reduction index is the ROW of a plain
// LDS matrix m (K or V at kvpos): lane (i = lane % 16, quad) gets column
// c0 + i at rows k0 + 4 quad + 0..3 and k0 + 16 + 4 quad + 0..3 -- the
// permuted reduction order above -- by two ds_read_b64_tr_b16.  That
// instruction transposes within each 16-lane group: lane 4m + e receives, in
// slot j, element e of the 8 bytes addressed by lane 4j + m.  So lane
// 4j + m of the group addresses row k0 (+16) + 4 quad + j, columns
// c0 + 4m .. c0 + 4m + 3 (half m % 2 of piece c0 / 8 + m / 2).
typedef short s16x4v __attribute__((ext_vector_type(4)));
typedef short s16x8v __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) s16x4v lds_s16x4v;
__device__ __forceinline__ bf16x8_t lds8t(const uint4* m, int k0, int c0, int lane) {
  const int i = lane & 15, quad = lane >> 4, mm = i & 3;
  const int r = k0 + 4 * quad + (i >> 2), pc = (c0 >> 3) + (mm >> 1);
  const uint2* p0 = reinterpret_cast<const uint2*>(&m[kvpos(r, pc)]) + (mm & 1);
  const uint2* p1 = reinterpret_cast<const uint2*>(&m[kvpos(r + 16, pc)]) + (mm & 1);
  const s16x4v lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4v*)(p0));
  const s16x4v hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4v*)(p1));
  return __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}
// The same transposed read of K for the state rows of accumulator tile dt
// (state_row order): lane i = 4 mm + e of a 16-lane group gets key column
// 32 (dt / 2) + 4 (dt % 2) + 8 mm + e, so addressing lane 4 j + mm reads the
// 8 bytes at columns 32 (dt / 2) + 4 (dt % 2) + 8 mm .. + 3 -- piece
// 4 (dt / 2) + mm, half dt % 2 -- of row k0 (+ 16) + 4 quad + j.
__device__ __forceinline__ bf16x8_t lds8t_key(const uint4* m, int k0, int dt, int lane) {
  const int i = lane & 15, quad = lane >> 4;
  const int r = k0 + 4 * quad + (i >> 2), pc = 4 * (dt >> 1) + (i & 3);
  const uint2* p0 = reinterpret_cast<const uint2*>(&m[qkpos(r, pc)]) + (dt & 1);
  const uint2* p1 = reinterpret_cast<const uint2*>(&m[qkpos(r + 16, pc)]) + (dt & 1);
  const s16x4v lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4v*)(p0));
  const s16x4v hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4v*)(p1));
  return __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

// ---------------------------------------------------------------------------
// chunk_fused_kernel.  Iteration j prepares chunk j in LDS buffer Y from the
// q / k rows already there, and runs the state-dependent products of chunk
// j - 1 from buffer X:
//   P1  L2 norms, decay cumsum, K K^T / Q K^T of j,
//       copy v of j into Y (over the previous T)       | Q S, K S of j - 1
//   P2  L (fp32, over Y's T rows), A, scalings of j     | v_new of j - 1; copy q of j + 1 into X
//   P3a the inverse's diagonal blocks (wave 0), T fp32
//       over X's V rows (dead since P2)                 | state update of j - 1
//   P3b its first off-diagonal level (waves 0, 1)       | output of j - 1 (stored);
//                                                         copy k and gates of j + 1 into X
//   P3c its second level (waves 0..3); T diag(beta)
//       rows 0-31 as bf16 hi / lo (waves 4..7)
//   P4  T diag(beta) rows 32-63 as hi / lo; wait for the copies
// Six barriers per chunk.  Copies go through the buffer units straight into
// LDS (dma16 / dma4), in the swizzled layouts, each issued in a phase where
// its target is dead and by waves with time to spare there.
struct FusedArgs {
  const uint16_t* q;     // [total, H, K]
  const uint16_t* k;
  const uint16_t* v;     // [total, HV, V]
  const void* g;         // [total, HV]
  const void* beta;
  const int32_t* cu;     // [N + 1]
  const int32_t* order;  // [N] or null
  const float* h0;       // [N, HV, K, V] or null
  float* ht;             // [N, HV, K, V]
  uint16_t* o;           // [total, HV, V]
  int n_seqs, H, HV;
  float scale;
  int l2, g_dt, beta_dt;
};

struct __align__(16) FBuf {
  uint4 q[kC * 16];  // Q [t][d] at qkpos
  uint4 k[kC * 16];  // K [t][d] at qkpos
  union {
    uint4 v[kC * 16];  // V [t][v] at kvpos
    float t[kC * SF];  // T (fp32) of the chunk prepared while this one is scanned
  } vt;
  union {
    uint4 p[kC * 16];    // T diag(beta) [t][s] as bf16 hi and lo at tpos (thi / tlo)
    float l[kC * SF];    // L (fp32) while this chunk is prepared
  } tt;
  uint4 aqk[kC * 8];     // A [t][s] at tpos
  float scal[4 * kC];    // orow [0, 64), d2 [64, 128), -ek [128, 192), e^{G_last} [192]
  uint32_t gw[2 * kC];   // the words holding g [0, 64) and beta [64, 128) of each token
};
struct __align__(16) FPrep {
  float rk[kC], rqs[kC], G[kC], G2[kC], beta[kC];
  float gl;
};
static_assert(2 * sizeof(FBuf) + sizeof(FPrep) <= 160 * 1024, "fused chunk LDS");

// The 64 rows of a chunk of one bf16 matrix (row stride `stride` bytes in
// global memory, `pieces` 16-byte pieces a row) into LDS rows of 16 pieces,
// piece p of row r at p ^ swz_qk(r) (QK) or p ^ swz_kv(r), by waves W0 ..
// W0 + NWV - 1, one copy instruction per 4 rows.  `r` covers the chunk's
// valid rows: rows past it and pieces past `pieces` arrive as zeros.
template <bool QK, int W0, int NWV>
__device__ __forceinline__ void dma_rows(uint4* dst, __amdgpu_buffer_rsrc_t r, int stride, int pieces) {
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (w < W0 || w >= W0 + NWV) return;
  for (int bl = w - W0; bl < 16; bl += NWV) {
    const int row = 4 * bl + (lane >> 4);
    const int lp = ((lane & 15) ^ (QK ? swz_qk(row) : swz_kv(row))) & 15;
    dma16(r, &dst[64 * bl], lp < pieces ? row * stride + lp * 16 : 0x7ffffff0);
  }
}
// Buffer resource over the Lc valid rows of a chunk that starts at `base`.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t chunk_rsrc(const uint16_t* base, int Lc, int stride, int row_bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(base), 0, (Lc - 1) * stride + row_bytes, 0x00020000);
}
template <int W0, int NWV>
__device__ __forceinline__ void fdma_q(FBuf& b, const FusedArgs& a, int64_t tok0, int Lc, int hk) {
  dma_rows<true, W0, NWV>(b.q, chunk_rsrc(a.q + (tok0 * a.H + hk) * kK, Lc, a.H * kK * 2, kK * 2), a.H * kK * 2, 16);
}
template <int W0, int NWV>
__device__ __forceinline__ void fdma_k(FBuf& b, const FusedArgs& a, int64_t tok0, int Lc, int hk) {
  dma_rows<true, W0, NWV>(b.k, chunk_rsrc(a.k + (tok0 * a.H + hk) * kK, Lc, a.H * kK * 2, kK * 2), a.H * kK * 2, 16);
}
template <int V, int W0, int NWV>
__device__ __forceinline__ void fdma_v(FBuf& b, const FusedArgs& a, int64_t tok0, int Lc, int hv) {
  dma_rows<false, W0, NWV>(b.vt.v, chunk_rsrc(a.v + (tok0 * a.HV + hv) * V, Lc, a.HV * V * 2, V * 2), a.HV * V * 2,
                           V / 8);
}
// The gate words of chunk (tok0, Lc), by waves W0 (g) and W0 + 1 (beta); rows
// past Lc repeat the last row's words (masked on use).
template <int W0>
__device__ __forceinline__ void fdma_g(FBuf& b, const FusedArgs& a, int64_t tok0, int Lc, int hv) {
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) - W0;
  if (w == 0 || w == 1) {
    const void* src = w == 0 ? a.g : a.beta;
    const int dt = w == 0 ? a.g_dt : a.beta_dt;
    const int64_t i = (tok0 + (lane < Lc ? lane : Lc - 1)) * a.HV + hv;
    const int off = static_cast<int>(dt == YH_F32 ? i * 4 : (i * 2) & ~static_cast<int64_t>(3));
    const __amdgpu_buffer_rsrc_t rg = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(src), 0, 0x7fffffff,
                                                                        0x00020000);
    dma4(rg, &b.gw[64 * w], off);
  }
}


// T = (I + L)^{-1} for strictly lower triangular L (64 x 64 fp32 in LDS, row
// stride SF), by 16 x 16 blocks, in three barrier-free pieces so that the
// state-dependent products fill the phases between them (the strictly upper
// blocks of T are left unwritten):
//   inv_diag    diagonal blocks T_bb by column-parallel forward substitution
//               (one lane per column, one wave);
//   inv_level1  T_10 = -T_11 L_10 T_00 and T_32 = -T_33 L_32 T_22;
//   inv_level2  the lower-left 32 x 32 block -B^{-1} C A^{-1} of the 2 x 2
//               block inverse, with Y = C A^{-1}: T_20 = -T_22 Y_00,
//               T_21 = -T_22 Y_01, T_30 = -(T_32 Y_00 + T_33 Y_10),
//               T_31 = -(T_32 Y_01 + T_33 Y_11) (one wave each, Y recomputed
//               where needed; _pre / _fin split at the first level).
// The block products run on fp32 MFMA.
__device__ __forceinline__ void inv_diag(const float* l, float* t) {  // one wave
  const int lane = threadIdx.x & 63;
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
__device__ __forceinline__ void inv_level1(const float* l, float* t, int u) {  // u = 0, 1: T_10, T_32
  const int lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
  const int i = u == 0 ? 1 : 3, j = i - 1;
  f32x4v x = {0.f, 0.f, 0.f, 0.f}, o = {0.f, 0.f, 0.f, 0.f};
  acc_lt(x, l, t, i, j, j, r, g);
  acc_tx(o, t, i, i, x, r, g);
  put_block(t, i, j, o, r, g);
}
// The second level in two parts, so that the products that need only the
// diagonal blocks run a phase earlier: inv_level2_pre forms Y_0j's (and, for
// block row 3, Y_1j's) terms with T_00 or T_11, inv_level2_fin adds the terms
// with T_10 and forms the block.
__device__ __forceinline__ void inv_level2_pre(const float* l, const float* t, int u, f32x4v& y0, f32x4v& y1) {
  const int lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
  const int i = 2 + (u >> 1), j = u & 1;
  y0 = y1 = f32x4v{0.f, 0.f, 0.f, 0.f};
  acc_lt(y0, l, t, 2, j, j, r, g);  // L_20 T_00 or L_21 T_11
  if (i == 3) acc_lt(y1, l, t, 3, j, j, r, g);
}
__device__ __forceinline__ void inv_level2_fin(const float* l, float* t, int u, f32x4v& y0, f32x4v& y1) {
  const int lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
  const int i = 2 + (u >> 1), j = u & 1;
  f32x4v o = {0.f, 0.f, 0.f, 0.f};
  if (j == 0) {
    acc_lt(y0, l, t, 2, 1, 0, r, g);  // + L_21 T_10
    if (i == 3) acc_lt(y1, l, t, 3, 1, 0, r, g);
  }
  if (i == 2) {
    acc_tx(o, t, 2, 2, y0, r, g);
  } else {
    acc_tx(o, t, 3, 2, y0, r, g);
    acc_tx(o, t, 3, 3, y1, r, g);
  }
  put_block(t, i, j, o, r, g);
}

// Elements e .. e + 3 (row e / 64) of T diag(beta) as bf16 hi / lo; blocks
// the products read as zeros are written as zeros.
__device__ __forceinline__ void t_hilo(FBuf& Y, const float* tf, const FPrep& pp, int e) {
  const int t = e >> 6, s4 = e & 63;
  const int bi = t >> 4, bj = s4 >> 4;
  const bool keep = bj <= bi;                                      // lower block
  const bool zero = (bi == 0 && bj == 1) || (bi == 2 && bj == 3);  // read as zeros by the products
  if (keep || zero) {
    uint32_t h[2] = {0u, 0u}, lo[2] = {0u, 0u};
    if (keep) {
      const float4 x = *reinterpret_cast<const float4*>(&tf[t * SF + s4]);
      const float4 bv = *reinterpret_cast<const float4*>(&pp.beta[s4]);
      split2(x.x * bv.x, x.y * bv.y, h[0], lo[0]);
      split2(x.z * bv.z, x.w * bv.w, h[1], lo[1]);
    }
    const int pc = pcol(s4);
    reinterpret_cast<uint2*>(&Y.tt.p[thi(t, pc >> 3)])[(pc >> 2) & 1] = make_uint2(h[0], h[1]);
    reinterpret_cast<uint2*>(&Y.tt.p[tlo(t, pc >> 3)])[(pc >> 2) & 1] = make_uint2(lo[0], lo[1]);
  }
}

// Inclusive prefix sum over the 64 lanes: DPP row shifts by 1, 2, 4, 8 within
// each 16-lane row, then the row broadcasts of lanes 15 and 31.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp0(float v) {  // lanes without a source (or outside ROW_MASK) get 0
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xf, true));
}
__device__ __forceinline__ float wave_prefix_sum(float x) {
  x += dpp0<0x111, 0xf>(x);  // row_shr:1
  x += dpp0<0x112, 0xf>(x);  // row_shr:2
  x += dpp0<0x114, 0xf>(x);  // row_shr:4
  x += dpp0<0x118, 0xf>(x);  // row_shr:8
  x += dpp0<0x142, 0xa>(x);  // row_bcast:15 into rows 1 and 3
  x += dpp0<0x143, 0xc>(x);  // row_bcast:31 into rows 2 and 3
  return x;
}

constexpr int kNP = 4;  // prep waves

// K K^T / Q K^T tile ti (0..9, lower 16 x 16 blocks of the chunk) of Y,
// transposed: [s][t] = k_s . k_t and k_s . q_t (lane: t, elements: 4 s).  A
// diagonal tile (ti = 0, 2, 5, 9) also yields the squared L2 norms of its 16
// keys (its diagonal) and, with Q Q^T on the same reads, of its queries: the
// lane holding [t][t] writes rk[t] and rqs[t] (scale included).
__device__ __forceinline__ void kq_tile(const FBuf& Y, FPrep& pp, const FusedArgs& a, int ti, f32x4v& kk, f32x4v& qk,
                                        int r16, int quad) {
  kk = qk = f32x4v{0.f, 0.f, 0.f, 0.f};
  const int mt = lblock_row(ti), m0 = 16 * mt, n0 = 16 * (ti - mt * (mt + 1) / 2);
  const bool diag = m0 == n0;  // uniform
  f32x4v qq = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    const bf16x8_t as = lds_k(Y.k, n0 + r16, ks, quad);
    const bf16x8_t bq = lds_k(Y.q, m0 + r16, ks, quad);
    kk = mfma(as, lds_k(Y.k, m0 + r16, ks, quad), kk);
    qk = mfma(as, bq, qk);
    if (diag) qq = mfma(bq, bq, qq);
  }
  if (diag && quad == (r16 >> 2)) {
    const int e = r16 & 3;
    const float k2 = e == 0 ? kk[0] : e == 1 ? kk[1] : e == 2 ? kk[2] : kk[3];
    const float q2 = e == 0 ? qq[0] : e == 1 ? qq[1] : e == 2 ? qq[2] : qq[3];
    pp.rk[m0 + r16] = a.l2 ? rsqrtf(k2 + 1e-6f) : 1.f;
    pp.rqs[m0 + r16] = (a.l2 ? rsqrtf(q2 + 1e-6f) : 1.f) * a.scale;
  }
}
// ... and its L and A entries: row t = m0 + r16, columns s = n0 + 4 quad + 0..3
// (one 16-byte L write and one 8-byte A write); the decay exponents G_t - G_s
// are <= 0 for s <= t.
__device__ __forceinline__ void la_tile(FBuf& Y, const FPrep& pp, int ti, const f32x4v& kk, const f32x4v& qk, int r16,
                                        int quad) {
  const int mt = lblock_row(ti), m0 = 16 * mt, n0 = 16 * (ti - mt * (mt + 1) / 2);
  const int t = m0 + r16, s0 = n0 + 4 * quad;
  const float g2t = pp.G2[t], lt = pp.beta[t] * pp.rk[t], at = pp.rqs[t];
  const float4 g2s = *reinterpret_cast<const float4*>(&pp.G2[s0]);
  const float4 rks = *reinterpret_cast<const float4*>(&pp.rk[s0]);
  const float g2v[4] = {g2s.x, g2s.y, g2s.z, g2s.w}, rkv[4] = {rks.x, rks.y, rks.z, rks.w};
  float lv[4], av[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int s = s0 + e;
    const float dec = s <= t ? __builtin_amdgcn_exp2f(g2t - g2v[e]) * rkv[e] : 0.f;
    lv[e] = s < t ? lt * dec * kk[e] : 0.f;
    av[e] = at * dec * qk[e];
  }
  *reinterpret_cast<float4*>(&Y.tt.l[t * SF + s0]) = make_float4(lv[0], lv[1], lv[2], lv[3]);
  const int pc = pcol(s0);
  const f32x4v af = {av[0], av[1], av[2], av[3]};
  typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
  reinterpret_cast<uint2*>(&Y.aqk[tpos(t, pc >> 3)])[(pc >> 2) & 1] =
      __builtin_bit_cast(uint2, __builtin_convertvector(af, bf16x4_t));
}
// Both roles run one iteration per chunk (plus one) with the same six
// workgroup barriers, each role in its own loop: the state and the scan's
// products are live on the scan waves only, the prep tiles on the prep waves.

// Scan waves 0 .. NW - 1: value columns 16 w .. 16 w + 15, the state in
// registers.  P1 Q S, K S of j - 1; tile w of j (waves 0-3) | P2 v_new; L, A
// of tile w; copy v of j into Y (waves 0-3) | P3a state update | P3b output,
// staged; copy k of j + 1 into X | P3c its stores; T diag(beta)
// rows 0-31 of j as bf16 hi / lo | P4 rows 32-63.
template <int NW, bool PREP, bool SCAN>
__device__ __forceinline__ void scan_iter(const FusedArgs& a, FBuf* __restrict__ Yp, FBuf* __restrict__ Xp,
                                          FPrep& pp, f32x4v (&S)[8], int j, int nch, int64_t seq0, int seqlen,
                                          int hv, int hk) {
  FBuf& Y = *Yp;
  FBuf& X = *Xp;
  constexpr int V = 16 * NW, NS = NW * 64;
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));  // offsets computed where used, not hoisted out of the chunk loop
  const int lane = tid & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r16 = lane & 15, quad = lane >> 4, rq4 = quad * 4;
  const int64_t toks = seq0 + static_cast<int64_t>(j - 1) * kC;
  const int Ls = min(kC, seqlen - (j - 1) * kC);

  // ---- P1 ----
  f32x4v kk, qk;
  if constexpr (PREP)
    if (w < 4) kq_tile(Y, pp, a, w, kk, qk, r16, quad);  // tile w of chunk j (the first wave of each SIMD)
  f32x4v qs[4], ps[4];
  if constexpr (SCAN) {
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) qs[mt] = ps[mt] = f32x4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      bf16x8_t bh, bl;
      pack_b(S[2 * ks], S[2 * ks + 1], bh, bl);
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const bf16x8_t aq = lds_k(X.q, 16 * mt + r16, ks, quad);
        const bf16x8_t ak = lds_k(X.k, 16 * mt + r16, ks, quad);
        qs[mt] = mfma(bh, aq, qs[mt]);  // (Q S)^T: lane (token, quad) holds 4 value columns
        ps[mt] = mfma(ak, bh, ps[mt]);
        ps[mt] = mfma(ak, bl, ps[mt]);
      }
    }
  }
  lds_barrier();

  // ---- P2 ----
  if constexpr (PREP) {
    if (w < 4) la_tile(Y, pp, w, kk, qk, r16, quad);
    fdma_v<V, 0, 4>(Y, a, seq0 + static_cast<int64_t>(j) * kC, min(kC, seqlen - j * kC), hv);  // v of j into Y (over the previous T)
  }
  f32x4v vn[4];
  if constexpr (SCAN) {
    // v_new = T diag(beta) (V - W' S), W' S = diag(e^G rk) K S: D = V + (-scaled K S)
    // in fp32 (V from its bf16 rows, in the accumulator row order), split once
    // into bf16 hi / lo, then three passes T_hi D_hi + T_hi D_lo + T_lo D_hi
    bf16x8_t dh[2], dl[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const uint4 vw = __builtin_bit_cast(uint4, lds8t(X.vt.v, 32 * ks, 16 * w, lane));
      const uint32_t vv[4] = {vw.x, vw.y, vw.z, vw.w};
      const f32x4v p0 = ps[2 * ks], p1 = ps[2 * ks + 1];
      float d[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t w0 = vv[i >> 1], w1 = vv[2 + (i >> 1)];
        const float v0 = __uint_as_float((i & 1) ? (w0 & 0xffff0000u) : (w0 << 16));
        const float v1 = __uint_as_float((i & 1) ? (w1 & 0xffff0000u) : (w1 << 16));
        d[i] = fmaf(p0[i], X.scal[2 * kC + 32 * ks + rq4 + i], v0);
        d[4 + i] = fmaf(p1[i], X.scal[2 * kC + 32 * ks + 16 + rq4 + i], v1);
      }
      split8(d, dh[ks], dl[ks]);
    }
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      f32x4v u = {0.f, 0.f, 0.f, 0.f}, y = {0.f, 0.f, 0.f, 0.f};  // two chains: the MFMA latency stays hidden
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        if (32 * ks <= 16 * mt + 15) {
          const bf16x8_t th = __builtin_bit_cast(bf16x8_t, X.tt.p[thi(16 * mt + r16, 4 * ks + quad)]);
          const bf16x8_t tl = __builtin_bit_cast(bf16x8_t, X.tt.p[tlo(16 * mt + r16, 4 * ks + quad)]);
          u = mfma(th, dh[ks], u);
          u = mfma(th, dl[ks], u);
          y = mfma(tl, dh[ks], y);
        }
      }
      vn[mt] = u + y;
    }
  }
  lds_barrier();

  // ---- P3a ----
  if constexpr (SCAN) {
    bf16x8_t zh[2], zl[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      f32x4v z0 = vn[2 * ks], z1 = vn[2 * ks + 1];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        z0[i] *= X.scal[kC + 32 * ks + rq4 + i];
        z1[i] *= X.scal[kC + 32 * ks + 16 + rq4 + i];
      }
      pack_b(z0, z1, zh[ks], zl[ks]);
    }
    const float egl = X.scal[3 * kC];
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      f32x4v sv = S[dt] * egl;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const bf16x8_t ak = lds8t_key(X.k, 32 * ks, dt, lane);
        sv = mfma(ak, zh[ks], sv);
        sv = mfma(ak, zl[ks], sv);
      }
      S[dt] = sv;
    }
  }
  lds_barrier();

  // ---- P3b: o^T = (Q S)^T diag(orow) + v_new^T A^T: lane (r16, quad) holds
  // value columns 16 w + 4 quad .. + 3 of token 16 mt + r16.  The tile is staged
  // row-major in X's T hi / lo storage (read for the last time in P2), 16-byte
  // piece p of row t at p ^ (t % 16), and stored as whole rows in P3c ----
  if constexpr (SCAN) {
    bf16x8_t vnb[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const float x[8] = {vn[2 * ks][0], vn[2 * ks][1], vn[2 * ks][2], vn[2 * ks][3],
                          vn[2 * ks + 1][0], vn[2 * ks + 1][1], vn[2 * ks + 1][2], vn[2 * ks + 1][3]};
      vnb[ks] = round8v(x);
    }
    typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const int t = 16 * mt + r16;
      f32x4v acc = qs[mt] * X.scal[t];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
        if (32 * ks <= 16 * mt + 15) acc = mfma(vnb[ks], lds_t(X.aqk, t, ks, quad), acc);
      uint2* st = reinterpret_cast<uint2*>(&X.tt.p[t * (V / 8) + (((4 * w + quad) >> 1) ^ (r16 & (V / 8 - 1)))]);
      st[quad & 1] = __builtin_bit_cast(uint2, __builtin_convertvector(acc, bf16x4_t));
    }
  }
  if (j + 1 < nch)  // k of chunk j + 1 into X (X's K was read for the last time in P3a)
    fdma_k<0, NW>(X, a, seq0 + static_cast<int64_t>(j + 1) * kC, min(kC, seqlen - (j + 1) * kC), hk);
  lds_barrier();

  // ---- P3c: T diag(beta) rows 0-31 of chunk j (final after P3b) as hi / lo
  // over L's dead rows 0-31 ----
  if constexpr (SCAN) {  // whole output rows, 16 bytes a lane
    constexpr int PPR = V / 8, RPI = kWave / PPR;  // pieces a row, rows an instruction
#pragma unroll
    for (int it = 0; it < kC / (RPI * NW); ++it) {
      const int t = (it * NW + w) * RPI + lane / PPR, pc = lane % PPR;
      const uint4 val = X.tt.p[t * PPR + (pc ^ (t & (PPR - 1)))];
      if (t < Ls)  // nontemporal: the output is not read again here
        __builtin_nontemporal_store(__builtin_bit_cast(u32x4n, val),
                                    reinterpret_cast<u32x4n*>(a.o + ((toks + t) * a.HV + hv) * V + 8 * pc));
    }
  }
  const float* tf = X.vt.t;
  if constexpr (PREP) {
#pragma unroll
    for (int it = 0; it < 512 / NS; ++it) t_hilo(Y, tf, pp, (it * NS + tid) * 4);
  }
  lds_barrier();

  // ---- P4: rows 32-63 ----
  if constexpr (PREP) {
#pragma unroll
    for (int it = 0; it < 512 / NS; ++it) t_hilo(Y, tf, pp, 32 * kC + (it * NS + tid) * 4);
  }
  dma_wait();     // the copy of v of j has landed
  lds_barrier();  // chunk j is ready; X may be reused as chunk j + 1's buffer
}

// Prep waves NW .. NW + kNP - 1, chunk j in Y: P1 decay cumsum, K K^T / Q K^T
// tiles 4..9 | P2 their L, A; the scalings | P3a the inverse's diagonal
// blocks (T over X's V rows, dead since P2); copy q of j + 1 into X | P3b its
// first level and the second level's products with the diagonal blocks;
// copy the gates of j + 1 into X | P3c the second level | P4 wait for the
// copies.  (The L2 norms come from the diagonal tiles.)
template <int NW, bool PREP>
__device__ __forceinline__ void prep_iter(const FusedArgs& a, FBuf* __restrict__ Yp, FBuf* __restrict__ Xp,
                                          FPrep& pp, int j, int nch, int64_t seq0, int seqlen, int hv, int hk) {
  FBuf& Y = *Yp;
  FBuf& X = *Xp;
  constexpr int V = 16 * NW, NS = NW * 64;
  constexpr int kTPW = 2;  // tiles per prep wave
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));
  const int lane = tid & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int pw = w - NW, ptid = tid - NS;
  // tiles 4..9: one diagonal tile (5, 9) on each of the two waves with two tiles
  auto tile_of = [&](int slot) {
    return slot == 0 ? (pw == 0 ? 4 : pw == 1 ? 5 : pw == 2 ? 9 : 8) : (pw == 1 ? 6 : pw == 2 ? 7 : 10);
  };
  const int r16 = lane & 15, quad = lane >> 4, rq4 = quad * 4;
  const int64_t tokp = seq0 + static_cast<int64_t>(j) * kC;
  const int Lp = min(kC, seqlen - j * kC), Ln = min(kC, seqlen - (j + 1) * kC);

  // ---- P1 ----
  f32x4v kk[kTPW], qk[kTPW];
  if constexpr (PREP) {
    if (pw == kNP - 1) {  // decay cumsum; lane t: token t
      const int64_t gi = (tokp + (lane < Lp ? lane : Lp - 1)) * a.HV + hv;
      const float bt = lane < Lp ? gate_value(Y.gw[kC + lane], gi, a.beta_dt) : 0.f;
      const float x = wave_prefix_sum(lane < Lp ? gate_value(Y.gw[lane], gi, a.g_dt) : 0.f);
      pp.G[lane] = x;
      pp.G2[lane] = x * 1.4426950408889634f;
      pp.beta[lane] = bt;
      if (lane == kWave - 1) pp.gl = x;
    }
#pragma unroll
    for (int slot = 0; slot < kTPW; ++slot) {
      const int ti = tile_of(slot);
      if (ti < 10) kq_tile(Y, pp, a, ti, kk[slot], qk[slot], r16, quad);
    }
  }
  lds_barrier();

  // ---- P2 ----
  if constexpr (PREP) {
    if (pw == 0) {  // lane t: token t
      const float eg = expf(pp.G[lane]);
      Y.scal[lane] = eg * pp.rqs[lane];                           // output row scale of Q S
      Y.scal[kC + lane] = pp.rk[lane] * expf(pp.gl - pp.G[lane]);  // state-update scale of v_new row t
      Y.scal[2 * kC + lane] = -eg * pp.rk[lane];                  // row scale of K S inside -W S
      if (lane == 0) Y.scal[3 * kC] = expf(pp.gl);
    }
#pragma unroll
    for (int slot = 0; slot < kTPW; ++slot) {
      const int ti = tile_of(slot);
      if (ti < 10) la_tile(Y, pp, ti, kk[slot], qk[slot], r16, quad);
    }
  }
  lds_barrier();

  // ---- P3a ----
  float* tf = X.vt.t;  // T of chunk j over X's V rows (dead since P2)
  if constexpr (PREP) {
    if (pw == 0) inv_diag(Y.tt.l, tf);
  }
  if (j + 1 < nch) fdma_q<NW + 1, kNP - 1>(X, a, tokp + kC, Ln, hk);  // X's Q was read for the last time in P1
  lds_barrier();

  // ---- P3b ----
  f32x4v y0, y1;
  if constexpr (PREP) {
    if (pw < 2) inv_level1(Y.tt.l, tf, pw);
    inv_level2_pre(Y.tt.l, tf, pw, y0, y1);
  }
  if (j + 1 < nch) fdma_g<NW + 2>(X, a, tokp + kC, Ln, hv);  // X's gate words were read in the previous iteration
  lds_barrier();

  // ---- P3c ----
  if constexpr (PREP) inv_level2_fin(Y.tt.l, tf, pw, y0, y1);
  lds_barrier();

  // ---- P4 ----
  dma_wait();     // the copies into Y (v of j) and X (q, k, gates of j + 1) have landed
  lds_barrier();  // chunk j is ready; X may be reused as chunk j + 1's buffer
}

// NW scan waves (value columns 16 w .. 16 w + 15 each, the state in registers)
// and kNP prep waves.
template <int NW>
__global__ void __launch_bounds__((NW + kNP) * 64) chunk_fused_kernel(FusedArgs a) {
  __shared__ FBuf bufs[2];
  __shared__ FPrep pp;
  constexpr int V = 16 * NW, NT = (NW + kNP) * 64;
  const int hv = blockIdx.x % a.HV;
  const int sidx = blockIdx.x / a.HV;
  const int n = a.order ? a.order[sidx] : sidx;
  const int hk = hv / (a.HV / a.H);
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, quad = lane >> 4;
  const int64_t seq0 = a.cu[n];
  const int seqlen = a.cu[n + 1] - a.cu[n];
  const int nch = (seqlen + kC - 1) / kC;
  // A's halves in the upper blocks (0, 1) and (2, 3) are read as zeros and
  // nothing else writes them: clear them once in both buffers
  for (int e = tid; e < 2 * 32 * 4; e += NT) {  // buffer, row (0..15 or 32..47), piece 0..3
    const int bsel = e >> 7, rr = (e >> 2) & 31, pc = e & 3;
    const int t = rr < 16 ? rr : 16 + rr, p = t < 16 ? pc : 4 + pc;
    reinterpret_cast<uint2*>(&bufs[bsel].aqk[tpos(t, p)])[1] = make_uint2(0, 0);
  }
  // the first iteration only prepares, the last only runs the products; the
  // ones between do both, with each phase one block of straight-line code
  if (w < NW) {
    const int vcol = 16 * w + r16;
    // S[dt][i] = S[state_row(dt, quad, i)][vcol]
    f32x4v S[8];
    const int64_t sbase = (static_cast<int64_t>(n) * a.HV + hv) * kK;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) S[dt][i] = a.h0 ? a.h0[(sbase + state_row(dt, quad, i)) * V + vcol] : 0.f;
    wait_vmem();  // the state has arrived before the loop
    lds_barrier();  // (the prep waves' first copies)
    if (nch > 0) scan_iter<NW, true, false>(a, &bufs[0], &bufs[1], pp, S, 0, nch, seq0, seqlen, hv, hk);
#pragma unroll 1
    for (int j = 1; j < nch; ++j)
      scan_iter<NW, true, true>(a, &bufs[j & 1], &bufs[(j + 1) & 1], pp, S, j, nch, seq0, seqlen, hv, hk);
    if (nch > 0) scan_iter<NW, false, true>(a, &bufs[nch & 1], &bufs[(nch + 1) & 1], pp, S, nch, nch, seq0, seqlen, hv, hk);
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) a.ht[(sbase + state_row(dt, quad, i)) * V + vcol] = S[dt][i];
  } else {
    if (nch > 0) {
      fdma_q<NW, kNP>(bufs[0], a, seq0, min(kC, seqlen), hk);
      fdma_k<NW, kNP>(bufs[0], a, seq0, min(kC, seqlen), hk);
      fdma_g<NW>(bufs[0], a, seq0, min(kC, seqlen), hv);
      dma_wait();
    }
    lds_barrier();
    if (nch > 0) prep_iter<NW, true>(a, &bufs[0], &bufs[1], pp, 0, nch, seq0, seqlen, hv, hk);
#pragma unroll 1
    for (int j = 1; j < nch; ++j) prep_iter<NW, true>(a, &bufs[j & 1], &bufs[(j + 1) & 1], pp, j, nch, seq0, seqlen, hv, hk);
    if (nch > 0) prep_iter<NW, false>(a, &bufs[nch & 1], &bufs[(nch + 1) & 1], pp, nch, nch, seq0, seqlen, hv, hk);
  }
}

}  // namespace
}  // namespace yh

extern "C" int64_t yh_gdn_chunk_workspace_bytes(int64_t total_tokens, int64_t n_seqs, int64_t HV, int64_t V) {
  (void)total_tokens;
  (void)n_seqs;
  (void)HV;
  (void)V;
  return 0;  // the one-pass kernel keeps every per-chunk quantity on chip
}

extern "C" int yh_gdn_chunk_varlen(const void* q, const void* k, const void* v, const void* g, const void* beta,
                                   const float* initial_state, float* final_state, void* o,
                                   const int32_t* cu_seqlens, const int32_t* order, int64_t n_seqs,
                                   int64_t total_tokens, int64_t H, int64_t HV, int64_t K, int64_t V, float scale,
                                   int use_qk_l2norm, int qkv_dtype, int g_dtype, int beta_dtype, void* workspace,
                                   int64_t workspace_bytes, yh_stream_t stream) {
  using namespace yh;
  (void)workspace;
  (void)workspace_bytes;
  YH_CHECK_ARG(n_seqs >= 0 && total_tokens >= 0 && H > 0 && HV > 0 && HV % H == 0, "gdn_chunk: bad sizes");
  YH_CHECK_ARG(K == 128, "gdn_chunk: K must be 128 (got %lld)", (long long)K);
  YH_CHECK_ARG(V == 64 || V == 128, "gdn_chunk: V must be 64 or 128 (got %lld)", (long long)V);
  YH_CHECK_ARG(qkv_dtype == YH_BF16, "gdn_chunk: q/k/v must be bfloat16");
  YH_CHECK_ARG(is_float_dtype(g_dtype) && is_float_dtype(beta_dtype), "gdn_chunk: bad gate dtypes");
  if (n_seqs == 0) return YH_OK;
  YH_CHECK_ARG(q && k && v && g && beta && final_state && o && cu_seqlens, "gdn_chunk: null pointer");
  YH_CHECK_ARG(((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v) |
                 reinterpret_cast<uintptr_t>(o)) &
                15) == 0,
               "gdn_chunk: q/k/v/o must be 16-byte aligned");
  // 32-bit byte offsets of the copies: the gate tensors and one chunk's rows
  YH_CHECK_ARG(n_seqs * HV < (1LL << 31) && total_tokens * HV * 4 < (1LL << 31) && 64 * H * K * 2 < (1LL << 31) &&
                   64 * HV * V * 2 < (1LL << 31),
               "gdn_chunk: sizes too large");
  hipStream_t st = static_cast<hipStream_t>(stream);
  FusedArgs f{static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k), static_cast<const uint16_t*>(v), g,
              beta, cu_seqlens, order, initial_state, final_state, static_cast<uint16_t*>(o), (int)n_seqs, (int)H,
              (int)HV, scale, use_qk_l2norm ? 1 : 0, g_dtype, beta_dtype};
  const dim3 grid(static_cast<unsigned>(n_seqs * HV));
  if (V == 128)
    hipLaunchKernelGGL(chunk_fused_kernel<8>, grid, dim3((8 + kNP) * 64), 0, st, f);
  else
    hipLaunchKernelGGL(chunk_fused_kernel<4>, grid, dim3((4 + kNP) * 64), 0, st, f);
  YH_CHECK_LAUNCH("gdn_chunk");
  return YH_OK;
}
