// Decode projection on packed weights, generalised over the work split of a
// workgroup: out[M, N] = x[M, K] . W[N, K]^T for M <= 256 rows, bf16 in,
// fp32 accumulation (the decode step's projections: modeling_yanchor.py:
// 147-176 and the Qwen3.5 GDN / attention / MLP projections of the
// transformers wheel).  W is in the MFMA fragment order of yh_linear_pack
// (K blocks outermost, the N/16 column tiles of a block side by side).
//
// Workgroup = NCG column groups x KP K parts = NCG * KP waves.  A column
// group owns 32 output columns (two 16-column MFMA tiles), so every x
// fragment read from LDS feeds two MFMAs; the KP waves of a group take the
// 32-wide K blocks of each phase in turn and add their accumulators through
// LDS at the end (fixed order).  Per phase the workgroup stages x rows
// [0, 16 MT) x (32 KP BPW) of K in LDS (loaded into registers a phase
// ahead, one barrier a phase); each wave streams its weight fragments WD K
// blocks ahead of use (a register ring with static slots: the phase loop is
// unrolled WD / BPW times).  The grid is (column blocks of 32 NCG, S K
// slices); with S > 1 each slice writes fp32 partials and yh_linear_reduce /
// the consumer's norm sums them in slice order.
//
// Knobs (the host picks them per shape): NCG sets the columns per workgroup
// (how many of the 256 CUs a projection covers, and x's restaging cost per
// weight byte, M / (32 NCG)); KP the waves per column group (latency
// hiding); WD the weight bytes in flight per CU (64 NCG KP WD fragments of
// 1 KiB).
#include <algorithm>

#include "common.h"

namespace yh {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4v __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4v __attribute__((ext_vector_type(4)));

constexpr int kMaxRows = 256;

struct ProjArgs {
  const uint16_t* x;   // [M, K], row stride xs
  const uint16_t* w;   // packed [N, K]
  uint16_t* out;       // [M, N] (or [M, N/2] with silu pairs), row stride os
  float* part;         // [S, M, N] fp32 partials (S > 1)
  int64_t xs, os;
  int M, N, K, S, phases_per_slice;
  const uint16_t* res;  // residual [M, N] (S == 1): out = bf16(bf16(x . W^T) + res)
  int64_t rs;
  int silu_pairs;       // [gate; up] packed with pair halves: out = bf16(bf16(silu(gate)) * up)
};

__device__ __forceinline__ u32x4v ldw(const uint16_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4v*>(p));
}
__device__ __forceinline__ void sync_lds() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
__device__ __forceinline__ f32x4v mma(bf16x8_t a, bf16x8_t b, f32x4v c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

template <int MT, int NCG, int KP, int BPW, int WD>
struct Cfg {
  static constexpr int W = NCG * KP;             // waves
  static constexpr int NT = 64 * W;              // threads
  static constexpr int PB = KP * BPW;            // 32-wide K blocks per phase
  static constexpr int PK = 32 * PB;             // K per phase
  static constexpr int PAD = PK + 8;             // LDS row stride (elements)
  static constexpr int ROWS = 16 * MT;
  static constexpr int XT = ROWS * PK / 8;        // 16-byte x vectors per phase
  static constexpr int XV = (XT + NT - 1) / NT;   // per thread (the last round may be partial)
  static constexpr int UF = WD / BPW;            // phases per turn of the weight ring
  static constexpr int UR = UF % 2 ? 2 * UF : UF;  // phases per unrolled loop turn (x buffers alternate)
  static_assert(WD % BPW == 0, "the ring turns in whole phases");
  static_assert(UR <= 4 && BPW <= 4, "at most four phases per loop turn, four blocks per phase");
  static constexpr int XBYTES = 2 * ROWS * PAD * 2;
  static constexpr int RBYTES = NCG * MT * 2 * 64 * 16;  // one K part's accumulators
  static constexpr int TW = 32 * NCG;                     // output tile width (columns)
  static constexpr int TBYTES = ROWS * TW * 4;            // the output tile (fp32 for partials)
  static constexpr int SMEM0 = XBYTES > RBYTES ? XBYTES : RBYTES;
  static constexpr int SMEM = SMEM0 > TBYTES ? SMEM0 : TBYTES;
  static_assert(SMEM <= 160 * 1024, "LDS");
};

template <int MT, int WD>
struct Regs {
  u32x4v wr[WD][2];
  f32x4v acc[MT][2];
};

template <class C, int MT>
__device__ __forceinline__ void load_x(const ProjArgs& a, int k0, u32x4v (&r)[C::XV]) {
#pragma unroll
  for (int i = 0; i < C::XV; ++i) {
    const int idx = i * C::NT + threadIdx.x;
    const int row = idx / (C::PK / 8), c8 = (idx % (C::PK / 8)) * 8;
    if (C::XT % C::NT == 0 || idx < C::XT)
      r[i] = *reinterpret_cast<const u32x4v*>(a.x + min(row, a.M - 1) * a.xs + k0 + c8);
  }
}
template <class C>
__device__ __forceinline__ void store_x(uint16_t* buf, const u32x4v (&r)[C::XV]) {
#pragma unroll
  for (int i = 0; i < C::XV; ++i) {
    const int idx = i * C::NT + threadIdx.x;
    const int row = idx / (C::PK / 8), c8 = (idx % (C::PK / 8)) * 8;
    if (C::XT % C::NT == 0 || idx < C::XT) *reinterpret_cast<u32x4v*>(buf + row * C::PAD + c8) = r[i];
  }
}

struct WaveLoc {
  const uint16_t* wp[2];  // this lane's 16 bytes of K block 0 of each column tile
  int kb0;                // first K block of the slice
  int last;               // last K block of the slice
  int part;               // K part of this wave
  int col, quad;
  int64_t bstride;        // elements from one K block of a tile to the next (N/16 fragments)
};

// Block I of the wave's BPW blocks in phase ph at unroll position U: A
// fragments from LDS, 2 MT MFMAs, then ring slot (U BPW + I) % WD (a
// compile-time slot) refilled with the wave's block WD ahead.
template <int MT, int NCG, int KP, int BPW, int WD, int U, int I>
__device__ __forceinline__ void block_step(Regs<MT, WD>& g, const uint16_t* cur, const WaveLoc& v, int ph) {
  using C = Cfg<MT, NCG, KP, BPW, WD>;
  constexpr int slot = (U * BPW + I) % WD;
  const int kk = (v.part + KP * I) * 32 + v.quad * 8;
  const bf16x8_t b0 = __builtin_bit_cast(bf16x8_t, g.wr[slot][0]);
  const bf16x8_t b1 = __builtin_bit_cast(bf16x8_t, g.wr[slot][1]);
  bf16x8_t av[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t)
    av[t] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const u32x4v*>(cur + (t * 16 + v.col) * C::PAD + kk));
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    g.acc[t][0] = mma(av[t], b0, g.acc[t][0]);
    g.acc[t][1] = mma(av[t], b1, g.acc[t][1]);
  }
  __builtin_amdgcn_sched_barrier(0);
  const int tn = ph * BPW + I + WD;  // the wave's block WD ahead
  const int blk = min(v.kb0 + (tn / BPW) * KP * BPW + v.part + KP * (tn % BPW), v.last);
  g.wr[slot][0] = ldw(v.wp[0] + static_cast<int64_t>(blk) * v.bstride);
  g.wr[slot][1] = ldw(v.wp[1] + static_cast<int64_t>(blk) * v.bstride);
  __builtin_amdgcn_sched_barrier(0);
}

// Phase ph at unroll position U: x of the next phase into registers, the
// wave's BPW blocks, then the next x phase to LDS and a barrier.
template <int MT, int NCG, int KP, int BPW, int WD, int U>
__device__ __forceinline__ void phase(Regs<MT, WD>& g, u32x4v (&xr)[Cfg<MT, NCG, KP, BPW, WD>::XV], uint16_t* xs,
                                      const ProjArgs& a, const WaveLoc& v, int ph, int nph) {
  using C = Cfg<MT, NCG, KP, BPW, WD>;
  load_x<C, MT>(a, v.kb0 * 32 + min(ph + 1, nph - 1) * C::PK, xr);
  __builtin_amdgcn_sched_barrier(0);
  const uint16_t* cur = xs + (U & 1) * C::ROWS * C::PAD;
  block_step<MT, NCG, KP, BPW, WD, U, 0>(g, cur, v, ph);
  if constexpr (BPW > 1) block_step<MT, NCG, KP, BPW, WD, U, 1>(g, cur, v, ph);
  if constexpr (BPW > 2) block_step<MT, NCG, KP, BPW, WD, U, 2>(g, cur, v, ph);
  if constexpr (BPW > 3) block_step<MT, NCG, KP, BPW, WD, U, 3>(g, cur, v, ph);
  store_x<C>(xs + ((U + 1) & 1) * C::ROWS * C::PAD, xr);
  sync_lds();
}

// The workgroup's output goes through LDS: part-0 waves leave their finished
// values in a row-major tile [16 MT][32 NCG] (bf16 products, bf16 silu
// products [16 MT][16 NCG], or fp32 partials), then every thread stores whole
// rows 16 bytes at a time.  Stores straight from the MFMA layout (2 or 4
// bytes a lane, 16 lanes a row) took ~4 us more per call than the staged
// rows: the kernel's last step is on every decode projection's critical path.
template <class C, int MT, int NCG>
__device__ __forceinline__ void stage_tile(const f32x4v (&acc)[MT][2], char* smem, const ProjArgs& a, int cg, int col,
                                           int quad) {
  if (a.silu_pairs) {
    uint16_t* tile = reinterpret_cast<uint16_t*>(smem);
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float gt = bf16_to_f32(f32_to_bf16(acc[t][0][i])), up = bf16_to_f32(f32_to_bf16(acc[t][1][i]));
        const float sg = bf16_to_f32(f32_to_bf16(gt / (1.f + expf(-gt))));
        tile[(t * 16 + quad * 4 + i) * (C::TW / 2) + cg * 16 + col] = f32_to_bf16(sg * up);
      }
  } else if (a.S == 1) {
    uint16_t* tile = reinterpret_cast<uint16_t*>(smem);
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int ct = 0; ct < 2; ++ct)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          tile[(t * 16 + quad * 4 + i) * C::TW + cg * 32 + ct * 16 + col] = f32_to_bf16(acc[t][ct][i]);
  } else {
    float* tile = reinterpret_cast<float*>(smem);
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int ct = 0; ct < 2; ++ct)
#pragma unroll
        for (int i = 0; i < 4; ++i) tile[(t * 16 + quad * 4 + i) * C::TW + cg * 32 + ct * 16 + col] = acc[t][ct][i];
  }
}

template <class C>
__device__ __forceinline__ void store_rows(const char* smem, const ProjArgs& a, int slice) {
  if (a.silu_pairs) {   // bf16 [ROWS][TW / 2] -> out columns blockIdx.x * TW / 2 ..
    constexpr int W2 = C::TW / 2, VPR = W2 / 8;
    const uint16_t* tile = reinterpret_cast<const uint16_t*>(smem);
    const int c0 = blockIdx.x * W2;
    for (int e = threadIdx.x; e < C::ROWS * VPR; e += C::NT) {
      const int r = e / VPR, c8 = (e % VPR) * 8;
      if (r < a.M && c0 + c8 < a.N / 2)
        *reinterpret_cast<u32x4v*>(a.out + r * a.os + c0 + c8) = *reinterpret_cast<const u32x4v*>(tile + r * W2 + c8);
    }
  } else if (a.S == 1) {   // bf16 [ROWS][TW], plus the residual
    constexpr int VPR = C::TW / 8;
    const uint16_t* tile = reinterpret_cast<const uint16_t*>(smem);
    const int c0 = blockIdx.x * C::TW;
    for (int e = threadIdx.x; e < C::ROWS * VPR; e += C::NT) {
      const int r = e / VPR, c8 = (e % VPR) * 8;
      if (r >= a.M || c0 + c8 >= a.N) continue;
      u32x4v y = *reinterpret_cast<const u32x4v*>(tile + r * C::TW + c8);
      if (a.res) {   // out = bf16(bf16(x . W^T) + residual)
        const u32x4v rv = *reinterpret_cast<const u32x4v*>(a.res + r * a.rs + c0 + c8);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float lo = bf16_to_f32(y[j] & 0xffff) + bf16_to_f32(rv[j] & 0xffff);
          const float hi = bf16_to_f32(y[j] >> 16) + bf16_to_f32(rv[j] >> 16);
          y[j] = static_cast<uint32_t>(f32_to_bf16(lo)) | (static_cast<uint32_t>(f32_to_bf16(hi)) << 16);
        }
      }
      *reinterpret_cast<u32x4v*>(a.out + r * a.os + c0 + c8) = y;
    }
  } else {   // fp32 partials [ROWS][TW] of this slice
    constexpr int VPR = C::TW / 4;
    const float* tile = reinterpret_cast<const float*>(smem);
    float* mine = a.part + static_cast<int64_t>(slice) * a.M * a.N;
    const int c0 = blockIdx.x * C::TW;
    for (int e = threadIdx.x; e < C::ROWS * VPR; e += C::NT) {
      const int r = e / VPR, c4 = (e % VPR) * 4;
      if (r < a.M && c0 + c4 < a.N)
        *reinterpret_cast<f32x4v*>(mine + static_cast<int64_t>(r) * a.N + c0 + c4) =
            *reinterpret_cast<const f32x4v*>(tile + r * C::TW + c4);
    }
  }
}

template <int MT, int NCG, int KP, int BPW, int WD>
__global__ void __launch_bounds__(64 * NCG * KP) proj_kernel(ProjArgs a) {
  using C = Cfg<MT, NCG, KP, BPW, WD>;
  __shared__ __align__(16) char smem[C::SMEM];
  uint16_t* xs = reinterpret_cast<uint16_t*>(smem);

  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int cg = w % NCG;
  const int slice = blockIdx.y;
  const int ph0 = slice * a.phases_per_slice;
  const int nph = min(a.K / C::PK, ph0 + a.phases_per_slice) - ph0;
  WaveLoc v;
  v.part = w / NCG;
  v.col = lane & 15;
  v.quad = lane >> 4;
  v.kb0 = ph0 * C::PB;
  v.last = v.kb0 + max(nph, 1) * C::PB - 1;
  v.bstride = static_cast<int64_t>(a.N / 16) * 512;
#pragma unroll
  for (int ct = 0; ct < 2; ++ct) {
    const int T = min(static_cast<int>(blockIdx.x) * 2 * NCG + cg * 2 + ct, a.N / 16 - 1);
    v.wp[ct] = a.w + static_cast<int64_t>(T) * 512 + lane * 8;
  }
  Regs<MT, WD> g;
  u32x4v xr[C::XV];
#pragma unroll
  for (int t = 0; t < MT; ++t) g.acc[t][0] = g.acc[t][1] = f32x4v{0.f, 0.f, 0.f, 0.f};

  if (nph > 0) {  // uniform over the workgroup
    load_x<C, MT>(a, v.kb0 * 32, xr);
#pragma unroll
    for (int s = 0; s < WD; ++s) {
      const int blk = min(v.kb0 + (s / BPW) * KP * BPW + v.part + KP * (s % BPW), v.last);
      g.wr[s][0] = ldw(v.wp[0] + static_cast<int64_t>(blk) * v.bstride);
      g.wr[s][1] = ldw(v.wp[1] + static_cast<int64_t>(blk) * v.bstride);
    }
    store_x<C>(xs, xr);
    sync_lds();
    // phase ph runs at unroll position ph % UR: its x buffer is ph % 2 and
    // its ring slots (ph BPW + i) % WD, both static
    int ph = 0;
    for (; ph + C::UR <= nph; ph += C::UR) {
      phase<MT, NCG, KP, BPW, WD, 0>(g, xr, xs, a, v, ph, nph);
      phase<MT, NCG, KP, BPW, WD, 1>(g, xr, xs, a, v, ph + 1, nph);
      if constexpr (C::UR > 2) phase<MT, NCG, KP, BPW, WD, 2>(g, xr, xs, a, v, ph + 2, nph);
      if constexpr (C::UR > 2) phase<MT, NCG, KP, BPW, WD, 3>(g, xr, xs, a, v, ph + 3, nph);
    }
    if (ph < nph) phase<MT, NCG, KP, BPW, WD, 0>(g, xr, xs, a, v, ph, nph);
    if (ph + 1 < nph) phase<MT, NCG, KP, BPW, WD, 1>(g, xr, xs, a, v, ph + 1, nph);
    if constexpr (C::UR > 2) if (ph + 2 < nph) phase<MT, NCG, KP, BPW, WD, 2>(g, xr, xs, a, v, ph + 2, nph);
  }

  // K parts meet in LDS, one part a round, added to part 0's accumulators
  // in part order (a fixed order); part 0 stores
  f32x4v* red = reinterpret_cast<f32x4v*>(smem);
#pragma unroll 1
  for (int p = 1; p < KP; ++p) {
    sync_lds();
    if (v.part == p) {
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) red[((cg * MT + t) * 2 + ct) * 64 + lane] = g.acc[t][ct];
    }
    sync_lds();
    if (v.part == 0) {
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) g.acc[t][ct] += red[((cg * MT + t) * 2 + ct) * 64 + lane];
    }
  }
  sync_lds();   // every part-0 wave has read its partners' accumulators
  if (v.part == 0) stage_tile<C, MT, NCG>(g.acc, smem, a, cg, v.col, v.quad);
  sync_lds();
  store_rows<C>(smem, a, slice);
}

template <int MT, int NCG, int KP, int BPW, int WD>
int launch_cfg(const ProjArgs& a, int64_t col_blocks, int S, hipStream_t st) {
  using C = Cfg<MT, NCG, KP, BPW, WD>;
  hipLaunchKernelGGL((proj_kernel<MT, NCG, KP, BPW, WD>), dim3(static_cast<unsigned>(col_blocks), S), dim3(C::NT), 0,
                     st, a);
  return C::PK;
}

// Configurations compiled in (id -> NCG, KP, BPW, WD), each for 32, 64 and
// 128 rows (MT = 2, 4, 8).  Measured on MI355X at M = 128 in HIP graphs over
// rotating weights (us; ms scale in brackets is the kernel alone before a
// split-K reduce):
//   0: 128 columns, 8 waves   -- N <= 4096 with split K (2560 x 4096: 10.7
//                                at S = 8; 2560 x 9728: 16.7 at S = 10)
//   1:  64 columns, 8 waves   -- N ~ 8k-12k (12352 x 2560: 21.9, 9280 x
//                                2560: 21.0; 2048 x 2560 at S = 5: 9.4)
//   2:  96 columns, 12 waves  -- N ~ 16k-20k (19456 x 2560: 27.3; 16448 x
//                                2560: 26.3)
//   3: 160 columns, 10 waves  -- the head (151936 x 2560: 170)
struct CfgRow {
  int ncg, kp, bpw, wd;
};
constexpr CfgRow kCfgs[] = {{4, 2, 2, 2}, {2, 4, 2, 2}, {3, 4, 1, 2}, {5, 2, 2, 2}};
constexpr int kNumCfgs = sizeof(kCfgs) / sizeof(kCfgs[0]);

int phase_k(int id) { return 32 * kCfgs[id].kp * kCfgs[id].bpw; }

template <int MT>
void launch_mt(int id, const ProjArgs& a, int64_t col_blocks, int S, hipStream_t st) {
  switch (id) {
    case 0: launch_cfg<MT, 4, 2, 2, 2>(a, col_blocks, S, st); break;
    case 1: launch_cfg<MT, 2, 4, 2, 2>(a, col_blocks, S, st); break;
    case 2: launch_cfg<MT, 3, 4, 1, 2>(a, col_blocks, S, st); break;
    default: launch_cfg<MT, 5, 2, 2, 2>(a, col_blocks, S, st); break;
  }
}

// Past 128 rows only configuration 0 runs, with 256-row tiles (8 waves at
// 250 VGPRs, 136 KiB of LDS; the other configurations' registers or x
// phases do not fit).  At M = 256 it beats hipBLASLt on the decode
// projections: 29.5 against 40.9 us for 2560 x 9728 (S = 12), 17.1 against
// 21.5 for 2560 x 4096, 28.5 against 36.5 for 9280 x 2560 (S = 2), 44.7
// against 46.4 for 16448 x 2560; even for 151936 x 2560.
void launch_id(int id, const ProjArgs& a, int64_t col_blocks, int S, hipStream_t st) {
  if (a.M > 128) launch_cfg<16, 4, 2, 2, 2>(a, col_blocks, S, st);
  else if (a.M <= 32) launch_mt<2>(id, a, col_blocks, S, st);
  else if (a.M <= 64) launch_mt<4>(id, a, col_blocks, S, st);
  else launch_mt<8>(id, a, col_blocks, S, st);
}

// Configuration and K split for a shape: the workgroup width that puts at
// most one workgroup on each of the 256 CUs with the fewest idle CUs (wider
// tiles restage x less often per weight byte); a projection narrower than
// the chip splits K instead, over at most 16 slices of at least two phases.
void pick(int64_t M, int64_t N, int64_t K, int silu, int* cfg, int* split) {
  if (M > 128) {  // configuration 0 only, K split as below for narrow projections
    const int64_t blocks = (N + 32 * kCfgs[0].ncg - 1) / (32 * kCfgs[0].ncg), phases = K / phase_k(0);
    *cfg = 0;
    *split = blocks < 128 && !silu
                 ? static_cast<int>(std::max<int64_t>(1, std::min<int64_t>({256 / blocks, phases / 2, 16})))
                 : 1;
    return;
  }
  auto usable = [&](int id) { return K % phase_k(id) == 0; };
  int best = -1;
  int64_t best_blocks = 0;
  for (int id : {0, 1, 2, 3}) {
    if (!usable(id)) continue;
    const int64_t blocks = (N + 32 * kCfgs[id].ncg - 1) / (32 * kCfgs[id].ncg);
    if (blocks > 256) continue;
    if (best < 0 || blocks > best_blocks) best = id, best_blocks = blocks;
  }
  if (best < 0) {  // wider than the chip at every width: the widest tiles
    *cfg = usable(3) ? 3 : 0;
    *split = 1;
    return;
  }
  *cfg = best;
  *split = 1;
  if (best_blocks < 128 && !silu) {  // a narrow projection: K slices fill the chip
    *cfg = usable(0) ? 0 : best;
    const int64_t blocks = (N + 32 * kCfgs[*cfg].ncg - 1) / (32 * kCfgs[*cfg].ncg);
    const int64_t phases = K / phase_k(*cfg);
    *split = static_cast<int>(std::max<int64_t>(1, std::min<int64_t>({256 / blocks, phases / 2, 16})));
  }
}

}  // namespace
}  // namespace yh

extern "C" int yh_proj_config_count(void) { return yh::kNumCfgs; }

extern "C" int yh_proj_phase_k(int config) {
  return config >= 0 && config < yh::kNumCfgs ? yh::phase_k(config) : 0;
}

extern "C" int yh_proj_columns(int config) {
  return config >= 0 && config < yh::kNumCfgs ? 32 * yh::kCfgs[config].ncg : 0;
}

extern "C" int yh_proj(const void* x, int64_t x_stride, const void* w_packed, void* out, int64_t out_stride, int64_t M,
                       int64_t N, int64_t K, const void* residual, int64_t residual_stride, int silu_pairs, int config,
                       int64_t split_k, void* workspace, int64_t workspace_bytes, int64_t* slices_out,
                       yh_stream_t stream) {
  using namespace yh;
  YH_CHECK_ARG(config >= 0 && config < kNumCfgs, "proj: unknown configuration %d", config);
  const int pk = phase_k(config), cols = 32 * kCfgs[config].ncg;
  YH_CHECK_ARG(M >= 0 && M <= kMaxRows, "proj: M must be in [0, %d]", kMaxRows);
  YH_CHECK_ARG(M <= 128 || config == 0, "proj: more than 128 rows run on configuration 0 only");
  YH_CHECK_ARG(N > 0 && N % 16 == 0 && (!silu_pairs || N % 32 == 0),
               "proj: N must be a positive multiple of 16 (32 with the silu epilogue)");
  YH_CHECK_ARG(K > 0 && K % pk == 0, "proj: K must be a positive multiple of %d for configuration %d", pk, config);
  YH_CHECK_ARG(x_stride >= K && x_stride % 8 == 0 && out_stride >= (silu_pairs ? N / 2 : N), "proj: bad strides");
  YH_CHECK_ARG(!silu_pairs || (!residual && split_k == 1), "proj: the silu epilogue needs no residual, split_k 1");
  const int64_t phases = K / pk;
  YH_CHECK_ARG(split_k >= 1 && split_k <= phases, "proj: split_k must be in [1, K / %d]", pk);
  if (M == 0) {
    if (slices_out) *slices_out = 1;
    return YH_OK;
  }
  YH_CHECK_ARG(x && w_packed && out, "proj: null pointer");
  YH_CHECK_ARG(((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w_packed)) & 15) == 0,
               "proj: x and the packed weights must be 16-byte aligned");
  const int64_t pps = (phases + split_k - 1) / split_k;
  const int S = static_cast<int>((phases + pps - 1) / pps);
  const int64_t need = S > 1 ? static_cast<int64_t>(S) * M * N * 4 : 0;
  YH_CHECK_ARG(S == 1 || (workspace && workspace_bytes >= need), "proj: workspace of %lld bytes required",
               (long long)need);
  YH_CHECK_ARG(S == 1 || (reinterpret_cast<uintptr_t>(workspace) & 15) == 0, "proj: workspace must be 16-byte aligned");
  YH_CHECK_ARG(!residual || (residual_stride >= N && S == 1), "proj: a residual needs split_k 1");
  // the output rows (and the residual's) are written / read 16 bytes at a time
  YH_CHECK_ARG((reinterpret_cast<uintptr_t>(out) & 15) == 0 && out_stride % 8 == 0,
               "proj: output rows must be 16-byte aligned");
  YH_CHECK_ARG(!residual || ((reinterpret_cast<uintptr_t>(residual) & 15) == 0 && residual_stride % 8 == 0),
               "proj: residual rows must be 16-byte aligned");
  ProjArgs a{static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(w_packed), static_cast<uint16_t*>(out),
             S > 1 ? static_cast<float*>(workspace) : nullptr, x_stride, out_stride, (int)M, (int)N, (int)K, S,
             static_cast<int>(pps), static_cast<const uint16_t*>(residual), residual_stride, silu_pairs};
  const int64_t col_blocks = (N + cols - 1) / cols;
  YH_CHECK_ARG(col_blocks < (1LL << 31), "proj: too many columns");
  launch_id(config, a, col_blocks, S, static_cast<hipStream_t>(stream));
  YH_CHECK_LAUNCH("proj");
  if (slices_out) *slices_out = S;
  return YH_OK;
}

extern "C" int yh_proj_pick(int64_t M, int64_t N, int64_t K, int silu_pairs, int* config, int64_t* split_k) {
  using namespace yh;
  YH_CHECK_ARG(config && split_k, "proj_pick: null pointer");
  YH_CHECK_ARG(M >= 0 && N > 0 && K > 0 && K % 128 == 0, "proj_pick: K must be a positive multiple of 128");
  int c = 0, s = 1;
  pick(M, N, K, silu_pairs, &c, &s);
  *config = c;
  *split_k = s;
  return YH_OK;
}

extern "C" int yh_linear_packed_split(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N < 16 || K < 128 || K % 128) return 1;
  int c = 0, s = 1;
  yh::pick(M, N, K, 0, &c, &s);
  return s;
}

extern "C" int yh_linear_packed(const void* x, int64_t x_stride, const void* w_packed, void* out, int64_t out_stride,
                                int64_t M, int64_t N, int64_t K, const void* residual, int64_t residual_stride,
                                int silu_pairs, int64_t split_k, void* workspace, int64_t workspace_bytes,
                                int defer_reduce, int64_t* slices_out, yh_stream_t stream) {
  using namespace yh;
  YH_CHECK_ARG(K > 0 && K % 128 == 0, "linear_packed: K must be a positive multiple of 128");
  YH_CHECK_ARG(M >= 0 && N > 0, "linear_packed: bad sizes");
  YH_CHECK_ARG(split_k >= 1 && split_k <= K / 128, "linear_packed: split_k must be in [1, K/128]");
  int c = 0, s = 1;
  pick(M, N, K, silu_pairs, &c, &s);
  // an explicit split keeps its meaning: K slices of whole phases (the
  // configuration's phase, or 128 wide if the split needs finer slices)
  if (split_k > K / phase_k(c)) c = 0;
  const int64_t phases = K / phase_k(c), pps = (phases + split_k - 1) / split_k;
  const bool one = (phases + pps - 1) / pps == 1;  // one slice: the residual goes into the store
  int64_t slices = 1;
  const int rc = yh_proj(x, x_stride, w_packed, out, out_stride, M, N, K, one ? residual : nullptr, residual_stride,
                         silu_pairs, c, split_k, workspace, workspace_bytes, &slices, stream);
  if (rc != YH_OK) return rc;
  if (slices_out) *slices_out = slices;
  if (slices > 1 && !defer_reduce) return yh_linear_reduce(static_cast<const float*>(workspace), out, out_stride, M, N,
                                                           slices, residual, residual_stride, stream);
  return YH_OK;
}
