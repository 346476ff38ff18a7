// Fixed-slot anchor memory: decode read and decode push / Top-K commit.
//
// State layout (IndependentMemoryState, reference modeling_yanchor.py:80-120),
// each field [NB, ...] with its own row stride (elements between consecutive
// state rows; the dense stride unless the state lives in a slot page such as
// the vLLM wire format, vllm_yanchor.py:21-24, 49-64):
//   keys, values      [NB, G, KC, D]   (bf16 / fp16 / fp32)
//   scores            [NB, G, KC]      fp32, -inf = empty
//   positions         [NB, G, KC]      int32, -1 = empty (the validity mask)
//   pending_keys/vals [NB, G, PC, D]
//   pending_scores    [NB, G, PC]      fp32
//   count, total      [NB]             int64
//
// anchor_read_kernel   replaces _read_parts + _read_reduce / committed_gqa
//                      (runtime/model/independent_memory.py:47-88, 177-188) and
//                      the torch branch modeling_yanchor.py:283-290.
// anchor_commit_kernel replaces _push_select + _gather_commit + _write_commit
//                      (independent_memory.py:90-164) and modeling_yanchor.py:
//                      291-310.
// anchor_advance_kernel replaces _advance (independent_memory.py:166-175).
#include "common.h"

namespace yh {
namespace {

constexpr int kMaxCap = 1024;

struct ReadArgs {
  const void* q;          // [B, H, D]
  const void* keys;       // [NB, G, KC, D]
  const void* values;
  const int32_t* pos;     // [NB, G, KC]
  const int32_t* idx;     // [B] or null
  void* out;              // [B, H, D]
  int B, G, KC;
  int64_t n_rows;
  int64_t k_rs, v_rs, p_rs;  // row strides (elements) of keys, values, positions
  float scale;
  // optional epilogue, in the order the decode layer applies it to the read:
  //   x = 0 where row_valid[row] == 0; x *= head_gate[row, h];
  //   x *= sigmoid(gate[row, h, d])   (every product rounded to the dtype)
  const uint8_t* row_valid;   // [B]
  const float* head_gate;     // [B, H]
  const void* gate;           // rows gate_ts apart, heads gate_hs apart
  int64_t gate_ts, gate_hs;
};

// A value rounded to the storage precision of DT (a bf16 / fp16 tensor op
// rounds every intermediate it materialises).
template <int DT>
__device__ __forceinline__ float round_dt(float x) {
  if constexpr (DT == YH_BF16) return bf16_to_f32(f32_to_bf16(x));
  else if constexpr (DT == YH_F16) return f16_to_f32(f32_to_f16(x));
  else return x;
}

template <int DT>
__device__ __forceinline__ float read_epilogue(const ReadArgs& a, int row, int H, int head, int d, float x) {
  if (a.row_valid && a.row_valid[row] == 0) return 0.f;
  x = round_dt<DT>(x);
  if (a.head_gate) x = round_dt<DT>(x * round_dt<DT>(a.head_gate[static_cast<int64_t>(row) * H + head]));
  if (a.gate) {
    const float gv = load_any(a.gate, row * a.gate_ts + head * a.gate_hs + d, DT);
    x = round_dt<DT>(x * round_dt<DT>(1.f / (1.f + expf(-gv))));
  }
  return x;
}

// 8 consecutive elements of a bf16/fp16/fp32 row as floats (16 B for 2-byte
// types, 2 x 16 B for fp32).
template <int DT>
__device__ __forceinline__ void load8(const void* p, int64_t i, float* f) {
  if constexpr (DT == YH_F32) {
    const float4 a = reinterpret_cast<const float4*>(static_cast<const float*>(p) + i)[0];
    const float4 b = reinterpret_cast<const float4*>(static_cast<const float*>(p) + i)[1];
    f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w; f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
  } else {
    const uint4 w = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p) + i)[0];
    const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if constexpr (DT == YH_BF16) {
        f[2 * j] = __uint_as_float(u[j] << 16);
        f[2 * j + 1] = __uint_as_float(u[j] & 0xffff0000u);
      } else {
        f[2 * j] = f16_to_f32(u[j] & 0xffff);
        f[2 * j + 1] = f16_to_f32(u[j] >> 16);
      }
    }
  }
}

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
// Raw 8 elements (16 B for 2-byte types, 32 B for fp32) of a key/value row.
template <int DT> struct Raw8 { uint4 w[DT == YH_F32 ? 2 : 1]; };

template <int DT>
__device__ __forceinline__ void ld_raw8(Raw8<DT>& r, const void* p, int64_t i) {
  if constexpr (DT == YH_F32) {
    r.w[0] = reinterpret_cast<const uint4*>(static_cast<const float*>(p) + i)[0];
    r.w[1] = reinterpret_cast<const uint4*>(static_cast<const float*>(p) + i)[1];
  } else {
    r.w[0] = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p) + i)[0];
  }
}
// Dot product of 8 packed 16-bit elements, fp32 accumulation (dot2 pairs).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
template <int DT>
__device__ __forceinline__ float dot8(const Raw8<DT>& a, const Raw8<DT>& b) {
  const uint32_t x[4] = {a.w[0].x, a.w[0].y, a.w[0].z, a.w[0].w};
  const uint32_t y[4] = {b.w[0].x, b.w[0].y, b.w[0].z, b.w[0].w};
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if constexpr (DT == YH_BF16)
      acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, x[j]), __builtin_bit_cast(bf16x2_t, y[j]),
                                            acc, false);
    else
      acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, x[j]), __builtin_bit_cast(f16x2_t, y[j]), acc, false);
  }
  return acc;
}

// The NI rows of one block: row pointer p (this lane's 8 elements of the
// block's first row), rows `stride` elements apart -- constant offsets from
// one base, so the loads need no per-row address registers.  Key and value
// rows are read once per token: the loads are nontemporal, so they stream
// past the caches instead of evicting what the other kernels of the step
// reuse (measured: 39.1 -> 34.5 us for 64 rows x 32 memories x 256 slots,
// 103 -> 95 us for the 1024-slot window ring at 128 rows x 8 groups).
template <int DT, int NI, int STRIDE>
__device__ __forceinline__ void ld_block(Raw8<DT> (&r)[NI], const void* p) {
  constexpr int kEsz = DT == YH_F32 ? 4 : 2;
  const char* c = static_cast<const char*>(p);
#pragma unroll
  for (int i = 0; i < NI; ++i) {
#pragma unroll
    for (int j = 0; j < (DT == YH_F32 ? 2 : 1); ++j) {
      const u32x4_t v = __builtin_nontemporal_load(
          reinterpret_cast<const u32x4_t*>(c + static_cast<int64_t>(i) * STRIDE * kEsz + j * 16));
      r[i].w[j] = make_uint4(v.x, v.y, v.z, v.w);
    }
  }
}

// The NI rows of one block of a compacted live-slot list through a buffer
// resource: row i of this lane is list entry e0 + i * RPI (slot lid[e], at
// byte offset slot * D * esize + lane_byte_off); entries past n get an offset
// past the resource's num_records, which the buffer load answers with zeros
// and no memory request (no branch: the load stream and its wait counts are
// those of a full block).  Cache policy 2 = nontemporal, as in ld_block.
constexpr int kDeadOffset = 0x7ffffff0;

template <int DT, int NI, int D, int RPI>
__device__ __forceinline__ void ld_block_list(Raw8<DT> (&r)[NI], __amdgpu_buffer_rsrc_t rsrc, const uint16_t* lid,
                                              int e0, int n, int lane_byte_off) {
  constexpr int kEsz = DT == YH_F32 ? 4 : 2;
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int e = e0 + i * RPI;
    const int o = e < n ? static_cast<int>(lid[e < n ? e : 0]) * D * kEsz + lane_byte_off : kDeadOffset;
#pragma unroll
    for (int j = 0; j < (DT == YH_F32 ? 2 : 1); ++j) {
      const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(rsrc, o + j * 16, 0, 2);
      r[i].w[j] = make_uint4(v.x, v.y, v.z, v.w);
    }
  }
}

template <int DT>
__device__ __forceinline__ void zero_raw8(Raw8<DT>& r) {
#pragma unroll
  for (int j = 0; j < (DT == YH_F32 ? 2 : 1); ++j) r.w[j] = make_uint4(0, 0, 0, 0);
}
template <int DT>
__device__ __forceinline__ void cvt8(const Raw8<DT>& r, float* f) {
  if constexpr (DT == YH_F32) {
    const uint32_t u[8] = {r.w[0].x, r.w[0].y, r.w[0].z, r.w[0].w, r.w[1].x, r.w[1].y, r.w[1].z, r.w[1].w};
#pragma unroll
    for (int j = 0; j < 8; ++j) f[j] = __uint_as_float(u[j]);
  } else {
    const uint32_t u[4] = {r.w[0].x, r.w[0].y, r.w[0].z, r.w[0].w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if constexpr (DT == YH_BF16) {
        f[2 * j] = __uint_as_float(u[j] << 16);
        f[2 * j + 1] = __uint_as_float(u[j] & 0xffff0000u);
      } else {
        f[2 * j] = f16_to_f32(u[j] & 0xffff);
        f[2 * j + 1] = f16_to_f32(u[j] >> 16);
      }
    }
  }
}

// One workgroup per (batch row, group), one pass over the slots.  Its waves
// take BS-slot blocks (32, or 16 for a capacity that is an odd multiple of
// 16) in turn.  Within a block LPR = D/8 lanes cover one row (8 elements
// each) and a wave instruction covers RPI = 64/LPR rows, so NI = BS/RPI
// instructions cover the block; a reduce-scatter butterfly over the
// LPR lanes leaves the logit of slot i*RPI + rr on the F = LPR/NI lanes
// s = i*F .. i*F + F-1 of row group rr.  Loads are unconditional and
// software-pipelined: the keys (and positions) of a wave's next block are
// requested as soon as the current logits are formed, its values as soon as
// the current P.V is done, so every wave keeps a block of keys and a block of
// values in flight while it computes (a conditional load would make the
// compiler wait for every load in flight).  A dead slot (position < 0) gets
// logit -inf and a zero value row, so stale or uninitialised contents never
// reach the sum.  Past its last block a wave re-reads that block (a cache hit).
// Each wave keeps a running (max, sum, P.V) over its blocks (online softmax);
// waves are combined at the end together with the sink logit 0, which has
// value 0:
//   out = sum_w acc_w e^{m_w - M} / (e^{-M} + sum_w l_w e^{m_w - M}),
//   M = max(0, max_w m_w).
// Waves per workgroup: 2 for one head per memory (its 256-slot pass is short:
// each wave then keeps its pipeline over twice the blocks) and for four heads
// per memory (128 rows x 8 memories: the 1024-slot window ring and the
// 256-slot anchor memory read in 92.9 us and 27.2 us with two waves, against
// 97.0 us and 34.1 us with four); 4 for two heads.
template <int R> constexpr int read_waves() { return R == 2 ? 4 : 2; }

//
// SKIP (anchor memories of at most 256 slots, one or two heads each): a wave fetches its first
// block whole while every slot position of (b, g) arrives; then each wave
// compacts the live slots past the waves' first blocks into a list in LDS
// (ballot + popcount ranks) and the later steps take BS list entries at a
// time (ld_block_list).  The read moves the live slots' bytes plus the dead
// rows of the first blocks, and takes ceil(live / BS) list steps.
constexpr int kSkipMaxCap = 256;

// SKIP takes 16-slot blocks (kSkipBS) and a register budget of four waves
// per SIMD: at 64 rows x 32 memories that keeps all 2048 two-wave workgroups
// resident at once (8 per CU), each wave with 16 key and 16 value rows in
// flight -- 39.7 us per read against 43.4 us for 32-slot blocks at two waves
// per SIMD and 41.3 us at three.  Two heads per memory fit three waves per
// SIMD without spilling.  Four heads per memory (128 rows x 8 memories) take
// 16-slot blocks at three waves per SIMD (kR4BS): 92.9 us for the 1024-slot
// window ring and 27.2 us for the 256-slot anchor memory, against 95.3 us and
// 31.0 us with 32-slot blocks at two (fp32 rows, twice the registers: at two).
// The other reads without SKIP: two waves per SIMD (each wave keeps a block
// of keys and one of values in flight).
constexpr int kSkipBS = 16;
constexpr int kR4BS = 16;
template <int DT, int R, bool SKIP> constexpr int read_occupancy() {
  return DT == YH_F32 ? 2 : SKIP ? (R == 1 ? 4 : 3) : R == 4 ? 3 : 2;
}

template <int DT, int D, int R, bool SINK, int BS, bool SKIP>
__global__ void __launch_bounds__((read_waves<R>() * 64))
__attribute__((amdgpu_waves_per_eu(read_occupancy<DT, R, SKIP>(), read_occupancy<DT, R, SKIP>())))
anchor_read_kernel(ReadArgs a) {
  constexpr int kReadWaves = read_waves<R>();
  constexpr int kReadThreads = kReadWaves * 64;
  constexpr int LPR = D / 8;
  constexpr int RPI = kWave / LPR;
  constexpr int NI = BS / RPI;
  constexpr int F = LPR / NI;
  static_assert(NI * RPI == BS && F * NI == LPR && F >= 1 && BS <= 32, "slot blocks");
  // window reads skip whole blocks without a live slot (a ring fills from slot
  // 0, so a sequence shorter than the window leaves its tail blocks dead)
  constexpr bool BSKIP = !SINK;
  static_assert(kMaxCap / 16 <= 64 && kMaxCap % 64 == 0, "one bit per block");

  __shared__ float wm[kReadWaves][R];
  __shared__ float wl[kReadWaves][R];
  __shared__ float accs[kReadWaves][R][D];
  __shared__ uint16_t lidx[SKIP ? kReadWaves : 1][SKIP ? kSkipMaxCap : 1];

  const int bg = blockIdx.x;
  const int row = bg / a.G, g = bg % a.G;
  const int H = a.G * R;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: the block loop runs on scalar branches
  const int s = lane % LPR, rr = lane / LPR;
  const int64_t b = a.idx ? static_cast<int64_t>(a.idx[row]) : static_cast<int64_t>(row);
  const int64_t qbase = (static_cast<int64_t>(row) * H + static_cast<int64_t>(g) * R) * D;
  if (b < 0 || b >= a.n_rows) {  // reads nothing: 0 (x any gate is 0)
    for (int e = tid; e < R * D; e += kReadThreads) store_any(a.out, qbase + e, DT, 0.f);
    return;
  }
  const int32_t* pos = a.pos + b * a.p_rs + static_cast<int64_t>(g) * a.KC;  // slots of (b, g)
  constexpr int kEsz = DT == YH_F32 ? 4 : 2;
  const char* kptr = static_cast<const char*>(a.keys) +
                     (b * a.k_rs + static_cast<int64_t>(g) * a.KC * D + rr * D + s * 8) * kEsz;
  const char* vptr = static_cast<const char*>(a.values) +
                     (b * a.v_rs + static_cast<int64_t>(g) * a.KC * D + rr * D + s * 8) * kEsz;

  // 16-bit queries stay packed (dot2 instructions take bf16 / fp16 pairs and
  // accumulate in fp32; the 1/sqrt(D) scale is applied to the summed logit);
  // fp32 queries are pre-scaled
  Raw8<DT> qraw[R];
  float qf[DT == YH_F32 ? R : 1][8];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    ld_raw8<DT>(qraw[r], a.q, qbase + static_cast<int64_t>(r) * D + s * 8);
    if constexpr (DT == YH_F32) {
      cvt8<DT>(qraw[r], qf[r]);
#pragma unroll
      for (int j = 0; j < 8; ++j) qf[r][j] *= a.scale;
    }
  }

  float m_run[R], l_run[R], acc[R][8];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    m_run[r] = -INFINITY;
    l_run[r] = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[r][j] = 0.f;
  }

  const int nblk = a.KC / BS;
  __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(nullptr, 0, 0, 0x00020000), vrs = krs;
  if constexpr (SKIP) {
    const int bytes = a.KC * D * kEsz;
    krs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<char*>(static_cast<const char*>(a.keys) + (b * a.k_rs + static_cast<int64_t>(g) * a.KC * D) * kEsz),
        0, bytes, 0x00020000);
    vrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<char*>(static_cast<const char*>(a.values) + (b * a.v_rs + static_cast<int64_t>(g) * a.KC * D) * kEsz),
        0, bytes, 0x00020000);
  }
  const uint16_t* lid = lidx[SKIP ? wid : 0];
  const int lane_off = s * 8 * kEsz;
  if (wid < nblk) {  // uniform over the wave
    Raw8<DT> kr[NI], vr[NI];
    // same issue order as the loop (positions, keys, values), so the wait
    // counts derived at the loop head are those of the steady state; the
    // first block is fetched whole
    // SKIP: every position of (b, g) is requested first; the vector-memory
    // counter is in order, so the ballots below wait for these loads only
    // BSKIP: the same for every slot of the ring (up to kMaxCap)
    int32_t pv[SKIP ? kSkipMaxCap / 64 : BSKIP ? kMaxCap / 64 : 1];
    if constexpr (SKIP || BSKIP) {
#pragma unroll
      for (int c = 0; c < (SKIP ? kSkipMaxCap : kMaxCap) / 64; ++c) {
        const int slot = c * 64 + lane;
        pv[c] = pos[slot < a.KC ? slot : 0] | (slot < a.KC ? 0 : int32_t(0x80000000));
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    int32_t pcur = pos[wid * BS + (lane & (BS - 1))];
    ld_block<DT, NI, RPI * D>(kr, kptr + static_cast<int64_t>(wid * BS) * D * kEsz);
    __builtin_amdgcn_sched_barrier(0);
    ld_block<DT, NI, RPI * D>(vr, vptr + static_cast<int64_t>(wid * BS) * D * kEsz);
    __builtin_amdgcn_sched_barrier(0);
    // SKIP: the list of live slots past the waves' first blocks (slots below
    // kReadWaves * BS are fetched whole)
    int n_list = 0;
    if constexpr (SKIP) {
      const uint64_t below = lane ? (~0ull >> (64 - lane)) : 0ull;  // lanes under this one
#pragma unroll
      for (int c = 0; c < kSkipMaxCap / 64; ++c) {
        const bool lv = pv[c] >= 0 && c * 64 + lane >= kReadWaves * BS;
        const uint64_t m = __ballot(lv);
        if (lv) lidx[wid][n_list + __popcll(m & below)] = static_cast<uint16_t>(c * 64 + lane);
        n_list += __popcll(m);
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    const int n_lblk = (n_list + BS - 1) / BS;
    // one block step: logits of the rows in kr, the next keys (next_k), the
    // online softmax and P.V of the rows in vr, the next values (next_v)
    auto step_block = [&](Raw8<DT> (&kb)[NI], Raw8<DT> (&vb)[NI], uint32_t live, auto&& next_k,
                          auto&& next_v) {
      float part[R][NI];
#pragma unroll
        for (int i = 0; i < NI; ++i) {
          if constexpr (DT == YH_F32) {
            float kf[8];
            cvt8<DT>(kb[i], kf);
#pragma unroll
            for (int r = 0; r < R; ++r) {
              float x = 0.f;
#pragma unroll
              for (int j = 0; j < 8; ++j) x = fmaf(qf[r][j], kf[j], x);
              part[r][i] = x;
            }
          } else {
#pragma unroll
            for (int r = 0; r < R; ++r) part[r][i] = dot8<DT>(qraw[r], kb[i]);
          }
        }
      // the keys (and positions) of the next block (sched_barrier: issued
      // here, not sunk to their use in the next step)
      __builtin_amdgcn_sched_barrier(0);
      next_k();
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int m = LPR / 2, h = NI / 2; m >= 1; m >>= 1, h >>= 1) {
          if (h >= 1) {
            const bool up = (s & m) != 0;
#pragma unroll
            for (int r = 0; r < R; ++r) {
#pragma unroll
              for (int j = 0; j < h; ++j) {
                const float send = up ? part[r][j] : part[r][j + h];
                const float keep = up ? part[r][j + h] : part[r][j];
                part[r][j] = keep + __shfl_xor(send, m, kWave);
              }
            }
          } else {
#pragma unroll
            for (int r = 0; r < R; ++r) part[r][0] += __shfl_xor(part[r][0], m, kWave);
          }
        }
        // lane (s, rr) holds the logit of slot (s / F) * RPI + rr
        const bool mine_live = (live >> ((s / F) * RPI + rr)) & 1u;
        const bool counts = (s % F) == 0;  // one lane of the F copies enters the sum
        float pw[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const float logit = mine_live ? (DT == YH_F32 ? part[r][0] : part[r][0] * a.scale) : -INFINITY;
          const float bm = wave_max(logit);
          const float m_new = fmaxf(m_run[r], bm);
          const float m_safe = m_new == -INFINITY ? 0.f : m_new;
          const float alpha = __expf(m_run[r] - m_safe);
          const float p = __expf(logit - m_safe);
          l_run[r] = l_run[r] * alpha + wave_sum(counts ? p : 0.f);
          m_run[r] = m_new;
#pragma unroll
          for (int j = 0; j < 8; ++j) acc[r][j] *= alpha;
          pw[r] = p;
        }
        // P.V: each value row is converted once and used for all R heads
#pragma unroll
        for (int i = 0; i < NI; ++i) {
          float vf[8];
          cvt8<DT>(vb[i], vf);
          const bool vlive = (live >> (i * RPI + rr)) & 1u;
#pragma unroll
          for (int j = 0; j < 8; ++j) vf[j] = vlive ? vf[j] : 0.f;
#pragma unroll
          for (int r = 0; r < R; ++r) {
            // weight of the row this lane loaded at instruction i (slot i*RPI + rr)
            const float w = __shfl(pw[r], rr * LPR + i * F, kWave);
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[r][j] = fmaf(w, vf[j], acc[r][j]);
          }
        }
      // the values of the next block
      __builtin_amdgcn_sched_barrier(0);
      next_v();
      __builtin_amdgcn_sched_barrier(0);
    };
    if constexpr (SKIP) {
      uint32_t live = static_cast<uint32_t>(__ballot(pcur >= 0));  // the whole first block
      for (int step = 0;; ++step) {  // step k >= 1 is list block wid + kReadWaves * (k - 1)
        const int nb = wid + kReadWaves * step;  // the list block of the next step
        const bool more = nb < n_lblk;
        const int e_next = more ? nb * BS + rr : n_list;  // past the list: nothing is fetched
        const int rem = n_list - nb * BS;
        const uint32_t lnxt = !more ? 0u : rem >= 32 ? 0xffffffffu : (1u << rem) - 1u;
        step_block(kr, vr, live, [&] { ld_block_list<DT, NI, D, RPI>(kr, krs, lid, e_next, n_list, lane_off); },
                   [&] { ld_block_list<DT, NI, D, RPI>(vr, vrs, lid, e_next, n_list, lane_off); });
        if (!more) break;
        live = lnxt;
      }
    } else {
      // BSKIP: this wave's blocks (blk = wid mod kReadWaves) that hold a live
      // slot; the others are never fetched.  A dead block is a no-op of the
      // online softmax (its logits are -inf, its values 0), so the sum is the
      // one over every block, bit for bit.
      uint64_t mine = 0;
      if constexpr (BSKIP) {
        constexpr uint64_t kBlkBits = (1ull << BS) - 1;
#pragma unroll
        for (int c = 0; c < kMaxCap / 64; ++c) {
          const uint64_t m = __ballot(pv[c] >= 0);
#pragma unroll
          for (int j = 0; j < 64 / BS; ++j)
            mine |= static_cast<uint64_t>(((m >> (j * BS)) & kBlkBits) != 0) << (c * (64 / BS) + j);
        }
        uint64_t res = 0;  // bits wid, wid + kReadWaves, ...
#pragma unroll
        for (int j = 0; j < 64; j += kReadWaves) res |= 1ull << j;
        mine &= res << wid;
      }
      for (int blk = wid; blk < nblk;) {
        int nb = blk + kReadWaves;
        if constexpr (BSKIP) {
          const uint64_t rest = mine & ~((2ull << blk) - 1);  // live blocks of this wave past blk
          nb = rest ? static_cast<int>(__builtin_ctzll(rest)) : nblk;
        }
        const int nxt = (nb < nblk ? nb : blk) * BS;  // past the end: this block again
        const uint32_t live = static_cast<uint32_t>(__ballot(pcur >= 0));
        step_block(kr, vr, live,
                   [&] {
                     pcur = pos[nxt + (lane & (BS - 1))];
                     ld_block<DT, NI, RPI * D>(kr, kptr + static_cast<int64_t>(nxt) * D * kEsz);
                   },
                   [&] { ld_block<DT, NI, RPI * D>(vr, vptr + static_cast<int64_t>(nxt) * D * kEsz); });
        blk = nb;
      }
    }
  }
#pragma unroll
  for (int off = LPR; off < kWave; off <<= 1)
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[r][j] += __shfl_xor(acc[r][j], off, kWave);
  if (rr == 0) {
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int j = 0; j < 8; ++j) accs[wid][r][s * 8 + j] = acc[r][j];
  }
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      wm[wid][r] = m_run[r];
      wl[wid][r] = l_run[r];
    }
  }
  __syncthreads();
  for (int e = tid; e < R * D; e += kReadThreads) {
    const int r = e / D, d = e % D;
    float mx = SINK ? 0.f : -INFINITY;  // the sink logit is 0
#pragma unroll
    for (int w = 0; w < kReadWaves; ++w) mx = fmaxf(mx, wm[w][r]);
    const float ms = mx == -INFINITY ? 0.f : mx;  // no live slot and no sink
    float den = SINK ? __expf(-ms) : 0.f, x = 0.f;
#pragma unroll
    for (int w = 0; w < kReadWaves; ++w) {
      const float f = __expf(wm[w][r] - ms);  // 0 for a wave with no live slot
      den = fmaf(wl[w][r], f, den);
      x = fmaf(accs[w][r][d], f, x);
    }
    const float o = den > 0.f ? x / den : 0.f;
    store_any(a.out, qbase + e, DT, read_epilogue<DT>(a, row, H, g * R + r, d, o));
  }
}

// ---------------------------------------------------------------------------
struct CommitArgs {
  const void* key;          // [B, G, D]
  const void* value;        // [B, G, D]
  const float* score;       // [B, G]
  const uint8_t* active;    // [B]
  const int32_t* idx;       // [B] or null
  void* keys;               // [NB, G, KC, D]
  void* values;
  float* scores;            // [NB, G, KC]
  int32_t* pos;             // [NB, G, KC]
  void* pkeys;              // [NB, G, PC, D]
  void* pvalues;
  float* pscores;           // [NB, G, PC]
  const int64_t* count;     // [NB]
  const int64_t* total;     // [NB]
  int B, G, KC, PC, C, D, esize;
  int64_t n_rows;
  int64_t rs[9];  // row strides (elements) in IndependentMemoryState field order
  int64_t key_rs, value_rs;  // elements between batch rows of key / value
};

enum { kRsKeys, kRsValues, kRsScores, kRsPos, kRsPKeys, kRsPValues, kRsPScores, kRsCount, kRsTotal };

constexpr int kCommitThreads = 512;
constexpr int kMaxCand = 2048;
constexpr int kMaxPieces = 16;  // 16-byte pieces per thread per tensor: 128 KiB per (row, group)

// Copy `n` bytes (multiple of 16) between two 16-byte aligned rows.
__device__ __forceinline__ void copy_row16(void* dst, const void* src, int n, int lane, int lanes) {
  const uint4* s = static_cast<const uint4*>(src);
  uint4* d = static_cast<uint4*>(dst);
  for (int i = lane; i < n / 16; i += lanes) d[i] = s[i];
}

// Gather every selected row of one tensor into registers, then (after a
// barrier) write them over the committed rows.  Sources include the committed
// rows themselves, so no row may be written before all are read.
__device__ __forceinline__ void commit_gather_pass(char* committed, const char* pending, const int32_t* chosen,
                                                   const int32_t* cpos, int KC, int chunks, int total_pieces,
                                                   int64_t rowbytes) {
  const int tid = threadIdx.x;
  uint4 buf[kMaxPieces];
#pragma unroll
  for (int i = 0; i < kMaxPieces; ++i) {
    const int piece = tid + i * kCommitThreads;
    buf[i] = make_uint4(0, 0, 0, 0);
    if (piece < total_pieces) {
      const int slot = piece / chunks, c = piece % chunks;
      const int src = chosen[slot];
      // an invalid selection reads committed row 0, as the reference does
      const char* from = cpos[src] < 0 ? committed
                         : (src < KC ? committed + src * rowbytes : pending + (src - KC) * rowbytes);
      buf[i] = reinterpret_cast<const uint4*>(from)[c];
    }
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kMaxPieces; ++i) {
    const int piece = tid + i * kCommitThreads;
    if (piece < total_pieces) {
      const int slot = piece / chunks, c = piece % chunks;
      reinterpret_cast<uint4*>(committed + slot * rowbytes)[c] = buf[i];
    }
  }
}

// One workgroup per (batch row, group).  Push the token into pending[count];
// on a full chunk rank the KC + C candidates by counting (score desc, position
// asc with invalid last, candidate index asc) and rewrite the committed slots.
// count / total are only read here (every group of a row reads them); the
// advance kernel updates them afterwards.
__global__ void __launch_bounds__(kCommitThreads) anchor_commit_kernel(CommitArgs a) {
  __shared__ uint64_t ckey[kMaxCand];   // (~score_key << 32) | position key
  __shared__ float cscore[kMaxCand];
  __shared__ int32_t cpos[kMaxCand];
  __shared__ int32_t chosen[kMaxCand];

  const int bg = blockIdx.x;
  const int row = bg / a.G, g = bg % a.G;
  const int tid = threadIdx.x;
  const int64_t b = a.idx ? static_cast<int64_t>(a.idx[row]) : static_cast<int64_t>(row);
  if (b < 0 || b >= a.n_rows || a.active[row] == 0) return;
  const int64_t cnt = a.count[b * a.rs[kRsCount]];
  if (cnt < 0 || cnt >= a.C) return;  // corrupt counter: leave the row untouched
  const int64_t rowbytes = static_cast<int64_t>(a.D) * a.esize;
  char* pk = static_cast<char*>(a.pkeys) + b * a.rs[kRsPKeys] * a.esize + static_cast<int64_t>(g) * a.PC * rowbytes;
  char* pv = static_cast<char*>(a.pvalues) + b * a.rs[kRsPValues] * a.esize + static_cast<int64_t>(g) * a.PC * rowbytes;
  const char* src_k = static_cast<const char*>(a.key) + (row * a.key_rs + static_cast<int64_t>(g) * a.D) * a.esize;
  const char* src_v = static_cast<const char*>(a.value) + (row * a.value_rs + static_cast<int64_t>(g) * a.D) * a.esize;
  float* ps = a.pscores + b * a.rs[kRsPScores] + static_cast<int64_t>(g) * a.PC;
  const float new_score = a.score[static_cast<int64_t>(row) * a.G + g];
  // push
  if (tid < 64) copy_row16(pk + cnt * rowbytes, src_k, static_cast<int>(rowbytes), tid, 64);
  else if (tid < 128) copy_row16(pv + cnt * rowbytes, src_v, static_cast<int>(rowbytes), tid - 64, 64);
  else if (tid == 128) ps[cnt] = new_score;
  if (cnt + 1 != a.C) return;  // uniform over the workgroup
  __syncthreads();             // the pushed row is visible to the whole workgroup

  const int KC = a.KC, C = a.C, N = KC + C;
  float* scores = a.scores + b * a.rs[kRsScores] + static_cast<int64_t>(g) * KC;
  int32_t* pos = a.pos + b * a.rs[kRsPos] + static_cast<int64_t>(g) * KC;
  const int64_t base_pos = a.total[b * a.rs[kRsTotal]] - cnt;
  for (int n = tid; n < N; n += kCommitThreads) {
    float sc;
    int32_t p;
    if (n < KC) {
      sc = scores[n];
      p = pos[n];
      if (p < 0) p = -1;
    } else {
      sc = n - KC == cnt ? new_score : ps[n - KC];
      p = static_cast<int32_t>(base_pos + (n - KC));
    }
    ckey[n] = topk_key(sc, p);
    cscore[n] = sc;
    cpos[n] = p;
  }
  __syncthreads();
  for (int n = tid; n < N; n += kCommitThreads) {
    const uint64_t mine = ckey[n];
    int rank = 0;
    for (int j = 0; j < N; ++j) {
      const uint64_t o = ckey[j];
      rank += (o < mine) | ((o == mine) & (j < n));
    }
    if (rank < KC) chosen[rank] = n;
  }
  __syncthreads();
  // Keys, then values: gather every selected row of the tensor into registers
  // before any committed row of it is overwritten (the sources include the
  // committed rows themselves), then write them back.
  const int chunks = static_cast<int>(rowbytes / 16);  // 16-byte pieces per row
  const int total_pieces = KC * chunks;
  char* ck = static_cast<char*>(a.keys) + b * a.rs[kRsKeys] * a.esize + static_cast<int64_t>(g) * KC * rowbytes;
  char* cv = static_cast<char*>(a.values) + b * a.rs[kRsValues] * a.esize + static_cast<int64_t>(g) * KC * rowbytes;
  commit_gather_pass(ck, pk, chosen, cpos, KC, chunks, total_pieces, rowbytes);
  commit_gather_pass(cv, pv, chosen, cpos, KC, chunks, total_pieces, rowbytes);
  for (int n = tid; n < KC; n += kCommitThreads) {
    const int src = chosen[n];
    scores[n] = cscore[src];
    pos[n] = cpos[src];
  }
}

// count = (count + active) % C, total += active, once per state row.
__global__ void anchor_advance_kernel(int64_t* count, int64_t* total, const uint8_t* active,
                                      const int32_t* idx, int B, int C, int64_t n_rows, int64_t count_rs,
                                      int64_t total_rs) {
  const int row = blockIdx.x * blockDim.x + threadIdx.x;
  if (row >= B) return;
  const int64_t b = idx ? static_cast<int64_t>(idx[row]) : static_cast<int64_t>(row);
  if (b < 0 || b >= n_rows) return;
  const int64_t act = active[row] ? 1 : 0;
  const int64_t c = count[b * count_rs] + act;
  count[b * count_rs] = c == C ? 0 : c;
  total[b * total_rs] += act;
}

// 32-slot blocks, or 16-slot blocks for a capacity that is an odd multiple of 16.
template <int DT, int D, bool SINK, int BS>
int launch_read_r(int R, const ReadArgs& a, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>(static_cast<int64_t>(a.B) * a.G));
  const dim3 b1(read_waves<1>() * 64), b2(read_waves<2>() * 64), b4(read_waves<4>() * 64);
  // anchor memories of up to 256 slots read by one or two heads fetch live
  // rows only (four heads' state leaves no registers for the list step)
  const bool skip = SINK && a.KC <= kSkipMaxCap && R <= 2;
  switch (R * 2 + (skip ? 1 : 0)) {
    case 2: hipLaunchKernelGGL((anchor_read_kernel<DT, D, 1, SINK, BS, false>), grid, b1, 0, st, a); break;
    case 3: hipLaunchKernelGGL((anchor_read_kernel<DT, D, 1, SINK, kSkipBS, SINK>), grid, b1, 0, st, a); break;
    case 4: hipLaunchKernelGGL((anchor_read_kernel<DT, D, 2, SINK, BS, false>), grid, b2, 0, st, a); break;
    case 5: hipLaunchKernelGGL((anchor_read_kernel<DT, D, 2, SINK, kSkipBS, SINK>), grid, b2, 0, st, a); break;
    case 8: hipLaunchKernelGGL((anchor_read_kernel<DT, D, 4, SINK, kR4BS, false>), grid, b4, 0, st, a); break;
    default: set_error("anchor_read: heads per group must be 1, 2 or 4 (got %d)", R); return YH_ERR_INVALID;
  }
  YH_CHECK_LAUNCH("anchor_read");
  return YH_OK;
}

template <int DT, int D>
int launch_read_b(int R, bool sink, const ReadArgs& a, hipStream_t st) {
  if (a.KC % 32 == 0)
    return sink ? launch_read_r<DT, D, true, 32>(R, a, st) : launch_read_r<DT, D, false, 32>(R, a, st);
  return sink ? launch_read_r<DT, D, true, 16>(R, a, st) : launch_read_r<DT, D, false, 16>(R, a, st);
}

template <int DT>
int launch_read_d(int D, int R, bool sink, const ReadArgs& a, hipStream_t st) {
  if (D == 128) return launch_read_b<DT, 128>(R, sink, a, st);
  if (D == 64) return launch_read_b<DT, 64>(R, sink, a, st);
  set_error("anchor_read: head dim must be 64 or 128 (got %d)", D);
  return YH_ERR_INVALID;
}

}  // namespace
}  // namespace yh

static int anchor_read_impl(bool sink, const void* query, const void* keys, const void* values,
                              const int32_t* positions, const int32_t* indices, void* out,
                              int64_t B, int64_t H, int64_t G, int64_t capacity, int64_t D,
                              int64_t n_state_rows, int64_t keys_rs, int64_t values_rs, int64_t positions_rs,
                              int dtype, yh_stream_t stream, const uint8_t* row_valid = nullptr,
                              const float* head_gate = nullptr, const void* gate = nullptr, int64_t gate_ts = 0,
                              int64_t gate_hs = 0) {
  using namespace yh;
  YH_CHECK_ARG(query && keys && values && positions && out, "anchor_read: null tensor pointer");
  YH_CHECK_ARG(B >= 0 && G > 0 && H > 0 && H % G == 0, "anchor_read: bad B/H/G (%lld/%lld/%lld)",
               (long long)B, (long long)H, (long long)G);
  YH_CHECK_ARG(capacity > 0 && capacity % 16 == 0 && capacity <= kMaxCap,
               "anchor_read: capacity must be a positive multiple of 16 up to %d (got %lld)", kMaxCap,
               (long long)capacity);
  YH_CHECK_ARG(is_float_dtype(dtype), "anchor_read: unsupported dtype %d", dtype);
  YH_CHECK_ARG(indices != nullptr || n_state_rows >= B, "anchor_read: state has fewer rows than the batch");
  YH_CHECK_ARG(B * G < (1LL << 31), "anchor_read: grid too large");
  const uintptr_t al = 15;
  YH_CHECK_ARG(((reinterpret_cast<uintptr_t>(query) | reinterpret_cast<uintptr_t>(keys) |
                 reinterpret_cast<uintptr_t>(values)) & al) == 0,
               "anchor_read: query/keys/values must be 16-byte aligned");
  const int64_t dense_kv = G * capacity * D, dense_pos = G * capacity;
  if (keys_rs == 0) keys_rs = dense_kv;
  if (values_rs == 0) values_rs = dense_kv;
  if (positions_rs == 0) positions_rs = dense_pos;
  YH_CHECK_ARG(keys_rs >= dense_kv && values_rs >= dense_kv && positions_rs >= dense_pos,
               "anchor_read: a row stride is smaller than one state row");
  const int64_t esz = dtype == YH_F32 ? 4 : 2;
  YH_CHECK_ARG((keys_rs * esz) % 16 == 0 && (values_rs * esz) % 16 == 0,
               "anchor_read: key/value row strides must keep 16-byte alignment");
  if (B == 0) return YH_OK;
  ReadArgs a{query, keys, values, positions, indices, out, (int)B, (int)G, (int)capacity, n_state_rows,
             keys_rs, values_rs, positions_rs, 1.0f / sqrtf(static_cast<float>(D)), row_valid, head_gate, gate,
             gate_ts, gate_hs};
  const int R = static_cast<int>(H / G);
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case YH_BF16: return launch_read_d<YH_BF16>((int)D, R, sink, a, st);
    case YH_F16: return launch_read_d<YH_F16>((int)D, R, sink, a, st);
    default: return launch_read_d<YH_F32>((int)D, R, sink, a, st);
  }
}

extern "C" int yh_anchor_read(const void* query, const void* keys, const void* values, const int32_t* positions,
                              const int32_t* indices, void* out, int64_t B, int64_t H, int64_t G, int64_t capacity,
                              int64_t D, int64_t n_state_rows, int64_t keys_row_stride, int64_t values_row_stride,
                              int64_t positions_row_stride, int dtype, yh_stream_t stream) {
  return anchor_read_impl(true, query, keys, values, positions, indices, out, B, H, G, capacity, D, n_state_rows,
                          keys_row_stride, values_row_stride, positions_row_stride, dtype, stream);
}

extern "C" int yh_window_attend(const void* query, const void* keys, const void* values, const int32_t* positions,
                                const int32_t* indices, void* out, int64_t B, int64_t H, int64_t G, int64_t window,
                                int64_t D, int64_t n_state_rows, int dtype, yh_stream_t stream) {
  return anchor_read_impl(false, query, keys, values, positions, indices, out, B, H, G, window, D, n_state_rows,
                          0, 0, 0, dtype, stream);
}

extern "C" int yh_anchor_read_gated(const void* query, const void* keys, const void* values,
                                    const int32_t* positions, const int32_t* indices, void* out, int64_t B, int64_t H,
                                    int64_t G, int64_t capacity, int64_t D, int64_t n_state_rows,
                                    int64_t keys_row_stride, int64_t values_row_stride, int64_t positions_row_stride,
                                    const uint8_t* row_valid, const float* head_gate, int dtype,
                                    yh_stream_t stream) {
  return anchor_read_impl(true, query, keys, values, positions, indices, out, B, H, G, capacity, D, n_state_rows,
                          keys_row_stride, values_row_stride, positions_row_stride, dtype, stream, row_valid,
                          head_gate);
}

extern "C" int yh_window_attend_gated(const void* query, const void* keys, const void* values,
                                      const int32_t* positions, const int32_t* indices, void* out, int64_t B,
                                      int64_t H, int64_t G, int64_t window, int64_t D, int64_t n_state_rows,
                                      const void* gate, int64_t gate_tok_stride, int64_t gate_head_stride, int dtype,
                                      yh_stream_t stream) {
  if (!gate) {
    yh::set_error("window_attend_gated: gate required");
    return YH_ERR_INVALID;
  }
  return anchor_read_impl(false, query, keys, values, positions, indices, out, B, H, G, window, D, n_state_rows, 0,
                          0, 0, dtype, stream, nullptr, nullptr, gate, gate_tok_stride, gate_head_stride);
}

extern "C" int yh_anchor_commit(const void* key, const void* value, const float* score,
                                const uint8_t* active, const int32_t* indices, void* keys, void* values,
                                float* scores, int32_t* positions, void* pending_keys,
                                void* pending_values, float* pending_scores, int64_t* count,
                                int64_t* total, int64_t B, int64_t G, int64_t capacity,
                                int64_t pending_capacity, int64_t chunk, int64_t D, int64_t n_state_rows,
                                const int64_t* row_strides, int64_t key_row_stride, int64_t value_row_stride,
                                int dtype, yh_stream_t stream) {
  using namespace yh;
  YH_CHECK_ARG(key && value && score && active && keys && values && scores && positions && pending_keys &&
                   pending_values && pending_scores && count && total,
               "anchor_commit: null tensor pointer");
  YH_CHECK_ARG(B >= 0 && G > 0 && capacity > 0 && D > 0, "anchor_commit: bad sizes");
  YH_CHECK_ARG(chunk >= 1 && chunk <= pending_capacity, "anchor_commit: chunk %lld outside [1, %lld]",
               (long long)chunk, (long long)pending_capacity);
  YH_CHECK_ARG(capacity + chunk <= kMaxCand, "anchor_commit: capacity + chunk must be <= %d", kMaxCand);
  YH_CHECK_ARG(is_float_dtype(dtype), "anchor_commit: unsupported dtype %d", dtype);
  const int esize = dtype == YH_F32 ? 4 : 2;
  YH_CHECK_ARG((D * esize) % 16 == 0, "anchor_commit: a row must be a multiple of 16 bytes");
  YH_CHECK_ARG(capacity * D * esize <= static_cast<int64_t>(kCommitThreads) * kMaxPieces * 16,
               "anchor_commit: capacity x row bytes exceeds %d", kCommitThreads * kMaxPieces * 16);
  YH_CHECK_ARG(indices != nullptr || n_state_rows >= B, "anchor_commit: state has fewer rows than the batch");
  YH_CHECK_ARG(((reinterpret_cast<uintptr_t>(key) | reinterpret_cast<uintptr_t>(value) |
                 reinterpret_cast<uintptr_t>(keys) | reinterpret_cast<uintptr_t>(values) |
                 reinterpret_cast<uintptr_t>(pending_keys) | reinterpret_cast<uintptr_t>(pending_values)) & 15) == 0,
               "anchor_commit: key/value rows must be 16-byte aligned");
  YH_CHECK_ARG(B * G < (1LL << 31), "anchor_commit: grid too large");
  const int64_t dense[9] = {G * capacity * D, G * capacity * D, G * capacity, G * capacity,
                            G * pending_capacity * D, G * pending_capacity * D, G * pending_capacity, 1, 1};
  CommitArgs a{key, value, score, active, indices, keys, values, scores, positions, pending_keys, pending_values,
               pending_scores, count, total, (int)B, (int)G, (int)capacity, (int)pending_capacity, (int)chunk,
               (int)D, esize, n_state_rows, {}, key_row_stride > 0 ? key_row_stride : G * D,
               value_row_stride > 0 ? value_row_stride : G * D};
  YH_CHECK_ARG(a.key_rs >= G * D && a.value_rs >= G * D && (a.key_rs * esize) % 16 == 0 &&
                   (a.value_rs * esize) % 16 == 0,
               "anchor_commit: key/value batch rows must hold G x D elements and keep 16-byte alignment");
  for (int i = 0; i < 9; ++i) {
    a.rs[i] = row_strides ? row_strides[i] : dense[i];
    YH_CHECK_ARG(a.rs[i] >= dense[i], "anchor_commit: row stride %d (%lld) is smaller than one state row", i,
                 (long long)a.rs[i]);
  }
  for (int i : {(int)kRsKeys, (int)kRsValues, (int)kRsPKeys, (int)kRsPValues})
    YH_CHECK_ARG((a.rs[i] * esize) % 16 == 0, "anchor_commit: key/value row strides must keep 16-byte alignment");
  if (B == 0) return YH_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(anchor_commit_kernel, dim3(static_cast<unsigned>(B * G)), dim3(kCommitThreads), 0, st, a);
  YH_CHECK_LAUNCH("anchor_commit");
  const int threads = 256;
  hipLaunchKernelGGL(anchor_advance_kernel, dim3(static_cast<unsigned>((B + threads - 1) / threads)), dim3(threads),
                     0, st, count, total, active, indices, (int)B, (int)chunk, n_state_rows, a.rs[kRsCount],
                     a.rs[kRsTotal]);
  YH_CHECK_LAUNCH("anchor_advance");
  return YH_OK;
}
