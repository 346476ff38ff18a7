// HBM calibration streams: the rate a plain streaming kernel reaches on this
// GPU, measured beside the kernels' rooflines (their fractions are quoted
// against the 8 TB/s spec figure).  16-byte elements, one per lane per step,
// UNR steps in flight per lane, grid-stride over the buffer:
//   copy   dst <- src                      (bytes read + bytes written)
//   rmw    dst <- 0.5 dst + 1, in place    (read + write of one buffer)
//   read   sum of src, one float per workgroup into dst
//   write  dst <- constant
// each with plain or nontemporal loads and stores.  No counterpart in the
// reference: it is the measuring stick for the HBM-bound kernels here.
#include "common.h"

namespace yh {
namespace {

typedef float f32x4n __attribute__((ext_vector_type(4)));
constexpr int kCalThreads = 256, kCalUnr = 4;

template <bool NT>
__device__ __forceinline__ f32x4n cal_ld(const f32x4n* p) {
  if constexpr (NT) return __builtin_nontemporal_load(p);
  return *p;
}
template <bool NT>
__device__ __forceinline__ void cal_st(f32x4n v, f32x4n* p) {
  if constexpr (NT)
    __builtin_nontemporal_store(v, p);
  else
    *p = v;
}

// KIND 0 copy, 1 rmw, 2 read, 3 write
template <int KIND, bool NT>
__global__ void __launch_bounds__(kCalThreads) hbm_stream_kernel(const f32x4n* __restrict__ src,
                                                                 f32x4n* __restrict__ dst, int64_t n) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kCalThreads * kCalUnr;
  float s = 0.f;
  for (int64_t i0 = static_cast<int64_t>(blockIdx.x) * kCalThreads * kCalUnr + threadIdx.x; i0 < n; i0 += stride) {
    f32x4n v[kCalUnr];
    if constexpr (KIND != 3) {
#pragma unroll
      for (int u = 0; u < kCalUnr; ++u) {
        const int64_t i = i0 + u * kCalThreads;
        v[u] = i < n ? cal_ld<NT>((KIND == 1 ? dst : src) + i) : f32x4n{0.f, 0.f, 0.f, 0.f};
      }
    }
#pragma unroll
    for (int u = 0; u < kCalUnr; ++u) {
      const int64_t i = i0 + u * kCalThreads;
      if constexpr (KIND == 2) {
        s += (v[u].x + v[u].y) + (v[u].z + v[u].w);
      } else if constexpr (KIND == 3) {
        if (i < n) cal_st<NT>(f32x4n{1.f, 2.f, 3.f, static_cast<float>(u)}, dst + i);
      } else {
        if constexpr (KIND == 1) v[u] = v[u] * 0.5f + 1.f;
        if (i < n) cal_st<NT>(v[u], dst + i);
      }
    }
  }
  if constexpr (KIND == 2) {  // one partial sum per workgroup keeps the loads live
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
    __shared__ float ws[kCalThreads / 64];
    if ((threadIdx.x & 63) == 0) ws[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
      float t = 0.f;
      for (int w = 0; w < kCalThreads / 64; ++w) t += ws[w];
      reinterpret_cast<float*>(dst)[blockIdx.x] = t;
    }
  }
}

template <int KIND>
void launch_stream(bool nt, const f32x4n* src, f32x4n* dst, int64_t n, int grid, hipStream_t st) {
  if (nt)
    hipLaunchKernelGGL((hbm_stream_kernel<KIND, true>), dim3(grid), dim3(kCalThreads), 0, st, src, dst, n);
  else
    hipLaunchKernelGGL((hbm_stream_kernel<KIND, false>), dim3(grid), dim3(kCalThreads), 0, st, src, dst, n);
}

}  // namespace
}  // namespace yh

extern "C" int yh_hbm_stream(int kind, int nontemporal, const void* src, void* dst, int64_t bytes, int grid,
                             yh_stream_t stream) {
  using namespace yh;
  YH_CHECK_ARG(kind >= 0 && kind <= 3, "hbm_stream: kind must be 0 (copy), 1 (rmw), 2 (read) or 3 (write)");
  YH_CHECK_ARG(bytes > 0 && bytes % 16 == 0, "hbm_stream: bytes must be a positive multiple of 16");
  YH_CHECK_ARG(grid > 0 && grid <= (1 << 20), "hbm_stream: grid must be in 1 .. 2^20");
  YH_CHECK_ARG(dst && (kind == 1 || kind == 3 || src), "hbm_stream: null pointer");
  YH_CHECK_ARG(((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15) == 0,
               "hbm_stream: buffers must be 16-byte aligned");
  // read: dst receives one float per workgroup
  YH_CHECK_ARG(kind != 2 || static_cast<int64_t>(grid) * 4 <= bytes, "hbm_stream: read needs grid floats of dst");
  const int64_t n = bytes / 16;
  const auto* s = static_cast<const f32x4n*>(src);
  auto* d = static_cast<f32x4n*>(dst);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool nt = nontemporal != 0;
  switch (kind) {
    case 0: launch_stream<0>(nt, s, d, n, grid, st); break;
    case 1: launch_stream<1>(nt, s, d, n, grid, st); break;
    case 2: launch_stream<2>(nt, s, d, n, grid, st); break;
    default: launch_stream<3>(nt, s, d, n, grid, st); break;
  }
  YH_CHECK_LAUNCH("hbm_stream");
  return YH_OK;
}
