// Shared helpers for the yanchor_amd HIP kernels (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdarg.h>
#include <stdio.h>

#include "../../include/yanchor_amd.h"

namespace yh {

constexpr int kWave = 64;

// ---- error reporting (thread-local message behind yh_last_error) ----------
void set_error(const char* fmt, ...);

#define YH_CHECK_ARG(cond, ...)                         \
  do {                                                  \
    if (!(cond)) {                                      \
      ::yh::set_error(__VA_ARGS__);                     \
      return YH_ERR_INVALID;                            \
    }                                                   \
  } while (0)

#define YH_CHECK_LAUNCH(what)                                              \
  do {                                                                     \
    hipError_t e_ = hipGetLastError();                                     \
    if (e_ != hipSuccess) {                                                \
      ::yh::set_error("%s: launch failed: %s", what, hipGetErrorString(e_)); \
      return YH_ERR_HIP;                                                   \
    }                                                                      \
  } while (0)

// ---- scalar conversions ----------------------------------------------------
// bf16 -> f32 by a shift; f32 -> bf16 on the hardware conversion
// (v_cvt_pk_bf16_f32), which rounds to nearest even as torch's
// .to(torch.bfloat16) does, and turns NaN into a quiet NaN.
__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}
__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

// Load element i of a tensor whose element type is given at run time.
__device__ __forceinline__ float load_any(const void* p, int64_t i, int dtype) {
  switch (dtype) {
    case YH_BF16: return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
    case YH_F16:  return f16_to_f32(static_cast<const uint16_t*>(p)[i]);
    default:      return static_cast<const float*>(p)[i];
  }
}
__device__ __forceinline__ void store_any(void* p, int64_t i, int dtype, float x) {
  switch (dtype) {
    case YH_BF16: static_cast<uint16_t*>(p)[i] = f32_to_bf16(x); break;
    case YH_F16:  static_cast<uint16_t*>(p)[i] = f32_to_f16(x); break;
    default:      static_cast<float*>(p)[i] = x; break;
  }
}

// Compile-time element types for the hot tensors.
template <int DT> struct Elem;
template <> struct Elem<YH_F32> {
  using T = float;
  __device__ static float ld(const T* p, int64_t i) { return p[i]; }
  __device__ static void st(T* p, int64_t i, float x) { p[i] = x; }
};
template <> struct Elem<YH_BF16> {
  using T = uint16_t;
  __device__ static float ld(const T* p, int64_t i) { return bf16_to_f32(p[i]); }
  __device__ static void st(T* p, int64_t i, float x) { p[i] = f32_to_bf16(x); }
};
template <> struct Elem<YH_F16> {
  using T = uint16_t;
  __device__ static float ld(const T* p, int64_t i) { return f16_to_f32(p[i]); }
  __device__ static void st(T* p, int64_t i, float x) { p[i] = f32_to_f16(x); }
};

// Load 4 consecutive elements (i must be a multiple of 4) as float4.
template <int DT>
__device__ __forceinline__ float4 load4(const void* p, int64_t i) {
  if constexpr (DT == YH_F32) {
    return reinterpret_cast<const float4*>(static_cast<const float*>(p) + i)[0];
  } else {
    uint2 w = reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(p) + i)[0];
    float4 r;
    if constexpr (DT == YH_BF16) {
      r.x = __uint_as_float(w.x << 16);
      r.y = __uint_as_float(w.x & 0xffff0000u);
      r.z = __uint_as_float(w.y << 16);
      r.w = __uint_as_float(w.y & 0xffff0000u);
    } else {
      r.x = f16_to_f32(w.x & 0xffff);
      r.y = f16_to_f32(w.x >> 16);
      r.z = f16_to_f32(w.y & 0xffff);
      r.w = f16_to_f32(w.y >> 16);
    }
    return r;
  }
}

template <int DT>
__device__ __forceinline__ void store4(void* p, int64_t i, float4 x) {
  if constexpr (DT == YH_F32) {
    reinterpret_cast<float4*>(static_cast<float*>(p) + i)[0] = x;
  } else {
    uint2 w;
    if constexpr (DT == YH_BF16) {
      w.x = f32_to_bf16(x.x) | (static_cast<uint32_t>(f32_to_bf16(x.y)) << 16);
      w.y = f32_to_bf16(x.z) | (static_cast<uint32_t>(f32_to_bf16(x.w)) << 16);
    } else {
      w.x = f32_to_f16(x.x) | (static_cast<uint32_t>(f32_to_f16(x.y)) << 16);
      w.y = f32_to_f16(x.z) | (static_cast<uint32_t>(f32_to_f16(x.w)) << 16);
    }
    reinterpret_cast<uint2*>(static_cast<uint16_t*>(p) + i)[0] = w;
  }
}

// Streaming (nontemporal) 16-byte access for data touched exactly once per
// launch, e.g. the recurrent state read-modify-write: it keeps the stream from
// displacing reusable lines in L2 / the Infinity Cache.
typedef float f32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 ld_stream4(const float* p) {
  const f32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const f32x4_t*>(p));
  return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void st_stream4(float* p, float4 x) {
  const f32x4_t v = {x.x, x.y, x.z, x.w};
  __builtin_nontemporal_store(v, reinterpret_cast<f32x4_t*>(p));
}
// Four fp16 values (8 bytes), widened exactly / rounded to nearest even.
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float4 ld_stream_h4(const uint16_t* p) {
  const u32x2_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(p));
  return make_float4(f16_to_f32(v.x & 0xffffu), f16_to_f32(v.x >> 16), f16_to_f32(v.y & 0xffffu),
                     f16_to_f32(v.y >> 16));
}
__device__ __forceinline__ void st_stream_h4(uint16_t* p, float4 x) {
  // the float32 values first: without this the compiler fuses the producing
  // FMA into the conversion (v_fma_mix), one rounding instead of the float32
  // value's rounding to fp16
  asm volatile("" : "+v"(x.x), "+v"(x.y), "+v"(x.z), "+v"(x.w));
  const u32x2_t v = {static_cast<uint32_t>(f32_to_f16(x.x)) | (static_cast<uint32_t>(f32_to_f16(x.y)) << 16),
                     static_cast<uint32_t>(f32_to_f16(x.z)) | (static_cast<uint32_t>(f32_to_f16(x.w)) << 16)};
  __builtin_nontemporal_store(v, reinterpret_cast<u32x2_t*>(p));
}

// Wave-wide sum (64 lanes) with xor shuffles.
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off, kWave);
  return x;
}
__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x = fmaxf(x, __shfl_xor(x, off, kWave));
  return x;
}

inline bool is_float_dtype(int dt) { return dt == YH_F32 || dt == YH_BF16 || dt == YH_F16; }

// ---- anchor-memory Top-K ordering ---------------------------------------------
// Order-preserving 32-bit key of an fp32 score (bigger score -> bigger key);
// -0.0 is mapped to +0.0 first so the two compare equal.
__device__ __forceinline__ uint32_t score_key(float x) {
  if (x == 0.f) x = 0.f;
  const uint32_t u = __float_as_uint(x);
  return (u & 0x80000000u) ? ~u : (u ^ 0x80000000u);
}
// Candidate key whose ascending order is the Top-K order: score descending,
// then position ascending with invalid (negative) positions last.  Equal keys
// are broken by candidate index, which only ever separates invalid entries.
__device__ __forceinline__ uint64_t topk_key(float score, int32_t position) {
  const uint32_t pkey = position >= 0 ? static_cast<uint32_t>(position) : 0x7fffffffu;
  return (static_cast<uint64_t>(~score_key(score)) << 32) | pkey;
}

}  // namespace yh
