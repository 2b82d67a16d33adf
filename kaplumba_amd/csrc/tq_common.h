// Shared device/host helpers for the TurboQuant HIP kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cfloat>
#include <cmath>
#include <cstdio>
#include <string>

#include "kaplumba_tq.h"

namespace tq {

constexpr int kWave = 64;
constexpr float kNormEps = 1e-6f;  // turboquant_cache.py:12 (_EPS)

// ---------------------------------------------------------------- errors ----
void set_error(const char* fmt, ...);
int fail(int code, const char* fmt, ...);
int check_launch(const char* what);
int device_cu_count();

// ------------------------------------------------------------- dtype I/O ----
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// Round-to-nearest-even f32 -> bf16 bits (NaN kept quiet).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
  _Float16 v = __builtin_bit_cast(_Float16, h);
  return static_cast<float>(v);
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  _Float16 v = static_cast<_Float16>(f);  // IEEE round-to-nearest-even
  return __builtin_bit_cast(uint16_t, v);
}

template <int DT>
__device__ __forceinline__ float load_elem(const void* p, int64_t i) {
  if constexpr (DT == TQ_DTYPE_F32) {
    return static_cast<const float*>(p)[i];
  } else if constexpr (DT == TQ_DTYPE_F16) {
    return f16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
  } else {
    return bf16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
  }
}

template <int DT>
__device__ __forceinline__ void store_elem(void* p, int64_t i, float v) {
  if constexpr (DT == TQ_DTYPE_F32) {
    static_cast<float*>(p)[i] = v;
  } else if constexpr (DT == TQ_DTYPE_F16) {
    static_cast<uint16_t*>(p)[i] = f32_to_f16_bits(v);
  } else {
    static_cast<uint16_t*>(p)[i] = f32_to_bf16_bits(v);
  }
}

// Round an f32 value to the given storage dtype and back (RNE).
template <int DT>
__device__ __forceinline__ float round_to(float v) {
  if constexpr (DT == TQ_DTYPE_F32) {
    return v;
  } else if constexpr (DT == TQ_DTYPE_F16) {
    return f16_bits_to_f32(f32_to_f16_bits(v));
  } else {
    return bf16_bits_to_f32(f32_to_bf16_bits(v));
  }
}

inline float host_round_to(int dt, float v) {
  if (dt == TQ_DTYPE_F32) return v;
  if (dt == TQ_DTYPE_F16) return static_cast<float>(static_cast<_Float16>(v));
  uint32_t u;
  __builtin_memcpy(&u, &v, 4);
  u += 0x7fffu + ((u >> 16) & 1u);
  u &= 0xffff0000u;
  float r;
  __builtin_memcpy(&r, &u, 4);
  return r;
}

// Norm storage.
__device__ __forceinline__ float load_norm(const void* p, int norm_dtype, int64_t i) {
  return norm_dtype == TQ_DTYPE_F16 ? f16_bits_to_f32(static_cast<const uint16_t*>(p)[i])
                                    : static_cast<const float*>(p)[i];
}

// IEEE correctly rounded single-precision square root.  The hardware
// v_sqrt_f32 is accurate to 1 ulp; the result s is corrected by the signs of
// the exact residuals x - s_down*s and x - s_up*s (one fma each), which decide
// on which side of the rounding midpoints sqrt(x) lies.  Inputs below 2^-96
// are scaled by 2^32 first so the residuals stay out of the subnormal range.
__device__ __forceinline__ float sqrt_rn(float x) {
  const bool small = x < 0x1p-96f;
  const float xs = small ? x * 0x1p32f : x;
  float s = __builtin_amdgcn_sqrtf(xs);
  if (xs > 0.f && xs < INFINITY) {
    const int si = __float_as_int(s);
    const float s_dn = __int_as_float(si - 1);
    const float s_up = __int_as_float(si + 1);
    const float e_dn = __builtin_fmaf(-s_dn, s, xs);
    const float e_up = __builtin_fmaf(-s_up, s, xs);
    if (e_dn <= 0.f) s = s_dn;
    if (e_up > 0.f) s = s_up;
  }
  return small ? s * 0x1p-16f : s;
}

// ----------------------------------------------------------- bit fields ----
// Value of bits [pos, pos+nb) of a little-endian word array held in registers.
// pos and nb are compile-time after unrolling, so this folds to v_bfe_u32 or
// v_alignbit_b32 + v_bfe_u32 for fields that straddle two words.
template <int NB, int NW>
__device__ __forceinline__ uint32_t field(const uint32_t (&w)[NW], int pos) {
  const int wi = pos >> 5;
  const int sh = pos & 31;
  uint32_t v;
  if (sh + NB <= 32) {
    v = w[wi] >> sh;
  } else {
    v = __builtin_amdgcn_alignbit(w[wi + 1], w[wi], sh);
  }
  return v & ((1u << NB) - 1u);
}

}  // namespace tq
