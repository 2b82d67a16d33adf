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
  const uint32_t u = __float_as_uint(f);
  const uint32_t rne = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  // NaN stays a (quiet) NaN; a select, so unrolled callers stay straight-line
  return static_cast<uint16_t>((u & 0x7fffffffu) > 0x7f800000u ? ((u >> 16) | 0x40u) : rne);
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

// ------------------------------------------------- quantization buckets ----
// idx(y) = #{m : y > mid_m} for sorted midpoints through one table lookup.
// y goes to cell(y) = clamp(round(y k + c), 0, kQbN - 1), a monotone function
// of y; k and c spread the midpoints over cells 1 .. kQbN - 1.  The rounding
// is the float's own: t = RN(y k + c + 1.5 * 2^23) is an integer-valued float
// in [2^23, 2^24) while |y k + c| < 2^22, whose bits are those of
// 1.5 * 2^23 plus the integer; outside that range the bits (as int32) lie
// below or above the clamp bounds, so one integer clamp of the bits finishes
// the cell (fma, med3, and the table address).
// Entry j holds (the number of midpoints in cells below j, the midpoint in
// cell j or +inf).  For every y with cell(y) = j, a midpoint in a lower cell
// is below y and one in a higher cell above it (monotonicity), so the lookup
// plus one compare is exact whenever no cell holds two midpoints, which
// qb_entry_grid reports so that a kernel can fall back to plain comparisons.
constexpr int kQbN = 256;

constexpr int kQbMagic = 0x4B400000;  // bits of 1.5 * 2^23

struct QbGrid {
  float k, c;  // c includes 1.5 * 2^23
  bool ok;     // finite, increasing
};

__device__ __forceinline__ QbGrid qb_grid(float lo, float hi) {
  QbGrid g;
  g.k = static_cast<float>(kQbN - 2) / (hi - lo);
  const float c0 = 1.f - lo * g.k;
  g.c = c0 + 0x1.8p23f;
  g.ok = g.k > 0.f && g.k < INFINITY && fabsf(c0) < 0x1p20f;
  return g;
}

__device__ __forceinline__ uint32_t qb_cell(float y, const QbGrid& g) {
  const int t = __float_as_int(__builtin_fmaf(y, g.k, g.c));
  return static_cast<uint32_t>(min(max(t, kQbMagic), kQbMagic + kQbN - 1) - kQbMagic);
}

// Neighbouring floats of a finite t (+-0 count as one value).
__device__ __forceinline__ float next_up(float t) {
  if (t == 0.f) return __uint_as_float(1u);
  const uint32_t u = __float_as_uint(t);
  return __uint_as_float(t > 0.f ? u + 1u : u - 1u);
}
__device__ __forceinline__ float next_down(float t) { return -next_up(-t); }

// The largest float T with RN(T * s) <= mid, for s > 0: then RN(v * s) > mid
// exactly when v > T (RN(v * s) is monotone in v), so a compare against T
// replaces the product.  A walk of a few ulps from RN(mid / s); midpoints at
// or near zero walk up through the subnormals (about 2^-150 / s / 2^-149
// steps, under 32 for s >= 2^-6).  Returns false when the walk does not
// settle (the caller then compares RN(v * s) itself).
__device__ __forceinline__ bool unscaled_threshold(float mid, float s, float& T) {
  if (!(fabsf(mid) < INFINITY) || !(s > 0.f) || !(s < INFINITY)) return false;
  float t = __fdiv_rn(mid, s);
  if (!(fabsf(t) < INFINITY)) return false;
#pragma unroll 1
  for (int k = 0; k < 4 && __fmul_rn(t, s) > mid; ++k) t = next_down(t);
#pragma unroll 1
  for (int k = 0; k < 32 && __fmul_rn(next_up(t), s) <= mid; ++k) t = next_up(t);
  T = t;
  return __fmul_rn(t, s) <= mid && __fmul_rn(next_up(t), s) > mid;
}

// Table entry t from thresholds thr[0 .. n) (cells taken with grid g);
// returns false when two of them share cell t.
__device__ __forceinline__ bool qb_entry_grid(uint32_t t, const float* thr, int n, const QbGrid& g,
                                              uint2& ent) {
  uint32_t base = 0;
  int inside = 0;
  float tm = INFINITY;
  for (int m = 0; m < n; ++m) {
    const float th = thr[m];
    const uint32_t cm = qb_cell(th, g);
    base += cm < t ? 1u : 0u;
    if (cm == t) {
      ++inside;
      tm = th;
    }
  }
  ent = make_uint2(base, __float_as_uint(tm));
  return inside <= 1;
}

// Lane value of the partner lane ^ OFF (OFF < 32), all in the vector ALU
// (no LDS round trip): DPP inside a row of 16 lanes, the gfx950 row swap
// across rows.
//   1, 2: quad_perm [1,0,3,2], [2,3,0,1]
//   4:    row_half_mirror (lane j of 8 <- 7 - j, i.e. ^7), then quad_perm
//         [3,2,1,0] (^3): ^7 ^3 = ^4
//   8:    row_ror:8 (lane j of 16 <- j + 8 mod 16 = j ^ 8)
//   16:   v_permlane16_swap of the value with itself gives rows (0,0,2,2) and
//         (1,1,3,3); the partner is the other one
template <int OFF>
__device__ __forceinline__ float xor_lane(float v) {
  static_assert(OFF == 1 || OFF == 2 || OFF == 4 || OFF == 8 || OFF == 16, "lane xor distance");
  const int x = __float_as_int(v);
  if constexpr (OFF == 1) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0xB1, 0xf, 0xf, true));
  } else if constexpr (OFF == 2) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0x4E, 0xf, 0xf, true));
  } else if constexpr (OFF == 4) {
    const int t = __builtin_amdgcn_mov_dpp(x, 0x141, 0xf, 0xf, true);
    return __int_as_float(__builtin_amdgcn_mov_dpp(t, 0x1B, 0xf, 0xf, true));
  } else if constexpr (OFF == 8) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0x128, 0xf, 0xf, true));
  } else {
    const auto r = __builtin_amdgcn_permlane16_swap(static_cast<unsigned>(x), static_cast<unsigned>(x), false, false);
    return __uint_as_float((__lane_id() & 16) ? r[0] : r[1]);
  }
}

// Rows of 16 lanes exchanged in pairs (v_permlane16_swap): .x = x of lane l
// for even rows and of lane l - 16 for odd rows, .y = x of lane l + 16 for
// even rows and of lane l otherwise; op(.x, .y) is the pairwise op of lanes
// l, l ^ 16, and fma(s, .y, .x) with s = -1 on odd rows is the butterfly
// (x_l + x_l^16 on even rows, x_l^16 - x_l on odd).
__device__ __forceinline__ float2 rows16_pair(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return make_float2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Issue priority from a wave's progress through its n loop steps: 3 at the
// start down to 0 in the last quarter (uniform arithmetic; s_setprio takes
// an immediate).  Two waves share a SIMD, and at equal priority the older is
// picked first, runs ahead and leaves the younger alone on the SIMD at the
// end; with priority falling as a wave advances, the one behind takes
// precedence and the pair stays level.
__device__ __forceinline__ void prio_by_progress(int i, int n) {
  const int left4 = 4 * (n - i);
  if (left4 > 3 * n)
    __builtin_amdgcn_s_setprio(3);
  else if (left4 > 2 * n)
    __builtin_amdgcn_s_setprio(2);
  else if (left4 > n)
    __builtin_amdgcn_s_setprio(1);
  else
    __builtin_amdgcn_s_setprio(0);
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
