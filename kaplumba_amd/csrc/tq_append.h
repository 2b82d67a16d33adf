// Arguments shared by the append-time quantizers (Hadamard and dense rotation).
#pragma once

#include "tq_common.h"

namespace tq {

struct AppendArgs {
  const void* x;
  int64_t sb, sh, sl;  // element strides of x
  int B, H, L;
  const float* rot;    // Hadamard: signs (D); dense: R (D x D, row-major)
  const float* mid;    // 2^bits - 1 midpoints
  uint32_t* packed;
  void* norms;
  int norm_dtype;
  int64_t cap, offset;
  float scale;         // f32(1/sqrt(D)), Hadamard only
};

// a or b, field by field (each field a uniform select: the result stays in
// scalar registers, where picking a whole kernel argument makes a copy in
// scratch memory)
__device__ __forceinline__ AppendArgs select_args(bool pick_a, const AppendArgs& a, const AppendArgs& b) {
  AppendArgs r;
  r.x = pick_a ? a.x : b.x;
  r.sb = pick_a ? a.sb : b.sb;
  r.sh = pick_a ? a.sh : b.sh;
  r.sl = pick_a ? a.sl : b.sl;
  r.B = pick_a ? a.B : b.B;
  r.H = pick_a ? a.H : b.H;
  r.L = pick_a ? a.L : b.L;
  r.rot = pick_a ? a.rot : b.rot;
  r.mid = pick_a ? a.mid : b.mid;
  r.packed = pick_a ? a.packed : b.packed;
  r.norms = pick_a ? a.norms : b.norms;
  r.norm_dtype = pick_a ? a.norm_dtype : b.norm_dtype;
  r.cap = pick_a ? a.cap : b.cap;
  r.offset = pick_a ? a.offset : b.offset;
  r.scale = pick_a ? a.scale : b.scale;
  return r;
}

// Workgroup barrier over LDS only: outstanding global loads stay in flight
// across it (__syncthreads would wait for them too).
__device__ __forceinline__ void append_lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// u[i] = x[i] / den with IEEE (correctly rounded) division, den = max(n, 1e-6)
// the vector's norm.  The quotient comes from the correctly rounded
// reciprocal r = RN(1 / den), one division per vector: q = RN(x r) is within
// an ulp of x / den, the residual e = x - q den is exact in one fma, and
// RN(q + e r) is the correctly rounded quotient (Markstein's theorem) while
// quotient and residual stay clear of the subnormal range.  That holds for
// every f16 input (|x| >= 2^-24 or 0, den < 2^21); bf16 and f32 inputs take
// the division itself when an element is below 2^-100 in magnitude (zeros
// aside: a zero quotient may differ only in its sign, which no index or sum
// sees) or den is not below 2^100.  x and u may be the same array.
template <int XDT>
__device__ __forceinline__ void div_by_norm(const float (&x)[32], float den, float (&u)[32]) {
  bool slow = false;
  if constexpr (XDT != TQ_DTYPE_F16) {
    slow = !(den < 0x1p100f);
#pragma unroll
    for (int i = 0; i < 32; ++i) slow |= x[i] != 0.f && fabsf(x[i]) < 0x1p-100f;
  }
  if (slow) {
#pragma unroll
    for (int i = 0; i < 32; ++i) u[i] = __fdiv_rn(x[i], den);
  } else {
    const float r = __fdiv_rn(1.f, den);
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      const float q = __fmul_rn(x[i], r);
      u[i] = __builtin_fmaf(__builtin_fmaf(-q, den, x[i]), r, q);
    }
  }
}

// Dense-rotation quantizer on the matrix cores (tq_append_dense.hip).
int launch_append_dense(const AppendArgs& a, int dim, int bits, int x_dtype, hipStream_t st);
// Keys and values in one launch (16-bit input, dim 64 / 128 / 256, equal
// widths or v_bits = k_bits + 1); returns -1 for other cases.
int launch_append_dense_kv(const AppendArgs& k, const AppendArgs& v, int dim, int kbits, int vbits,
                           int x_dtype, hipStream_t st);
// Dense rotation at any dim (multiples of 8 up to 512) on the vector ALUs
// (tq_append_general.hip), for the dims the matrix-core kernels do not take.
int launch_append_dense_general(const AppendArgs& a, int dim, int bits, int x_dtype, hipStream_t st);

struct DequantGeneralArgs {
  const uint32_t* packed;
  const void* norms;
  int norm_dtype;
  int B, H, T, D, bits, PW;
  int64_t cap;
  const float* cb;
  int rot_kind;
  const float* rot;
  float scale;  // f32(1/sqrt(D)), Hadamard only
  float* out;
};
// Dequantize at any dim (multiples of 8 up to 512; Hadamard: powers of two).
int launch_dequant_general(const DequantGeneralArgs& a, int64_t n_vec, hipStream_t st);

// The same product for f32 input with a one-bit output (x @ R^T >= 0), the
// Prod codec's QJL signs; norms receive ||x||.  d = 64 / 128 / 256 on the
// matrix cores, other dims on the vector ALUs (tq_append_general.hip).
int launch_append_dense_signs(const AppendArgs& a, int dim, hipStream_t st);
int launch_append_dense_signs_general(const AppendArgs& a, int dim, hipStream_t st);
// The Prod codec's MSE part at mb = bits - 1 with the dense rotation (any dim
// in 8..512): indices to a.packed, ||x|| to a.norms, the residual
// u - c[idx] @ R to resid [n_vec, dim] f32 (tq_append_general.hip).
int launch_prod_residual_dense(const AppendArgs& a, int dim, int mb, int x_dtype, float* resid,
                               const float* cb, hipStream_t st);

}  // namespace tq
