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

// Dense-rotation quantizer on the matrix cores (tq_append_dense.hip).
int launch_append_dense(const AppendArgs& a, int dim, int bits, int x_dtype, hipStream_t st);
// Keys and values in one launch (16-bit input, dim 64 / 128 / 256, equal
// widths or v_bits = k_bits + 1); returns -1 for other cases.
int launch_append_dense_kv(const AppendArgs& k, const AppendArgs& v, int dim, int kbits, int vbits,
                           int x_dtype, hipStream_t st);
// The same product for f32 input with a one-bit output (x @ R^T >= 0), the
// Prod codec's QJL signs; norms receive ||x||.
int launch_append_dense_signs(const AppendArgs& a, int dim, hipStream_t st);

}  // namespace tq
