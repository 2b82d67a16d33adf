// Helpers shared by the attention kernels: query / output dtype access, the
// query rows of a row group (RowSet), and the finish of a problem that fits
// one split (normalise by 1/max(l, 1e-6), apply R_V^-1, store in the query
// dtype).  Problems with several splits are merged by attn_merge_kernel.
#pragma once

#include "tq_attention.h"

namespace tq {

__device__ __forceinline__ float load_q(const void* q, int dt, int64_t i) {
  if (dt == TQ_DTYPE_F32) return static_cast<const float*>(q)[i];
  const uint16_t h = static_cast<const uint16_t*>(q)[i];
  return dt == TQ_DTYPE_F16 ? f16_bits_to_f32(h) : bf16_bits_to_f32(h);
}

__device__ __forceinline__ float round_q(int dt, float v) {
  if (dt == TQ_DTYPE_F32) return v;
  return dt == TQ_DTYPE_F16 ? round_to<TQ_DTYPE_F16>(v) : round_to<TQ_DTYPE_BF16>(v);
}

__device__ __forceinline__ void store_out(void* o, int dt, int64_t i, float v) {
  if (dt == TQ_DTYPE_F32)
    static_cast<float*>(o)[i] = v;
  else if (dt == TQ_DTYPE_F16)
    static_cast<uint16_t*>(o)[i] = f32_to_f16_bits(v);
  else
    static_cast<uint16_t*>(o)[i] = f32_to_bf16_bits(v);
}


// In-place unnormalised Walsh-Hadamard transform of NQ rows of length D in
// LDS (stride D), all NT threads of the block participating.
template <int D, int NQ, int NT>
__device__ __forceinline__ void lds_fwht(float* y) {
#pragma unroll 1
  for (int hs = 1; hs < D; hs <<= 1) {
    for (int idx = threadIdx.x; idx < NQ * D / 2; idx += NT) {
      const int j = idx / (D / 2);
      const int k = idx % (D / 2);
      const int i0 = (k / hs) * 2 * hs + (k % hs);
      const float a = y[j * D + i0];
      const float b = y[j * D + i0 + hs];
      y[j * D + i0] = a + b;
      y[j * D + i0 + hs] = a - b;
    }
    __syncthreads();
  }
}

// Query row bookkeeping of one workgroup: rows rg*nq + j of kv head gk's GQA
// group, row rr -> (repeat, position) = (rr / L, rr % L).  Computed on demand
// so that a 16-row workgroup keeps no per-row arrays in registers.
struct RowSet {
  int b, gk, rg, nq, rows, R, L, Hq;
  __device__ __forceinline__ void init(const AttnParams& p, int b_, int gk_, int rg_, int nq_) {
    b = b_;
    gk = gk_;
    rg = rg_;
    nq = nq_;
    rows = p.R * p.L;
    R = p.R;
    L = p.L;
    Hq = p.Hq;
  }
  __device__ __forceinline__ bool valid(int j) const { return rg * nq + j < rows; }
  __device__ __forceinline__ int lpos(int j) const { return (rg * nq + j) % L; }
  __device__ __forceinline__ int head(int j) const { return gk * R + (rg * nq + j) / L; }
  // (b*Hq + h)*L + l
  __device__ __forceinline__ int64_t qoff(int j) const {
    return (static_cast<int64_t>(b) * Hq + head(j)) * L + lpos(j);
  }
};

// Normalise s_o rows by 1/max(l, eps), apply R_V^-1 and store.  s_o: [NQ][D];
// s_vsign: D floats of LDS scratch.
template <int D, int NQ, int NT>
__device__ void finalize_rows(const AttnParams& p, const RowSet& rs, float* s_o,
                              const float* s_l, float* s_vsign, bool plain, bool dense) {
  if (!plain && !dense)
    for (int d = threadIdx.x; d < D; d += NT) s_vsign[d] = p.vrot[d];
  for (int idx = threadIdx.x; idx < NQ * D; idx += NT)
    s_o[idx] = s_o[idx] / fmaxf(s_l[idx / D], kNormEps);
  __syncthreads();
  if (!plain && !dense) lds_fwht<D, NQ, NT>(s_o);
  for (int idx = threadIdx.x; idx < NQ * D; idx += NT) {
    const int j = idx / D;
    const int d = idx % D;
    if (!rs.valid(j)) continue;
    float r = s_o[idx];
    if (!plain) {
      if (!dense) {
        r = r * p.rscale * s_vsign[d];
      } else {
        float a2 = 0.f;  // x_d = sum_k y_k R[k][d]
        for (int k2 = 0; k2 < D; ++k2)
          a2 = fmaf(s_o[j * D + k2], p.vrot[static_cast<int64_t>(k2) * D + d], a2);
        r = a2;
      }
    }
    store_out(p.out, p.q_dtype, rs.qoff(j) * D + d, r);
  }
}

}  // namespace tq
