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


// The two wave halves exchanged (v_permlane32_swap): .x = x of lane l for
// l < 32 and of lane l - 32 otherwise, .y = x of lane l + 32 for l < 32 and
// of lane l otherwise; so op(.x, .y) is the pairwise op of lanes l, l ^ 32.
__device__ __forceinline__ float2 halves(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return make_float2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float wave_max(float x) {
  x = fmaxf(x, xor_lane<1>(x));
  x = fmaxf(x, xor_lane<2>(x));
  x = fmaxf(x, xor_lane<4>(x));
  x = fmaxf(x, xor_lane<8>(x));
  const float2 r = rows16_pair(x);
  x = fmaxf(r.x, r.y);
  const float2 h = halves(x);
  return fmaxf(h.x, h.y);
}

__device__ __forceinline__ float wave_sum(float x) {
  x += xor_lane<1>(x);
  x += xor_lane<2>(x);
  x += xor_lane<4>(x);
  x += xor_lane<8>(x);
  const float2 r = rows16_pair(x);
  x = r.x + r.y;
  const float2 h = halves(x);
  return h.x + h.y;
}

// Unnormalised Walsh-Hadamard transform of a D-vector held by one wave as
// y[e] = x[lane + 64 e]: butterflies across e in-lane, across lanes by DPP,
// swizzles and the half swap.  sgn[k] = -1 where lane bit k is set, else 1.
template <int D>
__device__ __forceinline__ void wave_fwht(float (&y)[D / kWave], const float (&sgn)[6]) {
  constexpr int E = D / kWave;
#pragma unroll
  for (int s = E / 2; s >= 1; s >>= 1)
#pragma unroll
    for (int e = 0; e < E; ++e)
      if ((e & s) == 0) {
        const float a = y[e], b = y[e + s];
        y[e] = a + b;
        y[e + s] = a - b;
      }
#pragma unroll
  for (int e = 0; e < E; ++e) {
    float v = y[e];
    v = fmaf(sgn[0], v, xor_lane<1>(v));
    v = fmaf(sgn[1], v, xor_lane<2>(v));
    v = fmaf(sgn[2], v, xor_lane<4>(v));
    v = fmaf(sgn[3], v, xor_lane<8>(v));
    const float2 r = rows16_pair(v);  // even rows: v + v[l + 16]; odd: v[l - 16] - v
    v = fmaf(sgn[4], r.y, r.x);
    const float2 h = halves(v);  // lanes < 32: v + v[l + 32]; others: v[l - 32] - v
    y[e] = fmaf(sgn[5], h.y, h.x);
  }
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

// Rows j < nrows of y (LDS, [NQ][D] f32) through the dense R_V^-1:
// x[j][d] = scl(j) * sum_k y[j][k] R_V[k][d], stored as output row qoff(j).
// One pass over R_V (D x D f32, row-major, read from L2 once per workgroup):
// thread (column group c, k slice ks) owns four columns of every row over
// D / KS values of k and streams its R_V rows as float4, up to 32 loads in
// flight (the read is latency-bound: few round trips matter more than
// instruction count).  The y reads are LDS broadcasts.  The slices are added
// through s_part ([NT / 64][NQ][D] f32 of LDS, not aliasing y).  Rows past
// nrows are summed too (uniform work, never stored).  All threads call it.
template <int D, int NQ, int NT, class Off, class Scale>
__device__ __forceinline__ void dense_rows_out(const AttnParams& p, const float* y, float* s_part,
                                               int nrows, Off qoff, Scale scl) {
  constexpr int C4 = D / 4;
  constexpr int NW = NT / kWave;
  constexpr int KS = NT / C4 < NW ? NT / C4 : NW;  // k slices (s_part holds NW)
  constexpr int KR = D / KS;                        // k values per slice
  constexpr int KU = KR < 32 ? KR : 32;             // loads in flight
  static_assert(KS >= 1 && D % KS == 0 && KR % KU == 0 && KU % 4 == 0, "dense rows mapping");
  const int c = threadIdx.x % C4;
  const int ks = threadIdx.x / C4;
  if (ks < KS) {
    float4 acc[NQ];
#pragma unroll
    for (int j = 0; j < NQ; ++j) acc[j] = make_float4(0.f, 0.f, 0.f, 0.f);
    const float4* r4 = reinterpret_cast<const float4*>(p.vrot) + c;
    const float4* y4 = reinterpret_cast<const float4*>(y);
#pragma unroll 1
    for (int k0 = ks * KR; k0 < (ks + 1) * KR; k0 += KU) {
      float4 r[KU];
#pragma unroll
      for (int u = 0; u < KU; ++u) r[u] = r4[(k0 + u) * C4];
#pragma unroll
      for (int j = 0; j < NQ; ++j)
#pragma unroll
        for (int u4 = 0; u4 < KU / 4; ++u4) {
          const float4 yv = y4[(j * D + k0) / 4 + u4];
          const float ys[4] = {yv.x, yv.y, yv.z, yv.w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float4 rv = r[4 * u4 + e];
            acc[j].x = fmaf(ys[e], rv.x, acc[j].x);
            acc[j].y = fmaf(ys[e], rv.y, acc[j].y);
            acc[j].z = fmaf(ys[e], rv.z, acc[j].z);
            acc[j].w = fmaf(ys[e], rv.w, acc[j].w);
          }
        }
    }
    float4* part4 = reinterpret_cast<float4*>(s_part);
#pragma unroll
    for (int j = 0; j < NQ; ++j) part4[(ks * NQ + j) * C4 + c] = acc[j];
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < NQ * C4; idx += NT) {
    const int j = idx / C4;
    const int cc = idx % C4;
    if (j >= nrows) break;  // idx grows: every later index is past nrows too
    const float4* part4 = reinterpret_cast<const float4*>(s_part);
    float4 a = part4[j * C4 + cc];
#pragma unroll
    for (int k = 1; k < KS; ++k) {
      const float4 t = part4[(k * NQ + j) * C4 + cc];
      a.x += t.x;
      a.y += t.y;
      a.z += t.z;
      a.w += t.w;
    }
    const float s = scl(j);
    const int64_t o = qoff(j) * D + 4 * cc;
    store_out(p.out, p.q_dtype, o, a.x * s);
    store_out(p.out, p.q_dtype, o + 1, a.y * s);
    store_out(p.out, p.q_dtype, o + 2, a.z * s);
    store_out(p.out, p.q_dtype, o + 3, a.w * s);
  }
}

// Normalise s_o rows by 1/max(l, eps), apply R_V^-1 and store.  s_o: [NQ][D];
// s_vsign: D floats of LDS scratch; s_part: [NT / 64][NQ][D] f32 of LDS
// scratch for the dense rotation (unused otherwise).
template <int D, int NQ, int NT>
__device__ void finalize_rows(const AttnParams& p, const RowSet& rs, float* s_o,
                              const float* s_l, float* s_vsign, float* s_part, bool plain, bool dense) {
  if (!plain && !dense)
    for (int d = threadIdx.x; d < D; d += NT) s_vsign[d] = p.vrot[d];
  for (int idx = threadIdx.x; idx < NQ * D; idx += NT)
    s_o[idx] = s_o[idx] / fmaxf(s_l[idx / D], kNormEps);
  __syncthreads();
  if (!plain && dense) {
    int nrows = 0;
    while (nrows < NQ && rs.valid(nrows)) ++nrows;  // valid rows are a prefix
    dense_rows_out<D, NQ, NT>(p, s_o, s_part, nrows, [&](int j) { return rs.qoff(j); },
                              [](int) { return 1.f; });
    return;
  }
  if (!plain) lds_fwht<D, NQ, NT>(s_o);
  for (int idx = threadIdx.x; idx < NQ * D; idx += NT) {
    const int j = idx / D;
    const int d = idx % D;
    if (!rs.valid(j)) continue;
    float r = s_o[idx];
    if (!plain) r = r * p.rscale * s_vsign[d];
    store_out(p.out, p.q_dtype, rs.qoff(j) * D + d, r);
  }
}

}  // namespace tq
