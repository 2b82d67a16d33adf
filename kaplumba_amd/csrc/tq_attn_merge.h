// Split-K publication and merge shared by the attention kernels.
//
// Each workgroup ends with its split's (max m, sum l, o[D]) per query row in
// LDS (o unnormalised, in rotated space).  It stores them to the workspace
// with agent-scope (sc1, write-through) stores, waits for the stores to
// complete, and bumps the group's counter.  The workgroup that brings the
// counter to the number of live splits merges: it reads every split with
// agent-scope loads (so no stale L2 line from another XCD is used), combines
// them by log-sum-exp, divides by max(l, 1e-6), applies R_V^-1 and stores the
// rows in the query dtype.  No cache-wide write-back or invalidate is needed
// because every shared value goes through sc1 accesses.
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

__device__ __forceinline__ void st_agent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float ld_agent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// In-place unnormalised Walsh-Hadamard transform of NQ rows of length D in
// LDS (stride D), all NT threads of the block participating.
template <int D, int NQ, int NT = kAttnThreads>
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
template <int D, int NQ, int NT = kAttnThreads>
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

// Publish this workgroup's split and, in the last workgroup of the group,
// merge all splits and write the output.
//   s_o  [NQ][D] LDS: o of this split (rotated space, true scale)
//   s_ml [NQ][2] LDS: (m, l) of this split
//   scratch: LDS of at least merge_scratch_floats(NQ, D, NT) floats
//   s_aux: LDS of at least NQ + D floats; s_flag: one int of LDS
// Workspace layout per group g = (b, kv head, row group):
//   po [g][split][NQ][D], pml [g][split][NQ][2]   (contiguous per split)
template <int D, int NQ, int NT = kAttnThreads>
__device__ void publish_and_merge(const AttnParams& p, const RowSet& rs, float* s_o,
                                  float* s_ml, float* scratch, float* s_aux, int* s_flag,
                                  int64_t grp, int split, int nvalid, bool plain, bool dense) {
  const int tid = threadIdx.x;
  float* s_tot = s_aux;        // [NQ]
  float* s_vsign = s_aux + NQ;  // [D]

  if (nvalid == 1) {  // the only split: finish from LDS
    if (tid < NQ) s_tot[tid] = s_ml[2 * tid + 1];
    __syncthreads();
    finalize_rows<D, NQ, NT>(p, rs, s_o, s_tot, s_vsign, plain, dense);
    return;
  }

  float* po_g = p.po + grp * static_cast<int64_t>(p.n_splits) * NQ * D;
  float* pml_g = p.pml + grp * static_cast<int64_t>(p.n_splits) * NQ * 2;
  for (int idx = tid; idx < NQ * D; idx += NT)
    st_agent(po_g + static_cast<int64_t>(split) * NQ * D + idx, s_o[idx]);
  if (tid < 2 * NQ) st_agent(pml_g + static_cast<int64_t>(split) * NQ * 2 + tid, s_ml[tid]);
  __builtin_amdgcn_s_waitcnt(0);  // every sc1 store of this thread has completed
  __syncthreads();
  if (tid == 0) {
    const uint32_t prev =
        __hip_atomic_fetch_add(p.counters + grp, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int last = (prev + 1 == static_cast<uint32_t>(nvalid)) ? 1 : 0;
    if (last) __hip_atomic_store(p.counters + grp, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *s_flag = last;
  }
  __syncthreads();
  if (!*s_flag) return;

  // ---- merge (last workgroup only).  Thread t owns float4 column c of row j
  // (several, when NQ * D / 4 > NT) for the splits sg, sg + SG, ...; it loads
  // a batch of them with independent loads, folds them with an online
  // log-sum-exp, and the SG thread groups of a (row, column) fold through LDS
  // at the end.
  constexpr int C4 = D / 4;
  constexpr int COLS = C4 * NQ;                 // (row, float4 column) pairs
  constexpr int SG = COLS >= NT ? 1 : NT / COLS;  // split groups
  constexpr int BATCH = 16;                     // splits per thread per round trip
  static_assert(COLS >= NT ? COLS % NT == 0 : NT % COLS == 0, "merge mapping");
  float* s_po = scratch;  // [SG][NQ][D] o, then [SG][NQ] m and l
  float* s_pm = scratch + SG * NQ * D;
  float* s_pl = s_pm + SG * NQ;
  for (int col = tid % (SG == 1 ? NT : COLS); col < COLS; col += (SG == 1 ? NT : COLS)) {
    const int c = col % C4;
    const int j = col / C4;
    const int sg = SG == 1 ? 0 : tid / COLS;
    float M = -INFINITY, Ls = 0.f;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int sp0 = sg; sp0 < nvalid; sp0 += SG * BATCH) {
      float mm[BATCH], ll[BATCH];
      float4 oo[BATCH];
#pragma unroll
      for (int u = 0; u < BATCH; ++u) {
        const int sp = sp0 + u * SG;
        if (sp < nvalid) {
          const float* e = pml_g + (static_cast<int64_t>(sp) * NQ + j) * 2;
          const float* o4 = po_g + (static_cast<int64_t>(sp) * NQ + j) * D + 4 * c;
          mm[u] = ld_agent(e);
          ll[u] = ld_agent(e + 1);
          oo[u] = make_float4(ld_agent(o4), ld_agent(o4 + 1), ld_agent(o4 + 2), ld_agent(o4 + 3));
        } else {
          mm[u] = -INFINITY;
          ll[u] = 0.f;
          oo[u] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
      }
      float bm = M;
#pragma unroll
      for (int u = 0; u < BATCH; ++u) bm = fmaxf(bm, mm[u]);
      const float r = (M == -INFINITY) ? 0.f : __expf(M - bm);
      Ls *= r;
      acc.x *= r;
      acc.y *= r;
      acc.z *= r;
      acc.w *= r;
#pragma unroll
      for (int u = 0; u < BATCH; ++u) {
        const float sc = (mm[u] == -INFINITY) ? 0.f : __expf(mm[u] - bm);
        Ls = fmaf(sc, ll[u], Ls);
        acc.x = fmaf(sc, oo[u].x, acc.x);
        acc.y = fmaf(sc, oo[u].y, acc.y);
        acc.z = fmaf(sc, oo[u].z, acc.z);
        acc.w = fmaf(sc, oo[u].w, acc.w);
      }
      M = bm;
    }
    reinterpret_cast<float4*>(s_po + (sg * NQ + j) * D)[c] = acc;
    if (c == 0) {
      s_pm[sg * NQ + j] = M;
      s_pl[sg * NQ + j] = Ls;
    }
  }
  __syncthreads();
  for (int idx = tid; idx < NQ * D; idx += NT) {
    const int jj = idx / D;
    float Mt = -INFINITY;
#pragma unroll
    for (int g2 = 0; g2 < SG; ++g2) Mt = fmaxf(Mt, s_pm[g2 * NQ + jj]);
    float a = 0.f, lt = 0.f;
#pragma unroll
    for (int g2 = 0; g2 < SG; ++g2) {
      const float m2 = s_pm[g2 * NQ + jj];
      const float sc = (m2 == -INFINITY) ? 0.f : __expf(m2 - Mt);
      a = fmaf(sc, s_po[(g2 * NQ) * D + idx], a);
      lt = fmaf(sc, s_pl[g2 * NQ + jj], lt);
    }
    s_o[idx] = a;
    if (idx % D == 0) s_tot[jj] = lt;
  }
  __syncthreads();
  finalize_rows<D, NQ, NT>(p, rs, s_o, s_tot, s_vsign, plain, dense);
}

// Dynamic LDS the merge needs (floats).
__host__ __device__ constexpr int merge_scratch_floats(int nq, int d, int nt = kAttnThreads) {
  return ((d / 4) * nq >= nt ? 1 : nt / ((d / 4) * nq)) * nq * (d + 2) + 4;
}

}  // namespace tq
