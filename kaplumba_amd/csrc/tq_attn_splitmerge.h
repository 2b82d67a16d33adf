// Split-K merge as a second kernel on the same stream (packed caches).
//
// The partial kernel writes, per (sequence, kv head, row group) and split,
// the unnormalised o[NQ][D] (already back in the unrotated basis for the
// Hadamard rotation) and (m, l) per row with plain stores; kernel-boundary
// ordering on the stream makes them visible here, so no atomics, counters or
// cache-bypassing accesses are needed.  Thread (float4 column c, split group
// sg) folds the splits sg, sg + SG, ... of a row by log-sum-exp, the split
// groups fold through LDS, and the row is normalised by 1/max(l, 1e-6).
//   Hadamard: grid.x = rows per group, one row per workgroup, stored directly.
//   Dense: grid.x = D / 64 column blocks per row group.  Every block merges
//   all rows of the group into LDS (the partials are small), then computes
//   its 64 output columns of y @ R_V for all rows at once: 4 thread groups
//   each sum a quarter of the k range with 16 loads of R_V in flight, so the
//   D x D matrix is read once per row group, spread over D / 64 workgroups.
// Semantics: quantized_attention's final o / max(l, eps), turboquant_cache.py:5190-5203.
#pragma once

#include "tq_attn_merge.h"

// Phase stamps of attn_merge_rot_kernel (build option TQ_PHASE_STAMPS, read
// with tq_dbg_merge_stamps()): rows 0 entry, 1 loads in, 2 folded, 3 stored.
#ifdef TQ_PHASE_STAMPS
namespace tq {
static __device__ uint64_t g_merge_stamps[4][1024];
}
#define MERGE_STAMP(i)                                                                            \
  do {                                                                                            \
    if (threadIdx.x == 0)                                                                         \
      g_merge_stamps[i][blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z)] =         \
          __builtin_amdgcn_s_memrealtime();                                                       \
  } while (0)
#else
#define MERGE_STAMP(i) \
  do {               \
  } while (0)
#endif

namespace tq {

constexpr int kMergeThreads = 256;

template <int D>
__global__ __launch_bounds__(kMergeThreads) void attn_merge_kernel(AttnParams p) {
  constexpr int C4 = D / 4;
  constexpr int SG = kMergeThreads / C4;  // split groups
  constexpr int BATCH = 8;                 // splits per thread per round trip
  constexpr int MAXR = D >= 256 ? 4 : 16;  // rows per group (the partial kernel's NQ bound)
  static_assert(kMergeThreads % C4 == 0, "merge mapping");
  __shared__ float4 s_po[SG][C4];
  __shared__ float s_pm[SG], s_pl[SG];
  __shared__ float s_y[MAXR * D];
  __shared__ float s_part[4][MAXR][64];

  const int tid = threadIdx.x;
  const int gk = blockIdx.y / p.n_rg;
  const int rg = blockIdx.y % p.n_rg;
  const int b = blockIdx.z;
  RowSet rs;
  rs.init(p, b, gk, rg, p.nq);
  const SeqWindow win = seq_window(p, b);
  const int64_t Tb = win.len;  // token positions below are relative to win.start
  const int nvalid = Tb > 0 ? static_cast<int>((Tb + p.chunk - 1) / p.chunk) : 0;
  if (nvalid <= 1) return;  // the partial kernel wrote these rows itself
  const bool dense = p.rot_kind == TQ_ROT_DENSE;

  const int64_t grp = (static_cast<int64_t>(b) * p.Hkv + gk) * p.n_rg + rg;
  const float* po_g = p.po + grp * static_cast<int64_t>(p.n_splits) * p.nq * D;
  const float* pml_g = p.pml + grp * static_cast<int64_t>(p.n_splits) * p.nq * 2;
  const int c = tid % C4;
  const int sg = tid / C4;
  const int j0 = dense ? 0 : static_cast<int>(blockIdx.x);
  const int jstep = dense ? 1 : p.nq;
  for (int j = j0; j < p.nq; j += jstep) {
    if (!rs.valid(j)) break;  // valid rows are a prefix of the group
    float M = -INFINITY, L = 0.f;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int sp0 = sg; sp0 < nvalid; sp0 += SG * BATCH) {
      float2 ml[BATCH];
      float4 oo[BATCH];
#pragma unroll
      for (int u = 0; u < BATCH; ++u) {
        const int sp = sp0 + u * SG;
        if (sp < nvalid) {
          const int64_t r = static_cast<int64_t>(sp) * p.nq + j;
          ml[u] = reinterpret_cast<const float2*>(pml_g)[r];
          oo[u] = reinterpret_cast<const float4*>(po_g + r * D)[c];
        } else {
          ml[u] = make_float2(-INFINITY, 0.f);
          oo[u] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
      }
      float bm = M;
#pragma unroll
      for (int u = 0; u < BATCH; ++u) bm = fmaxf(bm, ml[u].x);
      const float r0 = (M == -INFINITY) ? 0.f : __expf(M - bm);
      L *= r0;
      acc.x *= r0;
      acc.y *= r0;
      acc.z *= r0;
      acc.w *= r0;
#pragma unroll
      for (int u = 0; u < BATCH; ++u) {
        const float sc = (ml[u].x == -INFINITY) ? 0.f : __expf(ml[u].x - bm);
        L = fmaf(sc, ml[u].y, L);
        acc.x = fmaf(sc, oo[u].x, acc.x);
        acc.y = fmaf(sc, oo[u].y, acc.y);
        acc.z = fmaf(sc, oo[u].z, acc.z);
        acc.w = fmaf(sc, oo[u].w, acc.w);
      }
      M = bm;
    }
    s_po[sg][c] = acc;
    if (c == 0) {
      s_pm[sg] = M;
      s_pl[sg] = L;
    }
    __syncthreads();
    if (tid < C4) {
      float Mt = -INFINITY;
#pragma unroll
      for (int g2 = 0; g2 < SG; ++g2) Mt = fmaxf(Mt, s_pm[g2]);
      float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
      float lt = 0.f;
#pragma unroll
      for (int g2 = 0; g2 < SG; ++g2) {
        const float sc = (s_pm[g2] == -INFINITY) ? 0.f : __expf(s_pm[g2] - Mt);
        lt = fmaf(sc, s_pl[g2], lt);
        a.x = fmaf(sc, s_po[g2][tid].x, a.x);
        a.y = fmaf(sc, s_po[g2][tid].y, a.y);
        a.z = fmaf(sc, s_po[g2][tid].z, a.z);
        a.w = fmaf(sc, s_po[g2][tid].w, a.w);
      }
      const float den = fmaxf(lt, kNormEps);
      const float v[4] = {a.x / den, a.y / den, a.z / den, a.w / den};
      const int64_t qo = rs.qoff(j) * D;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (dense)
          s_y[j * D + 4 * tid + e] = v[e];
        else
          store_out(p.out, p.q_dtype, qo + 4 * tid + e, v[e]);
      }
    }
    __syncthreads();  // s_po / s_pm are reused by the next row
  }
  if (!dense) return;
  // x_d = sum_k y_k R[k][d] for every valid row, columns d of this block
  int nrows = 0;
  while (nrows < p.nq && nrows < MAXR && rs.valid(nrows)) ++nrows;
  constexpr int KQ = D / 4;  // k range of one thread group
  const int col = tid % 64;
  const int kq = tid / 64;
  const int d = static_cast<int>(blockIdx.x) * 64 + col;
  float a2[MAXR];
#pragma unroll
  for (int j = 0; j < MAXR; ++j) a2[j] = 0.f;
  for (int k0 = kq * KQ; k0 < (kq + 1) * KQ; k0 += 16) {
    float r[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) r[u] = p.vrot[static_cast<int64_t>(k0 + u) * D + d];
#pragma unroll
    for (int u = 0; u < 16; ++u)
#pragma unroll
      for (int j = 0; j < MAXR; ++j) a2[j] = fmaf(s_y[j * D + k0 + u], r[u], a2[j]);
  }
#pragma unroll
  for (int j = 0; j < MAXR; ++j) s_part[kq][j][col] = a2[j];
  __syncthreads();
  if (tid < 64) {
    for (int j = 0; j < nrows; ++j) {
      const float x = (s_part[0][j][tid] + s_part[1][j][tid]) + (s_part[2][j][tid] + s_part[3][j][tid]);
      store_out(p.out, p.q_dtype, rs.qoff(j) * D + d, x);
    }
  }
}

// Merge of the splits of the staged row-group kernel (tq_attn_stage.h, NQ =
// 4 rows per group) and of the 16-row kernel (tq_attn_rows16.h, NQ = 16, n_rg
// groups per kv head): Hadamard partials still in the rotated basis.  The hot
// arguments (partial buffers, split counts, R_V's signs, kv heads, row
// groups) come first and are preloaded into SGPRs, so the partial loads go
// out without waiting for the argument segment; valid = the split count of a
// sequence when no per-sequence windows exist (-1: from seq_window).
// Workgroup = one wave = one query row of one (sequence, kv head, row
// group); grid (NQ, kv heads x row groups, batch); lane l owns coordinates
// l + 64 e.  Lane u
// loads split u's (m, l) and every lane its o values of the MB splits, all
// loads in flight at once; the log-sum-exp weights come from wave
// reductions and reach every lane by readlane, so the fold needs no LDS and
// no barrier (longer rows fold MB splits per round trip).  R_V^-1 is a wave
// Walsh-Hadamard transform; the row is stored in the query dtype.
constexpr int kMergeRotSplits = 32;  // splits per round trip of attn_merge_rot_kernel

template <int D, int NQ>
__global__ __launch_bounds__(kWave) void attn_merge_rot_kernel(const float* po, const float* pml,
                                                               const float* vrot, int n_splits,
                                                               int valid, int hkv, int n_rg, AttnParams p) {
  constexpr int QE = D / kWave;
  constexpr int MB = kMergeRotSplits;
  const int lane = threadIdx.x;
  const int j = blockIdx.x;
  const int gk = static_cast<int>(blockIdx.y) / n_rg;
  const int rg = static_cast<int>(blockIdx.y) % n_rg;
  const int b = blockIdx.z;
  MERGE_STAMP(0);
  const int nvalid = valid >= 0 ? valid : [&] {
    const SeqWindow win = seq_window(p, b);
    return win.len > 0 ? static_cast<int>((win.len + p.chunk - 1) / p.chunk) : 0;
  }();
  if (nvalid <= 1) return;  // the partial kernel wrote these rows itself
  // (hkv and n_rg preloaded: no wait for the grid size or the argument segment)
  const int64_t grp = static_cast<int64_t>(b) * hkv * n_rg + blockIdx.y;
  const float* po_g = po + grp * static_cast<int64_t>(n_splits) * NQ * D;
  const float2* pml_g = reinterpret_cast<const float2*>(pml) + grp * static_cast<int64_t>(n_splits) * NQ;
  // R_V^-1's signs, loaded with the partials
  float vr[QE];
#pragma unroll
  for (int e = 0; e < QE; ++e) vr[e] = vrot[lane + e * kWave];
  float M = -INFINITY, Lsum = 0.f;
  float acc[QE];
#pragma unroll
  for (int e = 0; e < QE; ++e) acc[e] = 0.f;
  for (int s0 = 0; s0 < nvalid; s0 += MB) {
    // lane u < MB holds split s0 + u's (m, l); every lane holds its o values
    // of the MB splits (past the last split: a repeat of it, weighted 0)
    const bool has = lane < MB && s0 + lane < nvalid;
    const float2 mlu = has ? pml_g[static_cast<int64_t>(s0 + lane) * NQ + j] : make_float2(-INFINITY, 0.f);
    float oo[MB][QE];
#pragma unroll
    for (int u = 0; u < MB; ++u) {
      const int sp = s0 + u < nvalid ? s0 + u : nvalid - 1;
#pragma unroll
      for (int e = 0; e < QE; ++e) oo[u][e] = po_g[(static_cast<int64_t>(sp) * NQ + j) * D + lane + e * kWave];
    }
    if (s0 == 0) MERGE_STAMP(1);
    const float bm = fmaxf(M, wave_max(mlu.x));
    const float r0 = M == -INFINITY ? 0.f : __expf(M - bm);
    const float w = mlu.x == -INFINITY ? 0.f : __expf(mlu.x - bm);
    Lsum = fmaf(Lsum, r0, wave_sum(w * mlu.y));
#pragma unroll
    for (int e = 0; e < QE; ++e) acc[e] *= r0;
#pragma unroll
    for (int u = 0; u < MB; ++u) {
      const float wu = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), u));
#pragma unroll
      for (int e = 0; e < QE; ++e) acc[e] = fmaf(wu, oo[u][e], acc[e]);
    }
    M = bm;
  }
  MERGE_STAMP(2);
  const float inv = 1.f / fmaxf(Lsum, kNormEps);
  float y[QE];
#pragma unroll
  for (int e = 0; e < QE; ++e) y[e] = acc[e] * inv;
  float sg6[6];
#pragma unroll
  for (int k = 0; k < 6; ++k) sg6[k] = (lane >> k) & 1 ? -1.f : 1.f;
  wave_fwht<D>(y, sg6);
  // (rows past the group's last exist in the partials but not in the output;
  // checked only here, so the partial loads above go out first)
  const int jr = rg * NQ + j;  // row of the kv head's GQA group
  if (jr >= p.R * p.L) return;
  const int64_t qo = ((static_cast<int64_t>(b) * p.Hq + gk * p.R + jr / p.L) * p.L + jr % p.L) * D;
#pragma unroll
  for (int e = 0; e < QE; ++e) store_out(p.out, p.q_dtype, qo + lane + e * kWave, y[e] * p.rscale * vr[e]);
  MERGE_STAMP(3);
}

}  // namespace tq
