// Fused split-K attention kernel template (included by tq_attn_d*.hip).
//
// Work decomposition for one workgroup (256 threads = 4 wave64s), which owns
// tokens [t_begin, t_end) of kv head `gk` of sequence `b` and NQ query rows:
//   prologue:        the NQ query rows are scaled, rounded to the query
//                    dtype and (Hadamard) rotated in LDS.
//   pass 1 (keys):   D/32 lanes per token, each lane holds 32 coordinates of
//                    the NQ rotated queries in registers and reads `KB`
//                    consecutive packed words (32 coords x KB bits), decodes
//                    codebook values from LDS, and FMAs; partial dots are
//                    combined across the token's lanes with xor shuffles.
//                    Scores (times ||k||) go to LDS; running max per row.
//   pass 2 (softmax): one thread per token: p = exp(s - m), l += p,
//                    w = p * ||v|| written back over the score.
//   pass 3 (values): 16 lanes per token, D/16 coordinates per lane; a lane
//                    funnel-shifts its bit range out of the packed row and
//                    accumulates w * codebook_v[idx] for every row; the 4
//                    token slots of a wave are folded with shuffles and the
//                    4 waves through LDS.
//   merge:           partials (o, max, sum) go to the workspace; the last
//                    workgroup of the (b, kv head, row group) merges them,
//                    inverse-rotates and writes the output.
// Plain (fp16/bf16) caches use the same passes with direct element loads.
#pragma once

#include "tq_attn_merge.h"
#include "tq_attn_mfma.h"

namespace tq {

template <int KVDT>
__device__ __forceinline__ void unpack8(const uint4 t, float* v) {
  const uint32_t w[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint16_t lo = static_cast<uint16_t>(w[j] & 0xffffu);
    const uint16_t hi = static_cast<uint16_t>(w[j] >> 16);
    if constexpr (KVDT == TQ_DTYPE_F16) {
      v[2 * j] = f16_bits_to_f32(lo);
      v[2 * j + 1] = f16_bits_to_f32(hi);
    } else {
      v[2 * j] = bf16_bits_to_f32(lo);
      v[2 * j + 1] = bf16_bits_to_f32(hi);
    }
  }
}

template <int D, int KB, int VB, int NQ, int KVDT>
__global__ __launch_bounds__(kAttnThreads) void attn_partial_kernel(AttnParams p) {
  constexpr bool PLAIN = (KB == 0);
  constexpr int CGK = 32;
  constexpr int LK = D / CGK;
  constexpr int TPWK = kWave / LK;
  constexpr int SLOTK = TPWK * kAttnWaves;
  constexpr int LV = 16;
  constexpr int CGV = D / LV;
  constexpr int TPWV = kWave / LV;
  constexpr int SLOTV = TPWV * kAttnWaves;
  constexpr int PWK = PLAIN ? 0 : D * KB / 32;
  constexpr int PWV = PLAIN ? 0 : D * VB / 32;

  extern __shared__ float smem[];
  float* s_w = smem;  // [chunk][NQ] scores -> weights; later [waves][NQ][D]
  __shared__ float s_q[NQ * D];  // rotated queries, later the merged rows
  __shared__ float s_kcb[16];
  __shared__ float s_vcb[16];
  __shared__ float s_red[kAttnWaves][NQ];
  __shared__ float s_ml[2 * NQ];
  __shared__ int s_last;

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int split = blockIdx.x;
  const int gk = blockIdx.y / p.n_rg;
  const int rg = blockIdx.y % p.n_rg;
  const int b = blockIdx.z;

  int64_t Tb = p.seq_lens ? static_cast<int64_t>(p.seq_lens[b]) : p.T;
  if (Tb > p.T) Tb = p.T;  // lengths beyond max_tokens are clipped
  const int64_t t_begin = static_cast<int64_t>(split) * p.chunk;
  const int rows = p.R * p.L;
  if (t_begin >= Tb) {
    // No tokens for this split.  An empty sequence still needs its output:
    // split 0 writes zeros (the reference divides a zero sum by 1e-6).
    if (Tb <= 0 && split == 0) {
      for (int idx = threadIdx.x; idx < NQ * D; idx += kAttnThreads) {
        const int rr = rg * NQ + idx / D;
        if (rr >= rows) continue;
        const int h = gk * p.R + rr / p.L;
        const int64_t qo = (static_cast<int64_t>(b) * p.Hq + h) * p.L + rr % p.L;
        store_out(p.out, p.q_dtype, qo * D + idx % D, 0.f);
      }
    }
    return;  // whole workgroup leaves together
  }
  const int64_t t_end = Tb < t_begin + p.chunk ? Tb : t_begin + p.chunk;
  const int n_tok = static_cast<int>(t_end - t_begin);
  const int nvalid = static_cast<int>((Tb + p.chunk - 1) / p.chunk);

  if constexpr (!PLAIN) {
    if (tid < (1 << KB)) s_kcb[tid] = p.kcb[tid];
    if (tid < (1 << VB)) s_vcb[tid] = p.vcb[tid];
  }

  // Query rows of this workgroup: rr = rg*NQ + j -> (rep, l) = (rr / L, rr % L).
  int64_t lim[NQ];  // causal: row may see keys t <= lim
  int64_t qoff[NQ];
  bool rvalid[NQ];
#pragma unroll
  for (int j = 0; j < NQ; ++j) {
    const int rr = rg * NQ + j;
    rvalid[j] = rr < rows;
    const int rep = rvalid[j] ? rr / p.L : 0;
    const int l = rvalid[j] ? rr % p.L : 0;
    const int h = gk * p.R + rep;
    qoff[j] = ((static_cast<int64_t>(b) * p.Hq + h) * p.L + l);
    lim[j] = p.causal ? (Tb - p.L + l) : INT64_MAX;
  }

  // ---------------------------------------------------------- prologue ----
  // q_s = round(q * scale_q) in the query dtype; then R_K.
  const bool dense = !PLAIN && p.rot_kind == TQ_ROT_DENSE;
  for (int idx = tid; idx < NQ * D; idx += kAttnThreads) {
    const int j = idx / D;
    const int d = idx % D;
    const int rr = rg * NQ + j;
    float val = 0.f;
    if (rr < rows) {
      const int h = gk * p.R + rr / p.L;
      const int l = rr % p.L;
      const int64_t qo = (static_cast<int64_t>(b) * p.Hq + h) * p.L + l;
      if (dense) {
        val = p.qrot[qo * D + d];
      } else {
        val = round_q(p.q_dtype, load_q(p.q, p.q_dtype, b * p.q_sb + h * p.q_sh + l * p.q_sl + d) *
                                     p.scale_q);
        if constexpr (!PLAIN) val *= p.krot[d];
      }
    }
    s_q[idx] = val;
  }
  __syncthreads();
  if constexpr (!PLAIN) {
    if (!dense) {
      lds_fwht<D, NQ>(s_q);
    }
  }

  // ------------------------------------------------------------ pass 1 ----
  const int gK = lane % LK;
  const int slotK = wave * TPWK + lane / LK;
  const float qmul = (!PLAIN && !dense) ? p.rscale : 1.f;
  float qreg[NQ][CGK];
#pragma unroll
  for (int j = 0; j < NQ; ++j) {
#pragma unroll
    for (int e = 0; e < CGK; ++e) qreg[j][e] = s_q[j * D + gK * CGK + e] * qmul;
  }

  const int64_t kvrow0 = (static_cast<int64_t>(b) * p.Hkv + gk) * p.cap;
  float mloc[NQ];
#pragma unroll
  for (int j = 0; j < NQ; ++j) mloc[j] = -INFINITY;

  for (int64_t t0 = t_begin; t0 < t_end; t0 += SLOTK) {
    const int64_t t = t0 + slotK;
    const bool valid = t < t_end;
    const int64_t tr = kvrow0 + (valid ? t : t_begin);
    float val[CGK];
    if constexpr (PLAIN) {
      const uint4* kp = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p.k) + tr * D +
                                                       gK * CGK);
#pragma unroll
      for (int i = 0; i < 4; ++i) unpack8<KVDT>(kp[i], &val[8 * i]);
    } else {
      const uint32_t* kp = static_cast<const uint32_t*>(p.k) + tr * PWK + gK * KB;
      uint32_t w[KB];
#pragma unroll
      for (int i = 0; i < KB; ++i) w[i] = kp[i];
#pragma unroll
      for (int e = 0; e < CGK; ++e) val[e] = s_kcb[field<KB>(w, e * KB)];
    }
    float acc[NQ];
#pragma unroll
    for (int j = 0; j < NQ; ++j) {
      float a = 0.f;
#pragma unroll
      for (int e = 0; e < CGK; ++e) a = fmaf(qreg[j][e], val[e], a);
      acc[j] = a;
    }
#pragma unroll
    for (int off = 1; off < LK; off <<= 1) {
#pragma unroll
      for (int j = 0; j < NQ; ++j) acc[j] += __shfl_xor(acc[j], off, kWave);
    }
    float nk = 1.f;
    if constexpr (!PLAIN) nk = load_norm(p.kn, p.norm_dtype, tr);
#pragma unroll
    for (int j = 0; j < NQ; ++j) {
      float s = acc[j] * nk;
      if (t > lim[j]) s = -FLT_MAX;
      if (!valid) s = -INFINITY;
      acc[j] = s;
      mloc[j] = fmaxf(mloc[j], s);
    }
    if (valid && gK == 0) {
#pragma unroll
      for (int j = 0; j < NQ; ++j) s_w[(t - t_begin) * NQ + j] = acc[j];
    }
  }

  // block max per row
#pragma unroll
  for (int j = 0; j < NQ; ++j) {
    float m = mloc[j];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, kWave));
    if (lane == 0) s_red[wave][j] = m;
  }
  __syncthreads();
  float mrow[NQ];
#pragma unroll
  for (int j = 0; j < NQ; ++j) {
    float m = s_red[0][j];
#pragma unroll
    for (int w = 1; w < kAttnWaves; ++w) m = fmaxf(m, s_red[w][j]);
    mrow[j] = m;
  }
  __syncthreads();

  // ------------------------------------------------------------ pass 2 ----
  float lsum[NQ];
#pragma unroll
  for (int j = 0; j < NQ; ++j) lsum[j] = 0.f;
  for (int i = tid; i < n_tok; i += kAttnThreads) {
    float nv = 1.f;
    if constexpr (!PLAIN) nv = load_norm(p.vn, p.norm_dtype, kvrow0 + t_begin + i);
#pragma unroll
    for (int j = 0; j < NQ; ++j) {
      const float pj = __expf(s_w[i * NQ + j] - mrow[j]);
      lsum[j] += pj;
      s_w[i * NQ + j] = pj * nv;
    }
  }
#pragma unroll
  for (int j = 0; j < NQ; ++j) {
    float s = lsum[j];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off, kWave);
    if (lane == 0) s_red[wave][j] = s;
  }
  __syncthreads();

  // ------------------------------------------------------------ pass 3 ----
  const int gV = lane % LV;
  const int slotV = wave * TPWV + lane / LV;
  float o[NQ][CGV];
#pragma unroll
  for (int j = 0; j < NQ; ++j)
#pragma unroll
    for (int e = 0; e < CGV; ++e) o[j][e] = 0.f;

  for (int64_t t0 = t_begin; t0 < t_end; t0 += SLOTV) {
    const int64_t t = t0 + slotV;
    if (t < t_end) {
      const int64_t tr = kvrow0 + t;
      float val[CGV];
      if constexpr (PLAIN) {
        const uint16_t* vp = static_cast<const uint16_t*>(p.v) + tr * D + gV * CGV;
        if constexpr (CGV >= 8) {
#pragma unroll
          for (int i = 0; i < CGV / 8; ++i) unpack8<KVDT>(reinterpret_cast<const uint4*>(vp)[i], &val[8 * i]);
        } else {
          const uint2 t2 = *reinterpret_cast<const uint2*>(vp);
          const uint16_t hv[4] = {static_cast<uint16_t>(t2.x & 0xffffu), static_cast<uint16_t>(t2.x >> 16),
                                  static_cast<uint16_t>(t2.y & 0xffffu), static_cast<uint16_t>(t2.y >> 16)};
#pragma unroll
          for (int i = 0; i < 4; ++i)
            val[i] = KVDT == TQ_DTYPE_F16 ? f16_bits_to_f32(hv[i]) : bf16_bits_to_f32(hv[i]);
        }
      } else {
        constexpr int VBITS = CGV * VB;
        constexpr bool ALIGNED = (VBITS % 32) == 0;
        constexpr int NRAW = ALIGNED ? VBITS / 32 : VBITS / 32 + 2;
        constexpr int NAL = ALIGNED ? NRAW : NRAW - 1;
        const uint32_t* vp = static_cast<const uint32_t*>(p.v) + tr * PWV;
        const int start = gV * VBITS;
        const int w0 = start >> 5;
        uint32_t al[NAL];
        if constexpr (ALIGNED) {
#pragma unroll
          for (int i = 0; i < NAL; ++i) al[i] = vp[w0 + i];
        } else {
          const int sh = start & 31;
          uint32_t raw[NRAW];
#pragma unroll
          for (int i = 0; i < NRAW; ++i) raw[i] = vp[min(w0 + i, PWV - 1)];
#pragma unroll
          for (int i = 0; i < NAL; ++i) al[i] = __builtin_amdgcn_alignbit(raw[i + 1], raw[i], sh);
        }
#pragma unroll
        for (int e = 0; e < CGV; ++e) val[e] = s_vcb[field<VB>(al, e * VB)];
      }
      const float* wp = s_w + (t - t_begin) * NQ;
      float w[NQ];
#pragma unroll
      for (int j = 0; j < NQ; ++j) w[j] = wp[j];
#pragma unroll
      for (int j = 0; j < NQ; ++j)
#pragma unroll
        for (int e = 0; e < CGV; ++e) o[j][e] = fmaf(w[j], val[e], o[j][e]);
    }
  }
  // fold the token slots of the wave (lanes gV, gV+16, gV+32, gV+48)
#pragma unroll
  for (int off = LV; off < kWave; off <<= 1)
#pragma unroll
    for (int j = 0; j < NQ; ++j)
#pragma unroll
      for (int e = 0; e < CGV; ++e) o[j][e] += __shfl_xor(o[j][e], off, kWave);

  float ltot[NQ];
#pragma unroll
  for (int j = 0; j < NQ; ++j) {
    float s = s_red[0][j];
#pragma unroll
    for (int w = 1; w < kAttnWaves; ++w) s += s_red[w][j];
    ltot[j] = s;
  }
  __syncthreads();  // all weight reads done: reuse s_w for the wave fold
  float* s_o = smem;  // [waves][NQ][D]
  if (lane < LV) {
#pragma unroll
    for (int j = 0; j < NQ; ++j)
#pragma unroll
      for (int e = 0; e < CGV; ++e) s_o[(wave * NQ + j) * D + gV * CGV + e] = o[j][e];
  }
  __syncthreads();
  // combine the waves into s_q and hand over to the split publication / merge
  for (int idx = tid; idx < NQ * D; idx += kAttnThreads) {
    float a = 0.f;
#pragma unroll
    for (int w = 0; w < kAttnWaves; ++w) a += s_o[w * NQ * D + idx];
    s_q[idx] = a;
  }
  if (tid < NQ) {
    float mv = mrow[0], lv = ltot[0];
#pragma unroll
    for (int jj = 1; jj < NQ; ++jj)
      if (jj == tid) {
        mv = mrow[jj];
        lv = ltot[jj];
      }
    s_ml[2 * tid] = mv;
    s_ml[2 * tid + 1] = lv;
  }
  __syncthreads();
  RowSet rs;
  rs.init(p, b, gk, rg, NQ);
  const int64_t grp = (static_cast<int64_t>(b) * p.Hkv + gk) * p.n_rg + rg;
  __shared__ float s_aux[NQ + D];
  publish_and_merge<D, NQ>(p, rs, s_q, s_ml, smem, s_aux, &s_last, grp, split, nvalid, PLAIN, dense);
}

template <int D, int KB, int VB, int KVDT>
int launch_partial_nq(const AttnParams& p, hipStream_t st) {
  const dim3 grid(p.n_splits, p.Hkv * p.n_rg, p.B);
  const SplitPlan sp{p.n_splits, p.chunk, p.n_rg, p.nq};
  const size_t lds = attn_lds_bytes(sp, D);
  switch (p.nq) {
    case 1:
      hipLaunchKernelGGL((attn_partial_kernel<D, KB, VB, 1, KVDT>), grid, dim3(kAttnThreads), lds, st, p);
      break;
    case 2:
      hipLaunchKernelGGL((attn_partial_kernel<D, KB, VB, 2, KVDT>), grid, dim3(kAttnThreads), lds, st, p);
      break;
    case 4:
      if constexpr (D < 256) {  // the planner caps D >= 256 at two rows (register budget)
        hipLaunchKernelGGL((attn_partial_kernel<D, KB, VB, 4, KVDT>), grid, dim3(kAttnThreads), lds, st, p);
        break;
      }
      [[fallthrough]];
    default:
      return fail(TQ_ERR_INVALID_ARGUMENT, "attention: rows per group %d", p.nq);
  }
  return check_launch("attn_partial_kernel");
}

template <int D, int KB>
int launch_partial_vb(const AttnParams& p, int vb, hipStream_t st) {
  switch (vb) {
    case 1: return launch_mfma_nq<D, KB, 1>(p, st);
    case 2: return launch_mfma_nq<D, KB, 2>(p, st);
    case 3: return launch_mfma_nq<D, KB, 3>(p, st);
    case 4: return launch_mfma_nq<D, KB, 4>(p, st);
  }
  return fail(TQ_ERR_INVALID_ARGUMENT, "attention: v_bits %d not in 1..4", vb);
}

template <int D>
int launch_partial_dim(const AttnParams& p, int kv_kind, int kv_dtype, int kb, int vb,
                       hipStream_t st) {
  if (kv_kind == TQ_KV_PLAIN) {
    if (kv_dtype == TQ_DTYPE_F16) return launch_partial_nq<D, 0, 0, TQ_DTYPE_F16>(p, st);
    if (kv_dtype == TQ_DTYPE_BF16) return launch_partial_nq<D, 0, 0, TQ_DTYPE_BF16>(p, st);
    return fail(TQ_ERR_INVALID_ARGUMENT, "attention: plain kv_dtype %d (F16/BF16)", kv_dtype);
  }
  switch (kb) {
    case 1: return launch_partial_vb<D, 1>(p, vb, st);
    case 2: return launch_partial_vb<D, 2>(p, vb, st);
    case 3: return launch_partial_vb<D, 3>(p, vb, st);
    case 4: return launch_partial_vb<D, 4>(p, vb, st);
  }
  return fail(TQ_ERR_INVALID_ARGUMENT, "attention: k_bits %d not in 1..4", kb);
}

}  // namespace tq
