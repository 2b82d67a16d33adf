// TurboQuant decode / verify attention straight from packed indices (gfx950).
//
// One workgroup (4 wave64s, one per SIMD, up to 512 VGPRs each) owns tokens
// [t_begin, t_end) of one kv head of one sequence and up to NQ query rows of
// that head's GQA group.  The tokens are cut into 32-token sub-chunks;
// sub-chunk i belongs to wave i % 4.  Each wave keeps the global loads of its
// next P sub-chunks in flight in registers (a software pipeline: the loads
// of sub-chunk i + P are issued as soon as sub-chunk i has been consumed), so
// a CU always has tens of KB of requests outstanding and HBM latency is
// covered without relying on other waves.  Per sub-chunk, with an online
// softmax (no workgroup barrier in the token loop):
//
//   keys   : D/32 lanes per token, 32 coordinates per lane = KB packed words,
//            the lane's 32 rotated query coordinates of every row in f32
//            registers.  Coordinates are taken in pairs: a 2*KB-bit field
//            indexes a pair table holding (c[i0], c[i1]) in f32, and two f32
//            FMAs per row add q[2c]*c[i0] + q[2c+1]*c[i1].  Scores are exact
//            f32 arithmetic (no logit-proportional rounding error).  The
//            token's lanes add their partial dots with xor shuffles.
//   softmax: sub-chunk max, rescale of the running (m, l, o), then
//            p = exp(s - m) and the value weight w = p * ||v|| (scaled into
//            [0, 1]) stored to LDS as f16, two tokens per 32-bit pair.
//   values : 16 lanes per token pair, D/16 coordinates per lane.  The two
//            tokens' indices of one coordinate form a 2*VB-bit key into the
//            value pair table, and v_dot2_f32_f16 with the weight pair adds
//            both tokens' contributions to the f32 accumulator.
//
// Pair tables live in LDS, replicated so that neighbouring lanes read
// distinct banks.  The value path is the only one in f16: the weights are
// scaled into [0, 1] by a power of two, and the value codebook by a scale
// chosen (identically in every workgroup) among 256 candidates for the
// smallest worst-case relative f16 rounding error, so that the codebook's
// rounding does not leave a common bias in every rotated coordinate (which
// the inverse Hadamard transform would pile into one output coordinate).
// Products in v_dot2_f32_f16 are exact and accumulate in f32; the remaining
// approximation is ~2^-12 relative on the value reconstruction.
#pragma once

#include "tq_attn_merge.h"

namespace tq {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pack_h2(float lo, float hi) {
  return static_cast<uint32_t>(f32_to_f16_bits(lo)) | (static_cast<uint32_t>(f32_to_f16_bits(hi)) << 16);
}

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, a), __builtin_bit_cast(half2_t, b), c, false);
}

// 2^-e such that max|x| * 2^-e lies in [0.5, 1) (1 for x == 0).
__device__ __forceinline__ float pow2_scale_for(float maxabs) {
  if (!(maxabs > 0.f) || !(maxabs < INFINITY)) return 1.f;
  int e;
  frexpf(maxabs, &e);
  return ldexpf(1.f, -e);
}

template <int B>
struct PairLut {
  static constexpr int KEYS = 1 << (2 * B);
  static constexpr int REP = KEYS <= 64 ? 16 : 4;  // replicas: spread lanes over banks
  static constexpr int WORDS = KEYS * REP;
};

// Replicated f16 pair table: entry k = (c[k & mask], c[k >> B]) * scale.
template <int B>
__device__ __forceinline__ void build_pair_lut(uint32_t* lut, const float* cb, float scale) {
  constexpr int mask = (1 << B) - 1;
  for (int i = threadIdx.x; i < PairLut<B>::WORDS; i += kAttnThreads) {
    const int k = i / PairLut<B>::REP;
    lut[i] = pack_h2(cb[k & mask] * scale, cb[k >> B] * scale);
  }
}

// Replicated f32 pair table: entry k = (c[k & mask], c[k >> B]).
template <int B>
__device__ __forceinline__ void build_pair_lut_f32(float2* lut, const float* cb) {
  constexpr int mask = (1 << B) - 1;
  for (int i = threadIdx.x; i < PairLut<B>::WORDS; i += kAttnThreads) {
    const int k = i / PairLut<B>::REP;
    lut[i] = make_float2(cb[k & mask], cb[k >> B]);
  }
}

// Codebook scale for f16 storage: among s = (0.5 + i/512) / max|c|,
// i = 0..255 (one candidate per thread), the one whose worst entry has the
// smallest |f16(c*s) - c*s| / |c*s| (ties: smallest i).  The comparison uses
// the same instructions in every workgroup, so all pick the same scale.
template <int B>
__device__ float f16_codebook_scale(const float* cb, float* s_err, int* s_idx) {
  float cm = 0.f;
#pragma unroll
  for (int i = 0; i < (1 << B); ++i) cm = fmaxf(cm, fabsf(cb[i]));
  if (!(cm > 0.f)) return 1.f;
  const int i = threadIdx.x;
  const float sc = (0.5f + i * (1.f / 512.f)) / cm;
  float best = 0.f;
#pragma unroll
  for (int j = 0; j < (1 << B); ++j) {
    const float v = cb[j] * sc;
    if (v != 0.f)
      best = fmaxf(best, fabsf(f16_bits_to_f32(f32_to_f16_bits(v)) - v) * __builtin_amdgcn_rcpf(fabsf(v)));
  }
  int besti = i;
  const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float ob = __shfl_xor(best, off, kWave);
    const int oi = __shfl_xor(besti, off, kWave);
    if (ob < best || (ob == best && oi < besti)) {
      best = ob;
      besti = oi;
    }
  }
  if (lane == 0) {
    s_err[threadIdx.x / kWave] = best;
    s_idx[threadIdx.x / kWave] = besti;
  }
  __syncthreads();
  float b2 = s_err[0];
  int i2 = s_idx[0];
#pragma unroll
  for (int w = 1; w < kAttnWaves; ++w)
    if (s_err[w] < b2 || (s_err[w] == b2 && s_idx[w] < i2)) {
      b2 = s_err[w];
      i2 = s_idx[w];
    }
  return (0.5f + i2 * (1.f / 512.f)) / cm;
}

// Registers holding one 32-token sub-chunk of a wave.
template <int KP, int KB, int VP, int NRAW>
struct SubBuf {
  uint32_t k[KP][KB];       // key words: one token per key pass
  float nk[KP];             // key norms of those tokens
  float nv[KP];             // value norms of those tokens (weight lanes)
  uint32_t v[VP][2][NRAW];  // value words: two tokens per value pass
};

template <int D, int KB, int VB, int NQ>
__global__ __launch_bounds__(kAttnThreads, 1) void attn_tq_kernel(AttnParams p) {
  constexpr int LK = D / 32;           // lanes per token, key pass
  constexpr int TPK = kWave / LK;      // tokens per key pass
  constexpr int SUB = 32;              // tokens per sub-chunk
  constexpr int KP = SUB / TPK;        // key passes per sub-chunk
  constexpr int LV = 16;               // lanes per token pair, value pass
  constexpr int CGV = D / LV;          // coordinates per lane, value pass
  constexpr int SLV = kWave / LV;      // token-pair slots per value pass
  constexpr int VP = SUB / (2 * SLV);  // value passes per sub-chunk
  constexpr int PWK = D * KB / 32;
  constexpr int PWV = D * VB / 32;
  constexpr int VBITS = CGV * VB;      // bits of one token a value lane reads
  constexpr bool VALIGNED = (VBITS % 32) == 0;
  constexpr int NRAW = VALIGNED ? VBITS / 32 : VBITS / 32 + 2;
  constexpr int NAL = VALIGNED ? NRAW : NRAW - 1;
  constexpr int REPK = PairLut<KB>::REP;
  constexpr int REPV = PairLut<VB>::REP;
  constexpr int P = 4;                 // sub-chunks in flight per wave
  static_assert(KP * TPK == SUB && VP * 2 * SLV == SUB, "sub-chunk shape");
  using Buf = SubBuf<KP, KB, VP, NRAW>;

  extern __shared__ float smem[];  // merge scratch
  __shared__ float2 s_lutk[PairLut<KB>::WORDS];
  __shared__ uint32_t s_lutv[PairLut<VB>::WORDS];
  __shared__ float s_q[NQ * D];                       // rotated queries; later merged rows
  __shared__ uint32_t s_wp[kAttnWaves][SUB / 2][NQ];  // value weight pairs (f16x2)
  __shared__ float s_wo[kAttnWaves * SLV][NQ * D];    // per-slot o for the workgroup combine
  __shared__ float s_wm[kAttnWaves][NQ];
  __shared__ float s_wl[kAttnWaves][NQ];
  __shared__ float s_ml[NQ * 2];
  __shared__ float s_vmax[kAttnWaves];
  __shared__ float s_serr[kAttnWaves];
  __shared__ int s_sidx[kAttnWaves];
  __shared__ float s_cbk[16];
  __shared__ float s_cbv[16];
  __shared__ float s_ksign[D];
  __shared__ int s_flag;

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int split = blockIdx.x;
  const int gk = blockIdx.y / p.n_rg;
  const int rg = blockIdx.y % p.n_rg;
  const int b = blockIdx.z;

  int64_t Tb = p.seq_lens ? static_cast<int64_t>(p.seq_lens[b]) : p.T;
  if (Tb > p.T) Tb = p.T;
  const int64_t t_begin = static_cast<int64_t>(split) * p.chunk;
  RowSet<NQ> rs;
  rs.init(p, b, gk, rg);
  if (t_begin >= Tb) {
    if (Tb <= 0 && split == 0) {  // empty sequence: zeros (0 / max(0, 1e-6))
      for (int idx = tid; idx < NQ * D; idx += kAttnThreads) {
        const int j = idx / D;
#pragma unroll
        for (int jj = 0; jj < NQ; ++jj)
          if (jj == j && rs.valid[jj]) store_out(p.out, p.q_dtype, rs.qoff[jj] * D + idx % D, 0.f);
      }
    }
    return;
  }
  const int64_t t_end = Tb < t_begin + p.chunk ? Tb : t_begin + p.chunk;
  const int n_tok = static_cast<int>(t_end - t_begin);
  const int nvalid = static_cast<int>((Tb + p.chunk - 1) / p.chunk);
  const int64_t kvrow0 = (static_cast<int64_t>(b) * p.Hkv + gk) * p.cap;
  const bool dense = p.rot_kind == TQ_ROT_DENSE;
  const uint32_t* kw = static_cast<const uint32_t*>(p.k);
  const uint32_t* vw = static_cast<const uint32_t*>(p.v);

  // lane roles
  const int gK = lane % LK;
  const int kslot = lane / LK;
  const int gV = lane % LV;
  const int vslot = lane / LV;
  const int lrk = lane % REPK;
  const int lrv = lane % REPV;
  const int vw0 = (gV * VBITS) >> 5;
  const int vsh = (gV * VBITS) & 31;

  // this wave's sub-chunks: i = 0 .. n_my-1 start at t_begin + (4i + wave) * SUB
  const int n_my = n_tok > wave * SUB ? (n_tok - wave * SUB + kAttnWaves * SUB - 1) / (kAttnWaves * SUB) : 0;
  auto sub_start = [&](int i) -> int64_t {
    return t_begin + static_cast<int64_t>(i * kAttnWaves + wave) * SUB;
  };
  auto load_sub = [&](Buf& bf, int64_t s0) {
#pragma unroll
    for (int kp = 0; kp < KP; ++kp) {
      int64_t t = s0 + kp * TPK + kslot;
      t = t < t_end ? t : t_end - 1;
      const uint32_t* r = kw + (kvrow0 + t) * PWK + gK * KB;
#pragma unroll
      for (int i = 0; i < KB; ++i) bf.k[kp][i] = r[i];
      bf.nk[kp] = load_norm(p.kn, p.norm_dtype, kvrow0 + t);
      bf.nv[kp] = load_norm(p.vn, p.norm_dtype, kvrow0 + t);
    }
#pragma unroll
    for (int vp = 0; vp < VP; ++vp)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        int64_t t = s0 + 2 * (vp * SLV + vslot) + h;
        t = t < t_end ? t : t_end - 1;
        const uint32_t* r = vw + (kvrow0 + t) * PWV;
#pragma unroll
        for (int i = 0; i < NRAW; ++i) bf.v[vp][h][i] = r[VALIGNED ? vw0 + i : min(vw0 + i, PWV - 1)];
      }
  };

  // ---- issue the pipeline's first loads before any prologue work
  Buf buf[P];
#pragma unroll
  for (int s = 0; s < P; ++s)
    if (s < n_my) load_sub(buf[s], sub_start(s));

  // ------------------------------------------------------------ prologue ----
  // codebooks and key signs to LDS, this thread's query elements to registers
  if (tid < (1 << KB)) s_cbk[tid] = p.kcb[tid];
  if (tid >= 32 && tid < 32 + (1 << VB)) s_cbv[tid - 32] = p.vcb[tid - 32];
  if (!dense)
    for (int d = tid; d < D; d += kAttnThreads) s_ksign[d] = p.krot[d];
  constexpr int QPT = (NQ * D + kAttnThreads - 1) / kAttnThreads;  // query elements per thread
  float qv[QPT];
#pragma unroll
  for (int i = 0; i < QPT; ++i) {
    const int idx = tid + i * kAttnThreads;
    const int j = idx / D;
    const int d = idx % D;
    qv[i] = 0.f;
#pragma unroll
    for (int jj = 0; jj < NQ; ++jj) {
      if (jj != j || idx >= NQ * D || !rs.valid[jj]) continue;
      qv[i] = dense ? p.qrot[rs.qoff[jj] * D + d]
                    : load_q(p.q, p.q_dtype,
                             b * p.q_sb + rs.head[jj] * p.q_sh + rs.lpos[jj] * p.q_sl + d);
    }
  }
  // value-norm scale over the chunk: w = p * ||v|| * vs stays in [0, 1]
  float vmax = 0.f;
  for (int64_t t = t_begin + tid; t < t_end; t += kAttnThreads)
    vmax = fmaxf(vmax, load_norm(p.vn, p.norm_dtype, kvrow0 + t));
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) vmax = fmaxf(vmax, __shfl_xor(vmax, off, kWave));
  if (lane == 0) s_vmax[wave] = vmax;
  __syncthreads();

  // pair tables: keys in f32, values in f16 at the chosen scale
  const float cbs_v = f16_codebook_scale<VB>(s_cbv, s_serr, s_sidx);
  build_pair_lut_f32<KB>(s_lutk, s_cbk);
  build_pair_lut<VB>(s_lutv, s_cbv, cbs_v);

  // queries: q_s = round(q * scale_q) * s_K, then the Hadamard butterflies
#pragma unroll
  for (int i = 0; i < QPT; ++i) {
    const int idx = tid + i * kAttnThreads;
    if (idx < NQ * D)
      s_q[idx] = dense ? qv[i] : round_q(p.q_dtype, qv[i] * p.scale_q) * s_ksign[idx % D];
  }
  __syncthreads();
  if (!dense) lds_fwht<D, NQ>(s_q);
  const float qmul = dense ? 1.f : p.rscale;
  const float vs = pow2_scale_for(fmaxf(fmaxf(s_vmax[0], s_vmax[1]), fmaxf(s_vmax[2], s_vmax[3])));
  float qf[NQ][32];
#pragma unroll
  for (int j = 0; j < NQ; ++j)
#pragma unroll
    for (int c = 0; c < 32; ++c) qf[j][c] = s_q[j * D + gK * 32 + c] * qmul;
  int64_t lim[NQ];  // causal: query row j sees keys t <= lim[j]
#pragma unroll
  for (int j = 0; j < NQ; ++j) lim[j] = p.causal ? (Tb - p.L + rs.lpos[j]) : INT64_MAX;

  // ------------------------------------------------------------ streaming ----
  float m_run[NQ], l_run[NQ];
  float o[NQ][CGV];
#pragma unroll
  for (int j = 0; j < NQ; ++j) {
    m_run[j] = -INFINITY;
    l_run[j] = 0.f;
#pragma unroll
    for (int e = 0; e < CGV; ++e) o[j][e] = 0.f;
  }

  auto process = [&](const Buf& bf, int64_t s0) {
    // ---- scores
    float sc[KP][NQ];
#pragma unroll
    for (int kp = 0; kp < KP; ++kp) {
      float acc[NQ];
#pragma unroll
      for (int j = 0; j < NQ; ++j) acc[j] = 0.f;
#pragma unroll
      for (int c = 0; c < 16; ++c) {
        const uint32_t key = field<2 * KB>(bf.k[kp], c * 2 * KB);
        const float2 cb2 = s_lutk[key * REPK + lrk];
#pragma unroll
        for (int j = 0; j < NQ; ++j) {
          acc[j] = fmaf(qf[j][2 * c], cb2.x, acc[j]);
          acc[j] = fmaf(qf[j][2 * c + 1], cb2.y, acc[j]);
        }
      }
#pragma unroll
      for (int off = 1; off < LK; off <<= 1)
#pragma unroll
        for (int j = 0; j < NQ; ++j) acc[j] += __shfl_xor(acc[j], off, kWave);
      const int64_t t = s0 + kp * TPK + kslot;
#pragma unroll
      for (int j = 0; j < NQ; ++j) {
        float s = acc[j] * bf.nk[kp];
        if (t > lim[j]) s = -FLT_MAX;
        if (t >= t_end) s = -INFINITY;
        sc[kp][j] = s;
      }
    }
    // ---- online softmax update
#pragma unroll
    for (int j = 0; j < NQ; ++j) {
      float cm = sc[0][j];
#pragma unroll
      for (int kp = 1; kp < KP; ++kp) cm = fmaxf(cm, sc[kp][j]);
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) cm = fmaxf(cm, __shfl_xor(cm, off, kWave));
      const float mn = fmaxf(m_run[j], cm);
      const float alpha = __expf(m_run[j] - mn);  // exp(-inf) = 0 on the first sub-chunk
      m_run[j] = mn;
      l_run[j] *= alpha;
#pragma unroll
      for (int e = 0; e < CGV; ++e) o[j][e] *= alpha;
    }
    // weights: lane gK of a token's lanes handles rows j with j % LK == gK
#pragma unroll
    for (int kp = 0; kp < KP; ++kp) {
      const int tl = kp * TPK + kslot;  // token index inside the sub-chunk
      uint16_t* wp16 = reinterpret_cast<uint16_t*>(&s_wp[wave][tl >> 1][0]) + (tl & 1);
#pragma unroll
      for (int j = 0; j < NQ; ++j) {
        if (j % LK != gK) continue;
        const float pj = __expf(sc[kp][j] - m_run[j]);
        l_run[j] += pj;
        wp16[2 * j] = f32_to_f16_bits(pj * bf.nv[kp] * vs);
      }
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    // ---- values
#pragma unroll
    for (int vp = 0; vp < VP; ++vp) {
      const int u = vp * SLV + vslot;  // token pair inside the sub-chunk
      uint32_t al[2][NAL];
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int i = 0; i < NAL; ++i)
          al[h][i] = VALIGNED ? bf.v[vp][h][i] : __builtin_amdgcn_alignbit(bf.v[vp][h][i + 1], bf.v[vp][h][i], vsh);
      uint32_t w2[NQ];
#pragma unroll
      for (int j = 0; j < NQ; ++j) w2[j] = s_wp[wave][u][j];
#pragma unroll
      for (int e = 0; e < CGV; ++e) {
        const uint32_t key = field<VB>(al[0], e * VB) | (field<VB>(al[1], e * VB) << VB);
        const uint32_t cb2 = s_lutv[key * REPV + lrv];
#pragma unroll
        for (int j = 0; j < NQ; ++j) o[j][e] = dot2(w2[j], cb2, o[j][e]);
      }
    }
    __builtin_amdgcn_wave_barrier();
  };

  for (int base = 0; base < n_my; base += P) {
#pragma unroll
    for (int s = 0; s < P; ++s) {
      const int i = base + s;
      if (i < n_my) {
        process(buf[s], sub_start(i));
        if (i + P < n_my) load_sub(buf[s], sub_start(i + P));
      }
    }
  }

  // ------------------------------------------------- combine the 4 waves ----
  // Each value slot of each wave writes its o through LDS; the partial
  // accumulators of a coordinate are then added with the softmax rescale.
#pragma unroll
  for (int j = 0; j < NQ; ++j) {
    float l = l_run[j];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) l += __shfl_xor(l, off, kWave);
    if (lane == 0) {
      s_wm[wave][j] = m_run[j];
      s_wl[wave][j] = l;
    }
  }
  const float oscale = 1.f / (vs * cbs_v);
#pragma unroll
  for (int j = 0; j < NQ; ++j)
#pragma unroll
    for (int e = 0; e < CGV; ++e) s_wo[wave * SLV + vslot][j * D + gV * CGV + e] = o[j][e] * oscale;
  __syncthreads();
  if (tid < NQ) {
    float M = s_wm[0][tid];
#pragma unroll
    for (int w = 1; w < kAttnWaves; ++w) M = fmaxf(M, s_wm[w][tid]);
    float L = 0.f;
#pragma unroll
    for (int w = 0; w < kAttnWaves; ++w) {
      const float wm = s_wm[w][tid];
      if (wm != -INFINITY) L += s_wl[w][tid] * __expf(wm - M);
    }
    s_ml[2 * tid] = M;
    s_ml[2 * tid + 1] = L;
  }
  __syncthreads();
  for (int idx = tid; idx < NQ * D; idx += kAttnThreads) {
    const int j = idx / D;
    const float M = s_ml[2 * j];
    float a = 0.f;
#pragma unroll
    for (int w = 0; w < kAttnWaves; ++w) {
      const float wm = s_wm[w][j];
      if (wm == -INFINITY) continue;
      float sw = 0.f;
#pragma unroll
      for (int sl = 0; sl < SLV; ++sl) sw += s_wo[w * SLV + sl][idx];
      a += sw * __expf(wm - M);
    }
    s_q[idx] = a;
  }
  __syncthreads();
  const int64_t grp = (static_cast<int64_t>(b) * p.Hkv + gk) * p.n_rg + rg;
  publish_and_merge<D, NQ>(p, rs, s_q, s_ml, smem, &s_flag, grp, split, nvalid, false, dense);
}

}  // namespace tq
