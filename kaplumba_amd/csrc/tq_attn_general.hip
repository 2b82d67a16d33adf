// Kernels and host side of the general attention path (see tq_attn_general.h).
#include <algorithm>

#include <cstdlib>

#include "tq_attn_general.h"
#include "tq_attn_merge.h"
#include "tq_attn_tile.h"

namespace tq {
namespace {

constexpr int kQpRows = 16;  // query rows per qprep workgroup

__device__ __forceinline__ float wave_sum(float x) {
  x += xor_lane<1>(x);
  x += xor_lane<2>(x);
  x += xor_lane<4>(x);
  x += xor_lane<8>(x);
  x += xor_lane<16>(x);
  const float2 h = halves(x);
  return h.x + h.y;
}

// Cache rows [start, start + len) of sequence b (as seq_window).
__device__ __forceinline__ void gen_window(const GenParams& p, int b, int64_t& start, int64_t& len) {
  int64_t end = p.seq_lens ? static_cast<int64_t>(p.seq_lens[b]) : p.T;
  end = end > p.T ? p.T : (end < 0 ? 0 : end);
  int64_t s = p.seq_starts ? static_cast<int64_t>(p.seq_starts[b]) : 0;
  s = s < 0 ? 0 : (s > end ? end : s);
  start = s;
  len = end - s;
}

// ------------------------------------------------------------------ qprep ---
// q_s = round_qdtype(q * scale_q) for kQpRows query rows, then
//   mode 0: dst = q_s                        (plain keys)
//   mode 1: dst = H(s * q_s) * rscale_k      (Hadamard, mat = the sign vector s;
//                                             _rht_forward, :3550-3561)
//   mode 2: dst = q_s @ mat^T                (dense R_K, :4144, or the Prod
//                                             projection, prepare_queries :4692-4698)
// dst rows have stride DkP, columns Dk..DkP-1 zero.  Mode 2 runs one workgroup
// per 64 output columns: thread (column c, quarter jq) sums a quarter of the
// coordinates for every row, the four quarters fold through LDS.
template <int QDT>
__global__ __launch_bounds__(kGenThreads) void gen_qprep_kernel(GenParams p, int64_t n_rows, int mode,
                                                                const float* __restrict__ mat,
                                                                float* __restrict__ dst) {
  __shared__ float4 s_q4[kQpRows * kGenMaxDim / 4];
  __shared__ float s_part[4][kQpRows][64];
  __shared__ int64_t s_off[kQpRows];
  float* s_q = reinterpret_cast<float*>(s_q4);
  const int tid = threadIdx.x;
  const int Dk = p.Dk;
  const int DkP = p.DkP;
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * kQpRows;
  const int nr = static_cast<int>(n_rows - row0 < kQpRows ? n_rows - row0 : kQpRows);  // rows of this block
  // element offset of each row's query (one division chain per row; rows
  // past the end repeat the block's first row and are dropped below)
  if (tid < kQpRows) {
    const int64_t row = row0 + (tid < nr ? tid : 0);
    const int l = static_cast<int>(row % p.L);
    const int64_t bh = row / p.L;
    const int h = static_cast<int>(bh % p.Hq);
    const int64_t b = bh / p.Hq;
    s_off[tid] = b * p.q_sb + h * p.q_sh + l * p.q_sl;
  }
  __syncthreads();
  // all of a thread's loads are issued before the first is used
  for (int d0 = 0; d0 < DkP; d0 += kGenThreads) {
    const int d = d0 + tid;
    const int dc = d < Dk ? d : 0;
    float v[kQpRows];
#pragma unroll
    for (int r = 0; r < kQpRows; ++r) v[r] = load_elem<QDT>(p.q, s_off[r] + dc);
    if (d < DkP) {
#pragma unroll
      for (int r = 0; r < kQpRows; ++r)
        s_q[r * DkP + d] = (r < nr && d < Dk) ? round_to<QDT>(v[r] * p.scale_q) : 0.f;
    }
  }
  __syncthreads();
  if (mode == 2) {
    const int c = tid % 64;
    const int jq = tid / 64;
    const int col = blockIdx.y * 64 + c;
    // quarter jq of the 4-coordinate groups; the last quarter also takes the
    // Dk % 4 coordinates past them (rows of mat are 16-byte aligned only when
    // Dk % 4 == 0: other dims read them one element at a time)
    const int n4 = Dk / 4;
    const int a4 = jq * n4 / 4;
    const int b4 = (jq + 1) * n4 / 4;
    float acc[kQpRows];
#pragma unroll
    for (int r = 0; r < kQpRows; ++r) acc[r] = 0.f;
    if (col < Dk) {
      const float* mr = mat + static_cast<int64_t>(col) * Dk;
      const bool vec4 = (Dk & 3) == 0;
      for (int m = a4; m < b4; ++m) {
        const float4 rv = vec4 ? reinterpret_cast<const float4*>(mr)[m]
                               : make_float4(mr[4 * m], mr[4 * m + 1], mr[4 * m + 2], mr[4 * m + 3]);
#pragma unroll
        for (int r = 0; r < kQpRows; ++r) {
          const float4 qv = s_q4[r * (DkP / 4) + m];
          acc[r] = fmaf(qv.x, rv.x, acc[r]);
          acc[r] = fmaf(qv.y, rv.y, acc[r]);
          acc[r] = fmaf(qv.z, rv.z, acc[r]);
          acc[r] = fmaf(qv.w, rv.w, acc[r]);
        }
      }
      if (jq == 3)
        for (int d = 4 * n4; d < Dk; ++d) {
          const float rv = mr[d];
#pragma unroll
          for (int r = 0; r < kQpRows; ++r) acc[r] = fmaf(s_q[r * DkP + d], rv, acc[r]);
        }
    }
#pragma unroll
    for (int r = 0; r < kQpRows; ++r) s_part[jq][r][c] = acc[r];
    __syncthreads();
    for (int idx = tid; idx < kQpRows * 64; idx += kGenThreads) {
      const int r = idx / 64;
      const int cc = idx % 64;
      const int64_t row = row0 + r;
      const int colx = blockIdx.y * 64 + cc;
      if (row < n_rows && colx < DkP)
        dst[row * DkP + colx] =
            colx < Dk ? (s_part[0][r][cc] + s_part[1][r][cc]) + (s_part[2][r][cc] + s_part[3][r][cc]) : 0.f;
    }
    return;
  }
  float scl = 1.f;
  if (mode == 1) {
    for (int r = 0; r < kQpRows; ++r)
      for (int d = tid; d < Dk; d += kGenThreads) s_q[r * DkP + d] *= mat[d];
    __syncthreads();
    // butterflies of distance 1, 2, ..., Dk/2 over each row (stride DkP):
    // thread (row r0 + j * rpp, pair k); Dk is a power of two here
    const int hp = Dk / 2;
    const int rpp = hp < kGenThreads ? kGenThreads / hp : 1;
    const int r0 = tid / hp;
    const int k0 = tid % hp;
    for (int hs = 1; hs < Dk; hs <<= 1) {
      for (int k = k0; k < hp; k += kGenThreads)
        for (int r = r0; r < kQpRows; r += rpp) {
          const int i0 = r * DkP + ((k & ~(hs - 1)) << 1) + (k & (hs - 1));
          const float a = s_q[i0];
          const float b = s_q[i0 + hs];
          s_q[i0] = a + b;
          s_q[i0 + hs] = a - b;
        }
      __syncthreads();
    }
    scl = p.rscale_k;
  }
  for (int r = 0; r < nr; ++r)
    for (int d = tid; d < DkP; d += kGenThreads) dst[(row0 + r) * DkP + d] = s_q[r * DkP + d] * scl;
}

// -------------------------------------------------------------- partial ---
template <int KB>
__device__ __forceinline__ uint32_t group_field(const uint32_t (&w)[KB > 0 ? KB : 1], int j) {
  if constexpr (KB == 0) {
    return 0u;
  } else {
    return field<KB, KB>(w, j * KB);
  }
}

__device__ __forceinline__ float mask_apply(const GenParams& p, int64_t off, float x) {
  switch (p.mask_kind) {
    case TQ_MASK_BOOL:
      return static_cast<const uint8_t*>(p.mask)[off] ? x : -FLT_MAX;
    case TQ_MASK_ADD_F32:
      return x + static_cast<const float*>(p.mask)[off];
    case TQ_MASK_ADD_F16:
      return x + f16_bits_to_f32(static_cast<const uint16_t*>(p.mask)[off]);
    case TQ_MASK_ADD_BF16:
      return x + bf16_bits_to_f32(static_cast<const uint16_t*>(p.mask)[off]);
    default:
      return x;
  }
}

// One split of one (sequence, kv head, row group).  KIND: GenKeyKind; KB: key
// (MSE part) bits, 0 for plain keys and 1-bit Prod; VB: value bits, 0 for
// plain values (with plain keys).
template <int KIND, int KB, int VB>
__global__ __launch_bounds__(kGenThreads) void gen_partial_kernel(GenParams p) {
  constexpr bool PROD = KIND == kGenProd;
  constexpr bool PLAIN = KIND == kGenPlainF16 || KIND == kGenPlainBf16;
  constexpr int PDT = KIND == kGenPlainBf16 ? TQ_DTYPE_BF16 : TQ_DTYPE_F16;
  constexpr int NQ = kGenNQ;
  constexpr int TT = kGenTT;
  static_assert(NQ == 8, "two softmax rows per wave, two float4 weight reads per token");
  __shared__ float4 s_q4[NQ * kGenMaxDim / 4];  // query rows (stride DkP); the epilogue's sums
  __shared__ float4 s_qp4[PROD ? NQ * kGenMaxDim / 4 : 1];
  __shared__ float s_part[PROD ? 8 : 4][NQ][TT];
  __shared__ float4 s_pv4[TT][NQ / 4];  // p * ||v|| per token and row
  __shared__ float s_alpha[NQ];
  __shared__ float s_kcb[16];
  __shared__ float s_vcb[16];
  float* s_q = reinterpret_cast<float*>(s_q4);
  float* s_qp = reinterpret_cast<float*>(s_qp4);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int split = blockIdx.x;
  const int gk = blockIdx.y / p.n_rg;
  const int rg = blockIdx.y % p.n_rg;
  const int b = blockIdx.z;
  const int row0 = rg * NQ;
  const int nrows = min(NQ, p.R * p.L - row0);
  const int64_t gi = (static_cast<int64_t>(b) * p.Hkv + gk) * p.n_rg + rg;
  float* pml = p.pml + (gi * p.n_splits + split) * NQ * 2;
  float* po = p.po + (gi * p.n_splits + split) * NQ * p.Dv;
  int64_t start, len;
  gen_window(p, b, start, len);
  const int64_t t_begin = static_cast<int64_t>(split) * p.chunk;
  const int64_t t_end = min(len, t_begin + p.chunk);
  if (t_begin >= t_end) {  // no tokens: a neutral partial (the merge skips it)
    if (tid < NQ) {
      pml[2 * tid] = -INFINITY;
      pml[2 * tid + 1] = 0.f;
    }
    return;
  }
  const int Dk = p.Dk;
  const int DkP = p.DkP;
  const int Dv = p.Dv;
  // query rows: row i -> head gk*R + (row0+i)/L, position (row0+i)%L
  for (int idx = tid; idx < NQ * DkP; idx += kGenThreads) {
    const int i = idx / DkP;
    const int d = idx % DkP;
    float v = 0.f, vp = 0.f;
    if (i < nrows) {
      const int rr = row0 + i;
      const int64_t qrow = (static_cast<int64_t>(b) * p.Hq + gk * p.R + rr / p.L) * p.L + rr % p.L;
      if (KB > 0 || PLAIN) v = p.qrot[qrow * DkP + d];
      if constexpr (PROD) vp = p.qproj[qrow * DkP + d];
    }
    s_q[idx] = v;
    if constexpr (PROD) s_qp[idx] = vp;
  }
  if constexpr (KB > 0)
    if (tid < (1 << KB)) s_kcb[tid] = p.kcb[tid];
  if constexpr (VB > 0)
    if (tid < (1 << VB)) s_vcb[tid] = p.vcb[tid];
  __syncthreads();

  const int64_t rowbase = (static_cast<int64_t>(b) * p.Hkv + gk) * p.cap + start;
  // softmax rows of this wave: wave, wave + 4
  float m_run[2] = {-INFINITY, -INFINITY};
  float l_run[2] = {0.f, 0.f};
  int64_t mrow[2] = {0, 0};
  int64_t lim[2] = {0, 0};
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const int i = wave + 4 * s;
    const int rr = row0 + (i < nrows ? i : 0);
    const int r = rr / p.L;
    const int l = rr % p.L;
    lim[s] = len - p.L + l;  // causal: relative token t is visible iff t <= lim
    mrow[s] = b * p.m_sb + gk * p.m_sg + r * p.m_sr + l * p.m_sl;
  }
  // value mapping: coordinate pair d0, d0 + 1 of token subset ts
  const int NP = p.DvP / 2;
  const int pi = tid % NP;
  const int ts = tid / NP;
  const int TPT = TT / (kGenThreads / NP);
  const int d0 = 2 * pi;
  const bool vact = d0 < Dv;
  float acc[NQ][2];
#pragma unroll
  for (int i = 0; i < NQ; ++i) acc[i][0] = acc[i][1] = 0.f;
  const int vbit = d0 * (VB > 0 ? VB : 1);
  const int vw0 = vbit >> 5;
  const int vsh = vbit & 31;
  const bool vtwo = VB == 3 && vw0 + 1 < p.vpw;
  const int G = DkP / 32;
  const bool k_vec8 = (Dk & 7) == 0;  // plain key rows 16-byte aligned

  for (int64_t t0 = t_begin; t0 < t_end; t0 += TT) {
    const int n = static_cast<int>(min<int64_t>(TT, t_end - t0));
    const bool tv = lane < n;
    const int64_t tr = t0 + lane;  // token of this lane, relative to the window
    // ---- partial scores: wave = group slice, lane = token
    float sm[NQ], sq[NQ];
#pragma unroll
    for (int i = 0; i < NQ; ++i) sm[i] = sq[i] = 0.f;
    for (int g = wave; g < G; g += 4) {
      if constexpr (PLAIN) {
        const uint16_t* kr = static_cast<const uint16_t*>(p.k) + (rowbase + tr) * Dk + 32 * g;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          // 8 keys in one 16-byte load when Dk % 8 == 0 (rows 16-byte
          // aligned); else one element at a time, zeros past Dk
          uint4 h = make_uint4(0, 0, 0, 0);
          const int c0 = 32 * g + 8 * u;
          if (tv && c0 < Dk) {
            if (k_vec8) {
              h = reinterpret_cast<const uint4*>(kr)[u];
            } else {
              uint32_t e16[8];
#pragma unroll
              for (int e = 0; e < 8; ++e) e16[e] = c0 + e < Dk ? kr[8 * u + e] : 0u;
              h = make_uint4(e16[0] | (e16[1] << 16), e16[2] | (e16[3] << 16), e16[4] | (e16[5] << 16),
                             e16[6] | (e16[7] << 16));
            }
          }
          const uint32_t hw[4] = {h.x, h.y, h.z, h.w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float k0 = PDT == TQ_DTYPE_BF16 ? bf16_bits_to_f32(hw[e] & 0xffffu) : f16_bits_to_f32(hw[e] & 0xffffu);
            const float k1 = PDT == TQ_DTYPE_BF16 ? bf16_bits_to_f32(hw[e] >> 16) : f16_bits_to_f32(hw[e] >> 16);
#pragma unroll
            for (int i = 0; i < NQ; ++i) {
              const float2 qv = reinterpret_cast<const float2*>(s_q)[(i * DkP + 32 * g + 8 * u + 2 * e) / 2];
              sm[i] = fmaf(qv.x, k0, sm[i]);
              sm[i] = fmaf(qv.y, k1, sm[i]);
            }
          }
        }
      } else {
        uint32_t w[KB > 0 ? KB : 1];
        w[0] = 0;
        if constexpr (KB > 0) {
          const uint32_t* kr = static_cast<const uint32_t*>(p.k) + (rowbase + tr) * p.kpw;
#pragma unroll
          for (int u = 0; u < KB; ++u) {
            const int wi = g * KB + u;
            w[u] = (tv && wi < p.kpw) ? kr[wi] : 0u;
          }
        }
        uint32_t sw = 0;
        // ceil(Dk / 32) sign words per row: group g is word g (G of them)
        if constexpr (PROD) sw = tv ? static_cast<const uint32_t*>(p.ksg)[(rowbase + tr) * G + g] : 0u;
#pragma unroll
        for (int j4 = 0; j4 < 8; ++j4) {
          float c[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) c[e] = KB > 0 ? s_kcb[group_field<KB>(w, 4 * j4 + e)] : 0.f;
#pragma unroll
          for (int i = 0; i < NQ; ++i) {
            if constexpr (KB > 0) {
              const float4 qv = s_q4[(i * DkP + 32 * g) / 4 + j4];
              sm[i] = fmaf(qv.x, c[0], sm[i]);
              sm[i] = fmaf(qv.y, c[1], sm[i]);
              sm[i] = fmaf(qv.z, c[2], sm[i]);
              sm[i] = fmaf(qv.w, c[3], sm[i]);
            }
            if constexpr (PROD) {
              const float4 pv = s_qp4[(i * DkP + 32 * g) / 4 + j4];
              const float pe[4] = {pv.x, pv.y, pv.z, pv.w};
#pragma unroll
              for (int e = 0; e < 4; ++e) sq[i] += ((sw >> (4 * j4 + e)) & 1u) ? pe[e] : -pe[e];
            }
          }
        }
      }
    }
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      s_part[wave][i][lane] = sm[i];
      if constexpr (PROD) s_part[4 + wave][i][lane] = sq[i];
    }
    __syncthreads();
    // ---- online softmax: wave owns rows wave and wave + 4, lane = token
    float kn = 0.f, vn = 0.f, rn = 0.f;
    if (tv) {
      if constexpr (!PLAIN) {
        kn = load_norm(p.kn, p.norm_dtype, rowbase + tr);
        vn = load_norm(p.vn, p.norm_dtype, rowbase + tr);
      } else {
        vn = 1.f;
      }
      if constexpr (PROD) rn = load_norm(p.krn, p.norm_dtype, rowbase + tr);
    }
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int i = wave + 4 * s;
      float* pvrow = reinterpret_cast<float*>(s_pv4);
      if (i >= nrows) {
        pvrow[lane * NQ + i] = 0.f;
        if (lane == 0) s_alpha[i] = 1.f;
        continue;
      }
      float x = -INFINITY;
      if (tv) {
        const float dot = (s_part[0][i][lane] + s_part[1][i][lane]) + (s_part[2][i][lane] + s_part[3][i][lane]);
        if constexpr (PLAIN) {
          x = dot;
        } else if constexpr (PROD) {
          const float qd = (s_part[4][i][lane] + s_part[5][i][lane]) + (s_part[6][i][lane] + s_part[7][i][lane]);
          const float qjl = p.qjl_scale * rn * qd;
          x = KB > 0 ? kn * dot + kn * qjl : kn * qjl;
        } else {
          x = kn * dot;
        }
        if (p.causal && tr > lim[s]) x = -FLT_MAX;
        if (p.mask_kind != TQ_MASK_NONE) x = mask_apply(p, mrow[s] + (start + tr) * p.m_st, x);
      }
      const float mt = wave_max(x);
      const float mnew = fmaxf(m_run[s], mt);
      float alpha = 1.f, pe = 0.f;
      if (mnew != -INFINITY) {
        alpha = expf(m_run[s] - mnew);
        pe = expf(x - mnew);
      }
      l_run[s] = l_run[s] * alpha + wave_sum(pe);
      m_run[s] = mnew;
      pvrow[lane * NQ + i] = pe * vn;
      if (lane == 0) s_alpha[i] = alpha;
    }
    __syncthreads();
    // ---- weighted value sum: thread = coordinate pair x token subset
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      const float a = s_alpha[i];
      acc[i][0] *= a;
      acc[i][1] *= a;
    }
    if (vact) {
      const int tb = ts * TPT;
      const int te = min(tb + TPT, n);
      for (int tt0 = tb; tt0 < te; tt0 += 4) {
        float c0[4], c1[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int tt = tt0 + u;
          const bool ok = tt < te;
          const int64_t trow = rowbase + t0 + tt;
          if constexpr (VB == 0) {
            uint32_t hw = 0;
            if (ok) {
              // an element pair in one 4-byte load when Dv is even; else two
              // loads, the second only inside the row
              const uint16_t* ve = static_cast<const uint16_t*>(p.v) + trow * Dv + d0;
              if ((Dv & 1) == 0)
                hw = *reinterpret_cast<const uint32_t*>(ve);
              else
                hw = ve[0] | (d0 + 1 < Dv ? static_cast<uint32_t>(ve[1]) << 16 : 0u);
            }
            c0[u] = PDT == TQ_DTYPE_BF16 ? bf16_bits_to_f32(hw & 0xffffu) : f16_bits_to_f32(hw & 0xffffu);
            c1[u] = PDT == TQ_DTYPE_BF16 ? bf16_bits_to_f32(hw >> 16) : f16_bits_to_f32(hw >> 16);
          } else {
            const uint32_t* vr = static_cast<const uint32_t*>(p.v) + trow * p.vpw;
            const uint32_t a = ok ? vr[vw0] : 0u;
            const uint32_t a2 = (ok && vtwo) ? vr[vw0 + 1] : 0u;
            const uint32_t x = VB == 3 ? __builtin_amdgcn_alignbit(a2, a, vsh) : (a >> vsh);
            constexpr uint32_t M = (1u << (VB > 0 ? VB : 1)) - 1u;
            c0[u] = s_vcb[x & M];
            c1[u] = s_vcb[(x >> (VB > 0 ? VB : 1)) & M];
          }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          if (tt0 + u >= te) break;
          const float4 w0 = s_pv4[tt0 + u][0];
          const float4 w1 = s_pv4[tt0 + u][1];
          const float wv[NQ] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
          for (int i = 0; i < NQ; ++i) {
            acc[i][0] = fmaf(wv[i], c0[u], acc[i][0]);
            acc[i][1] = fmaf(wv[i], c1[u], acc[i][1]);
          }
        }
      }
    }
    __syncthreads();
  }
  // ---- epilogue: (max, sum) per row; o summed over the token subsets
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const int i = wave + 4 * s;
    if (i < nrows && lane == 0) {
      pml[2 * i] = m_run[s];
      pml[2 * i + 1] = l_run[s];
    }
  }
  float* s_o = s_q;  // [subset][NQ][DvP]: (256 / NP) * NQ * DvP = NQ * 512 floats
  const int DvP = p.DvP;
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
    s_o[(ts * NQ + i) * DvP + d0] = acc[i][0];
    s_o[(ts * NQ + i) * DvP + d0 + 1] = acc[i][1];
  }
  __syncthreads();
  const int nsub = kGenThreads / NP;
  for (int idx = tid; idx < nrows * Dv; idx += kGenThreads) {
    const int i = idx / Dv;
    const int d = idx % Dv;
    float o = 0.f;
    for (int s = 0; s < nsub; ++s) o += s_o[(s * NQ + i) * DvP + d];
    po[i * Dv + d] = o;
  }
}

// ---------------------------------------------------------------- merge ---
// grid (kv head * row group, sequence, column block): the splits' partials of
// every row of the group combined by log-sum-exp, normalised by
// 1/max(sum, 1e-6), then R_V^-1: Hadamard butterflies over whole rows (one
// column block) or, for the dense rotation, the 64 output columns of this
// block (thread = column x quarter of the contraction); plain values are
// stored as they are.
__global__ __launch_bounds__(kGenThreads) void gen_merge_kernel(GenParams p) {
  constexpr int NQ = kGenNQ;
  __shared__ float s_w[kGenMaxSplits * NQ];
  __shared__ float4 s_y4[NQ * kGenMaxDim / 4];
  __shared__ float s_part[4][NQ][64];
  __shared__ float s_l[NQ];
  float* s_y = reinterpret_cast<float*>(s_y4);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int gk = blockIdx.x / p.n_rg;
  const int rg = blockIdx.x % p.n_rg;
  const int b = blockIdx.y;
  const int row0 = rg * NQ;
  const int nrows = min(NQ, p.R * p.L - row0);
  const int ns = p.n_splits;
  const int Dv = p.Dv;
  const int DvP = p.DvP;
  const int64_t gi = (static_cast<int64_t>(b) * p.Hkv + gk) * p.n_rg + rg;
  const float* pml = p.pml + gi * ns * NQ * 2;
  const float* po = p.po + gi * ns * NQ * Dv;
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const int i = wave + 4 * s;
    if (i >= nrows) continue;
    float mx = -INFINITY;
    for (int k = lane; k < ns; k += 64) mx = fmaxf(mx, pml[(k * NQ + i) * 2]);
    mx = wave_max(mx);
    float lsum = 0.f;
    for (int k = lane; k < ns; k += 64) {
      const float m = pml[(k * NQ + i) * 2];
      const float w = (m == -INFINITY) ? 0.f : expf(m - mx);
      s_w[k * NQ + i] = w;
      lsum += w * pml[(k * NQ + i) * 2 + 1];
    }
    lsum = wave_sum(lsum);
    if (lane == 0) s_l[i] = lsum;
  }
  __syncthreads();
  for (int idx = tid; idx < NQ * DvP; idx += kGenThreads) {
    const int i = idx / DvP;
    const int d = idx % DvP;
    float y = 0.f;
    if (i < nrows && d < Dv) {
      float a = 0.f;
      for (int k = 0; k < ns; ++k) {
        const float w = s_w[k * NQ + i];
        if (w != 0.f) a = fmaf(w, po[(k * NQ + i) * Dv + d], a);
      }
      y = a / fmaxf(s_l[i], kNormEps);
    }
    s_y[idx] = y;
  }
  __syncthreads();
  const bool plain = p.key_kind == kGenPlainF16 || p.key_kind == kGenPlainBf16 || p.po_natural;
  auto out_off = [&](int i) {
    const int rr = row0 + i;
    return ((static_cast<int64_t>(b) * p.Hq + gk * p.R + rr / p.L) * p.L + rr % p.L) * Dv;
  };
  if (!plain && p.v_rot_kind == TQ_ROT_DENSE) {
    const int c = tid % 64;
    const int jq = tid / 64;
    const int col = blockIdx.z * 64 + c;
    const int a = jq * Dv / 4;
    const int e = (jq + 1) * Dv / 4;
    float acc[NQ];
#pragma unroll
    for (int i = 0; i < NQ; ++i) acc[i] = 0.f;
    if (col < Dv) {
      for (int d = a; d < e; ++d) {
        const float r = p.vrot[static_cast<int64_t>(d) * Dv + col];
#pragma unroll
        for (int i = 0; i < NQ; ++i) acc[i] = fmaf(s_y[i * DvP + d], r, acc[i]);
      }
    }
#pragma unroll
    for (int i = 0; i < NQ; ++i) s_part[jq][i][c] = acc[i];
    __syncthreads();
    for (int idx = tid; idx < nrows * 64; idx += kGenThreads) {
      const int i = idx / 64;
      const int cc = idx % 64;
      const int colx = blockIdx.z * 64 + cc;
      if (colx < Dv)
        store_out(p.out, p.q_dtype, out_off(i) + colx,
                  (s_part[0][i][cc] + s_part[1][i][cc]) + (s_part[2][i][cc] + s_part[3][i][cc]));
    }
    return;
  }
  if (!plain) {
    for (int hs = 1; hs < Dv; hs <<= 1) {
      for (int idx = tid; idx < nrows * (Dv / 2); idx += kGenThreads) {
        const int i = idx / (Dv / 2);
        const int k = idx % (Dv / 2);
        const int i0 = i * DvP + (k / hs) * 2 * hs + (k % hs);
        const float x0 = s_y[i0];
        const float x1 = s_y[i0 + hs];
        s_y[i0] = x0 + x1;
        s_y[i0 + hs] = x0 - x1;
      }
      __syncthreads();
    }
  }
  for (int idx = tid; idx < nrows * Dv; idx += kGenThreads) {
    const int i = idx / Dv;
    const int d = idx % Dv;
    float r = s_y[i * DvP + d];
    if (!plain) r = r * p.rscale_v * p.vrot[d];
    store_out(p.out, p.q_dtype, out_off(i) + d, r);
  }
}

// Element-wise merge: partials in the natural basis (plain values), or the
// tile kernel's Hadamard-rotated ones (merge_had, Dv = 128).  Thread = (row,
// 4 output columns): the splits' (m, l) and o by log-sum-exp, / max(l,
// 1e-6); for merge_had then R_V^-1 on the merged row (the 32 threads of a
// row are 32 consecutive lanes: butterflies over the 4 columns in registers,
// over column bits 2-6 across lanes, then the signs and 1/sqrt(Dv), the
// order of _rht_inverse, turboquant_cache.py:3564-3575); output in the
// query dtype.  A split without tokens (m = -inf) has no o written; it is
// selected away, never multiplied.  Index type I: int when the item count
// fits, so no 64-bit divisions.
template <typename I>
__global__ __launch_bounds__(256) void gen_merge_flat_kernel(GenParams p, I n_items) {
  I blk = static_cast<I>(blockIdx.x);
  if (p.merge_bpp > 0) {
    // the blocks of (b, kv head) pair q run on XCD q % 8, where the tile
    // kernel wrote that pair's partials (workgroup id % 8 picks the XCD)
    const I k = blk >> 3;
    const I pair = (blk & 7) + 8 * (k / p.merge_bpp);
    blk = pair * p.merge_bpp + k % p.merge_bpp;
  }
  const I idx = blk * 256 + static_cast<I>(threadIdx.x);
  if (idx >= n_items) return;
  const int C4 = p.Dv / 4;
  const I RL = static_cast<I>(p.R) * p.L;
  const int c4 = static_cast<int>(idx % C4);
  const I row = idx / C4;  // (b * Hkv + gk) * RL + rr
  const int rr = static_cast<int>(row % RL);
  const I bg = row / RL;
  const int gk = static_cast<int>(bg % p.Hkv);
  const I b = bg / p.Hkv;
  const int64_t gi = static_cast<int64_t>(bg) * p.n_rg + rr / 8;
  const int ns = p.n_splits;
  const int64_t r0 = gi * ns * kGenNQ + rr % 8;  // split k: partial r0 + k * kGenNQ
  const float2* ml = reinterpret_cast<const float2*>(p.pml) + r0;
  const float4* po = reinterpret_cast<const float4*>(p.po) + r0 * C4 + c4;
  const int64_t ostep = static_cast<int64_t>(kGenNQ) * C4;
  // chunks of 8 splits: every load of a chunk in flight at once, one
  // rescale of the running sums per chunk
  float M = -INFINITY;
  float Lsum = 0.f;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int k0 = 0; k0 < ns; k0 += 8) {
    float2 m[8];
    float4 v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int k = k0 + u < ns ? k0 + u : k0;  // past the last split: reread one (dropped below)
      m[u] = ml[k * kGenNQ];
      v[u] = po[k * ostep];
    }
    float bm = M;
#pragma unroll
    for (int u = 0; u < 8; ++u) bm = k0 + u < ns ? fmaxf(bm, m[u].x) : bm;
    if (bm == -INFINITY) continue;
    const float r = M == -INFINITY ? 0.f : expf(M - bm);
    Lsum *= r;
    acc.x *= r;
    acc.y *= r;
    acc.z *= r;
    acc.w *= r;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const bool live = k0 + u < ns && m[u].x != -INFINITY;
      const float sc = live ? expf(m[u].x - bm) : 0.f;
      Lsum = fmaf(sc, m[u].y, Lsum);
      acc.x = live ? fmaf(sc, v[u].x, acc.x) : acc.x;
      acc.y = live ? fmaf(sc, v[u].y, acc.y) : acc.y;
      acc.z = live ? fmaf(sc, v[u].z, acc.z) : acc.z;
      acc.w = live ? fmaf(sc, v[u].w, acc.w) : acc.w;
    }
    M = bm;
  }
  const float inv = M == -INFINITY ? 0.f : 1.f / fmaxf(Lsum, kNormEps);
  const int64_t o = ((static_cast<int64_t>(b) * p.Hq + gk * p.R + rr / p.L) * p.L + rr % p.L) * p.Dv + 4 * c4;
  float v0 = acc.x * inv, v1 = acc.y * inv, v2 = acc.z * inv, v3 = acc.w * inv;
  if (p.merge_had) {
    const float a0 = v0 + v1, a1 = v0 - v1, a2 = v2 + v3, a3 = v2 - v3;
    v0 = a0 + a2;
    v2 = a0 - a2;
    v1 = a1 + a3;
    v3 = a1 - a3;
    float o;
#define TQ_MERGE_STAGE(HB)                 \
  o = xor_lane<HB>(v0);                    \
  v0 = (c4 & HB) ? o - v0 : v0 + o;        \
  o = xor_lane<HB>(v1);                    \
  v1 = (c4 & HB) ? o - v1 : v1 + o;        \
  o = xor_lane<HB>(v2);                    \
  v2 = (c4 & HB) ? o - v2 : v2 + o;        \
  o = xor_lane<HB>(v3);                    \
  v3 = (c4 & HB) ? o - v3 : v3 + o;
    TQ_MERGE_STAGE(1)
    TQ_MERGE_STAGE(2)
    TQ_MERGE_STAGE(4)
    TQ_MERGE_STAGE(8)
    TQ_MERGE_STAGE(16)
#undef TQ_MERGE_STAGE
    const float4 sg = reinterpret_cast<const float4*>(p.vrot)[c4];
    v0 *= sg.x * p.rscale_v;
    v1 *= sg.y * p.rscale_v;
    v2 *= sg.z * p.rscale_v;
    v3 *= sg.w * p.rscale_v;
  }
  if (p.q_dtype == TQ_DTYPE_F32) {
    *reinterpret_cast<float4*>(static_cast<float*>(p.out) + o) = make_float4(v0, v1, v2, v3);
  } else {
    const bool f16 = p.q_dtype == TQ_DTYPE_F16;
    const uint32_t a = f16 ? (f32_to_f16_bits(v0) | (static_cast<uint32_t>(f32_to_f16_bits(v1)) << 16))
                           : (f32_to_bf16_bits(v0) | (static_cast<uint32_t>(f32_to_bf16_bits(v1)) << 16));
    const uint32_t c = f16 ? (f32_to_f16_bits(v2) | (static_cast<uint32_t>(f32_to_f16_bits(v3)) << 16))
                           : (f32_to_bf16_bits(v2) | (static_cast<uint32_t>(f32_to_bf16_bits(v3)) << 16));
    *reinterpret_cast<uint2*>(static_cast<uint16_t*>(p.out) + o) = make_uint2(a, c);
  }
}

// --------------------------------------------------------------- launch ---
struct GenPlan {
  int n_splits, chunk, n_rg;
};

GenPlan gen_plan(int B, int Hq, int Hkv, int L, int64_t T) {
  GenPlan gp{};
  const int64_t rows = static_cast<int64_t>(Hq / Hkv) * L;
  gp.n_rg = static_cast<int>((rows + kGenNQ - 1) / kGenNQ);
  const int64_t groups = static_cast<int64_t>(B) * Hkv * gp.n_rg;
  const int64_t target = 2 * static_cast<int64_t>(device_cu_count());
  int64_t ns = groups > 0 ? (target + groups - 1) / groups : 1;
  ns = std::max<int64_t>(1, std::min<int64_t>(ns, (T + 127) / 128));
  int64_t chunk = (T + ns - 1) / ns;
  chunk = std::max<int64_t>(kGenTT, (chunk + kGenTT - 1) / kGenTT * kGenTT);
  if ((T + chunk - 1) / chunk > kGenMaxSplits) {
    chunk = (T + kGenMaxSplits - 1) / kGenMaxSplits;
    chunk = (chunk + kGenTT - 1) / kGenTT * kGenTT;
  }
  chunk = std::min<int64_t>(chunk, int64_t(1) << 30);
  gp.chunk = static_cast<int>(chunk);
  gp.n_splits = static_cast<int>(std::max<int64_t>(1, (T + chunk - 1) / chunk));
  return gp;
}

// The tile kernel's plan: 128-row blocks, splits aiming at one workgroup per
// CU (its LDS holds one), whole 32-token sub-chunks.
GenPlan tile_plan(int B, int Hq, int Hkv, int L, int64_t T) {
  GenPlan gp{};
  const int64_t rows = static_cast<int64_t>(Hq / Hkv) * L;
  gp.n_rg = static_cast<int>((rows + kGenNQ - 1) / kGenNQ);
  const int64_t blocks = static_cast<int64_t>(B) * Hkv * ((rows + kTileRows - 1) / kTileRows);
  const int64_t target = static_cast<int64_t>(device_cu_count());
  int64_t ns = blocks > 0 ? (target + blocks - 1) / blocks : 1;
  ns = std::max<int64_t>(1, std::min<int64_t>(ns, (T + 255) / 256));
  int64_t chunk = (T + ns - 1) / ns;
  chunk = std::max<int64_t>(32, (chunk + 31) / 32 * 32);
  if ((T + chunk - 1) / chunk > kGenMaxSplits) chunk = ((T + kGenMaxSplits - 1) / kGenMaxSplits + 31) / 32 * 32;
  chunk = std::min<int64_t>(chunk, int64_t(1) << 30);
  gp.chunk = static_cast<int>(chunk);
  gp.n_splits = static_cast<int>(std::max<int64_t>(1, (T + chunk - 1) / chunk));
  return gp;
}

int64_t a256(int64_t x) { return (x + 255) / 256 * 256; }
int round32(int d) { return (d + 31) / 32 * 32; }
int pow2_at_least(int d) {
  int r = 32;
  while (r < d) r <<= 1;
  return r;
}

template <int KB, int VB>
int launch_tile(const GenParams& p, hipStream_t st) {
  const int n_blocks = (p.R * p.L + kTileRows - 1) / kTileRows;
  const int64_t wgs = static_cast<int64_t>(p.B) * p.Hkv * n_blocks * p.n_splits;
  if (wgs > INT32_MAX) return fail(TQ_ERR_UNSUPPORTED, "attention: %lld tile workgroups", static_cast<long long>(wgs));
  hipLaunchKernelGGL((gen_tile_kernel<KB, VB>), dim3(static_cast<unsigned>(wgs)), dim3(kTileThreads), 0, st, p,
                     n_blocks);
  return check_launch("gen_tile_kernel");
}

template <int KB>
int launch_tile_vb(const GenParams& p, int vb, hipStream_t st) {
  switch (vb) {
    case 1: return launch_tile<KB, 1>(p, st);
    case 2: return launch_tile<KB, 2>(p, st);
    case 3: return launch_tile<KB, 3>(p, st);
    case 4: return launch_tile<KB, 4>(p, st);
  }
  return fail(TQ_ERR_INVALID_ARGUMENT, "attention: v_bits %d not in 1..4", vb);
}

int launch_tile_partial(const GenParams& p, int kb, int vb, hipStream_t st) {
  switch (kb) {
    case 1: return launch_tile_vb<1>(p, vb, st);
    case 2: return launch_tile_vb<2>(p, vb, st);
    case 3: return launch_tile_vb<3>(p, vb, st);
    case 4: return launch_tile_vb<4>(p, vb, st);
  }
  return fail(TQ_ERR_INVALID_ARGUMENT, "attention: k_bits %d not in 1..4", kb);
}

template <int KIND, int KB, int VB>
int launch_gen(const GenParams& p, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>(p.n_splits), static_cast<unsigned>(p.Hkv * p.n_rg),
                  static_cast<unsigned>(p.B));
  hipLaunchKernelGGL((gen_partial_kernel<KIND, KB, VB>), grid, dim3(kGenThreads), 0, st, p);
  return check_launch("gen_partial_kernel");
}

template <int KIND, int KB>
int launch_gen_vb(const GenParams& p, int vb, hipStream_t st) {
  switch (vb) {
    case 1: return launch_gen<KIND, KB, 1>(p, st);
    case 2: return launch_gen<KIND, KB, 2>(p, st);
    case 3: return launch_gen<KIND, KB, 3>(p, st);
    case 4: return launch_gen<KIND, KB, 4>(p, st);
  }
  return fail(TQ_ERR_INVALID_ARGUMENT, "attention: v_bits %d not in 1..4", vb);
}

int launch_gen_partial(const GenParams& p, int kb, int vb, hipStream_t st) {
  switch (p.key_kind) {
    case kGenPlainF16: return launch_gen<kGenPlainF16, 0, 0>(p, st);
    case kGenPlainBf16: return launch_gen<kGenPlainBf16, 0, 0>(p, st);
    case kGenProd:
      switch (kb) {
        case 0: return launch_gen_vb<kGenProd, 0>(p, vb, st);
        case 1: return launch_gen_vb<kGenProd, 1>(p, vb, st);
        case 2: return launch_gen_vb<kGenProd, 2>(p, vb, st);
        case 3: return launch_gen_vb<kGenProd, 3>(p, vb, st);
      }
      break;
    default:
      switch (kb) {
        case 1: return launch_gen_vb<kGenMse, 1>(p, vb, st);
        case 2: return launch_gen_vb<kGenMse, 2>(p, vb, st);
        case 3: return launch_gen_vb<kGenMse, 3>(p, vb, st);
        case 4: return launch_gen_vb<kGenMse, 4>(p, vb, st);
      }
  }
  return fail(TQ_ERR_INVALID_ARGUMENT, "attention: key bits %d", kb);
}

void launch_qprep_mode(const GenParams& p, int64_t rows, int mode, const float* mat, float* dst,
                       hipStream_t st) {
  const unsigned ycols = mode == 2 ? static_cast<unsigned>((p.DkP + 63) / 64) : 1u;
  const dim3 grid(static_cast<unsigned>((rows + kQpRows - 1) / kQpRows), ycols);
  switch (p.q_dtype) {
    case TQ_DTYPE_F32: hipLaunchKernelGGL(gen_qprep_kernel<TQ_DTYPE_F32>, grid, dim3(kGenThreads), 0, st, p, rows, mode, mat, dst); break;
    case TQ_DTYPE_F16: hipLaunchKernelGGL(gen_qprep_kernel<TQ_DTYPE_F16>, grid, dim3(kGenThreads), 0, st, p, rows, mode, mat, dst); break;
    default: hipLaunchKernelGGL(gen_qprep_kernel<TQ_DTYPE_BF16>, grid, dim3(kGenThreads), 0, st, p, rows, mode, mat, dst); break;
  }
}

bool pow2(int d) { return d > 0 && (d & (d - 1)) == 0; }

}  // namespace

bool tile_rows_path(int kv_kind, int Dk, int Dv, int rows) {
  return kv_kind == TQ_KV_PACKED && Dk == 128 && Dv == 128 && rows >= kTileMinRows;
}

int64_t general_workspace_bytes(int B, int Hq, int Hkv, int L, int Dk, int Dv, int64_t T, bool prod) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || L <= 0 || Dk <= 0 || Dv <= 0 || Hq % Hkv) return 0;
  T = std::max<int64_t>(T, 1);
  GenPlan gp = gen_plan(B, Hq, Hkv, L, T);
  const int64_t rows = static_cast<int64_t>(B) * Hq * L;
  int64_t tile_q = 0;  // the tile kernel's prepared query rows
  if (tile_rows_path(TQ_KV_PACKED, Dk, Dv, (Hq / Hkv) * L)) {
    const GenPlan tp = tile_plan(B, Hq, Hkv, L, T);
    if (tp.n_splits > gp.n_splits) gp = tp;
    tile_q = a256(rows * Dk * 4) + a256(rows * 4);
  }
  const int64_t groups = static_cast<int64_t>(B) * Hkv * gp.n_rg;
  return a256(rows * round32(Dk) * 4) * (prod ? 2 : 1) +
         a256(groups * gp.n_splits * kGenNQ * static_cast<int64_t>(Dv) * 4) +
         a256(groups * gp.n_splits * kGenNQ * 2 * 4) + tile_q;
}

int general_attention(const GenCall& c) {
  const bool plain = c.kv_kind == TQ_KV_PLAIN;
  const bool prod = c.kv_kind == TQ_KV_PROD;
  if (c.B < 0 || c.Hq <= 0 || c.Hkv <= 0 || c.L < 1 || c.Hq % c.Hkv)
    return fail(TQ_ERR_INVALID_ARGUMENT, "attention: bad heads/L (Hq %d, Hkv %d, L %d)", c.Hq, c.Hkv, c.L);
  if (c.Dk < 8 || c.Dk > kGenMaxDim || c.Dv < 8 || c.Dv > kGenMaxDim)
    return fail(TQ_ERR_UNSUPPORTED, "attention: head dims k %d / v %d (8..512 are built)", c.Dk, c.Dv);
  if (c.q_dtype != TQ_DTYPE_F32 && c.q_dtype != TQ_DTYPE_F16 && c.q_dtype != TQ_DTYPE_BF16)
    return fail(TQ_ERR_INVALID_ARGUMENT, "attention: q_dtype %d", c.q_dtype);
  if (c.kv_kind != TQ_KV_PACKED && c.kv_kind != TQ_KV_PLAIN && c.kv_kind != TQ_KV_PROD)
    return fail(TQ_ERR_INVALID_ARGUMENT, "attention: kv_kind %d", c.kv_kind);
  if (c.max_tokens < 0 || c.max_tokens > c.capacity)
    return fail(TQ_ERR_INVALID_ARGUMENT, "attention: max_tokens %lld > capacity %lld",
                (long long)c.max_tokens, (long long)c.capacity);
  if (c.mask_kind < TQ_MASK_NONE || c.mask_kind > TQ_MASK_ADD_BF16)
    return fail(TQ_ERR_INVALID_ARGUMENT, "attention: mask_kind %d", c.mask_kind);
  if (c.mask_kind != TQ_MASK_NONE && (!c.mask || !c.mask_strides))
    return fail(TQ_ERR_INVALID_ARGUMENT, "attention: null mask or mask strides");
  int kb = 0;
  if (plain) {
    if (c.kv_dtype != TQ_DTYPE_F16 && c.kv_dtype != TQ_DTYPE_BF16)
      return fail(TQ_ERR_INVALID_ARGUMENT, "attention: plain kv_dtype %d", c.kv_dtype);
  } else {
    if (c.v_bits < 1 || c.v_bits > 4)
      return fail(TQ_ERR_INVALID_ARGUMENT, "attention: v_bits %d not in 1..4", c.v_bits);
    if (c.norm_dtype != TQ_DTYPE_F32 && c.norm_dtype != TQ_DTYPE_F16)
      return fail(TQ_ERR_INVALID_ARGUMENT, "attention: norm_dtype %d", c.norm_dtype);
    if (c.k_bits < 1 || c.k_bits > 4)
      return fail(TQ_ERR_INVALID_ARGUMENT, "attention: k_bits %d not in 1..4", c.k_bits);
    for (int rk : {c.k_rot_kind, c.v_rot_kind})
      if (rk != TQ_ROT_HADAMARD && rk != TQ_ROT_DENSE)
        return fail(TQ_ERR_INVALID_ARGUMENT, "attention: rot_kind %d", rk);
    if (c.k_rot_kind == TQ_ROT_HADAMARD && !pow2(c.Dk))
      return fail(TQ_ERR_INVALID_ARGUMENT, "attention: Hadamard key rotation needs a power-of-two dim, got %d", c.Dk);
    if (c.v_rot_kind == TQ_ROT_HADAMARD && !pow2(c.Dv))
      return fail(TQ_ERR_INVALID_ARGUMENT, "attention: Hadamard value rotation needs a power-of-two dim, got %d", c.Dv);
    if (!c.v_codebook || !c.v_rot || !c.k_rot)
      return fail(TQ_ERR_INVALID_ARGUMENT, "attention: null codec pointer");
    kb = prod ? c.k_bits - 1 : c.k_bits;
    if (kb > 0 && !c.k_codebook) return fail(TQ_ERR_INVALID_ARGUMENT, "attention: null key codebook");
    if (prod) {
      if (c.k_rot_kind == TQ_ROT_HADAMARD && c.Dk < 32)
        return fail(TQ_ERR_INVALID_ARGUMENT, "attention: Prod keys with the Hadamard rotation need dim >= 32");
      if (!c.projection) return fail(TQ_ERR_INVALID_ARGUMENT, "attention: null projection matrix");
      if (c.max_tokens > 0 && (!c.k_signs || !c.k_rnorms))
        return fail(TQ_ERR_INVALID_ARGUMENT, "attention: null Prod key pointer");
    }
    if (c.max_tokens > 0 && (!c.k_norms || !c.v_norms))
      return fail(TQ_ERR_INVALID_ARGUMENT, "attention: null norms pointer");
  }
  if (c.B == 0) return TQ_OK;
  if (!c.q || !c.out || !c.workspace) return fail(TQ_ERR_INVALID_ARGUMENT, "attention: null pointer");
  if (c.max_tokens > 0 && (!c.v || (!c.k && !(prod && kb == 0))))
    return fail(TQ_ERR_INVALID_ARGUMENT, "attention: null cache pointer");
  const int64_t T = std::max<int64_t>(c.max_tokens, 1);
  const bool tile = c.kv_kind == TQ_KV_PACKED && c.mask_kind == TQ_MASK_NONE &&
                    tile_rows_path(c.kv_kind, c.Dk, c.Dv, (c.Hq / c.Hkv) * c.L) &&
                    static_cast<int64_t>(c.B) * c.Hq * c.L < (int64_t(1) << 30);
  const GenPlan gp = tile ? tile_plan(c.B, c.Hq, c.Hkv, c.L, T) : gen_plan(c.B, c.Hq, c.Hkv, c.L, T);
  if (static_cast<int64_t>(c.Hkv) * gp.n_rg > 65535 || c.B > 65535)
    return fail(TQ_ERR_UNSUPPORTED, "attention: %lld kv head row groups / %d sequences exceed one launch",
                (long long)c.Hkv * gp.n_rg, c.B);
  const int64_t need = general_workspace_bytes(c.B, c.Hq, c.Hkv, c.L, c.Dk, c.Dv, T, prod);
  if (c.workspace_bytes < need)
    return fail(TQ_ERR_WORKSPACE, "attention: workspace %lld < %lld bytes", (long long)c.workspace_bytes,
                (long long)need);
  if ((reinterpret_cast<uintptr_t>(c.workspace) & 255u) != 0)
    return fail(TQ_ERR_INVALID_ARGUMENT, "attention: workspace must be 256-byte aligned");

  GenParams p{};
  p.q = c.q;
  p.q_sb = c.q_sb;
  p.q_sh = c.q_sh;
  p.q_sl = c.q_sl;
  p.q_dtype = c.q_dtype;
  p.scale_q = host_round_to(c.q_dtype, c.scale);
  p.B = c.B;
  p.Hq = c.Hq;
  p.Hkv = c.Hkv;
  p.L = c.L;
  p.R = c.Hq / c.Hkv;
  p.Dk = c.Dk;
  p.Dv = c.Dv;
  p.DkP = round32(c.Dk);
  p.DvP = pow2_at_least(c.Dv);
  p.key_kind = plain ? (c.kv_dtype == TQ_DTYPE_BF16 ? kGenPlainBf16 : kGenPlainF16) : (prod ? kGenProd : kGenMse);
  p.k = c.k;
  p.kn = c.k_norms;
  p.ksg = c.k_signs;
  p.krn = c.k_rnorms;
  p.kpw = plain ? 0 : tq_packed_width(c.Dk, kb);
  p.kcb = c.k_codebook;
  p.k_rot_kind = c.k_rot_kind;
  p.krot = c.k_rot;
  p.proj = c.projection;
  p.v = c.v;
  p.vn = c.v_norms;
  p.vpw = plain ? 0 : tq_packed_width(c.Dv, c.v_bits);
  p.vcb = c.v_codebook;
  p.v_rot_kind = c.v_rot_kind;
  p.vrot = c.v_rot;
  p.norm_dtype = c.norm_dtype;
  p.cap = c.capacity;
  p.T = c.max_tokens;
  p.seq_lens = c.seq_lens;
  p.seq_starts = c.seq_starts;
  p.causal = c.causal ? 1 : 0;
  p.mask = c.mask;
  p.mask_kind = c.mask_kind;
  if (c.mask_kind != TQ_MASK_NONE) {
    p.m_sb = c.mask_strides[0];
    p.m_sg = c.mask_strides[1];
    p.m_sr = c.mask_strides[2];
    p.m_sl = c.mask_strides[3];
    p.m_st = c.mask_strides[4];
  }
  p.n_splits = gp.n_splits;
  p.chunk = gp.chunk;
  p.n_rg = gp.n_rg;
  const int64_t rows = static_cast<int64_t>(c.B) * c.Hq * c.L;
  char* ws = static_cast<char*>(c.workspace);
  p.qrot = reinterpret_cast<float*>(ws);
  ws += a256(rows * p.DkP * 4);
  if (prod) {
    p.qproj = reinterpret_cast<float*>(ws);
    ws += a256(rows * p.DkP * 4);
  }
  const int64_t groups = static_cast<int64_t>(c.B) * c.Hkv * gp.n_rg;
  p.po = reinterpret_cast<float*>(ws);
  ws += a256(groups * gp.n_splits * kGenNQ * static_cast<int64_t>(c.Dv) * 4);
  p.pml = reinterpret_cast<float*>(ws);
  ws += a256(groups * gp.n_splits * kGenNQ * 2 * 4);
  if (tile) {
    p.qhl = reinterpret_cast<uint32_t*>(ws);
    ws += a256(rows * c.Dk * 4);
    p.qsq = reinterpret_cast<float*>(ws);
  }
  p.rscale_k = static_cast<float>(1.0 / __builtin_sqrt(static_cast<double>(c.Dk)));
  p.rscale_v = static_cast<float>(1.0 / __builtin_sqrt(static_cast<double>(c.Dv)));
  p.qjl_scale = static_cast<float>(__builtin_sqrt(3.14159265358979323846 / 2.0) / c.Dk);
  p.out = c.out;

  hipStream_t st = static_cast<hipStream_t>(c.stream);
  // the tile kernel takes its query rows split per row (gen_tile_qprep_kernel,
  // which rotates Hadamard queries itself); its Hadamard-rotated partials go
  // to the element-wise merge, which applies R_V^-1 once per row
  p.po_natural = plain ? 1 : 0;
  p.merge_had = (tile && c.v_rot_kind == TQ_ROT_HADAMARD) ? 1 : 0;
  if (plain)
    launch_qprep_mode(p, rows, 0, nullptr, p.qrot, st);
  else if (tile && c.k_rot_kind == TQ_ROT_HADAMARD)
    ;
  else if (c.k_rot_kind == TQ_ROT_HADAMARD && kb > 0)
    launch_qprep_mode(p, rows, 1, c.k_rot, p.qrot, st);
  else if (c.k_rot_kind == TQ_ROT_DENSE)
    launch_qprep_mode(p, rows, 2, c.k_rot, p.qrot, st);
  if (prod) launch_qprep_mode(p, rows, 2, c.projection, p.qproj, st);
  int rc = check_launch("gen_qprep_kernel");
  if (rc) return rc;
  if (tile) {
    const int64_t wgs = (rows + kTileQpRows * (kTileQpThreads / 64) - 1) / (kTileQpRows * (kTileQpThreads / 64));
    hipLaunchKernelGGL(gen_tile_qprep_kernel, dim3(static_cast<unsigned>(wgs)), dim3(kTileQpThreads), 0, st, p,
                       static_cast<int>(rows));
    rc = check_launch("gen_tile_qprep_kernel");
    if (rc) return rc;
  }
  rc = tile ? launch_tile_partial(p, kb, c.v_bits, st) : launch_gen_partial(p, kb, plain ? 0 : c.v_bits, st);
  if (rc) return rc;
  // the flat merge takes 4 value columns per thread: plain values need Dv % 4 == 0
  if ((plain && c.Dv % 4 == 0) || p.merge_had) {
    const int64_t items = static_cast<int64_t>(c.B) * c.Hkv * (c.Hq / c.Hkv) * c.L * (c.Dv / 4);
    const int64_t pair_items = static_cast<int64_t>(c.Hq / c.Hkv) * c.L * (c.Dv / 4);
    // after the tile kernel, each pair's merge blocks run on the XCD whose
    // L2 took that pair's partials
    p.merge_bpp = (tile && (static_cast<int64_t>(c.B) * c.Hkv) % 8 == 0 && pair_items % 256 == 0)
                      ? static_cast<int>(pair_items / 256)
                      : 0;
    const dim3 fgrid(static_cast<unsigned>((items + 255) / 256));
    if (items < (int64_t(1) << 31) - 256)
      hipLaunchKernelGGL(gen_merge_flat_kernel<int>, fgrid, dim3(256), 0, st, p, static_cast<int>(items));
    else
      hipLaunchKernelGGL(gen_merge_flat_kernel<int64_t>, fgrid, dim3(256), 0, st, p, items);
    return check_launch("gen_merge_flat_kernel");
  }
  const unsigned zc = (!plain && c.v_rot_kind == TQ_ROT_DENSE) ? static_cast<unsigned>((c.Dv + 63) / 64) : 1u;
  const dim3 mgrid(static_cast<unsigned>(c.Hkv * gp.n_rg), static_cast<unsigned>(c.B), zc);
  hipLaunchKernelGGL(gen_merge_kernel, mgrid, dim3(kGenThreads), 0, st, p);
  return check_launch("gen_merge_kernel");
}

}  // namespace tq

using namespace tq;

extern "C" int64_t tq_attention_general_workspace_size(int B, int Hq, int Hkv, int L, int k_dim,
                                                       int v_dim, int64_t max_tokens) {
  if (max_tokens < 0) return 0;
  return general_workspace_bytes(B, Hq, Hkv, L, k_dim, v_dim, max_tokens, true);
}

extern "C" int tq_attention_general(
    const void* q, int q_dtype, int B, int Hq, int Hkv, int L, int k_dim, int v_dim,
    int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_l, float scale, int kv_kind,
    int kv_dtype, const void* k, const void* k_norms, const void* k_signs,
    const void* k_residual_norms, int k_bits, const float* k_codebook, int k_rot_kind,
    const float* k_rot, const float* projection, const void* v, const void* v_norms, int v_bits,
    const float* v_codebook, int v_rot_kind, const float* v_rot, int norm_dtype, int64_t capacity,
    int64_t max_tokens, const int32_t* seq_starts, const int32_t* seq_lens, int causal,
    const void* mask, int mask_kind, const int64_t* mask_strides, void* out, void* workspace,
    int64_t workspace_bytes, void* stream) {
  GenCall c{};
  c.q = q;
  c.q_dtype = q_dtype;
  c.B = B;
  c.Hq = Hq;
  c.Hkv = Hkv;
  c.L = L;
  c.Dk = k_dim;
  c.Dv = v_dim;
  c.q_sb = q_stride_b;
  c.q_sh = q_stride_h;
  c.q_sl = q_stride_l;
  c.scale = scale;
  c.kv_kind = kv_kind;
  c.kv_dtype = kv_dtype;
  c.k = k;
  c.k_norms = k_norms;
  c.k_signs = k_signs;
  c.k_rnorms = k_residual_norms;
  c.k_bits = k_bits;
  c.k_codebook = k_codebook;
  c.k_rot_kind = k_rot_kind;
  c.k_rot = k_rot;
  c.projection = projection;
  c.v = v;
  c.v_norms = v_norms;
  c.v_bits = v_bits;
  c.v_codebook = v_codebook;
  c.v_rot_kind = v_rot_kind;
  c.v_rot = v_rot;
  c.norm_dtype = norm_dtype;
  c.capacity = capacity;
  c.max_tokens = max_tokens;
  c.seq_starts = seq_starts;
  c.seq_lens = seq_lens;
  c.causal = causal;
  c.mask = mask;
  c.mask_kind = mask_kind;
  c.mask_strides = mask_strides;
  c.out = out;
  c.workspace = workspace;
  c.workspace_bytes = workspace_bytes;
  c.stream = stream;
  return general_attention(c);
}
