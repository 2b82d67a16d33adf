// Decode / verify attention over unquantized fp16 / bf16 K/V (the
// mixed-precision layers) on gfx950's matrix cores.
//
// Same work split, online softmax, wave combine and split partials as the
// packed kernel (tq_attn_mfma.h); the operands come straight from the cache:
//   scores  S[row][tok] = q_s[row] . k[tok]      (16 x 16 tiles, k = coordinates)
//     A = query rows as hi + lo parts in the cache's 16-bit type (f16:
//         q_s = hi + lo to ~2^-22 at a power-of-two scale; bf16: hi + lo to
//         ~2^-16), lane (row n, g) holds coordinates 32s + 8g .. +7 for k-step s,
//     B = lane (token n, g) holds the same coordinates of token n: one
//         16-byte load from its row per k-step (K is used as stored).
//   values  O[row][d] = sum_tok w[row][tok] v[tok][d]  (k = tokens)
//     The contraction runs over tokens while a V row is contiguous over
//     coordinates, so each wave stages its 32-token V tile in LDS and reads
//     the B operands transposed with ds_read_b64_tr_b16: in every 16-lane
//     group, lane i receives element i % 4 of the 8-byte piece addressed by
//     lane 4j + i / 4, for j = 0..3.  Lane (coordinate n, g) of coordinate
//     tile c therefore addresses token 8g + 4h + n / 4, coordinates
//     16c + 4 (n % 4) .. +3 (h = 0, 1) and receives V[8g + 4h + j][16c + n].
//     The tile is row-major with its 8-byte pieces XOR-swizzled per token,
//     so the eight rows one half-wave reads land on distinct banks.
//     A = softmax weights (f16, or bf16 hi + lo for bf16 values), exactly as
//     in the packed kernel.
// Semantics: scaled_dot_product_attention on the fp16 layers, base.py:218-226,
// with the same f32 softmax as the TurboQuant layers (turboquant_cache.py:5110-5203).
#pragma once

#include "tq_attn_mfma.h"

namespace tq {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));

template <int KVDT>
__device__ __forceinline__ f32x4_t mfma_kv(u32x4_t a, u32x4_t b, f32x4_t c) {
  if constexpr (KVDT == TQ_DTYPE_BF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                    __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  else
    return mfma_f16(a, b, c);
}

// hi + lo split of x in the cache's 16-bit type.
template <int KVDT>
__device__ __forceinline__ void split_kv(float x, uint32_t& hi, uint32_t& lo) {
  if constexpr (KVDT == TQ_DTYPE_BF16) {
    hi = f32_to_bf16_bits(x);
    lo = f32_to_bf16_bits(x - bf16_bits_to_f32(static_cast<uint16_t>(hi)));
  } else {
    split_f16(x, hi, lo);
  }
}

template <int D, int KVDT, int NQ>
struct PlainShape {
  static constexpr int NW = D >= 256 ? 4 : 8;
  static constexpr int NT = NW * kWave;
  static constexpr int SUB = 32;
  static constexpr int P = D >= 256 ? 1 : 2;  // sub-chunks in flight per wave
  static constexpr int KS = D / 32;           // score k-steps
  static constexpr int CPL = D / 16;          // value coordinate tiles
  static constexpr int ROWB = D * 2;          // bytes per token row
  static constexpr int LPR = D / 8;           // lanes per token row in a 16-byte load
  static constexpr int TPI = kWave / LPR;     // tokens per V load instruction
  static constexpr int VLD = SUB / TPI;       // V loads per lane and sub-chunk
  static constexpr bool BF = KVDT == TQ_DTYPE_BF16;
  static constexpr int WPARTS = BF ? 2 : 1;   // weight parts (bf16: hi + lo)
  static constexpr int QSTRIDE = D + 4;
  static constexpr int VT_BYTES = SUB * ROWB;  // one wave's V tile
  static constexpr int V_OFF = 0;
  static constexpr int Q_OFF = V_OFF + NW * VT_BYTES;      // [NQ][QSTRIDE] f32 scaled queries
  static constexpr int QS_OFF = Q_OFF + NQ * QSTRIDE * 4;  // [NQ] f32 max |q_s|
  static constexpr int W_OFF = QS_OFF + 64;                // [NW][WPARTS][16][32] weights
  static constexpr int LOOP_BYTES = W_OFF + NW * WPARTS * 16 * SUB * 2;
  // after the token loop (a barrier separates the phases) the buffers restart at 0
  static constexpr int CO_OFF = 0;
  static constexpr int CM_OFF = CO_OFF + NW * NQ * D * 4;
  static constexpr int CL_OFF = CM_OFF + NW * NQ * 4;
  static constexpr int O_OFF = CL_OFF + NW * NQ * 4;
  static constexpr int ML_OFF = O_OFF + NQ * D * 4;
  static constexpr int AUX_OFF = ML_OFF + (NQ * 8 + 15) / 16 * 16;
  static constexpr int POST_BYTES = AUX_OFF + (NQ + D) * 4;
  static constexpr int BYTES = LOOP_BYTES > POST_BYTES ? LOOP_BYTES : POST_BYTES;
  static_assert(BYTES <= 160 * 1024, "LDS per workgroup");
  static_assert(SUB % TPI == 0, "V loads");
};

// XOR applied to the 8-byte piece index of token row t of a V tile: a
// multiple of 4 below the row's piece count D / 4, so the two pieces of a
// 16-byte store stay adjacent, the four pieces one lane group reads stay
// contiguous, and the pieces stay inside their row.  At d = 128 the eight
// rows a half-wave reads (tokens 8g + 4h + j, g = 0, 1) get eight distinct
// 32-byte windows of the banks.
template <int D>
__device__ __forceinline__ int v_swizzle(int t) {
  return (4 * ((t & 3) | ((t >> 1) & 4))) & (D / 4 - 1);
}

template <int D, int KVDT, int NQ>
__global__ __launch_bounds__(D >= 256 ? 256 : 512, 1) void attn_plain_kernel(AttnParams p) {
  using S = PlainShape<D, KVDT, NQ>;
  static_assert(S::NT == (D >= 256 ? 256 : 512), "launch bounds");
  constexpr int NW = S::NW;
  constexpr int NT = S::NT;
  constexpr int SUB = S::SUB;
  constexpr int P = S::P;
  constexpr int KS = S::KS;
  constexpr int CPL = S::CPL;
  constexpr int ROWB = S::ROWB;
  constexpr int LPR = S::LPR;
  constexpr int TPI = S::TPI;
  constexpr int VLD = S::VLD;
  constexpr bool BF = S::BF;
  constexpr int RPW = (NQ + NW - 1) / NW;
  constexpr int QPL = D / kWave;

  __shared__ __align__(16) unsigned char lds[S::BYTES];
  float* s_q = reinterpret_cast<float*>(lds + S::Q_OFF);
  float* s_qs = reinterpret_cast<float*>(lds + S::QS_OFF);
  uint16_t* s_w = reinterpret_cast<uint16_t*>(lds + S::W_OFF);
  float* s_co = reinterpret_cast<float*>(lds + S::CO_OFF);
  float* s_cm = reinterpret_cast<float*>(lds + S::CM_OFF);
  float* s_cl = reinterpret_cast<float*>(lds + S::CL_OFF);
  float* s_o = reinterpret_cast<float*>(lds + S::O_OFF);
  float* s_ml = reinterpret_cast<float*>(lds + S::ML_OFF);
  float* s_aux = reinterpret_cast<float*>(lds + S::AUX_OFF);

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int n = lane & 15;
  const int g = lane >> 4;
  const int split = blockIdx.x;
  const int gk = blockIdx.y / p.n_rg;
  const int rg = blockIdx.y % p.n_rg;
  const int b = blockIdx.z;
  RowSet rs;
  rs.init(p, b, gk, rg, NQ);

  const SeqWindow win = seq_window(p, b);
  const int64_t Tb = win.len;  // token positions below are relative to win.start
  const int64_t t_begin64 = static_cast<int64_t>(split) * p.chunk;
  if (t_begin64 >= Tb) {
    if (Tb <= 0 && split == 0)
      for (int idx = tid; idx < NQ * D; idx += NT)
        if (rs.valid(idx / D)) store_out(p.out, p.q_dtype, rs.qoff(idx / D) * D + idx % D, 0.f);
    return;  // the whole workgroup leaves together
  }
  const int t_begin = static_cast<int>(t_begin64);
  const int t_end = static_cast<int>(Tb < t_begin64 + p.chunk ? Tb : t_begin64 + p.chunk);
  const int nvalid = static_cast<int>((Tb + p.chunk - 1) / p.chunk);
  // buffer resources over tokens [0, t_end) of this (sequence, kv head) row:
  // rows at or past t_end read as zeros
  const int64_t kvrow0 = (static_cast<int64_t>(b) * p.Hkv + gk) * p.cap + win.start;
  const uint32_t tn = static_cast<uint32_t>(t_end);
  const auto krs = buffer_rsrc(static_cast<const char*>(p.k) + kvrow0 * ROWB, tn * ROWB);
  const auto vrs = buffer_rsrc(static_cast<const char*>(p.v) + kvrow0 * ROWB, tn * ROWB);
  const uint32_t k_lane = n * ROWB + g * 16;
  const uint32_t v_lane = (lane / LPR) * ROWB + (lane % LPR) * 16;

  const int n_tok = t_end - t_begin;
  const int n_my = n_tok > wave * SUB ? (n_tok - wave * SUB + NW * SUB - 1) / (NW * SUB) : 0;
  auto sub_start = [&](int i) -> int { return t_begin + (i * NW + wave) * SUB; };

  struct Buf {
    u32x4_t k[2][KS];  // token n of the two 16-token tiles, coordinates 32s + 8g ..
    u32x4_t v[VLD];    // V rows for the LDS tile
  };
  auto load_sub = [&](Buf& bf, int s0) {
    const uint32_t t0 = static_cast<uint32_t>(s0);
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int s = 0; s < KS; ++s)
        bf.k[tt][s] = __builtin_bit_cast(
            u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(krs, (t0 + 16 * tt) * ROWB + k_lane + s * 64, 0, 0));
#pragma unroll
    for (int i = 0; i < VLD; ++i)
      bf.v[i] = __builtin_bit_cast(
          u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(vrs, (t0 + i * TPI) * ROWB + v_lane, 0, 0));
  };

  // ---- query rows (raw bits first, so no load is waited for here)
  uint32_t qraw[RPW][QPL];
  const bool q32 = p.q_dtype == TQ_DTYPE_F32;
#pragma unroll
  for (int rr = 0; rr < RPW; ++rr) {
    const int r = wave + rr * NW;
    const bool ok = r < NQ && rs.valid(r);
    const int64_t qb = !ok ? 0
                           : b * p.q_sb + static_cast<int64_t>(rs.head(r)) * p.q_sh +
                                 static_cast<int64_t>(rs.lpos(r)) * p.q_sl;
#pragma unroll
    for (int e = 0; e < QPL; ++e) {
      const int64_t i = qb + lane + e * kWave;
      if (!ok)
        qraw[rr][e] = 0u;
      else if (q32)
        qraw[rr][e] = static_cast<const uint32_t*>(p.q)[i];
      else
        qraw[rr][e] = static_cast<const uint16_t*>(p.q)[i];
    }
  }
  Buf buf[P];
  load_sub(buf[0], sub_start(0));

  // ---- prologue: q_s = round_qdtype(q * scale_q) into LDS, row maxima
#pragma unroll
  for (int rr = 0; rr < RPW; ++rr) {
    const int r = wave + rr * NW;
    if (r >= NQ) break;
    float* y = s_q + r * S::QSTRIDE;
    float m = 0.f;
#pragma unroll
    for (int e = 0; e < QPL; ++e) {
      const uint32_t raw = qraw[rr][e];
      const float qv = q32 ? __builtin_bit_cast(float, raw)
                           : (p.q_dtype == TQ_DTYPE_F16 ? f16_bits_to_f32(static_cast<uint16_t>(raw))
                                                        : bf16_bits_to_f32(static_cast<uint16_t>(raw)));
      const float v = round_q(p.q_dtype, qv * p.scale_q);
      y[lane + e * kWave] = v;
      m = fmaxf(m, fabsf(v));
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, kWave));
    if (lane == 0) s_qs[r] = m;
  }
  lds_barrier();
  // query operands: hi + lo in the cache type at one power-of-two scale
  float qmax = 0.f;
#pragma unroll
  for (int r = 0; r < NQ; ++r) qmax = fmaxf(qmax, s_qs[r]);
  const float sq = f16_split_scale(qmax);
  u32x4_t qh[KS], ql[KS];
  {
    const float qsl = n < NQ ? sq : 0.f;  // rows n >= NQ: zeros, no branches
    const float* y = s_q + (n < NQ ? n : 0) * S::QSTRIDE + g * 8;
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint32_t h0, l0, h1, l1;
        split_kv<KVDT>(y[32 * s + 2 * j] * qsl, h0, l0);
        split_kv<KVDT>(y[32 * s + 2 * j + 1] * qsl, h1, l1);
        qh[s][j] = h0 | (h1 << 16);
        ql[s][j] = l0 | (l1 << 16);
      }
  }
  const float qk_inv = 1.4426950408889634f / sq;  // scores in log2 units
  int lim[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 4 * g + i;
    const bool ok = r < NQ && rs.valid(r);
    lim[i] = (p.causal && ok) ? static_cast<int>(Tb - p.L + rs.lpos(r)) : INT32_MAX;
  }
  int lim_min = INT32_MAX;
#pragma unroll
  for (int i = 0; i < 4; ++i) lim_min = min(lim_min, lim[i]);
  for (int off = 16; off < 64; off <<= 1) lim_min = min(lim_min, __shfl_xor(lim_min, off, kWave));
#pragma unroll
  for (int s = 1; s < P; ++s) load_sub(buf[s], sub_start(s));

  // ---- streaming
  float m_run[4], l_run[4];
  f32x4_t O[CPL];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    m_run[i] = -INFINITY;
    l_run[i] = 0.f;
  }
#pragma unroll
  for (int c = 0; c < CPL; ++c) O[c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  uint16_t* w_mine = s_w + wave * S::WPARTS * 16 * SUB;
  unsigned char* vt = lds + S::V_OFF + wave * S::VT_BYTES;
  // V tile addresses: store i of this lane, and the transposed reads of
  // coordinate tile c, half h (bytes inside the wave's tile)
  uint32_t v_st[VLD];
#pragma unroll
  for (int i = 0; i < VLD; ++i) {
    const int t = i * TPI + lane / LPR;
    v_st[i] = t * ROWB + ((2 * (lane % LPR)) ^ v_swizzle<D>(t)) * 8;
  }
  // transposed reads: piece (4c + n % 4) ^ swizzle of token 8g + 4h + n / 4,
  // i.e. byte v_tr[h] + 32 (c ^ v_xq[h]) for coordinate tile c
  uint32_t v_tr[2], v_xq[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int t = 8 * g + 4 * h + (n >> 2);
    v_tr[h] = t * ROWB + (n & 3) * 8;
    v_xq[h] = static_cast<uint32_t>(v_swizzle<D>(t) >> 2);
  }
  typedef __attribute__((address_space(3))) unsigned char lds_u8;
  typedef __attribute__((address_space(3))) s16x4_t lds_s16x4;
  lds_u8* vt3 = (lds_u8*)vt;

  auto scores = [&](const Buf& bf, f32x4_t (&Sc)[2]) {
    f32x4_t Sa[2], Sb[2];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) Sa[tt] = Sb[tt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        Sa[tt] = mfma_kv<KVDT>(qh[s], bf.k[tt][s], Sa[tt]);
        Sb[tt] = mfma_kv<KVDT>(ql[s], bf.k[tt][s], Sb[tt]);
      }
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) Sc[tt] = Sa[tt] + Sb[tt];
  };
  auto finish = [&](const Buf& bf, const f32x4_t (&Sc)[2], int s0) {
    // stage this sub-chunk's V tile (after the previous tile's reads)
    wave_sync();
#pragma unroll
    for (int i = 0; i < VLD; ++i) *reinterpret_cast<u32x4_t*>(vt + v_st[i]) = bf.v[i];
    float sv[2][4];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int i = 0; i < 4; ++i) sv[tt][i] = Sc[tt][i] * qk_inv;
    if (s0 + SUB > t_end || s0 + SUB - 1 > lim_min) {  // wave-uniform
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        const int t = s0 + 16 * tt + n;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (t > lim[i]) sv[tt][i] = -FLT_MAX;
          if (t >= t_end) sv[tt][i] = -INFINITY;
        }
      }
    }
    // online softmax with the lazy reference max of the packed kernel
    constexpr float kLazy = 8.f;
    float cmx[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) cmx[i] = fmaxf(sv[0][i], sv[1][i]);
    row16_max4(cmx);
    bool move = false;
#pragma unroll
    for (int i = 0; i < 4; ++i) move |= cmx[i] > m_run[i] + kLazy;
    if (__any(move ? 1 : 0)) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float mn = cmx[i] > m_run[i] + kLazy ? fmaxf(m_run[i], cmx[i]) : m_run[i];
        const float alpha = __builtin_amdgcn_exp2f(m_run[i] - mn);
        l_run[i] *= alpha;
        m_run[i] = mn;
#pragma unroll
        for (int c = 0; c < CPL; ++c) O[c][i] *= alpha;
      }
    }
    float pw[2][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      pw[0][i] = __builtin_amdgcn_exp2f(sv[0][i] - m_run[i]);
      pw[1][i] = __builtin_amdgcn_exp2f(sv[1][i] - m_run[i]);
      l_run[i] += pw[0][i] + pw[1][i];
    }
    // weights to LDS: [part][row][token]
    if (4 * g < NQ) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
          const int at = (4 * g + i) * SUB + 16 * tt + n;
          if constexpr (BF) {
            uint32_t h, l;
            split_kv<KVDT>(pw[tt][i], h, l);
            w_mine[at] = static_cast<uint16_t>(h);
            w_mine[16 * SUB + at] = static_cast<uint16_t>(l);
          } else {
            w_mine[at] = static_cast<uint16_t>(f16_bits(pw[tt][i]));
          }
        }
    }
    wave_sync();
    const u32x4_t A = *reinterpret_cast<const u32x4_t*>(w_mine + n * SUB + 8 * g);
    u32x4_t A2 = A;
    if constexpr (BF) A2 = *reinterpret_cast<const u32x4_t*>(w_mine + 16 * SUB + n * SUB + 8 * g);
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const s16x4_t v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (lds_s16x4*)(vt3 + v_tr[0] + 32 * (static_cast<uint32_t>(c) ^ v_xq[0])));
      const s16x4_t v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (lds_s16x4*)(vt3 + v_tr[1] + 32 * (static_cast<uint32_t>(c) ^ v_xq[1])));
      const uint2 u0 = __builtin_bit_cast(uint2, v0);
      const uint2 u1 = __builtin_bit_cast(uint2, v1);
      const u32x4_t B = {u0.x, u0.y, u1.x, u1.y};
      O[c] = mfma_kv<KVDT>(A, B, O[c]);
      if constexpr (BF) O[c] = mfma_kv<KVDT>(A2, B, O[c]);
    }
  };

  f32x4_t Sc[2];
  if (n_my > 0) scores(buf[0], Sc);
  for (int base = 0; base < n_my; base += P) {
#pragma unroll
    for (int s = 0; s < P; ++s) {
      const int i = base + s;
      if (i < n_my) {
        finish(buf[s], Sc, sub_start(i));
        if (P == 1) load_sub(buf[s], sub_start(i + 1));
        if (i + 1 < n_my) scores(buf[(s + 1) % P], Sc);
      }
      if (P > 1) load_sub(buf[s], sub_start(i + P));
    }
  }

  // ---- combine the waves (the loop's LDS buffers are dead after the barrier)
  lds_barrier();
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float l = row16_sum(l_run[i]);
    const int r = 4 * g + i;
    if (r < NQ) {
      if (n == 0) {
        s_cm[wave * NQ + r] = m_run[i];
        s_cl[wave * NQ + r] = l;
      }
      float* dst = s_co + (wave * NQ + r) * D;
#pragma unroll
      for (int c = 0; c < CPL; ++c) dst[16 * c + n] = O[c][i];
    }
  }
  lds_barrier();
  for (int idx = tid; idx < NQ * D; idx += NT) {
    const int r = idx / D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, s_cm[w * NQ + r]);
    float a = 0.f, lt = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float wm = s_cm[w * NQ + r];
      if (wm == -INFINITY) continue;
      const float f = __builtin_amdgcn_exp2f(wm - M);
      a = fmaf(s_co[(w * NQ) * D + idx], f, a);
      lt = fmaf(s_cl[w * NQ + r], f, lt);
    }
    s_o[idx] = a;
    if (idx % D == 0) {
      s_ml[2 * r] = M * 0.6931471805599453f;  // the merge works in natural-log units
      s_ml[2 * r + 1] = lt;
    }
  }
  lds_barrier();
  if (nvalid == 1) {  // the only split: finish here
    if (tid < NQ) s_aux[tid] = s_ml[2 * tid + 1];
    lds_barrier();
    finalize_rows<D, NQ, NT>(p, rs, s_o, s_aux, s_aux + NQ, nullptr, true, false);
    return;
  }
  const int64_t grp = (static_cast<int64_t>(b) * p.Hkv + gk) * p.n_rg + rg;
  float4* po4 = reinterpret_cast<float4*>(p.po + (grp * p.n_splits + split) * static_cast<int64_t>(NQ) * D);
  for (int idx = tid; idx < NQ * D / 4; idx += NT) po4[idx] = reinterpret_cast<const float4*>(s_o)[idx];
  if (tid < 2 * NQ) p.pml[(grp * p.n_splits + split) * static_cast<int64_t>(NQ) * 2 + tid] = s_ml[tid];
}

template <int D, int KVDT>
int launch_plain(const AttnParams& p, hipStream_t st) {
  const dim3 grid(p.n_splits, p.Hkv * p.n_rg, p.B);
  if (p.nq == 4) {
    hipLaunchKernelGGL((attn_plain_kernel<D, KVDT, 4>), grid, dim3(PlainShape<D, KVDT, 4>::NT), 0, st, p);
  } else if (p.nq == 16) {
    if constexpr (D <= 128) {
      hipLaunchKernelGGL((attn_plain_kernel<D, KVDT, 16>), grid, dim3(PlainShape<D, KVDT, 16>::NT), 0, st, p);
    } else {
      return fail(TQ_ERR_INVALID_ARGUMENT, "attention: 16-row groups need dim <= 128");
    }
  } else {
    return fail(TQ_ERR_INVALID_ARGUMENT, "attention: rows per group %d", p.nq);
  }
  return check_launch("attn_plain_kernel");
}

}  // namespace tq
