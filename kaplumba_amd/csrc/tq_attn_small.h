// TurboQuant decode / verify attention for small row groups (at most 4 query
// rows per kv head: GQA decode with R <= 4, or verify with R * L <= 4) and
// head dims 64 / 128, straight from packed indices.
//
// Workgroup: 8 wave64s own tokens [t_begin, t_end) of one (sequence, kv head)
// and all (<= 4) query rows of its GQA group.  Tokens are cut into 32-token
// sub-chunks; sub-chunk i belongs to wave i % 8, and each wave keeps the
// global loads of its next P sub-chunks in flight.
//
// Lane roles (l = lane, n = l % 16, g = l / 16):
//   scores  S^T[tok][col] = sum_d k[tok][d] * q_col[d]    (16 x 16 tile, 32 tokens)
//     A = keys: lane (m, g) holds token 16 (g >> 1) + m, coordinate half
//         g & 1 (D/2 coordinates: a contiguous bit span of its packed row),
//         eight coordinates per MFMA, hi parts in one MFMA and lo parts in
//         the next (f16 hi + lo carry ~22 significant bits),
//     B = queries: column n = 8p + 4j + r is piece p (hi / lo f16 split) of
//         query row r for token subset j; the k slots of lane groups that
//         hold the other subset's tokens are zero.  So every output element
//         is useful: lane (g', n) register i holds piece p of the score of
//         token 16j + 4g' + i against row r, and one DPP row rotation by 8
//         adds the two pieces (f32 accuracy: (q_hi + q_lo)(k_hi + k_lo)).
//   softmax per lane: 4 tokens of one row (both pieces' lanes hold copies).
//   values  O[row][d] = sum_tok w[row][tok] * v[tok][d]      (16 x 16 tiles)
//     A = weights: lane (row r, g) holds tokens 4g .. 4g+3 and 16+4g .. 16+4g+3
//         as f16: its own four scores' weights plus those of lane n + 4
//         (token subset 1), fetched with one DPP rotation; no LDS transpose,
//     B = values: lane (coordinate n of tile c, g) holds the same 8 tokens'
//         codebook values as (hi pair, lo pair) of two tokens per 8-byte
//         table read (the table is keyed by the two tokens' fields), against
//         weights (w_a, w_b, w_a, w_b): four tokens per MFMA and lane group.
//     Output: lane (g = 0, n), register i = row i, coordinate (D/16) n + c.
// Codebook lookups go through pair tables in LDS (keys: hi and lo f16 halves
// in two tables sharing one key address; values: one 8-byte entry),
// replicated per lane so that the lanes of one read hit distinct banks.
//
// Softmax: base 2 with log2(e) and the hi/lo scales folded into one factor;
// the reference maximum moves lazily (only when a score exceeds it by 2^7),
// and weights p * ||v|| * 2^-E carry a per-wave value-norm exponent E that
// keeps them inside f16 range, so the common sub-chunk takes no reductions.
//
// Splits: a problem with one split is finished here; otherwise every
// workgroup writes its (o, m, l) partial (o already through R_V^-1 for the
// Hadamard rotation, m in natural-log units) in the layout attn_merge_kernel
// reads, and that kernel merges them on the same stream.  (A last-arriver
// merge inside this kernel costs more: its store -> wait -> count -> load
// chain is four serial memory round trips, against one launch gap.)
// Semantics: quantized_attention, turboquant_cache.py:5110-5203.
#pragma once

#include "tq_attn_mfma.h"

namespace tq {

template <int D, int KB, int VB, bool PROD = false>
struct SmallShape {
  static constexpr int NW = 8;
  static constexpr int NT = NW * kWave;
  static constexpr int SUB = 32;  // tokens per sub-chunk
#ifndef TQ_SMALL_PREFETCH
#define TQ_SMALL_PREFETCH 2
#endif
  static constexpr int P = TQ_SMALL_PREFETCH;  // sub-chunks in flight per wave
  // the next sub-chunk's scores are formed while this one's buffer is still
  // being consumed, so at least two buffers are needed
  static_assert(P >= 2, "prefetch depth");
  static constexpr int NQ = 4;    // query rows
  // keys: a lane holds half a token row
  static constexpr int HALF = D / 2;
  static constexpr int KW = HALF * KB / 32;  // words per lane
  static constexpr int PWK = D * KB / 32;
  static constexpr int NKI = D / 16;         // MFMAs per key piece (8 coordinates each)
  static constexpr int KKEYS = 1 << (2 * KB);
  static constexpr int REPK = KKEYS <= 64 ? 64 : 16;
  static constexpr int LOGSK = REPK == 64 ? 8 : 6;  // log2(REPK * 4)
  // values: a lane holds CPL consecutive coordinates of 8 tokens
  static constexpr int CPL = D / 16;
  static constexpr int PWV = D * VB / 32;
  static constexpr int SEGBITS = CPL * VB;  // <= 32 for D <= 128
  static constexpr int VRAW = (VB == 3) ? 2 : 1;  // a 3-bit segment can cross a word
  static constexpr int VKEYS = 1 << (2 * VB);
  static constexpr int REPV = VKEYS <= 64 ? 64 : 16;
  static constexpr int LOGSV = REPV == 64 ? 9 : 7;  // log2(REPV * 8): (hi pair, lo pair) entries
  // Prod-coded keys (PROD): a second query set (q_proj) against one-bit QJL
  // signs, looked up in a table of (+-1, +-1) f16 pairs
  static constexpr int NQS = PROD ? 2 : 1;      // query sets
  static constexpr int SW = PROD ? D / 64 : 1;  // sign words per lane (half a row)
  static constexpr int STAB = PROD ? 4 * 64 * 4 : 0;
  // LDS (bytes): [sign table][K hi table][K lo table][V (hi, lo) table][q staging][zeros][rows][row max]
  static constexpr int KTAB = KKEYS * REPK * 4;
  static constexpr int VTAB = VKEYS * REPV * 8;
  static constexpr int SGN_OFF = 0;
  static constexpr int LUTK_OFF = STAB;
  static constexpr int LUTV_OFF = LUTK_OFF + 2 * KTAB;
  static constexpr int QST_OFF = LUTV_OFF + VTAB;  // [set][p][r][h][i] 8 x f16 = 16 B
  static constexpr int QST_BYTES = NQS * 2 * NQ * 2 * NKI * 16;
  static constexpr int ZBYTES = PROD ? NKI * 16 : 16;
  static constexpr int ZERO_OFF = QST_OFF + QST_BYTES;        // ZBYTES zero bytes
  static constexpr int QY_OFF = ZERO_OFF + ZBYTES;            // [set][NQ][D] f32 rotated queries
  static constexpr int QMAX_OFF = QY_OFF + NQS * NQ * D * 4;  // [set][NQ] f32
  static constexpr int LOOP_BYTES = QMAX_OFF + NQS * 16;
  // epilogue (after a barrier the loop's buffers are dead)
  static constexpr int WO_OFF = 0;                       // [NW][NQ][D] f32
  static constexpr int WM_OFF = WO_OFF + NW * NQ * D * 4;  // [NW][NQ]
  static constexpr int WL_OFF = WM_OFF + NW * NQ * 4;
  static constexpr int WE_OFF = WL_OFF + NW * NQ * 4;      // [NW][NQ] 2^E of the wave
  static constexpr int WF_OFF = WE_OFF + NW * NQ * 4;      // [NW][NQ] combine factors
  static constexpr int FO_OFF = WF_OFF + NW * NQ * 4;      // [NQ][D] final rows
  static constexpr int FL_OFF = FO_OFF + NQ * D * 4;       // [NQ] l, [NQ] m
  static_assert(FO_OFF % 16 == 0, "final rows are read as float4");
  static constexpr int FLAG_OFF = FL_OFF + 2 * NQ * 4;
  static constexpr int POST_BYTES = FLAG_OFF + 16;
  static constexpr int BYTES = LOOP_BYTES > POST_BYTES ? LOOP_BYTES : POST_BYTES;
  static_assert(D == 64 || D == 128, "small row-group kernel: head dim 64 or 128");
  static_assert(KW * 32 == HALF * KB, "key half rows are whole words");
  static_assert(SEGBITS <= 32, "value segment in one word");
  static_assert(BYTES <= 160 * 1024, "LDS per workgroup");
  static_assert(LUTV_OFF < 65536, "table offsets fit the instruction offset field");
};

// x of lane n - K (mod 16) of its 16-lane row: DPP row_ror:K (so row_ror:12
// reads lane n + 4).
template <int K>
__device__ __forceinline__ uint32_t row_ror_u(uint32_t x) {
  return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(x), 0x120 + K, 0xf, 0xf, true));
}

// Element i of an MFMA result copied into a register of its own.  A DPP
// operation folded into its user (v_add_f32_dpp) otherwise reads the tuple's
// first register for every element: the fold drops the sub-register index.
__device__ __forceinline__ float own_reg(float x) {
  asm volatile("" : "+v"(x));
  return x;
}

__device__ __forceinline__ uint32_t pack_f16x2(float a, float b) {
  typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
  const h2_t v = {static_cast<_Float16>(a), static_cast<_Float16>(b)};
  return __builtin_bit_cast(uint32_t, v);
}

// c[i] for i < 2^NB from a register array, by a select tree over the bits of i.
template <int NB>
__device__ __forceinline__ float mux_pick(const float (&c)[1 << NB], int i) {
  float v[1 << NB];
#pragma unroll
  for (int k = 0; k < (1 << NB); ++k) v[k] = c[k];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const bool hi = (i >> b) & 1;
#pragma unroll
    for (int k = 0; k < (1 << (NB - 1 - b)); ++k) v[k] = hi ? v[2 * k + 1] : v[2 * k];
  }
  return v[0];
}

template <int D, int KB, int VB, bool PROD = false>
__global__ __launch_bounds__(512, 1) void attn_small_kernel(AttnParams p) {
  using S = SmallShape<D, KB, VB, PROD>;
  constexpr int NW = S::NW;
  constexpr int NT = S::NT;
  constexpr int SUB = S::SUB;
  constexpr int P = S::P;
  constexpr int NQ = S::NQ;
  constexpr int KW = S::KW;
  constexpr int NKI = S::NKI;
  constexpr int CPL = S::CPL;
  constexpr int VRAW = S::VRAW;
  constexpr int PWK = S::PWK;
  constexpr int PWV = S::PWV;
  constexpr int QE = D / kWave;  // query elements per lane

  __shared__ __align__(16) unsigned char lds[S::BYTES];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int n = lane & 15;
  const int g = lane >> 4;
  const int split = blockIdx.x;
  const int gk = blockIdx.y;
  const int b = blockIdx.z;
  // rows r < R * L of this kv head's group: query head gk * R + r / L, position r % L
  const int nrows = p.R * p.L;
  auto row_qoff = [&](int r) -> int64_t {  // (b * Hq + head) * L + position
    return (static_cast<int64_t>(b) * p.Hq + gk * p.R + p.row_head[r]) * p.L + p.row_lpos[r];
  };

  const SeqWindow win = seq_window(p, b);
  const int64_t Tb = win.len;  // token positions below are relative to win.start
  const int64_t t_begin64 = static_cast<int64_t>(split) * p.chunk;
  const bool dense = p.rot_kind == TQ_ROT_DENSE;
  if (t_begin64 >= Tb) {
    // No tokens for this split (it takes no part in the merge).  An empty
    // sequence still needs its output: split 0 writes zeros (the reference
    // divides a zero sum by 1e-6).
    if (Tb <= 0 && split == 0)
      for (int idx = tid; idx < NQ * D; idx += NT)
        if (idx / D < nrows) store_out(p.out, p.q_dtype, row_qoff(idx / D) * D + idx % D, 0.f);
    return;
  }
  const int t_begin = static_cast<int>(t_begin64);
  const int t_end = static_cast<int>(Tb < t_begin64 + p.chunk ? Tb : t_begin64 + p.chunk);
  const int nvalid = static_cast<int>((Tb + p.chunk - 1) / p.chunk);
  const bool nf16 = p.norm_dtype == TQ_DTYPE_F16;

  const int64_t kvrow0 = (static_cast<int64_t>(b) * p.Hkv + gk) * p.cap + win.start;
  const uint32_t tn = static_cast<uint32_t>(t_end);
  const uint32_t nb = nf16 ? 2u : 4u;
  const auto krs = buffer_rsrc(static_cast<const char*>(p.k) + kvrow0 * (PWK * 4), tn * (PWK * 4));
  const auto vrs = buffer_rsrc(static_cast<const char*>(p.v) + kvrow0 * (PWV * 4), tn * (PWV * 4));
  const auto knrs = buffer_rsrc(static_cast<const char*>(p.kn) + kvrow0 * nb, tn * nb);
  const auto vnrs = buffer_rsrc(static_cast<const char*>(p.vn) + kvrow0 * nb, tn * nb);
  // Prod keys: QJL sign rows (D / 8 bytes) and residual norms
  const auto srs = buffer_rsrc(PROD ? static_cast<const char*>(p.ksg) + kvrow0 * (D / 8) : nullptr,
                               PROD ? tn * (D / 8) : 0u);
  const auto rnrs = buffer_rsrc(PROD ? static_cast<const char*>(p.krn) + kvrow0 * nb : nullptr,
                                PROD ? tn * nb : 0u);

  // ---- lane roles
  float lsg[6];  // -1 where lane bit k is set (Hadamard butterflies)
#pragma unroll
  for (int k = 0; k < 6; ++k) lsg[k] = (lane >> k) & 1 ? -1.f : 1.f;
  const int jq = (n >> 2) & 1;  // token subset of this lane's score column
  const int rq = n & 3;         // query row of this lane's score column
  // keys: token 16 (g >> 1) + n, half g & 1
  const uint32_t k_lane = (16 * (g >> 1) + n) * (PWK * 4) + (g & 1) * (KW * 4);
  const uint32_t s_lane = (16 * (g >> 1) + n) * (D / 8) + (g & 1) * (S::SW * 4);
  // norms: tokens 16 jq + 4 g .. + 3 of the sub-chunk
  const uint32_t n_lane = (16 * jq + 4 * g) * nb;
  // values: coordinates CPL n .. CPL n + CPL - 1 of tokens 4g + e, 16 + 4g + e
  const int vbit = CPL * n * VB;
  const uint32_t v_lane = (vbit >> 5) * 4;
  const int vsh = vbit & 31;
  const uint32_t lutk_lane = (lane % S::REPK) * 4;
  const uint32_t lutv_lane = (lane % S::REPV) * 8;
  uint32_t kmask = (S::KKEYS - 1u) << S::LOGSK;
  uint32_t vmask = (S::VKEYS - 1u) << S::LOGSV;
  uint32_t smask = 3u << 8;
  asm volatile("" : "+s"(kmask), "+s"(vmask), "+s"(smask));

  const int n_tok = t_end - t_begin;
  const int n_my = n_tok > wave * SUB ? (n_tok - wave * SUB + NW * SUB - 1) / (NW * SUB) : 0;
  auto sub_start = [&](int i) -> int { return t_begin + (i * NW + wave) * SUB; };

  struct Buf {
    uint32_t k[KW];
    uint32_t nk[4], nv[4];
    uint32_t v[8][VRAW];
    uint32_t sg[PROD ? S::SW : 1], rn[PROD ? 4 : 1];
  };
  auto load_sub = [&](Buf& bf, int s0) {
    const uint32_t t0 = static_cast<uint32_t>(s0);
    load_words<KW>(bf.k, krs, t0 * (PWK * 4) + k_lane);
    if constexpr (PROD) {
      load_words<S::SW>(bf.sg, srs, t0 * (D / 8) + s_lane);
      const auto r = __builtin_amdgcn_raw_buffer_load_b128(rnrs, t0 * nb + n_lane, 0, 0);
#pragma unroll
      for (int e = 0; e < 4; ++e) bf.rn[e] = r[e];
    }
    // 4 norms: 16 bytes (f32) or 8 bytes (f16, the upper two words unused);
    // one load shape for both keeps the buffers in registers
    const uint32_t no = t0 * nb + n_lane;
    const auto a = __builtin_amdgcn_raw_buffer_load_b128(knrs, no, 0, 0);
    const auto c = __builtin_amdgcn_raw_buffer_load_b128(vnrs, no, 0, 0);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      bf.nk[e] = a[e];
      bf.nv[e] = c[e];
    }
    const uint32_t vo = t0 * (PWV * 4) + v_lane;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int tok = (e < 4 ? 4 * g + e : 16 + 4 * g + (e - 4));
      load_words<VRAW>(bf.v[e], vrs, vo + tok * (PWV * 4));
    }
  };
  auto norm4 = [&](const uint32_t (&raw)[4], float (&x)[4]) {
    if (nf16) {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        x[e] = f16_bits_to_f32(static_cast<uint16_t>(raw[e >> 1] >> (16 * (e & 1))));
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) x[e] = __builtin_bit_cast(float, raw[e]);
    }
  };

  // ---- prologue loads first (query row of this wave, signs, codebooks), then
  // the pipeline's sub-chunks (loads complete in order)
  // waves 0..NQ-1 rotate one query row each; with Prod keys waves NQ..2NQ-1
  // bring the projected rows q_proj (set 1, from qprep_kernel)
  const bool qset1 = PROD && wave >= NQ;
  const int qrow = PROD ? (wave & (NQ - 1)) : wave;
  const bool qok = (!PROD || wave < 2 * NQ) && qrow < nrows;
  uint32_t qraw[QE];
  float sgn[QE];
  {
    const bool q32 = dense || qset1 || p.q_dtype == TQ_DTYPE_F32;
    const int64_t qb = !qok ? 0
                       : (dense || qset1) ? row_qoff(qrow) * D
                                          : b * p.q_sb + static_cast<int64_t>(gk * p.R + p.row_head[qrow]) * p.q_sh +
                                                static_cast<int64_t>(p.row_lpos[qrow]) * p.q_sl;
    const void* qsrc = qset1 ? static_cast<const void*>(p.qproj) : dense ? static_cast<const void*>(p.qrot) : p.q;
#pragma unroll
    for (int e = 0; e < QE; ++e) {
      const int64_t i = qb + lane + e * kWave;
      qraw[e] = !qok ? 0u : q32 ? static_cast<const uint32_t*>(qsrc)[i] : static_cast<const uint16_t*>(qsrc)[i];
      sgn[e] = dense ? 1.f : p.krot[lane + e * kWave];
    }
  }
  float ckb[1 << KB], cvb[1 << VB];
#pragma unroll
  for (int i = 0; i < (1 << KB); ++i) ckb[i] = p.kcb[i];
#pragma unroll
  for (int i = 0; i < (1 << VB); ++i) cvb[i] = p.vcb[i];
  // f16 norms with an odd slab end: the dword holding the last token's norm
  // also spans token t_end, so the bounded 16-byte load reads it as zero
  // (range checks are per dword).  That token's norms come from 2-byte loads
  // here and replace the zeros in its sub-chunk (an edge sub-chunk, so the
  // slow path).
  const bool odd_tail = nf16 && (t_end & 1);
  uint32_t tail_k = 0, tail_v = 0, tail_r = 0;
  if (odd_tail) {
    const uint32_t off = static_cast<uint32_t>(t_end - 1) * 2u;
    tail_k = __builtin_amdgcn_raw_buffer_load_b16(knrs, off, 0, 0);
    tail_v = __builtin_amdgcn_raw_buffer_load_b16(vnrs, off, 0, 0);
    if constexpr (PROD) tail_r = __builtin_amdgcn_raw_buffer_load_b16(rnrs, off, 0, 0);
  }
  Buf buf[P];
#pragma unroll
  for (int s = 0; s < P; ++s) load_sub(buf[s], sub_start(s));

  // ---- pair tables: hi and lo f16 parts of (c[a] * s, c[b] * s) for key
  // a | b << bits: keys as a hi table and a lo table of 4-byte entries, values
  // as one table of 8-byte (hi pair, lo pair) entries.  A thread writes 8
  // consecutive replicas of one key with 16-byte stores (lanes write
  // consecutive chunks).
  float kmax = 0.f, vmax = 0.f;
#pragma unroll
  for (int i = 0; i < (1 << KB); ++i) kmax = fmaxf(kmax, fabsf(ckb[i]));
#pragma unroll
  for (int i = 0; i < (1 << VB); ++i) vmax = fmaxf(vmax, fabsf(cvb[i]));
  const float sk = f16_split_scale(kmax);
  const float cbs_v = f16_split_scale(vmax);
  // This thread's table entries (at most one key and one value entry) take
  // their codebook values from the scalar copies (a mux over the index
  // bits).  Vector loads here would complete only after the cache prefetch
  // issued above: loads retire in order.
  static_assert(S::KKEYS * S::REPK / 8 <= NT && S::VKEYS * S::REPV / 8 <= NT, "one table slot per thread");
  const int kslot = tid < S::KKEYS * S::REPK / 8 ? tid : 0;
  const int vslot = tid < S::VKEYS * S::REPV / 8 ? tid : 0;
  const int kkey = kslot / (S::REPK / 8), vkey = vslot / (S::REPV / 8);
  const float cka = mux_pick<KB>(ckb, kkey & ((1 << KB) - 1)), ckb2 = mux_pick<KB>(ckb, kkey >> KB);
  const float cva = mux_pick<VB>(cvb, vkey & ((1 << VB) - 1)), cvb2 = mux_pick<VB>(cvb, vkey >> VB);
  if (tid < S::KKEYS * S::REPK / 8) {
    uint32_t h0, l0, h1, l1;
    split_f16(cka * sk, h0, l0);
    split_f16(ckb2 * sk, h1, l1);
    const uint32_t hi = h0 | (h1 << 16), lo = l0 | (l1 << 16);
    uint4* dh = reinterpret_cast<uint4*>(lds + S::LUTK_OFF) + kslot * 2;
    uint4* dl = reinterpret_cast<uint4*>(lds + S::LUTK_OFF + S::KTAB) + kslot * 2;
    dh[0] = dh[1] = make_uint4(hi, hi, hi, hi);
    dl[0] = dl[1] = make_uint4(lo, lo, lo, lo);
  }
  if (tid < S::VKEYS * S::REPV / 8) {
    uint32_t h0, l0, h1, l1;
    split_f16(cva * cbs_v, h0, l0);
    split_f16(cvb2 * cbs_v, h1, l1);
    const uint32_t hi = h0 | (h1 << 16), lo = l0 | (l1 << 16);
    uint4* d = reinterpret_cast<uint4*>(lds + S::LUTV_OFF) + vslot * 4;
    d[0] = d[1] = d[2] = d[3] = make_uint4(hi, lo, hi, lo);
  }
  if constexpr (PROD) {
    // QJL sign pairs: key a | b << 1 -> (+-1, +-1), 64 replicas, 8 per thread
    if (tid < 32) {
      const int key = tid / 8;
      const uint32_t e = pack_f16x2((key & 1) ? 1.f : -1.f, (key & 2) ? 1.f : -1.f);
      uint4* d = reinterpret_cast<uint4*>(lds + S::SGN_OFF) + tid * 2;
      d[0] = d[1] = make_uint4(e, e, e, e);
    }
  }
  if (tid < S::ZBYTES / 4) reinterpret_cast<uint32_t*>(lds + S::ZERO_OFF)[tid] = 0u;

  // ---- query rows: q_s = round_qdtype(q * scale_q) * s_K, Hadamard, * 1/sqrt(D)
  // (dense: rotated by qprep_kernel), into LDS with the row's max |y|
  if (wave < NQ * S::NQS) {
    float y[QE];
    const bool q32 = dense || qset1 || p.q_dtype == TQ_DTYPE_F32;
    const bool asis = dense || qset1;  // rows already prepared by qprep_kernel
#pragma unroll
    for (int e = 0; e < QE; ++e) {
      const uint32_t raw = qraw[e];
      const float qv = q32 ? __builtin_bit_cast(float, raw)
                           : (p.q_dtype == TQ_DTYPE_F16 ? f16_bits_to_f32(static_cast<uint16_t>(raw))
                                                        : bf16_bits_to_f32(static_cast<uint16_t>(raw)));
      y[e] = asis ? qv : round_q(p.q_dtype, qv * p.scale_q) * sgn[e];
    }
    if (!asis) {
      wave_fwht<D>(y, lsg);
#pragma unroll
      for (int e = 0; e < QE; ++e) y[e] *= p.rscale;
    }
    float m = 0.f;
    float* qy = reinterpret_cast<float*>(lds + S::QY_OFF) + wave * D;  // set 1 rows follow set 0
#pragma unroll
    for (int e = 0; e < QE; ++e) {
      qy[lane + e * kWave] = y[e];
      m = fmaxf(m, fabsf(y[e]));
    }
    m = wave_max(m);
    if (lane == 0) reinterpret_cast<float*>(lds + S::QMAX_OFF)[wave] = m;
  }
  lds_barrier();
  // query pieces in B-operand order: staging [p][r][h][i] holds
  // q_p,r[h D/2 + 8 i + e], e = 0..7, as f16 (one hi/lo scale for all rows)
  const float* qmaxs = reinterpret_cast<const float*>(lds + S::QMAX_OFF);
  const float sq = f16_split_scale(fmaxf(fmaxf(qmaxs[0], qmaxs[1]), fmaxf(qmaxs[2], qmaxs[3])));
  const float sqp = PROD ? f16_split_scale(fmaxf(fmaxf(qmaxs[4], qmaxs[5]), fmaxf(qmaxs[6], qmaxs[7]))) : 1.f;
  for (int idx = tid; idx < S::NQS * NQ * D; idx += NT) {
    const int set = idx / (NQ * D);
    const int r = (idx / D) % NQ;
    const int c = idx % D;
    uint32_t hi, lo;
    split_f16(reinterpret_cast<const float*>(lds + S::QY_OFF)[idx] * (set ? sqp : sq), hi, lo);
    const int h = c / (D / 2);
    const int i = (c % (D / 2)) / 8;
    const int e = c % 8;
    uint16_t* st = reinterpret_cast<uint16_t*>(lds + S::QST_OFF);
    st[((((set * 2 + 0) * NQ + r) * 2 + h) * NKI + i) * 8 + e] = static_cast<uint16_t>(hi);
    st[((((set * 2 + 1) * NQ + r) * 2 + h) * NKI + i) * 8 + e] = static_cast<uint16_t>(lo);
  }
  lds_barrier();
  // B operands: lane (column n = 8 p + 4 jq + rq, g) -- zero unless lane
  // group g holds tokens of subset jq
  u32x4_t qb[NKI];
  uint32_t qb2_addr = 0;  // Prod keys: q_proj operands stay in LDS (registers are full)
  {
    const int pc = n >> 3;
    const bool on = (g >> 1) == jq;
    const uint32_t base = S::QST_OFF + (((pc * NQ + rq) * 2 + (g & 1)) * NKI) * 16;
#pragma unroll
    for (int i = 0; i < NKI; ++i)
      qb[i] = lds_at<u32x4_t>(lds, on ? base + i * 16 : static_cast<uint32_t>(S::ZERO_OFF));
    if constexpr (PROD) qb2_addr = on ? base + 2 * NQ * 2 * NKI * 16 : static_cast<uint32_t>(S::ZERO_OFF);
  }
  // score scale: S * ||k|| * log2(e) / (s_K s_Q) in log2 units
  const float kscale = 1.4426950408889634f * __builtin_amdgcn_rcpf(sk) * __builtin_amdgcn_rcpf(sq);  // powers of two: exact
  // Prod keys: the QJL term's scale sqrt(pi/2) / D * log2(e) / s_P (times n * rn per token)
  const float kscale2 = PROD ? 1.4426950408889634f * p.qjl_scale * __builtin_amdgcn_rcpf(sqp) : 0.f;
  // causal limit of this lane's row (keys t <= lim are visible)
  int lim = INT32_MAX, lim_min = INT32_MAX;
  if (p.causal) {
    const int base_lim = static_cast<int>(Tb - p.L);
#pragma unroll
    for (int r = 0; r < NQ; ++r)
      if (r < nrows) {
        const int lr_ = base_lim + p.row_lpos[r];
        lim_min = min(lim_min, lr_);
        if (rq == r) lim = lr_;
      }
  }

  // ------------------------------------------------------------ streaming ----
  constexpr float kLazy = 7.f;
  f32x4_t O[CPL];
#pragma unroll
  for (int c = 0; c < CPL; ++c) O[c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m_row = -INFINITY;  // reference max of this lane's row (log2 units)
  int E = -1000;            // value-norm exponent of the wave (max ||v|| <= 2^E when set)
  float vsc = 0.f;          // 2^-E
  float nv_lim = 0.f;       // 2^(E + 8): larger norms could overflow an f16 weight
  float l_acc = 0.f;        // sum of p over this lane's tokens

  // two independent accumulator chains (key hi parts, key lo parts); with
  // Prod keys a third against the QJL signs (exact +-1 in f16) and q_proj
  struct Sc {
    f32x4_t c, c2;
  };
  auto scores = [&](const Buf& bf) -> Sc {
    f32x4_t Ch = {0.f, 0.f, 0.f, 0.f}, Cl = {0.f, 0.f, 0.f, 0.f}, Cs = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < NKI; ++i) {
      u32x4_t ah, al;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const uint32_t a = key_addr<2 * KB, S::LOGSK>(bf.k, (8 * i + 2 * u) * KB, lutk_lane, kmask);
        ah[u] = lds_at<uint32_t>(lds, S::LUTK_OFF + a);
        al[u] = lds_at<uint32_t>(lds, S::LUTK_OFF + S::KTAB + opaque(a));
      }
      Ch = mfma_f16(ah, qb[i], Ch);
      Cl = mfma_f16(al, qb[i], Cl);
      if constexpr (PROD) {
        u32x4_t as;
#pragma unroll
        for (int u = 0; u < 4; ++u)
          as[u] = lds_at<uint32_t>(lds, S::SGN_OFF + key_addr<2, 8>(bf.sg, 8 * i + 2 * u, (lane & 63) * 4u, smask));
        Cs = mfma_f16(as, lds_at<u32x4_t>(lds, qb2_addr + i * 16), Cs);
      }
    }
    return Sc{Ch + Cl, Cs};
  };

  auto finish = [&](const Buf& bf, const Sc& SC, int s0) {
    const f32x4_t C = SC.c;
    // ---- value operands first (they do not depend on the softmax, and the
    // slow-path branch below would otherwise keep their table reads behind
    // it): pairs (4g, 4g+1), (4g+2, 4g+3), (16+4g, ..) of coordinate CPL n + c
    constexpr uint32_t MEVEN = [] {
      uint32_t m = 0;
      for (int j = 0; j < CPL; j += 2) m |= ((1u << VB) - 1u) << (j * VB);
      return m;
    }();
    uint32_t zl[4], zh[4];
#pragma unroll
    for (int e2 = 0; e2 < 4; ++e2) {
      uint32_t xa, xb;
      if constexpr (VRAW == 2) {
        xa = __builtin_amdgcn_alignbit(bf.v[2 * e2][1], bf.v[2 * e2][0], vsh);
        xb = __builtin_amdgcn_alignbit(bf.v[2 * e2 + 1][1], bf.v[2 * e2 + 1][0], vsh);
      } else if constexpr (S::SEGBITS < 32) {
        xa = bf.v[2 * e2][0] >> vsh;
        xb = bf.v[2 * e2 + 1][0] >> vsh;
      } else {
        xa = bf.v[2 * e2][0];
        xb = bf.v[2 * e2 + 1][0];
      }
      zl[e2] = (xa & MEVEN) | ((xb << VB) & ~MEVEN);
      zh[e2] = ((xa >> VB) & MEVEN) | (xb & ~MEVEN);
    }
    uint2 vop[CPL][4];
#pragma unroll
    for (int c = 0; c < CPL; ++c)
#pragma unroll
      for (int e2 = 0; e2 < 4; ++e2) {
        const uint32_t z[1] = {(c & 1) ? zh[e2] : zl[e2]};
        vop[c][e2] = lds_at<uint2>(lds, S::LUTV_OFF + key_addr<2 * VB, S::LOGSV>(z, (c >> 1) * 2 * VB, lutv_lane, vmask));
      }
    float nk[4], nv[4], sc[4], d[4];
    norm4(bf.nk, nk);
    norm4(bf.nv, nv);
    // Prod keys: score = n (q_rot . c[idx]) + n * rn * sqrt(pi/2)/D (q_proj . s)
    float ks2[4], sc2[4];
    if constexpr (PROD) {
      float rn[4];
      norm4(bf.rn, rn);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        ks2[i] = nk[i] * rn[i] * kscale2;
        const float ci = own_reg(SC.c2[i]);
        sc2[i] = ci + __builtin_bit_cast(float, row_ror_u<8>(__builtin_bit_cast(uint32_t, ci)));
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float ci = own_reg(C[i]);
      sc[i] = ci + __builtin_bit_cast(float, row_ror_u<8>(__builtin_bit_cast(uint32_t, ci)));
      d[i] = fmaf(sc[i], nk[i] * kscale, PROD ? fmaf(sc2[i], ks2[i], -m_row) : -m_row);
    }
    const float dmax = fmaxf(fmaxf(d[0], d[1]), fmaxf(d[2], d[3]));
    float nvmax = fmaxf(fmaxf(nv[0], nv[1]), fmaxf(nv[2], nv[3]));
    const bool edge = s0 + SUB > t_end || s0 + SUB - 1 > lim_min;  // wave-uniform
    if (edge || __any((dmax > kLazy || nvmax > nv_lim) ? 1 : 0)) {
      // ---- slow path: masks, new reference max / norm exponent, rescale
      const int tbase = s0 + 16 * jq + 4 * g;
      if (odd_tail && edge) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (tbase + i == t_end - 1) {
            nk[i] = f16_bits_to_f32(static_cast<uint16_t>(tail_k));
            nv[i] = f16_bits_to_f32(static_cast<uint16_t>(tail_v));
            if constexpr (PROD) ks2[i] = nk[i] * f16_bits_to_f32(static_cast<uint16_t>(tail_r)) * kscale2;
          }
        nvmax = fmaxf(fmaxf(nv[0], nv[1]), fmaxf(nv[2], nv[3]));
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        sc[i] = PROD ? fmaf(sc[i], nk[i] * kscale, sc2[i] * ks2[i]) : sc[i] * (nk[i] * kscale);
        if (edge) {
          if (tbase + i > lim) sc[i] = -FLT_MAX;
          if (tbase + i >= t_end) sc[i] = -INFINITY;
        }
      }
      float rm = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
      rm = fmaxf(rm, __builtin_bit_cast(float, row_ror_u<4>(__builtin_bit_cast(uint32_t, rm))));
      rm = fmaxf(rm, __builtin_bit_cast(float, row_ror_u<8>(__builtin_bit_cast(uint32_t, rm))));
      rm = fmaxf(rm, xor_lane<16>(rm));
      {
        const float2 h = halves(rm);
        rm = fmaxf(h.x, h.y);  // max of this lane's row over the sub-chunk
      }
      const float vm = wave_max(nvmax);
      int ev;
      frexpf(vm, &ev);
      const int e2 = ev > E ? ev : E;
      const float mn = (rm > m_row + kLazy || m_row == -INFINITY) ? fmaxf(m_row, rm) : m_row;
      // l scales by 2^(m_old - m_new), O also by 2^(E_old - E_new); both
      // start at zero (the first sub-chunk has m_old = -inf)
      const float am = (m_row == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m_row - mn);
      const float ao = am * ldexpf(1.f, E - e2);
      l_acc *= am;
      float ar[NQ];
#pragma unroll
      for (int r = 0; r < NQ; ++r) ar[r] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ao), r));
#pragma unroll
      for (int c = 0; c < CPL; ++c)
#pragma unroll
        for (int r = 0; r < NQ; ++r) O[c][r] *= ar[r];
      m_row = mn;
      E = e2;
      vsc = ldexpf(1.f, -E);
      nv_lim = ldexpf(1.f, E + 8);
      // masked keys (-FLT_MAX) get weight 1 when their whole row is masked
      // (m = -FLT_MAX), else 0; keys past the end (-inf) always 0
#pragma unroll
      for (int i = 0; i < 4; ++i) d[i] = sc[i] - m_row;
    }
    float w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float pe = __builtin_amdgcn_exp2f(d[i]);
      l_acc += pe;
      w[i] = pe * (nv[i] * vsc);
    }
    // ---- weights to the A operands: own 4 tokens (subset 0), then those of
    // lane n + 4 (subset 1); each pair twice, against the (hi pair, lo pair)
    // k slots of the value operand
    const uint32_t w01 = pack_f16x2(w[0], w[1]);
    const uint32_t w23 = pack_f16x2(w[2], w[3]);
    const uint32_t x01 = row_ror_u<12>(w01);
    const uint32_t x23 = row_ror_u<12>(w23);
    const u32x4_t A0 = {w01, w01, w23, w23};
    const u32x4_t A1 = {x01, x01, x23, x23};
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      O[c] = mfma_f16(A0, u32x4_t{vop[c][0].x, vop[c][0].y, vop[c][1].x, vop[c][1].y}, O[c]);
      O[c] = mfma_f16(A1, u32x4_t{vop[c][2].x, vop[c][2].y, vop[c][3].x, vop[c][3].y}, O[c]);
    }
  };

  // Loads are issued unconditionally (past t_end they read zeros for free),
  // so the count of outstanding loads is exact for every sub-chunk.
  Sc Cn;
  if (n_my > 0) Cn = scores(buf[0]);
  for (int base = 0; base < n_my; base += P) {
#pragma unroll
    for (int s = 0; s < P; ++s) {
      const int i = base + s;
      if (i < n_my) {
        const Sc C = Cn;
        finish(buf[s], C, sub_start(i));
        if (i + 1 < n_my) Cn = scores(buf[(s + 1) % P]);
      }
      load_sub(buf[s], sub_start(i + P));
    }
  }

  // --------------------------------------------------- combine the waves ----
  // l of row r: lanes (g', n) with n < 8 (piece 0), subsets n and n + 4
  float lr = l_acc + __builtin_bit_cast(float, row_ror_u<12>(__builtin_bit_cast(uint32_t, l_acc)));
  lr += xor_lane<16>(lr);
  {
    const float2 h = halves(lr);
    lr = h.x + h.y;
  }
  lds_barrier();  // every wave is done with the tables and staging
  float* s_wo = reinterpret_cast<float*>(lds + S::WO_OFF);
  float* s_wm = reinterpret_cast<float*>(lds + S::WM_OFF);
  float* s_wl = reinterpret_cast<float*>(lds + S::WL_OFF);
  float* s_we = reinterpret_cast<float*>(lds + S::WE_OFF);
  float* s_wf = reinterpret_cast<float*>(lds + S::WF_OFF);
  if (g == 0) {
#pragma unroll
    for (int r = 0; r < NQ; ++r) {
      float* dst = s_wo + (wave * NQ + r) * D + CPL * n;
#pragma unroll
      for (int c = 0; c < CPL; ++c) dst[c] = O[c][r];
    }
    if (n < NQ) {
      // a wave without tokens keeps m = -inf and contributes nothing
      s_wm[wave * NQ + n] = m_row;
      s_wl[wave * NQ + n] = lr;
      s_we[wave * NQ + n] = ldexpf(1.f, E);  // undoes the weights' 2^-E
    }
  }
  lds_barrier();
  float* s_fo = reinterpret_cast<float*>(lds + S::FO_OFF);
  float* s_fl = reinterpret_cast<float*>(lds + S::FL_OFF);
  if (tid < NQ) {  // per row: the waves' log-sum-exp factors, l and the reference m
    const int r = tid;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, s_wm[w * NQ + r]);
    float lt = 0.f;
    const float oscale = __builtin_amdgcn_rcpf(cbs_v);  // a power of two: exact
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float wm = s_wm[w * NQ + r];
      const float f = wm == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(wm - M);
      lt = fmaf(s_wl[w * NQ + r], f, lt);
      s_wf[w * NQ + r] = f * s_we[w * NQ + r] * oscale;
    }
    s_fl[r] = lt;
    s_fl[NQ + r] = M;
  }
  lds_barrier();
  for (int idx = tid; idx < NQ * D; idx += NT) {
    const int r = idx / D;
    float a = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) a = fmaf(s_wo[(w * NQ) * D + idx], s_wf[w * NQ + r], a);
    s_fo[idx] = a;
  }
  lds_barrier();

  if (nvalid > 1) {
    // this split's partial for attn_merge_kernel: o through R_V^-1 (Hadamard;
    // it commutes with the merge's weighted sum and normalisation), then
    // o[r][:] and (m, l) per row with m in natural-log units
    if (!dense && wave < NQ) {
      float y[QE];
#pragma unroll
      for (int e = 0; e < QE; ++e) y[e] = s_fo[wave * D + lane + e * kWave];
      wave_fwht<D>(y, lsg);
#pragma unroll
      for (int e = 0; e < QE; ++e) s_fo[wave * D + lane + e * kWave] = y[e] * p.rscale * p.vrot[lane + e * kWave];
    }
    lds_barrier();
    const int64_t grp = static_cast<int64_t>(b) * p.Hkv + gk;
    float4* po4 = reinterpret_cast<float4*>(p.po + (grp * p.n_splits + split) * static_cast<int64_t>(NQ) * D);
    for (int idx = tid; idx < NQ * D / 4; idx += NT) po4[idx] = reinterpret_cast<const float4*>(s_fo)[idx];
    if (tid < NQ) {
      float* pm = p.pml + ((grp * p.n_splits + split) * NQ + tid) * 2;
      pm[0] = s_fl[NQ + tid] * 0.6931471805599453f;
      pm[1] = s_fl[tid];
    }
    return;
  }

  // ---- finish: o / l (0 when no token is visible), R_V^-1, store
  if (!dense) {
    if (wave < nrows) {
      const float lt = s_fl[wave];
      const float inv = lt > 0.f ? 1.f / lt : 0.f;
      float y[QE];
#pragma unroll
      for (int e = 0; e < QE; ++e) y[e] = s_fo[wave * D + lane + e * kWave] * inv;
      wave_fwht<D>(y, lsg);
      const int64_t qo = row_qoff(wave) * D;
#pragma unroll
      for (int e = 0; e < QE; ++e)
        store_out(p.out, p.q_dtype, qo + lane + e * kWave, y[e] * p.rscale * p.vrot[lane + e * kWave]);
    }
  } else {
    dense_rows_out<D, NQ, NT>(p, s_fo, s_wo, nrows, row_qoff, [&](int r) {  // s_wo is dead
      const float lt = s_fl[r];
      return lt > 0.f ? 1.f / lt : 0.f;
    });
  }
}

template <int D, int KB, int VB, bool PROD = false>
int launch_small(const AttnParams& p, hipStream_t st) {
  const dim3 grid(p.n_splits, p.Hkv, p.B);
  hipLaunchKernelGGL((attn_small_kernel<D, KB, VB, PROD>), grid, dim3(SmallShape<D, KB, VB, PROD>::NT), 0, st, p);
  return check_launch("attn_small_kernel");
}

}  // namespace tq
