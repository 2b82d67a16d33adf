// TurboQuant verify / prefill / wide-GQA attention for 16-row groups at head
// dim 128, straight from packed indices: the layout of the small row-group
// kernel (tq_attn_small.h) with all 16 MFMA columns holding query rows.
//
// Workgroup: 8 wave64s own tokens [t_begin, t_end) of one (sequence, kv head)
// and 16 query rows of its GQA group (row group rg: rows 16 rg .. 16 rg + 15
// of the R * L rows, row -> (head r / L, position r % L)).  Tokens are cut
// into 32-token sub-chunks; sub-chunk i belongs to wave i % 8, and each wave
// keeps the global loads of its next P sub-chunks in flight.
//
// Lane roles (l = lane, n = l % 16, g = l / 16):
//   scores  S^T[tok][row] = sum_d k[tok][d] * q_row[d]   (two 16 x 16 tiles)
//     A = keys: lane (m, g) holds tokens m and 16 + m, coordinate quarter g
//         (D/4 coordinates: a contiguous bit span of each packed row); MFMA
//         j of a tile takes coordinates g D/4 + 8 j .. + 7 of every lane,
//         hi and lo f16 parts of the codebook values from two tables,
//     B = queries: lane (row n, g) holds the same coordinates of row n, hi
//         and lo f16 parts in separate operands.  k_hi q_hi + k_hi q_lo +
//         k_lo q_hi keeps f32-class accuracy (the dropped k_lo q_lo term is
//         below 2^-22 relative).
//     Output: lane (g, row n), register i = token 4g + i of the tile.
//   softmax per lane: 8 tokens of row n (4 per tile).
//     With 1- and 2-bit keys one table read gives four coordinates (an
//     8-byte hi entry and an 8-byte lo entry, 32 replicas: conflict-free).
//   values  O[row][d] = sum_tok w[row][tok] * v[tok][d]   (16 x 16 tiles)
//     A = weights: lane (row n, g) holds tokens 4g .. 4g+3 and 16+4g ..
//         16+4g+3 as f16 -- exactly its own 8 weights: no transpose,
//     B = values: as in the small kernel, (hi pair, lo pair) of two tokens
//         per 8-byte table read against weights (w_a, w_b, w_a, w_b);
//         1-bit values as v = mid + half * s: the signs s = +-1 of four
//         tokens per 8-byte read, exact in f16, all 32 tokens in one MFMA.
//     Output: lane (g, n), register i = row 4g + i, coordinate (D/16) n + c.
// Softmax, value-norm exponent and table replication are those of the small
// kernel.  Splits leave o in the rotated basis for the merge (16 rows per
// group): attn_merge_rot_kernel applies R_V^-1 once per row.
// Semantics: quantized_attention, turboquant_cache.py:5110-5203.
#pragma once

#include "tq_attn_small.h"

namespace tq {

// log2 of a power of two
constexpr int ilog2(int x) { return x <= 1 ? 0 : 1 + ilog2(x / 2); }

template <int KB, int VB>
struct Rows16Shape {
  static constexpr int D = 128;
  static constexpr int NW = 8;
  static constexpr int NT = NW * kWave;
  static constexpr int SUB = 32;  // tokens per sub-chunk (two 16-token tiles)
  static constexpr int P = 2;     // sub-chunks in flight per wave
  static constexpr int NQ = 16;   // query rows
  // keys: a lane holds a quarter row of two tokens
  static constexpr int QTR = D / 4;
  static constexpr int KW = QTR * KB / 32;  // words per token and lane
  static constexpr int PWK = D * KB / 32;
  static constexpr int NKJ = D / 32;        // MFMAs per tile and key piece
  // A key-table read covers KCO coordinates of one token: four at 1 and 2
  // bits (8-byte entries of four f16), else two (4-byte entries).
  static constexpr bool QUADK = KB <= 2;
  static constexpr int KCO = QUADK ? 4 : 2;
  static constexpr int KEB = 2 * KCO;  // bytes per hi or lo entry
  static constexpr int KKEYS = 1 << (KCO * KB);
  // 32 replicas of 8-byte entries: the 32 lanes of one half-wave read
  // distinct banks whatever their keys (16 where the LDS cannot hold 2 x 64
  // KiB of key tables beside wide value tables)
  static constexpr int REPK = QUADK ? (KKEYS <= 16 || VB <= 2 ? 32 : 16) : (KKEYS <= 64 ? 64 : 16);
  static constexpr int LOGSK = ilog2(REPK * KEB);
  // values: a lane holds CPL consecutive coordinates of 8 tokens
  static constexpr int CPL = D / 16;
  static constexpr int PWV = D * VB / 32;
  static constexpr int SEGBITS = CPL * VB;
  static constexpr int VRAW = (VB == 3) ? 2 : 1;
  // 1-bit values: v = m + h s with s = +-1 exact in f16, so the value
  // operand needs no hi/lo split; a table read gives s of four tokens for one
  // coordinate (16 keys, four f16).  Wider values: a read gives the (hi
  // pair, lo pair) of two tokens' codebook values.
  static constexpr bool SIGNV = VB == 1;
  static constexpr int VKEYS = SIGNV ? 16 : 1 << (2 * VB);
  static constexpr int REPV = SIGNV ? 32 : (VKEYS <= 64 ? 64 : 16);
  static constexpr int LOGSV = ilog2(REPV * 8);
  // LDS (bytes): [K hi table][K lo table][V table][q staging][rows][row max]
  static constexpr int KTAB = KKEYS * REPK * KEB;
  static constexpr int VTAB = VKEYS * REPV * 8;
  static constexpr int LUTK_OFF = 0;
  static constexpr int LUTV_OFF = 2 * KTAB;
  // A table offset beyond the 16-bit instruction offset goes into the lane
  // base instead (by OR: the offset is a multiple of the table size).
  static constexpr bool VOFF_IN_BASE = LUTV_OFF > 65535;
  static constexpr int QST_OFF = LUTV_OFF + VTAB;  // [piece][row][g][j] 8 x f16 = 16 B
  static constexpr int QST_BYTES = 2 * NQ * 4 * NKJ * 16;
  static constexpr int QY_OFF = QST_OFF + QST_BYTES;    // [NQ][D] f32 rotated queries
  static constexpr int QMAX_OFF = QY_OFF + NQ * D * 4;  // [NQ] f32
  static constexpr int LOOP_BYTES = QMAX_OFF + NQ * 4;
  // epilogue (after a barrier the loop's buffers are dead)
  static constexpr int WO_OFF = 0;                         // [NW][NQ][D] f32
  static constexpr int WM_OFF = WO_OFF + NW * NQ * D * 4;  // [NW][NQ]
  static constexpr int WL_OFF = WM_OFF + NW * NQ * 4;
  static constexpr int WE_OFF = WL_OFF + NW * NQ * 4;
  static constexpr int WF_OFF = WE_OFF + NW * NQ * 4;
  static constexpr int WV_OFF = WF_OFF + NW * NQ * 4;      // [NW][NQ] weight sums (1-bit values)
  static constexpr int FO_OFF = WV_OFF + NW * NQ * 4;      // [NQ][D] final rows
  static constexpr int FL_OFF = FO_OFF + NQ * D * 4;       // [NQ] l, [NQ] m, [NQ] v_mid term
  static constexpr int POST_BYTES = FL_OFF + 3 * NQ * 4;
  static constexpr int BYTES = LOOP_BYTES > POST_BYTES ? LOOP_BYTES : POST_BYTES;
  static_assert(KW * 32 == QTR * KB, "key quarter rows are whole words");
  static_assert(SEGBITS <= 32, "value segment in one word");
  static_assert(BYTES <= 160 * 1024, "LDS per workgroup");
  // the lo table sits at an instruction offset when that fits, else its
  // offset (a power of two above every hi-table address) is ORed in
  static constexpr bool KLO_IN_BASE = LUTK_OFF + KTAB > 65535;
  static_assert(!KLO_IN_BASE || (LUTK_OFF == 0 && (KTAB & (KTAB - 1)) == 0), "lo table offset ORs into the address");
  static_assert(!VOFF_IN_BASE || LUTV_OFF % VTAB == 0, "value table offset ORs into the lane base");
};

template <int KB, int VB>
__global__ __launch_bounds__(512, 1) void attn_rows16_kernel(AttnParams p) {
  using S = Rows16Shape<KB, VB>;
  constexpr int D = S::D;
  constexpr int NW = S::NW;
  constexpr int NT = S::NT;
  constexpr int SUB = S::SUB;
  constexpr int P = S::P;
  constexpr int NQ = S::NQ;
  constexpr int KW = S::KW;
  constexpr int NKJ = S::NKJ;
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
  const int gk = blockIdx.y / p.n_rg;
  const int rg = blockIdx.y % p.n_rg;
  const int b = blockIdx.z;
  RowSet rs;
  rs.init(p, b, gk, rg, NQ);

  const SeqWindow win = seq_window(p, b);
  const int64_t Tb = win.len;  // token positions below are relative to win.start
  const int64_t t_begin64 = static_cast<int64_t>(split) * p.chunk;
  const bool dense = p.rot_kind == TQ_ROT_DENSE;
  if (t_begin64 >= Tb) {
    // No tokens for this split (it takes no part in the merge); an empty
    // sequence's rows are zeros, written by split 0.
    if (Tb <= 0 && split == 0)
      for (int idx = tid; idx < NQ * D; idx += NT)
        if (rs.valid(idx / D)) store_out(p.out, p.q_dtype, rs.qoff(idx / D) * D + idx % D, 0.f);
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

  // ---- lane roles
  float lsg[6];  // -1 where lane bit k is set (Hadamard butterflies)
#pragma unroll
  for (int k = 0; k < 6; ++k) lsg[k] = (lane >> k) & 1 ? -1.f : 1.f;
  // keys: tokens n and 16 + n, quarter g
  const uint32_t k_lane = n * (PWK * 4) + g * (KW * 4);
  // norms: tokens 4g .. 4g + 3 of each tile
  const uint32_t n_lane = 4 * g * nb;
  // values: coordinates CPL n .. CPL n + CPL - 1 of tokens 4g + e, 16 + 4g + e
  const int vbit = CPL * n * VB;
  const uint32_t v_lane = (vbit >> 5) * 4;
  const int vsh = vbit & 31;
  const uint32_t lutk_lane = (lane % S::REPK) * S::KEB;
  const uint32_t lutv_lane = (S::VOFF_IN_BASE ? S::LUTV_OFF : 0) + (lane % S::REPV) * 8;
  constexpr int VOFF = S::VOFF_IN_BASE ? 0 : S::LUTV_OFF;  // instruction offset of value-table reads
  uint32_t kmask = (S::KKEYS - 1u) << S::LOGSK;
  uint32_t vmask = (S::VKEYS - 1u) << S::LOGSV;
  asm volatile("" : "+s"(kmask), "+s"(vmask));

  const int n_tok = t_end - t_begin;
  const int n_my = n_tok > wave * SUB ? (n_tok - wave * SUB + NW * SUB - 1) / (NW * SUB) : 0;
  auto sub_start = [&](int i) -> int { return t_begin + (i * NW + wave) * SUB; };

  struct Buf {
    uint32_t k[2][KW];
    uint32_t nk[2][4], nv[2][4];
    uint32_t v[8][VRAW];
  };
  auto load_sub = [&](Buf& bf, int s0) {
    const uint32_t t0 = static_cast<uint32_t>(s0);
#pragma unroll
    for (int t = 0; t < 2; ++t) load_words<KW>(bf.k[t], krs, (t0 + 16 * t) * (PWK * 4) + k_lane);
    // 4 norms per tile: 16 bytes (f32) or 8 bytes (f16, the upper two words
    // unused); one load shape for both keeps the buffers in registers
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const uint32_t no = (t0 + 16 * t) * nb + n_lane;
      const auto a = __builtin_amdgcn_raw_buffer_load_b128(knrs, no, 0, 0);
      const auto c = __builtin_amdgcn_raw_buffer_load_b128(vnrs, no, 0, 0);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        bf.nk[t][e] = a[e];
        bf.nv[t][e] = c[e];
      }
    }
    if constexpr (S::SIGNV) {
      // the lane's CPL = 8 one-bit fields of each token are byte n of the
      // row; tokens 4g + e and 16 + 4g + e at constant offsets from one base
      const uint32_t vo = (t0 + 4 * g) * (PWV * 4) + n;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t dt = e < 4 ? e : 16 + (e - 4);
        bf.v[e][0] = __builtin_amdgcn_raw_buffer_load_b8(vrs, vo + dt * (PWV * 4), 0, 0);
      }
    } else {
      const uint32_t vo = t0 * (PWV * 4) + v_lane;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int tok = (e < 4 ? 4 * g + e : 16 + 4 * g + (e - 4));
        load_words<VRAW>(bf.v[e], vrs, vo + tok * (PWV * 4));
      }
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

  float ckb[1 << KB], cvb[1 << VB];
#pragma unroll
  for (int i = 0; i < (1 << KB); ++i) ckb[i] = p.kcb[i];
#pragma unroll
  for (int i = 0; i < (1 << VB); ++i) cvb[i] = p.vcb[i];
  // ---- prologue: the codebooks first, then this wave's two query rows and
  // the signs; the pair tables are built before the pipeline's sub-chunks are
  // requested, so that waiting for the codebooks never waits for the
  // sub-chunks behind them (loads complete in order)
  uint32_t qraw[2][QE];
  float sgn[QE];
  {
    const bool q32 = dense || p.q_dtype == TQ_DTYPE_F32;
    const void* qsrc = dense ? static_cast<const void*>(p.qrot) : p.q;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int r = wave + NW * h;
      const bool ok = rs.valid(r);
      const int64_t qb = !ok ? 0
                         : dense ? rs.qoff(r) * D
                                 : b * p.q_sb + static_cast<int64_t>(rs.head(r)) * p.q_sh +
                                       static_cast<int64_t>(rs.lpos(r)) * p.q_sl;
#pragma unroll
      for (int e = 0; e < QE; ++e) {
        const int64_t i = qb + lane + e * kWave;
        qraw[h][e] = !ok ? 0u : q32 ? static_cast<const uint32_t*>(qsrc)[i] : static_cast<const uint16_t*>(qsrc)[i];
      }
    }
#pragma unroll
    for (int e = 0; e < QE; ++e) sgn[e] = dense ? 1.f : p.krot[lane + e * kWave];
  }
  // f16 norms with an odd slab end: the last token's norms are read with
  // 2-byte loads (the 16-byte load reads the dword that also spans token
  // t_end as zero) and patched in its sub-chunk's slow path
  const bool odd_tail = nf16 && (t_end & 1);
  uint32_t tail_k = 0, tail_v = 0;
  if (odd_tail) {
    const uint32_t off = static_cast<uint32_t>(t_end - 1) * 2u;
    tail_k = __builtin_amdgcn_raw_buffer_load_b16(knrs, off, 0, 0);
    tail_v = __builtin_amdgcn_raw_buffer_load_b16(vnrs, off, 0, 0);
  }
  // ---- pair tables (as in the small kernel): keys as hi and lo tables of
  // 4-byte entries, values as (hi pair, lo pair) entries
  float kmax = 0.f, vmax = 0.f;
#pragma unroll
  for (int i = 0; i < (1 << KB); ++i) kmax = fmaxf(kmax, fabsf(ckb[i]));
#pragma unroll
  for (int i = 0; i < (1 << VB); ++i) vmax = fmaxf(vmax, fabsf(cvb[i]));
  const float sk = f16_split_scale(kmax);
  const float cbs_v = f16_split_scale(vmax);
  static_assert((S::QUADK || S::KKEYS * S::REPK / 8 <= NT) && S::VKEYS * S::REPV / 8 <= NT, "one table slot per thread");
  // a thread writes 8 consecutive replicas of one key
  {
    const int kslot = tid < S::KKEYS * S::REPK / 8 ? tid : 0;
    const int vslot = tid < S::VKEYS * S::REPV / 8 ? tid : 0;
    const int kkey = kslot / (S::REPK / 8), vkey = vslot / (S::REPV / 8);
    if constexpr (S::QUADK) {
      // key f0 | f1 << KB | f2 << 2 KB | f3 << 3 KB: f16 parts of c[f0] s .. c[f3] s
#pragma unroll
      for (int t = tid; t < S::KKEYS * S::REPK / 8; t += NT) {
        const int key = t / (S::REPK / 8);
        uint32_t h[4], l[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) split_f16(mux_pick<KB>(ckb, (key >> (KB * i)) & ((1 << KB) - 1)) * sk, h[i], l[i]);
        const uint32_t h01 = h[0] | (h[1] << 16), h23 = h[2] | (h[3] << 16);
        const uint32_t l01 = l[0] | (l[1] << 16), l23 = l[2] | (l[3] << 16);
        uint4* dh = reinterpret_cast<uint4*>(lds + S::LUTK_OFF) + t * 4;
        uint4* dl = reinterpret_cast<uint4*>(lds + S::LUTK_OFF + S::KTAB) + t * 4;
        dh[0] = dh[1] = dh[2] = dh[3] = make_uint4(h01, h23, h01, h23);
        dl[0] = dl[1] = dl[2] = dl[3] = make_uint4(l01, l23, l01, l23);
      }
    } else {
      const float cka = mux_pick<KB>(ckb, kkey & ((1 << KB) - 1)), ckb2 = mux_pick<KB>(ckb, kkey >> KB);
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
    }
    if constexpr (S::SIGNV) {
      // entry e: s = +1 (f16 0x3c00) where bit e of the key is set, else -1 (0xbc00)
      uint32_t sg[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) sg[e] = (vkey >> e) & 1 ? 0x3c00u : 0xbc00u;
      if (tid < S::VKEYS * S::REPV / 8) {
        const uint32_t x = sg[0] | (sg[1] << 16), y = sg[2] | (sg[3] << 16);
        uint4* d = reinterpret_cast<uint4*>(lds + S::LUTV_OFF) + vslot * 4;
        d[0] = d[1] = d[2] = d[3] = make_uint4(x, y, x, y);
      }
    } else {
      const float cva = mux_pick<VB>(cvb, vkey & ((1 << VB) - 1)), cvb2 = mux_pick<VB>(cvb, vkey >> VB);
      if (tid < S::VKEYS * S::REPV / 8) {
        uint32_t h0, l0, h1, l1;
        split_f16(cva * cbs_v, h0, l0);
        split_f16(cvb2 * cbs_v, h1, l1);
        const uint32_t hi = h0 | (h1 << 16), lo = l0 | (l1 << 16);
        uint4* d = reinterpret_cast<uint4*>(lds + S::LUTV_OFF) + vslot * 4;
        d[0] = d[1] = d[2] = d[3] = make_uint4(hi, lo, hi, lo);
      }
    }
  }

  Buf buf[P];
#pragma unroll
  for (int s = 0; s < P; ++s) load_sub(buf[s], sub_start(s));

  // ---- query rows: q_s = round_qdtype(q * scale_q) * s_K, Hadamard, * 1/sqrt(D)
  // (dense: rotated by qprep_kernel), into LDS with each row's max |y|
  {
    const bool q32 = dense || p.q_dtype == TQ_DTYPE_F32;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int r = wave + NW * h;
      float y[QE];
#pragma unroll
      for (int e = 0; e < QE; ++e) {
        const uint32_t raw = qraw[h][e];
        const float qv = q32 ? __builtin_bit_cast(float, raw)
                             : (p.q_dtype == TQ_DTYPE_F16 ? f16_bits_to_f32(static_cast<uint16_t>(raw))
                                                          : bf16_bits_to_f32(static_cast<uint16_t>(raw)));
        y[e] = dense ? qv : round_q(p.q_dtype, qv * p.scale_q) * sgn[e];
      }
      if (!dense) {
        wave_fwht<D>(y, lsg);
#pragma unroll
        for (int e = 0; e < QE; ++e) y[e] *= p.rscale;
      }
      float m = 0.f;
      float* qy = reinterpret_cast<float*>(lds + S::QY_OFF) + r * D;
#pragma unroll
      for (int e = 0; e < QE; ++e) {
        qy[lane + e * kWave] = y[e];
        m = fmaxf(m, fabsf(y[e]));
      }
      m = wave_max(m);
      if (lane == 0) reinterpret_cast<float*>(lds + S::QMAX_OFF)[r] = m;
    }
  }
  lds_barrier();
  // query pieces in B-operand order: staging [piece][r][g][j] holds
  // q_r[g D/4 + 8 j + e], e = 0..7, as f16 (one hi/lo scale for all rows)
  float qm = 0.f;
#pragma unroll
  for (int r = 0; r < NQ; ++r) qm = fmaxf(qm, reinterpret_cast<const float*>(lds + S::QMAX_OFF)[r]);
  const float sq = f16_split_scale(qm);
  for (int idx = tid; idx < NQ * D; idx += NT) {
    const int r = idx / D;
    const int c = idx % D;
    uint32_t hi, lo;
    split_f16(reinterpret_cast<const float*>(lds + S::QY_OFF)[idx] * sq, hi, lo);
    const int qg = c / S::QTR;
    const int j = (c % S::QTR) / 8;
    const int e = c % 8;
    uint16_t* st = reinterpret_cast<uint16_t*>(lds + S::QST_OFF);
    st[(((0 * NQ + r) * 4 + qg) * NKJ + j) * 8 + e] = static_cast<uint16_t>(hi);
    st[(((1 * NQ + r) * 4 + qg) * NKJ + j) * 8 + e] = static_cast<uint16_t>(lo);
  }
  lds_barrier();
  u32x4_t qbh[NKJ], qbl[NKJ];
#pragma unroll
  for (int j = 0; j < NKJ; ++j) {
    qbh[j] = lds_at<u32x4_t>(lds, S::QST_OFF + (((0 * NQ + n) * 4 + g) * NKJ + j) * 16);
    qbl[j] = lds_at<u32x4_t>(lds, S::QST_OFF + (((1 * NQ + n) * 4 + g) * NKJ + j) * 16);
  }
  // score scale: S * ||k|| * log2(e) / (s_K s_Q) in log2 units
  const float kscale = 1.4426950408889634f * __builtin_amdgcn_rcpf(sk) * __builtin_amdgcn_rcpf(sq);  // powers of two: exact
  // causal limit of this lane's row n (keys t <= lim are visible)
  int lim = INT32_MAX, lim_min = INT32_MAX;
  if (p.causal) {
    const int base_lim = static_cast<int>(Tb - p.L);
    for (int r = 0; r < NQ; ++r)
      if (rs.valid(r)) {
        const int lr_ = base_lim + rs.lpos(r);
        lim_min = min(lim_min, lr_);
        if (n == r) lim = lr_;
      }
  }

  // ------------------------------------------------------------ streaming ----
  constexpr float kLazy = 7.f;
  f32x4_t O[CPL];
#pragma unroll
  for (int c = 0; c < CPL; ++c) O[c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m_row = -INFINITY;  // reference max of row n (log2 units)
  int E = -1000;            // value-norm exponent of the wave (max ||v|| <= 2^E when set)
  // The weights are p 2^-E ||v||: 2^-E rides in the exponent, p 2^-E =
  // exp2(s - (m_row + E)), so l and O both count in units of 2^E.
  float mE = -INFINITY;     // m_row + E
  float d_lim = 0.f;        // kLazy - E: the lazy bound on s - mE
  float nv_lim = 0.f;       // 2^(E + 8): larger norms could overflow an f16 weight
  float l_acc = 0.f;        // sum of p 2^-E over this lane's tokens of row n
  // 1-bit values: v = v_mid + v_half s.  Lw accumulates the f16 weights
  // (row 4g + i in register i, every column alike) when v_mid != 0.
  f32x4_t Lw = {0.f, 0.f, 0.f, 0.f};
  const float v_mid = 0.5f * (cvb[0] + cvb[(1 << VB) - 1]);
  const float v_half = 0.5f * (cvb[(1 << VB) - 1] - cvb[0]);

  struct Scores {
    f32x4_t c[2];
  };
  // per tile two accumulator chains (key hi parts against both query
  // pieces, key lo parts against the query hi part)
  auto scores = [&](const Buf& bf) -> Scores {
    f32x4_t Ch[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
    f32x4_t Cl[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int j = 0; j < NKJ; ++j)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        u32x4_t ah, al;
        if constexpr (S::QUADK && KB == 2 && S::REPK == 32) {
          // the 8-bit key is byte k of a key word: v_perm_b32 puts it into
          // address byte 1 (entries of one key span 256 B) beside the lane's
          // replica offset (byte 0) and the lo table's offset (byte 2)
          static_assert(S::LOGSK == 8 && S::LUTK_OFF == 0 && S::KTAB == 65536, "byte-addressed key tables");
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            const int pos = (8 * j + 4 * u) * KB;
            const uint32_t sel = (4u + ((pos >> 3) & 3)) << 8;
            const uint32_t wv = bf.k[t][pos >> 5];
            const uint2 eh = lds_at<uint2>(lds, __builtin_amdgcn_perm(wv, lutk_lane, 0x0c0c0000u | sel));
            const uint2 el = lds_at<uint2>(lds, __builtin_amdgcn_perm(wv, lutk_lane | S::KTAB, 0x0c020000u | sel));
            ah[2 * u] = eh.x, ah[2 * u + 1] = eh.y;
            al[2 * u] = el.x, al[2 * u + 1] = el.y;
          }
        } else if constexpr (S::QUADK) {
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            const uint32_t a = key_addr<4 * KB, S::LOGSK>(bf.k[t], (8 * j + 4 * u) * KB, lutk_lane, kmask);
            const uint2 eh = lds_at<uint2>(lds, S::LUTK_OFF + a);
            const uint2 el = S::KLO_IN_BASE ? lds_at<uint2>(lds, opaque(a) | S::KTAB)
                                            : lds_at<uint2>(lds, S::LUTK_OFF + S::KTAB + opaque(a));
            ah[2 * u] = eh.x, ah[2 * u + 1] = eh.y;
            al[2 * u] = el.x, al[2 * u + 1] = el.y;
          }
        } else {
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const uint32_t a = key_addr<2 * KB, S::LOGSK>(bf.k[t], (8 * j + 2 * u) * KB, lutk_lane, kmask);
            ah[u] = lds_at<uint32_t>(lds, S::LUTK_OFF + a);
            al[u] = lds_at<uint32_t>(lds, S::LUTK_OFF + S::KTAB + opaque(a));
          }
        }
        Ch[t] = mfma_f16(ah, qbh[j], Ch[t]);
        Cl[t] = mfma_f16(al, qbh[j], Cl[t]);
        Ch[t] = mfma_f16(ah, qbl[j], Ch[t]);
      }
    return Scores{{Ch[0] + Cl[0], Ch[1] + Cl[1]}};
  };

  auto finish = [&](const Buf& bf, const Scores& C, int s0) {
    // ---- value operands first (independent of the softmax)
    constexpr int NVR = S::SIGNV ? 2 : 4;  // value-table reads per coordinate
    uint2 vop[CPL][NVR];
    if constexpr (S::SIGNV) {
      // nibble keys of 4 tokens (bit e: token e of a tile) for one coordinate.
      // The tile's four bytes (token e = byte e, coordinate c = bit c) form
      // a 4 x 8 bit matrix; two delta swaps transpose its 4 x 4 blocks, after
      // which the nibble at bit 8 (c & 3) + 4 (c >> 2) holds coordinate c's
      // four tokens.
      static_assert(CPL == 8, "one byte of one-bit fields per token and lane");
      uint32_t y[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        uint32_t x = bf.v[4 * t][0] | (bf.v[4 * t + 1][0] << 8) | (bf.v[4 * t + 2][0] << 16) |
                     (bf.v[4 * t + 3][0] << 24);
        uint32_t u = ((x >> 7) ^ x) & 0x00aa00aau;  // 2 x 2 blocks
        x ^= u ^ (u << 7);
        u = ((x >> 14) ^ x) & 0x0000ccccu;  // 4 x 4 blocks of them
        x ^= u ^ (u << 14);
        y[t] = x;
      }
#pragma unroll
      for (int c = 0; c < CPL; ++c)
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const uint32_t z[1] = {y[t]};
          vop[c][t] = lds_at<uint2>(lds, VOFF + key_addr<4, S::LOGSV>(z, 8 * (c & 3) + 4 * (c >> 2), lutv_lane, vmask));
        }
    } else {
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
#pragma unroll
      for (int c = 0; c < CPL; ++c)
#pragma unroll
        for (int e2 = 0; e2 < 4; ++e2) {
          const uint32_t z[1] = {(c & 1) ? zh[e2] : zl[e2]};
          vop[c][e2] = lds_at<uint2>(lds, VOFF + key_addr<2 * VB, S::LOGSV>(z, (c >> 1) * 2 * VB, lutv_lane, vmask));
        }
    }
    float nk[8], nv[8], sc[8], d[8];
    {
      float a0[4], a1[4], c0[4], c1[4];
      norm4(bf.nk[0], a0);
      norm4(bf.nk[1], a1);
      norm4(bf.nv[0], c0);
      norm4(bf.nv[1], c1);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        nk[e] = a0[e];
        nk[4 + e] = a1[e];
        nv[e] = c0[e];
        nv[4 + e] = c1[e];
      }
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      sc[k] = own_reg(C.c[k >> 2][k & 3]);
      d[k] = fmaf(sc[k], nk[k] * kscale, -mE);
    }
    float dmax = d[0], nvmax = nv[0];
#pragma unroll
    for (int k = 1; k < 8; ++k) {
      dmax = fmaxf(dmax, d[k]);
      nvmax = fmaxf(nvmax, nv[k]);
    }
    const bool edge = s0 + SUB > t_end || s0 + SUB - 1 > lim_min;  // wave-uniform
    if (edge || __any((dmax > d_lim || nvmax > nv_lim) ? 1 : 0)) {
      // ---- slow path: masks, new reference max / norm exponent, rescale
      if (odd_tail && edge) {
#pragma unroll
        for (int k = 0; k < 8; ++k)
          if (s0 + 16 * (k >> 2) + 4 * g + (k & 3) == t_end - 1) {
            nk[k] = f16_bits_to_f32(static_cast<uint16_t>(tail_k));
            nv[k] = f16_bits_to_f32(static_cast<uint16_t>(tail_v));
          }
        nvmax = nv[0];
#pragma unroll
        for (int k = 1; k < 8; ++k) nvmax = fmaxf(nvmax, nv[k]);
      }
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        sc[k] *= nk[k] * kscale;
        if (edge) {
          const int t = s0 + 16 * (k >> 2) + 4 * g + (k & 3);
          if (t > lim) sc[k] = -FLT_MAX;
          if (t >= t_end) sc[k] = -INFINITY;
        }
      }
      float rm = sc[0];
#pragma unroll
      for (int k = 1; k < 8; ++k) rm = fmaxf(rm, sc[k]);
      rm = fmaxf(rm, xor_lane<16>(rm));
      {
        const float2 h = halves(rm);
        rm = fmaxf(h.x, h.y);  // max of row n over the sub-chunk
      }
      const float vm = wave_max(nvmax);
      int ev;
      frexpf(vm, &ev);
      const int e2 = ev > E ? ev : E;
      const float mn = (rm > m_row + kLazy || m_row == -INFINITY) ? fmaxf(m_row, rm) : m_row;
      // l and O scale by 2^(m_old - m_new) 2^(E_old - E_new); both start at
      // zero (the first sub-chunk has m_old = -inf)
      const float am = (m_row == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m_row - mn);
      const float ao = am * ldexpf(1.f, E - e2);
      l_acc *= ao;
      // O register i of lane group g' is row 4 g' + i: its factor sits in lane 4 g' + i
      float ar[NQ];
#pragma unroll
      for (int r = 0; r < NQ; ++r) ar[r] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ao), r));
      float fr[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) fr[i] = g == 0 ? ar[i] : g == 1 ? ar[4 + i] : g == 2 ? ar[8 + i] : ar[12 + i];
#pragma unroll
      for (int c = 0; c < CPL; ++c)
#pragma unroll
        for (int i = 0; i < 4; ++i) O[c][i] *= fr[i];
      if constexpr (S::SIGNV) {
#pragma unroll
        for (int i = 0; i < 4; ++i) Lw[i] *= fr[i];
      }
      m_row = mn;
      E = e2;
      mE = m_row + static_cast<float>(E);
      d_lim = kLazy - static_cast<float>(E);
      nv_lim = ldexpf(1.f, E + 8);
      // masked keys (-FLT_MAX) get weight 2^-E when their whole row is masked
      // (m = -FLT_MAX; s - m first, so that the exponent is exact), else 0;
      // keys past the end (-inf) always 0
#pragma unroll
      for (int k = 0; k < 8; ++k) d[k] = (sc[k] - m_row) - static_cast<float>(E);
    }
    float w[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float pe = __builtin_amdgcn_exp2f(d[k]);  // p 2^-E
      l_acc += pe;
      w[k] = pe * nv[k];
    }
    // ---- weights to the A operands: tile 0's four tokens, then tile 1's;
    // each pair twice, against the (hi pair, lo pair) k slots of the values
    const uint32_t w01 = pack_f16x2(w[0], w[1]);
    const uint32_t w23 = pack_f16x2(w[2], w[3]);
    const uint32_t x01 = pack_f16x2(w[4], w[5]);
    const uint32_t x23 = pack_f16x2(w[6], w[7]);
    if constexpr (S::SIGNV) {
      // k slots: the lane's 8 tokens (tile 0's four, then tile 1's) against
      // their signs; the weight sums ride along when the codebook's midpoint
      // is not zero
      const u32x4_t A = {w01, w23, x01, x23};
#pragma unroll
      for (int c = 0; c < CPL; ++c)
        O[c] = mfma_f16(A, u32x4_t{vop[c][0].x, vop[c][0].y, vop[c][1].x, vop[c][1].y}, O[c]);
      if (v_mid != 0.f) Lw = mfma_f16(A, u32x4_t{0x3c003c00u, 0x3c003c00u, 0x3c003c00u, 0x3c003c00u}, Lw);
    } else {
      const u32x4_t A0 = {w01, w01, w23, w23};
      const u32x4_t A1 = {x01, x01, x23, x23};
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        O[c] = mfma_f16(A0, u32x4_t{vop[c][0].x, vop[c][0].y, vop[c][1].x, vop[c][1].y}, O[c]);
        O[c] = mfma_f16(A1, u32x4_t{vop[c][2].x, vop[c][2].y, vop[c][3].x, vop[c][3].y}, O[c]);
      }
    }
  };

  // Loads are issued unconditionally (past t_end they read zeros for free),
  // so the count of outstanding loads is exact for every sub-chunk.
  Scores Cn;
  if (n_my > 0) Cn = scores(buf[0]);
  for (int base = 0; base < n_my; base += P) {
#pragma unroll
    for (int s = 0; s < P; ++s) {
      const int i = base + s;
      if (i < n_my) {
        const Scores C = Cn;
        finish(buf[s], C, sub_start(i));
        if (i + 1 < n_my) Cn = scores(buf[(s + 1) % P]);
      }
      load_sub(buf[s], sub_start(i + P));
    }
  }

  // --------------------------------------------------- combine the waves ----
  // l of row n: lanes (g', n) for every g'
  float lr = l_acc + xor_lane<16>(l_acc);
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
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float* dst = s_wo + (wave * NQ + 4 * g + i) * D + CPL * n;
#pragma unroll
    for (int c = 0; c < CPL; ++c) dst[c] = O[c][i];
  }
  if (g == 0) {
    // a wave without tokens keeps m = -inf and contributes nothing
    s_wm[wave * NQ + n] = m_row;
    s_wl[wave * NQ + n] = lr;
    s_we[wave * NQ + n] = ldexpf(1.f, E);  // undoes the 2^-E of l and O
  }
  float* s_wv = reinterpret_cast<float*>(lds + S::WV_OFF);
  if (S::SIGNV && n == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) s_wv[wave * NQ + 4 * g + i] = Lw[i];
  }
  lds_barrier();
  float* s_fo = reinterpret_cast<float*>(lds + S::FO_OFF);
  float* s_fl = reinterpret_cast<float*>(lds + S::FL_OFF);
  if (tid < NQ) {  // per row: the waves' log-sum-exp factors, l and the reference m
    const int r = tid;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, s_wm[w * NQ + r]);
    float lt = 0.f, lv = 0.f;
    // table values carry the factor cbs_v (a power of two: exact); signs v_half
    const float oscale = S::SIGNV ? v_half : __builtin_amdgcn_rcpf(cbs_v);
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float wm = s_wm[w * NQ + r];
      const float f = wm == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(wm - M);
      const float fe = f * s_we[w * NQ + r];
      lt = fmaf(s_wl[w * NQ + r], fe, lt);
      s_wf[w * NQ + r] = fe * oscale;
      if (S::SIGNV) lv = fmaf(s_wv[w * NQ + r], fe, lv);
    }
    s_fl[r] = lt;
    s_fl[NQ + r] = M;
    s_fl[2 * NQ + r] = S::SIGNV ? v_mid * lv : 0.f;
  }
  lds_barrier();
  for (int idx = tid; idx < NQ * D; idx += NT) {
    const int r = idx / D;
    float a = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) a = fmaf(s_wo[(w * NQ) * D + idx], s_wf[w * NQ + r], a);
    s_fo[idx] = S::SIGNV ? a + s_fl[2 * NQ + r] : a;
  }
  lds_barrier();

  if (nvalid > 1) {
    // this split's partial: o[r][:] still in the rotated basis (the merge
    // applies R_V^-1 once per row: attn_merge_rot_kernel for the Hadamard
    // rotation, attn_merge_kernel for the dense one), and (m, l) per row
    // with m in natural-log units
    const int64_t grp = (static_cast<int64_t>(b) * p.Hkv + gk) * p.n_rg + rg;
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
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int r = wave + NW * h;
      if (!rs.valid(r)) continue;  // wave-uniform
      const float lt = s_fl[r];
      const float inv = lt > 0.f ? 1.f / lt : 0.f;
      float y[QE];
#pragma unroll
      for (int e = 0; e < QE; ++e) y[e] = s_fo[r * D + lane + e * kWave] * inv;
      wave_fwht<D>(y, lsg);
      const int64_t qo = rs.qoff(r) * D;
#pragma unroll
      for (int e = 0; e < QE; ++e)
        store_out(p.out, p.q_dtype, qo + lane + e * kWave, y[e] * p.rscale * p.vrot[lane + e * kWave]);
    }
  } else {
    for (int idx = tid; idx < NQ * D; idx += NT) {
      const int r = idx / D;
      const int c = idx % D;
      if (!rs.valid(r)) continue;
      const float lt = s_fl[r];
      const float inv = lt > 0.f ? 1.f / lt : 0.f;
      float a2 = 0.f;  // x_c = sum_k y_k R[k][c]
      for (int k2 = 0; k2 < D; ++k2) a2 = fmaf(s_fo[r * D + k2], p.vrot[static_cast<int64_t>(k2) * D + c], a2);
      store_out(p.out, p.q_dtype, rs.qoff(r) * D + c, a2 * inv);
    }
  }
}

template <int KB, int VB>
int launch_rows16(const AttnParams& p, hipStream_t st) {
  if (p.nq != Rows16Shape<KB, VB>::NQ)
    return fail(TQ_ERR_UNSUPPORTED, "attention: 16-row kernel launched with %d-row groups", p.nq);
  const dim3 grid(p.n_splits, p.Hkv * p.n_rg, p.B);
  hipLaunchKernelGGL((attn_rows16_kernel<KB, VB>), grid, dim3(Rows16Shape<KB, VB>::NT), 0, st, p);
  return check_launch("attn_rows16_kernel");
}

}  // namespace tq
