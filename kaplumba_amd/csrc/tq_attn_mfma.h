// TurboQuant decode / verify attention straight from packed indices, with the
// dot products on gfx950's matrix cores (v_mfma_f32_16x16x32_f16).
//
// Workgroup: 8 wave64s (two per SIMD; 4 for d = 256 with 3- or 4-bit values) own tokens [t_begin, t_end) of one kv
// head of one sequence and up to NQ (4 or 16) query rows of that head's GQA
// group.  Tokens are cut into 32-token sub-chunks; sub-chunk i belongs to wave
// i % 8 (i % 4).  Every wave keeps the global loads of its next P sub-chunks in flight
// in registers and runs an online softmax over its own sub-chunks; the waves
// are combined through LDS at the end and the split is published for the
// cross-workgroup merge.
//
// Lane roles inside a wave (l = lane, n = l % 16, g = l / 16):
//   scores  S[row][tok] = sum_d q_rot[row][d] * c[idx[tok][d]]   (16 x 16 tile)
//     A = query rows, lane (row n, g) holds rotated coordinates
//         g*D/4 .. g*D/4 + D/4 - 1 of row n, eight per MFMA step,
//     B = keys, lane (token n, g) holds the same coordinates of token n: a
//         contiguous bit span of its packed row (96 bits, three words, for
//         d = 128 at 3 bits), so unpacking needs no cross-lane traffic.
//     Both operands are split hi + lo in f16 (x = hi + lo to ~2^-22), and
//     hi*hi + hi*lo + lo*hi gives the f32 dot product to ~2^-21 relative: the
//     scores keep f32 accuracy, as the reference's fp32 arithmetic does.
//     Output: lane (g, token n), register i = row 4g + i.
//   softmax over the 16 lanes of a row (DPP row rotations), per register.
//   values  O[row][d] = sum_tok w[row][tok] * c[idx[tok][d]]     (16 x 16 tiles)
//     A = weights from LDS, lane (row n, g) holds tokens 8g .. 8g+7,
//     B = values, lane (coordinate group n, g) holds tokens 8g .. 8g+7 of
//         coordinate (D/16)*n + c for MFMA c; the two tokens of an f16 pair
//         form one table key (their two fields interleaved with v_bfi).
//     Output: lane (g, n), register i = row 4g + i, coordinate (D/16)*n + c.
// Codebook lookups go through small pair tables in LDS (two coordinates or
// two tokens per entry), replicated so the 16 lanes of a row hit distinct
// banks.  Table entries hold hi + lo f16 parts of the scaled codebook values
// (~22 significant bits): a single f16 would leave a per-entry rounding error
// that every token with that index repeats, i.e. a bias that does not average
// out over the context.  Weights are p * ||v|| scaled by a per-wave power of
// two into [0, 1] and stored in f16 (their rounding is independent per token).
#pragma once

#include "tq_attn_merge.h"

namespace tq {

typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));


__device__ __forceinline__ f32x4_t mfma_f16(u32x4_t a, u32x4_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                 __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

// x rotated by K lanes inside each 16-lane row (DPP row_ror:K).
template <int K>
__device__ __forceinline__ float row_ror(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x120 + K, 0xf, 0xf, true));
}

__device__ __forceinline__ float row16_max(float x) {
  x = fmaxf(x, row_ror<8>(x));
  x = fmaxf(x, row_ror<4>(x));
  x = fmaxf(x, row_ror<2>(x));
  return fmaxf(x, row_ror<1>(x));
}

// row16_max of four values, the reduction steps interleaved (independent
// DPP operations hide each other's hazards).
__device__ __forceinline__ void row16_max4(float (&x)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) x[i] = fmaxf(x[i], row_ror<8>(x[i]));
#pragma unroll
  for (int i = 0; i < 4; ++i) x[i] = fmaxf(x[i], row_ror<4>(x[i]));
#pragma unroll
  for (int i = 0; i < 4; ++i) x[i] = fmaxf(x[i], row_ror<2>(x[i]));
#pragma unroll
  for (int i = 0; i < 4; ++i) x[i] = fmaxf(x[i], row_ror<1>(x[i]));
}

__device__ __forceinline__ float row16_sum(float x) {
  x += row_ror<8>(x);
  x += row_ror<4>(x);
  x += row_ror<2>(x);
  return x + row_ror<1>(x);
}

// Orders this wave's LDS accesses across lanes: LDS operations of one wave
// execute in program order, so only the compiler must not move them.
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

__device__ __forceinline__ uint32_t f16_bits(float x) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(x));
}

// hi + lo split of x in f16: hi = f16(x), lo = f16(x - hi).
__device__ __forceinline__ void split_f16(float x, uint32_t& hi, uint32_t& lo) {
  const _Float16 h = static_cast<_Float16>(x);
  hi = __builtin_bit_cast(uint16_t, h);
  lo = f16_bits(x - static_cast<float>(h));
}

// 2^(13 - e) for max |x| = f * 2^e, f in [0.5, 1): scales the largest
// magnitude into [2^12, 2^13), far from f16 overflow and with the lo parts
// of a hi/lo split still normal numbers.
__device__ __forceinline__ float f16_split_scale(float maxabs) {
  if (!(maxabs > 0.f) || !(maxabs < INFINITY)) return 1.f;
  int e;
  frexpf(maxabs, &e);
  return ldexpf(1.f, 13 - e);
}

template <int D, int KB, int VB, int NQ>
struct MfmaShape {
  // d = 256 runs one wave per SIMD (512 registers each), smaller heads two
  // two waves per SIMD; d = 256 with 3- and 4-bit values one (their value
  // words and tables do not fit 256 registers per wave)
  static constexpr int NW = (D >= 256 && VB >= 3) ? 4 : 8;
  static constexpr int NT = NW * kWave;
  static constexpr int SUB = 32;  // tokens per sub-chunk
  static constexpr int P = 2;     // sub-chunks in flight per wave
  // scores
  static constexpr int KSPAN = D / 4;  // coordinates of one token per lane
  static constexpr int KPP = KSPAN / 4;  // 4-coordinate groups per lane span (MFMA pairs)
  static constexpr int KBITS = KSPAN * KB;
  static constexpr bool KALIGNED = KBITS % 32 == 0;
  static constexpr int KAL = (KBITS + 31) / 32;
  static constexpr int KRAW = KALIGNED ? KAL : KAL + 1;
  static constexpr int PWK = D * KB / 32;
  static constexpr int KKEYS = 1 << (2 * KB);
  static constexpr int REPK = KKEYS <= 64 ? 64 : 8;  // replicas: one per lane when they fit
  // values
  static constexpr int CPL = D / 16;  // coordinates per lane
  static constexpr int SEGMAX = VB == 3 ? 8 : 32 / VB;
  static constexpr int SEGC = SEGMAX < CPL ? SEGMAX : CPL;  // coordinates per 32-bit segment
  static constexpr int NSEG = CPL / SEGC;
  static constexpr int SEGBITS = SEGC * VB;
  static constexpr int VRAW = VB == 3 ? 2 : 1;  // a 3-bit segment can cross a word
  static constexpr int PWV = D * VB / 32;
  static constexpr int VKEYS = 1 << (2 * VB);
  static constexpr int REPV = VKEYS <= 64 ? 64 : 16;  // (hi pair, lo pair) entries, like keys
  // LDS layout (bytes)
  // Pair tables sit on aligned blocks: an entry's byte address is
  // base | key << LOG_STRIDE with the key bits clear in base (replica
  // offset of the lane + block start).
  static constexpr int LOGSK = REPK == 64 ? 9 : 6;  // log2(REPK * 8): (hi pair, lo pair) entries
  static constexpr int LOGSV = REPV == 64 ? 9 : 7;  // log2(REPV * 8): (hi pair, lo pair) entries
  static constexpr int LUTK_BYTES = KKEYS * REPK * 8;
  static constexpr int LUTV_BYTES = VKEYS * REPV * 8;
  static constexpr int pow2ceil(int x) { return x <= 1 ? 1 : 2 * pow2ceil((x + 1) / 2); }
  static constexpr int BK = pow2ceil(LUTK_BYTES);  // table blocks: power-of-two sizes,
  static constexpr int BV = pow2ceil(LUTV_BYTES);  // each aligned to its size
  static constexpr int LUTK_OFF = BK >= BV ? 0 : BV;
  static constexpr int LUTV_OFF = BK >= BV ? BK : 0;
  static constexpr int QSTRIDE = D + 4;   // padded rows: the 16 rows read apart land on distinct banks
  static constexpr int Q_OFF = BK + BV;   // [NQ][QSTRIDE] f32 rotated queries
  static constexpr int QS_OFF = Q_OFF + NQ * QSTRIDE * 4;  // [NQ] f32 max |q_rot| per row
  static constexpr int W_OFF = QS_OFF + 64;                // [NW][16][32] f16 weights
  // 4-row groups: the query A operands of every MFMA step, [KPP][64 lanes]
  // x 16 B, shared by the waves (their rows are the same)
  static constexpr bool QLDS = 2 * NQ <= 16;
  static constexpr int QOP_OFF = W_OFF + NW * 16 * SUB * 2;
  static constexpr int LOOP_BYTES = QOP_OFF + (QLDS ? KPP * kWave * 16 : 0);
  // after the token loop the buffers above are dead: the epilogue's buffers
  // start again at 0 (a barrier separates the two phases)
  static constexpr int CO_OFF = 0;                          // [NW][NQ][D] f32 wave outputs
  static constexpr int CM_OFF = CO_OFF + NW * NQ * D * 4;
  static constexpr int CL_OFF = CM_OFF + NW * NQ * 4;
  static constexpr int O_OFF = CL_OFF + NW * NQ * 4;  // [NQ][D] combined rows
  static constexpr int ML_OFF = O_OFF + NQ * D * 4;   // [NQ][2]
  static constexpr int AUX_OFF = ML_OFF + (NQ * 8 + 15) / 16 * 16;  // [NQ + D] f32 finalize scratch
  static constexpr int POST_BYTES = AUX_OFF + (NQ + D) * 4;
  static_assert(O_OFF % 16 == 0, "combined rows are read as float4");
  static constexpr int BYTES = LOOP_BYTES > POST_BYTES ? LOOP_BYTES : POST_BYTES;
  static constexpr int RPW = (NQ + NW - 1) / NW;  // query rows rotated per wave
  static constexpr int QPL = D / kWave;           // query elements per lane and row
  static_assert(D % 64 == 0, "head dim");
  static_assert(CPL % SEGC == 0, "value segments");
  static_assert(LUTK_BYTES <= 32768 && LUTV_BYTES <= 32768, "pair table blocks");
  static_assert(BYTES <= 160 * 1024, "LDS per workgroup");
};

// LDS barrier that orders only LDS traffic: unlike __syncthreads it does not
// wait for outstanding global loads, so the prefetched sub-chunks stay in
// flight across it.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

template <typename T>
__device__ __forceinline__ T lds_at(const unsigned char* lds, uint32_t byte_off) {
  return *reinterpret_cast<const T*>(lds + byte_off);
}

// Byte address base | key << LOGS of the pair-table entry for the NB-bit key
// at constant bit position pos of a word array: one shift (or alignbit across
// a word boundary) and one and-or.  base must have the key bits clear.
// mask = ((1 << NB) - 1) << LOGS, kept in an SGPR (v_and_or_b32 takes no
// literal operand).
template <int NB, int LOGS, int NW>
__device__ __forceinline__ uint32_t key_addr(const uint32_t (&w)[NW], int pos, uint32_t base,
                                             uint32_t mask) {
  const int wi = pos >> 5;
  const int sh = pos & 31;
  uint32_t x;
  if (sh + NB <= 32)
    x = sh >= LOGS ? (w[wi] >> (sh - LOGS)) : (w[wi] << (LOGS - sh));
  else  // sh > 32 - NB >= LOGS
    x = __builtin_amdgcn_alignbit(w[wi + 1], w[wi], sh - LOGS);
  return (x & mask) | base;
}

// The value unchanged, but opaque to the optimiser (keeps two table reads
// that differ by a constant from being fused into one two-register read).
__device__ __forceinline__ uint32_t opaque(uint32_t x) {
  asm volatile("" : "+v"(x));
  return x;
}

constexpr uint32_t kBufferFlags = 0x00020000;  // raw buffer, 32-bit data format

// N consecutive dwords at byte offset off of a buffer, in as few loads as the
// 4-dword maximum allows.
template <int N>
__device__ __forceinline__ void load_words(uint32_t (&w)[N], __amdgpu_buffer_rsrc_t r, uint32_t off) {
  int i = 0;
#pragma unroll
  for (; i + 4 <= N; i += 4) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off + i * 4, 0, 0);
    w[i] = v[0];
    w[i + 1] = v[1];
    w[i + 2] = v[2];
    w[i + 3] = v[3];
  }
  if constexpr (N % 4 == 3) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b96(r, off + i * 4, 0, 0);
    w[i] = v[0];
    w[i + 1] = v[1];
    w[i + 2] = v[2];
  } else if constexpr (N % 4 == 2) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, off + i * 4, 0, 0);
    w[i] = v[0];
    w[i + 1] = v[1];
  } else if constexpr (N % 4 == 1) {
    w[i] = __builtin_amdgcn_raw_buffer_load_b32(r, off + i * 4, 0, 0);
  }
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, kBufferFlags);
}

template <int D, int KB, int VB, int NQ>
// block size: MfmaShape<D, KB, VB, NQ>::NT
__global__ __launch_bounds__((MfmaShape<D, KB, VB, NQ>::NT), 1) void attn_mfma_kernel(AttnParams p) {
  using S = MfmaShape<D, KB, VB, NQ>;
  constexpr int NW = S::NW;
  constexpr int NT = S::NT;
  constexpr int SUB = S::SUB;
  constexpr int P = S::P;
  constexpr int KPP = S::KPP;
  constexpr int KRAW = S::KRAW;
  constexpr int KAL = S::KAL;
  constexpr int PWK = S::PWK;
  constexpr int CPL = S::CPL;
  constexpr int SEGC = S::SEGC;
  constexpr int NSEG = S::NSEG;
  constexpr int VRAW = S::VRAW;
  constexpr int PWV = S::PWV;
  constexpr int REPK = S::REPK;
  constexpr int REPV = S::REPV;
  constexpr int RPW = S::RPW;
  constexpr int QPL = S::QPL;

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
  // (the kernel's only LDS object: it starts at address 0, so the 4 KiB-aligned
  // table offsets are absolute addresses and fold into the instructions)

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
    // No tokens for this split.  An empty sequence still needs its output:
    // split 0 writes zeros (the reference divides a zero sum by 1e-6).
    if (Tb <= 0 && split == 0)
      for (int idx = tid; idx < NQ * D; idx += NT)
        if (rs.valid(idx / D)) store_out(p.out, p.q_dtype, rs.qoff(idx / D) * D + idx % D, 0.f);
    return;  // the whole workgroup leaves together
  }
  // Token indices relative to the sequence start, and byte offsets inside
  // one (sequence, kv head) row of the cache, fit in 32 bits (host check).
  const int t_begin = static_cast<int>(t_begin64);
  const int t_end = static_cast<int>(Tb < t_begin64 + p.chunk ? Tb : t_begin64 + p.chunk);
  const int nvalid = static_cast<int>((Tb + p.chunk - 1) / p.chunk);
  const bool dense = p.rot_kind == TQ_ROT_DENSE;
  const bool nf16 = p.norm_dtype == TQ_DTYPE_F16;
  // Buffer resources over tokens [0, t_end) of this (sequence, kv head) row:
  // tokens at or past t_end read as zeros without touching memory, so the
  // last sub-chunk needs no clamping and prefetches past the end are free.
  const int64_t kvrow0 = (static_cast<int64_t>(b) * p.Hkv + gk) * p.cap + win.start;
  const uint32_t tn = static_cast<uint32_t>(t_end);
  const uint32_t nb = nf16 ? 2u : 4u;
  const auto krs = buffer_rsrc(static_cast<const char*>(p.k) + kvrow0 * (PWK * 4), tn * (PWK * 4));
  const auto vrs = buffer_rsrc(static_cast<const char*>(p.v) + kvrow0 * (PWV * 4), tn * (PWV * 4));
  const auto knrs = buffer_rsrc(static_cast<const char*>(p.kn) + kvrow0 * nb, tn * nb);
  const auto vnrs = buffer_rsrc(static_cast<const char*>(p.vn) + kvrow0 * nb, tn * nb);

  // ---- per-lane constants
  const int ksh = (g * S::KBITS) & 31;  // bit offset of this lane's key span in its first word
  const uint32_t k_lane = n * (PWK * 4) + ((g * S::KBITS) >> 5) * 4;  // byte offsets from the
  const uint32_t n_lane = n * nb;                                     // sub-chunk's first token
  uint32_t v_lane[NSEG];  // value segment byte offsets and shifts of coordinate group n
  int vsh[NSEG];
#pragma unroll
  for (int k = 0; k < NSEG; ++k) {
    const int bit = (CPL * n + k * SEGC) * VB;
    v_lane[k] = 8 * g * (PWV * 4) + (bit >> 5) * 4;
    vsh[k] = bit & 31;
  }
  const uint32_t lutk_lane = S::LUTK_OFF + (lane % REPK) * 8;  // byte address of the lane's replica
  const uint32_t lutv_lane = S::LUTV_OFF + (lane % REPV) * 8;
  uint32_t kmask = (S::KKEYS - 1u) << S::LOGSK;  // table key masks in SGPRs
  uint32_t vmask = (S::VKEYS - 1u) << S::LOGSV;
  asm volatile("" : "+s"(kmask), "+s"(vmask));

  // ---- this wave's sub-chunks: i = 0 .. n_my-1 start at t_begin + (NW*i + wave) * 32
  const int n_tok = t_end - t_begin;
  const int n_my = n_tok > wave * SUB ? (n_tok - wave * SUB + NW * SUB - 1) / (NW * SUB) : 0;
  auto sub_start = [&](int i) -> int { return t_begin + (i * NW + wave) * SUB; };

  struct Buf {
    uint32_t k[2][KRAW];        // key words: token n of the two 16-token tiles
    uint32_t nk[2], nv[2];      // their norms (raw f32 or f16 bits)
    uint32_t v[8][NSEG][VRAW];  // value words: tokens 8g .. 8g+7
  };
  auto load_norm_raw = [&](__amdgpu_buffer_rsrc_t rs_, uint32_t off) -> uint32_t {
    if (nf16) return __builtin_amdgcn_raw_buffer_load_b16(rs_, off, 0, 0);
    return __builtin_amdgcn_raw_buffer_load_b32(rs_, off, 0, 0);
  };
  auto norm_of = [&](uint32_t raw) -> float {
    return nf16 ? f16_bits_to_f32(static_cast<uint16_t>(raw)) : __builtin_bit_cast(float, raw);
  };
  // A lane's words are consecutive dwords (fused into one multi-dword load).
  // A trailing word past its span may belong to the next token's row or lie
  // past t_end (buffer range checks are per dword: it reads zero); its bits
  // are never used.
  // The key words feed scores(), the norms and value words finish(); the
  // two halves of a buffer are refilled separately (see the loop).
  auto load_keys = [&](Buf& bf, int s0) {
    const uint32_t ko = static_cast<uint32_t>(s0) * (PWK * 4) + k_lane;
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) load_words<KRAW>(bf.k[tt], krs, ko + tt * 16 * PWK * 4);
  };
  auto load_rest = [&](Buf& bf, int s0) {
    const uint32_t t0 = static_cast<uint32_t>(s0);
    const uint32_t no = t0 * nb + n_lane;
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      bf.nk[tt] = load_norm_raw(knrs, no + tt * 16 * nb);
      bf.nv[tt] = load_norm_raw(vnrs, no + tt * 16 * nb);
    }
    const uint32_t vo = t0 * (PWV * 4);
#pragma unroll
    for (int e = 0; e < 8; ++e)
#pragma unroll
      for (int k = 0; k < NSEG; ++k)
        load_words<VRAW>(bf.v[e][k], vrs, vo + v_lane[k] + e * PWV * 4);
  };
  auto load_sub = [&](Buf& bf, int s0) {
    load_keys(bf, s0);
    load_rest(bf, s0);
  };

  // ---- prologue loads first (the query elements of this wave's rows, key
  // signs, codebooks), then the pipeline's first sub-chunks: loads complete
  // in order, so the prologue's operands arrive before the bulk data
  // (raw bits: the conversions come later, so no load is waited for here)
  uint32_t qraw[RPW][QPL];
  float sgn[QPL], vsg[QPL];  // R_K and R_V sign vectors at d = lane + 64e
  const bool q32 = dense || p.q_dtype == TQ_DTYPE_F32;
#pragma unroll
  for (int rr = 0; rr < RPW; ++rr) {
    const int r = wave + rr * NW;
    const bool ok = r < NQ && rs.valid(r);
    const int64_t qb = !ok ? 0
                       : dense ? rs.qoff(r) * D
                               : b * p.q_sb + static_cast<int64_t>(rs.head(r)) * p.q_sh +
                                     static_cast<int64_t>(rs.lpos(r)) * p.q_sl;
    const void* qsrc = dense ? static_cast<const void*>(p.qrot) : p.q;
#pragma unroll
    for (int e = 0; e < QPL; ++e) {
      const int64_t i = qb + lane + e * kWave;
      if (!ok)
        qraw[rr][e] = 0u;
      else if (q32)
        qraw[rr][e] = static_cast<const uint32_t*>(qsrc)[i];
      else
        qraw[rr][e] = static_cast<const uint16_t*>(qsrc)[i];
    }
  }
#pragma unroll
  for (int e = 0; e < QPL; ++e) {
    sgn[e] = dense ? 1.f : p.krot[lane + e * kWave];
    vsg[e] = dense ? 1.f : p.vrot[lane + e * kWave];
  }
  float ckb[1 << KB], cvb[1 << VB];  // codebooks (uniform loads)
#pragma unroll
  for (int i = 0; i < (1 << KB); ++i) ckb[i] = p.kcb[i];
#pragma unroll
  for (int i = 0; i < (1 << VB); ++i) cvb[i] = p.vcb[i];

  // only the first sub-chunk before the prologue: its transfer overlaps the
  // prologue's work (the rest is issued after it, ahead of the loop)
  Buf buf[P];
  load_sub(buf[0], sub_start(0));

  // ------------------------------------------------------------ prologue ----
  float kmax = 0.f, vmax = 0.f;
#pragma unroll
  for (int i = 0; i < (1 << KB); ++i) kmax = fmaxf(kmax, fabsf(ckb[i]));
#pragma unroll
  for (int i = 0; i < (1 << VB); ++i) vmax = fmaxf(vmax, fabsf(cvb[i]));

  // query rows: wave w rotates rows w, w + NW, ... in its own LDS rows
  //   q_s = round_qdtype(q * scale_q) * s_K, Hadamard butterflies, * 1/sqrt(D)
  //   (dense: the rows were rotated by qprep_kernel), then the hi/lo scale.
#pragma unroll
  for (int rr = 0; rr < RPW; ++rr) {
    const int r = wave + rr * NW;
    if (r >= NQ) break;
    float* y = s_q + r * S::QSTRIDE;
#pragma unroll
    for (int e = 0; e < QPL; ++e) {
      const uint32_t raw = qraw[rr][e];
      const float qv = q32 ? __builtin_bit_cast(float, raw)
                           : (p.q_dtype == TQ_DTYPE_F16 ? f16_bits_to_f32(static_cast<uint16_t>(raw))
                                                        : bf16_bits_to_f32(static_cast<uint16_t>(raw)));
      y[lane + e * kWave] = dense ? qv : round_q(p.q_dtype, qv * p.scale_q) * sgn[e];
    }
    if (!dense) {
      wave_sync();
#pragma unroll
      for (int st = 0; (1 << st) < D; ++st) {
        const int hs = 1 << st;
#pragma unroll
        for (int k0 = 0; k0 < D / 2; k0 += kWave) {
          const int k = k0 + lane;
          if (k < D / 2) {
            const int i0 = ((k >> st) << (st + 1)) + (k & (hs - 1));
            const float a = y[i0];
            const float c = y[i0 + hs];
            y[i0] = a + c;
            y[i0 + hs] = a - c;
          }
        }
        wave_sync();
      }
    }
    const float ysc = dense ? 1.f : p.rscale;
    float m = 0.f;
#pragma unroll
    for (int e = 0; e < QPL; ++e) {
      const float v = y[lane + e * kWave] * ysc;
      y[lane + e * kWave] = v;
      m = fmaxf(m, fabsf(v));
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, kWave));
    if (lane == 0) s_qs[r] = m;
  }
  lds_barrier();

  // pair tables: keys and values as (hi pair, lo pair) f16 at power-of-two
  // scales, so an entry carries ~22 significant bits (a single f16 would leave
  // a per-entry rounding error that every token with that index repeats, i.e.
  // a bias that does not average out over the context)
  const float sk = f16_split_scale(kmax);
  const float cbs_v = f16_split_scale(vmax);
  {
    // Thread t computes the entry of key t % K once (K = min(KEYS, NT);
    // keys t, t + NT, ... when there are more keys than threads) and stores
    // it in the replicas (s + key) % REP for its slots s = t / K, t / K + NT / K,
    // ...: rotating the replica by the key keeps the lanes of one store on
    // distinct banks (key-major addresses alone would put them all on one).
    constexpr int KK = S::KKEYS < NT ? S::KKEYS : NT;
    constexpr int VK = S::VKEYS < NT ? S::VKEYS : NT;
    static_assert(NT % KK == 0 && NT % VK == 0, "table build mapping");
    uint2* lk = reinterpret_cast<uint2*>(lds + S::LUTK_OFF);
    for (int key = tid % KK; key < S::KKEYS; key += KK) {
      uint32_t h0, l0, h1, l1;
      split_f16(ckb[key & ((1 << KB) - 1)] * sk, h0, l0);
      split_f16(ckb[key >> KB] * sk, h1, l1);
      const uint2 ent = make_uint2(h0 | (h1 << 16), l0 | (l1 << 16));
      for (int sl = tid / KK; sl < REPK; sl += NT / KK)
        lk[key * REPK + (sl + key) % REPK] = ent;
    }
    uint2* lv = reinterpret_cast<uint2*>(lds + S::LUTV_OFF);
    for (int key = tid % VK; key < S::VKEYS; key += VK) {
      uint32_t h0, l0, h1, l1;
      split_f16(cvb[key & ((1 << VB) - 1)] * cbs_v, h0, l0);
      split_f16(cvb[key >> VB] * cbs_v, h1, l1);
      const uint2 ent = make_uint2(h0 | (h1 << 16), l0 | (l1 << 16));
      for (int sl = tid / VK; sl < REPV; sl += NT / VK)
        lv[key * REPV + (sl + key) % REPV] = ent;
    }
  }

  // query operands, one hi/lo scale s_Q for all rows (a row far below the
  // largest keeps full precision: its hi and lo parts stay normal f16).
  // Lane (row n, g) holds coordinates g*D/4 + c; MFMA j covers the pairs
  // p = 2j, 2j + 1 as [hi p, hi p, hi p+1, hi p+1] x [kh p, kl p, kh p+1, kl p+1]
  // (and the same with the lo parts), i.e. (q_hi + q_lo) . (k_hi + k_lo).
  float qmax = 0.f;
#pragma unroll
  for (int r = 0; r < NQ; ++r) qmax = fmaxf(qmax, s_qs[r]);
  const float sq = f16_split_scale(qmax);
  // With 4-row groups the hi and lo pieces share one operand: A rows 0..3
  // hold the rows' hi parts, rows 4..7 their lo parts (rows 8..15 zero), so
  // one MFMA per k step gives both products and a lane exchange adds them
  // (PIECE_ROWS); 16-row groups keep a second operand for the lo parts.
  constexpr bool PIECE_ROWS = S::QLDS;
  u32x4_t qa[PIECE_ROWS ? 1 : KPP], qb[PIECE_ROWS ? 1 : KPP];
  {
    // rows past the group read row 0 and scale it by zero (no per-lane branches)
    const int qrow = PIECE_ROWS ? (n < NQ ? n : n - NQ) : n;
    const bool qok = PIECE_ROWS ? n < 2 * NQ : n < NQ;
    const bool lo_row = PIECE_ROWS && n >= NQ;
    const float qsl = qok ? sq : 0.f;
    const float* y = s_q + (qok ? qrow : 0) * S::QSTRIDE + g * S::KSPAN;
#pragma unroll
    for (int j = 0; j < KPP; ++j)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        uint32_t h0, l0, h1, l1;
        split_f16(y[4 * j + 2 * h] * qsl, h0, l0);
        split_f16(y[4 * j + 2 * h + 1] * qsl, h1, l1);
        const uint32_t hp = h0 | (h1 << 16), lp = l0 | (l1 << 16);
        if constexpr (PIECE_ROWS) {
          // every wave forms the same operands: wave 0 stores them
          if (wave == 0) {
            uint32_t* qo = reinterpret_cast<uint32_t*>(lds + S::QOP_OFF + (j * kWave + lane) * 16);
            qo[2 * h] = qo[2 * h + 1] = lo_row ? lp : hp;
          }
        } else {
          qa[j][2 * h] = qa[j][2 * h + 1] = hp;
          qb[j][2 * h] = qb[j][2 * h + 1] = lp;
        }
      }
  }
  // scores in log2 units: S * ||k|| * log2(e) / (s_K s_Q); per register i
  // (row 4g + i) the causal limit (keys t <= lim are visible)
  const float qk_inv = 1.4426950408889634f / (sk * sq);
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
  lds_barrier();
#pragma unroll
  for (int s = 1; s < P; ++s) load_sub(buf[s], sub_start(s));

  // ------------------------------------------------------------ streaming ----
  float m_run[4], l_run[4];
  f32x4_t O[CPL];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    m_run[i] = -INFINITY;
    l_run[i] = 0.f;
  }
#pragma unroll
  for (int c = 0; c < CPL; ++c) O[c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  int E = -1000;    // value-norm exponent of this wave: w = p * ||v|| * 2^-E
  float vsc = 0.f;  // 2^-E
  uint16_t* w_mine = s_w + wave * 16 * SUB;

  // Software pipeline: the scores of sub-chunk i + 1 are computed right after
  // the value pass of sub-chunk i, in one region without fences, so their
  // table lookups and matrix operations interleave (each alone is a long
  // dependency chain).
  //   scores(bf, Sc): raw q.k of the sub-chunk's two 16-token tiles
  //   finish(bf, Sc, s0): scale and mask, online softmax, weights, values
  auto scores = [&](const Buf& bf, f32x4_t (&Sc)[2]) {
    // four independent accumulator chains (tile x {q hi, q lo})
    uint32_t al[2][KAL];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int i = 0; i < KAL; ++i)
        al[tt][i] = S::KALIGNED ? bf.k[tt][i] : __builtin_amdgcn_alignbit(bf.k[tt][i + 1], bf.k[tt][i], ksh);
    f32x4_t Sa[2], Sb[2];  // (Sb: 16-row groups only)
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) Sa[tt] = Sb[tt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < KPP; ++j) {
      u32x4_t bk[2];
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint2 v = lds_at<uint2>(lds, key_addr<2 * KB, S::LOGSK>(al[tt], (4 * j + 2 * h) * KB, lutk_lane, kmask));
          bk[tt][2 * h] = v.x;
          bk[tt][2 * h + 1] = v.y;
        }
      u32x4_t aj;
      if constexpr (PIECE_ROWS)
        aj = lds_at<u32x4_t>(lds, S::QOP_OFF + (j * kWave + lane) * 16);
      else
        aj = qa[j];
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        Sa[tt] = mfma_f16(aj, bk[tt], Sa[tt]);
        if constexpr (!PIECE_ROWS) Sb[tt] = mfma_f16(qb[j], bk[tt], Sb[tt]);
      }
    }
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      if constexpr (PIECE_ROWS) {
        // lane (g, token n) register i is A row 4 g + i: lanes of group 0
        // hold the hi products of rows 0..3, group 1 the lo products; lanes
        // n and n + 16 swap and add (groups 0 and 1 then both hold the rows'
        // scores, groups 2 and 3 zeros, as the rows past the group did)
#pragma unroll
        for (int i = 0; i < 4; ++i) Sc[tt][i] = Sa[tt][i] + xor_lane<16>(Sa[tt][i]);
      } else {
        Sc[tt] = Sa[tt] + Sb[tt];
      }
    }
  };
  auto finish = [&](const Buf& bf, const f32x4_t (&Sc)[2], int s0) {
    float sv[2][4];  // scores in log2 units
    float nvt[2];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const float nk = norm_of(bf.nk[tt]);
      nvt[tt] = norm_of(bf.nv[tt]);
      const float f = nk * qk_inv;
#pragma unroll
      for (int i = 0; i < 4; ++i) sv[tt][i] = Sc[tt][i] * f;
    }
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
    // ---- online softmax, rows 4g + i over the 16 lanes of the row.  Lazy
    // reference max: m_run moves only when a row's sub-chunk max exceeds it
    // by more than kLazy (log2 units), so exponents stay <= 2^kLazy and the
    // accumulators are rescaled rarely (a wave-uniform branch).
    constexpr float kLazy = 8.f;
    float cmx[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) cmx[i] = fmaxf(sv[0][i], sv[1][i]);
    row16_max4(cmx);
    const float nv0 = nvt[0];
    const float nv1 = nvt[1];
    int enew;
    frexpf(row16_max(fmaxf(nv0, nv1)), &enew);  // wave-uniform value-norm exponent
    bool move = enew > E;
#pragma unroll
    for (int i = 0; i < 4; ++i) move |= cmx[i] > m_run[i] + kLazy;
    if (__any(move ? 1 : 0)) {
      float alpha[4];
      const int e2 = enew > E ? enew : E;
      const float f = ldexpf(1.f, E - e2);  // exact power of two (0 on the first sub-chunk)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float mn = cmx[i] > m_run[i] + kLazy ? fmaxf(m_run[i], cmx[i]) : m_run[i];
        alpha[i] = __builtin_amdgcn_exp2f(m_run[i] - mn);  // exp2(-inf) = 0 on the first sub-chunk
        l_run[i] *= alpha[i];
        alpha[i] *= f;
        m_run[i] = mn;
      }
      E = e2;
      vsc = ldexpf(1.f, -E);
#pragma unroll
      for (int c = 0; c < CPL; ++c)
#pragma unroll
        for (int i = 0; i < 4; ++i) O[c][i] *= alpha[i];
    }
    float pw[2][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      pw[0][i] = __builtin_amdgcn_exp2f(sv[0][i] - m_run[i]);
      pw[1][i] = __builtin_amdgcn_exp2f(sv[1][i] - m_run[i]);
      l_run[i] += pw[0][i] + pw[1][i];
    }
    // ---- weights to LDS: [row][token] f16 (after the previous sub-chunk's
    // reads of the weight buffer)
    wave_sync();
    if (4 * g < NQ) {
      const float f0 = nv0 * vsc;
      const float f1 = nv1 * vsc;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        w_mine[(4 * g + i) * SUB + n] = static_cast<uint16_t>(f16_bits(pw[0][i] * f0));
        w_mine[(4 * g + i) * SUB + 16 + n] = static_cast<uint16_t>(f16_bits(pw[1][i] * f1));
      }
    }
    wave_sync();
    const u32x4_t A = *reinterpret_cast<const u32x4_t*>(w_mine + n * SUB + 8 * g);
    // value products run hi/lo in the k dimension: k-slots
    // [a hi, b hi, a lo, b lo, c hi, d hi, c lo, d lo] against weights
    // [w_a, w_b, w_a, w_b, w_c, w_d, w_c, w_d], so one 8-byte table read (the
    // hi pair and the lo pair of two tokens) fills half a B operand in place
    const u32x4_t A0 = {A[0], A[0], A[1], A[1]};
    const u32x4_t A1 = {A[2], A[2], A[3], A[3]};
    // ---- values: interleave the two tokens of each pair, one key per coordinate
    constexpr uint32_t MEVEN = [] {
      uint32_t m = 0;
      for (int j = 0; j < SEGC; j += 2) m |= ((1u << VB) - 1u) << (j * VB);
      return m;
    }();
    uint32_t zl[4][NSEG], zh[4][NSEG];
#pragma unroll
    for (int e2 = 0; e2 < 4; ++e2)
#pragma unroll
      for (int k = 0; k < NSEG; ++k) {
        uint32_t xa, xb;
        if constexpr (VRAW == 2) {
          xa = __builtin_amdgcn_alignbit(bf.v[2 * e2][k][1], bf.v[2 * e2][k][0], vsh[k]);
          xb = __builtin_amdgcn_alignbit(bf.v[2 * e2 + 1][k][1], bf.v[2 * e2 + 1][k][0], vsh[k]);
        } else if constexpr (S::SEGBITS % 32 != 0) {
          xa = bf.v[2 * e2][k][0] >> vsh[k];
          xb = bf.v[2 * e2 + 1][k][0] >> vsh[k];
        } else {
          xa = bf.v[2 * e2][k][0];
          xb = bf.v[2 * e2 + 1][k][0];
        }
        zl[e2][k] = (xa & MEVEN) | ((xb << VB) & ~MEVEN);
        zh[e2][k] = ((xa >> VB) & MEVEN) | (xb & ~MEVEN);
      }
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int k = c / SEGC;
      const int cc = c % SEGC;
      uint2 v[4];
#pragma unroll
      for (int e2 = 0; e2 < 4; ++e2) {
        const uint32_t z[1] = {(cc & 1) ? zh[e2][k] : zl[e2][k]};
        v[e2] = lds_at<uint2>(lds, key_addr<2 * VB, S::LOGSV>(z, (cc >> 1) * 2 * VB, lutv_lane, vmask));
      }
      O[c] = mfma_f16(A0, u32x4_t{v[0].x, v[0].y, v[1].x, v[1].y}, O[c]);
      O[c] = mfma_f16(A1, u32x4_t{v[2].x, v[2].y, v[3].x, v[3].y}, O[c]);
    }
  };

  // Prefetches are issued unconditionally (past the end they are free), so
  // the compiler's count of outstanding loads is exact and each sub-chunk
  // waits for its own loads only.
  // Buffer s % P holds sub-chunk s.  A buffer's key words are refilled as
  // soon as scores() has read them (sub-chunk i + 1 + P right after the
  // scores of i + 1), its norms and value words after finish(): the key
  // loads are in flight for about two steps, not only during one finish().
  f32x4_t Sc[2];
  if (n_my > 0) scores(buf[0], Sc);
  load_keys(buf[0], sub_start(P));
  for (int base = 0; base < n_my; base += P) {
#pragma unroll
    for (int s = 0; s < P; ++s) {
      const int i = base + s;
      if (i < n_my) {
        finish(buf[s], Sc, sub_start(i));
        if (i + 1 < n_my) scores(buf[(s + 1) % P], Sc);
      }
      load_rest(buf[s], sub_start(i + P));
      load_keys(buf[(s + 1) % P], sub_start(i + 1 + P));
    }
  }

  // --------------------------------------------------- combine the waves ----
  lds_barrier();  // every wave is done with the tables, queries and weights
  const float oscale = ldexpf(1.f, E) / cbs_v;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float l = row16_sum(l_run[i]);
    const int r = 4 * g + i;
    if (r < NQ) {
      if (n == 0) {
        s_cm[wave * NQ + r] = m_run[i];
        s_cl[wave * NQ + r] = l;
      }
      float* dst = s_co + (wave * NQ + r) * D + CPL * n;
#pragma unroll
      for (int c = 0; c < CPL; ++c) dst[c] = O[c][i] * oscale;
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
  // Hadamard: apply R_V^-1 = diag(s_V) H / sqrt(D) to this split's rows now,
  // in parallel across all workgroups (it commutes with the merge's weighted
  // sum and normalisation), so the final merge only adds and stores.
  if (!dense) {
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr) {
      const int r = wave + rr * NW;
      if (r >= NQ) break;
      float* y = s_o + r * D;
#pragma unroll
      for (int st = 0; (1 << st) < D; ++st) {
        const int hs = 1 << st;
#pragma unroll
        for (int k0 = 0; k0 < D / 2; k0 += kWave) {
          const int k = k0 + lane;
          if (k < D / 2) {
            const int i0 = ((k >> st) << (st + 1)) + (k & (hs - 1));
            const float a = y[i0];
            const float c = y[i0 + hs];
            y[i0] = a + c;
            y[i0 + hs] = a - c;
          }
        }
        wave_sync();
      }
#pragma unroll
      for (int e = 0; e < QPL; ++e) y[lane + e * kWave] *= p.rscale * vsg[e];
    }
    lds_barrier();
  }
  if (nvalid == 1) {  // the only split: finish here (plain = no rotation left for Hadamard)
    if (tid < NQ) s_aux[tid] = s_ml[2 * tid + 1];
    lds_barrier();
    finalize_rows<D, NQ, NT>(p, rs, s_o, s_aux, s_aux + NQ, s_co, !dense, dense);  // s_co is dead
    return;
  }
  // the split's partial, merged by attn_merge_kernel after this kernel
  const int64_t grp = (static_cast<int64_t>(b) * p.Hkv + gk) * p.n_rg + rg;
  float4* po4 = reinterpret_cast<float4*>(p.po + (grp * p.n_splits + split) * static_cast<int64_t>(NQ) * D);
  for (int idx = tid; idx < NQ * D / 4; idx += NT) po4[idx] = reinterpret_cast<const float4*>(s_o)[idx];
  if (tid < 2 * NQ) p.pml[(grp * p.n_splits + split) * static_cast<int64_t>(NQ) * 2 + tid] = s_ml[tid];
}

template <int D, int KB, int VB>
int launch_mfma_nq(const AttnParams& p, hipStream_t st) {
  const dim3 grid(p.n_splits, p.Hkv * p.n_rg, p.B);
  if (p.nq == 4) {
    using S4 = MfmaShape<D, KB, VB, 4>;
    hipLaunchKernelGGL((attn_mfma_kernel<D, KB, VB, 4>), grid, dim3(S4::NT), 0, st, p);
  } else if (p.nq == 16) {
    if constexpr (D <= 128) {
      using S16 = MfmaShape<D, KB, VB, 16>;
      hipLaunchKernelGGL((attn_mfma_kernel<D, KB, VB, 16>), grid, dim3(S16::NT), 0, st, p);
    } else {
      return fail(TQ_ERR_INVALID_ARGUMENT, "attention: 16-row groups need dim <= 128");
    }
  } else {
    return fail(TQ_ERR_INVALID_ARGUMENT, "attention: rows per group %d", p.nq);
  }
  return check_launch("attn_mfma_kernel");
}

}  // namespace tq
