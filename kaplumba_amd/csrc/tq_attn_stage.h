// TurboQuant decode / verify attention for small row groups (at most 4 query
// rows per kv head: GQA decode with R <= 4, or verify with R * L <= 4) at head
// dims 64 / 128 with MSE-coded keys, the packed cache staged through LDS.
//
// Workgroup: NW wave64s (16 when the LDS holds them, else 8) own tokens
// [t_begin, t_end) of one (sequence, kv head) and all (<= 4) query rows of its
// GQA group.  Sub-chunk i of 32 tokens belongs to wave i % NW.  Every wave has
// two LDS slots; a slot receives one sub-chunk's packed K and V rows and
// their norms straight from memory (buffer_load ... lds), so no registers
// hold data in flight: a wave issues the loads of sub-chunk i + 2 as soon as
// it has read sub-chunk i out of its slot, and computes sub-chunk i meanwhile.
//
// The hot scalar arguments (cache pointers, the key codebook, capacity,
// length, chunk, shape bits: 14 SGPRs) come first in the kernel signature and
// are preloaded into SGPRs at dispatch (-amdgpu-kernarg-preload-count), so
// the first sub-chunks' loads go out without waiting for the kernel-argument
// segment.
//
// Lane roles (l = lane, n = l % 16, g = l / 16), as in attn_small_kernel:
//   scores  S^T[tok][col] = sum_d k[tok][d] * q_col[d]    (16 x 16 tile, 32 tokens)
//     A = keys: lane (m, g) holds token 16 (g >> 1) + m, coordinate half
//         g & 1, four coordinates per MFMA as two pair-table entries read
//         straight into the operand: k slots (hi c0, hi c1, lo c0, lo c1,
//         hi c2, hi c3, lo c2, lo c3),
//     B = queries: column n = 8p + 4j + r is piece p (hi / lo) of query row r
//         for token subset j (zero where the lane group holds the other
//         subset), each coordinate pair twice against the hi and lo slots;
//         held in registers for the whole loop; one DPP row rotation by 8
//         adds the pieces.
//   softmax per lane: 4 tokens of one row, lazy reference maximum.
//   values  O[row][d] = sum_tok w[row][tok] * v[tok][d]      (16 x 16 tiles)
//     A = weights (f16, own four tokens and those of lane n + 4 by DPP),
//     B = values: (hi pair, lo pair) of two tokens' codebook values.
// Pair tables (keys: two coordinates of a token; values: one coordinate of two
// tokens) hold 8-byte (hi pair, lo pair) entries, 32 replicas per key (16 for
// 256-key tables) so that the lanes of one read hit distinct banks.
//
// Splits: a problem with one split is finished here; otherwise every workgroup
// writes its (o, m, l) partial with o still in the rotated basis (R_V^-1 is
// linear and commutes with the merge, so attn_merge_kernel applies it once per
// row after normalising).
// Semantics: quantized_attention, turboquant_cache.py:5110-5203.
#pragma once

#include "tq_attn_small.h"

// Phase stamps (build option TQ_PHASE_STAMPS; the shipped library has none):
// the 100 MHz wall clock at the phase boundaries of attn_stage_kernel,
// thread 0 of a workgroup (STAGE_STAMP) or lane 0 of every wave
// (STAGE_WSTAMP, rows r + wave), read back with tq_dbg_stage_stamps() from
// libkaplumba_tq_stamps.so (make -C kaplumba_amd/csrc stamps).  Rows:
// 0 entry, 1 codebooks in registers, 2 tables stored, 3 query row in LDS,
// 4 query staged, 5 staging barrier, 6 query operands loaded, 8+w loop start,
// 16+w first slot ready, 24+w loop end, 32 combine barrier, 33 partial stored.
#ifdef TQ_PHASE_STAMPS
namespace tq {
static __device__ uint64_t g_stage_stamps[40][1024];
}
#define STAGE_STAMP(i)                                                                              \
  do {                                                                                              \
    if (threadIdx.x == 0)                                                                           \
      g_stage_stamps[i][blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z)] =           \
          __builtin_amdgcn_s_memrealtime();                                                         \
  } while (0)
#define STAGE_WSTAMP(i)                                                                             \
  do {                                                                                              \
    if ((threadIdx.x & 63) == 0)                                                                    \
      g_stage_stamps[(i) + threadIdx.x / 64][blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z)] = \
          __builtin_amdgcn_s_memrealtime();                                                         \
  } while (0)
#else
#define STAGE_STAMP(i) \
  do {               \
  } while (0)
#define STAGE_WSTAMP(i) \
  do {                \
  } while (0)
#endif

namespace tq {

// Shape bits of attn_stage_kernel's `pack` argument.
constexpr int kStageHkvBits = kSmallRowsHkvBits;  // bits 0..11: kv heads (the host rejects more)
constexpr int kStageRShift = 12;   // bits 12..14: GQA group R (<= 4)
constexpr int kStageLShift = 15;   // bits 15..17: query length L (<= 4)
constexpr int kStageF16Norms = 1 << 18;
constexpr int kStageSeqArrays = 1 << 19;  // seq_lens or seq_starts present
constexpr int kStageQContig = 1 << 20;    // q addressed as contiguous [B, Hq, L, D]
constexpr int kStageQDtShift = 21;        // bits 21..22: q dtype

template <int D, int KB, int VB>
struct StageShape {
  static constexpr int SUB = 32;  // tokens per sub-chunk
  static constexpr int NQ = 4;    // query rows
  static constexpr int HALF = D / 2;
  static constexpr int KW = HALF * KB / 32;  // key words per lane (half a row)
  static constexpr int PWK = D * KB / 32;
  static constexpr int PWV = D * VB / 32;
  static constexpr int KKEYS = 1 << (2 * KB);
  static constexpr int VKEYS = 1 << (2 * VB);
  static constexpr int REPK = KKEYS <= 64 ? 32 : 16;
  static constexpr int REPV = VKEYS <= 64 ? 32 : 16;
  static constexpr int LOGSK = REPK == 32 ? 8 : 7;  // log2(REPK * 8)
  static constexpr int LOGSV = REPV == 32 ? 8 : 7;
  static constexpr int CPL = D / 16;  // value coordinates per lane
  static constexpr int SEGBITS = CPL * VB;
  static constexpr int VRAW = (VB == 3) ? 2 : 1;  // a 3-bit segment can cross a word
  static constexpr int KTAB = KKEYS * REPK * 8;
  static constexpr int VTAB = VKEYS * REPV * 8;
  // one slot: [K rows][V rows][K norms][V norms] of a sub-chunk (norms sized for f32)
  static constexpr int SK = 0;
  static constexpr int SV = SUB * PWK * 4;
  static constexpr int SKN = SV + SUB * PWV * 4;
  static constexpr int SVN = SKN + SUB * 4;
  static constexpr int SLOT = SVN + SUB * 4;
  // LDS: [K table][V table][q staging][zeros][rotated q rows][row max]
  //      [query rows as loaded][key signs][slots: wave w owns NS consecutive]
  static constexpr int LUTK_OFF = 0;
  static constexpr int LUTV_OFF = KTAB;
  static constexpr int QST_OFF = LUTV_OFF + VTAB;  // [i][p][r][h] 8 x f16 = 16 B
  static constexpr int QST_BYTES = 2 * NQ * 2 * (D / 8) * 16;
  static constexpr int ZERO_OFF = QST_OFF + QST_BYTES;
  static constexpr int QSC_OFF = ZERO_OFF + 16;            // [NQ] f32 hi/lo scale of each query row
  static constexpr int QRAW_OFF = QSC_OFF + 16;            // [NQ][D] query rows as loaded (<= 4 B each)
  static constexpr int QSGN_OFF = QRAW_OFF + NQ * D * 4;    // [NQ][D] f32 key signs (one copy per query wave)
  static constexpr int SLOT_OFF = QSGN_OFF + NQ * D * 4;
  // 8 waves (two per SIMD), each with NS = 2 slots in flight.  Measured on
  // the 32k-token decode: 16 waves (four per SIMD) or 3 slots per wave start
  // a larger share of the slab's loads at once, and the prologue's loads
  // then wait behind them for longer than the deeper pipeline saves.
  static constexpr int NW = 8;
  static constexpr int NS = 2;
  static constexpr int NT = NW * kWave;
  static constexpr int LOOP_BYTES = SLOT_OFF + NS * NW * SLOT;
  // epilogue (after a barrier the loop's buffers are dead)
  static constexpr int WO_OFF = 0;                          // [NW][NQ][D] f32
  static constexpr int WM_OFF = WO_OFF + NW * NQ * D * 4;  // [NW][NQ] m (log2 units)
  static constexpr int WL_OFF = WM_OFF + NW * NQ * 4;      // [NW][NQ] l
  static constexpr int WE_OFF = WL_OFF + NW * NQ * 4;      // [NW][NQ] 2^E
  static constexpr int FO_OFF = WE_OFF + NW * NQ * 4;      // [NQ][D] final rows
  static constexpr int POST_BYTES = FO_OFF + NQ * D * 4;
  static constexpr int BYTES = LOOP_BYTES > POST_BYTES ? LOOP_BYTES : POST_BYTES;
  // direct-to-LDS loads per slot: K rows and V rows in 1 KiB pieces, and
  // one each for the two norm vectors (32 lanes: f32 as 4 bytes, f16 as 2
  // bytes widened to a dword, so a slot's norms are 4 bytes per token either way)
  static constexpr int DMA_PER_SLOT = (SUB * PWK * 4 + 1023) / 1024 + (SUB * PWV * 4 + 1023) / 1024 + 2;
  static_assert(D == 64 || D == 128, "staged row-group kernel: head dim 64 or 128");
  static_assert(KW * 32 == HALF * KB, "key half rows are whole words");
  static_assert(SEGBITS <= 32, "value segment in one word");
  static_assert(SLOT % 16 == 0 && SKN % 16 == 0 && SLOT_OFF % 16 == 0, "slot alignment");
  static_assert(BYTES <= 160 * 1024, "LDS per workgroup");
  static_assert(LUTV_OFF < 65536, "table offsets fit the instruction offset field");
};

// Workgroup barrier ordering LDS stores and loads only: the staged loads
// are issued in inline assembly and waited for explicitly (a wave reads only
// the LDS it staged itself, after its own wait), so no fence needs them.
__device__ __forceinline__ void lds_only_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// s_waitcnt with only the vector-memory count limited (expcnt and lgkmcnt at
// their maxima); gfx9 encoding: vmcnt bits 3:0 and 15:14.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
  asm volatile("" ::: "memory");  // no LDS access moves above the wait
}

// Buffer descriptor words in SGPRs (raw buffer, 32-bit format: the layout
// __builtin_amdgcn_make_buffer_rsrc builds, here as plain words for inline
// assembly).  Loads past `bytes` return zeros and move no memory.
typedef uint32_t rsrc_words_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ rsrc_words_t rsrc_words(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  return rsrc_words_t{static_cast<uint32_t>(a), static_cast<uint32_t>(a >> 32) & 0xffffu, bytes, kBufferFlags};
}

// LDS byte address of a pointer into a __shared__ array (the low word of its
// generic address).
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p));
}

// Direct-to-LDS loads (buffer_load ... lds) in inline assembly, so that the
// compiler, which cannot tell one LDS destination from another, inserts no
// waits for them: every wait is explicit (wait_vmcnt).  M0 holds the LDS base
// and is restored afterwards.  Lane layout in LDS, per width: 16 and 4 bytes
// land contiguous (lane i at base + 16 i / 4 i); 2 bytes land zero-extended
// in dwords (lane i at base + 4 i).  Exec-masked lanes load nothing.
template <int W>
__device__ __forceinline__ void dma_lds(rsrc_words_t r, uint32_t lds_base, uint32_t voff) {
  uint32_t save;
  if constexpr (W == 16)
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\tbuffer_load_dwordx4 %2, %3, 0 offen lds\n\ts_mov_b32 m0, %0"
                 : "=&s"(save) : "s"(lds_base), "v"(voff), "s"(r) : "memory");
  else if constexpr (W == 4)
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\tbuffer_load_dword %2, %3, 0 offen lds\n\ts_mov_b32 m0, %0"
                 : "=&s"(save) : "s"(lds_base), "v"(voff), "s"(r) : "memory");
  else if constexpr (W == 2)
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\tbuffer_load_ushort %2, %3, 0 offen lds\n\ts_mov_b32 m0, %0"
                 : "=&s"(save) : "s"(lds_base), "v"(voff), "s"(r) : "memory");
  else
    static_assert(W == 16, "unsupported direct-to-LDS width");
}

// BYTES contiguous bytes at byte offset off of buffer r into LDS at base, in
// pieces of 64 lanes x W bytes (the last piece with the lanes it needs).
template <int BYTES, int W>
__device__ __forceinline__ void dma_bytes(rsrc_words_t r, uint32_t base, uint32_t off, int lane) {
  static_assert(BYTES % W == 0, "whole lane pieces");
  constexpr int PIECE = 64 * W;
#pragma unroll
  for (int j = 0; j < (BYTES + PIECE - 1) / PIECE; ++j) {
    const int left = BYTES - j * PIECE;
    if (left >= PIECE || lane < left / W) dma_lds<W>(r, base + j * PIECE, off + j * PIECE + lane * W);
  }
}

template <int D, int KB, int VB>
__global__ __launch_bounds__((StageShape<D, KB, VB>::NT), 1) void attn_stage_kernel(
    const void* pk, const void* pv, const void* pkn, const void* pvn, const float* __restrict__ kcb, int cap,
    int tlen, int chunk, int pack, const float* __restrict__ vcb, AttnParams p) {
  using S = StageShape<D, KB, VB>;
  constexpr int NW = S::NW;
  constexpr int NT = S::NT;
  constexpr int SUB = S::SUB;
  constexpr int NQ = S::NQ;
  constexpr int KW = S::KW;
  constexpr int CPL = S::CPL;
  constexpr int VRAW = S::VRAW;
  constexpr int PWK = S::PWK;
  constexpr int PWV = S::PWV;
  constexpr int QE = D / kWave;  // query elements per lane

  __shared__ __align__(16) unsigned char lds[S::BYTES];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int n = lane & 15;
  const int g = lane >> 4;
  const int split = blockIdx.x;
  const int gk = blockIdx.y;
  const int b = blockIdx.z;
  const int Hkv = pack & ((1 << kStageHkvBits) - 1);
  STAGE_STAMP(0);
  const int R = (pack >> kStageRShift) & 7;
  const int L = (pack >> kStageLShift) & 7;
  const int nrows = R * L;
  const bool nf16 = (pack & kStageF16Norms) != 0;
  const uint32_t nb = nf16 ? 2u : 4u;

  SeqWindow win{0, tlen};
  if (pack & kStageSeqArrays) win = seq_window(p, b);
  const int64_t Tb = win.len;  // token positions below are relative to win.start
  const int64_t t_begin64 = static_cast<int64_t>(split) * chunk;
  auto row_qoff = [&](int r) -> int64_t {  // (b * Hq + head) * L + position
    return (static_cast<int64_t>(b) * p.Hq + gk * R + r / L) * L + r % L;
  };
  if (t_begin64 >= Tb) {
    // no tokens for this split; an empty sequence still needs its output:
    // split 0 writes zeros (the reference divides a zero sum by 1e-6)
    if (Tb <= 0 && split == 0)
      for (int idx = tid; idx < NQ * D; idx += NT)
        if (idx / D < nrows) store_out(p.out, p.q_dtype, row_qoff(idx / D) * D + idx % D, 0.f);
    return;
  }
  const int t_begin = static_cast<int>(t_begin64);
  const int t_end = static_cast<int>(Tb < t_begin64 + chunk ? Tb : t_begin64 + chunk);
  const int nvalid = static_cast<int>((Tb + chunk - 1) / chunk);

  const int64_t kvrow0 = (static_cast<int64_t>(b) * Hkv + gk) * cap + win.start;
  const uint32_t tn = static_cast<uint32_t>(t_end);
  const auto krs = rsrc_words(static_cast<const char*>(pk) + kvrow0 * (PWK * 4), tn * (PWK * 4));
  const auto vrs = rsrc_words(static_cast<const char*>(pv) + kvrow0 * (PWV * 4), tn * (PWV * 4));
  const auto knrs = rsrc_words(static_cast<const char*>(pkn) + kvrow0 * nb, tn * nb);
  const auto vnrs = rsrc_words(static_cast<const char*>(pvn) + kvrow0 * nb, tn * nb);

  const int n_tok = t_end - t_begin;
  const int n_my = n_tok > wave * SUB ? (n_tok - wave * SUB + NW * SUB - 1) / (NW * SUB) : 0;
  auto sub_start = [&](int i) -> int { return t_begin + (i * NW + wave) * SUB; };
  constexpr int NS = S::NS;
  unsigned char* const slots = lds + S::SLOT_OFF + wave * (NS * S::SLOT);
  // One sub-chunk into one of this wave's slots: DMA_PER_SLOT transfers,
  // bounded at t_end (the loads past it write zeros and move no memory).
  auto stage = [&](int slot, int s0) {
    const uint32_t d = lds_addr(slots + slot * S::SLOT);
    const uint32_t t0 = static_cast<uint32_t>(s0);
    dma_bytes<SUB * PWK * 4, 16>(krs, d + S::SK, t0 * (PWK * 4), lane);
    dma_bytes<SUB * PWV * 4, 16>(vrs, d + S::SV, t0 * (PWV * 4), lane);
    if (lane < SUB) {
      if (nf16) {
        dma_lds<2>(knrs, d + S::SKN, (t0 + lane) * 2u);
        dma_lds<2>(vnrs, d + S::SVN, (t0 + lane) * 2u);
      } else {
        dma_lds<4>(knrs, d + S::SKN, (t0 + lane) * 4u);
        dma_lds<4>(vnrs, d + S::SVN, (t0 + lane) * 4u);
      }
    }
  };

  // ---- prologue.  The small loads go out first: the query waves stage
  // their row and the key signs, every wave loads its codebooks.  Only after
  // a workgroup barrier does any wave stage its first two sub-chunks: staged
  // loads issued earlier would queue ahead of the query loads in the memory
  // system (every CU requests its whole slab at once) and delay the prologue
  // by their drain.
  float lsg[6];  // -1 where lane bit k is set (Hadamard butterflies)
#pragma unroll
  for (int k = 0; k < 6; ++k) lsg[k] = (lane >> k) & 1 ? -1.f : 1.f;
  const bool dense = p.rot_kind == TQ_ROT_DENSE;
  const bool qwave = wave < NQ;
  const int qdt = dense ? TQ_DTYPE_F32 : (pack >> kStageQDtShift) & 3;
  const bool q32 = qdt == TQ_DTYPE_F32;
  if (qwave) {
    const bool qok = wave < nrows;
    int64_t qb = 0;
    if (qok) {
      if (dense || (pack & kStageQContig)) {
        qb = row_qoff(wave) * D;
      } else {
        qb = b * p.q_sb + static_cast<int64_t>(gk * R + wave / L) * p.q_sh +
             static_cast<int64_t>(wave % L) * p.q_sl;
      }
    }
    const char* qsrc = dense ? reinterpret_cast<const char*>(p.qrot) : static_cast<const char*>(p.q);
    const uint32_t qbytes = q32 ? D * 4u : D * 2u;
    // a row that does not exist loads zeros (an empty descriptor)
    const auto qrs = rsrc_words(qsrc + qb * (q32 ? 4 : 2), qok ? qbytes : 0u);
    const uint32_t qd = lds_addr(lds + S::QRAW_OFF + wave * D * 4);
    if (q32)
      dma_bytes<D * 4, 4>(qrs, qd, 0u, lane);
    else
      dma_bytes<D * 2, 4>(qrs, qd, 0u, lane);
    if (!dense) dma_bytes<D * 4, 4>(rsrc_words(p.krot, D * 4u), lds_addr(lds + S::QSGN_OFF + wave * D * 4), 0u, lane);
  }
  float ckb[1 << KB], cvb[1 << VB];
#pragma unroll
  for (int i = 0; i < (1 << KB); ++i) ckb[i] = kcb[i];
#pragma unroll
  for (int i = 0; i < (1 << VB); ++i) cvb[i] = vcb[i];
  __builtin_amdgcn_s_barrier();
  // the first sub-chunk alone: with every CU requesting only its first
  // slots, they arrive sooner; the second goes out after the set-up below
  stage(0, sub_start(0));

  // ---- pair tables: hi and lo f16 parts of (c[a] * s, c[b] * s) for key
  // a | b << bits, entry (hi pair, lo pair); keys: REPK replicas, a thread
  // writes 4 consecutive replicas of one key with two 16-byte stores
  float kmax = 0.f, vmax = 0.f;
#pragma unroll
  for (int i = 0; i < (1 << KB); ++i) kmax = fmaxf(kmax, fabsf(ckb[i]));
#pragma unroll
  for (int i = 0; i < (1 << VB); ++i) vmax = fmaxf(vmax, fabsf(cvb[i]));
  STAGE_STAMP(1);
  const float sk = f16_split_scale(kmax);
  const float cbs_v = f16_split_scale(vmax);
  {
    constexpr int KSLOTS = S::KKEYS * S::REPK / 4;
    constexpr int VSLOTS = S::VKEYS * S::REPV / 4;
    for (int t = tid; t < KSLOTS; t += NT) {
      const int key = t / (S::REPK / 4);
      uint32_t h0, l0, h1, l1;
      split_f16(mux_pick<KB>(ckb, key & ((1 << KB) - 1)) * sk, h0, l0);
      split_f16(mux_pick<KB>(ckb, key >> KB) * sk, h1, l1);
      const uint32_t hi = h0 | (h1 << 16), lo = l0 | (l1 << 16);
      uint4* d = reinterpret_cast<uint4*>(lds + S::LUTK_OFF) + t * 2;
      d[0] = d[1] = make_uint4(hi, lo, hi, lo);
    }
    for (int t = tid; t < VSLOTS; t += NT) {
      const int key = t / (S::REPV / 4);
      uint32_t h0, l0, h1, l1;
      split_f16(mux_pick<VB>(cvb, key & ((1 << VB) - 1)) * cbs_v, h0, l0);
      split_f16(mux_pick<VB>(cvb, key >> VB) * cbs_v, h1, l1);
      const uint32_t hi = h0 | (h1 << 16), lo = l0 | (l1 << 16);
      uint4* d = reinterpret_cast<uint4*>(lds + S::LUTV_OFF) + t * 2;
      d[0] = d[1] = make_uint4(hi, lo, hi, lo);
    }
  }
  if (tid < 4) reinterpret_cast<uint32_t*>(lds + S::ZERO_OFF)[tid] = 0u;
  STAGE_STAMP(2);

  // ---- query rows: q_s = round_qdtype(q * scale_q) * s_K, Hadamard, * 1/sqrt(D)
  // (dense: rotated by qprep_kernel).  Query wave r splits its row into f16
  // hi and lo pieces at the row's own scale (a power of two from max |y|) and
  // writes them straight into the B-operand staging [jj][p][r][h]: as f16
  // pairs, (q01, q01, q23, q23) of coordinates h D/2 + 4 jj + 0..3 of piece p.
  // The 16 entries of one jj are contiguous, so the lanes' reads of one
  // operand hit distinct banks.
  if (qwave) {
    // this wave's row and sign loads were issued before its first slot's
    // DMA_PER_SLOT staged loads (loads complete in order for vmcnt)
    wait_vmcnt<S::DMA_PER_SLOT>();
    STAGE_STAMP(3);
    float y[QE];
#pragma unroll
    for (int e = 0; e < QE; ++e) {
      const int idx = lane + e * kWave;
      const uint32_t raw = q32 ? reinterpret_cast<const uint32_t*>(lds + S::QRAW_OFF + wave * D * 4)[idx]
                               : reinterpret_cast<const uint16_t*>(lds + S::QRAW_OFF + wave * D * 4)[idx];
      const float sgn_e = dense ? 1.f : reinterpret_cast<const float*>(lds + S::QSGN_OFF + wave * D * 4)[idx];
      const float qv = q32 ? __builtin_bit_cast(float, raw)
                           : (qdt == TQ_DTYPE_F16 ? f16_bits_to_f32(static_cast<uint16_t>(raw))
                                                  : bf16_bits_to_f32(static_cast<uint16_t>(raw)));
      y[e] = dense ? qv : round_q(qdt, qv * p.scale_q) * sgn_e;
    }
    if (!dense) {
      wave_fwht<D>(y, lsg);
#pragma unroll
      for (int e = 0; e < QE; ++e) y[e] *= p.rscale;
    }
    float m = 0.f;
#pragma unroll
    for (int e = 0; e < QE; ++e) m = fmaxf(m, fabsf(y[e]));
    const float sq_row = f16_split_scale(wave_max(m));
    if (lane == 0) reinterpret_cast<float*>(lds + S::QSC_OFF)[wave] = sq_row;
    STAGE_STAMP(4);
    uint32_t* st = reinterpret_cast<uint32_t*>(lds + S::QST_OFF);
#pragma unroll
    for (int e = 0; e < QE; ++e) {
      uint32_t hi, lo;
      split_f16(y[e] * sq_row, hi, lo);
      // lanes 2k, 2k + 1 hold the two coordinates of one f16 pair
      const uint32_t hi_n = __float_as_uint(xor_lane<1>(__uint_as_float(hi)));
      const uint32_t lo_n = __float_as_uint(xor_lane<1>(__uint_as_float(lo)));
      if ((lane & 1) == 0) {
        const int c = lane + e * kWave;
        const int h = c / (D / 2);
        const int jj = (c % (D / 2)) / 4;  // 4-coordinate group
        const int e2 = (c % 4) / 2;        // pair within the group
        const int base0 = (((jj * 2 + 0) * NQ + wave) * 2 + h) * 4 + 2 * e2;
        const int base1 = (((jj * 2 + 1) * NQ + wave) * 2 + h) * 4 + 2 * e2;
        st[base0] = st[base0 + 1] = hi | (hi_n << 16);
        st[base1] = st[base1 + 1] = lo | (lo_n << 16);
      }
    }
  }
  lds_only_barrier();
  STAGE_STAMP(5);
#pragma unroll
  for (int k = 1; k < NS; ++k) stage(k, sub_start(k));

  // ---- lane constants
  const int jq = (n >> 2) & 1;  // token subset of this lane's score column
  const int rq = n & 3;         // query row of this lane's score column
  // B operands of lane (column n = 8 p + 4 jq + rq, g): zero unless lane
  // group g holds tokens of subset jq
  u32x4_t qd[D / 8];
  {
    const uint32_t qb_addr = ((g >> 1) == jq)
                                 ? static_cast<uint32_t>(S::QST_OFF + (((n >> 3) * NQ + rq) * 2 + (g & 1)) * 16)
                                 : static_cast<uint32_t>(S::ZERO_OFF);
    const uint32_t qb_step = ((g >> 1) == jq) ? 2u * NQ * 2 * 16 : 0u;
#pragma unroll
    for (int j = 0; j < D / 8; ++j) qd[j] = lds_at<u32x4_t>(lds, qb_addr + j * qb_step);
  }
  STAGE_STAMP(6);
  // keys: token 16 (g >> 1) + n, half g & 1 of the slot's rows
  const uint32_t k_lane = (16 * (g >> 1) + n) * (PWK * 4) + (g & 1) * (KW * 4);
  // norms: tokens 16 jq + 4 g .. + 3 of the sub-chunk
  const uint32_t n_tok4 = 16 * jq + 4 * g;
  // values: coordinates CPL n .. CPL n + CPL - 1 of tokens 4g + e, 16 + 4g + e
  const int vbit = CPL * n * VB;
  const uint32_t v_lane = (vbit >> 5) * 4;
  const int vsh = vbit & 31;
  const uint32_t lutk_lane = (lane % S::REPK) * 8;
  const uint32_t lutv_lane = (lane % S::REPV) * 8;
  uint32_t kmask = (S::KKEYS - 1u) << S::LOGSK;
  uint32_t vmask = (S::VKEYS - 1u) << S::LOGSV;
  asm volatile("" : "+s"(kmask), "+s"(vmask));
  // score scale: S * ||k|| * log2(e) / (s_K s_Q) in log2 units
  const float kscale = 1.4426950408889634f * __builtin_amdgcn_rcpf(sk) *
                       __builtin_amdgcn_rcpf(reinterpret_cast<const float*>(lds + S::QSC_OFF)[rq]);
  // causal limit of this lane's row (keys t <= lim are visible)
  int lim = INT32_MAX, lim_min = INT32_MAX;
  if (p.causal) {
    const int base_lim = static_cast<int>(Tb - L);
#pragma unroll
    for (int r = 0; r < NQ; ++r)
      if (r < nrows) {
        const int lr_ = base_lim + r % L;
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

  constexpr uint32_t MEVEN = [] {
    uint32_t m = 0;
    for (int j = 0; j < CPL; j += 2) m |= ((1u << VB) - 1u) << (j * VB);
    return m;
  }();

  int slot = 0;  // i % NS
  STAGE_WSTAMP(8);
#pragma unroll 1
  for (int i = 0; i < n_my; ++i) {
    const int s0 = sub_start(i);
    // (without it, waves 0-3 finished about one sub-chunk before 4-7)
    prio_by_progress(i, n_my);
    // this slot's transfers are complete once at most the other slots' remain
    // (sub-chunks past the wave's last are never staged, so near the end
    // fewer slots are in flight)
    if (i + NS - 1 < n_my)
      wait_vmcnt<(NS - 1) * S::DMA_PER_SLOT>();
    else
      wait_vmcnt<0>();
    if (i == 0) STAGE_WSTAMP(16);
    const unsigned char* sl = slots + slot * S::SLOT;
    uint32_t kw[KW];
    {
      const unsigned char* kp = sl + S::SK + k_lane;
      if constexpr (KW % 2 == 0 && (PWK * 4) % 8 == 0) {
#pragma unroll
        for (int w = 0; w < KW; w += 2) {
          const uint2 x = *reinterpret_cast<const uint2*>(kp + w * 4);
          kw[w] = x.x;
          kw[w + 1] = x.y;
        }
      } else {
#pragma unroll
        for (int w = 0; w < KW; ++w) kw[w] = *reinterpret_cast<const uint32_t*>(kp + w * 4);
      }
    }
    uint32_t vw[8][VRAW];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int tok = (e < 4 ? 4 * g + e : 16 + 4 * g + (e - 4));
#pragma unroll
      for (int w = 0; w < VRAW; ++w)
        vw[e][w] = *reinterpret_cast<const uint32_t*>(sl + S::SV + tok * (PWV * 4) + v_lane + w * 4);
    }
    float nk[4], nv[4];
    if (nf16) {  // one f16 norm in the low half of each dword
      const uint4 a = *reinterpret_cast<const uint4*>(sl + S::SKN + n_tok4 * 4);
      const uint4 c = *reinterpret_cast<const uint4*>(sl + S::SVN + n_tok4 * 4);
      const uint32_t aa[4] = {a.x, a.y, a.z, a.w}, cc[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        nk[e] = f16_bits_to_f32(static_cast<uint16_t>(aa[e]));
        nv[e] = f16_bits_to_f32(static_cast<uint16_t>(cc[e]));
      }
    } else {
      const float4 a = *reinterpret_cast<const float4*>(sl + S::SKN + n_tok4 * 4);
      const float4 c = *reinterpret_cast<const float4*>(sl + S::SVN + n_tok4 * 4);
      nk[0] = a.x, nk[1] = a.y, nk[2] = a.z, nk[3] = a.w;
      nv[0] = c.x, nv[1] = c.y, nv[2] = c.z, nv[3] = c.w;
    }
    // the slot is read out (the values are in registers): its next
    // transfers may overwrite it
#pragma unroll
    for (int w = 0; w < KW; ++w) asm volatile("" ::"v"(kw[w]));
#pragma unroll
    for (int e = 0; e < 8; ++e)
#pragma unroll
      for (int w = 0; w < VRAW; ++w) asm volatile("" ::"v"(vw[e][w]));
#pragma unroll
    for (int e = 0; e < 4; ++e) asm volatile("" ::"v"(nk[e]), "v"(nv[e]));
    if (i + NS < n_my) stage(slot, sub_start(i + NS));
    slot = slot + 1 == NS ? 0 : slot + 1;

    // ---- scores: D / 8 MFMAs in two alternating accumulator chains; the
    // table reads run KPF MFMAs ahead (about a dozen reads in flight, within
    // the lgkm counter), which hides the LDS latency behind the products
    f32x4_t Ch = {0.f, 0.f, 0.f, 0.f}, Cl = {0.f, 0.f, 0.f, 0.f};
    {
      constexpr int KPF = 6;
      uint2 eb[D / 8][2];
      auto kload = [&](int j) {
        eb[j][0] = lds_at<uint2>(lds, S::LUTK_OFF + key_addr<2 * KB, S::LOGSK>(kw, (4 * j) * KB, lutk_lane, kmask));
        eb[j][1] = lds_at<uint2>(lds, S::LUTK_OFF + key_addr<2 * KB, S::LOGSK>(kw, (4 * j + 2) * KB, lutk_lane, kmask));
      };
#pragma unroll
      for (int j = 0; j < KPF && j < D / 8; ++j) kload(j);
#pragma unroll
      for (int j = 0; j < D / 8; ++j) {
        if (j + KPF < D / 8) kload(j + KPF);
        const u32x4_t a = {eb[j][0].x, eb[j][0].y, eb[j][1].x, eb[j][1].y};
        if (j & 1)
          Cl = mfma_f16(a, qd[j], Cl);
        else
          Ch = mfma_f16(a, qd[j], Ch);
      }
    }
    const f32x4_t C = Ch + Cl;

    // ---- value keys: pairs (4g, 4g+1), (4g+2, 4g+3), (16+4g, ..) of
    // coordinate CPL n + c, the two tokens' fields interleaved
    uint32_t zl[4], zh[4];
#pragma unroll
    for (int e2 = 0; e2 < 4; ++e2) {
      uint32_t xa, xb;
      if constexpr (VRAW == 2) {
        xa = __builtin_amdgcn_alignbit(vw[2 * e2][1], vw[2 * e2][0], vsh);
        xb = __builtin_amdgcn_alignbit(vw[2 * e2 + 1][1], vw[2 * e2 + 1][0], vsh);
      } else if constexpr (S::SEGBITS < 32) {
        xa = vw[2 * e2][0] >> vsh;
        xb = vw[2 * e2 + 1][0] >> vsh;
      } else {
        xa = vw[2 * e2][0];
        xb = vw[2 * e2 + 1][0];
      }
      zl[e2] = (xa & MEVEN) | ((xb << VB) & ~MEVEN);
      zh[e2] = ((xa >> VB) & MEVEN) | (xb & ~MEVEN);
    }

    // ---- softmax over this lane's 4 tokens of its row
    float sc[4], d[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float ci = own_reg(C[k]);
      sc[k] = ci + __builtin_bit_cast(float, row_ror_u<8>(__builtin_bit_cast(uint32_t, ci)));
      d[k] = fmaf(sc[k], nk[k] * kscale, -m_row);
    }
    const float dmax = fmaxf(fmaxf(d[0], d[1]), fmaxf(d[2], d[3]));
    const float nvmax = fmaxf(fmaxf(nv[0], nv[1]), fmaxf(nv[2], nv[3]));
    const bool edge = s0 + SUB > t_end || s0 + SUB - 1 > lim_min;  // wave-uniform
    if (edge || __any((dmax > kLazy || nvmax > nv_lim) ? 1 : 0)) {
      // slow path: masks, new reference max / norm exponent, rescale
      const int tbase = s0 + 16 * jq + 4 * g;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        sc[k] = sc[k] * (nk[k] * kscale);
        if (edge) {
          if (tbase + k > lim) sc[k] = -FLT_MAX;
          if (tbase + k >= t_end) sc[k] = -INFINITY;
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
      for (int r = 0; r < NQ; ++r)
        ar[r] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ao), r));
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
      for (int k = 0; k < 4; ++k) d[k] = sc[k] - m_row;
    }
    float w[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float pe = __builtin_amdgcn_exp2f(d[k]);
      l_acc += pe;
      w[k] = pe * (nv[k] * vsc);
    }
    // weights to the A operands: own 4 tokens (subset 0), then those of lane
    // n + 4 (subset 1); each pair twice, against the (hi pair, lo pair) k
    // slots of the value operand
    const uint32_t w01 = pack_f16x2(w[0], w[1]);
    const uint32_t w23 = pack_f16x2(w[2], w[3]);
    const uint32_t x01 = row_ror_u<12>(w01);
    const uint32_t x23 = row_ror_u<12>(w23);
    const u32x4_t A0 = {w01, w01, w23, w23};
    const u32x4_t A1 = {x01, x01, x23, x23};
    // value table reads run VPF coordinates (two MFMAs each) ahead
    {
      constexpr int VPF = 4;
      uint2 vop[CPL][4];
      auto vload = [&](int c) {
#pragma unroll
        for (int e2 = 0; e2 < 4; ++e2) {
          const uint32_t z[1] = {(c & 1) ? zh[e2] : zl[e2]};
          vop[c][e2] = lds_at<uint2>(lds, S::LUTV_OFF + key_addr<2 * VB, S::LOGSV>(z, (c >> 1) * 2 * VB, lutv_lane, vmask));
        }
      };
#pragma unroll
      for (int c = 0; c < VPF && c < CPL; ++c) vload(c);
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        if (c + VPF < CPL) vload(c + VPF);
        O[c] = mfma_f16(A0, u32x4_t{vop[c][0].x, vop[c][0].y, vop[c][1].x, vop[c][1].y}, O[c]);
        O[c] = mfma_f16(A1, u32x4_t{vop[c][2].x, vop[c][2].y, vop[c][3].x, vop[c][3].y}, O[c]);
      }
    }
  }
  __builtin_amdgcn_s_setprio(0);
  // every staged transfer has landed (waves without sub-chunks wait here)
  wait_vmcnt<0>();
  STAGE_WSTAMP(24);

  // --------------------------------------------------- combine the waves ----
  // l of row r: lanes (g', n) with n < 8 (piece 0), subsets n and n + 4
  float lr = l_acc + __builtin_bit_cast(float, row_ror_u<12>(__builtin_bit_cast(uint32_t, l_acc)));
  lr += xor_lane<16>(lr);
  {
    const float2 h = halves(lr);
    lr = h.x + h.y;
  }
  lds_barrier();  // every wave is done with the tables and staging
  STAGE_STAMP(32);
  float* s_wo = reinterpret_cast<float*>(lds + S::WO_OFF);
  float* s_wm = reinterpret_cast<float*>(lds + S::WM_OFF);
  float* s_wl = reinterpret_cast<float*>(lds + S::WL_OFF);
  float* s_we = reinterpret_cast<float*>(lds + S::WE_OFF);
  if (g == 0) {
#pragma unroll
    for (int r = 0; r < NQ; ++r) {
      float4* dst = reinterpret_cast<float4*>(s_wo + (wave * NQ + r) * D + CPL * n);
#pragma unroll
      for (int c = 0; c < CPL; c += 4) dst[c / 4] = make_float4(O[c][r], O[c + 1][r], O[c + 2][r], O[c + 3][r]);
    }
    if (n < NQ) {
      // a wave without tokens keeps m = -inf and contributes nothing
      s_wm[wave * NQ + n] = m_row;
      s_wl[wave * NQ + n] = lr;
      s_we[wave * NQ + n] = ldexpf(1.f, E);  // undoes the weights' 2^-E
    }
  }
  lds_barrier();
  // thread (row r, coordinate d): the waves' log-sum-exp factors, o and l
  float* s_fo = reinterpret_cast<float*>(lds + S::FO_OFF);
  const float oscale = __builtin_amdgcn_rcpf(cbs_v);  // a power of two: exact
  const int64_t grp = static_cast<int64_t>(b) * Hkv + gk;
  for (int idx = tid; idx < NQ * D; idx += NT) {
    const int r = idx / D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, s_wm[w * NQ + r]);
    float a = 0.f, lt = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float wm = s_wm[w * NQ + r];
      const float f = wm == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(wm - M);
      lt = fmaf(s_wl[w * NQ + r], f, lt);
      a = fmaf(s_wo[(w * NQ) * D + idx], f * s_we[w * NQ + r], a);
    }
    a *= oscale;
    if (nvalid > 1) {
      // this split's partial for attn_merge_kernel, o in the rotated basis
      p.po[(grp * p.n_splits + split) * static_cast<int64_t>(NQ) * D + idx] = a;
      if (idx % D == 0) {
        float* pm = p.pml + ((grp * p.n_splits + split) * NQ + r) * 2;
        pm[0] = M * 0.6931471805599453f;  // natural-log units
        pm[1] = lt;
      }
    } else {
      s_fo[idx] = lt > 0.f ? a / lt : 0.f;  // 0 when no token is visible
    }
  }
  STAGE_STAMP(33);
  if (nvalid > 1) return;

  // ---- finish a single split: R_V^-1, store
  lds_barrier();
  if (!dense) {
    if (wave < nrows) {
      float y[QE];
#pragma unroll
      for (int e = 0; e < QE; ++e) y[e] = s_fo[wave * D + lane + e * kWave];
      wave_fwht<D>(y, lsg);
      const int64_t qo = row_qoff(wave) * D;
#pragma unroll
      for (int e = 0; e < QE; ++e)
        store_out(p.out, p.q_dtype, qo + lane + e * kWave, y[e] * p.rscale * p.vrot[lane + e * kWave]);
    }
  } else {
    dense_rows_out<D, NQ, NT>(p, s_fo, s_wo, nrows, row_qoff, [](int) { return 1.f; });
  }
}

template <int D, int KB, int VB>
int launch_stage(const AttnParams& p, hipStream_t st) {
  using S = StageShape<D, KB, VB>;
  const dim3 grid(p.n_splits, p.Hkv, p.B);
  const bool contig = (p.L == 1 || p.q_sl == D) && (p.Hq == 1 || p.q_sh == static_cast<int64_t>(p.L) * D) &&
                      (p.B == 1 || p.q_sb == static_cast<int64_t>(p.Hq) * p.L * D);
  const int pack = p.Hkv | (p.R << kStageRShift) | (p.L << kStageLShift) |
                   (p.norm_dtype == TQ_DTYPE_F16 ? kStageF16Norms : 0) |
                   ((p.seq_lens || p.seq_starts) ? kStageSeqArrays : 0) | (contig ? kStageQContig : 0) |
                   (p.q_dtype << kStageQDtShift);
  hipLaunchKernelGGL((attn_stage_kernel<D, KB, VB>), grid, dim3(S::NT), 0, st, p.k, p.v, p.kn, p.vn, p.kcb,
                     static_cast<int>(p.cap), static_cast<int>(p.T), p.chunk, pack, p.vcb, p);
  return check_launch("attn_stage_kernel");
}

}  // namespace tq
