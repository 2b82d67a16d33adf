// Many query rows per kv head (prefill chunks, wide verify) at d = 128 over
// MSE-coded K/V: a partial kernel of the general path (tq_attn_general.h)
// that decodes each 32-token sub-chunk of K and V into LDS once and lets 8
// waves -- 256 query rows, 32 per wave -- read it as matrix-core operands.
// A wave's two 16-row tiles share every K and V operand it reads from LDS,
// which halves the LDS traffic per query row (the bound of this kernel).
//
// Per sub-chunk i (one __syncthreads per step; staging and decoded buffers
// rotate over three slots, so every LDS address of an unrolled step is a
// register base plus an immediate):
//   load    packed K/V words and norms of sub-chunk i + 4 into registers
//           (three register sets rotate, so a load has two steps to land);
//   scores  S^T = K Q^T on v_mfma_f32_16x16x32_f16: A = key rows
//           (ds_read_b128), B = the wave's query rows (hi / lo f16 in
//           registers); K_hi Q_hi + K_hi Q_lo + K_lo Q_hi, f32-class
//           products.  The two 16-token tiles hold tokens 8 (m / 4) + 4 h +
//           m % 4 in row m of tile h, so lane (row n, g) ends with tokens
//           8 g .. 8 g + 7;
//   decode  sub-chunk i + 1, by the four lead waves between their softmax
//           and their P V: thread (token, 8 coordinates) looks up the K and V
//           pair tables and writes 16 bytes each of the hi and lo f16 parts
//           of the scaled codebook values; K rows go to the slot the score
//           MFMA reads them from, V rows into 16-column blocks (32 bytes per
//           token, token slots permuted so a transposed read meets every
//           bank once), whole blocks per wave so the stores also spread over
//           all banks;
//   softmax in log2 units with a lazy reference maximum (moved only when a
//           score exceeds it by 2^7) and a lazy value-norm exponent, checked
//           by one vote per sub-chunk;
//   O += P V: A = the lane's own 8 weights, B = V through ds_read_b64_tr_b16
//           (lane (coordinate n, g) receives tokens 8 g .. 8 g + 7 of its
//           coordinate), hi and lo parts;
//   stage   sub-chunk i + 2's registers into its LDS staging slot.
// Queries arrive prepared per row by gen_tile_qprep_kernel (below).
// Output: (o, max, sum) per row in the general path's 8-row partial layout,
// o in the rotated value basis (the merge applies R_V^-1 once per row).  Scores are
// s_t = n_t <q_rot, c[idx_t]>, values n_t c[idx_t] (quantized_attention,
// turboquant_cache.py:5110-5203); the causal rule, ragged lengths and left
// padding as in the general path; no array mask (those take gen_partial_kernel).
#pragma once

#include <type_traits>

#include "tq_attn_general.h"
#include "tq_attn_mfma.h"
#include "tq_attn_small.h"

namespace tq {

constexpr int kTileRT = 2;  // 16-row MFMA tiles per wave
constexpr int kTileNW = 8;  // waves per workgroup
constexpr int kTileThreads = 64 * kTileNW;
constexpr int kTileRows = 16 * kTileRT * kTileNW;  // query rows per workgroup

template <int KB, int VB>
struct TileShape {
  static constexpr int D = 128;
  static constexpr int SUB = 32;
  static constexpr int NBUF = 3;  // staging / decoded slots
  static constexpr int PWK = D * KB / 32;
  static constexpr int PWV = D * VB / 32;
  static constexpr int KKEYS = 1 << (2 * KB);
  static constexpr int VKEYS = 1 << (2 * VB);
  static constexpr int REPK = KKEYS <= 64 ? 32 : 8;
  static constexpr int REPV = VKEYS <= 64 ? 32 : 8;
  static constexpr int KROW = 2 * D + 16;  // bytes per decoded key row (f16, padded)
  static constexpr int VCT = SUB * 32;     // bytes per 16-column block of decoded values
  // LDS: [K pair table][V pair table][staging x3][decoded x3]
  static constexpr int KTAB_OFF = 0;
  static constexpr int VTAB_OFF = KTAB_OFF + KKEYS * REPK * 8;
  static constexpr int STG_K = 0;                       // SUB * PWK words
  static constexpr int STG_V = STG_K + SUB * PWK * 4;   // SUB * PWV words
  static constexpr int STG_KN = STG_V + SUB * PWV * 4;  // SUB f32
  static constexpr int STG_VN = STG_KN + SUB * 4;
  static constexpr int STG_BYTES = STG_VN + SUB * 4;
  static constexpr int STG_OFF = VTAB_OFF + VKEYS * REPV * 8;
  static constexpr int DEC_KHI = 0;
  static constexpr int DEC_KLO = DEC_KHI + SUB * KROW;
  static constexpr int DEC_VHI = DEC_KLO + SUB * KROW;
  static constexpr int DEC_VLO = DEC_VHI + (D / 16) * VCT;
  static constexpr int DEC_KN = DEC_VLO + (D / 16) * VCT;  // SUB f32 key norms
  static constexpr int DEC_VN = DEC_KN + SUB * 4;          // SUB f32 value norms
  static constexpr int DEC_BYTES = DEC_VN + SUB * 4;
  static constexpr int DEC_OFF = STG_OFF + NBUF * STG_BYTES;
  static constexpr int BYTES = DEC_OFF + NBUF * DEC_BYTES;
  // staging loads: one thread per word / norm, in staging order
  static constexpr int LOAD_SLOTS = SUB * PWK + SUB * PWV + 2 * SUB;
  static constexpr int LOADS = (LOAD_SLOTS + kTileThreads - 1) / kTileThreads;
  static_assert(kTileThreads >= 4 * SUB, "norm copy by the lead waves");
  static_assert(BYTES <= 160 * 1024, "tile kernel LDS");
  static_assert(KROW % 16 == 0 && STG_BYTES % 16 == 0 && DEC_BYTES % 16 == 0, "16-byte aligned LDS rows");
  static_assert(STG_V == SUB * PWK * 4 && STG_KN == STG_V + SUB * PWV * 4, "staging in load-slot order");
};

// Slot of token t's decoded key row: row m = 4 (t / 8) + t % 4 of tile
// h = (t / 4) % 2, so that score lane group g collects tokens 8 g .. 8 g + 7.
__device__ __forceinline__ int tile_kslot(int t) { return 16 * ((t >> 2) & 1) + 4 * (t >> 3) + (t & 3); }

// Slot of token t's 32-byte row in a 16-column value block: bit 3 of t
// folded into bit 2, so the eight rows a half-wave's transposed read touches
// (8 g + 4 h + 0..3 for g = 2 k, 2 k + 1) sit in eight distinct 32-byte bank
// groups.  An involution, hence a permutation of 0..31.
__device__ __forceinline__ int tile_vslot(int t) { return t ^ ((t >> 1) & 4); }

template <int KB, int VB>
__global__ __launch_bounds__(kTileThreads) void gen_tile_kernel(GenParams p, int n_blocks) {
  using S = TileShape<KB, VB>;
  constexpr int D = S::D;
  constexpr int SUB = S::SUB;
  constexpr float kLazy = 7.f;
  __shared__ __align__(16) unsigned char lds[S::BYTES];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int n = lane & 15;
  const int g = lane >> 4;
  // Workgroup ids go to the 8 XCDs in turn (id % 8).  When the number of
  // (sequence, kv head) pairs is a multiple of 8, pair h runs entirely on
  // XCD h % 8, so its queries and its K/V are fetched into one L2 once.
  int pair, wi;
  {
    const int id = blockIdx.x;
    const int per = n_blocks * p.n_splits;  // workgroups per pair
    if ((p.B * p.Hkv) % 8 == 0) {
      const int k = id >> 3;
      pair = (k / per) * 8 + (id & 7);
      wi = k % per;
    } else {
      pair = id / per;
      wi = id % per;
    }
  }
  const int split = wi % p.n_splits;
  const int rb = wi / p.n_splits;
  const int gk = pair % p.Hkv;
  const int b = pair / p.Hkv;
  const int RL = p.R * p.L;
  constexpr int RT = kTileRT;
  const int row_w0 = rb * kTileRows + 16 * RT * wave;  // first kv-head row of this wave
  const int64_t grp0 = (static_cast<int64_t>(b) * p.Hkv + gk) * p.n_rg;  // 8-row groups of this head

  int64_t start, len;
  {
    int64_t end = p.seq_lens ? static_cast<int64_t>(p.seq_lens[b]) : p.T;
    end = end > p.T ? p.T : (end < 0 ? 0 : end);
    int64_t s0 = p.seq_starts ? static_cast<int64_t>(p.seq_starts[b]) : 0;
    s0 = s0 < 0 ? 0 : (s0 > end ? end : s0);
    start = s0;
    len = end - s0;
  }
  const int64_t t_begin64 = static_cast<int64_t>(split) * p.chunk;
  if (t_begin64 >= len) {  // no tokens: a neutral partial per row (the merge skips it)
    for (int r = tid; r < kTileRows; r += kTileThreads) {
      const int rr = rb * kTileRows + r;
      if (rr >= RL) continue;
      float* pm = p.pml + ((grp0 + rr / 8) * p.n_splits + split) * 16 + (rr % 8) * 2;
      pm[0] = -INFINITY;
      pm[1] = 0.f;
    }
    return;
  }
  // token positions relative to the window fit 32 bits (capacity < 2^31)
  const int t_begin = static_cast<int>(t_begin64);
  const int t_end = static_cast<int>(min(len, t_begin64 + p.chunk));
  const int ntiles = (t_end - t_begin + SUB - 1) / SUB;
  const int64_t rowbase = (static_cast<int64_t>(b) * p.Hkv + gk) * p.cap + start;
  const bool nf16 = p.norm_dtype == TQ_DTYPE_F16;

  // ---- loads: slot sl -> word of the K rows, of the V rows, a key norm, a
  // value norm (staging order).  Every lane loads from a valid address (a
  // token past the split's end reads the first token instead) and the stage
  // writes zero for those; 16-bit norms widen to f32 at the stage.
  const char* lsrc[S::LOADS];  // address of the slot's element at token 0 of the window
  int lstride[S::LOADS];       // bytes per token
  int ltok[S::LOADS];          // token within the sub-chunk
  bool lwide[S::LOADS];        // 32-bit element (else an f16 norm)
#pragma unroll
  for (int u = 0; u < S::LOADS; ++u) {
    const int sl = tid + u * kTileThreads;
    const char* src = static_cast<const char*>(p.k) + rowbase * S::PWK * 4;
    int stride = S::PWK * 4, tok = 0;
    bool wide = true;
    if (sl < SUB * S::PWK) {
      tok = sl / S::PWK;
      src += (sl % S::PWK) * 4;
    } else if (sl < SUB * (S::PWK + S::PWV)) {
      const int j = sl - SUB * S::PWK;
      tok = j / S::PWV;
      src = static_cast<const char*>(p.v) + rowbase * S::PWV * 4 + (j % S::PWV) * 4;
      stride = S::PWV * 4;
    } else if (sl < S::LOAD_SLOTS) {
      const int j = sl - SUB * (S::PWK + S::PWV);
      tok = j & (SUB - 1);
      stride = nf16 ? 2 : 4;
      src = static_cast<const char*>(j < SUB ? p.kn : p.vn) + rowbase * stride;
      wide = !nf16;
    }
    lsrc[u] = src;
    lstride[u] = stride;
    ltok[u] = tok;
    lwide[u] = wide;
  }
  auto load_tile = [&](int tile, uint32_t (&r)[S::LOADS]) {
    const int t0 = t_begin + tile * SUB;
#pragma unroll
    for (int u = 0; u < S::LOADS; ++u) {
      const int tok = t0 + ltok[u];
      const char* a = lsrc[u] + static_cast<int64_t>(tok < t_end ? tok : t_begin) * lstride[u];
      r[u] = lwide[u] ? *reinterpret_cast<const uint32_t*>(a) : *reinterpret_cast<const uint16_t*>(a);
    }
  };
  auto store_stage = [&](int sb, int tile, const uint32_t (&r)[S::LOADS]) {
    uint32_t* st = reinterpret_cast<uint32_t*>(lds + S::STG_OFF + sb * S::STG_BYTES);
    const int t0 = t_begin + tile * SUB;
#pragma unroll
    for (int u = 0; u < S::LOADS; ++u) {
      const int sl = tid + u * kTileThreads;
      if (sl < S::LOAD_SLOTS) {
        uint32_t x = lwide[u] ? r[u] : __float_as_uint(f16_bits_to_f32(static_cast<uint16_t>(r[u])));
        st[sl] = t0 + ltok[u] < t_end ? x : 0u;
      }
    }
  };

  // the first four sub-chunks' loads go out before the table and query
  // set-up, which then hides their latency (sub-chunk 0 in a set of its own)
  uint32_t rgt[S::LOADS], rg0[S::LOADS], rg1[S::LOADS], rg2[S::LOADS];
  load_tile(0, rgt);
  if (ntiles > 1) load_tile(1, rg1);
  if (ntiles > 2) load_tile(2, rg2);
  if (ntiles > 3) load_tile(3, rg0);

  // ---- pair tables: entry (a | b << BITS) = (hi c_a | hi c_b << 16, lo c_a | lo c_b << 16)
  // of the codebooks scaled by a power of two (largest magnitude in
  // [2^12, 2^13): normal lo parts)
  // The codebooks pass through LDS (decoded slot 2, first written in step
  // 1), so each table entry reads them there rather than from memory.
  float* cbl = reinterpret_cast<float*>(lds + S::DEC_OFF + 2 * S::DEC_BYTES);
  if (tid < (1 << KB)) cbl[tid] = p.kcb[tid];
  if (tid < (1 << VB)) cbl[16 + tid] = p.vcb[tid];
  // ---- this wave's query rows (prepared by gen_tile_qprep_kernel): tile
  // rt, lane (row n, g) holds coordinates 32 s + 8 g .. + 7 of row
  // row_w0 + 16 rt + n as hi / lo f16 parts of q_rot * sq.  A row past the
  // end reads row 0 and then holds zeros.
  bool row_ok[RT];
  u32x4_t qh[RT][4], ql[RT][4];
  float qmul[RT];  // log2(e) / (sk * sq): MFMA units -> score units (log2)
  int lim[RT];     // causal: tokens t <= lim (relative to the window) are visible
  {
    const int64_t pair_row0 = static_cast<int64_t>(pair) * RL;  // query row of kv-head row 0
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int rr_lane = row_w0 + 16 * rt + n;
      row_ok[rt] = rr_lane < RL;
      const int rr = row_ok[rt] ? rr_lane : 0;
      const int l = rr % p.L;
      lim[rt] = !row_ok[rt] ? -1 : (p.causal ? static_cast<int>(len - p.L + l) : INT32_MAX);
      const u32x4_t* src = reinterpret_cast<const u32x4_t*>(p.qhl) + (pair_row0 + rr) * 32 + g;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        qh[rt][s] = src[4 * s];
        ql[rt][s] = src[16 + 4 * s];
      }
      qmul[rt] = p.qsq[pair_row0 + rr];
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const u32x4_t z = {0u, 0u, 0u, 0u};
        qh[rt][s] = row_ok[rt] ? qh[rt][s] : z;
        ql[rt][s] = row_ok[rt] ? ql[rt][s] : z;
      }
    }
  }
  // smallest causal limit over the wave's rows: sub-chunks past it take the slow path
  int lim_min = INT32_MAX;
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) lim_min = min(lim_min, row_ok[rt] ? lim[rt] : INT32_MAX);
  lim_min = min(lim_min, __shfl_xor(lim_min, 1, 64));
  lim_min = min(lim_min, __shfl_xor(lim_min, 2, 64));
  lim_min = min(lim_min, __shfl_xor(lim_min, 4, 64));
  lim_min = min(lim_min, __shfl_xor(lim_min, 8, 64));
  lim_min = __builtin_amdgcn_readfirstlane(lim_min);  // equal in every lane

  f32x4_t O[RT][8];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int ct = 0; ct < 8; ++ct) O[rt][ct] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m_row[RT];  // reference maximum of the row (log2 units)
  float l_acc[RT];  // this lane's share of the row's sum
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    m_row[rt] = -INFINITY;
    l_acc[rt] = 0.f;
  }
  int E = -126;  // value norms <= 2^E (weights carry 2^-E), shared by the wave's rows
  float vsc = ldexpf(1.f, 126);
  float vlim = ldexpf(1.f, -126);

  __syncthreads();  // codebooks in LDS
  float kmax = 0.f, vmax = 0.f;
#pragma unroll
  for (int i = 0; i < (1 << KB); ++i) kmax = fmaxf(kmax, fabsf(cbl[i]));
#pragma unroll
  for (int i = 0; i < (1 << VB); ++i) vmax = fmaxf(vmax, fabsf(cbl[16 + i]));
  const float sk = f16_split_scale(kmax);
  const float sv = f16_split_scale(vmax);
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) qmul[rt] = 1.4426950408889634f / (sk * qmul[rt]);  // log2 units (qmul held sq)
#pragma unroll
  for (int e = tid; e < S::KKEYS * S::REPK; e += kTileThreads) {
    const int key = e / S::REPK;
    uint32_t h0, l0, h1, l1;
    split_f16(cbl[key & ((1 << KB) - 1)] * sk, h0, l0);
    split_f16(cbl[key >> KB] * sk, h1, l1);
    *reinterpret_cast<uint2*>(lds + S::KTAB_OFF + e * 8) = make_uint2(h0 | (h1 << 16), l0 | (l1 << 16));
  }
#pragma unroll
  for (int e = tid; e < S::VKEYS * S::REPV; e += kTileThreads) {
    const int key = e / S::REPV;
    uint32_t h0, l0, h1, l1;
    split_f16(cbl[16 + (key & ((1 << VB) - 1))] * sv, h0, l0);
    split_f16(cbl[16 + (key >> VB)] * sv, h1, l1);
    *reinterpret_cast<uint2*>(lds + S::VTAB_OFF + e * 8) = make_uint2(h0 | (h1 << 16), l0 | (l1 << 16));
  }

  // ---- decode of one sub-chunk, by the four lead waves (which otherwise
  // wait at the step's barrier for the trailing ones): every lead thread does
  // 8 coordinates of two key rows and of two value rows.  Keys: thread
  // (token tid / 16 + 16 u, c8 = tid % 16), 16 lanes filling one 256-byte
  // row.  Values: wave w fills the 16-column blocks w and w + 4 (one KiB
  // each: lane (token lane / 2, half lane % 2)), so a wave's stores cover
  // every bank evenly.  All offsets are fixed per thread.
  static_assert(kTileNW == D / 16 && SUB == 32, "decode mapping: 4 lead waves x two 16-column blocks");
  const uint32_t ktab_lane = S::KTAB_OFF + (lane % S::REPK) * 8;
  const uint32_t vtab_lane = S::VTAB_OFF + (lane % S::REPV) * 8;
  const int kdt = (tid >> 4) & 15, kc8 = tid & 15;
  const int vdt = lane >> 1;
  const int vc8 = 2 * (wave & 3) + (lane & 1);  // 16-column blocks wave % 4 and wave % 4 + 4
  const uint32_t ks_off = S::STG_K + (kdt * S::PWK + ((8 * KB * kc8) >> 5)) * 4;
  const uint32_t dk_off = tile_kslot(kdt) * S::KROW + kc8 * 16;
  const uint32_t vs_off = S::STG_V + (vdt * S::PWV + ((8 * VB * vc8) >> 5)) * 4;
  const uint32_t dv_off = (vc8 >> 1) * S::VCT + tile_vslot(vdt) * 32 + (lane & 1) * 16;
  const int ksh = (8 * KB * kc8) & 31;
  const int vsh = (8 * VB * vc8) & 31;
  // the second unit (tokens + 16, blocks + 4) sits at fixed distances:
  // tile_kslot(t + 16) = tile_kslot(t) + 8, coordinates + 64 start 8 VB
  // bytes further in a value row with the same shift
  constexpr uint32_t kStepK = 16 * S::PWK * 4, kStepDK = 8 * S::KROW;
  constexpr uint32_t kStepV = 8 * VB, kStepDV = 4 * S::VCT;
  auto decode = [&](int sb, int db) {
    const unsigned char* st = lds + S::STG_OFF + sb * S::STG_BYTES;
    unsigned char* dc = lds + S::DEC_OFF + db * S::DEC_BYTES;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      // the word after a row's last one is still staging memory; its bits
      // land above the 8 * BITS used ones
      const uint32_t* wk = reinterpret_cast<const uint32_t*>(st + ks_off + u * kStepK);
      const uint32_t* wv = reinterpret_cast<const uint32_t*>(st + vs_off + u * kStepV);
      const uint32_t xk = __builtin_amdgcn_alignbit(wk[1], wk[0], ksh);
      const uint32_t xv = __builtin_amdgcn_alignbit(wv[1], wv[0], vsh);
      uint2 ek[4], ev[4];
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        ek[m] = lds_at<uint2>(lds, ktab_lane + ((xk >> (2 * m * KB)) & (S::KKEYS - 1u)) * (S::REPK * 8));
        ev[m] = lds_at<uint2>(lds, vtab_lane + ((xv >> (2 * m * VB)) & (S::VKEYS - 1u)) * (S::REPV * 8));
      }
      unsigned char* dk = dc + dk_off + u * kStepDK;
      unsigned char* dv = dc + dv_off + u * kStepDV;
      *reinterpret_cast<uint4*>(dk + S::DEC_KHI) = make_uint4(ek[0].x, ek[1].x, ek[2].x, ek[3].x);
      *reinterpret_cast<uint4*>(dk + S::DEC_KLO) = make_uint4(ek[0].y, ek[1].y, ek[2].y, ek[3].y);
      *reinterpret_cast<uint4*>(dv + S::DEC_VHI) = make_uint4(ev[0].x, ev[1].x, ev[2].x, ev[3].x);
      *reinterpret_cast<uint4*>(dv + S::DEC_VLO) = make_uint4(ev[0].y, ev[1].y, ev[2].y, ev[3].y);
    }
    if (tid < 2 * SUB)  // key norms then value norms (staged in that order)
      reinterpret_cast<float*>(dc + S::DEC_KN)[tid] = reinterpret_cast<const float*>(st + S::STG_KN)[tid];
  };

  // key-row reads (tile h, row n) and transposed value reads (half h)
  uint32_t ka[2], vtr[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    ka[h] = S::DEC_OFF + S::DEC_KHI + (16 * h + n) * S::KROW + 16 * g;
    vtr[h] = S::DEC_OFF + S::DEC_VHI + tile_vslot(8 * g + 4 * h + (n >> 2)) * 32 + (n & 3) * 8;
  }
  typedef __attribute__((address_space(3))) unsigned char lds_u8;
  typedef short s16x4v __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) s16x4v lds_s16x4;
  lds_u8* const l3 = (lds_u8*)lds;
  auto read_tr = [&](uint32_t off) {
    return __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(l3 + off)));
  };

  // S^T of sub-chunk in decoded slot DB (a compile-time slot)
  auto scores = [&](auto DB, f32x4_t (&C)[RT][2]) {
    constexpr uint32_t db = decltype(DB)::value * S::DEC_BYTES;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) C[rt][h] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const u32x4_t ah = lds_at<u32x4_t>(lds, ka[h] + db + 64 * s);
        const u32x4_t al = lds_at<u32x4_t>(lds, ka[h] + db + (S::DEC_KLO - S::DEC_KHI) + 64 * s);
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          C[rt][h] = mfma_f16(ah, qh[rt][s], C[rt][h]);
          C[rt][h] = mfma_f16(ah, ql[rt][s], C[rt][h]);
          C[rt][h] = mfma_f16(al, qh[rt][s], C[rt][h]);
        }
      }
    }
  };

  // softmax of sub-chunk i (decoded slot DB): the weights as A operands
  auto softmax = [&](int i, auto DB, const f32x4_t (&C)[RT][2], u32x4_t (&A)[RT]) {
    constexpr uint32_t db = decltype(DB)::value * S::DEC_BYTES;
    const unsigned char* dc = lds + S::DEC_OFF + db;
    const float4 kn0 = *reinterpret_cast<const float4*>(dc + S::DEC_KN + 32 * g);
    const float4 kn1 = *reinterpret_cast<const float4*>(dc + S::DEC_KN + 32 * g + 16);
    const float4 vn0 = *reinterpret_cast<const float4*>(dc + S::DEC_VN + 32 * g);
    const float4 vn1 = *reinterpret_cast<const float4*>(dc + S::DEC_VN + 32 * g + 16);
    const float knv[8] = {kn0.x, kn0.y, kn0.z, kn0.w, kn1.x, kn1.y, kn1.z, kn1.w};
    const float vnv[8] = {vn0.x, vn0.y, vn0.z, vn0.w, vn1.x, vn1.y, vn1.z, vn1.w};
    const int t0 = t_begin + i * SUB;  // tokens t0 + 8 g + j of this lane
    // y = n_t <q, c> in MFMA units of the row; x = y * qmul in log2 units
    float y[RT][8];
    float vm = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) vm = fmaxf(vm, vnv[j]);
    bool grow = vm > vlim;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      float ym = -INFINITY;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        y[rt][j] = own_reg(C[rt][j >> 2][j & 3]) * knv[j];
        ym = fmaxf(ym, y[rt][j]);
      }
      grow |= ym * qmul[rt] > m_row[rt] + kLazy;
    }
    const bool edge = t0 + SUB > t_end || t0 + SUB - 1 > lim_min;  // wave-uniform
    float pe[RT][8];
    if (edge || __any(grow ? 1 : 0)) {
      // slow path: masks, a new reference maximum or norm exponent, rescale
      const float vw = wave_max(vm);
      int e2 = E;
      if (vw > vlim) {
        int ev;
        frexpf(vw, &ev);
        e2 = ev;
      }
      const float esc = ldexpf(1.f, E - e2);
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        float x[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          x[j] = y[rt][j] * qmul[rt];
          if (edge) {
            const int tok = t0 + 8 * g + j;
            if (tok > lim[rt]) x[j] = -FLT_MAX;
            if (tok >= t_end) x[j] = -INFINITY;
          }
        }
        float rm = -INFINITY;
#pragma unroll
        for (int j = 0; j < 8; ++j) rm = fmaxf(rm, x[j]);
        rm = fmaxf(rm, xor_lane<16>(rm));
        {
          const float2 hh = halves(rm);
          rm = fmaxf(hh.x, hh.y);  // the row's maximum over the sub-chunk
        }
        const float mo = m_row[rt];
        const float mn = (mo == -INFINITY || rm > mo + kLazy) ? fmaxf(mo, rm) : mo;
        const float am = mo == mn ? 1.f : (mo == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mo - mn));
        const float ao = am * esc;
        l_acc[rt] *= am;
        // O rows 4 g + k of this lane take the factor of row 4 g + k
        float ar[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) ar[k] = __shfl(ao, 4 * g + k, 64);
#pragma unroll
        for (int ct = 0; ct < 8; ++ct)
#pragma unroll
          for (int k = 0; k < 4; ++k) O[rt][ct][k] *= ar[k];
        m_row[rt] = mn;
        // masked keys (-FLT_MAX) weigh 1 when their whole row is masked
        // (m = -FLT_MAX), else 0; keys past the end (-inf) always 0
#pragma unroll
        for (int j = 0; j < 8; ++j) pe[rt][j] = mn == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(x[j] - mn);
      }
      E = e2;
      vsc = ldexpf(1.f, -E);
      vlim = ldexpf(1.f, E);
    } else {
      // every score within 2^7 of a finite reference maximum
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        const float nm = -m_row[rt];
#pragma unroll
        for (int j = 0; j < 8; ++j) pe[rt][j] = __builtin_amdgcn_exp2f(__builtin_fmaf(y[rt][j], qmul[rt], nm));
      }
    }
    float vs[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) vs[j] = vnv[j] * vsc;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      float w[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        l_acc[rt] += pe[rt][j];
        w[j] = pe[rt][j] * vs[j];
      }
      A[rt] = u32x4_t{pack_f16x2(w[0], w[1]), pack_f16x2(w[2], w[3]), pack_f16x2(w[4], w[5]),
                      pack_f16x2(w[6], w[7])};
    }
  };

  // O += P V for the sub-chunk in decoded slot DB
  auto pv = [&](auto DB, const u32x4_t (&A)[RT]) {
    constexpr uint32_t db = decltype(DB)::value * S::DEC_BYTES;
#pragma unroll
    for (int ct = 0; ct < 8; ++ct) {
      const uint2 h0 = read_tr(vtr[0] + db + ct * S::VCT);
      const uint2 h1 = read_tr(vtr[1] + db + ct * S::VCT);
      const uint2 g0 = read_tr(vtr[0] + db + (S::DEC_VLO - S::DEC_VHI) + ct * S::VCT);
      const uint2 g1 = read_tr(vtr[1] + db + (S::DEC_VLO - S::DEC_VHI) + ct * S::VCT);
      const u32x4_t bh = {h0.x, h0.y, h1.x, h1.y};
      const u32x4_t bl = {g0.x, g0.y, g1.x, g1.y};
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        O[rt][ct] = mfma_f16(A[rt], bh, O[rt][ct]);
        O[rt][ct] = mfma_f16(A[rt], bl, O[rt][ct]);
      }
    }
  };

  // ---- prologue: sub-chunks 0 and 1 staged (slots 0, 1), 0 decoded (slot
  // 0), 2 and 3 loading.  Sub-chunk j's packed words wait in register set
  // j % 3 from step j - 4 (issued first in the step) to step j - 2 (staged
  // last); its staging and decoded slot is j % 3.
  store_stage(0, 0, rgt);
  if (ntiles > 1) store_stage(1, 1, rg1);
  __syncthreads();
  const bool lead = __builtin_amdgcn_readfirstlane(wave) < kTileNW / 2;
  if (lead) decode(0, 0);
  __syncthreads();

  const bool wave_live = __builtin_amdgcn_readfirstlane(row_w0) < RL;  // wave-uniform
  // step i (i % 3 == U): load i + 4 into set (i + 1) % 3, stage i + 2 from
  // set (i + 2) % 3.  Waves 0-3 ("lead") run scores -> softmax -> decode of
  // i + 1 (past the last sub-chunk: stale staging, never read) -> P V of
  // sub-chunk i; waves 4-7 ("trail", the other wave on each SIMD) run
  // P V of sub-chunk i - 1 -> scores -> softmax of i, so that one wave's
  // vector work tends to meet the other's matrix products rather than its
  // own kind.  A trailing wave keeps sub-chunk i - 1's weights in Ap over
  // the barrier; slot (i - 1) % 3 is rewritten only in step i + 1.
  auto step_lead = [&](int i, auto U, uint32_t (&lset)[S::LOADS], uint32_t (&sset)[S::LOADS]) {
    constexpr int u = decltype(U)::value;
    using Cur = std::integral_constant<int, u>;
    if (i + 4 < ntiles) load_tile(i + 4, lset);
    f32x4_t C[RT][2];
    u32x4_t A[RT];
    if (wave_live) {
      scores(Cur{}, C);
      softmax(i, Cur{}, C, A);
    }
    decode((u + 1) % 3, (u + 1) % 3);
    if (wave_live) pv(Cur{}, A);
    if (i + 2 < ntiles) store_stage((u + 2) % 3, i + 2, sset);
    __syncthreads();
  };
  u32x4_t Ap[RT];
  auto step_trail = [&](int i, auto U, uint32_t (&lset)[S::LOADS], uint32_t (&sset)[S::LOADS]) {
    constexpr int u = decltype(U)::value;
    using Cur = std::integral_constant<int, u>;
    using Prev = std::integral_constant<int, (u + 2) % 3>;
    if (i + 4 < ntiles) load_tile(i + 4, lset);
    f32x4_t C[RT][2];
    if (wave_live && i > 0) pv(Prev{}, Ap);
    if (wave_live) scores(Cur{}, C);
    if (wave_live) softmax(i, Cur{}, C, Ap);
    if (i + 2 < ntiles) store_stage((u + 2) % 3, i + 2, sset);
    __syncthreads();
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  if (lead) {
#pragma unroll 1
    for (int i = 0; i < ntiles; i += 3) {
      step_lead(i, I0{}, rg1, rg2);
      if (i + 1 < ntiles) step_lead(i + 1, I1{}, rg2, rg0);
      if (i + 2 < ntiles) step_lead(i + 2, I2{}, rg0, rg1);
    }
  } else {
#pragma unroll 1
    for (int i = 0; i < ntiles; i += 3) {
      step_trail(i, I0{}, rg1, rg2);
      if (i + 1 < ntiles) step_trail(i + 1, I1{}, rg2, rg0);
      if (i + 2 < ntiles) step_trail(i + 2, I2{}, rg0, rg1);
    }
    if (wave_live) {  // the last sub-chunk's P V
      switch ((ntiles - 1) % 3) {
        case 0: pv(I0{}, Ap); break;
        case 1: pv(I1{}, Ap); break;
        default: pv(I2{}, Ap); break;
      }
    }
  }
  // ---- partials: (o, m, l) per row, o = O * 2^E / sv in the rotated basis
  if (!wave_live) return;
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    float lr = l_acc[rt] + xor_lane<16>(l_acc[rt]);
    {
      const float2 h = halves(lr);
      lr = h.x + h.y;
    }
    const int rr_lane = row_w0 + 16 * rt + n;
    if (g == 0 && row_ok[rt]) {
      float* pm = p.pml + ((grp0 + rr_lane / 8) * p.n_splits + split) * 16 + (rr_lane % 8) * 2;
      pm[0] = m_row[rt] * 0.6931471805599453f;  // natural-log units
      pm[1] = lr;
    }
  }
  const float osc = ldexpf(1.f, E) / sv;
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int rr = row_w0 + 16 * rt + 4 * g + k;
      if (rr >= RL) continue;
      float* po = p.po + (((grp0 + rr / 8) * p.n_splits + split) * 8 + rr % 8) * static_cast<int64_t>(D);
#pragma unroll
      for (int ct = 0; ct < 8; ++ct) po[16 * ct + n] = O[rt][ct][k] * osc;
    }
}

// Coordinates 16 g8 + j (register j) of one query row from element offset
// qo (lane group g8's first coordinate): round_DT(q * scale) times the
// Hadamard signs, all loads issued before the first use.
template <int DT>
__device__ __forceinline__ void tile_q_signed(const void* q, int64_t qo, float scale, const float (&kr)[16],
                                              float (&qv)[16]) {
  if constexpr (DT == TQ_DTYPE_F32) {
    const float* qp = static_cast<const float*>(q) + qo;
#pragma unroll
    for (int e = 0; e < 16; ++e) qv[e] = qp[e];
  } else {
    const uint16_t* qp = static_cast<const uint16_t*>(q) + qo;
    uint16_t raw[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) raw[e] = qp[e];
#pragma unroll
    for (int e = 0; e < 16; ++e)
      qv[e] = DT == TQ_DTYPE_F16 ? f16_bits_to_f32(raw[e]) : bf16_bits_to_f32(raw[e]);
  }
#pragma unroll
  for (int e = 0; e < 16; ++e) qv[e] = round_to<DT>(qv[e] * scale) * kr[e];
}

// Query rows for the tile kernel, once per row rather than once per split:
// q_rot (the Hadamard transform here, or the dense transform's rows from the
// workspace), times sq (a power of two putting the row's largest magnitude
// in [2^12, 2^13)), split into hi and lo f16 parts and stored in the order
// the tile kernel's B operands take them: row-major, per row 16 hi words of
// 8 halves (word 4 s + g holds coordinates 32 s + 8 g .. + 7), then 16 lo.
// Wave = 8 consecutive query rows, lane (row n8 = lane % 8, g8 = lane / 8)
// holds coordinates 16 g8 + j in register j: butterflies over coordinate
// bits 0-3 in registers, bits 4-6 across lanes (lane bits 3-5).  A lane
// stores words 2 g8, 2 g8 + 1 of both halves (32 contiguous bytes each).
constexpr int kTileQpThreads = 256;
constexpr int kTileQpRows = 8;  // query rows per wave

__global__ __launch_bounds__(kTileQpThreads) void gen_tile_qprep_kernel(GenParams p, int rows) {
  const int lane = threadIdx.x & 63;
  const int n8 = lane & 7;
  const int g8 = lane >> 3;
  const int row0 = (blockIdx.x * (kTileQpThreads / 64) + (threadIdx.x >> 6)) * kTileQpRows;
  if (__builtin_amdgcn_readfirstlane(row0) >= rows) return;  // whole wave past the end
  const int row = row0 + n8;
  const bool ok = row < rows;
  const int qrow = ok ? row : 0;
  float qv[16];
  if (p.k_rot_kind == TQ_ROT_HADAMARD) {
    float kr[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) kr[e] = p.krot[16 * g8 + e];
    const int l = qrow % p.L;
    const int bh = qrow / p.L;
    const int h = bh % p.Hq;
    const int b = bh / p.Hq;
    const int64_t qo = static_cast<int64_t>(b) * p.q_sb + static_cast<int64_t>(h) * p.q_sh +
                       static_cast<int64_t>(l) * p.q_sl + 16 * g8;
    switch (p.q_dtype) {
      case TQ_DTYPE_F32: tile_q_signed<TQ_DTYPE_F32>(p.q, qo, p.scale_q, kr, qv); break;
      case TQ_DTYPE_F16: tile_q_signed<TQ_DTYPE_F16>(p.q, qo, p.scale_q, kr, qv); break;
      default: tile_q_signed<TQ_DTYPE_BF16>(p.q, qo, p.scale_q, kr, qv); break;
    }
#pragma unroll
    for (int hb = 1; hb < 16; hb <<= 1)
#pragma unroll
      for (int e = 0; e < 16; ++e)
        if ((e & hb) == 0) {
          const float a0 = qv[e], a1 = qv[e + hb];
          qv[e] = a0 + a1;
          qv[e + hb] = a0 - a1;
        }
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      float v = qv[e];
      float o = xor_lane<8>(v);
      v = (g8 & 1) ? o - v : v + o;
      o = xor_lane<16>(v);
      v = (g8 & 2) ? o - v : v + o;
      const float2 hv = halves(v);  // lanes < 32: (v, v[l + 32]); others (v[l - 32], v)
      v = (g8 & 4) ? hv.x - hv.y : hv.x + hv.y;
      qv[e] = v * p.rscale_k;
    }
  } else {
    const float* qp = p.qrot + static_cast<int64_t>(qrow) * p.DkP + 16 * g8;
#pragma unroll
    for (int e = 0; e < 16; ++e) qv[e] = qp[e];
  }
  float mx = 0.f;
#pragma unroll
  for (int e = 0; e < 16; ++e) mx = fmaxf(mx, fabsf(qv[e]));
  mx = fmaxf(mx, xor_lane<8>(mx));
  mx = fmaxf(mx, xor_lane<16>(mx));
  {
    const float2 hv = halves(mx);
    mx = fmaxf(hv.x, hv.y);  // the row's largest magnitude
  }
  const float sq = f16_split_scale(mx);
  if (!ok) return;
  u32x4_t* dst = reinterpret_cast<u32x4_t*>(p.qhl) + static_cast<int64_t>(row) * 32 + 2 * g8;
#pragma unroll
  for (int w = 0; w < 2; ++w) {
    uint32_t hw[4], lw[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t h0, l0, h1, l1;
      split_f16(qv[8 * w + 2 * j] * sq, h0, l0);
      split_f16(qv[8 * w + 2 * j + 1] * sq, h1, l1);
      hw[j] = h0 | (h1 << 16);
      lw[j] = l0 | (l1 << 16);
    }
    dst[w] = u32x4_t{hw[0], hw[1], hw[2], hw[3]};
    dst[16 + w] = u32x4_t{lw[0], lw[1], lw[2], lw[3]};
  }
  if (g8 == 0) p.qsq[row] = sq;
}

}  // namespace tq
