// Append-time kernels: TurboQuant quantize + pack (randomized Hadamard),
// unquantized append for the fp16/bf16 layers, and dequantize.
//
// Quantize follows _TurboQuantMSECodec.quantize (turboquant_cache.py:4186-4254)
// with one fixed fp32 operation order that the CPU oracle reproduces bit for
// bit:
//   * lane g of a vector owns elements [32g, 32g+32) (D/32 lanes per vector);
//   * ||x||^2: a lane squares its 32 elements and folds them at distances
//     16, 8, 4, 2, 1, then lanes combine by xor-butterfly 1, 2, 4 ...;
//   * n = sqrt (IEEE, correctly rounded), u = x / max(n, 1e-6) (IEEE division);
//   * Walsh-Hadamard butterflies at distances 1, 2, ..., D/2, each mapping
//     (a, b) -> (a + b, a - b); distances < 32 run inside a lane, the rest
//     across lanes with shuffles;
//   * y = v * f32(1/sqrt(D)); idx = #{m : y > mid[m]} (strict compare);
//   * a lane's 32 indices fill exactly `bits` consecutive words of the
//     LSB-first stream, so packing is thread-local (no shared-word races).
#include <type_traits>

#include "tq_append.h"

namespace tq {

// 32 consecutive input elements as loaded (16-byte pieces), converted to f32
// by widen32 once they are needed.
template <int DT>
struct Raw32 {
  static constexpr int N = DT == TQ_DTYPE_F32 ? 8 : 4;
  uint4 w[N];
};

__device__ __forceinline__ uint32_t u4_word(const uint4& u, int k) {
  return k == 0 ? u.x : (k == 1 ? u.y : (k == 2 ? u.z : u.w));
}

template <int DT>
__device__ __forceinline__ void load_raw32(const void* p, Raw32<DT>& r) {
  const uint4* q = static_cast<const uint4*>(p);
#pragma unroll
  for (int i = 0; i < Raw32<DT>::N; ++i) r.w[i] = q[i];
}

template <int DT>
__device__ __forceinline__ void widen32(const Raw32<DT>& r, float (&v)[32]) {
#pragma unroll
  for (int i = 0; i < Raw32<DT>::N; ++i) {
    const uint32_t w[4] = {r.w[i].x, r.w[i].y, r.w[i].z, r.w[i].w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if constexpr (DT == TQ_DTYPE_F32) {
        v[4 * i + j] = __uint_as_float(w[j]);
      } else {
        const uint16_t lo = static_cast<uint16_t>(w[j] & 0xffffu);
        const uint16_t hi = static_cast<uint16_t>(w[j] >> 16);
        v[8 * i + 2 * j] = DT == TQ_DTYPE_F16 ? f16_bits_to_f32(lo) : bf16_bits_to_f32(lo);
        v[8 * i + 2 * j + 1] = DT == TQ_DTYPE_F16 ? f16_bits_to_f32(hi) : bf16_bits_to_f32(hi);
      }
    }
  }
}

// v[I0 .. I0 + 7] += c * (the same register of lane ^ OFF): one v_fmac_f32 per
// element, its first source read from the partner lane through DPP.  c is +-1,
// so the product is exact and each result is one rounding of the sum.  A DPP
// source needs two wait states after a VALU write of its register, and the
// compiler does not look inside the block: hence the s_nop 1 on either side.
#define TQ_FMAC_DPP8(CTRL)                                                                   \
  asm("s_nop 1\n\t"                                                                          \
      "v_fmac_f32_dpp %0, %0, %8 " CTRL "\n\t"                                               \
      "v_fmac_f32_dpp %1, %1, %8 " CTRL "\n\t"                                               \
      "v_fmac_f32_dpp %2, %2, %8 " CTRL "\n\t"                                               \
      "v_fmac_f32_dpp %3, %3, %8 " CTRL "\n\t"                                               \
      "v_fmac_f32_dpp %4, %4, %8 " CTRL "\n\t"                                               \
      "v_fmac_f32_dpp %5, %5, %8 " CTRL "\n\t"                                               \
      "v_fmac_f32_dpp %6, %6, %8 " CTRL "\n\t"                                               \
      "v_fmac_f32_dpp %7, %7, %8 " CTRL "\n\t"                                               \
      "s_nop 1"                                                                              \
      : "+v"(v[I0]), "+v"(v[I0 + 1]), "+v"(v[I0 + 2]), "+v"(v[I0 + 3]), "+v"(v[I0 + 4]),   \
        "+v"(v[I0 + 5]), "+v"(v[I0 + 6]), "+v"(v[I0 + 7])                                    \
      : "v"(c))

template <int OFF, int I0>
__device__ __forceinline__ void fmac_xor8(float (&v)[32], float c) {
  static_assert(OFF == 1 || OFF == 2 || OFF == 8, "one-instruction DPP lane xor");
  if constexpr (OFF == 1) {
    TQ_FMAC_DPP8("quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf");
  } else if constexpr (OFF == 2) {
    TQ_FMAC_DPP8("quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf");
  } else {
    TQ_FMAC_DPP8("row_ror:8 row_mask:0xf bank_mask:0xf");
  }
}
#undef TQ_FMAC_DPP8

// One block's share of a quantize launch: vectors [block * VPB, block * VPB + VPB)
// of a (256 threads).  Shared by the one-tensor and the key + value kernels.
//
// Signs.  Multiplying by s_i = +-1 commutes exactly with the division by the
// norm (IEEE division is sign-symmetric), so the signs are applied to the raw
// input as sign-bit xors (two f16 / bf16 elements per instruction).  The same
// xor also flips lane g's elements by (-1)^popcount(g): with that flip, every
// cross-lane butterfly stage becomes v + c * partner with c = -1 on the lower
// lane of a pair and +1 on the upper one (one DPP fma per element), and every
// lane ends with the unflipped value.  Proof by induction over the stages: a
// lane entering the stage of lane bit j holds its value times
// (-1)^popcount(g >> j), and its partner the opposite sign, so the lower lane
// forms a + b and the upper a - b times the lane's incoming sign, which is
// (-1)^popcount(g >> (j + 1)) for both.  Results are bit-identical (rounding
// to nearest is symmetric); at most the sign of a zero differs, which no
// compare against a midpoint sees.  A sign vector with an entry other than
// +-1 makes the block multiply by it after the division instead.
template <int D, int BITS, int XDT>
__device__ __forceinline__ void rht_quantize_block(const AppendArgs& a, int64_t block) {
  constexpr int NL = D / 32;          // lanes per vector
  constexpr int VPB = 256 / NL;       // vectors per block
  constexpr int NMID = (1 << BITS) - 1;
  constexpr int PW = D * BITS / 32;
  constexpr bool LUT = NMID > 3;  // bucket table beyond three midpoints
  constexpr int EPW = XDT == TQ_DTYPE_F32 ? 1 : 2;  // elements per sign word
  constexpr int SW = D / EPW;                        // sign words
  constexpr int SPT = (SW + 255) / 256;              // sign words per thread
  __shared__ __align__(16) uint32_t s_smask[SW];
  __shared__ float s_mid[NMID];
  __shared__ float s_thr[LUT ? NMID : 1];  // the midpoints moved before the scale (unscaled_threshold)
  __shared__ uint2 s_qb[LUT ? kQbN : 1];
  __shared__ int s_bad;  // bit 0: a sign is not +-1; bit 1: no exact table

  // The block's small constants are requested first, then this lane's 32
  // input elements; the table set-up below runs while the rows are in flight.
  float sgn[SPT][EPW];
#pragma unroll
  for (int k = 0; k < SPT; ++k) {
    const int w = threadIdx.x + 256 * k;
#pragma unroll
    for (int j = 0; j < EPW; ++j) sgn[k][j] = w < SW ? a.rot[w * EPW + j] : 1.f;
  }
  const float mid_t = threadIdx.x < NMID ? a.mid[threadIdx.x] : 0.f;

  const int64_t n_vec = static_cast<int64_t>(a.B) * a.H * a.L;
  const int tv = threadIdx.x / NL;
  const int64_t vec = block * VPB + tv;
  const int g = threadIdx.x % NL;
  const bool live = vec < n_vec;
  int l, h, b;
  if (a.L % VPB == 0) {
    // the block's vectors share one (b, h) row and are all live: the
    // divisions are the block's, on uniform values
    const int64_t bh = (block * VPB) / a.L;
    l = static_cast<int>(block * VPB - bh * a.L) + tv;
    h = static_cast<int>(bh % a.H);
    b = static_cast<int>(bh / a.H);
  } else {
    // lanes past the last vector load vector 0 (launches have n_vec >= 1) and
    // drop it: unconditional loads keep the wait counts exact
    const int64_t vl = live ? vec : 0;
    l = static_cast<int>(vl % a.L);
    const int64_t bh = vl / a.L;
    h = static_cast<int>(bh % a.H);
    b = static_cast<int>(bh / a.H);
  }
  constexpr int ES = XDT == TQ_DTYPE_F32 ? 4 : 2;
  Raw32<XDT> raw;
  load_raw32<XDT>(static_cast<const char*>(a.x) + (b * a.sb + h * a.sh + l * a.sl + g * 32) * ES, raw);

  int bad = 0;
#pragma unroll
  for (int k = 0; k < SPT; ++k) {
    const int w = threadIdx.x + 256 * k;
    uint32_t m = 0;
#pragma unroll
    for (int j = 0; j < EPW; ++j) {
      const int e = w * EPW + j;
      bad |= fabsf(sgn[k][j]) != 1.f ? 1 : 0;
      const bool flip = (sgn[k][j] < 0.f) != ((__popc(static_cast<uint32_t>(e) >> 5) & 1) != 0);
      m |= flip ? (EPW == 1 ? 0x80000000u : (0x8000u << (16 * j))) : 0u;
    }
    if (w < SW) s_smask[w] = m;
  }
  if (threadIdx.x == 0) s_bad = 0;
  if constexpr (LUT) {
    // the table indexes the Hadamard output v before the scale: v > T_m
    // exactly when RN(v * scale) > mid_m
    if (threadIdx.x < NMID) {
      float T = 0.f;
      if (!unscaled_threshold(mid_t, a.scale, T)) bad |= 2;
      s_thr[threadIdx.x] = T;
    }
  }
  if (threadIdx.x < NMID) s_mid[threadIdx.x] = mid_t;
  append_lds_barrier();
  if (bad) atomicOr(&s_bad, bad);
  QbGrid grid{};
  if constexpr (LUT) {
    grid = qb_grid(s_thr[0], s_thr[NMID - 1]);
    for (int t = threadIdx.x; t < kQbN; t += blockDim.x) {
      uint2 ent;
      if (!qb_entry_grid(static_cast<uint32_t>(t), s_thr, NMID, grid, ent)) atomicOr(&s_bad, 2);
      s_qb[t] = ent;
    }
  }
  append_lds_barrier();
  const int bad_all = s_bad;
  const bool sign_mul = (bad_all & 1) != 0;
  const bool use_lut = LUT && (bad_all & 2) == 0 && grid.ok;

  // Every lane of a vector shares `vec`, so a vector's lanes leave together
  // and the xor-shuffles below stay inside live lane groups.
  if (!live) return;
  {
    const uint32_t flip0 = (__popc(static_cast<uint32_t>(g)) & 1) ? (EPW == 1 ? 0x80000000u : 0x80008000u) : 0u;
    const uint4* mk = reinterpret_cast<const uint4*>(s_smask) + g * Raw32<XDT>::N;
#pragma unroll
    for (int i = 0; i < Raw32<XDT>::N; ++i) {
      const uint4 m = sign_mul ? make_uint4(flip0, flip0, flip0, flip0) : mk[i];
      raw.w[i].x ^= m.x;
      raw.w[i].y ^= m.y;
      raw.w[i].z ^= m.z;
      raw.w[i].w ^= m.w;
    }
  }
  float v[32];
  if constexpr (XDT != TQ_DTYPE_F16) widen32<XDT>(raw, v);

  // ---- norm: in-lane fold 16, 8, 4, 2, 1 then cross-lane xor butterfly.  The
  // square of an f16 value is exact in f32 (22 significand bits, exponent in
  // range), so the first fold's RN(a^2 + RN(b^2)) equals RN(RN(a^2) + RN(b^2)).
  float s[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    if constexpr (XDT == TQ_DTYPE_F16) {
      // element i is half (i & 1) of word i / 2 of the lane's 16 (raw.w[i / 8])
      const uint32_t wa = u4_word(raw.w[i / 8], (i / 2) % 4), wb = u4_word(raw.w[(i + 16) / 8], ((i + 16) / 2) % 4);
      const float a0 = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>((i & 1) ? (wa >> 16) : wa)));
      const float b0 = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>((i & 1) ? (wb >> 16) : wb)));
      s[i] = __builtin_fmaf(a0, a0, __builtin_fmaf(b0, b0, 0.f));  // b^2 >= 0: adding +0 keeps it
    } else {
      s[i] = __fadd_rn(__fmul_rn(v[i], v[i]), __fmul_rn(v[i + 16], v[i + 16]));
    }
  }
#pragma unroll
  for (int w = 8; w >= 1; w >>= 1) {
#pragma unroll
    for (int i = 0; i < w; ++i) s[i] = __fadd_rn(s[i], s[i + w]);
  }
  float ss = s[0];
  if constexpr (NL >= 2) ss = __fadd_rn(ss, xor_lane<1>(ss));
  if constexpr (NL >= 4) ss = __fadd_rn(ss, xor_lane<2>(ss));
  if constexpr (NL >= 8) ss = __fadd_rn(ss, xor_lane<4>(ss));
  if constexpr (NL >= 16) ss = __fadd_rn(ss, xor_lane<8>(ss));
  const float n = sqrt_rn(ss);
  const float den = fmaxf(n, kNormEps);

  // ---- normalise (IEEE x / den, div_by_norm); the signs are already in.
  // f16 input: the two fmas that read x take it as an f16 source straight
  // from the packed words (v_fma_mix_f32, either half), so no element is
  // converted on its own; q = fma(x, r, +0) is RN(x r) for every x != 0 (x r
  // is a normal number), and for x = +-0 both forms end in u = +0.
  if constexpr (XDT == TQ_DTYPE_F16) {
    const float r = __fdiv_rn(1.f, den);
#pragma unroll
    for (int i = 0; i < Raw32<XDT>::N; ++i) {
      const uint32_t w[4] = {raw.w[i].x, raw.w[i].y, raw.w[i].z, raw.w[i].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float q0, q1, e0, e1;
        asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel:[0,0,0] op_sel_hi:[1,0,0]" : "=v"(q0) : "v"(w[j]), "v"(r));
        asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(q1) : "v"(w[j]), "v"(r));
        asm("v_fma_mix_f32 %0, -%1, %2, %3 op_sel:[0,0,0] op_sel_hi:[0,0,1]" : "=v"(e0) : "v"(q0), "v"(den), "v"(w[j]));
        asm("v_fma_mix_f32 %0, -%1, %2, %3 op_sel:[0,0,1] op_sel_hi:[0,0,1]" : "=v"(e1) : "v"(q1), "v"(den), "v"(w[j]));
        v[8 * i + 2 * j] = __builtin_fmaf(e0, r, q0);
        v[8 * i + 2 * j + 1] = __builtin_fmaf(e1, r, q1);
      }
    }
  } else {
    div_by_norm<XDT>(v, den, v);
  }
  if (sign_mul) {
#pragma unroll
    for (int i = 0; i < 32; ++i) v[i] = __fmul_rn(v[i], a.rot[g * 32 + i]);
  }

  // ---- Walsh-Hadamard: in-lane stages (distance 1..16)
#pragma unroll
  for (int hstep = 1; hstep < 32; hstep <<= 1) {
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      if ((i & hstep) == 0) {
        const float x0 = v[i];
        const float x1 = v[i + hstep];
        v[i] = __fadd_rn(x0, x1);
        v[i + hstep] = __fsub_rn(x0, x1);
      }
    }
  }
  // ---- cross-lane stages (distance 32, 64, ...): lane bit j <-> element bit
  // 5 + j; v + c * partner with c = -1 on the lower lane, +1 on the upper
  auto cross = [&](auto off_tag) {
    constexpr int OFF = decltype(off_tag)::value;
    const float c = (g & OFF) != 0 ? 1.f : -1.f;
    if constexpr (OFF == 1 || OFF == 2 || OFF == 8) {
      fmac_xor8<OFF, 0>(v, c);
      fmac_xor8<OFF, 8>(v, c);
      fmac_xor8<OFF, 16>(v, c);
      fmac_xor8<OFF, 24>(v, c);
    } else {
#pragma unroll
      for (int i = 0; i < 32; ++i) v[i] = __builtin_fmaf(xor_lane<OFF>(v[i]), c, v[i]);
    }
  };
  if constexpr (NL >= 2) cross(std::integral_constant<int, 1>{});
  if constexpr (NL >= 4) cross(std::integral_constant<int, 2>{});
  if constexpr (NL >= 8) cross(std::integral_constant<int, 4>{});
  if constexpr (NL >= 16) cross(std::integral_constant<int, 8>{});

  // ---- quantize against midpoints, pack thread-locally (one shift-or per
  // index: v_lshl_or_b32)
  uint32_t words[BITS];
  auto pack_all = [&](auto idx_of) {
    // all indices first (the table reads batch), then the shift-ors
    uint32_t ix[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) ix[i] = idx_of(v[i]);
#pragma unroll
    for (int w = 0; w < BITS; ++w) words[w] = 0u;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      const uint32_t idx = ix[i];
      const int pos = i * BITS;
      const int wi = pos >> 5;
      const int sh = pos & 31;
      asm("v_lshl_or_b32 %0, %1, %2, %3" : "=v"(words[wi]) : "v"(idx), "i"(sh), "v"(words[wi]));
      if (sh + BITS > 32) words[wi + 1] |= idx >> (32 - sh);
    }
  };
  // a NaN / infinite norm makes every y NaN, and NaN compares below every midpoint
  if (use_lut && n < INFINITY) {
    pack_all([&](float x) -> uint32_t {
      const uint2 ent = s_qb[qb_cell(x, grid)];
      return ent.x + ((x > __uint_as_float(ent.y)) ? 1u : 0u);
    });
  } else {
    pack_all([&](float x) -> uint32_t {
      const float y = __fmul_rn(x, a.scale);
      uint32_t idx = 0;
#pragma unroll
      for (int m = 0; m < NMID; ++m) idx += (y > s_mid[m]) ? 1u : 0u;
      return idx;
    });
  }

  const int64_t row = (static_cast<int64_t>(b) * a.H + h) * a.cap + a.offset + l;
  uint32_t* dst = a.packed + row * PW + g * BITS;
#pragma unroll
  for (int w = 0; w < BITS; ++w) dst[w] = words[w];
  if (g == 0) {
    if (a.norm_dtype == TQ_DTYPE_F16)
      static_cast<uint16_t*>(a.norms)[row] = f32_to_f16_bits(n);
    else
      static_cast<float*>(a.norms)[row] = n;
  }
}

template <int D, int BITS, int XDT>
__global__ __launch_bounds__(256) void append_rht_kernel(AppendArgs a) {
  rht_quantize_block<D, BITS, XDT>(a, blockIdx.x);
}

// Keys and values of one update_and_fetch in one launch: blocks below
// k_blocks quantize the keys, the rest the values (each block one side, so
// the branch is uniform).  One launch instead of two halves the fixed cost
// (launch, first-load latency, tail) of a decode or prefill append.
template <int D, int KBITS, int VBITS, int XDT>
__global__ __launch_bounds__(256) void append_rht_kv_kernel(AppendArgs k, AppendArgs v, int64_t k_blocks) {
  const bool key = static_cast<int64_t>(blockIdx.x) < k_blocks;
  if constexpr (KBITS == VBITS) {
    // one copy of the body for both sides (the side's arguments picked
    // first): half the code for the instruction cache
    rht_quantize_block<D, KBITS, XDT>(key ? k : v, key ? blockIdx.x : blockIdx.x - k_blocks);
  } else {
    if (key)
      rht_quantize_block<D, KBITS, XDT>(k, blockIdx.x);
    else
      rht_quantize_block<D, VBITS, XDT>(v, blockIdx.x - k_blocks);
  }
}

// ------------------------------------------------------------------ plain ---
struct PlainArgs {
  const uint16_t* x;
  int64_t sb, sh, sl;
  int B, H, L, D;
  uint16_t* dst;
  int64_t cap, offset;
};

// One thread copies 8 elements (16 bytes); D is a multiple of 8 and the rows
// are 16-byte aligned.  Index type I: 32-bit when the piece count fits, so
// the index divisions are not 64-bit ones.
template <typename I>
__global__ __launch_bounds__(256) void append_plain_kernel(PlainArgs a) {
  const I per_row = static_cast<I>(a.D / 8);
  const I total = static_cast<I>(a.B) * a.H * a.L * per_row;
  const I i = static_cast<I>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int c = static_cast<int>(i % per_row);
  const I vec = i / per_row;
  const int l = static_cast<int>(vec % static_cast<I>(a.L));
  const I bh = vec / static_cast<I>(a.L);
  const int h = static_cast<int>(bh % static_cast<I>(a.H));
  const int b = static_cast<int>(bh / static_cast<I>(a.H));
  const uint4* src = reinterpret_cast<const uint4*>(a.x + b * a.sb + h * a.sh + l * a.sl) + c;
  uint4* dst = reinterpret_cast<uint4*>(
                   a.dst + ((static_cast<int64_t>(b) * a.H + h) * a.cap + a.offset + l) * a.D) +
               c;
  *dst = *src;
}

// Any other dim or alignment: one thread per element.
__global__ __launch_bounds__(256) void append_plain_elem_kernel(PlainArgs a) {
  const int64_t total = static_cast<int64_t>(a.B) * a.H * a.L * a.D;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int d = static_cast<int>(i % a.D);
  const int64_t vec = i / a.D;
  const int l = static_cast<int>(vec % a.L);
  const int64_t bh = vec / a.L;
  const int h = static_cast<int>(bh % a.H);
  const int b = static_cast<int>(bh / a.H);
  a.dst[((static_cast<int64_t>(b) * a.H + h) * a.cap + a.offset + l) * a.D + d] =
      a.x[b * a.sb + h * a.sh + l * a.sl + d];
}

// ------------------------------------------------------------- dequantize ---
struct DequantArgs {
  const uint32_t* packed;
  const void* norms;
  int norm_dtype;
  int B, H, T, D, bits, PW;
  int64_t cap;
  const float* cb;
  int rot_kind;
  const float* rot;
  float scale;
  float* out;
};

// One block per vector; D threads (64..256).  Test/API path, not hot.
__global__ __launch_bounds__(256) void dequant_kernel(DequantArgs a) {
  __shared__ float y[256];
  const int64_t vec = blockIdx.x;  // (b*H + h)*T + t
  const int t = static_cast<int>(vec % a.T);
  const int64_t bh = vec / a.T;
  const int64_t row = bh * a.cap + t;
  const int i = threadIdx.x;
  const uint32_t* w = a.packed + row * a.PW;
  const int pos = i * a.bits;
  uint32_t idx = w[pos >> 5] >> (pos & 31);
  if ((pos & 31) + a.bits > 32) idx |= w[(pos >> 5) + 1] << (32 - (pos & 31));
  idx &= (1u << a.bits) - 1u;
  y[i] = a.cb[idx];
  __syncthreads();
  float r;
  if (a.rot_kind == TQ_ROT_HADAMARD) {
    for (int hstep = 1; hstep < a.D; hstep <<= 1) {
      float mine = y[i];
      float other = y[i ^ hstep];
      __syncthreads();
      y[i] = (i & hstep) ? __fsub_rn(other, mine) : __fadd_rn(mine, other);
      __syncthreads();
    }
    r = __fmul_rn(__fmul_rn(y[i], a.scale), a.rot[i]);
  } else {
    // x = y @ R : x[i] = sum_j y[j] R[j][i]
    float acc = 0.f;
    for (int j = 0; j < a.D; ++j) acc = fmaf(y[j], a.rot[static_cast<int64_t>(j) * a.D + i], acc);
    r = acc;
  }
  const float nrm = load_norm(a.norms, a.norm_dtype, row);
  a.out[vec * a.D + i] = nrm * r;
}

}  // namespace tq

using namespace tq;

namespace {

template <int D, int BITS>
int launch_append_rht_bits(int x_dtype, const AppendArgs& a, hipStream_t st) {
  constexpr int NL = D / 32;
  constexpr int VPB = 256 / NL;
  const int64_t n_vec = static_cast<int64_t>(a.B) * a.H * a.L;
  const int64_t blocks = (n_vec + VPB - 1) / VPB;
  if (blocks > 0x7fffffff) return fail(TQ_ERR_INVALID_ARGUMENT, "append: too many vectors");
  dim3 grid(static_cast<unsigned>(blocks));
  switch (x_dtype) {
    case TQ_DTYPE_F32:
      hipLaunchKernelGGL((append_rht_kernel<D, BITS, TQ_DTYPE_F32>), grid, dim3(256), 0, st, a);
      break;
    case TQ_DTYPE_F16:
      hipLaunchKernelGGL((append_rht_kernel<D, BITS, TQ_DTYPE_F16>), grid, dim3(256), 0, st, a);
      break;
    case TQ_DTYPE_BF16:
      hipLaunchKernelGGL((append_rht_kernel<D, BITS, TQ_DTYPE_BF16>), grid, dim3(256), 0, st, a);
      break;
    default:
      return fail(TQ_ERR_INVALID_ARGUMENT, "append: x_dtype %d", x_dtype);
  }
  return check_launch("append_rht_kernel");
}

template <int D>
int launch_append_rht(int bits, int x_dtype, const AppendArgs& a, hipStream_t st) {
  switch (bits) {
    case 1: return launch_append_rht_bits<D, 1>(x_dtype, a, st);
    case 2: return launch_append_rht_bits<D, 2>(x_dtype, a, st);
    case 3: return launch_append_rht_bits<D, 3>(x_dtype, a, st);
    case 4: return launch_append_rht_bits<D, 4>(x_dtype, a, st);
  }
  return fail(TQ_ERR_INVALID_ARGUMENT, "append: bits %d not in 1..4", bits);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

template <int D, int KBITS, int VBITS, int XDT>
int launch_kv_pair(const AppendArgs& k, const AppendArgs& v, hipStream_t st) {
  constexpr int VPB = 256 / (D / 32);
  const int64_t n_vec = static_cast<int64_t>(k.B) * k.H * k.L;
  const int64_t kb = (n_vec + VPB - 1) / VPB;
  if (2 * kb > 0x7fffffff) return fail(TQ_ERR_INVALID_ARGUMENT, "append: too many vectors");
  hipLaunchKernelGGL((append_rht_kv_kernel<D, KBITS, VBITS, XDT>), dim3(static_cast<unsigned>(2 * kb)),
                     dim3(256), 0, st, k, v, kb);
  return check_launch("append_rht_kv_kernel");
}

// Paired launch for equal widths or the x.5-bit split (values one bit wider),
// 16-bit inputs and head dims 64 / 128 / 256; returns -1 for other cases
// (the caller then launches the two sides separately).
template <int D, int XDT>
int launch_kv_bits(int kbits, int vbits, const AppendArgs& k, const AppendArgs& v, hipStream_t st) {
  switch (kbits * 8 + vbits) {
    case 1 * 8 + 1: return launch_kv_pair<D, 1, 1, XDT>(k, v, st);
    case 2 * 8 + 2: return launch_kv_pair<D, 2, 2, XDT>(k, v, st);
    case 3 * 8 + 3: return launch_kv_pair<D, 3, 3, XDT>(k, v, st);
    case 4 * 8 + 4: return launch_kv_pair<D, 4, 4, XDT>(k, v, st);
    case 1 * 8 + 2: return launch_kv_pair<D, 1, 2, XDT>(k, v, st);
    case 2 * 8 + 3: return launch_kv_pair<D, 2, 3, XDT>(k, v, st);
    case 3 * 8 + 4: return launch_kv_pair<D, 3, 4, XDT>(k, v, st);
  }
  return -1;
}

template <int D>
int launch_kv_dtype(int x_dtype, int kbits, int vbits, const AppendArgs& k, const AppendArgs& v,
                    hipStream_t st) {
  if (x_dtype == TQ_DTYPE_F16) return launch_kv_bits<D, TQ_DTYPE_F16>(kbits, vbits, k, v, st);
  if (x_dtype == TQ_DTYPE_BF16) return launch_kv_bits<D, TQ_DTYPE_BF16>(kbits, vbits, k, v, st);
  return -1;
}

}  // namespace

namespace {

// Argument checks of one quantize call; fills a on success.  *empty is set
// when there is nothing to do.
int check_append(const void* x, int x_dtype, int B, int H, int L, int dim, int64_t sb, int64_t sh,
                 int64_t sl, int bits, const float* rot, const float* midpoints, uint32_t* packed,
                 void* norms, int norm_dtype, int64_t capacity, int64_t offset, AppendArgs& a,
                 bool* empty) {
  *empty = false;
  if (B < 0 || H < 0 || L < 0) return fail(TQ_ERR_INVALID_ARGUMENT, "append: negative shape");
  if (bits < 1 || bits > 4) return fail(TQ_ERR_INVALID_ARGUMENT, "append: bits %d not in 1..4", bits);
  if (norm_dtype != TQ_DTYPE_F32 && norm_dtype != TQ_DTYPE_F16)
    return fail(TQ_ERR_INVALID_ARGUMENT, "append: norm_dtype %d", norm_dtype);
  if (x_dtype != TQ_DTYPE_F32 && x_dtype != TQ_DTYPE_F16 && x_dtype != TQ_DTYPE_BF16)
    return fail(TQ_ERR_INVALID_ARGUMENT, "append: x_dtype %d", x_dtype);
  if (offset < 0 || offset + L > capacity)
    return fail(TQ_ERR_INVALID_ARGUMENT, "append: tokens [%lld, %lld) exceed capacity %lld",
                (long long)offset, (long long)(offset + L), (long long)capacity);
  if (static_cast<int64_t>(B) * H * L == 0) {
    *empty = true;
    return TQ_OK;
  }
  if (!x || !rot || !midpoints || !packed || !norms)
    return fail(TQ_ERR_INVALID_ARGUMENT, "append: null pointer");
  // the vector-load kernels (every dim that is a multiple of 8) need 16-byte
  // rows; other dims run the general kernel, which loads single elements
  const int es = x_dtype == TQ_DTYPE_F32 ? 4 : 2;
  if (dim % 8 == 0 && (!aligned16(x) || (sb * es) % 16 || (sh * es) % 16 || (sl * es) % 16))
    return fail(TQ_ERR_INVALID_ARGUMENT, "append: x and its strides must be 16-byte aligned");
  a = AppendArgs{x, sb, sh, sl, B, H, L, rot, midpoints, packed, norms, norm_dtype, capacity, offset,
                 static_cast<float>(1.0 / __builtin_sqrt(static_cast<double>(dim)))};
  return TQ_OK;
}

int launch_one(const AppendArgs& a, int dim, int bits, int x_dtype, int rot_kind, hipStream_t st) {
  if (rot_kind == TQ_ROT_HADAMARD) {
    switch (dim) {
      case 32: return launch_append_rht<32>(bits, x_dtype, a, st);
      case 64: return launch_append_rht<64>(bits, x_dtype, a, st);
      case 128: return launch_append_rht<128>(bits, x_dtype, a, st);
      case 256: return launch_append_rht<256>(bits, x_dtype, a, st);
      case 512: return launch_append_rht<512>(bits, x_dtype, a, st);
    }
    return fail(TQ_ERR_UNSUPPORTED, "append: Hadamard rotation needs dim in {32..512} pow2, got %d", dim);
  }
  if (rot_kind == TQ_ROT_DENSE) return launch_append_dense(a, dim, bits, x_dtype, st);
  return fail(TQ_ERR_INVALID_ARGUMENT, "append: rot_kind %d", rot_kind);
}

}  // namespace

extern "C" int tq_append_quantize(const void* x, int x_dtype, int B, int H, int L, int dim,
                                  int64_t x_stride_b, int64_t x_stride_h, int64_t x_stride_l,
                                  int bits, int rot_kind, const float* rot,
                                  const float* midpoints, uint32_t* packed, void* norms,
                                  int norm_dtype, int64_t capacity, int64_t offset,
                                  void* stream) {
  AppendArgs a{};
  bool empty = false;
  int rc = check_append(x, x_dtype, B, H, L, dim, x_stride_b, x_stride_h, x_stride_l, bits, rot,
                        midpoints, packed, norms, norm_dtype, capacity, offset, a, &empty);
  if (rc || empty) return rc;
  return launch_one(a, dim, bits, x_dtype, rot_kind, static_cast<hipStream_t>(stream));
}

extern "C" int tq_append_quantize_kv(const void* k_x, const void* v_x, int x_dtype, int B, int H,
                                     int L, int dim, int64_t k_stride_b, int64_t k_stride_h,
                                     int64_t k_stride_l, int64_t v_stride_b, int64_t v_stride_h,
                                     int64_t v_stride_l, int k_bits, int v_bits, int rot_kind,
                                     const float* k_rot, const float* v_rot,
                                     const float* k_midpoints, const float* v_midpoints,
                                     uint32_t* k_packed, void* k_norms, uint32_t* v_packed,
                                     void* v_norms, int norm_dtype, int64_t capacity,
                                     int64_t offset, void* stream) {
  AppendArgs ka{}, va{};
  bool empty = false;
  int rc = check_append(k_x, x_dtype, B, H, L, dim, k_stride_b, k_stride_h, k_stride_l, k_bits, k_rot,
                        k_midpoints, k_packed, k_norms, norm_dtype, capacity, offset, ka, &empty);
  if (rc) return rc;
  rc = check_append(v_x, x_dtype, B, H, L, dim, v_stride_b, v_stride_h, v_stride_l, v_bits, v_rot,
                    v_midpoints, v_packed, v_norms, norm_dtype, capacity, offset, va, &empty);
  if (rc || empty) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (rot_kind == TQ_ROT_DENSE) {
    rc = launch_append_dense_kv(ka, va, dim, k_bits, v_bits, x_dtype, st);
    if (rc != -1) return rc;
  }
  if (rot_kind == TQ_ROT_HADAMARD) {
    switch (dim) {
      case 64: rc = launch_kv_dtype<64>(x_dtype, k_bits, v_bits, ka, va, st); break;
      case 128: rc = launch_kv_dtype<128>(x_dtype, k_bits, v_bits, ka, va, st); break;
      case 256: rc = launch_kv_dtype<256>(x_dtype, k_bits, v_bits, ka, va, st); break;
      default: rc = -1;
    }
    if (rc != -1) return rc;
  }
  rc = launch_one(ka, dim, k_bits, x_dtype, rot_kind, st);
  if (rc) return rc;
  return launch_one(va, dim, v_bits, x_dtype, rot_kind, st);
}

extern "C" int tq_append_plain(const void* x, int dtype, int B, int H, int L, int dim,
                               int64_t x_stride_b, int64_t x_stride_h, int64_t x_stride_l,
                               void* dst, int64_t capacity, int64_t offset, void* stream) {
  if (dtype != TQ_DTYPE_F16 && dtype != TQ_DTYPE_BF16)
    return fail(TQ_ERR_INVALID_ARGUMENT, "append_plain: dtype %d (F16/BF16 only)", dtype);
  if (B < 0 || H < 0 || L < 0 || dim <= 0)
    return fail(TQ_ERR_INVALID_ARGUMENT, "append_plain: bad shape");
  if (offset < 0 || offset + L > capacity)
    return fail(TQ_ERR_INVALID_ARGUMENT, "append_plain: tokens exceed capacity");
  if (static_cast<int64_t>(B) * H * L == 0) return TQ_OK;
  if (!x || !dst) return fail(TQ_ERR_INVALID_ARGUMENT, "append_plain: null pointer");
  PlainArgs a{static_cast<const uint16_t*>(x), x_stride_b, x_stride_h, x_stride_l, B, H, L, dim,
              static_cast<uint16_t*>(dst), capacity, offset};
  if (dim % 8 == 0 && aligned16(x) && aligned16(dst) && (x_stride_b * 2) % 16 == 0 &&
      (x_stride_h * 2) % 16 == 0 && (x_stride_l * 2) % 16 == 0) {
    const int64_t total = static_cast<int64_t>(B) * H * L * (dim / 8);
    const dim3 grid(static_cast<unsigned>((total + 255) / 256));
    if (total + 256 < (int64_t(1) << 32))
      hipLaunchKernelGGL(append_plain_kernel<uint32_t>, grid, dim3(256), 0, static_cast<hipStream_t>(stream), a);
    else
      hipLaunchKernelGGL(append_plain_kernel<int64_t>, grid, dim3(256), 0, static_cast<hipStream_t>(stream), a);
    return check_launch("append_plain_kernel");
  }
  const int64_t total = static_cast<int64_t>(B) * H * L * dim;
  hipLaunchKernelGGL(append_plain_elem_kernel, dim3(static_cast<unsigned>((total + 255) / 256)),
                     dim3(256), 0, static_cast<hipStream_t>(stream), a);
  return check_launch("append_plain_elem_kernel");
}

extern "C" int tq_dequantize(const uint32_t* packed, const void* norms, int norm_dtype, int B,
                             int H, int T, int dim, int bits, int64_t capacity,
                             const float* codebook, int rot_kind, const float* rot, float* out,
                             void* stream) {
  if (bits < 1 || bits > 4) return fail(TQ_ERR_INVALID_ARGUMENT, "dequantize: bits %d", bits);
  if (dim < 8 || dim > 512)
    return fail(TQ_ERR_UNSUPPORTED, "dequantize: dim %d (8..512)", dim);
  if (rot_kind == TQ_ROT_HADAMARD && (dim & (dim - 1)))
    return fail(TQ_ERR_INVALID_ARGUMENT, "dequantize: Hadamard rotation needs a power-of-two dim, got %d", dim);
  if (T < 0 || T > capacity) return fail(TQ_ERR_INVALID_ARGUMENT, "dequantize: T > capacity");
  if (rot_kind != TQ_ROT_HADAMARD && rot_kind != TQ_ROT_DENSE)
    return fail(TQ_ERR_INVALID_ARGUMENT, "dequantize: rot_kind %d", rot_kind);
  const int64_t n = static_cast<int64_t>(B) * H * T;
  if (n == 0) return TQ_OK;
  if (!packed || !norms || !codebook || !rot || !out)
    return fail(TQ_ERR_INVALID_ARGUMENT, "dequantize: null pointer");
  if (dim < 32 || dim > 256 || (dim & (dim - 1))) {
    const DequantGeneralArgs g{packed, norms, norm_dtype, B, H, T, dim, bits,
                               tq_packed_width(dim, bits), capacity, codebook, rot_kind, rot,
                               static_cast<float>(1.0 / __builtin_sqrt(static_cast<double>(dim))), out};
    return launch_dequant_general(g, n, static_cast<hipStream_t>(stream));
  }
  DequantArgs a{packed, norms, norm_dtype, B, H, T, dim, bits, tq_packed_width(dim, bits),
                capacity, codebook, rot_kind, rot,
                static_cast<float>(1.0 / __builtin_sqrt(static_cast<double>(dim))), out};
  hipLaunchKernelGGL(dequant_kernel, dim3(static_cast<unsigned>(n)), dim3(dim), 0,
                     static_cast<hipStream_t>(stream), a);
  return check_launch("dequant_kernel");
}
