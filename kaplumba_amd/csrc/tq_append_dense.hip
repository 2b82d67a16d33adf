// Dense-rotation append on the matrix cores (gfx950, v_mfma_f32_32x32x16_bf16).
//
// Semantics: _TurboQuantMSECodec.quantize with the dense rotation
// (turboquant_cache.py:4248-4254, _rotate_forward = u @ R^T at :4141-4144):
//   n = ||x||_2 (f32), u = x / max(n, 1e-6), y = u @ R^T, idx_i = #{m : y_i > mid_m},
// packed LSB-first like the Hadamard path.  The norm uses the Hadamard
// kernel's reduction tree, so norms are bit-identical to it.
//
// Arithmetic.  The matrix cores compute y * max(n, eps) = x @ R^T: R is split
// once per workgroup into three bf16 pieces R = R0 + R1 + R2 (each the
// round-to-nearest-even bf16 of what the previous pieces leave; together they
// carry R's full 24-bit significand), x enters as bf16 (exact for bf16 input;
// f32 input is the exact sum of three bf16 pieces), every piece product is
// exact and the sum runs in f32.  Products whose piece orders add up to more
// than 2 are below f32 resolution and skipped.  f16 input feeds
// v_mfma_f32_32x32x16_f16 exactly as loaded, against three f16 pieces of
// 2^rs R, where 2^rs brings the workgroup's largest |R| entry into
// [2^14, 2^15): three products per tile and k-step instead of five, and no
// split of x.  The scale is exact and is applied to the thresholds too.  Instead
// of dividing, each coordinate is compared with mid_m * max(n, eps), computed
// once per vector.  The result therefore differs from an f32 `u @ R^T` only in
// the last bits of the sum, so an index can differ only where y lies within a
// few f32 ulps of a midpoint (MLX's own f32 matmul order is not specified
// either).
//
// Work split.  One workgroup = 8 waves x 32 vectors.  A wave computes
// Y^T[coords][32 vectors] = R_slice (A, from LDS) x X^T (B, from HBM):
//   * B lane (v = lane % 32, g = lane / 32) loads the D/2 consecutive elements
//     [g*D/2, (g+1)*D/2) of vector v, which is exactly its B operand over all
//     k-steps once the contraction index is permuted: MFMA k-slot 8g + j of
//     k-step s stands for element g*D/2 + 8s + j (A uses the same permutation).
//     These are also the elements whose squares the norm tree sums first.
//   * A tile t of 32 rows holds R rows permuted so that, in the 32x32 output
//     layout (lane l, register i = row 8(i/4) + 4(l/32) + i%4, column l%32),
//     lane g of the pair of tiles (2p, 2p+1) ends up with the 32 consecutive
//     coordinates c0 + 64p + 32g + [0, 32): packing is thread-local.
//   * R pieces live in LDS in fragment order (one 16-byte slot per lane per
//     tile, k-step and piece), so every A read is a conflict-free ds_read_b128.
// For D = 256 the 256 coordinates are split over 4 workgroups of 64 (LDS
// holds R pieces for 64 x 256); each of them reads the whole vector.
#include "tq_append.h"

namespace tq {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kDenseThreads = 512;
constexpr int kDenseWaves = kDenseThreads / kWave;

template <int D>
struct DenseShape {
  static constexpr int CT = D == 128 ? 128 : 64;          // coordinates per workgroup
  static constexpr int NSLICE = D / CT;                   // workgroups per vector tile
  static constexpr int NT = CT / 32;                      // 32-row coordinate tiles
  static constexpr int KS = D / 16;                       // k-steps
  static constexpr int LE = D / 2;                        // x elements per lane
  static constexpr int NRP = 3;                           // bf16 pieces of R
  static constexpr int SLOTS = NRP * NT * KS * kWave;     // 16-byte A fragments
  static constexpr int VPT = kDenseWaves * 32;            // vectors per workgroup tile
  static_assert(NT % 2 == 0, "coordinate tiles come in pairs");
};

template <int XDT>
struct XPieces {  // bf16 pieces whose sum is the input element exactly
  static constexpr int N = XDT == TQ_DTYPE_BF16 ? 1 : (XDT == TQ_DTYPE_F16 ? 2 : 3);
  static constexpr int ES = XDT == TQ_DTYPE_F32 ? 4 : 2;
};

__device__ __forceinline__ f32x16_t mfma32(u32x4_t a, u32x4_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                  __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));

__device__ __forceinline__ f32x16_t mfma32h(u32x4_t a, u32x4_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                 __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

// Split a and b into NP f16 pieces each (round to nearest even, exact f32
// remainders), packed per piece as (a_i, b_i).
template <int NP>
__device__ __forceinline__ void split_f16x2(float a, float b, uint32_t (&w)[NP]) {
  float ra = a, rb = b;
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    const f16x2_t v = {static_cast<_Float16>(ra), static_cast<_Float16>(rb)};
    w[i] = __builtin_bit_cast(uint32_t, v);
    ra = __fsub_rn(ra, static_cast<float>(v[0]));
    rb = __fsub_rn(rb, static_cast<float>(v[1]));
  }
}

// Split a and b into NP bf16 pieces each (round-to-nearest-even, exact
// remainders), packed per piece as (a_i, b_i): one v_cvt_pk_bf16_f32 per piece
// and pair.
template <int NP>
__device__ __forceinline__ void split_bf16x2(float a, float b, uint32_t (&w)[NP]) {
  float ra = a, rb = b;
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    const bf16x2_t v = {static_cast<__bf16>(ra), static_cast<__bf16>(rb)};
    w[i] = __builtin_bit_cast(uint32_t, v);
    ra = __fsub_rn(ra, __uint_as_float(w[i] << 16));
    rb = __fsub_rn(rb, __uint_as_float(w[i] & 0xffff0000u));
  }
}

// Element e of the lane's run of x, as f32.
template <int XDT, int NX>
__device__ __forceinline__ float x_elem(const u32x4_t (&xr)[NX], int e) {
  if constexpr (XDT == TQ_DTYPE_F32) {
    return __uint_as_float(xr[e >> 2][e & 3]);
  } else {
    const uint32_t w = xr[e >> 3][(e >> 1) & 3];
    const uint16_t h = static_cast<uint16_t>((e & 1) ? (w >> 16) : (w & 0xffffu));
    return XDT == TQ_DTYPE_F16 ? f16_bits_to_f32(h) : bf16_bits_to_f32(h);
  }
}

// GE: one-bit signs of x @ R^T, bit = (y >= 0) (the QJL sketch of the Prod
// codec, turboquant_cache.py:4662-4663); midpoints are not read.
// Workgroup bid of nblk (persistent over vector tiles) of one quantize side;
// s_r: the workgroup's LDS for the R pieces (S::SLOTS fragments).
template <int D, int BITS, int XDT, bool GE>
__device__ __forceinline__ void dense_body(const AppendArgs& a, u32x4_t* s_r, int bid, int nblk) {
  using S = DenseShape<D>;
  using XP = XPieces<XDT>;
  constexpr int NMID = (1 << BITS) - 1;
  constexpr int PW = D * BITS / 32;
  constexpr int NX = S::LE * XP::ES / 16;  // 16-byte loads per lane

  // f16 input feeds f16 MFMAs as loaded (one x piece); R then goes into f16
  // pieces, scaled by 2^rs so that the largest entry sits just below 2^15.
  constexpr bool HX = XDT == TQ_DTYPE_F16;
  constexpr int NXP = HX ? 1 : XP::N;
  __shared__ uint32_t s_rmax;

  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wave = tid / kWave;
  const int vl = lane % 32;
  const int g = lane / 32;
  const int slice = bid % S::NSLICE;
  const int c0 = slice * S::CT;
  const int64_t tile_stride = nblk / S::NSLICE;
  const int64_t n_vec = static_cast<int64_t>(a.B) * a.H * a.L;

  // Input run of this lane for a given tile.  A lane past the last vector
  // reads vector 0 (launches have n_vec >= 1) and gets row -1: its column
  // of the products is its own and is never stored.  Loads without a branch
  // keep the compiler's wait counts exact.
  auto load_x = [&](int64_t tile, u32x4_t (&xr)[NX], int64_t& row) {
    const int64_t vec = tile * S::VPT + wave * 32 + vl;
    int l, h, b;
    if (a.L % S::VPT == 0) {
      // the tile's vectors share one (b, h) row and are all live: the
      // divisions are the tile's, on uniform values
      const int64_t bh = (tile * S::VPT) / a.L;
      l = static_cast<int>(tile * S::VPT - bh * a.L) + wave * 32 + vl;
      h = static_cast<int>(bh % a.H);
      b = static_cast<int>(bh / a.H);
    } else {
      const int64_t vc = vec < n_vec ? vec : 0;
      l = static_cast<int>(vc % a.L);
      const int64_t bh = vc / a.L;
      h = static_cast<int>(bh % a.H);
      b = static_cast<int>(bh / a.H);
    }
    const int64_t xoff = b * a.sb + h * a.sh + l * a.sl + g * S::LE;
    const u32x4_t* src =
        reinterpret_cast<const u32x4_t*>(static_cast<const char*>(a.x) + xoff * XP::ES);
#pragma unroll
    for (int i = 0; i < NX; ++i) xr[i] = src[i];
    row = vec < n_vec ? (static_cast<int64_t>(b) * a.H + h) * a.cap + a.offset + l : -1;
  };

  if constexpr (HX) {
    if (tid == 0) s_rmax = 0u;
    append_lds_barrier();
  }

  // ---- R pieces -> LDS in A-fragment order.  This thread's fragments are
  // requested first, then its first input tile, so the tile's loads are in
  // flight while R is split (waiting for R does not wait for them).
  constexpr int FPT = S::NT * S::KS * kWave / kDenseThreads;  // fragments per thread
  static_assert(S::NT * S::KS * kWave % kDenseThreads == 0, "R fragments per thread");
  float4 rv[FPT][2];
#pragma unroll
  for (int i = 0; i < FPT; ++i) {
    const int f = tid + i * kDenseThreads;
    const int ln = f % kWave;
    const int ks = (f / kWave) % S::KS;
    const int t = f / (kWave * S::KS);
    const int r = ln % 32;
    const int coord = c0 + 64 * (t / 2) + 32 * ((r >> 2) & 1) + 16 * (t & 1) + 4 * (r >> 3) + (r & 3);
    const float4* src =
        reinterpret_cast<const float4*>(a.rot + static_cast<int64_t>(coord) * D + (ln / 32) * S::LE + 8 * ks);
    rv[i][0] = src[0];
    rv[i][1] = src[1];
  }
  int64_t tile = bid / S::NSLICE;
  u32x4_t xr[NX];
  int64_t row;
  load_x(tile, xr, row);
  // 2^rs: the power of two that brings the workgroup's largest |R| entry into
  // [2^14, 2^15) (2^15 for an all-zero R); exact, and undone on the thresholds
  float r_scale = 1.f;
  if constexpr (HX) {
    float m = 0.f;
#pragma unroll
    for (int i = 0; i < FPT; ++i)
      m = fmaxf(m, fmaxf(fmaxf(fmaxf(fabsf(rv[i][0].x), fabsf(rv[i][0].y)), fmaxf(fabsf(rv[i][0].z), fabsf(rv[i][0].w))),
                         fmaxf(fmaxf(fabsf(rv[i][1].x), fabsf(rv[i][1].y)), fmaxf(fabsf(rv[i][1].z), fabsf(rv[i][1].w)))));
    atomicMax(&s_rmax, __float_as_uint(m));  // non-negative floats order as their bits
    append_lds_barrier();
    int e = 0;
    frexpf(__uint_as_float(s_rmax), &e);  // max < 2^e
    r_scale = ldexpf(1.f, min(max(15 - e, -100), 100));
  }
#pragma unroll
  for (int i = 0; i < FPT; ++i) {
    const int f = tid + i * kDenseThreads;
    const float4 v0 = rv[i][0], v1 = rv[i][1];
    const float e[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
    uint32_t w[S::NRP][4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t pr[S::NRP];
      if constexpr (HX)
        split_f16x2<S::NRP>(__fmul_rn(e[2 * j], r_scale), __fmul_rn(e[2 * j + 1], r_scale), pr);
      else
        split_bf16x2<S::NRP>(e[2 * j], e[2 * j + 1], pr);
#pragma unroll
      for (int p = 0; p < S::NRP; ++p) w[p][j] = pr[p];
    }
#pragma unroll
    for (int p = 0; p < S::NRP; ++p)
      s_r[(p * S::NT * S::KS) * kWave + f] = u32x4_t{w[p][0], w[p][1], w[p][2], w[p][3]};
  }
  float mid[NMID];
#pragma unroll
  for (int m = 0; m < NMID; ++m) mid[m] = GE ? 0.f : a.mid[m];

  __syncthreads();

  for (; tile * S::VPT < n_vec; tile += tile_stride) {
    // ---- norm: 32-element folds 16, 8, 4, 2, 1, groups pairwise, then the partner lane
    constexpr int NG = S::LE / 32;
    float gs[NG];
#pragma unroll
    for (int q = 0; q < NG; ++q) {
      float s[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float u0 = x_elem<XDT, NX>(xr, 32 * q + i);
        const float u1 = x_elem<XDT, NX>(xr, 32 * q + i + 16);
        // f16 squares are exact in f32: RN(a^2 + RN(b^2)) = RN(RN(a^2) + RN(b^2))
        s[i] = HX ? __builtin_fmaf(u0, u0, __fmul_rn(u1, u1)) : __fadd_rn(__fmul_rn(u0, u0), __fmul_rn(u1, u1));
      }
#pragma unroll
      for (int w = 8; w >= 1; w >>= 1) {
#pragma unroll
        for (int i = 0; i < w; ++i) s[i] = __fadd_rn(s[i], s[i + w]);
      }
      gs[q] = s[0];
    }
#pragma unroll
    for (int w = 1; w < NG; w <<= 1) {
#pragma unroll
      for (int q = 0; q < NG; q += 2 * w) gs[q] = __fadd_rn(gs[q], gs[q + w]);
    }
    const float ss = __fadd_rn(gs[0], __shfl_xor(gs[0], 32, kWave));
    const float n = sqrt_rn(ss);
    const float den = fmaxf(n, kNormEps);
    float thr[NMID];
#pragma unroll
    for (int m = 0; m < NMID; ++m) thr[m] = __fmul_rn(__fmul_rn(mid[m], den), r_scale);

    // ---- x @ R^T for this slice's coordinates
    f32x16_t acc[S::NT];
#pragma unroll
    for (int t = 0; t < S::NT; ++t) acc[t] = f32x16_t{};
#pragma unroll
    for (int ks = 0; ks < S::KS; ++ks) {
      u32x4_t xb[NXP];
      if constexpr (XDT == TQ_DTYPE_BF16 || HX) {
        xb[0] = xr[ks];
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          uint32_t pr[XP::N];
          split_bf16x2<XP::N>(x_elem<XDT, NX>(xr, 8 * ks + 2 * j), x_elem<XDT, NX>(xr, 8 * ks + 2 * j + 1), pr);
#pragma unroll
          for (int p = 0; p < XP::N; ++p) xb[p][j] = pr[p];
        }
      }
      // smallest terms first
#pragma unroll
      for (int rp = S::NRP - 1; rp >= 0; --rp) {
#pragma unroll
        for (int xp = NXP - 1; xp >= 0; --xp) {
          if (rp + xp > 2) continue;
#pragma unroll
          for (int t = 0; t < S::NT; ++t) {
            const u32x4_t ra = s_r[((rp * S::NT + t) * S::KS + ks) * kWave + lane];
            acc[t] = HX ? mfma32h(ra, xb[xp], acc[t]) : mfma32(ra, xb[xp], acc[t]);
          }
        }
      }
      // keep each k-step's fragment reads next to its products (hoisting all
      // of them ahead of the first product would need 4 VGPRs per fragment)
      __builtin_amdgcn_sched_barrier(0);
    }

    // ---- the next tile's input is requested now (x is dead after the
    // products), so its loads are in flight during the quantize and stores
    const int64_t row_cur = row;
    if ((tile + tile_stride) * S::VPT < n_vec) load_x(tile + tile_stride, xr, row);

    // ---- quantize against mid * max(n, eps), pack 32 coordinates per lane and pair
    if (row_cur >= 0) {
      uint32_t* dst_row = a.packed + row_cur * PW;
      auto pack_pairs = [&](auto idx_of) {
#pragma unroll
        for (int p = 0; p < S::NT / 2; ++p) {
          uint32_t words[BITS];
#pragma unroll
          for (int w = 0; w < BITS; ++w) words[w] = 0u;
#pragma unroll
          for (int e = 0; e < 32; ++e) {
            const uint32_t idx = idx_of(acc[2 * p + e / 16][e % 16]);
            const int pos = e * BITS;
            const int wi = pos >> 5;
            const int sh = pos & 31;
            words[wi] |= idx << sh;
            if (sh + BITS > 32) words[wi + 1] |= idx >> (32 - sh);
          }
          uint32_t* dst = dst_row + ((c0 + 64 * p + 32 * g) / 32) * BITS;
#pragma unroll
          for (int w = 0; w < BITS; ++w) dst[w] = words[w];
        }
      };
      pack_pairs([&](float y) -> uint32_t {
        uint32_t idx = 0;
        if constexpr (NMID >= 7) {
          // thr is sorted, so the middle threshold decides which half
          // can still hold y: count that half (H compares, its thresholds
          // chosen by H selects) on top of the H + 1 below it or none.
          // The same count as NMID compares, in 2H + 2 fewer operations.
          constexpr int H = NMID / 2;
          const bool up = GE ? (y >= thr[H]) : (y > thr[H]);
          idx = up ? static_cast<uint32_t>(H + 1) : 0u;
#pragma unroll
          for (int m = 0; m < H; ++m) {
            const float t = up ? thr[H + 1 + m] : thr[m];
            idx += (GE ? (y >= t) : (y > t)) ? 1u : 0u;
          }
        } else {
#pragma unroll
          for (int m = 0; m < NMID; ++m) idx += (GE ? (y >= thr[m]) : (y > thr[m])) ? 1u : 0u;
        }
        return idx;
      });
      if (slice == 0 && g == 0) {
        if (a.norm_dtype == TQ_DTYPE_F16)
          static_cast<uint16_t*>(a.norms)[row_cur] = f32_to_f16_bits(n);
        else
          static_cast<float*>(a.norms)[row_cur] = n;
      }
    }
  }
}

template <int D, int BITS, int XDT, bool GE = false>
__global__ __launch_bounds__(kDenseThreads) void append_dense_kernel(AppendArgs a) {
  __shared__ u32x4_t s_r[DenseShape<D>::SLOTS];
  dense_body<D, BITS, XDT, GE>(a, s_r, blockIdx.x, gridDim.x);
}

// Keys and values of one append in one launch: workgroups below nk quantize
// the keys (R_K), the rest the values (R_V); each splits its side's R once and
// walks that side's tiles, sharing one LDS buffer between the two bodies.
template <int D, int KBITS, int VBITS, int XDT>
__global__ __launch_bounds__(kDenseThreads) void append_dense_kv_kernel(AppendArgs k, AppendArgs v, int nk) {
  __shared__ u32x4_t s_r[DenseShape<D>::SLOTS];
  const bool key = static_cast<int>(blockIdx.x) < nk;
  if constexpr (KBITS == VBITS) {
    // one copy of the body for both sides (the side's arguments picked
    // first): half the code for the instruction cache
    const AppendArgs side = select_args(key, k, v);
    dense_body<D, KBITS, XDT, false>(side, s_r, key ? blockIdx.x : blockIdx.x - nk, key ? nk : gridDim.x - nk);
  } else {
    if (key)
      dense_body<D, KBITS, XDT, false>(k, s_r, blockIdx.x, nk);
    else
      dense_body<D, VBITS, XDT, false>(v, s_r, blockIdx.x - nk, gridDim.x - nk);
  }
}

template <int D, int BITS>
int launch_dense_bits(const AppendArgs& a, int x_dtype, hipStream_t st) {
  using S = DenseShape<D>;
  const int64_t n_vec = static_cast<int64_t>(a.B) * a.H * a.L;
  const int64_t tiles = (n_vec + S::VPT - 1) / S::VPT;
  // One workgroup per CU fits next to the 96 KiB of R pieces; larger batches loop.
  const int64_t per_slice = std::min<int64_t>(tiles, std::max(1, device_cu_count() / S::NSLICE));
  const dim3 grid(static_cast<unsigned>(per_slice * S::NSLICE));
  switch (x_dtype) {
    case TQ_DTYPE_F32:
      hipLaunchKernelGGL((append_dense_kernel<D, BITS, TQ_DTYPE_F32>), grid, dim3(kDenseThreads), 0, st, a);
      break;
    case TQ_DTYPE_F16:
      hipLaunchKernelGGL((append_dense_kernel<D, BITS, TQ_DTYPE_F16>), grid, dim3(kDenseThreads), 0, st, a);
      break;
    default:
      hipLaunchKernelGGL((append_dense_kernel<D, BITS, TQ_DTYPE_BF16>), grid, dim3(kDenseThreads), 0, st, a);
      break;
  }
  return check_launch("append_dense_kernel");
}

template <int D>
int launch_dense_dim(const AppendArgs& a, int bits, int x_dtype, hipStream_t st) {
  switch (bits) {
    case 1: return launch_dense_bits<D, 1>(a, x_dtype, st);
    case 2: return launch_dense_bits<D, 2>(a, x_dtype, st);
    case 3: return launch_dense_bits<D, 3>(a, x_dtype, st);
    case 4: return launch_dense_bits<D, 4>(a, x_dtype, st);
  }
  return fail(TQ_ERR_INVALID_ARGUMENT, "append: bits %d not in 1..4", bits);
}

template <int D>
int launch_dense_signs_dim(const AppendArgs& a, hipStream_t st) {
  using S = DenseShape<D>;
  const int64_t n_vec = static_cast<int64_t>(a.B) * a.H * a.L;
  const int64_t tiles = (n_vec + S::VPT - 1) / S::VPT;
  const int64_t per_slice = std::min<int64_t>(tiles, std::max(1, device_cu_count() / S::NSLICE));
  hipLaunchKernelGGL((append_dense_kernel<D, 1, TQ_DTYPE_F32, true>), dim3(static_cast<unsigned>(per_slice * S::NSLICE)),
                     dim3(kDenseThreads), 0, st, a);
  return check_launch("append_dense_kernel (signs)");
}

template <int D, int KBITS, int VBITS, int XDT>
int launch_dense_kv_pair(const AppendArgs& k, const AppendArgs& v, hipStream_t st) {
  using S = DenseShape<D>;
  const int64_t n_vec = static_cast<int64_t>(k.B) * k.H * k.L;
  const int64_t tiles = (n_vec + S::VPT - 1) / S::VPT;
  // half the CUs per side, one workgroup each (the R pieces fill the LDS)
  const int64_t per_slice = std::min<int64_t>(tiles, std::max(1, device_cu_count() / S::NSLICE / 2));
  const int nk = static_cast<int>(per_slice * S::NSLICE);
  hipLaunchKernelGGL((append_dense_kv_kernel<D, KBITS, VBITS, XDT>), dim3(static_cast<unsigned>(2 * nk)),
                     dim3(kDenseThreads), 0, st, k, v, nk);
  return check_launch("append_dense_kv_kernel");
}

template <int D, int XDT>
int launch_dense_kv_bits(int kbits, int vbits, const AppendArgs& k, const AppendArgs& v, hipStream_t st) {
  switch (kbits * 8 + vbits) {
    case 1 * 8 + 1: return launch_dense_kv_pair<D, 1, 1, XDT>(k, v, st);
    case 2 * 8 + 2: return launch_dense_kv_pair<D, 2, 2, XDT>(k, v, st);
    case 3 * 8 + 3: return launch_dense_kv_pair<D, 3, 3, XDT>(k, v, st);
    case 4 * 8 + 4: return launch_dense_kv_pair<D, 4, 4, XDT>(k, v, st);
    case 1 * 8 + 2: return launch_dense_kv_pair<D, 1, 2, XDT>(k, v, st);
    case 2 * 8 + 3: return launch_dense_kv_pair<D, 2, 3, XDT>(k, v, st);
    case 3 * 8 + 4: return launch_dense_kv_pair<D, 3, 4, XDT>(k, v, st);
  }
  return -1;
}

template <int D>
int launch_dense_kv_dim(int x_dtype, int kbits, int vbits, const AppendArgs& k, const AppendArgs& v,
                        hipStream_t st) {
  if (x_dtype == TQ_DTYPE_F16) return launch_dense_kv_bits<D, TQ_DTYPE_F16>(kbits, vbits, k, v, st);
  if (x_dtype == TQ_DTYPE_BF16) return launch_dense_kv_bits<D, TQ_DTYPE_BF16>(kbits, vbits, k, v, st);
  return -1;
}

}  // namespace

int launch_append_dense_kv(const AppendArgs& k, const AppendArgs& v, int dim, int kbits, int vbits,
                           int x_dtype, hipStream_t st) {
  if ((reinterpret_cast<uintptr_t>(k.rot) & 15u) != 0 || (reinterpret_cast<uintptr_t>(v.rot) & 15u) != 0)
    return fail(TQ_ERR_INVALID_ARGUMENT, "append: dense rotation matrix must be 16-byte aligned");
  switch (dim) {
    case 64: return launch_dense_kv_dim<64>(x_dtype, kbits, vbits, k, v, st);
    case 128: return launch_dense_kv_dim<128>(x_dtype, kbits, vbits, k, v, st);
    case 256: return launch_dense_kv_dim<256>(x_dtype, kbits, vbits, k, v, st);
  }
  return -1;
}

int launch_append_dense_signs(const AppendArgs& a, int dim, hipStream_t st) {
  if ((reinterpret_cast<uintptr_t>(a.rot) & 15u) != 0)
    return fail(TQ_ERR_INVALID_ARGUMENT, "prod: projection matrix must be 16-byte aligned");
  switch (dim) {
    case 64: return launch_dense_signs_dim<64>(a, st);
    case 128: return launch_dense_signs_dim<128>(a, st);
    case 256: return launch_dense_signs_dim<256>(a, st);
  }
  return launch_append_dense_signs_general(a, dim, st);
}

int launch_append_dense(const AppendArgs& a, int dim, int bits, int x_dtype, hipStream_t st) {
  if ((reinterpret_cast<uintptr_t>(a.rot) & 15u) != 0)
    return fail(TQ_ERR_INVALID_ARGUMENT, "append: dense rotation matrix must be 16-byte aligned");
  switch (dim) {
    case 64: return launch_dense_dim<64>(a, bits, x_dtype, st);
    case 128: return launch_dense_dim<128>(a, bits, x_dtype, st);
    case 256: return launch_dense_dim<256>(a, bits, x_dtype, st);
  }
  return launch_append_dense_general(a, dim, bits, x_dtype, st);
}

}  // namespace tq
