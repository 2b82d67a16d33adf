// Append-time quantize with the dense rotation, and dequantize, at any head
// dim the fixed-size kernels do not cover (8..512: the dims that are not
// powers of two take the dense rotation in the reference,
// _TurboQuantMSECodec.__init__, turboquant_cache.py:4122-4139).
//
// Quantize (turboquant_cache.py:4186-4254, array path :4248-4254) per vector:
//   * ||x||^2 in the fixed tree of the other quantizers, the dim zero-padded to
//     a power-of-two number of 32-element lanes (the padding adds exact
//     zeros): a lane squares its elements and folds them at distances 16, 8,
//     4, 2, 1; lane sums combine pairwise (0+1, 2+3, then the pairs), which is
//     the xor-butterfly order;
//   * n = sqrt (IEEE), u = x / max(n, 1e-6) (IEEE division);
//   * y = u @ R^T with f32 fused multiply-adds in four interleaved partial
//     sums (coordinates d mod 4, in order of d) added pairwise at the end;
//   * idx = #{m : y > mid[m]}; LSB-first packing into ceil(D*bits/32) words.
// One workgroup of 256 threads owns 16 vectors: x and u stay in LDS, thread j
// forms output coordinate j of all 16 vectors from row j of R (R crosses L2
// once per 16 vectors), then threads pack whole words.  This path is
// VALU-bound (D multiply-adds per coordinate); the power-of-two dims of the
// real models take the Hadamard or matrix-core kernels instead.
#include "tq_append.h"

namespace tq {
namespace {

constexpr int kGaVec = 16;     // vectors per workgroup
constexpr int kGaMaxDim = 512;

__device__ __forceinline__ int pow2_ceil(int x) {  // x >= 1
  int r = 1;
  while (r < x) r <<= 1;
  return r;
}

// Modes:
//   kGaQuantize  indices of y = u @ R^T against the midpoints, packed;
//   kGaSigns     the Prod codec's QJL signs (BITS = 1, no midpoints): bit =
//                y >= 0 for y = u @ P^T, which has the sign of residual @ P^T
//                (u is the residual over its norm); the norm written is the
//                residual's;
//   kGaProdResid the Prod codec's MSE part at BITS = bits - 1 (0..3) with the
//                dense rotation (_quantize_unit_with_estimate,
//                turboquant_cache.py:4151-4166): indices packed as in
//                kGaQuantize, then the estimate c[idx] @ R (thread j: column
//                j of R, rows in order, fused multiply-adds) and the residual
//                u - estimate (u itself when BITS = 0) written to resid
//                [n_vec, D] f32; norms receive ||x||.
constexpr int kGaQuantize = 0, kGaSigns = 1, kGaProdResid = 2;

template <int BITS, int XDT, int MODE = kGaQuantize>
__global__ __launch_bounds__(256) void append_dense_general_kernel(AppendArgs a, int D, float* resid,
                                                                   const float* cb) {
  constexpr bool SGN = MODE == kGaSigns;
  __shared__ float s_u[kGaVec][kGaMaxDim];
  __shared__ uint8_t s_idx[kGaVec][kGaMaxDim];
  __shared__ float s_lane[kGaVec][16];
  __shared__ float s_den[kGaVec];
  __shared__ float s_nrm[kGaVec];
  __shared__ float s_mid[16];
  __shared__ float s_cb[16];
  constexpr int NMID = (1 << BITS) - 1;
  const int tid = threadIdx.x;
  const int64_t n_vec = static_cast<int64_t>(a.B) * a.H * a.L;
  const int64_t vec0 = static_cast<int64_t>(blockIdx.x) * kGaVec;
  // the norm tree's extent: 32-element lanes, a power-of-two count of them
  // (zeros past D; a dim below 32 folded inside one zero-padded lane gives
  // the same sums as its own power-of-two tree, since the first folds add
  // exact zeros)
  const int LP = D <= 32 ? 32 : 32 * pow2_ceil((D + 31) / 32);
  const int NL = LP / 32;
  if (!SGN && tid < NMID) s_mid[tid] = a.mid[tid];
  if (MODE == kGaProdResid && BITS > 0 && tid < (1 << BITS)) s_cb[tid] = cb[tid];
  auto vec_coords = [&](int64_t vec, int& b, int& h, int& l) {
    l = static_cast<int>(vec % a.L);
    const int64_t bh = vec / a.L;
    h = static_cast<int>(bh % a.H);
    b = static_cast<int>(bh / a.H);
  };
  // x -> LDS (zero beyond D and for vectors past the end)
  for (int idx = tid; idx < kGaVec * LP; idx += 256) {
    const int v = idx / LP;
    const int d = idx % LP;
    const int64_t vec = vec0 + v;
    float x = 0.f;
    if (vec < n_vec && d < D) {
      int b, h, l;
      vec_coords(vec, b, h, l);
      x = load_elem<XDT>(a.x, b * a.sb + h * a.sh + l * a.sl + d);
    }
    s_u[v][d] = x;
  }
  __syncthreads();
  // norm: thread (vector v, lane g) squares its 32 elements and folds them
  // at distances 16, 8, 4, 2, 1
  if (tid < kGaVec * NL) {
    const int v = tid / NL;
    const int g = tid % NL;
    float s[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float e0 = s_u[v][g * 32 + i];
      const float e1 = s_u[v][g * 32 + i + 16];
      s[i] = __fadd_rn(__fmul_rn(e0, e0), __fmul_rn(e1, e1));
    }
#pragma unroll
    for (int w = 8; w >= 1; w >>= 1)
#pragma unroll
      for (int i = 0; i < w; ++i) s[i] = __fadd_rn(s[i], s[i + w]);
    s_lane[v][g] = s[0];
  }
  __syncthreads();
  if (tid < kGaVec) {
    for (int n = NL; n > 1; n >>= 1)
      for (int i = 0; i < n / 2; ++i) s_lane[tid][i] = __fadd_rn(s_lane[tid][2 * i], s_lane[tid][2 * i + 1]);
    const float nrm = sqrt_rn(s_lane[tid][0]);
    s_nrm[tid] = nrm;
    s_den[tid] = fmaxf(nrm, kNormEps);
  }
  __syncthreads();
  for (int idx = tid; idx < kGaVec * D; idx += 256) {
    const int v = idx / D;
    const int d = idx % D;
    s_u[v][d] = __fdiv_rn(s_u[v][d], s_den[v]);
  }
  __syncthreads();
  // y = u @ R^T, indices
  // a row of R is 16-byte aligned when D % 4 == 0 (R itself is); other
  // dims read it one element at a time and finish with the D % 4 last
  // coordinates (partial sums 0, 1, 2: u is zero past D in LDS)
  const bool r_vec4 = (D & 3) == 0;
  for (int j = tid; j < D && !(MODE == kGaProdResid && BITS == 0); j += 256) {
    float4 acc[kGaVec];
#pragma unroll
    for (int v = 0; v < kGaVec; ++v) acc[v] = make_float4(0.f, 0.f, 0.f, 0.f);
    const float* rrow = a.rot + static_cast<int64_t>(j) * D;
    auto fma4 = [&](int m, float4 r) {
#pragma unroll
      for (int v = 0; v < kGaVec; ++v) {
        const float4 u = reinterpret_cast<const float4*>(s_u[v])[m];
        acc[v].x = __builtin_fmaf(u.x, r.x, acc[v].x);
        acc[v].y = __builtin_fmaf(u.y, r.y, acc[v].y);
        acc[v].z = __builtin_fmaf(u.z, r.z, acc[v].z);
        acc[v].w = __builtin_fmaf(u.w, r.w, acc[v].w);
      }
    };
    if (r_vec4) {
      const float4* r4 = reinterpret_cast<const float4*>(rrow);
      for (int m = 0; m < D / 4; ++m) fma4(m, r4[m]);
    } else {
      for (int m = 0; m < D / 4; ++m)
        fma4(m, make_float4(rrow[4 * m], rrow[4 * m + 1], rrow[4 * m + 2], rrow[4 * m + 3]));
      const int d0 = D & ~3;
      const float r0 = rrow[d0];  // D % 4 >= 1 here
      const float r1 = (D & 3) > 1 ? rrow[d0 + 1] : 0.f;
      const float r2 = (D & 3) > 2 ? rrow[d0 + 2] : 0.f;
#pragma unroll
      for (int v = 0; v < kGaVec; ++v) {
        acc[v].x = __builtin_fmaf(s_u[v][d0], r0, acc[v].x);
        if ((D & 3) > 1) acc[v].y = __builtin_fmaf(s_u[v][d0 + 1], r1, acc[v].y);
        if ((D & 3) > 2) acc[v].z = __builtin_fmaf(s_u[v][d0 + 2], r2, acc[v].z);
      }
    }
#pragma unroll
    for (int v = 0; v < kGaVec; ++v) {
      const float y = __fadd_rn(__fadd_rn(acc[v].x, acc[v].y), __fadd_rn(acc[v].z, acc[v].w));
      uint32_t q = 0;
      if constexpr (SGN) {
        q = y >= 0.f ? 1u : 0u;
      } else {
#pragma unroll
        for (int m = 0; m < NMID; ++m) q += y > s_mid[m] ? 1u : 0u;
      }
      s_idx[v][j] = static_cast<uint8_t>(q);
    }
  }
  __syncthreads();
  // pack: thread (vector, word)
  const int PW = (D * BITS + 31) / 32;
  for (int idx = tid; BITS > 0 && idx < kGaVec * PW; idx += 256) {
    const int v = idx / PW;
    const int w = idx % PW;
    const int64_t vec = vec0 + v;
    if (vec >= n_vec) continue;
    uint32_t word = 0;
    constexpr int BD = BITS > 0 ? BITS : 1;  // (no words at 0 bits)
    const int c0 = (32 * w) / BD;
    const int c1 = min(D - 1, (32 * w + 31) / BD);
    for (int c = c0; c <= c1; ++c) {
      const int sh = c * BITS - 32 * w;  // may be negative for a field straddling the word start
      const uint32_t q = s_idx[v][c];
      word |= sh >= 0 ? (q << sh) : (q >> -sh);
    }
    int b, h, l;
    vec_coords(vec, b, h, l);
    const int64_t row = (static_cast<int64_t>(b) * a.H + h) * a.cap + a.offset + l;
    a.packed[row * PW + w] = word;
  }
  if (tid < kGaVec && vec0 + tid < n_vec) {
    int b, h, l;
    vec_coords(vec0 + tid, b, h, l);
    const int64_t row = (static_cast<int64_t>(b) * a.H + h) * a.cap + a.offset + l;
    if (a.norm_dtype == TQ_DTYPE_F16)
      static_cast<uint16_t*>(a.norms)[row] = f32_to_f16_bits(s_nrm[tid]);
    else
      static_cast<float*>(a.norms)[row] = s_nrm[tid];
  }
  if constexpr (MODE == kGaProdResid) {
    // s_idx is complete (the barrier after the products); u is still in s_u
    for (int j = tid; j < D; j += 256) {
      float est[kGaVec];
#pragma unroll
      for (int v = 0; v < kGaVec; ++v) est[v] = 0.f;
      if constexpr (BITS > 0) {
        for (int i = 0; i < D; ++i) {
          const float r = a.rot[static_cast<int64_t>(i) * D + j];
#pragma unroll
          for (int v = 0; v < kGaVec; ++v) est[v] = __builtin_fmaf(s_cb[s_idx[v][i]], r, est[v]);
        }
      }
#pragma unroll
      for (int v = 0; v < kGaVec; ++v)
        if (vec0 + v < n_vec) resid[(vec0 + v) * D + j] = __fsub_rn(s_u[v][j], est[v]);
    }
  }
}

template <int BITS>
int launch_general_bits(const AppendArgs& a, int dim, int x_dtype, hipStream_t st) {
  const int64_t n_vec = static_cast<int64_t>(a.B) * a.H * a.L;
  const dim3 grid(static_cast<unsigned>((n_vec + kGaVec - 1) / kGaVec));
  switch (x_dtype) {
    case TQ_DTYPE_F32: hipLaunchKernelGGL((append_dense_general_kernel<BITS, TQ_DTYPE_F32>), grid, dim3(256), 0, st, a, dim, nullptr, nullptr); break;
    case TQ_DTYPE_F16: hipLaunchKernelGGL((append_dense_general_kernel<BITS, TQ_DTYPE_F16>), grid, dim3(256), 0, st, a, dim, nullptr, nullptr); break;
    default: hipLaunchKernelGGL((append_dense_general_kernel<BITS, TQ_DTYPE_BF16>), grid, dim3(256), 0, st, a, dim, nullptr, nullptr); break;
  }
  return check_launch("append_dense_general_kernel");
}

// ------------------------------------------------------------- dequantize ---
// out[b,h,t,:] = n * R^-1(codebook[idx]) for one vector per workgroup:
// codebook values in LDS, then Hadamard butterflies in LDS (x rscale x signs)
// or the dense product out[j] = sum_d y[d] R[d][j] (coalesced over j).
__global__ __launch_bounds__(256) void dequant_general_kernel(DequantGeneralArgs a) {
  __shared__ float s_y[kGaMaxDim];
  const int64_t vec = blockIdx.x;  // (b*H + h)*T + t
  const int t = static_cast<int>(vec % a.T);
  const int64_t bh = vec / a.T;
  const int64_t row = bh * a.cap + t;
  const int D = a.D;
  const uint32_t* w = a.packed + row * a.PW;
  for (int d = threadIdx.x; d < D; d += 256) {
    const int bit = d * a.bits;
    const int wi = bit >> 5;
    const int sh = bit & 31;
    uint32_t x = w[wi] >> sh;
    if (sh + a.bits > 32) x |= w[wi + 1] << (32 - sh);
    s_y[d] = a.cb[x & ((1u << a.bits) - 1u)];
  }
  __syncthreads();
  const float n = load_norm(a.norms, a.norm_dtype, row);
  float* out = a.out + vec * D;
  if (a.rot_kind == TQ_ROT_HADAMARD) {
    for (int hs = 1; hs < D; hs <<= 1) {
      for (int k = threadIdx.x; k < D / 2; k += 256) {
        const int i0 = (k / hs) * 2 * hs + (k % hs);
        const float p = s_y[i0];
        const float q = s_y[i0 + hs];
        s_y[i0] = p + q;
        s_y[i0 + hs] = p - q;
      }
      __syncthreads();
    }
    for (int d = threadIdx.x; d < D; d += 256) out[d] = n * (s_y[d] * a.scale * a.rot[d]);
    return;
  }
  for (int j = threadIdx.x; j < D; j += 256) {
    float acc = 0.f;
    for (int d = 0; d < D; ++d) acc = __builtin_fmaf(s_y[d], a.rot[static_cast<int64_t>(d) * D + j], acc);
    out[j] = n * acc;
  }
}

}  // namespace

int launch_append_dense_general(const AppendArgs& a, int dim, int bits, int x_dtype, hipStream_t st) {
  if (dim < 8 || dim > kGaMaxDim)
    return fail(TQ_ERR_UNSUPPORTED, "append: dense rotation at dim %d (8..512)", dim);
  if ((reinterpret_cast<uintptr_t>(a.rot) & 15u) != 0)
    return fail(TQ_ERR_INVALID_ARGUMENT, "append: dense rotation matrix must be 16-byte aligned");
  switch (bits) {
    case 1: return launch_general_bits<1>(a, dim, x_dtype, st);
    case 2: return launch_general_bits<2>(a, dim, x_dtype, st);
    case 3: return launch_general_bits<3>(a, dim, x_dtype, st);
    case 4: return launch_general_bits<4>(a, dim, x_dtype, st);
  }
  return fail(TQ_ERR_INVALID_ARGUMENT, "append: bits %d not in 1..4", bits);
}

int launch_append_dense_signs_general(const AppendArgs& a, int dim, hipStream_t st) {
  if (dim < 8 || dim > kGaMaxDim)
    return fail(TQ_ERR_UNSUPPORTED, "prod: dim %d (8..512)", dim);
  const int64_t n_vec = static_cast<int64_t>(a.B) * a.H * a.L;
  hipLaunchKernelGGL((append_dense_general_kernel<1, TQ_DTYPE_F32, kGaSigns>),
                     dim3(static_cast<unsigned>((n_vec + kGaVec - 1) / kGaVec)), dim3(256), 0, st, a, dim,
                     nullptr, nullptr);
  return check_launch("append_dense_general_kernel (signs)");
}

template <int MB>
int launch_prod_resid_mb(const AppendArgs& a, int dim, int x_dtype, float* resid, const float* cb,
                         hipStream_t st) {
  const int64_t n_vec = static_cast<int64_t>(a.B) * a.H * a.L;
  const dim3 grid(static_cast<unsigned>((n_vec + kGaVec - 1) / kGaVec));
  switch (x_dtype) {
    case TQ_DTYPE_F32: hipLaunchKernelGGL((append_dense_general_kernel<MB, TQ_DTYPE_F32, kGaProdResid>), grid, dim3(256), 0, st, a, dim, resid, cb); break;
    case TQ_DTYPE_F16: hipLaunchKernelGGL((append_dense_general_kernel<MB, TQ_DTYPE_F16, kGaProdResid>), grid, dim3(256), 0, st, a, dim, resid, cb); break;
    default: hipLaunchKernelGGL((append_dense_general_kernel<MB, TQ_DTYPE_BF16, kGaProdResid>), grid, dim3(256), 0, st, a, dim, resid, cb); break;
  }
  return check_launch("append_dense_general_kernel (prod residual)");
}

int launch_prod_residual_dense(const AppendArgs& a, int dim, int mb, int x_dtype, float* resid,
                               const float* cb, hipStream_t st) {
  if (dim < 8 || dim > kGaMaxDim)
    return fail(TQ_ERR_UNSUPPORTED, "prod: dim %d (8..512)", dim);
  if ((reinterpret_cast<uintptr_t>(a.rot) & 15u) != 0)
    return fail(TQ_ERR_INVALID_ARGUMENT, "prod: dense rotation matrix must be 16-byte aligned");
  switch (mb) {
    case 0: return launch_prod_resid_mb<0>(a, dim, x_dtype, resid, cb, st);
    case 1: return launch_prod_resid_mb<1>(a, dim, x_dtype, resid, cb, st);
    case 2: return launch_prod_resid_mb<2>(a, dim, x_dtype, resid, cb, st);
    case 3: return launch_prod_resid_mb<3>(a, dim, x_dtype, resid, cb, st);
  }
  return fail(TQ_ERR_INVALID_ARGUMENT, "prod: bits %d not in 1..4", mb + 1);
}

int launch_dequant_general(const DequantGeneralArgs& a, int64_t n_vec, hipStream_t st) {
  hipLaunchKernelGGL(dequant_general_kernel, dim3(static_cast<unsigned>(n_vec)), dim3(256), 0, st, a);
  return check_launch("dequant_general_kernel");
}

}  // namespace tq
