// Prod codec (turboquant_cache.py:4572-4766): MSE quantization at bits - 1
// plus a one-bit QJL sketch of the residual, for keys whose inner products
// with queries should be unbiased.
//
// Quantize (array path, :4653-4666) runs as two kernels on the caller's
// stream:
//   prod_residual_kernel  n = ||x||, u = x / max(n, 1e-6), the MSE indices of
//                         u at bits - 1 (Hadamard rotation, same f32 order as
//                         append_rht_kernel), the estimate R^-1(c[idx]) and the
//                         residual u - estimate, written in f32 to a workspace;
//   append_dense_kernel   (signs variant) residual @ P^T on the matrix cores
//                         with one-bit output (>= 0) and ||residual|| (d = 32
//                         and 512: the general dense kernel's signs mode).
// Dequantize (:4668-4677): n * (R^-1(c[idx]) + sqrt(pi/2)/D * rn * (s @ P)).
#include <type_traits>

#include "tq_append.h"

namespace tq {

struct ProdArgs {
  const void* x;
  int64_t sb, sh, sl;
  int B, H, L;
  const float* signs;  // Hadamard signs of the MSE rotation (D)
  const float* mid;    // 2^mb - 1 midpoints (mb = bits - 1 >= 1)
  const float* cb;     // 2^mb centroids
  uint32_t* mse;       // (B, H, cap, D * mb / 32), may be null when mb = 0
  void* norms;
  int norm_dtype;
  int64_t cap, offset;
  float scale;         // f32(1/sqrt(D))
  float* resid;        // (B * H * L, D) f32 workspace
};

template <int DT>
__device__ __forceinline__ void load32p(const void* p, float (&v)[32]) {
  if constexpr (DT == TQ_DTYPE_F32) {
    const float4* q = static_cast<const float4*>(p);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float4 t = q[i];
      v[4 * i] = t.x;
      v[4 * i + 1] = t.y;
      v[4 * i + 2] = t.z;
      v[4 * i + 3] = t.w;
    }
  } else {
    const uint4* q = static_cast<const uint4*>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint4 t = q[i];
      const uint32_t w[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint16_t lo = static_cast<uint16_t>(w[j] & 0xffffu), hi = static_cast<uint16_t>(w[j] >> 16);
        v[8 * i + 2 * j] = DT == TQ_DTYPE_F16 ? f16_bits_to_f32(lo) : bf16_bits_to_f32(lo);
        v[8 * i + 2 * j + 1] = DT == TQ_DTYPE_F16 ? f16_bits_to_f32(hi) : bf16_bits_to_f32(hi);
      }
    }
  }
}

// Unnormalised Walsh-Hadamard transform of the D-vector a group of NL = D/32
// lanes holds (lane g: elements 32g .. 32g + 31): distances 1 .. 16 in the
// lane, then 32, 64, ... across lanes -- the order of append_rht_kernel.
template <int NL>
__device__ __forceinline__ void group_fwht(float (&v)[32], int g) {
#pragma unroll
  for (int hstep = 1; hstep < 32; hstep <<= 1) {
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      if ((i & hstep) == 0) {
        const float x0 = v[i], x1 = v[i + hstep];
        v[i] = __fadd_rn(x0, x1);
        v[i + hstep] = __fsub_rn(x0, x1);
      }
    }
  }
  auto cross = [&](auto off_tag) {
    constexpr int OFF = decltype(off_tag)::value;
    const float sg = (g & OFF) != 0 ? -1.f : 1.f;
#pragma unroll
    for (int i = 0; i < 32; ++i) v[i] = __builtin_fmaf(v[i], sg, xor_lane<OFF>(v[i]));
  };
  if constexpr (NL >= 2) cross(std::integral_constant<int, 1>{});
  if constexpr (NL >= 4) cross(std::integral_constant<int, 2>{});
  if constexpr (NL >= 8) cross(std::integral_constant<int, 4>{});
  if constexpr (NL >= 16) cross(std::integral_constant<int, 8>{});
}

template <int D, int MB, int XDT>
__global__ __launch_bounds__(256) void prod_residual_kernel(ProdArgs a) {
  constexpr int NL = D / 32;
  constexpr int VPB = 256 / NL;
  constexpr int NMID = MB > 0 ? (1 << MB) - 1 : 1;
  constexpr int PW = D * MB / 32;
  __shared__ float s_sign[D];
  __shared__ float s_mid[NMID];
  __shared__ float s_cb[NMID + 1];
  for (int i = threadIdx.x; i < D; i += blockDim.x) s_sign[i] = a.signs[i];
  if constexpr (MB > 0) {
    if (threadIdx.x < NMID) s_mid[threadIdx.x] = a.mid[threadIdx.x];
    if (threadIdx.x <= NMID) s_cb[threadIdx.x] = a.cb[threadIdx.x];
  }
  __syncthreads();

  const int64_t n_vec = static_cast<int64_t>(a.B) * a.H * a.L;
  const int64_t vec = static_cast<int64_t>(blockIdx.x) * VPB + threadIdx.x / NL;
  const int g = threadIdx.x % NL;
  if (vec >= n_vec) return;  // whole lane groups leave together
  const int l = static_cast<int>(vec % a.L);
  const int64_t bh = vec / a.L;
  const int h = static_cast<int>(bh % a.H);
  const int b = static_cast<int>(bh / a.H);
  constexpr int ES = XDT == TQ_DTYPE_F32 ? 4 : 2;
  float v[32];
  load32p<XDT>(static_cast<const char*>(a.x) + (b * a.sb + h * a.sh + l * a.sl + g * 32) * ES, v);

  // ---- norm (the append kernels' tree) and u = x / max(n, eps)
  float s[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) s[i] = __fadd_rn(__fmul_rn(v[i], v[i]), __fmul_rn(v[i + 16], v[i + 16]));
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
  float u[32];
  div_by_norm<XDT>(v, den, u);

  const int64_t row = (static_cast<int64_t>(b) * a.H + h) * a.cap + a.offset + l;
  if constexpr (MB > 0) {
    // ---- MSE indices of u: y = H(s * u) / sqrt(D), idx = #{y > mid}
#pragma unroll
    for (int i = 0; i < 32; ++i) v[i] = __fmul_rn(u[i], s_sign[g * 32 + i]);
    group_fwht<NL>(v, g);
    uint32_t words[MB];
#pragma unroll
    for (int w = 0; w < MB; ++w) words[w] = 0u;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      const float y = __fmul_rn(v[i], a.scale);
      uint32_t idx = 0;
#pragma unroll
      for (int m = 0; m < NMID; ++m) idx += (y > s_mid[m]) ? 1u : 0u;
      v[i] = s_cb[idx];  // the estimate in the rotated basis
      const int pos = i * MB;
      words[pos >> 5] |= idx << (pos & 31);
      if ((pos & 31) + MB > 32) words[(pos >> 5) + 1] |= idx >> (32 - (pos & 31));
    }
    uint32_t* dst = a.mse + row * PW + g * MB;
#pragma unroll
    for (int w = 0; w < MB; ++w) dst[w] = words[w];
    // ---- estimate R^-1(c[idx]) = s * (H(c[idx]) / sqrt(D)); residual u - estimate
    group_fwht<NL>(v, g);
#pragma unroll
    for (int i = 0; i < 32; ++i) u[i] = __fsub_rn(u[i], __fmul_rn(__fmul_rn(v[i], a.scale), s_sign[g * 32 + i]));
  }
  float4* rdst = reinterpret_cast<float4*>(a.resid + vec * D + g * 32);
#pragma unroll
  for (int i = 0; i < 8; ++i) rdst[i] = make_float4(u[4 * i], u[4 * i + 1], u[4 * i + 2], u[4 * i + 3]);
  if (g == 0) {
    if (a.norm_dtype == TQ_DTYPE_F16)
      static_cast<uint16_t*>(a.norms)[row] = f32_to_f16_bits(n);
    else
      static_cast<float*>(a.norms)[row] = n;
  }
}

// ------------------------------------------------------------- dequantize ---
struct ProdDequantArgs {
  const void* norms;
  const uint32_t* mse;
  const void* rnorms;
  const uint32_t* sgn;
  int norm_dtype;
  int B, H, T, D, mb;
  int dense;  // MSE rotation: 0 Hadamard (signs = its D signs), 1 dense (signs = R, D x D)
  int spw;    // sign words per row, ceil(D / 32)
  int64_t cap;
  const float* signs;
  const float* cb;
  const float* proj;
  float scale, qjl_scale;
  float* out;  // (B, H, T, D)
};

__device__ __forceinline__ float load_nrm(const void* p, int dt, int64_t i) {
  return dt == TQ_DTYPE_F16 ? f16_bits_to_f32(static_cast<const uint16_t*>(p)[i]) : static_cast<const float*>(p)[i];
}

// One block per token vector (min(D, 256) threads); thread i forms
// coordinates i, i + 256, ... (D up to 512; Hadamard: a power of two).  The
// MSE estimate is R^-1(c[idx]): Hadamard butterflies, or c[idx] @ R for the
// dense rotation (_rotate_inverse, turboquant_cache.py:4146-4149).
constexpr int kProdDqMaxDim = 512;

__global__ __launch_bounds__(256) void prod_dequant_kernel(ProdDequantArgs a) {
  __shared__ float s_y[kProdDqMaxDim];
  __shared__ float s_s[kProdDqMaxDim];
  const int nt = blockDim.x;
  const int64_t vec = blockIdx.x;  // (b * H + h) * T + t
  const int t = static_cast<int>(vec % a.T);
  const int64_t bh = vec / a.T;
  const int64_t row = bh * a.cap + t;
  const int D = a.D;
  for (int i = threadIdx.x; i < D; i += nt) {
    s_s[i] = ((a.sgn[row * a.spw + i / 32] >> (i % 32)) & 1u) ? 1.f : -1.f;
    if (a.mb > 0) {
      const int pw = (D * a.mb + 31) / 32;
      const int pos = i * a.mb;
      uint32_t idx = a.mse[row * pw + (pos >> 5)] >> (pos & 31);
      if ((pos & 31) + a.mb > 32) idx |= a.mse[row * pw + (pos >> 5) + 1] << (32 - (pos & 31));
      s_y[i] = a.cb[idx & ((1u << a.mb) - 1u)];
    }
  }
  __syncthreads();
  if (a.mb > 0 && !a.dense) {
    // butterflies at distance hs: thread k of D / 2 takes the pair (i0, i0 + hs)
    for (int hs = 1; hs < D; hs <<= 1) {
      for (int k = threadIdx.x; k < D / 2; k += nt) {
        const int i0 = (k / hs) * 2 * hs + (k % hs);
        const float x0 = s_y[i0], x1 = s_y[i0 + hs];
        s_y[i0] = x0 + x1;
        s_y[i0 + hs] = x0 - x1;
      }
      __syncthreads();
    }
  }
  const float n = load_nrm(a.norms, a.norm_dtype, row);
  const float rn = load_nrm(a.rnorms, a.norm_dtype, row);
  for (int i = threadIdx.x; i < D; i += nt) {
    float mse = 0.f;
    if (a.mb > 0 && a.dense) {
      for (int d = 0; d < D; ++d) mse = fmaf(s_y[d], a.signs[static_cast<int64_t>(d) * D + i], mse);
    } else if (a.mb > 0) {
      mse = s_y[i] * a.scale * a.signs[i];
    }
    float qjl = 0.f;  // (s @ P)[i]
    for (int j = 0; j < D; ++j) qjl = fmaf(s_s[j], a.proj[static_cast<int64_t>(j) * D + i], qjl);
    a.out[vec * D + i] = n * (mse + a.qjl_scale * rn * qjl);
  }
}

}  // namespace tq

using namespace tq;

namespace {

template <int D, int MB>
int launch_residual_mb(const ProdArgs& a, int x_dtype, hipStream_t st) {
  constexpr int VPB = 256 / (D / 32);
  const int64_t n_vec = static_cast<int64_t>(a.B) * a.H * a.L;
  const dim3 grid(static_cast<unsigned>((n_vec + VPB - 1) / VPB));
  switch (x_dtype) {
    case TQ_DTYPE_F32: hipLaunchKernelGGL((prod_residual_kernel<D, MB, TQ_DTYPE_F32>), grid, dim3(256), 0, st, a); break;
    case TQ_DTYPE_F16: hipLaunchKernelGGL((prod_residual_kernel<D, MB, TQ_DTYPE_F16>), grid, dim3(256), 0, st, a); break;
    default: hipLaunchKernelGGL((prod_residual_kernel<D, MB, TQ_DTYPE_BF16>), grid, dim3(256), 0, st, a); break;
  }
  return check_launch("prod_residual_kernel");
}

template <int D>
int launch_residual(const ProdArgs& a, int mb, int x_dtype, hipStream_t st) {
  switch (mb) {
    case 0: return launch_residual_mb<D, 0>(a, x_dtype, st);
    case 1: return launch_residual_mb<D, 1>(a, x_dtype, st);
    case 2: return launch_residual_mb<D, 2>(a, x_dtype, st);
    case 3: return launch_residual_mb<D, 3>(a, x_dtype, st);
  }
  return fail(TQ_ERR_INVALID_ARGUMENT, "prod: bits %d not in 1..4", mb + 1);
}

bool aligned16p(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

extern "C" int64_t tq_prod_workspace_size(int B, int H, int L, int dim) {
  if (B < 0 || H < 0 || L < 0 || dim <= 0) return 0;
  return (static_cast<int64_t>(B) * H * L * dim * 4 + 255) / 256 * 256;
}

extern "C" int tq_prod_quantize(const void* x, int x_dtype, int B, int H, int L, int dim,
                                int64_t x_stride_b, int64_t x_stride_h, int64_t x_stride_l,
                                int bits, const float* signs, const float* mse_midpoints,
                                const float* mse_codebook, const float* projection,
                                uint32_t* mse_packed, void* norms, uint32_t* qjl_signs,
                                void* residual_norms, int norm_dtype, int64_t capacity,
                                int64_t offset, void* workspace, int64_t workspace_bytes,
                                void* stream) {
  if (B < 0 || H < 0 || L < 0) return fail(TQ_ERR_INVALID_ARGUMENT, "prod: negative shape");
  if (bits < 1 || bits > 4) return fail(TQ_ERR_INVALID_ARGUMENT, "prod: bits %d not in 1..4", bits);
  // powers of two in 32..512: the Hadamard rotation (signs = its dim signs);
  // other dims in 8..512: the dense one (signs = R, dim x dim), as the MSE
  // codec picks (turboquant_cache.py:4122-4139)
  const bool pow2d = (dim & (dim - 1)) == 0;
  if (dim < 8 || dim > 512 || (pow2d && dim < 32))
    return fail(TQ_ERR_UNSUPPORTED, "prod: dim %d (8..512; powers of two from 32)", dim);
  if (norm_dtype != TQ_DTYPE_F32 && norm_dtype != TQ_DTYPE_F16)
    return fail(TQ_ERR_INVALID_ARGUMENT, "prod: norm_dtype %d", norm_dtype);
  if (x_dtype != TQ_DTYPE_F32 && x_dtype != TQ_DTYPE_F16 && x_dtype != TQ_DTYPE_BF16)
    return fail(TQ_ERR_INVALID_ARGUMENT, "prod: x_dtype %d", x_dtype);
  if (offset < 0 || offset + L > capacity)
    return fail(TQ_ERR_INVALID_ARGUMENT, "prod: tokens [%lld, %lld) exceed capacity %lld",
                (long long)offset, (long long)(offset + L), (long long)capacity);
  const int64_t n_vec = static_cast<int64_t>(B) * H * L;
  if (n_vec == 0) return TQ_OK;
  const int mb = bits - 1;
  if (!x || !signs || !projection || !norms || !qjl_signs || !residual_norms || !workspace ||
      (mb > 0 && (!mse_midpoints || !mse_codebook || !mse_packed)))
    return fail(TQ_ERR_INVALID_ARGUMENT, "prod: null pointer");
  if (workspace_bytes < tq_prod_workspace_size(B, H, L, dim))
    return fail(TQ_ERR_WORKSPACE, "prod: workspace %lld < %lld bytes", (long long)workspace_bytes,
                (long long)tq_prod_workspace_size(B, H, L, dim));
  const int es = x_dtype == TQ_DTYPE_F32 ? 4 : 2;
  if (!aligned16p(workspace) || (pow2d && (!aligned16p(x) || (x_stride_b * es) % 16 ||
                                           (x_stride_h * es) % 16 || (x_stride_l * es) % 16)))
    return fail(TQ_ERR_INVALID_ARGUMENT, "prod: x, its strides and the workspace must be 16-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  ProdArgs a{x, x_stride_b, x_stride_h, x_stride_l, B, H, L, signs, mse_midpoints, mse_codebook,
             mse_packed, norms, norm_dtype, capacity, offset,
             static_cast<float>(1.0 / __builtin_sqrt(static_cast<double>(dim))),
             static_cast<float*>(workspace)};
  int rc = TQ_OK;
  if (!pow2d) {
    AppendArgs r{};
    r.x = x;
    r.sb = x_stride_b;
    r.sh = x_stride_h;
    r.sl = x_stride_l;
    r.B = B;
    r.H = H;
    r.L = L;
    r.rot = signs;
    r.mid = mse_midpoints;
    r.packed = mse_packed;
    r.norms = norms;
    r.norm_dtype = norm_dtype;
    r.cap = capacity;
    r.offset = offset;
    r.scale = 1.f;
    rc = launch_prod_residual_dense(r, dim, mb, x_dtype, static_cast<float*>(workspace), mse_codebook, st);
  } else switch (dim) {
    case 32: rc = launch_residual<32>(a, mb, x_dtype, st); break;
    case 64: rc = launch_residual<64>(a, mb, x_dtype, st); break;
    case 128: rc = launch_residual<128>(a, mb, x_dtype, st); break;
    case 256: rc = launch_residual<256>(a, mb, x_dtype, st); break;
    default: rc = launch_residual<512>(a, mb, x_dtype, st); break;
  }
  if (rc) return rc;
  // signs of residual @ P^T and ||residual||, written at the same rows
  AppendArgs s{};
  s.x = workspace;
  s.sl = dim;
  s.sh = static_cast<int64_t>(L) * dim;
  s.sb = static_cast<int64_t>(H) * L * dim;
  s.B = B;
  s.H = H;
  s.L = L;
  s.rot = projection;
  s.mid = nullptr;
  s.packed = qjl_signs;
  s.norms = residual_norms;
  s.norm_dtype = norm_dtype;
  s.cap = capacity;
  s.offset = offset;
  s.scale = 1.f;
  return launch_append_dense_signs(s, dim, st);
}

extern "C" int tq_prod_dequantize(const void* norms, const uint32_t* mse_packed,
                                  const void* residual_norms, const uint32_t* qjl_signs,
                                  int norm_dtype, int B, int H, int T, int dim, int bits,
                                  int64_t capacity, const float* signs, const float* mse_codebook,
                                  const float* projection, float* out, void* stream) {
  if (B < 0 || H < 0 || T < 0 || T > capacity)
    return fail(TQ_ERR_INVALID_ARGUMENT, "prod dequantize: bad shape");
  if (bits < 1 || bits > 4) return fail(TQ_ERR_INVALID_ARGUMENT, "prod dequantize: bits %d", bits);
  const bool pow2d = (dim & (dim - 1)) == 0;
  if (dim < 8 || dim > 512 || (pow2d && dim < 32))
    return fail(TQ_ERR_UNSUPPORTED, "prod dequantize: dim %d (8..512; powers of two from 32)", dim);
  if (norm_dtype != TQ_DTYPE_F32 && norm_dtype != TQ_DTYPE_F16)
    return fail(TQ_ERR_INVALID_ARGUMENT, "prod dequantize: norm_dtype %d", norm_dtype);
  const int64_t n = static_cast<int64_t>(B) * H * T;
  if (n == 0) return TQ_OK;
  if (!norms || !residual_norms || !qjl_signs || !signs || !projection || !out ||
      (bits > 1 && (!mse_packed || !mse_codebook)))
    return fail(TQ_ERR_INVALID_ARGUMENT, "prod dequantize: null pointer");
  if (n > 0x7fffffff) return fail(TQ_ERR_UNSUPPORTED, "prod dequantize: too many vectors");
  ProdDequantArgs a{norms, mse_packed, residual_norms, qjl_signs, norm_dtype, B, H, T, dim, bits - 1,
                    pow2d ? 0 : 1, (dim + 31) / 32, capacity, signs, mse_codebook, projection,
                    static_cast<float>(1.0 / __builtin_sqrt(static_cast<double>(dim))),
                    static_cast<float>(__builtin_sqrt(3.14159265358979323846 / 2.0) / dim), out};
  hipLaunchKernelGGL(prod_dequant_kernel, dim3(static_cast<unsigned>(n)), dim3(dim < 256 ? dim : 256), 0,
                     static_cast<hipStream_t>(stream), a);
  return check_launch("prod_dequant_kernel");
}
