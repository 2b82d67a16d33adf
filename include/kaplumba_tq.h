/*
 * kaplumba_tq.h -- C ABI of the MI355X TurboQuant KV-cache library
 * (libkaplumba_tq.so, hand-written HIP kernels for gfx950).
 *
 * Every entry point takes plain device pointers, sizes and a hipStream_t
 * passed as void*, returns a status code (0 = success) and never throws.
 * Work is enqueued asynchronously on the given stream; all buffers are
 * caller-allocated device memory.  No entry point allocates device memory.
 *
 * Layouts (row-major, innermost last):
 *   input vectors x      : [B, H, L, dim] with element strides (sb, sh, sl), last dim contiguous
 *   packed indices       : [B, H, capacity, PW] uint32, PW = ceil(dim*bits/32),
 *                          LSB-first bit stream: element i occupies bits i*bits.. of the row
 *   norms                : [B, H, capacity] float32 or float16
 *   plain (fp16/bf16) KV : [B, H, capacity, dim]
 *   attention output     : [B, Hq, L, dim] in the query dtype
 *
 * The reference is the mlx-lm TurboQuant cache of zayutaha/kaplumba,
 * mlx_lm/models/turboquant_cache.py (cited below as tq.py) and
 * mlx_lm/models/base.py / cache.py.  The reference is Python calling Metal
 * kernels through mx.fast.metal_kernel; a maintainer binds these symbols with
 * ctypes (see kaplumba_amd/_lib.py).
 */
#ifndef KAPLUMBA_TQ_H
#define KAPLUMBA_TQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------ */
enum {
  TQ_OK = 0,
  TQ_ERR_INVALID_ARGUMENT = 1, /* bad shape, bits, dtype, null pointer, ... */
  TQ_ERR_UNSUPPORTED = 2,      /* valid request outside the compiled kernel set */
  TQ_ERR_WORKSPACE = 3,        /* workspace smaller than tq_attention_workspace_size() */
  TQ_ERR_HIP = 4               /* a HIP runtime call failed (message has the HIP error) */
};

/* ---- enums ------------------------------------------------------------- */
enum { TQ_DTYPE_F32 = 0, TQ_DTYPE_F16 = 1, TQ_DTYPE_BF16 = 2 };
enum { TQ_ROT_HADAMARD = 0, TQ_ROT_DENSE = 1 };
enum { TQ_KV_PACKED = 0, TQ_KV_PLAIN = 1, TQ_KV_PROD = 2 /* tq_attention_prod keys */ };
/* Array attention masks (tq_attention_general): boolean (uint8, nonzero keeps
 * the score) or additive in f32 / f16 / bf16. */
enum { TQ_MASK_NONE = 0, TQ_MASK_BOOL = 1, TQ_MASK_ADD_F32 = 2, TQ_MASK_ADD_F16 = 3,
       TQ_MASK_ADD_BF16 = 4 };

/* Library version string, e.g. "kaplumba_tq 0.1.0 gfx950". */
const char* tq_version(void);

/* Human-readable message for the last failing call on this host thread. */
const char* tq_last_error(void);

/* Packed row width in uint32 words: ceil(dim*bits/32)
 * (replaces _packed_width, tq.py:3699-3702). */
int tq_packed_width(int dim, int bits);

/*
 * Append-time quantization of L new tokens per (batch, head).
 *
 * Replaces _TurboQuantMSECodec.quantize (tq.py:4186-4254) together with
 * _write_state (tq.py:3978-3986) as used by TurboQuantKVCache.update_and_fetch
 * (tq.py:5026-5064): for every vector x,
 *   n = ||x||_2 (f32), u = x / max(n, 1e-6),
 *   y = H(s * u) / sqrt(dim)   (rot_kind TQ_ROT_HADAMARD, rot = s: dim floats)
 *   y = u @ R^T                (rot_kind TQ_ROT_DENSE, rot = R: dim*dim floats, row-major)
 *   idx_i = #{ m : y_i > midpoints[m] }   (2^bits - 1 ascending midpoints)
 * and writes the packed row and the norm at token position offset + l of the
 * (b, h) row of the destination buffers (capacity tokens per (b, h)).
 * Hadamard: dim a power of two in [32, 512].  Dense: any dim in [8, 512]
 * (64 / 128 / 256 on the matrix cores, other dims on the vector ALUs).  x and
 * its strides must be 16-byte aligned when dim is a multiple of 8.
 * bits in 1..4.  x_dtype: F32/F16/BF16.  norm_dtype: F32 or F16.
 */
int tq_append_quantize(const void* x, int x_dtype, int B, int H, int L, int dim,
                       int64_t x_stride_b, int64_t x_stride_h, int64_t x_stride_l,
                       int bits, int rot_kind, const float* rot, const float* midpoints,
                       uint32_t* packed, void* norms, int norm_dtype,
                       int64_t capacity, int64_t offset, void* stream);

/*
 * The keys and the values of one update_and_fetch (tq.py:5026-5064: its two
 * _TurboQuantMSECodec.quantize calls, tq.py:4186-4254, and their
 * _write_state) in one call.  Each side is exactly tq_append_quantize with
 * its own x, strides, bits, rotation vector / matrix, midpoints and
 * destination; the shape (B, H, L, dim), x_dtype, rot_kind, norm_dtype,
 * capacity and offset are shared.  F16 / BF16 input at dim 64 / 128 / 256
 * with equal widths or v_bits = k_bits + 1 (the x.5-bit split) runs both
 * sides in one kernel launch, for either rotation; other cases run the two
 * quantizers one after the other.  Results are identical either way.
 */
int tq_append_quantize_kv(const void* k_x, const void* v_x, int x_dtype, int B, int H, int L,
                          int dim, int64_t k_stride_b, int64_t k_stride_h, int64_t k_stride_l,
                          int64_t v_stride_b, int64_t v_stride_h, int64_t v_stride_l,
                          int k_bits, int v_bits, int rot_kind,
                          const float* k_rot, const float* v_rot,
                          const float* k_midpoints, const float* v_midpoints,
                          uint32_t* k_packed, void* k_norms, uint32_t* v_packed, void* v_norms,
                          int norm_dtype, int64_t capacity, int64_t offset, void* stream);

/*
 * Append L tokens unquantized into an fp16/bf16 layer buffer (the
 * mixed-precision layers).  Replaces the slice assignment of
 * KVCache.update_and_fetch (cache.py:415-441).  dtype: F16 or BF16; x and dst
 * share it.  dst is [B, H, capacity, dim].  Any dim >= 1 (16-byte copies when
 * dim is a multiple of 8 and the rows are 16-byte aligned, else per element).
 */
int tq_append_plain(const void* x, int dtype, int B, int H, int L, int dim,
                    int64_t x_stride_b, int64_t x_stride_h, int64_t x_stride_l,
                    void* dst, int64_t capacity, int64_t offset, void* stream);

/*
 * Unpack and dequantize vectors: out[b,h,t,:] = n * R^-1(codebook[idx]),
 * f32 output [B, H, T, dim] for tokens 0..T-1.  Replaces
 * TurboQuantKVCache.dequantize (tq.py:5070-5077).  Used by tests and by the
 * cache's dequantize() API, not by attention.
 */
int tq_dequantize(const uint32_t* packed, const void* norms, int norm_dtype,
                  int B, int H, int T, int dim, int bits, int64_t capacity,
                  const float* codebook, int rot_kind, const float* rot,
                  float* out, void* stream);

/*
 * Prod codec (_TurboQuantProdCodec, tq.py:4572-4766): MSE at mb = bits - 1
 * bits plus a one-bit QJL sketch of the residual.  Replaces its quantize
 * (array path, tq.py:4653-4666; the fused single-token kernel,
 * tq.py:2968-3116, computes the same quantities): for every vector x,
 *   n = ||x||_2 (f32), u = x / max(n, 1e-6),
 *   idx = MSE indices of u at mb bits (the midpoints and order of
 *         tq_append_quantize) with the MSE codec's rotation: the Hadamard
 *         one at power-of-two dims (`signs` = its dim signs), the dense one
 *         at other dims (`signs` = R, dim x dim row-major, 16-byte aligned),
 *         as turboquant_cache.py:4122-4139 picks; packed to mse_packed
 *         [B, H, capacity, ceil(dim*mb/32)]; with bits == 1 no MSE part,
 *   r = u - R^-1(codebook[idx]): s * (H(codebook[idx]) / sqrt(dim)), or
 *       codebook[idx] @ R for the dense rotation   (u when bits == 1),
 *   rn = ||r||_2, signs of r @ P^T (1 where >= 0) packed one bit each to
 *   qjl_signs [B, H, capacity, ceil(dim/32)]; n and rn go to norms /
 *   residual_norms [B, H, capacity] in norm_dtype.
 * P (projection, dim x dim f32 row-major, 16-byte aligned) is
 * default_rng(seed + 1 + 2971*dim + 17).standard_normal (tq.py:3579-3584).
 * dim: powers of two in 32..512, other dims in 8..512 (the sign projection
 * of d = 64 / 128 / 256 on the matrix cores, of the others on the vector
 * ALUs; x and its strides 16-byte aligned at the powers of two); the workspace
 * (>= tq_prod_workspace_size bytes,
 * 16-byte aligned) holds the f32 residuals between the two kernels.
 */
int64_t tq_prod_workspace_size(int B, int H, int L, int dim);
int tq_prod_quantize(const void* x, int x_dtype, int B, int H, int L, int dim,
                     int64_t x_stride_b, int64_t x_stride_h, int64_t x_stride_l,
                     int bits, const float* signs, const float* mse_midpoints,
                     const float* mse_codebook, const float* projection,
                     uint32_t* mse_packed, void* norms, uint32_t* qjl_signs,
                     void* residual_norms, int norm_dtype, int64_t capacity, int64_t offset,
                     void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Prod dequantize (tq.py:4668-4677), f32 [B, H, T, dim]:
 *   out = n * (R^-1(codebook[idx]) + sqrt(pi/2)/dim * rn * (q @ P)),
 * q_j = +1 where sign bit j is set, else -1; R^-1 and `signs` as in
 * tq_prod_quantize (dims as there).
 */
int tq_prod_dequantize(const void* norms, const uint32_t* mse_packed, const void* residual_norms,
                       const uint32_t* qjl_signs, int norm_dtype, int B, int H, int T, int dim,
                       int bits, int64_t capacity, const float* signs, const float* mse_codebook,
                       const float* projection, float* out, void* stream);

/*
 * Bytes of workspace tq_attention() / tq_attention_ranged() need for this
 * problem (split-K partials and rotated queries).  max_tokens is the largest
 * per-sequence cache length.  tq_attention_prod_workspace_size() is the same
 * for tq_attention_prod (its general-kernel shapes add a projected-query
 * region).
 */
int64_t tq_attention_workspace_size(int B, int Hq, int Hkv, int L, int dim,
                                    int64_t max_tokens);
int64_t tq_attention_prod_workspace_size(int B, int Hq, int Hkv, int L, int dim,
                                         int64_t max_tokens);

/*
 * Decode / speculative-verify attention straight from the cache.
 *
 * Replaces TurboQuantKVCache.decode_attention (tq.py:5776-5947) for L == 1,
 * the dequantize + SDPA fallback of scaled_dot_product_attention
 * (base.py:177-189) for L > 1, and the plain SDPA of the fp16 layers
 * (base.py:218-226).  Semantics follow quantized_attention (tq.py:5110-5203):
 *   q_s   = round_qdtype(q * round_qdtype(scale))
 *   q_rot = R_K(q_s)
 *   s_t   = n_k[t] * <q_rot, codebook_k[idx_k[t]]>         (packed)
 *   s_t   = <q_s, k[t]>                                     (plain)
 *   causal: query row l of L sees keys t <= T_b - L + l, others get -FLT_MAX
 *   o     = R_V^-1( sum_t p_t n_v[t] codebook_v[idx_v[t]] ) / max(sum_t p_t, 1e-6)
 * GQA: query head h reads kv head h / (Hq / Hkv).
 * kv_kind TQ_KV_PACKED: k/v are packed uint32 rows, k_norms/v_norms given,
 *   norm_dtype F32/F16, bits 1..4 each, rot_kind selects R_K/R_V as in append.
 * kv_kind TQ_KV_PLAIN: k/v are [B, Hkv, capacity, dim] in kv_dtype (F16/BF16);
 *   norms, codebooks and rotations are ignored (may be NULL).
 * seq_lens: NULL (every sequence holds max_tokens tokens) or a device int32
 *   array of B lengths, each <= max_tokens (ragged batches).
 * q: [B, Hq, L, dim] with element strides; out: contiguous [B, Hq, L, dim].
 * dim: 8..512 (powers of two for the Hadamard rotation);
 * 64 / 128 / 256 run the tuned kernels, other dims the kernels of
 * tq_attention_general.  L >= 1; Hq % Hkv == 0.
 * workspace: >= tq_attention_workspace_size() bytes, 256-byte aligned, no
 *   initial contents needed (a call overwrites what it reads).  Calls that
 *   may run concurrently (other streams) must use different workspaces.
 */
int tq_attention(const void* q, int q_dtype, int B, int Hq, int Hkv, int L, int dim,
                 int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_l, float scale,
                 int kv_kind, int kv_dtype,
                 const void* k, const void* k_norms, const void* v, const void* v_norms,
                 int norm_dtype, int k_bits, int v_bits,
                 const float* k_codebook, const float* v_codebook,
                 int rot_kind, const float* k_rot, const float* v_rot,
                 int64_t capacity, int64_t max_tokens, const int32_t* seq_lens, int causal,
                 void* out, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * tq_attention over a left-padded batch: sequence b's tokens are the cache
 * rows [seq_starts[b], end_b), end_b = seq_lens[b] (or max_tokens when
 * seq_lens is NULL).  Rows before seq_starts[b] are padding and are never
 * read; the causal rule counts positions from end_b as in tq_attention.
 * seq_starts: NULL (no padding) or a device int32 array of B values in
 * [0, end_b].  A sequence with no tokens gets a zero output.  Every other
 * argument is as in tq_attention, which is this call with seq_starts NULL.
 *
 * Replaces the attention of the reference's continuous-batching caches:
 * BatchTurboQuantKVCache (tq.py:6082-6309) stores each batch row
 * left-padded to a common length with `left_padding` per row, as
 * BatchKVCache does (cache.py:1099-1260), whose make_mask masks keys before
 * left_padding (cache.py:1195-1198, base.py:24-42).
 */
int tq_attention_ranged(const void* q, int q_dtype, int B, int Hq, int Hkv, int L, int dim,
                        int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_l, float scale,
                        int kv_kind, int kv_dtype,
                        const void* k, const void* k_norms, const void* v, const void* v_norms,
                        int norm_dtype, int k_bits, int v_bits,
                        const float* k_codebook, const float* v_codebook,
                        int rot_kind, const float* k_rot, const float* v_rot,
                        int64_t capacity, int64_t max_tokens, const int32_t* seq_starts,
                        const int32_t* seq_lens, int causal,
                        void* out, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Decode / verify attention with Prod-coded keys (tq_prod_quantize) and
 * MSE-coded values.  Replaces the fused Prod decode kernel
 * (_fully_fused_decode_kernel, tq.py:2000-2206) and quantized_attention
 * with a Prod key codec (score_prepared, tq.py:4700-4766):
 *   s_t = n_t (R_K q_s) . c[idx_t] + n_t rn_t sqrt(pi/2)/dim (q_s @ P^T) . sgn_t
 * with sgn = +-1 from the sign bits; softmax, value sum, R_V^-1 and the
 * causal / ragged / left-padding rules as tq_attention_ranged.
 * k_bits is the Prod width (1..4; the MSE part k_mse has k_bits - 1 bits and
 * is not read for k_bits == 1).  Dim 64 / 128 with at most 4 query rows per kv
 * head (Hq/Hkv * L) and k_bits >= 2 run the fused row-group kernel; every
 * other shape (power-of-two dims 32..512) runs the kernels of
 * tq_attention_general.  Hadamard rotations on both sides; Prod keys whose
 * MSE part takes the dense rotation (dims that are not powers of two) go to
 * tq_attention_general with k_rot_kind TQ_ROT_DENSE.  Workspace as
 * tq_attention, sized by
 * tq_attention_prod_workspace_size().
 */
int tq_attention_prod(const void* q, int q_dtype, int B, int Hq, int Hkv, int L, int dim,
                      int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_l, float scale,
                      const void* k_mse, const void* k_norms, const void* k_signs,
                      const void* k_residual_norms, int k_bits, const float* k_mse_codebook,
                      const float* k_rot_signs, const float* projection,
                      const void* v, const void* v_norms, int v_bits, const float* v_codebook,
                      const float* v_rot_signs, int norm_dtype, int64_t capacity,
                      int64_t max_tokens, const int32_t* seq_starts, const int32_t* seq_lens,
                      int causal, void* out, void* workspace, int64_t workspace_bytes,
                      void* stream);

/*
 * Bytes of workspace tq_attention_general() needs (rotated and projected
 * queries, split partials).
 */
int64_t tq_attention_general_workspace_size(int B, int Hq, int Hkv, int L, int k_dim, int v_dim,
                                            int64_t max_tokens);

/*
 * Attention with the full generality of quantized_attention (tq.py:5110-5203):
 *   - key and value head dims chosen independently (k_dim, v_dim: any dim in
 *     8..512); q is [B, Hq, L, k_dim], out is contiguous
 *     [B, Hq, L, v_dim] in q_dtype (the output takes value_codec.dim, :5131);
 *   - a rotation kind per side (k_rot_kind, v_rot_kind; Hadamard needs a
 *     power-of-two dim), as each _TurboQuantMSECodec picks its own (:4122-4139);
 *   - kv_kind TQ_KV_PACKED (MSE keys, k_bits 1..4), TQ_KV_PROD (Prod keys of
 *     width k_bits 1..4: k is the MSE part at k_bits - 1 bits, k_signs /
 *     k_residual_norms / projection as tq_attention_prod; the MSE part's
 *     rotation per k_rot_kind: Hadamard at power-of-two dims from 32, dense
 *     at any dim, with ceil(k_dim / 32) sign words per key) or
 *     TQ_KV_PLAIN (k / v [B, Hkv, capacity, dim] in kv_dtype F16/BF16; norms,
 *     codebooks and rotations ignored);
 *   - an optional array mask, applied as _apply_attention_mask
 *     (tq.py:5079-5108): the score of query row (b, head h = g*R + r,
 *     position l) for cache row t (absolute, left padding included) reads
 *       mask[b*s[0] + g*s[1] + r*s[2] + l*s[3] + t*s[4]]   (s = mask_strides,
 *     5 element strides, 0 along broadcast axes; R = Hq / Hkv);
 *     TQ_MASK_BOOL keeps the score where nonzero and sets -FLT_MAX elsewhere,
 *     TQ_MASK_ADD_* adds the value to the f32 score.  This is the reference's
 *     broadcast of a mask over the grouped scores (B, Hkv, R, L, T) (a 4-D
 *     (B, H, L, T) mask gets its repeat axis inserted at position 2).
 *     A row whose every score is -inf (additive -inf masks) gets a zero output.
 *     mask_kind TQ_MASK_NONE ignores mask / mask_strides;
 *   - causal, seq_starts, seq_lens as tq_attention_ranged; a mask and the
 *     causal rule may be combined.
 * Replaces the array-mask paths of quantized_attention and decode_attention
 * (tq.py:5949-5992) and the array-mask SDPA of the fp16 layers
 * (base.py:218-226).  The tuned entry points route here by themselves for
 * shapes outside their kernels.
 */
int tq_attention_general(const void* q, int q_dtype, int B, int Hq, int Hkv, int L, int k_dim,
                         int v_dim, int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_l,
                         float scale, int kv_kind, int kv_dtype,
                         const void* k, const void* k_norms, const void* k_signs,
                         const void* k_residual_norms, int k_bits, const float* k_codebook,
                         int k_rot_kind, const float* k_rot, const float* projection,
                         const void* v, const void* v_norms, int v_bits, const float* v_codebook,
                         int v_rot_kind, const float* v_rot, int norm_dtype, int64_t capacity,
                         int64_t max_tokens, const int32_t* seq_starts, const int32_t* seq_lens,
                         int causal, const void* mask, int mask_kind, const int64_t* mask_strides,
                         void* out, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * tq_attention_ranged without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference, which
 * never exposes a workspace.  The split partials and rotated queries live in
 * a static device array of TQ_NOALLOC_SCRATCH_BYTES per GPU, held until the
 * process ends; the entry point calls no hipMalloc / hipFree.  Problems whose
 * tq_attention_workspace_size() exceeds that size return TQ_ERR_WORKSPACE
 * (use tq_attention with a caller workspace).  Every call on one GPU shares
 * the array: calls that overlap on that GPU (other streams, other host
 * threads) race.  No initial contents are needed: a call writes every
 * scratch byte it reads.  Every other argument and the results are those of
 * tq_attention_ranged.
 */
#define TQ_NOALLOC_SCRATCH_BYTES (16ll << 20)
int tq_attention_noalloc(const void* q, int q_dtype, int B, int Hq, int Hkv, int L, int dim,
                         int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_l, float scale,
                         int kv_kind, int kv_dtype,
                         const void* k, const void* k_norms, const void* v, const void* v_norms,
                         int norm_dtype, int k_bits, int v_bits,
                         const float* k_codebook, const float* v_codebook,
                         int rot_kind, const float* k_rot, const float* v_rot,
                         int64_t capacity, int64_t max_tokens, const int32_t* seq_starts,
                         const int32_t* seq_lens, int causal, void* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* KAPLUMBA_TQ_H */
