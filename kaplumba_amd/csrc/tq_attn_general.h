// General split-K attention: the path for every problem outside the tuned
// kernels' shapes, with the full semantics of quantized_attention
// (turboquant_cache.py:5110-5203):
//   * key and value head dims chosen independently (8..512, multiples of 8;
//     the output has the value dim, :5131),
//   * a rotation kind per side (Hadamard for powers of two, dense otherwise,
//     _TurboQuantMSECodec.__init__, :4122-4139),
//   * MSE-coded, Prod-coded (any width 1..4, score_prepared :4700-4766) or
//     plain fp16/bf16 keys, MSE-coded or plain values,
//   * an optional array mask applied as _apply_attention_mask (:5079-5108):
//     boolean masks keep scores where set (f32 min elsewhere), additive masks
//     are added to the f32 scores, both over absolute cache positions,
//   * the causal rule, ragged lengths and left padding of tq_attention_ranged.
//
// Three launches on the caller's stream:
//   gen_qprep_kernel    q_s = round_qdtype(q * scale) per row, then the key
//                       side's transform into the workspace: R_K q_s (Hadamard
//                       butterflies in LDS or a dense product), q_s @ P^T for
//                       Prod keys, or q_s itself for plain keys.
//   gen_partial_kernel  grid (split, kv head * row group, sequence): up to 8
//                       query rows of one kv head over one contiguous slab of
//                       its tokens, in 64-token tiles: scores (four waves each
//                       own a quarter of the 32-coordinate groups of the key
//                       rows, lane = token), an online softmax per row, and
//                       the weighted value sum (thread = coordinate pair x
//                       token subset); writes (o, max, sum) per row as the
//                       split's partial, o still in the rotated value basis.
//   gen_merge_kernel    log-sum-exp over the splits, / max(sum, 1e-6), R_V^-1
//                       (butterflies in LDS, or a dense product per 64 output
//                       columns), output in the query dtype.
// All arithmetic is f32 on the vector ALUs, in the reference's operation order
// per token (score = n * <q_rot, c[idx]>; Prod adds n * scale * rn * <q_proj, sgn>).
#pragma once

#include "tq_attention.h"

namespace tq {

enum GenKeyKind { kGenMse = 0, kGenProd = 1, kGenPlainF16 = 2, kGenPlainBf16 = 3 };

constexpr int kGenMaxDim = 512;
constexpr int kGenNQ = 8;         // query rows per workgroup
constexpr int kGenTT = 64;        // tokens per tile
constexpr int kGenThreads = 256;  // four wave64s
constexpr int kGenMaxSplits = 1024;

struct GenParams {
  // queries [B, Hq, L, Dk] with element strides
  const void* q;
  int64_t q_sb, q_sh, q_sl;
  int q_dtype;
  float scale_q;  // scale rounded to the query dtype
  int B, Hq, Hkv, L, R;
  int Dk, Dv;    // key / value head dims
  int DkP, DvP;  // Dk rounded up to 32; Dv rounded up to a power of two >= 32
  // keys
  int key_kind;      // GenKeyKind
  const void* k;     // packed MSE rows [B, Hkv, cap, kpw] u32, or plain [B, Hkv, cap, Dk]
  const void* kn;    // key norms [B, Hkv, cap] (packed and Prod)
  const void* ksg;   // Prod QJL sign rows [B, Hkv, cap, Dk / 32] u32
  const void* krn;   // Prod residual norms [B, Hkv, cap]
  int kpw;           // packed MSE key row width in words (0 for 1-bit Prod)
  const float* kcb;  // key (MSE part) codebook
  int k_rot_kind;
  const float* krot;  // Hadamard signs (Dk) or dense R_K (Dk x Dk)
  const float* proj;  // Prod projection P (Dk x Dk)
  // values
  const void* v;     // packed rows [B, Hkv, cap, vpw] u32, or plain [B, Hkv, cap, Dv]
  const void* vn;    // value norms (packed)
  int vpw;
  const float* vcb;
  int v_rot_kind;
  const float* vrot;  // Hadamard signs (Dv) or dense R_V (Dv x Dv)
  int norm_dtype;
  // tokens
  int64_t cap, T;
  const int32_t* seq_lens;
  const int32_t* seq_starts;
  int causal;
  // array mask: element (b, kv head, repeat, query, key) at
  // mask + b*m_sb + g*m_sg + r*m_sr + l*m_sl + t*m_st (t = cache row)
  const void* mask;
  int mask_kind;  // TQ_MASK_*
  int64_t m_sb, m_sg, m_sr, m_sl, m_st;
  // split-K
  int n_splits, chunk, n_rg;
  // workspace
  float* qrot;   // [B*Hq*L, DkP]
  float* qproj;  // [B*Hq*L, DkP] (Prod)
  float* po;     // [B*Hkv*n_rg, n_splits, 8, Dv]
  float* pml;    // [B*Hkv*n_rg, n_splits, 8, 2]
  float rscale_k, rscale_v;  // f32(1/sqrt(Dk)), f32(1/sqrt(Dv))
  float qjl_scale;           // f32(sqrt(pi/2) / Dk)
  int po_natural;            // partials already in the natural value basis (plain values)
  int merge_had;             // the element-wise merge applies R_V^-1 (Hadamard) per merged row
  int merge_bpp;             // > 0: flat-merge blocks per (b, kv head), mapped to that pair's XCD
  uint32_t* qhl;             // tile kernel: per query row, q_rot * sq as hi then lo f16 [rows, 2, Dk / 2] u32
  float* qsq;                // tile kernel: sq per query row
  void* out;                 // [B, Hq, L, Dv] in the query dtype
};

// Query rows per kv head from which packed caches at d = 128 run the tile
// kernel (tq_attn_tile.h): its K/V decode is shared by 128 rows.
constexpr int kTileMinRows = 64;
bool tile_rows_path(int kv_kind, int Dk, int Dv, int rows);

// Workspace bytes of the general path for this problem.
int64_t general_workspace_bytes(int B, int Hq, int Hkv, int L, int Dk, int Dv, int64_t T,
                                bool prod);

// Arguments of one general attention call (validated by general_attention).
struct GenCall {
  const void* q;
  int q_dtype, B, Hq, Hkv, L, Dk, Dv;
  int64_t q_sb, q_sh, q_sl;
  float scale;
  int kv_kind, kv_dtype;
  const void* k;
  const void* k_norms;
  const void* k_signs;
  const void* k_rnorms;
  int k_bits;  // MSE key bits, or the Prod width (MSE part k_bits - 1)
  const float* k_codebook;
  int k_rot_kind;
  const float* k_rot;
  const float* projection;
  const void* v;
  const void* v_norms;
  int v_bits;
  const float* v_codebook;
  int v_rot_kind;
  const float* v_rot;
  int norm_dtype;
  int64_t capacity, max_tokens;
  const int32_t* seq_starts;
  const int32_t* seq_lens;
  int causal;
  const void* mask;
  int mask_kind;
  const int64_t* mask_strides;
  void* out;
  void* workspace;
  int64_t workspace_bytes;
  void* stream;
};

int general_attention(const GenCall& c);

}  // namespace tq
