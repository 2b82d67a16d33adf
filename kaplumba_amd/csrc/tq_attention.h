// Split-K attention over a TurboQuant (packed) or plain fp16/bf16 KV cache.
//
// On the caller's stream:
//   qprep     (dense rotation only) q_rot = R_K round_qdtype(q * scale) per row.
//   partial   grid (split, kv head * row group, batch): a workgroup owns a
//             contiguous slab of one kv head's tokens and up to NQ query rows
//             of its GQA group (every cache byte is read once per row group),
//             runs scores, an online softmax and the weighted value sum on the
//             matrix cores, and writes (o[D], max, sum) per row as the split's
//             partial; a problem with a single split is finished right there.
//   merge     log-sum-exp over the splits, / max(sum, 1e-6), R_V^-1 for the
//             dense rotation, output in the query dtype.
// Semantics: quantized_attention, turboquant_cache.py:5110-5203.
#pragma once

#include "tq_common.h"

namespace tq {

// Longest split in tokens.  The split count aims at one wave of workgroups
// over the device, and only that bounds a split's length: every extra
// round of workgroups repeats the prologue (tables, query rotation) and the
// epilogue (wave combine, partial write) in series.
constexpr int kMaxChunk = 1 << 20;
constexpr int kMaxSplits = 1024;  // splits per sequence
// (sequence, kv head, row group) groups of one call: bounds the partial
// buffers of the workspace
constexpr int kMaxGroups = 16384;

struct AttnParams {
  // queries
  const void* q;
  int64_t q_sb, q_sh, q_sl;
  int q_dtype;
  float scale_q;  // scale rounded to the query dtype
  // cache
  const void* k;
  const void* kn;
  const void* v;
  const void* vn;
  int norm_dtype;
  const float* kcb;
  const float* vcb;
  int rot_kind;
  const float* krot;
  const float* vrot;
  const int32_t* seq_lens;    // end of each sequence's tokens (NULL: T)
  const int32_t* seq_starts;  // first token of each sequence (left padding; NULL: 0)
  // shape
  int B, Hq, Hkv, L, R, D;
  int row_head[4], row_lpos[4];  // row r < 4 of a row group: (r / L, r % L)
  int64_t cap, T;  // capacity per (b, kv head); max tokens
  int causal;
  // split-K
  int n_splits, chunk, n_rg, nq;  // nq: rows per row group
  // workspace
  float* qrot;         // [B, Hq, L, D] (dense rotation only)
  float* po;           // [B, Hq, L, n_splits, D]
  float* pml;          // [B, Hq, L, n_splits, 2]
  float rscale;        // f32(1/sqrt(D))
  int merge_rot;       // Hadamard partials left in the rotated basis: the merge applies R_V^-1
  // Prod-coded keys (kv kind TQ_KV_PROD): k / kn are the MSE part at bits - 1
  const void* ksg;     // QJL sign rows [B, Hkv, cap, D / 32] u32
  const void* krn;     // residual norms [B, Hkv, cap] (norm_dtype)
  const float* qproj;  // q_s @ P^T rows [B, Hq, L, D] (workspace, from qprep_kernel)
  float qjl_scale;     // f32(sqrt(pi / 2) / D)
  // output
  void* out;
};

// Cache rows [start, start + len) of sequence b: the tokens its queries may
// see.  Kernels address them from a base moved to row `start`, so splits,
// causal limits and the merge all work on positions relative to it.
struct SeqWindow {
  int64_t start, len;
};

__device__ __forceinline__ SeqWindow seq_window(const AttnParams& p, int b) {
  int64_t end = p.seq_lens ? static_cast<int64_t>(p.seq_lens[b]) : p.T;
  if (end > p.T) end = p.T;  // lengths beyond max_tokens are clipped
  if (end < 0) end = 0;
  int64_t start = p.seq_starts ? static_cast<int64_t>(p.seq_starts[b]) : 0;
  if (start < 0) start = 0;
  if (start > end) start = end;
  return SeqWindow{start, end - start};
}

struct SplitPlan {
  int n_splits, chunk, n_rg, nq;
};

SplitPlan plan_splits(int B, int Hq, int Hkv, int L, int64_t T, int D, bool packed);

// Packed caches whose row group is at most 4 query rows (GQA decode with
// R <= 4, or verify with R * L <= 4) at head dim 64 / 128 run the small
// row-group kernels: MSE-coded keys the LDS-staged kernel of tq_attn_stage.h,
// Prod-coded keys attn_small_kernel (tq_attn_small.h).  Their launch packs
// the kv head count into kSmallRowsHkvBits bits.
bool small_rows_path(int kv_kind, int D, int rows);
constexpr int kSmallRowsHkvBits = 12;
// Packed caches at head dim 128 with more rows run 16-row groups on the
// register-softmax kernel of tq_attn_rows16.h.
bool rows16_path(int kv_kind, int D, int rows);
int64_t workspace_bytes(const SplitPlan& p, int B, int Hq, int Hkv, int L, int D);

// Kernel launchers instantiated per head dim in tq_attn_d*.hip.
int launch_partial_d64(const AttnParams& p, int kv_kind, int kv_dtype, int kb, int vb,
                       hipStream_t st);
int launch_partial_d128(const AttnParams& p, int kv_kind, int kv_dtype, int kb, int vb,
                        hipStream_t st);
int launch_partial_d256(const AttnParams& p, int kv_kind, int kv_dtype, int kb, int vb,
                        hipStream_t st);

}  // namespace tq
