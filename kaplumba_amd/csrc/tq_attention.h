// Split-K attention over a TurboQuant (packed) or plain fp16/bf16 KV cache.
//
// One fused kernel per call (plus a small query-rotation kernel for the dense
// rotation), on the caller's stream:
//   grid (split, kv head * row group, batch).  A workgroup owns a contiguous
//   slab of one kv head's tokens and up to NQ query rows of that head's GQA
//   group, so every packed byte of the slab is read once per row group.
//   prologue : q_s = round_qdtype(q * round_qdtype(scale)); q_rot = R_K q_s
//              (Hadamard in LDS; dense reads the pre-rotated rows; plain
//              caches use q_s).
//   pass 1-3 : scores -> LDS, softmax weights, weighted codebook sum in
//              rotated space; (o[D], max, sum) per row written as a partial.
//   merge    : the last workgroup of a (batch, kv head, row group) to finish
//              (a counter in the workspace, reset to zero by that workgroup)
//              merges the partials by log-sum-exp, divides by max(sum, 1e-6),
//              applies R_V^-1 and writes the output in the query dtype.
// Semantics: quantized_attention, turboquant_cache.py:5110-5203.
#pragma once

#include "tq_common.h"

namespace tq {

constexpr int kAttnThreads = 256;
constexpr int kAttnWaves = kAttnThreads / kWave;
constexpr int kMaxChunk = 2048;   // tokens per split (LDS score buffer bound)
constexpr int kMaxSplits = 1024;  // splits per sequence (merge scratch bound)
// The workspace starts with a fixed counter region, so a workspace zeroed once
// stays valid across calls of any shape (each call resets what it used).
constexpr int kMaxGroups = 16384;
constexpr int64_t kCounterBytes = kMaxGroups * 4;

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
  const int32_t* seq_lens;
  // shape
  int B, Hq, Hkv, L, R, D;
  int64_t cap, T;  // capacity per (b, kv head); max tokens
  int causal;
  // split-K
  int n_splits, chunk, n_rg, nq;  // nq: rows per row group
  // workspace
  uint32_t* counters;  // [B, Hkv, n_rg], zero between calls
  float* qrot;         // [B, Hq, L, D] (dense rotation only)
  float* po;           // [B, Hq, L, n_splits, D]
  float* pml;          // [B, Hq, L, n_splits, 2]
  float rscale;        // f32(1/sqrt(D))
  // output
  void* out;
};

struct SplitPlan {
  int n_splits, chunk, n_rg, nq;
};

SplitPlan plan_splits(int B, int Hq, int Hkv, int L, int64_t T, int D, bool packed);
int64_t workspace_bytes(const SplitPlan& p, int B, int Hq, int Hkv, int L, int D);
size_t attn_lds_bytes(const SplitPlan& p, int D);

// Kernel launchers instantiated per head dim in tq_attn_d*.hip.
int launch_partial_d64(const AttnParams& p, int kv_kind, int kv_dtype, int kb, int vb,
                       hipStream_t st);
int launch_partial_d128(const AttnParams& p, int kv_kind, int kv_dtype, int kb, int vb,
                        hipStream_t st);
int launch_partial_d256(const AttnParams& p, int kv_kind, int kv_dtype, int kb, int vb,
                        hipStream_t st);

}  // namespace tq
