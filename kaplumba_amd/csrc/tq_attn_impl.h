// Kernel dispatch of the split-K attention (included by tq_attn_d*.hip):
// packed TurboQuant caches go to the small row-group kernel (<= 4 rows,
// d <= 128), the 16-row kernel (d = 128) or the general matrix-core kernel
// of tq_attn_mfma.h; plain fp16 / bf16 caches to the one of tq_attn_plain.h.
// Each writes split partials that attn_merge_kernel combines (a single split
// is finished in the partial kernel itself).
#pragma once

#include "tq_attn_mfma.h"
#include "tq_attn_plain.h"
#include "tq_attn_rows16.h"
#include "tq_attn_small.h"
#include "tq_attn_stage.h"

namespace tq {

template <int D, int KB>
int launch_small_vb(const AttnParams& p, int vb, hipStream_t st) {
  switch (vb) {
    case 1: return launch_stage<D, KB, 1>(p, st);
    case 2: return launch_stage<D, KB, 2>(p, st);
    case 3: return launch_stage<D, KB, 3>(p, st);
    case 4: return launch_stage<D, KB, 4>(p, st);
  }
  return fail(TQ_ERR_INVALID_ARGUMENT, "attention: v_bits %d not in 1..4", vb);
}

template <int KB>
int launch_rows16_vb(const AttnParams& p, int vb, hipStream_t st) {
  switch (vb) {
    case 1: return launch_rows16<KB, 1>(p, st);
    case 2: return launch_rows16<KB, 2>(p, st);
    case 3: return launch_rows16<KB, 3>(p, st);
    case 4: return launch_rows16<KB, 4>(p, st);
  }
  return fail(TQ_ERR_INVALID_ARGUMENT, "attention: v_bits %d not in 1..4", vb);
}

template <int D, int KB>
int launch_partial_vb(const AttnParams& p, int vb, hipStream_t st) {
  if constexpr (D <= 128) {
    if (small_rows_path(TQ_KV_PACKED, D, p.R * p.L)) return launch_small_vb<D, KB>(p, vb, st);
  }
  if constexpr (D == 128) {
    if (rows16_path(TQ_KV_PACKED, D, p.R * p.L)) return launch_rows16_vb<KB>(p, vb, st);
  }
  switch (vb) {
    case 1: return launch_mfma_nq<D, KB, 1>(p, st);
    case 2: return launch_mfma_nq<D, KB, 2>(p, st);
    case 3: return launch_mfma_nq<D, KB, 3>(p, st);
    case 4: return launch_mfma_nq<D, KB, 4>(p, st);
  }
  return fail(TQ_ERR_INVALID_ARGUMENT, "attention: v_bits %d not in 1..4", vb);
}

// Prod-coded keys (MSE part kb = bits - 1 >= 1): the small row-group kernel only.
template <int D, int KB>
int launch_prod_vb(const AttnParams& p, int vb, hipStream_t st) {
  switch (vb) {
    case 1: return launch_small<D, KB, 1, true>(p, st);
    case 2: return launch_small<D, KB, 2, true>(p, st);
    case 3: return launch_small<D, KB, 3, true>(p, st);
    case 4: return launch_small<D, KB, 4, true>(p, st);
  }
  return fail(TQ_ERR_INVALID_ARGUMENT, "attention: v_bits %d not in 1..4", vb);
}

template <int D>
int launch_partial_dim(const AttnParams& p, int kv_kind, int kv_dtype, int kb, int vb,
                       hipStream_t st) {
  if (kv_kind == TQ_KV_PROD) {
    if constexpr (D <= 128) {
      switch (kb) {
        case 1: return launch_prod_vb<D, 1>(p, vb, st);
        case 2: return launch_prod_vb<D, 2>(p, vb, st);
        case 3: return launch_prod_vb<D, 3>(p, vb, st);
      }
      return fail(TQ_ERR_UNSUPPORTED, "attention: Prod keys need an MSE part of 1..3 bits, got %d", kb);
    }
    return fail(TQ_ERR_UNSUPPORTED, "attention: Prod keys at head dim %d (64 / 128 are built)", D);
  }
  if (kv_kind == TQ_KV_PLAIN) {
    if (kv_dtype == TQ_DTYPE_F16) return launch_plain<D, TQ_DTYPE_F16>(p, st);
    if (kv_dtype == TQ_DTYPE_BF16) return launch_plain<D, TQ_DTYPE_BF16>(p, st);
    return fail(TQ_ERR_INVALID_ARGUMENT, "attention: plain kv_dtype %d (F16/BF16)", kv_dtype);
  }
  switch (kb) {
    case 1: return launch_partial_vb<D, 1>(p, vb, st);
    case 2: return launch_partial_vb<D, 2>(p, vb, st);
    case 3: return launch_partial_vb<D, 3>(p, vb, st);
    case 4: return launch_partial_vb<D, 4>(p, vb, st);
  }
  return fail(TQ_ERR_INVALID_ARGUMENT, "attention: k_bits %d not in 1..4", kb);
}

}  // namespace tq
