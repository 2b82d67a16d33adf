"""SDPA dispatch of the model layer (models/base.py:160-226 of the reference).

TurboQuant layers attend straight from packed indices; the unquantized
(mixed-precision) layers use the same split-K kernel with plain fp16/bf16
loads.  Both run on libkaplumba_tq.so; there is no dequantize fallback.
"""
from __future__ import annotations

from typing import Optional

import torch

from . import ops
from .batch_cache import BatchKVCache
from .cache import _split_mask


def scaled_dot_product_attention(queries: torch.Tensor, keys, values, cache, scale: float,
                                 mask, sinks: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Route attention by cache type, as models/base.py:160-226 does.

    Left-padded batch caches (BatchTurboQuantKVCache, BatchKVCache) attend
    over each row's tokens ``[left_padding[b], _idx)``; their ``make_mask``
    returns None / "causal" and the padding is skipped by the kernel.
    """
    if type(cache).__name__ in ("TurboQuantKVCache", "BatchTurboQuantKVCache"):
        if sinks is not None:
            raise ValueError("TurboQuant KV cache does not support attention sinks.")
        if queries.shape[-2] == 1:
            return cache.decode_attention(queries, keys_state=keys, values_state=values,
                                          scale=scale, mask=mask)
        return cache.prefill_attention(queries, keys_state=keys, values_state=values,
                                       scale=scale, mask=mask)
    if sinks is not None:
        raise NotImplementedError("attention sinks are not supported by the HIP kernels")
    causal, arr = _split_mask(mask, queries.shape[-2])
    starts = cache._seq_starts(queries.device) if isinstance(cache, BatchKVCache) else None
    return ops.attention_plain(queries, keys, values, scale, causal, seq_starts=starts, mask=arr)
