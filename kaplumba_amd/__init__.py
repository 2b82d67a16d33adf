"""kaplumba_amd -- MI355X-native TurboQuant KV-cache hot path.

A from-scratch HIP/gfx950 implementation of the TurboQuant KV cache of
zayutaha/kaplumba (mlx_lm/models/turboquant_cache.py), behind the same cache
API: append-time quantization, decode/verify attention straight from packed
indices, and the mixed-precision fp16-layer split.
"""
from .cache import (  # noqa: F401
    KVCache,
    TurboQuantKVCache,
    TurboQuantMSEState,
    can_trim_prompt_cache,
    create_attention_mask,
    create_causal_mask,
    load_prompt_cache,
    make_prompt_cache,
    save_prompt_cache,
    trim_prompt_cache,
)
from .batch_cache import BatchKVCache, BatchTurboQuantKVCache  # noqa: F401
from .base import scaled_dot_product_attention  # noqa: F401

__version__ = "0.1.0"
