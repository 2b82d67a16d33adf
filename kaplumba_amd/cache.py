"""Drop-in TurboQuant KV cache over torch tensors on MI355X.

Mirrors the cache protocol of the reference (mlx_lm/models/cache.py and
mlx_lm/models/turboquant_cache.py in zayutaha/kaplumba): the same class and
method names, argument meanings and error behaviour, with the MLX arrays
replaced by torch device tensors and every kernel replaced by the HIP kernels
of libkaplumba_tq.so.

Storage per TurboQuant layer (all in HBM, contiguous, capacity grows in
256-token steps like the reference, or is preallocated with ``reserve``):
  keys.indices  (B, H_kv, cap, PW_k) uint32   LSB-first packed codebook indices
  keys.norms    (B, H_kv, cap)       f32 (default) or f16 (reference layout)
  values.*      the same with the value codec
"""
from __future__ import annotations

import json
import math
from typing import Any, Dict, List, NamedTuple, Optional, Sequence

import torch

from . import ops
from .codebook import DEFAULT_TURBOQUANT_SEED
from .prod import ProdCodec, TurboQuantProdState, attention_prod

__all__ = [
    "TurboQuantMSEState", "TurboQuantProdState", "TurboQuantKVCache", "KVCache", "make_prompt_cache",
    "save_prompt_cache", "load_prompt_cache", "can_trim_prompt_cache", "trim_prompt_cache",
    "create_attention_mask", "create_causal_mask",
]


class TurboQuantMSEState(NamedTuple):
    """(norms (B,H,T), indices (B,H,T,PW) uint32) -- turboquant_cache.py:3448-3450."""

    norms: torch.Tensor
    indices: torch.Tensor


def _validate_bits(bits: float) -> float:
    """bits >= 1, integer or .5 only (turboquant_cache.py:3477-3486)."""
    bits = float(bits)
    if bits < 1:
        raise ValueError("TurboQuant requires kv_bits >= 1.")
    rounded = round(bits * 2) / 2
    if not math.isclose(bits, rounded, abs_tol=1e-6):
        raise ValueError(f"TurboQuant currently supports integer and .5 bit-widths, got {bits}.")
    return rounded


def _split_bits(bits: float):
    """K takes floor, V takes ceil for x.5 widths (turboquant_cache.py:4948-4967)."""
    if math.isclose(bits, round(bits), abs_tol=1e-6):
        return int(round(bits)), int(round(bits))
    return int(math.floor(bits)), int(math.ceil(bits))


class _QuantizedStateProxy:
    """State wrapper exposing ``.shape = (B, H, T, D)`` (turboquant_cache.py:4898-4916).

    Models read ``keys.shape[-2]`` after ``update_and_fetch``; the proxy answers
    without dequantizing.  (The reference hard-codes B = 1; this uses the
    real batch size.)
    """

    __slots__ = ("_state", "shape")

    def __init__(self, state, n_tokens: int, n_heads: int, head_dim: int = 0, batch: int = 1):
        self._state = state
        self.shape = (batch, n_heads, n_tokens, head_dim)

    def __getattr__(self, name):
        # only names the slots do not hold get here; an unset slot (an object
        # under construction or being copied) is missing, not forwarded
        if name in _QuantizedStateProxy.__slots__:
            raise AttributeError(name)
        return getattr(self._state, name)

    def __iter__(self):
        return iter(self._state)


def _unwrap(state):
    return state._state if isinstance(state, _QuantizedStateProxy) else state


def _codec_meta_fields(key_quantizer: str, key_bits: int, val_bits: int, rotation: str,
                       codebook: str) -> tuple:
    """The codec options a saved TurboQuant cache carries after the reference's
    meta fields: (key_quantizer, key_bits, val_bits, rotation, codebook)."""
    return (key_quantizer, int(key_bits), int(val_bits), rotation, codebook)


def _parse_codec_meta_fields(extra) -> Dict[str, Any]:
    """Options from the fields after (offset, bits, seed, k_dim, v_dim).

    Accepts none (the reference's files), one (the key quantizer alone) or all
    five; anything else is a malformed file.
    """
    extra = list(extra)
    if not extra:
        return {}
    opts: Dict[str, Any] = {"key_quantizer": extra[0]}
    if extra[0] not in ("mse", "prod"):
        raise ValueError(f"unknown TurboQuant key quantizer {extra[0]!r} in meta_state")
    if len(extra) == 1:
        return opts
    if len(extra) != 5:
        raise ValueError(f"TurboQuant meta_state has {5 + len(extra)} fields; expected 5, 6 or 10")
    kb, vb = int(float(extra[1])), int(float(extra[2]))
    if not (1 <= kb <= 4 and 1 <= vb <= 4):
        raise ValueError(f"TurboQuant meta_state bits {kb}/{vb} not in 1..4")
    if extra[3] not in ("auto", "hadamard", "dense"):
        raise ValueError(f"unknown rotation {extra[3]!r} in meta_state")
    if extra[4] not in ("beta", "gaussian"):
        raise ValueError(f"unknown codebook {extra[4]!r} in meta_state")
    opts.update(key_bits=kb, val_bits=vb, rotation=extra[3], codebook=extra[4])
    return opts


def _split_mask(mask, n_queries: int):
    """(causal, array mask or None) of an attention mask argument.

    None, ``"causal"`` (meaningful for more than one query) or an array
    (boolean keep-mask or additive), as ``_apply_attention_mask`` accepts
    (turboquant_cache.py:5079-5108); other strings are rejected there too.
    """
    if mask is None:
        return False, None
    if isinstance(mask, str):
        if mask == "causal":
            return n_queries > 1, None
        raise ValueError(f"Unsupported TurboQuant attention mask: {mask}")
    return False, mask


class _BaseCache:
    """Cache protocol defaults (models/cache.py:193-243)."""

    @property
    def state(self):
        return []

    @state.setter
    def state(self, v):
        if v is not None and v:
            raise ValueError("This cache has no state but a state was set.")

    @property
    def meta_state(self):
        return ""

    @meta_state.setter
    def meta_state(self, v):
        if v is not None and v:
            raise ValueError("This cache has no meta_state but a meta_state was set.")

    def is_trimmable(self):
        return False

    def size(self):
        return 0

    @property
    def nbytes(self):
        raise NotImplementedError("Cache sub-class must implement nbytes")

    def empty(self):
        raise NotImplementedError("Cache sub-class must implement this.")

    @classmethod
    def from_state(cls, state, meta_state):
        obj = cls.__new__(cls)
        obj.state = state
        obj.meta_state = meta_state
        return obj


class TurboQuantKVCache(_BaseCache):
    """TurboQuant KV cache (turboquant_cache.py:4919-6076) backed by HIP kernels.

    Extra keyword options (the reference's behaviour is the default):
      key_bits / val_bits : explicit per-side widths (override ``bits``)
      rotation            : "auto" (Hadamard for power-of-two dims, as the
                            reference), "hadamard" or "dense"
      codebook            : "beta" (reference) or "gaussian" (N(0,1) Lloyd-Max / sqrt(d))
      norm_dtype          : torch.float32 (default) or torch.float16 (reference layout)
      key_quantizer       : "mse" (reference) or "prod": keys with the Prod codec
                            (MSE at bits - 1 plus one-bit QJL signs of the residual,
                            turboquant_cache.py:4572-4766), values stay MSE
    """

    decode_key_chunk_size = 1 << 30
    prefill_key_chunk_size = 2048
    prefill_query_block_size = 16
    cache_step = 256

    # class-level defaults so from_state() objects (built without __init__) work
    key_codec = None
    value_codec = None
    key_bits_override = None
    val_bits_override = None
    rotation = "auto"
    codebook_kind = "beta"
    norm_dtype = torch.float32
    key_quantizer = "mse"
    _dims = (0, 0)

    def __init__(self, bits: float, seed: int = DEFAULT_TURBOQUANT_SEED, *,
                 key_bits: Optional[int] = None, val_bits: Optional[int] = None,
                 rotation: str = "auto", codebook: str = "beta",
                 norm_dtype: torch.dtype = torch.float32, key_quantizer: str = "mse"):
        self.bits = _validate_bits(bits)
        self.seed = seed
        self.offset = 0
        self.keys: Optional[TurboQuantMSEState] = None
        self.values: Optional[TurboQuantMSEState] = None
        self.key_codec = None
        self.value_codec = None
        for b in (key_bits, val_bits):
            if b is not None and (int(b) != b or not 1 <= b <= 4):
                raise ValueError(f"key_bits/val_bits must be integers in 1..4, got {b}")
        self.key_bits_override = key_bits
        self.val_bits_override = val_bits
        if rotation not in ("auto", "hadamard", "dense"):
            raise ValueError(f"rotation must be 'auto', 'hadamard' or 'dense', got {rotation!r}")
        if codebook not in ("beta", "gaussian"):
            raise ValueError(f"codebook must be 'beta' or 'gaussian', got {codebook!r}")
        if norm_dtype not in (torch.float32, torch.float16):
            raise ValueError("norm_dtype must be torch.float32 or torch.float16")
        if key_quantizer not in ("mse", "prod"):
            raise ValueError(f"key_quantizer must be 'mse' or 'prod', got {key_quantizer!r}")
        if key_quantizer == "prod" and (rotation == "dense" or codebook != "beta"):
            raise ValueError("Prod keys use the Hadamard rotation and the Beta codebook")
        self.rotation = rotation
        self.codebook_kind = codebook
        self.norm_dtype = norm_dtype
        self.key_quantizer = key_quantizer

    # ------------------------------------------------------------ codecs ---
    @classmethod
    def from_cache(cls, cache, bits: float, seed: int = DEFAULT_TURBOQUANT_SEED, **kw):
        """Re-quantize an fp16 KVCache (turboquant_cache.py:4938-4946)."""
        tq = cls(bits=bits, seed=seed, **kw)
        keys, values = cache.state
        if keys is not None and keys.shape[2] > 0:
            tq.update_and_fetch(keys, values)
        return tq

    def _side_bits(self):
        kb, vb = _split_bits(self.bits)
        if self.key_bits_override is not None:
            kb = int(self.key_bits_override)
        if self.val_bits_override is not None:
            vb = int(self.val_bits_override)
        return kb, vb

    def _build_codecs(self, k_dim: int, v_dim: int) -> None:
        kb, vb = self._side_bits()
        if self.key_codec is None:
            if self.key_quantizer == "prod":
                self.key_codec = ProdCodec(k_dim, kb, self.seed)
            else:
                self.key_codec = ops.Codec(k_dim, kb, self.seed, self.rotation, self.codebook_kind)
        if self.value_codec is None:
            self.value_codec = ops.Codec(v_dim, vb, self.seed + 1, self.rotation, self.codebook_kind)

    def _ensure_codecs(self, keys: torch.Tensor, values: torch.Tensor) -> None:
        """Codecs from the first append's head dims (turboquant_cache.py:4948-4967)."""
        self._build_codecs(keys.shape[-1], values.shape[-1])

    def _ensure_codecs_from_meta(self) -> None:
        if self.key_codec is None or self.value_codec is None:
            kd, vd = self._dims
            if not kd or not vd:
                raise ValueError("TurboQuant cache has no codecs yet (append tokens first)")
            self._build_codecs(kd, vd)

    # ------------------------------------------------------------ storage ---
    def _alloc(self, codec, B: int, H: int, cap: int, device):
        if isinstance(codec, ProdCodec):
            return codec.alloc(B, H, cap, device, self.norm_dtype)
        return TurboQuantMSEState(
            torch.zeros((B, H, cap), dtype=self.norm_dtype, device=device),
            torch.zeros((B, H, cap, codec.packed_width), dtype=torch.uint32, device=device),
        )

    def _grow(self, st: TurboQuantMSEState, codec: ops.Codec, needed: int) -> TurboQuantMSEState:
        """_reserve_state_capacity (turboquant_cache.py:4108-4119): round up to a
        256-token step and copy the used prefix."""
        cap = st.norms.shape[2]
        if cap >= needed:
            return st
        new_cap = ((needed + self.cache_step - 1) // self.cache_step) * self.cache_step
        B, H = st.norms.shape[:2]
        grown = self._alloc(codec, B, H, new_cap, st.norms.device)
        if self.offset > 0:
            for dst, src in zip(grown, st):
                dst[:, :, : self.offset].copy_(src[:, :, : self.offset])
        return grown

    def reserve(self, n_tokens: int, batch: int, n_kv_heads: int, k_dim: int, v_dim: int,
                device) -> None:
        """Preallocate capacity for ``n_tokens`` (ring-buffer style, no regrowth)."""
        self._build_codecs(k_dim, v_dim)
        if self.keys is None:
            self.keys = self._alloc(self.key_codec, batch, n_kv_heads, n_tokens, device)
            self.values = self._alloc(self.value_codec, batch, n_kv_heads, n_tokens, device)
        else:
            self.keys = self._grow(self.keys, self.key_codec, n_tokens)
            self.values = self._grow(self.values, self.value_codec, n_tokens)

    def update_and_fetch(self, keys: torch.Tensor, values: torch.Tensor):
        """Quantize and append (B, H, L, D) keys/values (turboquant_cache.py:5026-5064)."""
        self._ensure_codecs(keys, values)
        B, H, L = keys.shape[0], keys.shape[1], keys.shape[2]
        new_end = self.offset + L
        if self.keys is None:
            self.keys = self._alloc(self.key_codec, B, H, new_end, keys.device)
            self.values = self._alloc(self.value_codec, B, H, new_end, keys.device)
        else:
            if self.keys.norms.shape[:2] != (B, H):
                raise ValueError(f"batch/heads {(B, H)} differ from the cache's "
                                 f"{tuple(self.keys.norms.shape[:2])}")
            self.keys = self._grow(self.keys, self.key_codec, new_end)
            self.values = self._grow(self.values, self.value_codec, new_end)
        if isinstance(self.key_codec, ProdCodec):
            self.key_codec.quantize_into(keys, self.keys, self.offset)
            ops.append_quantize(values, self.value_codec, self.values.indices, self.values.norms,
                                self.offset)
        else:
            ops.append_quantize_kv(keys, values, self.key_codec, self.value_codec, self.keys.indices,
                                   self.keys.norms, self.values.indices, self.values.norms,
                                   self.offset)
        self.offset = new_end
        ks, vs = self.state
        return (
            _QuantizedStateProxy(ks, self.offset, H, keys.shape[-1], B),
            _QuantizedStateProxy(vs, self.offset, H, values.shape[-1], B),
        )

    # ------------------------------------------------------------ readout ---
    def _states(self, keys_state, values_state):
        if keys_state is None or values_state is None:
            keys_state, values_state = self.state
        return _unwrap(keys_state), _unwrap(values_state)

    def dequantize(self, keys_state=None, values_state=None):
        """f32 reconstructions (B, H, T, D) (turboquant_cache.py:5070-5077)."""
        ks, vs = self._states(keys_state, values_state)
        self._ensure_codecs_from_meta()
        if isinstance(self.key_codec, ProdCodec):
            k = self.key_codec.dequantize(ks)
        else:
            k = ops.dequantize(ks.indices, ks.norms, self.key_codec)
        return k, ops.dequantize(vs.indices, vs.norms, self.value_codec)

    def _attend(self, queries, keys_state, values_state, scale, mask):
        ks, vs = self._states(keys_state, values_state)
        self._ensure_codecs_from_meta()
        causal, arr = _split_mask(mask, queries.shape[-2])
        if isinstance(self.key_codec, ProdCodec):
            return attention_prod(queries, ks, vs.norms, vs.indices, self.key_codec,
                                  self.value_codec, scale, causal, mask=arr)
        return ops.attention_packed(queries, ks.norms, ks.indices, vs.norms, vs.indices,
                                    self.key_codec, self.value_codec, scale, causal, mask=arr)

    def decode_attention(self, queries, keys_state=None, values_state=None, scale: float = 1.0,
                         mask=None):
        """Single-token attention from packed indices (turboquant_cache.py:5776-5947)."""
        if queries.shape[-2] != 1:
            raise ValueError("TurboQuant decode attention expects a single query token.")
        return self._attend(queries, keys_state, values_state, scale, mask)

    def prefill_attention(self, queries, keys_state=None, values_state=None, scale: float = 1.0,
                          mask=None):
        """L > 1 attention straight from packed indices.

        The reference returns None here for MSE codecs and falls back to
        dequantize + SDPA (turboquant_cache.py:5205-5226, base.py:177-189);
        this cache answers with the packed-domain kernel instead.
        """
        return self._attend(queries, keys_state, values_state, scale, mask)

    def quantized_attention(self, queries, keys_state=None, values_state=None,
                            scale: float = 1.0, mask=None):
        """Any-L attention with the semantics of turboquant_cache.py:5110-5203."""
        return self._attend(queries, keys_state, values_state, scale, mask)

    # ------------------------------------------------------- housekeeping ---
    def size(self):
        return self.offset

    @property
    def quant_bits(self):
        return int(self.bits)

    @property
    def state(self):
        """(key_state, value_state) sliced to ``offset`` (turboquant_cache.py:6001-6012)."""
        if self.keys is None:
            return []
        o = self.offset
        return (type(self.keys)(*(t[:, :, :o] for t in self.keys)),
                TurboQuantMSEState(self.values.norms[..., :o], self.values.indices[..., :o, :]))

    @state.setter
    def state(self, value):
        if value is None or (isinstance(value, (list, tuple, dict)) and len(value) == 0):
            self.keys, self.values = None, None
            self.offset = 0
            return
        if isinstance(value, dict):
            value = (value.get("keys"), value.get("values"))
        if isinstance(value, (list, tuple)) and len(value) == 2:
            k, v = value
            if not isinstance(k, (TurboQuantMSEState, TurboQuantProdState)):
                k = TurboQuantProdState(*k) if len(k) == 4 else TurboQuantMSEState(*k)
            if isinstance(k, TurboQuantProdState):
                self.key_quantizer = "prod"
            self.values = TurboQuantMSEState(*v) if not isinstance(v, TurboQuantMSEState) else v
            self.keys = type(k)(*(t.contiguous() for t in k))
            self.values = TurboQuantMSEState(self.values.norms.contiguous(),
                                             self.values.indices.contiguous())
            self.offset = self.keys.norms.shape[2]
            self.norm_dtype = self.keys.norms.dtype
            return
        raise ValueError(f"Expected (key_state, val_state) tuple, got {type(value)}")

    @property
    def meta_state(self):
        """(offset, bits, seed, k_dim, v_dim) as strings (turboquant_cache.py:6046-6050),
        then the codec options: (key_quantizer, key_bits, val_bits, rotation, codebook).

        The reference's five fields come first and its setter reads only the
        first three, so files stay readable both ways; the trailing fields let
        a cache built with non-default codecs reload with the same codecs.
        """
        k_dim = self.key_codec.dim if self.key_codec else self._dims[0]
        v_dim = self.value_codec.dim if self.value_codec else self._dims[1]
        fields = (self.offset, self.bits, self.seed, k_dim, v_dim) + _codec_meta_fields(
            self.key_quantizer, *self._side_bits(), self.rotation, self.codebook_kind)
        return tuple(map(str, fields))

    @meta_state.setter
    def meta_state(self, value):
        self.offset = int(float(value[0]))
        self.bits = float(value[1])
        self.seed = int(float(value[2]))
        if len(value) >= 5:
            self._dims = (int(float(value[3])), int(float(value[4])))
        opts = _parse_codec_meta_fields(value[5:])
        if opts:
            self.key_quantizer = opts.get("key_quantizer", self.key_quantizer)
            self.key_bits_override = opts.get("key_bits", self.key_bits_override)
            self.val_bits_override = opts.get("val_bits", self.val_bits_override)
            self.rotation = opts.get("rotation", self.rotation)
            self.codebook_kind = opts.get("codebook", self.codebook_kind)
            self.key_codec = self.value_codec = None  # rebuilt from the restored options

    def is_trimmable(self):
        return True

    def trim(self, n):
        """Drop the last n tokens; stale rows are overwritten by the next append."""
        n = min(self.offset, n)
        self.offset -= n
        return n

    def make_mask(self, *args, **kwargs):
        return create_attention_mask(*args, offset=self.offset, **kwargs)

    def empty(self):
        return self.keys is None

    @property
    def nbytes(self):
        st = self.state
        if not st:
            return 0
        return sum(t.numel() * t.element_size() for s in st for t in s)


class KVCache(_BaseCache):
    """Unquantized model-dtype cache of the mixed-precision layers (cache.py:411-508).

    Appends go through the HIP plain-append kernel; attention over it uses the
    same split-K kernel as the TurboQuant layers with plain fp16/bf16 loads.
    """

    step = 256

    def __init__(self):
        self.keys = None
        self.values = None
        self.offset = 0

    def update_and_fetch(self, keys, values):
        prev = self.offset
        B, H, L, kd = keys.shape
        vd = values.shape[3]
        if self.keys is None or prev + L > self.keys.shape[2]:
            n_steps = (self.step + L - 1) // self.step
            new_cap = (prev if self.keys is not None else 0) + n_steps * self.step
            new_cap = max(new_cap, prev + L)
            nk = torch.zeros((B, H, new_cap, kd), dtype=keys.dtype, device=keys.device)
            nv = torch.zeros((B, H, new_cap, vd), dtype=values.dtype, device=values.device)
            if self.keys is not None and prev > 0:
                nk[..., :prev, :].copy_(self.keys[..., :prev, :])
                nv[..., :prev, :].copy_(self.values[..., :prev, :])
            self.keys, self.values = nk, nv
        ops.append_plain(keys, self.keys, prev)
        ops.append_plain(values, self.values, prev)
        self.offset += L
        return self.keys[..., : self.offset, :], self.values[..., : self.offset, :]

    def size(self):
        return self.offset

    @property
    def state(self):
        if self.keys is None:
            z = torch.zeros((1, 1, 0, 1), dtype=torch.float16)
            return z, z.clone()
        if self.offset == self.keys.shape[2]:
            return self.keys, self.values
        return self.keys[..., : self.offset, :], self.values[..., : self.offset, :]

    @state.setter
    def state(self, v):
        k, v_ = v
        if k.ndim >= 3 and k.shape[2] > 0:
            self.keys, self.values = k.contiguous(), v_.contiguous()
            self.offset = k.shape[2]
        else:
            self.keys, self.values = None, None
            self.offset = 0

    @property
    def meta_state(self):
        return str(self.offset)

    @meta_state.setter
    def meta_state(self, v):
        self.offset = int(v)

    def is_trimmable(self):
        return True

    def trim(self, n):
        n = min(self.offset, n)
        self.offset -= n
        return n

    def to_turbo_quantized(self, bits: int = 3, **kw) -> TurboQuantKVCache:
        """cache.py:499-508."""
        tq = TurboQuantKVCache(bits=bits, **kw)
        if self.keys is not None and self.offset > 0:
            tq.update_and_fetch(self.keys[..., : self.offset, :], self.values[..., : self.offset, :])
        return tq

    def make_mask(self, *args, **kwargs):
        return create_attention_mask(*args, offset=self.offset, **kwargs)

    def empty(self):
        return self.keys is None

    @property
    def nbytes(self):
        if self.keys is None:
            return 0
        return sum(t.numel() * t.element_size() for t in (self.keys, self.values))


# ---------------------------------------------------------------- masks ----
def create_causal_mask(N: int, offset: int = 0, window_size: Optional[int] = None,
                       right_padding=None, left_padding=None, lengths=None,
                       device=None) -> torch.Tensor:
    """Boolean causal mask (models/base.py:24-42): (N, offset+N), or
    (B, 1, N, offset+N) with per-row ``right_padding`` / ``left_padding``
    (keys ``k < offset+N-right_padding[b]`` and ``k >= left_padding[b]``)
    or ``lengths`` (keys ``k < lengths[b]``)."""
    rinds = torch.arange(offset + N, device=device)
    linds = torch.arange(offset, offset + N, device=device)[:, None]
    rinds = rinds[None]
    mask = linds >= rinds
    if window_size is not None:
        mask = mask & (linds < rinds + window_size)
    if right_padding is not None:
        rp = torch.as_tensor(right_padding, device=device)[:, None, None, None]
        mask = mask & (rinds < (offset + N) - rp)
    if left_padding is not None:
        lp = torch.as_tensor(left_padding, device=device)[:, None, None, None]
        mask = mask & (lp <= rinds)
    if lengths is not None:
        lengths = torch.as_tensor(lengths, device=device)[:, None, None, None]
        mask = mask & (rinds < lengths)
    return mask


def create_attention_mask(N, offset: int = 0, return_array: bool = False,
                          window_size: Optional[int] = None, cache=None):
    """cache.py:182-192.  ``N`` may also be a hidden-state tensor (B, N, ...),
    as models/base.py's helper accepts; with ``cache`` the cache offset is used."""
    if isinstance(N, torch.Tensor):
        N = N.shape[1]
    if cache is not None:
        return cache.make_mask(N, return_array=return_array, window_size=window_size)
    if window_size is not None:
        return create_causal_mask(N, offset, window_size=window_size)
    if N == 1:
        return None
    if return_array:
        return create_causal_mask(N, offset, window_size=window_size)
    return "causal"


# ------------------------------------------------------- construction -----
def make_prompt_cache(model=None, max_kv_size: Optional[int] = None,
                      turbo_kv_bits: Optional[float] = None, turbo_fp16_layers: int = 1, *,
                      num_layers: Optional[int] = None, fp16_layer_policy: str = "first_last",
                      **turbo_kwargs) -> List[Any]:
    """Per-layer cache list (cache.py:15-68).

    With ``turbo_kv_bits``: layer i keeps a model-dtype ``KVCache`` when
    ``i < N or i >= num_layers - N`` (``fp16_layer_policy="first_last"``, the
    reference policy) or only ``i < N`` (``"first"``), else a
    ``TurboQuantKVCache``.  Models with ``make_cache`` get every ``KVCache``
    entry replaced and ``turbo_fp16_layers`` ignored, as in the reference.
    ``num_layers`` stands in for ``len(model.layers)`` when no model is given.
    """
    if model is not None and hasattr(model, "make_cache"):
        caches = model.make_cache()
        if turbo_kv_bits is not None:
            for i, c in enumerate(caches):
                if isinstance(c, KVCache):
                    caches[i] = TurboQuantKVCache(bits=turbo_kv_bits, **turbo_kwargs)
        return caches
    n = num_layers if num_layers is not None else len(model.layers)
    if turbo_kv_bits is not None:
        if fp16_layer_policy not in ("first_last", "first"):
            raise ValueError("fp16_layer_policy must be 'first_last' or 'first'")
        out = []
        for i in range(n):
            keep = i < turbo_fp16_layers or (fp16_layer_policy == "first_last"
                                             and i >= n - turbo_fp16_layers)
            out.append(KVCache() if keep else TurboQuantKVCache(bits=turbo_kv_bits, **turbo_kwargs))
        return out
    if max_kv_size is not None:
        raise NotImplementedError("RotatingKVCache (max_kv_size) is outside this library's scope")
    return [KVCache() for _ in range(n)]


def can_trim_prompt_cache(cache: List[Any]) -> bool:
    return all(c.is_trimmable() for c in cache)


def trim_prompt_cache(cache: List[Any], num_tokens: int):
    if not can_trim_prompt_cache(cache) or len(cache) == 0:
        return 0
    return [c.trim(num_tokens) for c in cache][0]


# ---------------------------------------------------------- save / load ----
def _tree_flatten(tree, prefix=""):
    """mlx.utils.tree_flatten naming: list/tuple index and dict keys joined by '.'."""
    if isinstance(tree, (list, tuple)):
        out = []
        for i, t in enumerate(tree):
            out.extend(_tree_flatten(t, f"{prefix}.{i}" if prefix else str(i)))
        return out
    if isinstance(tree, dict):
        out = []
        for k, t in tree.items():
            out.extend(_tree_flatten(t, f"{prefix}.{k}" if prefix else str(k)))
        return out
    return [(prefix, tree)]


def _tree_unflatten(items):
    """Inverse of _tree_flatten: integer keys become lists, others dicts."""
    root: Dict[str, Any] = {}
    for key, val in items:
        parts = key.split(".")
        node = root
        for p in parts[:-1]:
            node = node.setdefault(p, {})
        node[parts[-1]] = val

    def fix(node):
        if not isinstance(node, dict):
            return node
        if node and all(k.isdigit() for k in node):
            n = max(int(k) for k in node) + 1
            return [fix(node.get(str(i), [])) for i in range(n)]
        return {k: fix(v) for k, v in node.items()}

    return fix(root)


_ALLOWED_CACHE_CLASSES = {"KVCache", "TurboQuantKVCache", "BatchKVCache", "BatchTurboQuantKVCache"}


def save_prompt_cache(file_name: str, cache: List[Any], metadata: Dict[str, str] = {}):
    """Safetensors file with the reference's flattening (cache.py:71-99)."""
    from safetensors.torch import save_file

    def safe(x):
        if x is None or x.numel() == 0:
            return torch.zeros((1,), dtype=torch.float16)
        return x.detach().contiguous().cpu()

    data = {}
    for k, v in _tree_flatten([c.state for c in cache]):
        if v is not None:
            data[k] = safe(v)
    info = [c.meta_state for c in cache]
    classes = [type(c).__name__ for c in cache]
    meta = {k: str(v) for k, v in _tree_flatten([info, metadata, classes])}
    save_file(data, file_name, metadata=meta)


def load_prompt_cache(file_name: str, return_metadata: bool = False, device=None):
    """Rebuild caches from a file written by save_prompt_cache (cache.py:102-153)."""
    from safetensors.torch import load_file
    from safetensors import safe_open

    arrays = load_file(file_name, device="cpu")
    with safe_open(file_name, framework="pt") as f:
        meta = f.metadata() or {}
    if device is None:
        device = "cuda" if torch.cuda.is_available() else "cpu"
    arrays = {k: v.to(device) for k, v in arrays.items()}
    tree = _tree_unflatten(list(arrays.items())) if arrays else []
    info, metadata, classes = _tree_unflatten(list(meta.items()))
    if isinstance(metadata, list) and not metadata:
        metadata = {}
    from .batch_cache import BatchKVCache, BatchTurboQuantKVCache

    def mse_state(x):
        ok = isinstance(x, list) and len(x) == 2 and all(isinstance(t, torch.Tensor) for t in x)
        return TurboQuantMSEState(*x) if ok else None

    def tensor_or_none(x):
        return x if isinstance(x, torch.Tensor) else None

    caches = []
    for i, cls_name in enumerate(classes):
        if cls_name not in _ALLOWED_CACHE_CLASSES:
            raise ValueError(f"Untrusted cache class '{cls_name}' in prompt cache file.")
        st = tree[i] if isinstance(tree, list) and i < len(tree) else []
        ms = info[i]
        if cls_name == "TurboQuantKVCache":
            cls = TurboQuantKVCache
            if isinstance(st, list) and len(st) == 2 and all(isinstance(s, list) for s in st):
                kst = TurboQuantProdState(*st[0]) if len(st[0]) == 4 else TurboQuantMSEState(*st[0])
                st = (kst, TurboQuantMSEState(*st[1]))
            else:
                st = []
        elif cls_name in ("BatchTurboQuantKVCache", "BatchKVCache"):
            # (keys, values, offset, left_padding); absent keys were not saved
            st = list(st) + [[]] * (4 - len(st)) if isinstance(st, list) else [[]] * 4
            if cls_name == "BatchTurboQuantKVCache":
                cls = BatchTurboQuantKVCache
                st = (mse_state(st[0]), mse_state(st[1]), st[2], st[3])
            else:
                cls = BatchKVCache
                st = (tensor_or_none(st[0]), tensor_or_none(st[1]), st[2], st[3])
            st = st[:2] + tuple(t.cpu() if isinstance(t, torch.Tensor) else [] for t in st[2:])
        else:
            cls = KVCache
        caches.append(cls.from_state(st, ms))
    if return_metadata:
        return caches, metadata
    return caches
