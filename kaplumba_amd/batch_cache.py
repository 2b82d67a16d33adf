"""Continuous-batching caches over the HIP kernels.

Mirrors ``BatchTurboQuantKVCache`` (turboquant_cache.py:6082-6309) and
``BatchKVCache`` (models/cache.py:1099-1315) of the reference: the same
methods, attributes and state layout.  Every batch row is left-padded to one
common length ``_idx``: row b's tokens are cache rows
``[left_padding[b], _idx)``, and ``offset[b] = _idx - left_padding[b]`` is
its token count.  All rows append at ``_idx`` together, so an append is one
kernel launch for the whole batch.

Attention skips each row's padding (``tq_attention_ranged``: the kernels
start row b at ``left_padding[b]``) instead of masking it with a boolean
array.  It computes what ``BatchKVCache.make_mask``'s array mask
(``left_padding <= k`` and causal, models/cache.py:1198-1201 with
models/base.py:24-42) asks of SDPA, and
needs no array: ``make_mask`` returns ``None`` / ``"causal"`` unless an
array is asked for.  In the reference, a ``BatchTurboQuantKVCache`` reaches
``quantized_scaled_dot_product_attention`` (base.py:206-217, it has a
``bits`` attribute), which cannot read TurboQuant states; here it takes the
packed-domain kernel like ``TurboQuantKVCache``.

Row selection (``filter``) and concatenation (``extend``) copy into fresh
contiguous buffers: they run when a request joins or leaves the batch, not
per token, and the kernels need one capacity stride for the whole batch.
"""
from __future__ import annotations

from typing import Any, Dict, List, Optional, Sequence

import torch

from . import ops
from .cache import (KVCache, TurboQuantKVCache, TurboQuantMSEState, _BaseCache,
                    _codec_meta_fields, _split_mask, _parse_codec_meta_fields,
                    _QuantizedStateProxy, _unwrap, _validate_bits, create_causal_mask)
from .codebook import DEFAULT_TURBOQUANT_SEED

__all__ = ["BatchTurboQuantKVCache", "BatchKVCache"]


def _round_up(n: int, step: int) -> int:
    return max(step, ((n + step - 1) // step) * step)


def _as_index(batch_indices) -> torch.Tensor:
    return torch.as_tensor(batch_indices, dtype=torch.int64).reshape(-1).cpu()


class _LeftPadded:
    """Per-row left padding and token counts shared by both batch caches."""

    left_padding: torch.Tensor
    offset: torch.Tensor
    _idx: int

    def _init_padding(self, left_padding: Sequence[int]) -> None:
        self.left_padding = torch.tensor([int(x) for x in left_padding], dtype=torch.int64)
        self.offset = -self.left_padding.clone()
        self._idx = 0
        self._starts_key = None
        self._starts_dev = None

    def _seq_starts(self, device) -> torch.Tensor:
        """Device int32 copy of left_padding, refreshed when the values change."""
        key = (str(device), tuple(self.left_padding.tolist()))
        if self._starts_key != key:
            self._starts_dev = self.left_padding.to(device=device, dtype=torch.int32)
            self._starts_key = key
        return self._starts_dev

    def _batch_mask(self, N: int, return_array: bool, window_size: Optional[int]):
        """None / "causal", or the full (B, 1, N, _idx + N) boolean mask."""
        if return_array or window_size is not None:
            return create_causal_mask(N, offset=self._idx, window_size=window_size,
                                      left_padding=self.left_padding)
        return None if N == 1 else "causal"


class BatchTurboQuantKVCache(_LeftPadded, _BaseCache):
    """Batch-aware TurboQuant cache (turboquant_cache.py:6082-6309).

    ``left_padding`` lists each row's padding; ``bits`` and ``seed`` as in
    ``TurboQuantKVCache``, whose extra keyword options (``key_bits``,
    ``val_bits``, ``rotation``, ``codebook``, ``norm_dtype``) are accepted
    too.  Differences from the reference: the value codec takes the value
    head dim (the reference reuses the key dim); ``filter`` on a cache with
    no tokens keeps the padding (the reference drives ``_idx`` negative);
    ``meta_state`` appends the key and value head dims so a loaded cache can
    attend before its next append.
    """

    cache_step = 256

    def __init__(self, left_padding: list, bits: float,
                 seed: int = DEFAULT_TURBOQUANT_SEED, **turbo_kwargs):
        self.bits = _validate_bits(bits)
        self.seed = seed
        TurboQuantKVCache(bits=self.bits, seed=seed, **turbo_kwargs)  # validates the options
        if turbo_kwargs.get("key_quantizer", "mse") != "mse":
            raise ValueError("BatchTurboQuantKVCache holds MSE-coded keys only")
        self._turbo_kwargs: Dict[str, Any] = dict(turbo_kwargs)
        self.keys: Optional[TurboQuantMSEState] = None
        self.values: Optional[TurboQuantMSEState] = None
        self.key_codec = None
        self.value_codec = None
        self._dims = (0, 0)
        self._init_padding(left_padding)

    # ------------------------------------------------------------ codecs ---
    def _build_codecs(self, k_dim: int, v_dim: int) -> None:
        tmp = TurboQuantKVCache(bits=self.bits, seed=self.seed, **self._turbo_kwargs)
        tmp._build_codecs(k_dim, v_dim)
        self.key_codec, self.value_codec = tmp.key_codec, tmp.value_codec
        self._dims = (k_dim, v_dim)

    def _ensure_codecs(self, keys: torch.Tensor, values: Optional[torch.Tensor] = None) -> None:
        """Codecs from the first append's head dims (turboquant_cache.py:6111-6120)."""
        if self.key_codec is None or self.value_codec is None:
            self._build_codecs(keys.shape[-1], (values if values is not None else keys).shape[-1])

    def _codecs_ready(self) -> None:
        if self.key_codec is None or self.value_codec is None:
            kd, vd = self._dims
            if not kd or not vd:
                raise ValueError("TurboQuant cache has no codecs yet (append tokens first)")
            self._build_codecs(kd, vd)

    @property
    def _norm_dtype(self) -> torch.dtype:
        return self._turbo_kwargs.get("norm_dtype", torch.float32)

    # ------------------------------------------------------------ storage ---
    @staticmethod
    def _alloc(codec, B: int, H: int, cap: int, norm_dtype, device) -> TurboQuantMSEState:
        return TurboQuantMSEState(
            torch.zeros((B, H, cap), dtype=norm_dtype, device=device),
            torch.zeros((B, H, cap, codec.packed_width), dtype=torch.uint32, device=device))

    @staticmethod
    def _alloc_like(st: TurboQuantMSEState, B: int, cap: int) -> TurboQuantMSEState:
        H, pw = st.indices.shape[1], st.indices.shape[3]
        return TurboQuantMSEState(
            torch.zeros((B, H, cap), dtype=st.norms.dtype, device=st.norms.device),
            torch.zeros((B, H, cap, pw), dtype=torch.uint32, device=st.indices.device))

    def _grow(self, st: TurboQuantMSEState, needed: int) -> TurboQuantMSEState:
        """_reserve_state_capacity (turboquant_cache.py:4108-4119)."""
        if st.norms.shape[2] >= needed:
            return st
        grown = self._alloc_like(st, st.norms.shape[0], _round_up(needed, self.cache_step))
        if self._idx > 0:
            grown.norms[..., : self._idx].copy_(st.norms[..., : self._idx])
            grown.indices[..., : self._idx, :].copy_(st.indices[..., : self._idx, :])
        return grown

    def _sliced(self, st: TurboQuantMSEState) -> TurboQuantMSEState:
        return TurboQuantMSEState(st.norms[..., : self._idx], st.indices[..., : self._idx, :])

    def update_and_fetch(self, keys: torch.Tensor, values: torch.Tensor):
        """Quantize (B, H, L, D) keys/values and append them at ``_idx`` for every
        row (turboquant_cache.py:6126-6159)."""
        self._ensure_codecs(keys, values)
        B, H, L = keys.shape[0], keys.shape[1], keys.shape[2]
        if B != self.left_padding.numel():
            raise ValueError(f"batch of {B} rows, but the cache has {self.left_padding.numel()}")
        prev, new_end = self._idx, self._idx + L
        if self.keys is None:
            nd = self._norm_dtype
            self.keys = self._alloc(self.key_codec, B, H, new_end, nd, keys.device)
            self.values = self._alloc(self.value_codec, B, H, new_end, nd, keys.device)
        else:
            if tuple(self.keys.norms.shape[:2]) != (B, H):
                raise ValueError(f"batch/heads {(B, H)} differ from the cache's "
                                 f"{tuple(self.keys.norms.shape[:2])}")
            self.keys = self._grow(self.keys, new_end)
            self.values = self._grow(self.values, new_end)
        ops.append_quantize_kv(keys, values, self.key_codec, self.value_codec, self.keys.indices,
                               self.keys.norms, self.values.indices, self.values.norms, prev)
        self.offset = self.offset + L
        self._idx = new_end
        return (_QuantizedStateProxy(self._sliced(self.keys), self._idx, H, keys.shape[-1], B),
                _QuantizedStateProxy(self._sliced(self.values), self._idx, H, values.shape[-1], B))

    # --------------------------------------------------- batch operations ---
    def _rebuild(self, parts, B: int, n_tokens: int):
        """Fresh (keys, values) of B rows with room for ``n_tokens``, filled from
        parts (first row, key state, value state, first source token, last
        source token, destination token)."""
        ks0, vs0 = parts[0][1], parts[0][2]
        cap = _round_up(n_tokens, self.cache_step)
        nk, nv = self._alloc_like(ks0, B, cap), self._alloc_like(vs0, B, cap)
        for row0, ks, vs, lo, hi, dst0 in parts:
            nb, n = ks.norms.shape[0], hi - lo
            for dst, src in ((nk, ks), (nv, vs)):
                dst.norms[row0:row0 + nb, :, dst0:dst0 + n].copy_(src.norms[:, :, lo:hi])
                dst.indices[row0:row0 + nb, :, dst0:dst0 + n, :].copy_(src.indices[:, :, lo:hi, :])
        return nk, nv

    def filter(self, batch_indices) -> None:
        """Keep the given batch rows, then drop the padding every row shares
        (turboquant_cache.py:6165-6188)."""
        idx = _as_index(batch_indices)
        self.offset = self.offset[idx]
        self.left_padding = self.left_padding[idx]
        if self.keys is None:
            return
        min_lp = int(self.left_padding.min()) if idx.numel() else 0
        min_lp = max(0, min(min_lp, self._idx))
        dev = idx.to(self.keys.norms.device)
        sel = [TurboQuantMSEState(st.norms.index_select(0, dev), st.indices.index_select(0, dev))
               for st in (self.keys, self.values)]
        self.keys, self.values = self._rebuild([(0, sel[0], sel[1], min_lp, self._idx, 0)],
                                               idx.numel(), self._idx - min_lp)
        self._idx -= min_lp
        self.left_padding = self.left_padding - min_lp

    def extend(self, other: "BatchTurboQuantKVCache") -> None:
        """Append other's rows after this cache's, right-aligned at the longer
        ``_idx`` by extra left padding (turboquant_cache.py:6190-6245)."""
        if self.keys is None and other.keys is None:
            self.left_padding = torch.cat([self.left_padding, other.left_padding])
            self.offset = torch.cat([self.offset, other.offset])
            return
        for c in (self, other):
            if c.keys is not None and c.key_codec is None:
                c._codecs_ready()
        if self.keys is not None and other.keys is not None:
            same = (self.key_codec.bits == other.key_codec.bits
                    and self.value_codec.bits == other.value_codec.bits
                    and self.key_codec.dim == other.key_codec.dim
                    and self.value_codec.dim == other.value_codec.dim
                    and self.seed == other.seed
                    and self.key_codec.rotation == other.key_codec.rotation
                    and self.value_codec.rotation == other.value_codec.rotation
                    and self.key_codec.codebook_kind == other.key_codec.codebook_kind
                    and self.value_codec.codebook_kind == other.value_codec.codebook_kind
                    and tuple(self.keys.norms.shape[1:2]) == tuple(other.keys.norms.shape[1:2])
                    and self.keys.norms.dtype == other.keys.norms.dtype)
            if not same:
                raise ValueError("extend: the two caches use different codecs or shapes")
        max_idx = max(self._idx, other._idx)
        nb_self, nb_other = self.left_padding.numel(), other.left_padding.numel()
        parts, lps = [], []
        for row0, c in ((0, self), (nb_self, other)):
            if c.keys is None:
                lps.append(c.left_padding + max_idx)   # every row of c is padding
            else:
                left = max_idx - c._idx
                lps.append(c.left_padding + left)
                parts.append((row0, c.keys, c.values, 0, c._idx, left))
        if self.key_codec is None:
            self.key_codec, self.value_codec, self._dims = other.key_codec, other.value_codec, other._dims
        self.keys, self.values = self._rebuild(parts, nb_self + nb_other, max_idx)
        self.left_padding = torch.cat(lps)
        self.offset = torch.cat([self.offset, other.offset])
        self._idx = max_idx

    # ------------------------------------------------------------ readout ---
    def _states(self, keys_state, values_state):
        if keys_state is None or values_state is None:
            if self.keys is None:
                raise ValueError("the cache holds no tokens")
            keys_state, values_state = self._sliced(self.keys), self._sliced(self.values)
        return _unwrap(keys_state), _unwrap(values_state)

    def dequantize(self, keys_state=None, values_state=None):
        """f32 reconstructions (B, H, _idx, D), padding rows included
        (turboquant_cache.py:6251-6262)."""
        ks, vs = self._states(keys_state, values_state)
        self._codecs_ready()
        return (ops.dequantize(ks.indices, ks.norms, self.key_codec),
                ops.dequantize(vs.indices, vs.norms, self.value_codec))

    def _attend(self, queries, keys_state, values_state, scale, mask):
        ks, vs = self._states(keys_state, values_state)
        self._codecs_ready()
        causal, arr = _split_mask(mask, queries.shape[-2])
        return ops.attention_packed(queries, ks.norms, ks.indices, vs.norms, vs.indices,
                                    self.key_codec, self.value_codec, scale, causal,
                                    seq_starts=self._seq_starts(queries.device), mask=arr)

    def decode_attention(self, queries, keys_state=None, values_state=None, scale: float = 1.0,
                         mask=None):
        """One query token per row over each row's tokens."""
        if queries.shape[-2] != 1:
            raise ValueError("TurboQuant decode attention expects a single query token.")
        return self._attend(queries, keys_state, values_state, scale, mask)

    def prefill_attention(self, queries, keys_state=None, values_state=None, scale: float = 1.0,
                          mask=None):
        """L > 1 queries per row (the last L positions), causal under ``"causal"``."""
        return self._attend(queries, keys_state, values_state, scale, mask)

    def quantized_attention(self, queries, keys_state=None, values_state=None,
                            scale: float = 1.0, mask=None):
        return self._attend(queries, keys_state, values_state, scale, mask)

    # ------------------------------------------------------- housekeeping ---
    @property
    def state(self):
        """(key_state, value_state, offset, left_padding) (turboquant_cache.py:6268-6280)."""
        if self.keys is None:
            return None, None, self.offset, self.left_padding
        return self._sliced(self.keys), self._sliced(self.values), self.offset, self.left_padding

    @state.setter
    def state(self, val):
        k, v, offset, left_padding = val
        self.offset = torch.as_tensor(offset, dtype=torch.int64).reshape(-1).cpu()
        self.left_padding = torch.as_tensor(left_padding, dtype=torch.int64).reshape(-1).cpu()
        if k is None or v is None:
            self.keys = self.values = None
            return
        k = k if isinstance(k, TurboQuantMSEState) else TurboQuantMSEState(*k)
        v = v if isinstance(v, TurboQuantMSEState) else TurboQuantMSEState(*v)
        self.keys = TurboQuantMSEState(k.norms.contiguous(), k.indices.contiguous())
        self.values = TurboQuantMSEState(v.norms.contiguous(), v.indices.contiguous())
        self._idx = self.keys.norms.shape[2]
        if "norm_dtype" not in self._turbo_kwargs and self.keys.norms.dtype != torch.float32:
            self._turbo_kwargs["norm_dtype"] = self.keys.norms.dtype

    @property
    def meta_state(self):
        """(_idx, bits, seed, k_dim, v_dim) as strings, then the codec options
        (key_quantizer, key_bits, val_bits, rotation, codebook).  The reference
        stores the first three (turboquant_cache.py:6282-6290) and reads only
        those, so a loader accepts either form."""
        kd = self.key_codec.dim if self.key_codec else self._dims[0]
        vd = self.value_codec.dim if self.value_codec else self._dims[1]
        tmp = TurboQuantKVCache(bits=self.bits, seed=self.seed, **self._codec_kwargs())
        return tuple(map(str, (self._idx, self.bits, self.seed, kd, vd) + _codec_meta_fields(
            tmp.key_quantizer, *tmp._side_bits(), tmp.rotation, tmp.codebook_kind)))

    @meta_state.setter
    def meta_state(self, v):
        self._idx = int(float(v[0]))
        self.bits = float(v[1])
        self.seed = int(float(v[2]))
        if len(v) >= 5:
            self._dims = (int(float(v[3])), int(float(v[4])))
        opts = _parse_codec_meta_fields(v[5:])
        if opts.get("key_quantizer", "mse") != "mse":
            raise ValueError("BatchTurboQuantKVCache holds MSE-coded keys only")
        opts.pop("key_quantizer", None)
        if opts:
            self._turbo_kwargs.update(opts)
            self.key_codec = self.value_codec = None  # rebuilt from the restored options

    def _codec_kwargs(self) -> Dict[str, Any]:
        """The codec options of _turbo_kwargs (norm_dtype lives in the state)."""
        return {k: v for k, v in self._turbo_kwargs.items() if k != "norm_dtype"}

    @classmethod
    def from_state(cls, state, meta_state):
        obj = cls.__new__(cls)
        obj._turbo_kwargs = {}
        obj.key_codec = obj.value_codec = None
        obj._dims = (0, 0)
        obj._init_padding([])
        obj.state = state
        obj.meta_state = meta_state
        if obj.keys is not None:
            obj._idx = obj.keys.norms.shape[2]
        return obj

    def is_trimmable(self):
        return False

    def trim(self, n):
        return 0

    def empty(self):
        return self.keys is None

    def make_mask(self, N: int, return_array: bool = False, window_size: Optional[int] = None,
                  **kwargs):
        return self._batch_mask(N, return_array, window_size)

    @property
    def group_size(self):
        return 64

    @property
    def nbytes(self):
        if self.keys is None:
            return 0
        return sum(t.numel() * t.element_size()
                   for s in (self._sliced(self.keys), self._sliced(self.values)) for t in s)


class BatchKVCache(_LeftPadded, _BaseCache):
    """Left-padded model-dtype cache of the mixed-precision layers in a
    continuous batch (models/cache.py:1099-1315); appends through the HIP
    plain-append kernel, attention through the plain split-K kernel."""

    step = 256

    def __init__(self, left_padding: List[int]):
        self.keys = None
        self.values = None
        self._init_padding(left_padding)
        self._right_padding = None

    def update_and_fetch(self, keys, values):
        prev = self._idx
        B, H, L, kd = keys.shape
        if B != self.left_padding.numel():
            raise ValueError(f"batch of {B} rows, but the cache has {self.left_padding.numel()}")
        if self.keys is None or prev + L > self.keys.shape[2]:
            cap = _round_up(prev + L, self.step)
            nk = torch.zeros((B, H, cap, kd), dtype=keys.dtype, device=keys.device)
            nv = torch.zeros((B, H, cap, values.shape[3]), dtype=values.dtype, device=values.device)
            if self.keys is not None and prev > 0:
                nk[..., :prev, :].copy_(self.keys[..., :prev, :])
                nv[..., :prev, :].copy_(self.values[..., :prev, :])
            self.keys, self.values = nk, nv
        ops.append_plain(keys, self.keys, prev)
        ops.append_plain(values, self.values, prev)
        self.offset = self.offset + L
        self._idx += L
        return self.keys[..., : self._idx, :], self.values[..., : self._idx, :]

    def prepare(self, *, left_padding=None, lengths=None, right_padding=None):
        """Extra left padding on an empty cache, or right padding to move to
        the left at ``finalize`` (models/cache.py:1154-1166)."""
        if left_padding is not None:
            if self.keys is not None:
                raise ValueError("Left padding can only be added to an empty BatchKVCache")
            lp = torch.as_tensor(left_padding, dtype=torch.int64).reshape(-1)
            self.left_padding = self.left_padding + lp
            self.offset = self.offset - lp
        if right_padding is not None and max(int(x) for x in right_padding) > 0:
            self._right_padding = torch.as_tensor(right_padding, dtype=torch.int64).reshape(-1)

    def finalize(self):
        """Rotate each row right by its right padding, so the padding becomes
        left padding (models/cache.py:1168-1176, ``dynamic_roll``)."""
        if self._right_padding is None:
            return
        pad = self._right_padding
        if self.keys is not None and self._idx > 0:
            n = self._idx
            dev = self.keys.device
            pos = torch.arange(n, device=dev)[None, :]
            src = (pos - pad.to(dev)[:, None]) % n                      # (B, n)
            for name in ("keys", "values"):
                t = getattr(self, name)
                g = src[:, None, :, None].expand(t.shape[0], t.shape[1], n, t.shape[3])
                t[..., :n, :] = torch.gather(t[..., :n, :], 2, g)
        self.offset = self.offset - pad
        self.left_padding = self.left_padding + pad
        self._right_padding = None

    @property
    def state(self):
        k, v = self.keys, self.values
        if k is not None and self._idx < k.shape[2]:
            k, v = k[..., : self._idx, :], v[..., : self._idx, :]
        return k, v, self.offset, self.left_padding

    @state.setter
    def state(self, v):
        k, v_, offset, left_padding = v
        self.offset = torch.as_tensor(offset, dtype=torch.int64).reshape(-1).cpu()
        self.left_padding = torch.as_tensor(left_padding, dtype=torch.int64).reshape(-1).cpu()
        if k is None:
            self.keys = self.values = None
            self._idx = 0
        else:
            self.keys, self.values = k.contiguous(), v_.contiguous()
            self._idx = self.keys.shape[2]

    @classmethod
    def from_state(cls, state, meta_state):
        obj = cls.__new__(cls)
        obj._right_padding = None
        obj._init_padding([])
        obj.state = state
        obj.meta_state = meta_state
        return obj

    def is_trimmable(self):
        return True

    def trim(self, n):
        n = min(self._idx, n)
        self._idx -= n
        self.offset = self.offset - n
        return n

    def make_mask(self, N: int, return_array: bool = False, window_size: Optional[int] = None,
                  **kwargs):
        return self._batch_mask(N, return_array, window_size)

    def filter(self, batch_indices):
        """Keep the given rows, then drop the padding every row shares
        (models/cache.py:1203-1220)."""
        idx = _as_index(batch_indices)
        self.offset = self.offset[idx]
        self.left_padding = self.left_padding[idx]
        if self.keys is None:
            return
        min_lp = int(self.left_padding.min()) if idx.numel() else 0
        min_lp = max(0, min(min_lp, self._idx))
        dev = idx.to(self.keys.device)
        n = self._idx - min_lp
        cap = _round_up(n, self.step)
        out = []
        for t in (self.keys, self.values):
            sel = t.index_select(0, dev)
            nt = torch.zeros((sel.shape[0], sel.shape[1], cap, sel.shape[3]), dtype=t.dtype,
                             device=t.device)
            nt[..., :n, :].copy_(sel[..., min_lp:self._idx, :])
            out.append(nt)
        self.keys, self.values = out
        self._idx = n
        self.left_padding = self.left_padding - min_lp

    def extend(self, other: "BatchKVCache"):
        """Append other's rows, right-aligned at the longer ``_idx``
        (models/cache.py:1222-1262)."""
        if self.keys is None and other.keys is None:
            self.left_padding = torch.cat([self.left_padding, other.left_padding])
            self.offset = torch.cat([self.offset, other.offset])
            return
        ref = self if self.keys is not None else other
        max_idx = max(self._idx, other._idx)
        nbs = (self.left_padding.numel(), other.left_padding.numel())
        B, H, Dk, Dv = sum(nbs), ref.keys.shape[1], ref.keys.shape[3], ref.values.shape[3]
        cap = _round_up(max_idx, self.step)
        nk = torch.zeros((B, H, cap, Dk), dtype=ref.keys.dtype, device=ref.keys.device)
        nv = torch.zeros((B, H, cap, Dv), dtype=ref.values.dtype, device=ref.values.device)
        lps, row0 = [], 0
        for c, nb in zip((self, other), nbs):
            left = max_idx - c._idx
            if c.keys is not None:
                if c.keys.shape[1] != H or c.keys.shape[3] != Dk or c.keys.dtype != nk.dtype:
                    raise ValueError("extend: the two caches differ in heads, dims or dtype")
                nk[row0:row0 + nb, :, left:max_idx].copy_(c.keys[..., : c._idx, :])
                nv[row0:row0 + nb, :, left:max_idx].copy_(c.values[..., : c._idx, :])
            lps.append(c.left_padding + left)
            row0 += nb
        self.keys, self.values = nk, nv
        self.left_padding = torch.cat(lps)
        self.offset = torch.cat([self.offset, other.offset])
        self._idx = max_idx

    def extract(self, idx: int) -> KVCache:
        """Row idx as a single-sequence KVCache without its padding
        (models/cache.py:1264-1270)."""
        pad = int(self.left_padding[idx])
        cache = KVCache()
        cache.keys = self.keys[idx:idx + 1, :, pad:self._idx].contiguous()
        cache.values = self.values[idx:idx + 1, :, pad:self._idx].contiguous()
        cache.offset = cache.keys.shape[2]
        return cache

    @classmethod
    def merge(cls, caches: List[KVCache]) -> "BatchKVCache":
        """Left-pad single-sequence caches to one batch (models/cache.py:1272-1305)."""
        lengths = [c.size() for c in caches]
        max_length = max(lengths) if lengths else 0
        if max_length == 0:
            return cls([0] * len(caches))
        padding = [max_length - n for n in lengths]
        full = [c for c in caches if c.keys is not None]
        H = max(c.keys.shape[1] for c in full)
        Dk = max(c.keys.shape[3] for c in full)
        Dv = max(c.values.shape[3] for c in full)
        dt, dev = full[0].keys.dtype, full[0].keys.device
        cap = _round_up(max_length, cls.step)
        keys = torch.zeros((len(caches), H, cap, Dk), dtype=dt, device=dev)
        values = torch.zeros((len(caches), H, cap, Dv), dtype=dt, device=dev)
        for i, (p, c) in enumerate(zip(padding, caches)):
            if c.keys is None:
                continue
            keys[i:i + 1, :, p:p + c.offset].copy_(c.keys[..., : c.offset, :])
            values[i:i + 1, :, p:p + c.offset].copy_(c.values[..., : c.offset, :])
        cache = cls(padding)
        cache.keys, cache.values = keys, values
        cache.offset = cache.offset + max_length
        cache._idx = max_length
        return cache

    def size(self):
        return self._idx

    def empty(self):
        return self.keys is None

    @property
    def nbytes(self):
        if self.keys is None:
            return 0
        return sum(t.numel() * t.element_size() for t in (self.keys, self.values))
