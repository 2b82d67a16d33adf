"""The hot-path kernels as PyTorch custom operators (``torch.ops.kaplumba.*``).

The functions of ``ops`` call the C ABI through ctypes, which the torch
dispatcher cannot see: ``torch.compile`` would break its graph at every call.
The operators registered here wrap the same functions with a schema and a
shape-only (fake) implementation, so that traced and compiled programs keep
the append and attention calls inside one graph; ``ops`` routes its calls
here whenever torch is compiling.  Eager calls keep the direct ctypes path,
which skips the dispatcher's per-call cost.

A codec crosses the operator boundary as its defining fields (head dim, bits,
seed, rotation kind, codebook kind), the arguments of
``_TurboQuantMSECodec.__init__`` (turboquant_cache.py:4122-4139); equal
fields give the same codec, so the registered functions keep one ``Codec``
per field tuple and with it one copy of its device tables.

Operators:
  append_quantize(x, packed!, norms!, offset, dim, bits, seed, rotation, codebook)
  append_quantize_kv(k, v, k_packed!, k_norms!, v_packed!, v_norms!, offset, <key codec>, <value codec>)
  append_plain(x, dst!, offset)
  dequantize(indices, norms, dim, bits, seed, rotation, codebook) -> f32 (B, H, T, dim)
  attention_packed(q, k_norms, k_idx, v_norms, v_idx, <key codec>, <value codec>, scale, causal,
                   seq_lens?, seq_starts?, mask?) -> (B, Hq, L, Dv) in q's dtype
  attention_plain(q, keys, values, scale, causal, seq_lens?, seq_starts?, mask?) -> (B, Hq, L, Dv)
  prod_quantize(x, norms!, mse_indices!, residual_norms!, qjl_signs!, offset, dim, bits, seed)
  prod_dequantize(norms, mse_indices, residual_norms, qjl_signs, dim, bits, seed) -> f32
  attention_prod(q, <Prod key state>, v_norms, v_idx, k_dim, k_bits, k_seed, <value codec>,
                 scale, causal, seq_lens?, seq_starts?, mask?) -> (B, Hq, L, Dv)
(``!``: written in place.)
"""
from __future__ import annotations

import functools
from typing import Optional

import torch

from . import ops
from . import prod


@functools.lru_cache(maxsize=None)
def codec(dim: int, bits: int, seed: int, rotation: str, codebook: str) -> "ops.Codec":
    """The one Codec object for these fields (its device tables are cached on it)."""
    return ops.Codec(dim, bits, seed, rotation, codebook)


@functools.lru_cache(maxsize=None)
def prod_codec(dim: int, bits: int, seed: int) -> "prod.ProdCodec":
    """The one ProdCodec object for these fields (``_TurboQuantProdCodec(dim, bits, seed)``)."""
    return prod.ProdCodec(dim, bits, seed)


@torch.library.custom_op("kaplumba::append_quantize", mutates_args=("packed", "norms"))
def append_quantize(x: torch.Tensor, packed: torch.Tensor, norms: torch.Tensor, offset: int,
                    dim: int, bits: int, seed: int, rotation: str, codebook: str) -> None:
    ops.append_quantize(x, codec(dim, bits, seed, rotation, codebook), packed, norms, offset,
                        _direct=True)


@append_quantize.register_fake
def _(x, packed, norms, offset, dim, bits, seed, rotation, codebook):
    return None


@torch.library.custom_op("kaplumba::append_quantize_kv",
                         mutates_args=("k_packed", "k_norms", "v_packed", "v_norms"))
def append_quantize_kv(k: torch.Tensor, v: torch.Tensor, k_packed: torch.Tensor,
                       k_norms: torch.Tensor, v_packed: torch.Tensor, v_norms: torch.Tensor,
                       offset: int, k_dim: int, k_bits: int, k_seed: int, k_rotation: str,
                       k_codebook: str, v_dim: int, v_bits: int, v_seed: int, v_rotation: str,
                       v_codebook: str) -> None:
    ops.append_quantize_kv(k, v, codec(k_dim, k_bits, k_seed, k_rotation, k_codebook),
                           codec(v_dim, v_bits, v_seed, v_rotation, v_codebook),
                           k_packed, k_norms, v_packed, v_norms, offset, _direct=True)


@append_quantize_kv.register_fake
def _(k, v, k_packed, k_norms, v_packed, v_norms, offset, *codec_args):
    return None


@torch.library.custom_op("kaplumba::append_plain", mutates_args=("dst",))
def append_plain(x: torch.Tensor, dst: torch.Tensor, offset: int) -> None:
    ops.append_plain(x, dst, offset, _direct=True)


@append_plain.register_fake
def _(x, dst, offset):
    return None


@torch.library.custom_op("kaplumba::dequantize", mutates_args=())
def dequantize(indices: torch.Tensor, norms: torch.Tensor, dim: int, bits: int, seed: int,
               rotation: str, codebook: str) -> torch.Tensor:
    return ops.dequantize(indices, norms, codec(dim, bits, seed, rotation, codebook), _direct=True)


@dequantize.register_fake
def _(indices, norms, dim, bits, seed, rotation, codebook):
    B, H, T = norms.shape
    return norms.new_empty((B, H, T, dim), dtype=torch.float32)


@torch.library.custom_op("kaplumba::attention_packed", mutates_args=())
def attention_packed(queries: torch.Tensor, k_norms: torch.Tensor, k_idx: torch.Tensor,
                     v_norms: torch.Tensor, v_idx: torch.Tensor, k_dim: int, k_bits: int,
                     k_seed: int, k_rotation: str, k_codebook: str, v_dim: int, v_bits: int,
                     v_seed: int, v_rotation: str, v_codebook: str, scale: float, causal: bool,
                     seq_lens: Optional[torch.Tensor], seq_starts: Optional[torch.Tensor],
                     mask: Optional[torch.Tensor]) -> torch.Tensor:
    return ops.attention_packed(queries, k_norms, k_idx, v_norms, v_idx,
                                codec(k_dim, k_bits, k_seed, k_rotation, k_codebook),
                                codec(v_dim, v_bits, v_seed, v_rotation, v_codebook),
                                scale, causal, seq_lens=seq_lens, seq_starts=seq_starts, mask=mask,
                                _direct=True)


@attention_packed.register_fake
def _(queries, k_norms, k_idx, v_norms, v_idx, k_dim, k_bits, k_seed, k_rotation, k_codebook,
      v_dim, v_bits, v_seed, v_rotation, v_codebook, scale, causal, seq_lens, seq_starts, mask):
    B, Hq, L, _ = queries.shape
    return queries.new_empty((B, Hq, L, v_dim))


@torch.library.custom_op("kaplumba::attention_plain", mutates_args=())
def attention_plain(queries: torch.Tensor, keys: torch.Tensor, values: torch.Tensor, scale: float,
                    causal: bool, seq_lens: Optional[torch.Tensor],
                    seq_starts: Optional[torch.Tensor], mask: Optional[torch.Tensor]) -> torch.Tensor:
    return ops.attention_plain(queries, keys, values, scale, causal, seq_lens=seq_lens,
                               seq_starts=seq_starts, mask=mask, _direct=True)


@attention_plain.register_fake
def _(queries, keys, values, scale, causal, seq_lens, seq_starts, mask):
    B, Hq, L, _ = queries.shape
    return queries.new_empty((B, Hq, L, values.shape[-1]))


@torch.library.custom_op("kaplumba::prod_quantize",
                         mutates_args=("norms", "mse_indices", "residual_norms", "qjl_signs"))
def prod_quantize(x: torch.Tensor, norms: torch.Tensor, mse_indices: torch.Tensor,
                  residual_norms: torch.Tensor, qjl_signs: torch.Tensor, offset: int, dim: int,
                  bits: int, seed: int) -> None:
    st = prod.TurboQuantProdState(norms, mse_indices, residual_norms, qjl_signs)
    prod_codec(dim, bits, seed).quantize_into(x, st, offset, _direct=True)


@prod_quantize.register_fake
def _(x, norms, mse_indices, residual_norms, qjl_signs, offset, dim, bits, seed):
    return None


@torch.library.custom_op("kaplumba::prod_dequantize", mutates_args=())
def prod_dequantize(norms: torch.Tensor, mse_indices: torch.Tensor, residual_norms: torch.Tensor,
                    qjl_signs: torch.Tensor, dim: int, bits: int, seed: int) -> torch.Tensor:
    st = prod.TurboQuantProdState(norms, mse_indices, residual_norms, qjl_signs)
    return prod_codec(dim, bits, seed).dequantize(st, _direct=True)


@prod_dequantize.register_fake
def _(norms, mse_indices, residual_norms, qjl_signs, dim, bits, seed):
    B, H, T = norms.shape
    return norms.new_empty((B, H, T, dim), dtype=torch.float32)


@torch.library.custom_op("kaplumba::attention_prod", mutates_args=())
def attention_prod(queries: torch.Tensor, norms: torch.Tensor, mse_indices: torch.Tensor,
                   residual_norms: torch.Tensor, qjl_signs: torch.Tensor, v_norms: torch.Tensor,
                   v_idx: torch.Tensor, k_dim: int, k_bits: int, k_seed: int, v_dim: int,
                   v_bits: int, v_seed: int, v_rotation: str, v_codebook: str, scale: float,
                   causal: bool, seq_lens: Optional[torch.Tensor], seq_starts: Optional[torch.Tensor],
                   mask: Optional[torch.Tensor]) -> torch.Tensor:
    keys = prod.TurboQuantProdState(norms, mse_indices, residual_norms, qjl_signs)
    return prod.attention_prod(queries, keys, v_norms, v_idx, prod_codec(k_dim, k_bits, k_seed),
                               codec(v_dim, v_bits, v_seed, v_rotation, v_codebook), scale, causal,
                               seq_lens=seq_lens, seq_starts=seq_starts, mask=mask, _direct=True)


@attention_prod.register_fake
def _(queries, norms, mse_indices, residual_norms, qjl_signs, v_norms, v_idx, k_dim, k_bits, k_seed,
      v_dim, v_bits, v_seed, v_rotation, v_codebook, scale, causal, seq_lens, seq_starts, mask):
    B, Hq, L, _ = queries.shape
    return queries.new_empty((B, Hq, L, v_dim))
