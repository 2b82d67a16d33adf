"""Prod codec: MSE at bits - 1 plus a one-bit QJL sketch of the residual.

Mirrors ``_TurboQuantProdCodec`` (turboquant_cache.py:4572-4766) over torch
device tensors and the HIP kernels of libkaplumba_tq.so: ``quantize`` (norm,
MSE indices, residual, signs of ``residual @ P^T``), ``dequantize`` and
attention with Prod-coded keys (``ops.attention_prod``).  The reference
defines the codec but never builds one (no cache constructs it); here it is
reachable through ``ProdCodec`` and ``TurboQuantKVCache(key_quantizer="prod")``.

State per token (``TurboQuantProdState``, :3453-3457): norms, MSE indices
(bits - 1 per coordinate, none at 1 bit), residual norms, QJL sign bits.
"""
from __future__ import annotations

import math
from typing import Dict, NamedTuple, Optional

import numpy as np
import torch

from . import _lib
from . import codebook as cbmod
from .ops import (Codec, _attention_general, _capacity_of, _fields, _opt_tensor, _require_device,
                  _seq_array, _stream, _workspace)

__all__ = ["ProdCodec", "TurboQuantProdState", "attention_prod"]


class TurboQuantProdState(NamedTuple):
    """(norms, mse_indices, residual_norms, qjl_signs) -- turboquant_cache.py:3453-3457."""

    norms: torch.Tensor
    mse_indices: torch.Tensor
    residual_norms: torch.Tensor
    qjl_signs: torch.Tensor


class ProdCodec:
    """``_TurboQuantProdCodec(dim, bits, seed)``: the MSE codec at ``bits - 1``
    with ``seed`` and that codec's own rotation (Hadamard at power-of-two
    dims, dense otherwise, :4122-4139), the projection drawn with
    ``seed + 1`` and ``scale = sqrt(pi / 2) / dim`` (:4573-4585)."""

    def __init__(self, dim: int, bits: int, seed: int):
        pow2 = dim & (dim - 1) == 0
        if dim < 8 or dim > 512 or (pow2 and dim < 32):
            raise NotImplementedError(f"Prod codec kernels are built for head dims 8..512 "
                                      f"(powers of two from 32), got {dim}")
        if int(bits) != bits or not 1 <= bits <= 4:
            raise ValueError(f"Prod codec bits must be 1..4, got {bits}")
        self.dim = dim
        self.bits = int(bits)
        self.seed = seed
        self.mse_bits = self.bits - 1
        # the rotation comes from the MSE codec's seed even at 0 MSE bits
        self.rotation = "hadamard" if pow2 else "dense"
        self.mse_codec = Codec(dim, max(self.mse_bits, 1), seed, self.rotation)
        self.projection = cbmod.projection_matrix(dim, seed + 1)
        self.scale = math.sqrt(math.pi / 2) / dim
        self.mse_width = cbmod.packed_width(dim, self.mse_bits)
        self.sign_width = (dim + 31) // 32
        self._dev: Dict[str, Dict[str, torch.Tensor]] = {}

    def device_tensors(self, device) -> Dict[str, torch.Tensor]:
        key = str(device)
        d = self._dev.get(key)
        if d is None:
            m = self.mse_codec.device_tensors(device)
            d = {"signs": m["rot"], "codebook": m["codebook"], "midpoints": m["midpoints"],
                 "projection": torch.from_numpy(np.ascontiguousarray(self.projection)).to(device)}
            self._dev[key] = d
        return d

    def alloc(self, B: int, H: int, cap: int, device, norm_dtype=torch.float32) -> TurboQuantProdState:
        return TurboQuantProdState(
            torch.zeros((B, H, cap), dtype=norm_dtype, device=device),
            torch.zeros((B, H, cap, self.mse_width), dtype=torch.uint32, device=device),
            torch.zeros((B, H, cap), dtype=norm_dtype, device=device),
            torch.zeros((B, H, cap, self.sign_width), dtype=torch.uint32, device=device))

    def quantize_into(self, x: torch.Tensor, st: TurboQuantProdState, offset: int,
                      _direct: bool = False) -> None:
        """Quantize x (B, H, L, D) into rows offset .. offset + L of capacity buffers."""
        if not _direct and torch.compiler.is_compiling():
            return torch.ops.kaplumba.prod_quantize(x, *st, offset, self.dim, self.bits, self.seed)
        _require_device(x, *st)
        B, H, L, D = x.shape
        if D != self.dim:
            raise ValueError(f"head dim {D} != codec dim {self.dim}")
        cap = st.norms.shape[2]
        want = ((B, H, cap), (B, H, cap, self.mse_width), (B, H, cap), (B, H, cap, self.sign_width))
        if tuple(tuple(t.shape) for t in st) != want or not all(t.is_contiguous() for t in st):
            raise ValueError(f"Prod state buffers must be contiguous {want}")
        if st.norms.dtype != st.residual_norms.dtype:
            raise ValueError("norms and residual norms must share a dtype")
        es = x.element_size()
        if x.stride(-1) != 1 or x.data_ptr() % 16 or any((s * es) % 16 for s in x.stride()[:3]):
            x = x.contiguous()
        lib = _lib.load()
        wsb = lib.tq_prod_workspace_size(B, H, L, D)
        ws = torch.empty(max(wsb, 256), dtype=torch.uint8, device=x.device)
        dt = self.device_tensors(x.device)
        mse = st.mse_indices.data_ptr() if self.mse_bits > 0 else None
        rc = lib.tq_prod_quantize(
            x.data_ptr(), _lib.torch_dtype_code(x.dtype), B, H, L, D,
            x.stride(0), x.stride(1), x.stride(2), self.bits, dt["signs"].data_ptr(),
            dt["midpoints"].data_ptr(), dt["codebook"].data_ptr(), dt["projection"].data_ptr(),
            mse, st.norms.data_ptr(), st.qjl_signs.data_ptr(), st.residual_norms.data_ptr(),
            _lib.torch_dtype_code(st.norms.dtype), cap, offset, ws.data_ptr(), ws.numel(),
            _stream(x))
        _lib.check(rc, "tq_prod_quantize")

    def quantize(self, vectors: torch.Tensor, norm_dtype=torch.float16) -> TurboQuantProdState:
        """``quantize`` (:4597-4666): a fresh state of the vectors' length (norms
        f16, as the reference stores them)."""
        B, H, L, _ = vectors.shape
        st = self.alloc(B, H, L, vectors.device, norm_dtype)
        self.quantize_into(vectors, st, 0)
        return st

    def dequantize(self, state: TurboQuantProdState, _direct: bool = False) -> torch.Tensor:
        """``dequantize`` (:4668-4677): f32 (B, H, T, D)."""
        if not _direct and torch.compiler.is_compiling():
            return torch.ops.kaplumba.prod_dequantize(*state, self.dim, self.bits, self.seed)
        _require_device(*state)
        B, H, T = state.norms.shape
        cap = _capacity_of(state.norms, state.qjl_signs, self.sign_width)
        if self.mse_bits > 0 and _capacity_of(state.norms, state.mse_indices, self.mse_width) != cap:
            raise ValueError("Prod state buffers must share a capacity")
        out = torch.empty((B, H, T, self.dim), dtype=torch.float32, device=state.norms.device)
        dt = self.device_tensors(out.device)
        lib = _lib.load()
        rc = lib.tq_prod_dequantize(
            state.norms.data_ptr(), state.mse_indices.data_ptr() if self.mse_bits > 0 else None,
            state.residual_norms.data_ptr(), state.qjl_signs.data_ptr(),
            _lib.torch_dtype_code(state.norms.dtype), B, H, T, self.dim, self.bits, cap,
            dt["signs"].data_ptr(), dt["codebook"].data_ptr(), dt["projection"].data_ptr(),
            out.data_ptr(), _stream(out))
        _lib.check(rc, "tq_prod_dequantize")
        return out


def attention_prod(queries: torch.Tensor, keys: TurboQuantProdState, v_norms: torch.Tensor,
                   v_idx: torch.Tensor, key_codec: ProdCodec, value_codec: Codec, scale: float,
                   causal: bool, seq_lens: Optional[torch.Tensor] = None,
                   seq_starts: Optional[torch.Tensor] = None, mask=None,
                   _direct: bool = False) -> torch.Tensor:
    """Attention with Prod-coded keys and MSE-coded values (``tq_attention_prod``):
    the fused Prod decode kernel's scores (turboquant_cache.py:2000-2206) with
    ``quantized_attention``'s softmax and masks.  Views (B, Hkv, T[, W]) of
    contiguous capacity buffers, as the cache hands them out.  ``mask`` is an
    optional array mask (``ops.prepare_mask``); a value codec of another dim or
    rotation, or a mask, runs ``tq_attention_general``."""
    if not _direct and torch.compiler.is_compiling():
        return torch.ops.kaplumba.attention_prod(
            queries, *keys, v_norms, v_idx, key_codec.dim, key_codec.bits, key_codec.seed,
            *_fields(value_codec), float(scale), bool(causal), _opt_tensor(seq_lens, torch.int32),
            _opt_tensor(seq_starts, torch.int32), _opt_tensor(mask, None))
    _require_device(queries, *keys, v_norms, v_idx)
    B, Hq, L, D = queries.shape
    Hkv, T = keys.norms.shape[1], keys.norms.shape[2]
    if key_codec.dim != D:
        raise ValueError(f"query head dim {D} != key codec dim {key_codec.dim}")
    if Hq % Hkv:
        raise ValueError(f"{Hq} query heads are not a multiple of {Hkv} kv heads")
    if queries.stride(-1) != 1:
        queries = queries.contiguous()
    cap = _capacity_of(keys.norms, keys.qjl_signs, key_codec.sign_width)
    for nrm, idx, w in ((keys.norms, keys.mse_indices, key_codec.mse_width),
                        (v_norms, v_idx, value_codec.packed_width)):
        if w and _capacity_of(nrm, idx, w) != cap:
            raise ValueError("key and value buffers must share a capacity")
    if keys.residual_norms.shape != keys.norms.shape or keys.residual_norms.stride() != keys.norms.stride():
        raise ValueError("residual norms must share the norms' layout")
    if not (keys.norms.dtype == keys.residual_norms.dtype == v_norms.dtype):
        raise ValueError("key norms, residual norms and value norms must share a dtype")
    seq_lens = _seq_array(seq_lens, B, queries.device)
    seq_starts = _seq_array(seq_starts, B, queries.device)
    kt, vt = key_codec.device_tensors(queries.device), value_codec.device_tensors(queries.device)
    if (mask is not None or value_codec.dim != D or value_codec.rotation != "hadamard"
            or key_codec.rotation != "hadamard"):
        return _attention_general(
            queries, Dv=value_codec.dim, kv_kind=_lib.TQ_KV_PROD, kv_dtype=0,
            k=keys.mse_indices if key_codec.mse_bits > 0 else None, k_norms=keys.norms,
            k_signs=keys.qjl_signs, k_rnorms=keys.residual_norms, k_bits=key_codec.bits,
            k_codebook=kt["codebook"], k_rot_kind=key_codec.mse_codec.rot_kind, k_rot=kt["signs"],
            projection=kt["projection"], v=v_idx, v_norms=v_norms, v_bits=value_codec.bits,
            v_codebook=vt["codebook"], v_rot_kind=value_codec.rot_kind, v_rot=vt["rot"],
            norm_dtype=_lib.torch_dtype_code(v_norms.dtype), cap=cap, T=T, scale=scale,
            causal=causal, mask=mask, seq_lens=seq_lens, seq_starts=seq_starts)
    out = torch.empty((B, Hq, L, D), dtype=queries.dtype, device=queries.device)
    lib = _lib.load()
    ws = _workspace(queries.device, lib.tq_attention_prod_workspace_size(B, Hq, Hkv, L, D, T))
    rc = lib.tq_attention_prod(
        queries.data_ptr(), _lib.torch_dtype_code(queries.dtype), B, Hq, Hkv, L, D,
        queries.stride(0), queries.stride(1), queries.stride(2), float(scale),
        keys.mse_indices.data_ptr(), keys.norms.data_ptr(), keys.qjl_signs.data_ptr(),
        keys.residual_norms.data_ptr(), key_codec.bits, kt["codebook"].data_ptr(),
        kt["signs"].data_ptr(), kt["projection"].data_ptr(), v_idx.data_ptr(), v_norms.data_ptr(),
        value_codec.bits, vt["codebook"].data_ptr(), vt["rot"].data_ptr(),
        _lib.torch_dtype_code(v_norms.dtype), cap, T,
        seq_starts.data_ptr() if seq_starts is not None else None,
        seq_lens.data_ptr() if seq_lens is not None else None, 1 if causal else 0,
        out.data_ptr(), ws.data_ptr(), ws.numel(), _stream(queries))
    _lib.check(rc, "tq_attention_prod")
    return out
