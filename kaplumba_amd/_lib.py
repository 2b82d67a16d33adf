"""ctypes binding of libkaplumba_tq.so (the C ABI declared in include/kaplumba_tq.h).

torch is imported first on purpose: torch ships the HIP runtime
(libamdhip64.so.7), and loading it before this library makes both share one
runtime, so the hipStream_t handles and device pointers torch hands out are
valid here.  There is no fallback: if the library is missing, every op raises.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import c_float, c_int, c_int64, c_void_p, c_char_p

import torch  # noqa: F401  (must precede the CDLL load, see module docstring)

LIB_NAME = "libkaplumba_tq.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

TQ_OK = 0
TQ_ERR_INVALID_ARGUMENT = 1
TQ_ERR_UNSUPPORTED = 2
TQ_ERR_WORKSPACE = 3
TQ_ERR_HIP = 4

TQ_DTYPE_F32, TQ_DTYPE_F16, TQ_DTYPE_BF16 = 0, 1, 2
TQ_ROT_HADAMARD, TQ_ROT_DENSE = 0, 1
TQ_KV_PACKED, TQ_KV_PLAIN, TQ_KV_PROD = 0, 1, 2
TQ_MASK_NONE, TQ_MASK_BOOL, TQ_MASK_ADD_F32, TQ_MASK_ADD_F16, TQ_MASK_ADD_BF16 = 0, 1, 2, 3, 4

# name -> (restype, argtypes); the single source of truth for the exported set.
SIGNATURES = {
    "tq_version": (c_char_p, []),
    "tq_last_error": (c_char_p, []),
    "tq_packed_width": (c_int, [c_int, c_int]),
    "tq_append_quantize": (c_int, [
        c_void_p, c_int, c_int, c_int, c_int, c_int,      # x, dtype, B, H, L, dim
        c_int64, c_int64, c_int64,                          # strides
        c_int, c_int, c_void_p, c_void_p,                   # bits, rot_kind, rot, midpoints
        c_void_p, c_void_p, c_int,                          # packed, norms, norm_dtype
        c_int64, c_int64, c_void_p]),                       # capacity, offset, stream
    "tq_append_quantize_kv": (c_int, [
        c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int,   # k_x, v_x, dtype, B, H, L, dim
        c_int64, c_int64, c_int64, c_int64, c_int64, c_int64,    # k strides, v strides
        c_int, c_int, c_int, c_void_p, c_void_p,                 # k_bits, v_bits, rot_kind, rots
        c_void_p, c_void_p,                                      # midpoints
        c_void_p, c_void_p, c_void_p, c_void_p, c_int,           # k packed/norms, v packed/norms, norm_dtype
        c_int64, c_int64, c_void_p]),                            # capacity, offset, stream
    "tq_prod_workspace_size": (c_int64, [c_int, c_int, c_int, c_int]),
    "tq_prod_quantize": (c_int, [
        c_void_p, c_int, c_int, c_int, c_int, c_int,           # x, dtype, B, H, L, dim
        c_int64, c_int64, c_int64,                              # strides
        c_int, c_void_p, c_void_p, c_void_p, c_void_p,          # bits, signs, mids, codebook, P
        c_void_p, c_void_p, c_void_p, c_void_p, c_int,          # mse, norms, qjl signs, rnorms, norm_dtype
        c_int64, c_int64, c_void_p, c_int64, c_void_p]),        # capacity, offset, workspace, bytes, stream
    "tq_prod_dequantize": (c_int, [
        c_void_p, c_void_p, c_void_p, c_void_p, c_int,          # norms, mse, rnorms, signs, norm_dtype
        c_int, c_int, c_int, c_int, c_int, c_int64,             # B, H, T, dim, bits, capacity
        c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),     # signs, codebook, P, out, stream
    "tq_append_plain": (c_int, [
        c_void_p, c_int, c_int, c_int, c_int, c_int,
        c_int64, c_int64, c_int64, c_void_p, c_int64, c_int64, c_void_p]),
    "tq_dequantize": (c_int, [
        c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int, c_int, c_int64,
        c_void_p, c_int, c_void_p, c_void_p, c_void_p]),
    "tq_attention_workspace_size": (c_int64, [c_int, c_int, c_int, c_int, c_int, c_int64]),
    "tq_attention_prod_workspace_size": (c_int64, [c_int, c_int, c_int, c_int, c_int, c_int64]),
    "tq_attention": (c_int, [
        c_void_p, c_int, c_int, c_int, c_int, c_int, c_int,   # q, dtype, B, Hq, Hkv, L, dim
        c_int64, c_int64, c_int64, c_float,                    # q strides, scale
        c_int, c_int,                                          # kv_kind, kv_dtype
        c_void_p, c_void_p, c_void_p, c_void_p,                # k, k_norms, v, v_norms
        c_int, c_int, c_int,                                   # norm_dtype, k_bits, v_bits
        c_void_p, c_void_p,                                    # codebooks
        c_int, c_void_p, c_void_p,                             # rot_kind, k_rot, v_rot
        c_int64, c_int64, c_void_p, c_int,                     # capacity, max_tokens, seq_lens, causal
        c_void_p, c_void_p, c_int64, c_void_p]),               # out, workspace, ws bytes, stream
    "tq_attention_prod": (c_int, [
        c_void_p, c_int, c_int, c_int, c_int, c_int, c_int,   # q, dtype, B, Hq, Hkv, L, dim
        c_int64, c_int64, c_int64, c_float,                    # q strides, scale
        c_void_p, c_void_p, c_void_p, c_void_p, c_int,         # k mse, norms, signs, rnorms, k_bits
        c_void_p, c_void_p, c_void_p,                          # k mse codebook, k rot signs, P
        c_void_p, c_void_p, c_int, c_void_p, c_void_p,         # v, v_norms, v_bits, v codebook, v signs
        c_int, c_int64, c_int64, c_void_p, c_void_p, c_int,    # norm dtype, cap, T, starts, lens, causal
        c_void_p, c_void_p, c_int64, c_void_p]),               # out, workspace, ws bytes, stream
    "tq_attention_ranged": (c_int, [
        c_void_p, c_int, c_int, c_int, c_int, c_int, c_int,
        c_int64, c_int64, c_int64, c_float,
        c_int, c_int,
        c_void_p, c_void_p, c_void_p, c_void_p,
        c_int, c_int, c_int,
        c_void_p, c_void_p,
        c_int, c_void_p, c_void_p,
        c_int64, c_int64, c_void_p, c_void_p, c_int,           # ..., seq_starts, seq_lens, causal
        c_void_p, c_void_p, c_int64, c_void_p]),
    "tq_attention_noalloc": (c_int, [
        c_void_p, c_int, c_int, c_int, c_int, c_int, c_int,
        c_int64, c_int64, c_int64, c_float,
        c_int, c_int,
        c_void_p, c_void_p, c_void_p, c_void_p,
        c_int, c_int, c_int,
        c_void_p, c_void_p,
        c_int, c_void_p, c_void_p,
        c_int64, c_int64, c_void_p, c_void_p, c_int,           # ..., seq_starts, seq_lens, causal
        c_void_p, c_void_p]),                                  # out, stream (static scratch)
    "tq_attention_general_workspace_size": (c_int64, [c_int, c_int, c_int, c_int, c_int, c_int,
                                                      c_int64]),
    "tq_attention_general": (c_int, [
        c_void_p, c_int, c_int, c_int, c_int, c_int, c_int, c_int,  # q, dtype, B, Hq, Hkv, L, k_dim, v_dim
        c_int64, c_int64, c_int64, c_float,                    # q strides, scale
        c_int, c_int,                                          # kv_kind, kv_dtype
        c_void_p, c_void_p, c_void_p, c_void_p, c_int,         # k, k_norms, k_signs, k_rnorms, k_bits
        c_void_p, c_int, c_void_p, c_void_p,                   # k codebook, k_rot_kind, k_rot, projection
        c_void_p, c_void_p, c_int, c_void_p, c_int, c_void_p,  # v, v_norms, v_bits, v codebook, v_rot_kind, v_rot
        c_int, c_int64, c_int64, c_void_p, c_void_p, c_int,    # norm dtype, cap, T, starts, lens, causal
        c_void_p, c_int, c_void_p,                             # mask, mask_kind, mask_strides (5 x int64)
        c_void_p, c_void_p, c_int64, c_void_p]),               # out, workspace, ws bytes, stream
}

# Scratch bytes of tq_attention_noalloc (TQ_NOALLOC_SCRATCH_BYTES in the header).
TQ_NOALLOC_SCRATCH_BYTES = 16 << 20


class TurboQuantLibraryError(RuntimeError):
    """The native library is missing or a call into it failed."""


_lib = None


def load() -> ctypes.CDLL:
    """Load (once) and return the native library; raise if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise TurboQuantLibraryError(
            f"{LIB_NAME} not found at {LIB_PATH}; build it with "
            "`python -c 'import __graft_entry__ as g; g.build()'` or "
            "`make -C kaplumba_amd/csrc`.")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(rc: int, what: str) -> None:
    """Turn a status code into a Python exception (ValueError for bad input)."""
    if rc == TQ_OK:
        return
    msg = load().tq_last_error().decode(errors="replace")
    if rc in (TQ_ERR_INVALID_ARGUMENT, TQ_ERR_WORKSPACE):
        raise ValueError(f"{what}: {msg}")
    if rc == TQ_ERR_UNSUPPORTED:
        raise NotImplementedError(f"{what}: {msg}")
    raise TurboQuantLibraryError(f"{what}: {msg} (status {rc})")


def torch_dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.float32:
        return TQ_DTYPE_F32
    if dtype == torch.float16:
        return TQ_DTYPE_F16
    if dtype == torch.bfloat16:
        return TQ_DTYPE_BF16
    raise ValueError(f"unsupported dtype {dtype} (float32, float16 or bfloat16)")
