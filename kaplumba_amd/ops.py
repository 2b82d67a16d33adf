"""torch-facing wrappers over the C ABI (device pointers + the current stream).

Every function here enqueues HIP kernels from libkaplumba_tq.so on torch's
current stream for the tensor's device.  Tensors must live on a ROCm device;
there is no CPU path.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field
from typing import Dict, Optional

import numpy as np
import torch

from . import _lib
from . import codebook as cbmod

ROTATIONS = {"hadamard": _lib.TQ_ROT_HADAMARD, "dense": _lib.TQ_ROT_DENSE}


def _fields(c: "Codec") -> tuple:
    """A codec's defining fields, as the torch.ops.kaplumba operators take them."""
    return (c.dim, c.bits, c.seed, c.rotation, c.codebook_kind)


def _opt_tensor(x, dtype):
    """None, a tensor, or x as a tensor (lists and arrays of lengths, starts or masks)."""
    if x is None or isinstance(x, torch.Tensor):
        return x
    return torch.as_tensor(np.asarray(x), dtype=dtype)


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _require_device(*ts: torch.Tensor) -> None:
    for t in ts:
        if not isinstance(t, torch.Tensor) or t.device.type != "cuda":
            raise ValueError("TurboQuant kernels need ROCm device tensors "
                             f"(got {getattr(t, 'device', type(t))}); there is no CPU path")


@dataclass
class Codec:
    """One quantizer: dim, bits, seed, rotation kind and codebook kind.

    Mirrors ``_TurboQuantMSECodec.__init__`` (turboquant_cache.py:4122-4139):
    Hadamard rotation with signs for power-of-two dims, a dense QR rotation
    otherwise (or when asked for), the Lloyd-Max codebook and its midpoints.
    """

    dim: int
    bits: int
    seed: int
    rotation: str = "auto"
    codebook_kind: str = "beta"
    _dev: Dict[str, Dict[str, torch.Tensor]] = field(default_factory=dict, repr=False)

    def __post_init__(self) -> None:
        pow2 = self.dim > 0 and (self.dim & (self.dim - 1)) == 0
        if self.rotation == "auto":
            self.rotation = "hadamard" if pow2 else "dense"
        if self.rotation not in ROTATIONS:
            raise ValueError(f"rotation must be 'auto', 'hadamard' or 'dense', got {self.rotation!r}")
        if self.rotation == "hadamard" and not pow2:
            raise ValueError(f"Hadamard rotation needs a power-of-two head dim, got {self.dim}")
        self.use_rht = self.rotation == "hadamard"
        self.codebook = cbmod.codebook(self.dim, self.bits, self.codebook_kind)
        self.midpoints = cbmod.midpoints(self.codebook)
        self.packed_width = cbmod.packed_width(self.dim, self.bits)

    @property
    def rot_kind(self) -> int:
        return ROTATIONS[self.rotation]

    @property
    def rot_host(self) -> np.ndarray:
        if self.use_rht:
            return cbmod.rht_sign_vector(self.dim, self.seed)
        return cbmod.rotation_matrix(self.dim, self.seed)

    def device_tensors(self, device: torch.device) -> Dict[str, torch.Tensor]:
        key = str(device)
        d = self._dev.get(key)
        if d is None:
            d = {
                "rot": torch.from_numpy(np.array(self.rot_host, dtype=np.float32, order="C")).to(device),
                "codebook": torch.from_numpy(self.codebook.copy()).to(device),
                "midpoints": torch.from_numpy(
                    self.midpoints.copy() if self.midpoints.size else np.zeros(1, np.float32)).to(device),
            }
            self._dev[key] = d
        return d


def append_quantize(x: torch.Tensor, codec: Codec, packed: torch.Tensor, norms: torch.Tensor,
                    offset: int, _direct: bool = False) -> None:
    """Quantize x (B, H, L, D) into rows offset..offset+L of the capacity buffers.

    packed: (B, H, cap, PW) uint32 contiguous; norms: (B, H, cap) f32/f16 contiguous.
    """
    if not _direct and torch.compiler.is_compiling():
        return torch.ops.kaplumba.append_quantize(x, packed, norms, offset, *_fields(codec))
    _require_device(x, packed, norms)
    x = _check_append_buffers(x, codec, packed, norms)
    B, H, L, D = x.shape
    cap = packed.shape[2]
    dt = codec.device_tensors(x.device)
    lib = _lib.load()
    rc = lib.tq_append_quantize(
        x.data_ptr(), _lib.torch_dtype_code(x.dtype), B, H, L, D,
        x.stride(0), x.stride(1), x.stride(2),
        codec.bits, codec.rot_kind, dt["rot"].data_ptr(), dt["midpoints"].data_ptr(),
        packed.data_ptr(), norms.data_ptr(), _lib.torch_dtype_code(norms.dtype),
        cap, offset, _stream(x))
    _lib.check(rc, "tq_append_quantize")


def _check_append_buffers(x: torch.Tensor, codec: Codec, packed: torch.Tensor,
                          norms: torch.Tensor) -> torch.Tensor:
    """Validated (and, if needed, compacted) input of one quantize side."""
    B, H, L, D = x.shape
    if D != codec.dim:
        raise ValueError(f"head dim {D} != codec dim {codec.dim}")
    if x.stride(-1) != 1:
        x = x.contiguous()
    if not (packed.is_contiguous() and norms.is_contiguous()):
        raise ValueError("cache buffers must be contiguous")
    cap = packed.shape[2]
    if packed.shape != (B, H, cap, codec.packed_width) or norms.shape != (B, H, cap):
        raise ValueError(f"buffer shapes {tuple(packed.shape)}/{tuple(norms.shape)} "
                         f"do not match ({B}, {H}, cap, {codec.packed_width})")
    es = x.element_size()
    if x.data_ptr() % 16 or any((s * es) % 16 for s in x.stride()[:3]):
        x = x.contiguous()
    return x


def append_quantize_kv(k: torch.Tensor, v: torch.Tensor, key_codec: Codec, value_codec: Codec,
                       k_packed: torch.Tensor, k_norms: torch.Tensor, v_packed: torch.Tensor,
                       v_norms: torch.Tensor, offset: int, _direct: bool = False) -> None:
    """Quantize keys and values (B, H, L, D) of one append in one library call.

    Both sides share shape, dtype, rotation kind, norm dtype and capacity;
    anything else goes through two append_quantize calls.
    """
    if not _direct and torch.compiler.is_compiling():
        return torch.ops.kaplumba.append_quantize_kv(k, v, k_packed, k_norms, v_packed, v_norms,
                                                     offset, *_fields(key_codec),
                                                     *_fields(value_codec))
    same = (k.shape == v.shape and k.dtype == v.dtype and key_codec.dim == value_codec.dim
            and key_codec.rot_kind == value_codec.rot_kind and k_norms.dtype == v_norms.dtype
            and k_packed.shape[2] == v_packed.shape[2])
    if not same:
        append_quantize(k, key_codec, k_packed, k_norms, offset, _direct=True)
        append_quantize(v, value_codec, v_packed, v_norms, offset, _direct=True)
        return
    _require_device(k, v, k_packed, k_norms, v_packed, v_norms)
    k = _check_append_buffers(k, key_codec, k_packed, k_norms)
    v = _check_append_buffers(v, value_codec, v_packed, v_norms)
    B, H, L, D = k.shape
    kt, vt = key_codec.device_tensors(k.device), value_codec.device_tensors(k.device)
    rc = _lib.load().tq_append_quantize_kv(
        k.data_ptr(), v.data_ptr(), _lib.torch_dtype_code(k.dtype), B, H, L, D,
        k.stride(0), k.stride(1), k.stride(2), v.stride(0), v.stride(1), v.stride(2),
        key_codec.bits, value_codec.bits, key_codec.rot_kind, kt["rot"].data_ptr(),
        vt["rot"].data_ptr(), kt["midpoints"].data_ptr(), vt["midpoints"].data_ptr(),
        k_packed.data_ptr(), k_norms.data_ptr(), v_packed.data_ptr(), v_norms.data_ptr(),
        _lib.torch_dtype_code(k_norms.dtype), k_packed.shape[2], offset, _stream(k))
    _lib.check(rc, "tq_append_quantize_kv")


def append_plain(x: torch.Tensor, dst: torch.Tensor, offset: int, _direct: bool = False) -> None:
    """Copy x (B, H, L, D) into rows offset.. of dst (B, H, cap, D) (fp16/bf16)."""
    if not _direct and torch.compiler.is_compiling():
        return torch.ops.kaplumba.append_plain(x, dst, offset)
    _require_device(x, dst)
    B, H, L, D = x.shape
    if x.dtype != dst.dtype:
        x = x.to(dst.dtype)
    if x.stride(-1) != 1 or x.data_ptr() % 16 or any((s * 2) % 16 for s in x.stride()[:3]):
        x = x.contiguous()
    if not dst.is_contiguous() or dst.shape[:2] != (B, H) or dst.shape[3] != D:
        raise ValueError("plain buffer must be contiguous (B, H, cap, D)")
    rc = _lib.load().tq_append_plain(
        x.data_ptr(), _lib.torch_dtype_code(x.dtype), B, H, L, D,
        x.stride(0), x.stride(1), x.stride(2), dst.data_ptr(), dst.shape[2], offset, _stream(x))
    _lib.check(rc, "tq_append_plain")


def _capacity_of(norms: torch.Tensor, indices: torch.Tensor, pw: int) -> int:
    """Token capacity of the contiguous (B, H, cap[, PW]) buffer a state view slices.

    State views returned by the cache are ``buf[..., :T]`` slices, so the
    capacity is recovered from the strides; a fresh contiguous state has
    capacity T.
    """
    B, H, T = norms.shape
    if H > 1:
        cap = norms.stride(1)
    elif B > 1:
        cap = norms.stride(0)
    else:
        cap = max(T, 1)
    ok = indices.shape[:3] == norms.shape and indices.shape[3] == pw
    ok = ok and (T <= 1 or (norms.stride(2) == 1 and indices.stride(2) == pw))
    ok = ok and indices.stride(3) == 1 and cap >= T
    if H > 1:
        ok = ok and indices.stride(1) == cap * pw
    if B > 1:
        ok = ok and norms.stride(0) == H * cap and indices.stride(0) == H * cap * pw
    if not ok:
        raise ValueError("state views must slice contiguous (B, H, cap) norms and "
                         f"(B, H, cap, {pw}) index buffers")
    return cap


def dequantize(indices: torch.Tensor, norms: torch.Tensor, codec: Codec,
               _direct: bool = False) -> torch.Tensor:
    """f32 (B, H, T, D) reconstruction n * R^-1(codebook[idx])."""
    if not _direct and torch.compiler.is_compiling():
        return torch.ops.kaplumba.dequantize(indices, norms, *_fields(codec))
    _require_device(indices, norms)
    B, H, T = norms.shape
    out = torch.empty((B, H, T, codec.dim), dtype=torch.float32, device=norms.device)
    if B * H * T == 0:
        return out
    cap = _capacity_of(norms, indices, codec.packed_width)
    dt = codec.device_tensors(norms.device)
    rc = _lib.load().tq_dequantize(
        indices.data_ptr(), norms.data_ptr(), _lib.torch_dtype_code(norms.dtype),
        B, H, T, codec.dim, codec.bits, cap, dt["codebook"].data_ptr(), codec.rot_kind,
        dt["rot"].data_ptr(), out.data_ptr(), _stream(norms))
    _lib.check(rc, "tq_dequantize")
    return out


_WORKSPACES: Dict[tuple, torch.Tensor] = {}
# Workspaces replaced by a larger one.  They are never freed: a HIP graph
# captured while one of them was current still holds its address, and a replay
# must not write into memory the allocator has handed to another tensor.
# Sizes grow at least twofold per replacement, so the kept buffers add up to
# less than the current one.
_RETIRED_WORKSPACES: list = []


def _grown_size(current: int, need: int) -> int:
    """Size of the buffer that replaces one of ``current`` bytes (0: none) when
    a call needs ``need`` bytes: at least 1 MiB, ``need``, and twice
    ``current``."""
    return max(need, 1 << 20, 2 * current)


def _workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """Persistent attention workspace per (device, stream).

    The kernels write every workspace byte they read (rotated queries and
    split partials), so one buffer serves every later call on that stream,
    whatever the shapes, and needs no initial contents; calls on other
    streams get their own.  A request beyond the current size allocates a
    larger buffer (at least twice the old size) and keeps the old one alive
    (see _RETIRED_WORKSPACES); ``reserve_workspace`` sizes it once before
    graph capture.
    """
    key = (str(device), torch.cuda.current_stream(device).cuda_stream)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        if ws is not None:
            _RETIRED_WORKSPACES.append(ws)
        size = _grown_size(0 if ws is None else ws.numel(), nbytes)
        ws = torch.empty(size, dtype=torch.uint8, device=device)
        _WORKSPACES[key] = ws
    return ws


def reserve_workspace(device, B: int, Hq: int, Hkv: int, L: int, dim: int,
                      max_tokens: int) -> int:
    """Size the current stream's attention workspace for the largest problem a
    caller will run (for example before capturing decode graphs for several
    batch sizes), so no later call on that stream replaces it.  Returns bytes."""
    device = torch.device(device)
    nbytes = int(_lib.load().tq_attention_workspace_size(B, Hq, Hkv, L, dim, max_tokens))
    _workspace(device, nbytes)
    return nbytes


def _seq_array(x, B: int, device) -> Optional[torch.Tensor]:
    """(B,) int32 device copy of per-sequence starts / lengths (or None)."""
    if x is None:
        return None
    x = torch.as_tensor(x).to(device=device, dtype=torch.int32).reshape(-1).contiguous()
    if x.numel() != B:
        raise ValueError(f"expected {B} per-sequence values, got {x.numel()}")
    return x


def _call_attention(lib, head, seq_starts, seq_lens, tail, what: str) -> None:
    """tq_attention, or tq_attention_ranged when sequences carry left padding."""
    lens = seq_lens.data_ptr() if seq_lens is not None else None
    if seq_starts is None:
        rc = lib.tq_attention(*head, lens, *tail)
    else:
        rc = lib.tq_attention_ranged(*head, seq_starts.data_ptr(), lens, *tail)
    _lib.check(rc, what)


def prepare_mask(mask, B: int, Hkv: int, R: int, L: int, T: int, device, grouped: bool = True):
    """An array mask as (tensor kept alive, mask kind, 5 element strides) over
    the grouped scores (B, Hkv, R, L, T).

    ``grouped`` follows ``_apply_attention_mask`` (turboquant_cache.py:5101-5104):
    the mask is sliced ``[..., :L, :T]``, a 4-D mask gets its repeat axis
    inserted at position 2, and the rest is broadcasting against
    (B, Hkv, R, L, T).  Otherwise (the fp16 layers' SDPA, base.py:218-226) it
    broadcasts against (B, Hq, L, T) and head h = g * R + r.  Boolean masks
    keep a score where True; float masks are added.  Key index t is the cache
    row (left padding included).
    """
    m = mask if isinstance(mask, torch.Tensor) else torch.as_tensor(np.asarray(mask))
    m = m.to(device)
    if m.dtype == torch.bool:
        kind = _lib.TQ_MASK_BOOL
    elif m.dtype == torch.float32:
        kind = _lib.TQ_MASK_ADD_F32
    elif m.dtype == torch.float16:
        kind = _lib.TQ_MASK_ADD_F16
    elif m.dtype == torch.bfloat16:
        kind = _lib.TQ_MASK_ADD_BF16
    else:
        m, kind = m.to(torch.float32), _lib.TQ_MASK_ADD_F32
    if m.dim() < 2:
        raise ValueError(f"attention mask needs (..., queries, keys) axes, got shape {tuple(m.shape)}")
    m = m[..., :L, :T]
    try:
        if grouped:
            if m.dim() == 4:
                m = m.unsqueeze(2)
            if m.dim() > 5:
                raise RuntimeError("more than 5 axes")
            m = m.expand(B, Hkv, R, L, T)
            strides = m.stride()
        else:
            if m.dim() > 4:
                raise RuntimeError("more than 4 axes")
            m = m.expand(B, Hkv * R, L, T)
            sb, sh, sl, st = m.stride()
            strides = (sb, R * sh, sh, sl, st)
    except RuntimeError as e:
        want = f"(B, Hkv, R, L, T) = {(B, Hkv, R, L, T)}" if grouped else f"(B, Hq, L, T) = {(B, Hkv * R, L, T)}"
        raise ValueError(f"attention mask of shape {tuple(mask.shape)} does not broadcast to {want}: {e}")
    st5 = (ctypes.c_int64 * 5)(*strides)
    return m, kind, st5


def _attention_general(queries: torch.Tensor, *, Dv: int, kv_kind: int, kv_dtype: int, k, k_norms,
                       k_signs, k_rnorms, k_bits: int, k_codebook, k_rot_kind: int, k_rot,
                       projection, v, v_norms, v_bits: int, v_codebook, v_rot_kind: int, v_rot,
                       norm_dtype: int, cap: int, T: int, scale: float, causal: bool, mask,
                       seq_lens, seq_starts, grouped_mask: bool = True) -> torch.Tensor:
    """One tq_attention_general call (pointers may be None where unused)."""
    B, Hq, L, Dk = queries.shape
    Hkv = (k_norms if k_norms is not None else k).shape[1]
    R = Hq // Hkv
    mt, mkind, mstr = (None, _lib.TQ_MASK_NONE, None)
    if mask is not None:
        mt, mkind, mstr = prepare_mask(mask, B, Hkv, R, L, T, queries.device, grouped_mask)
    out = torch.empty((B, Hq, L, Dv), dtype=queries.dtype, device=queries.device)
    lib = _lib.load()
    ws = _workspace(queries.device, lib.tq_attention_general_workspace_size(B, Hq, Hkv, L, Dk, Dv, T))

    def ptr(t):
        return t.data_ptr() if t is not None else None

    rc = lib.tq_attention_general(
        queries.data_ptr(), _lib.torch_dtype_code(queries.dtype), B, Hq, Hkv, L, Dk, Dv,
        queries.stride(0), queries.stride(1), queries.stride(2), float(scale), kv_kind, kv_dtype,
        ptr(k), ptr(k_norms), ptr(k_signs), ptr(k_rnorms), k_bits, ptr(k_codebook), k_rot_kind,
        ptr(k_rot), ptr(projection), ptr(v), ptr(v_norms), v_bits, ptr(v_codebook), v_rot_kind,
        ptr(v_rot), norm_dtype, cap, T, ptr(seq_starts), ptr(seq_lens), 1 if causal else 0,
        ptr(mt), mkind, mstr, out.data_ptr(), ws.data_ptr(), ws.numel(), _stream(queries))
    _lib.check(rc, "tq_attention_general")
    return out


def attention_packed(queries: torch.Tensor, k_norms: torch.Tensor, k_idx: torch.Tensor,
                     v_norms: torch.Tensor, v_idx: torch.Tensor, key_codec: Codec,
                     value_codec: Codec, scale: float, causal: bool,
                     seq_lens: Optional[torch.Tensor] = None,
                     seq_starts: Optional[torch.Tensor] = None, mask=None,
                     _direct: bool = False) -> torch.Tensor:
    """Attention straight from packed K/V state views (B, Hkv, T[, PW]).

    ``seq_lens`` (B,) ends each sequence before T (ragged batches);
    ``seq_starts`` (B,) skips each sequence's left padding; ``mask`` is an
    optional array mask (``prepare_mask``).  Key and value codecs may differ
    in head dim and rotation; the output has the value dim
    (turboquant_cache.py:5131).
    """
    if not _direct and torch.compiler.is_compiling():
        return torch.ops.kaplumba.attention_packed(
            queries, k_norms, k_idx, v_norms, v_idx, *_fields(key_codec), *_fields(value_codec),
            float(scale), bool(causal), _opt_tensor(seq_lens, torch.int32),
            _opt_tensor(seq_starts, torch.int32), _opt_tensor(mask, None))
    _require_device(queries, k_norms, k_idx, v_norms, v_idx)
    B, Hq, L, D = queries.shape
    Hkv, T = k_norms.shape[1], k_norms.shape[2]
    if key_codec.dim != D:
        raise ValueError(f"query head dim {D} != key codec dim {key_codec.dim}")
    if Hq % Hkv:
        raise ValueError(f"{Hq} query heads are not a multiple of {Hkv} kv heads")
    if queries.stride(-1) != 1:
        queries = queries.contiguous()
    cap = _capacity_of(k_norms, k_idx, key_codec.packed_width)
    vcap = _capacity_of(v_norms, v_idx, value_codec.packed_width)
    if vcap != cap:
        raise ValueError("key and value buffers must share a capacity")
    if k_norms.dtype != v_norms.dtype:
        raise ValueError("key and value norms must share a dtype")
    seq_lens = _seq_array(seq_lens, B, queries.device)
    seq_starts = _seq_array(seq_starts, B, queries.device)
    kt = key_codec.device_tensors(queries.device)
    vt = value_codec.device_tensors(queries.device)
    if (mask is not None or value_codec.dim != D or key_codec.rotation != value_codec.rotation):
        return _attention_general(
            queries, Dv=value_codec.dim, kv_kind=_lib.TQ_KV_PACKED, kv_dtype=0, k=k_idx,
            k_norms=k_norms, k_signs=None, k_rnorms=None, k_bits=key_codec.bits,
            k_codebook=kt["codebook"], k_rot_kind=key_codec.rot_kind, k_rot=kt["rot"],
            projection=None, v=v_idx, v_norms=v_norms, v_bits=value_codec.bits,
            v_codebook=vt["codebook"], v_rot_kind=value_codec.rot_kind, v_rot=vt["rot"],
            norm_dtype=_lib.torch_dtype_code(k_norms.dtype), cap=cap, T=T, scale=scale,
            causal=causal, mask=mask, seq_lens=seq_lens, seq_starts=seq_starts)
    out = torch.empty((B, Hq, L, D), dtype=queries.dtype, device=queries.device)
    lib = _lib.load()
    wsb = lib.tq_attention_workspace_size(B, Hq, Hkv, L, D, T)
    ws = _workspace(queries.device, wsb)
    head = (queries.data_ptr(), _lib.torch_dtype_code(queries.dtype), B, Hq, Hkv, L, D,
            queries.stride(0), queries.stride(1), queries.stride(2), float(scale),
            _lib.TQ_KV_PACKED, 0,
            k_idx.data_ptr(), k_norms.data_ptr(), v_idx.data_ptr(), v_norms.data_ptr(),
            _lib.torch_dtype_code(k_norms.dtype), key_codec.bits, value_codec.bits,
            kt["codebook"].data_ptr(), vt["codebook"].data_ptr(), key_codec.rot_kind,
            kt["rot"].data_ptr(), vt["rot"].data_ptr(), cap, T)
    tail = (1 if causal else 0, out.data_ptr(), ws.data_ptr(), ws.numel(), _stream(queries))
    _call_attention(lib, head, seq_starts, seq_lens, tail, "tq_attention")
    return out


def _plain_capacity(t: torch.Tensor) -> int:
    """Token capacity of a (B, H, T, D) view of a contiguous (B, H, cap, D) buffer."""
    B, H, T, D = t.shape
    if t.stride(3) != 1 or (T > 1 and t.stride(2) != D):
        raise ValueError("plain K/V views must slice contiguous (B, H, cap, D) buffers")
    if H > 1:
        cap = t.stride(1) // D
    elif B > 1:
        cap = t.stride(0) // D
    else:
        cap = max(T, 1)
    if (H > 1 and t.stride(1) != cap * D) or (B > 1 and t.stride(0) != H * cap * D) or cap < T:
        raise ValueError("plain K/V views must slice contiguous (B, H, cap, D) buffers")
    return cap


def attention_plain(queries: torch.Tensor, keys: torch.Tensor, values: torch.Tensor,
                    scale: float, causal: bool,
                    seq_lens: Optional[torch.Tensor] = None,
                    seq_starts: Optional[torch.Tensor] = None, mask=None,
                    _direct: bool = False) -> torch.Tensor:
    """Attention over unquantized fp16/bf16 K/V views (B, Hkv, T, Dk / Dv) of
    (B, Hkv, cap, D) buffers.

    ``seq_lens`` / ``seq_starts`` as in ``attention_packed``; ``mask`` is an
    array mask broadcast as the fp16 layers' SDPA does (against
    (B, Hq, L, T), base.py:218-226).
    """
    if not _direct and torch.compiler.is_compiling():
        return torch.ops.kaplumba.attention_plain(
            queries, keys, values, float(scale), bool(causal),
            _opt_tensor(seq_lens, torch.int32), _opt_tensor(seq_starts, torch.int32),
            _opt_tensor(mask, None))
    _require_device(queries, keys, values)
    B, Hq, L, D = queries.shape
    Hkv, T = keys.shape[1], keys.shape[2]
    Dv = values.shape[-1]
    if keys.dtype != values.dtype or keys.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("plain K/V must both be float16 or bfloat16")
    if keys.shape[-1] != D:
        raise ValueError(f"query head dim {D} != key head dim {keys.shape[-1]}")
    if values.shape[:3] != keys.shape[:3]:
        raise ValueError("plain keys and values must share (B, H, T)")
    if Hq % Hkv:
        raise ValueError(f"{Hq} query heads are not a multiple of {Hkv} kv heads")
    cap = _plain_capacity(keys)
    if _plain_capacity(values) != cap:
        raise ValueError("plain keys and values must share a capacity")
    if queries.stride(-1) != 1:
        queries = queries.contiguous()
    seq_lens = _seq_array(seq_lens, B, queries.device)
    seq_starts = _seq_array(seq_starts, B, queries.device)
    if mask is not None or Dv != D:
        return _attention_general(
            queries, Dv=Dv, kv_kind=_lib.TQ_KV_PLAIN, kv_dtype=_lib.torch_dtype_code(keys.dtype),
            k=keys, k_norms=None, k_signs=None, k_rnorms=None, k_bits=0, k_codebook=None,
            k_rot_kind=0, k_rot=None, projection=None, v=values, v_norms=None, v_bits=0,
            v_codebook=None, v_rot_kind=0, v_rot=None, norm_dtype=0, cap=cap, T=T, scale=scale,
            causal=causal, mask=mask, seq_lens=seq_lens, seq_starts=seq_starts,
            grouped_mask=False)
    out = torch.empty((B, Hq, L, D), dtype=queries.dtype, device=queries.device)
    lib = _lib.load()
    wsb = lib.tq_attention_workspace_size(B, Hq, Hkv, L, D, T)
    ws = _workspace(queries.device, wsb)
    head = (queries.data_ptr(), _lib.torch_dtype_code(queries.dtype), B, Hq, Hkv, L, D,
            queries.stride(0), queries.stride(1), queries.stride(2), float(scale),
            _lib.TQ_KV_PLAIN, _lib.torch_dtype_code(keys.dtype),
            keys.data_ptr(), None, values.data_ptr(), None, 0, 0, 0, None, None, 0, None, None,
            cap, T)
    tail = (1 if causal else 0, out.data_ptr(), ws.data_ptr(), ws.numel(), _stream(queries))
    _call_attention(lib, head, seq_starts, seq_lens, tail, "tq_attention(plain)")
    return out


# Registers torch.ops.kaplumba.* (they call back into the functions above).
from . import torch_ops  # noqa: E402,F401
