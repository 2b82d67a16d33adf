"""torch-CPU restatement of the reference's array-path attention (TEST ORACLE ONLY).

The same computation as ``tq_oracle.attention_chunked_f32`` -- the f32
chunked online softmax of ``quantized_attention``
(``mlx_lm/models/turboquant_cache.py:5110-5203``, with ``score_prepared``
:4281-4284 and ``weighted_sum`` :4301-4309) -- written with torch tensor ops so
that it runs on every host core (``torch.set_num_threads``).  It serves as
the multi-threaded CPU baseline of the benchmark and is checked against the
numpy oracle in the CPU tests.  Hadamard rotation, packed Beta-codebook
indices, f32 or f16 norms.

Not part of the product: ``kaplumba_amd`` never imports this module.
"""
from __future__ import annotations

import math

import numpy as np
import torch

from . import tq_oracle as O


def unpack_lowbit(packed: torch.Tensor, bits: int, length: int) -> torch.Tensor:
    """LSB-first bit stream -> int64 indices (``_unpack_lowbit`` :3744-3780).

    ``packed`` is int64 holding the u32 words; element i sits at bits
    i*bits .. of the concatenated little-endian words.
    """
    lead = packed.shape[:-1]
    pw = packed.shape[-1]
    # join consecutive word pairs so a field crossing a word boundary is one shift
    nxt = torch.cat([packed[..., 1:], torch.zeros_like(packed[..., :1])], dim=-1)
    wide = packed | (nxt << 32)
    off = torch.arange(length, dtype=torch.int64) * bits
    word = off // 32
    shift = off % 32
    assert int(word.max()) < pw
    sel = wide.index_select(-1, word)
    return ((sel >> shift) & ((1 << bits) - 1)).reshape(*lead, length)


def fwht(x: torch.Tensor) -> torch.Tensor:
    """Unnormalised Walsh-Hadamard transform over the last axis (Sylvester order)."""
    d = x.shape[-1]
    y = x.reshape(-1, d).clone()
    h = 1
    while h < d:
        y = y.view(-1, d // (2 * h), 2, h)
        a, b = y[:, :, 0, :], y[:, :, 1, :]
        y = torch.stack((a + b, a - b), dim=2).reshape(-1, d)
        h *= 2
    return y.reshape(x.shape)


def attention_chunked(q, k_packed, k_norms, v_packed, v_norms, *, k_bits, v_bits, k_codebook,
                      v_codebook, signs_k, signs_v, scale, q_dtype, key_chunk=2048):
    """f32 chunked online-softmax TurboQuant attention, numpy arrays in and out.

    q (B, Hq, L, D) float; packed (B, Hkv, T, PW) u32; norms (B, Hkv, T).
    Non-causal (decode); returns float32 (B, Hq, L, D).
    """
    B, Hq, L, D = q.shape
    Hkv = k_packed.shape[1]
    R = Hq // Hkv
    T = k_packed.shape[2]
    rs = float(O.rht_scale(D))
    qs = torch.from_numpy(O.scale_queries(q, scale, q_dtype)).reshape(B, Hkv, R * L, D)
    sk = torch.from_numpy(np.asarray(signs_k, np.float32))
    sv = torch.from_numpy(np.asarray(signs_v, np.float32))
    qr = fwht(qs * sk) * rs
    kc = torch.from_numpy(np.asarray(k_codebook, np.float32))
    vc = torch.from_numpy(np.asarray(v_codebook, np.float32))
    kp = torch.from_numpy(np.asarray(k_packed, np.uint32).astype(np.int64))
    vp = torch.from_numpy(np.asarray(v_packed, np.uint32).astype(np.int64))
    kn = torch.from_numpy(np.asarray(k_norms, np.float32))
    vn = torch.from_numpy(np.asarray(v_norms, np.float32))
    out = torch.zeros(B, Hkv, R * L, D)
    den = torch.zeros(B, Hkv, R * L)
    mx = torch.full((B, Hkv, R * L), -math.inf)
    for k0 in range(0, T, key_chunk):
        k1 = min(T, k0 + key_chunk)
        kd = kc[unpack_lowbit(kp[:, :, k0:k1], k_bits, D)]              # (B, Hkv, t, D)
        s = torch.matmul(qr, kd.transpose(-1, -2)) * kn[:, :, None, k0:k1]
        cm = s.amax(dim=-1)
        w = torch.exp(s - cm[..., None])
        vd = vc[unpack_lowbit(vp[:, :, k0:k1], v_bits, D)] * vn[:, :, k0:k1, None]
        co = torch.matmul(w, vd)
        co = sv * (fwht(co) * rs)
        nm = torch.maximum(mx, cm)
        ps = torch.exp(mx - nm)
        cs = torch.exp(cm - nm)
        out = out * ps[..., None] + co * cs[..., None]
        den = den * ps + w.sum(dim=-1) * cs
        mx = nm
    res = out / torch.clamp(den[..., None], min=float(O.EPS))
    return res.reshape(B, Hq, L, D).numpy()
