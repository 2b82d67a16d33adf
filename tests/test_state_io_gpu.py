"""Saved caches reload with their own codecs, checked against the oracle.

A prompt-cache file (save_prompt_cache / load_prompt_cache, models/cache.py:
71-153) holds each layer's packed state and its meta_state strings.  The
reference's meta_state keeps offset, bits and seed (turboquant_cache.py:
6046-6056); this library appends the codec options, so a cache built with a
dense rotation, the Gaussian codebook or per-side widths decodes with those
codecs after a reload.  Each loaded cache's attention is compared with the
oracle over the saved packed rows, using the codecs the cache was built with:
a reload that picked other codecs (Hadamard instead of dense, Beta instead of
Gaussian, 3/3 instead of 4/2 bits) fails the comparison or the width check.
"""
import math
import os
import tempfile

import numpy as np
import pytest
import torch

from oracle import tq_oracle as O
from kaplumba_amd import (BatchTurboQuantKVCache, TurboQuantKVCache, load_prompt_cache,
                          save_prompt_cache, scaled_dot_product_attention)
from tests.test_attention_gpu import assert_close

pytestmark = pytest.mark.gpu


def _reload(caches):
    with tempfile.TemporaryDirectory() as d:
        f = os.path.join(d, "c.safetensors")
        save_prompt_cache(f, caches)
        return load_prompt_cache(f)


def _codebook(kind, d, bits):
    return O.beta_codebook(d, bits) if kind == "beta" else O.gaussian_codebook(d, bits)


def _rot(kind, d, seed):
    return O.rht_signs(d, seed) if kind == "hadamard" else O.rotation_matrix(d, seed)


@pytest.mark.parametrize("d,opts,kb,vb,rot,cbk", [
    (256, dict(bits=3, rotation="dense", key_bits=4, val_bits=2), 4, 2, "dense", "beta"),
    (128, dict(bits=3, codebook="gaussian"), 3, 3, "hadamard", "gaussian"),
    (128, dict(bits=2.5, rotation="dense", codebook="gaussian"), 2, 3, "dense", "gaussian"),
])
def test_reloaded_cache_decodes_with_its_codecs(device, d, opts, kb, vb, rot, cbk):
    B, Hq, Hkv, T = 1, 8, 2, 333
    g = torch.Generator().manual_seed(d + kb)
    k = torch.randn(B, Hkv, T, d, generator=g).to(torch.bfloat16)
    v = torch.randn(B, Hkv, T, d, generator=g).to(torch.bfloat16)
    cache = TurboQuantKVCache(seed=3, **opts)
    cache.update_and_fetch(k.to(device), v.to(device))
    (loaded,) = _reload([cache])
    assert loaded.meta_state == cache.meta_state
    st = loaded.state
    kp = st[0].indices.cpu().numpy().astype(np.uint32)
    vp = st[1].indices.cpu().numpy().astype(np.uint32)
    assert kp.shape[-1] == O.packed_width(d, kb) and vp.shape[-1] == O.packed_width(d, vb)
    assert np.array_equal(kp, cache.state[0].indices.cpu().numpy().astype(np.uint32))
    for L in (1, 4):
        q = torch.randn(B, Hq, L, d, generator=g).to(torch.bfloat16)
        out = scaled_dot_product_attention(q.to(device), st[0], st[1], loaded, 1 / math.sqrt(d),
                                           "causal" if L > 1 else None)
        want = O.attention(q.float().numpy(), kp, st[0].norms.cpu().numpy(), vp,
                           st[1].norms.cpu().numpy(), k_bits=kb, v_bits=vb,
                           k_codebook=_codebook(cbk, d, kb), v_codebook=_codebook(cbk, d, vb),
                           rot_kind=rot, k_rot=_rot(rot, d, 3), v_rot=_rot(rot, d, 4),
                           scale=1 / math.sqrt(d), q_dtype="bf16", causal=L > 1)
        assert_close(out, want, "bf16", f"reloaded d{d} {opts} L{L}")
    # the reloaded cache keeps appending with the same codecs: the new rows are
    # the ones the original cache writes for the same tokens
    k2 = torch.randn(B, Hkv, 5, d, generator=g).to(torch.bfloat16)
    v2 = torch.randn(B, Hkv, 5, d, generator=g).to(torch.bfloat16)
    cache.update_and_fetch(k2.to(device), v2.to(device))
    loaded.update_and_fetch(k2.to(device), v2.to(device))
    for a, b in zip(cache.state, loaded.state):
        assert torch.equal(a.indices, b.indices) and torch.equal(a.norms, b.norms)


def test_reloaded_batch_cache_decodes_with_its_codecs(device):
    d, Hq, Hkv = 128, 8, 2
    lp = [3, 0]
    g = torch.Generator().manual_seed(11)
    L0 = 40
    k = torch.randn(2, Hkv, L0, d, generator=g).to(torch.bfloat16)
    v = torch.randn(2, Hkv, L0, d, generator=g).to(torch.bfloat16)
    cache = BatchTurboQuantKVCache(lp, bits=3, seed=5, rotation="dense", codebook="gaussian",
                                   key_bits=4, val_bits=2)
    cache.update_and_fetch(k.to(device), v.to(device))
    (loaded,) = _reload([cache])
    assert loaded.meta_state == cache.meta_state
    assert loaded.left_padding.tolist() == lp
    q = torch.randn(2, Hq, 1, d, generator=g).to(torch.bfloat16)
    ks, vs = loaded.state[:2]
    out = loaded.decode_attention(q.to(device), scale=1 / math.sqrt(d))
    kp = ks.indices.cpu().numpy().astype(np.uint32)
    vp = vs.indices.cpu().numpy().astype(np.uint32)
    assert kp.shape[-1] == O.packed_width(d, 4) and vp.shape[-1] == O.packed_width(d, 2)
    want = O.attention(q.float().numpy(), kp, ks.norms.cpu().numpy(), vp, vs.norms.cpu().numpy(),
                       k_bits=4, v_bits=2, k_codebook=O.gaussian_codebook(d, 4),
                       v_codebook=O.gaussian_codebook(d, 2), rot_kind="dense",
                       k_rot=O.rotation_matrix(d, 5), v_rot=O.rotation_matrix(d, 6),
                       scale=1 / math.sqrt(d), q_dtype="bf16", starts=lp)
    assert_close(out, want, "bf16", "reloaded batch cache")
