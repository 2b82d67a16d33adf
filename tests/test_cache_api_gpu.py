"""The reference's TurboQuant cache API tests, restated in torch on the GPU.

Mirrors tests/test_turboquant.py:152-487 and :683-746 of the reference (same
shapes and assertions), plus a harness that replays the generate loop's call
order (per layer: update_and_fetch then scaled_dot_product_attention, prefill
chunk, decode steps, trim and re-append) and checks the result against the
oracle.
"""
import math
import os
import tempfile

import numpy as np
import pytest
import torch

from oracle import tq_oracle as O
from kaplumba_amd import (KVCache, TurboQuantKVCache, create_attention_mask, create_causal_mask,
                          load_prompt_cache, make_prompt_cache, save_prompt_cache,
                          scaled_dot_product_attention, trim_prompt_cache)

pytestmark = pytest.mark.gpu


def randn(*shape, device):
    return torch.randn(*shape, device=device)


def test_single_update(device):
    cache = TurboQuantKVCache(bits=3)
    B, H, S, D = 1, 8, 10, 64
    k_ret, v_ret = cache.update_and_fetch(randn(B, H, S, D, device=device), randn(B, H, S, D, device=device))
    assert cache.offset == 10 and cache.size() == 10 and not cache.empty()
    assert k_ret.shape == (B, H, 10, D) and v_ret.shape == (B, H, 10, D)


def test_sequential_updates(device):
    cache = TurboQuantKVCache(bits=3)
    B, H, D = 1, 8, 64
    k_ret, _ = cache.update_and_fetch(randn(B, H, 20, D, device=device), randn(B, H, 20, D, device=device))
    assert cache.offset == 20 and k_ret.shape == (B, H, 20, D)
    for i in range(5):
        k_ret, v_ret = cache.update_and_fetch(randn(B, H, 1, D, device=device), randn(B, H, 1, D, device=device))
        assert cache.offset == 21 + i
        assert k_ret.shape == (B, H, 21 + i, D) and v_ret.shape == (B, H, 21 + i, D)


def test_asymmetric_kv_dims(device):
    cache = TurboQuantKVCache(bits=3)
    k_ret, v_ret = cache.update_and_fetch(randn(1, 4, 5, 128, device=device), randn(1, 4, 5, 64, device=device))
    assert k_ret.shape == (1, 4, 5, 128) and v_ret.shape == (1, 4, 5, 64)


@pytest.mark.parametrize("bits", [1, 2, 3, 4, 2.5, 3.5])
def test_different_bit_widths(device, bits):
    cache = TurboQuantKVCache(bits=bits)
    k_ret, _ = cache.update_and_fetch(randn(1, 4, 8, 64, device=device), randn(1, 4, 8, 64, device=device))
    assert cache.offset == 8 and k_ret.shape == (1, 4, 8, 64)
    assert cache.key_codec.bits == math.floor(bits) and cache.value_codec.bits == math.ceil(bits)


def test_quantization_quality(device):
    cache = TurboQuantKVCache(bits=3)
    k = randn(1, 4, 16, 128, device=device)
    k_ret, v_ret = cache.update_and_fetch(k, randn(1, 4, 16, 128, device=device))
    dq_k, _ = cache.dequantize(k_ret._state, v_ret._state)
    kf, rf = k.reshape(-1, 128), dq_k.reshape(-1, 128)
    cos = ((kf * rf).sum(-1) / (kf.norm(dim=-1) * rf.norm(dim=-1) + 1e-10)).mean().item()
    assert cos > 0.85


def test_compression_ratio(device):
    for norm_dtype, want in ((torch.float16, 5.12), (torch.float32, 4.92)):
        cache = TurboQuantKVCache(bits=3, norm_dtype=norm_dtype)
        B, H, S, D = 1, 8, 100, 128
        cache.update_and_fetch(randn(B, H, S, D, device=device), randn(B, H, S, D, device=device))
        ratio = (2 * B * H * S * D * 2) / cache.nbytes
        assert ratio > 3.0 and abs(ratio - want) < 0.01


def test_trim_and_trim_past_end(device):
    cache = TurboQuantKVCache(bits=3)
    cache.update_and_fetch(randn(1, 4, 20, 64, device=device), randn(1, 4, 20, 64, device=device))
    assert cache.trim(5) == 5 and cache.offset == 15 and cache.size() == 15
    assert cache.trim(100) == 15 and cache.offset == 0
    assert cache.is_trimmable()


def test_state_roundtrip_and_meta(device):
    cache = TurboQuantKVCache(bits=3, seed=99)
    assert cache.state == []
    cache.update_and_fetch(randn(1, 4, 10, 64, device=device), randn(1, 4, 10, 128, device=device))
    ks, vs = cache.state
    assert ks.norms.shape[2] == 10 and vs.norms.shape[2] == 10
    meta = cache.meta_state
    # the reference's five fields, then the codec options
    assert len(meta) == 10 and int(float(meta[0])) == 10 and float(meta[1]) == 3.0
    assert int(float(meta[2])) == 99 and int(meta[3]) == 64 and int(meta[4]) == 128
    assert meta[5:] == ("mse", "3", "3", "auto", "beta")
    new = TurboQuantKVCache(bits=3)
    new.state = cache.state
    new.meta_state = meta
    assert new.offset == cache.offset and new.quant_bits == 3 and new.seed == 99
    restored = TurboQuantKVCache.from_state(cache.state, cache.meta_state)
    assert restored.offset == 10 and restored.quant_bits == 3 and restored.seed == 99


def test_make_mask_with_offset(device):
    cache = TurboQuantKVCache(bits=3)
    S, N = 20, 4
    cache.update_and_fetch(randn(1, 4, S, 64, device=device), randn(1, 4, S, 64, device=device))
    mask = create_attention_mask(torch.zeros(1, N, 64), cache=cache, return_array=True)
    assert mask.shape == (N, S + N)
    assert torch.equal(mask, create_causal_mask(N, offset=S))


def test_trim_then_update_and_incremental_consistency(device):
    cache = TurboQuantKVCache(bits=3)
    k_full, v_full = cache.update_and_fetch(randn(1, 4, 20, 64, device=device), randn(1, 4, 20, 64, device=device))
    dq_full = cache.dequantize(k_full._state, v_full._state)
    dq_full = (dq_full[0].clone(), dq_full[1].clone())
    for _ in range(5):
        cache.update_and_fetch(randn(1, 4, 1, 64, device=device), randn(1, 4, 1, 64, device=device))
    assert cache.offset == 25 and cache.trim(5) == 5 and cache.offset == 20
    k_ret, v_ret = cache.update_and_fetch(randn(1, 4, 3, 64, device=device), randn(1, 4, 3, 64, device=device))
    assert cache.offset == 23 and k_ret.shape == (1, 4, 23, 64)
    dq_inc = cache.dequantize(k_ret._state, v_ret._state)
    assert torch.allclose(dq_full[0], dq_inc[0][..., :20, :], atol=1e-5)
    assert torch.allclose(dq_full[1], dq_inc[1][..., :20, :], atol=1e-5)


def test_conversion_from_kvcache(device):
    kv = KVCache()
    tq = kv.to_turbo_quantized(bits=3)
    assert isinstance(tq, TurboQuantKVCache) and tq.empty() and tq.offset == 0
    kv.update_and_fetch(randn(1, 4, 16, 128, device=device).half(), randn(1, 4, 16, 128, device=device).half())
    for bits in (1, 2, 3, 4):
        t = kv.to_turbo_quantized(bits=bits)
        assert t.quant_bits == bits and t.offset == 16
    t = kv.to_turbo_quantized(bits=4)
    k_ret, _ = t.update_and_fetch(randn(1, 4, 1, 128, device=device), randn(1, 4, 1, 128, device=device))
    assert k_ret.shape == (1, 4, 17, 128) and t.offset == 17
    t2 = TurboQuantKVCache.from_cache(kv, bits=3)
    assert t2.offset == 16


def test_save_load_mixed_cache(device):
    cache = [KVCache(), TurboQuantKVCache(bits=3), TurboQuantKVCache(bits=3), KVCache()]
    for c in cache:
        c.update_and_fetch(randn(1, 4, 10, 64, device=device).half(), randn(1, 4, 10, 64, device=device).half())
    with tempfile.TemporaryDirectory() as d:
        f = os.path.join(d, "mixed.safetensors")
        save_prompt_cache(f, cache, {"model": "test", "version": "1"})
        loaded, meta = load_prompt_cache(f, return_metadata=True)
    assert meta == {"model": "test", "version": "1"}
    assert [type(c).__name__ for c in loaded] == ["KVCache", "TurboQuantKVCache", "TurboQuantKVCache", "KVCache"]
    for c, lc in zip(cache, loaded):
        assert c.offset == lc.offset
    # a loaded TurboQuant layer attends without a warm-up append (dims come from meta_state)
    q = randn(1, 8, 1, 64, device=device).to(torch.bfloat16)
    a = cache[1].decode_attention(q, scale=0.125)
    b = loaded[1].decode_attention(q, scale=0.125)
    assert torch.equal(a, b)


def test_generate_loop_replay_matches_oracle(device):
    """Per layer: update_and_fetch then SDPA, over prefill, decode, trim, re-append."""
    n_layers, B, Hq, Hkv, D = 6, 1, 8, 2, 128
    caches = make_prompt_cache(num_layers=n_layers, turbo_kv_bits=3, turbo_fp16_layers=1)
    assert [type(c).__name__ for c in caches] == ["KVCache"] + ["TurboQuantKVCache"] * 4 + ["KVCache"]
    g = torch.Generator(device="cpu").manual_seed(0)
    hist_k = [[] for _ in range(n_layers)]
    hist_v = [[] for _ in range(n_layers)]

    def step(L):
        outs = []
        for i, c in enumerate(caches):
            k = torch.randn(B, Hkv, L, D, generator=g).to(torch.bfloat16)
            v = torch.randn(B, Hkv, L, D, generator=g).to(torch.bfloat16)
            q = torch.randn(B, Hq, L, D, generator=g).to(torch.bfloat16)
            hist_k[i].append(k)
            hist_v[i].append(v)
            mask = c.make_mask(L)
            ks, vs = c.update_and_fetch(k.to(device), v.to(device))
            outs.append((q, scaled_dot_product_attention(q.to(device), ks, vs, c, 1 / math.sqrt(D), mask), mask))
        return outs

    step(64)            # prefill chunk
    for _ in range(3):  # decode
        step(1)
    trim_prompt_cache(caches, 2)
    for i in range(n_layers):
        # drop the trimmed tokens from the host history too
        kk = torch.cat(hist_k[i], dim=2)[:, :, :-2]
        vv = torch.cat(hist_v[i], dim=2)[:, :, :-2]
        hist_k[i], hist_v[i] = [kk], [vv]
    outs = step(4)      # MTP-style verify chunk, causal
    for i, (q, out, mask) in enumerate(outs):
        k = torch.cat(hist_k[i], dim=2).float().numpy()
        v = torch.cat(hist_v[i], dim=2).float().numpy()
        qn = q.float().numpy()
        if isinstance(caches[i], TurboQuantKVCache):
            kp, kn = O.quantize_rht(k, 3, O.rht_signs(D, 0), O.beta_codebook(D, 3))
            vp, vn = O.quantize_rht(v, 3, O.rht_signs(D, 1), O.beta_codebook(D, 3))
            want = O.attention(qn, kp, kn, vp, vn, k_bits=3, v_bits=3, k_codebook=O.beta_codebook(D, 3),
                               v_codebook=O.beta_codebook(D, 3), rot_kind="hadamard",
                               k_rot=O.rht_signs(D, 0), v_rot=O.rht_signs(D, 1),
                               scale=1 / math.sqrt(D), q_dtype="bf16", causal=True)
            st = caches[i].state
            assert np.array_equal(st[0].indices.cpu().numpy().astype(np.uint32), kp)
        else:
            want = O.attention_plain(qn, k, v, scale=1 / math.sqrt(D), q_dtype="bf16", causal=True)
        from tests.test_attention_gpu import assert_close

        assert_close(out, want, "bf16", f"layer {i}")


@pytest.mark.parametrize("d", [128, 256])
def test_dense_rotation_cache_end_to_end(device, d):
    """rotation="dense": matrix-core append, then decode and verify through the cache API."""
    from tests.test_append_dense_gpu import BAND
    from tests.test_attention_gpu import assert_close

    B, Hq, Hkv = 2, 8, 4
    g = torch.Generator(device="cpu").manual_seed(d)
    k = torch.randn(B, Hkv, 600, d, generator=g).to(torch.bfloat16)
    v = torch.randn(B, Hkv, 600, d, generator=g).to(torch.bfloat16)
    cache = TurboQuantKVCache(bits=3.5, rotation="dense")     # K 3-bit, V 4-bit
    cache.update_and_fetch(k[:, :, :597].to(device), v[:, :, :597].to(device))
    ks, vs = cache.update_and_fetch(k[:, :, 597:].to(device), v[:, :, 597:].to(device))
    kr, vr = O.rotation_matrix(d, 0), O.rotation_matrix(d, 1)
    kcb, vcb = O.beta_codebook(d, 3), O.beta_codebook(d, 4)
    kp, kn, ky = O.quantize_dense(k.float().numpy(), 3, kr, kcb)
    vp, vn, vy = O.quantize_dense(v.float().numpy(), 4, vr, vcb)
    st = cache.state
    assert np.array_equal(st[0].norms.cpu().numpy(), kn)
    assert np.array_equal(st[1].norms.cpu().numpy(), vn)
    for got, want, y, bits, cb in ((st[0].indices, kp, ky, 3, kcb), (st[1].indices, vp, vy, 4, vcb)):
        gi = O.unpack_lowbit(got.cpu().numpy().astype(np.uint32), bits, d).astype(np.int64)
        wi = O.unpack_lowbit(want, bits, d).astype(np.int64)
        bad = gi != wi
        if bad.any():
            dist = np.abs(y[bad][:, None].astype(np.float64) - O.midpoints(cb)[None, :]).min(axis=1)
            assert dist.max() <= BAND
        # flips are rare: at most 8 per 8.4M coordinates on a full config-3 layer
        assert int(bad.sum()) <= 4, f"{int(bad.sum())} index flips in {bad.size} coordinates"
    # attention over the cache's own packed state (decode, then a causal verify of 3 rows)
    gp = [s_.indices.cpu().numpy().astype(np.uint32) for s_ in st]
    for L in (1, 3):
        q = torch.randn(B, Hq, L, d, generator=g).to(torch.bfloat16)
        mask = "causal" if L > 1 else None
        out = scaled_dot_product_attention(q.to(device), ks, vs, cache, 1 / math.sqrt(d), mask)
        want = O.attention(q.float().numpy(), gp[0], kn, gp[1], vn, k_bits=3, v_bits=4,
                           k_codebook=kcb, v_codebook=vcb, rot_kind="dense", k_rot=kr, v_rot=vr,
                           scale=1 / math.sqrt(d), q_dtype="bf16", causal=L > 1)
        assert_close(out, want, "bf16", f"dense cache d{d} L{L}")
