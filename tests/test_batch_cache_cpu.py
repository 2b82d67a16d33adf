"""Continuous-batching caches on the CPU: bookkeeping, filter/extend, masks,
state round trips, and the oracle's left-padding form.

Host logic only (no kernel runs): states are set directly with synthetic
tensors.  The reference's BatchTurboQuantKVCache (turboquant_cache.py:
6082-6309) and BatchKVCache (models/cache.py:1099-1315) define the
semantics; each check below is a property those define (a row keeps its own
tokens in order through filter and extend, the shared padding is dropped,
rows right-align at the longer length), not a restatement of the code.
"""
import os
import tempfile

import numpy as np
import pytest
import torch

from oracle import tq_oracle as O
from kaplumba_amd import (BatchKVCache, BatchTurboQuantKVCache, KVCache, TurboQuantMSEState,
                          create_causal_mask, load_prompt_cache, save_prompt_cache)

H, PW, D = 2, 12, 128


def synth_tq(left_padding, idx, seed=0):
    """A BatchTurboQuantKVCache holding synthetic rows: token t of row b has
    norm 1000 b + t + 1 (0 in the padding) and indices filled with that value."""
    c = BatchTurboQuantKVCache(left_padding, bits=3)
    B = len(left_padding)
    norms = torch.zeros((B, H, idx), dtype=torch.float32)
    ind = torch.zeros((B, H, idx, PW), dtype=torch.int64)
    for b, lp in enumerate(left_padding):
        for t in range(lp, idx):
            norms[b, :, t] = 1000 * (b + seed * 100) + t + 1
            ind[b, :, t, :] = 1000 * (b + seed * 100) + t + 1
    st = (TurboQuantMSEState(norms, ind.to(torch.uint32)),
          TurboQuantMSEState(norms.clone() * 2, ind.to(torch.uint32)),
          torch.tensor([idx - lp for lp in left_padding]), torch.tensor(left_padding))
    c.state = st
    c.meta_state = (str(idx), "3.0", "0", str(D), str(D))
    return c


def rows_tokens(c):
    """Per row, the list of token labels in [left_padding, _idx)."""
    k = c.state[0]
    out = []
    for b, lp in enumerate(c.left_padding.tolist()):
        lab = k.norms[b, 0, lp:c._idx].tolist()
        assert torch.equal(k.indices[b, 0, lp:c._idx, 0].to(torch.int64),
                           torch.tensor(lab).to(torch.int64))
        assert float(k.norms[b, :, :lp].abs().sum()) == 0.0  # padding holds zeros
        out.append(lab)
    return out


def test_construction_and_protocol():
    c = BatchTurboQuantKVCache([1, 3, 0], bits=3.5)
    assert c.bits == 3.5 and c.seed == 0
    assert c.left_padding.tolist() == [1, 3, 0] and c.offset.tolist() == [-1, -3, 0]
    assert c._idx == 0 and c.empty() and not c.is_trimmable() and c.trim(5) == 0
    assert c.nbytes == 0 and c.group_size == 64
    assert c.state[0] is None and c.state[1] is None
    assert c.meta_state[:3] == ("0", "3.5", "0")
    assert c.make_mask(1) is None and c.make_mask(4) == "causal"
    with pytest.raises(ValueError):
        BatchTurboQuantKVCache([0], bits=0.5)
    with pytest.raises(ValueError):
        BatchTurboQuantKVCache([0], bits=3, rotation="nope")


def test_array_mask_has_left_padding_and_causality():
    c = synth_tq([2, 0], 5)
    m = c.make_mask(3, return_array=True)
    assert m.shape == (2, 1, 3, 8)
    for b, lp in enumerate([2, 0]):
        for i in range(3):
            for k in range(8):
                assert bool(m[b, 0, i, k]) == (lp <= k <= 5 + i)
    # the generic helper with right padding: keys at or past offset+N-rp are cut
    m2 = create_causal_mask(2, offset=3, right_padding=torch.tensor([1, 0]))
    assert m2.shape == (2, 1, 2, 5)
    assert not bool(m2[0, 0, 1, 4]) and bool(m2[1, 0, 1, 4])


def test_filter_keeps_rows_and_drops_shared_padding():
    c = synth_tq([3, 1, 4, 2], 9)
    before = rows_tokens(c)
    off = c.offset.clone()
    c.filter([2, 0])
    assert c.left_padding.min().item() == 0
    assert c._idx == 9 - 3
    assert c.offset.tolist() == [off[2].item(), off[0].item()]
    assert rows_tokens(c) == [before[2], before[0]]
    assert c.state[0].norms.shape[2] == c._idx
    # capacity is a whole number of cache steps and contiguous for the kernels
    assert c.keys.norms.shape[2] % 256 == 0 and c.keys.indices.is_contiguous()


def test_filter_on_empty_cache_keeps_padding():
    c = BatchTurboQuantKVCache([2, 5], bits=3)
    c.filter([1])
    assert c.left_padding.tolist() == [5] and c._idx == 0 and c.empty()


@pytest.mark.parametrize("a,b", [((5, [1, 0]), (8, [0, 3, 2])), ((8, [2]), (3, [0, 1]))])
def test_extend_right_aligns_both_sides(a, b):
    ca = synth_tq(a[1], a[0], seed=0)
    cb = synth_tq(b[1], b[0], seed=1)
    ra, rb = rows_tokens(ca), rows_tokens(cb)
    offs = ca.offset.tolist() + cb.offset.tolist()
    ca.extend(cb)
    assert ca._idx == max(a[0], b[0])
    assert ca.offset.tolist() == offs
    assert rows_tokens(ca) == ra + rb
    assert ca.left_padding.numel() == len(a[1]) + len(b[1])


def test_extend_with_an_empty_side():
    ca = synth_tq([0, 2], 6)
    ra = rows_tokens(ca)
    cb = BatchTurboQuantKVCache([1], bits=3)
    ca.extend(cb)
    assert ca._idx == 6 and ca.left_padding.tolist() == [0, 2, 7]
    assert rows_tokens(ca)[:2] == ra
    e1, e2 = BatchTurboQuantKVCache([1], bits=3), BatchTurboQuantKVCache([0, 2], bits=3)
    e1.extend(e2)
    assert e1.left_padding.tolist() == [1, 0, 2] and e1.empty()


def test_extend_rejects_mismatched_codecs():
    ca = synth_tq([0], 4)
    cb = synth_tq([0], 4)
    cb.bits = 2.0
    cb.key_codec = cb.value_codec = None
    with pytest.raises(ValueError):
        ca.extend(cb)


def test_extend_rejects_mismatched_codebooks():
    """Rows coded with another codebook would decode wrongly after a merge."""
    ca = synth_tq([0], 4)
    cb = synth_tq([0], 4)
    cb._turbo_kwargs["codebook"] = "gaussian"
    cb.key_codec = cb.value_codec = None
    with pytest.raises(ValueError):
        ca.extend(cb)
    with pytest.raises(ValueError):
        BatchTurboQuantKVCache([0], bits=3, key_quantizer="prod")


def test_save_load_keeps_codec_options_batch():
    c = BatchTurboQuantKVCache([1, 0], bits=3, rotation="dense", codebook="gaussian",
                               key_bits=4, val_bits=2)
    g = torch.Generator().manual_seed(3)
    mk = lambda pw: TurboQuantMSEState(torch.rand(2, H, 5, generator=g),
                                       torch.randint(0, 1 << 30, (2, H, 5, pw), generator=g).to(torch.uint32))
    c.state = (mk(32), mk(16), torch.tensor([4, 5]), torch.tensor([1, 0]))
    c.meta_state = ("5", "3.0", "0", "256", "256")  # dims only: the options stay
    with tempfile.TemporaryDirectory() as td:
        f = os.path.join(td, "c.safetensors")
        save_prompt_cache(f, [c])
        (r,) = load_prompt_cache(f, device="cpu")
    assert r.meta_state == c.meta_state
    r._codecs_ready()
    assert (r.key_codec.bits, r.value_codec.bits) == (4, 2)
    assert r.key_codec.rotation == "dense" and r.value_codec.codebook_kind == "gaussian"
    assert r.key_codec.packed_width == r.state[0].indices.shape[-1]


def test_save_load_round_trip_cpu():
    c = synth_tq([1, 0], 5)
    e = BatchTurboQuantKVCache([3], bits=3)
    p = BatchKVCache([0, 2])
    p.state = (torch.randn(2, H, 4, D).half(), torch.randn(2, H, 4, D).half(),
               torch.tensor([4, 2]), torch.tensor([0, 2]))
    with tempfile.TemporaryDirectory() as td:
        f = os.path.join(td, "c.safetensors")
        save_prompt_cache(f, [c, e, p])
        got = load_prompt_cache(f, device="cpu")
    assert [type(x).__name__ for x in got] == ["BatchTurboQuantKVCache", "BatchTurboQuantKVCache",
                                               "BatchKVCache"]
    g = got[0]
    assert g._idx == 5 and g.left_padding.tolist() == [1, 0] and g.offset.tolist() == [4, 5]
    assert g._dims == (D, D) and g.bits == 3.0
    for s_new, s_old in zip(g.state[:2], c.state[:2]):
        assert torch.equal(s_new.norms, s_old.norms) and torch.equal(s_new.indices, s_old.indices)
    assert got[1].empty() and got[1].left_padding.tolist() == [3]
    assert torch.equal(got[2].state[0], p.state[0]) and got[2].left_padding.tolist() == [0, 2]


def synth_plain(left_padding, idx, seed=0):
    B = len(left_padding)
    k = torch.zeros((B, H, idx, D), dtype=torch.float16)
    for b, lp in enumerate(left_padding):
        for t in range(lp, idx):
            k[b, :, t, :] = (b + 10 * seed) * 64 + t + 1
    c = BatchKVCache(left_padding)
    c.state = (k, k.clone() * 2, torch.tensor([idx - lp for lp in left_padding]),
               torch.tensor(left_padding))
    return c


def plain_rows(c):
    k, _, _, lp = c.state
    return [k[b, 0, int(l):c._idx, 0].tolist() for b, l in enumerate(lp.tolist())]


def test_batch_kv_filter_extend_extract_merge_trim():
    c = synth_plain([2, 0, 1], 6)
    rows = plain_rows(c)
    c.filter([0, 2])
    assert c.left_padding.tolist() == [1, 0] and c._idx == 5
    assert plain_rows(c) == [rows[0], rows[2]]
    d = synth_plain([0], 9, seed=1)
    rd = plain_rows(d)
    c.extend(d)
    assert c._idx == 9 and plain_rows(c) == [rows[0], rows[2]] + rd
    one = c.extract(1)
    assert isinstance(one, KVCache) and one.offset == len(rows[2])
    assert one.keys[0, 0, :, 0].tolist() == rows[2]
    m = BatchKVCache.merge([one, c.extract(2)])
    assert m.left_padding.tolist() == [9 - len(rows[2]), 0] and m._idx == 9
    assert plain_rows(m) == [rows[2]] + rd
    assert m.trim(2) == 2 and m._idx == 7 and m.offset.tolist() == [len(rows[2]) - 2, 7]


def test_batch_kv_finalize_moves_right_padding_left():
    # rows right-padded during a batched prefill: row 0 has 2 real tokens and
    # 2 padding tokens after them, row 1 has 4 real tokens
    c = BatchKVCache([0, 0])
    c.prepare(right_padding=[2, 0])
    k = torch.zeros((2, H, 4, D), dtype=torch.float16)
    k[0, :, :2] = torch.tensor([5.0, 6.0])[None, :, None]
    k[1, :, :4] = torch.tensor([1.0, 2.0, 3.0, 4.0])[None, :, None]
    c.state = (k, k.clone(), torch.tensor([4, 4]), torch.tensor([0, 0]))
    c._right_padding = torch.tensor([2, 0])
    c.finalize()
    assert c.left_padding.tolist() == [2, 0] and c.offset.tolist() == [2, 4]
    assert plain_rows(c) == [[5.0, 6.0], [1.0, 2.0, 3.0, 4.0]]
    with pytest.raises(ValueError):
        c.prepare(left_padding=[1, 1])


def _random_packed(rng, B, Hkv, T, d, bits):
    idx = rng.integers(0, 1 << bits, size=(B, Hkv, T, d))
    return O.pack_lowbit(idx, bits), rng.uniform(0.5, 2.0, size=(B, Hkv, T)).astype(np.float32)


def test_oracle_left_padding_is_the_sliced_problem():
    """starts[b] removes the first starts[b] tokens of row b: the same as the
    oracle over the row's slice, whatever the padding rows hold."""
    rng = np.random.default_rng(5)
    B, Hq, Hkv, L, T, d = 3, 4, 2, 3, 40, 64
    kp, kn = _random_packed(rng, B, Hkv, T, d, 3)
    vp, vn = _random_packed(rng, B, Hkv, T, d, 2)
    q = rng.standard_normal((B, Hq, L, d)).astype(np.float32)
    starts, lens = [5, 0, 39], [40, 33, 40]
    kw = dict(k_bits=3, v_bits=2, k_codebook=O.beta_codebook(d, 3), v_codebook=O.beta_codebook(d, 2),
              rot_kind="hadamard", k_rot=O.rht_signs(d, 0), v_rot=O.rht_signs(d, 1), scale=0.125,
              q_dtype="f32", causal=True)
    got = O.attention(q, kp, kn, vp, vn, lengths=lens, starts=starts, **kw)
    for b in range(B):
        s, e = starts[b], lens[b]
        want = O.attention(q[b:b + 1], kp[b:b + 1, :, s:e], kn[b:b + 1, :, s:e], vp[b:b + 1, :, s:e],
                           vn[b:b + 1, :, s:e], **kw)
        np.testing.assert_array_equal(got[b:b + 1], want)
    # garbage in the padding changes nothing
    kp2, kn2 = kp.copy(), kn.copy()
    kp2[0, :, :5] ^= 0x5A5A5A5A
    kn2[0, :, :5] = 1e30
    np.testing.assert_array_equal(O.attention(q, kp2, kn2, vp, vn, lengths=lens, starts=starts, **kw), got)


def test_oracle_left_padding_matches_the_array_mask_form():
    """Left padding as the boolean mask BatchKVCache.make_mask builds
    (keys >= left_padding, causal from the end) applied to a plain float64
    softmax over the whole padded row: equal for every query row that sees a
    key."""
    rng = np.random.default_rng(9)
    B, Hq, Hkv, L, T, d = 2, 2, 1, 4, 24, 64
    k = rng.standard_normal((B, Hkv, T, d)).astype(np.float32)
    v = rng.standard_normal((B, Hkv, T, d)).astype(np.float32)
    q = rng.standard_normal((B, Hq, L, d)).astype(np.float32)
    starts = [3, 22]
    got = O.attention_plain(q, k, v, scale=0.2, q_dtype="f32", causal=True, starts=starts)
    mask = create_causal_mask(L, offset=T - L, left_padding=torch.tensor(starts)).numpy()
    qs = O.scale_queries(q, 0.2, "f32").astype(np.float64)
    for b in range(B):
        for h in range(Hq):
            s = qs[b, h] @ k[b, 0].astype(np.float64).T
            for i in range(L):
                vis = mask[b, 0, i]
                if not vis.any():
                    continue
                p = np.exp(s[i][vis] - s[i][vis].max())
                want = (p @ v[b, 0][vis].astype(np.float64)) / p.sum()
                np.testing.assert_allclose(got[b, h, i], want, rtol=1e-12, atol=1e-12)
