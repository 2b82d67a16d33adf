"""Host-side cache logic that needs no GPU: validation, policy, state plumbing, masks, I/O."""
import os
import tempfile

import numpy as np
import pytest
import torch

from kaplumba_amd import (KVCache, TurboQuantKVCache, TurboQuantMSEState, can_trim_prompt_cache,
                          create_attention_mask, create_causal_mask, load_prompt_cache,
                          make_prompt_cache, save_prompt_cache, trim_prompt_cache)
from kaplumba_amd import ops
from kaplumba_amd.cache import _tree_flatten, _tree_unflatten


def test_init():
    cache = TurboQuantKVCache(bits=3)
    assert cache.quant_bits == 3 and cache.offset == 0 and cache.empty()
    assert cache.size() == 0 and cache.nbytes == 0 and cache.state == []


@pytest.mark.parametrize("bits", [0, 0.5, 3.3, -1])
def test_invalid_bits_raise(bits):
    with pytest.raises(ValueError):
        TurboQuantKVCache(bits=bits)


def test_half_bits_split_and_overrides():
    c = TurboQuantKVCache(bits=3.5)
    assert c._side_bits() == (3, 4) and c.quant_bits == 3
    c = TurboQuantKVCache(bits=3, key_bits=4, val_bits=2)
    assert c._side_bits() == (4, 2)
    with pytest.raises(ValueError):
        TurboQuantKVCache(bits=3, key_bits=5)
    with pytest.raises(ValueError):
        TurboQuantKVCache(bits=3, rotation="givens")
    with pytest.raises(ValueError):
        TurboQuantKVCache(bits=3, codebook="uniform")


def _cpu_state(B, H, T, pw, norm_dtype=torch.float16):
    g = torch.Generator().manual_seed(0)
    mk = lambda: TurboQuantMSEState(torch.rand(B, H, T, generator=g).to(norm_dtype),
                                    torch.randint(0, 2 ** 31 - 1, (B, H, T, pw), generator=g).to(torch.uint32))
    return mk(), mk()


def test_state_setter_trim_meta_from_state():
    st = _cpu_state(1, 4, 10, 6)
    c = TurboQuantKVCache(bits=3, seed=7)
    c.state = st
    c.meta_state = ("10", "3.0", "7", "64", "64")
    assert c.offset == 10 and not c.empty() and c.size() == 10
    # the reference's five fields, then (key_quantizer, key_bits, val_bits, rotation, codebook)
    assert c.meta_state == ("10", "3.0", "7", "64", "64", "mse", "3", "3", "auto", "beta")
    assert c.trim(3) == 3 and c.offset == 7 and c.state[0].norms.shape[2] == 7
    assert c.trim(100) == 7 and c.offset == 0
    r = TurboQuantKVCache.from_state(st, ("10", "3.0", "7", "64", "64"))
    assert r.offset == 10 and r.quant_bits == 3 and r.seed == 7 and r.meta_state[3] == "64"
    assert r.nbytes == sum(t.numel() * t.element_size() for s in st for t in s)
    c.state = []
    assert c.empty() and c.offset == 0


def test_make_prompt_cache_policies():
    class M:
        layers = [None] * 8

    caches = make_prompt_cache(M(), turbo_kv_bits=3, turbo_fp16_layers=2)
    kinds = [type(c).__name__ for c in caches]
    assert kinds == ["KVCache"] * 2 + ["TurboQuantKVCache"] * 4 + ["KVCache"] * 2
    caches = make_prompt_cache(num_layers=36, turbo_kv_bits=3, turbo_fp16_layers=4,
                               fp16_layer_policy="first")
    assert [isinstance(c, KVCache) for c in caches] == [True] * 4 + [False] * 32
    assert all(isinstance(c, KVCache) for c in make_prompt_cache(M()))

    class Hybrid:
        def make_cache(self):
            return [KVCache(), "ssm-state", KVCache()]

    caches = make_prompt_cache(Hybrid(), turbo_kv_bits=2, turbo_fp16_layers=5)
    assert isinstance(caches[0], TurboQuantKVCache) and caches[1] == "ssm-state"
    with pytest.raises(NotImplementedError):
        make_prompt_cache(M(), max_kv_size=128)
    assert can_trim_prompt_cache(make_prompt_cache(M(), turbo_kv_bits=3))
    assert trim_prompt_cache([], 3) == 0


def test_masks():
    m = create_causal_mask(3, offset=2)
    assert m.shape == (3, 5)
    assert m.tolist() == [[True, True, True, False, False], [True, True, True, True, False],
                          [True, True, True, True, True]]
    assert create_attention_mask(1, offset=5) is None
    assert create_attention_mask(4, offset=5) == "causal"
    assert create_attention_mask(4, offset=5, return_array=True).shape == (4, 9)
    w = create_attention_mask(4, offset=5, window_size=2)
    assert w.sum().item() == 8
    c = TurboQuantKVCache(bits=3)
    c.state = _cpu_state(1, 2, 6, 12)
    assert c.make_mask(3) == "causal" and c.make_mask(1) is None


def test_tree_flatten_naming_round_trip():
    tree = [[("a", "b"), "c"], {"model": "x"}, ["KVCache", "TurboQuantKVCache"]]
    flat = _tree_flatten(tree)
    assert flat[0] == ("0.0.0", "a") and ("1.model", "x") in flat and ("2.1", "TurboQuantKVCache") in flat
    back = _tree_unflatten(flat)
    assert back[0][0] == ["a", "b"] and back[1] == {"model": "x"}


def test_save_load_cpu_state():
    tq = TurboQuantKVCache(bits=3, seed=4)
    tq.state = _cpu_state(1, 4, 10, 12)
    tq.meta_state = ("10", "3.0", "4", "128", "128")
    kv = KVCache()
    kv.state = (torch.randn(1, 4, 10, 64).half(), torch.randn(1, 4, 10, 64).half())
    empty = TurboQuantKVCache(bits=2)
    with tempfile.TemporaryDirectory() as d:
        f = os.path.join(d, "c.safetensors")
        save_prompt_cache(f, [kv, tq, empty], {"k": "v"})
        loaded, meta = load_prompt_cache(f, return_metadata=True, device="cpu")
    assert meta == {"k": "v"}
    assert isinstance(loaded[0], KVCache) and loaded[0].offset == 10
    assert isinstance(loaded[1], TurboQuantKVCache) and loaded[1].offset == 10 and loaded[1].seed == 4
    assert torch.equal(loaded[1].state[0].indices, tq.state[0].indices)
    assert loaded[1].state[0].indices.dtype == torch.uint32
    assert loaded[2].empty() and loaded[2].quant_bits == 2


def test_untrusted_class_rejected():
    from safetensors.torch import save_file

    with tempfile.TemporaryDirectory() as d:
        f = os.path.join(d, "bad.safetensors")
        save_file({"0.0": torch.zeros(1)}, f, metadata={"0.0": "1", "2.0": "EvilCache"})
        with pytest.raises(ValueError, match="Untrusted"):
            load_prompt_cache(f, device="cpu")


def test_ops_refuse_cpu_tensors():
    codec = ops.Codec(128, 3, 0)
    with pytest.raises(ValueError, match="no CPU path"):
        ops.append_quantize(torch.zeros(1, 1, 1, 128), codec, torch.zeros(1, 1, 4, 12, dtype=torch.uint32),
                            torch.zeros(1, 1, 4), 0)
    with pytest.raises(ValueError, match="Hadamard"):
        ops.Codec(96, 3, 0, rotation="hadamard")
    assert ops.Codec(96, 3, 0).rotation == "dense"


def test_prod_key_quantizer_options_and_meta_state():
    c = TurboQuantKVCache(bits=3, key_quantizer="prod")
    assert c.key_quantizer == "prod"
    with pytest.raises(ValueError):
        TurboQuantKVCache(bits=3, key_quantizer="qjl")
    with pytest.raises(ValueError):
        TurboQuantKVCache(bits=3, key_quantizer="prod", rotation="dense")
    # the key quantizer is the sixth field, and a CPU state round trip keeps it
    assert TurboQuantKVCache(bits=3).meta_state[5] == "mse"
    from kaplumba_amd.prod import TurboQuantProdState
    st = (TurboQuantProdState(torch.ones(1, 2, 7), torch.zeros(1, 2, 7, 8, dtype=torch.uint32),
                              torch.ones(1, 2, 7), torch.zeros(1, 2, 7, 4, dtype=torch.uint32)),
          TurboQuantMSEState(torch.ones(1, 2, 7), torch.zeros(1, 2, 7, 12, dtype=torch.uint32)))
    c2 = TurboQuantKVCache.from_state(st, ("7", "3.0", "0", "128", "128", "prod"))
    assert c2.key_quantizer == "prod" and c2.offset == 7 and c2.meta_state[5] == "prod"
    assert isinstance(c2.state[0], TurboQuantProdState) and c2.nbytes > 0


@pytest.mark.parametrize("opts", [
    dict(bits=3, rotation="dense", codebook="gaussian", key_bits=4, val_bits=2),
    dict(bits=3.5, codebook="gaussian"),
    dict(bits=2, rotation="hadamard", key_bits=1),
    dict(bits=3, key_quantizer="prod"),
])
def test_meta_state_restores_codec_options(opts):
    """A cache rebuilt from (state, meta_state) builds the codecs the saved one
    used: rotation, codebook and per-side widths (the reference keeps only
    offset, bits and seed, turboquant_cache.py:6046-6056)."""
    c = TurboQuantKVCache(seed=5, **opts)
    c._build_codecs(256, 256)
    r = TurboQuantKVCache.from_state([], c.meta_state)
    r._dims = (256, 256)
    r._ensure_codecs_from_meta()
    assert r.meta_state == c.meta_state
    assert type(r.key_codec) is type(c.key_codec)
    for a, b in ((r.key_codec, c.key_codec), (r.value_codec, c.value_codec)):
        assert (a.dim, a.bits, a.seed) == (b.dim, b.bits, b.seed)
        if isinstance(a, ops.Codec):
            assert (a.rotation, a.codebook_kind) == (b.rotation, b.codebook_kind)
            assert np.array_equal(a.codebook, b.codebook)


def test_meta_state_reference_and_round1_forms():
    """Five fields (the reference's files) give the default codecs; six carry
    the key quantizer alone; other lengths and unknown values are refused."""
    r = TurboQuantKVCache.from_state([], ("0", "3.0", "0", "128", "128"))
    r._ensure_codecs_from_meta()
    assert (r.key_codec.rotation, r.key_codec.codebook_kind, r.key_codec.bits) == ("hadamard", "beta", 3)
    r = TurboQuantKVCache.from_state([], ("0", "3.0", "0", "128", "128", "prod"))
    assert r.key_quantizer == "prod"
    for bad in [("0", "3", "0", "128", "128", "mse", "3"),
                ("0", "3", "0", "128", "128", "qjl"),
                ("0", "3", "0", "128", "128", "mse", "3", "3", "givens", "beta"),
                ("0", "3", "0", "128", "128", "mse", "3", "3", "dense", "uniform"),
                ("0", "3", "0", "128", "128", "mse", "5", "3", "dense", "beta")]:
        with pytest.raises(ValueError):
            TurboQuantKVCache.from_state([], bad)


def test_save_load_keeps_codec_options():
    """Through a prompt-cache file: a dense / Gaussian K4-V2 cache comes back
    with the same codecs (its packed widths match the saved rows)."""
    c = TurboQuantKVCache(bits=3, seed=2, rotation="dense", codebook="gaussian", key_bits=4, val_bits=2)
    c._build_codecs(256, 256)
    g = torch.Generator().manual_seed(1)
    mk = lambda pw: TurboQuantMSEState(torch.rand(1, 2, 9, generator=g),
                                       torch.randint(0, 1 << 30, (1, 2, 9, pw), generator=g).to(torch.uint32))
    c.state = (mk(32), mk(16))
    with tempfile.TemporaryDirectory() as d:
        f = os.path.join(d, "c.safetensors")
        save_prompt_cache(f, [c])
        (r,) = load_prompt_cache(f, device="cpu")
    r._ensure_codecs_from_meta()
    assert (r.key_codec.bits, r.value_codec.bits) == (4, 2)
    assert r.key_codec.rotation == r.value_codec.rotation == "dense"
    assert r.key_codec.codebook_kind == "gaussian" and r.seed == 2
    assert r.key_codec.packed_width == r.state[0].indices.shape[-1]
    assert r.value_codec.packed_width == r.state[1].indices.shape[-1]
    assert torch.equal(r.state[0].indices, c.state[0].indices)


def test_state_proxy_copies_and_forwards():
    """The (B, H, T, D) state proxy forwards attributes to its state and can be
    copied (a copy reads the slots before they are set: no recursion)."""
    import copy

    from kaplumba_amd.cache import TurboQuantMSEState, _QuantizedStateProxy

    st = TurboQuantMSEState(torch.zeros(1, 2, 8), torch.zeros(1, 2, 8, 12, dtype=torch.int32))
    p = _QuantizedStateProxy(st, 5, 2, 128, 1)
    assert p.shape == (1, 2, 5, 128) and p.norms is st.norms
    q = copy.copy(p)
    assert q.shape == p.shape and q.indices is st.indices
    blank = _QuantizedStateProxy.__new__(_QuantizedStateProxy)
    with pytest.raises(AttributeError):
        blank._state
