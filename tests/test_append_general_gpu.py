"""GPU parity of the dense-rotation append and dequantize at the dims the
fixed-size kernels do not take (any dim in 8..512; the reference picks
the dense rotation for every dim that is not a power of two,
turboquant_cache.py:4122-4139), and of caches built at such dims.

Bar: norms bit-exact (the oracle's norm tree with the dim zero-padded to a
power-of-two number of 32-element lanes); packed indices equal to the
oracle's except where the oracle's rotated coordinate lies within BAND(d) of
a midpoint.  The kernel forms y = u @ R^T with f32 fused multiply-adds in four
partial sums of d/4 terms, each bounded by |u| |R_j| = 1 in magnitude, so its
y is within (d/4 + 2) f32 ulps of 1.0 of the exact product; the oracle rounds
the exact product once.  BAND(d) = (d/4 + 4) * 2^-24 holds that worst case.
Flips inside the band move the index by exactly one step.
"""
import math

import numpy as np
import pytest
import torch

from oracle import tq_oracle as O
from kaplumba_amd import ops
from tests.test_attention_gpu import assert_close

pytestmark = pytest.mark.gpu


def band(d):
    return (d / 4 + 4) * 2.0 ** -24


def _check(x_in, bits, d, seed, got_packed, got_norms, norm_dtype="float32"):
    cb = O.beta_codebook(d, bits)
    wp, wn, y = O.quantize_dense(x_in, bits, O.rotation_matrix(d, seed), cb, norm_dtype)
    assert np.array_equal(got_norms, wn), "norms differ"
    gi = O.unpack_lowbit(got_packed, bits, d).astype(np.int64)
    wi = O.unpack_lowbit(wp, bits, d).astype(np.int64)
    bad = gi != wi
    if bad.any():
        mids = O.midpoints(cb).astype(np.float64)
        dist = np.abs(y[bad].astype(np.float64)[:, None] - mids[None, :]).min(axis=1)
        assert dist.max() <= band(d), f"index differs {dist.max():.3g} away from a midpoint"
        assert np.abs(gi[bad] - wi[bad]).max() == 1
    return int(bad.sum())


@pytest.mark.parametrize("d", [8, 13, 24, 38, 48, 80, 96, 99, 130, 160, 192, 320, 509, 512])
@pytest.mark.parametrize("xdt", ["bf16", "f16", "f32"])
def test_dense_append_any_dim(device, d, xdt):
    rng = np.random.default_rng(2000 + d)
    bits = 1 + d % 4
    B, H, L = 2, 3, 21   # 126 vectors: whole 16-vector workgroups plus a ragged one
    x32 = (rng.standard_normal((B, H, L, d)) * np.exp(rng.normal(0, 0.5, (1, H, 1, d)))).astype(np.float32)
    tdt = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[xdt]
    x = torch.from_numpy(x32).to(tdt).to(device)
    codec = ops.Codec(d, bits, 0, rotation="dense")
    packed = torch.zeros((B, H, 30, codec.packed_width), dtype=torch.uint32, device=device)
    norms = torch.zeros((B, H, 30), dtype=torch.float32, device=device)
    ops.append_quantize(x, codec, packed, norms, offset=5)
    gp = packed.cpu().numpy().astype(np.uint32)
    gn = norms.cpu().numpy()
    flips = _check(x.float().cpu().numpy(), bits, d, 0, gp[:, :, 5:26], gn[:, :, 5:26])
    assert flips <= 3, flips
    assert not gp[:, :, :5].any() and not gp[:, :, 26:].any()
    assert not gn[:, :, :5].any() and not gn[:, :, 26:].any()


def test_dense_append_f16_norms_and_division_edges(device):
    """f16 norms; zero, tiny and huge rows take the same IEEE division as the oracle."""
    d, bits = 96, 3
    rng = np.random.default_rng(2100)
    x32 = rng.standard_normal((1, 2, 40, d)).astype(np.float32)
    x32[0, 0, 0] = 0.0
    x32[0, 0, 1] *= 1e-30
    x32[0, 1, 2] *= 1e15
    x = torch.from_numpy(x32).to(device)
    codec = ops.Codec(d, bits, 3, rotation="dense")
    packed = torch.zeros((1, 2, 40, codec.packed_width), dtype=torch.uint32, device=device)
    norms = torch.zeros((1, 2, 40), dtype=torch.float16, device=device)
    ops.append_quantize(x, codec, packed, norms, offset=0)
    _check(x32, bits, d, 3, packed.cpu().numpy().astype(np.uint32),
           norms.cpu().numpy().astype(np.float16), norm_dtype="float16")


@pytest.mark.parametrize("d,rot", [(96, "dense"), (320, "dense"), (512, "hadamard"), (512, "dense"),
                                   (40, "dense"), (13, "dense"), (99, "dense"), (130, "dense")])
def test_dequantize_any_dim(device, d, rot):
    rng = np.random.default_rng(2200 + d)
    bits = 3
    x32 = rng.standard_normal((1, 2, 17, d)).astype(np.float32)
    r = O.rht_signs(d, 4) if rot == "hadamard" else O.rotation_matrix(d, 4)
    cb = O.beta_codebook(d, bits)
    if rot == "hadamard":
        wp, wn = O.quantize_rht(x32, bits, r, cb)
    else:
        wp, wn, _ = O.quantize_dense(x32, bits, r, cb)
    codec = ops.Codec(d, bits, 4, rotation=rot)
    got = ops.dequantize(torch.from_numpy(wp.astype(np.uint32)).to(device),
                         torch.from_numpy(wn).to(device), codec)
    want = O.dequantize(wp, wn, bits, d, cb, rot, r)
    np.testing.assert_allclose(got.cpu().numpy(), want, atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("k_dim,v_dim", [(96, 96), (192, 128), (128, 80), (100, 100), (75, 58)])
def test_cache_at_other_head_dims(device, k_dim, v_dim):
    """TurboQuantKVCache whose codecs pick the dense rotation for the dims that
    are not powers of two: prefill + decode appends through update_and_fetch,
    then decode and verify attention vs the oracle on the cache's own state
    (whose packed rows are checked against the oracle's quantizer first)."""
    from kaplumba_amd import TurboQuantKVCache

    B, Hq, Hkv = 1, 8, 2
    g = torch.Generator().manual_seed(k_dim + v_dim)
    cache = TurboQuantKVCache(bits=3)
    ks = [torch.randn(B, Hkv, 300, k_dim, generator=g).to(torch.bfloat16)]
    vs = [torch.randn(B, Hkv, 300, v_dim, generator=g).to(torch.bfloat16)]
    cache.update_and_fetch(ks[0].to(device), vs[0].to(device))
    for _ in range(2):
        ks.append(torch.randn(B, Hkv, 1, k_dim, generator=g).to(torch.bfloat16))
        vs.append(torch.randn(B, Hkv, 1, v_dim, generator=g).to(torch.bfloat16))
        kst, vst = cache.update_and_fetch(ks[-1].to(device), vs[-1].to(device))
    assert cache.offset == 302
    st_k, st_v = cache.state
    kc, vc = cache.key_codec, cache.value_codec
    assert kc.rotation == ("hadamard" if k_dim & (k_dim - 1) == 0 else "dense")
    assert vc.rotation == ("hadamard" if v_dim & (v_dim - 1) == 0 else "dense")
    flips = 0
    for codec, xs, stt in ((kc, ks, st_k), (vc, vs, st_v)):
        x = torch.cat(xs, dim=2).float().numpy()
        got_p = stt.indices.cpu().numpy().astype(np.uint32)
        got_n = stt.norms.float().cpu().numpy()
        if codec.rotation == "dense":
            flips += _check(x, codec.bits, codec.dim, codec.seed, got_p, got_n)
        else:
            wp, wn = O.quantize_rht(x, codec.bits, O.rht_signs(codec.dim, codec.seed),
                                    O.beta_codebook(codec.dim, codec.bits))
            assert np.array_equal(got_p, wp) and np.array_equal(got_n, wn)
    assert flips <= 3
    for L in (1, 3):
        q = torch.randn(B, Hq, L, k_dim, generator=g).to(torch.bfloat16)
        out = cache.quantized_attention(q.to(device), scale=1 / math.sqrt(k_dim),
                                        mask="causal" if L > 1 else None)
        assert out.shape == (B, Hq, L, v_dim)
        want = O.attention(q.float().numpy(), st_k.indices.cpu().numpy().astype(np.uint32),
                           st_k.norms.float().cpu().numpy(), st_v.indices.cpu().numpy().astype(np.uint32),
                           st_v.norms.float().cpu().numpy(), k_bits=kc.bits, v_bits=vc.bits,
                           k_codebook=kc.codebook, v_codebook=vc.codebook, rot_kind=kc.rotation,
                           k_rot=kc.rot_host, v_rot=vc.rot_host, scale=1 / math.sqrt(k_dim),
                           q_dtype="bf16", causal=L > 1, v_dim=v_dim, v_rot_kind=vc.rotation)
        assert_close(out, want, "bf16", f"cache k{k_dim} v{v_dim} L{L}")
