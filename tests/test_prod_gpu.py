"""GPU parity of the Prod codec (MSE at bits - 1 + one-bit QJL residual sketch).

The reference defines ``_TurboQuantProdCodec`` (turboquant_cache.py:4572-4766)
but builds none; the oracle restates its array path.  Bar:
  * norms and MSE indices bit-exact (the MSE part is the append kernel's f32
    order at bits - 1);
  * residual norms within 1 f32 ulp-scale (2^-22 relative): the residual is
    u - estimate in that same order, then normed with the same tree -- equal
    bits are expected, a few ulps are allowed for the estimate's FWHT;
  * QJL signs: equal wherever |residual @ P^T| exceeds 2^-18 of the row's
    scale (a matrix-core product has no fixed summation order, so a sign can
    differ only next to zero), and no more than 2 flips per 10^4 signs;
  * dequantize within 1e-5 relative of the float64 restatement.
"""
import numpy as np
import pytest
import torch

from oracle import tq_oracle as O
from kaplumba_amd.prod import ProdCodec

pytestmark = pytest.mark.gpu


def _oracle(x, codec, norm_dtype):
    d = codec.dim
    cb = O.beta_codebook(d, codec.bits - 1) if codec.bits > 1 else None
    return O.quantize_prod(x, codec.bits, O.rht_signs(d, codec.seed), cb, O.projection_matrix(d, codec.seed + 1),
                           norm_dtype)


@pytest.mark.parametrize("d", [32, 64, 128, 256, 512])
@pytest.mark.parametrize("bits", [1, 2, 3, 4])
def test_prod_quantize_matches_oracle(device, d, bits):
    rng = np.random.default_rng(d + bits)
    B, H, L = 2, 3, 45
    s = np.exp(rng.normal(0, 0.5, size=(1, H, 1, d)))
    x = (rng.standard_normal((B, H, L, d)) * s).astype(np.float16)
    codec = ProdCodec(d, bits, 0)
    st = codec.alloc(B, H, L + 9, device, torch.float32)
    codec.quantize_into(torch.from_numpy(x).to(device), st, 4)
    n, mse, rn, sg, proj = _oracle(x.astype(np.float32), codec, "float32")
    sl = slice(4, 4 + L)
    assert np.array_equal(st.norms.cpu().numpy()[:, :, sl], n)
    if bits > 1:
        assert np.array_equal(st.mse_indices.cpu().numpy().astype(np.uint32)[:, :, sl], mse)
    grn = st.residual_norms.cpu().numpy()[:, :, sl]
    assert np.allclose(grn, rn, rtol=2.0 ** -20, atol=0), float(np.abs(grn / rn - 1).max())
    gs = O.unpack_lowbit(st.qjl_signs.cpu().numpy().astype(np.uint32)[:, :, sl], 1, d)
    ws = O.unpack_lowbit(sg, 1, d)
    bad = gs != ws
    scale = np.abs(proj).max(axis=-1, keepdims=True)
    assert (np.abs(proj)[bad] <= (2.0 ** -18) * np.broadcast_to(scale, proj.shape)[bad]).all()
    assert bad.sum() <= max(2, bad.size // 5000), int(bad.sum())
    # rows outside [offset, offset + L) untouched
    assert not st.norms.cpu().numpy()[:, :, :4].any()
    assert not st.qjl_signs.cpu().numpy()[:, :, 4 + L:].any()


@pytest.mark.parametrize("d", [48, 99, 100, 200])
@pytest.mark.parametrize("bits", [1, 2, 3, 4])
def test_prod_quantize_dense_dims(device, d, bits):
    """Dims that are not powers of two: the MSE part takes the dense rotation
    (turboquant_cache.py:4122-4139), estimate c[idx] @ R (:4146-4149).
    Indices as the dense append's bar (equal except within (d/4 + 4) 2^-24
    of a midpoint); the residual then follows the kernel's indices.  Its
    estimate sums d products in f32 where the oracle rounds the exact one
    once, so residual norms agree within d 2^-22 and signs may flip only
    within 2^-12 of the row's largest projection."""
    rng = np.random.default_rng(50 + d + bits)
    B, H, L = 2, 3, 37
    x = (rng.standard_normal((B, H, L, d)) * np.exp(rng.normal(0, 0.5, size=(1, H, 1, d)))).astype(np.float16)
    codec = ProdCodec(d, bits, 0)
    assert codec.rotation == "dense" and codec.sign_width == (d + 31) // 32
    st = codec.alloc(B, H, L + 9, device, torch.float32)
    codec.quantize_into(torch.from_numpy(x).to(device), st, 4)
    sl = slice(4, 4 + L)
    xf = x.astype(np.float32)
    R, P = O.rotation_matrix(d, 0), O.projection_matrix(d, 1)
    mb = bits - 1
    cb = O.beta_codebook(d, mb) if mb else None
    gi = None
    if mb:
        wp, _, y = O.quantize_dense(xf, mb, R, cb)
        gi = O.unpack_lowbit(st.mse_indices.cpu().numpy().astype(np.uint32)[:, :, sl], mb, d).astype(np.int64)
        wi = O.unpack_lowbit(wp, mb, d).astype(np.int64)
        bad = gi != wi
        if bad.any():
            mids = O.midpoints(cb).astype(np.float64)
            dist = np.abs(y[bad].astype(np.float64)[:, None] - mids[None, :]).min(axis=1)
            assert dist.max() <= (d / 4 + 4) * 2.0 ** -24
            assert np.abs(gi[bad] - wi[bad]).max() == 1
        assert bad.sum() <= 3
    n, _, rn, sg, proj = O.quantize_prod(xf, bits, R, cb, P, rot_kind="dense", indices=gi)
    assert np.array_equal(st.norms.cpu().numpy()[:, :, sl], n)
    grn = st.residual_norms.cpu().numpy()[:, :, sl]
    assert np.abs(grn - rn).max() <= d * 2.0 ** -22, float(np.abs(grn - rn).max())
    gs = O.unpack_lowbit(st.qjl_signs.cpu().numpy().astype(np.uint32)[:, :, sl], 1, d)
    bad = gs != O.unpack_lowbit(sg, 1, d)
    scale = np.abs(proj).max(axis=-1, keepdims=True)
    assert (np.abs(proj)[bad] <= 2.0 ** -12 * np.broadcast_to(scale, proj.shape)[bad]).all()
    assert bad.sum() <= max(2, bad.size // 2000), int(bad.sum())
    assert not st.norms.cpu().numpy()[:, :, :4].any()
    assert not st.qjl_signs.cpu().numpy()[:, :, 4 + L:].any()


@pytest.mark.parametrize("d,bits", [(48, 3), (100, 1), (99, 4)])
def test_prod_dequantize_dense_dims(device, d, bits):
    rng = np.random.default_rng(13 + d)
    x = rng.standard_normal((2, 2, 20, d)).astype(np.float32)
    codec = ProdCodec(d, bits, 1)
    st = codec.quantize(torch.from_numpy(x).to(device), norm_dtype=torch.float32)
    got = codec.dequantize(st).cpu().numpy().astype(np.float64)
    cb = O.beta_codebook(d, bits - 1) if bits > 1 else None
    want = O.prod_key_vectors(st.norms.cpu().numpy(), st.mse_indices.cpu().numpy().astype(np.uint32),
                              st.residual_norms.cpu().numpy(), st.qjl_signs.cpu().numpy().astype(np.uint32),
                              bits=bits, dim=d, signs=O.rotation_matrix(d, 1), mse_codebook=cb,
                              proj=O.projection_matrix(d, 2), rot_kind="dense")
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5 * np.abs(want).max())


@pytest.mark.parametrize("bits", [3, 4])
def test_prod_quantize_division_edge_rows(device, bits):
    # f32 rows on both sides of the quotient method's switch (elements below
    # 2^-100 take the IEEE division itself): norms and MSE indices bit-exact.
    d = 128
    rng = np.random.default_rng(90 + bits)
    x = rng.standard_normal((1, 2, 6, d)).astype(np.float32)
    x[0, 0, 0, :3] = [1e-36, -4e-39, 0.0]      # tiny elements beside normal ones
    x[0, 0, 1] = 3e-32                         # every element below 2^-100
    x[0, 0, 2, ::2] = 0.0                      # zeros between normal values
    x[0, 1, 3] *= 2.0 ** -95                   # small, fast side of the switch
    codec = ProdCodec(d, bits, 0)
    st = codec.alloc(1, 2, 6, device, torch.float32)
    codec.quantize_into(torch.from_numpy(x).to(device), st, 0)
    n, mse, rn, sg, proj = _oracle(x, codec, "float32")
    assert np.array_equal(st.norms.cpu().numpy(), n)
    assert np.array_equal(st.mse_indices.cpu().numpy().astype(np.uint32), mse)


def test_prod_quantize_f16_norms_bf16_input(device):
    rng = np.random.default_rng(3)
    x = torch.from_numpy(rng.standard_normal((1, 2, 33, 128)).astype(np.float32)).to(torch.bfloat16)
    codec = ProdCodec(128, 3, 5)
    st = codec.quantize(x.to(device))                 # reference layout: f16 norms
    n, mse, rn, sg, proj = _oracle(x.float().numpy(), codec, "float16")
    assert st.norms.dtype == torch.float16
    assert np.array_equal(st.norms.float().cpu().numpy(), n)
    assert np.array_equal(st.mse_indices.cpu().numpy().astype(np.uint32), mse)
    # f16 residual norms: at most one f16 ulp apart (the f32 value rounds the same almost always)
    grn = st.residual_norms.float().cpu().numpy()
    assert (np.abs(grn - rn) <= np.spacing(rn.astype(np.float16)).astype(np.float32)).all()


@pytest.mark.parametrize("d,bits", [(64, 1), (128, 3), (256, 4), (32, 2), (512, 3), (512, 1)])
def test_prod_dequantize_matches_oracle(device, d, bits):
    rng = np.random.default_rng(11 + d)
    x = rng.standard_normal((2, 2, 20, d)).astype(np.float32)
    codec = ProdCodec(d, bits, 1)
    st = codec.quantize(torch.from_numpy(x).to(device), norm_dtype=torch.float32)
    got = codec.dequantize(st).cpu().numpy().astype(np.float64)
    cb = O.beta_codebook(d, bits - 1) if bits > 1 else None
    want = O.prod_key_vectors(st.norms.cpu().numpy(), st.mse_indices.cpu().numpy().astype(np.uint32),
                              st.residual_norms.cpu().numpy(), st.qjl_signs.cpu().numpy().astype(np.uint32),
                              bits=bits, dim=d, signs=O.rht_signs(d, 1), mse_codebook=cb,
                              proj=O.projection_matrix(d, 2))
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5 * np.abs(want).max())


def test_prod_inner_products_are_unbiased(device):
    """The QJL term makes <q, dequant(k)> an unbiased estimate of <q, k>
    (the codec's purpose): over many keys the mean error is far below the
    MSE-only estimate's bias, which the 1-bit MSE part alone would show."""
    rng = np.random.default_rng(21)
    d = 128
    k = rng.standard_normal((1, 1, 4096, d)).astype(np.float32)
    q = rng.standard_normal(d).astype(np.float32)
    codec = ProdCodec(d, 2, 0)
    st = codec.quantize(torch.from_numpy(k).to(device), norm_dtype=torch.float32)
    kh = codec.dequantize(st).cpu().numpy()[0, 0].astype(np.float64)
    exact = k[0, 0].astype(np.float64) @ q
    est = kh @ q
    slope = float(est @ exact / (exact @ exact))
    assert abs(slope - 1.0) < 0.03, slope
    corr = np.corrcoef(est, exact)[0, 1]
    assert corr > 0.8, corr


def _prod_case(device, seed, B, Hq, Hkv, L, T, d, kb, vb, qdt="bf16", lengths=None, starts=None,
               causal=None, norm_dtype=torch.float32):
    from kaplumba_amd import ops
    from kaplumba_amd.prod import attention_prod
    from tests import test_attention_gpu as _A
    assert_close, q_tensor = _A.assert_close, _A.q_tensor

    causal = (L > 1) if causal is None else causal
    rng = np.random.default_rng(seed)
    s = np.exp(rng.normal(0, 0.5, size=(1, Hkv, 1, d)))
    k = (rng.standard_normal((B, Hkv, T, d)) * s).astype(np.float16)
    v = (rng.standard_normal((B, Hkv, T, d)) * s).astype(np.float16)
    q = O.round_to_dtype(rng.standard_normal((B, Hq, L, d)).astype(np.float32), qdt)
    kc, vc = ProdCodec(d, kb, 0), ops.Codec(d, vb, 1)
    cap = T + 5
    kst = kc.alloc(B, Hkv, cap, device, norm_dtype)
    kc.quantize_into(torch.from_numpy(k).to(device), kst, 0)
    vp = torch.zeros((B, Hkv, cap, vc.packed_width), dtype=torch.uint32, device=device)
    vn = torch.zeros((B, Hkv, cap), dtype=norm_dtype, device=device)
    ops.append_quantize(torch.from_numpy(v).to(device), vc, vp, vn, 0)
    view = type(kst)(*(t[:, :, :T] for t in kst))
    sl = torch.tensor(lengths, dtype=torch.int32) if lengths is not None else None
    ss = torch.tensor(starts, dtype=torch.int32) if starts is not None else None
    out = attention_prod(q_tensor(q, qdt, device), view, vn[:, :, :T], vp[:, :, :T], kc, vc,
                         1 / np.sqrt(d), causal, seq_lens=sl, seq_starts=ss)
    # the oracle reads the kernel-written state (its bits are checked above)
    kn, km, kr, ks = (t[:, :, :T].float().cpu().numpy() if t.dtype != torch.uint32
                      else t[:, :, :T].cpu().numpy().astype(np.uint32) for t in kst)
    want = O.attention_prod(q, kn, km, kr, ks, vp[:, :, :T].cpu().numpy().astype(np.uint32),
                            vn[:, :, :T].float().cpu().numpy(), k_bits=kb, v_bits=vb,
                            k_signs_rot=O.rht_signs(d, 0), k_mse_codebook=O.beta_codebook(d, kb - 1),
                            proj=O.projection_matrix(d, 1), v_codebook=O.beta_codebook(d, vb),
                            v_rot=O.rht_signs(d, 1), scale=1 / np.sqrt(d), q_dtype=qdt,
                            causal=causal, lengths=None if lengths is None else
                            [min(x, T) for x in lengths]) if starts is None else None
    if starts is not None:
        parts = []
        for b in range(B):
            e = T if lengths is None else lengths[b]
            sl_ = slice(starts[b], e)
            parts.append(O.attention_prod(
                q[b:b + 1], kn[b:b + 1, :, sl_], km[b:b + 1, :, sl_], kr[b:b + 1, :, sl_],
                ks[b:b + 1, :, sl_], vp[b:b + 1, :, sl_].cpu().numpy().astype(np.uint32),
                vn[b:b + 1, :, sl_].float().cpu().numpy(), k_bits=kb, v_bits=vb,
                k_signs_rot=O.rht_signs(d, 0), k_mse_codebook=O.beta_codebook(d, kb - 1),
                proj=O.projection_matrix(d, 1), v_codebook=O.beta_codebook(d, vb),
                v_rot=O.rht_signs(d, 1), scale=1 / np.sqrt(d), q_dtype=qdt, causal=causal))
        want = np.concatenate(parts)
    assert_close(out, want, qdt, f"prod B{B} Hq{Hq} Hkv{Hkv} L{L} T{T} d{d} k{kb}v{vb}")


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("kb,vb", [(2, 1), (3, 3), (4, 2), (4, 4)])
def test_prod_decode_attention(device, d, kb, vb):
    _prod_case(device, 30 + d + kb * 10 + vb, 1, 8, 2, 1, 2500, d, kb, vb)


def test_prod_verify_ragged_f16_norms(device):
    """causal 2-draft verify (4 rows per kv head), ragged lengths, f16 norms, f16 queries."""
    _prod_case(device, 7, 3, 4, 2, 2, 3000, 128, 3, 3, qdt="f16", lengths=[3000, 5, 1234],
               norm_dtype=torch.float16)


def test_prod_f16_norms_odd_sequence_ends(device):
    _prod_case(device, 12, 3, 8, 2, 1, 701, 128, 4, 2, lengths=[5, 701, 33], norm_dtype=torch.float16)


def test_prod_left_padded_rows(device):
    _prod_case(device, 8, 2, 8, 2, 1, 2100, 128, 4, 3, starts=[0, 1500])


def test_prod_sixteen_rows_per_kv_head(device):
    """16 query rows per kv head run the general kernels (tq_attention_prod routes them)."""
    _prod_case(device, 9, 1, 32, 8, 4, 300, 128, 3, 3)


def test_cache_with_prod_keys_decode_and_save_load(device, tmp_path):
    """TurboQuantKVCache(key_quantizer="prod"): append, decode through the
    model-layer dispatch, dequantize, and a save / load round trip."""
    import math

    from kaplumba_amd import (TurboQuantKVCache, load_prompt_cache, save_prompt_cache,
                              scaled_dot_product_attention)
    from kaplumba_amd.prod import TurboQuantProdState
    from tests import test_attention_gpu as _A

    B, Hq, Hkv, D = 1, 8, 2, 128
    g = torch.Generator().manual_seed(5)
    cache = TurboQuantKVCache(bits=3.5, key_quantizer="prod")   # keys: Prod 3 bits, values: MSE 4
    ks = [torch.randn(B, Hkv, 300, D, generator=g).to(torch.bfloat16)]
    vs = [torch.randn(B, Hkv, 300, D, generator=g).to(torch.bfloat16)]
    kst, vst = cache.update_and_fetch(ks[0].to(device), vs[0].to(device))
    for _ in range(3):
        ks.append(torch.randn(B, Hkv, 1, D, generator=g).to(torch.bfloat16))
        vs.append(torch.randn(B, Hkv, 1, D, generator=g).to(torch.bfloat16))
        kst, vst = cache.update_and_fetch(ks[-1].to(device), vs[-1].to(device))
    assert cache.offset == 303 and isinstance(cache.state[0], TurboQuantProdState)
    assert cache.meta_state[5] == "prod" and cache.key_codec.bits == 3 and cache.value_codec.bits == 4
    q = torch.randn(B, Hq, 1, D, generator=g).to(torch.bfloat16)
    out = scaled_dot_product_attention(q.to(device), kst, vst, cache, 1 / math.sqrt(D), None)
    k_all = torch.cat(ks, dim=2).float().numpy()
    n, mse, rn, sg, _ = O.quantize_prod(k_all, 3, O.rht_signs(D, 0), O.beta_codebook(D, 2),
                                        O.projection_matrix(D, 1))
    st = cache.state
    assert np.array_equal(st[0].mse_indices.cpu().numpy().astype(np.uint32), mse)
    v_np = torch.cat(vs, dim=2).float().numpy()
    vp, vn = O.quantize_rht(v_np, 4, O.rht_signs(D, 1), O.beta_codebook(D, 4))
    want = O.attention_prod(q.float().numpy(), st[0].norms.cpu().numpy(),
                            st[0].mse_indices.cpu().numpy().astype(np.uint32),
                            st[0].residual_norms.cpu().numpy(),
                            st[0].qjl_signs.cpu().numpy().astype(np.uint32), vp, vn, k_bits=3,
                            v_bits=4, k_signs_rot=O.rht_signs(D, 0), k_mse_codebook=O.beta_codebook(D, 2),
                            proj=O.projection_matrix(D, 1), v_codebook=O.beta_codebook(D, 4),
                            v_rot=O.rht_signs(D, 1), scale=1 / math.sqrt(D), q_dtype="bf16")
    _A.assert_close(out, want, "bf16", "prod cache decode")
    kd, vd = cache.dequantize()
    assert kd.shape == (B, Hkv, 303, D) and vd.shape == (B, Hkv, 303, D)
    f = str(tmp_path / "prod.safetensors")
    save_prompt_cache(f, [cache])
    loaded = load_prompt_cache(f)[0]
    assert loaded.key_quantizer == "prod" and isinstance(loaded.state[0], TurboQuantProdState)
    out2 = loaded.decode_attention(q.to(device), scale=1 / math.sqrt(D))
    assert torch.equal(out, out2)


def test_cache_with_prod_keys_at_a_dense_dim(device):
    """TurboQuantKVCache(key_quantizer="prod") at head dim 100: both codecs take
    the dense rotation; decode through the model-layer dispatch against the
    oracle on the cache's own state."""
    import math

    from kaplumba_amd import TurboQuantKVCache, scaled_dot_product_attention
    from tests.test_attention_gpu import assert_close
    from tests.test_general_attention_gpu import _prod_general_oracle

    B, Hq, Hkv, D = 1, 8, 2, 100
    g = torch.Generator().manual_seed(6)
    cache = TurboQuantKVCache(bits=3.5, key_quantizer="prod")
    cache.update_and_fetch(torch.randn(B, Hkv, 260, D, generator=g).to(torch.bfloat16).to(device),
                           torch.randn(B, Hkv, 260, D, generator=g).to(torch.bfloat16).to(device))
    kst, vst = cache.update_and_fetch(torch.randn(B, Hkv, 1, D, generator=g).to(torch.bfloat16).to(device),
                                      torch.randn(B, Hkv, 1, D, generator=g).to(torch.bfloat16).to(device))
    assert cache.key_codec.rotation == "dense" and cache.value_codec.rotation == "dense"
    q = torch.randn(B, Hq, 1, D, generator=g).to(torch.bfloat16)
    out = scaled_dot_product_attention(q.to(device), kst, vst, cache, 1 / math.sqrt(D), None)
    ks, vs = cache.state
    kn, km, kr, ksg = (t.float().cpu().numpy() if t.dtype != torch.uint32 else t.cpu().numpy().astype(np.uint32)
                       for t in ks)
    want = _prod_general_oracle(q.float().numpy(), kn, km, kr, ksg, vs.indices.cpu().numpy().astype(np.uint32),
                                vs.norms.float().cpu().numpy(), 3, 4, D, D, O.rotation_matrix(D, 1), "dense",
                                "bf16", False, None, None)
    assert_close(out, want, "bf16", "prod cache at d = 100")
    kd, vd = cache.dequantize()
    assert kd.shape == (B, Hkv, 261, D) and vd.shape == (B, Hkv, 261, D)
