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


@pytest.mark.parametrize("d", [64, 128, 256])
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


@pytest.mark.parametrize("d,bits", [(64, 1), (128, 3), (256, 4)])
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
