"""GPU parity of the append-time quantizer (C ABI tq_append_quantize) vs the oracle.

Bar: packed index words and norms bit-exact.  Covers every Hadamard dim
(32..512), bits 1..4, f16/bf16/f32 inputs, f32/f16 norms, strided inputs,
writes at an offset inside a capacity buffer, zero / tiny / large vectors and
the full config-0 layer (K and V f16 [1, 8, 4096, 128], 3-bit).
"""
import numpy as np
import pytest
import torch

from oracle import tq_oracle as O
from kaplumba_amd import _lib, ops

pytestmark = pytest.mark.gpu


def _buffers(B, H, cap, codec, norm_dtype, device):
    packed = torch.zeros((B, H, cap, codec.packed_width), dtype=torch.uint32, device=device)
    norms = torch.zeros((B, H, cap), dtype=norm_dtype, device=device)
    return packed, norms


def _np_u32(t):
    return t.cpu().numpy().astype(np.uint32)


@pytest.mark.parametrize("d", [32, 64, 128, 256, 512])
@pytest.mark.parametrize("bits", [1, 2, 3, 4])
def test_fixture_vectors_bit_exact(golden, device, d, bits):
    q = golden["quantize"]
    x = torch.from_numpy(q[f"x_{d}"].reshape(1, 2, 24, d)).to(device)
    codec = ops.Codec(d, bits, 0)
    packed, norms = _buffers(1, 2, 30, codec, torch.float32, device)
    ops.append_quantize(x, codec, packed, norms, offset=3)
    got_p = _np_u32(packed)
    got_n = norms.cpu().numpy()
    want_p = q[f"packed_{d}_{bits}"].reshape(1, 2, 24, -1)
    want_n = q[f"norms_{d}_{bits}"].reshape(1, 2, 24)
    assert np.array_equal(got_p[:, :, 3:27], want_p)
    assert np.array_equal(got_n[:, :, 3:27], want_n)
    assert not got_p[:, :, :3].any() and not got_p[:, :, 27:].any()
    assert not got_n[:, :, :3].any() and not got_n[:, :, 27:].any()


def test_fixture_f32_input_f16_norms_seed1(golden, device):
    q = golden["quantize"]
    x = torch.from_numpy(q["x32_128"].reshape(1, 1, 40, 128)).to(device)
    codec = ops.Codec(128, 3, 1)
    packed, norms = _buffers(1, 1, 40, codec, torch.float16, device)
    ops.append_quantize(x, codec, packed, norms, 0)
    assert np.array_equal(_np_u32(packed)[0, 0], q["packed32_128_3_seed1"])
    assert np.array_equal(norms.cpu().numpy()[0, 0], q["norms16_128_3_seed1"])


def test_fixture_bf16_input_gaussian_codebook(golden, device):
    q = golden["quantize"]
    bits16 = torch.from_numpy(q["xbf16_bits_128"].astype(np.int16))
    x = bits16.view(torch.bfloat16).reshape(1, 1, 40, 128).to(device)
    codec = ops.Codec(128, 4, 0, codebook_kind="gaussian")
    packed, norms = _buffers(1, 1, 40, codec, torch.float32, device)
    ops.append_quantize(x, codec, packed, norms, 0)
    assert np.array_equal(_np_u32(packed)[0, 0], q["packedbf16_128_4_gauss"])
    assert np.array_equal(norms.cpu().numpy()[0, 0], q["normsbf16_128_4_gauss"])


def _synth(rng, shape, dtype):
    B, H, L, D = shape
    s = np.exp(rng.normal(0, 0.5, size=(1, H, 1, D)))
    return (rng.standard_normal(shape) * s).astype(np.float32), dtype


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("bits", [1, 2, 3, 4])
@pytest.mark.parametrize("norm_dtype", [torch.float32, torch.float16])
def test_random_batches_strided_input(device, dtype, bits, norm_dtype):
    rng = np.random.default_rng(bits * 10 + (dtype == torch.bfloat16))
    B, H, L, D = 2, 8, 37, 128
    x32, _ = _synth(rng, (B, H, L, D), dtype)
    # model layout (B, L, H, D) transposed to (B, H, L, D): non-contiguous view
    xt = torch.from_numpy(x32).to(dtype).transpose(1, 2).contiguous().transpose(1, 2).to(device)
    assert not xt.is_contiguous()
    xin = xt.float().cpu().numpy()
    codec = ops.Codec(D, bits, 5)
    packed, norms = _buffers(B, H, 64, codec, norm_dtype, device)
    ops.append_quantize(xt, codec, packed, norms, offset=11)
    nd = "float16" if norm_dtype == torch.float16 else "float32"
    wp, wn = O.quantize_rht(xin, bits, O.rht_signs(D, 5), O.beta_codebook(D, bits), nd)
    assert np.array_equal(_np_u32(packed)[:, :, 11:48], wp)
    assert np.array_equal(norms.float().cpu().numpy()[:, :, 11:48], wn)


def test_edge_vectors(device):
    D = 128
    x = np.zeros((1, 1, 6, D), np.float32)
    x[0, 0, 1] = 1e-30                           # subnormal-scale input, norm ~1e-29
    x[0, 0, 2, 5] = 3.0                          # one-hot
    x[0, 0, 3] = 60000.0                         # near f16 max
    x[0, 0, 4] = np.linspace(-1, 1, D)
    x[0, 0, 5, ::2] = -2.5
    for bits in (1, 2, 3, 4):
        codec = ops.Codec(D, bits, 0)
        packed, norms = _buffers(1, 1, 6, codec, torch.float32, device)
        ops.append_quantize(torch.from_numpy(x).to(device), codec, packed, norms, 0)
        wp, wn = O.quantize_rht(x, bits, O.rht_signs(D, 0), O.beta_codebook(D, bits))
        assert np.array_equal(_np_u32(packed), wp), bits
        assert np.array_equal(norms.cpu().numpy(), wn), bits


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_division_edge_vectors(device, dtype):
    # u = x / max(n, 1e-6) is formed from the reciprocal with one fma
    # refinement except where the quotient or its residual could leave the
    # normal range; these rows take each side of that switch and must stay
    # bit-exact with the IEEE division of the oracle.
    D = 128
    rng = np.random.default_rng(77)
    x = rng.standard_normal((1, 1, 8, D)).astype(np.float32)
    x[0, 0, 0, :4] = [1e-36, -3e-38, 5e-39, 0.0]   # tiny elements beside normal ones
    x[0, 0, 1] *= 1e30                             # squares overflow: inf norm
    x[0, 0, 2] = 1e-31                             # every element below 2^-100
    x[0, 0, 3, ::3] = 0.0                          # zeros between normal values
    x[0, 0, 4] *= 2.0 ** -90                       # small but on the fast side
    x[0, 0, 5] = 1.0                               # all equal: |x| / n = 2^-3.5
    x[0, 0, 6, 0] = 7.0                            # one-hot
    xt = torch.from_numpy(x).to(dtype)
    xin = xt.float().numpy()
    for bits in (1, 3, 4):
        codec = ops.Codec(D, bits, 2)
        packed, norms = _buffers(1, 1, 8, codec, torch.float32, device)
        ops.append_quantize(xt.to(device), codec, packed, norms, 0)
        with np.errstate(over="ignore", invalid="ignore"):  # row 1's squares overflow to an inf norm
            wp, wn = O.quantize_rht(xin, bits, O.rht_signs(D, 2), O.beta_codebook(D, bits))
        assert np.array_equal(_np_u32(packed), wp), (dtype, bits)
        assert np.array_equal(norms.cpu().numpy(), wn), (dtype, bits)


def test_config0_full_layer_bit_exact(device):
    """K and V f16 [1, 8, 4096, 128], per-channel log-normal scales, 3-bit."""
    rs, rk, rv = (np.random.default_rng(s) for s in (1000, 1001, 1002))
    scale = np.exp(rs.normal(0.0, 0.5, size=(1, 8, 1, 128)))
    k = (rk.standard_normal((1, 8, 4096, 128)) * scale).astype(np.float16)
    v = (rv.standard_normal((1, 8, 4096, 128)) * scale).astype(np.float16)
    for x, seed in ((k, 0), (v, 1)):
        codec = ops.Codec(128, 3, seed)
        packed, norms = _buffers(1, 8, 4096, codec, torch.float32, device)
        ops.append_quantize(torch.from_numpy(x).to(device), codec, packed, norms, 0)
        wp, wn = O.quantize_rht(x, 3, O.rht_signs(128, seed), O.beta_codebook(128, 3))
        gp = _np_u32(packed)
        mism = int((gp != wp).sum())
        assert mism == 0, f"{mism} packed words differ"
        assert np.array_equal(norms.cpu().numpy(), wn)
        # reconstruction quality (reference test: cosine > 0.85 at 3 bits)
        deq = ops.dequantize(packed, norms, codec).cpu().numpy().astype(np.float64)
        xf = x.astype(np.float64)
        cos = (deq * xf).sum(-1) / (np.linalg.norm(deq, axis=-1) * np.linalg.norm(xf, axis=-1))
        assert cos.mean() > 0.97


def _append_raw(x, bits, rot, mids, packed, norms, offset=0):
    """tq_append_quantize with caller-chosen sign vector and midpoints."""
    B, H, L, D = x.shape
    rc = _lib.load().tq_append_quantize(
        x.data_ptr(), _lib.torch_dtype_code(x.dtype), B, H, L, D,
        x.stride(0), x.stride(1), x.stride(2), bits, _lib.TQ_ROT_HADAMARD,
        rot.data_ptr(), mids.data_ptr(), packed.data_ptr(), norms.data_ptr(),
        _lib.torch_dtype_code(norms.dtype), packed.shape[2], offset, ops._stream(x))
    _lib.check(rc, "tq_append_quantize")


def _quantize_mids(x, bits, signs, mids):
    """The oracle's quantize with explicit midpoints."""
    xf = np.asarray(x, np.float32)
    n = O.norm_f32(xf)
    u = xf / np.maximum(n, O.EPS)[..., None]
    return O.pack_lowbit(O.quantize_indices(O.rht_forward_f32(u, signs), mids), bits), n


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("d", [64, 128, 256, 512])
def test_sign_vector_with_non_unit_entries(device, dtype, d):
    """Signs other than +-1 are multiplied after the division, as the oracle does."""
    rng = np.random.default_rng(d + 7)
    signs = O.rht_signs(d, 3).astype(np.float32)
    signs[rng.choice(d, 5, replace=False)] = np.array([0.5, -2.0, 0.0, -0.25, 3.0], np.float32)
    x = rng.standard_normal((1, 4, 70, d)).astype(np.float32)
    xt = torch.from_numpy(x).to(dtype)
    xin = xt.float().numpy()
    for bits in (2, 3, 4):
        mids = O.midpoints(O.beta_codebook(d, bits))
        codec = ops.Codec(d, bits, 3)
        packed, norms = _buffers(1, 4, 70, codec, torch.float32, device)
        _append_raw(xt.to(device), bits, torch.from_numpy(signs).to(device),
                    torch.from_numpy(mids).to(device), packed, norms)
        wp, wn = _quantize_mids(xin, bits, signs, mids)
        assert np.array_equal(_np_u32(packed), wp), bits
        assert np.array_equal(norms.cpu().numpy(), wn), bits


@pytest.mark.parametrize("bits", [3, 4])
def test_midpoints_sharing_a_table_cell(device, bits):
    """Two midpoints closer than a table cell: the kernel compares against every midpoint.

    Also midpoints at 0 and at +-tiny values, and inputs whose coordinates land on
    midpoints exactly (one-hot vectors put +-1/sqrt(D) on every coordinate)."""
    d = 128
    rng = np.random.default_rng(bits)
    nm = (1 << bits) - 1
    base = np.sort(rng.uniform(-0.25, 0.25, nm)).astype(np.float32)
    close = base.copy()
    close[nm // 2] = np.float32(1e-7)
    close[nm // 2 + 1] = np.float32(3e-7)
    exact = base.copy()
    exact[nm // 2] = np.float32(0.0)
    exact[nm // 2 - 1] = -O.rht_scale(d)
    exact[nm // 2 + 1] = O.rht_scale(d)
    exact = np.sort(exact).astype(np.float32)
    x = rng.standard_normal((1, 2, 64, d)).astype(np.float32)
    x[0, 0, :8] = 0.0
    for j in range(8):
        x[0, 0, j, 3 * j] = 1.0 + j
    x[0, 1, 0] = 0.0
    signs = O.rht_signs(d, 1)
    for mids in (np.sort(close), exact):
        mids = mids.astype(np.float32)
        codec = ops.Codec(d, bits, 1)
        packed, norms = _buffers(1, 2, 64, codec, torch.float32, device)
        xt = torch.from_numpy(x).to(torch.float16)
        _append_raw(xt.to(device), bits, torch.from_numpy(signs).to(device),
                    torch.from_numpy(mids).to(device), packed, norms)
        wp, wn = _quantize_mids(xt.float().numpy(), bits, signs, mids)
        assert np.array_equal(_np_u32(packed), wp)
        assert np.array_equal(norms.cpu().numpy(), wn)


@pytest.mark.parametrize("d", [32, 64, 128, 256, 512])
def test_whole_row_blocks_batched(device, d):
    """L a multiple of every block size (the row indices are then the block's):
    several (b, h) rows, model-layout strides, an offset inside the capacity."""
    rng = np.random.default_rng(d + 3)
    B, H, L, bits = 2, 3, 256, 3
    x32, _ = _synth(rng, (B, H, L, d), torch.float16)
    xt = torch.from_numpy(x32).to(torch.float16).transpose(1, 2).contiguous().transpose(1, 2).to(device)
    codec = ops.Codec(d, bits, 4)
    packed, norms = _buffers(B, H, L + 9, codec, torch.float32, device)
    ops.append_quantize(xt, codec, packed, norms, offset=7)
    wp, wn = O.quantize_rht(xt.float().cpu().numpy(), bits, O.rht_signs(d, 4), O.beta_codebook(d, bits))
    gp = _np_u32(packed)
    assert np.array_equal(gp[:, :, 7:7 + L], wp)
    assert np.array_equal(norms.cpu().numpy()[:, :, 7:7 + L], wn)
    assert not gp[:, :, :7].any() and not gp[:, :, 7 + L:].any()


@pytest.mark.parametrize("d,bits", [(64, 2), (128, 3), (256, 4)])
def test_dequantize_matches_oracle(device, d, bits):
    rng = np.random.default_rng(d)
    x = rng.standard_normal((2, 3, 9, d)).astype(np.float32)
    codec = ops.Codec(d, bits, 0)
    packed, norms = _buffers(2, 3, 16, codec, torch.float32, device)
    ops.append_quantize(torch.from_numpy(x).to(device), codec, packed, norms, 0)
    got = ops.dequantize(packed[:, :, :9], norms[:, :, :9], codec).cpu().numpy()
    want = O.dequantize(_np_u32(packed[:, :, :9]), norms[:, :, :9].cpu().numpy(), bits, d,
                        O.beta_codebook(d, bits), "hadamard", O.rht_signs(d, 0))
    np.testing.assert_allclose(got, want, atol=1e-5)


@pytest.mark.parametrize("d", [128, 100, 13])
def test_plain_append_copies_rows(device, d):
    """16-byte copies for dims that are multiples of 8, single elements otherwise."""
    x = torch.randn(2, 4, 5, d, dtype=torch.float16, device=device)
    dst = torch.zeros(2, 4, 16, d, dtype=torch.float16, device=device)
    ops.append_plain(x.transpose(1, 2).contiguous().transpose(1, 2), dst, 7)
    assert torch.equal(dst[:, :, 7:12], x)
    assert not dst[:, :, :7].any() and not dst[:, :, 12:].any()


@pytest.mark.parametrize("d,kb,vb,dtype", [
    (128, 3, 3, torch.float16),    # config 0: one paired launch
    (64, 1, 2, torch.bfloat16),    # x.5-bit split (values one bit wider), paired
    (256, 4, 4, torch.float16),
    (128, 2, 3, torch.bfloat16),
    (128, 4, 3, torch.float16),    # keys wider: two launches
    (128, 3, 3, torch.float32),    # f32 input: two launches
    (512, 2, 2, torch.float16),    # dim outside the paired set: two launches
])
@pytest.mark.parametrize("norm_dtype", [torch.float32, torch.float16])
def test_key_value_pair_append(device, d, kb, vb, dtype, norm_dtype):
    """tq_append_quantize_kv: both sides bit-exact against the oracle, strided
    inputs, an offset inside the capacity, untouched rows around it."""
    rng = np.random.default_rng(d + 10 * kb + vb)
    B, H, L = 2, 4, 29
    k32, _ = _synth(rng, (B, H, L, d), dtype)
    v32, _ = _synth(rng, (B, H, L, d), dtype)
    ks = torch.from_numpy(k32).to(dtype).transpose(1, 2).contiguous().transpose(1, 2).to(device)
    vs = torch.from_numpy(v32).to(dtype).to(device)
    kc, vc = ops.Codec(d, kb, 0), ops.Codec(d, vb, 1)
    kp, kn = _buffers(B, H, 40, kc, norm_dtype, device)
    vp, vn = _buffers(B, H, 40, vc, norm_dtype, device)
    ops.append_quantize_kv(ks, vs, kc, vc, kp, kn, vp, vn, 5)
    nd = "float16" if norm_dtype == torch.float16 else "float32"
    for x, p, n, bits, seed in ((ks, kp, kn, kb, 0), (vs, vp, vn, vb, 1)):
        wp, wn = O.quantize_rht(x.float().cpu().numpy(), bits, O.rht_signs(d, seed),
                                O.beta_codebook(d, bits), nd)
        gp, gn = _np_u32(p), n.float().cpu().numpy()
        assert np.array_equal(gp[:, :, 5:5 + L], wp), (d, kb, vb, seed)
        assert np.array_equal(gn[:, :, 5:5 + L], wn), (d, kb, vb, seed)
        assert not gp[:, :, :5].any() and not gp[:, :, 5 + L:].any()
        assert not gn[:, :, :5].any() and not gn[:, :, 5 + L:].any()


def test_key_value_pair_append_dense_rotation(device):
    """Dense rotation goes through the two matrix-core launches: identical to
    two single-side calls."""
    rng = np.random.default_rng(77)
    B, H, L, d = 1, 4, 40, 128
    k = torch.from_numpy(rng.standard_normal((B, H, L, d)).astype(np.float32)).half().to(device)
    v = torch.from_numpy(rng.standard_normal((B, H, L, d)).astype(np.float32)).half().to(device)
    kc, vc = ops.Codec(d, 3, 0, "dense"), ops.Codec(d, 4, 1, "dense")
    a = [_buffers(B, H, 48, c, torch.float32, device) for c in (kc, vc)]
    b = [_buffers(B, H, 48, c, torch.float32, device) for c in (kc, vc)]
    ops.append_quantize_kv(k, v, kc, vc, a[0][0], a[0][1], a[1][0], a[1][1], 3)
    ops.append_quantize(k, kc, b[0][0], b[0][1], 3)
    ops.append_quantize(v, vc, b[1][0], b[1][1], 3)
    for (p1, n1), (p2, n2) in zip(a, b):
        assert torch.equal(p1, p2) and torch.equal(n1, n2)
