"""GPU parity of the dense-rotation append (matrix-core kernel) vs the oracle.

Bar: norms bit-exact; packed indices equal to the oracle's except where the
oracle's rotated coordinate y lies within BAND of a midpoint.  The oracle's y
is the f32 rounding of the exact product u @ R^T (u = x / max(n, 1e-6) in f32);
the kernel sums bf16 piece products in f32 on the matrix cores and compares
x @ R^T against mid * max(n, 1e-6), so its y differs from the oracle's by a
few f32 ulps at most.  For unit vectors |y| <= 1 and every partial sum is
bounded by 1, so an absolute band of 2^-20 (16 ulps of 1.0) holds the
worst case with margin.  Flips inside the band must also move the index by
exactly one step.  Anything outside the band is a real error.
"""
import numpy as np
import pytest
import torch

from oracle import tq_oracle as O
from kaplumba_amd import _lib, ops

pytestmark = pytest.mark.gpu

BAND = 2.0 ** -20


def _buffers(B, H, cap, codec, norm_dtype, device):
    packed = torch.zeros((B, H, cap, codec.packed_width), dtype=torch.uint32, device=device)
    norms = torch.zeros((B, H, cap), dtype=norm_dtype, device=device)
    return packed, norms


def _synth(rng, shape):
    B, H, L, D = shape
    s = np.exp(rng.normal(0, 0.5, size=(1, H, 1, D)))
    return (rng.standard_normal(shape) * s).astype(np.float32)


def _check(x_in, bits, d, seed, got_packed, got_norms, norm_dtype="float32", kind="beta"):
    """Compare kernel output with the oracle; returns the number of band flips."""
    cb = O.beta_codebook(d, bits) if kind == "beta" else O.gaussian_codebook(d, bits)
    wp, wn, y = O.quantize_dense(x_in, bits, O.rotation_matrix(d, seed), cb, norm_dtype)
    assert np.array_equal(got_norms, wn), "norms differ"
    gi = O.unpack_lowbit(got_packed, bits, d).astype(np.int64)
    wi = O.unpack_lowbit(wp, bits, d).astype(np.int64)
    bad = gi != wi
    if bad.any():
        mids = O.midpoints(cb).astype(np.float64)
        dist = np.abs(y[bad].astype(np.float64)[:, None] - mids[None, :]).min(axis=1)
        assert dist.max() <= BAND, f"index differs {dist.max():.3g} away from a midpoint"
        assert np.abs(gi[bad] - wi[bad]).max() == 1
    return int(bad.sum())


@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("bits", [1, 2, 3, 4])
def test_dense_bf16_matches_oracle(device, d, bits):
    rng = np.random.default_rng(100 * d + bits)
    B, H, L = 2, 3, 45   # 270 vectors: a full 256-vector tile plus a ragged one
    x32 = _synth(rng, (B, H, L, d))
    x = torch.from_numpy(x32).to(torch.bfloat16).to(device)
    codec = ops.Codec(d, bits, 0, rotation="dense")
    packed, norms = _buffers(B, H, 60, codec, torch.float32, device)
    ops.append_quantize(x, codec, packed, norms, offset=7)
    gp = packed.cpu().numpy().astype(np.uint32)
    gn = norms.cpu().numpy()
    flips = _check(x.float().cpu().numpy(), bits, d, 0, gp[:, :, 7:52], gn[:, :, 7:52])
    assert flips <= 2
    assert not gp[:, :, :7].any() and not gp[:, :, 52:].any()
    assert not gn[:, :, :7].any() and not gn[:, :, 52:].any()


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("d,bits", [(64, 4), (128, 3), (256, 2)])
@pytest.mark.parametrize("norm_dtype", [torch.float32, torch.float16])
def test_dense_f16_f32_inputs_strided(device, dtype, d, bits, norm_dtype):
    rng = np.random.default_rng(d + bits + (dtype == torch.float32))
    B, H, L = 1, 4, 70
    x32 = _synth(rng, (B, H, L, d))
    # (B, L, H, D) storage viewed as (B, H, L, D): the model's layout
    xt = torch.from_numpy(x32).to(dtype).transpose(1, 2).contiguous().transpose(1, 2).to(device)
    assert not xt.is_contiguous()
    codec = ops.Codec(d, bits, 1, rotation="dense")
    packed, norms = _buffers(B, H, 80, codec, norm_dtype, device)
    ops.append_quantize(xt, codec, packed, norms, offset=5)
    nd = "float16" if norm_dtype == torch.float16 else "float32"
    flips = _check(xt.float().cpu().numpy(), bits, d, 1,
                   packed.cpu().numpy().astype(np.uint32)[:, :, 5:75],
                   norms.float().cpu().numpy()[:, :, 5:75], nd)
    assert flips <= 2


def test_dense_edge_vectors(device):
    d = 128
    x = np.zeros((1, 1, 6, d), np.float32)
    x[0, 0, 1] = 1e-30                   # norm far below eps: u = x / 1e-6
    x[0, 0, 2, 5] = 3.0                  # one-hot: y is a column of R
    x[0, 0, 3] = 60000.0                 # near f16 max
    x[0, 0, 4] = np.linspace(-1, 1, d)
    x[0, 0, 5, ::2] = -2.5
    for bits in (1, 2, 3, 4):
        codec = ops.Codec(d, bits, 0, rotation="dense")
        packed, norms = _buffers(1, 1, 6, codec, torch.float32, device)
        ops.append_quantize(torch.from_numpy(x).to(device), codec, packed, norms, 0)
        flips = _check(x, bits, d, 0, packed.cpu().numpy().astype(np.uint32), norms.cpu().numpy())
        assert flips == 0, bits
        # the zero vector maps every coordinate to #{mid < 0}
        idx0 = O.unpack_lowbit(packed.cpu().numpy().astype(np.uint32)[0, 0, 0], bits, d)
        assert (idx0 == int((O.midpoints(O.beta_codebook(d, bits)) < 0).sum())).all()


def test_dense_power_of_two_scaling_invariance(device):
    """Scaling x by 2^k scales every product exactly: same indices, norm * 2^k."""
    rng = np.random.default_rng(5)
    x = _synth(rng, (1, 8, 300, 128))
    codec = ops.Codec(128, 3, 0, rotation="dense")
    outs = []
    for k in (0, 7, -9):
        packed, norms = _buffers(1, 8, 300, codec, torch.float32, device)
        ops.append_quantize(torch.from_numpy(x * np.float32(2.0 ** k)).to(device), codec, packed, norms, 0)
        outs.append((packed.cpu().numpy(), norms.cpu().numpy() / np.float32(2.0 ** k)))
    for p, n in outs[1:]:
        assert np.array_equal(p, outs[0][0])
        assert np.array_equal(n, outs[0][1])


def test_dense_config3_layer(device):
    """Config 3's per-layer append: bf16 K [1, 8, 8192, 128], dense 128x128, 3-bit."""
    rs, rk = np.random.default_rng(1000), np.random.default_rng(1001)
    scale = np.exp(rs.normal(0.0, 0.5, size=(1, 8, 1, 128)))
    k = torch.from_numpy((rk.standard_normal((1, 8, 8192, 128)) * scale).astype(np.float32))
    kb = k.to(torch.bfloat16)
    codec = ops.Codec(128, 3, 0, rotation="dense")
    packed, norms = _buffers(1, 8, 8192, codec, torch.float32, device)
    ops.append_quantize(kb.to(device), codec, packed, norms, 0)
    xin = kb.float().numpy()
    flips = _check(xin, 3, 128, 0, packed.cpu().numpy().astype(np.uint32), norms.cpu().numpy())
    assert flips <= 8   # of 8.4M coordinates
    deq = ops.dequantize(packed, norms, codec).cpu().numpy().astype(np.float64)
    xf = xin.astype(np.float64)
    cos = (deq * xf).sum(-1) / (np.linalg.norm(deq, axis=-1) * np.linalg.norm(xf, axis=-1))
    assert cos.mean() > 0.97


@pytest.mark.parametrize("scale", [1.0, 300.0, 2.0 ** -13, 3e4])
def test_dense_f16_rotation_of_any_scale(device, scale):
    """f16 input runs f16 products against a power-of-two-scaled split of R: any
    magnitude of R gives the oracle's indices (band scaled with R)."""
    d, bits = 128, 3
    rng = np.random.default_rng(int(scale * 7) % 1000)
    R = (O.rotation_matrix(d, 2) * np.float32(scale)).astype(np.float32)
    R[3, 5] = np.float32(scale * 0.9)   # one large entry next to small ones
    x = _synth(rng, (1, 4, 96, d)).astype(np.float16)
    cb = O.beta_codebook(d, bits)
    mids = O.midpoints(cb)
    codec = ops.Codec(d, bits, 0, rotation="dense")
    packed, norms = _buffers(1, 4, 96, codec, torch.float32, device)
    xt = torch.from_numpy(x).to(device)
    rt = torch.from_numpy(R).to(device)
    mt = torch.from_numpy(mids).to(device)
    rc = _lib.load().tq_append_quantize(
        xt.data_ptr(), _lib.torch_dtype_code(xt.dtype), 1, 4, 96, d,
        xt.stride(0), xt.stride(1), xt.stride(2), bits, _lib.TQ_ROT_DENSE,
        rt.data_ptr(), mt.data_ptr(),
        packed.data_ptr(), norms.data_ptr(), _lib.torch_dtype_code(norms.dtype), 96, 0, ops._stream(xt))
    _lib.check(rc, "tq_append_quantize")
    torch.cuda.synchronize()
    wp, wn, y = O.quantize_dense(x.astype(np.float32), bits, R, cb)
    assert np.array_equal(norms.cpu().numpy(), wn)
    gi = O.unpack_lowbit(packed.cpu().numpy().astype(np.uint32), bits, d).astype(np.int64)
    wi = O.unpack_lowbit(wp, bits, d).astype(np.int64)
    bad = gi != wi
    if bad.any():
        dist = np.abs(y[bad].astype(np.float64)[:, None] - mids.astype(np.float64)[None, :]).min(axis=1)
        assert dist.max() <= BAND * max(1.0, scale)
        assert np.abs(gi[bad] - wi[bad]).max() == 1
    assert int(bad.sum()) <= 2


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_dense_whole_tiles_batched(device, dtype):
    """L a multiple of the 256-vector tile (the row indices are then the tile's):
    several (b, h) rows, model-layout strides, an offset inside the capacity."""
    rng = np.random.default_rng(17)
    B, H, L, d, bits = 2, 3, 512, 128, 3
    x = _synth(rng, (B, H, L, d))
    xt = torch.from_numpy(x).to(dtype).transpose(1, 2).contiguous().transpose(1, 2).to(device)
    codec = ops.Codec(d, bits, 0, rotation="dense")
    packed, norms = _buffers(B, H, L + 5, codec, torch.float32, device)
    ops.append_quantize(xt, codec, packed, norms, 3)
    gp = packed.cpu().numpy().astype(np.uint32)
    flips = _check(xt.float().cpu().numpy(), bits, d, 0, gp[:, :, 3:3 + L], norms.cpu().numpy()[:, :, 3:3 + L])
    assert flips <= 2
    assert not gp[:, :, :3].any() and not gp[:, :, 3 + L:].any()
