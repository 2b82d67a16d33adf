"""Pin the CPU oracle (oracle/tq_oracle.py) to independent facts.

Each check is chosen so that a plausible slip in the restatement (a dropped
term, a wrong sign or index, a transposed operand, a wrong stage order) fails
it: closed forms (Sylvester Hadamard from scipy), published tables (Max 1960),
float64 quadrature of the Beta density, brute-force nearest-centroid search,
hand-computed packed words, and torch SDPA on the dequantized cache.
"""
import math

import numpy as np
import pytest
import torch

from oracle import tq_oracle as O


# ------------------------------------------------------------------ signs ---
def test_sign_vector_known_prefix():
    # numpy PCG64 stream for default_rng(0 + 128*7919).choice([-1, 1]), the
    # reference's seeding (turboquant_cache.py:3545-3546).
    want = [-1, -1, -1, -1, 1, -1, -1, -1, -1, 1, -1, -1, 1, 1, -1, -1]
    assert O.rht_signs(128, 0)[:16].tolist() == want
    s = O.rht_signs(256, 1)
    assert s.dtype == np.float32 and set(np.unique(s)) == {-1.0, 1.0}
    assert not np.array_equal(O.rht_signs(128, 0), O.rht_signs(128, 1))


# --------------------------------------------------------------- rotation ---
@pytest.mark.parametrize("d", [64, 128, 256])
def test_rotation_orthogonal_and_sign_fixed(d):
    R = O.rotation_matrix(d, 0).astype(np.float64)
    assert np.abs(R.T @ R - np.eye(d)).max() < 2e-5
    assert abs(abs(np.linalg.det(R)) - 1.0) < 1e-3
    # sign fix: Q' = Q diag(sign(diag r)) makes diag(Q'^T M) = |diag r| > 0
    M = np.random.default_rng(0 + d * 7919).standard_normal((d, d), dtype=np.float32)
    U = R.T @ M.astype(np.float64)
    assert (np.diag(U) > 0).all()
    # R is the Q factor of exactly that draw: R^T M is upper triangular (a
    # transposed R, another seed, or a missing sign fix all leave a full or
    # negative-diagonal product)
    assert np.abs(np.tril(U, -1)).max() < 1e-3 * np.abs(U).max()
    assert np.abs(np.triu(U)).max() > 1.0


# --------------------------------------------------------------- codebooks ---
MAX_1960 = {
    1: [0.7979],
    2: [0.4528, 1.5104],
    3: [0.2451, 0.7560, 1.3440, 2.1520],
    4: [0.1284, 0.3881, 0.6568, 0.9424, 1.2562, 1.6181, 2.0690, 2.7326],
}


@pytest.mark.parametrize("bits", [1, 2, 3, 4])
def test_gaussian_lloyd_max_matches_published_table(bits):
    c = O.gaussian_lloyd_max(bits)
    pos = c[len(c) // 2:]
    np.testing.assert_allclose(pos, MAX_1960[bits], atol=6e-4)
    np.testing.assert_allclose(c, -c[::-1], atol=1e-12)


def _beta_cell_mean(d, a, b):
    from scipy.integrate import quad
    from scipy.special import gammaln

    logc = gammaln(d / 2) - 0.5 * math.log(math.pi) - gammaln((d - 1) / 2)
    pdf = lambda x: math.exp(logc + (d - 3) / 2 * math.log(max(1 - x * x, 1e-300)))
    m0 = quad(pdf, a, b, limit=200)[0]
    m1 = quad(lambda x: x * pdf(x), a, b, limit=200)[0]
    return m1 / m0


@pytest.mark.parametrize("d,bits", [(64, 2), (128, 3), (128, 4), (256, 2)])
def test_beta_codebook_centroid_condition(d, bits):
    """Each level is (close to) the conditional mean of its cell under the exact pdf.

    The reference stops after at most 100 Lloyd iterations on a 32768-point
    grid, so the 16-level books sit ~0.3% of a cell away from the fixed point;
    a wrong density exponent ((d-1)/2 instead of (d-3)/2) moves levels ~9%.
    """
    c = O.beta_codebook(d, bits).astype(np.float64)
    edges = np.concatenate([[-1.0], 0.5 * (c[:-1] + c[1:]), [1.0]])
    means = np.array([_beta_cell_mean(d, edges[i], edges[i + 1]) for i in range(len(c))])
    spacing = np.diff(c).min()
    assert np.abs(means - c).max() < 1e-2 * spacing


def test_beta_codebook_matches_survey_probe_and_gaussian_shape():
    c = O.beta_codebook(128, 3) * math.sqrt(128)
    np.testing.assert_allclose(
        c, [-2.1302, -1.3352, -0.7521, -0.2443, 0.2433, 0.7515, 1.3345, 2.1296], atol=2e-4)
    for d, b in [(128, 1), (128, 2), (256, 3), (256, 4)]:
        cb = O.beta_codebook(d, b) * math.sqrt(d)
        g = O.gaussian_lloyd_max(b)
        assert np.all(np.diff(cb) > 0)
        assert np.abs(cb - g).max() / np.abs(g).max() < 0.03
    # centre midpoints of the slightly asymmetric f32 solution
    assert abs(O.midpoints(O.beta_codebook(128, 3))[3] - (-4.54681e-05)) < 1e-10
    assert O.midpoints(O.beta_codebook(128, 1))[0] == 0.0


# ---------------------------------------------------------------- Hadamard ---
@pytest.mark.parametrize("d", [32, 64, 128, 256, 512])
def test_fwht_matches_sylvester_closed_form(d):
    from scipy.linalg import hadamard

    x = np.random.default_rng(d).standard_normal((5, d)).astype(np.float32)
    want = x.astype(np.float64) @ hadamard(d).T
    got = O.fwht_f32(x)
    assert np.abs(got - want).max() < 1e-5 * math.sqrt(d) * np.abs(x).max()


def test_fwht_planted_mistake_is_caught():
    """A butterfly with (a+b, b-a) instead of (a+b, a-b) must fail the closed form."""
    from scipy.linalg import hadamard

    def bad(v):
        v = v.copy()
        d = v.shape[-1]
        h = 1
        while h < d:
            w = v.reshape(-1, d // (2 * h), 2, h)
            a, b = w[:, :, 0, :], w[:, :, 1, :]
            v = np.stack([a + b, b - a], axis=2).reshape(-1, d)
            h *= 2
        return v

    x = np.random.default_rng(3).standard_normal((2, 64)).astype(np.float32)
    assert np.abs(bad(x) - x @ hadamard(64).T).max() > 1.0


@pytest.mark.parametrize("d", [64, 128, 256])
def test_rht_round_trip_and_basis_vector(d):
    s = O.rht_signs(d, 0)
    x = np.random.default_rng(1).standard_normal((4, d)).astype(np.float32)
    np.testing.assert_allclose(O.rht_inverse_f32(O.rht_forward_f32(x, s), s), x, atol=1e-5)
    np.testing.assert_allclose(O.rht_forward_f32(x, s), O.rht_forward_f64(x, s), atol=1e-5)
    e0 = np.zeros(d, np.float32)
    e0[0] = 1.0
    y = O.rht_forward_f32(e0, s)
    assert np.all(y == s[0] * np.float32(1.0 / math.sqrt(d)))


# -------------------------------------------------------------------- norm ---
def _norm_scalar_tree(x):
    """The append kernel's reduction written out with scalar f32 arithmetic."""
    f = np.float32
    d = len(x)
    lanes = []
    for g in range(max(1, d // 32)):
        s = [f(x[32 * g + i]) * f(x[32 * g + i]) for i in range(min(32, d))]
        w = len(s) // 2
        while w >= 1:
            s = [f(s[i] + s[i + w]) for i in range(w)]
            w //= 2
        lanes.append(s[0])
    while len(lanes) > 1:
        lanes = [f(lanes[i] + lanes[i + 1]) for i in range(0, len(lanes), 2)]
    return f(np.sqrt(lanes[0]))


@pytest.mark.parametrize("d", [32, 128, 256])
def test_norm_tree_order_and_accuracy(d):
    x = (np.random.default_rng(d).standard_normal((6, d)) * 3).astype(np.float32)
    got = O.norm_f32(x)
    for i in range(6):
        assert got[i] == _norm_scalar_tree(x[i])
    np.testing.assert_allclose(got, np.linalg.norm(x.astype(np.float64), axis=-1), rtol=1e-6)
    v = np.zeros(d, np.float32)
    v[:2] = [3, 4]
    assert O.norm_f32(v) == 5.0


# ---------------------------------------------------------------- quantize ---
@pytest.mark.parametrize("bits", [1, 2, 3, 4])
def test_indices_match_brute_force_nearest_centroid(bits):
    cb = O.beta_codebook(128, bits)
    y = (np.random.default_rng(bits).standard_normal(20000) / math.sqrt(128)).astype(np.float32)
    idx = O.quantize_indices(y, O.midpoints(cb))
    dist = np.abs(y[:, None].astype(np.float64) - cb[None, :].astype(np.float64))
    near = dist.argmin(axis=1)
    mids = O.midpoints(cb).astype(np.float64)
    clear = np.abs(y[:, None] - mids[None, :]).min(axis=1) > 1e-7
    assert np.array_equal(idx[clear], near[clear])


def test_strict_compare_tie_goes_low():
    cb = O.beta_codebook(128, 2)
    m = O.midpoints(cb)
    idx = O.quantize_indices(m, m)  # y exactly at each midpoint
    assert idx.tolist() == [0, 1, 2]


@pytest.mark.parametrize("d,bits,want", [(128, 1, 0), (128, 2, 2), (128, 3, 4), (128, 4, 8),
                                         (256, 1, 1), (256, 3, 3), (256, 4, 7)])
def test_zero_vector_indices(d, bits, want):
    # the f32 Beta codebooks are not exactly symmetric, so 0.0 lands on the
    # side of the centre midpoint's sign (documented in the survey)
    p, n = O.quantize_rht(np.zeros((1, d), np.float32), bits, O.rht_signs(d, 0),
                          O.beta_codebook(d, bits))
    assert n[0] == 0.0
    assert np.all(O.unpack_lowbit(p, bits, d) == want)


@pytest.mark.parametrize("d,bits", [(64, 3), (128, 2), (256, 4)])
def test_quantize_against_float64_pipeline(d, bits):
    x = np.random.default_rng(d + bits).standard_normal((64, d)).astype(np.float32)
    s = O.rht_signs(d, 0)
    cb = O.beta_codebook(d, bits)
    p, n = O.quantize_rht(x, bits, s, cb)
    u = x.astype(np.float64) / np.linalg.norm(x.astype(np.float64), axis=-1, keepdims=True)
    y = O.rht_forward_f64(u, s)
    near = np.abs(y[..., None] - cb.astype(np.float64)).argmin(-1)
    mids = O.midpoints(cb).astype(np.float64)
    clear = np.abs(y[..., None] - mids).min(-1) > 1e-6
    got = O.unpack_lowbit(p, bits, d)
    assert np.array_equal(got[clear], near[clear])
    assert clear.mean() > 0.99


# ------------------------------------------------------------------ packing ---
def test_pack_hand_computed_words():
    codes = np.zeros((1, 32), np.uint32)
    codes[0, :8] = np.arange(8)
    w = O.pack_lowbit(codes, 3)
    assert w.shape == (1, 3) and w[0, 0] == 0x00FAC688 and w[0, 1] == 0 and w[0, 2] == 0
    codes = np.zeros((1, 32), np.uint32)
    codes[0, 10] = 7  # bits 30..32 straddle words 0 and 1
    w = O.pack_lowbit(codes, 3)
    assert w[0, 0] == 0xC0000000 and w[0, 1] == 1


@pytest.mark.parametrize("bits", [1, 2, 3, 4])
@pytest.mark.parametrize("d", [64, 128, 256])
def test_pack_matches_bigint_and_round_trips(bits, d):
    rng = np.random.default_rng(bits * d)
    codes = rng.integers(0, 1 << bits, size=(7, d)).astype(np.uint32)
    w = O.pack_lowbit(codes, bits)
    assert w.shape == (7, (d * bits + 31) // 32)
    for r in range(7):
        big = sum(int(c) << (i * bits) for i, c in enumerate(codes[r]))
        want = [(big >> (32 * k)) & 0xFFFFFFFF for k in range(w.shape[1])]
        assert w[r].tolist() == want
    assert np.array_equal(O.unpack_lowbit(w, bits, d), codes)


# ---------------------------------------------------------------- attention ---
def _attn_case(rng, B, Hq, Hkv, L, T, d, kb, vb, rot):
    k = rng.standard_normal((B, Hkv, T, d)).astype(np.float32)
    v = rng.standard_normal((B, Hkv, T, d)).astype(np.float32)
    if rot == "hadamard":
        kr, vr = O.rht_signs(d, 0), O.rht_signs(d, 1)
        kp, kn = O.quantize_rht(k, kb, kr, O.beta_codebook(d, kb))
        vp, vn = O.quantize_rht(v, vb, vr, O.beta_codebook(d, vb))
    else:
        kr, vr = O.rotation_matrix(d, 0), O.rotation_matrix(d, 1)
        kp, kn, _ = O.quantize_dense(k, kb, kr, O.beta_codebook(d, kb))
        vp, vn, _ = O.quantize_dense(v, vb, vr, O.beta_codebook(d, vb))
    q = O.round_to_dtype(rng.standard_normal((B, Hq, L, d)).astype(np.float32), "bf16")
    return q, kp, kn, vp, vn, kr, vr


@pytest.mark.parametrize("rot", ["hadamard", "dense"])
def test_attention_equals_sdpa_on_dequantized_cache(rot):
    rng = np.random.default_rng(11)
    B, Hq, Hkv, L, T, d, kb, vb = 2, 4, 2, 3, 40, 64, 3, 2
    q, kp, kn, vp, vn, kr, vr = _attn_case(rng, B, Hq, Hkv, L, T, d, kb, vb, rot)
    scale = 1 / math.sqrt(d)
    got = O.attention(q, kp, kn, vp, vn, k_bits=kb, v_bits=vb, k_codebook=O.beta_codebook(d, kb),
                      v_codebook=O.beta_codebook(d, vb), rot_kind=rot, k_rot=kr, v_rot=vr,
                      scale=scale, q_dtype="bf16", causal=True)
    K = O.dequantize(kp, kn, kb, d, O.beta_codebook(d, kb), rot, kr)
    V = O.dequantize(vp, vn, vb, d, O.beta_codebook(d, vb), rot, vr)
    qs = O.scale_queries(q, scale, "bf16").astype(np.float64)
    R = Hq // Hkv
    Kt = torch.from_numpy(K).repeat_interleave(R, dim=1)
    Vt = torch.from_numpy(V).repeat_interleave(R, dim=1)
    mask = torch.arange(T)[None, :] <= (T - L + torch.arange(L))[:, None]
    want = torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(qs), Kt, Vt, attn_mask=mask, scale=1.0).numpy()
    np.testing.assert_allclose(got, want, atol=1e-9)


def test_decode_is_last_causal_row_and_f32_chunked_agrees():
    rng = np.random.default_rng(12)
    B, Hq, Hkv, L, T, d, kb, vb = 1, 8, 2, 4, 300, 128, 3, 3
    q, kp, kn, vp, vn, kr, vr = _attn_case(rng, B, Hq, Hkv, L, T, d, kb, vb, "hadamard")
    kw = dict(k_bits=kb, v_bits=vb, k_codebook=O.beta_codebook(d, kb),
              v_codebook=O.beta_codebook(d, vb), rot_kind="hadamard", k_rot=kr, v_rot=vr,
              scale=1 / math.sqrt(d), q_dtype="bf16")
    full = O.attention(q, kp, kn, vp, vn, causal=True, **kw)
    last = O.attention(q[:, :, -1:], kp, kn, vp, vn, causal=False, **kw)
    np.testing.assert_allclose(full[:, :, -1:], last, atol=1e-12)
    f32 = O.attention_chunked_f32(q, kp, kn, vp, vn, k_bits=kb, v_bits=vb,
                                  k_codebook=O.beta_codebook(d, kb), v_codebook=O.beta_codebook(d, vb),
                                  signs_k=kr, signs_v=vr, scale=1 / math.sqrt(d), q_dtype="bf16",
                                  causal=True, key_chunk=128)
    np.testing.assert_allclose(f32, full, atol=2e-5)


@pytest.mark.parametrize("kb,vb", [(3, 3), (2, 1), (4, 2), (1, 4)])
def test_torch_cpu_baseline_equals_float64_oracle(kb, vb):
    """The multi-threaded CPU baseline computes the oracle's attention."""
    from oracle import tq_oracle_torch as OT

    rng = np.random.default_rng(20 + kb)
    B, Hq, Hkv, L, T, d = 1, 8, 2, 1, 3000, 128
    q, kp, kn, vp, vn, kr, vr = _attn_case(rng, B, Hq, Hkv, L, T, d, kb, vb, "hadamard")
    kw = dict(k_bits=kb, v_bits=vb, k_codebook=O.beta_codebook(d, kb),
              v_codebook=O.beta_codebook(d, vb), scale=1 / math.sqrt(d), q_dtype="bf16")
    want = O.attention(q, kp, kn, vp, vn, rot_kind="hadamard", k_rot=kr, v_rot=vr, **kw)
    got = OT.attention_chunked(q, kp, kn, vp, vn, signs_k=kr, signs_v=vr, key_chunk=1024, **kw)
    np.testing.assert_allclose(got, want, atol=2e-6)
    # the unpack agrees with the big-integer restatement's inverse on random words
    words = rng.integers(0, 2 ** 32, size=(4, O.packed_width(d, kb)), dtype=np.uint64).astype(np.uint32)
    np.testing.assert_array_equal(
        OT.unpack_lowbit(torch.from_numpy(words.astype(np.int64)), kb, d).numpy(),
        O.unpack_lowbit(words, kb, d))


def test_ragged_lengths_equal_truncated_cache():
    rng = np.random.default_rng(13)
    B, Hq, Hkv, L, T, d = 2, 4, 2, 1, 50, 64
    q, kp, kn, vp, vn, kr, vr = _attn_case(rng, B, Hq, Hkv, L, T, d, 2, 2, "hadamard")
    kw = dict(k_bits=2, v_bits=2, k_codebook=O.beta_codebook(d, 2), v_codebook=O.beta_codebook(d, 2),
              rot_kind="hadamard", k_rot=kr, v_rot=vr, scale=0.125, q_dtype="bf16")
    rag = O.attention(q, kp, kn, vp, vn, lengths=[20, 50], **kw)
    cut = O.attention(q[:1], kp[:1, :, :20], kn[:1, :, :20], vp[:1, :, :20], vn[:1, :, :20], **kw)
    np.testing.assert_allclose(rag[:1], cut, atol=1e-12)


def test_bf16_rounding_matches_torch():
    x = np.random.default_rng(5).standard_normal(10000).astype(np.float32) * 100
    want = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(O.round_to_dtype(x, "bf16"), want)


# ---------------------------------------------------------------- Prod codec
def test_prod_projection_matrix_is_the_seeded_gaussian():
    """``_projection_matrix`` (:3579-3584): default_rng(seed + 2971 d + 17)."""
    p = O.projection_matrix(64, 1)
    assert p.dtype == np.float32 and p.shape == (64, 64)
    ref = np.random.default_rng(1 + 64 * 2971 + 17).standard_normal((64, 64), dtype=np.float32)
    assert np.array_equal(p, ref)
    assert abs(float(p.mean())) < 0.05 and abs(float(p.std()) - 1.0) < 0.05
    assert not np.array_equal(O.projection_matrix(64, 2), p)


def test_prod_quantize_parts_against_closed_forms():
    """MSE part = quantize_rht at bits - 1; the estimate and residual agree with
    the Sylvester-matrix float64 forms; one bit = pure QJL of u."""
    from scipy.linalg import hadamard

    rng = np.random.default_rng(4)
    d = 64
    x = rng.standard_normal((3, 2, 7, d)).astype(np.float32)
    sg = O.rht_signs(d, 0)
    cb = O.beta_codebook(d, 2)
    n, mse, rn, packed_signs, proj = O.quantize_prod(x, 3, sg, cb, O.projection_matrix(d, 1))
    wp, wn = O.quantize_rht(x, 2, sg, cb)
    assert np.array_equal(mse, wp) and np.array_equal(n, wn)
    u = x.astype(np.float64) / np.maximum(n, 1e-6)[..., None]
    idx = O.unpack_lowbit(mse, 2, d)
    Hm = hadamard(d).astype(np.float64) / np.sqrt(d)
    est = (cb.astype(np.float64)[idx] @ Hm.T) * sg       # R^-1 c = s * (H c) / sqrt(d)
    res = u - est
    np.testing.assert_allclose(rn, np.linalg.norm(res, axis=-1), rtol=1e-5)
    np.testing.assert_allclose(proj, res @ O.projection_matrix(d, 1).astype(np.float64).T,
                               rtol=1e-4, atol=1e-5)
    # one bit: no MSE part, the residual is the unit vector
    n1, mse1, rn1, _, _ = O.quantize_prod(x, 1, sg, None, O.projection_matrix(d, 1))
    assert mse1.shape[-1] == 0
    np.testing.assert_allclose(rn1, 1.0, rtol=1e-6)


def test_prod_dense_rotation_reduces_to_the_hadamard_one():
    """With R = H diag(s) / sqrt(d) -- the Hadamard rotation as a matrix --
    the dense-rotation Prod (estimate c[idx] @ R) reproduces the Hadamard
    Prod: the same indices (away from a midpoint), residual norms and signs
    (away from zero), and the same dequantized keys; an estimate formed as
    R @ c (transposed) would not."""
    from scipy.linalg import hadamard

    rng = np.random.default_rng(12)
    d = 64
    x = rng.standard_normal((2, 3, 9, d)).astype(np.float32)
    sg = O.rht_signs(d, 0)
    Rm = (hadamard(d) * sg[None, :] / np.sqrt(d)).astype(np.float32)   # y = u @ Rm.T = H(s u)/sqrt(d)
    cb, P = O.beta_codebook(d, 2), O.projection_matrix(d, 1)
    h = O.quantize_prod(x, 3, sg, cb, P)
    g = O.quantize_prod(x, 3, Rm, cb, P, rot_kind="dense", indices=O.unpack_lowbit(h[1], 2, d))
    assert np.array_equal(g[1], h[1]) and np.array_equal(g[0], h[0])
    np.testing.assert_allclose(g[2], h[2], rtol=1e-5)
    flip = O.unpack_lowbit(g[3], 1, d) != O.unpack_lowbit(h[3], 1, d)
    assert (np.abs(h[4][flip]) < 1e-4).all()
    # the dense indices themselves: equal except within rounding of a midpoint
    gi = O.quantize_prod(x, 3, Rm, cb, P, rot_kind="dense")[1]
    assert (O.unpack_lowbit(gi, 2, d) != O.unpack_lowbit(h[1], 2, d)).mean() < 1e-3
    kw = dict(bits=3, dim=d, mse_codebook=cb, proj=P)
    kh = O.prod_key_vectors(h[0], h[1], h[2], h[3], signs=sg, **kw)
    kd = O.prod_key_vectors(h[0], h[1], h[2], h[3], signs=Rm, rot_kind="dense", **kw)
    np.testing.assert_allclose(kd, kh, rtol=1e-6, atol=1e-6)
    # a non-symmetric R separates c @ R from R @ c
    Q = O.rotation_matrix(48, 3)
    idx = rng.integers(0, 4, size=(5, 48))
    c = O.beta_codebook(48, 2)
    xs = rng.standard_normal((5, 48)).astype(np.float32)
    _, _, rn, _, _ = O.quantize_prod(xs, 3, Q, c, O.projection_matrix(48, 1), rot_kind="dense", indices=idx)
    u = xs.astype(np.float64) / np.linalg.norm(xs.astype(np.float64), axis=-1, keepdims=True)
    want = np.linalg.norm(u - c.astype(np.float64)[idx] @ Q.astype(np.float64), axis=-1)
    wrong = np.linalg.norm(u - c.astype(np.float64)[idx] @ Q.astype(np.float64).T, axis=-1)
    np.testing.assert_allclose(rn, want, rtol=1e-5)
    assert np.abs(rn - wrong).max() > 1e-3


def test_prod_signs_follow_the_projection_rows():
    """A permutation projection makes the signs the permuted residual's
    signs (catches a transposed P) and ties at zero give 1 (``>= 0``)."""
    d = 64
    rng = np.random.default_rng(6)
    perm = rng.permutation(d)
    P = np.zeros((d, d), np.float32)
    P[np.arange(d), perm] = 1.0                          # (P r)_j = r[perm[j]]
    x = rng.standard_normal((5, d)).astype(np.float32)
    _, _, _, sg, proj = O.quantize_prod(x, 1, O.rht_signs(d, 0), None, P)
    u = x / O.norm_f32(x)[:, None]
    assert np.array_equal(O.unpack_lowbit(sg, 1, d), (u[:, perm] >= 0).astype(np.uint32))
    _, _, _, sg0, _ = O.quantize_prod(np.zeros((1, d), np.float32), 1, O.rht_signs(d, 0), None, P)
    assert O.unpack_lowbit(sg0, 1, d).all()              # zero residual: every sign bit set


def test_prod_dequantize_is_an_unbiased_inner_product():
    """QJL scale sqrt(pi/2)/d and orientation s @ P: the regression slope of
    <q, k_hat> on <q, k> is 1 (a wrong scale or P^T would move it)."""
    rng = np.random.default_rng(8)
    d = 64
    k = rng.standard_normal((1, 1, 3000, d)).astype(np.float32)
    q = rng.standard_normal(d)
    sg, P = O.rht_signs(d, 0), O.projection_matrix(d, 1)
    n, mse, rn, bits_, _ = O.quantize_prod(k, 2, sg, O.beta_codebook(d, 1), P)
    kh = O.prod_key_vectors(n, mse, rn, bits_, bits=2, dim=d, signs=sg,
                            mse_codebook=O.beta_codebook(d, 1), proj=P)[0, 0]
    exact = k[0, 0].astype(np.float64) @ q
    est = kh @ q
    slope = float(est @ exact / (exact @ exact))
    assert abs(slope - 1.0) < 0.04, slope


@pytest.mark.parametrize("bits", [2, 3, 1])
def test_prod_attention_against_sdpa_and_score_prepared(bits):
    """attention_prod equals (1) torch SDPA over the dequantized Prod keys
    under an explicit causal + left-padding + length mask, and (2) a softmax
    over scores formed the way score_prepared and the fused Prod decode kernel
    form them (:4700-4766, :2000-2206): n * (R q_s) . c[idx] plus
    n * rn * sqrt(pi/2)/d * (P q_s) . s, never building a key vector."""
    rng = np.random.default_rng(30 + bits)
    B, Hq, Hkv, L, T, d = 3, 4, 2, 3, 70, 64
    sg, P = O.rht_signs(d, 0), O.projection_matrix(d, 1)
    mcb = O.beta_codebook(d, bits - 1) if bits > 1 else None
    k = rng.standard_normal((B, Hkv, T, d)).astype(np.float32)
    n, mse, rn, sbits, _ = O.quantize_prod(k, bits, sg, mcb, P)
    vp, vn = O.quantize_rht(rng.standard_normal((B, Hkv, T, d)).astype(np.float32), 2,
                            O.rht_signs(d, 1), O.beta_codebook(d, 2))
    q = O.round_to_dtype(rng.standard_normal((B, Hq, L, d)).astype(np.float32), "bf16")
    lengths, starts = [70, 41, 9], [0, 13, 9]
    scale = 1 / math.sqrt(d)
    got = O.attention_prod(q, n, mse, rn, sbits, vp, vn, k_bits=bits, v_bits=2, k_signs_rot=sg,
                           k_mse_codebook=mcb, proj=P, v_codebook=O.beta_codebook(d, 2),
                           v_rot=O.rht_signs(d, 1), scale=scale, q_dtype="bf16", causal=True,
                           lengths=lengths, starts=starts)
    # (1) SDPA with the boolean mask of create_causal_mask(left_padding=...) plus the lengths
    K = O.prod_key_vectors(n, mse, rn, sbits, bits=bits, dim=d, signs=sg, mse_codebook=mcb, proj=P)
    V = O.dequantize(vp, vn, 2, d, O.beta_codebook(d, 2), "hadamard", O.rht_signs(d, 1))
    qs = torch.from_numpy(O.scale_queries(q, scale, "bf16").astype(np.float64))
    R = Hq // Hkv
    for b in range(B):
        s0, e = starts[b], lengths[b]
        if e == s0:
            assert not got[b].any()
            continue
        kpos = torch.arange(T)
        qpos = e - L + torch.arange(L)
        mask = (kpos[None, :] <= qpos[:, None]) & (kpos[None, :] >= s0) & (kpos[None, :] < e)
        Kt = torch.from_numpy(K[b]).repeat_interleave(R, dim=0)
        Vt = torch.from_numpy(V[b]).repeat_interleave(R, dim=0)
        want = torch.nn.functional.scaled_dot_product_attention(qs[b], Kt, Vt, attn_mask=mask,
                                                                scale=1.0).numpy()
        np.testing.assert_allclose(got[b], want, atol=1e-9)
    # (2) the kernel's score form over the packed fields
    from scipy.linalg import hadamard

    Hm = hadamard(d).astype(np.float64) / np.sqrt(d)
    q_rot = (qs.numpy() * sg) @ Hm.T                     # R_K q_s = H (s * q) / sqrt(d)
    q_proj = qs.numpy() @ P.astype(np.float64).T         # P q_s
    sgn = O.unpack_lowbit(sbits, 1, d).astype(np.float64) * 2 - 1
    c = mcb.astype(np.float64)[O.unpack_lowbit(mse, bits - 1, d)] if bits > 1 else 0.0 * sgn
    n64, rn64 = n.astype(np.float64), rn.astype(np.float64)
    b, e = 0, lengths[0]
    for h in range(Hq):
        g = h // R
        sc = n64[b, g][None, :] * (q_rot[b, h] @ c[b, g].T) + \
            n64[b, g][None, :] * rn64[b, g][None, :] * float(O.prod_scale(d)) * (q_proj[b, h] @ sgn[b, g].T)
        qpos = e - L + np.arange(L)
        sc = np.where(np.arange(T)[None, :] <= qpos[:, None], sc, -np.inf)
        p = np.exp(sc - sc.max(axis=-1, keepdims=True))
        o = (p @ V[b, g]) / p.sum(axis=-1, keepdims=True)
        np.testing.assert_allclose(got[b, h], o, atol=1e-9)


def _sdpa_masked(qs, K, V, R, keep=None, add=None):
    """torch float64 SDPA of one sequence with per-query-head masks (Hq, L, T)."""
    Kt = torch.from_numpy(K).repeat_interleave(R, dim=0)
    Vt = torch.from_numpy(V).repeat_interleave(R, dim=0)
    mask = torch.from_numpy(keep) if keep is not None else torch.from_numpy(add)
    return torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(qs), Kt, Vt, attn_mask=mask, scale=1.0).numpy()


@pytest.mark.parametrize("form", ["bool2d", "bool4d", "add5d", "add3d"])
@pytest.mark.parametrize("v_rot_kind", ["hadamard", "dense"])
def test_attention_array_masks_against_sdpa(form, v_rot_kind):
    """attention(mask=...) equals torch SDPA over the dequantized cache with the
    mask laid out per query head by the reference's rule (_apply_attention_mask,
    :5101-5108): the mask is broadcast against the grouped scores
    (B, Hkv, R, L, T), a 4-D mask getting its repeat axis at position 2, so
    query head h = g*R + r reads mask[b, g, r].  Also covers K and V of
    different dims and rotation kinds (the output takes the value dim)."""
    rng = np.random.default_rng(hash((form, v_rot_kind)) % 1000)
    B, Hq, Hkv, L, T, dk = 2, 6, 2, 3, 50, 64
    dv = 64 if v_rot_kind == "hadamard" else 48
    R = Hq // Hkv
    kr, kb = O.rht_signs(dk, 0), 3
    kp, kn = O.quantize_rht(rng.standard_normal((B, Hkv, T, dk)).astype(np.float32), kb, kr,
                            O.beta_codebook(dk, kb))
    vr = O.rht_signs(dv, 1) if v_rot_kind == "hadamard" else O.rotation_matrix(dv, 1)
    vx = rng.standard_normal((B, Hkv, T, dv)).astype(np.float32)
    if v_rot_kind == "hadamard":
        vp, vn = O.quantize_rht(vx, 2, vr, O.beta_codebook(dv, 2))
    else:
        vp, vn, _ = O.quantize_dense(vx, 2, vr, O.beta_codebook(dv, 2))
    q = O.round_to_dtype(rng.standard_normal((B, Hq, L, dk)).astype(np.float32), "bf16")
    shapes = {"bool2d": (L, T), "bool4d": (B, Hkv, L, T), "add5d": (B, Hkv, R, L, T),
              "add3d": (R, L, T)}
    if form.startswith("bool"):
        m = rng.random(shapes[form]) < 0.6
        m[..., 0] = True  # no row fully masked (SDPA gives NaN there)
    else:
        m = rng.normal(0, 3, shapes[form]).astype(np.float32)
    got = O.attention(q, kp, kn, vp, vn, k_bits=kb, v_bits=2, k_codebook=O.beta_codebook(dk, kb),
                      v_codebook=O.beta_codebook(dv, 2), rot_kind="hadamard", k_rot=kr, v_rot=vr,
                      scale=0.125, q_dtype="bf16", v_dim=dv, mask=m, v_rot_kind=v_rot_kind)
    K = O.dequantize(kp, kn, kb, dk, O.beta_codebook(dk, kb), "hadamard", kr)
    V = O.dequantize(vp, vn, 2, dv, O.beta_codebook(dv, 2), v_rot_kind, vr)
    qs = O.scale_queries(q, 0.125, "bf16").astype(np.float64)
    # per query head: explicit index arithmetic, not a broadcast
    per_head = np.zeros((B, Hq, L, T), m.dtype)
    for b in range(B):
        for h in range(Hq):
            g, r = h // R, h % R
            if form == "bool2d":
                per_head[b, h] = m
            elif form == "bool4d":
                per_head[b, h] = m[b, g]
            elif form == "add5d":
                per_head[b, h] = m[b, g, r]
            else:
                per_head[b, h] = m[r]
    for b in range(B):
        want = _sdpa_masked(qs[b], K[b], V[b], R,
                            keep=per_head[b] if form.startswith("bool") else None,
                            add=None if form.startswith("bool") else per_head[b].astype(np.float64))
        np.testing.assert_allclose(got[b], want, atol=1e-9)


def test_mask_broadcast_rejects_query_head_masks_on_grouped_scores():
    """A 4-D mask broadcasts over kv heads, as the reference's expand_dims at
    axis 2 does: a per-query-head (B, Hq, L, T) mask with Hq != Hkv does not
    broadcast there (the fp16 layers' SDPA takes it instead)."""
    m = np.ones((1, 8, 2, 10), bool)
    assert O.mask_5d(m[:, :2], 1, 2, 4, 2, 10).shape == (1, 2, 4, 2, 10)
    with pytest.raises(ValueError):
        O.mask_5d(m, 1, 2, 4, 2, 10)


def test_plain_attention_mask_against_sdpa():
    rng = np.random.default_rng(77)
    B, Hq, Hkv, L, T, d = 2, 4, 2, 3, 30, 32
    k = O.round_to_dtype(rng.standard_normal((B, Hkv, T, d)).astype(np.float32), "f16")
    v = O.round_to_dtype(rng.standard_normal((B, Hkv, T, 48)).astype(np.float32), "f16")
    q = O.round_to_dtype(rng.standard_normal((B, Hq, L, d)).astype(np.float32), "f16")
    m = rng.random((B, Hq, L, T)) < 0.7
    m[..., 0] = True
    got = O.attention_plain(q, k, v, scale=0.2, q_dtype="f16", mask=m)
    qs = O.scale_queries(q, 0.2, "f16").astype(np.float64)
    for b in range(B):
        want = _sdpa_masked(qs[b], k[b].astype(np.float64), v[b].astype(np.float64), Hq // Hkv,
                            keep=m[b])
        np.testing.assert_allclose(got[b], want, atol=1e-9)


@pytest.mark.parametrize("d", [8, 24, 40, 96, 160, 320, 480])
def test_norm_tree_at_any_dim(d):
    """norm_f32 at a dim that is not a power of two: the zero padding leaves the
    value that of the padded power-of-two vector, within an ulp of the float64
    norm, and the tree of a dim below 32 equals the in-lane fold of one padded
    32-element lane."""
    rng = np.random.default_rng(d)
    x = rng.standard_normal((50, d)).astype(np.float32) * np.float32(3.0)
    got = O.norm_f32(x)
    exact = np.sqrt((x.astype(np.float64) ** 2).sum(axis=-1))
    assert np.all(np.abs(got - exact) <= 2 * np.spacing(exact.astype(np.float32)))
    lanes = 32 << max(0, (-(-d // 32) - 1).bit_length()) if d > 32 else 32
    padded = np.concatenate([x, np.zeros((50, lanes - d), np.float32)], axis=-1)
    assert np.array_equal(got, O.norm_f32(padded))
