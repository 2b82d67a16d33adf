"""numpy restatement of kaplumba's TurboQuant KV-cache path (TEST ORACLE ONLY).

Every function cites the reference lines it restates
(``mlx_lm/models/turboquant_cache.py`` unless another file is named).  The
reference is MLX code and cannot run here (MLX is absent), so the numerics
below fix one explicit fp32 operation order; the HIP kernels implement the
same order, which makes packed indices and norms comparable bit for bit.

Not part of the product: ``kaplumba_amd`` never imports this module.
"""
from __future__ import annotations

import math
from typing import Optional, Sequence

import numpy as np

DEFAULT_SEED = 0            # turboquant_cache.py:11
EPS = np.float32(1e-6)      # turboquant_cache.py:12 (weak python scalar -> f32)
LANE_ELEMS = 32             # elements each append lane owns (kernel layout)


# ---------------------------------------------------------------------------
# a1 / a2: rotations
# ---------------------------------------------------------------------------
def rht_signs(dim: int, seed: int) -> np.ndarray:
    """Random +-1 vector of the randomized Hadamard transform.

    Restates ``_rht_sign_vector`` (turboquant_cache.py:3540-3547):
    ``default_rng(seed + dim*7919).choice([-1.0, 1.0], size=dim)`` as f32.
    """
    if dim <= 0:
        return np.zeros((0,), np.float32)
    rng = np.random.default_rng(seed + dim * 7919)
    return rng.choice([-1.0, 1.0], size=dim).astype(np.float32)


def rotation_matrix(dim: int, seed: int) -> np.ndarray:
    """Dense orthogonal rotation, restating ``_rotation_matrix`` (:3517-3528).

    QR of an f32 Gaussian matrix from ``default_rng(seed + dim*7919)``, columns
    multiplied by sign(diag(R)).  Forward rotation is ``u @ R.T`` (:4144),
    inverse ``y @ R`` (:4149).
    """
    if dim <= 0:
        return np.zeros((0, 0), np.float32)
    if dim == 1:
        return np.ones((1, 1), np.float32)
    rng = np.random.default_rng(seed + dim * 7919)
    matrix = rng.standard_normal((dim, dim), dtype=np.float32)
    q, r = np.linalg.qr(matrix)
    q *= np.sign(np.diag(r))
    return q.astype(np.float32)


# ---------------------------------------------------------------------------
# a3: codebooks
# ---------------------------------------------------------------------------
def _beta_pdf(grid: np.ndarray, dim: int) -> np.ndarray:
    """Restates ``_beta_pdf`` (:3587-3603) with identical f32 dtype flow."""
    if dim <= 1:
        pdf = np.ones_like(grid)
    else:
        log_coeff = (
            math.lgamma(dim / 2) - 0.5 * math.log(math.pi) - math.lgamma((dim - 1) / 2)
        )
        log_pdf = log_coeff + ((dim - 3) / 2) * np.log(
            np.clip(1.0 - grid ** 2, 1e-30, None)
        )
        pdf = np.exp(log_pdf - np.max(log_pdf))
    pdf_sum = pdf.sum()
    if pdf_sum == 0:
        return np.full_like(grid, 1.0 / len(grid))
    return pdf / pdf_sum


def beta_codebook(dim: int, bits: int) -> np.ndarray:
    """Lloyd-Max codebook of one coordinate of a uniform unit vector in R^dim.

    Restates ``_codebook`` (:3606-3642): 32768-point f32 grid, CDF-quantile
    initialisation, at most 100 Lloyd iterations, tolerance 1e-6.
    """
    if bits <= 0:
        return np.zeros((0,), np.float32)
    levels = 1 << bits
    if dim <= 1:
        return np.linspace(-1.0, 1.0, levels, dtype=np.float32)
    grid = np.linspace(-1.0 + 1e-6, 1.0 - 1e-6, 32768, dtype=np.float32)
    weights = _beta_pdf(grid, dim)
    cdf = np.cumsum(weights)
    quantiles = (np.arange(levels, dtype=np.float32) + 0.5) / levels
    centroids = np.interp(quantiles, cdf, grid).astype(np.float32)
    for _ in range(100):
        boundaries = np.empty(levels + 1, dtype=np.float32)
        boundaries[0] = -1.0
        boundaries[-1] = 1.0
        boundaries[1:-1] = 0.5 * (centroids[:-1] + centroids[1:])
        new_centroids = centroids.copy()
        for i in range(levels):
            if i == levels - 1:
                mask = (grid >= boundaries[i]) & (grid <= boundaries[i + 1])
            else:
                mask = (grid >= boundaries[i]) & (grid < boundaries[i + 1])
            bucket_weights = weights[mask]
            if bucket_weights.size == 0:
                continue
            total_weight = bucket_weights.sum()
            if total_weight > 0:
                new_centroids[i] = np.sum(bucket_weights * grid[mask]) / total_weight
        if np.max(np.abs(new_centroids - centroids)) < 1e-6:
            centroids = new_centroids
            break
        centroids = new_centroids
    return centroids.astype(np.float32)


def _phi(x: float) -> float:
    return math.exp(-0.5 * x * x) / math.sqrt(2.0 * math.pi)


def _Phi(x: float) -> float:
    return 0.5 * (1.0 + math.erf(x / math.sqrt(2.0)))


def gaussian_lloyd_max(bits: int, iters: int = 2000) -> np.ndarray:
    """Lloyd-Max quantizer of N(0,1) (Max 1960), float64.

    Not in the reference's live path: BASELINE.json names this codebook.  The
    centroid of cell (a, b) is (phi(a) - phi(b)) / (Phi(b) - Phi(a)).
    """
    levels = 1 << bits
    c = np.linspace(-2.0, 2.0, levels)
    for _ in range(iters):
        edges = np.concatenate([[-math.inf], 0.5 * (c[:-1] + c[1:]), [math.inf]])
        new = np.empty_like(c)
        for i in range(levels):
            a, b = edges[i], edges[i + 1]
            pa = 0.0 if a == -math.inf else _phi(a)
            pb = 0.0 if b == math.inf else _phi(b)
            Pa = 0.0 if a == -math.inf else _Phi(a)
            Pb = 1.0 if b == math.inf else _Phi(b)
            new[i] = (pa - pb) / (Pb - Pa)
        if np.max(np.abs(new - c)) < 1e-15:
            c = new
            break
        c = new
    return c


def gaussian_codebook(dim: int, bits: int) -> np.ndarray:
    """N(0,1) Lloyd-Max levels scaled to unit-vector coordinates (/sqrt(dim))."""
    return (gaussian_lloyd_max(bits) / math.sqrt(dim)).astype(np.float32)


def midpoints(codebook: np.ndarray) -> np.ndarray:
    """``(c[:-1] + c[1:]) / 2`` in f32 (turboquant_cache.py:4136-4139)."""
    cb = codebook.astype(np.float32)
    if cb.shape[0] <= 1:
        return np.zeros((0,), np.float32)
    return ((cb[:-1] + cb[1:]) / np.float32(2)).astype(np.float32)


# ---------------------------------------------------------------------------
# a4: randomized Hadamard transform, explicit f32 butterfly order
# ---------------------------------------------------------------------------
def fwht_f32(v: np.ndarray) -> np.ndarray:
    """Unnormalised Sylvester Walsh-Hadamard transform in f32.

    Stage order: butterfly distance 1, 2, 4, ..., D/2.  Each butterfly maps
    (a, b) = (v[i], v[i+h]) with bit h of i clear to (a + b, a - b).
    """
    v = np.asarray(v, dtype=np.float32)
    lead = v.shape[:-1]
    d = v.shape[-1]
    h = 1
    while h < d:
        w = v.reshape(*lead, d // (2 * h), 2, h)
        a = w[..., 0, :]
        b = w[..., 1, :]
        v = np.stack([a + b, a - b], axis=-2).reshape(*lead, d)
        h *= 2
    return v


def rht_scale(dim: int) -> np.float32:
    """``1.0 / math.sqrt(D)`` as passed to ``mx.hadamard_transform`` (:3558)."""
    return np.float32(1.0 / math.sqrt(dim))


def rht_forward_f32(x: np.ndarray, signs: np.ndarray) -> np.ndarray:
    """``H(s*x)/sqrt(D)`` (``_rht_forward``, :3550-3561) in f32."""
    v = np.asarray(x, np.float32) * signs.astype(np.float32)
    return fwht_f32(v) * rht_scale(signs.shape[0])


def rht_inverse_f32(y: np.ndarray, signs: np.ndarray) -> np.ndarray:
    """``s * H(y)/sqrt(D)`` (``_rht_inverse``, :3564-3575) in f32."""
    return (fwht_f32(np.asarray(y, np.float32)) * rht_scale(signs.shape[0])) * signs


def rht_forward_f64(x: np.ndarray, signs: np.ndarray) -> np.ndarray:
    """Closed form with the Sylvester matrix, float64 (independent check)."""
    from scipy.linalg import hadamard

    d = signs.shape[0]
    H = hadamard(d).astype(np.float64)
    return (np.asarray(x, np.float64) * signs) @ H.T / math.sqrt(d)


def rht_inverse_f64(y: np.ndarray, signs: np.ndarray) -> np.ndarray:
    from scipy.linalg import hadamard

    d = signs.shape[0]
    H = hadamard(d).astype(np.float64)
    return (np.asarray(y, np.float64) @ H.T / math.sqrt(d)) * signs


# ---------------------------------------------------------------------------
# a5-a8: quantize and pack
# ---------------------------------------------------------------------------
def norm_f32(x: np.ndarray) -> np.ndarray:
    """L2 norm in f32 with the append kernel's reduction tree.

    The kernel gives each lane ``LANE_ELEMS`` consecutive elements (fewer when
    D < 32).  A lane squares its elements and folds them with distances
    16, 8, 4, 2, 1; lanes are then combined pairwise (xor 1, xor 2, ...).
    A dim that is not a power of two is zero-padded to the next power of two
    (below 32) or to a power-of-two number of 32-element lanes: the padding
    adds exact zeros, so the tree is the same for every dim.
    ``sqrt`` is IEEE (correctly rounded).  Reference: ``mx.linalg.norm`` on
    f32 (:4192, :4249); MLX's own order is parity unpinned.
    """
    xf = np.asarray(x, np.float32)
    lead = xf.shape[:-1]
    d = xf.shape[-1]
    if d <= LANE_ELEMS:
        dp = 1 << (d - 1).bit_length()
    else:
        dp = LANE_ELEMS << (-(-d // LANE_ELEMS) - 1).bit_length()
    if dp != d:
        xf = np.concatenate([xf, np.zeros((*lead, dp - d), np.float32)], axis=-1)
        d = dp
    ce = min(LANE_ELEMS, d)
    nl = d // ce
    s = (xf * xf).reshape(*lead, nl, ce)
    h = ce // 2
    while h >= 1:
        s = s[..., :h] + s[..., h : 2 * h]
        h //= 2
    s = s[..., 0]
    while s.shape[-1] > 1:
        s = s[..., 0::2] + s[..., 1::2]
    return np.sqrt(s[..., 0]).astype(np.float32)


def quantize_indices(rotated: np.ndarray, mids: np.ndarray) -> np.ndarray:
    """``idx = sum_m [y > mid_m]`` with strict ``>`` (:4173-4175)."""
    y = np.asarray(rotated, np.float32)
    idx = np.zeros(y.shape, np.uint32)
    for m in mids.astype(np.float32):
        idx += (y > m).astype(np.uint32)
    return idx


def packed_width(length: int, bits: int) -> int:
    """``_packed_width`` (:3699-3702)."""
    if length == 0 or bits == 0:
        return 0
    return (length * bits + 31) // 32


def pack_lowbit(values: np.ndarray, bits: int) -> np.ndarray:
    """LSB-first bit stream over u32 words (``_pack_lowbit`` :3705-3741)."""
    v = np.asarray(values).astype(np.uint64)
    lead = v.shape[:-1]
    length = v.shape[-1]
    pw = packed_width(length, bits)
    flat = v.reshape(-1, length)
    out = np.zeros((flat.shape[0], pw), np.uint64)
    for i in range(length):
        off = i * bits
        w, s = off // 32, off % 32
        out[:, w] |= (flat[:, i] << np.uint64(s)) & np.uint64(0xFFFFFFFF)
        spill = s + bits - 32
        if spill > 0:
            out[:, w + 1] |= flat[:, i] >> np.uint64(bits - spill)
    return out.astype(np.uint32).reshape(*lead, pw)


def unpack_lowbit(packed: np.ndarray, bits: int, length: int) -> np.ndarray:
    """Inverse of ``pack_lowbit`` (``_unpack_lowbit`` :3744-3780)."""
    p = np.asarray(packed, np.uint32).astype(np.uint64)
    lead = p.shape[:-1]
    flat = p.reshape(-1, p.shape[-1])
    out = np.zeros((flat.shape[0], length), np.uint64)
    mask = np.uint64((1 << bits) - 1)
    for i in range(length):
        off = i * bits
        w, s = off // 32, off % 32
        val = flat[:, w] >> np.uint64(s)
        spill = s + bits - 32
        if spill > 0:
            val |= flat[:, w + 1] << np.uint64(bits - spill)
        out[:, i] = val & mask
    return out.astype(np.uint32).reshape(*lead, length)


def round_to_dtype(x: np.ndarray, dtype: str) -> np.ndarray:
    """Round f32 values to ``dtype`` (RNE) and return them as f32."""
    x = np.asarray(x, np.float32)
    if dtype in ("float32", "f32"):
        return x
    if dtype in ("float16", "f16"):
        return x.astype(np.float16).astype(np.float32)
    if dtype in ("bfloat16", "bf16"):
        u = x.view(np.uint32).astype(np.uint64)
        r = ((u >> np.uint64(16)) & np.uint64(1)) + np.uint64(0x7FFF)
        u = ((u + r) & np.uint64(0xFFFF0000)).astype(np.uint32)
        nan = np.isnan(x)
        out = u.view(np.float32).copy()
        out[nan] = np.nan
        return out
    raise ValueError(dtype)


def quantize_rht(x: np.ndarray, bits: int, signs: np.ndarray, codebook: np.ndarray,
                 norm_dtype: str = "float32"):
    """Quantize vectors with the randomized Hadamard rotation.

    Restates ``_TurboQuantMSECodec.quantize`` (:4186-4254): ``n = ||x||``,
    ``u = x / max(n, 1e-6)``, ``y = H(s*u)/sqrt(D)``, ``idx = sum[y > mid]``,
    LSB-first pack, norm stored as ``norm_dtype`` (the reference stores f16,
    :4209/:4252).  Returns (packed u32 (..., PW), norms (...,)).
    """
    xf = np.asarray(x, np.float32)
    n = norm_f32(xf)
    denom = np.maximum(n, EPS)
    u = xf / denom[..., None]
    y = rht_forward_f32(u, signs)
    idx = quantize_indices(y, midpoints(codebook))
    packed = pack_lowbit(idx, bits)
    norms = round_to_dtype(n, norm_dtype)
    return packed, norms


def rotate_dense_f32(u: np.ndarray, rot: np.ndarray) -> np.ndarray:
    """``u @ R.T`` evaluated in float64 and rounded once to f32."""
    return (np.asarray(u, np.float64) @ rot.astype(np.float64).T).astype(np.float32)


def quantize_dense(x: np.ndarray, bits: int, rot: np.ndarray, codebook: np.ndarray,
                   norm_dtype: str = "float32"):
    """Dense-rotation quantize (array path :4248-4254 with ``u @ R.T``).

    Returns (packed, norms, rotated) -- ``rotated`` lets tests measure how
    close each coordinate is to a midpoint, since a matrix-core GEMM has no
    fixed summation order and may flip indices inside that band.
    """
    xf = np.asarray(x, np.float32)
    n = norm_f32(xf)
    u = xf / np.maximum(n, EPS)[..., None]
    y = rotate_dense_f32(u, rot)
    idx = quantize_indices(y, midpoints(codebook))
    return pack_lowbit(idx, bits), round_to_dtype(n, norm_dtype), y


def dequantize(packed: np.ndarray, norms: np.ndarray, bits: int, dim: int,
               codebook: np.ndarray, rot_kind: str, rot: np.ndarray) -> np.ndarray:
    """``n * R^-1(c[idx])`` (``dequantize`` :4178-4184, :4256-4258), float64."""
    idx = unpack_lowbit(packed, bits, dim)
    y = codebook.astype(np.float64)[idx]
    if rot_kind == "hadamard":
        u = rht_inverse_f64(y, rot)
    else:
        u = y @ rot.astype(np.float64)
    return np.asarray(norms, np.float64)[..., None] * u


# ---------------------------------------------------------------------------
# Prod codec: MSE at bits - 1 plus a 1-bit QJL sketch of the residual
# (_TurboQuantProdCodec, turboquant_cache.py:4572-4766)
# ---------------------------------------------------------------------------
def projection_matrix(dim: int, seed: int) -> np.ndarray:
    """Gaussian QJL projection (``_projection_matrix``, :3579-3584); the codec
    draws it with ``seed + 1`` (:4577)."""
    rng = np.random.default_rng(seed + dim * 2971 + 17)
    return rng.standard_normal((dim, dim), dtype=np.float32)


def prod_scale(dim: int) -> np.float32:
    """``sqrt(pi / 2) / dim`` (:4584), as the f32 ``scale_array`` the kernels read."""
    return np.float32(math.sqrt(math.pi / 2) / dim)


def quantize_prod(x: np.ndarray, bits: int, signs: np.ndarray, mse_codebook: Optional[np.ndarray],
                  proj: np.ndarray, norm_dtype: str = "float32", rot_kind: str = "hadamard",
                  indices: Optional[np.ndarray] = None):
    """Array path of ``_TurboQuantProdCodec.quantize`` (:4653-4666) in f32.

    ``n = ||x||``, ``u = x / max(n, 1e-6)``; the MSE codec at ``bits - 1``
    quantizes ``u`` (indices as ``quantize_rht``, or ``quantize_dense`` when
    ``rot_kind == "dense"`` and ``signs`` is the rotation R) and its estimate
    is ``R^-1(c[idx])`` (``_quantize_unit_with_estimate``, :4149-4166):
    ``_rht_inverse``, or ``c[idx] @ R`` (``_rotate_inverse``, :4146-4149)
    formed exactly and rounded once to f32; the residual ``u - estimate``
    keeps its norm and the signs of ``residual @ P^T`` (``>= 0`` -> 1),
    packed one bit each.  With ``bits == 1`` there is no MSE part and the
    residual is ``u``.  ``indices`` (tests only) replaces the MSE indices, so
    that the residual can follow a kernel's indices where a coordinate lies
    within rounding of a midpoint.
    Returns (norms, mse_packed, residual_norms, sign_packed, projected): the
    f32 ``projected`` lets tests bound sign flips near zero, where the order
    of a matrix product's sum decides.
    """
    xf = np.asarray(x, np.float32)
    n = norm_f32(xf)
    u = xf / np.maximum(n, EPS)[..., None]
    mb = bits - 1
    if mb >= 1:
        dense = rot_kind == "dense"
        y = rotate_dense_f32(u, signs) if dense else rht_forward_f32(u, signs)
        idx = quantize_indices(y, midpoints(mse_codebook)) if indices is None else np.asarray(indices)
        mse_packed = pack_lowbit(idx, mb)
        c = mse_codebook.astype(np.float32)[idx]
        if dense:
            est = (c.astype(np.float64) @ np.asarray(signs, np.float64)).astype(np.float32)
        else:
            est = rht_inverse_f32(c, signs)
        residual = (u - est).astype(np.float32)
    else:
        mse_packed = np.zeros((*xf.shape[:-1], 0), np.uint32)
        residual = u
    rn = norm_f32(residual)
    projected = (residual.astype(np.float64) @ proj.astype(np.float64).T).astype(np.float32)
    sign_packed = pack_lowbit((projected >= 0).astype(np.uint32), 1)
    return (round_to_dtype(n, norm_dtype), mse_packed, round_to_dtype(rn, norm_dtype), sign_packed,
            projected)


def prod_key_vectors(norms, mse_packed, residual_norms, sign_packed, *, bits: int, dim: int,
                     signs: np.ndarray, mse_codebook: Optional[np.ndarray],
                     proj: np.ndarray, rot_kind: str = "hadamard") -> np.ndarray:
    """Dequantized keys ``n * (R^-1 c[idx] + scale * rn * (s @ P))`` in float64
    (``_TurboQuantProdCodec.dequantize``, :4668-4677), with s = +-1 from the
    bits; ``R^-1 c = c @ R`` for the dense rotation (``signs`` is then R)."""
    n = np.asarray(norms, np.float64)[..., None]
    rn = np.asarray(residual_norms, np.float64)[..., None]
    s = unpack_lowbit(sign_packed, 1, dim).astype(np.float64) * 2.0 - 1.0
    qjl = float(prod_scale(dim)) * rn * (s @ proj.astype(np.float64))
    if bits - 1 >= 1:
        idx = unpack_lowbit(mse_packed, bits - 1, dim)
        c = mse_codebook.astype(np.float64)[idx]
        mse = c @ np.asarray(signs, np.float64) if rot_kind == "dense" else rht_inverse_f64(c, signs)
    else:
        mse = 0.0
    return n * (mse + qjl)


def attention_prod(q: np.ndarray, k_norms, k_mse, k_rnorms, k_signs, v_packed: np.ndarray,
                   v_norms: np.ndarray, *, k_bits: int, v_bits: int, k_signs_rot: np.ndarray,
                   k_mse_codebook: Optional[np.ndarray], proj: np.ndarray,
                   v_codebook: np.ndarray, v_rot: np.ndarray, scale: float, q_dtype: str,
                   causal: bool = False, lengths: Optional[Sequence[int]] = None,
                   starts: Optional[Sequence[int]] = None,
                   mask: Optional[np.ndarray] = None) -> np.ndarray:
    """Attention with Prod-coded keys and MSE-coded values, float64.

    Scores follow ``score_prepared`` (:4700-4766) -- ``n * q_rot . c[idx] +
    n * scale * rn * (q_proj . s)`` with ``q_rot = R_K q_s`` and ``q_proj =
    q_s @ P^T`` (``prepare_queries``, :4692-4698) -- which is what the
    fused Prod decode kernel computes per token (:2000-2206); the rest is
    ``quantized_attention`` (:5110-5203) as in ``attention``.  Evaluated on
    the dequantized keys, which is the same bilinear form.
    """
    B, Hq, L, D = q.shape
    Hkv = np.asarray(k_norms).shape[1]
    R = Hq // Hkv
    qs = scale_queries(q, scale, q_dtype).astype(np.float64)
    kd_all = prod_key_vectors(k_norms, k_mse, k_rnorms, k_signs, bits=k_bits, dim=D,
                              signs=k_signs_rot, mse_codebook=k_mse_codebook, proj=proj)
    vc = v_codebook.astype(np.float64)
    Dv = np.asarray(v_rot).shape[0]
    out = np.zeros((B, Hq, L, Dv), np.float64)
    fmin = float(np.finfo(np.float32).min)
    cap = kd_all.shape[2]
    m5 = None if mask is None else mask_5d(mask, B, Hkv, R, L, cap)
    for b in range(B):
        end = cap if lengths is None else int(lengths[b])
        t0 = 0 if starts is None else min(int(starts[b]), end)
        T = end - t0
        if T == 0:
            continue
        for g in range(Hkv):
            kd = kd_all[b, g, t0:end]
            vidx = unpack_lowbit(v_packed[b, g, t0:end], v_bits, Dv)
            vd = vc[vidx] * np.asarray(v_norms[b, g, t0:end], np.float64)[:, None]
            for r in range(R):
                h = g * R + r
                s = qs[b, h] @ kd.T
                if causal:
                    qi = (T - L) + np.arange(L)[:, None]
                    s = np.where(qi >= np.arange(T)[None, :], s, fmin)
                if m5 is not None:
                    s = apply_mask(s, m5[b, g, r, :, t0:end])
                m = s.max(axis=-1, keepdims=True)
                p = np.exp(s - m)
                l = p.sum(axis=-1, keepdims=True)
                out[b, h] = rht_inverse_f64(p @ vd, v_rot) / np.maximum(l, float(EPS))
    return out


# ---------------------------------------------------------------------------
# a11-a15: attention over the packed cache
# ---------------------------------------------------------------------------
def scale_queries(q: np.ndarray, scale: float, q_dtype: str) -> np.ndarray:
    """``queries * scale`` in the query dtype (:5802, :5123).

    MLX casts a python scalar to the array's dtype, multiplies and rounds the
    product back to that dtype; emulated here with RNE rounding.
    """
    s = round_to_dtype(np.array([scale], np.float32), q_dtype)[0]
    return round_to_dtype(np.asarray(q, np.float32) * s, q_dtype)


def mask_5d(mask: np.ndarray, B: int, Hkv: int, R: int, L: int, T: int) -> np.ndarray:
    """An array mask broadcast to the scores' shape (B, Hkv, R, L, T).

    ``_apply_attention_mask`` (:5079-5108) slices ``mask[..., q, k]`` and, when
    the mask has one dimension fewer than the 5-D grouped scores (a 4-D
    ``(B, H, L, T)`` mask), inserts the repeat axis at position 2, so its
    head axis lines up with the kv heads; otherwise numpy broadcasting
    aligns it from the right.
    """
    m = np.asarray(mask)
    m = m[..., :L, :T]
    if m.ndim == 4:
        m = np.expand_dims(m, 2)
    return np.broadcast_to(m, (B, Hkv, R, L, T))


def apply_mask(s: np.ndarray, m: np.ndarray) -> np.ndarray:
    """Boolean masks keep scores where True (f32 min elsewhere); other masks
    are added (:5104-5108)."""
    if m.dtype == np.bool_:
        return np.where(m, s, float(np.finfo(np.float32).min))
    return s + m.astype(np.float64)


def attention(q: np.ndarray, k_packed: np.ndarray, k_norms: np.ndarray,
              v_packed: np.ndarray, v_norms: np.ndarray, *, k_bits: int, v_bits: int,
              k_codebook: np.ndarray, v_codebook: np.ndarray, rot_kind: str,
              k_rot: np.ndarray, v_rot: np.ndarray, scale: float, q_dtype: str,
              causal: bool = False, lengths: Optional[Sequence[int]] = None,
              v_dim: Optional[int] = None,
              starts: Optional[Sequence[int]] = None,
              mask: Optional[np.ndarray] = None,
              v_rot_kind: Optional[str] = None) -> np.ndarray:
    """TurboQuant attention in float64, ``quantized_attention`` semantics.

    Restates :5110-5203 with ``_apply_attention_mask`` (:5079-5108) and the
    array-path ``score_prepared``/``weighted_sum`` (:4281-4309): scores are
    ``n_k * (R_K q_s) . c_k[idx]``; causal rows see keys ``k <= T - L + i``
    (masked scores become f32 min, as ``mx.finfo(f32).min``); softmax;
    ``sum p * n_v * c_v[idx]`` in rotated space; ``R_V^-1``; divide by
    ``max(sum p, 1e-6)``.  ``lengths`` gives per-sequence cache lengths for
    ragged batches (tokens beyond a length do not exist for that sequence).
    ``starts`` gives per-sequence left padding: keys before it do not exist
    either, which is the left-padding mask ``left_padding <= k`` of
    models/base.py:40-41 that BatchKVCache.make_mask applies
    (models/cache.py:1195-1198); the causal rule still counts from the end.
    ``mask`` is an array mask over absolute key positions (``mask_5d``,
    ``apply_mask``).  ``v_rot_kind`` (default ``rot_kind``) is the value
    codec's own rotation kind: each codec picks Hadamard or dense from its own
    dim (:4122-4139).  Returns float64 (B, Hq, L, Dv); callers round to the
    query dtype.
    """
    B, Hq, L, D = q.shape
    Hkv = k_packed.shape[1]
    R = Hq // Hkv
    Dv = v_dim if v_dim is not None else D
    cap = k_packed.shape[2]
    m5 = None if mask is None else mask_5d(mask, B, Hkv, R, L, cap)
    qs = scale_queries(q, scale, q_dtype).astype(np.float64)
    if rot_kind == "hadamard":
        qr = rht_forward_f64(qs, k_rot)
    else:
        qr = qs @ k_rot.astype(np.float64).T
    kc = k_codebook.astype(np.float64)
    vc = v_codebook.astype(np.float64)
    out = np.zeros((B, Hq, L, Dv), np.float64)
    fmin = float(np.finfo(np.float32).min)
    for b in range(B):
        end = cap if lengths is None else int(lengths[b])
        t0 = 0 if starts is None else min(int(starts[b]), end)
        T = end - t0
        if T == 0:
            continue
        for g in range(Hkv):
            kidx = unpack_lowbit(k_packed[b, g, t0:end], k_bits, D)
            vidx = unpack_lowbit(v_packed[b, g, t0:end], v_bits, Dv)
            kd = kc[kidx] * np.asarray(k_norms[b, g, t0:end], np.float64)[:, None]
            vd = vc[vidx] * np.asarray(v_norms[b, g, t0:end], np.float64)[:, None]
            for r in range(R):
                h = g * R + r
                s = qr[b, h] @ kd.T                      # (L, T)
                if causal:
                    qi = (T - L) + np.arange(L)[:, None]
                    kj = np.arange(T)[None, :]
                    s = np.where(qi >= kj, s, fmin)
                if m5 is not None:
                    s = apply_mask(s, m5[b, g, r, :, t0:end])
                m = s.max(axis=-1, keepdims=True)
                p = np.exp(s - m)
                l = p.sum(axis=-1, keepdims=True)
                o_rot = p @ vd                            # (L, Dv)
                if (v_rot_kind or rot_kind) == "hadamard":
                    o = rht_inverse_f64(o_rot, v_rot)
                else:
                    o = o_rot @ v_rot.astype(np.float64)
                out[b, h] = o / np.maximum(l, float(EPS))
    return out


def attention_plain(q: np.ndarray, k: np.ndarray, v: np.ndarray, *, scale: float,
                    q_dtype: str, causal: bool = False,
                    lengths: Optional[Sequence[int]] = None,
                    starts: Optional[Sequence[int]] = None,
                    mask: Optional[np.ndarray] = None) -> np.ndarray:
    """Standard SDPA over an unquantized (fp16/bf16) cache, float64.

    The mixed-precision layers of the reference keep model-dtype K/V and call
    ``mx.fast.scaled_dot_product_attention`` (models/base.py:218-226,
    models/cache.py:55-61).  Queries are scaled in their dtype as above;
    ``lengths`` and ``starts`` as in ``attention``.  An array ``mask``
    broadcasts against the (B, Hq, L, T) scores, as the fast SDPA's does
    (sliced ``[..., :L, :T]`` over absolute key positions; boolean keeps,
    other dtypes add, as ``apply_mask``).
    """
    B, Hq, L, D = q.shape
    Hkv = k.shape[1]
    R = Hq // Hkv
    qs = scale_queries(q, scale, q_dtype).astype(np.float64)
    out = np.zeros((B, Hq, L, v.shape[-1]), np.float64)
    fmin = float(np.finfo(np.float32).min)
    m4 = None
    if mask is not None:
        m4 = np.broadcast_to(np.asarray(mask)[..., :L, :k.shape[2]], (B, Hq, L, k.shape[2]))
    for b in range(B):
        end = k.shape[2] if lengths is None else int(lengths[b])
        t0 = 0 if starts is None else min(int(starts[b]), end)
        T = end - t0
        if T == 0:
            continue
        for h in range(Hq):
            g = h // R
            s = qs[b, h] @ np.asarray(k[b, g, t0:end], np.float64).T
            if causal:
                qi = (T - L) + np.arange(L)[:, None]
                s = np.where(qi >= np.arange(T)[None, :], s, fmin)
            if m4 is not None:
                s = apply_mask(s, m4[b, h, :, t0:end])
            m = s.max(axis=-1, keepdims=True)
            p = np.exp(s - m)
            out[b, h] = (p @ np.asarray(v[b, g, t0:end], np.float64)) / np.maximum(
                p.sum(axis=-1, keepdims=True), float(EPS))
    return out


def attention_chunked_f32(q, k_packed, k_norms, v_packed, v_norms, *, k_bits, v_bits,
                          k_codebook, v_codebook, signs_k, signs_v, scale, q_dtype,
                          causal=False, key_chunk=2048):
    """f32 chunked online softmax in the order of ``quantized_attention``.

    Hadamard rotation only; used as the CPU baseline ("port") and to show the
    f32 order agrees with the float64 form.  Vectorised over heads.
    """
    B, Hq, L, D = q.shape
    Hkv = k_packed.shape[1]
    R = Hq // Hkv
    T = k_packed.shape[2]
    qs = scale_queries(q, scale, q_dtype).reshape(B, Hkv, R, L, D)
    qr = rht_forward_f32(qs, signs_k)
    kc = k_codebook.astype(np.float32)
    vc = v_codebook.astype(np.float32)
    out = np.zeros((B, Hkv, R, L, D), np.float32)
    norm = np.zeros((B, Hkv, R, L), np.float32)
    mx_ = np.full((B, Hkv, R, L), -np.inf, np.float32)
    fmin = np.finfo(np.float32).min
    for k0 in range(0, T, key_chunk):
        k1 = min(T, k0 + key_chunk)
        kidx = unpack_lowbit(k_packed[:, :, k0:k1], k_bits, D)
        kd = kc[kidx]
        s = np.einsum("bgrld,bgtd->bgrlt", qr, kd) * k_norms[:, :, None, None, k0:k1].astype(np.float32)
        if causal:
            qi = (T - L) + np.arange(L)[:, None]
            kj = np.arange(k0, k1)[None, :]
            s = np.where(qi >= kj, s, fmin)
        cm = s.max(axis=-1)
        w = np.exp(s - cm[..., None])
        vidx = unpack_lowbit(v_packed[:, :, k0:k1], v_bits, D)
        vd = vc[vidx] * v_norms[:, :, k0:k1, None].astype(np.float32)
        co = np.einsum("bgrlt,bgtd->bgrld", w, vd)
        co = rht_inverse_f32(co, signs_v)
        cden = w.sum(axis=-1)
        nm = np.maximum(mx_, cm)
        ps = np.exp(mx_ - nm)
        cs = np.exp(cm - nm)
        out = out * ps[..., None] + co * cs[..., None]
        norm = norm * ps + cden * cs
        mx_ = nm
    res = out / np.maximum(norm[..., None], EPS)
    return res.reshape(B, Hq, L, D)
