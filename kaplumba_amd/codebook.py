"""Host-side codec constants: sign vectors, dense rotations, Lloyd-Max codebooks.

These are computed once on the CPU (numpy), exactly as the reference does,
then uploaded to HBM and cached per device.  They are kernel *inputs*, so
"same rotation and codebook" parity between this library and the reference
is structural.  The arithmetic is deliberately the reference's own, step for
step, because the codebook values are part of the storage contract (a
midpoint that moved by one ulp would change stored indices).
"""
from __future__ import annotations

import math
from functools import lru_cache

import numpy as np

DEFAULT_TURBOQUANT_SEED = 0  # turboquant_cache.py:11
EPS = 1e-6                   # turboquant_cache.py:12


@lru_cache(maxsize=None)
def rht_sign_vector(dim: int, seed: int) -> np.ndarray:
    """+-1 signs of the randomized Hadamard transform (turboquant_cache.py:3540-3547)."""
    if dim <= 0:
        return np.zeros((0,), np.float32)
    rng = np.random.default_rng(seed + dim * 7919)
    out = rng.choice([-1.0, 1.0], size=dim).astype(np.float32)
    out.setflags(write=False)
    return out


@lru_cache(maxsize=None)
def rotation_matrix(dim: int, seed: int) -> np.ndarray:
    """Dense orthogonal rotation R (turboquant_cache.py:3517-3528): QR of an f32
    Gaussian matrix, columns sign-fixed by sign(diag(R)).  Rotate: u @ R.T."""
    if dim <= 0:
        return np.zeros((0, 0), np.float32)
    if dim == 1:
        return np.ones((1, 1), np.float32)
    rng = np.random.default_rng(seed + dim * 7919)
    matrix = rng.standard_normal((dim, dim), dtype=np.float32)
    q, r = np.linalg.qr(matrix)
    q *= np.sign(np.diag(r))
    out = q.astype(np.float32)
    out.setflags(write=False)
    return out


def _beta_pdf(grid: np.ndarray, dim: int) -> np.ndarray:
    # Density of one coordinate of a uniform unit vector in R^dim,
    # proportional to (1 - x^2)^((dim-3)/2) (turboquant_cache.py:3587-3603).
    if dim <= 1:
        pdf = np.ones_like(grid)
    else:
        log_coeff = (
            math.lgamma(dim / 2) - 0.5 * math.log(math.pi) - math.lgamma((dim - 1) / 2)
        )
        log_pdf = log_coeff + ((dim - 3) / 2) * np.log(np.clip(1.0 - grid ** 2, 1e-30, None))
        pdf = np.exp(log_pdf - np.max(log_pdf))
    total = pdf.sum()
    if total == 0:
        return np.full_like(grid, 1.0 / len(grid))
    return pdf / total


@lru_cache(maxsize=None)
def beta_codebook(dim: int, bits: int) -> np.ndarray:
    """Lloyd-Max levels for the Beta coordinate marginal (turboquant_cache.py:3606-3642)."""
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
        edges = np.empty(levels + 1, dtype=np.float32)
        edges[0] = -1.0
        edges[-1] = 1.0
        edges[1:-1] = 0.5 * (centroids[:-1] + centroids[1:])
        updated = centroids.copy()
        for i in range(levels):
            upper_closed = i == levels - 1
            sel = (grid >= edges[i]) & ((grid <= edges[i + 1]) if upper_closed else (grid < edges[i + 1]))
            w = weights[sel]
            if w.size == 0:
                continue
            tw = w.sum()
            if tw > 0:
                updated[i] = np.sum(w * grid[sel]) / tw
        done = np.max(np.abs(updated - centroids)) < 1e-6
        centroids = updated
        if done:
            break
    out = centroids.astype(np.float32)
    out.setflags(write=False)
    return out


def _std_normal_pdf(x: float) -> float:
    return math.exp(-0.5 * x * x) / math.sqrt(2.0 * math.pi)


def _std_normal_cdf(x: float) -> float:
    return 0.5 * (1.0 + math.erf(x / math.sqrt(2.0)))


@lru_cache(maxsize=None)
def gaussian_levels(bits: int) -> np.ndarray:
    """Lloyd-Max (Max 1960) levels of N(0,1) in float64."""
    n = 1 << bits
    c = np.linspace(-2.0, 2.0, n)
    for _ in range(2000):
        e = np.concatenate([[-math.inf], 0.5 * (c[:-1] + c[1:]), [math.inf]])
        nxt = np.empty_like(c)
        for i in range(n):
            lo, hi = e[i], e[i + 1]
            mass = (1.0 if hi == math.inf else _std_normal_cdf(hi)) - (
                0.0 if lo == -math.inf else _std_normal_cdf(lo))
            first = (0.0 if lo == -math.inf else _std_normal_pdf(lo)) - (
                0.0 if hi == math.inf else _std_normal_pdf(hi))
            nxt[i] = first / mass
        if np.max(np.abs(nxt - c)) < 1e-15:
            c = nxt
            break
        c = nxt
    return c


@lru_cache(maxsize=None)
def gaussian_codebook(dim: int, bits: int) -> np.ndarray:
    """N(0,1) Lloyd-Max levels in unit-vector scale (divided by sqrt(dim))."""
    out = (gaussian_levels(bits) / math.sqrt(dim)).astype(np.float32)
    out.setflags(write=False)
    return out


def codebook(dim: int, bits: int, kind: str = "beta") -> np.ndarray:
    if kind == "beta":
        return beta_codebook(dim, bits)
    if kind == "gaussian":
        return gaussian_codebook(dim, bits)
    raise ValueError(f"Unknown TurboQuant codebook {kind!r} (expected 'beta' or 'gaussian').")


def midpoints(cb: np.ndarray) -> np.ndarray:
    """Decision thresholds (c[i] + c[i+1]) / 2 in f32 (turboquant_cache.py:4136-4139)."""
    cb = np.asarray(cb, np.float32)
    if cb.shape[0] <= 1:
        return np.zeros((0,), np.float32)
    return ((cb[:-1] + cb[1:]) / np.float32(2)).astype(np.float32)


def projection_matrix(dim: int, seed: int) -> np.ndarray:
    """Gaussian QJL projection of the Prod codec (``_projection_matrix``,
    turboquant_cache.py:3579-3584): ``default_rng(seed + 2971 dim + 17)``
    standard normals, f32 (dim, dim).  The codec passes ``seed + 1`` (:4577)."""
    rng = np.random.default_rng(seed + dim * 2971 + 17)
    return rng.standard_normal((dim, dim), dtype=np.float32)


def packed_width(length: int, bits: int) -> int:
    """u32 words per packed row (turboquant_cache.py:3699-3702)."""
    if length == 0 or bits == 0:
        return 0
    return (length * bits + 31) // 32
