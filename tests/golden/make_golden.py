"""Write the golden fixtures under tests/golden/ from the numpy oracle.

The reference (MLX) cannot run in this environment, so these vectors come
from ``oracle/tq_oracle.py`` -- a restatement of the reference algorithm
pinned by the closed-form / brute-force checks in tests/test_oracle.py.  The
fixtures freeze the oracle's outputs (codebooks, signs, dense rotations,
packed bytes, norms, attention outputs) so that any later drift of either
the oracle or the product shows up as a fixture mismatch.

Run from the repository root:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import tq_oracle as O  # noqa: E402

DIMS_RHT = (32, 64, 128, 256, 512)


def synth_kv(rng_scale, rng_val, n_heads, n_tok, dim, dtype=np.float16):
    """N(0,1) entries times a per-(head, channel) log-normal(0, 0.5) scale."""
    s = np.exp(rng_scale.normal(0.0, 0.5, size=(n_heads, 1, dim)))
    z = rng_val.standard_normal((n_heads, n_tok, dim))
    return (z * s).astype(dtype)


def make_codebooks():
    out = {}
    for d in DIMS_RHT:
        for b in range(1, 5):
            out[f"beta_{d}_{b}"] = O.beta_codebook(d, b)
    for b in range(1, 5):
        out[f"gauss_{b}"] = O.gaussian_lloyd_max(b)
    np.savez_compressed(os.path.join(HERE, "codebooks.npz"), **out)


def make_rotations():
    out = {}
    for d in DIMS_RHT:
        for seed in (0, 1, 99, 100):
            out[f"signs_{d}_{seed}"] = O.rht_signs(d, seed)
    for d in (64, 128, 256):
        for seed in (0, 1):
            out[f"rot_{d}_{seed}"] = O.rotation_matrix(d, seed)
    np.savez_compressed(os.path.join(HERE, "rotations.npz"), **out)


def make_quantize():
    out = {}
    for d in (32, 64, 128, 256, 512):
        rs, rv = np.random.default_rng(7000 + d), np.random.default_rng(8000 + d)
        x = synth_kv(rs, rv, 2, 24, d).reshape(48, d)
        x[0] = 0.0                      # zero vector: n = 0, u = 0
        x[1] = np.float16(1e-4)         # tiny norm
        out[f"x_{d}"] = x
        for b in range(1, 5):
            packed, norms = O.quantize_rht(x, b, O.rht_signs(d, 0), O.beta_codebook(d, b))
            out[f"packed_{d}_{b}"] = packed
            out[f"norms_{d}_{b}"] = norms
    # other input dtypes and f16 norms at d = 128
    rs, rv = np.random.default_rng(9001), np.random.default_rng(9002)
    x32 = (rv.standard_normal((40, 128)) * np.exp(rs.normal(0, 0.5, (1, 128)))).astype(np.float32)
    out["x32_128"] = x32
    packed, norms = O.quantize_rht(x32, 3, O.rht_signs(128, 1), O.beta_codebook(128, 3), "float16")
    out["packed32_128_3_seed1"] = packed
    out["norms16_128_3_seed1"] = norms.astype(np.float16)
    xb = O.round_to_dtype(x32, "bf16")
    out["xbf16_bits_128"] = (xb.view(np.uint32) >> 16).astype(np.uint16)
    packed, norms = O.quantize_rht(xb, 4, O.rht_signs(128, 0), O.gaussian_codebook(128, 4))
    out["packedbf16_128_4_gauss"] = packed
    out["normsbf16_128_4_gauss"] = norms
    np.savez_compressed(os.path.join(HERE, "quantize.npz"), **out)


def _cache(rng, B, Hkv, T, d, kb, vb, rot_kind, seeds=(0, 1), norm_dtype="float32"):
    rs, rv = np.random.default_rng(rng.integers(1 << 30)), np.random.default_rng(rng.integers(1 << 30))
    k = synth_kv(rs, rv, B * Hkv, T, d).reshape(B, Hkv, T, d)
    v = synth_kv(rs, rv, B * Hkv, T, d).reshape(B, Hkv, T, d)
    if rot_kind == "hadamard":
        kr, vr = O.rht_signs(d, seeds[0]), O.rht_signs(d, seeds[1])
        kp, kn = O.quantize_rht(k, kb, kr, O.beta_codebook(d, kb), norm_dtype)
        vp, vn = O.quantize_rht(v, vb, vr, O.beta_codebook(d, vb), norm_dtype)
    else:
        kr, vr = O.rotation_matrix(d, seeds[0]), O.rotation_matrix(d, seeds[1])
        kp, kn, _ = O.quantize_dense(k, kb, kr, O.beta_codebook(d, kb), norm_dtype)
        vp, vn, _ = O.quantize_dense(v, vb, vr, O.beta_codebook(d, vb), norm_dtype)
    return kp, kn, vp, vn, kr, vr


def make_attention():
    out = {}
    rng = np.random.default_rng(4242)
    cases = [
        # name, B, Hq, Hkv, L, T, d, kb, vb, rot, causal, lengths, q dtype
        ("decode_d128_k3v3", 1, 8, 2, 1, 300, 128, 3, 3, "hadamard", False, None, "bf16"),
        ("verify_d128_k2v1", 1, 8, 2, 4, 300, 128, 2, 1, "hadamard", True, None, "bf16"),
        ("ragged_d256_k4v2_dense", 2, 4, 2, 1, 257, 256, 4, 2, "dense", False, [150, 257], "bf16"),
        ("decode_d64_k4v4_f32q", 1, 4, 4, 1, 70, 64, 4, 4, "hadamard", False, None, "f32"),
    ]
    for name, B, Hq, Hkv, L, T, d, kb, vb, rot, causal, lengths, qdt in cases:
        kp, kn, vp, vn, kr, vr = _cache(rng, B, Hkv, T, d, kb, vb, rot)
        q = rng.standard_normal((B, Hq, L, d)).astype(np.float32)
        q = O.round_to_dtype(q, qdt)
        scale = 1.0 / np.sqrt(d)
        ref = O.attention(q, kp, kn, vp, vn, k_bits=kb, v_bits=vb,
                          k_codebook=O.beta_codebook(d, kb), v_codebook=O.beta_codebook(d, vb),
                          rot_kind=rot, k_rot=kr, v_rot=vr, scale=scale, q_dtype=qdt,
                          causal=causal, lengths=lengths)
        meta = np.array([B, Hq, Hkv, L, T, d, kb, vb, int(rot == "dense"), int(causal)], np.int64)
        out[f"{name}/meta"] = meta
        out[f"{name}/q"] = q
        out[f"{name}/k_packed"] = kp
        out[f"{name}/k_norms"] = kn
        out[f"{name}/v_packed"] = vp
        out[f"{name}/v_norms"] = vn
        out[f"{name}/lengths"] = np.array(lengths if lengths else [T] * B, np.int32)
        out[f"{name}/expected"] = ref.astype(np.float32)
        out[f"{name}/qdtype"] = np.array([{"bf16": 2, "f16": 1, "f32": 0}[qdt]], np.int32)
    # plain fp16 layer
    B, Hq, Hkv, L, T, d = 1, 8, 2, 4, 200, 128
    k = rng.standard_normal((B, Hkv, T, d)).astype(np.float16)
    v = rng.standard_normal((B, Hkv, T, d)).astype(np.float16)
    q = O.round_to_dtype(rng.standard_normal((B, Hq, L, d)).astype(np.float32), "f16")
    ref = O.attention_plain(q, k.astype(np.float32), v.astype(np.float32), scale=1 / np.sqrt(d),
                            q_dtype="f16", causal=True)
    out["plain_f16/q"] = q
    out["plain_f16/k"] = k
    out["plain_f16/v"] = v
    out["plain_f16/expected"] = ref.astype(np.float32)
    np.savez_compressed(os.path.join(HERE, "attention.npz"), **out)


if __name__ == "__main__":
    make_codebooks()
    make_rotations()
    make_quantize()
    make_attention()
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)))
