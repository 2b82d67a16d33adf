"""Parity at BASELINE.json's full sizes for configs 0, 2 and 4.

The oracle runs in float64 over every token, so at these sizes it checks a
few (sequence, kv head) groups against the kernels; the rest of each problem
is checked through properties that do not depend on size (config 0, the
append, is checked whole and bit-exact):
  * config 4 (4 x 4 causal drafts over 131,076 tokens, K2/V1): draft row
    L-1 sees every key, so it equals a decode (L = 1) call with that query;
  * config 2 (32 ragged sequences, d = 256, K4/V2, dense rotation): each
    sequence's output equals a batch-of-one call over its own rows (batch
    invariance, which also covers the ragged lengths).
Bar as in test_attention_gpu (within max(2e-3, 1 ulp) and 1e-3 mean-rel of
the float64 oracle); kernel-vs-kernel comparisons use the same bar against
the other call's output.
"""
import math

import numpy as np
import pytest
import torch

from oracle import tq_oracle as O
from kaplumba_amd import ops
from tests.test_attention_gpu import assert_close, q_tensor

pytestmark = pytest.mark.gpu


def _synth(g, shape, device):
    B, H, T, D = shape
    s = torch.exp(torch.randn(1, H, 1, D, generator=g) * 0.5).to(device)
    return [(torch.randn(shape, generator=g).to(device) * s).to(torch.bfloat16) for _ in range(2)]


def _quantize(x, codec, device):
    B, H, T, _ = x.shape
    pk = torch.zeros((B, H, T, codec.packed_width), dtype=torch.uint32, device=device)
    nm = torch.zeros((B, H, T), dtype=torch.float32, device=device)
    ops.append_quantize(x, codec, pk, nm, 0)
    return nm, pk


@pytest.mark.parametrize("codebook", ["beta", "gaussian"])
def test_config0_kv_launch_full_size(device, codebook):
    """The benched config-0 launch: one tq_append_quantize_kv call on K and V
    f16 [1, 8, 4096, 128] (per-channel log-normal scales), 3-bit, f32 norms,
    packed words and norms bit-exact against the oracle; BASELINE's second
    check, reconstruction MSE, against the 3-bit Lloyd-Max distortion."""
    rs, rk, rv = (np.random.default_rng(s) for s in (1000, 1001, 1002))
    scale = np.exp(rs.normal(0.0, 0.5, size=(1, 8, 1, 128)))
    k = (rk.standard_normal((1, 8, 4096, 128)) * scale).astype(np.float16)
    v = (rv.standard_normal((1, 8, 4096, 128)) * scale).astype(np.float16)
    kc = ops.Codec(128, 3, 0, codebook_kind=codebook)
    vc = ops.Codec(128, 3, 1, codebook_kind=codebook)
    cb = O.beta_codebook(128, 3) if codebook == "beta" else O.gaussian_codebook(128, 3)
    bufs = [(torch.zeros((1, 8, 4096, 12), dtype=torch.uint32, device=device),
             torch.zeros((1, 8, 4096), dtype=torch.float32, device=device)) for _ in range(2)]
    (kp, kn), (vp, vn) = bufs
    ops.append_quantize_kv(torch.from_numpy(k).to(device), torch.from_numpy(v).to(device), kc, vc,
                           kp, kn, vp, vn, 0)
    for x, (p, n), codec in ((k, bufs[0], kc), (v, bufs[1], vc)):
        wp, wn = O.quantize_rht(x, 3, O.rht_signs(128, codec.seed), cb)
        mism = int((p.cpu().numpy().astype(np.uint32) != wp).sum())
        assert mism == 0, f"{mism} packed words differ ({codebook}, seed {codec.seed})"
        assert np.array_equal(n.cpu().numpy(), wn)
        deq = ops.dequantize(p, n, codec).cpu().numpy().astype(np.float64)
        xf = x.astype(np.float64)
        rel_mse = ((deq - xf) ** 2).sum(-1).mean() / (xf ** 2).sum(-1).mean()
        # 3-bit Lloyd-Max distortion of N(0,1) (Max 1960): 0.03454
        assert 0.030 < rel_mse < 0.040, (codebook, codec.seed, rel_mse)


@pytest.mark.parametrize("codebook", ["beta", "gaussian"])
def test_config4_full_size(device, codebook):
    B, Hq, Hkv, L, T, D, kb, vb = 4, 32, 8, 4, 131072 + 4, 128, 2, 1
    g = torch.Generator().manual_seed(44)
    k, v = _synth(g, (B, Hkv, T, D), device)
    kc = ops.Codec(D, kb, 0, codebook_kind=codebook)
    vc = ops.Codec(D, vb, 1, codebook_kind=codebook)
    (kn, kp), (vn, vp) = _quantize(k, kc, device), _quantize(v, vc, device)
    q = torch.randn(B, Hq, L, D, generator=g).to(torch.bfloat16)
    scale = 1 / math.sqrt(D)
    out = ops.attention_packed(q.to(device), kn, kp, vn, vp, kc, vc, scale, True)
    # draft row L-1 = a decode of that query
    dec = ops.attention_packed(q[:, :, L - 1:].contiguous().to(device), kn, kp, vn, vp, kc, vc,
                               scale, False)
    assert_close(out[:, :, L - 1:], dec.float().cpu().numpy().astype(np.float64), "bf16",
                 f"cfg4 last draft vs decode, {codebook}")
    # float64 oracle on two (sequence, kv head) groups over all 131,076 tokens
    for b, gk in ((0, 0), (3, 7)):
        sl = slice(gk * (Hq // Hkv), (gk + 1) * (Hq // Hkv))
        want = O.attention(q[b:b + 1, sl].float().numpy(), kp[b:b + 1, gk:gk + 1].cpu().numpy().astype(np.uint32),
                           kn[b:b + 1, gk:gk + 1].cpu().numpy(),
                           vp[b:b + 1, gk:gk + 1].cpu().numpy().astype(np.uint32),
                           vn[b:b + 1, gk:gk + 1].cpu().numpy(), k_bits=kb, v_bits=vb,
                           k_codebook=kc.codebook, v_codebook=vc.codebook, rot_kind="hadamard",
                           k_rot=O.rht_signs(D, 0), v_rot=O.rht_signs(D, 1), scale=scale,
                           q_dtype="bf16", causal=True)
        assert_close(out[b:b + 1, sl], want, "bf16", f"cfg4 full size oracle b{b} kv{gk}, {codebook}")


def test_config2_full_size(device):
    B, Hq, Hkv, D, kb, vb = 32, 16, 8, 256, 4, 2
    lens = np.random.default_rng(1004).integers(2048, 8192 + 1, size=B)
    cap = 8192
    g = torch.Generator().manual_seed(22)
    k, v = _synth(g, (B, Hkv, cap, D), device)
    kc, vc = ops.Codec(D, kb, 0, "dense"), ops.Codec(D, vb, 1, "dense")
    (kn, kp), (vn, vp) = _quantize(k, kc, device), _quantize(v, vc, device)
    q = torch.randn(B, Hq, 1, D, generator=g).to(torch.bfloat16)
    scale = 1 / math.sqrt(D)
    out = ops.attention_packed(q.to(device), kn, kp, vn, vp, kc, vc, scale, False,
                               seq_lens=torch.from_numpy(lens.astype(np.int32)))
    for b in range(B):  # batch invariance: each sequence alone, over its own rows only
        T = int(lens[b])
        one = ops.attention_packed(q[b:b + 1].to(device), kn[b:b + 1, :, :T], kp[b:b + 1, :, :T],
                                   vn[b:b + 1, :, :T], vp[b:b + 1, :, :T], kc, vc, scale, False)
        assert_close(out[b:b + 1], one.float().cpu().numpy().astype(np.float64), "bf16",
                     f"cfg2 batch vs alone b{b}")
    for b in (int(np.argmin(lens)), int(np.argmax(lens))):
        T = int(lens[b])
        want = O.attention(q[b:b + 1].float().numpy(), kp[b:b + 1, :, :T].cpu().numpy().astype(np.uint32),
                           kn[b:b + 1, :, :T].cpu().numpy(),
                           vp[b:b + 1, :, :T].cpu().numpy().astype(np.uint32),
                           vn[b:b + 1, :, :T].cpu().numpy(), k_bits=kb, v_bits=vb,
                           k_codebook=kc.codebook, v_codebook=vc.codebook, rot_kind="dense",
                           k_rot=O.rotation_matrix(D, 0), v_rot=O.rotation_matrix(D, 1), scale=scale,
                           q_dtype="bf16")
        assert_close(out[b:b + 1], want, "bf16", f"cfg2 oracle b{b} T{T}")
