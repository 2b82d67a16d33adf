"""Parity of exactly the launches bench.py times, at their full sizes.

* config 3: one layer's keys and values through append_quantize_kv (the
  paired dense-rotation kernel at bits (3, 3), bf16 input, f32 norms), and
  the unquantized copy of the fp16 layers;
* config 4's fp16-layer leg: causal verify of 4 x 4 drafts over 131,076
  plain fp16 tokens;
* prefill attention: causal chunks of L = 128, 256 (the bench leg) and 2,048
  queries over the packed cache (the reference's prefill_query_block_size 16
  and key chunk 2048 split the same problem, turboquant_cache.py:5146-5199).

The float64 oracle runs over every token of a few (sequence, kv head) groups;
the rest of each problem is checked through a size-independent property
(the last causal row equals a decode of that query).  Bars as in
test_append_dense_gpu (dense indices) and test_attention_gpu (attention).
"""
import math

import numpy as np
import pytest
import torch

from oracle import tq_oracle as O
from kaplumba_amd import ops
from tests.test_append_dense_gpu import BAND
from tests.test_attention_gpu import assert_close

pytestmark = pytest.mark.gpu


def _cfg0_distribution(shape, seeds):
    """N(0,1) x per-(head, channel) log-normal(0, 0.5) scales, as bench.py's inputs."""
    B, H, T, D = shape
    scale = np.exp(np.random.default_rng(seeds[0]).normal(0.0, 0.5, size=(1, H, 1, D)))
    return [(np.random.default_rng(s).standard_normal(shape) * scale).astype(np.float32)
            for s in seeds[1:]]


def _dense_flips(x_in, bits, d, seed, got_packed, got_norms):
    """Norms bit-exact; index flips only inside BAND and by one step. Returns the count."""
    cb = O.beta_codebook(d, bits)
    wp, wn, y = O.quantize_dense(x_in, bits, O.rotation_matrix(d, seed), cb, "float32")
    assert np.array_equal(got_norms, wn), "norms differ"
    gi = O.unpack_lowbit(got_packed, bits, d).astype(np.int8)
    wi = O.unpack_lowbit(wp, bits, d).astype(np.int8)
    bad = gi != wi
    if bad.any():
        mids = O.midpoints(cb).astype(np.float64)
        dist = np.abs(y[bad].astype(np.float64)[:, None] - mids[None, :]).min(axis=1)
        assert dist.max() <= BAND, f"index differs {dist.max():.3g} away from a midpoint"
        assert np.abs(gi[bad].astype(np.int64) - wi[bad]).max() == 1
    return int(bad.sum())


def test_config3_layer_keys_and_values(device):
    """bench.py's cfg3 quantized layer: append_dense_kv_kernel<128, 3, 3, bf16>."""
    H, T, D = 8, 8192, 128
    k32, v32 = _cfg0_distribution((1, H, T, D), (3000, 3001, 3002))
    k = torch.from_numpy(k32).to(torch.bfloat16)
    v = torch.from_numpy(v32).to(torch.bfloat16)
    kc, vc = ops.Codec(D, 3, 0, rotation="dense"), ops.Codec(D, 3, 1, rotation="dense")
    bufs = [(torch.empty((1, H, T, c.packed_width), dtype=torch.uint32, device=device),
             torch.empty((1, H, T), dtype=torch.float32, device=device)) for c in (kc, vc)]
    (kp, kn), (vp, vn) = bufs
    ops.append_quantize_kv(k.to(device), v.to(device), kc, vc, kp, kn, vp, vn, 0)
    for x, (p, n), seed in ((k, bufs[0], 0), (v, bufs[1], 1)):
        flips = _dense_flips(x.float().numpy(), 3, D, seed, p.cpu().numpy().astype(np.uint32),
                             n.cpu().numpy())
        assert flips <= 8, f"seed {seed}: {flips} flips in {H * T * D} coordinates"


def test_config3_plain_layer_copy(device):
    """The fp16 layers of cfg3: a bf16 chunk copied unquantized into the layer buffer."""
    g = torch.Generator().manual_seed(7)
    x = torch.randn(1, 8, 8192, 128, generator=g).to(torch.bfloat16).to(device)
    dst = torch.full((1, 8, 8192 + 256, 128), 7.0, dtype=torch.bfloat16, device=device)
    ops.append_plain(x, dst, 0)
    assert torch.equal(dst[:, :, :8192], x)
    assert (dst[:, :, 8192:] == 7.0).all()


def test_config4_fp16_layer_full_size(device):
    """bench.py's cfg4 fp16-layer leg: attn_plain_kernel over 131,076 fp16 tokens."""
    B, Hq, Hkv, L, T, D = 4, 32, 8, 4, 131072 + 4, 128
    g = torch.Generator().manual_seed(404)
    s = torch.exp(torch.randn(1, Hkv, 1, D, generator=g) * 0.5)
    k = (torch.randn(B, Hkv, T, D, generator=g) * s).half()
    v = (torch.randn(B, Hkv, T, D, generator=g) * s).half()
    q = torch.randn(B, Hq, L, D, generator=g).to(torch.bfloat16)
    scale = 1 / math.sqrt(D)
    kd, vd = k.to(device), v.to(device)
    out = ops.attention_plain(q.to(device), kd, vd, scale, True)
    dec = ops.attention_plain(q[:, :, L - 1:].contiguous().to(device), kd, vd, scale, False)
    assert_close(out[:, :, L - 1:], dec.float().cpu().numpy().astype(np.float64), "bf16",
                 "cfg4 fp16 last draft vs decode")
    R = Hq // Hkv
    for b, gk in ((0, 0), (3, 7)):
        want = O.attention_plain(q[b:b + 1, gk * R:(gk + 1) * R].float().numpy(),
                                 k[b:b + 1, gk:gk + 1].float().numpy(),
                                 v[b:b + 1, gk:gk + 1].float().numpy(), scale=scale,
                                 q_dtype="bf16", causal=True)
        assert_close(out[b:b + 1, gk * R:(gk + 1) * R], want, "bf16", f"cfg4 fp16 b{b} kv{gk}")


@pytest.mark.parametrize("L,T", [(128, 8192), (256, 8192), (2048, 4096)])
def test_prefill_chunk_over_packed_cache(device, L, T):
    """A causal chunk of L queries ending a T-token cache, 32 q / 8 kv heads, 3-bit."""
    Hq, Hkv, D = 32, 8, 128
    k32, v32 = _cfg0_distribution((1, Hkv, T, D), (5000 + L, 5001, 5002))
    kc, vc = ops.Codec(D, 3, 0), ops.Codec(D, 3, 1)
    state = []
    for x, c in ((k32, kc), (v32, vc)):
        pk = torch.empty((1, Hkv, T, c.packed_width), dtype=torch.uint32, device=device)
        nm = torch.empty((1, Hkv, T), dtype=torch.float32, device=device)
        ops.append_quantize(torch.from_numpy(x).half().to(device), c, pk, nm, 0)
        state.append((nm, pk))
    (kn, kp), (vn, vp) = state
    q = torch.from_numpy(np.random.default_rng(L).standard_normal((1, Hq, L, D)).astype(np.float32))
    q = q.to(torch.bfloat16)
    scale = 1 / math.sqrt(D)
    out = ops.attention_packed(q.to(device), kn, kp, vn, vp, kc, vc, scale, True)
    dec = ops.attention_packed(q[:, :, L - 1:].contiguous().to(device), kn, kp, vn, vp, kc, vc,
                               scale, False)
    assert_close(out[:, :, L - 1:], dec.float().cpu().numpy().astype(np.float64), "bf16",
                 f"prefill L{L} last row vs decode")
    R = Hq // Hkv
    groups = (0, 5) if L <= 256 else (3,)
    for gk in groups:
        sl = slice(gk * R, (gk + 1) * R)
        want = O.attention(q[:, sl].float().numpy(), kp[:, gk:gk + 1].cpu().numpy().astype(np.uint32),
                           kn[:, gk:gk + 1].cpu().numpy(),
                           vp[:, gk:gk + 1].cpu().numpy().astype(np.uint32),
                           vn[:, gk:gk + 1].cpu().numpy(), k_bits=3, v_bits=3,
                           k_codebook=kc.codebook, v_codebook=vc.codebook, rot_kind="hadamard",
                           k_rot=O.rht_signs(D, 0), v_rot=O.rht_signs(D, 1), scale=scale,
                           q_dtype="bf16", causal=True)
        assert_close(out[:, sl], want, "bf16", f"prefill L{L} kv{gk}")
