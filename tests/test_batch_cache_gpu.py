"""GPU parity of left-padded (continuous-batching) attention and the batch caches.

tq_attention_ranged skips each row's left padding; the oracle restates the
same problem as attention over the row's own tokens (``starts``), which the
CPU tests tie to the boolean-mask form BatchKVCache.make_mask builds
(models/cache.py:1198-1201).  The cache test replays a continuous-batching
loop (left-padded prefill, decode, a request leaving through ``filter``, a
new one joining through ``extend``) and checks every real query row against
the oracle run on that request alone.  Bar as in test_attention_gpu.
"""
import math

import numpy as np
import pytest
import torch

from oracle import tq_oracle as O
from kaplumba_amd import (BatchKVCache, BatchTurboQuantKVCache, ops,
                          scaled_dot_product_attention)
from tests.test_attention_gpu import TORCH_QDT, assert_close, q_tensor, run_case

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("Hq,Hkv,L,d,kb,vb,rot", [
    (8, 4, 1, 128, 3, 3, "hadamard"),    # small row groups (2 heads x 1 row)
    (8, 4, 2, 64, 4, 2, "hadamard"),     # small row groups at d = 64, causal verify
    (32, 8, 4, 128, 2, 1, "hadamard"),   # 16-row groups
    (16, 8, 1, 256, 4, 2, "dense"),      # d = 256, dense rotation (query prep + dense merge)
])
@pytest.mark.parametrize("norm", ["float32", "float16"])
def test_ranged_packed_attention(device, Hq, Hkv, L, d, kb, vb, rot, norm):
    # rows: no padding; padding inside the first split; one token left;
    # nothing left (zero output); padding and a shorter end together.  With
    # f16 norms an odd start puts the row's norms at an address 2 mod 4, and
    # odd ends exercise the last-token norm patch.
    starts = [0, 700, 2599, 1000, 301]
    lens = [2600, 2600, 2600, 1000, 2001]
    run_case(device, 7 + d + L, 5, Hq, Hkv, L, 2600, d, kb, vb, rot=rot, lengths=lens,
             starts=starts, norm=norm)


@pytest.mark.parametrize("L", [1, 3])
def test_ranged_plain_attention(device, L):
    rng = np.random.default_rng(40 + L)
    B, Hq, Hkv, T, d = 3, 16, 2, 2600, 128
    starts = [0, 1500, 2600]
    k = torch.from_numpy(rng.standard_normal((B, Hkv, T, d)).astype(np.float32)).half()
    v = torch.from_numpy(rng.standard_normal((B, Hkv, T, d)).astype(np.float32)).half()
    q = O.round_to_dtype(rng.standard_normal((B, Hq, L, d)).astype(np.float32), "bf16")
    want = O.attention_plain(q, k.float().numpy(), v.float().numpy(), scale=1 / math.sqrt(d),
                             q_dtype="bf16", causal=L > 1, starts=starts)
    kb = torch.zeros((B, Hkv, T + 5, d), dtype=torch.float16, device=device)
    vb = torch.zeros_like(kb)
    kb[:, :, :T] = k.to(device)
    vb[:, :, :T] = v.to(device)
    out = ops.attention_plain(q_tensor(q, "bf16", device), kb[:, :, :T], vb[:, :, :T],
                              1 / math.sqrt(d), L > 1, seq_starts=torch.tensor(starts))
    assert_close(out, want, "bf16", f"plain ranged L{L}")


class _Request:
    """One sequence's history, replayed through the oracle on its own."""

    def __init__(self):
        self.k, self.v = [], []

    def add(self, k, v):
        self.k.append(k)
        self.v.append(v)

    def oracle(self, q, turbo: bool, D: int):
        k = np.concatenate(self.k, axis=1)[None]  # (1, Hkv, T, D)
        v = np.concatenate(self.v, axis=1)[None]
        if not turbo:
            return O.attention_plain(q[None], k, v, scale=1 / math.sqrt(D), q_dtype="bf16",
                                     causal=q.shape[1] > 1)[0]
        kp, kn = O.quantize_rht(k, 3, O.rht_signs(D, 0), O.beta_codebook(D, 3))
        vp, vn = O.quantize_rht(v, 3, O.rht_signs(D, 1), O.beta_codebook(D, 3))
        return O.attention(q[None], kp, kn, vp, vn, k_bits=3, v_bits=3,
                           k_codebook=O.beta_codebook(D, 3), v_codebook=O.beta_codebook(D, 3),
                           rot_kind="hadamard", k_rot=O.rht_signs(D, 0), v_rot=O.rht_signs(D, 1),
                           scale=1 / math.sqrt(D), q_dtype="bf16", causal=q.shape[1] > 1)[0]


def test_continuous_batching_loop(device):
    """Left-padded prefill, decode, filter (a request leaves), extend (one
    joins), over a TurboQuant layer and an fp16 layer side by side."""
    Hq, Hkv, D = 8, 2, 128
    g = np.random.default_rng(3)

    def rnd(*shape):
        return O.round_to_dtype(g.standard_normal(shape).astype(np.float32), "bf16")

    prompt_lens = [37, 100, 5]
    B, Tp = len(prompt_lens), max(prompt_lens)
    lp = [Tp - n for n in prompt_lens]
    layers = [BatchTurboQuantKVCache(lp, bits=3), BatchKVCache(lp)]
    reqs = [[_Request() for _ in range(B)] for _ in layers]

    def step(caches, requests, kv_rows, q_rows, L, label):
        """kv_rows[b] / q_rows[b]: (Hkv, L, D) / (Hq, L, D) arrays (padding rows zero)."""
        for li, c in enumerate(caches):
            turbo = isinstance(c, BatchTurboQuantKVCache)
            k = np.stack([r[0] for r in kv_rows])
            v = np.stack([r[1] for r in kv_rows])
            mask = c.make_mask(L)
            kt = torch.from_numpy(k).to(torch.bfloat16).to(device)
            vt = torch.from_numpy(v).to(torch.bfloat16).to(device)
            ks, vs = c.update_and_fetch(kt, vt)
            q = np.stack(q_rows)
            out = scaled_dot_product_attention(q_tensor(q, "bf16", device), ks, vs, c,
                                               1 / math.sqrt(D), mask)
            for b, rq in enumerate(requests[li]):
                n_real = min(L, int(c.offset[b]))  # padding rows of a prefill are skipped
                rq.add(k[b][:, L - n_real:], v[b][:, L - n_real:])
                want = rq.oracle(q[b][:, L - n_real:], turbo, D)
                assert_close(out[b:b + 1, :, L - n_real:], want[None], "bf16",
                             f"{label} layer {li} row {b}")
            if turbo:  # the packed rows of each request are the oracle's, bit for bit
                st = c.state[0]
                for b, rq in enumerate(requests[li]):
                    kp, kn = O.quantize_rht(np.concatenate(rq.k, axis=1)[None], 3,
                                            O.rht_signs(D, 0), O.beta_codebook(D, 3))
                    got = st.indices[b:b + 1, :, int(c.left_padding[b]):].cpu().numpy()
                    assert np.array_equal(got.astype(np.uint32), kp), (label, b)

    def rows(n_rows, L, pads=None):
        kv = []
        for b in range(n_rows):
            k, v = rnd(Hkv, L, D), rnd(Hkv, L, D)
            if pads is not None:
                k[:, : pads[b]] = 0
                v[:, : pads[b]] = 0
            kv.append((k, v))
        return kv, [rnd(Hq, L, D) for _ in range(n_rows)]

    kv, q = rows(B, Tp, lp)
    step(layers, reqs, kv, q, Tp, "prefill")
    for i in range(2):
        kv, q = rows(B, 1)
        step(layers, reqs, kv, q, 1, f"decode {i}")
    # the longest request finishes: the others' shared padding is dropped
    for c in layers:
        c.filter([0, 2])
    reqs = [[r[0], r[2]] for r in reqs]
    assert [int(x) for x in layers[0].left_padding] == [0, 32]
    kv, q = rows(2, 1)
    step(layers, reqs, kv, q, 1, "after filter")
    # a new request (prefilled on its own) joins the batch
    newc = [BatchTurboQuantKVCache([0], bits=3), BatchKVCache([0])]
    newr = [[_Request()] for _ in newc]
    kv, q = rows(1, 20)
    step(newc, newr, kv, q, 20, "new prefill")
    for c, n in zip(layers, newc):
        c.extend(n)
    reqs = [r + n for r, n in zip(reqs, newr)]
    for i in range(2):
        kv, q = rows(3, 1)
        step(layers, reqs, kv, q, 1, f"after extend {i}")
    # a verify chunk of 3 draft tokens per row, causal
    kv, q = rows(3, 3)
    step(layers, reqs, kv, q, 3, "verify")
