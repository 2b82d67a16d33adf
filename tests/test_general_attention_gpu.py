"""GPU parity of the general attention path (tq_attention_general and the
shapes the tuned entry points hand to it) vs the float64 oracle.

Covers what the tuned kernels do not build: head dim 512 (Gemma-4 global
layers, gemma4_text.py:24, 185-190), dims that are not powers of two (the
dense rotation, turboquant_cache.py:4125-4133), key and value dims that
differ (the output takes the value dim, :5131), array masks applied as
_apply_attention_mask (:5079-5108) on the TurboQuant path and as the fp16
layers' SDPA mask (base.py:218-226), and Prod-coded keys beyond d <= 128 /
4 rows per kv head, including 1-bit Prod (score_prepared, :4700-4766).
Bar as in test_attention_gpu: within max(2e-3, 1 ulp of the query dtype) and
1e-3 mean-rel of the oracle.
"""
import math

import numpy as np
import pytest
import torch

from oracle import tq_oracle as O
from kaplumba_amd import ops
from kaplumba_amd.cache import create_causal_mask
from tests.test_attention_gpu import assert_close, q_tensor, run_case, to_buffers

pytestmark = pytest.mark.gpu


def _side(rng, shape, bits, d, rot, seed, norm):
    s = np.exp(rng.normal(0, 0.5, size=(1, shape[1], 1, d)))
    x = (rng.standard_normal(shape) * s).astype(np.float16).astype(np.float32)
    if rot == "hadamard":
        r = O.rht_signs(d, seed)
        p, n = O.quantize_rht(x, bits, r, O.beta_codebook(d, bits), norm)
    else:
        r = O.rotation_matrix(d, seed)
        p, n, _ = O.quantize_dense(x, bits, r, O.beta_codebook(d, bits), norm)
    return p, n, r


def packed_case(device, seed, B, Hq, Hkv, L, T, dk, dv, kb, vb, krot="hadamard", vrot="hadamard",
                qdt="bf16", causal=None, lengths=None, starts=None, mask_np=None, mask_t=None,
                norm="float32"):
    """One packed-cache call through ops.attention_packed vs O.attention."""
    causal = (L > 1) if causal is None else causal
    rng = np.random.default_rng(seed)
    kp, kn, kr = _side(rng, (B, Hkv, T, dk), kb, dk, krot, 0, norm)
    vp, vn, vr = _side(rng, (B, Hkv, T, dv), vb, dv, vrot, 1, norm)
    q = O.round_to_dtype(rng.standard_normal((B, Hq, L, dk)).astype(np.float32), qdt)
    want = O.attention(q, kp, kn, vp, vn, k_bits=kb, v_bits=vb, k_codebook=O.beta_codebook(dk, kb),
                       v_codebook=O.beta_codebook(dv, vb), rot_kind=krot, k_rot=kr, v_rot=vr,
                       scale=1 / math.sqrt(dk), q_dtype=qdt, causal=causal, lengths=lengths,
                       starts=starts, v_dim=dv, mask=mask_np, v_rot_kind=vrot)
    nd = torch.float16 if norm == "float16" else torch.float32
    kn_t, ki, vn_t, vi = to_buffers(kp, kn, vp, vn, device, norm_dtype=nd)
    out = ops.attention_packed(
        q_tensor(q, qdt, device), kn_t, ki, vn_t, vi, ops.Codec(dk, kb, 0, krot),
        ops.Codec(dv, vb, 1, vrot), 1 / math.sqrt(dk), causal,
        seq_lens=None if lengths is None else torch.tensor(lengths, dtype=torch.int32),
        seq_starts=None if starts is None else torch.tensor(starts, dtype=torch.int32),
        mask=mask_t if mask_t is not None else (None if mask_np is None else torch.from_numpy(mask_np).to(device)))
    assert out.shape == (B, Hq, L, dv)
    assert_close(out, want, qdt, f"B{B} Hq{Hq} Hkv{Hkv} L{L} T{T} k{dk}{krot[0]}{kb} v{dv}{vrot[0]}{vb}")
    return out


# --------------------------------------------------------------- head dims ---
@pytest.mark.parametrize("Hq,Hkv,L,T", [(8, 2, 1, 3000), (32, 4, 1, 777), (8, 2, 4, 2100),
                                        (16, 16, 1, 64)])
@pytest.mark.parametrize("kb,vb", [(3, 3), (4, 2), (2, 1)])
def test_head_dim_512_hadamard(device, Hq, Hkv, L, T, kb, vb):
    """Gemma-4 global layers: d = 512 through tq_attention (routed to the general kernels)."""
    run_case(device, 500 + 7 * kb + vb + L, 1, Hq, Hkv, L, T, 512, kb, vb)


@pytest.mark.parametrize("d", [80, 96, 192, 320, 512, 13, 50, 99, 130])
def test_dense_rotation_other_dims(device, d):
    """Non-power-of-two dims take the dense rotation (turboquant_cache.py:4125-4133);
    d = 512 asks for it explicitly."""
    run_case(device, 600 + d, 2, 8, 2, 1, 900, d, 3, 3, rot="dense", lengths=[900, 417])


def test_head_dim_512_verify_ragged_f16_norms(device):
    run_case(device, 611, 3, 8, 4, 3, 1500, 512, 3, 4, qdt="f16", norm="float16",
             lengths=[1500, 3, 611])


def test_head_dim_512_left_padding(device):
    run_case(device, 612, 2, 8, 2, 1, 1300, 512, 4, 3, starts=[0, 1000], lengths=[1300, 1250])


# ------------------------------------------------------- K and V dims differ ---
@pytest.mark.parametrize("dk,krot,dv,vrot", [(128, "hadamard", 64, "hadamard"),
                                             (192, "dense", 128, "hadamard"),
                                             (64, "hadamard", 96, "dense"),
                                             (128, "hadamard", 128, "dense"),
                                             (256, "hadamard", 512, "hadamard"),
                                             (100, "dense", 37, "dense"),
                                             (64, "hadamard", 130, "dense")])
def test_key_and_value_dims_differ(device, dk, krot, dv, vrot):
    packed_case(device, 700 + dk + dv, 2, 8, 2, 1, 1700, dk, dv, 3, 2, krot, vrot,
                lengths=[1700, 900])
    packed_case(device, 701 + dk + dv, 1, 4, 2, 3, 500, dk, dv, 4, 3, krot, vrot)


# ------------------------------------------------------------------ masks ---
@pytest.mark.parametrize("L", [1, 4])
def test_sliding_window_bool_mask(device, L):
    """create_causal_mask(window_size=...) returns an array the attention now takes."""
    T, W = 2000, 256
    m = create_causal_mask(L, offset=T - L, window_size=W)
    assert m.shape == (L, T) and m.dtype == torch.bool
    packed_case(device, 800 + L, 1, 32, 8, L, T, 128, 128, 3, 3, causal=False, mask_np=m.numpy())


@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("shape", ["2d", "4d", "5d"])
def test_additive_masks(device, dt, shape):
    B, Hq, Hkv, L, T = 2, 8, 2, 2, 1100
    R = Hq // Hkv
    rng = np.random.default_rng(810)
    full = {"2d": (L, T), "4d": (B, Hkv, L, T), "5d": (B, Hkv, R, L, T)}[shape]
    m = rng.normal(0, 2.0, size=full).astype(np.float32)
    m[rng.random(full) < 0.3] = -6e4  # finite in every mask dtype
    m = O.round_to_dtype(m, dt)
    tdt = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}[dt]
    mt = torch.from_numpy(m).to(tdt).to(device)
    packed_case(device, 811, B, Hq, Hkv, L, T, 128, 128, 4, 2, causal=True, mask_np=m, mask_t=mt)


def test_bool_mask_ragged_left_padded_and_dense(device):
    B, Hq, Hkv, L, T = 3, 8, 2, 2, 1400
    rng = np.random.default_rng(820)
    m = rng.random((B, 1, 1, L, T)) < 0.7
    packed_case(device, 821, B, Hq, Hkv, L, T, 256, 256, 3, 3, "dense", "dense", causal=True,
                lengths=[1400, 700, 1399], starts=[0, 100, 1300], mask_np=m)


def test_fully_masked_rows_average_every_value(device):
    """A row whose mask hides every key: every score is f32 min, so the softmax
    is uniform (the reference's where(mask, s, finfo.min) then softmax)."""
    B, Hq, Hkv, L, T = 1, 4, 1, 3, 800
    m = np.ones((L, T), bool)
    m[1] = False
    packed_case(device, 830, B, Hq, Hkv, L, T, 128, 128, 3, 3, causal=False, mask_np=m)


def test_mask_through_the_cache_api(device):
    """TurboQuantKVCache + scaled_dot_product_attention with a sliding-window
    array mask from create_attention_mask, vs the oracle on the cache's own state."""
    from kaplumba_amd import TurboQuantKVCache, create_attention_mask, scaled_dot_product_attention

    B, Hq, Hkv, D, T0 = 1, 8, 2, 128, 600
    g = torch.Generator().manual_seed(840)
    cache = TurboQuantKVCache(bits=3)
    cache.update_and_fetch(torch.randn(B, Hkv, T0, D, generator=g).to(torch.bfloat16).to(device),
                           torch.randn(B, Hkv, T0, D, generator=g).to(torch.bfloat16).to(device))
    L = 3
    ks, vs = cache.update_and_fetch(torch.randn(B, Hkv, L, D, generator=g).to(torch.bfloat16).to(device),
                                    torch.randn(B, Hkv, L, D, generator=g).to(torch.bfloat16).to(device))
    q = torch.randn(B, Hq, L, D, generator=g).to(torch.bfloat16)
    mask = create_attention_mask(torch.zeros(B, L, D), cache=None, window_size=100, offset=T0)
    assert isinstance(mask, torch.Tensor)
    out = scaled_dot_product_attention(q.to(device), ks, vs, cache, 1 / math.sqrt(D), mask)
    st_k, st_v = cache.state
    want = O.attention(q.float().numpy(), st_k.indices.cpu().numpy().astype(np.uint32),
                       st_k.norms.float().cpu().numpy(), st_v.indices.cpu().numpy().astype(np.uint32),
                       st_v.norms.float().cpu().numpy(), k_bits=3, v_bits=3,
                       k_codebook=O.beta_codebook(D, 3), v_codebook=O.beta_codebook(D, 3),
                       rot_kind="hadamard", k_rot=O.rht_signs(D, cache.seed),
                       v_rot=O.rht_signs(D, cache.seed + 1), scale=1 / math.sqrt(D), q_dtype="bf16",
                       mask=mask.numpy())
    assert_close(out, want, "bf16", "cache api window mask")


# --------------------------------------------------------- plain fp16 layers ---
def _plain_case(device, seed, B, Hq, Hkv, L, T, dk, dv, kvdt=torch.float16, mask_np=None,
                causal=None, lengths=None):
    causal = (L > 1) if causal is None else causal
    rng = np.random.default_rng(seed)
    kvn = "f16" if kvdt == torch.float16 else "bf16"
    k = O.round_to_dtype(rng.standard_normal((B, Hkv, T, dk)).astype(np.float32), kvn)
    v = O.round_to_dtype(rng.standard_normal((B, Hkv, T, dv)).astype(np.float32), kvn)
    q = O.round_to_dtype(rng.standard_normal((B, Hq, L, dk)).astype(np.float32), "bf16")
    want = O.attention_plain(q, k, v, scale=1 / math.sqrt(dk), q_dtype="bf16", causal=causal,
                             lengths=lengths, mask=mask_np)
    cap = T + 9
    kb = torch.zeros((B, Hkv, cap, dk), dtype=kvdt, device=device)
    vb = torch.zeros((B, Hkv, cap, dv), dtype=kvdt, device=device)
    kb[:, :, :T] = torch.from_numpy(k).to(kvdt).to(device)
    vb[:, :, :T] = torch.from_numpy(v).to(kvdt).to(device)
    out = ops.attention_plain(q_tensor(q, "bf16", device), kb[:, :, :T], vb[:, :, :T],
                              1 / math.sqrt(dk), causal,
                              seq_lens=None if lengths is None else torch.tensor(lengths, dtype=torch.int32),
                              mask=None if mask_np is None else torch.from_numpy(mask_np).to(device))
    assert out.shape == (B, Hq, L, dv)
    assert_close(out, want, "bf16", f"plain B{B} Hq{Hq} Hkv{Hkv} L{L} T{T} k{dk} v{dv}")


@pytest.mark.parametrize("dk,dv", [(512, 512), (96, 96), (192, 128), (100, 100), (13, 37), (130, 66)])
def test_plain_layers_other_dims(device, dk, dv):
    _plain_case(device, 900 + dk + dv, 2, 8, 2, 2, 1300, dk, dv, lengths=[1300, 640])


def test_plain_layers_with_array_mask(device):
    """The fp16 layers' SDPA broadcasts the mask against (B, Hq, L, T)."""
    B, Hq, Hkv, L, T = 2, 8, 2, 3, 900
    rng = np.random.default_rng(910)
    m = rng.random((B, Hq, L, T)) < 0.8
    _plain_case(device, 911, B, Hq, Hkv, L, T, 128, 128, torch.bfloat16, mask_np=m, causal=False)
    ma = O.round_to_dtype(rng.normal(0, 1, (1, 1, L, T)).astype(np.float32), "f32")
    _plain_case(device, 912, B, Hq, Hkv, L, T, 128, 128, mask_np=ma)


# -------------------------------------------------------------------- Prod ---
def prod_case(device, seed, B, Hq, Hkv, L, T, d, kb, vb, qdt="bf16", lengths=None, causal=None,
              mask_np=None, vd=None, vrot="hadamard"):
    from kaplumba_amd.prod import ProdCodec, attention_prod

    causal = (L > 1) if causal is None else causal
    vd = d if vd is None else vd
    rng = np.random.default_rng(seed)
    k = (rng.standard_normal((B, Hkv, T, d))).astype(np.float16)
    q = O.round_to_dtype(rng.standard_normal((B, Hq, L, d)).astype(np.float32), qdt)
    kc = ProdCodec(d, kb, 0)
    kst = kc.alloc(B, Hkv, T + 7, device)  # the capacity to_buffers gives the values
    kc.quantize_into(torch.from_numpy(k).to(device), kst, 0)
    vp, vn, vr = _side(rng, (B, Hkv, T, vd), vb, vd, vrot, 1, "float32")
    vn_t, vi, _, _ = to_buffers(vp, vn, vp, vn, device)
    view = type(kst)(*(t[:, :, :T] for t in kst))
    out = attention_prod(q_tensor(q, qdt, device), view, vn_t, vi, kc, ops.Codec(vd, vb, 1, vrot),
                         1 / math.sqrt(d), causal,
                         seq_lens=None if lengths is None else torch.tensor(lengths, dtype=torch.int32),
                         mask=None if mask_np is None else torch.from_numpy(mask_np).to(device))
    kn, km, kr, ks = (t[:, :, :T].float().cpu().numpy() if t.dtype != torch.uint32
                      else t[:, :, :T].cpu().numpy().astype(np.uint32) for t in kst)
    if vrot == "hadamard" and vd == d:
        want = O.attention_prod(q, kn, km, kr, ks, vp, vn, k_bits=kb, v_bits=vb,
                                k_signs_rot=O.rht_signs(d, 0),
                                k_mse_codebook=O.beta_codebook(d, kb - 1) if kb > 1 else None,
                                proj=O.projection_matrix(d, 1), v_codebook=O.beta_codebook(vd, vb),
                                v_rot=vr, scale=1 / math.sqrt(d), q_dtype=qdt, causal=causal,
                                lengths=lengths, mask=mask_np)
    else:
        # keys dequantized by the pinned prod_key_vectors, values through the
        # packed oracle's value path: the same bilinear forms as attention_prod
        want = _prod_general_oracle(q, kn, km, kr, ks, vp, vn, kb, vb, d, vd, vr, vrot, qdt,
                                    causal, lengths, mask_np)
    assert out.shape == (B, Hq, L, vd)
    assert_close(out, want, qdt, f"prod B{B} Hq{Hq} Hkv{Hkv} L{L} T{T} d{d} v{vd}{vrot[0]} k{kb}v{vb}")


def _prod_general_oracle(q, kn, km, kr, ks, vp, vn, kb, vb, d, vd, vr, vrot, qdt, causal, lengths,
                         mask_np):
    B, Hq, L, _ = q.shape
    Hkv = kn.shape[1]
    R = Hq // Hkv
    pow2 = d & (d - 1) == 0  # the Prod codec's MSE rotation: Hadamard, else dense
    keys = O.prod_key_vectors(kn, km, kr, ks, bits=kb, dim=d,
                              signs=O.rht_signs(d, 0) if pow2 else O.rotation_matrix(d, 0),
                              mse_codebook=O.beta_codebook(d, kb - 1) if kb > 1 else None,
                              proj=O.projection_matrix(d, 1), rot_kind="hadamard" if pow2 else "dense")
    vals = O.dequantize(vp, vn, vb, vd, O.beta_codebook(vd, vb), vrot, vr).astype(np.float64)
    qs = O.scale_queries(q, 1 / math.sqrt(d), qdt).astype(np.float64)
    T = kn.shape[2]
    m5 = None if mask_np is None else O.mask_5d(mask_np, B, Hkv, R, L, T)
    out = np.zeros((B, Hq, L, vd))
    for b in range(B):
        e = T if lengths is None else lengths[b]
        for h in range(Hq):
            g, r = h // R, h % R
            s = qs[b, h] @ keys[b, g, :e].T
            if causal:
                s = np.where((e - L) + np.arange(L)[:, None] >= np.arange(e)[None, :], s,
                             float(np.finfo(np.float32).min))
            if m5 is not None:
                s = O.apply_mask(s, m5[b, g, r, :, :e])
            p = np.exp(s - s.max(axis=-1, keepdims=True))
            out[b, h] = (p @ vals[b, g, :e]) / np.maximum(p.sum(axis=-1, keepdims=True), 1e-6)
    return out


@pytest.mark.parametrize("kb,vb", [(3, 3), (4, 2), (2, 1)])
def test_prod_head_dim_256(device, kb, vb):
    prod_case(device, 1000 + kb * 10 + vb, 1, 8, 2, 1, 1800, 256, kb, vb)


@pytest.mark.parametrize("d,kb,vb", [(512, 3, 3), (512, 4, 2), (32, 3, 3), (32, 2, 1)])
def test_prod_head_dims_32_and_512(device, d, kb, vb):
    """Prod keys quantized at d = 32 and 512 (the residual kernel's one- and
    sixteen-lane groups, the general signs projection) and attended over."""
    prod_case(device, 1040 + d + kb * 10 + vb, 1, 8, 2, 1, 1300, d, kb, vb)


def test_prod_many_rows_per_kv_head(device):
    """16 query rows per kv head (GQA 4 x 4 causal drafts)."""
    prod_case(device, 1010, 2, 32, 8, 4, 700, 128, 3, 3, lengths=[700, 333])


@pytest.mark.parametrize("d,kb,vb", [(48, 3, 3), (100, 4, 2), (99, 1, 3), (200, 2, 2)])
def test_prod_dense_rotation_dims(device, d, kb, vb):
    """Prod keys at dims that are not powers of two (dense MSE rotation,
    ceil(d / 32) sign words) with dense values."""
    prod_case(device, 1100 + d + kb, 1, 8, 2, 1, 900, d, kb, vb, vrot="dense")
    prod_case(device, 1101 + d + kb, 2, 8, 4, 3, 400, d, kb, vb, vrot="dense", lengths=[400, 151])


@pytest.mark.parametrize("d", [32, 64, 128, 256, 512])
def test_prod_one_bit(device, d):
    """1-bit Prod: no MSE part, the score is the QJL term alone."""
    prod_case(device, 1020 + d, 1, 8, 2, 1, 900, d, 1, 3)


def test_prod_with_mask_and_dense_values(device):
    rng = np.random.default_rng(1030)
    m = rng.random((1, 2, 2, 600)) < 0.75
    prod_case(device, 1031, 1, 8, 2, 2, 600, 128, 3, 2, mask_np=m)
    prod_case(device, 1032, 1, 8, 2, 1, 600, 128, 4, 3, vd=96, vrot="dense")
