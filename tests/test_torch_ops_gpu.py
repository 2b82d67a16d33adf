"""torch.ops.kaplumba.*: the hot-path kernels as PyTorch custom operators.

A compiled append + attention step (torch.compile with fullgraph=True, so a
graph break fails the test) must give the same bits as the eager ctypes
path, for packed and plain caches, and torch.library.opcheck must accept
every operator's schema, mutation declarations and shape functions.
"""
import math

import pytest
import torch

from kaplumba_amd import ops

pytestmark = pytest.mark.gpu


def _packed_buffers(device, B, H, cap, kc, vc, norm_dtype=torch.float32):
    return (torch.zeros(B, H, cap, kc.packed_width, dtype=torch.uint32, device=device),
            torch.zeros(B, H, cap, dtype=norm_dtype, device=device),
            torch.zeros(B, H, cap, vc.packed_width, dtype=torch.uint32, device=device),
            torch.zeros(B, H, cap, dtype=norm_dtype, device=device))


def _step(kc, vc, scale):
    def step(q, k, v, kp, kn, vp, vn, off: int):
        ops.append_quantize_kv(k, v, kc, vc, kp, kn, vp, vn, off)
        T = off + k.shape[2]
        return ops.attention_packed(q, kn[:, :, :T], kp[:, :, :T], vn[:, :, :T], vp[:, :, :T],
                                    kc, vc, scale, q.shape[2] > 1)
    return step


@pytest.mark.parametrize("backend", ["aot_eager", "inductor"])
@pytest.mark.parametrize("d,kb,vb,rot", [(128, 3, 3, "hadamard"), (256, 4, 2, "dense")])
def test_compiled_packed_step_matches_eager(device, backend, d, kb, vb, rot):
    torch._dynamo.reset()
    g = torch.Generator(device=device).manual_seed(d + kb)
    B, Hq, Hkv, cap, T0 = 2, 8, 2, 512, 300
    kc, vc = ops.Codec(d, kb, 0, rot), ops.Codec(d, vb, 1, rot)
    scale = 1 / math.sqrt(d)
    steps = [(torch.randn(B, Hq, L, d, device=device, generator=g).to(torch.bfloat16),
              torch.randn(B, Hkv, L, d, device=device, generator=g).to(torch.bfloat16),
              torch.randn(B, Hkv, L, d, device=device, generator=g).to(torch.bfloat16))
             for L in (T0, 1, 1, 4)]
    eager_bufs = _packed_buffers(device, B, Hkv, cap, kc, vc)
    comp_bufs = _packed_buffers(device, B, Hkv, cap, kc, vc)
    eager = _step(kc, vc, scale)
    compiled = torch.compile(_step(kc, vc, scale), backend=backend, fullgraph=True)
    off = 0
    for q, k, v in steps:
        want = eager(q, k, v, *eager_bufs, off)
        got = compiled(q, k, v, *comp_bufs, off)
        torch.cuda.synchronize()
        assert got.shape == want.shape and got.dtype == want.dtype
        assert torch.equal(got, want), f"{backend}: step at offset {off} differs from eager"
        for a, b in zip(comp_bufs, eager_bufs):
            assert torch.equal(a, b), f"{backend}: cache buffers differ after offset {off}"
        off += k.shape[2]


@pytest.mark.parametrize("backend", ["aot_eager", "inductor"])
def test_compiled_plain_and_dequantize_match_eager(device, backend):
    torch._dynamo.reset()
    g = torch.Generator(device=device).manual_seed(7)
    B, Hq, Hkv, cap, T, d = 1, 8, 2, 256, 200, 128
    kc = ops.Codec(d, 3, 0)
    x = torch.randn(B, Hkv, T, d, device=device, generator=g).to(torch.float16)
    q = torch.randn(B, Hq, 1, d, device=device, generator=g).to(torch.float16)

    def fn(x, q, kb, vb, pk, nk):
        ops.append_plain(x, kb, 0)
        ops.append_plain(x * 0.5, vb, 0)
        ops.append_quantize(x, kc, pk, nk, 0)
        o = ops.attention_plain(q, kb[:, :, :T], vb[:, :, :T], 0.125, False,
                                seq_lens=torch.tensor([150], dtype=torch.int32, device=q.device))
        return o, ops.dequantize(pk[:, :, :T], nk[:, :, :T], kc)

    def bufs():
        return (torch.zeros(B, Hkv, cap, d, dtype=torch.float16, device=device),
                torch.zeros(B, Hkv, cap, d, dtype=torch.float16, device=device),
                torch.zeros(B, Hkv, cap, kc.packed_width, dtype=torch.uint32, device=device),
                torch.zeros(B, Hkv, cap, dtype=torch.float32, device=device))

    be, bc = bufs(), bufs()
    want = fn(x, q, *be)
    got = torch.compile(fn, backend=backend, fullgraph=True)(x, q, *bc)
    torch.cuda.synchronize()
    for a, b in zip(got, want):
        assert torch.equal(a, b)
    for a, b in zip(bc, be):
        assert torch.equal(a, b)


def test_opcheck_every_operator(device):
    g = torch.Generator(device=device).manual_seed(11)
    B, Hq, Hkv, cap, T, d = 1, 4, 2, 96, 70, 64
    kc, vc = ops.Codec(d, 2, 0), ops.Codec(d, 3, 1)
    f = ops._fields
    x = torch.randn(B, Hkv, T, d, device=device, generator=g).to(torch.bfloat16)
    kp, kn, vp, vn = _packed_buffers(device, B, Hkv, cap, kc, vc)
    torch.library.opcheck(torch.ops.kaplumba.append_quantize.default, (x, kp, kn, 0, *f(kc)))
    kp, kn, vp, vn = _packed_buffers(device, B, Hkv, cap, kc, vc)
    torch.library.opcheck(torch.ops.kaplumba.append_quantize_kv.default,
                          (x, x * 2, kp, kn, vp, vn, 0, *f(kc), *f(vc)))
    q = torch.randn(B, Hq, 2, d, device=device, generator=g).to(torch.bfloat16)
    lens = torch.tensor([50], dtype=torch.int32, device=device)
    torch.library.opcheck(torch.ops.kaplumba.attention_packed.default,
                          (q, kn[:, :, :T], kp[:, :, :T], vn[:, :, :T], vp[:, :, :T], *f(kc), *f(vc),
                           0.125, True, lens, None, None))
    torch.library.opcheck(torch.ops.kaplumba.dequantize.default,
                          (kp[:, :, :T], kn[:, :, :T], *f(kc)))
    plain = torch.zeros(B, Hkv, cap, d, dtype=torch.bfloat16, device=device)
    torch.library.opcheck(torch.ops.kaplumba.append_plain.default, (x, plain, 0))
    mask = torch.ones(2, T, dtype=torch.bool, device=device).tril(T - 2)
    torch.library.opcheck(torch.ops.kaplumba.attention_plain.default,
                          (q, plain[:, :, :T], plain[:, :, :T], 0.125, False, None, None, mask))


@pytest.mark.parametrize("bits,quantizer", [(3, "mse"), (3.5, "mse"), (3, "prod")])
def test_compiled_cache_layer_matches_eager(device, bits, quantizer):
    """A model layer's cache calls (update_and_fetch, then the SDPA dispatch) under
    torch.compile: prefill, cache growth and decode steps give the eager bits."""
    from kaplumba_amd import TurboQuantKVCache, scaled_dot_product_attention

    torch._dynamo.reset()

    def layer(cache, q, k, v):
        ks, vs = cache.update_and_fetch(k, v)
        mask = "causal" if q.shape[2] > 1 else None
        return scaled_dot_product_attention(q, ks, vs, cache, 1 / math.sqrt(q.shape[-1]), mask)

    g = torch.Generator(device=device).manual_seed(int(bits * 10))
    ce = TurboQuantKVCache(bits=bits, key_quantizer=quantizer)
    cc = TurboQuantKVCache(bits=bits, key_quantizer=quantizer)
    compiled = torch.compile(layer, backend="aot_eager")
    for L in (40, 1, 1, 3, 300):
        q = torch.randn(1, 8, L, 128, device=device, generator=g).to(torch.bfloat16)
        k = torch.randn(1, 2, L, 128, device=device, generator=g).to(torch.bfloat16)
        v = torch.randn(1, 2, L, 128, device=device, generator=g).to(torch.bfloat16)
        want = layer(ce, q, k, v)
        got = compiled(cc, q, k, v)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"L={L}: compiled layer differs from eager"
        assert cc.offset == ce.offset


def test_opcheck_prod_operators(device):
    from kaplumba_amd import prod

    g = torch.Generator(device=device).manual_seed(13)
    B, Hq, Hkv, cap, T, d = 1, 4, 2, 96, 70, 128
    pc, vc = prod.ProdCodec(d, 3, 0), ops.Codec(d, 3, 1)
    x = torch.randn(B, Hkv, T, d, device=device, generator=g).to(torch.bfloat16)
    st = pc.alloc(B, Hkv, cap, device)
    torch.library.opcheck(torch.ops.kaplumba.prod_quantize.default, (x, *st, 0, d, 3, 0))
    pc.quantize_into(x, st, 0)
    view = [t[:, :, :T] for t in st]
    torch.library.opcheck(torch.ops.kaplumba.prod_dequantize.default, (*view, d, 3, 0))
    vp = torch.zeros(B, Hkv, cap, vc.packed_width, dtype=torch.uint32, device=device)
    vn = torch.zeros(B, Hkv, cap, dtype=torch.float32, device=device)
    ops.append_quantize(x, vc, vp, vn, 0)
    q = torch.randn(B, Hq, 1, d, device=device, generator=g).to(torch.bfloat16)
    torch.library.opcheck(torch.ops.kaplumba.attention_prod.default,
                          (q, *view, vn[:, :, :T], vp[:, :, :T], d, 3, 0, *ops._fields(vc), 0.09,
                           False, None, None, None))
