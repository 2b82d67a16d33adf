"""torch.ops.kaplumba.* without a GPU: registration, schemas and shape functions.

The operators' fake (shape-only) implementations run on fake ROCm tensors,
so the shapes, dtypes and mutation declarations a compiled graph relies on
are checked here; the GPU tests compare compiled and eager results.
"""
import torch
from torch._subclasses.fake_tensor import FakeTensorMode
from torch.fx.experimental.proxy_tensor import make_fx

from kaplumba_amd import ops

OPS = ("append_quantize", "append_quantize_kv", "append_plain", "dequantize", "attention_packed",
       "attention_plain", "prod_quantize", "prod_dequantize", "attention_prod")


def _schema(name):
    return getattr(torch.ops.kaplumba, name).default._schema


def test_operators_registered_with_mutations_declared():
    written = {
        "append_quantize": {"packed", "norms"},
        "append_quantize_kv": {"k_packed", "k_norms", "v_packed", "v_norms"},
        "append_plain": {"dst"},
        "dequantize": set(),
        "attention_packed": set(),
        "attention_plain": set(),
        "prod_quantize": {"norms", "mse_indices", "residual_norms", "qjl_signs"},
        "prod_dequantize": set(),
        "attention_prod": set(),
    }
    for name in OPS:
        s = _schema(name)
        got = {a.name for a in s.arguments if a.alias_info is not None and a.alias_info.is_write}
        assert got == written[name], (name, str(s))
        # outputs never alias inputs
        assert all(r.alias_info is None for r in s.returns), str(s)


def test_fake_shapes():
    kc, vc = ops.Codec(128, 3, 0), ops.Codec(64, 2, 1, "dense")
    f = ops._fields
    with FakeTensorMode():
        B, Hq, Hkv, L, T, cap = 2, 8, 2, 3, 100, 128
        q = torch.empty(B, Hq, L, 128, device="cuda", dtype=torch.bfloat16)
        kn = torch.empty(B, Hkv, cap, device="cuda")[:, :, :T]
        kp = torch.empty(B, Hkv, cap, kc.packed_width, device="cuda", dtype=torch.uint32)[:, :, :T]
        vp = torch.empty(B, Hkv, cap, vc.packed_width, device="cuda", dtype=torch.uint32)[:, :, :T]
        o = torch.ops.kaplumba.attention_packed(q, kn, kp, kn, vp, *f(kc), *f(vc), 0.1, True,
                                                None, None, None)
        assert (o.shape, o.dtype, o.device.type) == ((B, Hq, L, 64), torch.bfloat16, "cuda")
        dq = torch.ops.kaplumba.dequantize(vp, kn, *f(vc))
        assert (dq.shape, dq.dtype) == ((B, Hkv, T, 64), torch.float32)
        keys = torch.empty(B, Hkv, cap, 128, device="cuda", dtype=torch.float16)[:, :, :T]
        vals = torch.empty(B, Hkv, cap, 96, device="cuda", dtype=torch.float16)[:, :, :T]
        q16 = q.to(torch.float16)
        o = torch.ops.kaplumba.attention_plain(q16, keys, vals, 0.1, False, None, None, None)
        assert (o.shape, o.dtype) == ((B, Hq, L, 96), torch.float16)
        sg = torch.empty(B, Hkv, cap, 4, device="cuda", dtype=torch.uint32)[:, :, :T]
        o = torch.ops.kaplumba.attention_prod(q, kn, kp, kn, sg, kn, vp, 128, 3, 0, *f(vc), 0.1,
                                              True, None, None, None)
        assert (o.shape, o.dtype) == ((B, Hq, L, 64), torch.bfloat16)
        dq = torch.ops.kaplumba.prod_dequantize(kn, kp, kn, sg, 128, 3, 0)
        assert (dq.shape, dq.dtype) == ((B, Hkv, T, 128), torch.float32)


def test_step_traces_into_one_graph():
    """An append + attention step traces to the two operators (no host calls in between)."""
    kc, vc = ops.Codec(128, 3, 0), ops.Codec(128, 3, 1)
    f = ops._fields

    def step(q, k, v, kp, kn, vp, vn):
        torch.ops.kaplumba.append_quantize_kv(k, v, kp, kn, vp, vn, 5, *f(kc), *f(vc))
        return torch.ops.kaplumba.attention_packed(q, kn[:, :, :6], kp[:, :, :6], vn[:, :, :6],
                                                   vp[:, :, :6], *f(kc), *f(vc), 0.1, False,
                                                   None, None, None)

    with FakeTensorMode():
        B, Hq, Hkv, cap, d = 1, 4, 2, 16, 128
        args = (torch.empty(B, Hq, 1, d, device="cuda", dtype=torch.bfloat16),
                torch.empty(B, Hkv, 1, d, device="cuda", dtype=torch.bfloat16),
                torch.empty(B, Hkv, 1, d, device="cuda", dtype=torch.bfloat16),
                torch.empty(B, Hkv, cap, kc.packed_width, device="cuda", dtype=torch.uint32),
                torch.empty(B, Hkv, cap, device="cuda"),
                torch.empty(B, Hkv, cap, vc.packed_width, device="cuda", dtype=torch.uint32),
                torch.empty(B, Hkv, cap, device="cuda"))
        gm = make_fx(step)(*args)
    targets = [str(n.target) for n in gm.graph.nodes if n.op == "call_function"]
    assert any("kaplumba.append_quantize_kv" in t for t in targets), targets
    assert any("kaplumba.attention_packed" in t for t in targets), targets
