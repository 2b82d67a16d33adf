"""tq_attention_noalloc: attention with the library's static scratch array.

The entry point takes no workspace: its split partials and rotated queries
live in a per-GPU static device array.  Called through the C ABI, it must
give exactly the output of tq_attention_ranged (the same kernels with a
caller workspace), on two calls in a row with the second one smaller (the
array keeps the first call's contents, which the second must not read), and
on a left-padded dense-rotation problem.
"""
import math

import numpy as np
import pytest
import torch

from kaplumba_amd import _lib, ops
from tests.test_attention_gpu import build_case, q_tensor, to_buffers

pytestmark = pytest.mark.gpu


def _problem(device, seed, B, Hq, Hkv, L, T, d, kb, vb, rot="hadamard", norm="float32"):
    q, kp, kn, vp, vn, _, _ = build_case(seed, B, Hq, Hkv, L, T, d, kb, vb, rot, "bf16", norm)
    nd = torch.float16 if norm == "float16" else torch.float32
    kn_t, ki, vn_t, vi = to_buffers(kp, kn, vp, vn, device, norm_dtype=nd)
    kc, vc = ops.Codec(d, kb, 0, rot), ops.Codec(d, vb, 1, rot)
    return q_tensor(q, "bf16", device), (kn_t, ki, vn_t, vi), kc, vc


def _args(q, kv, kc, vc, causal, starts, lens):
    kn, ki, vn, vi = kv
    B, Hq, L, D = q.shape
    Hkv, T = kn.shape[1], kn.shape[2]
    cap = ops._capacity_of(kn, ki, kc.packed_width)
    dev = q.device
    kt, vt = kc.device_tensors(dev), vc.device_tensors(dev)
    head = (q.data_ptr(), _lib.TQ_DTYPE_BF16, B, Hq, Hkv, L, D, q.stride(0), q.stride(1),
            q.stride(2), 1 / math.sqrt(D), _lib.TQ_KV_PACKED, 0, ki.data_ptr(), kn.data_ptr(),
            vi.data_ptr(), vn.data_ptr(), _lib.torch_dtype_code(kn.dtype), kc.bits, vc.bits,
            kt["codebook"].data_ptr(), vt["codebook"].data_ptr(), kc.rot_kind, kt["rot"].data_ptr(),
            vt["rot"].data_ptr(), cap, T,
            starts.data_ptr() if starts is not None else None,
            lens.data_ptr() if lens is not None else None, 1 if causal else 0)
    return head


def _both(device, q, kv, kc, vc, causal=False, starts=None, lens=None):
    """(no-alloc output, tq_attention_ranged output with a caller workspace)."""
    lib = _lib.load()
    B, Hq, L, D = q.shape
    st = torch.cuda.current_stream(device).cuda_stream
    head = _args(q, kv, kc, vc, causal, starts, lens)
    a = torch.empty((B, Hq, L, D), dtype=q.dtype, device=device)
    b = torch.empty_like(a)
    _lib.check(lib.tq_attention_noalloc(*head, a.data_ptr(), st), "tq_attention_noalloc")
    wsb = lib.tq_attention_workspace_size(B, Hq, kv[0].shape[1], L, D, kv[0].shape[2])
    ws = torch.empty(wsb, dtype=torch.uint8, device=device)
    _lib.check(lib.tq_attention_ranged(*head, b.data_ptr(), ws.data_ptr(), wsb, st),
               "tq_attention_ranged")
    torch.cuda.synchronize(device)
    return a, b


def test_noalloc_matches_the_workspace_entry_point(device):
    # first call: many splits and groups (cfg1-like, 4 sequences); second: a
    # smaller problem, so stale partials of the first sit beyond what it reads
    big = _problem(device, 1, 4, 32, 8, 1, 9000, 128, 3, 3)
    small = _problem(device, 2, 1, 8, 2, 1, 700, 128, 4, 2)
    for q, kv, kc, vc in (big, small):
        a, b = _both(device, q, kv, kc, vc)
        assert torch.equal(a, b)
        assert a.float().abs().sum().item() > 0


def test_noalloc_verify_dense_and_left_padding(device):
    q, kv, kc, vc = _problem(device, 3, 3, 16, 8, 2, 2600, 256, 4, 2, rot="dense", norm="float16")
    starts = torch.tensor([0, 901, 2599], dtype=torch.int32, device=device)
    lens = torch.tensor([2600, 2001, 2600], dtype=torch.int32, device=device)
    a, b = _both(device, q, kv, kc, vc, causal=True, starts=starts, lens=lens)
    assert torch.equal(a, b)
    q2, kv2, kc2, vc2 = _problem(device, 4, 1, 32, 8, 4, 5000, 128, 2, 1)
    a, b = _both(device, q2, kv2, kc2, vc2, causal=True)
    assert torch.equal(a, b)


def test_noalloc_rejects_problems_beyond_the_scratch(device):
    lib = _lib.load()
    need = lib.tq_attention_workspace_size(64, 32, 8, 16, 128, 1 << 20)
    assert need > _lib.TQ_NOALLOC_SCRATCH_BYTES
    rc = lib.tq_attention_noalloc(None, _lib.TQ_DTYPE_BF16, 64, 32, 8, 16, 128, 0, 0, 0, 0.1,
                                  _lib.TQ_KV_PACKED, 0, None, None, None, None, 0, 3, 3, None, None,
                                  0, None, None, 1 << 20, 1 << 20, None, None, 0, None, None)
    assert rc == _lib.TQ_ERR_WORKSPACE and b"scratch" in lib.tq_last_error()
