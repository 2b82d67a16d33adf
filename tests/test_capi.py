"""The C-ABI library loads, exports every declared symbol and validates input (CPU only).

No test here launches a kernel: argument checks run on the host before any
HIP call, so they are exercised without a GPU.
"""
import ctypes
import os
import re

import pytest

from kaplumba_amd import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include",
                      "kaplumba_tq.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tq_[a-z_]+)\s*\(", text)))


def test_header_declares_the_bound_set():
    assert declared_functions() == sorted(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_functions():
        assert hasattr(lib, name), name
        assert ctypes.cast(getattr(lib, name), ctypes.c_void_p).value


def test_version_and_packed_width():
    lib = _lib.load()
    assert lib.tq_version().startswith(b"kaplumba_tq")
    assert lib.tq_packed_width(128, 3) == 12
    assert lib.tq_packed_width(256, 4) == 32
    assert lib.tq_packed_width(64, 1) == 2
    assert lib.tq_packed_width(0, 3) == 0


def test_workspace_size_is_positive_and_grows():
    lib = _lib.load()
    a = lib.tq_attention_workspace_size(1, 32, 8, 1, 128, 32768)
    b = lib.tq_attention_workspace_size(4, 32, 8, 4, 128, 131072)
    assert 0 < a < b
    assert lib.tq_attention_workspace_size(1, 32, 7, 1, 128, 10) == 0  # Hq % Hkv != 0


@pytest.mark.parametrize("bits", [0, 5])
def test_append_rejects_bad_bits_without_touching_the_gpu(bits):
    lib = _lib.load()
    rc = lib.tq_append_quantize(None, 1, 1, 1, 1, 128, 128, 128, 128, bits, 0, None, None,
                                None, None, 0, 16, 0, None)
    assert rc == _lib.TQ_ERR_INVALID_ARGUMENT
    assert b"bits" in lib.tq_last_error()


def test_append_rejects_capacity_overflow_and_nulls():
    lib = _lib.load()
    rc = lib.tq_append_quantize(None, 1, 1, 1, 5, 128, 640, 640, 128, 3, 0, None, None,
                                None, None, 0, 4, 0, None)
    assert rc == _lib.TQ_ERR_INVALID_ARGUMENT and b"capacity" in lib.tq_last_error()
    rc = lib.tq_append_quantize(None, 1, 1, 1, 1, 128, 128, 128, 128, 3, 0, None, None,
                                None, None, 0, 4, 0, None)
    assert rc == _lib.TQ_ERR_INVALID_ARGUMENT and b"null" in lib.tq_last_error()
    # empty append is a no-op success
    assert lib.tq_append_quantize(None, 1, 0, 1, 1, 128, 0, 0, 0, 3, 0, None, None,
                                  None, None, 0, 4, 0, None) == _lib.TQ_OK


def test_attention_rejects_unsupported_dim_and_bad_heads():
    lib = _lib.load()
    args = [None, 2, 1, 32, 8, 1, 1024, 0, 0, 0, 0.1, 0, 0, None, None, None, None, 0, 3, 3,
            None, None, 0, None, None, 16, 16, None, 0, None, None, 0, None]
    assert lib.tq_attention(*args) == _lib.TQ_ERR_UNSUPPORTED
    args[6] = 96  # not a power of two: only the dense rotation
    assert lib.tq_attention(*args) == _lib.TQ_ERR_INVALID_ARGUMENT
    assert b"power-of-two" in lib.tq_last_error()
    args[6] = 128
    args[4] = 7
    assert lib.tq_attention(*args) == _lib.TQ_ERR_INVALID_ARGUMENT
    args[4] = 8
    args[18] = 5  # k_bits
    assert lib.tq_attention(*args) == _lib.TQ_ERR_INVALID_ARGUMENT


def test_attention_rejects_kv_heads_beyond_the_small_rows_field():
    # decode with <= 4 query rows per kv head packs the kv head count into 12
    # bits of a launch argument: 4096 kv heads are refused before any launch
    # (the pointers are never dereferenced: the check precedes every HIP call)
    lib = _lib.load()
    fake = 1 << 20
    args = [fake, 2, 2, 4096, 4096, 1, 128, 0, 0, 0, 0.1, 0, 0, None, None, None, None, 0, 3, 3,
            fake, fake, 0, fake, fake, 16, 0, None, 0, fake, fake, 1 << 30, None]
    assert lib.tq_attention(*args) == _lib.TQ_ERR_UNSUPPORTED
    assert b"kv heads" in lib.tq_last_error()


def test_workspace_growth_keeps_retired_buffers_bounded():
    # a long decode asks for a larger workspace as T grows; replacements at
    # least double, so the buffers kept alive for captured graphs add up to
    # less than the current one
    from kaplumba_amd import ops
    lib = _lib.load()
    for (B, Hq, Hkv, D) in ((1, 8, 1, 128), (1, 8, 1, 256), (1, 32, 8, 512), (4, 32, 8, 128)):
        cur, retired, replacements = 0, 0, 0
        for T in range(1, 128 * 1024 + 1, 97):
            need = lib.tq_attention_workspace_size(B, Hq, Hkv, 1, D, T)
            if need > cur:
                retired += cur
                cur = ops._grown_size(cur, need)
                replacements += 1
        assert retired <= cur, (B, Hq, Hkv, D, retired, cur)
        assert replacements <= 16, replacements


def _general_args(**kw):
    """tq_attention_general arguments of a B = 0 call (validated, nothing launched)."""
    a = dict(q=None, q_dtype=2, B=0, Hq=32, Hkv=8, L=1, k_dim=128, v_dim=64, sb=0, sh=0, sl=0,
             scale=0.1, kv_kind=_lib.TQ_KV_PACKED, kv_dtype=0, k=None, kn=None, ks=None, krn=None,
             k_bits=3, kcb=None, k_rot_kind=0, k_rot=None, proj=None, v=None, vn=None, v_bits=3,
             vcb=None, v_rot_kind=1, v_rot=None, norm_dtype=0, cap=16, T=0, starts=None,
             lens=None, causal=0, mask=None, mask_kind=0, mstrides=None, out=None, ws=None,
             wsb=0, stream=None)
    a.update(kw)
    return list(a.values())


def test_general_attention_validates_without_the_gpu():
    lib = _lib.load()
    fake = ctypes.c_void_p(16)
    ok = dict(kcb=fake, k_rot=fake, vcb=fake, v_rot=fake)
    assert lib.tq_attention_general(*_general_args(**ok)) == _lib.TQ_OK  # B = 0
    # any dim in 8..512 with the dense rotation, odd ones included
    for kw in (dict(v_dim=100), dict(v_dim=37), dict(k_rot_kind=1, k_dim=99)):
        assert lib.tq_attention_general(*_general_args(**dict(ok, **kw))) == _lib.TQ_OK, kw
    bad = [
        (dict(k_dim=520), _lib.TQ_ERR_UNSUPPORTED, b"head dims"),
        (dict(v_dim=7), _lib.TQ_ERR_UNSUPPORTED, b"head dims"),
        (dict(k_dim=96), _lib.TQ_ERR_INVALID_ARGUMENT, b"power-of-two"),   # Hadamard keys
        (dict(v_rot_kind=0, v_dim=96), _lib.TQ_ERR_INVALID_ARGUMENT, b"power-of-two"),
        (dict(mask_kind=1), _lib.TQ_ERR_INVALID_ARGUMENT, b"mask"),
        (dict(mask_kind=7, mask=fake, mstrides=fake), _lib.TQ_ERR_INVALID_ARGUMENT, b"mask_kind"),
        (dict(k_bits=5), _lib.TQ_ERR_INVALID_ARGUMENT, b"k_bits"),
        (dict(kv_kind=_lib.TQ_KV_PROD, k_dim=16), _lib.TQ_ERR_INVALID_ARGUMENT, b"Prod"),
        (dict(kv_kind=_lib.TQ_KV_PROD), _lib.TQ_ERR_INVALID_ARGUMENT, b"projection"),
        (dict(Hkv=7), _lib.TQ_ERR_INVALID_ARGUMENT, b"heads"),
        (dict(kv_kind=_lib.TQ_KV_PLAIN, kv_dtype=0), _lib.TQ_ERR_INVALID_ARGUMENT, b"plain"),
    ]
    for kw, code, text in bad:
        args = dict(ok)
        args.update(kw)
        assert lib.tq_attention_general(*_general_args(**args)) == code, kw
        assert text in lib.tq_last_error(), (kw, lib.tq_last_error())
    # the workspace queries cover the general kernels, where the tuned entry
    # points route shapes outside their kernels (Prod keys need the projected
    # queries too)
    assert lib.tq_attention_general_workspace_size(1, 32, 8, 1, 128, 64, 4096) > 0
    assert lib.tq_attention_prod_workspace_size(1, 32, 8, 1, 512, 4096) >= \
        lib.tq_attention_general_workspace_size(1, 32, 8, 1, 512, 512, 4096)
    assert lib.tq_attention_prod_workspace_size(1, 32, 8, 1, 512, 4096) > \
        lib.tq_attention_workspace_size(1, 32, 8, 1, 512, 4096)


def test_check_maps_status_to_exceptions():
    lib = _lib.load()
    lib.tq_packed_width(1, 1)
    with pytest.raises(ValueError):
        _lib.check(_lib.TQ_ERR_INVALID_ARGUMENT, "x")
    with pytest.raises(NotImplementedError):
        _lib.check(_lib.TQ_ERR_UNSUPPORTED, "x")
    with pytest.raises(_lib.TurboQuantLibraryError):
        _lib.check(_lib.TQ_ERR_HIP, "x")


def test_key_value_append_checks_both_sides_without_the_gpu():
    lib = _lib.load()
    base = [None, None, 1, 1, 2, 1, 128, 256, 128, 128, 256, 128, 128, 3, 3, 0,
            None, None, None, None, None, None, None, None, 0, 16, 0, None]
    for side in (13, 14):                          # k_bits, then v_bits (L = 0: no pointer use)
        args = list(base)
        args[5] = 0
        args[side] = 5
        assert lib.tq_append_quantize_kv(*args) == _lib.TQ_ERR_INVALID_ARGUMENT
        assert b"bits" in lib.tq_last_error()
    args = list(base)
    args[25] = 0                                   # capacity 0 < offset + L
    assert lib.tq_append_quantize_kv(*args) == _lib.TQ_ERR_INVALID_ARGUMENT
    assert b"capacity" in lib.tq_last_error()
    args = list(base)
    assert lib.tq_append_quantize_kv(*args) == _lib.TQ_ERR_INVALID_ARGUMENT  # null pointers
    assert b"null" in lib.tq_last_error()
    args = list(base)
    args[5] = 0                                    # L = 0: nothing to do
    assert lib.tq_append_quantize_kv(*args) == _lib.TQ_OK
