"""The C-ABI library loads and exports every entry point include/qdiy/*.h
declares; argument validation answers with status codes before any GPU work
(these calls make no device allocation and launch nothing)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", "qdiy", h) for h in ("attn.h", "decode.h", "engine.h")]


def _declared():
    text = "".join(open(h).read() for h in HEADERS)
    return sorted(set(re.findall(r"^(?:int|const char\*|size_t|long long)\s+(qd_\w+)\s*\(", text, re.M)))


@pytest.fixture(scope="module")
def qdiy():
    import qdiy as m
    if not os.path.exists(m.LIB_PATH):
        import __graft_entry__
        __graft_entry__.build()
    return m


def test_header_declares_the_boundary():
    names = _declared()
    for want in ("qd_ctx_create", "qd_ctx_destroy", "qd_qkv_bias_rope_cache", "qd_decode_attention",
                 "qd_decode_attention_fused", "qd_decode_attention_split"):
        assert want in names


def test_library_exports_every_declared_symbol(qdiy):
    lib = qdiy.load()
    for name in _declared():
        assert hasattr(lib, name), name
    assert set(_declared()) == set(qdiy.EXPORTS)


def test_version_and_limits(qdiy):
    assert re.match(r"^\d+\.\d+\.\d+$", qdiy.version())
    assert qdiy.max_splits() >= 64


def test_ctx_create_rejects_bad_cfg_without_touching_the_gpu(qdiy):
    lib = qdiy.load()
    h = ctypes.c_void_p()
    for cfg in (qdiy.Cfg(16, 64, 128, 2048, 128, 10000.0),      # head_dim must be 128
                qdiy.Cfg(0, 128, 128, 2048, 128, 10000.0),      # no heads
                qdiy.Cfg(16, 128, 0, 2048, 128, 10000.0),       # no rows
                qdiy.Cfg(16, 128, 128, 2047, 128, 10000.0),     # stride not a multiple of 8
                qdiy.Cfg(16, 128, 128, 2048, 128, 0.0),         # rope base
                qdiy.Cfg(16, 128, 1 << 20, 2048, 128, 1e4)):    # row span beyond 32-bit offsets
        assert lib.qd_ctx_create(ctypes.byref(cfg), ctypes.byref(h)) == qdiy.QD_EINVAL
        assert h.value is None
        assert lib.qd_last_error()
    assert lib.qd_ctx_create(None, ctypes.byref(h)) == qdiy.QD_EINVAL
    assert lib.qd_ctx_create(ctypes.byref(qdiy.Cfg(16, 128, 8, 2048, 128, 1e4)), None) == qdiy.QD_EINVAL


def test_calls_reject_null_context(qdiy):
    lib = qdiy.load()
    buf = ctypes.create_string_buffer(64)
    p = ctypes.c_void_p(ctypes.addressof(buf))
    assert lib.qd_decode_attention(None, p, p, p, p, 1, 16, 128, None) == qdiy.QD_EINVAL
    assert lib.qd_decode_attention_fused(None, p, p, p, p, 1, 16, 128, None) == qdiy.QD_EINVAL
    assert lib.qd_decode_attention_split(None, p, p, p, p, 1, 16, 128, 4, None) == qdiy.QD_EINVAL
    assert lib.qd_qkv_bias_rope_cache(None, p, None, p, p, 0, 8, 16, 128, None) == qdiy.QD_EINVAL
    assert b"ctx" in lib.qd_last_error()
    v, s = ctypes.c_int(), ctypes.c_int()
    assert lib.qd_decode_attention_plan(None, 1, ctypes.byref(v), ctypes.byref(s)) == qdiy.QD_EINVAL
    assert lib.qd_ctx_destroy(None) == qdiy.QD_OK
