"""The C-ABI library loads and exports every entry point include/qdiy/*.h
declares; argument validation answers with status codes before any GPU work
(these calls make no device allocation and launch nothing)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", "qdiy", h) for h in ("attn.h", "decode.h", "engine.h", "bench.h")]


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


def test_missing_library_fails_loudly(qdiy, monkeypatch):
    """Without libqdiy.so the package raises; there is no other code path."""
    monkeypatch.setattr(qdiy, "_lib", None)
    monkeypatch.setattr(qdiy, "LIB_PATH", os.path.join(ROOT, "no_such_dir", "libqdiy.so"))
    with pytest.raises(RuntimeError, match="is not built"):
        qdiy.load()
    with pytest.raises(RuntimeError, match="is not built"):
        qdiy.Context(num_heads=16, max_seqlen=8)


def test_product_sources_do_not_reach_the_oracle():
    """The package (Python binding and native sources) never imports, includes or
    links the oracle: it is test infrastructure only."""
    pkg = os.path.join(ROOT, "llm-inference-diy_amd")
    pat = re.compile(r"^\s*(?:from\s+oracle\b|import\s+oracle\b|#\s*include\s*[<\"][^>\"]*qd_oracle)"
                     r"|libqd_oracle|oracle/", re.M)
    hits = []
    for d, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".cpp", ".h")):
                path = os.path.join(d, f)
                if pat.search(open(path, errors="replace").read()):
                    hits.append(os.path.relpath(path, ROOT))
    assert hits == []


def test_engine_cli_rejects_bad_options_before_any_gpu_work(qdiy):
    """qdiy_engine exits with status 2 and a message on an unknown option or
    prefill mode, before it loads a model or touches a GPU."""
    import subprocess
    for args, env_mode, msg in ((["--bogus"], None, "unknown option"),
                                (["--prefill", "fast"], None, "exact or mfma"),
                                (["--prefill=tensor"], None, "exact or mfma"),
                                ([], "fp8", "exact or mfma")):
        env = dict(os.environ)
        env.pop("QDIY_PREFILL", None)
        if env_mode:
            env["QDIY_PREFILL"] = env_mode
        res = subprocess.run([qdiy.ENGINE_EXE, *args, "no_such_model.bin"], input="exit\n",
                             capture_output=True, text=True, timeout=120, env=env)
        assert res.returncode == 2, (args, res.stderr)
        assert msg in res.stderr


def test_bench_hooks_reject_bad_arguments(qdiy):
    """Test and measurement hooks (qdiy/bench.h) check their arguments before
    any GPU work."""
    lib = qdiy.load()
    assert lib.qd_ctx_set_scan_depth(None, 1) == qdiy.QD_EINVAL
    assert lib.qd_ctx_count_xmerges(None, 1) == qdiy.QD_EINVAL
    assert lib.qd_ctx_xmerge_stats(None, None, None, None) == qdiy.QD_EINVAL
    assert lib.qd_ctx_set_merge(None, 0) == qdiy.QD_EINVAL
    assert lib.qd_ctx_set_recompute_mask(None, 1) == qdiy.QD_EINVAL


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
    assert lib.qd_prefill_attention(None, p, 2048, p, p, p, 2048, 0, 4, 16, 128, qdiy.GEMM_MFMA,
                                    None) == qdiy.QD_EINVAL
    assert b"ctx" in lib.qd_last_error()
    v, s = ctypes.c_int(), ctypes.c_int()
    assert lib.qd_decode_attention_plan(None, 1, ctypes.byref(v), ctypes.byref(s)) == qdiy.QD_EINVAL
    assert lib.qd_ctx_destroy(None) == qdiy.QD_OK


def _host_buf(nbytes):
    """A host buffer and its first 256-byte-aligned address (argument checks
    run before any HIP call, so host addresses exercise them without a GPU)."""
    buf = ctypes.create_string_buffer(nbytes + 256)
    base = (ctypes.addressof(buf) + 255) & ~255
    return buf, base


def test_decode_ops_reject_overlapping_outputs_without_a_gpu(qdiy):
    lib = qdiy.load()
    P = ctypes.c_void_p
    _keep, b = _host_buf(1 << 20)
    n, k = 64, 512
    x, w, res = b, b + 4096, b + 4096 + n * k * 2
    # out inside x, inside w, and straddling residual (not equal to it)
    for out in (x + 16, w + 64, res + 2):
        assert lib.qd_proj_residual(P(x), P(w), P(res), P(out), n, k, None) == qdiy.QD_EINVAL
        assert b"overlaps" in lib.qd_last_error()
    H, I = 512, 32
    xs, nw, w1, w2 = b, b + 1024, b + 2048, b + 2048 + I * H * 2
    for act in (xs + 2, nw, w1 + 100, w2 + I * H * 2 - 2):
        assert lib.qd_ffn_up_swiglu(P(xs), P(nw), ctypes.c_float(1e-6), P(w1), P(w2), P(act), H, I,
                                    None) == qdiy.QD_EINVAL
        assert b"overlaps" in lib.qd_last_error()
    V = 64
    ws_n = lib.qd_lm_head_workspace_bytes(V)
    wl = b + 2048
    logits, ws, tok = b + 2048 + V * H * 2, b + 4096 + V * H * 2, b + 8192 + V * H * 2
    bad = [(xs, ws, tok), (logits, logits + 8, tok), (logits, ws, ws), (logits, ws, wl + 64)]
    for lg, wk, tk in bad:
        assert lib.qd_lm_head_argmax(P(xs), P(nw), ctypes.c_float(1e-6), P(wl), P(lg), V, H, P(wk),
                                     ctypes.c_size_t(ws_n), P(tk), None) == qdiy.QD_EINVAL
        assert b"overlap" in lib.qd_last_error()
