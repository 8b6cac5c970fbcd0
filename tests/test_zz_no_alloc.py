"""qd_decode_attention_noalloc: the allocation-free decode attention.

It runs the kernels and launch plan of qd_decode_attention with the split
partials in the library's static per-GPU scratch instead of a context's, so
its outputs must equal qd_decode_attention's bit for bit.  The GPU test makes
calls in a row on one GPU, each later call smaller than the one before, so
every call after the first finds the previous call's partials in the shared
scratch.  Argument validation is checked on the CPU: it answers before any
HIP call.
"""
import ctypes

import numpy as np
import pytest
import torch

from common import AttnCase
from oracle import oracle

ATOL = 2e-3


@pytest.fixture(scope="module")
def qdiy():
    import os

    import qdiy as m
    if not os.path.exists(m.LIB_PATH):
        import __graft_entry__
        __graft_entry__.build()
    m.load()
    return m


def _host_buf(nbytes):
    buf = ctypes.create_string_buffer(nbytes + 256)
    return buf, (ctypes.addressof(buf) + 255) & ~255


def test_noalloc_rejects_bad_arguments_without_a_gpu(qdiy):
    lib = qdiy.load()
    P = ctypes.c_void_p
    _keep, b = _host_buf(1 << 20)
    q, k, v, out = b, b + (64 << 10), b + (256 << 10), b + (512 << 10)
    good = dict(seqlen=4, heads=16, hd=128, rs=2048, hs=128)

    def call(q=q, k=k, v=v, out=out, **kw):
        a = dict(good, **kw)
        return lib.qd_decode_attention_noalloc(P(q), P(k), P(v), P(out), a["seqlen"], a["heads"],
                                               a["hd"], a["rs"], a["hs"], None)

    for rc in (call(q=None), call(out=None), call(k=q + 2), call(out=out + 8),
               call(hd=64), call(heads=0), call(heads=5000), call(rs=2047), call(hs=0),
               call(seqlen=0), call(seqlen=1 << 20, rs=4096)):
        assert rc == qdiy.QD_EINVAL
        assert lib.qd_last_error()
    # out inside the K rows being read
    assert call(out=k + 256) == qdiy.QD_EINVAL
    assert b"overlaps" in lib.qd_last_error()


def _run_pair(qdiy, ctx, case, L):
    """The same call through the context entry point and the allocation-free one."""
    H = case.H
    q = torch.from_numpy(case.q.reshape(-1)).cuda()
    kc = torch.from_numpy(case.kc).cuda()
    vc = torch.from_numpy(case.vc).cuda()
    tail = 64
    want = torch.full((H * 128 + tail,), 7.0, dtype=torch.float16, device="cuda")
    got = torch.full((H * 128 + tail,), 7.0, dtype=torch.float16, device="cuda")
    ctx.decode_attention(q, kc, vc, want, L)
    qdiy.decode_attention_noalloc(q, kc, vc, got, L, H, case.row_stride, case.head_stride)
    torch.cuda.synchronize()
    w, g = want.cpu().numpy(), got.cpu().numpy()
    assert np.all(g[H * 128:] == np.float16(7.0)), "write past the end of out"
    return w[:H * 128].reshape(H, 128), g[:H * 128].reshape(H, 128)


@pytest.mark.gpu
def test_noalloc_equals_context_entry_point_on_calls_in_a_row(qdiy):
    torch.cuda.set_device(0)
    # (L, heads, layout, seed): each call smaller than the one before it.  On a
    # 256-CU MI355X: 8192 rows plan 16 splits per head (256 partial slots); 8 heads
    # at 2000 rows 32 splits (256 slots); 16 heads at 300 rows 15 splits (240
    # slots); 129-224 rows are where a default context (round-robin dispatch, 16
    # heads a multiple of its period, so the merge runs in the scan kernel) runs
    # split plans although a context that never merges in the kernel would run
    # them fused; 100 rows is fused either way and uses no scratch.
    calls = [(8192, 16, "engine", 1), (2000, 8, "head_major", 2), (300, 16, "engine", 3),
             (224, 16, "engine", 5), (200, 16, "engine", 6), (160, 16, "head_major", 7),
             (129, 16, "engine", 8), (100, 16, "engine", 4)]
    for L, H, layout, seed in calls:
        case = AttnCase(L, H=H, seed=seed, kscale=0.5, layout=layout)
        with qdiy.Context(num_heads=H, max_seqlen=case.max_seqlen, kv_row_stride=case.row_stride,
                          kv_head_stride=case.head_stride) as ctx:
            want, got = _run_pair(qdiy, ctx, case, L)
            plan = ctx.plan_detail(L)
        print(f"noalloc L={L} H={H} {layout}: plan {plan.as_tuple()}", flush=True)
        same = want.view(np.uint16) == got.view(np.uint16)
        assert same.all(), (f"L={L} H={H}: {np.count_nonzero(~same)} outputs differ from "
                            f"qd_decode_attention under {plan.as_tuple()}")
        if L <= 2000:
            ref = oracle.decode_attention(case.q, case.kc, case.vc, L, H, case.row_stride, 128,
                                          oracle.ENGINE, 8) if layout == "engine" else None
            if ref is not None:
                err = float(np.max(np.abs(got.astype(np.float32) - ref.astype(np.float32))))
                assert err <= ATOL, f"L={L}: max abs err {err} vs the reference-order oracle"


@pytest.mark.gpu
def test_noalloc_fills_the_top_of_its_static_scratch(qdiy):
    """Head counts above the CU count plan one split per head: 1000 heads at 300 rows
    use 1000 of the 1024 static partial slots, then 520 heads at 260 rows 520 of them
    (the second call finds the first's partials in the shared scratch).  Bit for bit
    against qd_decode_attention with a context."""
    torch.cuda.set_device(0)
    for L, H, seed in ((300, 1000, 11), (260, 520, 12)):
        case = AttnCase(L, H=H, seed=seed, kscale=0.5)
        with qdiy.Context(num_heads=H, max_seqlen=L) as ctx:
            want, got = _run_pair(qdiy, ctx, case, L)
            plan = ctx.plan_detail(L)
        print(f"noalloc L={L} H={H}: plan {plan.as_tuple()}", flush=True)
        assert plan.variant == qdiy.SPLIT and plan.num_splits == 1
        same = want.view(np.uint16) == got.view(np.uint16)
        assert same.all(), f"L={L} H={H}: {np.count_nonzero(~same)} outputs differ"


@pytest.mark.gpu
def test_noalloc_rejects_plans_beyond_its_static_scratch(qdiy):
    """2048 heads plan one split each: 2048 partial slots, over the 1024 the static
    scratch holds.  The call is refused before any launch; the buffers are still
    sized for the call so that a launch could not read out of bounds."""
    torch.cuda.set_device(0)
    H, L = 2048, 240
    row = H * 128
    q = torch.zeros(row, dtype=torch.float16, device="cuda")
    out = torch.zeros(row, dtype=torch.float16, device="cuda")
    kc = torch.zeros(L * row, dtype=torch.float16, device="cuda")
    vc = torch.zeros(L * row, dtype=torch.float16, device="cuda")
    with pytest.raises(qdiy.QdError, match="static scratch"):
        qdiy.decode_attention_noalloc(q, kc, vc, out, L, H)
    torch.cuda.synchronize()
