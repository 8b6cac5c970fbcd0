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
    # (L, heads, layout, seed): each call smaller than the one before it
    # (8192 -> 2000 -> 300 -> 100 rows); 8 heads at 2000 rows plan two split
    # workgroups per CU (512 partial slots), 16 heads at 300 rows 15 splits
    # (240 slots), 100 rows the fused plan, which uses no scratch.
    calls = [(8192, 16, "engine", 1), (2000, 8, "head_major", 2), (300, 16, "engine", 3),
             (100, 16, "engine", 4)]
    for L, H, layout, seed in calls:
        case = AttnCase(L, H=H, seed=seed, kscale=0.5, layout=layout)
        with qdiy.Context(num_heads=H, max_seqlen=case.max_seqlen, kv_row_stride=case.row_stride,
                          kv_head_stride=case.head_stride) as ctx:
            want, got = _run_pair(qdiy, ctx, case, L)
            plan = ctx.plan_detail(L)
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
