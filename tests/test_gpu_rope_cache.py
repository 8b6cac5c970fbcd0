"""GPU parity of bias + RoPE + KV-cache append (bit-exact against the oracle),
and of the per-token decode sequence feeder -> attention (config 4 shape).

The whole qkv buffer and both caches are compared bit for bit, with caches
filled with a sentinel so any write outside row `pos` shows up
(fused_qkv_rope_cache.cuh:49-54 writes exactly one row per layer).
"""
import numpy as np
import pytest
import torch

from common import normal_f16, AttnCase
from oracle import oracle

pytestmark = pytest.mark.gpu

H, D = 16, 128
HID = H * D
SENTINEL = np.float16(-3.25)


@pytest.fixture(scope="module")
def qdiy():
    import qdiy as m
    torch.cuda.set_device(0)
    m.load()
    return m


def _strides(layout, max_seqlen):
    return (HID, D) if layout == "engine" else (D, max_seqlen * D)


def _run_both(qdiy, ctx, qkv, bias, pos, max_seqlen, layout):
    rs, hs = _strides(layout, max_seqlen)
    o_qkv = qkv.copy()
    o_k = np.full(max_seqlen * HID, SENTINEL, np.float16)
    o_v = o_k.copy()
    oracle.qkv_bias_rope_cache(o_qkv, bias, o_k, o_v, pos, H, D, rs, hs)
    g_qkv = torch.from_numpy(qkv).cuda()
    g_b = None if bias is None else torch.from_numpy(bias).cuda()
    g_k = torch.full((max_seqlen * HID,), float(SENTINEL), dtype=torch.float16, device="cuda")
    g_v = g_k.clone()
    ctx.qkv_bias_rope_cache(g_qkv, g_b, g_k, g_v, pos)
    torch.cuda.synchronize()
    return (o_qkv, o_k, o_v), (g_qkv.cpu().numpy(), g_k.cpu().numpy(), g_v.cpu().numpy())


def _same(a, b):
    return np.array_equal(a.view(np.uint16), b.view(np.uint16))


@pytest.mark.parametrize("layout", ["engine", "head_major"])
@pytest.mark.parametrize("with_bias", [False, True])
@pytest.mark.parametrize("pos", [0, 1, 3, 5, 1000, 2047])
def test_bit_exact_vs_oracle(qdiy, layout, with_bias, pos):
    S = 2048
    rs, hs = _strides(layout, S)
    rng = np.random.default_rng(pos * 4 + with_bias)
    qkv = normal_f16(rng, 3 * HID)
    bias = normal_f16(rng, 3 * HID, 0.02) if with_bias else None
    with qdiy.Context(num_heads=H, max_seqlen=S, kv_row_stride=rs, kv_head_stride=hs) as ctx:
        want, got = _run_both(qdiy, ctx, qkv, bias, pos, S, layout)
    for name, w, g in zip(("qkv", "k_cache", "v_cache"), want, got):
        assert _same(w, g), name


def test_odd_element_offsets_bit_exact(qdiy):
    """qkv and bias need only 2-byte alignment: views one element into larger
    buffers give the same bits as aligned ones."""
    S, pos = 64, 17
    rng = np.random.default_rng(77)
    qkv = normal_f16(rng, 3 * HID)
    bias = normal_f16(rng, 3 * HID, 0.02)
    o_qkv = qkv.copy()
    o_k = np.full(S * HID, SENTINEL, np.float16)
    o_v = o_k.copy()
    oracle.qkv_bias_rope_cache(o_qkv, bias, o_k, o_v, pos, H)
    qbuf = torch.zeros(3 * HID + 1, dtype=torch.float16, device="cuda")
    bbuf = torch.zeros(3 * HID + 1, dtype=torch.float16, device="cuda")
    qbuf[1:] = torch.from_numpy(qkv).cuda()
    bbuf[1:] = torch.from_numpy(bias).cuda()
    g_k = torch.full((S * HID,), float(SENTINEL), dtype=torch.float16, device="cuda")
    g_v = g_k.clone()
    with qdiy.Context(num_heads=H, max_seqlen=S) as ctx:
        ctx.qkv_bias_rope_cache(qbuf[1:], bbuf[1:], g_k, g_v, pos)
        torch.cuda.synchronize()
    assert _same(o_qkv, qbuf[1:].cpu().numpy())
    assert _same(o_k, g_k.cpu().numpy()) and _same(o_v, g_v.cpu().numpy())


def test_long_context_positions_bit_exact(qdiy):
    S = 32768
    rng = np.random.default_rng(99)
    with qdiy.Context(num_heads=H, max_seqlen=S) as ctx:
        for pos in (4095, 8191, 16384, 32767):
            qkv = normal_f16(rng, 3 * HID)
            bias = normal_f16(rng, 3 * HID, 0.02)
            want, got = _run_both(qdiy, ctx, qkv, bias, pos, S, "engine")
            for w, g in zip(want, got):
                assert _same(w, g), pos


def test_pos_out_of_range_rejected(qdiy):
    with qdiy.Context(num_heads=H, max_seqlen=8) as ctx:
        qkv = torch.zeros(3 * HID, dtype=torch.float16, device="cuda")
        kc = torch.zeros(8 * HID, dtype=torch.float16, device="cuda")
        for pos in (-1, 8):
            with pytest.raises(qdiy.QdError) as e:
                ctx.qkv_bias_rope_cache(qkv, None, kc, kc, pos)
            assert e.value.code == qdiy.QD_EINVAL
        with pytest.raises(qdiy.QdError):
            ctx.qkv_bias_rope_cache(qkv, None, kc, kc, 3, max_seqlen=9)   # beyond the ctx table


def test_decode_sequence_matches_oracle(qdiy):
    """Per-token loop of QwenEngine::step's attention section
    (qwen_infer.cu:631-678): feeder at pos, attention over pos+1 rows."""
    S, steps = 96, 80
    rng = np.random.default_rng(7)
    bias = normal_f16(rng, 3 * HID, 0.02)
    o_k = np.zeros(S * HID, np.float16)
    o_v = np.zeros(S * HID, np.float16)
    g_k = torch.zeros(S * HID, dtype=torch.float16, device="cuda")
    g_v = torch.zeros_like(g_k)
    g_b = torch.from_numpy(bias).cuda()
    out = torch.empty(HID, dtype=torch.float16, device="cuda")
    worst = 0.0
    with qdiy.Context(num_heads=H, max_seqlen=S) as ctx:
        for pos in range(steps):
            qkv = normal_f16(rng, 3 * HID)
            o_qkv = qkv.copy()
            oracle.qkv_bias_rope_cache(o_qkv, bias, o_k, o_v, pos, H)
            want = oracle.decode_attention(o_qkv[:HID].reshape(H, D), o_k, o_v, pos + 1, H, HID, D)
            g_qkv = torch.from_numpy(qkv).cuda()
            ctx.qkv_bias_rope_cache(g_qkv, g_b, g_k, g_v, pos)
            ctx.decode_attention(g_qkv, g_k, g_v, out, pos + 1)
            torch.cuda.synchronize()
            assert _same(g_qkv.cpu().numpy(), o_qkv), pos
            got = out.cpu().numpy().reshape(H, D).astype(np.float32)
            worst = max(worst, float(np.max(np.abs(got - want.astype(np.float32)))))
        assert _same(g_k.cpu().numpy(), o_k) and _same(g_v.cpu().numpy(), o_v)
    assert worst <= 2e-3, worst


def test_config4_front_end_after_gemv(qdiy):
    """Config 4 minus the QKV GEMV: bias + RoPE at pos 2047, append at slot
    2047, attention over 2048 rows whose slots 0..2046 are pre-filled."""
    S, pos = 2048, 2047
    case = AttnCase(pos, H=H, seed=44, max_seqlen=S)
    rng = np.random.default_rng(45)
    qkv = normal_f16(rng, 3 * HID)
    bias = normal_f16(rng, 3 * HID, 0.02)
    o_qkv, o_k, o_v = qkv.copy(), case.kc.copy(), case.vc.copy()
    oracle.qkv_bias_rope_cache(o_qkv, bias, o_k, o_v, pos, H)
    want = oracle.decode_attention(o_qkv[:HID].reshape(H, D), o_k, o_v, pos + 1, H, HID, D, nthreads=8)
    with qdiy.Context(num_heads=H, max_seqlen=S) as ctx:
        g_qkv = torch.from_numpy(qkv).cuda()
        g_k = torch.from_numpy(case.kc).cuda()
        g_v = torch.from_numpy(case.vc).cuda()
        out = torch.empty(HID, dtype=torch.float16, device="cuda")
        ctx.qkv_bias_rope_cache(g_qkv, torch.from_numpy(bias).cuda(), g_k, g_v, pos)
        ctx.decode_attention(g_qkv, g_k, g_v, out, pos + 1)
        torch.cuda.synchronize()
        assert _same(g_k.cpu().numpy(), o_k) and _same(g_v.cpu().numpy(), o_v)
        got = out.cpu().numpy().reshape(H, D).astype(np.float32)
    assert float(np.max(np.abs(got - want.astype(np.float32)))) <= 2e-3
