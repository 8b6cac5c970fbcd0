"""GPU parity of the fused attention front end (qd_qkv_proj_rope_cache):
[RMSNorm] -> QKV GEMV -> bias -> RoPE -> KV append, and config 4 end to end.

Bars: bit-exact against the oracle evaluated in the kernels' fixed reduction
order (QD_ORDER_WAVE64); within one fp16 ulp of the GEMV outputs in the
reference's sequential order (hgemm_final.cuh:278-293); attention <= 2e-3.
"""
import numpy as np
import pytest
import torch

from common import normal_f16, ulp16
from oracle import oracle

pytestmark = pytest.mark.gpu

H, D = 16, 128
HID = H * D
SENT = np.float16(-2.5)


@pytest.fixture(scope="module")
def qdiy():
    import qdiy as m
    torch.cuda.set_device(0)
    m.load()
    return m


@pytest.fixture(scope="module")
def weights():
    rng = np.random.default_rng(404)
    return {"W": normal_f16(rng, (3 * HID, HID), 0.02), "b": normal_f16(rng, 3 * HID, 0.02),
            "nw": (1.0 + normal_f16(rng, HID, 0.1).astype(np.float32)).astype(np.float16)}


def _same(a, b):
    return np.array_equal(np.asarray(a).view(np.uint16), np.asarray(b).view(np.uint16))


def _run(qdiy, ctx, x, nw, W, b, pos, S, layout="engine", gW=None):
    rs, hs = (HID, D) if layout == "engine" else (D, S * D)
    o_qkv = np.zeros(3 * HID, np.float16)
    o_k = np.full(S * HID, SENT, np.float16)
    o_v = o_k.copy()
    oracle.qkv_front(x, nw, W, b, o_qkv, o_k, o_v, pos, H, row_stride=rs, head_stride=hs)
    g_qkv = torch.zeros(3 * HID, dtype=torch.float16, device="cuda")
    g_k = torch.full((S * HID,), float(SENT), dtype=torch.float16, device="cuda")
    g_v = g_k.clone()
    gW = torch.from_numpy(W).cuda() if gW is None else gW
    ctx.qkv_proj_rope_cache(torch.from_numpy(x).cuda(), None if nw is None else torch.from_numpy(nw).cuda(),
                            gW, None if b is None else torch.from_numpy(b).cuda(), g_qkv, g_k, g_v, pos)
    torch.cuda.synchronize()
    return (o_qkv, o_k, o_v), (g_qkv.cpu().numpy(), g_k.cpu().numpy(), g_v.cpu().numpy())


@pytest.mark.parametrize("with_norm", [False, True])
@pytest.mark.parametrize("with_bias", [False, True])
@pytest.mark.parametrize("pos", [0, 5, 2047])
def test_bit_exact_vs_oracle(qdiy, weights, with_norm, with_bias, pos):
    rng = np.random.default_rng(pos * 7 + with_norm * 2 + with_bias)
    x = normal_f16(rng, HID)
    with qdiy.Context(num_heads=H, max_seqlen=2048) as ctx:
        want, got = _run(qdiy, ctx, x, weights["nw"] if with_norm else None, weights["W"],
                         weights["b"] if with_bias else None, pos, 2048)
    for name, w, g in zip(("qkv", "k_cache", "v_cache"), want, got):
        assert _same(w, g), name


@pytest.mark.parametrize("heads", [4, 8, 20, 32])
def test_bit_exact_other_widths(qdiy, heads):
    """hidden 512 / 1024 keep all six rows of a pair in flight at once; 2560
    and 4096 load them in two phases of three rows."""
    hid = heads * D
    rng = np.random.default_rng(900 + heads)
    W, b = normal_f16(rng, (3 * hid, hid), 0.02), normal_f16(rng, 3 * hid, 0.02)
    nw = (1.0 + normal_f16(rng, hid, 0.1).astype(np.float32)).astype(np.float16)
    x = normal_f16(rng, hid)
    S, pos = 16, 11
    o_qkv = np.zeros(3 * hid, np.float16)
    o_k = np.full(S * hid, SENT, np.float16)
    o_v = o_k.copy()
    oracle.qkv_front(x, nw, W, b, o_qkv, o_k, o_v, pos, heads)
    g_qkv = torch.zeros(3 * hid, dtype=torch.float16, device="cuda")
    g_k = torch.full((S * hid,), float(SENT), dtype=torch.float16, device="cuda")
    g_v = g_k.clone()
    with qdiy.Context(num_heads=heads, max_seqlen=S) as ctx:
        ctx.qkv_proj_rope_cache(torch.from_numpy(x).cuda(), torch.from_numpy(nw).cuda(), torch.from_numpy(W).cuda(),
                                torch.from_numpy(b).cuda(), g_qkv, g_k, g_v, pos)
        torch.cuda.synchronize()
    for name, w, g in zip(("qkv", "k_cache", "v_cache"), (o_qkv, o_k, o_v), (g_qkv, g_k, g_v)):
        assert _same(w, g.cpu().numpy()), name


def test_bias_and_outputs_at_odd_offsets(qdiy, weights):
    """bias, qkv and the caches need only 2-byte alignment: views one element
    into larger buffers give the same bits as aligned ones."""
    S, pos = 32, 9
    rng = np.random.default_rng(4242)
    x = normal_f16(rng, HID)
    o_qkv = np.zeros(3 * HID, np.float16)
    o_k = np.full(S * HID, SENT, np.float16)
    o_v = o_k.copy()
    oracle.qkv_front(x, weights["nw"], weights["W"], weights["b"], o_qkv, o_k, o_v, pos, H)

    def odd(n, fill=0.0):
        return torch.full((n + 1,), float(fill), dtype=torch.float16, device="cuda")[1:]
    g_b = odd(3 * HID)
    g_b.copy_(torch.from_numpy(weights["b"]).cuda())
    g_qkv, g_k, g_v = odd(3 * HID), odd(S * HID, SENT), odd(S * HID, SENT)
    with qdiy.Context(num_heads=H, max_seqlen=S) as ctx:
        ctx.qkv_proj_rope_cache(torch.from_numpy(x).cuda(), torch.from_numpy(weights["nw"]).cuda(),
                                torch.from_numpy(weights["W"]).cuda(), g_b, g_qkv, g_k, g_v, pos)
        torch.cuda.synchronize()
    for name, w, g in zip(("qkv", "k_cache", "v_cache"), (o_qkv, o_k, o_v), (g_qkv, g_k, g_v)):
        assert _same(w, g.cpu().numpy()), name


def test_head_major_layout(qdiy, weights):
    rng = np.random.default_rng(3)
    x = normal_f16(rng, HID)
    with qdiy.Context(num_heads=H, max_seqlen=64, kv_row_stride=D, kv_head_stride=64 * D) as ctx:
        want, got = _run(qdiy, ctx, x, weights["nw"], weights["W"], weights["b"], 17, 64, "head_major")
    for w, g in zip(want, got):
        assert _same(w, g)


def test_close_to_reference_order(qdiy, weights):
    """Against the reference's sequential-k GEMV: the pre-rotation QKV values
    are the same fp32 sum in another order -- within one fp16 ulp plus the
    fp32 reordering bound K * 2^-24 * sum|x w| (which only matters for outputs
    near zero), and identical for almost all outputs."""
    rng = np.random.default_rng(8)
    x = normal_f16(rng, HID)
    ref = oracle.gemv(x, weights["W"], 3 * HID, HID, 0, oracle.ORDER_REF)
    with qdiy.Context(num_heads=H, max_seqlen=8) as ctx:
        _, (g_qkv, _, _) = _run(qdiy, ctx, x, None, weights["W"], None, 0, 8)   # pos 0: no rotation
    g, r = g_qkv.astype(np.float64), ref.astype(np.float64)
    d = np.abs(g - r)
    absum = np.abs(weights["W"].astype(np.float64)) @ np.abs(x.astype(np.float64))
    assert np.all(d <= np.maximum(ulp16(r), ulp16(g)) + HID * 2.0 ** -24 * absum)
    assert np.mean(d > 0) < 0.05


def test_config4_front_end(qdiy, weights):
    """Config 4: x ~N(0,1) [2048]; W [6144 x 2048] ~N(0,0.02); b ~N(0,0.02);
    GEMV + bias + RoPE at pos 2047, append at slot 2047, attention over 2048
    rows whose slots 0..2046 hold N(0,1) K/V."""
    S, pos = 2048, 2047
    rng = np.random.default_rng(4)
    x = normal_f16(rng, HID)
    kc = normal_f16(rng, S * HID)
    vc = normal_f16(rng, S * HID)
    kc[pos * HID:] = 0
    vc[pos * HID:] = 0
    o_qkv, o_k, o_v = np.zeros(3 * HID, np.float16), kc.copy(), vc.copy()
    oracle.qkv_front(x, None, weights["W"], weights["b"], o_qkv, o_k, o_v, pos, H)
    want = oracle.decode_attention(o_qkv[:HID].reshape(H, D), o_k, o_v, pos + 1, H, HID, D, nthreads=8)
    with qdiy.Context(num_heads=H, max_seqlen=S) as ctx:
        g_qkv = torch.zeros(3 * HID, dtype=torch.float16, device="cuda")
        g_k, g_v = torch.from_numpy(kc).cuda(), torch.from_numpy(vc).cuda()
        out = torch.empty(HID, dtype=torch.float16, device="cuda")
        ctx.qkv_proj_rope_cache(torch.from_numpy(x).cuda(), None, torch.from_numpy(weights["W"]).cuda(),
                                torch.from_numpy(weights["b"]).cuda(), g_qkv, g_k, g_v, pos)
        ctx.decode_attention(g_qkv, g_k, g_v, out, pos + 1)
        torch.cuda.synchronize()
        assert _same(g_qkv.cpu().numpy(), o_qkv)
        assert _same(g_k.cpu().numpy(), o_k) and _same(g_v.cpu().numpy(), o_v)
        got = out.cpu().numpy().reshape(H, D).astype(np.float32)
    assert float(np.max(np.abs(got - want.astype(np.float32)))) <= 2e-3


def test_invalid_arguments(qdiy, weights):
    with qdiy.Context(num_heads=H, max_seqlen=8) as ctx:
        x = torch.zeros(HID, dtype=torch.float16, device="cuda")
        W = torch.zeros(3 * HID * HID, dtype=torch.float16, device="cuda")
        qkv = torch.zeros(3 * HID, dtype=torch.float16, device="cuda")
        kc = torch.zeros(8 * HID, dtype=torch.float16, device="cuda")
        with pytest.raises(qdiy.QdError):
            ctx.qkv_proj_rope_cache(x, None, W, None, qkv, kc, kc, 8)          # pos == max_seqlen
        xbig = torch.zeros(HID + 8, dtype=torch.float16, device="cuda")
        with pytest.raises(qdiy.QdError):
            ctx.qkv_proj_rope_cache(xbig[1:HID + 1], None, W, None, qkv, kc, kc, 0)   # misaligned x
        big = torch.zeros(4 * HID, dtype=torch.float16, device="cuda")
        with pytest.raises(qdiy.QdError, match="overlap"):                    # x inside qkv
            ctx.qkv_proj_rope_cache(big[HID:2 * HID], None, W, None, big[:3 * HID], kc, kc, 0)
        with pytest.raises(qdiy.QdError, match="overlap"):                    # out inside the V rows
            ctx.decode_attention(qkv[:HID], kc, kc, kc[HID:2 * HID], 4)
        ctx.decode_attention(qkv[:HID], kc, kc, qkv[:HID], 4)                  # out == q is allowed
        torch.cuda.synchronize()
    with qdiy.Context(num_heads=3, max_seqlen=8) as ctx3:                      # hidden 384
        x = torch.zeros(384, dtype=torch.float16, device="cuda")
        W = torch.zeros(3 * 384 * 384, dtype=torch.float16, device="cuda")
        qkv = torch.zeros(3 * 384, dtype=torch.float16, device="cuda")
        kc = torch.zeros(8 * 384, dtype=torch.float16, device="cuda")
        with pytest.raises(qdiy.QdError):
            ctx3.qkv_proj_rope_cache(x, None, W, None, qkv, kc, kc, 0)
