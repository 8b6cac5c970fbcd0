"""qd_qkv_proj_rope_cache_attention: the attention front end and decode
attention of one layer (qwen_infer.cu:626-678) in one call.

Where the attention plan merges in the scan kernel (up to 3072 rows, one
workgroup per CU, 8 or 16 heads), the call is one launch in which each workgroup computes its
share of the QKV GEMV, bias, RoPE and append and then its split of the
attention, reading its head's rotated Q (and the appended row's K and V)
from tagged words written by the producers on its XCD.  Every output must
equal, bit for bit, the two separate calls (qd_qkv_proj_rope_cache then
qd_decode_attention) on the same inputs: the qkv buffer, both whole caches
(sentinel-filled rows included) and out; and the kernel-order oracle.  Also
with the test hook that makes every split compute its head's front end
itself, on calls in a row (per-call tags), and at lengths where the call
falls back to two launches.  Every split of the one-launch form must have
read its producers' words (qd_ctx_front_misses 0): a split that recomputes
the front end gives the same bits, so only the counter shows it.
"""
import numpy as np
import pytest
import torch

from common import normal_f16
from oracle import oracle

pytestmark = pytest.mark.gpu
D = 128


@pytest.fixture(scope="module")
def qdiy():
    import qdiy as m
    torch.cuda.set_device(0)
    m.load()
    return m


def _same(a, b):
    return np.array_equal(np.asarray(a).view(np.uint16), np.asarray(b).view(np.uint16))


class Layer:
    """One layer's inputs: x, ln_1, W_qkv [3 hid][hid], bias, and caches of S rows
    whose rows below pos hold N(0,1) K/V and the rest a sentinel."""

    def __init__(self, H, S, pos, seed, norm=True, bias=True):
        hid = H * D
        rng = np.random.default_rng(seed)
        self.H, self.S, self.pos, self.hid = H, S, pos, hid
        self.x = normal_f16(rng, hid)
        self.nw = (1.0 + 0.1 * rng.standard_normal(hid)).astype(np.float16) if norm else None
        self.W = normal_f16(rng, 3 * hid * hid, 0.02)
        self.b = normal_f16(rng, 3 * hid, 0.02) if bias else None
        self.kc = np.full(S * hid, np.float16(7.5))
        self.vc = np.full(S * hid, np.float16(-3.25))
        self.kc[:pos * hid] = normal_f16(rng, pos * hid, 0.5)
        self.vc[:pos * hid] = normal_f16(rng, pos * hid)

    def dev(self):
        c = lambda a: None if a is None else torch.from_numpy(a.copy()).cuda()
        return dict(x=c(self.x), nw=c(self.nw), W=c(self.W), b=c(self.b), k=c(self.kc), v=c(self.vc),
                    qkv=torch.full((3 * self.hid,), 5.0, dtype=torch.float16, device="cuda"),
                    out=torch.full((self.hid + 64,), 9.0, dtype=torch.float16, device="cuda"))


def _run(ctx, L, fused):
    t = L.dev()
    if fused:
        ctx.qkv_proj_rope_cache_attention(t["x"], t["nw"], t["W"], t["b"], t["qkv"], t["k"], t["v"],
                                          t["out"], L.pos)
    else:
        ctx.qkv_proj_rope_cache(t["x"], t["nw"], t["W"], t["b"], t["qkv"], t["k"], t["v"], L.pos)
        ctx.decode_attention(t["qkv"], t["k"], t["v"], t["out"], L.pos + 1)
    torch.cuda.synchronize()
    return {k: t[k].cpu().numpy() for k in ("qkv", "k", "v", "out")}


def _check_equal(a, b, what):
    for key in ("qkv", "k", "v", "out"):
        diff = a[key].view(np.uint16) != b[key].view(np.uint16)
        assert not diff.any(), f"{what}: {key} differs in {np.count_nonzero(diff)} elements"


@pytest.mark.parametrize("H,seqlen,norm,bias", [
    (16, 129, True, True), (16, 200, True, True), (16, 256, False, True), (16, 300, True, False),
    (16, 512, True, True), (8, 300, True, True),
    (16, 513, True, True), (16, 1000, True, True), (16, 2048, False, True), (16, 3072, True, True),
    # 8 heads at 2000 rows: 32 splits, so workgroups 128-255 have no producer role
    (8, 2000, True, True),
    # two launches: a fused attention plan, a two-launch split plan
    (16, 100, True, True), (16, 3073, True, True)])
def test_one_call_equals_the_two_calls(qdiy, H, seqlen, norm, bias):
    pos = seqlen - 1
    L = Layer(H, seqlen + 3, pos, seed=seqlen * 7 + H, norm=norm, bias=bias)
    with qdiy.Context(num_heads=H, max_seqlen=L.S) as ctx:
        plan = ctx.plan_detail(seqlen)
        print(f"H={H} L={seqlen}: plan {plan.as_tuple()} merge in kernel {plan.merge_in_kernel}", flush=True)
        two = _run(ctx, L, False)
        one = _run(ctx, L, True)
        # every split saw its producers' words (a miss is correct but slow)
        assert ctx.front_misses() == 0, "splits computed their head's front end themselves"
        ctx.set_front_local(True)
        local = _run(ctx, L, True)
        ctx.set_front_local(False)
        assert ctx.front_misses() == 0, "forced splits are not counted as misses"
    _check_equal(one, two, "one call against the two calls")
    _check_equal(local, two, "one call, every split computing its front end")
    assert np.all(one["out"][L.hid:] == np.float16(9.0)), "write past the end of out"
    # against the oracle: the front end, then the kernel-order attention of the plan
    o_qkv, o_k, o_v = np.zeros(3 * L.hid, np.float16), L.kc.copy(), L.vc.copy()
    oracle.qkv_front(L.x, L.nw, L.W, L.b, o_qkv, o_k, o_v, pos, H)
    assert _same(one["qkv"], o_qkv) and _same(one["k"], o_k) and _same(one["v"], o_v)
    want = oracle.attention_planned(o_qkv[:L.hid].reshape(H, D), o_k, o_v, seqlen, H, L.hid, D,
                                    oracle.Plan(*plan.as_tuple()), nthreads=8)
    assert _same(one["out"][:L.hid], want.reshape(-1))


def test_calls_in_a_row(qdiy):
    """A decode sequence through one context: each call appends a row and attends
    over it, the next call reads it back from the cache; tags change per call."""
    H, S = 16, 400
    L = Layer(H, S, 250, seed=77)
    with qdiy.Context(num_heads=H, max_seqlen=S) as ctx:
        t1, t2 = L.dev(), L.dev()
        xs = [normal_f16(np.random.default_rng(100 + i), L.hid) for i in range(12)]
        for i, x in enumerate(xs):
            pos = 250 + i
            xd = torch.from_numpy(x).cuda()
            ctx.qkv_proj_rope_cache_attention(xd, t1["nw"], t1["W"], t1["b"], t1["qkv"], t1["k"], t1["v"],
                                              t1["out"], pos)
            ctx.qkv_proj_rope_cache(xd, t2["nw"], t2["W"], t2["b"], t2["qkv"], t2["k"], t2["v"], pos)
            ctx.decode_attention(t2["qkv"], t2["k"], t2["v"], t2["out"], pos + 1)
            torch.cuda.synchronize()
            for key in ("qkv", "out"):
                assert _same(t1[key].cpu().numpy(), t2[key].cpu().numpy()), (i, key)
        assert _same(t1["k"].cpu().numpy(), t2["k"].cpu().numpy())
        assert _same(t1["v"].cpu().numpy(), t2["v"].cpu().numpy())
        assert ctx.front_misses() == 0


def test_rejects_out_over_its_inputs(qdiy):
    H, S = 16, 300
    L = Layer(H, S, 200, seed=5)
    with qdiy.Context(num_heads=H, max_seqlen=S) as ctx:
        t = L.dev()
        with pytest.raises(qdiy.QdError, match="overlap"):
            ctx.qkv_proj_rope_cache_attention(t["x"], t["nw"], t["W"], t["b"], t["qkv"], t["k"], t["v"],
                                              t["x"], L.pos)
        with pytest.raises(qdiy.QdError, match="overlap"):
            ctx.qkv_proj_rope_cache_attention(t["x"], t["nw"], t["W"], t["b"], t["qkv"], t["k"], t["v"],
                                              t["k"][: L.hid], L.pos)
        # out aliasing q is allowed (the two-launch form runs)
        ctx.qkv_proj_rope_cache_attention(t["x"], t["nw"], t["W"], t["b"], t["qkv"], t["k"], t["v"],
                                          t["qkv"][: L.hid], L.pos)
        torch.cuda.synchronize()
