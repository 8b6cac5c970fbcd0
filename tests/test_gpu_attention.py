"""GPU parity of decode attention (C ABI -> HIP kernels) against the CPU oracle.

Bars, on every call:
  * bit-exact against the oracle's restatement of this build's kernels
    (oracle.attention_planned) under the plan the library reports for the call
    (qd_decode_attention_plan_detail);
  * max abs error <= 2e-3 against the oracle's restatement of the reference
    kernels (flash_decode_q1_opt.cuh);
  * within half a binary16 ulp (+1e-5) of float64 attention, since the
    kernels keep every intermediate in fp32 and round once.
Closed forms (L=1, constant inputs) are bit-exact.  Configs 1-3 of the
benchmark run at full size.
"""
import numpy as np
import pytest
import torch

from common import AttnCase, ulp16
from oracle import oracle

pytestmark = pytest.mark.gpu

ATOL = 2e-3          # north-star tolerance on fp16 attention outputs
TAIL = 64            # sentinel elements after `out` that must stay untouched


@pytest.fixture(scope="module")
def qdiy():
    import qdiy as m
    torch.cuda.set_device(0)
    m.load()
    return m


class GpuCase:
    def __init__(self, qdiy, case: AttnCase):
        self.case = case
        self.ctx = qdiy.Context(num_heads=case.H, max_seqlen=case.max_seqlen,
                                kv_row_stride=case.row_stride, kv_head_stride=case.head_stride)
        self.q = torch.from_numpy(case.q.reshape(-1)).cuda()
        self.kc = torch.from_numpy(case.kc).cuda()
        self.vc = torch.from_numpy(case.vc).cuda()

    def run(self, seqlen=None, variant="auto", num_splits=0):
        H = self.case.H
        out = torch.full((H * 128 + TAIL,), 7.0, dtype=torch.float16, device="cuda")
        self.ctx.decode_attention(self.q, self.kc, self.vc, out, seqlen or self.case.L, variant,
                                  num_splits)
        torch.cuda.synchronize()
        o = out.cpu().numpy()
        assert np.all(o[H * 128:] == np.float16(7.0)), "write past the end of out"
        o = o[:H * 128].reshape(H, 128)
        L = seqlen or self.case.L
        plan = self.ctx.plan_detail(L, variant, num_splits)
        want = oracle.attention_planned(self.case.q, self.case.kc, self.case.vc, L, H,
                                        self.case.row_stride, self.case.head_stride,
                                        oracle.Plan(*plan.as_tuple()), nthreads=8)
        same = o.view(np.uint16) == want.view(np.uint16)
        assert same.all(), (f"{np.count_nonzero(~same)} outputs differ from the kernel-order "
                            f"oracle under {plan.as_tuple()}")
        return o

    def close(self):
        self.ctx.close()


def _oracle(case, variant=oracle.ENGINE, seqlen=None):
    return oracle.decode_attention(case.q, case.kc, case.vc, seqlen or case.L, case.H,
                                   case.row_stride, case.head_stride, variant, nthreads=8)


def _check(got, case, want_oracle, fp64=None):
    g = got.astype(np.float64)
    err = np.max(np.abs(g - want_oracle.astype(np.float64)))
    assert err <= ATOL, f"max abs err vs oracle {err}"
    ref = case.fp64() if fp64 is None else fp64
    bad = np.abs(g - ref) > 0.5 * ulp16(ref) + 1e-5
    assert not bad.any(), f"{bad.sum()} outputs off float64 by > 0.5 ulp, max {np.max(np.abs(g - ref))}"
    return err


def test_config1_fused_L512(qdiy):
    case = AttnCase(512, H=16, seed=1)
    g = GpuCase(qdiy, case)
    _check(g.run(variant="fused"), case, _oracle(case, oracle.FUSED))
    _check(g.run(variant="auto"), case, _oracle(case, oracle.FUSED))
    g.close()


def test_config2_split_L8192(qdiy):
    case = AttnCase(8192, H=16, seed=2, kscale=0.5)
    g = GpuCase(qdiy, case)
    want = _oracle(case)
    _check(g.run(), case, want)
    for n in (1, 16, 64, 256):
        _check(g.run(variant="split", num_splits=n), case, want)
    g.close()


@pytest.mark.parametrize("spike", [0, 100])
def test_config3_long_context_L32768(qdiy, spike):
    case = AttnCase(32768, H=16, seed=3, spike_every=spike)
    g = GpuCase(qdiy, case)
    _check(g.run(), case, _oracle(case))
    g.close()


EDGE_L = [1, 2, 3, 4, 5, 8, 15, 16, 17, 31, 32, 33, 63, 64, 65, 100, 127, 128, 129, 255, 256,
          257, 511, 513, 1000, 2047, 4097]


@pytest.mark.parametrize("L", EDGE_L)
def test_edge_lengths_all_variants(qdiy, L):
    case = AttnCase(L, H=4, seed=1000 + L, max_seqlen=L + 37)
    g = GpuCase(qdiy, case)
    want = _oracle(case)
    ref = case.fp64()
    _check(g.run(variant="auto"), case, want, ref)
    _check(g.run(variant="fused"), case, want, ref)
    for n in sorted({1, 2, 3, 7, 64, 256}):
        if n <= L:
            _check(g.run(variant="split", num_splits=n), case, want, ref)
    g.close()


@pytest.mark.parametrize("layout", ["engine", "head_major"])
def test_rows_beyond_seqlen_are_not_read(qdiy, layout):
    case = AttnCase(3000, H=16, seed=5, layout=layout, max_seqlen=3300)
    S = case.max_seqlen
    kc = case.kc.copy()
    if layout == "engine":
        kc.reshape(S, 16, 128)[3000:] = np.float16(60.0)     # would dominate any softmax
    else:
        kc.reshape(16, S, 128)[:, 3000:] = np.float16(60.0)
    case.kc = kc
    g = GpuCase(qdiy, case)
    _check(g.run(), case, _oracle(case))
    _check(g.run(variant="fused"), case, _oracle(case))
    g.close()


def test_single_row_is_v0_bit_exact(qdiy):
    case = AttnCase(1, H=16, seed=6, max_seqlen=16)
    g = GpuCase(qdiy, case)
    for variant in ("auto", "fused", "split"):
        assert np.array_equal(g.run(variant=variant).view(np.uint16), case.Vh[:, 0].view(np.uint16))
    g.close()


@pytest.mark.parametrize("L", [256, 512, 8192, 32768])
def test_bench_constant_inputs_bit_exact(qdiy, L):
    fill = np.array([0x3C3C], np.uint16).view(np.float16)[0]   # bench_fd_opt.cu:134-136
    case = AttnCase(L, H=16, fill=fill)
    g = GpuCase(qdiy, case)
    for variant in ("auto", "fused", "split"):
        assert np.all(g.run(variant=variant).view(np.uint16) == 0x3C3C), variant
    g.close()


def test_repeat_calls_are_deterministic_and_scratch_is_reused(qdiy):
    case = AttnCase(5000, H=16, seed=7)
    g = GpuCase(qdiy, case)
    a = g.run(variant="split", num_splits=40)
    b = g.run(variant="split", num_splits=13)      # different grid, same context
    c = g.run(variant="split", num_splits=40)
    assert np.array_equal(a.view(np.uint16), c.view(np.uint16))
    assert np.max(np.abs(a.astype(np.float32) - b.astype(np.float32))) <= ATOL
    for _ in range(3):
        assert np.array_equal(g.run().view(np.uint16), g.run().view(np.uint16))
    g.close()


def test_inputs_are_not_modified(qdiy):
    case = AttnCase(777, H=16, seed=8)
    g = GpuCase(qdiy, case)
    g.run()
    g.run(variant="fused")
    assert np.array_equal(g.kc.cpu().numpy().view(np.uint16), case.kc.view(np.uint16))
    assert np.array_equal(g.vc.cpu().numpy().view(np.uint16), case.vc.view(np.uint16))
    assert np.array_equal(g.q.cpu().numpy().view(np.uint16), case.q.reshape(-1).view(np.uint16))
    g.close()


def test_head_independence(qdiy):
    case = AttnCase(1500, H=16, seed=9)
    g = GpuCase(qdiy, case)
    a = g.run()
    kc = g.kc.view(1500, 16, 128)
    kc[:, 5] = -kc[:, 5]
    case.kc = g.kc.cpu().numpy()          # the oracle check in run() sees the same cache
    b = g.run()
    keep = [h for h in range(16) if h != 5]
    assert np.array_equal(a[keep].view(np.uint16), b[keep].view(np.uint16))
    assert not np.array_equal(a[5], b[5])
    g.close()


@pytest.mark.parametrize("variant", ["auto", "fused", "split"])
def test_non_finite_inputs_match_the_oracle(qdiy, variant):
    """A NaN key element makes its row's exponent NaN, which the exponential
    maps to 0: the row drops out and the head stays finite (the reference's
    expf would make that head NaN; this deviation is deliberate).  An inf in a
    V row makes the head inf/NaN; an inf key element makes the head's maximum
    inf and its output NaN (0/0), as in the reference.  The GPU must give the
    kernel-order oracle's NaN positions and bits everywhere else (NaN payloads
    differ between GPU and host), and a clean head must not change."""
    L, H, S = 700, 4, 720
    clean = AttnCase(L, H=H, seed=31, max_seqlen=S)
    case = AttnCase(L, H=H, seed=31, max_seqlen=S)
    kc = case.kc.copy().reshape(S, H, 128)
    vc = case.vc.copy().reshape(S, H, 128)
    kc[123, 0, 17] = np.float16(np.nan)
    vc[456, 1, 3] = np.float16(np.inf)
    kc[321, 2, 40] = np.float16(np.inf) * np.sign(case.q.reshape(H, 128)[2, 40] or 1)
    case.kc, case.vc = kc.reshape(-1), vc.reshape(-1)
    ctx = qdiy.Context(num_heads=H, max_seqlen=S)
    outs = {}
    for name, c in (("clean", clean), ("planted", case)):
        out = torch.empty(H * 128, dtype=torch.float16, device="cuda")
        ctx.decode_attention(torch.from_numpy(c.q.reshape(-1)).cuda(), torch.from_numpy(c.kc).cuda(),
                             torch.from_numpy(c.vc).cuda(), out, L, variant, 5 if variant == "split" else 0)
        torch.cuda.synchronize()
        outs[name] = out.cpu().numpy().reshape(H, 128)
    plan = ctx.plan_detail(L, variant, 5 if variant == "split" else 0)
    ctx.close()
    want = oracle.attention_planned(case.q, case.kc, case.vc, L, H, case.row_stride, case.head_stride,
                                    oracle.Plan(*plan.as_tuple()), nthreads=8)
    got = outs["planted"]
    assert np.array_equal(np.isnan(got), np.isnan(want))
    fin = ~np.isnan(want)
    assert np.array_equal(got[fin].view(np.uint16), want[fin].view(np.uint16))
    assert np.isfinite(got[0]).all()                      # the NaN key row dropped out
    ref = _oracle(case)                                    # the reference kernels' order (expf)
    assert np.isnan(ref[0]).all()                          # ... where expf poisons the head
    assert np.array_equal(np.isnan(got[1:]), np.isnan(ref[1:]))
    assert np.array_equal(np.isinf(got[1:]), np.isinf(ref[1:]))
    assert not np.isfinite(got[1]).all() and np.isnan(got[2]).all()
    assert np.array_equal(got[3].view(np.uint16), outs["clean"][3].view(np.uint16))


def test_invalid_arguments_raise(qdiy):
    case = AttnCase(64, H=16, seed=10)
    g = GpuCase(qdiy, case)
    out = torch.empty(16 * 128 + 8, dtype=torch.float16, device="cuda")
    with pytest.raises(qdiy.QdError) as e:
        g.ctx.decode_attention(g.q, g.kc, g.vc, out, 0)
    assert e.value.code == qdiy.QD_EINVAL
    with pytest.raises(qdiy.QdError):
        g.ctx.decode_attention(g.q, g.kc, g.vc, out, 65)              # > max_seqlen
    with pytest.raises(qdiy.QdError):
        g.ctx.decode_attention(g.q, g.kc, g.vc, out[1:], 10)          # misaligned out
    with pytest.raises(qdiy.QdError):
        g.ctx.decode_attention(g.q, g.kc, g.vc, out, 10, "split", qdiy.max_splits() + 1)
    with pytest.raises(ValueError):
        g.ctx.decode_attention(g.q, g.kc[:1000], g.vc, out, 64)       # cache too small (host check)
    g.close()


def _interleaved_rows(L, block, splits, c):
    full, rem = divmod(L, block)
    nfull = (full - 1 - c) // splits + 1 if full > c else 0
    return nfull * block + (rem if rem > 0 and full % splits == c else 0)


def _planner_rules(L, H, cus, variant="auto", requested=0, period=0):
    """The launch planner as its measured rules state it: fused (one 16-wave
    workgroup per head, 4-row tiles) up to 128 rows where the context merges
    split plans in the scan kernel (dispatch round-robin with a period that
    divides H), else up to 224; above, one split workgroup per CU in total,
    at most one per 16 rows, at most 256, rows per split rounded up to a
    multiple of 4, no empty workgroups, 4 waves, 4-row tiles from 64 rows per
    split; automatic plans beyond 3072 rows of such a context, with at most 64
    splits and one workgroup per CU, deal the rows to the splits in blocks of
    32 rows of 2-row tiles up to 16384 rows, of 64 rows of 4-row tiles beyond
    (the reported rows per split are split 0's)."""
    xmerge = period >= 1 and H % period == 0
    fused_max = 128 if xmerge else 224
    if variant == "fused" or (variant == "auto" and L <= fused_max):
        return (0, 1, L, 4, 16, 0)
    if requested > 0:
        s = min(requested, 256)
    else:
        s = max(1, min(cus // H, (L + 15) // 16, 256))
    rows = -(-L // s)
    rows = (rows + 3) & ~3
    splits = -(-L // rows)
    if requested <= 0 and xmerge and L > 3072 and splits <= 64 and splits * H <= cus:
        block = 32 if L <= 16384 else 64
        splits = min(splits, -(-L // block))
        return (1, splits, _interleaved_rows(L, block, splits, 0), block // 16, 4, block)
    return (1, splits, rows, 4 if rows >= 64 else 2, 4, 0)


@pytest.mark.parametrize("H", [1, 4, 12, 16, 24, 40])
def test_planner_follows_its_rules(qdiy, H):
    """Every plan the library reports equals the planner's stated rules at this
    device's CU count, for automatic, fused and explicit split plans."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    lengths = sorted(set(list(range(1, 300)) + list(range(1000, 1100)) + list(range(2000, 2100)) +
                         [3071, 3072, 3073, 4095, 4096, 4097, 8191, 8192, 8193, 16384, 16385,
                          32767, 32768]))
    with qdiy.Context(num_heads=H, max_seqlen=32768) as ctx:
        period = ctx.xcd_period()
        for L in lengths:
            assert ctx.plan_detail(L).as_tuple() == _planner_rules(L, H, cus, period=period), (H, L)
            plan = ctx.plan_detail(L)
            want_in_kernel = int(plan.variant == qdiy.SPLIT and period >= 1 and H % period == 0
                                 and (L <= 3072 or plan.block_rows) and plan.num_splits <= 64
                                 and plan.num_splits * H <= cus)
            assert plan.merge_in_kernel == want_in_kernel, (H, L)
        for L in (1, 300, 8192):
            assert ctx.plan_detail(L, "fused").as_tuple() == _planner_rules(L, H, cus, "fused"), L
            for req in (1, 5, 16, 64, 300):
                assert ctx.plan_detail(L, "split", min(req, qdiy.max_splits())).as_tuple() == \
                    _planner_rules(L, H, cus, "split", min(req, qdiy.max_splits())), (L, req)
