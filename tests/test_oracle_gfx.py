"""Pins the oracle's restatement of this build's gfx950 attention arithmetic
(oracle.exp2, oracle.attention_planned), the functions the GPU kernels are
compared with bit for bit.

What pins them (the kernels' own order is this build's design, so no reference
output can; the pins are independent of the restatement):
  * exp2: float64 exp2 within 1.25 fp32 ulp over its whole domain, exact powers
    of two at integers, 0 below -125, +inf above 128; a dropped polynomial term
    misses the bound;
  * attention: float64 brute force within half a binary16 ulp (+1e-5) for
    every plan shape (fused, split, tile depth, waves, ragged last split);
    within 2e-3 of the reference-order oracle; closed forms (L=1 -> V0,
    constant 0x3C inputs -> 0x3C3C, constant V, identical keys, a dominant
    key); layout and head independence bit-exact; rows beyond seqlen unread;
  * different plans agree within one binary16 ulp of each other;
  * interleaved split plans: bit-equal to a contiguous plan over rows reordered
    by hand, and to the one-split contiguous plan; ragged lengths covered.
"""
import numpy as np
import pytest

from common import AttnCase, ulp16
from oracle import oracle


# --------------------------------------------------------------------- exp2

def test_exp2_within_1_25_ulp_of_float64():
    rng = np.random.default_rng(0)
    x = np.concatenate([np.linspace(-124.99, 127.99, 2_000_001, dtype=np.float32),
                        rng.uniform(-0.5, 0.5, 1_000_000).astype(np.float32),
                        rng.uniform(-30, 0, 1_000_000).astype(np.float32)])
    got = oracle.exp2(x).astype(np.float64)
    want = np.exp2(x.astype(np.float64))
    ulp = np.spacing(want.astype(np.float32)).astype(np.float64)
    assert np.max(np.abs(got - want) / ulp) <= 1.25


def test_exp2_special_values():
    ints = np.arange(-124, 128, dtype=np.float32)
    assert np.array_equal(oracle.exp2(ints), np.exp2(ints.astype(np.float64)).astype(np.float32))
    assert oracle.exp2(np.float32([0.0]))[0] == np.float32(1.0)
    low = np.float32([-125.0, -126.0, -1e6, -np.inf, np.nan])
    assert np.all(oracle.exp2(low) == 0.0)
    assert np.all(np.isinf(oracle.exp2(np.float32([128.0, 1000.0, np.inf]))))


def _fma32(a, b, c):
    """One rounding of a*b + c to float32 (the products of two float32 values are
    exact in long double's 64-bit significand)."""
    return (np.longdouble(a) * np.longdouble(b) + np.longdouble(c)).astype(np.float32)


def test_exp2_bound_has_teeth():
    """The same Estrin evaluation with the highest-order term dropped breaks the
    bound by far: the bound is tight enough to see a missing coefficient."""
    c1, c2, c3, c4, c5 = (np.float32(float.fromhex(v)) for v in
                          ("0x1.62e430p-1", "0x1.ebfbdcp-3", "0x1.c6aee8p-5", "0x1.3b2d4ep-7",
                           "0x1.5f3e54p-10"))
    f = np.linspace(-0.5, 0.5, 100001).astype(np.float32)
    f2 = (f.astype(np.float64) * f).astype(np.float32)
    q = _fma32(_fma32(c5, f2, _fma32(c4, f, c3)), f2, _fma32(c2, f, c1))
    p = _fma32(q, f, np.float32(1.0))
    want = np.exp2(f.astype(np.float64))
    ulp = np.spacing(want.astype(np.float32)).astype(np.float64)
    assert np.max(np.abs(p.astype(np.float64) - want) / ulp) > 4.0


# ---------------------------------------------------------------- attention

PLANS = {
    "fused16x4": lambda L: oracle.fused_plan(L),
    "fused16x2": lambda L: oracle.fused_plan(L, rows_per_tile=2),
    "split1": lambda L: oracle.split_plan(L, 1),
    "split3x8": lambda L: oracle.split_plan(L, 3, rows_per_tile=8),
    "split16": lambda L: oracle.split_plan(L, 16),
    "split64w8": lambda L: oracle.split_plan(L, 64, waves=8),
    "split200w16": lambda L: oracle.split_plan(L, 200, waves=16),
    "inter16w8x2": lambda L: oracle.interleaved_plan(L, 16),
    "inter5w8x4": lambda L: oracle.interleaved_plan(L, 5, rows_per_tile=4),
    "inter16w4x4": lambda L: oracle.interleaved_plan(L, 16, rows_per_tile=4, waves=4),
}


def _run(case, plan, L=None, nthreads=4):
    return oracle.attention_planned(case.q, case.kc, case.vc, L or case.L, case.H,
                                    case.row_stride, case.head_stride, plan, nthreads)


@pytest.mark.parametrize("name", sorted(PLANS))
@pytest.mark.parametrize("L", [1, 2, 5, 33, 255, 256, 257, 1000, 3001])
def test_planned_matches_fp64_and_reference_order(name, L):
    plan = PLANS[name](L)
    if plan.variant == 1 and plan.num_splits > L:
        pytest.skip("more splits than rows")
    case = AttnCase(L, H=2, seed=L * 31 + len(name))
    out = _run(case, plan).astype(np.float64)
    ref = case.fp64()
    bad = np.abs(out - ref) > 0.5 * ulp16(ref) + 1e-5
    assert not bad.any(), (plan, np.max(np.abs(out - ref)))
    want = oracle.decode_attention(case.q, case.kc, case.vc, L, 2, case.row_stride,
                                   case.head_stride, oracle.ENGINE)
    assert np.max(np.abs(out - want.astype(np.float64))) <= 2e-3


@pytest.mark.parametrize("spike", [0, 100])
def test_planned_long_context(spike):
    case = AttnCase(32768, H=2, seed=3, spike_every=spike)
    ref = case.fp64()
    for plan in (oracle.split_plan(32768, 16), oracle.split_plan(32768, 256, rows_per_tile=2)):
        out = _run(case, plan).astype(np.float64)
        assert np.all(np.abs(out - ref) <= 0.5 * ulp16(ref) + 1e-5)


@pytest.mark.parametrize("name", sorted(PLANS))
def test_planned_single_row_is_v0(name):
    case = AttnCase(1, H=3, seed=5)
    out = _run(case, PLANS[name](1) if PLANS[name](1).num_splits <= 1 else oracle.split_plan(1, 1))
    assert np.array_equal(out.view(np.uint16), case.Vh[:, 0].view(np.uint16))


@pytest.mark.parametrize("L", [256, 4096])
def test_planned_constant_inputs(L):
    fill = np.array([0x3C3C], np.uint16).view(np.float16)[0]   # bench_fd_opt.cu:134-136
    case = AttnCase(L, H=2, fill=fill)
    for plan in (oracle.fused_plan(L), oracle.split_plan(L, 16), oracle.split_plan(L, 7, 8, 8)):
        assert np.all(_run(case, plan).view(np.uint16) == 0x3C3C)


def test_planned_constant_v_and_identical_keys():
    case = AttnCase(777, H=2, seed=9)
    case.Vh[:] = case.Vh[:, :1]
    case.vc[:] = np.ascontiguousarray(case.Vh.transpose(1, 0, 2)).reshape(-1)
    v0 = case.Vh[:, 0].astype(np.float64)
    for plan in (oracle.fused_plan(777), oracle.split_plan(777, 13)):
        assert np.all(np.abs(_run(case, plan).astype(np.float64) - v0) <= ulp16(v0))
    case = AttnCase(300, H=1, seed=11)
    case.Kh[:] = case.Kh[:, :1]
    case.kc[:] = np.ascontiguousarray(case.Kh.transpose(1, 0, 2)).reshape(-1)
    mean = case.Vh[0].astype(np.float64).mean(axis=0)
    for plan in (oracle.fused_plan(300), oracle.split_plan(300, 9)):
        out = _run(case, plan)[0].astype(np.float64)
        assert np.all(np.abs(out - mean) <= 0.5 * ulp16(mean) + 1e-5)


def test_planned_dominant_key():
    case = AttnCase(1500, H=1, seed=12)
    j = 1234
    case.Kh[0, j] = (case.q[0].astype(np.float32) * 4).astype(np.float16)
    case.kc[:] = np.ascontiguousarray(case.Kh.transpose(1, 0, 2)).reshape(-1)
    vj = case.Vh[0, j].astype(np.float64)
    for plan in (oracle.fused_plan(1500), oracle.split_plan(1500, 16)):
        assert np.all(np.abs(_run(case, plan)[0].astype(np.float64) - vj) <= ulp16(vj))


def test_planned_layout_head_and_range_independence():
    eng = AttnCase(600, H=4, seed=33, layout="engine", max_seqlen=640)
    hm = AttnCase(600, H=4, seed=33, layout="head_major", max_seqlen=700)
    plan = oracle.split_plan(600, 10)
    a = _run(eng, plan)
    assert np.array_equal(a.view(np.uint16), _run(hm, plan).view(np.uint16))
    kc = eng.kc.reshape(640, 4, 128).copy()
    kc[:, 2] = -kc[:, 2]
    kc[600:] = np.float16(30.0)                          # rows beyond seqlen
    eng.kc = kc.reshape(-1)
    b = _run(eng, plan)
    assert np.array_equal(a[[0, 1, 3]].view(np.uint16), b[[0, 1, 3]].view(np.uint16))
    assert not np.array_equal(a[2], b[2])


def test_plans_agree_within_rounding():
    """Different plans sum in different orders; in fp32 that stays far below one
    binary16 ulp of the outputs."""
    case = AttnCase(4096, H=4, seed=21)
    outs = [_run(case, p).astype(np.float64)
            for p in (oracle.fused_plan(4096), oracle.split_plan(4096, 16),
                      oracle.split_plan(4096, 16, rows_per_tile=2), oracle.split_plan(4096, 64, waves=8))]
    for o in outs[1:]:
        assert np.all(np.abs(o - outs[0]) <= ulp16(outs[0]))


def _split_rows_by_hand(L, block, splits):
    """Rows of each split of an interleaved plan, listed from its definition:
    blocks of `block` rows dealt to the splits in turn."""
    blocks = [list(range(b, min(b + block, L))) for b in range(0, L, block)]
    return [[r for i in range(c, len(blocks), splits) for r in blocks[i]] for c in range(splits)]


@pytest.mark.parametrize("L,splits,tile,waves", [(1024, 4, 2, 8), (8192, 16, 2, 8), (3072, 6, 4, 8),
                                                 (2048, 16, 4, 4), (8192, 16, 2, 4), (32768, 16, 4, 4)])
def test_interleaved_plan_is_a_contiguous_plan_over_permuted_rows(L, splits, tile, waves):
    """With equal splits, an interleaved plan over the cache must give the bits of a
    contiguous plan of the same shape over a cache whose rows are reordered so that
    each split's rows (listed by hand) lie together.  Attention does not depend on
    row order up to rounding, so float64 parity cannot see a wrong row mapping; this
    check can (a mapping off by one block, or ignoring the split index, fails it)."""
    block = waves * 4 * tile
    assert L % (splits * block) == 0
    case = AttnCase(L, H=3, seed=L + splits)
    # Order-sensitive values: keys 0 (every weight exactly 1, so the outputs are
    # plain fp32 sums of V), V rows of +-2^15 on a random tenth of the rows (as many
    # + as -) among small values that a big partial sum absorbs: which small values
    # survive depends on how the rows are grouped and ordered.
    rng = np.random.default_rng(L * 7 + splits)
    big = rng.choice(L, size=(L // 20) * 2, replace=False)
    vh = (rng.integers(1, 9, size=(3, L, 128)) * 2.0 ** -10).astype(np.float16)
    vh[:, big[: len(big) // 2]] = np.float16(32768.0)
    vh[:, big[len(big) // 2:]] = np.float16(-32768.0)
    case.vc = np.ascontiguousarray(vh.transpose(1, 0, 2)).reshape(-1)
    case.kc = np.zeros_like(case.kc)
    order = [r for rows in _split_rows_by_hand(L, block, splits) for r in rows]
    assert sorted(order) == list(range(L))
    perm = AttnCase(L, H=3, seed=0)
    kc = case.kc.reshape(L, 3, 128)
    vc = case.vc.reshape(L, 3, 128)
    perm.kc = np.ascontiguousarray(kc[order]).reshape(-1)
    perm.vc = np.ascontiguousarray(vc[order]).reshape(-1)
    perm.q = case.q
    inter = oracle.interleaved_plan(L, splits, rows_per_tile=tile, waves=waves)
    assert (inter.num_splits, inter.rows_per_split, inter.block_rows) == (splits, L // splits, block)
    contiguous = oracle.Plan(1, splits, L // splits, tile, waves, 0)
    a = _run(case, inter)
    b = _run(perm, contiguous)
    assert np.array_equal(a.view(np.uint16), b.view(np.uint16))
    # on these values the row grouping shows in the bits: the contiguous plan over
    # the original rows, and the interleaved plan over rows grouped one block off,
    # both differ
    assert not np.array_equal(a.view(np.uint16), _run(case, contiguous).view(np.uint16))
    shifted = [r for rows in _split_rows_by_hand(L, block, splits)[1:] + _split_rows_by_hand(L, block, splits)[:1]
               for r in rows]
    perm.kc = np.ascontiguousarray(kc[shifted]).reshape(-1)
    perm.vc = np.ascontiguousarray(vc[shifted]).reshape(-1)
    assert not np.array_equal(a.view(np.uint16), _run(perm, contiguous).view(np.uint16))


def test_interleaved_single_split_is_the_contiguous_plan():
    """One split takes every block in order: the interleaved plan is then the
    contiguous one-split plan, bit for bit (ragged last block included)."""
    case = AttnCase(1000, H=2, seed=71)
    inter = oracle.interleaved_plan(1000, 1)
    assert (inter.num_splits, inter.rows_per_split) == (1, 1000)
    a = _run(case, inter)
    b = _run(case, oracle.Plan(1, 1, 1000, 2, 8, 0))
    assert np.array_equal(a.view(np.uint16), b.view(np.uint16))


@pytest.mark.parametrize("L", [65, 127, 1000, 1100, 8191])
def test_interleaved_ragged_lengths_cover_every_row(L):
    """Ragged lengths (a short last block, splits with unequal block counts):
    float64 parity, and a key spike planted in the short last block is found."""
    case = AttnCase(L, H=2, seed=L)
    j = L - 1
    case.Kh[1, j] = (case.q[1].astype(np.float32) * 4).astype(np.float16)
    case.kc[:] = np.ascontiguousarray(case.Kh.transpose(1, 0, 2)).reshape(-1)
    ref = case.fp64()
    for plan in (oracle.interleaved_plan(L, 16), oracle.interleaved_plan(L, 3, rows_per_tile=4),
                 oracle.interleaved_plan(L, 16, rows_per_tile=2, waves=4),
                 oracle.interleaved_plan(L, 5, rows_per_tile=4, waves=4)):
        out = _run(case, plan).astype(np.float64)
        assert np.all(np.abs(out - ref) <= 0.5 * ulp16(ref) + 1e-5), plan
        assert np.all(np.abs(out[1] - case.Vh[1, j].astype(np.float64)) <= ulp16(case.Vh[1, j])), plan


def test_planned_threads_and_validation():
    case = AttnCase(2000, H=4, seed=66)
    plan = oracle.split_plan(2000, 32)
    assert np.array_equal(_run(case, plan, nthreads=1).view(np.uint16),
                          _run(case, plan, nthreads=4).view(np.uint16))
    with pytest.raises(ValueError):      # last split would be empty
        _run(case, oracle.Plan(1, 40, 64, 4, 4))
    with pytest.raises(ValueError):      # splits do not cover seqlen
        _run(case, oracle.Plan(1, 10, 64, 4, 4))
    with pytest.raises(ValueError):
        _run(case, oracle.Plan(1, 32, 64, 0, 4))
    with pytest.raises(ValueError):      # interleaved blocks other than one load round
        _run(case, oracle.Plan(1, 16, 128, 2, 8, 32))
    with pytest.raises(ValueError):      # a split without a block
        _run(case, oracle.Plan(1, 40, 64, 2, 8, 64))
    with pytest.raises(ValueError):      # a fused plan is not interleaved
        _run(case, oracle.Plan(0, 1, 2000, 4, 16, 64))
