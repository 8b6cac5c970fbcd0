"""In-kernel merge of split plans (decode_attention_xmerge_kernel).

The last split workgroup of each head folds the head's partials inside the
scan kernel, with the merge kernel's arithmetic, so a call is one launch.
Its outputs must equal the two-launch path's bit for bit (and so the
kernel-order oracle's), also on the path where the merging workgroup scans
again the splits whose partials it cannot see (forced here through the test
hook qd_ctx_set_recompute_mask), and across calls of changing length on one
context (per-call tags; the arrival counters are never reset: each call's
host side passes the value they hold when it starts).
"""
import numpy as np
import pytest
import torch

from common import AttnCase
from oracle import oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def qdiy():
    import qdiy as m
    torch.cuda.set_device(0)
    m.load()
    return m


def _upload(case):
    return (torch.from_numpy(case.q.reshape(-1)).cuda(), torch.from_numpy(case.kc).cuda(),
            torch.from_numpy(case.vc).cuda())


def _attend(ctx, tensors, L, H, variant="auto", splits=0):
    q, kc, vc = tensors
    out = torch.full((H * 128 + 64,), 7.0, dtype=torch.float16, device="cuda")
    ctx.decode_attention(q, kc, vc, out, L, variant, splits)
    torch.cuda.synchronize()
    o = out.cpu().numpy()
    assert np.all(o[H * 128:] == np.float16(7.0)), "write past the end of out"
    return o[:H * 128].reshape(H, 128)


def _oracle(case, ctx, L, variant="auto", splits=0):
    plan = ctx.plan_detail(L, variant, splits)
    return oracle.attention_planned(case.q, case.kc, case.vc, L, case.H, case.row_stride,
                                    case.head_stride, oracle.Plan(*plan.as_tuple()), nthreads=8)


def _same(a, b, what):
    diff = a.view(np.uint16) != b.view(np.uint16)
    assert not diff.any(), f"{what}: {np.count_nonzero(diff)} outputs differ"


def test_context_finds_round_robin_dispatch(qdiy):
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    with qdiy.Context(num_heads=16, max_seqlen=8192) as ctx:
        period = ctx.xcd_period()
        assert period >= 1, (f"workgroup dispatch was not found round-robin over XCDs; a probe "
                             f"now places workgroups 0..31 on {qdiy.xcd_placement(256)[:32]}")
        if cus == 256:
            assert period == 8          # MI355X: 8 XCDs of 32 CUs
        for L, in_kernel in ((100, 0), (129, 1), (1024, 1), (2048, 1), (3072, 1), (3073, 1), (8192, 1)):
            plan = ctx.plan_detail(L)
            assert plan.merge_in_kernel == in_kernel, L           # 100 rows: fused, nothing to merge
            assert plan.variant == (qdiy.FUSED if L <= 128 else qdiy.SPLIT), L
            assert plan.block_rows == (32 if L > 3072 else 0), L  # long plans: interleaved blocks
        ctx.set_merge(qdiy.MERGE_IN_KERNEL)
        assert ctx.plan_detail(8192).merge_in_kernel == 1
        ctx.set_merge(qdiy.MERGE_TWO_LAUNCHES)
        assert ctx.plan_detail(1024).merge_in_kernel == 0
        assert ctx.plan_detail(8192).merge_in_kernel == 0
        assert ctx.plan_detail(8192).block_rows == 32           # the same plan: the same bits
        assert ctx.plan_detail(200).variant == qdiy.FUSED       # fused up to 224 rows then


@pytest.mark.parametrize("H,L,layout", [(16, 8192, "engine"), (16, 300, "engine"),
                                        (16, 1500, "engine"), (16, 32768, "engine"),
                                        (8, 5000, "head_major"), (32, 2000, "engine"),
                                        (24, 4000, "engine"), (12, 3000, "engine")])
def test_in_kernel_merge_equals_two_launches(qdiy, H, L, layout):
    """Same bits in every merge mode, and as the kernel-order oracle.  12 heads
    are not a multiple of the dispatch period: that context keeps two launches
    in every mode."""
    case = AttnCase(L, H=H, seed=L + H, kscale=0.5, layout=layout)
    t = _upload(case)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    with qdiy.Context(num_heads=H, max_seqlen=case.max_seqlen, kv_row_stride=case.row_stride,
                      kv_head_stride=case.head_stride) as ctx:
        period = ctx.xcd_period()
        outs = []
        for mode in (qdiy.MERGE_IN_KERNEL, qdiy.MERGE_AUTO, qdiy.MERGE_TWO_LAUNCHES):
            ctx.set_merge(mode)
            plan = ctx.plan_detail(L)
            can = (plan.variant == qdiy.SPLIT and period >= 1 and H % period == 0
                   and plan.num_splits <= 64 and plan.num_splits * H <= cus)
            want = {qdiy.MERGE_IN_KERNEL: can, qdiy.MERGE_AUTO: can and (L <= 3072 or plan.block_rows > 0),
                    qdiy.MERGE_TWO_LAUNCHES: False}[mode]
            assert plan.merge_in_kernel == int(want), (H, L, mode, plan.as_tuple(), period)
            outs.append(_attend(ctx, t, L, H))
        _same(outs[0], outs[2], f"H={H} L={L}: in-kernel vs two-launch merge")
        _same(outs[1], outs[2], f"H={H} L={L}: automatic vs two-launch merge")
        _same(outs[0], _oracle(case, ctx, L), f"H={H} L={L}: vs the kernel-order oracle")


@pytest.mark.parametrize("H,L", [(16, 8192), (8, 5000), (16, 260)])
@pytest.mark.parametrize("mask", [0xFFFFFFFF, 0x1, 0x8000, 0x55555555])
def test_recompute_path_gives_the_same_bits(qdiy, H, L, mask):
    """The merging workgroup scans the masked splits again itself (the path it
    takes for partials written on another XCD): the outputs do not change.
    8 heads at 5000 rows plan 32 splits per head (the 32-slot merger), 260 rows
    16 splits of 16-20 rows."""
    case = AttnCase(L, H=H, seed=L, kscale=0.5)
    t = _upload(case)
    with qdiy.Context(num_heads=H, max_seqlen=L) as ctx:
        ctx.set_merge(qdiy.MERGE_IN_KERNEL)
        assert ctx.plan_detail(L).merge_in_kernel == 1
        want = _attend(ctx, t, L, H)
        ctx.set_recompute_mask(mask)
        got = _attend(ctx, t, L, H)
        again = _attend(ctx, t, L, H)
        ctx.set_recompute_mask(0)
        after = _attend(ctx, t, L, H)
    _same(got, want, f"L={L} mask={mask:#x}")
    _same(again, want, f"L={L} mask={mask:#x}, second call")
    _same(after, want, f"L={L}: after the hook is cleared")


def test_calls_in_sequence_with_changing_lengths(qdiy):
    """One context, calls of changing length, inputs and merge mode back to back
    on one stream without host synchronisation between them: the arrival
    counters keep the values the host expects across calls of either kind, and
    stale slots of earlier calls (more splits, older tags) are never read as
    this call's."""
    H, S = 16, 8192
    calls = [(8192, qdiy.MERGE_IN_KERNEL), (300, qdiy.MERGE_AUTO), (8192, qdiy.MERGE_AUTO),
             (1500, qdiy.MERGE_AUTO), (4000, qdiy.MERGE_IN_KERNEL), (300, qdiy.MERGE_TWO_LAUNCHES),
             (2000, qdiy.MERGE_IN_KERNEL), (8192, qdiy.MERGE_IN_KERNEL), (260, qdiy.MERGE_AUTO)]
    cases = [AttnCase(S, H=H, seed=100 + i, kscale=0.5) for i in range(len(calls))]
    ups = [_upload(c) for c in cases]
    outs = [torch.empty(H * 128, dtype=torch.float16, device="cuda") for _ in calls]
    with qdiy.Context(num_heads=H, max_seqlen=S) as ctx:
        for (q, kc, vc), out, (L, mode) in zip(ups, outs, calls):
            ctx.set_merge(mode)
            ctx.decode_attention(q, kc, vc, out, L)
        torch.cuda.synchronize()
        ctx.set_merge(qdiy.MERGE_AUTO)
        for i, (case, out, (L, mode)) in enumerate(zip(cases, outs, calls)):
            _same(out.cpu().numpy().reshape(H, 128), _oracle(case, ctx, L), f"call {i} (L={L})")


def test_explicit_split_counts(qdiy):
    """qd_decode_attention_split merges in the kernel while the grid is at most one
    workgroup per CU, and with a merge kernel beyond; both equal the oracle bit
    for bit."""
    H, L = 16, 6000
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    case = AttnCase(L, H=H, seed=9, kscale=0.5)
    t = _upload(case)
    with qdiy.Context(num_heads=H, max_seqlen=L) as ctx:
        ctx.set_merge(qdiy.MERGE_IN_KERNEL)
        for n in (1, 2, 7, 16, 33, 64, 65, 128):
            plan = ctx.plan_detail(L, "split", n)
            assert plan.merge_in_kernel == int(plan.num_splits * H <= cus), (n, plan.as_tuple())
            _same(_attend(ctx, t, L, H, "split", n), _oracle(case, ctx, L, "split", n), f"{n} splits")


def test_stage_hook_with_in_kernel_merge(qdiy):
    """With the merge in the kernel, the scan stage is the whole call, and a merge-only
    call is refused (QD_EINVAL, nothing launched, out untouched): there is no merge
    kernel to run alone.  The same holds for a fused plan."""
    import ctypes

    H, L = 16, 3000
    case = AttnCase(L, H=H, seed=3, kscale=0.5)
    q, kc, vc = _upload(case)
    lib = qdiy.load()
    with qdiy.Context(num_heads=H, max_seqlen=L) as ctx:
        ctx.set_merge(qdiy.MERGE_IN_KERNEL)
        want = _attend(ctx, (q, kc, vc), L, H)
        for stages, expect in ((1, want), (2, None)):
            out = torch.full((H * 128,), 7.0, dtype=torch.float16, device="cuda")
            rc = lib.qd_decode_attention_stage(ctx._h, ctypes.c_void_p(q.data_ptr()),
                                               ctypes.c_void_p(kc.data_ptr()),
                                               ctypes.c_void_p(vc.data_ptr()),
                                               ctypes.c_void_p(out.data_ptr()), L, H, 128, stages,
                                               ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
            assert rc == (0 if expect is not None else qdiy.QD_EINVAL)
            if expect is None:
                assert b"no merge kernel" in lib.qd_last_error()
            torch.cuda.synchronize()
            o = out.cpu().numpy().reshape(H, 128)
            if expect is None:
                assert np.all(o == np.float16(7.0))
            else:
                _same(o, expect, "scan stage")
        # a fused plan (100 rows) has no merge kernel either
        rc = lib.qd_decode_attention_stage(ctx._h, ctypes.c_void_p(q.data_ptr()),
                                           ctypes.c_void_p(kc.data_ptr()),
                                           ctypes.c_void_p(vc.data_ptr()),
                                           ctypes.c_void_p(out.data_ptr()), 100, H, 128, 2,
                                           ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        assert rc == qdiy.QD_EINVAL


@pytest.mark.parametrize("L", [300, 768, 1280, 3000, 8192, 16385, 20000])
def test_loads_per_round_give_the_same_bits(qdiy, L):
    """A wave may issue the loads of 1, 2 or 4 of its tiles before consuming
    them in order, or keep its next tile's loads in flight while it consumes
    one (QD_SCAN_ROLLING): the arithmetic is the same, so is every output bit,
    with the merge in the kernel or in a merge kernel.  The planner's own
    choice (two tiles per round with the merge in the kernel where a wave of a
    contiguous plan has two or more; rolling for interleaved 2-row plans, one
    per round for 4-row ones; interleaved plans load one tile per round
    whatever depth is forced, rolling aside) is what plan_detail reports."""
    H = 16
    case = AttnCase(L, H=H, seed=L + 1, kscale=0.5)
    t = _upload(case)
    with qdiy.Context(num_heads=H, max_seqlen=L) as ctx:
        want = _oracle(case, ctx, L)
        for mode in (qdiy.MERGE_IN_KERNEL, qdiy.MERGE_TWO_LAUNCHES):
            ctx.set_merge(mode)
            plan = ctx.plan_detail(L)
            tiles = -(-plan.rows_per_split // (16 * plan.rows_per_tile))
            auto = ((0 if plan.rows_per_tile == 2 else 1) if plan.block_rows else
                    2 if plan.merge_in_kernel and tiles >= 2 else 1)
            assert plan.loads_per_round == auto, (L, mode, plan.as_tuple(), plan.loads_per_round)
            _same(_attend(ctx, t, L, H), want, f"L={L} mode={mode}, planner's depth {auto}")
            for depth in (1, 2, 4, qdiy.SCAN_ROLLING):
                ctx.set_scan_depth(depth)
                reported = 0 if depth == qdiy.SCAN_ROLLING else 1 if plan.block_rows else depth
                assert ctx.plan_detail(L).loads_per_round == reported, (L, depth)
                _same(_attend(ctx, t, L, H), want, f"L={L} mode={mode} depth={depth}")
            ctx.set_scan_depth(0)


def test_merge_statistics(qdiy):
    """qd_ctx_xmerge_stats: with counting on, one merge per head per call and at
    least one read of the slots per merge; splits the test hook marks are
    counted as scanned again whether or not counting is on."""
    H, L = 16, 2000
    case = AttnCase(L, H=H, seed=11, kscale=0.5)
    t = _upload(case)
    with qdiy.Context(num_heads=H, max_seqlen=L) as ctx:
        ctx.set_merge(qdiy.MERGE_IN_KERNEL)
        splits = ctx.plan_detail(L).num_splits
        assert ctx.xmerge_stats() == (0, 0, 0)
        _attend(ctx, t, L, H)
        assert ctx.xmerge_stats()[:2] == (0, 0)          # counting is off by default
        ctx.count_xmerges(True)
        for _ in range(3):
            _attend(ctx, t, L, H)
        merges, reads, rescans = ctx.xmerge_stats()
        assert merges == 3 * H and reads >= merges and rescans == 0
        ctx.count_xmerges(False)
        ctx.set_recompute_mask(0b101)                     # splits 0 and 2 of each head
        _attend(ctx, t, L, H)
        m2, r2, x2 = ctx.xmerge_stats()
        assert (m2, r2) == (merges, reads) and x2 == 2 * H, (m2, r2, x2, splits)
