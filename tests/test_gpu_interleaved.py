"""Split plans with interleaved blocks (qd_ctx_set_split_shape).

Workgroups of 8 (or 4) waves whose rows form blocks of one load round dealt to
the splits in turn.  Each shape has its own summation order; the kernel must
give the kernel-order oracle's bits for the plan it reports
(qd_decode_attention_plan_detail), with the merge in the scan kernel and with
a merge kernel, also where the merging workgroup scans splits again, and for
ragged lengths (a short last block, splits with unequal block counts).
"""
import numpy as np
import pytest
import torch

from common import AttnCase, ulp16
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


SHAPES = [(8, 2, 1), (8, 4, 1), (4, 4, 1), (4, 2, 1)]


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("H,L,layout", [(16, 8192, "engine"), (16, 1000, "engine"),
                                        (16, 3001, "head_major"), (8, 20000, "engine"),
                                        (16, 32768, "engine"), (24, 5000, "engine"),
                                        (16, 65, "engine")])
def test_interleaved_shapes_match_the_oracle(qdiy, shape, H, L, layout):
    case = AttnCase(L, H=H, seed=L + 7 * H, kscale=0.5, layout=layout)
    t = _upload(case)
    with qdiy.Context(num_heads=H, max_seqlen=case.max_seqlen, kv_row_stride=case.row_stride,
                      kv_head_stride=case.head_stride) as ctx:
        ctx.set_split_shape(*shape)
        outs = {}
        for mode in (qdiy.MERGE_IN_KERNEL, qdiy.MERGE_TWO_LAUNCHES):
            ctx.set_merge(mode)
            plan = ctx.plan_detail(L, "split")
            print(f"H={H} L={L} {layout} shape={shape} mode={mode}: plan {plan.as_tuple()} "
                  f"in-kernel {plan.merge_in_kernel}", flush=True)
            assert plan.block_rows == shape[0] * 4 * shape[1] and plan.waves == shape[0]
            outs[mode] = _attend(ctx, t, L, H, "split")
        want = oracle.attention_planned(case.q, case.kc, case.vc, L, H, case.row_stride,
                                        case.head_stride, oracle.Plan(*plan.as_tuple()), nthreads=8)
    for mode, got in outs.items():
        diff = got.view(np.uint16) != want.view(np.uint16)
        assert not diff.any(), f"merge mode {mode}: {np.count_nonzero(diff)} outputs differ from the oracle"
    ref = case.fp64()
    assert np.all(np.abs(want.astype(np.float64) - ref) <= 0.5 * ulp16(ref) + 1e-5)


@pytest.mark.parametrize("mask", [0xFFFFFFFF, 0x5])
def test_interleaved_rescan_path(qdiy, mask):
    """The merging workgroup scans the masked splits again from the KV cache, with
    the interleaved row mapping of those splits: the same bits."""
    H, L = 16, 8192
    case = AttnCase(L, H=H, seed=91, kscale=0.5)
    t = _upload(case)
    with qdiy.Context(num_heads=H, max_seqlen=L) as ctx:
        ctx.set_split_shape(8, 2, 1)
        ctx.set_merge(qdiy.MERGE_IN_KERNEL)
        want = _attend(ctx, t, L, H)
        assert ctx.plan_detail(L).merge_in_kernel == 1
        ctx.set_recompute_mask(mask)
        got = _attend(ctx, t, L, H)
        ctx.set_recompute_mask(0)
    assert np.array_equal(want.view(np.uint16), got.view(np.uint16))


def test_split_shape_validation(qdiy):
    with qdiy.Context(num_heads=16, max_seqlen=1024) as ctx:
        for bad in ((8, 8, 1), (16, 2, 1), (8, 2, 0), (4, 2, 0), (4, 3, 1), (0, 2, 0)):
            with pytest.raises(qdiy.QdError):
                ctx.set_split_shape(*bad)
        ctx.set_split_shape(8, 2, 1)
        ctx.set_split_shape(0, 0, 0)
        assert ctx.plan_detail(1000).block_rows == 0
