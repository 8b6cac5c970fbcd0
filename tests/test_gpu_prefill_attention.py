"""GPU parity of qd_prefill_attention: causal attention of a prompt's queries,
query t at position pos0 + t over cache rows [0, pos0 + t].

Bars:
  * QD_GEMM_EXACT: every query's output is bit-identical to qd_decode_attention
    at that query's length (the decode kernels' arithmetic, batched), which the
    attention tests pin to the oracle;
  * QD_GEMM_MFMA (FlashAttention on the matrix cores): within 2e-3 of a float64
    causal softmax attention of the same fp16 inputs, the bar for attention
    outputs, at every query;
  * both: rows outside the queries' outputs are left untouched, and the
    layouts (engine rows, head-major cache, strided Q and out rows) give the
    same results.
"""
import numpy as np
import pytest
import torch

from common import normal_f16

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


def causal_fp64(Q, K, V, pos0):
    """Q [T,H,128], K/V [L,H,128] float64: out[t,h] = softmax over keys
    j <= pos0 + t of Q[t,h].K[j,h] / sqrt(128), applied to V."""
    T, H, _ = Q.shape
    out = np.empty((T, H, D))
    j = np.arange(K.shape[0])[None, :]
    mask = j > (pos0 + np.arange(T))[:, None]
    for h in range(H):
        s = Q[:, h, :] @ K[:, h, :].T / np.sqrt(128.0)
        s[mask] = -np.inf
        s -= s.max(axis=1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(axis=1, keepdims=True)
        out[:, h, :] = p @ V[:, h, :]
    return out


class Prompt:
    """Random Q rows and a cache holding rows [0, pos0 + T) in the chosen layout."""

    def __init__(self, qdiy, H, pos0, T, seed, layout="engine", q_pad=0, out_pad=0, spike=False,
                 max_seqlen=None):
        rng = np.random.default_rng(seed)
        self.H, self.pos0, self.T = H, pos0, T
        L = pos0 + T
        S = max_seqlen or L + 3
        self.Q = normal_f16(rng, (T, H, D))
        self.K = normal_f16(rng, (L, H, D))
        self.V = normal_f16(rng, (L, H, D))
        if spike:   # adversarial logits: every 100th key equals the last query's Q
            self.K[::100] = self.Q[-1][None]
        row = H * D
        self.q_stride, self.out_stride = row + q_pad, row + out_pad
        if layout == "engine":
            self.ctx = qdiy.Context(num_heads=H, max_seqlen=S)
            kc = np.zeros((S, H, D), np.float16)
            vc = np.zeros((S, H, D), np.float16)
            kc[:L], vc[:L] = self.K, self.V
        else:      # head-major [H][S][128]
            self.ctx = qdiy.Context(num_heads=H, max_seqlen=S, kv_row_stride=D, kv_head_stride=S * D)
            kc = np.zeros((H, S, D), np.float16)
            vc = np.zeros((H, S, D), np.float16)
            kc[:, :L], vc[:, :L] = self.K.transpose(1, 0, 2), self.V.transpose(1, 0, 2)
        self.kc = torch.from_numpy(kc.reshape(-1)).cuda()
        self.vc = torch.from_numpy(vc.reshape(-1)).cuda()
        qrows = np.zeros((T, self.q_stride), np.float16)
        qrows[:, :row] = self.Q.reshape(T, row)
        self.q = torch.from_numpy(qrows.reshape(-1)).cuda()

    def run(self, qdiy, mode):
        out = torch.full((self.T * self.out_stride + 64,), 7.0, dtype=torch.float16, device="cuda")
        self.ctx.prefill_attention(self.q, self.kc, self.vc, out, self.pos0, self.T, mode=mode,
                                   q_stride=self.q_stride, out_stride=self.out_stride)
        torch.cuda.synchronize()
        o = out.cpu().numpy()
        rows = o[:self.T * self.out_stride].reshape(self.T, self.out_stride)
        row = self.H * D
        assert np.all(rows[:, row:] == np.float16(7.0)), "write into a row's padding"
        assert np.all(o[self.T * self.out_stride:] == np.float16(7.0)), "write past the last row"
        return rows[:, :row].reshape(self.T, self.H, D)

    def decode_rows(self, qdiy, ts):
        """qd_decode_attention of query t over pos0 + t + 1 rows, for t in ts."""
        got = {}
        out = torch.empty(self.H * D, dtype=torch.float16, device="cuda")
        for t in ts:
            q = torch.from_numpy(np.ascontiguousarray(self.Q[t].reshape(-1))).cuda()
            self.ctx.decode_attention(q, self.kc, self.vc, out, self.pos0 + t + 1)
            torch.cuda.synchronize()
            got[t] = out.cpu().numpy().reshape(self.H, D).copy()
        return got

    def close(self):
        self.ctx.close()


CASES = [  # H, pos0, T, layout, q_pad, out_pad
    (16, 0, 1, "engine", 0, 0),
    (16, 0, 127, "engine", 4096, 0),     # the engine's Q rows: q_stride = 3 * H * 128
    (16, 0, 256, "engine", 0, 8),
    (16, 200, 40, "engine", 0, 0),       # crosses the fused / split plan boundary of 224 rows
    (16, 100, 60, "engine", 0, 0),       # crosses the fused / split plan boundary of 128 rows
    (16, 777, 33, "head_major", 8, 8),
    (4, 1000, 256, "engine", 0, 0),
    (12, 31, 17, "head_major", 0, 0),
    (12, 5, 40, "engine", 0, 0),         # 36 workgroups: not a multiple of the 8 XCDs
    (16, 3040, 70, "engine", 0, 0),      # crosses 3072 rows: long queries deal rows in 64-row blocks
    (8, 3060, 30, "head_major", 0, 0),
]


@pytest.mark.parametrize("H,pos0,T,layout,q_pad,out_pad", CASES)
def test_exact_mode_is_decode_attention(qdiy, H, pos0, T, layout, q_pad, out_pad):
    pr = Prompt(qdiy, H, pos0, T, seed=H * 7 + pos0 + T, layout=layout, q_pad=q_pad, out_pad=out_pad)
    try:
        got = pr.run(qdiy, qdiy.GEMM_EXACT)
        edges = {max(0, b - pos0 - d) for b in (128, 224, 3072) for d in (0, 1)}
        ts = sorted(({0, T // 3, T // 2, T - 1} | edges) & set(range(T)))
        want = pr.decode_rows(qdiy, ts)
        for t in ts:
            assert _same(got[t], want[t]), f"query {t} (position {pos0 + t})"
    finally:
        pr.close()


@pytest.mark.parametrize("H,pos0,T,layout,q_pad,out_pad",
                         CASES + [(16, 1792, 256, "engine", 4096, 0), (4, 0, 2048, "engine", 1024, 0),
                                  (16, 0, 2048, "engine", 4096, 0),      # a full pass at Qwen-1.8B's heads
                                  (8, 300, 1000, "head_major", 0, 8)])   # ragged last tile, continuing a prompt
def test_mfma_mode_within_2e3(qdiy, H, pos0, T, layout, q_pad, out_pad):
    pr = Prompt(qdiy, H, pos0, T, seed=H * 11 + pos0 + T, layout=layout, q_pad=q_pad, out_pad=out_pad)
    try:
        got = pr.run(qdiy, qdiy.GEMM_MFMA).astype(np.float64)
        want = causal_fp64(pr.Q.astype(np.float64), pr.K.astype(np.float64), pr.V.astype(np.float64), pos0)
        err = np.abs(got - want)
        assert np.all(np.isfinite(got))
        assert float(err.max()) <= 2e-3, (float(err.max()), np.unravel_index(err.argmax(), err.shape))
    finally:
        pr.close()


@pytest.mark.parametrize("seed", range(24))
def test_mfma_mode_random_prompts(qdiy, seed):
    """Seeded random head counts, cache layouts, positions, query counts (ragged
    against the 64-query tiles and 32-key blocks) and Q / out row padding: every
    query within 2e-3 of float64, nothing written outside the output rows."""
    rng = np.random.default_rng(91000 + seed)
    H = int(rng.integers(1, 17))
    pos0 = int(rng.integers(0, 1200)) if rng.random() < 0.6 else 0
    T = int(rng.integers(1, 80)) if rng.random() < 0.4 else int(rng.integers(80, 420))
    layout = ("engine", "head_major")[int(rng.integers(0, 2))]
    q_pad, out_pad = 8 * int(rng.integers(0, 4)), 8 * int(rng.integers(0, 4))
    pr = Prompt(qdiy, H, pos0, T, seed=91000 + seed, layout=layout, q_pad=q_pad, out_pad=out_pad)
    try:
        got = pr.run(qdiy, qdiy.GEMM_MFMA).astype(np.float64)
        want = causal_fp64(pr.Q.astype(np.float64), pr.K.astype(np.float64), pr.V.astype(np.float64), pos0)
        err = np.abs(got - want)
        assert np.all(np.isfinite(got))
        assert float(err.max()) <= 2e-3, (H, pos0, T, layout, float(err.max()))
    finally:
        pr.close()


def test_mfma_mode_logit_spike(qdiy):
    """Keys equal to the last query dominate its softmax (logits ~ |q|^2 / sqrt(128)
    ~ 11 against ~N(0,1)): the running-max rescaling keeps every output in bounds."""
    pr = Prompt(qdiy, 16, 500, 64, seed=5, spike=True)
    try:
        got = pr.run(qdiy, qdiy.GEMM_MFMA).astype(np.float64)
        want = causal_fp64(pr.Q.astype(np.float64), pr.K.astype(np.float64), pr.V.astype(np.float64), 500)
        assert float(np.abs(got - want).max()) <= 2e-3
    finally:
        pr.close()


def test_prefill_attention_rejects_bad_arguments(qdiy):
    H, S = 4, 64
    with qdiy.Context(num_heads=H, max_seqlen=S) as ctx:
        kc = torch.zeros(S * H * D, dtype=torch.float16, device="cuda")
        vc = torch.zeros(S * H * D, dtype=torch.float16, device="cuda")
        q = torch.zeros(8 * H * D, dtype=torch.float16, device="cuda")
        out = torch.zeros(8 * H * D, dtype=torch.float16, device="cuda")
        with pytest.raises(qdiy.QdError, match="unknown mode"):
            ctx.prefill_attention(q, kc, vc, out, 0, 8, mode=5)
        with pytest.raises(qdiy.QdError, match="outside"):
            ctx.prefill_attention(q, kc, vc, out, 60, 8)
        with pytest.raises(qdiy.QdError, match="multiples of 8"):
            ctx.prefill_attention(q, kc, vc, out, 0, 2, q_stride=H * D + 4)
        with pytest.raises(qdiy.QdError, match="overlaps"):
            ctx.prefill_attention(q, kc, vc, q[H * D:], 0, 4)
        with pytest.raises(qdiy.QdError, match="overlaps"):
            ctx.prefill_attention(q, kc, vc, kc[2 * H * D:], 0, 4)
        ctx.prefill_attention(q, kc, vc, out, 0, 8, mode=qdiy.GEMM_MFMA)
        torch.cuda.synchronize()
