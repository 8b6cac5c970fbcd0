"""Shared input builders and fp64 references for the parity tests.

Inputs are drawn from numpy's PCG64 generator (portable across platforms for a
given numpy version) in float32 and rounded to fp16 with numpy's RNE cast.
"""
from __future__ import annotations

import numpy as np

D = 128


def normal_f16(rng: np.random.Generator, shape, scale: float = 1.0) -> np.ndarray:
    x = rng.standard_normal(size=shape, dtype=np.float32)
    if scale != 1.0:
        x *= np.float32(scale)
    return x.astype(np.float16)


def ulp16(x) -> np.ndarray:
    """Spacing of binary16 at |x| (2^-24 in the subnormal range)."""
    a = np.abs(np.asarray(x, dtype=np.float64))
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -14)))
    return np.where(a < 2.0 ** -14, 2.0 ** -24, 2.0 ** (e - 10))


def attn_fp64(q: np.ndarray, K: np.ndarray, V: np.ndarray) -> np.ndarray:
    """Textbook q=1 attention in float64: softmax(K q / sqrt(128)) V."""
    s = K.astype(np.float64) @ q.astype(np.float64) / np.sqrt(128.0)
    p = np.exp(s - s.max())
    p /= p.sum()
    return p @ V.astype(np.float64)


class AttnCase:
    """Q [H,128] and K/V for H heads x L rows, stored in a cache layout.

    layout "engine": the reference engine's [pos][head*128] rows
    (qwen_infer.cu:75-76, row stride H*128, head stride 128), with
    max_seqlen >= L rows allocated.  layout "head_major": [head][max_seqlen][128]
    (row stride 128, head stride max_seqlen*128).
    """

    def __init__(self, L, H=16, seed=0, kscale=1.0, spike_every=0, layout="engine",
                 max_seqlen=None, fill=None):
        self.L, self.H = L, H
        self.max_seqlen = max_seqlen or L
        rng = np.random.default_rng(seed)
        if fill is not None:
            self.q = np.full((H, D), fill, np.float16)
            Kh = np.full((H, L, D), fill, np.float16)
            Vh = np.full((H, L, D), fill, np.float16)
        else:
            self.q = normal_f16(rng, (H, D))
            Kh = normal_f16(rng, (H, L, D), kscale)
            Vh = normal_f16(rng, (H, L, D))
        if spike_every:
            # adversarial logit spike: every spike_every-th key equals Q
            Kh[:, ::spike_every, :] = self.q[:, None, :]
        self.Kh, self.Vh = Kh, Vh
        self.layout = layout
        S = self.max_seqlen
        if layout == "engine":
            self.row_stride, self.head_stride = H * D, D
            kc = np.zeros((S, H, D), np.float16)
            vc = np.zeros((S, H, D), np.float16)
            kc[:L] = Kh.transpose(1, 0, 2)
            vc[:L] = Vh.transpose(1, 0, 2)
        elif layout == "head_major":
            self.row_stride, self.head_stride = D, S * D
            kc = np.zeros((H, S, D), np.float16)
            vc = np.zeros((H, S, D), np.float16)
            kc[:, :L] = Kh
            vc[:, :L] = Vh
        else:
            raise ValueError(layout)
        self.kc = np.ascontiguousarray(kc).reshape(-1)
        self.vc = np.ascontiguousarray(vc).reshape(-1)

    def fp64(self) -> np.ndarray:
        return np.stack([attn_fp64(self.q[h], self.Kh[h], self.Vh[h]) for h in range(self.H)])
