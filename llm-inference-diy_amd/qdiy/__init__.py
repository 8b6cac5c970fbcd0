"""Python binding of libqdiy.so, the C ABI declared in include/qdiy/attn.h.

Device memory and streams come from PyTorch (ROCm); every call goes straight to
the HIP kernels through ctypes.  There is no fallback: if the library is not
built, or a call fails, an exception is raised.

torch is imported before the library is loaded so that the library binds to
the HIP runtime torch already has in the process (both carry the SONAME
libamdhip64.so.7): torch's streams and device pointers are then valid
arguments.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np
import torch

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(PKG_DIR, "lib", "libqdiy.so")
ENGINE_EXE = os.path.join(PKG_DIR, "lib", "qdiy_engine")
HEAD_DIM = 128

QD_OK, QD_EINVAL, QD_EHIP, QD_ENOMEM = 0, 1, 2, 3
FUSED, SPLIT = 0, 1

EXPORTS = (
    "qd_ctx_create", "qd_ctx_destroy", "qd_qkv_bias_rope_cache", "qd_qkv_proj_rope_cache",
    "qd_decode_attention",
    "qd_decode_attention_fused", "qd_decode_attention_split", "qd_decode_attention_plan",
    "qd_decode_attention_plan_detail", "qd_decode_attention_noalloc",
    # qdiy/bench.h
    "qd_decode_attention_stage", "qd_ctx_set_merge", "qd_ctx_set_recompute_mask",
    "qd_ctx_xcd_period", "qd_xcd_placement", "qd_ctx_xmerge_stats", "qd_ctx_count_xmerges", "qd_ctx_set_scan_depth",
    "qd_ctx_set_split_shape", "qd_ctx_set_front_local", "qd_ctx_front_misses", "qd_qkv_proj_rope_cache_attention",
    "qd_max_splits", "qd_last_error", "qd_version",
    # qdiy/decode.h
    "qd_proj_residual", "qd_ffn_up_swiglu", "qd_lm_head_workspace_bytes", "qd_lm_head_argmax",
    "qd_gemm_nt", "qd_gemm_swiglu", "qd_prefill_attention",
    # qdiy/engine.h
    "qd_model_image_bytes", "qd_model_fill_random", "qd_model_write_random", "qd_engine_create",
    "qd_engine_create_from_image", "qd_engine_destroy", "qd_engine_config", "qd_engine_reset",
    "qd_engine_prefill", "qd_engine_step", "qd_engine_logits", "qd_engine_generate", "qd_engine_kv_rows",
    "qd_engine_set_prefill_mode",
)

GEMM_EXACT, GEMM_MFMA = 0, 1      # qd_gemm_nt / qd_prefill_attention / qd_engine_set_prefill_mode modes
MERGE_AUTO, MERGE_TWO_LAUNCHES, MERGE_IN_KERNEL = 0, 1, 2   # qd_ctx_set_merge modes (qdiy/bench.h)
SCAN_ROLLING = -1   # qd_ctx_set_scan_depth: tile i + 1's loads issued before tile i is consumed


class QdError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"qdiy status {code}: {msg}")
        self.code = code


class Cfg(ctypes.Structure):
    _fields_ = [("num_heads", ctypes.c_int), ("head_dim", ctypes.c_int),
                ("max_seqlen", ctypes.c_int), ("kv_row_stride", ctypes.c_longlong),
                ("kv_head_stride", ctypes.c_longlong), ("rope_base", ctypes.c_float)]


class ModelCfg(ctypes.Structure):
    """qd_model_cfg: the .bin header's model configuration."""
    _fields_ = [("vocab_size", ctypes.c_uint32), ("hidden_size", ctypes.c_uint32),
                ("num_layers", ctypes.c_uint32), ("num_heads", ctypes.c_uint32),
                ("intermediate_size", ctypes.c_uint32), ("max_seqlen", ctypes.c_uint32)]

    def as_dict(self):
        return {f: int(getattr(self, f)) for f, _ in self._fields_}


QWEN_1_8B = dict(vocab_size=151936, hidden_size=2048, num_layers=24, num_heads=16,
                 intermediate_size=5504, max_seqlen=32768)


class AttnPlan(ctypes.Structure):
    """qd_attn_plan: the complete launch plan of one decode-attention call."""
    _fields_ = [("variant", ctypes.c_int), ("num_splits", ctypes.c_int),
                ("rows_per_split", ctypes.c_int), ("rows_per_tile", ctypes.c_int),
                ("waves", ctypes.c_int), ("merge_in_kernel", ctypes.c_int),
                ("loads_per_round", ctypes.c_int), ("block_rows", ctypes.c_int)]

    def as_tuple(self):
        """The plan fields that fix the output bits (merge_in_kernel and
        loads_per_round do not), in oracle.Plan's field order."""
        return (self.variant, self.num_splits, self.rows_per_split, self.rows_per_tile, self.waves,
                self.block_rows)


_lib = None


def load() -> ctypes.CDLL:
    """Loads libqdiy.so (raises if it is not built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is not built: run python llm-inference-diy_amd/build.py")
    L = ctypes.CDLL(LIB_PATH)
    vp, i, ll = ctypes.c_void_p, ctypes.c_int, ctypes.c_longlong
    L.qd_ctx_create.argtypes = [ctypes.POINTER(Cfg), ctypes.POINTER(vp)]
    L.qd_ctx_destroy.argtypes = [vp]
    L.qd_qkv_bias_rope_cache.argtypes = [vp, vp, vp, vp, vp, i, i, i, i, vp]
    L.qd_qkv_proj_rope_cache.argtypes = [vp, vp, vp, ctypes.c_float, vp, vp, vp, vp, vp, i, i, i,
                                         i, vp]
    L.qd_qkv_proj_rope_cache_attention.argtypes = [vp, vp, vp, ctypes.c_float, vp, vp, vp, vp, vp, vp,
                                                   i, i, i, i, vp]
    L.qd_decode_attention.argtypes = [vp, vp, vp, vp, vp, i, i, i, vp]
    L.qd_decode_attention_fused.argtypes = [vp, vp, vp, vp, vp, i, i, i, vp]
    L.qd_decode_attention_split.argtypes = [vp, vp, vp, vp, vp, i, i, i, i, vp]
    L.qd_decode_attention_noalloc.argtypes = [vp, vp, vp, vp, i, i, i, ll, ll, vp]
    L.qd_decode_attention_stage.argtypes = [vp, vp, vp, vp, vp, i, i, i, i, vp]
    L.qd_ctx_set_merge.argtypes = [vp, i]
    L.qd_ctx_set_recompute_mask.argtypes = [vp, ctypes.c_uint]
    L.qd_ctx_xcd_period.argtypes = [vp, ctypes.POINTER(i)]
    ull_p = ctypes.POINTER(ctypes.c_ulonglong)
    L.qd_ctx_xmerge_stats.argtypes = [vp, ull_p, ull_p, ull_p]
    L.qd_ctx_count_xmerges.argtypes = [vp, i]
    L.qd_ctx_set_scan_depth.argtypes = [vp, i]
    L.qd_ctx_set_split_shape.argtypes = [vp, i, i, i]
    L.qd_ctx_set_front_local.argtypes = [vp, i]
    L.qd_ctx_front_misses.argtypes = [vp, ull_p]
    L.qd_xcd_placement.argtypes = [ctypes.POINTER(ctypes.c_uint), i]
    L.qd_decode_attention_plan.argtypes = [vp, i, ctypes.POINTER(i), ctypes.POINTER(i)]
    L.qd_decode_attention_plan_detail.argtypes = [vp, i, i, i, ctypes.POINTER(AttnPlan)]
    u16p = ctypes.POINTER(ctypes.c_uint16)
    ip = ctypes.POINTER(ctypes.c_int)
    L.qd_proj_residual.argtypes = [vp, vp, vp, vp, i, i, vp]
    L.qd_gemm_nt.argtypes = [vp, ll, vp, vp, vp, ll, i, i, i, i, vp]
    L.qd_gemm_swiglu.argtypes = [vp, ll, vp, vp, vp, ll, i, i, i, vp]
    L.qd_prefill_attention.argtypes = [vp, vp, ll, vp, vp, vp, ll, i, i, i, i, i, vp]
    L.qd_engine_set_prefill_mode.argtypes = [vp, i]
    L.qd_ffn_up_swiglu.argtypes = [vp, vp, ctypes.c_float, vp, vp, vp, i, i, vp]
    L.qd_lm_head_workspace_bytes.argtypes = [i]
    L.qd_lm_head_workspace_bytes.restype = ctypes.c_size_t
    L.qd_lm_head_argmax.argtypes = [vp, vp, ctypes.c_float, vp, vp, i, i, vp, ctypes.c_size_t, vp, vp]
    L.qd_model_image_bytes.argtypes = [ctypes.POINTER(ModelCfg)]
    L.qd_model_image_bytes.restype = ll
    L.qd_model_fill_random.argtypes = [vp, ll, ctypes.POINTER(ModelCfg), ctypes.c_uint64,
                                       ctypes.c_float, i]
    L.qd_model_write_random.argtypes = [ctypes.c_char_p, ctypes.POINTER(ModelCfg), ctypes.c_uint64,
                                        ctypes.c_float]
    L.qd_engine_create.argtypes = [ctypes.c_char_p, ctypes.POINTER(vp)]
    L.qd_engine_create_from_image.argtypes = [vp, ll, ctypes.POINTER(vp)]
    L.qd_engine_destroy.argtypes = [vp]
    L.qd_engine_config.argtypes = [vp, ctypes.POINTER(ModelCfg)]
    L.qd_engine_reset.argtypes = [vp]
    L.qd_engine_prefill.argtypes = [vp, ip, i, ip]
    L.qd_engine_step.argtypes = [vp, i, i, ip]
    L.qd_engine_logits.argtypes = [vp, u16p]
    L.qd_engine_kv_rows.argtypes = [vp, i, i, i, u16p, u16p]
    L.qd_engine_generate.argtypes = [vp, ip, i, i, i, ip, ip]
    L.qd_last_error.restype = ctypes.c_char_p
    L.qd_version.restype = ctypes.c_char_p
    _lib = L
    return L


def _check(rc: int) -> None:
    if rc != QD_OK:
        raise QdError(rc, load().qd_last_error().decode())


def _stream(stream) -> ctypes.c_void_p:
    if stream is None:
        stream = torch.cuda.current_stream()
    if isinstance(stream, torch.cuda.Stream):
        stream = stream.cuda_stream
    return ctypes.c_void_p(int(stream))


def _ptr(t: torch.Tensor, name: str, contiguous: bool = True) -> ctypes.c_void_p:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.dtype != torch.float16:
        raise TypeError(f"{name} must be float16, got {t.dtype}")
    if not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor")
    if contiguous and not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    return ctypes.c_void_p(t.data_ptr())


class Context:
    """Owns a qd_ctx (split-KV partials and the RoPE cos/sin table) on the current device."""

    def __init__(self, num_heads: int = 16, max_seqlen: int = 2048, kv_row_stride: int | None = None,
                 kv_head_stride: int = HEAD_DIM, rope_base: float = 10000.0,
                 head_dim: int = HEAD_DIM):
        L = load()
        self.num_heads = num_heads
        self.max_seqlen = max_seqlen
        self.kv_row_stride = num_heads * HEAD_DIM if kv_row_stride is None else kv_row_stride
        self.kv_head_stride = kv_head_stride
        cfg = Cfg(num_heads, head_dim, max_seqlen, self.kv_row_stride, kv_head_stride, rope_base)
        h = ctypes.c_void_p()
        _check(L.qd_ctx_create(ctypes.byref(cfg), ctypes.byref(h)))
        self._h = h

    def close(self) -> None:
        if getattr(self, "_h", None):
            load().qd_ctx_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # -- host-side extent checks (the C ABI takes raw pointers) ---------------
    def _check_cache(self, t: torch.Tensor, name: str, rows: int) -> None:
        last = (rows - 1) * self.kv_row_stride + (self.num_heads - 1) * self.kv_head_stride + HEAD_DIM
        if t.storage_offset() + last > t.untyped_storage().nbytes() // 2 or t.numel() < last:
            raise ValueError(f"{name} holds {t.numel()} elements; {rows} rows need {last}")

    def set_merge(self, mode: int) -> None:
        """qd_ctx_set_merge: MERGE_AUTO (in-kernel where possible) or MERGE_TWO_LAUNCHES."""
        _check(load().qd_ctx_set_merge(self._h, mode))

    def set_recompute_mask(self, mask: int) -> None:
        """qd_ctx_set_recompute_mask (test hook of the in-kernel merge)."""
        _check(load().qd_ctx_set_recompute_mask(self._h, mask & 0xFFFFFFFF))

    def set_scan_depth(self, depth: int) -> None:
        """qd_ctx_set_scan_depth: tiles per load round of split plans (0: planner's;
        SCAN_ROLLING: each wave's next tile in flight while it consumes one)."""
        _check(load().qd_ctx_set_scan_depth(self._h, depth))

    def set_split_shape(self, waves: int, rows_per_tile: int, interleave: int) -> None:
        """qd_ctx_set_split_shape: waves, rows per tile and interleaved blocks of split
        plans ((0, 0, 0): the planner's shape)."""
        _check(load().qd_ctx_set_split_shape(self._h, waves, rows_per_tile, interleave))

    def count_xmerges(self, on: bool = True) -> None:
        """qd_ctx_count_xmerges: count merges and slot reads (off by default)."""
        _check(load().qd_ctx_count_xmerges(self._h, int(on)))

    def xmerge_stats(self) -> tuple:
        """qd_ctx_xmerge_stats: (heads merged, reads of their slots, splits scanned
        again) over the context's in-kernel merges so far."""
        m, r, x = ctypes.c_ulonglong(), ctypes.c_ulonglong(), ctypes.c_ulonglong()
        _check(load().qd_ctx_xmerge_stats(self._h, ctypes.byref(m), ctypes.byref(r), ctypes.byref(x)))
        return m.value, r.value, x.value

    def xcd_period(self) -> int:
        """qd_ctx_xcd_period: round-robin period of workgroup dispatch (0: not round-robin)."""
        v = ctypes.c_int()
        _check(load().qd_ctx_xcd_period(self._h, ctypes.byref(v)))
        return v.value

    def plan(self, seqlen: int):
        v, s = ctypes.c_int(), ctypes.c_int()
        _check(load().qd_decode_attention_plan(self._h, seqlen, ctypes.byref(v), ctypes.byref(s)))
        return ("fused" if v.value == FUSED else "split"), s.value

    def plan_detail(self, seqlen: int, variant: str = "auto", num_splits: int = 0) -> AttnPlan:
        """The complete launch plan decode_attention(variant=...) uses at seqlen."""
        entry = {"auto": 0, "fused": 1, "split": 2}[variant]
        plan = AttnPlan()
        _check(load().qd_decode_attention_plan_detail(self._h, seqlen, entry, num_splits,
                                                      ctypes.byref(plan)))
        return plan

    def decode_attention(self, q: torch.Tensor, k_layer: torch.Tensor, v_layer: torch.Tensor,
                         out: torch.Tensor, seqlen: int, variant: str = "auto", num_splits: int = 0,
                         stream=None) -> torch.Tensor:
        """out[h] = softmax(q[h] K[:seqlen,h]^T / sqrt(128)) V[:seqlen,h] for all heads."""
        H = self.num_heads
        if q.numel() < H * HEAD_DIM or out.numel() < H * HEAD_DIM:
            raise ValueError("q and out need num_heads*128 elements")
        if 1 <= seqlen <= self.max_seqlen:      # out-of-range lengths are the C ABI's to reject
            self._check_cache(k_layer, "k_layer", seqlen)
            self._check_cache(v_layer, "v_layer", seqlen)
        args = (self._h, _ptr(q, "q"), _ptr(k_layer, "k_layer", False), _ptr(v_layer, "v_layer", False),
                _ptr(out, "out"), seqlen, H, HEAD_DIM)
        L = load()
        if variant == "auto":
            _check(L.qd_decode_attention(*args, _stream(stream)))
        elif variant == "fused":
            _check(L.qd_decode_attention_fused(*args, _stream(stream)))
        elif variant == "split":
            _check(L.qd_decode_attention_split(*args, num_splits, _stream(stream)))
        else:
            raise ValueError(f"unknown variant {variant!r}")
        return out

    def prefill_attention(self, q: torch.Tensor, k_layer: torch.Tensor, v_layer: torch.Tensor,
                          out: torch.Tensor, pos0: int, tokens: int, mode: int = GEMM_EXACT,
                          q_stride: int | None = None, out_stride: int | None = None,
                          stream=None) -> torch.Tensor:
        """Causal attention of prompt queries pos0 .. pos0+tokens-1, all heads: query t
        (row t of q, q_stride apart) over cache rows [0, pos0 + t] into row t of out."""
        H = self.num_heads
        row = H * HEAD_DIM
        q_stride = row if q_stride is None else q_stride
        out_stride = row if out_stride is None else out_stride
        if tokens >= 1 and (q.numel() < (tokens - 1) * q_stride + row
                            or out.numel() < (tokens - 1) * out_stride + row):
            raise ValueError("q and out need (tokens-1)*stride + num_heads*128 elements")
        if tokens >= 1 and 0 <= pos0 and pos0 + tokens <= self.max_seqlen:
            self._check_cache(k_layer, "k_layer", pos0 + tokens)
            self._check_cache(v_layer, "v_layer", pos0 + tokens)
        _check(load().qd_prefill_attention(self._h, _ptr(q, "q"), q_stride,
                                           _ptr(k_layer, "k_layer", False),
                                           _ptr(v_layer, "v_layer", False), _ptr(out, "out"),
                                           out_stride, pos0, tokens, H, HEAD_DIM, mode,
                                           _stream(stream)))
        return out

    def qkv_bias_rope_cache(self, qkv: torch.Tensor, bias, k_layer: torch.Tensor,
                            v_layer: torch.Tensor, pos: int, max_seqlen: int | None = None,
                            stream=None) -> None:
        """Bias + RoPE on qkv[3*H*128] in place; rotated K / biased V into cache row pos."""
        H = self.num_heads
        if qkv.numel() < 3 * H * HEAD_DIM:
            raise ValueError("qkv needs 3*num_heads*128 elements")
        if bias is not None and bias.numel() < 3 * H * HEAD_DIM:
            raise ValueError("bias needs 3*num_heads*128 elements")
        if max_seqlen is None:
            max_seqlen = self.max_seqlen
        if 0 <= pos < max_seqlen:
            self._check_cache(k_layer, "k_layer", pos + 1)
            self._check_cache(v_layer, "v_layer", pos + 1)
        bptr = None if bias is None else _ptr(bias, "bias")
        _check(load().qd_qkv_bias_rope_cache(self._h, _ptr(qkv, "qkv"), bptr,
                                             _ptr(k_layer, "k_layer", False),
                                             _ptr(v_layer, "v_layer", False), pos, max_seqlen, H,
                                             HEAD_DIM, _stream(stream)))


    def qkv_proj_rope_cache_attention(self, x: torch.Tensor, norm_w, w_qkv: torch.Tensor, bias,
                                      qkv: torch.Tensor, k_layer: torch.Tensor,
                                      v_layer: torch.Tensor, out: torch.Tensor, pos: int,
                                      eps: float = 1e-6, max_seqlen: int | None = None,
                                      stream=None) -> None:
        """qkv_proj_rope_cache at pos, then decode_attention over pos + 1 rows into out
        (one launch where the plan allows: qd_qkv_proj_rope_cache_attention)."""
        H = self.num_heads
        hid = H * HEAD_DIM
        if x.numel() < hid or qkv.numel() < 3 * hid or w_qkv.numel() < 3 * hid * hid:
            raise ValueError("x needs H*128, qkv 3*H*128 and w_qkv 3*H*128*H*128 elements")
        if norm_w is not None and norm_w.numel() < hid:
            raise ValueError("norm_w needs H*128 elements")
        if bias is not None and bias.numel() < 3 * hid:
            raise ValueError("bias needs 3*H*128 elements")
        if out.numel() < hid:
            raise ValueError("out needs H*128 elements")
        if max_seqlen is None:
            max_seqlen = self.max_seqlen
        if 0 <= pos < max_seqlen:
            self._check_cache(k_layer, "k_layer", pos + 1)
            self._check_cache(v_layer, "v_layer", pos + 1)
        opt = lambda t, n: None if t is None else _ptr(t, n)
        _check(load().qd_qkv_proj_rope_cache_attention(
            self._h, _ptr(x, "x"), opt(norm_w, "norm_w"), eps, _ptr(w_qkv, "w_qkv"), opt(bias, "bias"),
            _ptr(qkv, "qkv"), _ptr(k_layer, "k_layer", False), _ptr(v_layer, "v_layer", False),
            _ptr(out, "out"), pos, max_seqlen, H, HEAD_DIM, _stream(stream)))

    def set_front_local(self, on: bool) -> None:
        """qd_ctx_set_front_local: every split computes its head's front end itself."""
        _check(load().qd_ctx_set_front_local(self._h, 1 if on else 0))

    def front_misses(self) -> int:
        """qd_ctx_front_misses: split workgroups of the one-launch front end +
        attention that computed their head's front end themselves (not forced)."""
        n = ctypes.c_ulonglong(0)
        _check(load().qd_ctx_front_misses(self._h, ctypes.byref(n)))
        return n.value

    def qkv_proj_rope_cache(self, x: torch.Tensor, norm_w, w_qkv: torch.Tensor, bias,
                            qkv: torch.Tensor, k_layer: torch.Tensor, v_layer: torch.Tensor,
                            pos: int, eps: float = 1e-6, max_seqlen: int | None = None,
                            stream=None) -> None:
        """[RMSNorm] + QKV GEMV ([out][in] weight) + bias + RoPE + cache append at pos."""
        H = self.num_heads
        hid = H * HEAD_DIM
        if x.numel() < hid or qkv.numel() < 3 * hid or w_qkv.numel() < 3 * hid * hid:
            raise ValueError("x needs H*128, qkv 3*H*128 and w_qkv 3*H*128*H*128 elements")
        if norm_w is not None and norm_w.numel() < hid:
            raise ValueError("norm_w needs H*128 elements")
        if bias is not None and bias.numel() < 3 * hid:
            raise ValueError("bias needs 3*H*128 elements")
        if max_seqlen is None:
            max_seqlen = self.max_seqlen
        if 0 <= pos < max_seqlen:
            self._check_cache(k_layer, "k_layer", pos + 1)
            self._check_cache(v_layer, "v_layer", pos + 1)
        opt = lambda t, n: None if t is None else _ptr(t, n)
        _check(load().qd_qkv_proj_rope_cache(self._h, _ptr(x, "x"), opt(norm_w, "norm_w"), eps,
                                             _ptr(w_qkv, "w_qkv"), opt(bias, "bias"),
                                             _ptr(qkv, "qkv"), _ptr(k_layer, "k_layer", False),
                                             _ptr(v_layer, "v_layer", False), pos, max_seqlen, H,
                                             HEAD_DIM, _stream(stream)))


def xcd_placement(count: int = 256) -> list:
    """qd_xcd_placement: the XCD each workgroup of one count-workgroup launch ran on."""
    buf = (ctypes.c_uint * count)()
    _check(load().qd_xcd_placement(buf, count))
    return list(buf)


def decode_attention_noalloc(q: torch.Tensor, k_layer: torch.Tensor, v_layer: torch.Tensor,
                             out: torch.Tensor, seqlen: int, num_heads: int,
                             kv_row_stride: int | None = None, kv_head_stride: int = HEAD_DIM,
                             stream=None) -> torch.Tensor:
    """qd_decode_attention_noalloc: Context.decode_attention without a context; the
    split partials live in the library's static per-GPU scratch (no allocation)."""
    row = num_heads * HEAD_DIM if kv_row_stride is None else kv_row_stride
    if q.numel() < num_heads * HEAD_DIM or out.numel() < num_heads * HEAD_DIM:
        raise ValueError("q and out need num_heads*128 elements")
    if seqlen >= 1:
        last = (seqlen - 1) * row + (num_heads - 1) * kv_head_stride + HEAD_DIM
        for t, name in ((k_layer, "k_layer"), (v_layer, "v_layer")):
            if t.numel() < last:
                raise ValueError(f"{name} holds {t.numel()} elements; {seqlen} rows need {last}")
    _check(load().qd_decode_attention_noalloc(_ptr(q, "q"), _ptr(k_layer, "k_layer", False),
                                              _ptr(v_layer, "v_layer", False), _ptr(out, "out"),
                                              seqlen, num_heads, HEAD_DIM, row, kv_head_stride,
                                              _stream(stream)))
    return out


# ---------------------------------------------------------------- decode.h

def proj_residual(x: torch.Tensor, w: torch.Tensor, residual: torch.Tensor, out: torch.Tensor,
                  n_out: int, k_in: int, stream=None) -> torch.Tensor:
    """out[n] = half(residual[n] + half(W[n] . x)); W is [n_out][k_in]."""
    if x.numel() < k_in or w.numel() < n_out * k_in or residual.numel() < n_out or out.numel() < n_out:
        raise ValueError("x needs k_in, w n_out*k_in, residual and out n_out elements")
    _check(load().qd_proj_residual(_ptr(x, "x"), _ptr(w, "w"), _ptr(residual, "residual"),
                                   _ptr(out, "out"), n_out, k_in, _stream(stream)))
    return out


def gemm_nt(x: torch.Tensor, w: torch.Tensor, y: torch.Tensor, m: int, n: int, k: int,
            residual: torch.Tensor | None = None, mode: int = GEMM_EXACT, ldx: int | None = None,
            ldy: int | None = None, stream=None) -> torch.Tensor:
    """y[i][j] = half(sum_k x[i][k] w[j][k]) (+ residual: half(r + half(sum))) for i < m,
    j < n; w is [n][k]; x rows ldx (default k) and y rows ldy (default n) apart."""
    ldx = k if ldx is None else ldx
    ldy = n if ldy is None else ldy
    if x.numel() < (m - 1) * ldx + k or w.numel() < n * k or y.numel() < (m - 1) * ldy + n:
        raise ValueError("x, w or y too small for m, n, k and the strides")
    _check(load().qd_gemm_nt(_ptr(x, "x"), ldx, _ptr(w, "w"),
                             None if residual is None else _ptr(residual, "residual"), _ptr(y, "y"),
                             ldy, m, n, k, mode, _stream(stream)))
    return y


def gemm_swiglu(x: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor, act: torch.Tensor, m: int,
                n: int, k: int, ldx: int | None = None, ldy: int | None = None,
                stream=None) -> torch.Tensor:
    """act[i][j] = half(g * silu(u)), g = half(x[i] . w1[j]), u = half(x[i] . w2[j]), on the
    matrix cores (qd_gemm_swiglu); w1, w2 [n][k]; x rows ldx and act rows ldy apart."""
    ldx = k if ldx is None else ldx
    ldy = n if ldy is None else ldy
    if (x.numel() < (m - 1) * ldx + k or w1.numel() < n * k or w2.numel() < n * k
            or act.numel() < (m - 1) * ldy + n):
        raise ValueError("x, w1, w2 or act too small for m, n, k and the strides")
    _check(load().qd_gemm_swiglu(_ptr(x, "x"), ldx, _ptr(w1, "w1"), _ptr(w2, "w2"), _ptr(act, "act"),
                                 ldy, m, n, k, _stream(stream)))
    return act


def ffn_up_swiglu(x: torch.Tensor, norm_w: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor,
                  act: torch.Tensor, hidden: int, inter: int, eps: float = 1e-6,
                  stream=None) -> torch.Tensor:
    """act[i] = half(g * silu(u)) with g, u the W1 / W2 rows times RMSNorm(x) * norm_w."""
    if (x.numel() < hidden or norm_w.numel() < hidden or w1.numel() < inter * hidden
            or w2.numel() < inter * hidden or act.numel() < inter):
        raise ValueError("buffer smaller than hidden / inter imply")
    _check(load().qd_ffn_up_swiglu(_ptr(x, "x"), _ptr(norm_w, "norm_w"), eps, _ptr(w1, "w1"),
                                   _ptr(w2, "w2"), _ptr(act, "act"), hidden, inter,
                                   _stream(stream)))
    return act


def lm_head_workspace_bytes(vocab: int) -> int:
    return int(load().qd_lm_head_workspace_bytes(vocab))


def lm_head_argmax(x: torch.Tensor, norm_w: torch.Tensor, w: torch.Tensor, logits: torch.Tensor,
                   vocab: int, hidden: int, workspace: torch.Tensor, token: torch.Tensor,
                   eps: float = 1e-6, stream=None) -> None:
    """logits = half(W . RMSNorm(x) * norm_w); token[0] = argmax (lowest index on ties)."""
    if x.numel() < hidden or norm_w.numel() < hidden or w.numel() < vocab * hidden or logits.numel() < vocab:
        raise ValueError("buffer smaller than vocab / hidden imply")
    if token.dtype != torch.int32 or not token.is_cuda or workspace.device.type != "cuda":
        raise TypeError("token must be a GPU int32 tensor and workspace a GPU tensor")
    ws = workspace.numel() * workspace.element_size()
    _check(load().qd_lm_head_argmax(_ptr(x, "x"), _ptr(norm_w, "norm_w"), eps, _ptr(w, "w"),
                                    _ptr(logits, "logits"), vocab, hidden,
                                    ctypes.c_void_p(workspace.data_ptr()), ws,
                                    ctypes.c_void_p(token.data_ptr()), _stream(stream)))


# ---------------------------------------------------------------- engine.h

def model_cfg(**kw) -> ModelCfg:
    d = dict(QWEN_1_8B)
    d.update(kw)
    return ModelCfg(*(d[f] for f, _ in ModelCfg._fields_))


def model_image_bytes(cfg: ModelCfg) -> int:
    n = load().qd_model_image_bytes(ctypes.byref(cfg))
    if n < 0:
        raise ValueError(f"invalid model configuration {cfg.as_dict()}")
    return int(n)


def random_model_image(cfg: ModelCfg, seed: int, std: float = 0.02, nthreads: int = 8) -> np.ndarray:
    """A complete .bin image (uint8 array) with qd_model_fill_random's weights."""
    img = np.empty(model_image_bytes(cfg), np.uint8)
    _check(load().qd_model_fill_random(img.ctypes.data_as(ctypes.c_void_p), img.size,
                                       ctypes.byref(cfg), seed, std, nthreads))
    return img


def write_random_model(path: str, cfg: ModelCfg, seed: int, std: float = 0.02) -> None:
    _check(load().qd_model_write_random(path.encode(), ctypes.byref(cfg), seed, std))


class Engine:
    """The greedy decode engine (qd_engine) on the current device."""

    def __init__(self, path: str | None = None, image: np.ndarray | None = None):
        L = load()
        h = ctypes.c_void_p()
        if (path is None) == (image is None):
            raise ValueError("give exactly one of path and image")
        if path is not None:
            _check(L.qd_engine_create(path.encode(), ctypes.byref(h)))
        else:
            img = np.ascontiguousarray(image).view(np.uint8)
            _check(L.qd_engine_create_from_image(img.ctypes.data_as(ctypes.c_void_p), img.size,
                                                 ctypes.byref(h)))
        self._h = h
        c = ModelCfg()
        _check(L.qd_engine_config(h, ctypes.byref(c)))
        self.cfg = c

    def close(self) -> None:
        if getattr(self, "_h", None):
            load().qd_engine_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def reset(self) -> None:
        _check(load().qd_engine_reset(self._h))

    def set_prefill_mode(self, mode: int) -> None:
        """GEMM_EXACT (default; bit-identical to token-by-token decode) or GEMM_MFMA."""
        _check(load().qd_engine_set_prefill_mode(self._h, mode))

    def prefill(self, tokens, pos: int = 0) -> int:
        t = (ctypes.c_int * len(tokens))(*tokens)
        p = ctypes.c_int(pos)
        _check(load().qd_engine_prefill(self._h, t, len(tokens), ctypes.byref(p)))
        return p.value

    def step(self, token: int, pos: int) -> int:
        n = ctypes.c_int()
        _check(load().qd_engine_step(self._h, token, pos, ctypes.byref(n)))
        return n.value

    def logits(self) -> np.ndarray:
        out = np.empty(self.cfg.vocab_size, np.float16)
        _check(load().qd_engine_logits(self._h, out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16))))
        return out

    def kv_rows(self, layer: int, pos0: int, n: int):
        """qd_engine_kv_rows: (K, V) rows [pos0, pos0 + n) of `layer`, fp16 [n][hidden]."""
        k = np.empty((n, self.cfg.hidden_size), np.float16)
        v = np.empty_like(k)
        p = ctypes.POINTER(ctypes.c_uint16)
        _check(load().qd_engine_kv_rows(self._h, layer, pos0, n, k.ctypes.data_as(p), v.ctypes.data_as(p)))
        return k, v

    def generate(self, prompt, max_new: int, stop_at_eos: bool = True) -> list:
        p = (ctypes.c_int * len(prompt))(*prompt)
        out = (ctypes.c_int * max(1, max_new))()
        n = ctypes.c_int()
        _check(load().qd_engine_generate(self._h, p, len(prompt), max_new, int(stop_at_eos), out,
                                         ctypes.byref(n)))
        return list(out[:n.value])


def version() -> str:
    return load().qd_version().decode()


def max_splits() -> int:
    return load().qd_max_splits()
