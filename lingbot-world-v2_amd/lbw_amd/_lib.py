"""Loaders of the in-tree libraries: liblbw_attn.so (the C ABI declared in
include/lbw_attn.h, with a ctypes binding for direct ABI use) and liblbw_torch.so, which
registers that ABI as the torch op set ``torch.ops.lbw`` that lbw_amd calls.

Both are built in-tree (``make -C lingbot-world-v2_amd/csrc``) and loaded from this directory.
There is no fallback: if a library is missing or a call fails, a RuntimeError says so.
"""
from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liblbw_attn.so")
OPS_PATH = os.path.join(_HERE, "liblbw_torch.so")

MAX_KV_SEGMENTS = 8
FP8_BLOCK = 64
ABI_VERSION = 4

OUT_BF16 = 0
OUT_FP32 = 1

LBW_OK = 0
_ERR_NAMES = {1: "invalid argument", 2: "unsupported", 3: "HIP error", 4: "workspace"}


class KvSegment(ctypes.Structure):
    _fields_ = [
        ("k", ctypes.c_void_p), ("v", ctypes.c_void_p), ("len", ctypes.c_int64),
        ("k_stride_b", ctypes.c_int64), ("k_stride_l", ctypes.c_int64), ("k_stride_h", ctypes.c_int64),
        ("v_stride_b", ctypes.c_int64), ("v_stride_l", ctypes.c_int64), ("v_stride_h", ctypes.c_int64),
        ("k_scale", ctypes.c_void_p), ("v_scale", ctypes.c_void_p),
        ("k_stride_d", ctypes.c_int64),
    ]


class AttnParams(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_int32), ("heads", ctypes.c_int32), ("head_dim", ctypes.c_int32),
        ("lq", ctypes.c_int32),
        ("q", ctypes.c_void_p),
        ("q_stride_b", ctypes.c_int64), ("q_stride_l", ctypes.c_int64), ("q_stride_h", ctypes.c_int64),
        ("out", ctypes.c_void_p),
        ("o_stride_b", ctypes.c_int64), ("o_stride_l", ctypes.c_int64), ("o_stride_h", ctypes.c_int64),
        ("n_segments", ctypes.c_int32),
        ("seg", KvSegment * MAX_KV_SEGMENTS),
        ("kv_lo", ctypes.c_int64), ("kv_hi", ctypes.c_int64),
        ("k_lens", ctypes.c_void_p),
        ("softmax_scale", ctypes.c_float),
        ("num_splits", ctypes.c_int32),
        ("part_o", ctypes.c_void_p), ("part_m", ctypes.c_void_p), ("part_l", ctypes.c_void_p),
        ("out_dtype", ctypes.c_int32),
        ("kv_lo_dev", ctypes.c_void_p), ("kv_hi_dev", ctypes.c_void_p),
        ("key_bias", ctypes.c_void_p),
    ]


class QkNormRopeParams(ctypes.Structure):
    _fields_ = [
        ("tokens", ctypes.c_int32), ("dim", ctypes.c_int32), ("heads", ctypes.c_int32),
        ("q", ctypes.c_void_p), ("q_stride", ctypes.c_int64),
        ("k", ctypes.c_void_p), ("k_stride", ctypes.c_int64),
        ("bq", ctypes.c_void_p), ("bk", ctypes.c_void_p),
        ("wq", ctypes.c_void_p), ("wk", ctypes.c_void_p),
        ("eps", ctypes.c_float),
        ("rope", ctypes.c_void_p),
        ("grid_f", ctypes.c_int32), ("grid_h", ctypes.c_int32), ("grid_w", ctypes.c_int32),
        ("s0", ctypes.c_int32), ("s1", ctypes.c_int32),
        ("q_out", ctypes.c_void_p), ("q_out_stride", ctypes.c_int64),
        ("k_out", ctypes.c_void_p), ("k_out_stride", ctypes.c_int64),
        ("q_out_scale", ctypes.c_float), ("k_out_scale", ctypes.c_float),
        ("v", ctypes.c_void_p), ("v_stride", ctypes.c_int64),
        ("v_out", ctypes.c_void_p), ("v_out_stride", ctypes.c_int64),
        ("out_layout", ctypes.c_int32),
    ]


EXPORTS = (
    "lbw_attention_workspace_size", "lbw_attention_fp8kv_workspace_size", "lbw_attention_fwd",
    "lbw_cross_attention_fwd",
    "lbw_cross_attention_dedup_fwd",
    "lbw_attention_fwd_fp8kv", "lbw_attention_fwd_noalloc", "lbw_attn_merge",
    "lbw_attn_merge_partials", "lbw_qk_norm_rope",
    "lbw_kv_quant_fp8",
    "lbw_last_error", "lbw_abi_version",
)

_lock = threading.Lock()
_lib = None


def _declare(lib):
    P = ctypes.POINTER
    vp, i32, i64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64
    lib.lbw_attention_workspace_size.argtypes = [P(AttnParams)]
    lib.lbw_attention_workspace_size.restype = ctypes.c_size_t
    lib.lbw_attention_fp8kv_workspace_size.argtypes = [P(AttnParams)]
    lib.lbw_attention_fp8kv_workspace_size.restype = ctypes.c_size_t
    lib.lbw_attention_fwd.argtypes = [P(AttnParams), vp, ctypes.c_size_t, vp]
    lib.lbw_attention_fwd.restype = ctypes.c_int
    lib.lbw_cross_attention_fwd.argtypes = [P(AttnParams), vp]
    lib.lbw_cross_attention_fwd.restype = ctypes.c_int
    lib.lbw_cross_attention_dedup_fwd.argtypes = [P(AttnParams), i64, vp]
    lib.lbw_cross_attention_dedup_fwd.restype = ctypes.c_int
    lib.lbw_attention_fwd_fp8kv.argtypes = [P(AttnParams), vp, ctypes.c_size_t, vp]
    lib.lbw_attention_fwd_fp8kv.restype = ctypes.c_int
    lib.lbw_attention_fwd_noalloc.argtypes = [P(AttnParams), vp]
    lib.lbw_attention_fwd_noalloc.restype = ctypes.c_int
    lib.lbw_attn_merge.argtypes = [i32, P(vp), P(vp), P(vp), i32, i32, i32, i32, vp, i64, i64,
                                   i64, vp]
    lib.lbw_attn_merge.restype = ctypes.c_int
    lib.lbw_attn_merge_partials.argtypes = [i32, P(vp), P(vp), P(vp), i32, i32, i32, i32, vp, vp,
                                            vp, vp]
    lib.lbw_attn_merge_partials.restype = ctypes.c_int
    lib.lbw_qk_norm_rope.argtypes = [P(QkNormRopeParams), vp]
    lib.lbw_qk_norm_rope.restype = ctypes.c_int
    lib.lbw_kv_quant_fp8.argtypes = [vp, i32, i64, i32, i32, i64, i64, i64, vp, vp, i32, vp]
    lib.lbw_kv_quant_fp8.restype = ctypes.c_int
    lib.lbw_last_error.argtypes = []
    lib.lbw_last_error.restype = ctypes.c_char_p
    lib.lbw_abi_version.argtypes = []
    lib.lbw_abi_version.restype = ctypes.c_int


def load():
    """Load (once) and return the library handle. Raises RuntimeError when it is absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `make -C lingbot-world-v2_amd/csrc` "
                "(or __graft_entry__.build()). The attention path has no CPU fallback.")
        # torch first: its libamdhip64 (same soname) then serves the library's HIP calls,
        # so there is exactly one HIP runtime in the process.
        import torch  # noqa: F401
        lib = ctypes.CDLL(LIB_PATH)
        _declare(lib)
        if lib.lbw_abi_version() != ABI_VERSION:
            raise RuntimeError(f"liblbw_attn ABI {lib.lbw_abi_version()} != {ABI_VERSION}")
        _lib = lib
        return lib


_ops = None


def ops():
    """``torch.ops.lbw``, loading liblbw_torch.so (and the C ABI library under it) once.
    Raises RuntimeError when either library is missing."""
    global _ops
    if _ops is not None:
        return _ops
    load()
    with _lock:
        if _ops is None:
            if not os.path.exists(OPS_PATH):
                raise RuntimeError(
                    f"{OPS_PATH} is missing: build it with `make -C lingbot-world-v2_amd/csrc` "
                    "(or __graft_entry__.build()). The attention path has no CPU fallback.")
            import torch
            torch.ops.load_library(OPS_PATH)
            _ops = torch.ops.lbw
    return _ops


def attn_params(q, out, segments, kv_lo=None, kv_hi=None, k_lens=None, softmax_scale=None,
                num_splits=0, parts=None) -> AttnParams:
    """``lbw_attn_params`` for direct calls of the C ABI: q ``[B, Lq, N, D]``, out of q's shape
    (bf16 or fp32) or None, segments ``[(k, v)]`` or ``[(k, v, k_scale, v_scale)]`` (fp8),
    optional partial outputs ``(O, m, l)``. ``kv_lo`` / ``kv_hi`` may be one-element int64
    tensors on q's device (read by the kernel on the device)."""
    import torch
    p = AttnParams()
    B, Lq, H, D = q.shape
    p.batch, p.heads, p.head_dim, p.lq = B, H, D, Lq
    p.q = q.data_ptr()
    p.q_stride_b, p.q_stride_l, p.q_stride_h = q.stride(0), q.stride(1), q.stride(2)
    if out is not None:
        p.out = out.data_ptr()
        p.o_stride_b, p.o_stride_l, p.o_stride_h = out.stride(0), out.stride(1), out.stride(2)
        p.out_dtype = OUT_FP32 if out.dtype == torch.float32 else OUT_BF16
    if not 1 <= len(segments) <= MAX_KV_SEGMENTS:
        raise ValueError(f"{len(segments)} KV segments: 1..{MAX_KV_SEGMENTS} supported")
    p.n_segments = len(segments)
    for i, sg in enumerate(segments):
        k, v = sg[0], sg[1]
        seg = p.seg[i]
        seg.k, seg.v, seg.len = k.data_ptr(), v.data_ptr(), k.shape[1]
        seg.k_stride_b, seg.k_stride_l, seg.k_stride_h = k.stride(0), k.stride(1), k.stride(2)
        if k.stride(3) != 1:   # d-major K: [B, L, N, D] view with token stride 1
            seg.k_stride_d = k.stride(3)
        seg.v_stride_b, seg.v_stride_l, seg.v_stride_h = v.stride(0), v.stride(1), v.stride(2)
        if len(sg) > 2:
            seg.k_scale, seg.v_scale = sg[2].data_ptr(), sg[3].data_ptr()
    p.kv_lo, p.kv_hi = 0, -1
    for name, b in (("lo", kv_lo), ("hi", kv_hi)):
        if b is None:
            continue
        if torch.is_tensor(b) and b.device.type != "cpu":
            if b.dtype != torch.int64 or b.numel() != 1:
                raise ValueError(f"kv_{name} on the device must be a one-element int64 tensor")
            setattr(p, f"kv_{name}_dev", b.data_ptr())
        else:
            setattr(p, f"kv_{name}", int(b))
    p.k_lens = k_lens.data_ptr() if k_lens is not None else None
    p.softmax_scale = 0.0 if softmax_scale is None else float(softmax_scale)
    p.num_splits = int(num_splits)
    if parts is not None:
        p.part_o, p.part_m, p.part_l = (t.data_ptr() for t in parts)
    return p


def check(rc: int, what: str):
    if rc != LBW_OK:
        msg = load().lbw_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed ({_ERR_NAMES.get(rc, rc)}): {msg}")


def stream_ptr(device=None) -> int:
    """The current torch stream on `device` as a hipStream_t address."""
    import torch
    return torch.cuda.current_stream(device).cuda_stream
