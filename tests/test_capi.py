"""CPU checks of the C ABI: the in-tree library loads, exports every function that
include/lbw_attn.h declares, and the ctypes structs match the header's field lists.
No compute call is made (no GPU here)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "lbw_attn.h")


def _header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(lbw_[a-z0-9_]+)\s*\(", text)))


def _lib_path():
    from lbw_amd import _lib
    return _lib.LIB_PATH


def test_header_declares_expected_entry_points():
    from lbw_amd import _lib
    assert _header_functions() == sorted(_lib.EXPORTS)


def test_library_exports_every_declared_symbol():
    path = _lib_path()
    if not os.path.exists(path):
        pytest.fail(f"{path} not built: run __graft_entry__.build()")
    lib = ctypes.CDLL(path)
    for name in _header_functions():
        assert hasattr(lib, name), name
    lib.lbw_abi_version.restype = ctypes.c_int
    from lbw_amd import _lib
    assert lib.lbw_abi_version() == _lib.ABI_VERSION == 4


def _header_struct_fields(name):
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    m = re.search(r"typedef struct %s \{(.*?)\} %s;" % (name, name), text, flags=re.S)
    assert m, name
    fields = []
    for decl in m.group(1).split(";"):
        decl = decl.strip()
        if not decl:
            continue
        decl = re.sub(r"\[[^\]]*\]", "", decl)
        names = decl.split(None, 1)[1] if " " in decl else decl
        for n in names.split(","):
            fields.append(n.replace("*", "").strip().split()[-1])
    return fields


@pytest.mark.parametrize("cname,pyname", [("lbw_kv_segment", "KvSegment"),
                                          ("lbw_attn_params", "AttnParams"),
                                          ("lbw_qk_norm_rope_params", "QkNormRopeParams")])
def test_ctypes_structs_match_header(cname, pyname):
    from lbw_amd import _lib
    py = [f[0] for f in getattr(_lib, pyname)._fields_]
    assert py == _header_struct_fields(cname)


_CTYPE = {"int32_t": ctypes.c_int32, "int64_t": ctypes.c_int64, "float": ctypes.c_float}


def _header_struct(name, known):
    """A ctypes struct built from the header's own declaration of `name` (pointers as
    c_void_p, `T x[N]` as arrays, nested structs from `known`), for layout comparisons."""
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    consts = dict(re.findall(r"#define (LBW_[A-Z_]+) (\d+)\b", text))
    m = re.search(r"typedef struct %s \{(.*?)\} %s;" % (name, name), text, flags=re.S)
    assert m, name
    fields = []
    for decl in m.group(1).split(";"):
        decl = " ".join(decl.split())
        if not decl:
            continue
        decl = decl.replace("const ", "")
        base, rest = decl.split(" ", 1)
        for item in rest.split(","):
            item = item.strip()
            ptr = base.endswith("*") or item.startswith("*")
            item = item.lstrip("*").strip()
            arr = re.match(r"(\w+)\[(\w+)\]", item)
            fname = arr.group(1) if arr else item
            t = ctypes.c_void_p if ptr else (known[base] if base in known else _CTYPE[base])
            if arr:
                n = arr.group(2)
                t = t * int(consts.get(n, n))
            fields.append((fname, t))
    return type(name, (ctypes.Structure,), {"_fields_": fields})


GUIDE = os.path.join(ROOT, "INTEGRATION.md")   # the integration guide a maintainer follows


def _integration_stub():
    """The Seg and Params classes of the integration guide's ctypes stub, executed as written."""
    import ast
    text = open(GUIDE).read()
    blocks = re.findall(r"```python\n(.*?)```", text, flags=re.S)
    block = next(b for b in blocks if "class Params(ctypes.Structure)" in b)
    tree = ast.parse(block)
    classes = [n for n in tree.body if isinstance(n, ast.ClassDef)]
    ns = {"ctypes": ctypes}
    exec(compile(ast.Module(body=classes, type_ignores=[]), GUIDE, "exec"), ns)
    return ns["Seg"], ns["Params"]


def _layout(struct):
    return [(f[0], getattr(struct, f[0]).offset, getattr(struct, f[0]).size)
            for f in struct._fields_]


def test_integration_stub_matches_header():
    """The binding the integration guide shows a maintainer has every field of the header's structs,
    in order, at the same offsets and sizes: a stub missing a trailing field would let the
    library read past the caller's struct."""
    seg_h = _header_struct("lbw_kv_segment", {})
    par_h = _header_struct("lbw_attn_params", {"lbw_kv_segment": seg_h})
    seg_d, par_d = _integration_stub()
    assert _layout(seg_d) == _layout(seg_h)
    assert _layout(par_d) == _layout(par_h)
    assert ctypes.sizeof(par_d) == ctypes.sizeof(par_h)
    from lbw_amd import _lib
    assert _layout(_lib.AttnParams) == _layout(par_h)
    assert "lbw_abi_version() == %d" % _lib.ABI_VERSION in open(GUIDE).read()


def test_entry_points_reject_bad_arguments_without_gpu():
    """Validation runs before any HIP call: bad params return LBW_ERR_* with a message."""
    from lbw_amd import _lib
    lib = ctypes.CDLL(_lib_path())
    _lib._declare(lib)
    p = _lib.AttnParams()
    p.batch, p.heads, p.head_dim, p.lq = 1, 1, 64, 4
    assert lib.lbw_attention_fwd(ctypes.byref(p), None, 0, None) == 2
    assert b"head_dim" in lib.lbw_last_error()
    p.head_dim = 128
    p.n_segments = 0
    assert lib.lbw_attention_fwd(ctypes.byref(p), None, 0, None) == 1
    assert lib.lbw_attention_workspace_size(ctypes.byref(p)) == 0
    assert lib.lbw_kv_quant_fp8(None, 1, 10, 1, 128, 0, 0, 0, None, None, 32, None) == 2


def test_qk_norm_rope_layout_checks_without_gpu():
    """out_layout validation (rows / d-major) runs before any HIP call."""
    from lbw_amd import _lib
    lib = ctypes.CDLL(_lib_path())
    _lib._declare(lib)
    fake = 1 << 20                                   # aligned, never dereferenced
    p = _lib.QkNormRopeParams()
    p.tokens, p.dim, p.heads, p.s0, p.s1 = 16, 512, 4, 22, 21
    p.q = p.wq = p.q_out = fake
    p.q_stride = 512
    p.out_layout = 7
    assert lib.lbw_qk_norm_rope(ctypes.byref(p), None) == 1
    assert b"out_layout" in lib.lbw_last_error()
    p.out_layout = 1                                 # d-major: the d stride must cover the tokens
    p.q_out_stride = 8
    assert lib.lbw_qk_norm_rope(ctypes.byref(p), None) == 1
    assert b"d stride" in lib.lbw_last_error()
    p.dim, p.heads = 6144, 48                        # two rows of more than 5120 features
    assert lib.lbw_qk_norm_rope(ctypes.byref(p), None) == 2
    assert b"d-major" in lib.lbw_last_error()
    p.dim, p.heads, p.out_layout, p.q_out_stride = 512, 4, 0, 512
    p.q_out = fake + 2                               # rows layout needs 16-byte aligned outputs
    assert lib.lbw_qk_norm_rope(ctypes.byref(p), None) == 1


def _split_count(H, LQ, LK):
    """KV splits the library plans for q [1, LQ, H, 128] over one LK-key segment, read back
    from the workspace size (splits x rows x (D + 2) fp32; 0 for a single pass). Host-only."""
    from lbw_amd import _lib
    lib = _lib.load()
    p = _lib.AttnParams()
    p.batch, p.heads, p.head_dim, p.lq = 1, H, 128, LQ
    p.q = p.out = 256
    p.q_stride_b = p.o_stride_b = LQ * H * 128
    p.q_stride_l = p.o_stride_l = H * 128
    p.q_stride_h = p.o_stride_h = 128
    p.n_segments = 1
    s = p.seg[0]
    s.k = s.v = 256
    s.len = LK
    s.k_stride_b = s.v_stride_b = LK * H * 128
    s.k_stride_l = s.v_stride_l = H * 128
    s.k_stride_h = s.v_stride_h = 128
    p.kv_lo, p.kv_hi = 0, -1
    n = lib.lbw_attention_workspace_size(ctypes.byref(p))
    return n // (LQ * H * 130 * 4)


def test_workspace_layout_without_gpu():
    """Workspace = split partials (splits x rows x (D + 2) fp32) rounded up to 256 bytes, then
    the counters: 8 work-queue counters and, for a split plan (its pieces merge in the kernel),
    one arrival counter per (batch, head, 256-query tile), rounded up to 256 bytes (at least
    256); a single-pass plan needs only the queue counters."""
    from lbw_amd import _lib
    lib = _lib.load()
    for H, LQ, LK in [(2, 256, 1024), (40, 3600, 46800), (40, 4680, 32760), (12, 4680, 14040)]:
        p = _lib.AttnParams()
        p.batch, p.heads, p.head_dim, p.lq = 1, H, 128, LQ
        p.q = p.out = 256
        p.q_stride_b = p.o_stride_b = LQ * H * 128
        p.q_stride_l = p.o_stride_l = H * 128
        p.q_stride_h = p.o_stride_h = 128
        p.n_segments = 1
        sg = p.seg[0]
        sg.k = sg.v = 256
        sg.len = LK
        sg.k_stride_b = sg.v_stride_b = LK * H * 128
        sg.k_stride_l = sg.v_stride_l = H * 128
        sg.k_stride_h = sg.v_stride_h = 128
        p.kv_lo, p.kv_hi = 0, -1
        n = lib.lbw_attention_workspace_size(ctypes.byref(p))
        splits = _split_count(H, LQ, LK)
        parts = splits * LQ * H * 130 * 4 if splits > 1 else 0
        units = H * ((LQ + 255) // 256)
        cnt = 4 * (8 + (units if splits > 1 else 0))
        assert n == ((parts + 255) // 256) * 256 + max(256, (cnt + 255) // 256 * 256), \
            (H, LQ, LK, n, splits)


def test_segment_length_limit_without_gpu():
    """Segments longer than 2^30 keys are refused before any HIP call (32-bit key indices)."""
    from lbw_amd import _lib
    lib = _lib.load()
    p = _lib.AttnParams()
    p.batch, p.heads, p.head_dim, p.lq = 1, 1, 128, 4
    p.q = p.out = 256
    p.q_stride_b = p.o_stride_b = 4 * 128
    p.q_stride_l = p.o_stride_l = 128
    p.q_stride_h = p.o_stride_h = 128
    p.n_segments = 1
    s = p.seg[0]
    s.k = s.v = 256
    s.len = (1 << 30) + 1
    s.k_stride_l = s.v_stride_l = 128
    s.k_stride_b = s.v_stride_b = s.len * 128
    s.k_stride_h = s.v_stride_h = 128
    p.kv_lo, p.kv_hi = 0, -1
    assert lib.lbw_attention_fwd(ctypes.byref(p), None, 0, None) == 2
    assert b"2^30" in lib.lbw_last_error()


def test_split_plan_for_the_measured_shapes():
    """The split heuristic's choices for the shapes it was fitted on (gfx950, 256 CUs): 14B
    720p (3 splits), 14B 480p and 1.3B 480p 3-frame chunks (single pass), 1.3B one frame (3)."""
    assert _split_count(40, 3600, 46800) == 3
    assert _split_count(40, 4680, 32760) == 0
    assert _split_count(12, 4680, 14040) == 0
    assert _split_count(12, 1560, 4680) == 3


def test_prescaled_pairing_is_exactly_one_in_fp32():
    """The host (capi.hip: scale_log2 = scale * 1.4426950408889634f in fp32) takes the folded
    kernel when that product is exactly 1.0f: PRESCALED_SOFTMAX_SCALE must round so, and
    prescaled_q_scale(D) * PRESCALED_SOFTMAX_SCALE must be the usual 1/sqrt(D)."""
    import math
    import numpy as np
    from lbw_amd import PRESCALED_SOFTMAX_SCALE, prescaled_q_scale
    assert np.float32(PRESCALED_SOFTMAX_SCALE) * np.float32(1.4426950408889634) == np.float32(1.0)
    # one ulp either way is the plain kernel
    up = np.nextafter(np.float32(PRESCALED_SOFTMAX_SCALE), np.float32(1))
    assert up * np.float32(1.4426950408889634) != np.float32(1.0)
    for d in (64, 128):
        assert math.isclose(prescaled_q_scale(d) * PRESCALED_SOFTMAX_SCALE, 1 / math.sqrt(d),
                            rel_tol=1e-15)


def test_torch_op_set_registers_with_shapes():
    """liblbw_torch.so registers the C ABI as torch.ops.lbw; its Meta kernels give every
    functional op's output shape and dtype (what tracing under torch.compile needs), with no
    GPU and no launch."""
    import torch
    from lbw_amd import _lib
    ops = _lib.ops()
    for name in ("attention", "attention_out", "cross_attention", "cross_attention_out",
                 "attention_fp8kv", "attention_fp8kv_out", "attention_partial",
                 "attention_merge", "attention_merge_out", "qk_norm_rope_", "kv_quant_fp8_"):
        assert hasattr(ops, name), name
    q = torch.empty(2, 10, 3, 128, dtype=torch.bfloat16, device="meta")
    k = torch.empty(2, 70, 3, 128, dtype=torch.bfloat16, device="meta")
    o = ops.attention(q, [k, k], [k, k], 0, -1, None, 0.0, 0, False)
    assert o.shape == q.shape and o.dtype == torch.bfloat16
    assert ops.attention(q, [k], [k], 0, -1, None, 0.0, 0, True).dtype == torch.float32
    assert ops.cross_attention(q, k, k, None, -1, 0, -1, 0.0, False).shape == q.shape
    po, pm, pl = ops.attention_partial(q, [k], [k], 0, -1, 0.0)
    assert po.shape == (2, 3, 10, 128) and pm.shape == (2, 3, 10) and pl.dtype == torch.float32
    assert ops.attention_merge([po, po], [pm, pm], [pl, pl]).shape == q.shape
    c8 = torch.empty(2, 70, 3, 128, dtype=torch.uint8, device="meta")
    s8 = torch.empty(2, 3, 2, dtype=torch.float32, device="meta")
    assert ops.attention_fp8kv(q, [c8], [c8], [s8], [s8], 0, -1, 0.0, 0, False).shape == q.shape
    # the window as device tensors (one-element int64, read by the kernel)
    lo = torch.empty(1, dtype=torch.int64, device="meta")
    assert ops.attention(q, [k], [k], 0, -1, None, 0.0, 0, False, lo, lo).shape == q.shape
    assert ops.attention(q, [k], [k], kv_lo_dev=lo, kv_hi_dev=lo).shape == q.shape
    assert ops.attention_partial(q, [k], [k], 0, -1, 0.0, lo, lo)[0].shape == (2, 3, 10, 128)
    assert ops.attention_fp8kv(q, [c8], [c8], [s8], [s8], kv_hi_dev=lo).shape == q.shape
