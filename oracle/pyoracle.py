"""ctypes wrapper over oracle/liboracle.so (the C restatement of the q36 MoE
arithmetic).  TEST INFRASTRUCTURE ONLY -- see oracle/q36moe_oracle.c."""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_LIB_PATH = os.path.join(HERE, "_ref", "libref_dequant.so")

_lib = None


def build(ref=True):
    """Compile liboracle.so (and _ref/ when the reference tree is present)."""
    target = ["all"] if ref else ["liboracle.so"]
    subprocess.run(["make", "-s", "-C", HERE] + target, check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build(ref=False)
        L = ctypes.CDLL(LIB_PATH)
        vp, i, f = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
        L.or_e8m0.argtypes = [ctypes.c_uint8]
        L.or_e8m0.restype = ctypes.c_double
        L.or_e2m1.argtypes = [ctypes.c_uint8]
        L.or_e2m1.restype = ctypes.c_double
        L.or_e4m3_decode.argtypes = [ctypes.c_uint8]
        L.or_e4m3_decode.restype = ctypes.c_float
        L.or_e4m3_encode.argtypes = [ctypes.c_float]
        L.or_e4m3_encode.restype = ctypes.c_uint8
        L.or_quant_exp.argtypes = [ctypes.c_float]
        L.or_quant_exp.restype = ctypes.c_int
        L.or_deq_mxfp4_block.argtypes = [vp, vp]
        L.or_deq_mxfp4_row.argtypes = [vp, i, vp]
        L.or_quant_e4m3.argtypes = [vp, i, i, vp, vp]
        L.or_dequant_e4m3.argtypes = [vp, vp, i, i, vp]
        L.or_router_topk.argtypes = [vp, i, i, i, i, f, i, vp, vp]
        L.or_sort.argtypes = [vp, i, i, vp, vp, vp]
        L.or_gemv_mxfp4_f32.argtypes = [vp, i, i, vp, vp, vp]
        L.or_gemv_mxfp4_f32_mt.argtypes = [vp, i, i, vp, vp, vp, i]
        L.or_expert_h.argtypes = [vp, vp, i, i, vp, vp]
        L.or_expert_down.argtypes = [vp, i, i, vp, vp]
        L.or_moe_forward.argtypes = [vp, vp, vp, i, vp, i, i, f, i, vp, i, vp]
        L.or_moe_forward_f32.argtypes = [vp, vp, vp, i, vp, i, i, f, vp, i]
        L.or_f16_encode.argtypes = [ctypes.c_float]
        L.or_f16_encode.restype = ctypes.c_uint16
        L.or_f16_decode.argtypes = [ctypes.c_uint16]
        L.or_f16_decode.restype = ctypes.c_float
        L.or_deq_row.argtypes = [ctypes.c_uint32, vp, i, vp]
        L.or_requant_q8_row.argtypes = [vp, i, vp, vp]
        L.or_requant_q8.argtypes = [ctypes.c_uint32, vp, i, i, vp, vp]
        L.or_quant_q8b.argtypes = [vp, i, vp, vp]
        L.or_expert_down_q8.argtypes = [vp, vp, i, i, vp, vp]
        L.or_expert_h_q8.argtypes = [vp, vp, vp, vp, i, i, vp, vp]
        _lib = L
    return _lib


def _p(a):
    return ctypes.c_void_p(a.ctypes.data) if a is not None else None


class _W(ctypes.Structure):
    _fields_ = [("gate", ctypes.c_void_p), ("up", ctypes.c_void_p), ("down", ctypes.c_void_p),
                ("sh_gate", ctypes.c_void_p), ("sh_up", ctypes.c_void_p), ("sh_down", ctypes.c_void_p),
                ("n_expert", ctypes.c_int), ("d_model", ctypes.c_int), ("d_ff", ctypes.c_int),
                ("d_ff_sh", ctypes.c_int), ("down_q8", ctypes.c_void_p), ("down_q8d", ctypes.c_void_p),
                ("sh_gate_q8", ctypes.c_void_p), ("sh_up_q8", ctypes.c_void_p), ("sh_down_q8", ctypes.c_void_p),
                ("sh_gate_q8d", ctypes.c_void_p), ("sh_up_q8d", ctypes.c_void_p), ("sh_down_q8d", ctypes.c_void_p)]


def _wstruct(w):
    """w: gate/up (/down) GGUF MXFP4 blocks [E][M][K/32][17], optional
    sh_*; or down_q8 (int8 [E][D][FF]) + down_q8d (f16 bits [E][D][FF/32])
    for the q8_0-split routed down; sh_{gate,up,down}_q8 (int8) + _q8d (f16
    bits) for a q8_0-split shared expert."""
    keep = {}
    for k, v in w.items():
        if v is None:
            continue
        dt = np.int8 if k.endswith("_q8") else np.uint16 if k.endswith("_q8d") else np.uint8
        keep[k] = np.ascontiguousarray(v, dtype=dt)
    E, FF, nb, _ = keep["gate"].shape
    ffsh = keep["sh_gate"].shape[0] if "sh_gate" in keep else keep["sh_gate_q8"].shape[0] if "sh_gate_q8" in keep else 0
    s = _W(_p(keep["gate"]), _p(keep["up"]), _p(keep.get("down")),
           _p(keep.get("sh_gate")), _p(keep.get("sh_up")), _p(keep.get("sh_down")),
           E, nb * 32, FF, ffsh,
           _p(keep.get("down_q8")), _p(keep.get("down_q8d")),
           *[_p(keep.get(f"sh_{m}_q8")) for m in ("gate", "up", "down")],
           *[_p(keep.get(f"sh_{m}_q8d")) for m in ("gate", "up", "down")])
    return s, keep


# ---- scalar / block helpers ----
def e8m0(e):
    return lib().or_e8m0(e)


def e2m1(c):
    return lib().or_e2m1(c)


def e4m3_decode(b):
    return lib().or_e4m3_decode(b)


def e4m3_encode(v):
    return lib().or_e4m3_encode(float(v))


def e4m3_encode_array(v):
    v = np.ascontiguousarray(v, dtype=np.float32).reshape(-1)
    return np.array([lib().or_e4m3_encode(float(x)) for x in v], dtype=np.uint8)


def e4m3_decode_table():
    return np.array([lib().or_e4m3_decode(b) for b in range(256)], dtype=np.float32)


def quant_exp(a):
    return lib().or_quant_exp(float(a))


def deq_mxfp4_row(blocks):
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    n = blocks.size // 17 * 32
    out = np.empty(n, dtype=np.float32)
    lib().or_deq_mxfp4_row(_p(blocks), n, _p(out))
    return out


def quant_e4m3(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    T, K = x.shape
    xq = np.empty((T, K), dtype=np.uint8)
    xs = np.empty((T, K // 32), dtype=np.uint8)
    lib().or_quant_e4m3(_p(x), T, K, _p(xq), _p(xs))
    return xq, xs


def dequant_e4m3(xq, xs):
    xq = np.ascontiguousarray(xq, dtype=np.uint8)
    xs = np.ascontiguousarray(xs, dtype=np.uint8)
    T, K = xq.shape
    out = np.empty((T, K), dtype=np.float64)
    lib().or_dequant_e4m3(_p(xq), _p(xs), T, K, _p(out))
    return out


def router_topk(logits, k=8, scale=1.0, renorm=True, n_expert=None):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    T, ld = logits.shape
    E = n_expert or ld
    idx = np.empty((T, k), dtype=np.int32)
    wt = np.empty((T, k), dtype=np.float64)
    lib().or_router_topk(_p(logits), T, E, ld, k, scale, 1 if renorm else 0, _p(idx), _p(wt))
    return idx, wt


def sort_entries(idx, n_expert):
    idx = np.ascontiguousarray(idx, dtype=np.int32).reshape(-1)
    n = idx.size
    off = np.empty(n_expert + 1, dtype=np.int32)
    perm = np.empty(n, dtype=np.int32)
    pos = np.empty(n, dtype=np.int32)
    lib().or_sort(_p(idx), n, n_expert, _p(off), _p(perm), _p(pos))
    return off, perm, pos


def gemv_mxfp4(W, xq, xs, nthreads=1):
    W = np.ascontiguousarray(W, dtype=np.uint8)
    M, nb, _ = W.shape
    K = nb * 32
    xq = np.ascontiguousarray(xq, dtype=np.uint8).reshape(-1)
    xs = np.ascontiguousarray(xs, dtype=np.uint8).reshape(-1)
    y = np.empty(M, dtype=np.float32)
    if nthreads > 1:
        lib().or_gemv_mxfp4_f32_mt(_p(W), M, K, _p(xq), _p(xs), _p(y), nthreads)
    else:
        lib().or_gemv_mxfp4_f32(_p(W), M, K, _p(xq), _p(xs), _p(y))
    return y


def expert_h(gate_e, up_e, xd):
    """fp64 SwiGLU rows of one expert for a dequantised input row."""
    g = np.ascontiguousarray(gate_e, dtype=np.uint8)
    u = np.ascontiguousarray(up_e, dtype=np.uint8)
    xd = np.ascontiguousarray(xd, dtype=np.float64)
    FF, nb, _ = g.shape
    h = np.empty(FF, dtype=np.float64)
    lib().or_expert_h(_p(g), _p(u), nb * 32, FF, _p(xd), _p(h))
    return h


def expert_down(down_e, hd):
    d = np.ascontiguousarray(down_e, dtype=np.uint8)
    hd = np.ascontiguousarray(hd, dtype=np.float64)
    D, nb, _ = d.shape
    y = np.empty(D, dtype=np.float64)
    lib().or_expert_down(_p(d), D, nb * 32, _p(hd), _p(y))
    return y


# ---- Q8 formats ----
def f16_encode(v):
    return lib().or_f16_encode(float(v))


def f16_decode(h):
    return lib().or_f16_decode(int(h))


def deq_row(ggml_type, blocks, n):
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    out = np.empty(n, dtype=np.float32)
    if lib().or_deq_row(ggml_type, _p(blocks), n, _p(out)) != 0:
        raise ValueError("unsupported type or size")
    return out


def requant_q8_row(x):
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    qs = np.empty(x.size, dtype=np.int8)
    ds = np.empty(x.size // 32, dtype=np.uint16)
    lib().or_requant_q8_row(_p(x), x.size, _p(qs), _p(ds))
    return qs, ds


def requant_q8(ggml_type, src, M, K):
    """One expert matrix of GGUF blocks -> (codes int8 [M][K], f16 bits [M][K/32])."""
    src = np.ascontiguousarray(src, dtype=np.uint8)
    qs = np.empty((M, K), dtype=np.int8)
    ds = np.empty((M, K // 32), dtype=np.uint16)
    if lib().or_requant_q8(ggml_type, _p(src), M, K, _p(qs), _p(ds)) != 0:
        raise ValueError("unsupported type or size")
    return qs, ds


def quant_q8b(x):
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    q = np.empty(x.size, dtype=np.int8)
    d = np.empty(x.size // 32, dtype=np.float32)
    lib().or_quant_q8b(_p(x), x.size, _p(q), _p(d))
    return q, d


def expert_down_q8(qs, ds, hd):
    qs = np.ascontiguousarray(qs, dtype=np.int8)
    ds = np.ascontiguousarray(ds, dtype=np.uint16)
    hd = np.ascontiguousarray(hd, dtype=np.float64)
    D, FF = qs.shape
    y = np.empty(D, dtype=np.float64)
    lib().or_expert_down_q8(_p(qs), _p(ds), D, FF, _p(hd), _p(y))
    return y


def expert_h_q8(gq, gd, uq, ud, xd):
    gq = np.ascontiguousarray(gq, dtype=np.int8)
    uq = np.ascontiguousarray(uq, dtype=np.int8)
    gd = np.ascontiguousarray(gd, dtype=np.uint16)
    ud = np.ascontiguousarray(ud, dtype=np.uint16)
    xd = np.ascontiguousarray(xd, dtype=np.float64)
    FF, D = gq.shape
    h = np.empty(FF, dtype=np.float64)
    lib().or_expert_h_q8(_p(gq), _p(gd), _p(uq), _p(ud), D, FF, _p(xd), _p(h))
    return h


def moe_forward(w, x, logits, shg=None, k=8, scale=1.0, act_mode=0, tokens=None):
    """double [n_tok, d_model]; act_mode 0 = W4A8 (the build's numerics), 1 =
    W4A32 (the reference's decode), 2 = e4m3 x with f32 h rounded to fp16 for
    the down projection (the reference's prefill)."""
    s, keep = _wstruct(w)
    x = np.ascontiguousarray(x, dtype=np.float32)
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    T, D = x.shape
    shg_a = np.ascontiguousarray(shg, dtype=np.float32) if shg is not None else None
    tok = np.ascontiguousarray(tokens, dtype=np.int32) if tokens is not None else None
    n = T if tok is None else tok.size
    out = np.empty((n, D), dtype=np.float64)
    lib().or_moe_forward(ctypes.byref(s), _p(x), _p(logits), logits.shape[1], _p(shg_a), T, k,
                         scale, act_mode, _p(tok), n, _p(out))
    return out


def moe_forward_f32(w, x, logits, shg=None, k=8, scale=1.0, nthreads=1):
    s, keep = _wstruct(w)
    x = np.ascontiguousarray(x, dtype=np.float32)
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    T, D = x.shape
    shg_a = np.ascontiguousarray(shg, dtype=np.float32) if shg is not None else None
    out = np.empty((T, D), dtype=np.float32)
    lib().or_moe_forward_f32(ctypes.byref(s), _p(x), _p(logits), logits.shape[1], _p(shg_a), T, k,
                             scale, _p(out), nthreads)
    return out


# ---- the reference's own dequant, compiled from its header into _ref/ ----
_ref = None


def ref_lib():
    """The reference's q36_deq_mxfp4 / q36_e8m0_half (oracle/_ref), or None."""
    global _ref
    if _ref is None and os.path.exists(REF_LIB_PATH):
        L = ctypes.CDLL(REF_LIB_PATH)
        L.ref_deq_mxfp4.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        L.ref_e8m0_half.argtypes = [ctypes.c_uint8]
        L.ref_e8m0_half.restype = ctypes.c_float
        L.ref_deq_row_mxfp4.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
        L.ref_sizeof_block_mxfp4.restype = ctypes.c_int
        L.ref_deq_row.argtypes = [ctypes.c_uint32, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
        L.ref_fp16.argtypes = [ctypes.c_uint16]
        L.ref_fp16.restype = ctypes.c_float
        _ref = L
    return _ref
