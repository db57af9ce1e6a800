"""Python host mirror of the q36 MoE layer over the C ABI of libq36moe.so.

The layer keeps the reference's boundary: router logits in, combined hidden
state out (moe_ffn, q36_engine.cu:1592-1654; pf_moe_block,
q36_engine.cu:3423-3472).  torch supplies device memory and the stream; all
compute runs in the HIP kernels of libq36moe.so.  There is no CPU fallback:
a missing library, a tensor that is not on the GPU or a non-zero return code
raises.
"""
import ctypes
import os

import numpy as np
import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libq36moe.so")

FMT_F32 = 0
FMT_BF16 = 1

TAP_TOPK_IDX, TAP_TOPK_W, TAP_XQ, TAP_XS, TAP_EOFF, TAP_PERM, TAP_POS, TAP_HQ, TAP_HS, TAP_DNW = range(10)
TAP_HSF, TAP_XQ8, TAP_XSF = 10, 11, 12
GGML_Q8_0, GGML_Q5_K, GGML_Q6_K, GGML_MXFP4 = 8, 13, 14, 39

_ERRORS = {-22: "EINVAL", -12: "ENOMEM", -1000: "EHIP"}

_lib = None


class Q36MoEError(RuntimeError):
    pass


def lib():
    """The loaded C library (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise Q36MoEError(f"{LIB_PATH} is missing: build it with `python -m q36_amd.build`")
    L = ctypes.CDLL(LIB_PATH)
    vp, i, sz, f = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t, ctypes.c_float
    pp = ctypes.POINTER(ctypes.c_void_p)
    L.q36moe_version.restype = ctypes.c_char_p
    L.q36moe_expert_bytes.argtypes = [i, i]
    L.q36moe_expert_bytes.restype = sz
    L.q36moe_weights_upload.argtypes = [vp] * 6 + [i] * 4 + [pp]
    L.q36moe_weights_upload_typed.argtypes = [vp] * 3 + [i] + [vp] * 3 + [i] * 5 + [pp]
    L.q36moe_weights_down_type.argtypes = [vp]
    L.q36moe_weights_shared_type.argtypes = [vp]
    L.q36moe_requant_q8.argtypes = [i, vp, i, i, vp, vp]
    L.q36moe_pack_q8.argtypes = [vp, vp, i, i, vp]
    L.q36moe_unpack_q8.argtypes = [vp, i, i, vp, vp]
    L.q36moe_weights_alloc.argtypes = [i] * 4 + [pp]
    L.q36moe_weights_device_ptrs.argtypes = [vp] + [pp] * 6 + [ctypes.POINTER(sz)] * 2
    L.q36moe_weights_fill_synthetic.argtypes = [vp, ctypes.c_uint64, i, i, vp]
    L.q36moe_weights_free.argtypes = [vp]
    L.q36moe_weights_free.restype = None
    L.q36moe_pack_mxfp4.argtypes = [vp, i, i, vp]
    L.q36moe_unpack_mxfp4.argtypes = [vp, i, i, vp]
    L.q36moe_ctx_create.argtypes = [i] * 5 + [vp, pp]
    L.q36moe_ctx_set_stream.argtypes = [vp, vp]
    L.q36moe_ctx_free.argtypes = [vp]
    L.q36moe_ctx_free.restype = None
    L.q36moe_forward.argtypes = [vp, vp, vp, i, vp, i, vp, i, i, f, vp, i]
    L.q36moe_router_topk.argtypes = [vp, i, i, i, i, f, i, vp, vp, vp]
    L.q36moe_router_logits.argtypes = [vp, i, i, vp, i, i, i, i, vp, i, vp, vp]
    L.q36moe_quant_e4m3.argtypes = [vp, i, i, i, vp, vp, vp]
    L.q36moe_add_rmsnorm_quant.argtypes = [vp, vp, vp, i, i, f, vp, vp, vp, vp]
    L.q36moe_forward_q8.argtypes = [vp, vp, vp, vp, vp, i, vp, i, i, f, vp, i]
    L.q36moe_forward_noalloc.argtypes = [vp, vp, i, vp, i, vp, i, i, i, f, vp, i, vp]
    L.q36moe_ctx_copy_tap.argtypes = [vp, i, vp, sz, ctypes.POINTER(sz)]
    L.q36moe_ctx_set_path.argtypes = [vp, i]
    L.q36moe_ctx_last_path.argtypes = [vp]
    L.q36moe_ctx_check.argtypes = [vp]
    L.q36moe_ctx_set_timing.argtypes = [vp, i]
    L.q36moe_ctx_stage_times.argtypes = [vp, ctypes.POINTER(ctypes.c_double),
                                         ctypes.POINTER(ctypes.c_int), i, i]
    L.q36moe_stage_name.argtypes = [i]
    L.q36moe_stage_name.restype = ctypes.c_char_p
    L.q36moe_num_stages.argtypes = []
    L.q36moe_probe_mfma.argtypes = [vp, vp, vp, vp, i, i, vp, vp]
    L.q36moe_probe_mfma32.argtypes = [vp, vp, vp, vp, vp, vp]
    L.q36moe_ctx_replay.argtypes = [vp, vp, i]
    u32p, u64p = ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(ctypes.c_uint64)
    L.q36moe_gguf_open.argtypes = [ctypes.c_char_p, pp]
    L.q36moe_gguf_close.argtypes = [vp]
    L.q36moe_gguf_close.restype = None
    L.q36moe_gguf_info.argtypes = [vp, u32p, u64p, u64p, u32p, u64p]
    L.q36moe_gguf_tensor.argtypes = [vp, ctypes.c_char_p, u32p, u32p, u64p, u64p, pp, u64p]
    L.q36moe_gguf_u32.argtypes = [vp, ctypes.c_char_p, u32p]
    L.q36moe_weights_from_gguf.argtypes = [vp, i, i, pp]
    L.q36moe_router_from_gguf.argtypes = [vp, i, vp, sz, ctypes.POINTER(i), ctypes.POINTER(i)]
    _lib = L
    return L


def check(rc, what):
    if rc != 0:
        raise Q36MoEError(f"{what} returned {rc} ({_ERRORS.get(rc, '?')})")


def _stream(stream=None):
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


def _dev(t, name, dtype=None):
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise Q36MoEError(f"{name} must be a GPU tensor")
    if not t.is_contiguous():
        raise Q36MoEError(f"{name} must be contiguous")
    if dtype is not None and t.dtype != dtype:
        raise Q36MoEError(f"{name} must be {dtype}, got {t.dtype}")
    return ctypes.c_void_p(t.data_ptr())


def _shg(shg, T):
    """(pointer, element stride) of a [T] f32 GPU tensor of shared-gate
    logits, which may be a strided view such as column 256 of 257-wide
    router rows; (None, 0) without one.  A broadcast view (stride 0) and a
    length other than T are refused: the kernels read T elements at the
    stride given."""
    if shg is None:
        return None, 0
    if not isinstance(shg, torch.Tensor) or not shg.is_cuda or shg.dtype != torch.float32 or shg.dim() != 1:
        raise Q36MoEError("shg must be a 1-D float32 GPU tensor")
    if shg.shape[0] != T:
        raise Q36MoEError(f"shg must have T={T} elements, got {shg.shape[0]}")
    if T > 1 and shg.stride(0) < 1:
        raise Q36MoEError("shg must have a positive stride (no broadcast views)")
    return ctypes.c_void_p(shg.data_ptr()), shg.stride(0) if T > 1 else 1


def _host_u8(a):
    a = np.ascontiguousarray(a, dtype=np.uint8)
    return a, ctypes.c_void_p(a.ctypes.data)


# ---------------------------------------------------------------------------
# weights
# ---------------------------------------------------------------------------
class MoEWeights:
    """One layer's routed experts (+ optional shared expert) on the device,
    in the packed fragment layout (mirrors the MXFP4 branch of upload(),
    q36_engine.cu:196-228)."""

    def __init__(self, handle, n_expert, d_model, d_ff, d_ff_sh):
        self._h = handle
        self.n_expert, self.d_model, self.d_ff, self.d_ff_sh = n_expert, d_model, d_ff, d_ff_sh

    @classmethod
    def upload(cls, gate, up, down, sh_gate=None, sh_up=None, sh_down=None, down_type=GGML_MXFP4,
               sh_type=GGML_MXFP4):
        """gate/up [E, d_ff, d_model/32, 17] GGUF block_mxfp4 bytes (numpy
        uint8); down [E, d_model, row bytes] blocks of ggml type down_type
        (GGML_MXFP4 [.., d_ff/32, 17], or GGML_Q8_0 / GGML_Q5_K / GGML_Q6_K,
        requantised to the q8_0-split layout as upload() does for k-quant
        experts, q36_engine.cu:229-252).  sh_* are the shared expert's three
        matrices, all of ggml type sh_type ([rows, row bytes] blocks; the
        release file's are GGML_Q8_0)."""
        E, d_ff, nbk, _ = gate.shape
        d_model = nbk * 32
        keep = []
        ptrs = []
        for a in (gate, up, down):
            a, p = _host_u8(a)
            keep.append(a)
            ptrs.append(p)
        d_ff_sh = 0
        if sh_gate is not None:
            d_ff_sh = d_ff
            for a in (sh_gate, sh_up, sh_down):
                a, p = _host_u8(a)
                keep.append(a)
                ptrs.append(p)
        else:
            ptrs += [None, None, None]
        h = ctypes.c_void_p()
        check(lib().q36moe_weights_upload_typed(*ptrs[:3], down_type, *ptrs[3:], sh_type, E, d_model, d_ff,
                                                d_ff_sh, ctypes.byref(h)),
              "q36moe_weights_upload_typed")
        return cls(h, E, d_model, d_ff, d_ff_sh)

    @property
    def down_type(self):
        """ggml type of the routed down on the device: GGML_MXFP4 or GGML_Q8_0
        (the q8_0-split layout, whatever type it was uploaded from)."""
        return lib().q36moe_weights_down_type(self._h)

    @property
    def shared_type(self):
        """GGML_MXFP4 or GGML_Q8_0 (q8_0-split) for the shared expert, 0 without one."""
        return lib().q36moe_weights_shared_type(self._h)

    @classmethod
    def from_gguf(cls, gguf, layer, with_shared=False):
        """Block `layer`'s MXFP4 experts (and shared expert) of an open GGUF."""
        h = ctypes.c_void_p()
        check(lib().q36moe_weights_from_gguf(gguf._h, layer, int(with_shared), ctypes.byref(h)),
              "q36moe_weights_from_gguf")
        t = gguf.tensor(f"blk.{layer}.ffn_gate_exps.weight")
        D, FF, E = t["dims"][:3]
        return cls(h, E, D, FF, FF if with_shared else 0)

    @classmethod
    def alloc(cls, n_expert, d_model, d_ff, d_ff_sh=0):
        h = ctypes.c_void_p()
        check(lib().q36moe_weights_alloc(n_expert, d_model, d_ff, d_ff_sh, ctypes.byref(h)),
              "q36moe_weights_alloc")
        return cls(h, n_expert, d_model, d_ff, d_ff_sh)

    def fill_synthetic(self, seed, exp_lo=-8, exp_hi=0, stream=None):
        """Seeded synthetic MXFP4 contents written on the device."""
        check(lib().q36moe_weights_fill_synthetic(self._h, seed, exp_lo, exp_hi, _stream(stream)),
              "q36moe_weights_fill_synthetic")
        return self

    def device_ptrs(self):
        """dict name -> (device address, bytes of the whole region)."""
        p = [ctypes.c_void_p() for _ in range(6)]
        gb, db = ctypes.c_size_t(), ctypes.c_size_t()
        check(lib().q36moe_weights_device_ptrs(self._h, *[ctypes.byref(x) for x in p],
                                               ctypes.byref(gb), ctypes.byref(db)),
              "q36moe_weights_device_ptrs")
        E = self.n_expert
        out = {"gate": (p[0].value, gb.value * E), "up": (p[1].value, gb.value * E),
               "down": (p[2].value, db.value * E)}
        if self.d_ff_sh:
            sb = gb.value if self.shared_type == GGML_MXFP4 else self.d_model * self.d_ff * 17 // 16
            out.update({"sh_gate": (p[3].value, sb), "sh_up": (p[4].value, sb), "sh_down": (p[5].value, sb)})
        return out

    def free(self):
        if self._h:
            lib().q36moe_weights_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def pack_mxfp4(blocks):
    """Host repack of one [M, K/32, 17] GGUF matrix to the device layout."""
    M, nb, _ = blocks.shape
    K = nb * 32
    src, p = _host_u8(blocks)
    out = np.empty(M * K // 2 + M * K // 32, dtype=np.uint8)
    check(lib().q36moe_pack_mxfp4(p, M, K, ctypes.c_void_p(out.ctypes.data)), "q36moe_pack_mxfp4")
    return out


def requant_q8(ggml_type, blocks, M, K):
    """Host: one [M][K] matrix of GGUF Q8_0 / Q5_K / Q6_K blocks -> (int8 codes
    [M, K], f16 scale bits [M, K/32]) in the q8_0-split layout."""
    src, p = _host_u8(blocks)
    codes = np.empty((M, K), dtype=np.int8)
    scales = np.empty((M, K // 32), dtype=np.uint16)
    check(lib().q36moe_requant_q8(ggml_type, p, M, K, ctypes.c_void_p(codes.ctypes.data),
                                  ctypes.c_void_p(scales.ctypes.data)), "q36moe_requant_q8")
    return codes, scales


def pack_q8(codes, scales):
    M, K = codes.shape
    codes = np.ascontiguousarray(codes, dtype=np.int8)
    scales = np.ascontiguousarray(scales, dtype=np.uint16)
    out = np.empty(M * K + M * K // 16, dtype=np.uint8)
    check(lib().q36moe_pack_q8(ctypes.c_void_p(codes.ctypes.data), ctypes.c_void_p(scales.ctypes.data), M, K,
                               ctypes.c_void_p(out.ctypes.data)), "q36moe_pack_q8")
    return out


def unpack_q8(packed, M, K):
    src, p = _host_u8(packed)
    codes = np.empty((M, K), dtype=np.int8)
    scales = np.empty((M, K // 32), dtype=np.uint16)
    check(lib().q36moe_unpack_q8(p, M, K, ctypes.c_void_p(codes.ctypes.data), ctypes.c_void_p(scales.ctypes.data)),
          "q36moe_unpack_q8")
    return codes, scales


def unpack_mxfp4(packed, M, K):
    src, p = _host_u8(packed)
    out = np.empty((M, K // 32, 17), dtype=np.uint8)
    check(lib().q36moe_unpack_mxfp4(p, M, K, ctypes.c_void_p(out.ctypes.data)),
          "q36moe_unpack_mxfp4")
    return out


# ---------------------------------------------------------------------------
# the layer
# ---------------------------------------------------------------------------
class MoELayer:
    """Scratch + launch context for the MoE forward (moe_ffn / pf_moe_block
    boundary).  All scratch is allocated at construction."""

    def __init__(self, max_tokens, n_expert=256, d_model=2048, d_ff=512, top_k=8, stream=None):
        self.max_tokens, self.n_expert, self.d_model, self.d_ff, self.top_k = (
            max_tokens, n_expert, d_model, d_ff, top_k)
        self._h = ctypes.c_void_p()
        check(lib().q36moe_ctx_create(max_tokens, n_expert, d_model, d_ff, top_k, _stream(stream),
                                      ctypes.byref(self._h)), "q36moe_ctx_create")
        self.last_T = 0
        self.last_shared = False

    def set_stream(self, stream):
        check(lib().q36moe_ctx_set_stream(self._h, _stream(stream)), "q36moe_ctx_set_stream")

    def forward(self, weights, x, logits, shg=None, scale=1.0, out_dtype=torch.bfloat16, out=None):
        """x [T, d_model] f32|bf16, logits [T, >=n_expert] f32 (row stride
        free), shg [T] f32 (any stride, e.g. column 256 of 257-wide router
        rows) or None -> out [T, d_model] (bf16 or f32)."""
        T = x.shape[0]
        xf = FMT_F32 if x.dtype == torch.float32 else FMT_BF16
        if x.dtype not in (torch.float32, torch.bfloat16):
            raise Q36MoEError("x must be float32 or bfloat16")
        if out is None:
            out = torch.empty((T, self.d_model), dtype=out_dtype, device=x.device)
        of = FMT_F32 if out.dtype == torch.float32 else FMT_BF16
        if logits.dim() != 2 or logits.shape[0] != T:
            raise Q36MoEError("logits must be [T, n_expert]")
        ld = logits.stride(0)
        if logits.stride(1) != 1:
            raise Q36MoEError("logits rows must be contiguous")
        lp = ctypes.c_void_p(logits.data_ptr()) if T else None
        if T and (not logits.is_cuda or logits.dtype != torch.float32):
            raise Q36MoEError("logits must be a float32 GPU tensor")
        sp, sld = _shg(shg, T)
        xp = _dev(x, "x") if T else None
        op = _dev(out, "out") if T else None
        check(lib().q36moe_forward(self._h, weights._h, xp, xf, lp, ld, sp, sld, T, float(scale), op, of),
              "q36moe_forward")
        self.last_T = T
        self.last_shared = shg is not None
        return out

    def forward_q8(self, weights, xq, xs, logits, shg=None, scale=1.0, out_dtype=torch.bfloat16, out=None):
        """forward on activations already quantised (add_rmsnorm_quant or
        quant_e4m3): xq u8 [T, d_model] e4m3, xs u8 [T, d_model/32] E8M0."""
        T = xq.shape[0]
        if out is None:
            out = torch.empty((T, self.d_model), dtype=out_dtype, device=xq.device)
        of = FMT_F32 if out.dtype == torch.float32 else FMT_BF16
        if logits.dim() != 2 or logits.shape[0] != T or logits.stride(1) != 1:
            raise Q36MoEError("logits must be [T, n_expert] with contiguous rows")
        if T and (not logits.is_cuda or logits.dtype != torch.float32):
            raise Q36MoEError("logits must be a float32 GPU tensor")
        lp = ctypes.c_void_p(logits.data_ptr()) if T else None
        sp, sld = _shg(shg, T)
        qp = _dev(xq, "xq", torch.uint8) if T else None
        sc = _dev(xs, "xs", torch.uint8) if T else None
        op = _dev(out, "out") if T else None
        check(lib().q36moe_forward_q8(self._h, weights._h, qp, sc, lp, logits.stride(0), sp, sld, T, float(scale),
                                      op, of), "q36moe_forward_q8")
        self.last_T = T
        self.last_shared = shg is not None
        return out

    def tap(self, which):
        """Copy of an internal buffer of the last forward (see TAP_*)."""
        T, k, D, FF, E = self.last_T, self.top_k, self.d_model, self.d_ff, self.n_expert
        rows = T * k + (T if self.last_shared else 0)
        shapes = {
            TAP_TOPK_IDX: ((T, k), torch.int32), TAP_TOPK_W: ((T, k), torch.float32),
            TAP_XQ: ((T, D), torch.uint8), TAP_XS: ((T, D // 32), torch.uint8),
            TAP_EOFF: ((E + 1,), torch.int32), TAP_PERM: ((T * k,), torch.int32),
            TAP_POS: ((T * k,), torch.int32), TAP_HQ: ((rows, FF), torch.uint8),
            TAP_HS: ((rows, FF // 32), torch.uint8), TAP_DNW: ((rows, D), torch.float32),
            TAP_HSF: ((rows, FF // 32), torch.float32),
            TAP_XQ8: ((T, D), torch.int8), TAP_XSF: ((T, D // 32), torch.float32),
        }
        shape, dt = shapes[which]
        dst = torch.empty(shape, dtype=dt, device="cuda")
        n = ctypes.c_size_t()
        check(lib().q36moe_ctx_copy_tap(self._h, which, ctypes.c_void_p(dst.data_ptr()),
                                        dst.numel() * dst.element_size(), ctypes.byref(n)),
              "q36moe_ctx_copy_tap")
        return dst

    PATH_AUTO, PATH_SORTED, PATH_DIRECT, PATH_SORTED_SKINNY, PATH_SORTED_FUSED = 0, 1, 2, 4, 5

    def set_path(self, mode):
        """0 auto (direct for T <= 16, skinny tiles while T*k <= 8*n_expert --
        16*n_expert in one kernel per tile for MXFP4 layers),
        1 sorted (fat tiles), 2 direct, 4 sorted (skinny tiles, gate/up and
        down as two kernels), 5 sorted (skinny tiles, one kernel per tile;
        layers with an int8 down or shared expert take 4); 3 is refused
        (EINVAL)."""
        check(lib().q36moe_ctx_set_path(self._h, mode), "q36moe_ctx_set_path")

    @property
    def last_path(self):
        """0 sorted (fat tiles), 1 direct, 2 sorted (skinny tiles, two
        kernels), 3 sorted (skinny tiles, one kernel per tile)."""
        return lib().q36moe_ctx_last_path(self._h)

    def check(self):
        """Synchronise the layer's stream; raise on a HIP error."""
        check(lib().q36moe_ctx_check(self._h), "q36moe_ctx_check")

    def set_timing(self, on):
        check(lib().q36moe_ctx_set_timing(self._h, 1 if on else 0), "q36moe_ctx_set_timing")

    def stage_times(self, reset=False):
        """dict stage -> (total ms, calls) since the last reset."""
        n = lib().q36moe_num_stages()
        ms = (ctypes.c_double * n)()
        calls = (ctypes.c_int * n)()
        check(lib().q36moe_ctx_stage_times(self._h, ms, calls, n, 1 if reset else 0),
              "q36moe_ctx_stage_times")
        return {lib().q36moe_stage_name(i).decode(): (ms[i], calls[i]) for i in range(n)}

    STAGES = ("route", "scan", "gateup", "down", "combine")

    def replay(self, weights, stage):
        """Launch the kernels of one stage of the last forward again with
        `weights` (asynchronous, on the layer's stream)."""
        st = self.STAGES.index(stage) if isinstance(stage, str) else int(stage)
        check(lib().q36moe_ctx_replay(self._h, weights._h, st), "q36moe_ctx_replay")

    def free(self):
        if self._h:
            lib().q36moe_ctx_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


# ---------------------------------------------------------------------------
# stage entry points
# ---------------------------------------------------------------------------
def router_topk(logits, k=8, scale=1.0, renorm=True, n_expert=None):
    """k_router_topk (q36_ops.cuh:397-431): -> idx int32 [T,k], wt f32 [T,k]."""
    T = logits.shape[0]
    E = n_expert or logits.shape[1]
    idx = torch.empty((T, k), dtype=torch.int32, device=logits.device)
    wt = torch.empty((T, k), dtype=torch.float32, device=logits.device)
    if logits.stride(1) != 1:
        raise Q36MoEError("logits rows must be contiguous")
    lp = ctypes.c_void_p(logits.data_ptr()) if T else None
    if T and (not logits.is_cuda or logits.dtype != torch.float32):
        raise Q36MoEError("logits must be a float32 GPU tensor")
    check(lib().q36moe_router_topk(lp, T, E, logits.stride(0), k, float(scale), 1 if renorm else 0,
                                   ctypes.c_void_p(idx.data_ptr()), ctypes.c_void_p(wt.data_ptr()),
                                   _stream()), "q36moe_router_topk")
    return idx, wt


ROUTER_AUTO, ROUTER_F32, ROUTER_F16 = 0, 1, 2


def router_logits(w, x, n_expert, mode=ROUTER_AUTO):
    """Router matvec (k_matvec_f32_row / pf_gemm, q36_ops.cuh:331-342,
    q36_engine.cu:3403-3414): w [n_rows, 2048] f32, x [T, 2048] f32|bf16 ->
    logits f32 [T, n_expert] and, with n_rows == n_expert + 1, the
    shared-gate logit f32 [T] (else None)."""
    T = x.shape[0]
    n_rows = w.shape[0]
    logits = torch.empty((T, n_expert), dtype=torch.float32, device=x.device)
    shg = torch.empty((T,), dtype=torch.float32, device=x.device) if n_rows > n_expert else None
    fmt = FMT_F32 if x.dtype == torch.float32 else FMT_BF16
    wp = _dev(w, "w", torch.float32)
    xp = _dev(x, "x") if T else None
    check(lib().q36moe_router_logits(wp, n_rows, n_expert, xp, fmt, T, x.shape[1], mode,
                                     ctypes.c_void_p(logits.data_ptr()), n_expert,
                                     ctypes.c_void_p(shg.data_ptr()) if shg is not None else None,
                                     _stream()), "q36moe_router_logits")
    return logits, shg


class GGUF:
    """A GGUF v3 file mapped by the library (q36moe_gguf_*)."""

    def __init__(self, path):
        self._h = ctypes.c_void_p()
        check(lib().q36moe_gguf_open(os.fsencode(path), ctypes.byref(self._h)), "q36moe_gguf_open")

    def close(self):
        if self._h:
            lib().q36moe_gguf_close(self._h)
            self._h = ctypes.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def info(self):
        v, al = ctypes.c_uint32(), ctypes.c_uint32()
        nt, nk, off = ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint64()
        check(lib().q36moe_gguf_info(self._h, ctypes.byref(v), ctypes.byref(nt), ctypes.byref(nk),
                                     ctypes.byref(al), ctypes.byref(off)), "q36moe_gguf_info")
        return {"version": v.value, "n_tensors": nt.value, "n_kv": nk.value, "alignment": al.value,
                "data_offset": off.value}

    def tensor(self, name):
        ty, nd = ctypes.c_uint32(), ctypes.c_uint32()
        dims = (ctypes.c_uint64 * 4)()
        off, nb = ctypes.c_uint64(), ctypes.c_uint64()
        data = ctypes.c_void_p()
        check(lib().q36moe_gguf_tensor(self._h, name.encode(), ctypes.byref(ty), ctypes.byref(nd), dims,
                                       ctypes.byref(off), ctypes.byref(data), ctypes.byref(nb)),
              "q36moe_gguf_tensor")
        return {"type": ty.value, "n_dims": nd.value, "dims": list(dims), "file_offset": off.value,
                "nbytes": nb.value}

    def u32(self, key):
        v = ctypes.c_uint32()
        check(lib().q36moe_gguf_u32(self._h, key.encode(), ctypes.byref(v)), "q36moe_gguf_u32")
        return v.value

    def router(self, layer):
        """Host f32 router rows [n_expert (+1 shared gate), d_model]."""
        t = self.tensor(f"blk.{layer}.ffn_gate_inp.weight")
        dst = np.empty((t["dims"][1] + 1) * t["dims"][0], dtype=np.float32)
        nr, dm = ctypes.c_int(), ctypes.c_int()
        check(lib().q36moe_router_from_gguf(self._h, layer, ctypes.c_void_p(dst.ctypes.data), dst.size,
                                            ctypes.byref(nr), ctypes.byref(dm)), "q36moe_router_from_gguf")
        return dst[: nr.value * dm.value].reshape(nr.value, dm.value).copy()


def add_rmsnorm_quant(h, a, w, eps=1e-6, want_y=True, want_q=True):
    """Residual add + RMSNorm + per-32 quantisation in one kernel
    (k_add_rmsnorm q36_engine.cu:696-706, then k_quant_e4m3 :2411-2428):
    h [T, 2048] f32 (h += a in place when a is given), w [2048] f32 ->
    (y f32 [T, 2048] or None, xq u8 [T, 2048] or None, xs u8 [T, 64] or None)."""
    T, D = h.shape
    y = torch.empty((T, D), dtype=torch.float32, device=h.device) if want_y else None
    xq = torch.empty((T, D), dtype=torch.uint8, device=h.device) if want_q else None
    xs = torch.empty((T, D // 32), dtype=torch.uint8, device=h.device) if want_q else None
    hp = _dev(h, "h", torch.float32) if T else None
    ap = _dev(a, "a", torch.float32) if (a is not None and T) else None
    ptr = lambda t: ctypes.c_void_p(t.data_ptr()) if (t is not None and T) else None
    check(lib().q36moe_add_rmsnorm_quant(hp, ap, _dev(w, "w", torch.float32), T, D, float(eps),
                                         ptr(y), ptr(xq), ptr(xs), _stream()), "q36moe_add_rmsnorm_quant")
    return y, xq, xs


def quant_e4m3(x):
    """k_quant_e4m3 (q36_engine.cu:2411-2428): x [T,K] f32|bf16 ->
    (xq u8 [T,K] e4m3, xs u8 [T,K/32] E8M0)."""
    T, K = x.shape
    xq = torch.empty((T, K), dtype=torch.uint8, device=x.device)
    xs = torch.empty((T, K // 32), dtype=torch.uint8, device=x.device)
    fmt = FMT_F32 if x.dtype == torch.float32 else FMT_BF16
    xp = _dev(x, "x") if T else None
    check(lib().q36moe_quant_e4m3(xp, fmt, T, K, ctypes.c_void_p(xq.data_ptr()),
                                  ctypes.c_void_p(xs.data_ptr()), _stream()), "q36moe_quant_e4m3")
    return xq, xs


def probe_mfma(a, b, sa, sb, fmt_a, fmt_b):
    """One scaled 16x16x128 MFMA: a, b uint8 [64, 32]; sa, sb int32/uint32 [64]."""
    c = torch.empty((64, 4), dtype=torch.float32, device=a.device)
    check(lib().q36moe_probe_mfma(_dev(a, "a"), _dev(b, "b"), _dev(sa, "sa"), _dev(sb, "sb"),
                                  fmt_a, fmt_b, ctypes.c_void_p(c.data_ptr()), _stream()),
          "q36moe_probe_mfma")
    return c


def probe_mfma32(a, b, sa, sb):
    """One scaled 32x32x64 MFMA (A e2m1, B e4m3): a, b uint8 [64, 32]; sa, sb
    int32/uint32 [64] -> [64, 16] lane results."""
    c = torch.empty((64, 16), dtype=torch.float32, device=a.device)
    check(lib().q36moe_probe_mfma32(_dev(a, "a"), _dev(b, "b"), _dev(sa, "sa"), _dev(sb, "sb"),
                                    ctypes.c_void_p(c.data_ptr()), _stream()), "q36moe_probe_mfma32")
    return c


NOALLOC_MAX_T = 64


def forward_noalloc(weights, x, logits, shg=None, top_k=8, scale=1.0, out=None, out_dtype=torch.bfloat16,
                    stream=None):
    """q36moe_forward_noalloc: the layer without a context, on the library's
    static per-GPU scratch (T <= NOALLOC_MAX_T).  `out` may be given so the
    call itself allocates nothing on the device either."""
    T = x.shape[0]
    if x.dtype not in (torch.float32, torch.bfloat16):
        raise Q36MoEError("x must be float32 or bfloat16")
    xf = FMT_F32 if x.dtype == torch.float32 else FMT_BF16
    if out is None:
        out = torch.empty((T, weights.d_model), dtype=out_dtype, device=x.device)
    of = FMT_F32 if out.dtype == torch.float32 else FMT_BF16
    if logits.dim() != 2 or logits.shape[0] != T or logits.stride(1) != 1:
        raise Q36MoEError("logits must be [T, n_expert] with contiguous rows")
    if T and (not logits.is_cuda or logits.dtype != torch.float32):
        raise Q36MoEError("logits must be a float32 GPU tensor")
    sp, sld = _shg(shg, T)
    check(lib().q36moe_forward_noalloc(weights._h, _dev(x, "x") if T else None, xf,
                                       ctypes.c_void_p(logits.data_ptr()) if T else None, logits.stride(0),
                                       sp, sld, T, top_k, float(scale), _dev(out, "out") if T else None, of,
                                       _stream(stream)), "q36moe_forward_noalloc")
    return out
