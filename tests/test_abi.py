"""C-ABI checks that need no GPU: the library loads, exports every symbol
include/q36moe.h declares, the host repack is a bijection with the documented
fragment layout, and argument validation rejects bad calls before any HIP
call is made."""
import ctypes
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "q36moe.h")


@pytest.fixture(scope="module")
def L():
    from q36_amd import moe
    return moe.lib()


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(q36moe_\w+)\s*\(", text)))


def test_exports_every_declared_symbol(L):
    syms = declared_symbols()
    assert len(syms) >= 20
    for s in syms:
        assert hasattr(L, s), s


def test_version_and_sizes(L):
    assert b"gfx950" in L.q36moe_version()
    assert L.q36moe_expert_bytes(2048, 512) == 1671168      # 3 x 557,056 B
    assert L.q36moe_num_stages() == 5


def test_pack_unpack_roundtrip():
    from q36_amd import moe, synth
    rng = np.random.default_rng(1)
    for M, K in ((512, 2048), (2048, 512), (16, 512)):
        W = synth.mxfp4_blocks(rng, M, K)
        p = moe.pack_mxfp4(W)
        assert p.size == M * K // 2 + M * K // 32
        np.testing.assert_array_equal(moe.unpack_mxfp4(p, M, K), W)


def _code_gguf(W, r, k):
    blk = W[r, k // 32]
    j = k % 32
    return (blk[1 + j] & 15) if j < 16 else (blk[1 + j - 16] >> 4)


def test_pack_layout_matches_fragment_order():
    """Packed byte (mt, kt, lane, j) holds codes k=2j, 2j+1 of row
    mt*16+lane%16, block kt*4+lane/16 (low nibble first); the E8M0 of that
    lane sits at scale byte (mt*64+lane)*(K/128)+kt."""
    from q36_amd import moe, synth
    rng = np.random.default_rng(2)
    M, K = 32, 1024
    W = synth.mxfp4_blocks(rng, M, K)
    p = moe.pack_mxfp4(W)
    nkt = K // 128
    for _ in range(2000):
        r, k = int(rng.integers(M)), int(rng.integers(K))
        mt, kb = r // 16, k // 32
        kt, lane = kb // 4, r % 16 + 16 * (kb % 4)
        j = k % 32
        byte = p[(mt * nkt + kt) * 1024 + lane * 16 + j // 2]
        code = (byte >> 4) if (j & 1) else (byte & 15)
        assert code == _code_gguf(W, r, k)
        assert p[M * K // 2 + (mt * 64 + lane) * nkt + kt] == W[r, kb, 0]


def test_pack_rejects_bad_args(L):
    buf = np.zeros(1 << 16, dtype=np.uint8)
    vp = ctypes.c_void_p(buf.ctypes.data)
    assert L.q36moe_pack_mxfp4(vp, 15, 512, vp) == -22        # M % 16
    assert L.q36moe_pack_mxfp4(vp, 16, 500, vp) == -22        # K % 512
    assert L.q36moe_pack_mxfp4(None, 16, 512, vp) == -22
    blk = np.zeros((16, 16, 17), dtype=np.uint8)
    blk[3, 2, 0] = 255                                        # NaN scale
    out = np.zeros(16 * 512 // 2 + 16 * 512 // 32, dtype=np.uint8)
    assert L.q36moe_pack_mxfp4(ctypes.c_void_p(blk.ctypes.data), 16, 512,
                               ctypes.c_void_p(out.ctypes.data)) == -22


def test_entry_points_reject_bad_args_without_gpu(L):
    """Validation happens before any HIP call, so these run on a CPU host."""
    assert L.q36moe_forward(None, None, None, 0, None, 256, None, 0, 1, ctypes.c_float(1.0), None, 0) == -22
    assert L.q36moe_router_topk(None, 4, 300, 300, 8, ctypes.c_float(1.0), 1, None, None, None) == -22
    assert L.q36moe_router_topk(None, 4, 256, 256, 9, ctypes.c_float(1.0), 1, None, None, None) == -22
    assert L.q36moe_router_topk(None, 0, 256, 256, 8, ctypes.c_float(1.0), 1, None, None, None) == 0
    assert L.q36moe_quant_e4m3(None, 0, 4, 100, None, None, None) == -22
    rl = L.q36moe_router_logits
    assert rl(None, 257, 256, None, 0, 4, 2000, 0, None, 256, None, None) == -22   # d_model
    assert rl(None, 258, 256, None, 0, 4, 2048, 0, None, 256, None, None) == -22   # rows > E+1
    assert rl(None, 256, 256, None, 0, 4, 2048, 3, None, 256, None, None) == -22   # mode
    assert rl(None, 256, 256, None, 0, 4, 2048, 0, None, 255, None, None) == -22   # ld < E
    assert rl(None, 257, 256, None, 0, 0, 2048, 0, None, 256, None, None) == 0     # T = 0
    arq = L.q36moe_add_rmsnorm_quant
    assert arq(None, None, None, 4, 1024, ctypes.c_float(1e-6), None, None, None, None) == -22  # d_model
    assert arq(None, None, None, 4, 2048, ctypes.c_float(-1.0), None, None, None, None) == -22  # eps
    assert arq(None, None, None, 4, 2048, ctypes.c_float(1e-6), None, None, ctypes.c_void_p(8), None) == -22  # xq w/o xs
    assert arq(None, None, None, 0, 2048, ctypes.c_float(1e-6), None, None, None, None) == 0
    assert L.q36moe_forward_q8(None, None, None, None, None, 256, None, 0, 1, ctypes.c_float(1.0), None, 0) == -22
    assert L.q36moe_quant_e4m3(None, 2, 4, 128, None, None, None) == -22
    assert L.q36moe_quant_e4m3(None, 0, 0, 128, None, None, None) == 0
    h = ctypes.c_void_p()
    assert L.q36moe_ctx_create(0, 256, 2048, 512, 8, None, ctypes.byref(h)) == -22
    assert L.q36moe_ctx_create(16, 257, 2048, 512, 8, None, ctypes.byref(h)) == -22
    assert L.q36moe_ctx_create(16, 256, 2048, 512, 9, None, ctypes.byref(h)) == -22
    assert L.q36moe_weights_alloc(256, 2000, 512, 0, ctypes.byref(h)) == -22
    assert L.q36moe_weights_alloc(256, 2048, 512, 256, ctypes.byref(h)) == -22
    assert L.q36moe_probe_mfma(None, None, None, None, 4, 0, None, None) == -22
    assert L.q36moe_stage_name(0) == b"route"
    assert L.q36moe_stage_name(99) is None


def test_product_does_not_reference_oracle():
    """The product sources never load the oracle."""
    pat = re.compile(r"(from\s+oracle|import\s+oracle|liboracle|pyoracle|or_moe_forward)")
    for d, _, files in os.walk(os.path.join(ROOT, "q36_amd")):
        for f in files:
            if f.endswith((".py", ".hip", ".cpp", ".h")):
                assert not pat.search(open(os.path.join(d, f)).read()), f
