"""The reference's requantised expert format (q8_0-split) for the routed down
projection: Q5_K / Q6_K experts dequantised and requantised per 32 to int8
with an f16 scale (upload(), q36_engine.cu:229-252, h_q8_row :73-86), h
quantised per 32 to int8 with an fp32 scale (k_quant_q8b :2627-2640) and the
down GEMM on integer MMA with both scales per 32-block (k_gemm_expert_i8
:2526-2618).

CPU tests pin the oracle's restatement (f16 against numpy.float16, the
k-quant dequantisers bit-exactly against the reference's own q36_deq_row
compiled from its header, closed forms and hand-computed blocks) and check the
product's host requantiser and packer against it bit for bit.  GPU tests
(marked gpu) run the layer through the C ABI on every path, with the bars of
test_gpu_parity.py: int8 h codes equal the oracle's quantisation of fp32(h)
except at rounding midpoints; down + combine from the GPU's own h within
2e-3 of fp64; end to end within 2e-3 per token (against the plain oracle, or
with the GPU's codes substituted at the flipped elements of a token that has
midpoint flips).  The Q8_0 shared-expert tests check the shared row's codes
only, so their end-to-end figure keeps a 1e-2 backstop.
"""
import ctypes

import numpy as np
import pytest

from q36_amd import synth

Q8_0, Q5_K, Q6_K = synth.GGML_Q8_0, synth.GGML_Q5_K, synth.GGML_Q6_K
TYPES = [pytest.param(Q5_K, id="q5_k"), pytest.param(Q6_K, id="q6_k"), pytest.param(Q8_0, id="q8_0")]


# ---------------------------------------------------------------------------
# f16
# ---------------------------------------------------------------------------
def test_f16_decode_all_patterns(oracle):
    bits = np.arange(65536, dtype=np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([oracle.f16_decode(int(b)) for b in bits], dtype=np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f16_encode_matches_numpy(oracle):
    rng = np.random.default_rng(5)
    # random magnitudes over the whole f16 range and beyond (subnormals, overflow)
    v = (rng.standard_normal(20000) * 2.0 ** rng.integers(-30, 20, 20000)).astype(np.float32)
    # every rounding midpoint between consecutive finite f16 values of a slice
    h = np.arange(0, 0x7bff, 7, dtype=np.uint16).view(np.float16).astype(np.float64)
    hn = np.arange(1, 0x7c00, 7, dtype=np.uint16).view(np.float16).astype(np.float64)
    mids = ((h + hn) / 2).astype(np.float32)
    v = np.concatenate([v, mids, -mids, np.float32([65504, 65519.99, 65520, 1e-8, 0, -0.0, np.inf, -np.inf])])
    with np.errstate(over="ignore"):
        want = v.astype(np.float16).view(np.uint16)
    got = np.array([oracle.f16_encode(float(x)) for x in v], dtype=np.uint16)
    np.testing.assert_array_equal(got, want)


# ---------------------------------------------------------------------------
# k-quant dequantisers
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("ggml_type", TYPES)
def test_deq_matches_reference_build(oracle, ggml_type):
    ref = oracle.ref_lib()
    if ref is None:
        pytest.skip("oracle/_ref not built (reference tree absent)")
    rng = np.random.default_rng(ggml_type)
    elems, size = synth.KQUANT_BLOCK[ggml_type]
    blk = synth.kquant_blocks(rng, 64, 1024, ggml_type)
    # also raw random bytes (any finite or non-finite f16 scale)
    raw = np.frombuffer(rng.bytes(blk.size), dtype=np.uint8).reshape(blk.shape)
    for b in (blk, raw):
        n = b.size // size * elems
        got = oracle.deq_row(ggml_type, b, n)
        want = np.empty(n, dtype=np.float32)
        ref.ref_deq_row(ggml_type, b.ctypes.data, n, want.ctypes.data)
        # bit-exact, except NaN payloads (from NaN f16 scales in raw bytes)
        nan = np.isnan(want)
        np.testing.assert_array_equal(np.isnan(got), nan)
        np.testing.assert_array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


@pytest.mark.parametrize("name,ggml_type", [("q8_0", Q8_0), ("q5_k", Q5_K), ("q6_k", Q6_K)])
def test_deq_golden_fixture(oracle, name, ggml_type):
    """The oracle against the reference's q36_deq_row outputs committed in
    tests/golden/kquant_dequant_ref.npz (made by tests/golden/make_golden.py
    from the reference's own header), bit for bit; holds where the
    reference tree is absent."""
    import os
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "kquant_dequant_ref.npz")
    g = np.load(path)
    blocks, want = g[name + "_blocks"], g[name + "_values"]
    got = oracle.deq_row(ggml_type, blocks, want.size).reshape(want.shape)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    # and the product's requantiser consumes exactly these values
    from q36_amd import moe
    elems = synth.KQUANT_BLOCK[ggml_type][0]
    K = 256 if elems == 256 else 32
    pc, ps = moe.requant_q8(ggml_type, blocks.reshape(-1, blocks.shape[1] * (K // elems)), blocks.shape[0] * elems // K, K)
    oc, os_ = oracle.requant_q8(ggml_type, blocks.reshape(-1, blocks.shape[1] * (K // elems)), blocks.shape[0] * elems // K, K)
    np.testing.assert_array_equal(pc, oc)
    np.testing.assert_array_equal(ps, os_)


def _f16(v):
    return np.frombuffer(np.float16(v).tobytes(), dtype=np.uint8)


def test_deq_q5_k_hand_computed(oracle):
    b = np.zeros(176, dtype=np.uint8)
    b[0:2], b[2:4] = _f16(1.0), _f16(0.5)
    sm = b[4:16]
    sm[0], sm[4] = 2, 3                    # sub-block 0: scale 2, min 3
    # sub-block 5: scale = (sm[9] & 15) | (sm[1] >> 6) << 4, min = (sm[9] >> 4) | (sm[5] >> 6) << 4
    sm[9] = 0x7 | (0x2 << 4)
    sm[1] = 0x40                           # scale high bits 01 -> 16 + 7 = 23
    sm[5] = 0x80                           # min high bits 10 -> 32 + 2 = 34
    qh, qs = b[16:48], b[48:176]
    qs[0] = 0x5 | (0x9 << 4)               # value 0: low nibble 5; value 32: high nibble 9
    qh[0] = 0b100001                       # bit 0 (sub-block 0) and bit 5 (sub-block 5)
    qs[64 + 3] = 0xA0                      # value 64*2 + 32 + 3 (sub-block 5): high nibble 10
    qh[3] = 0b100000
    y = oracle.deq_row(Q5_K, b, 256)
    assert y[0] == 1.0 * 2 * (5 + 16) - 0.5 * 3        # 40.5
    assert y[32] == 0.0                                 # sub-block 1: scale and min 0
    assert y[160 + 3] == 1.0 * 23 * (10 + 16) - 0.5 * 34
    assert y[160 + 4] == -0.5 * 34                      # code 0 in sub-block 5


def test_deq_q6_k_hand_computed(oracle):
    b = np.zeros(210, dtype=np.uint8)
    b[208:210] = _f16(0.25)
    sc = b[192:208].view(np.int8)
    sc[:] = np.arange(16) - 8                          # scale s -> s - 8
    ql, qh = b[0:128], b[128:192]
    # value 128 + 96 + 20 (n=1, g=3, l=20): high nibble of ql[64+32+20], bits 6-7 of qh[32+20]
    ql[64 + 32 + 20] = 0xB0
    qh[32 + 20] = 0b11000000
    y = oracle.deq_row(Q6_K, b, 256)
    q = (0xB | (3 << 4)) - 32                          # 27
    assert y[128 + 96 + 20] == np.float32(0.25 * (8 + 6 + 1 - 8)) * q
    assert y[0] == np.float32(0.25 * -8) * -32         # all-zero codes give q = -32


# ---------------------------------------------------------------------------
# requantiser, packer, h quantiser
# ---------------------------------------------------------------------------
def test_requant_q8_row_closed_form(oracle):
    rng = np.random.default_rng(11)
    x = (rng.standard_normal(32 * 200) * 2.0 ** rng.integers(-12, 4, 32 * 200)).astype(np.float32)
    x[:32] = 0.0                                       # an all-zero block
    qs, ds = oracle.requant_q8_row(x)
    xb = x.reshape(-1, 32)
    amax = np.abs(xb).max(axis=1)
    d = (amax / np.float32(127)).astype(np.float32)
    np.testing.assert_array_equal(ds, d.astype(np.float16).view(np.uint16))
    q = qs.reshape(-1, 32).astype(np.int64)
    assert np.all(q[0] == 0)
    # the largest magnitude of each non-zero block maps to +-127
    nz = amax > 0
    big = np.abs(xb).argmax(axis=1)
    assert np.all(np.abs(q[nz, big[nz]]) == 127)
    # codes are the nearest integers to v / d (fp32 d), so the error is <= d/2
    err = np.abs(q[nz] * d[nz, None].astype(np.float64) - xb[nz])
    assert np.all(err <= d[nz, None] * (0.5 + 1e-6))


@pytest.mark.parametrize("ggml_type", TYPES)
def test_product_requant_equals_oracle(oracle, ggml_type):
    from q36_amd import moe
    rng = np.random.default_rng(100 + ggml_type)
    M, K = 48, 512
    src = synth.kquant_blocks(rng, M, K, ggml_type)
    pc, ps = moe.requant_q8(ggml_type, src, M, K)
    oc, os_ = oracle.requant_q8(ggml_type, src, M, K)
    np.testing.assert_array_equal(pc, oc)
    np.testing.assert_array_equal(ps, os_)
    # and it is the round trip of the dequantised values: codes are nearest
    # to v/d (d/2) and the stored f16 d is within 2^-11 of d (127 codes)
    vals = oracle.deq_row(ggml_type, src, M * K).reshape(M, K)
    back = oc.astype(np.float64) * np.repeat(os_.view(np.float16).astype(np.float64), 32, axis=1)
    scale = np.repeat(np.abs(vals).reshape(M, -1, 32).max(axis=2), 32, axis=1).astype(np.float64)
    assert np.all(np.abs(back - vals) <= scale / 127 * (0.5 + 127 * 2.0 ** -11) * 1.001 + 1e-12)


def test_pack_q8_layout_and_roundtrip():
    from q36_amd import moe
    rng = np.random.default_rng(3)
    M, K = 64, 512
    codes = rng.integers(-128, 128, (M, K)).astype(np.int8)
    scales = rng.uniform(0.001, 0.1, (M, K // 32)).astype(np.float16).view(np.uint16)
    pk = moe.pack_q8(codes, scales)
    assert pk.size == M * K + M * K // 16
    c2, s2 = moe.unpack_q8(pk, M, K)
    np.testing.assert_array_equal(c2, codes)
    np.testing.assert_array_equal(s2, scales)
    # codes: (row tile mt, K pair kp) at 1024 B, lane L = row mt*16 + L%16,
    # bytes 0-7 = K 64kp + 8(L//16).. (block 2kp), bytes 8-15 block 2kp+1
    for r, k in rng.integers(0, [M, K], (200, 2)):
        mt, kb, j = r // 16, k // 32, k % 32
        lane = r % 16 + 16 * (j // 8)
        off = (mt * (K // 64) + kb // 2) * 1024 + lane * 16 + (kb & 1) * 8 + j % 8
        assert pk[off].view(np.int8) == codes[r, k]
    # scales: half ((mt*4 + q)*(K/32) + kb)*4 + i for row mt*16 + 4q + i
    sv = pk[M * K:].view(np.uint16)
    for r, kb in rng.integers(0, [M, K // 32], (200, 2)):
        mt, q, i = r // 16, (r % 16) // 4, r % 4
        assert sv[((mt * 4 + q) * (K // 32) + kb) * 4 + i] == scales[r, kb]
    # a non-finite scale is rejected
    bad = scales.copy()
    bad[5, 3] = 0x7c00
    with pytest.raises(moe.Q36MoEError):
        moe.pack_q8(codes, bad)


def test_quant_q8b_closed_form(oracle):
    rng = np.random.default_rng(12)
    x = (rng.standard_normal(32 * 300) * 2.0 ** rng.integers(-10, 6, 32 * 300)).astype(np.float32)
    x[64:96] = 0.0
    q, d = oracle.quant_q8b(x)
    xb = x.reshape(-1, 32)
    amax = np.abs(xb).max(axis=1)
    np.testing.assert_array_equal(d, (amax / np.float32(127)).astype(np.float32))
    qb = q.reshape(-1, 32).astype(np.int64)
    assert np.all(qb[2] == 0) and d[2] == 0
    assert np.all(np.abs(qb) <= 127)
    inv = np.where(amax > 0, np.float32(127) / np.where(amax > 0, amax, 1), 0).astype(np.float32)
    np.testing.assert_array_equal(qb, np.rint((xb * inv[:, None]).astype(np.float32)).astype(np.int64))


def test_oracle_down_q8_and_layer_composition(oracle):
    rng = np.random.default_rng(13)
    D, FF = 64, 512
    src = synth.kquant_blocks(rng, D, FF, Q5_K)
    codes, scales = oracle.requant_q8(Q5_K, src, D, FF)
    h = rng.standard_normal(FF)
    y = oracle.expert_down_q8(codes, scales, h)
    W = codes.astype(np.float64) * np.repeat(scales.view(np.float16).astype(np.float64), 32, axis=1)
    np.testing.assert_allclose(y, W @ h, rtol=1e-12, atol=1e-12)
    # the layer with a q8 down is routing + expert_h + (q8b h) + this down
    E, Dm, F, T, k = 4, 512, 512, 3, 2
    w = synth.expert_weights(14, n_expert=E, d_model=Dm, d_ff=F)
    dsrc = synth.kquant_blocks(rng, E * Dm, F, Q6_K).reshape(E, Dm, -1)
    dq = np.stack([oracle.requant_q8(Q6_K, dsrc[e], Dm, F)[0] for e in range(E)])
    dd = np.stack([oracle.requant_q8(Q6_K, dsrc[e], Dm, F)[1] for e in range(E)])
    wq = {"gate": w["gate"], "up": w["up"], "down_q8": dq, "down_q8d": dd}
    x = rng.standard_normal((T, Dm)).astype(np.float32)
    lg = rng.standard_normal((T, E)).astype(np.float32)
    got = oracle.moe_forward(wq, x, lg, k=k)
    idx, wt = oracle.router_topk(lg, k)
    xq, xs = oracle.quant_e4m3(x)
    xd = oracle.dequant_e4m3(xq, xs)
    for t in range(T):
        ref = np.zeros(Dm)
        for s in range(k):
            e = idx[t, s]
            hf = oracle.expert_h(w["gate"][e], w["up"][e], xd[t]).astype(np.float32)
            q, hs = oracle.quant_q8b(hf)
            hd = q.astype(np.float64) * np.repeat(hs.astype(np.float64), 32)
            ref += wt[t, s] * oracle.expert_down_q8(dq[e], dd[e], hd)
        np.testing.assert_allclose(got[t], ref, rtol=1e-12, atol=1e-12 * np.abs(ref).max())


def test_upload_typed_rejects_bad_args_without_gpu():
    from q36_amd import moe
    L = moe.lib()
    buf = np.zeros(4096, dtype=np.uint8)
    p = ctypes.c_void_p(buf.ctypes.data)
    out = ctypes.c_void_p()
    # unknown down type; a k-quant with d_ff not a multiple of 256 cannot occur
    # at d_ff % 512 == 0, so an unknown type and null pointers are the cases
    assert L.q36moe_weights_upload_typed(p, p, p, 2, None, None, None, 39, 4, 512, 512, 0, ctypes.byref(out)) == -22
    assert L.q36moe_weights_upload_typed(p, p, None, Q5_K, None, None, None, 39, 4, 512, 512, 0,
                                         ctypes.byref(out)) == -22
    assert L.q36moe_requant_q8(Q5_K, p, 4, 100, p, p) == -22      # K % 256
    assert L.q36moe_requant_q8(30, p, 4, 512, p, p) == -22        # not a k-quant / Q8_0
    assert L.q36moe_weights_down_type(None) == -22


# ---------------------------------------------------------------------------
# GPU: the layer with a q8_0-split routed down, through the C ABI
# ---------------------------------------------------------------------------
TOL = 2e-3
FLOOR = 5e-2


@pytest.fixture(scope="module")
def q8_layer():
    import torch
    from q36_amd import moe
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    w = synth.expert_weights(2027, shared=True)
    rng = np.random.default_rng(2028)
    E, D, FF = synth.N_EXPERT, synth.D_MODEL, synth.D_FF
    down = synth.kquant_blocks(rng, E * D, FF, Q5_K).reshape(E, D, -1)
    dw = moe.MoEWeights.upload(w["gate"], w["up"], down, w["sh_gate"], w["sh_up"], w["sh_down"],
                               down_type=Q5_K)
    assert dw.down_type == Q8_0
    dq = np.empty((E, D, FF), dtype=np.int8)
    dd = np.empty((E, D, FF // 32), dtype=np.uint16)
    for e in range(E):
        dq[e], dd[e] = moe.requant_q8(Q5_K, down[e], D, FF)
    w = dict(w)
    w["down_src"] = down
    w["down_q8"], w["down_q8d"] = dq, dd
    return w, dw


def _oracle_w(w):
    return {k: w[k] for k in ("gate", "up", "sh_gate", "sh_up", "sh_down", "down_q8", "down_q8d")}


# The down rows are staged (for the combine) as f16 with a power-of-two
# scale per 16 columns: each staged term carries a rounding of at most 2^-11
# of itself.  Near outputs where the weighted terms cancel, the element-wise
# bar admits that rounding -- STAGE_SLACK times the sum of |terms| of the
# element -- on top of its own 2e-3.
STAGE_SLACK = 2.0 ** -10


def _row_err(y, ref, absterms=None):
    """(element-wise, normwise) max relative error per row: element-wise
    |y - ref| (less STAGE_SLACK * absterms when given) over max(|ref|, FLOOR *
    rowmax); normwise max |y - ref| / max |ref|."""
    scale = np.abs(ref).max(axis=1, keepdims=True)
    d = np.abs(y - ref)
    if absterms is not None:
        d = np.maximum(d - STAGE_SLACK * absterms, 0.0)
    rel = d / np.maximum(np.abs(ref), FLOOR * scale)
    return float(rel.max()), float((np.abs(y - ref).max(axis=1) / scale[:, 0]).max())


def _q8_0_blocks(codes, scales):
    """Q8_0 blocks (f16 d, 32 int8) holding exactly the q8_0-split matrix."""
    M, K = codes.shape
    blk = np.empty((M, K // 32, 34), dtype=np.uint8)
    blk[:, :, 0:2] = scales.reshape(M, K // 32, 1).view(np.uint8).reshape(M, K // 32, 2)
    blk[:, :, 2:] = codes.reshape(M, K // 32, 32).view(np.uint8)
    return blk.reshape(M, -1)


@pytest.mark.gpu
@pytest.mark.parametrize("ggml_type", [pytest.param(Q5_K, id="q5_k"), pytest.param(Q6_K, id="q6_k")])
@pytest.mark.parametrize("T", [3, 40])
def test_upload_typed_equals_oracle_requant(oracle, ggml_type, T):
    """A k-quant down uploaded through the library's requantiser gives
    bit-identical layer outputs to the oracle's requantisation of the same
    blocks handed over losslessly as Q8_0: the device holds exactly the
    oracle's int8 codes and f16 scales."""
    import torch
    from q36_amd import moe
    rng = np.random.default_rng(300 + ggml_type)
    E, D, FF = 16, 2048, 512
    w = synth.expert_weights(301, n_expert=E)
    down = synth.kquant_blocks(rng, E * D, FF, ggml_type).reshape(E, D, -1)
    q80 = np.stack([_q8_0_blocks(*oracle.requant_q8(ggml_type, down[e], D, FF)) for e in range(E)])
    wa = moe.MoEWeights.upload(w["gate"], w["up"], down, down_type=ggml_type)
    wb = moe.MoEWeights.upload(w["gate"], w["up"], q80, down_type=Q8_0)
    x = torch.from_numpy(synth.hidden(rng, T)).cuda()
    lg = torch.from_numpy(rng.standard_normal((T, E)).astype(np.float32)).cuda()
    outs = []
    for wt in (wa, wb):
        layer = moe.MoELayer(T, n_expert=E)
        outs.append(layer.forward(wt, x, lg, out_dtype=torch.float32).cpu().numpy())
    torch.cuda.synchronize()
    np.testing.assert_array_equal(outs[0], outs[1])
    assert np.abs(outs[0]).max() > 0


def _run(dw, x, lg, shg, path, max_tokens=None):
    import torch
    from q36_amd import moe
    T = x.shape[0]
    layer = moe.MoELayer(max_tokens or max(T, 1))
    layer.set_path(path)
    xt = torch.from_numpy(x).cuda()
    lt = torch.from_numpy(lg).cuda()
    st = torch.from_numpy(shg).cuda() if shg is not None else None
    y32 = layer.forward(dw, xt, lt, st, out_dtype=torch.float32)
    y16 = layer.forward(dw, xt, lt, st, out_dtype=torch.bfloat16)
    layer.check()
    torch.cuda.synchronize()
    return layer, y32.cpu().numpy(), y16.float().cpu().numpy()


def _check_q8_layer(oracle, q8_layer, x, lg, shg, path, sample=None):
    import torch
    from q36_amd import moe
    w, dw = q8_layer
    T, k = x.shape[0], 8
    layer, y32, y16 = _run(dw, x, lg, shg, path)
    y16_ref = torch.from_numpy(y32).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(y16, y16_ref)
    gi, _ = oracle.router_topk(lg, k)
    np.testing.assert_array_equal(layer.tap(moe.TAP_TOPK_IDX).cpu().numpy(), gi)
    _, ow = oracle.router_topk(lg, k)
    toks = np.arange(T) if sample is None else np.asarray(sample)
    pos = layer.tap(moe.TAP_POS).cpu().numpy()
    hq = layer.tap(moe.TAP_HQ).cpu().numpy().view(np.int8)
    hs = layer.tap(moe.TAP_HS).cpu().numpy()
    hsf = layer.tap(moe.TAP_HSF).cpu().numpy()
    xq, xs = oracle.quant_e4m3(x)
    xd = oracle.dequant_e4m3(xq, xs)
    flips = 0
    ref_h = np.zeros((toks.size, x.shape[1]))
    ref_sub = np.zeros((toks.size, x.shape[1]))   # oracle h codes, the GPU's at flips
    absterms = np.zeros_like(ref_h)
    tok_flips = np.zeros(toks.size, dtype=np.int64)
    for j, t in enumerate(toks):
        for s in range(k):
            p, e = int(pos[t * k + s]), int(gi[t, s])
            # stage 1: int8 h of this row vs the oracle's k_quant_q8b of fp32(h)
            hg = oracle.expert_h(w["gate"][e], w["up"][e], xd[t])
            oq, od = oracle.quant_q8b(hg.astype(np.float32))
            # fp32 (GPU) vs fp64 (oracle) accumulation of h: scales agree to
            # 1e-4 relative, codes except within 127e-4 of a rounding midpoint
            np.testing.assert_allclose(hsf[p], od, rtol=1e-4, atol=0)
            bad = np.nonzero(hq[p].astype(np.int64) != oq.astype(np.int64))[0]
            if bad.size:
                v = hg[bad] * 127.0 / np.repeat(np.abs(hg).reshape(-1, 32).max(axis=1), 32)[bad]
                assert np.all(np.abs(np.abs(v - np.floor(v)) - 0.5) <= 127e-4), f"token {t} slot {s}: codes {bad}"
                assert np.all(np.abs(hq[p, bad].astype(np.int64) - oq[bad]) == 1)
                flips += bad.size
                tok_flips[j] += bad.size
            sub = oq.astype(np.float64)
            sub[bad] = hq[p, bad]
            ref_sub[j] += ow[t, s] * oracle.expert_down_q8(w["down_q8"][e], w["down_q8d"][e],
                                                           sub * np.repeat(od.astype(np.float64), 32))
            # stage 2: down from the GPU's own int8 h
            hd = hq[p].astype(np.float64) * np.repeat(hsf[p].astype(np.float64), 32)
            term = ow[t, s] * oracle.expert_down_q8(w["down_q8"][e], w["down_q8d"][e], hd)
            ref_h[j] += term
            absterms[j] += np.abs(term)
        if shg is not None:   # the shared expert stays MXFP4 with e4m3 h
            p = T * k + int(t)
            hd = oracle.dequant_e4m3(hq[p:p + 1].view(np.uint8), hs[p:p + 1])[0]
            term = 1 / (1 + np.exp(-float(shg[t]))) * oracle.expert_down(w["sh_down"], hd)
            ref_h[j] += term
            ref_sub[j] += term
            absterms[j] += np.abs(term)
    el_h, norm_h = _row_err(y32[toks], ref_h, absterms)
    # end to end: tokens without flipped routed h codes against the plain
    # oracle; the others against the oracle with the GPU's codes at the flips
    # (the shared expert's MXFP4 h is the GPU's in both; its parity is held by
    # the MXFP4 layer tests)
    ref = oracle.moe_forward(_oracle_w(w), x, lg, shg, tokens=toks.astype(np.int32))
    if shg is not None:
        ref = ref_sub.copy()
    else:
        ref[tok_flips > 0] = ref_sub[tok_flips > 0]
    el, e2e = _row_err(y32[toks], ref, absterms)
    assert flips <= 0.01 * toks.size * k * 512
    assert norm_h <= TOL and el_h <= TOL, f"down/combine error {norm_h:.3g} / {el_h:.3g}"
    assert e2e <= TOL and el <= TOL, f"end-to-end error {e2e:.3g} / {el:.3g}"
    return layer


Q8_PATHS = [(1, 0), (1, 2), (5, 2), (16, 0), (40, 4), (40, 5), (40, 1), (200, 1), (600, 0)]


@pytest.mark.gpu
@pytest.mark.parametrize("T,path", Q8_PATHS)
@pytest.mark.parametrize("shared", [False, True])
def test_forward_q8_down(oracle, q8_layer, T, path, shared):
    rng = np.random.default_rng(400 + T + path)
    x = synth.hidden(rng, T)
    lg = synth.normal_logits(rng, T)
    shg = rng.standard_normal(T).astype(np.float32) if shared else None
    sample = None if T <= 40 else rng.choice(T, 24, replace=False)
    layer = _check_q8_layer(oracle, q8_layer, x, lg, shg, path, sample)
    # int8 layers keep two skinny kernels: mode 5 (one kernel per tile) falls back to 4
    assert layer.last_path == (1 if (path == 2 or (path == 0 and T <= 16)) else 2 if path in (4, 5) or
                               (path == 0 and T * 8 <= 8 * 256) else 0)


@pytest.mark.gpu
def test_forward_q8_down_zipf_ragged(oracle, q8_layer):
    rng = np.random.default_rng(450)
    x = synth.hidden(rng, 64)
    lg = synth.zipf_logits(rng, 64)
    _check_q8_layer(oracle, q8_layer, x, lg, None, 0)


@pytest.mark.gpu
def test_q8_down_path_and_replay_format_checks(q8_layer):
    import torch
    from q36_amd import moe
    w, dw = q8_layer
    rng = np.random.default_rng(460)
    x = torch.from_numpy(synth.hidden(rng, 2)).cuda()
    lg = torch.from_numpy(synth.normal_logits(rng, 2)).cuda()
    layer = moe.MoELayer(4)
    with pytest.raises(moe.Q36MoEError):
        layer.set_path(3)   # the one-kernel decode mode no longer exists
    layer.forward(dw, x, lg)
    # a plan made for a q8 down does not replay over MXFP4 weights
    mx = moe.MoEWeights.upload(w["gate"], w["up"], synth.expert_weights(2027)["down"])
    with pytest.raises(moe.Q36MoEError):
        layer.replay(mx, 3)
    layer.replay(dw, 3)
    torch.cuda.synchronize()


# ---------------------------------------------------------------------------
# q8_0-split shared expert (the release file's Q8_0 _shexp tensors)
# ---------------------------------------------------------------------------
def _shared_q8(oracle, rng, D=2048, FF=512, src_type=Q8_0):
    """Shared gate/up/down as GGUF blocks of src_type and their q8_0-split form."""
    blocks = {"sh_gate": synth.kquant_blocks(rng, FF, D, src_type),
              "sh_up": synth.kquant_blocks(rng, FF, D, src_type),
              "sh_down": synth.kquant_blocks(rng, D, FF, src_type)}
    split = {}
    for k, (M, K) in (("sh_gate", (FF, D)), ("sh_up", (FF, D)), ("sh_down", (D, FF))):
        split[k + "_q8"], split[k + "_q8d"] = oracle.requant_q8(src_type, blocks[k], M, K)
    return blocks, split


def test_oracle_shared_q8_composition(oracle):
    rng = np.random.default_rng(21)
    E, Dm, F, T, k = 4, 512, 512, 3, 2
    w = synth.expert_weights(22, n_expert=E, d_model=Dm, d_ff=F)
    _, sq = _shared_q8(oracle, rng, Dm, F)
    wq = {"gate": w["gate"], "up": w["up"], "down": w["down"], **sq}
    x = rng.standard_normal((T, Dm)).astype(np.float32)
    lg = rng.standard_normal((T, E)).astype(np.float32)
    shg = rng.standard_normal(T).astype(np.float32)
    got = oracle.moe_forward(wq, x, lg, shg, k=k)
    routed = oracle.moe_forward({"gate": w["gate"], "up": w["up"], "down": w["down"]}, x, lg, k=k)
    for t in range(T):
        q, s = oracle.quant_q8b(x[t])
        xd = q.astype(np.float64) * np.repeat(s.astype(np.float64), 32)
        hf = oracle.expert_h_q8(sq["sh_gate_q8"], sq["sh_gate_q8d"], sq["sh_up_q8"], sq["sh_up_q8d"],
                                xd).astype(np.float32)
        hq, hs = oracle.quant_q8b(hf)
        hd = hq.astype(np.float64) * np.repeat(hs.astype(np.float64), 32)
        ysh = oracle.expert_down_q8(sq["sh_down_q8"], sq["sh_down_q8d"], hd)
        ref = routed[t] + ysh / (1 + np.exp(-float(shg[t])))
        np.testing.assert_allclose(got[t], ref, rtol=1e-12, atol=1e-12 * np.abs(ref).max())


def test_upload_typed_rejects_bad_shared_type_without_gpu():
    from q36_amd import moe
    L = moe.lib()
    buf = np.zeros(4096, dtype=np.uint8)
    p = ctypes.c_void_p(buf.ctypes.data)
    out = ctypes.c_void_p()
    assert L.q36moe_weights_upload_typed(p, p, p, 39, p, p, p, 30, 4, 512, 512, 512, ctypes.byref(out)) == -22
    assert L.q36moe_weights_upload_typed(p, p, p, 39, p, None, p, 8, 4, 512, 512, 512, ctypes.byref(out)) == -22
    assert L.q36moe_weights_shared_type(None) == -22


@pytest.fixture(scope="module")
def q8_shared_layer(oracle):
    import torch
    from q36_amd import moe
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    w = synth.expert_weights(2031)
    rng = np.random.default_rng(2032)
    blocks, sq = _shared_q8(oracle, rng)
    E, D, FF = synth.N_EXPERT, synth.D_MODEL, synth.D_FF
    down = synth.kquant_blocks(rng, E * D, FF, Q6_K).reshape(E, D, -1)
    dq = np.empty((E, D, FF), dtype=np.int8)
    dd = np.empty((E, D, FF // 32), dtype=np.uint16)
    for e in range(E):
        dq[e], dd[e] = oracle.requant_q8(Q6_K, down[e], D, FF)
    # the same routed experts with an MXFP4 down (shared Q8 alone) and with a Q6_K down (both)
    dw_mx = moe.MoEWeights.upload(w["gate"], w["up"], w["down"], blocks["sh_gate"], blocks["sh_up"],
                                  blocks["sh_down"], sh_type=Q8_0)
    dw_both = moe.MoEWeights.upload(w["gate"], w["up"], down, blocks["sh_gate"], blocks["sh_up"],
                                    blocks["sh_down"], down_type=Q6_K, sh_type=Q8_0)
    assert dw_mx.shared_type == Q8_0 and dw_mx.down_type == 39
    assert dw_both.shared_type == Q8_0 and dw_both.down_type == Q8_0
    return {"w": w, "sq": sq, "dq": dq, "dd": dd, "mx": dw_mx, "both": dw_both}


def _check_shared_q8(oracle, L, which, T, path, seed):
    import torch
    from q36_amd import moe
    w, sq = L["w"], L["sq"]
    dw = L[which]
    k = 8
    rng = np.random.default_rng(seed)
    x = synth.hidden(rng, T)
    lg = synth.normal_logits(rng, T)
    shg = rng.standard_normal(T).astype(np.float32)
    layer, y32, y16 = _run(dw, x, lg, shg, path)
    np.testing.assert_array_equal(y16, torch.from_numpy(y32).to(torch.bfloat16).float().numpy())
    gi, ow = oracle.router_topk(lg, k)
    np.testing.assert_array_equal(layer.tap(moe.TAP_TOPK_IDX).cpu().numpy(), gi)
    if layer.last_path != 1:   # sorted path: the int8 x the shared expert reads, bit-exact
        q, s = zip(*[oracle.quant_q8b(x[t]) for t in range(T)])
        np.testing.assert_array_equal(layer.tap(moe.TAP_XQ8).cpu().numpy(), np.stack(q))
        np.testing.assert_array_equal(layer.tap(moe.TAP_XSF).cpu().numpy(), np.stack(s))
    toks = np.arange(T) if T <= 40 else rng.choice(T, 24, replace=False)
    pos = layer.tap(moe.TAP_POS).cpu().numpy()
    hq = layer.tap(moe.TAP_HQ).cpu().numpy()
    hs = layer.tap(moe.TAP_HS).cpu().numpy()
    hsf = layer.tap(moe.TAP_HSF).cpu().numpy()
    ref_h = np.zeros((toks.size, x.shape[1]))
    absterms = np.zeros_like(ref_h)
    flips = 0
    for j, t in enumerate(toks):
        for s in range(k):
            p, e = int(pos[t * k + s]), int(gi[t, s])
            if which == "both":
                hd = hq[p].view(np.int8).astype(np.float64) * np.repeat(hsf[p].astype(np.float64), 32)
                y = oracle.expert_down_q8(L["dq"][e], L["dd"][e], hd)
            else:
                hd = oracle.dequant_e4m3(hq[p:p + 1], hs[p:p + 1])[0]
                y = oracle.expert_down(w["down"][e], hd)
            ref_h[j] += ow[t, s] * y
            absterms[j] += np.abs(ow[t, s] * y)
        # the shared row: int8 h vs the oracle's q8b of fp32(h), then its down
        p = T * k + int(t)
        qx, sx = oracle.quant_q8b(x[t])
        xd = qx.astype(np.float64) * np.repeat(sx.astype(np.float64), 32)
        hg = oracle.expert_h_q8(sq["sh_gate_q8"], sq["sh_gate_q8d"], sq["sh_up_q8"], sq["sh_up_q8d"], xd)
        oq, od = oracle.quant_q8b(hg.astype(np.float32))
        np.testing.assert_allclose(hsf[p], od, rtol=1e-4, atol=0)
        bad = np.nonzero(hq[p].view(np.int8).astype(np.int64) != oq.astype(np.int64))[0]
        if bad.size:
            v = hg[bad] * 127.0 / np.repeat(np.abs(hg).reshape(-1, 32).max(axis=1), 32)[bad]
            assert np.all(np.abs(np.abs(v - np.floor(v)) - 0.5) <= 127e-4), f"token {t}: shared codes {bad}"
            flips += bad.size
        hd = hq[p].view(np.int8).astype(np.float64) * np.repeat(hsf[p].astype(np.float64), 32)
        term = oracle.expert_down_q8(sq["sh_down_q8"], sq["sh_down_q8d"], hd) / (1 + np.exp(-float(shg[t])))
        ref_h[j] += term
        absterms[j] += np.abs(term)
    el_h, norm_h = _row_err(y32[toks], ref_h, absterms)
    ow_ = {"gate": w["gate"], "up": w["up"], **sq}
    if which == "both":
        ow_.update(down_q8=L["dq"], down_q8d=L["dd"])
    else:
        ow_["down"] = w["down"]
    ref = oracle.moe_forward(ow_, x, lg, shg, tokens=toks.astype(np.int32))
    _, e2e = _row_err(y32[toks], ref)
    assert flips <= 0.01 * toks.size * 512
    assert norm_h <= TOL and el_h <= TOL, f"down/combine error {norm_h:.3g} / {el_h:.3g}"
    assert e2e <= 1e-2, f"end-to-end max relative error {e2e:.3g}"


@pytest.mark.gpu
@pytest.mark.parametrize("which", ["mx", "both"])
@pytest.mark.parametrize("T,path", [(1, 0), (5, 2), (40, 4), (40, 1), (600, 0)])
def test_forward_q8_shared(oracle, q8_shared_layer, which, T, path):
    _check_shared_q8(oracle, q8_shared_layer, which, T, path, 500 + T + path)


@pytest.mark.gpu
def test_q8_shared_refusals(q8_shared_layer):
    import torch
    from q36_amd import moe
    dw = q8_shared_layer["mx"]
    rng = np.random.default_rng(510)
    x = torch.from_numpy(synth.hidden(rng, 2)).cuda()
    lg = torch.from_numpy(synth.normal_logits(rng, 2)).cuda()
    shg = torch.from_numpy(rng.standard_normal(2).astype(np.float32)).cuda()
    layer = moe.MoELayer(4)
    xq, xs = moe.quant_e4m3(x)
    with pytest.raises(moe.Q36MoEError):     # int8 x needs the unquantised input
        layer.forward_q8(dw, xq, xs, lg, shg)
    layer.forward_q8(dw, xq, xs, lg)          # without the shared expert it is fine
    torch.cuda.synchronize()


@pytest.mark.gpu
@pytest.mark.parametrize("T", [1, 40, 600])
def test_q8_layer_in_hip_graph(q8_shared_layer, T):
    """The release-file layout (Q6_K routed down, Q8_0 shared expert)
    captured in a HIP graph: every replay, with eager forwards of other
    inputs and synchronisations between, equals the eager result bit for bit
    (direct, skinny and fat sorted paths)."""
    import torch
    from q36_amd import moe
    dw = q8_shared_layer["both"]
    rng = np.random.default_rng(1100 + T)
    x = torch.from_numpy(synth.hidden(rng, T)).cuda()
    lg = torch.from_numpy(synth.normal_logits(rng, T)).cuda()
    shg = torch.from_numpy(rng.standard_normal(T).astype(np.float32)).cuda()
    x2 = torch.from_numpy(synth.hidden(rng, T)).cuda()
    lg2 = torch.from_numpy(synth.normal_logits(rng, T)).cuda()
    layer = moe.MoELayer(T)
    out = torch.empty((T, 2048), dtype=torch.float32, device="cuda")
    ref = layer.forward(dw, x, lg, shg, out_dtype=torch.float32).clone()
    cap = torch.cuda.Stream()
    layer.set_stream(cap)
    with torch.cuda.stream(cap):
        layer.forward(dw, x, lg, shg, out=out)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=cap):
        layer.forward(dw, x, lg, shg, out=out)
    torch.cuda.synchronize()
    layer.set_stream(torch.cuda.current_stream())
    for rep in range(4):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {rep}"
        other = layer.forward(dw, x2, lg2, shg, out_dtype=torch.float32)
        torch.cuda.synchronize()
        assert not torch.equal(other, ref)
