"""GPU parity of the HIP path against the CPU oracle, called through the C ABI
(q36_amd.moe is a thin ctypes mirror).  Bars:
  * routing indices, sort offsets / permutation, FP8 activation codes and
    E8M0 scales: bit-exact;
  * routing weights: |dw| <= 2e-6 * w (fp32 exp/div vs fp64);
  * staged layer parity, per token row t (fp32 result, before bf16 rounding):
      1. gate/up + SwiGLU + h quantisation: GPU e4m3 codes / E8M0 scales equal
         the oracle's quantisation of fp32(h) except at rounding midpoints
         (fp32 vs fp64 accumulation), counted and capped at 1%;
      2. down + combine from the GPU's own h rows vs fp64:
           max relative error  max_i |y_ti - ref_ti| / max_i |ref_ti|   <= 2e-3
           element-wise  |y_ti - ref_ti| / max(|ref_ti|, 0.05 max_i |ref_ti|) <= 2e-3,
           less 2^-10 * sum_s |w_s d_s|_i (the combine stages the weighted down
           rows as f16 with a power-of-two scale per 16 columns: <= 2^-11 of
           each term)
      3. end to end vs the fp64 oracle, the same two 2e-3 bars, per token:
         a token none of whose h rows has a midpoint flip is held against
         the plain oracle (q36moe_oracle.c, its own fp64 path); a token with
         flips against the oracle with the GPU's code substituted at each
         flipped element only (everything else of that reference is the
         oracle's own arithmetic; stage 1 has shown every other code equal),
         because one legitimate flip of a large h code (up to 1/16 of the
         value) moves outputs by up to ~2e-3 of the row max;
    an element-wise bound needs the floor near zero, and bf16's own half-ulp
    is up to 2^-8 relative, above 2e-3, so the bars apply to the fp32 result;
  * bf16 output: the RNE bf16 rounding of the f32 output, bit for bit.
"""
import json
import os

import numpy as np
import pytest
import torch

from q36_amd import moe, synth

import fullcheck

pytestmark = pytest.mark.gpu

TOL = 2e-3
FLOOR = 5e-2
_LAST_METRICS = {}


def _metrics(name, **kv):
    path = os.environ.get("Q36_METRICS_FILE")
    if path:
        with open(path, "a") as f:
            f.write(json.dumps({"test": name, **kv}) + "\n")


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    return torch.device("cuda:0")


# ---------------------------------------------------------------------------
# MFMA calibration (the analogue of test_mma_bs.cu for gfx950)
# ---------------------------------------------------------------------------
E2M1 = np.array([0, .5, 1, 1.5, 2, 3, 4, 6, -0., -.5, -1, -1.5, -2, -3, -4, -6])


def _e4m3_table():
    return torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).double().numpy()


def _fp4_k(q, n):
    return 32 * q + n


def _fp8_k(q, i):
    return 64 * (i >> 4) + 16 * q + (i & 15)


def _interp(lanes, scales, fmt, tab, transpose):
    """Logical operand [16][128] (A) or [128][16] (B) from lane bytes, with
    the gfx950 layout: E2M1 lane group q holds K 32q..32q+31 (nibble n -> K
    32q+n); E4M3 byte i of lane group q holds K 64*(i>>4)+16q+(i&15); the scale
    of K block kb comes from lane group kb."""
    M = np.zeros((16, 128))
    for L in range(64):
        r, q = L % 16, L // 16
        for i in range(32):
            if fmt == 4:
                byte = lanes[L, i // 2]
                code = (byte >> 4) if (i & 1) else (byte & 15)
                k, v = _fp4_k(q, i), E2M1[code]
            else:
                k, v = _fp8_k(q, i), tab[lanes[L, i]]
            M[r, k] = v * 2.0 ** (int(scales[r + 16 * (k // 32)] & 255) - 127)
    return M.T if transpose else M


def _lanes(C):
    out = np.zeros((64, 4))
    for L in range(64):
        for i in range(4):
            out[L, i] = C[4 * (L // 16) + i, L % 16]
    return out


def _rand_fp8(rng, shape):
    b = rng.integers(0, 256, size=shape).astype(np.uint8)
    b[(b & 0x7F) == 0x7F] = 0x38
    return b


@pytest.mark.parametrize("fmt_a,spread", [(4, True), (0, True), (4, False), (0, False)])
def test_mfma_probe_layout(dev, fmt_a, spread):
    """Calibrates the operand / scale / output layout of the scaled MFMA the
    kernels use (the role of test_mma_bs.cu on sm_120a): random codes and
    scales, upper scale bytes random to show that only byte 0 is read."""
    rng = np.random.default_rng(100 + fmt_a)
    tab = _e4m3_table()
    if fmt_a == 4:
        codes = rng.integers(0, 16, size=(64, 32)).astype(np.uint8)
        a_lane = np.zeros((64, 32), dtype=np.uint8)
        a_lane[:, :16] = codes[:, 0::2] | (codes[:, 1::2] << 4)
    else:
        a_lane = _rand_fp8(rng, (64, 32))
    b_lane = _rand_fp8(rng, (64, 32))
    hi = lambda: rng.integers(0, 1 << 24, size=64).astype(np.uint32) << 8
    lo, hi_e = (120, 135) if spread else (127, 128)
    sa = rng.integers(lo, hi_e, size=64).astype(np.uint32) | hi()
    sb = rng.integers(lo, hi_e, size=64).astype(np.uint32) | hi()
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    c = moe.probe_mfma(t(a_lane), t(b_lane), t(sa.view(np.int32)), t(sb.view(np.int32)), fmt_a, 0)
    got = c.double().cpu().numpy()
    A = _interp(a_lane, sa, fmt_a, tab, False)
    B = _interp(b_lane, sb, 0, tab, True)
    want = _lanes(A @ B)
    err = np.abs(got - want).max() / np.abs(want).max()
    _metrics("mfma_probe", fmt_a=fmt_a, spread=spread, err=float(err))
    # a wrong layout gives O(1) errors.  The MFMA's internal accumulation of
    # full-range e4m3 products is not exact fp32: ~5e-5 of max|C| measured on
    # gfx950 with either scale range, so the bar is 2e-4.
    assert err < 2e-4, err


def _interp32(a_lane, sa, b_lane, sb, tab):
    """Logical A [32][64] (e2m1) and B [64][32] (e4m3) of the 32x32x64 scaled
    MFMA from lane bytes, gfx950 layout: A lane L holds row L%32, K
    32(L/32)..+31 (nibble j -> K 32(L/32)+j); B lane L holds column L%32,
    bytes 0-15 K 16(L/32)..+15 and bytes 16-31 K 32+16(L/32)..+15; K block kb
    (32 K) is scaled by lane row/col + 32kb."""
    A = np.zeros((32, 64))
    B = np.zeros((64, 32))
    for L in range(64):
        h = L // 32
        for j in range(32):
            byte = a_lane[L, j // 2]
            A[L % 32, 32 * h + j] = E2M1[(byte >> 4) if (j & 1) else (byte & 15)]
            k = 16 * h + j if j < 16 else 32 + 16 * h + j - 16
            B[k, L % 32] = tab[b_lane[L, j]]
    for kb in range(2):
        A[:, 32 * kb:32 * kb + 32] *= (2.0 ** (np.int64(sa[32 * kb:32 * kb + 32] & 255) - 127))[:, None]
        B[32 * kb:32 * kb + 32, :] *= (2.0 ** (np.int64(sb[32 * kb:32 * kb + 32] & 255) - 127))[None, :]
    return A, B


@pytest.mark.parametrize("spread", [True, False])
def test_mfma32_probe_layout(dev, spread):
    """Calibrates v_mfma_scale_f32_32x32x64_f8f6f4 (A e2m1, B e4m3), the tile
    of the fat gate/up: operand, scale and output layout (C lane L holds
    column L%32, result i is row 8(i/4) + 4(L/32) + i%4)."""
    rng = np.random.default_rng(200 + spread)
    tab = _e4m3_table()
    codes = rng.integers(0, 16, size=(64, 32)).astype(np.uint8)
    a_lane = np.zeros((64, 32), dtype=np.uint8)
    a_lane[:, :16] = codes[:, 0::2] | (codes[:, 1::2] << 4)
    b_lane = _rand_fp8(rng, (64, 32))
    hi = lambda: rng.integers(0, 1 << 24, size=64).astype(np.uint32) << 8
    lo, hi_e = (120, 135) if spread else (127, 128)
    sa = rng.integers(lo, hi_e, size=64).astype(np.uint32) | hi()
    sb = rng.integers(lo, hi_e, size=64).astype(np.uint32) | hi()
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(dev)
    got = moe.probe_mfma32(t(a_lane), t(b_lane), t(sa.view(np.int32)), t(sb.view(np.int32))).double().cpu().numpy()
    A, B = _interp32(a_lane, sa, b_lane, sb, tab)
    C = A @ B
    want = np.array([[C[8 * (i // 4) + 4 * (L // 32) + i % 4, L % 32] for i in range(16)] for L in range(64)])
    err = np.abs(got - want).max() / np.abs(want).max()
    _metrics("mfma32_probe", spread=spread, err=float(err))
    # a wrong layout gives O(1) errors; the MFMA's own accumulation of
    # full-range e4m3 products read up to 1.2e-4 of max|C| over six random
    # probes on gfx950, so the bar is 5e-4
    assert err < 5e-4, err


# ---------------------------------------------------------------------------
# stage entry points
# ---------------------------------------------------------------------------
def _quant_inputs(rng):
    x = (rng.standard_normal((64, 2048)) * 10.0 ** rng.uniform(-4, 4, (64, 1))).astype(np.float32)
    x[0, :32] = 0.0
    x[1, :32] = 1e-40
    x[2, :64] = np.float32(2.0 ** -5) * np.float32(1 + 2.0 ** -23) * 448   # log2 edge amax
    # exact e4m3 midpoints after scaling (amax 448 -> e2 = 0)
    tab = _e4m3_table()
    fin = np.sort(np.unique(tab[np.isfinite(tab) & (tab >= 0)]))
    mids = ((fin[:-1] + fin[1:]) / 2).astype(np.float32)
    x[3, :] = np.resize(np.concatenate([[448.0], mids]), 2048)
    x[3, ::32] = 448.0
    # non-finite values: +-inf blocks (scale byte 254, finite codes 0, the
    # infinite element NaN as the reference's saturating conversion gives),
    # NaN elements (ignored by the block maximum, coded 0x7f)
    x[4, 5] = np.inf
    x[4, 40] = -np.inf
    x[5, 7] = np.nan
    x[5, 100] = -np.nan
    x[6, :32] = np.float32(3.0e38)
    return x


def test_quant_stage_bit_exact(dev, oracle):
    rng = np.random.default_rng(21)
    x = _quant_inputs(rng)
    xq, xs = moe.quant_e4m3(torch.from_numpy(x).to(dev))
    oq, os_ = oracle.quant_e4m3(x)
    np.testing.assert_array_equal(xs.cpu().numpy(), os_)
    np.testing.assert_array_equal(xq.cpu().numpy(), oq)
    # bf16 input: the oracle sees the same values widened to f32
    xb = torch.from_numpy(x).to(dev).to(torch.bfloat16)
    bq, bs = moe.quant_e4m3(xb)
    oq, os_ = oracle.quant_e4m3(xb.float().cpu().numpy())
    np.testing.assert_array_equal(bs.cpu().numpy(), os_)
    np.testing.assert_array_equal(bq.cpu().numpy(), oq)


@pytest.mark.parametrize("E,ld,k", [(256, 256, 8), (256, 257, 8), (100, 128, 4), (64, 64, 1)])
def test_router_stage(dev, oracle, E, ld, k):
    rng = np.random.default_rng(22 + E + k)
    T = 300
    lg = rng.standard_normal((T, ld)).astype(np.float32)
    lg[0] = 0.25
    lg[1, 5:40] = 2.0
    lg[2] = np.round(lg[2] * 2) / 2
    idx, wt = moe.router_topk(torch.from_numpy(lg).to(dev), k=k, n_expert=E)
    oi, ow = oracle.router_topk(lg, k, n_expert=E)
    np.testing.assert_array_equal(idx.cpu().numpy(), oi)
    err = np.abs(wt.cpu().double().numpy() - ow) / ow
    _metrics("router_stage", E=E, k=k, max_rel_w=float(err.max()))
    assert err.max() <= 2e-6


# ---------------------------------------------------------------------------
# the layer
# ---------------------------------------------------------------------------
@pytest.fixture(scope="module")
def layer_w():
    w = synth.expert_weights(2026, shared=True)
    dw = moe.MoEWeights.upload(w["gate"], w["up"], w["down"], w["sh_gate"], w["sh_up"], w["sh_down"])
    return w, dw


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


def _bf16_of(y32):
    return torch.from_numpy(y32.astype(np.float32)).to(torch.bfloat16).float().numpy()


def _run_layer(dev, dw, x, lg, shg, max_tokens=None, x_dtype=torch.float32, path=0):
    T = x.shape[0]
    layer = moe.MoELayer(max_tokens or max(T, 1))
    layer.set_path(path)
    xt = torch.from_numpy(x).to(dev).to(x_dtype)
    lt = torch.from_numpy(lg).to(dev)
    st = torch.from_numpy(shg).to(dev) if shg is not None else None
    y32 = layer.forward(dw, xt, lt, st, out_dtype=torch.float32)
    y16 = layer.forward(dw, xt, lt, st, out_dtype=torch.bfloat16)
    layer.check()
    torch.cuda.synchronize()
    return layer, y32.cpu().numpy(), y16.float().cpu().numpy()


def _check_routing(layer, oracle, lg, E=256, k=8):
    oi, ow = oracle.router_topk(lg, k)
    gi = layer.tap(moe.TAP_TOPK_IDX).cpu().numpy()
    np.testing.assert_array_equal(gi, oi)
    gw = layer.tap(moe.TAP_TOPK_W).cpu().double().numpy()
    assert np.abs(gw - ow).max() <= 2e-6
    if layer.last_path in (0, 2, 3):   # sorted paths: offsets and permutation bit-exact
        off, perm, pos = oracle.sort_entries(gi, E)
        np.testing.assert_array_equal(layer.tap(moe.TAP_EOFF).cpu().numpy(), off)
        np.testing.assert_array_equal(layer.tap(moe.TAP_PERM).cpu().numpy(), perm)
        np.testing.assert_array_equal(layer.tap(moe.TAP_POS).cpu().numpy(), pos)
    else:                           # direct path: rows stay in entry order
        ident = np.arange(gi.size, dtype=np.int32)
        np.testing.assert_array_equal(layer.tap(moe.TAP_PERM).cpu().numpy(), ident)
        np.testing.assert_array_equal(layer.tap(moe.TAP_POS).cpu().numpy(), ident)
    return gi


def _fp8_mid_distance(v):
    """Distance of |v| (in fp8 units) to the nearest e4m3 rounding midpoint."""
    tab = _e4m3_table()
    fin = np.sort(np.unique(np.abs(tab[np.isfinite(tab)])))
    mids = (fin[:-1] + fin[1:]) / 2
    a = np.abs(v)
    return np.abs(a[:, None] - mids[None, :]).min(axis=1)


def _check_h_rows(oracle, w, x, gi, perm, hq, hs, rows, n_expert=256, k=8):
    """Gate/up + SwiGLU + h quantisation, row by row: the GPU's e4m3 codes and
    E8M0 scales equal the oracle's quantisation of fp32(h), except codes whose
    fp64 value lies within 1e-4 * blockmax of a rounding midpoint (fp32 vs
    fp64 accumulation order) and scales whose block amax lies within 1e-4 of a
    power-of-two boundary.  Returns {row: (flips, codes, scales)}: the number
    of such flips in the row and the oracle's codes / scales of the row with
    the GPU's value substituted at each flipped element (a flipped scale
    substitutes its block)."""
    xq, xs = oracle.quant_e4m3(x)
    xd = oracle.dequant_e4m3(xq, xs)
    out = {}
    T = x.shape[0]
    for p in rows:
        if p < T * k:
            i = perm[p]
            t, e = i // k, gi[i // k, i % k]
            hg = oracle.expert_h(w["gate"][e], w["up"][e], xd[t])
        else:
            t = p - T * k
            hg = oracle.expert_h(w["sh_gate"], w["sh_up"], xd[t])
        oq, os_ = oracle.quant_e4m3(hg.astype(np.float32)[None])
        oq, os_ = oq[0].copy(), os_[0].copy()
        flips = 0
        for b in range(hg.size // 32):
            sl = slice(32 * b, 32 * b + 32)
            if hs[p, b] != os_[b]:
                amax = np.abs(hg[sl]).max() / 448.0
                rel = abs(amax / 2.0 ** np.round(np.log2(amax)) - 1)
                assert rel < 1e-4, f"row {p} block {b}: scale {hs[p, b]} vs {os_[b]}"
                flips += 1
                os_[b], oq[sl] = hs[p, b], hq[p, sl]
                continue
            bad = np.nonzero(hq[p, sl] != oq[sl])[0]
            if bad.size:
                v = hg[sl] * 2.0 ** -(int(os_[b]) - 127)
                d = _fp8_mid_distance(v[bad])
                assert np.all(d <= 1e-4 * np.abs(v).max()), f"row {p} block {b}: codes {bad}"
                flips += bad.size
                oq[32 * b + bad] = hq[p, 32 * b + bad]
        out[p] = (flips, oq, os_)
    return out


def _check_layer(name, dev, oracle, layer_w, x, lg, shg, sample=None, x_dtype=torch.float32,
                 path=0, every_token=False):
    """Staged parity on the sampled tokens through the C oracle's per-token
    path; with every_token, also all three stages on every token through the
    expert-grouped fp64 reference (tests/fullcheck.py)."""
    w, dw = layer_w
    T = x.shape[0]
    layer, y32, y16 = _run_layer(dev, dw, x, lg, shg, x_dtype=x_dtype, path=path)
    name = f"{name}/{({1: 'direct', 2: 'sorted_skinny', 3: 'sorted_fused'}).get(layer.last_path, 'sorted')}"
    gi = _check_routing(layer, oracle, lg)
    oq, os_ = oracle.quant_e4m3(x)
    np.testing.assert_array_equal(layer.tap(moe.TAP_XQ).cpu().numpy(), oq)
    np.testing.assert_array_equal(layer.tap(moe.TAP_XS).cpu().numpy(), os_)
    # bf16 output is the RNE rounding of the f32 output
    np.testing.assert_array_equal(y16, _bf16_of(y32))
    toks = np.arange(T, dtype=np.int32) if sample is None else np.asarray(sample, np.int32)
    perm = layer.tap(moe.TAP_PERM).cpu().numpy()
    pos = layer.tap(moe.TAP_POS).cpu().numpy()
    hq = layer.tap(moe.TAP_HQ).cpu().numpy()
    hs = layer.tap(moe.TAP_HS).cpu().numpy()
    # stage 1: gate/up/SwiGLU/h quantisation on the rows of the sampled tokens
    rows = [int(pos[t * 8 + s]) for t in toks for s in range(8)]
    if shg is not None:
        rows += [T * 8 + int(t) for t in toks]
    hrows = _check_h_rows(oracle, w, x, gi, perm, hq, hs, rows)
    flips = sum(v[0] for v in hrows.values())
    # stage 2: down + combine from the GPU's own h
    _, ow = oracle.router_topk(lg, 8)
    ref_h = np.zeros((toks.size, x.shape[1]))
    absterms = np.zeros_like(ref_h)
    for j, t in enumerate(toks):
        for s in range(8):
            p = int(pos[t * 8 + s])
            hd = oracle.dequant_e4m3(hq[p:p + 1], hs[p:p + 1])[0]
            term = ow[t, s] * oracle.expert_down(w["down"][gi[t, s]], hd)
            ref_h[j] += term
            absterms[j] += np.abs(term)
        if shg is not None:
            p = T * 8 + int(t)
            hd = oracle.dequant_e4m3(hq[p:p + 1], hs[p:p + 1])[0]
            term = 1 / (1 + np.exp(-float(shg[t]))) * oracle.expert_down(w["sh_down"], hd)
            ref_h[j] += term
            absterms[j] += np.abs(term)
    el_h, norm_h = _row_err(y32[toks], ref_h, absterms)
    # stage 3: end to end, per token: the plain fp64 oracle for tokens without
    # flips, the oracle with the flipped codes substituted for the others
    ref = oracle.moe_forward(w, x, lg, shg, tokens=toks)
    tok_rows = {int(t): [int(pos[t * 8 + s]) for s in range(8)] + ([T * 8 + int(t)] if shg is not None else [])
                for t in toks}
    ref_sub = ref.copy()
    n_flipped_tok = 0
    for j, t in enumerate(toks):
        if sum(hrows[p][0] for p in tok_rows[int(t)]) == 0:
            continue
        n_flipped_tok += 1
        ref_sub[j] = 0.0
        for s in range(8):
            p = int(pos[t * 8 + s])
            hd = oracle.dequant_e4m3(hrows[p][1][None], hrows[p][2][None])[0]
            ref_sub[j] += ow[t, s] * oracle.expert_down(w["down"][gi[t, s]], hd)
        if shg is not None:
            p = T * 8 + int(t)
            hd = oracle.dequant_e4m3(hrows[p][1][None], hrows[p][2][None])[0]
            ref_sub[j] += 1 / (1 + np.exp(-float(shg[t]))) * oracle.expert_down(w["sh_down"], hd)
    el, normwise = _row_err(y32[toks], ref_sub, absterms)
    _, raw_norm = _row_err(y32[toks], ref)
    _, bf16_norm = _row_err(y16[toks], ref_sub)
    # distance from the reference's own numeric paths (reported, not a bar):
    # W4A32 (its decode matvecs) and e4m3 x with fp16 h (its prefill GEMMs)
    ref32 = oracle.moe_forward(w, x, lg, shg, act_mode=1, tokens=toks)
    refpf = oracle.moe_forward(w, x, lg, shg, act_mode=2, tokens=toks)
    drift = float(np.abs(ref32 - ref).max() / np.abs(ref).max())
    _, drift_w4a32 = _row_err(y32[toks], ref32)
    _, drift_prefill = _row_err(y32[toks], refpf)
    global _LAST_METRICS
    _LAST_METRICS = dict(e2e_max_rel=normwise, drift_vs_ref_decode_w4a32=drift_w4a32,
                         drift_vs_ref_prefill_fp16h=drift_prefill)
    _metrics(name, T=int(T), tokens_checked=int(toks.size), h_rows=len(rows), h_flips=int(flips),
             tokens_with_flips=n_flipped_tok, stage2_max_rel=norm_h, stage2_elementwise=el_h,
             e2e_max_rel=normwise, e2e_elementwise=el, e2e_unsubstituted_max_rel=raw_norm,
             bf16_max_rel=bf16_norm, distinct_experts=int(np.unique(gi).size), w4a32_drift=drift,
             drift_vs_ref_decode_w4a32=drift_w4a32, drift_vs_ref_prefill_fp16h=drift_prefill)
    assert flips <= 0.01 * len(rows) * hq.shape[1]
    assert norm_h <= TOL and el_h <= TOL, f"{name}: down/combine error {norm_h:.3g} / {el_h:.3g}"
    assert normwise <= TOL and el <= TOL, f"{name}: end-to-end error {normwise:.3g} / {el:.3g}"
    if every_token:
        m = fullcheck.check_every_token(oracle, w, x, lg, shg, y32, gi, pos, hq, hs)
        _metrics(name + "/every_token", T=int(T), **m)
    return layer


PATHS = [pytest.param(1, id="sorted"), pytest.param(4, id="sorted_skinny"),
         pytest.param(5, id="sorted_fused"), pytest.param(2, id="direct")]


@pytest.mark.parametrize("path", PATHS)
def test_forward_decode1(dev, oracle, layer_w, path):
    x, lg, _ = synth.config_inputs("decode1", 1)
    _check_layer("decode1", dev, oracle, layer_w, x, lg, None, path=path)


# Batch sizes between the named configurations, each on a forced path (0 =
# the automatic choice), with Zipf routing on every other case and the
# shared expert on some: (T, path, zipf, shared).
# The one-kernel skinny path (path 5) finds its own tiles for up to 4096
# routed entries (T = 512 at top-8: the case (512, 5) sits on that limit);
# above it, (600, 5), the tiles come from k_scatter and the kernel writes its
# rows in sorted order.
SWEEP = [(3, 2, False, True), (9, 4, True, False), (17, 0, False, False), (31, 1, True, True),
         (48, 5, True, True), (100, 4, False, True), (200, 5, False, False), (256, 5, True, True),
         (257, 0, True, False), (300, 5, False, True), (512, 5, True, False), (600, 5, False, True),
         (1000, 1, False, False), (2049, 0, True, True)]


@pytest.mark.parametrize("T,path,zipf,shared", SWEEP, ids=[f"T{c[0]}_p{c[1]}" for c in SWEEP])
def test_forward_batch_sweep(dev, oracle, layer_w, T, path, zipf, shared):
    rng = np.random.default_rng(700 + T)
    x = synth.hidden(rng, T)
    lg = synth.zipf_logits(rng, T) if zipf else synth.normal_logits(rng, T)
    shg = rng.standard_normal(T).astype(np.float32) if shared else None
    sample = None if T <= 32 else np.sort(rng.choice(T, size=24, replace=False))
    _check_layer(f"sweep{T}", dev, oracle, layer_w, x, lg, shg, sample=sample, path=path)


def _random_case(seed):
    rng = np.random.default_rng(4000 + seed)
    T = int(np.exp(rng.uniform(np.log(2), np.log(3000))))
    paths = [0, 1, 4, 5] + ([2] if T <= 16 else [])
    path = int(rng.choice(paths))
    zipf, shared, bf16 = bool(rng.integers(2)), bool(rng.integers(2)), bool(rng.integers(2))
    return rng, T, path, zipf, shared, bf16


RANDOM_CASES = [_random_case(i)[1:] for i in range(8)]


@pytest.mark.parametrize("seed", range(8), ids=[f"T{c[0]}_p{c[1]}{'_zipf' if c[2] else ''}{'_sh' if c[3] else ''}"
                                                 f"{'_bf16' if c[4] else ''}" for c in RANDOM_CASES])
def test_forward_random_every_token(dev, oracle, layer_w, seed):
    """Seeded random configurations (T log-uniform in 2..3000, any path that
    serves T, Zipf or normal routing, with or without the shared expert, f32
    or bf16 x), every token through the three staged 2e-3 bars."""
    w, dw = layer_w
    rng, T, path, zipf, shared, bf16 = _random_case(seed)
    x = synth.hidden(rng, T)
    if bf16:
        x = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    lg = synth.zipf_logits(rng, T) if zipf else synth.normal_logits(rng, T)
    shg = rng.standard_normal(T).astype(np.float32) if shared else None
    layer, y32, y16 = _run_layer(dev, dw, x, lg, shg, x_dtype=torch.bfloat16 if bf16 else torch.float32, path=path)
    gi = _check_routing(layer, oracle, lg)
    oq, os_ = oracle.quant_e4m3(x)
    np.testing.assert_array_equal(layer.tap(moe.TAP_XQ).cpu().numpy(), oq)
    np.testing.assert_array_equal(layer.tap(moe.TAP_XS).cpu().numpy(), os_)
    np.testing.assert_array_equal(y16, _bf16_of(y32))
    pos = layer.tap(moe.TAP_POS).cpu().numpy()
    hq, hs = layer.tap(moe.TAP_HQ).cpu().numpy(), layer.tap(moe.TAP_HS).cpu().numpy()
    m = fullcheck.check_every_token(oracle, w, x, lg, shg, y32, gi, pos, hq, hs)
    _metrics(f"random{seed}", T=T, path=path, ran=layer.last_path, zipf=zipf, shared=shared, bf16=bf16, **m)


@pytest.mark.parametrize("path", PATHS)
@pytest.mark.parametrize("T", [2, 7, 16])
def test_forward_small_batches(dev, oracle, layer_w, T, path):
    rng = np.random.default_rng(300 + T)
    x, lg = synth.hidden(rng, T), synth.normal_logits(rng, T)
    _check_layer(f"small{T}", dev, oracle, layer_w, x, lg, None, path=path)


@pytest.mark.parametrize("path", [pytest.param(0, id="auto"), pytest.param(1, id="sorted")])
def test_forward_small33(dev, oracle, layer_w, path):
    rng = np.random.default_rng(333)
    x, lg = synth.hidden(rng, 33), synth.normal_logits(rng, 33)
    _check_layer("small33", dev, oracle, layer_w, x, lg, None, path=path)


@pytest.mark.parametrize("T", [1, 5, 16])
def test_direct_equals_sorted_inputs(dev, layer_w, T):
    """Both paths see the same routing and quantised x; their outputs agree
    to the stage-2 bar (they differ only in accumulation order)."""
    _, dw = layer_w
    rng = np.random.default_rng(900 + T)
    x, lg = synth.hidden(rng, T), synth.normal_logits(rng, T)
    outs, taps = [], []
    for path in (1, 2, 4, 5):
        layer, y32, _ = _run_layer(dev, dw, x, lg, None, path=path)
        outs.append(y32)
        taps.append([layer.tap(m).cpu().numpy() for m in (moe.TAP_TOPK_IDX, moe.TAP_TOPK_W,
                                                          moe.TAP_XQ, moe.TAP_XS)])
    for other in taps[1:]:
        for a, b in zip(taps[0], other):
            np.testing.assert_array_equal(a, b)
    for o in outs[1:]:
        _, normwise = _row_err(o, outs[0].astype(np.float64))
        assert normwise <= TOL


@pytest.mark.parametrize("path", [pytest.param(0, id="auto_fused"), pytest.param(4, id="sorted_skinny"),
                                  pytest.param(1, id="sorted")])
def test_forward_ragged64_zipf(dev, oracle, layer_w, path):
    x, lg, _ = synth.config_inputs("ragged64", 2)
    _check_layer("ragged64", dev, oracle, layer_w, x, lg, None, path=path)


def test_forward_fat_skewed(dev, oracle, layer_w):
    """Fat-tile path with Zipf routing at T=700: the most popular experts hold
    more rows than one fat tile (split tiles), the tail holds 0-2 rows, so
    every column-tile count per wave occurs."""
    rng = np.random.default_rng(66)
    x, lg = synth.hidden(rng, 700), synth.zipf_logits(rng, 700)
    counts = np.bincount(np.argsort(-lg, axis=1)[:, :8].ravel(), minlength=256)
    assert counts.max() > 3 * 192 and (counts <= 2).sum() > 10
    rng2 = np.random.default_rng(67)
    sample = np.sort(rng2.choice(700, size=40, replace=False))
    _check_layer("fat_skewed", dev, oracle, layer_w, x, lg, None, path=1, sample=sample)


def test_forward_prefill_past_4096(dev, oracle, layer_w):
    """T=4500: 282 routing blocks, so each column-scan thread sums 9 blocks
    (past the 8 it holds in registers) -- the loop form of the scan."""
    rng = np.random.default_rng(45)
    x, lg = synth.hidden(rng, 4500), synth.normal_logits(rng, 4500)
    sample = np.sort(rng.choice(4500, size=32, replace=False))
    _check_layer("prefill4500", dev, oracle, layer_w, x, lg, None, sample=sample)


def test_forward_prefill4096(dev, oracle, layer_w):
    """Every one of the 4,096 tokens through all three stages, plus 48 tokens
    through the C oracle's per-token path."""
    x, lg, _ = synth.config_inputs("prefill4096", 3)
    rng = np.random.default_rng(33)
    sample = np.sort(rng.choice(4096, size=48, replace=False))
    _check_layer("prefill4096", dev, oracle, layer_w, x, lg, None, sample=sample, every_token=True)


def test_forward_mixed_shared(dev, oracle, layer_w):
    """Every one of the 4,006 tokens, shared expert included."""
    x, lg, shg = synth.config_inputs("mixed", 4)
    rng = np.random.default_rng(44)
    sample = np.concatenate([np.arange(6), 6 + np.sort(rng.choice(4000, size=40, replace=False))])
    _check_layer("mixed", dev, oracle, layer_w, x, lg, shg, sample=sample, every_token=True)


@pytest.mark.parametrize("seed", [5001, 5002, 5003])
def test_forward_mixed_fresh_weights(dev, oracle, seed):
    """The mixed step names 40 layers of fresh seeded weights: three more
    weight seeds (with their own shared expert and inputs), every token."""
    w = synth.expert_weights(seed, shared=True)
    dw = moe.MoEWeights.upload(w["gate"], w["up"], w["down"], w["sh_gate"], w["sh_up"], w["sh_down"])
    x, lg, shg = synth.config_inputs("mixed", seed)
    _check_layer(f"mixed_seed{seed}", dev, oracle, (w, dw), x, lg, shg, sample=np.arange(6),
                 every_token=True)
    del dw


@pytest.mark.parametrize("path", [1, 4, 5])
def test_dnw_tap_staged_rows(dev, oracle, layer_w, path):
    """The DNW tap: every staged weighted down row (f16 with an exponent per
    column group, widened to f32) equals w * Down_e(h) of its entry from the
    GPU's own h codes, to the f16 rounding (2^-11 relative) plus the scaled
    MFMA's own accumulation error (up to ~5e-5 of max|C| on gfx950, as the
    operand calibration measures; bar 2e-4 of the row maximum).  Rows are in sorted-slot order on the sorted paths and in
    entry order on the one-kernel path that finds its own tiles; shared
    rows follow at T*k + t."""
    w, dw = layer_w
    rng = np.random.default_rng(58)
    T = 24
    x, lg = synth.hidden(rng, T), synth.normal_logits(rng, T)
    shg = rng.standard_normal(T).astype(np.float32)
    layer, _, _ = _run_layer(dev, dw, x, lg, shg, path=path)
    gi = layer.tap(moe.TAP_TOPK_IDX).cpu().numpy()
    pos = layer.tap(moe.TAP_POS).cpu().numpy()
    hq, hs = layer.tap(moe.TAP_HQ).cpu().numpy(), layer.tap(moe.TAP_HS).cpu().numpy()
    dnw = layer.tap(moe.TAP_DNW).cpu().numpy().astype(np.float64)
    _, ow = oracle.router_topk(lg, 8)
    entry_order = layer.last_path == 3
    worst = 0.0
    for t in range(T):
        for s in range(9):
            if s < 8:
                p = int(pos[t * 8 + s])
                row = t * 8 + s if entry_order else p
                ref = ow[t, s] * oracle.expert_down(w["down"][gi[t, s]], oracle.dequant_e4m3(hq[p:p + 1], hs[p:p + 1])[0])
            else:
                p = row = T * 8 + t
                ref = (1 / (1 + np.exp(-float(shg[t])))) * oracle.expert_down(
                    w["sh_down"], oracle.dequant_e4m3(hq[p:p + 1], hs[p:p + 1])[0])
            err = np.abs(dnw[row] - ref) - 2.0 ** -11 * np.abs(ref)
            worst = max(worst, float(err.max() / np.abs(ref).max()))
    _metrics("dnw_tap", path=path, worst_excess=worst)
    assert worst <= 2e-4, worst


@pytest.mark.parametrize("path", PATHS)
def test_forward_shared_small(dev, oracle, layer_w, path):
    rng = np.random.default_rng(55)
    x, lg = synth.hidden(rng, 5), synth.normal_logits(rng, 5)
    shg = rng.standard_normal(5).astype(np.float32)
    _check_layer("shared5", dev, oracle, layer_w, x, lg, shg, path=path)


def test_forward_bf16_input(dev, oracle, layer_w):
    """bf16 activations: the oracle sees the same values widened to f32."""
    rng = np.random.default_rng(66)
    x, lg = synth.hidden(rng, 9), synth.normal_logits(rng, 9)
    xb = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    _check_layer("bf16_in", dev, oracle, layer_w, xb, lg, None, x_dtype=torch.bfloat16)
    _check_layer("bf16_in", dev, oracle, layer_w, xb[:4], lg[:4], None, x_dtype=torch.bfloat16,
                 path=2)


@pytest.mark.parametrize("T,path", [(40, 5), (40, 1), (600, 1)])
def test_forward_bf16_input_sorted(dev, oracle, layer_w, T, path):
    """bf16 activations through the routing kernels of the sorted paths (one
    token per workgroup on the one-kernel skinny path, the per-block counting
    kernel otherwise), each compiled per input format."""
    rng = np.random.default_rng(67)
    x, lg = synth.hidden(rng, T), synth.normal_logits(rng, T)
    xb = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    sample = None if T <= 64 else list(range(0, T, 37))
    _check_layer("bf16_in_sorted", dev, oracle, layer_w, xb, lg, None, sample=sample, x_dtype=torch.bfloat16,
                 path=path)


def test_forward_deterministic_and_reusable(dev, layer_w):
    """Two runs give identical bits; a smaller call after a larger one on the
    same context matches a fresh context."""
    _, dw = layer_w
    rng = np.random.default_rng(77)
    x, lg = synth.hidden(rng, 300), synth.normal_logits(rng, 300)
    layer = moe.MoELayer(300)
    xt, lt = torch.from_numpy(x).to(dev), torch.from_numpy(lg).to(dev)
    a = layer.forward(dw, xt, lt, out_dtype=torch.float32).clone()
    b = layer.forward(dw, xt, lt, out_dtype=torch.float32).clone()
    assert torch.equal(a, b)
    small = layer.forward(dw, xt[:3], lt[:3], out_dtype=torch.float32).clone()
    fresh = moe.MoELayer(3).forward(dw, xt[:3], lt[:3], out_dtype=torch.float32)
    assert torch.equal(small, fresh)


def test_forward_empty_and_errors(dev, layer_w):
    _, dw = layer_w
    layer = moe.MoELayer(4)
    x = torch.zeros((0, 2048), device=dev)
    lg = torch.zeros((0, 256), device=dev)
    out = layer.forward(dw, x, lg)
    assert out.shape == (0, 2048)
    with pytest.raises(moe.Q36MoEError):
        layer.forward(dw, torch.zeros((5, 2048), device=dev), torch.zeros((5, 256), device=dev))
    with pytest.raises(moe.Q36MoEError):
        moe.MoELayer(4).forward(dw, torch.zeros((1, 2048)), torch.zeros((1, 256)))
    # shared-gate logits: one per token, at a real stride (no broadcast view)
    x3, lg3 = torch.zeros((3, 2048), device=dev), torch.zeros((3, 256), device=dev)
    with pytest.raises(moe.Q36MoEError):
        layer.forward(dw, x3, lg3, torch.zeros(2, device=dev))
    with pytest.raises(moe.Q36MoEError):
        layer.forward(dw, x3, lg3, torch.zeros(1, device=dev).expand(3))
    with pytest.raises(moe.Q36MoEError):
        moe.forward_noalloc(dw, x3, lg3, torch.zeros(4, device=dev))


@pytest.mark.parametrize("T", [1, 64, 600])
def test_forward_in_hip_graph(dev, layer_w, T):
    """forward captured in a HIP graph (as a model's layer loop runs it):
    every replay, with eager forwards of other inputs and synchronisations
    in between, equals the eager result bit for bit (covers the direct,
    skinny and fat sorted paths)."""
    _, dw = layer_w
    rng = np.random.default_rng(1000 + T)
    x = torch.from_numpy(synth.hidden(rng, T)).to(dev)
    lg = torch.from_numpy(synth.normal_logits(rng, T)).to(dev)
    x2 = torch.from_numpy(synth.hidden(rng, T)).to(dev)
    lg2 = torch.from_numpy(synth.normal_logits(rng, T)).to(dev)
    layer = moe.MoELayer(T)
    out = torch.empty((T, 2048), dtype=torch.float32, device=dev)
    ref = layer.forward(dw, x, lg, out_dtype=torch.float32).clone()
    cap = torch.cuda.Stream()
    layer.set_stream(cap)
    with torch.cuda.stream(cap):
        layer.forward(dw, x, lg, out=out)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=cap):
        layer.forward(dw, x, lg, out=out)
    torch.cuda.synchronize()
    layer.set_stream(torch.cuda.current_stream())
    for rep in range(4):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {rep}"
        other = layer.forward(dw, x2, lg2, out_dtype=torch.float32)   # eager work between
        torch.cuda.synchronize()
        assert not torch.equal(other, ref)


def _router_ref(w, x, f16):
    """fp64 dot products of (optionally fp16-rounded, RNE by numpy) inputs,
    and the sum of |terms| that bounds fp32 accumulation error."""
    if f16:
        w = w.astype(np.float16)
        x = x.astype(np.float16)
    w64, x64 = w.astype(np.float64), x.astype(np.float64)
    return x64 @ w64.T, np.abs(x64) @ np.abs(w64).T


@pytest.mark.parametrize("T,mode", [(1, 1), (5, 1), (16, 1), (16, 0), (17, 0), (300, 2), (64, 2)])
def test_router_logits(dev, T, mode):
    """Router matvec against fp64 (fp32 path) or fp64 over fp16-rounded
    inputs (fp16 path); error within fp32 accumulation of |terms|."""
    rng = np.random.default_rng(500 + T)
    w = (rng.standard_normal((257, 2048)) * 0.02).astype(np.float32)
    x = rng.standard_normal((T, 2048)).astype(np.float32)
    lg, shg = moe.router_logits(torch.from_numpy(w).to(dev), torch.from_numpy(x).to(dev), 256, mode)
    torch.cuda.synchronize()
    f16 = mode == 2 or (mode == 0 and T > 16)
    ref, mag = _router_ref(w, x, f16)
    got = np.concatenate([lg.cpu().numpy(), shg.cpu().numpy()[:, None]], axis=1).astype(np.float64)
    err = np.abs(got - ref) / mag
    _metrics("router_logits", T=T, mode=mode, max_rel_to_abs_terms=float(err.max()))
    assert err.max() <= 2e-6, err.max()


def test_router_logits_bf16_input_and_no_shared(dev):
    rng = np.random.default_rng(77)
    w = (rng.standard_normal((256, 2048)) * 0.02).astype(np.float32)
    x = rng.standard_normal((3, 2048)).astype(np.float32)
    xb = torch.from_numpy(x).to(dev).to(torch.bfloat16)
    lg, shg = moe.router_logits(torch.from_numpy(w).to(dev), xb, 256, 1)
    torch.cuda.synchronize()
    assert shg is None
    ref, mag = _router_ref(w, xb.float().cpu().numpy(), False)
    assert (np.abs(lg.cpu().numpy() - ref) / mag).max() <= 2e-6


@pytest.mark.parametrize("T,with_a", [(1, True), (5, True), (300, True), (7, False)])
def test_add_rmsnorm_quant(dev, oracle, T, with_a):
    """Fused residual add + RMSNorm + quantisation: h += a bit-exact (one
    fp32 add), y against fp64 within fp32 rounding of the sum and rsqrt, and
    the codes / scales bit-exact against the oracle's quantisation of y."""
    rng = np.random.default_rng(900 + T)
    h = (rng.standard_normal((T, 2048)) * 3).astype(np.float32)
    a = rng.standard_normal((T, 2048)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(2048)).astype(np.float32)
    h[0, :64] = 0.0                                   # a zero 32-block (scale 2^-127)
    ht = torch.from_numpy(h).to(dev)
    y, xq, xs = moe.add_rmsnorm_quant(ht, torch.from_numpy(a).to(dev) if with_a else None,
                                      torch.from_numpy(w).to(dev), eps=1e-6)
    torch.cuda.synchronize()
    v = (h + a) if with_a else h                      # fp32 add, as the kernel
    np.testing.assert_array_equal(ht.cpu().numpy(), v)
    v64 = v.astype(np.float64)
    ref = v64 / np.sqrt((v64 * v64).mean(axis=1, keepdims=True) + 1e-6) * w
    yg = y.cpu().numpy()
    err = np.abs(yg - ref).max() / np.abs(ref).max()
    _metrics("add_rmsnorm_quant", T=T, with_a=with_a, max_rel=float(err))
    assert err <= 4e-6, err
    oq, os_ = oracle.quant_e4m3(yg)
    np.testing.assert_array_equal(xq.cpu().numpy(), oq)
    np.testing.assert_array_equal(xs.cpu().numpy(), os_)


@pytest.fixture(scope="module")
def layer_w64():
    w = synth.expert_weights(2031, n_expert=64, shared=True)
    dw = moe.MoEWeights.upload(w["gate"], w["up"], w["down"], w["sh_gate"], w["sh_up"], w["sh_down"])
    return w, dw


@pytest.mark.parametrize("T", [5, 24, 40])
def test_forward_64_experts_top4(dev, oracle, layer_w64, T):
    """A layer of 64 experts with top-4 routing (the library takes any
    n_expert <= 256 and top_k <= 8) on every path that serves T: routing,
    sort and output against the oracle, the output through the three staged
    2e-3 bars on every token (tests/fullcheck.py: h codes equal but for
    midpoint flips, down + combine from the GPU's h, end to end with the
    flipped codes substituted)."""
    w, dw = layer_w64
    E, k = 64, 4
    rng = np.random.default_rng(1300 + T)
    x = synth.hidden(rng, T)
    lg = synth.normal_logits(rng, T, n_expert=E)
    shg = rng.standard_normal(T).astype(np.float32)
    ref = oracle.moe_forward(w, x, lg, shg, k=k)
    oi, _ = oracle.router_topk(lg, k, n_expert=E)
    off, perm, pos = oracle.sort_entries(oi, E)
    paths = [0, 1, 4, 5] + ([2] if T <= 16 else [])
    seen = set()
    for path in paths:
        layer = moe.MoELayer(T, n_expert=E, top_k=k)
        layer.set_path(path)
        y = layer.forward(dw, torch.from_numpy(x).to(dev), torch.from_numpy(lg).to(dev),
                          torch.from_numpy(shg).to(dev), out_dtype=torch.float32)
        layer.check()
        seen.add(layer.last_path)
        np.testing.assert_array_equal(layer.tap(moe.TAP_TOPK_IDX).cpu().numpy(), oi)
        if layer.last_path != 1:
            np.testing.assert_array_equal(layer.tap(moe.TAP_EOFF).cpu().numpy(), off)
            np.testing.assert_array_equal(layer.tap(moe.TAP_PERM).cpu().numpy(), perm)
            np.testing.assert_array_equal(layer.tap(moe.TAP_POS).cpu().numpy(), pos)
        gi = layer.tap(moe.TAP_TOPK_IDX).cpu().numpy()
        gpos = layer.tap(moe.TAP_POS).cpu().numpy()
        hq, hs = layer.tap(moe.TAP_HQ).cpu().numpy(), layer.tap(moe.TAP_HS).cpu().numpy()
        y64 = y.cpu().numpy().astype(np.float64)
        m = fullcheck.check_every_token(oracle, w, x, lg, shg, y64, gi, gpos, hq, hs, k=k)
        _metrics(f"experts64_top4/T{T}/path{path}", **m)
        # and the C oracle's own per-token forward with its own h codes, as a
        # loose backstop (a midpoint flip of a large h code moves a token by
        # up to ~2e-3 of its row max)
        _, normwise = _row_err(y64, ref)
        assert normwise <= 1e-2, f"path {path} (ran {layer.last_path}): {normwise:.3g}"
    assert 3 in seen and 2 in seen and 0 in seen


@pytest.mark.parametrize("T,path", [(1, 0), (5, 2), (40, 4), (40, 5), (40, 1), (600, 0)])
def test_forward_q8_equals_forward(dev, layer_w, T, path):
    """The pre-quantised entry gives bit-identical results (outputs and
    routing/quantisation taps) to forward on the x it was quantised from, on
    every path."""
    _, dw = layer_w
    rng = np.random.default_rng(950 + T)
    x = torch.from_numpy(synth.hidden(rng, T)).to(dev)
    lg = torch.from_numpy(synth.normal_logits(rng, T)).to(dev)
    shg = torch.from_numpy(rng.standard_normal(T).astype(np.float32)).to(dev)
    xq, xs = moe.quant_e4m3(x)
    la, lb = moe.MoELayer(T), moe.MoELayer(T)
    la.set_path(path)
    lb.set_path(path)
    ya = la.forward(dw, x, lg, shg, out_dtype=torch.float32)
    yb = lb.forward_q8(dw, xq, xs, lg, shg, out_dtype=torch.float32)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(ya.cpu().numpy(), yb.cpu().numpy())
    for tap in (moe.TAP_TOPK_IDX, moe.TAP_XQ, moe.TAP_XS, moe.TAP_HQ):
        np.testing.assert_array_equal(la.tap(tap).cpu().numpy(), lb.tap(tap).cpu().numpy())


@pytest.mark.parametrize("T,path", [(1, 2), (5, 2), (40, 5), (600, 1)])
def test_forward_strided_shared_gate(dev, layer_w, T, path):
    """The reference's batched decode keeps the shared-gate logit in column
    256 of each 257-wide router row (q36_engine.cu:2092-2095): forward takes
    logits = rows[:, :256] and shg = rows[:, 256] (stride 257) directly and
    gives the same bits as the gathered contiguous copy, on the direct,
    skinny (one kernel per tile) and fat paths."""
    _, dw = layer_w
    rng = np.random.default_rng(1200 + T)
    rows = np.concatenate([synth.normal_logits(rng, T), rng.standard_normal((T, 1)).astype(np.float32)], axis=1)
    x = torch.from_numpy(synth.hidden(rng, T)).to(dev)
    rt = torch.from_numpy(np.ascontiguousarray(rows)).to(dev)
    la, lb = moe.MoELayer(T), moe.MoELayer(T)
    la.set_path(path)
    lb.set_path(path)
    ya = la.forward(dw, x, rt[:, :256], rt[:, 256], out_dtype=torch.float32)
    yb = lb.forward(dw, x, rt[:, :256].contiguous(), rt[:, 256].contiguous(), out_dtype=torch.float32)
    xq, xs = moe.quant_e4m3(x)
    yc = moe.MoELayer(T).forward_q8(dw, xq, xs, rt[:, :256], rt[:, 256], out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert rt[:, 256].stride(0) == 257
    np.testing.assert_array_equal(ya.cpu().numpy(), yb.cpu().numpy())
    # the automatic path of these sizes is the forced one
    np.testing.assert_array_equal(ya.cpu().numpy(), yc.cpu().numpy())
    # and the shared expert is really in the sum
    yn = moe.MoELayer(T).forward(dw, x, rt[:, :256].contiguous(), None, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert not torch.equal(ya, yn)


@pytest.mark.parametrize("cfg,path", [("decode1", 2), ("ragged64", 0), ("prefill4096", 0), ("mixed", 0)])
def test_drift_from_reference_numerics(dev, oracle, layer_w, cfg, path):
    """Distance of the build (W4A8: e4m3 x and h) from the reference's own
    numeric paths, reported (stdout and Q36_METRICS_FILE) with a loose sanity
    bound, on a configuration that also passes the parity bars of
    _check_layer: W4A32, the reference's decode matvecs
    (q36_engine.cu:1610-1618), and e4m3 x with f32 h rounded to fp16, its
    prefill GEMMs (q36_engine.cu:3437-3462).  The north star mandates FP8
    activations for both GEMMs, so this is a stated number, not a bar; the
    per-32 e4m3 of h (relative step up to 2^-3) is what separates them."""
    x, lg, shg = synth.config_inputs(cfg, 5)
    T = x.shape[0]
    sample = None if T <= 64 else np.sort(np.random.default_rng(51).choice(T, 32, replace=False))
    _check_layer(f"drift_{cfg}", dev, oracle, layer_w, x, lg, shg, sample=sample, path=path)
    m = _LAST_METRICS
    print(f"drift {cfg}: vs W4A32 {m['drift_vs_ref_decode_w4a32']:.2e}, "
          f"vs e4m3-x/fp16-h {m['drift_vs_ref_prefill_fp16h']:.2e} (parity e2e {m['e2e_max_rel']:.2e})")
    assert m["drift_vs_ref_decode_w4a32"] < 0.15 and m["drift_vs_ref_prefill_fp16h"] < 0.15
