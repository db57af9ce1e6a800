"""Every-token parity of a layer forward against an fp64 reference built
expert by expert (test infrastructure).

The per-token checks in test_gpu_parity.py call the C oracle once per
(token, slot): exact, but too slow for 4,096 tokens.  This module computes
the same three stages for every token of a large batch by grouping the
routed entries by expert, so each expert's matrices are dequantised once
(by the oracle's own MXFP4 dequant) and applied to all of its rows with one
fp64 matrix product:

  1. h = silu(G x) * (U x) in fp64 from the oracle's dequantised e4m3 x,
     rounded to fp32 and quantised by the oracle's quantiser; the GPU's h
     codes / E8M0 scales must equal these except at rounding midpoints
     (fp32 vs fp64 accumulation), counted and capped at 1%;
  2. down + combine from the GPU's own h codes: sum_s w_s (Dn_e hd_gpu), in
     fp64, against the GPU's f32 output, with the element-wise slack of the
     f16 staging (2^-10 * sum |terms|);
  3. end to end: a token without flips against the reference computed from
     the oracle's own h codes (which then equal the GPU's); every token
     against the reference with the GPU's codes at the accepted flips.

The routing weights are the oracle's fp64 ones (q36_ops.cuh:424-430), the
combine is in slot order then the gated shared expert
(q36_engine.cu:3393-3401).  ``layer_reference`` is held against the C
oracle's per-token forward in tests/test_oracle.py.
"""
import numpy as np

TOL = 2e-3
FLOOR = 5e-2
STAGE_SLACK = 2.0 ** -10


def _deq(oracle, blocks):
    M = blocks.shape[0]
    return oracle.deq_mxfp4_row(blocks).reshape(M, -1).astype(np.float64)


def _silu(g):
    return g / (1.0 + np.exp(-g))


def _groups(gi, n_expert):
    """{expert: (tokens, slots)} of the routed entries, entry order."""
    T, k = gi.shape
    flat = gi.ravel()
    order = np.argsort(flat, kind="stable")
    bounds = np.searchsorted(flat[order], np.arange(n_expert + 1))
    out = {}
    for e in range(n_expert):
        ent = order[bounds[e]:bounds[e + 1]]
        if ent.size:
            out[e] = (ent // k, ent % k)
    return out


def _mid_distance(v, mids):
    a = np.abs(v)
    j = np.clip(np.searchsorted(mids, a), 1, mids.size - 1)
    return np.minimum(np.abs(a - mids[j - 1]), np.abs(a - mids[j]))


def _e4m3_mids():
    import torch
    tab = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).double().numpy()
    fin = np.sort(np.unique(np.abs(tab[np.isfinite(tab)])))
    return (fin[:-1] + fin[1:]) / 2


def h_compare(h64, gq, gs, oq, os_):
    """Stage 1 for a block of rows: returns (flips, substituted codes,
    substituted scales).  h64 [n][FF] fp64, gq/gs the GPU's codes / scales,
    oq/os_ the oracle's quantisation of fp32(h64)."""
    n, FF = h64.shape
    nb = FF // 32
    sq, ss = oq.copy(), os_.copy()
    flips = 0
    # a scale may differ only where the block amax / 448 sits within 1e-4 of
    # a power of two; the whole block then takes the GPU's codes
    bad_s = gs != os_
    if bad_s.any():
        amax = np.abs(h64.reshape(n, nb, 32)).max(axis=2) / 448.0
        rel = np.abs(amax / 2.0 ** np.round(np.log2(np.maximum(amax, 1e-300))) - 1)
        r, b = np.nonzero(bad_s)
        assert np.all(rel[r, b] < 1e-4), f"h scale mismatch away from a boundary at rows {r[:5]} blocks {b[:5]}"
        flips += int(r.size)
        ss[bad_s] = gs[bad_s]
        blk = np.repeat(bad_s, 32, axis=1)
        sq[blk] = gq[blk]
    # a code may differ only within 1e-4 * blockmax of a rounding midpoint
    bad_c = (gq != oq) & ~np.repeat(bad_s, 32, axis=1)
    if bad_c.any():
        v = h64 * np.repeat(2.0 ** -(os_.astype(np.int64) - 127), 32, axis=1)
        vmax = np.repeat(np.abs(v.reshape(n, nb, 32)).max(axis=2), 32, axis=1)
        r, c = np.nonzero(bad_c)
        d = _mid_distance(v[r, c], _e4m3_mids())
        assert np.all(d <= 1e-4 * vmax[r, c]), f"h code mismatch away from a midpoint at rows {r[:5]} cols {c[:5]}"
        flips += int(r.size)
        sq[bad_c] = gq[bad_c]
    return flips, sq, ss


def layer_reference(oracle, w, x, logits, shg=None, k=8, gpu_h=None):
    """fp64 layer output for every token.  Without gpu_h: the oracle's own
    numerics (its h codes).  With gpu_h = (idx, pos, hq, hs) from a forward:
    returns a dict with the reference from the GPU's h codes ('ref'), from
    the oracle's codes with the GPU's at accepted flips ('ref_sub'), from the
    oracle's codes alone ('ref0'), sum |terms| ('absterms'), the flip count,
    the per-token flip flags and the number of h rows compared."""
    T, D = x.shape
    E = w["gate"].shape[0]
    xq, xs = oracle.quant_e4m3(x)
    xd = oracle.dequant_e4m3(xq, xs)
    oi, ow = oracle.router_topk(logits, k, n_expert=E)
    ref0 = np.zeros((T, D))
    if gpu_h is None:
        groups = _groups(oi, E)
    else:
        gi, pos, hq, hs = gpu_h
        np.testing.assert_array_equal(gi, oi)
        groups = _groups(gi, E)
        ref = np.zeros((T, D))
        ref_sub = np.zeros((T, D))
        absterms = np.zeros((T, D))
        tok_flip = np.zeros(T, dtype=bool)
        flips = 0
        nrows = 0

    def run(Gm, Um, Dm, toks, rows, wv):
        nonlocal flips, nrows
        X = xd[toks]
        h = _silu(X @ Gm.T) * (X @ Um.T)
        oq, os_ = oracle.quant_e4m3(h.astype(np.float32))
        ref0[toks] += wv[:, None] * (oracle.dequant_e4m3(oq, os_) @ Dm.T)
        if gpu_h is None:
            return
        gq, gs = hq[rows], hs[rows]
        nf, sq, ss = h_compare(h, gq, gs, oq, os_)
        if nf:
            rowflip = np.any(sq != oq, axis=1) | np.any(ss != os_, axis=1)
            tok_flip[toks[rowflip]] = True
            flips += nf
        nrows += rows.size
        term = wv[:, None] * (oracle.dequant_e4m3(gq, gs) @ Dm.T)
        ref[toks] += term
        absterms[toks] += np.abs(term)
        ref_sub[toks] += wv[:, None] * (oracle.dequant_e4m3(sq, ss) @ Dm.T)

    for e, (toks, slots) in groups.items():
        rows = pos[toks * k + slots] if gpu_h is not None else None
        run(_deq(oracle, w["gate"][e]), _deq(oracle, w["up"][e]), _deq(oracle, w["down"][e]),
            toks, rows, ow[toks, slots])
    if shg is not None:
        toks = np.arange(T)
        gate = 1.0 / (1.0 + np.exp(-shg.astype(np.float64)))
        rows = T * k + toks if gpu_h is not None else None
        run(_deq(oracle, w["sh_gate"]), _deq(oracle, w["sh_up"]), _deq(oracle, w["sh_down"]), toks, rows, gate)
    if gpu_h is None:
        return ref0
    return dict(ref=ref, ref_sub=ref_sub, ref0=ref0, absterms=absterms, flips=flips,
                tok_flip=tok_flip, h_rows=nrows)


def row_err(y, ref, absterms=None):
    """(element-wise, normwise) max relative error over rows, as in the
    per-token checks: element-wise |y - ref| (less STAGE_SLACK * absterms)
    over max(|ref|, FLOOR * rowmax); normwise max |y - ref| / max |ref|."""
    scale = np.abs(ref).max(axis=1, keepdims=True)
    d = np.abs(y - ref)
    if absterms is not None:
        d = np.maximum(d - STAGE_SLACK * absterms, 0.0)
    rel = d / np.maximum(np.abs(ref), FLOOR * scale)
    return float(rel.max()), float((np.abs(y - ref).max(axis=1) / scale[:, 0]).max())


def check_every_token(oracle, w, x, logits, shg, y32, gi, pos, hq, hs, k=8):
    """All three stages on every token; returns the metrics and asserts the
    2e-3 bars."""
    r = layer_reference(oracle, w, x, logits, shg, k, gpu_h=(gi, pos, hq, hs))
    el2, norm2 = row_err(y32, r["ref"], r["absterms"])
    el3, norm3 = row_err(y32, r["ref_sub"], r["absterms"])
    clean = ~r["tok_flip"]
    el0, norm0 = row_err(y32[clean], r["ref0"][clean], r["absterms"][clean]) if clean.any() else (0.0, 0.0)
    m = dict(tokens_checked=int(x.shape[0]), h_rows=int(r["h_rows"]), h_flips=int(r["flips"]),
             tokens_with_flips=int(r["tok_flip"].sum()), stage2_max_rel=norm2, stage2_elementwise=el2,
             e2e_max_rel=norm3, e2e_elementwise=el3, e2e_clean_tokens_max_rel=norm0,
             e2e_clean_tokens_elementwise=el0)
    assert r["flips"] <= 0.01 * r["h_rows"] * hq.shape[1], m
    assert norm2 <= TOL and el2 <= TOL, m
    assert norm3 <= TOL and el3 <= TOL, m
    assert norm0 <= TOL and el0 <= TOL, m
    return m
