"""Pins the CPU oracle (oracle/q36moe_oracle.c) against the reference's own
known answers and code, closed forms, an independent library routine
(torch.float8_e4m3fn) and brute force.  CPU only."""
import os
import subprocess

import numpy as np
import pytest
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
GOLDEN = os.path.join(HERE, "golden", "mxfp4_dequant_ref.npz")


# ---------------------------------------------------------------------------
# MXFP4 / E8M0
# ---------------------------------------------------------------------------
def test_reference_test_dequant_binary():
    """The reference's own CPU unit test, built from its sources
    (oracle/Makefile), passes: struct sizes and dequant constants."""
    exe = os.path.join(ROOT, "oracle", "_ref", "test_dequant")
    if not os.path.exists(exe):
        pytest.skip("reference build absent (oracle/_ref)")
    r = subprocess.run([exe], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout
    assert "constants: OK" in r.stdout


def test_e8m0_known_answers(oracle):
    # test_dequant.c:51-56: e8m0_half(127/128/129) = 0.5/1/2; the oracle's
    # scale is the unhalved 2^(e-127)
    assert oracle.e8m0(127) == 1.0
    assert oracle.e8m0(128) == 2.0
    assert oracle.e8m0(129) == 4.0
    assert oracle.e8m0(0) == 2.0 ** -127
    assert oracle.e8m0(254) == 2.0 ** 127


def test_mxfp4_known_answers(oracle):
    # test_dequant.c:58-61: e=128, codes 0..7 -> {0,1,2,3,4,6,8,12}
    blk = np.zeros(17, dtype=np.uint8)
    blk[0] = 128
    blk[1:] = np.arange(16, dtype=np.uint8)
    out = oracle.deq_mxfp4_row(blk)
    assert list(out[:8]) == [0, 1, 2, 3, 4, 6, 8, 12]
    # low nibbles 8..15 are the negated magnitudes; high nibbles are 0
    assert list(out[8:16]) == [-0.0, -1, -2, -3, -4, -6, -8, -12]
    assert np.all(out[16:] == 0)


def test_e2m1_closed_form(oracle):
    # OCP E2M1: s.ee.m, bias 1; subnormal e=0 -> m*0.5
    for c in range(16):
        s, e, m = c >> 3, (c >> 1) & 3, c & 1
        v = m * 0.5 if e == 0 else (1 + m / 2) * 2.0 ** (e - 1)
        assert oracle.e2m1(c) == (-v if s else v)


def test_deq_golden_fixture(oracle):
    """Oracle dequant == reference q36_deq_mxfp4 on the committed vectors."""
    g = np.load(GOLDEN)
    blocks, vals = g["blocks"], g["values"]
    ok = blocks[:, 0] < 255
    out = oracle.deq_mxfp4_row(blocks[ok]).reshape(-1, 32)
    # equal values (code 8 is -0 in OCP E2M1 and +0 in the reference table)
    np.testing.assert_array_equal(out, vals[ok])
    # the reference's halved scale times two is the oracle's scale
    for e in range(255):
        assert oracle.e8m0(e) == 2.0 * float(g["e8m0_half"][e])


def test_deq_exhaustive_vs_reference_build(oracle):
    """All 16 codes in every nibble position x all 255 finite exponents
    against the reference's dequant compiled from its header."""
    ref = oracle.ref_lib()
    if ref is None:
        pytest.skip("reference build absent (oracle/_ref)")
    import ctypes
    codes = np.arange(16, dtype=np.uint8)
    blocks = []
    for e in range(255):
        for sh in range(16):
            b = np.empty(17, dtype=np.uint8)
            b[0] = e
            lo = np.roll(codes, sh)
            hi = np.roll(codes[::-1], sh)
            b[1:] = lo | (hi << 4)
            blocks.append(b)
    blocks = np.stack(blocks)
    mine = oracle.deq_mxfp4_row(blocks).reshape(-1, 32)
    theirs = np.empty_like(mine)
    for i in range(blocks.shape[0]):
        ref.ref_deq_mxfp4(ctypes.c_void_p(blocks[i].ctypes.data),
                          ctypes.c_void_p(theirs[i].ctypes.data))
    np.testing.assert_array_equal(mine, theirs)   # values; +-0 compare equal


# ---------------------------------------------------------------------------
# E4M3
# ---------------------------------------------------------------------------
def _e4m3_closed(b):
    s, e, m = b >> 7, (b >> 3) & 15, b & 7
    if e == 15 and m == 7:
        return float("nan")
    v = m * 2.0 ** -9 if e == 0 else (1 + m / 8) * 2.0 ** (e - 7)
    return -v if s else v


def test_e4m3_decode_all_codes(oracle):
    tab = oracle.e4m3_decode_table()
    lib_vals = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    for b in range(256):
        want = _e4m3_closed(b)
        if np.isnan(want):
            assert np.isnan(tab[b]) and np.isnan(lib_vals[b])
        else:
            assert tab[b] == want == lib_vals[b], b


def test_e4m3_encode_roundtrip_and_ties(oracle):
    tab = oracle.e4m3_decode_table()
    for b in range(256):
        if np.isnan(tab[b]):
            continue
        got = oracle.e4m3_encode(tab[b])
        assert tab[got] == tab[b]                      # +-0 both decode to 0
    # every midpoint between neighbouring positive codes rounds to even
    pos = [b for b in range(0x7f)]
    for b in pos[:-1]:
        lo, hi = float(tab[b]), float(tab[b + 1])
        mid = np.float32((lo + hi) / 2)
        assert float(mid) == (lo + hi) / 2             # exactly representable
        want = b if b % 2 == 0 else b + 1
        assert oracle.e4m3_encode(mid) == want, (b, mid)
        assert oracle.e4m3_encode(-mid) == 0x80 | want
        # just above / below the midpoint
        assert oracle.e4m3_encode(np.nextafter(mid, np.float32(1e9))) == b + 1
        assert oracle.e4m3_encode(np.nextafter(mid, np.float32(-1e9))) == b


def test_quant_exp_infinite_amax(oracle):
    # ceil(log2(inf / 448)) saturates to the largest int, clamped to 127
    assert oracle.quant_exp(float("inf")) == 127
    xq, xs = oracle.quant_e4m3(np.array([[1.0, np.inf] + [0.5] * 30], dtype=np.float32))
    assert xs[0, 0] == 254
    assert xq[0, 0] == 0 and xq[0, 1] == 0x7F and np.all(xq[0, 2:] == 0)


def test_e4m3_encode_saturation_nan(oracle):
    for v in (448.0, 449.0, 463.9, 464.0, 480.0, 1e6, float("inf")):
        assert oracle.e4m3_encode(v) == 0x7E
        assert oracle.e4m3_encode(-v) == 0xFE
    assert oracle.e4m3_encode(float("nan")) & 0x7F == 0x7F


def test_e4m3_encode_vs_torch(oracle):
    """Independent library routine: torch's float -> float8_e4m3fn (RNE) on
    random values inside the finite range."""
    rng = np.random.default_rng(3)
    v = np.concatenate([
        rng.uniform(-460, 460, 20000), rng.standard_normal(20000) * 0.01,
        rng.standard_normal(20000) * 2.0 ** -8, rng.standard_normal(20000) * 50,
    ]).astype(np.float32)
    v = v[np.abs(v) < 464]
    mine = oracle.e4m3_encode_array(v)
    theirs = torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    tab = oracle.e4m3_decode_table()
    np.testing.assert_array_equal(tab[mine], tab[theirs])


# ---------------------------------------------------------------------------
# activation quantiser
# ---------------------------------------------------------------------------
def test_quant_exp_closed_form(oracle):
    rng = np.random.default_rng(4)
    a = np.abs(rng.standard_normal(5000) * 10.0 ** rng.uniform(-30, 30, 5000)).astype(np.float32)
    for x in a:
        e2 = oracle.quant_exp(x)
        q = np.float32(x) / np.float32(448.0)
        if -127 < e2 < 127:
            assert 2.0 ** (e2 - 1) < float(q) <= 2.0 ** e2, (x, e2)
    assert oracle.quant_exp(0.0) == -127
    assert oracle.quant_exp(448.0) == 0
    assert oracle.quant_exp(448.0 * 2 ** 5) == 5
    # the log2f rounding edge: q = 2^n (1 + 2^-23) must give n + 1
    q = np.float32(2.0 ** -5) * np.float32(1 + 2.0 ** -23)
    a_edge = np.float32(q * np.float32(448.0))
    assert np.float32(a_edge) / np.float32(448.0) > np.float32(2.0 ** -5)
    assert oracle.quant_exp(float(a_edge)) == -4


def test_quant_e4m3_invariants(oracle):
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((16, 2048)) * 10.0 ** rng.uniform(-3, 3, (16, 1))).astype(np.float32)
    x[0, :32] = 0.0                                   # all-zero block
    x[1, 5] = 1e-40                                   # fp32 subnormal
    xq, xs = oracle.quant_e4m3(x)
    xd = oracle.dequant_e4m3(xq, xs)
    tab = oracle.e4m3_decode_table()
    for t in range(x.shape[0]):
        for b in range(64):
            blk = x[t, b * 32:(b + 1) * 32].astype(np.float64)
            e2 = int(xs[t, b]) - 127
            a = np.abs(blk).max()
            if a == 0:
                assert e2 == -127 and np.all(xd[t, b * 32:(b + 1) * 32] == 0)
                continue
            # minimal scale: amax fits at e2 but not at e2-1
            assert a <= 448 * 2.0 ** e2 and a > 448 * 2.0 ** (e2 - 1)
            q = tab[xq[t, b * 32:(b + 1) * 32]].astype(np.float64)
            assert np.all(np.abs(q) <= 448)
            # each code is the nearest e4m3 value of v * 2^-e2
            scaled = blk * 2.0 ** -e2
            fin = tab[np.isfinite(tab)].astype(np.float64)
            near = np.abs(scaled[:, None] - fin[None, :]).min(axis=1)
            assert np.all(np.abs(scaled - q) <= near + 1e-12)


# ---------------------------------------------------------------------------
# router top-k and sort
# ---------------------------------------------------------------------------
def _brute_topk(l, k):
    order = sorted(range(len(l)), key=lambda j: (-float(l[j]), j))
    return order[:k]


def test_router_topk_brute_force(oracle):
    rng = np.random.default_rng(6)
    T, E, k = 200, 256, 8
    lg = rng.standard_normal((T, E)).astype(np.float32)
    lg[0, :] = 0.5                                    # all ties
    lg[1, 10:20] = 3.0                                # 10-way tie at the top
    lg[2] = np.round(lg[2] * 2) / 2                   # many ties
    idx, wt = oracle.router_topk(lg, k)
    for t in range(T):
        want = _brute_topk(lg[t], k)
        assert list(idx[t]) == want
        ex = np.exp(lg[t].astype(np.float64) - lg[t].max())
        w = ex[want] / ex[want].sum()
        np.testing.assert_allclose(wt[t], w, rtol=1e-13)
    _, wt2 = oracle.router_topk(lg, k, scale=2.5)
    np.testing.assert_allclose(wt2, 2.5 * wt, rtol=1e-15)
    _, wt3 = oracle.router_topk(lg, k, renorm=False)
    ex = np.exp(lg.astype(np.float64) - lg.max(1, keepdims=True))
    full = ex / ex.sum(1, keepdims=True)
    np.testing.assert_allclose(wt3, np.take_along_axis(full, idx.astype(np.int64), 1), rtol=1e-12)


def test_sort_brute_force(oracle):
    rng = np.random.default_rng(7)
    for T, E in ((1, 256), (3, 8), (64, 256), (4096, 256), (100, 1)):
        k = min(8, E)
        idx = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32)
        off, perm, pos = oracle.sort_entries(idx, E)
        flat = idx.reshape(-1)
        np.testing.assert_array_equal(perm, np.argsort(flat, kind="stable"))
        np.testing.assert_array_equal(pos[perm], np.arange(flat.size))
        np.testing.assert_array_equal(np.diff(off), np.bincount(flat, minlength=E))
        assert off[0] == 0 and off[-1] == flat.size


# ---------------------------------------------------------------------------
# GEMV and the layer
# ---------------------------------------------------------------------------
def _deq_matrix(oracle, W):
    M = W.shape[0]
    return oracle.deq_mxfp4_row(W).reshape(M, -1).astype(np.float64)


def test_gemv_vs_numpy(oracle):
    from q36_amd import synth
    rng = np.random.default_rng(8)
    W = synth.mxfp4_blocks(rng, 512, 2048)
    x = synth.hidden(rng, 1)
    xq, xs = oracle.quant_e4m3(x)
    y = oracle.gemv_mxfp4(W, xq, xs)
    ym = oracle.gemv_mxfp4(W, xq, xs, nthreads=4)
    np.testing.assert_array_equal(y, ym)
    ref = _deq_matrix(oracle, W) @ oracle.dequant_e4m3(xq, xs)[0]
    err = np.abs(y - ref).max() / np.abs(ref).max()
    assert err < 1e-5


def test_gemv_single_block_closed_form(oracle):
    """One non-zero block: y = E2M1(c)*2^(e-127) * x-dot over that block."""
    W = np.zeros((16, 64, 17), dtype=np.uint8)
    W[:, :, 0] = 127
    W[3, 5, 0] = 130                                  # x8
    W[3, 5, 1:] = 0x22                                # every element 1.0
    xq = np.full(2048, 0x38, dtype=np.uint8)          # e4m3 1.0
    xs = np.full(64, 127, dtype=np.uint8)
    y = oracle.gemv_mxfp4(W, xq, xs)
    assert y[3] == 32 * 8.0 and np.all(np.delete(y, 3) == 0)


def _numpy_layer(oracle, w, x, lg, shg, k, act_mode):
    """Independent vectorised fp64 implementation for small shapes."""
    E, FF = w["gate"].shape[:2]
    D = w["down"].shape[1]
    G = np.stack([_deq_matrix(oracle, w["gate"][e]) for e in range(E)])
    U = np.stack([_deq_matrix(oracle, w["up"][e]) for e in range(E)])
    Dn = np.stack([_deq_matrix(oracle, w["down"][e]) for e in range(E)])
    if act_mode in (0, 2):
        xq, xs = oracle.quant_e4m3(x)
        xd = oracle.dequant_e4m3(xq, xs)
    else:
        xd = x.astype(np.float64)
    out = np.zeros((x.shape[0], D))
    for t in range(x.shape[0]):
        sel = _brute_topk(lg[t], k)
        ex = np.exp(lg[t].astype(np.float64) - lg[t].max())[sel]
        wts = ex / ex.sum()
        mats = [(G[e], U[e], Dn[e], wts[i]) for i, e in enumerate(sel)]
        if shg is not None:
            mats.append((_deq_matrix(oracle, w["sh_gate"]), _deq_matrix(oracle, w["sh_up"]),
                         _deq_matrix(oracle, w["sh_down"]), 1 / (1 + np.exp(-float(shg[t])))))
        for g_, u_, d_, wv in mats:
            g = g_ @ xd[t]
            u = u_ @ xd[t]
            h = (g / (1 + np.exp(-g)) * u).astype(np.float32)
            if act_mode == 0:
                hq, hs = oracle.quant_e4m3(h[None])
                hd = oracle.dequant_e4m3(hq, hs)[0]
            elif act_mode == 2:   # the reference's prefill: f32 h rounded to fp16 (numpy's RNE)
                hd = h.astype(np.float16).astype(np.float64)
            else:
                hd = h.astype(np.float64)
            out[t] += wv * (d_ @ hd)
    return out


@pytest.mark.parametrize("act_mode", [0, 1, 2])
def test_layer_vs_numpy(oracle, act_mode):
    from q36_amd import synth
    w = synth.expert_weights(11, n_expert=6, d_model=512, d_ff=512, shared=True)
    rng = np.random.default_rng(12)
    x = synth.hidden(rng, 5, 512)
    lg = synth.normal_logits(rng, 5, 6)
    shg = rng.standard_normal(5).astype(np.float32)
    got = oracle.moe_forward(w, x, lg, shg, k=3, act_mode=act_mode)
    want = _numpy_layer(oracle, w, x, lg, shg, 3, act_mode)
    np.testing.assert_allclose(got, want, rtol=1e-9, atol=1e-9 * np.abs(want).max())


def test_layer_properties(oracle):
    from q36_amd import synth
    E = 8
    w = synth.expert_weights(13, n_expert=E, d_model=512, d_ff=512)
    rng = np.random.default_rng(14)
    x = synth.hidden(rng, 3, 512)
    lg = synth.normal_logits(rng, 3, E)
    base = oracle.moe_forward(w, x, lg, k=4)
    # linear in the routing scale
    np.testing.assert_allclose(oracle.moe_forward(w, x, lg, k=4, scale=2.0), 2 * base, rtol=1e-14)
    # relabelling experts (weights and logits together) changes nothing
    p = rng.permutation(E)
    w2 = {kk: v[p] for kk, v in w.items()}
    np.testing.assert_allclose(oracle.moe_forward(w2, x, lg[:, p], k=4), base, rtol=1e-12)
    # token subset == rows of the full run
    sub = oracle.moe_forward(w, x, lg, k=4, tokens=np.array([2, 0], dtype=np.int32))
    np.testing.assert_array_equal(sub, base[[2, 0]])
    # fp32 accumulation path agrees to fp32 precision
    f = oracle.moe_forward_f32(w, x, lg, k=4)
    assert np.abs(f - base).max() <= 1e-4 * np.abs(base).max()


def test_expert_stages_vs_numpy(oracle):
    from q36_amd import synth
    rng = np.random.default_rng(15)
    g, u = synth.mxfp4_blocks(rng, 64, 512), synth.mxfp4_blocks(rng, 64, 512)
    d = synth.mxfp4_blocks(rng, 512, 64 * 0 + 512)[:, :2]          # [512][64/32]
    xd = rng.standard_normal(512)
    G, U = _deq_matrix(oracle, g), _deq_matrix(oracle, u)
    gv, uv = G @ xd, U @ xd
    np.testing.assert_allclose(oracle.expert_h(g, u, xd), gv / (1 + np.exp(-gv)) * uv, rtol=1e-12)
    hd = rng.standard_normal(64)
    np.testing.assert_allclose(oracle.expert_down(d, hd), _deq_matrix(oracle, d) @ hd, rtol=1e-12,
                               atol=1e-12)


# ---------------------------------------------------------------------------
# the every-token checker of the GPU parity tests (tests/fullcheck.py)
# ---------------------------------------------------------------------------
def _fullcheck():
    import fullcheck   # tests/ is on sys.path under pytest's default import mode
    return fullcheck


@pytest.mark.parametrize("shared", [False, True])
def test_fullcheck_reference_vs_oracle(oracle, shared):
    """The expert-grouped fp64 layer equals the C oracle's per-token forward
    (its own code path: dequant per block, per-token loops)."""
    from q36_amd import synth
    fc = _fullcheck()
    w = synth.expert_weights(31, n_expert=16, d_model=2048, d_ff=512, shared=shared)
    rng = np.random.default_rng(32)
    T = 12
    x = synth.hidden(rng, T)
    lg = synth.normal_logits(rng, T, 16)
    shg = rng.standard_normal(T).astype(np.float32) if shared else None
    got = fc.layer_reference(oracle, w, x, lg, shg, k=4)
    want = oracle.moe_forward(w, x, lg, shg, k=4)
    np.testing.assert_allclose(got, want, rtol=1e-9, atol=1e-9 * np.abs(want).max())


def test_fullcheck_accepts_oracle_codes_and_rejects_a_wrong_row(oracle):
    """Fed h codes from the oracle's per-token path (expert_h + quantiser)
    and the oracle's output, the checker finds no flip and no error; the
    row's largest code moved by one step (far from a midpoint: the flip
    allowance is 1e-4 of the block maximum), or 1% taken off a token's
    output, fails it."""
    from q36_amd import synth
    fc = _fullcheck()
    E, k, T = 16, 4, 10
    w = synth.expert_weights(33, n_expert=E, d_model=2048, d_ff=512)
    rng = np.random.default_rng(34)
    x = synth.hidden(rng, T)
    lg = synth.normal_logits(rng, T, E)
    gi, _ = oracle.router_topk(lg, k, n_expert=E)
    xq, xs = oracle.quant_e4m3(x)
    xd = oracle.dequant_e4m3(xq, xs)
    pos = np.arange(T * k, dtype=np.int32)[::-1].copy()      # any bijection of rows
    hq = np.zeros((T * k, 512), np.uint8)
    hs = np.zeros((T * k, 16), np.uint8)
    for t in range(T):
        for s in range(k):
            h = oracle.expert_h(w["gate"][gi[t, s]], w["up"][gi[t, s]], xd[t]).astype(np.float32)
            q, sc = oracle.quant_e4m3(h[None])
            hq[pos[t * k + s]], hs[pos[t * k + s]] = q[0], sc[0]
    y = oracle.moe_forward(w, x, lg, k=k).astype(np.float32)
    m = fc.check_every_token(oracle, w, x, lg, None, y, gi, pos, hq, hs, k=k)
    assert m["h_flips"] == 0 and m["e2e_max_rel"] < 1e-6
    bad = hq.copy()
    col = int(np.argmax(bad[5] & 0x7f))       # the row's largest code: far from any midpoint
    bad[5, col] ^= 0x01
    with pytest.raises(AssertionError):
        fc.check_every_token(oracle, w, x, lg, None, y, gi, pos, bad, hs, k=k)
    y2 = y.copy()
    y2[3] -= oracle.moe_forward(w, x[3:4], lg[3:4], k=k)[0].astype(np.float32) * 0.01
    with pytest.raises(AssertionError):
        fc.check_every_token(oracle, w, x, lg, None, y2, gi, pos, hq, hs, k=k)
