"""GGUF ingest (q36moe_gguf_*, q36moe_weights_from_gguf,
q36moe_router_from_gguf).  The reader is checked against the reference's
own reader (gguf.c, compiled from its sources into oracle/_ref by
oracle/Makefile) on the same synthetic files; the upload is checked on the
GPU against q36moe_weights_upload of the same block arrays."""
import ctypes
import os

import numpy as np
import pytest
import torch

from q36_amd import moe, synth
from tests import gguf_file as gf

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_GGUF = os.path.join(ROOT, "oracle", "_ref", "libref_gguf.so")
D, FF = 2048, 512


def _layer_file(path, E=16, layer=0, router_bf16=False, shared="mxfp4", seed=5, alignment=64,
                down_type=gf.T_MXFP4, gate_type=gf.T_MXFP4):
    """One MoE block of a q36-style file with E experts, plus unrelated
    metadata and tensors; returns the arrays written.  down_type 13 / 14 / 8
    writes a Q5_K / Q6_K / Q8_0 down (the k-quant experts of real files);
    gate_type other than MXFP4 only relabels the gate bytes (for rejection
    tests)."""
    rng = np.random.default_rng(seed)
    w = synth.expert_weights(seed, n_expert=E, shared=True)
    if down_type != gf.T_MXFP4:
        w["down"] = synth.kquant_blocks(rng, E * D, FF, down_type).reshape(E, D, -1)
    router = (rng.standard_normal((E, D)) * 0.02).astype(np.float32)
    shg_row = (rng.standard_normal(D) * 0.02).astype(np.float32)
    norm = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    p = f"blk.{layer}."
    kvs = [("general.architecture", gf.STR, "qwen35moe"),
           ("general.alignment", gf.U32, alignment),
           ("qwen35moe.expert_count", gf.U32, E),
           ("qwen35moe.expert_used_count", gf.U32, 8),
           ("qwen35moe.rope.freq_base", gf.F32, 1e7),
           ("tokenizer.ggml.tokens", gf.ARR, (gf.STR, ["<a>", "bb", "c"])),
           ("tokenizer.ggml.token_type", gf.ARR, (gf.I32, [1, 2, 3])),
           ("general.file_type", gf.U64, 39)]
    tensors = [(p + "post_attention_norm.weight", [D], gf.T_F32, norm.tobytes()),
               (p + "ffn_gate_inp.weight", [D, E], gf.T_BF16 if router_bf16 else gf.T_F32,
                gf.bf16_bytes(router) if router_bf16 else router.tobytes()),
               (p + "ffn_gate_inp_shexp.weight", [D], gf.T_BF16, gf.bf16_bytes(shg_row)),
               (p + "ffn_gate_exps.weight", [D, FF, E], gate_type, w["gate"].tobytes()),
               (p + "ffn_up_exps.weight", [D, FF, E], gf.T_MXFP4, w["up"].tobytes()),
               (p + "ffn_down_exps.weight", [FF, D, E], down_type, w["down"].tobytes()),
               ("token_embd.weight", [64, 8], gf.T_Q8_0, bytes(8 * 2 * 34))]
    if shared == "mxfp4":
        tensors += [(p + "ffn_gate_shexp.weight", [D, FF], gf.T_MXFP4, w["sh_gate"].tobytes()),
                    (p + "ffn_up_shexp.weight", [D, FF], gf.T_MXFP4, w["sh_up"].tobytes()),
                    (p + "ffn_down_shexp.weight", [FF, D], gf.T_MXFP4, w["sh_down"].tobytes())]
    elif shared in ("q8_0", "mixed"):   # the release file's shared expert type
        for n, dims in (("sh_gate", [D, FF]), ("sh_up", [D, FF]), ("sh_down", [FF, D])):
            w[n] = synth.kquant_blocks(rng, dims[1], dims[0], gf.T_Q8_0)
        # "mixed": the down relabelled MXFP4 (one type is required for all three)
        sh_down_t = gf.T_MXFP4 if shared == "mixed" else gf.T_Q8_0
        tensors += [(p + "ffn_gate_shexp.weight", [D, FF], gf.T_Q8_0, w["sh_gate"].tobytes()),
                    (p + "ffn_up_shexp.weight", [D, FF], gf.T_Q8_0, w["sh_up"].tobytes()),
                    (p + "ffn_down_shexp.weight", [FF, D], sh_down_t,
                     w["sh_down"].tobytes()[:FF * D // 32 * 17] if shared == "mixed" else w["sh_down"].tobytes())]
    gf.write(path, kvs, tensors, alignment=alignment)
    return {"w": w, "router": router, "shg_row": shg_row, "tensors": tensors, "n_kv": len(kvs)}


# --- the reference reader (gguf.h layout), loaded only as a checker --------
class _Str(ctypes.Structure):
    _fields_ = [("ptr", ctypes.c_char_p), ("len", ctypes.c_uint64)]


class _Tensor(ctypes.Structure):
    _fields_ = [("name", _Str), ("n_dims", ctypes.c_uint32), ("dims", ctypes.c_uint64 * 4),
                ("ggml_type", ctypes.c_uint32), ("offset", ctypes.c_uint64), ("data", ctypes.c_void_p),
                ("nbytes", ctypes.c_uint64)]


class _File(ctypes.Structure):
    _fields_ = [("fd", ctypes.c_int), ("map", ctypes.c_void_p), ("map_size", ctypes.c_size_t),
                ("version", ctypes.c_uint32), ("n_tensors", ctypes.c_uint64), ("n_kv", ctypes.c_uint64),
                ("kv", ctypes.c_void_p), ("tensors", ctypes.POINTER(_Tensor)),
                ("data_base", ctypes.c_void_p), ("alignment", ctypes.c_uint32)]


@pytest.fixture(scope="module")
def ref():
    if not os.path.exists(REF_GGUF):
        pytest.skip("reference GGUF reader not built (oracle/_ref absent)")
    L = ctypes.CDLL(REF_GGUF)
    L.gguf_open.argtypes = [ctypes.POINTER(_File), ctypes.c_char_p, ctypes.c_char_p, ctypes.c_size_t]
    L.gguf_close.argtypes = [ctypes.POINTER(_File)]
    L.gguf_close.restype = None
    L.gguf_tensor_find.argtypes = [ctypes.POINTER(_File), ctypes.c_char_p]
    L.gguf_tensor_find.restype = ctypes.POINTER(_Tensor)
    L.gguf_u32.argtypes = [ctypes.POINTER(_File), ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint32)]
    L.gguf_u32.restype = ctypes.c_bool
    return L


def _ref_open(ref, path):
    f = _File()
    err = ctypes.create_string_buffer(256)
    rc = ref.gguf_open(ctypes.byref(f), os.fsencode(path), err, 256)
    return rc, f


@pytest.mark.parametrize("alignment,router_bf16", [(32, False), (64, True), (4096, False)])
def test_reader_matches_reference(tmp_path, ref, alignment, router_bf16):
    path = str(tmp_path / "l.gguf")
    spec = _layer_file(path, alignment=alignment, router_bf16=router_bf16)
    rc, rf = _ref_open(ref, path)
    assert rc == 0
    try:
        with moe.GGUF(path) as g:
            info = g.info()
            assert info["version"] == rf.version == 3
            assert info["n_tensors"] == rf.n_tensors == len(spec["tensors"])
            assert info["n_kv"] == rf.n_kv == spec["n_kv"]
            assert info["alignment"] == rf.alignment == alignment
            assert info["data_offset"] == rf.data_base - rf.map
            for name, dims, ty, data in spec["tensors"]:
                mine = g.tensor(name)
                t = ref.gguf_tensor_find(ctypes.byref(rf), name.encode()).contents
                assert mine["type"] == t.ggml_type == ty
                assert mine["n_dims"] == t.n_dims == len(dims)
                assert mine["dims"][:len(dims)] == list(t.dims)[:len(dims)] == dims
                assert mine["file_offset"] == t.data - rf.map
                if ty != gf.T_BF16:   # the reference reader has no BF16 block size (nbytes 0)
                    assert mine["nbytes"] == t.nbytes == len(data)
                else:
                    assert mine["nbytes"] == len(data)
                raw = ctypes.string_at(rf.map + mine["file_offset"], len(data))
                assert raw == bytes(data)
            v = ctypes.c_uint32()
            assert ref.gguf_u32(ctypes.byref(rf), b"qwen35moe.expert_count", ctypes.byref(v))
            assert g.u32("qwen35moe.expert_count") == v.value == 16
    finally:
        ref.gguf_close(ctypes.byref(rf))


def _corrupt(path, out, fn):
    b = bytearray(open(path, "rb").read())
    open(out, "wb").write(bytes(fn(b)))


@pytest.mark.parametrize("case", ["magic", "version", "truncated_dir", "past_eof", "huge_count"])
def test_reader_rejects_malformed(tmp_path, ref, case):
    good = str(tmp_path / "g.gguf")
    _layer_file(good, E=2)
    bad = str(tmp_path / "b.gguf")
    if case == "magic":
        _corrupt(good, bad, lambda b: b"GGUG" + b[4:])
    elif case == "version":
        _corrupt(good, bad, lambda b: b[:4] + (2).to_bytes(4, "little") + b[8:])
    elif case == "truncated_dir":
        _corrupt(good, bad, lambda b: b[:300])
    elif case == "past_eof":   # drop the last tensor's data
        _corrupt(good, bad, lambda b: b[:-4096])
    else:                      # a tensor count no file of this size can hold
        _corrupt(good, bad, lambda b: b[:8] + (1 << 40).to_bytes(8, "little") + b[16:])
    if case != "huge_count":   # the reference allocates the count unchecked: not run on it
        rc, rf = _ref_open(ref, bad)
        if rc == 0:
            ref.gguf_close(ctypes.byref(rf))
        assert rc != 0
    with pytest.raises(moe.Q36MoEError) as e:
        moe.GGUF(bad)
    assert "-22" in str(e.value)


def test_reader_missing_file_and_names(tmp_path):
    with pytest.raises(moe.Q36MoEError) as e:
        moe.GGUF(str(tmp_path / "none.gguf"))
    assert "-5" in str(e.value)
    path = str(tmp_path / "l.gguf")
    _layer_file(path, E=2)
    with moe.GGUF(path) as g:
        with pytest.raises(moe.Q36MoEError) as e:
            g.tensor("blk.7.ffn_gate_exps.weight")
        assert "-2" in str(e.value)
        with pytest.raises(moe.Q36MoEError):
            g.u32("general.architecture")     # a string, not a u32


@pytest.mark.parametrize("router_bf16", [False, True])
def test_router_from_gguf(tmp_path, router_bf16):
    path = str(tmp_path / "l.gguf")
    spec = _layer_file(path, E=16, router_bf16=router_bf16)
    with moe.GGUF(path) as g:
        rows = g.router(0)
    assert rows.shape == (17, D)
    def widened(a):
        return np.frombuffer(gf.bf16_bytes(a), dtype=np.uint16).astype(np.uint32) << 16
    want = spec["router"].view(np.uint32) if not router_bf16 else widened(spec["router"]).reshape(16, D)
    np.testing.assert_array_equal(rows[:16].view(np.uint32), want)
    np.testing.assert_array_equal(rows[16].view(np.uint32), widened(spec["shg_row"]))


def test_weights_from_gguf_rejects_before_upload(tmp_path):
    """Type and name checks run before any device call."""
    path = str(tmp_path / "l.gguf")
    _layer_file(path, E=2, shared="mixed")
    L = moe.lib()
    with moe.GGUF(path) as g:
        h = ctypes.c_void_p()
        assert L.q36moe_weights_from_gguf(g._h, 0, 1, ctypes.byref(h)) == -22   # shared tensors of two types
        assert L.q36moe_weights_from_gguf(g._h, 3, 0, ctypes.byref(h)) == -2    # no block 3
        assert L.q36moe_weights_from_gguf(g._h, -1, 0, ctypes.byref(h)) == -22
    # routed gate/up must be MXFP4 (the bytes are relabelled Q8_0 here: a
    # type error, caught before the size of the data matters)
    _layer_file(path, E=2, gate_type=gf.T_Q8_0)
    with moe.GGUF(path) as g:
        assert L.q36moe_weights_from_gguf(g._h, 0, 0, ctypes.byref(h)) == -22


@pytest.mark.gpu
@pytest.mark.parametrize("down_type", [gf.T_Q5_K, gf.T_Q6_K])
def test_weights_from_gguf_kquant_down(tmp_path, down_type):
    """A k-quant down projection (blk.0.ffn_down_exps of the real file is
    Q5_K) ingested from the file gives bit-identical outputs to
    q36moe_weights_upload_typed of the same blocks, on the direct and the
    sorted path, with the MXFP4 shared expert."""
    dev = torch.device("cuda:0")
    path = str(tmp_path / "l.gguf")
    spec = _layer_file(path, E=16, down_type=down_type)
    w = spec["w"]
    with moe.GGUF(path) as g:
        wg = moe.MoEWeights.from_gguf(g, 0, with_shared=True)
    assert wg.down_type == gf.T_Q8_0
    wu = moe.MoEWeights.upload(w["gate"], w["up"], w["down"], w["sh_gate"], w["sh_up"], w["sh_down"],
                               down_type=down_type)
    for T in (3, 40):
        rng = np.random.default_rng(80 + T)
        x = torch.from_numpy(synth.hidden(rng, T)).to(dev)
        lg = torch.from_numpy(rng.standard_normal((T, 16)).astype(np.float32)).to(dev)
        shg = torch.from_numpy(rng.standard_normal(T).astype(np.float32)).to(dev)
        outs = []
        for wt in (wg, wu):
            layer = moe.MoELayer(T, n_expert=16)
            outs.append(layer.forward(wt, x, lg, shg, out_dtype=torch.float32).cpu().numpy())
        torch.cuda.synchronize()
        np.testing.assert_array_equal(outs[0], outs[1])
        assert np.abs(outs[0]).max() > 0


@pytest.mark.gpu
def test_weights_from_gguf_q8_0_shared(tmp_path):
    """The release file's layout: MXFP4 experts with a Q5_K down and a Q8_0
    shared expert, ingested from the file, give bit-identical outputs to the
    typed upload of the same blocks (direct and sorted paths)."""
    dev = torch.device("cuda:0")
    path = str(tmp_path / "l.gguf")
    spec = _layer_file(path, E=16, shared="q8_0", down_type=gf.T_Q5_K)
    w = spec["w"]
    with moe.GGUF(path) as g:
        wg = moe.MoEWeights.from_gguf(g, 0, with_shared=True)
    assert wg.shared_type == gf.T_Q8_0 and wg.down_type == gf.T_Q8_0
    wu = moe.MoEWeights.upload(w["gate"], w["up"], w["down"], w["sh_gate"], w["sh_up"], w["sh_down"],
                               down_type=gf.T_Q5_K, sh_type=gf.T_Q8_0)
    for T in (3, 40):
        rng = np.random.default_rng(90 + T)
        x = torch.from_numpy(synth.hidden(rng, T)).to(dev)
        lg = torch.from_numpy(rng.standard_normal((T, 16)).astype(np.float32)).to(dev)
        shg = torch.from_numpy(rng.standard_normal(T).astype(np.float32)).to(dev)
        outs = []
        for wt in (wg, wu):
            layer = moe.MoELayer(T, n_expert=16)
            outs.append(layer.forward(wt, x, lg, shg, out_dtype=torch.float32).cpu().numpy())
        torch.cuda.synchronize()
        np.testing.assert_array_equal(outs[0], outs[1])
        assert np.abs(outs[0]).max() > 0


@pytest.mark.gpu
@pytest.mark.parametrize("T", [1, 40])
def test_weights_from_gguf_equals_upload(tmp_path, T):
    """Experts + shared expert ingested from the file give bit-identical
    layer outputs to q36moe_weights_upload of the same block arrays."""
    dev = torch.device("cuda:0")
    path = str(tmp_path / "l.gguf")
    spec = _layer_file(path, E=16)
    w = spec["w"]
    with moe.GGUF(path) as g:
        wg = moe.MoEWeights.from_gguf(g, 0, with_shared=True)
        router = g.router(0)
    wu = moe.MoEWeights.upload(w["gate"], w["up"], w["down"], w["sh_gate"], w["sh_up"], w["sh_down"])
    rng = np.random.default_rng(70 + T)
    x = torch.from_numpy(synth.hidden(rng, T)).to(dev)
    lg = torch.from_numpy(rng.standard_normal((T, 16)).astype(np.float32)).to(dev)
    shg = torch.from_numpy(rng.standard_normal(T).astype(np.float32)).to(dev)
    outs = []
    for wt in (wg, wu):
        layer = moe.MoELayer(T, n_expert=16)
        outs.append(layer.forward(wt, x, lg, shg, out_dtype=torch.float32).cpu().numpy())
    torch.cuda.synchronize()
    np.testing.assert_array_equal(outs[0], outs[1])
    # the router rows feed q36moe_router_logits as read
    lgr, shr = moe.router_logits(torch.from_numpy(router).to(dev), x, 16)
    ref = x.cpu().double().numpy() @ router.astype(np.float64).T
    mag = np.abs(x.cpu().double().numpy()) @ np.abs(router.astype(np.float64)).T
    got = np.concatenate([lgr.cpu().numpy(), shr.cpu().numpy()[:, None]], axis=1)
    f16 = T > 16
    if not f16:
        assert (np.abs(got - ref) / mag).max() <= 2e-6
