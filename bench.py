"""Benchmark of the W4A8 MoE layer on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config decode1]

A step is one MoE layer forward (router logits in, combined bf16 hidden out)
over one batch of synthetic inputs already resident in HBM.  Weights rotate
over --layers distinct seeded layers (40 x 428 MB = 17 GB by default) so the
256 MB MALL cannot serve them.  Prints ONE JSON line (rank 0).

Workload (configs of the q36 MoE layer, hidden 2048, 256 experts, top-8,
expert FF 512, MXFP4 weights, e4m3 activations with per-32 E8M0 scales):
  decode1      T=1, N(0,1) router logits (the headline configuration)
  decode2/4/8/16  T=2/4/8/16, N(0,1) router logits (decode batches)
  decode32     T=32, N(0,1) router logits (decode batch)
  ragged64     T=64, Zipf(1.1) expert popularity
  prefill4096  T=4096, N(0,1) logits
  mixed        T=4006 (6x1 decode + 3000 + 1000 prefill) + shared expert

--down-type q5_k runs the same configuration with the routed down
projection uploaded as Q5_K blocks (the k-quant experts of real files,
requantised on upload to int8 + f16 per 32, h quantised to int8 + fp32 per
32, down on int8 MFMA); --shared-type q8_0 (configurations with a shared
expert) uploads the shared expert as Q8_0 blocks, as the release file has it
(int8 x and h, int8 MFMA).  These weights are host-generated and uploaded, so
such runs rotate fewer layers (--layers defaults to 16) and have no CPU leg.

The roofline object is for the dominant kernel of the configuration, timed
with HIP events around that kernel on the stream it runs on; cpu_baseline is
the C oracle's fp32 layer forward (oracle/liboracle.so) on host cores.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E
MFMA_FP8_PEAK_TFS = 5000.0   # dense FP8 MFMA (scaled f8f6f4 with an e4m3 operand)
D, E, FF, K = 2048, 256, 512, 8
MAT_BYTES = D * FF // 2 + D * FF // 32         # one packed expert matrix, 557,056 B
EXPERT_BYTES = 3 * MAT_BYTES                   # gate + up + down, 1,671,168 B
Q8_MAT_BYTES = D * FF + D * FF // 16           # q8_0-split down matrix, 1,114,112 B

CONFIGS = {
    "decode1": dict(T=1, shared=False, steps=2000, warmup=200),
    "decode2": dict(T=2, shared=False, steps=2000, warmup=200),
    "decode4": dict(T=4, shared=False, steps=2000, warmup=200),
    "decode8": dict(T=8, shared=False, steps=2000, warmup=200),
    "decode16": dict(T=16, shared=False, steps=2000, warmup=200),
    "decode32": dict(T=32, shared=False, steps=1000, warmup=100),
    "ragged64": dict(T=64, shared=False, steps=1000, warmup=100),
    "prefill4096": dict(T=4096, shared=False, steps=100, warmup=10),
    "mixed": dict(T=4006, shared=True, steps=100, warmup=10),
}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--config", default="decode1", choices=sorted(CONFIGS))
    ap.add_argument("--layers", type=int, default=None, help="weight layers rotated (40; 16 for q5_k)")
    ap.add_argument("--down-type", default="mxfp4", choices=["mxfp4", "q5_k"],
                    help="format of the routed down projection")
    ap.add_argument("--shared-type", default="mxfp4", choices=["mxfp4", "q8_0"],
                    help="format of the shared expert (configurations with one)")
    ap.add_argument("--inputs", type=int, default=16, help="distinct input batches cycled")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--path", type=int, default=0, help="q36moe_ctx_set_path mode (0 auto)")
    ap.add_argument("--graph", type=int, default=1,
                    help="1: time a HIP graph of one forward per weight layer (how a model's "
                         "layer loop runs when captured); 0: eager launches only")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="only run a plain device copy of this many MiB (counter calibration)")
    return ap.parse_args()


def make_inputs(cfg_name, T, n, seed, dev):
    import torch
    from q36_amd import synth
    xs, ls, ss = [], [], []
    for j in range(n):
        rng = np.random.default_rng(seed + j)
        x = synth.hidden(rng, T)
        if cfg_name == "ragged64":
            lg = synth.zipf_logits(rng, T)
        else:
            lg = synth.normal_logits(rng, T)
        xs.append(torch.from_numpy(x).to(dev))
        ls.append(torch.from_numpy(lg).to(dev))
        ss.append(torch.from_numpy(rng.standard_normal(T).astype(np.float32)).to(dev))
    return xs, ls, ss


def distinct_experts(layer, moe):
    idx = layer.tap(moe.TAP_TOPK_IDX).cpu().numpy()
    return int(np.unique(idx).size)


def kernel_bytes(stage, T, U, shared, dn_q8=False, sh_q8=False):
    """Algorithmic HBM bytes of one launch of a stage.  U = distinct routed
    experts hit; P = routed (token, slot) rows, plus T shared rows.  A
    q8_0-split matrix is int8 + f16 per 32; int8 activations carry an fp32
    scale per 32 (h rows of a q8_0-split down; x of a q8_0-split shared
    expert, read besides the e4m3 x)."""
    P = T * K + (T if shared else 0)
    sh_mat = Q8_MAT_BYTES if sh_q8 else MAT_BYTES
    xq = T * D + T * D // 32 + (T * D + T * D // 8 if sh_q8 else 0)
    hq = T * K * FF + T * K * FF // 32 * (4 if dn_q8 else 1)
    if shared:
        hq += T * FF + T * FF // 32 * (4 if sh_q8 else 1)
    if stage == "gateup":
        # gate+up weights of the hit experts, the activations, h out
        return U * 2 * MAT_BYTES + (2 * sh_mat if shared else 0) + xq + hq
    if stage == "down":
        # down weights, h in, weighted f32 rows out
        dn = U * (Q8_MAT_BYTES if dn_q8 else MAT_BYTES) + (sh_mat if shared else 0)
        return dn + hq + P * D * 4
    raise ValueError(stage)


def kernel_flops(stage, T, shared):
    P = T * K + (T if shared else 0)
    return P * (2 * D * 2 * FF if stage == "gateup" else 2 * FF * D)


def measured_traffic(config, stage):
    """HBM bytes per launch of a stage's kernel from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary (profiles/hbm_traffic.md), each counter
    scaled by its reading on a plain copy of known size; None when absent."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic.md")
    if not os.path.exists(path):
        return None
    for line in open(path):
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) >= 5 and cells[0] == config and cells[1] == stage:
            try:
                return float(cells[4])
            except ValueError:
                return None
    return None


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _layer_tokens_per_s(pyoracle, w, cfg_name, T, shared, seconds, nth, seed):
    from q36_amd import synth
    rng = np.random.default_rng(seed)
    busy, tokens, t0 = 0.0, 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        Tb = min(T, 4)
        x = synth.hidden(rng, Tb)
        lg = synth.zipf_logits(rng, Tb) if cfg_name == "ragged64" else synth.normal_logits(rng, Tb)
        shg = rng.standard_normal(Tb).astype(np.float32) if shared else None
        t1 = time.perf_counter()
        pyoracle.moe_forward_f32(w, x, lg, shg, nthreads=nth)
        busy += time.perf_counter() - t1
        tokens += Tb
    return tokens / busy, tokens, busy


def _gemv_config0(pyoracle, nth, seconds):
    """one 512x2048 MXFP4 matrix times one e4m3 vector
    (dequant + GEMV, fp32 accumulation), through the oracle port; and the
    reference's own q36_deq_row (built from its sources into oracle/_ref)
    timed on the same blocks for the dequant alone, where it is present."""
    from q36_amd import synth
    rng = np.random.default_rng(9)
    W = synth.mxfp4_blocks(rng, 512, 2048)
    xq, xs = pyoracle.quant_e4m3(synth.hidden(rng, 1))
    out = {}
    for threads in (1, nth):
        n, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < seconds:
            pyoracle.gemv_mxfp4(W, xq, xs, nthreads=threads)
            n += 1
        out[f"port_gemv_us_{threads}t"] = (time.perf_counter() - t0) / n * 1e6
    ref = pyoracle.ref_lib()
    if ref is not None:
        import ctypes
        buf = np.ascontiguousarray(W.reshape(-1))
        row = np.empty(2048, dtype=np.float32)
        n, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < seconds:
            for r in range(512):
                ref.ref_deq_row(39, ctypes.c_void_p(buf.ctypes.data + r * 64 * 17), 2048,
                                ctypes.c_void_p(row.ctypes.data))
            n += 1
        out["reference_dequant_us_1t"] = (time.perf_counter() - t0) / n * 1e6
    return out


def cpu_baseline(cfg_name, T, seconds, shared):
    """The C oracle's fp32 layer forward on host cores over a bounded sample
    of tokens of the same configuration (OpenMP over the host's cores, and
    a shorter single-threaded sample), plus BASELINE config 0 (the CPU
    dequant + GEMV of one expert matrix)."""
    from oracle import pyoracle
    from q36_amd import synth
    pyoracle.lib()
    nth = len(os.sched_getaffinity(0))
    w = synth.expert_weights(7, shared=shared)
    value, tokens, busy = _layer_tokens_per_s(pyoracle, w, cfg_name, T, shared, seconds, nth, 8)
    single, tok1, busy1 = _layer_tokens_per_s(pyoracle, w, cfg_name, T, shared, seconds / 4, 1, 18)
    return {"value": value, "unit": "tokens/s", "cores": nth, "kind": "port",
            "sample": f"{tokens} tokens of {cfg_name} (batches of <=4) through or_moe_forward_f32, "
                      f"{busy:.1f} s, OpenMP {nth} threads",
            "single_thread": {"value": single, "unit": "tokens/s", "cores": 1,
                              "sample": f"{tok1} tokens, {busy1:.1f} s"},
            "cpu_model": _cpu_model(),
            "config0_gemv": _gemv_config0(pyoracle, nth, 1.0)}


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU; --gpus must be 1 "
                                   "(expert-parallel sharding is described in DESIGN.md, not run)"}))
        sys.exit(2)
    import torch
    from q36_amd import moe

    if args.copy_mib:
        # a plain copy of known size: the reference point that scales the
        # FETCH_SIZE / WRITE_SIZE counters of the layer kernels
        n = args.copy_mib << 20
        src = torch.ones(n, dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(4):
            dst.copy_(src)
        torch.cuda.synchronize()
        # achievable-bandwidth reference points: the copy (read + write) and a
        # read-only reduction over the same bytes, as f32
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
        f = src.view(torch.float32)
        f.sum()
        ev[0].record()
        for _ in range(10):
            dst.copy_(src)
        ev[1].record()
        ev[2].record()
        for _ in range(10):
            f.sum()
        ev[3].record()
        torch.cuda.synchronize()
        copy_us = ev[0].elapsed_time(ev[1]) * 100.0
        read_us = ev[2].elapsed_time(ev[3]) * 100.0
        print(json.dumps({"copy_bytes": n, "launches": 4,
                          "copy_us": copy_us, "copy_gbs": 2 * n / copy_us / 1e3,
                          "read_us": read_us, "read_gbs": n / read_us / 1e3}))
        return

    cfg = CONFIGS[args.config]
    T, shared = cfg["T"], cfg["shared"]
    steps = args.steps if args.steps is not None else cfg["steps"]
    warmup = args.warmup if args.warmup is not None else cfg["warmup"]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream()

    dn_q8 = args.down_type == "q5_k"
    sh_q8 = shared and args.shared_type == "q8_0"
    host_up = dn_q8 or sh_q8
    if args.layers is None:
        args.layers = 16 if host_up else 40
    layers = []
    for l in range(args.layers):
        if host_up:
            from q36_amd import synth
            sw = synth.expert_weights(args.seed * 1000 + l, shared=shared)
            rng = np.random.default_rng(args.seed * 1000 + l)
            dn, dn_t = sw["down"], 39   # MXFP4
            if dn_q8:
                dn, dn_t = synth.kquant_blocks(rng, E * D, FF, synth.GGML_Q5_K).reshape(E, D, -1), synth.GGML_Q5_K
            sh_t = 39
            if sh_q8:
                sh_t = synth.GGML_Q8_0
                sw["sh_gate"] = synth.kquant_blocks(rng, FF, D, sh_t)
                sw["sh_up"] = synth.kquant_blocks(rng, FF, D, sh_t)
                sw["sh_down"] = synth.kquant_blocks(rng, D, FF, sh_t)
            w = moe.MoEWeights.upload(sw["gate"], sw["up"], dn, sw.get("sh_gate"), sw.get("sh_up"),
                                      sw.get("sh_down"), down_type=dn_t, sh_type=sh_t)
            del sw, dn
        else:
            w = moe.MoEWeights.alloc(E, D, FF, FF if shared else 0)
            w.fill_synthetic(args.seed * 1000 + l)
        layers.append(w)
    xs, ls, ss = make_inputs(args.config, T, args.inputs, args.seed, dev)
    layer = moe.MoELayer(T, stream=stream)
    layer.set_path(args.path)
    out = torch.empty((T, D), dtype=torch.bfloat16, device=dev)
    torch.cuda.synchronize()

    def step(i):
        j = i % args.inputs
        layer.forward(layers[i % args.layers], xs[j], ls[j], ss[j] if shared else None,
                      out=out)

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record(stream)
    for i in range(steps):
        step(warmup + i)
    ev1.record(stream)
    torch.cuda.synchronize()
    ms_eager = ev0.elapsed_time(ev1) / steps
    ms = ms_eager
    graph_layers = 0
    if args.graph:
        # one forward per weight layer (inputs cycling) captured once, then
        # replayed: the host issues one launch per args.layers layers
        graph_layers = args.layers
        cap = torch.cuda.Stream()
        layer.set_stream(cap)
        with torch.cuda.stream(cap):
            for i in range(graph_layers):
                step(i)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=cap):
            for i in range(graph_layers):
                step(i)
        torch.cuda.synchronize()
        layer.set_stream(stream)
        reps = max(1, steps // graph_layers)
        g.replay()
        torch.cuda.synchronize()
        ev0.record(stream)
        for _ in range(reps):
            g.replay()
        ev1.record(stream)
        torch.cuda.synchronize()
        ms = ev0.elapsed_time(ev1) / (reps * graph_layers)
        steps = reps * graph_layers

    # per-kernel durations: one more forward fixes the stage inputs, then
    # each stage's kernels are launched again `reps` times back to back over
    # the rotating weight sets, bracketed by two HIP events on the layer's
    # stream (the stream the kernels run on)
    step(0)
    torch.cuda.synchronize()
    U = distinct_experts(layer, moe)
    reps = max(50, min(2000, int(2e5 / max(ms * 1e3, 1.0))))
    st_us = {}
    for st in moe.MoELayer.STAGES:
        for i in range(5):
            layer.replay(layers[i % args.layers], st)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for i in range(reps):
            layer.replay(layers[i % args.layers], st)
        e1.record(stream)
        torch.cuda.synchronize()
        st_us[st] = 1e3 * e0.elapsed_time(e1) / reps
    # stages without kernels on this path time as the empty-launch floor;
    # report them as 0
    path = layer.last_path
    if path == 1:
        for st in ("route", "scan", "combine"):
            st_us[st] = 0.0
    dom = "gateup" if st_us["gateup"] >= st_us["down"] else "down"
    prefill = T >= 256
    if prefill:
        fl = kernel_flops(dom, T, shared)
        ach = fl / (st_us[dom] * 1e-6) / 1e12
        roof = {"bound": "mfma", "achieved": ach, "peak": MFMA_FP8_PEAK_TFS, "unit": "TFLOP/s",
                "frac": ach / MFMA_FP8_PEAK_TFS, "traffic": None, "kernel": dom,
                "kernel_us": st_us[dom], "flops_per_launch": fl,
                "hbm_gbs": kernel_bytes(dom, T, U, shared, dn_q8, sh_q8) / (st_us[dom] * 1e-6) / 1e9}
    else:
        by = kernel_bytes(dom, T, U, shared, dn_q8, sh_q8)
        ach = by / (st_us[dom] * 1e-6) / 1e9
        roof = {"bound": "hbm", "achieved": ach, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": ach / HBM_PEAK_GBS, "traffic": None, "kernel": dom,
                "kernel_us": st_us[dom], "bytes_per_launch": by}
    roof["traffic"] = None if host_up else measured_traffic(args.config, dom)
    # both grouped GEMMs against both ceilings (the dominant one is `roof`)
    gemm = {}
    for st in ("gateup", "down"):
        fl, by = kernel_flops(st, T, shared), kernel_bytes(st, T, U, shared, dn_q8, sh_q8)
        gemm[st] = {"us": st_us[st], "tflops": fl / (st_us[st] * 1e-6) / 1e12,
                    "mfma_frac": fl / (st_us[st] * 1e-6) / 1e12 / MFMA_FP8_PEAK_TFS,
                    "gbs": by / (st_us[st] * 1e-6) / 1e9,
                    "hbm_frac": by / (st_us[st] * 1e-6) / 1e9 / HBM_PEAK_GBS}
    # the forward once more, so `out` holds a real result again
    step(0)
    torch.cuda.synchronize()

    layer_bytes = (U + (1 if shared else 0)) * EXPERT_BYTES + T * (D * 4 + E * 4 + D * 2)
    if dn_q8:
        layer_bytes += U * (Q8_MAT_BYTES - MAT_BYTES)
    if sh_q8:
        layer_bytes += 3 * (Q8_MAT_BYTES - MAT_BYTES)
    res = {
        "metric": "MoE layer tokens/s (W4A8, 1 GPU)",
        "value": T / (ms * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": ms,
        "us_per_layer": ms * 1e3,
        "us_per_layer_eager": ms_eager * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8e4m3 x mxfp4 (fp32 accumulate, bf16 out)",
        "data": (f"synthetic (seeded MXFP4 gate/up, {args.down_type} down, {args.shared_type if shared else 'no'} "
                 "shared expert, blocks uploaded from the host; N(0,1) x and logits)"
                 if host_up else "synthetic (seeded MXFP4 weights filled on device, N(0,1) x and logits)"),
        "config": {"workload": args.config + ("_q5k_down" if dn_q8 else "") + ("_q8_0_shared" if sh_q8 else ""),
                   "tokens": T, "d_model": D, "n_expert": E, "down_type": args.down_type,
                   "shared_type": args.shared_type if shared else None,
                   "top_k": K, "d_ff": FF, "shared_expert": shared,
                   "weight_layers_rotated": args.layers,
                   "launch": (f"HIP graph of {graph_layers} layer forwards, replayed"
                              if graph_layers else "eager stream launches")},
        "layer_hbm_fraction": layer_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
        "distinct_experts": U,
        "stage_us": st_us,
        "roofline": roof,
        "grouped_gemms": gemm,
    }
    if not args.no_cpu and not host_up:
        res["cpu_baseline"] = cpu_baseline(args.config, T, args.cpu_seconds, shared)
    print(json.dumps(res))


if __name__ == "__main__":
    main()
