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

# the configurations measured beside the headline one, in the same run
SWEEP = ["decode1", "decode2", "decode4", "decode8", "decode16", "decode32", "ragged64", "prefill4096", "mixed"]

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
    ap.add_argument("--tokens", type=int, default=None,
                    help="override the configuration's token count (path threshold measurements)")
    ap.add_argument("--graph", type=int, default=1,
                    help="1: time the K steps as one HIP graph (how a model's layer loop runs "
                         "when captured); 0: eager launches only")
    ap.add_argument("--replays", type=int, default=5, help="timed replays of the K-step graph (median)")
    ap.add_argument("--no-sweep", action="store_true",
                    help="skip the other configurations (configs sub-object)")
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


def kernel_bytes(stage, T, U, shared, dn_q8=False, sh_q8=False):
    """(algorithmic, overhead) HBM bytes of one launch of a stage.  U =
    distinct routed experts hit; P = routed (token, slot) rows, plus T
    shared rows.  Algorithmic bytes are what the layer must move: the hit
    experts' weights and the stage's activation input (e4m3 x + E8M0 scales
    into gate/up, the quantised h rows into the down).  Overhead bytes are
    this build's own intermediates: h written by gate/up and the staged
    weighted down rows (f16 + an exponent byte per 16 columns) the combine
    reads back.  A q8_0-split matrix is int8 + f16 per 32; int8 activations
    carry an fp32 scale per 32 (h rows of a q8_0-split down; x of a
    q8_0-split shared expert, read besides the e4m3 x)."""
    P = T * K + (T if shared else 0)
    sh_mat = Q8_MAT_BYTES if sh_q8 else MAT_BYTES
    xq = T * D + T * D // 32 + (T * D + T * D // 8 if sh_q8 else 0)
    hq = T * K * FF + T * K * FF // 32 * (4 if dn_q8 else 1)
    if shared:
        hq += T * FF + T * FF // 32 * (4 if sh_q8 else 1)
    staged = P * (D * 2 + D // 16)
    if stage == "gateup":
        return U * 2 * MAT_BYTES + (2 * sh_mat if shared else 0) + xq, hq
    if stage == "down":
        dn = U * (Q8_MAT_BYTES if dn_q8 else MAT_BYTES) + (sh_mat if shared else 0)
        return dn + hq, staged
    if stage == "expert":
        # one kernel per skinny tile: h stays in LDS (the tap copy is written)
        return U * 3 * MAT_BYTES + (3 * sh_mat if shared else 0) + xq, hq + staged
    raise ValueError(stage)


def kernels_of(path):
    """The grouped-GEMM kernels of a path: one per skinny tile on the
    one-kernel skinny path (3), else gate/up and down."""
    return ("expert",) if path == 3 else ("gateup", "down")


def kernel_us(st_us, kernel):
    """Replay-timed duration of a kernel: the fused skinny kernel is the
    gateup stage's launch."""
    return st_us["gateup"] if kernel == "expert" else st_us[kernel]


def kernel_flops(stage, T, shared):
    P = T * K + (T if shared else 0)
    return P * {"gateup": 2 * D * 2 * FF, "down": 2 * FF * D, "expert": 3 * 2 * FF * D}[stage]


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


def flush_mall(buf):
    """Evict the 256 MB memory-side cache: one copy over 2 x 512 MiB."""
    buf[1].copy_(buf[0])


def algorithmic(T, U, shared, dn_q8=False, sh_q8=False):
    """Algorithmic HBM bytes and MFMA FLOPs of one layer forward: the weights
    of the U routed experts hit (+ the shared expert), f32 x, f32 logits and
    bf16 out per token."""
    by = (U + (1 if shared else 0)) * EXPERT_BYTES + T * (D * 4 + E * 4 + D * 2)
    if dn_q8:
        by += U * (Q8_MAT_BYTES - MAT_BYTES)
    if sh_q8:
        by += 3 * (Q8_MAT_BYTES - MAT_BYTES)
    fl = kernel_flops("gateup", T, shared) + kernel_flops("down", T, shared)
    return by, fl


class Bench:
    """One configuration on a shared set of weight layers and one context."""

    def __init__(self, args, layers, layer, stream, flush):
        self.args, self.layers, self.layer, self.stream, self.flush = args, layers, layer, stream, flush

    def setup(self, cfg_name, seed):
        import torch
        cfg = CONFIGS[cfg_name]
        self.name, self.T, self.shared = cfg_name, cfg["T"], cfg["shared"]
        n_in = self.args.inputs if self.T < 1024 else min(self.args.inputs, 4)
        self.xs, self.ls, self.ss = make_inputs(cfg_name, self.T, n_in, seed, torch.device("cuda:0"))
        self.out = torch.empty((self.T, D), dtype=torch.bfloat16, device="cuda:0")

    def step(self, i):
        j = i % len(self.xs)
        self.layer.forward(self.layers[i % len(self.layers)], self.xs[j], self.ls[j],
                           self.ss[j] if self.shared else None, out=self.out)

    def graph(self, first, count):
        """A HIP graph of `count` consecutive forwards from step `first`."""
        import torch
        cap = torch.cuda.Stream()
        self.layer.set_stream(cap)
        with torch.cuda.stream(cap):
            self.step(first)          # allocator / first-launch work outside the capture
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=cap):
            for i in range(count):
                self.step(first + i)
        torch.cuda.synchronize()
        self.layer.set_stream(self.stream)
        return g

    def time_replays(self, g, n):
        """Milliseconds of each of n replays of g, the memory-side cache
        flushed before each (untimed)."""
        import torch
        out = []
        for _ in range(n):
            flush_mall(self.flush)
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(self.stream)
            g.replay()
            e1.record(self.stream)
            torch.cuda.synchronize()
            out.append(e0.elapsed_time(e1))
        return out

    def stage_times(self, budget_us=2e5):
        """Average duration of each stage's kernels: the stage of the last
        forward launched again back to back over the rotating weight sets,
        bracketed by two HIP events on the layer's stream."""
        import torch
        from q36_amd import moe
        self.step(0)
        torch.cuda.synchronize()
        U = int(np.unique(self.layer.tap(moe.TAP_TOPK_IDX).cpu().numpy()).size)
        path = self.layer.last_path
        st_us = {}
        for st in moe.MoELayer.STAGES:
            for i in range(5):
                self.layer.replay(self.layers[i % len(self.layers)], st)
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(self.stream)
            reps = 0
            t0 = time.perf_counter()
            while True:
                for i in range(20):
                    self.layer.replay(self.layers[(reps + i) % len(self.layers)], st)
                reps += 20
                if reps >= 2000 or (time.perf_counter() - t0) * 1e6 > budget_us:
                    break
            e1.record(self.stream)
            torch.cuda.synchronize()
            st_us[st] = 1e3 * e0.elapsed_time(e1) / reps
        # stages without kernels on a path time as the empty-launch floor
        if path == 1:
            for st in ("route", "scan", "combine"):
                st_us[st] = 0.0
        if path == 3:             # gate/up and down in one kernel (the gateup stage)
            st_us["down"] = 0.0
        self.step(0)              # `out` holds a real result again
        torch.cuda.synchronize()
        return U, path, st_us

    def summary(self, ms_layer, U, path, st_us, dn_q8=False, sh_q8=False):
        T, shared = self.T, self.shared
        by, fl = algorithmic(T, U, shared, dn_q8, sh_q8)
        r = {"tokens": T, "us_per_layer": ms_layer * 1e3, "tokens_per_s": T / (ms_layer * 1e-3),
             "distinct_experts": U,
             "path": {0: "sorted_fat", 1: "direct", 2: "sorted_skinny", 3: "sorted_fused"}.get(path, path),
             "layer_bytes": by, "layer_hbm_frac": by / (ms_layer * 1e-3) / 1e9 / HBM_PEAK_GBS,
             "layer_flops": fl, "layer_mfma_frac": fl / (ms_layer * 1e-3) / 1e12 / MFMA_FP8_PEAK_TFS,
             "stage_us": st_us}
        for st in kernels_of(path):
            us = kernel_us(st_us, st)
            kf = kernel_flops(st, T, shared)
            kb, ko = kernel_bytes(st, T, U, shared, dn_q8, sh_q8)
            r[st] = {"us": us, "mfma_frac": kf / (us * 1e-6) / 1e12 / MFMA_FP8_PEAK_TFS,
                     "hbm_frac": kb / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, "flops": kf, "bytes": kb,
                     "overhead_bytes": ko,
                     "hbm_frac_with_overhead": (kb + ko) / (us * 1e-6) / 1e9 / HBM_PEAK_GBS}
        return r


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU; --gpus must be 1 "
                                   "(expert-parallel sharding over several GPUs is designed, not run)"}))
        sys.exit(2)
    import torch
    from q36_amd import moe

    if args.copy_mib:
        copy_reference(args.copy_mib)
        return

    if args.tokens is not None:
        if args.tokens < 1:
            print(json.dumps({"error": "--tokens must be >= 1"}))
            sys.exit(2)
        CONFIGS[args.config] = dict(CONFIGS[args.config], T=args.tokens)
    cfg = CONFIGS[args.config]
    T, shared = cfg["T"], cfg["shared"]
    steps = args.steps if args.steps is not None else cfg["steps"]
    warmup = args.warmup if args.warmup is not None else cfg["warmup"]
    if steps < 1 or warmup < 0:
        print(json.dumps({"error": "--steps must be >= 1 and --warmup >= 0"}))
        sys.exit(2)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream()

    dn_q8 = args.down_type == "q5_k"
    sh_q8 = shared and args.shared_type == "q8_0"
    host_up = dn_q8 or sh_q8
    if args.layers is None:
        args.layers = 16 if host_up else 40
    sweep = [] if (args.no_sweep or host_up) else [c for c in SWEEP if c != args.config]
    with_shared = shared or any(CONFIGS[c]["shared"] for c in sweep)
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
            w = moe.MoEWeights.alloc(E, D, FF, FF if with_shared else 0)
            w.fill_synthetic(args.seed * 1000 + l)
        layers.append(w)
    max_T = max([T] + [CONFIGS[c]["T"] for c in sweep])
    layer = moe.MoELayer(max_T, stream=stream)
    layer.set_path(args.path)
    flush = torch.empty((2, 512 << 20), dtype=torch.uint8, device=dev)
    B = Bench(args, layers, layer, stream, flush)
    B.setup(args.config, args.seed)
    torch.cuda.synchronize()

    # the contract: W untimed warmup steps, then exactly K timed steps
    for i in range(warmup):
        B.step(i)
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record(stream)
    for i in range(steps):
        B.step(warmup + i)
    ev1.record(stream)
    torch.cuda.synchronize()
    ms_eager = ev0.elapsed_time(ev1) / steps
    ms, timed = ms_eager, "eager stream launches"
    replay_ms = []
    if args.graph:
        # the same K steps (layers and inputs rotating as above) captured as
        # one HIP graph -- how a model's captured layer loop issues them --
        # replayed with the memory-side cache flushed first; the first replay
        # is untimed, the median of the timed ones is the figure
        g = B.graph(warmup, steps)
        B.time_replays(g, 1)
        replay_ms = B.time_replays(g, args.replays)
        ms = float(np.median(replay_ms)) / steps
        timed = (f"HIP graph of the {steps} timed layer forwards; median of {args.replays} replays, "
                 "memory-side cache flushed before each")
        del g

    U, path, st_us = B.stage_times()
    head = B.summary(ms, U, path, st_us, dn_q8, sh_q8)
    dom = max(kernels_of(path), key=lambda k: kernel_us(st_us, k))
    prefill = T >= 256
    if prefill:
        fl = kernel_flops(dom, T, shared)
        ach = fl / (kernel_us(st_us, dom) * 1e-6) / 1e12
        roof = {"bound": "mfma", "achieved": ach, "peak": MFMA_FP8_PEAK_TFS, "unit": "TFLOP/s",
                "frac": ach / MFMA_FP8_PEAK_TFS, "traffic": None, "kernel": dom,
                "kernel_us": kernel_us(st_us, dom), "flops_per_launch": fl,
                "layer_mfma_frac": head["layer_mfma_frac"], "layer_hbm_frac": head["layer_hbm_frac"]}
    else:
        by, ovh = kernel_bytes(dom, T, U, shared, dn_q8, sh_q8)
        ach = by / (kernel_us(st_us, dom) * 1e-6) / 1e9
        roof = {"bound": "hbm", "achieved": ach, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": ach / HBM_PEAK_GBS, "traffic": None, "kernel": dom,
                "kernel_us": kernel_us(st_us, dom), "bytes_per_launch": by, "overhead_bytes_per_launch": ovh,
                "layer_hbm_frac": head["layer_hbm_frac"], "layer_bytes": head["layer_bytes"]}
    roof["traffic"] = None if host_up else measured_traffic(args.config, dom)
    if roof["traffic"] is not None:
        roof["traffic_source"] = ("rocprofv3 FETCH_SIZE + WRITE_SIZE of this kernel and configuration, "
                                  "scaled by a plain copy's reading (profiles/hbm_traffic.md)")

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
        "replay_ms": replay_ms,
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
                   "weight_layers_rotated": args.layers, "launch": timed},
        "layer_hbm_fraction": head["layer_hbm_frac"],
        "distinct_experts": U,
        "stage_us": st_us,
        "roofline": roof,
        "grouped_gemms": {st: head[st] for st in kernels_of(path)},
    }
    # the other BASELINE configurations, measured in the same run on the same
    # weight layers: a HIP graph of one forward per layer, median of replays
    cfgs = {}
    for c in sweep:
        B.setup(c, args.seed + 17)
        for i in range(3):
            B.step(i)
        # as many forwards per graph as the configuration's own run (at most
        # 1000): a replay's launch and cache-flush overhead spread over only
        # 40 forwards added ~4 us per layer at decode32
        n_c = max(args.layers, min(CONFIGS[c]["steps"], 1000))
        g = B.graph(0, n_c)
        B.time_replays(g, 1)
        rms = B.time_replays(g, 3)
        del g
        U_c, path_c, st_c = B.stage_times(budget_us=5e4)
        cfgs[c] = B.summary(float(np.median(rms)) / n_c, U_c, path_c, st_c)
    if cfgs:
        res["configs"] = cfgs
    if not args.no_cpu and not host_up:
        res["cpu_baseline"] = cpu_baseline(args.config, T, args.cpu_seconds, shared)
    print(json.dumps(res))


def copy_reference(mib):
    """A plain copy of known size: the reference point that scales the
    FETCH_SIZE / WRITE_SIZE counters of the layer kernels, and the
    achievable-bandwidth reference points (copy, read-only f32 sum)."""
    import torch
    n = mib << 20
    src = torch.ones(n, dtype=torch.uint8, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(4):
        dst.copy_(src)
    torch.cuda.synchronize()
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


if __name__ == "__main__":
    main()
