#!/usr/bin/env python3
"""Benchmark of the MI355X selective scan: config 2 forward + backward on one GPU.

Step = one forward (mss_fwd) and one backward (mss_bwd_scan + mss_bwd_reduce) pass of the
fused scan over the config-2 batch (fp32, B=4, D=1536, L=2048, N=16; softplus(delta +
bias), D skip, silu(z) gate, last state), inputs resident in HBM, seeded synthetic data.
Timing: HIP events recorded on the stream the kernels run on (torch's current stream,
which the C ABI launches on), W untimed warmup steps, then exactly K timed steps
bracketed by device synchronisation, for each way of launching the step's three kernels
(eager launches; replays of one captured HIP graph) in three trials that alternate which
goes first; the faster way's median trial is the step time (`launch` names it, both rates
are reported); per-kernel means come from a separate eager run with events between the
launches, taken before the timed trials. Prints ONE JSON line on stdout; progress to stderr.

Fields beyond the driver contract:
  roofline      dominant kernel: algorithmic bytes / its average event-timed duration
                vs the 8 TB/s HBM peak; `traffic` = measured HBM bytes per launch from
                the rocprofv3 FETCH_SIZE / WRITE_SIZE summary under profiles/ (or null)
  cpu_baseline  torch-CPU restatement of the reference's pure-JAX scan path
                (oracle/assoc_torch.py) timed on this host on a channel slice
  fwd_bwd_hbm_frac  (fwd + bwd algorithmic bytes) / step time / 8 TB/s
  configs       per config (c2 and, by default, c3 bf16 and c4 variable-length): ms fwd/bwd,
                tokens/s, algorithmic MB and HBM fractions, and a CPU baseline of its own
  train_c5      the metric's second half: tokens/s of one training step of the Mamba-1
                130M-shape LM (config 5) through the HIP scan
  decode_c5     single-token decode of the same model after a 2048-token prefill
  complex_c2    the complex-A scan (mss_cfwd + mss_cbwd) at the config-2 shape with the
                reference's complex A initialisation, and a CPU baseline of the reference's
                complex path (torch restatement of mamba/mamba1.py:143-176)
  reference_api_c2  the reference-signature entry points (mss_scan_fwd + mss_scan_bwd_ws,
                the backward from the forward's chunk_states) at the config-2 shape, and
                mss_scan_fwd_repeat at the reference README's own shapes beside its numbers
Inputs are drawn on the GPU from each config's recipe (seeded torch generator).
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "jax-mambas_amd"))

METRIC = "selective_scan fwd+bwd ms & % HBM roofline; Mamba-1 130M train tokens/s"
HBM_PEAK_GBS = 8000.0


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def cpu_model():
    """The host CPU for the CPU baselines: /proc/cpuinfo's model name (a VM may show only
    the vendor's family name), its family/model/stepping numbers and the logical CPUs."""
    fields = {}
    n_cpus = 0
    try:
        for line in open("/proc/cpuinfo"):
            key, _, val = line.partition(":")
            key = key.strip()
            if key == "processor":
                n_cpus += 1
            elif key in ("model name", "cpu family", "model", "stepping") and key not in fields:
                fields[key] = val.strip()
    except OSError:
        return None
    if "model name" not in fields:
        return None
    ids = ", ".join(f"{k} {fields[k]}" for k in ("cpu family", "model", "stepping") if k in fields)
    return f"{fields['model name']} ({ids}; {n_cpus} logical CPUs on the host)"


def read_traffic(kernel_tag):
    """HBM bytes per launch from profiles/<kernel_tag>_traffic.txt (key=value lines)."""
    path = os.path.join(ROOT, "profiles", f"{kernel_tag}_traffic.txt")
    if not os.path.exists(path):
        return None
    kv = {}
    for line in open(path):
        m = re.match(r"\s*([a-z_]+)\s*=\s*([0-9.eE+-]+)\s*$", line)
        if m:
            kv[m.group(1)] = float(m.group(2))
    if "hbm_bytes_per_launch" in kv:
        return kv["hbm_bytes_per_launch"]
    return None


def gpu_inputs(torch, cfg, seed=0):
    """The config's input recipe (configs.py) drawn on the GPU with a seeded torch
    generator: u, delta_raw, z, dout, B, C ~ N(0, 1) in the config's activation dtype;
    delta_bias = inverse softplus of U[1e-3, 1e-1]; A = -(n + 1); D = 1. Variable-length
    configs take lengths from np.random.default_rng(seed).integers(lo, hi + 1, B)."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    b, d, l, n = cfg.batch, cfg.dim, cfg.length, cfg.dstate
    act = torch.bfloat16 if cfg.dtype == "bf16" else torch.float32
    t = {}
    for k, shape in (("u", (b, d, l)), ("delta", (b, d, l)), ("z", (b, d, l)), ("dout", (b, d, l)),
                     ("B", (b, n, l)), ("C", (b, n, l))):
        t[k] = torch.randn(shape, generator=g, device="cuda").to(act)
    dt = torch.rand(d, generator=g, device="cuda") * (1e-1 - 1e-3) + 1e-3
    t["delta_bias"] = dt + torch.log(-torch.expm1(-dt))
    t["A"] = -(torch.arange(n, device="cuda", dtype=torch.float32) + 1).repeat(d, 1)
    t["D"] = torch.ones(d, device="cuda")
    lens = None
    if cfg.varlen is not None:
        lo, hi = cfg.varlen
        lens = np.random.default_rng(seed).integers(lo, hi + 1, size=b).astype(np.int32)
        t["seq_lens"] = torch.from_numpy(lens).cuda()
    return t, lens


def gpu_step_setup(torch, cfg):
    from mamba_amd import _lib

    lib = _lib.register_hip_kernel()
    t, lens = gpu_inputs(torch, cfg)
    dev = "cuda"
    b, d, l, n = cfg.batch, cfg.dim, cfg.length, cfg.dstate
    io = _lib.MSS_BF16 if cfg.dtype == "bf16" else _lib.MSS_F32
    n_seg = (l + _lib.MSS_SEG_STEPS - 1) // _lib.MSS_SEG_STEPS
    t["out"] = torch.empty_like(t["u"])
    t["last"] = torch.empty(b, d, n, device=dev)
    t["carries"] = torch.empty(b, d, n, n_seg, device=dev)
    t["y_pre"] = torch.empty_like(t["u"])
    t["dlast"] = torch.zeros(b, d, n, device=dev)
    for k in ("u", "delta", "z", "A", "B", "C", "D", "delta_bias"):
        t["d" + k] = torch.empty_like(t[k])
    P = lambda k: t[k].data_ptr() if k in t else None
    common = dict(batch=b, dim=d, seqlen=l, dstate=n, discretization=_lib.MSS_EULER, delta_softplus=1,
                  io_dtype=io, bc_dtype=io, u=P("u"), delta=P("delta"), A=P("A"), B=P("B"), C=P("C"),
                  D=P("D"), z=P("z"), delta_bias=P("delta_bias"), seq_lens=P("seq_lens"))
    fa = _lib.FwdArgs(**common, out=P("out"), last_state=P("last"), carries=P("carries"), y_pre=P("y_pre"))
    ba = _lib.BwdArgs(**common, carries=P("carries"), y_pre=P("y_pre"), out=P("out"), dout=P("dout"),
                      dlast_state=P("dlast"),
                      du=P("du"), ddelta=P("ddelta"), dA=P("dA"), dB=P("dB"), dC=P("dC"), dD=P("dD"), dz=P("dz"),
                      ddelta_bias=P("ddelta_bias"))
    ws_bytes = int(lib.mss_bwd_workspace_bytes(ba))
    t["ws"] = torch.empty(ws_bytes, device=dev, dtype=torch.uint8)
    ba.workspace = t["ws"].data_ptr()
    ba.workspace_bytes = ws_bytes
    return lib, t, fa, ba, lens


DEVICE_WARMUP_S = 0.2


def warm_up_device(torch):
    """Back-to-back bf16 GEMMs for about DEVICE_WARMUP_S seconds, right before a timed leg's
    warmup steps (its inputs already set up): a GPU that idled, even for the few tens of ms a
    leg's host-side setup takes, runs its next tens of milliseconds of work slower (kernel
    trace of a bench run: every config's scan kernels start 8-15 % slow and settle after about
    60 ms of work), which a short warmup of the measured step alone does not cover. The leg's
    own warmup and timed steps are unchanged."""
    if DEVICE_WARMUP_S <= 0:
        return
    a = torch.randn(2048, 2048, device="cuda", dtype=torch.bfloat16)
    b = torch.randn(2048, 2048, device="cuda", dtype=torch.bfloat16)
    t0 = None  # timed from the end of the first batch: the library's one-time setup is host work
    while t0 is None or time.perf_counter() - t0 < DEVICE_WARMUP_S:
        for _ in range(40):
            a = torch.mm(a, b).mul_(1.0 / 45)
        torch.cuda.synchronize()
        t0 = time.perf_counter() if t0 is None else t0
    del a, b


def run_gpu(torch, cfg, steps, warmup, graph=True):
    """Times `steps` fwd+bwd steps of the scan at `cfg`. The step rate comes from timed
    regions holding only the steps: eager launches and (when `graph`) replays of one
    captured HIP graph of the step's three launches, three trials each in alternating order;
    the faster way's median trial is `ms`. Per-kernel means come from a second, eager run
    with events between the launches (ms)."""
    from mamba_amd import _lib

    lib, t, fa, ba, lens = gpu_step_setup(torch, cfg)

    def step(sp, stream=None, evs=None):
        if evs:
            evs[0].record(stream)
        _lib.check(lib.mss_fwd(fa, sp), "mss_fwd")
        if evs:
            evs[1].record(stream)
        _lib.check(lib.mss_bwd_scan(ba, sp), "mss_bwd_scan")
        if evs:
            evs[2].record(stream)
        _lib.check(lib.mss_bwd_reduce(ba, sp), "mss_bwd_reduce")
        if evs:
            evs[3].record(stream)

    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream
    g = None
    if graph:  # captured before the warm-up: no host work between it and the timed steps
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            step(torch.cuda.current_stream().cuda_stream)
        g.replay()  # the first replay uploads the graph
        torch.cuda.synchronize()
    warm_up_device(torch)
    for _ in range(warmup):
        step(sp)
    torch.cuda.synchronize()
    log(f"[bench] {cfg.name}: warmup done ({warmup} steps)")

    def timed(fn):
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record(stream)
        for _ in range(steps):
            fn()
        end.record(stream)
        torch.cuda.synchronize()
        return start.elapsed_time(end) / steps

    # Per-kernel means first, from eager steps with events between the launches: after graph
    # replays the next eager steps on the stream run slow for a while (a c2 forward measured
    # 0.115-0.122 ms instead of 0.101), which would skew them.
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(steps)]
    for i in range(steps):
        step(sp, stream, evs[i])
    torch.cuda.synchronize()
    fwd = float(np.mean([e[0].elapsed_time(e[1]) for e in evs]))
    bws = float(np.mean([e[1].elapsed_time(e[2]) for e in evs]))
    red = float(np.mean([e[2].elapsed_time(e[3]) for e in evs]))

    trials = {"eager": []}
    modes = [("eager", lambda: step(sp))]
    if graph:
        trials["graph"] = []
        modes.append(("graph", g.replay))
    for i in range(3):
        for name, fn in (modes if i % 2 == 0 else modes[::-1]):
            trials[name].append(timed(fn))
    eager_ms = float(np.median(trials["eager"]))
    graph_ms = float(np.median(trials["graph"])) if graph else None
    use_graph = graph_ms is not None and graph_ms < eager_ms
    ms = graph_ms if use_graph else eager_ms
    if graph:
        del g
    log(f"[bench] {cfg.name}: timed {steps} steps x 3 trials per launch mode: {ms:.4f} ms/step "
        f"({'hip graph' if use_graph else 'eager'}; eager {eager_ms:.4f}, graph {graph_ms}); kernels fwd {fwd:.4f}, "
        f"bwd_scan {bws:.4f}, bwd_reduce {red:.4f} ms")
    del t
    torch.cuda.empty_cache()
    return dict(ms=ms, eager_ms=eager_ms, graph_ms=graph_ms, graph=use_graph, fwd=fwd, bwd_scan=bws, bwd_reduce=red,
                lens=lens)


def _ref_inputs(torch, b, d, l, n, seed):
    """The reference benchmark's recipe (benchmarks/benchmark_selective_scan.py:83-92) in the
    kernel boundary's physical layout: A = -exp(N(0,1)) (D, N); deltas = softplus(N(0,1)),
    u ~ N(0,1) as [B][D][L]; B, C ~ N(0,1) as [B][N][L]; initial_x ~ N(0,1) (B, D, N)."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    r = lambda *shape: torch.randn(*shape, generator=g, device="cuda")
    return dict(A=-torch.exp(r(d, n)), deltas=torch.nn.functional.softplus(r(b, d, l)), B=r(b, n, l),
                C=r(b, n, l), u=r(b, d, l), x0=r(b, d, n))


def run_reference_api(torch, steps, warmup):
    """The reference-signature entry points (the XLA-FFI handlers' counterparts, float32,
    Euler, no fused extras): mss_scan_fwd + mss_scan_bwd_ws at the config-2 shape (the
    backward starts from the forward's 2048-step chunk_states, as the reference's does), and
    mss_scan_fwd_repeat with 100 launches per call at the reference README's own shapes
    (B=1, D=256, N=16, L in {512, 2048, 8192}; mamba/README.md:75-83), per launch."""
    from mamba_amd import _lib
    from mamba_amd.configs import C2

    lib = _lib.register_hip_kernel()
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream
    P = lambda t: t.data_ptr()

    def timed(fn, n):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record(stream)
        for _ in range(n):
            fn()
        end.record(stream)
        torch.cuda.synchronize()
        return start.elapsed_time(end) / n

    b, d, l, n = C2.batch, C2.dim, C2.length, C2.dstate
    x = _ref_inputs(torch, b, d, l, n, 0)
    y = torch.empty(b, d, l, device="cuda")
    fin = torch.empty(b, d, n, device="cuda")
    cs = torch.empty(b, d, -(-l // 2048), n, 2, device="cuda")
    dy = torch.randn(b, d, l, device="cuda")
    dfin = torch.zeros(b, d, n, device="cuda")
    grads = [torch.empty_like(x[k]) for k in ("A", "deltas", "B", "C", "u", "x0")]
    ws_bytes = int(lib.mss_scan_bwd_workspace_bytes(b, l, d, n))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
    fwd_args = (sp, 0, b, l, d, n, P(x["A"]), P(x["deltas"]), P(x["B"]), P(x["C"]), P(x["u"]), P(x["x0"]),
                P(y), P(fin), P(cs))
    bwd_args = (sp, b, l, d, n, P(x["A"]), P(x["deltas"]), P(x["B"]), P(x["C"]), P(x["u"]), P(x["x0"]), P(cs),
                P(dy), P(dfin), *[P(t) for t in grads], P(ws), ws_bytes)
    fwd = lambda: _lib.check(lib.mss_scan_fwd(*fwd_args), "mss_scan_fwd")
    bwd = lambda: _lib.check(lib.mss_scan_bwd_ws(*bwd_args), "mss_scan_bwd_ws")
    warm_up_device(torch)
    for _ in range(warmup):
        fwd()
        bwd()
    ms_fwd = timed(fwd, steps)
    ms_bwd = timed(bwd, steps)
    ms_step = timed(lambda: (fwd(), bwd()), steps)
    log(f"[bench] reference API c2: fwd {ms_fwd:.4f} ms, bwd {ms_bwd:.4f} ms, step {ms_step:.4f} ms")
    out = {"workload": "mss_scan_fwd + mss_scan_bwd_ws (reference signature, fp32, Euler, no fused extras), "
                       "B=4 D=1536 L=2048 N=16, reference input recipe",
           "ms_fwd": round(ms_fwd, 5), "ms_bwd": round(ms_bwd, 5), "ms_fwd_bwd": round(ms_step, 5),
           "tokens_per_s": round(b * l / (ms_step * 1e-3), 1)}
    del x, y, fin, cs, dy, dfin, grads, ws
    published = {512: 0.0282, 2048: 0.0560, 8192: 0.1584}  # A100, mamba/README.md:75-83
    rows = []
    for length in (512, 2048, 8192):
        b, d, n, launches = 1, 256, 16, 100
        x = _ref_inputs(torch, b, d, length, n, 1)
        y = torch.empty(b, d, length, device="cuda")
        fin = torch.empty(b, d, n, device="cuda")
        cs = torch.empty(b, d, -(-length // 2048), n, 2, device="cuda")
        args = (sp, 0, launches, b, length, d, n, P(x["A"]), P(x["deltas"]), P(x["B"]), P(x["C"]), P(x["u"]),
                P(x["x0"]), P(y), P(fin), P(cs))
        call = lambda: _lib.check(lib.mss_scan_fwd_repeat(*args), "mss_scan_fwd_repeat")
        call()
        trials = sorted(timed(call, 1) / launches for _ in range(5))
        rows.append({"length": length, "ms_per_launch_median": round(trials[2], 5),
                     "reference_a100_ms": published[length]})
        log(f"[bench] reference shapes L={length}: {trials[2] * 1e3:.1f} us per launch "
            f"(reference on A100: {published[length] * 1e3:.1f} us)")
    out["reference_shapes_fwd"] = {
        "workload": "mss_scan_fwd_repeat, 100 launches per call, B=1 D=256 N=16, fp32, median of 5 calls",
        "rows": rows,
        "note": "reference_a100_ms: the reference's own forward kernel on an A100-SXM4-40GB "
                "(mamba/README.md:75-83), other hardware, context only"}
    return out


# What the backward's algorithmic bytes are divided over in `roofline`.
BWD_BYTES_OVER = ("bwd_kernel alone: every tensor the backward reads or writes once, including the dB/dC "
                  "(and dA/dD/dbias) outputs that reduce_kernel writes from the scan's partial sums")


def as_launched(bwd_bytes, scan_ms, reduce_ms):
    """The backward as launched (scan kernel + reduction kernel) against the HBM roofline."""
    ms = scan_ms + reduce_ms
    achieved = bwd_bytes / (ms * 1e-3) / 1e9
    return {"kernels": ["bwd_kernel", "reduce_kernel"], "ms": round(ms, 5), "achieved": round(achieved, 1),
            "frac": round(achieved / HBM_PEAK_GBS, 4)}


def scan_report(cfg, r):
    """ms, tokens/s and fractions of the 8 TB/s HBM roofline for one config's timings."""
    from mamba_amd.configs import algorithmic_bytes

    lens = r["lens"]
    fwd_b, bwd_b = algorithmic_bytes(cfg, lens)
    tokens = int(np.sum(lens)) if lens is not None else cfg.batch * cfg.length
    frac = lambda nbytes, ms: round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
    rep = {
        "workload": cfg.description, "dtype": cfg.dtype,
        "ms_fwd": round(r["fwd"], 5), "ms_bwd": round(r["bwd_scan"] + r["bwd_reduce"], 5),
        "ms_fwd_bwd": round(r["ms"], 5), "tokens_per_s": round(tokens / (r["ms"] * 1e-3), 1),
        "launch": "hip graph" if r["graph"] else "eager", "ms_fwd_bwd_eager": round(r["eager_ms"], 5),
        "ms_fwd_bwd_graph": None if r.get("graph_ms") is None else round(r["graph_ms"], 5),
        "algorithmic_mb": {"fwd": round(fwd_b / 1e6, 1), "bwd": round(bwd_b / 1e6, 1)},
        "hbm_frac": {"fwd": frac(fwd_b, r["fwd"]), "bwd": frac(bwd_b, r["bwd_scan"] + r["bwd_reduce"]),
                     "fwd_bwd": frac(fwd_b + bwd_b, r["ms"])},
    }
    # The config's dominant kernel (the backward scan) against the HBM roofline, as the
    # headline line's `roofline`; `traffic` = measured HBM bytes per launch of that kernel and
    # workload (profiles/bwd_scan_<config>_traffic.txt), or null.
    kern = f"bwd_scan_{cfg.name}"
    achieved = bwd_b / (r["bwd_scan"] * 1e-3) / 1e9
    rep["roofline"] = {"bound": "hbm", "kernel": kern, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                       "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": read_traffic(kern),
                       "algorithmic_bytes": int(bwd_b), "avg_launch_ms": round(r["bwd_scan"], 5),
                       "bytes_over": BWD_BYTES_OVER,
                       "backward_as_launched": as_launched(bwd_b, r["bwd_scan"], r["bwd_reduce"]),
                       "fwd_traffic": read_traffic(f"fwd_{cfg.name}")}
    if lens is not None:
        rep["seq_lens"] = [int(x) for x in lens]
        rep["valid_fraction"] = round(float(np.sum(lens)) / (cfg.batch * cfg.length), 4)
    return rep


def complex_a(torch, d, n, device):
    """The reference's complex A: -exp(Re log(1/2 - i n)) + i Im log(1/2 - i n), n < N
    (mamba/mamba1.py:47, 162), the same row for every channel."""
    k = torch.arange(n, dtype=torch.float64)
    a_log = torch.log(torch.complex(torch.full_like(k, 0.5), -k))
    a = torch.complex(-torch.exp(a_log.real), a_log.imag).to(torch.complex64)
    return a.repeat(d, 1).to(device)


def run_complex_c2(torch, steps, warmup):
    """Complex-A scan fwd + bwd (mss_cfwd, mss_cbwd) on the config-2 inputs and shape."""
    from mamba_amd import _lib
    from mamba_amd.configs import C2, algorithmic_bytes

    cfg = C2
    lib, t, fa, ba, _ = gpu_step_setup(torch, cfg)
    b, d, l, n = cfg.batch, cfg.dim, cfg.length, cfg.dstate
    n_seg = (l + _lib.MSS_SEG_STEPS - 1) // _lib.MSS_SEG_STEPS
    rv = lambda x: torch.view_as_real(x).data_ptr()
    t["cA"] = complex_a(torch, d, n, "cuda")
    t["cdA"] = torch.empty_like(t["cA"])
    t["clast"] = torch.empty(b, d, n, dtype=torch.complex64, device="cuda")
    t["cdlast"] = torch.zeros(b, d, n, dtype=torch.complex64, device="cuda")
    t["ccarries"] = torch.empty(b, d, n, n_seg, dtype=torch.complex64, device="cuda")
    fa.A, fa.last_state, fa.carries = rv(t["cA"]), rv(t["clast"]), rv(t["ccarries"])
    ba.A, ba.carries, ba.dlast_state, ba.dA = rv(t["cA"]), rv(t["ccarries"]), rv(t["cdlast"]), rv(t["cdA"])
    ws_bytes = int(lib.mss_cbwd_workspace_bytes(ba))
    t["cws"] = torch.empty(ws_bytes, device="cuda", dtype=torch.uint8)
    ba.workspace, ba.workspace_bytes = t["cws"].data_ptr(), ws_bytes
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream

    def step(evs=None):
        if evs:
            evs[0].record(stream)
        _lib.check(lib.mss_cfwd(fa, sp), "mss_cfwd")
        if evs:
            evs[1].record(stream)
        _lib.check(lib.mss_cbwd(ba, sp), "mss_cbwd")
        if evs:
            evs[2].record(stream)

    warm_up_device(torch)
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
    for i in range(steps):
        step(evs[i])
    torch.cuda.synchronize()
    fwd = float(np.mean([e[0].elapsed_time(e[1]) for e in evs]))
    bwd = float(np.mean([e[1].elapsed_time(e[2]) for e in evs]))
    log(f"[bench] complex c2: fwd {fwd:.4f} ms, bwd {bwd:.4f} ms")
    # Algorithmic bytes of the real scan plus the complex parts of A, dA and the states.
    fwd_b, bwd_b = algorithmic_bytes(cfg)
    fwd_b += 4 * (d * n + b * d * n)
    bwd_b += 4 * (2 * d * n + b * d * n)
    tokens = b * l
    frac = lambda nbytes, ms: round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
    del t
    torch.cuda.empty_cache()
    return {"workload": "complex-A selective_scan fp32 B=4 D=1536 L=2048 N=16, reference complex A init, "
                        "softplus(delta+bias), D skip, silu(z) gate",
            "ms_fwd": round(fwd, 5), "ms_bwd": round(bwd, 5), "ms_fwd_bwd": round(fwd + bwd, 5),
            "tokens_per_s": round(tokens / ((fwd + bwd) * 1e-3), 1),
            "hbm_frac": {"fwd": frac(fwd_b, fwd), "bwd": frac(bwd_b, bwd)}}


def cpu_baseline_complex(torch, target_s, d0=8):
    """The reference's complex path on the CPU (oracle/mamba1_torch.complex_s6_scan:
    mamba/mamba1.py:143-176, associative scan over complex64 states) with the config-2
    fusions, forward + autograd backward, timed on a channel slice and scaled."""
    from mamba_amd.configs import C2, ScanConfig, make_scan_inputs
    from oracle.mamba1_torch import complex_s6_scan

    cfg = C2
    threads = max(1, min(len(os.sched_getaffinity(0)), 16))
    torch.set_num_threads(threads)

    def run(dslice):
        sub = ScanConfig("slice", cfg.batch, dslice, cfg.length, cfg.dstate, cfg.dtype)
        x = make_scan_inputs(sub, seed=0, with_z=True, with_dout=True)
        tr = lambda a: torch.from_numpy(np.ascontiguousarray(np.swapaxes(a, 1, 2))).requires_grad_(True)
        u, dr, z, Bs, Cs = (tr(x[k]) for k in ("u", "delta", "z", "B", "C"))
        dout = torch.from_numpy(np.ascontiguousarray(np.swapaxes(x["dout"], 1, 2)))
        A = complex_a(torch, dslice, cfg.dstate, "cpu").requires_grad_(True)
        bias = torch.from_numpy(x["delta_bias"]).requires_grad_(True)
        D = torch.from_numpy(x["D"]).requires_grad_(True)
        t0 = time.perf_counter()
        deltas = torch.nn.functional.softplus(dr + bias)
        y, _ = complex_s6_scan(A, deltas, Bs, Cs, u)
        out = (y.real + D * u) * torch.nn.functional.silu(z)
        (out * dout).sum().backward()
        return time.perf_counter() - t0

    run(d0)
    t_probe = run(d0)
    dslice = max(8, int(np.clip(d0 * (target_s / 4.0) / max(t_probe, 1e-3), d0, cfg.dim)) // 8 * 8)
    if dslice != d0:
        run(dslice)
    times = [run(dslice) for _ in range(3)]
    t_med = float(np.median(times))
    t_full = t_med * cfg.dim / dslice
    log(f"[bench] complex c2 cpu baseline: D={dslice} median {t_med:.2f} s")
    return {"value": cfg.batch * cfg.length / t_full, "unit": "tokens/s", "cores": threads,
            "cpu_model": cpu_model(), "kind": "port",
            "sample": (f"complex c2: B={cfg.batch} L={cfg.length} N={cfg.dstate} complex64 states, {dslice} of "
                       f"{cfg.dim} channels, fwd+bwd (autograd) median of 3 = {t_med:.3f} s, scaled "
                       f"x{cfg.dim / dslice:.1f} ({t_full:.2f} s per step)")}


C5_MODEL = dict(vocab=50280, d_model=768, n_layers=24, expand=2, d_state=16, dt_rank=48, d_conv=4)
C5_BATCH, C5_LENGTH = 8, 2048


def run_train_c5(torch, steps, warmup, graph=True):
    """Config 5: one training step of the Mamba-1 130M-shape LM (random init, uniform random
    tokens): bf16 activations with fp32 master weights and residual stream, forward,
    cross-entropy (fp32 math on bf16 logits, HIP kernel) over all next-token positions,
    backward (HIP scan, conv, norm and loss backward inside), AdamW step (mss_adamw, which also
    writes the bf16 copies of the GEMM weights the next forward reads). Timed with
    events on the current stream around exactly `steps` steps: first eagerly, then (graph)
    as one captured HIP graph replayed per step; `value` is the faster of the two (`launch`)."""
    from mamba_amd.lm_ops import cross_entropy
    from mamba_amd.mamba1 import GraphedTrainStep, MambaLM
    from mamba_amd.optim import AdamW

    torch.manual_seed(0)
    m = C5_MODEL
    model = MambaLM(m["vocab"], m["d_model"], m["n_layers"], m["expand"], m["d_state"], m["dt_rank"],
                    m["d_conv"], device="cuda")
    n_params = sum(p.numel() for p in model.parameters())
    opt = AdamW(model.parameters(), lr=1e-4, shadows=model.shadow_weights)
    gen = torch.Generator(device="cuda").manual_seed(0)
    tokens = torch.randint(0, m["vocab"], (C5_BATCH, C5_LENGTH + 1), device="cuda", generator=gen)
    inp = tokens[:, :-1].contiguous()
    tgt = tokens[:, 1:].reshape(-1).contiguous()

    def eager_step():
        opt.zero_grad(set_to_none=True)
        loss = cross_entropy(model(inp, act_dtype=torch.bfloat16), tgt)
        loss.backward()
        opt.step()
        return loss

    def timed(fn, n):
        stream = torch.cuda.current_stream()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record(stream)
        for _ in range(n):
            loss = fn()
        end.record(stream)
        torch.cuda.synchronize()
        return start.elapsed_time(end) / n, loss

    for _ in range(warmup):
        loss = eager_step()
    torch.cuda.synchronize()
    log(f"[bench] c5 warmup done ({warmup} steps, loss {loss.item():.4f}, {n_params / 1e6:.1f} M params)")
    eager_ms, loss = timed(eager_step, steps)
    log(f"[bench] c5 eager: timed {steps} steps: {eager_ms:.2f} ms/step, loss {loss.item():.4f}")
    # Drop the last eager autograd graph: its AccumulateGrad nodes are bound to the stream
    # they ran on, and capture needs them recreated on the capture stream.
    del loss
    torch.cuda.synchronize()
    graph_ms = None
    if graph:
        gs = GraphedTrainStep(model, opt, cross_entropy, inp, tgt, warmup=1)
        gs.step()
        graph_ms, loss = timed(gs.step, steps)
        log(f"[bench] c5 hip graph: timed {steps} steps: {graph_ms:.2f} ms/step, loss {loss.item():.4f}")
        del gs
    # The same step either way; the faster way of launching it is reported.
    use_graph = graph_ms is not None and graph_ms < eager_ms
    ms = graph_ms if use_graph else eager_ms
    del model, opt
    torch.cuda.empty_cache()
    return {
        "metric": "Mamba-1 130M train tokens/s",
        "value": round(C5_BATCH * C5_LENGTH / (ms * 1e-3), 1),
        "unit": "tokens/s",
        "ms_per_step": round(ms, 3),
        "eager_ms_per_step": round(eager_ms, 3),
        "graph_ms_per_step": None if graph_ms is None else round(graph_ms, 3),
        "launch": "hip graph" if use_graph else "eager",
        "steps": steps,
        "warmup": warmup,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"model": "Mamba-1 130M shape", "params_m": round(n_params / 1e6, 2), **m,
                   "global_batch": C5_BATCH, "seq_len": C5_LENGTH, "optimizer": "AdamW (mss_adamw: one launch per step, writes the bf16 weight shadows)",
                   "parallelism": "none (1 GPU)"},
    }


def run_decode_c5(torch, steps, prompt_len=2048, graph=True):
    """Decode with the config-5 model (B=8, bf16): prefill a `prompt_len` prompt, then time
    `steps` single-token steps (HIP state/conv-window updates in place), eagerly and as one
    captured HIP graph per step (the caches and the token are static buffers)."""
    from mamba_amd.mamba1 import MambaLM

    torch.manual_seed(0)
    m = C5_MODEL
    model = MambaLM(m["vocab"], m["d_model"], m["n_layers"], m["expand"], m["d_state"], m["dt_rank"],
                    m["d_conv"], device="cuda")
    gen = torch.Generator(device="cuda").manual_seed(1)
    prompt = torch.randint(0, m["vocab"], (C5_BATCH, prompt_len), device="cuda", generator=gen)
    _, caches = model.prefill(prompt)
    token = torch.randint(0, m["vocab"], (C5_BATCH,), device="cuda", generator=gen)

    def timed(fn, n):
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record()
        for _ in range(n):
            fn()
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / n

    eager = lambda: model.step(token, caches)
    for _ in range(3):
        eager()
    eager_ms = timed(eager, steps)
    ms = eager_ms
    if graph:
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            model.step(token, caches)
        torch.cuda.current_stream().wait_stream(side)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            model.step(token, caches)
        g.replay()
        ms = timed(g.replay, steps)
        del g
    log(f"[bench] c5 decode: {eager_ms:.3f} ms/token eager, {ms:.3f} ms/token {'graph' if graph else 'eager'}")
    del model, caches
    torch.cuda.empty_cache()
    return {"metric": "Mamba-1 130M decode tokens/s", "value": round(C5_BATCH / (ms * 1e-3), 1),
            "unit": "tokens/s", "ms_per_token_step": round(ms, 4), "eager_ms_per_token_step": round(eager_ms, 4),
            "hip_graph": bool(graph), "batch": C5_BATCH, "prompt_len": prompt_len, "steps": steps,
            "dtype": "bf16"}


def cpu_baseline(torch, cfg, target_s, lens=None, d0=32):
    """Reference composition on the CPU: softplus(delta + bias) (x validity mask for
    variable lengths, mamba/mamba1.py:165-168) -> pure-JAX-style scan (oracle/assoc_torch.py,
    mamba/selective_scan_cuda.py:56-90) -> + D*u -> * silu(z); loss-weighted backward
    through autograd, in fp32 (bf16 configs use bf16-rounded inputs). Timed on a slice of
    channels (channels are independent) and scaled to the full channel count."""
    from mamba_amd.configs import make_scan_inputs, ScanConfig
    from oracle.assoc_torch import selective_scan_reference

    threads = max(1, min(len(os.sched_getaffinity(0)), 16))
    torch.set_num_threads(threads)
    mask = None
    if lens is not None:
        mask = (torch.arange(cfg.length)[None, :, None] < torch.as_tensor(lens)[:, None, None]).float()

    def run(dslice):
        sub = ScanConfig("slice", cfg.batch, dslice, cfg.length, cfg.dstate, cfg.dtype)
        x = make_scan_inputs(sub, seed=0, with_z=True, with_dout=True)
        tr = lambda a: torch.from_numpy(np.ascontiguousarray(np.swapaxes(a, 1, 2)))
        u, dr, z, dout = (tr(x[k]) for k in ("u", "delta", "z", "dout"))
        Bs, Cs = tr(x["B"]), tr(x["C"])
        A = torch.from_numpy(x["A"]).requires_grad_(True)
        bias = torch.from_numpy(x["delta_bias"]).requires_grad_(True)
        D = torch.from_numpy(x["D"]).requires_grad_(True)
        for v in (u, dr, z, Bs, Cs):
            v.requires_grad_(True)
        t0 = time.perf_counter()
        deltas = torch.nn.functional.softplus(dr + bias)
        if mask is not None:
            deltas = deltas * mask
        y, last = selective_scan_reference(A, deltas, Bs, Cs, u)
        out = (y + D * u) * torch.nn.functional.silu(z)
        loss = (out * dout).sum() + last.sum() * 0.0
        loss.backward()
        return time.perf_counter() - t0

    run(d0)
    t_probe = run(d0)
    dslice = max(8, int(np.clip(d0 * (target_s / 4.0) / max(t_probe, 1e-3), d0, cfg.dim)) // 8 * 8)
    log(f"[bench] {cfg.name} cpu baseline probe D={d0}: {t_probe:.2f} s; timing slice D={dslice} x3 "
        f"on {threads} threads")
    if dslice != d0:
        run(dslice)
    times = []
    for i in range(3):
        times.append(run(dslice))
        log(f"[bench] {cfg.name} cpu baseline rep {i}: {times[-1]:.2f} s")
    t_med = float(np.median(times))
    t_full = t_med * cfg.dim / dslice
    tokens = int(np.sum(lens)) if lens is not None else cfg.batch * cfg.length
    return {
        "value": tokens / t_full,
        "unit": "tokens/s",
        "cores": threads,
        "cpu_model": cpu_model(),
        "kind": "port",
        "sample": (f"{cfg.name}: B={cfg.batch} L={cfg.length} N={cfg.dstate} ({cfg.dtype} inputs, fp32 math), "
                   f"{dslice} of {cfg.dim} channels, fwd+bwd (autograd) median of 3 = {t_med:.3f} s, "
                   f"scaled x{cfg.dim / dslice:.1f} to all channels ({t_full:.2f} s per step)"),
    }


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--cpu-seconds", type=float, default=8.0,
                    help="approximate CPU work for the CPU baseline (0 disables it)")
    ap.add_argument("--configs", default="c2,c3,c4",
                    help="scan configs to measure (c2 is always the headline line)")
    ap.add_argument("--config-steps", type=int, default=10, help="timed steps for c3/c4")
    ap.add_argument("--train-steps", type=int, default=10,
                    help="timed config-5 training steps (0 skips the training measurement)")
    ap.add_argument("--train-warmup", type=int, default=3)
    ap.add_argument("--decode-steps", type=int, default=50,
                    help="timed single-token decode steps of the config-5 model (0 skips them)")
    ap.add_argument("--complex-steps", type=int, default=10,
                    help="timed steps of the complex-A scan at the config-2 shape (0 skips them)")
    ap.add_argument("--reference-api-steps", type=int, default=20,
                    help="timed steps of the reference-signature entry points at the config-2 shape, "
                         "plus their forward at the reference's own shapes (0 skips them)")
    ap.add_argument("--train-eager", action="store_true",
                    help="time the config-5 step eagerly only (no HIP graph capture)")
    ap.add_argument("--device-warmup-s", type=float, default=0.2,
                    help="seconds of bf16 GEMMs run right before each timed leg's warmup steps, so that "
                         "the GPU has left its idle clocks (0 disables it)")
    ap.add_argument("--calibration-copy-mib", type=int, default=0,
                    help="after the timed region, copy a device buffer of this many MiB twice "
                         "(a kernel of known traffic for scaling rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE={world}); "
              "this build has no multi-GPU path.", file=sys.stderr)
        sys.exit(2)

    import torch
    from mamba_amd.configs import CONFIGS, C2, algorithmic_bytes

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(1)
    cfg = C2
    global DEVICE_WARMUP_S
    DEVICE_WARMUP_S = args.device_warmup_s
    r2 = run_gpu(torch, cfg, args.steps, args.warmup)
    ms, fwd_ms, bwd_ms, red_ms = r2["ms"], r2["fwd"], r2["bwd_scan"], r2["bwd_reduce"]
    fwd_bytes, bwd_bytes = algorithmic_bytes(cfg)
    tokens = cfg.batch * cfg.length
    # Dominant kernel: the backward scan (backward algorithmic bytes attributed to it; the
    # reduction kernels that finish dB/dC/dA/dD/dbias are timed separately).
    if bwd_ms >= fwd_ms:
        tag, bytes_, dur = "bwd_scan_c2", bwd_bytes, bwd_ms
    else:
        tag, bytes_, dur = "fwd_c2", fwd_bytes, fwd_ms
    achieved = bytes_ / (dur * 1e-3) / 1e9
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": read_traffic(tag),
                "kernel": tag, "algorithmic_bytes": bytes_, "avg_launch_ms": round(dur, 5)}
    if tag.startswith("bwd"):
        roofline["bytes_over"] = BWD_BYTES_OVER
        roofline["backward_as_launched"] = as_launched(bwd_bytes, bwd_ms, red_ms)
    if args.calibration_copy_mib > 0:
        src = torch.ones(args.calibration_copy_mib * (1 << 20) // 4, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(2):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"[bench] calibration copy of {args.calibration_copy_mib} MiB done")
        del src, dst
    per_config = {"c2": scan_report(cfg, r2)}
    others = [c for c in args.configs.split(",") if c and c != "c2"]
    results = {}
    for name in others:
        c = CONFIGS[name]
        results[name] = run_gpu(torch, c, args.config_steps, max(1, args.config_steps // 4))
        per_config[name] = scan_report(c, results[name])
    train = None
    if args.train_steps > 0:
        train = run_train_c5(torch, args.train_steps, args.train_warmup, graph=not args.train_eager)
    decode = None
    if args.decode_steps > 0:
        decode = run_decode_c5(torch, args.decode_steps, graph=not args.train_eager)
    ref_api = None
    if args.reference_api_steps > 0:
        ref_api = run_reference_api(torch, args.reference_api_steps, max(1, args.reference_api_steps // 4))
    cplx = None
    if args.complex_steps > 0:
        cplx = run_complex_c2(torch, args.complex_steps, max(1, args.complex_steps // 4))
    cpu = None
    if args.cpu_seconds > 0:
        cpu = cpu_baseline(torch, cfg, args.cpu_seconds)
        per_config["c2"]["cpu_baseline"] = cpu
        for name in others:
            per_config[name]["cpu_baseline"] = cpu_baseline(torch, CONFIGS[name], args.cpu_seconds / 2,
                                                            results[name]["lens"], d0=8)
        if cplx is not None:
            cplx["cpu_baseline"] = cpu_baseline_complex(torch, args.cpu_seconds / 2)
    step_bytes = fwd_bytes + bwd_bytes
    result = {
        "metric": METRIC,
        "value": round(tokens / (ms * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "ms_per_step_eager": round(r2["eager_ms"], 5),
        "ms_per_step_graph": None if r2.get("graph_ms") is None else round(r2["graph_ms"], 5),
        "launch": ("hip graph replay of the step's three launches" if r2["graph"] else
                   "eager launches of the step's three kernels") + " (the faster median of 3 trials each)",
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "c2: selective_scan fwd+bwd fp32, softplus(delta+bias), D skip, silu(z) gate, "
                               "last state", "batch": cfg.batch, "dim": cfg.dim, "seq_len": cfg.length,
                   "dstate": cfg.dstate, "parallelism": "none (1 GPU)"},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "fwd_bwd_hbm_frac": round(step_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "kernels_ms": {"fwd": round(fwd_ms, 5), "bwd_scan": round(bwd_ms, 5), "bwd_reduce": round(red_ms, 5)},
        "configs": per_config,
        "train_c5": train,
        "decode_c5": decode,
        "complex_c2": cplx,
        "reference_api_c2": ref_api,
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
