#!/usr/bin/env python3
"""Benchmark of First Passage Attention on one MI355X (the BASELINE.json metric).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config cfg2|cfg3|cfg4] [--no-extra] [--no-cpu]
    python bench.py --shape B,H,T,D [--dtype fp16|fp32] [--rounds N] [--json FILE]   # any shape
    python bench.py --workload lm [--steps K] [--warmup W]     # the cfg5 LM training step alone

A step is one forward + backward of ``first_passage_attention(..., impl="hip")`` over one batch of
synthetic inputs already resident in HBM (BASELINE.json config 2 by default: B4 H12 T2048 D64 fp16;
q,k,v ~ N(0,1); phi = cumsum N(0,1); psi = phi + N(0,1); beta = 1; the gradients of the config's loss
o.float().sum(), i.e. dO = 1, w.r.t. q, k, v, phi, psi, beta).  W untimed steps, then K steps timed
between two device synchronisations.  Before the W warm-up steps the step runs for ``--settle``
seconds (0.3) untimed: MI355X needs some tens of milliseconds of load before its clocks settle, and a
timed region of a few milliseconds right after start measures up to 15% slow (20 steps after 5
warm-ups, cfg2: 0.275-0.279 ms; after 0.05 s of steps: 0.237 ms, the sum of the kernels).  One JSON line.  ``value`` is fwd+bwd TFLOP/s of the algorithmic
flops 14*D*P (P = B*H*T*(T+1)/2 causal pairs; bias and soft-min work not counted).
``fwd_bwd_ms_with_clones`` times the reference bench's step (bench.py:46-48 of the reference: fresh
clones of the six inputs, forward, backward) beside it.

The default run adds, under ``configs``, the other BASELINE.json workloads: cfg3 and cfg4 (forward and
forward+backward ms, % of the dtype's MFMA peak) and cfg5 (one training step of fpa.lm.FPADecoder: a
12-layer d768 H12 pre-norm decoder over B8 x T2048 random tokens, fp16 autocast, gradient scaler,
AdamW, fused where torch has it; tokens/s; and the forward+backward alone, as BASELINE.json's cfg5
defines it: ``fwd_bwd_tokens_per_s``).

``ref_protocol`` repeats the measurement with the reference bench's protocol (its bench.py:11-23,
50-54): each call timed alone between two HIP events, 3 warm-ups + 15 timed calls, the median, over
--rounds rounds (5), the median of the rounds; its fwd+bwd call clones the six inputs as the
reference's does.  --shape / --dtype time any shape with that protocol and the step above (the
config's distributions, dO = 1); --json also writes the line to a file.

Per-kernel times come from HIP events recorded on torch's current stream (the stream every kernel is
launched on) around C-ABI calls that enqueue one kernel each; the dominant kernel's duration gives
``roofline``.  ``roofline.traffic`` is that kernel's HBM bytes per launch from the committed rocprofv3
FETCH_SIZE/WRITE_SIZE summary (profiles/fpa_<config>_traffic.txt), null when there is none.
``cpu_baseline`` times the float32 CPU oracle (a port of the reference's dense path) on a bounded
sample of heads of the same workload; ``cpu_baseline_cfg1`` times it on BASELINE.json config 1.
"""
import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "first-passage-attention_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "FPA fwd & fwd+bwd ms + TFLOP/s (% MFMA peak) at B4 H12 T2048 D64 fp16"
PEAK_TFLOPS = {"f16": 2516.6, "f32": 157.3}  # MI355X dense MFMA (AMD public figures)

CONFIGS = {
    "cfg1": dict(B=1, H=2, T=256, D=32, dtype="f32", beta="ones", drift=0.0),
    "cfg2": dict(B=4, H=12, T=2048, D=64, dtype="f16", beta="ones", drift=0.0),
    "cfg3": dict(B=2, H=8, T=4096, D=128, dtype="f32", beta="softplus", drift=0.0),
    "cfg4": dict(B=1, H=12, T=16381, D=64, dtype="f16", beta="ones", drift=0.01),
}


def make_inputs(cfg, seed=0, random_do=False):
    """(q, k, v, phi, psi, beta, do) of a config, drawn from one CPU generator in the order q, k, v, dO,
    phi increments, psi noise (then beta for "softplus").  do is the gradient of o.float().sum() (ones)
    unless random_do."""
    import torch
    dt = torch.float16 if cfg["dtype"] == "f16" else torch.float32
    B, H, T, D = cfg["B"], cfg["H"], cfg["T"], cfg["D"]
    g = torch.Generator().manual_seed(seed)
    q, k, v, do = (torch.randn(B, H, T, D, generator=g).to(dt) for _ in range(4))
    phi = torch.randn(B, H, T, generator=g).cumsum(-1) - cfg["drift"] * torch.arange(T, dtype=torch.float32)
    psi = phi + torch.randn(B, H, T, generator=g)
    if cfg["beta"] == "ones":
        beta = torch.ones(H)
    else:
        beta = torch.nn.functional.softplus(torch.randn(H, generator=g))
    if not random_do:
        do = torch.ones_like(do)
    return q, k, v, phi, psi, beta, do


def measured_traffic(config, kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary
    (profiles/fpa_<config>_traffic.txt), or None when there is none for this workload."""
    path = os.path.join(ROOT, "profiles", f"fpa_{config}_traffic.txt")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith(kernel + ":"):
            return int(float(line.split(":", 1)[1]))
    return None


def pairs(cfg):
    return cfg["B"] * cfg["H"] * cfg["T"] * (cfg["T"] + 1) // 2


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(cfg, seconds):
    """Time the float32 CPU oracle (fwd + bwd of single heads of the workload) for ~`seconds`, on the
    host's torch threads (16 on the GPU boxes: OMP_NUM_THREADS)."""
    import torch
    from oracle import fpa_oracle as O
    cores = torch.get_num_threads()
    T, D = cfg["T"], cfg["D"]
    q, k, v, phi, psi, beta, do = make_inputs(dict(cfg, B=1, H=1), seed=1)
    O.fpa_grads(q[..., :128, :], k[..., :128, :], v[..., :128, :], phi[..., :128], psi[..., :128], beta,
                do[..., :128, :], dtype=torch.float32)  # warm-up
    times = []
    t_end = time.perf_counter() + seconds
    while True:
        t0 = time.perf_counter()
        O.fpa_grads(q, k, v, phi, psi, beta, do, dtype=torch.float32)
        times.append(time.perf_counter() - t0)
        if time.perf_counter() > t_end:
            break
    t = statistics.median(times)
    flops = 14 * D * T * (T + 1) / 2
    return {"value": flops / t / 1e12, "unit": "TFLOP/s", "cores": cores, "kind": "port",
            "host_cpus": os.cpu_count(), "cpu_model": _cpu_model(),
            "sample": f"{len(times)} x one head (B1 H1 T{T} D{D}) fwd+bwd of the float32 dense oracle "
                      f"(dO = 1), median {t:.3f} s/head"}


def cpu_baseline_cfg1():
    """BASELINE.json config 1 (B1 H2 T256 D32 fp32, loss o.sum(), seed 0) forward+backward on the float32
    CPU oracle: 3 warm-ups, median of 15."""
    import torch
    from oracle import fpa_oracle as O
    q, k, v, phi, psi, beta, do = make_inputs(CONFIGS["cfg1"], seed=0)
    times = []
    for i in range(18):
        t0 = time.perf_counter()
        O.fpa_grads(q, k, v, phi, psi, beta, do, dtype=torch.float32)
        if i >= 3:
            times.append(time.perf_counter() - t0)
    ms = statistics.median(times) * 1e3
    return {"ms": round(ms, 3), "cores": torch.get_num_threads(), "host_cpus": os.cpu_count(),
            "cpu_model": _cpu_model(), "kind": "port",
            "sample": "B1 H2 T256 D32 fp32 forward+backward of the float32 dense oracle, median of 15"}


# The backward kernels of a step: (name, phases bitmask of fpa_bwd, algorithmic flops per causal pair / D).
# The key side (S, dP, dV, dK: 8 D per pair) and the query side (dQ: 2 D per pair; it recomputes S and
# dP) run as one launch.
BWD_KERNELS = (("fpa_bwd_prep", 1, 0), ("fpa_bwd_kvq_kernel", 2 | 4, 10), ("fpa_bwd_combine_kernel", 8, 0))

LM = dict(B=8, T=2048, d_model=768, n_heads=12, layers=12, d_mlp=3072, vocab=32000)


def lm_step_ms(steps, warmup, fb=True):
    """cfg5: ms per training step of the LM (see the module docstring), the last loss, ms of the
    forward+backward alone (BASELINE.json's cfg5: one forward+backward, no optimizer step; None when
    fb is False) and the optimizer used."""
    import torch
    from fpa.lm import FPADecoder

    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    model = FPADecoder(LM["vocab"], LM["d_model"], LM["n_heads"], LM["layers"], LM["d_mlp"], impl="hip").to(dev)
    try:  # one fused kernel per step for all parameters where this torch build has it
        opt, opt_name = torch.optim.AdamW(model.parameters(), lr=1e-4, fused=True), "AdamW (fused)"
    except (RuntimeError, ValueError, TypeError):
        opt, opt_name = torch.optim.AdamW(model.parameters(), lr=1e-4), "AdamW"
    scaler = torch.amp.GradScaler("cuda")
    g = torch.Generator().manual_seed(0)
    tokens = torch.randint(0, LM["vocab"], (LM["B"], LM["T"] + 1), generator=g).to(dev)

    def step():
        with torch.autocast("cuda", dtype=torch.float16):
            loss = model.loss(tokens)
        opt.zero_grad(set_to_none=True)
        scaler.scale(loss).backward()
        scaler.step(opt)
        scaler.update()
        return loss

    def fwd_bwd():
        with torch.autocast("cuda", dtype=torch.float16):
            loss = model.loss(tokens)
        model.zero_grad(set_to_none=True)
        scaler.scale(loss).backward()
        return loss

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        loss = step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    loss = loss.item()
    fb_ms = time_steps(fwd_bwd, steps, warmup) if fb else None
    del model, opt
    torch.cuda.empty_cache()
    return ms, loss, fb_ms, opt_name


def run_lm(a):
    """--workload lm: the cfg5 training step as the bench line."""
    import torch
    torch.cuda.set_device(0)
    ms, loss, fb_ms, opt_name = lm_step_ms(a.steps, a.warmup, fb=not a.no_extra)
    ntok = LM["B"] * LM["T"]
    res = {
        "metric": "LM training step tokens/s (cfg5: 12-layer d768 H12 FPA decoder, B8 T2048, fp16 autocast)",
        "value": round(ntok / (ms * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (uniform random tokens, random-init weights)",
        "fwd_bwd_ms": round(fb_ms, 3) if fb_ms else None,
        "fwd_bwd_tokens_per_s": round(ntok / (fb_ms * 1e-3), 1) if fb_ms else None,
        "config": {"workload": f"cfg5: FPADecoder training step ({opt_name}, grad scaler)", **LM,
                   "parallelism": "single GPU"},
        "final_loss": round(loss, 4),
        "roofline": None,
        "cpu_baseline": None,
    }
    print(json.dumps(res), flush=True)


def settle(fn, seconds):
    """Run fn untimed for about `seconds` of wall time (device clocks settle under load)."""
    import torch
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end:
        for _ in range(10):
            fn()
        torch.cuda.synchronize()


def time_steps(fn, steps, warmup):
    """ms per call of fn over `steps` back-to-back calls between two device synchronisations."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / steps


def time_ref_protocol(fn, rounds, warm=3, n=15):
    """The reference bench's timing (its bench.py:11-23, 50-54): per round, `warm` untimed calls, then `n`
    calls each between two events on the current stream with a synchronisation after each, median; the
    median over `rounds` rounds.  Returns (median ms, per-round ms)."""
    import torch
    per_round = []
    for _ in range(rounds):
        for _ in range(warm):
            fn()
        torch.cuda.synchronize()
        ts = []
        for _ in range(n):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            fn()
            b.record()
            torch.cuda.synchronize()
            ts.append(a.elapsed_time(b))
        per_round.append(statistics.median(ts))
    return statistics.median(per_round), per_round


def committed_counters(config, kernel):
    """MfmaUtil and VALUBusy (%) of `kernel` from the committed counter summary
    (profiles/fpa_<config>_counters.md), or None."""
    path = os.path.join(ROOT, "profiles", f"fpa_{config}_counters.md")
    if not os.path.exists(path):
        return None
    for line in open(path):
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) >= 3 and cells[0].startswith(kernel):
            try:
                return {"mfma_util_pct": float(cells[1]), "valu_busy_pct": float(cells[2])}
            except ValueError:
                return None
    return None


def committed_kernel_us(config, kernel):
    """Average duration (us) of `kernel` in the committed rocprofv3 kernel-trace summary
    (profiles/fpa_<config>_kernel_trace.md), or None."""
    path = os.path.join(ROOT, "profiles", f"fpa_{config}_kernel_trace.md")
    if not os.path.exists(path):
        return None
    for line in open(path):
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) >= 3 and cells[0].startswith(kernel):
            try:
                return float(cells[2])
            except ValueError:
                return None
    return None


def time_config(cfg, steps, warmup):
    """Forward and forward+backward ms of one config (inputs resident, leaves kept across steps)."""
    import torch
    import fpa
    dev = torch.device("cuda:0")
    q, k, v, phi, psi, beta, do = (t.to(dev) for t in make_inputs(cfg))
    leaves = [t.clone().requires_grad_() for t in (q, k, v, phi, psi, beta)]

    def step():
        o = fpa.first_passage_attention(*leaves, impl="hip")
        torch.autograd.grad(o, leaves, do)

    def fwd():
        with torch.no_grad():
            fpa.first_passage_attention(q, k, v, phi, psi, beta, impl="hip")

    fb = time_steps(step, steps, warmup)
    f = time_steps(fwd, steps, warmup)
    P, D = pairs(cfg), cfg["D"]
    peak = PEAK_TFLOPS[cfg["dtype"]]
    return {"workload": f"B{cfg['B']} H{cfg['H']} T{cfg['T']} D{D} {cfg['dtype']}",
            "fwd_ms": round(f, 4), "fwd_bwd_ms": round(fb, 4),
            "fwd_pct_peak": round(100 * 4 * D * P / (f * 1e-3) / 1e12 / peak, 2),
            "fwd_bwd_pct_peak": round(100 * 14 * D * P / (fb * 1e-3) / 1e12 / peak, 2)}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="cfg2", choices=[c for c in sorted(CONFIGS) if c != "cfg1"])
    ap.add_argument("--workload", default="fpa", choices=("fpa", "lm"),
                    help="fpa: the attention forward+backward of --config; lm: the cfg5 LM training step")
    ap.add_argument("--kernel-reps", type=int, default=20)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true", help="skip the cpu_baseline legs")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the other configs (cfg3, cfg4, cfg5); with --workload lm, the forward+backward timing")
    ap.add_argument("--shape", help="B,H,T,D: time this shape instead of --config (the config's distributions)")
    ap.add_argument("--dtype", choices=("fp16", "fp32"), default=None, help="with --shape (default fp16)")
    ap.add_argument("--rounds", type=int, default=5, help="rounds of the reference's timing protocol")
    ap.add_argument("--json", help="also write the JSON line to this file")
    ap.add_argument("--settle", type=float, default=0.3,
                    help="seconds of untimed steps before the warm-up (device clocks settle under load)")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="first run one device-to-device copy of this many MiB (a known-size kernel that "
                         "calibrates the FETCH_SIZE / WRITE_SIZE counters of a profiling run)")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(FPA shards over batch and heads with no communication, so one GPU's share is the "
              "same kernel at B/n or H/n)", file=sys.stderr)
        sys.exit(2)

    if a.workload == "lm":
        run_lm(a)
        return

    import torch
    import fpa
    from fpa import _hip, _lib

    cfg = dict(CONFIGS[a.config])
    custom = a.shape is not None
    if custom:
        B, H, T, D = (int(x) for x in a.shape.split(","))
        cfg.update(B=B, H=H, T=T, D=D, dtype="f32" if a.dtype == "fp32" else "f16")
        a.no_extra = True
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if a.copy_mib:
        src = torch.ones(a.copy_mib << 18, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    q, k, v, phi, psi, beta, do = (t.to(dev) for t in make_inputs(cfg))
    inputs = (q, k, v, phi, psi, beta)
    leaves = [t.clone().requires_grad_() for t in inputs]

    def step():
        o = fpa.first_passage_attention(*leaves, impl="hip")
        torch.autograd.grad(o, leaves, do)

    def step_with_clones():  # the reference bench's step (its bench.py:46-48)
        x = [t.clone().requires_grad_() for t in inputs]
        fpa.first_passage_attention(*x, impl="hip").backward(do)

    settle(step, a.settle)
    fwd_bwd_ms = time_steps(step, a.steps, a.warmup)
    clones_ms = time_steps(step_with_clones, a.steps, a.warmup)

    # The same step captured once in a HIP graph and replayed: the kernels without the host's
    # launch gaps (reported beside the eager step, which stays the bench value).
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    graph_ms = time_steps(graph.replay, a.steps, a.warmup)
    del graph

    def fwd():
        with torch.no_grad():
            fpa.first_passage_attention(*inputs, impl="hip")

    fwd_ms = time_steps(fwd, a.steps, a.warmup)
    ref_fwd, ref_fwd_rounds = time_ref_protocol(fwd, a.rounds)
    ref_fb, ref_fb_rounds = time_ref_protocol(step_with_clones, a.rounds)

    # Per-kernel durations: one C-ABI call per kernel (phases), HIP events on the launch stream, each
    # kernel (a) in the order of a step, one event after each call, so that it starts from the caches
    # the kernel before it left, as inside the timed steps and a kernel trace of them, and (b) repeated
    # alone, its inputs warm in the caches.
    qr, kr, vr = _hip.rows(q), _hip.rows(k), _hip.rows(v)
    phi32, psi32, beta32 = phi.float().contiguous(), psi.float().contiguous(), beta.float().contiguous()
    fb = _hip.FwdBuffers(qr)
    fa = _hip.fwd_args(qr, kr, vr, phi32, psi32, beta32, 1.0, fb)
    _hip.run_fwd(fa, dev)
    gb = _hip.BwdBuffers(qr)
    ba = _hip.bwd_args(qr, kr, vr, beta32, 1.0, fb, _hip.rows(do), gb)
    _hip.run_bwd(ba, dev)
    torch.cuda.synchronize()

    def time_call(args, runner, phases):
        args.phases = phases
        runner(args, dev)
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(a.kernel_reps):
            runner(args, dev)
        e.record()
        e.synchronize()
        args.phases = 0
        return s.elapsed_time(e) / a.kernel_reps

    P = pairs(cfg)
    D = cfg["D"]
    # The kernels of a step in their order, with their algorithmic flops.
    seq = [("fpa_stats", fa, _hip.run_fwd, _lib.FPA_FWD_STATS, 0),
           ("fpa_fwd_kernel", fa, _hip.run_fwd, _lib.FPA_FWD_MAIN, 4 * D * P)]
    if fb.ws is not None:  # split row tiles: their merge
        seq.append(("fpa_fwd_merge", fa, _hip.run_fwd, _lib.FPA_FWD_MERGE, 0))
    seq += [(name, ba, _hip.run_bwd, phases, flops * D * P) for name, phases, flops in BWD_KERNELS]

    def time_sequence(reps, warm=3):
        """Median over `reps` sequences (after `warm` untimed ones) of each kernel's event-to-event time."""
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(len(seq) + 1)]
        samples = [[] for _ in seq]
        for r in range(warm + reps):
            ev[0].record()
            for i, (_, args, runner, phases, _) in enumerate(seq):
                args.phases = phases
                runner(args, dev)
                ev[i + 1].record()
            ev[-1].synchronize()
            if r >= warm:
                for i in range(len(seq)):
                    samples[i].append(ev[i].elapsed_time(ev[i + 1]))
        fa.phases = ba.phases = 0
        return [statistics.median(s) for s in samples]

    in_seq = time_sequence(a.kernel_reps)
    kernels = {name: (ms, flops) for (name, _, _, _, flops), ms in zip(seq, in_seq)}
    # Alone: the merge reads and rewrites o, so it goes after the rest.
    order = [s for s in seq if s[0] != "fpa_fwd_merge"] + [s for s in seq if s[0] == "fpa_fwd_merge"]
    alone = {name: time_call(args, runner, phases) for name, args, runner, phases, _ in order}
    dom = max(kernels, key=lambda n: kernels[n][0])
    dom_ms, dom_flops = kernels[dom]
    peak = PEAK_TFLOPS[cfg["dtype"]]

    fwd_flops, fb_flops = 4 * D * P, 14 * D * P
    fb_tflops = fb_flops / (fwd_bwd_ms * 1e-3) / 1e12
    fwd_tflops = fwd_flops / (fwd_ms * 1e-3) / 1e12
    del fb, gb, fa, ba, leaves, q, k, v, phi, psi, beta, do, inputs
    torch.cuda.empty_cache()

    extra = {}
    if not a.no_extra:
        for name in ("cfg3", "cfg4"):
            if name != a.config:
                extra[name] = time_config(CONFIGS[name], 10, 3)
                torch.cuda.empty_cache()
        lm_ms, lm_loss, lm_fb_ms, opt_name = lm_step_ms(5, 2)
        ntok = LM["B"] * LM["T"]
        extra["cfg5"] = {"workload": f"FPADecoder training step: 12 layers d768 H12, B8 T2048, fp16 autocast, {opt_name}",
                         "ms_per_step": round(lm_ms, 3),
                         "tokens_per_s": round(ntok / (lm_ms * 1e-3), 1),
                         "fwd_bwd_ms": round(lm_fb_ms, 3),
                         "fwd_bwd_tokens_per_s": round(ntok / (lm_fb_ms * 1e-3), 1),
                         "loss": round(lm_loss, 4)}

    cpu = cpu1 = None
    if not a.no_cpu:
        cpu = cpu_baseline(cfg, a.cpu_seconds)
        cpu1 = cpu_baseline_cfg1()

    res = {
        "metric": METRIC,
        "value": round(fb_tflops, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(fwd_bwd_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": cfg["dtype"],
        "data": "synthetic",
        "config": {"workload": f"{'custom' if custom else a.config}: FPA forward+backward B{cfg['B']} H{cfg['H']} "
                               f"T{cfg['T']} D{cfg['D']} {cfg['dtype']}, dO = 1 (loss o.float().sum())",
                   "B": cfg["B"], "H": cfg["H"], "T": cfg["T"], "D": D, "parallelism": "single GPU"},
        "settle_s": a.settle,
        "fwd_ms": round(fwd_ms, 4),
        "fwd_bwd_ms": round(fwd_bwd_ms, 4),
        "fwd_bwd_ms_with_clones": round(clones_ms, 4),
        "fwd_bwd_graph_ms": round(graph_ms, 4),
        "fwd_tflops": round(fwd_tflops, 3),
        "fwd_pct_peak": round(100 * fwd_tflops / peak, 2),
        "fwd_bwd_pct_peak": round(100 * fb_tflops / peak, 2),
        "ref_protocol": {"fwd_ms": round(ref_fwd, 4), "fwd_bwd_ms": round(ref_fb, 4),
                         "fwd_bwd_pct_peak": round(100 * fb_flops / (ref_fb * 1e-3) / 1e12 / peak, 2),
                         "rounds_ms": {"fwd": [round(x, 4) for x in ref_fwd_rounds],
                                       "fwd_bwd": [round(x, 4) for x in ref_fb_rounds]},
                         "protocol": f"median of {a.rounds} rounds x (3 warm-ups + median of 15 event-timed "
                                     "calls, synchronised after each); fwd+bwd clones the inputs "
                                     "(reference bench.py:11-23, 44-54)"},
        "kernel_ms": {n: round(t, 4) for n, (t, _) in kernels.items()},
        "kernel_ms_alone": {n: round(t, 4) for n, t in alone.items()},
        "roofline": roofline(a.config, custom, dom, dom_ms, dom_flops, peak),
        "configs": extra,
        "cpu_baseline": cpu,
        "cpu_baseline_cfg1": cpu1,
    }
    line = json.dumps(res)
    print(line, flush=True)
    if a.json:
        with open(a.json, "w") as f:
            f.write(line + "\n")


def roofline(config, custom, dom, dom_ms, dom_flops, peak):
    """The dominant kernel against the dense MFMA peak of the dtype.  `bound` is its roofline regime by
    arithmetic intensity (10 D flops per pair against a few bytes: far above the ridge of 2.5e15 / 8e12
    flop/B, so "mfma"); `limiter` is what the committed counters show issuing most (VALU or MFMA), and
    `frac_profile` the same fraction from the committed rocprofv3 trace, measured on another box (MI355X
    boxes differ by a few percent)."""
    achieved = dom_flops / (dom_ms * 1e-3) / 1e12
    r = {"kernel": dom, "bound": "mfma", "achieved": round(achieved, 3), "peak": peak, "unit": "TFLOP/s",
         "frac": round(achieved / peak, 4), "traffic": None if custom else measured_traffic(config, dom)}
    cnt = None if custom else committed_counters(config, dom)
    if cnt:
        r["limiter"] = dict(cnt, unit="VALU" if cnt["valu_busy_pct"] > cnt["mfma_util_pct"] else "MFMA",
                            source=f"profiles/fpa_{config}_counters.md")
    us = None if custom else committed_kernel_us(config, dom)
    if us:
        r["profile_us"] = us
        r["frac_profile"] = round(dom_flops / (us * 1e-6) / 1e12 / peak, 4)
    return r


if __name__ == "__main__":
    main()
