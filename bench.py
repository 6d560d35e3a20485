#!/usr/bin/env python3
"""Benchmark of First Passage Attention on one MI355X (the BASELINE.json metric).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config cfg2|cfg3|cfg4]
    python bench.py --workload lm [--steps K] [--warmup W]     # cfg5 LM training step

A step is one forward + backward of ``first_passage_attention(..., impl="hip")`` over
one batch of synthetic inputs already resident in HBM (BASELINE.json config 2 by
default: B4 H12 T2048 D64 fp16; q,k,v ~ N(0,1); phi = cumsum N(0,1); psi = phi + N(0,1);
beta = 1; gradients of o.float().sum() w.r.t. q, k, v, phi, psi, beta).  W untimed
steps, then K steps timed between two device synchronisations.  Rank 0 prints one
JSON line.  ``value`` is fwd+bwd TFLOP/s of the algorithmic flops 14*D*P
(P = B*H*T*(T+1)/2 causal pairs; bias and soft-min work not counted).

``--workload lm`` times instead one training step (fp16 autocast forward, backward with a
gradient scaler, AdamW update) of fpa.lm.FPADecoder, a 12-layer d768 H12 pre-norm decoder
whose attention is the FirstPassageAttention layer on the HIP kernels, over B8 x T2048 random
tokens (cfg5); ``value`` is tokens per second.

Per-kernel times come from HIP events recorded on torch's current stream (the stream
every kernel is launched on) around C-ABI calls that enqueue one kernel each; the
dominant kernel's duration gives ``roofline``.  ``roofline.traffic`` is that kernel's HBM
bytes per launch from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE summary
(profiles/fpa_<config>_traffic.txt), null when the workload has none.  ``cpu_baseline`` times the float32
CPU oracle (a port of the reference's dense path) on a bounded sample of heads of
the same workload.
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
    "cfg2": dict(B=4, H=12, T=2048, D=64, dtype="f16", beta="ones", drift=0.0),
    "cfg3": dict(B=2, H=8, T=4096, D=128, dtype="f32", beta="softplus", drift=0.0),
    "cfg4": dict(B=1, H=12, T=16381, D=64, dtype="f16", beta="ones", drift=0.01),
}


def make_inputs(cfg, seed=0):
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


def cpu_baseline(cfg, seconds):
    """Time the float32 CPU oracle (fwd + bwd of single heads of the workload) for ~`seconds`."""
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
            "sample": f"{len(times)} x one head (B1 H1 T{T} D{D}) fwd+bwd of the float32 dense oracle, "
                      f"median {t:.3f} s/head"}


LM = dict(B=8, T=2048, d_model=768, n_heads=12, layers=12, d_mlp=3072, vocab=32000)


def run_lm(a):
    """cfg5: tokens/s of one LM training step (see the module docstring)."""
    import torch
    from fpa.lm import FPADecoder

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    torch.manual_seed(0)
    model = FPADecoder(LM["vocab"], LM["d_model"], LM["n_heads"], LM["layers"], LM["d_mlp"], impl="hip").to(dev)
    opt = torch.optim.AdamW(model.parameters(), lr=1e-4)
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

    for _ in range(a.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(a.steps):
        loss = step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / a.steps
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
        "config": {"workload": "cfg5: FPADecoder training step (AdamW, grad scaler)", **LM,
                   "parallelism": "single GPU"},
        "final_loss": round(loss.item(), 4),
        "roofline": None,
        "cpu_baseline": None,
    }
    print(json.dumps(res), flush=True)


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="cfg2", choices=sorted(CONFIGS))
    ap.add_argument("--workload", default="fpa", choices=("fpa", "lm"),
                    help="fpa: the attention forward+backward of --config; lm: the cfg5 LM training step")
    ap.add_argument("--kernel-reps", type=int, default=20)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true", help="skip the cpu_baseline leg")
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

    cfg = CONFIGS[a.config]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if a.copy_mib:
        src = torch.ones(a.copy_mib << 18, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    q, k, v, phi, psi, beta, do = (t.to(dev) for t in make_inputs(cfg))
    leaves = [t.clone().requires_grad_() for t in (q, k, v, phi, psi, beta)]

    def step():
        o = fpa.first_passage_attention(*leaves, impl="hip")
        torch.autograd.grad(o, leaves, do)

    for _ in range(a.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(a.steps):
        step()
    torch.cuda.synchronize()
    fwd_bwd_ms = (time.perf_counter() - t0) * 1e3 / a.steps

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
    for _ in range(a.warmup):
        graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(a.steps):
        graph.replay()
    torch.cuda.synchronize()
    graph_ms = (time.perf_counter() - t0) * 1e3 / a.steps
    del graph

    with torch.no_grad():
        for _ in range(a.warmup):
            fpa.first_passage_attention(q, k, v, phi, psi, beta, impl="hip")
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(a.steps):
            fpa.first_passage_attention(q, k, v, phi, psi, beta, impl="hip")
        torch.cuda.synchronize()
        fwd_ms = (time.perf_counter() - t0) * 1e3 / a.steps

    # Per-kernel durations: one C-ABI call per kernel (phases), HIP events on the launch stream.
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
    # The kernels of a step, with their algorithmic flops.  The backward's key side (S, dP, dV, dK:
    # 8*D per pair) and query side (dQ: 2*D per pair; it recomputes S and dP) run as one launch.
    kernels = {
        "fpa_stats": (time_call(fa, _hip.run_fwd, _lib.FPA_FWD_STATS), 0),
        "fpa_fwd_kernel": (time_call(fa, _hip.run_fwd, _lib.FPA_FWD_MAIN), 4 * D * P),
        "fpa_bwd_prep": (time_call(ba, _hip.run_bwd, _lib.FPA_BWD_DELTA), 0),
        "fpa_bwd_kvq_kernel": (time_call(ba, _hip.run_bwd, _lib.FPA_BWD_KEYS | _lib.FPA_BWD_QUERIES), 10 * D * P),
        "fpa_bwd_combine_kernel": (time_call(ba, _hip.run_bwd, _lib.FPA_BWD_PHI), 0),
    }
    # Each side launched alone (not part of the step): for comparison with the fused launch.
    alone = {"fpa_bwd_kv_kernel": time_call(ba, _hip.run_bwd, _lib.FPA_BWD_KEYS),
             "fpa_bwd_q_kernel": time_call(ba, _hip.run_bwd, _lib.FPA_BWD_QUERIES)}
    dom = max(kernels, key=lambda n: kernels[n][0])
    dom_ms, dom_flops = kernels[dom]
    peak = PEAK_TFLOPS[cfg["dtype"]]
    achieved = dom_flops / (dom_ms * 1e-3) / 1e12

    fwd_flops, fb_flops = 4 * D * P, 14 * D * P
    fb_tflops = fb_flops / (fwd_bwd_ms * 1e-3) / 1e12
    fwd_tflops = fwd_flops / (fwd_ms * 1e-3) / 1e12

    cpu = None
    if not a.no_cpu:
        cpu = cpu_baseline(cfg, a.cpu_seconds)

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
        "config": {"workload": f"{a.config}: FPA forward+backward B{cfg['B']} H{cfg['H']} T{cfg['T']} "
                               f"D{cfg['D']} {cfg['dtype']}",
                   "B": cfg["B"], "H": cfg["H"], "T": cfg["T"], "D": D, "parallelism": "single GPU"},
        "fwd_ms": round(fwd_ms, 4),
        "fwd_bwd_ms": round(fwd_bwd_ms, 4),
        "fwd_bwd_graph_ms": round(graph_ms, 4),
        "fwd_tflops": round(fwd_tflops, 3),
        "fwd_pct_peak": round(100 * fwd_tflops / peak, 2),
        "fwd_bwd_pct_peak": round(100 * fb_tflops / peak, 2),
        "kernel_ms": {n: round(t, 4) for n, (t, _) in kernels.items()},
        "kernel_ms_alone": {n: round(t, 4) for n, t in alone.items()},
        "roofline": {"kernel": dom, "bound": "mfma", "achieved": round(achieved, 3), "peak": peak,
                     "unit": "TFLOP/s", "frac": round(achieved / peak, 4),
                     "traffic": measured_traffic(a.config, dom)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
