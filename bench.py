#!/usr/bin/env python
"""Atlas memory-layer chunk-scan throughput on one MI355X.

Workload (default): the 8 memory layers of the ~59M Atlas
LM, each a chunk scan + read-out over B=8 x T=4096 tokens, H=8 heads,
D=64, E=128 (memory_expand 2), chunk 64, Omega window 32, 5 Polar-Express
steps; bf16 q/k/v, fp32 gates and fp32 carried state.  Synthetic inputs with
the config-1 distributions (q, k unit-norm rows, v ~ N(0,1), gates = sigmoid of
N(0,1) logits, eta times max_lr 0.1), resident in HBM before timing; every
layer starts from the model's initial state (W1=0, W2=[I;0], S=0).

A step = the 8 layer scans.  value = memory-layer tokens/s = B*T*layers / t.
Prints one JSON line on stdout (logs go to stderr).
"""

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (ROOT, os.path.join(ROOT, "atlas-jax_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

PEAK_BF16_TFLOPS = 2516.6      # MI355X dense bf16/fp16 MFMA
METRIC = "memory-layer tokens/sec on 1 MI355X (4K–128K seq); MFMA util % of peak"

CONFIGS = {
    "c2": dict(workload="C2: Atlas ~59M LM memory layers (8 layers, B8 T4096 H8 D64 E128 cs64 w32 ns5)",
               B=8, T=4096, H=8, D=64, E=128, cs=64, w=32, ns=5, layers=8),
    "c1": dict(workload="C1: isolated layer (B1 T1024 H4 D32 E32 cs64 w16 ns5, fp32)",
               B=1, T=1024, H=4, D=32, E=32, cs=64, w=16, ns=5, layers=1),
    "c3": dict(workload="C3: Atlas ~170M LM memory layers (12 layers, B16 T4096 H12 D64 E256 cs64 w64 ns5)",
               B=16, T=4096, H=12, D=64, E=256, cs=64, w=64, ns=5, layers=12),
    "c4": dict(workload="C4: long-context layer (B1 T131072 H16 D64 E128 cs64 w64 ns5)",
               B=1, T=131072, H=16, D=64, E=128, cs=64, w=64, ns=5, layers=1),
    "c5": dict(workload="C5: MAG stack memory layers (12 layers, B4 T16384 H12 D64 E256 cs128 w16 ns5)",
               B=4, T=16384, H=12, D=64, E=256, cs=128, w=16, ns=5, layers=12),
}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def flops_per_token_head(D, E, ns):
    """Algorithmic flops of one token-head: Polar-Express on both memory
    matrices (Gram 2D^2E, A^2 2D^3, update 2D^2E per matrix and step) plus the
    inner-gradient, outer-product and read-out matvecs (12DE)."""
    return ns * (8 * D * D * E + 4 * D ** 3) + 12 * D * E


def make_layer_inputs(cfg, io_dtype, seed):
    import torch
    g = torch.Generator(device="cuda").manual_seed(seed)
    B, T, H, D = cfg["B"], cfg["T"], cfg["H"], cfg["D"]

    def unit(x):
        return x / x.norm(dim=-1, keepdim=True)

    q = unit(torch.randn(B, T, H, D, device="cuda", generator=g)).to(io_dtype)
    k = unit(torch.randn(B, T, H, D, device="cuda", generator=g)).to(io_dtype)
    v = torch.randn(B, T, H, D, device="cuda", generator=g).to(io_dtype)
    gates = [torch.sigmoid(torch.randn(B, T, H, device="cuda", generator=g)) for _ in range(4)]
    gates[1] = gates[1] * 0.1
    return q, k, v, gates


def initial_state(cfg):
    import torch
    from atlas_amd import DeepMemoryState
    B, H, D, E = cfg["B"], cfg["H"], cfg["D"], cfg["E"]
    W1 = torch.zeros(B, H, D, E, device="cuda")
    W2 = torch.zeros(B, H, E, D, device="cuda")
    W2[:, :, :D, :D] = torch.eye(D, device="cuda")
    return DeepMemoryState(W1, W2, torch.zeros_like(W1), torch.zeros_like(W2))


def measured_traffic(config, precision):
    """HBM bytes per phase-kernel launch (mean of the W2 and W1 phases), as
    measured by rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE runs and scaled by
    the same counters on a copy of known size; read from the committed
    summary profiles/phase_<config>_<precision>_traffic.md (None if absent)."""
    path = os.path.join(ROOT, "profiles", f"phase_{config}_{precision}_traffic.md")
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch:"):
                return float(line.split(":", 1)[1].strip())
    except OSError:
        pass
    return None


MODEL_CFGS = {
    # ~59M Atlas LM, bf16 weights/activations, fp32 scan state
    "c2": dict(n_layer=8, n_embd=512, n_head=8, memory_expand=2, chunk_size=64, omega_window=32, ns_steps=5,
               poly_degree=2, vocab_size=32768, B=8, T=4096),
    # ~170M Atlas LM
    "c3": dict(n_layer=12, n_embd=768, n_head=12, memory_expand=4, chunk_size=64, omega_window=64, ns_steps=5,
               poly_degree=2, vocab_size=32768, B=16, T=4096),
    # MAG stack (sliding-window attention, window 2048, + gated memory on every layer)
    "c5": dict(n_layer=12, n_embd=768, n_head=12, memory_expand=4, chunk_size=128, omega_window=16, ns_steps=5,
               poly_degree=2, vocab_size=32768, window_size=2048, B=4, T=16384, mag=True),
}


def model_forward(config_name, steps, warmup, precision):
    """Full Atlas LM forward (embedding, 8 blocks of memory layer + GEGLU MLP,
    final norm, LM head) on token ids drawn uniformly from the vocabulary,
    weights ~ N(0, 0.02); returns tokens/s = B*T / forward time."""
    import torch
    from atlas_amd import Atlas, AtlasConfig, MAGTransformer
    mc = dict(MODEL_CFGS[config_name])
    B, T, mag = mc.pop("B"), mc.pop("T"), mc.pop("mag", False)
    cfg = AtlasConfig(**mc, scan_precision=precision)
    gen = torch.Generator(device="cuda").manual_seed(0)
    if mag:
        # layer-default initialisation (uniform +-1/sqrt(fan_in), memory W_init Xavier)
        model = MAGTransformer(cfg, generator=gen, device="cuda", dtype=torch.bfloat16)
    else:
        model = Atlas(cfg, generator=gen, device="cuda", dtype=torch.bfloat16, init_std=0.02)
    idx = torch.randint(0, cfg.vocab_size, (B, T), device="cuda", generator=gen)
    with torch.no_grad():
        for _ in range(warmup):
            model(idx)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            model(idx)
        torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1000.0 / steps
    n_params = sum(p.numel() for p in model.parameters())
    return {"tokens_per_s": B * T / (ms / 1000.0), "ms_per_forward": ms, "steps": steps,
            "config": (f"{config_name}: {'MAG transformer' if mag else 'Atlas LM'} {n_params / 1e6:.1f}M params, "
                       f"{cfg.n_layer} layers, d_model {cfg.n_embd}, {cfg.n_head} heads, "
                       + (f"attention window {cfg.window_size}, " if mag else "")
                       + f"B{B} T{T}, bf16 weights/activations, fp32 scan state, "
                       + ("layer-default random init" if mag else "random init N(0, 0.02)")
                       + ", synthetic token ids")}


def training_step(cfg, batch, steps, warmup, backward="hip", train_precision=None):
    """One memory layer's training step at the config's shape with `batch`
    rows: the differentiable memory_scan forward, then the backward of
    sum(y * c) + sum(final state) for a fixed random c into q, k, v, the four
    gates and the initial state (W1 ~ N(0, 1/D) rather than the model's
    W1 = 0, so that every gradient is non-trivial; W2 = [I;0], S = 0).
    backward="hip": the HIP forward and the library's atlas_scan_bwd --
    train_precision None / "f32": all fp32; "f16": the forward on fp16
    matrix cores keeping its chunk-start states, and Polar-Express and its
    VJP on fp16 matrix cores in the backward (everything else fp32);
    backward="torch": the inner gradient and Omega window as fp32 torch ops
    around the HIP fused-chunk operator and its custom VJP.  Returns
    layer-tokens/s (fwd+bwd)."""
    import torch
    from atlas_amd import DeepMemoryState, memory_scan
    from atlas_amd.autograd import hip_backward_supported
    c = dict(cfg, B=batch)
    if backward == "hip" and not hip_backward_supported(c["D"], c["E"], c["cs"], train_precision):
        backward = "torch"   # shapes the library backward is not built for
    q, k, v, gates = make_layer_inputs(c, torch.float32, seed=7)
    W1, W2, S1, S2 = initial_state(c)
    W1 = torch.randn_like(W1) / c["D"] ** 0.5
    leaves = [t.requires_grad_(True) for t in (q, k, v, *gates, W1, W2, S1, S2)]
    ct = torch.randn_like(q)

    def one():
        y, st = memory_scan(*leaves[:7], DeepMemoryState(*leaves[7:]), c["cs"], c["w"], c["ns"],
                            backward=backward, train_precision=train_precision)
        torch.autograd.grad((y * ct).sum() + sum(s.sum() for s in st), leaves)

    for _ in range(warmup):
        one()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        one()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1000.0 / steps
    return {"tokens_per_s": batch * c["T"] / (ms / 1000.0), "ms_per_step": ms, "steps": steps,
            "peak_mem_gib": torch.cuda.max_memory_allocated() / 2 ** 30,
            "workload": (f"1 memory layer, B{batch} T{c['T']} H{c['H']} D{c['D']} E{c['E']} cs{c['cs']} "
                         f"w{c['w']} ns{c['ns']}, {train_precision or 'f32'} Polar-Express arithmetic, "
                         f"{backward} backward (forward + "
                         "backward into q, k, v, gates and initial state; initial W1 ~ N(0, 1/D), "
                         "W2 = [I;0], S = 0)")}


def cpu_baseline(cfg, seconds):
    """Time the torch-CPU restatement of the reference's non-fused chunk loop
    (oracle/cpu_baseline.py) on a bounded sample of the same workload: one
    layer, all H heads, whole batch rows of T tokens (one row per call, the
    CPU path's fastest shape).  Protocol: one untimed warm-up row, then three
    timed repetitions of the same number of rows (sized so that the three
    take about `seconds` together); value = the median repetition's rate."""
    import statistics
    import torch
    from oracle import cpu_baseline as CB
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    T, H, D, E, cs, w, ns = cfg["T"], cfg["H"], cfg["D"], cfg["E"], cfg["cs"], cfg["w"], cfg["ns"]
    gen = torch.Generator().manual_seed(1)

    def inputs(rows, T):
        q = torch.randn(rows, T, H, D, generator=gen)
        q = q / q.norm(dim=-1, keepdim=True)
        k = torch.randn(rows, T, H, D, generator=gen)
        k = k / k.norm(dim=-1, keepdim=True)
        v = torch.randn(rows, T, H, D, generator=gen)
        gs = [torch.sigmoid(torch.randn(rows, T, H, generator=gen)) for _ in range(4)]
        gs[1] = gs[1] * 0.1
        W1 = torch.zeros(rows, H, D, E)
        W2 = torch.zeros(rows, H, E, D)
        W2[:, :, :D, :D] = torch.eye(D)
        return q, k, v, gs, (W1, W2, torch.zeros_like(W1), torch.zeros_like(W2))

    def run(rows, T):
        dt = 0.0
        for _ in range(rows):
            q, k, v, gs, st = inputs(1, T)
            t0 = time.perf_counter()
            CB.memory_scan(q, k, v, gs[0], gs[1], gs[2], gs[3], st, cs, w, ns)
            dt += time.perf_counter() - t0
        return dt

    t_row = run(1, T)                                 # warm-up (untimed) and size estimate
    rows = max(1, min(cfg["B"], int(seconds / 3 / max(t_row, 1e-3))))
    rates = [rows * T / run(rows, T) for _ in range(3)]
    med = statistics.median(rates)
    return {"value": med, "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"torch-CPU fp32 restatement of the reference non-fused JAX chunk loop; 1 layer, "
                      f"{rows} of {cfg['B']} batch rows (one per call) x {T} tokens x {H} heads per repetition; "
                      f"1 warm-up row, median of 3 repetitions ({', '.join(f'{r:.0f}' for r in rates)} tok/s); "
                      f"value = layer-tokens/s (each token through one memory layer, all heads)"}


def main():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--config", default="c2", choices=sorted(CONFIGS))
    ap.add_argument("--precision", default="f16", choices=["f16", "f32"])
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-model", action="store_true", help="skip the full-model forward measurement")
    ap.add_argument("--train-batch", type=int, default=8,
                    help="batch rows of the one-layer training-step measurement (0 = skip it)")
    ap.add_argument("--train-backward", default="hip", choices=["hip", "torch"],
                    help="training path of the one-layer training-step measurement")
    ap.add_argument("--train-precision", default="f16", choices=["f16", "f32"],
                    help="Polar-Express arithmetic of the training-step measurement (forward and backward)")
    ap.add_argument("--layers", type=int, default=0,
                    help="override the number of memory layers (profiling runs only; 0 = the config's)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run a 256 MiB device copy first (scales rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    ap.add_argument("--mfma-calibration", action="store_true",
                    help="only print the sustained matrix-core rate at 1, 2 and 4 waves per SIMD and exit")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build runs the scan on a single MI355X "
              f"(--gpus {args.gpus} requested). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch
    from atlas_amd import memory_scan
    from atlas_amd import _lib as L

    if args.mfma_calibration:
        for rep in range(2):
            for wps in (1, 2, 4):
                r = L.mfma_rate(wps)
                log(f"[bench] mfma calibration pass {rep + 1}, {wps} wave(s) per SIMD: {r:.0f} TFLOP/s "
                    f"({100 * r / PEAK_BF16_TFLOPS:.1f}% of {PEAK_BF16_TFLOPS})")
        return

    cfg = dict(CONFIGS[args.config])
    if args.layers > 0:
        cfg["layers"] = args.layers
    io_dtype = torch.float32 if args.precision == "f32" else torch.bfloat16
    B, T, H, D, E, cs, w, ns, layers = (cfg[k] for k in ("B", "T", "H", "D", "E", "cs", "w", "ns", "layers"))
    log(f"[bench] {cfg['workload']} precision={args.precision}")
    torch.cuda.init()
    data = [make_layer_inputs(cfg, io_dtype, seed=100 + i) for i in range(layers)]
    states = [initial_state(cfg) for _ in range(layers)]
    torch.cuda.synchronize()

    def step():
        for (q, k, v, gs), st in zip(data, states):
            memory_scan(q, k, v, gs[0], gs[1], gs[2], gs[3], st, cs, w, ns, precision=args.precision)

    if args.copy_calibration:
        # a plain device copy of known size, for scaling the FETCH_SIZE /
        # WRITE_SIZE counters of a rocprofv3 --pmc run of this command
        nbytes = 256 << 20
        src = torch.ones(nbytes // 4, device="cuda")
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"[bench] calibration copy: {nbytes} bytes read, {nbytes} bytes written")
        del src, dst

    for i in range(args.warmup):
        step()
        log(f"[bench] warmup step {i + 1}/{args.warmup} done")
    torch.cuda.synchronize()

    # Timed region (value): the K steps, nothing else enqueued.
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms = (t1 - t0) * 1000.0 / args.steps
    tokens = B * T * layers
    value = tokens / (ms / 1000.0)
    flops_step = flops_per_token_head(D, E, ns) * B * T * H * layers
    scan_frac = flops_step / (ms / 1000.0) / 1e12 / PEAK_BF16_TFLOPS
    log(f"[bench] timed {args.steps} steps: {ms:.2f} ms/step, {value:.4g} tok/s, "
        f"scan MFMA util {100 * scan_frac:.2f}% of bf16 peak")

    # Per-kernel durations: the same K steps again, with HIP events recorded
    # around every launch on the stream the kernels run on.
    lib = L.get_lib()
    L.check(lib.atlas_profile_enable(1))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step()
    torch.cuda.synchronize()
    ms_ev = (time.perf_counter() - t0) * 1000.0 / args.steps
    kern = {}
    for kind, name in ((0, "prep"), (1, "phase_w2"), (2, "phase_w1"), (4, "prefix"), (3, "finalize"),
                       (5, "prep_next+y")):
        try:
            n, tot = L.profile_read(kind)
        except L.AtlasError:
            n, tot = 0, 0.0   # kind unknown to this library build
        if n == 0 and kind == 5:
            continue   # no merged launches (slice prefix in use)
        kern[name] = {"launches": n, "avg_us": 1000.0 * tot / max(n, 1), "total_ms": tot}
    L.check(lib.atlas_profile_enable(0))
    log(f"[bench] kernels: " + ", ".join(f"{k} {v['avg_us']:.1f} us x{v['launches']}" for k, v in kern.items())
        + f" (event pass {ms_ev:.2f} ms/step, {100 * (ms_ev / ms - 1):+.1f}% vs the timed pass)")

    # dominant kernels: the two Polar-Express phases; each launch covers one
    # chunk of all B*H streams for one memory matrix.
    pe_flops_per_launch = B * H * cs * (ns * (4 * D * D * E + 2 * D ** 3) + 4 * D * E)
    avg_phase_s = 0.5 * (kern["phase_w2"]["avg_us"] + kern["phase_w1"]["avg_us"]) * 1e-6
    achieved = pe_flops_per_launch / avg_phase_s / 1e12
    traffic = measured_traffic(args.config, args.precision)
    # what the matrix cores sustain on this part for real data (pseudo-random
    # fp16 operands, power-limited clock), next to the datasheet peak
    attainable = L.mfma_rate(1)
    log(f"[bench] matrix-core calibration: {attainable:.0f} TFLOP/s sustained with random fp16 operands "
        f"({100 * attainable / PEAK_BF16_TFLOPS:.1f}% of the {PEAK_BF16_TFLOPS} datasheet peak)")

    model = None
    if not args.no_model and args.config in MODEL_CFGS and args.layers == 0:
        del data, states
        torch.cuda.empty_cache()
        model = model_forward(args.config, max(1, args.steps), max(1, args.warmup), args.precision)
        log(f"[bench] model forward: {model['ms_per_forward']:.2f} ms, {model['tokens_per_s']:.4g} tok/s")

    train = None
    if args.train_batch > 0 and args.layers == 0:
        torch.cuda.empty_cache()
        torch.cuda.reset_peak_memory_stats()
        train = training_step(cfg, args.train_batch, 3, 1, args.train_backward,
                              None if args.train_precision == "f32" else args.train_precision)
        if args.train_batch == B:   # the same rows as the forward: the step against one layer's forward
            train["vs_forward_layer"] = train["ms_per_step"] / (ms / layers)
            train["vs_forward_layer_definition"] = ("training step ms / (timed scan ms per step / layers), "
                                                    "both measured in this run")
        log(f"[bench] training step (1 layer): {train['ms_per_step']:.1f} ms, {train['tokens_per_s']:.4g} tok/s")

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(cfg, args.cpu_seconds)
        log(f"[bench] cpu baseline {cpu['value']:.4g} tok/s on {cpu['cores']} cores")

    out = {
        "metric": METRIC,
        "value": value,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16" if args.precision == "f16" else "f32",
        "data": "synthetic",
        "config": {"workload": cfg["workload"], "B": B, "T": T, "H": H, "D": D, "E": E, "chunk": cs,
                   "omega_window": w, "ns_steps": ns, "layers": layers,
                   "io": "bf16 q/k/v, fp32 gates and state" if args.precision == "f16" else "fp32",
                   "value_definition": "memory-layer tokens/s = B*T*layers / step time (a step = all layer scans)"},
        "scan_mfma_util_pct": 100.0 * scan_frac,
        "roofline": {"bound": "mfma", "achieved": achieved, "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": achieved / PEAK_BF16_TFLOPS, "traffic": traffic,
                     "kernel": "phase (Polar-Express) kernels, mean of the W2 and W1 phase launches",
                     "flops_per_launch": pe_flops_per_launch,
                     "timing": "HIP events around every launch on the kernels' stream, over a second pass "
                               "of the same K steps",
                     "attainable": attainable, "frac_of_attainable": achieved / attainable,
                     "attainable_definition": "dense fp16 32x32x16 MFMA chains with pseudo-random operands on "
                                              "every CU, measured in this run (atlas_profile_mfma_rate): the "
                                              "rate the part sustains under its power limit"},
        "kernels": kern,
        "model_forward": model,
        "training_layer": train,
        "cpu_baseline": cpu,
        "speedup_vs_cpu": (value / cpu["value"]) if cpu else None,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
