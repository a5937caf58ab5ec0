#!/usr/bin/env python3
"""Benchmark: the int8 W8A8 DiT linear stack, one Euler step per bench step.

Workload (the stack configuration, one GPU): 12 DiT blocks, hidden 1024,
MLP 2816, 3 CFG branches x 750 latent frames (M = 2250 rows).  Per block:
the modulation linear 1024 -> 6x1024 on the 3 conditioning rows, fused QKVG
1024 -> 4x1024, Wo 1024 -> 1024 with the gated residual, fused W1/W3
1024 -> 2x2816 with the SiLU gate, and W2 2816 -> 1024 on the two-term
requantized hidden state (the reference default) with the gated residual.
Every quantization, int8 GEMM and epilogue of the step runs on the GPU
through the C ABI; inputs and weights are resident in HBM before timing.
The fp32 attention core and RMSNorm-modulate are not part of the stack.

`--workload conv7` (T=24000, 512->512, kernel 7, padding 3) and
`--workload conv7-dil3` (T=6000, 1024->256, dilation 3, padding 9) measure
the codec's int8 Conv1d instead: one conv per step, same JSON line;
`--workload convt-stage0` / `convt-stage2` the decoder's int8 upsampling
ConvTranspose1d (stage 0: 750 frames, 1536->768, kernel 24, stride 12;
stage 2: 90000 frames, 384->192, kernel 16, stride 8).
`--workload adaln` the fp32 adaLN apply step of a DiT block on the same
M = 2250 rows (one call per step), `--workload qknorm` the per-head RMSNorm
and half-RoPE of q and k, `--workload attention` the attention core (scores,
softmax, P@V, gate) with a context of up to 300 rows, `--workload block` one
whole DiT block (adaLN parameters from cond, every fp32 and int8 step) at the
reference model's dimensions, `--workload sampler-step` one whole Euler step
of the sampler (12 such layers, heads, CFG / Euler update); `--workload weights` the int8 weight build
from a safetensors checkpoint.

Prints one JSON line on stdout; diagnostics go to stderr.
"""
import argparse
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
for sub in ("irodori-c_amd", "oracle"):
    sys.path.insert(0, os.path.join(REPO, sub))

import numpy as np  # noqa: E402

import iro_hip  # noqa: E402
from iro_synth import gauss  # noqa: E402

PEAK_INT8_TOPS = 5000.0  # MI355X dense int8 MFMA
PEAK_HBM_GBS = 8000.0

# HBM bytes per launch of each kernel kind at the M = 2250 step (the one the
# profiling steps run), from two rocprofv3 --pmc runs of this script
# (FETCH_SIZE, then WRITE_SIZE, per dispatch, separated by grid size),
# scaled by what the same counters read for a 64 MiB device copy
# (--copy-calibration 64: FETCH_SIZE x 1.999, WRITE_SIZE x 1.000); summary
# and commands in profiles/dit_stack_M2250_hbm_traffic.md.  Counters cannot
# be read from inside the process, so the figure is the last profile's.
MEASURED_TRAFFIC = {
    "gemm_swiglu": 74.9e6,
    "gemm_gated_two_term": 56.1e6,
    "gemm_qkvg": 60.2e6,
    "gemm_gated": 29.7e6,
    "quant_rows_residual": 38.2e6,
    "quant_rows": 11.6e6,
}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def stack_ops(blocks, B, S, D, H, rm):
    M = B * S
    per = (2 * B * D * 6 * D
           + 2 * M * D * 4 * D * (2 if rm & 1 else 1)
           + 2 * M * D * D * (2 if rm & 2 else 1)
           + 2 * M * D * 2 * H * (2 if rm & 4 else 1)
           + 2 * M * H * D * (2 if rm & 8 else 1))
    return blocks * per


def block_weights(base, b):
    """Block b's fp32 weights: the base draws with rows rotated by a
    block-dependent offset, so every block holds distinct matrices."""
    return [np.ascontiguousarray(np.roll(w, 97 * b + 13 * i, axis=0)) for i, w in enumerate(base)]


def base_weights(D, H, seed=1000):
    shapes = [(6 * D, D), (D, D), (D, D), (D, D), (D, D), (D, D), (H, D), (H, D), (D, H)]
    return [gauss(seed + i, s, 0.02) for i, s in enumerate(shapes)]


def cpu_topology(limit=16):
    """The host's CPU model, nproc, and the physical cores of the NUMA node of
    the first CPU this process may run on (one hardware thread per core,
    within the process's affinity, at most `limit`)."""
    allowed = sorted(os.sched_getaffinity(0))
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass

    def cpulist(text):
        out = []
        for part in text.strip().split(","):
            if "-" in part:
                a, b = part.split("-")
                out += range(int(a), int(b) + 1)
            elif part:
                out.append(int(part))
        return out

    node, node_cpus = 0, set(allowed)
    base = "/sys/devices/system/node"
    if os.path.isdir(base):
        for d in sorted(os.listdir(base)):
            if d.startswith("node") and d[4:].isdigit():
                try:
                    cpus = set(cpulist(open(os.path.join(base, d, "cpulist")).read()))
                except OSError:
                    continue
                if allowed[0] in cpus:
                    node, node_cpus = int(d[4:]), cpus
                    break
    cores, seen = [], set()
    for c in allowed:
        if c not in node_cpus:
            continue
        try:
            sib = open(f"/sys/devices/system/cpu/cpu{c}/topology/thread_siblings_list").read()
            key = min(cpulist(sib))
        except OSError:
            key = c
        if key not in seen:
            seen.add(key)
            cores.append(c)
    return {"cpu_model": model, "nproc": os.cpu_count(), "allowed_cpus": len(allowed),
            "numa_node": node, "physical_cores_used": cores[:limit]}


def _median_block_seconds(cpu, conv, wq, x0, cond, args, D, H, repeats=5):
    """One warm-up block, then the median wall time of `repeats` blocks, each
    from the same input rows (block-0 weights)."""
    times = []
    for i in range(repeats + 1):
        x = np.array(x0, copy=True)
        t0 = time.perf_counter()
        cpu.dit_block(conv, wq, x, cond, args.batch, args.frames, D, H, args.residual_mask)
        if i:
            times.append(time.perf_counter() - t0)
    return float(np.median(times)), times


def cpu_baseline(args, base, x0, cond, D, H, ops_per_step, x_gpu):
    """The reference's oneMKL int8 path on the host (oracle/cpu_baseline.c):
    one whole step of all blocks with the GPU's weights, compared bit for bit
    with the GPU's x; then the median of 5 blocks after a warm-up on all
    physical cores of one NUMA node (pinned) and on one pinned core, each
    scaled to a step."""
    from oracle import CpuBaseline, Oracle
    topo = cpu_topology()
    cores = topo["physical_cores_used"]
    saved = os.sched_getaffinity(0)
    conv = 0 if args.convention == "strict" else 1
    o = Oracle()
    try:
        os.sched_setaffinity(0, cores)
        cpu = CpuBaseline(len(cores))
        # parity at the bench's own configuration: every block's weights
        x = np.array(x0, copy=True)
        t0 = time.perf_counter()
        for b in range(args.blocks):
            wq = [o.weight_quantize(conv, w) for w in block_weights(base, b)]
            cpu.dit_block(conv, wq, x, cond, args.batch, args.frames, D, H, args.residual_mask)
        log(f"cpu baseline: full {args.blocks}-block step (parity) in "
            f"{time.perf_counter() - t0:.2f}s")
        if x_gpu is None:
            parity = {"status": "not compared"}
        else:
            ndiff = int(np.count_nonzero(x.view(np.int32) != x_gpu.view(np.int32)))
            parity = {"status": "bit-exact" if ndiff == 0 else "MISMATCH",
                      "elements_differing": ndiff, "elements": int(x.size),
                      "compared": f"x after one {args.blocks}-block step on the GPU (graph "
                                  f"replay) vs the host's step, {args.convention} rounding"}
        wq0 = [o.weight_quantize(conv, w) for w in block_weights(base, 0)]
        med_all, t_all = _median_block_seconds(cpu, conv, wq0, x0, cond, args, D, H)
        os.sched_setaffinity(0, cores[:1])
        cpu1 = CpuBaseline(1)
        med_one, t_one = _median_block_seconds(cpu1, conv, wq0, x0, cond, args, D, H)
    finally:
        os.sched_setaffinity(0, saved)
    step_all, step_one = med_all * args.blocks, med_one * args.blocks
    log(f"cpu baseline ({cpu.backend}): block median {med_all * 1e3:.1f} ms on {len(cores)} "
        f"cores, {med_one * 1e3:.1f} ms on 1 core; parity {parity['status']}")
    return {
        "value": round(ops_per_step / step_all / 1e12, 4),
        "unit": "TOPS",
        "cores": len(cores),
        "kind": "port",
        "ms_per_step": round(step_all * 1e3, 2),
        "one_core": {"value": round(ops_per_step / step_one / 1e12, 4), "unit": "TOPS",
                     "ms_per_step": round(step_one * 1e3, 2), "cores": 1},
        "backend": cpu.backend,
        **topo,
        "timing": "median of 5 DiT blocks after 1 warm-up (block-0 weights, same input rows), "
                  "x blocks; process pinned to the listed cores (sched_setaffinity)",
        "sample": (f"one DiT block of the {args.blocks}-block step at M={x0.shape[0]} (the "
                   f"modulation, QKVG, Wo, W1/W3 + SiLU, two-term W2 and both gated residuals), "
                   f"scaled x{args.blocks}; quantize/epilogue single-threaded as ops.c, GEMM on "
                   f"{len(cores)} MKL threads (and on 1)"),
        "parity": parity,
    }


CONV_WORKLOADS = {  # T, C_in, C_out, kernel, stride, dilation, padding
    "conv7": (24000, 512, 512, 7, 1, 1, 3),
    "conv7-dil3": (6000, 1024, 256, 7, 1, 3, 9),
}
# Decoder upsampling ConvTranspose1d (dacvae.c:150-160, 177-179) on 750
# latent frames: T_in, C_in, C_out, kernel, stride, padding, output_padding.
CONVT_WORKLOADS = {
    "convt-stage0": (750, 1536, 768, 24, 12, 6, 0),
    "convt-stage2": (90000, 384, 192, 16, 8, 4, 0),
}


def roofline_of(prof):
    """Dominant kernel kind (largest share of profiled time) against its
    roofline: int8 MFMA peak when it does MFMA work, else HBM."""
    if not prof:
        return None
    name, (n, kms, kops, kby) = max(prof.items(), key=lambda kv: kv[1][1])
    avg_ms = kms / n
    if kops:
        achieved = kops / n / (avg_ms * 1e-3) / 1e12
        return {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_INT8_TOPS,
                "unit": "TOPS", "frac": round(achieved / PEAK_INT8_TOPS, 4),
                "traffic": MEASURED_TRAFFIC.get(name), "kernel": name,
                "avg_us": round(avg_ms * 1e3, 2), "ops_per_launch": kops / n}
    achieved = kby / n / (avg_ms * 1e-3) / 1e9
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": MEASURED_TRAFFIC.get(name),
            "kernel": name, "avg_us": round(avg_ms * 1e3, 2), "bytes_per_launch": kby / n}


def log_profile(prof):
    total_ms = sum(v[1] for v in prof.values()) or 1.0
    for k, (n, kms, kops, kby) in sorted(prof.items(), key=lambda kv: -kv[1][1]):
        log(f"  {k:24s} launches {n:5d}  avg {kms / n * 1e3:8.2f} us  share {kms / total_ms:6.1%}  "
            f"{kops / kms / 1e9 if kops else 0:8.1f} TOPS  {kby / kms / 1e6:8.1f} GB/s")
    return {k: {"launches": v[0], "avg_us": round(v[1] / v[0] * 1e3, 2),
                "share": round(v[1] / total_ms, 4)} for k, v in prof.items()}


def conv_main(args):
    """The codec's int8 Conv1d (dacvae.c:543-688) at its measured shapes:
    one step = one conv (input ranges, quantized im2col, int8 GEMM with the
    bias epilogue) with input and weights resident in HBM."""
    T, Cin, N, k, st, dil, pad = CONV_WORKLOADS[args.workload]
    To = (T + 2 * pad - dil * (k - 1) - 1) // st + 1
    planes = 2 if args.conv_residual else 1
    ops = 2 * To * N * k * Cin * planes
    conv = iro_hip.STRICT if args.convention == "strict" else iro_hip.GCC_FASTMATH
    x = gauss(42, (T, Cin))
    w = gauss(43, (N, k * Cin), 0.02)
    b = gauss(44, (N,), 0.01)
    ctx = iro_hip.Context(0, conv)
    log("backend:", ctx.backend())
    wd = ctx.to_device(w)
    W = ctx.weight(wd, N, k * Cin)
    wd.free()
    xd, bd = ctx.to_device(x), ctx.to_device(b)
    y = ctx.empty((To, N), np.float32)

    def step():
        ctx.conv1d(xd, T, Cin, W, k, st, dil, pad, bd, args.conv_residual, y)

    for _ in range(args.warmup):
        step()
    ctx.sync()
    e0, e1 = ctx.event(), ctx.event()
    t0 = time.perf_counter()
    ctx.record(e0)
    for _ in range(args.steps):
        step()
    ctx.record(e1)
    ctx.sync()
    wall = time.perf_counter() - t0
    ev_ms = ctx.elapsed_ms(e0, e1)
    ms_step = wall * 1e3 / args.steps
    log(f"{args.workload}: {ms_step:.3f} ms/conv wall, {ev_ms / args.steps:.3f} ms/conv events")
    ctx.profile(True)
    for _ in range(args.profile_steps):
        step()
    prof = ctx.profile_read()
    ctx.profile(False)
    kernels = log_profile(prof)
    roof = roofline_of(prof)
    ygpu = y.numpy()
    ctx.close()

    cpu = None
    if not args.no_cpu_baseline:
        from oracle import CpuBaseline, Oracle
        threads = min(16, len(os.sched_getaffinity(0)))
        cb = CpuBaseline(threads)
        wq = Oracle().weight_quantize(0 if conv == iro_hip.STRICT else 1, w)
        times = []
        start = time.perf_counter()
        while len(times) < 5 and time.perf_counter() - start < args.cpu_seconds:
            t1 = time.perf_counter()
            ycpu, parts = cb.conv1d(0 if conv == iro_hip.STRICT else 1, x, *wq, k, st, dil, pad,
                                    bias=b, residual=args.conv_residual)
            times.append(time.perf_counter() - t1)
        med = sorted(times)[len(times) // 2]
        same = bool(np.array_equal(ycpu.view(np.uint32), ygpu.view(np.uint32)))
        log(f"cpu baseline: {len(times)} convs, median {med * 1e3:.1f} ms on {threads} threads "
            f"({cb.backend}); last: quantize {parts[0]:.3f}s gemm {parts[1]:.3f}s "
            f"epilogue {parts[2]:.3f}s; GPU output bit-identical: {same}")
        cpu = {"value": round(ops / med / 1e12, 4), "unit": "TOPS", "cores": threads,
               "kind": "port", "ms_per_step": round(med * 1e3, 2), "backend": cb.backend,
               "sample": (f"the full conv ({len(times)} runs, median): im2col quantization on one "
                          f"thread as dacvae.c, GEMM on {threads} threads, epilogue on one thread"),
               "gpu_output_bit_identical": same}

    out = {
        "metric": f"int8 Conv1d TOPS ({args.workload}), 1 GPU",
        "value": round(ops * args.steps / wall / 1e12, 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded Irwin-Hall Gaussian input, random-init weights)",
        "config": {"workload": (f"int8 Conv1d T={T}, {Cin}->{N}, kernel {k}, stride {st}, "
                                f"dilation {dil}, padding {pad}, {planes} plane(s), bias; one conv "
                                f"per step"),
                   "T": T, "c_in": Cin, "c_out": N, "kernel": k, "dilation": dil,
                   "padding": pad, "planes": planes, "ops_per_step": ops,
                   "convention": args.convention, "parallelism": "single GPU"},
        "roofline": roof,
        "kernels": kernels,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


def decoder_ops(p, frames, residual_mask=12, residual_stages=8):
    """Multiply-adds x2 of the int8 convolutions of the decoder core."""
    t = frames
    ops = 2 * t * p["channels"] * 7 * p["latent_channels"] * (2 if residual_mask & 1 else 1)
    for si, st in enumerate(p["stages"]):
        k, s_, pad, op = st["kernel"], st["stride"], st["padding"], st["output_padding"]
        ops += 2 * t * k * st["c_out"] * st["c_in"] * (2 if residual_mask & 2 else 1)
        t = (t - 1) * s_ - 2 * pad + k + op
        on = residual_stages >> si & 1
        C = st["c_out"]
        for _ in st["residual"]:
            ops += 2 * t * C * 7 * C * (2 if (residual_mask & 4) and on else 1)
            ops += 2 * t * C * C * (2 if (residual_mask & 8) and on else 1)
    return ops


def decoder_main(args):
    """The DACVAE decoder's int8 core (dacvae.c:1221-1277) at the reference's
    channel counts: one step = one decode of `frames` latent frames from the
    quantizer_out state (initial Conv7, four stages of snake + int8
    ConvTranspose and three residual units of snake, int8 Conv7, snake_bias
    and int8 1x1 onto the skip), state and weights resident in HBM."""
    sys.path.insert(0, os.path.join(REPO, "tests"))
    import codec_params as cp
    frames = args.decoder_frames
    conv = iro_hip.STRICT if args.convention == "strict" else iro_hip.GCC_FASTMATH
    p = cp.decoder(77)
    ops = decoder_ops(p, frames)
    state = np.random.default_rng(78).standard_normal((frames, cp.LATENT), dtype=np.float32)
    ctx = iro_hip.Context(0, conv)
    log("backend:", ctx.backend())
    d = iro_hip.DACVAE(ctx, cp.to_device(ctx, p))
    T = d.output_frames(frames)
    sd = ctx.to_device(state)
    out = ctx.empty((T, cp.FINAL), np.float32)

    def step():
        d.decode_int8(sd, frames, out)

    for _ in range(args.warmup):
        step()
    ctx.sync()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    ctx.sync()
    wall = time.perf_counter() - t0
    ms_step = wall * 1e3 / args.steps
    log(f"decoder: {frames} frames -> {T} x {cp.FINAL}: {ms_step:.3f} ms per decode")
    ctx.profile(True)
    for _ in range(args.profile_steps):
        step()
    prof = ctx.profile_read()
    ctx.profile(False)
    kernels = log_profile(prof)
    roof = roofline_of(prof)
    # parity and CPU baseline on a bounded sample of the same decode
    sf = min(frames, 2)
    small = ctx.empty((d.output_frames(sf), cp.FINAL), np.float32)
    d.decode_int8(ctx.to_device(state[:sf]), sf, small)
    g_small = small.numpy()
    int8_bytes = d.nbytes()
    d.destroy()
    ctx.close()
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import Oracle
        o = Oracle()
        times = []
        start = time.perf_counter()
        while len(times) < 3 and time.perf_counter() - start < args.cpu_seconds:
            t1 = time.perf_counter()
            want = o.decode_core(0 if conv == iro_hip.STRICT else 1, state[:sf], p)
            times.append(time.perf_counter() - t1)
        med = sorted(times)[len(times) // 2]
        same = bool(np.array_equal(want.view(np.uint32), g_small.view(np.uint32)))
        sops = decoder_ops(p, sf)
        log(f"cpu baseline: oracle decode of {sf} frames, median {med:.2f} s on {o.threads} "
            f"threads; GPU output bit-identical: {same}")
        cpu = {"value": round(sops / med / 1e12, 5), "unit": "TOPS", "cores": o.threads,
               "kind": "port", "sample": (f"the oracle's decoder core on {sf} of the {frames} "
                                          f"latent frames ({len(times)} runs, median)"),
               "gpu_output_bit_identical": same}
    out = {
        "metric": "int8 DACVAE decoder core TOPS and ms per decode, 1 GPU",
        "value": round(ops * args.steps / wall / 1e12, 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded Gaussian state, random-init weights at the decoder's shapes)",
        "config": {"workload": (f"DACVAE decoder int8 core: {frames} latent frames -> {T} "
                                f"samples x 96 channels, residual planes in stage 3"),
                   "frames": frames, "output_frames": T, "ops_per_step": ops,
                   "latent_frames_per_s": round(frames / (ms_step / 1e3), 1),
                   "resident_int8_bytes": int8_bytes, "convention": args.convention,
                   "parallelism": "single GPU"},
        "roofline": roof,
        "kernels": kernels,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


def adaln_main(args):
    """The adaLN apply step (dit.c:593-606) on the stack's rows: one step =
    one call of iro_hip_dit_adaln_apply on x [B*S, D] resident in HBM.  The
    per-row sum of squares is a serial chain of D dependent fp32 additions
    (bit-exact to the strict build), which bounds the kernel before HBM does;
    the roofline line still prices the algorithmic bytes (x read once, h
    written once) against HBM."""
    B, S, D = args.batch, args.frames, args.hidden
    M = B * S
    conv = iro_hip.STRICT if args.convention == "strict" else iro_hip.GCC_FASTMATH
    x = gauss(71, (M, D))
    shift, scale = gauss(72, (B, D), 0.3), gauss(73, (B, D), 0.3)
    eps = 1e-6
    ctx = iro_hip.Context(0, conv)
    log("backend:", ctx.backend())
    xd, shd, scd = ctx.to_device(x), ctx.to_device(shift), ctx.to_device(scale)
    h = ctx.empty((M, D), np.float32)

    def step():
        ctx.dit_adaln_apply(xd, B, S, D, shd, scd, eps, h)

    for _ in range(args.warmup):
        step()
    ctx.sync()
    e0, e1 = ctx.event(), ctx.event()
    t0 = time.perf_counter()
    ctx.record(e0)
    for _ in range(args.steps):
        step()
    ctx.record(e1)
    ctx.sync()
    wall = time.perf_counter() - t0
    ev_ms = ctx.elapsed_ms(e0, e1) / args.steps
    hgpu = h.numpy()
    ctx.close()
    alg_bytes = 8 * M * D + 8 * B * D
    achieved = alg_bytes / (ev_ms * 1e-3) / 1e9
    log(f"adaln: {wall * 1e3 / args.steps:.4f} ms/call wall, {ev_ms * 1e3:.2f} us/call events, "
        f"{achieved:.0f} GB/s")

    cpu = None
    if not args.no_cpu_baseline:
        from oracle import Oracle
        o = Oracle()
        times = []
        start = time.perf_counter()
        while len(times) < 20 and time.perf_counter() - start < args.cpu_seconds:
            t1 = time.perf_counter()
            hcpu = o.adaln_apply(x, shift, scale, B, S, eps)
            times.append(time.perf_counter() - t1)
        med = sorted(times)[len(times) // 2]
        same = bool(np.array_equal(hcpu.view(np.uint32), hgpu.view(np.uint32)))
        log(f"cpu baseline: {len(times)} calls, median {med * 1e3:.2f} ms; GPU output "
            f"bit-identical: {same}")
        cpu = {"value": round(M / med / 1e6, 4), "unit": "Mrows/s", "cores": 1, "kind": "port",
               "ms_per_step": round(med * 1e3, 3),
               "sample": f"the oracle's dit.c:593-606 restatement on all {M} rows "
                         f"({len(times)} calls, median), one thread",
               "gpu_output_bit_identical": same}
    out = {
        "metric": "adaLN apply rows/s (Mrows/s), 1 GPU",
        "value": round(M / (ev_ms * 1e-3) / 1e6, 2),
        "unit": "Mrows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ev_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded Irwin-Hall Gaussian x, shift, scale)",
        "config": {"workload": f"fp32 adaLN apply on {B} x {S} rows of {D}, one call per step",
                   "rows": M, "dim": D, "wall_ms_per_step": round(wall * 1e3 / args.steps, 5),
                   "convention": args.convention, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": None,
                     "note": (f"algorithmic bytes {alg_bytes} per launch (x read and h written "
                              f"once, shift/scale rows); the serial sum of {D} dependent fp32 "
                              f"additions per row bounds the kernel first")},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


def qknorm_main(args):
    """QK-norm + half-RoPE (dit.c:638-706) on the stack's q and k: one step =
    one call of iro_hip_dit_qk_norm_rope, in place on q, k [B*S, D] resident
    in HBM (x D/64 heads of 64).  Algorithmic bytes: q and k read and written
    once."""
    B, S, D = args.batch, args.frames, args.hidden
    M = B * S
    q, k = gauss(81, (M, D)), gauss(82, (M, D))
    qw, kw = gauss(83, (D,), 0.2) + 1.0, gauss(84, (D,), 0.2) + 1.0
    eps = 1e-6
    ctx = iro_hip.Context(0, iro_hip.STRICT)
    log("backend:", ctx.backend())
    qd, kd, qwd, kwd = ctx.to_device(q), ctx.to_device(k), ctx.to_device(qw), ctx.to_device(kw)
    ctx.dit_qk_norm_rope(qd, qwd, kd, kwd, B, S, D, eps)
    first_q, first_k = qd.numpy(), kd.numpy()
    for _ in range(args.warmup):
        ctx.dit_qk_norm_rope(qd, qwd, kd, kwd, B, S, D, eps)
    ctx.sync()
    e0, e1 = ctx.event(), ctx.event()
    t0 = time.perf_counter()
    ctx.record(e0)
    for _ in range(args.steps):
        ctx.dit_qk_norm_rope(qd, qwd, kd, kwd, B, S, D, eps)
    ctx.record(e1)
    ctx.sync()
    wall = time.perf_counter() - t0
    ev_ms = ctx.elapsed_ms(e0, e1) / args.steps
    ctx.close()
    alg_bytes = 16 * M * D + 8 * D + 256 * S
    achieved = alg_bytes / (ev_ms * 1e-3) / 1e9
    log(f"qknorm: {ev_ms * 1e3:.2f} us/call events, {achieved:.0f} GB/s")
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import Oracle
        o = Oracle()
        times = []
        start = time.perf_counter()
        while len(times) < 20 and time.perf_counter() - start < args.cpu_seconds:
            t1 = time.perf_counter()
            oq, ok = o.head_norm_rope(q, qw, k, kw, B, S, eps)
            times.append(time.perf_counter() - t1)
        med = sorted(times)[len(times) // 2]
        same = bool(np.array_equal(oq.view(np.uint32), first_q.view(np.uint32))
                    and np.array_equal(ok.view(np.uint32), first_k.view(np.uint32)))
        log(f"cpu baseline: {len(times)} calls, median {med * 1e3:.2f} ms; first GPU call "
            f"bit-identical: {same}")
        cpu = {"value": round(2 * M * D // 64 / med / 1e6, 4), "unit": "Mheads/s", "cores": 1,
               "kind": "port", "ms_per_step": round(med * 1e3, 3),
               "sample": f"the oracle's dit.c:638-706 restatement on all {M} rows of q and k "
                         f"({len(times)} calls, median, rotation table included), one thread",
               "gpu_output_bit_identical": same}
    out = {
        "metric": "QK-norm + half-RoPE head rows/s (Mheads/s), 1 GPU",
        "value": round(2 * M * D // 64 / (ev_ms * 1e-3) / 1e6, 2),
        "unit": "Mheads/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ev_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded Irwin-Hall Gaussian q, k and norm weights)",
        "config": {"workload": f"fp32 per-head RMSNorm + half-RoPE of q and k, {B} x {S} rows "
                               f"of {D} ({D // 64} heads of 64), in place, one call per step",
                   "rows": M, "dim": D, "wall_ms_per_step": round(wall * 1e3 / args.steps, 5),
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": None,
                     "note": f"algorithmic bytes {alg_bytes} per launch (q and k read and "
                             f"written once, norm weights, rotation table rows)"},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


def attention_main(args):
    """The attention core (dit.c:808-870) on the stack's rows: one step = one
    call of iro_hip_dit_attention on q, k, v, gate [B*S, D] resident in HBM
    and C = 300 context rows per batch, of which the masks keep 250, 150 and
    200 (joined keys 1000, 900, 950).  Every sum in the scalar build's order;
    priced against the fp32 vector ALU: 2 operations (a multiply and an add)
    per term of every score and every P@V output."""
    B, S, D, C = args.batch, args.frames, args.hidden, 300
    H = D // 64
    keep = [250, 150, 200] + [100] * max(0, B - 3)
    mask = np.zeros((B, C), np.uint8)
    for b in range(B):
        mask[b, :keep[b]] = 1
    q, k, v, gate = (gauss(91 + i, (B * S, D)) for i in range(4))
    ck, cv = gauss(95, (B * C, D)), gauss(96, (B * C, D))
    ctx = iro_hip.Context(0, iro_hip.STRICT)
    log("backend:", ctx.backend())
    actx = ctx.attn_context(mask, B)
    dev = [ctx.to_device(a) for a in (q, k, v, gate, ck, cv)]
    mix = ctx.empty((B * S, D), np.float32)

    def step():
        ctx.dit_attention(actx, dev[0], dev[1], dev[2], dev[3], B, S, D, dev[4], dev[5], mix)

    step()
    first = mix.numpy()
    for _ in range(args.warmup):
        step()
    ctx.sync()
    e0, e1 = ctx.event(), ctx.event()
    t0 = time.perf_counter()
    ctx.record(e0)
    for _ in range(args.steps):
        step()
    ctx.record(e1)
    ctx.sync()
    wall = time.perf_counter() - t0
    ev_ms = ctx.elapsed_ms(e0, e1) / args.steps
    actx.destroy()
    ctx.close()
    joined = [S + int(mask[b].sum()) for b in range(B)]
    flops = sum(2 * 2 * H * S * 64 * j for j in joined)  # scores + P@V, mul and add
    tflops = flops / (ev_ms * 1e-3) / 1e12
    log(f"attention: {ev_ms * 1e3:.1f} us/call events, {tflops:.1f} TFLOP/s (mul+add)")
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import Oracle
        o = Oracle()
        t1 = time.perf_counter()
        want = o.attention_core(q, k, v, gate, B, S, ck, cv, mask, B)
        dt = time.perf_counter() - t1
        same = bool(np.array_equal(want.view(np.uint32), first.view(np.uint32)))
        log(f"cpu baseline: {dt:.2f} s on {o.threads} threads; GPU output bit-identical: {same}")
        cpu = {"value": round(flops / dt / 1e12, 5), "unit": "TFLOP/s", "cores": o.threads,
               "kind": "port", "ms_per_step": round(dt * 1e3, 1),
               "sample": "the oracle's dit.c:808-870 restatement (scalar loops, OpenMP over "
                         "batch x head) on the whole call, once",
               "gpu_output_bit_identical": same}
    out = {
        "metric": "attention core TFLOP/s (fp32 multiply + add, scalar-build order), 1 GPU",
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ev_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded Irwin-Hall Gaussian q, k, v, gate, context rows)",
        "config": {"workload": f"fp32 attention core, {B} x {S} queries, {H} heads of 64, "
                               f"joined keys {joined}, one call per step",
                   "flops_per_step": flops, "wall_ms_per_step": round(wall * 1e3 / args.steps, 4),
                   "parallelism": "single GPU"},
        "roofline": {"bound": "valu", "achieved": round(tflops, 2), "peak": 157.3,
                     "unit": "TFLOP/s", "frac": round(tflops / 157.3, 4), "traffic": None,
                     "note": "peak is MI355X's fp32 vector figure (FMA counted twice, packed "
                             "math); the scalar build's order forbids both FMA and packed "
                             "pairs, so 78.6 is the reachable ceiling for separate multiply "
                             "and add"},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


def block_main(args):
    """One DiT block forward (dit.c:984-1040) at the reference model's
    dimensions (hidden 1280, 20 heads, MLP 3680, adaLN rank 192): one step =
    the adaLN parameters of both halves from cond (iro_hip_dit_adaln_params)
    and the block (iro_hip_dit_stack_block_forward) on 3 x 750 latent tokens
    with 300 context rows (masks keep 250, 150, 200).  Bit-identical to the
    reference's iro_dit_block (tests/test_gpu_dit_block.py).  The CPU
    baseline is the reference's own scalar build (oracle/_ref) on a bounded
    sample of the same block."""
    D, H, R, C = 1280, 3680, 192, 300
    B, S = args.batch, args.frames
    keep = [250, 150, 200] + [100] * max(0, B - 3)
    mask = np.zeros((B, C), np.uint8)
    for b in range(B):
        mask[b, :keep[b]] = 1
    ctx = iro_hip.Context(0, iro_hip.STRICT)
    log("backend:", ctx.backend())
    stack = iro_hip.DiTStack(ctx, 1, D, H, args.residual_mask)
    w = [gauss(100 + i, (D, D), 0.03) for i in range(5)]
    wn = [gauss(105, (D,), 0.2) + 1.0, gauss(106, (D,), 0.2) + 1.0]
    wm = [gauss(107, (H, D), 0.03), gauss(108, (H, D), 0.03), gauss(109, (D, H), 0.02)]
    ada = []
    for i in range(6):
        ada += [gauss(110 + 3 * i, (R, D), 0.05), gauss(111 + 3 * i, (D, R), 0.05),
                gauss(112 + 3 * i, (D,), 0.1)]
    wd = [ctx.to_device(a) for a in w + wn + wm]
    stack.set_block(0, ctx.to_device(np.zeros((6 * D, D), np.float32)), *wd[:5], *wd[7:])
    adad = [ctx.to_device(a) for a in ada]
    actx = ctx.attn_context(mask, B)
    x0 = gauss(120, (B * S, D))
    cond = ctx.to_device(gauss(121, (B, 3 * D), 0.5))
    ck, cv = ctx.to_device(gauss(122, (B * C, D))), ctx.to_device(gauss(123, (B * C, D)))
    ada_attn, ada_mlp = ctx.empty((3, B, D), np.float32), ctx.empty((3, B, D), np.float32)
    x = ctx.to_device(x0)

    def step():
        ctx.dit_adaln_params(cond, B, D, R, adad[:9], ada_attn)
        ctx.dit_adaln_params(cond, B, D, R, adad[9:], ada_mlp)
        stack.block_forward(0, x, B, S, ada_attn, ada_mlp, wd[5], wd[6], 1e-6, actx, ck, cv)

    for _ in range(args.warmup):
        step()
    ctx.sync()
    e0, e1 = ctx.event(), ctx.event()
    t0 = time.perf_counter()
    ctx.record(e0)
    for _ in range(args.steps):
        step()
    ctx.record(e1)
    ctx.sync()
    wall = time.perf_counter() - t0
    ev_ms = ctx.elapsed_ms(e0, e1) / args.steps
    actx.destroy()
    stack.destroy()
    ctx.close()
    rate = B * S / (ev_ms * 1e-3)
    log(f"block: {ev_ms:.3f} ms/block events, {rate:.0f} tokens/s")
    cpu = None
    ref_lib = os.path.join(REPO, "oracle", "_ref", "libref_strict.so")
    if not args.no_cpu_baseline and os.path.exists(ref_lib):
        from oracle import Reference
        ref = Reference("strict")
        Bs, Ss, Cs = 1, 256, 64
        ms = np.zeros((Bs, Cs), np.uint8)
        ms[0, :32] = 1
        xs, conds = gauss(124, (Bs * Ss, D)), gauss(125, (Bs, 3 * D), 0.5)
        cks, cvs = gauss(126, (Bs * Cs, D)), gauss(127, (Bs * Cs, D))
        t1 = time.perf_counter()
        ref.dit_block(xs, conds, ada, w + wn + wm, cks, cvs, ms, Bs, Ss, 1e-6, use_int8=True)
        dt = time.perf_counter() - t1
        log(f"cpu baseline: reference block at B={Bs} S={Ss} in {dt:.2f} s")
        cpu = {"value": round(Bs * Ss / dt, 2), "unit": "tokens/s", "cores": 1,
               "kind": "reference", "ms_per_step": round(dt * 1e3, 1),
               "sample": (f"the reference's iro_dit_block (scalar -O2 build, int8 weights "
                          f"quantized in the call) on {Bs} x {Ss} tokens with {Cs} context "
                          f"rows (32 kept), once, one thread")}
    out = {
        "metric": "DiT block forward tokens/s (hidden 1280, MLP 3680, 20 heads), 1 GPU",
        "value": round(rate, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ev_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32+int8",
        "data": "synthetic (seeded Irwin-Hall Gaussian activations and random-init weights)",
        "config": {"workload": f"one DiT block forward incl. adaLN parameters, {B} x {S} latent "
                               f"tokens, {C} context rows (kept {keep[:B]}), int8 QKVG/Wo/W1W3/W2",
                   "wall_ms_per_step": round(wall * 1e3 / args.steps, 4),
                   "residual_mask": args.residual_mask, "parallelism": "single GPU"},
        "roofline": None,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


def sampler_step_main(args):
    """One Euler step of the sampler (sampler.c:259-297) at the reference
    model's dimensions (12 layers, hidden 1280, 20 heads, MLP 3680, adaLN
    rank 192) through iro_hip_dit_sampler_step: input projection of the
    state [750, 32], broadcast to 3 CFG rows, every layer's adaLN parameters
    and block (300 shared context rows; masks keep 250, 150, 200), output
    head, CFG combine and Euler update.  Each layer holds distinct weights
    (shifted copies of one seeded set).  Bit-identical to the reference's
    step (tests/test_gpu_dit_step.py).  No CPU baseline: the reference's
    scalar build needs minutes for one step at this size (the block
    workload times it per block)."""
    D, H, R, C, L, LAT = 1280, 3680, 192, 300, args.blocks, 32
    B, S = min(args.batch, 3), args.frames
    keep = [250, 150, 200][:B]
    mask = np.zeros((B, C), np.uint8)
    for b in range(B):
        mask[b, :keep[b]] = 1
    ctx = iro_hip.Context(0, iro_hip.STRICT)
    log("backend:", ctx.backend())
    stack = iro_hip.DiTStack(ctx, L, D, H, args.residual_mask)
    w = [gauss(100 + i, (D, D), 0.03) for i in range(5)]
    wn = [gauss(105, (D,), 0.2) + 1.0, gauss(106, (D,), 0.2) + 1.0]
    wm = [gauss(107, (H, D), 0.03), gauss(108, (H, D), 0.03), gauss(109, (D, H), 0.02)]
    ada = []
    for i in range(6):
        ada += [gauss(110 + 3 * i, (R, D), 0.05), gauss(111 + 3 * i, (D, R), 0.05),
                gauss(112 + 3 * i, (D,), 0.1)]
    zeros = ctx.to_device(np.zeros((6 * D, D), np.float32))
    ck, cv = ctx.to_device(gauss(122, (C, D))), ctx.to_device(gauss(123, (C, D)))
    keepalive = []
    for l in range(L):
        wl = [ctx.to_device(np.roll(a, l, axis=-1)) for a in w + wn + wm]
        stack.set_block(l, zeros, *wl[:5], *wl[7:])
        adl = [ctx.to_device(np.roll(a, l, axis=-1)) for a in ada]
        stack.set_layer_f32(l, adl, wl[5], wl[6], ck, cv)
        keepalive += wl + adl
    head = [gauss(130, (D, LAT), 0.2), gauss(131, (D,), 0.1), gauss(132, (D,), 0.2) + 1.0,
            gauss(133, (LAT, D), 0.03), gauss(134, (LAT,), 0.1)]
    headd = [ctx.to_device(a) for a in head]
    stack.set_head(*headd, LAT, R, 1e-6)
    actx = ctx.attn_context(mask, 1)
    cond = ctx.to_device(np.repeat(gauss(121, (1, 3 * D), 0.5), B, axis=0))
    state = ctx.to_device(gauss(120, (S, LAT)))
    vel = ctx.empty((B * S, LAT), np.float32)
    rows = (1, 2 if B > 2 else -1, -1) if B > 1 else (-1, -1, -1)
    scales = (1.5, 0.75 if B > 2 else 0.0, 0.0)

    def step():
        stack.sampler_step(state, cond, B, S, actx, B > 1, rows, scales, -1.0 / 8, vel)

    for _ in range(args.warmup):
        step()
    ctx.sync()
    e0, e1 = ctx.event(), ctx.event()
    t0 = time.perf_counter()
    ctx.record(e0)
    for _ in range(args.steps):
        step()
    ctx.record(e1)
    ctx.sync()
    wall = time.perf_counter() - t0
    ev_ms = ctx.elapsed_ms(e0, e1) / args.steps
    finite = bool(np.isfinite(state.numpy()).all())
    ctx.profile(True)
    for _ in range(args.profile_steps):
        step()
    prof = ctx.profile_read()
    ctx.profile(False)
    kernels = log_profile(prof)
    actx.destroy()
    stack.destroy()
    ctx.close()
    rate = B * S / (ev_ms * 1e-3)
    log(f"sampler step: {ev_ms:.3f} ms/step events, {rate:.0f} tokens/s")
    out = {
        "metric": "Euler sampler step latency (ms) and tokens/s, DiT hidden 1280 x 12 layers, 1 GPU",
        "value": round(rate, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ev_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32+int8",
        "data": "synthetic (seeded Irwin-Hall Gaussian activations and random-init weights)",
        "config": {"workload": f"one Euler sampler step: input projection, {L} DiT layers "
                               f"(adaLN parameters + block), output head, CFG / Euler update; "
                               f"{B} CFG rows x {S} latent frames, {C} shared context rows "
                               f"(kept {keep}), int8 QKVG/Wo/W1W3/W2",
                   "wall_ms_per_step": round(wall * 1e3 / args.steps, 4),
                   "residual_mask": args.residual_mask, "parallelism": "single GPU"},
        "roofline": None,
        "kernels": kernels,
        "cpu_baseline": None,
        "state_finite": finite,
    }
    print(json.dumps(out), flush=True)


def weights_main(args):
    """The weight source (safetensors.c:302-530, generate.c:526-544): one step
    = the int8 weights of one DiT block (modulation, Wq/Wk/Wv/Wgate, Wo, W1,
    W3, W2) built from an fp32 safetensors checkpoint (mmap, upload,
    quantization and packing), and the same weights read back from their
    packed files.  Host-to-device copies are inside the timing: this path
    starts from a file."""
    import tempfile
    from safetensors.numpy import save_file
    D, H = args.hidden, args.mlp
    shapes = {"ada": (6 * D, D), "wq": (D, D), "wk": (D, D), "wv": (D, D), "wgate": (D, D),
              "wo": (D, D), "w1": (H, D), "w3": (H, D), "w2": (D, H)}
    tensors = {f"blocks.0.{k}.weight": gauss(60 + i, s, 0.02)
               for i, (k, s) in enumerate(shapes.items())}
    src_bytes = sum(a.nbytes for a in tensors.values())
    conv = iro_hip.STRICT if args.convention == "strict" else iro_hip.GCC_FASTMATH
    ctx = iro_hip.Context(0, conv)
    log("backend:", ctx.backend())
    with tempfile.TemporaryDirectory() as tmp:
        path = os.path.join(tmp, "block.safetensors")
        save_file(tensors, path)
        st = iro_hip.Safetensors(path)

        def build():
            ws = [ctx.weight_from_st(st, n) for n in tensors]
            ctx.sync()
            return ws

        for _ in range(args.warmup):
            for w in build():
                w.destroy()
        times, ws = [], []
        for _ in range(args.steps):
            t0 = time.perf_counter()
            ws = build()
            times.append(time.perf_counter() - t0)
            if len(times) < args.steps:
                for w in ws:
                    w.destroy()
        files = [os.path.join(tmp, f"w{i}.iro8") for i in range(len(ws))]
        for w, f in zip(ws, files):
            ctx.weight_save(w, f)
        packed_bytes = sum(os.path.getsize(f) for f in files)
        ltimes = []
        for _ in range(args.steps):
            t0 = time.perf_counter()
            ls = [ctx.weight_load(f) for f in files]
            ctx.sync()
            ltimes.append(time.perf_counter() - t0)
            same = all(np.array_equal(a.export()[0], b.export()[0]) for a, b in zip(ls, ws))
            for w in ls:
                w.destroy()
        st.close()
    med, lmed = sorted(times)[len(times) // 2], sorted(ltimes)[len(ltimes) // 2]
    log(f"weights: build {med * 1e3:.1f} ms/block ({src_bytes / med / 1e9:.2f} GB/s of fp32), "
        f"packed-file load {lmed * 1e3:.1f} ms/block; reloaded codes identical: {same}")
    ctx.close()

    cpu = None
    if not args.no_cpu_baseline:
        from oracle import Oracle
        o = Oracle()
        c = 0 if conv == iro_hip.STRICT else 1
        t0 = time.perf_counter()
        for a in tensors.values():
            o.weight_quantize(c, a)
        dt = time.perf_counter() - t0
        cpu = {"value": round(src_bytes / dt / 1e9, 3), "unit": "GB/s", "cores": 1,
               "kind": "port", "ms_per_step": round(dt * 1e3, 1),
               "sample": "the oracle's iro_int8_weight_quantize restatement (ops.c:259-293) on "
                         "the block's nine fp32 tensors, one thread, packing not included"}
    out = {
        "metric": "int8 weight build from a safetensors checkpoint (GB/s of fp32 source), 1 GPU",
        "value": round(src_bytes / med / 1e9, 3),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(med * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32->int8",
        "data": "synthetic (seeded Irwin-Hall Gaussian weights written with safetensors.numpy)",
        "config": {"workload": f"one DiT block's int8 weights (hidden {D}, MLP {H}) from fp32 "
                               f"safetensors: mmap, upload, quantize, pack",
                   "fp32_bytes": src_bytes, "packed_file_bytes": packed_bytes,
                   "packed_file_load_ms": round(lmed * 1e3, 3),
                   "convention": args.convention, "parallelism": "single GPU"},
        "roofline": None,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


def convt_main(args):
    """The codec's int8 ConvTranspose1d (dacvae.c:696-795, no snake): one step
    = row quantization, the GEMM to the expanded taps and the ordered
    gather-add with bias, input and weights resident in HBM."""
    T, Cin, Co, k, st, pad, opad = CONVT_WORKLOADS[args.workload]
    To = (T - 1) * st - 2 * pad + k + opad
    planes = 2 if args.conv_residual else 1
    ops = 2 * T * k * Co * Cin * planes
    conv = iro_hip.STRICT if args.convention == "strict" else iro_hip.GCC_FASTMATH
    x = gauss(42, (T, Cin))
    w = gauss(43, (Cin, k * Co), 0.02)  # [C_in, kernel, C_out] export layout
    b = gauss(44, (Co,), 0.01)
    ctx = iro_hip.Context(0, conv)
    log("backend:", ctx.backend())
    wd = ctx.to_device(w)
    W = ctx.weight(wd, k * Co, Cin, transposed=True)
    wd.free()
    xd, bd = ctx.to_device(x), ctx.to_device(b)
    y = ctx.empty((To, Co), np.float32)

    def step():
        ctx.convtranspose1d(xd, T, Cin, W, Co, k, st, pad, opad, bd, args.conv_residual, y)

    for _ in range(args.warmup):
        step()
    ctx.sync()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    ctx.sync()
    wall = time.perf_counter() - t0
    ms_step = wall * 1e3 / args.steps
    log(f"{args.workload}: {ms_step:.3f} ms/step wall")
    ctx.profile(True)
    for _ in range(args.profile_steps):
        step()
    prof = ctx.profile_read()
    ctx.profile(False)
    kernels = log_profile(prof)
    roof = roofline_of(prof)
    ygpu = y.numpy()
    ctx.close()

    cpu = None
    if not args.no_cpu_baseline:
        from oracle import Oracle
        threads = min(16, len(os.sched_getaffinity(0)))
        o = Oracle()
        o.threads = threads
        cv = 0 if conv == iro_hip.STRICT else 1
        wq = o.weight_quantize_transposed(cv, w, k * Co, Cin)
        # Bounded sample: the first rows of the input (the work is linear in
        # T_in), timed as the oracle's restatement with its OpenMP GEMM.
        Ts = T
        while 2.0 * Ts * k * Co * Cin * planes > 40e9 and Ts > 16:
            Ts //= 2
        xs = np.ascontiguousarray(x[:Ts])
        t1 = time.perf_counter()
        ycpu = o.convtranspose1d(cv, xs, *wq, Co, k, st, pad, opad, bias=b,
                                 residual=args.conv_residual)
        sec = time.perf_counter() - t1
        Tso = (Ts - 1) * st - 2 * pad + k + opad
        # Rows the sample's last input row does not finish differ only in
        # the missing contributions; compare the rows it completes.
        full = max(0, (Ts - 1) * st - pad)
        same = bool(np.array_equal(ycpu[:full].view(np.uint32), ygpu[:full].view(np.uint32)))
        sops = 2.0 * Ts * k * Co * Cin * planes
        log(f"cpu baseline: T_in sample {Ts} ({sops / 1e9:.1f} GOP) in {sec:.2f}s on {threads} "
            f"threads (oracle restatement); completed rows bit-identical to the GPU: {same}")
        cpu = {"value": round(sops / sec / 1e12, 4), "unit": "TOPS", "cores": threads,
               "kind": "port", "ms_per_step": round(sec * ops / sops * 1e3, 2),
               "sample": (f"the first {Ts} of {T} input rows ({Tso} output rows), oracle "
                          f"restatement with its OpenMP GEMM on {threads} threads, scaled by work"),
               "gpu_output_bit_identical": same}

    out = {
        "metric": f"int8 ConvTranspose1d TOPS ({args.workload}), 1 GPU",
        "value": round(ops * args.steps / wall / 1e12, 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded Irwin-Hall Gaussian input, random-init weights)",
        "config": {"workload": (f"int8 ConvTranspose1d T_in={T}, {Cin}->{Co}, kernel {k}, stride "
                                f"{st}, padding {pad}, output_padding {opad}, {planes} plane(s), "
                                f"bias; one layer per step"),
                   "T_in": T, "T_out": To, "c_in": Cin, "c_out": Co, "kernel": k, "stride": st,
                   "planes": planes, "ops_per_step": ops, "convention": args.convention,
                   "parallelism": "single GPU"},
        "roofline": roof,
        "kernels": kernels,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


def vendor_gemm_main(args):
    """The vendor library's int8 GEMM beside this library's fused kernels at
    the same shapes: hipBLASLt through torch._int_mm (s8 x s8 -> s32, no
    dequantization, activation, quantization or fp32 store; B given
    row-major and column-major, the faster counted) against the event
    profiler's mean launch time of the stack's four GEMM kinds (an eagerly
    launched step at M = 2250 and at M = 750, D = 1024, H = 2816) and of
    the kernel-7 Conv1d's GEMM (T = 24000, 512 -> 512).  The two-term W2
    runs two activation planes per launch; the vendor figure for it is two
    single-plane calls.  A reference point for what the hardware and its
    library reach at these sizes, not a parity check."""
    import torch
    D, H, blocks = args.hidden, args.mlp, 2
    base = base_weights(D, H)
    ctx = iro_hip.Context(0, iro_hip.STRICT)
    log("backend:", ctx.backend())
    stack = iro_hip.DiTStack(ctx, blocks, D, H, args.residual_mask)
    for b in range(blocks):
        dev = [ctx.to_device(w) for w in block_weights(base, b)]
        stack.set_block(b, *dev)
        for a in dev:
            a.free()
    ours = {}
    for B in (3, 1):
        M = B * args.frames
        xd = ctx.to_device(gauss(7, (M, D)))
        cd = ctx.to_device(gauss(8, (B, D), 0.1))
        for _ in range(2):
            stack.step(xd, cd, B, args.frames)
        ctx.sync()
        ctx.profile(True)
        ctx.profile_reset()
        for _ in range(3):
            stack.step(xd, cd, B, args.frames)
        prof = ctx.profile_read()
        ctx.profile(False)
        for kind, (n_, ms, _ops, _by) in prof.items():
            ours[(M, kind)] = ms * 1e3 / n_
    T, Cin, N, k, st, dil, pad = CONV_WORKLOADS["conv7"]
    W = ctx.weight(ctx.to_device(gauss(43, (N, k * Cin), 0.02)), N, k * Cin)
    xc, bc = ctx.to_device(gauss(42, (T, Cin))), ctx.to_device(gauss(44, (N,), 0.01))
    yc = ctx.empty((T, N), np.float32)
    for _ in range(2):
        ctx.conv1d(xc, T, Cin, W, k, st, dil, pad, bc, False, yc)
    ctx.sync()
    ctx.profile(True)
    ctx.profile_reset()
    for _ in range(5):
        ctx.conv1d(xc, T, Cin, W, k, st, dil, pad, bc, False, yc)
    prof = ctx.profile_read()
    ctx.profile(False)
    ours[(T, "conv7")] = prof["gemm_linear"][1] * 1e3 / prof["gemm_linear"][0]
    ctx.close()

    def vendor_us(M, K, N):
        a = torch.randint(-128, 127, (M, K), dtype=torch.int8, device="cuda")
        b = torch.randint(-128, 127, (K, N), dtype=torch.int8, device="cuda")
        best = None
        for bb in (b, b.t().contiguous().t()):
            torch._int_mm(a, bb)
            torch.cuda.synchronize()
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(args.steps):
                torch._int_mm(a, bb)
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / args.steps
            best = us if best is None else min(best, us)
        return best

    rows = []
    for M in (3 * args.frames, args.frames):
        for name, kind, K, Nn, planes in (("QKVG", "gemm_qkvg", D, 4 * D, 1),
                                          ("Wo + gated residual", "gemm_gated", D, D, 1),
                                          ("W1/W3 + SiLU gate", "gemm_swiglu", D, 2 * H, 1),
                                          ("W2 two-term + gated residual", "gemm_gated_two_term",
                                           H, D, 2)):
            rows.append((f"{name}, M={M}", M, K, Nn, planes, ours[(M, kind)],
                         planes * vendor_us(M, K, Nn)))
    rows.append(("Conv1d k7 GEMM + bias, T=24000", T, k * Cin, N, 1, ours[(T, "conv7")],
                 vendor_us(T, k * Cin, N)))
    shapes = []
    for name, M, K, Nn, planes, o, v in rows:
        ops = 2.0 * M * K * Nn * planes
        log(f"{name:38s} ours {o:8.2f} us ({ops / o / 1e6:7.1f} TOPS)   "
            f"hipBLASLt {v:8.2f} us ({ops / v / 1e6:7.1f} TOPS)")
        shapes.append({"gemm": name, "M": M, "K": K, "N": Nn, "planes": planes,
                       "ours_us": round(o, 2), "ours_tops": round(ops / o / 1e6, 1),
                       "vendor_us": round(v, 2), "vendor_tops": round(ops / v / 1e6, 1)})
    ratio = sum(r[6] for r in rows) / sum(r[5] for r in rows)
    sq = vendor_us(8192, 8192, 8192)
    sq_tops = 2.0 * 8192 ** 3 / sq / 1e6
    log(f"hipBLASLt 8192 x 8192 x 8192: {sq:.1f} us ({sq_tops:.1f} TOPS, "
        f"{sq_tops / PEAK_INT8_TOPS:.3f} of peak)")
    out = {
        "metric": "int8 GEMM time at the stack's and the Conv1d's shapes: vendor library "
                  "(hipBLASLt, s32 output, no epilogue) time / this library's fused kernels' time",
        "value": round(ratio, 3), "unit": "x", "n_gpus": 1, "steps": args.steps,
        "higher_is_better": True, "dtype": "int8", "data": "synthetic",
        "config": {"workload": "vendor int8 GEMM comparison", "parallelism": "single GPU"},
        "shapes": shapes,
        "vendor_square_8192": {"us": round(sq, 1), "tops": round(sq_tops, 1),
                               "frac_of_peak": round(sq_tops / PEAK_INT8_TOPS, 3)},
    }
    print(json.dumps(out), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--convention", choices=["strict", "fastmath"], default="strict")
    ap.add_argument("--blocks", type=int, default=12)
    ap.add_argument("--batch", type=int, default=3)
    ap.add_argument("--frames", type=int, default=750)
    ap.add_argument("--hidden", type=int, default=1024)
    ap.add_argument("--mlp", type=int, default=2816)
    ap.add_argument("--residual-mask", type=int, default=8)
    ap.add_argument("--profile-steps", type=int, default=3)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--workload", choices=["stack", "weights", "adaln", "qknorm", "attention",
                                           "block", "sampler-step", "decoder", "vendor-gemm"]
                    + sorted(CONV_WORKLOADS)
                    + sorted(CONVT_WORKLOADS),
                    default="stack",
                    help="stack (default): the DiT linear stack; conv7*: the codec int8 Conv1d; "
                         "convt-*: the codec int8 ConvTranspose1d")
    ap.add_argument("--decoder-frames", type=int, default=250,
                    help="decoder workload: latent frames per decode (1920 samples each)")
    ap.add_argument("--conv-residual", action="store_true",
                    help="conv workloads: add the fixed-scale second plane")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run three device-to-device copies of MIB MiB (the known-size "
                         "copy that scales rocprofv3 FETCH_SIZE / WRITE_SIZE) and exit")
    args = ap.parse_args()

    if args.copy_calibration > 0:
        ctx = iro_hip.Context(0, iro_hip.STRICT)
        n = args.copy_calibration << 18  # float32 elements
        a, b = ctx.empty(n, np.float32), ctx.empty(n, np.float32)
        ctx.fill(a, 1)
        for _ in range(3):
            ctx.copy(b, a)
        ctx.sync()
        log(f"copied {args.copy_calibration} MiB x3")
        ctx.close()
        return

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(--gpus must be 1)", file=sys.stderr)
        sys.exit(2)
    if args.workload in CONV_WORKLOADS:
        conv_main(args)
        return
    if args.workload in CONVT_WORKLOADS:
        convt_main(args)
        return
    if args.workload == "weights":
        weights_main(args)
        return
    if args.workload == "adaln":
        adaln_main(args)
        return
    if args.workload == "decoder":
        decoder_main(args)
        return
    if args.workload == "qknorm":
        qknorm_main(args)
        return
    if args.workload == "attention":
        attention_main(args)
        return
    if args.workload == "sampler-step":
        return sampler_step_main(args)
    if args.workload == "block":
        block_main(args)
        return
    if args.workload == "vendor-gemm":
        vendor_gemm_main(args)
        return

    B, S, D, H = args.batch, args.frames, args.hidden, args.mlp
    M = B * S
    rm = args.residual_mask
    ops = stack_ops(args.blocks, B, S, D, H, rm)
    conv = iro_hip.STRICT if args.convention == "strict" else iro_hip.GCC_FASTMATH

    base = base_weights(D, H)
    x0 = gauss(7, (M, D))
    cond = gauss(8, (B, D), 0.1)

    ctx = iro_hip.Context(0, conv)
    log("backend:", ctx.backend())
    stack = iro_hip.DiTStack(ctx, args.blocks, D, H, rm)
    for b in range(args.blocks):
        dev = [ctx.to_device(w) for w in block_weights(base, b)]
        stack.set_block(b, *dev)
        for a in dev:
            a.free()
    ctx._arrays = [a for a in ctx._arrays if a.ptr]
    x_init = ctx.to_device(x0)
    x = ctx.to_device(x0)
    c = ctx.to_device(cond)

    # Each step starts from the same hidden state, as each Euler step's
    # blocks start from the input projection of the current latent
    # (dit.c:532); the 9 MB device copy is inside the timed region.
    def step():
        ctx.copy(x, x_init)
        stack.step(x, c, B, S)

    for _ in range(args.warmup):
        step()
    ctx.sync()
    e0, e1 = ctx.event(), ctx.event()
    t0 = time.perf_counter()
    ctx.record(e0)
    for _ in range(args.steps):
        step()
    ctx.record(e1)
    ctx.sync()
    wall = time.perf_counter() - t0
    ev_ms = ctx.elapsed_ms(e0, e1)
    ms_step = wall * 1e3 / args.steps
    finite = bool(np.isfinite(x.numpy()).all())
    log(f"stack: {ms_step:.3f} ms/step wall, {ev_ms / args.steps:.3f} ms/step events, "
        f"x finite: {finite}")

    # The reference sampler's schedule (sampler.c:247-250): CFG steps run the
    # B branches, plain steps (t below the CFG window) one branch of S rows.
    # Each shape keeps its own captured graph.
    x1_init = ctx.to_device(x0[:S])
    x1 = ctx.to_device(x0[:S])
    c1 = ctx.to_device(cond[:1])

    def step1():
        ctx.copy(x1, x1_init)
        stack.step(x1, c1, 1, S)

    for _ in range(args.warmup):
        step1()
    ctx.sync()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step1()
    ctx.sync()
    ms_b1 = (time.perf_counter() - t0) * 1e3 / args.steps
    ops_b1 = stack_ops(args.blocks, 1, S, D, H, rm)
    reps = max(1, args.steps // 4)
    for _ in range(4):
        step()
    for _ in range(4):
        step1()
    ctx.sync()
    t0 = time.perf_counter()
    for _ in range(reps):
        for _ in range(4):
            step()
        for _ in range(4):
            step1()
    ctx.sync()
    ms_sched = (time.perf_counter() - t0) * 1e3 / reps
    schedule = {
        "m_cfg_rows": M, "m_cfg_ms_per_step": round(ms_step, 4),
        "m_plain_rows": S, "m_plain_ms_per_step": round(ms_b1, 4),
        "m_plain_tops": round(ops_b1 / ms_b1 / 1e9, 2),
        "eight_step_ms": round(ms_sched, 4),
        "eight_step_tops": round((4 * ops + 4 * ops_b1) / ms_sched / 1e9, 2),
        "note": ("4 CFG steps at M=B*S then 4 plain steps at M=S, as the reference "
                 "sampler's default CFG window gives (sampler.c:247-250); graph replay"),
    }
    log(f"schedule: plain M={S} {ms_b1:.3f} ms/step, 8 steps {ms_sched:.3f} ms")

    # Per-kernel durations on the stack's stream (HIP events), after the
    # timed region.
    ctx.profile(True)
    for _ in range(args.profile_steps):
        step()
    prof = ctx.profile_read()
    ctx.profile(False)
    kernels = log_profile(prof)
    roof = roofline_of(prof)
    stack_bytes = stack.nbytes()
    # x after one step (the profiled steps restart from x_init too)
    x_gpu = x.numpy()
    stack.destroy()
    ctx.close()

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(args, base, x0, cond, D, H, ops, x_gpu)

    value = ops * args.steps / wall / 1e12
    out = {
        "metric": "int8 DiT linear TOPS + % of int8 MFMA peak; Euler-step latency (ms), 1 GPU",
        "value": round(value, 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded Irwin-Hall Gaussian inputs, random-init weights)",
        "config": {
            "workload": (f"int8 DiT linear stack: {args.blocks} blocks, hidden {D}, MLP {H}, "
                         f"M={B}x{S} rows, modulation 1024->6x1024 at M={B}, W2 two-term "
                         f"(residual mask {rm}), one Euler step per step"),
            "blocks": args.blocks, "batch": B, "frames": S, "hidden": D, "mlp": H,
            "convention": args.convention, "ops_per_step": ops,
            "frac_of_peak_stack": round(value / PEAK_INT8_TOPS, 4),
            "resident_int8_bytes": stack_bytes, "parallelism": "single GPU",
        },
        "roofline": roof,
        "schedule": schedule,
        "kernels": kernels,
        "kernels_source": ("per-kernel HIP events around each launch of directly launched "
                           "(not graph-replayed) steps after the timed region"),
        "cpu_baseline": cpu,
        "parity": cpu["parity"]["status"] if cpu else "not compared (--no-cpu-baseline)",
        "x_finite": finite,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
