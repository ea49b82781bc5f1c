#!/usr/bin/env python3
"""Benchmark of the fused spectral-SSM layer (GatedCSSM) on one MI355X.

Workload ("C2"): gated cell, fp32, batch 128 of one
128x128x64 image repeated over T = 8 frames (materialised; the kernels do not
see the repetition), x ~ N(0, 1), kernel_size 11, factored B/C/Delta gates,
softplus Delta, no short convolutions, random-init weights (synthetic data).

A step is one full layer forward, x -> out (in_proj GEMM with the plane-major
split + SiLU + spatial-mean epilogue -> gate planes -> fused rfft2 / scan /
irfft2 / x SiLU(z) kernel -> out_proj GEMM), with x already in HBM.
value = frames/s = B * T / step time.  The roofline entry is for the fused
scan kernel (the dominant kernel), timed with HIP events on its stream inside
the timed steps; its algorithmic bytes per launch are
B*T*(3*H*W*C*4 + 3*(H+W/2+1)*4) + C*H*(W/2+1)*8 (read u and z, write y, read
the factored gate vectors and K_hat once).  cpu_baseline times the float64
numpy restatement (oracle/) of the same layer on a bounded slice of the
batch, on one host thread.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

WORKLOAD = dict(name="C2 gated 128x128 T=8", B=128, T=8, H=128, W=128, C=64, kernel_size=11,
                gate_type="factored", gate_activation="softplus")
HBM_PEAK_GBS = 8000.0


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--batch", type=int, default=WORKLOAD["B"], help="override B (parity/debug runs only)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="target CPU baseline wall time")
    ap.add_argument("--traffic", default=os.path.join(ROOT, "profiles", "gated_scan_c2_traffic.txt"),
                    help="rocprofv3 FETCH/WRITE summary giving HBM bytes per scan launch")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="BYTES",
                    help="first run one device-to-device copy of BYTES (a known-size kernel that scales "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE counters); not timed")
    return ap.parse_args()


def scan_algorithmic_bytes(B, T, H, W, C):
    Wf = W // 2 + 1
    return B * T * (3 * H * W * C * 4 + 3 * (H + Wf) * 4) + C * H * Wf * 8


def read_traffic(path):
    """HBM bytes per scan launch from the committed rocprofv3 summary, or None."""
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return float(line.split(":", 1)[1].split()[0])
    except OSError:
        return None
    return None


def cpu_baseline(seconds):
    """float64 numpy restatement of the layer (oracle/), one image (T frames) at a time."""
    import numpy as np
    from oracle import cssm_oracle as O
    try:
        from threadpoolctl import threadpool_limits
        limiter = threadpool_limits(limits=1)
    except Exception:          # threadpoolctl absent: numpy's FFT is single-threaded anyway
        limiter = None
    w = WORKLOAD
    cfg = O.GatedConfig(channels=w["C"], kernel_size=w["kernel_size"], gate_type=w["gate_type"],
                        gate_activation=w["gate_activation"], short_conv_size=0, short_conv_spatial_size=0)
    rng = np.random.default_rng(1)
    p = O.init_params(O.gated_param_shapes(cfg, w["C"], w["H"], w["W"]), rng)
    img = rng.standard_normal((1, 1, w["H"], w["W"], w["C"]))
    x = np.repeat(img, w["T"], axis=1)
    frames, t0 = 0, time.perf_counter()
    while True:
        O.gated_forward(p, x, cfg)
        frames += w["T"]
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    if limiter is not None:
        limiter.unregister() if hasattr(limiter, "unregister") else None
    return dict(value=frames / el, unit="frames/s", cores=1, kind="port",
                sample=f"{frames // w['T']} image(s) x T={w['T']} (of B={w['B']}), full C={w['C']} at "
                       f"{w['H']}x{w['W']}, float64 numpy oracle, {el:.1f} s, "
                       f"{platform.processor() or platform.machine()} x{os.cpu_count()} logical cpus")


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}); "
              "the layer shards over batch with no exchange, see DESIGN.md", file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    from cssm_amd import cells, spectral as S

    w = dict(WORKLOAD)
    B, T, H, W, C = args.batch, w["T"], w["H"], w["W"], w["C"]
    dev = "cuda"
    if args.copy_calibration > 0:
        # a streaming kernel of known traffic (read n*4 B, write n*4 B): torch's neg, which
        # nothing else in this run launches, so its dispatch is easy to find in the counters
        n = args.copy_calibration // 4
        src = torch.ones(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        torch.neg(src, out=dst)
        torch.cuda.synchronize()
        del src, dst
    torch.manual_seed(0)
    gen = torch.Generator(device=dev).manual_seed(0)
    img = torch.randn((B, 1, H, W, C), generator=gen, device=dev)
    x = img.expand(B, T, H, W, C).contiguous()
    del img
    cell = cells.GatedCSSM(channels=C, kernel_size=w["kernel_size"], gate_type=w["gate_type"],
                           gate_activation=w["gate_activation"], short_conv_size=0, short_conv_spatial_size=0)
    variables = cell.init(1, x.shape)
    for name, sub in variables["params"].items():       # non-zero biases exercise the bias paths
        if isinstance(sub, dict) and "bias" in sub:
            sub["bias"].normal_(0.0, 0.1, generator=gen)

    # instrumented step: the same calls GatedCSSM.apply makes, with events around each kernel
    p = variables["params"]
    F, HW = B * T, H * W
    ev = {k: [] for k in ("in_proj", "gates", "scan", "out_proj")}

    def step(record):
        marks = []
        if record:
            marks = [torch.cuda.Event(enable_timing=True) for _ in range(5)]
            marks[0].record()
        u, z, ctx = S.proj_in(x, p["in_proj"]["kernel"], p["in_proj"]["bias"], F, HW, silu_lo=True,
                              silu_hi=True, want_ctx=True)
        if record:
            marks[1].record()
        gates = S.gated_gates(ctx.view(B, T, C), p, H, W, w["gate_type"], w["gate_activation"], c_scale=1.0 / HW)
        khat = cell.spectral_kernel(p, H, W)
        if record:
            marks[2].record()
        y = S.gated_scan(u.view(B, T, C, H, W), z.view(B, T, C, H, W), gates, khat)
        if record:
            marks[3].record()
        out = S.proj_out(y.view(F, C, HW), p["out_proj"]["kernel"], p["out_proj"]["bias"])
        if record:
            marks[4].record()
            for i, k in enumerate(("in_proj", "gates", "scan", "out_proj")):
                ev[k].append((marks[i], marks[i + 1]))
        return out

    for _ in range(args.warmup):
        step(False)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step(True)
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    ms_step = el * 1e3 / args.steps
    # the instrumented step must equal the module's forward bit for bit
    if not torch.equal(step(False).view(B, T, H, W, C), cell.apply(variables, x)):
        print("instrumented step differs from GatedCSSM.apply", file=sys.stderr)
        sys.exit(1)
    kern_ms = {k: sum(a.elapsed_time(b) for a, b in v) / len(v) for k, v in ev.items()}
    scan_ms = kern_ms["scan"]
    alg = scan_algorithmic_bytes(B, T, H, W, C)
    achieved = alg / (scan_ms * 1e-3) / 1e9
    traffic = read_traffic(args.traffic) if B == WORKLOAD["B"] else None
    res = {
        "metric": "frames/sec per fused spectral-SSM layer (1 GPU) + % HBM roofline",
        "value": B * T / (ms_step * 1e-3),
        "unit": "frames/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: one N(0,1) 128x128x64 image repeated over T=8 (materialised), random-init weights",
        "config": {"workload": w["name"], "cell": "gated", "batch": B, "T": T, "H": H, "W": W, "channels": C,
                   "kernel_size": w["kernel_size"], "gate_type": w["gate_type"], "short_convs": "0/0",
                   "io": "f32", "step": "full layer forward x -> out_proj"},
        "images_per_s": B / (ms_step * 1e-3),
        "kernel_ms": {k: round(v, 4) for k, v in kern_ms.items()},
        "scan_frames_per_s": B * T / (scan_ms * 1e-3),
        "roofline": {"kernel": "gated_scan_pow2<7,7,1,64,f32>", "bound": "hbm", "achieved": achieved,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
                     "algorithmic_bytes": alg, "traffic": traffic},
    }
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
