#!/usr/bin/env python3
"""Benchmark of the fused spectral-SSM layer (GatedCSSM / GatedDeltaNetCSSM) on one MI355X.

Default workload ("C2"): gated cell, fp32, batch 128
of one 128x128x64 image repeated over T = 8 frames (materialised; the kernels
do not see the repetition), x ~ N(0, 1), kernel_size 11, factored B/C/Delta
gates, softplus Delta, no short convolutions, random-init weights with
N(0, 0.1^2) biases (synthetic data).  ``--workload`` selects the other
BASELINE configs as the headline; by default the others (c1, c3, c4, c5) are
measured in the same run, each the same way, and reported under "configs".
The launch-bound ones (c1, c5) also carry "graph": the same step captured once
in a HIP graph and replayed (checked bit for bit against the eager step); their
value and ms_per_step stay the eager caller's.

A step is one full layer forward with x already in HBM:
  gated: in_proj GEMM (plane-major split + SiLU + spatial-mean epilogue) ->
         gate planes -> fused rfft2 / scan / irfft2 / x SiLU(z) kernel -> out_proj GEMM
  gdn:   frame mean + gates -> [qkv depthwise conv] -> qkv_proj -> short conv + SiLU +
         input gates -> gate_proj -> rfft2 -> per-bin delta-rule scan -> irfft2 ->
         RMSNorm x gate + output_proj
value = frames/s = B * T / step time (whole layer), from K timed steps.

roofline: the dominant kernel, timed with HIP events on its stream over a
second run of K steps with an event after every kernel; where the event records
make the host the slower side, each step is queued behind a bounded spin kernel
covering the host's deficit, so that the spans hold GPU time only (value comes
from the first run, which records nothing).  gated: the fused scan, algorithmic bytes per launch
B*T*(3*H*W*C*s + 3*(H+W/2+1)*4) + C*H*(W/2+1)*8 (read u and z, write y, read the
factored gate vectors, K_hat once).  gdn: the spectral core (rfft2 + scan +
irfft2 launches together), B*T*(4*H*W*C*s + 2*(H+W/2+1)*4) + n_h*H*(W/2+1)*8
(read q, k, v, write o, gates, W_hat once).  s = bytes per I/O element.
training (``--train``, default c2): the same workload's training step, forward +
backward (loss = mean(out^2); gradients of x and every parameter), frames/s of
the whole step with its forward / backward split, and the roofline of the
reverse recurrence cssm_gated_scan_bwd on its algorithmic bytes.
cpu_baseline times the float32 torch-CPU restatement (oracle/cssm_cpu_fp32.py)
of the same layer on a batch slice, on the process's host-core share (warmup 5,
median of up to 20 calls for the headline; warmup 1 and a shorter budget for
the other configs).
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

HBM_PEAK_GBS = 8000.0
METRIC = "frames/sec per fused spectral-SSM layer (1 GPU) + % HBM roofline"

WORKLOADS = {
    "c1": dict(cell="gated", name="C1 gated 1x1 T=1 32x32 expand 2", B=8, T=1, H=32, W=32, C=64, expand=2,
               kernel_size=1, gate_type="factored", io="f32", data="normal"),
    "c2": dict(cell="gated", name="C2 gated 128x128 T=8", B=128, T=8, H=128, W=128, C=64, expand=1, kernel_size=11,
               gate_type="factored", io="f32", data="repeat"),
    "c3": dict(cell="gdn", name="C3 GDN d_k=4 128x128 T=8", B=128, T=8, H=128, W=128, C=64, dk=4, kernel_size=11,
               qkv_conv_size=5, gate_type="factored", io="f32", data="normal"),
    "c4": dict(cell="gdn", name="C4 GDN video d_k=4 32x32 T=32 bf16", B=128, T=32, H=32, W=32, C=64, dk=4,
               kernel_size=11, qkv_conv_size=1, gate_type="factored", io="bf16", data="dots"),
    # CSSM-SHViT-S1-shaped stack: (H, C, layers) per stage, each layer GatedCSSM with expand 2
    "c5": dict(cell="stack", name="C5 gated CSSM-SHViT-shaped stack (11 layers) T=1 bf16", B=512, T=1,
               stages=((14, 128, 2), (7, 224, 4), (4, 320, 5)), H=14, W=14, C=128, expand=2, kernel_size=1,
               gate_type="factored", io="bf16", data="normal"),
}


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="c2", choices=sorted(WORKLOADS))
    ap.add_argument("--batch", type=int, default=0, help="override B (parity/debug runs only)")
    ap.add_argument("--configs", default="c1,c3,c4,c5",
                    help="other BASELINE configs measured in the same run and reported under 'configs' "
                         "(comma-separated; 'none' for the headline workload only)")
    ap.add_argument("--config-steps", type=int, default=20, help="timed steps of each extra config (at least ~30 ms of them, at most 300)")
    ap.add_argument("--train", default="c2",
                    help="workload whose training step (forward + backward) is also measured, reported under "
                         "'training' ('none' to skip)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=20.0,
                    help="time budget of the headline CPU baseline (a quarter of it for each extra config)")
    ap.add_argument("--traffic", default=None,
                    help="rocprofv3 FETCH/WRITE summary giving HBM bytes per dominant-kernel launch "
                         "(default profiles/<kernel>_<workload>_traffic.txt)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="BYTES",
                    help="first run one streaming kernel over BYTES (a known-size kernel that scales "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE counters); not timed")
    return ap.parse_args()


def io_bytes(w):
    return 2 if w["io"] == "bf16" else 4


def algorithmic_bytes(w, B):
    if w["cell"] == "stack":
        return sum(n * algorithmic_bytes(dict(w, cell="gated", H=h, W=h, C=c), B) for h, c, n in w["stages"])
    T, H, W = w["T"], w["H"], w["W"]
    Wf = W // 2 + 1
    s = io_bytes(w)
    if w["cell"] == "gated":
        C = w["C"] * w["expand"]
        return B * T * (3 * H * W * C * s + 3 * (H + Wf) * 4) + C * H * Wf * 8
    C, nh = w["C"], w["C"] // w["dk"]
    return B * T * (4 * H * W * C * s + 2 * (H + Wf) * 4) + nh * H * Wf * 8


def read_traffic(path):
    """HBM bytes per dominant-kernel launch from a committed rocprofv3 summary, or None."""
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return float(line.split(":", 1)[1].split()[0])
    except OSError:
        return None
    return None


# ----------------------------------------------------------------- inputs

def make_input(w, B, torch, dev):
    T, H, W, C = w["T"], w["H"], w["W"], w["C"]
    gen = torch.Generator(device=dev).manual_seed(0)
    dt = torch.bfloat16 if w["io"] == "bf16" else torch.float32
    if w["data"] == "repeat":
        img = torch.randn((B, 1, H, W, C), generator=gen, device=dev)
        return img.expand(B, T, H, W, C).contiguous().to(dt)
    if w["data"] == "dots":
        # ~2 % of pixels set to 1.0 along random-walk dot tracks, N(0, 0.01^2) background
        x = torch.randn((B, T, H, W, C), generator=gen, device=dev) * 0.01
        ndots = max(1, int(0.02 * H * W))
        pos = torch.randint(0, H * W, (B, ndots), generator=gen, device=dev)
        steps = torch.tensor([1, -1, W, -W, 0], device=dev)
        for t in range(T):
            mask = torch.zeros((B, H * W), dtype=torch.bool, device=dev)
            mask.scatter_(1, pos, True)
            x[:, t] = torch.where(mask.view(B, H, W, 1), torch.ones((), device=dev), x[:, t])
            mv = steps[torch.randint(0, 5, (B, ndots), generator=gen, device=dev)]
            pos = (pos + mv) % (H * W)
        return x.to(dt)
    return torch.randn((B, T, H, W, C), generator=gen, device=dev).to(dt)


def make_cell(w, cells):
    if w["cell"] == "stack":
        return [[make_cell(dict(w, cell="gated", H=h, W=h, C=c), cells) for _ in range(n)] for h, c, n in w["stages"]]
    if w["cell"] == "gated":
        return cells.GatedCSSM(channels=w["C"], expand=w["expand"], kernel_size=w["kernel_size"],
                               gate_type=w["gate_type"], short_conv_size=0, short_conv_spatial_size=0)
    return cells.GatedDeltaNetCSSM(channels=w["C"], delta_key_dim=w["dk"], kernel_size=w["kernel_size"],
                                   gate_type=w["gate_type"], qkv_conv_size=w["qkv_conv_size"])


def randomise_biases(variables, torch, dev):
    gen = torch.Generator(device=dev).manual_seed(1)
    for sub in variables["params"].values():     # non-zero biases exercise the bias paths
        if isinstance(sub, dict) and "bias" in sub:
            sub["bias"].normal_(0.0, 0.1, generator=gen)


# ------------------------------------------------------ instrumented steps

class Marks:
    """HIP events on torch's current stream (the stream every kernel is launched on).

    ``pool`` holds events created before the timed region, so the timed steps only
    record them (creating an event costs far more host time than recording one, and
    would show up as GPU idle time in the launch-bound workloads)."""

    def __init__(self, torch, record, pool=None):
        self.torch, self.record, self.seq, self.pool = torch, record, [], pool
        self.count = 0

    def __call__(self, name):
        self.count += 1
        if self.record:
            ev = self.pool.pop() if self.pool else self.torch.cuda.Event(enable_timing=True)
            ev.record()
            self.seq.append((name, ev))

    def spans(self):
        return [(self.seq[i + 1][0], self.seq[i][1], self.seq[i + 1][1]) for i in range(len(self.seq) - 1)]


def gated_step(cell, variables, x, w, S, mark, start=True):
    """The calls GatedCSSM.apply makes (short convolutions off), with a mark after each kernel."""
    import torch
    p = variables["params"]
    B, T, H, W, _ = x.shape
    Ci, F, HW = cell.channels * cell.expand, B * T, H * W
    if start:
        mark("start")
    # in_proj with the gates from its ctx (the gate kernel reduces the projection's channel sums)
    u, z, _, gates = S.proj_in_gates(x, p["in_proj"]["kernel"], p["in_proj"]["bias"], B, T, H, W, p, cell.gate_type,
                                     cell.gate_activation, c_scale=S.scan_c_scale(H, W), silu_lo=True,
                                     silu_hi=True, out_dtype=torch.float32)
    khat = cell.spectral_kernel(p, H, W)
    mark("in_proj_gates")
    y = S.gated_scan(u.view(B, T, Ci, H, W), z.view(B, T, Ci, H, W), gates, khat)
    mark("scan")
    out = S.proj_out(y.view(F, Ci, HW), p["out_proj"]["kernel"], p["out_proj"]["bias"], out_dtype=x.dtype)
    mark("out_proj")
    return out.view(B, T, H, W, cell.channels)


def stack_step(cells_, variables, xs, w, S, mark):
    """Every stage's layers back to back (stage inputs are synthetic: the reference's downsampling
    between stages is outside the layer); returns the last stage's output."""
    mark("start")
    out = None
    for stage, (layer_cells, layer_vars, x) in enumerate(zip(cells_, variables, xs)):
        for cell, v in zip(layer_cells, layer_vars):
            x = gated_step(cell, v, x, w, S, mark, start=False)
        out = x
    return out


def gdn_step(cell, variables, x, w, S, mark):
    """The calls GatedDeltaNetCSSM.apply makes (factored gates, input gates, short conv, RMSNorm)."""
    import torch
    p = variables["params"]
    B, T, H, W, C = x.shape
    F, HW, f32 = B * T, H * W, torch.float32
    mark("start")
    what = cell.spectral_kernel(p, H, W)
    fused = (S.depthwise_conv_mean(x, p["qkv_dw"]["kernel"], p["qkv_dw"]["bias"], out_dtype=f32)
             if cell.qkv_conv_size > 1 else None)
    if fused is not None:
        xq, ctx = fused
        mark("qkv_dw_mean")   # the qkv depthwise conv with the context mean in the same pass over x
    else:
        ctx = S.frame_mean(x)
        xq = (S.depthwise_conv(x, p["qkv_dw"]["kernel"], p["qkv_dw"]["bias"], out_dtype=f32)
              if cell.qkv_conv_size > 1 else x)
    ab, bkv = S.gdn_gates(ctx, p, H, W, cell.delta_key_dim, cell.gate_type, True, "sinusoid", cell.rope_base)
    mark("gates")
    convs = [p["short_conv_q"], p["short_conv_k"], p["short_conv_v"]]
    # the output projection computes gate_proj from x itself (no gate planes in HBM)
    xgate = S.gdn_proj_out_xgate_supported(C, C, HW)
    gv = None
    if cell.qkv_conv_size > 1 or xgate:
        qkv = S.gdn_qkv_proj(xq, p["qkv_proj"]["kernel"], p["qkv_proj"]["bias"], B, T, H, W, convs, 1, bkv,
                             out_dtype=f32)
        mark("qkv_proj")   # with the short conv, SiLU and input gates (one kernel where cssm_gdn_qkv_fused says so)
        if not xgate:
            gv = S.proj_planes(x, p["gate_proj"]["kernel"], p["gate_proj"]["bias"], F, HW, act="silu",
                               out_dtype=f32)
            mark("gate_proj")
    else:
        # both projections read x: gate_proj's columns ride in the fused qkv launch
        qkv, gv = S.gdn_qkv_gate_proj(x, p["qkv_proj"]["kernel"], p["qkv_proj"]["bias"], B, T, H, W, convs, 1, bkv,
                                      p["gate_proj"]["kernel"], p["gate_proj"]["bias"], "silu", out_dtype=f32)
        mark("qkv_gate_proj")
    if S.gdn_core_fused_supported(H, W, cell.delta_key_dim):
        o = S.gdn_core_fused(qkv, True, ab, cell.gate_type, what, cell.delta_key_dim, cell.scan_variant)
        mark("core_fused")   # rfft2 -> norms -> delta rule -> irfft2 in one kernel
    else:
        spec, norms = S.rfft2(qkv, want_norms=True)
        mark("rfft2")
        ohat = S.gdn_scan_bins(spec, norms, ab, cell.gate_type, what, cell.delta_key_dim, cell.scan_variant)
        mark("scan_bins")
        o = S.irfft2(ohat, W, out_dtype=f32)
        mark("irfft2")
    if xgate:
        out = S.gdn_proj_out_xgate(o.view(F, C, HW), x, "rms", p["rms_scale"], None, p["gate_proj"]["kernel"],
                                   p["gate_proj"]["bias"], "silu", p["output_proj"]["kernel"], p["output_proj"]["bias"],
                                   out_dtype=x.dtype)
        mark("proj_out_xgate")   # RMSNorm x SiLU(gate_proj(x)) computed in front of output_proj
    else:
        out = S.gdn_proj_out(o.view(F, C, HW), gv, "rms", p["rms_scale"], None, p["output_proj"]["kernel"],
                             p["output_proj"]["bias"], out_dtype=x.dtype)
        mark("proj_out")
    return out.view(B, T, H, W, C)


# ----------------------------------------------------------- CPU baseline

CPU_SLICE = {"c1": 8, "c2": 2, "c3": 2, "c4": 8, "c5": 16}   # batch elements the CPU baseline runs


def cpu_threads():
    """Host threads for the CPU baseline: the process's CPU share (OMP_NUM_THREADS when set,
    which the GPU boxes set to the one-GPU share, else the affinity mask)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    env = os.environ.get("OMP_NUM_THREADS", "")
    return max(1, min(n, int(env))) if env.isdigit() and int(env) > 0 else n


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def cpu_baseline(w, budget_s, warmup, max_repeats):
    """The float32 torch-CPU restatement of the layer (oracle/cssm_cpu_fp32.py) on the host's
    cores: one batch slice of the workload, `warmup` untimed calls, then timed calls until
    `max_repeats` or the time budget (at least 3); the median call gives frames/s."""
    import numpy as np
    import torch
    from oracle import cssm_oracle as O
    from oracle import cssm_cpu_fp32 as P
    n = cpu_threads()
    prev = torch.get_num_threads()
    torch.set_num_threads(n)
    rng = np.random.default_rng(1)
    gen = torch.Generator().manual_seed(0)
    Bs = min(CPU_SLICE.get(w["key"], 2), w["B"])
    T = w["T"]
    if w["cell"] == "stack":
        layers = []
        for h, c, nl in w["stages"]:
            cfg = O.GatedConfig(channels=c, expand=w["expand"], kernel_size=w["kernel_size"],
                                gate_type=w["gate_type"], short_conv_size=0, short_conv_spatial_size=0)
            for _ in range(nl):
                prm = O.init_params(O.gated_param_shapes(cfg, c, h, h), rng)
                layers.append((P.GatedCPU(prm, c, expand=w["expand"], kernel_size=w["kernel_size"],
                                          gate_type=w["gate_type"]), h, c))
        xs = {(h, c): torch.randn((Bs, T, h, h, c), generator=gen) for _, h, c in layers}

        def run():
            for cell, h, c in layers:
                cell(xs[(h, c)])
        what = f"{len(layers)} layers"
    else:
        H, W, C = w["H"], w["W"], w["C"]
        if w["cell"] == "gated":
            cfg = O.GatedConfig(channels=C, expand=w["expand"], kernel_size=w["kernel_size"],
                                gate_type=w["gate_type"], short_conv_size=0, short_conv_spatial_size=0)
            cell = P.GatedCPU(O.init_params(O.gated_param_shapes(cfg, C, H, W), rng), C, expand=w["expand"],
                              kernel_size=w["kernel_size"], gate_type=w["gate_type"])
        else:
            cfg = O.GDNConfig(channels=C, delta_key_dim=w["dk"], kernel_size=w["kernel_size"],
                              gate_type=w["gate_type"], qkv_conv_size=w["qkv_conv_size"])
            cell = P.GdnCPU(O.init_params(O.gdn_param_shapes(cfg, H, W), rng, spectral_init="xavier"), C, w["dk"],
                            qkv_conv_size=w["qkv_conv_size"])
        if w["data"] == "repeat":
            x = torch.randn((Bs, 1, H, W, C), generator=gen).expand(Bs, T, H, W, C).contiguous()
        else:
            x = torch.randn((Bs, T, H, W, C), generator=gen)
        if w["io"] == "bf16":
            x = x.bfloat16().float()

        def run():
            cell(x)
        what = f"{H}x{W}x{C}"
    times = []
    with torch.inference_mode():
        for _ in range(warmup):
            run()
        t_all = time.perf_counter()
        while len(times) < max_repeats and (len(times) < 3 or time.perf_counter() - t_all < budget_s):
            t0 = time.perf_counter()
            run()
            times.append(time.perf_counter() - t0)
    torch.set_num_threads(prev)
    med = sorted(times)[len(times) // 2]
    return dict(value=Bs * T / med, unit="frames/s", cores=n, kind="port",
                sample=f"float32 torch-CPU restatement of the layer (oracle/cssm_cpu_fp32.py), batch slice "
                       f"B'={Bs} of B={w['B']} (T={T}, {what}), warmup {warmup}, median of {len(times)} timed "
                       f"calls ({med * 1e3:.1f} ms per call), {n} threads on {cpu_model()} "
                       f"(os.cpu_count()={os.cpu_count()})")


# ------------------------------------------------------------------ training

def run_training(key, args, torch, cells, S):
    """The layer's training step on the GPU (training.gated_train_apply / gdn_train_apply): forward,
    loss = mean(out^2), gradients of x and every parameter.  value = frames/s of the whole step;
    the roofline line prices the gated cell's reverse recurrence (cssm_gated_scan_bwd) on its
    algorithmic bytes, timed with HIP events around direct calls on the stream the step uses."""
    from cssm_amd import training, _lib
    w = dict(WORKLOADS[key], key=key)
    if w["cell"] not in ("gated", "gdn"):
        raise ValueError(f"no training step for {key}")
    B = args.batch or w["B"]
    T, H, W = w["T"], w["H"], w["W"]
    cell = make_cell(w, cells)
    x = make_input(w, B, torch, "cuda").float()
    variables = cell.init(1, x.shape)
    randomise_biases(variables, torch, "cuda")

    def leaves(t):
        out = []
        for v in t.values():
            out += leaves(v) if isinstance(v, dict) else [v]
        return out
    ps = leaves(variables["params"])
    for t in ps:
        t.requires_grad_(True)
    xr = x.clone().requires_grad_(True)
    fn = training.gated_train_apply if w["cell"] == "gated" else training.gdn_train_apply
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]

    class _MeanSquare(torch.autograd.Function):
        """loss = mean(out^2) as one reduction forward and one elementwise pass backward
        (2 out / n times the incoming gradient)."""

        @staticmethod
        def forward(ctx, o):
            ctx.save_for_backward(o)
            return torch.linalg.vector_norm(o).square() / o.numel()

        @staticmethod
        def backward(ctx, g):
            (o,) = ctx.saved_tensors
            return o * (g * (2.0 / o.numel()))

    def step(timed):
        if timed:
            ev[0].record()
        out = fn(cell, variables, xr)
        loss = _MeanSquare.apply(out.float())
        if timed:
            ev[1].record()
        grads = torch.autograd.grad(loss, [xr] + ps)
        if timed:
            ev[2].record()
        return grads
    for _ in range(2):
        step(False)
    steps = max(1, min(args.config_steps, 10))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step(False)
    torch.cuda.synchronize()
    ms_step = (time.perf_counter() - t0) * 1e3 / steps
    fwd = bwd = 0.0
    for _ in range(steps):
        step(True)
        torch.cuda.synchronize()
        fwd += ev[0].elapsed_time(ev[1]) / steps
        bwd += ev[1].elapsed_time(ev[2]) / steps
    res = {"value": B * T / (ms_step * 1e-3), "unit": "frames/s", "steps": steps, "ms_per_step": ms_step,
           "ms_forward": fwd, "ms_backward": bwd, "dtype": "f32",
           "config": {"workload": w["name"], "cell": w["cell"], "batch": B, "T": T, "H": H, "W": W,
                      "channels": w["C"], "step": "forward + backward: loss = mean(out^2), gradients of x and "
                                                  "every parameter"},
           "data": "synthetic, as the forward line of the same workload; random-init weights"}
    if w["cell"] == "gated":
        # the reverse recurrence alone, on spectra of the step's shape and the cell's gate planes / K_hat
        C = w["C"] * w["expand"]
        Wf = W // 2 + 1
        p = variables["params"]
        g = torch.Generator(device="cuda").manual_seed(3)
        with torch.no_grad():
            cs = S.scan_c_scale(H, W)
            ctx = torch.randn((B, T, C), generator=g, device="cuda") * 0.1
            gates = training.gate_planes(ctx, p, H, W, cell.gate_type, cell.gate_activation, cs).contiguous()
            khat = training.khat_planes(p["kernel"], H, W, cell.spectral_rho).contiguous()
            uspec = torch.randn((B, T, C, H, Wf), dtype=torch.complex64, generator=g, device="cuda")
            dspec = torch.randn_like(uspec)
            outs = [torch.empty_like(uspec), torch.empty_like(uspec), torch.empty_like(gates),
                    torch.empty((B, C, H, Wf), dtype=torch.complex64, device="cuda")]
            st = torch.cuda.current_stream().cuda_stream

            def bwd_bins():
                _lib.call("cssm_gated_scan_bwd", uspec.data_ptr(), dspec.data_ptr(), gates.data_ptr(),
                          khat.data_ptr(), B, T, C, H, W, float(cs), *[o.data_ptr() for o in outs], st)
            bwd_bins()
            reps = 5
            ev[0].record()
            for _ in range(reps):
                bwd_bins()
            ev[1].record()
            torch.cuda.synchronize()
            k_ms = ev[0].elapsed_time(ev[1]) / reps
        spec = B * T * C * H * Wf * 8
        alg = 4 * spec + 2 * B * T * H * Wf * 16 + C * H * Wf * 8 + B * C * H * Wf * 8
        res["roofline"] = {"kernel": "gated_scan_bwd_bins", "bound": "hbm", "ms": k_ms,
                           "achieved": alg / (k_ms * 1e-3) / 1e9, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                           "frac": alg / (k_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, "algorithmic_bytes": alg,
                           "bytes": "U and dY spectra read, C h and dU spectra written, gate planes read and "
                                    "their gradient written, K_hat read and its per-batch gradient written"}
        del uspec, dspec, outs
    del x, xr, variables, ps
    torch.cuda.empty_cache()
    return res


# ------------------------------------------------------------------- main

# configurations whose eager step is launch-bound: also timed replaying one captured HIP graph
GRAPH_WORKLOADS = ("c1", "c5")


def graph_replay_ms(step, cell, variables, x, w, S, torch, steps):
    """ms per step of the same layer step captured once in a HIP graph (torch.cuda.graph) and
    replayed `steps` times: the same kernels on the same resident x and weights, one graph launch
    per step instead of one host round trip per kernel.  Its output must equal the eager step's
    bit for bit."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step(cell, variables, x, w, S, Marks(torch, False))
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = step(cell, variables, x, w, S, Marks(torch, False))
    for _ in range(3):
        graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        graph.replay()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    ref = step(cell, variables, x, w, S, Marks(torch, False))
    torch.cuda.synchronize()
    if not torch.equal(out, ref):
        raise RuntimeError(f"{w['key']}: graph replay differs from the eager step")
    del graph, out, ref
    return ms


def run_workload(key, args, torch, cells, S, headline):
    """One workload on the GPU: warmup, `steps` timed layer forwards, per-kernel HIP-event times;
    returns the result dict (the bench line's keys for the headline, a compact record otherwise)."""
    w = dict(WORKLOADS[key], key=key)
    B = args.batch or w["B"]
    T, H, W = w["T"], w["H"], w["W"]
    dev = "cuda"
    torch.manual_seed(0)
    cell = make_cell(w, cells)
    if w["cell"] == "stack":
        x = [make_input(dict(w, H=h, W=h, C=c), B, torch, dev) for h, c, _ in w["stages"]]
        variables = [[cl.init(1 + i, xs.shape) for i, cl in enumerate(layer)] for layer, xs in zip(cell, x)]
        for layer in variables:
            for v in layer:
                randomise_biases(v, torch, dev)
    else:
        x = make_input(w, B, torch, dev)
        variables = cell.init(1, x.shape)
        randomise_biases(variables, torch, dev)
    step = {"gated": gated_step, "gdn": gdn_step, "stack": stack_step}[w["cell"]]
    core = ("scan",) if w["cell"] in ("gated", "stack") else (
        ("core_fused",) if S.gdn_core_fused_supported(H, W, w["dk"]) else ("rfft2", "scan_bins", "irfft2"))
    steps = args.steps if headline else max(1, args.config_steps)

    per_step = 0
    for _ in range(max(1, args.warmup)):
        m = Marks(torch, False)
        step(cell, variables, x, w, S, m)
        per_step = m.count
    if not headline:
        # tiny steps (C1: ~50 us): enough of them for ~30 ms of timed work, not a host-jittered 1 ms
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(3):
            step(cell, variables, x, w, S, Marks(torch, False))
        torch.cuda.synchronize()
        est_ms = (time.perf_counter() - t0) * 1e3 / 3
        steps = max(steps, min(300, int(30.0 / max(est_ms, 1e-3))))
    # timed region 1: the layer as a caller runs it (value, ms_per_step)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step(cell, variables, x, w, S, Marks(torch, False))
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    ms_step = el * 1e3 / steps
    graph_ms = graph_replay_ms(step, cell, variables, x, w, S, torch, steps) if key in GRAPH_WORKLOADS else None
    # timed region 2: the same steps with a HIP event recorded after every kernel on the stream
    # they run on (per-kernel times, the dominant kernel's roofline).  Where recording the
    # events makes the host slower than the GPU (the launch-bound C5 stack: 55 per step), each
    # step is queued behind a bounded spin kernel (torch.cuda._sleep) so no span contains GPU
    # idle time spent waiting for the host; the spin starts at the host's measured deficit and
    # doubles while the spans still add up to more than the plain step plus the events' own GPU
    # gaps (at most three tries).  Where the GPU is the slower side nothing is added: a long idle
    # spin would let the clock drop before the step.
    pool = [torch.cuda.Event(enable_timing=True) for _ in range(steps * per_step + 2 + per_step)]
    for ev in pool:             # an event's first record sets it up on the host: done here, untimed
        ev.record()
    torch.cuda.synchronize()
    e0, e1 = pool.pop(), pool.pop()
    t0 = time.perf_counter()
    probe = Marks(torch, True, pool)
    step(cell, variables, x, w, S, probe)                       # host enqueue time of a marked step
    host_ms = (time.perf_counter() - t0) * 1e3
    torch.cuda.synchronize()
    pool += [ev for _, ev in probe.seq]
    cal = 1_000_000
    e0.record()
    torch.cuda._sleep(cal)
    e1.record()
    torch.cuda.synchronize()
    cycles_per_ms = cal / max(e0.elapsed_time(e1), 1e-3)
    head_ms = 1.5 * (host_ms - ms_step) + 0.2 if host_ms > ms_step else 0.0
    gap_ms = 0.008 * per_step          # GPU time between a recorded event and the next kernel
    for attempt in range(3):
        marks = []
        for _ in range(steps):
            if head_ms > 0.0:
                torch.cuda._sleep(int(cycles_per_ms * head_ms))
            m = Marks(torch, True, pool)
            step(cell, variables, x, w, S, m)
            marks.append(m)
        torch.cuda.synchronize()
        span_sum = sum(a.elapsed_time(b) for m in marks for _, a, b in m.spans()) / len(marks)
        if span_sum <= 1.05 * ms_step + gap_ms or attempt == 2:
            break
        pool += [ev for m in marks for _, ev in m.seq]
        head_ms = max(2.0 * head_ms, ms_step + 0.5)
    # the instrumented step must equal the module's forward bit for bit
    if w["cell"] == "stack":
        ref = None
        for layer_cells, layer_vars, xs in zip(cell, variables, x):
            for cl, v in zip(layer_cells, layer_vars):
                xs = cl.apply(v, xs)
            ref = xs
    else:
        ref = cell.apply(variables, x)
    if not torch.equal(step(cell, variables, x, w, S, Marks(torch, False)), ref):
        raise RuntimeError(f"{key}: instrumented step differs from the module's apply")
    kern_ms = {}
    for m in marks:
        for name, a, b in m.spans():
            kern_ms[name] = kern_ms.get(name, 0.0) + a.elapsed_time(b) / len(marks)
    core_ms = sum(kern_ms[k] for k in core)
    alg = algorithmic_bytes(w, B)
    achieved = alg / (core_ms * 1e-3) / 1e9
    kname = "gdn_core" if w["cell"] == "gdn" else "gated_scan"
    # committed traffic summary of the roofline's launches: <kernel>_<workload>_traffic.txt, or for the
    # stack the per-step summary of its 11 scans
    tname = "gated_stack_c5_traffic.md" if w["cell"] == "stack" else f"{kname}_{key}_traffic.txt"
    tpath = args.traffic if (headline and args.traffic) else os.path.join(ROOT, "profiles", tname)
    traffic = read_traffic(tpath) if B == w["B"] else None
    Ci = w["C"] * w.get("expand", 1)
    del x, variables, ref, cell, marks
    torch.cuda.empty_cache()
    data = {"repeat": f"synthetic: one N(0,1) {H}x{W}x{w['C']} image repeated over T={T} (materialised)",
            "normal": f"synthetic: N(0,1) {H}x{W}x{w['C']} frames, T={T}",
            "dots": f"synthetic: 2% moving dots = 1.0 on N(0,0.01^2) background, {H}x{W}x{w['C']}, "
                    f"T={T}"}[w["data"]] + ", random-init weights"
    config = {"workload": w["name"], "cell": w["cell"], "batch": B, "T": T, "H": H, "W": W,
              "channels": w["C"], "inner_channels": Ci, "kernel_size": w["kernel_size"],
              "gate_type": w["gate_type"], "io": w["io"], "step": "full layer forward x -> out",
              # K_hat / W_hat depend only on the spectral kernel weights: the module computes them once
              # per weight version (cssm_spectral_kernel, ~0.22 ms at C2) and caches them, so they are
              # outside the timed step, as in any inference loop with fixed weights
              "excluded": "spectral kernel prep (K_hat / W_hat), cached per weight version"}
    if w["cell"] == "gdn":
        config.update(delta_key_dim=w["dk"], qkv_conv_size=w["qkv_conv_size"])
    if w["cell"] == "stack":
        config.update(stages=[{"H": h, "W": h, "channels": c, "inner_channels": c * w["expand"], "layers": n}
                              for h, c, n in w["stages"]], layers=sum(n for _, _, n in w["stages"]))
        for k in ("H", "W", "channels", "inner_channels"):
            config.pop(k)
    roof = {"kernel": kname, "launches": list(core), "bound": "hbm", "achieved": achieved,
            "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
            "algorithmic_bytes": alg, "traffic": traffic}
    res = {
        "metric": METRIC,
        "value": B * T / (ms_step * 1e-3),
        "unit": "frames/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        # sum of the per-kernel spans of one step: GPU time of the step's kernels back to back
        "ms_kernel_sum": round(sum(kern_ms.values()), 4),
        # spin queued before each event-timed step (0 where the GPU is the slower side)
        "event_step_spin_ms": round(head_ms, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        # the arithmetic runs in float32 (FFT passes, recurrence, split-bf16 MFMA products at
        # float32 level) whatever the I/O dtype; io_dtype is what x and the output are stored in
        "dtype": "f32",
        "io_dtype": w["io"],
        "data": data,
        "config": config,
        "images_per_s": B / (ms_step * 1e-3),
        "kernel_ms": {k: round(v, 4) for k, v in kern_ms.items()},
        "core_ms": round(core_ms, 4),
        "core_frames_per_s": B * T / (core_ms * 1e-3),
        "roofline": roof,
    }
    if graph_ms is not None:
        # the same step replayed from one captured HIP graph (value and ms_per_step stay the eager ones)
        res["graph"] = {"ms_per_step": round(graph_ms, 5), "frames_per_s": B * T / (graph_ms * 1e-3)}
    if not headline:
        for k in ("metric", "n_gpus", "higher_is_better", "scaling", "vs_baseline", "warmup"):
            res.pop(k)
    return res


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}); "
              "the layer shards over batch with no exchange between GPUs", file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    from cssm_amd import cells, spectral as S

    if args.copy_calibration > 0:
        # a streaming kernel of known traffic (read n*4 B, write n*4 B): torch's neg, which
        # nothing else in this run launches, so its dispatch is easy to find in the counters
        n = args.copy_calibration // 4
        src = torch.ones(n, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        torch.neg(src, out=dst)
        torch.cuda.synchronize()
        del src, dst
    extra = [] if args.configs in ("", "none") else [k for k in args.configs.split(",") if k != args.workload]
    for k in extra:
        if k not in WORKLOADS:
            print(f"unknown workload {k!r} in --configs (have {sorted(WORKLOADS)})", file=sys.stderr)
            sys.exit(2)
    res = run_workload(args.workload, args, torch, cells, S, headline=True)
    if extra:
        res["configs"] = {}
        for k in extra:
            print(f"bench: workload {k}", file=sys.stderr, flush=True)
            res["configs"][k] = run_workload(k, args, torch, cells, S, headline=False)
    if args.train not in ("", "none"):
        print(f"bench: training step {args.train}", file=sys.stderr, flush=True)
        res["training"] = run_training(args.train, args, torch, cells, S)
    # the CPU baselines run after every GPU measurement, so the host's thread pool never
    # competes with the launch thread of a timed GPU loop
    if not args.no_cpu_baseline:
        print("bench: cpu baselines", file=sys.stderr, flush=True)
        res["cpu_baseline"] = cpu_baseline(dict(WORKLOADS[args.workload], key=args.workload),
                                           budget_s=args.cpu_seconds, warmup=5, max_repeats=20)
        for k in extra:
            res["configs"][k]["cpu_baseline"] = cpu_baseline(dict(WORKLOADS[k], key=k), budget_s=args.cpu_seconds / 4,
                                                             warmup=1, max_repeats=20)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
