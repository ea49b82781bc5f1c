"""Torch-tensor wrappers over the C ABI: one function per ABI entry point.

Tensors must live on the GPU; each call is enqueued on torch's current HIP
stream.  Nothing here computes on the CPU and there is no fallback path.
"""
from __future__ import annotations

import ctypes
from typing import Dict, List, Optional

import torch

from . import _lib

_DTYPES = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16}
_GATE_ACTS = {"softplus": _lib.ACT_SOFTPLUS, "sigmoid": _lib.ACT_SIGMOID2, "exp": _lib.ACT_EXP}


# the current stream's raw handle without building a torch.cuda.Stream object per call (the
# per-kernel host cost that small batches pay); torch.cuda.current_stream() where torch lacks it
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream() -> int:
    if _raw_stream is not None:
        return _raw_stream(torch.cuda.current_device())
    return torch.cuda.current_stream().cuda_stream


def _dev(t: torch.Tensor, name: str, dtype=None) -> torch.Tensor:
    if not isinstance(t, torch.Tensor) or t.device.type != "cuda":
        raise ValueError(f"{name} must be a GPU tensor")
    if dtype is not None and t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    return t


def spectral_kernel(k: torch.Tensor, H: int, W: int, rho: float = 0.999, squash: bool = True,
                    goom_floor: bool = True, scan_order: bool = False) -> torch.Tensor:
    """K_hat (C, H, W//2+1) complex64 from k (C, K, K) (cssm.py:505-529, 4711-4716).

    ``scan_order`` stores the bins in the scan layout :func:`gated_scan` reads (the
    slots of :func:`scan_khat_order`: columns in :func:`scan_col_order`, at 128 x 128
    also rows paired); otherwise in natural order.
    """
    _dev(k, "k", torch.float32)
    C, K, K2 = k.shape
    if K != K2:
        raise ValueError("spectral kernel must be square (C, K, K)")
    out = torch.empty((C, H, W // 2 + 1), dtype=torch.complex64, device=k.device)
    _lib.call("cssm_spectral_kernel", k.data_ptr(), C, K, H, W, float(rho), int(squash),
              int(goom_floor), int(scan_order), out.data_ptr(), _stream())
    return out


def scan_col_order(H: int, W: int) -> List[int]:
    """Column order of the per-bin planes :func:`gated_scan` reads (gates, K_hat):
    entry p is the frequency column stored at position p of a row (the identity
    except at 128 x 128)."""
    cols = (ctypes.c_int * (W // 2 + 1))()
    _lib.call("cssm_gated_scan_col_order", H, W, cols)
    return list(cols)


def scan_khat_order(H: int, W: int) -> List[int]:
    """Slots of K_hat in the scan layout (:func:`spectral_kernel` with ``scan_order``):
    entry s is the natural index u (W//2+1) + v of the bin stored in complex slot s of
    a channel's plane, so ``natural.view(C, -1)[:, order]`` is the scan layout.  Columns
    follow :func:`scan_col_order`; rows are row-major except at 128 x 128, where rows u
    and u + 16 alternate within each column's slot pairs."""
    idx = (ctypes.c_int * (H * (W // 2 + 1)))()
    _lib.call("cssm_gated_scan_khat_order", H, W, idx)
    return list(idx)


def scan_c_scale(H: int, W: int) -> float:
    """The c_scale :func:`gated_gates` takes for :func:`gated_scan`: the irfft2
    normalisation and the 1/2 of the scan's doubled spectrum, folded into C."""
    return 0.5 / (H * W)


def plane_mean(x: torch.Tensor, silu: bool = False) -> torch.Tensor:
    """Mean over the last two axes of a plane-major tensor (cssm.py:536)."""
    _dev(x, "x")
    if x.dtype not in _DTYPES:
        raise ValueError(f"unsupported dtype {x.dtype}")
    H, W = x.shape[-2:]
    out = torch.empty(x.shape[:-2], dtype=torch.float32, device=x.device)
    _lib.call("cssm_plane_mean", x.data_ptr(), _DTYPES[x.dtype], out.numel(), H, W,
              _lib.LOAD_SILU if silu else _lib.LOAD_IDENTITY, out.data_ptr(), _stream())
    return out


def gate_params_struct(gp: Dict[str, Dict[str, torch.Tensor]], gate_type: str,
                       activation: str) -> _lib.GateParams:
    """cssm_gate_params from a Flax-named parameter dict (delta_proj / B_proj / C_proj)."""
    s = _lib.GateParams()
    s.gate_type = _lib.GATE_FACTORED if gate_type == "factored" else _lib.GATE_DENSE
    s.activation = _GATE_ACTS.get(activation, _lib.ACT_SOFTPLUS)   # unknown -> softplus (cssm.py:441)
    for i, name in enumerate(("delta_proj", "B_proj", "C_proj")):
        if gate_type == "factored":
            ph, pw = gp[f"{name}_h"], gp[f"{name}_w"]
            s.kernel[i] = _dev(ph["kernel"], f"{name}_h.kernel", torch.float32).data_ptr()
            s.bias[i] = _dev(ph["bias"], f"{name}_h.bias", torch.float32).data_ptr()
            s.kernel_w[i] = _dev(pw["kernel"], f"{name}_w.kernel", torch.float32).data_ptr()
            s.bias_w[i] = _dev(pw["bias"], f"{name}_w.bias", torch.float32).data_ptr()
        else:
            p = gp[name]
            s.kernel[i] = _dev(p["kernel"], f"{name}.kernel", torch.float32).data_ptr()
            s.bias[i] = _dev(p["bias"], f"{name}.bias", torch.float32).data_ptr()
    return s


def gated_gates(ctx: torch.Tensor, params: Dict, H: int, W: int, gate_type: str = "dense",
                activation: str = "softplus", c_scale: float = 1.0,
                out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """(B, T, H, Wf, 4) = [exp(-Delta), (Delta + 1e-8) B, 2e-7 (Delta + 1e-8), C * c_scale]
    per bin (cssm.py:536-567), columns in :func:`scan_col_order`: the gate planes
    :func:`gated_scan` reads with ``c_scale = scan_c_scale(H, W)``."""
    _dev(ctx, "ctx", torch.float32)
    B, T, C = ctx.shape
    if out is None:
        out = torch.empty((B, T, H, W // 2 + 1, 4), dtype=torch.float32, device=ctx.device)
    _dev(out, "out", torch.float32)
    s = gate_params_struct(params, gate_type, activation)
    _lib.call("cssm_gated_gates", ctx.data_ptr(), B, T, C, H, W, s, float(c_scale), out.data_ptr(),
              _stream())
    return out


def gated_gates_backward(ctx: torch.Tensor, params: Dict, H: int, W: int, dgates: torch.Tensor,
                         gate_type: str = "dense", activation: str = "softplus",
                         c_scale: float = 1.0) -> torch.Tensor:
    """Adjoint of :func:`gated_gates` (autodiff of cssm.py:536-567): from ``dgates``, the gradient
    of the (B, T, H, Wf, 4) planes, the gradients of the gate pre-activations, float32
    (B, T, 3, H * Wf) for dense gates (natural bin order) or (B, T, 3, H + Wf) for factored ones
    (row factors, then column factors), for delta / B / C."""
    _dev(ctx, "ctx", torch.float32)
    _dev(dgates, "dgates", torch.float32)
    B, T, C = ctx.shape
    Wf = W // 2 + 1
    if tuple(dgates.shape) != (B, T, H, Wf, 4):
        raise ValueError(f"dgates {tuple(dgates.shape)} != {(B, T, H, Wf, 4)}")
    n = H + Wf if gate_type == "factored" else H * Wf
    out = torch.empty((B, T, 3, n), dtype=torch.float32, device=ctx.device)
    s = gate_params_struct(params, gate_type, activation)
    _lib.call("cssm_gated_gates_bwd", ctx.data_ptr(), B, T, C, H, W, s, float(c_scale), dgates.data_ptr(),
              out.data_ptr(), _stream())
    return out


def gated_scan(u: torch.Tensor, z: torch.Tensor, gates: torch.Tensor, khat: torch.Tensor,
               u_silu: bool = False, z_silu: bool = False,
               out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Fused rfft2 -> recurrence -> irfft2 -> x z for plane-major (B, T, C, H, W) u, z.

    ``gates`` are the per-bin planes (B, T, H, Wf, 4) from :func:`gated_gates`
    made with ``c_scale = scan_c_scale(H, W)``; ``khat`` comes from
    :func:`spectral_kernel` with ``goom_floor=True, scan_order=True``.
    """
    _dev(u, "u")
    _dev(z, "z", u.dtype)
    if u.dtype not in _DTYPES:
        raise ValueError(f"unsupported dtype {u.dtype}")
    B, T, C, H, W = u.shape
    Wf = W // 2 + 1
    if z.shape != u.shape:
        raise ValueError("u and z must have the same shape")
    _dev(gates, "gates", torch.float32)
    if tuple(gates.shape) != (B, T, H, Wf, 4):
        raise ValueError(f"gates shape {tuple(gates.shape)} != {(B, T, H, Wf, 4)}")
    _dev(khat, "khat", torch.complex64)
    if tuple(khat.shape) != (C, H, Wf):
        raise ValueError(f"khat shape {tuple(khat.shape)} != {(C, H, Wf)}")
    if out is None:
        out = torch.empty_like(u)
    _dev(out, "out", u.dtype)
    _lib.call("cssm_gated_scan_fwd", u.data_ptr(), z.data_ptr(), out.data_ptr(), _DTYPES[u.dtype],
              B, T, C, H, W, gates.data_ptr(), khat.data_ptr(), int(u_silu), int(z_silu), _stream())
    return out


def gated_scan_backward(u: torch.Tensor, z: torch.Tensor, gates: torch.Tensor, khat: torch.Tensor,
                        dy: torch.Tensor, c_scale: float):
    """Vector-Jacobian product of :func:`gated_scan` (identity load activations) for the
    cotangent dy of its output: returns (du, dz, dgates, dkhat) with the shapes and column
    orders of (u, z, gates, khat).  Batched rfft2 of u and of dy * z, the per-bin reverse
    recurrence (cssm_gated_scan_bwd), then batched irfft2 of the bin gradients and of C h."""
    for t, n in ((u, "u"), (z, "z"), (dy, "dy")):
        _dev(t, n, torch.float32)
    B, T, C, H, W = u.shape
    Wf = W // 2 + 1
    _dev(gates, "gates", torch.float32)
    _dev(khat, "khat", torch.complex64)
    uspec, _ = rfft2(u)
    dspec, _ = rfft2(dy * z)
    yspec = torch.empty_like(uspec)
    sdu = torch.empty_like(uspec)
    dgates = torch.empty_like(gates)
    dkh = torch.empty((B, C, H, Wf), dtype=torch.complex64, device=u.device)
    gated_scan_bwd_bins(uspec, dspec, gates, khat, B, T, C, H, W, c_scale, yspec, sdu, dgates, dkh)
    del dspec, uspec
    dz = dy * irfft2(yspec, W)
    du = irfft2(sdu, W)
    return du, dz, dgates, dkh.sum(dim=0)


def gated_scan_bwd_bins(uspec, dspec, gates, khat, B: int, T: int, C: int, H: int, W: int, c_scale: float,
                        yspec, sdu, dgates, dkh) -> None:
    """The per-bin reverse recurrence of the gated scan (cssm_gated_scan_bwd) on contiguous spectra
    (B, T, C, H, W//2+1) laid out as the batched transforms write them; outputs written in place."""
    for t_, n in ((uspec, "uspec"), (dspec, "dspec"), (yspec, "yspec"), (sdu, "sdu"), (khat, "khat"), (dkh, "dkh")):
        _dev(t_, n, torch.complex64)
    _dev(gates, "gates", torch.float32)
    _dev(dgates, "dgates", torch.float32)
    _lib.call("cssm_gated_scan_bwd", uspec.data_ptr(), dspec.data_ptr(), gates.data_ptr(), khat.data_ptr(),
              B, T, C, H, W, float(c_scale), yspec.data_ptr(), sdu.data_ptr(), dgates.data_ptr(), dkh.data_ptr(),
              _stream())


def gated_scan_supported(H: int, W: int) -> bool:
    return bool(_lib.load().cssm_gated_scan_supported(H, W))


def gated_scan_min_group(H: int, W: int) -> int:
    return int(_lib.load().cssm_gated_scan_min_group(H, W))


def proj_in(x: torch.Tensor, kernel: torch.Tensor, bias: torch.Tensor, frames: int, hw: int,
            silu_lo: bool = False, silu_hi: bool = False, want_ctx: bool = False,
            out_dtype: Optional[torch.dtype] = None, ctx_of_silu: bool = False):
    """Dense(N) on channels-last rows with the plane-major split (cssm.py:480-484).

    x: (..., K) with frames * hw rows.  Returns (lo, hi, ctx): lo, hi are
    (frames, N/2, hw) plane-major; ctx (frames, N/2) = spatial mean of lo, or None.
    ``ctx_of_silu``: lo is stored without activation and ctx is the mean of SiLU(lo)
    (CSSM_PROJ_STORE_PRE_CTX_SILU; silu_lo must be False).
    """
    if ctx_of_silu and silu_lo:
        raise ValueError("ctx_of_silu stores lo without activation")
    _dev(x, "x")
    if x.dtype not in _DTYPES:
        raise ValueError(f"unsupported dtype {x.dtype}")
    K = x.shape[-1]
    if x.numel() != frames * hw * K:
        raise ValueError("x does not hold frames * hw rows")
    _dev(kernel, "kernel", torch.float32)
    _dev(bias, "bias", torch.float32)
    Kk, N = kernel.shape
    if Kk != K or bias.shape != (N,) or N % 2:
        raise ValueError(f"kernel {tuple(kernel.shape)} / bias {tuple(bias.shape)} do not match K={K}")
    od = out_dtype or x.dtype
    lo = torch.empty((frames, N // 2, hw), dtype=od, device=x.device)
    hi = torch.empty_like(lo)
    ctx = ws = None
    nbytes = 0
    if want_ctx:
        ctx = torch.empty((frames, N // 2), dtype=torch.float32, device=x.device)
        nbytes = int(_lib.load().cssm_proj_in_workspace_size(frames, hw, K, N))
        if nbytes:
            ws = torch.empty(nbytes // 4, dtype=torch.float32, device=x.device)
    _lib.call("cssm_proj_in", x.data_ptr(), _DTYPES[x.dtype], frames, hw, K, N, kernel.data_ptr(),
              bias.data_ptr(), lo.data_ptr(), hi.data_ptr(), _DTYPES[od], 3 if ctx_of_silu else int(silu_lo),
              int(silu_hi), ctx.data_ptr() if ctx is not None else None, ws.data_ptr() if ws is not None else None,
              nbytes, _stream())
    return lo, hi, ctx


def proj_in_gates(x: torch.Tensor, kernel: torch.Tensor, bias: torch.Tensor, B: int, T: int, H: int, W: int,
                  params: Dict, gate_type: str = "dense", activation: str = "softplus", c_scale: float = 1.0,
                  silu_lo: bool = False, silu_hi: bool = False, out_dtype: Optional[torch.dtype] = None,
                  ctx_of_silu: bool = False):
    """:func:`proj_in` with ``want_ctx`` followed by :func:`gated_gates` on its ctx, in one call
    (cssm_proj_in_gates: the gate kernel reduces the projection's channel sums itself).
    Returns (lo, hi, ctx, gates) with the shapes of those two functions; the same values."""
    if ctx_of_silu and silu_lo:
        raise ValueError("ctx_of_silu stores lo without activation")
    _dev(x, "x")
    if x.dtype not in _DTYPES:
        raise ValueError(f"unsupported dtype {x.dtype}")
    K = x.shape[-1]
    F, hw = B * T, H * W
    if x.numel() != F * hw * K:
        raise ValueError("x does not hold B * T * H * W rows")
    _dev(kernel, "kernel", torch.float32)
    _dev(bias, "bias", torch.float32)
    Kk, N = kernel.shape
    if Kk != K or bias.shape != (N,) or N % 2:
        raise ValueError(f"kernel {tuple(kernel.shape)} / bias {tuple(bias.shape)} do not match K={K}")
    od = out_dtype or x.dtype
    lo = torch.empty((F, N // 2, hw), dtype=od, device=x.device)
    hi = torch.empty_like(lo)
    ctx = torch.empty((B, T, N // 2), dtype=torch.float32, device=x.device)
    gates = torch.empty((B, T, H, W // 2 + 1, 4), dtype=torch.float32, device=x.device)
    nbytes = int(_lib.load().cssm_proj_in_workspace_size(F, hw, K, N))
    ws = torch.empty(nbytes // 4, dtype=torch.float32, device=x.device) if nbytes else None
    s = gate_params_struct(params, gate_type, activation)
    _lib.call("cssm_proj_in_gates", x.data_ptr(), _DTYPES[x.dtype], B, T, H, W, K, N, kernel.data_ptr(),
              bias.data_ptr(), lo.data_ptr(), hi.data_ptr(), _DTYPES[od], 3 if ctx_of_silu else int(silu_lo),
              int(silu_hi), ctx.data_ptr(), s, float(c_scale), gates.data_ptr(),
              ws.data_ptr() if ws is not None else None, nbytes, _stream())
    return lo, hi, ctx, gates


def proj_out(y: torch.Tensor, kernel: torch.Tensor, bias: torch.Tensor,
             out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """Dense(N) from plane-major (frames, K, hw) to channels-last (frames * hw, N) (cssm.py:584)."""
    _dev(y, "y")
    if y.dtype not in _DTYPES:
        raise ValueError(f"unsupported dtype {y.dtype}")
    F, K, hw = y.shape
    _dev(kernel, "kernel", torch.float32)
    _dev(bias, "bias", torch.float32)
    if kernel.shape[0] != K or bias.shape != (kernel.shape[1],):
        raise ValueError(f"kernel {tuple(kernel.shape)} does not match K={K}")
    N = kernel.shape[1]
    od = out_dtype or y.dtype
    out = torch.empty((F * hw, N), dtype=od, device=y.device)
    _lib.call("cssm_proj_out", y.data_ptr(), _DTYPES[y.dtype], F, hw, K, N, kernel.data_ptr(), bias.data_ptr(),
              out.data_ptr(), _DTYPES[od], _stream())
    return out


def short_conv(x: torch.Tensor, spatial: Optional[Dict[str, torch.Tensor]],
               temporal: Optional[Dict[str, torch.Tensor]], want_ctx: bool = True,
               out_dtype: Optional[torch.dtype] = None):
    """SiLU(causal temporal conv(depthwise spatial conv(x))) on plane-major (B, T, C, H, W)
    x, plus its spatial mean (cssm.py:487-502, 536).  Returns (u, ctx)."""
    _dev(x, "x")
    B, T, C, H, W = x.shape
    od = out_dtype or x.dtype
    u = torch.empty((B, T, C, H, W), dtype=od, device=x.device)
    ctx = torch.empty((B, T, C), dtype=torch.float32, device=x.device) if want_ctx else None
    ks = kt = 0
    ws = bs = wt = bt = None
    if spatial is not None:
        ks = spatial["kernel"].shape[0]
        ws = _dev(spatial["kernel"], "short_conv_spatial.kernel", torch.float32).data_ptr()
        bs = _dev(spatial["bias"], "short_conv_spatial.bias", torch.float32).data_ptr()
    if temporal is not None:
        kt = temporal["kernel"].shape[0]
        wt = _dev(temporal["kernel"], "short_conv_temporal.kernel", torch.float32).data_ptr()
        bt = _dev(temporal["bias"], "short_conv_temporal.bias", torch.float32).data_ptr()
    _lib.call("cssm_short_conv", x.data_ptr(), _DTYPES[x.dtype], B, T, C, H, W, ks, ws, bs, kt, wt, bt,
              u.data_ptr(), _DTYPES[od], ctx.data_ptr() if ctx is not None else None, _stream())
    return u, ctx


# ----------------------------------------------------------------- GDN cell

_GDN_GATE_TYPES = {"dense": _lib.GDN_GATE_DENSE, "factored": _lib.GDN_GATE_FACTORED,
                   "channel": _lib.GDN_GATE_CHANNEL, "scalar": _lib.GDN_GATE_SCALAR}
_ACTS = {"identity": _lib.ACT_IDENTITY, "silu": _lib.ACT_SILU, "sigmoid": _lib.ACT_SIGMOID}
_NORMS = {"none": _lib.NORM_NONE, "rms": _lib.NORM_RMS, "layer": _lib.NORM_LAYER}


def proj_planes(x: torch.Tensor, kernel: torch.Tensor, bias: torch.Tensor, frames: int, hw: int,
                act: str = "identity", out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """Dense(N) of channels-last rows into one plane-major (frames, N, hw) tensor
    (qkv_proj / gate_proj / channel input gates, cssm.py:4753-4859)."""
    _dev(x, "x")
    if x.dtype not in _DTYPES:
        raise ValueError(f"unsupported dtype {x.dtype}")
    K = x.shape[-1]
    if x.numel() != frames * hw * K:
        raise ValueError("x does not hold frames * hw rows")
    _dev(kernel, "kernel", torch.float32)
    _dev(bias, "bias", torch.float32)
    Kk, N = kernel.shape
    if Kk != K or bias.shape != (N,):
        raise ValueError(f"kernel {tuple(kernel.shape)} / bias {tuple(bias.shape)} do not match K={K}")
    od = out_dtype or x.dtype
    out = torch.empty((frames, N, hw), dtype=od, device=x.device)
    _lib.call("cssm_proj_planes", x.data_ptr(), _DTYPES[x.dtype], frames, hw, K, N, kernel.data_ptr(),
              bias.data_ptr(), out.data_ptr(), _DTYPES[od], _ACTS[act], _stream())
    return out


def frame_mean(x: torch.Tensor) -> torch.Tensor:
    """(B, T, H, W, C) channels-last -> (B, T, C) spatial mean (cssm.py:4785)."""
    _dev(x, "x")
    if x.dtype not in _DTYPES:
        raise ValueError(f"unsupported dtype {x.dtype}")
    *lead, H, W, C = x.shape
    F = int(torch.tensor(lead).prod()) if lead else 1
    out = torch.empty((*lead, C), dtype=torch.float32, device=x.device)
    _lib.call("cssm_frame_mean", x.data_ptr(), _DTYPES[x.dtype], F, H * W, C, out.data_ptr(), _stream())
    return out


def depthwise_conv(x: torch.Tensor, kernel: torch.Tensor, bias: torch.Tensor,
                   out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """Depthwise ks x ks SAME conv of channels-last (..., H, W, C) frames (qkv_dw, cssm.py:4744-4750)."""
    _dev(x, "x")
    *lead, H, W, C = x.shape
    F = 1
    for d in lead:
        F *= d
    _dev(kernel, "kernel", torch.float32)
    _dev(bias, "bias", torch.float32)
    ks = kernel.shape[0]
    if tuple(kernel.shape) != (ks, ks, 1, C) or bias.shape != (C,):
        raise ValueError(f"depthwise kernel {tuple(kernel.shape)} does not match C={C}")
    od = out_dtype or x.dtype
    out = torch.empty(x.shape, dtype=od, device=x.device)
    _lib.call("cssm_depthwise_conv", x.data_ptr(), _DTYPES[x.dtype], F, H, W, C, ks, kernel.data_ptr(),
              bias.data_ptr(), out.data_ptr(), _DTYPES[od], _stream())
    return out


def depthwise_conv_mean(x: torch.Tensor, kernel: torch.Tensor, bias: torch.Tensor,
                        out_dtype: Optional[torch.dtype] = None):
    """depthwise_conv and frame_mean of the same x in one pass -> (y, ctx (..., C) float32), or None
    where the fused form does not apply (the caller then runs the two calls): qkv_dw and the GDN
    context mean (cssm.py:4744-4750, :4785) both read the layer input."""
    _dev(x, "x")
    *lead, H, W, C = x.shape
    F = 1
    for d in lead:
        F *= d
    _dev(kernel, "kernel", torch.float32)
    _dev(bias, "bias", torch.float32)
    ks = kernel.shape[0]
    if tuple(kernel.shape) != (ks, ks, 1, C) or bias.shape != (C,):
        raise ValueError(f"depthwise kernel {tuple(kernel.shape)} does not match C={C}")
    n = _lib.load().cssm_depthwise_conv_mean_workspace(F, H, W, C, ks)
    if n <= 0 or kernel.data_ptr() % 16 or bias.data_ptr() % 16:
        return None
    od = out_dtype or x.dtype
    out = torch.empty(x.shape, dtype=od, device=x.device)
    ws = torch.empty(n, dtype=torch.float32, device=x.device)
    ctx = torch.empty((*lead, C), dtype=torch.float32, device=x.device)
    _lib.call("cssm_depthwise_conv_mean", x.data_ptr(), _DTYPES[x.dtype], F, H, W, C, ks, kernel.data_ptr(),
              bias.data_ptr(), out.data_ptr(), _DTYPES[od], ws.data_ptr(), ctx.data_ptr(), _stream())
    return out, ctx


def gdn_gate_params_struct(p: Dict, gate_type: str, input_gates: bool) -> _lib.GdnGateParams:
    """cssm_gdn_gate_params from the Flax-named parameter dict (alpha, beta, B_k, B_v)."""
    s = _lib.GdnGateParams()
    s.gate_type = _GDN_GATE_TYPES[gate_type]
    names = ["alpha", "beta"] + (["B_k", "B_v"] if input_gates and gate_type != "channel" else [])
    for i, name in enumerate(names):
        if gate_type == "factored":
            ph, pw = p[f"{name}_h"], p[f"{name}_w"]
            s.kernel[i] = _dev(ph["kernel"], f"{name}_h.kernel", torch.float32).data_ptr()
            s.bias[i] = _dev(ph["bias"], f"{name}_h.bias", torch.float32).data_ptr()
            s.kernel_w[i] = _dev(pw["kernel"], f"{name}_w.kernel", torch.float32).data_ptr()
            s.bias_w[i] = _dev(pw["bias"], f"{name}_w.bias", torch.float32).data_ptr()
        else:
            s.kernel[i] = _dev(p[name]["kernel"], f"{name}.kernel", torch.float32).data_ptr()
            s.bias[i] = _dev(p[name]["bias"], f"{name}.bias", torch.float32).data_ptr()
    return s


def gdn_gates(ctx: torch.Tensor, params: Dict, H: int, W: int, delta_key_dim: int, gate_type: str,
              input_gates: bool, temporal: str = "sinusoid", rope_base: float = 10000.0,
              temporal_table: Optional[torch.Tensor] = None):
    """(ab, bkv): alpha/beta pairs (B, T, n_ab, 2) and B_k/B_v pairs (B, T, n_kv, 2) or None
    (cssm.py:4785-4869).  temporal in {'none', 'sinusoid', 'learned'}."""
    _dev(ctx, "ctx", torch.float32)
    B, T, C = ctx.shape
    Wf = W // 2 + 1
    n_ab = {"dense": H * Wf, "factored": H * Wf, "channel": C // delta_key_dim, "scalar": 1}[gate_type]
    ab = torch.empty((B, T, n_ab, 2), dtype=torch.float32, device=ctx.device)
    bkv = None
    if input_gates and gate_type != "channel":
        n_kv = 1 if gate_type == "scalar" else H * W
        bkv = torch.empty((B, T, n_kv, 2), dtype=torch.float32, device=ctx.device)
    s = gdn_gate_params_struct(params, gate_type, input_gates)
    tmode = {"none": 0, "sinusoid": 1, "learned": 2}[temporal]
    tt = None
    if tmode == 2:
        tt = _dev(temporal_table, "temporal_table", torch.float32).data_ptr()
    _lib.call("cssm_gdn_gates", ctx.data_ptr(), B, T, C, H, W, delta_key_dim, s, tmode, float(rope_base), tt,
              ab.data_ptr(), bkv.data_ptr() if bkv is not None else None, _stream())
    return ab, bkv


def gdn_qkv_post(qkv: torch.Tensor, convs, gate_mode: int = 0, gates: Optional[torch.Tensor] = None) -> torch.Tensor:
    """In place on plane-major qkv (B, T, 3C, H, W): causal short conv + SiLU (convs = [q, k, v]
    dicts or None) and the input gates on k, v (cssm.py:4763-4848)."""
    _dev(qkv, "qkv")
    B, T, C3, H, W = qkv.shape
    C = C3 // 3
    kt = 0
    kern = bias = None
    if convs is not None:
        kt = convs[0]["kernel"].shape[0]
        ks = [_dev(c["kernel"], "short_conv.kernel", torch.float32) for c in convs]
        bs = [_dev(c["bias"], "short_conv.bias", torch.float32) for c in convs]
        kern = (ctypes.c_void_p * 3)(*[k.data_ptr() for k in ks])
        bias = (ctypes.c_void_p * 3)(*[b.data_ptr() for b in bs])
    gp = None
    if gate_mode:
        _dev(gates, "gates", torch.float32)
        gp = gates.data_ptr()
    _lib.call("cssm_gdn_qkv_post", qkv.data_ptr(), _DTYPES[qkv.dtype], B, T, C, H, W, kt, kern, bias, gate_mode,
              gp, _stream())
    return qkv


def _qkv_args(x, kernel, bias, B, T, H, W, convs, gate_mode, gates):
    _dev(x, "x")
    if x.dtype not in _DTYPES:
        raise ValueError(f"unsupported dtype {x.dtype}")
    K = x.shape[-1]
    if x.numel() != B * T * H * W * K:
        raise ValueError("x does not hold B * T * H * W rows")
    _dev(kernel, "kernel", torch.float32)
    _dev(bias, "bias", torch.float32)
    Kk, N = kernel.shape
    if Kk != K or bias.shape != (N,) or N % 3:
        raise ValueError(f"kernel {tuple(kernel.shape)} / bias {tuple(bias.shape)} do not match K={K}, N=3C")
    kt = 0
    kern = cb = None
    if convs is not None:
        kt = convs[0]["kernel"].shape[0]
        ks = [_dev(c["kernel"], "short_conv.kernel", torch.float32) for c in convs]
        bs = [_dev(c["bias"], "short_conv.bias", torch.float32) for c in convs]
        kern = (ctypes.c_void_p * 3)(*[k.data_ptr() for k in ks])
        cb = (ctypes.c_void_p * 3)(*[b.data_ptr() for b in bs])
    gp = None
    if gate_mode:
        _dev(gates, "gates", torch.float32)
        gp = gates.data_ptr()
    return K, N // 3, kt, kern, cb, gp


def gdn_qkv_proj(x: torch.Tensor, kernel: torch.Tensor, bias: torch.Tensor, B: int, T: int, H: int, W: int,
                 convs, gate_mode: int = 0, gates: Optional[torch.Tensor] = None,
                 out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """qkv_proj of channels-last x (B, T, H, W, K) with the causal short conv + SiLU (convs = [q, k, v]
    dicts or None) and the input gates on k, v fused in (cssm.py:4753-4848) -> (B, T, 3C, H, W)."""
    K, C, kt, kern, cb, gp = _qkv_args(x, kernel, bias, B, T, H, W, convs, gate_mode, gates)
    od = out_dtype or x.dtype
    out = torch.empty((B, T, 3 * C, H, W), dtype=od, device=x.device)
    _lib.call("cssm_gdn_qkv_proj", x.data_ptr(), _DTYPES[x.dtype], B, T, H, W, K, C, kernel.data_ptr(),
              bias.data_ptr(), kt, kern, cb, gate_mode, gp, out.data_ptr(), _DTYPES[od], _stream())
    return out


def gdn_qkv_gate_proj(x: torch.Tensor, kernel: torch.Tensor, bias: torch.Tensor, B: int, T: int, H: int, W: int,
                      convs, gate_mode: int, gates: Optional[torch.Tensor], gate_kernel: torch.Tensor,
                      gate_bias: torch.Tensor, gate_act: str = "silu",
                      out_dtype: Optional[torch.dtype] = None):
    """gdn_qkv_proj and gate_proj (act SiLU or sigmoid, cssm.py:4853-4859) of the same x in one call
    -> (qkv (B, T, 3C, H, W), gv (B, T, C, H, W)); where the qkv projection runs fused the gate columns
    ride in the same launch, so x is read once."""
    K, C, kt, kern, cb, gp = _qkv_args(x, kernel, bias, B, T, H, W, convs, gate_mode, gates)
    _dev(gate_kernel, "gate_kernel", torch.float32)
    _dev(gate_bias, "gate_bias", torch.float32)
    if tuple(gate_kernel.shape) != (K, C) or tuple(gate_bias.shape) != (C,):
        raise ValueError(f"gate kernel {tuple(gate_kernel.shape)} / bias {tuple(gate_bias.shape)} are not ({K}, {C})")
    if gate_act not in ("silu", "sigmoid"):
        raise ValueError(f"gate_act {gate_act!r}")
    od = out_dtype or x.dtype
    out = torch.empty((B, T, 3 * C, H, W), dtype=od, device=x.device)
    gv = torch.empty((B, T, C, H, W), dtype=od, device=x.device)
    _lib.call("cssm_gdn_qkv_gate_proj", x.data_ptr(), _DTYPES[x.dtype], B, T, H, W, K, C, kernel.data_ptr(),
              bias.data_ptr(), kt, kern, cb, gate_mode, gp, gate_kernel.data_ptr(), gate_bias.data_ptr(),
              _ACTS[gate_act], out.data_ptr(), gv.data_ptr(), _DTYPES[od], _stream())
    return out, gv


def gdn_qkv_fused(T: int, H: int, W: int, K: int, kt: int) -> bool:
    """True when gdn_qkv_proj runs as one fused kernel for this shape and short-conv length."""
    return bool(_lib.load().cssm_gdn_qkv_fused(T, H, W, K, kt))


def rfft2(x: torch.Tensor, want_norms: bool = False):
    """Batched rfft2 of (..., H, W) real planes -> (spec (..., H, W//2+1) complex64, norms (...) or None)."""
    _dev(x, "x")
    *lead, H, W = x.shape
    P = 1
    for d in lead:
        P *= d
    spec = torch.empty((*lead, H, W // 2 + 1), dtype=torch.complex64, device=x.device)
    norms = torch.empty(tuple(lead), dtype=torch.float32, device=x.device) if want_norms else None
    _lib.call("cssm_rfft2", x.data_ptr(), _DTYPES[x.dtype], P, H, W, spec.data_ptr(),
              norms.data_ptr() if norms is not None else None, _stream())
    return spec, norms


def irfft2(spec: torch.Tensor, W: int, out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Batched irfft2(s=(H, W)) of (..., H, W//2+1) complex64 spectra -> (..., H, W) real."""
    _dev(spec, "spec", torch.complex64)
    *lead, H, Wf = spec.shape
    if Wf != W // 2 + 1:
        raise ValueError(f"spectrum width {Wf} does not match W={W}")
    P = 1
    for d in lead:
        P *= d
    y = torch.empty((*lead, H, W), dtype=out_dtype, device=spec.device)
    _lib.call("cssm_irfft2", spec.data_ptr(), P, H, W, y.data_ptr(), _DTYPES[out_dtype], _stream())
    return y


def fft_supported(H: int, W: int) -> bool:
    return bool(_lib.load().cssm_fft_min_group(H, W))


def conv_full_planes(x: torch.Tensor, kernel: torch.Tensor, bias: torch.Tensor,
                     max_bytes: int = 1 << 29) -> torch.Tensor:
    """SAME ks x ks conv with full channel mixing of channels-last x (F, H, W, C) into plane-major
    (F, N, H*W) float32 (nn.Conv(N, (ks, ks), padding='SAME'), cssm.py:4751-4753): im2col rows of a
    chunk of frames (cssm_im2col_same, at most ``max_bytes`` of them) times the kernel viewed as
    (ks ks C, N) on the projection kernel (cssm_proj_planes)."""
    _dev(x, "x")
    F, H, W, C = x.shape
    ks = kernel.shape[0]
    if tuple(kernel.shape[:3]) != (ks, ks, C):
        raise ValueError(f"kernel {tuple(kernel.shape)} does not match ({ks}, {ks}, {C}, N)")
    N = kernel.shape[3]
    wk = kernel.reshape(ks * ks * C, N).contiguous()
    out = torch.empty((F, N, H * W), dtype=torch.float32, device=x.device)
    K = ks * ks * C
    fc = max(1, min(F, max_bytes // (H * W * K * 4)))
    cols = torch.empty((fc * H * W, K), dtype=torch.float32, device=x.device)
    for f0 in range(0, F, fc):
        n = min(fc, F - f0)
        xs = x[f0:f0 + n]
        _lib.call("cssm_im2col_same", xs.data_ptr(), _DTYPES[x.dtype], n, H, W, C, ks, cols.data_ptr(), _stream())
        out[f0:f0 + n] = proj_planes(cols[:n * H * W], wk, bias, n, H * W, out_dtype=torch.float32)
    return out


def fft_ex_supported(H: int, W: int) -> bool:
    return bool(_lib.load().cssm_fft_ex_supported(H, W))


def _plane_set(t: Optional[torch.Tensor], C: int, HW: int, name: str):
    """(pointer, frame stride in planes) of a float32 plane set viewed as (F, C, HW) inside a
    contiguous (F, S, HW) tensor, S >= C (a channel slice of a plane-major tensor)."""
    if t is None:
        return None, C
    if not isinstance(t, torch.Tensor) or t.device.type != "cuda" or t.dtype != torch.float32:
        raise ValueError(f"{name} must be a float32 GPU tensor")
    F = t.shape[0]
    if t.dim() != 3 or t.shape[1] != C or t.shape[2] != HW or t.stride(2) != 1 or t.stride(1) != HW \
            or t.stride(0) % HW or t.stride(0) // HW < C:
        raise ValueError(f"{name}: a (F, {C}, {HW}) channel slice of a plane-major tensor is needed")
    return t.data_ptr(), t.stride(0) // HW


def rfft2_ex(x: torch.Tensor, H: int, W: int, x_silu: bool = False, a: Optional[torch.Tensor] = None,
             a_silu: bool = False) -> torch.Tensor:
    """spec = rfft2(act(x) * act(a)) of float32 plane sets x, a (F, C, H*W) (channel slices of
    plane-major tensors allowed): (F, C, H, W//2+1) complex64 (cssm_rfft2_ex)."""
    F, C, HW = x.shape
    xp, xfs = _plane_set(x, C, HW, "x")
    ap, afs = _plane_set(a, C, HW, "a")
    spec = torch.empty((F, C, H, W // 2 + 1), dtype=torch.complex64, device=x.device)
    _lib.call("cssm_rfft2_ex", xp, xfs, int(x_silu), ap, afs, int(a_silu), C, F * C, H, W, spec.data_ptr(),
              _stream())
    return spec


def irfft2_ex_sums_supported(P: int, H: int, W: int) -> bool:
    return bool(_lib.load().cssm_irfft2_ex_sums_supported(P, H, W))


def irfft2_ex(spec: torch.Tensor, W: int, y: torch.Tensor, add: Optional[torch.Tensor] = None,
              m: Optional[torch.Tensor] = None, d: Optional[torch.Tensor] = None,
              sums: Optional[torch.Tensor] = None) -> torch.Tensor:
    """y = (irfft2(spec) + add[p]) * m * SiLU'(d) into the float32 plane set y (F, C, H*W) (a
    channel slice of a plane-major tensor allowed); add (F, C) or None, m / d plane sets or None;
    sums (F, C) float32 receives each plane's sum of y where :func:`irfft2_ex_sums_supported`
    (cssm_irfft2_ex).  Returns y."""
    _dev(spec, "spec", torch.complex64)
    F, C, H, Wf = spec.shape
    HW = H * W
    yp, yfs = _plane_set(y, C, HW, "y")
    mp, mfs = _plane_set(m, C, HW, "m")
    dp, dfs = _plane_set(d, C, HW, "d")
    if add is not None:
        _dev(add, "add", torch.float32)
        if tuple(add.shape) != (F, C) or not add.is_contiguous():
            raise ValueError(f"add must be contiguous ({F}, {C})")
    if sums is not None:
        _dev(sums, "sums", torch.float32)
        if tuple(sums.shape) != (F, C):
            raise ValueError(f"sums must be ({F}, {C})")
    _lib.call("cssm_irfft2_ex", spec.data_ptr(), F * C, H, W, C, yp, yfs,
              add.data_ptr() if add is not None else None, mp, mfs, dp, dfs,
              sums.data_ptr() if sums is not None else None, _stream())
    return y


# how the delta-rule scan sees the entries of M and Delta (cssm_gdn_scan_variant)
GDN_SCAN_VARIANTS = {"goom": 0, "linear": 1, "log_eps": 2}


def gdn_scan_variant(use_log: bool, use_goom: bool, scan_mode: str, delta_key_dim: int) -> str:
    """The scan GatedDeltaNetCSSM's slow path runs for its flags (cssm.py:4939-4991): 'linear' for
    scan_mode='pallas' at d_k = 2 (pallas_matrix_2x2_scan) and for use_log=False (the direct complex
    scan), 'goom' for use_log with use_goom, 'log_eps' for use_log without it (log(|x| + 1e-8),
    cssm.py:4693-4701)."""
    if scan_mode == "pallas" and delta_key_dim == 2:
        return "linear"
    if not use_log:
        return "linear"
    return "goom" if use_goom else "log_eps"


def _variant(scan_variant: str) -> int:
    if scan_variant not in GDN_SCAN_VARIANTS:
        raise ValueError(f"scan_variant {scan_variant!r}: one of {sorted(GDN_SCAN_VARIANTS)}")
    return GDN_SCAN_VARIANTS[scan_variant]


def gdn_scan_bins(spec: torch.Tensor, norms: Optional[torch.Tensor], ab: torch.Tensor, gate_type: str,
                  what: torch.Tensor, delta_key_dim: int, scan_variant: str = "goom") -> torch.Tensor:
    """Delta-rule recurrence over T per (b, head, bin) (cssm.py:4890-5000).

    spec (B, T, 3C, H, Wf) complex64, norms (B, T, 3C) or None, ab from :func:`gdn_gates`,
    what (n_h, H, Wf) complex64, scan_variant from :func:`gdn_scan_variant`.  Returns ohat
    (B, T, C, H, Wf) complex64."""
    _dev(spec, "spec", torch.complex64)
    B, T, C3, H, Wf = spec.shape
    C = C3 // 3
    W = 2 * (Wf - 1)
    _dev(ab, "ab", torch.float32)
    _dev(what, "what", torch.complex64)
    if norms is not None:
        _dev(norms, "norms", torch.float32)
    n_ab = ab.shape[2]
    strides = {"dense": (n_ab, 0, 1), "factored": (n_ab, 0, 1), "channel": (n_ab, 1, 0), "scalar": (1, 0, 0)}
    fs, hs, bs = strides[gate_type]
    ohat = torch.empty((B, T, C, H, Wf), dtype=torch.complex64, device=spec.device)
    _lib.call("cssm_gdn_scan_bins", spec.data_ptr(), norms.data_ptr() if norms is not None else None,
              ab.data_ptr(), fs, hs, bs, what.data_ptr(), B, T, C, H, W, delta_key_dim, _variant(scan_variant),
              ohat.data_ptr(), _stream())
    return ohat


def depthwise_conv_wgrad_supported(W: int, C: int, ks: int) -> bool:
    return bool(_lib.load().cssm_depthwise_conv_wgrad_supported(W, C, ks))


def depthwise_conv_wgrad(x: torch.Tensor, dy: torch.Tensor, ks: int, blocks: int = 1024) -> torch.Tensor:
    """dL/d kernel (ks, ks, 1, C) of :func:`depthwise_conv` for its input x and output gradient dy,
    both float32 channels-last (..., H, W, C): block partial sums on the GPU, added here."""
    _dev(x, "x", torch.float32)
    _dev(dy, "dy", torch.float32)
    *lead, H, W, C = x.shape
    F = 1
    for d in lead:
        F *= d
    blocks = max(1, min(blocks, (F * H * (W // 8) + 63) // 64))
    partial = torch.empty((blocks, ks, ks, C), dtype=torch.float32, device=x.device)
    _lib.call("cssm_depthwise_conv_wgrad", x.data_ptr(), dy.data_ptr(), F, H, W, C, ks, partial.data_ptr(), blocks,
              _stream())
    return partial.sum(dim=0).unsqueeze(2)


def _ab_strides(ab: torch.Tensor, gate_type: str):
    n_ab = ab.shape[2]
    return {"dense": (n_ab, 0, 1), "factored": (n_ab, 0, 1), "channel": (n_ab, 1, 0), "scalar": (1, 0, 0)}[gate_type]


def gdn_scan_bins_train(spec: torch.Tensor, ab: torch.Tensor, gate_type: str, what: torch.Tensor,
                        delta_key_dim: int, scan_variant: str = "goom"):
    """Training forward of the delta rule (cssm.py:4898-5000): spec (B, T, 3C, H, Wf) complex64 with
    q and k already scaled by the spectral L2 norms.  Returns (ohat (B, T, C, H, Wf), states
    (B, T, C / d_k, d_k, d_k, H*Wf): the state entering every step, for
    :func:`gdn_scan_bins_backward`)."""
    _dev(spec, "spec", torch.complex64)
    _dev(ab, "ab", torch.float32)
    _dev(what, "what", torch.complex64)
    B, T, C3, H, Wf = spec.shape
    C, dk = C3 // 3, delta_key_dim
    W = 2 * (Wf - 1)
    fs, hs, bs = _ab_strides(ab, gate_type)
    ohat = torch.empty((B, T, C, H, Wf), dtype=torch.complex64, device=spec.device)
    states = torch.empty((B, T, C // dk, dk, dk, H * Wf), dtype=torch.complex64, device=spec.device)
    _lib.call("cssm_gdn_scan_bins_train", spec.data_ptr(), ab.data_ptr(), fs, hs, bs, what.data_ptr(), B, T, C, H,
              W, dk, _variant(scan_variant), ohat.data_ptr(), states.data_ptr(), _stream())
    return ohat, states


def gdn_scan_bins_backward(spec: torch.Tensor, ab: torch.Tensor, gate_type: str, what: torch.Tensor,
                           states: torch.Tensor, dohat: torch.Tensor, delta_key_dim: int,
                           scan_variant: str = "goom"):
    """Reverse pass of :func:`gdn_scan_bins_train` (gradients as dL/dRe + i dL/dIm).  Returns
    (dspec (B, T, 3C, H, Wf) complex64, dab (B, T, C / d_k, H*Wf, 2) float32 per (head, bin) --
    summed by the caller over what the gate type shares --, dwhat (B, C / d_k, H, Wf) complex64 per
    batch element)."""
    for t, n in ((spec, "spec"), (what, "what"), (states, "states"), (dohat, "dohat")):
        _dev(t, n, torch.complex64)
    _dev(ab, "ab", torch.float32)
    B, T, C3, H, Wf = spec.shape
    C, dk = C3 // 3, delta_key_dim
    W = 2 * (Wf - 1)
    if tuple(dohat.shape) != (B, T, C, H, Wf) or tuple(states.shape) != (B, T, C // dk, dk, dk, H * Wf):
        raise ValueError("dohat / states shapes do not match spec")
    fs, hs, bs = _ab_strides(ab, gate_type)
    dspec = torch.empty_like(spec)
    dab = torch.empty((B, T, C // dk, H * Wf, 2), dtype=torch.float32, device=spec.device)
    dwhat = torch.empty((B, C // dk, H, Wf), dtype=torch.complex64, device=spec.device)
    _lib.call("cssm_gdn_scan_bins_bwd", spec.data_ptr(), ab.data_ptr(), fs, hs, bs, what.data_ptr(),
              states.data_ptr(), dohat.data_ptr(), B, T, C, H, W, dk, _variant(scan_variant), dspec.data_ptr(),
              dab.data_ptr(), dwhat.data_ptr(), _stream())
    return dspec, dab, dwhat


def gdn_core_fused_supported(H: int, W: int, delta_key_dim: int) -> bool:
    return bool(_lib.load().cssm_gdn_core_fused_supported(H, W, delta_key_dim))


def gdn_core_fused(qkv: torch.Tensor, use_l2: bool, ab: torch.Tensor, gate_type: str, what: torch.Tensor,
                   delta_key_dim: int, scan_variant: str = "goom") -> torch.Tensor:
    """The GDN spectral core in one kernel (cssm.py:4875-5025): plane-major float32 qkv
    (B, T, 3C, H, W) -> o (B, T, C, H, W) float32, the irfft2 of the readout; the same as
    :func:`rfft2` + :func:`gdn_scan_bins` + :func:`irfft2` where
    :func:`gdn_core_fused_supported` holds."""
    _dev(qkv, "qkv", torch.float32)
    B, T, C3, H, W = qkv.shape
    C = C3 // 3
    _dev(ab, "ab", torch.float32)
    _dev(what, "what", torch.complex64)
    n_ab = ab.shape[2]
    strides = {"dense": (n_ab, 0, 1), "factored": (n_ab, 0, 1), "channel": (n_ab, 1, 0), "scalar": (1, 0, 0)}
    fs, hs, bs = strides[gate_type]
    o = torch.empty((B, T, C, H, W), dtype=torch.float32, device=qkv.device)
    _lib.call("cssm_gdn_core_fused", qkv.data_ptr(), int(bool(use_l2)), ab.data_ptr(), fs, hs, bs, what.data_ptr(),
              B, T, C, H, W, delta_key_dim, _variant(scan_variant), o.data_ptr(), _stream())
    return o


def gdn_proj_out(o: torch.Tensor, gate: torch.Tensor, norm: str, norm_scale: Optional[torch.Tensor],
                 norm_bias: Optional[torch.Tensor], kernel: torch.Tensor, bias: torch.Tensor,
                 out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """out = (norm(o) * gate) W + b from plane-major (F, K, hw) o and gate to channels-last (F * hw, N)
    (cssm.py:5026-5141)."""
    _dev(o, "o")
    _dev(gate, "gate", o.dtype)
    F, K, hw = o.shape
    _dev(kernel, "kernel", torch.float32)
    _dev(bias, "bias", torch.float32)
    N = kernel.shape[1]
    od = out_dtype or o.dtype
    out = torch.empty((F * hw, N), dtype=od, device=o.device)
    ns = _dev(norm_scale, "norm_scale", torch.float32).data_ptr() if norm_scale is not None else None
    nb = _dev(norm_bias, "norm_bias", torch.float32).data_ptr() if norm_bias is not None else None
    _lib.call("cssm_gdn_proj_out", o.data_ptr(), gate.data_ptr(), _DTYPES[o.dtype], F, hw, K, N, _NORMS[norm], ns, nb,
              kernel.data_ptr(), bias.data_ptr(), out.data_ptr(), _DTYPES[od], _stream())
    return out


def gdn_proj_out_xgate_supported(K: int, N: int, hw: int) -> bool:
    """True when :func:`gdn_proj_out_xgate` has a kernel for these widths and plane size."""
    return bool(_lib.load().cssm_gdn_proj_out_xgate_supported(K, N, hw))


def gdn_proj_out_xgate(o: torch.Tensor, x: torch.Tensor, norm: str, norm_scale: Optional[torch.Tensor],
                       norm_bias: Optional[torch.Tensor], gate_kernel: torch.Tensor, gate_bias: torch.Tensor,
                       gate_act: str, kernel: torch.Tensor, bias: torch.Tensor,
                       out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """:func:`gdn_proj_out` with the gate computed in the kernel from the layer input x (F hw rows of K
    channels, float32 or bfloat16): gate = SiLU / sigmoid(x gate_kernel + gate_bias) (gate_proj,
    cssm.py:4853-4859)."""
    _dev(o, "o")
    _dev(x, "x")
    if x.dtype not in _DTYPES:
        raise ValueError(f"unsupported x dtype {x.dtype}")
    F, K, hw = o.shape
    if x.numel() != F * hw * K:
        raise ValueError("x does not hold F * hw rows of K channels")
    for t, nm in ((gate_kernel, "gate_kernel"), (gate_bias, "gate_bias"), (kernel, "kernel"), (bias, "bias")):
        _dev(t, nm, torch.float32)
    if tuple(gate_kernel.shape) != (K, K) or tuple(gate_bias.shape) != (K,):
        raise ValueError(f"gate kernel {tuple(gate_kernel.shape)} / bias {tuple(gate_bias.shape)} are not ({K}, {K})")
    if gate_act not in ("silu", "sigmoid"):
        raise ValueError(f"gate_act {gate_act!r}")
    N = kernel.shape[1]
    od = out_dtype or o.dtype
    out = torch.empty((F * hw, N), dtype=od, device=o.device)
    ns = _dev(norm_scale, "norm_scale", torch.float32).data_ptr() if norm_scale is not None else None
    nb = _dev(norm_bias, "norm_bias", torch.float32).data_ptr() if norm_bias is not None else None
    _lib.call("cssm_gdn_proj_out_xgate", o.data_ptr(), _DTYPES[o.dtype], x.data_ptr(), _DTYPES[x.dtype], F, hw, K, N,
              _NORMS[norm], ns,
              nb, gate_kernel.data_ptr(), gate_bias.data_ptr(), _ACTS[gate_act], kernel.data_ptr(), bias.data_ptr(),
              out.data_ptr(), _DTYPES[od], _stream())
    return out


# --------------------------------------------------------- CSSMSHViTBlock wiring

BLOCK_NORMS = {"global_layer": 0, "temporal_layer": 1, "layer": 2}
OUTPUT_ACTS = {"none": 0, "gelu": 1, "silu": 2}


def block_norm_stats(x: torch.Tensor, block_norm: str, eps: float = 1e-6) -> torch.Tensor:
    """norm1 statistics (mean, rstd) per group of channels-last (B, T, H, W, C) x
    (cssm_shvit.py:106-114): one group per b ('global_layer'), per (b, h, w)
    ('temporal_layer') or per (b, t, h, w) ('layer')."""
    _dev(x, "x")
    if x.dtype not in _DTYPES:
        raise ValueError(f"unsupported dtype {x.dtype}")
    B, T, H, W, C = x.shape
    mode = BLOCK_NORMS[block_norm]
    groups = B if mode == 0 else (B * H * W if mode == 1 else B * T * H * W)
    stats = torch.empty((groups, 2), dtype=torch.float32, device=x.device)
    _lib.call("cssm_block_norm_stats", x.data_ptr(), _DTYPES[x.dtype], B, T, H, W, C, mode, float(eps),
              stats.data_ptr(), _stream())
    return stats


def block_norm_posconv(x: torch.Tensor, stats: torch.Tensor, block_norm: str, scale: torch.Tensor,
                       bias: torch.Tensor, pos_kernel: Optional[torch.Tensor], pos_bias: Optional[torch.Tensor],
                       T_out: int) -> torch.Tensor:
    """(B, T_out, H, W, C) = norm1(x) + pos_conv(norm1(x)) (cssm_shvit.py:104-145);
    x with T = T_out frames or one image frame repeated to T_out."""
    _dev(x, "x")
    B, T_in, H, W, C = x.shape
    _dev(stats, "stats", torch.float32)
    _dev(scale, "scale", torch.float32)
    _dev(bias, "bias", torch.float32)
    pk = pb = 0
    if pos_kernel is not None:
        if tuple(pos_kernel.shape) != (3, 3, 1, C):
            raise ValueError(f"pos_conv kernel shape {tuple(pos_kernel.shape)} != {(3, 3, 1, C)}")
        pk = _dev(pos_kernel, "pos_kernel", torch.float32).data_ptr()
        pb = _dev(pos_bias, "pos_bias", torch.float32).data_ptr()
    out = torch.empty((B, T_out, H, W, C), dtype=x.dtype, device=x.device)
    _lib.call("cssm_block_norm_posconv", x.data_ptr(), _DTYPES[x.dtype], B, T_in, T_out, H, W, C,
              BLOCK_NORMS[block_norm], stats.data_ptr(), scale.data_ptr(), bias.data_ptr(), pk or None, pb or None,
              out.data_ptr(), _stream())
    return out


def block_residual(res: torch.Tensor, y: torch.Tensor, T_out: int, output_act: str = "none") -> torch.Tensor:
    """res + act(y) (cssm_shvit.py:211-228): the last frame of each when T_out = 1,
    frame by frame otherwise; (B, T_out, H, W, C)."""
    _dev(res, "res")
    _dev(y, "y", res.dtype)
    B, T_res, H, W, C = res.shape
    T_y = y.shape[1]
    out = torch.empty((B, T_out, H, W, C), dtype=res.dtype, device=res.device)
    _lib.call("cssm_block_residual", res.data_ptr(), T_res, y.data_ptr(), T_y, _DTYPES[res.dtype], B, T_out, H, W,
              C, OUTPUT_ACTS[output_act], out.data_ptr(), _stream())
    return out
