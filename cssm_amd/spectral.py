"""Torch-tensor wrappers over the C ABI: one function per ABI entry point.

Tensors must live on the GPU; each call is enqueued on torch's current HIP
stream.  Nothing here computes on the CPU and there is no fallback path.
"""
from __future__ import annotations

from typing import Dict, Optional

import torch

from . import _lib

_DTYPES = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16}
_GATE_ACTS = {"softplus": _lib.ACT_SOFTPLUS, "sigmoid": _lib.ACT_SIGMOID2, "exp": _lib.ACT_EXP}


def _stream() -> int:
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
                    goom_floor: bool = True) -> torch.Tensor:
    """K_hat (C, H, W//2+1) complex64 from k (C, K, K) (cssm.py:505-529, 4711-4716)."""
    _dev(k, "k", torch.float32)
    C, K, K2 = k.shape
    if K != K2:
        raise ValueError("spectral kernel must be square (C, K, K)")
    out = torch.empty((C, H, W // 2 + 1), dtype=torch.complex64, device=k.device)
    _lib.call("cssm_spectral_kernel", k.data_ptr(), C, K, H, W, float(rho), int(squash),
              int(goom_floor), out.data_ptr(), _stream())
    return out


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
    """(B, T, H, Wf, 4) = [exp(-Delta), (Delta + 1e-8) B, (Delta + 1e-8) 1e-7, C * c_scale]
    (cssm.py:536-567)."""
    _dev(ctx, "ctx", torch.float32)
    B, T, C = ctx.shape
    if out is None:
        out = torch.empty((B, T, H, W // 2 + 1, 4), dtype=torch.float32, device=ctx.device)
    _dev(out, "out", torch.float32)
    s = gate_params_struct(params, gate_type, activation)
    _lib.call("cssm_gated_gates", ctx.data_ptr(), B, T, C, H, W, s, float(c_scale), out.data_ptr(),
              _stream())
    return out


def gated_scan(u: torch.Tensor, z: torch.Tensor, gates: torch.Tensor, khat: torch.Tensor,
               u_silu: bool = False, z_silu: bool = False,
               out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Fused rfft2 -> recurrence -> irfft2 -> x z for plane-major (B, T, C, H, W) u, z.

    ``gates`` are the per-bin planes (B, T, H, Wf, 4) from :func:`gated_gates`
    made with ``c_scale = 1/(H*W)``; ``khat`` comes from
    :func:`spectral_kernel` with ``goom_floor=True``.
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


def gated_scan_supported(H: int, W: int) -> bool:
    return bool(_lib.load().cssm_gated_scan_supported(H, W))


def gated_scan_min_group(H: int, W: int) -> int:
    return int(_lib.load().cssm_gated_scan_min_group(H, W))


def proj_in(x: torch.Tensor, kernel: torch.Tensor, bias: torch.Tensor, frames: int, hw: int,
            silu_lo: bool = False, silu_hi: bool = False, want_ctx: bool = False,
            out_dtype: Optional[torch.dtype] = None):
    """Dense(N) on channels-last rows with the plane-major split (cssm.py:480-484).

    x: (..., K) with frames * hw rows.  Returns (lo, hi, ctx): lo, hi are
    (frames, N/2, hw) plane-major; ctx (frames, N/2) = spatial mean of lo, or None.
    """
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
              bias.data_ptr(), lo.data_ptr(), hi.data_ptr(), _DTYPES[od], int(silu_lo), int(silu_hi),
              ctx.data_ptr() if ctx is not None else None, ws.data_ptr() if ws is not None else None,
              nbytes, _stream())
    return lo, hi, ctx


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
