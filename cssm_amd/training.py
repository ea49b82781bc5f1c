"""Training path of the gated cell: forward and backward through the HIP scan.

The reference trains through the layer with ``jax.value_and_grad``
(main.py:283).  Here the spectral core -- rfft2, the GOOM-gated complex
recurrence over T, irfft2, x SiLU(z), the part of the layer that costs the
time -- runs forward in ``cssm_gated_scan_fwd`` and backward in the reverse
recurrence ``cssm_gated_scan_bwd`` between batched FFTs (``_ScanFn``).  The
rest of the layer is a handful of small or GEMM-shaped ops that torch
differentiates on the same stream: in_proj / out_proj (library GEMMs), the
short convolutions, SiLU, the spatial mean ctx, and the construction of the
per-bin gate planes and the floored K_hat, written here exactly as the HIP
prep kernels lay them out (columns in the scan's order, the GOOM floor
terms folded in).

``gated_train_apply(cell, params, x)`` returns the layer output with the
autograd graph attached; ``params`` is the cell's parameter tree of leaf
tensors (``requires_grad`` where gradients are wanted).
"""
from __future__ import annotations

from typing import Any, Dict

import torch
import torch.nn.functional as Fn

from . import spectral as S


class _ScanFn(torch.autograd.Function):
    """y = gated_scan(u, z, gates, khat) with its VJP on the HIP reverse recurrence."""

    @staticmethod
    def forward(ctx, u, z, gates, khat, c_scale):
        ctx.save_for_backward(u, z, gates, khat)
        ctx.c_scale = c_scale
        return S.gated_scan(u, z, gates, khat)

    @staticmethod
    def backward(ctx, dy):
        u, z, gates, khat = ctx.saved_tensors
        du, dz, dgates, dkhat = S.gated_scan_backward(u, z, gates, khat, dy.contiguous(), ctx.c_scale)
        return du, dz, dgates, dkhat, None


def _col_index(H: int, W: int, device) -> torch.Tensor:
    return torch.tensor(S.scan_col_order(H, W), dtype=torch.long, device=device)


def gate_planes(ctx: torch.Tensor, p: Dict[str, Any], H: int, W: int, gate_type: str, activation: str,
                c_scale: float) -> torch.Tensor:
    """The per-bin planes cssm_gated_gates writes, differentiably: (B, T, H, Wf, 4) =
    [exp(-Delta), (Delta + 1e-8) B, 2e-7 (Delta + 1e-8), C c_scale], columns in scan order
    (cssm.py:536-567)."""
    B, T, _ = ctx.shape
    Wf = W // 2 + 1

    def make(name):
        if gate_type == "factored":
            gh = ctx @ p[f"{name}_h"]["kernel"] + p[f"{name}_h"]["bias"]
            gw = ctx @ p[f"{name}_w"]["kernel"] + p[f"{name}_w"]["bias"]
            return gh[..., :, None] * gw[..., None, :]
        return (ctx @ p[name]["kernel"] + p[name]["bias"]).view(B, T, H, Wf)
    g = make("delta_proj")
    if activation == "sigmoid":
        d = 2.0 * torch.sigmoid(g)
    elif activation == "exp":
        d = torch.exp(g.clamp(-4.0, 2.0))
    else:
        d = Fn.softplus(g)
    dd = d + 1e-8
    planes = torch.stack([torch.exp(-d), dd * make("B_proj"), dd * 2e-7, make("C_proj") * c_scale], dim=-1)
    return planes.index_select(3, _col_index(H, W, ctx.device)).contiguous()


def khat_planes(k: torch.Tensor, H: int, W: int, rho: float) -> torch.Tensor:
    """The floored K_hat cssm_spectral_kernel(goom_floor=1, scan_order=1) writes, differentiably:
    rho F / (1 + |F|) with F = rfft2(pad / crop of k) (cssm.py:505-529), |K| < 1e-7 -> 1e-7 + 0j,
    columns in scan order."""
    K = k.shape[-1]
    if K > H or K > W:
        sh, sw = (K - H) // 2, (K - W) // 2
        kp = k[:, sh:sh + H, sw:sw + W]
    else:
        ph, pw = (H - K) // 2, (W - K) // 2
        kp = Fn.pad(k, (pw, W - K - pw, ph, H - K - ph))
    F = torch.fft.rfft2(kp)
    kh = F * rho / (1.0 + F.abs())
    kh = torch.where(kh.abs() < 1e-7, torch.full_like(kh, 1e-7), kh)
    return kh.index_select(2, _col_index(H, W, k.device)).contiguous()


def _causal_t(x5, p):
    """Causal depthwise conv over T of plane-major (B, T, C, H, W) with bias (cssm.py:494-500)."""
    k = p["kernel"].shape[0]
    T = x5.shape[1]
    out = p["bias"][None, None, :, None, None].expand_as(x5)
    terms = [out]
    for j in range(k):
        s = k - 1 - j                                       # tap j reads frame t - s
        if s < T:
            w = p["kernel"][j, 0][None, None, :, None, None]
            terms.append(Fn.pad(x5[:, :T - s], (0, 0, 0, 0, 0, 0, s, 0)) * w)
    return sum(terms)


def gated_train_apply(cell, params: Dict[str, Any], x: torch.Tensor) -> torch.Tensor:
    """GatedCSSM forward with autograd (x (B, T, H, W, C) float32 on the GPU; params: the cell's
    tree of float32 device tensors).  Same results as ``cell.apply`` up to float32 rounding."""
    p = params["params"] if "params" in params else params
    B, T, H, W, cin = x.shape
    Ci = cell.channels * cell.expand
    F, HW = B * T, H * W
    if not S.gated_scan_supported(H, W):
        raise NotImplementedError(f"no fused scan kernel for {H}x{W} planes")
    xz = torch.addmm(p["in_proj"]["bias"], x.reshape(-1, cin).float(), p["in_proj"]["kernel"])
    xz = xz.view(F, HW, 2 * Ci).transpose(1, 2)                          # plane-major (F, 2C, HW)
    xm, z = xz[:, :Ci].reshape(B, T, Ci, H, W), xz[:, Ci:].reshape(B, T, Ci, H, W)
    if cell.short_conv_spatial_size > 0:
        sp = p["short_conv_spatial"]
        k = sp["kernel"].shape[0]
        lo, hi = (k - 1) // 2, k // 2
        w = sp["kernel"].permute(3, 2, 0, 1)                                 # (C, 1, k, k)
        xm = (Fn.conv2d(Fn.pad(xm.reshape(F, Ci, H, W), (lo, hi, lo, hi)), w, groups=Ci)
              + sp["bias"][None, :, None, None]).view(B, T, Ci, H, W)
    if cell.short_conv_size > 0:
        xm = _causal_t(xm, p["short_conv_temporal"])
    u = Fn.silu(xm).contiguous()
    zg = Fn.silu(z).contiguous()
    c_scale = S.scan_c_scale(H, W)
    gates = gate_planes(u.mean(dim=(3, 4)), p, H, W, cell.gate_type, cell.gate_activation, c_scale)
    khat = khat_planes(p["kernel"], H, W, cell.spectral_rho)
    y = _ScanFn.apply(u, zg, gates, khat, c_scale)                           # (B, T, C, H, W)
    out = torch.addmm(p["out_proj"]["bias"], y.view(F, Ci, HW).transpose(1, 2).reshape(-1, Ci),
                      p["out_proj"]["kernel"])
    return out.view(B, T, H, W, cell.channels)
