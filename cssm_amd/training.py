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


class _SplitSiluFn(torch.autograd.Function):
    """(SiLU(xz[:, :n]), SiLU(xz[:, n:])) of plane-major (F, 2n, HW).  The backward writes both halves'
    SiLU gradients straight into one (F, 2n, HW) tensor, where two slice gradients would each be a
    zero-filled full tensor to add (six passes over xz instead of two)."""

    @staticmethod
    def forward(ctx, xz, n):
        ctx.save_for_backward(xz)
        ctx.n = n
        return Fn.silu(xz[:, :n]), Fn.silu(xz[:, n:])

    @staticmethod
    def backward(ctx, du, dz):
        (xz,) = ctx.saved_tensors
        n = ctx.n
        dxz = torch.empty_like(xz)
        for g, part in ((du, slice(None, n)), (dz, slice(n, None))):
            if g is None:
                dxz[:, part].zero_()
            else:
                torch.ops.aten.silu_backward.grad_input(g, xz[:, part], grad_input=dxz[:, part])
        return dxz, None


class _ProjPlanesFn(torch.autograd.Function):
    """Dense over channels-last rows x (F HW, K) into plane-major (F, N, HW) on the HIP projection
    kernel.  Adjoint: dx = dy W^T back to channels-last (the plane-major -> channels-last kernel with
    W^T), dW = sum_f (dy_f x_f)^T (one batched GEMM over frames), db = sum of dy."""

    @staticmethod
    def forward(ctx, x2, kernel, bias, frames, hw):
        ctx.save_for_backward(x2, kernel)
        ctx.frames, ctx.hw = frames, hw
        return S.proj_planes(x2, kernel, bias, frames, hw, out_dtype=torch.float32)

    @staticmethod
    def backward(ctx, dy):
        x2, kernel = ctx.saved_tensors
        dy = dy.contiguous()
        K, N = kernel.shape
        dx = S.proj_out(dy, kernel.t().contiguous(), kernel.new_zeros(K), out_dtype=torch.float32)
        dw = torch.bmm(dy, x2.view(ctx.frames, ctx.hw, K)).sum(dim=0).t()
        return dx, dw, dy.sum(dim=(0, 2)), None, None


def _col_sums(x: torch.Tensor) -> torch.Tensor:
    """Column sums of a contiguous float32 (M, N) tensor on the frame-mean kernel: the rows as M / R
    'frames' of R rows (R the largest power of two <= 1024 dividing M, so the mean's 1 / R and the
    rescale are exact), their means summed in a fixed order."""
    M, N = x.shape
    R = min(M & -M, 1024)
    return S.frame_mean(x.view(M // R, R, 1, N)).sum(dim=0) * R


class _PermuteIndex(torch.autograd.Function):
    """x.index_select(dim, idx) for a permutation idx, with the gradient gathered back through the
    inverse permutation (instead of index_select's scatter-add into a zeroed tensor)."""

    @staticmethod
    def forward(ctx, x, dim, idx, inv):
        ctx.dim = dim
        ctx.save_for_backward(inv)
        return x.index_select(dim, idx)

    @staticmethod
    def backward(ctx, g):
        (inv,) = ctx.saved_tensors
        return g.index_select(ctx.dim, inv), None, None, None


class _ProjOutFn(torch.autograd.Function):
    """Dense over plane-major y (F, K, HW) into channels-last (F HW, N) on the HIP projection kernel.
    Adjoint: dy = dout W^T back to plane-major (the channels-last -> plane-major kernel with W^T),
    dW = sum_f y_f dout_f (one batched GEMM over frames), db = sum of dout."""

    @staticmethod
    def forward(ctx, y, kernel, bias):
        ctx.save_for_backward(y, kernel)
        return S.proj_out(y, kernel, bias, out_dtype=torch.float32)

    @staticmethod
    def backward(ctx, dout):
        y, kernel = ctx.saved_tensors
        dout = dout.contiguous()
        F, K, hw = y.shape
        N = kernel.shape[1]
        dy = S.proj_planes(dout, kernel.t().contiguous(), kernel.new_zeros(K), F, hw, out_dtype=torch.float32)
        dw = torch.bmm(y, dout.view(F, hw, N)).sum(dim=0)
        return dy, dw, _col_sums(dout)


class _DwConvFn(torch.autograd.Function):
    """Depthwise ks x ks SAME conv with bias of channels-last (F, H, W, C) frames on the HIP kernel.
    Adjoints: dx = the same conv of dy with the taps flipped (odd ks: the padding is symmetric),
    dW from the weight-gradient kernel, db = sum of dy."""

    @staticmethod
    def forward(ctx, x, kernel, bias):
        ctx.save_for_backward(x, kernel)
        return S.depthwise_conv(x, kernel, bias, out_dtype=torch.float32)

    @staticmethod
    def backward(ctx, dy):
        x, kernel = ctx.saved_tensors
        dy = dy.contiguous()
        C = x.shape[-1]
        dx = S.depthwise_conv(dy, kernel.flip(0, 1).contiguous(), kernel.new_zeros(C), out_dtype=torch.float32)
        dw = S.depthwise_conv_wgrad(x, dy, kernel.shape[0])
        return dx, dw, _col_sums(dy.view(-1, C))


def _dwconv_cl(x4, q):
    """Depthwise SAME conv of channels-last (F, H, W, C) frames: the HIP kernels where they apply
    (odd ks in 3..7, C / 4 dividing 64, W % 8 == 0), else torch's conv."""
    ks = q["kernel"].shape[0]
    F, H, W, C = x4.shape
    if ks % 2 == 1 and S.depthwise_conv_wgrad_supported(W, C, ks):
        return _DwConvFn.apply(x4.contiguous(), q["kernel"], q["bias"])
    lo, hi = (ks - 1) // 2, ks // 2
    w = q["kernel"].permute(3, 2, 0, 1)                                      # (C, 1, k, k)
    return (Fn.conv2d(Fn.pad(x4.permute(0, 3, 1, 2), (lo, hi, lo, hi)), w, groups=C)
            + q["bias"][None, :, None, None]).permute(0, 2, 3, 1)


def _perm(order, device):
    idx = torch.tensor(order, dtype=torch.long, device=device)
    return idx, torch.argsort(idx)


def _col_index(H: int, W: int, device):
    """(scan column order, its inverse) as index tensors."""
    return _perm(S.scan_col_order(H, W), device)


def _khat_index(H: int, W: int, device):
    """(K_hat scan slot order, its inverse) as index tensors."""
    return _perm(S.scan_khat_order(H, W), device)


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
    return _PermuteIndex.apply(planes, 3, *_col_index(H, W, ctx.device)).contiguous()


def khat_planes(k: torch.Tensor, H: int, W: int, rho: float) -> torch.Tensor:
    """The floored K_hat cssm_spectral_kernel(goom_floor=1, scan_order=1) writes, differentiably:
    rho F / (1 + |F|) with F = rfft2(pad / crop of k) (cssm.py:505-529), |K| < 1e-7 -> 1e-7 + 0j,
    in the scan layout (:func:`cssm_amd.spectral.scan_khat_order`)."""
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
    C = kh.shape[0]
    return _PermuteIndex.apply(kh.reshape(C, -1), 1, *_khat_index(H, W, k.device)).view(C, H, W // 2 + 1)


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


def _gate_leaves(p: Dict[str, Any], gate_type: str):
    """The gate projections' parameter tensors in a fixed order, and a function rebuilding the
    dict gate_planes reads from such a list."""
    names = []
    for n in ("delta_proj", "B_proj", "C_proj"):
        names += [f"{n}_h", f"{n}_w"] if gate_type == "factored" else [n]
    leaves = [p[n][k] for n in names for k in ("kernel", "bias")]

    def rebuild(ts):
        return {n: {"kernel": ts[2 * i], "bias": ts[2 * i + 1]} for i, n in enumerate(names)}
    return leaves, rebuild


class _GatedInScanFn(torch.autograd.Function):
    """in_proj -> SiLU -> ctx -> gates -> fused scan -> x SiLU(z) of the gated cell without short
    convolutions (cssm.py:480-581 up to out_proj), as one autograd node whose backward runs on HIP
    kernels end to end: in_proj stores the pre-activations and takes ctx as the mean of their
    SiLU in the same pass (CSSM_PROJ_STORE_PRE_CTX_SILU); the scan applies both SiLUs on load.
    Backward: rfft2 of SiLU(x_main) and of dy * SiLU(z) (cssm_rfft2_ex), the reverse recurrence
    (cssm_gated_scan_bwd), the gates' adjoint (cssm_gated_gates_bwd) with the gate projections'
    gradients as GEMMs over frames, K_hat's construction differentiated by torch on its small
    tensors, then cssm_irfft2_ex writes the two pre-activation gradients straight into one
    plane-major (F, 2C, HW) tensor: dz = irfft2(Y) * dy * SiLU'(z) and
    dx_main = (irfft2(dU) + dctx / HW) * SiLU'(x_main), the ctx term being the spatial mean's
    gradient; in_proj's gradients follow from that tensor (dx on the projection kernel with W^T,
    dW as one batched GEMM over frames)."""

    @staticmethod
    def forward(ctx, x2, w_in, b_in, kernel, meta, *gate_params):
        B, T, H, W, Ci, gate_type, activation, rho, rebuild = meta
        F, HW = B * T, H * W
        xm, z, cx = S.proj_in(x2, w_in, b_in, F, HW, want_ctx=True, out_dtype=torch.float32, ctx_of_silu=True)
        c_scale = S.scan_c_scale(H, W)
        gates = S.gated_gates(cx.view(B, T, Ci), rebuild(list(gate_params)), H, W, gate_type, activation, c_scale)
        khat = S.spectral_kernel(kernel, H, W, rho, goom_floor=True, scan_order=True)
        y = S.gated_scan(xm.view(B, T, Ci, H, W), z.view(B, T, Ci, H, W), gates, khat, u_silu=True, z_silu=True)
        ctx.save_for_backward(x2, w_in, xm, z, cx, kernel, khat, *gate_params)
        ctx.meta = meta
        return y

    @staticmethod
    def backward(ctx, dy):
        x2, w_in, xm, z, cx, kernel, khat_f, *gate_params = ctx.saved_tensors
        B, T, H, W, Ci, gate_type, activation, rho, rebuild = ctx.meta
        F, HW, Wf = B * T, H * W, W // 2 + 1
        K = x2.shape[1]
        dy = dy.contiguous().view(F, Ci, HW)
        c_scale = S.scan_c_scale(H, W)
        gps = rebuild(list(gate_params))
        cx3 = cx.view(B, T, Ci)
        with torch.enable_grad():
            k_l = kernel.detach().requires_grad_(True)
            khat = khat_planes(k_l, H, W, rho)
        gates_c = S.gated_gates(cx3, gps, H, W, gate_type, activation, c_scale)
        uspec = S.rfft2_ex(xm, H, W, x_silu=True)
        dspec = S.rfft2_ex(dy, H, W, a=z, a_silu=True)
        yspec = torch.empty_like(uspec)
        sdu = torch.empty_like(uspec)
        dgates = torch.empty_like(gates_c)
        dkh = torch.empty((B, Ci, H, Wf), dtype=torch.complex64, device=dy.device)
        # the reverse recurrence on the forward's own K_hat; torch's construction only differentiates it
        S.gated_scan_bwd_bins(uspec, dspec, gates_c, khat_f, B, T, Ci, H, W, c_scale, yspec, sdu, dgates, dkh)
        del uspec, dspec, gates_c
        (dk,) = torch.autograd.grad([khat], [k_l], [dkh.sum(dim=0)])
        # the gate pre-activations' gradients (cssm_gated_gates_bwd), then the projections' as GEMMs
        # over frames: every gate kernel side by side is one (Ci, 3 n) matrix, the layout of dfac
        dfac = S.gated_gates_backward(cx3, gps, H, W, dgates, gate_type, activation, c_scale).view(F, -1)
        del dgates
        wcat = torch.cat(gate_params[0::2], dim=1)
        dcx = dfac @ wcat.t()
        dwcat = cx.view(F, Ci).t() @ dfac
        dbcat = dfac.sum(dim=0)
        gp_grads, off = [], 0
        for kp in gate_params[0::2]:
            n = kp.shape[1]
            gp_grads += [dwcat[:, off:off + n], dbcat[off:off + n]]
            off += n
        dxz = torch.empty((F, 2 * Ci, HW), dtype=torch.float32, device=dy.device)
        # the bias gradient from the plane sums the inverse transforms take while storing
        sums = (torch.empty((2, F, Ci), dtype=torch.float32, device=dy.device)
                if S.irfft2_ex_sums_supported(F * Ci, H, W) else None)
        S.irfft2_ex(yspec, W, dxz[:, Ci:], m=dy, d=z, sums=sums[1] if sums is not None else None)
        S.irfft2_ex(sdu, W, dxz[:, :Ci], add=(dcx.reshape(F, Ci) * (1.0 / HW)).contiguous(), d=xm,
                    sums=sums[0] if sums is not None else None)
        del yspec, sdu
        dx = S.proj_out(dxz, w_in.t().contiguous(), w_in.new_zeros(K), out_dtype=torch.float32)
        dw = torch.bmm(dxz, x2.view(F, HW, K)).sum(dim=0).t()
        db = sums.sum(dim=1).reshape(-1) if sums is not None else dxz.sum(dim=(0, 2))
        return (dx, dw, db, dk, None, *gp_grads)


def gated_train_apply(cell, params: Dict[str, Any], x: torch.Tensor) -> torch.Tensor:
    """GatedCSSM forward with autograd (x (B, T, H, W, C) float32 on the GPU; params: the cell's
    tree of float32 device tensors).  Same results as ``cell.apply`` up to float32 rounding."""
    p = params["params"] if "params" in params else params
    B, T, H, W, cin = x.shape
    Ci = cell.channels * cell.expand
    F, HW = B * T, H * W
    if not S.gated_scan_supported(H, W):
        raise NotImplementedError(f"no fused scan kernel for {H}x{W} planes")
    no_convs = cell.short_conv_spatial_size == 0 and cell.short_conv_size == 0
    if no_convs and S.fft_ex_supported(H, W):
        # in_proj through the scan as one node whose backward runs on the fused HIP transforms
        gps, rebuild = _gate_leaves(p, cell.gate_type)
        meta = (B, T, H, W, Ci, cell.gate_type, cell.gate_activation, cell.spectral_rho, rebuild)
        y = _GatedInScanFn.apply(x.reshape(-1, cin).float().contiguous(), p["in_proj"]["kernel"],
                                 p["in_proj"]["bias"], p["kernel"], meta, *gps)
        out = _ProjOutFn.apply(y.view(B * T, Ci, H * W), p["out_proj"]["kernel"], p["out_proj"]["bias"])
        return out.view(B, T, H, W, cell.channels)
    xz = _ProjPlanesFn.apply(x.reshape(-1, cin).float().contiguous(), p["in_proj"]["kernel"], p["in_proj"]["bias"],
                             F, HW)                                        # plane-major (F, 2C, HW)
    c_scale = S.scan_c_scale(H, W)
    if no_convs:
        u, zg = _SplitSiluFn.apply(xz, Ci)
        u, zg = u.view(B, T, Ci, H, W), zg.view(B, T, Ci, H, W)
        return _gated_core(cell, p, u, zg, B, T, H, W, Ci, c_scale)
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
    return _gated_core(cell, p, u, zg, B, T, H, W, Ci, c_scale)


def _gated_core(cell, p, u, zg, B, T, H, W, Ci, c_scale):
    """Gates from ctx, K_hat, the fused scan and out_proj, from u = SiLU(x_m) and SiLU(z)."""
    gates = gate_planes(u.mean(dim=(3, 4)), p, H, W, cell.gate_type, cell.gate_activation, c_scale)
    khat = khat_planes(p["kernel"], H, W, cell.spectral_rho)
    y = _ScanFn.apply(u, zg, gates, khat, c_scale)                           # (B, T, C, H, W)
    out = _ProjOutFn.apply(y.view(B * T, Ci, H * W), p["out_proj"]["kernel"], p["out_proj"]["bias"])
    return out.view(B, T, H, W, cell.channels)


# ----------------------------------------------------------------------------- GDN cell
#
# GatedDeltaNetCSSM trains the same way: torch differentiates the prologue (qkv_dw, qkv_proj, short
# conv, SiLU, input gates, gate_proj), the gates alpha / beta from ctx, W_hat, the spectral L2 norms
# and the output path (norm x gate, output_proj); the batched transforms run on the HIP FFT kernels
# with their adjoints, and the delta rule runs forward in cssm_gdn_scan_bins_train (which keeps the
# state entering every step) and backward in cssm_gdn_scan_bins_bwd.

def _c2r_weights(W: int, device) -> torch.Tensor:
    """c_v of the C2R rule: 1 at v = 0 and (W even) at the Nyquist column v = W/2, else 2.
    For odd W the last column v = (W - 1)/2 is an interior bin and keeps weight 2."""
    c = torch.full((W // 2 + 1,), 2.0, device=device)
    c[0] = 1.0
    if W % 2 == 0:
        c[-1] = 1.0
    return c


class _Rfft2Fn(torch.autograd.Function):
    """spec = rfft2(x) over the last two axes (float32 planes -> complex64), on the HIP kernels.
    Adjoint: dx = H W irfft2(dspec / c_v)."""

    @staticmethod
    def forward(ctx, x):
        ctx.hw = tuple(x.shape[-2:])
        spec, _ = S.rfft2(x.contiguous())
        return spec

    @staticmethod
    def backward(ctx, dspec):
        H, W = ctx.hw
        w = 1.0 / _c2r_weights(W, dspec.device)
        return S.irfft2((dspec * w).contiguous(), W) * float(H * W)


class _Irfft2Fn(torch.autograd.Function):
    """y = irfft2(spec, s=(H, W)) over the last two axes, on the HIP kernels.
    Adjoint: dspec = rfft2(dy) c_v / (H W)."""

    @staticmethod
    def forward(ctx, spec, W):
        ctx.W = W
        return S.irfft2(spec.contiguous(), W)

    @staticmethod
    def backward(ctx, dy):
        H, W = dy.shape[-2], ctx.W
        d, _ = S.rfft2(dy.contiguous())
        return d * (_c2r_weights(W, dy.device) / float(H * W)), None


class _GdnBinsFn(torch.autograd.Function):
    """ohat = delta-rule recurrence of the (norm-scaled) spectra, cssm.py:4898-5000."""

    @staticmethod
    def forward(ctx, spec, ab, what, gate_type, dk, variant):
        ohat, states = S.gdn_scan_bins_train(spec, ab, gate_type, what, dk, variant)
        ctx.save_for_backward(spec, ab, what, states)
        ctx.gate_type, ctx.dk, ctx.variant = gate_type, dk, variant
        return ohat

    @staticmethod
    def backward(ctx, dohat):
        spec, ab, what, states = ctx.saved_tensors
        dspec, dab, dwhat = S.gdn_scan_bins_backward(spec, ab, ctx.gate_type, what, states, dohat.contiguous(),
                                                     ctx.dk, ctx.variant)
        if ctx.gate_type in ("dense", "factored"):      # one (alpha, beta) per bin, shared by the heads
            dab = dab.sum(dim=2)
        elif ctx.gate_type == "channel":                # one per head, shared by the bins
            dab = dab.sum(dim=3)
        else:                                           # one per frame
            dab = dab.sum(dim=(2, 3)).unsqueeze(2)
        return dspec, dab, dwhat.sum(dim=0), None, None, None


def what_planes(k: torch.Tensor, H: int, W: int, rho: float, squash: bool) -> torch.Tensor:
    """W_hat (n_h, H, Wf) = rho F / (1 + |F|) (or F), F = rfft2 of the padded / cropped kernel,
    differentiably (cssm.py:4711-4716; no floor for the GDN cell)."""
    K = k.shape[-1]
    if K > H or K > W:
        sh, sw = (K - H) // 2, (K - W) // 2
        kp = k[:, sh:sh + H, sw:sw + W]
    else:
        ph, pw = (H - K) // 2, (W - K) // 2
        kp = Fn.pad(k, (pw, W - K - pw, ph, H - K - ph))
    F = torch.fft.rfft2(kp)
    return (F * rho / (1.0 + F.abs())) if squash else F


def _temporal_encoding(T: int, C: int, base: float, device) -> torch.Tensor:
    """E[t, 2j] = sin(t / base^(2j / C)), E[t, 2j + 1] = cos(.) (cssm.py:353-383), in float64."""
    inv = 1.0 / (base ** (torch.arange(0, C, 2, dtype=torch.float64, device=device) / C))
    th = torch.arange(T, dtype=torch.float64, device=device)[:, None] * inv[None]
    return torch.stack([torch.sin(th), torch.cos(th)], -1).reshape(T, C).float()


def _gdn_gate(p, name, gate_type, ctx, x, H, W, nh, bounded=False, spatial=False):
    """_gate (cssm.py:4798-4842).  Spatial gates come back broadcastable against plane-major
    (B, T, C, H, W); the others as the (B, T, n_ab) alpha / beta planes the bins kernel reads."""
    B, T, C = ctx.shape
    Wf = W // 2 + 1

    def dense(z, q):
        return z @ q["kernel"] + q["bias"]
    if gate_type == "channel":
        if spatial:
            q = p[name]
            g = torch.sigmoid(x @ q["kernel"].reshape(C, C) + q["bias"])     # (B, T, H, W, C)
            return g.permute(0, 1, 4, 2, 3)
        raw = torch.sigmoid(dense(ctx, p[name]))                             # (B, T, n_h)
    elif gate_type == "factored":
        raw = torch.sigmoid(dense(ctx, p[f"{name}_h"])[..., :, None] + dense(ctx, p[f"{name}_w"])[..., None, :])
        if spatial:
            return raw[:, :, None]                                           # (B, T, 1, H, W)
        raw = raw.reshape(B, T, H * Wf)
    elif gate_type == "scalar":
        raw = torch.sigmoid(dense(ctx, p[name]))                             # (B, T, 1)
        if spatial:
            return raw[..., None, None]
    else:
        raw = torch.sigmoid(dense(ctx, p[name]))
        if spatial:
            return raw.view(B, T, 1, H, W)
    return 0.1 + 0.89 * raw if bounded else raw


def gdn_train_apply(cell, params: Dict[str, Any], x: torch.Tensor) -> torch.Tensor:
    """GatedDeltaNetCSSM forward with autograd (x (B, T, H, W, C) float32 on the GPU; params the
    cell's tree of float32 device tensors).  Same results as ``cell.apply`` up to float32 rounding."""
    p = params["params"] if "params" in params else params
    B, T, H, W, C = x.shape
    dk = cell.delta_key_dim
    nh, F, HW = C // dk, B * T, H * W
    if not S.fft_supported(H, W):
        raise NotImplementedError(f"no spectral transform kernel for {H}x{W} planes")
    x = x.float()
    what = what_planes(p["kernel"], H, W, cell.spectral_rho, not cell.no_spectral_clamp).contiguous()
    ctx = x.mean(dim=(2, 3))
    if not cell.position_independent_gates:
        ctx = ctx + _temporal_encoding(T, C, cell.rope_base, x.device)[None]
    xq = x.reshape(F, H, W, C)
    ks = cell.qkv_conv_size
    if ks > 1 and not cell.qkv_conv_separable:
        # full-channel SAME conv (cssm.py:4750-4753), lo = (ks - 1) // 2 rows / columns of zeros before
        # and ks // 2 after, as lax pads; torch's conv2d correlates like lax does
        lo, hi = (ks - 1) // 2, ks // 2
        xp = Fn.pad(xq.permute(0, 3, 1, 2), (lo, hi, lo, hi))
        qkv = Fn.conv2d(xp, p["qkv_proj"]["kernel"].permute(3, 2, 0, 1), p["qkv_proj"]["bias"])
        qkv = qkv.reshape(B, T, 3 * C, H, W)                                # plane-major
    else:
        if ks > 1:
            xq = _dwconv_cl(xq, p["qkv_dw"])
        qkv = _ProjPlanesFn.apply(xq.reshape(-1, C).contiguous(), p["qkv_proj"]["kernel"], p["qkv_proj"]["bias"],
                                  F, HW).view(B, T, 3 * C, H, W)          # plane-major
    q, k, v = qkv[:, :, :C], qkv[:, :, C:2 * C], qkv[:, :, 2 * C:]
    if cell.short_conv_size > 0:
        q = Fn.silu(_causal_t(q, p["short_conv_q"]))
        k = Fn.silu(_causal_t(k, p["short_conv_k"]))
        v = Fn.silu(_causal_t(v, p["short_conv_v"]))
    if cell.use_input_gates:
        k = k * _gdn_gate(p, "B_k", cell.gate_type, ctx, x, H, W, nh, spatial=True)
        v = v * _gdn_gate(p, "B_v", cell.gate_type, ctx, x, H, W, nh, spatial=True)
    gv = _ProjPlanesFn.apply(x.reshape(-1, C).contiguous(), p["gate_proj"]["kernel"], p["gate_proj"]["bias"], F, HW)
    gv = Fn.silu(gv) if cell.output_gate_act == "silu" else torch.sigmoid(gv)   # plane-major (F, C, HW)
    alpha = _gdn_gate(p, "alpha", cell.gate_type, ctx, x, H, W, nh, bounded=True)
    beta = _gdn_gate(p, "beta", cell.gate_type, ctx, x, H, W, nh)
    ab = torch.stack([alpha, beta], dim=-1).contiguous()                    # (B, T, n_ab, 2)
    spec = _Rfft2Fn.apply(torch.cat([q, k, v], dim=2))                       # (B, T, 3C, H, Wf)
    if cell.use_spectral_l2_norm:
        qk = spec[:, :, :2 * C]
        qk = qk * torch.rsqrt((qk.real ** 2 + qk.imag ** 2).sum(dim=(3, 4), keepdim=True) + 1e-6)
        spec = torch.cat([qk, spec[:, :, 2 * C:]], dim=2)
    ohat = _GdnBinsFn.apply(spec.contiguous(), ab, what, cell.gate_type, dk, cell.scan_variant)
    o = _Irfft2Fn.apply(ohat, W).view(F, C, HW)                              # plane-major
    # per-pixel norm over the channels (dim 1 of the plane-major frames)
    if cell.output_norm == "rms":
        o = o * torch.rsqrt((o * o).mean(dim=1, keepdim=True) + 1e-6) * p["rms_scale"][None, :, None]
    elif cell.output_norm == "layer":
        mu = o.mean(dim=1, keepdim=True)
        var = ((o - mu) ** 2).mean(dim=1, keepdim=True)
        o = ((o - mu) * torch.rsqrt(var + 1e-6) * p["output_layernorm"]["scale"][None, :, None]
             + p["output_layernorm"]["bias"][None, :, None])
    out = _ProjOutFn.apply((o * gv).contiguous(), p["output_proj"]["kernel"], p["output_proj"]["bias"])
    return out.view(B, T, H, W, C)
