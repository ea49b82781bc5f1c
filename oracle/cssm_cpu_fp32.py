"""torch-CPU restatement of the CSSM layer: the reported CPU baseline (float32)
and the gradient reference of the training path (float64).

TEST INFRASTRUCTURE ONLY.  ``bench.py``'s ``cpu_baseline`` leg times this
module on the host's cores (torch's intra-op threads), and ``tests/`` pins it
against the float64 oracle (``oracle/cssm_oracle.py``) and, for gradients,
against central finite differences.  The product path (``cssm_amd``) never
imports it; it is never the thing measured on the GPU.

It follows the reference's op order with torch CPU kernels in float32 /
complex64, which is how the reference's JAX CPU path runs (the reference
itself cannot run here: JAX/Flax are absent):

  gated (cssm.py:476-585): in_proj -> [short convs] -> SiLU -> rfft2 -> ctx ->
      factored / dense Delta, B, C gates -> GOOM floors -> sequential complex
      recurrence over T -> x C -> irfft2 -> x SiLU(z) -> out_proj.
  gdn (cssm.py:4685-5141): [qkv_dw] -> qkv_proj -> causal short conv + SiLU ->
      input gates -> gate_proj -> rfft2 -> spectral / key norms -> delta rule
      per (head, bin) over T -> readout -> irfft2 -> RMSNorm -> x gate ->
      output_proj.

The recurrence is the exact linear form of the reference's log-space scan
(GOOM log_add_exp is exact addition), evaluated sequentially over T.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as Fn


def params_to_torch(tree, dtype=torch.float32, requires_grad=False):
    """Nested dict of numpy arrays -> CPU tensors of dtype (leaf tensors when requires_grad)."""
    if isinstance(tree, dict):
        return {k: params_to_torch(v, dtype, requires_grad) for k, v in tree.items()}
    t = torch.as_tensor(tree, dtype=dtype).clone().contiguous()
    return t.requires_grad_(requires_grad)


def _dense(x, p):
    return torch.addmm(p["bias"], x.reshape(-1, x.shape[-1]), p["kernel"]).reshape(*x.shape[:-1], -1)


def _floor(z):
    """to_goom's floor (goom.py:161-174): |z| < 1e-7 -> 1e-7 + 0j."""
    r = torch.view_as_real(z)
    small = (r[..., 0] * r[..., 0] + r[..., 1] * r[..., 1]) < 1e-14
    return torch.where(small, torch.full_like(z, 1e-7), z)


def _scan_entries(z, variant):
    """M / Delta entries as the GDN scan variant sees them (cssm.py:4693-4701, 4939-4991; the
    oracle's gdn_scan_entries): 'goom' to_goom's floor, 'linear' unchanged, 'log_eps'
    exp(log(|z| + 1e-8) + i angle(z)) = (|z| + 1e-8) z / |z| and 1e-8 at z = 0, which passes no
    gradient there."""
    if variant == "goom":
        return _floor(z)
    if variant == "linear":
        return z
    if variant == "log_eps":
        r = torch.view_as_real(z)
        r2 = r[..., 0] * r[..., 0] + r[..., 1] * r[..., 1]
        zero = r2 == 0
        mag = torch.sqrt(torch.where(zero, torch.ones_like(r2), r2))
        return torch.where(zero, torch.full_like(z, 1e-8), z * (1.0 + 1e-8 / mag))
    raise ValueError(variant)


def scan_core(u, z, gates, khat, c_scale, cols, korder=None):
    """The contract of the fused scan kernel (cssm_gated_scan_fwd with identity load
    activations): u, z (B, T, C, H, W); gates (B, T, H, Wf, 4) = [exp(-Delta),
    (Delta + 1e-8) B, 2 VF, C c_scale] with column p holding frequency column cols[p];
    floored khat (C, H, Wf) in the scan layout: complex slot s of a channel's plane holds
    natural bin korder[s] (cssm_gated_scan_khat_order; korder None: columns permuted by
    cols, rows in order).  Returns irfft2(C h_t) * z with
    h_t = khat e^{-Delta_t} h_{t-1} + (V_t := (Delta + 1e-8) B U_t, or VF where |U_t B| < 1e-7)."""
    inv = torch.argsort(torch.as_tensor(cols))
    g = gates.index_select(3, inv)
    if korder is None:
        kh = khat.index_select(2, inv)
    else:
        Cc, Hh, Wfh = khat.shape
        kinv = torch.argsort(torch.as_tensor(korder))
        kh = khat.reshape(Cc, -1).index_select(1, kinv).view(Cc, Hh, Wfh)
    B, T, C, H, W = u.shape
    U = torch.fft.rfft2(u)
    h = torch.zeros_like(U[:, 0])
    Y = []
    for t in range(T):
        E, DB, VF2, GC = (g[:, t, None, ..., i] for i in range(4))
        P = U[:, t] * DB
        r = torch.view_as_real(P)
        small = (r[..., 0] ** 2 + r[..., 1] ** 2) < (0.5 * VF2) ** 2
        V = torch.where(small, (0.5 * VF2).to(P.dtype), P)
        h = kh * E * h + V
        Y.append(h * (GC / c_scale))
    return torch.fft.irfft2(torch.stack(Y, 1), s=(H, W)) * z


def _planes_in(x, p):
    """Dense over the channels of channels-last frames (F, H, W, K), written plane-major
    (F, N, H, W) by one batched matmul: W^T (N, K) @ x^T (K, HW) per frame."""
    F, H, W, K = x.shape
    y = torch.matmul(p["kernel"].t(), x.reshape(F, H * W, K).transpose(1, 2))
    return (y + p["bias"][None, :, None]).reshape(F, -1, H, W)


def _planes_out(y, p):
    """Dense over the channels of plane-major frames (F, C, H, W) -> channels-last (F, H, W, N)."""
    F, C, H, W = y.shape
    return (torch.matmul(y.reshape(F, C, H * W).transpose(1, 2), p["kernel"]) + p["bias"]).reshape(F, H, W, -1)


def _pad_kernel(k, H, W):
    """cssm.py:510-526: zero-pad with (H-K)//2 before, centre-crop when K > H."""
    K = k.shape[-1]
    if K > H or K > W:
        sh, sw = (K - H) // 2, (K - W) // 2
        return k[:, sh:sh + H, sw:sw + W]
    ph, pw = (H - K) // 2, (W - K) // 2
    return Fn.pad(k, (pw, W - K - pw, ph, H - K - ph))


def spectral_kernel(k, H, W, rho, squash=True):
    F = torch.fft.rfft2(_pad_kernel(k, H, W))
    return F * rho / (1.0 + F.abs()) if squash else F


def _gate_act(x, kind):
    """cssm.py:432-441."""
    if kind == "sigmoid":
        return torch.sigmoid(x) * 2.0
    if kind == "exp":
        return torch.exp(x.clamp(-4.0, 2.0))
    return Fn.softplus(x)


def _dwconv_same(x, p):
    """Depthwise k x k SAME conv with bias on (N, H, W, C) (flax Conv, HWIO kernel)."""
    k = p["kernel"].shape[0]
    C = x.shape[-1]
    w = p["kernel"].permute(3, 2, 0, 1).contiguous()          # (C, 1, k, k)
    lo, hi = (k - 1) // 2, k // 2
    xp = Fn.pad(x.permute(0, 3, 1, 2), (lo, hi, lo, hi))
    return (Fn.conv2d(xp, w, groups=C) + p["bias"][None, :, None, None]).permute(0, 2, 3, 1)


def _conv_same(x, p):
    """k x k SAME conv with full channel mixing and bias on (N, H, W, C) (flax Conv, HWIO kernel
    (k, k, C, N); the full qkv conv of cssm.py:4750-4753)."""
    k = p["kernel"].shape[0]
    w = p["kernel"].permute(3, 2, 0, 1).contiguous()          # (N, C, k, k)
    lo, hi = (k - 1) // 2, k // 2
    xp = Fn.pad(x.permute(0, 3, 1, 2), (lo, hi, lo, hi))
    return (Fn.conv2d(xp, w) + p["bias"][None, :, None, None]).permute(0, 2, 3, 1)


def _causal_t(x5, p):
    """cssm.py:494-500 on plane-major (B, T, C, H, W): left pad k-1 frames, VALID
    depthwise conv over T, bias per channel."""
    k = p["kernel"].shape[0]
    T = x5.shape[1]
    w = p["kernel"][:, 0, :, None, None]                   # (k, C, 1, 1)
    out = p["bias"][:, None, None].expand_as(x5).clone()
    for t in range(T):
        for j in range(k):
            s = t - (k - 1) + j
            if s >= 0:
                out[:, t] += x5[:, s] * w[j]
    return out


def _dwconv_planes(x, p):
    """Depthwise k x k SAME conv with bias on plane-major (N, C, H, W)."""
    k = p["kernel"].shape[0]
    C = x.shape[1]
    w = p["kernel"].permute(3, 2, 0, 1).contiguous()          # (C, 1, k, k)
    lo, hi = (k - 1) // 2, k // 2
    return Fn.conv2d(Fn.pad(x, (lo, hi, lo, hi)), w, groups=C) + p["bias"][None, :, None, None]


class GatedCPU:
    """GatedCSSM forward (cssm.py:476-585) in float32 on the CPU."""

    def __init__(self, params, channels, expand=1, kernel_size=11, spectral_rho=0.999, gate_type="factored",
                 gate_activation="softplus", short_conv_size=0, short_conv_spatial_size=0, dtype=torch.float32,
                 requires_grad=False):
        self.p = params_to_torch(params, dtype, requires_grad)
        self.Ci = channels * expand
        self.rho = spectral_rho
        self.gate_type = gate_type
        self.act = gate_activation
        self.kt, self.ks = short_conv_size, short_conv_spatial_size
        self._khat = {}

    def __call__(self, x):
        p, Ci = self.p, self.Ci
        B, T, H, W, _ = x.shape
        Wf = W // 2 + 1
        xz = _planes_in(x.reshape(B * T, H, W, -1), p["in_proj"])      # (F, 2C, H, W)
        xm, z = xz[:, :Ci], xz[:, Ci:]
        if self.ks > 0:
            xm = _dwconv_planes(xm, p["short_conv_spatial"])
        xm = xm.reshape(B, T, Ci, H, W)
        if self.kt > 0:
            xm = _causal_t(xm, p["short_conv_temporal"])
        xm = Fn.silu(xm)
        # K_hat is reused only for the same kernel tensor object when no derivative flows through it
        # (a perturbed, differentiated or forward-mode dual kernel is recomputed)
        kern = p["kernel"]
        hit = self._khat.get((H, W))
        if hit is None or hit[0] is not kern or kern.requires_grad:
            hit = (kern, _floor(spectral_kernel(kern, H, W, self.rho)))
            self._khat[(H, W)] = hit
        kh = hit[1]
        U = torch.fft.rfft2(xm)                                         # (B, T, C, H, Wf)
        ctx = xm.mean(dim=(3, 4))

        def make(name):
            if self.gate_type == "factored":
                return _dense(ctx, p[name + "_h"])[..., :, None] * _dense(ctx, p[name + "_w"])[..., None, :]
            return _dense(ctx, p[name]).reshape(B, T, H, Wf)
        d = _gate_act(make("delta_proj"), self.act)[:, :, None]
        gB, gC = make("B_proj")[:, :, None], make("C_proj")[:, :, None]
        h = torch.zeros_like(U[:, 0])
        Y = torch.empty_like(U)
        for t in range(T):
            h = kh * torch.exp(-d[:, t]) * h + (d[:, t] + 1e-8) * _floor(U[:, t] * gB[:, t])
            Y[:, t] = h * gC[:, t]
        y = torch.fft.irfft2(Y, s=(H, W)).reshape(B * T, Ci, H, W) * Fn.silu(z)
        return _planes_out(y, p["out_proj"]).reshape(B, T, H, W, -1)


class GdnCPU:
    """GatedDeltaNetCSSM slow-path forward (cssm.py:4685-5141) in float32 on the CPU,
    factored gates, sinusoid temporal context, RMS output norm, SiLU output gate."""

    def __init__(self, params, channels, delta_key_dim=4, spectral_rho=0.999, qkv_conv_size=1, short_conv_size=4,
                 use_input_gates=True, rope_base=10000.0):
        self.p = params_to_torch(params)
        self.C, self.dk = channels, delta_key_dim
        self.rho = spectral_rho
        self.q = qkv_conv_size
        self.kt = short_conv_size
        self.input_gates = use_input_gates
        self.base = rope_base
        self._what = {}

    def __call__(self, x):
        p, C, dk = self.p, self.C, self.dk
        B, T, H, W, _ = x.shape
        nh, Wf = C // dk, W // 2 + 1
        if (H, W) not in self._what:
            self._what[(H, W)] = spectral_kernel(p["kernel"], H, W, self.rho)
        what = self._what[(H, W)]
        xf = x.reshape(B * T, H, W, C)
        xq = _dwconv_same(xf, p["qkv_dw"]) if self.q > 1 else xf
        qkv = _planes_in(xq, p["qkv_proj"]).reshape(B, T, 3 * C, H, W)
        q, k, v = qkv[:, :, :C], qkv[:, :, C:2 * C], qkv[:, :, 2 * C:]
        if self.kt > 0:
            q = Fn.silu(_causal_t(q, p["short_conv_q"]))
            k = Fn.silu(_causal_t(k, p["short_conv_k"]))
            v = Fn.silu(_causal_t(v, p["short_conv_v"]))
        ctx = x.mean(dim=(2, 3))
        inv = 1.0 / (self.base ** (torch.arange(0, C, 2, dtype=torch.float32) / C))
        th = torch.arange(T, dtype=torch.float32)[:, None] * inv[None]
        ctx = ctx + torch.stack([torch.sin(th), torch.cos(th)], -1).reshape(T, C)[None]

        def fgate(name):
            return torch.sigmoid(_dense(ctx, p[name + "_h"])[..., :, None] + _dense(ctx, p[name + "_w"])[..., None, :])
        if self.input_gates:
            k = k * fgate("B_k")[:, :, None]
            v = v * fgate("B_v")[:, :, None]
        gv = Fn.silu(_planes_in(xf, p["gate_proj"]))                  # (F, C, H, W)
        al = (0.1 + 0.89 * fgate("alpha"))[:, :, None]                 # (B, T, 1, H, Wf)
        be = fgate("beta")[:, :, None]

        def spec(z):                                                   # (B, T, nh, dk, H, Wf)
            return torch.fft.rfft2(z).reshape(B, T, nh, dk, H, Wf)

        def l2(z):
            return z / torch.sqrt((z.abs() ** 2).sum(dim=(4, 5), keepdim=True) + 1e-6)
        qs, ks, vs = l2(spec(q)), l2(spec(k)), spec(v)
        ks = ks / torch.sqrt((ks.abs() ** 2).sum(dim=3, keepdim=True) + 1e-6)
        s = torch.zeros((B, nh, dk, dk, H, Wf), dtype=torch.complex64)     # s[b, n, i, a, u, v]
        O = torch.empty((B, T, nh, dk, H, Wf), dtype=torch.complex64)
        for t in range(T):
            kk = ks[:, t]
            a_t = al[:, t][:, :, None, None] * what[None, :, None, None]
            b_t = be[:, t][:, :, None, None]
            khs = torch.einsum("bnauv,bniauv->bniuv", kk.conj(), s)
            s = a_t * (s - b_t * kk[:, :, None] * khs[:, :, :, None])
            s = s + b_t * vs[:, t][:, :, :, None] * kk.conj()[:, :, None]
            O[:, t] = torch.einsum("bniauv,bnauv->bniuv", s, qs[:, t])
        o = torch.fft.irfft2(O.reshape(B * T, C, H, W // 2 + 1), s=(H, W))   # (F, C, H, W)
        o = o * torch.rsqrt((o ** 2).mean(1, keepdim=True) + 1e-6) * p["rms_scale"][None, :, None, None]
        return _planes_out(o * gv, p["output_proj"]).reshape(B, T, H, W, C)


class GdnRef:
    """GatedDeltaNetCSSM slow-path forward (cssm.py:4685-5141) in torch on the CPU, float64 by
    default, with autograd through every parameter and the input: the gradient reference of the
    training path.  Every gate type, the rms / layer / no output norm, the qkv depthwise conv, the
    short conv and the input gates; M = alpha W (I - beta k k^H) and Delta = beta v k^H are
    materialised per step with to_goom's floor applied entry by entry through torch.where, so a
    floored entry passes no gradient to its inputs (cssm.py:4911-4937, goom.py:161-174), or
    mapped as the scan variant of cfg's use_log / use_goom / scan_mode says (_scan_entries).
    ``cfg`` is the oracle's GDNConfig (rope_mode 'none': the sinusoid context table)."""

    def __init__(self, params, cfg, dtype=torch.float64, requires_grad=True):
        self.p = params_to_torch(params, dtype, requires_grad)
        self.cfg = cfg
        self.dtype = dtype

    def _gate(self, name, ctx, x, H, W, nh, bounded=False, spatial=False):
        p, gt = self.p, self.cfg.gate_type
        B, T, C = ctx.shape
        Wf = W // 2 + 1
        if gt == "channel":
            if spatial:
                q = p[name]
                k2 = q["kernel"].reshape(C, C)
                return torch.sigmoid(x @ k2 + q["bias"])                     # (B, T, H, W, C)
            raw = torch.sigmoid(_dense(ctx, p[name])).reshape(B, T, nh, 1, 1)
        elif gt == "factored":
            raw = torch.sigmoid(_dense(ctx, p[f"{name}_h"])[..., :, None] + _dense(ctx, p[f"{name}_w"])[..., None, :])
            if spatial:
                return raw[..., None]                                        # (B, T, H, W, 1)
            raw = raw.reshape(B, T, 1, H, Wf)
        elif gt == "scalar":
            raw = torch.sigmoid(_dense(ctx, p[name])).reshape(B, T, 1, 1, 1)
            if spatial:
                return raw
        else:
            raw = torch.sigmoid(_dense(ctx, p[name]))
            if spatial:
                return raw.reshape(B, T, H, W, 1)
            raw = raw.reshape(B, T, 1, H, Wf)
        return 0.1 + 0.89 * raw if bounded else raw

    def __call__(self, x):
        p, cfg, dt = self.p, self.cfg, self.dtype
        B, T, H, W, C = x.shape
        dk = cfg.delta_key_dim
        nh, Wf = C // dk, W // 2 + 1
        what = spectral_kernel(p["kernel"], H, W, cfg.spectral_rho, squash=not cfg.no_spectral_clamp)
        xf = x.reshape(B * T, H, W, C)
        if cfg.qkv_conv_size > 1 and not cfg.qkv_conv_separable:
            qkv = _conv_same(xf, p["qkv_proj"]).reshape(B, T, H, W, 3 * C)
        else:
            xq = _dwconv_same(xf, p["qkv_dw"]) if cfg.qkv_conv_size > 1 else xf
            qkv = _dense(xq, p["qkv_proj"]).reshape(B, T, H, W, 3 * C)
        q, k, v = qkv[..., :C], qkv[..., C:2 * C], qkv[..., 2 * C:]
        if cfg.short_conv_size > 0:
            def conv(z, name):                                               # channels-last -> plane-major and back
                zp = z.permute(0, 1, 4, 2, 3)
                return Fn.silu(_causal_t(zp, p[name])).permute(0, 1, 3, 4, 2)
            q, k, v = conv(q, "short_conv_q"), conv(k, "short_conv_k"), conv(v, "short_conv_v")
        inv = 1.0 / (cfg.rope_base ** (torch.arange(0, C, 2, dtype=torch.float64) / C))
        th = torch.arange(T, dtype=torch.float64)[:, None] * inv[None]
        ctx = x.mean(dim=(2, 3)) + torch.stack([torch.sin(th), torch.cos(th)], -1).reshape(T, C).to(dt)[None]
        if cfg.use_input_gates:
            k = k * self._gate("B_k", ctx, x, H, W, nh, spatial=True)
            v = v * self._gate("B_v", ctx, x, H, W, nh, spatial=True)
        gv = _dense(x, p["gate_proj"])
        gv = Fn.silu(gv) if cfg.output_gate_act == "silu" else torch.sigmoid(gv)
        al = self._gate("alpha", ctx, x, H, W, nh, bounded=True).expand(B, T, nh, H, Wf)
        be = self._gate("beta", ctx, x, H, W, nh).expand(B, T, nh, H, Wf)

        def spec(z):                                                         # (B, T, nh, dk, H, Wf)
            return torch.fft.rfft2(z.permute(0, 1, 4, 2, 3)).reshape(B, T, nh, dk, H, Wf)

        def l2(z):
            if not cfg.use_spectral_l2_norm:
                return z
            return z / torch.sqrt((z.real ** 2 + z.imag ** 2).sum(dim=(4, 5), keepdim=True) + 1e-6)
        qs, ks, vs = l2(spec(q)), l2(spec(k)), spec(v)
        ks = ks / torch.sqrt((ks.real ** 2 + ks.imag ** 2).sum(dim=3, keepdim=True) + 1e-6)
        eye = torch.eye(dk, dtype=dt)[None, None, :, :, None, None]
        variant = _gdn_variant(cfg)
        s = torch.zeros((B, nh, dk, dk, H, Wf), dtype=qs.dtype)              # s[b, n, i, r, u, v]
        outs = []
        for t in range(T):
            kk = ks[:, t]                                                    # (B, nh, dk, H, Wf)
            aw = al[:, t][:, :, None, None] * what[None, :, None, None]      # (B, nh, 1, 1, H, Wf)
            b_t = be[:, t][:, :, None, None]
            M = _scan_entries(aw * (eye - b_t * kk[:, :, :, None] * kk.conj()[:, :, None, :]), variant)
            D = _scan_entries(b_t * vs[:, t][:, :, :, None] * kk.conj()[:, :, None, :], variant)   # D[b, n, i, r]
            s = torch.einsum("bnrcuv,bnicuv->bniruv", M, s) + D
            outs.append(torch.einsum("bniruv,bnruv->bniuv", s, qs[:, t]))
        O = torch.stack(outs, dim=1)                                         # (B, T, nh, dk, H, Wf)
        o = torch.fft.irfft2(O.reshape(B, T, C, H, Wf), s=(H, W)).permute(0, 1, 3, 4, 2)   # (B, T, H, W, C)
        if cfg.output_norm == "rms":
            o = o * torch.rsqrt((o * o).mean(dim=-1, keepdim=True) + 1e-6) * p["rms_scale"]
        elif cfg.output_norm == "layer":
            mu = o.mean(dim=-1, keepdim=True)
            var = ((o - mu) ** 2).mean(dim=-1, keepdim=True)
            o = (o - mu) * torch.rsqrt(var + 1e-6) * p["output_layernorm"]["scale"] + p["output_layernorm"]["bias"]
        return _dense(o * gv, p["output_proj"])


def _gdn_variant(cfg):
    """The scan variant of a GDNConfig (cssm.py:4939-4991), as the oracle's gdn_scan_variant."""
    if cfg.scan_mode == "pallas" and cfg.delta_key_dim == 2:
        return "linear"
    if not cfg.use_log:
        return "linear"
    return "goom" if cfg.use_goom else "log_eps"


def gdn_bins_core(spec, ab, what, gate_type, dk, variant="goom"):
    """The contract of cssm_gdn_scan_bins_train (cssm.py:4898-5000): spec (B, T, 3C, H, Wf) with q
    and k already scaled by the spectral L2 norms, ab (B, T, n_ab, 2) (alpha, beta) laid out per
    gate type, what (n_h, H, Wf).  Per-bin key norm, M and Delta mapped as the scan variant says
    (floored by default, torch.where), s_t = M s_{t-1} + Delta, o_t = s_t q.  Returns ohat
    (B, T, C, H, Wf)."""
    B, T, C3, H, Wf = spec.shape
    C = C3 // 3
    nh = C // dk
    q = spec[:, :, :C].reshape(B, T, nh, dk, H, Wf)
    k = spec[:, :, C:2 * C].reshape(B, T, nh, dk, H, Wf)
    v = spec[:, :, 2 * C:].reshape(B, T, nh, dk, H, Wf)
    k = k / torch.sqrt((k.real ** 2 + k.imag ** 2).sum(dim=3, keepdim=True) + 1e-6)
    shp = {"dense": (B, T, 1, H, Wf), "factored": (B, T, 1, H, Wf), "channel": (B, T, nh, 1, 1),
           "scalar": (B, T, 1, 1, 1)}[gate_type]
    al = ab[..., 0].reshape(shp).expand(B, T, nh, H, Wf)
    be = ab[..., 1].reshape(shp).expand(B, T, nh, H, Wf)
    eye = torch.eye(dk, dtype=ab.dtype)[None, None, :, :, None, None]
    s = torch.zeros((B, nh, dk, dk, H, Wf), dtype=spec.dtype)
    outs = []
    for t in range(T):
        kk = k[:, t]
        aw = al[:, t][:, :, None, None] * what[None, :, None, None]
        b_t = be[:, t][:, :, None, None]
        M = _scan_entries(aw * (eye - b_t * kk[:, :, :, None] * kk.conj()[:, :, None, :]), variant)
        D = _scan_entries(b_t * v[:, t][:, :, :, None] * kk.conj()[:, :, None, :], variant)
        s = torch.einsum("bnrcuv,bnicuv->bniruv", M, s) + D
        outs.append(torch.einsum("bniruv,bnruv->bniuv", s, q[:, t]))
    return torch.stack(outs, dim=1).reshape(B, T, C, H, Wf)
