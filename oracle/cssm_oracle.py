"""CPU restatement of the CSSM spectral state-space layer (gated and GDN cells).

TEST INFRASTRUCTURE ONLY.  This module is the parity checker for the HIP
kernels in ``cssm_amd``.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it, and only as the checker or
the reported CPU baseline -- never as the thing that is measured or shipped.
The product path (``cssm_amd``) never imports this file.

It restates, in float64 numpy, the algorithm of the reference JAX/Flax code
(``/root/reference`` = drewlinsley/CSSM, read as text; JAX/Flax are not
installed here, so the reference itself cannot be run).  Every function cites
the reference lines it follows.

Pinning (see ``tests/test_oracle.py``): numpy pocketfft vs a brute-force DFT
matrix evaluation (incl. odd / non-power-of-2 sizes), the K=1 closed form of
the spectral kernel, the T=1 closed form of the gated core, the static-gate
geometric-series closed form of the recurrence, a faithful GOOM log-space scan
(to_goom / log_add_exp with the reference floors) against the linear scan,
circular-shift equivariance, causality, the GDN T=1 closed form, the unit
key-norm invariant, and the reference's published parameter counts.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Dict, Optional

import numpy as np

# ---------------------------------------------------------------------------
# numerics helpers
# ---------------------------------------------------------------------------

GOOM_EPS = 1e-7                                   # goom.py:161 (to_goom eps)
FLT_MIN = float(np.finfo(np.float32).tiny)        # jnp.finfo(float32).smallest_normal
GOOM_FINITE_FLOOR = 2.0 * math.log(FLT_MIN)       # goom.py:99-100  (= -174.67)


def silu(x):
    """jax.nn.silu: x * sigmoid(x)."""
    return x * sigmoid(x)


def sigmoid(x):
    x = np.asarray(x, dtype=np.float64)
    return 0.5 * (1.0 + np.tanh(0.5 * x))


def softplus(x):
    """jax.nn.softplus = logaddexp(x, 0)."""
    return np.logaddexp(x, 0.0)


def gate_activation(x, kind: str):
    """GatedCSSM._compute_gate (cssm.py:432-441)."""
    if kind == 'softplus':
        return softplus(x)
    if kind == 'sigmoid':
        return sigmoid(x) * 2.0
    if kind == 'exp':
        return np.exp(np.clip(x, -4.0, 2.0))
    return softplus(x)


def stable_spectral_magnitude(K, rho=0.999):
    """_stable_spectral_magnitude (cssm.py:29-46): K * rho / (1 + |K|)."""
    return K * rho / (1.0 + np.abs(K))


def rms_norm(x, weight, eps=1e-6):
    """_rms_norm (cssm.py:49-52): x * rsqrt(mean(x^2, -1) + eps) * weight."""
    ms = np.mean(x ** 2, axis=-1, keepdims=True)
    return x / np.sqrt(ms + eps) * weight


def layer_norm(x, scale, bias, eps=1e-6):
    """flax.linen.LayerNorm over the last axis (epsilon 1e-6)."""
    mu = np.mean(x, axis=-1, keepdims=True)
    var = np.mean((x - mu) ** 2, axis=-1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * scale + bias


def goom_floor(x):
    """to_goom's complex-safe floor (goom.py:161-174): |x| < 1e-7 -> 1e-7 + 0j."""
    x = np.asarray(x, dtype=np.complex128)
    return np.where(np.abs(x) < GOOM_EPS, GOOM_EPS + 0j, x)


def to_goom(x):
    """to_goom + goom_log (goom.py:89-137, 144-178): floored complex log."""
    lg = np.log(goom_floor(x))
    re = np.where(lg.real < GOOM_FINITE_FLOOR, GOOM_FINITE_FLOOR, lg.real)
    return re + 1j * lg.imag


def from_goom(lx):
    """from_goom (goom.py:181-196): complex exp."""
    return np.exp(lx)


def log_add_exp(a, b):
    """operations.log_add_exp (operations.py:17-41): max shift, exp, add, floored log."""
    c = np.maximum(a.real, b.real)
    s = from_goom(a - c) + from_goom(b - c)
    return to_goom(s) + c


def dense(x, p):
    """flax.linen.Dense: x @ kernel + bias (kernel shape (in, out))."""
    y = np.tensordot(x, p['kernel'], axes=([-1], [0]))
    if 'bias' in p:
        y = y + p['bias']
    return y


def same_pad(k):
    """lax 'SAME' padding for stride 1: low=(k-1)//2, high=k//2."""
    return (k - 1) // 2, k // 2


def depthwise_conv2d_same(x, p):
    """nn.Conv(C, (k,k), feature_group_count=C, padding='SAME') on (N,H,W,C).

    Cross-correlation (no flip); kernel HWIO (k,k,1,C); bias (C,).
    """
    kern = p['kernel']
    kh, kw = kern.shape[0], kern.shape[1]
    lo_h, hi_h = same_pad(kh)
    lo_w, hi_w = same_pad(kw)
    N, H, W, C = x.shape
    xp = np.pad(x, ((0, 0), (lo_h, hi_h), (lo_w, hi_w), (0, 0)))
    out = np.zeros_like(x, dtype=np.float64)
    for i in range(kh):
        for j in range(kw):
            out += xp[:, i:i + H, j:j + W, :] * kern[i, j, 0, :]
    if 'bias' in p:
        out = out + p['bias']
    return out


def full_conv2d_same(x, p):
    """nn.Conv(Cout, (k,k), padding='SAME') with full channel mixing; kernel (k,k,Cin,Cout)."""
    kern = p['kernel']
    kh, kw = kern.shape[0], kern.shape[1]
    lo_h, hi_h = same_pad(kh)
    lo_w, hi_w = same_pad(kw)
    N, H, W, C = x.shape
    xp = np.pad(x, ((0, 0), (lo_h, hi_h), (lo_w, hi_w), (0, 0)))
    out = np.zeros((N, H, W, kern.shape[3]), dtype=np.float64)
    for i in range(kh):
        for j in range(kw):
            out += np.tensordot(xp[:, i:i + H, j:j + W, :], kern[i, j], axes=([-1], [0]))
    if 'bias' in p:
        out = out + p['bias']
    return out


def causal_conv_t(x5, p):
    """Causal depthwise temporal conv (cssm.py:494-500, 4766-4776).

    x5 (B,T,H,W,C); kernel (k,1,C); out[t] = sum_j w_j x[t-k+1+j] + b, zeros for t<0.
    """
    kern = p['kernel']
    k = kern.shape[0]
    B, T, H, W, C = x5.shape
    xp = np.concatenate([np.zeros((B, k - 1, H, W, C)), x5], axis=1)
    out = np.zeros_like(x5, dtype=np.float64)
    for j in range(k):
        out += xp[:, j:j + T] * kern[j, 0, :]
    if 'bias' in p:
        out = out + p['bias']
    return out


# ---------------------------------------------------------------------------
# FFT conventions (jnp.fft.rfft2 / irfft2 = numpy pocketfft semantics)
# ---------------------------------------------------------------------------

def rfft2(x):
    """Unnormalised forward real 2-D FFT over the last two axes (cssm.py:533)."""
    return np.fft.rfft2(np.asarray(x, dtype=np.float64), axes=(-2, -1))


def irfft2(X, H, W):
    """irfft2(X, s=(H,W)) over the last two axes (cssm.py:577).

    C2R rule: complex inverse over H, then a real inverse over W that keeps only
    Re of the v=0 column (and of v=W/2 for even W).
    """
    return np.fft.irfft2(np.asarray(X, dtype=np.complex128), s=(H, W), axes=(-2, -1))


def rfft2_bruteforce(x):
    """Brute-force DFT-matrix evaluation of rfft2 (for pinning pocketfft)."""
    x = np.asarray(x, dtype=np.float64)
    H, W = x.shape[-2:]
    Wf = W // 2 + 1
    FH = np.exp(-2j * np.pi * np.outer(np.arange(H), np.arange(H)) / H)
    FW = np.exp(-2j * np.pi * np.outer(np.arange(W), np.arange(Wf)) / W)
    return np.einsum('uh,...hw,wv->...uv', FH, x, FW)


def irfft2_bruteforce(X, H, W):
    """Brute-force evaluation of the C2R rule written out in closed form.

    Z[h,v] = (1/H) sum_u X[u,v] e^{+2pi i u h/H}
    y[h,w] = (1/W) [Re Z[h,0] + 2 sum_{0<v<W/2} Re(Z[h,v] e^{2pi i v w/W})
                    + (W even) (-1)^w Re Z[h,W/2]]
    """
    X = np.asarray(X, dtype=np.complex128)
    Wf = W // 2 + 1
    FHi = np.exp(2j * np.pi * np.outer(np.arange(H), np.arange(H)) / H) / H
    Z = np.einsum('hu,...uv->...hv', FHi, X)
    w = np.arange(W)
    y = np.repeat(Z[..., :, 0:1].real, W, axis=-1).astype(np.float64)
    vmax = (W - 1) // 2  # last fully doubled bin
    for v in range(1, vmax + 1):
        y = y + 2.0 * (Z[..., :, v:v + 1] * np.exp(2j * np.pi * v * w / W)).real
    if W % 2 == 0:
        y = y + Z[..., :, Wf - 1:Wf].real * ((-1.0) ** w)
    return y / W


# ---------------------------------------------------------------------------
# spectral kernel
# ---------------------------------------------------------------------------

def pad_kernel(k, H, W):
    """Kernel pad / crop rule (cssm.py:510-526, GDN pad_kernel 4698-4709).

    K <= H: zero-pad with pad_before = (H-K)//2; K > H: centre crop at (K-H)//2.
    k: (C, K, K) -> (C, H, W).
    """
    K = k.shape[-1]
    if K > H or K > W:
        sh = (K - H) // 2
        sw = (K - W) // 2
        return k[:, sh:sh + H, sw:sw + W]
    ph = max(0, (H - K) // 2)
    pw = max(0, (W - K) // 2)
    return np.pad(k, ((0, 0), (ph, max(0, H - K - ph)), (pw, max(0, W - K - pw))))


def spectral_kernel(k, H, W, rho=0.999, squash=True):
    """K_hat = rho * F / (1 + |F|), F = rfft2(pad(k)) (cssm.py:505-529, 4711-4716)."""
    F = rfft2(pad_kernel(np.asarray(k, dtype=np.float64), H, W))
    return stable_spectral_magnitude(F, rho) if squash else F


# ---------------------------------------------------------------------------
# scans
# ---------------------------------------------------------------------------

def linear_scalar_scan(A, V):
    """h_t = A_t h_{t-1} + V_t over axis 1, h_{-1} = 0 (the algebra of cssm.py:570-575)."""
    h = np.zeros_like(V[:, 0])
    out = np.empty_like(V)
    for t in range(V.shape[1]):
        h = A[:, t] * h + V[:, t]
        out[:, t] = h
    return out


def goom_scalar_scan(K_log, U_log):
    """Faithful log-space prefix over axis 1 with cssm_scalar_scan_op (math.py:24-54).

    Evaluated sequentially (the associative scan computes the same prefix up to
    rounding order): (k, u) o (k', u') = (k + k', log_add_exp(k' + u, u')).
    """
    k = K_log[:, 0]
    u = U_log[:, 0]
    out = np.empty_like(U_log)
    out[:, 0] = u
    for t in range(1, U_log.shape[1]):
        kj, uj = K_log[:, t], U_log[:, t]
        u = log_add_exp(kj + u, uj)
        k = kj + k
        out[:, t] = u
    return out


# ---------------------------------------------------------------------------
# gated cell (GatedCSSM._forward_depthwise, cssm.py:476-585)
# ---------------------------------------------------------------------------

@dataclass
class GatedConfig:
    """GatedCSSM attributes (cssm.py:416-430) + the build's `expand` (A.6 of the design)."""
    channels: int
    kernel_size: int = 15
    spectral_rho: float = 0.999
    gate_activation: str = 'softplus'
    rope_mode: str = 'none'
    short_conv_size: int = 4
    short_conv_spatial_size: int = 3
    gate_type: str = 'dense'
    dense_mixing: bool = False
    expand: int = 1


def gated_gates(ctx, params, cfg: GatedConfig, H, W):
    """Per-frequency gates from ctx (cssm.py:536-556): returns (Delta, G_B, G_C), each (B,T,H,Wf)."""
    Wf = W // 2 + 1
    B, T, _ = ctx.shape

    def make(name):
        if cfg.gate_type == 'factored':
            gh = dense(ctx, params[f'{name}_h'])
            gw = dense(ctx, params[f'{name}_w'])
            return gh[..., :, None] * gw[..., None, :]
        return dense(ctx, params[name]).reshape(B, T, H, Wf)

    delta = gate_activation(make('delta_proj'), cfg.gate_activation)
    return delta, make('B_proj'), make('C_proj')


def gated_core(xm_act, z_gate, khat, delta, gB, gC, scan='linear'):
    """The spectral core between the in_proj split and out_proj (cssm.py:531-581).

    xm_act: (B,T,C,H,W) post-activation x_main (plane-major)
    z_gate: (B,T,C,H,W) multiplier applied after irfft2 (= SiLU(z)), or None
    khat  : (C,H,Wf) complex squashed spectral kernel
    delta, gB, gC: (B,T,H,Wf) gates (broadcast over C)
    Returns (B,T,C,H,W) = irfft2(gC * h) * z_gate with h_t = A_t h_{t-1} + V_t,
    A = floor(K_hat) e^{-Delta}, V = (Delta + 1e-8) floor(gB * U_hat).
    scan='goom' evaluates the recurrence exactly as the reference does, in GOOM log space.
    """
    B, T, C, H, W = xm_act.shape
    U = rfft2(xm_act)                                   # (B,T,C,H,Wf)
    d = delta[:, :, None]
    if scan == 'goom':
        K_log = to_goom(khat)[None, None]               # cssm.py:559-560
        K_log = np.broadcast_to(K_log, U.shape)
        U_log = to_goom(U * gB[:, :, None])             # cssm.py:562-563
        K_g = (K_log.real - d) + 1j * K_log.imag        # cssm.py:566
        U_g = (U_log.real + np.log(d + 1e-8)) + 1j * U_log.imag  # cssm.py:567
        X = from_goom(goom_scalar_scan(K_g, U_g))       # cssm.py:570-575
    else:
        A = goom_floor(khat)[None, None] * np.exp(-d)
        V = (d + 1e-8) * goom_floor(U * gB[:, :, None])
        X = linear_scalar_scan(A, V)
    Y = X * gC[:, :, None]                              # cssm.py:576
    y = irfft2(Y, H, W)                                 # cssm.py:577
    if z_gate is not None:
        y = y * z_gate
    return y


def gated_forward(params, x, cfg: GatedConfig, scan='linear', return_intermediates=False):
    """GatedCSSM forward (cssm.py:443-474, 476-585); x (B,T,H,W,C_in) channels-last."""
    if cfg.rope_mode != 'none':
        raise NotImplementedError('rope_mode != none is outside the restated path')
    if cfg.dense_mixing:
        raise NotImplementedError('dense_mixing is outside the restated path')
    x = np.asarray(x, dtype=np.float64)
    B, T, H, W, Cin = x.shape
    Ci = cfg.channels * cfg.expand
    xz = dense(x, params['in_proj'])                    # cssm.py:481
    x_main, z = xz[..., :Ci], xz[..., Ci:]              # cssm.py:483-484
    if cfg.short_conv_spatial_size > 0:                 # cssm.py:487-492
        x_main = depthwise_conv2d_same(x_main.reshape(B * T, H, W, Ci),
                                       params['short_conv_spatial']).reshape(B, T, H, W, Ci)
    if cfg.short_conv_size > 0:                         # cssm.py:494-500
        x_main = causal_conv_t(x_main, params['short_conv_temporal'])
    x_main = silu(x_main)                               # cssm.py:502
    khat = spectral_kernel(params['kernel'], H, W, cfg.spectral_rho)   # cssm.py:505-529
    ctx = x_main.mean(axis=(2, 3))                      # cssm.py:536
    delta, gB, gC = gated_gates(ctx, params, cfg, H, W)
    xm_pm = x_main.transpose(0, 1, 4, 2, 3)             # cssm.py:532
    zg_pm = silu(z).transpose(0, 1, 4, 2, 3)            # cssm.py:581 (SiLU(z))
    y_pm = gated_core(xm_pm, zg_pm, khat, delta, gB, gC, scan=scan)
    y = y_pm.transpose(0, 1, 3, 4, 2)                   # cssm.py:578
    out = dense(y, params['out_proj'])                  # cssm.py:584
    if return_intermediates:
        return out, dict(x_main=x_main, z=z, ctx=ctx, khat=khat, delta=delta, gB=gB, gC=gC,
                         y_core=y_pm)
    return out


def gated_param_shapes(cfg: GatedConfig, c_in, H, W) -> Dict[str, Dict[str, tuple]]:
    """Parameter tree of GatedCSSM (Flax names; Dense kernel (in,out), Conv HWIO)."""
    Ci = cfg.channels * cfg.expand
    Wf = W // 2 + 1
    s = {'in_proj': {'kernel': (c_in, 2 * Ci), 'bias': (2 * Ci,)}}
    if cfg.short_conv_spatial_size > 0:
        k = cfg.short_conv_spatial_size
        s['short_conv_spatial'] = {'kernel': (k, k, 1, Ci), 'bias': (Ci,)}
    if cfg.short_conv_size > 0:
        s['short_conv_temporal'] = {'kernel': (cfg.short_conv_size, 1, Ci), 'bias': (Ci,)}
    s['kernel'] = (Ci, cfg.kernel_size, cfg.kernel_size)
    for g in ('delta_proj', 'B_proj', 'C_proj'):
        if cfg.gate_type == 'factored':
            s[f'{g}_h'] = {'kernel': (Ci, H), 'bias': (H,)}
            s[f'{g}_w'] = {'kernel': (Ci, Wf), 'bias': (Wf,)}
        else:
            s[g] = {'kernel': (Ci, H * Wf), 'bias': (H * Wf,)}
    s['out_proj'] = {'kernel': (Ci, cfg.channels), 'bias': (cfg.channels,)}
    return s


# ---------------------------------------------------------------------------
# GDN cell (GatedDeltaNetCSSM slow path, cssm.py:4685-5141)
# ---------------------------------------------------------------------------

@dataclass
class GDNConfig:
    """GatedDeltaNetCSSM attributes used by the slow path (cssm.py:4298-4338)."""
    channels: int
    delta_key_dim: int = 2
    kernel_size: int = 11
    rope_mode: str = 'none'
    rope_base: float = 10000.0
    spectral_rho: float = 0.999
    gate_type: str = 'channel'
    use_goom: bool = True
    use_log: bool = True
    scan_mode: str = 'associative'
    short_conv_size: int = 4
    output_norm: str = 'rms'
    use_input_gates: bool = True
    output_gate_act: str = 'silu'
    use_spectral_l2_norm: bool = True
    qkv_conv_size: int = 1
    qkv_conv_separable: bool = True
    cross_freq_conv_size: int = 0
    no_spectral_clamp: bool = False
    int_attention_mode: str = 'none'
    gate_proj_bias_init: float = 0.0


def temporal_context_encoding(T, C, base=10000.0):
    """apply_temporal_rope_to_context's additive table E (cssm.py:353-383): E[t,2j]=sin, E[t,2j+1]=cos."""
    t_pos = np.arange(T, dtype=np.float64)
    dim = np.arange(0, C, 2, dtype=np.float64)
    inv_freq = 1.0 / (base ** (dim / C))
    theta = np.outer(t_pos, inv_freq)
    return np.stack([np.sin(theta), np.cos(theta)], axis=-1).reshape(T, C)


def gdn_gate(name, params, cfg: GDNConfig, ctx, gate_input, H, W, bounded=False, spatial=False):
    """_gate (cssm.py:4798-4842)."""
    B, T, C = ctx.shape
    dk = cfg.delta_key_dim
    nh = C // dk
    Wf = W // 2 + 1
    gt = cfg.gate_type
    if gt == 'channel':
        if spatial:
            # nn.Conv(C, (1,1)) on the gate input: a per-pixel Dense C->C (kernel (1,1,C,C))
            pc = params[name]
            p2 = {'kernel': pc['kernel'].reshape(pc['kernel'].shape[-2], pc['kernel'].shape[-1]),
                  'bias': pc['bias']}
            return sigmoid(dense(gate_input, p2))                       # (B,T,H,W,C)
        raw = sigmoid(dense(ctx, params[name])).reshape(B, T, nh, 1, 1)
        return 0.1 + 0.89 * raw if bounded else raw
    if gt == 'factored':
        if spatial:
            row = dense(ctx, params[f'{name}_h'])
            col = dense(ctx, params[f'{name}_w'])
            return sigmoid(row[..., :, None] + col[..., None, :]).reshape(B, T, H, W, 1)
        row = dense(ctx, params[f'{name}_h'])
        col = dense(ctx, params[f'{name}_w'])
        raw = sigmoid(row[..., :, None] + col[..., None, :]).reshape(B, T, 1, H, Wf)
        return 0.1 + 0.89 * raw if bounded else raw
    if gt == 'scalar':
        raw = sigmoid(dense(ctx, params[name])).reshape(B, T, 1, 1, 1)
        if spatial:
            return raw
        return 0.1 + 0.89 * raw if bounded else raw
    # 'dense'
    if spatial:
        return sigmoid(dense(ctx, params[name])).reshape(B, T, H, W, 1)
    raw = sigmoid(dense(ctx, params[name])).reshape(B, T, 1, H, Wf)
    return 0.1 + 0.89 * raw if bounded else raw


def gdn_prologue(params, x, cfg: GDNConfig):
    """Everything of the GDN slow path before the rfft2 (cssm.py:4713-4869).

    Returns dict with q_in, k_in, v_in (B,T,H,W,C), gate_val (B,T,H,W,C),
    alpha, beta (broadcastable to (B,T,n_h|1,H|1,Wf|1)), W_hat (n_h,H,Wf).
    """
    if cfg.rope_mode not in ('none', 'learned_t'):
        raise NotImplementedError('rope_mode other than none/learned_t is outside the restated path')
    x = np.asarray(x, dtype=np.float64)
    B, T, H, W, C = x.shape
    dk = cfg.delta_key_dim
    assert C % dk == 0
    W_hat = spectral_kernel(params['kernel'], H, W, cfg.spectral_rho,
                            squash=not cfg.no_spectral_clamp)          # cssm.py:4711-4716
    x_flat = x.reshape(B * T, H, W, C)
    if cfg.qkv_conv_size > 1:                                           # cssm.py:4740-4754
        if cfg.qkv_conv_separable:
            qkv = dense(depthwise_conv2d_same(x_flat, params['qkv_dw']), params['qkv_proj'])
        else:
            qkv = full_conv2d_same(x_flat, params['qkv_proj'])
    else:
        qkv = dense(x_flat, params['qkv_proj'])
    qkv = qkv.reshape(B, T, H, W, 3 * C)
    q_in, k_in, v_in = qkv[..., :C], qkv[..., C:2 * C], qkv[..., 2 * C:]
    if cfg.short_conv_size > 0:                                          # cssm.py:4763-4780
        q_in = silu(causal_conv_t(q_in, params['short_conv_q']))
        k_in = silu(causal_conv_t(k_in, params['short_conv_k']))
        v_in = silu(causal_conv_t(v_in, params['short_conv_v']))
    ctx = x.mean(axis=(2, 3))                                            # cssm.py:4785
    if cfg.rope_mode == 'learned_t':
        ctx = ctx + params['temporal_embed'][None]                       # cssm.py:4787-4791
    else:
        ctx = ctx + temporal_context_encoding(T, C, cfg.rope_base)[None]  # cssm.py:4793
    if cfg.use_input_gates:                                              # cssm.py:4844-4848
        k_in = k_in * gdn_gate('B_k', params, cfg, ctx, x, H, W, spatial=True)
        v_in = v_in * gdn_gate('B_v', params, cfg, ctx, x, H, W, spatial=True)
    gv = dense(x_flat, params['gate_proj']).reshape(B, T, H, W, C)      # cssm.py:4853-4855
    gate_val = silu(gv) if cfg.output_gate_act == 'silu' else sigmoid(gv)
    alpha = gdn_gate('alpha', params, cfg, ctx, x, H, W, bounded=True)   # cssm.py:4864
    beta = gdn_gate('beta', params, cfg, ctx, x, H, W)                   # cssm.py:4865
    return dict(q_in=q_in, k_in=k_in, v_in=v_in, gate_val=gate_val, alpha=alpha,
                beta=beta, W_hat=W_hat, ctx=ctx)


def _gate_bins(g, B, T, nh, H, Wf):
    """alpha/beta broadcast to (B,T,n_h,H,Wf): 'channel' gates are (B,T,n_h,1,1),
    the others (B,T,1,H,Wf) or (B,T,1,1,1) (cssm.py:4918-4923)."""
    return np.broadcast_to(g, (B, T, nh, H, Wf))


def gdn_spectral_norms(q_spec, k_spec, cfg: GDNConfig):
    """Spectral and key-vector L2 norms (cssm.py:4890-4906); specs (B,T,nh,dk,H,Wf)."""
    def spec_norm(z):
        if not cfg.use_spectral_l2_norm:
            return z
        n = np.sqrt(np.sum(np.abs(z) ** 2, axis=(4, 5), keepdims=True) + 1e-6)
        return z / n
    k = spec_norm(k_spec)
    k = k / np.sqrt(np.sum(np.abs(k) ** 2, axis=3, keepdims=True) + 1e-6)
    return spec_norm(q_spec), k


def gdn_scan_variant(cfg: GDNConfig):
    """Which evaluation of the delta-rule scan the slow path takes (cssm.py:4939-4991):
    'linear'  scan_mode='pallas' at d_k=2 (pallas_matrix_2x2_scan) or use_log=False (the direct
              complex scan): the recurrence on M and Delta as they are, no floors;
    'goom'    use_log and use_goom: to_goom on every M / Delta entry (|x| < 1e-7 -> 1e-7 + 0j);
    'log_eps' use_log without use_goom: log(|x| + 1e-8) + i angle(x) on every entry
              (cssm.py:4697-4699), exp afterwards.
    The log-space combine (log_matmul / log_add_exp, operations.py:17-61, 314-390) evaluates the
    linear recurrence on those entries (to_goom of an intermediate sum binds only at a relative
    cancellation below 1e-7 of its largest term)."""
    if cfg.scan_mode == 'pallas' and cfg.delta_key_dim == 2:
        return 'linear'
    if not cfg.use_log:
        return 'linear'
    return 'goom' if cfg.use_goom else 'log_eps'


def gdn_scan_entries(z, variant):
    """M / Delta entries as the chosen scan sees them after its log map and exp (cssm.py:4693-4701,
    4945-4958): 'goom' to_goom's floor; 'log_eps' exp(log(|z| + 1e-8) + i angle(z)); 'linear'
    unchanged.  A zero entry under 'log_eps' becomes 1e-8 + 0j here: the reference's angle is
    atan2(Im, Re), which gives 0 or +-pi for the signed zeros its FFT and complex products happen
    to leave, so its value there is +-1e-8 depending on sign bits the algorithm does not fix."""
    if variant == 'goom':
        return goom_floor(z)
    if variant == 'log_eps':
        z = np.asarray(z)
        mapped = np.exp(np.log(np.abs(z) + 1e-8) + 1j * np.angle(z))
        return np.where(z == 0, 1e-8 + 0j, mapped)
    if variant == 'linear':
        return z
    raise ValueError(variant)


def gdn_matrix_scan(M, D):
    """s_t = M_t s_{t-1} + Delta_t[i, :], s_{-1} = 0 (math.py:384-411 in linear algebra).
    M (B,T,nh,H,Wf,dk,dk) [row a, column b]; D (B,T,nh,dv,H,Wf,dk); returns S like D."""
    B, T, nh, dv, H, Wf, dk = D.shape
    s = np.zeros((B, nh, dv, H, Wf, dk), dtype=np.complex128)
    S = np.empty((B, T, nh, dv, H, Wf, dk), dtype=np.complex128)
    for t in range(T):
        s = np.einsum('znuvab,zniuvb->zniuva', M[:, t], s) + D[:, t]
        S[:, t] = s
    return S


def gdn_core(q_in, k_in, v_in, alpha, beta, W_hat, cfg: GDNConfig, scan='linear'):
    """rfft2 -> norms -> delta-rule matrix scan -> readout -> irfft2 (cssm.py:4875-5025).

    q_in/k_in/v_in: (B,T,H,W,C) channels-last; returns o_spatial (B,T,C,H,W).
    scan='linear': materialises M_t and Delta_t, maps every entry as the configured scan
    sees it (gdn_scan_variant: to_goom's floors, log(|x| + 1e-8), or nothing) and runs the
    complex linear recurrence s_t = M_t s_{t-1} + Delta_t[i,:] (exact algebra of the
    log-space scan); scan='rank1': the same recurrence in rank-1 form without
    materialising M and with no map on M or Delta entries -- equal to 'linear'
    wherever no floor binds.
    """
    B, T, H, W, C = q_in.shape
    dk = cfg.delta_key_dim
    dv = dk
    nh = C // dk
    Wf = W // 2 + 1

    def heads(z):
        return z.reshape(B, T, H, W, nh, dk).transpose(0, 1, 4, 5, 2, 3)
    q_spec, k_spec, v_spec = rfft2(heads(q_in)), rfft2(heads(k_in)), rfft2(heads(v_in))
    q_n, k_n = gdn_spectral_norms(q_spec, k_spec, cfg)
    al = _gate_bins(alpha, B, T, nh, H, Wf)
    be = _gate_bins(beta, B, T, nh, H, Wf)
    if scan == 'linear':
        a_bc = al[:, :, :, None, None]                                         # (B,T,nh,1,1,H,Wf)
        b_bc = be[:, :, :, None, None]
        Wh = W_hat[None, None, :, None, None, :, :]
        k_outer = k_n[..., :, None, :, :] * np.conj(k_n[..., None, :, :, :])   # (B,T,nh,dk,dk,H,Wf)
        I = np.eye(dk).reshape(1, 1, 1, dk, dk, 1, 1)
        M = a_bc * Wh * (I - b_bc * k_outer)                                   # cssm.py:4925
        vk = v_spec[..., :, None, :, :] * np.conj(k_n[..., None, :, :, :])    # (B,T,nh,dv,dk,H,Wf)
        D = b_bc * vk                                                          # cssm.py:4927-4929
        variant = gdn_scan_variant(cfg)                                        # cssm.py:4939-4991
        M = gdn_scan_entries(M, variant)
        D = gdn_scan_entries(D, variant)
        S = gdn_matrix_scan(np.moveaxis(M, (3, 4), (5, 6)),   # (B,T,nh,H,Wf,dk,dk)
                            np.moveaxis(D, (4,), (6,)))       # (B,T,nh,dv,H,Wf,dk)
    else:
        s = np.zeros((B, nh, dv, dk, H, Wf), dtype=np.complex128)   # s[..., i, a, u, v]
        S = np.empty((B, T, nh, dv, H, Wf, dk), dtype=np.complex128)
        for t in range(T):
            kk = k_n[:, t]                                             # (B,nh,dk,H,Wf)
            a_t = al[:, t][:, :, None, None]                           # (B,nh,1,1,H,Wf)
            b_t = be[:, t][:, :, None, None]
            khs = np.einsum('bnauv,bniauv->bniuv', np.conj(kk), s)     # k^H s_i
            s = a_t * W_hat[None, :, None, None] * (s - b_t * kk[:, :, None] * khs[:, :, :, None])
            s = s + b_t * v_spec[:, t][:, :, :, None] * np.conj(kk)[:, :, None]
            S[:, t] = np.moveaxis(s, 3, 5)
    q_read = q_n.transpose(0, 1, 2, 4, 5, 3)[:, :, :, None]              # cssm.py:4998
    o_hat = np.sum(S * q_read, axis=-1).reshape(B, T, C, H, Wf)          # cssm.py:4999-5000
    if cfg.cross_freq_conv_size > 0:
        raise NotImplementedError('cross_freq_conv is outside the restated path')
    return irfft2(o_hat, H, W)                                           # cssm.py:5025


def gdn_forward(params, x, cfg: GDNConfig, scan='linear', return_intermediates=False):
    """GatedDeltaNetCSSM slow-path forward (cssm.py:4685-5141)."""
    if cfg.int_attention_mode != 'none':
        raise NotImplementedError('InT attention modes are outside the restated path')
    pro = gdn_prologue(params, x, cfg)
    o = gdn_core(pro['q_in'], pro['k_in'], pro['v_in'], pro['alpha'], pro['beta'],
                 pro['W_hat'], cfg, scan=scan)
    out = o.transpose(0, 1, 3, 4, 2)                                     # cssm.py:5026
    if cfg.output_norm == 'rms':
        out = rms_norm(out, params['rms_scale'])                         # cssm.py:5029-5031
    elif cfg.output_norm == 'layer':
        out = layer_norm(out, params['output_layernorm']['scale'], params['output_layernorm']['bias'])
    out = out * pro['gate_val']                                          # cssm.py:5126
    res = dense(out, params['output_proj'])                              # cssm.py:5141
    if return_intermediates:
        pro['o_spatial'] = o
        return res, pro
    return res


# ---------------------------------------------------------------------------
# CSSMSHViTBlock wiring (cssm_shvit.py:86-229), the token-mixer half
# ---------------------------------------------------------------------------

BLOCK_NORM_AXES = {'global_layer': (1, 2, 3, 4), 'temporal_layer': (1, 4), 'layer': (4,)}


def block_norm1(x5, scale, bias, block_norm='global_layer', eps=1e-6):
    """norm1 of CSSMSHViTBlock (cssm_shvit.py:104-114): flax LayerNorm with
    reduction axes (1, 2, 3, 4) ('global_layer'), (1, 4) ('temporal_layer') or
    the channel axis ('layer', per frame), feature axis -1 (per-channel scale and
    bias), epsilon 1e-6 and flax's fast variance E[x^2] - E[x]^2."""
    axes = BLOCK_NORM_AXES[block_norm]
    mu = np.mean(x5, axis=axes, keepdims=True)
    var = np.maximum(np.mean(x5 * x5, axis=axes, keepdims=True) - mu * mu, 0.0)
    return (x5 - mu) / np.sqrt(var + eps) * scale + bias


def gelu_tanh(x):
    """jax.nn.gelu with its default approximate=True (the tanh form)."""
    return 0.5 * x * (1.0 + np.tanh(math.sqrt(2.0 / math.pi) * (x + 0.044715 * x ** 3)))


def timestep_gate_pool(params, residual, y):
    """timestep_gate (cssm_shvit.py:195-210): softmax pooling of the cell's T frames with
    logits from [mean of the first input frame, mean of frame t] through gate_fc1 -> gelu
    -> gate_fc2, plus a prior of 4 on the last frame.  residual, y (B, T, H, W, C)."""
    T = y.shape[1]
    q = residual[:, 0].mean(axis=(1, 2))                                  # (B, C)
    k = y.mean(axis=(2, 3))                                               # (B, T, C)
    gate_in = np.concatenate([np.broadcast_to(q[:, None], k.shape), k], axis=-1)
    h = gelu_tanh(dense(gate_in, params['gate_fc1']))
    logits = dense(h, params['gate_fc2'])[..., 0]
    prior = np.zeros(T)
    prior[-1] = 4.0
    z = logits + prior
    w = np.exp(z - z.max(axis=-1, keepdims=True))
    w = w / w.sum(axis=-1, keepdims=True)
    return np.einsum('bt,bthwc->bhwc', w, y)


def shvit_mlp_half(params, x, use_dwconv=True):
    """The block's second half (cssm_shvit.py:231-266, Mlp shvit.py:156-182): x + fc2(h'),
    h = gelu(fc1(LayerNorm_norm2(x))), h' = h + dwconv(h) (depthwise 3 x 3 'SAME')."""
    shp = x.shape
    x4 = x.reshape(-1, *shp[-3:])                                          # frames as batch (:241-244)
    h = flax_layer_norm(x4, params['norm2'])
    h = gelu_tanh(dense(h, params['mlp']['fc1']))
    if use_dwconv:
        h = h + depthwise_conv2d_same(h, params['mlp']['dwconv']['dwconv'])
    h = dense(h, params['mlp']['fc2'])
    return x + h.reshape(shp)


def shvit_block(params, x, cell_forward, num_timesteps=8, block_norm='global_layer', use_pos_conv=True,
                output_act='none', timestep_gate=False, use_dwconv=True):
    """CSSMSHViTBlock.__call__ (cssm_shvit.py:65-266): the token mixer, then norm2 -> Mlp -> residual."""
    x = shvit_block_mixer(params, x, cell_forward, num_timesteps, block_norm, use_pos_conv, output_act,
                          timestep_gate)
    return shvit_mlp_half(params, x, use_dwconv)


def shvit_block_mixer(params, x, cell_forward, num_timesteps=8, block_norm='global_layer',
                      use_pos_conv=True, output_act='none', timestep_gate=False):
    """CSSMSHViTBlock.__call__ up to the token-mixer residual (cssm_shvit.py:86-228).

    x (B, H, W, C) image -> repeated to (B, T, H, W, C) (:99-101), or (B, T, H, W, C)
    video; residual = that 5-D input (:104); norm1 (:106-114); pos_conv: depthwise
    3 x 3 'SAME' per frame, added (:132-145); the cell (:185) by ``cell_forward(p, x5)``;
    the last frame for an image, every frame for video (keep_time, :191-213);
    output_act (:215-218); + the matching residual (:220-228).
    """
    is_image = x.ndim == 4
    x5 = np.repeat(x[:, None], num_timesteps, axis=1) if is_image else x
    residual = x5
    h = block_norm1(x5, params['norm1']['scale'], params['norm1']['bias'], block_norm)
    if use_pos_conv:
        B, T, H, W, C = h.shape
        h = h + depthwise_conv2d_same(h.reshape(B * T, H, W, C), params['pos_conv']).reshape(h.shape)
    y = cell_forward(params['cssm'], h)
    if timestep_gate:                                                     # :195-210
        y = timestep_gate_pool(params, x5, y)
        is_image = True                                                   # T collapsed (:191)
    else:
        y = y[:, -1] if is_image else y
    if output_act == 'gelu':
        y = gelu_tanh(y)
    elif output_act == 'silu':
        y = silu(y)
    return (residual[:, -1] if is_image else residual) + y


def gdn_param_shapes(cfg: GDNConfig, H, W) -> Dict[str, object]:
    """Parameter tree of GatedDeltaNetCSSM's slow path (Flax names)."""
    C = cfg.channels
    dk = cfg.delta_key_dim
    nh = C // dk
    Wf = W // 2 + 1
    s: Dict[str, object] = {'kernel': (nh, cfg.kernel_size, cfg.kernel_size)}
    q = cfg.qkv_conv_size
    if q > 1:
        if cfg.qkv_conv_separable:
            s['qkv_dw'] = {'kernel': (q, q, 1, C), 'bias': (C,)}
            s['qkv_proj'] = {'kernel': (C, 3 * C), 'bias': (3 * C,)}
        else:
            s['qkv_proj'] = {'kernel': (q, q, C, 3 * C), 'bias': (3 * C,)}
    else:
        s['qkv_proj'] = {'kernel': (C, 3 * C), 'bias': (3 * C,)}
    if cfg.short_conv_size > 0:
        for n in ('q', 'k', 'v'):
            s[f'short_conv_{n}'] = {'kernel': (cfg.short_conv_size, 1, C), 'bias': (C,)}
    if cfg.rope_mode == 'learned_t':
        s['temporal_embed'] = None   # (T, C): resolution of T known only at init
    gt = cfg.gate_type

    def gate(name, spatial):
        if gt == 'channel':
            if spatial:
                s[name] = {'kernel': (1, 1, C, C), 'bias': (C,)}
            else:
                s[name] = {'kernel': (C, nh), 'bias': (nh,)}
        elif gt == 'factored':
            s[f'{name}_h'] = {'kernel': (C, H), 'bias': (H,)}
            s[f'{name}_w'] = {'kernel': (C, W if spatial else Wf), 'bias': (W if spatial else Wf,)}
        elif gt == 'scalar':
            s[name] = {'kernel': (C, 1), 'bias': (1,)}
        else:
            n = H * W if spatial else H * Wf
            s[name] = {'kernel': (C, n), 'bias': (n,)}
    if cfg.use_input_gates:
        gate('B_k', True)
        gate('B_v', True)
    s['gate_proj'] = {'kernel': (C, C), 'bias': (C,)}
    gate('alpha', False)
    gate('beta', False)
    if cfg.output_norm == 'rms':
        s['rms_scale'] = (C,)
    elif cfg.output_norm == 'layer':
        s['output_layernorm'] = {'scale': (C,), 'bias': (C,)}
    s['output_proj'] = {'kernel': (C, C), 'bias': (C,)}
    return s


def count_params(shapes) -> int:
    n = 0
    for v in shapes.values():
        if isinstance(v, dict):
            n += count_params(v)
        elif v is not None:
            n += int(np.prod(v))
    return n


# ---------------------------------------------------------------------------
# seeded parameter draws (reference init *distributions*; numpy PCG64)
# ---------------------------------------------------------------------------

def _fan_in(shape):
    if len(shape) == 2:
        return shape[0]
    if len(shape) == 4:          # HWIO
        return shape[0] * shape[1] * shape[2]
    if len(shape) == 3:          # (k, 1, C) temporal conv: fan_in = k * 1
        return shape[0] * shape[1]
    return shape[0]


def init_params(shapes, rng: np.random.Generator, bias_std=0.1, spectral_std=None,
                spectral_init='normal', gate_proj_bias_init=None):
    """Draw a parameter tree: lecun-normal kernels, N(0, bias_std^2) biases
    (non-zero so the bias paths are exercised), spectral `kernel` N(0,0.02^2) (gated,
    cssm.py:506-510) or xavier-normal (GDN, cssm.py:4717), `rms_scale` around 1."""
    out = {}
    for name, v in shapes.items():
        if isinstance(v, dict):
            sub = {}
            for pn, shp in v.items():
                if pn == 'kernel':
                    std = 1.0 / math.sqrt(max(1, _fan_in(shp)))
                    sub[pn] = rng.standard_normal(shp) * std
                elif pn == 'scale':
                    sub[pn] = 1.0 + 0.1 * rng.standard_normal(shp)
                else:
                    sub[pn] = rng.standard_normal(shp) * bias_std
            out[name] = sub
        elif v is None:
            continue
        elif name == 'kernel':
            if spectral_init == 'xavier':
                nh, K, _ = v
                std = math.sqrt(2.0 / (2.0 * K * nh))
            else:
                std = 0.02 if spectral_std is None else spectral_std
            out[name] = rng.standard_normal(v) * std
        elif name == 'rms_scale':
            out[name] = 1.0 + 0.1 * rng.standard_normal(v)
        else:
            out[name] = rng.standard_normal(v) * 0.1
    return out


# ---------------------------------------------------------------------------
# SimpleCSSM caller (simple_cssm.py:63-558): stem -> cells with residual ->
# readout, for the cells of this path (gated / gdn / gdn_d2 / gdn_d3) and the
# position embeddings that add no RoPE ('none', 'learnable')
# ---------------------------------------------------------------------------

@dataclass
class SimpleConfig:
    """SimpleCSSM attributes that shape the computation around the cells."""
    num_classes: int = 2
    embed_dim: int = 32
    depth: int = 1
    cssm_type: str = 'gated'
    kernel_size: int = 15
    frame_readout: str = 'last'
    norm_type: str = 'layer'
    stem_norm: str = ''
    body_norm: str = ''
    pos_embed: str = 'none'
    act_type: str = 'softplus'
    pool_type: str = 'mean'
    seq_len: int = 8
    n_register_tokens: int = 0
    stem_mode: str = 'default'
    stem_layers: int = 2
    stem_norm_order: str = 'post'
    readout_norm: str = 'pre'
    inter_mlp_ratio: float = 0.0
    gate_type: str = 'dense'
    short_conv_size: int = 4
    short_conv_spatial_size: int = 3
    delta_key_dim: int = 2
    output_norm: str = 'rms'
    use_input_gates: bool = True
    output_gate_act: str = 'silu'
    use_spectral_l2_norm: bool = True
    qkv_conv_size: int = 1
    no_spectral_clamp: bool = False


def simple_cell_config(cfg: SimpleConfig):
    """The cell config SimpleCSSM builds for block i (simple_cssm.py:325-443)."""
    if cfg.cssm_type == 'gated':
        return GatedConfig(channels=cfg.embed_dim, kernel_size=cfg.kernel_size, gate_type=cfg.gate_type,
                           short_conv_size=cfg.short_conv_size,
                           short_conv_spatial_size=cfg.short_conv_spatial_size)
    dk = {'gdn_d2': 2, 'gdn_d3': 3}.get(cfg.cssm_type, cfg.delta_key_dim)
    return GDNConfig(channels=cfg.embed_dim, delta_key_dim=dk, kernel_size=cfg.kernel_size, gate_type=cfg.gate_type,
                     short_conv_size=cfg.short_conv_size, output_norm=cfg.output_norm,
                     use_input_gates=cfg.use_input_gates, output_gate_act=cfg.output_gate_act,
                     use_spectral_l2_norm=cfg.use_spectral_l2_norm, qkv_conv_size=cfg.qkv_conv_size,
                     no_spectral_clamp=cfg.no_spectral_clamp)


def _act(x, kind):
    """SimpleCSSM._get_act (simple_cssm.py:155-164): softplus / gelu (tanh form) / relu."""
    if kind == 'gelu':
        return gelu_tanh(x)
    if kind == 'relu':
        return np.maximum(x, 0.0)
    return softplus(x)


def flax_layer_norm(x, p, axes=(-1,), eps=1e-6):
    """flax LayerNorm: stats over `axes` with the fast variance E[x^2] - E[x]^2 (clipped at 0),
    per-channel scale and bias on the last axis."""
    mu = np.mean(x, axis=axes, keepdims=True)
    var = np.maximum(np.mean(x * x, axis=axes, keepdims=True) - mu * mu, 0.0)
    return (x - mu) / np.sqrt(var + eps) * p['scale'] + p['bias']


def simple_norm(x, kind, p, stats=None, training=False):
    """_apply_norm (simple_cssm.py:192-235)."""
    if kind == 'batch':
        # flax BatchNorm (epsilon 1e-5): running statistics in inference, batch statistics otherwise
        if training:
            axes = tuple(range(x.ndim - 1))
            mu = np.mean(x, axis=axes)
            var = np.maximum(np.mean(x * x, axis=axes) - mu * mu, 0.0)
        else:
            mu, var = stats['mean'], stats['var']
        return (x - mu) / np.sqrt(var + 1e-5) * p['scale'] + p['bias']
    if kind == 'instance':
        # GroupNorm(num_groups=C): one group per channel, stats over every non-batch axis but C
        # (flax GroupNorm reduces over axes 1..ndim-2 and the size-1 within-group axis).  A pooled
        # (B, C) vector leaves only the within-group axis: each group is one element, mean = x and
        # var = 0, so the output is the bias.
        axes = tuple(range(1, x.ndim - 1))
        if not axes:
            return (x - x) / np.sqrt(0.0 + 1e-6) * p['scale'] + p['bias']
        return flax_layer_norm(x, p, axes=axes)
    if x.ndim == 5 and kind == 'temporal_layer':
        return flax_layer_norm(x, p, axes=(1, 4))
    if x.ndim == 5 and kind == 'global_layer':
        return flax_layer_norm(x, p, axes=(1, 2, 3, 4))
    if x.ndim == 5 and kind == 'global_instance':
        return flax_layer_norm(x, p, axes=(1, 2, 3))
    return flax_layer_norm(x, p)


def conv2d_same(x, p):
    """flax Conv with 'SAME' padding, stride 1, bias: (N, H, W, Cin) -> (N, H, W, Cout)."""
    return full_conv2d_same(x, p)


def max_pool_2x2_same(x):
    """nn.max_pool(window (2, 2), strides (2, 2), 'SAME') on (N, H, W, C): odd sizes pad
    the far edge with -inf."""
    N, H, W, C = x.shape
    Ho, Wo = (H + 1) // 2, (W + 1) // 2
    xp = np.full((N, 2 * Ho, 2 * Wo, C), -np.inf)
    xp[:, :H, :W] = x
    return xp.reshape(N, Ho, 2, Wo, 2, C).max(axis=(2, 4))


def simple_param_shapes(cfg: SimpleConfig, x_shape):
    """SimpleCSSM parameter tree (Flax names) and batch_stats for input (B, [T,] H, W, C_in)."""
    H, W, cin = x_shape[-3], x_shape[-2], x_shape[-1]
    D = cfg.embed_dim
    stem_norm = cfg.stem_norm or cfg.norm_type
    body_norm = cfg.body_norm or cfg.norm_type
    p: Dict[str, object] = {}
    bs: Dict[str, object] = {}

    def norm(name, c, kind):
        p[name] = {'scale': (c,), 'bias': (c,)}
        if kind == 'batch':
            bs[name] = {'mean': (c,), 'var': (c,)}
    if cfg.stem_mode == 'pathtracker':
        p['conv1'] = {'kernel': (1, 1, cin, D), 'bias': (D,)}
        norm('norm1', cin if cfg.stem_norm_order == 'pre' else D, stem_norm)
    else:
        c = cin
        for i in range(cfg.stem_layers):
            norm(f'norm{i + 1}', c if cfg.stem_norm_order == 'pre' else D, stem_norm)
            p[f'conv{i + 1}'] = {'kernel': (3, 3, c, D), 'bias': (D,)}
            c = D
            H, W = (H + 1) // 2, (W + 1) // 2
    if cfg.pos_embed == 'learnable':
        p['pos_embed'] = (1, 1, H, W, D)
    if cfg.n_register_tokens > 0:
        p['register_tokens'] = (1, cfg.n_register_tokens, H, W, D)
    ccfg = simple_cell_config(cfg)
    for i in range(cfg.depth):
        p[f'cssm_{i}'] = (gated_param_shapes(ccfg, D, H, W) if cfg.cssm_type == 'gated'
                          else gdn_param_shapes(ccfg, H, W))
        if cfg.depth > 1 and i < cfg.depth - 1:
            norm(f'body_norm_{i}', D, body_norm)
            if cfg.inter_mlp_ratio > 0:
                hid = int(D * cfg.inter_mlp_ratio)
                p[f'mlp_{i}_up'] = {'kernel': (D, hid), 'bias': (hid,)}
                p[f'mlp_{i}_down'] = {'kernel': (hid, D), 'bias': (D,)}
    norm('norm_pre', D, body_norm)
    norm('norm_post', D, body_norm)
    p['head'] = {'kernel': (D, cfg.num_classes), 'bias': (cfg.num_classes,)}
    return p, bs


def simple_cssm_forward(params, x, cfg: SimpleConfig, batch_stats=None, training=False,
                        return_features=False, return_spatial=False, injected_post_cssm=None):
    """SimpleCSSM.__call__ (simple_cssm.py:166-558) for the cells of this path."""
    if cfg.pos_embed not in ('none', 'learnable'):
        raise NotImplementedError('RoPE position embeddings are outside the restated path')
    act = lambda v: _act(v, cfg.act_type)                      # noqa: E731
    stem_norm = cfg.stem_norm or cfg.norm_type
    body_norm = cfg.body_norm or cfg.norm_type
    bs = batch_stats or {}

    def norm(v, kind, name):
        return simple_norm(v, kind, params[name], bs.get(name), training)
    x = np.asarray(x, dtype=np.float64)
    if x.ndim == 4:                                                         # :239-240
        x = np.repeat(x[:, None], cfg.seq_len, axis=1)
    B, T, H, W, C = x.shape
    x = x.reshape(B * T, H, W, C)                                           # :245

    def norm_act(v, name):                                                  # :247-255
        if cfg.stem_norm_order == 'pre':
            return act(norm(v, stem_norm, name))
        return norm(act(v), stem_norm, name)
    if cfg.stem_mode == 'pathtracker':                                      # :257-264
        if cfg.stem_norm_order == 'pre':
            x = conv2d_same(norm_act(x, 'norm1'), params['conv1'])
        else:
            x = norm_act(conv2d_same(x, params['conv1']), 'norm1')
    else:                                                                   # :266-274
        for i in range(cfg.stem_layers):
            if cfg.stem_norm_order == 'pre':
                x = conv2d_same(norm_act(x, f'norm{i + 1}'), params[f'conv{i + 1}'])
            else:
                x = norm_act(conv2d_same(x, params[f'conv{i + 1}']), f'norm{i + 1}')
            x = max_pool_2x2_same(x)
    _, Hn, Wn, D = x.shape
    x = x.reshape(B, T, Hn, Wn, D)                                          # :277-278
    if cfg.pos_embed == 'learnable':                                        # :281-285
        x = x + params['pos_embed']
    nreg = cfg.n_register_tokens
    if nreg > 0:                                                            # :302-306
        reg = np.broadcast_to(params['register_tokens'], (B, nreg, Hn, Wn, D))
        x = np.concatenate([reg, x], axis=1)
    ccfg = simple_cell_config(cfg)
    for i in range(cfg.depth):                                              # :319-496
        cp = params[f'cssm_{i}']
        y = gated_forward(cp, x, ccfg) if cfg.cssm_type == 'gated' else gdn_forward(cp, x, ccfg)
        x = x + y                                                           # :482
        if cfg.depth > 1 and i < cfg.depth - 1:                             # :486-496
            x = act(norm(x, body_norm, f'body_norm_{i}'))
            if cfg.inter_mlp_ratio > 0:
                h = act(dense(x, params[f'mlp_{i}_up']))
                x = x + dense(h, params[f'mlp_{i}_down'])
    if injected_post_cssm is not None:                                      # :500-501
        x = np.asarray(injected_post_cssm, dtype=np.float64)
    if return_features:                                                     # :502-503
        return x
    if nreg > 0:                                                            # :507-508
        x = x[:, nreg:]
    if return_spatial:                                                      # :510-521
        x = act(norm(x, body_norm, 'norm_pre')) if cfg.readout_norm == 'pre' else \
            norm(act(x), body_norm, 'norm_pre')
        return dense(x, params['head'])
    if cfg.frame_readout == 'last':                                         # :524-527
        x = x[:, -1]
    if cfg.readout_norm == 'pre':                                           # :530-535
        x = act(norm(x, body_norm, 'norm_pre'))
    else:
        x = norm(act(x), body_norm, 'norm_pre')
    axes = (1, 2) if cfg.frame_readout == 'last' else (1, 2, 3)             # :538-549
    x = x.max(axis=axes) if cfg.pool_type == 'max' else x.mean(axis=axes)
    x = norm(x, body_norm, 'norm_post')                                     # :552
    return dense(x, params['head'])                                         # :555
