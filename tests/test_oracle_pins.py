"""Pins of the oracle's small helpers, each shown to catch a named mistake.

Every pin is a plain check on ``oracle.cssm_oracle``.  The first test of each
pair runs it on the oracle as it is and must pass; the second plants the named
mistake in the oracle module (monkeypatched, CPU only) and requires the same
check to fail, so a pin that a plausible mistake would slip past is caught
here.  The facts each check uses come from the reference text:

  causal_conv_t     cssm.py:494-500, 4766-4776 (left pad k-1, VALID conv,
                    a cross-correlation: out[t] = sum_j w[j] x[t - (k-1) + j])
  gated_gates       cssm.py:538-545 (factored: g_h[u] * g_w[v]; dense:
                    Dense(H*Wf).reshape(H, Wf)); :548-556 (only Delta activated)
  gate_activation   cssm.py:432-441 (softplus; 2 sigmoid; exp(clip(x, -4, 2));
                    anything else softplus)
  gdn_gate          cssm.py:4798-4842 (sigmoid(row[u] + col[v]); bounded
                    0.1 + 0.89 sigmoid; spatial gates over W, spectral over Wf)
  rms_norm          cssm.py:49-52 with the call at :5029-5031 (last axis = C)
  layer_norm        flax LayerNorm at cssm.py:5033 (last axis, epsilon 1e-6)
"""
import math

import numpy as np
import pytest

from oracle import cssm_oracle as O


# --------------------------------------------------------------- causal conv

def pin_causal_conv_tap_order():
    """An impulse at frame t0 puts tap j at frame t0 + k - 1 - j (plus the bias everywhere)."""
    k, T, C = 4, 9, 3
    w = np.arange(1.0, 1.0 + k * C).reshape(k, 1, C)          # distinct taps per channel
    b = np.array([0.5, -0.25, 0.125])
    for t0 in (0, 3, T - 1):
        x = np.zeros((1, T, 1, 1, C))
        x[0, t0] = 1.0
        out = O.causal_conv_t(x, {"kernel": w, "bias": b})[0, :, 0, 0, :]
        expect = np.tile(b, (T, 1))
        for j in range(k):
            t = t0 + k - 1 - j
            if t < T:
                expect[t] += w[j, 0]
        assert np.array_equal(out, expect), f"tap order wrong for an impulse at t0={t0}"
    # causality of the zero padding: nothing before the impulse sees it
    x = np.zeros((1, T, 1, 1, C))
    x[0, 5] = 1.0
    out = O.causal_conv_t(x, {"kernel": w, "bias": np.zeros(C)})
    assert np.all(out[0, :5] == 0.0)


def _conv_reversed_taps(x5, p):
    q = dict(p, kernel=p["kernel"][::-1].copy())
    return _orig_causal_conv_t(x5, q)


_orig_causal_conv_t = O.causal_conv_t


def test_causal_conv_tap_order():
    pin_causal_conv_tap_order()


def test_causal_conv_pin_catches_reversed_taps(monkeypatch):
    monkeypatch.setattr(O, "causal_conv_t", _conv_reversed_taps)
    with pytest.raises(AssertionError):
        pin_causal_conv_tap_order()


# ----------------------------------------------------------- gate activation

def pin_gate_activation():
    big = 60.0
    assert O.gate_activation(np.array(0.0), "softplus") == pytest.approx(math.log(2.0), abs=1e-15)
    assert O.gate_activation(np.array(big), "softplus") == pytest.approx(big, abs=1e-12)
    assert O.gate_activation(np.array(-big), "softplus") == pytest.approx(0.0, abs=1e-20)
    # 2 sigmoid: range (0, 2), 1 at 0
    assert O.gate_activation(np.array(big), "sigmoid") == pytest.approx(2.0, abs=1e-12)
    assert O.gate_activation(np.array(-big), "sigmoid") == pytest.approx(0.0, abs=1e-20)
    assert O.gate_activation(np.array(0.0), "sigmoid") == pytest.approx(1.0, abs=1e-15)
    # bounded exp: clip to [-4, 2] first
    assert O.gate_activation(np.array(-10.0), "exp") == pytest.approx(math.exp(-4.0), rel=1e-15)
    assert O.gate_activation(np.array(10.0), "exp") == pytest.approx(math.exp(2.0), rel=1e-15)
    assert O.gate_activation(np.array(1.0), "exp") == pytest.approx(math.e, rel=1e-15)
    assert O.gate_activation(np.array(-3.0), "exp") == pytest.approx(math.exp(-3.0), rel=1e-15)
    # an unknown name falls back to softplus (cssm.py:440-441)
    assert O.gate_activation(np.array(0.0), "relu") == pytest.approx(math.log(2.0), abs=1e-15)


def _act_sigmoid_unscaled(x, kind):
    return O.sigmoid(x) if kind == "sigmoid" else _orig_gate_activation(x, kind)


def _act_exp_unclipped(x, kind):
    return np.exp(x) if kind == "exp" else _orig_gate_activation(x, kind)


def _act_exp_clip_swapped(x, kind):
    return np.exp(np.clip(x, -2.0, 4.0)) if kind == "exp" else _orig_gate_activation(x, kind)


def _act_unknown_identity(x, kind):
    return x if kind not in ("softplus", "sigmoid", "exp") else _orig_gate_activation(x, kind)


_orig_gate_activation = O.gate_activation


def test_gate_activation_values():
    pin_gate_activation()


@pytest.mark.parametrize("mutant", [_act_sigmoid_unscaled, _act_exp_unclipped, _act_exp_clip_swapped,
                                    _act_unknown_identity])
def test_gate_activation_pin_catches(mutant, monkeypatch):
    monkeypatch.setattr(O, "gate_activation", mutant)
    with pytest.raises(AssertionError):
        pin_gate_activation()


# ---------------------------------------------------------- gated cell gates

def _gated_zero_kernel_params(cfg, C, H, W, rng):
    shapes = O.gated_param_shapes(cfg, C, H, W)
    p = O.init_params(shapes, rng)
    for g in ("delta_proj", "B_proj", "C_proj"):
        for suffix in (("_h", "_w") if cfg.gate_type == "factored" else ("",)):
            p[g + suffix]["kernel"] = np.zeros_like(p[g + suffix]["kernel"])
    return p


def pin_gated_gates():
    rng = np.random.default_rng(7)
    H, W, C, B, T = 6, 10, 5, 2, 3
    Wf = W // 2 + 1
    # factored, zero kernels: the gate of every frame is exactly b_h (x) b_w
    cfg = O.GatedConfig(channels=C, gate_type="factored", gate_activation="softplus")
    p = _gated_zero_kernel_params(cfg, C, H, W, rng)
    ctx = rng.standard_normal((B, T, C))
    delta, gB, gC = O.gated_gates(ctx, p, cfg, H, W)
    for g, name in ((gB, "B_proj"), (gC, "C_proj")):
        expect = np.outer(p[name + "_h"]["bias"], p[name + "_w"]["bias"])
        assert g.shape == (B, T, H, Wf)
        assert np.array_equal(g, np.broadcast_to(expect, g.shape)), f"{name}: factored bias gate"
    d_expect = O.softplus(np.outer(p["delta_proj_h"]["bias"], p["delta_proj_w"]["bias"]))
    assert np.array_equal(delta, np.broadcast_to(d_expect, delta.shape)), "Delta = act(g_h g_w)"
    # B and C are unconstrained (cssm.py:551-555): negative values survive
    assert gB.min() < 0 and gC.min() < 0
    # factored with random kernels: every frame's gate matrix is rank 1
    p = O.init_params(O.gated_param_shapes(cfg, C, H, W), rng)
    _, gB, gC = O.gated_gates(ctx, p, cfg, H, W)
    for g in (gB, gC):
        for b in range(B):
            for t in range(T):
                s = np.linalg.svd(g[b, t], compute_uv=False)
                assert s[1] <= 1e-12 * s[0], "factored gate is not rank 1"
    # dense: a one-hot bias at index u * Wf + v lands on bin (u, v)
    cfg = O.GatedConfig(channels=C, gate_type="dense", gate_activation="softplus")
    p = _gated_zero_kernel_params(cfg, C, H, W, rng)
    for u, v in ((0, 0), (1, 4), (H - 1, Wf - 1), (4, 2)):
        for g in ("delta_proj", "B_proj", "C_proj"):
            p[g]["bias"] = np.zeros(H * Wf)
            p[g]["bias"][u * Wf + v] = 3.0
        delta, gB, gC = O.gated_gates(ctx, p, cfg, H, W)
        hot = np.zeros((H, Wf))
        hot[u, v] = 3.0
        assert np.array_equal(gB[0, 0], hot) and np.array_equal(gC[1, 2], hot), f"dense bin ({u},{v})"
        assert np.array_equal(delta[0, 1], O.softplus(hot))


def _gates_sum_form(ctx, params, cfg, H, W):
    """Mistake: the factored gate as g_h[u] + g_w[v] (the GDN form) instead of the product."""
    if cfg.gate_type != "factored":
        return _orig_gated_gates(ctx, params, cfg, H, W)

    def make(name):
        gh = O.dense(ctx, params[f"{name}_h"])
        gw = O.dense(ctx, params[f"{name}_w"])
        return gh[..., :, None] + gw[..., None, :]
    return O.gate_activation(make("delta_proj"), cfg.gate_activation), make("B_proj"), make("C_proj")


def _gates_dense_transposed(ctx, params, cfg, H, W):
    """Mistake: the dense gate reshaped column-major ((Wf, H) then transposed)."""
    if cfg.gate_type != "dense":
        return _orig_gated_gates(ctx, params, cfg, H, W)
    Wf = W // 2 + 1
    B, T, _ = ctx.shape

    def make(name):
        return np.swapaxes(O.dense(ctx, params[name]).reshape(B, T, Wf, H), -1, -2)
    return O.gate_activation(make("delta_proj"), cfg.gate_activation), make("B_proj"), make("C_proj")


def _gates_b_activated(ctx, params, cfg, H, W):
    """Mistake: the activation applied to B as well as Delta."""
    d, gB, gC = _orig_gated_gates(ctx, params, cfg, H, W)
    return d, O.gate_activation(gB, cfg.gate_activation), gC


_orig_gated_gates = O.gated_gates


def test_gated_gates_layout():
    pin_gated_gates()


@pytest.mark.parametrize("mutant", [_gates_sum_form, _gates_dense_transposed, _gates_b_activated])
def test_gated_gates_pin_catches(mutant, monkeypatch):
    monkeypatch.setattr(O, "gated_gates", mutant)
    with pytest.raises(AssertionError):
        pin_gated_gates()


# ------------------------------------------------------------------ GDN gates

def _gdn_zero_kernel(p):
    for v in p.values():
        if isinstance(v, dict) and "kernel" in v:
            v["kernel"] = np.zeros_like(v["kernel"])
    return p


def pin_gdn_gate():
    rng = np.random.default_rng(11)
    B, T, H, W, C, dk = 2, 2, 6, 8, 8, 2
    Wf, nh = W // 2 + 1, C // dk
    ctx = rng.standard_normal((B, T, C))
    x = rng.standard_normal((B, T, H, W, C))
    # factored, zero kernels: sigmoid(b_h[u] + b_w[v]); spectral over Wf, spatial over W
    cfg = O.GDNConfig(channels=C, delta_key_dim=dk, gate_type="factored")
    p = _gdn_zero_kernel(O.init_params(O.gdn_param_shapes(cfg, H, W), rng))
    beta = O.gdn_gate("beta", p, cfg, ctx, x, H, W)
    expect = O.sigmoid(p["beta_h"]["bias"][:, None] + p["beta_w"]["bias"][None, :])
    assert beta.shape[-2:] == (H, Wf)
    assert np.allclose(np.broadcast_to(beta, (B, T, 1, H, Wf)), expect, rtol=0, atol=1e-15), "factored logit"
    bk = O.gdn_gate("B_k", p, cfg, ctx, x, H, W, spatial=True)
    expect = O.sigmoid(p["B_k_h"]["bias"][:, None] + p["B_k_w"]["bias"][None, :])
    assert bk.shape == (B, T, H, W, 1)
    assert np.allclose(bk[..., 0], expect, rtol=0, atol=1e-15), "factored spatial logit"
    # bounded alpha: 0.1 + 0.89 sigmoid -> 0.1 and 0.99 at bias -inf / +inf, 0.545 at 0
    for lim, want in ((-80.0, 0.1), (80.0, 0.99), (0.0, 0.545)):
        p["alpha_h"]["bias"] = np.full(H, lim / 2)
        p["alpha_w"]["bias"] = np.full(Wf, lim / 2)
        a = O.gdn_gate("alpha", p, cfg, ctx, x, H, W, bounded=True)
        assert np.allclose(a, want, rtol=0, atol=1e-14), f"bounded gate at bias {lim}"
    # the unbounded beta reaches 0 and 1
    for lim, want in ((-80.0, 0.0), (80.0, 1.0)):
        p["beta_h"]["bias"] = np.full(H, lim / 2)
        p["beta_w"]["bias"] = np.full(Wf, lim / 2)
        assert np.allclose(O.gdn_gate("beta", p, cfg, ctx, x, H, W), want, rtol=0, atol=1e-14)
    # channel: one gate per head, broadcast over the plane
    cfg = O.GDNConfig(channels=C, delta_key_dim=dk, gate_type="channel")
    p = _gdn_zero_kernel(O.init_params(O.gdn_param_shapes(cfg, H, W), rng))
    a = O.gdn_gate("alpha", p, cfg, ctx, x, H, W, bounded=True)
    assert a.shape == (B, T, nh, 1, 1)
    assert np.allclose(a[0, 0, :, 0, 0], 0.1 + 0.89 * O.sigmoid(p["alpha"]["bias"]), rtol=0, atol=1e-15)
    # dense: a one-hot logit at u * Wf + v lands on bin (u, v)
    cfg = O.GDNConfig(channels=C, delta_key_dim=dk, gate_type="dense")
    p = _gdn_zero_kernel(O.init_params(O.gdn_param_shapes(cfg, H, W), rng))
    p["beta"]["bias"] = np.full(H * Wf, -80.0)
    p["beta"]["bias"][2 * Wf + 3] = 80.0
    g = O.gdn_gate("beta", p, cfg, ctx, x, H, W)
    hot = np.zeros((H, Wf))
    hot[2, 3] = 1.0
    assert np.allclose(g[1, 1, 0], hot, rtol=0, atol=1e-14)


def _gdn_gate_bound_09(name, params, cfg, ctx, gate_input, H, W, bounded=False, spatial=False):
    """Mistake: bounded gates as 0.1 + 0.9 sigmoid (upper bound 1.0)."""
    g = _orig_gdn_gate(name, params, cfg, ctx, gate_input, H, W, bounded=False, spatial=spatial)
    return 0.1 + 0.9 * g if bounded and not spatial else g


def _gdn_gate_product_logit(name, params, cfg, ctx, gate_input, H, W, bounded=False, spatial=False):
    """Mistake: the factored logit as row[u] * col[v] (the gated cell's form)."""
    if cfg.gate_type != "factored":
        return _orig_gdn_gate(name, params, cfg, ctx, gate_input, H, W, bounded, spatial)
    B, T, _ = ctx.shape
    row = O.dense(ctx, params[f"{name}_h"])
    col = O.dense(ctx, params[f"{name}_w"])
    raw = O.sigmoid(row[..., :, None] * col[..., None, :])
    if spatial:
        return raw.reshape(B, T, H, W, 1)
    raw = raw.reshape(B, T, 1, H, W // 2 + 1)
    return 0.1 + 0.89 * raw if bounded else raw


_orig_gdn_gate = O.gdn_gate


def test_gdn_gate_values():
    pin_gdn_gate()


@pytest.mark.parametrize("mutant", [_gdn_gate_bound_09, _gdn_gate_product_logit])
def test_gdn_gate_pin_catches(mutant, monkeypatch):
    monkeypatch.setattr(O, "gdn_gate", mutant)
    with pytest.raises(AssertionError):
        pin_gdn_gate()


# ----------------------------------------------------------------- norms

def _gdn_norm_probe(norm):
    """GDN forward whose gate is a constant 20 and whose output projection is the
    identity: the output is 20 x the normed channel vector of every pixel."""
    rng = np.random.default_rng(3)
    B, T, H, W, C = 1, 2, 4, 4, 8
    cfg = O.GDNConfig(channels=C, delta_key_dim=2, gate_type="factored", output_norm=norm)
    p = O.init_params(O.gdn_param_shapes(cfg, H, W), rng)
    p["gate_proj"] = {"kernel": np.zeros((C, C)), "bias": np.full(C, 40.0)}   # silu(40) = 40 - 2e-16
    p["output_proj"] = {"kernel": np.eye(C), "bias": np.zeros(C)}
    if norm == "rms":
        p["rms_scale"] = np.ones(C)
    else:
        p["output_layernorm"] = {"scale": np.ones(C), "bias": np.zeros(C)}
    x = rng.standard_normal((B, T, H, W, C))
    out, pro = O.gdn_forward(p, x, cfg, return_intermediates=True)
    o = pro["o_spatial"].transpose(0, 1, 3, 4, 2)          # (B, T, H, W, C) before the norm
    return out / O.silu(40.0), o


def pin_rms_norm():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((2, 3, 4, 5, 8)) * rng.uniform(0.5, 4.0, (2, 3, 4, 5, 1))
    w = rng.standard_normal(8)
    y = O.rms_norm(x, np.ones(8), eps=0.0)
    assert np.allclose(np.mean(y ** 2, axis=-1), 1.0, rtol=0, atol=1e-13), "unit RMS per pixel across C"
    y = O.rms_norm(x, w)
    ms = np.mean(x ** 2, axis=-1, keepdims=True)
    assert np.allclose(y, x / np.sqrt(ms + 1e-6) * w, rtol=1e-14, atol=0), "eps 1e-6 inside the rsqrt, scale per C"
    # no mean subtraction: a constant channel vector keeps its sign and value / |value|
    c = np.full((1, 8), -2.5)
    assert np.allclose(O.rms_norm(c, np.ones(8), eps=0.0), -1.0, rtol=0, atol=1e-15)
    # in the GDN forward the norm runs across the channels of each pixel
    y, o = _gdn_norm_probe("rms")
    assert np.allclose(np.mean(y ** 2, axis=-1), np.mean(o ** 2, axis=-1) / (np.mean(o ** 2, axis=-1) + 1e-6),
                       rtol=1e-12, atol=0), "GDN output RMSNorm over C per pixel"


def pin_layer_norm():
    rng = np.random.default_rng(6)
    x = rng.standard_normal((2, 3, 4, 8)) * 3.0 + rng.standard_normal((2, 3, 4, 1)) * 5.0
    y = O.layer_norm(x, np.ones(8), np.zeros(8), eps=0.0)
    assert np.allclose(np.mean(y, axis=-1), 0.0, rtol=0, atol=1e-13), "zero mean per pixel across C"
    assert np.allclose(np.var(y, axis=-1), 1.0, rtol=0, atol=1e-12), "unit variance per pixel across C"
    s, b = rng.standard_normal(8), rng.standard_normal(8)
    mu = x.mean(-1, keepdims=True)
    var = x.var(-1, keepdims=True)
    assert np.allclose(O.layer_norm(x, s, b), (x - mu) / np.sqrt(var + 1e-6) * s + b, rtol=1e-13, atol=1e-13)
    y, o = _gdn_norm_probe("layer")
    assert np.allclose(np.mean(y, axis=-1), 0.0, rtol=0, atol=1e-10), "GDN output LayerNorm over C per pixel"
    var_o = o.var(-1)
    assert np.allclose(np.var(y, axis=-1), var_o / (var_o + 1e-6), rtol=1e-10, atol=0)


def _rms_over_pixels(x, weight, eps=1e-6):
    """Mistake: the mean taken over the spatial axes instead of the channels."""
    ms = np.mean(x ** 2, axis=tuple(range(max(0, x.ndim - 3), x.ndim - 1)) or (-1,), keepdims=True)
    return x / np.sqrt(ms + eps) * weight


def _rms_with_mean(x, weight, eps=1e-6):
    """Mistake: a mean subtracted (LayerNorm without bias)."""
    mu = np.mean(x, axis=-1, keepdims=True)
    return (x - mu) / np.sqrt(np.mean((x - mu) ** 2, axis=-1, keepdims=True) + eps) * weight


def _ln_over_pixels(x, scale, bias, eps=1e-6):
    ax = tuple(range(max(0, x.ndim - 3), x.ndim - 1)) or (-1,)
    mu = np.mean(x, axis=ax, keepdims=True)
    var = np.mean((x - mu) ** 2, axis=ax, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * scale + bias


def _ln_no_centre(x, scale, bias, eps=1e-6):
    var = np.mean(x ** 2, axis=-1, keepdims=True)
    return x / np.sqrt(var + eps) * scale + bias


def test_rms_norm_axis():
    pin_rms_norm()


def test_layer_norm_axis():
    pin_layer_norm()


@pytest.mark.parametrize("mutant", [_rms_over_pixels, _rms_with_mean])
def test_rms_norm_pin_catches(mutant, monkeypatch):
    monkeypatch.setattr(O, "rms_norm", mutant)
    with pytest.raises(AssertionError):
        pin_rms_norm()


@pytest.mark.parametrize("mutant", [_ln_over_pixels, _ln_no_centre])
def test_layer_norm_pin_catches(mutant, monkeypatch):
    monkeypatch.setattr(O, "layer_norm", mutant)
    with pytest.raises(AssertionError):
        pin_layer_norm()


# ================================================================ layer wiring
#
# The pins below fix how each layer wires its pieces together (which half of in_proj is the
# state input, where ctx is taken, which qkv slice is which, which stream each input gate
# scales, what gate_proj and ctx read), each through an identity of the reference's wiring:
#   gated   cssm.py:480-484 (x_main = xz[..., :C], z = xz[..., C:]), :502 (SiLU), :536 (ctx =
#           mean of the activated x_main), :581 (y * SiLU(z)), :584 (out_proj)
#   GDN     cssm.py:4740-4758 (qkv_dw -> qkv_proj; q, k, v = slices 0, 1, 2), :4785-4786 (ctx from
#           the layer input x), :4844-4848 (B_k scales k_in, B_v scales v_in), :4853-4855
#           (gate_proj reads x_flat), :5026-5041 (norm, x gate, output_proj)
# Each mutant re-runs the layer with exactly one wiring mistake.


def _gated_forward_mistake(mistake):
    """O.gated_forward with one wiring mistake: 'swap_split' (x_main and z exchanged),
    'ctx_pre_silu' (ctx from x_main before the SiLU), 'ctx_from_x' (ctx from the layer input)."""
    def fwd(params, x, cfg, scan="linear", return_intermediates=False):
        x = np.asarray(x, dtype=np.float64)
        B, T, H, W, Cin = x.shape
        Ci = cfg.channels * cfg.expand
        xz = O.dense(x, params["in_proj"])
        x_main, z = xz[..., :Ci], xz[..., Ci:]
        if mistake == "swap_split":
            x_main, z = z, x_main
        if cfg.short_conv_spatial_size > 0:
            x_main = O.depthwise_conv2d_same(x_main.reshape(B * T, H, W, Ci),
                                             params["short_conv_spatial"]).reshape(B, T, H, W, Ci)
        if cfg.short_conv_size > 0:
            x_main = O.causal_conv_t(x_main, params["short_conv_temporal"])
        pre = x_main
        x_main = O.silu(x_main)
        khat = O.spectral_kernel(params["kernel"], H, W, cfg.spectral_rho)
        ctx = {"ctx_pre_silu": pre, "ctx_from_x": x}.get(mistake, x_main).mean(axis=(2, 3))
        delta, gB, gC = O.gated_gates(ctx, params, cfg, H, W)
        y = O.gated_core(x_main.transpose(0, 1, 4, 2, 3), O.silu(z).transpose(0, 1, 4, 2, 3), khat, delta,
                         gB, gC, scan=scan)
        return O.dense(y.transpose(0, 1, 3, 4, 2), params["out_proj"])
    return fwd


def pin_gated_split_order():
    """With the z half of in_proj zeroed, SiLU(z) = 0 and y * SiLU(z) = 0, so the layer returns
    out_proj's bias exactly (short convs on, so a swapped split would feed their bias through)."""
    rng = np.random.default_rng(21)
    C, H, W = 4, 8, 8
    cfg = O.GatedConfig(channels=C, kernel_size=3, gate_type="factored", short_conv_size=2,
                        short_conv_spatial_size=3)
    p = O.init_params(O.gated_param_shapes(cfg, C, H, W), rng)
    p["in_proj"]["kernel"][:, C:] = 0.0
    p["in_proj"]["bias"][C:] = 0.0
    x = rng.standard_normal((2, 3, H, W, C))
    out = O.gated_forward(p, x, cfg)
    assert np.array_equal(out, np.broadcast_to(p["out_proj"]["bias"], out.shape)), "z half must gate the output"


def _silu_twin(b=-0.5):
    """a < -1.278 with SiLU(a) = SiLU(b): SiLU is not injective below its minimum."""
    from scipy.optimize import brentq
    return brentq(lambda a: float(O.silu(a) - O.silu(b)), -20.0, -1.2785, xtol=1e-15, rtol=1e-15)


def pin_gated_ctx_source():
    """ctx is the spatial mean of the activated x_main: two inputs whose x_main differ only by
    swapping SiLU twins (SiLU(a) = SiLU(b), a != b) give the same SiLU(x_main) and z, hence the
    same output, while any pre-SiLU mean (or the mean of x) differs between them by O(1)."""
    rng = np.random.default_rng(22)
    C, H, W = 3, 8, 8
    cfg = O.GatedConfig(channels=C, kernel_size=3, gate_type="factored", short_conv_size=0,
                        short_conv_spatial_size=0)
    p = O.init_params(O.gated_param_shapes(cfg, C, H, W), rng)
    p["in_proj"]["kernel"][:, :C] = np.eye(C)             # x_main = x exactly
    p["in_proj"]["bias"][:C] = 0.0
    p["in_proj"]["kernel"][0, C:] = 0.0                   # z does not read channel 0
    for g in ("delta_proj", "B_proj", "C_proj"):          # gates strongly ctx-dependent
        for s in ("_h", "_w"):
            p[g + s]["kernel"] *= 8.0
    a, b = _silu_twin(), -0.5
    mask = rng.random((1, 2, H, W)) < 0.3
    x1 = rng.standard_normal((1, 2, H, W, C))
    x2 = x1.copy()
    x1[..., 0] = np.where(mask, a, b)
    x2[..., 0] = np.where(mask, b, a)
    y1, y2 = O.gated_forward(p, x1, cfg), O.gated_forward(p, x2, cfg)
    assert np.max(np.abs(y1 - y2)) <= 1e-10 * np.sqrt(np.mean(y1 ** 2)), "ctx must follow SiLU(x_main)"


def test_gated_split_order():
    pin_gated_split_order()


def test_gated_ctx_source():
    pin_gated_ctx_source()


@pytest.mark.parametrize("mistake", ["swap_split"])
def test_gated_split_pin_catches(mistake, monkeypatch):
    monkeypatch.setattr(O, "gated_forward", _gated_forward_mistake(mistake))
    with pytest.raises(AssertionError):
        pin_gated_split_order()


@pytest.mark.parametrize("mistake", ["ctx_pre_silu", "ctx_from_x"])
def test_gated_ctx_pin_catches(mistake, monkeypatch):
    monkeypatch.setattr(O, "gated_forward", _gated_forward_mistake(mistake))
    with pytest.raises(AssertionError):
        pin_gated_ctx_source()


def _gdn_prologue_mistake(mistake):
    """O.gdn_prologue with one wiring mistake: 'slices_kqv' / 'slices_vkq' / 'slices_qvk' (the
    qkv_proj slices in another order), 'gates_swapped' (B_v on k, B_k on v), 'bk_on_q' / 'bv_on_q'
    (an input gate on q instead of its stream), 'gate_proj_after_conv' (gate_proj reads the qkv_dw
    output), 'ctx_after_conv' (ctx from the qkv_dw output)."""
    def pro(params, x, cfg):
        x = np.asarray(x, dtype=np.float64)
        B, T, H, W, C = x.shape
        W_hat = O.spectral_kernel(params["kernel"], H, W, cfg.spectral_rho, squash=not cfg.no_spectral_clamp)
        x_flat = x.reshape(B * T, H, W, C)
        xc = O.depthwise_conv2d_same(x_flat, params["qkv_dw"]) if cfg.qkv_conv_size > 1 else x_flat
        qkv = O.dense(xc, params["qkv_proj"]).reshape(B, T, H, W, 3 * C)
        sl = [qkv[..., :C], qkv[..., C:2 * C], qkv[..., 2 * C:]]
        order = {"slices_kqv": (1, 0, 2), "slices_vkq": (2, 1, 0), "slices_qvk": (0, 2, 1)}.get(mistake, (0, 1, 2))
        q_in, k_in, v_in = (sl[i] for i in order)
        if cfg.short_conv_size > 0:
            q_in = O.silu(O.causal_conv_t(q_in, params["short_conv_q"]))
            k_in = O.silu(O.causal_conv_t(k_in, params["short_conv_k"]))
            v_in = O.silu(O.causal_conv_t(v_in, params["short_conv_v"]))
        ctx_src = xc.reshape(B, T, H, W, C) if mistake == "ctx_after_conv" else x
        ctx = ctx_src.mean(axis=(2, 3)) + O.temporal_context_encoding(T, C, cfg.rope_base)[None]
        if cfg.use_input_gates:
            gk = O.gdn_gate("B_k", params, cfg, ctx, x, H, W, spatial=True)
            gv_ = O.gdn_gate("B_v", params, cfg, ctx, x, H, W, spatial=True)
            if mistake == "gates_swapped":
                gk, gv_ = gv_, gk
            if mistake == "bk_on_q":
                q_in = q_in * gk
            else:
                k_in = k_in * gk
            if mistake == "bv_on_q":
                q_in = q_in * gv_
            else:
                v_in = v_in * gv_
        g_src = xc if mistake == "gate_proj_after_conv" else x_flat
        gv = O.dense(g_src, params["gate_proj"]).reshape(B, T, H, W, C)
        gate_val = O.silu(gv) if cfg.output_gate_act == "silu" else O.sigmoid(gv)
        alpha = O.gdn_gate("alpha", params, cfg, ctx, x, H, W, bounded=True)
        beta = O.gdn_gate("beta", params, cfg, ctx, x, H, W)
        return dict(q_in=q_in, k_in=k_in, v_in=v_in, gate_val=gate_val, alpha=alpha, beta=beta, W_hat=W_hat,
                    ctx=ctx)
    return pro


def pin_gdn_slice_order():
    """With the q columns of qkv_proj zeroed (no short conv): q_hat = 0, so o = S q = 0, the norm of
    0 is 0 and the layer returns output_proj's bias exactly.  A k or v slice in q's place feeds
    real values, and a zero k or v reaches the floored entries (1e-7), so any other order leaves
    a non-zero o.  k and v are told apart by scaling (0-homogeneous in k, linear in v)."""
    rng = np.random.default_rng(23)
    C, H, W = 8, 6, 6
    cfg = O.GDNConfig(channels=C, delta_key_dim=4, kernel_size=3, gate_type="factored", short_conv_size=0)
    p = O.init_params(O.gdn_param_shapes(cfg, H, W), rng, spectral_init="xavier")
    p["qkv_proj"]["kernel"][:, :C] = 0.0
    p["qkv_proj"]["bias"][:C] = 0.0
    x = rng.standard_normal((2, 3, H, W, C))
    out = O.gdn_forward(p, x, cfg)
    assert np.array_equal(out, np.broadcast_to(p["output_proj"]["bias"], out.shape)), "q is slice 0"
    # k is normalised per bin and v enters s linearly: with no output norm and no short conv the
    # output minus its bias is unchanged when the k columns are scaled and scales with the v columns
    cfg = O.GDNConfig(channels=C, delta_key_dim=4, kernel_size=3, gate_type="factored", short_conv_size=0,
                      output_norm="none")
    p = O.init_params(O.gdn_param_shapes(cfg, H, W), rng, spectral_init="xavier")

    def scaled(sl, lam):
        q = {k: (dict(v) if isinstance(v, dict) else v) for k, v in p.items()}
        kern, bias = p["qkv_proj"]["kernel"].copy(), p["qkv_proj"]["bias"].copy()
        kern[:, sl * C:(sl + 1) * C] *= lam
        bias[sl * C:(sl + 1) * C] *= lam
        q["qkv_proj"] = {"kernel": kern, "bias": bias}
        return O.gdn_forward(q, x, cfg) - p["output_proj"]["bias"]
    r1 = scaled(1, 1.0)
    assert np.max(np.abs(scaled(1, 3.0) - r1)) <= 1e-6 * np.max(np.abs(r1)), "k is slice 1 (normalised)"
    assert np.max(np.abs(scaled(2, 3.0) - 3.0 * r1)) <= 1e-9 * np.max(np.abs(r1)), "v is slice 2 (linear)"


def _gdn_gate_scaling_case(use_l2, bk, bv):
    """T = 1, output_norm 'none', no short conv, factored input gates with zero kernels, so B_k and
    B_v are the uniform sigmoid(bk) and sigmoid(bv); returns out - output_proj bias."""
    rng = np.random.default_rng(24)
    C, H, W = 8, 6, 6
    cfg = O.GDNConfig(channels=C, delta_key_dim=4, kernel_size=3, gate_type="factored", short_conv_size=0,
                      output_norm="none", use_spectral_l2_norm=use_l2)
    p = O.init_params(O.gdn_param_shapes(cfg, H, W), rng, spectral_init="xavier")
    for name, b in (("B_k", bk), ("B_v", bv)):
        for s, n in (("_h", H), ("_w", W)):
            p[name + s] = {"kernel": np.zeros((C, n)), "bias": np.full(n, b / 2.0)}
    x = rng.standard_normal((1, 1, H, W, C))
    return O.gdn_forward(p, x, cfg) - p["output_proj"]["bias"]


def pin_gdn_input_gate_streams():
    """B_k scales k, which the key-vector norm removes: with the spectral L2 norm off (so q keeps
    its scale) the output cannot depend on B_k.  B_v scales v, on which o is linear: with the
    spectral norm on (q and k both normalised) the output scales by B_v's ratio."""
    r0 = _gdn_gate_scaling_case(False, 0.0, 0.0)
    rk = _gdn_gate_scaling_case(False, 2.0, 0.0)
    assert np.max(np.abs(rk - r0)) <= 1e-6 * np.max(np.abs(r0)), "B_k must scale only k"
    r0 = _gdn_gate_scaling_case(True, 0.0, 0.0)
    rv = _gdn_gate_scaling_case(True, 0.0, 2.0)
    ratio = float(O.sigmoid(2.0) / O.sigmoid(0.0))
    assert np.max(np.abs(rv - ratio * r0)) <= 1e-9 * np.max(np.abs(rv)), "B_v must scale v"


def pin_gdn_gate_proj_and_ctx_inputs():
    """qkv_dw = 2 delta with qkv_proj W gives the same q, k, v as qkv_dw = delta with qkv_proj 2W.
    gate_proj and ctx read the layer input x (not the conv output), so both parameter sets give
    the same output; reading the conv output would see 2x against x."""
    rng = np.random.default_rng(25)
    C, H, W = 8, 6, 6
    cfg = O.GDNConfig(channels=C, delta_key_dim=4, kernel_size=3, gate_type="factored", qkv_conv_size=3)
    p1 = O.init_params(O.gdn_param_shapes(cfg, H, W), rng, spectral_init="xavier")
    for name in ("alpha", "beta", "B_k", "B_v"):                  # gates strongly ctx-dependent
        for s in ("_h", "_w"):
            p1[name + s]["kernel"] *= 6.0
    p2 = {k: (dict(v) if isinstance(v, dict) else v) for k, v in p1.items()}
    d = np.zeros((3, 3, 1, C))
    d[1, 1] = 1.0
    p1["qkv_dw"] = {"kernel": 2.0 * d, "bias": np.zeros(C)}
    p2["qkv_dw"] = {"kernel": d, "bias": np.zeros(C)}
    p2["qkv_proj"] = {"kernel": 2.0 * p1["qkv_proj"]["kernel"], "bias": p1["qkv_proj"]["bias"]}
    x = rng.standard_normal((1, 3, H, W, C))
    y1, y2 = O.gdn_forward(p1, x, cfg), O.gdn_forward(p2, x, cfg)
    assert np.max(np.abs(y1 - y2)) <= 1e-12 * np.max(np.abs(y1)), "gate_proj / ctx must read x"


def test_gdn_slice_order():
    pin_gdn_slice_order()


def test_gdn_input_gate_streams():
    pin_gdn_input_gate_streams()


def test_gdn_gate_proj_and_ctx_inputs():
    pin_gdn_gate_proj_and_ctx_inputs()


@pytest.mark.parametrize("mistake", ["slices_kqv", "slices_vkq", "slices_qvk"])
def test_gdn_slice_pin_catches(mistake, monkeypatch):
    monkeypatch.setattr(O, "gdn_prologue", _gdn_prologue_mistake(mistake))
    with pytest.raises(AssertionError):
        pin_gdn_slice_order()


@pytest.mark.parametrize("mistake", ["gates_swapped", "bk_on_q", "bv_on_q"])
def test_gdn_input_gate_pin_catches(mistake, monkeypatch):
    monkeypatch.setattr(O, "gdn_prologue", _gdn_prologue_mistake(mistake))
    with pytest.raises(AssertionError):
        pin_gdn_input_gate_streams()


@pytest.mark.parametrize("mistake", ["gate_proj_after_conv", "ctx_after_conv"])
def test_gdn_gate_proj_ctx_pin_catches(mistake, monkeypatch):
    monkeypatch.setattr(O, "gdn_prologue", _gdn_prologue_mistake(mistake))
    with pytest.raises(AssertionError):
        pin_gdn_gate_proj_and_ctx_inputs()


def test_gdn_prologue_mistake_free_copy_agrees():
    """The mutant harness with no mistake reproduces the oracle (so each mutant differs from the
    oracle only by its mistake)."""
    rng = np.random.default_rng(26)
    cfg = O.GDNConfig(channels=8, delta_key_dim=4, kernel_size=3, gate_type="factored", qkv_conv_size=3)
    p = O.init_params(O.gdn_param_shapes(cfg, 6, 6), rng, spectral_init="xavier")
    x = rng.standard_normal((1, 3, 6, 6, 8))
    a, b = O.gdn_prologue(p, x, cfg), _gdn_prologue_mistake(None)(p, x, cfg)
    for k in ("q_in", "k_in", "v_in", "gate_val", "alpha", "beta", "W_hat", "ctx"):
        assert np.allclose(a[k], b[k], rtol=0, atol=1e-13), k
    cfgg = O.GatedConfig(channels=4, kernel_size=3, gate_type="factored", short_conv_size=2)
    pg = O.init_params(O.gated_param_shapes(cfgg, 4, 8, 8), rng)
    xg = rng.standard_normal((1, 3, 8, 8, 4))
    assert np.allclose(O.gated_forward(pg, xg, cfgg), _gated_forward_mistake(None)(pg, xg, cfgg), rtol=0,
                       atol=1e-13)


# ------------------------------------------------------- GDN scan variants

def pin_gdn_scan_variants():
    """Which scan each configuration takes (cssm.py:4939-4991) and how each maps a zero, a tiny
    negative, a tiny imaginary and an ordinary entry (to_goom: |x| < 1e-7 -> 1e-7 + 0j;
    log(|x| + 1e-8) + i angle(x) then exp; the direct / pallas scans: unchanged).  Through the
    layer core, a head with zero values at T = 1 has s = Delta' = c everywhere, so o_i = c sum_a q_a
    with c = 1e-7, 1e-8 or 0 for the three scans."""
    V = lambda **kw: O.gdn_scan_variant(O.GDNConfig(channels=8, **kw))
    assert V(delta_key_dim=4) == "goom"
    assert V(delta_key_dim=4, use_goom=False) == "log_eps"
    assert V(delta_key_dim=4, use_log=False) == "linear"
    assert V(delta_key_dim=4, use_log=False, use_goom=False) == "linear"
    assert V(delta_key_dim=2, scan_mode="pallas") == "linear"
    assert V(delta_key_dim=2, scan_mode="pallas", use_goom=False) == "linear"
    assert V(delta_key_dim=4, scan_mode="pallas") == "goom"
    assert V(delta_key_dim=3, scan_mode="pallas", use_goom=False) == "log_eps"
    z = np.array([0.0, -3e-8, 5e-8j, 0.3 * np.exp(0.7j), -2.0])
    want = {"goom": [1e-7, 1e-7, 1e-7, z[3], -2.0],
            "log_eps": [1e-8, -4e-8, 6e-8j, (0.3 + 1e-8) * np.exp(0.7j), -(2.0 + 1e-8)],
            "linear": list(z)}
    for var, w in want.items():
        got = O.gdn_scan_entries(z, var)
        assert np.allclose(got, np.array(w, dtype=complex), rtol=1e-15, atol=1e-22), var
    # through gdn_core: head 0 has v = 0 at T = 1
    rng = np.random.default_rng(27)
    B, T, H, W, C, dk = 1, 1, 6, 6, 8, 4
    Wf = W // 2 + 1
    q, k, v = (rng.standard_normal((B, T, H, W, C)) for _ in range(3))
    v[..., :dk] = 0.0
    alpha = 0.1 + 0.89 * O.sigmoid(rng.standard_normal((B, T, 1, H, Wf)))
    beta = O.sigmoid(rng.standard_normal((B, T, 1, H, Wf)))
    Wh = O.spectral_kernel(rng.standard_normal((C // dk, 3, 3)), H, W)
    qs = np.fft.rfft2(q[0, 0, :, :, :dk].transpose(2, 0, 1))
    qn = qs / np.sqrt(np.sum(np.abs(qs) ** 2, axis=(1, 2), keepdims=True) + 1e-6)
    for kw, c in ((dict(), 1e-7), (dict(use_goom=False), 1e-8), (dict(use_log=False), 0.0)):
        cfg = O.GDNConfig(channels=C, delta_key_dim=dk, kernel_size=3, gate_type="factored", **kw)
        o = O.gdn_core(q, k, v, alpha, beta, Wh, cfg)
        expect = np.fft.irfft2(np.broadcast_to(c * qn.sum(axis=0), (dk, H, Wf)), s=(H, W))
        assert np.allclose(o[0, 0, :dk], expect, rtol=0, atol=1e-12 * max(c, 1e-30)), kw


def _variant_goom_false_is_linear(cfg):
    """Mistake (the earlier oracle): use_goom=False drops every floor instead of adding 1e-8."""
    return "linear" if not cfg.use_goom else _orig_scan_variant(cfg)


def _variant_pallas_ignored(cfg):
    """Mistake: scan_mode='pallas' at d_k=2 still takes the log-space scan."""
    return ("goom" if cfg.use_goom else "log_eps") if cfg.use_log else "linear"


def _entries_log_eps_as_max(z, variant):
    """Mistake: max(|x|, 1e-8) with the phase, instead of |x| + 1e-8."""
    if variant == "log_eps":
        return np.maximum(np.abs(z), 1e-8) * np.exp(1j * np.angle(z))
    return _orig_scan_entries(z, variant)


def _entries_log_eps_no_phase(z, variant):
    """Mistake: the phase dropped (exp of the real log only)."""
    if variant == "log_eps":
        return (np.abs(z) + 1e-8).astype(complex)
    return _orig_scan_entries(z, variant)


_orig_scan_variant = O.gdn_scan_variant
_orig_scan_entries = O.gdn_scan_entries


def test_gdn_scan_variants():
    pin_gdn_scan_variants()


@pytest.mark.parametrize("name,mutant", [("gdn_scan_variant", _variant_goom_false_is_linear),
                                         ("gdn_scan_variant", _variant_pallas_ignored),
                                         ("gdn_scan_entries", _entries_log_eps_as_max),
                                         ("gdn_scan_entries", _entries_log_eps_no_phase)])
def test_gdn_scan_variant_pin_catches(name, mutant, monkeypatch):
    monkeypatch.setattr(O, name, mutant)
    with pytest.raises(AssertionError):
        pin_gdn_scan_variants()
