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
