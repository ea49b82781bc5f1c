"""Pins the CPU oracle (oracle/cssm_oracle.py) against closed forms, brute force,
the reference's log-space algebra, invariants and the reference's published
parameter counts.  CPU only."""
import math

import numpy as np
import pytest

from oracle import cssm_oracle as O

SHAPES = [(8, 8), (7, 7), (14, 14), (4, 4), (6, 10), (5, 9), (16, 16), (3, 12)]


def _rel(a, b):
    return float(np.max(np.abs(a - b)) / (np.sqrt(np.mean(np.abs(b) ** 2)) + 1e-300))


# --------------------------------------------------------------------- FFT rule

@pytest.mark.parametrize("H,W", SHAPES)
def test_rfft2_matches_dft_matrix(H, W, rng):
    x = rng.standard_normal((3, H, W))
    assert _rel(O.rfft2(x), O.rfft2_bruteforce(x)) < 1e-12


@pytest.mark.parametrize("H,W", SHAPES)
def test_irfft2_c2r_rule_on_non_hermitian_spectra(H, W, rng):
    """Gated spectra are not Hermitian: the C2R rule keeps only Re of the v=0
    and v=W/2 columns after the H inverse (closed form in irfft2_bruteforce)."""
    Wf = W // 2 + 1
    X = rng.standard_normal((2, H, Wf)) + 1j * rng.standard_normal((2, H, Wf))
    assert _rel(O.irfft2(X, H, W), O.irfft2_bruteforce(X, H, W)) < 1e-12


def test_irfft2_discards_dc_and_nyquist_imag(rng):
    H, W = 6, 8
    X = np.zeros((H, W // 2 + 1), complex)
    X[2, 0] = 1j          # purely imaginary DC column entry after the H-inverse
    y = O.irfft2(X, H, W)
    # Z[h,0] = (1/H) i e^{2 pi i 2h/H}: Re Z = -(1/H) sin(4 pi h/H), constant along w
    h = np.arange(H)
    expect = (-np.sin(4 * np.pi * h / H) / H / W)[:, None] * np.ones((1, W))
    assert np.allclose(y, expect, atol=1e-15)


# --------------------------------------------------------------- spectral kernel

@pytest.mark.parametrize("H,W", [(32, 32), (128, 128), (7, 7), (14, 14), (4, 4), (9, 6)])
def test_spectral_kernel_k1_closed_form(H, W, rng):
    """K=1: the single tap sits at ((H-1)//2, (W-1)//2) -> a pure linear phase."""
    C = 3
    k = rng.standard_normal((C, 1, 1)) * 0.5
    rho = 0.999
    kh = O.spectral_kernel(k, H, W, rho)
    ph, pw = (H - 1) // 2, (W - 1) // 2
    u = np.arange(H)[:, None]
    v = np.arange(W // 2 + 1)[None, :]
    phase = np.exp(-2j * np.pi * (u * ph / H + v * pw / W))
    mag = rho * k[:, 0, 0] / (1 + np.abs(k[:, 0, 0]))
    assert np.allclose(kh, mag[:, None, None] * phase[None], atol=1e-13)


@pytest.mark.parametrize("H,K", [(128, 11), (32, 11), (16, 15), (8, 15), (7, 11), (4, 11), (14, 11)])
def test_spectral_kernel_centre_tap_position(H, K):
    """A delta at the kernel centre lands at pad_before + K//2 (K<=H) or K//2 - (K-H)//2 (crop)."""
    k = np.zeros((1, K, K))
    k[0, K // 2, K // 2] = 1.0
    kh = O.spectral_kernel(k, H, H, rho=1.0)
    if K <= H:
        pos = (H - K) // 2 + K // 2
    else:
        pos = K // 2 - (K - H) // 2
    u = np.arange(H)[:, None]
    v = np.arange(H // 2 + 1)[None, :]
    expect = 0.5 * np.exp(-2j * np.pi * (u + v) * pos / H)
    assert np.allclose(kh[0], expect, atol=1e-13)
    if H == 128 and K == 11:
        assert pos == 63


# ------------------------------------------------------------------ gated core

def _rand_gates(rng, B, T, H, W):
    Wf = W // 2 + 1
    delta = O.softplus(rng.standard_normal((B, T, H, Wf)))
    gB = rng.standard_normal((B, T, H, Wf))
    gC = rng.standard_normal((B, T, H, Wf))
    return delta, gB, gC


@pytest.mark.parametrize("H,W", [(8, 8), (7, 7), (6, 10)])
def test_gated_core_T1_impulse_closed_form(H, W, rng):
    """x = delta at (0,0) => U_hat == 1 => y = irfft2(gC (Delta+1e-8) gB) * zg."""
    B, C = 2, 3
    x = np.zeros((B, 1, C, H, W))
    x[:, :, :, 0, 0] = 1.0
    zg = rng.standard_normal((B, 1, C, H, W))
    kh = rng.standard_normal((C, H, W // 2 + 1)) + 1j * rng.standard_normal((C, H, W // 2 + 1))
    d, gB, gC = _rand_gates(rng, B, 1, H, W)
    y = O.gated_core(x, zg, kh, d, gB, gC)
    Y = (gC * (d + 1e-8) * gB)[:, :, None]
    expect = O.irfft2_bruteforce(np.broadcast_to(Y, (B, 1, C, H, W // 2 + 1)), H, W) * zg
    assert _rel(y, expect) < 1e-12


def test_gated_core_static_gates_geometric_series(rng):
    """Identical frames and gates over T: h_t = V (1 - A^{t+1}) / (1 - A)."""
    B, T, C, H, W = 1, 6, 2, 8, 8
    Wf = W // 2 + 1
    frame = rng.standard_normal((B, 1, C, H, W))
    x = np.repeat(frame, T, axis=1)
    kh = 0.9 * np.exp(2j * np.pi * rng.random((C, H, Wf)))
    d1, gB1, gC1 = _rand_gates(rng, B, 1, H, W)
    d, gB, gC = (np.repeat(a, T, axis=1) for a in (d1, gB1, gC1))
    y = O.gated_core(x, None, kh, d, gB, gC)
    U = np.fft.rfft2(frame[:, 0])                       # independent FFT route
    A = kh[None] * np.exp(-d1[:, 0][:, None])
    V = (d1[:, 0][:, None] + 1e-8) * U * gB1[:, 0][:, None]
    for t in range(T):
        h = V * (1 - A ** (t + 1)) / (1 - A)
        expect = O.irfft2_bruteforce(gC1[:, 0][:, None] * h, H, W)
        assert _rel(y[:, t], expect) < 1e-11


def test_gated_core_goom_log_space_equals_linear(rng):
    """The reference evaluates the recurrence in GOOM log space; the oracle's
    linear form must agree (exact algebra up to rounding)."""
    B, T, C, H, W = 2, 7, 3, 8, 6
    x = rng.standard_normal((B, T, C, H, W))
    zg = rng.standard_normal((B, T, C, H, W))
    kh = O.spectral_kernel(rng.standard_normal((C, 5, 5)) * 0.3, H, W)
    d, gB, gC = _rand_gates(rng, B, T, H, W)
    y_lin = O.gated_core(x, zg, kh, d, gB, gC, scan='linear')
    y_log = O.gated_core(x, zg, kh, d, gB, gC, scan='goom')
    assert _rel(y_log, y_lin) < 1e-10


def test_gated_core_goom_floor_on_zero_inputs(rng):
    """Exact zeros in U*B hit to_goom's 1e-7+0j floor; both forms apply it identically."""
    B, T, C, H, W = 1, 4, 2, 4, 4
    x = np.zeros((B, T, C, H, W))
    x[:, 1:] = rng.standard_normal((B, T - 1, C, H, W))
    kh = O.spectral_kernel(rng.standard_normal((C, 3, 3)) * 0.3, H, W)
    d, gB, gC = _rand_gates(rng, B, T, H, W)
    gB[:, :, 1, :] = 0.0                                 # zero gate row -> U*B == 0
    y_lin = O.gated_core(x, None, kh, d, gB, gC, scan='linear')
    y_log = O.gated_core(x, None, kh, d, gB, gC, scan='goom')
    assert _rel(y_log, y_lin) < 1e-9
    # the t=0 frame is all zeros: its output is exactly the floor's contribution
    Y0 = gC[:, 0][:, None] * (d[:, 0][:, None] + 1e-8) * 1e-7
    assert np.allclose(y_lin[:, 0], O.irfft2_bruteforce(np.broadcast_to(Y0, (B, C, H, W // 2 + 1)), H, W),
                       atol=1e-20)


def _gated_cfg(**kw):
    base = dict(channels=4, kernel_size=3, gate_type='factored', short_conv_size=0,
                short_conv_spatial_size=0)
    base.update(kw)
    return O.GatedConfig(**base)


def test_gated_forward_circular_shift_equivariance(rng):
    cfg = _gated_cfg()
    H = W = 8
    shapes = O.gated_param_shapes(cfg, 4, H, W)
    p = O.init_params(shapes, rng)
    x = rng.standard_normal((2, 3, H, W, 4))
    y = O.gated_forward(p, x, cfg)
    xs = np.roll(x, (3, -2), axis=(2, 3))
    ys = O.gated_forward(p, xs, cfg)
    assert _rel(ys, np.roll(y, (3, -2), axis=(2, 3))) < 1e-12


def test_gated_forward_causal_in_time(rng):
    cfg = _gated_cfg(short_conv_size=4, short_conv_spatial_size=3, gate_type='dense')
    H = W = 6
    p = O.init_params(O.gated_param_shapes(cfg, 4, H, W), rng)
    x = rng.standard_normal((1, 5, H, W, 4))
    y = O.gated_forward(p, x, cfg)
    x2 = x.copy()
    x2[:, 3:] += rng.standard_normal(x2[:, 3:].shape)
    y2 = O.gated_forward(p, x2, cfg)
    assert np.array_equal(y[:, :3], y2[:, :3])
    assert not np.allclose(y[:, 3:], y2[:, 3:])


def test_gated_core_linear_in_x_for_fixed_gates(rng):
    B, T, C, H, W = 1, 3, 2, 8, 8
    kh = O.spectral_kernel(rng.standard_normal((C, 3, 3)) * 0.3, H, W)
    d, gB, gC = _rand_gates(rng, B, T, H, W)
    x1 = rng.standard_normal((B, T, C, H, W))
    x2 = rng.standard_normal((B, T, C, H, W))
    f = lambda x: O.gated_core(x, None, kh, d, gB, gC)
    assert _rel(f(2.0 * x1 - 3.0 * x2), 2.0 * f(x1) - 3.0 * f(x2)) < 1e-11


# ------------------------------------------------------------------------ GDN

def _gdn_cfg(**kw):
    base = dict(channels=8, delta_key_dim=4, kernel_size=3, gate_type='factored',
                short_conv_size=0, qkv_conv_size=1)
    base.update(kw)
    return O.GDNConfig(**base)


def test_gdn_T1_closed_form(rng):
    """T=1: s = beta v_i conj(k)  =>  o_i = beta v_i (k^H q) per bin."""
    cfg = _gdn_cfg()
    B, T, H, W, C = 2, 1, 6, 6, 8
    dk = 4
    nh = C // dk
    Wf = W // 2 + 1
    q, k, v = (rng.standard_normal((B, T, H, W, C)) for _ in range(3))
    alpha = 0.1 + 0.89 * O.sigmoid(rng.standard_normal((B, T, 1, H, Wf)))
    beta = O.sigmoid(rng.standard_normal((B, T, 1, H, Wf)))
    Wh = O.spectral_kernel(rng.standard_normal((nh, 3, 3)), H, W)
    o = O.gdn_core(q, k, v, alpha, beta, Wh, cfg)

    def heads(z):
        return z.reshape(B, T, H, W, nh, dk).transpose(0, 1, 4, 5, 2, 3)
    qs, ks, vs = (O.rfft2_bruteforce(heads(z)) for z in (q, k, v))
    qn, kn = O.gdn_spectral_norms(qs, ks, cfg)
    kq = np.sum(np.conj(kn) * qn, axis=3, keepdims=True)             # (B,T,nh,1,H,Wf)
    o_hat = beta[:, :, :, None] * vs * kq
    expect = O.irfft2_bruteforce(o_hat.reshape(B, T, C, H, Wf), H, W)
    assert _rel(o, expect) < 1e-11


def test_gdn_key_vector_norm_is_unit(rng):
    cfg = _gdn_cfg()
    B, T, nh, dk, H, Wf = 1, 2, 2, 4, 6, 4
    ks = rng.standard_normal((B, T, nh, dk, H, Wf)) + 1j * rng.standard_normal((B, T, nh, dk, H, Wf))
    qs = rng.standard_normal(ks.shape) + 1j * rng.standard_normal(ks.shape)
    qn, kn = O.gdn_spectral_norms(qs, ks, cfg)
    nk = np.sum(np.abs(kn) ** 2, axis=3)
    ss = np.sum(np.abs(ks / np.sqrt(np.sum(np.abs(ks) ** 2, axis=(4, 5), keepdims=True) + 1e-6)) ** 2, axis=3)
    assert np.allclose(nk, ss / (ss + 1e-6), atol=1e-14)
    assert np.allclose(np.sum(np.abs(qn) ** 2, axis=(4, 5)),
                       np.sum(np.abs(qs) ** 2, axis=(4, 5)) / (np.sum(np.abs(qs) ** 2, axis=(4, 5)) + 1e-6))


@pytest.mark.parametrize("gate_type", ['factored', 'channel', 'dense', 'scalar'])
def test_gdn_rank1_equals_materialised_matrix_scan(gate_type, rng):
    cfg = _gdn_cfg(gate_type=gate_type)
    B, T, H, W, C = 1, 5, 6, 4, 8
    p = O.init_params(O.gdn_param_shapes(cfg, H, W), rng, spectral_init='xavier')
    x = rng.standard_normal((B, T, H, W, C))
    y_lin = O.gdn_forward(p, x, cfg, scan='linear')
    y_r1 = O.gdn_forward(p, x, cfg, scan='rank1')
    assert _rel(y_r1, y_lin) < 1e-9


def test_gdn_matrix_scan_bruteforce_per_bin(rng):
    """Per-bin python loop with explicit d_k x d_k matrices (cssm.py:4911-4958 read literally)."""
    cfg = _gdn_cfg()
    B, T, H, W, C = 1, 3, 4, 4, 4
    dk = 4
    Wf = W // 2 + 1
    q, k, v = (rng.standard_normal((B, T, H, W, C)) for _ in range(3))
    alpha = 0.1 + 0.89 * O.sigmoid(rng.standard_normal((B, T, 1, H, Wf)))
    beta = O.sigmoid(rng.standard_normal((B, T, 1, H, Wf)))
    Wh = O.spectral_kernel(rng.standard_normal((1, 3, 3)), H, W)
    o = O.gdn_core(q, k, v, alpha, beta, Wh, cfg)
    qs = np.fft.rfft2(q[0].transpose(0, 3, 1, 2))          # (T,dk,H,Wf)
    ks = np.fft.rfft2(k[0].transpose(0, 3, 1, 2))
    vs = np.fft.rfft2(v[0].transpose(0, 3, 1, 2))
    o_hat = np.zeros((T, dk, H, Wf), complex)
    for uu in range(H):
        for vv in range(Wf):
            S = np.zeros((dk, dk), complex)              # S[i, a]
            for t in range(T):
                kn = ks[t] / np.sqrt(np.sum(np.abs(ks[t]) ** 2, axis=(1, 2)) + 1e-6)[:, None, None]
                qn = qs[t] / np.sqrt(np.sum(np.abs(qs[t]) ** 2, axis=(1, 2)) + 1e-6)[:, None, None]
                kv = kn[:, uu, vv] / np.sqrt(np.sum(np.abs(kn[:, uu, vv]) ** 2) + 1e-6)
                a, b = alpha[0, t, 0, uu, vv], beta[0, t, 0, uu, vv]
                M = a * Wh[0, uu, vv] * (np.eye(dk) - b * np.outer(kv, np.conj(kv)))
                M = np.where(np.abs(M) < 1e-7, 1e-7, M)
                D = b * np.outer(vs[t][:, uu, vv], np.conj(kv))
                D = np.where(np.abs(D) < 1e-7, 1e-7, D)
                S = (M @ S.T).T + D                       # each row i: s_i <- M s_i + D[i,:]
                o_hat[t, :, uu, vv] = S @ qn[:, uu, vv]
    expect = np.fft.irfft2(o_hat, s=(H, W))
    assert _rel(o[0], expect) < 1e-11


# ----------------------------------------------------------- parameter trees

def _simple_cssm_extra(c_in, C):
    """pathtracker stem (1x1 conv + LayerNorm) + readout (2 LayerNorms + Dense(C->1))
    of SimpleCSSM (simple_cssm.py:258-265, 531-557) with num_classes=1."""
    return (c_in * C + C) + 2 * C + 2 * C + 2 * C + (C + 1)


def test_param_count_gated_matches_reference_csv():
    """bench_image_timing.csv:86 (gated, H=16, C=256, K=11, dense gates, convs 4/3) = 346,033
    and :148 (gated, H=32, C=64) = 127,969 — both with a 3-channel input."""
    cfg = O.GatedConfig(channels=256, kernel_size=11, gate_type='dense')
    n = O.count_params(O.gated_param_shapes(cfg, 256, 16, 16)) + _simple_cssm_extra(3, 256)
    assert n == 346033
    cfg = O.GatedConfig(channels=64, kernel_size=11, gate_type='dense')
    n = O.count_params(O.gated_param_shapes(cfg, 64, 32, 32)) + _simple_cssm_extra(3, 64)
    assert n == 127969


def test_param_count_gdn_matches_reference_csv():
    """bench_image_timing.csv:98 (gdn, H=16, C=256, d_k=2, dense gates) = 556,961."""
    cfg = O.GDNConfig(channels=256, delta_key_dim=2, kernel_size=11, gate_type='dense')
    n = O.count_params(O.gdn_param_shapes(cfg, 16, 16)) + _simple_cssm_extra(3, 256)
    assert n == 556961


def test_temporal_context_encoding_closed_form():
    E = O.temporal_context_encoding(3, 4)
    assert np.allclose(E[0], [0, 1, 0, 1])
    assert np.allclose(E[2], [math.sin(2), math.cos(2), math.sin(2 / 100), math.cos(2 / 100)])


def test_goom_log_add_exp_is_exact_addition(rng):
    a = rng.standard_normal(50) + 1j * rng.standard_normal(50)
    b = rng.standard_normal(50) + 1j * rng.standard_normal(50)
    r = O.from_goom(O.log_add_exp(O.to_goom(a), O.to_goom(b)))
    assert np.allclose(r, a + b, rtol=1e-12, atol=1e-12)


# ------------------------------------------------------------ CSSMSHViT block

@pytest.mark.parametrize("mode", ["global_layer", "temporal_layer", "layer"])
def test_block_norm1_normalises_its_groups(mode, rng):
    """Within each of the reference's reduction groups norm1 is one affine map
    x -> (x - mean) / sqrt(var + eps) (unit scale, zero bias); the input's scale
    and offset vary per pixel and frame, so any other grouping breaks that.  A
    per-channel scale / bias then maps through channel-wise."""
    shape = (2, 3, 4, 5, 6)
    x = (rng.uniform(0.5, 3.0, shape[:4] + (1,)) * rng.standard_normal(shape)
         + rng.uniform(-2.0, 2.0, shape[:4] + (1,)))
    y = O.block_norm1(x, np.ones(6), np.zeros(6), mode)
    axes = O.BLOCK_NORM_AXES[mode]
    keep = [a for a in range(5) if a not in axes]
    xg = np.transpose(x, keep + list(axes)).reshape(int(np.prod([shape[a] for a in keep])), -1)
    yg = np.transpose(y, keep + list(axes)).reshape(xg.shape)
    for xv, yv in zip(xg, yg):
        expect = (xv - xv.mean()) / np.sqrt(xv.var() + 1e-6)
        assert np.max(np.abs(yv - expect)) < 1e-12
    s, b = rng.standard_normal(6), rng.standard_normal(6)
    assert np.allclose(O.block_norm1(x, s, b, mode), y * s + b, atol=1e-12)
    for other in O.BLOCK_NORM_AXES:
        if other != mode:
            yo = np.transpose(O.block_norm1(x, np.ones(6), np.zeros(6), other), keep + list(axes)).reshape(xg.shape)
            assert max(np.max(np.abs(yv - (xv - xv.mean()) / np.sqrt(xv.var() + 1e-6)))
                       for xv, yv in zip(xg, yo)) > 1e-3


def test_block_global_norm_of_a_repeated_image_is_the_image_norm(rng):
    img = rng.standard_normal((2, 5, 5, 4))
    x5 = np.repeat(img[:, None], 3, axis=1)
    y = O.block_norm1(x5, np.ones(4), np.zeros(4), "global_layer")
    mu = img.mean(axis=(1, 2, 3), keepdims=True)
    sd = np.sqrt(img.var(axis=(1, 2, 3), keepdims=True) + 1e-6)
    assert np.allclose(y[:, 1], (img - mu) / sd, atol=1e-12)


def test_depthwise_conv_same_is_a_cross_correlation(rng):
    """An impulse at (h0, w0) lands tap (i, j) at (h0 + 1 - i, w0 + 1 - j): lax's
    SAME convolution correlates (no kernel flip), per channel, with bias."""
    k = rng.standard_normal((3, 3, 1, 2))
    bias = rng.standard_normal(2)
    x = np.zeros((1, 6, 7, 2))
    x[0, 3, 2, 1] = 1.0
    y = O.depthwise_conv2d_same(x, {"kernel": k, "bias": bias})
    assert np.allclose(y[0, :, :, 0], bias[0])
    for i in range(3):
        for j in range(3):
            assert abs(y[0, 3 + 1 - i, 2 + 1 - j, 1] - (k[i, j, 0, 1] + bias[1])) < 1e-15


@pytest.mark.parametrize("k", [3, 4])
def test_full_conv_same_is_a_channel_mixing_cross_correlation(rng, k):
    """An impulse in input channel c at (h0, w0) lands tap (i, j) at (h0 + lo - i, w0 + lo - j) of
    every output channel o with weight kernel[i, j, c, o] (lax's SAME correlation, lo = (k - 1) // 2
    before and k // 2 after, so an even k reaches one row further down than up); a kernel that is
    diagonal in (c, o) is the depthwise conv."""
    C, N = 3, 5
    kern = rng.standard_normal((k, k, C, N))
    bias = rng.standard_normal(N)
    x = np.zeros((1, 7, 8, C))
    x[0, 3, 4, 2] = 1.0
    y = O.full_conv2d_same(x, {"kernel": kern, "bias": bias})
    lo = (k - 1) // 2
    hit = np.zeros((7, 8), bool)
    for i in range(k):
        for j in range(k):
            assert np.allclose(y[0, 3 + lo - i, 4 + lo - j], kern[i, j, 2] + bias, atol=1e-14)
            hit[3 + lo - i, 4 + lo - j] = True
    assert np.allclose(y[0][~hit], bias, atol=1e-14)
    dw = rng.standard_normal((k, k, 1, C))
    xr = rng.standard_normal((2, 6, 5, C))
    diag = np.zeros((k, k, C, C))
    for c in range(C):
        diag[:, :, c, c] = dw[:, :, 0, c]
    assert np.allclose(O.full_conv2d_same(xr, {"kernel": diag}),
                       O.depthwise_conv2d_same(xr, {"kernel": dw, "bias": np.zeros(C)}), atol=1e-12)


def test_gelu_tanh_form():
    x = np.linspace(-6, 6, 101)
    erf_gelu = np.array([0.5 * v * (1 + math.erf(v / math.sqrt(2))) for v in x])
    g = O.gelu_tanh(x)
    assert np.max(np.abs(g - erf_gelu)) < 1e-3 and np.max(np.abs(g - erf_gelu)) > 1e-5   # the tanh form, not erf
    assert g[50] == 0.0 and abs(g[-1] - 6.0) < 1e-6


@pytest.mark.parametrize("image", [True, False])
def test_shvit_block_wiring_closed_forms(image, rng):
    """With a cell that returns zeros the block returns its input (last frame for
    an image); with the identity cell it returns input + norm1 + pos_conv of the
    last (image) or every (video) frame; the activation acts on the cell output."""
    B, T, H, W, C = 2, 3, 5, 4, 3
    x = rng.standard_normal((B, H, W, C) if image else (B, T, H, W, C))
    p = {"norm1": {"scale": rng.standard_normal(C), "bias": rng.standard_normal(C)},
         "pos_conv": {"kernel": rng.standard_normal((3, 3, 1, C)), "bias": rng.standard_normal(C)},
         "cssm": {}}
    out0 = O.shvit_block_mixer(p, x, lambda q, h: np.zeros_like(h), num_timesteps=T)
    assert np.array_equal(out0, x)
    x5 = np.repeat(x[:, None], T, axis=1) if image else x
    h = O.block_norm1(x5, p["norm1"]["scale"], p["norm1"]["bias"])
    h = h + O.depthwise_conv2d_same(h.reshape(-1, H, W, C), p["pos_conv"]).reshape(h.shape)
    outi = O.shvit_block_mixer(p, x, lambda q, hh: hh, num_timesteps=T)
    assert np.allclose(outi, x + (h[:, -1] if image else h), atol=1e-12)
    outs = O.shvit_block_mixer(p, x, lambda q, hh: hh, num_timesteps=T, output_act="silu", use_pos_conv=False)
    hn = O.block_norm1(x5, p["norm1"]["scale"], p["norm1"]["bias"])
    assert np.allclose(outs, x + O.silu(hn[:, -1] if image else hn), atol=1e-12)


# ------------------------------------------------------ CSSM-SHViT block, second half

def test_timestep_gate_prior_closed_form(rng):
    """With gate_fc2 zeroed the logits are 0 and the weights are softmax(prior):
    e^4 / (T - 1 + e^4) on the last frame, 1 / (T - 1 + e^4) on the others (cssm_shvit.py:205-209)."""
    B, T, H, W, C = 2, 4, 3, 3, 8
    p = {"gate_fc1": {"kernel": rng.standard_normal((2 * C, 8)), "bias": rng.standard_normal(8)},
         "gate_fc2": {"kernel": np.zeros((8, 1)), "bias": np.zeros(1)}}
    y = np.stack([np.full((B, H, W, C), float(t + 1)) for t in range(T)], axis=1)
    got = O.timestep_gate_pool(p, rng.standard_normal((B, T, H, W, C)), y)
    z = T - 1 + math.exp(4.0)
    expect = (sum(range(1, T)) + T * math.exp(4.0)) / z
    assert np.allclose(got, expect, rtol=1e-14, atol=0)


def test_timestep_gate_logits_use_first_input_frame_and_frame_means(rng):
    """A gate that reads only the query half (the first input frame's mean) weighs every frame the
    same as the prior does; one that reads frame t's mean moves weight toward the larger mean."""
    B, T, H, W, C = 1, 3, 2, 2, 8
    y = np.stack([np.full((B, H, W, C), v) for v in (0.0, 5.0, 0.0)], axis=1)
    res = rng.standard_normal((B, T, H, W, C))
    w1 = np.zeros((2 * C, 8))
    w1[C:, 0] = 1.0                                   # reads the frame means only
    p = {"gate_fc1": {"kernel": w1, "bias": np.zeros(8)},
         "gate_fc2": {"kernel": np.eye(8)[:, :1] * 10.0, "bias": np.zeros(1)}}
    got = O.timestep_gate_pool(p, res, y)
    assert got.mean() > 4.9                           # frame 1 (mean 5) takes almost all the weight
    w1 = np.zeros((2 * C, 8))
    w1[:C, 0] = 1.0                                   # reads the query only: equal logits
    p["gate_fc1"]["kernel"] = w1
    got = O.timestep_gate_pool(p, res, y)
    z = 2 + math.exp(4.0)
    assert np.allclose(got, 5.0 / z, rtol=1e-12)


def test_mlp_half_closed_forms(rng):
    """fc2 zeroed: the block returns its input (the residual); dwconv with only a centre tap a
    and fc1 / fc2 identities: x + (1 + a) gelu(LN(x)) + bias (h + dwconv(h), shvit.py:173-176)."""
    B, H, W, C = 2, 4, 5, 6
    x = rng.standard_normal((B, H, W, C))
    n2 = {"scale": np.ones(C), "bias": np.zeros(C)}
    dwk = np.zeros((3, 3, 1, C))
    dwk[1, 1, 0, :] = 0.5
    p = {"norm2": n2, "mlp": {"fc1": {"kernel": np.eye(C), "bias": np.zeros(C)},
                               "fc2": {"kernel": np.zeros((C, C)), "bias": np.zeros(C)},
                               "dwconv": {"dwconv": {"kernel": dwk, "bias": np.full(C, 0.25)}}}}
    assert np.array_equal(O.shvit_mlp_half(p, x), x)
    p["mlp"]["fc2"]["kernel"] = np.eye(C)
    mu = x.mean(-1, keepdims=True)
    ln = (x - mu) / np.sqrt(x.var(-1, keepdims=True) + 1e-6)
    assert np.allclose(O.shvit_mlp_half(p, x), x + 1.5 * O.gelu_tanh(ln) + 0.25, rtol=1e-12, atol=1e-12)
    # video: every frame through the same MLP
    xv = rng.standard_normal((B, 3, H, W, C))
    assert np.allclose(O.shvit_mlp_half(p, xv)[:, 1], O.shvit_mlp_half(p, xv[:, 1]), rtol=0, atol=1e-14)
