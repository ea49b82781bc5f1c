"""The float64 gradient reference of the training path (oracle/cssm_cpu_fp32.py at
float64): its forward equals the numpy oracle, and its autograd gradient equals central
finite differences along random directions, for the whole gated layer and for the scan
kernel's own contract (gate planes and K_hat in scan column order).  CPU only."""
import numpy as np
import pytest

from oracle import cssm_oracle as O

torch = pytest.importorskip("torch")
from oracle import cssm_cpu_fp32 as P  # noqa: E402

F64 = torch.float64
LAYERS = [
    dict(channels=4, expand=1, kernel_size=5, gate_type="factored", short_conv_size=0, short_conv_spatial_size=0),
    dict(channels=4, expand=1, kernel_size=3, gate_type="dense", short_conv_size=3, short_conv_spatial_size=3,
         gate_activation="sigmoid"),
    dict(channels=3, expand=2, kernel_size=1, gate_type="factored", short_conv_size=0, short_conv_spatial_size=0,
         gate_activation="exp"),
]


def _layer(kw, shape, seed):
    rng = np.random.default_rng(seed)
    cfg = O.GatedConfig(**kw)
    p = O.init_params(O.gated_param_shapes(cfg, shape[-1], shape[2], shape[3]), rng)
    x = rng.standard_normal(shape)
    return cfg, p, x


def _leaves(tree):
    if isinstance(tree, dict):
        out = []
        for v in tree.values():
            out += _leaves(v)
        return out
    return [tree]


@pytest.mark.parametrize("kw", LAYERS)
def test_float64_layer_forward_equals_oracle(kw):
    cfg, p, x = _layer(kw, (2, 3, 8, 8, kw["channels"]), 0)
    got = P.GatedCPU(p, dtype=F64, **kw)(torch.from_numpy(x)).numpy()
    ref = O.gated_forward(p, x, cfg)
    assert np.max(np.abs(got - ref)) <= 1e-11 * np.sqrt(np.mean(ref ** 2))


@pytest.mark.parametrize("kw", LAYERS)
def test_float64_layer_gradient_equals_finite_differences(kw):
    """<grad L, v> against (L(theta + e v) - L(theta - e v)) / 2e, L = <out, w>, over x and
    every parameter at once, along three random directions."""
    cfg, p, x = _layer(kw, (1, 3, 8, 8, kw["channels"]), 1)
    rng = np.random.default_rng(2)
    m = P.GatedCPU(p, dtype=F64, requires_grad=True, **kw)
    xt = torch.from_numpy(x).requires_grad_(True)
    leaves = [xt] + _leaves(m.p)
    out = m(xt)
    w = torch.from_numpy(rng.standard_normal(out.shape))
    grads = torch.autograd.grad((out * w).sum(), leaves)
    for _ in range(3):
        vs = [torch.from_numpy(rng.standard_normal(t.shape)) for t in leaves]
        analytic = sum(float((g * v).sum()) for g, v in zip(grads, vs))
        eps = 1e-6

        def loss(sign):
            with torch.no_grad():
                for t, v in zip(leaves, vs):
                    t.add_(sign * eps * v)
                val = float((m(xt) * w).sum())
                for t, v in zip(leaves, vs):
                    t.sub_(sign * eps * v)
            return val
        fd = (loss(1.0) - loss(-1.0)) / (2 * eps)
        assert abs(fd - analytic) <= 1e-6 * max(1.0, abs(analytic)), (fd, analytic)


def _core_inputs(rng, B, T, C, H, W):
    Wf = W // 2 + 1
    u = rng.standard_normal((B, T, C, H, W))
    z = rng.standard_normal((B, T, C, H, W))
    delta = O.softplus(rng.standard_normal((B, T, H, Wf)))
    gB, gC = rng.standard_normal((B, T, H, Wf)), rng.standard_normal((B, T, H, Wf))
    kh = O.goom_floor(0.9 * np.exp(2j * np.pi * rng.random((C, H, Wf))) * rng.random((C, H, Wf)))
    return u, z, delta, gB, gC, kh


def test_scan_core_contract_equals_oracle():
    """The kernel-contract restatement (gate planes with the folded GOOM terms, a permuted
    column order) reproduces the oracle's gated_core."""
    rng = np.random.default_rng(3)
    B, T, C, H, W = 2, 4, 3, 8, 8
    u, z, delta, gB, gC, kh = _core_inputs(rng, B, T, C, H, W)
    ref = O.gated_core(u, z, kh, delta, gB, gC)
    cols = np.array([0, 3, 1, 4, 2])                  # any permutation of the Wf columns
    cs = 0.5 / (H * W)
    gates = np.stack([np.exp(-delta), (delta + 1e-8) * gB, 2e-7 * (delta + 1e-8), gC * cs], -1)[:, :, :, cols]
    got = P.scan_core(torch.from_numpy(u), torch.from_numpy(z), torch.from_numpy(gates),
                      torch.from_numpy(kh[:, :, cols]), cs, cols).numpy()
    assert np.max(np.abs(got - ref)) <= 1e-12 * np.sqrt(np.mean(ref ** 2))


def test_scan_core_gradient_equals_finite_differences():
    rng = np.random.default_rng(4)
    B, T, C, H, W = 1, 3, 2, 8, 8
    u, z, delta, gB, gC, kh = _core_inputs(rng, B, T, C, H, W)
    cols = np.arange(W // 2 + 1)
    cs = 0.5 / (H * W)
    gates = np.stack([np.exp(-delta), (delta + 1e-8) * gB, 2e-7 * (delta + 1e-8), gC * cs], -1)
    ts = [torch.from_numpy(a).requires_grad_(True) for a in (u, z, gates, kh)]
    out = P.scan_core(*ts, cs, cols)
    w = torch.from_numpy(rng.standard_normal(out.shape))
    grads = torch.autograd.grad((out * w).sum(), ts)
    for _ in range(3):
        vs = [torch.from_numpy(rng.standard_normal(t.shape) + (1j * rng.standard_normal(t.shape) if t.is_complex()
                                                               else 0)) for t in ts]
        analytic = sum(float((g.conj() * v).real.sum()) if g.is_complex() else float((g * v).sum())
                       for g, v in zip(grads, vs))
        eps = 1e-6

        def loss(sign):
            with torch.no_grad():
                return float((P.scan_core(*[t + sign * eps * v for t, v in zip(ts, vs)], cs, cols) * w).sum())
        fd = (loss(1.0) - loss(-1.0)) / (2 * eps)
        assert abs(fd - analytic) <= 1e-6 * max(1.0, abs(analytic)), (fd, analytic)


def _slots(tree):
    """(dict, key) of every leaf, in the order _leaves lists them."""
    out = []
    for k, v in tree.items():
        out += _slots(v) if isinstance(v, dict) else [(tree, k)]
    return out


def _dot(a, b):
    return float((a.conj() * b).real.sum()) if a.is_complex() else float((a * b).sum())


def test_scan_core_adjoint_identity():
    """<J v, w> (forward mode, torch.func.jvp) = <v, J^T w> (reverse mode) for the scan contract."""
    rng = np.random.default_rng(6)
    B, T, C, H, W = 2, 4, 3, 8, 8
    u, z, delta, gB, gC, kh = _core_inputs(rng, B, T, C, H, W)
    cols = np.array([0, 3, 1, 4, 2])
    cs = 0.5 / (H * W)
    gates = np.stack([np.exp(-delta), (delta + 1e-8) * gB, 2e-7 * (delta + 1e-8), gC * cs], -1)[:, :, :, cols]
    prim = [torch.from_numpy(a) for a in (u, z, gates, kh[:, :, cols])]
    tang = [torch.from_numpy(rng.standard_normal(t.shape) + (1j * rng.standard_normal(t.shape) if t.is_complex()
                                                            else 0)) for t in prim]
    y, jv = torch.func.jvp(lambda *a: P.scan_core(*a, cs, cols), tuple(prim), tuple(tang))
    w = torch.from_numpy(rng.standard_normal(tuple(y.shape)))
    ts = [t.clone().requires_grad_(True) for t in prim]
    g = torch.autograd.grad((P.scan_core(*ts, cs, cols) * w).sum(), ts)
    lhs, rhs = _dot(jv, w), sum(_dot(a, b) for a, b in zip(g, tang))
    assert abs(lhs - rhs) <= 1e-12 * abs(lhs)


@pytest.mark.parametrize("kw", LAYERS)
def test_float64_layer_adjoint_identity(kw):
    """<J v, w> = <v, J^T w> for the whole layer over x and every parameter at once."""
    cfg, p, x = _layer(kw, (2, 3, 8, 8, kw["channels"]), 7)
    rng = np.random.default_rng(8)
    m = P.GatedCPU(p, dtype=F64, **kw)
    slots = _slots(m.p)
    prim = [torch.from_numpy(x)] + [d[k] for d, k in slots]
    tang = [torch.from_numpy(rng.standard_normal(tuple(t.shape))) for t in prim]

    def f(xx, *leaves):
        for (d, k), t in zip(slots, leaves):
            d[k] = t
        return m(xx)
    y, jv = torch.func.jvp(f, tuple(prim), tuple(tang))
    w = torch.from_numpy(rng.standard_normal(tuple(y.shape)))
    ts = [t.detach().clone().requires_grad_(True) for t in prim]
    g = torch.autograd.grad((f(*ts) * w).sum(), ts)
    lhs, rhs = _dot(jv, w), sum(_dot(a, b) for a, b in zip(g, tang))
    assert abs(lhs - rhs) <= 1e-11 * abs(lhs), (lhs, rhs)


# ------------------------------------------------------------------------- GDN cell

GDN_CFGS = [
    dict(gate_type="factored", output_norm="rms", delta_key_dim=4),
    dict(gate_type="dense", output_norm="layer", delta_key_dim=2, qkv_conv_size=3),
    dict(gate_type="channel", output_norm="none", delta_key_dim=4, short_conv_size=0),
    dict(gate_type="scalar", output_norm="rms", delta_key_dim=2, use_input_gates=False, use_spectral_l2_norm=False),
    # the other scan variants: the linear scan (use_log=False) and log(|x| + 1e-8) (use_goom=False)
    dict(gate_type="factored", output_norm="rms", delta_key_dim=2, use_log=False),
    dict(gate_type="dense", output_norm="rms", delta_key_dim=4, use_goom=False),
    # the full-channel qkv conv (qkv_conv_separable=False), an even tap count (SAME pads 1 before, 2 after)
    dict(gate_type="channel", output_norm="rms", delta_key_dim=2, qkv_conv_size=4, qkv_conv_separable=False),
]
GDN_IDS = ["factored", "dense", "channel", "scalar", "factored_linear_scan", "dense_logeps_scan", "full_qkv_conv4"]


def _gdn(kw, shape, seed):
    rng = np.random.default_rng(seed)
    cfg = O.GDNConfig(channels=shape[-1], kernel_size=5, **kw)
    p = O.init_params(O.gdn_param_shapes(cfg, shape[2], shape[3]), rng)
    return cfg, p, rng.standard_normal(shape)


@pytest.mark.parametrize("kw", GDN_CFGS, ids=GDN_IDS)
def test_gdn_float64_forward_equals_oracle(kw):
    cfg, p, x = _gdn(kw, (2, 3, 8, 8, 8), 10)
    ref = O.gdn_forward(p, x, cfg)
    got = P.GdnRef(p, cfg, requires_grad=False)(torch.from_numpy(x)).numpy()
    assert np.max(np.abs(got - ref)) <= 1e-11 * np.sqrt(np.mean(ref ** 2))


@pytest.mark.parametrize("kw", GDN_CFGS, ids=GDN_IDS)
def test_gdn_float64_gradient_equals_finite_differences(kw):
    cfg, p, x = _gdn(kw, (1, 3, 8, 8, 8), 11)
    rng = np.random.default_rng(12)
    m = P.GdnRef(p, cfg)
    xt = torch.from_numpy(x).requires_grad_(True)
    leaves = [xt] + _leaves(m.p)
    out = m(xt)
    w = torch.from_numpy(rng.standard_normal(tuple(out.shape)))
    grads = torch.autograd.grad((out * w).sum(), leaves)
    for _ in range(2):
        vs = [torch.from_numpy(rng.standard_normal(tuple(t.shape))) for t in leaves]
        analytic = sum(float((g * v).sum()) for g, v in zip(grads, vs))
        eps = 1e-6

        def loss(sign):
            with torch.no_grad():
                for t, v in zip(leaves, vs):
                    t.add_(sign * eps * v)
                val = float((m(xt) * w).sum())
                for t, v in zip(leaves, vs):
                    t.sub_(sign * eps * v)
            return val
        fd = (loss(1.0) - loss(-1.0)) / (2 * eps)
        assert abs(fd - analytic) <= 1e-6 * max(1.0, abs(analytic)), (fd, analytic)


def test_gdn_bins_contract_equals_oracle_core():
    """gdn_bins_core (the training kernels' contract: norms applied by the caller) reproduces the
    oracle's gdn_core once the spectral norms and the irfft2 are put around it."""
    rng = np.random.default_rng(13)
    B, T, H, W, C, dk = 2, 3, 8, 8, 8, 4
    nh, Wf = C // dk, W // 2 + 1
    cfg = O.GDNConfig(channels=C, delta_key_dim=dk, gate_type="factored")
    q, k, v = (rng.standard_normal((B, T, H, W, C)) for _ in range(3))
    alpha = 0.1 + 0.89 / (1.0 + np.exp(-rng.standard_normal((B, T, H * Wf))))
    beta = 1.0 / (1.0 + np.exp(-rng.standard_normal((B, T, H * Wf))))
    what = O.spectral_kernel(rng.standard_normal((nh, 5, 5)) * 0.2, H, W, 0.999)
    ref = O.gdn_core(q, k, v, alpha.reshape(B, T, 1, H, Wf), beta.reshape(B, T, 1, H, Wf), what, cfg)
    spec = torch.fft.rfft2(torch.from_numpy(np.concatenate([z.transpose(0, 1, 4, 2, 3) for z in (q, k, v)], 2)))
    qk = spec[:, :, :2 * C]
    qk = qk / torch.sqrt((qk.abs() ** 2).sum(dim=(3, 4), keepdim=True) + 1e-6)
    spec = torch.cat([qk, spec[:, :, 2 * C:]], 2)
    ab = torch.from_numpy(np.stack([alpha, beta], -1))
    ohat = P.gdn_bins_core(spec, ab, torch.from_numpy(what), "factored", dk)
    got = torch.fft.irfft2(ohat, s=(H, W)).numpy()
    assert np.max(np.abs(got - ref)) <= 1e-12 * np.sqrt(np.mean(ref ** 2))


@pytest.mark.parametrize("variant", ["goom", "linear", "log_eps"])
def test_gdn_scan_entry_maps_equal_oracle(variant):
    """The torch references' entry map (and so the training path's gradient reference) is the
    oracle's gdn_scan_entries, on random entries, exact zeros (both signs) and entries at the
    floor's edge."""
    rng = np.random.default_rng(16)
    z = (rng.standard_normal(64) + 1j * rng.standard_normal(64)) * np.logspace(-10, 0, 64)
    z = np.concatenate([z, [0.0, -0.0 + 0j, complex(0, -0.0), 9.9e-8, 1.01e-7]])
    got = P._scan_entries(torch.from_numpy(z), variant).numpy()
    ref = O.gdn_scan_entries(z, variant)
    assert np.max(np.abs(got - ref)) <= 1e-15 * np.max(np.abs(ref)) + 1e-22


def test_gdn_logeps_entry_gradient_is_the_tangential_stretch():
    """d/dx of (|x| + 1e-8) x / |x|: identity along x, (1 + 1e-8 / |x|) across it (what the backward
    kernel's entry adjoint applies); none through the constant at x = 0."""
    x = torch.tensor([3e-8 + 4e-8j, 0.6 - 0.8j, 0j], dtype=torch.complex128, requires_grad=True)
    for g in (1.0 + 0j, 1j):
        y = P._scan_entries(x, "log_eps")
        gr, = torch.autograd.grad(y, x, torch.full_like(y, g))
        xv = x.detach().numpy()
        u = xv[:2] / np.abs(xv[:2])
        expect = g + (1e-8 / np.abs(xv[:2])) * np.real(np.conj(g) * 1j * u) * 1j * u
        assert np.allclose(gr.numpy()[:2], expect, rtol=1e-12, atol=0)
        assert gr.numpy()[2] == 0


def test_gdn_float64_adjoint_identity():
    """<J v, w> (forward mode) = <v, J^T w> (reverse mode) for the GDN layer over x and every parameter."""
    cfg, p, x = _gdn(GDN_CFGS[0], (1, 2, 8, 8, 8), 14)
    rng = np.random.default_rng(15)
    m = P.GdnRef(p, cfg, requires_grad=False)
    slots = _slots(m.p)
    prim = [torch.from_numpy(x)] + [d[k] for d, k in slots]
    tang = [torch.from_numpy(rng.standard_normal(tuple(t.shape))) for t in prim]

    def f(xx, *leaves):
        for (d, k), t in zip(slots, leaves):
            d[k] = t
        return m(xx)
    y, jv = torch.func.jvp(f, tuple(prim), tuple(tang))
    w = torch.from_numpy(rng.standard_normal(tuple(y.shape)))
    ts = [t.detach().clone().requires_grad_(True) for t in prim]
    g = torch.autograd.grad((f(*ts) * w).sum(), ts)
    lhs, rhs = _dot(jv, w), sum(_dot(a, b) for a, b in zip(g, tang))
    assert abs(lhs - rhs) <= 1e-11 * abs(lhs), (lhs, rhs)


@pytest.mark.parametrize("H,W", [(8, 8), (7, 7), (6, 5)])
def test_c2r_weights_give_the_transform_adjoints(H, W):
    """The training path's FFT adjoints (rfft2: dx = H W irfft2(dspec / c_v); irfft2:
    dspec = rfft2(dy) c_v / (H W)) with c_v from training._c2r_weights equal float64 autograd
    of torch.fft on the CPU.  c_v = 1 at v = 0 and at the Nyquist column of even W, else 2: for
    odd W the last column is an interior bin, and weighting it 1 fails here."""
    from cssm_amd import training
    rng = np.random.default_rng(9)
    c = training._c2r_weights(W, "cpu").double()
    Wf = W // 2 + 1
    assert c.shape == (Wf,)
    spec = torch.from_numpy(rng.standard_normal((2, H, Wf)) + 1j * rng.standard_normal((2, H, Wf)))
    spec.requires_grad_(True)
    dy = torch.from_numpy(rng.standard_normal((2, H, W)))
    (g_spec,) = torch.autograd.grad(torch.fft.irfft2(spec, s=(H, W)), spec, dy)
    assert torch.allclose(g_spec, torch.fft.rfft2(dy) * c / (H * W), atol=1e-12)
    x = torch.from_numpy(rng.standard_normal((2, H, W))).requires_grad_(True)
    dspec = torch.from_numpy(rng.standard_normal((2, H, Wf)) + 1j * rng.standard_normal((2, H, Wf)))
    (g_x,) = torch.autograd.grad(torch.fft.rfft2(x), x, dspec)
    # torch's complex gradient convention is conj-linear; dL/dRe + i dL/dIm of a real loss
    assert torch.allclose(g_x, torch.fft.irfft2(dspec / c, s=(H, W)) * (H * W), atol=1e-10)
