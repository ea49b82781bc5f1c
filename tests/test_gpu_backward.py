"""GPU parity of the training path: the HIP scan VJP (batched FFTs around the reverse
recurrence cssm_gated_scan_bwd) and the whole gated layer's gradients (x and every
parameter) against float64 torch autograd of the restatement in oracle/cssm_cpu_fp32.py,
which tests/test_grad_reference.py pins to finite differences and to the numpy oracle.
Bar: max|g_gpu - g_ref| / RMS(g_ref) <= 1e-4 per gradient tensor (fp32 arithmetic); the
adjoint identity <v, J^T w> = <J v, w> against float64 forward-mode AD holds to 1e-4 of
sum |grad| |v| (the fp32 dot product's own error bound)."""
import numpy as np
import pytest

from oracle import cssm_oracle as O
from tests.gpu_util import print_case, rel_err

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu
from oracle import cssm_cpu_fp32 as P  # noqa: E402

TOL = 1e-4
F64 = torch.float64


@pytest.fixture(scope="module")
def mods():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from cssm_amd import cells, spectral, training
    return cells, spectral, training


def _np(t):
    t = t.detach().cpu()
    return t.numpy() if not t.is_complex() else t.numpy().astype(np.complex128)


SCAN_CASES = [(2, 4, 8, 16, 16), (1, 3, 8, 128, 128), (3, 1, 16, 32, 32), (1, 9, 8, 8, 8), (2, 3, 8, 7, 7)]


@pytest.mark.parametrize("shape", SCAN_CASES, ids=[f"{s[3]}x{s[4]}_T{s[1]}" for s in SCAN_CASES])
def test_scan_vjp_matches_float64_reference(mods, shape):
    _, S, _ = mods
    print_case(test="scan_vjp", shape=shape)
    rng = np.random.default_rng(40)
    B, T, C, H, W = shape
    Wf = W // 2 + 1
    cols = np.array(S.scan_col_order(H, W))
    cs = S.scan_c_scale(H, W)
    u, z = rng.standard_normal(shape), rng.standard_normal(shape)
    delta = O.softplus(rng.standard_normal((B, T, H, Wf)))
    gB, gC = rng.standard_normal((B, T, H, Wf)), rng.standard_normal((B, T, H, Wf))
    gates = np.stack([np.exp(-delta), (delta + 1e-8) * gB, 2e-7 * (delta + 1e-8), gC * cs], -1)[:, :, :, cols]
    korder = np.array(S.scan_khat_order(H, W))
    kh = O.goom_floor(0.95 * rng.random((C, H, Wf)) * np.exp(2j * np.pi * rng.random((C, H, Wf))))
    kh = kh.reshape(C, -1)[:, korder].reshape(C, H, Wf)                       # the scan layout
    dy = rng.standard_normal(shape)
    ts = [torch.from_numpy(a).requires_grad_(True) for a in (u, z, gates, kh)]
    ref_y = P.scan_core(*ts, cs, cols, korder)
    refs = torch.autograd.grad(ref_y, ts, torch.from_numpy(dy))
    dev = [torch.from_numpy(np.ascontiguousarray(a)).to("cuda", torch.float32 if a.dtype != np.complex128
                                                         else torch.complex64) for a in (u, z, gates, kh, dy)]
    y = S.gated_scan(*dev[:4])
    got = S.gated_scan_backward(*dev[:4], dev[4], cs)
    torch.cuda.synchronize()
    assert rel_err(_np(y), ref_y.detach().numpy()) <= TOL
    for name, g, r in zip(("du", "dz", "dgates", "dkhat"), got, refs):
        gn, rn = _np(g), r.numpy()
        assert gn.shape == rn.shape, name
        if np.iscomplexobj(rn):
            gn, rn = np.stack([gn.real, gn.imag]), np.stack([rn.real, rn.imag])
        assert rel_err(gn, rn) <= TOL, name


# (gate_type, activation, B, T, C, H, W): C = 64 at 128 x 128 is the C2 layer's frame; small
# planes split each factored product over many threads, 7 x 7 has no Nyquist column
GATE_BWD_CASES = [("factored", "softplus", 2, 3, 64, 128, 128), ("factored", "sigmoid", 3, 2, 16, 8, 8),
                  ("factored", "exp", 2, 2, 32, 32, 32), ("factored", "softplus", 1, 3, 8, 7, 7),
                  ("dense", "exp", 2, 2, 8, 16, 16), ("dense", "softplus", 1, 3, 12, 7, 7),
                  ("dense", "sigmoid", 1, 2, 4, 64, 64)]


@pytest.mark.parametrize("gate_type,act,B,T,C,H,W", GATE_BWD_CASES,
                         ids=[f"{c[0]}_{c[1]}_{c[5]}x{c[6]}" for c in GATE_BWD_CASES])
def test_gated_gates_backward_matches_float64_autograd(mods, gate_type, act, B, T, C, H, W):
    """cssm_gated_gates_bwd against float64 autograd of the gate construction (cssm.py:536-567,
    restated by the oracle's _dense / _gate_act): the gradients of the row / column factors
    (factored) or of the per-bin pre-activations (dense), given a random gradient of the planes."""
    _, S, _ = mods
    print_case(test="gates_bwd", gate_type=gate_type, act=act, shape=(B, T, C, H, W))
    rng = np.random.default_rng(43)
    Wf = W // 2 + 1
    cols = np.array(S.scan_col_order(H, W))
    cs = S.scan_c_scale(H, W)
    ctx = rng.standard_normal((B, T, C))
    names = ("delta_proj", "B_proj", "C_proj")
    if gate_type == "factored":
        parts = {f"{n}_{a}": (C, H if a == "h" else Wf) for n in names for a in ("h", "w")}
    else:
        parts = {n: (C, H * Wf) for n in names}
    p = {k: {"kernel": rng.standard_normal(sh) / np.sqrt(C), "bias": 0.5 * rng.standard_normal(sh[1])}
         for k, sh in parts.items()}
    pt = {k: {kk: torch.from_numpy(vv) for kk, vv in v.items()} for k, v in p.items()}
    ct = torch.from_numpy(ctx)
    if gate_type == "factored":
        leaves = [P._dense(ct, pt[f"{n}_{a}"]).requires_grad_(True) for n in names for a in ("h", "w")]
        G = [leaves[2 * i][..., :, None] * leaves[2 * i + 1][..., None, :] for i in range(3)]
    else:
        leaves = [P._dense(ct, pt[n]).requires_grad_(True) for n in names]
        G = [g.reshape(B, T, H, Wf) for g in leaves]
    d = P._gate_act(G[0], act)
    planes = torch.stack([torch.exp(-d), (d + 1e-8) * G[1], 2e-7 * (d + 1e-8), G[2] * cs], -1)
    dp = rng.standard_normal((B, T, H, Wf, 4))
    refs = torch.autograd.grad(planes, leaves, torch.from_numpy(dp))
    ref = torch.cat([r.reshape(B, T, -1) for r in refs], dim=-1).numpy()

    dev = {k: {kk: torch.from_numpy(vv).to("cuda", torch.float32) for kk, vv in v.items()} for k, v in p.items()}
    cd = torch.from_numpy(ctx).to("cuda", torch.float32)
    dgates = torch.from_numpy(np.ascontiguousarray(dp[:, :, :, cols])).to("cuda", torch.float32)
    got = S.gated_gates_backward(cd, dev, H, W, dgates, gate_type, act, cs)
    torch.cuda.synchronize()
    assert got.shape == (B, T, 3, H + Wf if gate_type == "factored" else H * Wf)
    assert rel_err(_np(got).reshape(B, T, -1), ref) <= TOL
    # the forward of the same parameters, for the same planes
    fwd = S.gated_gates(cd, dev, H, W, gate_type, act, cs)
    assert rel_err(_np(fwd), planes.detach().numpy()[:, :, :, cols]) <= TOL


LAYER_CASES = [
    ("factored_16", (2, 3, 16, 16, 8), dict(channels=8, kernel_size=5, gate_type="factored", short_conv_size=0,
                                            short_conv_spatial_size=0)),
    ("dense_convs_sigmoid_8", (1, 4, 8, 8, 8), dict(channels=8, kernel_size=3, gate_type="dense", short_conv_size=3,
                                                    short_conv_spatial_size=3, gate_activation="sigmoid")),
    ("c1_expand2_T1_k1", (4, 1, 32, 32, 16), dict(channels=16, expand=2, kernel_size=1, gate_type="factored",
                                                  short_conv_size=0, short_conv_spatial_size=0)),
    ("factored_128_exp", (1, 2, 128, 128, 4), dict(channels=4, kernel_size=11, gate_type="factored",
                                                   gate_activation="exp", short_conv_size=2,
                                                   short_conv_spatial_size=0)),
    # odd planes: the last column is an interior bin (no Nyquist column), weight 2 in the C2R rule
    ("factored_7x7_odd", (2, 2, 7, 7, 8), dict(channels=8, kernel_size=3, gate_type="factored", short_conv_size=0,
                                               short_conv_spatial_size=0)),
    # no short convs on power-of-two planes: in_proj through the scan as one node with the fused
    # transforms (cssm_rfft2_ex / cssm_irfft2_ex) in its backward
    ("dense_128_fused_node", (1, 2, 128, 128, 4), dict(channels=4, kernel_size=11, gate_type="dense",
                                                       short_conv_size=0, short_conv_spatial_size=0)),
    ("factored_4x4_expand2_fused_node", (3, 2, 4, 4, 8), dict(channels=8, expand=2, kernel_size=1,
                                                               gate_type="factored", gate_activation="sigmoid",
                                                               short_conv_size=0, short_conv_spatial_size=0)),
    ("factored_32_exp_fused_node", (2, 3, 32, 32, 8), dict(channels=8, kernel_size=7, gate_type="factored",
                                                            gate_activation="exp", short_conv_size=0,
                                                            short_conv_spatial_size=0)),
]


# (128, 150, 4) and (64, 261, 9): more plane groups than the persistent forward transform keeps
# resident, so workgroups take a second group (its loads issued during the first one's passes), the
# last group of the 64 x 64 case partial
@pytest.mark.parametrize("H,F,C", [(128, 2, 3), (64, 2, 4), (32, 3, 4), (8, 2, 8), (4, 3, 2), (128, 150, 4),
                                   (64, 261, 9)])
def test_fused_training_transforms_match_torch(mods, H, F, C):
    """cssm_rfft2_ex / cssm_irfft2_ex on the halves of a plane-major (F, 2C, HW) tensor (frame
    stride 2C) against torch's FFTs of the same elementwise expressions."""
    _, S, _ = mods
    print_case(test="fft_ex", H=H, F=F, C=C)
    rng = np.random.default_rng(46)
    W, HW, Wf = H, H * H, H // 2 + 1
    xz = torch.from_numpy(rng.standard_normal((F, 2 * C, HW))).to("cuda", torch.float32)
    dy = torch.from_numpy(rng.standard_normal((F, C, HW))).to("cuda", torch.float32)
    xm, z = xz[:, :C], xz[:, C:]
    silu, sg = torch.nn.functional.silu, torch.sigmoid
    d64 = lambda t: t.double().cpu()
    ref_u = torch.fft.rfft2(silu(d64(xm)).view(F, C, H, W))
    ref_d = torch.fft.rfft2((d64(dy) * silu(d64(z))).view(F, C, H, W))
    got_u = S.rfft2_ex(xm, H, W, x_silu=True)
    got_d = S.rfft2_ex(dy, H, W, a=z, a_silu=True)
    torch.cuda.synchronize()
    for g, r in ((got_u, ref_u), (got_d, ref_d)):
        assert rel_err(torch.view_as_real(g).cpu().numpy(), torch.view_as_real(r).numpy()) <= 1e-5
    spec = torch.from_numpy(rng.standard_normal((F, C, H, Wf)) + 1j * rng.standard_normal((F, C, H, Wf))).to(
        "cuda", torch.complex64)
    add = torch.from_numpy(rng.standard_normal((F, C))).to("cuda", torch.float32)
    out = torch.full((F, 2 * C, HW), 7.0, device="cuda")
    sums_ok = S.irfft2_ex_sums_supported(F * C, H, W)
    sums = torch.full((2, F, C), 7.0, device="cuda") if sums_ok else None
    S.irfft2_ex(spec, W, out[:, C:], m=dy, d=z, sums=sums[1] if sums_ok else None)
    S.irfft2_ex(spec, W, out[:, :C], add=add, d=xm, sums=sums[0] if sums_ok else None)
    torch.cuda.synchronize()
    if sums_ok:
        ps = out.view(F, 2, C, HW).sum(dim=3).transpose(0, 1).double().cpu()
        assert rel_err(sums.cpu().numpy(), ps.numpy()) <= 1e-5
    base = torch.fft.irfft2(spec.cpu().to(torch.complex128), s=(H, W)).view(F, C, HW)
    dsilu = lambda v: sg(v) * (1 + v * (1 - sg(v)))
    ref_hi = base * d64(dy) * dsilu(d64(z))
    ref_lo = (base + d64(add)[:, :, None]) * dsilu(d64(xm))
    assert rel_err(out[:, C:].cpu().numpy(), ref_hi.numpy()) <= 1e-5
    assert rel_err(out[:, :C].cpu().numpy(), ref_lo.numpy()) <= 1e-5


def _leaves(tree, prefix=""):
    if isinstance(tree, dict):
        out = []
        for k, v in tree.items():
            out += _leaves(v, f"{prefix}/{k}")
        return out
    return [(prefix, tree)]


@pytest.mark.parametrize("name,shape,kw", LAYER_CASES, ids=[c[0] for c in LAYER_CASES])
def test_layer_gradients_match_float64_reference(mods, name, shape, kw):
    cells, _, training = mods
    print_case(test="layer_grad", case=name)
    rng = np.random.default_rng(41)
    cfg = O.GatedConfig(**kw)
    p = O.init_params(O.gated_param_shapes(cfg, shape[-1], shape[2], shape[3]), rng)
    x = rng.standard_normal(shape)
    ref_m = P.GatedCPU(p, dtype=F64, requires_grad=True, **kw)
    xr = torch.from_numpy(x).requires_grad_(True)
    out_r = ref_m(xr)
    w = rng.standard_normal(tuple(out_r.shape))
    ref_leaves = [("x", xr)] + _leaves(ref_m.p)
    refs = torch.autograd.grad((out_r * torch.from_numpy(w)).sum(), [t for _, t in ref_leaves])

    cell = cells.GatedCSSM(**kw)
    v = cells.GatedCSSM.load_params(p)
    leaves = _leaves(v["params"])
    for _, t in leaves:
        t.requires_grad_(True)
    xd = torch.from_numpy(x).to("cuda", torch.float32).requires_grad_(True)
    out = training.gated_train_apply(cell, v, xd)
    with torch.no_grad():
        assert rel_err(_np(out), out_r.detach().numpy()) <= TOL
        assert rel_err(_np(out), _np(cell.apply(v, xd.detach()))) <= 1e-5
    grads = torch.autograd.grad((out * torch.from_numpy(w).to("cuda", torch.float32)).sum(),
                                [xd] + [t for _, t in leaves])
    torch.cuda.synchronize()
    names = ["x"] + [n for n, _ in leaves]
    assert names == [n for n, _ in ref_leaves]
    for n, g, r in zip(names, grads, refs):
        assert rel_err(_np(g), r.numpy()) <= TOL, n


def _dot(a, b):
    return float((a.conj() * b).real.sum()) if a.is_complex() else float((a * b).sum())


@pytest.mark.parametrize("name,shape,kw", LAYER_CASES[:2], ids=[c[0] for c in LAYER_CASES[:2]])
def test_layer_vjp_adjoint_to_float64_jvp(mods, name, shape, kw):
    """<v, J^T w> from the HIP backward equals <J v, w> from float64 forward-mode AD of the
    restatement (a derivative computed without any reverse pass), over x and every parameter."""
    cells, _, training = mods
    print_case(test="layer_adjoint", case=name)
    rng = np.random.default_rng(42)
    cfg = O.GatedConfig(**kw)
    p = O.init_params(O.gated_param_shapes(cfg, shape[-1], shape[2], shape[3]), rng)
    x = rng.standard_normal(shape)
    m = P.GatedCPU(p, dtype=F64, **kw)
    slots = []

    def collect(tree):
        for k, v in tree.items():
            collect(v) if isinstance(v, dict) else slots.append((tree, k))
    collect(m.p)
    prim = [torch.from_numpy(x)] + [d[k] for d, k in slots]
    tang = [torch.from_numpy(rng.standard_normal(tuple(t.shape))) for t in prim]

    def f(xx, *leaves):
        for (d, k), t in zip(slots, leaves):
            d[k] = t
        return m(xx)
    y, jv = torch.func.jvp(f, tuple(prim), tuple(tang))
    w = torch.from_numpy(rng.standard_normal(tuple(y.shape)))
    lhs = _dot(jv, w)

    cell = cells.GatedCSSM(**kw)
    v = cells.GatedCSSM.load_params(p)
    leaves = _leaves(v["params"])
    assert [n for n, _ in leaves] == [n for n, _ in _leaves(m.p)]        # tangents pair with gradients
    for _, t in leaves:
        t.requires_grad_(True)
    xd = torch.from_numpy(x).to("cuda", torch.float32).requires_grad_(True)
    out = training.gated_train_apply(cell, v, xd)
    grads = torch.autograd.grad((out * w.to("cuda", torch.float32)).sum(), [xd] + [t for _, t in leaves])
    torch.cuda.synchronize()
    rhs = sum(_dot(g.double().cpu(), t) for g, t in zip(grads, tang))
    scale = sum(float(g.double().cpu().norm() * t.norm()) for g, t in zip(grads, tang))
    assert abs(lhs - rhs) <= 1e-4 * scale, (lhs, rhs, scale)


# ------------------------------------------------------------------------- GDN cell

BINS_CASES = [("factored", 4, 16, False, "goom"), ("dense", 2, 8, False, "goom"), ("channel", 4, 8, False, "goom"),
              ("scalar", 1, 8, False, "goom"), ("factored_floored", 4, 16, True, "goom"),
              ("factored_zeros_linear", 4, 16, True, "linear"), ("dense_linear", 2, 8, False, "linear"),
              ("factored_zeros_logeps", 4, 16, True, "log_eps"), ("channel_logeps", 2, 8, False, "log_eps")]


@pytest.mark.parametrize("name,dk,H,floored,variant", BINS_CASES, ids=[c[0] for c in BINS_CASES])
def test_gdn_bins_vjp_matches_float64_reference(mods, name, dk, H, floored, variant):
    """cssm_gdn_scan_bins_train / _bwd through the autograd Function (its per-gate-type sums of
    the (alpha, beta) gradients included) against float64 autograd of the kernel contract under
    each scan variant.  The floored cases zero the keys of head 0 and the values of head 2, so
    M and Delta hold exact zeros there: to_goom's floor and the log-eps map's 1e-8 take them
    (a constant, which passes no gradient), the linear scan keeps them."""
    _, S, training = mods
    print_case(test="gdn_bins_vjp", case=name)
    gt = name.split("_")[0]
    rng = np.random.default_rng(43)
    B, T, C, W = 2, 5, 16, H
    nh, Wf = C // dk, W // 2 + 1
    spec = rng.standard_normal((B, T, 3 * C, H, Wf)) + 1j * rng.standard_normal((B, T, 3 * C, H, Wf))
    spec[:, :, :C] *= 0.05
    spec[:, :, C:2 * C] *= 0.05
    if floored:
        spec[:, :, C:C + dk] = 0.0
        spec[:, :, 2 * C + 2 * dk:2 * C + 3 * dk] = 0.0
    n_ab = {"factored": H * Wf, "dense": H * Wf, "channel": nh, "scalar": 1}[gt]
    alpha = 0.1 + 0.89 / (1.0 + np.exp(-rng.standard_normal((B, T, n_ab))))
    beta = 1.0 / (1.0 + np.exp(-rng.standard_normal((B, T, n_ab))))
    ab = np.stack([alpha, beta], -1)
    what = O.spectral_kernel(rng.standard_normal((nh, 5, 5)) * 0.2, H, W, 0.999)
    dohat = rng.standard_normal((B, T, C, H, Wf)) + 1j * rng.standard_normal((B, T, C, H, Wf))
    ts = [torch.from_numpy(a).requires_grad_(True) for a in (spec, ab, what)]
    ref = P.gdn_bins_core(ts[0], ts[1], ts[2], gt, dk, variant)
    refs = torch.autograd.grad(ref, ts, torch.from_numpy(dohat))
    dev = [torch.from_numpy(spec).to("cuda", torch.complex64).requires_grad_(True),
           torch.from_numpy(ab).to("cuda", torch.float32).requires_grad_(True),
           torch.from_numpy(what).to("cuda", torch.complex64).requires_grad_(True)]
    out = training._GdnBinsFn.apply(dev[0], dev[1], dev[2], gt, dk, variant)
    got = torch.autograd.grad(out, dev, torch.from_numpy(dohat).to("cuda", torch.complex64))
    torch.cuda.synchronize()
    assert rel_err(_ri(out), _ri(ref)) <= TOL
    for n, g, r in zip(("dspec", "dab", "dwhat"), got, refs):
        assert g.shape == r.shape, n
        assert rel_err(_ri(g), _ri(r)) <= TOL, n


def _ri(t):
    """Real and imaginary parts stacked (float64 numpy) for the parity metric."""
    a = t.detach().cpu().numpy()
    return np.stack([a.real, a.imag]).astype(np.float64) if np.iscomplexobj(a) else a.astype(np.float64)


GDN_LAYER_CASES = [
    ("factored_rms_16", (1, 3, 16, 16, 8), dict(gate_type="factored", output_norm="rms", delta_key_dim=4)),
    ("dense_layer_qkvdw_8", (2, 2, 8, 8, 8), dict(gate_type="dense", output_norm="layer", delta_key_dim=2,
                                                  qkv_conv_size=3)),
    ("channel_none_noconv_16", (1, 4, 16, 16, 8), dict(gate_type="channel", output_norm="none", delta_key_dim=4,
                                                       short_conv_size=0)),
    ("scalar_nol2_32", (1, 2, 32, 32, 4), dict(gate_type="scalar", output_norm="rms", delta_key_dim=2,
                                               use_input_gates=False, use_spectral_l2_norm=False)),
    ("factored_14x14_small_planes", (2, 3, 14, 14, 8), dict(gate_type="factored", output_norm="rms",
                                                           delta_key_dim=4, qkv_conv_size=3)),
    # odd planes (the 7 x 7 SHViT stage): the transforms' adjoints weight the last column 2
    ("factored_7x7_odd_planes", (2, 3, 7, 7, 8), dict(gate_type="factored", output_norm="rms", delta_key_dim=4)),
    # the scan variants of use_log=False (linear) and use_goom=False (log(|x| + 1e-8))
    ("factored_linear_scan_16", (1, 3, 16, 16, 8), dict(gate_type="factored", output_norm="rms", delta_key_dim=4,
                                                        use_log=False)),
    ("channel_logeps_scan_8", (2, 2, 8, 8, 8), dict(gate_type="channel", output_norm="rms", delta_key_dim=2,
                                                    use_goom=False)),
    # the k x k full-channel qkv conv (qkv_conv_separable=False), odd and even tap counts
    ("factored_full_qkv_conv3_16", (1, 3, 16, 16, 8), dict(gate_type="factored", output_norm="rms",
                                                          delta_key_dim=4, qkv_conv_size=3,
                                                          qkv_conv_separable=False)),
    ("channel_full_qkv_conv4_8", (2, 2, 8, 8, 8), dict(gate_type="channel", output_norm="rms", delta_key_dim=2,
                                                       qkv_conv_size=4, qkv_conv_separable=False)),
]


@pytest.mark.parametrize("name,shape,kw", GDN_LAYER_CASES, ids=[c[0] for c in GDN_LAYER_CASES])
def test_gdn_layer_gradients_match_float64_reference(mods, name, shape, kw):
    cells, _, training = mods
    print_case(test="gdn_layer_grad", case=name)
    rng = np.random.default_rng(44)
    cfg = O.GDNConfig(channels=shape[-1], kernel_size=5, **kw)
    p = O.init_params(O.gdn_param_shapes(cfg, shape[2], shape[3]), rng)
    x = rng.standard_normal(shape)
    ref_m = P.GdnRef(p, cfg)
    xr = torch.from_numpy(x).requires_grad_(True)
    out_r = ref_m(xr)
    w = rng.standard_normal(tuple(out_r.shape))
    ref_leaves = [("x", xr)] + _leaves(ref_m.p)
    refs = torch.autograd.grad((out_r * torch.from_numpy(w)).sum(), [t for _, t in ref_leaves])

    cell = cells.GatedDeltaNetCSSM(channels=shape[-1], kernel_size=5, **kw)
    v = cells.GatedDeltaNetCSSM.load_params(p)
    leaves = _leaves(v["params"])
    for _, t in leaves:
        t.requires_grad_(True)
    xd = torch.from_numpy(x).to("cuda", torch.float32).requires_grad_(True)
    out = training.gdn_train_apply(cell, v, xd)
    with torch.no_grad():
        assert rel_err(_np(out), out_r.detach().numpy()) <= TOL
        assert rel_err(_np(out), _np(cell.apply(v, xd.detach()))) <= 2e-5
    grads = torch.autograd.grad((out * torch.from_numpy(w).to("cuda", torch.float32)).sum(),
                                [xd] + [t for _, t in leaves])
    torch.cuda.synchronize()
    names = ["x"] + [n for n, _ in leaves]
    assert names == [n for n, _ in ref_leaves]
    for n, g, r in zip(names, grads, refs):
        assert rel_err(_np(g), r.numpy()) <= TOL, n


DW_CASES = [(3, (2, 16, 16, 8)), (5, (3, 8, 24, 16)), (7, (1, 12, 16, 64)), (5, (4, 32, 32, 4))]


@pytest.mark.parametrize("ks,shape", DW_CASES, ids=[f"k{c[0]}_{c[1][1]}x{c[1][2]}_C{c[1][3]}" for c in DW_CASES])
def test_depthwise_conv_vjp_matches_float64(mods, ks, shape):
    """The training path's depthwise SAME conv (HIP forward, flipped-tap data gradient, the
    weight-gradient kernel) against float64 autograd of torch's grouped conv."""
    _, S, training = mods
    print_case(test="dwconv_vjp", ks=ks, shape=shape)
    rng = np.random.default_rng(45)
    F, H, W, C = shape
    assert S.depthwise_conv_wgrad_supported(W, C, ks)
    x, k, b = rng.standard_normal(shape), rng.standard_normal((ks, ks, 1, C)) / ks, rng.standard_normal(C)
    dy = rng.standard_normal(shape)
    ts = [torch.from_numpy(a).requires_grad_(True) for a in (x, k, b)]
    lo, hi = (ks - 1) // 2, ks // 2
    ref = (torch.nn.functional.conv2d(torch.nn.functional.pad(ts[0].permute(0, 3, 1, 2), (lo, hi, lo, hi)),
                                      ts[1].permute(3, 2, 0, 1), groups=C) + ts[2][None, :, None, None]).permute(0, 2, 3, 1)
    refs = torch.autograd.grad(ref, ts, torch.from_numpy(dy))
    dev = [torch.from_numpy(a).to("cuda", torch.float32).requires_grad_(True) for a in (x, k, b)]
    out = training._DwConvFn.apply(*dev)
    got = torch.autograd.grad(out, dev, torch.from_numpy(dy).to("cuda", torch.float32))
    torch.cuda.synchronize()
    assert rel_err(_np(out), ref.detach().numpy()) <= 1e-5
    for n, g, r in zip(("dx", "dkernel", "dbias"), got, refs):
        assert rel_err(_np(g), r.numpy()) <= TOL, n
