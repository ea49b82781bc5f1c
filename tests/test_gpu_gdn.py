"""GPU parity of the GatedDeltaNetCSSM (`gdn`) kernels and layer against the
float64 oracle (oracle/cssm_oracle.py) and numpy, all through the C ABI.

Bar: max|y_gpu - y_ref| / RMS(y_ref) <= 1e-4 with
fp32 I/O, <= 5e-3 with bf16 I/O.
"""
import numpy as np
import pytest

from oracle import cssm_oracle as O
from tests.gpu_util import bf16_excess_err, print_case, rel_err, to_np

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

TOL_F32 = 1e-4
TOL_BF16 = 5e-3


@pytest.fixture(scope="module")
def mods():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from cssm_amd import cells, spectral
    return cells, spectral


def _dev(a, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda", dtype)


def _tree(p):
    if isinstance(p, dict):
        return {k: _tree(v) for k, v in p.items()}
    return _dev(p)


# ------------------------------------------------------- batched transforms

# powers of two 4..128 run the LDS radix passes; the other sizes 3..15 the direct small-plane DFTs
# (P not a multiple of a group's planes: the last group is partial)
FFT_SIZES = [(6, 128), (8, 64), (12, 32), (16, 16), (64, 8), (128, 4),
             (40, 14), (67, 7), (30, 3), (21, 5), (17, 15), (9, 12), (33, 6)]


@pytest.mark.parametrize("P,H", FFT_SIZES)
@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_rfft2_and_norms_match_numpy(mods, P, H, dt):
    _, S = mods
    print_case(test="rfft2", P=P, H=H, dtype=dt)
    rng = np.random.default_rng(P * H)
    x = rng.standard_normal((P, H, H))
    xd = _dev(x, torch.float32 if dt == "f32" else torch.bfloat16)
    spec, norms = S.rfft2(xd, want_norms=True)
    xr = to_np(xd)                                   # the (rounded) input the kernel saw
    ref = np.fft.rfft2(xr)
    got = spec.cpu().numpy().astype(np.complex128)
    assert np.max(np.abs(got - ref)) / np.sqrt(np.mean(np.abs(ref) ** 2)) < 2e-6
    assert rel_err(to_np(norms), np.sum(np.abs(ref) ** 2, axis=(1, 2))) < 2e-6


@pytest.mark.parametrize("P,H,dt", [(1100, 128, "f32"), (1100, 128, "bf16"), (2049, 64, "f32"), (6403, 32, "f32")])
def test_rfft2_more_groups_than_resident_workgroups(mods, P, H, dt):
    """The persistent forward transform (128 x 128) with more planes than workgroups resident at
    once (512 on 256 CUs): later planes are loaded during earlier planes' passes; 64 and 32 run one
    plane group per workgroup (partial last groups).  Then the inverse, persistent at 128 and 64,
    over the same spectra."""
    _, S = mods
    print_case(test="rfft2_groups", P=P, H=H, dtype=dt)
    x = torch.randn((P, H, H), device="cuda", generator=torch.Generator(device="cuda").manual_seed(P))
    x = x if dt == "f32" else x.to(torch.bfloat16)
    spec, norms = S.rfft2(x, want_norms=True)
    ref = np.fft.rfft2(to_np(x).astype(np.float64))
    got = spec.cpu().numpy().astype(np.complex128)
    assert np.max(np.abs(got - ref)) / np.sqrt(np.mean(np.abs(ref) ** 2)) < 2e-6
    assert rel_err(to_np(norms), np.sum(np.abs(ref) ** 2, axis=(1, 2))) < 2e-6
    y = S.irfft2(spec, H)
    yref = np.fft.irfft2(got, s=(H, H))
    assert rel_err(to_np(y), yref) < 2e-6
    if dt == "bf16":
        yb = S.irfft2(spec, H, out_dtype=torch.bfloat16)   # the float result rounded once
        assert bf16_excess_err(to_np(yb), yref) < 2e-5


@pytest.mark.parametrize("P,H", FFT_SIZES)
def test_irfft2_c2r_rule_matches_numpy(mods, P, H):
    _, S = mods
    print_case(test="irfft2", P=P, H=H)
    rng = np.random.default_rng(H)
    Wf = H // 2 + 1
    # arbitrary (non-Hermitian) spectra: only the C2R-surviving part may reach y
    X = rng.standard_normal((P, H, Wf)) + 1j * rng.standard_normal((P, H, Wf))
    y = S.irfft2(_dev(X, torch.complex64), H)
    ref = np.fft.irfft2(X.astype(np.complex64).astype(np.complex128), s=(H, H))
    assert rel_err(to_np(y), ref) < 2e-6


def test_rfft2_irfft2_round_trip_full_c3_plane_count(mods):
    """Size-independent check at C3's full plane count (B*T*3C = 128*8*192 = 196,608 planes of
    128x128, the q/k/v planes one C3 layer transforms): irfft2(rfft2(x)) = x.  ~39 GB resident."""
    _, S = mods
    P = 128 * 8 * 3 * 64
    print_case(test="fft_round_trip", P=P, H=128)
    x = torch.randn((P, 128, 128), device="cuda", generator=torch.Generator(device="cuda").manual_seed(5))
    rms = float(x.pow(2).mean().sqrt())
    spec, _ = S.rfft2(x)
    y = S.irfft2(spec, 128)
    del spec
    err = float(y.sub_(x).abs_().max())
    del x, y
    torch.cuda.empty_cache()
    assert err / rms < 2e-6


# ------------------------------------------------------------ prologue ops

@pytest.mark.parametrize("act", ["identity", "silu", "sigmoid"])
def test_proj_planes(mods, act):
    _, S = mods
    print_case(test="proj_planes", act=act)
    rng = np.random.default_rng(3)
    F, HW, K, N = 3, 1024, 64, 192
    x = rng.standard_normal((F * HW, K))
    Wt = rng.standard_normal((K, N)) / 8
    b = rng.standard_normal(N) * 0.1
    out = S.proj_planes(_dev(x), _dev(Wt), _dev(b), F, HW, act=act)
    ref = (x @ Wt + b).reshape(F, HW, N).transpose(0, 2, 1)
    ref = {"identity": ref, "silu": O.silu(ref), "sigmoid": O.sigmoid(ref)}[act]
    assert rel_err(to_np(out), ref) < 1e-5


@pytest.mark.parametrize("shape", [(2, 3, 16, 12, 20), (1, 2, 7, 8, 12), (1, 2, 32, 32, 64), (1, 2, 14, 8, 16),
                                   (1, 1, 8, 8, 336)])
def test_frame_mean_and_depthwise_conv(mods, shape):
    """Register-blocked (ks 3/5/7, even H, W % 4, C % 4: 8 rows per thread when H % 8 == 0, else 2;
    taps from LDS when C ks^2 <= 8192, as at C = 336 for ks 3 but not 5 / 7) and general depthwise
    convs, f32 and bf16 in."""
    _, S = mods
    print_case(test="frame_mean_dwconv", shape=shape)
    rng = np.random.default_rng(4)
    B, T, H, W, C = shape
    x = rng.standard_normal(shape)
    m = S.frame_mean(_dev(x))
    assert rel_err(to_np(m), x.mean(axis=(2, 3))) < 1e-6
    for ks in (5, 3, 4, 7):
        p = {"kernel": rng.standard_normal((ks, ks, 1, C)) / ks, "bias": rng.standard_normal(C) * 0.1}
        y = S.depthwise_conv(_dev(x), _dev(p["kernel"]), _dev(p["bias"]))
        ref = O.depthwise_conv2d_same(x.reshape(B * T, H, W, C), p).reshape(x.shape)
        assert rel_err(to_np(y), ref) < 5e-6, ks            # fp32 sums of up to 49 taps
        xb = _dev(x, torch.bfloat16)
        yb = S.depthwise_conv(xb, _dev(p["kernel"]), _dev(p["bias"]), out_dtype=torch.float32)
        refb = O.depthwise_conv2d_same(to_np(xb).reshape(B * T, H, W, C), p).reshape(x.shape)
        assert rel_err(to_np(yb), refb) < 5e-6, ks
        # bf16 out: the fp32 result rounded once to nearest even
        ybb = S.depthwise_conv(xb, _dev(p["kernel"]), _dev(p["bias"]), out_dtype=torch.bfloat16)
        assert ybb.dtype == torch.bfloat16
        assert bf16_excess_err(to_np(ybb), refb) < 2e-5, ks
        # taps and bias 4 bytes off a 16-byte boundary: the per-channel kernel, same values
        kbuf = torch.zeros(ks * ks * C + C + 2, device="cuda")
        kbuf[1:1 + ks * ks * C] = _dev(p["kernel"]).flatten()
        kbuf[2 + ks * ks * C:] = _dev(p["bias"])
        kmis, bmis = kbuf[1:1 + ks * ks * C].view(ks, ks, 1, C), kbuf[2 + ks * ks * C:]
        assert kmis.data_ptr() % 16 != 0
        ym = S.depthwise_conv(_dev(x), kmis, bmis)
        assert rel_err(to_np(ym), ref) < 5e-6, ks


# (B, T): the factored gates run 4, 2 or 1 frames per block as B T divides (6 -> 2, 8 -> 4, 5 -> 1)
@pytest.mark.parametrize("bt", [(2, 3), (2, 4), (1, 5)])
@pytest.mark.parametrize("gate_type", ["factored", "dense", "channel", "scalar"])
def test_gdn_gates_match_oracle(mods, gate_type, bt):
    _, S = mods
    print_case(test="gdn_gates", gate_type=gate_type, bt=bt)
    rng = np.random.default_rng(5)
    (B, T), H, W, C, dk = bt, 16, 16, 8, 2
    cfg = O.GDNConfig(channels=C, delta_key_dim=dk, gate_type=gate_type)
    p = O.init_params(O.gdn_param_shapes(cfg, H, W), rng)
    ctx = rng.standard_normal((B, T, C))
    ab, bkv = S.gdn_gates(_dev(ctx), _tree(p), H, W, dk, gate_type, True)
    ctx_t = ctx + O.temporal_context_encoding(T, C)[None]
    Wf = W // 2 + 1
    al = O.gdn_gate("alpha", p, cfg, ctx_t, None, H, W, bounded=True)
    be = O.gdn_gate("beta", p, cfg, ctx_t, None, H, W)
    ab_np = to_np(ab)
    n = ab_np.shape[2]
    assert rel_err(ab_np[..., 0], np.asarray(al).reshape(B, T, n)) < 1e-5
    assert rel_err(ab_np[..., 1], np.asarray(be).reshape(B, T, n)) < 1e-5
    if gate_type != "channel":
        bk = O.gdn_gate("B_k", p, cfg, ctx_t, None, H, W, spatial=True)
        bv = O.gdn_gate("B_v", p, cfg, ctx_t, None, H, W, spatial=True)
        m = bkv.shape[2]
        assert rel_err(to_np(bkv)[..., 0], np.asarray(bk).reshape(B, T, m)) < 1e-5
        assert rel_err(to_np(bkv)[..., 1], np.asarray(bv).reshape(B, T, m)) < 1e-5
    assert n == {"factored": H * Wf, "dense": H * Wf, "channel": C // dk, "scalar": 1}[gate_type]


@pytest.mark.parametrize("kt", [4, 0, 2])
def test_gdn_qkv_post_matches_oracle(mods, kt):
    _, S = mods
    print_case(test="gdn_qkv_post", kt=kt)
    rng = np.random.default_rng(6)
    B, T, C, H, W = 2, 5, 6, 8, 8
    qkv = rng.standard_normal((B, T, 3 * C, H, W))
    convs = [{"kernel": rng.standard_normal((kt, 1, C)) / 2, "bias": rng.standard_normal(C) * 0.1}
             for _ in range(3)] if kt else None
    gates = 1.0 / (1.0 + np.exp(-rng.standard_normal((B, T, H * W, 2))))
    got = S.gdn_qkv_post(_dev(qkv), [_tree(c) for c in convs] if convs else None, 1, _dev(gates))
    cl = qkv.reshape(B, T, 3, C, H, W).transpose(0, 1, 4, 5, 2, 3)       # (B, T, H, W, 3, C)
    outs = []
    for i in range(3):
        z = cl[..., i, :]
        if convs:
            z = O.silu(O.causal_conv_t(z, convs[i]))
        if i > 0:
            z = z * gates[..., i - 1].reshape(B, T, H, W, 1)
        outs.append(z)
    ref = np.stack(outs, axis=4).transpose(0, 1, 4, 5, 2, 3).reshape(qkv.shape)
    assert rel_err(to_np(got), ref) < 1e-5


# (B, T, H, W, K, C): with H*W a multiple of 64 and kt <= 4 (or T <= 4) one frame-sequential kernel
# (any T); else T = 4 or a multiple of 8 (chunks of 8 frames carrying 3, kt <= 4) with H*W a
# multiple of 128 / min(T, 8) the tiled kernel ((1, 4, 4, 8): T = 4; (1, 8, 4, 4): T = 8;
# (2, 24, 4, 4): chunks); the rest (kt = 6 at T = 8 or 16; T = 3 at 4 x 4) through proj_planes +
# qkv_post
QKV_CASES = [(2, 8, 16, 16, 64, 16), (1, 4, 8, 8, 32, 8), (3, 2, 8, 8, 64, 12), (2, 1, 16, 8, 48, 8),
             (2, 3, 8, 8, 64, 16), (1, 16, 8, 8, 32, 8), (2, 1, 8, 8, 64, 8), (1, 32, 8, 8, 64, 8),
             (2, 24, 4, 4, 32, 8), (1, 4, 4, 8, 32, 8), (1, 8, 4, 4, 32, 8), (2, 3, 4, 4, 32, 8)]


@pytest.mark.parametrize("shape", QKV_CASES)
@pytest.mark.parametrize("kt,gate_mode", [(4, 1), (0, 1), (3, 2), (4, 3), (2, 0), (6, 1)])
def test_gdn_qkv_proj_matches_two_step(mods, shape, kt, gate_mode):
    """The fused qkv projection equals proj_planes followed by qkv_post (fp32: bit for bit), and the oracle."""
    _, S = mods
    B, T, H, W, K, C = shape
    print_case(test="gdn_qkv_proj", shape=shape, kt=kt, gate_mode=gate_mode,
               fused=S.gdn_qkv_fused(T, H, W, K, kt))
    rng = np.random.default_rng(9)
    x = rng.standard_normal((B, T, H, W, K))
    Wt = rng.standard_normal((K, 3 * C)) / np.sqrt(K)
    b = rng.standard_normal(3 * C) * 0.1
    convs = [{"kernel": rng.standard_normal((kt, 1, C)) / 2, "bias": rng.standard_normal(C) * 0.1}
             for _ in range(3)] if kt else None
    gates = None
    if gate_mode == 1:
        gates = 1.0 / (1.0 + np.exp(-rng.standard_normal((B, T, H * W, 2))))
    elif gate_mode == 2:
        gates = 1.0 / (1.0 + np.exp(-rng.standard_normal((B, T, 2))))
    elif gate_mode == 3:
        gates = 1.0 / (1.0 + np.exp(-rng.standard_normal((B, T, 2 * C, H, W))))
    dc = [_tree(c) for c in convs] if convs else None
    dg = _dev(gates) if gates is not None else None
    got = S.gdn_qkv_proj(_dev(x), _dev(Wt), _dev(b), B, T, H, W, dc, gate_mode, dg, out_dtype=torch.float32)
    two = S.proj_planes(_dev(x), _dev(Wt), _dev(b), B * T, H * W, out_dtype=torch.float32).view(B, T, 3 * C, H, W)
    S.gdn_qkv_post(two, dc, gate_mode, dg)
    assert torch.equal(got, two)
    # oracle: x @ W + b, causal conv over T + SiLU per block, gates on k and v
    def oracle(xx):
        cl = (xx.reshape(-1, K) @ Wt + b).reshape(B, T, H, W, 3, C)
        outs = []
        for i in range(3):
            z = cl[..., i, :]
            if convs:
                z = O.silu(O.causal_conv_t(z, convs[i]))
            if i > 0 and gate_mode == 1:
                z = z * gates[..., i - 1].reshape(B, T, H, W, 1)
            elif i > 0 and gate_mode == 2:
                z = z * gates[..., i - 1].reshape(B, T, 1, 1, 1)
            elif i > 0 and gate_mode == 3:
                z = z * gates[:, :, (i - 1) * C:i * C].transpose(0, 1, 3, 4, 2)
            outs.append(z)
        return np.stack(outs, axis=4).transpose(0, 1, 4, 5, 2, 3).reshape(B, T, 3 * C, H, W)
    assert rel_err(to_np(got), oracle(x)) < 1e-5
    # bf16 in / bf16 out against the oracle of the bf16-rounded input: the fused path keeps the
    # projection in fp32 before the conv, so only the final store rounds; the two-step path stores the
    # projection in bf16 first (a second rounding, inside the conv)
    xb = _dev(x, torch.bfloat16)
    gb = S.gdn_qkv_proj(xb, _dev(Wt), _dev(b), B, T, H, W, dc, gate_mode, dg, out_dtype=torch.bfloat16)
    bar = 5e-3 if S.gdn_qkv_fused(T, H, W, K, kt) else 4e-2
    assert bf16_excess_err(to_np(gb.float()), oracle(to_np(xb.float()))) < bar


@pytest.mark.parametrize("shape", [(2, 8, 16, 16, 64, 16), (1, 4, 8, 8, 32, 8), (2, 1, 16, 8, 48, 8),
                                   (2, 3, 8, 8, 64, 16), (1, 32, 8, 8, 64, 8), (2, 2, 8, 8, 64, 40),
                                   (1, 16, 8, 8, 64, 64)])
@pytest.mark.parametrize("kt,gate_mode,gact", [(4, 1, "silu"), (0, 0, "sigmoid"), (3, 3, "silu"), (6, 2, "silu")])
def test_gdn_qkv_gate_proj_matches_separate_calls(mods, shape, kt, gate_mode, gact):
    """qkv and gate_proj in one call equal gdn_qkv_proj and proj_planes(act) on the same x (qkv bit for bit,
    the gate columns to fp32 rounding) and the oracle act(x Wg + bg), fused (gate columns in the qkv
    launch) and not (T = 3, kt = 6: a second projection); bf16 in / out against the oracle."""
    _, S = mods
    B, T, H, W, K, C = shape
    fused = S.gdn_qkv_fused(T, H, W, K, kt)
    print_case(test="gdn_qkv_gate_proj", shape=shape, kt=kt, gate_mode=gate_mode, gact=gact, fused=fused)
    rng = np.random.default_rng(21)
    x = rng.standard_normal((B, T, H, W, K))
    Wt = rng.standard_normal((K, 3 * C)) / np.sqrt(K)
    b = rng.standard_normal(3 * C) * 0.1
    Wg = rng.standard_normal((K, C)) / np.sqrt(K)
    bg = rng.standard_normal(C) * 0.1
    convs = [{"kernel": rng.standard_normal((kt, 1, C)) / 2, "bias": rng.standard_normal(C) * 0.1}
             for _ in range(3)] if kt else None
    gates = None
    if gate_mode == 1:
        gates = 1.0 / (1.0 + np.exp(-rng.standard_normal((B, T, H * W, 2))))
    elif gate_mode == 2:
        gates = 1.0 / (1.0 + np.exp(-rng.standard_normal((B, T, 2))))
    elif gate_mode == 3:
        gates = 1.0 / (1.0 + np.exp(-rng.standard_normal((B, T, 2 * C, H, W))))
    dc = [_tree(c) for c in convs] if convs else None
    dg = _dev(gates) if gates is not None else None
    qkv, gv = S.gdn_qkv_gate_proj(_dev(x), _dev(Wt), _dev(b), B, T, H, W, dc, gate_mode, dg, _dev(Wg), _dev(bg),
                                  gact, out_dtype=torch.float32)
    assert tuple(gv.shape) == (B, T, C, H, W)
    ref_qkv = S.gdn_qkv_proj(_dev(x), _dev(Wt), _dev(b), B, T, H, W, dc, gate_mode, dg, out_dtype=torch.float32)
    assert torch.equal(qkv, ref_qkv)
    ref_gv = S.proj_planes(_dev(x), _dev(Wg), _dev(bg), B * T, H * W, act=gact, out_dtype=torch.float32)
    assert rel_err(to_np(gv).reshape(B * T, C, H * W), to_np(ref_gv)) < 1e-6

    def oracle_gv(xx):
        z = xx.reshape(-1, K) @ Wg + bg
        z = O.silu(z) if gact == "silu" else 1.0 / (1.0 + np.exp(-z))
        return z.reshape(B, T, H, W, C).transpose(0, 1, 4, 2, 3)
    assert rel_err(to_np(gv), oracle_gv(x)) < 1e-5
    xb = _dev(x, torch.bfloat16)
    qb, gb = S.gdn_qkv_gate_proj(xb, _dev(Wt), _dev(b), B, T, H, W, dc, gate_mode, dg, _dev(Wg), _dev(bg), gact,
                                 out_dtype=torch.bfloat16)
    assert torch.equal(qb, S.gdn_qkv_proj(xb, _dev(Wt), _dev(b), B, T, H, W, dc, gate_mode, dg,
                                          out_dtype=torch.bfloat16))
    assert bf16_excess_err(to_np(gb.float()), oracle_gv(to_np(xb.float()))) < 5e-3


@pytest.mark.parametrize("shape,ks,dt", [((1, 2, 32, 32, 64), 5, torch.float32), ((2, 1, 32, 32, 32), 3, torch.float32),
                                         ((1, 3, 32, 16, 64), 7, torch.bfloat16), ((1, 1, 128, 128, 64), 5, torch.float32)])
def test_depthwise_conv_mean_matches_separate_calls(mods, shape, ks, dt):
    """The conv with the frame mean fused in: its conv output equals depthwise_conv bit for bit, its
    mean frame_mean's to rounding and numpy's.  The two fp32 means add H*W terms in different orders
    (up to 16384 here), so they agree to ~1e-6 of the means, not bit for bit: the inputs carry a mean
    of 0.5 so the comparison is not dominated by cancellation, and the bar is 1e-5."""
    _, S = mods
    print_case(test="dwconv_mean", shape=shape, ks=ks, dtype=str(dt))
    rng = np.random.default_rng(31)
    C = shape[-1]
    x = _dev(rng.standard_normal(shape) + 0.5, dt)
    kw = _dev(rng.standard_normal((ks, ks, 1, C)) / ks)
    b = _dev(rng.standard_normal(C) * 0.1)
    r = S.depthwise_conv_mean(x, kw, b, out_dtype=torch.float32)
    assert r is not None
    y, ctx = r
    assert torch.equal(y, S.depthwise_conv(x, kw, b, out_dtype=torch.float32))
    ref = S.frame_mean(x)
    assert ctx.shape == ref.shape
    assert rel_err(to_np(ctx), to_np(ref)) < 1e-5
    xn = to_np(x.float()).astype(np.float64)
    assert rel_err(to_np(ctx), xn.mean(axis=(2, 3))) < 1e-5


FULL_CONV_CASES = [(3, (4, 16, 16, 8), 24), (4, (3, 14, 14, 6), 18), (5, (2, 8, 8, 16), 48), (1, (2, 8, 8, 4), 12)]


@pytest.mark.parametrize("ks,shape,N", FULL_CONV_CASES,
                         ids=[f"k{c[0]}_{c[1][1]}x{c[1][2]}_C{c[1][3]}_N{c[2]}" for c in FULL_CONV_CASES])
def test_full_conv_planes_matches_oracle(mods, ks, shape, N):
    """The full-channel SAME conv (im2col rows through the projection GEMM) against the oracle's
    direct sum over taps, f32 and bf16 in, in one chunk of frames and in chunks of one frame."""
    _, S = mods
    print_case(test="full_conv_planes", ks=ks, shape=shape, N=N)
    rng = np.random.default_rng(8)
    F, H, W, C = shape
    x = rng.standard_normal(shape)
    p = {"kernel": rng.standard_normal((ks, ks, C, N)) / (ks * np.sqrt(C)), "bias": rng.standard_normal(N)}
    for xd in (_dev(x), _dev(x, torch.bfloat16)):
        ref = O.full_conv2d_same(to_np(xd).reshape(shape), p).reshape(F, H * W, N).transpose(0, 2, 1)
        for mb in (1 << 29, H * W * ks * ks * C * 4):
            y = S.conv_full_planes(xd, _dev(p["kernel"]), _dev(p["bias"]), max_bytes=mb)
            assert tuple(y.shape) == (F, N, H * W)
            assert rel_err(to_np(y), ref) < 5e-6, (xd.dtype, mb)


def test_depthwise_conv_mean_unsupported_shape(mods):
    """Where the blocked conv would leave a partial block the fused form declines (None): the cell
    then runs the conv and frame_mean."""
    _, S = mods
    x = _dev(np.zeros((1, 1, 16, 16, 64)))
    assert S.depthwise_conv_mean(x, _dev(np.zeros((5, 5, 1, 64))), _dev(np.zeros(64))) is None


# --------------------------------------------------------- spectral core

CORE_CASES = [
    # name, (B, T, H, W, C), d_k, gate_type, spectral l2 norm
    ("factored_dk4_32", (2, 6, 32, 32, 16), 4, "factored", True),
    ("channel_dk2_16", (2, 5, 16, 16, 8), 2, "channel", True),
    ("dense_dk3_16", (1, 4, 16, 16, 12), 3, "dense", False),
    ("scalar_dk1_8", (2, 3, 8, 8, 4), 1, "scalar", True),
    ("factored_dk4_128", (1, 3, 128, 128, 8), 4, "factored", True),
]


@pytest.mark.parametrize("name,shape,dk,gate_type,l2", CORE_CASES, ids=[c[0] for c in CORE_CASES])
def test_gdn_spectral_core_matches_oracle(mods, name, shape, dk, gate_type, l2):
    """rfft2 -> gdn_scan_bins -> irfft2 against the oracle's materialised-M GOOM scan."""
    _, S = mods
    print_case(test="gdn_core", case=name)
    rng = np.random.default_rng(11)
    B, T, H, W, C = shape
    nh, Wf = C // dk, W // 2 + 1
    cfg = O.GDNConfig(channels=C, delta_key_dim=dk, gate_type=gate_type, use_spectral_l2_norm=l2)
    q, k, v = (rng.standard_normal(shape) for _ in range(3))
    n_ab = {"factored": H * Wf, "dense": H * Wf, "channel": nh, "scalar": 1}[gate_type]
    alpha = 0.1 + 0.89 / (1.0 + np.exp(-rng.standard_normal((B, T, n_ab))))
    beta = 1.0 / (1.0 + np.exp(-rng.standard_normal((B, T, n_ab))))
    kern = rng.standard_normal((nh, 11, 11)) * 0.2
    what = O.spectral_kernel(kern, H, W, 0.999)
    shp = (B, T, nh, 1, 1) if gate_type == "channel" else ((B, T, 1, 1, 1) if gate_type == "scalar"
                                                           else (B, T, 1, H, Wf))
    ref = O.gdn_core(q, k, v, alpha.reshape(shp), beta.reshape(shp), what, cfg, scan="linear")
    planes = np.concatenate([z.transpose(0, 1, 4, 2, 3) for z in (q, k, v)], axis=2)     # (B, T, 3C, H, W)
    spec, norms = S.rfft2(_dev(planes), want_norms=l2)
    ab = _dev(np.stack([alpha, beta], axis=-1))
    ohat = S.gdn_scan_bins(spec, norms, ab, gate_type, _dev(what, torch.complex64), dk)
    o = S.irfft2(ohat, W)
    assert rel_err(to_np(o), ref) <= TOL_F32


FUSED_CASES = [
    # name, (B, T, H, W, C), gate_type, spectral l2 norm   (the fused core: 32 x 32, d_k = 4)
    ("factored_l2", (2, 7, 32, 32, 16), "factored", True),
    ("dense_no_l2", (1, 4, 32, 32, 8), "dense", False),
    ("channel_l2", (2, 3, 32, 32, 12), "channel", True),
    ("scalar_l2_T1", (3, 1, 32, 32, 8), "scalar", True),
    ("c4_heads_T32", (1, 32, 32, 32, 64), "factored", True),
]


# the reference's flags for each scan variant (cssm.py:4939-4991)
VARIANT_FLAGS = {"goom": dict(), "linear": dict(use_log=False), "log_eps": dict(use_goom=False)}


@pytest.mark.parametrize("variant", ["goom", "linear", "log_eps"])
@pytest.mark.parametrize("H", [32, 16])
def test_gdn_core_floored_heads(mods, H, variant):
    """Heads whose keys or values vanish put exact zeros into M and Delta, where the scan
    variants differ: to_goom's floor makes them 1e-7 (the materialised-M path), the log-eps map
    1e-8 (every entry moved), the linear scan leaves them 0 (rank-1 form throughout).  Checked per
    head against the oracle, so a head's small output is not hidden by the others' RMS.  Head 0:
    k = 0 (every off-diagonal M entry and all of Delta zero); head 1: k with one nonzero
    component; head 2: v = 0 (Delta zero); head 3: unconstrained.  A head whose reference is
    exactly zero (heads 0 and 2 of the linear scan) must come out exactly zero.  H = 32 runs the
    fused core, H = 16 the three-kernel core."""
    _, S = mods
    print_case(test="gdn_core_floored_heads", H=H, variant=variant)
    rng = np.random.default_rng(31)
    B, T, W, C, dk = 1, 4, H, 16, 4
    shape = (B, T, H, W, C)
    nh, Wf = C // dk, W // 2 + 1
    cfg = O.GDNConfig(channels=C, delta_key_dim=dk, gate_type="factored", use_spectral_l2_norm=True,
                      **VARIANT_FLAGS[variant])
    assert O.gdn_scan_variant(cfg) == variant == S.gdn_scan_variant(cfg.use_log, cfg.use_goom, cfg.scan_mode, dk)
    q, k, v = (rng.standard_normal(shape) for _ in range(3))
    k[..., 0:4] = 0.0
    k[..., 5:8] = 0.0
    v[..., 8:12] = 0.0
    alpha = 0.1 + 0.89 / (1.0 + np.exp(-rng.standard_normal((B, T, H * Wf))))
    beta = 1.0 / (1.0 + np.exp(-rng.standard_normal((B, T, H * Wf))))
    what = O.spectral_kernel(rng.standard_normal((nh, 11, 11)) * 0.2, H, W, 0.999)
    shp = (B, T, 1, H, Wf)
    ref = O.gdn_core(q, k, v, alpha.reshape(shp), beta.reshape(shp), what, cfg, scan="linear")
    planes = _dev(np.concatenate([z.transpose(0, 1, 4, 2, 3) for z in (q, k, v)], axis=2))
    ab = _dev(np.stack([alpha, beta], axis=-1))
    wd = _dev(what, torch.complex64)
    if S.gdn_core_fused_supported(H, W, dk):
        o = S.gdn_core_fused(planes, True, ab, "factored", wd, dk, variant)
    else:
        spec, norms = S.rfft2(planes, want_norms=True)
        o = S.irfft2(S.gdn_scan_bins(spec, norms, ab, "factored", wd, dk, variant), W)
    torch.cuda.synchronize()
    got, refp = to_np(o), ref                                 # (B, T, C, H, W)
    zero_heads = {0, 2} if variant == "linear" else set()
    for h in range(nh):
        sl = slice(h * dk, (h + 1) * dk)
        if h in zero_heads:
            assert np.all(refp[:, :, sl] == 0) and np.all(got[:, :, sl] == 0), h
            continue
        assert np.sqrt(np.mean(refp[:, :, sl] ** 2)) > 0, h
        assert rel_err(got[:, :, sl], refp[:, :, sl]) <= TOL_F32, h


@pytest.mark.parametrize("name,shape,gate_type,l2", FUSED_CASES, ids=[c[0] for c in FUSED_CASES])
def test_gdn_core_fused_matches_oracle_and_three_kernels(mods, name, shape, gate_type, l2):
    """The one-kernel core (per (b, head), state in VGPRs over T) against the oracle's
    materialised-M GOOM scan at the fp32 bar, and against rfft2 -> gdn_scan_bins -> irfft2
    (the same FFT passes; only the per-plane norm sums add in another order)."""
    _, S = mods
    print_case(test="gdn_core_fused", case=name)
    rng = np.random.default_rng(12)
    B, T, H, W, C = shape
    dk = 4
    assert S.gdn_core_fused_supported(H, W, dk)
    nh, Wf = C // dk, W // 2 + 1
    cfg = O.GDNConfig(channels=C, delta_key_dim=dk, gate_type=gate_type, use_spectral_l2_norm=l2)
    q, k, v = (rng.standard_normal(shape) for _ in range(3))
    n_ab = {"factored": H * Wf, "dense": H * Wf, "channel": nh, "scalar": 1}[gate_type]
    alpha = 0.1 + 0.89 / (1.0 + np.exp(-rng.standard_normal((B, T, n_ab))))
    beta = 1.0 / (1.0 + np.exp(-rng.standard_normal((B, T, n_ab))))
    what = O.spectral_kernel(rng.standard_normal((nh, 11, 11)) * 0.2, H, W, 0.999)
    shp = (B, T, nh, 1, 1) if gate_type == "channel" else ((B, T, 1, 1, 1) if gate_type == "scalar"
                                                           else (B, T, 1, H, Wf))
    ref = O.gdn_core(q, k, v, alpha.reshape(shp), beta.reshape(shp), what, cfg, scan="linear")
    planes = _dev(np.concatenate([z.transpose(0, 1, 4, 2, 3) for z in (q, k, v)], axis=2))
    ab = _dev(np.stack([alpha, beta], axis=-1))
    wd = _dev(what, torch.complex64)
    o = S.gdn_core_fused(planes, l2, ab, gate_type, wd, dk)
    spec, norms = S.rfft2(planes, want_norms=l2)
    o3 = S.irfft2(S.gdn_scan_bins(spec, norms, ab, gate_type, wd, dk), W)
    torch.cuda.synchronize()
    assert rel_err(to_np(o), ref) <= TOL_F32
    assert rel_err(to_np(o), to_np(o3)) <= 1e-5
    # deterministic: the norm sums add in a fixed order
    assert torch.equal(o, S.gdn_core_fused(planes, l2, ab, gate_type, wd, dk))


def test_gdn_proj_out_norm_gate(mods):
    _, S = mods
    print_case(test="gdn_proj_out")
    rng = np.random.default_rng(12)
    F, C, HW, N = 3, 64, 1024, 64
    o = rng.standard_normal((F, C, HW))
    g = rng.standard_normal((F, C, HW))
    Wt = rng.standard_normal((C, N)) / 8
    b = rng.standard_normal(N) * 0.1
    sc = 1.0 + 0.1 * rng.standard_normal(C)
    sh = 0.1 * rng.standard_normal(C)
    ocl = o.transpose(0, 2, 1)
    gcl = g.transpose(0, 2, 1)
    for norm, ref_n in (("rms", O.rms_norm(ocl, sc)), ("layer", O.layer_norm(ocl, sc, sh)), ("none", ocl)):
        out = S.gdn_proj_out(_dev(o), _dev(g), norm, _dev(sc) if norm != "none" else None,
                             _dev(sh) if norm == "layer" else None, _dev(Wt), _dev(b))
        ref = (ref_n * gcl).reshape(F * HW, C) @ Wt + b
        assert rel_err(to_np(out), ref) < 1e-5, norm


XGATE_CASES = [
    # F, HW, K, N, norm, gate act, o dtype, out dtype, x dtype: the C4 widths, narrower ones, a partial
    # last row tile (F HW not a multiple of 128), LayerNorm and no norm, sigmoid, bf16 o and f32 out;
    # fp32 x (the C3 widths among them), whose fragments come straight from its rows
    (3, 1024, 64, 64, "rms", "silu", torch.float32, torch.bfloat16, torch.bfloat16),
    (5, 196, 64, 64, "layer", "sigmoid", torch.float32, torch.float32, torch.bfloat16),
    (2, 1024, 32, 48, "none", "silu", torch.bfloat16, torch.float32, torch.bfloat16),
    (7, 16, 16, 16, "rms", "sigmoid", torch.float32, torch.float32, torch.bfloat16),
    (3, 64, 40, 40, "layer", "silu", torch.bfloat16, torch.bfloat16, torch.bfloat16),
    (2, 16384, 64, 64, "rms", "silu", torch.float32, torch.float32, torch.float32),
    (5, 196, 64, 64, "layer", "sigmoid", torch.float32, torch.float32, torch.float32),
    (3, 64, 40, 40, "none", "silu", torch.float32, torch.bfloat16, torch.float32),
    (7, 16, 16, 16, "rms", "sigmoid", torch.bfloat16, torch.float32, torch.float32),
]


@pytest.mark.parametrize("F,HW,K,N,norm,gact,odt,outdt,xdt", XGATE_CASES,
                         ids=[f"F{c[0]}_HW{c[1]}_K{c[2]}_N{c[3]}_{c[4]}_{c[5]}_x{str(c[8])[6:]}" for c in XGATE_CASES])
def test_gdn_proj_out_xgate_matches_gate_planes(mods, F, HW, K, N, norm, gact, odt, outdt, xdt):
    """The output projection computing gate_proj from the layer input against the float64 reference
    of norm(o) * act(x Wg + bg) then output_proj, and against the two-call path (the gate planes from a
    projection, then cssm_gdn_proj_out)."""
    _, S = mods
    print_case(test="gdn_proj_out_xgate", F=F, HW=HW, K=K, N=N, norm=norm, gact=gact, x=xdt)
    rng = np.random.default_rng(31)
    o = _dev(rng.standard_normal((F, K, HW)), odt)
    xb = _dev(rng.standard_normal((F * HW, K)), xdt)
    Wg = rng.standard_normal((K, K)) / np.sqrt(K)
    bg = rng.standard_normal(K) * 0.1
    Wt = rng.standard_normal((K, N)) / np.sqrt(K)
    b = rng.standard_normal(N) * 0.1
    sc = 1.0 + 0.1 * rng.standard_normal(K)
    sh = 0.1 * rng.standard_normal(K)
    ns = _dev(sc) if norm != "none" else None
    nb = _dev(sh) if norm == "layer" else None
    out = S.gdn_proj_out_xgate(o, xb, norm, ns, nb, _dev(Wg), _dev(bg), gact, _dev(Wt), _dev(b), out_dtype=outdt)
    assert out.dtype == outdt and tuple(out.shape) == (F * HW, N)
    ocl = to_np(o).transpose(0, 2, 1)
    ref_n = {"rms": lambda: O.rms_norm(ocl, sc), "layer": lambda: O.layer_norm(ocl, sc, sh), "none": lambda: ocl}[norm]()
    z = to_np(xb).reshape(F, HW, K) @ Wg + bg
    g = z / (1.0 + np.exp(-z)) if gact == "silu" else 1.0 / (1.0 + np.exp(-z))
    ref = (ref_n * g).reshape(F * HW, K) @ Wt + b
    if outdt == torch.bfloat16:
        assert bf16_excess_err(to_np(out), ref) < 2e-5
    else:
        assert rel_err(to_np(out), ref) < 1e-5
    gv = S.proj_planes(xb, _dev(Wg), _dev(bg), F, HW, act=gact, out_dtype=odt)
    two = S.gdn_proj_out(o, gv, norm, ns, nb, _dev(Wt), _dev(b), out_dtype=torch.float32)
    if odt == torch.float32:   # with bf16 o the two-call path rounds the gate planes to bf16 as well
        if outdt == torch.bfloat16:
            assert bf16_excess_err(to_np(out), to_np(two)) < 2e-5
        else:
            assert rel_err(to_np(out), to_np(two)) < 1e-5


# ------------------------------------------------------------------- layer

LAYER_CASES = [
    # name, (B, T, H, W, C), cfg kwargs
    ("c3_shape_small", (1, 3, 128, 128, 8),
     dict(delta_key_dim=4, gate_type="factored", qkv_conv_size=5, kernel_size=11)),
    ("c4_shape_small", (2, 8, 32, 32, 16),
     dict(delta_key_dim=4, gate_type="factored", kernel_size=11)),
    ("channel_dk2_layer_norm", (2, 4, 16, 16, 8),
     dict(delta_key_dim=2, gate_type="channel", output_norm="layer", output_gate_act="sigmoid")),
    ("dense_dk3_no_input_gates", (1, 5, 16, 16, 12),
     dict(delta_key_dim=3, gate_type="dense", use_input_gates=False, short_conv_size=0, qkv_conv_size=3)),
    ("scalar_no_norm_no_l2", (2, 3, 8, 8, 8),
     dict(delta_key_dim=2, gate_type="scalar", output_norm="none", use_spectral_l2_norm=False,
          no_spectral_clamp=True, position_independent_gates=True)),
    # CSSM-SHViT stage planes (not powers of two)
    ("shvit_14_factored_qkvdw", (2, 3, 14, 14, 16),
     dict(delta_key_dim=4, gate_type="factored", qkv_conv_size=3, kernel_size=5)),
    ("shvit_7_channel", (3, 2, 7, 7, 8), dict(delta_key_dim=2, gate_type="channel", kernel_size=3)),
    ("small_12_dense_T1", (2, 1, 12, 12, 8), dict(delta_key_dim=4, gate_type="dense", kernel_size=5)),
    # the k x k full-channel qkv conv (qkv_conv_separable=False): the fused 32 x 32 core, an even tap
    # count on 14 x 14 planes with d_k = 3, channel input gates
    ("full_qkv_conv3_fused32", (1, 3, 32, 32, 16),
     dict(delta_key_dim=4, gate_type="factored", qkv_conv_size=3, qkv_conv_separable=False)),
    ("full_qkv_conv4_14_dk3", (2, 3, 14, 14, 12),
     dict(delta_key_dim=3, gate_type="factored", qkv_conv_size=4, qkv_conv_separable=False, kernel_size=3)),
    ("full_qkv_conv5_channel_16", (2, 2, 16, 16, 8),
     dict(delta_key_dim=2, gate_type="channel", qkv_conv_size=5, qkv_conv_separable=False, kernel_size=5)),
]


def _layer(kw, shape, seed):
    rng = np.random.default_rng(seed)
    B, T, H, W, C = shape
    okw = {k: v for k, v in kw.items() if k != "position_independent_gates"}
    cfg = O.GDNConfig(channels=C, **okw)
    p = O.init_params(O.gdn_param_shapes(cfg, H, W), rng, spectral_init="xavier")
    x = rng.standard_normal(shape)
    return cfg, p, x


@pytest.mark.parametrize("name,shape,kw", LAYER_CASES, ids=[c[0] for c in LAYER_CASES])
def test_gdn_layer_matches_oracle(mods, name, shape, kw):
    cells, _ = mods
    print_case(test="gdn_layer", case=name)
    cfg, p, x = _layer(kw, shape, 21)
    if kw.get("position_independent_gates"):
        # no temporal encoding of ctx: compare against the oracle with the table cancelled
        T, C = shape[1], shape[4]
        enc = O.temporal_context_encoding(T, C)
        orig = O.temporal_context_encoding
        O.temporal_context_encoding = lambda T_, C_, base=10000.0: np.zeros((T_, C_))
        try:
            ref = O.gdn_forward(p, x, cfg)
        finally:
            O.temporal_context_encoding = orig
        assert enc.shape == (T, C)
    else:
        ref = O.gdn_forward(p, x, cfg)
    cell = cells.GatedDeltaNetCSSM(channels=shape[4], **kw)
    y = cell.apply(cells.GatedDeltaNetCSSM.load_params(p), _dev(x))
    torch.cuda.synchronize()
    assert tuple(y.shape) == shape
    assert rel_err(to_np(y), ref) <= TOL_F32


ZERO_FRAME_CASES = [
    # name, (B, T, H, W, C), cfg kwargs: the fused 32 x 32 core, the three-kernel core, a small plane
    ("fused32", (2, 6, 32, 32, 16), dict(delta_key_dim=4, gate_type="factored", kernel_size=11)),
    ("planes16_dk2", (2, 5, 16, 16, 8), dict(delta_key_dim=2, gate_type="channel", kernel_size=5)),
    ("small14", (1, 4, 14, 14, 8), dict(delta_key_dim=4, gate_type="dense", kernel_size=5, short_conv_size=0)),
]


@pytest.mark.parametrize("variant", ["goom", "linear", "log_eps", "pallas_d2"])
@pytest.mark.parametrize("name,shape,kw", ZERO_FRAME_CASES, ids=[c[0] for c in ZERO_FRAME_CASES])
def test_gdn_layer_zero_masked_frames_per_scan_variant(mods, name, shape, kw, variant):
    """The layer under each of the reference's scan flags (use_log=False, use_goom=False,
    scan_mode='pallas') with its first frames zeroed as --variable_seq_len does
    (main.py:1429-1438): those frames' q / k / v planes are constant (bias only), so every
    non-DC bin of their spectra is zero up to the transform's rounding, the entries the scan
    variants map differently.  Against the oracle under the same flags."""
    cells, _ = mods
    flags = dict(VARIANT_FLAGS.get(variant, {}))
    kw = dict(kw)
    if variant == "pallas_d2":
        flags = dict(scan_mode="pallas")     # the linear 2 x 2 scan at d_k = 2, ignored otherwise
    kw.update(flags)
    print_case(test="gdn_layer_zero_frames", case=name, variant=variant)
    cfg, p, x = _layer(kw, shape, 27)
    x[:, :2] = 0.0
    cell = cells.GatedDeltaNetCSSM(channels=shape[4], **kw)
    expect = ("linear" if kw["delta_key_dim"] == 2 else "goom") if variant == "pallas_d2" else variant
    assert cell.scan_variant == O.gdn_scan_variant(cfg) == expect
    ref = O.gdn_forward(p, x, cfg)
    y = cell.apply(cells.GatedDeltaNetCSSM.load_params(p), _dev(x))
    torch.cuda.synchronize()
    assert rel_err(to_np(y), ref) <= TOL_F32
    # the masked frames alone, against their own RMS
    assert rel_err(to_np(y[:, :2]), ref[:, :2]) <= TOL_F32


def test_gdn_layer_bf16_io(mods):
    """C4-shaped (video, 32x32, d_k = 4) with bf16 I/O: sparse dots + N(0, 0.01) background."""
    cells, _ = mods
    print_case(test="gdn_layer_bf16")
    kw = dict(delta_key_dim=4, gate_type="factored", kernel_size=11)
    shape = (2, 8, 32, 32, 16)
    cfg, p, _ = _layer(kw, shape, 22)
    rng = np.random.default_rng(23)
    x = rng.standard_normal(shape) * 0.01
    x[rng.random(shape[:4]) < 0.02] = 1.0
    xb = _dev(x, torch.bfloat16)
    y = cells.GatedDeltaNetCSSM(channels=16, **kw).apply(cells.GatedDeltaNetCSSM.load_params(p), xb)
    assert y.dtype == torch.bfloat16
    ref = O.gdn_forward(p, to_np(xb), cfg)
    assert np.sqrt(np.mean((to_np(y) - ref) ** 2)) <= TOL_BF16 * np.sqrt(np.mean(ref ** 2))
    assert bf16_excess_err(to_np(y), ref) <= TOL_BF16


def test_gdn_layer_c3_time_length_fused_qkv_128(mods):
    """C3's own frame count (T = 8) at 128 x 128 with the 5 x 5 qkv depthwise conv: the fused
    T = 8 qkv projection (short conv + SiLU + input gates in the GEMM epilogue) runs in the layer."""
    cells, S = mods
    print_case(test="gdn_layer_c3_T8_128")
    kw = dict(delta_key_dim=4, gate_type="factored", qkv_conv_size=5, kernel_size=11)
    shape = (1, 8, 128, 128, 8)
    assert S.gdn_qkv_fused(8, 128, 128, 8, 4)
    cfg, p, x = _layer(kw, shape, 26)
    ref = O.gdn_forward(p, x, cfg)
    y = cells.GatedDeltaNetCSSM(channels=8, **kw).apply(cells.GatedDeltaNetCSSM.load_params(p), _dev(x))
    assert rel_err(to_np(y), ref) <= TOL_F32


def _moving_dots(rng, shape):
    """~2 % of pixels = 1.0 on random-walk tracks over N(0, 0.01^2) background (the C4 input)."""
    B, T, H, W, C = shape
    x = rng.standard_normal(shape) * 0.01
    pos = rng.integers(0, H * W, (B, max(1, int(0.02 * H * W))))
    steps = np.array([1, -1, W, -W, 0])
    for t in range(T):
        for b in range(B):
            x[b, t].reshape(H * W, C)[pos[b]] = 1.0
        pos = (pos + steps[rng.integers(0, 5, pos.shape)]) % (H * W)
    return x


def test_gdn_layer_c4_shape_bf16_chunk_carry(mods):
    """C4's frame shape at full width (T = 32, 32 x 32, C = 64, d_k = 4, bf16 I/O) on moving dots:
    the frame-sequential qkv projection walks the 32 frames carrying the short conv's three
    previous frames in registers, with gate_proj's columns in the same launch, inside the layer."""
    cells, S = mods
    print_case(test="gdn_layer_c4_T32_bf16")
    kw = dict(delta_key_dim=4, gate_type="factored", kernel_size=11, short_conv_size=4)
    shape = (1, 32, 32, 32, 64)
    assert S.gdn_qkv_fused(32, 32, 32, 64, 4)
    cfg, p, _ = _layer(kw, shape, 27)
    x = _moving_dots(np.random.default_rng(28), shape)
    xb = _dev(x, torch.bfloat16)
    y = cells.GatedDeltaNetCSSM(channels=64, **kw).apply(cells.GatedDeltaNetCSSM.load_params(p), xb)
    assert y.dtype == torch.bfloat16
    ref = O.gdn_forward(p, to_np(xb), cfg)
    assert bf16_excess_err(to_np(y), ref) <= TOL_BF16
    # the same layer in fp32 I/O holds the fp32 bar (the carry is exact)
    y32 = cells.GatedDeltaNetCSSM(channels=64, **kw).apply(cells.GatedDeltaNetCSSM.load_params(p),
                                                           _dev(to_np(xb)))
    assert rel_err(to_np(y32), ref) <= TOL_F32


def test_gdn_layer_two_parameter_trees(mods):
    """One cell applied to two parameter trees of the same shape in turn: each output follows its
    own weights (the derived W_hat and input-gate buffers are not reused across trees)."""
    cells, _ = mods
    print_case(test="gdn_layer_two_trees")
    for gate_type in ("factored", "channel"):
        kw = dict(delta_key_dim=2, gate_type=gate_type)
        shape = (1, 3, 16, 16, 8)
        cell = cells.GatedDeltaNetCSSM(channels=8, **kw)
        for seed in (31, 32, 31):
            cfg, p, x = _layer(kw, shape, seed)
            v = cells.GatedDeltaNetCSSM.load_params(p)
            y = cell.apply(v, _dev(x))
            del v
            assert rel_err(to_np(y), O.gdn_forward(p, x, cfg)) <= TOL_F32, (gate_type, seed)


def test_gdn_layer_is_causal_in_time(mods):
    cells, _ = mods
    print_case(test="gdn_layer_causal")
    kw = dict(delta_key_dim=2, gate_type="factored")
    cfg, p, x = _layer(kw, (1, 6, 16, 16, 8), 24)
    cell = cells.GatedDeltaNetCSSM(channels=8, **kw)
    v = cells.GatedDeltaNetCSSM.load_params(p)
    y1 = to_np(cell.apply(v, _dev(x)))
    x2 = x.copy()
    x2[:, 4:] += 1.0
    y2 = to_np(cell.apply(v, _dev(x2)))
    assert np.array_equal(y1[:, :4], y2[:, :4])
    assert not np.allclose(y1[:, 4:], y2[:, 4:])


def test_gdn_layer_rejects_unsupported(mods):
    cells, _ = mods
    with pytest.raises(NotImplementedError):
        cells.GatedDeltaNetCSSM(channels=8, rope_mode="spatial")
    with pytest.raises(NotImplementedError):
        cells.GatedDeltaNetCSSM(channels=8, int_attention_mode="spectral")
    cell = cells.GatedDeltaNetCSSM(channels=8, delta_key_dim=2)
    v = cell.init(0, (1, 2, 20, 20, 8))                   # neither a power of two nor <= 15
    with pytest.raises(NotImplementedError):
        cell.apply(v, torch.zeros((1, 2, 20, 20, 8), device="cuda"))


def test_gdn_layer_is_deterministic(mods):
    """Two calls on the same input give bit-identical outputs (no order-dependent reductions)."""
    cells, _ = mods
    print_case(test="gdn_layer_deterministic")
    kw = dict(delta_key_dim=4, gate_type="factored", qkv_conv_size=5)
    cfg, p, x = _layer(kw, (2, 3, 128, 128, 16), 25)
    cell = cells.GatedDeltaNetCSSM(channels=16, **kw)
    v = cells.GatedDeltaNetCSSM.load_params(p)
    xd = _dev(x)
    assert torch.equal(cell.apply(v, xd), cell.apply(v, xd))
