"""GPU parity of the gated-cell kernels against the float64 oracle.

Bar: max|y_gpu - y_ref| / RMS(y_ref) <= 1e-4 for
fp32 I/O and <= 5e-3 for bf16 I/O.  All calls go through the C ABI.
"""
import math

import numpy as np
import pytest

from oracle import cssm_oracle as O
from tests.gpu_util import bf16_excess_err, print_case, rel_err, to_np

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

TOL_F32 = 1e-4
TOL_BF16 = 5e-3


@pytest.fixture(scope="module")
def S():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from cssm_amd import spectral
    return spectral


def _dev(a, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda", dtype)


def _rand_gates(rng, B, T, H, W, zero_rows=False):
    Wf = W // 2 + 1
    delta = O.softplus(rng.standard_normal((B, T, H, Wf)))
    gB = rng.standard_normal((B, T, H, Wf))
    gC = rng.standard_normal((B, T, H, Wf))
    if zero_rows:
        gB[:, :, 1, :] = 0.0
    return delta, gB, gC


def _scan_cols(H, W):
    from cssm_amd import spectral
    return np.asarray(spectral.scan_col_order(H, W))


def _pack_gates(delta, gB, gC, H, W):
    """The scan's gate planes from oracle gate values: [exp(-Delta), (Delta + 1e-8) B,
    2e-7 (Delta + 1e-8), C / (2 H W)], columns in the scan's order."""
    d = delta + 1e-8
    g = np.stack([np.exp(-delta), d * gB, d * 2e-7, gC * (0.5 / (H * W))], axis=-1)
    return _dev(g[:, :, :, _scan_cols(H, W), :])


def _scan_korder(H, W):
    from cssm_amd import spectral
    return np.asarray(spectral.scan_khat_order(H, W))


def _scan_khat(khat, H, W):
    """Floored K_hat (C, H, Wf) in the scan layout (slot s holds natural bin korder[s])."""
    C = khat.shape[0]
    return _dev(khat.reshape(C, -1)[:, _scan_korder(H, W)].reshape(khat.shape), torch.complex64)


# ------------------------------------------------------------- spectral kernel

@pytest.mark.parametrize("C,K,H,W", [(3, 11, 128, 128), (5, 11, 32, 32), (2, 1, 32, 32), (4, 15, 8, 8),
                                     (2, 3, 7, 7), (3, 11, 14, 14), (2, 5, 4, 4), (2, 11, 16, 16)])
def test_spectral_kernel_matches_oracle(S, C, K, H, W):
    print_case(test="spectral_kernel", C=C, K=K, H=H, W=W)
    rng = np.random.default_rng(7)
    k = rng.standard_normal((C, K, K)) * 0.3
    got = S.spectral_kernel(_dev(k), H, W, rho=0.999, squash=True, goom_floor=False)
    torch.cuda.synchronize()
    ref = O.spectral_kernel(k, H, W, 0.999)
    err = np.max(np.abs(got.cpu().numpy().astype(np.complex128) - ref))
    assert err < 1e-6 * max(1.0, np.max(np.abs(ref)))


def test_spectral_kernel_goom_floor(S):
    print_case(test="spectral_kernel_floor")
    k = np.zeros((2, 3, 3))
    k[1, 1, 1] = 0.5
    got = S.spectral_kernel(_dev(k), 8, 8, goom_floor=True).cpu().numpy()
    assert np.all(got[0] == np.complex64(1e-7))       # all-zero kernel -> every bin floored
    assert np.allclose(np.abs(got[1]), 0.999 * 0.5 / 1.5, rtol=1e-6)


@pytest.mark.parametrize("H", [128, 32])
def test_spectral_kernel_scan_order(S, H):
    """scan_order = 1 stores the same values in the scan layout: columns in the scan's
    order, and at 128 x 128 rows u and u + 16 paired within each column's slots."""
    print_case(test="spectral_kernel_scan_order", H=H)
    k = np.random.default_rng(8).standard_normal((3, 11, 11)) * 0.3
    nat = S.spectral_kernel(_dev(k), H, H, goom_floor=True)
    so = S.spectral_kernel(_dev(k), H, H, goom_floor=True, scan_order=True)
    ko = torch.as_tensor(_scan_korder(H, H), device="cuda")
    assert torch.equal(so.reshape(3, -1), nat.reshape(3, -1)[:, ko])
    if H == 128:
        # slot pair (2 s, 2 s + 1) of column position p holds rows u, u + 16 of one column
        assert torch.equal(so.reshape(3, -1)[:, 1], nat[:, 16, int(_scan_cols(H, H)[0])])


# ------------------------------------------------------------------ plane mean

# plane sizes on both sides of the lanes-per-plane switch points (16, 32, 64 lanes, whole block);
# 2 * 3 * 5 = 30 planes leave a partial last block for every size
@pytest.mark.parametrize("hw", [(4, 4), (7, 7), (14, 14), (16, 16), (32, 32), (40, 40)])
@pytest.mark.parametrize("silu", [False, True])
def test_plane_mean(S, silu, hw):
    print_case(test="plane_mean", silu=silu, hw=hw)
    rng = np.random.default_rng(3)
    x = rng.standard_normal((2, 3, 5) + hw)
    got = to_np(S.plane_mean(_dev(x), silu=silu))
    ref = (O.silu(x) if silu else x).mean(axis=(-2, -1))
    assert np.max(np.abs(got - ref)) < 1e-6


# ----------------------------------------------------------------------- gates

@pytest.mark.parametrize("gate_type", ["dense", "factored"])
@pytest.mark.parametrize("act", ["softplus", "sigmoid", "exp"])
# (C, H): the factored weights go through LDS where C % 4 == 0 and they fit 64 KB ((448, 7), (640, 4),
# (96, 14), (16, 16)); (64, 128) and C = 30 take the per-product loads
@pytest.mark.parametrize("shape", [(16, 16), (448, 7), (640, 4), (96, 14), (64, 128), (30, 7)])
def test_gated_gates_match_oracle(S, gate_type, act, shape):
    print_case(test="gated_gates", gate_type=gate_type, act=act, shape=shape)
    rng = np.random.default_rng(11)
    C, H = shape
    B, T, W = 2, 3, H
    cfg = O.GatedConfig(channels=C, gate_type=gate_type, gate_activation=act, short_conv_size=0,
                        short_conv_spatial_size=0, kernel_size=3)
    p = O.init_params(O.gated_param_shapes(cfg, C, H, W), rng)
    ctx = rng.standard_normal((B, T, C))
    delta, gB, gC = O.gated_gates(ctx, p, cfg, H, W)
    pd = {k: ({kk: _dev(vv) for kk, vv in v.items()} if isinstance(v, dict) else _dev(v))
          for k, v in p.items()}
    got = to_np(S.gated_gates(_dev(ctx), pd, H, W, gate_type, act, c_scale=0.5))
    # the planes come in the scan's column order
    cols = _scan_cols(H, W)
    delta, gB, gC = delta[..., cols], gB[..., cols], gC[..., cols]
    d = delta + 1e-8
    assert np.max(np.abs(got[..., 0] - np.exp(-delta))) < 1e-5
    # fp32 dot products over C, times exp's up-to-e^2 Delta: max error / RMS up to a few 1e-5
    assert rel_err(got[..., 1], d * gB) < 3e-5
    assert np.max(np.abs(got[..., 2] - d * 2e-7)) < 2e-12 * max(1, np.max(delta))
    assert rel_err(got[..., 3], 0.5 * gC) < 1e-5


# (B, T, H, K, N, dtype): the C5 stages on the K-chunked projection (channel sums per tile,
# tiles spanning frames), C1 / C2-like planes on the persistent one (one frame per tile), and
# 7 x 7 at K = 64, where the projection takes no sums and ctx is a plane mean
PIG_CASES = [(2, 1, 14, 128, 512, torch.bfloat16), (3, 1, 7, 224, 896, torch.bfloat16),
             (2, 1, 4, 320, 1280, torch.bfloat16), (2, 3, 32, 64, 256, torch.float32),
             (1, 2, 128, 64, 128, torch.float32), (2, 2, 7, 64, 128, torch.float32)]


@pytest.mark.parametrize("gate_type", ["factored", "dense"])
@pytest.mark.parametrize("B,T,H,K,N,dt", PIG_CASES, ids=[f"{c[2]}x{c[2]}_K{c[3]}_N{c[4]}" for c in PIG_CASES])
def test_proj_in_gates_matches_separate_calls(S, gate_type, B, T, H, K, N, dt):
    """cssm_proj_in_gates (the gate kernel reducing the projection's channel sums itself) against
    cssm_proj_in with ctx followed by cssm_gated_gates: the same planes, ctx and gates, bit for bit;
    the gates also against the oracle on the projection's own ctx."""
    print_case(test="proj_in_gates", gate_type=gate_type, shape=(B, T, H, K, N), dtype=dt)
    rng = np.random.default_rng(12)
    W, C = H, N // 2
    cfg = O.GatedConfig(channels=C, gate_type=gate_type, gate_activation="softplus", short_conv_size=0,
                        short_conv_spatial_size=0, kernel_size=3)
    p = O.init_params(O.gated_param_shapes(cfg, C, H, W), rng)
    pd = {k: ({kk: _dev(vv) for kk, vv in v.items()} if isinstance(v, dict) else _dev(v))
          for k, v in p.items()}
    x = _dev(rng.standard_normal((B * T * H * W, K)), dt)
    w_in = _dev(rng.standard_normal((K, N)) / math.sqrt(K))
    b_in = _dev(0.1 * rng.standard_normal(N))
    cs = S.scan_c_scale(H, W)
    lo, hi, ctx = S.proj_in(x, w_in, b_in, B * T, H * W, silu_lo=True, silu_hi=True, want_ctx=True,
                            out_dtype=torch.float32)
    gates = S.gated_gates(ctx.view(B, T, C), pd, H, W, gate_type, "softplus", c_scale=cs)
    lo2, hi2, ctx2, gates2 = S.proj_in_gates(x, w_in, b_in, B, T, H, W, pd, gate_type, "softplus", c_scale=cs,
                                             silu_lo=True, silu_hi=True, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(lo, lo2) and torch.equal(hi, hi2)
    assert torch.equal(ctx.view(B, T, C), ctx2)
    assert torch.equal(gates, gates2)
    delta, gB, gC = O.gated_gates(to_np(ctx2), p, cfg, H, W)
    cols = _scan_cols(H, W)
    d = (delta + 1e-8)[..., cols]
    got = to_np(gates2)
    assert rel_err(got[..., 1], d * gB[..., cols]) < 3e-5
    assert rel_err(got[..., 3], cs * gC[..., cols]) < 1e-5


# --------------------------------------------------------------- fused scan

SCAN_CASES = [
    # (B, T, C, H, W)
    (2, 1, 128, 4, 4), (1, 3, 128, 4, 4), (2, 3, 32, 8, 8), (2, 4, 16, 16, 16), (1, 3, 8, 32, 32),
    (2, 5, 8, 32, 32), (1, 3, 4, 64, 64), (2, 2, 2, 64, 64), (1, 3, 2, 128, 128), (2, 8, 1, 128, 128),
    # direct-DFT small planes (CSSM-SHViT stage shapes and odd sizes); groups span batch
    # elements and the last group is partial
    (3, 2, 20, 14, 14), (2, 3, 40, 7, 7), (1, 1, 8, 12, 12), (2, 2, 5, 5, 5), (1, 3, 33, 15, 15),
    (2, 2, 3, 9, 9), (1, 2, 70, 6, 6), (2, 1, 4, 3, 3),
    # groups inside one batch element move as 4-element vectors when their start is aligned:
    # every group at 7 x 7 / C = 128 over three steps; at 14 x 14 / C = 40 the groups alternate
    # between one batch element and two; at 3 x 3 / C = 301 some groups lie in one batch
    # element but start at an odd element (element path)
    (2, 3, 128, 7, 7), (1, 2, 40, 14, 14), (2, 2, 301, 3, 3),
    # more even sizes, and groups whose last planes lie past P
    (2, 3, 10, 10, 10), (1, 1, 7, 14, 14), (1, 4, 9, 12, 12),
]


@pytest.mark.parametrize("B,T,C,H,W", SCAN_CASES)
def test_gated_scan_matches_oracle(S, B, T, C, H, W):
    print_case(test="gated_scan", B=B, T=T, C=C, H=H, W=W)
    rng = np.random.default_rng(1000 + H + T)
    xm = rng.standard_normal((B, T, C, H, W))
    z = rng.standard_normal((B, T, C, H, W))
    khat = O.goom_floor(O.spectral_kernel(rng.standard_normal((C, 5, 5)) * 0.3, H, W))
    delta, gB, gC = _rand_gates(rng, B, T, H, W)
    y = S.gated_scan(_dev(xm), _dev(z), _pack_gates(delta, gB, gC, H, W), _scan_khat(khat, H, W),
                     u_silu=True, z_silu=True)
    torch.cuda.synchronize()
    ref = O.gated_core(O.silu(xm), O.silu(z), khat, delta, gB, gC)
    assert rel_err(to_np(y), ref) <= TOL_F32


@pytest.mark.parametrize("H", [8, 32, 128, 14])
def test_gated_scan_goom_floor_zero_inputs(S, H):
    """Exact zeros (a zero frame, a zero B row) take to_goom's 1e-7 floor."""
    print_case(test="gated_scan_floor", H=H)
    rng = np.random.default_rng(5)
    B, T, W = 1, 4, H
    C = {8: 32, 32: 8, 128: 2, 14: 4}[H]
    xm = rng.standard_normal((B, T, C, H, W))
    xm[:, 0] = 0.0
    zg = rng.standard_normal((B, T, C, H, W))
    khat = O.goom_floor(O.spectral_kernel(rng.standard_normal((C, 3, 3)) * 0.3, H, W))
    delta, gB, gC = _rand_gates(rng, B, T, H, W, zero_rows=True)
    y = S.gated_scan(_dev(xm), _dev(zg), _pack_gates(delta, gB, gC, H, W), _scan_khat(khat, H, W))
    ref = O.gated_core(xm, zg, khat, delta, gB, gC)
    assert rel_err(to_np(y), ref) <= TOL_F32
    # the all-zero first frame is pure floor: gC (Delta + 1e-8) 1e-7 through irfft2
    y0 = to_np(y)[:, 0]
    assert rel_err(y0, ref[:, 0]) <= TOL_F32


@pytest.mark.parametrize("B,T,C,H,W", [(2, 4, 8, 32, 32), (1, 3, 2, 128, 128), (2, 2, 16, 16, 16),
                                       (2, 1, 48, 14, 14), (2, 2, 24, 7, 7), (2, 2, 128, 7, 7),
                                       (1, 2, 170, 4, 4)])
def test_gated_scan_bf16_io(S, B, T, C, H, W):
    print_case(test="gated_scan_bf16", B=B, T=T, C=C, H=H, W=W)
    rng = np.random.default_rng(99)
    xm = rng.standard_normal((B, T, C, H, W))
    z = rng.standard_normal((B, T, C, H, W))
    xm_b = _dev(xm, torch.bfloat16)
    z_b = _dev(z, torch.bfloat16)
    khat = O.goom_floor(O.spectral_kernel(rng.standard_normal((C, 5, 5)) * 0.3, H, W))
    delta, gB, gC = _rand_gates(rng, B, T, H, W)
    y = S.gated_scan(xm_b, z_b, _pack_gates(delta, gB, gC, H, W), _scan_khat(khat, H, W),
                     u_silu=True, z_silu=True)
    assert y.dtype == torch.bfloat16
    # reference on the bf16-rounded inputs, exact arithmetic; the bar applies beyond the
    # output's own bf16 rounding
    ref = O.gated_core(O.silu(to_np(xm_b)), O.silu(to_np(z_b)), khat, delta, gB, gC)
    assert bf16_excess_err(to_np(y), ref) <= TOL_BF16
    assert np.sqrt(np.mean((to_np(y) - ref) ** 2)) <= TOL_BF16 * np.sqrt(np.mean(ref ** 2))


def test_gated_scan_c2_full_size_sampled(S):
    """BASELINE config 2 shape (B=128, T=8, 128x128, C=64) run whole; sampled planes vs oracle,
    and the scan must not depend on the frames being repeated."""
    print_case(test="gated_scan_c2_full")
    B, T, C, H, W = 128, 8, 64, 128, 128
    g = torch.Generator(device="cuda").manual_seed(0)
    img = torch.randn((B, 1, C, H, W), generator=g, device="cuda")
    u = img.expand(B, T, C, H, W).contiguous()
    del img
    z = torch.randn((B, T, C, H, W), generator=g, device="cuda")
    rng = np.random.default_rng(0)
    khat = O.goom_floor(O.spectral_kernel(rng.standard_normal((C, 11, 11)) * 0.02, H, W))
    delta, gB, gC = _rand_gates(rng, B, T, H, W)
    y = S.gated_scan(u, z, _pack_gates(delta, gB, gC, H, W), _scan_khat(khat, H, W),
                     u_silu=True, z_silu=True)
    torch.cuda.synchronize()
    for (b, c) in [(0, 0), (17, 33), (127, 63), (64, 1)]:
        ub = to_np(u[b:b + 1, :, c:c + 1])
        zb = to_np(z[b:b + 1, :, c:c + 1])
        ref = O.gated_core(O.silu(ub), O.silu(zb), khat[c:c + 1], delta[b:b + 1], gB[b:b + 1], gC[b:b + 1])
        assert rel_err(to_np(y[b:b + 1, :, c:c + 1]), ref) <= TOL_F32, (b, c)
    assert torch.isfinite(y).all().item()


def test_gated_scan_rejects_bad_input(S):
    from cssm_amd._lib import CssmError
    print_case(test="gated_scan_errors")
    u = torch.zeros((1, 1, 1, 24, 24), device="cuda")
    gates = torch.zeros((1, 1, 24, 13, 4), device="cuda")
    kh = torch.zeros((1, 24, 13), dtype=torch.complex64, device="cuda")
    with pytest.raises(CssmError, match="no fused kernel"):
        S.gated_scan(u, u, gates, kh)
