"""GPU parity of the full GatedCSSM layer and its projection / short-conv
kernels against the float64 oracle (C ABI through cssm_amd)."""
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


# K <= 64: persistent kernel; K > 64 with K % 4 == 0: K-chunked kernel (ctx fused as per-frame sums of
# each row tile for HW >= 16, including tiles that span 2-9 frames); K % 4 != 0: fp32 tiled kernel.
# N not a multiple of 128 / 4, odd HW and HW < 16 (ctx from the output planes) exercise the edges.
@pytest.mark.parametrize("F,HW,K,N,silu", [(4, 1024, 64, 256, True), (3, 16384, 64, 128, False),
                                           (5, 196, 40, 72, True), (2, 49, 130, 10, False),
                                           (2, 1024, 128, 512, True), (3, 196, 224, 896, True),
                                           (2, 16, 320, 1280, False), (1, 49, 448, 90, True),
                                           (5, 100, 200, 64, True), (3, 8, 96, 64, False),
                                           (3, 49, 96, 200, True)])
def test_proj_in_plane_major_and_ctx(mods, F, HW, K, N, silu):
    _, S = mods
    print_case(test="proj_in", F=F, HW=HW, K=K, N=N)
    rng = np.random.default_rng(0)
    x = rng.standard_normal((F * HW, K))
    Wt = rng.standard_normal((K, N)) / np.sqrt(K)
    b = rng.standard_normal(N) * 0.1
    lo, hi, ctx = S.proj_in(_dev(x), _dev(Wt), _dev(b), F, HW, silu_lo=silu, silu_hi=True, want_ctx=True)
    ref = (x @ Wt + b).reshape(F, HW, N).transpose(0, 2, 1)
    ref_lo = O.silu(ref[:, : N // 2]) if silu else ref[:, : N // 2]
    ref_hi = O.silu(ref[:, N // 2:])
    assert rel_err(to_np(lo), ref_lo) < 1e-5
    assert rel_err(to_np(hi), ref_hi) < 1e-5
    assert rel_err(to_np(ctx), ref_lo.mean(axis=2)) < 1e-5


# bf16 A (the bf16-I/O projections): the persistent kernel (K <= 64) stages one bf16 plane and the
# K-chunked kernel (K > 64) loads raw bf16; both take three split products instead of six.  The
# exact product of the bf16-rounded input is the reference, at the fp32 bar.
@pytest.mark.parametrize("F,HW,K,N", [(4, 1024, 64, 256), (3, 196, 40, 72), (2, 1024, 128, 512),
                                      (3, 196, 224, 896), (2, 16, 320, 1280)])
def test_proj_in_bf16_input(mods, F, HW, K, N):
    _, S = mods
    print_case(test="proj_in_bf16", F=F, HW=HW, K=K, N=N)
    rng = np.random.default_rng(10)
    xb = _dev(rng.standard_normal((F * HW, K)), torch.bfloat16)
    x = to_np(xb)
    Wt = rng.standard_normal((K, N)) / np.sqrt(K)
    b = rng.standard_normal(N) * 0.1
    lo, hi, ctx = S.proj_in(xb, _dev(Wt), _dev(b), F, HW, silu_lo=True, silu_hi=False, want_ctx=True,
                            out_dtype=torch.float32)
    ref = (x @ Wt + b).reshape(F, HW, N).transpose(0, 2, 1)
    ref_lo = O.silu(ref[:, : N // 2])
    assert rel_err(to_np(lo), ref_lo) < 1e-5
    assert rel_err(to_np(hi), ref[:, N // 2:]) < 1e-5
    assert rel_err(to_np(ctx), ref_lo.mean(axis=2)) < 1e-5


@pytest.mark.parametrize("F,HW,K,N", [(4, 1024, 64, 64), (2, 196, 256, 128), (2, 16, 640, 320), (3, 49, 448, 224),
                                      (2, 49, 128, 48)])
def test_proj_out_bf16_input(mods, F, HW, K, N):
    """Plane-major bf16 A into the output projection (persistent and K-chunked kernels)."""
    _, S = mods
    print_case(test="proj_out_bf16", F=F, HW=HW, K=K, N=N)
    rng = np.random.default_rng(11)
    yb = _dev(rng.standard_normal((F, K, HW)), torch.bfloat16)
    y = to_np(yb)
    Wt = rng.standard_normal((K, N)) / np.sqrt(K)
    b = rng.standard_normal(N) * 0.1
    out = S.proj_out(yb, _dev(Wt), _dev(b), out_dtype=torch.float32)
    ref = y.transpose(0, 2, 1).reshape(F * HW, K) @ Wt + b
    assert rel_err(to_np(out), ref) < 1e-5


@pytest.mark.parametrize("F,HW,K,N", [(4, 1024, 64, 192), (2, 256, 64, 64), (3, 196, 256, 128)])
def test_proj_planes_bf16_input(mods, F, HW, K, N):
    _, S = mods
    print_case(test="proj_planes_bf16", F=F, HW=HW, K=K, N=N)
    rng = np.random.default_rng(12)
    xb = _dev(rng.standard_normal((F * HW, K)), torch.bfloat16)
    x = to_np(xb)
    Wt = rng.standard_normal((K, N)) / np.sqrt(K)
    b = rng.standard_normal(N) * 0.1
    out = S.proj_planes(xb, _dev(Wt), _dev(b), F, HW, act="identity", out_dtype=torch.float32)
    ref = (x @ Wt + b).reshape(F, HW, N).transpose(0, 2, 1)
    assert rel_err(to_np(out), ref) < 1e-5


# K-chunked kernel (K > 64): 4-pixel loads of plane-major A where H*W % 4 == 0 (K = 70: channels past K
# within a chunk), element loads for H*W = 49; N <= 64 takes 64-column tiles (waves split as two row
# halves by two column halves), 64-row tiles when few tiles (M = 48, 147, 1372), 128-row ones with a
# partial last tile (M = 137200)
@pytest.mark.parametrize("F,HW,K,N", [(4, 1024, 64, 64), (2, 16384, 128, 64), (3, 196, 96, 150),
                                      (3, 49, 448, 224), (2, 16, 640, 320), (2, 196, 256, 128), (5, 49, 36, 30),
                                      (3, 16, 70, 40), (3, 49, 100, 64), (7, 196, 130, 50), (700, 196, 96, 64)])
def test_proj_out_channels_last(mods, F, HW, K, N):
    _, S = mods
    print_case(test="proj_out", F=F, HW=HW, K=K, N=N)
    rng = np.random.default_rng(1)
    y = rng.standard_normal((F, K, HW))
    Wt = rng.standard_normal((K, N)) / np.sqrt(K)
    b = rng.standard_normal(N) * 0.1
    out = S.proj_out(_dev(y), _dev(Wt), _dev(b))
    ref = y.transpose(0, 2, 1).reshape(F * HW, K) @ Wt + b
    assert rel_err(to_np(out), ref) < 1e-5


@pytest.mark.parametrize("F,HW,K,N", [(3, 49, 448, 224), (2, 16, 640, 320), (2, 196, 256, 128)])
def test_proj_out_bf16_output(mods, F, HW, K, N):
    """fp32 plane-major A with a bf16 channels-last output (the CSSM-SHViT stages' out_proj): the
    K-chunked kernel keeps the split products down to order 2^-16, so beyond the output's own
    rounding the error stays at that level."""
    _, S = mods
    print_case(test="proj_out_bf16_out", F=F, HW=HW, K=K, N=N)
    rng = np.random.default_rng(11)
    y = rng.standard_normal((F, K, HW))
    Wt = rng.standard_normal((K, N)) / np.sqrt(K)
    b = rng.standard_normal(N) * 0.1
    out = S.proj_out(_dev(y), _dev(Wt), _dev(b), out_dtype=torch.bfloat16)
    assert out.dtype == torch.bfloat16
    ref = y.transpose(0, 2, 1).reshape(F * HW, K) @ Wt + b
    assert bf16_excess_err(to_np(out), ref) < 1e-4


@pytest.mark.parametrize("ks,kt", [(3, 4), (3, 0), (0, 4), (5, 2)])
def test_short_conv_matches_oracle(mods, ks, kt):
    _, S = mods
    print_case(test="short_conv", ks=ks, kt=kt)
    rng = np.random.default_rng(2)
    B, T, C, H, W = 2, 5, 6, 16, 12
    x = rng.standard_normal((B, T, C, H, W))
    sp = {"kernel": rng.standard_normal((ks, ks, 1, C)) / 3, "bias": rng.standard_normal(C) * 0.1} if ks else None
    tp = {"kernel": rng.standard_normal((kt, 1, C)) / 2, "bias": rng.standard_normal(C) * 0.1} if kt else None
    u, ctx = S.short_conv(_dev(x), {k: _dev(v) for k, v in sp.items()} if sp else None,
                          {k: _dev(v) for k, v in tp.items()} if tp else None)
    xc = x.transpose(0, 1, 3, 4, 2)                           # channels-last for the oracle helpers
    if sp:
        xc = O.depthwise_conv2d_same(xc.reshape(B * T, H, W, C), sp).reshape(B, T, H, W, C)
    if tp:
        xc = O.causal_conv_t(xc, tp)
    ref = O.silu(xc).transpose(0, 1, 4, 2, 3)
    assert rel_err(to_np(u), ref) < 1e-5
    assert rel_err(to_np(ctx), ref.mean(axis=(3, 4))) < 1e-5


LAYER_CASES = [
    # name, (B, T, H, W, C_in), cfg kwargs
    ("c1_factored_expand2", (8, 1, 32, 32, 64),
     dict(channels=64, expand=2, kernel_size=1, gate_type="factored", short_conv_size=0, short_conv_spatial_size=0)),
    ("dense_convs", (2, 4, 16, 16, 32),
     dict(channels=32, kernel_size=11, gate_type="dense", short_conv_size=4, short_conv_spatial_size=3)),
    ("factored_convs_sigmoid", (2, 3, 32, 32, 16),
     dict(channels=16, kernel_size=5, gate_type="factored", gate_activation="sigmoid")),
    ("factored_exp_128", (1, 3, 128, 128, 8),
     dict(channels=8, kernel_size=11, gate_type="factored", gate_activation="exp", short_conv_size=0,
          short_conv_spatial_size=0)),
    ("dense_64_k15_crop", (2, 2, 64, 64, 8),
     dict(channels=8, kernel_size=15, gate_type="dense", short_conv_size=2, short_conv_spatial_size=0)),
    # CSSM-SHViT-shaped stage layers (configs C5): T = 1, K = 1, expand 2
    ("c5_stage1_14", (4, 1, 14, 14, 32),
     dict(channels=32, expand=2, kernel_size=1, gate_type="factored", short_conv_size=0,
          short_conv_spatial_size=0)),
    ("c5_stage2_7", (4, 1, 7, 7, 56),
     dict(channels=56, expand=2, kernel_size=1, gate_type="factored", short_conv_size=0,
          short_conv_spatial_size=0)),
    ("c5_stage3_4", (4, 1, 4, 4, 80),
     dict(channels=80, expand=2, kernel_size=1, gate_type="factored", short_conv_size=0,
          short_conv_spatial_size=0)),
    ("small_7_T3_convs", (2, 3, 7, 7, 12),
     dict(channels=12, kernel_size=11, gate_type="dense", short_conv_size=3, short_conv_spatial_size=3)),
]


def _layer_inputs(shape, kw, seed):
    rng = np.random.default_rng(seed)
    cfg = O.GatedConfig(**kw)
    B, T, H, W, c_in = shape
    p = O.init_params(O.gated_param_shapes(cfg, c_in, H, W), rng)
    x = rng.standard_normal(shape)
    return cfg, p, x


@pytest.mark.parametrize("name,shape,kw", LAYER_CASES, ids=[c[0] for c in LAYER_CASES])
def test_gated_layer_matches_oracle(mods, name, shape, kw):
    cells, _ = mods
    print_case(test="gated_layer", case=name)
    cfg, p, x = _layer_inputs(shape, kw, 42)
    ref = O.gated_forward(p, x, cfg)
    cell = cells.GatedCSSM(**kw)
    y = cell.apply(cells.GatedCSSM.load_params(p), _dev(x))
    torch.cuda.synchronize()
    assert y.shape == shape[:4] + (kw["channels"],)
    assert rel_err(to_np(y), ref) <= TOL_F32


def test_gated_layer_bf16_io(mods):
    cells, _ = mods
    print_case(test="gated_layer_bf16")
    kw = dict(channels=32, expand=2, kernel_size=1, gate_type="factored", short_conv_size=0,
              short_conv_spatial_size=0)
    cfg, p, x = _layer_inputs((4, 1, 16, 16, 32), kw, 7)
    xb = _dev(x, torch.bfloat16)
    y = cells.GatedCSSM(**kw).apply(cells.GatedCSSM.load_params(p), xb)
    assert y.dtype == torch.bfloat16
    ref = O.gated_forward(p, to_np(xb), cfg)
    # intermediates are fp32: beyond the output's own bf16 rounding the error is at the fp32 level
    assert bf16_excess_err(to_np(y), ref) <= TOL_BF16
    assert np.sqrt(np.mean((to_np(y) - ref) ** 2)) <= TOL_BF16 * np.sqrt(np.mean(ref ** 2))


C5_STAGES = [("c5_14x14x128", (2, 1, 14, 14, 128)), ("c5_7x7x224", (2, 1, 7, 7, 224)),
             ("c5_4x4x320", (2, 1, 4, 4, 320))]


@pytest.mark.parametrize("name,shape", C5_STAGES, ids=[c[0] for c in C5_STAGES])
def test_gated_layer_c5_stage_widths_bf16(mods, name, shape):
    """One layer of each CSSM-SHViT stage at its own width (C5: 128 / 224 / 320 channels, expand 2,
    T = 1, kernel_size 1, bf16 I/O): in_proj on the K-chunked kernel with its per-frame ctx
    epilogue at K = 128 / 224 / 320, the small-plane scan at 14 x 14 / 7 x 7 and the 4 x 4
    planes, out_proj at K = 256 / 448 / 640 with a bf16 output."""
    cells, _ = mods
    print_case(test="gated_layer_c5_width", case=name)
    C = shape[-1]
    kw = dict(channels=C, expand=2, kernel_size=1, gate_type="factored", short_conv_size=0,
              short_conv_spatial_size=0)
    cfg, p, x = _layer_inputs(shape, kw, 61)
    xb = _dev(x, torch.bfloat16)
    y = cells.GatedCSSM(**kw).apply(cells.GatedCSSM.load_params(p), xb)
    torch.cuda.synchronize()
    assert y.dtype == torch.bfloat16 and tuple(y.shape) == shape
    ref = O.gated_forward(p, to_np(xb), cfg)
    assert bf16_excess_err(to_np(y), ref) <= TOL_BF16
    assert np.sqrt(np.mean((to_np(y) - ref) ** 2)) <= TOL_BF16 * np.sqrt(np.mean(ref ** 2))
    # the same layer with float32 output holds the fp32 bar against the bf16-rounded input
    yf = cells.GatedCSSM(**kw).apply(cells.GatedCSSM.load_params(p), xb, out_dtype=torch.float32)
    assert rel_err(to_np(yf), ref) <= TOL_F32


def test_gated_layer_two_parameter_trees(mods):
    """One cell applied to two parameter trees of the same shape in turn (e.g. a reloaded
    checkpoint): each output follows its own weights, whatever addresses the allocator reuses."""
    cells, _ = mods
    print_case(test="gated_layer_two_trees")
    kw = dict(channels=8, kernel_size=5, gate_type="factored", short_conv_size=0, short_conv_spatial_size=0)
    cell = cells.GatedCSSM(**kw)
    for seed in (51, 52, 51):
        cfg, p, x = _layer_inputs((1, 2, 16, 16, 8), kw, seed)
        v = cells.GatedCSSM.load_params(p)
        y = cell.apply(v, _dev(x))
        del v
        assert rel_err(to_np(y), O.gated_forward(p, x, cfg)) <= TOL_F32, seed


def test_gated_layer_is_causal_in_time(mods):
    cells, _ = mods
    print_case(test="gated_layer_causal")
    kw = dict(channels=16, kernel_size=3, gate_type="dense", short_conv_size=4, short_conv_spatial_size=3)
    cfg, p, x = _layer_inputs((1, 6, 16, 16, 16), kw, 3)
    cell = cells.GatedCSSM(**kw)
    v = cells.GatedCSSM.load_params(p)
    y1 = to_np(cell.apply(v, _dev(x)))
    x2 = x.copy()
    x2[:, 4:] += 1.0
    y2 = to_np(cell.apply(v, _dev(x2)))
    assert np.array_equal(y1[:, :4], y2[:, :4])
    assert not np.allclose(y1[:, 4:], y2[:, 4:])
