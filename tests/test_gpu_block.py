"""GPU parity of the CSSMSHViTBlock wiring (norm1, pos_conv, the cell, frame
selection, output activation, residual) and its kernels against the float64
oracle, through the C ABI (cssm_amd.blocks / cssm_amd.spectral)."""
import numpy as np
import pytest

from oracle import cssm_oracle as O
from tests.gpu_util import bf16_excess_err, print_case, rel_err, to_np

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

TOL_F32 = 1e-4
TOL_BF16 = 5e-3
MODES = ["global_layer", "temporal_layer", "layer"]


@pytest.fixture(scope="module")
def mods():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from cssm_amd import blocks, spectral
    return blocks, spectral


def _dev(a, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda", dtype)


def _norm_pos_params(rng, C):
    return ({"scale": 1.0 + 0.2 * rng.standard_normal(C), "bias": 0.2 * rng.standard_normal(C)},
            {"kernel": rng.standard_normal((3, 3, 1, C)) / 3.0, "bias": 0.1 * rng.standard_normal(C)})


# ------------------------------------------------------------------- kernels

@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_block_norm_stats(mods, mode, dt):
    _, S = mods
    print_case(test="block_norm_stats", mode=mode, dt=dt)
    rng = np.random.default_rng(1)
    shape = (3, 2, 7, 9, 12)
    x = 1.5 + 2.0 * rng.standard_normal(shape)
    xd = _dev(x, torch.float32 if dt == "f32" else torch.bfloat16)
    xr = to_np(xd)
    st = to_np(S.block_norm_stats(xd, mode))
    axes = O.BLOCK_NORM_AXES[mode]
    keep = [a for a in range(5) if a not in axes]
    xg = np.transpose(xr, keep + list(axes)).reshape(st.shape[0], -1)
    mu = xg.mean(axis=1)
    rstd = 1.0 / np.sqrt(xg.var(axis=1) + 1e-6)
    assert np.max(np.abs(st[:, 0] - mu)) < 1e-6 * np.max(np.abs(mu))
    assert np.max(np.abs(st[:, 1] / rstd - 1.0)) < 1e-6


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("T_in,T_out,pos", [(3, 3, True), (1, 4, True), (2, 2, False), (1, 1, True)])
def test_block_norm_posconv(mods, mode, T_in, T_out, pos):
    _, S = mods
    print_case(test="block_norm_posconv", mode=mode, T_in=T_in, T_out=T_out, pos=pos)
    rng = np.random.default_rng(2)
    B, H, W, C = 2, 7, 6, 12
    x = 0.7 + 1.3 * rng.standard_normal((B, T_in, H, W, C))
    n1, pc = _norm_pos_params(rng, C)
    xd = _dev(x)
    st = S.block_norm_stats(xd, mode)
    got = S.block_norm_posconv(xd, st, mode, _dev(n1["scale"]), _dev(n1["bias"]),
                               _dev(pc["kernel"]) if pos else None, _dev(pc["bias"]) if pos else None, T_out)
    x5 = np.repeat(x, T_out, axis=1) if T_in == 1 else x
    h = O.block_norm1(x5, n1["scale"], n1["bias"], mode)
    if pos:
        h = h + O.depthwise_conv2d_same(h.reshape(-1, H, W, C), pc).reshape(h.shape)
    assert rel_err(to_np(got), h) <= 1e-5


@pytest.mark.parametrize("act", ["none", "gelu", "silu"])
@pytest.mark.parametrize("T_res,T_y,T_out", [(1, 4, 1), (3, 3, 3), (3, 2, 1)])
def test_block_residual(mods, act, T_res, T_y, T_out):
    _, S = mods
    print_case(test="block_residual", act=act, T_res=T_res, T_y=T_y, T_out=T_out)
    rng = np.random.default_rng(3)
    B, H, W, C = 2, 5, 4, 6
    res = rng.standard_normal((B, T_res, H, W, C))
    y = 2.0 * rng.standard_normal((B, T_y, H, W, C))
    got = to_np(S.block_residual(_dev(res), _dev(y), T_out, act))
    ys = y[:, -1:] if T_out == 1 else y
    ys = {"none": ys, "gelu": O.gelu_tanh(ys), "silu": O.silu(ys)}[act]
    ref = (res[:, -1:] if T_out == 1 else res) + ys
    assert rel_err(got, ref) <= 1e-6


# --------------------------------------------------------------------- block

BLOCK_CASES = [
    # name, block kwargs, input shape (4-D image or 5-D video), num_timesteps
    ("gated_image_global", dict(cssm_type="gated", kernel_size=5), (2, 14, 14, 16), 3),
    ("gated_image_T1_k1_no_convs", dict(cssm_type="gated", kernel_size=1, short_conv_size=0,
                                        short_conv_spatial_size=0), (3, 7, 7, 24), 1),
    ("gated_video_temporal_gelu", dict(cssm_type="gated", kernel_size=3, block_norm="temporal_layer",
                                       output_act="gelu"), (2, 3, 8, 8, 16), None),
    ("gated_image_layer_silu_no_pos", dict(cssm_type="gated", kernel_size=5, block_norm="layer",
                                           output_act="silu", use_pos_conv=False), (2, 16, 16, 8), 2),
    ("gdn_image_global", dict(cssm_type="gdn", delta_key_dim=2, kernel_size=5), (2, 8, 8, 16), 2),
    ("gdn_video_layer", dict(cssm_type="gdn", delta_key_dim=4, kernel_size=3, block_norm="layer"),
     (1, 3, 8, 8, 16), None),
    # the CSSM-SHViT stage shapes with the gdn cell (cssm_shvit_s1(cssm_type='gdn')): small-plane transforms
    ("gdn_image_14x14", dict(cssm_type="gdn", delta_key_dim=4, kernel_size=5), (2, 14, 14, 16), 3),
    ("gdn_image_7x7_T1", dict(cssm_type="gdn", delta_key_dim=2, kernel_size=3), (3, 7, 7, 8), 1),
]


def _oracle_block(kw, C, H, W, rng):
    kw = dict(kw)
    ctype = kw.pop("cssm_type")
    bk = {k: kw.pop(k) for k in ("block_norm", "use_pos_conv", "output_act") if k in kw}
    if ctype == "gdn":
        cfg = O.GDNConfig(channels=C, gate_type="factored", **kw)
        cell_p = O.init_params(O.gdn_param_shapes(cfg, H, W), rng, spectral_init="xavier")
        fwd = lambda q, h: O.gdn_forward(q, h, cfg)
    else:
        cfg = O.GatedConfig(channels=C, gate_type="factored", **kw)
        cell_p = O.init_params(O.gated_param_shapes(cfg, C, H, W), rng)
        fwd = lambda q, h: O.gated_forward(q, h, cfg)
    n1, pc = _norm_pos_params(rng, C)
    p = {"norm1": n1, "cssm": cell_p}
    if bk.get("use_pos_conv", True):
        p["pos_conv"] = pc
    return p, fwd, bk


@pytest.mark.parametrize("name,kw,shape,T", BLOCK_CASES, ids=[c[0] for c in BLOCK_CASES])
def test_block_matches_oracle(mods, name, kw, shape, T):
    blocks, _ = mods
    print_case(test="shvit_block", case=name)
    rng = np.random.default_rng(31)
    H, W, C = shape[-3:]
    p, fwd, bk = _oracle_block(kw, C, H, W, rng)
    x = rng.standard_normal(shape)
    ref = O.shvit_block_mixer(p, x, fwd, num_timesteps=T or shape[1], **bk)
    blk = blocks.CSSMSHViTBlock(dim=C, num_timesteps=T or shape[1], **kw)
    got = blk.token_mixer(blocks.CSSMSHViTBlock.load_params(p), _dev(x))
    torch.cuda.synchronize()
    assert tuple(got.shape) == shape
    assert rel_err(to_np(got), ref) <= TOL_F32


def test_block_bf16_io(mods):
    """C5-stage-shaped gated block (image, T = 1, kernel_size 1) with bf16 I/O."""
    blocks, _ = mods
    print_case(test="shvit_block_bf16")
    rng = np.random.default_rng(32)
    kw = dict(cssm_type="gated", kernel_size=1, short_conv_size=0, short_conv_spatial_size=0)
    shape = (4, 14, 14, 32)
    p, fwd, bk = _oracle_block(kw, 32, 14, 14, rng)
    xb = _dev(rng.standard_normal(shape), torch.bfloat16)
    got = blocks.CSSMSHViTBlock(dim=32, num_timesteps=1, **kw).token_mixer(blocks.CSSMSHViTBlock.load_params(p), xb)
    assert got.dtype == torch.bfloat16
    ref = O.shvit_block_mixer(p, to_np(xb), fwd, num_timesteps=1, **bk)
    assert bf16_excess_err(to_np(got), ref) <= TOL_BF16


def test_block_rejects_what_is_not_built(mods):
    blocks, _ = mods
    with pytest.raises(NotImplementedError):
        blocks.CSSMSHViTBlock(dim=16, cssm_type="gdn", static_image_fast_path=True)


def _full_block_params(p, rng, C, mlp_ratio, timestep_gate, use_dwconv):
    """norm2 / mlp (and gate_fc1 / gate_fc2) added to a token-mixer parameter tree."""
    hid = int(C * mlp_ratio)
    p = dict(p)
    p["norm2"] = {"scale": 1.0 + 0.2 * rng.standard_normal(C), "bias": 0.2 * rng.standard_normal(C)}
    p["mlp"] = {"fc1": {"kernel": rng.standard_normal((C, hid)) / np.sqrt(C), "bias": 0.1 * rng.standard_normal(hid)},
                "fc2": {"kernel": rng.standard_normal((hid, C)) / np.sqrt(hid), "bias": 0.1 * rng.standard_normal(C)}}
    if use_dwconv:
        p["mlp"]["dwconv"] = {"dwconv": {"kernel": rng.standard_normal((3, 3, 1, hid)) / 3,
                                         "bias": 0.1 * rng.standard_normal(hid)}}
    if timestep_gate:
        hg = max(C // 4, 8)
        p["gate_fc1"] = {"kernel": rng.standard_normal((2 * C, hg)) / np.sqrt(2 * C), "bias": 0.1 * rng.standard_normal(hg)}
        p["gate_fc2"] = {"kernel": rng.standard_normal((hg, 1)) / np.sqrt(hg), "bias": 0.1 * rng.standard_normal(1)}
    return p


FULL_CASES = [
    # name, block kwargs (incl. cssm_type), shape, num_timesteps, timestep_gate, use_dwconv, mlp_ratio
    ("gated_image_mlp", dict(cssm_type="gated", kernel_size=5), (2, 14, 14, 16), 3, False, True, 4.0),
    ("gated_image_timestep_gate", dict(cssm_type="gated", kernel_size=3, output_act="gelu"), (2, 8, 8, 16), 4,
     True, True, 2.0),
    ("gdn_video_keep_time_mlp", dict(cssm_type="gdn", delta_key_dim=2, kernel_size=3, block_norm="temporal_layer"),
     (1, 3, 8, 8, 16), None, False, True, 4.0),
    ("gdn_video_timestep_gate_no_dwconv", dict(cssm_type="gdn", delta_key_dim=4, kernel_size=3, block_norm="layer"),
     (2, 3, 8, 8, 16), None, True, False, 3.0),
]


@pytest.mark.parametrize("name,kw,shape,T,tg,dw,ratio", FULL_CASES, ids=[c[0] for c in FULL_CASES])
def test_full_block_matches_oracle(mods, name, kw, shape, T, tg, dw, ratio):
    """The whole block (cssm_shvit.py:65-266): token mixer, optional timestep-gate pooling,
    then norm2 -> Mlp (fc1 -> gelu -> + dwconv -> fc2) -> residual."""
    blocks, _ = mods
    print_case(test="shvit_full_block", case=name)
    rng = np.random.default_rng(33)
    H, W, C = shape[-3:]
    p, fwd, bk = _oracle_block(kw, C, H, W, rng)
    p = _full_block_params(p, rng, C, ratio, tg, dw)
    x = rng.standard_normal(shape)
    ref = O.shvit_block(p, x, fwd, num_timesteps=T or shape[1], timestep_gate=tg, use_dwconv=dw, **bk)
    blk = blocks.CSSMSHViTBlock(dim=C, num_timesteps=T or shape[1], timestep_gate=tg, use_dwconv=dw, mlp_ratio=ratio,
                                **kw)
    assert blk.param_shapes(H, W).keys() == p.keys()
    got = blk.apply(blocks.CSSMSHViTBlock.load_params(p), _dev(x))
    torch.cuda.synchronize()
    assert tuple(got.shape) == ref.shape
    assert rel_err(to_np(got), ref) <= TOL_F32


def test_full_block_bf16_io(mods):
    blocks, _ = mods
    print_case(test="shvit_full_block_bf16")
    rng = np.random.default_rng(34)
    kw = dict(cssm_type="gated", kernel_size=1, short_conv_size=0, short_conv_spatial_size=0)
    p, fwd, bk = _oracle_block(kw, 32, 7, 7, rng)
    p = _full_block_params(p, rng, 32, 4.0, False, True)
    xb = _dev(rng.standard_normal((4, 7, 7, 32)), torch.bfloat16)
    got = blocks.CSSMSHViTBlock(dim=32, num_timesteps=1, **kw).apply(blocks.CSSMSHViTBlock.load_params(p), xb)
    assert got.dtype == torch.bfloat16
    ref = O.shvit_block(p, to_np(xb), fwd, num_timesteps=1, **bk)
    assert bf16_excess_err(to_np(got), ref) <= TOL_BF16
