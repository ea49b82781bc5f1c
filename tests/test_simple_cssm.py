"""SimpleCSSM wiring (simple_cssm.py:63-558).  CPU: the product's parameter tree
reproduces the reference's published whole-model parameter counts
(benchmarks/results/bench_image_timing.csv, built by bench_image_timing.py:119-142),
and the oracle restatement is pinned by the image repeat, the residual, register
stripping, max-pool padding and readout closed forms."""
import numpy as np
import pytest

from oracle import cssm_oracle as O

torch = pytest.importorskip("torch")
from cssm_amd.simple_cssm import SimpleCSSM  # noqa: E402

BENCH = dict(num_classes=1, depth=1, kernel_size=11, seq_len=1, frame_readout="last", pos_embed="none",
             stem_mode="pathtracker", stem_layers=0, norm_type="layer")


@pytest.mark.parametrize("cssm,H,D,count", [("gated", 16, 256, 346033), ("gated", 32, 64, 127969),
                                            ("gdn", 16, 256, 556961)])
def test_param_count_matches_reference_csv(cssm, H, D, count):
    """bench_image_timing.csv:86 / :148 / :98 (3-channel input, dense gates, default convs)."""
    m = SimpleCSSM(cssm_type=cssm, embed_dim=D, **BENCH)
    p, bs = m.param_shapes((1, H, H, 3))
    assert O.count_params(p) == count and not bs
    cfg = O.SimpleConfig(cssm_type=cssm, embed_dim=D, **{k: v for k, v in BENCH.items() if k != "seq_len"})
    po, _ = O.simple_param_shapes(cfg, (1, H, H, 3))
    assert po == p


@pytest.mark.parametrize("kw", [dict(stem_mode="default", stem_layers=2, norm_type="batch", depth=2,
                                     inter_mlp_ratio=2.0, n_register_tokens=2, pos_embed="learnable",
                                     cssm_type="gdn_d3"),
                                dict(stem_mode="pathtracker", stem_norm_order="pre", norm_type="instance",
                                     body_norm="global_layer", cssm_type="gated", gate_type="factored",
                                     pos_embed="none")])
def test_param_tree_matches_oracle(kw):
    m = SimpleCSSM(embed_dim=12, **kw)
    cfg = O.SimpleConfig(embed_dim=12, **kw)
    assert m.param_shapes((2, 4, 15, 15, 3)) == O.simple_param_shapes(cfg, (2, 4, 15, 15, 3))


def test_rope_position_embeddings_are_outside_the_build():
    with pytest.raises(NotImplementedError):
        SimpleCSSM(cssm_type="gated")          # the reference default pos_embed is RoPE
    with pytest.raises(NotImplementedError):
        SimpleCSSM(cssm_type="hgru_bi", pos_embed="none")


# ----------------------------------------------------------------- oracle pins

def init_simple(shapes, rng):
    """Seeded draws for a SimpleCSSM tree: each cell subtree as a cell, the rest entry by entry."""
    return {k: (O.init_params(v, rng) if k.startswith("cssm_") else O.init_params({k: v}, rng)[k])
            for k, v in shapes.items()}


def _model(rng, **kw):
    cfg = O.SimpleConfig(**kw)
    shapes, bss = O.simple_param_shapes(cfg, (2, 3, 8, 8, 3))
    p = init_simple(shapes, rng)
    bs = {n: {"mean": rng.standard_normal(v["mean"]) * 0.1, "var": 1 + rng.random(v["var"])} for n, v in bss.items()}
    return cfg, p, bs


def _zero_cell(p, i=0):
    p[f"cssm_{i}"]["out_proj"] = {"kernel": np.zeros_like(p[f"cssm_{i}"]["out_proj"]["kernel"]),
                                  "bias": np.zeros_like(p[f"cssm_{i}"]["out_proj"]["bias"])}


def test_oracle_image_is_repeated_to_seq_len():
    rng = np.random.default_rng(0)
    cfg, p, bs = _model(rng, embed_dim=8, cssm_type="gated", kernel_size=3, stem_mode="pathtracker", seq_len=3,
                        gate_type="factored", short_conv_size=2, short_conv_spatial_size=0)
    img = rng.standard_normal((2, 8, 8, 3))
    a = O.simple_cssm_forward(p, img, cfg)
    b = O.simple_cssm_forward(p, np.repeat(img[:, None], 3, axis=1), cfg)
    assert np.array_equal(a, b)


def test_oracle_residual_and_registers():
    """With the cell's out_proj zeroed the cell adds exactly 0: the features after the block are the
    stem output (+ position embedding), with the register tokens in front."""
    rng = np.random.default_rng(1)
    cfg, p, bs = _model(rng, embed_dim=8, cssm_type="gated", kernel_size=3, stem_mode="default", stem_layers=1,
                        n_register_tokens=2, pos_embed="learnable", gate_type="factored")
    _zero_cell(p)
    x = rng.standard_normal((2, 3, 8, 8, 3))
    f = O.simple_cssm_forward(p, x, cfg, return_features=True)
    assert f.shape == (2, 5, 4, 4, 8)
    assert np.array_equal(f[:, :2], np.broadcast_to(p["register_tokens"], (2, 2, 4, 4, 8)))
    stem = O.flax_layer_norm(O.softplus(O.conv2d_same(x.reshape(6, 8, 8, 3), p["conv1"])), p["norm1"])
    stem = O.max_pool_2x2_same(stem).reshape(2, 3, 4, 4, 8) + p["pos_embed"]
    assert np.allclose(f[:, 2:], stem, rtol=0, atol=1e-12)


def test_oracle_max_pool_same_pads_with_minus_inf():
    x = -np.arange(1.0, 50.0).reshape(1, 7, 7, 1)          # all negative: zero padding would show
    y = O.max_pool_2x2_same(x)
    assert y.shape == (1, 4, 4, 1)
    assert y[0, 3, 3, 0] == x[0, 6, 6, 0] and y[0, 0, 0, 0] == x[0, 0, 0, 0] and y[0, 3, 0, 0] == x[0, 6, 0, 0]


@pytest.mark.parametrize("order,expect", [("pre", [-1 / np.sqrt(2), -1 / np.sqrt(2), np.sqrt(2)]),
                                          ("post", [-2 / np.sqrt(14 / 3), -1 / np.sqrt(14 / 3),
                                                    3 / np.sqrt(14 / 3)])])
def test_oracle_readout_order_closed_form(order, expect):
    """Features [1, 2, 6] at every pixel injected after the blocks (simple_cssm.py:500-501), relu,
    unit norms, identity head.  'pre' = norm -> act: [-2, -1, 3] / sd -> [0, 0, +] -> norm_post
    gives [-1, -1, 2] / sqrt 2; 'post' = act -> norm: [1, 2, 6] -> [-2, -1, 3] / sqrt(14 / 3),
    which norm_post keeps.  Both frame readouts and pools see the same constant features."""
    rng = np.random.default_rng(2)
    for readout, pool in (("last", "mean"), ("all", "max")):
        cfg, p, _ = _model(rng, embed_dim=3, num_classes=3, cssm_type="gated", kernel_size=3,
                           stem_mode="pathtracker", act_type="relu", readout_norm=order, frame_readout=readout,
                           pool_type=pool, gate_type="factored")
        for n in ("norm_pre", "norm_post"):
            p[n] = {"scale": np.ones(3), "bias": np.zeros(3)}
        p["head"] = {"kernel": np.eye(3), "bias": np.zeros(3)}
        feat = np.broadcast_to(np.array([1.0, 2.0, 6.0]), (2, 3, 4, 4, 3)).copy()
        out = O.simple_cssm_forward(p, np.zeros((2, 3, 8, 8, 3)), cfg, injected_post_cssm=feat)
        assert np.allclose(out, np.broadcast_to(expect, (2, 3)), rtol=0, atol=1e-5)


def test_instance_norm_on_pooled_vector_is_the_bias():
    """nn.GroupNorm(num_groups=C) (simple_cssm.py:212-214) on a pooled (B, C) vector: flax reduces
    over axes 1..ndim-2 (none here) and the size-1 within-group axis, so each group is one element
    (mean = x, var = 0) and the output is the bias alone.  On (B, H, W, C) it normalises each
    channel over H, W.  Both the oracle and the module's norm follow that."""
    rng = np.random.default_rng(5)
    C = 6
    p = {"scale": rng.standard_normal(C) + 2.0, "bias": rng.standard_normal(C)}
    x2 = rng.standard_normal((3, C)) * 4.0
    assert np.array_equal(O.simple_norm(x2, "instance", p), np.broadcast_to(p["bias"], (3, C)))
    x4 = rng.standard_normal((2, 5, 5, C))
    mu = x4.mean(axis=(1, 2), keepdims=True)
    sd = np.sqrt(x4.var(axis=(1, 2), keepdims=True) + 1e-6)
    assert np.allclose(O.simple_norm(x4, "instance", p), (x4 - mu) / sd * p["scale"] + p["bias"], atol=1e-12)
    m = SimpleCSSM(cssm_type="gated", embed_dim=C, pos_embed="none", body_norm="instance")
    pt = {"n": {k: torch.from_numpy(v) for k, v in p.items()}}
    for x in (x2, x4):
        got = m._norm(torch.from_numpy(x), "instance", "n", pt, None, False).numpy()
        assert np.allclose(got, O.simple_norm(x, "instance", p), rtol=0, atol=1e-12)
