"""GPU parity of the SimpleCSSM wrapper (stem -> cells + residual -> readout) against
the float64 oracle restatement (simple_cssm.py:166-558), through the HIP cells."""
import numpy as np
import pytest

from oracle import cssm_oracle as O
from tests.gpu_util import print_case, rel_err, to_np
from tests.test_simple_cssm import init_simple

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

TOL_F32 = 1e-4


@pytest.fixture(scope="module")
def simple():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from cssm_amd.simple_cssm import SimpleCSSM
    return SimpleCSSM


CASES = [
    # name, x shape, kwargs, apply kwargs
    ("bench_pathtracker_gated_image", (2, 16, 16, 3),
     dict(num_classes=1, embed_dim=32, depth=1, cssm_type="gated", kernel_size=11, seq_len=4, frame_readout="last",
          pos_embed="none", stem_mode="pathtracker", stem_layers=0, norm_type="layer"), {}),
    ("stem2_batchnorm_gdn_d3_depth2_mlp_registers", (2, 3, 32, 32, 3),
     dict(num_classes=5, embed_dim=12, depth=2, cssm_type="gdn_d3", kernel_size=5, stem_mode="default",
          stem_layers=2, norm_type="batch", inter_mlp_ratio=2.0, n_register_tokens=2, pos_embed="learnable",
          frame_readout="all", pool_type="max", readout_norm="post", act_type="gelu", gate_type="factored"), {}),
    ("pre_order_instance_global_layer_spatial", (1, 3, 16, 16, 4),
     dict(num_classes=3, embed_dim=16, depth=2, cssm_type="gated", kernel_size=5, stem_mode="pathtracker",
          stem_norm_order="pre", stem_norm="instance", body_norm="global_layer", pos_embed="none",
          gate_type="factored", act_type="relu"), dict(return_spatial=True)),
    ("temporal_layer_gdn_features", (2, 4, 16, 16, 3),
     dict(num_classes=2, embed_dim=8, depth=2, cssm_type="gdn", delta_key_dim=2, kernel_size=3,
          stem_mode="default", stem_layers=1, norm_type="temporal_layer", pos_embed="none", gate_type="factored"),
     dict(return_features=True)),
    ("global_instance_gated_batch_training", (2, 2, 16, 16, 3),
     dict(num_classes=2, embed_dim=16, depth=2, cssm_type="gated", kernel_size=3, stem_mode="pathtracker",
          stem_norm="batch", body_norm="global_instance", pos_embed="none", gate_type="dense",
          short_conv_size=2, short_conv_spatial_size=3), dict(training=True)),
]


@pytest.mark.parametrize("name,shape,kw,call", CASES, ids=[c[0] for c in CASES])
def test_simple_cssm_matches_oracle(simple, name, shape, kw, call):
    print_case(test="simple_cssm", case=name)
    rng = np.random.default_rng(5)
    model = simple(**kw)
    cfg = O.SimpleConfig(**{k: v for k, v in kw.items()})
    shapes, bss = O.simple_param_shapes(cfg, shape)
    p = init_simple(shapes, rng)
    bs = {n: {"mean": rng.standard_normal(v["mean"]) * 0.1, "var": 1 + rng.random(v["var"])} for n, v in bss.items()}
    x = rng.standard_normal(shape)
    ref = O.simple_cssm_forward(p, x, cfg, batch_stats=bs, **call)
    v = simple.load_params({"params": p, "batch_stats": bs})
    y = model.apply(v, torch.from_numpy(x).to("cuda", torch.float32), **call)
    torch.cuda.synchronize()
    assert tuple(y.shape) == ref.shape
    assert rel_err(to_np(y), ref) <= TOL_F32


def test_simple_cssm_from_checkpoint_file(simple, tmp_path):
    """A SimpleCheckpointer-format pickle (written here) read by the weights-only loader runs
    the model with the same result as the in-memory parameters."""
    import pickle
    from cssm_amd import checkpoint as ck
    kw = CASES[0][2]
    rng = np.random.default_rng(6)
    cfg = O.SimpleConfig(**kw)
    p = init_simple(O.simple_param_shapes(cfg, (2, 16, 16, 3))[0], rng)
    (tmp_path / "checkpoint.pkl").write_bytes(pickle.dumps({"params": p, "epoch": 3, "step": 10}))
    x = rng.standard_normal((2, 16, 16, 3))
    model = simple(**kw)
    y = model.apply(simple.load_params(ck.load_simple_checkpoint(str(tmp_path))),
                    torch.from_numpy(x).to("cuda", torch.float32))
    assert rel_err(to_np(y), O.simple_cssm_forward(p, x, cfg)) <= TOL_F32
