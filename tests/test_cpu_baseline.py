"""The fp32 torch-CPU restatement that bench.py times as the CPU baseline
(oracle/cssm_cpu_fp32.py) agrees with the float64 oracle at the fp32 bar."""
import numpy as np
import pytest

from oracle import cssm_oracle as O

torch = pytest.importorskip("torch")
from oracle import cssm_cpu_fp32 as P  # noqa: E402


def _rel(a, b):
    return float(np.max(np.abs(a - b)) / np.sqrt(np.mean(b ** 2)))


@pytest.mark.parametrize("gate_type,H,T,expand,K,convs", [("factored", 16, 4, 1, 11, False),
                                                          ("dense", 8, 3, 2, 5, True),
                                                          ("factored", 7, 1, 2, 1, False)])
def test_gated_cpu_fp32_matches_oracle(gate_type, H, T, expand, K, convs):
    rng = np.random.default_rng(0)
    C = 8
    kw = dict(channels=C, expand=expand, kernel_size=K, gate_type=gate_type,
              short_conv_size=4 if convs else 0, short_conv_spatial_size=3 if convs else 0)
    cfg = O.GatedConfig(**kw)
    p = O.init_params(O.gated_param_shapes(cfg, C, H, H), rng)
    x = rng.standard_normal((2, T, H, H, C))
    ref = O.gated_forward(p, x, cfg)
    got = P.GatedCPU(p, **kw)(torch.from_numpy(x).float()).double().numpy()
    assert _rel(got, ref) < 1e-4


@pytest.mark.parametrize("H,T,qkv", [(16, 4, 5), (8, 6, 1)])
def test_gdn_cpu_fp32_matches_oracle(H, T, qkv):
    rng = np.random.default_rng(1)
    C, dk = 16, 4
    cfg = O.GDNConfig(channels=C, delta_key_dim=dk, gate_type="factored", qkv_conv_size=qkv)
    p = O.init_params(O.gdn_param_shapes(cfg, H, H), rng, spectral_init="xavier")
    x = rng.standard_normal((2, T, H, H, C))
    ref = O.gdn_forward(p, x, cfg)
    got = P.GdnCPU(p, C, dk, qkv_conv_size=qkv)(torch.from_numpy(x).float()).double().numpy()
    assert _rel(got, ref) < 1e-4
