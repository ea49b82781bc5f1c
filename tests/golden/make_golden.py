"""Write the golden-vector fixtures of the spectral layer (tests/golden/*.npz).

The reference (drewlinsley/CSSM) ships no golden vectors for this path and
cannot run here (no JAX), so these fixtures are the float64 oracle's outputs
(oracle/cssm_oracle.py) on seeded inputs and parameter trees drawn with the
reference's init distributions.  They pin the oracle against regressions
(tests/test_golden.py) and give the GPU tests fixed vectors
(tests/test_gpu_golden.py).  Shapes are small versions of the BASELINE
configs.  Regenerate with ``python tests/golden/make_golden.py``.

Each file holds x, y (float64), the flattened parameter tree under
'params/<path>', and a JSON 'config' string (cell kind + constructor kwargs).
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from oracle import cssm_oracle as O  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))

CASES = [
    # name, cell, input shape (B, T, H, W, C), constructor kwargs, input kind
    ("gated_c1_small", "gated", (2, 1, 32, 32, 16),
     dict(channels=16, expand=2, kernel_size=1, gate_type="factored", short_conv_size=0, short_conv_spatial_size=0),
     "normal"),
    ("gated_c2_small", "gated", (2, 4, 32, 32, 8),
     dict(channels=8, kernel_size=11, gate_type="factored", short_conv_size=0, short_conv_spatial_size=0),
     "repeat"),
    ("gated_dense_convs", "gated", (1, 4, 16, 16, 8),
     dict(channels=8, kernel_size=11, gate_type="dense", short_conv_size=4, short_conv_spatial_size=3),
     "normal"),
    ("gated_c5_14", "gated", (2, 1, 14, 14, 16),
     dict(channels=16, expand=2, kernel_size=1, gate_type="factored", short_conv_size=0, short_conv_spatial_size=0),
     "normal"),
    ("gdn_c3_small", "gdn", (1, 3, 16, 16, 8),
     dict(channels=8, delta_key_dim=4, kernel_size=11, gate_type="factored", qkv_conv_size=5), "normal"),
    ("gdn_c4_small", "gdn", (2, 8, 16, 16, 8),
     dict(channels=8, delta_key_dim=4, kernel_size=11, gate_type="factored"), "dots"),
    ("gdn_channel_d2", "gdn", (1, 4, 8, 8, 8),
     dict(channels=8, delta_key_dim=2, kernel_size=5, gate_type="channel"), "normal"),
]


def flatten(tree, prefix="params"):
    out = {}
    for k, v in tree.items():
        if isinstance(v, dict):
            out.update(flatten(v, f"{prefix}/{k}"))
        else:
            out[f"{prefix}/{k}"] = np.asarray(v, dtype=np.float32)
    return out


def unflatten(npz):
    tree = {}
    for key in npz.files:
        if not key.startswith("params/"):
            continue
        parts = key.split("/")[1:]
        node = tree
        for p in parts[:-1]:
            node = node.setdefault(p, {})
        node[parts[-1]] = np.asarray(npz[key], dtype=np.float64)
    return tree


def make_input(rng, shape, kind):
    B, T, H, W, C = shape
    if kind == "repeat":
        return np.repeat(rng.standard_normal((B, 1, H, W, C)), T, axis=1)
    if kind == "dots":
        x = rng.standard_normal(shape) * 0.01
        x[rng.random(shape[:4]) < 0.02] = 1.0
        return x
    return rng.standard_normal(shape)


def forward(cell, params, x, kw):
    if cell == "gated":
        return O.gated_forward(params, x, O.GatedConfig(**kw))
    return O.gdn_forward(params, x, O.GDNConfig(**kw))


def build_case(name, cell, shape, kw, kind, seed):
    rng = np.random.default_rng(seed)
    B, T, H, W, C = shape
    if cell == "gated":
        shapes = O.gated_param_shapes(O.GatedConfig(**kw), C, H, W)
        params = O.init_params(shapes, rng)
    else:
        shapes = O.gdn_param_shapes(O.GDNConfig(**kw), H, W)
        params = O.init_params(shapes, rng, spectral_init="xavier")
    # parameters and inputs are stored (and used) at float32 precision
    params = {k: ({kk: np.float32(vv).astype(np.float64) for kk, vv in v.items()} if isinstance(v, dict)
                  else np.float32(v).astype(np.float64)) for k, v in params.items()}
    x = make_input(rng, shape, kind).astype(np.float32).astype(np.float64)
    y = forward(cell, params, x, kw)
    return dict(x=x.astype(np.float32), y=y, config=json.dumps({"cell": cell, "kwargs": kw}), **flatten(params))


def main():
    for i, (name, cell, shape, kw, kind) in enumerate(CASES):
        data = build_case(name, cell, shape, kw, kind, 100 + i)
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **data)
        print(f"{path}: x {data['x'].shape} y rms {np.sqrt(np.mean(data['y'] ** 2)):.4g}")


if __name__ == "__main__":
    main()
