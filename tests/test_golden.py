"""The float64 oracle reproduces the committed golden vectors (tests/golden/*.npz).

The fixtures were written by tests/golden/make_golden.py from the same oracle;
this test pins the oracle against later regressions (a changed formula, sign
or index fails here before it can move the GPU parity target).
"""
import glob
import json
import os

import numpy as np
import pytest

from oracle import cssm_oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURES = sorted(glob.glob(os.path.join(HERE, "golden", "*.npz")))


def load(path):
    from tests.golden.make_golden import unflatten
    z = np.load(path, allow_pickle=False)
    cfg = json.loads(str(z["config"]))
    return cfg, unflatten(z), np.asarray(z["x"], dtype=np.float64), np.asarray(z["y"])


def test_fixtures_present():
    assert len(FIXTURES) >= 7


@pytest.mark.parametrize("path", FIXTURES, ids=[os.path.basename(p)[:-4] for p in FIXTURES])
def test_oracle_reproduces_golden(path):
    cfg, params, x, y = load(path)
    kw = cfg["kwargs"]
    if cfg["cell"] == "gated":
        got = O.gated_forward(params, x, O.GatedConfig(**kw))
    else:
        got = O.gdn_forward(params, x, O.GDNConfig(**kw))
    assert got.shape == y.shape
    assert np.max(np.abs(got - y)) <= 1e-10 * np.sqrt(np.mean(y ** 2))
