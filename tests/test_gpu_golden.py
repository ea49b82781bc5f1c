"""The HIP layer (through the C ABI) against the committed golden vectors.

Bar: max|y_gpu - y_ref| / RMS(y_ref) <= 1e-4, fp32 I/O.
"""
import glob
import json
import os

import numpy as np
import pytest

from tests.gpu_util import print_case, rel_err, to_np

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURES = sorted(glob.glob(os.path.join(HERE, "golden", "*.npz")))


@pytest.mark.parametrize("path", FIXTURES, ids=[os.path.basename(p)[:-4] for p in FIXTURES])
def test_layer_matches_golden(path):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from cssm_amd import cells
    from tests.golden.make_golden import unflatten
    name = os.path.basename(path)[:-4]
    print_case(test="golden", case=name)
    z = np.load(path, allow_pickle=False)
    cfg = json.loads(str(z["config"]))
    cls = cells.GatedCSSM if cfg["cell"] == "gated" else cells.GatedDeltaNetCSSM
    cell = cls(**cfg["kwargs"])
    variables = cls.load_params(unflatten(z))
    x = torch.from_numpy(np.asarray(z["x"])).to("cuda", torch.float32)
    y = cell.apply(variables, x)
    torch.cuda.synchronize()
    assert rel_err(to_np(y), np.asarray(z["y"])) <= 1e-4
