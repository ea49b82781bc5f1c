"""The weights-only reader of SimpleCheckpointer pickles (main.py:70-142): files the
test writes in the reference's format (numpy trees inside flax FrozenDicts, epoch,
step, training_args, batch_stats) load to plain dicts of the same arrays; a file
naming any other global is refused without running it.  CPU only."""
import os
import pickle
import sys
import types
from collections.abc import Mapping

import numpy as np
import pytest

from cssm_amd import checkpoint as ck


def _fake_flax(monkeypatch, with_reduce):
    """A stand-in flax.core.frozen_dict module, so the test can write what the reference writes."""
    mod = types.ModuleType("flax.core.frozen_dict")

    class FrozenDict(Mapping):
        def __init__(self, *a, **k):
            self._dict = dict(*a, **k)
            self._hash = None

        def __getitem__(self, k):
            return self._dict[k]

        def __iter__(self):
            return iter(self._dict)

        def __len__(self):
            return len(self._dict)

        if with_reduce:
            def __reduce__(self):
                return FrozenDict, (dict(self._dict),)
    FrozenDict.__module__ = "flax.core.frozen_dict"
    FrozenDict.__qualname__ = "FrozenDict"
    mod.FrozenDict = FrozenDict
    flax = types.ModuleType("flax")
    core = types.ModuleType("flax.core")
    flax.core, core.frozen_dict = core, mod
    monkeypatch.setitem(sys.modules, "flax", flax)
    monkeypatch.setitem(sys.modules, "flax.core", core)
    monkeypatch.setitem(sys.modules, "flax.core.frozen_dict", mod)
    return FrozenDict


def _reference_like(FD, rng):
    cell = {"in_proj": FD({"kernel": rng.standard_normal((4, 8)).astype(np.float32),
                           "bias": np.zeros(8, np.float32)}),
            "kernel": rng.standard_normal((4, 3, 3)).astype(np.float32)}
    params = FD({"conv1": FD({"kernel": rng.standard_normal((1, 1, 3, 4)).astype(np.float32),
                              "bias": np.zeros(4, np.float32)}),
                 "cssm_0": FD(cell),
                 "head": FD({"kernel": rng.standard_normal((4, 2)), "bias": np.arange(2, dtype=np.int64)})})
    return {"params": params, "epoch": 7, "step": np.int64(1234),
            "training_args": {"lr": 1e-3, "cssm": "gated", "depth": 1, "tags": ["a", "b"], "seed": None},
            "batch_stats": FD({"norm1": FD({"mean": np.float32(0.5) * np.ones(4, np.float32),
                                            "var": np.ones(4, np.float32)})})}


def _eq_tree(a, b):
    if isinstance(b, Mapping):
        assert isinstance(a, dict) and not isinstance(a, Mapping.__class__)
        assert set(a) == set(b)
        for k in b:
            _eq_tree(a[k], b[k])
    elif isinstance(b, np.ndarray):
        assert isinstance(a, np.ndarray) and a.dtype == b.dtype and np.array_equal(a, b)
    else:
        assert a == b


@pytest.mark.parametrize("with_reduce", [True, False])
@pytest.mark.parametrize("protocol", [0, 2, pickle.HIGHEST_PROTOCOL])
def test_reads_reference_format(tmp_path, monkeypatch, with_reduce, protocol):
    FD = _fake_flax(monkeypatch, with_reduce)
    ref = _reference_like(FD, np.random.default_rng(0))
    d = tmp_path / "ckpt"
    d.mkdir()
    with open(d / "checkpoint.pkl", "wb") as f:
        pickle.dump(ref, f, protocol=protocol)
    for mod in ("flax", "flax.core", "flax.core.frozen_dict"):     # the reader needs no flax
        monkeypatch.delitem(sys.modules, mod)
    got = ck.load_simple_checkpoint(str(d))
    assert type(got["params"]) is dict and type(got["params"]["cssm_0"]["in_proj"]) is dict
    _eq_tree(got["params"], ref["params"])
    _eq_tree(got["batch_stats"], ref["batch_stats"])
    assert got["epoch"] == 7 and got["step"] == 1234 and got["training_args"]["tags"] == ["a", "b"]
    # the block's cell parameters load straight into a cell
    cell = ck.cell_params(got, 0)
    from cssm_amd.cells import GatedCSSM
    v = GatedCSSM.load_params(cell, device="cpu")
    assert np.array_equal(v["params"]["in_proj"]["kernel"].numpy(), ref["params"]["cssm_0"]["in_proj"]["kernel"])


class _Evil:
    def __reduce__(self):
        return (os.system, ("echo this must never run",))


def test_refuses_other_globals(tmp_path):
    data = pickle.dumps({"params": {"w": np.ones(2)}, "x": _Evil()})
    with pytest.raises(pickle.UnpicklingError, match="system"):
        ck.loads(data)
    data = pickle.dumps({"params": {"f": np.add}})
    with pytest.raises(pickle.UnpicklingError):
        ck.loads(data)


def test_rejects_files_without_params(tmp_path):
    p = tmp_path / "c.pkl"
    p.write_bytes(pickle.dumps({"epoch": 1}))
    with pytest.raises(ValueError):
        ck.load_simple_checkpoint(str(p))
