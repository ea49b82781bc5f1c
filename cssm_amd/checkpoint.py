"""Weights-only reader for the reference's SimpleCheckpointer files.

The reference saves ``checkpoint.pkl`` with ``pickle.dump`` of
``{'params', 'epoch', 'step'[, 'training_args'][, 'batch_stats']}``, the
parameter trees as numpy arrays, possibly inside flax ``FrozenDict``s
(main.py:70-116; restored by ``SimpleCheckpointer.restore``, main.py:118-142).

A pickle can name any callable, so this reader never runs ``pickle.load``
with the default class lookup.  Its unpickler admits only what such a file
holds: numpy arrays, dtypes and scalars (rebuilt by numpy's own
reconstructors) and plain containers; a ``FrozenDict`` becomes a ``dict``.
Any other global in the file raises ``pickle.UnpicklingError`` before it is
looked up, so nothing in the file is executed.

orbax checkpoints (the 'pytree' / 'standard' checkpointers, main.py:1181-1200)
need tensorstore and are not read here.
"""
from __future__ import annotations

import io
import os
import pickle
from typing import Any, Dict

import numpy as np


class _FrozenDictStandIn(dict):
    """What a flax FrozenDict unpickles to: its items as a plain dict.

    FrozenDict pickles either through its ``__reduce__`` (``FrozenDict(d)``) or
    as a plain object whose state holds ``_dict``; both land here.
    """

    def __init__(self, *args, **kwargs):
        super().__init__()
        if args or kwargs:
            self.update(dict(*args, **kwargs))

    def __setstate__(self, state):
        if isinstance(state, tuple) and len(state) == 2:      # (dict state, slot state)
            state = state[0] or state[1]
        if isinstance(state, dict):
            inner = state.get("_dict", state)
            self.update(inner)


def _rebuild_object(cls, base, state):
    """copyreg._reconstructor for the stand-in only (objects pickled without __reduce__)."""
    if cls is not _FrozenDictStandIn:
        raise pickle.UnpicklingError(f"refusing to rebuild {cls!r}")
    obj = _FrozenDictStandIn()
    if state is not None:
        obj.__setstate__(state)
    return obj


def _latin1_bytes(text, encoding="latin1"):
    """_codecs.encode as protocol 0-2 pickles use it for bytes (numpy's raw array data)."""
    if not isinstance(text, str) or encoding.lower().replace("_", "-") not in ("latin1", "latin-1"):
        raise pickle.UnpicklingError(f"refusing _codecs.encode(..., {encoding!r})")
    return text.encode("latin1")


def _numpy_reconstruct():
    try:
        from numpy._core.multiarray import _reconstruct, scalar   # numpy >= 2
        from numpy._core.numeric import _frombuffer
    except ImportError:                                          # pragma: no cover - numpy 1.x
        from numpy.core.multiarray import _reconstruct, scalar
        from numpy.core.numeric import _frombuffer
    return _reconstruct, scalar, _frombuffer


_RECONSTRUCT, _SCALAR, _FROMBUFFER = _numpy_reconstruct()

# (module, name) -> object: everything a SimpleCheckpointer file may name
_ALLOWED = {
    ("numpy.core.multiarray", "_reconstruct"): _RECONSTRUCT,
    ("numpy._core.multiarray", "_reconstruct"): _RECONSTRUCT,
    ("numpy.core.multiarray", "scalar"): _SCALAR,
    ("numpy._core.multiarray", "scalar"): _SCALAR,
    ("numpy.core.numeric", "_frombuffer"): _FROMBUFFER,      # protocol 5 out-of-band arrays
    ("numpy._core.numeric", "_frombuffer"): _FROMBUFFER,
    ("numpy", "ndarray"): np.ndarray,
    ("numpy", "dtype"): np.dtype,
    ("flax.core.frozen_dict", "FrozenDict"): _FrozenDictStandIn,
    ("flax.core", "FrozenDict"): _FrozenDictStandIn,
    ("copyreg", "_reconstructor"): _rebuild_object,
    ("_codecs", "encode"): _latin1_bytes,
    ("builtins", "object"): object,
    # the Python 2 names protocol 0 and 1 files carry for the same two
    ("copy_reg", "_reconstructor"): _rebuild_object,
    ("__builtin__", "object"): object,
}


class _WeightsOnlyUnpickler(pickle.Unpickler):
    def find_class(self, module, name):
        obj = _ALLOWED.get((module, name))
        if obj is None and module.startswith("numpy.dtypes") and name.endswith("DType"):
            obj = np.dtype                     # numpy 2 dtype classes: rebuilt through np.dtype
        if obj is None:
            raise pickle.UnpicklingError(f"checkpoint names {module}.{name}, which a weights file does not hold")
        return obj


def _plain(tree):
    """Stand-ins to dicts, all the way down."""
    if isinstance(tree, dict):
        return {k: _plain(v) for k, v in tree.items()}
    if isinstance(tree, (list, tuple)):
        return type(tree)(_plain(v) for v in tree)
    return tree


def loads(data: bytes) -> Dict[str, Any]:
    """Decode the bytes of a SimpleCheckpointer pickle without executing anything in it."""
    return _plain(_WeightsOnlyUnpickler(io.BytesIO(data)).load())


def load_simple_checkpoint(path: str) -> Dict[str, Any]:
    """Read ``<path>/checkpoint.pkl`` (or ``path`` itself if it is a file) as the reference's
    SimpleCheckpointer wrote it: returns ``{'params', 'epoch', 'step', ...}`` with numpy arrays
    and plain dicts, ready for ``Model.load_params``."""
    f = os.path.join(path, "checkpoint.pkl") if os.path.isdir(path) else path
    with open(f, "rb") as fh:
        ckpt = loads(fh.read())
    if not isinstance(ckpt, dict) or "params" not in ckpt:
        raise ValueError(f"{f} is not a SimpleCheckpointer file (no 'params')")
    return ckpt


def cell_params(ckpt: Dict[str, Any], index: int = 0) -> Dict[str, Any]:
    """The parameters of SimpleCSSM's block ``index`` (the Flax submodule ``cssm_<index>``),
    as a cell's ``{'params': ...}`` tree."""
    return {"params": ckpt["params"][f"cssm_{index}"]}
