"""Plugin table of the cells this build provides, under the reference's names.

Mirrors the hot-path entries of ``CSSM_REGISTRY`` (src/models/simple_cssm.py:23-60):
``'gated'`` -> GatedCSSM and ``'gdn'`` / ``'gdn_d2'`` / ``'gdn_d3'`` ->
GatedDeltaNetCSSM.  The reference's wrapper sets ``delta_key_dim`` from the
name (simple_cssm.py:432-443); :func:`make_cell` does the same.  The other
reference cells are not part of this build and raise KeyError.
"""
from __future__ import annotations

from .cells import GatedCSSM, GatedDeltaNetCSSM

CSSM_REGISTRY = {
    "gated": GatedCSSM,
    "gdn": GatedDeltaNetCSSM,
    "gdn_d2": GatedDeltaNetCSSM,
    "gdn_d3": GatedDeltaNetCSSM,
}

_DELTA_KEY_DIM = {"gdn_d2": 2, "gdn_d3": 3}


def make_cell(cssm_type: str, **kwargs):
    """Construct a cell by registry name, as SimpleCSSM does (simple_cssm.py:324-443)."""
    if cssm_type not in CSSM_REGISTRY:
        raise KeyError(f"cssm type {cssm_type!r} is not part of this build (have {sorted(CSSM_REGISTRY)})")
    if cssm_type in _DELTA_KEY_DIM:
        kwargs["delta_key_dim"] = _DELTA_KEY_DIM[cssm_type]
    return CSSM_REGISTRY[cssm_type](**kwargs)
