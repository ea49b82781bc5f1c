"""The plugin table under the reference's names (simple_cssm.py:21-60) and the
delta_key_dim rule of its cell construction (simple_cssm.py:408-436).  CPU only:
constructing a cell allocates nothing."""
import pytest

pytest.importorskip("torch")
from cssm_amd import registry  # noqa: E402
from cssm_amd.cells import GatedCSSM, GatedDeltaNetCSSM  # noqa: E402


def test_registry_names_map_to_cells():
    assert registry.CSSM_REGISTRY["gated"] is GatedCSSM
    for name in ("gdn", "gdn_d2", "gdn_d3"):
        assert registry.CSSM_REGISTRY[name] is GatedDeltaNetCSSM


@pytest.mark.parametrize("name,dk_arg,dk", [("gdn_d2", 4, 2), ("gdn_d3", 4, 3), ("gdn", 4, 4), ("gdn", None, 2)])
def test_make_cell_delta_key_dim_rule(name, dk_arg, dk):
    """gdn_d2 / gdn_d3 force delta_key_dim 2 / 3 whatever is passed; plain gdn keeps the
    caller's value (the reference's CLI default is 2, the cell's own default)."""
    kw = dict(channels=12)
    if dk_arg is not None:
        kw["delta_key_dim"] = dk_arg
    cell = registry.make_cell(name, **kw)
    assert isinstance(cell, GatedDeltaNetCSSM) and cell.delta_key_dim == dk


def test_make_cell_gated_passes_kwargs():
    cell = registry.make_cell("gated", channels=16, kernel_size=11, gate_type="factored", short_conv_size=0)
    assert isinstance(cell, GatedCSSM)
    assert (cell.channels, cell.kernel_size, cell.gate_type, cell.short_conv_size) == (16, 11, "factored", 0)


def test_make_cell_rejects_cells_outside_the_build():
    with pytest.raises(KeyError):
        registry.make_cell("hgru_bi", channels=8)
    with pytest.raises(NotImplementedError):
        registry.make_cell("gdn", channels=8, int_attention_mode="spectral")
