"""CPU checks of the C ABI: the library loads and exports every declared symbol."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "cssm_amd.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(cssm_\w+)\s*\(", text)))


def test_header_declares_entry_points():
    names = _declared()
    assert "cssm_gated_scan_fwd" in names and "cssm_abi_version" in names


def test_library_exports_every_declared_symbol():
    from cssm_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail("libcssm_hip.so is not built (run python -m cssm_amd.build)")
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in _declared() if not hasattr(lib, n)]
    assert not missing, missing
    assert set(_declared()) <= set(_lib.SIGNATURES), "ctypes signatures missing for some symbols"


def test_abi_version_and_errors_without_gpu():
    from cssm_amd import _lib
    lib = _lib.load()
    assert lib.cssm_abi_version() == 2
    assert lib.cssm_strerror(-1) == b"null pointer argument"
    # argument validation happens before any GPU work
    st = lib.cssm_gated_scan_fwd(None, None, None, 0, 1, 1, 1, 8, 8, None, None, 0, 0, None)
    assert st == -1
    assert b"non-null" in lib.cssm_last_error()
    buf = ctypes.create_string_buffer(64)
    p = ctypes.addressof(buf)
    st = lib.cssm_gated_scan_fwd(p, p, p, 0, 1, 1, 32, 24, 24, p, p, 0, 0, None)
    assert st == -3 and b"no fused kernel" in lib.cssm_last_error()
    st = lib.cssm_gated_scan_fwd(p, p, p, 7, 1, 1, 32, 8, 8, p, p, 0, 0, None)
    assert st == -4
    st = lib.cssm_gated_scan_fwd(p + 4, p, p, 0, 1, 1, 32, 8, 8, p, p, 0, 0, None)
    assert st == -5
    st = lib.cssm_gated_scan_fwd(p, p, p, 0, 1, 1, 4, 16, 16, p, p, 0, 0, None)
    assert st == -3 and b"multiple of 8" in lib.cssm_last_error()
    st = lib.cssm_gated_scan_fwd(p, p, p, 0, 1, 1, 32, 8, 8, p, p, 2, 0, None)
    assert st == -4
    st = lib.cssm_spectral_kernel(p, 1, 11, 8, 16, 0.9, 1, 1, 0, p, None)
    assert st == -2


@pytest.mark.parametrize("H", [4, 8, 14, 32, 64, 128])
def test_scan_col_order(H):
    """The per-bin planes' column order (host-side, no GPU): a permutation of the
    W/2 + 1 columns that keeps DC and Nyquist in place; at 128 x 128 each group of
    eight positions (one wave's columns) covers four consecutive row blocks of 16
    columns at two pair positions, and the identity elsewhere."""
    from cssm_amd import spectral
    cols = spectral.scan_col_order(H, H)
    Wf = H // 2 + 1
    assert sorted(cols) == list(range(Wf))
    assert cols[0] == 0 and cols[-1] == H // 2
    if H != 128:
        assert cols == list(range(Wf))
        return
    for g in range(8):
        grp = cols[8 * g:8 * g + 8]
        blocks = sorted({v % 16 for v in grp})
        pairs = sorted({v // 16 for v in grp})
        assert blocks == list(range(blocks[0], blocks[0] + 4)) and len(pairs) == 2
        assert len({(v % 16, v // 16) for v in grp}) == 8
