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
    assert lib.cssm_abi_version() == _lib.ABI_VERSION == 8
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
    # the GDN scan variant (cssm_gdn_scan_variant) is checked before any device work
    for v in (-1, 3):
        st = lib.cssm_gdn_scan_bins(p, None, p, 1, 0, 1, p, 1, 2, 8, 8, 8, 4, v, p, None)
        assert st == -4 and b"scan_variant" in lib.cssm_last_error()
        st = lib.cssm_gdn_core_fused(p, 1, p, 1, 0, 1, p, 1, 2, 8, 32, 32, 4, v, p, None)
        assert st == -4 and b"scan_variant" in lib.cssm_last_error()
        st = lib.cssm_gdn_scan_bins_train(p, p, 1, 0, 1, p, 1, 2, 8, 8, 8, 4, v, p, p, None)
        assert st == -4 and b"scan_variant" in lib.cssm_last_error()
        st = lib.cssm_gdn_scan_bins_bwd(p, p, 1, 0, 1, p, p, p, 1, 2, 8, 8, 8, 4, v, p, p, p, None)
        assert st == -4 and b"scan_variant" in lib.cssm_last_error()
    # the output projection with the computed gate: widths, gate activation and alignment checked first
    assert lib.cssm_gdn_proj_out_xgate_supported(64, 64, 1024) == 1
    assert lib.cssm_gdn_proj_out_xgate_supported(72, 64, 1024) == 0       # K > 64
    assert lib.cssm_gdn_proj_out_xgate_supported(60, 60, 1024) == 0       # K % 8
    assert lib.cssm_gdn_proj_out_xgate_supported(64, 128, 1024) == 0      # N > 64
    assert lib.cssm_gdn_proj_out_xgate_supported(64, 64, 49) == 0         # H W % 4
    st = lib.cssm_gdn_proj_out_xgate(p, 0, p, 1, 2, 1024, 72, 64, 1, None, None, p, p, 1, p, p, p, 1, None)
    assert st == -3 and b"K <= 64" in lib.cssm_last_error()
    st = lib.cssm_gdn_proj_out_xgate(p, 0, p, 1, 2, 1024, 64, 64, 1, None, None, p, p, 0, p, p, p, 1, None)
    assert st == -4 and b"gate_act" in lib.cssm_last_error()
    st = lib.cssm_gdn_proj_out_xgate(p, 0, p + 8, 1, 2, 1024, 64, 64, 1, None, None, p, p, 1, p, p, p, 1, None)
    assert st == -5
    st = lib.cssm_gdn_proj_out_xgate(p, 0, None, 1, 2, 1024, 64, 64, 1, None, None, p, p, 1, p, p, p, 1, None)
    assert st == -1
    st = lib.cssm_gdn_proj_out_xgate(p, 0, p, 5, 2, 1024, 64, 64, 1, None, None, p, p, 1, p, p, p, 1, None)
    assert st == -4 and b"dtypes" in lib.cssm_last_error()
    # the gates' adjoint: pointers, gate type, weights and alignment checked before any GPU work
    gp = _lib.GateParams()
    gp.gate_type, gp.activation = _lib.GATE_FACTORED, _lib.ACT_SOFTPLUS
    for i in range(3):
        gp.kernel[i] = gp.bias[i] = gp.kernel_w[i] = gp.bias_w[i] = p
    st = lib.cssm_gated_gates_bwd(p, 1, 1, 8, 8, 8, ctypes.byref(gp), 1.0, p, None, None)
    assert st == -1 and b"non-null" in lib.cssm_last_error()
    st = lib.cssm_gated_gates_bwd(p, 1, 1, 8, 8, 8, ctypes.byref(gp), 1.0, p + 4, p, None)
    assert st == -5
    st = lib.cssm_gated_gates_bwd(p, 1, 0, 8, 8, 8, ctypes.byref(gp), 1.0, p, p, None)
    assert st == -2
    gp.bias_w[1] = None
    st = lib.cssm_gated_gates_bwd(p, 1, 1, 8, 8, 8, ctypes.byref(gp), 1.0, p, p, None)
    assert st == -1 and b"gate 1" in lib.cssm_last_error()
    gp.gate_type = 7
    st = lib.cssm_gated_gates_bwd(p, 1, 1, 8, 8, 8, ctypes.byref(gp), 1.0, p, p, None)
    assert st == -4 and b"gate_type" in lib.cssm_last_error()
    # in_proj + gates: ctx, params and gates required; then the projection's and the gates' checks
    gp.gate_type, gp.bias_w[1] = _lib.GATE_FACTORED, p
    args = dict(x=p, in_dtype=1, B=2, T=1, H=14, W=14, K=128, N=512, kernel=p, bias=p, lo=p, hi=p, out_dtype=0,
                act_lo=1, act_hi=1, ctx=p, params=ctypes.byref(gp), c_scale=1.0, gates=p, ws=p, ws_bytes=1 << 30)

    def pig(**kw):
        a = dict(args, **kw)
        return lib.cssm_proj_in_gates(*a.values(), None)
    assert pig(ctx=None) == -1 and b"non-null" in lib.cssm_last_error()
    assert pig(N=511) == -2
    assert pig(act_lo=9) == -4
    assert pig(gates=p + 4) == -5
    assert pig(ws=None) == -4 and b"workspace" in lib.cssm_last_error()
    gp.activation = 5
    assert pig() == -4 and b"activation" in lib.cssm_last_error()


@pytest.mark.parametrize("H", [4, 8, 14, 32, 64, 128])
def test_scan_khat_order(H):
    """K_hat's slots in the scan layout (host-side, no GPU): a permutation of the H (W/2 + 1)
    bins whose columns follow scan_col_order; row-major except at 128 x 128, where slot
    pair (2 s, 2 s + 1) holds rows u and u + 16 of one column for u in the even blocks of
    16 rows -- the two bins a column-pass lane takes with one 16-byte load."""
    from cssm_amd import spectral
    Wf = H // 2 + 1
    order = spectral.scan_khat_order(H, H)
    cols = spectral.scan_col_order(H, H)
    assert sorted(order) == list(range(H * Wf))
    if H != 128:
        assert order == [u * Wf + cols[p] for u in range(H) for p in range(Wf)]
        return
    for s in range(0, H * Wf, 2):
        (ua, va), (ub, vb) = divmod(order[s], Wf), divmod(order[s + 1], Wf)
        assert va == vb and ub == ua + 16 and (ua // 16) % 2 == 0
        pr, p = divmod(s // 2, Wf)
        assert va == cols[p] and ua == pr % 16 + 32 * (pr // 16)


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


def test_projection_entry_points_reject_misaligned_pointers():
    """Every pointer a projection kernel reads or writes with 4-element vectors is
    checked before any GPU work: an offset pointer returns CSSM_ERR_ALIGN (-5)."""
    from cssm_amd import _lib
    lib = _lib.load()
    buf = ctypes.create_string_buffer(4096)
    p = (ctypes.addressof(buf) + 255) // 256 * 256
    F, HW, K, N = 2, 16, 8, 8
    f32, bf16 = _lib.F32, _lib.BF16
    # proj_in: x (f32 16 B, bf16 8 B)
    assert lib.cssm_proj_in(p + 4, f32, F, HW, K, N, p, p, p, p, f32, 0, 0, None, None, 0, None) == -5
    assert lib.cssm_proj_in(p + 4, bf16, F, HW, K, N, p, p, p, p, f32, 0, 0, None, None, 0, None) == -5
    assert b"x must be" in lib.cssm_last_error()
    # proj_out: y and a f32 out
    assert lib.cssm_proj_out(p + 8, f32, F, HW, K, N, p, p, p, f32, None) == -5
    assert lib.cssm_proj_out(p, f32, F, HW, K, N, p, p, p + 4, f32, None) == -5
    assert lib.cssm_proj_out(p + 2, bf16, F, HW, K, N, p, p, p, bf16, None) == -5
    # proj_planes: x
    assert lib.cssm_proj_planes(p + 4, f32, F, HW, K, N, p, p, p, f32, 0, None) == -5
    # gdn_qkv_proj: x
    assert lib.cssm_gdn_qkv_proj(p + 4, f32, 1, 2, 4, 4, K, 4, p, p, 0, None, None, 0, None, p, f32, None) == -5
    assert b"x / qkv" in lib.cssm_last_error()
    # gdn_qkv_gate_proj: x, gv; a missing gate bias / output or an unknown act before any GPU work
    assert lib.cssm_gdn_qkv_gate_proj(p + 4, f32, 1, 2, 4, 4, K, 4, p, p, 0, None, None, 0, None, p, p, 1, p, p,
                                      f32, None) == -5
    assert lib.cssm_gdn_qkv_gate_proj(p, f32, 1, 2, 4, 4, K, 4, p, p, 0, None, None, 0, None, p, p, 1, p, p + 4,
                                      f32, None) == -5
    assert b"gv" in lib.cssm_last_error()
    assert lib.cssm_gdn_qkv_gate_proj(p, f32, 1, 2, 4, 4, K, 4, p, p, 0, None, None, 0, None, p, None, 1, p, p,
                                      f32, None) == -1
    assert lib.cssm_gdn_qkv_gate_proj(p, f32, 1, 2, 4, 4, K, 4, p, p, 0, None, None, 0, None, None, p, 1, p, p,
                                      f32, None) == -1
    assert lib.cssm_gdn_qkv_gate_proj(p, f32, 1, 2, 4, 4, K, 4, p, p, 0, None, None, 0, None, p, p, 0, p, p,
                                      f32, None) == -4
    # gdn_proj_out: out
    assert lib.cssm_gdn_proj_out(p, p, f32, F, HW, K, N, 0, None, None, p, p, p + 4, f32, None) == -5


def test_depthwise_conv_mean_workspace_and_errors():
    """The fused conv + frame-mean form: its workspace query (blocks per frame x F x C floats, 0 where
    the blocked conv has partial blocks or C / 4 does not divide 256) and its argument errors, all
    before any GPU work."""
    from cssm_amd import _lib
    lib = _lib.load()
    # 128 x 128 x 64, ks 5: 8-row blocks, (128/8)(128/4)(64/4) = 8192 threads per frame = 32 blocks
    assert lib.cssm_depthwise_conv_mean_workspace(3, 128, 128, 64, 5) == 32 * 3 * 64
    # 32 x 32 x 32, ks 3: 4 * 8 * 8 = 256 threads = 1 block
    assert lib.cssm_depthwise_conv_mean_workspace(2, 32, 32, 32, 3) == 1 * 2 * 32
    assert lib.cssm_depthwise_conv_mean_workspace(2, 16, 16, 64, 5) == 0     # 128 threads: a partial block
    assert lib.cssm_depthwise_conv_mean_workspace(2, 32, 32, 36, 3) == 0     # C / 4 = 9 does not divide 256
    assert lib.cssm_depthwise_conv_mean_workspace(2, 32, 32, 32, 9) == 0     # no blocked kernel for 9 x 9
    buf = ctypes.create_string_buffer(4096)
    p = (ctypes.addressof(buf) + 255) // 256 * 256
    f32 = _lib.F32
    assert lib.cssm_depthwise_conv_mean(p, f32, 2, 32, 32, 32, 3, p, p, p + 1024, f32, None, p, None) == -1
    assert lib.cssm_depthwise_conv_mean(p, f32, 2, 16, 16, 64, 5, p, p, p + 1024, f32, p, p, None) == -3
    assert b"no fused form" in lib.cssm_last_error()
    assert lib.cssm_depthwise_conv_mean(p + 4, f32, 2, 32, 32, 32, 3, p, p, p + 1024, f32, p, p, None) == -5


def test_noalloc_refuses_sizes_beyond_its_scratch():
    """cssm_proj_in_noalloc checks the ctx partial sums against its static scratch before any
    device lookup or launch, so a request beyond it fails on the host (pointers never read)."""
    from cssm_amd import _lib
    lib = _lib.load()
    F, HW, K, N = 4096, 16384, 64, 128
    need = int(lib.cssm_proj_in_workspace_size(F, HW, K, N))
    assert need > (64 << 20)
    buf = ctypes.create_string_buffer(64)
    p = ctypes.addressof(buf)
    st = lib.cssm_proj_in_noalloc(p, _lib.F32, F, HW, K, N, p, p, p, p, _lib.F32, 0, 0, ctypes.c_void_p(p), None)
    assert st == -3 and b"scratch" in lib.cssm_last_error()
