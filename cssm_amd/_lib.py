"""ctypes binding of libcssm_hip.so (the C ABI in include/cssm_amd.h).

The library is built in-tree by ``cssm_amd.build``.  There is no fallback:
if the library is missing or fails to load, every call raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libcssm_hip.so")
ABI_VERSION = 8   # CSSM_ABI_VERSION of the include/cssm_amd.h these bindings follow

CSSM_OK = 0
F32, BF16 = 0, 1
GATE_DENSE, GATE_FACTORED = 0, 1
ACT_SOFTPLUS, ACT_SIGMOID2, ACT_EXP = 0, 1, 2
LOAD_IDENTITY, LOAD_SILU = 0, 1
ACT_IDENTITY, ACT_SILU, ACT_SIGMOID = 0, 1, 2
GDN_GATE_DENSE, GDN_GATE_FACTORED, GDN_GATE_CHANNEL, GDN_GATE_SCALAR = 0, 1, 2, 3
NORM_NONE, NORM_RMS, NORM_LAYER = 0, 1, 2

_c_float_p = ctypes.POINTER(ctypes.c_float)


class GateParams(ctypes.Structure):
    """cssm_gate_params (include/cssm_amd.h)."""
    _fields_ = [
        ("gate_type", ctypes.c_int),
        ("activation", ctypes.c_int),
        ("kernel", ctypes.c_void_p * 3),
        ("bias", ctypes.c_void_p * 3),
        ("kernel_w", ctypes.c_void_p * 3),
        ("bias_w", ctypes.c_void_p * 3),
    ]


class GdnGateParams(ctypes.Structure):
    """cssm_gdn_gate_params (include/cssm_amd.h): 0 alpha, 1 beta, 2 B_k, 3 B_v."""
    _fields_ = [
        ("gate_type", ctypes.c_int),
        ("kernel", ctypes.c_void_p * 4),
        ("bias", ctypes.c_void_p * 4),
        ("kernel_w", ctypes.c_void_p * 4),
        ("bias_w", ctypes.c_void_p * 4),
    ]


_P = ctypes.c_void_p
_I = ctypes.c_int
_LL = ctypes.c_longlong

# name -> (restype, argtypes); every symbol declared in include/cssm_amd.h
SIGNATURES = {
    "cssm_abi_version": (ctypes.c_int, []),
    "cssm_strerror": (ctypes.c_char_p, [ctypes.c_int]),
    "cssm_last_error": (ctypes.c_char_p, []),
    "cssm_spectral_kernel": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                            ctypes.c_int, ctypes.c_float, ctypes.c_int, ctypes.c_int,
                                            ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]),
    "cssm_plane_mean": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_longlong, ctypes.c_int,
                                       ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]),
    "cssm_gated_gates": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                        ctypes.c_int, ctypes.c_int, ctypes.POINTER(GateParams),
                                        ctypes.c_float, ctypes.c_void_p, ctypes.c_void_p]),
    "cssm_gated_gates_bwd": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                            ctypes.c_int, ctypes.c_int, ctypes.POINTER(GateParams),
                                            ctypes.c_float, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]),
    "cssm_gated_scan_fwd": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
                                           ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                           ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
                                           ctypes.c_int, ctypes.c_void_p]),
    "cssm_proj_in_gates": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                          ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
                                          ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                          ctypes.c_void_p, ctypes.POINTER(GateParams), ctypes.c_float,
                                          ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    "cssm_proj_in": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                    ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                    ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                    ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    "cssm_gated_scan_bwd": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, ctypes.c_float, _P, _P, _P, _P, _P]),
    "cssm_proj_in_workspace_size": (ctypes.c_size_t, [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int]),
    "cssm_proj_in_noalloc": (_I, [_P, _I, _I, _I, _I, _I, _P, _P, _P, _P, _I, _I, _I, _P, _P]),
    "cssm_proj_out": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                     ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                     ctypes.c_int, ctypes.c_void_p]),
    "cssm_short_conv": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                       ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
                                       ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                       ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]),
    "cssm_proj_planes": (_I, [_P, _I, _I, _I, _I, _I, _P, _P, _P, _I, _I, _P]),
    "cssm_frame_mean": (_I, [_P, _I, _I, _I, _I, _P, _P]),
    "cssm_depthwise_conv": (_I, [_P, _I, _I, _I, _I, _I, _I, _P, _P, _P, _I, _P]),
    "cssm_depthwise_conv_mean_workspace": (_LL, [_I, _I, _I, _I, _I]),
    "cssm_depthwise_conv_mean": (_I, [_P, _I, _I, _I, _I, _I, _I, _P, _P, _P, _I, _P, _P, _P]),
    "cssm_gdn_gates": (_I, [_P, _I, _I, _I, _I, _I, _I, ctypes.POINTER(GdnGateParams), _I, ctypes.c_float, _P,
                            _P, _P, _P]),
    "cssm_gdn_qkv_post": (_I, [_P, _I, _I, _I, _I, _I, _I, _I, _P, _P, _I, _P, _P]),
    "cssm_gdn_qkv_proj": (_I, [_P, _I, _I, _I, _I, _I, _I, _I, _P, _P, _I, _P, _P, _I, _P, _P, _I, _P]),
    "cssm_gdn_qkv_gate_proj": (_I, [_P, _I, _I, _I, _I, _I, _I, _I, _P, _P, _I, _P, _P, _I, _P, _P, _P, _I, _P, _P,
                                    _I, _P]),
    "cssm_gdn_qkv_fused": (_I, [_I, _I, _I, _I, _I]),
    "cssm_rfft2": (_I, [_P, _I, _LL, _I, _I, _P, _P, _P]),
    "cssm_irfft2": (_I, [_P, _LL, _I, _I, _P, _I, _P]),
    "cssm_fft_min_group": (_I, [_I, _I]),
    "cssm_gdn_scan_bins": (_I, [_P, _P, _P, _LL, _I, _I, _P, _I, _I, _I, _I, _I, _I, _I, _P, _P]),
    "cssm_depthwise_conv_wgrad": (_I, [_P, _P, _I, _I, _I, _I, _I, _P, _I, _P]),
    "cssm_depthwise_conv_wgrad_supported": (_I, [_I, _I, _I]),
    "cssm_gdn_scan_bins_train": (_I, [_P, _P, _LL, _I, _I, _P, _I, _I, _I, _I, _I, _I, _I, _P, _P, _P]),
    "cssm_gdn_scan_bins_bwd": (_I, [_P, _P, _LL, _I, _I, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P, _P, _P, _P]),
    "cssm_gdn_proj_out": (_I, [_P, _P, _I, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _I, _P]),
    "cssm_gdn_proj_out_xgate": (_I, [_P, _I, _P, _I, _I, _I, _I, _I, _I, _P, _P, _P, _P, _I, _P, _P, _P, _I, _P]),
    "cssm_gdn_proj_out_xgate_supported": (_I, [_I, _I, _I]),
    "cssm_gdn_core_fused": (_I, [_P, _I, _P, _LL, _I, _I, _P, _I, _I, _I, _I, _I, _I, _I, _P, _P]),
    "cssm_gdn_core_fused_supported": (_I, [_I, _I, _I]),
    "cssm_rfft2_ex": (_I, [_P, _I, _I, _P, _I, _I, _I, _LL, _I, _I, _P, _P]),
    "cssm_irfft2_ex": (_I, [_P, _LL, _I, _I, _I, _P, _I, _P, _P, _I, _P, _I, _P, _P]),
    "cssm_irfft2_ex_sums_supported": (_I, [_LL, _I, _I]),
    "cssm_fft_ex_supported": (_I, [_I, _I]),
    "cssm_im2col_same": (_I, [_P, _I, _I, _I, _I, _I, _I, _P, _P]),
    "cssm_gated_scan_supported": (ctypes.c_int, [ctypes.c_int, ctypes.c_int]),
    "cssm_gated_scan_min_group": (ctypes.c_int, [ctypes.c_int, ctypes.c_int]),
    "cssm_gated_scan_col_order": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_int)]),
    "cssm_gated_scan_khat_order": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_int)]),
    "cssm_block_norm_stats": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                             ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_float,
                                             ctypes.c_void_p, ctypes.c_void_p]),
    "cssm_block_norm_posconv": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                               ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                               ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                               ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]),
    "cssm_block_residual": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int,
                                           ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                           ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]),
}

_lock = threading.Lock()
_lib = None


class CssmError(RuntimeError):
    def __init__(self, fn: str, status: int, detail: str):
        super().__init__(f"{fn} failed ({status}): {detail}")
        self.status = status


def load() -> ctypes.CDLL:
    """Load (once) and return the HIP library; raises if it is not built."""
    global _lib
    lib = _lib
    if lib is not None:         # loaded: no lock on the per-call path
        return lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m cssm_amd.build`")
            lib = ctypes.CDLL(LIB_PATH)
            got = lib.cssm_abi_version()
            if got != ABI_VERSION:
                raise RuntimeError(f"{LIB_PATH} has ABI version {got}, these bindings expect {ABI_VERSION}: "
                                   "rebuild it with `python -m cssm_amd.build`")
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def check(fn_name: str, status: int) -> None:
    if status != CSSM_OK:
        lib = load()
        detail = lib.cssm_last_error().decode() or lib.cssm_strerror(status).decode()
        raise CssmError(fn_name, status, detail)


def call(fn_name: str, *args) -> None:
    """Call an int-returning entry point and raise CssmError on failure."""
    check(fn_name, getattr(load(), fn_name)(*args))
