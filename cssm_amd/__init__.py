"""MI355X-native (gfx950) spectral state-space layer of drewlinsley/CSSM.

Hot path: the `gated` (GatedCSSM) and `gdn` (GatedDeltaNetCSSM) cells of
src/models/cssm.py, computed by hand-written HIP kernels behind the C ABI in
include/cssm_amd.h (``libcssm_hip.so``, built by ``cssm_amd.build``).
"""
__version__ = "0.1.0"
