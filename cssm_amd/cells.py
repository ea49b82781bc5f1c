"""Host-side mirror of the reference's CSSM cell modules (src/models/cssm.py).

``GatedCSSM`` keeps the constructor attributes, the parameter names and shapes
(the Flax tree ``{'params': {...}}``) and the call signature
``cell.apply(variables, x, injected_qkv_spatial=None) -> y`` of the reference
Flax module, with x channels-last (B, T, H, W, C).  The arithmetic runs in the
HIP kernels of ``libcssm_hip.so`` (through :mod:`cssm_amd.spectral`); this
module only orders the calls and owns no numerics of its own.

Parameters are device tensors.  ``init`` draws them from the reference's
initializer families (lecun-normal Dense/Conv kernels, zero biases,
N(0, 0.02^2) spectral kernel) with a torch generator: the values differ from a
JAX PRNG draw of the same seed (JAX is not available here), the shapes and
distributions match.  ``load_params`` accepts a tree of numpy arrays in the
reference layout (e.g. a converted checkpoint).
"""
from __future__ import annotations

import math
from typing import Any, Dict, Optional

import numpy as np
import torch

from . import spectral as S

Params = Dict[str, Any]


def _lecun_normal(shape, fan_in, gen, device):
    # flax lecun_normal: truncated normal (+-2 sigma) with variance 1/fan_in
    std = math.sqrt(1.0 / max(1, fan_in)) / 0.87962566103423978
    t = torch.empty(shape, dtype=torch.float32, device=device)
    torch.nn.init.trunc_normal_(t, mean=0.0, std=std, a=-2 * std, b=2 * std, generator=gen)
    return t


def tree_to_device(tree, device="cuda"):
    """Nested dict of numpy arrays / tensors -> float32 contiguous device tensors."""
    if isinstance(tree, dict):
        return {k: tree_to_device(v, device) for k, v in tree.items()}
    t = torch.as_tensor(np.asarray(tree) if not isinstance(tree, torch.Tensor) else tree)
    return t.to(device=device, dtype=torch.float32).contiguous()


class GatedCSSM:
    """GatedCSSM (cssm.py:384-585): spectral Mamba cell, depthwise path.

    x -> in_proj -> (x_main, z); x_main -> [short convs] -> SiLU -> rfft2 ->
    per-frequency Delta/B/C gates from the spatial mean -> diagonal complex scan
    over T with decay K_hat e^{-Delta} -> x C -> irfft2 -> x SiLU(z) -> out_proj.

    ``expand`` (not a reference attribute; default 1 = the reference) widens the
    inner channel count to ``channels * expand`` (in_proj C -> 2 C expand,
    out_proj C expand -> C), the shape BASELINE configs 1 and 5 describe.
    """

    def __init__(self, channels: int, dense_mixing: bool = False, block_size: int = 32, mixing_rank: int = 0,
                 kernel_size: int = 15, spectral_rho: float = 0.999, gate_activation: str = "softplus",
                 rope_mode: str = "none", gate_rank: int = 0, rope_base: float = 10000.0, concat_xy: bool = True,
                 position_independent_gates: bool = False, short_conv_size: int = 4,
                 short_conv_spatial_size: int = 3, gate_type: str = "dense", expand: int = 1,
                 name: Optional[str] = None):
        if dense_mixing:
            raise NotImplementedError("dense_mixing (cssm.py:587-865) is not part of this build")
        if rope_mode != "none":
            raise NotImplementedError("rope_mode other than 'none' is not part of this build")
        self.channels = channels
        self.dense_mixing = dense_mixing
        self.block_size = block_size
        self.mixing_rank = mixing_rank
        self.kernel_size = kernel_size
        self.spectral_rho = spectral_rho
        self.gate_activation = gate_activation
        self.rope_mode = rope_mode
        self.gate_rank = gate_rank
        self.rope_base = rope_base
        self.concat_xy = concat_xy
        # the depthwise path derives the gates from x_main whatever this flag says
        self.position_independent_gates = position_independent_gates
        self.short_conv_size = short_conv_size
        self.short_conv_spatial_size = short_conv_spatial_size
        self.gate_type = gate_type
        self.expand = expand
        self.name = name
        self._khat_cache: Dict[Any, torch.Tensor] = {}

    # ------------------------------------------------------------- parameters
    def param_shapes(self, c_in: int, H: int, W: int) -> Dict[str, Any]:
        Ci = self.channels * self.expand
        Wf = W // 2 + 1
        s: Dict[str, Any] = {"in_proj": {"kernel": (c_in, 2 * Ci), "bias": (2 * Ci,)}}
        if self.short_conv_spatial_size > 0:
            k = self.short_conv_spatial_size
            s["short_conv_spatial"] = {"kernel": (k, k, 1, Ci), "bias": (Ci,)}
        if self.short_conv_size > 0:
            s["short_conv_temporal"] = {"kernel": (self.short_conv_size, 1, Ci), "bias": (Ci,)}
        s["kernel"] = (Ci, self.kernel_size, self.kernel_size)
        for g in ("delta_proj", "B_proj", "C_proj"):
            if self.gate_type == "factored":
                s[f"{g}_h"] = {"kernel": (Ci, H), "bias": (H,)}
                s[f"{g}_w"] = {"kernel": (Ci, Wf), "bias": (Wf,)}
            else:
                s[g] = {"kernel": (Ci, H * Wf), "bias": (H * Wf,)}
        s["out_proj"] = {"kernel": (Ci, self.channels), "bias": (self.channels,)}
        return s

    def init(self, seed: int, x_shape, device="cuda") -> Params:
        """Fresh parameters for inputs of shape (B, T, H, W, C_in)."""
        _, _, H, W, c_in = x_shape
        gen = torch.Generator(device=device).manual_seed(int(seed))
        params: Dict[str, Any] = {}
        for name, v in self.param_shapes(c_in, H, W).items():
            if name == "kernel":
                params[name] = torch.randn(v, generator=gen, device=device, dtype=torch.float32) * 0.02
                continue
            sub = {}
            for pn, shp in v.items():
                if pn == "kernel":
                    fan_in = shp[0] if len(shp) == 2 else int(np.prod(shp[:-1]))
                    sub[pn] = _lecun_normal(shp, fan_in, gen, device)
                else:
                    sub[pn] = torch.zeros(shp, dtype=torch.float32, device=device)
            params[name] = sub
        return {"params": params}

    @staticmethod
    def load_params(tree, device="cuda") -> Params:
        tree = tree.get("params", tree) if isinstance(tree, dict) else tree
        return {"params": tree_to_device(tree, device)}

    # ---------------------------------------------------------------- forward
    def spectral_kernel(self, p: Dict[str, Any], H: int, W: int) -> torch.Tensor:
        """Floored K_hat for (H, W); cached per kernel tensor version."""
        k = p["kernel"]
        key = (k.data_ptr(), k._version, H, W, self.spectral_rho)
        kh = self._khat_cache.get(key)
        if kh is None:
            kh = S.spectral_kernel(k, H, W, self.spectral_rho, squash=True, goom_floor=True)
            self._khat_cache = {key: kh}
        return kh

    def apply(self, variables: Params, x: torch.Tensor, injected_qkv_spatial=None) -> torch.Tensor:
        """y = GatedCSSM(x); x (B, T, H, W, C) float32 or bfloat16 on the GPU, y same dtype."""
        p = variables["params"]
        B, T, H, W, c_in = x.shape
        Ci = self.channels * self.expand
        F, HW = B * T, H * W
        if not S.gated_scan_supported(H, W):
            raise NotImplementedError(f"no fused scan kernel for {H}x{W} planes")
        g = S.gated_scan_min_group(H, W)
        if Ci % g:
            raise NotImplementedError(f"{Ci} inner channels is not a multiple of {g} for {H}x{W} planes")
        x = x.contiguous()
        has_conv = self.short_conv_spatial_size > 0 or self.short_conv_size > 0
        # in_proj straight into plane-major x_main and z; SiLU(z) (cssm.py:581) fused here,
        # SiLU(x_main) and ctx too unless the short convolutions come first
        xm, z, ctx = S.proj_in(x, p["in_proj"]["kernel"], p["in_proj"]["bias"], F, HW,
                               silu_lo=not has_conv, silu_hi=True, want_ctx=not has_conv)
        xm = xm.view(B, T, Ci, H, W)
        z = z.view(B, T, Ci, H, W)
        if has_conv:
            u, ctx = S.short_conv(xm, p.get("short_conv_spatial") if self.short_conv_spatial_size > 0 else None,
                                  p.get("short_conv_temporal") if self.short_conv_size > 0 else None)
            del xm
        else:
            u = xm
        ctx = ctx.view(B, T, Ci)
        gates = S.gated_gates(ctx, p, H, W, self.gate_type, self.gate_activation, c_scale=1.0 / HW)
        khat = self.spectral_kernel(p, H, W)
        y = S.gated_scan(u, z, gates, khat)
        out = S.proj_out(y.view(F, Ci, HW), p["out_proj"]["kernel"], p["out_proj"]["bias"])
        return out.view(B, T, H, W, self.channels)

    __call__ = apply
