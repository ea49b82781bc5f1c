"""Host-side mirror of the reference's CSSM-SHViT block wiring (src/models/cssm_shvit.py).

``CSSMSHViTBlock`` keeps the reference constructor attributes and parameter
names (``norm1``, ``pos_conv``, ``cssm``) and runs the token-mixer half of the
block (cssm_shvit.py:86-229) on the GPU:

    [image -> repeat to T] -> norm1 -> + pos_conv -> cell -> [last frame]
    -> output_act -> + residual

``apply`` returns the block state after that residual.  The second half of the
reference block (norm2 -> Mlp -> residual, :231-266) is not part of this
build: a caller applies its own MLP to the returned tensor (the ``norm2`` /
``mlp`` parameters are ignored if present).  The arithmetic runs in the HIP
kernels of ``libcssm_hip.so`` through :mod:`cssm_amd.spectral`.
"""
from __future__ import annotations

from typing import Any, Dict, Optional

import torch

from . import spectral as S
from .cells import GatedCSSM, GatedDeltaNetCSSM, Params, _lecun_normal, tree_to_device


class CSSMSHViTBlock:
    """CSSMSHViTBlock (cssm_shvit.py:19-266), token-mixer half.

    Not part of this build (NotImplementedError): ``timestep_gate`` (the
    softmax pooling over T, :195-210) and the GDN ``static_image_fast_path``
    (:79-94).  ``drop_path`` is the identity (inference).  Cell attributes that
    the cells themselves do not support raise there.
    """

    def __init__(self, dim: int, mlp_ratio: float = 4.0, drop_path: float = 0.0, cssm_type: str = "gated",
                 dense_mixing: bool = False, block_size: int = 32, mixing_rank: int = 0,
                 gate_activation: str = "softplus", num_timesteps: int = 8, kernel_size: int = 15,
                 spectral_rho: float = 0.999, rope_mode: str = "none", use_dwconv: bool = True,
                 output_act: str = "none", short_conv_size: int = 4, short_conv_spatial_size: int = 3,
                 delta_key_dim: int = 2, output_norm: str = "rms", gate_type: str = "factored",
                 block_norm: str = "global_layer", use_pos_conv: bool = True, gate_proj_bias_init: float = 0.0,
                 static_image_fast_path: bool = False, use_input_gates: bool = True, ssl_proj_dim: int = 0,
                 timestep_gate: bool = False, dtype=None, param_dtype=None, name: Optional[str] = None):
        if timestep_gate:
            raise NotImplementedError("CSSMSHViTBlock: timestep_gate (cssm_shvit.py:195-210) is not part of this build")
        if static_image_fast_path and cssm_type == "gdn":
            raise NotImplementedError("CSSMSHViTBlock: the GDN static-image fast path is not part of this build")
        if block_norm not in S.BLOCK_NORMS:
            raise ValueError(f"block_norm={block_norm!r}")
        if output_act not in S.OUTPUT_ACTS:
            raise ValueError(f"output_act={output_act!r}")
        self.dim = dim
        self.mlp_ratio = mlp_ratio
        self.drop_path = drop_path
        self.cssm_type = cssm_type
        self.num_timesteps = num_timesteps
        self.output_act = output_act
        self.block_norm = block_norm
        self.use_pos_conv = use_pos_conv
        self.use_dwconv = use_dwconv
        self.timestep_gate = timestep_gate
        self.static_image_fast_path = static_image_fast_path
        self.name = name
        # the cell with the kwargs the reference block passes (:147-185); 'gated'
        # passes no dtype, so the cell computes in fp32 whatever the block dtype
        if cssm_type == "gdn":
            self.cell = GatedDeltaNetCSSM(
                channels=dim, delta_key_dim=delta_key_dim, kernel_size=kernel_size, spectral_rho=spectral_rho,
                rope_mode=rope_mode, gate_type=gate_type, short_conv_size=short_conv_size, output_norm=output_norm,
                use_input_gates=use_input_gates, static_image_fast_path=static_image_fast_path,
                num_timesteps=num_timesteps, ssl_proj_dim=ssl_proj_dim, gate_proj_bias_init=gate_proj_bias_init,
                dtype=dtype, param_dtype=param_dtype)
        else:
            self.cell = GatedCSSM(
                channels=dim, dense_mixing=dense_mixing, gate_activation=gate_activation, kernel_size=kernel_size,
                spectral_rho=spectral_rho, rope_mode=rope_mode, short_conv_size=short_conv_size,
                short_conv_spatial_size=short_conv_spatial_size, block_size=block_size, mixing_rank=mixing_rank,
                gate_type=gate_type)

    # ------------------------------------------------------------- parameters
    def param_shapes(self, H: int, W: int) -> Dict[str, Any]:
        C = self.dim
        s: Dict[str, Any] = {"norm1": {"scale": (C,), "bias": (C,)}}
        if self.use_pos_conv:
            s["pos_conv"] = {"kernel": (3, 3, 1, C), "bias": (C,)}
        s["cssm"] = (self.cell.param_shapes(H, W) if self.cssm_type == "gdn"
                     else self.cell.param_shapes(C, H, W))
        return s

    def init(self, seed: int, x_shape, device="cuda") -> Params:
        """Fresh parameters for inputs (B, H, W, C) or (B, T, H, W, C): LayerNorm
        scale ones / bias zeros, lecun-normal pos_conv kernel, zero bias, and the
        cell's own initialisation."""
        H, W = x_shape[-3], x_shape[-2]
        C = self.dim
        gen = torch.Generator(device=device).manual_seed(int(seed) + 1)
        p: Dict[str, Any] = {"norm1": {"scale": torch.ones(C, device=device), "bias": torch.zeros(C, device=device)}}
        if self.use_pos_conv:
            p["pos_conv"] = {"kernel": _lecun_normal((3, 3, 1, C), 9, gen, device),
                             "bias": torch.zeros(C, device=device)}
        T = self.num_timesteps if len(x_shape) == 4 else x_shape[1]
        p["cssm"] = self.cell.init(seed, (x_shape[0], T, H, W, C), device)["params"]
        return {"params": p}

    @staticmethod
    def load_params(tree, device="cuda") -> Params:
        tree = tree.get("params", tree) if isinstance(tree, dict) else tree
        return {"params": tree_to_device(tree, device)}

    # ---------------------------------------------------------------- forward
    def apply(self, variables: Params, x: torch.Tensor, deterministic: bool = True) -> torch.Tensor:
        """Token-mixer half of the block: x (B, H, W, C) image or (B, T, H, W, C)
        video, float32 or bfloat16 on the GPU; returns (B, H, W, C) for an image
        (the cell's last frame, :224) or (B, T, H, W, C) for video (keep_time,
        :213), same dtype."""
        p = variables["params"]
        is_image = x.dim() == 4
        x = x.contiguous()
        x5 = x.unsqueeze(1) if is_image else x                  # (B, T_in, H, W, C)
        B, T_in, H, W, C = x5.shape
        if C != self.dim:
            raise ValueError(f"input has {C} channels, block dim is {self.dim}")
        T = self.num_timesteps if is_image else T_in
        # norm1 over the (repeated) input and the positional depthwise conv, written as the T cell frames
        n1 = p["norm1"]
        stats = S.block_norm_stats(x5, self.block_norm)
        pc = p.get("pos_conv") if self.use_pos_conv else None
        xc = S.block_norm_posconv(x5, stats, self.block_norm, n1["scale"], n1["bias"],
                                  pc["kernel"] if pc is not None else None, pc["bias"] if pc is not None else None, T)
        y = self.cell.apply({"params": p["cssm"]}, xc)
        del xc
        # frame selection, output activation and the residual with the block input
        out = S.block_residual(x5, y, 1 if is_image else T, self.output_act)
        return out[:, 0] if is_image else out

    __call__ = apply
