"""Host-side mirror of the reference's CSSM-SHViT block (src/models/cssm_shvit.py).

``CSSMSHViTBlock`` keeps the reference constructor attributes and parameter
names (``norm1``, ``pos_conv``, ``cssm``, ``gate_fc1`` / ``gate_fc2``,
``norm2``, ``mlp``) and runs the block on the GPU:

    [image -> repeat to T] -> norm1 -> + pos_conv -> cell
    -> [last frame | every frame (video) | timestep-gate softmax pooling]
    -> output_act -> + residual -> LayerNorm norm2 -> Mlp (fc1 -> gelu -> + dwconv
    -> fc2) -> + residual

``apply`` is the whole block (cssm_shvit.py:65-266); ``token_mixer`` stops
after the first residual.  The cell, the norms, the position and MLP depthwise
convolutions and the residuals run in the HIP kernels of ``libcssm_hip.so``
(through :mod:`cssm_amd.spectral`); the MLP's two dense layers and the small
timestep-gate MLP are torch GEMMs on the same stream.
"""
from __future__ import annotations

from typing import Any, Dict, Optional

import torch
import torch.nn.functional as Fn

from . import spectral as S
from .cells import GatedCSSM, GatedDeltaNetCSSM, Params, _lecun_normal, tree_to_device


class CSSMSHViTBlock:
    """CSSMSHViTBlock (cssm_shvit.py:19-266).

    Not part of this build (NotImplementedError): the GDN
    ``static_image_fast_path`` (:79-94).  ``drop_path`` is the identity
    (inference).  Cell attributes that the cells themselves do not support
    raise there.
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
        if self.timestep_gate:
            hg = max(C // 4, 8)
            s["gate_fc1"] = {"kernel": (2 * C, hg), "bias": (hg,)}
            s["gate_fc2"] = {"kernel": (hg, 1), "bias": (1,)}
        hid = int(C * self.mlp_ratio)
        s["norm2"] = {"scale": (C,), "bias": (C,)}
        s["mlp"] = {"fc1": {"kernel": (C, hid), "bias": (hid,)}, "fc2": {"kernel": (hid, C), "bias": (C,)}}
        if self.use_dwconv:
            s["mlp"]["dwconv"] = {"dwconv": {"kernel": (3, 3, 1, hid), "bias": (hid,)}}
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

        def dense(k_in, k_out):
            return {"kernel": _lecun_normal((k_in, k_out), k_in, gen, device),
                    "bias": torch.zeros(k_out, device=device)}
        if self.timestep_gate:
            hg = max(C // 4, 8)
            p["gate_fc1"], p["gate_fc2"] = dense(2 * C, hg), dense(hg, 1)
        hid = int(C * self.mlp_ratio)
        p["norm2"] = {"scale": torch.ones(C, device=device), "bias": torch.zeros(C, device=device)}
        p["mlp"] = {"fc1": dense(C, hid), "fc2": dense(hid, C)}
        if self.use_dwconv:
            p["mlp"]["dwconv"] = {"dwconv": {"kernel": _lecun_normal((3, 3, 1, hid), 9, gen, device),
                                             "bias": torch.zeros(hid, device=device)}}
        return {"params": p}

    @staticmethod
    def load_params(tree, device="cuda") -> Params:
        tree = tree.get("params", tree) if isinstance(tree, dict) else tree
        return {"params": tree_to_device(tree, device)}

    # ---------------------------------------------------------------- forward
    def token_mixer(self, variables: Params, x: torch.Tensor, deterministic: bool = True) -> torch.Tensor:
        """The block up to its first residual (cssm_shvit.py:86-228): x (B, H, W, C) image or
        (B, T, H, W, C) video, float32 or bfloat16 on the GPU; returns (B, H, W, C) for an image
        or with the timestep gate (the cell's last frame, or its softmax-pooled frames), and
        (B, T, H, W, C) for video (keep_time, :191-213), same dtype."""
        return self._mixer(variables, x, x.dtype)

    def _mixer(self, variables: Params, x: torch.Tensor, out_dtype: torch.dtype) -> torch.Tensor:
        """token_mixer with the cell output and the residual in out_dtype.  The whole block keeps
        them in float32 under bf16 I/O: the reference's gated cell returns float32 there (it
        computes with float32 parameters, cssm_shvit.py:170-183), so its first residual is float32."""
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
        y = self.cell.apply({"params": p["cssm"]}, xc, out_dtype=out_dtype)
        del xc
        res = x5 if x5.dtype == out_dtype else x5.to(out_dtype)
        if self.timestep_gate:
            # softmax pooling over the cell's frames (:195-210), then the last input frame as residual
            y = self._timestep_gate(p, x5, y)
            return S.block_residual(res, y, 1, self.output_act)[:, 0]
        # frame selection, output activation and the residual with the block input
        out = S.block_residual(res, y, 1 if is_image else T, self.output_act)
        return out[:, 0] if is_image else out

    @staticmethod
    def _timestep_gate(p, x5, y):
        """(B, 1, H, W, C): sum_t softmax_t(gate_fc2(gelu(gate_fc1([mean x5[:, 0], mean y_t]))) + prior) y_t,
        the prior 4 on the last frame (cssm_shvit.py:195-210)."""
        T = y.shape[1]
        q = x5[:, 0].float().mean(dim=(1, 2))
        k = y.float().mean(dim=(2, 3))
        gin = torch.cat([q[:, None].expand_as(k), k], dim=-1)
        h = Fn.gelu(gin @ p["gate_fc1"]["kernel"] + p["gate_fc1"]["bias"], approximate="tanh")
        logits = (h @ p["gate_fc2"]["kernel"] + p["gate_fc2"]["bias"])[..., 0]
        prior = torch.zeros(T, device=y.device)
        prior[-1] = 4.0
        w = torch.softmax(logits + prior, dim=-1)
        return torch.einsum("bt,bthwc->bhwc", w, y.float()).to(y.dtype).unsqueeze(1).contiguous()

    def _mlp_half(self, p, x):
        """x + Mlp(norm2(x)) per frame (cssm_shvit.py:231-266; Mlp shvit.py:156-182)."""
        shp = x.shape
        H, W, C = shp[-3:]
        x5 = x if x.dim() == 5 else x.unsqueeze(1)
        n2 = p["norm2"]
        h = S.block_norm_posconv(x5, S.block_norm_stats(x5, "layer"), "layer", n2["scale"], n2["bias"], None, None,
                                 x5.shape[1]).float()
        m = p["mlp"]
        h = Fn.gelu(torch.addmm(m["fc1"]["bias"], h.reshape(-1, C), m["fc1"]["kernel"]), approximate="tanh")
        hid = h.shape[-1]
        h = h.reshape(-1, H, W, hid)
        if self.use_dwconv:
            dw = m["dwconv"]["dwconv"]
            h = h + S.depthwise_conv(h, dw["kernel"], dw["bias"])
        h = torch.addmm(m["fc2"]["bias"], h.reshape(-1, hid), m["fc2"]["kernel"])
        return (x.float() + h.reshape(shp)).to(x.dtype)

    def apply(self, variables: Params, x: torch.Tensor, deterministic: bool = True) -> torch.Tensor:
        """The whole block: token mixer, then norm2 -> Mlp -> residual; same shapes as
        :meth:`token_mixer` returns, in x's dtype (float32 inside under bf16 I/O)."""
        return self._mlp_half(variables["params"], self._mixer(variables, x, torch.float32)).to(x.dtype)

    __call__ = apply
