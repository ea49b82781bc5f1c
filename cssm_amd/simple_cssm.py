"""Host-side mirror of the reference's SimpleCSSM model (src/models/simple_cssm.py).

``SimpleCSSM`` keeps the reference's constructor attributes, parameter names
(``conv1`` / ``norm1`` / ``cssm_0`` / ``norm_pre`` / ``norm_post`` / ``head``
...) and call ``model.apply(variables, x) -> logits``.  Around the cells it
runs the reference's stem and readout:

    [image -> repeat to seq_len] -> stem (1x1 conv, or conv 3x3 + norm/act +
    max-pool per layer) -> [learnable position embedding] -> [register tokens]
    -> depth x (x + cell(x) -> inter-block norm + act [+ channel MLP])
    -> [strip registers] -> frame selection -> norm/act -> pool -> norm -> head

The cells (``gated`` / ``gdn`` / ``gdn_d2`` / ``gdn_d3`` from
:mod:`cssm_amd.registry`) are the HIP layer; the residual ``x + cell(x)`` and
the LayerNorm family (per pixel, 'temporal_layer', 'global_layer') run on the
HIP block kernels; the stem convolution, pooling, BatchNorm / GroupNorm,
activations and the dense head are small torch ops on the same stream.

Not part of this build (NotImplementedError): cell types outside the registry,
and the position embeddings that rotate features (RoPE: 'spatiotemporal',
'spatial_only', 'temporal', 'mrope', 'separate', 'sinusoidal'); 'none' and
'learnable' are supported.  BatchNorm runs on its running statistics
(``training=False``, the inference the reference's benchmarks time) or on the
batch statistics without updating them (``training=True``).
"""
from __future__ import annotations

import math
from typing import Any, Dict, Optional

import torch
import torch.nn.functional as Fn

from . import spectral as S
from .cells import Params, _lecun_normal, tree_to_device
from .registry import CSSM_REGISTRY, make_cell

# reference attributes and defaults (simple_cssm.py:88-153)
_DEFAULTS = dict(
    num_classes=2, embed_dim=32, depth=1, cssm_type="hgru_bi", kernel_size=15, block_size=1, frame_readout="last",
    norm_type="layer", stem_norm="", body_norm="", pos_embed="spatiotemporal", act_type="softplus",
    pool_type="mean", seq_len=8, max_seq_len=32, position_independent_gates=False, use_goom=True, use_log=True,
    shared_kernel=False, additive_kv=False, spectral_clip=False, q_temporal=3, q_spatial=5, asymmetric_qk=False,
    no_feedback=False, no_spectral_clip=False, use_layernorm=False, no_k_state=False, transformer_readout="qka",
    gate_type="dense", n_register_tokens=0, learned_init=False, stem_mode="default", stem_layers=2,
    stem_norm_order="post", use_complex32=False, use_complex16=False, use_ssd=False, scan_mode="associative",
    ssd_chunk_size=8, readout_norm="pre", num_heads=4, mlp_ratio=4.0, drop_path_rate=0.0, short_conv_size=4,
    short_conv_spatial_size=3, output_norm="rms", use_input_gates=True, output_gate_act="silu",
    use_spectral_l2_norm=True, qkv_conv_size=1, qkv_conv_separable=True, cross_freq_conv_size=0, delta_key_dim=2,
    no_spectral_clamp=False, inter_mlp_ratio=0.0, attn_kernel_size=7, int_attn_dim=16, state_dim=16,
    expand_factor=2, flatten_mode="temporal_spatial", s4nd_d_state=64, s4nd_bidirectional=True,
    convs5_state_dim=16, convs5_num_groups=1,
)
_LN_MODES = {"global_layer": "global_layer", "temporal_layer": "temporal_layer"}


class SimpleCSSM:
    """SimpleCSSM (simple_cssm.py:63-558) around the cells of this build."""

    def __init__(self, name: Optional[str] = None, **kwargs):
        unknown = set(kwargs) - set(_DEFAULTS)
        if unknown:
            raise TypeError(f"SimpleCSSM: unknown attributes {sorted(unknown)}")
        for k, v in _DEFAULTS.items():
            setattr(self, k, kwargs.get(k, v))
        self.name = name
        if self.cssm_type not in CSSM_REGISTRY:
            raise NotImplementedError(f"SimpleCSSM: cssm_type={self.cssm_type!r} is not part of this build "
                                      f"(have {sorted(CSSM_REGISTRY)})")
        if self.pos_embed not in ("none", "learnable"):
            raise NotImplementedError(f"SimpleCSSM: pos_embed={self.pos_embed!r} (RoPE) is not part of this build")
        self.cells = [make_cell(self.cssm_type, **self._cell_kwargs(i)) for i in range(self.depth)]

    def _cell_kwargs(self, i: int) -> Dict[str, Any]:
        """The kwargs the reference passes to block i's cell (simple_cssm.py:325-443)."""
        kw: Dict[str, Any] = dict(channels=self.embed_dim, kernel_size=self.kernel_size, block_size=self.block_size,
                                  rope_mode="none", name=f"cssm_{i}")
        if self.cssm_type == "gated":
            kw.update(short_conv_spatial_size=self.short_conv_spatial_size, short_conv_size=self.short_conv_size,
                      gate_type=self.gate_type)
        else:
            kw.update(use_goom=self.use_goom, use_log=self.use_log, gate_type=self.gate_type,
                      learned_init=self.learned_init, use_complex32=self.use_complex32,
                      use_complex16=self.use_complex16, scan_mode=self.scan_mode, ssd_chunk_size=self.ssd_chunk_size,
                      short_conv_size=self.short_conv_size, output_norm=self.output_norm,
                      use_input_gates=self.use_input_gates, output_gate_act=self.output_gate_act,
                      use_spectral_l2_norm=self.use_spectral_l2_norm, qkv_conv_size=self.qkv_conv_size,
                      qkv_conv_separable=self.qkv_conv_separable, cross_freq_conv_size=self.cross_freq_conv_size,
                      no_spectral_clamp=self.no_spectral_clamp)
            if self.cssm_type == "gdn":
                kw["delta_key_dim"] = self.delta_key_dim   # gdn_d2 / gdn_d3 set theirs in make_cell
        return kw

    # ------------------------------------------------------------- parameters
    def _norms(self):
        return self.stem_norm or self.norm_type, self.body_norm or self.norm_type

    def param_shapes(self, x_shape):
        """(params, batch_stats) shapes for inputs (B, [T,] H, W, C_in)."""
        H, W, cin = x_shape[-3], x_shape[-2], x_shape[-1]
        D = self.embed_dim
        stem_norm, body_norm = self._norms()
        p: Dict[str, Any] = {}
        bs: Dict[str, Any] = {}

        def norm(name, c, kind):
            p[name] = {"scale": (c,), "bias": (c,)}
            if kind == "batch":
                bs[name] = {"mean": (c,), "var": (c,)}
        if self.stem_mode == "pathtracker":
            p["conv1"] = {"kernel": (1, 1, cin, D), "bias": (D,)}
            norm("norm1", cin if self.stem_norm_order == "pre" else D, stem_norm)
        else:
            c = cin
            for i in range(self.stem_layers):
                norm(f"norm{i + 1}", c if self.stem_norm_order == "pre" else D, stem_norm)
                p[f"conv{i + 1}"] = {"kernel": (3, 3, c, D), "bias": (D,)}
                c = D
                H, W = (H + 1) // 2, (W + 1) // 2
        if self.pos_embed == "learnable":
            p["pos_embed"] = (1, 1, H, W, D)
        if self.n_register_tokens > 0:
            p["register_tokens"] = (1, self.n_register_tokens, H, W, D)
        for i, cell in enumerate(self.cells):
            p[f"cssm_{i}"] = cell.param_shapes(D, H, W) if self.cssm_type == "gated" else cell.param_shapes(H, W)
            if self.depth > 1 and i < self.depth - 1:
                norm(f"body_norm_{i}", D, body_norm)
                if self.inter_mlp_ratio > 0:
                    hid = int(D * self.inter_mlp_ratio)
                    p[f"mlp_{i}_up"] = {"kernel": (D, hid), "bias": (hid,)}
                    p[f"mlp_{i}_down"] = {"kernel": (hid, D), "bias": (D,)}
        norm("norm_pre", D, body_norm)
        norm("norm_post", D, body_norm)
        p["head"] = {"kernel": (D, self.num_classes), "bias": (self.num_classes,)}
        return p, bs

    def init(self, seed: int, x_shape, device="cuda") -> Params:
        """Fresh variables: lecun-normal conv / dense kernels, zero biases, unit norm scales,
        N(0, 0.02^2) position / register embeddings, BatchNorm running mean 0 / var 1, and each
        cell's own initialisation."""
        ps, bss = self.param_shapes(x_shape)
        gen = torch.Generator(device=device).manual_seed(int(seed))
        H, W = x_shape[-3], x_shape[-2]
        params: Dict[str, Any] = {}
        for name, v in ps.items():
            if name.startswith("cssm_"):
                i = int(name.split("_")[1])
                hs, ws = self._feature_hw(H, W)
                T = self.seq_len if len(x_shape) == 4 else x_shape[1]
                shp = (x_shape[0], T + self.n_register_tokens, hs, ws, self.embed_dim)
                params[name] = self.cells[i].init(seed + 1 + i, shp, device)["params"]
            elif name in ("pos_embed", "register_tokens"):
                params[name] = torch.randn(v, generator=gen, device=device) * 0.02
            else:
                sub = {}
                for pn, shp in v.items():
                    if pn == "kernel":
                        sub[pn] = _lecun_normal(shp, int(math.prod(shp[:-1])), gen, device)
                    elif pn == "scale":
                        sub[pn] = torch.ones(shp, device=device)
                    else:
                        sub[pn] = torch.zeros(shp, device=device)
                params[name] = sub
        out = {"params": params}
        if bss:
            out["batch_stats"] = {n: {"mean": torch.zeros(v["mean"], device=device),
                                      "var": torch.ones(v["var"], device=device)} for n, v in bss.items()}
        return out

    def _feature_hw(self, H, W):
        if self.stem_mode != "pathtracker":
            for _ in range(self.stem_layers):
                H, W = (H + 1) // 2, (W + 1) // 2
        return H, W

    @staticmethod
    def load_params(tree, device="cuda") -> Params:
        """Variables from a tree of arrays ({'params': ..., 'batch_stats': ...} or the params alone),
        e.g. :func:`cssm_amd.checkpoint.load_simple_checkpoint` output."""
        if isinstance(tree, dict) and "params" in tree:
            out = {"params": tree_to_device(tree["params"], device)}
            if tree.get("batch_stats"):
                out["batch_stats"] = tree_to_device(tree["batch_stats"], device)
            return out
        return {"params": tree_to_device(tree, device)}

    # ---------------------------------------------------------------- forward
    def _act(self, x):
        if self.act_type == "gelu":
            return Fn.gelu(x, approximate="tanh")     # jax.nn.gelu's default form
        if self.act_type == "relu":
            return torch.relu(x)
        return Fn.softplus(x)

    @staticmethod
    def _layer_norm(x, p, mode):
        """flax LayerNorm on the HIP block-norm kernels: mode 'layer' per pixel over C,
        'temporal_layer' over (T, C), 'global_layer' over (T, H, W, C) of a (B, T, H, W, C) x."""
        shape = x.shape
        x5 = x.reshape(shape[0], 1, 1, 1, shape[-1]) if x.dim() == 2 else (x.unsqueeze(1) if x.dim() == 4 else x)
        x5 = x5.contiguous()
        stats = S.block_norm_stats(x5, mode)
        out = S.block_norm_posconv(x5, stats, mode, p["scale"], p["bias"], None, None, x5.shape[1])
        return out.reshape(shape)

    def _norm(self, x, kind, name, p, bs, training):
        """_apply_norm (simple_cssm.py:192-235)."""
        q = p[name]
        if kind == "batch":
            if training:
                axes = tuple(range(x.dim() - 1))
                mu = x.mean(dim=axes)
                var = torch.clamp((x * x).mean(dim=axes) - mu * mu, min=0.0)
            else:
                mu, var = bs[name]["mean"], bs[name]["var"]
            return (x - mu) * torch.rsqrt(var + 1e-5) * q["scale"] + q["bias"]
        if kind == "instance":
            # GroupNorm(num_groups=C) reduces over axes 1..ndim-2 and the size-1 within-group axis;
            # on a pooled (B, C) vector each group is one element (mean = x, var = 0): the bias
            axes = tuple(range(1, x.dim() - 1))
            if not axes:
                return (x - x) * (1.0 / math.sqrt(1e-6)) * q["scale"] + q["bias"]
            mu = x.mean(dim=axes, keepdim=True)
            var = torch.clamp((x * x).mean(dim=axes, keepdim=True) - mu * mu, min=0.0)
            return (x - mu) * torch.rsqrt(var + 1e-6) * q["scale"] + q["bias"]
        if x.dim() == 5 and kind == "global_instance":
            mu = x.mean(dim=(1, 2, 3), keepdim=True)
            var = torch.clamp((x * x).mean(dim=(1, 2, 3), keepdim=True) - mu * mu, min=0.0)
            return (x - mu) * torch.rsqrt(var + 1e-6) * q["scale"] + q["bias"]
        if x.dim() == 5 and kind in _LN_MODES:
            return self._layer_norm(x, q, _LN_MODES[kind])
        return self._layer_norm(x, q, "layer")

    @staticmethod
    def _conv(x, p):
        """flax Conv, stride 1, 'SAME', bias; x (N, H, W, Cin), kernel (k, k, Cin, Cout)."""
        k = p["kernel"]
        if k.shape[0] == 1 and k.shape[1] == 1:
            return torch.addmm(p["bias"], x.reshape(-1, x.shape[-1]), k[0, 0]).reshape(*x.shape[:-1], -1)
        kh = k.shape[0]
        lo, hi = (kh - 1) // 2, kh // 2
        xp = Fn.pad(x.permute(0, 3, 1, 2), (lo, hi, lo, hi))
        return Fn.conv2d(xp, k.permute(3, 2, 0, 1).contiguous(), p["bias"]).permute(0, 2, 3, 1).contiguous()

    def apply(self, variables: Params, x: torch.Tensor, training: bool = False, return_spatial: bool = False,
              return_features: bool = False, injected_features: Optional[torch.Tensor] = None,
              injected_qkv_spatial=None, injected_post_cssm: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Logits (B, num_classes) for x (B, T, H, W, C) or an image (B, H, W, C), float32 on the GPU."""
        p = variables["params"]
        bs = variables.get("batch_stats", {})
        stem_norm, body_norm = self._norms()
        x = x.float()
        if x.dim() == 4:                                                    # :239-240
            x = x.unsqueeze(1).expand(-1, self.seq_len, -1, -1, -1)
        B, T, H, W, C = x.shape
        x = x.reshape(B * T, H, W, C).contiguous()

        def norm_act(v, name):                                              # :247-255
            if self.stem_norm_order == "pre":
                return self._act(self._norm(v, stem_norm, name, p, bs, training))
            return self._norm(self._act(v), stem_norm, name, p, bs, training)
        if self.stem_mode == "pathtracker":                                 # :257-264
            if self.stem_norm_order == "pre":
                x = self._conv(norm_act(x, "norm1"), p["conv1"])
            else:
                x = norm_act(self._conv(x, p["conv1"]), "norm1")
        else:                                                               # :266-274
            for i in range(self.stem_layers):
                if self.stem_norm_order == "pre":
                    x = self._conv(norm_act(x, f"norm{i + 1}"), p[f"conv{i + 1}"])
                else:
                    x = norm_act(self._conv(x, p[f"conv{i + 1}"]), f"norm{i + 1}")
                x = Fn.max_pool2d(x.permute(0, 3, 1, 2), 2, 2, ceil_mode=True).permute(0, 2, 3, 1)
        _, Hn, Wn, D = x.shape
        x = x.reshape(B, T, Hn, Wn, D)                                      # :277-278
        if self.pos_embed == "learnable":                                   # :281-285
            x = x + p["pos_embed"]
        nreg = self.n_register_tokens
        if nreg > 0:                                                        # :302-306
            x = torch.cat([p["register_tokens"].expand(B, -1, -1, -1, -1), x], dim=1)
        if injected_features is not None:                                   # :309-310
            x = injected_features
        x = x.contiguous()
        for i, cell in enumerate(self.cells):                               # :319-496
            y = cell.apply({"params": p[f"cssm_{i}"]}, x, injected_qkv_spatial=injected_qkv_spatial)
            x = S.block_residual(x, y, x.shape[1], "none")                  # x + cssm(x), :482
            if self.depth > 1 and i < self.depth - 1:                       # :486-496
                x = self._act(self._norm(x, body_norm, f"body_norm_{i}", p, bs, training))
                if self.inter_mlp_ratio > 0:
                    h = self._act(Fn.linear(x, p[f"mlp_{i}_up"]["kernel"].t(), p[f"mlp_{i}_up"]["bias"]))
                    x = x + Fn.linear(h, p[f"mlp_{i}_down"]["kernel"].t(), p[f"mlp_{i}_down"]["bias"])
                x = x.contiguous()
        if injected_post_cssm is not None:                                  # :500-501
            x = injected_post_cssm
        if return_features:                                                 # :502-503
            return x
        if nreg > 0:                                                        # :507-508
            x = x[:, nreg:]
        x = x.contiguous()
        head = p["head"]
        if return_spatial:                                                  # :510-521
            if self.readout_norm == "pre":
                x = self._act(self._norm(x, body_norm, "norm_pre", p, bs, training))
            else:
                x = self._norm(self._act(x), body_norm, "norm_pre", p, bs, training)
            return Fn.linear(x, head["kernel"].t(), head["bias"])
        if self.frame_readout == "last":                                    # :524-527
            x = x[:, -1].contiguous()
        if self.readout_norm == "pre":                                      # :530-535
            x = self._act(self._norm(x, body_norm, "norm_pre", p, bs, training))
        else:
            x = self._norm(self._act(x), body_norm, "norm_pre", p, bs, training)
        axes = (1, 2) if self.frame_readout == "last" else (1, 2, 3)        # :538-549
        x = x.amax(dim=axes) if self.pool_type == "max" else x.mean(dim=axes)
        x = self._norm(x.contiguous(), body_norm, "norm_post", p, bs, training)   # :552
        return Fn.linear(x, head["kernel"].t(), head["bias"])               # :555

    __call__ = apply
