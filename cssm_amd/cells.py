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


class _DerivedCache:
    """Buffers derived from parameter tensors (K_hat, W_hat, concatenated gate weights).

    An entry is reused only while its source tensors are the same objects at the
    same in-place version: a new parameter tree (a reloaded checkpoint, fresh
    weights) never hits an entry made from an earlier one, even when the
    allocator hands the new tensors the old addresses.  One entry per slot.
    """

    def __init__(self):
        self._slots: Dict[str, Any] = {}

    def get(self, slot: str, sources, extra, make):
        hit = self._slots.get(slot)
        if hit is not None:
            srcs, vers, ex, val = hit
            if (ex == extra and len(srcs) == len(sources)
                    and all(a is b for a, b in zip(srcs, sources))
                    and vers == tuple(t._version for t in sources)):
                return val
        val = make()
        self._slots[slot] = (tuple(sources), tuple(t._version for t in sources), extra, val)
        return val


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
        self._cache = _DerivedCache()

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
        """Floored K_hat for (H, W); recomputed when the kernel tensor or its version changes."""
        k = p["kernel"]
        return self._cache.get("khat", (k,), (H, W, self.spectral_rho),
                               lambda: S.spectral_kernel(k, H, W, self.spectral_rho, squash=True, goom_floor=True,
                                                         scan_order=True))

    def apply(self, variables: Params, x: torch.Tensor, injected_qkv_spatial=None,
              out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
        """y = GatedCSSM(x); x (B, T, H, W, C) float32 or bfloat16 on the GPU, y of x's dtype
        (or ``out_dtype``: float32 is what the reference cell returns for bf16 input, since it
        computes with float32 parameters)."""
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
        # intermediates stay float32 whatever the I/O dtype (the reference computes with fp32
        # params); only x is read and the output written in the I/O dtype
        f32 = torch.float32
        has_conv = self.short_conv_spatial_size > 0 or self.short_conv_size > 0
        # in_proj straight into plane-major x_main and z; SiLU(z) (cssm.py:581) fused here,
        # SiLU(x_main) and ctx too unless the short convolutions come first
        c_scale = S.scan_c_scale(H, W)
        if has_conv:
            xm, z, _ = S.proj_in(x, p["in_proj"]["kernel"], p["in_proj"]["bias"], F, HW, silu_hi=True,
                                 out_dtype=f32)
            u, ctx = S.short_conv(xm.view(B, T, Ci, H, W),
                                  p.get("short_conv_spatial") if self.short_conv_spatial_size > 0 else None,
                                  p.get("short_conv_temporal") if self.short_conv_size > 0 else None)
            del xm
            gates = S.gated_gates(ctx.view(B, T, Ci), p, H, W, self.gate_type, self.gate_activation, c_scale=c_scale)
        else:
            # the gates from ctx in the same call (the gate kernel reduces the projection's sums)
            u, z, _, gates = S.proj_in_gates(x, p["in_proj"]["kernel"], p["in_proj"]["bias"], B, T, H, W, p,
                                             self.gate_type, self.gate_activation, c_scale=c_scale, silu_lo=True,
                                             silu_hi=True, out_dtype=f32)
            u = u.view(B, T, Ci, H, W)
        z = z.view(B, T, Ci, H, W)
        khat = self.spectral_kernel(p, H, W)
        y = S.gated_scan(u, z, gates, khat)
        out = S.proj_out(y.view(F, Ci, HW), p["out_proj"]["kernel"], p["out_proj"]["bias"],
                         out_dtype=out_dtype or x.dtype)
        return out.view(B, T, H, W, self.channels)

    __call__ = apply


class GatedDeltaNetCSSM:
    """GatedDeltaNetCSSM (cssm.py:4264-5141), slow path: the `gdn` cell.

    x -> [qkv_dw] -> qkv_proj (a k x k full-channel conv when qkv_conv_separable is
    False) -> causal short conv + SiLU -> input gates B_k, B_v
    -> rfft2 -> spectral / key L2 norms -> delta-rule recurrence over T with the
    d_k x d_k complex state per (head, bin) -> readout S q -> irfft2 -> RMSNorm
    -> x SiLU(gate_proj(x)) -> output_proj.  Gates alpha / beta / B_k / B_v come
    from the spatial mean of x plus the temporal context encoding.

    Not part of this build (NotImplementedError): rope_mode other than 'none',
    int_attention_mode, cross_freq_conv_size > 0, ssl_proj_dim > 0, the
    static-image fast path and bf16 / fp8 split-precision scans
    (use_complex32/16).  scan_mode and use_log / use_goom select how
    the scan sees the entries of M and Delta, as in the reference
    (cssm.py:4693-4701, 4939-4991): to_goom's 1e-7 floor (the default), none
    (use_log=False, or scan_mode='pallas' at d_k = 2) or log(|x| + 1e-8)
    (use_goom=False); see :func:`spectral.gdn_scan_variant`.
    """

    def __init__(self, channels: int, delta_key_dim: int = 2, kernel_size: int = 11, rope_mode: str = "none",
                 rope_base: float = 10000.0, spectral_rho: float = 0.999, position_independent_gates: bool = False,
                 block_size: int = 1, gate_type: str = "channel", use_goom: bool = True, use_log: bool = True,
                 use_complex32: bool = False, use_complex16: bool = False, scan_mode: str = "associative",
                 ssd_chunk_size: int = 8, learned_init: bool = False, short_conv_size: int = 4,
                 output_norm: str = "rms", use_input_gates: bool = True, output_gate_act: str = "silu",
                 use_spectral_l2_norm: bool = True, qkv_conv_size: int = 1, qkv_conv_separable: bool = True,
                 cross_freq_conv_size: int = 0, no_spectral_clamp: bool = False, int_attention_mode: str = "none",
                 attn_kernel_size: int = 7, int_attn_dim: int = 16, static_image_fast_path: bool = False,
                 num_timesteps: int = 0, ssl_proj_dim: int = 0, gate_proj_bias_init: float = 0.0,
                 dtype=None, param_dtype=None, name: Optional[str] = None):
        unsupported = []
        if rope_mode != "none":
            unsupported.append(f"rope_mode={rope_mode!r}")
        if int_attention_mode != "none":
            unsupported.append(f"int_attention_mode={int_attention_mode!r}")
        if cross_freq_conv_size > 0:
            unsupported.append("cross_freq_conv_size > 0")
        if ssl_proj_dim > 0:
            unsupported.append("ssl_proj_dim > 0")
        if static_image_fast_path:
            unsupported.append("static_image_fast_path")
        if (use_complex32 or use_complex16) and not use_log:
            unsupported.append("split-precision scans (use_complex32/16)")
        if gate_type not in ("dense", "factored", "channel", "scalar"):
            unsupported.append(f"gate_type={gate_type!r}")
        if output_norm not in ("rms", "layer", "none"):
            unsupported.append(f"output_norm={output_norm!r}")
        if unsupported:
            raise NotImplementedError("GatedDeltaNetCSSM: not part of this build: " + ", ".join(unsupported))
        if not 1 <= delta_key_dim <= 4 or channels % delta_key_dim:
            raise ValueError(f"channels={channels} must be divisible by delta_key_dim={delta_key_dim} (1..4)")
        self.channels = channels
        self.delta_key_dim = delta_key_dim
        self.kernel_size = kernel_size
        self.rope_mode = rope_mode
        self.rope_base = rope_base
        self.spectral_rho = spectral_rho
        self.position_independent_gates = position_independent_gates
        self.block_size = block_size
        self.gate_type = gate_type
        self.use_goom = use_goom
        self.use_log = use_log
        self.use_complex32 = use_complex32
        self.use_complex16 = use_complex16
        self.scan_mode = scan_mode
        self.scan_variant = S.gdn_scan_variant(use_log, use_goom, scan_mode, delta_key_dim)
        self.ssd_chunk_size = ssd_chunk_size
        self.learned_init = learned_init
        self.short_conv_size = short_conv_size
        self.output_norm = output_norm
        self.use_input_gates = use_input_gates
        self.output_gate_act = output_gate_act
        self.use_spectral_l2_norm = use_spectral_l2_norm
        self.qkv_conv_size = qkv_conv_size
        self.qkv_conv_separable = qkv_conv_separable
        self.cross_freq_conv_size = cross_freq_conv_size
        self.no_spectral_clamp = no_spectral_clamp
        self.int_attention_mode = int_attention_mode
        self.attn_kernel_size = attn_kernel_size
        self.int_attn_dim = int_attn_dim
        self.static_image_fast_path = static_image_fast_path
        self.num_timesteps = num_timesteps
        self.ssl_proj_dim = ssl_proj_dim
        self.gate_proj_bias_init = gate_proj_bias_init
        self.dtype = dtype
        self.param_dtype = param_dtype
        self.name = name
        self._cache = _DerivedCache()

    # ------------------------------------------------------------- parameters
    def param_shapes(self, H: int, W: int) -> Dict[str, Any]:
        """Flax parameter tree of the slow path (cssm.py:4717-5141)."""
        C, dk = self.channels, self.delta_key_dim
        nh, Wf = C // dk, W // 2 + 1
        s: Dict[str, Any] = {"kernel": (nh, self.kernel_size, self.kernel_size)}
        q = self.qkv_conv_size
        if q > 1 and self.qkv_conv_separable:
            s["qkv_dw"] = {"kernel": (q, q, 1, C), "bias": (C,)}
        # the full-channel conv is one (q, q, C, 3C) Conv under the same name (cssm.py:4750-4753)
        s["qkv_proj"] = ({"kernel": (q, q, C, 3 * C), "bias": (3 * C,)} if q > 1 and not self.qkv_conv_separable
                         else {"kernel": (C, 3 * C), "bias": (3 * C,)})
        if self.short_conv_size > 0:
            for n in ("q", "k", "v"):
                s[f"short_conv_{n}"] = {"kernel": (self.short_conv_size, 1, C), "bias": (C,)}

        def gate(name, spatial):
            gt = self.gate_type
            if gt == "channel":
                s[name] = {"kernel": (1, 1, C, C), "bias": (C,)} if spatial else {"kernel": (C, nh), "bias": (nh,)}
            elif gt == "factored":
                s[f"{name}_h"] = {"kernel": (C, H), "bias": (H,)}
                n = W if spatial else Wf
                s[f"{name}_w"] = {"kernel": (C, n), "bias": (n,)}
            elif gt == "scalar":
                s[name] = {"kernel": (C, 1), "bias": (1,)}
            else:
                n = H * W if spatial else H * Wf
                s[name] = {"kernel": (C, n), "bias": (n,)}
        if self.use_input_gates:
            gate("B_k", True)
            gate("B_v", True)
        s["gate_proj"] = {"kernel": (C, C), "bias": (C,)}
        gate("alpha", False)
        gate("beta", False)
        if self.output_norm == "rms":
            s["rms_scale"] = (C,)
        elif self.output_norm == "layer":
            s["output_layernorm"] = {"scale": (C,), "bias": (C,)}
        s["output_proj"] = {"kernel": (C, C), "bias": (C,)}
        return s

    def init(self, seed: int, x_shape, device="cuda") -> Params:
        """Fresh parameters for inputs (B, T, H, W, C): lecun-normal Dense/Conv kernels,
        zero biases (gate_proj: gate_proj_bias_init), xavier-normal spectral kernel, unit scales."""
        _, _, H, W, _ = x_shape
        gen = torch.Generator(device=device).manual_seed(int(seed))
        params: Dict[str, Any] = {}
        for name, v in self.param_shapes(H, W).items():
            if name == "kernel":
                nh, K, _ = v
                std = math.sqrt(2.0 / (K * nh + K * nh))   # xavier_normal over (K, K) fans of (n_h, K, K)
                params[name] = torch.randn(v, generator=gen, device=device, dtype=torch.float32) * std
                continue
            if name == "rms_scale":
                params[name] = torch.ones(v, dtype=torch.float32, device=device)
                continue
            sub = {}
            for pn, shp in v.items():
                if pn == "kernel":
                    fan_in = shp[0] if len(shp) == 2 else int(np.prod(shp[:-1]))
                    sub[pn] = _lecun_normal(shp, fan_in, gen, device)
                elif pn == "scale":
                    sub[pn] = torch.ones(shp, dtype=torch.float32, device=device)
                else:
                    fill = self.gate_proj_bias_init if name == "gate_proj" else 0.0
                    sub[pn] = torch.full(shp, float(fill), dtype=torch.float32, device=device)
            params[name] = sub
        return {"params": params}

    load_params = staticmethod(GatedCSSM.load_params)

    # ---------------------------------------------------------------- forward
    def spectral_kernel(self, p: Dict[str, Any], H: int, W: int) -> torch.Tensor:
        """W_hat (n_h, H, Wf) (cssm.py:4711-4734); recomputed when the kernel tensor or its version changes."""
        k = p["kernel"]
        return self._cache.get("what", (k,), (H, W, self.spectral_rho, self.no_spectral_clamp),
                               lambda: S.spectral_kernel(k, H, W, self.spectral_rho,
                                                         squash=not self.no_spectral_clamp, goom_floor=False))

    def _channel_input_gate_weights(self, p):
        """B_k | B_v 1x1-conv kernels concatenated to one (C, 2C) Dense (recomputed when a source changes)."""
        kk, kv = p["B_k"]["kernel"], p["B_v"]["kernel"]
        bk, bv = p["B_k"]["bias"], p["B_v"]["bias"]
        C = self.channels
        return self._cache.get("bkv", (kk, kv, bk, bv), None,
                               lambda: (torch.cat([kk.reshape(C, C), kv.reshape(C, C)], dim=1).contiguous(),
                                        torch.cat([bk, bv]).contiguous()))

    def apply(self, variables: Params, x: torch.Tensor, injected_qkv_spatial=None,
              out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
        """y = GatedDeltaNetCSSM(x); x (B, T, H, W, C) float32 or bfloat16 on the GPU, y of x's dtype
        (or ``out_dtype``)."""
        p = variables["params"]
        B, T, H, W, C = x.shape
        if C != self.channels:
            raise ValueError(f"input has {C} channels, the cell {self.channels}")
        dk = self.delta_key_dim
        F, HW = B * T, H * W
        if not S.fft_supported(H, W):
            raise NotImplementedError(f"no spectral transform kernel for {H}x{W} planes")
        x = x.contiguous()
        # intermediates stay float32 whatever the I/O dtype (the reference computes in fp32 params'
        # precision); only x is read and the output written in the I/O dtype
        f32 = torch.float32
        what = self.spectral_kernel(p, H, W)
        # gates from the spatial mean of the layer input (+ temporal encoding); with the qkv conv,
        # the mean comes out of the conv's pass over x where the fused form applies
        full_conv = self.qkv_conv_size > 1 and not self.qkv_conv_separable
        fused = (S.depthwise_conv_mean(x, p["qkv_dw"]["kernel"], p["qkv_dw"]["bias"], out_dtype=f32)
                 if self.qkv_conv_size > 1 and not full_conv else None)
        if fused is not None:
            xq, ctx = fused
        else:
            ctx = S.frame_mean(x)
            xq = (S.depthwise_conv(x, p["qkv_dw"]["kernel"], p["qkv_dw"]["bias"], out_dtype=f32)
                  if self.qkv_conv_size > 1 and not full_conv else x)
        temporal = "none" if self.position_independent_gates else "sinusoid"
        ab, bkv = S.gdn_gates(ctx, p, H, W, dk, self.gate_type, self.use_input_gates, temporal, self.rope_base)
        # q, k, v in plane-major blocks (B, T, 3C, H, W)
        gate_mode, gates = 0, None
        if self.use_input_gates:
            if self.gate_type == "channel":
                wk, bk = self._channel_input_gate_weights(p)
                gates, gate_mode = S.proj_planes(x, wk, bk, F, HW, act="sigmoid", out_dtype=torch.float32), 3
            else:
                gates, gate_mode = bkv, (2 if self.gate_type == "scalar" else 1)
        convs = None
        if self.short_conv_size > 0:
            convs = [p["short_conv_q"], p["short_conv_k"], p["short_conv_v"]]
        # qkv_proj with the short conv, SiLU and input gates in its epilogue.  gate_proj: where the widths
        # allow, the output projection computes it from x (its planes never reach HBM); otherwise, without
        # the qkv conv, as more columns of the qkv launch (x read once), else a projection of its own
        gact = "silu" if self.output_gate_act == "silu" else "sigmoid"
        xgate = S.gdn_proj_out_xgate_supported(C, C, HW)
        gv = None
        if full_conv:
            # k x k conv with full channel mixing (im2col rows through the projection GEMM), then the
            # short conv, SiLU and input gates in place on its planes
            qkv = S.conv_full_planes(x.view(F, H, W, C), p["qkv_proj"]["kernel"], p["qkv_proj"]["bias"])
            qkv = S.gdn_qkv_post(qkv.view(B, T, 3 * C, H, W), convs, gate_mode, gates)
            if not xgate:
                gv = S.proj_planes(x, p["gate_proj"]["kernel"], p["gate_proj"]["bias"], F, HW, act=gact,
                                   out_dtype=f32)
        elif xgate:
            qkv = S.gdn_qkv_proj(xq, p["qkv_proj"]["kernel"], p["qkv_proj"]["bias"], B, T, H, W, convs, gate_mode,
                                 gates, out_dtype=f32)
        elif xq is x:
            qkv, gv = S.gdn_qkv_gate_proj(x, p["qkv_proj"]["kernel"], p["qkv_proj"]["bias"], B, T, H, W, convs,
                                          gate_mode, gates, p["gate_proj"]["kernel"], p["gate_proj"]["bias"], gact,
                                          out_dtype=f32)
        else:
            qkv = S.gdn_qkv_proj(xq, p["qkv_proj"]["kernel"], p["qkv_proj"]["bias"], B, T, H, W, convs, gate_mode,
                                 gates, out_dtype=f32)
            gv = S.proj_planes(x, p["gate_proj"]["kernel"], p["gate_proj"]["bias"], F, HW, act=gact, out_dtype=f32)
        del xq, gates
        # spectral core: rfft2 -> delta-rule recurrence -> irfft2, in one kernel where a workgroup
        # holds a head's state (32 x 32, d_k = 4), else through spectra in HBM
        if S.gdn_core_fused_supported(H, W, dk):
            o = S.gdn_core_fused(qkv, self.use_spectral_l2_norm, ab, self.gate_type, what, dk, self.scan_variant)
            del qkv
        else:
            spec, norms = S.rfft2(qkv, want_norms=self.use_spectral_l2_norm)
            del qkv
            ohat = S.gdn_scan_bins(spec, norms, ab, self.gate_type, what, dk, self.scan_variant)
            del spec
            o = S.irfft2(ohat, W, out_dtype=f32)
            del ohat
        if self.output_norm == "rms":
            ns, nb = p["rms_scale"], None
        elif self.output_norm == "layer":
            ns, nb = p["output_layernorm"]["scale"], p["output_layernorm"]["bias"]
        else:
            ns = nb = None
        if xgate:
            out = S.gdn_proj_out_xgate(o.view(F, C, HW), x, self.output_norm, ns, nb, p["gate_proj"]["kernel"],
                                       p["gate_proj"]["bias"], gact, p["output_proj"]["kernel"],
                                       p["output_proj"]["bias"], out_dtype=out_dtype or x.dtype)
        else:
            out = S.gdn_proj_out(o.view(F, C, HW), gv, self.output_norm, ns, nb, p["output_proj"]["kernel"],
                                 p["output_proj"]["bias"], out_dtype=out_dtype or x.dtype)
        return out.view(B, T, H, W, C)

    __call__ = apply
