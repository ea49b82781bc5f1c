/*
 * cssm_amd.h -- C ABI of the MI355X (gfx950) spectral state-space layer.
 *
 * Drop-in boundary for the hot path of drewlinsley/CSSM: the `gated`
 * (GatedCSSM, Mamba-SCSSM) and `gdn` (GatedDeltaNetCSSM) cells of
 * src/models/cssm.py.  The reference is pure JAX/Flax and has no native FFI;
 * each entry point below replaces the span of reference code cited beside it,
 * so a binding (ctypes, jax.ffi custom call) can swap that span for one call.
 *
 * Conventions
 *   - Plain pointers to DEVICE memory, sizes as ints; no torch/JAX types.
 *   - `stream` is a hipStream_t passed as void* (NULL = default stream).  All
 *     work is enqueued on it; no entry point synchronises the device.
 *   - Entry points never allocate device memory and never abort or throw: they
 *     return CSSM_OK (0) or a negative cssm_status; cssm_last_error() gives a
 *     message for the calling thread.
 *   - Tensors are row-major.  "plane-major" means (B, T, C, H, W): every
 *     (b, t, c) plane is one contiguous H x W image.  The reference layout is
 *     channels-last (B, T, H, W, C); the projection entry points convert.
 *   - Complex tensors are interleaved (re, im) float32.  Wf = W/2 + 1.
 *   - Stateless and re-entrant; calls on one stream are ordered.
 */
#ifndef CSSM_AMD_H_
#define CSSM_AMD_H_

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* 3: K_hat's scan layout (cssm_spectral_kernel scan_order = 1) pairs rows at 128 x 128
 *    (cssm_gated_scan_khat_order).
 * 4: scan_variant arguments of the GDN delta-rule entry points.
 * 5: cssm_im2col_same, cssm_gdn_proj_out_xgate.
 * 6: cssm_gated_gates_bwd.
 * 7: cssm_proj_in_gates.
 * 8: x_dtype argument of cssm_gdn_proj_out_xgate (fp32 layer input). */
#define CSSM_ABI_VERSION 8

typedef enum cssm_status {
  CSSM_OK = 0,
  CSSM_ERR_NULL = -1,        /* a required pointer is NULL */
  CSSM_ERR_SHAPE = -2,       /* non-positive or inconsistent sizes */
  CSSM_ERR_UNSUPPORTED = -3, /* valid request this build has no kernel for */
  CSSM_ERR_ARG = -4,         /* bad enum value or flag */
  CSSM_ERR_ALIGN = -5,       /* pointer not aligned as the kernel requires */
  CSSM_ERR_HIP = -6          /* HIP runtime reported an error at launch */
} cssm_status;

typedef enum cssm_dtype { CSSM_F32 = 0, CSSM_BF16 = 1 } cssm_dtype;

/* gate_type of GatedCSSM (cssm.py:430, :538-545) */
typedef enum cssm_gate_type { CSSM_GATE_DENSE = 0, CSSM_GATE_FACTORED = 1 } cssm_gate_type;

/* gate_activation of GatedCSSM._compute_gate (cssm.py:432-441) */
typedef enum cssm_gate_act {
  CSSM_ACT_SOFTPLUS = 0, /* softplus(x)            */
  CSSM_ACT_SIGMOID2 = 1, /* 2 * sigmoid(x)         */
  CSSM_ACT_EXP = 2       /* exp(clip(x, -4, 2))    */
} cssm_gate_act;

/* elementwise activation applied when an input plane is loaded */
typedef enum cssm_load_act { CSSM_LOAD_IDENTITY = 0, CSSM_LOAD_SILU = 1 } cssm_load_act;

/* cssm_proj_in's act_lo only: store the lower half as it is (pre-activation), take ctx as the
 * spatial mean of its SiLU -- what the training path needs, which keeps the pre-activations for
 * the SiLU's backward and applies the SiLU when the scan loads them. */
#define CSSM_PROJ_STORE_PRE_CTX_SILU 3

/*
 * Gate projection weights of GatedCSSM (Flax parameter names in brackets).
 * Index 0 = delta_proj, 1 = B_proj, 2 = C_proj.
 *   dense    (cssm.py:545): kernel[i] (C, H*Wf) [<name>/kernel], bias[i] (H*Wf) [<name>/bias];
 *            kernel_w / bias_w unused.
 *   factored (cssm.py:541-543): kernel[i] (C, H) [<name>_h/kernel], bias[i] (H) [<name>_h/bias],
 *            kernel_w[i] (C, Wf) [<name>_w/kernel], bias_w[i] (Wf) [<name>_w/bias].
 */
typedef struct cssm_gate_params {
  int gate_type;  /* cssm_gate_type */
  int activation; /* cssm_gate_act */
  const float* kernel[3];
  const float* bias[3];
  const float* kernel_w[3];
  const float* bias_w[3];
} cssm_gate_params;

/* ABI version of the loaded library (CSSM_ABI_VERSION it was built with). */
int cssm_abi_version(void);

/* Static description of a status code. */
const char* cssm_strerror(int status);

/* Message of the last failing call made by this thread ("" if none). */
const char* cssm_last_error(void);

/*
 * Spectral kernel K_hat = rho * F / (1 + |F|), F = rfft2(pad(k)).
 * Replaces cssm.py:505-529 (GatedCSSM kernel pad + rfft2 + squash, helper
 * _stable_spectral_magnitude :29-46) and cssm.py:4711-4716 (GatedDeltaNetCSSM).
 *   k     (C, K, K) float32 spatial kernel [params 'kernel']
 *   khat  (C, H, Wf) complex64 out
 *   squash      1 = apply rho/(1+|F|) (0 = GDN no_spectral_clamp, cssm.py:4715)
 *   goom_floor  1 = replace |K_hat| < 1e-7 by 1e-7+0j (to_goom floor, goom.py:161-174),
 *               which is what the scan consumes.
 *   scan_order  1 = the scan layout cssm_gated_scan_fwd reads: columns in the
 *               order of cssm_gated_scan_col_order, each channel's bins in the
 *               slots of cssm_gated_scan_khat_order (row-major except at
 *               128 x 128); 0 = natural (C, H, Wf) order.
 * Pad rule: K <= H, W zero-pads with (H-K)//2 before; K >= H and K >= W
 * centre-crops from (K-H)//2.  K between H and W is rejected (the reference
 * produces mismatched shapes there).
 */
int cssm_spectral_kernel(const float* k, int C, int K, int H, int W, float rho, int squash,
                         int goom_floor, int scan_order, float* khat, void* stream);

/*
 * Spatial mean of every H x W plane: out[i] = mean(act(x[i, :, :])).
 * Replaces cssm.py:536 (ctx = x_main.mean(axis=(2, 3))) for plane-major x.
 *   x (nplanes, H, W) of dtype; out (nplanes) float32; act = cssm_load_act.
 */
int cssm_plane_mean(const void* x, int dtype, long long nplanes, int H, int W, int act,
                    float* out, void* stream);

/*
 * Per-frequency gates of GatedCSSM from ctx, with the GOOM shifts folded in.
 * Replaces cssm.py:538-556 (_make_gate for delta_proj, B_proj, C_proj and
 * _compute_gate) and the Delta terms of cssm.py:559-567.
 *   ctx   (B, T, C) float32
 *   gates (B, T, H, Wf, 4) float32 out: the per-bin planes cssm_gated_scan_fwd
 *         reads.  Position p of row u holds bin (u, v = cols[p]) of
 *         cssm_gated_scan_col_order, as
 *         [exp(-Delta), (Delta + 1e-8) B, 2e-7 (Delta + 1e-8), C * c_scale]
 *         = decay, input gain, the input term that replaces (Delta + 1e-8) 2 U B
 *         when |U B| < 1e-7 (the to_goom floor; the scan's forward transform
 *         yields 2 U, so the floor term is doubled), readout gain.
 * c_scale = 1 gives the reference C; cssm_gated_scan_fwd expects
 * c_scale = 1 / (2 H W) (the irfft2 normalisation and the 1/2 of the doubled
 * spectrum folded into C).
 */
int cssm_gated_gates(const float* ctx, int B, int T, int C, int H, int W,
                     const cssm_gate_params* params, float c_scale, float* gates, void* stream);

/*
 * Adjoint of cssm_gated_gates for training: what autodiff of cssm.py:536-567
 * (the gate projections, the activation and the GOOM shifts) hands back for
 * the gate pre-activations, given dgates (B, T, H, Wf, 4) float32, the
 * gradient of the gates output (same layout).  Per bin, with Delta = act(G_delta):
 *   dG_delta = (-exp(-Delta) dg0 + G_B dg1 + 2e-7 dg2) act'(G_delta)
 *   dG_B = (Delta + 1e-8) dg1,  dG_C = c_scale dg3
 * out, float32:
 *   dense:    (B, T, 3, H * Wf), dG of delta / B / C at bin u * Wf + v
 *             (natural column order);
 *   factored: (B, T, 3, H + Wf), the gradients of the row factors
 *             ctx . kernel + bias (first H) and the column factors
 *             ctx . kernel_w + bias_w (last Wf), each a sum in a fixed order.
 * The kernel, bias and ctx gradients are then GEMMs of out with ctx and the
 * gate kernels over the B*T frames (no per-call state; deterministic).
 * Same params and c_scale as the forward call.
 */
int cssm_gated_gates_bwd(const float* ctx, int B, int T, int C, int H, int W,
                         const cssm_gate_params* params, float c_scale, const float* dgates, float* out,
                         void* stream);

/*
 * Fused spectral scan of GatedCSSM for one layer call:
 *   U_t = rfft2(u_t); h_t = floor(K_hat) e^{-Delta_t} h_{t-1} + (Delta_t + 1e-8) floor(U_t B_t);
 *   y_t = irfft2(C_t h_t, s=(H, W)) * z_t          (h_{-1} = 0, all t in [0, T))
 * Replaces cssm.py:531-533 and 559-581 (rfft2, to_goom, Delta shifts,
 * jax.lax.associative_scan(cssm_scalar_scan_op), from_goom, x C, irfft2,
 * x SiLU(z)); math.py:24-54 and operations.py:17-41 are the combiner it
 * evaluates exactly (the log-space scan is this linear recurrence).
 *   u, z, y   (B, T, C, H, W) plane-major of dtype; u = x_main after the short
 *             convolutions, z = the gate branch; u_act / z_act select SiLU on
 *             load (the reference applies SiLU to both, cssm.py:502, :581).
 *   gates     (B, T, H, Wf, 4) from cssm_gated_gates with c_scale = 1/(2 H W)
 *             (the irfft2 normalisation and the 1/2 of the doubled spectrum
 *             folded into C); dense and factored gate_type both arrive in this
 *             per-bin form, columns in the order of cssm_gated_scan_col_order.
 *   khat      from cssm_spectral_kernel with goom_floor = 1 and scan_order = 1,
 *             C channels
 * Supported planes: H = W in {4, 8, 16, 32, 64, 128} (in-register FFT passes
 * through LDS; C a multiple of cssm_gated_scan_min_group(H, W)) and any
 * H = W in 3..15 (direct DFTs, any C) -- the CSSM-SHViT stage shapes 14 x 14
 * and 7 x 7.  u, z, y must be 16-byte aligned (f32) or 8-byte aligned (bf16);
 * gates 16; khat 8.
 */
int cssm_gated_scan_fwd(const void* u, const void* z, void* y, int dtype, int B, int T, int C,
                        int H, int W, const float* gates, const float* khat, int u_act,
                        int z_act, void* stream);

/*
 * Backward of cssm_gated_scan_fwd (with u_act = z_act = identity): the
 * spectral-domain reverse recurrence.  Replaces the gradient jax.value_and_grad
 * takes through cssm.py:531-581 (main.py:283; the log-space scan's custom VJPs,
 * goom.py:47-137) -- the reverse scan over conj(A) of the linear recurrence.
 * The caller runs the transforms' adjoints as batched FFTs around it:
 *   uspec = cssm_rfft2(u), dspec = cssm_rfft2(dy) with dy = dL/dy * z (the
 *   gradient at irfft2's output), and afterwards y_pre = cssm_irfft2(yspec)
 *   (so dL/dz = dL/dy * y_pre) and dL/du = cssm_irfft2(sdu).
 *   uspec, dspec     (B, T, C, H, Wf) complex64, natural column order
 *   gates, khat      exactly as cssm_gated_scan_fwd read them (scan layout)
 *   c_scale          the c_scale the gate planes were made with (1 / (2 H W))
 *   yspec  (B, T, C, H, Wf) out: C h_t                  (natural order)
 *   sdu    (B, T, C, H, Wf) out: dL/dU_t H W / c_v      (natural order; c_v = 1 at v = 0 and at
 *          v = W/2 for even W, else 2)
 *   dgates (B, T, H, Wf, 4) out: dL/d(gate planes), summed over channels (scan order)
 *   dkhat  (B, C, H, Wf)    out: dL/dkhat per batch element (sum over B; khat's scan layout)
 * T <= 32; any H, W (odd W has no Nyquist column).
 */
int cssm_gated_scan_bwd(const float* uspec, const float* dspec, const float* gates, const float* khat, int B, int T,
                        int C, int H, int W, float c_scale, float* yspec, float* sdu, float* dgates, float* dkhat,
                        void* stream);

/*
 * Input projection with the layout change to plane-major fused in.
 * Replaces cssm.py:480-484 (in_proj = Dense(2C) on channels-last x, split
 * into x_main and z), with the SiLU of cssm.py:502 / :581 optionally applied
 * to each half and the spatial mean ctx of the first half (cssm.py:536)
 * optionally produced.  Also serves the GDN projections (cssm.py:4753-4758,
 * 4853) with N = 3C or C.
 *   x        (F * HW, K) channels-last of in_dtype (F = B * T frames)
 *   kernel   (K, N) float32 [in_proj/kernel], bias (N) [in_proj/bias]
 *   out_lo   (F, N/2, HW) plane-major of out_dtype: output channels [0, N/2)
 *   out_hi   (F, N/2, HW): output channels [N/2, N) (N must be even)
 *   act_lo, act_hi  cssm_load_act applied to each half; act_lo may also be
 *            CSSM_PROJ_STORE_PRE_CTX_SILU (out_lo stored without activation, ctx of its SiLU)
 *   ctx      (F, N/2) float32 out = mean over HW of out_lo, or NULL (summed in fp32; with a
 *            bf16 out_lo the sums may be taken before or after its rounding)
 *   workspace  device scratch of cssm_proj_in_workspace_size(F, HW, K, N) bytes
 *              (used only when ctx is requested)
 * x must be 16-byte aligned (f32) or 8-byte aligned (bf16), f32 outputs 16-byte
 * aligned (CSSM_ERR_ALIGN otherwise).
 */
int cssm_proj_in(const void* x, int in_dtype, int F, int HW, int K, int N, const float* kernel,
                 const float* bias, void* out_lo, void* out_hi, int out_dtype, int act_lo, int act_hi,
                 float* ctx, void* workspace, size_t workspace_bytes, void* stream);

/*
 * cssm_proj_in followed by cssm_gated_gates on its ctx, for the gated cell without short
 * convolutions: replaces cssm.py:480-484 (in_proj), :536 (ctx) and :538-567 (gates) in one
 * call.  Where the projection kernel takes the frames' channel sums on the way
 * (cssm_proj_in_workspace_size(B * T, H * W, K, N) > 0), the gate kernel reduces them per
 * frame itself instead of a separate reduction launch; ctx is written either way.
 *   x, kernel, bias, out_lo, out_hi, out_dtype, act_lo, act_hi  as cssm_proj_in with
 *            F = B * T frames of HW = H * W pixels
 *   ctx      (B, T, N/2) float32 out (required)
 *   params, c_scale, gates  as cssm_gated_gates with C = N / 2
 *   workspace  device scratch of cssm_proj_in_workspace_size(B * T, H * W, K, N) bytes
 * Same results as the two calls, bit for bit.
 */
int cssm_proj_in_gates(const void* x, int in_dtype, int B, int T, int H, int W, int K, int N, const float* kernel,
                       const float* bias, void* out_lo, void* out_hi, int out_dtype, int act_lo, int act_hi,
                       float* ctx, const cssm_gate_params* params, float c_scale, float* gates, void* workspace,
                       size_t workspace_bytes, void* stream);

/* Bytes of device workspace cssm_proj_in needs to produce ctx. */
size_t cssm_proj_in_workspace_size(int F, int HW, int K, int N);

/* Size of the static device scratch of cssm_proj_in_noalloc (64 MiB per device). */
#define CSSM_PROJ_IN_SCRATCH_BYTES (64u << 20)

/*
 * cssm_proj_in without a workspace argument: the same kernels and results, with
 * the ctx partial sums in a static device array of CSSM_PROJ_IN_SCRATCH_BYTES
 * (one per device, held until the process ends).  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, hosts that forbid allocation).  It
 * calls no allocating routine.
 *   Arguments as cssm_proj_in.  ctx is rejected with CSSM_ERR_UNSUPPORTED when
 *   cssm_proj_in_workspace_size(F, HW, K, N) exceeds the scratch (C2's
 *   F = 1024 frames of 128 x 128 at K = 64, N = 128 need 32 MiB).
 *   The first call on a device, with that device current, looks up the array's
 *   device address; stream must belong to the current device.
 * Every call on one device shares its scratch: calls that overlap on one GPU
 * (different streams, or host threads) race and must be serialised by the
 * caller.  Each call writes every partial sum it reads, so nothing needs clearing.
 */
int cssm_proj_in_noalloc(const void* x, int in_dtype, int F, int HW, int K, int N, const float* kernel,
                         const float* bias, void* out_lo, void* out_hi, int out_dtype, int act_lo, int act_hi,
                         float* ctx, void* stream);

/*
 * Output projection from plane-major planes back to channels-last.
 * Replaces cssm.py:584 (out_proj = Dense(C) on the channels-last transpose
 * of the scan output, cssm.py:578).
 *   y       (F, K, HW) plane-major of in_dtype
 *   kernel  (K, N) float32, bias (N)
 *   out     (F * HW, N) channels-last of out_dtype
 * y must be 16-byte aligned (f32) or 8-byte aligned (bf16), a f32 out 16-byte aligned.
 */
int cssm_proj_out(const void* y, int in_dtype, int F, int HW, int K, int N, const float* kernel,
                  const float* bias, void* out, int out_dtype, void* stream);

/*
 * Factored short convolution + SiLU + spatial mean of GatedCSSM.
 * Replaces cssm.py:487-502 and :536 for plane-major x_main:
 *   s_t = DWConv_{ks x ks, SAME}(x_t) + b_s; o_t = sum_j w_t[j] s_{t-kt+1+j} + b_t;
 *   u_t = SiLU(o_t); ctx_t = mean_{h,w} u_t.
 *   x   (B, T, C, H, W) of in_dtype; u (B, T, C, H, W) of out_dtype; ctx (B, T, C) or NULL
 *   ks = 0 skips the spatial stage (ws, bs unused): kernel (ks, ks, 1, C)
 *        [short_conv_spatial/kernel], bias (C)
 *   kt = 0 skips the temporal stage (wt, bt unused): kernel (kt, 1, C)
 *        [short_conv_temporal/kernel], bias (C)
 */
int cssm_short_conv(const void* x, int in_dtype, int B, int T, int C, int H, int W, int ks,
                    const float* ws, const float* bs, int kt, const float* wt, const float* bt,
                    void* u, int out_dtype, float* ctx, void* stream);

/*
 * Dense projection of channels-last rows into ONE plane-major tensor.
 * Replaces the GDN projections qkv_proj (cssm.py:4753-4758, N = 3C: q, k, v
 * blocks), gate_proj + SiLU / sigmoid (:4853-4859, N = C) and the per-pixel
 * 1x1-conv input gates of gate_type 'channel' (:4800-4806, N = 2C, sigmoid).
 *   x      (F * HW, K) channels-last of in_dtype
 *   kernel (K, N) float32, bias (N)
 *   out    (F, N, HW) plane-major of out_dtype; act 0 identity, 1 SiLU, 2 sigmoid
 * x must be 16-byte aligned (f32) or 8-byte aligned (bf16), a f32 out 16-byte aligned.
 */
int cssm_proj_planes(const void* x, int in_dtype, int F, int HW, int K, int N, const float* kernel,
                     const float* bias, void* out, int out_dtype, int act, void* stream);

/*
 * Spatial mean of channels-last frames: out[f, c] = mean_p x[f, p, c].
 * Replaces cssm.py:4785 (ctx = gate_input.mean(axis=(2, 3)) of the GDN cell).
 *   x (F, HW, C) of dtype; out (F, C) float32
 */
int cssm_frame_mean(const void* x, int dtype, int F, int HW, int C, float* out, void* stream);

/*
 * Depthwise ks x ks SAME convolution of channels-last frames with bias.
 * Replaces qkv_dw (cssm.py:4744-4750; Flax 'SAME' pads (ks-1)//2 before).
 *   x (F, H, W, C) of dtype, out (F, H, W, C) of out_dtype; kernel (ks, ks, 1, C) [qkv_dw/kernel], bias (C)
 */
int cssm_depthwise_conv(const void* x, int dtype, int F, int H, int W, int C, int ks, const float* kernel,
                        const float* bias, void* out, int out_dtype, void* stream);

/*
 * cssm_depthwise_conv and cssm_frame_mean of the same x in one pass, where the
 * GDN cell has a qkv conv (cssm.py:4744-4750 and the context mean :4785 both
 * read the layer input): the conv's threads also add x at their own output
 * pixels, each block sums its threads in a fixed order into the workspace, and
 * a second small kernel adds a frame's blocks in order and divides by H*W
 * (the same sums as cssm_frame_mean up to the order of the additions).
 *   workspace  cssm_depthwise_conv_mean_workspace(F, H, W, C, ks) floats, 16-byte aligned
 *   ctx        (F, C) float32 out
 * Other arguments as cssm_depthwise_conv; kernel and bias 16-byte aligned.  Returns
 * CSSM_ERR_UNSUPPORTED where the workspace query returns 0 (the caller then runs the two calls).
 */
long long cssm_depthwise_conv_mean_workspace(int F, int H, int W, int C, int ks);
int cssm_depthwise_conv_mean(const void* x, int dtype, int F, int H, int W, int C, int ks, const float* kernel,
                             const float* bias, void* out, int out_dtype, float* workspace, float* ctx,
                             void* stream);

/* gate_type of GatedDeltaNetCSSM (cssm.py:4798-4842) */
typedef enum cssm_gdn_gate_type {
  CSSM_GDN_GATE_DENSE = 0,
  CSSM_GDN_GATE_FACTORED = 1,
  CSSM_GDN_GATE_CHANNEL = 2,
  CSSM_GDN_GATE_SCALAR = 3
} cssm_gdn_gate_type;

/*
 * Gate weights of GatedDeltaNetCSSM.  Index 0 = alpha, 1 = beta (spectral
 * gates), 2 = B_k, 3 = B_v (spatial input gates; kernel[2] = NULL skips them).
 *   dense    kernel[i] (C, n) [<name>/kernel], bias[i] (n): n = H*Wf (spectral), H*W (spatial)
 *   factored kernel[i] (C, H) [<name>_h/kernel], bias[i] (H); kernel_w[i] (C, Wf or W) [<name>_w/kernel],
 *            bias_w[i]; gate = sigmoid(row[u] + col[v])
 *   channel  alpha / beta: kernel (C, n_h), bias (n_h); B_k / B_v are per-pixel 1x1 convolutions of x,
 *            computed with cssm_proj_planes (act = sigmoid), so kernel[2] must be NULL here
 *   scalar   kernel (C, 1), bias (1)
 */
typedef struct cssm_gdn_gate_params {
  int gate_type; /* cssm_gdn_gate_type */
  const float* kernel[4];
  const float* bias[4];
  const float* kernel_w[4];
  const float* bias_w[4];
} cssm_gdn_gate_params;

/*
 * Gates of GatedDeltaNetCSSM from ctx.  Replaces cssm.py:4785-4869: the
 * temporal context encoding (apply_temporal_rope_to_context :353-383, or the
 * learned table), _gate (:4798-4842) for B_k / B_v (:4844-4848) and alpha /
 * beta (:4864-4865): alpha = 0.1 + 0.89 sigmoid(g), beta = sigmoid(g).
 *   ctx       (B, T, C) float32 (cssm_frame_mean of the layer input)
 *   temporal  0 none (position_independent_gates), 1 sinusoid table E[t] with rope_base,
 *             2 learned table temporal_table (T, C) [temporal_embed]
 *   ab        (B, T, n_ab, 2) float32 out (alpha, beta): n_ab = H*Wf (dense, factored), n_h (channel), 1 (scalar)
 *   bkv       (B, T, n_kv, 2) float32 out (B_k, B_v): n_kv = H*W (dense, factored), 1 (scalar); may be NULL
 */
int cssm_gdn_gates(const float* ctx, int B, int T, int C, int H, int W, int delta_key_dim,
                   const cssm_gdn_gate_params* params, int temporal, float rope_base,
                   const float* temporal_table, float* ab, float* bkv, void* stream);

/*
 * In place on the plane-major q, k, v blocks qkv (B, T, 3C, H, W): causal
 * depthwise short convolution over T + bias + SiLU (cssm.py:4763-4780; kt = 0
 * skips both), then the input gates on k and v (:4844-4848).
 *   conv_kernel[3] (kt, 1, C) [short_conv_q/k/v/kernel], conv_bias[3] (C); kt <= 8
 *   gate_mode 0 none; 1 gates (B, T, H*W, 2) per pixel; 2 gates (B, T, 2) per frame;
 *             3 gates (B, T, 2C, H, W) per channel and pixel (B_k then B_v)
 */
int cssm_gdn_qkv_post(void* qkv, int dtype, int B, int T, int C, int H, int W, int kt,
                      const float* const* conv_kernel, const float* const* conv_bias, int gate_mode,
                      const void* gates, void* stream);

/*
 * qkv projection of GatedDeltaNetCSSM with the causal short convolution, SiLU
 * and input gates of cssm_gdn_qkv_post fused into the GEMM's epilogue:
 *   qkv = post(proj(x)),  proj = cssm_proj_planes with N = 3C (identity act).
 * Replaces cssm.py:4753-4758 (qkv_proj), :4763-4780 and :4844-4848 in one pass
 * over qkv instead of three.  Fused when cssm_gdn_qkv_fused(T, H, W, K, kt)
 * (K <= 64, K % 4 == 0): any T with kt <= 4 or T <= 4 and H*W a multiple of 64
 * (tiles of 64 pixels of one frame, a workgroup walking the frames in order with
 * the three previous frames' projections in registers; 3C*H*W elements of
 * out_dtype under 2^31 bytes); else T = 4, or a multiple of 8 with kt <= 4, and
 * H*W a multiple of 128 / min(T, 8) (tiles of pixels x frames, chunks of 8 frames
 * carrying 3); otherwise it runs the two calls it replaces, with the same
 * results (fp32 qkv; a bf16 qkv then holds the projection in bf16 before the
 * convolution, where the fused path keeps it in fp32).
 *   x      (B, T, H*W, K) channels-last of in_dtype
 *   kernel (K, 3C) [qkv_proj/kernel], bias (3C) [qkv_proj/bias]
 *   kt, conv_kernel, conv_bias, gate_mode, gates: as cssm_gdn_qkv_post
 *   qkv    (B, T, 3C, H, W) plane-major of out_dtype out
 * x and qkv must be 16-byte aligned (f32) or 8-byte aligned (bf16); gates 8 (mode 1) or 16 (mode 3).
 */
int cssm_gdn_qkv_proj(const void* x, int in_dtype, int B, int T, int H, int W, int K, int C,
                      const float* kernel, const float* bias, int kt, const float* const* conv_kernel,
                      const float* const* conv_bias, int gate_mode, const void* gates, void* qkv,
                      int out_dtype, void* stream);

/*
 * cssm_gdn_qkv_proj and gate_proj of the same x in one call: besides qkv,
 *   gv = act(x gate_kernel + gate_bias)   (cssm.py:4853-4859, act 1 SiLU, 2 sigmoid)
 * where the layer has no qkv conv (qkv_conv_size <= 1, cssm.py:4740 / :4754),
 * so both projections read the layer input x_flat.  When the qkv projection runs fused, the C
 * gate columns are C more columns of the same launch (no conv, no input gate):
 * x is read once; otherwise a second projection computes gv.  Results equal
 * cssm_gdn_qkv_proj + cssm_proj_planes(act) on the same x.
 *   gate_kernel (K, C) [gate_proj/kernel], gate_bias (C) [gate_proj/bias]
 *   gv          (B, T, C, H, W) plane-major of out_dtype out, aligned as qkv
 * Other arguments and requirements as cssm_gdn_qkv_proj.
 */
int cssm_gdn_qkv_gate_proj(const void* x, int in_dtype, int B, int T, int H, int W, int K, int C,
                           const float* kernel, const float* bias, int kt, const float* const* conv_kernel,
                           const float* const* conv_bias, int gate_mode, const void* gates,
                           const float* gate_kernel, const float* gate_bias, int gate_act, void* qkv, void* gv,
                           int out_dtype, void* stream);

/* 1 if cssm_gdn_qkv_proj runs fused for (T, H, W, K, kt), else 0 (it then runs two kernels). */
int cssm_gdn_qkv_fused(int T, int H, int W, int K, int kt);

/*
 * Batched 2-D real FFT (numpy / XLA rfft2 convention) of P planes, with the
 * optional per-plane sum of |X|^2 over the half spectrum (the spectral L2 norm
 * of cssm.py:4890-4897).  Replaces the rfft2 calls of cssm.py:4880-4888.
 *   x (P, H, W) of dtype; spec (P, H, Wf) complex64 out; norms (P) float32 out or NULL
 * Supported planes: H = W in {4, ..., 128} (powers of two: in-register radix
 * passes) or in 3..15 (direct DFTs: the 14 x 14 / 7 x 7 CSSM-SHViT stages), any
 * P.  x 16-byte (f32) / 8-byte (bf16) aligned, spec 8.
 */
int cssm_rfft2(const void* x, int dtype, long long P, int H, int W, float* spec, float* norms, void* stream);

/*
 * Batched inverse 2-D real FFT (numpy / XLA irfft2, s = (H, W): only the
 * Hermitian part of the v = 0 and v = W/2 columns survives).  Replaces
 * cssm.py:5025.  spec (P, H, Wf) complex64; y (P, H, W) of dtype out.
 */
int cssm_irfft2(const float* spec, long long P, int H, int W, void* y, int dtype, void* stream);

/* 1 if cssm_rfft2 / cssm_irfft2 have a kernel for (H, W) planes, else 0. */
int cssm_fft_min_group(int H, int W);

/*
 * The transforms of the gated cell's training backward (the reference takes
 * these gradients with jax.value_and_grad through cssm.py:502-581, main.py:283)
 * with the elementwise work around them fused into their load and store
 * phases.  float32 planes are addressed as strided sets: plane p = f*C + c of
 * a set (ptr, fs) starts at ptr + (f*fs + c)*H*W, so the halves of a
 * plane-major (F, 2C, H*W) tensor are sets with fs = 2C.  P planes, a
 * multiple of C; H = W a power of two 4..128 (cssm_fft_ex_supported); sets
 * 16-byte aligned with fs >= C; spec (P, H, W/2+1) complex64, 8-byte aligned.
 *   cssm_rfft2_ex   spec = rfft2(x_act(x) * a_act(a)); a may be NULL (factor 1)
 *                   (x_act, a_act: cssm_load_act)
 *   cssm_irfft2_ex  y = (irfft2(spec) + add[p]) * m * SiLU'(d), each of add
 *                   (P floats), m and d optional (NULL); SiLU'(v) = s (1 + v (1 - s)),
 *                   s = sigmoid(v); sums (P floats, optional) receives each plane's sum of
 *                   y, in a fixed order (where cssm_irfft2_ex_sums_supported(P, H, W))
 */
int cssm_rfft2_ex(const float* x, int x_fs, int x_act, const float* a, int a_fs, int a_act, int C, long long P,
                  int H, int W, float* spec, void* stream);
int cssm_irfft2_ex(const float* spec, long long P, int H, int W, int C, float* y, int y_fs, const float* add,
                   const float* m, int m_fs, const float* d, int d_fs, float* sums, void* stream);

/* 1 if cssm_irfft2_ex can return plane sums for P planes of H x W, else 0. */
int cssm_irfft2_ex_sums_supported(long long P, int H, int W);

/*
 * im2col of a SAME ks x ks convolution over channels-last frames, for the
 * full-channel qkv conv of GatedDeltaNetCSSM (qkv_conv_separable=False,
 * cssm.py:4751-4753: nn.Conv(3C, (ks, ks), padding='SAME')), which is then
 * cssm_proj_planes of these rows with the conv kernel viewed as (ks*ks*C, 3C).
 *   x    (F, H, W, C) of dtype (cssm_dtype)
 *   out  (F*H*W, ks*ks*C) float32: row (f, h, w), column (a*ks + b)*C + c holds
 *        x[f][h + a - lo][w + b - lo][c], lo = (ks - 1) / 2, zero outside the frame
 * ks in 1..15; with C % 4 == 0 x and out vector-aligned (16 bytes, 8 for bf16 x).
 */
int cssm_im2col_same(const void* x, int dtype, int F, int H, int W, int C, int ks, float* out, void* stream);

/* 1 if cssm_rfft2_ex / cssm_irfft2_ex have a kernel for (H, W) planes, else 0. */
int cssm_fft_ex_supported(int H, int W);

/*
 * How the GDN delta-rule scan sees the entries of M_t and Delta_t: the three
 * evaluations GatedDeltaNetCSSM's slow path selects (cssm.py:4693-4701,
 * 4939-4991), each the linear recurrence s_t = M_t s_{t-1} + Delta_t on the
 * entries as mapped:
 *   GOOM     use_log and use_goom (the default): to_goom's floor on every
 *            entry, |x| < 1e-7 -> 1e-7 + 0j (goom.py:161-174)
 *   LINEAR   use_log=False (the direct complex scan, cssm.py:4960-4991), or
 *            scan_mode='pallas' at delta_key_dim 2 (pallas_matrix_2x2_scan,
 *            cssm.py:4940-4944): no map
 *   LOG_EPS  use_log without use_goom: exp(log(|x| + 1e-8) + i angle(x)),
 *            i.e. (|x| + 1e-8) x / |x|, and 1e-8 + 0j at x = 0
 */
typedef enum cssm_gdn_scan_variant {
  CSSM_GDN_SCAN_GOOM = 0,
  CSSM_GDN_SCAN_LINEAR = 1,
  CSSM_GDN_SCAN_LOG_EPS = 2
} cssm_gdn_scan_variant;

/*
 * Delta-rule recurrence of GatedDeltaNetCSSM per (batch, head, frequency bin)
 * with the d_k x d_k complex state held in registers over all T.  Replaces
 * cssm.py:4890-5000: spectral / key-vector L2 norms, M_t and Delta_t (their
 * entries mapped as scan_variant says), the matrix scan (math.py:384-411,
 * operations.py:314-390 -- exactly the linear recurrence
 * s_t = M_t s_{t-1} + Delta_t) and the readout o = S q.
 *   spec   (B, T, 3C, H, Wf) complex64: rfft2 of the q, k, v blocks
 *   norms  (B, T, 3C) from cssm_rfft2, or NULL when use_spectral_l2_norm is off
 *   ab     (alpha, beta) pairs: pair of (b, t, head, bin) at
 *          ((b T + t) ab_frame + head ab_head + bin ab_bin); dense / factored:
 *          (H*Wf, 0, 1), channel: (n_h, 1, 0), scalar: (1, 0, 0)
 *   what   (n_h, H, Wf) complex64 (cssm_spectral_kernel, goom_floor = 0)
 *   scan_variant  cssm_gdn_scan_variant
 *   ohat   (B, T, C, H, Wf) complex64 out; output channel head*d_k + i
 * delta_key_dim in {1, 2, 3, 4}, C a multiple of it.
 */
int cssm_gdn_scan_bins(const float* spec, const float* norms, const float* ab, long long ab_frame,
                       int ab_head, int ab_bin, const float* what, int B, int T, int C, int H, int W,
                       int delta_key_dim, int scan_variant, float* ohat, void* stream);

/*
 * Weight gradient of the depthwise ks x ks SAME convolution cssm_depthwise_conv
 * computes (qkv_dw, cssm.py:4744-4750; the reference takes it through
 * jax.value_and_grad, main.py:283): dW[a][b][c] = sum over frames and pixels of
 * x[h + a - (ks-1)/2][w + b - (ks-1)/2][c] dy[h][w][c], zero outside the frame.
 *   x, dy    (F, H, W, C) float32 channels-last
 *   partial  (blocks, ks, ks, C) float32 out: per-block partial sums (add them over blocks)
 * ks in {3, 5, 7}, C / 4 dividing 64, W a multiple of 8 (cssm_depthwise_conv_wgrad_supported);
 * 16-byte aligned tensors; blocks <= 65535.
 */
int cssm_depthwise_conv_wgrad(const float* x, const float* dy, int F, int H, int W, int C, int ks, float* partial,
                              int blocks, void* stream);

/* 1 if cssm_depthwise_conv_wgrad has a kernel for (W, C, ks), else 0. */
int cssm_depthwise_conv_wgrad_supported(int W, int C, int ks);

/*
 * Training forward of the delta-rule recurrence: cssm_gdn_scan_bins with the
 * spectral L2 norms left to the caller (spec holds q and k already scaled by
 * them, and v), plus the state entering every step, which the reverse pass
 * reads.  The reference takes its gradients with jax.value_and_grad through the
 * log-space scan (main.py:283; GOOM VJPs goom.py:47-137); this pair replaces
 * that span's forward and backward (cssm.py:4898-5000).
 *   spec, ab, ab_frame, ab_head, ab_bin, what, scan_variant: as cssm_gdn_scan_bins
 *   ohat    (B, T, C, H, Wf) complex64 out
 *   states  (B, T, C / d_k, d_k, d_k, H*Wf) complex64 out: s_{t-1} of step t
 */
int cssm_gdn_scan_bins_train(const float* spec, const float* ab, long long ab_frame, int ab_head, int ab_bin,
                             const float* what, int B, int T, int C, int H, int W, int delta_key_dim,
                             int scan_variant, float* ohat, float* states, void* stream);

/*
 * Reverse pass of cssm_gdn_scan_bins_train: the reverse recurrence over T per
 * (batch, head, bin) through the key-vector norm, M = alpha W (I - beta k k^H)
 * and Delta = beta v k^H through the entry map of scan_variant (no gradient
 * through an entry to_goom's floor took, or the LOG_EPS map's constant at 0),
 * with gradients written as dL/dRe + i dL/dIm.
 *   spec, ab, strides, what, scan_variant, states: as the forward call
 *   dohat  (B, T, C, H, Wf) complex64: dL/d ohat
 *   dspec  (B, T, 3C, H, Wf) complex64 out: dL/d spec (q and k as scaled in spec)
 *   dab    (B, T, C / d_k, H*Wf) (dalpha, dbeta) out per (b, t, head, bin): the caller
 *          sums them over what a gate type shares (heads, bins)
 *   dwhat  (B, C / d_k, H*Wf) complex64 out: dL/d W_hat per batch element (sum over B)
 */
int cssm_gdn_scan_bins_bwd(const float* spec, const float* ab, long long ab_frame, int ab_head, int ab_bin,
                           const float* what, const float* states, const float* dohat, int B, int T, int C, int H,
                           int W, int delta_key_dim, int scan_variant, float* dspec, float* dab, float* dwhat,
                           void* stream);

/*
 * The GDN spectral core as one kernel where a workgroup can hold a (batch,
 * head)'s state for all T (32 x 32 planes, delta_key_dim 4: the video-shaped
 * config): per step it reads the head's q, k, v planes once, runs their rfft2,
 * the spectral / key-vector norms, the delta rule and the readout S q, and
 * writes the irfft2 of o once; no spectrum reaches HBM.  Replaces cssm.py:4875-5025,
 * computing what cssm_rfft2 + cssm_gdn_scan_bins + cssm_irfft2 compute (the
 * per-plane norm sums add in another order).
 *   qkv    (B, T, 3C, H, W) float32 plane-major (the cssm_gdn_qkv_proj output)
 *   use_l2 1 = spectral L2 norms of q and k (use_spectral_l2_norm), 0 = none
 *   ab, ab_frame, ab_head, ab_bin, what, scan_variant: as cssm_gdn_scan_bins
 *   o      (B, T, C, H, W) float32 out: the irfft2 of the readout, channel head*d_k + i
 * qkv and o 16-byte aligned, ab and what 8.
 */
int cssm_gdn_core_fused(const float* qkv, int use_l2, const float* ab, long long ab_frame, int ab_head, int ab_bin,
                        const float* what, int B, int T, int C, int H, int W, int delta_key_dim, int scan_variant,
                        float* o, void* stream);

/* 1 if cssm_gdn_core_fused has a kernel for (H, W, delta_key_dim), else 0. */
int cssm_gdn_core_fused_supported(int H, int W, int delta_key_dim);

/* output_norm of GatedDeltaNetCSSM */
typedef enum cssm_norm { CSSM_NORM_NONE = 0, CSSM_NORM_RMS = 1, CSSM_NORM_LAYER = 2 } cssm_norm;

/*
 * GDN output path: per-pixel channel norm, times the gate, then the output
 * projection.  Replaces cssm.py:5026-5031 (RMSNorm _rms_norm :49-52, or
 * LayerNorm), :5126 (x gate_val) and :5141 (output_proj).
 *   o, gate  (F, K, HW) plane-major of in_dtype (irfft2 output; SiLU'd gate_proj)
 *   norm     cssm_norm; norm_scale (K) [rms_scale or output_layernorm/scale], norm_bias (K) or NULL
 *   kernel (K, N) [output_proj/kernel], bias (N); out (F * HW, N) channels-last of out_dtype
 * K <= 128 and K % 4 == 0; any HW (HW % 4 != 0 reads the planes element-wise).  o and
 * gate 16-byte aligned (f32) or 8-byte aligned (bf16), a f32 out 16-byte aligned.
 */
int cssm_gdn_proj_out(const void* o, const void* gate, int in_dtype, int F, int HW, int K, int N, int norm,
                      const float* norm_scale, const float* norm_bias, const float* kernel, const float* bias,
                      void* out, int out_dtype, void* stream);

/*
 * The same output path with the gate computed in the kernel from the layer
 * input instead of read: gate = act(x gate_kernel + gate_bias) (gate_proj,
 * cssm.py:4853-4859, act SiLU or sigmoid as output_gate_act), so gate_proj's
 * planes never reach HBM.
 *   x, x_dtype   (F * HW, K) channels-last layer input, CSSM_F32 or CSSM_BF16, 16-byte aligned
 *   gate_kernel  (K, K) [gate_proj/kernel], gate_bias (K); gate_act 1 SiLU, 2 sigmoid
 * Other arguments as cssm_gdn_proj_out.  K <= 64, K % 8 == 0, N <= 64 and HW % 4 == 0
 * (cssm_gdn_proj_out_xgate_supported), else CSSM_ERR_UNSUPPORTED.
 */
int cssm_gdn_proj_out_xgate(const void* o, int in_dtype, const void* x, int x_dtype, int F, int HW, int K, int N, int norm,
                            const float* norm_scale, const float* norm_bias, const float* gate_kernel,
                            const float* gate_bias, int gate_act, const float* kernel, const float* bias, void* out,
                            int out_dtype, void* stream);
int cssm_gdn_proj_out_xgate_supported(int K, int N, int HW);

/* 1 if cssm_gated_scan_fwd has a kernel for (H, W), else 0. */
int cssm_gated_scan_supported(int H, int W);

/* Channel-count granule of the fused scan for (H, W): C must be a multiple (0 = unsupported). */
int cssm_gated_scan_min_group(int H, int W);

/*
 * Column order of the per-bin planes cssm_gated_scan_fwd reads (gates, khat):
 * cols[p] (p < W/2 + 1) = the frequency column stored at position p of a row.
 * The identity except at 128 x 128, where the 64 packed columns are
 * interleaved (each wave's column passes then spread over the LDS banks while
 * its per-bin loads still cover whole cache lines); the Nyquist column stays
 * last.  No counterpart in the reference (the layout is this library's own).
 */
int cssm_gated_scan_col_order(int H, int W, int* cols);

/*
 * Slots of K_hat in the scan layout cssm_spectral_kernel(scan_order = 1) writes
 * and cssm_gated_scan_fwd / _bwd read: idx[s] (s < H (W/2 + 1)) = the natural
 * index u (W/2 + 1) + v of the bin stored in complex slot s of a channel's
 * plane.  Columns follow cssm_gated_scan_col_order; rows are row-major except at
 * 128 x 128, where rows u and u + 16 ((u / 16) even) alternate within each
 * column's slot pairs, so a column-pass lane loads two of its bins (rows k + 16 q
 * and k + 16 (q + 1)) with one 16-byte load over whole cache lines.  No
 * counterpart in the reference (the layout is this library's own).
 */
int cssm_gated_scan_khat_order(int H, int W, int* idx);

/*
 * CSSMSHViTBlock wiring around the cell, the token-mixer half of the block
 * (cssm_shvit.py:86-229): norm1 -> pos_conv -> cell -> frame selection ->
 * output activation -> residual.  Tensors are channels-last (B, T, H, W, C) of
 * dtype (CSSM_F32 / CSSM_BF16); an image is T = 1.
 *
 * norm1 statistics (flax LayerNorm, epsilon eps, variance E[x^2] - E[x]^2,
 * sums in double).  mode 0 global_layer: one group per b over T, H, W, C
 * (:106-108); 1 temporal_layer: per (b, h, w) over T, C (:109-111); 2 layer: per
 * (b, t, h, w) over C (:112-114).  stats (groups, 2) float32 = (mean, rstd).
 */
int cssm_block_norm_stats(const void* x, int dtype, int B, int T, int H, int W, int C, int mode, float eps,
                          float* stats, void* stream);

/*
 * out (B, T_out, H, W, C) = xn + pos_conv(xn), xn = (x - mean) rstd scale + bias
 * per norm1 group (stats from cssm_block_norm_stats with the same mode),
 * pos_conv = the depthwise 3 x 3 'SAME' convolution with bias
 * (cssm_shvit.py:122-145; kernel (3, 3, 1, C) HWIO, zero padding of xn).
 * pos_kernel = pos_bias = NULL: out = xn (use_pos_conv = False).  T_in = T_out,
 * or T_in = 1 with the image repeated to T_out frames (:99-101).
 */
int cssm_block_norm_posconv(const void* x, int dtype, int B, int T_in, int T_out, int H, int W, int C, int mode,
                            const float* stats, const float* scale, const float* bias, const float* pos_kernel,
                            const float* pos_bias, void* out, void* stream);

/*
 * out = res + act(y) (cssm_shvit.py:211-228): T_out = 1 takes the last frame
 * of res (T_res frames) and of y (T_y frames), T_out > 1 frame by frame
 * (keep_time; T_res = T_y = T_out).  act 0 none, 1 gelu (tanh form, as
 * jax.nn.gelu), 2 silu (output_act).  out (B, T_out, H, W, C).
 */
int cssm_block_residual(const void* res, int T_res, const void* y, int T_y, int dtype, int B, int T_out, int H,
                        int W, int C, int act, void* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* CSSM_AMD_H_ */
