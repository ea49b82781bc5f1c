// extern "C" entry points of libcssm_hip.so (declared in include/cssm_amd.h).
// Argument checking lives here; kernels assume validated shapes.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <mutex>

#include "../../include/cssm_amd.h"
#include "launch.h"

namespace {

thread_local char g_last_error[512] = "";

int fail(int status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return status;
}

int ok() {
  g_last_error[0] = '\0';
  return CSSM_OK;
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return ok();
  return fail(CSSM_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// alignment of the 4-element vector loads / stores the projection kernels make:
// 16 bytes for float32, 8 for bfloat16
size_t vec_align(int dtype) { return dtype == CSSM_F32 ? 16 : 8; }

}  // namespace

extern "C" {

int cssm_abi_version(void) { return CSSM_ABI_VERSION; }

const char* cssm_strerror(int status) {
  switch (status) {
    case CSSM_OK: return "ok";
    case CSSM_ERR_NULL: return "null pointer argument";
    case CSSM_ERR_SHAPE: return "invalid shape";
    case CSSM_ERR_UNSUPPORTED: return "unsupported configuration";
    case CSSM_ERR_ARG: return "invalid argument";
    case CSSM_ERR_ALIGN: return "misaligned pointer";
    case CSSM_ERR_HIP: return "HIP runtime error";
    default: return "unknown status";
  }
}

const char* cssm_last_error(void) { return g_last_error; }

int cssm_spectral_kernel(const float* k, int C, int K, int H, int W, float rho, int squash,
                         int goom_floor, int scan_order, float* khat, void* stream) {
  if (!k || !khat) return fail(CSSM_ERR_NULL, "cssm_spectral_kernel: k and khat must be non-null");
  if (C <= 0 || K <= 0 || H <= 0 || W <= 0)
    return fail(CSSM_ERR_SHAPE, "cssm_spectral_kernel: C=%d K=%d H=%d W=%d must be positive", C, K, H, W);
  if ((K > H || K > W) && (K < H || K < W))
    return fail(CSSM_ERR_SHAPE,
                "cssm_spectral_kernel: K=%d lies between H=%d and W=%d (reference pad/crop undefined)", K,
                H, W);
  if (!aligned(khat, 8)) return fail(CSSM_ERR_ALIGN, "cssm_spectral_kernel: khat must be 8-byte aligned");
  const hipError_t e = cssm::launch_spectral_kernel(k, C, K, H, W, rho, squash, goom_floor, scan_order ? 1 : 0,
                                                    reinterpret_cast<float2*>(khat),
                                                    static_cast<hipStream_t>(stream));
  if (e == hipErrorInvalidValue)
    return fail(CSSM_ERR_UNSUPPORTED, "cssm_spectral_kernel: plane %dx%d too large for the prep kernel", H, W);
  return hip_status(e, "cssm_spectral_kernel");
}

int cssm_plane_mean(const void* x, int dtype, long long nplanes, int H, int W, int act, float* out,
                    void* stream) {
  if (!x || !out) return fail(CSSM_ERR_NULL, "cssm_plane_mean: x and out must be non-null");
  if (nplanes < 0 || H <= 0 || W <= 0 || nplanes > 0x7fffffffLL)
    return fail(CSSM_ERR_SHAPE, "cssm_plane_mean: nplanes=%lld H=%d W=%d", nplanes, H, W);
  if (dtype != CSSM_F32 && dtype != CSSM_BF16) return fail(CSSM_ERR_ARG, "cssm_plane_mean: dtype=%d", dtype);
  if (act != CSSM_LOAD_IDENTITY && act != CSSM_LOAD_SILU)
    return fail(CSSM_ERR_ARG, "cssm_plane_mean: act=%d", act);
  return hip_status(cssm::launch_plane_mean(x, dtype, nplanes, H * W, act, out, static_cast<hipStream_t>(stream)),
                    "cssm_plane_mean");
}

// the gate projections of a cssm_gate_params, checked (0, or the failing status with its message set)
static int gate_weights(const cssm_gate_params* p, cssm::GateWeights& w, const char* who) {
  if (p->gate_type != CSSM_GATE_DENSE && p->gate_type != CSSM_GATE_FACTORED)
    return fail(CSSM_ERR_ARG, "%s: gate_type=%d", who, p->gate_type);
  if (p->activation < CSSM_ACT_SOFTPLUS || p->activation > CSSM_ACT_EXP)
    return fail(CSSM_ERR_ARG, "%s: activation=%d", who, p->activation);
  const bool fac = p->gate_type == CSSM_GATE_FACTORED;
  for (int i = 0; i < 3; ++i) {
    if (!p->kernel[i] || !p->bias[i] || (fac && (!p->kernel_w[i] || !p->bias_w[i])))
      return fail(CSSM_ERR_NULL, "%s: gate %d weights missing", who, i);
    w.kd[i] = p->kernel[i];
    w.bd[i] = p->bias[i];
    w.kw[i] = fac ? p->kernel_w[i] : nullptr;
    w.bw[i] = fac ? p->bias_w[i] : nullptr;
  }
  return CSSM_OK;
}

int cssm_gated_gates(const float* ctx, int B, int T, int C, int H, int W, const cssm_gate_params* p,
                     float c_scale, float* gates, void* stream) {
  if (!ctx || !p || !gates) return fail(CSSM_ERR_NULL, "cssm_gated_gates: ctx, params and gates must be non-null");
  if (B <= 0 || T <= 0 || C <= 0 || H <= 0 || W <= 0)
    return fail(CSSM_ERR_SHAPE, "cssm_gated_gates: B=%d T=%d C=%d H=%d W=%d", B, T, C, H, W);
  cssm::GateWeights w;
  if (const int st = gate_weights(p, w, "cssm_gated_gates")) return st;
  if (!aligned(gates, 16)) return fail(CSSM_ERR_ALIGN, "cssm_gated_gates: gates must be 16-byte aligned");
  const hipError_t e = cssm::launch_gated_gates(ctx, cssm::CtxPartials{nullptr, 0, 0, 0, nullptr}, B * T, C, H, W,
                                                p->gate_type == CSSM_GATE_FACTORED ? 1 : 0, p->activation, w,
                                                c_scale, reinterpret_cast<float4*>(gates),
                                                static_cast<hipStream_t>(stream));
  if (e == hipErrorInvalidValue)
    return fail(CSSM_ERR_UNSUPPORTED, "cssm_gated_gates: C=%d with %dx%d planes exceeds the staging buffer", C, H, W);
  return hip_status(e, "cssm_gated_gates");
}

int cssm_gated_gates_bwd(const float* ctx, int B, int T, int C, int H, int W, const cssm_gate_params* p,
                         float c_scale, const float* dgates, float* out, void* stream) {
  if (!ctx || !p || !dgates || !out)
    return fail(CSSM_ERR_NULL, "cssm_gated_gates_bwd: ctx, params, dgates and out must be non-null");
  if (B <= 0 || T <= 0 || C <= 0 || H <= 0 || W <= 0)
    return fail(CSSM_ERR_SHAPE, "cssm_gated_gates_bwd: B=%d T=%d C=%d H=%d W=%d", B, T, C, H, W);
  cssm::GateWeights w;
  if (const int st = gate_weights(p, w, "cssm_gated_gates_bwd")) return st;
  if (!aligned(dgates, 16)) return fail(CSSM_ERR_ALIGN, "cssm_gated_gates_bwd: dgates must be 16-byte aligned");
  const hipError_t e = cssm::launch_gated_gates_bwd(ctx, B * T, C, H, W, p->gate_type == CSSM_GATE_FACTORED ? 1 : 0,
                                                    p->activation, w, c_scale,
                                                    reinterpret_cast<const float4*>(dgates), out,
                                                    static_cast<hipStream_t>(stream));
  if (e == hipErrorInvalidValue)
    return fail(CSSM_ERR_UNSUPPORTED, "cssm_gated_gates_bwd: C=%d with %dx%d planes exceeds the staging buffer",
                C, H, W);
  return hip_status(e, "cssm_gated_gates_bwd");
}

int cssm_gated_scan_supported(int H, int W) { return cssm::gated_scan_has_kernel(H, W) ? 1 : 0; }

int cssm_gated_scan_min_group(int H, int W) { return cssm::gated_scan_min_group(H, W); }

int cssm_gated_scan_col_order(int H, int W, int* cols) {
  if (!cols) return fail(CSSM_ERR_NULL, "cssm_gated_scan_col_order: cols must be non-null");
  if (H <= 0 || W <= 0) return fail(CSSM_ERR_SHAPE, "cssm_gated_scan_col_order: H=%d W=%d", H, W);
  for (int p = 0; p < W / 2 + 1; ++p) cols[p] = cssm::scan_col(H, W, p);
  return CSSM_OK;
}

int cssm_gated_scan_khat_order(int H, int W, int* idx) {
  if (!idx) return fail(CSSM_ERR_NULL, "cssm_gated_scan_khat_order: idx must be non-null");
  if (H <= 0 || W <= 0) return fail(CSSM_ERR_SHAPE, "cssm_gated_scan_khat_order: H=%d W=%d", H, W);
  const int WF = W / 2 + 1;
  for (int u = 0; u < H; ++u)
    for (int p = 0; p < WF; ++p) idx[cssm::khat_pos(H, W, u, p)] = u * WF + cssm::scan_col(H, W, p);
  return CSSM_OK;
}

int cssm_gated_scan_fwd(const void* u, const void* z, void* y, int dtype, int B, int T, int C, int H, int W,
                        const float* gates, const float* khat, int u_act, int z_act, void* stream) {
  if (!u || !z || !y || !gates || !khat)
    return fail(CSSM_ERR_NULL, "cssm_gated_scan_fwd: u, z, y, gates and khat must be non-null");
  if (B <= 0 || T <= 0 || C <= 0 || H <= 0 || W <= 0)
    return fail(CSSM_ERR_SHAPE, "cssm_gated_scan_fwd: B=%d T=%d C=%d H=%d W=%d", B, T, C, H, W);
  if (dtype != CSSM_F32 && dtype != CSSM_BF16) return fail(CSSM_ERR_ARG, "cssm_gated_scan_fwd: dtype=%d", dtype);
  if ((u_act != CSSM_LOAD_IDENTITY && u_act != CSSM_LOAD_SILU) ||
      (z_act != CSSM_LOAD_IDENTITY && z_act != CSSM_LOAD_SILU))
    return fail(CSSM_ERR_ARG, "cssm_gated_scan_fwd: u_act=%d z_act=%d", u_act, z_act);
  if (!cssm::gated_scan_has_kernel(H, W))
    return fail(CSSM_ERR_UNSUPPORTED, "cssm_gated_scan_fwd: no fused kernel for %dx%d planes", H, W);
  const int g = cssm::gated_scan_min_group(H, W);
  if (C % g != 0)
    return fail(CSSM_ERR_UNSUPPORTED, "cssm_gated_scan_fwd: C=%d is not a multiple of %d for %dx%d planes", C, g,
                H, W);
  const size_t va = dtype == CSSM_F32 ? 16 : 8;
  if (!aligned(u, va) || !aligned(z, va) || !aligned(y, va) || !aligned(gates, 16) || !aligned(khat, 8))
    return fail(CSSM_ERR_ALIGN, "cssm_gated_scan_fwd: misaligned tensor pointer");
  if ((long long)B * T * C * H * W > (1LL << 40))
    return fail(CSSM_ERR_SHAPE, "cssm_gated_scan_fwd: tensor too large");
  const hipError_t e = cssm::launch_gated_scan(u, z, y, dtype, B, T, C, H, W, reinterpret_cast<const float4*>(gates),
                                               reinterpret_cast<const float2*>(khat), u_act, z_act,
                                               static_cast<hipStream_t>(stream));
  if (e == hipErrorInvalidValue)
    return fail(CSSM_ERR_UNSUPPORTED, "cssm_gated_scan_fwd: no plane-group split of C=%d for %dx%d", C, H, W);
  return hip_status(e, "cssm_gated_scan_fwd");
}

int cssm_gated_scan_bwd(const float* uspec, const float* dspec, const float* gates, const float* khat, int B, int T,
                        int C, int H, int W, float c_scale, float* yspec, float* sdu, float* dgates, float* dkhat,
                        void* stream) {
  if (!uspec || !dspec || !gates || !khat || !yspec || !sdu || !dgates || !dkhat)
    return fail(CSSM_ERR_NULL, "cssm_gated_scan_bwd: null argument");
  if (B <= 0 || T <= 0 || C <= 0 || H <= 0 || W <= 0 || !(c_scale > 0.0f))
    return fail(CSSM_ERR_SHAPE, "cssm_gated_scan_bwd: B=%d T=%d C=%d H=%d W=%d c_scale=%g", B, T, C, H, W,
                double(c_scale));
  if (T > 32) return fail(CSSM_ERR_UNSUPPORTED, "cssm_gated_scan_bwd: T=%d (the reverse pass holds T <= 32 states)", T);
  if (!aligned(gates, 16) || !aligned(dgates, 16) || !aligned(uspec, 8) || !aligned(dspec, 8) || !aligned(khat, 8) ||
      !aligned(yspec, 8) || !aligned(sdu, 8) || !aligned(dkhat, 8))
    return fail(CSSM_ERR_ALIGN, "cssm_gated_scan_bwd: gates 16-byte aligned, complex tensors 8");
  return hip_status(cssm::launch_gated_scan_bwd_bins(
                        reinterpret_cast<const float2*>(uspec), reinterpret_cast<const float2*>(dspec),
                        reinterpret_cast<const float4*>(gates), reinterpret_cast<const float2*>(khat), B, T, C, H, W,
                        c_scale, reinterpret_cast<float2*>(yspec), reinterpret_cast<float2*>(sdu),
                        reinterpret_cast<float4*>(dgates), reinterpret_cast<float2*>(dkhat),
                        static_cast<hipStream_t>(stream)),
                    "cssm_gated_scan_bwd");
}

size_t cssm_proj_in_workspace_size(int F, int HW, int K, int N) {
  if (F <= 0 || HW <= 0 || K <= 0 || N <= 0) return 0;
  const int tm = cssm::proj_in_tile_rows(K), slots = cssm::proj_in_ctx_slots(K, HW);
  const size_t tiles = (size_t(F) * HW + tm - 1) / tm;
  return tiles * slots * (N / 2) * sizeof(float);
}

// argument checks of the input projection (0, or the failing status with its message set)
static int proj_in_check(const void* x, int in_dtype, int F, int HW, int K, int N, const float* kernel,
                         const float* bias, void* out_lo, void* out_hi, int out_dtype, int act_lo, int act_hi,
                         const char* who) {
  if (!x || !kernel || !bias || !out_lo || !out_hi)
    return fail(CSSM_ERR_NULL, "%s: x, kernel, bias, out_lo and out_hi must be non-null", who);
  if (F <= 0 || HW <= 0 || K <= 0 || N <= 0 || (N % 2) != 0)
    return fail(CSSM_ERR_SHAPE, "%s: F=%d HW=%d K=%d N=%d (N must be even)", who, F, HW, K, N);
  if ((long long)F * HW > 0x7fffffffLL) return fail(CSSM_ERR_SHAPE, "%s: F*HW exceeds 2^31", who);
  if ((in_dtype != CSSM_F32 && in_dtype != CSSM_BF16) || (out_dtype != CSSM_F32 && out_dtype != CSSM_BF16))
    return fail(CSSM_ERR_ARG, "%s: dtypes %d/%d", who, in_dtype, out_dtype);
  if ((act_lo != CSSM_LOAD_IDENTITY && act_lo != CSSM_LOAD_SILU && act_lo != CSSM_PROJ_STORE_PRE_CTX_SILU) ||
      (act_hi != CSSM_LOAD_IDENTITY && act_hi != CSSM_LOAD_SILU))
    return fail(CSSM_ERR_ARG, "%s: act_lo=%d act_hi=%d", who, act_lo, act_hi);
  if (!aligned(x, vec_align(in_dtype)))
    return fail(CSSM_ERR_ALIGN, "%s: x must be %zu-byte aligned", who, vec_align(in_dtype));
  if (out_dtype == CSSM_F32 && (!aligned(out_lo, 16) || !aligned(out_hi, 16)))
    return fail(CSSM_ERR_ALIGN, "%s: f32 outputs must be 16-byte aligned", who);
  return CSSM_OK;
}

int cssm_proj_in(const void* x, int in_dtype, int F, int HW, int K, int N, const float* kernel, const float* bias,
                 void* out_lo, void* out_hi, int out_dtype, int act_lo, int act_hi, float* ctx, void* workspace,
                 size_t workspace_bytes, void* stream) {
  if (const int st = proj_in_check(x, in_dtype, F, HW, K, N, kernel, bias, out_lo, out_hi, out_dtype, act_lo, act_hi,
                                   "cssm_proj_in"))
    return st;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int M = F * HW;
  const int tm = cssm::proj_in_tile_rows(K), slots = cssm::proj_in_ctx_slots(K, HW);
  const bool fused_ctx = ctx != nullptr && slots > 0;
  float* partial = nullptr;
  if (fused_ctx) {
    const size_t need = cssm_proj_in_workspace_size(F, HW, K, N);
    if (!workspace || workspace_bytes < need)
      return fail(CSSM_ERR_ARG, "cssm_proj_in: ctx needs a %zu-byte workspace (got %zu)", need, workspace_bytes);
    partial = static_cast<float*>(workspace);
  }
  hipError_t e = cssm::launch_proj_in(x, in_dtype, M, K, N, kernel, bias, HW, out_lo, out_hi, out_dtype, act_lo,
                                      act_hi, partial, s);
  if (e != hipSuccess) return hip_status(e, "cssm_proj_in");
  if (ctx != nullptr) {
    e = fused_ctx ? cssm::launch_ctx_reduce(partial, F, HW, tm, slots, N / 2, ctx, s)
                  : cssm::launch_plane_mean(out_lo, out_dtype, (long long)F * (N / 2), HW,
                                            act_lo == CSSM_PROJ_STORE_PRE_CTX_SILU ? 1 : 0, ctx, s);
  }
  return hip_status(e, "cssm_proj_in");
}

int cssm_proj_in_gates(const void* x, int in_dtype, int B, int T, int H, int W, int K, int N, const float* kernel,
                       const float* bias, void* out_lo, void* out_hi, int out_dtype, int act_lo, int act_hi,
                       float* ctx, const cssm_gate_params* p, float c_scale, float* gates, void* workspace,
                       size_t workspace_bytes, void* stream) {
  if (!ctx || !p || !gates) return fail(CSSM_ERR_NULL, "cssm_proj_in_gates: ctx, params and gates must be non-null");
  if (B <= 0 || T <= 0 || H <= 0 || W <= 0 || (long long)B * T * H * W > 0x7fffffffLL)
    return fail(CSSM_ERR_SHAPE, "cssm_proj_in_gates: B=%d T=%d H=%d W=%d", B, T, H, W);
  const int F = B * T, HW = H * W;
  if (const int st = proj_in_check(x, in_dtype, F, HW, K, N, kernel, bias, out_lo, out_hi, out_dtype, act_lo, act_hi,
                                   "cssm_proj_in_gates"))
    return st;
  cssm::GateWeights w;
  if (const int st = gate_weights(p, w, "cssm_proj_in_gates")) return st;
  if (!aligned(gates, 16)) return fail(CSSM_ERR_ALIGN, "cssm_proj_in_gates: gates must be 16-byte aligned");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int M = F * HW, C = N / 2;
  const int tm = cssm::proj_in_tile_rows(K), slots = cssm::proj_in_ctx_slots(K, HW);
  cssm::CtxPartials cp{nullptr, 0, 0, 0, nullptr};
  float* partial = nullptr;
  if (slots > 0) {
    const size_t need = cssm_proj_in_workspace_size(F, HW, K, N);
    if (!workspace || workspace_bytes < need)
      return fail(CSSM_ERR_ARG, "cssm_proj_in_gates: a %zu-byte workspace is required (got %zu)", need,
                  workspace_bytes);
    partial = static_cast<float*>(workspace);
    cp = cssm::CtxPartials{partial, HW, tm, slots, ctx};
  }
  hipError_t e = cssm::launch_proj_in(x, in_dtype, M, K, N, kernel, bias, HW, out_lo, out_hi, out_dtype, act_lo,
                                      act_hi, partial, s);
  if (e != hipSuccess) return hip_status(e, "cssm_proj_in_gates");
  if (slots == 0) {
    e = cssm::launch_plane_mean(out_lo, out_dtype, (long long)F * C, HW,
                                act_lo == CSSM_PROJ_STORE_PRE_CTX_SILU ? 1 : 0, ctx, s);
    if (e != hipSuccess) return hip_status(e, "cssm_proj_in_gates");
  }
  // with the projection's per-tile sums the gate kernel reduces them per frame itself (and writes
  // ctx) instead of a separate reduction launch
  e = cssm::launch_gated_gates(slots > 0 ? nullptr : ctx, cp, F, C, H, W, p->gate_type == CSSM_GATE_FACTORED ? 1 : 0,
                               p->activation, w, c_scale, reinterpret_cast<float4*>(gates), s);
  if (e == hipErrorInvalidValue)
    return fail(CSSM_ERR_UNSUPPORTED, "cssm_proj_in_gates: C=%d with %dx%d planes exceeds the staging buffer", C, H,
                W);
  return hip_status(e, "cssm_proj_in_gates");
}

int cssm_proj_out(const void* y, int in_dtype, int F, int HW, int K, int N, const float* kernel, const float* bias,
                  void* out, int out_dtype, void* stream) {
  if (!y || !kernel || !bias || !out)
    return fail(CSSM_ERR_NULL, "cssm_proj_out: y, kernel, bias and out must be non-null");
  if (F <= 0 || HW <= 0 || K <= 0 || N <= 0) return fail(CSSM_ERR_SHAPE, "cssm_proj_out: F=%d HW=%d K=%d N=%d", F, HW, K, N);
  if ((long long)F * HW > 0x7fffffffLL) return fail(CSSM_ERR_SHAPE, "cssm_proj_out: F*HW exceeds 2^31");
  if ((in_dtype != CSSM_F32 && in_dtype != CSSM_BF16) || (out_dtype != CSSM_F32 && out_dtype != CSSM_BF16))
    return fail(CSSM_ERR_ARG, "cssm_proj_out: dtypes %d/%d", in_dtype, out_dtype);
  if (!aligned(y, vec_align(in_dtype)) || (out_dtype == CSSM_F32 && !aligned(out, 16)))
    return fail(CSSM_ERR_ALIGN, "cssm_proj_out: y must be %zu-byte aligned, a f32 out 16-byte aligned",
                vec_align(in_dtype));
  return hip_status(cssm::launch_proj_out(y, in_dtype, F * HW, K, N, kernel, bias, HW, out, out_dtype,
                                          static_cast<hipStream_t>(stream)),
                    "cssm_proj_out");
}

int cssm_short_conv(const void* x, int in_dtype, int B, int T, int C, int H, int W, int ks, const float* ws,
                    const float* bs, int kt, const float* wt, const float* bt, void* u, int out_dtype, float* ctx,
                    void* stream) {
  if (!x || !u) return fail(CSSM_ERR_NULL, "cssm_short_conv: x and u must be non-null");
  if ((ks > 0 && (!ws || !bs)) || (kt > 0 && (!wt || !bt)))
    return fail(CSSM_ERR_NULL, "cssm_short_conv: weights of an enabled convolution are missing");
  if (B <= 0 || T <= 0 || C <= 0 || H <= 0 || W <= 0 || ks < 0 || kt < 0 || ks > 15 || kt > 16)
    return fail(CSSM_ERR_SHAPE, "cssm_short_conv: B=%d T=%d C=%d H=%d W=%d ks=%d kt=%d", B, T, C, H, W, ks, kt);
  if ((in_dtype != CSSM_F32 && in_dtype != CSSM_BF16) || (out_dtype != CSSM_F32 && out_dtype != CSSM_BF16))
    return fail(CSSM_ERR_ARG, "cssm_short_conv: dtypes %d/%d", in_dtype, out_dtype);
  return hip_status(cssm::launch_short_conv(x, in_dtype, B, T, C, H, W, ks, ws, bs, kt, wt, bt, u, out_dtype, ctx,
                                            static_cast<hipStream_t>(stream)),
                    "cssm_short_conv");
}

}  // extern "C"

namespace {
bool dtype_ok(int d) { return d == CSSM_F32 || d == CSSM_BF16; }
}  // namespace

extern "C" {

int cssm_proj_planes(const void* x, int in_dtype, int F, int HW, int K, int N, const float* kernel, const float* bias,
                     void* out, int out_dtype, int act, void* stream) {
  if (!x || !kernel || !bias || !out) return fail(CSSM_ERR_NULL, "cssm_proj_planes: x, kernel, bias and out must be non-null");
  if (F <= 0 || HW <= 0 || K <= 0 || N <= 0) return fail(CSSM_ERR_SHAPE, "cssm_proj_planes: F=%d HW=%d K=%d N=%d", F, HW, K, N);
  if ((long long)F * HW > 0x7fffffffLL) return fail(CSSM_ERR_SHAPE, "cssm_proj_planes: F*HW exceeds 2^31");
  if (!dtype_ok(in_dtype) || !dtype_ok(out_dtype)) return fail(CSSM_ERR_ARG, "cssm_proj_planes: dtypes %d/%d", in_dtype, out_dtype);
  if (act < 0 || act > 2) return fail(CSSM_ERR_ARG, "cssm_proj_planes: act=%d", act);
  if (!aligned(x, vec_align(in_dtype)))
    return fail(CSSM_ERR_ALIGN, "cssm_proj_planes: x must be %zu-byte aligned", vec_align(in_dtype));
  if (out_dtype == CSSM_F32 && !aligned(out, 16)) return fail(CSSM_ERR_ALIGN, "cssm_proj_planes: f32 out must be 16-byte aligned");
  return hip_status(cssm::launch_proj_planes(x, in_dtype, F * HW, K, N, kernel, bias, HW, out, out, out_dtype, act, act,
                                             nullptr, N, static_cast<hipStream_t>(stream)),
                    "cssm_proj_planes");
}

int cssm_frame_mean(const void* x, int dtype, int F, int HW, int C, float* out, void* stream) {
  if (!x || !out) return fail(CSSM_ERR_NULL, "cssm_frame_mean: x and out must be non-null");
  if (F <= 0 || HW <= 0 || C <= 0) return fail(CSSM_ERR_SHAPE, "cssm_frame_mean: F=%d HW=%d C=%d", F, HW, C);
  if (!dtype_ok(dtype)) return fail(CSSM_ERR_ARG, "cssm_frame_mean: dtype=%d", dtype);
  return hip_status(cssm::launch_frame_mean(x, dtype, F, HW, C, out, static_cast<hipStream_t>(stream)), "cssm_frame_mean");
}

int cssm_depthwise_conv(const void* x, int dtype, int F, int H, int W, int C, int ks, const float* kernel,
                        const float* bias, void* out, int out_dtype, void* stream) {
  if (!x || !kernel || !bias || !out) return fail(CSSM_ERR_NULL, "cssm_depthwise_conv: null argument");
  if (F <= 0 || H <= 0 || W <= 0 || C <= 0 || ks <= 0 || ks > 31)
    return fail(CSSM_ERR_SHAPE, "cssm_depthwise_conv: F=%d H=%d W=%d C=%d ks=%d", F, H, W, C, ks);
  if (!dtype_ok(dtype) || !dtype_ok(out_dtype))
    return fail(CSSM_ERR_ARG, "cssm_depthwise_conv: dtypes %d/%d", dtype, out_dtype);
  if (x == out) return fail(CSSM_ERR_ARG, "cssm_depthwise_conv: out must not alias x");
  return hip_status(cssm::launch_depthwise_conv(x, dtype, F, H, W, C, ks, kernel, bias, out, out_dtype,
                                                static_cast<hipStream_t>(stream)),
                    "cssm_depthwise_conv");
}

long long cssm_depthwise_conv_mean_workspace(int F, int H, int W, int C, int ks) {
  if (F <= 0 || H <= 0 || W <= 0 || C <= 0) return 0;
  return (long long)cssm::depthwise_conv_mean_blocks(F, H, W, C, ks) * F * C;
}

int cssm_depthwise_conv_mean(const void* x, int dtype, int F, int H, int W, int C, int ks, const float* kernel,
                             const float* bias, void* out, int out_dtype, float* workspace, float* ctx, void* stream) {
  if (!x || !kernel || !bias || !out || !workspace || !ctx)
    return fail(CSSM_ERR_NULL, "cssm_depthwise_conv_mean: null argument");
  if (F <= 0 || H <= 0 || W <= 0 || C <= 0 || ks <= 0 || ks > 31)
    return fail(CSSM_ERR_SHAPE, "cssm_depthwise_conv_mean: F=%d H=%d W=%d C=%d ks=%d", F, H, W, C, ks);
  if (!dtype_ok(dtype) || !dtype_ok(out_dtype))
    return fail(CSSM_ERR_ARG, "cssm_depthwise_conv_mean: dtypes %d/%d", dtype, out_dtype);
  if (x == out) return fail(CSSM_ERR_ARG, "cssm_depthwise_conv_mean: out must not alias x");
  if (!cssm::depthwise_conv_mean_blocks(F, H, W, C, ks))
    return fail(CSSM_ERR_UNSUPPORTED, "cssm_depthwise_conv_mean: no fused form for H=%d W=%d C=%d ks=%d", H, W, C, ks);
  if (!aligned(x, vec_align(dtype)) || !aligned(out, vec_align(out_dtype)) || !aligned(kernel, 16) ||
      !aligned(bias, 16) || !aligned(workspace, 16))
    return fail(CSSM_ERR_ALIGN, "cssm_depthwise_conv_mean: misaligned x / out / kernel / bias / workspace");
  return hip_status(cssm::launch_depthwise_conv_mean(x, dtype, F, H, W, C, ks, kernel, bias, out, out_dtype, workspace,
                                                     ctx, static_cast<hipStream_t>(stream)),
                    "cssm_depthwise_conv_mean");
}

int cssm_gdn_gates(const float* ctx, int B, int T, int C, int H, int W, int dk, const cssm_gdn_gate_params* p,
                   int temporal, float rope_base, const float* temporal_table, float* ab, float* bkv, void* stream) {
  if (!ctx || !p || !ab) return fail(CSSM_ERR_NULL, "cssm_gdn_gates: ctx, params and ab must be non-null");
  if (B <= 0 || T <= 0 || C <= 0 || H <= 0 || W <= 0 || dk <= 0 || C % dk)
    return fail(CSSM_ERR_SHAPE, "cssm_gdn_gates: B=%d T=%d C=%d H=%d W=%d d_k=%d", B, T, C, H, W, dk);
  if (p->gate_type < CSSM_GDN_GATE_DENSE || p->gate_type > CSSM_GDN_GATE_SCALAR)
    return fail(CSSM_ERR_ARG, "cssm_gdn_gates: gate_type=%d", p->gate_type);
  if (temporal < 0 || temporal > 2 || (temporal == 2 && !temporal_table))
    return fail(CSSM_ERR_ARG, "cssm_gdn_gates: temporal=%d (table %p)", temporal, (const void*)temporal_table);
  const bool fac = p->gate_type == CSSM_GDN_GATE_FACTORED;
  const bool spatial = p->kernel[2] != nullptr;
  if (spatial && p->gate_type == CSSM_GDN_GATE_CHANNEL)
    return fail(CSSM_ERR_ARG, "cssm_gdn_gates: channel input gates are 1x1 convolutions (cssm_proj_planes)");
  if (spatial && !bkv) return fail(CSSM_ERR_NULL, "cssm_gdn_gates: bkv must be non-null with input gates");
  cssm::GdnGateWeights w;
  w.kind = p->gate_type;
  for (int g = 0; g < 4; ++g) {
    const bool need = g < 2 || spatial;
    if (need && (!p->kernel[g] || !p->bias[g] || (fac && (!p->kernel_w[g] || !p->bias_w[g]))))
      return fail(CSSM_ERR_NULL, "cssm_gdn_gates: gate %d weights missing", g);
    w.kd[g] = need ? p->kernel[g] : nullptr;
    w.bd[g] = need ? p->bias[g] : nullptr;
    w.kw[g] = need && fac ? p->kernel_w[g] : nullptr;
    w.bw[g] = need && fac ? p->bias_w[g] : nullptr;
  }
  const hipError_t e = cssm::launch_gdn_gates(ctx, B, T, C, H, W, C / dk, w, temporal, rope_base, temporal_table,
                                              reinterpret_cast<float2*>(ab), reinterpret_cast<float2*>(bkv),
                                              static_cast<hipStream_t>(stream));
  if (e == hipErrorInvalidValue)
    return fail(CSSM_ERR_UNSUPPORTED, "cssm_gdn_gates: C=%d with %dx%d planes exceeds the staging buffer", C, H, W);
  return hip_status(e, "cssm_gdn_gates");
}

int cssm_gdn_qkv_post(void* qkv, int dtype, int B, int T, int C, int H, int W, int kt, const float* const* conv_kernel,
                      const float* const* conv_bias, int gate_mode, const void* gates, void* stream) {
  if (!qkv) return fail(CSSM_ERR_NULL, "cssm_gdn_qkv_post: qkv must be non-null");
  if (B <= 0 || T <= 0 || C <= 0 || H <= 0 || W <= 0 || kt < 0 || kt > 8)
    return fail(CSSM_ERR_SHAPE, "cssm_gdn_qkv_post: B=%d T=%d C=%d H=%d W=%d kt=%d (kt <= 8)", B, T, C, H, W, kt);
  if (!dtype_ok(dtype)) return fail(CSSM_ERR_ARG, "cssm_gdn_qkv_post: dtype=%d", dtype);
  if (gate_mode < 0 || gate_mode > 3) return fail(CSSM_ERR_ARG, "cssm_gdn_qkv_post: gate_mode=%d", gate_mode);
  if (gate_mode != 0 && !gates) return fail(CSSM_ERR_NULL, "cssm_gdn_qkv_post: gates must be non-null");
  cssm::GdnShortConv sc{};
  if (kt > 0) {
    if (!conv_kernel || !conv_bias) return fail(CSSM_ERR_NULL, "cssm_gdn_qkv_post: short-conv weights missing");
    for (int i = 0; i < 3; ++i) {
      if (!conv_kernel[i] || !conv_bias[i]) return fail(CSSM_ERR_NULL, "cssm_gdn_qkv_post: short-conv %d missing", i);
      sc.w[i] = conv_kernel[i];
      sc.b[i] = conv_bias[i];
    }
  }
  if (!aligned(qkv, dtype == CSSM_F32 ? 16 : 8) || (gate_mode == 1 && !aligned(gates, 8)) ||
      (gate_mode == 3 && !aligned(gates, 16)))
    return fail(CSSM_ERR_ALIGN, "cssm_gdn_qkv_post: misaligned qkv / gates");
  return hip_status(cssm::launch_gdn_qkv_post(qkv, dtype, B, T, C, H * W, kt, sc, gate_mode, gates,
                                              static_cast<hipStream_t>(stream)),
                    "cssm_gdn_qkv_post");
}

// shared by the qkv projection and its gate_proj variant (wg != nullptr)
static int gdn_qkv_proj_impl(const char* fn, const void* x, int in_dtype, int B, int T, int H, int W, int K, int C,
                             const float* kernel, const float* bias, int kt, const float* const* conv_kernel,
                             const float* const* conv_bias, int gate_mode, const void* gates, void* qkv,
                             int out_dtype, void* stream, const float* wg, const float* bg, int gact, void* gv) {
  if (!x || !kernel || !bias || !qkv) return fail(CSSM_ERR_NULL, "%s: x, kernel, bias and qkv must be non-null", fn);
  if (B <= 0 || T <= 0 || H <= 0 || W <= 0 || K <= 0 || C <= 0 || kt < 0 || kt > 8)
    return fail(CSSM_ERR_SHAPE, "%s: B=%d T=%d H=%d W=%d K=%d C=%d kt=%d (kt <= 8)", fn, B, T, H, W, K, C, kt);
  if ((long long)B * T * H * W > 0x7fffffffLL) return fail(CSSM_ERR_SHAPE, "%s: B*T*H*W exceeds 2^31", fn);
  if (!dtype_ok(in_dtype) || !dtype_ok(out_dtype)) return fail(CSSM_ERR_ARG, "%s: dtypes %d/%d", fn, in_dtype, out_dtype);
  if (gate_mode < 0 || gate_mode > 3) return fail(CSSM_ERR_ARG, "%s: gate_mode=%d", fn, gate_mode);
  if (gate_mode != 0 && !gates) return fail(CSSM_ERR_NULL, "%s: gates must be non-null", fn);
  cssm::GdnShortConv sc{};
  if (kt > 0) {
    if (!conv_kernel || !conv_bias) return fail(CSSM_ERR_NULL, "%s: short-conv weights missing", fn);
    for (int i = 0; i < 3; ++i) {
      if (!conv_kernel[i] || !conv_bias[i]) return fail(CSSM_ERR_NULL, "%s: short-conv %d missing", fn, i);
      sc.w[i] = conv_kernel[i];
      sc.b[i] = conv_bias[i];
    }
  }
  if (!aligned(x, vec_align(in_dtype)) || !aligned(qkv, vec_align(out_dtype)) ||
      (gate_mode == 1 && !aligned(gates, 8)) || (gate_mode == 3 && !aligned(gates, 16)))
    return fail(CSSM_ERR_ALIGN, "%s: misaligned x / qkv / gates", fn);
  if (wg) {
    if (!bg || !gv) return fail(CSSM_ERR_NULL, "%s: gate_bias and gv must be non-null", fn);
    if (gact != 1 && gact != 2) return fail(CSSM_ERR_ARG, "%s: gate_act=%d (1 SiLU, 2 sigmoid)", fn, gact);
    if (!aligned(gv, vec_align(out_dtype))) return fail(CSSM_ERR_ALIGN, "%s: misaligned gv", fn);
  }
  return hip_status(cssm::launch_gdn_qkv_proj(x, in_dtype, B, T, H * W, K, C, kernel, bias, kt, sc, gate_mode, gates,
                                              qkv, out_dtype, static_cast<hipStream_t>(stream), wg, bg, gact, gv),
                    fn);
}

int cssm_gdn_qkv_proj(const void* x, int in_dtype, int B, int T, int H, int W, int K, int C, const float* kernel,
                      const float* bias, int kt, const float* const* conv_kernel, const float* const* conv_bias,
                      int gate_mode, const void* gates, void* qkv, int out_dtype, void* stream) {
  return gdn_qkv_proj_impl("cssm_gdn_qkv_proj", x, in_dtype, B, T, H, W, K, C, kernel, bias, kt, conv_kernel,
                           conv_bias, gate_mode, gates, qkv, out_dtype, stream, nullptr, nullptr, 0, nullptr);
}

int cssm_gdn_qkv_gate_proj(const void* x, int in_dtype, int B, int T, int H, int W, int K, int C, const float* kernel,
                           const float* bias, int kt, const float* const* conv_kernel, const float* const* conv_bias,
                           int gate_mode, const void* gates, const float* gate_kernel, const float* gate_bias,
                           int gate_act, void* qkv, void* gv, int out_dtype, void* stream) {
  if (!gate_kernel) return fail(CSSM_ERR_NULL, "cssm_gdn_qkv_gate_proj: gate_kernel must be non-null");
  return gdn_qkv_proj_impl("cssm_gdn_qkv_gate_proj", x, in_dtype, B, T, H, W, K, C, kernel, bias, kt, conv_kernel,
                           conv_bias, gate_mode, gates, qkv, out_dtype, stream, gate_kernel, gate_bias, gate_act, gv);
}

int cssm_gdn_qkv_fused(int T, int H, int W, int K, int kt) {
  return cssm::gdn_qkv_fused_supported(T, H * W, K, kt) ? 1 : 0;
}

int cssm_fft_min_group(int H, int W) { return cssm::fft_planes_min_group(H, W); }

int cssm_rfft2(const void* x, int dtype, long long P, int H, int W, float* spec, float* norms, void* stream) {
  if (!x || !spec) return fail(CSSM_ERR_NULL, "cssm_rfft2: x and spec must be non-null");
  if (P <= 0 || H <= 0 || W <= 0 || P > 0x7fffffffLL) return fail(CSSM_ERR_SHAPE, "cssm_rfft2: P=%lld H=%d W=%d", P, H, W);
  if (!dtype_ok(dtype)) return fail(CSSM_ERR_ARG, "cssm_rfft2: dtype=%d", dtype);
  if (!cssm::fft_planes_min_group(H, W)) return fail(CSSM_ERR_UNSUPPORTED, "cssm_rfft2: no kernel for %dx%d planes", H, W);
  if (!aligned(x, dtype == CSSM_F32 ? 16 : 8) || !aligned(spec, 8))
    return fail(CSSM_ERR_ALIGN, "cssm_rfft2: misaligned tensor pointer");
  return hip_status(cssm::launch_rfft2(x, dtype, P, H, W, reinterpret_cast<float2*>(spec), norms,
                                       static_cast<hipStream_t>(stream)),
                    "cssm_rfft2");
}

int cssm_irfft2(const float* spec, long long P, int H, int W, void* y, int dtype, void* stream) {
  if (!spec || !y) return fail(CSSM_ERR_NULL, "cssm_irfft2: spec and y must be non-null");
  if (P <= 0 || H <= 0 || W <= 0 || P > 0x7fffffffLL) return fail(CSSM_ERR_SHAPE, "cssm_irfft2: P=%lld H=%d W=%d", P, H, W);
  if (!dtype_ok(dtype)) return fail(CSSM_ERR_ARG, "cssm_irfft2: dtype=%d", dtype);
  if (!cssm::fft_planes_min_group(H, W)) return fail(CSSM_ERR_UNSUPPORTED, "cssm_irfft2: no kernel for %dx%d planes", H, W);
  if (!aligned(y, dtype == CSSM_F32 ? 16 : 8) || !aligned(spec, 8))
    return fail(CSSM_ERR_ALIGN, "cssm_irfft2: misaligned tensor pointer");
  return hip_status(cssm::launch_irfft2(reinterpret_cast<const float2*>(spec), P, H, W, y, dtype,
                                        static_cast<hipStream_t>(stream)),
                    "cssm_irfft2");
}

int cssm_fft_ex_supported(int H, int W) { return cssm::fft_ex_supported(H, W) ? 1 : 0; }

int cssm_im2col_same(const void* x, int dtype, int F, int H, int W, int C, int ks, float* out, void* stream) {
  if (!x || !out) return fail(CSSM_ERR_NULL, "cssm_im2col_same: x and out must be non-null");
  if (F <= 0 || H <= 0 || W <= 0 || C <= 0 || ks < 1 || ks > 15)
    return fail(CSSM_ERR_SHAPE, "cssm_im2col_same: F=%d H=%d W=%d C=%d ks=%d", F, H, W, C, ks);
  if (dtype != CSSM_F32 && dtype != CSSM_BF16) return fail(CSSM_ERR_ARG, "cssm_im2col_same: dtype %d", dtype);
  if (C % 4 == 0 && (!aligned(x, dtype == CSSM_F32 ? 16 : 8) || !aligned(out, 16)))
    return fail(CSSM_ERR_ALIGN, "cssm_im2col_same: x and out must be vector-aligned for C %% 4 == 0");
  return hip_status(cssm::launch_im2col_same(x, dtype, (long long)F * H * W, H, W, C, ks, out,
                                             static_cast<hipStream_t>(stream)),
                    "cssm_im2col_same");
}

static bool plane_set_ok(const float* p, int fs, int C) { return p == nullptr || (fs >= C && aligned(p, 16)); }

int cssm_rfft2_ex(const float* x, int x_fs, int x_act, const float* a, int a_fs, int a_act, int C, long long P,
                  int H, int W, float* spec, void* stream) {
  if (!x || !spec) return fail(CSSM_ERR_NULL, "cssm_rfft2_ex: x and spec must be non-null");
  if (P <= 0 || C <= 0 || P % C) return fail(CSSM_ERR_SHAPE, "cssm_rfft2_ex: P=%lld C=%d (P a multiple of C)", P, C);
  if (!cssm::fft_ex_supported(H, W))
    return fail(CSSM_ERR_UNSUPPORTED, "cssm_rfft2_ex: %dx%d planes (square powers of two 4..128)", H, W);
  if ((x_act != CSSM_LOAD_IDENTITY && x_act != CSSM_LOAD_SILU) || (a_act != CSSM_LOAD_IDENTITY && a_act != CSSM_LOAD_SILU))
    return fail(CSSM_ERR_ARG, "cssm_rfft2_ex: x_act=%d a_act=%d", x_act, a_act);
  if (!plane_set_ok(x, x_fs, C) || !plane_set_ok(a, a_fs, C) || !aligned(spec, 8))
    return fail(CSSM_ERR_ALIGN, "cssm_rfft2_ex: plane sets need fs >= C and 16-byte alignment, spec 8");
  cssm::FftEx e{};
  e.x = {x, x_fs};
  e.a = {a, a_fs};
  e.x_act = x_act;
  e.a_act = a_act;
  e.C = C;
  return hip_status(cssm::launch_rfft2_ex(e, P, H, W, reinterpret_cast<float2*>(spec), static_cast<hipStream_t>(stream)),
                    "cssm_rfft2_ex");
}

int cssm_irfft2_ex_sums_supported(long long P, int H, int W) { return cssm::irfft2_ex_sums_supported(P, H, W) ? 1 : 0; }

int cssm_irfft2_ex(const float* spec, long long P, int H, int W, int C, float* y, int y_fs, const float* add,
                   const float* m, int m_fs, const float* d, int d_fs, float* sums, void* stream) {
  if (!spec || !y) return fail(CSSM_ERR_NULL, "cssm_irfft2_ex: spec and y must be non-null");
  if (sums && !cssm::irfft2_ex_sums_supported(P, H, W))
    return fail(CSSM_ERR_UNSUPPORTED, "cssm_irfft2_ex: plane sums of %lld %dx%d planes", P, H, W);
  if (P <= 0 || C <= 0 || P % C) return fail(CSSM_ERR_SHAPE, "cssm_irfft2_ex: P=%lld C=%d (P a multiple of C)", P, C);
  if (!cssm::fft_ex_supported(H, W))
    return fail(CSSM_ERR_UNSUPPORTED, "cssm_irfft2_ex: %dx%d planes (square powers of two 4..128)", H, W);
  if (!plane_set_ok(y, y_fs, C) || !plane_set_ok(m, m_fs, C) || !plane_set_ok(d, d_fs, C) || !aligned(spec, 8))
    return fail(CSSM_ERR_ALIGN, "cssm_irfft2_ex: plane sets need fs >= C and 16-byte alignment, spec 8");
  cssm::FftEx e{};
  e.m = {m, m_fs};
  e.d = {d, d_fs};
  e.y = y;
  e.y_fs = y_fs;
  e.add = add;
  e.sums = sums;
  e.C = C;
  return hip_status(cssm::launch_irfft2_ex(reinterpret_cast<const float2*>(spec), P, H, W, e,
                                           static_cast<hipStream_t>(stream)),
                    "cssm_irfft2_ex");
}

static int gdn_variant_check(const char* fn, int scan_variant) {
  if (scan_variant != CSSM_GDN_SCAN_GOOM && scan_variant != CSSM_GDN_SCAN_LINEAR && scan_variant != CSSM_GDN_SCAN_LOG_EPS)
    return fail(CSSM_ERR_ARG, "%s: scan_variant=%d (0 goom, 1 linear, 2 log-eps)", fn, scan_variant);
  return CSSM_OK;
}

int cssm_gdn_scan_bins(const float* spec, const float* norms, const float* ab, long long ab_frame, int ab_head,
                       int ab_bin, const float* what, int B, int T, int C, int H, int W, int dk, int scan_variant,
                       float* ohat, void* stream) {
  if (!spec || !ab || !what || !ohat) return fail(CSSM_ERR_NULL, "cssm_gdn_scan_bins: spec, ab, what and ohat must be non-null");
  if (int e = gdn_variant_check("cssm_gdn_scan_bins", scan_variant)) return e;
  if (B <= 0 || T <= 0 || C <= 0 || H <= 0 || W <= 0 || dk < 1 || dk > 4 || C % dk)
    return fail(CSSM_ERR_SHAPE, "cssm_gdn_scan_bins: B=%d T=%d C=%d H=%d W=%d d_k=%d (1..4, divides C)", B, T, C, H, W, dk);
  if (ab_frame < 0 || ab_head < 0 || ab_bin < 0) return fail(CSSM_ERR_ARG, "cssm_gdn_scan_bins: negative gate stride");
  if (B > 65535 || C / dk > 65535) return fail(CSSM_ERR_SHAPE, "cssm_gdn_scan_bins: grid too large");
  if (!aligned(spec, 8) || !aligned(ab, 8) || !aligned(what, 8) || !aligned(ohat, 8))
    return fail(CSSM_ERR_ALIGN, "cssm_gdn_scan_bins: complex tensors must be 8-byte aligned");
  return hip_status(cssm::launch_gdn_scan_bins(reinterpret_cast<const float2*>(spec), norms,
                                               reinterpret_cast<const float2*>(ab), ab_frame, ab_head, ab_bin,
                                               reinterpret_cast<const float2*>(what), B, T, C, H, W, dk,
                                               scan_variant, reinterpret_cast<float2*>(ohat),
                                               static_cast<hipStream_t>(stream)),
                    "cssm_gdn_scan_bins");
}

static int gdn_train_check(const char* fn, int B, int T, int C, int H, int W, int dk, long long ab_frame, int ab_head,
                           int ab_bin) {
  if (B <= 0 || T <= 0 || C <= 0 || H <= 0 || W <= 0 || dk < 1 || dk > 4 || C % dk)
    return fail(CSSM_ERR_SHAPE, "%s: B=%d T=%d C=%d H=%d W=%d d_k=%d (1..4, divides C)", fn, B, T, C, H, W, dk);
  if (ab_frame < 0 || ab_head < 0 || ab_bin < 0) return fail(CSSM_ERR_ARG, "%s: negative gate stride", fn);
  if (B > 65535 || C / dk > 65535) return fail(CSSM_ERR_SHAPE, "%s: grid too large", fn);
  return CSSM_OK;
}

int cssm_gdn_scan_bins_train(const float* spec, const float* ab, long long ab_frame, int ab_head, int ab_bin,
                             const float* what, int B, int T, int C, int H, int W, int dk, int scan_variant,
                             float* ohat, float* states, void* stream) {
  if (!spec || !ab || !what || !ohat || !states)
    return fail(CSSM_ERR_NULL, "cssm_gdn_scan_bins_train: spec, ab, what, ohat and states must be non-null");
  if (int e = gdn_train_check("cssm_gdn_scan_bins_train", B, T, C, H, W, dk, ab_frame, ab_head, ab_bin)) return e;
  if (int e = gdn_variant_check("cssm_gdn_scan_bins_train", scan_variant)) return e;
  if (!aligned(spec, 8) || !aligned(ab, 8) || !aligned(what, 8) || !aligned(ohat, 8) || !aligned(states, 8))
    return fail(CSSM_ERR_ALIGN, "cssm_gdn_scan_bins_train: complex tensors must be 8-byte aligned");
  return hip_status(cssm::launch_gdn_scan_bins_train(
                        reinterpret_cast<const float2*>(spec), reinterpret_cast<const float2*>(ab), ab_frame, ab_head,
                        ab_bin, reinterpret_cast<const float2*>(what), B, T, C, H, W, dk, scan_variant,
                        reinterpret_cast<float2*>(ohat), reinterpret_cast<float2*>(states), nullptr, nullptr, nullptr,
                        nullptr, false, static_cast<hipStream_t>(stream)),
                    "cssm_gdn_scan_bins_train");
}

int cssm_gdn_scan_bins_bwd(const float* spec, const float* ab, long long ab_frame, int ab_head, int ab_bin,
                           const float* what, const float* states, const float* dohat, int B, int T, int C, int H,
                           int W, int dk, int scan_variant, float* dspec, float* dab, float* dwhat, void* stream) {
  if (!spec || !ab || !what || !states || !dohat || !dspec || !dab || !dwhat)
    return fail(CSSM_ERR_NULL, "cssm_gdn_scan_bins_bwd: null argument");
  if (int e = gdn_train_check("cssm_gdn_scan_bins_bwd", B, T, C, H, W, dk, ab_frame, ab_head, ab_bin)) return e;
  if (int e = gdn_variant_check("cssm_gdn_scan_bins_bwd", scan_variant)) return e;
  if (!aligned(spec, 8) || !aligned(ab, 8) || !aligned(what, 8) || !aligned(states, 8) || !aligned(dohat, 8) ||
      !aligned(dspec, 8) || !aligned(dab, 8) || !aligned(dwhat, 8))
    return fail(CSSM_ERR_ALIGN, "cssm_gdn_scan_bins_bwd: complex tensors must be 8-byte aligned");
  return hip_status(cssm::launch_gdn_scan_bins_train(
                        reinterpret_cast<const float2*>(spec), reinterpret_cast<const float2*>(ab), ab_frame, ab_head,
                        ab_bin, reinterpret_cast<const float2*>(what), B, T, C, H, W, dk, scan_variant, nullptr,
                        const_cast<float2*>(reinterpret_cast<const float2*>(states)),
                        reinterpret_cast<const float2*>(dohat), reinterpret_cast<float2*>(dspec),
                        reinterpret_cast<float2*>(dab), reinterpret_cast<float2*>(dwhat), true,
                        static_cast<hipStream_t>(stream)),
                    "cssm_gdn_scan_bins_bwd");
}

int cssm_depthwise_conv_wgrad_supported(int W, int C, int ks) { return cssm::dwconv_wgrad_supported(W, C, ks) ? 1 : 0; }

int cssm_depthwise_conv_wgrad(const float* x, const float* dy, int F, int H, int W, int C, int ks, float* partial,
                              int blocks, void* stream) {
  if (!x || !dy || !partial) return fail(CSSM_ERR_NULL, "cssm_depthwise_conv_wgrad: null argument");
  if (F <= 0 || H <= 0 || W <= 0 || C <= 0 || blocks <= 0 || blocks > 65535)
    return fail(CSSM_ERR_SHAPE, "cssm_depthwise_conv_wgrad: F=%d H=%d W=%d C=%d blocks=%d", F, H, W, C, blocks);
  if (!cssm::dwconv_wgrad_supported(W, C, ks))
    return fail(CSSM_ERR_UNSUPPORTED, "cssm_depthwise_conv_wgrad: ks=%d C=%d W=%d (ks 3/5/7, C/4 dividing 64, W %% 8 == 0)",
                ks, C, W);
  if (!aligned(x, 16) || !aligned(dy, 16) || !aligned(partial, 16))
    return fail(CSSM_ERR_ALIGN, "cssm_depthwise_conv_wgrad: tensors must be 16-byte aligned");
  return hip_status(cssm::launch_dwconv_wgrad(x, dy, F, H, W, C, ks, partial, blocks, static_cast<hipStream_t>(stream)),
                    "cssm_depthwise_conv_wgrad");
}

int cssm_gdn_core_fused_supported(int H, int W, int delta_key_dim) {
  return cssm::gdn_core_fused_supported(H, W, delta_key_dim) ? 1 : 0;
}

int cssm_gdn_core_fused(const float* qkv, int use_l2, const float* ab, long long ab_frame, int ab_head, int ab_bin,
                        const float* what, int B, int T, int C, int H, int W, int delta_key_dim, int scan_variant,
                        float* o, void* stream) {
  if (!qkv || !ab || !what || !o) return fail(CSSM_ERR_NULL, "cssm_gdn_core_fused: null argument");
  if (int e = gdn_variant_check("cssm_gdn_core_fused", scan_variant)) return e;
  if (B <= 0 || T <= 0 || C <= 0 || H <= 0 || W <= 0 || delta_key_dim < 1 || delta_key_dim > 4 ||
      C % delta_key_dim || ab_frame < 0 || ab_head < 0 || ab_bin < 0)
    return fail(CSSM_ERR_SHAPE, "cssm_gdn_core_fused: B=%d T=%d C=%d H=%d W=%d d_k=%d", B, T, C, H, W,
                delta_key_dim);
  if (!cssm::gdn_core_fused_supported(H, W, delta_key_dim))
    return fail(CSSM_ERR_UNSUPPORTED, "cssm_gdn_core_fused: no fused core for %dx%d planes at d_k=%d", H, W,
                delta_key_dim);
  if (use_l2 != 0 && use_l2 != 1) return fail(CSSM_ERR_ARG, "cssm_gdn_core_fused: use_l2=%d", use_l2);
  if ((long long)B * T * 3 * C * H * W >= (1LL << 40)) return fail(CSSM_ERR_SHAPE, "cssm_gdn_core_fused: too large");
  if (!aligned(qkv, 16) || !aligned(o, 16) || !aligned(ab, 8) || !aligned(what, 8))
    return fail(CSSM_ERR_ALIGN, "cssm_gdn_core_fused: qkv and o must be 16-byte aligned, ab and what 8");
  return hip_status(cssm::launch_gdn_core_fused(qkv, use_l2, reinterpret_cast<const float2*>(ab), ab_frame, ab_head,
                                                ab_bin, reinterpret_cast<const float2*>(what), B, T, C, H, W,
                                                delta_key_dim, scan_variant, o, static_cast<hipStream_t>(stream)),
                    "cssm_gdn_core_fused");
}

int cssm_gdn_proj_out(const void* o, const void* gate, int in_dtype, int F, int HW, int K, int N, int norm,
                      const float* norm_scale, const float* norm_bias, const float* kernel, const float* bias, void* out,
                      int out_dtype, void* stream) {
  if (!o || !gate || !kernel || !bias || !out) return fail(CSSM_ERR_NULL, "cssm_gdn_proj_out: null argument");
  if (F <= 0 || HW <= 0 || K <= 0 || N <= 0) return fail(CSSM_ERR_SHAPE, "cssm_gdn_proj_out: F=%d HW=%d K=%d N=%d", F, HW, K, N);
  if (K > 128 || K % 4)
    return fail(CSSM_ERR_UNSUPPORTED, "cssm_gdn_proj_out: needs K <= 128, K %% 4 == 0 (K=%d)", K);
  if ((long long)F * HW > 0x7fffffffLL) return fail(CSSM_ERR_SHAPE, "cssm_gdn_proj_out: F*HW exceeds 2^31");
  if (!dtype_ok(in_dtype) || !dtype_ok(out_dtype)) return fail(CSSM_ERR_ARG, "cssm_gdn_proj_out: dtypes %d/%d", in_dtype, out_dtype);
  if (norm < CSSM_NORM_NONE || norm > CSSM_NORM_LAYER) return fail(CSSM_ERR_ARG, "cssm_gdn_proj_out: norm=%d", norm);
  const size_t va = in_dtype == CSSM_F32 ? 16 : 8;
  if (!aligned(o, va) || !aligned(gate, va) || (out_dtype == CSSM_F32 && !aligned(out, 16)))
    return fail(CSSM_ERR_ALIGN, "cssm_gdn_proj_out: misaligned o / gate / out");
  return hip_status(cssm::launch_proj_out_norm_gate(o, gate, in_dtype, F * HW, K, N, norm, norm_scale, norm_bias, kernel,
                                                    bias, HW, out, out_dtype, static_cast<hipStream_t>(stream)),
                    "cssm_gdn_proj_out");
}

int cssm_gdn_proj_out_xgate_supported(int K, int N, int HW) { return cssm::proj_out_xgate_supported(K, N, HW) ? 1 : 0; }

int cssm_gdn_proj_out_xgate(const void* o, int in_dtype, const void* x, int x_dtype, int F, int HW, int K, int N, int norm,
                            const float* norm_scale, const float* norm_bias, const float* gate_kernel,
                            const float* gate_bias, int gate_act, const float* kernel, const float* bias, void* out,
                            int out_dtype, void* stream) {
  if (!o || !x || !gate_kernel || !gate_bias || !kernel || !bias || !out)
    return fail(CSSM_ERR_NULL, "cssm_gdn_proj_out_xgate: null argument");
  if (F <= 0 || HW <= 0 || K <= 0 || N <= 0)
    return fail(CSSM_ERR_SHAPE, "cssm_gdn_proj_out_xgate: F=%d HW=%d K=%d N=%d", F, HW, K, N);
  if (!cssm::proj_out_xgate_supported(K, N, HW))
    return fail(CSSM_ERR_UNSUPPORTED, "cssm_gdn_proj_out_xgate: needs K <= 64, K %% 8 == 0, N <= 64, HW %% 4 == 0 "
                "(K=%d N=%d HW=%d)", K, N, HW);
  if ((long long)F * HW > 0x7fffffffLL) return fail(CSSM_ERR_SHAPE, "cssm_gdn_proj_out_xgate: F*HW exceeds 2^31");
  if (!dtype_ok(in_dtype) || !dtype_ok(out_dtype) || !dtype_ok(x_dtype))
    return fail(CSSM_ERR_ARG, "cssm_gdn_proj_out_xgate: dtypes %d/%d/%d", in_dtype, x_dtype, out_dtype);
  if (norm < CSSM_NORM_NONE || norm > CSSM_NORM_LAYER) return fail(CSSM_ERR_ARG, "cssm_gdn_proj_out_xgate: norm=%d", norm);
  if (gate_act != 1 && gate_act != 2) return fail(CSSM_ERR_ARG, "cssm_gdn_proj_out_xgate: gate_act=%d", gate_act);
  const size_t va = in_dtype == CSSM_F32 ? 16 : 8;
  if (!aligned(o, va) || !aligned(x, 16) || (out_dtype == CSSM_F32 && !aligned(out, 16)))
    return fail(CSSM_ERR_ALIGN, "cssm_gdn_proj_out_xgate: misaligned o / x / out");
  return hip_status(cssm::launch_proj_out_norm_xgate(o, in_dtype, x, x_dtype, F * HW, K, N, norm, norm_scale,
                                                     norm_bias, gate_kernel, gate_bias, gate_act, kernel, bias, HW,
                                                     out, out_dtype, static_cast<hipStream_t>(stream)),
                    "cssm_gdn_proj_out_xgate");
}

}  // extern "C"

// ---------------------------------------------------------------- CSSMSHViTBlock wiring

int cssm_block_norm_stats(const void* x, int dtype, int B, int T, int H, int W, int C, int mode, float eps,
                          float* stats, void* stream) {
  if (!x || !stats) return fail(CSSM_ERR_NULL, "cssm_block_norm_stats: x and stats must be non-null");
  if (B <= 0 || T <= 0 || H <= 0 || W <= 0 || C <= 0)
    return fail(CSSM_ERR_SHAPE, "cssm_block_norm_stats: B=%d T=%d H=%d W=%d C=%d", B, T, H, W, C);
  if (!dtype_ok(dtype)) return fail(CSSM_ERR_ARG, "cssm_block_norm_stats: dtype=%d", dtype);
  if (mode < 0 || mode > 2) return fail(CSSM_ERR_ARG, "cssm_block_norm_stats: mode=%d", mode);
  if (!(eps >= 0.0f)) return fail(CSSM_ERR_ARG, "cssm_block_norm_stats: eps must be >= 0");
  if (!aligned(stats, 8)) return fail(CSSM_ERR_ALIGN, "cssm_block_norm_stats: stats must be 8-byte aligned");
  return hip_status(cssm::launch_block_norm_stats(x, dtype, B, T, H, W, C, mode, eps, stats,
                                                  static_cast<hipStream_t>(stream)),
                    "cssm_block_norm_stats");
}

int cssm_block_norm_posconv(const void* x, int dtype, int B, int T_in, int T_out, int H, int W, int C, int mode,
                            const float* stats, const float* scale, const float* bias, const float* pos_kernel,
                            const float* pos_bias, void* out, void* stream) {
  if (!x || !stats || !scale || !bias || !out)
    return fail(CSSM_ERR_NULL, "cssm_block_norm_posconv: x, stats, scale, bias and out must be non-null");
  if ((pos_kernel == nullptr) != (pos_bias == nullptr))
    return fail(CSSM_ERR_NULL, "cssm_block_norm_posconv: pos_kernel and pos_bias come together");
  if (B <= 0 || T_in <= 0 || T_out <= 0 || H <= 0 || W <= 0 || C <= 0 || (T_in != 1 && T_in != T_out))
    return fail(CSSM_ERR_SHAPE, "cssm_block_norm_posconv: B=%d T_in=%d T_out=%d H=%d W=%d C=%d", B, T_in, T_out, H,
                W, C);
  if (!dtype_ok(dtype)) return fail(CSSM_ERR_ARG, "cssm_block_norm_posconv: dtype=%d", dtype);
  if (mode < 0 || mode > 2) return fail(CSSM_ERR_ARG, "cssm_block_norm_posconv: mode=%d", mode);
  if (x == out) return fail(CSSM_ERR_ARG, "cssm_block_norm_posconv: out must not alias x");
  if (!aligned(stats, 8)) return fail(CSSM_ERR_ALIGN, "cssm_block_norm_posconv: stats must be 8-byte aligned");
  return hip_status(cssm::launch_block_norm_posconv(x, dtype, B, T_in, T_out, H, W, C, mode, stats, scale, bias,
                                                    pos_kernel, pos_bias, out, static_cast<hipStream_t>(stream)),
                    "cssm_block_norm_posconv");
}

int cssm_block_residual(const void* res, int T_res, const void* y, int T_y, int dtype, int B, int T_out, int H,
                        int W, int C, int act, void* out, void* stream) {
  if (!res || !y || !out) return fail(CSSM_ERR_NULL, "cssm_block_residual: res, y and out must be non-null");
  if (B <= 0 || T_res <= 0 || T_y <= 0 || T_out <= 0 || H <= 0 || W <= 0 || C <= 0 ||
      (T_out != 1 && (T_res != T_out || T_y != T_out)))
    return fail(CSSM_ERR_SHAPE, "cssm_block_residual: B=%d T_res=%d T_y=%d T_out=%d H=%d W=%d C=%d", B, T_res, T_y,
                T_out, H, W, C);
  if (!dtype_ok(dtype)) return fail(CSSM_ERR_ARG, "cssm_block_residual: dtype=%d", dtype);
  if (act < 0 || act > 2) return fail(CSSM_ERR_ARG, "cssm_block_residual: act=%d", act);
  return hip_status(cssm::launch_block_residual(res, T_res, y, T_y, dtype, B, T_out, H, W, C, act, out,
                                                static_cast<hipStream_t>(stream)),
                    "cssm_block_residual");
}

// ---------------------------------------------------------------- input projection without allocation

// Device scratch of cssm_proj_in_noalloc: the ctx partial sums (one float per
// (row tile, frame slot, channel)), CSSM_PROJ_IN_SCRATCH_BYTES per device,
// held until the process ends.  Host code never passes this name to a kernel:
// its device address comes from hipGetSymbolAddress, once per device.
static __device__ __align__(256) float scratch[CSSM_PROJ_IN_SCRATCH_BYTES / sizeof(float)];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// device address of `scratch` on the current device (looked up on the first call per device)
int scratch_for_current_device(void** out, const char* what) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_status(e, what);
  if (dev < 0 || dev >= kMaxDevices) return fail(CSSM_ERR_UNSUPPORTED, "%s: device ordinal %d", what, dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_status(e, what);
    if (p == nullptr) return fail(CSSM_ERR_HIP, "%s: no device address for the scratch array", what);
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return CSSM_OK;
}

}  // namespace

extern "C" {

int cssm_proj_in_noalloc(const void* x, int in_dtype, int F, int HW, int K, int N, const float* kernel,
                         const float* bias, void* out_lo, void* out_hi, int out_dtype, int act_lo, int act_hi,
                         float* ctx, void* stream) {
  if (ctx != nullptr && F > 0 && HW > 0 && K > 0 && N > 0) {
    const size_t need = cssm_proj_in_workspace_size(F, HW, K, N);
    if (need > CSSM_PROJ_IN_SCRATCH_BYTES)
      return fail(CSSM_ERR_UNSUPPORTED,
                  "cssm_proj_in_noalloc: ctx of F=%d HW=%d K=%d N=%d needs %zu bytes of scratch, the static scratch "
                  "holds %zu (use cssm_proj_in with a workspace)",
                  F, HW, K, N, need, (size_t)CSSM_PROJ_IN_SCRATCH_BYTES);
  }
  void* ws = nullptr;
  if (ctx != nullptr) {
    const int st = scratch_for_current_device(&ws, "cssm_proj_in_noalloc");
    if (st != CSSM_OK) return st;
  }
  return cssm_proj_in(x, in_dtype, F, HW, K, N, kernel, bias, out_lo, out_hi, out_dtype, act_lo, act_hi, ctx, ws,
                      ws ? (size_t)CSSM_PROJ_IN_SCRATCH_BYTES : 0, stream);
}

}  // extern "C"
