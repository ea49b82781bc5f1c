// extern "C" entry points of libcssm_hip.so (declared in include/cssm_amd.h).
// Argument checking lives here; kernels assume validated shapes.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

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
                         int goom_floor, float* khat, void* stream) {
  if (!k || !khat) return fail(CSSM_ERR_NULL, "cssm_spectral_kernel: k and khat must be non-null");
  if (C <= 0 || K <= 0 || H <= 0 || W <= 0)
    return fail(CSSM_ERR_SHAPE, "cssm_spectral_kernel: C=%d K=%d H=%d W=%d must be positive", C, K, H, W);
  if ((K > H || K > W) && (K < H || K < W))
    return fail(CSSM_ERR_SHAPE,
                "cssm_spectral_kernel: K=%d lies between H=%d and W=%d (reference pad/crop undefined)", K,
                H, W);
  if (!aligned(khat, 8)) return fail(CSSM_ERR_ALIGN, "cssm_spectral_kernel: khat must be 8-byte aligned");
  const hipError_t e = cssm::launch_spectral_kernel(k, C, K, H, W, rho, squash, goom_floor,
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

int cssm_gated_gates(const float* ctx, int B, int T, int C, int H, int W, const cssm_gate_params* p,
                     float c_scale, float* gates, void* stream) {
  if (!ctx || !p || !gates) return fail(CSSM_ERR_NULL, "cssm_gated_gates: ctx, params and gates must be non-null");
  if (B <= 0 || T <= 0 || C <= 0 || H <= 0 || W <= 0)
    return fail(CSSM_ERR_SHAPE, "cssm_gated_gates: B=%d T=%d C=%d H=%d W=%d", B, T, C, H, W);
  if (p->gate_type != CSSM_GATE_DENSE && p->gate_type != CSSM_GATE_FACTORED)
    return fail(CSSM_ERR_ARG, "cssm_gated_gates: gate_type=%d", p->gate_type);
  if (p->activation < CSSM_ACT_SOFTPLUS || p->activation > CSSM_ACT_EXP)
    return fail(CSSM_ERR_ARG, "cssm_gated_gates: activation=%d", p->activation);
  const bool fac = p->gate_type == CSSM_GATE_FACTORED;
  cssm::GateWeights w;
  for (int i = 0; i < 3; ++i) {
    if (!p->kernel[i] || !p->bias[i] || (fac && (!p->kernel_w[i] || !p->bias_w[i])))
      return fail(CSSM_ERR_NULL, "cssm_gated_gates: gate %d weights missing", i);
    w.kd[i] = p->kernel[i];
    w.bd[i] = p->bias[i];
    w.kw[i] = fac ? p->kernel_w[i] : nullptr;
    w.bw[i] = fac ? p->bias_w[i] : nullptr;
  }
  if (!aligned(gates, 16)) return fail(CSSM_ERR_ALIGN, "cssm_gated_gates: gates must be 16-byte aligned");
  const hipError_t e = cssm::launch_gated_gates(ctx, B * T, C, H, W, fac ? 1 : 0, p->activation, w, c_scale,
                                                reinterpret_cast<float4*>(gates),
                                                static_cast<hipStream_t>(stream));
  if (e == hipErrorInvalidValue)
    return fail(CSSM_ERR_UNSUPPORTED, "cssm_gated_gates: C=%d with %dx%d planes exceeds the staging buffer", C, H, W);
  return hip_status(e, "cssm_gated_gates");
}

int cssm_gated_scan_supported(int H, int W) { return cssm::gated_scan_has_kernel(H, W) ? 1 : 0; }

int cssm_gated_scan_min_group(int H, int W) { return cssm::gated_scan_min_group(H, W); }

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

size_t cssm_proj_in_workspace_size(int F, int HW, int K, int N) {
  if (F <= 0 || HW <= 0 || K <= 0 || N <= 0) return 0;
  const int tm = cssm::proj_in_tile_rows(K);
  if (HW % tm != 0) return 0;
  return size_t(F) * (HW / tm) * (N / 2) * sizeof(float);
}

int cssm_proj_in(const void* x, int in_dtype, int F, int HW, int K, int N, const float* kernel, const float* bias,
                 void* out_lo, void* out_hi, int out_dtype, int act_lo, int act_hi, float* ctx, void* workspace,
                 size_t workspace_bytes, void* stream) {
  if (!x || !kernel || !bias || !out_lo || !out_hi)
    return fail(CSSM_ERR_NULL, "cssm_proj_in: x, kernel, bias, out_lo and out_hi must be non-null");
  if (F <= 0 || HW <= 0 || K <= 0 || N <= 0 || (N % 2) != 0)
    return fail(CSSM_ERR_SHAPE, "cssm_proj_in: F=%d HW=%d K=%d N=%d (N must be even)", F, HW, K, N);
  if ((long long)F * HW > 0x7fffffffLL) return fail(CSSM_ERR_SHAPE, "cssm_proj_in: F*HW exceeds 2^31");
  if ((in_dtype != CSSM_F32 && in_dtype != CSSM_BF16) || (out_dtype != CSSM_F32 && out_dtype != CSSM_BF16))
    return fail(CSSM_ERR_ARG, "cssm_proj_in: dtypes %d/%d", in_dtype, out_dtype);
  if ((act_lo != CSSM_LOAD_IDENTITY && act_lo != CSSM_LOAD_SILU) || (act_hi != CSSM_LOAD_IDENTITY && act_hi != CSSM_LOAD_SILU))
    return fail(CSSM_ERR_ARG, "cssm_proj_in: act_lo=%d act_hi=%d", act_lo, act_hi);
  if (out_dtype == CSSM_F32 && (!aligned(out_lo, 16) || !aligned(out_hi, 16)))
    return fail(CSSM_ERR_ALIGN, "cssm_proj_in: f32 outputs must be 16-byte aligned");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int M = F * HW;
  const int tm = cssm::proj_in_tile_rows(K);
  const bool fused_ctx = ctx != nullptr && (HW % tm) == 0;
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
    e = fused_ctx ? cssm::launch_ctx_reduce(partial, F, HW / tm, N / 2, 1.0f / float(HW), ctx, s)
                  : cssm::launch_plane_mean(out_lo, out_dtype, (long long)F * (N / 2), HW, 0, ctx, s);
  }
  return hip_status(e, "cssm_proj_in");
}

int cssm_proj_out(const void* y, int in_dtype, int F, int HW, int K, int N, const float* kernel, const float* bias,
                  void* out, int out_dtype, void* stream) {
  if (!y || !kernel || !bias || !out)
    return fail(CSSM_ERR_NULL, "cssm_proj_out: y, kernel, bias and out must be non-null");
  if (F <= 0 || HW <= 0 || K <= 0 || N <= 0) return fail(CSSM_ERR_SHAPE, "cssm_proj_out: F=%d HW=%d K=%d N=%d", F, HW, K, N);
  if ((long long)F * HW > 0x7fffffffLL) return fail(CSSM_ERR_SHAPE, "cssm_proj_out: F*HW exceeds 2^31");
  if ((in_dtype != CSSM_F32 && in_dtype != CSSM_BF16) || (out_dtype != CSSM_F32 && out_dtype != CSSM_BF16))
    return fail(CSSM_ERR_ARG, "cssm_proj_out: dtypes %d/%d", in_dtype, out_dtype);
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
