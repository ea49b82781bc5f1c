// Internal launcher declarations shared by the kernel files and the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cssm {

struct GateWeights {
  const float* kd[3];
  const float* bd[3];
  const float* kw[3];
  const float* bw[3];
};

hipError_t launch_spectral_kernel(const float* k, int C, int K, int H, int W, float rho, int squash,
                                  int goom_floor, float2* khat, hipStream_t s);
hipError_t launch_plane_mean(const void* x, int dtype, long long nplanes, int HW, int act, float* out,
                             hipStream_t s);
hipError_t launch_gated_gates(const float* ctx, int BT, int C, int H, int W, int factored, int act,
                              const GateWeights& w, float c_scale, float4* gates, hipStream_t s);
// fused scan: plane sizes with a kernel, and the smallest plane group (C must be a multiple)
bool gated_scan_has_kernel(int H, int W);
int gated_scan_min_group(int H, int W);
// returns hipErrorInvalidValue if no kernel exists for the shape
hipError_t launch_gated_scan(const void* u, const void* z, void* y, int dtype, int B, int T, int C, int H,
                             int W, const float4* gates, const float2* khat, int u_act, int z_act,
                             hipStream_t s);

// projection GEMMs (fp32 MFMA)
// rows per proj_in tile (the channel partial sums come one per tile)
int proj_in_tile_rows(int K);
hipError_t launch_proj_in(const void* X, int in_dtype, int M, int K, int N, const float* W, const float* b, int HW,
                          void* out_lo, void* out_hi, int out_dtype, int act_lo, int act_hi, float* partial,
                          hipStream_t s);
hipError_t launch_proj_out(const void* Y, int in_dtype, int M, int K, int N, const float* W, const float* b, int HW,
                           void* out, int out_dtype, hipStream_t s);
hipError_t launch_ctx_reduce(const float* partial, int F, int tiles_per_frame, int C, float inv_hw, float* ctx,
                             hipStream_t s);

hipError_t launch_short_conv(const void* x, int in_dtype, int B, int T, int C, int H, int W, int ks, const float* ws,
                             const float* bs, int kt, const float* wt, const float* bt, void* u, int out_dtype,
                             float* ctx, hipStream_t s);

}  // namespace cssm
