// Internal launcher declarations shared by the kernel files and the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cssm {

// Column order of the per-bin planes the gated scan reads (gates, K_hat):
// position p of a row holds frequency column scan_col(H, W, p).  At 128 x 128
// the 64 packed columns are interleaved so that the eight columns a wave owns
// in the column passes lie in four row blocks at two pair positions (spread
// over the LDS banks) while its per-bin loads still cover whole 128-byte
// lines: positions 8 g .. 8 g + 7 map to blocks 4 (g % 4) + 0..3 at pairs
// 2 (g / 4) + {0, 1}.  The Nyquist column stays last; every other plane size
// keeps the natural order.
__host__ __device__ inline int scan_col(int H, int W, int p) {
  if (H != 128 || W != 128 || p >= 64) return p;
  const int qc = p % 8, g = p / 8;
  return 4 * (g % 4) + qc % 4 + 16 * (2 * (g / 4) + qc / 4);
}

// Slot (in float2 units, within one channel's H x (W/2+1) plane) of K_hat's
// bin at row u, column position p of the scan layout.  At 128 x 128 the rows u
// and u + 16 with (u / 16) even share each column's 16-byte slot pairs, so a
// column-pass lane, whose bins are rows k + 16 q, reads the bins of q and q + 1
// with one 16-byte load over whole cache lines; every other plane size keeps
// row-major order (u (W/2+1) + p).
__host__ __device__ inline int khat_pos(int H, int W, int u, int p) {
  const int WF = W / 2 + 1;
  if (H != 128 || W != 128) return u * WF + p;
  return ((u % 16 + 16 * (u / 32)) * WF + p) * 2 + (u / 16) % 2;
}

struct GateWeights {
  const float* kd[3];
  const float* bd[3];
  const float* kw[3];
  const float* bw[3];
};

// The projection's per-tile channel sums of ctx (cssm_proj_in's workspace): tile t of TM rows
// holds, for each of its slots' frames f, partial[(t slots + f - first frame of t) C + c].
struct CtxPartials {
  const float* partial;   // nullptr: ctx comes as (F, C) floats instead
  int HW, TM, slots;
  float* ctx;             // (F, C) mean written here as well (may be nullptr)
};

// Sum over the row tiles t0 + gi, t0 + gi + G, ... <= t1 of frame f's partial sums of channel
// c, in tile order with four loads in flight: one of G strided groups (the ctx reductions add
// the G group sums in group order, so ctx is deterministic and the same in every kernel that
// reduces it).
__device__ __forceinline__ float ctx_tile_sum(const float* __restrict__ partial, int f, int HW, int TM, int slots,
                                              int C, int c, int gi, int G) {
  const long long r0 = (long long)f * HW, r1 = r0 + HW - 1;
  const long long t0 = r0 / TM, t1 = r1 / TM;
  float s = 0.0f;
  long long t = t0 + gi;
  for (; t + 3 * G <= t1; t += 4 * G) {
    float v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const long long tt = t + u * G;
      v[u] = partial[(size_t(tt) * slots + int(f - (tt * TM) / HW)) * C + c];
    }
    s += v[0];
    s += v[1];
    s += v[2];
    s += v[3];
  }
  for (; t <= t1; t += G) s += partial[(size_t(t) * slots + int(f - (t * TM) / HW)) * C + c];
  return s;
}

hipError_t launch_spectral_kernel(const float* k, int C, int K, int H, int W, float rho, int squash,
                                  int goom_floor, int scan_order, float2* khat, hipStream_t s);
hipError_t launch_plane_mean(const void* x, int dtype, long long nplanes, int HW, int act, float* out,
                             hipStream_t s);
hipError_t launch_gated_gates(const float* ctx, const CtxPartials& cp, int BT, int C, int H, int W, int factored,
                              int act, const GateWeights& w, float c_scale, float4* gates, hipStream_t s);
// adjoint of launch_gated_gates: out = dG (BT, 3, H*WF) dense, or the factor gradients (BT, 3, H + WF)
hipError_t launch_gated_gates_bwd(const float* ctx, int BT, int C, int H, int W, int factored, int act,
                                  const GateWeights& w, float c_scale, const float4* dgates, float* out,
                                  hipStream_t s);
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
int proj_in_ctx_slots(int K, int HW);
hipError_t launch_proj_in(const void* X, int in_dtype, int M, int K, int N, const float* W, const float* b, int HW,
                          void* out_lo, void* out_hi, int out_dtype, int act_lo, int act_hi, float* partial,
                          hipStream_t s);
hipError_t launch_proj_out(const void* Y, int in_dtype, int M, int K, int N, const float* W, const float* b, int HW,
                           void* out, int out_dtype, hipStream_t s);
// single plane-major output (NH = N) or a split at channel NH; act 0 / 1 SiLU / 2 sigmoid
hipError_t launch_proj_planes(const void* X, int in_dtype, int M, int K, int N, const float* W, const float* b,
                              int HW, void* out_lo, void* out_hi, int out_dtype, int act_lo, int act_hi,
                              float* partial, int NH, hipStream_t s);
// output projection of plane-major Y with the per-pixel channel norm and gate G fused in front
hipError_t launch_proj_out_norm_gate(const void* Y, const void* G, int in_dtype, int M, int K, int N, int norm,
                                     const float* nscale, const float* nshift, const float* W, const float* b, int HW,
                                     void* out, int out_dtype, hipStream_t s);
// the same with the gate act(X wg + bg) computed in the kernel from the layer input X (x_dtype 0: f32,
// 1: bf16) (proj.hip)
bool proj_out_xgate_supported(int K, int N, int HW);
hipError_t launch_proj_out_norm_xgate(const void* Y, int in_dtype, const void* X, int x_dtype, int M, int K, int N,
                                      int norm, const float* nscale, const float* nshift, const float* wg,
                                      const float* bg, int gact, const float* W, const float* b, int HW, void* out,
                                      int out_dtype, hipStream_t s);
hipError_t launch_ctx_reduce(const float* partial, int F, int HW, int tile_rows, int slots, int C, float* ctx,
                             hipStream_t s);

hipError_t launch_short_conv(const void* x, int in_dtype, int B, int T, int C, int H, int W, int ks, const float* ws,
                             const float* bs, int kt, const float* wt, const float* bt, void* u, int out_dtype,
                             float* ctx, hipStream_t s);

// ---- GatedDeltaNetCSSM
// gate weights: index 0 alpha, 1 beta, 2 B_k, 3 B_v; kind 0 dense, 1 factored, 2 channel, 3 scalar.
// kd/bd: dense / channel / scalar kernel and bias, or the factored row (_h) pair; kw/bw: factored column (_w).
// kd[g] == nullptr skips gate g.
struct GdnGateWeights {
  int kind;
  const float* kd[4];
  const float* bd[4];
  const float* kw[4];
  const float* bw[4];
};
// causal short convolutions of the q / k / v blocks: kernel (kt, 1, C), bias (C)
struct GdnShortConv {
  const float* w[3];
  const float* b[3];
};

hipError_t launch_rfft2(const void* x, int dtype, long long P, int H, int W, float2* spec, float* norms,
                        hipStream_t s);
hipError_t launch_irfft2(const float2* spec, long long P, int H, int W, void* y, int dtype, hipStream_t s);
// training-path transforms with fused load / store work on strided float32 plane sets (gdn.hip):
// plane p = f C + c of a set (p, fs) starts at p + (f fs + c) H W
struct PlaneSet {
  const float* p;
  int fs;
  __device__ __forceinline__ size_t off(long long plane, int C, int HW) const {
    return (size_t(plane / C) * size_t(fs) + size_t(plane % C)) * size_t(HW);
  }
};
struct FftEx {
  PlaneSet x, a;      // rfft2: input and optional factor (a.p null: none)
  int x_act, a_act;   // cssm_load_act of each
  PlaneSet m, d;      // irfft2: optional factor m and SiLU'-argument d
  float* y;           // irfft2: output set (fs y_fs)
  int y_fs;
  const float* add;   // irfft2: per-plane addend, or null
  float* sums;        // irfft2: per-plane sums of y (P), or null (plane groups whose waves each hold one plane)
  int C;
};
bool irfft2_ex_sums_supported(long long P, int H, int W);
// im2col of a SAME ks x ks conv over channels-last frames: rows (F H W) x (ks ks C) float32 (gdn.hip)
hipError_t launch_im2col_same(const void* x, int dtype, long long rows, int H, int W, int C, int ks, float* out,
                              hipStream_t s);
bool fft_ex_supported(int H, int W);
hipError_t launch_rfft2_ex(const FftEx& e, long long P, int H, int W, float2* spec, hipStream_t s);
hipError_t launch_irfft2_ex(const float2* spec, long long P, int H, int W, const FftEx& e, hipStream_t s);
int fft_planes_min_group(int H, int W);
hipError_t launch_gdn_scan_bins(const float2* spec, const float* norms, const float2* ab, long long ab_frame,
                                int ab_head, int ab_bin, const float2* what, int B, int T, int C, int H, int W,
                                int dk, int variant, float2* ohat, hipStream_t s);
// weight gradient of the depthwise SAME conv of channels-last frames: per-block partial sums
// (blocks, ks*ks, C) for the caller to add; gdn_bwd.hip
bool dwconv_wgrad_supported(int W, int C, int ks);
hipError_t launch_dwconv_wgrad(const float* x, const float* dy, int F, int H, int W, int C, int ks, float* partial,
                               int blocks, hipStream_t s);
// training: forward with the state entering every step saved (backward = false), or the reverse
// pass from those states (backward = true); gdn_bwd.hip
hipError_t launch_gdn_scan_bins_train(const float2* spec, const float2* ab, long long ab_frame, int ab_head,
                                      int ab_bin, const float2* what, int B, int T, int C, int H, int W, int dk,
                                      int variant, float2* ohat, float2* states, const float2* dohat, float2* dspec,
                                      float2* dab, float2* dwhat, bool backward, hipStream_t s);
// backward of the gated scan: the spectral-domain reverse recurrence per (b, bin), T <= 32
hipError_t launch_gated_scan_bwd_bins(const float2* uspec, const float2* dspec, const float4* gates,
                                      const float2* khat, int B, int T, int C, int H, int W, float c_scale,
                                      float2* yspec, float2* sdu, float4* dgates, float2* dkhat, hipStream_t s);
// the GDN spectral core in one kernel (32 x 32 planes, d_k = 4): rfft2 -> norms -> delta rule -> irfft2
bool gdn_core_fused_supported(int H, int W, int dk);
hipError_t launch_gdn_core_fused(const float* qkv, int use_l2, const float2* ab, long long ab_frame, int ab_head,
                                 int ab_bin, const float2* what, int B, int T, int C, int H, int W, int dk, int variant,
                                 float* o, hipStream_t s);
hipError_t launch_frame_mean(const void* x, int dtype, int F, int HW, int C, float* out, hipStream_t s);
hipError_t launch_gdn_gates(const float* ctx, int B, int T, int C, int H, int W, int nh, const GdnGateWeights& w,
                            int temporal, float rope_base, const float* ttable, float2* ab, float2* bkv,
                            hipStream_t s);
hipError_t launch_depthwise_conv(const void* x, int dtype, int F, int H, int W, int C, int ks, const float* kw,
                                 const float* bias, void* y, int out_dtype, hipStream_t s);
// the depthwise conv and the per-(frame, channel) mean of x in one pass (the blocked kernel's centre
// taps): part (F, blocks, C) workspace, ctx (F, C); blocks = depthwise_conv_mean_blocks(...) > 0
int depthwise_conv_mean_blocks(int F, int H, int W, int C, int ks);
hipError_t launch_depthwise_conv_mean(const void* x, int dtype, int F, int H, int W, int C, int ks, const float* kw,
                                      const float* bias, void* y, int out_dtype, float* part, float* ctx,
                                      hipStream_t s);
hipError_t launch_gdn_qkv_post(void* qkv, int dtype, int B, int T, int C, int HW, int kt, const GdnShortConv& sc,
                               int gate_mode, const void* gates, hipStream_t s);
// qkv_proj + short conv + SiLU + input gates: one fused launch when gdn_qkv_fused_supported(T, HW, K, kt), else the two.
// With wg != nullptr also gate_proj of the same rows (wg (K, C), bg (C), act gact) into gv (B, T, C, HW): fused as
// C more columns of the same launch, else one more projection.
hipError_t launch_gdn_qkv_proj(const void* X, int in_dtype, int B, int T, int HW, int K, int C, const float* W,
                               const float* b, int kt, const GdnShortConv& sc, int gate_mode, const void* gates,
                               void* out, int out_dtype, hipStream_t s, const float* wg = nullptr,
                               const float* bg = nullptr, int gact = 0, void* gv = nullptr);
bool gdn_qkv_fused_supported(int T, int HW, int K, int kt);

// ---- CSSMSHViTBlock wiring (block.hip)
// norm1 statistics: mode 0 global_layer (per b), 1 temporal_layer (per b, pixel), 2 layer (per b, t, pixel);
// stats (groups, 2) = (mean, rsqrt(var + eps))
hipError_t launch_block_norm_stats(const void* x, int dtype, int B, int T, int H, int W, int C, int mode, float eps,
                                   float* stats, hipStream_t s);
hipError_t launch_block_norm_posconv(const void* x, int dtype, int B, int T_in, int T_out, int H, int W, int C,
                                     int mode, const float* stats, const float* scale, const float* bias,
                                     const float* pk, const float* pb, void* out, hipStream_t s);
hipError_t launch_block_residual(const void* res, int T_res, const void* y, int T_y, int dtype, int B, int T_out,
                                 int H, int W, int C, int act, void* out, hipStream_t s);

}  // namespace cssm
