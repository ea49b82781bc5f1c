// Backward of the fused gated scan (cssm_gated_scan_fwd) on gfx950: the
// spectral-domain reverse recurrence per (batch, frequency bin).
//
// The scan computes, per (b, c) plane and bin (true units; the forward kernel
// works on 2U and 2h and folds the factors into its gate planes):
//   A_t = Kf E_t,  P_t = DB_t U_t,  V_t = P_t, or VF_t where |P_t| < VF_t,
//   h_t = A_t h_{t-1} + V_t,  Y_t = Cs_t h_t,  y_t = irfft2(Y_t) z_t
// with the gate plane (E, DB, VF2, GCs) = (exp(-Delta), (Delta + 1e-8) B,
// 2 VF, C c_scale) and Kf the floored K_hat (cssm.py:559-581; the reference
// reaches these gradients through jax.value_and_grad of the log-space scan,
// main.py:283, whose custom VJPs are goom.py:47-137).  With gradients written
// as dL/dRe + i dL/dIm, the reverse pass is
//   g_t   = Cs_t dY_t + conj(A_{t+1}) g_{t+1}            (g_T = 0)
//   dA_t  = g_t conj(h_{t-1}),  dKf += E_t dA_t,  dE_t += Re(conj(Kf) dA_t)
//   dCs_t += Re(conj(h_t) dY_t)
//   unfloored: dU_t = DB_t g_t, dDB_t += Re(conj(U_t) g_t);  floored: dVF_t += Re(g_t)
// around the transforms' adjoints, which the caller runs as batched FFTs:
//   dY = rfft2(dy) c_v / (H W)         (y = irfft2(Y), C2R rule; c_v = 2 for
//                                       0 < v < W/2, else 1)
//   du = irfft2(dU H W / c_v)          (U = rfft2(u))
// One thread owns one bin of one batch element and walks every channel, so
// the channel sums of the gate gradients need no cross-thread reduction.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fft_reg.h"
#include "launch.h"

namespace cssm {

struct GatedBwdArgs {
  const float2* uspec;    // (B, T, C, H, WF) rfft2(u), natural column order
  const float2* dspec;    // (B, T, C, H, WF) rfft2(dy), natural order (dy = dL/dy_pre, y_pre = y / z)
  const float4* gates;    // (B, T, H, WF) (E, DB, VF2, GCs), scan column order
  const float2* khat;     // (C, H, WF) floored K_hat, scan layout (khat_pos)
  float2* yspec;          // (B, T, C, H, WF) out: Y_t = C h_t (irfft2 -> y_pre), natural order
  float2* sdu;            // (B, T, C, H, WF) out: dU_t H W / c_v (irfft2 -> du), natural order
  float4* dgates;         // (B, T, H, WF) out: (dE, dDB, dVF2, dGCs) summed over channels, scan order
  float2* dkhat;          // (B, C, H, WF) out: sum over t of E_t dA_t per batch element, khat's layout
  int T, C, H, W;
  float c_scale;          // the GCs = C c_scale of the gate planes
};

template <int MAXT>
__global__ void __launch_bounds__(256) gated_scan_bwd_bins(const GatedBwdArgs a) {
  const int H = a.H, W = a.W, WF = W / 2 + 1, HWF = H * WF;
  const int i = int(blockIdx.x) * 256 + int(threadIdx.x);
  if (i >= HWF) return;
  const int b = blockIdx.y, T = a.T, C = a.C;
  const int u = i / WF, p = i % WF, v = scan_col(H, W, p);
  const int nat = u * WF + v;                       // spectra: natural column order
  const int kpos = khat_pos(H, W, u, p);            // K_hat and its gradient: the scan's slot
  const float cv = (v == 0 || 2 * v == W) ? 1.0f : 2.0f;
  const float dscale = cv / float(H * W), uscale = float(H * W) / cv, inv_cs = 1.0f / a.c_scale;

  float4 g[MAXT], gs[MAXT];
#pragma unroll
  for (int t = 0; t < MAXT; ++t) {
    g[t] = t < T ? a.gates[(size_t(b) * T + t) * HWF + i] : make_float4(0.f, 0.f, 0.f, 0.f);
    gs[t] = make_float4(0.f, 0.f, 0.f, 0.f);
  }
  // the spectra do not alias the outputs, and channel c + 1's U and dY are loaded while channel c
  // computes and stores (without that, each channel's loads waited behind its own stores)
  const float2* __restrict__ us = a.uspec;
  const float2* __restrict__ dsp = a.dspec;
  const float2* __restrict__ kh = a.khat;
  float2* __restrict__ ys = a.yspec;
  float2* __restrict__ sd = a.sdu;
  auto fetch = [&](int c, float2& kn, float2 (&Uo)[MAXT], float2 (&Do)[MAXT]) {
    kn = kh[size_t(c) * HWF + kpos];
#pragma unroll
    for (int t = 0; t < MAXT; ++t) {
      if (t >= T) break;
      const size_t s = ((size_t(b) * T + t) * C + c) * HWF + nat;
      Uo[t] = us[s];
      Do[t] = dsp[s];
    }
  };
  // one channel ahead for T <= 8; at T <= 32 a second set of U and dY would exceed the register file,
  // so each channel's loads are issued at its top (still ahead of its stores)
  constexpr bool AHEAD = MAXT <= 8;
  float2 kn;
  float2 Un[AHEAD ? MAXT : 1], Dn[AHEAD ? MAXT : 1];
  if constexpr (AHEAD) fetch(0, kn, Un, Dn);
  for (int c = 0; c < C; ++c) {
    float2 h[MAXT], U[MAXT], D[MAXT];
    if constexpr (AHEAD) {
#pragma unroll
      for (int t = 0; t < MAXT; ++t) {
        U[t] = Un[t];
        D[t] = Dn[t];
      }
    } else {
      fetch(c, kn, U, D);
    }
    const float2 kf = kn;
    if constexpr (AHEAD) {
      if (c + 1 < C) fetch(c + 1, kn, Un, Dn);
    }
    float2 hp = make_float2(0.f, 0.f);
#pragma unroll
    for (int t = 0; t < MAXT; ++t) {
      if (t >= T) break;
      const size_t s = ((size_t(b) * T + t) * C + c) * HWF + nat;
      const float2 A = cscale(kf, g[t].x);
      const float2 P = cscale(U[t], g[t].y);
      const float vf = 0.5f * g[t].z;
      const float2 V = (P.x * P.x + P.y * P.y < vf * vf) ? make_float2(vf, 0.f) : P;
      hp = cadd(cmul(A, hp), V);
      h[t] = hp;
      ys[s] = cscale(hp, g[t].w * inv_cs);
    }
    float2 carry = make_float2(0.f, 0.f);             // conj(A_{t+1}) g_{t+1}
    float2 dkf = make_float2(0.f, 0.f);
#pragma unroll
    for (int tt = MAXT - 1; tt >= 0; --tt) {
      if (tt >= T) continue;
      const size_t s = ((size_t(b) * T + tt) * C + c) * HWF + nat;
      const float2 dY = cscale(D[tt], dscale);
      const float Ct = g[tt].w * inv_cs;
      const float2 gt = cadd(cscale(dY, Ct), carry);
      gs[tt].w += (h[tt].x * dY.x + h[tt].y * dY.y) * inv_cs;
      const float2 hprev = tt > 0 ? h[tt > 0 ? tt - 1 : 0] : make_float2(0.f, 0.f);
      const float2 dA = cmulc(gt, hprev);                // g conj(h_{t-1})
      gs[tt].x += kf.x * dA.x + kf.y * dA.y;             // Re(conj(Kf) dA)
      dkf = cadd(dkf, cscale(dA, g[tt].x));
      const float2 P = cscale(U[tt], g[tt].y);
      const float vf = 0.5f * g[tt].z;
      float2 dU = make_float2(0.f, 0.f);
      if (P.x * P.x + P.y * P.y < vf * vf) {
        gs[tt].z += 0.5f * gt.x;                         // VF = VF2 / 2
      } else {
        gs[tt].y += U[tt].x * gt.x + U[tt].y * gt.y;     // Re(conj(U) g)
        dU = cscale(gt, g[tt].y);
      }
      sd[s] = cscale(dU, uscale);
      const float2 A = cscale(kf, g[tt].x);
      carry = cmulc(gt, A);                              // conj(A_t) g_t
    }
    a.dkhat[(size_t(b) * C + c) * HWF + kpos] = dkf;
  }
#pragma unroll
  for (int t = 0; t < MAXT; ++t)
    if (t < T) a.dgates[(size_t(b) * T + t) * HWF + i] = gs[t];
}

hipError_t launch_gated_scan_bwd_bins(const float2* uspec, const float2* dspec, const float4* gates,
                                      const float2* khat, int B, int T, int C, int H, int W, float c_scale,
                                      float2* yspec, float2* sdu, float4* dgates, float2* dkhat, hipStream_t s) {
  GatedBwdArgs a{uspec, dspec, gates, khat, yspec, sdu, dgates, dkhat, T, C, H, W, c_scale};
  const int hwf = H * (W / 2 + 1);
  const dim3 grid(unsigned((hwf + 255) / 256), unsigned(B));
  if (T <= 8) hipLaunchKernelGGL(gated_scan_bwd_bins<8>, grid, dim3(256), 0, s, a);
  else if (T <= 32) hipLaunchKernelGGL(gated_scan_bwd_bins<32>, grid, dim3(256), 0, s, a);
  else return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace cssm
