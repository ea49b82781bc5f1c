// Training kernels of GatedDeltaNetCSSM's spectral recurrence on gfx950: the
// forward that keeps each step's incoming state, and the reverse pass per
// (batch, head, frequency bin).
//
// Per bin, with q, k, v the step's d_k-vectors (q and k after the spectral L2
// norms, which the caller applies; k raw here and normalised per bin) and
// aW = alpha W_hat (cssm.py:4890-5000; the reference reaches these gradients
// through jax.value_and_grad of its log-space general matrix scan, main.py:283,
// with the custom VJPs of goom.py:47-137):
//   k' = k / sqrt(|k|^2 + 1e-6)
//   M = floor(aW (I - beta k' k'^H)),  D[i][r] = floor(beta v_i conj(k'_r))
//   s_t[i][r] = sum_c M[r][c] s_{t-1}[i][c] + D[i][r],   o_t[i] = sum_r s_t[i][r] q_r
// With gradients written as dL/dRe + i dL/dIm, the reverse pass carries
// g = dL/ds_t backwards:
//   g[i][r] = carry[i][r] + do[i] conj(q_r),   dq_r = sum_i do[i] conj(s_t[i][r])
//   carry'[i][c] = sum_r conj(M[r][c]) g[i][r]
//   dM[r][c] = sum_i g[i][r] conj(s_{t-1}[i][c]),  dD[i][r] = g[i][r]
// and through M = aW m, m = delta - beta k'_r conj(k'_c), D = beta v_i conj(k'_r)
// into aW, beta, k', v.  A floored entry is the constant 1e-7: it passes no
// gradient to its inputs (the carry still uses the floored value, as the
// forward did).  The other scan variants (gdn_step.h): the linear scan maps no
// entry; the log-eps scan's map f(x) = x (1 + 1e-8 / |x|) stretches the
// tangential part of the gradient, df^T g = g + (1e-8 / |x|) Re(conj(g) i u) i u
// with u = x / |x| (its constant 1e-8 at x = 0 passes none).
// The key normalisation's backward is
//   dk = n dk' - n^3 k Re(sum_l dk'_l conj(k_l)),   n = (|k|^2 + 1e-6)^(-1/2).
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "gdn_step.h"
#include "launch.h"

namespace cssm {

struct GdnTrainArgs {
  const float2* spec;    // (B, T, 3C, H, WF): q and k with the spectral norms applied, v
  const float2* ab;      // (alpha, beta) at (b T + t) ab_frame + head ab_head + bin ab_bin
  long long ab_frame;
  int ab_head, ab_bin;
  const float2* what;    // (n_h, H, WF)
  float2* ohat;          // (B, T, C, H, WF) forward out
  float2* states;        // (B, T, n_h, DK, DK, H WF): s_{t-1} of step t (forward out, reverse in)
  const float2* dohat;   // (B, T, C, H, WF) reverse in
  float2* dspec;         // (B, T, 3C, H, WF) reverse out
  float2* dab;           // (B, T, n_h, H WF) reverse out: (dalpha, dbeta) of each (head, bin)
  float2* dwhat;         // (B, n_h, H WF) reverse out: dW_hat summed over t, per batch element
  int T, C, HWF;
  int variant;           // kScanGoom / kScanLinear / kScanLogEps (gdn_step.h)
};

template <int DK>
__device__ __forceinline__ size_t state_at(const GdnTrainArgs& a, int b, int t, int head, int i, int c, int bin) {
  const int nh = a.C / DK;
  return ((((size_t(b) * a.T + t) * nh + head) * DK + i) * DK + c) * a.HWF + bin;
}

template <int DK>
__global__ void __launch_bounds__(256) gdn_scan_bins_save(const GdnTrainArgs a) {
  const int bin = blockIdx.x * blockDim.x + threadIdx.x;
  if (bin >= a.HWF) return;
  const int head = blockIdx.y, b = blockIdx.z;
  const int C = a.C, HWF = a.HWF;
  const float2 wh = a.what[size_t(head) * HWF + bin];
  float2 s[DK][DK];
#pragma unroll
  for (int i = 0; i < DK; ++i)
#pragma unroll
    for (int j = 0; j < DK; ++j) s[i][j] = make_float2(0.f, 0.f);
  for (int t = 0; t < a.T; ++t) {
    const size_t fr = size_t(b) * a.T + t;
    const size_t ch0 = fr * 3 * C + size_t(head) * DK;
    float2 q[DK], k[DK], v[DK];
#pragma unroll
    for (int j = 0; j < DK; ++j) {
      q[j] = a.spec[(ch0 + j) * HWF + bin];
      k[j] = a.spec[(ch0 + C + j) * HWF + bin];
      v[j] = a.spec[(ch0 + 2 * C + j) * HWF + bin];
    }
#pragma unroll
    for (int i = 0; i < DK; ++i)
#pragma unroll
      for (int c = 0; c < DK; ++c) a.states[state_at<DK>(a, b, t, head, i, c, bin)] = s[i][c];
    const float2 g = a.ab[fr * a.ab_frame + size_t(head) * a.ab_head + size_t(bin) * a.ab_bin];
    float2 o[DK];
    gdn_bin_step<DK>(s, q, k, v, wh, g.x, g.y, a.variant, o);
#pragma unroll
    for (int i = 0; i < DK; ++i) a.ohat[(fr * C + size_t(head) * DK + i) * HWF + bin] = o[i];
  }
}

// an entry x of M or Delta as the scan variant sees it, and whether that value is a constant
// (to_goom's floor took x, or the log-eps map's 1e-8 at x = 0), which passes no gradient to x
__device__ __forceinline__ float2 mapped_entry(float2 x, int variant, bool& frozen) {
  const float r2 = x.x * x.x + x.y * x.y;
  if (variant == kScanLinear) {
    frozen = false;
    return x;
  }
  if (variant == kScanLogEps) {
    frozen = r2 == 0.0f;
    return logeps_entry(x);
  }
  frozen = r2 < 1e-14f;
  return frozen ? make_float2(1e-7f, 0.0f) : x;
}

// dL/dx from g = dL/d mapped_entry(x) where that value is not a constant
__device__ __forceinline__ float2 entry_adjoint(float2 g, float2 x, int variant) {
  if (variant != kScanLogEps) return g;
  const float rinv = rsqrtf(fmaf(x.x, x.x, x.y * x.y));
  const float2 iu = make_float2(-x.y * rinv, x.x * rinv);      // i x / |x|
  const float f = 1e-8f * rinv * (g.x * iu.x + g.y * iu.y);    // (1e-8 / |x|) Re(conj(g) i u)
  return make_float2(fmaf(f, iu.x, g.x), fmaf(f, iu.y, g.y));
}

// M[r][c] as the forward computes it (its materialised path): m = delta_rc - beta k_r conj(k_c), x = aW m
__device__ __forceinline__ float2 m_entry(float2 aw, float beta, float2 kr, float2 kc, bool diag, int variant,
                                          float2& m, float2& x, bool& frozen) {
  const float2 kk = cmulc(kr, kc);
  m = make_float2(-beta * kk.x, -beta * kk.y);
  if (diag) m.x += 1.0f;
  x = cmul(aw, m);
  return mapped_entry(x, variant, frozen);
}

__device__ __forceinline__ float2 d_entry(float beta, float2 vi, float2 kr, int variant, float2& x, bool& frozen) {
  x = cscale(cmulc(vi, kr), beta);
  return mapped_entry(x, variant, frozen);
}

template <int DK>
__global__ void __launch_bounds__(256) gdn_scan_bins_bwd(const GdnTrainArgs a) {
  const int bin = blockIdx.x * blockDim.x + threadIdx.x;
  if (bin >= a.HWF) return;
  const int head = blockIdx.y, b = blockIdx.z;
  const int C = a.C, HWF = a.HWF, nh = C / DK, variant = a.variant;
  const float2 wh = a.what[size_t(head) * HWF + bin];
  float2 carry[DK][DK];
#pragma unroll
  for (int i = 0; i < DK; ++i)
#pragma unroll
    for (int j = 0; j < DK; ++j) carry[i][j] = make_float2(0.f, 0.f);
  float2 dwh = make_float2(0.f, 0.f);
  for (int t = a.T - 1; t >= 0; --t) {
    const size_t fr = size_t(b) * a.T + t;
    const size_t ch0 = fr * 3 * C + size_t(head) * DK;
    float2 q[DK], kr[DK], v[DK], dov[DK], sp[DK][DK];
#pragma unroll
    for (int j = 0; j < DK; ++j) {
      q[j] = a.spec[(ch0 + j) * HWF + bin];
      kr[j] = a.spec[(ch0 + C + j) * HWF + bin];
      v[j] = a.spec[(ch0 + 2 * C + j) * HWF + bin];
      dov[j] = a.dohat[(fr * C + size_t(head) * DK + j) * HWF + bin];
    }
#pragma unroll
    for (int i = 0; i < DK; ++i)
#pragma unroll
      for (int c = 0; c < DK; ++c) sp[i][c] = a.states[state_at<DK>(a, b, t, head, i, c, bin)];
    const float2 g2 = a.ab[fr * a.ab_frame + size_t(head) * a.ab_head + size_t(bin) * a.ab_bin];
    const float alpha = g2.x, beta = g2.y;
    // key-vector normalisation, as gdn_bin_step
    float kk = 0.0f;
#pragma unroll
    for (int j = 0; j < DK; ++j) kk = fmaf(kr[j].x, kr[j].x, fmaf(kr[j].y, kr[j].y, kk));
    const float kn = 1.0f / sqrtf(kk + 1e-6f);
    float2 k[DK];
#pragma unroll
    for (int j = 0; j < DK; ++j) k[j] = cscale(kr[j], kn);
    const float2 aw = cscale(wh, alpha);

    // s_t (recomputed from s_{t-1}) for dq; g = carry + do conj(q)
    float2 dq[DK], g[DK][DK];
#pragma unroll
    for (int r = 0; r < DK; ++r) dq[r] = make_float2(0.f, 0.f);
#pragma unroll
    for (int i = 0; i < DK; ++i)
#pragma unroll
      for (int r = 0; r < DK; ++r) {
        bool fl;
        float2 xd;
        float2 st = d_entry(beta, v[i], k[r], variant, xd, fl);
#pragma unroll
        for (int c = 0; c < DK; ++c) {
          float2 m, xm;
          bool fm;
          const float2 M = m_entry(aw, beta, k[r], k[c], r == c, variant, m, xm, fm);
          st = cadd(st, cmul(M, sp[i][c]));
        }
        dq[r] = cadd(dq[r], cmulc(dov[i], st));
        g[i][r] = cadd(carry[i][r], cmulc(dov[i], q[r]));
      }

    // through M: carry' = M^H g, and the inputs of the entries the floor left alone
    float2 dk[DK], dv[DK];
#pragma unroll
    for (int j = 0; j < DK; ++j) dk[j] = dv[j] = make_float2(0.f, 0.f);
    float2 daw = make_float2(0.f, 0.f);
    float dbeta = 0.0f;
#pragma unroll
    for (int i = 0; i < DK; ++i)
#pragma unroll
      for (int c = 0; c < DK; ++c) carry[i][c] = make_float2(0.f, 0.f);
#pragma unroll
    for (int r = 0; r < DK; ++r)
#pragma unroll
      for (int c = 0; c < DK; ++c) {
        float2 m, xm;
        bool fm;
        const float2 M = m_entry(aw, beta, k[r], k[c], r == c, variant, m, xm, fm);
        float2 dM = make_float2(0.f, 0.f);
#pragma unroll
        for (int i = 0; i < DK; ++i) {
          carry[i][c] = cadd(carry[i][c], cmulc(g[i][r], M));   // conj(M) g
          dM = cadd(dM, cmulc(g[i][r], sp[i][c]));             // g conj(s_{t-1})
        }
        if (!fm) {
          dM = entry_adjoint(dM, xm, variant);                 // dL/d(aW m)
          daw = cadd(daw, cmulc(dM, m));                       // dM conj(m)
          const float2 dm = cmulc(dM, aw);                     // dM conj(aW)
          // m = delta - beta k_r conj(k_c)
          const float2 kk_rc = cmulc(k[r], k[c]);
          dbeta -= dm.x * kk_rc.x + dm.y * kk_rc.y;            // Re(conj(dm) k_r conj(k_c))
          dk[r] = cadd(dk[r], cscale(cmul(dm, k[c]), -beta));
          dk[c] = cadd(dk[c], cscale(cmul(make_float2(dm.x, -dm.y), k[r]), -beta));
        }
      }
    // through D[i][r] = beta v_i conj(k_r)
#pragma unroll
    for (int i = 0; i < DK; ++i)
#pragma unroll
      for (int r = 0; r < DK; ++r) {
        bool fl;
        float2 xd;
        d_entry(beta, v[i], k[r], variant, xd, fl);
        if (fl) continue;
        const float2 dD = entry_adjoint(g[i][r], xd, variant);
        const float2 vk = cmulc(v[i], k[r]);
        dbeta += dD.x * vk.x + dD.y * vk.y;                    // Re(conj(dD) v_i conj(k_r))
        dv[i] = cadd(dv[i], cscale(cmul(dD, k[r]), beta));
        dk[r] = cadd(dk[r], cscale(cmul(make_float2(dD.x, -dD.y), v[i]), beta));
      }
    // aW = alpha W_hat
    const float dalpha = daw.x * wh.x + daw.y * wh.y;          // Re(daW conj(W_hat))
    dwh = cadd(dwh, cscale(daw, alpha));
    // key normalisation
    float red = 0.0f;
#pragma unroll
    for (int j = 0; j < DK; ++j) red += dk[j].x * kr[j].x + dk[j].y * kr[j].y;   // Re(sum dk' conj(k))
    const float kn3 = kn * kn * kn;
#pragma unroll
    for (int j = 0; j < DK; ++j) {
      const float2 dkr = make_float2(kn * dk[j].x - kn3 * kr[j].x * red, kn * dk[j].y - kn3 * kr[j].y * red);
      a.dspec[(ch0 + j) * HWF + bin] = dq[j];
      a.dspec[(ch0 + C + j) * HWF + bin] = dkr;
      a.dspec[(ch0 + 2 * C + j) * HWF + bin] = dv[j];
    }
    a.dab[(fr * nh + head) * HWF + bin] = make_float2(dalpha, dbeta);
  }
  a.dwhat[(size_t(b) * nh + head) * HWF + bin] = dwh;
}

hipError_t launch_gdn_scan_bins_train(const float2* spec, const float2* ab, long long ab_frame, int ab_head,
                                      int ab_bin, const float2* what, int B, int T, int C, int H, int W, int dk,
                                      int variant, float2* ohat, float2* states, const float2* dohat, float2* dspec,
                                      float2* dab, float2* dwhat, bool backward, hipStream_t s) {
  GdnTrainArgs a{spec, ab, ab_frame, ab_head, ab_bin, what, ohat, states, dohat, dspec, dab, dwhat, T, C,
                 H * (W / 2 + 1), variant};
  const dim3 grid(unsigned((a.HWF + 255) / 256), unsigned(C / dk), unsigned(B));
#define CSSM_GDN_TRAIN(D)                                                                   \
  if (backward) hipLaunchKernelGGL(gdn_scan_bins_bwd<D>, grid, dim3(256), 0, s, a);         \
  else hipLaunchKernelGGL(gdn_scan_bins_save<D>, grid, dim3(256), 0, s, a);
  switch (dk) {
    case 1: CSSM_GDN_TRAIN(1) break;
    case 2: CSSM_GDN_TRAIN(2) break;
    case 3: CSSM_GDN_TRAIN(3) break;
    case 4: CSSM_GDN_TRAIN(4) break;
    default: return hipErrorInvalidValue;
  }
#undef CSSM_GDN_TRAIN
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Weight gradient of the depthwise KS x KS SAME convolution of channels-last
// frames (qkv_dw, cssm.py:4744-4750): dW[a][b][c] = sum over frames and pixels
// of x[h + a - lo][w + b - lo][c] dy[h][w][c] (zero outside the frame).  A thread
// owns 4 channels and strips of 8 pixels of a row: it loads the strip's dy and,
// per tap row, the 8 + KS - 1 inputs it needs once, and keeps all KS^2 taps'
// sums in registers.  Block partials (KS^2, C) are reduced in a fixed order
// (lane shuffles, then across waves through LDS); the caller sums the blocks.
namespace {
template <int KS>
__global__ void __launch_bounds__(256) dwconv_wgrad_cl(const float* __restrict__ x, const float* __restrict__ dy,
                                                        int F, int H, int W, int C, float* __restrict__ partial) {
  constexpr int LO = (KS - 1) / 2, RW = 8, NCOL = RW + KS - 1;
  const int CQ = C / 4, SPB = 256 / CQ;                     // channel quads; strips per block pass
  const int tid = int(threadIdx.x), cq = tid % CQ, sl = tid / CQ;
  const int c0 = cq * 4, WS = W / RW;
  const long long strips = (long long)F * H * WS;
  float4 acc[KS][KS];
#pragma unroll
  for (int a = 0; a < KS; ++a)
#pragma unroll
    for (int b = 0; b < KS; ++b) acc[a][b] = make_float4(0.f, 0.f, 0.f, 0.f);
  for (long long s = (long long)blockIdx.x * SPB + sl; s < strips; s += (long long)gridDim.x * SPB) {
    const int ws = int(s % WS);
    const long long fh = s / WS;
    const int h = int(fh % H);
    const long long f = fh / H;
    const int w0 = ws * RW;
    const float* xf = x + f * H * W * C;
    float4 g[RW];
#pragma unroll
    for (int q = 0; q < RW; ++q)
      g[q] = *reinterpret_cast<const float4*>(dy + ((f * H + h) * W + w0 + q) * C + c0);
#pragma unroll
    for (int a = 0; a < KS; ++a) {
      const int hh = h + a - LO;
      if (hh < 0 || hh >= H) continue;
      float4 xin[NCOL];
#pragma unroll
      for (int ic = 0; ic < NCOL; ++ic) {
        const int ww = w0 - LO + ic;
        xin[ic] = (ww >= 0 && ww < W) ? *reinterpret_cast<const float4*>(xf + (size_t(hh) * W + ww) * C + c0)
                                      : make_float4(0.f, 0.f, 0.f, 0.f);
      }
#pragma unroll
      for (int b = 0; b < KS; ++b)
#pragma unroll
        for (int q = 0; q < RW; ++q) {
          acc[a][b].x = fmaf(xin[q + b].x, g[q].x, acc[a][b].x);
          acc[a][b].y = fmaf(xin[q + b].y, g[q].y, acc[a][b].y);
          acc[a][b].z = fmaf(xin[q + b].z, g[q].z, acc[a][b].z);
          acc[a][b].w = fmaf(xin[q + b].w, g[q].w, acc[a][b].w);
        }
    }
  }
  // threads of one channel quad: lanes l, l + CQ, ... of a wave, then the waves
  __shared__ float4 red[4][64];
  const int lane = tid & 63, wave = tid >> 6;
#pragma unroll
  for (int a = 0; a < KS; ++a)
#pragma unroll
    for (int b = 0; b < KS; ++b) {
      float4 v = acc[a][b];
      for (int d = 32; d >= CQ; d >>= 1) {
        v.x += __shfl_xor(v.x, d, 64);
        v.y += __shfl_xor(v.y, d, 64);
        v.z += __shfl_xor(v.z, d, 64);
        v.w += __shfl_xor(v.w, d, 64);
      }
      if (lane < CQ) red[wave][lane] = v;      // CQ <= 64 here: every quad in every wave
      __syncthreads();
      if (tid < CQ) {
        float4 t = red[0][tid];
        for (int ww = 1; ww < 4; ++ww) {
          t.x += red[ww][tid].x;
          t.y += red[ww][tid].y;
          t.z += red[ww][tid].z;
          t.w += red[ww][tid].w;
        }
        *reinterpret_cast<float4*>(partial + (size_t(blockIdx.x) * KS * KS + a * KS + b) * C + tid * 4) = t;
      }
      __syncthreads();
    }
}
}  // namespace

bool dwconv_wgrad_supported(int W, int C, int ks) {
  const int cq = C / 4;
  return (ks == 3 || ks == 5 || ks == 7) && C % 4 == 0 && cq >= 1 && cq <= 64 && 64 % cq == 0 && W % 8 == 0;
}

hipError_t launch_dwconv_wgrad(const float* x, const float* dy, int F, int H, int W, int C, int ks, float* partial,
                               int blocks, hipStream_t s) {
  if (!dwconv_wgrad_supported(W, C, ks) || blocks <= 0) return hipErrorInvalidValue;
  switch (ks) {
    case 3: hipLaunchKernelGGL(dwconv_wgrad_cl<3>, dim3(unsigned(blocks)), dim3(256), 0, s, x, dy, F, H, W, C, partial); break;
    case 5: hipLaunchKernelGGL(dwconv_wgrad_cl<5>, dim3(unsigned(blocks)), dim3(256), 0, s, x, dy, F, H, W, C, partial); break;
    case 7: hipLaunchKernelGGL(dwconv_wgrad_cl<7>, dim3(unsigned(blocks)), dim3(256), 0, s, x, dy, F, H, W, C, partial); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace cssm
