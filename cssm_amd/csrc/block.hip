// Caller wiring of CSSMSHViTBlock around the cell: the token-mixer half of
// the block (cssm_shvit.py:86-229): norm1 -> pos_conv -> cell -> frame
// selection -> output activation -> residual.  The MLP half (:231-266) is not
// part of this build.
//
// Tensors are channels-last (B, T, H, W, C); an image input is (B, 1, H, W, C)
// and is repeated to the cell's T frames on the way out of the pos_conv pass.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fft_plane.h"
#include "launch.h"

namespace cssm {
namespace {

__device__ __forceinline__ float ldx(const float* p, size_t i) { return p[i]; }
__device__ __forceinline__ float ldx(const uint16_t* p, size_t i) { return bf16_to_f32(p[i]); }
__device__ __forceinline__ void stx(float* p, size_t i, float v) { p[i] = v; }
__device__ __forceinline__ void stx(uint16_t* p, size_t i, float v) { p[i] = uint16_t(f32_to_bf16(v)); }

// norm1 group of element (b, t, p, c) (p = h W + w) and its element count
//   mode 0 global_layer   (cssm_shvit.py:106-108): b        over T H W C
//   mode 1 temporal_layer (:109-111):              (b, p)   over T C
//   mode 2 layer          (:112-114):              (b, t, p) over C
__device__ __forceinline__ long long norm_group(int mode, int b, int t, int p, int T, int HW) {
  if (mode == 0) return b;
  if (mode == 1) return (long long)b * HW + p;
  return ((long long)b * T + t) * HW + p;
}

}  // namespace

// stats[g] = (mean, rsqrt(var + eps)) with var = E[x^2] - E[x]^2 (Flax's fast
// variance), sums in double in a fixed order: L lanes per group (256 for the
// global mode, 64 otherwise), 256 / L groups per workgroup.
template <class TI>
__global__ void __launch_bounds__(256)
block_norm_stats_kernel(const TI* __restrict__ x, int T, int HW, int C, int mode, long long groups, float eps,
                        float2* __restrict__ stats) {
  __shared__ double s1[256], s2[256];
  const int L = mode == 0 ? 256 : 64, GPB = 256 / L;
  const int tid = threadIdx.x, gl = tid / L, lane = tid % L;
  const long long g = (long long)blockIdx.x * GPB + gl;
  double a = 0.0, q = 0.0;
  long long n = 0;
  if (g < groups) {
    if (mode == 0) {
      n = (long long)T * HW * C;
      const TI* xg = x + g * n;
      for (long long e = lane; e < n; e += L) {
        const double v = ldx(xg, size_t(e));
        a += v;
        q += v * v;
      }
    } else if (mode == 1) {
      n = (long long)T * C;
      const long long b = g / HW, p = g % HW;
      for (long long e = lane; e < n; e += L) {
        const long long t = e / C, c = e % C;
        const double v = ldx(x, size_t(((b * T + t) * HW + p) * C + c));
        a += v;
        q += v * v;
      }
    } else {
      n = C;
      const TI* xg = x + g * C;
      for (int e = lane; e < C; e += L) {
        const double v = ldx(xg, size_t(e));
        a += v;
        q += v * v;
      }
    }
  }
  s1[tid] = a;
  s2[tid] = q;
  __syncthreads();
  if (lane == 0 && g < groups) {
    double sa = 0.0, sq = 0.0;
    for (int i = 0; i < L; ++i) {
      sa += s1[gl * L + i];
      sq += s2[gl * L + i];
    }
    const double mean = sa / double(n);
    const double var = fmax(sq / double(n) - mean * mean, 0.0);
    stats[g] = make_float2(float(mean), float(1.0 / sqrt(var + double(eps))));
  }
}

// out[b, t] = xn + [pos_conv(xn)] for t < T_out, xn = (x[b, t_in] - mean) rstd
// scale + bias with t_in = t (T_in = T_out) or 0 (an image, T_in = 1);
// pos_conv = depthwise 3x3 'SAME' cross-correlation with bias (cssm_shvit.py:
// 122-145), zero padding of xn.  One thread per (pixel, 4 channels) when
// C % 4 == 0, else per (pixel, channel).
template <class TI>
__global__ void __launch_bounds__(256)
block_norm_posconv_kernel(const TI* __restrict__ x, int T_in, int T_out, int H, int W, int C, int mode,
                          const float2* __restrict__ stats, const float* __restrict__ scale,
                          const float* __restrict__ bias, const float* __restrict__ pk, const float* __restrict__ pb,
                          TI* __restrict__ out, long long total) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int cv = (C % 4 == 0) ? 4 : 1, CG = C / cv, HW = H * W;
  const int c0 = int(i % CG) * cv;
  const long long pix = i / CG;                  // (b, t, p) of the output
  const int p = int(pix % HW);
  const long long bt = pix / HW;
  const int t = int(bt % T_out), b = int(bt / T_out);
  const int ti = T_in == T_out ? t : 0;
  const int h = p / W, w = p % W;
  const TI* xf = x + ((long long)b * T_in + ti) * HW * C;
  float sc[4], bs[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    sc[e] = e < cv ? scale[c0 + e] : 0.f;
    bs[e] = e < cv ? bias[c0 + e] : 0.f;
  }
  // normalised input at (hh, ww), channel c0 + e
  auto xn = [&](int hh, int ww, int e) -> float {
    const float2 st = stats[norm_group(mode, b, ti, hh * W + ww, T_in, HW)];
    return fmaf((ldx(xf, size_t(hh * W + ww) * C + c0 + e) - st.x) * st.y, sc[e], bs[e]);
  };
  float acc[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) acc[e] = e < cv ? xn(h, w, e) : 0.f;
  if (pk != nullptr) {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (e < cv) acc[e] += pb[c0 + e];
    for (int a = 0; a < 3; ++a) {
      const int hh = h + a - 1;
      if (hh < 0 || hh >= H) continue;
      for (int b2 = 0; b2 < 3; ++b2) {
        const int ww = w + b2 - 1;
        if (ww < 0 || ww >= W) continue;
        const float* kt = pk + (a * 3 + b2) * C + c0;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (e < cv) acc[e] = fmaf(kt[e], xn(hh, ww, e), acc[e]);
      }
    }
  }
  const size_t o = size_t(pix) * C + c0;
#pragma unroll
  for (int e = 0; e < 4; ++e)
    if (e < cv) stx(out, o + e, acc[e]);
}

// out[b, t] = res[b, tr] + act(y[b, ty]) over (H, W, C): T_out = 1 takes the
// last frame of each (cssm_shvit.py:211, :224), T_out > 1 frame t of both
// (keep_time, :213, :222).  act 0 none, 1 gelu (tanh form, jax.nn.gelu's
// default), 2 silu (:215-218).
template <class TI>
__global__ void __launch_bounds__(256)
block_residual_kernel(const TI* __restrict__ res, int T_res, const TI* __restrict__ y, int T_y, int T_out, int HWC,
                      int act, TI* __restrict__ out, long long total) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const long long e = i % HWC, bt = i / HWC;
  const int t = int(bt % T_out), b = int(bt / T_out);
  const int tr = T_out == 1 ? T_res - 1 : t, ty = T_out == 1 ? T_y - 1 : t;
  float v = ldx(y, size_t(((long long)b * T_y + ty) * HWC + e));
  if (act == 1) {
    const float u = 0.7978845608028654f * fmaf(0.044715f * v, v * v, v);
    v = 0.5f * v * (1.0f + tanhf(u));
  } else if (act == 2) {
    v = v / (1.0f + expf(-v));
  }
  stx(out, size_t(i), ldx(res, size_t(((long long)b * T_res + tr) * HWC + e)) + v);
}

static unsigned blocks_for(long long n, int per) { return unsigned((n + per - 1) / per); }

hipError_t launch_block_norm_stats(const void* x, int dtype, int B, int T, int H, int W, int C, int mode, float eps,
                                   float* stats, hipStream_t s) {
  const int HW = H * W;
  const long long groups = mode == 0 ? B : (mode == 1 ? (long long)B * HW : (long long)B * T * HW);
  const int gpb = mode == 0 ? 1 : 4;
  const unsigned grid = blocks_for(groups, gpb);
  if (dtype == 0)
    hipLaunchKernelGGL(block_norm_stats_kernel<float>, dim3(grid), dim3(256), 0, s, static_cast<const float*>(x), T,
                       HW, C, mode, groups, eps, reinterpret_cast<float2*>(stats));
  else
    hipLaunchKernelGGL(block_norm_stats_kernel<uint16_t>, dim3(grid), dim3(256), 0, s,
                       static_cast<const uint16_t*>(x), T, HW, C, mode, groups, eps, reinterpret_cast<float2*>(stats));
  return hipGetLastError();
}

hipError_t launch_block_norm_posconv(const void* x, int dtype, int B, int T_in, int T_out, int H, int W, int C,
                                     int mode, const float* stats, const float* scale, const float* bias,
                                     const float* pk, const float* pb, void* out, hipStream_t s) {
  const int cv = (C % 4 == 0) ? 4 : 1;
  const long long total = (long long)B * T_out * H * W * (C / cv);
  if (total == 0) return hipSuccess;
  const auto* st = reinterpret_cast<const float2*>(stats);
  if (dtype == 0)
    hipLaunchKernelGGL(block_norm_posconv_kernel<float>, dim3(blocks_for(total, 256)), dim3(256), 0, s,
                       static_cast<const float*>(x), T_in, T_out, H, W, C, mode, st, scale, bias, pk, pb,
                       static_cast<float*>(out), total);
  else
    hipLaunchKernelGGL(block_norm_posconv_kernel<uint16_t>, dim3(blocks_for(total, 256)), dim3(256), 0, s,
                       static_cast<const uint16_t*>(x), T_in, T_out, H, W, C, mode, st, scale, bias, pk, pb,
                       static_cast<uint16_t*>(out), total);
  return hipGetLastError();
}

hipError_t launch_block_residual(const void* res, int T_res, const void* y, int T_y, int dtype, int B, int T_out,
                                 int H, int W, int C, int act, void* out, hipStream_t s) {
  const int HWC = H * W * C;
  const long long total = (long long)B * T_out * HWC;
  if (total == 0) return hipSuccess;
  if (dtype == 0)
    hipLaunchKernelGGL(block_residual_kernel<float>, dim3(blocks_for(total, 256)), dim3(256), 0, s,
                       static_cast<const float*>(res), T_res, static_cast<const float*>(y), T_y, T_out, HWC, act,
                       static_cast<float*>(out), total);
  else
    hipLaunchKernelGGL(block_residual_kernel<uint16_t>, dim3(blocks_for(total, 256)), dim3(256), 0, s,
                       static_cast<const uint16_t*>(res), T_res, static_cast<const uint16_t*>(y), T_y, T_out, HWC,
                       act, static_cast<uint16_t*>(out), total);
  return hipGetLastError();
}

}  // namespace cssm
