// Factored short convolution of GatedCSSM on plane-major x_main (gfx950):
//   s_t   = DWConv_{ks x ks, SAME}(x_t) + b_s          (cssm.py:487-492)
//   o_t   = sum_{j < kt} w_t[j] s_{t - kt + 1 + j} + b_t (zeros for t < 0; cssm.py:494-500)
//   u_t   = SiLU(o_t)                                   (cssm.py:502)
//   ctx_t = mean_{h,w} u_t                              (cssm.py:536)
// Either convolution may be absent (ks = 0 / kt = 0).  One block per (b, c)
// plane sequence; threads stride over pixels, the T loop is outermost so the
// spatial mean of every step reduces inside the block.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "launch.h"

namespace cssm {

__device__ __forceinline__ float sc_ld(const float* p, size_t i) { return p[i]; }
__device__ __forceinline__ float sc_ld(const uint16_t* p, size_t i) { return __uint_as_float(uint32_t(p[i]) << 16); }
__device__ __forceinline__ void sc_st(float* p, size_t i, float v) { p[i] = v; }
__device__ __forceinline__ void sc_st(uint16_t* p, size_t i, float v) {
  uint32_t x = __float_as_uint(v);
  if ((x & 0x7f800000u) == 0x7f800000u) {
    p[i] = uint16_t((x >> 16) | ((x & 0x007fffffu) ? 0x40u : 0u));
  } else {
    x += 0x7fffu + ((x >> 16) & 1u);
    p[i] = uint16_t(x >> 16);
  }
}

template <class TI, class TO>
__global__ void __launch_bounds__(256)
short_conv_kernel(const TI* __restrict__ x, int T, int C, int H, int W, int ks, const float* __restrict__ ws,
                  const float* __restrict__ bs, int kt, const float* __restrict__ wt, const float* __restrict__ bt,
                  TO* __restrict__ u, float* __restrict__ ctx) {
  __shared__ float red[4];
  const int b = blockIdx.x / C, c = blockIdx.x % C;
  const int HW = H * W;
  const int lo = (ks - 1) / 2;
  const float bsc = (ks > 0) ? bs[c] : 0.0f;
  const float btc = (kt > 0) ? bt[c] : 0.0f;
  auto plane = [&](int t) -> size_t { return ((size_t(b) * T + t) * C + c) * size_t(HW); };
  // spatial stage at step t, pixel (h, w); HWIO kernel (ks, ks, 1, C)
  auto spatial = [&](int t, int h, int w) -> float {
    const size_t base = plane(t);
    if (ks == 0) return sc_ld(x, base + size_t(h) * W + w);
    float acc = bsc;
    for (int i = 0; i < ks; ++i) {
      const int hh = h + i - lo;
      if (hh < 0 || hh >= H) continue;
      for (int j = 0; j < ks; ++j) {
        const int ww = w + j - lo;
        if (ww < 0 || ww >= W) continue;
        acc = fmaf(sc_ld(x, base + size_t(hh) * W + ww), ws[(i * ks + j) * C + c], acc);
      }
    }
    return acc;
  };
  for (int t = 0; t < T; ++t) {
    float csum = 0.0f;
    for (int p = threadIdx.x; p < HW; p += blockDim.x) {
      const int h = p / W, w = p % W;
      float o;
      if (kt > 0) {
        o = btc;
        for (int j = 0; j < kt; ++j) {
          const int ts = t - kt + 1 + j;
          if (ts >= 0) o = fmaf(wt[j * C + c], spatial(ts, h, w), o);
        }
      } else {
        o = spatial(t, h, w);
      }
      const float v = o / (1.0f + expf(-o));
      sc_st(u, plane(t) + p, v);
      csum += v;
    }
    for (int off = 32; off > 0; off >>= 1) csum += __shfl_down(csum, off, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = csum;
    __syncthreads();
    if (threadIdx.x == 0 && ctx != nullptr) {
      float s = 0.0f;
      for (int i = 0; i < int(blockDim.x >> 6); ++i) s += red[i];
      ctx[(size_t(b) * T + t) * C + c] = s / float(HW);
    }
    __syncthreads();
  }
}

hipError_t launch_short_conv(const void* x, int in_dtype, int B, int T, int C, int H, int W, int ks, const float* ws,
                             const float* bs, int kt, const float* wt, const float* bt, void* u, int out_dtype,
                             float* ctx, hipStream_t s) {
  const dim3 grid(unsigned(B * C)), block(256);
  if (in_dtype == 0 && out_dtype == 0)
    hipLaunchKernelGGL((short_conv_kernel<float, float>), grid, block, 0, s, static_cast<const float*>(x), T, C, H, W,
                       ks, ws, bs, kt, wt, bt, static_cast<float*>(u), ctx);
  else if (in_dtype == 0)
    hipLaunchKernelGGL((short_conv_kernel<float, uint16_t>), grid, block, 0, s, static_cast<const float*>(x), T, C, H,
                       W, ks, ws, bs, kt, wt, bt, static_cast<uint16_t*>(u), ctx);
  else if (out_dtype == 0)
    hipLaunchKernelGGL((short_conv_kernel<uint16_t, float>), grid, block, 0, s, static_cast<const uint16_t*>(x), T, C,
                       H, W, ks, ws, bs, kt, wt, bt, static_cast<float*>(u), ctx);
  else
    hipLaunchKernelGGL((short_conv_kernel<uint16_t, uint16_t>), grid, block, 0, s, static_cast<const uint16_t*>(x), T,
                       C, H, W, ks, ws, bs, kt, wt, bt, static_cast<uint16_t*>(u), ctx);
  return hipGetLastError();
}

}  // namespace cssm
