// Direct DFTs of small planes (any size up to 15) with compile-time twiddles,
// shared by the fused small-plane scan (gated_scan.hip) and the batched
// small-plane transforms (gdn.hip).
#pragma once
#include <hip/hip_runtime.h>

#include "fft_reg.h"

namespace cssm {

template <int H, int W>
struct SmallGeom {
  // 128-thread groups from 8 x 8 up: more, smaller groups per CU overlap one
  // group's loads and stores with another's DFTs (one step per group at T = 1)
  static constexpr int WF = W / 2 + 1, HW = H * W, NT = WF >= 5 ? 128 : 256;
  static constexpr int NP = NT / WF;               // planes per group: one column per thread
  static constexpr int NCJ = NP * WF, NRJ = NP * H; // column / row jobs per group
  // spectra in LDS at pl PS + h RSP + v (complex units): an odd row stride
  // spreads the row passes' lanes (consecutive rows) over the banks, and a
  // plane stride of WF mod 32 puts the column pass's planes (WF lanes each) on
  // disjoint bank windows
  static constexpr int RSP = WF | 1;
  static constexpr int PS = H * RSP + ((WF - H * RSP) % 32 + 32) % 32;
  static_assert(NP * HW * 4 + NP * PS * 8 + NP * 12 <= 64 * 1024, "small-plane group exceeds LDS");
};

// cos / sin (2 pi J / N) as compile-time constants; mac_c / mac_s add
// v cos or v sin to acc, skipping zero factors and folding +-1
template <int N, int J, bool SIN>
constexpr double trig() {
  constexpr double x = 2.0 * kPi * double(((J % N) + N) % N) / double(N);
  return SIN ? cx_sin(x) : cx_cos(x);
}
template <int N, int J, bool SIN>
__device__ __forceinline__ void mac_t(float& acc, float v) {
  constexpr double d = trig<N, J, SIN>();
  if constexpr (d > -1e-12 && d < 1e-12) {
  } else if constexpr (d > 1.0 - 1e-12) {
    acc += v;
  } else if constexpr (d < -1.0 + 1e-12) {
    acc -= v;
  } else {
    acc = fmaf(v, float(d), acc);
  }
}
template <int N, int J, bool SIN>
__device__ __forceinline__ void mac_t(float2& acc, float2 v) {
  mac_t<N, J, SIN>(acc.x, v.x);
  mac_t<N, J, SIN>(acc.y, v.y);
}

// Complex N-point DFT (forward e^{-i}, INV: e^{+i}; any N) by the symmetry of
// the twiddles: with a_n = x_n + x_{N-n}, b_n = x_n - x_{N-n} (0 < n < N/2),
//   X[k], X[N-k] = A_k -+ i B_k (forward; +- for INV),
//   A_k = x_0 [+ (-1)^k x_{N/2}] + sum_n a_n cos(2 pi n k / N),  B_k = sum_n b_n sin(2 pi n k / N)
// which takes about a quarter of the direct form's multiply-adds.
template <int N, bool INV>
__device__ __forceinline__ void dft_sym(const float2 (&x)[N], float2 (&X)[N]) {
  constexpr int M = (N - 1) / 2;
  constexpr bool EVEN = (N % 2) == 0;
  float2 a[M + 1], b[M + 1];
  static_for<1, M + 1>([&](auto Nn) {
    constexpr int n = decltype(Nn)::value;
    a[n] = cadd(x[n], x[N - n]);
    b[n] = csub(x[n], x[N - n]);
  });
  static_for<0, M + 1>([&](auto K) {
    constexpr int k = decltype(K)::value;
    float2 A = x[0], B = make_float2(0.f, 0.f);
    if constexpr (EVEN) {
      if constexpr (k % 2 == 0) A = cadd(A, x[N / 2]);
      else A = csub(A, x[N / 2]);
    }
    static_for<1, M + 1>([&](auto Nn) {
      constexpr int n = decltype(Nn)::value;
      mac_t<N, n * k, false>(A, a[n]);
      if constexpr (k > 0) mac_t<N, n * k, true>(B, b[n]);
    });
    if constexpr (k == 0) {
      X[0] = A;
    } else {
      // -i B (forward) or +i B (inverse) for X[k]; the opposite for X[N - k]
      const float2 iB = INV ? make_float2(-B.y, B.x) : make_float2(B.y, -B.x);
      X[k] = cadd(A, iB);
      X[N - k] = csub(A, iB);
    }
  });
  if constexpr (EVEN) {
    float2 A = x[0];
    if constexpr ((N / 2) % 2 == 0) A = cadd(A, x[N / 2]);
    else A = csub(A, x[N / 2]);
    static_for<1, M + 1>([&](auto Nn) {
      constexpr int n = decltype(Nn)::value;
      if constexpr (n % 2 == 0) A = cadd(A, a[n]);
      else A = csub(A, a[n]);
    });
    X[N / 2] = A;
  }
}

// Real-input DFT of one row of W samples: R[v] = sum_w x[w] e^{-2 pi i v w / W}, v < W/2 + 1.
template <int W>
__device__ __forceinline__ void small_row_r2c(const float* xr, float2* rr) {
  constexpr int WF = W / 2 + 1;
  float x[W];
#pragma unroll
  for (int w = 0; w < W; ++w) x[w] = xr[w];
  // real input: R[v] = x_0 [+ (-1)^v x_{W/2}] + sum_w (x_w + x_{W-w}) cos - i (x_w - x_{W-w}) sin
  constexpr int MW = (W - 1) / 2;
  float ap[MW + 1], bm[MW + 1];
  static_for<1, MW + 1>([&](auto Wi) {
    constexpr int w = decltype(Wi)::value;
    ap[w] = x[w] + x[W - w];
    bm[w] = x[w] - x[W - w];
  });
  static_for<0, WF>([&](auto V) {
    constexpr int v = decltype(V)::value;
    float re = x[0], im = 0.f;
    if constexpr (W % 2 == 0) re += (v % 2 == 0) ? x[W / 2] : -x[W / 2];
    static_for<1, MW + 1>([&](auto Wi) {
      constexpr int w = decltype(Wi)::value;
      mac_t<W, v * w, false>(re, ap[w]);
      mac_t<W, v * w, true>(im, bm[w]);
    });
    rr[v] = make_float2(re, -im);
  });
}

// C2R of one row (numpy irfft's rule, unnormalised): y[w] = Re Z[0] + 2 sum_{0 < v < W/2}
// Re(Z[v] e^{2 pi i v w / W}) + [W even] (-1)^w Re Z[W/2].
template <int W>
__device__ __forceinline__ void small_row_c2r(const float2* zr, float* yr) {
  constexpr int WF = W / 2 + 1;
  float2 z[WF];
#pragma unroll
  for (int v = 0; v < WF; ++v) z[v] = zr[v];
  // Re(Z_v e^{+2 pi i v w / W}) = Z.x cos - Z.y sin, each bin counted twice but
  // the Nyquist bin of an even W: with P_w = sum Z.x cos and Q_w = sum Z.y sin
  // (weights folded in), y[w] = P_w - Q_w and y[W - w] = P_w + Q_w
  float zx[WF], zy[WF];
  zx[0] = z[0].x;
  zy[0] = 0.f;
#pragma unroll
  for (int v = 1; v < WF; ++v) {
    const float c = (W % 2 == 0 && v == W / 2) ? 1.0f : 2.0f;
    zx[v] = c * z[v].x;
    zy[v] = c * z[v].y;
  }
  static_for<0, W / 2 + 1>([&](auto Wi) {
    constexpr int w = decltype(Wi)::value;
    float P = zx[0], Q = 0.f;
    static_for<1, WF>([&](auto V) {
      constexpr int v = decltype(V)::value;
      mac_t<W, v * w, false>(P, zx[v]);
      mac_t<W, v * w, true>(Q, zy[v]);
    });
    yr[w] = P - Q;
    if constexpr (w > 0 && W - w != w) yr[W - w] = P + Q;
  });
}

}  // namespace cssm
