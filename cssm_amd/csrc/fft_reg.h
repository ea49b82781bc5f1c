// In-register complex DFT building blocks for gfx950 (CDNA4).
//
// Everything here is compile-time shaped: sizes, indices and twiddle factors
// are template parameters, so an N-point DFT unrolls into straight-line VALU
// code with the twiddles as immediate constants and the trivial twiddles
// (1, -1, +-i) folded into swaps and sign flips.
//
// Conventions (identical to numpy / XLA `fft`):
//   forward  X[k] = sum_n x[n] exp(-2 pi i n k / N)   (INV = false)
//   inverse  x[n] = sum_k X[k] exp(+2 pi i n k / N)   (INV = true, unnormalised)
//
// The functions are __host__ __device__ so the host-side unit test
// (tests/test_fft_reg_host.py) checks them against a brute-force DFT without a GPU.
#pragma once

#include <hip/hip_runtime.h>
#include <type_traits>

#define CSSM_HD __host__ __device__ __forceinline__

namespace cssm {

CSSM_HD float2 cadd(float2 a, float2 b) { return make_float2(a.x + b.x, a.y + b.y); }
CSSM_HD float2 csub(float2 a, float2 b) { return make_float2(a.x - b.x, a.y - b.y); }
CSSM_HD float2 cmul(float2 a, float2 b) {
  return make_float2(a.x * b.x - a.y * b.y, a.x * b.y + a.y * b.x);
}
// a * conj(b)
CSSM_HD float2 cmulc(float2 a, float2 b) {
  return make_float2(a.x * b.x + a.y * b.y, a.y * b.x - a.x * b.y);
}
CSSM_HD float2 cconj(float2 a) { return make_float2(a.x, -a.y); }
CSSM_HD float2 cscale(float2 a, float s) { return make_float2(a.x * s, a.y * s); }
// multiply by -i (forward quarter turn) or +i (inverse quarter turn)
template <bool INV>
CSSM_HD float2 mul_quarter(float2 a) {
  if constexpr (INV) return make_float2(-a.y, a.x);
  else return make_float2(a.y, -a.x);
}

// compile-time loop: f(std::integral_constant<int, I>) for I in [B, E)
template <int B, int E, class F>
CSSM_HD void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

// constexpr sine / cosine (Taylor series after range reduction; |err| < 1e-16
// for the angles used here) so twiddles are exact immediates.
constexpr double kPi = 3.14159265358979323846264338327950288;
constexpr double cx_sin_reduced(double x) {
  double term = x, sum = x;
  for (int n = 1; n < 40; ++n) {
    term *= -x * x / double((2 * n) * (2 * n + 1));
    sum += term;
  }
  return sum;
}
constexpr double cx_sin(double x) {
  while (x > kPi) x -= 2.0 * kPi;
  while (x < -kPi) x += 2.0 * kPi;
  return cx_sin_reduced(x);
}
constexpr double cx_cos(double x) { return cx_sin(x + 0.5 * kPi); }

// a * w_N^J with w_N = exp(-2 pi i / N) (forward) or its conjugate (inverse)
template <int N, int J, bool INV>
CSSM_HD float2 twiddle(float2 a) {
  constexpr int j = ((J % N) + N) % N;
  if constexpr (j == 0) {
    return a;
  } else if constexpr (2 * j == N) {
    return make_float2(-a.x, -a.y);
  } else if constexpr (4 * j == N) {
    return mul_quarter<INV>(a);
  } else if constexpr (4 * j == 3 * N) {
    return mul_quarter<!INV>(a);
  } else {
    constexpr float c = float(cx_cos(2.0 * kPi * double(j) / double(N)));
    constexpr float s = float((INV ? 1.0 : -1.0) * cx_sin(2.0 * kPi * double(j) / double(N)));
    return make_float2(a.x * c - a.y * s, a.x * s + a.y * c);
  }
}

// N-point DFT in registers, natural order in and out.
template <int N, bool INV>
struct Dft;

template <bool INV>
struct Dft<1, INV> {
  CSSM_HD static void run(float2*) {}
};

template <bool INV>
struct Dft<2, INV> {
  CSSM_HD static void run(float2* x) {
    const float2 a = x[0], b = x[1];
    x[0] = cadd(a, b);
    x[1] = csub(a, b);
  }
};

template <bool INV>
struct Dft<4, INV> {
  CSSM_HD static void run(float2* x) {
    const float2 a = cadd(x[0], x[2]);
    const float2 b = csub(x[0], x[2]);
    const float2 c = cadd(x[1], x[3]);
    const float2 d = mul_quarter<INV>(csub(x[1], x[3]));
    x[0] = cadd(a, c);
    x[1] = cadd(b, d);
    x[2] = csub(a, c);
    x[3] = csub(b, d);
  }
};

// Radix-2 butterfly with a compile-time twiddle w = w_N^J (the conjugate when
// INV): x <- x + w y, y <- x - w y.  The trivial twiddles (1, -1, +-i) cost
// four additions.  Otherwise w = c (1 + i t) with t = s / c (or w = s (t + i)
// with t = c / s, whichever keeps |t| <= 1), so w y = c z with
// z = (y.x - t y.y, y.y + t y.x): two FMAs for z and two for each output, six
// in all instead of a complex multiply (4) plus the four additions (Linzer and
// Feig's factoring of the twiddle into the butterfly, IBM J. Res. Dev. 1993).
template <int N, int J, bool INV>
CSSM_HD void bfly(float2& x, float2& y) {
  constexpr int j = ((J % N) + N) % N;
  const float2 a = x, b = y;
  if constexpr (j == 0) {
    x = cadd(a, b);
    y = csub(a, b);
  } else if constexpr (2 * j == N) {
    x = csub(a, b);
    y = cadd(a, b);
  } else if constexpr (4 * j == N || 4 * j == 3 * N) {
    const float2 wb = (4 * j == N) ? mul_quarter<INV>(b) : mul_quarter<!INV>(b);
    x = cadd(a, wb);
    y = csub(a, wb);
  } else {
    constexpr double cd = cx_cos(2.0 * kPi * double(j) / double(N));
    constexpr double sd = (INV ? 1.0 : -1.0) * cx_sin(2.0 * kPi * double(j) / double(N));
    constexpr bool CBIG = (cd < 0 ? -cd : cd) >= (sd < 0 ? -sd : sd);
    constexpr float f = float(CBIG ? cd : sd);          // the factored-out component
    constexpr float t = float(CBIG ? sd / cd : cd / sd);
    float2 z;
    if constexpr (CBIG) {   // w b = c (b.x - t b.y, b.y + t b.x)
      z = make_float2(fmaf(-t, b.y, b.x), fmaf(t, b.x, b.y));
    } else {                // w b = s (t b.x - b.y, t b.y + b.x)
      z = make_float2(fmaf(t, b.x, -b.y), fmaf(t, b.y, b.x));
    }
    x = make_float2(fmaf(f, z.x, a.x), fmaf(f, z.y, a.y));
    y = make_float2(fmaf(-f, z.x, a.x), fmaf(-f, z.y, a.y));
  }
}

// N = 2 N2 (N a power of two, >= 8): decimation in time, X[k] = E[k] + w_N^k O[k],
// X[k + N2] = E[k] - w_N^k O[k] with E, O the DFTs of the even and odd samples,
// each pair one bfly (52 operations for N = 8, 148 for N = 16).
template <int N, bool INV>
struct Dft {
  static_assert(N >= 8 && (N & (N - 1)) == 0, "composite in-register DFT needs a power of two >= 8");
  CSSM_HD static void run(float2* x) {
    constexpr int N2 = N / 2;
    float2 e[N2], o[N2];
    static_for<0, N2>([&](auto S) {
      constexpr int n = decltype(S)::value;
      e[n] = x[2 * n];
      o[n] = x[2 * n + 1];
    });
    Dft<N2, INV>::run(e);
    Dft<N2, INV>::run(o);
    static_for<0, N2>([&](auto K) {
      constexpr int k = decltype(K)::value;
      bfly<N, k, INV>(e[k], o[k]);
      x[k] = e[k];
      x[k + N2] = o[k];
    });
  }
};

}  // namespace cssm
