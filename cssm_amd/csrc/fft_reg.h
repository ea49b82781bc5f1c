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
// The functions are __host__ __device__ so the host-side unit test in
// tests/ can check them against a brute-force DFT without a GPU.
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

// N = N1 * N2 with N1 = 4: index n = s + N2 m, k = k1 + N1 q.
//   pass 1 (per s):  A_s[k1] = w_N^{s k1} * DFT_4{ x[s + N2 m] }[k1]
//   pass 2 (per k1): X[k1 + 4 q] = DFT_N2{ A_s[k1] }[q]
template <int N, bool INV>
struct Dft {
  static_assert(N % 4 == 0 && N >= 8, "composite in-register DFT needs N = 4 * N2");
  CSSM_HD static void run(float2* x) {
    constexpr int N1 = 4, N2 = N / 4;
    float2 a[N];
    static_for<0, N2>([&](auto S) {
      constexpr int s = decltype(S)::value;
      float2 t[N1];
      static_for<0, N1>([&](auto M) {
        constexpr int m = decltype(M)::value;
        t[m] = x[s + N2 * m];
      });
      Dft<N1, INV>::run(t);
      static_for<0, N1>([&](auto K) {
        constexpr int k = decltype(K)::value;
        a[s * N1 + k] = twiddle<N, s * k, INV>(t[k]);
      });
    });
    static_for<0, N1>([&](auto K) {
      constexpr int k1 = decltype(K)::value;
      float2 t[N2];
      static_for<0, N2>([&](auto S) {
        constexpr int s = decltype(S)::value;
        t[s] = a[s * N1 + k1];
      });
      Dft<N2, INV>::run(t);
      static_for<0, N2>([&](auto Q) {
        constexpr int q = decltype(Q)::value;
        x[k1 + N1 * q] = t[q];
      });
    });
  }
};

}  // namespace cssm
