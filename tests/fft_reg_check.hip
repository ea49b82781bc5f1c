// Host-side check of the in-register DFTs of cssm_amd/csrc/fft_reg.h (built and
// run by tests/test_fft_reg_host.py, no GPU): Dft<N, INV> for N = 2 .. 32 in
// both directions against a brute-force double-precision DFT on random complex
// inputs.  Prints one line per (N, INV): the max error relative to the RMS of
// the exact output.
#include <cmath>
#include <cstdio>
#include <random>

#include "fft_reg.h"

template <int N, bool INV>
static double check(std::mt19937& rng) {
  std::normal_distribution<double> nd(0.0, 1.0);
  double worst = 0.0;
  for (int rep = 0; rep < 200; ++rep) {
    float2 x[N];
    double xr[N], xi[N];
    for (int n = 0; n < N; ++n) {
      x[n] = make_float2(float(nd(rng)), float(nd(rng)));
      xr[n] = x[n].x;
      xi[n] = x[n].y;
    }
    cssm::Dft<N, INV>::run(x);
    double err = 0.0, rms = 0.0;
    for (int k = 0; k < N; ++k) {
      double re = 0.0, im = 0.0;
      for (int n = 0; n < N; ++n) {
        const double a = (INV ? 2.0 : -2.0) * M_PI * double(n) * double(k) / double(N);
        re += xr[n] * std::cos(a) - xi[n] * std::sin(a);
        im += xr[n] * std::sin(a) + xi[n] * std::cos(a);
      }
      err = std::fmax(err, std::fmax(std::fabs(x[k].x - re), std::fabs(x[k].y - im)));
      rms += re * re + im * im;
    }
    worst = std::fmax(worst, err / std::sqrt(rms / N));
  }
  return worst;
}

int main() {
  std::mt19937 rng(7);
  std::printf("2 0 %.3e\n", check<2, false>(rng));
  std::printf("2 1 %.3e\n", check<2, true>(rng));
  std::printf("4 0 %.3e\n", check<4, false>(rng));
  std::printf("4 1 %.3e\n", check<4, true>(rng));
  std::printf("8 0 %.3e\n", check<8, false>(rng));
  std::printf("8 1 %.3e\n", check<8, true>(rng));
  std::printf("16 0 %.3e\n", check<16, false>(rng));
  std::printf("16 1 %.3e\n", check<16, true>(rng));
  std::printf("32 0 %.3e\n", check<32, false>(rng));
  std::printf("32 1 %.3e\n", check<32, true>(rng));
  return 0;
}
