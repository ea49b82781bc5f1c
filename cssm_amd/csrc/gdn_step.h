// The per-bin step of GatedDeltaNetCSSM's delta rule, shared by the inference
// kernels (gdn.hip) and the training kernels (gdn_bwd.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <math.h>

#include "fft_reg.h"

namespace cssm {

// to_goom's floor (goom.py:161-174): |z| < 1e-7 -> 1e-7 + 0j
__device__ __forceinline__ float2 goom_floor2(float2 z) {
  return (z.x * z.x + z.y * z.y < 1e-14f) ? make_float2(1e-7f, 0.0f) : z;
}

// How the slow path's matrix scan sees the entries of M and Delta (cssm.py:4693-4701, 4939-4991):
//   kScanGoom    use_log and use_goom: to_goom's floor on every entry
//   kScanLinear  use_log=False (direct complex scan), or scan_mode='pallas' at d_k = 2
//                (pallas_matrix_2x2_scan): the entries as they are
//   kScanLogEps  use_log without use_goom: exp(log(|z| + 1e-8) + i angle(z)) = (|z| + 1e-8) z / |z|,
//                1e-8 at z = 0
// Each scan evaluates the linear recurrence s_t = M_t s_{t-1} + Delta_t on those entries.
enum : int { kScanGoom = 0, kScanLinear = 1, kScanLogEps = 2 };

__device__ __forceinline__ float2 logeps_entry(float2 z) {
  const float r2 = fmaf(z.x, z.x, z.y * z.y);
  if (r2 == 0.0f) return make_float2(1e-8f, 0.0f);
  const float f = 1.0f + 1e-8f * rsqrtf(r2);
  return make_float2(z.x * f, z.y * f);
}

// the entry the scan sees (kScanGoom or kScanLogEps; kScanLinear never materialises M)
__device__ __forceinline__ float2 scan_entry(float2 z, int variant) {
  return variant == kScanLogEps ? logeps_entry(z) : goom_floor2(z);
}

// One step of the recurrence for one bin: key-vector norm, M and D as the
// scan variant sees them, s_i <- M s_i + D[i], o_i = sum_a s_i[a] q_a.  q and k arrive with the
// spectral norms already applied; k is normalised here.  The rows i of the state
// update independently given k, v and the gates, so the step splits into a
// per-bin preamble (gdn_bin_prep) and a per-row update (gdn_bin_row) that
// gdn_bin_step runs for every row; lanes may also share a bin's rows.
template <int DK>
struct GdnBinPre {
  float2 aw;    // alpha W_hat
  bool rank1;   // no entry of M or Delta is mapped (rank-1 form of M s)
};

// normalises k in place; aw and which form of the step the scan variant needs
template <int DK>
__device__ __forceinline__ GdnBinPre<DK> gdn_bin_prep(float2 (&k)[DK], const float2 (&v)[DK], float2 wh, float alpha,
                                                      float beta, int variant) {
  float kk = 0.0f;
#pragma unroll
  for (int j = 0; j < DK; ++j) kk = fmaf(k[j].x, k[j].x, fmaf(k[j].y, k[j].y, kk));
  const float kn = 1.0f / sqrtf(kk + 1e-6f);
#pragma unroll
  for (int j = 0; j < DK; ++j) k[j] = cscale(k[j], kn);
  GdnBinPre<DK> pre;
  pre.aw = cscale(wh, alpha);
  // The entries of M = alpha W (I - beta k k^H) and Delta = beta v k^H have magnitudes
  //   |M_rc| = |aw| beta |k_r| |k_c| (r != c),  |M_rr| = |aw| |1 - beta |k_r|^2|,  |Delta_ir| = beta |v_i| |k_r|,
  // so whether to_goom's floor (|x|^2 < 1e-14) takes any of them follows from |aw|^2, |k_r|^2 and
  // |v_i|^2.  When every entry clears the floor by a margin far above the rounding of either
  // evaluation, M s = aw (s - beta k (k^H s)) in rank-1 form (about half the operations);
  // otherwise M and Delta are materialised with the floor applied entry by entry.
  float k2[DK], v2min = 3.0e38f;
#pragma unroll
  for (int j = 0; j < DK; ++j) {
    k2[j] = fmaf(k[j].x, k[j].x, k[j].y * k[j].y);
    v2min = fminf(v2min, fmaf(v[j].x, v[j].x, v[j].y * v[j].y));
  }
  const float aw2 = fmaf(pre.aw.x, pre.aw.x, pre.aw.y * pre.aw.y), b2 = beta * beta;
  constexpr float kLim = 1e-14f * 1.001f;
  float k2min = k2[0], kpair = 3.0e38f, dmin = 3.0e38f;
#pragma unroll
  for (int r = 0; r < DK; ++r) {
    k2min = fminf(k2min, k2[r]);
    const float d = 1.0f - beta * k2[r];
    dmin = fminf(dmin, d * d);
#pragma unroll
    for (int c = r + 1; c < DK; ++c) kpair = fminf(kpair, k2[r] * k2[c]);
  }
  pre.rank1 = aw2 * dmin > kLim && (DK == 1 || aw2 * b2 * kpair > kLim) && b2 * v2min * k2min > kLim;
  // the linear scan maps no entry; the log-eps scan moves every entry, so it always materialises
  if (variant != kScanGoom) pre.rank1 = variant == kScanLinear;
  return pre;
}

// row i of the state: s_i <- M s_i + Delta[i] (in place), returns o_i = sum_r s_ir q_r
template <int DK>
__device__ __forceinline__ float2 gdn_bin_row(float2 (&si)[DK], const float2 vi, const float2 (&q)[DK],
                                              const float2 (&k)[DK], const GdnBinPre<DK>& pre, float beta,
                                              int variant) {
  const float2 aw = pre.aw;
  if (pre.rank1) {
    float2 p = make_float2(0.f, 0.f);                 // sum_c conj(k_c) s_ic
#pragma unroll
    for (int c = 0; c < DK; ++c) {
      p.x = fmaf(k[c].x, si[c].x, fmaf(k[c].y, si[c].y, p.x));
      p.y = fmaf(k[c].x, si[c].y, fmaf(-k[c].y, si[c].x, p.y));
    }
    const float2 bp = cscale(p, beta), bv = cscale(vi, beta);
    float2 oi = make_float2(0.f, 0.f);
#pragma unroll
    for (int r = 0; r < DK; ++r) {
      // t = s_ir - k_r (beta p);  s_ir <- aw t + (beta v_i) conj(k_r)
      const float2 t = make_float2(fmaf(-k[r].x, bp.x, fmaf(k[r].y, bp.y, si[r].x)),
                                   fmaf(-k[r].x, bp.y, fmaf(-k[r].y, bp.x, si[r].y)));
      const float2 dl = cmulc(bv, k[r]);
      const float2 sn = make_float2(fmaf(aw.x, t.x, fmaf(-aw.y, t.y, dl.x)), fmaf(aw.x, t.y, fmaf(aw.y, t.x, dl.y)));
      si[r] = sn;
      oi.x = fmaf(sn.x, q[r].x, fmaf(-sn.y, q[r].y, oi.x));
      oi.y = fmaf(sn.x, q[r].y, fmaf(sn.y, q[r].x, oi.y));
    }
    return oi;
  }
  // entries of M recomputed where they are used (this path is rare; no 4 x 4 array held)
  float2 sn[DK];
#pragma unroll
  for (int r = 0; r < DK; ++r) {
    float2 acc = scan_entry(cscale(cmulc(vi, k[r]), beta), variant);
#pragma unroll
    for (int c = 0; c < DK; ++c) {
      // M_rc = alpha W (delta_rc - beta k_r conj k_c)
      const float2 kk_rc = cmulc(k[r], k[c]);
      float2 m = make_float2(-beta * kk_rc.x, -beta * kk_rc.y);
      if (r == c) m.x += 1.0f;
      const float2 M = scan_entry(cmul(aw, m), variant);
      acc.x = fmaf(M.x, si[c].x, fmaf(-M.y, si[c].y, acc.x));
      acc.y = fmaf(M.x, si[c].y, fmaf(M.y, si[c].x, acc.y));
    }
    sn[r] = acc;
  }
  float2 oi = make_float2(0.f, 0.f);
#pragma unroll
  for (int r = 0; r < DK; ++r) {
    si[r] = sn[r];
    oi.x = fmaf(sn[r].x, q[r].x, fmaf(-sn[r].y, q[r].y, oi.x));
    oi.y = fmaf(sn[r].x, q[r].y, fmaf(sn[r].y, q[r].x, oi.y));
  }
  return oi;
}

template <int DK>
__device__ __forceinline__ void gdn_bin_step(float2 (&s)[DK][DK], const float2 (&q)[DK], float2 (&k)[DK],
                                             const float2 (&v)[DK], float2 wh, float alpha, float beta,
                                             int variant, float2 (&o)[DK]) {
  const GdnBinPre<DK> pre = gdn_bin_prep<DK>(k, v, wh, alpha, beta, variant);
#pragma unroll
  for (int i = 0; i < DK; ++i) o[i] = gdn_bin_row<DK>(s[i], v[i], q, k, pre, beta, variant);
}

}  // namespace cssm
