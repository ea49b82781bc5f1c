// Fused gated spectral scan for power-of-two planes (gfx950).
//
// One workgroup owns NP consecutive (b, c) planes for all T steps.  Per step
// it loads u_t and z_t once from HBM, runs the 2-D real FFT through LDS,
// advances the complex diagonal state h (kept in VGPRs for the whole scan),
// applies C, runs the inverse (irfft2 C2R rule), multiplies by the z gate
// and writes y_t once.
//
// Reference semantics (drewlinsley/CSSM, src/models/cssm.py):
//   U   = rfft2(x_main)                                   :532-533
//   A_t = floor(K_hat) * exp(-Delta_t)                    :559-566 (GOOM form)
//   V_t = (Delta_t + 1e-8) * floor(U_t * B_t)             :562-567
//   h_t = A_t h_{t-1} + V_t,  h_{-1} = 0                  :570-575 (log-space
//         associative scan = this linear recurrence; goom.py:144-196,
//         math.py:24-54, operations.py:17-41)
//   y_t = irfft2(C_t * h_t, s=(H,W)) * z_gate_t           :576-581
// floor(a) = 1e-7 + 0j where |a| < 1e-7 (goom.py:161-174).
//
// The 2-D real FFT passes (and their LDS layout) are those of fft_plane.h.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <initializer_list>

#include "dft_small.h"
#include "fft_plane.h"
#include "launch.h"

namespace cssm {

// The forward row pass skips the 1/2 of the packed-row separation, so the
// spectrum the recurrence sees is U' = 2U for every bin (the edge unpack keeps
// its 1/2 and inherits the factor from the doubled DC/Nyquist column; the
// small-plane kernel doubles its input on load to match).  The state is then
// h' = 2h: the gate planes carry the floor term at that scale and C / 2
// (c_scale = 1 / (2 H W)), so y is unchanged.
//
// gate g = (E, DB, VF, GC): E = exp(-Delta), DB = (Delta + 1e-8) B,
// VF = 2e-7 (Delta + 1e-8) (the input term when |U B| < 1e-7), GC = C c_scale.
// |DB U'| < VF  <=>  |U B| < 1e-7 since Delta + 1e-8 > 0.
__device__ __forceinline__ float2 scan_bin(float2& h, float2 U, float4 g, float2 kh) {
  float2 V = make_float2(U.x * g.y, U.y * g.y);
  if (V.x * V.x + V.y * V.y < g.z * g.z) V = make_float2(g.z, 0.0f);
  const float2 A = make_float2(kh.x * g.x, kh.y * g.x);
  const float2 hn = make_float2(fmaf(A.x, h.x, fmaf(-A.y, h.y, V.x)), fmaf(A.x, h.y, fmaf(A.y, h.x, V.y)));
  h = hn;
  return make_float2(hn.x * g.w, hn.y * g.w);
}

struct ScanArgs {
  const void* u;
  const void* z;
  void* y;
  const float4* gates;   // (B, T, H, WF) per-bin (E, DB, VF, GC), columns in scan_col order
  const float2* khat;    // (C, H, WF), GOOM-floored, scan layout (columns in scan_col order, slots khat_pos)
  int T, C, u_act, z_act;
};


// C2 / edge policy of the fused scan: the state of the thread's C2 bins lives
// in registers for the whole launch (h); the DC / Nyquist bins, which only the
// waves owning a packed column touch, keep theirs in LDS (hE).
template <class G>
struct GatedScanOp {
  static constexpr int H = G::H, WH = G::WH, WF = G::WF, H1 = G::H1, H2 = G::H2;
  // the packed column's lanes may run bins(): their state slots serve no
  // other bin and their results are overwritten by the packed-column I1
  static constexpr bool kPackedColumnToo = true;
  // gates in batches of QB bins (fewer registers in flight at 4 waves / SIMD); the
  // first batch of a unit is issued before its column DFT (prefetch)
  static constexpr bool kPrefetch = true;
  static constexpr int QB = G::NT >= 512 ? 4 : G::H2;
  float2 (&h)[G::JC2][2][G::H2];
  float2* hE;   // LDS: state of the DC / Nyquist bins, 4 per edge job (pl, e)
  Buf gbuf;   // gates of (b, t): (H, WF) float4
  Buf kbuf;   // K_hat of the group's planes: (NP, H, WF) float2
  float4 pg[QB];   // the unit's first gate batch, in flight during its column DFT
  float2 pk[QB];
  // 128 x 128: K_hat's rows u and u + 16 share slot pairs (khat_pos), so bins q, q + 1 of a unit
  // (rows k + 16 q, k + 16 (q + 1), q even) come in one 16-byte load over whole cache lines
  static constexpr bool KPAIR = G::H == 128 && G::W == 128;
  static_assert(!KPAIR || (QB % 2 == 0 && H1 == 16), "paired K_hat rows need even batches of rows 16 apart");

  // K_hat of bins q0 .. q0 + QB - 1 of unit k at column position n of plane pl
  __device__ __forceinline__ void khat_batch(int pl, int k, int n, int q0, float2 (&kq)[QB]) const {
    if constexpr (KPAIR) {
      const unsigned kp = unsigned(pl * H * WF * 8) + unsigned(k * WF + n) * 16u;
#pragma unroll
      for (int p = 0; p < QB / 2; ++p) {
        const float4 v = kbuf.ld4(kp, (q0 / 2 + p) * H1 * WF * 16);
        kq[2 * p] = make_float2(v.x, v.y);
        kq[2 * p + 1] = make_float2(v.z, v.w);
      }
    } else {
      const unsigned ki = unsigned(pl * H * WF) + unsigned(k * WF + n);
#pragma unroll
      for (int q = 0; q < QB; ++q) kq[q] = kbuf.ld2(ki * 8u, (q0 + q) * H1 * WF * 8);
    }
  }

  __device__ __forceinline__ void prefetch(int pl, int k, int n) {
    const unsigned gi = unsigned(k * WF + n);
#pragma unroll
    for (int q = 0; q < QB; ++q) pg[q] = gbuf.ld4(gi * 16u, q * H1 * WF * 16);
    khat_batch(pl, k, n, 0, pk);
  }

  // gates of (b, t) and the spectral kernel of this plane at bins (k + H1 q,
  // column at position n)
  __device__ __forceinline__ void bins(int j, int a2, int pl, int k, int n, float2 (&sp)[G::H2]) const {
    const unsigned gi = unsigned(k * WF + n);
#pragma unroll
    for (int q0 = 0; q0 < H2; q0 += QB) {
      float4 gq[QB];
      float2 kq[QB];
      if (q0 != 0) khat_batch(pl, k, n, q0, kq);
#pragma unroll
      for (int q = 0; q < QB; ++q) {
        if (q0 == 0) {
          gq[q] = pg[q];
          kq[q] = pk[q];
        } else {
          gq[q] = gbuf.ld4(gi * 16u, (q0 + q) * H1 * WF * 16);
        }
      }
#pragma unroll
      for (int q = 0; q < QB; ++q) sp[q0 + q] = scan_bin(h[j][a2][q0 + q], sp[q0 + q], gq[q], kq[q]);
    }
  }

  __device__ __forceinline__ void edge(int j, int pl, int uA, int uB, int, float2 (&v4)[4]) const {
    const unsigned kp = unsigned(pl * H * WF);
    const unsigned bi[4] = {unsigned(uA * WF), unsigned(uA * WF + WH), unsigned(uB * WF), unsigned(uB * WF + WH)};
    const unsigned ks[4] = {unsigned(khat_pos(H, G::W, uA, 0)), unsigned(khat_pos(H, G::W, uA, WH)),
                            unsigned(khat_pos(H, G::W, uB, 0)), unsigned(khat_pos(H, G::W, uB, WH))};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float2& hs = hE[(pl * G::HP + uA) * 4 + i];
      float2 hv = hs;
      v4[i] = scan_bin(hv, v4[i], gbuf.ld4(bi[i] * 16u), kbuf.ld2((kp + ks[i]) * 8u));
      hs = hv;
    }
  }
};

template <int LH, int LW, int NP, int PPT, class IO>
__global__ void __launch_bounds__((NP << (LH + LW)) / PPT, PPT >= 64 ? 2 : ((NP << (LH + LW)) / PPT >= 512 ? 4 : 1))
gated_scan_pow2(const ScanArgs a) {
  using G = Geom<LH, LW, NP, PPT, true>;
  static_assert(G::NT == (NP << (LH + LW)) / PPT, "launch bound");
  constexpr int H = G::H, WF = G::WF, W = G::W, H2 = G::H2, NT = G::NT;
  using V4 = typename IO::V4;
  using TE = typename IO::T;

  __shared__ __attribute__((aligned(16))) float smem[G::LDS_FLOATS];
  const PlaneFft<G> fft(smem);

  const int T = a.T, C = a.C;
  // this workgroup: batch b, channels c0 .. c0 + NP - 1 (C % NP == 0)
  const int groups = C / NP;
  const int b = blockIdx.x / groups;
  const int c0 = (blockIdx.x % groups) * NP;
  const size_t HWs = size_t(H) * W;
  auto group_elems = [&](int t) -> size_t { return ((size_t(b) * T + t) * C + c0) * HWs; };
  const TE* __restrict__ up = static_cast<const TE*>(a.u);
  const TE* __restrict__ zp = static_cast<const TE*>(a.z);
  TE* __restrict__ yp = static_cast<TE*>(a.y);

  fft.init_twiddles(threadIdx.x);
  const int wv = __builtin_amdgcn_readfirstlane(int(threadIdx.x) / 64), ln = int(threadIdx.x) % 64;

  // state: the C2 bins of this thread in VGPRs, the DC / Nyquist bins (touched
  // only by the waves owning a packed column) in LDS
  __shared__ float2 hE[NP * G::HP * 4];
  float2 h[G::JC2][2][H2];
#pragma unroll
  for (int j = 0; j < G::JC2; ++j)
#pragma unroll
    for (int q = 0; q < H2; ++q) h[j][0][q] = h[j][1][q] = make_float2(0.f, 0.f);
  for (int i = threadIdx.x; i < NP * G::HP * 4; i += NT) hE[i] = make_float2(0.f, 0.f);

  // u_0 into the plane buffer (each wave loads the rows it owns)
  constexpr int VB = int(sizeof(V4));
  constexpr unsigned GROUP_BYTES = unsigned(NP * H * W * sizeof(TE));
  __syncthreads();   // twiddle tables
  {
    const auto m = G::v4_lane(ln);
    const auto col = PlaneFft<G>::v4_col(m.c4);
    const Buf ub(up + group_elems(0), GROUP_BYTES);
    V4 ld[G::JLD];
#pragma unroll
    for (int i = 0; i < G::JLD; ++i) {
      unsigned vo;
      int so;
      G::template v4_goff<VB>(wv, i, m, vo, so);
      ub.ld(ld[i], vo, so);
    }
#pragma unroll
    for (int i = 0; i < G::JLD; ++i) fft.v4_put(G::v4_row(wv, i, m), col, act4(IO::to_f4(ld[i]), a.u_act));
  }
  wave_sync();

  for (int t = 0; t < T; ++t) {
    // Re-derive the thread index inside the loop so the compiler rebuilds the
    // (cheap, base + constant) LDS addresses per step instead of hoisting
    // hundreds of them into registers for the whole scan.
    int lane = ln;
    asm volatile("" : "+v"(lane));
    __builtin_assume(lane >= 0 && lane < 64);   // keeps the index arithmetic unsigned and 24-bit
    GatedScanOp<G> op{h, hE, Buf(a.gates + (size_t(b) * T + t) * size_t(H) * WF, unsigned(H * WF * sizeof(float4))),
                      Buf(a.khat + size_t(c0) * H * WF, unsigned(NP * H * WF * sizeof(float2)))};

    fft.r1(wv, lane);
    fft.r2(wv, lane);
    fft.c1(wv, lane);
    fft.template c2<true, true>(wv, lane, op);
    fft.template edges<true, true>(wv, lane, op);
    fft.i1_packed(wv, lane);
    fft.i2(wv, lane);
    fft.i3(wv, lane);
    // z_t of the first chunk of this wave's rows is issued before the last
    // inverse pass, so those loads are in flight while it runs
    constexpr int CH = NT >= 512 ? 4 : (G::JLD < 8 ? G::JLD : 8);
    const auto m = G::v4_lane(lane);
    const Buf zb(zp + group_elems(t), GROUP_BYTES);
    V4 ldg[CH];
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      unsigned vo;
      int so;
      G::template v4_goff<VB>(wv, i, m, vo, so);
      zb.ld(ldg[i], vo, so);
    }
    fft.i4(wv, lane);

    // ---------- STORE y_t = y * z_gate, and LOAD u_{t+1} into the same slots
    // (in chunks of CH vectors to bound the registers in flight).  With 4-vector
    // chunks (512-thread groups) z runs one chunk ahead: z of chunk c + 1 is issued
    // with u of chunk c, so a chunk's stores never wait for a load issued after the
    // previous chunk's u arrived.
    {
      constexpr bool ZAHEAD = NT >= 512;
      const auto col = PlaneFft<G>::v4_col(m.c4);
      const Buf ub(up + group_elems(t + 1 < T ? t + 1 : t), GROUP_BYTES);
      const Buf yb(yp + group_elems(t), GROUP_BYTES);
#pragma unroll
      for (int c = 0; c < G::JLD; c += CH) {
        V4 ldu[CH], ldn[CH];
        const int cz = ZAHEAD ? c + CH : c;   // the chunk whose z is loaded now
        if (ZAHEAD ? cz < G::JLD : c > 0) {
#pragma unroll
          for (int i = 0; i < CH; ++i) {
            unsigned vo;
            int so;
            G::template v4_goff<VB>(wv, cz + i, m, vo, so);
            zb.ld(ZAHEAD ? ldn[i] : ldg[i], vo, so);
          }
        }
        if (t + 1 < T) {
#pragma unroll
          for (int i = 0; i < CH; ++i) {
            unsigned vo;
            int so;
            G::template v4_goff<VB>(wv, c + i, m, vo, so);
            ub.ld(ldu[i], vo, so);
          }
        }
#pragma unroll
        for (int i = 0; i < CH; ++i) {
          unsigned vo;
          int so;
          G::template v4_goff<VB>(wv, c + i, m, vo, so);
          const float4 yv = fft.v4_get(G::v4_row(wv, c + i, m), col);
          const float4 gv = act4(IO::to_f4(ldg[i]), a.z_act);
          yb.st(IO::from_f4(make_float4(yv.x * gv.x, yv.y * gv.y, yv.z * gv.z, yv.w * gv.w)), vo, so);
        }
        if (t + 1 < T) {
#pragma unroll
          for (int i = 0; i < CH; ++i)
            fft.v4_put(G::v4_row(wv, c + i, m), col, act4(IO::to_f4(ldu[i]), a.u_act));
        }
        if (ZAHEAD && cz < G::JLD) {
#pragma unroll
          for (int i = 0; i < CH; ++i) ldg[i] = ldn[i];
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    wave_sync();
  }
}


// ---------------------------------------------------------------------------
// Small planes of any size up to 16 x 16 (the CSSM-SHViT stage shapes 14 x 14
// and 7 x 7 are not powers of two): direct DFTs with compile-time twiddles.
//
// A workgroup owns NP consecutive planes of the flattened (b, c) index (the
// last group may be partial; a group may span two batch elements) for all T
// steps.  Per step:
//   rows   R[pl][h][v] = sum_w x[h][w] e^{-2 pi i v w / W}   (v < Wf; one thread
//          per row computes all Wf bins, the row read once from LDS)
//   cols   X[pl][u][v] = sum_h R[h][v] e^{-2 pi i u h / H}   (one thread per
//          column (pl, v), fixed for the launch, so the state of its H bins
//          stays in registers)
//   scan   h = floor(K_hat) e^{-Delta} h + (Delta + 1e-8) floor(X B);  S = C h / (H W)
//          (evaluated on 2X and 2h with the gate planes' doubled floor term and C / (2 H W))
//   icols  Z[pl][h][v] = sum_u S[u][v] e^{+2 pi i u h / H}
//   C2R    y[h][w] = Re Z[h][0] + 2 sum_{0 < v < W/2} Re(Z[h][v] e^{2 pi i v w / W})
//                    + [W even] (-1)^w Re Z[h][W/2]                 (numpy irfft2)
//   store  y * z_gate
// Every DFT unrolls over both indices with the twiddles as immediates (exact
// to float from a double-precision series); the trivial ones (1, -1, +-i)
// fold into adds and swaps.
// ---------------------------------------------------------------------------
// (at least 4 waves per SIMD below 8 x 8; from 8 x 8 up the column pass's registers would spill
// under that bound, so the compiler may take up to 256, or 168 for 3 waves at T = 1 up to 14 x 14)
// ONE (T = 1): the state enters at zero and is never read again, so h = V: no state registers,
// no K_hat loads and no decay (A h = 0 exactly: A is finite), the same results as the general form.
template <int H, int W, class IO, bool ONE>
__global__ void __launch_bounds__((SmallGeom<H, W>::NT), (H >= 8 ? (ONE && H <= 14 ? 3 : 2) : 512 / SmallGeom<H, W>::NT))
gated_scan_small(const ScanArgs a, long long P) {
  using G = SmallGeom<H, W>;
  constexpr int WF = G::WF, HW = G::HW, NT = G::NT, NP = G::NP;
  constexpr int NE = (NP * HW + NT - 1) / NT;   // plane elements per thread (element path)
  // vector path: a group inside one batch element is one contiguous run of NP H W elements;
  // when its start is 4-element aligned it moves as NV 4-element vectors, NEV per thread
  constexpr bool VEC_OK = (NP * HW) % 4 == 0;
  constexpr int NV = NP * HW / 4, NEV = (NV + NT - 1) / NT;
  constexpr bool GATES_EARLY = H < 8 && H != 4;
  static_assert(H < 128 && W < 128, "per-bin planes of these sizes are in natural column order");
  using TE = typename IO::T;
  using V4 = typename IO::V4;
  __shared__ __attribute__((aligned(16))) float xs[NP * HW];   // u_t, then y_t
  __shared__ float2 rs[NP * G::PS];      // row spectra, then the inverse column output
  __shared__ long long base_u[NP];       // element offset of plane pl at t = 0: (b T C + c) HW
  __shared__ int gate_b[NP];             // batch index of plane pl (-1: beyond P)

  const int T = a.T, C = a.C;
  const int tid = threadIdx.x;
  const long long p0 = (long long)blockIdx.x * NP;
  for (int i = tid; i < NP; i += NT) {
    const long long pp = p0 + i;
    const int b = int(pp / C), c = int(pp % C);
    gate_b[i] = pp < P ? b : -1;
    base_u[i] = pp < P ? ((long long)b * T * C + c) * HW : 0;
  }
  const TE* __restrict__ up = static_cast<const TE*>(a.u);
  const TE* __restrict__ zp = static_cast<const TE*>(a.z);
  TE* __restrict__ yp = static_cast<TE*>(a.y);
  const size_t tstride = size_t(C) * HW;   // one time step
  constexpr unsigned VA = unsigned(sizeof(V4)) - 1u;
  const bool ptr_ok = ((reinterpret_cast<uintptr_t>(up) | reinterpret_cast<uintptr_t>(zp) |
                        reinterpret_cast<uintptr_t>(yp)) & VA) == 0;

  // this thread's column (pl, v) and the state of its H bins
  const int cpl = tid / WF, cv = tid % WF;
  const bool has_col = tid < G::NCJ;
  float2 st[ONE ? 1 : H];
#pragma unroll
  for (int u = 0; u < (ONE ? 1 : H); ++u) st[u] = make_float2(0.f, 0.f);
  __syncthreads();
  // all planes of the group in one batch element: one contiguous run per step
  const bool contig = gate_b[0] >= 0 && gate_b[NP - 1] == gate_b[0];
  const int bcol = has_col ? gate_b[cpl] : -1;
  const int ccol = int((p0 + (has_col ? cpl : 0)) % C);

  for (int t = 0; t < T; ++t) {
    // the element offsets of the load / store loops are rebuilt every step
    // (cheap) instead of being hoisted into registers for the whole launch
    int tl = tid;
    asm volatile("" : "+v"(tl));
    const long long base0 = base_u[0] + (long long)t * tstride;
    const bool vec = VEC_OK && contig && ptr_ok && (base0 & 3) == 0;   // uniform over the group
    // The step's global loads are issued before any of them is used: u_t (doubled, act
    // applied: the recurrence runs on 2U as in the power-of-two kernel), on the vector path
    // z_t (read when y_t is stored), and the gates and K_hat of this thread's column (read
    // after its forward DFT) either here or after the row pass (GATES_EARLY: measured faster
    // at 7 x 7, slower at 4 x 4 and 14 x 14), so one memory latency per step is exposed
    // instead of three.
    float4 gq[H];
    float2 kq[ONE ? 1 : H];
    auto load_gates = [&]() {
      if (bcol >= 0) {
        const float4* gp = a.gates + (size_t(bcol) * T + t) * (H * WF) + cv;
        const float2* kp = a.khat + size_t(ccol) * (H * WF) + cv;
#pragma unroll
        for (int u = 0; u < H; ++u) {
          if constexpr (ONE) {
            // the decay component is not read: the input gain, floor term and readout gain only
            const float* g3 = reinterpret_cast<const float*>(gp + u * WF) + 1;
            gq[u] = make_float4(0.0f, g3[0], g3[1], g3[2]);
          } else {
            gq[u] = gp[u * WF];
            kq[u] = kp[u * WF];
          }
        }
      }
    };
    if constexpr (GATES_EARLY) load_gates();
    V4 zv[NEV];
    if (vec) {
      const V4* u4 = reinterpret_cast<const V4*>(up + base0);
      const V4* z4 = reinterpret_cast<const V4*>(zp + base0);
      V4 uv[NEV];
#pragma unroll
      for (int k = 0; k < NEV; ++k) {
        const int e = k * NT + tl;
        if (k * NT + NT <= NV || e < NV) uv[k] = u4[e];
      }
#pragma unroll
      for (int k = 0; k < NEV; ++k) {
        const int e = k * NT + tl;
        if (k * NT + NT <= NV || e < NV) zv[k] = z4[e];
      }
#pragma unroll
      for (int k = 0; k < NEV; ++k) {
        const int e = k * NT + tl;
        if (k * NT + NT <= NV || e < NV) {
          const float4 f = act4(IO::to_f4(uv[k]), a.u_act);
          *reinterpret_cast<float4*>(xs + 4 * e) = make_float4(2.0f * f.x, 2.0f * f.y, 2.0f * f.z, 2.0f * f.w);
        }
      }
    } else {
      float v[NE];
#pragma unroll
      for (int k = 0; k < NE; ++k) {
        const int e = k * NT + tl;
        v[k] = 0.0f;
        if (e < NP * HW) {
          if (contig) {
            v[k] = IO::to_f(up[size_t(base0 + e)]);
          } else {
            const int pl = e / HW, px = e % HW;
            if (gate_b[pl] >= 0) v[k] = IO::to_f(up[size_t(base_u[pl]) + t * tstride + px]);
          }
        }
      }
#pragma unroll
      for (int k = 0; k < NE; ++k) {
        const int e = k * NT + tl;
        if (e < NP * HW) xs[e] = 2.0f * (a.u_act == 1 ? silu_f(v[k]) : v[k]);
      }
    }
    __syncthreads();
    // rows: one thread per (pl, h), all Wf bins
    for (int j = tid; j < G::NRJ; j += NT) {
      small_row_r2c<W>(xs + j * W, rs + (j / H) * G::PS + (j % H) * G::RSP);   // row h of plane pl: j = pl H + h
    }
    __syncthreads();
    if constexpr (!GATES_EARLY) load_gates();
    // columns: forward DFT over h, the recurrence on the H bins, inverse DFT over u
    if (has_col) {
      float2 r[H];
#pragma unroll
      for (int h = 0; h < H; ++h) r[h] = rs[cpl * G::PS + h * G::RSP + cv];
      float2 sv[H];
      dft_sym<H, false>(r, sv);
      if (bcol >= 0) {
#pragma unroll
        for (int u = 0; u < H; ++u) {
          if constexpr (ONE) {
            float2 V = make_float2(sv[u].x * gq[u].y, sv[u].y * gq[u].y);
            if (V.x * V.x + V.y * V.y < gq[u].z * gq[u].z) V = make_float2(gq[u].z, 0.0f);
            sv[u] = make_float2(V.x * gq[u].w, V.y * gq[u].w);
          } else {
            sv[u] = scan_bin(st[u], sv[u], gq[u], kq[u]);
          }
        }
      } else {
#pragma unroll
        for (int u = 0; u < H; ++u) sv[u] = make_float2(0.f, 0.f);
      }
      dft_sym<H, true>(sv, r);
#pragma unroll
      for (int h = 0; h < H; ++h) rs[cpl * G::PS + h * G::RSP + cv] = r[h];
    }
    __syncthreads();
    // C2R rows into xs
    for (int j = tid; j < G::NRJ; j += NT) {
      small_row_c2r<W>(rs + (j / H) * G::PS + (j % H) * G::RSP, xs + j * W);
    }
    __syncthreads();
    // x z_gate, store y_t
    if (vec) {
      V4* y4 = reinterpret_cast<V4*>(yp + base0);
#pragma unroll
      for (int k = 0; k < NEV; ++k) {
        const int e = k * NT + tl;
        if (k * NT + NT <= NV || e < NV) {
          const float4 yv = *reinterpret_cast<const float4*>(xs + 4 * e);
          const float4 g = act4(IO::to_f4(zv[k]), a.z_act);
          y4[e] = IO::from_f4(make_float4(yv.x * g.x, yv.y * g.y, yv.z * g.z, yv.w * g.w));
        }
      }
    } else {
      float zg[NE];
#pragma unroll
      for (int k = 0; k < NE; ++k) {
        const int e = k * NT + tl;
        zg[k] = 0.0f;
        if (e < NP * HW) {
          if (contig) {
            zg[k] = IO::to_f(zp[size_t(base0 + e)]);
          } else {
            const int pl = e / HW, px = e % HW;
            if (gate_b[pl] >= 0) zg[k] = IO::to_f(zp[size_t(base_u[pl]) + t * tstride + px]);
          }
        }
      }
#pragma unroll
      for (int k = 0; k < NE; ++k) {
        const int e = k * NT + tl;
        if (e >= NP * HW) continue;
        const float g = a.z_act == 1 ? silu_f(zg[k]) : zg[k];
        if (contig) {
          yp[size_t(base0 + e)] = IO::from_f(xs[e] * g);
        } else {
          const int pl = e / HW, px = e % HW;
          if (gate_b[pl] >= 0) yp[size_t(base_u[pl]) + t * tstride + px] = IO::from_f(xs[e] * g);
        }
      }
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Planes of at most 16 samples (3 x 3; 4 x 4 has its own kernel below): one thread per (b, c)
// plane for all T steps, the whole plane, its spectrum and its state in registers, no LDS and
// no barriers.  The DFT functions, recurrence and C2R rule are those of gated_scan_small; the
// plane's u_t and z_t come as 4-element vectors when the plane size allows it and the tensors
// are aligned (one plane = H W contiguous elements).
// ---------------------------------------------------------------------------
template <int H, int W, class IO, bool ONE>
__global__ void __launch_bounds__(256) gated_scan_plane(const ScanArgs a, long long P) {
  constexpr int WF = W / 2 + 1, HW = H * W;
  static_assert(HW <= 16, "one plane per thread in registers");
  constexpr bool VEC_OK = HW % 4 == 0;
  using TE = typename IO::T;
  using V4 = typename IO::V4;
  const long long pl = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (pl >= P) return;   // (no barriers below)
  const int T = a.T, C = a.C;
  const int b = int(pl / C), c = int(pl % C);
  const TE* __restrict__ up = static_cast<const TE*>(a.u);
  const TE* __restrict__ zp = static_cast<const TE*>(a.z);
  TE* __restrict__ yp = static_cast<TE*>(a.y);
  constexpr unsigned VA = unsigned(sizeof(V4)) - 1u;
  const bool vec = VEC_OK && ((reinterpret_cast<uintptr_t>(up) | reinterpret_cast<uintptr_t>(zp) |
                               reinterpret_cast<uintptr_t>(yp)) & VA) == 0;
  float2 st[ONE ? 1 : H][WF];
  float2 kh[ONE ? 1 : H][WF];
  if constexpr (!ONE) {
    const float2* kp = a.khat + size_t(c) * (H * WF);
#pragma unroll
    for (int u = 0; u < H; ++u)
#pragma unroll
      for (int v = 0; v < WF; ++v) {
        kh[u][v] = kp[u * WF + v];
        st[u][v] = make_float2(0.f, 0.f);
      }
  }
  for (int t = 0; t < T; ++t) {
    const size_t base = ((size_t(b) * T + t) * C + c) * HW;
    float x[HW], zg[HW];
    if (vec) {
      const V4* u4 = reinterpret_cast<const V4*>(up + base);
      const V4* z4 = reinterpret_cast<const V4*>(zp + base);
      V4 uv[HW / 4 > 0 ? HW / 4 : 1], zv[HW / 4 > 0 ? HW / 4 : 1];
#pragma unroll
      for (int k = 0; k < HW / 4; ++k) uv[k] = u4[k];
#pragma unroll
      for (int k = 0; k < HW / 4; ++k) zv[k] = z4[k];
#pragma unroll
      for (int k = 0; k < HW / 4; ++k) {
        const float4 f = act4(IO::to_f4(uv[k]), a.u_act), g = act4(IO::to_f4(zv[k]), a.z_act);
        x[4 * k] = 2.0f * f.x;
        x[4 * k + 1] = 2.0f * f.y;
        x[4 * k + 2] = 2.0f * f.z;
        x[4 * k + 3] = 2.0f * f.w;
        zg[4 * k] = g.x;
        zg[4 * k + 1] = g.y;
        zg[4 * k + 2] = g.z;
        zg[4 * k + 3] = g.w;
      }
    } else {
#pragma unroll
      for (int e = 0; e < HW; ++e) {
        const float v = IO::to_f(up[base + e]);
        x[e] = 2.0f * (a.u_act == 1 ? silu_f(v) : v);
        const float g = IO::to_f(zp[base + e]);
        zg[e] = a.z_act == 1 ? silu_f(g) : g;
      }
    }
    // rows, then per column: forward DFT over h, the recurrence, inverse DFT over u
    float2 R[H][WF];
#pragma unroll
    for (int h = 0; h < H; ++h) small_row_r2c<W>(x + h * W, R[h]);
    const float4* gp = a.gates + (size_t(b) * T + t) * (H * WF);
#pragma unroll
    for (int v = 0; v < WF; ++v) {
      float2 r[H], sv[H];
#pragma unroll
      for (int h = 0; h < H; ++h) r[h] = R[h][v];
      dft_sym<H, false>(r, sv);
#pragma unroll
      for (int u = 0; u < H; ++u) {
        const float4 g = gp[u * WF + v];
        if constexpr (ONE) {
          float2 V = make_float2(sv[u].x * g.y, sv[u].y * g.y);
          if (V.x * V.x + V.y * V.y < g.z * g.z) V = make_float2(g.z, 0.0f);
          sv[u] = make_float2(V.x * g.w, V.y * g.w);
        } else {
          sv[u] = scan_bin(st[u][v], sv[u], g, kh[u][v]);
        }
      }
      dft_sym<H, true>(sv, r);
#pragma unroll
      for (int h = 0; h < H; ++h) R[h][v] = r[h];
    }
    // C2R rows, x z_gate, store y_t
    float y[HW];
#pragma unroll
    for (int h = 0; h < H; ++h) small_row_c2r<W>(R[h], y + h * W);
    if (vec) {
      V4* y4 = reinterpret_cast<V4*>(yp + base);
#pragma unroll
      for (int k = 0; k < HW / 4; ++k)
        y4[k] = IO::from_f4(make_float4(y[4 * k] * zg[4 * k], y[4 * k + 1] * zg[4 * k + 1],
                                        y[4 * k + 2] * zg[4 * k + 2], y[4 * k + 3] * zg[4 * k + 3]));
    } else {
#pragma unroll
      for (int e = 0; e < HW; ++e) yp[base + e] = IO::from_f(y[e] * zg[e]);
    }
  }
}

// ---------------------------------------------------------------------------
// 4 x 4 planes: four lanes per (b, c) plane, lane h holding row h.  Each lane takes its row's
// real DFT; the 4-point column DFTs are two radix-2 stages across the lane quad (DPP quad
// permutes, no LDS), after which lane h holds spectrum row [0, 2, 1, 3][h]; the recurrence
// runs on that row's three bins, the inverse column DFT undoes the stages (lane h back on
// row h) and each lane applies the C2R rule to its row.  Every load and store is one 16-byte
// row per lane: a wave moves 16 whole planes per instruction.
// ---------------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ float2 quad_xch(float2 v) {
  return make_float2(__int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v.x), CTRL, 0xf, 0xf, false)),
                     __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v.y), CTRL, 0xf, 0xf, false)));
}

template <class IO, bool ONE>
__global__ void __launch_bounds__(256) gated_scan_quad4(const ScanArgs a, long long P) {
  using V4 = typename IO::V4;
  using TE = typename IO::T;
  const long long gid = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const long long pl = gid >> 2;
  const int h = int(gid & 3);
  if (pl >= P) return;   // whole quads leave together (P planes = 4 P lanes); no barriers below
  const int T = a.T, C = a.C;
  const int b = int(pl / C), c = int(pl % C);
  const int uo = ((h & 1) << 1) | (h >> 1);   // the spectrum row this lane holds between the stages
  const TE* __restrict__ up = static_cast<const TE*>(a.u);
  const TE* __restrict__ zp = static_cast<const TE*>(a.z);
  TE* __restrict__ yp = static_cast<TE*>(a.y);
  float2 st[ONE ? 1 : 3], kh[ONE ? 1 : 3];
  if constexpr (!ONE) {
    const float2* kp = a.khat + size_t(c) * 12 + uo * 3;
#pragma unroll
    for (int v = 0; v < 3; ++v) {
      kh[v] = kp[v];
      st[v] = make_float2(0.f, 0.f);
    }
  }
  const bool lo1 = (h & 1) == 0, lo2 = h < 2;
  for (int t = 0; t < T; ++t) {
    const size_t base = ((size_t(b) * T + t) * C + c) * 16 + 4 * h;
    const float4 xu = act4(IO::to_f4(*reinterpret_cast<const V4*>(up + base)), a.u_act);
    const float4 g = act4(IO::to_f4(*reinterpret_cast<const V4*>(zp + base)), a.z_act);
    // row DFT of 2 u (the recurrence runs on 2U, as in the other scan kernels)
    const float s02 = 2.0f * (xu.x + xu.z), d02 = 2.0f * (xu.x - xu.z);
    const float s13 = 2.0f * (xu.y + xu.w), d13 = 2.0f * (xu.y - xu.w);
    float2 R[3] = {make_float2(s02 + s13, 0.f), make_float2(d02, -d13), make_float2(s02 - s13, 0.f)};
    const float4* gp = a.gates + (size_t(b) * T + t) * 12 + uo * 3;
#pragma unroll
    for (int v = 0; v < 3; ++v) {
      // forward columns: h, h + 2 (sum on lanes 0, 1; difference on 2, 3), then h, h + 1
      float2 o = quad_xch<0x4e>(R[v]);
      float2 x = lo2 ? make_float2(R[v].x + o.x, R[v].y + o.y) : make_float2(o.x - R[v].x, o.y - R[v].y);
      o = quad_xch<0xb1>(x);
      float2 X;
      if (h == 0) X = make_float2(x.x + o.x, x.y + o.y);            // X0 = a0 + a1
      else if (h == 1) X = make_float2(o.x - x.x, o.y - x.y);       // X2 = a0 - a1
      else if (h == 2) X = make_float2(x.x + o.y, x.y - o.x);       // X1 = s0 - i s1
      else X = make_float2(o.x - x.y, o.y + x.x);                   // X3 = s0 + i s1
      const float4 gg = gp[v];
      if constexpr (ONE) {
        float2 V = make_float2(X.x * gg.y, X.y * gg.y);
        if (V.x * V.x + V.y * V.y < gg.z * gg.z) V = make_float2(gg.z, 0.0f);
        X = make_float2(V.x * gg.w, V.y * gg.w);
      } else {
        X = scan_bin(st[v], X, gg, kh[v]);
      }
      // inverse columns: rows (0, 2), (1, 3) of the spectrum sit on lanes (0, 1), (2, 3)
      o = quad_xch<0xb1>(X);
      x = lo1 ? make_float2(X.x + o.x, X.y + o.y) : make_float2(o.x - X.x, o.y - X.y);
      o = quad_xch<0x4e>(x);
      if (h == 0) R[v] = make_float2(x.x + o.x, x.y + o.y);         // y0 = e0 + e1
      else if (h == 2) R[v] = make_float2(o.x - x.x, o.y - x.y);    // y2 = e0 - e1
      else if (h == 1) R[v] = make_float2(x.x - o.y, x.y + o.x);    // y1 = d0 + i d1
      else R[v] = make_float2(o.x + x.y, o.y - x.x);                // y3 = d0 - i d1
    }
    // C2R of row h (numpy's rule: the middle bin twice, the Nyquist bin once)
    const float z0 = R[0].x, zx1 = 2.0f * R[1].x, zy1 = 2.0f * R[1].y, z2 = R[2].x;
    const float4 y = make_float4(z0 + zx1 + z2, (z0 - z2) - zy1, z0 - zx1 + z2, (z0 - z2) + zy1);
    *reinterpret_cast<V4*>(yp + base) = IO::from_f4(make_float4(y.x * g.x, y.y * g.y, y.z * g.z, y.w * g.w));
  }
}

// ----------------------------------------------------------------- launchers

template <int LH, int LW, int NP, int PPT, class IO>
static hipError_t run_scan(const ScanArgs& a, int B, hipStream_t s) {
  using G = Geom<LH, LW, NP, PPT, true>;
  const long long blocks = (long long)B * a.C / NP;
  hipLaunchKernelGGL((gated_scan_pow2<LH, LW, NP, PPT, IO>), dim3(unsigned(blocks)), dim3(G::NT), 0, s, a);
  return hipGetLastError();
}

// plane-group sizes per plane size, largest first; a variant is usable when it
// divides C (one batch element per workgroup).  The largest group that still
// gives >= 512 workgroups wins; small planes need large groups to fill a
// workgroup with whole waves.
template <int H, class IO>
static hipError_t run_small(const ScanArgs& a, int B, hipStream_t s) {
  using G = SmallGeom<H, H>;
  const long long P = (long long)B * a.C;
  if constexpr (H == 4) {
    // four lanes per plane
    const dim3 grid(unsigned((4 * P + 255) / 256));
    if (a.T == 1)
      hipLaunchKernelGGL((gated_scan_quad4<IO, true>), grid, dim3(256), 0, s, a, P);
    else
      hipLaunchKernelGGL((gated_scan_quad4<IO, false>), grid, dim3(256), 0, s, a, P);
  } else if constexpr (H * H <= 16) {
    // one plane per thread
    const dim3 grid(unsigned((P + 255) / 256));
    if (a.T == 1)
      hipLaunchKernelGGL((gated_scan_plane<H, H, IO, true>), grid, dim3(256), 0, s, a, P);
    else
      hipLaunchKernelGGL((gated_scan_plane<H, H, IO, false>), grid, dim3(256), 0, s, a, P);
  } else {
    const dim3 grid(unsigned((P + G::NP - 1) / G::NP));
    if (a.T == 1)
      hipLaunchKernelGGL((gated_scan_small<H, H, IO, true>), grid, dim3(G::NT), 0, s, a, P);
    else
      hipLaunchKernelGGL((gated_scan_small<H, H, IO, false>), grid, dim3(G::NT), 0, s, a, P);
  }
  return hipGetLastError();
}

template <class IO>
static hipError_t dispatch_scan(const ScanArgs& a, int B, int H, int W, hipStream_t s) {
  if (H == W && (H & (H - 1)) != 0) {
    switch (H) {
      case 3: return run_small<3, IO>(a, B, s);
      case 5: return run_small<5, IO>(a, B, s);
      case 6: return run_small<6, IO>(a, B, s);
      case 7: return run_small<7, IO>(a, B, s);
      case 9: return run_small<9, IO>(a, B, s);
      case 10: return run_small<10, IO>(a, B, s);
      case 11: return run_small<11, IO>(a, B, s);
      case 12: return run_small<12, IO>(a, B, s);
      case 13: return run_small<13, IO>(a, B, s);
      case 14: return run_small<14, IO>(a, B, s);
      case 15: return run_small<15, IO>(a, B, s);
      default: return hipErrorInvalidValue;
    }
  }
  const int C = a.C;
  auto pick = [&](std::initializer_list<int> nps) -> int {
    int best = 0;
    for (int np : nps) {
      if (C % np) continue;
      best = np;
      if ((long long)B * C / np >= 512) return np;
    }
    return best;
  };
#define CSSM_SCAN_CASE(LH, NP_, PPT_) \
  if (np == NP_) return run_scan<LH, LH, NP_, PPT_, IO>(a, B, s);
  if (H == 128 && W == 128) {
    const int np = pick({1});
    CSSM_SCAN_CASE(7, 1, 32)
  } else if (H == 64 && W == 64) {
    const int np = pick({4, 2, 1});
    CSSM_SCAN_CASE(6, 4, 64) CSSM_SCAN_CASE(6, 2, 64) CSSM_SCAN_CASE(6, 1, 64)
  } else if (H == 32 && W == 32) {
    const int np = pick({8, 4, 2});
    CSSM_SCAN_CASE(5, 8, 32) CSSM_SCAN_CASE(5, 4, 32) CSSM_SCAN_CASE(5, 2, 32)
  } else if (H == 16 && W == 16) {
    const int np = pick({16, 8});
    CSSM_SCAN_CASE(4, 16, 32) CSSM_SCAN_CASE(4, 8, 32)
  } else if (H == 8 && W == 8) {
    const int np = pick({32});
    CSSM_SCAN_CASE(3, 32, 32)
    return run_small<8, IO>(a, B, s);        // C not a multiple of 32: direct DFTs
  } else if (H == 4 && W == 4) {
    return run_small<4, IO>(a, B, s);        // direct DFTs beat 128-plane FFT groups here
  }
#undef CSSM_SCAN_CASE
  return hipErrorInvalidValue;
}

bool gated_scan_has_kernel(int H, int W) {
  if (H != W) return false;
  if (H == 4 || H == 8 || H == 16 || H == 32 || H == 64 || H == 128) return true;
  return H >= 3 && H <= 15;   // direct-DFT small-plane kernel
}

int gated_scan_min_group(int H, int W) {
  if (H != W) return 0;
  if (H >= 3 && H <= 15 && H != 16) {
    if ((H & (H - 1)) != 0 || H == 4 || H == 8) return 1;   // direct-DFT kernel: any C
  }
  switch (H) {
    case 128: return 1;
    case 64: return 1;
    case 32: return 2;
    case 16: return 8;
    case 8: return 32;
    case 4: return 128;
    default: return 0;
  }
}

hipError_t launch_gated_scan(const void* u, const void* z, void* y, int dtype, int B, int T, int C, int H,
                             int W, const float4* gates, const float2* khat, int u_act, int z_act,
                             hipStream_t s) {
  ScanArgs a;
  a.u = u;
  a.z = z;
  a.y = y;
  a.gates = gates;
  a.khat = khat;
  a.T = T;
  a.C = C;
  a.u_act = u_act;
  a.z_act = z_act;
  if (dtype == 0) return dispatch_scan<IoF32>(a, B, H, W, s);
  return dispatch_scan<IoBF16>(a, B, H, W, s);
}

}  // namespace cssm
