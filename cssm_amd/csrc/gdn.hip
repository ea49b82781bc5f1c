// GatedDeltaNetCSSM (the `gdn` cell, src/models/cssm.py:4685-5141) on gfx950.
//
// Large planes cannot keep a (batch, head)'s state on one CU: at 128x128 and
// d_k = 4 the 4x4 complex state of every half-spectrum bin is 1.06 MB, against
// 512 KB of VGPRs and 160 KB of LDS per CU.  The spectral core therefore runs
// as three stream-ordered kernels:
//   rfft2_planes     q, k, v planes -> half spectra + per-plane sum |X|^2
//                    (the spectral L2 norms, :4890-4897)
//   gdn_scan_bins    per (b, head, bin): key-vector norm (:4899-4906), the
//                    delta-rule recurrence with the 4x4 state in VGPRs over
//                    all T (:4911-4991), readout o = S q (:4998-5000)
//   irfft2_planes    o spectra -> o planes (:5025, C2R rule)
// plus the prologue kernels (channels-last frame mean for ctx, the gate
// vectors, the qkv depthwise conv, the causal short conv + SiLU + input gates).
// The forward / inverse transforms are the LDS passes of fft_plane.h.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <initializer_list>

#include "dft_small.h"
#include "fft_plane.h"
#include "gdn_step.h"
#include "launch.h"

namespace cssm {

namespace {

__device__ __forceinline__ float ld_f(const float* p, size_t i) { return p[i]; }
__device__ __forceinline__ float ld_f(const uint16_t* p, size_t i) { return bf16_to_f32(p[i]); }
__device__ __forceinline__ float4 ld4v(const float* p, size_t i) { return *reinterpret_cast<const float4*>(p + i); }
__device__ __forceinline__ float4 ld4v(const uint16_t* p, size_t i) {
  const uint2 v = *reinterpret_cast<const uint2*>(p + i);
  return make_float4(bf16_to_f32(v.x & 0xffffu), bf16_to_f32(v.x >> 16), bf16_to_f32(v.y & 0xffffu),
                     bf16_to_f32(v.y >> 16));
}
__device__ __forceinline__ void st_f(float* p, size_t i, float v) { p[i] = v; }
// 4 consecutive elements at a 4-element-aligned index
__device__ __forceinline__ void st4v(float* p, size_t i, float4 v) { *reinterpret_cast<float4*>(p + i) = v; }
__device__ __forceinline__ void st4v(uint16_t* p, size_t i, float4 v) {
  const uint2 u = make_uint2(f32_to_bf16(v.x) | (f32_to_bf16(v.y) << 16), f32_to_bf16(v.z) | (f32_to_bf16(v.w) << 16));
  *reinterpret_cast<uint2*>(p + i) = u;
}
__device__ __forceinline__ void st_f(uint16_t* p, size_t i, float v) { p[i] = uint16_t(f32_to_bf16(v)); }

__device__ __forceinline__ float sigmoid_f(float x) { return 1.0f / (1.0f + expf(-x)); }

}  // namespace

// ---------------------------------------------------------------------------
// Batched 2-D real FFTs of power-of-two planes.
// ---------------------------------------------------------------------------

// forward policy: bins -> HBM spectrum (undoing the pass's factor 2).  The
// sum of |X|^2 per plane is reduced deterministically: every C2 unit pair and
// every edge job leaves its partial in a fixed LDS slot, (pl WH + v) H1/2 + pair
// and pl H/2 + e, summed per plane in a fixed order afterwards.
template <class G>
struct SpecStoreOp {
  static constexpr bool kPackedColumnToo = false;   // bins() writes HBM: only real columns
  static constexpr int H = G::H, WH = G::WH, WF = G::WF, H1 = G::H1, H2 = G::H2, HP = G::HP;
  float2* out;      // (NP, H, WF) of this workgroup
  float* part_c2;   // LDS (NC2) or nullptr: partial sums of the C2 jobs
  float* part_e;    // LDS (NE) or nullptr: partial sums of the edge jobs
  int nvalid;       // planes of the group that exist (the last group may be partial)

  __device__ __forceinline__ void bins(int, int a2, int pl, int k, int v, float2 (&sp)[G::H2]) const {
    float s = 0.0f;
    if (pl < nvalid) {
#pragma unroll
      for (int q = 0; q < H2; ++q) {
        const float2 x = make_float2(0.5f * sp[q].x, 0.5f * sp[q].y);
        out[size_t(pl * H + k + H1 * q) * WF + v] = x;
        s = fmaf(x.x, x.x, fmaf(x.y, x.y, s));
      }
    }
    if (part_c2) {
      // unit a2 = 0 is kA = pair, a2 = 1 is kB = -pair mod H1 (H1/2 for pair 0)
      const int pair = a2 == 0 ? k : (k == H1 / 2 ? 0 : H1 - k);
      float& slot = part_c2[(pl * WH + v) * (H1 / 2) + pair];
      slot = a2 ? slot + s : s;
    }
  }
  __device__ __forceinline__ void edge(int, int pl, int uA, int uB, int e, float2 (&v4)[4]) const {
    float s = 0.0f;
    if (pl < nvalid) {
      const int idx[4] = {uA * WF, uA * WF + WH, uB * WF, uB * WF + WH};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float2 x = make_float2(0.5f * v4[i].x, 0.5f * v4[i].y);
        out[size_t(pl * H) * WF + idx[i]] = x;
        s = fmaf(x.x, x.x, fmaf(x.y, x.y, s));
      }
    }
    if (part_e) part_e[pl * HP + e] = s;
  }
};

// inverse policy: bins <- HBM spectrum / (H W)
template <class G>
struct SpecLoadOp {
  static constexpr bool kPackedColumnToo = false;   // bins() writes HBM: only real columns
  static constexpr int H = G::H, WH = G::WH, WF = G::WF, H1 = G::H1, H2 = G::H2;
  const float2* in;   // (NP, H, WF) of this workgroup
  float scale;        // 1 / (H W)
  int nvalid;         // planes of the group that exist; the others transform zeros

  __device__ __forceinline__ void bins(int, int, int pl, int k, int v, float2 (&sp)[G::H2]) const {
    const bool ok = pl < nvalid;
#pragma unroll
    for (int q = 0; q < H2; ++q) {
      const float2 x = ok ? in[size_t(pl * H + k + H1 * q) * WF + v] : make_float2(0.f, 0.f);
      sp[q] = make_float2(x.x * scale, x.y * scale);
    }
  }
  __device__ __forceinline__ void edge(int, int pl, int uA, int uB, int, float2 (&v4)[4]) const {
    const bool ok = pl < nvalid;
    const int idx[4] = {uA * WF, uA * WF + WH, uB * WF, uB * WF + WH};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float2 x = ok ? in[size_t(pl * H) * WF + idx[i]] : make_float2(0.f, 0.f);
      v4[i] = make_float2(x.x * scale, x.y * scale);
    }
  }
};

// Which plane groups the transforms run persistently (a workgroup per resident slot looping over
// groups, the next group's loads issued during the current one's passes): where a wave's rows lie in
// one plane (V4_LINEAR).  Forward only for one plane per group (128 x 128): at 64 x 64 the
// persistent forward measured slower than one group per workgroup.
constexpr bool fwd_persistent(bool v4_linear, int np) { return v4_linear && np == 1; }
constexpr bool inv_persistent(bool v4_linear) { return v4_linear; }

// waves per SIMD the inverse kernels must keep: two 512-thread workgroups of 128 x 128 planes share
// a CU (LDS), i.e. four waves per SIMD, which caps a wave at 128 VGPRs with the prefetched bins
template <int LH, int PPT>
constexpr int kInvWavesPerSimd = (LH == 7 && PPT == 32) ? 4 : 1;

// inverse policy with the group's interior bins already in registers: SpecBins::fetch loads, for
// the lane's C2 units (the job map the pass uses), every bin SpecLoadOp::bins would read, so a
// persistent inverse issues the next group's loads while the current group's later passes run.
// The DC / Nyquist columns (one wave's edge jobs) are read from HBM in the edge pass.
template <class G>
struct SpecBins {
  static constexpr int H = G::H, WF = G::WF, H1 = G::H1, H2 = G::H2;
  float2 c[G::JC2][2][H2];   // C2 unit (j, a2): its H2 bins
  // group spectrum `in` of nv valid planes (the rest read as 0); lane l of wave w
  __device__ __forceinline__ void fetch(const float2* in, int nv, int w, int l) {
    const Buf src(in, unsigned(nv) * unsigned(H * WF * 8));
#pragma unroll
    for (int j = 0; j < G::JC2; ++j) {
      int pl, v, pair, n;
      G::col_job(w, j, l, pl, v, pair, n);
      int kA, kB;
      pair_units<H1>(pair, kA, kB);
#pragma unroll
      for (int a2 = 0; a2 < 2; ++a2) {
        const int k = a2 ? kB : kA;
        const unsigned vo = unsigned(((pl * H + k) * WF + n) * 8);
#pragma unroll
        for (int q = 0; q < H2; ++q) c[j][a2][q] = src.ld2(vo, q * H1 * WF * 8);
      }
    }
  }
};

template <class G>
struct SpecRegOp {
  static constexpr bool kPackedColumnToo = false;
  static constexpr int H2 = G::H2;
  const SpecBins<G>& b;
  SpecLoadOp<G> edges_from;   // the group's spectrum, for the edge pass
  __device__ __forceinline__ void bins(int j, int a2, int, int, int, float2 (&sp)[G::H2]) const {
    const float scale = edges_from.scale;
#pragma unroll
    for (int q = 0; q < H2; ++q) sp[q] = make_float2(b.c[j][a2][q].x * scale, b.c[j][a2][q].y * scale);
  }
  __device__ __forceinline__ void edge(int j, int pl, int uA, int uB, int e, float2 (&v4)[4]) const {
    edges_from.edge(j, pl, uA, uB, e, v4);
  }
};

// inverse policy of the persistent 128 x 128 inverse: interior bins from SpecBins, the DC / Nyquist columns
// from an LDS stage est[(pl H + u) 2 + (v ? 1 : 0)] that holds them already scaled (see irfft2_planes)
template <class G>
struct SpecRegEdgeOp {
  static constexpr bool kPackedColumnToo = false;
  static constexpr int H = G::H, H2 = G::H2;
  const SpecBins<G>& b;
  float scale;
  const float2* est;
  __device__ __forceinline__ void bins(int j, int a2, int, int, int, float2 (&sp)[G::H2]) const {
#pragma unroll
    for (int q = 0; q < H2; ++q) sp[q] = make_float2(b.c[j][a2][q].x * scale, b.c[j][a2][q].y * scale);
  }
  __device__ __forceinline__ void edge(int, int pl, int uA, int uB, int, float2 (&v4)[4]) const {
    v4[0] = est[(pl * H + uA) * 2];
    v4[1] = est[(pl * H + uA) * 2 + 1];
    v4[2] = est[(pl * H + uB) * 2];
    v4[3] = est[(pl * H + uB) * 2 + 1];
  }
};

// rfft2 of NP planes per group: x (P, H, W) real -> spec (P, H, WF), norms (P) = sum |X|^2 or skipped.
// The last group may hold fewer than NP planes: the missing ones are neither read nor written.
// Persistent: workgroup b transforms groups b, b + gridDim.x, ...  Where a wave's rows lie in one
// plane (V4_LINEAR) it loads the next group's planes into registers while the current group's passes
// run, so a CU's HBM reads do not stop for the transforms; each wave's loads are buffer loads off
// its plane's base with one per-lane offset and uniform row steps.
template <int LH, int LW, int NP, int PPT, class IO>
__global__ void __launch_bounds__((NP << (LH + LW)) / PPT)
rfft2_planes(const void* __restrict__ x, long long P, float2* __restrict__ spec, float* __restrict__ norms) {
  using G = Geom<LH, LW, NP, PPT>;
  constexpr int H = G::H, W = G::W, WF = G::WF, NT = G::NT;
  using V4 = typename IO::V4;
  using TE = typename IO::T;
  constexpr int UC2 = G::NC2 / NP, UE = G::NE / NP;     // C2 / edge jobs per plane
  constexpr int GR = NT / NP > 0 ? NT / NP : 1;          // reducing threads per plane
  __shared__ __attribute__((aligned(16))) float smem[G::LDS_FLOATS];
  __shared__ float part_c2[G::NC2], part_e[G::NE], red[NT];
  const PlaneFft<G> fft(smem);
  const unsigned tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(int(tid) / 64), l = int(tid) % 64;
  const long long NG = (P + NP - 1) / NP;
  fft.init_twiddles(tid);
  // C2 jobs on the packed DC / Nyquist column (v = 0) never reach the policy: their slots stay 0
  for (int i = tid; i < G::NC2; i += NT) part_c2[i] = 0.0f;
  __syncthreads();
  const auto m = G::v4_lane(l);
  const auto col = PlaneFft<G>::v4_col(m.c4);
  constexpr bool PF = fwd_persistent(G::V4_LINEAR, NP);
  V4 ld[G::JLD];
  auto load = [&](long long g) {
    const size_t q0 = size_t(g) * NP;
    const int nv = int(P - (long long)q0 < NP ? P - (long long)q0 : NP);
    if constexpr (PF) {
      constexpr int VB = int(sizeof(V4));
      const int pw = (w * G::RPW) / G::HP;   // this wave's plane in the group
      const Buf src(static_cast<const TE*>(x) + (q0 + pw) * H * W, pw < nv ? unsigned(H * W * sizeof(TE)) : 0u);
      const unsigned vo = unsigned(((G::v4_row(w, 0, m) - pw * H) * G::C4N + m.c4) * VB);
#pragma unroll
      for (int i = 0; i < G::JLD; ++i) src.ld(ld[i], vo, i * G::RK * G::C4N * VB);
    } else {
      const unsigned nv4 = unsigned(nv) * (H * W / 4);
      const V4* src = reinterpret_cast<const V4*>(static_cast<const TE*>(x) + q0 * H * W);
#pragma unroll
      for (int i = 0; i < G::JLD; ++i) {
        const unsigned f = G::v4_index(G::v4_row(w, i, m), m);
        ld[i] = f < nv4 ? src[f] : V4{};
      }
    }
  };
  auto group = [&](long long g) {
    const size_t p0 = size_t(g) * NP;
    const int nvalid = int(P - (long long)p0 < NP ? P - (long long)p0 : NP);
    if (!PF) load(g);
#pragma unroll
    for (int i = 0; i < G::JLD; ++i) fft.v4_put(G::v4_row(w, i, m), col, IO::to_f4(ld[i]));
    wave_sync();
    if (PF && g + gridDim.x < NG) load(g + gridDim.x);
    // the lane index re-derived per group, so the passes rebuild their (cheap) LDS addresses instead
    // of the compiler holding every pass's addresses in registers across the loop
    int ll = l;
    asm volatile("" : "+v"(ll));
    __builtin_assume(ll >= 0 && ll < 64);
    SpecStoreOp<G> op{spec + p0 * H * WF, norms ? part_c2 : nullptr, norms ? part_e : nullptr, nvalid};
    fft.r1(w, ll);
    fft.r2(w, ll);
    fft.c1(w, ll);
    fft.template c2<true, false>(w, ll, op);
    fft.template edges<true, false>(w, ll, op);
    __syncthreads();   // the passes are done with the plane buffer (and the norms' slots are written)
    if (norms) {
      // plane pl: GR threads each sum a fixed stride of its UC2 + UE slots, then one sums those in order
      for (int pl0 = 0; pl0 < NP; pl0 += NT / GR) {
        const int pl = pl0 + int(tid) / GR, r = int(tid) % GR;
        float acc = 0.0f;
        if (pl < NP) {
          for (int i = r; i < UC2; i += GR) acc += part_c2[pl * UC2 + i];
          for (int i = r; i < UE; i += GR) acc += part_e[pl * UE + i];
        }
        red[tid] = acc;
        __syncthreads();
        if (r == 0 && pl < nvalid) {
          float sum = 0.0f;
          for (int i = 0; i < GR; ++i) sum += red[tid + i];
          norms[p0 + pl] = sum;
        }
        __syncthreads();
      }
    }
  };
  if constexpr (PF) {
    long long g = blockIdx.x;
    if (g < NG) load(g);
    for (; g < NG; g += gridDim.x) group(g);
  } else {
    group(blockIdx.x);
  }
}

// irfft2 of NP planes per group: spec (P, H, WF) -> y (P, H, W) real (numpy C2R rule);
// a partial last group neither reads nor writes the missing planes.
// Persistent like rfft2_planes: with V4_LINEAR the next group's bins are loaded into registers
// (SpecBins) as soon as the current group's C2 / edge passes have taken theirs, and land while
// the remaining passes and the stores run.
template <int LH, int LW, int NP, int PPT, class IO>
__global__ void __launch_bounds__((NP << (LH + LW)) / PPT, (kInvWavesPerSimd<LH, PPT>))
irfft2_planes(const float2* __restrict__ spec, long long P, void* __restrict__ y) {
  using G = Geom<LH, LW, NP, PPT>;
  constexpr int H = G::H, W = G::W, WF = G::WF;
  constexpr bool PF = inv_persistent(G::V4_LINEAR);
  using V4 = typename IO::V4;
  using TE = typename IO::T;
  __shared__ __attribute__((aligned(16))) float smem[G::LDS_FLOATS];
  const PlaneFft<G> fft(smem);
  const unsigned tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(int(tid) / 64), l = int(tid) % 64;
  const long long NG = (P + NP - 1) / NP;
  const float scale = 1.0f / float(H * W);
  auto nvalid_of = [&](long long g) { return int(P - g * NP < NP ? P - g * NP : NP); };
  // 128 x 128: the next group's DC / Nyquist columns (u, 0) and (u, W/2), 2 H NP values, are loaded one per
  // lane after the current group's I2 pass and staged (scaled) in LDS at its end. Read in the edge pass
  // instead, a group after their lines came through L2 with the interior bins, they were fetched from HBM
  // again (issued with the interior bins, the extra VGPRs cost what the saved traffic gained).
  constexpr bool EST = PF && LH == 7;
  constexpr int NEV = 2 * H * NP;
  static_assert(!EST || NEV <= G::NT, "one staged DC / Nyquist value per lane");
  __shared__ float2 estage[EST ? NEV : 1];
  float2 ev = make_float2(0.f, 0.f);
  auto fetch_edge = [&](long long g) {
    if constexpr (EST) {
      const int e = int(tid);
      if (e < NEV) {
        const int pl = e / (2 * H), u = (e >> 1) % H;
        ev = pl < nvalid_of(g) ? spec[(size_t(g) * NP + pl) * H * WF + size_t(u) * WF + ((e & 1) ? WF - 1 : 0)]
                               : make_float2(0.f, 0.f);
      }
    }
  };
  auto stage_edge = [&]() {
    if constexpr (EST) {
      if (int(tid) < NEV) estage[tid] = make_float2(ev.x * scale, ev.y * scale);
    }
  };
  fft.init_twiddles(tid);
  if constexpr (EST) {
    if ((long long)blockIdx.x < NG) {
      fetch_edge(blockIdx.x);
      stage_edge();
    }
  }
  __syncthreads();
  const auto m = G::v4_lane(l);
  const auto col = PlaneFft<G>::v4_col(m.c4);
  SpecBins<G> bins;
  auto group = [&](long long g) {
    const size_t p0 = size_t(g) * NP;
    const int nvalid = nvalid_of(g);
    const unsigned nv4 = unsigned(nvalid) * (H * W / 4);
    int ll = l;   // re-derived per group, as in rfft2_planes
    asm volatile("" : "+v"(ll));
    __builtin_assume(ll >= 0 && ll < 64);
    if constexpr (EST) {
      const SpecRegEdgeOp<G> op{bins, scale, estage};
      fft.template c2<false, true>(w, ll, op);
      if (g + gridDim.x < NG) {
        bins.fetch(spec + (g + gridDim.x) * NP * H * WF, nvalid_of(g + gridDim.x), w, l);
      }
      fft.template edges<false, true>(w, ll, op);
    } else if constexpr (PF) {
      const SpecRegOp<G> op{bins, SpecLoadOp<G>{spec + p0 * H * WF, scale, nvalid}};
      fft.template c2<false, true>(w, ll, op);
      if (g + gridDim.x < NG) bins.fetch(spec + (g + gridDim.x) * NP * H * WF, nvalid_of(g + gridDim.x), w, l);
      fft.template edges<false, true>(w, ll, op);
    } else {
      SpecLoadOp<G> op{spec + p0 * H * WF, scale, nvalid};
      fft.template c2<false, true>(w, ll, op);
      fft.template edges<false, true>(w, ll, op);
    }
    fft.i1_packed(w, ll);
    fft.i2(w, ll);
    if (g + gridDim.x < NG) fetch_edge(g + gridDim.x);
    fft.i3(w, ll);
    fft.i4(w, ll);
    V4* dst = reinterpret_cast<V4*>(static_cast<TE*>(y) + p0 * H * W);
#pragma unroll
    for (int i = 0; i < G::JLD; ++i) {
      const int row = G::v4_row(w, i, m);
      const unsigned f = G::v4_index(row, m);
      if (f < nv4) dst[f] = IO::from_f4(fft.v4_get(row, col));
    }
    // the next group's DC / Nyquist columns (the edge pass, the only reader, finished before the I2 -> I3
    // barrier); the last group stages values no group reads
    stage_edge();
    __syncthreads();   // the stores have read the plane buffer before the next group's C2 writes it
  };
  if constexpr (PF) {
    long long g = blockIdx.x;
    if (g < NG) bins.fetch(spec + g * NP * H * WF, nvalid_of(g), w, l);
    for (; g < NG; g += gridDim.x) group(g);
  } else {
    group(blockIdx.x);
  }
}

namespace {

// plane group of the table (largest first): the largest that still gives >= 512 workgroups, else the smallest
int pick_group(long long P, std::initializer_list<int> nps) {
  int best = 0;
  for (int np : nps) {
    best = np;
    if ((P + np - 1) / np >= 512) return np;
  }
  return best;
}

// workgroups of a persistent launch over `groups` units: what fits on the device at once
unsigned resident_grid(const void* kernel, int nt, long long groups) {
  int dev = 0, cus = 256, per_cu = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) !=
                                              hipSuccess)
    cus = 256;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, nt, 0) != hipSuccess || per_cu < 1) per_cu = 1;
  const long long cap = (long long)cus * per_cu;
  return unsigned(groups < cap ? groups : cap);
}

template <int LH, int NP, int PPT, class IO>
hipError_t run_fwd(const void* x, long long P, float2* spec, float* norms, hipStream_t s) {
  using G = Geom<LH, LH, NP, PPT>;
  const auto k = rfft2_planes<LH, LH, NP, PPT, IO>;
  // persistent kernels: as many workgroups as fit at once; the others one per group
  static const unsigned grid = fwd_persistent(G::V4_LINEAR, NP) ? resident_grid(reinterpret_cast<const void*>(k), G::NT, 1LL << 40) : ~0u;
  const long long groups = (P + NP - 1) / NP;
  hipLaunchKernelGGL(k, dim3(unsigned(groups < grid ? groups : grid)), dim3(G::NT), 0, s, x, P, spec, norms);
  return hipGetLastError();
}

template <int LH, int NP, int PPT, class IO>
hipError_t run_inv(const float2* spec, long long P, void* y, hipStream_t s) {
  using G = Geom<LH, LH, NP, PPT>;
  const auto k = irfft2_planes<LH, LH, NP, PPT, IO>;
  // persistent kernels: as many workgroups as fit at once; the others one per group
  static const unsigned grid = inv_persistent(G::V4_LINEAR) ? resident_grid(reinterpret_cast<const void*>(k), G::NT, 1LL << 40) : ~0u;
  const long long groups = (P + NP - 1) / NP;
  hipLaunchKernelGGL(k, dim3(unsigned(groups < grid ? groups : grid)), dim3(G::NT), 0, s, spec, P, y);
  return hipGetLastError();
}

// the plane groups of the fused gated scan, per plane size
// (PPT128: samples per thread at 128 x 128; 64 = 256 threads, 32 = 512 threads)
#define CSSM_FFT_TABLE(CASE, PPT128)                                                \
  if (H == 128) {                                                                   \
    const int np = pick_group(P, {1});                                              \
    CASE(7, 1, PPT128)                                                              \
  } else if (H == 64) {                                                             \
    const int np = pick_group(P, {4, 2, 1});                                        \
    CASE(6, 4, 64) CASE(6, 2, 64) CASE(6, 1, 64)                                    \
  } else if (H == 32) {                                                             \
    const int np = pick_group(P, {8, 4, 2});                                        \
    CASE(5, 8, 32) CASE(5, 4, 32) CASE(5, 2, 32)                                    \
  } else if (H == 16) {                                                             \
    const int np = pick_group(P, {16, 8});                                          \
    CASE(4, 16, 32) CASE(4, 8, 32)                                                  \
  } else if (H == 8) {                                                              \
    const int np = pick_group(P, {32});                                             \
    CASE(3, 32, 32)                                                                 \
  } else if (H == 4) {                                                              \
    const int np = pick_group(P, {128});                                            \
    CASE(2, 128, 32)                                                                \
  }

template <class IO>
hipError_t dispatch_fwd(const void* x, long long P, int H, float2* spec, float* norms, hipStream_t s) {
#define CSSM_FWD_CASE(LH, NP_, PPT_) \
  if (np == NP_) return run_fwd<LH, NP_, PPT_, IO>(x, P, spec, norms, s);
  CSSM_FFT_TABLE(CSSM_FWD_CASE, 64)
#undef CSSM_FWD_CASE
  return hipErrorInvalidValue;
}

template <class IO>
hipError_t dispatch_inv(const float2* spec, long long P, int H, void* y, hipStream_t s) {
#define CSSM_INV_CASE(LH, NP_, PPT_) \
  if (np == NP_) return run_inv<LH, NP_, PPT_, IO>(spec, P, y, s);
  CSSM_FFT_TABLE(CSSM_INV_CASE, 32)
#undef CSSM_INV_CASE
  return hipErrorInvalidValue;
}

}  // namespace

// power-of-two planes 4..128, any plane count (a partial last group is masked)
// ---------------------------------------------------------------------------
// Batched 2-D real FFTs of small planes that are not powers of two (H = W in
// 3..15: the 14 x 14 and 7 x 7 CSSM-SHViT stages) by direct DFTs with
// compile-time twiddles (dft_small.h): rows R2C, then one thread per column
// (plane, v) for the column DFT; the inverse runs the column DFTs first, then
// numpy's C2R rule per row.  A workgroup transforms NP consecutive planes.
template <int H, class IO>
__global__ void __launch_bounds__((SmallGeom<H, H>::NT))
rfft2_small(const void* xv, long long P, float2* __restrict__ spec, float* __restrict__ norms) {
  using G = SmallGeom<H, H>;
  constexpr int W = H, WF = G::WF, HW = G::HW, NT = G::NT, NP = G::NP;
  __shared__ float xs[NP * HW];
  __shared__ float2 rs[NP * G::PS];
  __shared__ float cn[NP * WF];                      // per column sum |X|^2
  const typename IO::T* __restrict__ x = static_cast<const typename IO::T*>(xv);
  const int tid = int(threadIdx.x);
  const long long p0 = (long long)blockIdx.x * NP;
  const int np = int(P - p0 < NP ? P - p0 : NP);
  for (int e = tid; e < np * HW; e += NT) xs[e] = IO::to_f(x[size_t(p0) * HW + e]);
  __syncthreads();
  for (int j = tid; j < np * H; j += NT) small_row_r2c<W>(xs + j * W, rs + (j / H) * G::PS + (j % H) * G::RSP);
  __syncthreads();
  const int cpl = tid / WF, cv = tid % WF;
  if (tid < G::NCJ && cpl < np) {
    float2 r[H], X[H];
#pragma unroll
    for (int h = 0; h < H; ++h) r[h] = rs[cpl * G::PS + h * G::RSP + cv];
    dft_sym<H, false>(r, X);
    float2* out = spec + size_t(p0 + cpl) * (H * WF) + cv;
    float acc = 0.0f;
#pragma unroll
    for (int u = 0; u < H; ++u) {
      out[u * WF] = X[u];
      acc = fmaf(X[u].x, X[u].x, fmaf(X[u].y, X[u].y, acc));
    }
    cn[cpl * WF + cv] = acc;
  }
  if (norms) {
    __syncthreads();
    if (tid < np) {
      float sum = 0.0f;
#pragma unroll
      for (int v = 0; v < WF; ++v) sum += cn[tid * WF + v];
      norms[p0 + tid] = sum;
    }
  }
}

template <int H, class IO>
__global__ void __launch_bounds__((SmallGeom<H, H>::NT))
irfft2_small(const float2* __restrict__ spec, long long P, void* yv) {
  using G = SmallGeom<H, H>;
  constexpr int W = H, WF = G::WF, HW = G::HW, NT = G::NT, NP = G::NP;
  __shared__ float xs[NP * HW];
  __shared__ float2 rs[NP * G::PS];
  typename IO::T* __restrict__ y = static_cast<typename IO::T*>(yv);
  const int tid = int(threadIdx.x);
  const long long p0 = (long long)blockIdx.x * NP;
  const int np = int(P - p0 < NP ? P - p0 : NP);
  for (int e = tid; e < np * H * WF; e += NT) {
    const int pl = e / (H * WF), r = e % (H * WF);
    rs[pl * G::PS + (r / WF) * G::RSP + r % WF] = spec[size_t(p0) * (H * WF) + e];
  }
  __syncthreads();
  const int cpl = tid / WF, cv = tid % WF;
  if (tid < G::NCJ && cpl < np) {
    float2 r[H], Z[H];
#pragma unroll
    for (int u = 0; u < H; ++u) r[u] = rs[cpl * G::PS + u * G::RSP + cv];
    dft_sym<H, true>(r, Z);
    constexpr float inv = 1.0f / float(HW);
#pragma unroll
    for (int h = 0; h < H; ++h) rs[cpl * G::PS + h * G::RSP + cv] = cscale(Z[h], inv);
  }
  __syncthreads();
  for (int j = tid; j < np * H; j += NT) small_row_c2r<W>(rs + (j / H) * G::PS + (j % H) * G::RSP, xs + j * W);
  __syncthreads();
  for (int e = tid; e < np * HW; e += NT) y[size_t(p0) * HW + e] = IO::from_f(xs[e]);
}

template <class IO>
static hipError_t small_fwd(const void* x, long long P, int H, float2* spec, float* norms, hipStream_t s) {
#define CSSM_SMALL_FWD(N)                                                                                  \
  case N:                                                                                                  \
    hipLaunchKernelGGL((rfft2_small<N, IO>), dim3(unsigned((P + SmallGeom<N, N>::NP - 1) / SmallGeom<N, N>::NP)), \
                       dim3(SmallGeom<N, N>::NT), 0, s, x, P, spec, norms);                                \
    break;
  switch (H) {
    CSSM_SMALL_FWD(3) CSSM_SMALL_FWD(5) CSSM_SMALL_FWD(6) CSSM_SMALL_FWD(7) CSSM_SMALL_FWD(9) CSSM_SMALL_FWD(10)
    CSSM_SMALL_FWD(11) CSSM_SMALL_FWD(12) CSSM_SMALL_FWD(13) CSSM_SMALL_FWD(14) CSSM_SMALL_FWD(15)
    default: return hipErrorInvalidValue;
  }
#undef CSSM_SMALL_FWD
  return hipGetLastError();
}

template <class IO>
static hipError_t small_inv(const float2* spec, long long P, int H, void* y, hipStream_t s) {
#define CSSM_SMALL_INV(N)                                                                                  \
  case N:                                                                                                  \
    hipLaunchKernelGGL((irfft2_small<N, IO>), dim3(unsigned((P + SmallGeom<N, N>::NP - 1) / SmallGeom<N, N>::NP)), \
                       dim3(SmallGeom<N, N>::NT), 0, s, spec, P, y);                                       \
    break;
  switch (H) {
    CSSM_SMALL_INV(3) CSSM_SMALL_INV(5) CSSM_SMALL_INV(6) CSSM_SMALL_INV(7) CSSM_SMALL_INV(9) CSSM_SMALL_INV(10)
    CSSM_SMALL_INV(11) CSSM_SMALL_INV(12) CSSM_SMALL_INV(13) CSSM_SMALL_INV(14) CSSM_SMALL_INV(15)
    default: return hipErrorInvalidValue;
  }
#undef CSSM_SMALL_INV
  return hipGetLastError();
}

static bool small_plane(int H, int W) { return H == W && H >= 3 && H <= 15 && (H & (H - 1)) != 0; }

int fft_planes_min_group(int H, int W) {
  return ((H == W && H >= 4 && H <= 128 && (H & (H - 1)) == 0) || small_plane(H, W)) ? 1 : 0;
}

hipError_t launch_rfft2(const void* x, int dtype, long long P, int H, int W, float2* spec, float* norms,
                        hipStream_t s) {
  if (H != W) return hipErrorInvalidValue;
  if (small_plane(H, W))
    return dtype == 0 ? small_fwd<IoF32>(x, P, H, spec, norms, s) : small_fwd<IoBF16>(x, P, H, spec, norms, s);
  return dtype == 0 ? dispatch_fwd<IoF32>(x, P, H, spec, norms, s) : dispatch_fwd<IoBF16>(x, P, H, spec, norms, s);
}

hipError_t launch_irfft2(const float2* spec, long long P, int H, int W, void* y, int dtype, hipStream_t s) {
  if (H != W) return hipErrorInvalidValue;
  if (small_plane(H, W))
    return dtype == 0 ? small_inv<IoF32>(spec, P, H, y, s) : small_inv<IoBF16>(spec, P, H, y, s);
  return dtype == 0 ? dispatch_inv<IoF32>(spec, P, H, y, s) : dispatch_inv<IoBF16>(spec, P, H, y, s);
}

// ---------------------------------------------------------------------------
// The transforms of the gated cell's training backward with the elementwise
// work around them fused into their load / store phases, on float32 planes
// addressed as a strided set: plane p = f C + c of a set (ptr, fs) starts at
// ptr + (f fs + c) H W, so the halves of a plane-major (F, 2C, HW) tensor are
// sets with fs = 2C.
//   rfft2_ex   spec = rfft2(act_x(x) [* act_a(a)])        (act: identity or SiLU)
//   irfft2_ex  y = (irfft2(spec) + add[p]) [* m] [* SiLU'(d)]
// SiLU'(v) = s (1 + v (1 - s)), s = sigmoid(v).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float silu1(float v) { return v * __builtin_amdgcn_rcpf(1.0f + __expf(-v)); }
__device__ __forceinline__ float dsilu1(float v) {
  const float s = __builtin_amdgcn_rcpf(1.0f + __expf(-v));
  return s * fmaf(v, 1.0f - s, 1.0f);
}

// persistent like rfft2_planes (with V4_LINEAR the next group's x and a are in flight during the
// current passes); the activations and product are applied as the samples go into LDS
template <int LH, int LW, int NP, int PPT>
__global__ void __launch_bounds__((NP << (LH + LW)) / PPT)
rfft2_planes_ex(const FftEx e, long long P, float2* __restrict__ spec) {
  using G = Geom<LH, LW, NP, PPT>;
  constexpr int H = G::H, W = G::W, WF = G::WF, V4P = H * W / 4;
  __shared__ __attribute__((aligned(16))) float smem[G::LDS_FLOATS];
  const PlaneFft<G> fft(smem);
  const unsigned tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(int(tid) / 64), l = int(tid) % 64;
  const long long NG = (P + NP - 1) / NP;
  fft.init_twiddles(tid);
  __syncthreads();
  const auto m = G::v4_lane(l);
  const auto col = PlaneFft<G>::v4_col(m.c4);
  constexpr bool PF = fwd_persistent(G::V4_LINEAR, NP);
  float4 lx[G::JLD], la[G::JLD];
  const bool two = e.a.p != nullptr;
  auto load = [&](long long g) {
    const long long q0 = g * NP;
    const int nv = int(P - q0 < NP ? P - q0 : NP);
    if constexpr (PF) {
      const int pw = (w * G::RPW) / G::HP;   // this wave's plane in the group
      const unsigned bytes = pw < nv ? unsigned(H * W * sizeof(float)) : 0u;
      const long long pp = pw < nv ? q0 + pw : q0;
      const Buf sx(e.x.p + e.x.off(pp, e.C, H * W), bytes);
      const unsigned vo = unsigned(((G::v4_row(w, 0, m) - pw * H) * G::C4N + m.c4) * 16);
#pragma unroll
      for (int i = 0; i < G::JLD; ++i) sx.ld(lx[i], vo, i * G::RK * G::C4N * 16);
      if (two) {
        const Buf sa(e.a.p + e.a.off(pp, e.C, H * W), bytes);
#pragma unroll
        for (int i = 0; i < G::JLD; ++i) sa.ld(la[i], vo, i * G::RK * G::C4N * 16);
      }
    } else {
#pragma unroll
      for (int i = 0; i < G::JLD; ++i) {
        const unsigned f = G::v4_index(G::v4_row(w, i, m), m);
        const int pl = int(f / V4P), q = int(f % V4P);
        lx[i] = la[i] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (pl < nv) {
          lx[i] = *reinterpret_cast<const float4*>(e.x.p + e.x.off(q0 + pl, e.C, H * W) + 4 * q);
          if (two) la[i] = *reinterpret_cast<const float4*>(e.a.p + e.a.off(q0 + pl, e.C, H * W) + 4 * q);
        }
      }
    }
  };
  auto group = [&](long long g) {
    const long long p0 = g * NP;
    const int nvalid = int(P - p0 < NP ? P - p0 : NP);
    if (!PF) load(g);
#pragma unroll
    for (int i = 0; i < G::JLD; ++i) {
      float4 v = lx[i];
      if (e.x_act) v = make_float4(silu1(v.x), silu1(v.y), silu1(v.z), silu1(v.w));
      if (two) {
        float4 u = la[i];
        if (e.a_act) u = make_float4(silu1(u.x), silu1(u.y), silu1(u.z), silu1(u.w));
        v = make_float4(v.x * u.x, v.y * u.y, v.z * u.z, v.w * u.w);
      }
      fft.v4_put(G::v4_row(w, i, m), col, v);
    }
    wave_sync();
    if (PF && g + gridDim.x < NG) load(g + gridDim.x);
    int ll = l;   // re-derived per group, as in rfft2_planes
    asm volatile("" : "+v"(ll));
    __builtin_assume(ll >= 0 && ll < 64);
    SpecStoreOp<G> op{spec + p0 * H * WF, nullptr, nullptr, nvalid};
    fft.r1(w, ll);
    fft.r2(w, ll);
    fft.c1(w, ll);
    fft.template c2<true, false>(w, ll, op);
    fft.template edges<true, false>(w, ll, op);
    __syncthreads();   // the passes are done with the plane buffer
  };
  if constexpr (PF) {
    long long g = blockIdx.x;
    if (g < NG) load(g);
    for (; g < NG; g += gridDim.x) group(g);
  } else {
    group(blockIdx.x);
  }
}

// persistent like irfft2_planes
template <int LH, int LW, int NP, int PPT>
__global__ void __launch_bounds__((NP << (LH + LW)) / PPT, (kInvWavesPerSimd<LH, PPT>))
irfft2_planes_ex(const float2* __restrict__ spec, long long P, const FftEx e) {
  using G = Geom<LH, LW, NP, PPT>;
  constexpr int H = G::H, W = G::W, WF = G::WF, V4P = H * W / 4;
  constexpr bool PF = inv_persistent(G::V4_LINEAR);
  __shared__ __attribute__((aligned(16))) float smem[G::LDS_FLOATS];
  __shared__ float wsum[G::NW];
  const PlaneFft<G> fft(smem);
  const unsigned tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(int(tid) / 64), l = int(tid) % 64;
  const long long NG = (P + NP - 1) / NP;
  const float scale = 1.0f / float(H * W);
  fft.init_twiddles(tid);
  __syncthreads();
  const auto m = G::v4_lane(l);
  const auto col = PlaneFft<G>::v4_col(m.c4);
  const PlaneSet ys{e.y, e.y_fs};
  auto nvalid_of = [&](long long g) { return int(P - g * NP < NP ? P - g * NP : NP); };
  auto group = [&](long long g) {
    const long long p0 = g * NP;
    const int nvalid = nvalid_of(g);
    int ll = l;   // re-derived per group, as in rfft2_planes
    asm volatile("" : "+v"(ll));
    __builtin_assume(ll >= 0 && ll < 64);
    {
      SpecLoadOp<G> op{spec + p0 * H * WF, scale, nvalid};
      fft.template c2<false, true>(w, ll, op);
      fft.template edges<false, true>(w, ll, op);
    }
    fft.i1_packed(w, ll);
    fft.i2(w, ll);
    fft.i3(w, ll);
    fft.i4(w, ll);
    float psum = 0.0f;   // this lane's part of its wave's plane sum (e.sums)
    if constexpr (PF) {
      // the wave's rows lie in plane pw: buffer loads / stores off that plane's bases, one lane
      // offset and uniform row steps; the m and d loads issued four vectors at a time
      const int pw = (w * G::RPW) / G::HP;
      if (pw < nvalid) {
        const long long p = p0 + pw;
        constexpr unsigned PB = unsigned(H * W * sizeof(float));
        constexpr int STEP = G::RK * G::C4N * 16;
        const int row0 = G::v4_row(w, 0, m);
        const unsigned vo = unsigned(((row0 - pw * H) * G::C4N + m.c4) * 16);
        const Buf bm(e.m.p ? e.m.p + e.m.off(p, e.C, H * W) : e.y, e.m.p ? PB : 0u);
        const Buf bd(e.d.p ? e.d.p + e.d.off(p, e.C, H * W) : e.y, e.d.p ? PB : 0u);
        const float c = e.add ? e.add[p] : 0.0f;
        const Buf by(e.y + ys.off(p, e.C, H * W), PB);
        constexpr int CH = G::JLD < 4 ? G::JLD : 4;
#pragma unroll
        for (int i0 = 0; i0 < G::JLD; i0 += CH) {
          float4 mv[CH], dv[CH];
#pragma unroll
          for (int i = 0; i < CH; ++i) {
            if (e.m.p) bm.ld(mv[i], vo, (i0 + i) * STEP);
            if (e.d.p) bd.ld(dv[i], vo, (i0 + i) * STEP);
          }
#pragma unroll
          for (int i = 0; i < CH; ++i) {
            float4 v = fft.v4_get(row0 + (i0 + i) * G::RK, col);
            v = make_float4(v.x + c, v.y + c, v.z + c, v.w + c);
            if (e.m.p) v = make_float4(v.x * mv[i].x, v.y * mv[i].y, v.z * mv[i].z, v.w * mv[i].w);
            if (e.d.p)
              v = make_float4(v.x * dsilu1(dv[i].x), v.y * dsilu1(dv[i].y), v.z * dsilu1(dv[i].z),
                              v.w * dsilu1(dv[i].w));
            by.st(v, vo, (i0 + i) * STEP);
            psum += (v.x + v.y) + (v.z + v.w);
          }
        }
      }
    } else {
#pragma unroll
    for (int i = 0; i < G::JLD; ++i) {
      const int row = G::v4_row(w, i, m);
      const unsigned f = G::v4_index(row, m);
      const int pl = int(f / V4P), q = int(f % V4P);
      if (pl >= nvalid) continue;
      const long long p = p0 + pl;
      float4 v = fft.v4_get(row, col);
      if (e.add) {
        const float c = e.add[p];
        v = make_float4(v.x + c, v.y + c, v.z + c, v.w + c);
      }
      if (e.m.p) {
        const float4 u = *reinterpret_cast<const float4*>(e.m.p + e.m.off(p, e.C, H * W) + 4 * q);
        v = make_float4(v.x * u.x, v.y * u.y, v.z * u.z, v.w * u.w);
      }
      if (e.d.p) {
        const float4 u = *reinterpret_cast<const float4*>(e.d.p + e.d.off(p, e.C, H * W) + 4 * q);
        v = make_float4(v.x * dsilu1(u.x), v.y * dsilu1(u.y), v.z * dsilu1(u.z), v.w * dsilu1(u.w));
      }
      *reinterpret_cast<float4*>(e.y + ys.off(p, e.C, H * W) + 4 * q) = v;
      psum += (v.x + v.y) + (v.z + v.w);
    }
    }
    if constexpr (G::V4_LINEAR) {
      if (e.sums) {
        // each wave's rows lie in one plane: wave sums in a fixed order, then the plane's waves in order
        const float s = wave_sum(psum);
        if (l == 0) wsum[w] = s;
        __syncthreads();
        constexpr int WPP = G::HP / G::RPW;   // waves per plane
        if (int(tid) < NP && int(tid) < nvalid) {
          float acc = 0.0f;
          for (int k = 0; k < WPP; ++k) acc += wsum[int(tid) * WPP + k];
          e.sums[p0 + tid] = acc;
        }
      }
    }
    __syncthreads();   // the stores (and the sums) are done with LDS before the next group's C2
  };
  if constexpr (PF) {
    for (long long g = blockIdx.x; g < NG; g += gridDim.x) group(g);
  } else {
    group(blockIdx.x);
  }
}

namespace {
template <int LH, int NP, int PPT>
hipError_t run_fwd_ex(const FftEx& e, long long P, float2* spec, hipStream_t s) {
  using G = Geom<LH, LH, NP, PPT>;
  const auto k = rfft2_planes_ex<LH, LH, NP, PPT>;
  // persistent kernels: as many workgroups as fit at once; the others one per group
  static const unsigned grid = fwd_persistent(G::V4_LINEAR, NP) ? resident_grid(reinterpret_cast<const void*>(k), G::NT, 1LL << 40) : ~0u;
  const long long groups = (P + NP - 1) / NP;
  hipLaunchKernelGGL(k, dim3(unsigned(groups < grid ? groups : grid)), dim3(G::NT), 0, s, e, P, spec);
  return hipGetLastError();
}
template <int LH, int NP, int PPT>
hipError_t run_inv_ex(const float2* spec, long long P, const FftEx& e, hipStream_t s) {
  using G = Geom<LH, LH, NP, PPT>;
  const auto k = irfft2_planes_ex<LH, LH, NP, PPT>;
  // persistent kernels: as many workgroups as fit at once; the others one per group
  static const unsigned grid = inv_persistent(G::V4_LINEAR) ? resident_grid(reinterpret_cast<const void*>(k), G::NT, 1LL << 40) : ~0u;
  const long long groups = (P + NP - 1) / NP;
  hipLaunchKernelGGL(k, dim3(unsigned(groups < grid ? groups : grid)), dim3(G::NT), 0, s, spec, P, e);
  return hipGetLastError();
}
}  // namespace

// ---------------------------------------------------------------------------
// im2col of a SAME k x k convolution over channels-last frames (the full-channel
// qkv conv, cssm.py:4751-4753): row p = (f, h, w) of the output holds, for tap
// (a, b) and channel c, x[f][h + a - lo][w + b - lo][c] at column (a k + b) C + c,
// zero outside the frame (lo = (k - 1) / 2, as SAME pads).  The conv is then the
// projection kernel's GEMM of these rows with the (k k C, N) kernel.
// One thread per (row, tap, 4 channels) when C % 4 == 0, else per channel.
// ---------------------------------------------------------------------------
template <class TI, int VEC>
__global__ void __launch_bounds__(256) im2col_same_cl(const TI* __restrict__ x, long long rows, int H, int W, int C,
                                                      int ks, float* __restrict__ out) {
  const int CG = C / VEC, taps = ks * ks, lo = (ks - 1) / 2;
  const long long n = rows * taps * CG;
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long long)gridDim.x * blockDim.x) {
    const int cg = int(i % CG);
    const long long rt = i / CG;
    const int tap = int(rt % taps);
    const long long r = rt / taps;
    const int w = int(r % W), h = int((r / W) % H);
    const long long f = r / ((long long)H * W);
    const int hh = h + tap / ks - lo, ww = w + tap % ks - lo;
    float v[VEC];
    if (hh >= 0 && hh < H && ww >= 0 && ww < W) {
      const size_t src = ((size_t(f) * H + hh) * W + ww) * C + size_t(cg) * VEC;
#pragma unroll
      for (int e = 0; e < VEC; ++e) v[e] = ld_f(x, src + e);
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) v[e] = 0.0f;
    }
    const size_t dst = size_t(r) * size_t(taps) * C + size_t(tap) * C + size_t(cg) * VEC;
    if constexpr (VEC == 4) st4v(out, dst, make_float4(v[0], v[1], v[2], v[3]));
    else out[dst] = v[0];
  }
}

hipError_t launch_im2col_same(const void* x, int dtype, long long rows, int H, int W, int C, int ks, float* out,
                              hipStream_t s) {
  const bool v4 = C % 4 == 0;
  const long long n = rows * ks * ks * (v4 ? C / 4 : C);
  const unsigned blocks = unsigned(n / 256 + 1 < 65536 * 4 ? n / 256 + 1 : 65536 * 4);
  if (dtype == 0) {
    if (v4) hipLaunchKernelGGL((im2col_same_cl<float, 4>), dim3(blocks), dim3(256), 0, s, static_cast<const float*>(x), rows, H, W, C, ks, out);
    else hipLaunchKernelGGL((im2col_same_cl<float, 1>), dim3(blocks), dim3(256), 0, s, static_cast<const float*>(x), rows, H, W, C, ks, out);
  } else {
    if (v4) hipLaunchKernelGGL((im2col_same_cl<uint16_t, 4>), dim3(blocks), dim3(256), 0, s, static_cast<const uint16_t*>(x), rows, H, W, C, ks, out);
    else hipLaunchKernelGGL((im2col_same_cl<uint16_t, 1>), dim3(blocks), dim3(256), 0, s, static_cast<const uint16_t*>(x), rows, H, W, C, ks, out);
  }
  return hipGetLastError();
}

bool fft_ex_supported(int H, int W) { return H == W && H >= 4 && H <= 128 && (H & (H - 1)) == 0; }

bool irfft2_ex_sums_supported(long long P, int H, int W) {
  if (!fft_ex_supported(H, W) || P <= 0) return false;
#define CSSM_SUMS_CASE(LH, NP_, PPT_) \
  if (np == NP_) return Geom<LH, LH, NP_, PPT_>::V4_LINEAR;
  CSSM_FFT_TABLE(CSSM_SUMS_CASE, 32)
#undef CSSM_SUMS_CASE
  return false;
}

hipError_t launch_rfft2_ex(const FftEx& e, long long P, int H, int W, float2* spec, hipStream_t s) {
  if (!fft_ex_supported(H, W)) return hipErrorInvalidValue;
#define CSSM_FWD_EX_CASE(LH, NP_, PPT_) \
  if (np == NP_) return run_fwd_ex<LH, NP_, PPT_>(e, P, spec, s);
  CSSM_FFT_TABLE(CSSM_FWD_EX_CASE, 64)
#undef CSSM_FWD_EX_CASE
  return hipErrorInvalidValue;
}

hipError_t launch_irfft2_ex(const float2* spec, long long P, int H, int W, const FftEx& e, hipStream_t s) {
  if (!fft_ex_supported(H, W)) return hipErrorInvalidValue;
#define CSSM_INV_EX_CASE(LH, NP_, PPT_) \
  if (np == NP_) return run_inv_ex<LH, NP_, PPT_>(spec, P, e, s);
  CSSM_FFT_TABLE(CSSM_INV_EX_CASE, 32)
#undef CSSM_INV_EX_CASE
  return hipErrorInvalidValue;
}

// ---------------------------------------------------------------------------
// Delta-rule recurrence per (b, head, bin), all T steps, state in VGPRs.
//   q_a, k_a, v_i   spectra of channels head*DK + a of the q / k / v blocks
//   spectral norm:  x <- x / sqrt(sum_bins |x|^2 + 1e-6)        (q and k, :4890-4897)
//   key norm:       k <- k / sqrt(sum_a |k_a|^2 + 1e-6)          (:4899-4906)
//   M[a][b] = floor(alpha W_hat (delta_ab - beta k_a conj k_b))  (:4911-4925)
//   D[i][a] = floor(beta v_i conj k_a)                           (:4927-4929)
//   s_i     = M s_i + D[i]                                       (:4945-4958, math.py:384-411;
//             the log-space general matrix scan evaluates this linear recurrence,
//             operations.py:314-390, with to_goom's floors on M and D)
//   o_i     = sum_a s_i[a] q_a                                   (:4998-5000)
// ---------------------------------------------------------------------------
struct GdnBinArgs {
  const float2* spec;   // (B, T, 3C, H, WF)
  const float* norms;   // (B, T, 3C) sum |X|^2, or nullptr (no spectral L2 norm)
  const float2* ab;     // (alpha, beta) at (b T + t) ab_frame + head ab_head + bin ab_bin
  long long ab_frame;
  int ab_head, ab_bin;
  const float2* what;   // (n_h, H, WF)
  float2* ohat;         // (B, T, C, H, WF)
  int T, C, HWF;
  int variant;          // kScanGoom / kScanLinear / kScanLogEps (gdn_step.h)
};

template <int DK>
__global__ void __launch_bounds__(256) gdn_scan_bins(const GdnBinArgs a) {
  const int bin = blockIdx.x * blockDim.x + threadIdx.x;
  if (bin >= a.HWF) return;
  const int head = blockIdx.y, b = blockIdx.z;
  const int C = a.C, HWF = a.HWF;
  const float2 wh = a.what[size_t(head) * HWF + bin];
  float2 s[DK][DK];   // s[i][a]
#pragma unroll
  for (int i = 0; i < DK; ++i)
#pragma unroll
    for (int j = 0; j < DK; ++j) s[i][j] = make_float2(0.f, 0.f);

  for (int t = 0; t < a.T; ++t) {
    const size_t fr = size_t(b) * a.T + t;
    const size_t ch0 = fr * 3 * C + size_t(head) * DK;   // q block; k at + C, v at + 2C
    float2 q[DK], k[DK], v[DK];
#pragma unroll
    for (int j = 0; j < DK; ++j) {
      q[j] = a.spec[(ch0 + j) * HWF + bin];
      k[j] = a.spec[(ch0 + C + j) * HWF + bin];
      v[j] = a.spec[(ch0 + 2 * C + j) * HWF + bin];
    }
    if (a.norms) {
#pragma unroll
      for (int j = 0; j < DK; ++j) {
        const float nq = 1.0f / sqrtf(a.norms[ch0 + j] + 1e-6f);
        const float nk = 1.0f / sqrtf(a.norms[ch0 + C + j] + 1e-6f);
        q[j] = cscale(q[j], nq);
        k[j] = cscale(k[j], nk);
      }
    }
    const float2 g = a.ab[fr * a.ab_frame + size_t(head) * a.ab_head + size_t(bin) * a.ab_bin];
    float2 o[DK];
    gdn_bin_step<DK>(s, q, k, v, wh, g.x, g.y, a.variant, o);
#pragma unroll
    for (int i = 0; i < DK; ++i) a.ohat[(fr * C + size_t(head) * DK + i) * HWF + bin] = o[i];
  }
}

// ---------------------------------------------------------------------------
// Fused spectral core for 32 x 32 planes and d_k = 4 (the video-shaped
// config): one workgroup per (b, head) runs all T steps, so the 4 x 4 complex
// state of the head's 32 x 17 bins (70 KB) stays in VGPRs, and each step reads
// q, k, v and writes o once, with no spectra in HBM.  Per step:
//   load     the head's 12 q / k / v planes (issued a step ahead) -> LDS
//   forward  2-D real FFT of the 12 planes (fft_plane.h passes); the spectrum
//            stays in LDS: interior bin k + H1 q of unit k in the slot (row
//            q + H2 k) the column pass read it from, the DC / Nyquist columns
//            in esp
//   norms    per-plane sums of |X|^2 (spectral L2 norms of q and k), reduced
//            per wave and across the four waves in a fixed order
//   bins     per bin (thread-owned, state in VGPRs): gdn_bin_step, o / (H W)
//            written over the q slots of the bin
//   inverse  2-D real FFT of the 4 o planes -> HBM
// The forward passes see every bin doubled (the packed-row separation skips
// its 1/2); the bins are halved on reading.
// ---------------------------------------------------------------------------
namespace {
constexpr int kFusedDK = 4;
using FusedFwdG = Geom<5, 5, 3 * kFusedDK, 48>;   // the 12 q, k, v planes, 256 threads
using FusedInvG = Geom<5, 5, kFusedDK, 16>;       // the 4 o planes in the same buffer, 256 threads
static_assert(FusedFwdG::NT == 256 && FusedInvG::NT == 256, "one thread count for both plane groups");
static_assert(FusedFwdG::RS == FusedInvG::RS, "one row stride for both plane groups");
}  // namespace

// forward policy: the spectrum stays in LDS (interior bins in the slots the
// column pass read, DC / Nyquist bins of plane pl, row u in esp[(pl H + u) 2 + (0 | 1)])
template <class G>
struct SpecKeepOp {
  static constexpr bool kPackedColumnToo = false;
  static constexpr int H = G::H, H2 = G::H2;
  float* buf;
  float2* esp;
  __device__ __forceinline__ void bins(int, int, int pl, int k, int v, float2 (&sp)[G::H2]) const {
    const int col = G::p_col(v);
#pragma unroll
    for (int q = 0; q < H2; ++q) *reinterpret_cast<float2*>(buf + G::row_off(pl, q + H2 * k) + col) = sp[q];
  }
  __device__ __forceinline__ void edge(int, int pl, int uA, int uB, int, float2 (&v4)[4]) const {
    esp[(pl * H + uA) * 2] = v4[0];
    esp[(pl * H + uA) * 2 + 1] = v4[1];
    esp[(pl * H + uB) * 2] = v4[2];
    esp[(pl * H + uB) * 2 + 1] = v4[3];
  }
};

// inverse policy: the bins from the same places
template <class G>
struct SpecFromLdsOp {
  static constexpr bool kPackedColumnToo = false;
  static constexpr int H = G::H, H2 = G::H2;
  const float* buf;
  const float2* esp;
  __device__ __forceinline__ void bins(int, int, int pl, int k, int v, float2 (&sp)[G::H2]) const {
    const int col = G::p_col(v);
#pragma unroll
    for (int q = 0; q < H2; ++q) sp[q] = *reinterpret_cast<const float2*>(buf + G::row_off(pl, q + H2 * k) + col);
  }
  __device__ __forceinline__ void edge(int, int pl, int uA, int uB, int, float2 (&v4)[4]) const {
    v4[0] = esp[(pl * H + uA) * 2];
    v4[1] = esp[(pl * H + uA) * 2 + 1];
    v4[2] = esp[(pl * H + uB) * 2];
    v4[3] = esp[(pl * H + uB) * 2 + 1];
  }
};

struct GdnFusedArgs {
  const float* qkv;      // (B, T, 3C, H, W) float32
  const float2* ab;      // (alpha, beta) at (b T + t) ab_frame + head ab_head + bin ab_bin
  long long ab_frame;
  int ab_head, ab_bin;
  const float2* what;    // (n_h, H, WF)
  float* o;              // (B, T, C, H, W) float32
  int T, C, use_l2;
  int variant;           // kScanGoom / kScanLinear / kScanLogEps (gdn_step.h)
};

__global__ void __launch_bounds__(256, 2) gdn_core_fused32(const GdnFusedArgs a) {
  using GF = FusedFwdG;
  using GI = FusedInvG;
  constexpr int H = GF::H, W = GF::W, WF = GF::WF, WH = GF::WH, HW = H * W, DK = kFusedDK, NP = 3 * DK;
  // bins i = tid + NT j: j < BPT in registers; the NX = NB - BPT NT rest with their state in LDS, one
  // state row per lane: lane l < DK XW of wave w takes row l % DK of bin BPT NT + XW w + l / DK, so every
  // wave adds a fraction of a step instead of one wave adding a whole one
  constexpr int NT = GF::NT, NB = H * WF, NINT = H * (WH - 1), BPT = NB / NT, NX = NB - BPT * NT, BT = BPT + 1;
  constexpr int NW = NT / 64, JL = GI::JLD, XW = NX / NW;
  static_assert(NX % NW == 0 && XW * DK <= 64, "the bins beyond BPT per thread split evenly over the waves' lanes");
  static_assert(GI::V4_LINEAR && GI::RPW == GI::HP && NW == DK && GI::C4N == 8,
                "the norms' sums assume wave w loads all of plane w of a group, 8 lanes to a row");
  __shared__ __attribute__((aligned(16))) float smem[GF::LDS_FLOATS];
  __shared__ float2 esp[NP * H * 2];
  __shared__ float2 sx[NX * DK * DK];
  __shared__ float red[2 * DK];
  const PlaneFft<GF> fwd(smem);
  const PlaneFft<GI> inv(smem, reinterpret_cast<float2*>(smem + GF::OFF_EDGE),
                         reinterpret_cast<float2*>(smem + GF::OFF_TW));
  const int tid = int(threadIdx.x);
  const int w = __builtin_amdgcn_readfirstlane(tid / 64), l = tid % 64;
  const int head = blockIdx.x, b = blockIdx.y;
  const int T = a.T, C = a.C;
  fwd.init_twiddles(tid);

  // this thread's bins i = tid + NT j: interior (u, v) = (i / 15, 1 + i % 15) first (consecutive
  // threads along a row), then the DC / Nyquist bins (u, 0 | W / 2) = ((i - NINT) / 2, ...)
  auto bin_uv = [](int i, int& u, int& v) {
    if (i < NINT) {
      u = i / (WH - 1);
      v = 1 + i % (WH - 1);
    } else {
      const int e = i - NINT;
      u = e >> 1;
      v = (e & 1) ? WH : 0;
    }
  };
  float2 s[BPT][DK][DK];
#pragma unroll
  for (int j = 0; j < BPT; ++j)
#pragma unroll
    for (int r = 0; r < DK; ++r)
#pragma unroll
      for (int c = 0; c < DK; ++c) s[j][r][c] = make_float2(0.f, 0.f);
  for (int i = tid; i < NX * DK * DK; i += NT) sx[i] = make_float2(0.f, 0.f);
  // LDS place of bin (u, v) of plane pl
  auto bin_ptr = [&](int pl, int u, int v) -> float2* {
    if (v == 0 || v == WH) return &esp[(pl * H + u) * 2 + (v ? 1 : 0)];
    return reinterpret_cast<float2*>(smem + GF::row_off(pl, u / GF::H1 + GF::H2 * (u % GF::H1)) + GF::p_col(v));
  };

  // q, k, v planes of (b, t): three runs of DK contiguous planes, each loaded
  // with the 4-plane group's mapping (wave w, its rows)
  constexpr unsigned GB = unsigned(DK * HW * sizeof(float));
  float4 pf[3][JL];
  auto issue = [&](int t, int lane) {
    const auto m = GI::v4_lane(lane);
#pragma unroll
    for (int g = 0; g < 3; ++g) {
      const Buf src(a.qkv + ((size_t(b) * T + t) * 3 * C + size_t(g) * C + size_t(head) * DK) * HW, GB);
#pragma unroll
      for (int i = 0; i < JL; ++i) {
        unsigned vo;
        int so;
        GI::template v4_goff<16>(w, i, m, vo, so);
        src.ld(pf[g][i], vo, so);
      }
    }
  };
  issue(0, l);

  for (int t = 0; t < T; ++t) {
    // Re-derive the thread index inside the loop so the compiler rebuilds the (cheap) LDS and
    // bin addresses per step instead of holding them in registers for the whole scan
    int tl = tid;
    asm volatile("" : "+v"(tl));
    __builtin_assume(tl >= 0 && tl < NT);
    const int lane = tl % 64;
    int bu[BT], bv[BT];
    bool bok[BT];
    // slot BPT: the extra bin whose state row this lane updates
    const int xl = tl % 64, xbin = XW * (tl / 64) + xl / DK, xrow = xl % DK;
#pragma unroll
    for (int j = 0; j < BT; ++j) {
      const int i = j < BPT ? tl + NT * j : BPT * NT + xbin;
      bok[j] = j < BPT ? i < NB : xl < XW * DK;
      bin_uv(bok[j] ? i : 0, bu[j], bv[j]);
    }
    __syncthreads();   // the previous step's inverse and stores are done with the buffer
    {
      const auto m = GI::v4_lane(lane);
      const auto vcol = PlaneFft<GI>::v4_col(m.c4);
#pragma unroll
      for (int g = 0; g < 3; ++g)
#pragma unroll
        for (int i = 0; i < JL; ++i) inv.v4_put(GI::v4_row(w, i, m) + g * DK * H, vcol, pf[g][i]);
      // spectral L2 norms of the q and k planes by Parseval, from the planes as loaded: over the half
      // spectrum sum |X|^2 = (H W sum x^2 + H sum_h (r_h^2 + a_h^2)) / 2, r_h and a_h the plain and
      // alternating sums of row h (the columns v = 0 and v = W / 2 are the DFTs of those over h).
      // Wave w holds all of plane w of each group; the 8 lanes of a row hold its 4-vectors.
      if (a.use_l2) {
#pragma unroll
        for (int g = 0; g < 2; ++g) {
          float e = 0.0f, rr = 0.0f;
#pragma unroll
          for (int i = 0; i < JL; ++i) {
            const float4 v = pf[g][i];
            e = fmaf(v.x, v.x, fmaf(v.y, v.y, fmaf(v.z, v.z, fmaf(v.w, v.w, e))));
            float r = (v.x + v.y) + (v.z + v.w), al = (v.x - v.y) + (v.z - v.w);
            r += dpp_f<0xb1>(r);    // quad_perm [1, 0, 3, 2]
            al += dpp_f<0xb1>(al);
            r += dpp_f<0x4e>(r);    // quad_perm [2, 3, 0, 1]
            al += dpp_f<0x4e>(al);
            r += dpp_f<0x141>(r);   // row_half_mirror: the 8 lanes of the row
            al += dpp_f<0x141>(al);
            rr = fmaf(r, r, fmaf(al, al, rr));
          }
          const float x = wave_sum(fmaf(float(HW), e, m.c4 == 0 ? float(H) * rr : 0.0f));
          if (lane == 0) red[g * DK + w] = x;
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
    const size_t fr = size_t(b) * T + t;
    float2 gab[BT], wh[BT];
#pragma unroll
    for (int j = 0; j < BT; ++j) {
      const int bin = bu[j] * WF + bv[j];
      gab[j] = bok[j] ? a.ab[fr * a.ab_frame + size_t(head) * a.ab_head + size_t(bin) * a.ab_bin]
                      : make_float2(0.f, 0.f);
      wh[j] = bok[j] ? a.what[size_t(head) * H * WF + bin] : make_float2(0.f, 0.f);
    }
    // the next step's planes after this step's gates: loads retire in issue order, so the bin
    // steps' wait for the gates does not also wait for the next planes
    if (t + 1 < T) issue(t + 1, lane);
    __syncthreads();

    fwd.r1(w, lane);
    fwd.r2(w, lane);
    fwd.c1(w, lane);
    const SpecKeepOp<GF> keep{smem, esp};
    fwd.template c2<true, false>(w, lane, keep);
    fwd.template edges<true, false>(w, lane, keep);
    __syncthreads();

    // 1 / sqrt(sum |X|^2 + 1e-6) from the sums the waves stored before the forward transform
    float nrm[2 * DK];
#pragma unroll
    for (int p = 0; p < 2 * DK; ++p) nrm[p] = a.use_l2 ? 1.0f / sqrtf(0.5f * red[p] + 1e-6f) : 1.0f;

    // the recurrence of each of this thread's bins; o / (H W) over its q slots
    auto bin_step = [&](int j, float2 (&st)[DK][DK]) {
      float2 q[DK], k[DK], v[DK], o[DK];
#pragma unroll
      for (int c = 0; c < DK; ++c) {
        q[c] = cscale(*bin_ptr(c, bu[j], bv[j]), 0.5f * nrm[c]);
        k[c] = cscale(*bin_ptr(DK + c, bu[j], bv[j]), 0.5f * nrm[DK + c]);
        v[c] = cscale(*bin_ptr(2 * DK + c, bu[j], bv[j]), 0.5f);
      }
      gdn_bin_step<DK>(st, q, k, v, wh[j], gab[j].x, gab[j].y, a.variant, o);
#pragma unroll
      for (int c = 0; c < DK; ++c) *bin_ptr(c, bu[j], bv[j]) = cscale(o[c], 1.0f / float(HW));
    };
#pragma unroll
    for (int j = 0; j < BPT; ++j) bin_step(j, s[j]);
    if (bok[BPT]) {
      // row xrow of extra bin xbin (the bin's DK lanes are adjacent in one wave, so all of them have
      // read q, k, v before any writes its o row over q)
      float2 q[DK], k[DK], v[DK], si[DK];
#pragma unroll
      for (int c = 0; c < DK; ++c) {
        q[c] = cscale(*bin_ptr(c, bu[BPT], bv[BPT]), 0.5f * nrm[c]);
        k[c] = cscale(*bin_ptr(DK + c, bu[BPT], bv[BPT]), 0.5f * nrm[DK + c]);
        v[c] = cscale(*bin_ptr(2 * DK + c, bu[BPT], bv[BPT]), 0.5f);
        si[c] = sx[(xbin * DK + xrow) * DK + c];
      }
      const GdnBinPre<DK> pre = gdn_bin_prep<DK>(k, v, wh[BPT], gab[BPT].x, gab[BPT].y, a.variant);
      float2 vr = v[0];   // v[xrow] by selects (a lane-varying index would place v in memory)
#pragma unroll
      for (int c = 1; c < DK; ++c) vr = xrow == c ? v[c] : vr;
      const float2 oi = gdn_bin_row<DK>(si, vr, q, k, pre, gab[BPT].y, a.variant);
#pragma unroll
      for (int c = 0; c < DK; ++c) sx[(xbin * DK + xrow) * DK + c] = si[c];
      *bin_ptr(xrow, bu[BPT], bv[BPT]) = cscale(oi, 1.0f / float(HW));
    }
    __syncthreads();

    const SpecFromLdsOp<GI> from{smem, esp};
    inv.template c2<false, true>(w, lane, from);
    inv.template edges<false, true>(w, lane, from);
    inv.i1_packed(w, lane);
    inv.i2(w, lane);
    inv.i3(w, lane);
    inv.i4(w, lane);
    {
      const auto m = GI::v4_lane(lane);
      const auto vcol = PlaneFft<GI>::v4_col(m.c4);
      const Buf dst(a.o + (fr * C + size_t(head) * DK) * HW, GB);
#pragma unroll
      for (int i = 0; i < JL; ++i) {
        unsigned vo;
        int so;
        GI::template v4_goff<16>(w, i, m, vo, so);
        dst.st(inv.v4_get(GI::v4_row(w, i, m), vcol), vo, so);
      }
    }
  }
}

// fused core: 32 x 32 planes, d_k = 4, float32 qkv / o
bool gdn_core_fused_supported(int H, int W, int dk) { return H == 32 && W == 32 && dk == kFusedDK; }

hipError_t launch_gdn_core_fused(const float* qkv, int use_l2, const float2* ab, long long ab_frame, int ab_head,
                                 int ab_bin, const float2* what, int B, int T, int C, int H, int W, int dk, int variant,
                                 float* o, hipStream_t s) {
  if (!gdn_core_fused_supported(H, W, dk) || C % dk) return hipErrorInvalidValue;
  GdnFusedArgs a;
  a.qkv = qkv;
  a.ab = ab;
  a.ab_frame = ab_frame;
  a.ab_head = ab_head;
  a.ab_bin = ab_bin;
  a.what = what;
  a.o = o;
  a.T = T;
  a.C = C;
  a.use_l2 = use_l2;
  a.variant = variant;
  hipLaunchKernelGGL(gdn_core_fused32, dim3(unsigned(C / dk), unsigned(B)), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_gdn_scan_bins(const float2* spec, const float* norms, const float2* ab, long long ab_frame,
                                int ab_head, int ab_bin, const float2* what, int B, int T, int C, int H, int W,
                                int dk, int variant, float2* ohat, hipStream_t s) {
  GdnBinArgs a;
  a.spec = spec;
  a.norms = norms;
  a.ab = ab;
  a.ab_frame = ab_frame;
  a.ab_head = ab_head;
  a.ab_bin = ab_bin;
  a.what = what;
  a.ohat = ohat;
  a.T = T;
  a.C = C;
  a.HWF = H * (W / 2 + 1);
  a.variant = variant;
  const dim3 grid(unsigned((a.HWF + 255) / 256), unsigned(C / dk), unsigned(B));
  switch (dk) {
    case 1: hipLaunchKernelGGL(gdn_scan_bins<1>, grid, dim3(256), 0, s, a); break;
    case 2: hipLaunchKernelGGL(gdn_scan_bins<2>, grid, dim3(256), 0, s, a); break;
    case 3: hipLaunchKernelGGL(gdn_scan_bins<3>, grid, dim3(256), 0, s, a); break;
    case 4: hipLaunchKernelGGL(gdn_scan_bins<4>, grid, dim3(256), 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// ctx = mean over (H, W) of channels-last x (F, HW, C) -> (F, C)   (:4785)
// ---------------------------------------------------------------------------
template <class TI>
__global__ void __launch_bounds__(256) frame_mean_cl(const TI* __restrict__ x, int HW, int C, float* __restrict__ out) {
  __shared__ float4 red[256];
  const int f = blockIdx.x;
  const TI* xf = x + size_t(f) * HW * C;
  const int cv = (C % 4 == 0) ? 4 : 1;
  for (int c0 = 0; c0 < C; c0 += 256 * cv) {
    const int cw = min(256, (C - c0) / cv);          // channel groups of this chunk
    const int rows = 256 / cw;                        // pixels summed in parallel
    const int r = threadIdx.x / cw, c = c0 + (threadIdx.x % cw) * cv;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    if (r < rows) {
      int p = r;
      if (cv == 4) {
        // 4 independent loads in flight per iteration
        for (; p + 3 * rows < HW; p += 4 * rows) {
          float4 v[4];
#pragma unroll
          for (int u = 0; u < 4; ++u) v[u] = ld4v(xf, size_t(p + u * rows) * C + c);
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            acc.x += v[u].x; acc.y += v[u].y; acc.z += v[u].z; acc.w += v[u].w;
          }
        }
        for (; p < HW; p += rows) {
          const float4 v = ld4v(xf, size_t(p) * C + c);
          acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
        }
      } else {
        for (; p < HW; p += rows) acc.x += ld_f(xf, size_t(p) * C + c);
      }
    }
    red[threadIdx.x] = acc;
    __syncthreads();
    if (threadIdx.x < cw) {
      float4 sum = make_float4(0.f, 0.f, 0.f, 0.f);
      for (int i = 0; i < rows; ++i) {
        const float4 v = red[i * cw + threadIdx.x];
        sum.x += v.x; sum.y += v.y; sum.z += v.z; sum.w += v.w;
      }
      const float inv = 1.0f / float(HW);
      const float e[4] = {sum.x, sum.y, sum.z, sum.w};
      for (int k = 0; k < cv; ++k) out[size_t(f) * C + c0 + threadIdx.x * cv + k] = e[k] * inv;
    }
    __syncthreads();
  }
}

hipError_t launch_frame_mean(const void* x, int dtype, int F, int HW, int C, float* out, hipStream_t s) {
  if (dtype == 0)
    hipLaunchKernelGGL(frame_mean_cl<float>, dim3(F), dim3(256), 0, s, static_cast<const float*>(x), HW, C, out);
  else
    hipLaunchKernelGGL(frame_mean_cl<uint16_t>, dim3(F), dim3(256), 0, s, static_cast<const uint16_t*>(x), HW, C,
                       out);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Gate vectors of GatedDeltaNetCSSM from ctx (:4785-4869), one block per (b, t):
//   ctx_t = ctx + E[t]  (temporal: 1 = sinusoid table with rope_base, :353-383;
//                        2 = learned table (T, C); 0 = none)
//   alpha = 0.1 + 0.89 sigmoid(g_alpha), beta = sigmoid(g_beta)   (spectral, per bin / head)
//   B_k, B_v = sigmoid(g)                                          (spatial, per pixel)
// gate kinds: factored  g[u, v] = (ctx kh + bh)[u] + (ctx kw + bw)[v]
//             dense     g = ctx kd + bd          (n outputs)
//             channel   g = ctx kd + bd          (n_h outputs; spectral only)
//             scalar    g = ctx kd + bd          (1 output)
// ab (B T, n_ab) float2 (alpha, beta); bkv (B T, n_kv) float2 (B_k, B_v).
// ---------------------------------------------------------------------------
__device__ float dot_col(const float* ctx, const float* k, int C, int n, int col) {
  float acc = 0.0f;
  for (int c = 0; c < C; ++c) acc = fmaf(ctx[c], k[size_t(c) * n + col], acc);
  return acc;
}

// FB frames per block (factored gates, host-chosen): each weight is loaded once and applied to the
// FB frames' contexts (the per-frame sums keep their order, so the result does not depend on FB)
constexpr int kGatesMaxFB = 4;
__global__ void __launch_bounds__(1024)
gdn_gates_kernel(const float* __restrict__ ctx_in, int T, int C, int H, int W, int nh, GdnGateWeights w,
                 int temporal, float rope_base, const float* __restrict__ ttable, float2* __restrict__ ab,
                 float2* __restrict__ bkv, int FB) {
  extern __shared__ float sm[];
  const int f0 = int(blockIdx.x) * FB;   // first (b, t) frame of the block
  const int WF = W / 2 + 1;
  const int CW = W > WF ? W : WF;
  const int NV = 4 * (H + CW);
  const int P = w.kind == 1 ? (NV >= int(blockDim.x) ? 1 : int(blockDim.x) / NV) : 0;
  float* cx = sm;                      // FB x C
  float* rows = cx + FB * C;           // FB x 4 x H
  float* cols = rows + FB * 4 * H;     // FB x 4 x max(W, WF)
  float* part = cols + FB * 4 * CW;    // factored: FB x P partial sums of each of the 4 (H + CW) products
  for (int e = threadIdx.x; e < FB * C; e += blockDim.x) {
    const int fl = e / C, c = e % C, bt = f0 + fl, t = bt % T;
    float v = ctx_in[size_t(bt) * C + c];
    if (temporal == 1) {
      // E[t, 2j] = sin(t / base^(2j / C)), E[t, 2j + 1] = cos(.)
      const int j2 = c & ~1;
      const double th = double(t) / pow(double(rope_base), double(j2) / double(C));
      v += float((c & 1) ? cos(th) : sin(th));
    } else if (temporal == 2) {
      v += ttable[size_t(t) * C + c];
    }
    cx[e] = v;
  }
  __syncthreads();
  // gate g in {0 alpha, 1 beta, 2 B_k, 3 B_v}; spectral gates span (H, WF), spatial (H, W).
  // Factored: the row / column products of all four gates at once, product q = g (H + CW) + i,
  // each split over P threads (channel stride P) whose partials are summed in order.
  if (w.kind == 1) {
    for (int e = threadIdx.x; e < NV * P; e += blockDim.x) {
      const int q = e % NV, pc = e / NV;
      const int g = q / (H + CW), i = q % (H + CW);
      const int nc = g < 2 ? WF : W;
      float acc[kGatesMaxFB] = {0.0f, 0.0f, 0.0f, 0.0f};
      if (w.kd[g] && (i < H || i - H < nc)) {
        const float* k = i < H ? w.kd[g] + i : w.kw[g] + (i - H);
        const int n = i < H ? H : nc;
#pragma unroll 4
        for (int c = pc; c < C; c += P) {
          const float kv = k[size_t(c) * n];
#pragma unroll
          for (int fl = 0; fl < kGatesMaxFB; ++fl)
            if (fl < FB) acc[fl] = fmaf(cx[fl * C + c], kv, acc[fl]);
        }
      }
#pragma unroll
      for (int fl = 0; fl < kGatesMaxFB; ++fl)
        if (fl < FB) part[(fl * P + pc) * NV + q] = acc[fl];
    }
    __syncthreads();
    for (int e = threadIdx.x; e < FB * NV; e += blockDim.x) {
      const int fl = e / NV, q = e % NV;
      const int g = q / (H + CW), i = q % (H + CW);
      const int nc = g < 2 ? WF : W;
      if (!w.kd[g] || (i >= H && i - H >= nc)) continue;
      float acc = i < H ? w.bd[g][i] : w.bw[g][i - H];
      for (int pc = 0; pc < P; ++pc) acc += part[(fl * P + pc) * NV + q];
      if (i < H) rows[(fl * 4 + g) * H + i] = acc;
      else cols[(fl * 4 + g) * CW + i - H] = acc;
    }
  }
  __syncthreads();
  auto spectral = [&](int fl, int g, int i) -> float {       // raw gate at output i of frame fl
    if (w.kind == 1) return rows[(fl * 4 + g) * H + i / WF] + cols[(fl * 4 + g) * CW + i % WF];
    const int n = w.kind == 0 ? H * WF : (w.kind == 2 ? nh : 1);
    return dot_col(cx + fl * C, w.kd[g], C, n, i) + w.bd[g][i];
  };
  auto spatial = [&](int fl, int g, int i) -> float {
    if (w.kind == 1) return rows[(fl * 4 + g) * H + i / W] + cols[(fl * 4 + g) * CW + i % W];
    const int n = w.kind == 0 ? H * W : 1;
    return dot_col(cx + fl * C, w.kd[g], C, n, i) + w.bd[g][i];
  };
  const int n_ab = w.kind == 2 ? nh : (w.kind == 3 ? 1 : H * WF);
  for (int e = threadIdx.x; e < FB * n_ab; e += blockDim.x) {
    const int fl = e / n_ab, i = e % n_ab;
    const float al = 0.1f + 0.89f * sigmoid_f(spectral(fl, 0, i));
    const float be = sigmoid_f(spectral(fl, 1, i));
    ab[size_t(f0 + fl) * n_ab + i] = make_float2(al, be);
  }
  if (bkv && w.kd[2] && w.kind != 2) {
    const int n_kv = w.kind == 3 ? 1 : H * W;
    for (int e = threadIdx.x; e < FB * n_kv; e += blockDim.x) {
      const int fl = e / n_kv, i = e % n_kv;
      bkv[size_t(f0 + fl) * n_kv + i] = make_float2(sigmoid_f(spatial(fl, 2, i)), sigmoid_f(spatial(fl, 3, i)));
    }
  }
}

hipError_t launch_gdn_gates(const float* ctx, int B, int T, int C, int H, int W, int nh, const GdnGateWeights& w,
                            int temporal, float rope_base, const float* ttable, float2* ab, float2* bkv,
                            hipStream_t s) {
  const int WF = W / 2 + 1, CW = W > WF ? W : WF;
  constexpr int NT = 1024;
  const int NV = 4 * (H + CW), P = w.kind == 1 ? (NV >= NT ? 1 : NT / NV) : 0;
  const size_t per_frame = size_t(C) + 4 * size_t(H) + 4 * size_t(CW) + size_t(P) * NV;   // floats
  if (sizeof(float) * per_frame > 64 * 1024) return hipErrorInvalidValue;
  // factored gates: frames per block where they divide B T and fit the 64 KB
  int fb = 1;
  if (w.kind == 1)
    for (int c = kGatesMaxFB; c > 1; c /= 2)
      if ((B * T) % c == 0 && sizeof(float) * per_frame * c <= 64 * 1024) {
        fb = c;
        break;
      }
  hipLaunchKernelGGL(gdn_gates_kernel, dim3(unsigned(B * T / fb)), dim3(NT), sizeof(float) * per_frame * fb, s, ctx,
                     T, C, H, W, nh, w, temporal, rope_base, ttable, ab, bkv, fb);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Depthwise k x k SAME convolution on channels-last frames (qkv_dw, :4744-4750):
//   y[f, h, w, c] = b[c] + sum_{i, j} k[i, j, 0, c] x[f, h + i - lo, w + j - lo, c],
//   lo = (k - 1) // 2 (Flax 'SAME'), zeros outside the frame.
// ---------------------------------------------------------------------------
template <class TI, class TO>
__global__ void __launch_bounds__(256)
dwconv_cl(const TI* __restrict__ x, int H, int W, int C, int ks, const float* __restrict__ kw,
          const float* __restrict__ bias, TO* __restrict__ y, long long total, int vec) {
  // one thread per (pixel, 4 consecutive channels) when vec (C % 4 == 0 and x, y and the taps
  // aligned for 4-channel vectors, host-checked), else per (pixel, channel)
  const int cv = vec ? 4 : 1;
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int CG = C / cv;
  const int c0 = int(i % CG) * cv;
  const long long pix = i / CG;
  const int w = int(pix % W), h = int((pix / W) % H);
  const long long f = pix / (size_t(H) * W);
  const int lo = (ks - 1) / 2;
  const TI* xf = x + size_t(f) * H * W * C;
  float acc[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) acc[e] = e < cv ? bias[c0 + e] : 0.0f;
  for (int a = 0; a < ks; ++a) {
    const int hh = h + a - lo;
    if (hh < 0 || hh >= H) continue;
    for (int b2 = 0; b2 < ks; ++b2) {
      const int ww = w + b2 - lo;
      if (ww < 0 || ww >= W) continue;
      const size_t xi = (size_t(hh) * W + ww) * C + c0;
      const float* kt = kw + (a * ks + b2) * C + c0;
      if (cv == 4) {
        const float4 xv = ld4v(xf, xi);
        const float4 kv = *reinterpret_cast<const float4*>(kt);
        acc[0] = fmaf(xv.x, kv.x, acc[0]);
        acc[1] = fmaf(xv.y, kv.y, acc[1]);
        acc[2] = fmaf(xv.z, kv.z, acc[2]);
        acc[3] = fmaf(xv.w, kv.w, acc[3]);
      } else {
        acc[0] = fmaf(ld_f(xf, xi), kt[0], acc[0]);
      }
    }
  }
  const size_t o = size_t(pix) * C + c0;
  for (int e = 0; e < cv; ++e) st_f(y, o + e, acc[e]);
}

// Register-blocked variant for ks in {3, 5, 7}: a thread computes RH rows x 4
// columns x 4 channels, so each input float4 it loads feeds up to RH KS outputs.
// LDSW: the KS x KS x C taps are staged in LDS once per block (C KS^2 <= 8192)
// instead of being read from global memory per output row (C3's 5 x 5 conv:
// 2.9 -> 2.0 ms with 8 rows).  Needs C % 4 == 0, W % 4 == 0, H % RH == 0.  The
// sum per output runs over the taps in the same order for every RH.
constexpr int kDwMaxLdsTaps = 8192;   // floats
// SUM: also the frame's per-channel sums of x (the GDN context's spatial mean, cssm.py:4785): each
// thread adds the inputs at its own output pixels (the centre taps, so every pixel once), the block
// adds its threads' sums in a fixed order into part[(frame, block), C]; needs every block full
// (per_frame % 256 == 0) and C / 4 dividing 256 (host-checked).
template <int KS, int RH, bool LDSW, class TI, class TO, bool SUM = false>
__global__ void __launch_bounds__(256)
dwconv_cl_blocked(const TI* __restrict__ x, int H, int W, int C, const float* __restrict__ kw,
                  const float* __restrict__ bias, TO* __restrict__ y, int per_frame, float* __restrict__ part) {
  constexpr int LO = (KS - 1) / 2, RW = 4, NCOL = RW + KS - 1;
  extern __shared__ float4 kws[];   // LDSW: (KS, KS, C / 4) taps
  __shared__ float4 red[SUM ? 256 : 1];
  const int CG = C / 4, WG = W / RW;
  if constexpr (LDSW) {
    for (int j = int(threadIdx.x); j < KS * KS * CG; j += int(blockDim.x))
      kws[j] = *reinterpret_cast<const float4*>(kw + 4 * j);
    __syncthreads();
  }
  // frame blockIdx.y; (row group, column quad, channel quad) from 32-bit index arithmetic.  The
  // dispatcher deals the blocks of a launch round-robin over the 8 XCDs (each with its own L2), so with
  // a multiple of 8 blocks per frame, XCD k runs blocks k, k + 8, ...: they take the contiguous logical
  // blocks k n / 8 .. (k + 1) n / 8 - 1, whose row groups share their halo rows through that L2
  const int nb = int(gridDim.x), bx = int(blockIdx.x);
  const int blk = nb % 8 == 0 ? (bx % 8) * (nb / 8) + bx / 8 : bx;
  const int i = blk * int(blockDim.x) + int(threadIdx.x);
  if (i >= per_frame) return;
  const int cq = i % CG, c0 = cq * 4;
  const int t1 = i / CG;
  const int w0 = (t1 % WG) * RW;
  const int h0 = (t1 / WG) * RH;
  const size_t f = blockIdx.y;
  const TI* xf = x + f * H * W * C;
  float4 acc[RH][RW];
  float4 cs = make_float4(0.f, 0.f, 0.f, 0.f);   // SUM: this thread's pixels, its 4 channels
  const float4 bv = *reinterpret_cast<const float4*>(bias + c0);
#pragma unroll
  for (int r = 0; r < RH; ++r)
#pragma unroll
    for (int q = 0; q < RW; ++q) acc[r][q] = bv;
#pragma unroll
  for (int ih = 0; ih < RH + KS - 1; ++ih) {          // input rows h0 - LO .. h0 + RH - 1 + (KS - 1 - LO)
    const int hh = h0 - LO + ih;
    if (hh < 0 || hh >= H) continue;
    float4 xin[NCOL];
#pragma unroll
    for (int ic = 0; ic < NCOL; ++ic) {
      const int ww = w0 - LO + ic;
      xin[ic] = (ww >= 0 && ww < W) ? ld4v(xf, (size_t(hh) * W + ww) * C + c0) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    if constexpr (SUM) {
      if (ih >= LO && ih < LO + RH) {   // an output row of this thread: its RW centre inputs
#pragma unroll
        for (int q = 0; q < RW; ++q) {
          cs.x += xin[LO + q].x;
          cs.y += xin[LO + q].y;
          cs.z += xin[LO + q].z;
          cs.w += xin[LO + q].w;
        }
      }
    }
#pragma unroll
    for (int r = 0; r < RH; ++r) {
      const int a = ih - r;                               // tap row of output row h0 + r
      if (a < 0 || a >= KS) continue;
#pragma unroll
      for (int b2 = 0; b2 < KS; ++b2) {
        const float4 kv = LDSW ? kws[(a * KS + b2) * CG + cq]
                               : *reinterpret_cast<const float4*>(kw + (a * KS + b2) * C + c0);
#pragma unroll
        for (int q = 0; q < RW; ++q) {
          const float4 xv = xin[q + b2];
          acc[r][q].x = fmaf(xv.x, kv.x, acc[r][q].x);
          acc[r][q].y = fmaf(xv.y, kv.y, acc[r][q].y);
          acc[r][q].z = fmaf(xv.z, kv.z, acc[r][q].z);
          acc[r][q].w = fmaf(xv.w, kv.w, acc[r][q].w);
        }
      }
    }
  }
  // 4 consecutive channels per store: one 16-byte (f32) or 8-byte (bf16) store
#pragma unroll
  for (int r = 0; r < RH; ++r)
#pragma unroll
    for (int q = 0; q < RW; ++q) st4v(y, ((f * H + h0 + r) * W + w0 + q) * C + c0, acc[r][q]);
  if constexpr (SUM) {
    // every thread of the block is here (no block is partial); thread t holds channel quad t % CG
    red[threadIdx.x] = cs;
    __syncthreads();
    if (int(threadIdx.x) < CG) {
      float4 sum = red[threadIdx.x];
      for (int k = 1; k < 256 / CG; ++k) {
        const float4 v = red[threadIdx.x + k * CG];
        sum.x += v.x;
        sum.y += v.y;
        sum.z += v.z;
        sum.w += v.w;
      }
      *reinterpret_cast<float4*>(part + (f * gridDim.x + blk) * C + 4 * threadIdx.x) = sum;
    }
  }
}

// ctx[f, c] = (sum of the frame's block partials, in block order) / HW
__global__ void __launch_bounds__(256) dw_mean_reduce(const float* __restrict__ part, int nblk, int C, float inv,
                                                      float* __restrict__ ctx) {
  const size_t f = blockIdx.x;
  for (int c = int(threadIdx.x); c < C; c += int(blockDim.x)) {
    float sum = 0.f;
    for (int b = 0; b < nblk; ++b) sum += part[(f * nblk + b) * C + c];
    ctx[f * C + c] = sum * inv;
  }
}

template <int KS, int RH, bool LDSW, class TI, class TO>
static hipError_t run_dwconv_blocked(const void* x, int F, int H, int W, int C, const float* kw, const float* bias,
                                     void* y, float* part, hipStream_t s) {
  const int per_frame = (H / RH) * (W / 4) * (C / 4);
  const size_t shm = LDSW ? size_t(KS) * KS * C * sizeof(float) : 0;
  const dim3 grid(unsigned((per_frame + 255) / 256), unsigned(F));
  if (part)
    hipLaunchKernelGGL((dwconv_cl_blocked<KS, RH, LDSW, TI, TO, true>), grid, dim3(256), shm, s,
                       static_cast<const TI*>(x), H, W, C, kw, bias, static_cast<TO*>(y), per_frame, part);
  else
    hipLaunchKernelGGL((dwconv_cl_blocked<KS, RH, LDSW, TI, TO>), grid, dim3(256), shm, s, static_cast<const TI*>(x),
                       H, W, C, kw, bias, static_cast<TO*>(y), per_frame, part);
  return hipGetLastError();
}

// rows per thread of the blocked kernel: 8 when the taps fit LDS and H % 8 == 0, else 2
static int dwconv_rows(int H, int C, int ks) { return (C * ks * ks <= kDwMaxLdsTaps && H % 8 == 0) ? 8 : 2; }

template <int KS, class TI, class TO>
static hipError_t run_dwconv_rows(const void* x, int F, int H, int W, int C, const float* kw, const float* bias,
                                  void* y, float* part, hipStream_t s) {
  if (C * KS * KS <= kDwMaxLdsTaps) {
    if (dwconv_rows(H, C, KS) == 8) return run_dwconv_blocked<KS, 8, true, TI, TO>(x, F, H, W, C, kw, bias, y, part, s);
    return run_dwconv_blocked<KS, 2, true, TI, TO>(x, F, H, W, C, kw, bias, y, part, s);
  }
  return run_dwconv_blocked<KS, 2, false, TI, TO>(x, F, H, W, C, kw, bias, y, part, s);
}

template <class TI, class TO>
static bool try_dwconv_blocked(const void* x, int F, int H, int W, int C, int ks, const float* kw, const float* bias,
                               void* y, hipStream_t s, hipError_t& e, float* part = nullptr) {
  // float4 loads / stores of 4 channels: 16-byte aligned f32 (8-byte bf16) tensors and 16-byte
  // aligned taps and bias; one frame's work items must fit 32-bit indices and the frames the
  // grid's y dimension (otherwise the general kernel runs)
  const size_t ax = sizeof(TI) * 4, ay = sizeof(TO) * 4;
  if (C % 4 || W % 4 || H % 2 || reinterpret_cast<uintptr_t>(x) % ax || reinterpret_cast<uintptr_t>(y) % ay ||
      reinterpret_cast<uintptr_t>(kw) % 16 || reinterpret_cast<uintptr_t>(bias) % 16 ||
      (long long)H * W * C >= (1LL << 31) || F > 65535)
    return false;
  switch (ks) {
    case 3: e = run_dwconv_rows<3, TI, TO>(x, F, H, W, C, kw, bias, y, part, s); return true;
    case 5: e = run_dwconv_rows<5, TI, TO>(x, F, H, W, C, kw, bias, y, part, s); return true;
    case 7: e = run_dwconv_rows<7, TI, TO>(x, F, H, W, C, kw, bias, y, part, s); return true;
    default: return false;
  }
}

hipError_t launch_depthwise_conv(const void* x, int dtype, int F, int H, int W, int C, int ks, const float* kw,
                                 const float* bias, void* y, int out_dtype, hipStream_t s) {
  hipError_t e = hipSuccess;
  if (dtype == 0 && out_dtype == 0 && try_dwconv_blocked<float, float>(x, F, H, W, C, ks, kw, bias, y, s, e)) return e;
  if (dtype == 0 && out_dtype == 1 && try_dwconv_blocked<float, uint16_t>(x, F, H, W, C, ks, kw, bias, y, s, e)) return e;
  if (dtype == 1 && out_dtype == 0 && try_dwconv_blocked<uint16_t, float>(x, F, H, W, C, ks, kw, bias, y, s, e)) return e;
  if (dtype == 1 && out_dtype == 1 && try_dwconv_blocked<uint16_t, uint16_t>(x, F, H, W, C, ks, kw, bias, y, s, e)) return e;
  const size_t ax = (dtype == 0 ? 4 : 2) * 4, ay = (out_dtype == 0 ? 4 : 2) * 4;
  const int vec = C % 4 == 0 && reinterpret_cast<uintptr_t>(x) % ax == 0 && reinterpret_cast<uintptr_t>(y) % ay == 0 &&
                  reinterpret_cast<uintptr_t>(kw) % 16 == 0;
  const long long total = (long long)F * H * W * (vec ? C / 4 : C);
  const unsigned blocks = unsigned((total + 255) / 256);
  const dim3 g(blocks), b(256);
  if (dtype == 0 && out_dtype == 0)
    hipLaunchKernelGGL((dwconv_cl<float, float>), g, b, 0, s, static_cast<const float*>(x), H, W, C, ks, kw, bias,
                       static_cast<float*>(y), total, vec);
  else if (dtype == 0)
    hipLaunchKernelGGL((dwconv_cl<float, uint16_t>), g, b, 0, s, static_cast<const float*>(x), H, W, C, ks, kw, bias,
                       static_cast<uint16_t*>(y), total, vec);
  else if (out_dtype == 0)
    hipLaunchKernelGGL((dwconv_cl<uint16_t, float>), g, b, 0, s, static_cast<const uint16_t*>(x), H, W, C, ks, kw,
                       bias, static_cast<float*>(y), total, vec);
  else
    hipLaunchKernelGGL((dwconv_cl<uint16_t, uint16_t>), g, b, 0, s, static_cast<const uint16_t*>(x), H, W, C, ks, kw,
                       bias, static_cast<uint16_t*>(y), total, vec);
  return hipGetLastError();
}

// blocks per frame of the depthwise conv with the fused frame mean, 0 where it has no fused form (the
// blocked kernel with every block full and C / 4 dividing 256)
int depthwise_conv_mean_blocks(int F, int H, int W, int C, int ks) {
  if (C % 4 || W % 4 || H % 2 || (ks != 3 && ks != 5 && ks != 7) || (long long)H * W * C >= (1LL << 31) || F > 65535)
    return 0;
  const int CG = C / 4;
  if (256 % CG) return 0;
  const int per_frame = (H / dwconv_rows(H, C, ks)) * (W / 4) * CG;
  return per_frame % 256 ? 0 : per_frame / 256;
}

hipError_t launch_depthwise_conv_mean(const void* x, int dtype, int F, int H, int W, int C, int ks, const float* kw,
                                      const float* bias, void* y, int out_dtype, float* part, float* ctx,
                                      hipStream_t s) {
  const int nblk = depthwise_conv_mean_blocks(F, H, W, C, ks);
  if (!nblk) return hipErrorInvalidValue;
  hipError_t e = hipSuccess;
  bool ran = false;
  if (dtype == 0 && out_dtype == 0) ran = try_dwconv_blocked<float, float>(x, F, H, W, C, ks, kw, bias, y, s, e, part);
  else if (dtype == 0) ran = try_dwconv_blocked<float, uint16_t>(x, F, H, W, C, ks, kw, bias, y, s, e, part);
  else if (out_dtype == 0) ran = try_dwconv_blocked<uint16_t, float>(x, F, H, W, C, ks, kw, bias, y, s, e, part);
  else ran = try_dwconv_blocked<uint16_t, uint16_t>(x, F, H, W, C, ks, kw, bias, y, s, e, part);
  if (!ran) return hipErrorInvalidValue;   // alignment: the caller checks it first
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(dw_mean_reduce, dim3(unsigned(F)), dim3(256), 0, s, part, nblk, C, 1.0f / float(H * W), ctx);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// In place on plane-major qkv (B, T, 3C, HW): causal depthwise conv over T
// (kernel (kt, 1, C) per block, left zero padding) + bias + SiLU (:4763-4780),
// then the input gates on the k and v blocks (:4844-4848):
//   gate_mode 0: none; 1: per pixel, gates (B T, HW) float2 (B_k, B_v);
//   2: per frame, gates (B T) float2; 3: per channel and pixel, gates
//   plane-major (B T, 2C, HW) float (B_k channels then B_v channels).
// kt = 0 skips the convolution and the SiLU (the reference applies SiLU only
// inside the short convolution).  One thread per (b, channel, pixel), T loop
// inside with the last kt - 1 inputs in registers.
// ---------------------------------------------------------------------------
constexpr int kMaxShortConv = 8;

template <int KT, class T, int PX>
__global__ void __launch_bounds__(256)
gdn_qkv_post(T* __restrict__ qkv, int Tn, int C, int HW, GdnShortConv sc, int gate_mode, const void* __restrict__ gates,
             long long total) {
  // one thread per (b, channel, PX pixels): PX = 4 (vector loads) when HW % 4 == 0, else 1
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int HWq = HW / PX;
  const int p = int(i % HWq) * PX;
  const int c3 = int((i / HWq) % (3 * C));
  const int b = int(i / (size_t(HWq) * 3 * C));
  const int blk = c3 / C, c = c3 % C;
  float w[KT > 0 ? KT : 1];
#pragma unroll
  for (int j = 0; j < KT; ++j) w[j] = sc.w[blk][j * C + c];
  const float bt = KT > 0 ? sc.b[blk][c] : 0.0f;
  float hist[KT > 1 ? KT - 1 : 1][PX];   // x_{t-KT+1} .. x_{t-1}
#pragma unroll
  for (int j = 0; j < (KT > 1 ? KT - 1 : 1); ++j)
#pragma unroll
    for (int e = 0; e < PX; ++e) hist[j][e] = 0.0f;
  for (int t = 0; t < Tn; ++t) {
    const size_t fr = size_t(b) * Tn + t;
    const size_t idx = (fr * 3 * C + c3) * HW + p;
    float v[PX];
    if constexpr (PX == 4) {
      const float4 q = ld4v(qkv, idx);
      v[0] = q.x;
      v[1] = q.y;
      v[2] = q.z;
      v[3] = q.w;
    } else {
      v[0] = ld_f(qkv, idx);
    }
    if (KT > 0) {
      float o[PX];
#pragma unroll
      for (int e = 0; e < PX; ++e) o[e] = fmaf(w[KT > 0 ? KT - 1 : 0], v[e], bt);
#pragma unroll
      for (int j = 0; j < KT - 1; ++j)
#pragma unroll
        for (int e = 0; e < PX; ++e) o[e] = fmaf(w[j], hist[j][e], o[e]);
#pragma unroll
      for (int j = 0; j + 1 < KT - 1; ++j)
#pragma unroll
        for (int e = 0; e < PX; ++e) hist[j][e] = hist[j + 1][e];
      if (KT > 1)
#pragma unroll
        for (int e = 0; e < PX; ++e) hist[KT > 1 ? KT - 2 : 0][e] = v[e];
#pragma unroll
      for (int e = 0; e < PX; ++e) v[e] = o[e] * __builtin_amdgcn_rcpf(1.0f + __expf(-o[e]));
    }
    if (blk > 0 && gate_mode != 0) {
      float g[PX];
      if (gate_mode == 1) {
        const float2* gp = static_cast<const float2*>(gates) + fr * HW + p;
#pragma unroll
        for (int e = 0; e < PX; ++e) g[e] = blk == 1 ? gp[e].x : gp[e].y;
      } else if (gate_mode == 2) {
        const float2 gg = static_cast<const float2*>(gates)[fr];
#pragma unroll
        for (int e = 0; e < PX; ++e) g[e] = blk == 1 ? gg.x : gg.y;
      } else {
        const float* gq = static_cast<const float*>(gates) + (fr * 2 * C + size_t(blk - 1) * C + c) * HW + p;
#pragma unroll
        for (int e = 0; e < PX; ++e) g[e] = gq[e];
      }
#pragma unroll
      for (int e = 0; e < PX; ++e) v[e] *= g[e];
    }
#pragma unroll
    for (int e = 0; e < PX; ++e) st_f(qkv, idx + e, v[e]);
  }
}

template <class T, int PX>
static hipError_t run_qkv_post(T* qkv, int B, int Tn, int C, int HW, int kt, const GdnShortConv& sc, int gate_mode,
                               const void* gates, hipStream_t s) {
  const long long total = (long long)B * 3 * C * (HW / PX);
  const dim3 g(unsigned((total + 255) / 256)), b(256);
  switch (kt) {
#define CSSM_KT(K) \
  case K: hipLaunchKernelGGL((gdn_qkv_post<K, T, PX>), g, b, 0, s, qkv, Tn, C, HW, sc, gate_mode, gates, total); break;
    CSSM_KT(0) CSSM_KT(1) CSSM_KT(2) CSSM_KT(3) CSSM_KT(4) CSSM_KT(5) CSSM_KT(6) CSSM_KT(7) CSSM_KT(8)
#undef CSSM_KT
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_gdn_qkv_post(void* qkv, int dtype, int B, int T, int C, int HW, int kt, const GdnShortConv& sc,
                               int gate_mode, const void* gates, hipStream_t s) {
  if (kt > kMaxShortConv) return hipErrorInvalidValue;
  const bool v4 = HW % 4 == 0;
  if (dtype == 0)
    return v4 ? run_qkv_post<float, 4>(static_cast<float*>(qkv), B, T, C, HW, kt, sc, gate_mode, gates, s)
              : run_qkv_post<float, 1>(static_cast<float*>(qkv), B, T, C, HW, kt, sc, gate_mode, gates, s);
  return v4 ? run_qkv_post<uint16_t, 4>(static_cast<uint16_t*>(qkv), B, T, C, HW, kt, sc, gate_mode, gates, s)
            : run_qkv_post<uint16_t, 1>(static_cast<uint16_t*>(qkv), B, T, C, HW, kt, sc, gate_mode, gates, s);
}

}  // namespace cssm
