// Weight- and context-side kernels of the spectral layer (gfx950):
//   * spectral kernel K_hat = rho * F / (1 + |F|), F = rfft2(pad(k))
//   * per-frequency gates from the spatial mean ctx (dense or factored)
//   * spatial mean of a plane-major tensor
// These are small next to the fused scan; they run once per layer call.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "launch.h"

namespace cssm {

// ---------------------------------------------------------------------------
// K_hat (cssm.py:505-529 gated, 4711-4716 GDN; _stable_spectral_magnitude :29-46)
//
// pad rule: K <= H -> zero pad with pad_before = (H-K)//2 (the tap (i,j) lands
// at (i + ph, j + pw)); K > H -> centre crop starting at (K-H)//2.  The DFT of
// the padded plane only needs the K x K (or cropped) taps, evaluated separably
// in double precision.  One block per channel.
// out: (C, H, W/2+1) complex, optionally GOOM-floored (|x| < 1e-7 -> 1e-7+0j).
// ---------------------------------------------------------------------------
__global__ void spectral_kernel_prep(const float* __restrict__ k, int K, int H, int W, float rho,
                                     int squash, int goom_floor, int scan_order, float2* __restrict__ out) {
  extern __shared__ double sm_d[];   // rows x WF complex (re, im)
  const int c = blockIdx.x;
  const int WF = W / 2 + 1;
  // taps that survive: rows [r0, r0+nr) of k land on padded rows [oh, oh+nr)
  // (the host rejects K between H and W, which the reference cannot run either)
  int r0, nr, oh, q0, nq, ow;
  if (K > H || K > W) {   // centre crop of both axes
    r0 = (K - H) / 2; nr = H; oh = 0;
    q0 = (K - W) / 2; nq = W; ow = 0;
  } else {                // zero pad, tap (i, j) -> (i + (H-K)//2, j + (W-K)//2)
    r0 = 0; nr = K; oh = (H - K) / 2;
    q0 = 0; nq = K; ow = (W - K) / 2;
  }
  const float* kc = k + size_t(c) * K * K;
  // stage 1: R[i][v] = sum_j k[i][j] e^{-2 pi i v (j') / W}
  for (int idx = threadIdx.x; idx < nr * WF; idx += blockDim.x) {
    const int i = idx / WF, v = idx % WF;
    double re = 0.0, im = 0.0;
    for (int j = 0; j < nq; ++j) {
      const int jp = j + ow;
      const long long m = (long long)v * jp % W;
      double sn, cs;
      sincospi(2.0 * double(m) / double(W), &sn, &cs);
      const double kv = double(kc[(r0 + i) * K + (q0 + j)]);
      re += kv * cs;
      im -= kv * sn;
    }
    sm_d[2 * idx] = re;
    sm_d[2 * idx + 1] = im;
  }
  __syncthreads();
  // stage 2: F[u][v] = sum_i R[i][v] e^{-2 pi i u (i') / H}, at position
  // (u, p) of the output with v = scan_col(p) in the scan's column order, in
  // the scan's slot khat_pos(u, p)
  for (int idx = threadIdx.x; idx < H * WF; idx += blockDim.x) {
    const int u = idx / WF, v = scan_order ? scan_col(H, W, idx % WF) : idx % WF;
    double re = 0.0, im = 0.0;
    for (int i = 0; i < nr; ++i) {
      const int ip = i + oh;
      const long long m = (long long)u * ip % H;
      double sn, cs;
      sincospi(2.0 * double(m) / double(H), &sn, &cs);
      const double ar = sm_d[2 * (i * WF + v)], ai = sm_d[2 * (i * WF + v) + 1];
      // (ar + i ai)(cs - i sn)
      re += ar * cs + ai * sn;
      im += ai * cs - ar * sn;
    }
    if (squash) {
      const double mag = sqrt(re * re + im * im);
      const double f = double(rho) / (1.0 + mag);
      re *= f;
      im *= f;
    }
    float2 o = make_float2(float(re), float(im));
    if (goom_floor) {
      const float m2 = o.x * o.x + o.y * o.y;
      if (m2 < 1e-14f) o = make_float2(1e-7f, 0.0f);
    }
    out[size_t(c) * H * WF + (scan_order ? khat_pos(H, W, u, idx % WF) : idx)] = o;
  }
}

// ---------------------------------------------------------------------------
// Gates (cssm.py:536-556, _compute_gate :432-441, GOOM shifts :559-567).
// One block per (b, t).  Output per bin (u, v) of the (H, W/2+1) half
// spectrum, at position (u, p) with v = scan_col(H, W, p) (the scan's column
// order), float4 = (exp(-Delta), (Delta + 1e-8) B, 2e-7 (Delta + 1e-8), C * c_scale):
// the decay, the input gain, the input term that replaces (Delta + 1e-8) 2 U B
// when |U B| < 1e-7 (the to_goom floor, at the doubled spectrum 2 U the scan's
// forward transform produces), and the readout gain; where
//   Delta = act(G_delta), act in {softplus, 2*sigmoid, exp(clip(-4, 2))}
//   dense:    G_x[u, v] = ctx . kernel[:, u*WF + v] + bias[u*WF + v]
//   factored: G_x[u, v] = (ctx . kh[:, u] + bh[u]) * (ctx . kw[:, v] + bw[v])
// ---------------------------------------------------------------------------
// GateWeights (launch.h): kd/bd = dense kernel (C, H*WF) / bias (H*WF), or the
// factored row kernel (C, H) / bias (H); kw/bw = factored column kernel (C, WF) / bias (WF).

__device__ __forceinline__ float softplus_f(float x) {
  // jax.nn.softplus = logaddexp(x, 0) = max(x, 0) + log1p(exp(-|x|))
  return fmaxf(x, 0.0f) + log1pf(expf(-fabsf(x)));
}

__device__ __forceinline__ float gate_act(float x, int act) {
  if (act == 1) return 2.0f / (1.0f + expf(-x));            // sigmoid * 2
  if (act == 2) return expf(fminf(fmaxf(x, -4.0f), 2.0f));  // bounded exp
  return softplus_f(x);
}

// ctx of frame f into cx (LDS): read from ctx (F, C), or reduced from the projection's tile sums
// (cp.partial; with cp.ctx also written out).  The first 256 threads reduce exactly as
// ctx_reduce_kernel does, so ctx is the same bit for bit either way.  red: 256 floats of LDS.
// Ends with a barrier.
__device__ __forceinline__ void frame_ctx(const float* __restrict__ ctx, const CtxPartials& cp, int f, int C,
                                          float* cx, float* red) {
  const int tid = threadIdx.x, nt = blockDim.x;
  if (!cp.partial) {
    for (int i = tid; i < C; i += nt) cx[i] = ctx[size_t(f) * C + i];
    __syncthreads();
    return;
  }
  const float inv = 1.0f / float(cp.HW);
  const int G = C <= 128 ? 256 / C : 1;
  if (G > 1) {
    if (tid < 256) {
      const int g = tid / C, c = tid % C;
      red[tid] = g < G ? ctx_tile_sum(cp.partial, f, cp.HW, cp.TM, cp.slots, C, c, g, G) : 0.0f;
    }
    __syncthreads();
    if (tid < C) {
      float sum = 0.0f;
      for (int q = 0; q < G; ++q) sum += red[q * C + tid];
      const float v = sum * inv;
      cx[tid] = v;
      if (cp.ctx) cp.ctx[size_t(f) * C + tid] = v;
    }
  } else {
    for (int c = tid; c < C; c += nt) {
      const float v = ctx_tile_sum(cp.partial, f, cp.HW, cp.TM, cp.slots, C, c, 0, 1) * inv;
      cx[c] = v;
      if (cp.ctx) cp.ctx[size_t(f) * C + c] = v;
    }
  }
  __syncthreads();
}

// The 3 (H + WF) factored row / column products of one frame, fac[g (H + WF) + r] (rows r < H,
// columns H + v) = bias + ctx . kernel column.  Small planes (few products, long C) split each
// product over P threads (channels pc, pc + P, ...) and sum the parts in LDS in order of pc.
// The first KW weights of a thread are loaded by prefetch(), before ctx is ready (they do not
// depend on it), so a frame waits for one memory latency, not two; finish() runs after the
// barrier that publishes cx and ends with one.
template <int KW>
struct GateFactors {
  int nv, P, idx, pc, ws, u0, nr;
  bool mine;
  const float* wc;
  float wr[KW];

  // the row products of rows u0 .. u0 + nr - 1 and all column products: fac[g (nr + WF) + r]
  // (rows r < nr, columns nr + v)
  __device__ __forceinline__ void prefetch(const GateWeights& gw, int C, int H, int WF, int u0_, int nr_) {
    const int nt = blockDim.x, q = threadIdx.x;
    u0 = u0_;
    nr = nr_;
    nv = 3 * (nr + WF);
    P = nv >= nt ? 1 : nt / nv;
    idx = q % nv;
    pc = q / nv;
    mine = q < nv * P;
    const int g = idx / (nr + WF), r = idx % (nr + WF);
    wc = r < nr ? gw.kd[g] + (u0 + r) : gw.kw[g] + (r - nr);
    ws = r < nr ? H : WF;
#pragma unroll
    for (int k = 0; k < KW; ++k) {
      const int c = pc + k * P;
      wr[k] = mine && c < C ? wc[size_t(c) * ws] : 0.0f;
    }
  }

  // part: P * nv floats of LDS (may alias the ctx reduction's scratch)
  __device__ __forceinline__ void finish(const GateWeights& gw, const float* cx, int C, int H, int WF, float* fac,
                                         float* part) const {
    const int nt = blockDim.x, q = threadIdx.x;
    if (mine) {
      float acc = 0.0f;
#pragma unroll
      for (int k = 0; k < KW; ++k) {
        const int c = pc + k * P;
        if (c < C) acc = fmaf(cx[c], wr[k], acc);
      }
#pragma unroll 8
      for (int c = pc + KW * P; c < C; c += P) acc = fmaf(cx[c], wc[size_t(c) * ws], acc);
      part[pc * nv + idx] = acc;
    }
    // products beyond the block's threads (nv > blockDim: one part each, no prefetch)
    for (int i = q + nt; i < nv; i += nt) {
      const int g = i / (nr + WF), r = i % (nr + WF);
      const float* w = r < nr ? gw.kd[g] + (u0 + r) : gw.kw[g] + (r - nr);
      const int s = r < nr ? H : WF;
      float acc = 0.0f;
#pragma unroll 8
      for (int c = 0; c < C; ++c) acc = fmaf(cx[c], w[size_t(c) * s], acc);
      part[i] = acc;
    }
    __syncthreads();
    for (int i = q; i < nv; i += nt) {
      const int g = i / (nr + WF), r = i % (nr + WF);
      float acc = 0.0f;
      for (int p = 0; p < P; ++p) acc += part[p * nv + i];
      fac[i] = acc + (r < nr ? gw.bd[g][u0 + r] : gw.bw[g][r - nr]);
    }
    __syncthreads();
  }
};

// LDS of the gate kernels: cx (C), fac (nv), then max(nv, threads, 256) floats of scratch (the P nv
// parts of any row window: P nv <= threads whenever nv < threads)
__host__ __device__ inline int gate_lds_floats(int C, int H, int W, int nt, bool factored) {
  const int WF = W / 2 + 1, nv = 3 * (H + WF);
  int scratch = nv > nt ? nv : nt;
  if (scratch < 256) scratch = 256;
  return C + (factored ? nv : 0) + (factored ? scratch : 256);
}
// the weights in LDS (WLDS) start at the next 16-byte boundary and take 3 C (H + WF) floats
__host__ __device__ inline int gate_wlds_offset(int C, int H, int W, int nt) {
  return (gate_lds_floats(C, H, W, nt, true) + 3) / 4 * 4;
}

// 512 threads per frame (two frames per CU at up to 128 VGPRs: a 512-frame batch in one pass),
// each thread's weights loaded up front (up to 32 of them: 114 VGPRs)
constexpr int kGateThreads = 512, kGateKW = 32;
// WLDS (factored, the six weight arrays in 64 KB of LDS with 16-byte rows: C % 4 == 0, host-checked):
// the workgroup first copies them into LDS as one run of 16-byte pieces, consecutive threads on
// consecutive pieces, so every load covers whole cache lines; the per-product loads of
// GateFactors touch a line for every few lanes, and at the CSSM-SHViT stages those line requests,
// not the arithmetic, set the kernel's time.  The sums run in the same order either way.
// Few frames (a small batch): each frame's rows are split over gridDim.y workgroups of nr rows
// (blockIdx.y), each computing its rows' products and all column products (the latter in every
// workgroup of the frame) and writing its rows' bins; ctx is written by the first of them.
template <bool FACTORED, bool WLDS>
__global__ void __launch_bounds__(kGateThreads, 4) gated_gates_kernel(const float* __restrict__ ctx, CtxPartials cp, int C,
                                                              int H, int W, int act, GateWeights gw, float c_scale,
                                                              float4* __restrict__ out, int nr_split) {
  constexpr bool factored = FACTORED;
  static_assert(!WLDS || FACTORED, "weights in LDS for the factored products");
  extern __shared__ float sm_f[];
  const int WF = W / 2 + 1;
  const int bt = blockIdx.x;
  const int nbin = H * WF;
  float* cx = sm_f;                                    // C
  float* fac = sm_f + C;                               // 3 (H + WF) factored vectors
  float* scratch = fac + (factored ? 3 * (H + WF) : 0);
  if constexpr (WLDS) {
    const int nt = blockDim.x, tid = threadIdx.x;
    const int nv = 3 * (H + WF);
    const int P = nv >= nt ? 1 : nt / nv;
    // [g][C x H row kernel][C x WF column kernel], 16-byte aligned after the scratch
    float* Ws = sm_f + gate_wlds_offset(C, H, W, nt);
    {
      const int n4h = C * H / 4, n4 = n4h + C * WF / 4;
      float4* W4 = reinterpret_cast<float4*>(Ws);
#pragma unroll 4
      for (int e = tid; e < 3 * n4; e += nt) {
        const int g = e / n4, r = e % n4;
        W4[e] = r < n4h ? reinterpret_cast<const float4*>(gw.kd[g])[r]
                        : reinterpret_cast<const float4*>(gw.kw[g])[r - n4h];
      }
    }
    frame_ctx(ctx, cp, bt, C, cx, scratch);   // (its barrier also publishes the weights)
    const int idx = tid % nv, pc = tid / nv;
    if (tid < nv * P) {
      const int g = idx / (H + WF), r = idx % (H + WF);
      const float* wl = Ws + g * C * (H + WF) + (r < H ? r : C * H + (r - H));
      const int ws = r < H ? H : WF;
      float acc = 0.0f;
#pragma unroll 8
      for (int c = pc; c < C; c += P) acc = fmaf(cx[c], wl[c * ws], acc);
      scratch[pc * nv + idx] = acc;
    }
    for (int i = tid + nt; i < nv; i += nt) {   // products beyond the block's threads (P == 1)
      const int g = i / (H + WF), r = i % (H + WF);
      const float* wl = Ws + g * C * (H + WF) + (r < H ? r : C * H + (r - H));
      const int ws = r < H ? H : WF;
      float acc = 0.0f;
#pragma unroll 8
      for (int c = 0; c < C; ++c) acc = fmaf(cx[c], wl[c * ws], acc);
      scratch[i] = acc;
    }
    __syncthreads();
    for (int i = tid; i < nv; i += nt) {
      const int g = i / (H + WF), r = i % (H + WF);
      float acc = 0.0f;
      for (int p = 0; p < P; ++p) acc += scratch[p * nv + i];
      fac[i] = acc + (r < H ? gw.bd[g][r] : gw.bw[g][r - H]);
    }
    __syncthreads();
    for (int o = threadIdx.x; o < nbin; o += blockDim.x) {
      const int u = o / WF, v = scan_col(H, W, o % WF);
      float gr[3];
      for (int g = 0; g < 3; ++g) gr[g] = fac[g * (H + WF) + u] * fac[g * (H + WF) + H + v];
      const float d = gate_act(gr[0], act), dd = d + 1e-8f;
      out[size_t(bt) * nbin + o] = make_float4(expf(-d), dd * gr[1], dd * 2e-7f, gr[2] * c_scale);
    }
  } else if constexpr (factored) {
    const int u0 = int(blockIdx.y) * nr_split;
    const int nr = H - u0 < nr_split ? H - u0 : nr_split;
    CtxPartials cpb = cp;
    if (blockIdx.y != 0) cpb.ctx = nullptr;
    GateFactors<kGateKW> gf;
    gf.prefetch(gw, C, H, WF, u0, nr);
    frame_ctx(ctx, cpb, bt, C, cx, scratch);
    gf.finish(gw, cx, C, H, WF, fac, scratch);
    for (int o = u0 * WF + threadIdx.x; o < (u0 + nr) * WF; o += blockDim.x) {
      const int ur = o / WF - u0, v = scan_col(H, W, o % WF);
      float gr[3];
      for (int g = 0; g < 3; ++g) gr[g] = fac[g * (nr + WF) + ur] * fac[g * (nr + WF) + nr + v];
      const float d = gate_act(gr[0], act), dd = d + 1e-8f;
      out[size_t(bt) * nbin + o] = make_float4(expf(-d), dd * gr[1], dd * 2e-7f, gr[2] * c_scale);
    }
  } else {
    frame_ctx(ctx, cp, bt, C, cx, scratch);
    for (int o = threadIdx.x; o < nbin; o += blockDim.x) {
      const int bin = (o / WF) * WF + scan_col(H, W, o % WF);
      float gr[3];
      for (int g = 0; g < 3; ++g) {
        float acc = gw.bd[g][bin];
        const float* kk = gw.kd[g] + bin;
#pragma unroll 8
        for (int c = 0; c < C; ++c) acc = fmaf(cx[c], kk[size_t(c) * nbin], acc);
        gr[g] = acc;
      }
      const float d = gate_act(gr[0], act), dd = d + 1e-8f;
      out[size_t(bt) * nbin + o] = make_float4(expf(-d), dd * gr[1], dd * 2e-7f, gr[2] * c_scale);
    }
  }
}

// ---------------------------------------------------------------------------
// Adjoint of the gates (what autodiff of cssm.py:536-567 gives): from dP, the
// gradient of one bin's float4 above, the gradients of the three gate
// pre-activations G_delta, G_B, G_C at that bin:
//   dDelta = -exp(-Delta) dP.x + G_B dP.y + 2e-7 dP.z
//   dG_delta = dDelta act'(G_delta),  dG_B = (Delta + 1e-8) dP.y,  dG_C = c_scale dP.w
// with act' = sigmoid (softplus), 2 s (1 - s) (2*sigmoid), exp on [-4, 2] and 0
// outside (bounded exp; the clip passes the gradient at its bounds).
// dense: out (BT, 3, H*WF) = dG in natural bin order (u * WF + v).
// factored: out (BT, 3, H + WF) = the gradients of the row and column factors,
//   d(ctx.kh + bh)[u] = sum_v dG[u, v] (ctx.kw + bw)[v] and its column twin,
//   in the factors' layout; each sum runs in a fixed order (no atomics).
// The weight, bias and ctx gradients are products of this with ctx / the
// gate kernels over frames (plain GEMMs the caller runs).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float gate_act_grad(float x, int act) {
  if (act == 1) {
    const float s = 1.0f / (1.0f + expf(-x));
    return 2.0f * s * (1.0f - s);
  }
  if (act == 2) return (x >= -4.0f && x <= 2.0f) ? expf(x) : 0.0f;
  return 1.0f / (1.0f + expf(-x));                            // softplus' = sigmoid
}

__device__ __forceinline__ void gate_bin_grad(const float4 dp, const float gr[3], int act, float c_scale,
                                              float dg[3]) {
  const float d = gate_act(gr[0], act);
  const float dd = fmaf(-expf(-d), dp.x, fmaf(gr[1], dp.y, 2e-7f * dp.z));
  dg[0] = dd * gate_act_grad(gr[0], act);
  dg[1] = (d + 1e-8f) * dp.y;
  dg[2] = c_scale * dp.w;
}

__global__ void __launch_bounds__(1024) gated_gates_bwd_kernel(const float* __restrict__ ctx, int C, int H, int W,
                                                               int factored, int act, GateWeights gw, float c_scale,
                                                               const float4* __restrict__ dgates,
                                                               float* __restrict__ out) {
  extern __shared__ float sm_f[];
  const int WF = W / 2 + 1;
  const int bt = blockIdx.x;
  const int nbin = H * WF;
  const float4* dp = dgates + size_t(bt) * nbin;
  if (!factored) {
    float* cx = sm_f;
    for (int i = threadIdx.x; i < C; i += blockDim.x) cx[i] = ctx[size_t(bt) * C + i];
    __syncthreads();
    float* o3 = out + size_t(bt) * 3 * nbin;
    for (int o = threadIdx.x; o < nbin; o += blockDim.x) {
      const int bin = (o / WF) * WF + scan_col(H, W, o % WF);
      float gr[3];
      for (int g = 0; g < 3; ++g) {
        float acc = gw.bd[g][bin];
        const float* kk = gw.kd[g] + bin;
#pragma unroll 8
        for (int c = 0; c < C; ++c) acc = fmaf(cx[c], kk[size_t(c) * nbin], acc);
        gr[g] = acc;
      }
      float dg[3];
      gate_bin_grad(dp[o], gr, act, c_scale, dg);
      for (int g = 0; g < 3; ++g) o3[size_t(g) * nbin + bin] = dg[g];
    }
    return;
  }
  const int nv = 3 * (H + WF);
  float* cx = sm_f;                                  // C
  float* fac = cx + C;                               // nv factors
  float* scratch = fac + nv;                         // parts while the factors are built
  float* colp = sm_f + gate_lds_floats(C, H, W, int(blockDim.x), true);   // S * WF * 3 column partial sums
  {
    GateFactors<16> gf;
    gf.prefetch(gw, C, H, WF, 0, H);
    frame_ctx(ctx, CtxPartials{nullptr, 0, 0, 0, nullptr}, bt, C, cx, scratch);
    gf.finish(gw, cx, C, H, WF, fac, scratch);
  }
  float* o3 = out + size_t(bt) * nv;
  // rows: wave w takes rows w, w + nwaves, ...; its lanes walk the row's positions
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, nw = int(blockDim.x) >> 6;
  for (int u = wv; u < H; u += nw) {
    float acc[3] = {0.0f, 0.0f, 0.0f};
    for (int pos = lane; pos < WF; pos += 64) {
      const int v = scan_col(H, W, pos);
      float gr[3], dg[3];
      for (int g = 0; g < 3; ++g) gr[g] = fac[g * (H + WF) + u] * fac[g * (H + WF) + H + v];
      gate_bin_grad(dp[u * WF + pos], gr, act, c_scale, dg);
      for (int g = 0; g < 3; ++g) acc[g] = fmaf(dg[g], fac[g * (H + WF) + H + v], acc[g]);
    }
    for (int g = 0; g < 3; ++g)
      for (int off = 32; off > 0; off >>= 1) acc[g] += __shfl_xor(acc[g], off, 64);
    if (lane == 0)
      for (int g = 0; g < 3; ++g) o3[g * (H + WF) + u] = acc[g];
  }
  // columns: thread (s, pos) sums rows s, s + S, ... of position pos; the S parts
  // of each column then add up in order of s
  const int S = int(blockDim.x) / WF;
  if (int(threadIdx.x) < S * WF) {
    const int pos = threadIdx.x % WF, s = threadIdx.x / WF;
    const int v = scan_col(H, W, pos);
    float acc[3] = {0.0f, 0.0f, 0.0f};
    for (int u = s; u < H; u += S) {
      float gr[3], dg[3];
      for (int g = 0; g < 3; ++g) gr[g] = fac[g * (H + WF) + u] * fac[g * (H + WF) + H + v];
      gate_bin_grad(dp[u * WF + pos], gr, act, c_scale, dg);
      for (int g = 0; g < 3; ++g) acc[g] = fmaf(dg[g], fac[g * (H + WF) + u], acc[g]);
    }
    for (int g = 0; g < 3; ++g) colp[(size_t(s) * WF + v) * 3 + g] = acc[g];
  }
  __syncthreads();
  for (int q = threadIdx.x; q < 3 * WF; q += blockDim.x) {
    const int g = q / WF, v = q % WF;
    float acc = 0.0f;
    for (int s = 0; s < S; ++s) acc += colp[(size_t(s) * WF + v) * 3 + g];
    o3[g * (H + WF) + H + v] = acc;
  }
}

// ---------------------------------------------------------------------------
// mean over (H, W) of each plane of a plane-major tensor (cssm.py:536),
// optionally after SiLU; bf16 or f32 input.  Planes of up to 1024 samples
// share a 256-thread block (16-64 lanes each); larger ones get a block each.
// ---------------------------------------------------------------------------
template <class TIN>
__device__ __forceinline__ float load_as_f32(const TIN* p, size_t i);
template <>
__device__ __forceinline__ float load_as_f32<float>(const float* p, size_t i) { return p[i]; }
template <>
__device__ __forceinline__ float load_as_f32<uint16_t>(const uint16_t* p, size_t i) {
  return __uint_as_float(uint32_t(p[i]) << 16);
}

template <class TIN>
__global__ void plane_mean_kernel(const TIN* __restrict__ x, long long nplanes, int HW, int L, int act,
                                  float* __restrict__ out) {
  // L lanes per plane (a power of two <= 64 dividing the wave, or the whole
  // 256-thread block when L == 256): small planes share a block
  __shared__ float red[4];
  const int per = int(blockDim.x) / L;
  const int sub = int(threadIdx.x) / L, li = int(threadIdx.x) % L;
  const long long plane = (long long)blockIdx.x * per + sub;
  float acc = 0.0f;
  if (plane < nplanes) {
    const size_t base = size_t(plane) * HW;
    for (int i = li; i < HW; i += L) {
      float v = load_as_f32<TIN>(x, base + i);
      if (act == 1) v = v / (1.0f + expf(-v));
      acc += v;
    }
  }
  const int width = L < 64 ? L : 64;
  for (int off = width / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if (L <= 64) {
    if (li == 0 && plane < nplanes) out[plane] = acc / float(HW);
    return;
  }
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  if (lane == 0) red[wid] = acc;
  __syncthreads();
  if (threadIdx.x == 0 && plane < nplanes) out[plane] = ((red[0] + red[1]) + (red[2] + red[3])) / float(HW);
}

// ----------------------------------------------------------------- launchers

hipError_t launch_spectral_kernel(const float* k, int C, int K, int H, int W, float rho, int squash,
                                  int goom_floor, int scan_order, float2* khat, hipStream_t s) {
  const int WF = W / 2 + 1;
  const int rows = (K > H || K > W) ? H : K;
  const size_t shm = size_t(rows) * WF * 2 * sizeof(double);
  if (shm > 64 * 1024) return hipErrorInvalidValue;
  hipLaunchKernelGGL(spectral_kernel_prep, dim3(C), dim3(256), shm, s, k, K, H, W, rho, squash,
                     goom_floor, scan_order, khat);
  return hipGetLastError();
}

hipError_t launch_plane_mean(const void* x, int dtype, long long nplanes, int HW, int act, float* out,
                             hipStream_t s) {
  if (nplanes <= 0) return hipSuccess;
  // lanes per plane: about 4 elements per lane, 16 .. 64 lanes, or the whole block for large planes
  int L = 16;
  while (L < 64 && L * 4 < HW) L *= 2;
  if (HW > 64 * 16) L = 256;
  const long long blocks = (nplanes + 256 / L - 1) / (256 / L);
  if (dtype == 0)
    hipLaunchKernelGGL(plane_mean_kernel<float>, dim3(unsigned(blocks)), dim3(256), 0, s,
                       static_cast<const float*>(x), nplanes, HW, L, act, out);
  else
    hipLaunchKernelGGL(plane_mean_kernel<uint16_t>, dim3(unsigned(blocks)), dim3(256), 0, s,
                       static_cast<const uint16_t*>(x), nplanes, HW, L, act, out);
  return hipGetLastError();
}

hipError_t launch_gated_gates(const float* ctx, const CtxPartials& cp, int BT, int C, int H, int W, int factored,
                              int act, const GateWeights& w, float c_scale, float4* gates, hipStream_t s) {
  // the factored products split over P = threads / nv threads each, which keeps each thread's
  // chain of dependent FMAs at C / P (latency, not arithmetic, bounds it)
  constexpr int NT = kGateThreads;
  const size_t shm = size_t(gate_lds_floats(C, H, W, NT, factored != 0)) * sizeof(float);
  if (shm > 64 * 1024) return hipErrorInvalidValue;
  if (factored) {
    // the weights through LDS where they fit with 16-byte rows
    const int WF = W / 2 + 1;
    const size_t shm_w = (size_t(gate_wlds_offset(C, H, W, NT)) + size_t(3) * C * (H + WF)) * sizeof(float);
    bool wlds = C % 4 == 0 && shm_w <= 64 * 1024;
    for (int g = 0; g < 3; ++g)
      wlds = wlds && (reinterpret_cast<uintptr_t>(w.kd[g]) % 16) == 0 && (reinterpret_cast<uintptr_t>(w.kw[g]) % 16) == 0;
    if (wlds) {
      hipLaunchKernelGGL((gated_gates_kernel<true, true>), dim3(BT), dim3(NT), shm_w, s, ctx, cp, C, H, W, act, w,
                         c_scale, gates, H);
    } else {
      // fewer frames than two per CU: split each frame's rows over more workgroups
      int dev = 0, cus = 256;
      if (hipGetDevice(&dev) != hipSuccess ||
          hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        cus = 256;
      int splits = BT < 2 * cus ? (2 * cus + BT - 1) / BT : 1;
      if (splits > H) splits = H;
      const int nr = (H + splits - 1) / splits;
      splits = (H + nr - 1) / nr;
      hipLaunchKernelGGL((gated_gates_kernel<true, false>), dim3(BT, splits), dim3(NT), shm, s, ctx, cp, C, H, W,
                         act, w, c_scale, gates, nr);
    }
  } else {
    hipLaunchKernelGGL((gated_gates_kernel<false, false>), dim3(BT), dim3(NT), shm, s, ctx, cp, C, H, W, act, w,
                       c_scale, gates, H);
  }
  return hipGetLastError();
}

hipError_t launch_gated_gates_bwd(const float* ctx, int BT, int C, int H, int W, int factored, int act,
                                  const GateWeights& w, float c_scale, const float4* dgates, float* out,
                                  hipStream_t s) {
  const int WF = W / 2 + 1;
  constexpr int NT = 1024;
  if (factored && WF > NT) return hipErrorInvalidValue;
  const int S = NT / WF;
  const size_t shm = (size_t(gate_lds_floats(C, H, W, NT, factored != 0)) +
                      (factored ? size_t(S) * WF * 3 : 0)) * sizeof(float);
  if (shm > 64 * 1024) return hipErrorInvalidValue;
  hipLaunchKernelGGL(gated_gates_bwd_kernel, dim3(BT), dim3(NT), shm, s, ctx, C, H, W, factored, act, w,
                     c_scale, dgates, out);
  return hipGetLastError();
}

}  // namespace cssm
