// Projection GEMMs of the spectral layer on fp32 MFMA (gfx950), with the
// layout change between the reference's channels-last tensors and the scan's
// plane-major planes fused into the GEMM:
//   proj_in : X (M, K) channels-last  ->  two plane-major outputs (the two
//             halves of the N output channels), bias, optional SiLU on each
//             half, optional per-tile channel sums of the first half (the
//             spatial mean ctx), cssm.py:480-484 + :502 + :536 + :581.
//   proj_out: Y plane-major (F, K, HW) ->  out (M, N) channels-last, bias,
//             cssm.py:584.
// M = F * HW rows (F frames of HW pixels).  fp32 accumulation throughout.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "launch.h"

namespace cssm {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// fp32 -> three bf16 parts x1 + x2 + x3 = x to ~2^-27 relative (each rounds to nearest even)
__device__ __forceinline__ void split3_bf16(float x, __bf16& x1, __bf16& x2, __bf16& x3) {
  x1 = (__bf16)x;
  const float r = x - (float)x1;
  x2 = (__bf16)r;
  x3 = (__bf16)(r - (float)x2);
}

__device__ __forceinline__ float ld_el(const float* p, size_t i) { return p[i]; }
__device__ __forceinline__ float ld_el(const uint16_t* p, size_t i) { return __uint_as_float(uint32_t(p[i]) << 16); }
__device__ __forceinline__ void st_el(float* p, size_t i, float v) { p[i] = v; }
__device__ __forceinline__ void st_el(uint16_t* p, size_t i, float v) {
  uint32_t x = __float_as_uint(v);
  if ((x & 0x7f800000u) == 0x7f800000u) {
    p[i] = uint16_t((x >> 16) | ((x & 0x007fffffu) ? 0x40u : 0u));
  } else {
    x += 0x7fffu + ((x >> 16) & 1u);
    p[i] = uint16_t(x >> 16);
  }
}
__device__ __forceinline__ float silu_acc(float x) { return x / (1.0f + expf(-x)); }
// epilogue activation: 0 identity, 1 SiLU, 2 sigmoid
__device__ __forceinline__ float act_acc(float x, int act) {
  if (act == 1) return silu_acc(x);
  if (act == 2) return 1.0f / (1.0f + expf(-x));
  return x;
}
// orders one wave's LDS accesses across its lanes (the region is private to the wave)
__device__ __forceinline__ void wave_fence() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}
// buffer resource over [p, p + bytes): raw buffer loads beyond it return 0
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, int(bytes), 0x00020000);
}
// 4 consecutive elements at a 4-element-aligned index
__device__ __forceinline__ float4 ld4(const float* p, size_t i) { return *reinterpret_cast<const float4*>(p + i); }
__device__ __forceinline__ float4 ld4(const uint16_t* p, size_t i) {
  const uint2 v = *reinterpret_cast<const uint2*>(p + i);
  return make_float4(__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xffff0000u), __uint_as_float(v.y << 16),
                     __uint_as_float(v.y & 0xffff0000u));
}
__device__ __forceinline__ void st4(float* p, size_t i, const float* v) {
  *reinterpret_cast<float4*>(p + i) = make_float4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ void st4(uint16_t* p, size_t i, const float* v) {
  for (int r = 0; r < 4; ++r) st_el(p, i + r, v[r]);
}
// bf16 bits of v with st_el's rounding
__device__ __forceinline__ uint32_t bf16_bits(float v) {
  uint32_t x = __float_as_uint(v);
  if ((x & 0x7f800000u) == 0x7f800000u) return (x >> 16) | ((x & 0x007fffffu) ? 0x40u : 0u);
  x += 0x7fffu + ((x >> 16) & 1u);
  return x >> 16;
}
// 4 consecutive elements at byte offset off of a buffer resource; an offset past the
// resource's range drops the store
__device__ __forceinline__ void bst4(__amdgpu_buffer_rsrc_t r, unsigned off, const float* v, float*) {
  typedef unsigned u4 __attribute__((ext_vector_type(4)));
  const u4 w = {__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3])};
  __builtin_amdgcn_raw_buffer_store_b128(w, r, off, 0, 0);
}
__device__ __forceinline__ void bst4(__amdgpu_buffer_rsrc_t r, unsigned off, const float* v, uint16_t*) {
  typedef unsigned u2 __attribute__((ext_vector_type(2)));
  const u2 w = {bf16_bits(v[0]) | (bf16_bits(v[1]) << 16), bf16_bits(v[2]) | (bf16_bits(v[3]) << 16)};
  __builtin_amdgcn_raw_buffer_store_b64(w, r, off, 0, 0);
}

// Block tile TM rows x TN output channels, K staged through LDS in chunks of
// KC.  Wave layout WMW x WNW waves, each owning (TM / WMW) x (TN / WNW)
// outputs as 16x16 MFMA tiles (v_mfma_f32_16x16x4f32: lane l holds
// A[l % 16][l / 16], B[l / 16][l % 16] and D rows 4 (l / 16) .. +3 of column l % 16).
template <int TM, int TN, int WMW, int WNW>
struct ProjTile {
  static constexpr int KC = 32;
  static constexpr int NT = 64 * WMW * WNW;
  static constexpr int MT = TM / WMW / 16, NTL = TN / WNW / 16;   // 16x16 tiles per wave
  static constexpr int AP = KC + 1;     // A tile row pitch (rows = TM), padded
  static constexpr int BP = TN + 4;     // B tile row pitch (rows = KC)
};

// ---------------------------------------------------------------------------
// proj_in: out_lo[f][c][p] = act_lo(sum_k X[f*HW+p][k] W[k][c] + b[c]),   c < NH
//          out_hi[f][c][p] = act_hi(... c + NH ...),                      NH <= c < N
// (NH = N/2 for the in_proj split; NH = N writes one plane-major tensor)
// partial (optional): partial[tile][c] = sum over the tile's rows of out_lo
// (requires HW % TM == 0 so a tile lies in one frame).
// ---------------------------------------------------------------------------
template <int TM, int TN, int WMW, int WNW, class TI, class TO>
__global__ void __launch_bounds__(64 * WMW * WNW)
proj_in_kernel(const TI* __restrict__ X, int M, int K, int N, const float* __restrict__ Wt,
               const float* __restrict__ bias, int HW, TO* __restrict__ out_lo, TO* __restrict__ out_hi,
               int act_lo, int act_hi, float* __restrict__ partial, int NH) {
  using P = ProjTile<TM, TN, WMW, WNW>;
  __shared__ float As[TM * P::AP];
  __shared__ float Bs[P::KC * P::BP];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WNW, wn = wave % WNW;
  const int m0 = blockIdx.x * TM, n0 = blockIdx.y * TN;
  const int NL = N - NH;   // channels of out_hi

  floatx4 acc[P::MT][P::NTL];
#pragma unroll
  for (int i = 0; i < P::MT; ++i)
#pragma unroll
    for (int j = 0; j < P::NTL; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  for (int k0 = 0; k0 < K; k0 += P::KC) {
    // stage A (TM x KC) and B (KC x TN); zero-fill outside the matrix
    for (int i = tid; i < TM * P::KC; i += P::NT) {
      const int r = i / P::KC, kk = i % P::KC;
      const int gm = m0 + r, gk = k0 + kk;
      As[r * P::AP + kk] = (gm < M && gk < K) ? ld_el(X, size_t(gm) * K + gk) : 0.0f;
    }
    for (int i = tid; i < P::KC * TN; i += P::NT) {
      const int kk = i / TN, c = i % TN;
      const int gk = k0 + kk, gn = n0 + c;
      Bs[kk * P::BP + c] = (gk < K && gn < N) ? Wt[size_t(gk) * N + gn] : 0.0f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < P::KC; kk += 4) {
      float a[P::MT], b[P::NTL];
#pragma unroll
      for (int i = 0; i < P::MT; ++i)
        a[i] = As[((wm * P::MT + i) * 16 + (lane & 15)) * P::AP + kk + (lane >> 4)];
#pragma unroll
      for (int j = 0; j < P::NTL; ++j) b[j] = Bs[(kk + (lane >> 4)) * P::BP + (wn * P::NTL + j) * 16 + (lane & 15)];
#pragma unroll
      for (int i = 0; i < P::MT; ++i)
#pragma unroll
        for (int j = 0; j < P::NTL; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
  }

  // epilogue: lane holds rows 4 (lane / 16) + r of column lane % 16 of each
  // tile; with HW % 4 == 0 those 4 rows are 4 consecutive pixels of one plane.
  static_assert(WMW == 1, "proj_in keeps a whole row tile per wave (channel sums stay in-wave)");
  const bool vec = (HW % 4) == 0;
#pragma unroll
  for (int j = 0; j < P::NTL; ++j) {
    const int gn = n0 + (wn * P::NTL + j) * 16 + (lane & 15);
    const bool nok = gn < N;
    const float bv = nok ? bias[gn] : 0.0f;
    const bool lo = gn < NH;
    const int c = lo ? gn : gn - NH;
    const int NC = lo ? NH : NL;
    TO* dst = lo ? out_lo : out_hi;
    const int act = lo ? act_lo : act_hi;
    float csum = 0.0f;
#pragma unroll
    for (int i = 0; i < P::MT; ++i) {
      const int gm0 = m0 + (wm * P::MT + i) * 16 + (lane >> 4) * 4;
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] = act_acc(acc[i][j][r] + bv, act);
      if (nok && vec && gm0 + 3 < M) {
        const int f = gm0 / HW, p = gm0 % HW;
        st4(dst, (size_t(f) * NC + c) * HW + p, v);
        csum += (v[0] + v[1]) + (v[2] + v[3]);
      } else if (nok) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int gm = gm0 + r;
          if (gm < M) {
            const int f = gm / HW, p = gm % HW;
            st_el(dst, (size_t(f) * NC + c) * HW + p, v[r]);
            csum += v[r];
          }
        }
      }
    }
    if (partial != nullptr && lo) {
      // the wave holds all TM rows of the tile: reduce the 4 row groups
      csum += __shfl_xor(csum, 16, 64);
      csum += __shfl_xor(csum, 32, 64);
      if (lane < 16 && nok) partial[size_t(blockIdx.x) * NH + c] = csum;
    }
  }
}

// ctx[f][c] = sum over the row tiles t of TM rows that overlap frame f of
// partial[t][f - first frame of t][c], / HW.  One block per frame: with C <= 128
// the 256 threads split the frame's tiles into G = 256 / C strided groups (each
// summed in tile order, loads unrolled so several are in flight), and the group
// sums add in group order; wider C loops over channels with one group.  The
// order is fixed, so ctx is deterministic.
__global__ void __launch_bounds__(256) ctx_reduce_kernel(const float* __restrict__ partial, int F, int HW, int TM,
                                                         int slots, int C, float* __restrict__ ctx) {
  __shared__ float red[256];
  const int f = blockIdx.x, tid = threadIdx.x;
  const int G = C <= 128 ? 256 / C : 1;
  const int g = tid / C;   // (C <= 128: tid < G C covers every thread of the block)
  if (G > 1) {
    const int c = tid % C;
    red[tid] = g < G ? ctx_tile_sum(partial, f, HW, TM, slots, C, c, g, G) : 0.0f;
    __syncthreads();
    if (tid < C) {
      float s = 0.0f;
      for (int q = 0; q < G; ++q) s += red[q * C + tid];
      ctx[size_t(f) * C + tid] = s * (1.0f / float(HW));
    }
  } else {
    for (int c = tid; c < C; c += 256)
      ctx[size_t(f) * C + c] = ctx_tile_sum(partial, f, HW, TM, slots, C, c, 0, 1) * (1.0f / float(HW));
  }
}

// ---------------------------------------------------------------------------
// Persistent small-K GEMM (K <= KMAX, the layer's projections): the weight
// block (K x 128 columns) stays in LDS for the whole launch; each workgroup
// walks 128-row tiles, prefetching the next tile's A rows into registers while
// the MFMAs run on the current one.  Four waves split the 128 columns (32
// each) and keep all 128 rows, so every per-channel reduction stays in-wave.
//   PLANE_A = false: A is channels-last (M, K) rows; true: A is plane-major
//   (F, K, HW) (the scan output).  OUT_SPLIT = true: plane-major output,
//   channels [0, NH) to out_lo and [NH, N) to out_hi, each with its
//   activation, plus channel sums of out_lo (proj_in; NH = N writes a single
//   tensor); false: channels-last (M, N) (proj_out).
//   SPLIT: the product runs on bf16 MFMA (v_mfma_f32_16x16x32_bf16) with both
//   operands split into three bf16 parts (A = A1 + A2 + A3, |A2| <= 2^-9 |A|,
//   |A3| <= 2^-18 |A|) and the six products down to order 2^-18 kept:
//   A1 B1 + A1 B2 + A2 B1 + A1 B3 + A2 B2 + A3 B1, fp32 accumulation.  The
//   dropped terms are O(2^-27): fp32-level results at ~2.7x the fp32 MFMA
//   rate (the fp32 path is MFMA-bound at K = 64).  A is split once when it is
//   staged in LDS (three bf16 planes, k contiguous per row); the weight
//   fragments of the wave's 32 columns are split once per launch and stay in
//   VGPRs.
//   NORM (PLANE_A only): before the product, each pixel's K-vector is
//   normalised across channels (norm 1: RMSNorm x rsqrt(mean x^2 + 1e-6) s_k;
//   2: LayerNorm (x - mean) rsqrt(var + 1e-6) s_k + b_k; 0: none) and
//   multiplied by the matching pixel of the plane-major gate G -- the GDN
//   output path, cssm.py:5026-5031 and :5126, feeding output_proj :5141.
//   At K <= 64 on whole 4-pixel runs the product is the split-bf16 one too
//   (NSPLIT): the gate planes are prefetched in the MFMA output layout, the
//   norm x gate is evaluated in that layout and written as three bf16 planes
//   over the fp32 staging; elsewhere (K = 128, element-wise planes, XG) A is
//   normalised in place and the product runs on fp32 MFMA.
//   XG (with NORM): the gate is not read but computed in the kernel from the
//   layer input, G = act(X Wg + bg) (gate_proj, cssm.py:4853-4859), X the
//   tile's channels-last bf16 rows staged in LDS next to A, on bf16 MFMA with
//   Wg split into three bf16 parts (X is exactly its one part), then applied
//   with the norm in the MFMA output layout.  XF: fp32 X, each lane's
//   fragments (8 channels of one row, 32 bytes) loaded straight from the rows
//   into registers (no LDS: a staged fp32 tile would leave room for one
//   workgroup per CU) and split into three bf16 parts, six products.
// ---------------------------------------------------------------------------
struct NormGate {
  const void* G;        // plane-major (F, K, HW) gate, same dtype as A
  const float* scale;   // (K) or nullptr
  const float* shift;   // (K) or nullptr (LayerNorm bias)
  int kind;             // 0 none, 1 rms, 2 layer
  const uint16_t* X;    // XG: channels-last (M, K) bf16 layer input
  const float* Xf;      // XG with XF: the same in fp32
  const float* wg;      // XG: (K, K) gate_proj kernel
  const float* bg;      // XG: (K) its bias
  int gact;             // XG: 1 SiLU, 2 sigmoid
};

// GDN qkv epilogue (TT > 0; the tiled kernel, for the shapes the frame-sequential
// qkv_fseq_kernel does not take: H*W not a multiple of 64): the causal short
// convolution over T, SiLU and the input gates of cssm.py:4763-4780 / :4844-4848,
// in the operation order of gdn_qkv_post, on tiles of 128 / TT pixels x TT
// consecutive frames of one batch element (tile row r = t * (128 / TT) + pixel),
// so each lane holds the frames of its pixels (TT = 4 or 8).  The taps on frames t .. t - 3 are applied (kt <= 4,
// or T <= 4 where earlier taps only meet the zero padding).  T > TT (TT = 8)
// runs as T / 8 chunks of the same pixels, in order on one workgroup, the last
// 3 frames of each chunk kept in LDS for the next.  Output (B, T, N = 3C, HW)
// plane-major.
struct QkvPost {
  const float* w[3];     // (kt, C) per q / k / v block
  const float* b[3];     // (C)
  int kt;                // 0: no convolution and no SiLU
  int gate_mode;         // as cssm_gdn_qkv_post (0 none, 1 per pixel, 2 per frame, 3 per channel and pixel)
  const void* gates;
  int T;                 // frames per batch element (a multiple of TT)
  // gate_proj on the same rows (ng = C, else 0): kernel columns N .. N + C - 1 are
  // x wg + bg with SiLU (gact 1) or sigmoid (gact 2), no convolution and no input
  // gate, written plane-major to gv (B, T, C, HW) in the output dtype
  const float* wg;       // (K, C)
  const float* bg;       // (C)
  int ng;
  int gact;
  void* gv;
};

template <int KMAX, bool PLANE_A, bool OUT_SPLIT, int WN, class TI, class TO, bool NORM = false, bool SPLIT = false,
          int TT = 0, bool CARRY = false, bool PX1 = false, bool XG = false, bool XF = false>
__global__ void __launch_bounds__(256, 2)
proj_persist_kernel(const TI* __restrict__ A, int M, int K, int N, const float* __restrict__ Wt,
                    const float* __restrict__ bias, int HW, TO* __restrict__ out_lo, TO* __restrict__ out_hi,
                    int act_lo, int act_hi, float* __restrict__ partial, int NH, NormGate ng, QkvPost qp) {
  // WN waves along the TN = 32 WN columns, WM = 4 / WN along the TM = 128 rows;
  // a wave owns (128 / WM) rows x 32 columns = MI x 2 MFMA tiles
  constexpr int TM = 128, TN = 32 * WN, NT = 256, WM = 4 / WN, MI = TM / WM / 16;
  // plane-major outputs with WM > 1 (narrow N) come without channel sums (partial == nullptr, host-checked):
  // the sums need whole row tiles per wave
  static_assert(!OUT_SPLIT || WM == 1 || TT == 0, "the qkv epilogue needs whole row tiles per wave");
  static_assert(!NORM || (PLANE_A && !OUT_SPLIT), "the norm / gate prologue is for plane-major A");
  static_assert(!PX1 || NORM, "element-wise plane rows only for the norm / gate prologue");
  static_assert(!(NORM && SPLIT), "the norm / gate prologue splits A itself (NSPLIT), after the norm");
  // NORM at K <= 64 on whole 4-pixel runs (NSPLIT): the product runs on bf16 MFMA as well; the normalised
  // and gated A is split into three bf16 planes after the norm, over the fp32 staging (K = 128, and the
  // element-wise planes, keep the fp32 MFMA product)
  constexpr bool NSPLIT = NORM && KMAX == 64 && !PX1 && !XG;
  constexpr bool MSPLIT = SPLIT || NSPLIT;   // the product on split-bf16 MFMA, weight fragments in VGPRs
  static_assert(!XG || (NORM && KMAX == 64 && !PX1 && WN == 2), "computed gate: K <= 64 channels, N <= 64 columns");
  static_assert(!XF || XG, "fp32 x for the computed gate");
  static_assert(!SPLIT || KMAX % 32 == 0, "bf16 MFMA k-blocks of 32");
  constexpr int AP = PLANE_A ? (TM + 16) : (KMAX + 2);   // pitch: rows of A (row-major) or k-rows (plane)
  constexpr int BP = TN + 16;
  constexpr int KP = KMAX + 8;                            // SPLIT: bf16 pitch of the k-contiguous rows
  constexpr int KB = KMAX / 32;                           // SPLIT: bf16 MFMA k-blocks
  // SPLIT with bf16 A: A is exactly its first bf16 part, so one plane and three products
  constexpr bool A1_ONLY = SPLIT && sizeof(TI) == 2;
  constexpr int APL = A1_ONLY ? 1 : 3;
  constexpr int A_STAGE = SPLIT ? APL * TM * KP / 2 : (PLANE_A ? KMAX * AP : TM * AP);   // SPLIT: APL bf16 planes
  constexpr int A_FLOATS = (NSPLIT && 3 * TM * KP / 2 > A_STAGE) ? 3 * TM * KP / 2 : A_STAGE;   // NSPLIT: + 3 planes
  constexpr int OP = TN + 4;                              // output staging pitch (channels-last out)
  constexpr int AS_FLOATS = (!OUT_SPLIT && TM * OP > A_FLOATS) ? TM * OP : A_FLOATS;  // staging reuses As
  constexpr int PF = TM * KMAX / 4 / NT;                 // float4 of A prefetched per thread
  __shared__ __attribute__((aligned(16))) float As[AS_FLOATS];
  __shared__ __attribute__((aligned(16))) float Bs[MSPLIT ? 1 : KMAX * BP];
  // SPLIT views: the three A planes [TM][KP] as bf16
  __bf16* const A1 = reinterpret_cast<__bf16*>(As);
  __bf16* const A2 = A1 + TM * KP;   // (SPLIT, fp32 A only)
  __bf16* const A3 = A2 + TM * KP;
  __shared__ float rowsc[NORM ? 2 * NT : 1];             // per-pixel partial sums, then (scale, mean) of the norm
  __shared__ float nss[NORM ? 2 * KMAX : 1];             // the norm's per-channel scale and shift
  __shared__ __attribute__((aligned(16))) __bf16 Xs[(XG && !XF) ? TM * KP : 8];   // XG: the tile's X rows [row][k]
  __shared__ float2 gsh[TT > 0 ? TM : 1];                 // qkv epilogue: the tile's input gates
  constexpr int KH = 3;                                   // qkv epilogue: frames carried to the next chunk
  __shared__ float hsh[CARRY ? KH * TN * (TM / 8) : 1];   // their projections, [frame][column][pixel]
  // qkv epilogue: per column of the block, the conv taps on frames t, t-1, .., t-KH (zero beyond
  // kt), the projection bias and the conv bias, staged once per workgroup: [column][8].  Not for
  // fp32 A with the frame carry, whose LDS would then exceed two workgroups per CU: it reads them
  // per tile.
  constexpr bool QCW_LDS = TT > 0 && !(CARRY && !A1_ONLY);
  __shared__ __attribute__((aligned(16))) float qcw[QCW_LDS ? TN * 8 : 1];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int n0 = blockIdx.y * TN;
  const int NL = N - NH;
  const int tiles = (M + TM - 1) / TM;
  const TI* __restrict__ Gp = static_cast<const TI*>(ng.G);
  static_assert(TT == 0 || (SPLIT && !PLANE_A && OUT_SPLIT && TM % (16 * TT) == 0), "qkv epilogue: frames x pixels tiles");
  constexpr int TP = TT > 0 ? TM / TT : TM;   // pixels per tile (TT > 0)
  // global row of row r of tile `tile`
  // TT > 0: tile = (b * HW / TP + pixel block) * nch + chunk
  static_assert(!CARRY || TT == 8, "chunks of 8 frames carry frames");
  const int nch = CARRY ? qp.T / TT : 1;
  auto grow = [&](int tile, int r) -> int {
    if constexpr (TT == 0) {
      return tile * TM + r;
    } else {
      const int ch = tile % nch, q = tile / nch, tpf = HW / TP, bb = q / tpf, pb = q % tpf;
      return (bb * (CARRY ? qp.T : TT) + ch * TT + r / TP) * HW + pb * TP + r % TP;
    }
  };

  // SPLIT: lane l's B fragments, column wn 32 + 16 j + l % 16, k = 32 kb + 8 (l / 16) + e
  bf16x8 b1[MSPLIT ? 2 : 1][MSPLIT ? KB : 1], b2[MSPLIT ? 2 : 1][MSPLIT ? KB : 1], b3[MSPLIT ? 2 : 1][MSPLIT ? KB : 1];
  if constexpr (MSPLIT) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int gn = n0 + wn * 32 + j * 16 + (lane & 15);
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int kk = kb * 32 + (lane >> 4) * 8 + e;
          float w = 0.0f;
          if (kk < K) {
            if (gn < N) w = Wt[size_t(kk) * N + gn];
            else if (TT > 0 && gn < N + qp.ng) w = qp.wg[size_t(kk) * qp.ng + (gn - N)];
          }
          __bf16 x1, x2, x3;
          split3_bf16(w, x1, x2, x3);
          b1[j][kb][e] = x1;
          b2[j][kb][e] = x2;
          b3[j][kb][e] = x3;
        }
    }
  } else {
    for (int i = tid; i < KMAX * TN; i += NT) {
      const int kk = i / TN, c = i % TN;
      const int gn = n0 + c;
      Bs[kk * BP + c] = (kk < K && gn < N) ? Wt[size_t(kk) * N + gn] : 0.0f;
    }
  }
  if constexpr (NORM) {
    for (int kk = tid; kk < KMAX; kk += NT) {
      nss[2 * kk] = (ng.scale && kk < K) ? ng.scale[kk] : 1.f;
      nss[2 * kk + 1] = (ng.shift && kk < K) ? ng.shift[kk] : 0.f;
    }
  }
  // XG: lane l's gate_proj fragments, gate channel wn 32 + 16 j + l % 16, k = 32 kb + 8 (l / 16) + e, in three
  // bf16 parts, and that channel's bias
  bf16x8 g1[XG ? 2 : 1][XG ? KB : 1], g2[XG ? 2 : 1][XG ? KB : 1], g3[XG ? 2 : 1][XG ? KB : 1];
  float gb[2] = {0.f, 0.f};
  if constexpr (XG) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int gc = wn * 32 + j * 16 + (lane & 15);
      gb[j] = gc < K ? ng.bg[gc] : 0.f;
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int kk = kb * 32 + (lane >> 4) * 8 + e;
          const float w = (kk < K && gc < K) ? ng.wg[size_t(kk) * K + gc] : 0.0f;
          __bf16 x1, x2, x3;
          split3_bf16(w, x1, x2, x3);
          g1[j][kb][e] = x1;
          g2[j][kb][e] = x2;
          g3[j][kb][e] = x3;
        }
    }
  }
  if constexpr (QCW_LDS) {
    for (int cl = tid; cl < TN; cl += NT) {
      const int gn = n0 + cl, C = N / 3;
      float* e = &qcw[cl * 8];
      if (gn < N) {
        const int blk = gn / C, c = gn % C;
#pragma unroll
        for (int d = 0; d <= KH; ++d) e[d] = d < qp.kt ? qp.w[blk][(qp.kt - 1 - d) * C + c] : 0.0f;
        e[4] = bias[gn];
        e[5] = qp.kt > 0 ? qp.b[blk][c] : 0.0f;
      } else if (gn < N + qp.ng) {
#pragma unroll
        for (int d = 0; d <= KH; ++d) e[d] = 0.0f;
        e[4] = qp.bg[gn - N];
        e[5] = 0.0f;
      }
    }
  }
  // A prefetch: float4 f of the tile -> (row, k4) or (k, row4); SPLIT with
  // plane-major A: thread t holds KMAX/8 consecutive k of the 4 rows 4 (t % 32)
  auto fetch = [&](const TI* src, int tile, float4* pf) {
    const int m0 = tile * TM;
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      const int f = i * NT + tid;
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (SPLIT && PLANE_A) {
        const int kk = (tid / (TM / 4)) * (KMAX / 8) + i, r4 = (tid % (TM / 4)) * 4;
        const int gm = m0 + r4;
        if (kk < K && gm < M) {
          const int fr = gm / HW, p = gm % HW;
          v = ld4(src, (size_t(fr) * K + kk) * HW + p);
        }
      } else if (!PLANE_A) {
        const int r = f / (KMAX / 4), k4 = (f % (KMAX / 4)) * 4;
        const int gm = TT > 0 ? grow(tile, r) : m0 + r;
        if ((TT > 0 || gm < M) && k4 < K) {
          if constexpr (A1_ONLY) {
            // the raw bf16 bits (they are A's one bf16 part): no conversion here, so nothing waits
            // for the load before the stash copies them
            const uint2 raw = *reinterpret_cast<const uint2*>(src + size_t(gm) * K + k4);
            v = make_float4(__uint_as_float(raw.x), __uint_as_float(raw.y), 0.f, 0.f);
          } else {
            v = ld4(src, size_t(gm) * K + k4);
          }
        }
      } else {
        const int kk = f / (TM / 4), r4 = (f % (TM / 4)) * 4;
        const int gm = m0 + r4;
        if constexpr (PX1) {
          // PX1, planes of HW % 4 != 0 pixels (7 x 7, 14 x 14): the 4 rows may straddle two frames
          // and are not 16-byte aligned, so each is read on its own (the norm / gate prologue
          // only; the plain projections route such planes to the K-chunked kernel).  A separate
          // instantiation: a runtime branch here slowed the HW % 4 == 0 kernel's loads by 1.6x
          float e[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int g = gm + q;
            e[q] = (kk < K && g < M) ? ld_el(src, (size_t(g / HW) * K + kk) * HW + g % HW) : 0.0f;
          }
          v = make_float4(e[0], e[1], e[2], e[3]);
        } else {
          if (kk < K && gm < M) {
            const int fr = gm / HW, p = gm % HW;
            v = ld4(src, (size_t(fr) * K + kk) * HW + p);
          }
        }
      }
      pf[i] = v;
    }
  };
  auto stash = [&](const float4* pf) {
    if constexpr (SPLIT && PLANE_A) {
      // 4 rows x KMAX/8 consecutive k -> per row, runs of 8 bf16 of each part (16 B stores)
      const int k0 = (tid / (TM / 4)) * (KMAX / 8), r4 = (tid % (TM / 4)) * 4;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
#pragma unroll
        for (int c8 = 0; c8 < KMAX / 64; ++c8) {
          bf16x8 v1, v2, v3;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float4 v = pf[c8 * 8 + e];
            const float x = q == 0 ? v.x : (q == 1 ? v.y : (q == 2 ? v.z : v.w));
            __bf16 x1, x2 = __bf16(0.0f), x3 = __bf16(0.0f);
            if constexpr (A1_ONLY) x1 = (__bf16)x;   // exact for bf16 inputs
            else split3_bf16(x, x1, x2, x3);
            v1[e] = x1;
            v2[e] = x2;
            v3[e] = x3;
          }
          const int o = (r4 + q) * KP + k0 + c8 * 8;
          *reinterpret_cast<bf16x8*>(&A1[o]) = v1;
          if constexpr (!A1_ONLY) {
            *reinterpret_cast<bf16x8*>(&A2[o]) = v2;
            *reinterpret_cast<bf16x8*>(&A3[o]) = v3;
          }
        }
      }
      return;
    }
    if constexpr (SPLIT) {
      // row r, 4 consecutive k -> runs of 4 bf16 of each part (8 B stores)
#pragma unroll
      for (int i = 0; i < PF; ++i) {
        const int f = i * NT + tid;
        const int r = f / (KMAX / 4), k4 = (f % (KMAX / 4)) * 4;
        if constexpr (A1_ONLY) {
          // bf16 A: the fetched raw bits are the one part
          *reinterpret_cast<uint2*>(&A1[r * KP + k4]) = make_uint2(__float_as_uint(pf[i].x), __float_as_uint(pf[i].y));
          continue;
        }
        const float x[4] = {pf[i].x, pf[i].y, pf[i].z, pf[i].w};
        bf16x4 v1, v2, v3;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          __bf16 x1, x2 = __bf16(0.0f), x3 = __bf16(0.0f);
          if constexpr (A1_ONLY) x1 = (__bf16)x[e];   // exact for bf16 inputs
          else split3_bf16(x[e], x1, x2, x3);
          v1[e] = x1;
          v2[e] = x2;
          v3[e] = x3;
        }
        const int o = r * KP + k4;
        *reinterpret_cast<bf16x4*>(&A1[o]) = v1;
        if constexpr (!A1_ONLY) {
          *reinterpret_cast<bf16x4*>(&A2[o]) = v2;
          *reinterpret_cast<bf16x4*>(&A3[o]) = v3;
        }
      }
      return;
    }
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      const int f = i * NT + tid;
      if (!PLANE_A) {
        const int r = f / (KMAX / 4), k4 = (f % (KMAX / 4)) * 4;
        *reinterpret_cast<float2*>(&As[r * AP + k4]) = make_float2(pf[i].x, pf[i].y);
        *reinterpret_cast<float2*>(&As[r * AP + k4 + 2]) = make_float2(pf[i].z, pf[i].w);
      } else {
        const int kk = f / (TM / 4), r4 = (f % (TM / 4)) * 4;
        *reinterpret_cast<float4*>(&As[kk * AP + r4]) = pf[i];
      }
    }
  };
  // NORM: per-pixel statistics over the K channels of the staged tile, then
  // A[k][r] <- norm(A)[k][r] * G[k][r] in place (G from the prefetch registers)
  auto norm_gate = [&](const float4* pg) {
    // per-pixel sums over the K channels: NT / TM threads per pixel, each over its share of the
    // channels with four independent partial sums (not one dependent chain of K loads)
    {
      static_assert(!NORM || NT % TM == 0, "whole threads per pixel");
      constexpr int TPP = NORM ? NT / TM : 1;
      const int px = tid % TM, part = tid / TM, kc = (K + TPP - 1) / TPP;
      const int k0 = part * kc, k1 = k0 + kc < K ? k0 + kc : K;
      float a1[4] = {0.f, 0.f, 0.f, 0.f}, a2[4] = {0.f, 0.f, 0.f, 0.f};
      int kk = k0;
      for (; kk + 4 <= k1; kk += 4) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float v = As[(kk + q) * AP + px];
          a1[q] += v;
          a2[q] = fmaf(v, v, a2[q]);
        }
      }
      for (; kk < k1; ++kk) {
        const float v = As[kk * AP + px];
        a1[0] += v;
        a2[0] = fmaf(v, v, a2[0]);
      }
      rowsc[2 * tid] = (a1[0] + a1[1]) + (a1[2] + a1[3]);
      rowsc[2 * tid + 1] = (a2[0] + a2[1]) + (a2[2] + a2[3]);
    }
    __syncthreads();
    if (tid < TM) {
      float s1 = 0.f, s2 = 0.f;
#pragma unroll
      for (int q = 0; q < (NORM ? NT / TM : 1); ++q) {
        s1 += rowsc[2 * (tid + q * TM)];
        s2 += rowsc[2 * (tid + q * TM) + 1];
      }
      const float inv_k = 1.0f / float(K);
      float mean = 0.f, sc = 1.f;
      if (ng.kind == 1) {
        sc = rsqrtf(s2 * inv_k + 1e-6f);
      } else if (ng.kind == 2) {
        mean = s1 * inv_k;
        sc = rsqrtf(fmaxf(s2 * inv_k - mean * mean, 0.f) + 1e-6f);
      }
      // thread tid alone reads slot tid (its own) and slots tid + q TM (q >= 1, not written here)
      rowsc[2 * tid] = sc;
      rowsc[2 * tid + 1] = mean;
    }
    __syncthreads();
    if constexpr (!NSPLIT && !XG) {   // NSPLIT / XG: the statistics only; norm_split / xgate_norm apply them
#pragma unroll
      for (int i = 0; i < PF; ++i) {
        const int f = i * NT + tid;
        const int kk = f / (TM / 4), r4 = (f % (TM / 4)) * 4;
        if (kk >= K) continue;
        float4 v = *reinterpret_cast<const float4*>(&As[kk * AP + r4]);
        const float sk = nss[2 * kk], bk = nss[2 * kk + 1];
        float* e = &v.x;
        const float* g = &pg[i].x;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float sc = rowsc[2 * (r4 + q)], mu = rowsc[2 * (r4 + q) + 1];
          e[q] = (ng.kind == 0 ? e[q] : fmaf((e[q] - mu) * sc, sk, bk)) * g[q];
        }
        *reinterpret_cast<float4*>(&As[kk * AP + r4]) = v;
      }
    }
  };

  float4 pf[PF];
  float4 pg[(NORM && !NSPLIT && !XG) ? PF : 1];
  // NSPLIT without XG: the gate planes in the MFMA output layout, 4 pixels of gate channel wn 32 + 16 j + l % 16
  // at rows (wm MI + i) 16 + 4 (l / 16) + 0..3
  float4 pgm[(NSPLIT && !XG) ? MI : 1][2];
  auto fetch_gm = [&](int tile) {
    if constexpr (NSPLIT && !XG) {
      const int m0 = tile * TM;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int kk = wn * 32 + j * 16 + (lane & 15);
#pragma unroll
        for (int i = 0; i < MI; ++i) {
          const int gm = m0 + (wm * MI + i) * 16 + (lane >> 4) * 4;   // HW % 4 == 0: the 4 pixels share a frame
          pgm[i][j] = (kk < K && gm < M) ? ld4(Gp, (size_t(gm / HW) * K + kk) * HW + gm % HW)
                                         : make_float4(0.f, 0.f, 0.f, 0.f);
        }
      }
    }
  };
  // XG: the tile's X rows, 16-byte pieces c = i NT + tid: row c / (KMAX / 8), channels 8 (c % (KMAX / 8)) ..
  constexpr int PX = (XG && !XF) ? TM * KMAX / 8 / NT : 1;
  uint4 px[PX];
  auto fetch_x = [&](int tile) {
    if constexpr (XG && !XF) {
      const int m0 = tile * TM;
#pragma unroll
      for (int i = 0; i < PX; ++i) {
        const int c = i * NT + tid, r = c / (KMAX / 8), k8 = (c % (KMAX / 8)) * 8;
        px[i] = (m0 + r < M && k8 < K) ? *reinterpret_cast<const uint4*>(ng.X + size_t(m0 + r) * K + k8)
                                        : make_uint4(0u, 0u, 0u, 0u);
      }
    }
  };
  auto stash_x = [&]() {
    if constexpr (XG && !XF) {
#pragma unroll
      for (int i = 0; i < PX; ++i) {
        const int c = i * NT + tid, r = c / (KMAX / 8), k8 = (c % (KMAX / 8)) * 8;
        *reinterpret_cast<uint4*>(&Xs[r * KP + k8]) = px[i];
      }
    }
  };
  // XG: x Wg for this wave's rows (wm MI + i) 16 + 4 (l / 16) + q and gate channels wn 32 + 16 j + l % 16
  // (the MFMA output layout), issued before the norm's statistics so the MFMAs run under them; then
  // A <- norm(A) * act(x Wg + bg) for exactly those elements
  floatx4 ag[XG ? MI : 1][2];
  // XF: this wave's fp32 x fragments of a tile (rows past M and channels past K read as 0; K % 8 == 0,
  // host-checked), issued at the top of the tile so they land during its stash and barriers
  float4 xr[XF ? MI : 1][XF ? KB : 1][2];
  auto xf_fetch = [&](int tile) {
    if constexpr (XF) {
#pragma unroll
      for (int i = 0; i < MI; ++i) {
        const int row = tile * TM + (wm * MI + i) * 16 + (lane & 15);
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
          const int k8 = kb * 32 + (lane >> 4) * 8;
          const bool ok = row < M && k8 < K;
          const float4* src = reinterpret_cast<const float4*>(ng.Xf + size_t(ok ? row : 0) * K + (ok ? k8 : 0));
          xr[i][kb][0] = ok ? src[0] : make_float4(0.f, 0.f, 0.f, 0.f);
          xr[i][kb][1] = ok ? src[1] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
      }
    }
  };
  auto xgate_mma = [&](int tile) {
    if constexpr (XF) {
      // fp32 x: each fragment split into three bf16 parts, six products with the gate weights' parts
      (void)tile;
#pragma unroll
      for (int i = 0; i < MI; ++i) {
        ag[i][0] = ag[i][1] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
          if (kb * 32 >= K) break;
          bf16x8 x1, x2, x3;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            __bf16 a1, a2, a3;
            split3_bf16(e < 4 ? (&xr[i][kb][0].x)[e] : (&xr[i][kb][1].x)[e - 4], a1, a2, a3);
            x1[e] = a1;
            x2[e] = a2;
            x3[e] = a3;
          }
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            floatx4 c = ag[i][j];
            c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x3, g1[j][kb], c, 0, 0, 0);   // small terms first
            c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x2, g2[j][kb], c, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x1, g3[j][kb], c, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x2, g1[j][kb], c, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x1, g2[j][kb], c, 0, 0, 0);
            ag[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x1, g1[j][kb], c, 0, 0, 0);
          }
        }
      }
    } else if constexpr (XG) {
#pragma unroll
      for (int i = 0; i < MI; ++i) ag[i][0] = ag[i][1] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        if (kb * 32 >= K) break;
        const int koff = kb * 32 + (lane >> 4) * 8;
#pragma unroll
        for (int i = 0; i < MI; ++i) {
          const bf16x8 a1 = *reinterpret_cast<const bf16x8*>(&Xs[((wm * MI + i) * 16 + (lane & 15)) * KP + koff]);
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            floatx4 c = ag[i][j];
            c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, g3[j][kb], c, 0, 0, 0);   // small terms first
            c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, g2[j][kb], c, 0, 0, 0);
            ag[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, g1[j][kb], c, 0, 0, 0);
          }
        }
      }
    }
  };
  // XG: A <- norm(A) * act(x Wg + bg) in place for exactly this wave's elements of the MFMA output layout
  auto xgate_norm = [&]() {
    if constexpr (XG) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int kk = wn * 32 + j * 16 + (lane & 15);
        if (kk >= K) continue;
        const float sk = nss[2 * kk], bk = nss[2 * kk + 1];
#pragma unroll
        for (int i = 0; i < MI; ++i) {
          const int r0 = (wm * MI + i) * 16 + (lane >> 4) * 4;
          float4 v = *reinterpret_cast<const float4*>(&As[kk * AP + r0]);
          float* e = &v.x;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float z = ag[i][j][q] + gb[j];
            const float sg = __builtin_amdgcn_rcpf(1.0f + __expf(-z));
            const float g = ng.gact == 1 ? z * sg : sg;
            const float sc = rowsc[2 * (r0 + q)], mu = rowsc[2 * (r0 + q) + 1];
            e[q] = (ng.kind == 0 ? e[q] : fmaf((e[q] - mu) * sc, sk, bk)) * g;
          }
          *reinterpret_cast<float4*>(&As[kk * AP + r0]) = v;
        }
      }
    }
  };
  // NSPLIT: A <- norm(A) * gate for this wave's elements (rows (wm MI + i) 16 + 4 (l / 16) + q, channels
  // wn 32 + 16 j + l % 16: the MFMA output layout; the gate from the planes prefetched in that layout),
  // then, once every wave has read the fp32 staging, their three bf16 parts into the planes over it (zero for
  // channels past K, which the k-blocks still read)
  auto norm_split = [&]() {
    if constexpr (NSPLIT) {
      float4 nv[MI][2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int kk = wn * 32 + j * 16 + (lane & 15);
        const int kc = kk < K ? kk : 0;
        const float sk = nss[2 * kc], bk = nss[2 * kc + 1];
#pragma unroll
        for (int i = 0; i < MI; ++i) {
          const int r0 = (wm * MI + i) * 16 + (lane >> 4) * 4;
          float4 v = *reinterpret_cast<const float4*>(&As[kc * AP + r0]);
          float* e = &v.x;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float g = (&pgm[i][j].x)[q];
            const float sc = rowsc[2 * (r0 + q)], mu = rowsc[2 * (r0 + q) + 1];
            e[q] = kk < K ? (ng.kind == 0 ? e[q] : fmaf((e[q] - mu) * sc, sk, bk)) * g : 0.0f;
          }
          nv[i][j] = v;
        }
      }
      __syncthreads();   // every wave has read the fp32 staging the planes overwrite
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int kk = wn * 32 + j * 16 + (lane & 15);
#pragma unroll
        for (int i = 0; i < MI; ++i) {
          const int r0 = (wm * MI + i) * 16 + (lane >> 4) * 4;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            __bf16 x1, x2, x3;
            split3_bf16((&nv[i][j].x)[q], x1, x2, x3);
            const int o = (r0 + q) * KP + kk;
            A1[o] = x1;
            A2[o] = x2;
            A3[o] = x3;
          }
        }
      }
    }
  };
  // qkv epilogue: a tile's per-pixel / per-frame input gates (TT frames x TP pixels) are
  // loaded with its A rows and written to gsh by the stash, behind the barrier that follows it
  const bool tile_gates = TT > 0 && (qp.gate_mode == 1 || qp.gate_mode == 2);
  float2 gpf = make_float2(0.f, 0.f);
  auto fetch_gates = [&](int tl) {
    if constexpr (TT > 0) {
      if (tile_gates && tid < TT * TP) {
        const int ch = tl % nch, tq = tl / nch, tpf = HW / TP, bb = tq / tpf, pb = tq % tpf;
        const size_t fr = size_t(bb) * (CARRY ? qp.T : TT) + size_t(ch) * TT + tid / TP;
        gpf = qp.gate_mode == 1 ? static_cast<const float2*>(qp.gates)[fr * HW + pb * TP + tid % TP]
                                : static_cast<const float2*>(qp.gates)[fr];
      }
    }
  };
  // k-th tile of this workgroup.  The qkv epilogue (TT > 0) writes half cache
  // lines (16 pixels of a plane) per tile; the workgroup takes its pixel blocks
  // in adjacent pairs so both halves of each line pass through the same L2, and
  // the chunks of a pixel block in order (they carry frames to each other).
  auto tile_of = [&](int k) -> int {
    if constexpr (TT > 0) {
      const int ch = k % nch, pbk = k / nch;
      return (2 * (int(blockIdx.x) + (pbk >> 1) * int(gridDim.x)) + (pbk & 1)) * nch + ch;
    } else {
      return int(blockIdx.x) + k * int(gridDim.x);
    }
  };
  int kt_ = 0;
  int tile = tile_of(0);
  if (tile < tiles) {
    fetch(A, tile, pf);
    fetch_gates(tile);
    if constexpr (XG) fetch_x(tile);
    else if constexpr (NSPLIT) fetch_gm(tile);
    else if (NORM) fetch(Gp, tile, pg);
  }
  if (tile < tiles) xf_fetch(tile);
  for (; tile < tiles; tile = tile_of(++kt_)) {
    __syncthreads();            // previous tile is done with As, Xs, gsh (and Bs is staged)
    stash(pf);
    stash_x();
    if constexpr (TT > 0) {
      if (tile_gates && tid < TT * TP) gsh[tid] = gpf;
    }
    __syncthreads();
    if constexpr (NORM) {
      xgate_mma(tile);    // XG: x Wg, under the statistics
      norm_gate(pg);  // the per-pixel statistics (without NSPLIT / XG also the norm x gate in place)
      xgate_norm();   // XG: norm x computed gate in place
      norm_split();   // NSPLIT: norm x gate into the bf16 planes
      __syncthreads();
    }
    const int next = tile_of(kt_ + 1);
    if (next < tiles) {
      fetch(A, next, pf);
      fetch_gates(next);
      xf_fetch(next);   // XF: the x fragments were consumed by xgate_mma above
      if constexpr (XG) fetch_x(next);
      else if constexpr (NSPLIT) fetch_gm(next);
      else if (NORM) fetch(Gp, next, pg);
    }

    floatx4 acc[MI][2];
#pragma unroll
    for (int i = 0; i < MI; ++i) acc[i][0] = acc[i][1] = floatx4{0.f, 0.f, 0.f, 0.f};
    if constexpr (MSPLIT) {
      // lane l: A rows l % 16 and B columns l % 16, k = 32 kb + 8 (l / 16) + 0..7
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        if (kb * 32 >= K) break;
        const int koff = kb * 32 + (lane >> 4) * 8;
#pragma unroll
        for (int i = 0; i < MI; ++i) {
          const int o = ((wm * MI + i) * 16 + (lane & 15)) * KP + koff;
          const bf16x8 a1 = *reinterpret_cast<const bf16x8*>(&A1[o]);
          if constexpr (A1_ONLY) {
            // the three products with A's one nonzero part, in the six-product order
#pragma unroll
            for (int j = 0; j < 2; ++j) {
              floatx4 c = acc[i][j];
              c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b3[j][kb], c, 0, 0, 0);
              c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b2[j][kb], c, 0, 0, 0);
              acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b1[j][kb], c, 0, 0, 0);
            }
          } else {
            const bf16x8 a2 = *reinterpret_cast<const bf16x8*>(&A2[o]);
            const bf16x8 a3 = *reinterpret_cast<const bf16x8*>(&A3[o]);
#pragma unroll
            for (int j = 0; j < 2; ++j) {
              floatx4 c = acc[i][j];
              c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a3, b1[j][kb], c, 0, 0, 0);   // small terms first
              c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2, b2[j][kb], c, 0, 0, 0);
              c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b3[j][kb], c, 0, 0, 0);
              c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2, b1[j][kb], c, 0, 0, 0);
              c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b2[j][kb], c, 0, 0, 0);
              acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b1[j][kb], c, 0, 0, 0);
            }
          }
        }
      }
    }
    const int kend = MSPLIT ? 0 : (K + 3) / 4 * 4;
    for (int kk = 0; kk < kend; kk += 4) {
      const int ka = kk + (lane >> 4);
      float a[MI], b[2];
#pragma unroll
      for (int i = 0; i < MI; ++i) {
        const int r = (wm * MI + i) * 16 + (lane & 15);
        a[i] = PLANE_A ? As[ka * AP + r] : As[r * AP + ka];
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) b[j] = Bs[ka * BP + wn * 32 + j * 16 + (lane & 15)];
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i], b[j], acc[i][j], 0, 0, 0);
    }

    // epilogue: lane holds rows 16 i + 4 (lane / 16) + r of column lane % 16 of n-tile j
    const int m0 = tile * TM;
    if constexpr (TT > 0) {
      // GDN qkv: lane rows 16 i + 4 (lane / 16) + r are pixel pb TP + (16 i) % TP + 4 (lane / 16) + r of
      // frame t = 16 i / TP; frame t - d of the same pixels is row tile i - d IPF of the same lane
      constexpr int IPF = TP / 16;
      const int ch = tile % nch, tq = tile / nch, tpf = HW / TP, bb = tq / tpf, pb = tq % tpf;
      const size_t fr0 = size_t(bb) * (CARRY ? qp.T : TT) + size_t(ch) * TT;   // first frame of the tile
      const int C = N / 3;
      // the tile's input gates (TT frames x TP pixels x (B_k, B_v)) are in gsh (staged with A)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int cl = wn * 32 + j * 16 + (lane & 15), gn = n0 + cl;
        if (gn >= N + qp.ng) continue;
        const int blk = gn / C, c = gn % C;
        const bool gcol = gn >= N;   // a gate_proj column: bias and activation only
        // wd[d]: tap on frame t - d.  From LDS: taps on frames t .. t - KH (zero beyond kt, so those
        // products add nothing) with the projection bias folded into the accumulators once; read
        // per tile: up to 8 taps, the ones beyond kt skipped, the bias added per use.
        constexpr int NTAP = QCW_LDS ? KH + 1 : 8;
        float wd[NTAP], bv, bt;
        if constexpr (QCW_LDS) {
          const float4 w4 = *reinterpret_cast<const float4*>(&qcw[cl * 8]);
          const float2 bb2 = *reinterpret_cast<const float2*>(&qcw[cl * 8 + 4]);
          wd[0] = w4.x;
          wd[1] = w4.y;
          wd[2] = w4.z;
          wd[3] = w4.w;
          bv = bb2.x;
          bt = bb2.y;
#pragma unroll
          for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[i][j][r] += bv;
        } else {
#pragma unroll
          for (int d = 0; d < NTAP; ++d) wd[d] = (!gcol && d < qp.kt) ? qp.w[blk][(qp.kt - 1 - d) * C + c] : 0.0f;
          bv = gcol ? qp.bg[gn - N] : bias[gn];
          bt = (!gcol && qp.kt > 0) ? qp.b[blk][c] : 0.0f;
        }
        // the projection of frame i of this tile with its bias
        auto xb = [&](int i, int r) -> float {
          if constexpr (QCW_LDS) return acc[i][j][r];
          else return acc[i][j][r] + bv;
        };
#pragma unroll
        for (int i = 0; i < MI; ++i) {
          const int t = i / IPF;
          const int pl = (i % IPF) * 16 + (lane >> 4) * 4, px = pb * TP + pl;   // pixel in tile / in plane
          const size_t fr = fr0 + t;
          float v[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float x = xb(i, r);
            if (gcol) {
              const float sg = __builtin_amdgcn_rcpf(1.0f + __expf(-x));   // as the plain projection's epilogue
              x = qp.gact == 1 ? x * sg : sg;
            } else if (qp.kt > 0) {
              float o = fmaf(wd[0], x, bt);
#pragma unroll
              for (int d = NTAP - 1; d >= 1; --d) {
                if (!QCW_LDS && d >= qp.kt) continue;
                if (i >= d * IPF) {
                  o = fmaf(wd[d], xb(i - d * IPF, r), o);
                } else if (CARRY && ch > 0 && d - t <= KH) {
                  // frame t - d < 0 of this chunk: frame TT + t - d of the previous chunk
                  o = fmaf(wd[d], hsh[((KH - (d - t)) * TN + cl) * TP + pl + r], o);
                }   // else before the first frame: the zero left padding adds nothing
              }
              x = o * __builtin_amdgcn_rcpf(1.0f + __expf(-o));   // SiLU as gdn_qkv_post computes it
            }
            v[r] = x;
          }
          if (!gcol && blk > 0 && qp.gate_mode != 0) {
            float g[4];
            if (qp.gate_mode != 3) {
              const float2* gp = gsh + t * TP + (i % IPF) * 16 + (lane >> 4) * 4;
#pragma unroll
              for (int r = 0; r < 4; ++r) g[r] = blk == 1 ? gp[r].x : gp[r].y;
            } else {
              const float4 gg = *reinterpret_cast<const float4*>(static_cast<const float*>(qp.gates) +
                                                                 (fr * 2 * C + size_t(blk - 1) * C + c) * HW + px);
              g[0] = gg.x; g[1] = gg.y; g[2] = gg.z; g[3] = gg.w;
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) v[r] *= g[r];
          }
          if (gcol) st4(static_cast<TO*>(qp.gv), (fr * qp.ng + (gn - N)) * HW + px, v);
          else st4(out_lo, (fr * N + gn) * HW + px, v);
        }
        if constexpr (CARRY) {
          // this chunk's last KH frames for the next chunk of the same pixels (each lane its own slots)
          if (ch + 1 < nch) {
#pragma unroll
            for (int i = (TT - KH) * IPF; i < MI; ++i) {
              const int pl = (i % IPF) * 16 + (lane >> 4) * 4;
#pragma unroll
              for (int r = 0; r < 4; ++r) hsh[((i / IPF - (TT - KH)) * TN + cl) * TP + pl + r] = xb(i, r);
            }
          }
        }
      }
    } else if (OUT_SPLIT) {
      // 4 consecutive pixels of one channel per lane and MFMA tile: 16 B stores.
      // Frame / pixel of the lane's first row: one division per tile, then
      // advanced by 16 rows per i.
      const int gmb = m0 + wm * MI * 16 + (lane >> 4) * 4;
      const int fr_b = gmb / HW, p_b = gmb % HW;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int gn = n0 + wn * 32 + j * 16 + (lane & 15);
        const bool nok = gn < N;
        const float bv = nok ? bias[gn] : 0.0f;
        const bool lo = gn < NH;
        const int c = lo ? gn : gn - NH;
        const int NC = lo ? NH : NL;
        TO* dst = lo ? out_lo : out_hi;
        const int act = lo ? act_lo : act_hi;
        // bias and activation: one wave-uniform branch when both halves use the same activation
        if (act_lo == act_hi && act_lo == 0) {
#pragma unroll
          for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[i][j][r] += bv;
        } else {
#pragma unroll
          for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const float v = acc[i][j][r] + bv;
              const float sg = __builtin_amdgcn_rcpf(1.0f + __expf(-v));
              acc[i][j][r] = act == 1 ? v * sg : (act == 2 ? sg : v);
            }
        }
        float csum = 0.0f;
        int fr = fr_b, p = p_b;
        // act 3 (proj_in's lower half for training): values stored as they are, channel sums of SiLU
        const bool sum_silu = lo && act_lo == 3;
#pragma unroll
        for (int i = 0; i < MI; ++i) {
          const int gm0 = gmb + i * 16;
          const float v[4] = {acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]};
          float sv[4] = {v[0], v[1], v[2], v[3]};
          if (sum_silu) {
#pragma unroll
            for (int r = 0; r < 4; ++r) sv[r] = v[r] * __builtin_amdgcn_rcpf(1.0f + __expf(-v[r]));
          }
          if (nok && gm0 + 3 < M && (HW % 4) == 0) {
            st4(dst, (size_t(fr) * NC + c) * HW + p, v);
            csum += (sv[0] + sv[1]) + (sv[2] + sv[3]);
          } else if (nok) {
            int f2 = fr, p2 = p;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              if (gm0 + r < M) {
                st_el(dst, (size_t(f2) * NC + c) * HW + p2, v[r]);
                csum += sv[r];
              }
              if (++p2 == HW) {
                p2 = 0;
                ++f2;
              }
            }
          }
          p += 16;
          while (p >= HW) {
            p -= HW;
            ++fr;
          }
        }
        if (WM == 1 && partial != nullptr && lo) {
          csum += __shfl_xor(csum, 16, 64);
          csum += __shfl_xor(csum, 32, 64);
          if (lane < 16 && nok) partial[size_t(tile) * NH + c] = csum;
        }
      }
    } else {
      // stage the tile in LDS (over the A tile) and store whole rows: 16 B per lane
      __syncthreads();
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int cl = wn * 32 + j * 16 + (lane & 15);
        const int gn = n0 + cl;
        const float bv = gn < N ? bias[gn] : 0.0f;
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
          for (int r = 0; r < 4; ++r) As[((wm * MI + i) * 16 + (lane >> 4) * 4 + r) * OP + cl] = acc[i][j][r] + bv;
      }
      __syncthreads();
      constexpr int C4 = TN / 4;
      for (int f = tid; f < TM * C4; f += NT) {
        const int r = f / C4, c4 = (f % C4) * 4;
        const int gm = m0 + r, gn = n0 + c4;
        if (gm >= M) continue;
        const float* src = &As[r * OP + c4];
        if (gn + 3 < N && (N % 4) == 0) {
          float v[4] = {src[0], src[1], src[2], src[3]};
          st4(out_lo, size_t(gm) * N + gn, v);
        } else {
          for (int e = 0; e < 4; ++e)
            if (gn + e < N) st_el(out_lo, size_t(gm) * N + gn + e, src[e]);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// K-chunked projection for K beyond the persistent kernel's register-resident
// weights (the CSSM-SHViT stages: K = 128 .. 640), on bf16 MFMA with the
// operands split into bf16 parts (x = x1 + x2 + x3): fp32 A takes the same six
// products as the persistent kernel (three, down to order 2^-16, when the output
// is bf16); bf16 A is exactly its first part, so three products
// (A1 B1 + A1 B2 + A1 B3) give the same fp32-level result.  One
// 128 x 128 output tile per workgroup; four waves split the 128 columns (32
// each) and keep all 128 rows, as in the persistent kernel, so the proj_in
// channel sums stay in-wave.  K advances in chunks of 32 with one barrier per
// chunk and two chunks' loads in flight:
//   A   global -> registers two chunks ahead, then split into bf16 planes in
//       one of two LDS stages ([row][k], k contiguous: the MFMA operand order)
//       while the MFMAs read the other stage;
//   B   each wave loads its own 32 columns straight into registers (two
//       chunks ahead) and splits them there: the fragments never pass through
//       LDS and no other wave reads them.
//   PLANE_A = false: A is channels-last (M, K), K % 4 == 0; true: plane-major (F, K, HW).
//   OUT_SPLIT = true: plane-major output(s) as proj_in; false: channels-last (M, N).
// ---------------------------------------------------------------------------
// PX4 (plane-major A, H*W % 4 == 0, host-checked): a thread loads 4 consecutive pixels of one
// channel plane per 16-byte load (4 channels: 4 loads) instead of one element per load, and
// transposes them in registers for the [row][k] LDS layout: a quarter of the A load
// instructions, which otherwise fill the wave's outstanding-load counter and stall the issue
// TN_ = 64 (channels-last outputs with N <= 64): the four waves split the tile as two row halves
// by two 32-column halves instead of four column quarters, so no wave runs on columns past N.
template <bool PLANE_A, bool OUT_SPLIT, class TI, class TO, int TM_, bool PX4 = false, int TN_ = 128>
__global__ void __launch_bounds__(256, (sizeof(TI) == 2 && !PLANE_A) ? 3 : 2)
proj_kc_kernel(const TI* __restrict__ A, int M, int K, int N, const float* __restrict__ Wt,
               const float* __restrict__ bias, int HW, TO* __restrict__ out_lo, TO* __restrict__ out_hi,
               int act_lo, int act_hi, float* __restrict__ partial, int NH, int slots) {
  constexpr int TM = TM_, TN = TN_, NT = 256, KC = 32, KP = KC + 8;
  static_assert(TM == 64 || TM == 128, "row tiles of 64 or 128");
  static_assert(TN == 128 || (TN == 64 && !OUT_SPLIT), "64-column tiles for channels-last outputs only");
  // waves: WC across the tile's columns (32 each) by WR across its rows (RW each, MI blocks of 16)
  constexpr int WC = TN / 32, WR = 4 / WC, RW = TM / WR, MI = RW / 16;
  static_assert(!PX4 || PLANE_A, "4-pixel loads are for plane-major A");
  constexpr int NI = TM / 32, NKQ = 256 / TM;   // A load groups per thread; plane-major k groups
  constexpr bool A1_ONLY = sizeof(TI) == 2;      // bf16 A: one nonzero part
  // fp32 A with a bf16 output: the three products down to order 2^-16 (A1 B1 + A1 B2 + A2 B1) are far
  // inside the output's own rounding (2^-9), so A3 and the order-2^-16 products are dropped
  constexpr bool SIX = !A1_ONLY && sizeof(TO) == 4;
  constexpr int APL = A1_ONLY ? 1 : (SIX ? 3 : 2);   // A planes
  constexpr int OP = TN + 4;                     // channels-last staging pitch (floats), 64 rows at a time
  constexpr int AB = TM * KP;                    // bf16 per plane
  constexpr int STG = APL * AB;                  // bf16 per pipeline stage
  constexpr int SPC = TM + 4;                    // plane-major staging pitch (floats): [16 columns][SPC] per wave
  constexpr int OUT_N = OUT_SPLIT ? 4 * 16 * SPC * 2 : 64 * OP * 2;   // output staging, in bf16 units
  constexpr int LDS_N = OUT_N > 2 * STG ? OUT_N : 2 * STG;
  __shared__ __attribute__((aligned(16))) __bf16 lds[LDS_N];   // two A stages; the output staging reuses them
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int wn = wv % WC, wr = wv / WC;   // column group, row group of this wave
  // XCD-aware tile order: workgroup ids go round-robin over the 8 XCDs, so the
  // tiles are dealt to the XCDs in 8 contiguous runs, column tile fastest: the
  // column tiles of one row tile run on the same XCD and share its A rows in L2
  int rt, ct;
  {
    const int total = int(gridDim.x), ctiles = (N + TN - 1) / TN;
    const int x = int(blockIdx.x) % 8, li = int(blockIdx.x) / 8, q = total / 8, r = total % 8;
    const int t = x * q + (x < r ? x : r) + li;
    rt = t / ctiles;
    ct = t % ctiles;
  }
  const int m0 = rt * TM, n0 = ct * TN;
  const int NL = N - NH;

  // this thread's A loads per chunk: NI groups i of 4 consecutive k
  //   channels-last: rows (tid / 8) + 32 i, k 4 (tid % 8)
  //   plane-major:   row tid % TM, k groups NKQ i + tid / TM
  // All loads are buffer loads with a per-lane byte offset and a uniform
  // (SGPR) one, so the unrolled chunk offsets cost no VGPRs across the loop.
  const int rr = tid % TM, kq = tid / TM;
  const int ar = tid >> 3, ak = (tid & 7) * 4;
  constexpr int EA = sizeof(TI);
  __amdgpu_buffer_rsrc_t ra;   // A rows of this tile
  unsigned a_off;
  bool a_ok[NI];
  if constexpr (!PLANE_A) {
    const int rows = M - m0 < TM ? M - m0 : TM;
    ra = make_rsrc(A + size_t(m0) * K, unsigned(rows) * unsigned(K) * EA);
    a_off = unsigned(ar * K + ak) * EA;
#pragma unroll
    for (int i = 0; i < NI; ++i) a_ok[i] = m0 + ar + 32 * i < M;
  } else {
    const int last = (M - m0 < TM ? M : m0 + TM) - 1;
    const int fr0 = m0 / HW, nfr = last / HW - fr0 + 1;
    ra = make_rsrc(A + size_t(fr0) * K * HW, unsigned(nfr) * unsigned(K) * unsigned(HW) * EA);
    if constexpr (PX4) {
      // item (4-row group rg, 4-channel group kg) of thread tid < 2 TM; a group of 4 rows lies in one
      // frame (H*W and m0 are multiples of 4)
      const int rg = tid % (TM / 4), kg = tid / (TM / 4);
      const int gm = m0 + 4 * rg < M ? m0 + 4 * rg : m0;
      a_off = unsigned(((gm / HW - fr0) * K + 4 * kg) * HW + gm % HW) * EA;
#pragma unroll
      for (int i = 0; i < NI; ++i) a_ok[i] = tid < 2 * TM && m0 + 4 * rg < M;
    } else {
      const int gm = m0 + rr < M ? m0 + rr : m0;
      a_off = unsigned(((gm / HW - fr0) * K + 4 * kq) * HW + gm % HW) * EA;
#pragma unroll
      for (int i = 0; i < NI; ++i) a_ok[i] = m0 + rr < M;
    }
  }
  // this lane's B fragments: columns wn 32 + 16 j + lane % 16, k = chunk + 8 (lane / 16) + e
  const int kl = (lane >> 4) * 8;
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(Wt, unsigned(K) * unsigned(N) * 4u);
  unsigned b_off[2];
  bool b_ok[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int gn = n0 + wn * 32 + j * 16 + (lane & 15);
    b_ok[j] = gn < N;
    b_off[j] = unsigned(kl * N + (b_ok[j] ? gn : 0)) * 4u;
  }
  // register sets s = 0, 1: chunk j's loads land in set j % 2, its A in LDS stage j % 2.
  // Raw A: the bf16 bits themselves for channels-last bf16 A (they are the one bf16 part), else floats.
  constexpr bool RAW16 = A1_ONLY && !PLANE_A;
  using RawA = typename std::conditional<RAW16, uint2, float4>::type;
  constexpr int NA = PX4 ? 4 : NI;               // A registers per set (PX4: one per channel of the item)
  RawA pa[2][NA];
  float pw[2][2][8];
  // A lane whose element lies outside the tensor (rows beyond M, k beyond K)
  // loads at byte offset kOut instead: beyond every resource range, so the
  // buffer load returns 0 without touching memory.
  constexpr unsigned kOut = 0x80000000u;
  // Offsets are selected without branches: a lane's base offset is kOut where its row or column is
  // outside the tensor, and a channel at or beyond K ORs kOut in (past every resource's range: the
  // buffer load returns 0 without touching memory).  A select that the compiler turned into a
  // branch around the load made it wait for every load in flight.
  unsigned a_base[NI], b_base[2];
#pragma unroll
  for (int i = 0; i < NI; ++i) a_base[i] = a_ok[i] ? a_off : kOut;
#pragma unroll
  for (int j = 0; j < 2; ++j) b_base[j] = b_ok[j] ? b_off[j] : kOut;
  auto past_k = [&](int k) -> unsigned { return k < K ? 0u : kOut; };
  auto fetch = [&](int k0, int s) {
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      if constexpr (!PLANE_A) {
        const unsigned vo = a_base[i] | past_k(k0 + ak);
        const int so = (32 * i * K + k0) * EA;
        if constexpr (RAW16)
          pa[s][i] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(ra, int(vo), so, 0));
        else
          pa[s][i] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(ra, int(vo), so, 0));
      } else if constexpr (PX4) {
        // channel k0 + 4 kg + q of the item's 4 rows
        if (i == 0) {
          const int kg = tid / (TM / 4);
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const unsigned vo = a_base[0] | past_k(k0 + 4 * kg + q);
            const int so = (k0 + q) * HW * EA;
            if constexpr (EA == 2) {
              const uint2 raw = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(ra, int(vo), so, 0));
              pa[s][q] = make_float4(__uint_as_float(raw.x << 16), __uint_as_float(raw.x & 0xffff0000u),
                                     __uint_as_float(raw.y << 16), __uint_as_float(raw.y & 0xffff0000u));
            } else {
              pa[s][q] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(ra, int(vo), so, 0));
            }
          }
        }
      } else {
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int k = k0 + 4 * NKQ * i + e;   // relative to this thread's 4 kq
          const unsigned vo = a_base[i] | past_k(k + 4 * kq);
          const int so = k * HW * EA;
          if constexpr (EA == 2)
            v[e] = __uint_as_float(unsigned(__builtin_amdgcn_raw_buffer_load_b16(ra, int(vo), so, 0)) << 16);
          else
            v[e] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(ra, int(vo), so, 0));
        }
        pa[s][i] = make_float4(v[0], v[1], v[2], v[3]);
      }
    }
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const unsigned vo = b_base[j] | past_k(k0 + kl + e);
        pw[s][j][e] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rb, int(vo), (k0 + e) * N * 4, 0));
      }
  };
  // A of register set s -> the bf16 planes of LDS stage s
  auto stash = [&](int s) {
    __bf16* const planes = lds + s * STG;
    if constexpr (PX4) {
      if (tid < 2 * TM) {
        const int rg = tid % (TM / 4), kg = tid / (TM / 4);
#pragma unroll
        for (int q = 0; q < 4; ++q) {   // row 4 rg + q: its 4 channels from the 4 loads
          const float x[4] = {(&pa[s][0].x)[q], (&pa[s][1].x)[q], (&pa[s][2].x)[q], (&pa[s][3].x)[q]};
          bf16x4 v1, v2, v3;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            __bf16 x1, x2 = __bf16(0.0f), x3 = __bf16(0.0f);
            if constexpr (A1_ONLY) x1 = (__bf16)x[e];   // exact for bf16 inputs
            else split3_bf16(x[e], x1, x2, x3);
            v1[e] = x1;
            v2[e] = x2;
            v3[e] = x3;
          }
          const int off = (4 * rg + q) * KP + 4 * kg;
          *reinterpret_cast<bf16x4*>(planes + off) = v1;
          if constexpr (APL >= 2) *reinterpret_cast<bf16x4*>(planes + AB + off) = v2;
          if constexpr (APL == 3) *reinterpret_cast<bf16x4*>(planes + 2 * AB + off) = v3;
        }
      }
      return;
    }
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int off = PLANE_A ? rr * KP + (NKQ * i + kq) * 4 : (ar + 32 * i) * KP + ak;
      if constexpr (RAW16) {
        *reinterpret_cast<uint2*>(planes + off) = pa[s][i];
      } else {
        const float4 p = pa[s][i];
        const float x[4] = {p.x, p.y, p.z, p.w};
        bf16x4 v1, v2, v3;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          __bf16 x1, x2 = __bf16(0.0f), x3 = __bf16(0.0f);
          if constexpr (A1_ONLY) x1 = (__bf16)x[e];   // exact for bf16 inputs
          else split3_bf16(x[e], x1, x2, x3);
          v1[e] = x1;
          v2[e] = x2;
          v3[e] = x3;
        }
        *reinterpret_cast<bf16x4*>(planes + off) = v1;
        if constexpr (APL >= 2) *reinterpret_cast<bf16x4*>(planes + AB + off) = v2;
        if constexpr (APL == 3) *reinterpret_cast<bf16x4*>(planes + 2 * AB + off) = v3;
      }
    }
  };
  bf16x8 b1[2], b2[2], b3[2];
  auto split_b = [&](int s) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        __bf16 x1, x2, x3;
        split3_bf16(pw[s][j][e], x1, x2, x3);
        b1[j][e] = x1;
        b2[j][e] = x2;
        b3[j][e] = x3;
      }
  };

  floatx4 acc[MI][2];
#pragma unroll
  for (int i = 0; i < MI; ++i) acc[i][0] = acc[i][1] = floatx4{0.f, 0.f, 0.f, 0.f};
  // two chunks in flight: chunk j is loaded at the start of step j - 2 and
  // staged at the end of step j - 1, so its loads have two steps to land
  fetch(0, 0);
  if (KC < K) fetch(KC, 1);
  stash(0);
  for (int k0 = 0; k0 < K; k0 += 2 * KC) {
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int kc = k0 + s * KC;
      if (kc >= K) break;
      // stage s holds chunk kc; every wave is done with stage s ^ 1 (chunk kc - KC)
      __syncthreads();
      split_b(s);
      // unconditional: a chunk past K loads zeros (every lane's offset is past its resource), and a
      // conditional refill made the compiler wait for all loads in flight to merge the register sets
      fetch(kc + 2 * KC, s);
      const __bf16* const Ap = lds + s * STG;
      // lane l: A rows l % 16 and B columns l % 16, k = 8 (l / 16) + 0..7
#pragma unroll
      for (int i = 0; i < MI; ++i) {
        const int o = (wr * RW + i * 16 + (lane & 15)) * KP + kl;
        const bf16x8 a1 = *reinterpret_cast<const bf16x8*>(Ap + o);
        if constexpr (A1_ONLY) {
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            floatx4 c = acc[i][j];
            c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b3[j], c, 0, 0, 0);   // small terms first
            c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b2[j], c, 0, 0, 0);
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b1[j], c, 0, 0, 0);
          }
        } else {
          const bf16x8 a2 = *reinterpret_cast<const bf16x8*>(Ap + AB + o);
          if constexpr (SIX) {
            const bf16x8 a3 = *reinterpret_cast<const bf16x8*>(Ap + 2 * AB + o);
#pragma unroll
            for (int j = 0; j < 2; ++j) {
              floatx4 c = acc[i][j];
              c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a3, b1[j], c, 0, 0, 0);   // small terms first
              c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2, b2[j], c, 0, 0, 0);
              c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b3[j], c, 0, 0, 0);
              c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2, b1[j], c, 0, 0, 0);
              c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b2[j], c, 0, 0, 0);
              acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b1[j], c, 0, 0, 0);
            }
          } else {
#pragma unroll
            for (int j = 0; j < 2; ++j) {
              floatx4 c = acc[i][j];
              c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2, b1[j], c, 0, 0, 0);   // small terms first
              c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b2[j], c, 0, 0, 0);
              acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b1[j], c, 0, 0, 0);
            }
          }
        }
      }
      // the next chunk's A into the other stage
      if (kc + KC < K) stash(s ^ 1);
    }
  }

  // epilogue: lane holds rows 16 i + 4 (lane / 16) + r of column lane % 16 of n-tile j
  if constexpr (OUT_SPLIT) {
    // 1) bias and activation in place; the activation is one wave-uniform
    //    branch when both halves use the same one
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int gn = n0 + wn * 32 + j * 16 + (lane & 15);
      const float bv = gn < N ? bias[gn] : 0.0f;
      const int act = gn < NH ? act_lo : act_hi;
      if (act_lo == act_hi && act_lo == 0) {
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[i][j][r] += bv;
      } else {
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float v = acc[i][j][r] + bv;
            const float sg = __builtin_amdgcn_rcpf(1.0f + __expf(-v));
            acc[i][j][r] = act == 1 ? v * sg : (act == 2 ? sg : v);
          }
      }
    }
    // 2) channel sums per (tile, frame): the tile's rows m0 .. m0 + 127 cover
    //    frames tf0 .. tf0 + slots - 1; frame tf0 + q goes to slot q of the
    //    tile.  With HW >= 16 (host-checked) a 16-row block i spans frames fa,
    //    fa + 1 (fa = frame of row m0 + 16 i, uniform); each lane keeps its
    //    sums of the current frame rf (run) and of rf + 1 (nxt) and the wave
    //    writes a slot when the blocks leave its frame, so every slot is
    //    written once.
    if (partial != nullptr) {
      const int gmb = m0 + (lane >> 4) * 4;
      const int tf0 = m0 / HW;
      const int last_row = (M - m0 < TM ? M : m0 + TM) - 1;
      auto flush = [&](float x, int slot, int c, bool on) {
        x += __shfl_xor(x, 16, 64);
        x += __shfl_xor(x, 32, 64);
        if (on && lane < 16) partial[(size_t(rt) * slots + slot) * NH + c] = x;
      };
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int gn = n0 + wn * 32 + j * 16 + (lane & 15);
        const bool on = gn < N && gn < NH;
        float run = 0.0f, nxt = 0.0f;
        int rf = tf0, fa = tf0, pa_ = m0 % HW;   // uniform: frame / pixel of row m0 + 16 i
        int fr = gmb / HW, p = gmb % HW;          // this lane's row gmb + 16 i
#pragma unroll
        for (int i = 0; i < MI; ++i) {
          if (fa != rf) {   // fa == rf + 1
            flush(run, rf - tf0, gn, on);
            run = nxt;
            nxt = 0.0f;
            rf = fa;
          }
          // value r is row gmb + 16 i + r: frame fr, or fr + 1 once p + r passes HW; rows beyond M add nothing
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float x = gmb + i * 16 + r < M ? acc[i][j][r] : 0.0f;
            // act 3: the stored lower half stays pre-activation, its channel sums are of SiLU
            if (act_lo == 3) x = x * __builtin_amdgcn_rcpf(1.0f + __expf(-x));
            if (fr + (p + r >= HW ? 1 : 0) != rf) nxt += x;
            else run += x;
          }
          p += 16;
          while (p >= HW) {
            p -= HW;
            ++fr;
          }
          pa_ += 16;
          while (pa_ >= HW) {
            pa_ -= HW;
            ++fa;
          }
        }
        flush(run, rf - tf0, gn, on);
        if (last_row / HW > rf) flush(nxt, rf + 1 - tf0, gn, on);
      }
    }
    // 3) stores through LDS, one n-tile j (16 columns) per wave at a time:
    //    the wave writes its values as [column][row], then LPC lanes store
    //    one column's TM rows, 4 consecutive rows per lane, so a store
    //    instruction covers 64 / LPC runs of consecutive pixels
    __syncthreads();   // every wave is done reading the A stages
    float* const stg = reinterpret_cast<float*>(lds) + wn * (16 * SPC);
    constexpr int LPC = TM / 4, CPI = 64 / LPC;   // lanes per column, columns per store
    const int q = lane % LPC, half = lane / LPC;
    const int row0 = m0 + 4 * q;                  // this lane's 4 rows
    const int rfr = row0 / HW, rpx = row0 % HW;   // frame / pixel of row0
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      if (j > 0) wave_fence();   // every lane has read n-tile j - 1 before it is overwritten
#pragma unroll
      for (int i = 0; i < MI; ++i)
        *reinterpret_cast<floatx4*>(&stg[(lane & 15) * SPC + i * 16 + (lane >> 4) * 4]) = acc[i][j];
      wave_fence();              // the wave's writes are visible to its other lanes
#pragma unroll
      for (int cp = 0; cp < 16 / CPI; ++cp) {
        const int cl = CPI * cp + half;
        const int gn = n0 + wn * 32 + j * 16 + cl;
        if (gn >= N) continue;
        const bool lo = gn < NH;
        const int c = lo ? gn : gn - NH, NC = lo ? NH : NL;
        TO* dst = lo ? out_lo : out_hi;
        // one way for the whole tile (uniform), so every row is stored by exactly one lane
        if ((HW % 4) == 0 && m0 + TM <= M) {
          const floatx4 v4 = *reinterpret_cast<const floatx4*>(&stg[cl * SPC + 4 * q]);
          const float v[4] = {v4[0], v4[1], v4[2], v4[3]};
          st4(dst, size_t(rfr * NC + c) * HW + rpx, v);
        } else {
          // element stores: lane q takes rows q, q + TM/4, q + TM/2, q + 3TM/4 of the column, so one
          // store instruction writes TM/4 consecutive rows (pixels) instead of every fourth one
          int f2 = (m0 + q) / HW, p2 = (m0 + q) % HW;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int row = m0 + q + r * (TM / 4);
            if (row < M) st_el(dst, size_t(f2 * NC + c) * HW + p2, stg[cl * SPC + q + r * (TM / 4)]);
            p2 += TM / 4;
            while (p2 >= HW) {
              p2 -= HW;
              ++f2;
            }
          }
        }
      }
    }
  } else {
    // channels-last: stage 64 rows at a time in LDS, then whole-row stores of 4 columns per lane;
    // the waves whose row blocks fall in the 64 rows stage them
    float* st = reinterpret_cast<float*>(lds);
#pragma unroll
    for (int h = 0; h < TM / 64; ++h) {
      __syncthreads();
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int cl = wn * 32 + j * 16 + (lane & 15);
        const float bv = n0 + cl < N ? bias[n0 + cl] : 0.0f;
#pragma unroll
        for (int i = 0; i < MI; ++i) {
          const int rb = wr * RW + i * 16 - h * 64;   // block's first row within these 64 (uniform)
          if (rb < 0 || rb >= 64) continue;
#pragma unroll
          for (int r = 0; r < 4; ++r) st[(rb + (lane >> 4) * 4 + r) * OP + cl] = acc[i][j][r] + bv;
        }
      }
      __syncthreads();
      for (int f = tid; f < 64 * (TN / 4); f += NT) {
        const int r = f / (TN / 4), c4 = (f % (TN / 4)) * 4;
        const int gm = m0 + h * 64 + r, gn = n0 + c4;
        if (gm >= M) continue;
        const float* src = &st[r * OP + c4];
        if (gn + 3 < N && (N % 4) == 0) {
          const float v[4] = {src[0], src[1], src[2], src[3]};
          st4(out_lo, size_t(gm) * N + gn, v);
        } else {
          for (int e = 0; e < 4; ++e)
            if (gn + e < N) st_el(out_lo, size_t(gm) * N + gn + e, src[e]);
        }
      }
    }
  }
}

// ----------------------------------------------------------------- launchers

constexpr int kProjTM = 64;      // row tile of the general kernels
constexpr int kPersistTM = 128;  // row tile of the persistent small-K kernels

static int cu_count() {
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess) {
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) cus = 256;
  }
  return cus;
}

static int persistent_grid(int tiles) {
  const int g = 2 * cu_count();   // two workgroups per CU
  return tiles < g ? tiles : g;
}

// K <= kPersistMaxK: persistent kernel (weights in registers); larger K with K % 4 == 0
// (or any K for plane-major A): K-chunked kernel; otherwise the fp32 tiled kernels
constexpr int kPersistMaxK = 64;
constexpr int kKcTM = 128;   // row tile of the K-chunked kernel

int proj_in_tile_rows(int K) { return K % 4 == 0 ? kPersistTM : kProjTM; }

// channel-sum slots per row tile (partial sums of ctx): 1 when every tile
// lies in one frame; the K-chunked kernel also sums tiles spanning frames,
// one slot per frame (needs HW >= 16); 0: no fused sums for this shape
int proj_in_ctx_slots(int K, int HW) {
  const int tm = proj_in_tile_rows(K);
  if (HW % tm == 0) return 1;
  if (K > kPersistMaxK && K % 4 == 0 && HW >= 16) return (kKcTM - 2) / HW + 2;
  return 0;
}

template <bool PLANE_A, bool OUT_SPLIT, class TI, class TO, int TM, int TN = 128>
static hipError_t launch_kc_tm(const void* A, int M, int K, int N, const float* W, const float* b, int HW, void* lo,
                               void* hi, int act_lo, int act_hi, float* partial, int NH, hipStream_t s) {
  // the kernel's buffer resources (one row tile of A, all of W) must stay below 2^31 bytes, the
  // offset its out-of-range lanes load at
  const long long a_bytes = PLANE_A ? (long long)((TM - 2) / HW + 2) * K * HW * (long long)sizeof(TI)
                                    : (long long)TM * K * (long long)sizeof(TI);
  if (a_bytes >= (1LL << 31) || (long long)K * N * 4 >= (1LL << 31)) return hipErrorInvalidValue;
  const dim3 grid(unsigned((M + TM - 1) / TM) * unsigned((N + TN - 1) / TN));
  const int slots = partial ? proj_in_ctx_slots(K, HW) : 0;
  if constexpr (PLANE_A) {
    if (HW % 4 == 0) {
      hipLaunchKernelGGL((proj_kc_kernel<PLANE_A, OUT_SPLIT, TI, TO, TM, true, TN>), grid, dim3(256), 0, s,
                         static_cast<const TI*>(A), M, K, N, W, b, HW, static_cast<TO*>(lo), static_cast<TO*>(hi),
                         act_lo, act_hi, partial, NH, slots);
      return hipGetLastError();
    }
  }
  hipLaunchKernelGGL((proj_kc_kernel<PLANE_A, OUT_SPLIT, TI, TO, TM, false, TN>), grid, dim3(256), 0, s,
                     static_cast<const TI*>(A), M, K, N, W, b, HW, static_cast<TO*>(lo), static_cast<TO*>(hi), act_lo,
                     act_hi, partial, NH, slots);
  return hipGetLastError();
}

// 128-row tiles; channels-last outputs (proj_out, narrow N) whose 128-row
// tiles would leave CUs idle take 64-row tiles (twice the workgroups)
template <bool PLANE_A, bool OUT_SPLIT, class TI, class TO>
static hipError_t launch_kc(const void* A, int M, int K, int N, const float* W, const float* b, int HW, void* lo,
                            void* hi, int act_lo, int act_hi, float* partial, int NH, hipStream_t s) {
  if constexpr (!OUT_SPLIT) {
    // narrow outputs: 64-column tiles (no wave on columns past N)
    if (N <= 64) {
      const long long tiles = (M + kKcTM - 1) / kKcTM;
      if (tiles < cu_count())
        return launch_kc_tm<PLANE_A, OUT_SPLIT, TI, TO, 64, 64>(A, M, K, N, W, b, HW, lo, hi, act_lo, act_hi, partial,
                                                              NH, s);
      return launch_kc_tm<PLANE_A, OUT_SPLIT, TI, TO, kKcTM, 64>(A, M, K, N, W, b, HW, lo, hi, act_lo, act_hi, partial,
                                                                 NH, s);
    }
    const long long tiles = (long long)((M + kKcTM - 1) / kKcTM) * ((N + 127) / 128);
    if (tiles < cu_count())
      return launch_kc_tm<PLANE_A, OUT_SPLIT, TI, TO, 64>(A, M, K, N, W, b, HW, lo, hi, act_lo, act_hi, partial, NH, s);
  }
  return launch_kc_tm<PLANE_A, OUT_SPLIT, TI, TO, kKcTM>(A, M, K, N, W, b, HW, lo, hi, act_lo, act_hi, partial, NH, s);
}

template <class TI, class TO>
static void launch_in(const void* X, int M, int K, int N, const float* W, const float* b, int HW, void* lo, void* hi,
                      int act_lo, int act_hi, float* partial, int NH, hipStream_t s) {
  const dim3 grid((M + kProjTM - 1) / kProjTM, (N + 127) / 128);
  hipLaunchKernelGGL((proj_in_kernel<kProjTM, 128, 1, 4, TI, TO>), grid, dim3(256), 0, s, static_cast<const TI*>(X), M,
                     K, N, W, b, HW, static_cast<TO*>(lo), static_cast<TO*>(hi), act_lo, act_hi, partial, NH);
}

// bf16x3 MFMA for every persistent projection except the norm / gate prologue (fp32)
template <int KMAX, bool PLANE_A, bool OUT_SPLIT, bool NORM, class TI, class TO, bool PX1 = false, bool SPLIT = !NORM>
static void launch_persist(const void* A, int M, int K, int N, const float* W, const float* b, int HW, void* lo,
                           void* hi, int act_lo, int act_hi, float* partial, int NH, const NormGate& ng,
                           hipStream_t s) {
  const int tiles = (M + kPersistTM - 1) / kPersistTM;
  // narrow outputs (N <= 64) split the rows between wave pairs instead of idling half the waves
  // (plane-major outputs only without the channel sums, which need whole row tiles per wave)
  {
    if (N <= 64 && (!OUT_SPLIT || partial == nullptr)) {
      const dim3 grid(unsigned(persistent_grid(tiles)), unsigned((N + 63) / 64));
      hipLaunchKernelGGL((proj_persist_kernel<KMAX, PLANE_A, OUT_SPLIT, 2, TI, TO, NORM, SPLIT, 0, false, PX1>), grid, dim3(256), 0, s,
                         static_cast<const TI*>(A), M, K, N, W, b, HW, static_cast<TO*>(lo), static_cast<TO*>(hi),
                         act_lo, act_hi, partial, NH, ng, QkvPost{});
      return;
    }
  }
  const dim3 grid(unsigned(persistent_grid(tiles)), unsigned((N + 127) / 128));
  hipLaunchKernelGGL((proj_persist_kernel<KMAX, PLANE_A, OUT_SPLIT, 4, TI, TO, NORM, SPLIT, 0, false, PX1>), grid, dim3(256), 0, s,
                     static_cast<const TI*>(A), M, K, N, W, b, HW, static_cast<TO*>(lo), static_cast<TO*>(hi),
                     act_lo, act_hi, partial, NH, ng, QkvPost{});
}

template <bool PLANE_A, bool OUT_SPLIT, bool NORM, class TI, class TO, bool PX1 = false>
static bool try_persist(const void* A, int M, int K, int N, const float* W, const float* b, int HW, void* lo,
                        void* hi, int act_lo, int act_hi, float* partial, int NH, const NormGate& ng, hipStream_t s) {
  if (K % 4 != 0 || K > 128) return false;
  if (K <= 64) {
    launch_persist<64, PLANE_A, OUT_SPLIT, NORM, TI, TO, PX1>(A, M, K, N, W, b, HW, lo, hi, act_lo, act_hi, partial, NH, ng, s);
    return true;
  }
  // 64 < K <= 128 only for the norm / gate prologue (the other projections take the K-chunked kernel there)
  if constexpr (NORM) {
    launch_persist<128, PLANE_A, OUT_SPLIT, NORM, TI, TO, PX1>(A, M, K, N, W, b, HW, lo, hi, act_lo, act_hi, partial, NH, ng, s);
    return true;
  }
  return false;
}

// plane-major output(s) from channels-last X: channels [0, NH) -> lo, [NH, N) -> hi
hipError_t launch_proj_planes(const void* X, int in_dtype, int M, int K, int N, const float* W, const float* b,
                              int HW, void* out_lo, void* out_hi, int out_dtype, int act_lo, int act_hi,
                              float* partial, int NH, hipStream_t s) {
  const NormGate ng{nullptr, nullptr, nullptr, 0};
  if (K > kPersistMaxK && K % 4 == 0) {
    if (in_dtype == 0 && out_dtype == 0)
      return launch_kc<false, true, float, float>(X, M, K, N, W, b, HW, out_lo, out_hi, act_lo, act_hi, partial, NH, s);
    if (in_dtype == 0)
      return launch_kc<false, true, float, uint16_t>(X, M, K, N, W, b, HW, out_lo, out_hi, act_lo, act_hi, partial, NH,
                                                     s);
    if (out_dtype == 0)
      return launch_kc<false, true, uint16_t, float>(X, M, K, N, W, b, HW, out_lo, out_hi, act_lo, act_hi, partial, NH,
                                                     s);
    return launch_kc<false, true, uint16_t, uint16_t>(X, M, K, N, W, b, HW, out_lo, out_hi, act_lo, act_hi, partial,
                                                      NH, s);
  }
  if (K <= kPersistMaxK && K % 4 == 0) {
    if (in_dtype == 0 && out_dtype == 0)
      try_persist<false, true, false, float, float>(X, M, K, N, W, b, HW, out_lo, out_hi, act_lo, act_hi, partial, NH, ng, s);
    else if (in_dtype == 0)
      try_persist<false, true, false, float, uint16_t>(X, M, K, N, W, b, HW, out_lo, out_hi, act_lo, act_hi, partial, NH, ng, s);
    else if (out_dtype == 0)
      try_persist<false, true, false, uint16_t, float>(X, M, K, N, W, b, HW, out_lo, out_hi, act_lo, act_hi, partial, NH, ng, s);
    else
      try_persist<false, true, false, uint16_t, uint16_t>(X, M, K, N, W, b, HW, out_lo, out_hi, act_lo, act_hi, partial, NH, ng, s);
    return hipGetLastError();
  }
  if (in_dtype == 0 && out_dtype == 0) launch_in<float, float>(X, M, K, N, W, b, HW, out_lo, out_hi, act_lo, act_hi, partial, NH, s);
  else if (in_dtype == 0) launch_in<float, uint16_t>(X, M, K, N, W, b, HW, out_lo, out_hi, act_lo, act_hi, partial, NH, s);
  else if (out_dtype == 0) launch_in<uint16_t, float>(X, M, K, N, W, b, HW, out_lo, out_hi, act_lo, act_hi, partial, NH, s);
  else launch_in<uint16_t, uint16_t>(X, M, K, N, W, b, HW, out_lo, out_hi, act_lo, act_hi, partial, NH, s);
  return hipGetLastError();
}

hipError_t launch_proj_in(const void* X, int in_dtype, int M, int K, int N, const float* W, const float* b, int HW,
                          void* out_lo, void* out_hi, int out_dtype, int act_lo, int act_hi, float* partial,
                          hipStream_t s) {
  return launch_proj_planes(X, in_dtype, M, K, N, W, b, HW, out_lo, out_hi, out_dtype, act_lo, act_hi, partial,
                            N / 2, s);
}

// ---------------------------------------------------------------------------
// GDN qkv projection, frame-sequential: qkv_proj + causal short conv + SiLU +
// input gates (+ gate_proj columns), computing what the tiled epilogue of
// proj_persist_kernel (TT > 0) computes, operation for operation.  A tile is
// 64 consecutive pixels of ONE frame x 128 output columns; a workgroup walks
// the T frames of one (batch element, pixel block) in order, and each lane
// keeps the pre-conv projections of its 32 elements on the three previous
// frames in registers (the taps on frames t-1 .. t-3: kt <= 4, or T <= 4 where
// earlier taps only meet the zero padding).  A wave owns all 64 rows of its 32
// columns, so its four stores per column write 256 contiguous bytes of one
// plane; the tiles of 16 pixels x 8 frames wrote 64-byte runs into eight
// frames' planes at once, and that write pattern, not the arithmetic, bounded
// them (same loads and stores with no MFMA or epilogue math: same time).
// ---------------------------------------------------------------------------
constexpr int kFseqTM = 64;
// CBW 128-column blocks per workgroup (4 waves each) share one staged A tile: A is read from HBM
// once for all of them (separate workgroups per column block drift apart and miss in L2)
// GC: the launch has gate_proj columns (qp.ng > 0); false compiles out their stores
template <int CBW, class TI, class TO, bool GC = true>
__global__ void __launch_bounds__(256 * CBW, 2 / CBW)
qkv_fseq_kernel(const TI* __restrict__ A, int T, int HW, int K, int N, const float* __restrict__ Wt,
                const float* __restrict__ bias, int nseq, TO* __restrict__ out, QkvPost qp) {
  constexpr int TM = kFseqTM, TN = 128, NT = 256 * CBW, MI = TM / 16, KMAX = 64, KB = KMAX / 32, KP = KMAX + 8;
  constexpr bool A1_ONLY = sizeof(TI) == 2;      // bf16 A is exactly its first bf16 part
  constexpr int APL = A1_ONLY ? 1 : 3;
  constexpr int PF = TM * KMAX / 4 / NT;         // groups of 4 consecutive k per thread and tile
  constexpr int KH = 3;                          // earlier frames the conv reads
  constexpr unsigned kDrop = 0x80000000u;        // a buffer offset past every resource's range
  __shared__ __attribute__((aligned(16))) __bf16 Asm[APL * TM * KP];
  __shared__ __attribute__((aligned(16))) float qcw[CBW * TN * 8];
  __shared__ __attribute__((aligned(16))) float2 gsh[TM];   // 16-byte reads of 2 pixels' gates
  __bf16* const A1 = Asm;
  __bf16* const A2 = A1 + (APL > 1 ? TM * KP : 0);
  __bf16* const A3 = A2 + (APL > 1 ? TM * KP : 0);
  const int tid = threadIdx.x, lane = tid & 63, wn = (tid >> 6) & 3, cq = tid >> 8;
  const int nb = blockIdx.y * CBW * TN;          // the workgroup's first column
  const int n0 = nb + cq * TN, C = N / 3, NG = N + qp.ng;   // this wave's column block
  const int tpf = HW / TM;                       // pixel blocks per frame
  // column offset (within the workgroup's CBW * 128 columns) of this lane's column in its column tile j.
  // With gate columns filling a 256-column workgroup (3C + C = 256) the 16-column tiles are dealt so
  // that waves w and w + 4 together hold three qkv tiles and one gate tile: waves 0-3 take qkv tiles
  // 2w, 2w + 1, waves 4-7 qkv tile 8 + (w - 4) and gate tile 12 + (w - 4)
  const bool deal = CBW == 2 && qp.ng > 0 && N + qp.ng == 256;
  auto jcol = [&](int j) -> int {
    const int w = cq * 4 + wn;
    const int jt = !deal ? w * 2 + j : (w < 4 ? 2 * w + j : (j == 0 ? 8 + (w - 4) : 12 + (w - 4)));
    return jt * 16 + (lane & 15);
  };

  // B fragments: lane l holds column wn 32 + 16 j + l % 16, k = 32 kb + 8 (l / 16) + e, in three bf16 parts
  bf16x8 b1[2][KB], b2[2][KB], b3[2][KB];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int gn = nb + jcol(j);
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int kk = kb * 32 + (lane >> 4) * 8 + e;
        float w = 0.0f;
        if (kk < K) {
          if (gn < N) w = Wt[size_t(kk) * N + gn];
          else if (gn < NG) w = qp.wg[size_t(kk) * qp.ng + (gn - N)];
        }
        __bf16 x1, x2, x3;
        split3_bf16(w, x1, x2, x3);
        b1[j][kb][e] = x1;
        b2[j][kb][e] = x2;
        b3[j][kb][e] = x3;
      }
  }
  // per column: taps on frames t, t-1, t-2, t-3 (zero beyond kt), projection bias, conv bias;
  // gate_proj columns: no taps, their bias
  for (int cl = tid; cl < CBW * TN; cl += NT) {
    const int gn = nb + cl;
    float* e = &qcw[cl * 8];
#pragma unroll
    for (int d = 0; d < 8; ++d) e[d] = 0.0f;
    if (gn < N) {
      const int blk = gn / C, c = gn % C;
#pragma unroll
      for (int d = 0; d <= KH; ++d) e[d] = d < qp.kt ? qp.w[blk][(qp.kt - 1 - d) * C + c] : 0.0f;
      e[4] = bias[gn];
      e[5] = qp.kt > 0 ? qp.b[blk][c] : 0.0f;
    } else if (gn < NG) {
      e[4] = qp.bg[gn - N];
    }
  }
  // per lane and column tile j: the store offset within a frame's planes of qkv (eo) or gv (eg),
  // kDrop where the column is not in that output; block 0 q, 1 k, 2 v, 3 gate_proj; the column's
  // channel among the 2C per-channel input-gate planes
  unsigned eo[2], eg[2];
  int eblk[2], egch[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int gn = nb + jcol(j);
    const unsigned l4 = unsigned(lane >> 4) * 4u;
    const bool live = gn < NG, gcol = gn >= N;
    const int blk = live ? (gcol ? 3 : gn / C) : 0;
    eblk[j] = blk;
    egch[j] = (blk == 1 || blk == 2) ? gn - C : 0;
    eo[j] = (live && !gcol) ? (unsigned(gn) * unsigned(HW) + l4) * sizeof(TO) : kDrop;
    eg[j] = (live && gcol) ? (unsigned(gn - N) * unsigned(HW) + l4) * sizeof(TO) : kDrop;
  }

  // A rows of tile (seq, t): pixels pb TM .. pb TM + TM - 1 of frame b T + t, channels-last
  float4 pf[PF];
  float2 gpf = make_float2(0.f, 0.f);
  const bool tile_gates = qp.gate_mode == 1 || qp.gate_mode == 2;
  auto fetch = [&](int seq, int t) {
    const int b = seq / tpf, pb = seq % tpf;
    const size_t fr = size_t(b) * T + t, row0 = fr * HW + size_t(pb) * TM;
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      const int f = i * NT + tid;
      const int r = f / (KMAX / 4), k4 = (f % (KMAX / 4)) * 4;
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (k4 < K) {
        if constexpr (A1_ONLY) {
          const uint2 raw = *reinterpret_cast<const uint2*>(A + (row0 + r) * K + k4);
          v = make_float4(__uint_as_float(raw.x), __uint_as_float(raw.y), 0.f, 0.f);
        } else {
          v = ld4(A, (row0 + r) * K + k4);
        }
      }
      pf[i] = v;
    }
    if (tile_gates && tid < TM)
      gpf = qp.gate_mode == 1 ? static_cast<const float2*>(qp.gates)[fr * HW + size_t(pb) * TM + tid]
                              : static_cast<const float2*>(qp.gates)[fr];
  };
  auto stash = [&]() {
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      const int f = i * NT + tid;
      const int r = f / (KMAX / 4), k4 = (f % (KMAX / 4)) * 4;
      const int o = r * KP + k4;
      if constexpr (A1_ONLY) {
        *reinterpret_cast<uint2*>(&A1[o]) = make_uint2(__float_as_uint(pf[i].x), __float_as_uint(pf[i].y));
      } else {
        const float x[4] = {pf[i].x, pf[i].y, pf[i].z, pf[i].w};
        bf16x4 v1, v2, v3;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          __bf16 x1, x2, x3;
          split3_bf16(x[e], x1, x2, x3);
          v1[e] = x1;
          v2[e] = x2;
          v3[e] = x3;
        }
        *reinterpret_cast<bf16x4*>(&A1[o]) = v1;
        *reinterpret_cast<bf16x4*>(&A2[o]) = v2;
        *reinterpret_cast<bf16x4*>(&A3[o]) = v3;
      }
    }
    if (tile_gates && tid < TM) gsh[tid] = gpf;
  };

  // pre-conv projections (with bias) of the lane's elements on the three previous frames, in
  // three slots whose roles rotate with the tile step's phase P (a compile-time constant):
  // frame t-1 in slot (P+2)%3, t-2 in (P+1)%3, t-3 in P, which the current frame then takes;
  // the loop runs the phases in turn, so no register moves shift the history
  floatx4 hs[3][MI][2];
  int seq = blockIdx.x, t = 0;
  if (seq < nseq) fetch(seq, 0);
  auto tile_step = [&](auto phase) -> bool {
    constexpr int P = decltype(phase)::value;
    if (seq >= nseq) return false;
    __syncthreads();            // the previous tile is done with Asm and gsh (and qcw is staged)
    stash();
    __syncthreads();
    int nt = t + 1, ns = seq;
    if (nt == T) {
      nt = 0;
      ns += gridDim.x;
    }
    if (ns < nseq) fetch(ns, nt);
    if (t == 0) {
#pragma unroll
      for (int q = 0; q < 3; ++q)
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j) hs[q][i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
    }

    floatx4 acc[MI][2];
#pragma unroll
    for (int i = 0; i < MI; ++i) acc[i][0] = acc[i][1] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      if (kb * 32 >= K) break;
      const int koff = kb * 32 + (lane >> 4) * 8;
#pragma unroll
      for (int i = 0; i < MI; ++i) {
        const int o = (i * 16 + (lane & 15)) * KP + koff;
        const bf16x8 a1 = *reinterpret_cast<const bf16x8*>(&A1[o]);
        if constexpr (A1_ONLY) {
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            floatx4 c = acc[i][j];
            c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b3[j][kb], c, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b2[j][kb], c, 0, 0, 0);
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b1[j][kb], c, 0, 0, 0);
          }
        } else {
          const bf16x8 a2 = *reinterpret_cast<const bf16x8*>(&A2[o]);
          const bf16x8 a3 = *reinterpret_cast<const bf16x8*>(&A3[o]);
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            floatx4 c = acc[i][j];
            c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a3, b1[j][kb], c, 0, 0, 0);   // small terms first
            c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2, b2[j][kb], c, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b3[j][kb], c, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2, b1[j][kb], c, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b2[j][kb], c, 0, 0, 0);
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b1[j][kb], c, 0, 0, 0);
          }
        }
      }
    }

    // epilogue: lane holds pixels 16 i + 4 (lane / 16) + r of column lane % 16 of column tile j
    const int b = seq / tpf, pb = seq % tpf;
    const size_t fr = size_t(b) * T + t;
    const __amdgpu_buffer_rsrc_t ro = make_rsrc(out + fr * N * HW, unsigned(N) * unsigned(HW) * sizeof(TO));
    const __amdgpu_buffer_rsrc_t rg =
        make_rsrc(static_cast<TO*>(qp.gv) + fr * qp.ng * HW, unsigned(qp.ng) * unsigned(HW) * sizeof(TO));
    const unsigned pxo = unsigned(pb * TM) * sizeof(TO);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int cl = jcol(j);
      const int blk = eblk[j];
      const float4 w4 = *reinterpret_cast<const float4*>(&qcw[cl * 8]);
      const float2 bb2 = *reinterpret_cast<const float2*>(&qcw[cl * 8 + 4]);
      const float bv = bb2.x, bt = bb2.y;
      // every lane issues the same stores: a lane whose column is in neither output has both offsets
      // at kDrop.  Without gate columns (GC false) the gv store is not compiled: issued to an empty range
      // it still took its turn in the memory pipeline (C4 qkv 0.96 -> 0.89 ms without it)
      auto store = [&](int i, const float* v) {
        const unsigned po = pxo + unsigned(i * 16) * sizeof(TO);
        bst4(ro, eo[j] + po, v, out);
        if constexpr (GC) bst4(rg, eg[j] + po, v, out);
      };
      if (blk == 3) {
#pragma unroll
        for (int i = 0; i < MI; ++i) {
          float v[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float x = acc[i][j][r] + bv;
            const float sg = __builtin_amdgcn_rcpf(1.0f + __expf(-x));   // as the plain projection's epilogue
            v[r] = qp.gact == 1 ? x * sg : sg;
          }
          store(i, v);
        }
      } else {
        const bool gated = blk != 0, kcol = blk == 1;
        // the lane's input gates: component 0 (B_k) for a k column, 1 (B_v) for a v column, none for q.
        // The (B_k, B_v) pairs of the lane's 4 pixels are two 16-byte LDS reads, issued by every lane and
        // then selected (no branch around the reads, and no wait between them)
        auto in_gate = [&](int i, float (&v)[4]) {
          if (tile_gates) {
            const float4* gp = reinterpret_cast<const float4*>(gsh + i * 16 + (lane >> 4) * 4);
            const float4 g01 = gp[0], g23 = gp[1];
            const float g[4] = {kcol ? g01.x : g01.y, kcol ? g01.z : g01.w, kcol ? g23.x : g23.y,
                                kcol ? g23.z : g23.w};
#pragma unroll
            for (int r = 0; r < 4; ++r) v[r] *= gated ? g[r] : 1.0f;
          } else if (qp.gate_mode == 3 && gated) {
            const float4 gg = *reinterpret_cast<const float4*>(
                static_cast<const float*>(qp.gates) + (fr * 2 * C + size_t(egch[j])) * HW + size_t(pb) * TM + i * 16 +
                (lane >> 4) * 4);
            v[0] *= gg.x;
            v[1] *= gg.y;
            v[2] *= gg.z;
            v[3] *= gg.w;
          }
        };
        if (qp.kt > 0) {
#pragma unroll
          for (int i = 0; i < MI; ++i) {
            float v[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const float x = acc[i][j][r] + bv;
              // the tiled epilogue's order: tap 0 and the conv bias, then the taps on t-3, t-2, t-1
              // (frames before the first are the zero padding, held as zeros)
              float o = fmaf(w4.x, x, bt);
              o = fmaf(w4.w, hs[P][i][j][r], o);
              o = fmaf(w4.z, hs[(P + 1) % 3][i][j][r], o);
              o = fmaf(w4.y, hs[(P + 2) % 3][i][j][r], o);
              v[r] = o * __builtin_amdgcn_rcpf(1.0f + __expf(-o));   // SiLU as gdn_qkv_post computes it
              hs[P][i][j][r] = x;   // frame t becomes the next phase's t-1
            }
            in_gate(i, v);
            store(i, v);
          }
        } else {
#pragma unroll
          for (int i = 0; i < MI; ++i) {
            float v[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) v[r] = acc[i][j][r] + bv;
            in_gate(i, v);
            store(i, v);
          }
        }
      }
    }
    seq = ns;
    t = nt;
    return true;
  };
  while (tile_step(std::integral_constant<int, 0>{}) && tile_step(std::integral_constant<int, 1>{}) &&
         tile_step(std::integral_constant<int, 2>{})) {
  }
}

// The tiled GDN qkv projection (persistent kernel, tiles of 128 / T' pixels x
// T' = min(T, 8) frames, the short conv, SiLU and input gates in its epilogue);
// returns false when the shape has no tiled variant (the caller then runs
// launch_proj_planes + launch_gdn_qkv_post, which compute the same values)
template <int TT, bool CARRY, class TI, class TO>
static void launch_qkv_fused(const void* X, int M, int K, int N, const float* W, const float* b, int HW, void* out,
                             const QkvPost& qp, hipStream_t s) {
  const int tiles = M / kPersistTM;
  const NormGate ng{nullptr, nullptr, nullptr, 0};
  const int nch = CARRY ? qp.T / TT : 1;
  // pixel blocks in pairs, each with its nch chunks.  The column blocks (3C = 192: two) of one
  // sequence of pixel blocks are resident together: the grid is sized so that every workgroup
  // fits at once, and ids x and x + gridDim.x land on the same XCD, so the second block's A
  // rows come from L2 (C3: 7.17 -> 6.59 ms against one grid of column block 0 before block 1)
  const int cb = (N + qp.ng + 127) / 128;
  const int slots = (2 * cu_count()) / cb > 0 ? (2 * cu_count()) / cb : 1;
  const int pbs = (tiles / nch + 1) / 2;
  const dim3 grid(unsigned(pbs < slots ? pbs : slots), unsigned(cb));
  hipLaunchKernelGGL((proj_persist_kernel<64, false, true, 4, TI, TO, false, true, TT, CARRY>), grid, dim3(256), 0, s,
                     static_cast<const TI*>(X), M, K, N, W, b, HW, static_cast<TO*>(out), static_cast<TO*>(out), 0, 0,
                     nullptr, N, ng, qp);
}

template <class TI, class TO>
static bool qkv_fused_t(const void* X, int T, int M, int K, int N, const float* W, const float* b, int HW, void* out,
                        const QkvPost& qp, hipStream_t s) {
  switch (T) {
    case 4: launch_qkv_fused<4, false, TI, TO>(X, M, K, N, W, b, HW, out, qp, s); return true;
    case 8: launch_qkv_fused<8, false, TI, TO>(X, M, K, N, W, b, HW, out, qp, s); return true;
    default:
      if (T % 8 != 0) return false;
      launch_qkv_fused<8, true, TI, TO>(X, M, K, N, W, b, HW, out, qp, s);
      return true;
  }
}

// The frame-sequential kernel: any T with kt <= 4, or T <= 4 (the taps on frames before the third
// earlier one only meet the zero padding); pixel blocks of 64
static bool qkv_fseq_supported(int T, int HW, int K, int kt) {
  return (kt <= 4 || T <= 4) && K <= kPersistMaxK && K % 4 == 0 && HW % kFseqTM == 0;
}

// The tiled kernel (where the frame-sequential one does not apply): T = 4 (one chunk; taps beyond
// the third earlier frame only meet the zero padding), or a multiple of 8 with kt <= 4 (the epilogue
// applies the taps on frames t .. t - 3; chunks of 8 frames carry 3); tiles of 128 / min(T, 8) pixels
static bool qkv_tiled_supported(int T, int HW, int K, int kt) {
  const bool t_ok = T == 4 || (T % 8 == 0 && kt <= 4);
  const int tp = kPersistTM / (T < 8 ? T : 8);
  return t_ok && K <= kPersistMaxK && K % 4 == 0 && HW % tp == 0;
}

bool gdn_qkv_fused_supported(int T, int HW, int K, int kt) {
  return qkv_fseq_supported(T, HW, K, kt) || qkv_tiled_supported(T, HW, K, kt);
}

template <class TI, class TO>
static void launch_qkv_fseq(const void* X, int B, int T, int HW, int K, int N, const float* W, const float* b,
                            void* out, const QkvPost& qp, hipStream_t s) {
  // (batch element, pixel block) sequences; column blocks of 128 in pairs per workgroup (one when
  // a single block holds every column), two workgroups' worth of waves per CU
  const int nseq = B * (HW / kFseqTM);
  const int cb = (N + qp.ng + 127) / 128;
  if (cb == 1) {
    const int slots = 2 * cu_count();
    const dim3 grid(unsigned(nseq < slots ? nseq : slots), 1u);
    hipLaunchKernelGGL((qkv_fseq_kernel<1, TI, TO>), grid, dim3(256), 0, s, static_cast<const TI*>(X), T, HW, K, N,
                       W, b, nseq, static_cast<TO*>(out), qp);
    return;
  }
  const int cy = (cb + 1) / 2;
  const int slots = cu_count() / cy > 0 ? cu_count() / cy : 1;
  const dim3 grid(unsigned(nseq < slots ? nseq : slots), unsigned(cy));
  if (qp.ng > 0)
    hipLaunchKernelGGL((qkv_fseq_kernel<2, TI, TO>), grid, dim3(512), 0, s, static_cast<const TI*>(X), T, HW, K, N, W,
                       b, nseq, static_cast<TO*>(out), qp);
  else
    hipLaunchKernelGGL((qkv_fseq_kernel<2, TI, TO, false>), grid, dim3(512), 0, s, static_cast<const TI*>(X), T, HW, K,
                       N, W, b, nseq, static_cast<TO*>(out), qp);
}

hipError_t launch_gdn_qkv_proj(const void* X, int in_dtype, int B, int T, int HW, int K, int C, const float* W,
                               const float* b, int kt, const GdnShortConv& sc, int gate_mode, const void* gates,
                               void* out, int out_dtype, hipStream_t s, const float* wg, const float* bg, int gact,
                               void* gv) {
  const int M = B * T * HW, N = 3 * C;
  const QkvPost qp{{sc.w[0], sc.w[1], sc.w[2]}, {sc.b[0], sc.b[1], sc.b[2]}, kt, gate_mode, gates, T,
                   wg, bg, wg ? C : 0, gact, gv};
  // the frame-sequential kernel stores through buffer resources over one frame's planes
  const size_t esz = out_dtype == 0 ? 4 : 2;
  if (qkv_fseq_supported(T, HW, K, kt) && kt <= 8 && size_t(N) * HW * esz < (size_t(1) << 31)) {
    if (in_dtype == 0 && out_dtype == 0) launch_qkv_fseq<float, float>(X, B, T, HW, K, N, W, b, out, qp, s);
    else if (in_dtype == 0) launch_qkv_fseq<float, uint16_t>(X, B, T, HW, K, N, W, b, out, qp, s);
    else if (out_dtype == 0) launch_qkv_fseq<uint16_t, float>(X, B, T, HW, K, N, W, b, out, qp, s);
    else launch_qkv_fseq<uint16_t, uint16_t>(X, B, T, HW, K, N, W, b, out, qp, s);
    return hipGetLastError();
  }
  if (qkv_tiled_supported(T, HW, K, kt) && kt <= 8) {
    if (in_dtype == 0 && out_dtype == 0) qkv_fused_t<float, float>(X, T, M, K, N, W, b, HW, out, qp, s);
    else if (in_dtype == 0) qkv_fused_t<float, uint16_t>(X, T, M, K, N, W, b, HW, out, qp, s);
    else if (out_dtype == 0) qkv_fused_t<uint16_t, float>(X, T, M, K, N, W, b, HW, out, qp, s);
    else qkv_fused_t<uint16_t, uint16_t>(X, T, M, K, N, W, b, HW, out, qp, s);
    return hipGetLastError();
  }
  hipError_t e = launch_proj_planes(X, in_dtype, M, K, N, W, b, HW, out, nullptr, out_dtype, 0, 0, nullptr, N, s);
  if (e != hipSuccess) return e;
  if (wg) {
    e = launch_proj_planes(X, in_dtype, M, K, C, wg, bg, HW, gv, gv, out_dtype, gact, gact, nullptr, C, s);
    if (e != hipSuccess) return e;
  }
  return launch_gdn_qkv_post(out, out_dtype, B, T, C, HW, kt, sc, gate_mode, gates, s);
}

hipError_t launch_proj_out(const void* Y, int in_dtype, int M, int K, int N, const float* W, const float* b, int HW,
                           void* out, int out_dtype, hipStream_t s) {
  const NormGate ng{nullptr, nullptr, nullptr, 0};
  if (K > kPersistMaxK || K % 4 != 0 || HW % 4 != 0) {
    if (in_dtype == 0 && out_dtype == 0)
      return launch_kc<true, false, float, float>(Y, M, K, N, W, b, HW, out, nullptr, 0, 0, nullptr, N, s);
    if (in_dtype == 0)
      return launch_kc<true, false, float, uint16_t>(Y, M, K, N, W, b, HW, out, nullptr, 0, 0, nullptr, N, s);
    if (out_dtype == 0)
      return launch_kc<true, false, uint16_t, float>(Y, M, K, N, W, b, HW, out, nullptr, 0, 0, nullptr, N, s);
    return launch_kc<true, false, uint16_t, uint16_t>(Y, M, K, N, W, b, HW, out, nullptr, 0, 0, nullptr, N, s);
  }
  {
    if (in_dtype == 0 && out_dtype == 0)
      try_persist<true, false, false, float, float>(Y, M, K, N, W, b, HW, out, nullptr, 0, 0, nullptr, N, ng, s);
    else if (in_dtype == 0)
      try_persist<true, false, false, float, uint16_t>(Y, M, K, N, W, b, HW, out, nullptr, 0, 0, nullptr, N, ng, s);
    else if (out_dtype == 0)
      try_persist<true, false, false, uint16_t, float>(Y, M, K, N, W, b, HW, out, nullptr, 0, 0, nullptr, N, ng, s);
    else
      try_persist<true, false, false, uint16_t, uint16_t>(Y, M, K, N, W, b, HW, out, nullptr, 0, 0, nullptr, N, ng, s);
    return hipGetLastError();
  }
}

// output projection with the per-pixel channel norm and the gate fused in front
// (persistent kernel only: K <= 128, K % 4 == 0, HW % 4 == 0; else invalid value)
hipError_t launch_proj_out_norm_gate(const void* Y, const void* G, int in_dtype, int M, int K, int N, int norm,
                                     const float* nscale, const float* nshift, const float* W, const float* b, int HW,
                                     void* out, int out_dtype, hipStream_t s) {
  if (!(K <= 128 && K % 4 == 0)) return hipErrorInvalidValue;
  const NormGate ng{G, nscale, nshift, norm};
  if (HW % 4 == 0) {
    if (in_dtype == 0 && out_dtype == 0)
      try_persist<true, false, true, float, float>(Y, M, K, N, W, b, HW, out, nullptr, 0, 0, nullptr, N, ng, s);
    else if (in_dtype == 0)
      try_persist<true, false, true, float, uint16_t>(Y, M, K, N, W, b, HW, out, nullptr, 0, 0, nullptr, N, ng, s);
    else if (out_dtype == 0)
      try_persist<true, false, true, uint16_t, float>(Y, M, K, N, W, b, HW, out, nullptr, 0, 0, nullptr, N, ng, s);
    else
      try_persist<true, false, true, uint16_t, uint16_t>(Y, M, K, N, W, b, HW, out, nullptr, 0, 0, nullptr, N, ng, s);
  } else {
    if (in_dtype == 0 && out_dtype == 0)
      try_persist<true, false, true, float, float, true>(Y, M, K, N, W, b, HW, out, nullptr, 0, 0, nullptr, N, ng, s);
    else if (in_dtype == 0)
      try_persist<true, false, true, float, uint16_t, true>(Y, M, K, N, W, b, HW, out, nullptr, 0, 0, nullptr, N, ng, s);
    else if (out_dtype == 0)
      try_persist<true, false, true, uint16_t, float, true>(Y, M, K, N, W, b, HW, out, nullptr, 0, 0, nullptr, N, ng, s);
    else
      try_persist<true, false, true, uint16_t, uint16_t, true>(Y, M, K, N, W, b, HW, out, nullptr, 0, 0, nullptr, N, ng,
                                                               s);
  }
  return hipGetLastError();
}

// the same with the gate computed from the layer input X (bf16 channels-last (M, K)): gate_proj in the
// kernel (K <= 64, K % 8 == 0, N <= 64, HW % 4 == 0; else invalid value)
bool proj_out_xgate_supported(int K, int N, int HW) { return K <= 64 && K % 8 == 0 && N <= 64 && HW % 4 == 0; }

template <class TI, class TO, bool XF>
static void launch_xgate(const void* Y, int M, int K, int N, const NormGate& ng, const float* W, const float* b, int HW,
                         void* out, hipStream_t s) {
  const int tiles = (M + kPersistTM - 1) / kPersistTM;
  const dim3 grid(unsigned(persistent_grid(tiles)), 1);
  hipLaunchKernelGGL((proj_persist_kernel<64, true, false, 2, TI, TO, true, false, 0, false, false, true, XF>), grid,
                     dim3(256), 0, s, static_cast<const TI*>(Y), M, K, N, W, b, HW, static_cast<TO*>(out), nullptr, 0,
                     0, nullptr, N, ng, QkvPost{});
}

hipError_t launch_proj_out_norm_xgate(const void* Y, int in_dtype, const void* X, int x_dtype, int M, int K, int N,
                                      int norm, const float* nscale, const float* nshift, const float* wg,
                                      const float* bg, int gact, const float* W, const float* b, int HW, void* out,
                                      int out_dtype, hipStream_t s) {
  if (!proj_out_xgate_supported(K, N, HW)) return hipErrorInvalidValue;
  NormGate ng{nullptr, nscale, nshift, norm};
  ng.X = x_dtype == 0 ? nullptr : static_cast<const uint16_t*>(X);
  ng.Xf = x_dtype == 0 ? static_cast<const float*>(X) : nullptr;
  ng.wg = wg;
  ng.bg = bg;
  ng.gact = gact;
  if (x_dtype == 0) {
    if (in_dtype == 0 && out_dtype == 0) launch_xgate<float, float, true>(Y, M, K, N, ng, W, b, HW, out, s);
    else if (in_dtype == 0) launch_xgate<float, uint16_t, true>(Y, M, K, N, ng, W, b, HW, out, s);
    else if (out_dtype == 0) launch_xgate<uint16_t, float, true>(Y, M, K, N, ng, W, b, HW, out, s);
    else launch_xgate<uint16_t, uint16_t, true>(Y, M, K, N, ng, W, b, HW, out, s);
  } else {
    if (in_dtype == 0 && out_dtype == 0) launch_xgate<float, float, false>(Y, M, K, N, ng, W, b, HW, out, s);
    else if (in_dtype == 0) launch_xgate<float, uint16_t, false>(Y, M, K, N, ng, W, b, HW, out, s);
    else if (out_dtype == 0) launch_xgate<uint16_t, float, false>(Y, M, K, N, ng, W, b, HW, out, s);
    else launch_xgate<uint16_t, uint16_t, false>(Y, M, K, N, ng, W, b, HW, out, s);
  }
  return hipGetLastError();
}

hipError_t launch_ctx_reduce(const float* partial, int F, int HW, int tile_rows, int slots, int C, float* ctx,
                             hipStream_t s) {
  hipLaunchKernelGGL(ctx_reduce_kernel, dim3(unsigned(F)), dim3(256), 0, s, partial, F, HW, tile_rows, slots, C, ctx);
  return hipGetLastError();
}

}  // namespace cssm
