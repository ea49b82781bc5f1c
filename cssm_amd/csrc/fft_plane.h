// 2-D real FFT of power-of-two planes staged in LDS (gfx950), shared by the
// fused gated scan and the batched transforms of the GDN cell.
//
// A workgroup owns NP planes of H x W real samples.  The transform runs as
// in-register radix-H1/H2/W1/W2 passes with an LDS exchange between them
// (H = H1*H2, W = W1*W2); every pass writes its results back into exactly the
// LDS slots it read, so one plane-sized buffer suffices:
//   R1/R2  row transforms: rows r and r+H/2 are packed as one complex row,
//          separated after the DFT; the real DC and Nyquist bins of each row
//          are packed into one complex "column 0".
//   C1/C2  column transforms over the W/2 packed columns; column 0 carries
//          DC + i*Nyquist and is unpacked by the edge pass.
//   the inverse mirrors these passes (I1..I4); column 0 is re-packed from
//   the Hermitian parts of the DC and Nyquist columns, which is exactly the
//   information irfft2's C2R step keeps.
// Conventions are numpy's / XLA's (rfft2 unnormalised forward, irfft2 1/(HW)).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "fft_reg.h"
#include "launch.h"

namespace cssm {

// ---------------------------------------------------------------- I/O types

struct IoF32 {
  using T = float;
  using V4 = float4;
  static __device__ __forceinline__ float to_f(const float v) { return v; }
  static __device__ __forceinline__ float from_f(const float v) { return v; }
  static __device__ __forceinline__ float4 to_f4(const float4 v) { return v; }
  static __device__ __forceinline__ float4 from_f4(const float4 v) { return v; }
};

__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) { return __uint_as_float(bits16 << 16); }
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
  uint32_t x = __float_as_uint(f);
  if ((x & 0x7f800000u) == 0x7f800000u) {          // inf / nan: keep, force quiet nan
    return (x >> 16) | ((x & 0x007fffffu) ? 0x40u : 0u);
  }
  x += 0x7fffu + ((x >> 16) & 1u);                   // round to nearest even
  return x >> 16;
}

struct IoBF16 {
  using T = uint16_t;
  using V4 = uint2;   // 4 x bf16
  static __device__ __forceinline__ float to_f(const uint16_t v) { return bf16_to_f32(v); }
  static __device__ __forceinline__ uint16_t from_f(const float v) { return uint16_t(f32_to_bf16(v)); }
  static __device__ __forceinline__ float4 to_f4(const uint2 v) {
    return make_float4(bf16_to_f32(v.x & 0xffffu), bf16_to_f32(v.x >> 16),
                       bf16_to_f32(v.y & 0xffffu), bf16_to_f32(v.y >> 16));
  }
  static __device__ __forceinline__ uint2 from_f4(const float4 f) {
    return make_uint2(f32_to_bf16(f.x) | (f32_to_bf16(f.y) << 16),
                      f32_to_bf16(f.z) | (f32_to_bf16(f.w) << 16));
  }
};

__device__ __forceinline__ float silu_f(float x) {
  return x * __builtin_amdgcn_rcpf(1.0f + __expf(-x));
}

__device__ __forceinline__ float4 act4(float4 v, int act) {
  if (act == 1) {
    v.x = silu_f(v.x); v.y = silu_f(v.y); v.z = silu_f(v.z); v.w = silu_f(v.w);
  }
  return v;
}

// ------------------------------------------------------------------ geometry

constexpr int fft_radix1(int n) { return n >= 128 ? 16 : (n >= 32 ? 8 : (n >= 8 ? 4 : 2)); }

// LH, LW: log2 of the plane; NP planes per workgroup; PPT real samples per
// thread per plane load (64 for large planes: a 128x128 plane is one 256-thread
// workgroup, two of which share a CU so one's barriers and memory waits hide
// behind the other's arithmetic).  SO: the column passes walk the packed
// columns in scan_col order (per-bin planes stored in that order).
template <int LH, int LW, int NP, int PPT, bool SO = false>
struct Geom {
  static constexpr int H = 1 << LH, W = 1 << LW;
  static constexpr int HP = H / 2, WH = W / 2, WF = WH + 1;
  static constexpr int W1 = fft_radix1(W), W2 = W / W1;
  static constexpr int H1 = fft_radix1(H), H2 = H / H1;
  static constexpr int NT = NP * H * W / PPT;
  static constexpr int NR1 = NP * HP * W2, NR2 = NP * HP * (W1 / 2);
  static constexpr int NC1 = NP * WH * H2, NC2 = NP * WH * (H1 / 2);
  static constexpr int JR1 = NR1 / NT, JR2 = NR2 / NT, JC1 = NC1 / NT, JC2 = NC2 / NT;
  static constexpr int NE = NP * HP;
  static constexpr int NV4 = NP * H * W / 4;
  static constexpr int JLD = NV4 / NT;

  // LDS (floats): the plane buffer (row stride RS), the packed DC/Nyquist
  // column of each plane and four twiddle tables laid out so one thread's
  // entries are contiguous (rows padded by one entry against bank conflicts):
  //   R1 [s][k] = w_W^{s k}, C1 [s][k] = w_H^{s k},
  //   I1 [k][s] = conj w_H^{s k}, I3 [k][s] = conj w_W^{s k}.
  static constexpr int RS = W + 4;
  static constexpr int SZ_BUF = (NP * H * RS + 3) / 4 * 4;
  static constexpr int SZ_EDGE = 2 * NP * H;
  static constexpr int TR1 = W1 + 1, TC1 = H1 + 1, TI1 = H2, TI3 = W2 + 1;   // table row lengths (padded)
  static constexpr int N_R1 = W2 * TR1, N_C1 = H2 * TC1, N_I1 = H1 * TI1, N_I3 = W1 * TI3;
  static constexpr int SZ_TW = 2 * (N_R1 + N_C1 + N_I1 + N_I3);
  static constexpr int OFF_EDGE = SZ_BUF, OFF_TW = OFF_EDGE + SZ_EDGE;
  static constexpr int LDS_FLOATS = OFF_TW + SZ_TW;

  static_assert(LDS_FLOATS * 4 <= 160 * 1024, "plane group does not fit gfx950 LDS");
  static_assert(NT % 64 == 0 && NT <= 1024, "workgroup must be whole waves, <= 1024 threads");
  static_assert(JR1 * NT == NR1 && JR2 * NT == NR2 && JC1 * NT == NC1 && JC2 * NT == NC2,
                "every FFT pass must split evenly over the workgroup");
  static_assert(JLD * NT == NV4, "plane group must split into whole 4-vectors per thread");
  static_assert(W2 % 2 == 0 && H2 % 2 == 0 && W1 % 2 == 0 && H1 % 2 == 0, "radix split");

  // Sample (pl, r, w) lives at row (pl, r), column w, except that in the
  // upper half of each row's W2-float blocks (block index >= W1/2) the two
  // halves of the block are swapped.  With RS = W + 4 the passes are free of
  // LDS bank conflicts on 64 banks except the row-pair gather (2-way):
  // R1/I4 (scalar, rows two apart within a wave), R2/I3 (whole blocks),
  // C1/C2/I1/I2 (one packed-spectrum slot per lane along a row), load/store.
  static constexpr int HALF = W2 >= 4 ? W2 / 2 : 0;
  // (rows of a plane group stay far below 2^24, so the product is a full-rate 24-bit multiply)
  static __device__ __forceinline__ int row_off(int pl, int r) { return int(__umul24(unsigned(pl * H + r), unsigned(RS))); }
  // block blk < W1/2 (lo: halves in place) or >= W1/2 (hi: halves swapped), position pos < W2
  static __device__ __forceinline__ int lo_off(int pl, int r, int blk, int pos) {
    return row_off(pl, r) + blk * W2 + pos;
  }
  static __device__ __forceinline__ int hi_off(int pl, int r, int blk, int pos) {
    return row_off(pl, r) + blk * W2 + (pos ^ HALF);
  }
  // column of the packed-row spectrum P(pl, r, v), v < W/2: complex pair 2 (v / W1)
  // of block v % W1 (the slots the row pass that produces it has just read)
  static __device__ __forceinline__ int p_col(int v) {
    const int blk = v % W1, pos = 2 * (v / W1);
    return blk * W2 + (blk >= W1 / 2 ? (pos ^ HALF) : pos);
  }
  // 4-vector c4 of row r: contiguous unless the block is split by the swap
  static constexpr bool V4_SPLIT = (HALF == 2);
  // ---- wave ownership.  Wave w owns RPW consecutive row pairs (pl, p) /
  // (pl, p + H/2) and CPW consecutive packed columns (pl, v): every pass that
  // only touches its owner's rows (load, R1, R2, I3, I4, store) or columns
  // (C1, C2, edge, I1, I2) needs no workgroup barrier between passes; only
  // the two transposes (R2 -> C1, I2 -> I3) synchronise the workgroup.
  static constexpr int NW = NT / 64;
  static constexpr int NRP = NP * HP, RPW = NRP / NW;
  static constexpr int NCOL = NP * WH, CPW = NCOL / NW;
  static_assert(NRP % NW == 0 && NCOL % NW == 0, "rows / columns must split evenly over the waves");
  static_assert((RPW * W2) % 64 == 0 && (RPW * (W1 / 2)) % 64 == 0 && (CPW * H2) % 64 == 0 &&
                    (CPW * (H1 / 2)) % 64 == 0 && (RPW * (W / 2)) % 64 == 0,
                "every wave-local pass must fill whole waves");
  static_assert(CPW >= WH ? CPW % WH == 0 : WH % CPW == 0, "packed columns must not straddle waves");
  // the packed DC / Nyquist column of plane pl belongs to the wave owning column (pl, 0)
  static constexpr int PPWE = CPW >= WH ? CPW / WH : 1;        // such planes per owning wave
  static constexpr int NEW = PPWE * HP, NI1 = PPWE * (H1 / 2);  // edge / I1 jobs of an owning wave
  static constexpr int JE = (NEW + 63) / 64, JI1 = (NI1 + 63) / 64;
  static __device__ __forceinline__ bool owns_edge(int w) { return (w * CPW) % WH == 0; }
  static __device__ __forceinline__ int edge_plane0(int w) { return (w * CPW) / WH; }

  // R1/I4 job j of lane l in wave w -> (pl, p, s): s fastest.  LDS serves 32
  // lanes of 4-byte accesses per cycle from 32 banks and a row shifts the banks
  // by 4 (RS = W + 4), so with W2 = 8 the RG/2 rows of a half-wave are taken two
  // apart (even rows in lanes 0-31, odd rows in lanes 32-63 of each block of RG
  // row pairs): RG/2 rows x W2 lanes then hit each bank once.  With W2 = 4
  // consecutive rows already do.
  static constexpr int RG = 64 / W2;
  static constexpr bool R1_STRIDE2 = (W2 == 8) && (RPW % RG == 0);
  static __device__ __forceinline__ void r1_job(int w, int j, int l, int& pl, int& p, int& s) {
    s = l % W2;
    const int g = j * RG + l / W2;
    const int rp = R1_STRIDE2 ? (2 * (g % (RG / 2)) + (g / (RG / 2)) % 2 + RG * (g / RG)) : g;
    const int RP = w * RPW + rp;
    pl = RP / HP;
    p = RP % HP;
  }
  // R2/I3 job -> (pl, p, jj): jj (block pair) fastest
  static __device__ __forceinline__ void r2_job(int w, int j, int l, int& pl, int& p, int& jj) {
    const int q = j * 64 + l;
    jj = q % (W1 / 2);
    const int RP = w * RPW + q / (W1 / 2);
    pl = RP / HP;
    p = RP % HP;
  }
  // C1/I2 job -> (pl, v, s); C2 job -> (pl, v, pair): column fastest.  The
  // wave's columns are positions n = COL % W/2 of the per-bin planes, holding
  // column v = scan_col(n) under SO (else v = n).
  static __device__ __forceinline__ void col_job(int w, int j, int l, int& pl, int& v, int& r, int& n) {
    const int q = j * 64 + l;
    const int COL = w * CPW + q % CPW;
    r = q / CPW;
    pl = COL / WH;
    n = COL % WH;
    v = SO ? scan_col(H, W, n) : n;
  }
  // ---- load / store phase.  Lane l's 4-vector i (i < JLD) of wave w is column
  // c4 = l % (W/4) of group row v4_row(w, i, m) (row = pl * H + r): consecutive
  // lanes run along a row and the two rows of an owned pair alternate, so the
  // column is fixed per lane and the row advances by RK per i within a plane.
  static constexpr int C4N = W / 4, RK = 128 / W;
  static_assert(W <= 128 && 64 % C4N == 0, "load / store mapping needs W <= 128");
  struct V4Lane {
    int c4, rp, hh;   // column, row-pair offset, upper row of the pair
  };
  static __device__ __forceinline__ V4Lane v4_lane(int l) {
    return V4Lane{l % C4N, (l / C4N) / 2, (l / C4N) % 2};
  }
  // V4_LINEAR: a wave's row pairs lie in one plane, so row(i) = row(0) + RK i
  static constexpr bool V4_LINEAR = RPW <= HP && HP % RPW == 0;
  static __device__ __forceinline__ int v4_row(int w, int i, const V4Lane& m) {
    const int RP = w * RPW + i * RK + m.rp;
    const int pl = V4_LINEAR ? (w * RPW) / HP : RP / HP;
    return RP + (pl + m.hh) * HP;   // pl * H + RP % HP + hh * HP
  }
  // 4-vector index within the group (planes of H rows of W/4 vectors)
  static __device__ __forceinline__ unsigned v4_index(int row, const V4Lane& m) {
    return unsigned(row * C4N + m.c4);
  }
  // global byte offset of 4-vector i as a per-lane part and a uniform part
  // (the uniform part is the row step when V4_LINEAR; planes of H rows of W/4
  // vectors of VB bytes)
  template <int VB>
  static __device__ __forceinline__ void v4_goff(int w, int i, const V4Lane& m, unsigned& voff, int& soff) {
    if (V4_LINEAR) {
      voff = unsigned((v4_row(w, 0, m) * C4N + m.c4) * VB);
      soff = i * RK * C4N * VB;
    } else {
      voff = unsigned((v4_row(w, i, m) * C4N + m.c4) * VB);
      soff = 0;
    }
  }
};

// Policies may define `static constexpr bool kPrefetch = true` and
// `prefetch(pl, k, n)`: called at the start of each column-pass unit, before
// its column DFT, so loads the policy's bins() will need are in flight while
// the DFT runs.
template <class Op, class = void>
struct op_prefetches : std::false_type {};
template <class Op>
struct op_prefetches<Op, std::void_t<decltype(Op::kPrefetch)>> : std::bool_constant<Op::kPrefetch> {};

// pair-unit decode: pair jj of radix N1 -> units (kA, kB) with kB = -kA mod N1
// (jj = 0 groups the two self-paired units 0 and N1/2)
template <int N1>
__device__ __forceinline__ void pair_units(int jj, int& kA, int& kB) {
  kA = jj;
  kB = (jj == 0) ? (N1 / 2) : (N1 - jj);
}

// raw buffer access: 32-bit offsets from a uniform base (cheaper addressing
// than 64-bit pointers, and out-of-range reads return 0)
struct Buf {
  __amdgpu_buffer_rsrc_t r;
  __device__ __forceinline__ Buf(const void* p, unsigned bytes)
      : r(__builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, int(bytes), 0x00020000)) {}
  __device__ __forceinline__ float4 ld4(unsigned off) const {
    return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, int(off), 0, 0));
  }
  __device__ __forceinline__ float2 ld2(unsigned off) const {
    return __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(r, int(off), 0, 0));
  }
  // per-lane byte offset voff plus a uniform soff (kept in an SGPR, so a
  // constant stride costs no VALU address arithmetic)
  __device__ __forceinline__ float4 ld4(unsigned voff, int soff) const {
    return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, int(voff), soff, 0));
  }
  __device__ __forceinline__ float2 ld2(unsigned voff, int soff) const {
    return __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(r, int(voff), soff, 0));
  }
  // Streamed I/O vectors (float4 or 4 x bf16; each touched once): byte offset
  // voff (per lane) + soff (uniform), non-temporal cache policy so the planes
  // passing through do not evict what the workgroups re-read from L2 every
  // step (per-bin gates, spectral kernel)
  static constexpr int kStream = 2;   // cache-policy operand: NT
  __device__ __forceinline__ void ld(float4& v, unsigned voff, int soff) const {
    v = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, int(voff), soff, kStream));
  }
  __device__ __forceinline__ void ld(uint2& v, unsigned voff, int soff) const {
    v = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, int(voff), soff, kStream));
  }
  __device__ __forceinline__ void st(const float4& v, unsigned voff, int soff) const {
    typedef unsigned u32x4 __attribute__((__vector_size__(16)));
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, int(voff), soff, kStream);
  }
  __device__ __forceinline__ void st(const uint2& v, unsigned voff, int soff) const {
    typedef unsigned u32x2 __attribute__((__vector_size__(8)));
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, v), r, int(voff), soff, kStream);
  }
};


// LDS exchange within one wave: the wave's LDS operations execute in order, so
// a compiler / memory fence at wavefront scope is all a wave-local pass needs
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Sum of x over the 64 lanes of the wave, the same value in every lane, with no
// LDS round trip: quad swaps (lane ^ 1, lane ^ 2) and the half-row / row
// mirrors of DPP (sums of 4, 8, 16 lanes), then the four row sums read out of
// lanes 0, 16, 32, 48.  The order of the additions is fixed.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float wave_sum(float x) {
  x += dpp_f<0xb1>(x);    // quad_perm [1, 0, 3, 2]
  x += dpp_f<0x4e>(x);    // quad_perm [2, 3, 0, 1]
  x += dpp_f<0x141>(x);   // row_half_mirror
  x += dpp_f<0x140>(x);   // row_mirror
  auto rl = [](float v, int l) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l)); };
  return (rl(x, 0) + rl(x, 16)) + (rl(x, 32) + rl(x, 48));
}

// ---------------------------------------------------------------------------
// The passes of the 2-D real FFT of NP planes held in LDS, in the order a
// round trip runs them:
//   load -> R1 -> R2 -> C1 -> C2 (+ per-bin op, + I1) -> edge (+ op)
//        -> I1 packed column -> I2 -> I3 -> I4 -> store
// R2 and I2 end with a workgroup barrier (the transposes); every other pass is
// wave-local (wave_sync).  Passes take the thread's wave w and lane l.  The forward row pass skips the 1/2
// of the packed-row separation, so every bin a policy sees in the forward
// direction is 2U (the edge unpack keeps its 1/2 and inherits the factor from
// the doubled DC/Nyquist column).  The inverse passes take Y / (H W) for
// every bin and produce irfft2(Y) (numpy/XLA C2R rule: only the Hermitian part
// of the v = 0 and v = W/2 columns survives).
//
// Policies (Op):
//   op.bins(j, a2, pl, k, n, sp)  C2: sp[q] is bin (u = k + H1 q, v) of plane
//        pl, 0 < v < W/2, where n is the column's position in the per-bin
//        planes (v = scan_col(n) under SO, else n); on entry the forward value
//        (when FWD), on exit the inverse input (when INV).  (j, a2) name the
//        thread's unit slot, fixed for the whole launch, so per-bin state can
//        live in registers.  Op::kPackedColumnToo: also call it for the packed
//        DC / Nyquist column (v = 0; the values are discarded), which saves the
//        divergent branch where the op's side effects allow it.
//   op.edge(j, pl, uA, uB, e, v4) the DC / Nyquist bins of rows uA and uB
//        (uB = -uA mod H; e = uA): v4 = {(uA, 0), (uA, W/2), (uB, 0), (uB, W/2)};
//        forward value on entry (FWD), inverse input on exit (INV).
// ---------------------------------------------------------------------------
template <class G>
struct PlaneFft {
  static constexpr int H = G::H, HP = G::HP, WH = G::WH, W = G::W;
  static constexpr int W1 = G::W1, W2 = G::W2, H1 = G::H1, H2 = G::H2, NT = G::NT;

  float* buf;
  float2* edge;
  float2* twR1;
  float2* twC1;
  float2* twI1;
  float2* twI3;

  __device__ __forceinline__ explicit PlaneFft(float* smem)
      : buf(smem),
        edge(reinterpret_cast<float2*>(smem + G::OFF_EDGE)),
        twR1(reinterpret_cast<float2*>(smem + G::OFF_TW)),
        twC1(twR1 + G::N_R1),
        twI1(twC1 + G::N_C1),
        twI3(twI1 + G::N_I1) {}

  // a view of planes laid out by another geometry of the same plane size (same
  // row stride and twiddle tables): the caller supplies the plane buffer, the
  // packed-column scratch and the twiddle tables
  __device__ __forceinline__ PlaneFft(float* b, float2* e, float2* tw)
      : buf(b), edge(e), twR1(tw), twC1(twR1 + G::N_R1), twI1(twC1 + G::N_C1), twI3(twI1 + G::N_I1) {}

  __device__ __forceinline__ float2& cplx(int off) const { return *reinterpret_cast<float2*>(buf + off); }

  // twiddles w_N^m = exp(-2 pi i m / N) from double precision; call once
  // before the first pass (followed by a barrier)
  __device__ __forceinline__ void init_twiddles(int tid) const {
    auto tw = [](int m, int n) -> float2 {
      double sn, cs;
      sincospi(2.0 * double(m) / double(n), &sn, &cs);
      return make_float2(float(cs), float(-sn));
    };
    for (int i = tid; i < G::N_R1; i += NT) twR1[i] = tw((i / G::TR1) * (i % G::TR1), W);
    for (int i = tid; i < G::N_C1; i += NT) twC1[i] = tw((i / G::TC1) * (i % G::TC1), H);
    for (int i = tid; i < G::N_I1; i += NT) twI1[i] = cconj(tw((i % G::TI1) * (i / G::TI1), H));
    for (int i = tid; i < G::N_I3; i += NT) twI3[i] = cconj(tw((i % G::TI3) * (i / G::TI3), W));
  }

  // LDS offsets of 4-vector column c4 within a row: the two float2 halves sit
  // at a and b (b = a + 2 unless the half-swap of an upper block splits them)
  struct V4Col {
    int a, b;
  };
  static __device__ __forceinline__ V4Col v4_col(int c4) {
    const int w = 4 * c4, blk = w / W2, pos = w % W2;
    if (G::V4_SPLIT && blk >= W1 / 2) return V4Col{blk * W2 + (pos ^ 2), blk * W2 + pos};
    const int o = blk * W2 + (blk >= W1 / 2 ? (pos ^ G::HALF) : pos);
    return V4Col{o, o + 2};
  }
  __device__ __forceinline__ void v4_put(int row, const V4Col& c, float4 v) const {
    float* r = buf + G::row_off(0, row);
    if (G::V4_SPLIT) {
      *reinterpret_cast<float2*>(r + c.a) = make_float2(v.x, v.y);
      *reinterpret_cast<float2*>(r + c.b) = make_float2(v.z, v.w);
    } else {
      *reinterpret_cast<float4*>(r + c.a) = v;
    }
  }
  __device__ __forceinline__ float4 v4_get(int row, const V4Col& c) const {
    const float* r = buf + G::row_off(0, row);
    if (G::V4_SPLIT) {
      const float2 lo = *reinterpret_cast<const float2*>(r + c.a), hi = *reinterpret_cast<const float2*>(r + c.b);
      return make_float4(lo.x, lo.y, hi.x, hi.y);
    }
    return *reinterpret_cast<const float4*>(r + c.a);
  }

  // ---------------------------------------------- R1: DFT-W1 over m, twiddle
  __device__ __forceinline__ void r1(int w, int l) const {
#pragma unroll
    for (int j = 0; j < G::JR1; ++j) {
      int pl, p, s;
      G::r1_job(w, j, l, pl, p, s);
      float2 zz[W1];
#pragma unroll
      for (int m = 0; m < W1; ++m) {
        const int o = (m >= W1 / 2) ? (s ^ G::HALF) : s;
        zz[m] = make_float2(buf[G::row_off(pl, p) + m * W2 + o], buf[G::row_off(pl, p + HP) + m * W2 + o]);
      }
      Dft<W1, false>::run(zz);
#pragma unroll
      for (int k = 0; k < W1; ++k) {
        const float2 v = k ? cmul(zz[k], twR1[s * G::TR1 + k]) : zz[0];
        const int o = (k >= W1 / 2) ? (s ^ G::HALF) : s;
        buf[G::row_off(pl, p) + k * W2 + o] = v.x;
        buf[G::row_off(pl, p + HP) + k * W2 + o] = v.y;
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    wave_sync();
  }

  // ----------------- R2: DFT-W2 over s, separate packed row pairs (x2 scale)
  __device__ __forceinline__ void r2(int w, int l) const {
#pragma unroll
    for (int j = 0; j < G::JR2; ++j) {
      int pl, p, jj;
      G::r2_job(w, j, l, pl, p, jj);
      int kA, kB;
      pair_units<W1>(jj, kA, kB);
      float2 za[W2], zb[W2];
#pragma unroll
      for (int s = 0; s < W2; ++s) {
        za[s] = make_float2(buf[G::lo_off(pl, p, kA, s)], buf[G::lo_off(pl, p + HP, kA, s)]);
        zb[s] = make_float2(buf[G::hi_off(pl, p, kB, s)], buf[G::hi_off(pl, p + HP, kB, s)]);
      }
      Dft<W2, false>::run(za);
      Dft<W2, false>::run(zb);
      // Z[kA + W1 q] = za[q], Z[kB + W1 q] = zb[q]
      // 2 X_p[v] = Z[v] + conj Z[-v] ; 2 X_{p+HP}[v] = -i (Z[v] - conj Z[-v])
      // v = kA + W1 q sits in (lo) block kA, v = kB + W1 q in (hi) block kB
      auto emit = [&](bool hi, int blk, int q, float2 zv, float2 zm) {
        const int o0 = hi ? G::hi_off(pl, p, blk, 2 * q) : G::lo_off(pl, p, blk, 2 * q);
        const int o1 = hi ? G::hi_off(pl, p + HP, blk, 2 * q) : G::lo_off(pl, p + HP, blk, 2 * q);
        cplx(o0) = make_float2(zv.x + zm.x, zv.y - zm.y);
        cplx(o1) = make_float2(zv.y + zm.y, zm.x - zv.x);
      };
      if (jj != 0) {
#pragma unroll
        for (int q = 0; q < W2 / 2; ++q) {
          emit(false, kA, q, za[q], zb[W2 - 1 - q]);
          emit(true, kB, q, zb[q], za[W2 - 1 - q]);
        }
      } else {
        // packed column 0: 2 (DC + i Nyquist) of both rows
        const float2 z0 = za[0], zn = za[W2 / 2];
        cplx(G::lo_off(pl, p, 0, 0)) = make_float2(z0.x + z0.x, zn.x + zn.x);
        cplx(G::lo_off(pl, p + HP, 0, 0)) = make_float2(z0.y + z0.y, zn.y + zn.y);
#pragma unroll
        for (int q = 1; q < W2 / 2; ++q) emit(false, 0, q, za[q], za[W2 - q]);
#pragma unroll
        for (int q = 0; q < W2 / 2; ++q) emit(true, W1 / 2, q, zb[q], zb[W2 - 1 - q]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    __syncthreads();
  }

  // ------------------------------------------ C1: DFT-H1 over m, twiddle
  __device__ __forceinline__ void c1(int w, int l) const {
#pragma unroll
    for (int j = 0; j < G::JC1; ++j) {
      int pl, v, s, n;
      G::col_job(w, j, l, pl, v, s, n);
      const int col = G::p_col(v);
      float2 zz[H1];
#pragma unroll
      for (int m = 0; m < H1; ++m) zz[m] = cplx(G::row_off(pl, s + H2 * m) + col);
      Dft<H1, false>::run(zz);
#pragma unroll
      for (int k = 0; k < H1; ++k)
        cplx(G::row_off(pl, s + H2 * k) + col) = k ? cmul(zz[k], twC1[s * G::TC1 + k]) : zz[0];
      __builtin_amdgcn_sched_barrier(0);
    }
    wave_sync();
  }

  // ------ C2: DFT-H2 over s -> spectrum; op.bins; inverse DFT-H2 (I1)
  // One unit (kA, then kB) at a time keeps the live registers to one unit's
  // spectrum on top of whatever state the policy holds.  The packed DC /
  // Nyquist column (v = 0) goes to the edge buffer (FWD) and is left to the
  // edge pass and i1_packed.
  template <bool FWD, bool INV, class Op>
  __device__ __forceinline__ void c2(int w, int l, Op& op) const {
#pragma unroll
    for (int j = 0; j < G::JC2; ++j) {
      int pl, v, pair, n;
      G::col_job(w, j, l, pl, v, pair, n);
      int kA, kB;
      pair_units<H1>(pair, kA, kB);
      const int col = G::p_col(v);
#pragma unroll
      for (int a2 = 0; a2 < 2; ++a2) {
        const int k = a2 ? kB : kA;
        float2 sp[H2];
        if constexpr (op_prefetches<Op>::value) op.prefetch(pl, k, n);
        if (FWD) {
#pragma unroll
          for (int s = 0; s < H2; ++s) sp[s] = cplx(G::row_off(pl, s + H2 * k) + col);
          Dft<H2, false>::run(sp);
        }
        if constexpr (Op::kPackedColumnToo) {
          // the packed column's lanes run the per-bin work as well (no divergent
          // branch); what they write back is replaced by i1_packed
          if (FWD && v == 0) {
#pragma unroll
            for (int q = 0; q < H2; ++q) edge[pl * H + k + H1 * q] = sp[q];
          }
          op.bins(j, a2, pl, k, n, sp);
          if (INV) {
            Dft<H2, true>::run(sp);
#pragma unroll
            for (int s = 0; s < H2; ++s)
              cplx(G::row_off(pl, s + H2 * k) + col) = s ? cmul(sp[s], twI1[k * G::TI1 + s]) : sp[0];
          }
        } else if (v == 0) {
          if (FWD) {
#pragma unroll
            for (int q = 0; q < H2; ++q) edge[pl * H + k + H1 * q] = sp[q];
          }
        } else {
          op.bins(j, a2, pl, k, n, sp);
          if (INV) {
            Dft<H2, true>::run(sp);
#pragma unroll
            for (int s = 0; s < H2; ++s)
              cplx(G::row_off(pl, s + H2 * k) + col) = s ? cmul(sp[s], twI1[k * G::TI1 + s]) : sp[0];
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    wave_sync();
  }

  // ------------------- edge pass: DC and Nyquist columns (unpack, op, repack)
  template <bool FWD, bool INV, class Op>
  __device__ __forceinline__ void edges(int w, int l, Op& op) const {
    if (!G::owns_edge(w)) return;
#pragma unroll
    for (int j = 0; j < G::JE; ++j) {
      const int q = j * 64 + l;
      if (q < G::NEW) {
        const int e = q % HP, pl = G::edge_plane0(w) + q / HP;
        const int uA = e, uB = (e == 0) ? HP : H - e;
        float2 v4[4];
        if (FWD) {
          // partners -u mod H: uB for uA when e > 0; both self-partnered when e == 0
          const float2 cA = edge[pl * H + uA], cB = edge[pl * H + uB];
          const float2 cAm = (e == 0) ? cA : cB, cBm = (e == 0) ? cB : cA;
          // U(u,0) = (C[u] + conj C[-u]) / 2 ; U(u,W/2) = -i (C[u] - conj C[-u]) / 2
          v4[0] = make_float2(0.5f * (cA.x + cAm.x), 0.5f * (cA.y - cAm.y));
          v4[1] = make_float2(0.5f * (cA.y + cAm.y), 0.5f * (cAm.x - cA.x));
          v4[2] = make_float2(0.5f * (cB.x + cBm.x), 0.5f * (cB.y - cBm.y));
          v4[3] = make_float2(0.5f * (cB.y + cBm.y), 0.5f * (cBm.x - cB.x));
        }
        op.edge(j, pl, uA, uB, e, v4);
        if (INV) {
          const float2 y0A = v4[0], yNA = v4[1], y0B = v4[2], yNB = v4[3];
          // repack: c[u] = Herm(Y0)[u] + i Herm(YN)[u], Herm(X)[u] = (X[u] + conj X[-u]) / 2
          float2 cOutA, cOutB;
          if (e != 0) {
            const float2 h0A = make_float2(0.5f * (y0A.x + y0B.x), 0.5f * (y0A.y - y0B.y));
            const float2 hNA = make_float2(0.5f * (yNA.x + yNB.x), 0.5f * (yNA.y - yNB.y));
            const float2 h0B = make_float2(0.5f * (y0B.x + y0A.x), 0.5f * (y0B.y - y0A.y));
            const float2 hNB = make_float2(0.5f * (yNB.x + yNA.x), 0.5f * (yNB.y - yNA.y));
            cOutA = make_float2(h0A.x - hNA.y, h0A.y + hNA.x);
            cOutB = make_float2(h0B.x - hNB.y, h0B.y + hNB.x);
          } else {
            cOutA = make_float2(y0A.x, yNA.x);
            cOutB = make_float2(y0B.x, yNB.x);
          }
          edge[pl * H + uA] = cOutA;
          edge[pl * H + uB] = cOutB;
        }
      }
    }
    wave_sync();
  }

  // ---------------- I1 for the packed column: inverse DFT-H2, conj twiddle
  __device__ __forceinline__ void i1_packed(int w, int l) const {
    if (!G::owns_edge(w)) return;
    if constexpr (H2 == 8) {
      i1_packed_quads(w, l);
      return;
    }
#pragma unroll
    for (int j = 0; j < G::JI1; ++j) {
      const int q = j * 64 + l;
      if (q < G::NI1) {
        const int pl = G::edge_plane0(w) + q / (H1 / 2);
        int kA, kB;
        pair_units<H1>(q % (H1 / 2), kA, kB);
        float2 sa[H2], sb[H2];
#pragma unroll
        for (int q = 0; q < H2; ++q) {
          sa[q] = edge[pl * H + kA + H1 * q];
          sb[q] = edge[pl * H + kB + H1 * q];
        }
        Dft<H2, true>::run(sa);
        Dft<H2, true>::run(sb);
        const int col = G::p_col(0);
#pragma unroll
        for (int s = 0; s < H2; ++s) {
          cplx(G::row_off(pl, s + H2 * kA) + col) = s ? cmul(sa[s], twI1[kA * G::TI1 + s]) : sa[0];
          cplx(G::row_off(pl, s + H2 * kB) + col) = s ? cmul(sb[s], twI1[kB * G::TI1 + s]) : sb[0];
        }
      }
    }
    wave_sync();
  }

  // I1 of the packed column for H2 = 8 on four lanes per unit k, so a wave
  // runs 16 units at once instead of one pair of units per lane.  Lane c of a
  // quad takes q = c and c + 4 of X[k + H1 q]: a radix-2 step gives
  // a_c = x_c + x_{c+4} (even outputs) and b_c = (x_c - x_{c+4}) e^{2 pi i c / 8}
  // (odd outputs); the two inverse 4-point DFTs over c run across the quad
  // (pairs c ^ 2, then c ^ 1, exchanged by DPP), after which lane c holds
  // outputs s = 2 m and 2 m + 1 with m the 2-bit reversal of c.
  __device__ __forceinline__ void i1_packed_quads(int w, int l) const {
    static_assert(H2 == 8, "quad I1 needs H2 = 8");
    constexpr int NJ = G::PPWE * H1 * 4, J = (NJ + 63) / 64;
    constexpr float R = 0.70710678118654752f;
    // x + sgn * (the value of lane l ^ d in the quad), d = 2 (ctrl 0x4e) or 1 (0xb1)
    auto xch = [](float2 v, auto ctrl) -> float2 {
      constexpr int C = decltype(ctrl)::value;
      return make_float2(__int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v.x), C, 0xf, 0xf, false)),
                         __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v.y), C, 0xf, 0xf, false)));
    };
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int q = j * 64 + l;
      if (NJ % 64 == 0 || q < NJ) {
        const int c = q & 3, k = (q >> 2) % H1, pl = G::edge_plane0(w) + (q >> 2) / H1;
        const float2 x0 = edge[pl * H + k + H1 * c], x1 = edge[pl * H + k + H1 * (c + 4)];
        float2 a = cadd(x0, x1), b = csub(x0, x1);
        {  // b *= e^{2 pi i c / 8}
          const float cs = c == 0 ? 1.0f : (c == 1 ? R : (c == 2 ? 0.0f : -R));
          const float sn = c == 0 ? 0.0f : (c == 2 ? 1.0f : R);
          b = make_float2(b.x * cs - b.y * sn, b.x * sn + b.y * cs);
        }
        // stage over c ^ 2: c < 2 keeps v_c + v_{c+2}; c >= 2 takes (v_{c-2} - v_c) e^{2 pi i (c-2) / 4}
        const float sA = c < 2 ? 1.0f : -1.0f;
        float2 pa = xch(a, std::integral_constant<int, 0x4e>()), pb = xch(b, std::integral_constant<int, 0x4e>());
        a = make_float2(fmaf(sA, a.x, pa.x), fmaf(sA, a.y, pa.y));
        b = make_float2(fmaf(sA, b.x, pb.x), fmaf(sA, b.y, pb.y));
        if (c == 3) {   // x i
          a = make_float2(-a.y, a.x);
          b = make_float2(-b.y, b.x);
        }
        // stage over c ^ 1: even c keeps v_c + v_{c+1}, odd c takes v_{c-1} - v_c
        const float sB = (c & 1) ? -1.0f : 1.0f;
        pa = xch(a, std::integral_constant<int, 0xb1>());
        pb = xch(b, std::integral_constant<int, 0xb1>());
        a = make_float2(fmaf(sB, a.x, pa.x), fmaf(sB, a.y, pa.y));
        b = make_float2(fmaf(sB, b.x, pb.x), fmaf(sB, b.y, pb.y));
        const int s0 = 2 * (((c & 1) << 1) | (c >> 1));
        const int col = G::p_col(0);
        cplx(G::row_off(pl, s0 + H2 * k) + col) = s0 ? cmul(a, twI1[k * G::TI1 + s0]) : a;
        cplx(G::row_off(pl, s0 + 1 + H2 * k) + col) = cmul(b, twI1[k * G::TI1 + s0 + 1]);
      }
    }
    wave_sync();
  }

  // ----------------------------- I2: inverse DFT-H1 over k -> rows (P slots)
  __device__ __forceinline__ void i2(int w, int l) const {
#pragma unroll
    for (int j = 0; j < G::JC1; ++j) {
      int pl, v, s, n;
      G::col_job(w, j, l, pl, v, s, n);
      const int col = G::p_col(v);
      float2 zz[H1];
#pragma unroll
      for (int k = 0; k < H1; ++k) zz[k] = cplx(G::row_off(pl, s + H2 * k) + col);
      Dft<H1, true>::run(zz);
#pragma unroll
      for (int m = 0; m < H1; ++m) cplx(G::row_off(pl, s + H2 * m) + col) = zz[m];
      __builtin_amdgcn_sched_barrier(0);
    }
    __syncthreads();
  }

  // ------------- I3: build packed Hermitian row pair, inverse DFT-W2, twiddle
  __device__ __forceinline__ void i3(int w, int l) const {
#pragma unroll
    for (int j = 0; j < G::JR2; ++j) {
      int pl, p, jj;
      G::r2_job(w, j, l, pl, p, jj);
      int kA, kB;
      pair_units<W1>(jj, kA, kB);
      float2 za[W2], zb[W2];
      // Q[v] = Zp[v] + i Zq[v]; Q[W-v] = conj Zp[v] + i conj Zq[v]  (0 < v < W/2)
      auto fetch = [&](bool hi, int blk, int q, float2& qv, float2& qm) {
        const int o0 = hi ? G::hi_off(pl, p, blk, 2 * q) : G::lo_off(pl, p, blk, 2 * q);
        const int o1 = hi ? G::hi_off(pl, p + HP, blk, 2 * q) : G::lo_off(pl, p + HP, blk, 2 * q);
        const float2 x = cplx(o0), c = cplx(o1);
        qv = make_float2(x.x - c.y, x.y + c.x);
        qm = make_float2(x.x + c.y, c.x - x.y);
      };
      if (jj != 0) {
#pragma unroll
        for (int q = 0; q < W2 / 2; ++q) {
          fetch(false, kA, q, za[q], zb[W2 - 1 - q]);
          fetch(true, kB, q, zb[q], za[W2 - 1 - q]);
        }
      } else {
        const float2 cp = cplx(G::lo_off(pl, p, 0, 0)), cq = cplx(G::lo_off(pl, p + HP, 0, 0));
        za[0] = make_float2(cp.x, cq.x);          // Q[0]   = Re c_p + i Re c_q
        za[W2 / 2] = make_float2(cp.y, cq.y);     // Q[W/2] = Im c_p + i Im c_q
#pragma unroll
        for (int q = 1; q < W2 / 2; ++q) fetch(false, 0, q, za[q], za[W2 - q]);
#pragma unroll
        for (int q = 0; q < W2 / 2; ++q) fetch(true, W1 / 2, q, zb[q], zb[W2 - 1 - q]);
      }
      Dft<W2, true>::run(za);
      Dft<W2, true>::run(zb);
#pragma unroll
      for (int s = 0; s < W2; ++s) {
        const float2 oa = s ? cmul(za[s], twI3[kA * G::TI3 + s]) : za[0];
        const float2 ob = s ? cmul(zb[s], twI3[kB * G::TI3 + s]) : zb[0];
        buf[G::lo_off(pl, p, kA, s)] = oa.x;
        buf[G::lo_off(pl, p + HP, kA, s)] = oa.y;
        buf[G::hi_off(pl, p, kB, s)] = ob.x;
        buf[G::hi_off(pl, p + HP, kB, s)] = ob.y;
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    wave_sync();
  }

  // ------------------------ I4: inverse DFT-W1 over k -> real rows p, p+H/2
  __device__ __forceinline__ void i4(int w, int l) const {
#pragma unroll
    for (int j = 0; j < G::JR1; ++j) {
      int pl, p, s;
      G::r1_job(w, j, l, pl, p, s);
      float2 zz[W1];
#pragma unroll
      for (int k = 0; k < W1; ++k) {
        const int o = (k >= W1 / 2) ? (s ^ G::HALF) : s;
        zz[k] = make_float2(buf[G::row_off(pl, p) + k * W2 + o], buf[G::row_off(pl, p + HP) + k * W2 + o]);
      }
      Dft<W1, true>::run(zz);
#pragma unroll
      for (int m = 0; m < W1; ++m) {
        const int o = (m >= W1 / 2) ? (s ^ G::HALF) : s;
        buf[G::row_off(pl, p) + m * W2 + o] = zz[m].x;
        buf[G::row_off(pl, p + HP) + m * W2 + o] = zz[m].y;
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    wave_sync();
  }
};

}  // namespace cssm
