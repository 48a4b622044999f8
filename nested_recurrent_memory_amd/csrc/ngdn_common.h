// Device-side building blocks shared by the nested GDN kernels (gfx950 only).
//
// Matrix work runs on the CDNA4 matrix cores through two 16x16 MFMA shapes:
//   bf16 operands: v_mfma_f32_16x16x32_bf16  (8 k-values per lane)
//   fp32 operands: v_mfma_f32_16x16x4_f32    (1 k-value per lane)
// both accumulating in fp32. For a wave (64 lanes) and lane l:
//   A fragment: row (l & 15), k-values starting at kofs(l) = KPL * (l >> 4)
//   B fragment: col (l & 15), the same k-values
//   D (4 floats): rows 4 * (l >> 4) + r, r = 0..3, col (l & 15)
// Operands are addressed "k-contiguous": A as A[i][k], B as Bt[j][k].
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <type_traits>

namespace ngdn {

typedef __bf16 bf16;
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f4;

constexpr int WAVE = 64;
constexpr int CH = 64;  // tokens per chunk

__device__ __forceinline__ int lane_id() { return threadIdx.x & (WAVE - 1); }
// uniform across the wave: the compiler keeps it (and what derives from it) in
// scalar registers
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE); }

template <typename T> __device__ __forceinline__ float to_f(T x) { return (float)x; }
template <typename T> __device__ __forceinline__ T from_f(float x) { return (T)x; }

// logistic function from the hardware exp and reciprocal (about 2 ulp; the
// exact-division form costs several times the instructions in the
// elementwise kernels, where it dominates)
__device__ __forceinline__ float sigmoid_fast(float a) {
  return __builtin_amdgcn_rcpf(1.f + __expf(-a));
}
__device__ __forceinline__ f4 f4_zero() { f4 z = {0.f, 0.f, 0.f, 0.f}; return z; }

// ---------------------------------------------------------------- MFMA
//
// Operands come in two kinds. Exact operands are the op's bf16 inputs and
// parameters. Derived operands (everything computed: W, U, T, states, Vn,
// gradients) are stored in fp32. For bf16 inputs a derived value x enters the
// bf16 matrix core as a pair x = hi + lo (each bf16, together about 16
// mantissa bits) and a product takes 2 MFMAs (exact x derived: a*hi + a*lo) or
// 3 (derived x derived: hi*hi + hi*lo + lo*hi; lo*lo is below fp32 rounding of
// the sum). This keeps bf16 results within fp32-level agreement of an exact
// evaluation at bf16 matrix-core rates. For fp32 inputs both kinds are plain
// fp32 and every product is one fp32 MFMA.
//
// The fragment type follows the pointer: ld(const bf16*) gives an exact
// fragment, ld(const float*) a derived one.

template <typename E> struct Mma;

template <> struct Mma<bf16> {
  static constexpr int KS = 32;   // k per instruction
  static constexpr int KPL = 8;   // k-values per lane
  typedef bf16x8 Frag;            // exact
  struct SFrag { bf16x8 hi, lo; };  // derived, split
  __device__ __forceinline__ static f4 mma(f4 acc, Frag a, Frag b) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
  }
  __device__ __forceinline__ static f4 mma(f4 acc, Frag a, SFrag b) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b.lo, acc, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b.hi, acc, 0, 0, 0);
  }
  __device__ __forceinline__ static f4 mma(f4 acc, SFrag a, Frag b) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.lo, b, acc, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.hi, b, acc, 0, 0, 0);
  }
  __device__ __forceinline__ static f4 mma(f4 acc, SFrag a, SFrag b) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.lo, b.hi, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.hi, b.lo, acc, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.hi, b.hi, acc, 0, 0, 0);
  }
  __device__ __forceinline__ static Frag ld(const bf16* p) {
    return *reinterpret_cast<const bf16x8*>(p);
  }
  __device__ __forceinline__ static SFrag ld(const float* p) {
    const f4 x0 = *reinterpret_cast<const f4*>(p);
    const f4 x1 = *reinterpret_cast<const f4*>(p + 4);
    SFrag r;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      r.hi[e] = hi_of(x0[e]);
      r.lo[e] = lo_of(x0[e], r.hi[e]);
      r.hi[e + 4] = hi_of(x1[e]);
      r.lo[e + 4] = lo_of(x1[e], r.hi[e + 4]);
    }
    return r;
  }
  __device__ __forceinline__ static bf16 elem(const Frag& f, int e) { return f[e]; }
  // exact values (inputs, or products known to be exact in bf16)
  template <typename F>
  __device__ __forceinline__ static Frag make(F f) {  // f(e) -> float, e < KPL
    Frag r;
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = (bf16)f(e);
    return r;
  }
  // derived values
  template <typename F>
  __device__ __forceinline__ static SFrag makes(F f) {
    SFrag r;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float x = f(e);
      r.hi[e] = hi_of(x);
      r.lo[e] = lo_of(x, r.hi[e]);
    }
    return r;
  }
  __device__ __forceinline__ static Frag zero() {
    Frag r;
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = (bf16)0.f;
    return r;
  }
  __device__ __forceinline__ static SFrag szero() { return SFrag{zero(), zero()}; }
  // x = hi + lo: hi is x rounded to bf16, lo the rounded remainder
  __device__ __forceinline__ static bf16 hi_of(float x) { return (bf16)x; }
  __device__ __forceinline__ static bf16 lo_of(float x, bf16 hi) { return (bf16)(x - (float)hi); }
};

template <> struct Mma<float> {
  static constexpr int KS = 4;
  static constexpr int KPL = 1;
  typedef float Frag;
  typedef float SFrag;
  __device__ __forceinline__ static f4 mma(f4 acc, float a, float b) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc, 0, 0, 0);
  }
  __device__ __forceinline__ static float ld(const float* p) { return *p; }
  __device__ __forceinline__ static float elem(float f, int) { return f; }
  template <typename F>
  __device__ __forceinline__ static float make(F f) { return f(0); }
  template <typename F>
  __device__ __forceinline__ static float makes(F f) { return f(0); }
  __device__ __forceinline__ static float zero() { return 0.f; }
  __device__ __forceinline__ static float szero() { return 0.f; }
};

// An LDS tile of derived (fp32) values kept in the form the matrix core
// reads. For bf16 MFMAs: two bf16 planes, hi then lo (plane elements apart),
// so each value is split once by the wave that writes it rather than by every
// wave that reads it; for fp32 MFMAs: one fp32 plane. Rows are padded by PAD
// elements (16 bytes) so fragment reads stay 16-byte aligned.
template <typename E> struct SplitTile;
template <> struct SplitTile<bf16> {
  typedef bf16 T;
  static constexpr int NPLANE = 2, PAD = 8;
  T* p; int plane;
  // four consecutive values at element offset off (off % 4 == 0)
  __device__ __forceinline__ void put4(int off, f4 x) const {
    bf16x4 h, l;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      h[e] = Mma<bf16>::hi_of(x[e]);
      l[e] = Mma<bf16>::lo_of(x[e], h[e]);
    }
    *reinterpret_cast<bf16x4*>(p + off) = h;
    *reinterpret_cast<bf16x4*>(p + plane + off) = l;
  }
  __device__ __forceinline__ void put1(int off, float x) const {
    const bf16 h = Mma<bf16>::hi_of(x);
    p[off] = h;
    p[plane + off] = Mma<bf16>::lo_of(x, h);
  }
  // the KPL values of one fragment from element offset off (off % 8 == 0)
  __device__ __forceinline__ Mma<bf16>::SFrag get(int off) const {
    return Mma<bf16>::SFrag{*reinterpret_cast<const bf16x8*>(p + off),
                            *reinterpret_cast<const bf16x8*>(p + plane + off)};
  }
};
template <> struct SplitTile<float> {
  typedef float T;
  static constexpr int NPLANE = 1, PAD = 4;
  T* p; int plane;
  __device__ __forceinline__ void put4(int off, f4 x) const {
    *reinterpret_cast<f4*>(p + off) = x;
  }
  __device__ __forceinline__ void put1(int off, float x) const { p[off] = x; }
  __device__ __forceinline__ float get(int off) const { return p[off]; }
};

// Derived operands that only ever enter the matrix core are also kept in HBM
// in split form: for bf16, each per-unit tile [R][C] (a chunk's or a firing's)
// is two bf16 planes, hi then lo R*C elements apart, in the bytes of the fp32
// tile; for fp32, the fp32 values. split_at gives the SplitTile view of one
// unit (writes with put1 / put4, fragment reads with get), so the consumers
// load fragments without splitting them again at every use.
template <typename E>
__device__ __forceinline__ SplitTile<E> split_at(const float* unit, int plane) {
  return SplitTile<E>{reinterpret_cast<typename SplitTile<E>::T*>(const_cast<float*>(unit)), plane};
}

// Fragment order of a split bf16 tile [R][C] (R % 16 == 0, C % 32 == 0), for
// tensors read only as MFMA A operands by row tile: each 16 x 32 block (row
// block rb, column block cb) is 512 consecutive elements of a plane, at block
// rb * C/32 + cb, and inside it lane l of a 16x16x32 operand fragment holds
// row l % 16, columns 8 (l / 16) .. + 7 at element 8 l. The fragment of row
// tile rt, k-step s is then one contiguous 1 KB read per plane (row-major, it
// is 16 rows of 64 bytes).
__device__ __forceinline__ int frag_ofs(int row, int col, int C) {
  return ((row >> 4) * (C >> 5) + (col >> 5)) * 512 +
         ((((col & 31) >> 3) << 4) + (row & 15)) * 8 + (col & 7);
}
// the element (row, col) at fragment-order position p of a [.][C] tile
__device__ __forceinline__ void frag_pos(int p, int C, int& row, int& col) {
  const int blk = p >> 9, w = p & 511, l = w >> 3;
  row = (blk / (C >> 5)) * 16 + (l & 15);
  col = (blk % (C >> 5)) * 32 + (l >> 4) * 8 + (w & 7);
}
// offset of the fragment of row tile rt, k-step s in a fragment-order tile
// with rows of C elements
__device__ __forceinline__ int frag_at(int rt, int s, int C) {
  return (rt * (C >> 5) + s) * 512 + lane_id() * 8;
}

template <typename E> __device__ __forceinline__ int kofs(int lane) {
  return Mma<E>::KPL * (lane >> 4);
}

// D[16x16] += A[16 x kd] * B[kd x 16], A row-major (k contiguous, stride lda),
// B given as Bt[16][kd] (k contiguous, stride ldb). kd a multiple of KS. Each
// of A and Bt is exact (E) or derived (float) storage.
template <typename E, typename TA, typename TB>
__device__ __forceinline__ f4 mma_tile(f4 acc, const TA* A, int lda, const TB* Bt,
                                       int ldb, int kd) {
  const int l = lane_id();
  const TA* pa = A + (l & 15) * lda + kofs<E>(l);
  const TB* pb = Bt + (l & 15) * ldb + kofs<E>(l);
  for (int k = 0; k < kd; k += Mma<E>::KS)
    acc = Mma<E>::mma(acc, Mma<E>::ld(pa + k), Mma<E>::ld(pb + k));
  return acc;
}

// Mma<E>::KPL consecutive elements at p as floats (one 16-byte load for bf16).
template <typename E>
__device__ __forceinline__ void ld_vals(const E* p, float* out) {
  if constexpr (std::is_same<E, float>::value) {
    out[0] = *p;
  } else {
    const bf16x8 v = *reinterpret_cast<const bf16x8*>(p);
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = (float)v[e];
  }
}

// N consecutive fp32 values at p (16-byte loads when N is a multiple of 4).
template <int N>
__device__ __forceinline__ void ld_raw(const float* p, float* out) {
  if constexpr (N % 4 == 0) {
#pragma unroll
    for (int e = 0; e < N; e += 4) {
      const f4 x = *reinterpret_cast<const f4*>(p + e);
      out[e] = x[0]; out[e + 1] = x[1]; out[e + 2] = x[2]; out[e + 3] = x[3];
    }
  } else {
#pragma unroll
    for (int e = 0; e < N; ++e) out[e] = p[e];
  }
}

// 8 consecutive elements as floats (two 16-byte loads for fp32)
template <typename E>
__device__ __forceinline__ void load8f(const E* p, float* out) {
  if constexpr (std::is_same<E, float>::value) {
    const f4 a = *reinterpret_cast<const f4*>(p), b = *reinterpret_cast<const f4*>(p + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) { out[e] = a[e]; out[4 + e] = b[e]; }
  } else {
    const bf16x8 v = *reinterpret_cast<const bf16x8*>(p);
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = (float)v[e];
  }
}
template <typename E>
__device__ __forceinline__ void store8f(E* p, const float* x) {
  if constexpr (std::is_same<E, float>::value) {
    f4 a, b;
#pragma unroll
    for (int e = 0; e < 4; ++e) { a[e] = x[e]; b[e] = x[4 + e]; }
    *reinterpret_cast<f4*>(p) = a;
    *reinterpret_cast<f4*>(p + 4) = b;
  } else {
    bf16x8 v;
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = (bf16)x[e];
    *reinterpret_cast<bf16x8*>(p) = v;
  }
}

// A workgroup barrier that orders LDS only: global stores issued before it
// need not have completed (__syncthreads waits for every outstanding store).
// Global data exchanged between the waves of a workgroup needs __syncthreads.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Splits a grid of G = NB * NS blocks into (b, s), b in [0, NB), s in [0, NS),
// so that the NS slices of one b run on the same XCD (blocks are dealt to the
// 8 XCDs round robin, block x on XCD x % 8). Falls back to b = x / NS when
// NB is not a multiple of 8.
__device__ __forceinline__ void xcd_split(int x, int G, int NS, int& b, int& s) {
  const int NB = G / NS;
  if (NB % 8 != 0) {
    b = x / NS;
    s = x % NS;
    return;
  }
  const int xcd = x % 8, r = x / 8;
  b = (r / NS) * 8 + xcd;
  s = r % NS;
}

// Splits a grid of B * H * NF blocks, one per (batch, head, firing), so that
// every block of head h runs on XCD h % 8 when H is a multiple of 8: a head's
// parameters (read by every firing) then stay in one XCD's L2 instead of
// being fetched into all eight. Otherwise the blocks are in launch order.
__device__ __forceinline__ void head_xcd_split(int x, int H, int NF, int& b, int& h, int& i) {
  if (H % 8 != 0) {
    i = x % NF;
    const int bh = x / NF;
    h = bh % H;
    b = bh / H;
    return;
  }
  const int xcd = x % 8, r = x / 8, H8 = H / 8;
  i = r % NF;
  const int t = r / NF;
  h = (t % H8) * 8 + xcd;
  b = t / H8;
}


// Fragments gathered down a column: KPL consecutive rows of column 0 at p
// (row stride ld), for operands whose reduction index runs along the rows of
// a row-major array staged in LDS. Exact (E) or derived (fp32) storage.
template <typename E>
__device__ __forceinline__ typename Mma<E>::Frag gather_x(const E* p, int ld) {
  if constexpr (std::is_same<E, float>::value) {
    return p[0];
  } else {
    typename Mma<E>::Frag r;
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = p[e * ld];
    return r;
  }
}
template <typename E>
__device__ __forceinline__ typename Mma<E>::SFrag gather_s(const float* p, int ld) {
  return Mma<E>::makes([&](int e) { return p[e * ld]; });
}

// Row padding (elements) that keeps rows 16-byte aligned and staggers banks.
template <typename T> constexpr int pad16() { return 16 / (int)sizeof(T); }

// Accumulator element (r) of this lane lives at (row, col) of the 16x16 tile.
__device__ __forceinline__ int acc_row(int r) { return 4 * (lane_id() >> 4) + r; }
__device__ __forceinline__ int acc_col() { return lane_id() & 15; }

// Stages rows x cols fp32 (row stride src_ld) into LDS rows of stride ld with
// 16-byte accesses.
__device__ __forceinline__ void stage_f32(float* dst, int ld, const float* src, int src_ld,
                                          int rows, int cols) {
  const int segs = cols / 4;
  for (int e = threadIdx.x; e < rows * segs; e += blockDim.x) {
    const int r = e / segs, c = (e % segs) * 4;
    *reinterpret_cast<f4*>(dst + r * ld + c) = *reinterpret_cast<const f4*>(src + (size_t)r * src_ld + c);
  }
}

// ROWS x COLS fp32 values of a row-major global array (row stride src_ld)
// into fp32 LDS rows of stride ld, 16 bytes per access by NTH threads, every
// load of a thread issued before its first LDS write.
template <int NTH, int ROWS, int COLS>
__device__ __forceinline__ void stage_f32(float* dst, int ld, const float* src, int src_ld) {
  constexpr int SEGS = COLS / 4, NSEG = ROWS * SEGS, PER = (NSEG + NTH - 1) / NTH;
  static_assert(COLS % 4 == 0, "whole 16-byte groups");
  f4 x[PER];
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int e = threadIdx.x + NTH * u, r = e / SEGS, c = (e % SEGS) * 4;
    if (NSEG % NTH == 0 || e < NSEG) x[u] = *reinterpret_cast<const f4*>(src + (size_t)r * src_ld + c);
  }
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int e = threadIdx.x + NTH * u, r = e / SEGS, c = (e % SEGS) * 4;
    if (NSEG % NTH == 0 || e < NSEG) *reinterpret_cast<f4*>(dst + r * ld + c) = x[u];
  }
}

// ROWS x COLS fp32 values of a row-major global array (row stride src_ld)
// into a split LDS tile with row stride ld, 16 bytes per access by NTH
// threads: every load of a thread is issued before its first LDS write, so
// the loads are in flight together rather than one round trip each.
template <int NTH, int ROWS, int COLS, typename ST>
__device__ __forceinline__ void stage_split(const ST& dst, int ld, const float* src, int src_ld) {
  constexpr int SEGS = COLS / 4, NSEG = ROWS * SEGS, PER = (NSEG + NTH - 1) / NTH;
  static_assert(COLS % 4 == 0, "whole 16-byte groups");
  f4 x[PER];
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int e = threadIdx.x + NTH * u, r = e / SEGS, c = (e % SEGS) * 4;
    if (NSEG % NTH == 0 || e < NSEG) x[u] = *reinterpret_cast<const f4*>(src + (size_t)r * src_ld + c);
  }
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int e = threadIdx.x + NTH * u, r = e / SEGS, c = (e % SEGS) * 4;
    if (NSEG % NTH == 0 || e < NSEG) dst.put4(r * ld + c, x[u]);
  }
}

// ---------------------------------------------------------------- misc

// e^x on the hardware exp2 (v_exp_f32): x log2(e) rounded once, so the
// relative error is about |x| 2^-24 ln 2 on top of exp2's own (under 1e-6
// for the |x| < 20 of the decay factors, 5e-6 at the 88 clamp); a quarter of
// the instructions of the library expf, which dominated the chunk kernels'
// VALU time.
__device__ __forceinline__ float fexp(float x) {
  return __builtin_amdgcn_exp2f(x * 1.4426950408889634f);
}

// The probes' gates, evaluated N K (or N V) times per firing: from the
// hardware exp, log and reciprocal (a few ulp) rather than the library expf,
// log1pf and an IEEE division, which cost several times the instructions.
__device__ __forceinline__ float sigmoidf_(float x) {
  return __builtin_amdgcn_rcpf(1.f + fexp(-x));
}
// log(1 + e^x) with torch's threshold 20: max(x, 0) + log1p(t), t = e^-|x|;
// log1p(t) = log(u) t / (u - 1) with u = 1 + t rounded (the quotient undoes
// the rounding of u; Goldberg 1991, theorem 4)
__device__ __forceinline__ float softplusf_(float x) {
  if (x > 20.f) return x;
  const float t = fexp(-fabsf(x));
  const float u = 1.f + t;
  const float l = u == 1.f ? t : __logf(u) * (t * __builtin_amdgcn_rcpf(u - 1.f));
  return fmaxf(x, 0.f) + l;
}

// Sum over each row of 16 lanes (lanes 16r .. 16r + 15), every lane of the
// row receiving it: pairs, quads, halves, then the whole row, each step a DPP
// move inside the row (no trip through the LDS crossbar). Every lane of a
// row adds the same two partials, so all of them hold the same bits.
template <int CTRL>
__device__ __forceinline__ float dpp_row_mov(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float row16_sum(float x) {
  x += dpp_row_mov<0xB1>(x);    // quad_perm [1,0,3,2]: lane ^ 1
  x += dpp_row_mov<0x4E>(x);    // quad_perm [2,3,0,1]: lane ^ 2
  x += dpp_row_mov<0x141>(x);   // row_half_mirror: lane i <-> 7 - i within 8
  x += dpp_row_mov<0x140>(x);   // row_mirror: lane i <-> 15 - i
  return x;
}

// Bounded per-block LDS reductions are written inline in the kernels; this is
// the wave-level sum.
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o, WAVE);
  return x;
}

}  // namespace ngdn
