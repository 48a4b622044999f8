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
__device__ __forceinline__ int wave_id() { return threadIdx.x / WAVE; }

template <typename T> __device__ __forceinline__ float to_f(T x) { return (float)x; }
template <typename T> __device__ __forceinline__ T from_f(float x) { return (T)x; }

__device__ __forceinline__ f4 f4_zero() { f4 z = {0.f, 0.f, 0.f, 0.f}; return z; }

// ---------------------------------------------------------------- MFMA

template <typename E> struct Mma;

template <> struct Mma<bf16> {
  static constexpr int KS = 32;   // k per instruction
  static constexpr int KPL = 8;   // k-values per lane
  typedef bf16x8 Frag;
  __device__ __forceinline__ static f4 mma(f4 acc, Frag a, Frag b) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
  }
  __device__ __forceinline__ static Frag load(const bf16* p) {
    return *reinterpret_cast<const bf16x8*>(p);
  }
  template <typename F>
  __device__ __forceinline__ static Frag make(F f) {  // f(e) -> float, e < KPL
    Frag r;
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = (bf16)f(e);
    return r;
  }
  // x = hi + lo to about 16 mantissa bits: products against an operand built
  // this way keep fp32-level agreement between sums that must cancel.
  template <typename F>
  __device__ __forceinline__ static void make_split(F f, Frag& hi, Frag& lo) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float x = f(e);
      const bf16 h = (bf16)x;
      hi[e] = h;
      lo[e] = (bf16)(x - (float)h);
    }
  }
  static constexpr bool SPLIT = true;
};

template <> struct Mma<float> {
  static constexpr int KS = 4;
  static constexpr int KPL = 1;
  typedef float Frag;
  __device__ __forceinline__ static f4 mma(f4 acc, Frag a, Frag b) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc, 0, 0, 0);
  }
  __device__ __forceinline__ static Frag load(const float* p) { return *p; }
  template <typename F>
  __device__ __forceinline__ static Frag make(F f) { return f(0); }
  template <typename F>
  __device__ __forceinline__ static void make_split(F f, Frag& hi, Frag& lo) {
    hi = f(0);
    lo = 0.f;
  }
  static constexpr bool SPLIT = false;
};

template <typename E> __device__ __forceinline__ int kofs(int lane) {
  return Mma<E>::KPL * (lane >> 4);
}

// D[16x16] += A[16 x kd] * B[kd x 16], A row-major (k contiguous, stride lda),
// B given as Bt[16][kd] (k contiguous, stride ldb). kd a multiple of KS.
template <typename E>
__device__ __forceinline__ f4 mma_tile(f4 acc, const E* A, int lda, const E* Bt,
                                       int ldb, int kd) {
  const int l = lane_id();
  const E* pa = A + (l & 15) * lda + kofs<E>(l);
  const E* pb = Bt + (l & 15) * ldb + kofs<E>(l);
  for (int k = 0; k < kd; k += Mma<E>::KS)
    acc = Mma<E>::mma(acc, Mma<E>::load(pa + k), Mma<E>::load(pb + k));
  return acc;
}

// Accumulator element (r) of this lane lives at (row, col) of the 16x16 tile.
__device__ __forceinline__ int acc_row(int r) { return 4 * (lane_id() >> 4) + r; }
__device__ __forceinline__ int acc_col() { return lane_id() & 15; }

// ---------------------------------------------------------------- misc

__device__ __forceinline__ float sigmoidf_(float x) { return 1.f / (1.f + expf(-x)); }
__device__ __forceinline__ float softplusf_(float x) {
  // log(1 + e^x), stable on both tails
  return x > 20.f ? x : log1pf(expf(x));
}

// Bounded per-block LDS reductions are written inline in the kernels; this is
// the wave-level sum.
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o, WAVE);
  return x;
}

}  // namespace ngdn
