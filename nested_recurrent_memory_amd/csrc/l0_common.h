// Per-chunk level-0 building blocks shared by the forward (l0_intra.hip) and
// backward (l0_bwd.hip) kernels. A workgroup of 4 waves owns one
// (batch, head, chunk); wave w owns block-row w (16 rows) wherever rows split.
#pragma once

#include "ngdn_kernels.h"

namespace ngdn {

// Inputs of one chunk in the reference layout.
template <typename E, int K, int V>
struct ChunkIn {
  const E* q; const E* k; const E* b; const E* v; const E* w; const float* g;
  size_t rowQ, rowK, rowV;
  int t0, nvalid;
  float scale;

  __device__ __forceinline__ void init(const void* q_, const void* k_, const void* v_,
                                       const float* g_, const void* b_, const void* w_,
                                       int bi, int h, int n, int T, int H, int L, float sc) {
    const size_t bt = (size_t)bi * T * H + h;
    q = static_cast<const E*>(q_) + bt * L * K;
    k = static_cast<const E*>(k_) + bt * K;
    b = static_cast<const E*>(b_) + bt * K;
    v = static_cast<const E*>(v_) + bt * V;
    w = static_cast<const E*>(w_) + bt * V;
    g = g_ + bt * K;
    rowQ = (size_t)H * L * K; rowK = (size_t)H * K; rowV = (size_t)H * V;
    t0 = n * CH;
    nvalid = min(CH, T - t0);
    scale = sc;
  }
  // element loads, zero past the sequence end
  __device__ __forceinline__ float ld(const E* p, size_t row, int i, int c) const {
    return i < nvalid ? to_f(p[(size_t)(t0 + i) * row + c]) : 0.f;
  }
  __device__ __forceinline__ float K_(int i, int c) const { return ld(k, rowK, i, c); }
  __device__ __forceinline__ float B_(int i, int c) const { return ld(b, rowK, i, c); }
  __device__ __forceinline__ float Q_(int i, int c) const { return ld(q, rowQ, i, c); }
  __device__ __forceinline__ float V_(int i, int c) const { return ld(v, rowV, i, c); }
  __device__ __forceinline__ float W_(int i, int c) const { return ld(w, rowV, i, c); }
  // 16 bytes of row i from column c0 as floats (zero past the end)
  static constexpr int VE = 16 / (int)sizeof(E);
  __device__ __forceinline__ void vec16(const E* p, size_t row, int i, int c0, float* out) const {
    if (i < nvalid) {
      const E* src = p + (size_t)(t0 + i) * row + c0;
      if constexpr (std::is_same<E, float>::value) {
        const f4 x = *reinterpret_cast<const f4*>(src);
#pragma unroll
        for (int e = 0; e < 4; ++e) out[e] = x[e];
      } else {
        ld_vals<E>(src, out);
      }
    } else {
#pragma unroll
      for (int e = 0; e < VE; ++e) out[e] = 0.f;
    }
  }
  // 16 bytes of row i from column c0, kept raw (zero past the end), and
  // their VE values as floats: a load read ahead this way is not waited for
  // until raw16_vals converts it.
  typedef __attribute__((__vector_size__(16))) int R16;
  // Rows past the end read the last valid row and then take zero: the load
  // is not under a branch, so no register copy at a branch merge has to wait
  // for it (and for every load issued before it).
  __device__ __forceinline__ R16 raw16(const E* p, size_t row, int i, int c0) const {
    const int ic = i < nvalid ? i : nvalid - 1;
    const R16 x = *reinterpret_cast<const R16*>(p + (size_t)(t0 + ic) * row + c0);
    const R16 z = {0, 0, 0, 0};
    return i < nvalid ? x : z;
  }
  __device__ __forceinline__ static void raw16_vals(R16 x, float* out) {
    if constexpr (std::is_same<E, float>::value) {
      const f4 v = __builtin_bit_cast(f4, x);
#pragma unroll
      for (int e = 0; e < 4; ++e) out[e] = v[e];
    } else {
      const bf16x8 v = __builtin_bit_cast(bf16x8, x);
#pragma unroll
      for (int e = 0; e < 8; ++e) out[e] = (float)v[e];
    }
  }
  // Mma<E>::KPL consecutive elements of row i from column c0 (zero past the end)
  __device__ __forceinline__ void vals(const E* p, size_t row, int i, int c0, float* out) const {
    if (i < nvalid) {
      ld_vals<E>(p + (size_t)(t0 + i) * row + c0, out);
    } else {
#pragma unroll
      for (int e = 0; e < Mma<E>::KPL; ++e) out[e] = 0.f;
    }
  }
};

constexpr int GCP = 1;   // padding of gc rows
constexpr int AT_LD = CH + 1;


// gc[i][c] = sum_{s<=i} g_s[c0 + c] within the chunk (zero past the end) for
// the NC columns from c0, into dst [64][LDG]; glast (when set) receives row
// 63. TPC = 256 / NC adjacent lanes share a column, each summing 64 / TPC
// consecutive rows in registers (independent loads); the segment offsets come
// from the neighbouring lanes.
template <int NC, int LDG, typename E, int K, int V>
__device__ __forceinline__ void cumsum_cols(float* dst, const ChunkIn<E, K, V>& in, int c0,
                                            float* glast) {
  constexpr int TPC = 256 / NC;
  constexpr int SEG = CH / TPC;
  const int tid = threadIdx.x, c = tid / TPC, part = tid % TPC;
  float x[SEG];
#pragma unroll
  for (int r = 0; r < SEG; ++r) {
    const int i = part * SEG + r;
    x[r] = i < in.nvalid ? in.g[(size_t)(in.t0 + i) * in.rowK + c0 + c] : 0.f;
  }
#pragma unroll
  for (int r = 1; r < SEG; ++r) x[r] += x[r - 1];
  const int base = lane_id() & ~(TPC - 1);
  float off = 0.f;
#pragma unroll
  for (int p = 0; p < TPC - 1; ++p) {
    const float t = __shfl(x[SEG - 1], base + p, WAVE);
    if (p < part) off += t;
  }
#pragma unroll
  for (int r = 0; r < SEG; ++r) dst[(part * SEG + r) * LDG + c] = x[r] + off;
  if (glast && part == TPC - 1) glast[c] = x[SEG - 1] + off;
}

// gc over all K columns into s_gc [64][K + GCP].
template <typename E, int K, int V>
__device__ __forceinline__ void l0_cumsum(float* s_gc, const ChunkIn<E, K, V>& in) {
  cumsum_cols<K, K + GCP>(s_gc, in, 0, static_cast<float*>(nullptr));
}

// Largest decay inside 16-row block I over NC columns of gc (row stride LDG):
// max (gc[16 I] - gc[j]). When it is at most 80 nats, factors e^(gc_r - gc_j)
// for j in the block stay inside fp32 range.
template <int NC, int LDG>
__device__ __forceinline__ bool block_safe(const float* gc, int I) {
  const int lane = lane_id(), r = 16 * I;
  float dmax = 0.f;
  for (int e = lane; e < 16 * NC; e += WAVE) {
    const int j = r + e / NC, c = e % NC;
    dmax = fmaxf(dmax, gc[r * LDG + c] - gc[j * LDG + c]);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) dmax = fmaxf(dmax, __shfl_xor(dmax, o, WAVE));
  return dmax <= 80.f;
}
template <int K>
__device__ __forceinline__ bool l0_block_safe(const float* s_gc, int I) {
  return block_safe<K, K + GCP>(s_gc, I);
}

// Per-row outputs written while the chunk's rows are in registers (forward
// only; either pointer may be null): Qg = scale q e^gc [64][K] and
// Kt^T = (k e^(gc_last - gc))^T [K][64], both in split form (they enter the
// matrix cores only, as A operands by row tile), for bf16 in fragment
// order.
struct RowOut {
  float* Qg; float* KtT;
};

// A (strictly lower, into s_A fp32 [64][AT_LD]) and, when aqk_out != null,
// Aqk (lower incl. diagonal) to global [64][64] in split form. Wave w
// computes block-row w. With per-row outputs, s_x is LDS scratch of
// 64 x (64 + 4) floats for the transposed one, and the call ends with a
// barrier.
template <typename E, int K, int V>
__device__ __forceinline__ void l0_build_A(float* s_A, const float* s_gc,
                                           const ChunkIn<E, K, V>& in, float* aqk_out,
                                           const RowOut& ro = RowOut{},
                                           float* s_x = nullptr) {
  constexpr int GL = K + GCP;
  constexpr int NKS = K / Mma<E>::KS;
  constexpr int KPL = Mma<E>::KPL;
  typedef typename Mma<E>::SFrag SF;
  const int lane = lane_id(), I = wave_id(), r = 16 * I;
  const bool want_q = aqk_out != nullptr;
  // bf16: every split output in fragment order
  constexpr bool FRAG = std::is_same<E, bf16>::value;
  typedef typename Mma<E>::Frag FR;
  const int ri = r + (lane & 15);
  // Every global load of the phase first, all in flight together: this
  // wave's rows of b, k, q, and the k rows of the earlier tiles J < I (the
  // rows of tile I are this wave's own)
  // The loads are unconditional (rows past the sequence end read its last
  // row, tiles J >= I this wave's own rows again) and the unwanted values are
  // zeroed afterwards: a load under a branch leaves a register copy at the
  // merge, and the copy waits for every load issued before it.
  FR bo[NKS], ko[NKS], qo[NKS], kj[3][NKS];
  {
    const bool live = ri < in.nvalid;
    const int ric = live ? ri : in.nvalid - 1;
    const size_t rowk = (size_t)(in.t0 + ric) * in.rowK, rowq = (size_t)(in.t0 + ric) * in.rowQ;
    const bool use_q = live && (want_q || ro.Qg);
#pragma unroll
    for (int s = 0; s < NKS; ++s) {
      const int c0 = s * Mma<E>::KS + kofs<E>(lane);
      const FR xb = Mma<E>::ld(in.b + rowk + c0), xk = Mma<E>::ld(in.k + rowk + c0);
      const FR xq = Mma<E>::ld(in.q + rowq + c0);
      bo[s] = live ? xb : Mma<E>::zero();
      ko[s] = live ? xk : Mma<E>::zero();
      qo[s] = use_q ? xq : Mma<E>::zero();
    }
#pragma unroll
    for (int J = 0; J < 3; ++J) {
      // rows of an earlier tile can still lie past the sequence end when this
      // wave's own rows do (a partial last chunk): those read as zero
      const int rj = 16 * J + (lane & 15);
      const bool in_seq = J < I && rj < in.nvalid;
      const int rjc = J < I ? (rj < in.nvalid ? rj : in.nvalid - 1) : ric;
#pragma unroll
      for (int s = 0; s < NKS; ++s) {
        const int c0 = s * Mma<E>::KS + kofs<E>(lane);
        const FR x = Mma<E>::ld(in.k + (size_t)(in.t0 + rjc) * in.rowK + c0);
        kj[J][s] = in_seq ? x : Mma<E>::zero();
      }
    }
  }
  const bool safe = l0_block_safe<K>(s_gc, I);
  SF lf[NKS], qf[NKS];
#pragma unroll
  for (int s = 0; s < NKS; ++s) {
    const int c0 = s * Mma<E>::KS + kofs<E>(lane);
    float gi[KPL];
#pragma unroll
    for (int e = 0; e < KPL; ++e) gi[e] = s_gc[ri * GL + c0 + e];
    lf[s] = Mma<E>::makes([&](int e) {
      return to_f(Mma<E>::elem(bo[s], e)) * to_f(Mma<E>::elem(ko[s], e)) *
             fexp(gi[e] - s_gc[r * GL + c0 + e]);
    });
    if (want_q) {
      qf[s] = Mma<E>::makes([&](int e) {
        return to_f(Mma<E>::elem(qo[s], e)) * in.scale * fexp(gi[e] - s_gc[r * GL + c0 + e]);
      });
    }
  }
  // every load of the phase before its first global store
  f4 accAs[4], accQs[4];
#pragma unroll
  for (int J = 0; J < 4; ++J) {
    f4 accA = f4_zero(), accQ = f4_zero();
    if (J <= I) {
      const int rj = 16 * J + (lane & 15);
#pragma unroll
      for (int s = 0; s < NKS; ++s) {
        const int c0 = s * Mma<E>::KS + kofs<E>(lane);
        const FR kr = (J == 3 || J == I) ? ko[s] : kj[J < 3 ? J : 0][s];
        const SF kf = Mma<E>::makes([&](int e) {
          const float x = s_gc[r * GL + c0 + e] - s_gc[rj * GL + c0 + e];
          return to_f(Mma<E>::elem(kr, e)) * fexp(J < I ? x : fminf(x, 88.f));
        });
        accA = Mma<E>::mma(accA, lf[s], kf);
        if (want_q) accQ = Mma<E>::mma(accQ, qf[s], kf);
      }
      if (J == I && !safe) {
        // exact pairwise form for this diagonal tile
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          const int i = r + acc_row(rr), j = 16 * J + acc_col();
          float sa = 0.f, sq = 0.f;
          if (j <= i) {
            for (int c = 0; c < K; ++c) {
              const float d = fexp(fminf(s_gc[i * GL + c] - s_gc[j * GL + c], 0.f));
              const float kjv = in.K_(j, c);
              sa += in.B_(i, c) * in.K_(i, c) * kjv * d;
              if (want_q) sq += in.Q_(i, c) * kjv * d;
            }
          }
          accA[rr] = sa;
          accQ[rr] = sq * in.scale;
        }
      }
    }
    accAs[J] = accA;
    accQs[J] = accQ;
  }
#pragma unroll
  for (int J = 0; J < 4; ++J) {
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int i = r + acc_row(rr), j = 16 * J + acc_col();
      s_A[i * AT_LD + j] = (j < i) ? accAs[J][rr] : 0.f;
      if (aqk_out)
        split_at<E>(aqk_out, CH * CH).put1(FRAG ? frag_ofs(i, j, CH) : i * CH + j,
                                           (j <= i) ? accQs[J][rr] : 0.f);
    }
  }
  if (ro.Qg || ro.KtT) {
    // Kt^T, then Qg (split): each value computed once into the LDS scratch
    // s_x [64 columns][CH + 4], then written from there (transposed for
    // Kt^T), 16-byte rows both
    constexpr int LDX = CH + 4;
    for (int which = 0; which < 2; ++which) {
      float* tp = which ? nullptr : ro.KtT;
      float* rp = which ? ro.Qg : nullptr;
      if (!tp && !rp) continue;
      const SplitTile<E> tdst = split_at<E>(tp, K * CH), rdst = split_at<E>(rp, CH * K);
      for (int hh = 0; hh < K / 64; ++hh) {
#pragma unroll
        for (int s = 0; s < NKS; ++s) {
          if (s * Mma<E>::KS / 64 != hh) continue;
          const int c0 = s * Mma<E>::KS + kofs<E>(lane);
#pragma unroll
          for (int e = 0; e < KPL; ++e) {
            const float gi = s_gc[ri * GL + c0 + e];
            s_x[(c0 + e - 64 * hh) * LDX + ri] =
                which ? to_f(Mma<E>::elem(qo[s], e)) * in.scale * fexp(gi)
                      : to_f(Mma<E>::elem(ko[s], e)) * fexp(s_gc[(CH - 1) * GL + c0 + e] - gi);
          }
        }
        lds_barrier();
        if (tp) {
          // rows 64 hh .. + 63 of the transposed copy: contiguous in either order
          for (int idx = threadIdx.x; idx < 64 * CH / 4; idx += blockDim.x) {
            int kl, m;
            if (FRAG) {
              frag_pos(idx * 4, CH, kl, m);
            } else {
              kl = idx / (CH / 4);
              m = (idx % (CH / 4)) * 4;
            }
            tdst.put4(64 * hh * CH + idx * 4, *reinterpret_cast<const f4*>(s_x + kl * LDX + m));
          }
        }
        if (rp) {
          const bool fr = FRAG;
          for (int idx = threadIdx.x; idx < CH * 64 / 4; idx += blockDim.x) {
            int m, kl, off;
            if (fr) {
              // column blocks 2 hh, 2 hh + 1 of every row block
              const int q = idx * 4, bl = q >> 9, w = q & 511, l = w >> 3;
              m = (bl >> 1) * 16 + (l & 15);
              kl = (bl & 1) * 32 + (l >> 4) * 8 + (w & 7);
              off = ((bl >> 1) * (K / 32) + 2 * hh + (bl & 1)) * 512 + w;
            } else {
              m = idx / 16;
              kl = (idx % 16) * 4;
              off = m * K + 64 * hh + kl;
            }
            f4 x;
#pragma unroll
            for (int j = 0; j < 4; ++j) x[j] = s_x[(kl + j) * LDX + m];
            rdst.put4(off, x);
          }
        }
        lds_barrier();
      }
    }
  }
}

// T = (I + A)^-1 by 16-row blocks. The diagonal blocks by forward
// substitution (wave 0, one column of one block per lane); the blocks below
// the diagonal by two levels of 2 x 2 block inversion on the fp32 matrix
// cores (products exact in fp32, v_mfma_f32_16x16x4_f32), in three rounds:
//   T10 = -T11 A10 T00,  T32 = -T33 A32 T22         (waves 0, 1)
//   Y = A[32:64, 0:32] T[0:32, 0:32]                  (one 16 x 16 block per wave)
//   T[32:64, 0:32] = -T[32:64, 32:64] Y               (one block per wave)
// since [[L1, 0], [A21, L2]]^-1 = [[L1^-1, 0], [-L2^-1 A21 L1^-1, L2^-1]].
// The blocks of s_A above the diagonal are never read here: they hold the
// four Y blocks ((0,1), (0,2), (0,3), (1,2)) and the middle factor of the
// first round's triple products ((1,3) for wave 0, (2,3) for wave 1). s_T
// has row stride LDT. Ends with a barrier.
template <int LDT>
__device__ __forceinline__ void l0_invert(float* s_A, float* s_T) {
  typedef Mma<float> MF;
  const int lane = lane_id(), wv = wave_id(), tid = threadIdx.x;
  if (wv == 0) {
    const int I = lane >> 4, c = lane & 15, o = 16 * I;
    float t[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float val = (i == c) ? 1.f : 0.f;
#pragma unroll
      for (int j = 0; j < i; ++j)
        if (j >= c) val -= s_A[(o + i) * AT_LD + o + j] * t[j];
      t[i] = (i >= c) ? val : 0.f;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) s_T[(o + i) * LDT + o + c] = t[i];
  } else {
    for (int e = tid - WAVE; e < CH * CH; e += 3 * WAVE) {
      const int i = e / CH, j = e % CH;
      if ((i >> 4) != (j >> 4)) s_T[i * LDT + j] = 0.f;
    }
  }
  lds_barrier();
  // fp32 fragments (one k-value per lane): A operand of block (I, M) at
  // k-step s, B operand of block (M, J); accumulators hold rows
  // 4 (lane / 16) + r, column lane % 16
  const int lr = lane & 15, lk = lane >> 4;
  auto aA = [&](int I, int M, int s) { return s_A[(16 * I + lr) * AT_LD + 16 * M + 4 * s + lk]; };
  auto aT = [&](int I, int M, int s) { return s_T[(16 * I + lr) * LDT + 16 * M + 4 * s + lk]; };
  auto bT = [&](int M, int J, int s) { return s_T[(16 * M + 4 * s + lk) * LDT + 16 * J + lr]; };
  auto bP = [&](const float* p, int s) { return p[(4 * s + lk) * AT_LD + lr]; };
  auto put = [&](float* dst, int ld, f4 acc, float sign) {
#pragma unroll
    for (int r = 0; r < 4; ++r) dst[(4 * lk + r) * ld + lr] = sign * acc[r];
  };
  // block (r, c) of s_A above the diagonal, as scratch
  auto up = [&](int r, int c) { return s_A + 16 * r * AT_LD + 16 * c; };
  const int yr[4] = {0, 0, 0, 1}, yc[4] = {1, 2, 3, 2};   // Y_{M,J} in block q = 2 (M - 2) + J
  if (wv < 2) {
    const int I = wv ? 3 : 1, J = I - 1;
    float* own = up(wv + 1, 3);
    f4 p = f4_zero(), t = f4_zero();
#pragma unroll
    for (int s = 0; s < 4; ++s) p = MF::mma(p, aA(I, J, s), bT(J, J, s));
    put(own, AT_LD, p, 1.f);   // this wave's own scratch: read back in its program order
#pragma unroll
    for (int s = 0; s < 4; ++s) t = MF::mma(t, aT(I, I, s), bP(own, s));
    put(s_T + 16 * I * LDT + 16 * J, LDT, t, -1.f);
  }
  lds_barrier();
  const int I = 2 + (wv >> 1), J = wv & 1;
  {
    // Y_IJ = sum_{M = J..1} A_IM T_MJ
    f4 y = f4_zero();
#pragma unroll
    for (int M = 0; M < 2; ++M)
      if (M >= J) {
#pragma unroll
        for (int s = 0; s < 4; ++s) y = MF::mma(y, aA(I, M, s), bT(M, J, s));
      }
    put(up(yr[wv], yc[wv]), AT_LD, y, 1.f);
  }
  lds_barrier();
  {
    // T_IJ = -sum_{M = 2..I} T_IM Y_MJ
    f4 t = f4_zero();
#pragma unroll
    for (int M = 2; M < 4; ++M)
      if (M <= I) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const int q = (M - 2) * 2 + J;
          t = MF::mma(t, aT(I, M, s), bP(up(yr[q], yc[q]), s));
        }
      }
    put(s_T + 16 * I * LDT + 16 * J, LDT, t, -1.f);
  }
  lds_barrier();
}

// Right-hand sides transposed into s_X fp32 [(K+V)][LDX]: X[k][c] = b k e^gc,
// X[K+v][c] = w v.
template <typename E, int K, int V, int LDX>
__device__ __forceinline__ void l0_build_X(float* s_X, const float* s_gc, const ChunkIn<E, K, V>& in) {
  const int tid = threadIdx.x;
  for (int e = tid; e < CH * K; e += 256) {
    const int c = e / K, kk = e % K;
    s_X[kk * LDX + c] = in.B_(c, kk) * in.K_(c, kk) * fexp(s_gc[c * (K + GCP) + kk]);
  }
  for (int e = tid; e < CH * V; e += 256) {
    const int c = e / V, vv = e % V;
    s_X[(K + vv) * LDX + c] = in.W_(c, vv) * in.V_(c, vv);
  }
}

// MFMA depth for block-row I of a lower-triangular left operand.
template <typename E> __device__ __forceinline__ int tri_depth(int I) {
  return min(CH, ((16 * (I + 1) + Mma<E>::KS - 1) / Mma<E>::KS) * Mma<E>::KS);
}

}  // namespace ngdn
