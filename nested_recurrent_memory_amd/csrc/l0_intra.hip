// Level-0 intra-chunk forward: everything about a 64-token chunk that does not
// depend on the recurrent state.
//
// Restates the per-chunk terms of the reference's chunk form
// (nested_gdn2/ops/naive.py:329-358), which the reference obtains from fla's
// chunk_gdn2_fwd (called at nested_gdn2/ops/chunk.py:236-248):
//   gc   = cumsum(g) within the chunk
//   A_ij = sum_k b_i k_i k_j e^(gc_i - gc_j)             j <  i
//   T    = (I + A)^-1
//   W    = T (b * k * e^gc),  U = T (w * v)
//   Kt_i = k_i * e^(gc_last - gc_i)
//   Qg   = scale * q0 * e^gc
//   Aqk  = sum_k scale q_i k_j e^(gc_i - gc_j)            j <= i
//   gam  = e^gc_last
// The forward scan consumes W, U, Kt^T, Qg, Aqk; the reverse scan reads the
// same split tiles and transposes them on chip; the chunk backward reads
// T^T, written when its pointer is set. For bf16 inputs the products run on
// bf16 MFMA with the derived operands split in two (ngdn_common.h); the
// matrix-core operands W, Kt^T, Qg, Aqk are stored split (split_at), U, gam
// and T^T as fp32.
//
// One workgroup (4 waves) per (batch, head, chunk). Decay products are formed
// without overflow: inside block-row I (16 rows starting at r = 16 I) every
// pair uses r as the reference point, e^(gc_i - gc_j) = e^(gc_i - gc_r) e^(gc_r - gc_j).
// Both factors are <= 1 for j < r; on the diagonal block the right factor is
// e^(decay over at most 15 tokens), and when that could leave fp32 range
// (more than 80 nats in some channel) the diagonal tile is recomputed pair by
// pair with clamped exponents, exactly as the reference does.
#include "l0_common.h"

namespace ngdn {

template <typename E, int K, int V>
__global__ __launch_bounds__(256, sizeof(E) == 2 ? 2 : 1) void l0_intra_fwd_kernel(L0IntraArgs a) {
  constexpr int C = CH;
  constexpr int GL = K + GCP;                // gc rows
  constexpr int LT = C + 4;                  // T rows, 16-byte aligned for fragment loads
  constexpr int KS = Mma<E>::KS;
  typedef typename Mma<E>::SFrag SF;
  const int NT = a.NT, H = a.H;
  const int nn = a.nn > 0 ? a.nn : NT;
  const int n = a.n0 + (int)(blockIdx.x % nn);
  const int bh = blockIdx.x / nn;
  const int h = bh % H, b = bh / H;
  const int lane = lane_id(), wv = wave_id(), tid = threadIdx.x;

  // LDS: gc, and a region holding A and T, later the
  // transposed right-hand sides X_w^T, then X_u^T. Each wave keeps its 16 rows
  // of T in registers across the reuse.
  constexpr size_t SZ_GC = sizeof(float) * C * GL;
  constexpr size_t SZ_AT = sizeof(float) * (C * AT_LD + C * LT);
  constexpr size_t SZ_XT = sizeof(typename SplitTile<E>::T) * SplitTile<E>::NPLANE *
                           (K > V ? K : V) * (C + SplitTile<E>::PAD);
  constexpr size_t SZ_WU = sizeof(float) * C * (K + 4 + V + 4) - SZ_GC;
  constexpr size_t SZ_R = SZ_AT > SZ_XT ? (SZ_AT > SZ_WU ? SZ_AT : SZ_WU) : (SZ_XT > SZ_WU ? SZ_XT : SZ_WU);
  __shared__ __attribute__((aligned(16))) char smem[SZ_GC + SZ_R];
  float* s_gc = reinterpret_cast<float*>(smem);
  float* s_A = reinterpret_cast<float*>(smem + SZ_GC);
  float* s_T = s_A + C * AT_LD;

  ChunkIn<E, K, V> in;
  in.init(a.q, a.k, a.v, a.g, a.b, a.w, b, h, n, a.T, H, a.L, a.scale);
  const size_t cix = (size_t)bh * NT + n;

  // ---- 1. in-chunk cumulative log decay
  l0_cumsum(s_gc, in);
  lds_barrier();

  // ---- 2. A and Aqk; Qg and Kt^T while the rows are loaded
  {
    RowOut ro{a.Qg + cix * C * K, a.KtT + cix * K * C};
    // s_T (free until the inversion) is the scratch for the transposed rows
    l0_build_A(s_A, s_gc, in, a.Aqk + cix * C * C, ro, s_T);
  }
  if (tid < K) a.gam[cix * K + tid] = fexp(s_gc[(C - 1) * GL + tid]);
  lds_barrier();

  // the right-hand sides' inputs, read now so that the loads overlap the
  // inversion: thread e takes row m = e % C, 16 bytes from column c
  constexpr int VE = ChunkIn<E, K, V>::VE;      // elements per 16-byte load
  constexpr int PW = C * K / VE / 256, PU = C * V / VE / 256;
  static_assert(C * K / VE % 256 == 0 && C * V / VE % 256 == 0, "whole 16-byte groups per thread");
  // (raw: converted only where they are used, so nothing waits for them here)
  typedef typename ChunkIn<E, K, V>::R16 R16;
  R16 rb[PW], rk[PW], rw[PU], rv[PU];
#pragma unroll
  for (int q = 0; q < PW; ++q) {
    const int e = tid + 256 * q, m = e % C, c = (e / C) * VE;
    rb[q] = in.raw16(in.b, in.rowK, m, c);
    rk[q] = in.raw16(in.k, in.rowK, m, c);
  }
#pragma unroll
  for (int q = 0; q < PU; ++q) {
    const int e = tid + 256 * q, m = e % C, c = (e / C) * VE;
    rw[q] = in.raw16(in.w, in.rowV, m, c);
    rv[q] = in.raw16(in.v, in.rowV, m, c);
  }

  // ---- 3. T = (I + A)^-1; each wave takes its block-row into registers
  l0_invert<LT>(s_A, s_T);
  const int I = wv, R0 = 16 * I;
  const int kd = tri_depth<E>(I);
  SF tf[C / KS];
  {
    const float* trow = s_T + (R0 + (lane & 15)) * LT + kofs<E>(lane);
#pragma unroll
    for (int s = 0; s < C / KS; ++s) tf[s] = Mma<E>::ld(trow + s * KS);
    if (a.TT) {
      // TT[j][i] = T[i][j]: four consecutive i of one column j per thread
      float* tt = a.TT + cix * C * C;
      for (int e = tid; e < C * C / 4; e += 256) {
        const int j = e / (C / 4), i = (e % (C / 4)) * 4;
        f4 x;
#pragma unroll
        for (int r = 0; r < 4; ++r) x[r] = s_T[(i + r) * LT + j];
        *reinterpret_cast<f4*>(tt + j * C + i) = x;
      }
    }
  }
  lds_barrier();

  // ---- 4-5. W = T X_w, U = T X_u; wave w owns block-row w. X_w^T = (b k
  // e^gc)^T, then X_u^T = (w v)^T, take the A/T region as split tiles (rows
  // of m, each value split once by the thread that writes it), so every B
  // fragment is a 16-byte read. All tiles stay in registers until both
  // products are done; then W and U replace everything in LDS and leave in
  // 16-byte rows, instead of 2- and 4-byte column-strided stores.
  {
    using ST = SplitTile<E>;
    constexpr int LDX = C + ST::PAD;
    static_assert(sizeof(typename ST::T) * ST::NPLANE * (K > V ? K : V) * LDX <= SZ_R,
                  "X^T fits the A/T region");
    const ST sX{reinterpret_cast<typename ST::T*>(s_A), (K > V ? K : V) * LDX};
    constexpr int NTW = K / 16, NTU = V / 16;
    f4 wt[NTW], ut[NTU];
#pragma unroll
    for (int q = 0; q < PW; ++q) {
      const int e = tid + 256 * q, m = e % C, c = (e / C) * VE;
      float xb[VE], xk[VE];
      ChunkIn<E, K, V>::raw16_vals(rb[q], xb);
      ChunkIn<E, K, V>::raw16_vals(rk[q], xk);
#pragma unroll
      for (int j = 0; j < VE; ++j)
        sX.put1((c + j) * LDX + m, xb[j] * xk[j] * fexp(s_gc[m * GL + c + j]));
    }
    lds_barrier();
#pragma unroll
    for (int tc = 0; tc < NTW; ++tc) {
      const int col = tc * 16 + (lane & 15);
      f4 acc = f4_zero();
#pragma unroll
      for (int s = 0; s < C / KS; ++s)
        if (s * KS < kd)   // T is zero past the block diagonal
          acc = Mma<E>::mma(acc, tf[s], sX.get(col * LDX + s * KS + kofs<E>(lane)));
      wt[tc] = acc;
    }
    lds_barrier();   // X_u^T replaces X_w^T
#pragma unroll
    for (int q = 0; q < PU; ++q) {
      const int e = tid + 256 * q, m = e % C, c = (e / C) * VE;
      float xw[VE], xv[VE];
      ChunkIn<E, K, V>::raw16_vals(rw[q], xw);
      ChunkIn<E, K, V>::raw16_vals(rv[q], xv);
#pragma unroll
      for (int j = 0; j < VE; ++j) sX.put1((c + j) * LDX + m, xw[j] * xv[j]);
    }
    lds_barrier();
#pragma unroll
    for (int tc = 0; tc < NTU; ++tc) {
      const int col = tc * 16 + (lane & 15);
      f4 acc = f4_zero();
#pragma unroll
      for (int s = 0; s < C / KS; ++s)
        if (s * KS < kd)
          acc = Mma<E>::mma(acc, tf[s], sX.get(col * LDX + s * KS + kofs<E>(lane)));
      ut[tc] = acc;
    }
    lds_barrier();   // X_u^T is no longer read
    constexpr int LW = K + 4, LUU = V + 4;   // fp32 rows, 16-byte aligned
    float* s_w = reinterpret_cast<float*>(smem);    // [C][LW], then U [C][LUU]
    float* s_u = s_w + C * LW;
    static_assert(sizeof(float) * C * (LW + LUU) <= SZ_GC + SZ_R, "W and U fit the LDS");
#pragma unroll
    for (int t = 0; t < NTW; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) s_w[(R0 + acc_row(r)) * LW + t * 16 + acc_col()] = wt[t][r];
#pragma unroll
    for (int t = 0; t < NTU; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) s_u[(R0 + acc_row(r)) * LUU + t * 16 + acc_col()] = ut[t][r];
    lds_barrier();
    // W [C][K] (split; bf16: in fragment order), U [C][V] (fp32): four
    // consecutive columns per thread
    const SplitTile<E> Wo = split_at<E>(a.W + cix * C * K, C * K);
    for (int e = tid; e < C * K / 4; e += 256) {
      int i, c;
      if (std::is_same<E, bf16>::value) {
        frag_pos(e * 4, K, i, c);
      } else {
        i = e / (K / 4);
        c = (e % (K / 4)) * 4;
      }
      Wo.put4(e * 4, *reinterpret_cast<const f4*>(s_w + i * LW + c));
    }
    float* Uo = a.U + cix * C * V;
    for (int e = tid; e < C * V / 4; e += 256) {
      const int i = e / (V / 4), c = (e % (V / 4)) * 4;
      *reinterpret_cast<f4*>(Uo + i * V + c) = *reinterpret_cast<const f4*>(s_u + i * LUU + c);
    }
  }
}

template <typename E, int K, int V>
static hipError_t launch_l0_intra(const L0IntraArgs& a, hipStream_t st) {
  const unsigned grid = (unsigned)(a.B * a.H * (a.nn > 0 ? a.nn : a.NT));
  hipLaunchKernelGGL((l0_intra_fwd_kernel<E, K, V>), dim3(grid), dim3(256), 0, st, a);
  return hipGetLastError();
}

hipError_t l0_intra_fwd(const L0IntraArgs& a, int dtype, int K, int V, hipStream_t st) {
#define NGDN_L0I(E, KK, VV) \
  if (K == KK && V == VV) return launch_l0_intra<E, KK, VV>(a, st);
  if (dtype == NGDN_BF16) {
    NGDN_L0I(bf16, 64, 64) NGDN_L0I(bf16, 64, 128) NGDN_L0I(bf16, 128, 64) NGDN_L0I(bf16, 128, 128)
  } else {
    NGDN_L0I(float, 64, 64) NGDN_L0I(float, 64, 128) NGDN_L0I(float, 128, 64) NGDN_L0I(float, 128, 128)
  }
#undef NGDN_L0I
  return hipErrorInvalidValue;
}

}  // namespace ngdn
