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
// The forward consumes W, U, Kt^T, Qg, Aqk; the reverse scan consumes the
// transposed copies Kt, W^T, Qg^T, Aqk^T, written when their pointers are set.
// Every output is fp32; for bf16 inputs the products run on bf16 MFMA with
// the derived operands split in two (ngdn_common.h).
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
__global__ __launch_bounds__(256) void l0_intra_fwd_kernel(L0IntraArgs a) {
  constexpr int C = CH;
  constexpr int LDX = C + 4;                 // fp32 rows of length C, 16-byte aligned
  constexpr int GL = K + GCP;
  const int NT = a.NT, H = a.H;
  const int n = blockIdx.x % NT;
  const int bh = blockIdx.x / NT;
  const int h = bh % H, b = bh / H;
  const int wv = wave_id(), tid = threadIdx.x;

  // LDS: gc, T (fp32, MFMA rows), then a region used first for A and the
  // inversion scratch, then for the transposed right-hand sides X, then for
  // the Kt^T / Qg^T staging.
  constexpr size_t SZ_GC = sizeof(float) * C * GL;
  constexpr size_t SZ_T = sizeof(float) * C * LDX;
  constexpr size_t SZ_AP = sizeof(float) * C * AT_LD + sizeof(float) * 3 * 16 * 17;
  constexpr size_t SZ_X = sizeof(float) * (K + V) * LDX;
  constexpr size_t SZ_R = SZ_AP > SZ_X ? SZ_AP : SZ_X;
  __shared__ __attribute__((aligned(16))) char smem[SZ_GC + SZ_T + SZ_R];
  float* s_gc = reinterpret_cast<float*>(smem);
  float* s_T = reinterpret_cast<float*>(smem + SZ_GC);
  char* region = smem + SZ_GC + SZ_T;
  float* s_A = reinterpret_cast<float*>(region);
  float* s_P = s_A + C * AT_LD;               // [3][16][17]
  float* s_X = reinterpret_cast<float*>(region);

  ChunkIn<E, K, V> in;
  in.init(a.q, a.k, a.v, a.g, a.b, a.w, b, h, n, a.T, H, a.L, a.scale);
  const size_t cix = (size_t)bh * NT + n;

  // ---- 1. in-chunk cumulative log decay
  l0_cumsum(s_gc, in);
  __syncthreads();

  // ---- 2. A and Aqk
  l0_build_A(s_A, s_gc, in, a.Aqk + cix * C * C, a.AqkT ? a.AqkT + cix * C * C : nullptr);
  __syncthreads();

  // ---- 3. T = (I + A)^-1
  l0_invert<LDX>(s_A, s_T, s_P);
  if (a.TT) {
    float* tt = a.TT + cix * C * C;
    for (int e = tid; e < C * C; e += 256) tt[e] = s_T[(e % C) * LDX + e / C];
  }

  // ---- 4. right-hand sides, transposed (s_A and s_P are dead)
  l0_build_X<E, K, V, LDX>(s_X, s_gc, in);
  __syncthreads();

  // ---- 5. W = T X_w, U = T X_u; wave w owns block-row w
  {
    const int I = wv;
    const int kd = tri_depth<E>(I);
    float* Wo = a.W + cix * C * K;
    float* Uo = a.U + cix * C * V;
    float* WTo = a.WT ? a.WT + cix * K * C : nullptr;
    for (int tc = 0; tc < (K + V) / 16; ++tc) {
      f4 acc = mma_tile<E>(f4_zero(), s_T + 16 * I * LDX, LDX, s_X + 16 * tc * LDX, LDX, kd);
      const int i0 = 16 * I + acc_row(0), col = 16 * tc + acc_col();
      if (col < K) {
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) Wo[(i0 + rr) * K + col] = acc[rr];
        if (WTo) *reinterpret_cast<f4*>(WTo + col * C + i0) = acc;
      } else {
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) Uo[(i0 + rr) * V + (col - K)] = acc[rr];
      }
    }
  }
  __syncthreads();

  // ---- 6. Kt (and its transpose), Qg (and its transpose), gam
  float* s_kt = s_X;             // reuse: [K][LDX]
  float* s_qg = s_X + K * LDX;   // [K][LDX]; fits since (K + V) >= 2 K when V >= K,
                                 // otherwise Qg^T goes straight to global below
  const bool qg_in_lds = V >= K;
  float* Qgo = a.Qg + cix * C * K;
  for (int e = tid; e < C * K; e += 256) {
    const int c = e / K, kk = e % K;
    const float gcv = s_gc[c * GL + kk];
    s_kt[kk * LDX + c] = in.K_(c, kk) * expf(s_gc[(C - 1) * GL + kk] - gcv);
    const float qg = in.Q_(c, kk) * in.scale * expf(gcv);
    Qgo[c * K + kk] = qg;
    if (qg_in_lds) s_qg[kk * LDX + c] = qg;
    else if (a.QgT) a.QgT[cix * K * C + kk * C + c] = qg;
  }
  if (tid < K) a.gam[cix * K + tid] = expf(s_gc[(C - 1) * GL + tid]);
  __syncthreads();
  {
    // rows of 64 as 16-byte vectors
    float* Ko = a.KtT + cix * K * C;
    float* QTo = a.QgT ? a.QgT + cix * K * C : nullptr;
    for (int e = tid; e < K * C / 4; e += 256) {
      const int kk = e / (C / 4), c = (e % (C / 4)) * 4;
      *reinterpret_cast<f4*>(Ko + kk * C + c) = *reinterpret_cast<const f4*>(s_kt + kk * LDX + c);
      if (QTo && qg_in_lds)
        *reinterpret_cast<f4*>(QTo + kk * C + c) = *reinterpret_cast<const f4*>(s_qg + kk * LDX + c);
    }
    if (a.Kt) {
      float* Kn = a.Kt + cix * C * K;
      for (int e = tid; e < C * K; e += 256) {
        const int c = e / K, kk = e % K;
        Kn[c * K + kk] = s_kt[kk * LDX + c];
      }
    }
  }
}

template <typename E, int K, int V>
static hipError_t launch_l0_intra(const L0IntraArgs& a, hipStream_t st) {
  const unsigned grid = (unsigned)(a.B * a.H * a.NT);
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
