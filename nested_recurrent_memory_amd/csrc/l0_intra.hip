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
//   Kt_i = k_i * e^(gc_last - gc_i)                      (stored transposed)
//   Qg   = scale * q0 * e^gc
//   Aqk  = sum_k scale q_i k_j e^(gc_i - gc_j)            j <= i
//   gam  = e^gc_last
//
// One workgroup (4 waves) per (batch, head, chunk). Decay products are formed
// without overflow: inside block-row I (16 rows starting at r = 16 I) every
// pair uses r as the reference point, e^(gc_i - gc_j) = e^(gc_i - gc_r) e^(gc_r - gc_j).
// Both factors are <= 1 for j < r; on the diagonal block the right factor is
// e^(decay over at most 15 tokens), and when that could leave fp32 range
// (more than 80 nats in some channel) the diagonal tile is recomputed pair by
// pair with clamped exponents, exactly as the reference does.
#include "ngdn_kernels.h"

namespace ngdn {

template <typename E, int K, int V>
__global__ __launch_bounds__(256) void l0_intra_fwd_kernel(L0IntraArgs a) {
  constexpr int C = CH;
  constexpr int LDX = C + 8;                 // k-contiguous rows of length C
  const int NT = a.NT, H = a.H, T = a.T;
  const int n = blockIdx.x % NT;
  const int bh = blockIdx.x / NT;
  const int h = bh % H, b = bh / H;
  const int t0 = n * C;
  const int lane = lane_id(), wv = wave_id(), tid = threadIdx.x;

  // LDS: gc (fp32), then a region used first for A/T (fp32), then for the
  // transposed right-hand sides X (E), then for Kt^T (E); T in E.
  constexpr int GC_LD = K + 1;
  constexpr int AT_LD = C + 1;
  constexpr size_t SZ_GC = sizeof(float) * C * GC_LD;
  constexpr size_t SZ_AT = sizeof(float) * 2 * C * AT_LD + sizeof(float) * 3 * 16 * 17;
  constexpr size_t SZ_X = sizeof(E) * (K + V) * LDX;
  constexpr size_t SZ_R = SZ_AT > SZ_X ? SZ_AT : SZ_X;
  constexpr size_t SZ_TE = sizeof(E) * C * LDX;
  __shared__ __attribute__((aligned(16))) char smem[SZ_GC + SZ_R + SZ_TE];
  float* s_gc = reinterpret_cast<float*>(smem);
  char* region = smem + SZ_GC;
  float* s_A = reinterpret_cast<float*>(region);
  float* s_T = s_A + C * AT_LD;
  float* s_P = s_T + C * AT_LD;               // [3][16][17]
  E* s_X = reinterpret_cast<E*>(region);
  E* s_TE = reinterpret_cast<E*>(smem + SZ_GC + SZ_R);

  const size_t rowK = (size_t)H * K;          // token stride of k, b, g
  const size_t rowV = (size_t)H * V;          // token stride of v, w
  const size_t rowQ = (size_t)H * a.L * K;    // token stride of q
  const E* qp = static_cast<const E*>(a.q) + ((size_t)b * T * H + h) * a.L * K;
  const E* kp = static_cast<const E*>(a.k) + ((size_t)b * T * H + h) * K;
  const E* bp = static_cast<const E*>(a.b) + ((size_t)b * T * H + h) * K;
  const E* vp = static_cast<const E*>(a.v) + ((size_t)b * T * H + h) * V;
  const E* wp = static_cast<const E*>(a.w) + ((size_t)b * T * H + h) * V;
  const float* gp = a.g + ((size_t)b * T * H + h) * K;
  const int nvalid = min(C, T - t0);           // rows past T are zero padding

  // ---- 1. in-chunk cumulative log decay
  if (tid < K) {
    float acc = 0.f;
    for (int i = 0; i < C; ++i) {
      if (i < nvalid) acc += gp[(size_t)(t0 + i) * rowK + tid];
      s_gc[i * GC_LD + tid] = acc;
    }
  }
  __syncthreads();

  auto ld = [&](const E* base, size_t stride, int i, int c) -> float {
    return i < nvalid ? to_f(base[(size_t)(t0 + i) * stride + c]) : 0.f;
  };

  // ---- 2. A and Aqk, wave w owns block-row I = w
  {
    const int I = wv, r = 16 * I;
    typedef typename Mma<E>::Frag Frag;
    constexpr int NKS = K / Mma<E>::KS;
    // largest decay across the 16 rows of this block, any channel
    float dmax = 0.f;
    for (int e = lane; e < 16 * K; e += WAVE) {
      const int j = r + e / K, c = e % K;
      dmax = fmaxf(dmax, s_gc[r * GC_LD + c] - s_gc[j * GC_LD + c]);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) dmax = fmaxf(dmax, __shfl_xor(dmax, o, WAVE));
    const bool safe = dmax <= 80.f;

    Frag lf[NKS], qf[NKS];
    const int ri = r + (lane & 15);
#pragma unroll
    for (int s = 0; s < NKS; ++s) {
      const int c0 = s * Mma<E>::KS + kofs<E>(lane);
      lf[s] = Mma<E>::make([&](int e) {
        const int c = c0 + e;
        const float d = expf(s_gc[ri * GC_LD + c] - s_gc[r * GC_LD + c]);
        return ld(bp, rowK, ri, c) * ld(kp, rowK, ri, c) * d;
      });
      qf[s] = Mma<E>::make([&](int e) {
        const int c = c0 + e;
        const float d = expf(s_gc[ri * GC_LD + c] - s_gc[r * GC_LD + c]);
        return ld(qp, rowQ, ri, c) * a.scale * d;
      });
    }
    E* aqk = static_cast<E*>(a.Aqk) + (((size_t)b * H + h) * NT + n) * C * C;
    for (int J = 0; J < 4; ++J) {
      f4 accA = f4_zero(), accQ = f4_zero();
      if (J <= I) {
        const int rj = 16 * J + (lane & 15);
#pragma unroll
        for (int s = 0; s < NKS; ++s) {
          const int c0 = s * Mma<E>::KS + kofs<E>(lane);
          Frag kf = Mma<E>::make([&](int e) {
            const int c = c0 + e;
            const float x = s_gc[r * GC_LD + c] - s_gc[rj * GC_LD + c];
            return ld(kp, rowK, rj, c) * expf(J < I ? x : fminf(x, 88.f));
          });
          accA = Mma<E>::mma(accA, lf[s], kf);
          accQ = Mma<E>::mma(accQ, qf[s], kf);
        }
        if (J == I && !safe) {
          // exact pairwise form for this diagonal tile
#pragma unroll
          for (int rr = 0; rr < 4; ++rr) {
            const int i = r + acc_row(rr), j = 16 * J + acc_col();
            float sa = 0.f, sq = 0.f;
            if (j <= i) {
              for (int c = 0; c < K; ++c) {
                const float d = expf(fminf(s_gc[i * GC_LD + c] - s_gc[j * GC_LD + c], 0.f));
                const float kj = ld(kp, rowK, j, c);
                sa += ld(bp, rowK, i, c) * ld(kp, rowK, i, c) * kj * d;
                sq += ld(qp, rowQ, i, c) * kj * d;
              }
            }
            accA[rr] = sa;
            accQ[rr] = sq * a.scale;
          }
        }
      }
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int i = r + acc_row(rr), j = 16 * J + acc_col();
        s_A[i * AT_LD + j] = (j < i) ? accA[rr] : 0.f;
        aqk[i * C + j] = from_f<E>((j <= i) ? accQ[rr] : 0.f);
      }
    }
  }
  __syncthreads();

  // ---- 3. T = (I + A)^-1, by 16-row blocks
  if (wv == 0) {
    // diagonal blocks: lane = (block, column), forward substitution
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
    for (int i = 0; i < 16; ++i) s_T[(o + i) * AT_LD + o + c] = t[i];
  } else {
    // zero everything off the diagonal blocks; lower blocks are filled below
    for (int e = tid - WAVE; e < C * C; e += 3 * WAVE) {
      const int i = e / C, j = e % C;
      if ((i >> 4) != (j >> 4)) s_T[i * AT_LD + j] = 0.f;
    }
  }
  __syncthreads();
  for (int d = 1; d < 4; ++d) {
    const int nb = 4 - d;   // blocks (I, I-d), I = d..3
    // P_IJ = sum_{M=J}^{I-1} A_IM T_MJ
    for (int e = tid; e < nb * 256; e += 256) {
      const int blk = e >> 8, i = (e >> 4) & 15, j = e & 15;
      const int I = d + blk, J = I - d;
      float acc = 0.f;
      for (int m = 16 * J; m < 16 * I; ++m)
        acc += s_A[(16 * I + i) * AT_LD + m] * s_T[m * AT_LD + 16 * J + j];
      s_P[blk * 272 + i * 17 + j] = acc;
    }
    __syncthreads();
    // T_IJ = -T_II P_IJ
    for (int e = tid; e < nb * 256; e += 256) {
      const int blk = e >> 8, i = (e >> 4) & 15, j = e & 15;
      const int I = d + blk, J = I - d;
      float acc = 0.f;
#pragma unroll
      for (int m = 0; m < 16; ++m)
        acc += s_T[(16 * I + i) * AT_LD + 16 * I + m] * s_P[blk * 272 + m * 17 + j];
      s_T[(16 * I + i) * AT_LD + 16 * J + j] = -acc;
    }
    __syncthreads();
  }
  for (int e = tid; e < C * C; e += 256) {
    const int i = e / C, j = e % C;
    s_TE[i * LDX + j] = from_f<E>(s_T[i * AT_LD + j]);
  }
  __syncthreads();

  // ---- 4. right-hand sides, transposed: X[k][c] = b k e^gc, X[K+v][c] = w v
  for (int e = tid; e < C * K; e += 256) {
    const int c = e / K, kk = e % K;
    const float x = ld(bp, rowK, c, kk) * ld(kp, rowK, c, kk) * expf(s_gc[c * GC_LD + kk]);
    s_X[kk * LDX + c] = from_f<E>(x);
  }
  for (int e = tid; e < C * V; e += 256) {
    const int c = e / V, vv = e % V;
    s_X[(K + vv) * LDX + c] = from_f<E>(ld(wp, rowV, c, vv) * ld(vp, rowV, c, vv));
  }
  __syncthreads();

  // ---- 5. W = T X_w, U = T X_u; wave w owns block-row w
  {
    const int I = wv;
    const int kd = min(C, ((16 * (I + 1) + Mma<E>::KS - 1) / Mma<E>::KS) * Mma<E>::KS);
    E* Wo = static_cast<E*>(a.W) + (((size_t)b * H + h) * NT + n) * C * K;
    E* Uo = static_cast<E*>(a.U) + (((size_t)b * H + h) * NT + n) * C * V;
    for (int tc = 0; tc < (K + V) / 16; ++tc) {
      f4 acc = mma_tile<E>(f4_zero(), s_TE + 16 * I * LDX, LDX, s_X + 16 * tc * LDX, LDX, kd);
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int i = 16 * I + acc_row(rr), col = 16 * tc + acc_col();
        if (col < K) Wo[i * K + col] = from_f<E>(acc[rr]);
        else Uo[i * V + (col - K)] = from_f<E>(acc[rr]);
      }
    }
  }
  __syncthreads();

  // ---- 6. Kt^T, Qg, gam
  E* s_kt = s_X;   // reuse: [K][LDX]
  for (int e = tid; e < C * K; e += 256) {
    const int c = e / K, kk = e % K;
    const float x = ld(kp, rowK, c, kk) * expf(s_gc[(C - 1) * GC_LD + kk] - s_gc[c * GC_LD + kk]);
    s_kt[kk * LDX + c] = from_f<E>(x);
  }
  {
    E* Qo = static_cast<E*>(a.Qg) + (((size_t)b * H + h) * NT + n) * C * K;
    for (int e = tid; e < C * K; e += 256) {
      const int c = e / K, kk = e % K;
      Qo[c * K + kk] = from_f<E>(ld(qp, rowQ, c, kk) * a.scale * expf(s_gc[c * GC_LD + kk]));
    }
    if (tid < K)
      a.gam[(((size_t)b * H + h) * NT + n) * K + tid] = expf(s_gc[(C - 1) * GC_LD + tid]);
  }
  __syncthreads();
  {
    E* Ko = static_cast<E*>(a.KtT) + (((size_t)b * H + h) * NT + n) * K * C;
    for (int e = tid; e < K * C; e += 256) {
      const int kk = e / C, c = e % C;
      Ko[kk * C + c] = s_kt[kk * LDX + c];
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
