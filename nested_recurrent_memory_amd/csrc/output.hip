// Output of the op for one (batch, head, chunk): level 0's read from its chunk
// terms, every upper level's read with the state its group started with, and
// the per-token mix, written once (ops/chunk.py:129-156 read_level and the
// accumulation at :250-251,285-286; ops/naive.py:376-390).
//   o = mix_0 (Qg h_n + Aqk Vn) + sum_{l>=1} mix_l (scale q_l) S_l[group]
// Each product is staged through LDS as [64 x kd] x [kd x V] and run on MFMA;
// wave w owns output rows 16w..16w+15.
#include "ngdn_kernels.h"

namespace ngdn {

template <typename E, int K, int V>
__global__ __launch_bounds__(256) void output_fwd_kernel(OutputArgs a) {
  constexpr int C = CH;
  constexpr int LD = K + 8;
  constexpr int CTV = V / 16;
  __shared__ __attribute__((aligned(16))) E s_A[C * LD];
  __shared__ __attribute__((aligned(16))) E s_B[V * LD];

  const int NT = a.NT, H = a.H, T = a.T, L = a.L;
  const int n = blockIdx.x % NT;
  const int bh = blockIdx.x / NT;
  const int h = bh % H, b = bh / H;
  const int t0 = n * C;
  const int nvalid = min(C, T - t0);
  const int lane = lane_id(), wv = wave_id(), tid = threadIdx.x;
  const size_t cix = ((size_t)bh * NT + n);

  const E* mixp = static_cast<const E*>(a.mix) + ((size_t)b * T * H + h) * L;
  auto mixw = [&](int i, int l) -> float {
    return i < nvalid ? to_f(mixp[(size_t)(t0 + i) * H * L + l]) : 0.f;
  };

  f4 out[CTV];
#pragma unroll
  for (int c = 0; c < CTV; ++c) out[c] = f4_zero();
  f4 acc[CTV];

  auto run = [&](int kd) {
#pragma unroll
    for (int c = 0; c < CTV; ++c)
      acc[c] = mma_tile<E>(acc[c], s_A + wv * 16 * LD, LD, s_B + c * 16 * LD, LD, kd);
  };
  auto fold = [&](int l, float sc) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = wv * 16 + acc_row(r);
      const float m = mixw(i, l) * sc;
#pragma unroll
      for (int c = 0; c < CTV; ++c) out[c][r] += m * acc[c][r];
      if (a.reads && i < nvalid) {
        float* rp = a.reads + ((((size_t)l * a.B + b) * T + t0 + i) * H + h) * V;
#pragma unroll
        for (int c = 0; c < CTV; ++c) rp[c * 16 + acc_col()] = acc[c][r] * sc;
      }
    }
  };

  // ---- level 0: Qg h
#pragma unroll
  for (int c = 0; c < CTV; ++c) acc[c] = f4_zero();
  {
    const E* Qg = static_cast<const E*>(a.Qg) + cix * C * K;
    const E* hT = static_cast<const E*>(a.hT) + cix * V * K;
    for (int e = tid; e < C * K; e += 256) s_A[(e / K) * LD + e % K] = Qg[e];
    for (int e = tid; e < V * K; e += 256) s_B[(e / K) * LD + e % K] = hT[e];
  }
  __syncthreads();
  run(K);
  __syncthreads();
  // ---- level 0: Aqk Vn
  {
    const E* Aq = static_cast<const E*>(a.Aqk) + cix * C * C;
    const E* vT = static_cast<const E*>(a.vnT) + cix * V * C;
    for (int e = tid; e < C * C; e += 256) s_A[(e / C) * LD + e % C] = Aq[e];
    for (int e = tid; e < V * C; e += 256) s_B[(e / C) * LD + e % C] = vT[e];
  }
  __syncthreads();
  run(C);
  fold(0, 1.f);
  __syncthreads();

  // ---- upper levels
  const E* qb = static_cast<const E*>(a.q) + ((size_t)b * T * H + h) * L * K;
  for (int l = 1; l < L; ++l) {
    const int grp = n / a.f[l];
    const float* S = a.states[l] + (((size_t)b * a.NGl[l] + grp) * H + h) * K * V;
    for (int e = tid; e < C * K; e += 256) {
      const int i = e / K, k = e % K;
      s_A[i * LD + k] = i < nvalid ? qb[(size_t)(t0 + i) * H * L * K + (size_t)l * K + k] : from_f<E>(0.f);
    }
    for (int e = tid; e < K * V; e += 256) {
      const int k = e / V, v = e % V;
      s_B[v * LD + k] = from_f<E>(S[e]);
    }
    __syncthreads();
#pragma unroll
    for (int c = 0; c < CTV; ++c) acc[c] = f4_zero();
    run(K);
    fold(l, a.scale);
    __syncthreads();
  }

  // ---- write o
  E* op = static_cast<E*>(a.o) + ((size_t)b * T * H + h) * V;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int i = wv * 16 + acc_row(r);
    if (i < nvalid) {
#pragma unroll
      for (int c = 0; c < CTV; ++c)
        op[(size_t)(t0 + i) * H * V + c * 16 + acc_col()] = from_f<E>(out[c][r]);
    }
  }
}

template <typename E, int K, int V>
static hipError_t launch_output(const OutputArgs& a, hipStream_t st) {
  const unsigned grid = (unsigned)(a.B * a.H * a.NT);
  hipLaunchKernelGGL((output_fwd_kernel<E, K, V>), dim3(grid), dim3(256), 0, st, a);
  return hipGetLastError();
}

hipError_t output_fwd(const OutputArgs& a, int dtype, int K, int V, hipStream_t st) {
#define NGDN_OU(E, KK, VV) \
  if (K == KK && V == VV) return launch_output<E, KK, VV>(a, st);
  if (dtype == NGDN_BF16) {
    NGDN_OU(bf16, 64, 64) NGDN_OU(bf16, 128, 128)
  } else {
    NGDN_OU(float, 64, 64) NGDN_OU(float, 128, 128)
  }
#undef NGDN_OU
  return hipErrorInvalidValue;
}

}  // namespace ngdn
