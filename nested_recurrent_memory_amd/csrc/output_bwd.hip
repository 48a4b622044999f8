// Backward of the output and of the upper-level reads
// (nested_gdn2/ops/chunk.py:307-336 read_level_bwd, :423-449).
//
// output_bwd, per (batch, head, chunk):
//   read_0 = Qg h_n + Aqk Vn,  read_l = scale q_l S_l[group]   (recomputed)
//   dmix_l[t] = sum_v do[t][v] read_l[t][v]
//   dq_l      = scale (mix_l do) S_l[group]^T        (l >= 1)
// read_state_bwd, per (batch, group, head) of one level l >= 1:
//   dS_l[j] = scale sum_{t in group j} q_l[t]^T (mix_l[t] do[t])
#include "ngdn_kernels.h"

namespace ngdn {

template <typename E, int K, int V>
__global__ __launch_bounds__(256) void output_bwd_kernel(OutputBwdArgs ab) {
  const OutputArgs& a = ab.f;
  constexpr int C = CH;
  constexpr int LD = K + 4;
  constexpr int LDV = V + 4;
  constexpr int LDC = C + 4;
  constexpr int CTV = V / 16;
  constexpr int CTK = K / 16;
  constexpr int KS = Mma<E>::KS;
  constexpr int KPL = Mma<E>::KPL;
  constexpr int ROWS = V > K ? V : K;
  constexpr int LDM = LD > LDV ? (LD > LDC ? LD : LDC) : (LDV > LDC ? LDV : LDC);
  __shared__ __attribute__((aligned(16))) float s_B[ROWS * LDM];

  const int NT = a.NT, H = a.H, T = a.T, L = a.L;
  int n, bh;   // all chunks of one (batch, head) on one XCD: groups share states in its L2
  xcd_split(blockIdx.x, gridDim.x, NT, bh, n);
  const int h = bh % H, b = bh / H;
  const int t0 = n * C;
  const int nvalid = min(C, T - t0);
  const int lane = lane_id(), wv = wave_id();
  const size_t cix = ((size_t)bh * NT + n);
  const int ri = wv * 16 + (lane & 15);      // A-operand row of this lane
  const int rc = min(ri, nvalid - 1);        // a valid row to read in its place

  const E* mixp = static_cast<const E*>(a.mix) + ((size_t)b * T * H + h) * L;
  const E* dop = static_cast<const E*>(ab.dout) + ((size_t)b * T * H + h) * V;
  auto mixw = [&](int i, int l) -> float {
    return i < nvalid ? to_f(mixp[(size_t)(t0 + i) * H * L + l]) : 0.f;
  };
  auto dov = [&](int i, int v) -> float {
    return i < nvalid ? to_f(dop[(size_t)(t0 + i) * H * V + v]) : 0.f;
  };

  f4 acc[CTV];
  auto run = [&](const auto* arow, int ldb, int kd) {
    for (int k0 = 0; k0 < kd; k0 += KS) {
      const auto fa = Mma<E>::ld(arow + k0);
#pragma unroll
      for (int c = 0; c < CTV; ++c)
        acc[c] = Mma<E>::mma(acc[c], fa, Mma<E>::ld(s_B + (c * 16 + (lane & 15)) * ldb + kofs<E>(lane) + k0));
    }
  };
  // dmix[t, l] = sc * <do[t], acc[t]>; one lane group per row, no races
  auto dmix = [&](int l, float sc) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = wv * 16 + acc_row(r);
      float s = 0.f;
#pragma unroll
      for (int c = 0; c < CTV; ++c) s += dov(i, c * 16 + acc_col()) * acc[c][r];
      s += __shfl_xor(s, 1, WAVE);
      s += __shfl_xor(s, 2, WAVE);
      s += __shfl_xor(s, 4, WAVE);
      s += __shfl_xor(s, 8, WAVE);
      if ((lane & 15) == 0 && i < nvalid)
        ab.dmix[((size_t)b * T + t0 + i) * H * L + (size_t)h * L + l] = s * sc;
    }
  };

  // ---- level 0 read
#pragma unroll
  for (int c = 0; c < CTV; ++c) acc[c] = f4_zero();
  stage_f32(s_B, LD, a.hT + cix * V * K, K, V, K);
  __syncthreads();
  run(a.Qg + cix * C * K + (size_t)ri * K + kofs<E>(lane), LD, K);
  __syncthreads();
  stage_f32(s_B, LDC, a.vnT + cix * V * C, C, V, C);
  __syncthreads();
  run(a.Aqk + cix * C * C + (size_t)ri * C + kofs<E>(lane), LDC, C);
  dmix(0, 1.f);
  __syncthreads();

  // ---- upper levels
  const E* qrow = static_cast<const E*>(a.q) + ((size_t)b * T * H + h) * L * K +
                  (size_t)(t0 + rc) * H * L * K + kofs<E>(lane);
  const E* drow = dop + (size_t)(t0 + rc) * H * V + kofs<E>(lane);
  E* dqb = static_cast<E*>(ab.dq) + ((size_t)b * T * H + h) * L * K;
  for (int l = 1; l < L; ++l) {
    const int grp = n / a.f[l];
    const float* S = a.states[l] + (((size_t)b * a.NGl[l] + grp) * H + h) * K * V;
    stage_f32(s_B, LD, a.statesT[l] + (((size_t)b * a.NGl[l] + grp) * H + h) * V * K, K, V, K);
    __syncthreads();
#pragma unroll
    for (int c = 0; c < CTV; ++c) acc[c] = f4_zero();
    run(qrow + (size_t)l * K, LD, K);   // rows past the end repeat the last row; dmix drops them
    dmix(l, a.scale);
    __syncthreads();
    // dq_l = scale (mix_l do) S^T: A = mix_l do [C][V] (this wave's rows), Bt = S [K][V]
    stage_f32(s_B, LDV, S, V, K, V);
    const float m = ri < nvalid ? mixw(ri, l) : 0.f;
    typename Mma<E>::SFrag fa[V / KS];
#pragma unroll
    for (int s = 0; s < V / KS; ++s) {
      float x[KPL];
      ld_vals<E>(drow + s * KS, x);
      fa[s] = Mma<E>::makes([&](int e) { return x[e] * m; });
    }
    __syncthreads();
#pragma unroll
    for (int c = 0; c < CTK; ++c) {
      f4 d = f4_zero();
#pragma unroll
      for (int s = 0; s < V / KS; ++s)
        d = Mma<E>::mma(d, fa[s], Mma<E>::ld(s_B + (c * 16 + (lane & 15)) * LDV + kofs<E>(lane) + s * KS));
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = wv * 16 + acc_row(r);
        if (i < nvalid)
          dqb[(size_t)(t0 + i) * H * L * K + (size_t)l * K + c * 16 + acc_col()] =
              from_f<E>(d[r] * a.scale);
      }
    }
    __syncthreads();
  }
}

template <typename E, int K, int V>
__global__ __launch_bounds__(256) void read_state_bwd_kernel(ReadStateBwdArgs a) {
  constexpr int C = CH;
  constexpr int LDQ = K + 16 / (int)sizeof(E);   // staged q rows (exact)
  constexpr int LDD = V + 16 / (int)sizeof(E);   // staged do rows (exact)
  constexpr int KT = K / 16, VT = V / 16;
  constexpr int KTW = KT / 4;                   // k-tiles per wave (all v-tiles each)
  constexpr int KS = Mma<E>::KS;
  static_assert(KT % 4 == 0, "K must split over the 4 waves");
  __shared__ __attribute__((aligned(16))) E s_q[C * LDQ];
  __shared__ __attribute__((aligned(16))) E s_do[C * LDD];
  __shared__ float s_mix[C];

  const int NG = a.NG, H = a.H, T = a.T, L = a.L, l = a.level;
  const int j = blockIdx.x % NG;
  const int bh = blockIdx.x / NG;
  const int h = bh % H, b = bh / H;
  const int lane = lane_id(), wv = wave_id(), tid = threadIdx.x;
  const int NT = (T + C - 1) / C;
  const size_t rowQ = (size_t)H * L * K, rowV = (size_t)H * V;
  const E* qb = static_cast<const E*>(a.q) + ((size_t)b * T * H + h) * L * K + (size_t)l * K;
  const E* mb = static_cast<const E*>(a.mix) + ((size_t)b * T * H + h) * L + l;
  const E* db = static_cast<const E*>(a.dout) + ((size_t)b * T * H + h) * V;

  // dS[k][v] = sum_t q[t][k] (mix[t] do[t][v]): the reduction runs down the
  // staged rows; fragments are gathered down columns
  f4 acc[KTW][VT];
#pragma unroll
  for (int x = 0; x < KTW; ++x)
#pragma unroll
    for (int y = 0; y < VT; ++y) acc[x][y] = f4_zero();
  const int n1 = min((j + 1) * a.f, NT);
  for (int n = j * a.f; n < n1; ++n) {
    const int t0 = n * C, nv = min(C, T - t0);
    stage_rows<E>(s_q, LDQ, qb + (size_t)t0 * rowQ, rowQ, C, K, nv);
    stage_rows<E>(s_do, LDD, db + (size_t)t0 * rowV, rowV, C, V, nv);
    if (tid < C) s_mix[tid] = tid < nv ? to_f(mb[(size_t)(t0 + tid) * H * L]) : 0.f;
    __syncthreads();
#pragma unroll
    for (int s = 0; s < C / KS; ++s) {
      const int r0 = s * KS + kofs<E>(lane);
      typename Mma<E>::Frag fa[KTW];
#pragma unroll
      for (int x = 0; x < KTW; ++x)
        fa[x] = gather_x<E>(s_q + r0 * LDQ + (wv * KTW + x) * 16 + (lane & 15), LDQ);
#pragma unroll
      for (int y = 0; y < VT; ++y) {
        const E* pd = s_do + r0 * LDD + y * 16 + (lane & 15);
        const auto fb = Mma<E>::makes([&](int e) { return to_f(pd[e * LDD]) * s_mix[r0 + e]; });
#pragma unroll
        for (int x = 0; x < KTW; ++x) acc[x][y] = Mma<E>::mma(acc[x][y], fa[x], fb);
      }
    }
    __syncthreads();
  }
  float* out = a.d_states + (((size_t)b * NG + j) * H + h) * K * V;
#pragma unroll
  for (int x = 0; x < KTW; ++x)
#pragma unroll
    for (int y = 0; y < VT; ++y)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        out[(size_t)((wv * KTW + x) * 16 + acc_row(r)) * V + y * 16 + acc_col()] = acc[x][y][r] * a.scale;
}

template <typename E, int K, int V>
static hipError_t launch_output_bwd(const OutputBwdArgs& a, hipStream_t st) {
  const unsigned grid = (unsigned)(a.f.B * a.f.H * a.f.NT);
  hipLaunchKernelGGL((output_bwd_kernel<E, K, V>), dim3(grid), dim3(256), 0, st, a);
  return hipGetLastError();
}

hipError_t output_bwd(const OutputBwdArgs& a, int dtype, int K, int V, hipStream_t st) {
#define NGDN_OB(E, KK, VV) \
  if (K == KK && V == VV) return launch_output_bwd<E, KK, VV>(a, st);
  if (dtype == NGDN_BF16) {
    NGDN_OB(bf16, 64, 64) NGDN_OB(bf16, 128, 128)
  } else {
    NGDN_OB(float, 64, 64) NGDN_OB(float, 128, 128)
  }
#undef NGDN_OB
  return hipErrorInvalidValue;
}

template <typename E, int K, int V>
static hipError_t launch_read_state_bwd(const ReadStateBwdArgs& a, hipStream_t st) {
  const unsigned grid = (unsigned)(a.B * a.H * a.NG);
  hipLaunchKernelGGL((read_state_bwd_kernel<E, K, V>), dim3(grid), dim3(256), 0, st, a);
  return hipGetLastError();
}

hipError_t read_state_bwd(const ReadStateBwdArgs& a, int dtype, int K, int V, hipStream_t st) {
#define NGDN_RS(E, KK, VV) \
  if (K == KK && V == VV) return launch_read_state_bwd<E, KK, VV>(a, st);
  if (dtype == NGDN_BF16) {
    NGDN_RS(bf16, 64, 64) NGDN_RS(bf16, 128, 128)
  } else {
    NGDN_RS(float, 64, 64) NGDN_RS(float, 128, 128)
  }
#undef NGDN_RS
  return hipErrorInvalidValue;
}

}  // namespace ngdn
