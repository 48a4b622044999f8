// Backward of the reads and of the mix (ops/chunk.py:307-336 read_level_bwd,
// :423-449).
//
// dmix0_bwd: dmix_0[t] = <do[t], read_0[t]> with level 0's read stored by the
// forward.
// read_state_bwd, per (batch, group j, head) of one level l >= 1, over the
// group's chunks, with S = S_l[j] staged once and dO = mix_l do:
//   read_l = scale q_l S           -> dmix_l[t] = <do[t], read_l[t]>
//   dq_l   = scale dO S^T
//   dS_l[j] = scale sum_t q_l[t]^T dO[t]
#include "ngdn_kernels.h"

namespace ngdn {

template <typename E, int V>
__global__ __launch_bounds__(256) void dmix0_kernel(Dmix0Args a) {
  // one wave per 16 tokens of one head
  const int lane = lane_id();
  const size_t row0 = ((size_t)blockIdx.x * 4 + wave_id()) * 16;    // (b, t) * H + h rows
  const size_t rows = (size_t)a.B * a.T * a.H;
  const E* dob = static_cast<const E*>(a.dout);
  for (int q = 0; q < 16; ++q) {
    const size_t r = row0 + q;
    if (r >= rows) break;
    float s = 0.f;
    for (int v = lane; v < V; v += WAVE) s += to_f(dob[r * V + v]) * a.read0[r * V + v];
    s = wave_sum(s);
    if (lane == 0) a.dmix[r * a.L] = s;
  }
}

template <typename E, int K, int V>
__global__ __launch_bounds__(512) void read_state_bwd_kernel(ReadStateBwdArgs a) {
  // 8 waves: for the per-chunk products wave w owns row tile w % 4 and half
  // the columns (w / 4); the group's dS tiles are dealt round robin
  constexpr int NW = 8;
  constexpr int C = CH;
  constexpr int LDS = V + 4;                     // staged S rows (fp32)
  constexpr int LDQ = K + 16 / (int)sizeof(E);   // staged q rows (exact)
  constexpr int LDD = V + 16 / (int)sizeof(E);   // staged do rows (exact)
  constexpr int KT = K / 16, VT = V / 16;
  constexpr int VTH = VT / 2, KTH = KT / 2;      // column tiles per wave of read / dq
  constexpr int NDS = KT * VT / NW;              // dS tiles per wave
  constexpr int KS = Mma<E>::KS;
  static_assert(KT * VT % NW == 0 && VT % 2 == 0 && KT % 2 == 0, "tiles split over 8 waves");
  typedef typename Mma<E>::SFrag SF;
  __shared__ __attribute__((aligned(16))) float s_S[K * LDS];
  __shared__ __attribute__((aligned(16))) E s_q[C * LDQ];
  __shared__ __attribute__((aligned(16))) E s_do[C * LDD];
  __shared__ float s_mix[C], s_dm[C];

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
  E* dqb = static_cast<E*>(a.dq) + ((size_t)b * T * H + h) * L * K + (size_t)l * K;
  float* dmb = a.dmix + ((size_t)b * T * H + h) * L + l;

  stage_f32(s_S, LDS, a.states + (((size_t)b * NG + j) * H + h) * K * V, V, K, V);

  f4 acc[NDS];
#pragma unroll
  for (int x = 0; x < NDS; ++x) acc[x] = f4_zero();
  const int rt = wv % 4, half = wv / 4;
  const int ri = rt * 16 + (lane & 15);          // this wave's rows of the chunk
  const int n1 = min((j + 1) * a.f, NT);
  for (int n = j * a.f; n < n1; ++n) {
    const int t0 = n * C, nv = min(C, T - t0);
    stage_rows<E>(s_q, LDQ, qb + (size_t)t0 * rowQ, rowQ, C, K, nv);
    stage_rows<E>(s_do, LDD, db + (size_t)t0 * rowV, rowV, C, V, nv);
    if (tid < C) {
      s_mix[tid] = tid < nv ? to_f(mb[(size_t)(t0 + tid) * H * L]) : 0.f;
      s_dm[tid] = 0.f;
    }
    __syncthreads();

    // ---- read_l = q S on this wave's rows and half of V -> partial dmix_l
    {
      f4 rd[VTH];
#pragma unroll
      for (int y = 0; y < VTH; ++y) rd[y] = f4_zero();
#pragma unroll
      for (int s = 0; s < K / KS; ++s) {
        const int k0 = s * KS + kofs<E>(lane);
        const auto fa = Mma<E>::ld(s_q + ri * LDQ + k0);
#pragma unroll
        for (int y = 0; y < VTH; ++y)
          rd[y] = Mma<E>::mma(rd[y], fa,
                              gather_s<E>(s_S + k0 * LDS + (half * VTH + y) * 16 + (lane & 15), LDS));
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = rt * 16 + acc_row(r);
        float sm = 0.f;
#pragma unroll
        for (int y = 0; y < VTH; ++y) sm += to_f(s_do[i * LDD + (half * VTH + y) * 16 + acc_col()]) * rd[y][r];
        sm += __shfl_xor(sm, 1, WAVE);
        sm += __shfl_xor(sm, 2, WAVE);
        sm += __shfl_xor(sm, 4, WAVE);
        sm += __shfl_xor(sm, 8, WAVE);
        if ((lane & 15) == 0) atomicAdd(&s_dm[i], sm);
      }
    }
    // ---- dq_l = scale dO S^T on this wave's rows and half of K
    {
      f4 dq[KTH];
#pragma unroll
      for (int x = 0; x < KTH; ++x) dq[x] = f4_zero();
      const float m = s_mix[ri];
#pragma unroll
      for (int s = 0; s < V / KS; ++s) {
        const int v0 = s * KS + kofs<E>(lane);
        const SF fa = Mma<E>::makes([&](int e) { return to_f(s_do[ri * LDD + v0 + e]) * m; });
#pragma unroll
        for (int x = 0; x < KTH; ++x)
          dq[x] = Mma<E>::mma(dq[x], fa, Mma<E>::ld(s_S + ((half * KTH + x) * 16 + (lane & 15)) * LDS + v0));
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = rt * 16 + acc_row(r);
        if (i < nv) {
#pragma unroll
          for (int x = 0; x < KTH; ++x)
            dqb[(size_t)(t0 + i) * rowQ + (half * KTH + x) * 16 + acc_col()] = from_f<E>(dq[x][r] * a.scale);
        }
      }
    }
    // ---- dS += q^T dO: the reduction runs down the staged rows, fragments
    // gathered down columns
#pragma unroll
    for (int s = 0; s < C / KS; ++s) {
      const int r0 = s * KS + kofs<E>(lane);
#pragma unroll
      for (int x = 0; x < NDS; ++x) {
        const int g = wv + NW * x, kt = g / VT, vt = g % VT;
        const auto fa = gather_x<E>(s_q + r0 * LDQ + kt * 16 + (lane & 15), LDQ);
        const E* pd = s_do + r0 * LDD + vt * 16 + (lane & 15);
        const auto fb = Mma<E>::makes([&](int e) { return to_f(pd[e * LDD]) * s_mix[r0 + e]; });
        acc[x] = Mma<E>::mma(acc[x], fa, fb);
      }
    }
    __syncthreads();
    if (tid < nv) dmb[(size_t)(t0 + tid) * H * L] = s_dm[tid] * a.scale;
  }
  float* out = a.d_states + (((size_t)b * NG + j) * H + h) * K * V;
#pragma unroll
  for (int x = 0; x < NDS; ++x) {
    const int g = wv + NW * x, kt = g / VT, vt = g % VT;
#pragma unroll
    for (int r = 0; r < 4; ++r)
      out[(size_t)(kt * 16 + acc_row(r)) * V + vt * 16 + acc_col()] = acc[x][r] * a.scale;
  }
}

template <typename E, int V>
static hipError_t launch_dmix0(const Dmix0Args& a, hipStream_t st) {
  const size_t rows = (size_t)a.B * a.T * a.H;
  const unsigned grid = (unsigned)((rows + 63) / 64);
  hipLaunchKernelGGL((dmix0_kernel<E, V>), dim3(grid), dim3(256), 0, st, a);
  return hipGetLastError();
}

hipError_t dmix0_bwd(const Dmix0Args& a, int dtype, hipStream_t st) {
  if (a.V == 64) return dtype == NGDN_BF16 ? launch_dmix0<bf16, 64>(a, st) : launch_dmix0<float, 64>(a, st);
  if (a.V == 128) return dtype == NGDN_BF16 ? launch_dmix0<bf16, 128>(a, st) : launch_dmix0<float, 128>(a, st);
  return hipErrorInvalidValue;
}

template <typename E, int K, int V>
static hipError_t launch_read_state_bwd(const ReadStateBwdArgs& a, hipStream_t st) {
  const unsigned grid = (unsigned)(a.B * a.H * a.NG);
  hipLaunchKernelGGL((read_state_bwd_kernel<E, K, V>), dim3(grid), dim3(512), 0, st, a);
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
