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
  // V / 8 lanes per (b, t, h) row, 8 consecutive values each (16-byte loads);
  // a wave takes U passes of 64 / (V / 8) rows with every load in flight
  // before the first dot product. Each row's sum: per lane in order, then a
  // butterfly over its lanes.
  constexpr int LPR = V / 8, RPW = WAVE / LPR, U = 4;
  const int lane = lane_id();
  const int sub = lane / LPR, c = (lane % LPR) * 8;
  const size_t rows = (size_t)a.B * a.T * a.H;
  const size_t base = ((size_t)blockIdx.x * 4 + wave_id()) * RPW * U;
  const E* dob = static_cast<const E*>(a.dout);
  float x[U][8], y[U][8];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const size_t r = base + (size_t)u * RPW + sub;
    if (r < rows) {
      if constexpr (std::is_same<E, float>::value) {
        const f4 x0 = *reinterpret_cast<const f4*>(dob + r * V + c);
        const f4 x1 = *reinterpret_cast<const f4*>(dob + r * V + c + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) { x[u][e] = x0[e]; x[u][e + 4] = x1[e]; }
      } else {
        ld_vals<E>(dob + r * V + c, x[u]);
      }
      const f4 y0 = *reinterpret_cast<const f4*>(a.read0 + r * V + c);
      const f4 y1 = *reinterpret_cast<const f4*>(a.read0 + r * V + c + 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) { y[u][e] = y0[e]; y[u][e + 4] = y1[e]; }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) x[u][e] = y[u][e] = 0.f;
    }
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) s += x[u][e] * y[u][e];
#pragma unroll
    for (int o = LPR / 2; o > 0; o >>= 1) s += __shfl_xor(s, o, WAVE);
    const size_t r = base + (size_t)u * RPW + sub;
    if (lane % LPR == 0 && r < rows) a.dmix[r * a.L] = s;
  }
}

template <typename E, int K, int V>
__global__ __launch_bounds__(512) void read_state_bwd_kernel(ReadStateBwdArgs a) {
  // Per (batch, group j, head), over the group's chunks, with S = S_l[j]:
  //   P = do S^T                        (one product, exact do x split S)
  //   dq_l = scale mix_l P,  dmix_l = scale rowsum(q_l * P)
  //                                     (= <do, scale q_l S>, without forming q_l S)
  //   dS_l += scale q_l^T (mix_l do)    (exact q^T x split (mix do)^T)
  // S is staged once as a split tile; each chunk stages do rows (exact),
  // q^T (exact) and (mix do)^T (split), so every fragment is a 16-byte read.
  // 8 waves: for P, wave w owns row tile w % 4 and half the K tiles (w / 4);
  // the group's dS tiles are dealt round robin.
  constexpr int NW = 8, NTH = 512;
  constexpr int C = CH;
  using ST = SplitTile<E>;
  constexpr int PE = 16 / (int)sizeof(E);        // exact elements per 16 bytes
  constexpr int LDS_ = V + ST::PAD;              // S rows [K][V] (split)
  constexpr int LDD = V + PE;                    // do rows [C][V] (exact)
  constexpr int LDQT = C + PE;                   // q^T rows [K][C] (exact)
  constexpr int LDDT = C + ST::PAD;              // (mix do)^T rows [V][C] (split)
  constexpr int KT = K / 16, VT = V / 16;
  constexpr int KTH = KT / 2;                    // K tiles per wave of P
  constexpr int NDS = KT * VT / NW;              // dS tiles per wave
  constexpr int KS = Mma<E>::KS;
  static_assert(KT * VT % NW == 0 && KT % 2 == 0, "tiles split over 8 waves");
  // fp32 inputs (a test-only path) read the do rows of P from global memory:
  // a staged copy would not fit next to the fp32 tiles
  constexpr bool STAGE_DO = !std::is_same<E, float>::value;
  __shared__ __attribute__((aligned(16))) typename ST::T s_s[ST::NPLANE * K * LDS_];
  __shared__ __attribute__((aligned(16))) typename ST::T s_dt[ST::NPLANE * V * LDDT];
  __shared__ __attribute__((aligned(16))) E s_do[STAGE_DO ? C * LDD : 4];
  __shared__ __attribute__((aligned(16))) E s_qt[K * LDQT];
  // bf16: the chunk's dq rows gather here and leave as 16-byte rows (fp32
  // stores them from the registers: its tiles leave no room)
  constexpr int LDQ = K + PE;
  __shared__ __attribute__((aligned(16))) E s_dq[STAGE_DO ? C * LDQ : 4];
  __shared__ float s_mix[C], s_dm[2 * C];   // dmix partials of the two halves of K
  const ST sS{s_s, K * LDS_}, sDT{s_dt, V * LDDT};

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

  stage_split<NTH, K, V>(sS, LDS_, a.states + (((size_t)b * NG + j) * H + h) * K * V, V);

  f4 acc[NDS];
#pragma unroll
  for (int x = 0; x < NDS; ++x) acc[x] = f4_zero();
  const int rt = wv % 4, half = wv / 4;
  const int ri = rt * 16 + (lane & 15);          // this wave's rows of the chunk
  const int n1 = min((j + 1) * a.f, NT);
  // The next chunk's rows (and the mix of its rows, kept raw until staging)
  // are read into registers while this chunk computes, then written to LDS
  // at the top of the next iteration.
  constexpr int QG = C * K / PE / NTH, DG = C * V / PE / NTH;   // 16-byte groups per thread
  static_assert(C * K / PE % NTH == 0 && C * V / PE % NTH == 0, "whole groups per thread");
  typedef E EV __attribute__((__vector_size__(16)));
  EV qv[QG], dv[DG];
  E mv[DG], mrow;
  auto fetch = [&](int n) {
    const int t0 = n * C, nv = min(C, T - t0);
#pragma unroll
    for (int u = 0; u < QG; ++u) {
      const int e = tid + NTH * u, i = e % C, c = (e / C) * PE;
      qv[u] = i < nv ? *reinterpret_cast<const EV*>(qb + (size_t)(t0 + i) * rowQ + c) : EV{};
    }
#pragma unroll
    for (int u = 0; u < DG; ++u) {
      const int e = tid + NTH * u, i = e % C, c = (e / C) * PE;
      dv[u] = i < nv ? *reinterpret_cast<const EV*>(db + (size_t)(t0 + i) * rowV + c) : EV{};
      mv[u] = i < nv ? mb[(size_t)(t0 + i) * H * L] : E(0.f);
    }
    mrow = tid < nv ? mb[(size_t)(t0 + min(tid, C - 1)) * H * L] : E(0.f);
  };
  // The fetched rows of chunk n into LDS.
  auto stage = [&]() {
#pragma unroll
    for (int u = 0; u < QG; ++u) {
      const int e = tid + NTH * u, i = e % C, c = (e / C) * PE;
#pragma unroll
      for (int x = 0; x < PE; ++x) s_qt[(c + x) * LDQT + i] = qv[u][x];
    }
#pragma unroll
    for (int u = 0; u < DG; ++u) {
      const int e = tid + NTH * u, i = e % C, c = (e / C) * PE;
      if constexpr (STAGE_DO) *reinterpret_cast<EV*>(s_do + i * LDD + c) = dv[u];
      const float m = to_f(mv[u]);
#pragma unroll
      for (int x = 0; x < PE; ++x) sDT.put1((c + x) * LDDT + i, to_f(dv[u][x]) * m);
    }
    if (tid < C) {
      s_mix[tid] = to_f(mrow);
      s_dm[tid] = s_dm[C + tid] = 0.f;
    }
  };
  // One chunk, its rows already staged; the next chunk's rows are fetched
  // at its start and staged at its end, so the loads and the stores in
  // between are counted within one iteration. FULL (every chunk but a
  // partial last one): the stores carry no row guards, so the compiler's
  // wait before the staging covers the fetch only, not the stores after it.
  auto chunk = [&](auto full_c, int n) {
    constexpr bool FULL = decltype(full_c)::value;
    const int t0 = n * C, nv = FULL ? C : min(C, T - t0);
    const bool more = n + 1 < n1;
    lds_barrier();
    if (more) fetch(n + 1);

    // ---- P = do S^T on this wave's rows and half of K; dq and partial dmix
    {
      f4 pp[KTH];
#pragma unroll
      for (int x = 0; x < KTH; ++x) pp[x] = f4_zero();
#pragma unroll
      for (int s = 0; s < V / KS; ++s) {
        const int v0 = s * KS + kofs<E>(lane);
        typename Mma<E>::Frag fa;
        if constexpr (STAGE_DO) fa = Mma<E>::ld(s_do + ri * LDD + v0);
        else fa = ri < nv ? Mma<E>::ld(db + (size_t)(t0 + ri) * rowV + v0) : Mma<E>::zero();
#pragma unroll
        for (int x = 0; x < KTH; ++x)
          pp[x] = Mma<E>::mma(pp[x], fa, sS.get(((half * KTH + x) * 16 + (lane & 15)) * LDS_ + v0));
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = rt * 16 + acc_row(r);
        const float m = s_mix[i] * a.scale;
        float sm = 0.f;
#pragma unroll
        for (int x = 0; x < KTH; ++x) {
          const int k = (half * KTH + x) * 16 + acc_col();
          sm += to_f(s_qt[k * LDQT + i]) * pp[x][r];
          if constexpr (STAGE_DO) s_dq[i * LDQ + k] = from_f<E>(pp[x][r] * m);
          else if (FULL || i < nv) dqb[(size_t)(t0 + i) * rowQ + k] = from_f<E>(pp[x][r] * m);
        }
        sm = row16_sum(sm);
        if ((lane & 15) == 0) s_dm[half * C + i] = sm;   // each slot has one writer
      }
    }
    // ---- dS += q^T (mix do): q^T rows exact, (mix do)^T rows split
#pragma unroll
    for (int s = 0; s < C / KS; ++s) {
      const int r0 = s * KS + kofs<E>(lane);
#pragma unroll
      for (int x = 0; x < NDS; ++x) {
        const int g = wv + NW * x, kt = g / VT, vt = g % VT;
        const auto fa = Mma<E>::ld(s_qt + (kt * 16 + (lane & 15)) * LDQT + r0);
        acc[x] = Mma<E>::mma(acc[x], fa, sDT.get((vt * 16 + (lane & 15)) * LDDT + r0));
      }
    }
    lds_barrier();
    // each thread reads its two dmix slots before its own staging clears them
    if (FULL ? tid < C : tid < nv) dmb[(size_t)(t0 + tid) * H * L] = (s_dm[tid] + s_dm[C + tid]) * a.scale;
    if constexpr (STAGE_DO) {
      constexpr int RG = K / PE;                 // 16-byte groups per dq row
      static_assert(C * RG % NTH == 0, "whole groups per thread");
#pragma unroll
      for (int u = 0; u < C * RG / NTH; ++u) {
        const int e = tid + NTH * u, i = e / RG, c = (e % RG) * PE;
        if (FULL || i < nv)
          *reinterpret_cast<EV*>(dqb + (size_t)(t0 + i) * rowQ + c) =
              *reinterpret_cast<const EV*>(s_dq + i * LDQ + c);
      }
    }
    if (more) stage();
  };
  const int n_full = min(n1, T / C);   // chunks [j f, n_full) are whole
  if (j * a.f < n1) {
    fetch(j * a.f);
    stage();
  }
  for (int n = j * a.f; n < n_full; ++n) chunk(std::true_type{}, n);
  for (int n = max(j * a.f, n_full); n < n1; ++n) chunk(std::false_type{}, n);
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
  const size_t per = (size_t)4 * (WAVE / (V / 8)) * 4;   // rows per workgroup
  const unsigned grid = (unsigned)((rows + per - 1) / per);
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
