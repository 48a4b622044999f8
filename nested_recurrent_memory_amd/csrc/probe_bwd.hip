// Backward of one level's firings: through the update step and the probe.
//
// Update step (ops/update_bwd.py:115-158), with s = e^g * S_j (S_j the state
// entering group j), kb = keys * b, vn = vals * w - kb s and, from the reverse
// scan, dS' (gradient of the state after the firing) and dvn = keys dS':
//   P = dvn s^T,  Q = vn dS'^T
//   dkeys = Q - P * b,   db = -P * keys,   dvals = dvn * w,   dw = dvn * vals
//   dg_k  = sum_v dS'[k][v] s[k][v] - sum_n kb[n][k] P[n][k]
// Probe (ops/probe.py:59-102; the reference differentiates it by autograd
// replay, ops/chunk.py:339-371,486-517):
//   du    = (dkeys - keys <keys, dkeys>) / max(|u|, 1e-12)
//   dxb   = db * b (1 - b),  dxw = dw * w (1 - w),
//   dxg   = -(dg / N) * sigmoid(xg - 4)
//   dVals += du Wk + dxb Bp^T + dxw Wp^T + dxg Gp^T
//   dS_below = Bank^T dVals (learned) or dVals (merge),
//   dBank   += dVals S_below^T
// Parameter gradients other than the bank are reduced afterwards over all
// firings of a head (atb_accumulate) from the fp32 workspace written here.
#include "ngdn_kernels.h"

namespace ngdn {

template <typename E, int K, int N, bool MERGE>
__global__ __launch_bounds__(256) void probe_bwd_kernel(ProbeBwdArgs ab) {
  const ProbeArgs& a = ab.f;
  constexpr int V = K;
  constexpr int LD = K + 4;                        // fp32 rows
  constexpr int LDN = N + 4;
  constexpr int NTK = (N / 16) * (K / 16) / 4;     // [N,K] (= [N,V]) tiles per wave
  constexpr int KS = Mma<E>::KS;
  constexpr int NKS = K / KS;
  constexpr int NR1 = V * (LD > LDN ? LD : LDN);
  constexpr int RX = N > K ? N : K;
  typedef typename Mma<E>::SFrag SF;
  __shared__ __attribute__((aligned(16))) float s_R1[NR1];     // S^T, then s^T, then dVals^T
  __shared__ __attribute__((aligned(16))) float s_X[RX * LD];  // kb, then vn, then S_below
  __shared__ float s_nrm[N], s_rd[N], s_gs[K], s_dg[K];

  const int NF = a.NF, H = a.H;
  const int i = blockIdx.x % NF;
  const int bh = blockIdx.x / NF;
  const int h = bh % H, b = bh / H;
  const int lane = lane_id(), wv = wave_id(), tid = threadIdx.x;
  const size_t fo = (size_t)bh * NF + i;

  // ---- the gathered lower state (as in probe_fwd)
  const int src = ((i + 1) * a.f_here) / a.f_below;
  const bool fin = src >= a.NGb;
  const float* Sf = nullptr;    // [K][V]
  const float* Sh = nullptr;    // [V][K] (level-0 chunk states)
  if (fin) Sf = a.below_fin + b * a.bf_sb + h * a.bf_sh;
  else if (a.below_mode == 1) Sf = a.below + (((size_t)b * a.NGb + src) * H + h) * K * V;
  else Sh = a.below + (((size_t)b * H + h) * a.NGb + src) * V * K;
  auto sbelow = [&](int k, int v) -> float { return Sh ? Sh[(size_t)v * K + k] : Sf[(size_t)k * V + v]; };

  const float* Sj = ab.Sg + (((size_t)b * ab.NG + i) * H + h) * K * V;   // state before firing i
  const float* dSp = ab.dSp + fo * K * V;
  const float* dvn = ab.dvn + fo * N * V;
  float* wsV = ab.wsV + fo * N * V;
  float* wsdu = ab.wsdu + fo * N * K;
  float* wsdxb = ab.wsdxb + fo * N * K;
  float* wsdxg = ab.wsdxg + fo * N * K;
  float* wsdxw = ab.wsdxw + fo * N * V;
  float* wsdV = ab.wsdV + fo * N * V;

  for (int e = tid; e < N; e += 256) { s_nrm[e] = 0.f; s_rd[e] = 0.f; }
  for (int e = tid; e < K; e += 256) { s_gs[e] = 0.f; s_dg[e] = 0.f; }

  // ---- A. Vals
  if (!MERGE) {
    if (Sh) {
      stage_f32(s_R1, LD, Sh, K, V, K);
    } else {
      stage_state_T<K, V>(s_R1, LD, Sf);
    }
    __syncthreads();
    const E* bank = static_cast<const E*>(a.bank) + (size_t)h * a.Nmax * K;
#pragma unroll
    for (int t = 0; t < NTK; ++t) {
      const int g = wv + 4 * t, rt = g / (V / 16), ct = g % (V / 16);
      f4 acc = mma_tile<E>(f4_zero(), bank + rt * 16 * K, K, s_R1 + ct * 16 * LD, LD, K);
#pragma unroll
      for (int r = 0; r < 4; ++r)
        wsV[(rt * 16 + acc_row(r)) * V + ct * 16 + acc_col()] = acc[r];
    }
  } else {
    for (int e = tid; e < K * V; e += 256) wsV[e] = sbelow(e / V, e % V);
  }
  __syncthreads();

  // projections of Vals: A rows from the workspace, B rows from global params
  auto proj = [&](const void* P, int rt, int ct) -> f4 {
    const E* Pt = static_cast<const E*>(P) + (size_t)h * K * V;
    return mma_tile<E>(f4_zero(), wsV + rt * 16 * V, V, Pt + (size_t)ct * 16 * V, V, V);
  };

  // ---- B. decay and key norms
#pragma unroll
  for (int t = 0; t < NTK; ++t) {
    const int g = wv + 4 * t, rt = g / (K / 16), ct = g % (K / 16);
    f4 x = proj(a.gpT, rt, ct);
    float s = 0.f;
#pragma unroll
    for (int r = 0; r < 4; ++r) s += softplusf_(x[r] - 4.f);
    s += __shfl_xor(s, 16, WAVE);
    s += __shfl_xor(s, 32, WAVE);
    if (lane < 16) atomicAdd(&s_gs[ct * 16 + lane], s);
    if (!MERGE) {
      f4 u = proj(a.kp, rt, ct);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float q = u[r] * u[r];
        q += __shfl_xor(q, 1, WAVE);
        q += __shfl_xor(q, 2, WAVE);
        q += __shfl_xor(q, 4, WAVE);
        q += __shfl_xor(q, 8, WAVE);
        if ((lane & 15) == 0) atomicAdd(&s_nrm[rt * 16 + acc_row(r)], q);
      }
    }
  }
  __syncthreads();
  auto gam = [&](int k) { return expf(-s_gs[k] / (float)N); };
  auto keyval = [&](const f4& u, int rt, int ct, int r) -> float {
    const int n = rt * 16 + acc_row(r), k = ct * 16 + acc_col();
    if (MERGE) return n == k ? 1.f : 0.f;
    return u[r] / fmaxf(sqrtf(s_nrm[n]), 1e-12f);
  };

  // ---- C. s^T into LDS, kb into LDS
  for (int e = tid; e < K * V; e += 256) {
    const int k = e / V, v = e % V;
    s_R1[v * LD + k] = gam(k) * Sj[e];
  }
#pragma unroll
  for (int t = 0; t < NTK; ++t) {
    const int g = wv + 4 * t, rt = g / (K / 16), ct = g % (K / 16);
    f4 u = f4_zero();
    if (!MERGE) u = proj(a.kp, rt, ct);
    f4 xb = proj(a.bpT, rt, ct);
#pragma unroll
    for (int r = 0; r < 4; ++r)
      s_X[(rt * 16 + acc_row(r)) * LD + ct * 16 + acc_col()] =
          keyval(u, rt, ct, r) * sigmoidf_(xb[r] - 4.f);
  }
  __syncthreads();
  // vn = vals * w - kb s;  dw-side terms
  f4 vnt[NTK], dvd[NTK];
#pragma unroll
  for (int t = 0; t < NTK; ++t) {
    const int g = wv + 4 * t, rt = g / (V / 16), ct = g % (V / 16);
    f4 ks = mma_tile<E>(f4_zero(), s_X + rt * 16 * LD, LD, s_R1 + ct * 16 * LD, LD, K);
    f4 xw = proj(a.wpT, rt, ct);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int n = rt * 16 + acc_row(r), v = ct * 16 + acc_col();
      const float w = sigmoidf_(xw[r]);
      const float val = wsV[n * V + v];
      const float dv = dvn[n * V + v];
      vnt[t][r] = val * w - ks[r];
      dvd[t][r] = dv * w;
      wsdxw[n * V + v] = dv * val * w * (1.f - w);
    }
  }
  __syncthreads();
#pragma unroll
  for (int t = 0; t < NTK; ++t) {
    const int g = wv + 4 * t, rt = g / (V / 16), ct = g % (V / 16);
#pragma unroll
    for (int r = 0; r < 4; ++r)
      s_X[(rt * 16 + acc_row(r)) * LD + ct * 16 + acc_col()] = vnt[t][r];
  }
  __syncthreads();

  // ---- D. P = dvn s^T, Q = vn dS'^T; dkeys, db, the decay gradient
  f4 dkt[NTK];
#pragma unroll
  for (int t = 0; t < NTK; ++t) {
    const int g = wv + 4 * t, rt = g / (K / 16), ct = g % (K / 16);
    const int kc = ct * 16 + (lane & 15);
    const float gk = gam(kc);
    f4 P = f4_zero(), Q = f4_zero();
    const float* drow = dvn + (size_t)(rt * 16 + (lane & 15)) * V;
    const float* srow = Sj + (size_t)kc * V;
    const float* qrow = dSp + (size_t)kc * V;
#pragma unroll
    for (int s = 0; s < NKS; ++s) {
      const int v0 = s * KS + kofs<E>(lane);
      const SF fa = Mma<E>::ld(drow + v0);
      const SF fs = Mma<E>::makes([&](int e) { return gk * srow[v0 + e]; });
      const SF fv = Mma<E>::ld(s_X + (rt * 16 + (lane & 15)) * LD + v0);
      const SF fq = Mma<E>::ld(qrow + v0);
      P = Mma<E>::mma(P, fa, fs);
      Q = Mma<E>::mma(Q, fv, fq);
    }
    f4 u = f4_zero();
    if (!MERGE) u = proj(a.kp, rt, ct);
    f4 xb = proj(a.bpT, rt, ct);
    float cs = 0.f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int n = rt * 16 + acc_row(r), k = ct * 16 + acc_col();
      const float key = keyval(u, rt, ct, r), bb = sigmoidf_(xb[r] - 4.f);
      const float dkey = Q[r] - P[r] * bb;
      const float dbg = -P[r] * key;
      cs += key * bb * P[r];
      dkt[t][r] = dkey;
      wsdxb[n * K + k] = dbg * bb * (1.f - bb);
      if (!MERGE) {
        float rd = key * dkey;
        rd += __shfl_xor(rd, 1, WAVE);
        rd += __shfl_xor(rd, 2, WAVE);
        rd += __shfl_xor(rd, 4, WAVE);
        rd += __shfl_xor(rd, 8, WAVE);
        if ((lane & 15) == 0) atomicAdd(&s_rd[n], rd);
      }
    }
    cs += __shfl_xor(cs, 16, WAVE);
    cs += __shfl_xor(cs, 32, WAVE);
    if (lane < 16) atomicAdd(&s_dg[ct * 16 + lane], -cs);
  }
  // + sum_v dS'[k][v] s[k][v]
  for (int k = wv; k < K; k += 4) {
    float s = 0.f;
    for (int v = lane; v < V; v += WAVE) s += dSp[(size_t)k * V + v] * Sj[(size_t)k * V + v];
    s = wave_sum(s);
    if (lane == 0) atomicAdd(&s_dg[k], gam(k) * s);
  }
  __syncthreads();

  // ---- D2. du and dxg
#pragma unroll
  for (int t = 0; t < NTK; ++t) {
    const int g = wv + 4 * t, rt = g / (K / 16), ct = g % (K / 16);
    f4 u = f4_zero();
    if (!MERGE) u = proj(a.kp, rt, ct);
    f4 xg = proj(a.gpT, rt, ct);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int n = rt * 16 + acc_row(r), k = ct * 16 + acc_col();
      if (!MERGE) {
        const float nr = sqrtf(s_nrm[n]);
        const float key = u[r] / fmaxf(nr, 1e-12f);
        // F.normalize: below the clamp the denominator is the constant eps
        const float du = nr >= 1e-12f ? (dkt[t][r] - key * s_rd[n]) / nr : dkt[t][r] / 1e-12f;
        wsdu[n * K + k] = du;
      }
      wsdxg[n * K + k] = -(s_dg[k] / (float)N) * sigmoidf_(xg[r] - 4.f);
    }
  }
  __syncthreads();

  // ---- E. dVals = dvn * w + du Wk + dxb Bp^T + dxw Wp^T + dxg Gp^T
  {
    const E* kpT = static_cast<const E*>(ab.kpT) + (size_t)h * V * K;
    const E* bp = static_cast<const E*>(ab.bp) + (size_t)h * V * K;
    const E* wp = static_cast<const E*>(ab.wp) + (size_t)h * V * V;
    const E* gp = static_cast<const E*>(ab.gp) + (size_t)h * V * K;
    float* s_dVT = s_R1;   // [V][LDN]
#pragma unroll
    for (int t = 0; t < NTK; ++t) {
      const int g = wv + 4 * t, rt = g / (V / 16), ct = g % (V / 16);
      f4 acc = dvd[t];
      if (!MERGE) acc = mma_tile<E>(acc, wsdu + rt * 16 * K, K, kpT + (size_t)ct * 16 * K, K, K);
      acc = mma_tile<E>(acc, wsdxb + rt * 16 * K, K, bp + (size_t)ct * 16 * K, K, K);
      acc = mma_tile<E>(acc, wsdxw + rt * 16 * V, V, wp + (size_t)ct * 16 * V, V, V);
      acc = mma_tile<E>(acc, wsdxg + rt * 16 * K, K, gp + (size_t)ct * 16 * K, K, K);
      dvd[t] = acc;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int n = rt * 16 + acc_row(r), v = ct * 16 + acc_col();
        wsdV[n * V + v] = acc[r];
        s_dVT[v * LDN + n] = acc[r];
      }
    }
    if (!MERGE) {
      // S_below rows k (v contiguous) for dBank
      for (int e = tid; e < K * V; e += 256) s_X[(e / V) * LD + e % V] = sbelow(e / V, e % V);
    }
  }
  __syncthreads();

  // ---- F. dS_below and dBank
  auto scatter = [&](int k, int v, float x) {
    if (a.f_below == 1 && a.below_mode == 0) {
      ab.inj[fo * K * V + (size_t)k * V + v] = x;
    } else if (fin) {
      ab.d_below_fin[b * a.bf_sb + h * a.bf_sh + (long long)k * V + v] += x;
    } else {
      ab.d_below[(((size_t)b * a.NGb + src) * H + h) * K * V + (size_t)k * V + v] += x;
    }
  };
  if (MERGE) {
#pragma unroll
    for (int t = 0; t < NTK; ++t) {
      const int g = wv + 4 * t, rt = g / (V / 16), ct = g % (V / 16);
#pragma unroll
      for (int r = 0; r < 4; ++r) scatter(rt * 16 + acc_row(r), ct * 16 + acc_col(), dvd[t][r]);
    }
  } else {
    const E* bankT = static_cast<const E*>(ab.bankT) + (size_t)h * K * a.Nmax;
    const float* s_dVT = s_R1;
    constexpr int NTKV = (K / 16) * (V / 16) / 4;
    for (int t = 0; t < NTKV; ++t) {
      const int g = wv + 4 * t, rt = g / (V / 16), ct = g % (V / 16);
      f4 acc = f4_zero();
      const E* arow = bankT + (size_t)(rt * 16 + (lane & 15)) * a.Nmax + kofs<E>(lane);
      const float* brow = s_dVT + (ct * 16 + (lane & 15)) * LDN + kofs<E>(lane);
      constexpr int NSN = (N + KS - 1) / KS;
#pragma unroll
      for (int s = 0; s < NSN; ++s) {
        const bool live = s * KS + kofs<E>(lane) < N;
        typename Mma<E>::Frag fa = Mma<E>::zero();
        SF fb = Mma<E>::szero();
        if (live) {
          fa = Mma<E>::ld(arow + s * KS);
          fb = Mma<E>::ld(brow + s * KS);
        }
        acc = Mma<E>::mma(acc, fa, fb);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) scatter(rt * 16 + acc_row(r), ct * 16 + acc_col(), acc[r]);
    }
    // dBank[n][k] += sum_v dVals[n][v] S_below[k][v]
    float* dbank = ab.dbank + (size_t)h * a.Nmax * K;
#pragma unroll
    for (int t = 0; t < NTK; ++t) {
      const int g = wv + 4 * t, rt = g / (K / 16), ct = g % (K / 16);
      f4 acc = mma_tile<E>(f4_zero(), wsdV + rt * 16 * V, V, s_X + ct * 16 * LD, LD, V);
#pragma unroll
      for (int r = 0; r < 4; ++r)
        atomicAdd(&dbank[(rt * 16 + acc_row(r)) * K + ct * 16 + acc_col()], acc[r]);
    }
  }
}

// ---------------------------------------------------------------- A^T B sums

template <typename E, int X, int Y>
__global__ __launch_bounds__(256) void atb_kernel(AtBArgs a) {
  constexpr int LDM = 32 + 4;
  constexpr int TPW = (X / 16) * (Y / 16) / 4;
  __shared__ __attribute__((aligned(16))) float s_AT[X * LDM];
  __shared__ __attribute__((aligned(16))) float s_BT[Y * LDM];
  const int H = a.H, NF = a.NF, N = a.N;
  const int part = blockIdx.x % a.split;
  const int h = blockIdx.x / a.split;
  const int wv = wave_id(), tid = threadIdx.x;
  const int items = a.B * NF;
  const int per = (items + a.split - 1) / a.split;
  const int it0 = part * per, it1 = min(items, it0 + per);
  f4 acc[TPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t) acc[t] = f4_zero();
  for (int it = it0; it < it1; ++it) {
    const int b = it / NF, i = it % NF;
    const size_t base = (((size_t)b * H + h) * NF + i) * N;
    const float* Ap = a.A + base * X;
    const float* Bp = a.Bm + base * Y;
    for (int n0 = 0; n0 < N; n0 += 32) {
      // 32 rows of the reduction, transposed into LDS (zero past N)
      for (int e = tid; e < 32 * X; e += 256) {
        const int n = e / X, x = e % X;
        s_AT[x * LDM + n] = n0 + n < N ? Ap[(size_t)(n0 + n) * X + x] : 0.f;
      }
      for (int e = tid; e < 32 * Y; e += 256) {
        const int n = e / Y, y = e % Y;
        s_BT[y * LDM + n] = n0 + n < N ? Bp[(size_t)(n0 + n) * Y + y] : 0.f;
      }
      __syncthreads();
#pragma unroll
      for (int t = 0; t < TPW; ++t) {
        const int g = wv * TPW + t, rt = g / (Y / 16), ct = g % (Y / 16);
        acc[t] = mma_tile<E>(acc[t], s_AT + rt * 16 * LDM, LDM, s_BT + ct * 16 * LDM, LDM, 32);
      }
      __syncthreads();
    }
  }
  if (it0 >= it1) return;
  float* C = a.C + (size_t)h * X * Y;
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    const int g = wv * TPW + t, rt = g / (Y / 16), ct = g % (Y / 16);
#pragma unroll
    for (int r = 0; r < 4; ++r)
      atomicAdd(&C[(rt * 16 + acc_row(r)) * Y + ct * 16 + acc_col()], acc[t][r]);
  }
}

template <typename E, int K, int N, bool MERGE>
static hipError_t launch_probe_bwd(const ProbeBwdArgs& a, hipStream_t st) {
  const unsigned grid = (unsigned)(a.f.B * a.f.H * a.f.NF);
  if (grid == 0) return hipSuccess;
  hipLaunchKernelGGL((probe_bwd_kernel<E, K, N, MERGE>), dim3(grid), dim3(256), 0, st, a);
  return hipGetLastError();
}

template <typename E>
static hipError_t probe_bwd_dispatch(const ProbeBwdArgs& a, int K, hipStream_t st) {
  if (a.f.V != K) return hipErrorInvalidValue;
  if (a.f.merge) {
    if (a.f.N != K) return hipErrorInvalidValue;
    if (K == 64) return launch_probe_bwd<E, 64, 64, true>(a, st);
    if (K == 128) return launch_probe_bwd<E, 128, 128, true>(a, st);
    return hipErrorInvalidValue;
  }
#define NGDN_PB(KK, NN) \
  if (K == KK && a.f.N == NN) return launch_probe_bwd<E, KK, NN, false>(a, st);
  NGDN_PB(64, 16) NGDN_PB(64, 32) NGDN_PB(64, 64) NGDN_PB(64, 128)
  NGDN_PB(128, 16) NGDN_PB(128, 32) NGDN_PB(128, 64) NGDN_PB(128, 128)
#undef NGDN_PB
  return hipErrorInvalidValue;
}

hipError_t probe_bwd(const ProbeBwdArgs& a, int dtype, int K, hipStream_t st) {
  return dtype == NGDN_BF16 ? probe_bwd_dispatch<bf16>(a, K, st) : probe_bwd_dispatch<float>(a, K, st);
}

template <typename E, int X, int Y>
static hipError_t launch_atb(const AtBArgs& a, hipStream_t st) {
  const unsigned grid = (unsigned)(a.H * a.split);
  if (grid == 0 || a.B * a.NF == 0) return hipSuccess;
  hipLaunchKernelGGL((atb_kernel<E, X, Y>), dim3(grid), dim3(256), 0, st, a);
  return hipGetLastError();
}

template <typename E>
static hipError_t atb_dispatch(const AtBArgs& a, hipStream_t st) {
#define NGDN_AB(XX, YY) \
  if (a.X == XX && a.Y == YY) return launch_atb<E, XX, YY>(a, st);
  NGDN_AB(64, 64) NGDN_AB(128, 128)
#undef NGDN_AB
  return hipErrorInvalidValue;
}

hipError_t atb_accumulate(const AtBArgs& a, int dtype, hipStream_t st) {
  return dtype == NGDN_BF16 ? atb_dispatch<bf16>(a, st) : atb_dispatch<float>(a, st);
}

}  // namespace ngdn
