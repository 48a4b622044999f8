// Backward of one level's firings: through the update step and the probe.
//
// Update step (ops/update_bwd.py:115-158), with s = e^g * S_j (S_j the state
// entering group j), kb = keys * b, vn = vals * w - kb s and, from the reverse
// scan, dS' (gradient of the state after the firing) and dvn = keys dS':
//   P = dvn s^T,  Q = vn dS'^T
//   dkeys = Q - P * b,   db = -P * keys,   dvals = dvn * w,   dw = dvn * vals
//   dg_k  = sum_v dS'[k][v] s[k][v] - sum_n kb[n][k] P[n][k]
// Probe (ops/probe.py:59-102; the reference differentiates it by autograd
// replay, ops/chunk.py:339-371,486-517), with u = Vals Wk^T:
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

// One workgroup (8 waves) per firing-head. The [N,K] (= [N,V]) tile grid is
// dealt to the waves so that every wave keeps one column tile (ctw) and takes
// the row tiles rt: the B operands of every product (the state rows, the
// parameter rows) are then loaded once per wave and shared by its row tiles,
// all of them issued together. A operands come from LDS: Vals, kb, vn and
// dvn in fp32 rows, the four workspaces of the dVals product and dVals itself
// as split tiles. Barriers that only order LDS do not wait for the
// workspace stores (lds_barrier).
template <typename E, int K, int N, bool MERGE>
__global__ __launch_bounds__(512) void probe_bwd_kernel(ProbeBwdArgs ab) {
  const ProbeArgs& a = ab.f;
  constexpr int V = K;
  constexpr int NW = 8;                             // waves
  constexpr int LD = K + 4;                         // fp32 rows of K (= V) values
  constexpr int LDN = N + 4;
  constexpr int CTK = K / 16;
  constexpr int NTL = (N / 16) * CTK;               // [N,K] (= [N,V]) tiles
  constexpr int TPW = (NTL + NW - 1) / NW;          // tiles per wave
  constexpr int NTKV = CTK * CTK;                   // [K,V] tiles
  constexpr int TPW2 = (NTKV + NW - 1) / NW;
  constexpr int KS = Mma<E>::KS;
  constexpr int KPL = Mma<E>::KPL;
  constexpr int NKS = K / KS;
  static_assert(NW % CTK == 0, "every wave keeps one column tile");
  typedef typename Mma<E>::SFrag SF;
  typedef typename Mma<E>::Frag FR;
  using ST = SplitTile<E>;
  typedef typename ST::T TT;
  constexpr int LDT = K + ST::PAD;                  // split tile rows
  // LDS: phases 1-5 use fp32 rows Vals, kb (later vn) and, when it fits, dvn;
  // phases 6-7 the four workspaces as split tiles (when they fit); phase 8
  // dVals as a split tile and dVals^T in fp32.
  constexpr size_t BUDGET = 150 * 1024;
  constexpr size_t SZ_F = sizeof(float) * N * LD;
  constexpr size_t SZ_T = sizeof(TT) * ST::NPLANE * N * LDT;
  constexpr size_t SZ_DVT = sizeof(float) * V * LDN;
  constexpr bool DVN_LDS = 3 * SZ_F <= BUDGET;
  constexpr bool WS_LDS = 4 * SZ_T <= BUDGET;
  constexpr size_t SZ_A = (DVN_LDS ? 3 : 2) * SZ_F;
  constexpr size_t SZ_B = WS_LDS ? 4 * SZ_T : 0;
  constexpr size_t SZ_C = (MERGE ? 0 : SZ_T) + SZ_DVT;
  constexpr size_t SZ_AB = SZ_A > SZ_B ? SZ_A : SZ_B;
  __shared__ __attribute__((aligned(16))) char smem[SZ_AB > SZ_C ? SZ_AB : SZ_C];
  // Sums across waves go through one slot per contributing wave (column tile
  // or wave group), added in a fixed order: the results do not depend on the
  // order in which the waves finish.
  constexpr int NPW = NW / CTK;                     // waves per column tile
  __shared__ float s_nrm[CTK * N], s_rd[CTK * N], s_gs[NPW * K], s_dg[NPW * K];
  __shared__ float s_gam[K], s_nsum[N], s_rdt[N], s_dgt[K];
  float* s_V = reinterpret_cast<float*>(smem);
  float* s_kb = reinterpret_cast<float*>(smem + SZ_F);
  float* s_vn = s_kb;
  float* s_dvn = reinterpret_cast<float*>(smem + 2 * SZ_F);
  auto ws_tile = [&](int j) {
    return ST{reinterpret_cast<TT*>(smem + j * SZ_T), N * LDT};
  };
  const ST sDV{reinterpret_cast<TT*>(smem), N * LDT};
  float* s_dVT = reinterpret_cast<float*>(smem + (MERGE ? 0 : SZ_T));

  const int NF = a.NF, H = a.H;
  int b, h, i;
  head_xcd_split(blockIdx.x, H, NF, b, h, i);
  const int bh = b * H + h;
  const int lane = lane_id(), wv = wave_id(), tid = threadIdx.x;
  const int rl = lane & 15, ko = kofs<E>(lane);
  const int ctw = wv % CTK;                         // this wave's column tile
  const size_t fo = (size_t)bh * NF + i;

  // ---- the gathered lower state: rows (kv) and, when stored, transposed (vk)
  const int src = ((i + 1) * a.f_here) / a.f_below;
  const bool fin = src >= a.NGb;
  const size_t sbase = (a.below_mode == 0 ? ((size_t)b * H + h) * a.NGb + src
                                          : ((size_t)b * a.NGb + src) * H + h) * K * V;
  const float* Skv = fin ? a.below_fin + b * a.bf_sb + h * a.bf_sh : ab.below_kv + sbase;
  const float* Svk = fin ? nullptr : ab.below_vk + sbase;
  // this level's state before firing i, rows and transposed
  const size_t jbase = (((size_t)b * ab.NG + i) * H + h) * K * V;
  const float* Sj = ab.Sg + jbase;
  const float* SjT = ab.SgT + jbase;
  const float* dSp = ab.dSp + fo * K * V;
  const float* dvn = ab.dvn + fo * N * V;
  float* wsV = ab.wsV + fo * N * V;
  float* wsdu = ab.wsdu + fo * N * K;
  float* wsdxb = ab.wsdxb + fo * N * K;
  float* wsdxg = ab.wsdxg + fo * N * K;
  float* wsdxw = ab.wsdxw + fo * N * V;
  float* wsdV = ab.wsdV + fo * N * V;

  for (int e = tid; e < CTK * N; e += blockDim.x) { s_nrm[e] = 0.f; s_rd[e] = 0.f; }
  for (int e = tid; e < NPW * K; e += blockDim.x) { s_gs[e] = 0.f; s_dg[e] = 0.f; }

  // row tile of this wave's t-th tile (its column tile is ctw)
  auto tile = [&](int t, int& rt) -> bool {
    const int g = wv + NW * t;
    rt = g / CTK;
    return g < NTL;
  };

  // ---- 1. Vals = Bank[:N] S (learned) or S (merge)
  if (!MERGE) {
    const E* bank = static_cast<const E*>(a.bank) + (size_t)h * a.Nmax * K;
    const int v = ctw * 16 + rl;
    // the state rows' loads first, all in flight, then their splits; each
    // tile's bank rows likewise before its products
    float xs[NKS][KPL];
#pragma unroll
    for (int s = 0; s < NKS; ++s) {
      const int k0 = s * KS + ko;
      if (Svk) {
        ld_raw<KPL>(Svk + (size_t)v * K + k0, xs[s]);
      } else {
#pragma unroll
        for (int e = 0; e < KPL; ++e) xs[s][e] = Skv[(size_t)(k0 + e) * V + v];
      }
    }
    __builtin_amdgcn_sched_barrier(0);   // the state loads stay ahead of their splits
    SF fS[NKS];
#pragma unroll
    for (int s = 0; s < NKS; ++s) fS[s] = Mma<E>::makes([&](int e) { return xs[s][e]; });
    f4 vt[TPW];
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      vt[t] = f4_zero();
      int rt;
      if (!tile(t, rt)) continue;
      const E* arow = bank + (size_t)(rt * 16 + rl) * K + ko;
      FR fb[NKS];   // the tile's bank rows, all in flight before its products
#pragma unroll
      for (int s = 0; s < NKS; ++s) fb[s] = Mma<E>::ld(arow + s * KS);
      __builtin_amdgcn_sched_barrier(0);   // keep the loads ahead of the products
#pragma unroll
      for (int s = 0; s < NKS; ++s) vt[t] = Mma<E>::mma(vt[t], fb[s], fS[s]);
    }
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      int rt;
      if (!tile(t, rt)) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int n = rt * 16 + acc_row(r), vv = ctw * 16 + acc_col();
        s_V[n * LD + vv] = vt[t][r];
        wsV[n * V + vv] = vt[t][r];
      }
    }
  } else {
    for (int e = tid; e < K * V / 4; e += blockDim.x) {
      const int k = e / (V / 4), v = (e % (V / 4)) * 4;
      const f4 x = *reinterpret_cast<const f4*>(Skv + (size_t)k * V + v);
      *reinterpret_cast<f4*>(s_V + k * LD + v) = x;
      *reinterpret_cast<f4*>(wsV + (size_t)k * V + v) = x;
    }
  }
  lds_barrier();

  // ---- 2. the four projections of Vals, once: u = Vals Wk^T (learned),
  // xb = Vals Bp, xw = Vals Wp, xg = Vals Gp; key norms and decay sums
  f4 u[TPW], xb[TPW], xw[TPW], xg[TPW];
  {
    const size_t pr = (size_t)(ctw * 16 + rl) * V + ko;
    const E* kpH = static_cast<const E*>(a.kp) + (size_t)h * K * V + pr;
    const E* bpH = static_cast<const E*>(a.bpT) + (size_t)h * K * V + pr;
    const E* wpH = static_cast<const E*>(a.wpT) + (size_t)h * V * V + pr;
    const E* gpH = static_cast<const E*>(a.gpT) + (size_t)h * K * V + pr;
    FR pk[NKS], pb[NKS], pw[NKS], pg[NKS];
#pragma unroll
    for (int s = 0; s < NKS; ++s) {
      if (!MERGE) pk[s] = Mma<E>::ld(kpH + s * KS);
      pb[s] = Mma<E>::ld(bpH + s * KS);
      pw[s] = Mma<E>::ld(wpH + s * KS);
      pg[s] = Mma<E>::ld(gpH + s * KS);
    }
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      u[t] = xb[t] = xw[t] = xg[t] = f4_zero();
      int rt;
      if (!tile(t, rt)) continue;
      const float* arow = s_V + (rt * 16 + rl) * LD + ko;
#pragma unroll
      for (int s = 0; s < NKS; ++s) {
        const SF fa = Mma<E>::ld(arow + s * KS);
        if (!MERGE) u[t] = Mma<E>::mma(u[t], fa, pk[s]);
        xb[t] = Mma<E>::mma(xb[t], fa, pb[s]);
        xw[t] = Mma<E>::mma(xw[t], fa, pw[s]);
        xg[t] = Mma<E>::mma(xg[t], fa, pg[s]);
      }
      float sg = 0.f;
#pragma unroll
      for (int r = 0; r < 4; ++r) sg += softplusf_(xg[t][r] - 4.f);
      sg += __shfl_xor(sg, 16, WAVE);
      sg += __shfl_xor(sg, 32, WAVE);
      if (lane < 16) s_gs[(wv / CTK) * K + ctw * 16 + lane] += sg;
      if (!MERGE) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float q = u[t][r] * u[t][r];
          q = row16_sum(q);
          if (rl == 0) s_nrm[ctw * N + rt * 16 + acc_row(r)] += q;
        }
      }
    }
  }
  // dvn staged for phases 4-5 (loads issued before the barrier)
  if constexpr (DVN_LDS) stage_f32<512, N, V>(s_dvn, LD, dvn, V);
  lds_barrier();
  // the decay and the squared key norms from their per-wave slots, in order
  if (tid < K) {
    float x = 0.f;
#pragma unroll
    for (int p = 0; p < NPW; ++p) x += s_gs[p * K + tid];
    s_gam[tid] = expf(-x / (float)N);
  } else if (!MERGE && tid < K + N) {
    const int n = tid - K;
    float x = 0.f;
#pragma unroll
    for (int c = 0; c < CTK; ++c) x += s_nrm[c * N + n];
    s_nsum[n] = x;
  }
  lds_barrier();

  auto keyval = [&](int t, int rt, int r) -> float {
    const int n = rt * 16 + acc_row(r), k = ctw * 16 + acc_col();
    if (MERGE) return n == k ? 1.f : 0.f;
    return u[t][r] * __builtin_amdgcn_rcpf(fmaxf(sqrtf(s_nsum[n]), 1e-12f));
  };

  // ---- 3. kb = keys * b into LDS; gam = e^g
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    int rt;
    if (!tile(t, rt)) continue;
#pragma unroll
    for (int r = 0; r < 4; ++r)
      s_kb[(rt * 16 + acc_row(r)) * LD + ctw * 16 + acc_col()] =
          keyval(t, rt, r) * sigmoidf_(xb[t][r] - 4.f);
  }
  lds_barrier();

  // ---- 4. vn = Vals w - kb s with s = e^g S_j (s^T rows scaled per k);
  // dw-side terms
  f4 vnt[TPW], dvd[TPW];
  {
    SF fT[NKS];
    const float* brow = SjT + (size_t)(ctw * 16 + rl) * K + ko;
#pragma unroll
    for (int s = 0; s < NKS; ++s) {
      const int k0 = s * KS + ko;
      float x[KPL];
      ld_raw<KPL>(brow + s * KS, x);
      fT[s] = Mma<E>::makes([&](int e) { return x[e] * s_gam[k0 + e]; });
    }
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      vnt[t] = dvd[t] = f4_zero();
      int rt;
      if (!tile(t, rt)) continue;
      const float* arow = s_kb + (rt * 16 + rl) * LD + ko;
      f4 ks = f4_zero();
#pragma unroll
      for (int s = 0; s < NKS; ++s) ks = Mma<E>::mma(ks, Mma<E>::ld(arow + s * KS), fT[s]);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int n = rt * 16 + acc_row(r), v = ctw * 16 + acc_col();
        const float w = sigmoidf_(xw[t][r]);
        const float val = s_V[n * LD + v];
        const float dv = DVN_LDS ? s_dvn[n * LD + v] : dvn[(size_t)n * V + v];
        vnt[t][r] = val * w - ks[r];
        dvd[t][r] = dv * w;
        // dxw goes to its workspace at once (not held through phase 5);
        // phase 6 reads this lane's own values back for the LDS tile
        wsdxw[(size_t)n * V + v] = dv * val * w * (1.f - w);
      }
    }
  }
  lds_barrier();   // vn replaces kb
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    int rt;
    if (!tile(t, rt)) continue;
#pragma unroll
    for (int r = 0; r < 4; ++r)
      s_vn[(rt * 16 + acc_row(r)) * LD + ctw * 16 + acc_col()] = vnt[t][r];
  }
  lds_barrier();

  // ---- 5. P = dvn s^T, Q = vn dS'^T; dkeys, db, the decay gradient
  f4 dkt[TPW], dxbt[TPW];
  {
    const int kc = ctw * 16 + rl;
    const float gk = s_gam[kc];
    SF fP[NKS], fQ[NKS];
    float dgp = 0.f;   // sum over this lane's v of dS'[kc][v] S_j[kc][v]
#pragma unroll
    for (int s = 0; s < NKS; ++s) {
      const int v0 = s * KS + ko;
      float x[KPL], y[KPL];
      ld_raw<KPL>(Sj + (size_t)kc * V + v0, x);
      ld_raw<KPL>(dSp + (size_t)kc * V + v0, y);
      fP[s] = Mma<E>::makes([&](int e) { return gk * x[e]; });
      fQ[s] = Mma<E>::makes([&](int e) { return y[e]; });
#pragma unroll
      for (int e = 0; e < KPL; ++e) dgp += x[e] * y[e];
    }
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      dkt[t] = dxbt[t] = f4_zero();
      int rt;
      if (!tile(t, rt)) continue;
      const int ar = (rt * 16 + rl) * LD + ko;
      f4 P = f4_zero(), Q = f4_zero();
#pragma unroll
      for (int s = 0; s < NKS; ++s) {
        const SF fa = DVN_LDS ? Mma<E>::ld(s_dvn + ar + s * KS)
                              : Mma<E>::ld(dvn + (size_t)(rt * 16 + rl) * V + ko + s * KS);
        P = Mma<E>::mma(P, fa, fP[s]);
        Q = Mma<E>::mma(Q, Mma<E>::ld(s_vn + ar + s * KS), fQ[s]);
      }
      float cs = 0.f;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int n = rt * 16 + acc_row(r);
        const float key = keyval(t, rt, r), bb = sigmoidf_(xb[t][r] - 4.f);
        const float dkey = Q[r] - P[r] * bb;
        const float dbg = -P[r] * key;
        cs += key * bb * P[r];
        dkt[t][r] = dkey;
        dxbt[t][r] = dbg * bb * (1.f - bb);
        if (!MERGE) {
          float rd = key * dkey;
          rd = row16_sum(rd);
          if (rl == 0) s_rd[ctw * N + n] += rd;
        }
      }
      cs += __shfl_xor(cs, 16, WAVE);
      cs += __shfl_xor(cs, 32, WAVE);
      if (lane < 16) s_dg[(wv / CTK) * K + ctw * 16 + lane] += -cs;
    }
    // + sum_v dS'[k][v] s[k][v] (one wave per column tile adds it)
    dgp += __shfl_xor(dgp, 16, WAVE);
    dgp += __shfl_xor(dgp, 32, WAVE);
    if (wv < CTK && lane < 16) s_dg[kc] += gk * dgp;   // the first wave group's slot
  }
  lds_barrier();
  // the key-norm and decay gradients from their per-wave slots, in order
  if (tid < K) {
    float x = 0.f;
#pragma unroll
    for (int p = 0; p < NPW; ++p) x += s_dg[p * K + tid];
    s_dgt[tid] = x;
  } else if (!MERGE && tid < K + N) {
    const int n = tid - K;
    float x = 0.f;
#pragma unroll
    for (int c = 0; c < CTK; ++c) x += s_rd[c * N + n];
    s_rdt[n] = x;
  }
  lds_barrier();

  // ---- 6. du and dxg; the dVals product's parameter rows are loaded ahead
  // of the workspace stores
  f4 dut[TPW], dxgt[TPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    dut[t] = dxgt[t] = f4_zero();
    int rt;
    if (!tile(t, rt)) continue;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int n = rt * 16 + acc_row(r), k = ctw * 16 + acc_col();
      if (!MERGE) {
        const float nr = sqrtf(s_nsum[n]);
        const float rn = __builtin_amdgcn_rcpf(fmaxf(nr, 1e-12f));
        const float key = u[t][r] * rn;
        // F.normalize: below the clamp the denominator is the constant eps
        dut[t][r] = nr >= 1e-12f ? (dkt[t][r] - key * s_rdt[n]) * rn : dkt[t][r] * 1e12f;
      }
      dxgt[t][r] = -(s_dgt[k] * (1.f / (float)N)) * sigmoidf_(xg[t][r] - 4.f);
    }
  }
  FR qk[NKS], qb[NKS], qw[NKS], qg[NKS];
  {
    const size_t br = (size_t)(ctw * 16 + rl) * K + ko;
    const E* kpT = static_cast<const E*>(ab.kpT) + (size_t)h * V * K + br;
    const E* bp = static_cast<const E*>(ab.bp) + (size_t)h * V * K + br;
    const E* wp = static_cast<const E*>(ab.wp) + (size_t)h * V * V + br;
    const E* gp = static_cast<const E*>(ab.gp) + (size_t)h * V * K + br;
#pragma unroll
    for (int s = 0; s < NKS; ++s) {
      if (!MERGE) qk[s] = Mma<E>::ld(kpT + s * KS);
      qb[s] = Mma<E>::ld(bp + s * KS);
      qw[s] = Mma<E>::ld(wp + s * KS);
      qg[s] = Mma<E>::ld(gp + s * KS);
    }
  }
  // workspaces of the parameter gradients, and (when they fit) the same
  // values as split LDS tiles for the dVals product
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    int rt;
    if (!tile(t, rt)) continue;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int n = rt * 16 + acc_row(r), k = ctw * 16 + acc_col();
      if (!MERGE) wsdu[(size_t)n * K + k] = dut[t][r];
      wsdxb[(size_t)n * K + k] = dxbt[t][r];
      wsdxg[(size_t)n * K + k] = dxgt[t][r];
      if constexpr (WS_LDS) {
        if (!MERGE) ws_tile(0).put1(n * LDT + k, dut[t][r]);
        ws_tile(1).put1(n * LDT + k, dxbt[t][r]);
        ws_tile(2).put1(n * LDT + k, wsdxw[(size_t)n * V + k]);
        ws_tile(3).put1(n * LDT + k, dxgt[t][r]);
      }
    }
  }
  if constexpr (WS_LDS) lds_barrier();
  else __syncthreads();   // the workspaces are read back from global memory

  // ---- 7. dVals = dvn * w + du Wk + dxb Bp^T + dxw Wp^T + dxg Gp^T
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    int rt;
    if (!tile(t, rt)) continue;
    f4 acc = dvd[t];
#pragma unroll
    for (int s = 0; s < NKS; ++s) {
      const int off = (rt * 16 + rl) * LDT + s * KS + ko;
      const size_t go = (size_t)(rt * 16 + rl) * K + s * KS + ko;
      if (!MERGE) acc = Mma<E>::mma(acc, WS_LDS ? ws_tile(0).get(off) : Mma<E>::ld(wsdu + go), qk[s]);
      acc = Mma<E>::mma(acc, WS_LDS ? ws_tile(1).get(off) : Mma<E>::ld(wsdxb + go), qb[s]);
      acc = Mma<E>::mma(acc, WS_LDS ? ws_tile(2).get(off) : Mma<E>::ld(wsdxw + go), qw[s]);
      acc = Mma<E>::mma(acc, WS_LDS ? ws_tile(3).get(off) : Mma<E>::ld(wsdxg + go), qg[s]);
    }
    dvd[t] = acc;
  }
  // Phase 8's operands from global memory, ahead of this phase's stores:
  // the lower state's rows (dBank) and the bank's columns (dS_below)
  const E* bankT = static_cast<const E*>(ab.bankT) + (size_t)h * K * a.Nmax;
  constexpr int NSN = (N + KS - 1) / KS;
  SF fSk[NKS];
  FR fBt[TPW2][NSN];
  if (!MERGE) {
    const float* srow = Skv + (size_t)(ctw * 16 + rl) * V + ko;
#pragma unroll
    for (int s = 0; s < NKS; ++s) fSk[s] = Mma<E>::ld(srow + s * KS);
#pragma unroll
    for (int t = 0; t < TPW2; ++t) {
      // unconditional loads (an unused slot reads column 0 of a valid row)
      // whose unwanted values are zeroed: a load under a branch leaves a
      // register copy at the merge that waits for every load before it
      const int g = wv + NW * t;
      const E* arow = bankT + (size_t)(((g < NTKV ? g : 0) / CTK) * 16 + rl) * a.Nmax;
#pragma unroll
      for (int s = 0; s < NSN; ++s) {
        const bool ok = g < NTKV && s * KS + ko < N;
        const FR x = Mma<E>::ld(arow + (ok ? s * KS + ko : 0));
        fBt[t][s] = ok ? x : Mma<E>::zero();
      }
    }
  }
  lds_barrier();   // dVals replaces the workspace tiles
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    int rt;
    if (!tile(t, rt)) continue;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int n = rt * 16 + acc_row(r), v = ctw * 16 + acc_col();
      wsdV[(size_t)n * V + v] = dvd[t][r];
      if (!MERGE) {
        sDV.put1(n * LDT + v, dvd[t][r]);
        s_dVT[v * LDN + n] = dvd[t][r];
      }
    }
  }
  lds_barrier();

  // ---- 8. dS_below and dBank
  // The [K,V] tiles g = wv + NW t of dS_below go to this firing's slot of
  // the injection inj [B,H,NF,K,V], which the lower level's reverse scan adds
  // to the gradient of the state the firing read (level 1: every firing; a
  // level above: firings that read a stored state), or, for a firing above
  // level 1 that reads the lower level's final state, are added to that
  // state's gradient (every addend read before any store)
  auto scatter_all = [&](const f4* x) {
    constexpr int NT2 = TPW2;
    const bool to_fin = a.below_mode != 0 && fin;
    float prev[NT2][4];
#pragma unroll
    for (int t = 0; t < NT2; ++t) {
      const int g = wv + NW * t;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        prev[t][r] = 0.f;
        if (g >= NTKV || !to_fin) continue;
        const int k = (g / CTK) * 16 + acc_row(r), v = (g % CTK) * 16 + acc_col();
        prev[t][r] = ab.d_below_fin[b * a.bf_sb + h * a.bf_sh + (long long)k * V + v];
      }
    }
#pragma unroll
    for (int t = 0; t < NT2; ++t) {
      const int g = wv + NW * t;
      if (g >= NTKV) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int k = (g / CTK) * 16 + acc_row(r), v = (g % CTK) * 16 + acc_col();
        if (to_fin)
          ab.d_below_fin[b * a.bf_sb + h * a.bf_sh + (long long)k * V + v] = prev[t][r] + x[t][r];
        else
          ab.inj[fo * K * V + (size_t)k * V + v] = x[t][r];
      }
    }
  };
  if (MERGE) {
    // [N,K] tiles are the [K,V] tiles here (N = K = V): same numbering
    static_assert(!MERGE || TPW == TPW2, "merge: one tile grid");
    scatter_all(dvd);
  } else {
    // dS_below[k][v] = sum_n Bank[n][k] dVals[n][v]: B = dVals^T rows v of
    // this wave's column tile (the [K,V] tiles of a wave share it too)
    SF fd[NSN];
#pragma unroll
    for (int s = 0; s < NSN; ++s)
      fd[s] = s * KS + ko < N ? Mma<E>::ld(s_dVT + (ctw * 16 + rl) * LDN + s * KS + ko) : Mma<E>::szero();
    f4 dsb[TPW2];
#pragma unroll
    for (int t = 0; t < TPW2; ++t) {
      dsb[t] = f4_zero();
      if (wv + NW * t >= NTKV) continue;
#pragma unroll
      for (int s = 0; s < NSN; ++s) dsb[t] = Mma<E>::mma(dsb[t], fBt[t][s], fd[s]);
    }
    // dBank[n][k] += sum_v dVals[n][v] S_below[k][v]
    f4 dbt[TPW];
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      dbt[t] = f4_zero();
      int rt;
      if (!tile(t, rt)) continue;
#pragma unroll
      for (int s = 0; s < NKS; ++s)
        dbt[t] = Mma<E>::mma(dbt[t], sDV.get((rt * 16 + rl) * LDT + s * KS + ko), fSk[s]);
    }
    scatter_all(dsb);
    float* dbank = ab.dbank + fo * N * K;   // this firing's partial, summed by ngdn_param_grads
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      int rt;
      if (!tile(t, rt)) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r)
        dbank[(rt * 16 + acc_row(r)) * K + ctw * 16 + acc_col()] = dbt[t][r];
    }
  }
}

// ---------------------------------------------------------------- A^T B sums

template <typename E, int X, int Y>
__global__ __launch_bounds__(256) void atb_kernel(AtBArgs a) {
  // C[h] += sum over rows n of A[n]^T B[n]. Slabs of R rows are staged
  // transposed as split tiles (A^T [X][R], B^T [Y][R], the reduction index
  // contiguous), each value split once by the thread that stages it; every
  // fragment is then a 16-byte read.
  constexpr int R = 32;                      // rows per staged slab
  using ST = SplitTile<E>;
  constexpr int LDT = R + ST::PAD;
  constexpr int XT = X / 16, YT = Y / 16;
  constexpr int XTW = XT / 4;                // x-tiles per wave (all y-tiles each)
  constexpr int KS = Mma<E>::KS;
  static_assert(XT % 4 == 0, "X must split over the 4 waves");
  static_assert(X * R % (256 * 4) == 0 && Y * R % (256 * 4) == 0, "whole groups of 4 rows");
  __shared__ __attribute__((aligned(16))) typename ST::T s_at[ST::NPLANE * X * LDT];
  __shared__ __attribute__((aligned(16))) typename ST::T s_bt[ST::NPLANE * Y * LDT];
  const ST sA{s_at, X * LDT}, sB{s_bt, Y * LDT};
  const int H = a.H, NF = a.NF, N = a.N;
  const int prod = blockIdx.x / (H * a.split);
  const int part = blockIdx.x % a.split;
  const int h = (blockIdx.x / a.split) % H;
  const float* Ap = a.A[prod];
  const float* Bp = a.Bm[prod];
  const int lane = lane_id(), wv = wave_id(), tid = threadIdx.x;
  const int items = a.B * NF;
  const int per = (items + a.split - 1) / a.split;
  const int it0 = part * per, it1 = min(items, it0 + per);   // may be empty: zeros are written
  f4 acc[XTW][YT];
#pragma unroll
  for (int x = 0; x < XTW; ++x)
#pragma unroll
    for (int y = 0; y < YT; ++y) acc[x][y] = f4_zero();
  // A thread stages 4 consecutive rows of one column (a wave reads whole
  // rows); the next slab is read into registers while this one is multiplied.
  constexpr int GA = X * R / 4 / 256, GB = Y * R / 4 / 256;   // 4-row groups per thread
  f4 ra[GA], rb[GB];
  const int slabs_per_item = (N + R - 1) / R;
  const int nslab = it1 > it0 ? (it1 - it0) * slabs_per_item : 0;
  auto fetch = [&](int sl) {
    const int it = it0 + sl / slabs_per_item, n0 = (sl % slabs_per_item) * R;
    const int b = it / NF, i = it % NF, nr = min(R, N - n0);
    const size_t row0 = (((size_t)b * H + h) * NF + i) * N + n0;
#pragma unroll
    for (int u = 0; u < GA; ++u) {
      const int e = tid + 256 * u, c = e % X, r4 = (e / X) * 4;
#pragma unroll
      for (int j = 0; j < 4; ++j) ra[u][j] = r4 + j < nr ? Ap[(row0 + r4 + j) * X + c] : 0.f;
    }
#pragma unroll
    for (int u = 0; u < GB; ++u) {
      const int e = tid + 256 * u, c = e % Y, r4 = (e / Y) * 4;
#pragma unroll
      for (int j = 0; j < 4; ++j) rb[u][j] = r4 + j < nr ? Bp[(row0 + r4 + j) * Y + c] : 0.f;
    }
  };
  if (nslab > 0) fetch(0);
  for (int sl = 0; sl < nslab; ++sl) {
#pragma unroll
    for (int u = 0; u < GA; ++u) {
      const int e = tid + 256 * u;
      sA.put4((e % X) * LDT + (e / X) * 4, ra[u]);
    }
#pragma unroll
    for (int u = 0; u < GB; ++u) {
      const int e = tid + 256 * u;
      sB.put4((e % Y) * LDT + (e / Y) * 4, rb[u]);
    }
    lds_barrier();
    if (sl + 1 < nslab) fetch(sl + 1);
#pragma unroll
    for (int s = 0; s < R / KS; ++s) {
      const int r0 = s * KS + kofs<E>(lane);
      typename Mma<E>::SFrag fa[XTW];
#pragma unroll
      for (int x = 0; x < XTW; ++x) fa[x] = sA.get(((wv * XTW + x) * 16 + (lane & 15)) * LDT + r0);
#pragma unroll
      for (int y = 0; y < YT; ++y) {
        const auto fb = sB.get((y * 16 + (lane & 15)) * LDT + r0);
#pragma unroll
        for (int x = 0; x < XTW; ++x) acc[x][y] = Mma<E>::mma(acc[x][y], fa[x], fb);
      }
    }
    lds_barrier();
  }
  // this workgroup's partial sum, added to C in a fixed order by ordered_sum
  float* P = a.parts + (((size_t)prod * H + h) * a.split + part) * X * Y;
#pragma unroll
  for (int x = 0; x < XTW; ++x)
#pragma unroll
    for (int y = 0; y < YT; ++y)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        P[((wv * XTW + x) * 16 + acc_row(r)) * Y + y * 16 + acc_col()] = acc[x][y][r];
}

// out_w[g][x] += sum over j1 < n1, j2 < n2 (in that order) of
// parts_w[g pg + j1 s1 + j2 s2 + x]: one thread per output element, so every
// element is a fixed-order sum written once.
__global__ __launch_bounds__(256) void ordered_sum_kernel(OrderedSumArgs a) {
  const int w = blockIdx.x / a.ng, g = blockIdx.x % a.ng;
  const long long x = (long long)blockIdx.y * 256 + threadIdx.x;
  if (x >= a.n[w]) return;
  const float* p = a.parts[w] + g * a.pg[w] + x;
  float acc = 0.f;
  for (int j1 = 0; j1 < a.n1[w]; ++j1)
    for (int j2 = 0; j2 < a.n2[w]; ++j2) acc += p[j1 * a.s1[w] + j2 * a.s2[w]];
  a.out[w][g * a.og[w] + x] += acc;
}

hipError_t ordered_sum(const OrderedSumArgs& a, hipStream_t st) {
  long long nmax = 0;
  for (int w = 0; w < a.nsum; ++w) nmax = a.n[w] > nmax ? a.n[w] : nmax;
  if (a.nsum == 0 || nmax == 0 || a.ng == 0) return hipSuccess;
  const dim3 grid((unsigned)(a.nsum * a.ng), (unsigned)((nmax + 255) / 256));
  hipLaunchKernelGGL(ordered_sum_kernel, grid, dim3(256), 0, st, a);
  return hipGetLastError();
}

template <typename E, int K, int N, bool MERGE>
static hipError_t launch_probe_bwd(const ProbeBwdArgs& a, hipStream_t st) {
  const unsigned grid = (unsigned)(a.f.B * a.f.H * a.f.NF);
  if (grid == 0) return hipSuccess;
  hipLaunchKernelGGL((probe_bwd_kernel<E, K, N, MERGE>), dim3(grid), dim3(512), 0, st, a);
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
  const unsigned grid = (unsigned)(a.nprod * a.H * a.split);
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
