// Promotion probe: turn the level below into the pairs and gates this level
// writes at one firing (nested_gdn2/ops/probe.py:34-136).
//
// learned (ops/probe.py:69-102):
//   Vals = Bank[:N] S            [N,V]
//   u    = Vals Wk^T             [N,K]   keys = u / max(|u|, 1e-12)
//   b    = sigmoid(Vals Bp - 4)  [N,K]
//   w    = sigmoid(Vals Wp)      [N,V]
//   g    = -mean_n softplus(Vals Gp - 4)   [K]   (fp32)
// merge (ops/probe.py:105-136): keys = I, Vals = S, same gates.
//
// The gathered state is the lower level's state after this level's firing
// (ops/chunk.py:39-93). Outputs are written in the form the scan consumes:
// A = keys*b*e^g, KT = keys^T, U = Vals*w, gam = e^g.
// One workgroup (8 waves) per (batch, head, firing); the five N x K x V
// products run on MFMA (exact bf16 parameters against the fp32 state / Vals
// split in two) with the gates in fp32. Every wave keeps one column tile and
// takes the row tiles, so the B operands of its products (state rows,
// parameter rows) are loaded once and shared by its tiles; the A operands are
// the bank rows and Vals in LDS.
#include "ngdn_kernels.h"

namespace ngdn {

template <typename E, int K, int N, bool MERGE>
__global__ __launch_bounds__(512) void probe_fwd_kernel(ProbeArgs a) {
  constexpr int V = K;
  constexpr int NW = 8;                                    // waves
  constexpr int LD = K + 4;                                // fp32 rows
  constexpr int CTK = K / 16;
  constexpr int NTL = (N / 16) * CTK;                      // [N,K] (= [N,V]) tiles
  constexpr int TPW = (NTL + NW - 1) / NW;                 // tiles per wave
  constexpr int NPW = NW / CTK;                            // waves per column tile
  constexpr int KS = Mma<E>::KS;
  constexpr int KPL = Mma<E>::KPL;
  constexpr int NKS = K / KS;
  static_assert(NW % CTK == 0, "every wave keeps one column tile");
  typedef typename Mma<E>::SFrag SF;
  typedef typename Mma<E>::Frag FR;
  __shared__ __attribute__((aligned(16))) float s_V[N * LD];   // Vals, v contiguous
  // per-wave partial sums (each slot has one writer), added in wave order so
  // that the result does not depend on the order in which waves finish
  __shared__ float s_nrm[NW][N], s_gs[NPW][K];

  const int NF = a.NF, H = a.H;
  int b, h, i;
  head_xcd_split(blockIdx.x, H, a.ni > 0 ? a.ni : NF, b, h, i);
  i += a.i0;
  const int bh = b * H + h;
  const int lane = lane_id(), wv = wave_id(), tid = threadIdx.x;
  const int rl = lane & 15, ko = kofs<E>(lane);
  const int ctw = wv % CTK;
  if (gated_out(a.gate, b)) return;

  // ---- the gathered lower state
  const int src = ((i + 1) * a.f_here) / a.f_below;
  const bool fin = src >= a.NGb;
  const float* Sf = nullptr;    // [K][V] source
  const float* Sh = nullptr;    // [V][K] source (level-0 chunk states)
  if (fin) Sf = a.below_fin + b * a.bf_sb + h * a.bf_sh;
  else if (a.below_mode == 1) Sf = a.below + (((size_t)b * a.NGb + src) * H + h) * K * V;
  else Sh = a.below + (((size_t)b * H + h) * a.NGb + src) * V * K;
  for (int e = tid; e < NW * N; e += blockDim.x) (&s_nrm[0][0])[e] = 0.f;
  for (int e = tid; e < NPW * K; e += blockDim.x) (&s_gs[0][0])[e] = 0.f;

  const size_t fo = ((size_t)bh * NF + i);                 // scan-ready firing index
  const size_t ro = (((size_t)b * NF + i) * H + h);        // reference-format index
  auto tile = [&](int t, int& rt) -> bool {
    const int g = wv + NW * t;
    rt = g / CTK;
    return g < NTL;
  };

  // ---- Vals = Bank[:N] S (learned; B = rows v of S^T) or S (merge)
  if (!MERGE) {
    const E* bank = static_cast<const E*>(a.bank) + (size_t)h * a.Nmax * K;
    const int v = ctw * 16 + rl;
    // the state rows' loads first, all in flight, then their splits; each
    // tile's bank rows likewise before its products
    float xs[NKS][KPL];
#pragma unroll
    for (int s = 0; s < NKS; ++s) {
      const int k0 = s * KS + ko;
      if (Sh) {
        ld_raw<KPL>(Sh + (size_t)v * K + k0, xs[s]);
      } else {
#pragma unroll
        for (int e = 0; e < KPL; ++e) xs[s][e] = Sf[(size_t)(k0 + e) * V + v];
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
      typename Mma<E>::Frag fb[NKS];
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
      for (int r = 0; r < 4; ++r) s_V[(rt * 16 + acc_row(r)) * LD + ctw * 16 + acc_col()] = vt[t][r];
    }
  } else if (Sf) {
    for (int e = tid; e < K * V / 4; e += blockDim.x) {
      const int r = e / (V / 4), c = (e % (V / 4)) * 4;
      *reinterpret_cast<f4*>(s_V + r * LD + c) = *reinterpret_cast<const f4*>(Sf + (size_t)r * V + c);
    }
  } else {
    for (int e = tid; e < V * K; e += blockDim.x) s_V[(e % K) * LD + e / K] = Sh[e];
  }
  lds_barrier();
  if (a.vals) {
    for (int e = tid; e < N * V / 4; e += blockDim.x) {
      const int n = e / (V / 4), c = (e % (V / 4)) * 4;
      *reinterpret_cast<f4*>(a.vals + ro * N * V + (size_t)n * V + c) = *reinterpret_cast<const f4*>(s_V + n * LD + c);
    }
  }

  // ---- projections of Vals: A = Vals rows (LDS), B = parameter rows of this
  // wave's column tile, loaded once
  f4 ut[TPW], bt[TPW];
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
    float* Uo = a.U + fo * N * V;
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      ut[t] = bt[t] = f4_zero();
      int rt;
      if (!tile(t, rt)) continue;
      const float* arow = s_V + (rt * 16 + rl) * LD + ko;
      f4 xg = f4_zero(), xb = f4_zero(), xw = f4_zero(), xu = f4_zero();
#pragma unroll
      for (int s = 0; s < NKS; ++s) {
        const SF fa = Mma<E>::ld(arow + s * KS);
        if (!MERGE) xu = Mma<E>::mma(xu, fa, pk[s]);
        xb = Mma<E>::mma(xb, fa, pb[s]);
        xw = Mma<E>::mma(xw, fa, pw[s]);
        xg = Mma<E>::mma(xg, fa, pg[s]);
      }
      // decay logits: column sums of softplus over the N pairs
      float sg = 0.f;
#pragma unroll
      for (int r = 0; r < 4; ++r) sg += softplusf_(xg[r] - 4.f);
      sg += __shfl_xor(sg, 16, WAVE);
      sg += __shfl_xor(sg, 32, WAVE);
      if (lane < 16) s_gs[wv / CTK][ctw * 16 + lane] += sg;
      // erase gate; key norms (learned)
#pragma unroll
      for (int r = 0; r < 4; ++r) bt[t][r] = sigmoidf_(xb[r] - 4.f);
      if (!MERGE) {
        ut[t] = xu;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float q = xu[r] * xu[r];
          q = row16_sum(q);
          if (rl == 0) s_nrm[wv][rt * 16 + acc_row(r)] += q;
        }
      }
      // write gate, and U = Vals * w
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int n = rt * 16 + acc_row(r), v = ctw * 16 + acc_col();
        const float w = sigmoidf_(xw[r]);
        Uo[n * V + v] = s_V[n * LD + v] * w;
        if (a.wo) a.wo[ro * N * V + n * V + v] = w;
      }
    }
  }
  lds_barrier();

  // ---- finalize: g, keys, A = keys*b*e^g, KT = keys^T
  auto gsum = [&](int k) {
    float x = 0.f;
#pragma unroll
    for (int p = 0; p < NPW; ++p) x += s_gs[p][k];
    return x;
  };
  if (tid < K) {
    const float g = -gsum(tid) / (float)N;
    a.gam[fo * K + tid] = expf(g);
    if (a.go) a.go[ro * K + tid] = g;
  }
  // the scan's operands in split form (bf16 with N % 32 == 0: KT and AT in
  // fragment order, where a put4 of 16 lanes is 512 contiguous bytes)
  constexpr bool FRG = std::is_same<E, bf16>::value && N % 32 == 0;
  const SplitTile<E> Ao = split_at<E>(a.A + fo * N * K, N * K);
  const SplitTile<E> KTo = split_at<E>(a.KT + fo * K * N, K * N);
  const SplitTile<E> KNo = split_at<E>(a.keysN ? a.keysN + fo * N * K : nullptr, N * K);
  const SplitTile<E> ATo = split_at<E>(a.AT ? a.AT + fo * K * N : nullptr, K * N);
  const int k = ctw * 16 + acc_col();
  const float gam = expf(-gsum(k) / (float)N);
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    int rt;
    if (!tile(t, rt)) continue;
    const int n0 = rt * 16 + acc_row(0);
    f4 kv4, av4;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int n = n0 + r;
      float key;
      if (MERGE) {
        key = (n == k) ? 1.f : 0.f;
      } else {
        float nr = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) nr += s_nrm[w][n];
        key = ut[t][r] * __builtin_amdgcn_rcpf(fmaxf(sqrtf(nr), 1e-12f));
      }
      kv4[r] = key;
      av4[r] = key * bt[t][r] * gam;
      Ao.put1(n * K + k, av4[r]);
      if (a.keysN) KNo.put1(n * K + k, key);
      if (a.keys) a.keys[ro * N * K + n * K + k] = key;
      if (a.bo) a.bo[ro * N * K + n * K + k] = bt[t][r];
    }
    KTo.put4(FRG ? frag_ofs(k, n0, N) : k * N + n0, kv4);
    if (a.AT) ATo.put4(FRG ? frag_ofs(k, n0, N) : k * N + n0, av4);
  }
}

template <typename E, int K, int N, bool MERGE>
static hipError_t launch_probe(const ProbeArgs& a, hipStream_t st) {
  const unsigned grid = (unsigned)(a.B * a.H * (a.ni > 0 ? a.ni : a.NF));
  if (grid == 0) return hipSuccess;
  hipLaunchKernelGGL((probe_fwd_kernel<E, K, N, MERGE>), dim3(grid), dim3(512), 0, st, a);
  return hipGetLastError();
}

template <typename E>
static hipError_t probe_dispatch(const ProbeArgs& a, int K, hipStream_t st) {
  if (a.V != K) return hipErrorInvalidValue;
  if (a.merge) {
    if (a.N != K) return hipErrorInvalidValue;
    if (K == 64) return launch_probe<E, 64, 64, true>(a, st);
    if (K == 128) return launch_probe<E, 128, 128, true>(a, st);
    return hipErrorInvalidValue;
  }
#define NGDN_PR(KK, NN) \
  if (K == KK && a.N == NN) return launch_probe<E, KK, NN, false>(a, st);
  NGDN_PR(64, 16) NGDN_PR(64, 32) NGDN_PR(64, 64) NGDN_PR(64, 128)
  NGDN_PR(128, 16) NGDN_PR(128, 32) NGDN_PR(128, 64) NGDN_PR(128, 128)
#undef NGDN_PR
  return hipErrorInvalidValue;
}

hipError_t probe_fwd(const ProbeArgs& a, int dtype, int K, hipStream_t st) {
  return dtype == NGDN_BF16 ? probe_dispatch<bf16>(a, K, st) : probe_dispatch<float>(a, K, st);
}

}  // namespace ngdn
