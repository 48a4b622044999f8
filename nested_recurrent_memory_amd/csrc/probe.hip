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
// One workgroup per (batch, head, firing); the five N x K x V products run on
// MFMA (exact bf16 parameters against the fp32 state / Vals split in two) with
// the gates in fp32.
#include "ngdn_kernels.h"

namespace ngdn {

template <typename E, int K, int N, bool MERGE>
__global__ __launch_bounds__(256) void probe_fwd_kernel(ProbeArgs a) {
  constexpr int V = K;
  constexpr int LD = K + 4;                                // fp32 rows
  constexpr int NTK = (N / 16) * (K / 16) / 4;             // [N,K] tiles per wave
  // S^T (learned) and then Vals share one buffer
  constexpr int ROWS = (MERGE ? N : (V > N ? V : N));
  __shared__ __attribute__((aligned(16))) float s_buf[ROWS * LD];
  // per-wave partial sums (each slot has one writer), added in wave order so
  // that the result does not depend on the order in which waves finish
  __shared__ float s_nrm[4][N], s_gs[4][K];
  float* s_S = s_buf;      // [V][LD]: S^T, k contiguous
  float* s_V = s_buf;      // [N][LD]: Vals, v contiguous

  const int NF = a.NF, H = a.H;
  int b, h, i;
  head_xcd_split(blockIdx.x, H, NF, b, h, i);
  const int bh = b * H + h;
  const int lane = lane_id(), wv = wave_id(), tid = threadIdx.x;
  if (gated_out(a.gate, b)) return;

  // ---- the gathered lower state
  const int src = ((i + 1) * a.f_here) / a.f_below;
  const bool fin = src >= a.NGb;
  const float* Sf = nullptr;    // [K][V] source
  const float* Sh = nullptr;    // [V][K] source (level-0 chunk states)
  if (fin) Sf = a.below_fin + b * a.bf_sb + h * a.bf_sh;
  else if (a.below_mode == 1) Sf = a.below + (((size_t)b * a.NGb + src) * H + h) * K * V;
  else Sh = a.below + (((size_t)b * H + h) * a.NGb + src) * V * K;

  // learned: S^T rows (k contiguous); merge: Vals = S rows (v contiguous)
  {
    const float* same = MERGE ? Sf : Sh;     // already in the wanted orientation
    const float* swap = MERGE ? Sh : Sf;
    if (same) {
      for (int e = tid; e < V * K / 4; e += 256) {
        const int r = e / (K / 4), c = (e % (K / 4)) * 4;
        *reinterpret_cast<f4*>(s_buf + r * LD + c) = *reinterpret_cast<const f4*>(same + r * K + c);
      }
    } else {
      for (int e = tid; e < V * K; e += 256) s_buf[(e % K) * LD + e / K] = swap[e];
    }
  }
  for (int e = tid; e < 4 * N; e += 256) (&s_nrm[0][0])[e] = 0.f;
  for (int e = tid; e < 4 * K; e += 256) (&s_gs[0][0])[e] = 0.f;
  __syncthreads();

  const size_t fo = ((size_t)bh * NF + i);                 // scan-ready firing index
  const size_t ro = (((size_t)b * NF + i) * H + h);        // reference-format index

  // ---- Vals = Bank[:N] S (tiles in registers, then over S^T)
  if (!MERGE) {
    const E* bank = static_cast<const E*>(a.bank) + (size_t)h * a.Nmax * K;
    f4 vt[NTK];
#pragma unroll
    for (int t = 0; t < NTK; ++t) {
      const int g = wv + 4 * t, rt = g / (V / 16), ct = g % (V / 16);
      vt[t] = mma_tile<E>(f4_zero(), bank + rt * 16 * K, K, s_S + ct * 16 * LD, LD, K);
    }
    __syncthreads();
#pragma unroll
    for (int t = 0; t < NTK; ++t) {
      const int g = wv + 4 * t, rt = g / (V / 16), ct = g % (V / 16);
#pragma unroll
      for (int r = 0; r < 4; ++r) s_V[(rt * 16 + acc_row(r)) * LD + ct * 16 + acc_col()] = vt[t][r];
    }
    __syncthreads();
  }
  if (a.vals) {
    for (int e = tid; e < N * V; e += 256)
      a.vals[ro * N * V + e] = s_V[(e / V) * LD + e % V];
  }

  // ---- projections of Vals: A operand s_V (reduce over V), B from global
  auto proj_tile = [&](const E* Pt, int rt, int ct) -> f4 {
    // Pt: [cols][V] with V contiguous
    return mma_tile<E>(f4_zero(), s_V + rt * 16 * LD, LD, Pt + (size_t)ct * 16 * V, V, V);
  };
  const E* kpH = static_cast<const E*>(a.kp) + (size_t)h * K * V;
  const E* bpH = static_cast<const E*>(a.bpT) + (size_t)h * K * V;
  const E* wpH = static_cast<const E*>(a.wpT) + (size_t)h * V * V;
  const E* gpH = static_cast<const E*>(a.gpT) + (size_t)h * K * V;

  f4 ut[NTK], bt[NTK];
#pragma unroll
  for (int t = 0; t < NTK; ++t) {
    const int g = wv + 4 * t, rt = g / (K / 16), ct = g % (K / 16);
    // decay logits: column sums of softplus over the N pairs
    {
      f4 x = proj_tile(gpH, rt, ct);
      float s = 0.f;
#pragma unroll
      for (int r = 0; r < 4; ++r) s += softplusf_(x[r] - 4.f);
      s += __shfl_xor(s, 16, WAVE);
      s += __shfl_xor(s, 32, WAVE);
      if (lane < 16) s_gs[wv][ct * 16 + lane] += s;
    }
    // erase gate
    {
      f4 x = proj_tile(bpH, rt, ct);
#pragma unroll
      for (int r = 0; r < 4; ++r) bt[t][r] = sigmoidf_(x[r] - 4.f);
    }
    // write keys (learned)
    if (!MERGE) {
      ut[t] = proj_tile(kpH, rt, ct);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float s = ut[t][r] * ut[t][r];
        s += __shfl_xor(s, 1, WAVE);
        s += __shfl_xor(s, 2, WAVE);
        s += __shfl_xor(s, 4, WAVE);
        s += __shfl_xor(s, 8, WAVE);
        if ((lane & 15) == 0) s_nrm[wv][rt * 16 + acc_row(r)] += s;
      }
    }
  }
  // write gate, and U = Vals * w
  {
    float* Uo = a.U + fo * N * V;
    for (int g = wv; g < (N / 16) * (V / 16); g += 4) {
      const int rt = g / (V / 16), ct = g % (V / 16);
      f4 x = proj_tile(wpH, rt, ct);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int n = rt * 16 + acc_row(r), v = ct * 16 + acc_col();
        const float w = sigmoidf_(x[r]);
        Uo[n * V + v] = s_V[n * LD + v] * w;
        if (a.wo) a.wo[ro * N * V + n * V + v] = w;
      }
    }
  }
  __syncthreads();

  // ---- finalize: g, keys, A = keys*b*e^g, KT = keys^T
  if (tid < K) {
    const float g = -(s_gs[0][tid] + s_gs[1][tid] + s_gs[2][tid] + s_gs[3][tid]) / (float)N;
    a.gam[fo * K + tid] = expf(g);
    if (a.go) a.go[ro * K + tid] = g;
  }
  // the scan's operands in split form
  const SplitTile<E> Ao = split_at<E>(a.A + fo * N * K, N * K);
  const SplitTile<E> KTo = split_at<E>(a.KT + fo * K * N, K * N);
  const SplitTile<E> KNo = split_at<E>(a.keysN ? a.keysN + fo * N * K : nullptr, N * K);
  const SplitTile<E> ATo = split_at<E>(a.AT ? a.AT + fo * K * N : nullptr, K * N);
#pragma unroll
  for (int t = 0; t < NTK; ++t) {
    const int g = wv + 4 * t, rt = g / (K / 16), ct = g % (K / 16);
    const int k = ct * 16 + acc_col(), n0 = rt * 16 + acc_row(0);
    const float gam = expf(-(s_gs[0][k] + s_gs[1][k] + s_gs[2][k] + s_gs[3][k]) / (float)N);
    f4 kv4, av4;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int n = n0 + r;
      float key;
      if (MERGE) key = (n == k) ? 1.f : 0.f;
      else key = ut[t][r] / fmaxf(sqrtf(s_nrm[0][n] + s_nrm[1][n] + s_nrm[2][n] + s_nrm[3][n]),
                                  1e-12f);
      kv4[r] = key;
      av4[r] = key * bt[t][r] * gam;
      Ao.put1(n * K + k, av4[r]);
      if (a.keysN) KNo.put1(n * K + k, key);
      if (a.keys) a.keys[ro * N * K + n * K + k] = key;
      if (a.bo) a.bo[ro * N * K + n * K + k] = bt[t][r];
    }
    KTo.put4(k * N + n0, kv4);
    if (a.AT) ATo.put4(k * N + n0, av4);
  }
}

template <typename E, int K, int N, bool MERGE>
static hipError_t launch_probe(const ProbeArgs& a, hipStream_t st) {
  const unsigned grid = (unsigned)(a.B * a.H * a.NF);
  if (grid == 0) return hipSuccess;
  hipLaunchKernelGGL((probe_fwd_kernel<E, K, N, MERGE>), dim3(grid), dim3(256), 0, st, a);
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
