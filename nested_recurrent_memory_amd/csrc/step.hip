// One decoding token (nested_gdn2/ops/naive.py:42-134), level-0 half:
//   S0 <- e^g S0 - k ((k*b)^T (e^g S0)) + k (v*w)^T      (ops/naive.py:7-39 with N = 1)
//   read_l = (scale q_l)^T S_l  for every level, S0 already updated
//   o = sum_l mix_l read_l
// The promotions that follow at chunk boundaries reuse the probe and the
// firing scan (one firing), gated per row on the device by the position.
//
// Columns of V never interact here either: a workgroup owns SV = 32 columns
// of one (batch, head), the grid is B*H*(V/32), and the slices of one
// (batch, head) sit on one XCD. Each thread holds 4 adjacent columns (one
// 16-byte load per row) of K/32 rows of every level's state; the two sums over
// K (the erase projection and the reads) go through wave shuffles and a
// 4-wave LDS exchange. The work is one pass over the state: HBM-bound.
#include "ngdn_kernels.h"

namespace ngdn {

template <typename E, int K, int V>
__global__ __launch_bounds__(256) void step_kernel(StepArgs a) {
  constexpr int SV = 32;                 // columns per workgroup
  constexpr int CQ = SV / 4;             // threads across one row (4 columns each)
  constexpr int RG = 256 / CQ;           // row groups
  constexpr int RPT = K / RG;            // rows per thread
  constexpr int NW = 256 / WAVE;
  static_assert(RPT >= 1 && K % RG == 0, "K must be a multiple of 32");
  __shared__ __attribute__((aligned(16))) float s_red[NW][SV];
  __shared__ __attribute__((aligned(16))) float s_rd[NW][MAXL][SV];

  const int H = a.H, L = a.L;
  int bh, vs;
  xcd_split(blockIdx.x, gridDim.x, V / SV, bh, vs);
  const int h = bh % H, b = bh / H;
  const int tid = threadIdx.x, lane = lane_id(), wv = wave_id();
  const int cq = tid % CQ, rg = tid / CQ;
  const int col = vs * SV + cq * 4;

  const E* q = static_cast<const E*>(a.q) + (size_t)bh * L * K;
  const E* kk = static_cast<const E*>(a.k) + (size_t)bh * K;
  const E* bb = static_cast<const E*>(a.b) + (size_t)bh * K;
  const float* gg = a.g + (size_t)bh * K;
  const size_t sbase = (size_t)bh * L * K * V;
  const float* Sin = a.s_in + sbase;
  float* Sout = a.s_out + sbase;
  const bool copy_up = a.s_out != a.s_in;

  // ---- level 0: decay, erase projection r = (k*b)^T (e^g S0)
  f4 s0[RPT];
  float key[RPT];
  f4 part = f4_zero();
#pragma unroll
  for (int r = 0; r < RPT; ++r) {
    const int k = rg * RPT + r;
    s0[r] = *reinterpret_cast<const f4*>(Sin + (size_t)k * V + col);
    const float gam = expf(gg[k]);
    key[r] = to_f(kk[k]);
    const float kb = key[r] * to_f(bb[k]);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      s0[r][c] *= gam;
      part[c] += kb * s0[r][c];
    }
  }
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    part[c] += __shfl_xor(part[c], 8, WAVE);
    part[c] += __shfl_xor(part[c], 16, WAVE);
    part[c] += __shfl_xor(part[c], 32, WAVE);
  }
  if (lane < CQ) *reinterpret_cast<f4*>(&s_red[wv][cq * 4]) = part;

  // reads of the upper levels (unchanged by this token)
  f4 rd[MAXL];
#pragma unroll
  for (int l = 0; l < MAXL; ++l) rd[l] = f4_zero();
#pragma unroll
  for (int l = 1; l < MAXL; ++l) {
    if (l < L) {
      const float* Sl = Sin + (size_t)l * K * V;
#pragma unroll
      for (int r = 0; r < RPT; ++r) {
        const int k = rg * RPT + r;
        const f4 x = *reinterpret_cast<const f4*>(Sl + (size_t)k * V + col);
        const float ql = to_f(q[(size_t)l * K + k]) * a.scale;
#pragma unroll
        for (int c = 0; c < 4; ++c) rd[l][c] += ql * x[c];
      }
    }
  }
  lds_barrier();
  f4 u;
  {
    const E* vv = static_cast<const E*>(a.v) + (size_t)bh * V + col;
    const E* ww = static_cast<const E*>(a.w) + (size_t)bh * V + col;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float r = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) r += s_red[w][cq * 4 + c];
      u[c] = to_f(vv[c]) * to_f(ww[c]) - r;
    }
  }

  // ---- S0 += k u^T, written; reads of every level (the upper levels were
  // read above, before any store)
#pragma unroll
  for (int r = 0; r < RPT; ++r) {
    const int k = rg * RPT + r;
#pragma unroll
    for (int c = 0; c < 4; ++c) s0[r][c] += key[r] * u[c];
    *reinterpret_cast<f4*>(Sout + (size_t)k * V + col) = s0[r];
    const float ql = to_f(q[k]) * a.scale;
#pragma unroll
    for (int c = 0; c < 4; ++c) rd[0][c] += ql * s0[r][c];
  }
#pragma unroll
  for (int l = 0; l < MAXL; ++l) {
    if (l < L) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        rd[l][c] += __shfl_xor(rd[l][c], 8, WAVE);
        rd[l][c] += __shfl_xor(rd[l][c], 16, WAVE);
        rd[l][c] += __shfl_xor(rd[l][c], 32, WAVE);
      }
      if (lane < CQ) *reinterpret_cast<f4*>(&s_rd[wv][l][cq * 4]) = rd[l];
    }
  }
  lds_barrier();

  // ---- o = sum_l mix_l read_l
  if (tid < CQ) {
    const E* mix = static_cast<const E*>(a.mix) + (size_t)bh * L;
    E* o = static_cast<E*>(a.o) + (size_t)bh * V + col;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float acc = 0.f;
      for (int l = 0; l < L; ++l) {
        float r = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) r += s_rd[w][l][cq * 4 + c];
        acc += r * to_f(mix[l]);
      }
      o[c] = from_f<E>(acc);
    }
  }
  // out of place: the upper levels are copied last (after every load)
  if (copy_up) {
    for (int l = 1; l < L; ++l) {
#pragma unroll
      for (int r = 0; r < RPT; ++r) {
        const size_t off = (size_t)l * K * V + (size_t)(rg * RPT + r) * V + col;
        *reinterpret_cast<f4*>(Sout + off) = *reinterpret_cast<const f4*>(Sin + off);
      }
    }
  }
}

// ---------------------------------------------------------------- promotions
//
// One level's promotion for one (b, h) (ops/naive.py:101-123 with
// ops/probe.py:69-136 and the update of ops/naive.py:7-39):
//   Vals = Bank[:N] S_below (learned) or S_below (merge)          [N,V]
//   keys = u / max(|u|, 1e-12), u = Vals Wk^T; b = sigmoid(Vals Bp - 4);
//   w = sigmoid(Vals Wp); g = -mean_n softplus(Vals Gp - 4)      (fp32)
//   S~ = e^g S;  Vn = Vals w - (keys b) S~;  S <- S~ + keys^T Vn
// Eight waves; wave w keeps column tile w % (K/16) of every [N,K], [N,V]
// and [K,V] tile grid, so the B operands of its products are loaded once
// and the tiles of U = Vals w, Vn and S stay in its registers from one
// product to the next. LDS (one buffer, regions reused): Vals fp32, later
// S~^T, later Vn^T (split); keys b [N][K] and keys^T [K][N] (split); the
// per-wave partial sums (added in wave order, so replays are bitwise equal).
template <int K>
struct PromoteLds {
  static constexpr int PADB = 8;                     // split-tile padding (elements)
  static constexpr size_t R1 = 4 * (size_t)K * (K + PADB);   // >= Vals, S~^T, Vn^T
  static constexpr size_t R2 = 4 * (size_t)PROMOTE_NMAX * (K + PADB);   // keys b
  static constexpr size_t R3 = 4 * (size_t)K * (PROMOTE_NMAX + PADB);   // keys^T
  static constexpr size_t BYTES = R1 + R2 + R3;
};

template <typename E, int K, int N, bool MERGE>
__device__ __forceinline__ void promote_level(const PromoteArgs& a, char* smem, float* s_nrm,
                                              float* s_gs, float* s_gam, int b, int h, int l) {
  constexpr int V = K, NW = 8;
  constexpr int LD = K + 4;                          // fp32 Vals rows
  constexpr int CTK = K / 16;
  constexpr int NTL = (N / 16) * CTK;                // [N,K] (= [N,V]) tiles
  constexpr int TPW = (NTL + NW - 1) / NW;
  constexpr int TKV = CTK * CTK / NW;                // [K,V] tiles per wave
  constexpr int NPW = NW / CTK;                      // waves per column tile
  constexpr int KS = Mma<E>::KS, NKS = K / KS, NSN = (N + KS - 1) / KS;
  using ST = SplitTile<E>;
  typedef typename ST::T TT;
  constexpr int LDKB = K + ST::PAD, LDKT = N + ST::PAD, LDST = K + ST::PAD, LDVN = N + ST::PAD;
  typedef typename Mma<E>::SFrag SF;
  typedef typename Mma<E>::Frag FR;
  static_assert(NW % CTK == 0 && N <= PROMOTE_NMAX, "tile split");
  static_assert(sizeof(float) * N * LD <= PromoteLds<K>::R1 &&
                sizeof(TT) * ST::NPLANE * V * LDST <= PromoteLds<K>::R1 &&
                sizeof(TT) * ST::NPLANE * V * LDVN <= PromoteLds<K>::R1 &&
                sizeof(TT) * ST::NPLANE * N * LDKB <= PromoteLds<K>::R2 &&
                sizeof(TT) * ST::NPLANE * K * LDKT <= PromoteLds<K>::R3, "LDS regions");
  float* s_V = reinterpret_cast<float*>(smem);
  const ST sST{reinterpret_cast<TT*>(smem), V * LDST};
  const ST sVnT{reinterpret_cast<TT*>(smem), V * LDVN};
  const ST sKB{reinterpret_cast<TT*>(smem + PromoteLds<K>::R1), N * LDKB};
  const ST sKT{reinterpret_cast<TT*>(smem + PromoteLds<K>::R1 + PromoteLds<K>::R2), K * LDKT};

  const int H = a.H, L = a.L;
  const int lane = lane_id(), wv = wave_id(), tid = threadIdx.x;
  const int rl = lane & 15, ko = kofs<E>(lane), ctw = wv % CTK;
  const size_t skv = (size_t)K * V;
  const float* Sb = a.state + ((size_t)(b * H + h) * L + (l - 1)) * skv;   // level below, updated
  float* Sl = a.state + ((size_t)(b * H + h) * L + l) * skv;
  const size_t hkv = (size_t)H * K * V, lp = (size_t)(l - 1);
  auto tile = [&](int t, int& rt) -> bool {
    const int g = wv + NW * t;
    rt = g / CTK;
    return g < NTL;
  };
  for (int e = tid; e < NW * N; e += blockDim.x) s_nrm[e] = 0.f;
  for (int e = tid; e < NPW * K; e += blockDim.x) s_gs[e] = 0.f;

  // ---- Vals
  if (!MERGE) {
    const E* bank = static_cast<const E*>(a.bank) + (lp * H + h) * (size_t)a.Nmax * K;
    const int v = ctw * 16 + rl;
    SF fS[NKS];
#pragma unroll
    for (int s = 0; s < NKS; ++s) {
      const int k0 = s * KS + ko;
      fS[s] = Mma<E>::makes([&](int e) { return Sb[(size_t)(k0 + e) * V + v]; });
    }
    f4 vt[TPW];
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      vt[t] = f4_zero();
      int rt;
      if (!tile(t, rt)) continue;
      const E* arow = bank + (size_t)(rt * 16 + rl) * K + ko;
#pragma unroll
      for (int s = 0; s < NKS; ++s) vt[t] = Mma<E>::mma(vt[t], Mma<E>::ld(arow + s * KS), fS[s]);
    }
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      int rt;
      if (!tile(t, rt)) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) s_V[(rt * 16 + acc_row(r)) * LD + ctw * 16 + acc_col()] = vt[t][r];
    }
  } else {
    for (int e = tid; e < K * V / 4; e += blockDim.x) {
      const int r = e / (V / 4), c = (e % (V / 4)) * 4;
      *reinterpret_cast<f4*>(s_V + r * LD + c) = *reinterpret_cast<const f4*>(Sb + (size_t)r * V + c);
    }
  }
  lds_barrier();

  // ---- projections; U = Vals w and the keys' parts stay in registers
  f4 ut[TPW], bt[TPW], uu[TPW];
  {
    const size_t pr = (size_t)(ctw * 16 + rl) * V + ko;
    const E* kpH = static_cast<const E*>(a.kp) + (lp * H + h) * (size_t)K * V + pr;
    const E* bpH = static_cast<const E*>(a.bpT) + lp * hkv + (size_t)h * K * V + pr;
    const E* wpH = static_cast<const E*>(a.wpT) + lp * hkv + (size_t)h * V * V + pr;
    const E* gpH = static_cast<const E*>(a.gpT) + lp * hkv + (size_t)h * K * V + pr;
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
      ut[t] = bt[t] = uu[t] = f4_zero();
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
      float sg = 0.f;
#pragma unroll
      for (int r = 0; r < 4; ++r) sg += softplusf_(xg[r] - 4.f);
      sg += __shfl_xor(sg, 16, WAVE);
      sg += __shfl_xor(sg, 32, WAVE);
      if (lane < 16) s_gs[(wv / CTK) * K + ctw * 16 + lane] += sg;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int n = rt * 16 + acc_row(r), v = ctw * 16 + acc_col();
        bt[t][r] = sigmoidf_(xb[r] - 4.f);
        uu[t][r] = s_V[n * LD + v] * sigmoidf_(xw[r]);
      }
      if (!MERGE) {
        ut[t] = xu;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float q = xu[r] * xu[r];
          q = row16_sum(q);
          if (rl == 0) s_nrm[wv * N + rt * 16 + acc_row(r)] += q;
        }
      }
    }
  }
  lds_barrier();

  // ---- gam = e^g; keys b and keys^T as split tiles
  for (int e = tid; e < K; e += blockDim.x) {
    float x = 0.f;
#pragma unroll
    for (int p = 0; p < NPW; ++p) x += s_gs[p * K + e];
    s_gam[e] = expf(-x / (float)N);
  }
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    int rt;
    if (!tile(t, rt)) continue;
    const int k = ctw * 16 + acc_col(), n0 = rt * 16 + acc_row(0);
    f4 kv4;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int n = n0 + r;
      float key;
      if (MERGE) {
        key = (n == k) ? 1.f : 0.f;
      } else {
        float nr = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) nr += s_nrm[w * N + n];
        key = ut[t][r] * __builtin_amdgcn_rcpf(fmaxf(sqrtf(nr), 1e-12f));
      }
      kv4[r] = key;
      sKB.put1(n * LDKB + k, key * bt[t][r]);
    }
    sKT.put4(k * LDKT + n0, kv4);
  }
  lds_barrier();   // gam ready; Vals no longer read

  // ---- S~ = e^g S: this wave's [K,V] tiles in registers and S~^T in LDS
  f4 st[TKV];
#pragma unroll
  for (int t = 0; t < TKV; ++t) {
    const int rt = (wv + NW * t) / CTK, k0 = rt * 16 + acc_row(0), v = ctw * 16 + acc_col();
#pragma unroll
    for (int r = 0; r < 4; ++r) st[t][r] = Sl[(size_t)(k0 + r) * V + v] * s_gam[k0 + r];
    sST.put4(v * LDST + k0, st[t]);
  }
  lds_barrier();

  // ---- Vn = U - (keys b) S~ on this wave's [N,V] tiles
  f4 vn[TPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    vn[t] = f4_zero();
    int rt;
    if (!tile(t, rt)) continue;
    f4 acc = f4_zero();
#pragma unroll
    for (int s = 0; s < NKS; ++s)
      acc = Mma<E>::mma(acc, sKB.get((rt * 16 + rl) * LDKB + s * KS + ko),
                        sST.get((ctw * 16 + rl) * LDST + s * KS + ko));
#pragma unroll
    for (int r = 0; r < 4; ++r) vn[t][r] = uu[t][r] - acc[r];
  }
  lds_barrier();   // Vn^T replaces S~^T
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    int rt;
    if (!tile(t, rt)) continue;
    sVnT.put4((ctw * 16 + acc_col()) * LDVN + rt * 16 + acc_row(0), vn[t]);
  }
  lds_barrier();

  // ---- S <- S~ + keys^T Vn, written in place
#pragma unroll
  for (int t = 0; t < TKV; ++t) {
    const int rt = (wv + NW * t) / CTK;
    f4 acc = st[t];
#pragma unroll
    for (int s = 0; s < NSN; ++s) {
      const bool live = s * KS + ko < N;
      SF fa = Mma<E>::szero(), fb = Mma<E>::szero();
      if (live) {
        fa = sKT.get((rt * 16 + rl) * LDKT + s * KS + ko);
        fb = sVnT.get((ctw * 16 + rl) * LDVN + s * KS + ko);
      }
      acc = Mma<E>::mma(acc, fa, fb);
    }
    const int k0 = rt * 16 + acc_row(0), v = ctw * 16 + acc_col();
#pragma unroll
    for (int r = 0; r < 4; ++r) Sl[(size_t)(k0 + r) * V + v] = acc[r];
  }
}

template <typename E, int K>
__global__ __launch_bounds__(512) void promote_kernel(PromoteArgs a) {
  __shared__ __attribute__((aligned(16))) char smem[PromoteLds<K>::BYTES];
  __shared__ float s_nrm[8 * PROMOTE_NMAX], s_gs[8 * K], s_gam[K];
  const int bh = blockIdx.x, h = bh % a.H, b = bh / a.H;
  const long long end = (a.pos ? a.pos[b] : a.pos_all) + 1;
  if (end % a.chunk != 0) return;
  const long long nchunk = end / a.chunk;
  for (int l = 1; l < a.L; ++l) {
    if (nchunk % a.f[l] != 0) continue;
    const int N = a.N[l];
    if (a.merge) {
      if constexpr (K <= PROMOTE_NMAX) promote_level<E, K, K, true>(a, smem, s_nrm, s_gs, s_gam, b, h, l);
    } else if (N == 16) {
      promote_level<E, K, 16, false>(a, smem, s_nrm, s_gs, s_gam, b, h, l);
    } else if (N == 32) {
      promote_level<E, K, 32, false>(a, smem, s_nrm, s_gs, s_gam, b, h, l);
    } else {
      promote_level<E, K, 64, false>(a, smem, s_nrm, s_gs, s_gam, b, h, l);
    }
    // the next level's probe reads this level's new state, written by every
    // wave: a barrier that also orders global memory
    __syncthreads();
  }
}

template <typename E, int K>
static hipError_t launch_promote(const PromoteArgs& a, hipStream_t st) {
  const unsigned grid = (unsigned)(a.B * a.H);
  if (grid == 0) return hipSuccess;
  hipLaunchKernelGGL((promote_kernel<E, K>), dim3(grid), dim3(512), 0, st, a);
  return hipGetLastError();
}

hipError_t promote_fwd(const PromoteArgs& a, int dtype, int K, hipStream_t st) {
  for (int l = 1; l < a.L; ++l) {
    const int N = a.merge ? K : a.N[l];
    if (N > PROMOTE_NMAX || (N != 16 && N != 32 && N != 64)) return hipErrorInvalidValue;
  }
  if (K == 64) return dtype == NGDN_BF16 ? launch_promote<bf16, 64>(a, st) : launch_promote<float, 64>(a, st);
  if (K == 128) return dtype == NGDN_BF16 ? launch_promote<bf16, 128>(a, st) : launch_promote<float, 128>(a, st);
  return hipErrorInvalidValue;
}

template <typename E, int K, int V>
static hipError_t launch_step(const StepArgs& a, hipStream_t st) {
  const unsigned grid = (unsigned)(a.B * a.H * (V / 32));
  hipLaunchKernelGGL((step_kernel<E, K, V>), dim3(grid), dim3(256), 0, st, a);
  return hipGetLastError();
}

hipError_t step_fwd(const StepArgs& a, int dtype, int K, int V, hipStream_t st) {
#define NGDN_ST(E, KK, VV) \
  if (K == KK && V == VV) return launch_step<E, KK, VV>(a, st);
  if (dtype == NGDN_BF16) {
    NGDN_ST(bf16, 64, 64) NGDN_ST(bf16, 64, 128) NGDN_ST(bf16, 128, 64) NGDN_ST(bf16, 128, 128)
  } else {
    NGDN_ST(float, 64, 64) NGDN_ST(float, 64, 128) NGDN_ST(float, 128, 64) NGDN_ST(float, 128, 128)
  }
#undef NGDN_ST
  return hipErrorInvalidValue;
}

}  // namespace ngdn
