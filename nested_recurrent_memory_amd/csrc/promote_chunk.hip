// The promotion ladder of the chunk op, fused per level: for one (batch,
// head), every firing of the level in order, each one the reference's chain
//   gather_source -> probe -> update_state
// (nested_gdn2/ops/chunk.py:257-290; ops/probe.py:34-136; ops/update_fwd.py:
// 21-128 with the store-then-fire group contract of :86-128):
//   for i < NF:   states[i] = S
//                 Sb   = the lower level's state after firing i
//                        (source index ((i+1) f_here) / f_below, the lower
//                        final state when it equals the lower group count)
//                 Vals = Bank[:N] Sb (learned) or Sb (merge)          [N,V]
//                 keys = u / max(|u|, 1e-12), u = Vals Wk^T;  b = sigmoid(Vals Bp - 4)
//                 w    = sigmoid(Vals Wp);  g = -mean_n softplus(Vals Gp - 4)
//                 S~ = e^g S;  Vn = Vals w - (keys b) S~;  S = S~ + keys^T Vn
//   for NF <= j < NG: states[j] = S;   final = S
// The lower snapshot, the probe's pairs and gates and the level's state stay
// on chip between the probe's read and the update's write: only the group
// states (the op's saved states) and, for the backward, each firing's keys,
// (keys b e^g)^T and e^g leave the workgroup.
//
// One workgroup of 8 waves per (b, h). Wave w keeps column tile w % (K/16)
// of every [N,K], [N,V] and [K,V] tile grid: its [K,V] tiles of the state stay
// in its registers for the whole sequence of firings, and the B operands of
// its products (snapshot rows, parameter rows) are loaded once per firing.
// LDS regions (reused within a firing): Vals fp32 and split, then S~^T,
// then Vn^T (split); keys b [N][K] and keys^T [K][N] (split); per-wave
// partial sums added in wave order (results do not depend on wave timing).
#include "ngdn_kernels.h"

namespace ngdn {

namespace {

template <int K, int N>
struct ChainLds {
  static constexpr int PADB = 8;
  static constexpr size_t VALS = 4 * (size_t)N * (K + 4);               // Vals fp32
  static constexpr size_t VALS2 = VALS + 4 * (size_t)N * (K + PADB);    // + Vals split
  static constexpr size_t ST = 4 * (size_t)K * (K + PADB);              // S~^T, Vn^T
  static constexpr size_t R1 = VALS2 > ST ? VALS2 : ST;
  static constexpr size_t R2 = 4 * (size_t)N * (K + PADB);              // keys b
  static constexpr size_t R3 = 4 * (size_t)K * (N + PADB);              // keys^T
  static constexpr size_t BANK = 2 * (size_t)N * (K + PADB);            // the bank, bf16 / fp32 rows
  static constexpr size_t BYTES = R1 + R2 + R3;
};

}  // namespace

template <typename E, int K, int N, bool MERGE>
__global__ __launch_bounds__(512) void promote_chain_kernel(PromoteChainArgs a) {
  constexpr int V = K, NW = 8;
  constexpr int LD = K + 4;                          // fp32 Vals rows
  constexpr int CTK = K / 16;
  constexpr int NTL = (N / 16) * CTK;                // [N,K] (= [N,V]) tiles
  constexpr int TPW = (NTL + NW - 1) / NW;
  constexpr int TKV = CTK * CTK / NW;                // [K,V] tiles per wave
  constexpr int NPW = NW / CTK;                      // waves per column tile
  constexpr int KS = Mma<E>::KS, KPL = Mma<E>::KPL, NKS = K / KS, NSN = (N + KS - 1) / KS;
  // bf16: the firing's parameter fragments are all issued before the Vals
  // product (4 NKS fragments of 16 bytes); fp32 loads them per k-step
  constexpr bool PRELOAD = sizeof(E) == 2;
  using ST = SplitTile<E>;
  typedef typename ST::T TT;
  constexpr int LDKB = K + ST::PAD, LDKT = N + ST::PAD, LDST = K + ST::PAD, LDVN = N + ST::PAD;
  typedef typename Mma<E>::SFrag SF;
  typedef typename Mma<E>::Frag FR;
  static_assert(NW % CTK == 0 && N <= PROMOTE_NMAX, "tile split");
  static_assert(ChainLds<K, N>::VALS2 <= ChainLds<K, N>::R1 &&
                sizeof(TT) * ST::NPLANE * V * LDST <= ChainLds<K, N>::R1 &&
                sizeof(TT) * ST::NPLANE * V * LDVN <= ChainLds<K, N>::R1 &&
                sizeof(TT) * ST::NPLANE * N * LDKB <= ChainLds<K, N>::R2 &&
                sizeof(TT) * ST::NPLANE * K * LDKT <= ChainLds<K, N>::R3, "LDS regions");
  __shared__ __attribute__((aligned(16))) char smem[ChainLds<K, N>::BYTES];
  // the level's query bank rows of this head (the same for every firing),
  // staged once for bf16 (the Vals product's A operand); fp32 reads them from
  // global memory (staged, they would not fit beside the rest at K = 128)
  constexpr bool BANK_LDS = !MERGE && sizeof(E) == 2;
  constexpr int LDB = K + 16 / (int)sizeof(E);
  __shared__ __attribute__((aligned(16))) E s_bank[BANK_LDS ? N * LDB : 1];
  __shared__ float s_nrm[NW * N], s_gs[NPW * K], s_gam[K], s_rn[N];
  float* s_V = reinterpret_cast<float*>(smem);
  // Vals again in split form: the projections' A operand, split once by its
  // writer instead of at every read by every wave
  const ST sVs{reinterpret_cast<TT*>(smem + ChainLds<K, N>::VALS), N * LDKB};
  const ST sST{reinterpret_cast<TT*>(smem), V * LDST};
  const ST sVnT{reinterpret_cast<TT*>(smem), V * LDVN};
  const ST sKB{reinterpret_cast<TT*>(smem + ChainLds<K, N>::R1), N * LDKB};
  const ST sKT{reinterpret_cast<TT*>(smem + ChainLds<K, N>::R1 + ChainLds<K, N>::R2), K * LDKT};

  const int H = a.H, NF = a.NF;
  const int bh = blockIdx.x, h = bh % H, b = bh / H;
  const int lane = lane_id(), wv = wave_id(), tid = threadIdx.x;
  const int ctw = wv % CTK;
  const size_t skv = (size_t)K * V;
  // Tile t of this wave in the [N,K] grid. When the waves cover the grid
  // evenly the test is a compile-time constant: no branch splits the tile
  // loops into basic blocks, so their loads can be issued ahead together.
  auto tile = [&](int t, int& rt) -> bool {
    const int g = wv + NW * t;
    rt = g / CTK;
    return (NTL % NW == 0) || g < NTL;
  };
  auto kv_row = [&](int t) { return (wv + NW * t) / CTK; };   // row tile of [K,V] tile t

  // the level's state: this wave's [K,V] tiles (rows k of row tile kv_row(t),
  // columns v of column tile ctw)
  f4 st[TKV];
  {
    const float* ib = a.init ? a.init + b * a.init_sb + h * a.init_sh : nullptr;
#pragma unroll
    for (int t = 0; t < TKV; ++t) {
      const int k0 = kv_row(t) * 16 + acc_row(0), v = ctw * 16 + acc_col();
#pragma unroll
      for (int r = 0; r < 4; ++r) st[t][r] = ib ? ib[(unsigned)((k0 + r) * V + v)] : 0.f;
    }
  }
  // uniform base pointers with 32-bit per-lane offsets: one address register
  // per access instead of a 64-bit pointer per element kept across firings
  auto group_vk = [&](int j) { return a.st_vk + (((size_t)b * a.NG + j) * H + h) * skv; };
  auto store_group = [&](int j, int ln) {
    float* kvb = a.st_kv + (((size_t)b * a.NG + j) * H + h) * skv;
    float* vkb = group_vk(j);
#pragma unroll
    for (int t = 0; t < TKV; ++t) {
      const int k0 = kv_row(t) * 16 + 4 * (ln >> 4), v = ctw * 16 + (ln & 15);
      *reinterpret_cast<f4*>(vkb + (unsigned)(v * K + k0)) = st[t];
#pragma unroll
      for (int r = 0; r < 4; ++r) kvb[(unsigned)((k0 + r) * V + v)] = st[t][r];
    }
  };
  // The learned probe's B operand of firing i (rows v = this wave's column of
  // the snapshot^T, KPL values per k-step), loaded as raw fp32 so that the
  // loads can be issued a firing ahead and split when used.
  auto load_snap = [&](int i, int ln, float* raw) {
    const int src = ((i + 1) * a.f_here) / a.f_below;
    const int v = ctw * 16 + (ln & 15);
    if (src >= a.NGb) {
      const float* Sf = a.below_fin + b * a.bf_sb + h * a.bf_sh;   // [K][V] rows
#pragma unroll
      for (int s = 0; s < NKS; ++s)
#pragma unroll
        for (int e = 0; e < KPL; ++e)
          raw[s * KPL + e] = Sf[(unsigned)((s * KS + kofs<E>(ln) + e) * V + v)];
    } else {
      const float* Sh = a.below_mode == 1 ? a.below + (((size_t)b * a.NGb + src) * H + h) * skv
                                          : a.below + (((size_t)b * H + h) * a.NGb + src) * skv;
#pragma unroll
      for (int s = 0; s < NKS; ++s) {
        const float* p = Sh + (unsigned)(v * K + s * KS + kofs<E>(ln));
        if constexpr (KPL == 8) {
          const f4 x0 = *reinterpret_cast<const f4*>(p), x1 = *reinterpret_cast<const f4*>(p + 4);
#pragma unroll
          for (int e = 0; e < 4; ++e) { raw[s * KPL + e] = x0[e]; raw[s * KPL + 4 + e] = x1[e]; }
        } else {
          raw[s * KPL] = *p;
        }
      }
    }
  };

  const E* bank = MERGE ? nullptr : static_cast<const E*>(a.bank) + (size_t)h * a.Nmax * K;
  const size_t pr = (size_t)(ctw * 16 + (lane & 15)) * V + kofs<E>(lane);
  const E* kpH = MERGE ? nullptr : static_cast<const E*>(a.kp) + (size_t)h * K * V + pr;
  const E* bpH = static_cast<const E*>(a.bpT) + (size_t)h * K * V + pr;
  const E* wpH = static_cast<const E*>(a.wpT) + (size_t)h * V * V + pr;
  const E* gpH = static_cast<const E*>(a.gpT) + (size_t)h * K * V + pr;

  for (int e = tid; e < NW * N; e += blockDim.x) s_nrm[e] = 0.f;
  for (int e = tid; e < NPW * K; e += blockDim.x) s_gs[e] = 0.f;
  if constexpr (BANK_LDS) {
    constexpr int VE = 16 / (int)sizeof(E), SEGS = K / VE;
    typedef __attribute__((__vector_size__(16))) int v4i;
    for (int e = tid; e < N * SEGS; e += blockDim.x) {
      const int n = e / SEGS, c = (e % SEGS) * VE;
      *reinterpret_cast<v4i*>(s_bank + n * LDB + c) =
          *reinterpret_cast<const v4i*>(bank + (size_t)n * K + c);
    }
  }
  float raw[NKS * KPL];
  if (!MERGE && NF > 0) load_snap(0, lane, raw);
  lds_barrier();   // the staged bank and the cleared partial sums

#pragma unroll 1
  for (int i = 0; i < NF; ++i) {
    // Per-lane offsets are derived inside the loop from a lane index the
    // compiler cannot see through: recomputed each firing (a few VALU
    // operations) rather than hoisted out of the loop and kept live, which
    // would not fit the register file beside the state.
    int lane_v = lane;
    asm volatile("" : "+v"(lane_v));
    const int rl = lane_v & 15, ko = kofs<E>(lane_v);
    auto arow_ = [&](int r) { return 4 * (lane_v >> 4) + r; };
    auto acol_ = [&]() { return lane_v & 15; };

    // ---- Vals = Bank[:N] Sb (learned) or Sb (merge), Sb the lower snapshot
    // after firing i
    // the snapshot's fragments split first (their loads are the oldest in
    // flight), then the parameter fragments of this wave's column tile are
    // issued, arriving during the Vals product
    SF fS[MERGE ? 1 : NKS];
    if (!MERGE) {
#pragma unroll
      for (int s = 0; s < NKS; ++s) fS[s] = Mma<E>::makes([&](int e) { return raw[s * KPL + e]; });
    }
    FR pk[PRELOAD ? NKS : 1], pb[PRELOAD ? NKS : 1], pw[PRELOAD ? NKS : 1], pg[PRELOAD ? NKS : 1];
    if constexpr (PRELOAD) {
#pragma unroll
      for (int s = 0; s < NKS; ++s) {
        if (!MERGE) pk[s] = Mma<E>::ld(kpH + s * KS);
        pb[s] = Mma<E>::ld(bpH + s * KS);
        pw[s] = Mma<E>::ld(wpH + s * KS);
        pg[s] = Mma<E>::ld(gpH + s * KS);
      }
    }
    if (!MERGE) {
      f4 vt[TPW];
#pragma unroll
      for (int t = 0; t < TPW; ++t) {
        vt[t] = f4_zero();
        int rt;
        if (!tile(t, rt)) continue;
        const E* arow = BANK_LDS ? s_bank + (rt * 16 + rl) * LDB + ko
                                 : bank + (unsigned)((rt * 16 + rl) * K + ko);
#pragma unroll
        for (int s = 0; s < NKS; ++s) vt[t] = Mma<E>::mma(vt[t], Mma<E>::ld(arow + s * KS), fS[s]);
      }
#pragma unroll
      for (int t = 0; t < TPW; ++t) {
        int rt;
        if (!tile(t, rt)) continue;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int n = rt * 16 + arow_(r), v = ctw * 16 + acol_();
          s_V[n * LD + v] = vt[t][r];
          sVs.put1(n * LDKB + v, vt[t][r]);
        }
      }
    } else {
      const int src = ((i + 1) * a.f_here) / a.f_below;
      if (src >= a.NGb) {
        const float* Sf = a.below_fin + b * a.bf_sb + h * a.bf_sh;
        for (int e = tid; e < K * V / 4; e += blockDim.x) {
          const int r = e / (V / 4), c = (e % (V / 4)) * 4;
          const f4 x = *reinterpret_cast<const f4*>(Sf + (unsigned)(r * V + c));
          *reinterpret_cast<f4*>(s_V + r * LD + c) = x;
          sVs.put4(r * LDKB + c, x);
        }
      } else {
        const float* Sh = a.below_mode == 1 ? a.below + (((size_t)b * a.NGb + src) * H + h) * skv
                                            : a.below + (((size_t)b * H + h) * a.NGb + src) * skv;
        for (int e = tid; e < V * K; e += blockDim.x) {
          const float x = Sh[e];
          s_V[(e % K) * LD + e / K] = x;
          sVs.put1((e % K) * LDKB + e / K, x);
        }
      }
    }
    // the state entering group i, stored after this phase's loads were issued
    store_group(i, lane_v);
    lds_barrier();

    // ---- the state's tiles back from the group state just stored (their
    // registers are free during the probe), issued first so that the round
    // trip overlaps the projections
    {
      const float* vkb = group_vk(i);
#pragma unroll
      for (int t = 0; t < TKV; ++t) {
        const int k0 = kv_row(t) * 16 + arow_(0), v = ctw * 16 + acol_();
        st[t] = *reinterpret_cast<const f4*>(vkb + (unsigned)(v * K + k0));
      }
    }

    // ---- projections; U = Vals w and the keys' parts stay in registers. The
    // wave's tiles go in groups of at most two, each group's four
    // accumulators becoming its gates in place before the next group starts.
    constexpr int TG = TPW < 2 ? TPW : 2;
    static_assert(TPW % TG == 0, "whole groups of tiles");
    f4 ut[TPW], bt[TPW], uu[TPW];
#pragma unroll
    for (int t0 = 0; t0 < TPW; t0 += TG) {
      f4 xg[TG];
#pragma unroll
      for (int u = 0; u < TG; ++u) ut[t0 + u] = bt[t0 + u] = uu[t0 + u] = xg[u] = f4_zero();
#pragma unroll
      for (int s = 0; s < NKS; ++s) {
        FR qk{}, qb, qw, qg;
        if constexpr (PRELOAD) {
          qk = pk[s]; qb = pb[s]; qw = pw[s]; qg = pg[s];
        } else {
          if (!MERGE) qk = Mma<E>::ld(kpH + s * KS);
          qb = Mma<E>::ld(bpH + s * KS);
          qw = Mma<E>::ld(wpH + s * KS);
          qg = Mma<E>::ld(gpH + s * KS);
        }
#pragma unroll
        for (int u = 0; u < TG; ++u) {
          const int t = t0 + u;
          int rt;
          if (!tile(t, rt)) continue;
          const SF fa = sVs.get((rt * 16 + rl) * LDKB + ko + s * KS);
          if (!MERGE) ut[t] = Mma<E>::mma(ut[t], fa, qk);
          bt[t] = Mma<E>::mma(bt[t], fa, qb);
          uu[t] = Mma<E>::mma(uu[t], fa, qw);
          xg[u] = Mma<E>::mma(xg[u], fa, qg);
        }
      }
#pragma unroll
      for (int u = 0; u < TG; ++u) {
        const int t = t0 + u;
        int rt;
        if (!tile(t, rt)) continue;
        float sg = 0.f;
#pragma unroll
        for (int r = 0; r < 4; ++r) sg += softplusf_(xg[u][r] - 4.f);
        sg += __shfl_xor(sg, 16, WAVE);
        sg += __shfl_xor(sg, 32, WAVE);
        if (lane < 16) s_gs[(wv / CTK) * K + ctw * 16 + lane] += sg;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int n = rt * 16 + arow_(r), v = ctw * 16 + acol_();
          bt[t][r] = sigmoidf_(bt[t][r] - 4.f);
          uu[t][r] = s_V[n * LD + v] * sigmoidf_(uu[t][r]);
        }
        if (!MERGE) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float q = ut[t][r] * ut[t][r];
            q = row16_sum(q);
            if (rl == 0) s_nrm[wv * N + rt * 16 + arow_(r)] += q;
          }
        }
      }
    }
    // ---- the next firing's snapshot, in flight through the rest of this one
    if (!MERGE && i + 1 < NF) load_snap(i + 1, lane_v, raw);
    lds_barrier();

    // ---- per-pair key norms and per-column decay, once each
    const size_t fo = (size_t)bh * NF + i;
    if (tid < K) {
      float x = 0.f;
#pragma unroll
      for (int p = 0; p < NPW; ++p) x += s_gs[p * K + tid];
      const float gm = expf(-x / (float)N);
      s_gam[tid] = gm;
      if (a.gam) a.gam[fo * K + tid] = gm;
    } else if (!MERGE && tid < K + N) {
      const int n = tid - K;
      float nr = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) nr += s_nrm[w * N + n];
      s_rn[n] = __builtin_amdgcn_rcpf(fmaxf(sqrtf(nr), 1e-12f));
    }
    lds_barrier();

    // ---- keys b and keys^T as split tiles, the backward's copies; S~ = e^g S
    // in registers and S~^T in LDS; the partial sums cleared for the next firing
    {
      // (bf16 with N % 32 == 0: AT in fragment order, as the reverse scan reads it)
      constexpr bool FRG = std::is_same<E, bf16>::value && N % 32 == 0;
      const SplitTile<E> KNo = split_at<E>(a.keysN ? a.keysN + fo * N * K : nullptr, N * K);
      const SplitTile<E> ATo = split_at<E>(a.AT ? a.AT + fo * K * N : nullptr, K * N);
      const int k = ctw * 16 + acol_();
      const float gk = s_gam[k];
#pragma unroll
      for (int t = 0; t < TPW; ++t) {
        int rt;
        if (!tile(t, rt)) continue;
        const int n0 = rt * 16 + arow_(0);
        f4 kv4, av4;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int n = n0 + r;
          const float key = MERGE ? ((n == k) ? 1.f : 0.f) : ut[t][r] * s_rn[n];
          kv4[r] = key;
          av4[r] = key * bt[t][r] * gk;
          sKB.put1(n * LDKB + k, key * bt[t][r]);
          if (a.keysN) KNo.put1(n * K + k, key);
        }
        sKT.put4(k * LDKT + n0, kv4);
        if (a.AT) ATo.put4(FRG ? frag_ofs(k, n0, N) : k * N + n0, av4);
      }
    }
    for (int e = tid; e < NW * N; e += blockDim.x) s_nrm[e] = 0.f;
    for (int e = tid; e < NPW * K; e += blockDim.x) s_gs[e] = 0.f;
#pragma unroll
    for (int t = 0; t < TKV; ++t) {
      const int k0 = kv_row(t) * 16 + arow_(0), v = ctw * 16 + acol_();
#pragma unroll
      for (int r = 0; r < 4; ++r) st[t][r] *= s_gam[k0 + r];
      sST.put4(v * LDST + k0, st[t]);
    }
    lds_barrier();

    // ---- Vn = U - (keys b) S~ on this wave's [N,V] tiles (their shared B
    // fragment loaded once per k-step)
    f4 vn[TPW];
#pragma unroll
    for (int t = 0; t < TPW; ++t) vn[t] = f4_zero();
#pragma unroll
    for (int s = 0; s < NKS; ++s) {
      const SF fb = sST.get((ctw * 16 + rl) * LDST + s * KS + ko);
#pragma unroll
      for (int t = 0; t < TPW; ++t) {
        int rt;
        if (!tile(t, rt)) continue;
        vn[t] = Mma<E>::mma(vn[t], sKB.get((rt * 16 + rl) * LDKB + s * KS + ko), fb);
      }
    }
#pragma unroll
    for (int t = 0; t < TPW; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) vn[t][r] = uu[t][r] - vn[t][r];
    lds_barrier();   // Vn^T replaces S~^T
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      int rt;
      if (!tile(t, rt)) continue;
      sVnT.put4((ctw * 16 + acol_()) * LDVN + rt * 16 + arow_(0), vn[t]);
    }
    lds_barrier();

    // ---- S = S~ + keys^T Vn (the shared B fragment loaded once per k-step)
#pragma unroll
    for (int s = 0; s < NSN; ++s) {
      const bool live = s * KS + ko < N;
      const SF fb = live ? sVnT.get((ctw * 16 + rl) * LDVN + s * KS + ko) : Mma<E>::szero();
#pragma unroll
      for (int t = 0; t < TKV; ++t) {
        const SF fa = live ? sKT.get((kv_row(t) * 16 + rl) * LDKT + s * KS + ko) : Mma<E>::szero();
        st[t] = Mma<E>::mma(st[t], fa, fb);
      }
    }
    lds_barrier();   // the next firing's Vals replace Vn^T
  }
  for (int j = NF; j < a.NG; ++j) store_group(j, lane);
  float* fb = a.fin + b * a.fin_sb + h * a.fin_sh;
#pragma unroll
  for (int t = 0; t < TKV; ++t) {
    const int k0 = kv_row(t) * 16 + acc_row(0), v = ctw * 16 + acc_col();
#pragma unroll
    for (int r = 0; r < 4; ++r) fb[(unsigned)((k0 + r) * V + v)] = st[t][r];
  }
}

template <typename E, int K, int N, bool MERGE>
static hipError_t launch_chain(const PromoteChainArgs& a, hipStream_t st) {
  const unsigned grid = (unsigned)(a.B * a.H);
  if (grid == 0) return hipSuccess;
  hipLaunchKernelGGL((promote_chain_kernel<E, K, N, MERGE>), dim3(grid), dim3(512), 0, st, a);
  return hipGetLastError();
}

template <typename E>
static hipError_t chain_dispatch(const PromoteChainArgs& a, int K, int N, bool merge, hipStream_t st) {
  if (merge) {
    if (K == 64 && N == 64) return launch_chain<E, 64, 64, true>(a, st);
    return hipErrorInvalidValue;
  }
#define NGDN_CH(KK, NN) \
  if (K == KK && N == NN) return launch_chain<E, KK, NN, false>(a, st);
  NGDN_CH(64, 16) NGDN_CH(64, 32) NGDN_CH(64, 64)
  NGDN_CH(128, 16) NGDN_CH(128, 32) NGDN_CH(128, 64)
#undef NGDN_CH
  return hipErrorInvalidValue;
}

bool promote_chain_supported(int K, int N, bool merge) {
  if (merge) return K == 64 && N == 64;
  return (K == 64 || K == 128) && (N == 16 || N == 32 || N == 64);
}

hipError_t promote_chain_fwd(const PromoteChainArgs& a, int dtype, int K, int N, bool merge,
                             hipStream_t st) {
  return dtype == NGDN_BF16 ? chain_dispatch<bf16>(a, K, N, merge, st)
                            : chain_dispatch<float>(a, K, N, merge, st);
}

}  // namespace ngdn
