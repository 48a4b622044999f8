// The sequential half of every level: a chain of delta-rule steps
//   Vn = U - A S,   S <- diag(gam) S + BT Vn
// run per (batch, head, 32-column slice of V) with the fp32 state held in
// registers across all steps.
//
// Level 0 (the state recurrence of fla's chunk_gdn2_fwd, reached from
// nested_gdn2/ops/chunk.py:236-248; semantics ops/naive.py:367-392): one step
// per chunk with A = W, BT = Kt^T, U = U, gam = e^gc_last.
// Levels >= 1 (ops/update_fwd.py:21-128): one step per firing with
// A = keys * b * e^g, BT = keys^T, U = values * w, gam = e^g, which is
// S' = e^g S - keys^T ((keys*b)(e^g S)) + keys^T (values*w).
//
// Columns of V never interact, so a workgroup owns BV = SCAN_BV of them and
// the grid is B*H*(V/BV), the slices of one (batch, head) placed on one XCD so
// they share its L2. Per step: the state slice is written (transposed, fp32)
// to LDS as the B operand of A S; Vn goes through LDS as the B operand of
// BT Vn. A, BT, U and gam do not depend on the state: each wave reads the
// rows it needs one step ahead into registers, so the loads of step j+1
// overlap step j. Every operand is derived (fp32); for bf16 inputs each
// product is three bf16 MFMAs on split operands.
#include "ngdn_kernels.h"

#ifndef SCAN_WAVES_128
#define SCAN_WAVES_128 4
#endif
#ifndef SCAN_LATE_STORES
#define SCAN_LATE_STORES 1
#endif

namespace ngdn {

// OUT (level 0): each step also forms the chunk's level-0 read
//   read0 = Qg S + Aqk Vn
// on the same tiles as Vn, with S^T and Vn^T already in LDS as the B
// operands (the state is on chip, so the output pass needs neither the state
// sequence nor Vn from HBM).
// FRM (bf16): bit 0, BT in fragment order (M % 32 == 0); bit 1, A (and, OUT,
// Qg and Aqk) too.
template <typename E, int K, int M, int BV, int NWV, bool OUT, int FRM>
__global__ __launch_bounds__(NWV * WAVE) void scan_fwd_kernel(ScanArgs a) {
  constexpr int CT = BV / 16;                 // column tiles
  constexpr int RTS = K / 16;                 // state row tiles
  constexpr int TPW = RTS * CT / NWV;         // state tiles per wave
  constexpr int TRT = (TPW + CT - 1) / CT;    // distinct state row tiles per wave
  constexpr int RTV = M / 16;                 // Vn row tiles
  // Vn tiles of a wave, p < NVP: when the waves cover the row tiles a whole
  // number of times (ONE_RT), tile g = wv + NWV p at rt = g % RTV, ct = g / RTV
  // (one row tile per wave); otherwise row tiles wv + NWV q, every column.
  constexpr int NVT = RTV * CT;
  constexpr int NVP = (NVT + NWV - 1) / NWV;
  constexpr bool ONE_RT = (NWV % RTV) == 0;
  constexpr int NAR = ONE_RT ? 1 : RTV / NWV; // A row tiles held per wave
  using ST = SplitTile<E>;
  constexpr int LDS_ST = K + ST::PAD;
  constexpr int LDS_VN = M + ST::PAD;
  constexpr int KS = Mma<E>::KS;
  constexpr int NSK = K / KS;                 // k-steps over K
  constexpr int NSM = (M + KS - 1) / KS;      // k-steps over M
  constexpr bool PADM = (M % KS) != 0;
  constexpr bool FRB = FRM & 1, FRA = FRM & 2;
  static_assert(TPW >= 1 && (TPW % CT == 0 || CT % TPW == 0),
                "state tiles of a wave: whole rows, or a part of one row");
  static_assert(ONE_RT || RTV % NWV == 0, "Vn row tiles spread evenly over the waves");
  // S^T and Vn^T, split once by their writers
  __shared__ __attribute__((aligned(16))) typename ST::T s_st[ST::NPLANE * BV * LDS_ST];
  __shared__ __attribute__((aligned(16))) typename ST::T s_vn[ST::NPLANE * BV * LDS_VN];
  const ST sST{s_st, BV * LDS_ST}, sVn{s_vn, BV * LDS_VN};

  const int V = a.V, S = a.S, H = a.H;
  const int nvt = V / BV;
  int vt, bh;
  xcd_split(blockIdx.x, gridDim.x, nvt, bh, vt);
  const int h = bh % H, b = bh / H;
  const int v0 = vt * BV;
  const int lane = lane_id(), wv = wave_id();
  if (gated_out(a.gate, b)) return;

  // state tiles of this wave: g = wv * TPW + i, rt = g / CT, ct = g % CT
  f4 st[TPW];
#pragma unroll
  for (int i = 0; i < TPW; ++i) {
    const int g = wv * TPW + i, rt = g / CT, ct = g % CT;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int k = rt * 16 + acc_row(r), v = v0 + ct * 16 + acc_col();
      st[i][r] = a.init ? a.init[b * a.init_sb + h * a.init_sh + (long long)k * V + v] : 0.f;
    }
  }

  const float* Ab = a.A + (size_t)bh * S * M * K;
  const float* Bb = a.BT + (size_t)bh * S * K * M;
  const float* Ub = a.U + (size_t)bh * S * M * V;
  const float* Gb = a.gam + (size_t)bh * S * K;

  // Operands of one step, read a step ahead: they do not depend on the state.
  typedef typename Mma<E>::SFrag SF;
  constexpr int RA = OUT ? NAR : 1, RQ = OUT ? NSK : 1, RP = OUT ? NSM : 1;
  struct Ops {
    SF a[NAR][NSK];             // A rows of this wave's Vn tiles
    float u[NVP][4];            // U at the Vn tiles
    SF bt[TRT][NSM];            // BT rows of this wave's state tiles
    f4 g[TRT];                  // gam at the state rows (one 16-byte load)
    SF qg[RA][RQ];              // OUT: Qg rows of this wave's tiles
    SF aq[RA][RP];              // OUT: Aqk rows
  };
  // p-th Vn tile of this wave: valid, row tile, column tile, A row set
  auto vn_tile = [&](int p, int& rt, int& ct) -> bool {
    if (ONE_RT) {
      const int g = wv + NWV * p;
      rt = g % RTV;
      ct = g / RTV;
      return g < NVT;
    }
    rt = wv + NWV * (p / CT);
    ct = p % CT;
    return true;
  };
  auto load = [&](int j, Ops& o) {
    const SplitTile<E> Aj = split_at<E>(Ab + (size_t)j * M * K, M * K);
    const float* Uj = Ub + (size_t)j * M * V;
    const SplitTile<E> Bj = split_at<E>(Bb + (size_t)j * K * M, K * M);
    const float* Gj = Gb + (size_t)j * K;
#pragma unroll
    for (int p = 0; p < NVP; ++p) {
      int rt, ct;
      if (vn_tile(p, rt, ct)) {
        if (ONE_RT ? p == 0 : p % CT == 0) {
          const int arow = (rt * 16 + (lane & 15)) * K + kofs<E>(lane);
#pragma unroll
          for (int s = 0; s < NSK; ++s)
            o.a[ONE_RT ? 0 : p / CT][s] = Aj.get(FRA ? frag_at(rt, s, K) : arow + s * KS);
          if constexpr (OUT) {
            const SplitTile<E> Qj = split_at<E>(a.Qg + ((size_t)bh * S + j) * M * K, M * K);
            const SplitTile<E> Pj = split_at<E>(a.Aqk + ((size_t)bh * S + j) * M * M, M * M);
            const int prow = (rt * 16 + (lane & 15)) * M + kofs<E>(lane);
#pragma unroll
            for (int s = 0; s < NSK; ++s)
              o.qg[ONE_RT ? 0 : p / CT][s] = Qj.get(FRA ? frag_at(rt, s, K) : arow + s * KS);
#pragma unroll
            for (int s = 0; s < NSM; ++s)
              o.aq[ONE_RT ? 0 : p / CT][s] = Pj.get(FRA ? frag_at(rt, s, M) : prow + s * KS);
          }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r)
          o.u[p][r] = Uj[(size_t)(rt * 16 + acc_row(r)) * V + v0 + ct * 16 + acc_col()];
      }
    }
#pragma unroll
    for (int t = 0; t < TRT; ++t) {
      const int rt = (wv * TPW) / CT + t;
      const int brow = (rt * 16 + (lane & 15)) * M + kofs<E>(lane);
#pragma unroll
      for (int s = 0; s < NSM; ++s)
        o.bt[t][s] = FRB ? Bj.get(frag_at(rt, s, M))
                        : (!PADM || s * KS + kofs<E>(lane) < M) ? Bj.get(brow + s * KS)
                                                                : Mma<E>::szero();
      o.g[t] = *reinterpret_cast<const f4*>(Gj + rt * 16 + acc_row(0));
    }
  };

  auto store_state = [&](int j) {
    const size_t base = (a.state_mode == 0 ? (size_t)bh * S + j
                                           : ((size_t)b * a.NG + j) * H + h) * K * V;
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      const int g = wv * TPW + i, rt = g / CT, ct = g % CT;
      const int k0 = rt * 16 + acc_row(0), vl = ct * 16 + acc_col(), v = v0 + vl;
      if (a.st_vk && (a.vk_every <= 1 || j % a.vk_every == 0))
        *reinterpret_cast<f4*>(a.st_vk + base + (size_t)v * K + k0) = st[i];
      if (a.st_kv) {
#pragma unroll
        for (int r = 0; r < 4; ++r) a.st_kv[base + (size_t)(k0 + r) * V + v] = st[i][r];
      }
    }
  };

  // Vn and (OUT) the read of a step are stored at the start of the next
  // step, beside the state entering it and ahead of that step's operand
  // loads: the vector memory pipe is in order, so stores issued after the
  // loads would wait for them to drain and hold the wave up mid-step.
  // (fp32 operands with K = 128 and M >= 64 keep the stores in place: the
  // held Vn tiles would not fit in their registers)
  constexpr bool DEFER = OUT || sizeof(E) == 2 || K < 128 || M < 64;
  // LATE: stores after the step's products instead of at its start
  constexpr bool LATE = SCAN_LATE_STORES && DEFER;
  f4 pvn[NVP], prd[OUT ? NVP : 1];
  auto flush_tile = [&](int jj, int p) {
      int rt, ct;
      if (vn_tile(p, rt, ct)) {
        const int m0 = rt * 16 + acc_row(0), vl = ct * 16 + acc_col();
        if (a.vnT)
          *reinterpret_cast<f4*>(a.vnT + (((size_t)bh * S + jj) * V + v0 + vl) * M + m0) = pvn[p];
        if (a.vn) {
          float* vp = a.vn + ((size_t)bh * S + jj) * M * V + (size_t)m0 * V + v0 + vl;
#pragma unroll
          for (int r = 0; r < 4; ++r) vp[(size_t)r * V] = pvn[p][r];
        }
        if constexpr (OUT) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int t = jj * M + rt * 16 + acc_row(r);
            if (t < a.T) a.read0[(((size_t)b * a.T + t) * H + h) * V + v0 + vl] = prd[p][r];
          }
        }
      }
  };
  auto flush = [&](int jj) {
#pragma unroll
    for (int p = 0; p < NVP; ++p) flush_tile(jj, p);
  };

  // One step with its operands already loaded.
  auto step = [&](int j, const Ops& cur) {
      // ---- the state, transposed, to LDS
#pragma unroll
      for (int i = 0; i < TPW; ++i) {
        const int g = wv * TPW + i, rt = g / CT, ct = g % CT;
        const int k0 = rt * 16 + acc_row(0), vl = ct * 16 + acc_col();
        sST.put4(vl * LDS_ST + k0, st[i]);
      }
      lds_barrier();

      // ---- Vn = U - A S (and, OUT, the read's Qg S on the same tiles)
      f4 rd[OUT ? NVP : 1];
#pragma unroll
      for (int p = 0; p < NVP; ++p) {
        int rt, ct;
        if (vn_tile(p, rt, ct)) {
          f4 acc = f4_zero();
          if constexpr (OUT) rd[p] = f4_zero();
          const int brow = (ct * 16 + (lane & 15)) * LDS_ST + kofs<E>(lane);
#pragma unroll
          for (int s = 0; s < NSK; ++s) {
            const auto fb = sST.get(brow + s * KS);
            acc = Mma<E>::mma(acc, cur.a[ONE_RT ? 0 : p / CT][s], fb);
            if constexpr (OUT) {
              rd[p] = Mma<E>::mma(rd[p], cur.qg[ONE_RT ? 0 : p / CT][s], fb);
            }
          }
          const int m0 = rt * 16 + acc_row(0), vl = ct * 16 + acc_col();
          f4 vn;
#pragma unroll
          for (int r = 0; r < 4; ++r) vn[r] = cur.u[p][r] - acc[r];
          sVn.put4(vl * LDS_VN + m0, vn);
          pvn[p] = vn;
          if constexpr (!DEFER) flush_tile(j, p);
        }
      }
      lds_barrier();

      // ---- OUT: read0 = Qg S + Aqk Vn for the chunk's rows in the sequence
      if constexpr (OUT) {
#pragma unroll
        for (int p = 0; p < NVP; ++p) {
          int rt, ct;
          if (vn_tile(p, rt, ct)) {
            const int brow = (ct * 16 + (lane & 15)) * LDS_VN + kofs<E>(lane);
#pragma unroll
            for (int s = 0; s < NSM; ++s) {
              rd[p] = Mma<E>::mma(rd[p], cur.aq[ONE_RT ? 0 : p / CT][s], sVn.get(brow + s * KS));
            }
            prd[p] = rd[p];
          }
        }
      }
      if constexpr (LATE) {
        // ---- this step's stores after its products, while the next step's
        // operand loads (issued before them) are in flight: the stores neither
        // hold the wave up behind those loads nor delay their completion. The
        // state registers still hold the state entering step j.
        store_state(j);
        flush(j);
      }

      // ---- S <- diag(gam) S + BT Vn
#pragma unroll
      for (int i = 0; i < TPW; ++i) {
        // t must be a compile-time index into the operand registers
        constexpr bool WHOLE = TPW % CT == 0;
        const int t = WHOLE ? i / CT : 0;
        const int ct = WHOLE ? i % CT : (wv * TPW + i) % CT;
#pragma unroll
        for (int r = 0; r < 4; ++r) st[i][r] *= cur.g[t][r];
        const int brow = (ct * 16 + (lane & 15)) * LDS_VN + kofs<E>(lane);
#pragma unroll
        for (int s = 0; s < NSM; ++s) {
          // M = 16 with 32-deep bf16 MFMAs: the upper half of the k range is zero
          const bool live = !PADM || (s * KS + kofs<E>(lane) < M);
          typename Mma<E>::SFrag fb = Mma<E>::szero();
          if (live) fb = sVn.get(brow + s * KS);
          st[i] = Mma<E>::mma(st[i], cur.bt[t][s], fb);
        }
      }
    // no barrier needed here: the next writes to s_st do not alias s_vn, and
    // the next writes to s_vn follow the next step's barrier
  };

  Ops nxt;
  // steps [j0, j1): the state registers start from init, the state entering j0
  const int j0 = a.j0, j1 = a.j1 > 0 ? a.j1 : S;
  if (j1 > j0) load(j0, nxt);
  for (int j = j0; j < j1; ++j) {
    const Ops cur = nxt;
    if constexpr (LATE) {
      // ---- the next step's operand loads first (the last step reloads its
      // own, so that no branch guards them); this step's stores follow its
      // products
      load(j + 1 < j1 ? j + 1 : j, nxt);
    } else {
      // ---- state entering step j (and the previous step's Vn and read) to
      // global, then the next step's operand loads
      store_state(j);
      if (DEFER && j > j0) flush(j - 1);
      if (j + 1 < j1) load(j + 1, nxt);
    }
    step(j, cur);
  }
  if (!LATE && DEFER && j1 > j0) flush(j1 - 1);
  if (a.state_mode == 1 && j1 == S) {
    for (int j = S; j < a.NG; ++j) store_state(j);
  }
#pragma unroll
  for (int i = 0; i < TPW; ++i) {
    const int g = wv * TPW + i, rt = g / CT, ct = g % CT;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int k = rt * 16 + acc_row(r), v = v0 + ct * 16 + acc_col();
      a.fin[b * a.fin_sb + h * a.fin_sh + (long long)k * V + v] = st[i][r];
    }
  }
}


// Waves per workgroup: four, one per SIMD. Eight (two per SIMD) leave each
// wave half the registers, less than a step's operands read ahead need.
template <int K> constexpr int scan_waves() { return K == 128 ? SCAN_WAVES_128 : 4; }

template <typename E, int K, int M, int BV>
static hipError_t launch_scan_bv(const ScanArgs& a, hipStream_t st) {
  constexpr int NWV = scan_waves<K>();
  const unsigned grid = (unsigned)(a.B * a.H * (a.V / BV));
  constexpr bool BF = std::is_same<E, bf16>::value;
  if (a.frag && !(BF && M % 32 == 0 && (a.frag == 1 || (a.frag == 3 && M == CH))))
    return hipErrorInvalidValue;
  // level 0's read is formed only by the chunk-step (M == CH) kernels whose
  // operand groups share one layout (frag 0 or 3)
  if (a.read0 && (M != CH || a.frag == 1)) return hipErrorInvalidValue;
  if constexpr (BF && M == CH) {
    if (a.frag == 3) {
      if (a.read0)
        hipLaunchKernelGGL((scan_fwd_kernel<E, K, M, BV, NWV, true, 3>), dim3(grid),
                           dim3(NWV * WAVE), 0, st, a);
      else
        hipLaunchKernelGGL((scan_fwd_kernel<E, K, M, BV, NWV, false, 3>), dim3(grid),
                           dim3(NWV * WAVE), 0, st, a);
      return hipGetLastError();
    }
  }
  if constexpr (BF && M % 32 == 0) {
    if (a.frag == 1) {
      hipLaunchKernelGGL((scan_fwd_kernel<E, K, M, BV, NWV, false, 1>), dim3(grid),
                         dim3(NWV * WAVE), 0, st, a);
      return hipGetLastError();
    }
  }
  if constexpr (M == CH) {
    if (a.read0) {
      hipLaunchKernelGGL((scan_fwd_kernel<E, K, M, BV, NWV, true, 0>), dim3(grid),
                         dim3(NWV * WAVE), 0, st, a);
      return hipGetLastError();
    }
  }
  hipLaunchKernelGGL((scan_fwd_kernel<E, K, M, BV, NWV, false, 0>), dim3(grid),
                     dim3(NWV * WAVE), 0, st, a);
  return hipGetLastError();
}

template <typename E, int K, int M>
static hipError_t launch_scan(const ScanArgs& a, hipStream_t st) {
  // Few (batch, head) pairs (a long sequence in a small batch): the bf16
  // matrix-core paths take 16-column slices, twice the workgroups with half
  // the products per step each; a step's operands are then read by twice as
  // many workgroups, which costs more than it saves once the grid fills the
  // chip.
  if constexpr (std::is_same<E, bf16>::value && M % 32 == 0) {
    if (a.frag && a.B * a.H * (a.V / SCAN_BV) <= SCAN_NARROW_GRID)
      return launch_scan_bv<E, K, M, 16>(a, st);
  }
  return launch_scan_bv<E, K, M, SCAN_BV>(a, st);
}

hipError_t scan_fwd(const ScanArgs& a, int dtype, int K, hipStream_t st) {
  if (a.V % SCAN_BV != 0) return hipErrorInvalidValue;
#define NGDN_SC(E, KK, MM) \
  if (K == KK && a.M == MM) return launch_scan<E, KK, MM>(a, st);
#define NGDN_SC_K(E, KK) NGDN_SC(E, KK, 16) NGDN_SC(E, KK, 32) NGDN_SC(E, KK, 64) NGDN_SC(E, KK, 128)
  if (dtype == NGDN_BF16) {
    NGDN_SC_K(bf16, 64) NGDN_SC_K(bf16, 128)
  } else {
    NGDN_SC_K(float, 64) NGDN_SC_K(float, 128)
  }
#undef NGDN_SC_K
#undef NGDN_SC
  return hipErrorInvalidValue;
}

}  // namespace ngdn
