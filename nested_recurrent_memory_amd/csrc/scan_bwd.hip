// Reverse of the delta-rule step chain (scan.hip), run per (batch, head,
// 32-column slice of V) with the fp32 state gradient in registers.
//
// Forward step: Vn = U - A S;  S' = diag(gam) S + BT Vn.  Given dS' (the
// gradient of the state after the step):
//   dVn = Bop dS'             (Bop = BT^T)
//   dS  = diag(gam) dS' - AT dVn      (AT = A^T)
// Level 0 (the reverse dh recurrence of the reference's vendored fla
// backward, nested_gdn2/ops/_vendor/common_chunk_delta_h.py:25-380) also
// carries the chunk's output o = Qg S + Aqk Vn with dO = mix_0 * do:
//   dVn += Aqk^T dO,   dS += Qg^T dO,
// and takes the promotion gradient of level 1 at every firing chunk: before
// the step of chunk n with (n+1) % f1 == 0 the injection inj[(n+1)/f1 - 1] is
// added -- the gradient of the state entering chunk n+1, which the reference
// hands to fla as dh_ext (ops/chunk.py:519-528).
// Levels >= 1 (ops/update_bwd.py:93-158): after group j's firing, the read
// gradient of the state entering group j joins: dS += d_states[j].
//
// Stores, per step (fp32): dS' (the gradient of the state after it) and dVn.
// Every operand but do is derived; for bf16 inputs each product is three bf16
// MFMAs on split operands. As in the forward scan, the slices of one (batch,
// head) share an XCD and each step's operands (which do not depend on the
// state gradient) are read one step ahead into registers.
#include "ngdn_kernels.h"

namespace ngdn {

// FRM (bf16, M % 32 == 0): bit 0, AT (and, level 0, QgT) in fragment order;
// bit 1, Bop (and, level 0, AqkT) too.
template <typename E, int K, int M, int FRM>
__global__ __launch_bounds__(256) void scan_bwd_kernel(ScanBwdArgs a) {
  constexpr int BV = SCAN_BV;
  constexpr int CT = BV / 16;
  constexpr int RTS = K / 16;
  constexpr int TPW = RTS * CT / 4;
  constexpr int TRT = TPW / CT;               // distinct state row tiles per wave
  constexpr int RTV = M / 16;
  constexpr int RPW = (RTV + 3) / 4;          // dVn row tiles per wave (at most)
  using ST = SplitTile<E>;
  constexpr int LDS_ST = K + ST::PAD;
  constexpr int LDS_VN = M + ST::PAD;
  constexpr int KS = Mma<E>::KS;
  constexpr int KPL = Mma<E>::KPL;
  constexpr int NSK = K / KS;
  constexpr int NSM = (M + KS - 1) / KS;
  constexpr bool PADM = (M % KS) != 0;
  constexpr bool FRB = FRM & 1, FRA = FRM & 2;
  constexpr int DOE = M * BV / 256;           // dO elements staged per thread
  static_assert(M != CH || (BV % DOE == 0 && 256 / (BV / DOE) == M && DOE % 8 == 0),
                "level 0: one token row slice per thread");
  static_assert(TPW % CT == 0, "state tiles of a wave come in whole rows");
  // dS'^T, dVn^T and (mix_0 dO)^T, split once by their writers
  __shared__ __attribute__((aligned(16))) typename ST::T s_dst[ST::NPLANE * BV * LDS_ST];
  __shared__ __attribute__((aligned(16))) typename ST::T s_dvn[ST::NPLANE * BV * LDS_VN];
  __shared__ __attribute__((aligned(16))) typename ST::T s_dot[ST::NPLANE * BV * LDS_VN];
  const ST sdS{s_dst, BV * LDS_ST}, sdV{s_dvn, BV * LDS_VN}, sdO{s_dot, BV * LDS_VN};

  const int V = a.V, S = a.S, H = a.H;
  const int nvt = V / BV;
  int vt, bh;
  xcd_split(blockIdx.x, gridDim.x, nvt, bh, vt);
  const int h = bh % H, b = bh / H;
  const int v0 = vt * BV;
  const int lane = lane_id(), wv = wave_id(), tid = threadIdx.x;
  const bool l0 = a.QgT != nullptr;

  f4 ds[TPW];
#pragma unroll
  for (int i = 0; i < TPW; ++i) {
    const int g = wv * TPW + i, rt = g / CT, ct = g % CT;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int k = rt * 16 + acc_row(r), v = v0 + ct * 16 + acc_col();
      ds[i][r] = a.d_final ? a.d_final[b * a.df_sb + h * a.df_sh + (long long)k * V + v] : 0.f;
    }
  }
  // values of a [K][V] fp32 array at this wave's state tiles
  auto read_kv = [&](const float* src, f4* out) {
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      const int g = wv * TPW + i, rt = g / CT, ct = g % CT;
#pragma unroll
      for (int r = 0; r < 4; ++r)
        out[i][r] = src[(size_t)(rt * 16 + acc_row(r)) * V + v0 + ct * 16 + acc_col()];
    }
  };
  auto dstates = [&](int j) {
    return a.d_states + (((size_t)b * a.NG + j) * H + h) * K * V;
  };
  if (a.d_states) {
    for (int j = a.NG - 1; j >= S; --j) {
      f4 x[TPW];
      read_kv(dstates(j), x);
#pragma unroll
      for (int i = 0; i < TPW; ++i) ds[i] += x[i];
    }
  }

  const float* Bb = a.Bop + (size_t)bh * S * M * K;
  const float* Ab = a.AT + (size_t)bh * S * K * M;
  const float* Gb = a.gam + (size_t)bh * S * K;
  const E* dob = l0 ? static_cast<const E*>(a.dout) + ((size_t)b * a.T * H + h) * V : nullptr;
  const E* mixb = l0 ? static_cast<const E*>(a.mix) + ((size_t)b * a.T * H + h) * a.L : nullptr;

  // Operands of one step, read a step ahead: they do not depend on the state gradient.
  typedef typename Mma<E>::SFrag SF;
  typedef E DV __attribute__((__vector_size__(DOE * sizeof(E))));
  struct Ops {
    SF bop[RPW][NSK];           // Bop rows of this wave's dVn tiles
    SF aqk[RPW][NSM];           // Aqk^T rows (level 0)
    SF at[TRT][NSM];            // A^T rows of this wave's state tiles
    SF qg[TRT][NSM];            // Qg^T rows (level 0)
    float g[TRT][4];
    DV dor;                     // do at this thread's staging slots (level 0), raw
    E dm;                       // and mix_0 of its token, raw: both are converted
                                // when staged, so the load is not waited for here
    f4 add[TPW];                // injection (level 0) or read gradient (upper) of the step
    bool has_add;
  };
  auto load = [&](int j, Ops& o) {
    const SplitTile<E> Bj = split_at<E>(Bb + (size_t)j * M * K, M * K);
    const SplitTile<E> Aj = split_at<E>(Ab + (size_t)j * K * M, K * M);
    const float* Gj = Gb + (size_t)j * K;
#pragma unroll
    for (int p = 0; p < RPW; ++p) {
      const int rt = wv + 4 * p;
      if (rt < RTV) {
        const int brow = (rt * 16 + (lane & 15)) * K + kofs<E>(lane);
#pragma unroll
        for (int s = 0; s < NSK; ++s) o.bop[p][s] = Bj.get(FRA ? frag_at(rt, s, K) : brow + s * KS);
        if (l0) {
          const SplitTile<E> Qj = split_at<E>(a.AqkT + ((size_t)bh * S + j) * M * M, M * M);
          const int qrow = (rt * 16 + (lane & 15)) * M + kofs<E>(lane);
#pragma unroll
          for (int s = 0; s < NSM; ++s) o.aqk[p][s] = Qj.get(FRA ? frag_at(rt, s, M) : qrow + s * KS);
        }
      }
    }
#pragma unroll
    for (int t = 0; t < TRT; ++t) {
      const int rt = (wv * TPW) / CT + t;
      const int arow = (rt * 16 + (lane & 15)) * M + kofs<E>(lane);
#pragma unroll
      for (int s = 0; s < NSM; ++s)
        o.at[t][s] = FRB ? Aj.get(frag_at(rt, s, M))
                        : (!PADM || s * KS + kofs<E>(lane) < M) ? Aj.get(arow + s * KS)
                                                                : Mma<E>::szero();
      if (l0) {
        const SplitTile<E> QTj = split_at<E>(a.QgT + ((size_t)bh * S + j) * K * M, K * M);
#pragma unroll
        for (int s = 0; s < NSM; ++s) o.qg[t][s] = QTj.get(FRB ? frag_at(rt, s, M) : arow + s * KS);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) o.g[t][r] = Gj[rt * 16 + acc_row(r)];
    }
    if (l0) {
      // DOE consecutive columns of one token per thread: one vector load
      const int c = tid / (BV / DOE), vl = (tid % (BV / DOE)) * DOE, t = j * M + c;
      if (t < a.T) {
        o.dor = *reinterpret_cast<const DV*>(dob + (size_t)t * H * V + v0 + vl);
        o.dm = mixb[(size_t)t * H * a.L];
      } else {
        o.dor = DV{};
        o.dm = E(0.f);
      }
    }
    // added before the step (level-0 injection) or after it (upper read gradient)
    o.has_add = false;
    if (a.inj && (j + 1) % a.inj_every == 0) {
      read_kv(a.inj + ((size_t)bh * a.inj_nf + (j + 1) / a.inj_every - 1) * K * V, o.add);
      o.has_add = true;
    } else if (a.d_states) {
      read_kv(dstates(j), o.add);
      o.has_add = true;
    }
  };

  // dVn of a step is stored at the start of the step after it, beside dS',
  // ahead of that step's operand loads: the vector memory pipe is in order,
  // so stores issued after the loads would wait for them to drain and hold
  // the wave up mid-step. (M = K = 128 keeps the stores in place: its
  // registers are already short.)
  constexpr bool DEFER = !(K == 128 && M == 128);
  f4 pdv[RPW][CT];
  auto store_dv = [&](int jj, int p, int ct) {
    const int rt = wv + 4 * p;
    const int m0 = rt * 16 + acc_row(0), vl = ct * 16 + acc_col();
    if (a.dVn) {
      float* o = a.dVn + ((size_t)bh * S + jj) * M * V + (size_t)m0 * V + v0 + vl;
#pragma unroll
      for (int r = 0; r < 4; ++r) o[(size_t)r * V] = pdv[p][ct][r];
    }
    if (a.dVnT)
      *reinterpret_cast<f4*>(a.dVnT + (((size_t)bh * S + jj) * V + v0 + vl) * M + m0) = pdv[p][ct];
  };
  auto flush_dv = [&](int jj) {
#pragma unroll
    for (int p = 0; p < RPW; ++p) {
      if (wv + 4 * p < RTV) {
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) store_dv(jj, p, ct);
      }
    }
  };

  Ops nxt;
  if (S > 0) load(S - 1, nxt);
  for (int j = S - 1; j >= 0; --j) {
    const Ops cur = nxt;
    if (a.inj && cur.has_add) {
#pragma unroll
      for (int i = 0; i < TPW; ++i) ds[i] += cur.add[i];
    }

    // ---- dS' (and the previous step's dVn) to global, then the next step's
    // operand loads
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      const int g = wv * TPW + i, rt = g / CT, ct = g % CT;
      const int k0 = rt * 16 + acc_row(0), vl = ct * 16 + acc_col();
      float* o = a.dSp + ((size_t)bh * S + j) * K * V + (size_t)k0 * V + v0 + vl;
#pragma unroll
      for (int r = 0; r < 4; ++r) o[(size_t)r * V] = ds[i][r];
    }
    if (DEFER && j + 1 < S) flush_dv(j + 1);
    if (j > 0) load(j - 1, nxt);

    // ---- dS' staged (transposed) as the B operand of Bop dS'
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      const int g = wv * TPW + i, rt = g / CT, ct = g % CT;
      const int k0 = rt * 16 + acc_row(0), vl = ct * 16 + acc_col();
      sdS.put4(vl * LDS_ST + k0, ds[i]);
    }
    if (l0) {
      const int c = tid / (BV / DOE), vl = (tid % (BV / DOE)) * DOE;
      const float m = to_f(cur.dm);
#pragma unroll
      for (int q = 0; q < DOE; ++q) sdO.put1((vl + q) * LDS_VN + c, to_f(cur.dor[q]) * m);
    }
    lds_barrier();

    // ---- dVn = Bop dS' (+ Aqk^T dO)
#pragma unroll
    for (int p = 0; p < RPW; ++p) {
      const int rt = wv + 4 * p;
      if (rt < RTV) {
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
          f4 acc = f4_zero();
          const int srow = (ct * 16 + (lane & 15)) * LDS_ST + kofs<E>(lane);
#pragma unroll
          for (int s = 0; s < NSK; ++s)
            acc = Mma<E>::mma(acc, cur.bop[p][s], sdS.get(srow + s * KS));
          if (l0) {
            const int orow = (ct * 16 + (lane & 15)) * LDS_VN + kofs<E>(lane);
#pragma unroll
            for (int s = 0; s < NSM; ++s)
              acc = Mma<E>::mma(acc, cur.aqk[p][s], sdO.get(orow + s * KS));
          }
          const int m0 = rt * 16 + acc_row(0), vl = ct * 16 + acc_col();
          sdV.put4(vl * LDS_VN + m0, acc);
          pdv[p][ct] = acc;
          if constexpr (!DEFER) store_dv(j, p, ct);
        }
      }
    }
    lds_barrier();

    // ---- dS = diag(gam) dS' - A^T dVn (+ Qg^T dO)
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      const int t = i / CT, ct = i % CT;
      f4 acc = f4_zero();
      const int vrow = (ct * 16 + (lane & 15)) * LDS_VN + kofs<E>(lane);
#pragma unroll
      for (int s = 0; s < NSM; ++s) {
        const bool live = !PADM || (s * KS + kofs<E>(lane) < M);
        typename Mma<E>::SFrag fb = Mma<E>::szero();
        if (live) fb = sdV.get(vrow + s * KS);
        acc = Mma<E>::mma(acc, cur.at[t][s], fb);
      }
      f4 qacc = f4_zero();
      if (l0) {
        const int orow = (ct * 16 + (lane & 15)) * LDS_VN + kofs<E>(lane);
#pragma unroll
        for (int s = 0; s < NSM; ++s)
          qacc = Mma<E>::mma(qacc, cur.qg[t][s], sdO.get(orow + s * KS));
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) ds[i][r] = cur.g[t][r] * ds[i][r] - acc[r] + qacc[r];
    }
    if (a.d_states && cur.has_add) {
#pragma unroll
      for (int i = 0; i < TPW; ++i) ds[i] += cur.add[i];
    }
    // s_dot and s_dvn are rewritten by the next step
    lds_barrier();
  }
  if (DEFER && S > 0) flush_dv(0);
  if (a.dinit) {
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      const int g = wv * TPW + i, rt = g / CT, ct = g % CT;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int k = rt * 16 + acc_row(r), v = v0 + ct * 16 + acc_col();
        a.dinit[b * a.di_sb + h * a.di_sh + (long long)k * V + v] = ds[i][r];
      }
    }
  }
}

template <typename E, int K, int M>
static hipError_t launch_scan_bwd(const ScanBwdArgs& a, hipStream_t st) {
  const unsigned grid = (unsigned)(a.B * a.H * (a.V / SCAN_BV));
  constexpr bool CAN = M % 32 == 0 && std::is_same<E, bf16>::value;
  if (a.frag && !(CAN && (a.frag == 1 || a.frag == 3))) return hipErrorInvalidValue;
  if (CAN && a.frag == 3)
    hipLaunchKernelGGL((scan_bwd_kernel<E, K, M, CAN ? 3 : 0>), dim3(grid), dim3(256), 0, st, a);
  else if (CAN && a.frag == 1)
    hipLaunchKernelGGL((scan_bwd_kernel<E, K, M, CAN ? 1 : 0>), dim3(grid), dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((scan_bwd_kernel<E, K, M, 0>), dim3(grid), dim3(256), 0, st, a);
  return hipGetLastError();
}

hipError_t scan_bwd(const ScanBwdArgs& a, int dtype, int K, hipStream_t st) {
  if (a.V % SCAN_BV != 0) return hipErrorInvalidValue;
  if (a.QgT && a.M != CH) return hipErrorInvalidValue;
#define NGDN_SB(E, KK, MM) \
  if (K == KK && a.M == MM) return launch_scan_bwd<E, KK, MM>(a, st);
#define NGDN_SB_K(E, KK) NGDN_SB(E, KK, 16) NGDN_SB(E, KK, 32) NGDN_SB(E, KK, 64) NGDN_SB(E, KK, 128)
  if (dtype == NGDN_BF16) {
    NGDN_SB_K(bf16, 64) NGDN_SB_K(bf16, 128)
  } else {
    NGDN_SB_K(float, 64) NGDN_SB_K(float, 128)
  }
#undef NGDN_SB_K
#undef NGDN_SB
  return hipErrorInvalidValue;
}

}  // namespace ngdn
