// Level-0 chunk backward: the gradients the reference takes from fla's
// chunk_gdn2_bwd helpers (nested_gdn2/ops/_vendor/gdn2_chunk_bwd.py:104-177:
// chunk_kda_bwd_dAv, chunk_gdn2_bwd_wy_dqkg_fused, chunk_gdn2_bwd_intra and
// the reverse chunk_local_cumsum), derived here from the chunk form
// (ops/naive.py:329-392):
//   Vn = U - W S,  o = Qg S + Aqk Vn,  S' = diag(gam) S + Kt^T Vn,
//   W = T X_w, U = T X_u, T = (I + A)^-1, X_w = b k e^gc, X_u = w v.
// Given dO = mix_0 do, the state gradient after the chunk dS' and dVn from the
// reverse scan:
//   state half (l0_bwd_state):
//     dQg = dO S^T, dW = -dVn S^T, dKt = Vn dS'^T, dAqk = mask(dO Vn^T),
//     dgam = rowsum(dS' * S)
//   intra half (l0_bwd_intra):
//     dX_u = T^T dVn, dX_w = T^T dW, dA = -mask(dX_w W^T + dX_u U^T)
//     (in one launch, l0_bwd: dX_w = -dX_u S^T, and as W S = U - Vn,
//     dA = -mask(dX_u Vn^T))
//     then through the decay products of A and Aqk, the gates and the
//     cumulative sum of g (reverse cumsum within the chunk).
#include "l0_common.h"

namespace ngdn {

template <typename E, int K, int V>
__global__ __launch_bounds__(256, sizeof(E) == 2 ? 3 : 2) void l0_bwd_state_kernel(L0BwdStateArgs a) {
  // Per (b, h, chunk) and half of K: output column k of dQg, dW and dKt needs
  // only row k of S and dS', so the two halves of K are two workgroups (on one
  // XCD) that each read their half of the state once. Within a workgroup, in
  // halves of V, S[khalf, vhalf] and dS'[khalf, vhalf] are staged once as
  // split tiles (each value split by one thread, not by every wave that reads
  // it) and every product accumulates over the halves; dgam, a plain fp32 dot
  // product, is summed from the fp32 values while they are staged. Wave w owns
  // rows 16 w of the chunk; the dAqk tiles J = khalf, khalf + 2 of its rows.
  constexpr int C = CH;
  constexpr int KH = K / 2;                    // rows of K per workgroup
  constexpr int VH = V > 64 ? 64 : V;          // columns of V per half
  constexpr int NHV = V / VH;
  using ST = SplitTile<E>;
  constexpr int LDH = VH + ST::PAD;
  constexpr int CTW = KH / 16;                 // column tiles per wave
  constexpr int KS = Mma<E>::KS;
  constexpr int KPL = Mma<E>::KPL;
  constexpr int NKH = VH / KS;                 // k-steps per half
  constexpr int Q4 = VH / 4;                   // 16-byte groups per staged row
  constexpr int SIT = KH * Q4 / 256;           // staged groups per thread per tensor
  static_assert(KH * Q4 % 256 == 0 && WAVE % Q4 == 0, "staging covers whole rows");
  typedef typename Mma<E>::SFrag SF;
  __shared__ __attribute__((aligned(16))) typename ST::T s_s[ST::NPLANE * KH * LDH];
  __shared__ __attribute__((aligned(16))) typename ST::T s_d[ST::NPLANE * KH * LDH];
  const ST sS{s_s, KH * LDH}, sD{s_d, KH * LDH};

  const int NT = a.NT, H = a.H, T = a.T;
  int unit, kh;
  xcd_split(blockIdx.x, gridDim.x, 2, unit, kh);
  const int n = unit % NT;
  const int bh = unit / NT;
  const int h = bh % H, b = bh / H;
  const int t0 = n * C;
  const int nvalid = min(C, T - t0);
  const int lane = lane_id(), tid = threadIdx.x;
  const int wv = __builtin_amdgcn_readfirstlane(wave_id());
  const size_t cix = (size_t)bh * NT + n;
  // uniform bases with 32-bit per-lane offsets (one address register each)
  const float* Sg = a.h + cix * K * V + (size_t)kh * KH * V;
  const float* dsp = a.dSp + cix * K * V + (size_t)kh * KH * V;

  // A fragments of this wave's 16 rows: dO (from do and mix_0), dVn, Vn
  const int ri = wv * 16 + (lane & 15);
  const int rc = min(ri, nvalid - 1);
  const E* dob = static_cast<const E*>(a.dout) + ((size_t)b * T * H + h) * V + (size_t)t0 * H * V;
  const unsigned dor = (unsigned)(rc * H * V);
  const float m0 = ri < nvalid ? to_f(static_cast<const E*>(a.mix)[((size_t)b * T + t0 + ri) * H * a.L + (size_t)h * a.L]) : 0.f;
  const float* dvnb = a.dVn + cix * C * V;
  const float* vnc = a.vn + cix * C * V;

  f4 aq[CTW], aw[CTW], ak[CTW], adq[2];
#pragma unroll
  for (int c = 0; c < CTW; ++c) { aq[c] = f4_zero(); aw[c] = f4_zero(); ak[c] = f4_zero(); }
  adq[0] = adq[1] = f4_zero();
  float dg[SIT];
#pragma unroll
  for (int i = 0; i < SIT; ++i) dg[i] = 0.f;

#pragma unroll 1
  for (int hv = 0; hv < NHV; ++hv) {
    const int vb = hv * VH;
    if (hv) lds_barrier();                   // the previous half's reads are done
    f4 xs[SIT], ys[SIT];
#pragma unroll
    for (int i = 0; i < SIT; ++i) {
      const int e = tid + 256 * i;
      const unsigned o = (unsigned)((e / Q4) * V + vb + (e % Q4) * 4);
      xs[i] = *reinterpret_cast<const f4*>(Sg + o);
      ys[i] = *reinterpret_cast<const f4*>(dsp + o);
    }
#pragma unroll
    for (int i = 0; i < SIT; ++i) {
      const int e = tid + 256 * i, k = e / Q4, c = (e % Q4) * 4;
      dg[i] += xs[i][0] * ys[i][0] + xs[i][1] * ys[i][1] + xs[i][2] * ys[i][2] + xs[i][3] * ys[i][3];
      sS.put4(k * LDH + c, xs[i]);
      sD.put4(k * LDH + c, ys[i]);
    }
    lds_barrier();
    // one k-step of A fragments live at a time
#pragma unroll
    for (int s = 0; s < NKH; ++s) {
      const int v0 = vb + s * KS + kofs<E>(lane);
      float x[KPL];
      ld_vals<E>(dob + (dor + (unsigned)v0), x);
      const SF fo = Mma<E>::makes([&](int e) { return x[e] * m0; });
      const SF fd = Mma<E>::ld(dvnb + (unsigned)(ri * V + v0));
      const SF fv = Mma<E>::ld(vnc + (unsigned)(ri * V + v0));
#pragma unroll
      for (int c = 0; c < CTW; ++c) {
        const int row = (c * 16 + (lane & 15)) * LDH + s * KS + kofs<E>(lane);
        const SF sb = sS.get(row);
        aq[c] = Mma<E>::mma(aq[c], fo, sb);
        aw[c] = Mma<E>::mma(aw[c], fd, sb);
        ak[c] = Mma<E>::mma(ak[c], fv, sD.get(row));
      }
      // dAqk = dO Vn^T, lower including the diagonal (Vn rows from global)
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const int J = kh + 2 * jj;
        if (J <= wv)
          adq[jj] = Mma<E>::mma(adq[jj], fo, Mma<E>::ld(vnc + (unsigned)((J * 16 + (lane & 15)) * V + v0)));
      }
    }
  }

  float* dQg = a.dQg + cix * C * K;
  float* dWT = a.dWT + cix * K * C;
  float* dKt = a.dKt + cix * C * K;
#pragma unroll
  for (int c = 0; c < CTW; ++c) {
    const int i0 = wv * 16 + acc_row(0), k = kh * KH + c * 16 + acc_col();
    f4 w;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      dQg[(i0 + r) * K + k] = aq[c][r];
      dKt[(i0 + r) * K + k] = ak[c][r];
      w[r] = -aw[c][r];
    }
    *reinterpret_cast<f4*>(dWT + k * C + i0) = w;
  }
  float* dAq = a.dAqk + cix * C * C;
#pragma unroll
  for (int jj = 0; jj < 2; ++jj) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = wv * 16 + acc_row(r), j = (kh + 2 * jj) * 16 + acc_col();
      dAq[i * C + j] = j <= i ? adq[jj][r] : 0.f;
    }
  }
  // dgam_k = sum_v dS'[k][v] S[k][v]: the Q4 threads of row k are adjacent lanes
#pragma unroll
  for (int i = 0; i < SIT; ++i) {
    float x = dg[i];
#pragma unroll
    for (int o = 1; o < Q4; o <<= 1) x += __shfl_xor(x, o, WAVE);
    const int e = tid + 256 * i;
    if (e % Q4 == 0) a.dgam[cix * K + kh * KH + e / Q4] = x;
  }
}

// FUSED (the l0_bwd entry point): the state half is phase 1 and part of
// phase 2 of this kernel instead of l0_bwd_state's outputs (see below).
template <typename E, int K, int V, bool FUSED>
__global__ __launch_bounds__(256, 2) void l0_bwd_intra_kernel(L0BwdIntraArgs a) {
  constexpr int C = CH;
  constexpr int NH = K > 64 ? 64 : K;          // columns per pass of the decay backward
  constexpr int NPASS = K / NH;
  constexpr int CTH = NH / 16;
  constexpr int GH = NH + GCP;                 // gc rows of one pass
  constexpr int LDI = NH + 16 / (int)sizeof(E); // staged input rows of one pass
  constexpr int LXK = K + 4, LXV = V + 4;      // fp32 rows
  constexpr int CTK = K / 16, CTV = V / 16;
  constexpr int KS = Mma<E>::KS;
  // bf16: each pass stages the chunk's k, b, q columns in LDS; fp32 (a
  // test-only path) reads them from global memory
  constexpr bool STAGE = !std::is_same<E, float>::value;
  typedef typename Mma<E>::SFrag SF;
  typedef Mma<float> MF;
  // Phases 2-3 hold dX_w, dX_u; phases 4-6 reuse the space for dA, dAqk and,
  // per pass, gc (later its gradient, in place) and the k, b, q columns.
  constexpr size_t SZ_X = sizeof(float) * C * (LXK + LXV);
  constexpr size_t SZ_DA = sizeof(float) * 2 * C * AT_LD;
  constexpr size_t SZ_G = sizeof(float) * C * GH;
  constexpr size_t SZ_IN = STAGE ? sizeof(E) * 3 * C * LDI : 0;
  constexpr size_t SZ_P = SZ_DA + SZ_G + SZ_IN;
  // fused phase 1: the chunk's Vn rows (split tile) and do rows (exact)
  using ST1 = SplitTile<E>;
  constexpr int LDV1 = V + ST1::PAD, LDO1 = V + 16 / (int)sizeof(E);
  constexpr size_t SZ_V1 = sizeof(typename ST1::T) * ST1::NPLANE * C * LDV1;
  constexpr size_t SZ_1 = FUSED ? SZ_V1 + sizeof(E) * C * LDO1 : 0;
  // fused phases 2-3: phase 1's Vn tile stays at the start until dA is formed
  // from it, dX_u follows it, and dX_w then takes the Vn tile's space (or
  // follows dX_u where that space is smaller); two-launch form: dX_w, dX_u
  constexpr size_t SZ_XW = sizeof(float) * C * LXK, SZ_XU = sizeof(float) * C * LXV;
  constexpr size_t OFF_XU = FUSED ? SZ_V1 : SZ_XW;
  constexpr size_t OFF_XW = (!FUSED || SZ_XW <= SZ_V1) ? 0 : SZ_V1 + SZ_XU;
  constexpr size_t SZ_2 = FUSED ? (OFF_XW ? OFF_XW + SZ_XW : SZ_V1 + SZ_XU) : SZ_X;
  constexpr size_t SZ_R0 = SZ_2 > SZ_P ? SZ_2 : SZ_P;
  constexpr size_t SZ_R = SZ_R0 > SZ_1 ? SZ_R0 : SZ_1;
  __shared__ __attribute__((aligned(16))) char smem[SZ_R + sizeof(float) * (6 * K + 256 + C)];
  float* s_dXw = reinterpret_cast<float*>(smem + OFF_XW);
  float* s_dXu = reinterpret_cast<float*>(smem + OFF_XU);
  float* s_dA = reinterpret_cast<float*>(smem);
  float* s_dQ = s_dA + C * AT_LD;
  float* s_g = reinterpret_cast<float*>(smem + SZ_DA);
  E* s_k = reinterpret_cast<E*>(smem + SZ_DA + SZ_G);
  E* s_b = s_k + C * LDI;
  E* s_q = s_b + C * LDI;
  float* s_gl = reinterpret_cast<float*>(smem + SZ_R);   // gc of the last row, per column
  float* s_col = s_gl + K;                                // [4 waves][K] column sums of phase 5
  float* s_part = s_col + 4 * K;                          // [256 / NH][NH] block sums of phase 6
  float* s_dgam = s_part + 256;                           // fused: dgam of the pass columns
  float* s_m0 = s_dgam + K;                               // fused: mix_0 of the chunk's rows

  const int NT = a.NT, H = a.H, T = a.T;
  const int nn = a.nn > 0 ? a.nn : NT;
  const int n = a.n0 + (int)(blockIdx.x % nn);
  const int bh = blockIdx.x / nn;
  const int h = bh % H, b = bh / H;
  const int lane = lane_id(), wv = wave_id(), tid = threadIdx.x;
  const size_t cix = (size_t)bh * NT + n;
  ChunkIn<E, K, V> in;
  in.init(a.q, a.k, a.v, a.g, a.b, a.w, b, h, n, T, H, a.L, a.scale);
  const int t0 = in.t0, nvalid = in.nvalid;
  for (int e = tid; e < 4 * K; e += 256) s_col[e] = 0.f;

  constexpr int CPW = CTK / 4;                 // fused: column tiles of K per wave
  constexpr int NKV = V / KS;                  // k-steps over V
  f4 daq[4];                                   // fused: this wave's dAqk tiles
  // fused: this wave's rows k of S as B fragments (8 consecutive v per lane),
  // loaded in phase 1 and used again for dX_w in phase 2
  SF fSk[FUSED ? CPW : 1][NKV];
  // fused: the chunk's Vn rows (split), phases 1-2
  const ST1 sVn1{reinterpret_cast<typename ST1::T*>(smem), C * LDV1};
  if constexpr (FUSED) {
    // ---- 1. the state half (what l0_bwd_state computes), from S = h, dS',
    // Vn, do and mix_0 of this chunk:
    //   dQg = dO S^T, dKt = Vn dS'^T  (to the workspaces, read back in phase 4)
    //   dgam = rowsum(dS' * S)        (LDS, read in phase 6)
    //   dAqk = mask(dO Vn^T)          (registers until phase 3)
    // with dO = mix_0 do (a row scale, applied to the products). Wave w owns
    // CPW column tiles (rows k of S and dS', loaded once per workgroup) and
    // every row of the chunk; Vn (split) and do (exact) rows come from LDS.
    // Phase 2 forms dX_w = T^T dW from dX_u instead of reading dW.
    static_assert(CTK % 4 == 0, "column tiles of K split over the 4 waves");
    E* s_do1 = reinterpret_cast<E*>(smem + SZ_V1);
    {
      constexpr int VE = 16 / (int)sizeof(E);
      constexpr int PV = C * V / 4 / 256, PO = C * V / VE / 256;
      static_assert(C * V / 4 % 256 == 0 && C * V / VE % 256 == 0, "whole groups per thread");
      typedef __attribute__((__vector_size__(16))) int v4i;
      const float* vnc = a.vn + cix * C * V;
      const E* dob = static_cast<const E*>(a.dout) + ((size_t)b * T * H + h) * V;
      f4 xv[PV];
      v4i xo[PO];
#pragma unroll
      for (int u = 0; u < PV; ++u) {
        const int e = tid + 256 * u;
        xv[u] = *reinterpret_cast<const f4*>(vnc + (size_t)(e / (V / 4)) * V + (e % (V / 4)) * 4);
      }
#pragma unroll
      for (int u = 0; u < PO; ++u) {
        const int e = tid + 256 * u, i = e / (V / VE), c = (e % (V / VE)) * VE;
        const v4i z = {0, 0, 0, 0};
        // rows past the end read the last valid row, then take zero (no branch)
        const v4i x = *reinterpret_cast<const v4i*>(dob + (size_t)(t0 + min(i, nvalid - 1)) * H * V + c);
        xo[u] = i < nvalid ? x : z;
      }
      if (tid < C)
        s_m0[tid] = tid < nvalid ? to_f(static_cast<const E*>(a.mix)[((size_t)b * T + t0 + tid) * H * a.L +
                                                                      (size_t)h * a.L])
                                 : 0.f;
#pragma unroll
      for (int u = 0; u < PV; ++u) {
        const int e = tid + 256 * u;
        sVn1.put4((e / (V / 4)) * LDV1 + (e % (V / 4)) * 4, xv[u]);
      }
#pragma unroll
      for (int u = 0; u < PO; ++u) {
        const int e = tid + 256 * u, i = e / (V / VE), c = (e % (V / VE)) * VE;
        *reinterpret_cast<v4i*>(s_do1 + i * LDO1 + c) = xo[u];
      }
    }
    lds_barrier();
    const float* Sg = a.h + cix * K * V;
    const float* dSg = a.dSp + cix * K * V;
    float* wq = a.wsQ + cix * C * K;
    float* wk = a.wsK + cix * C * K;
    constexpr int KPL = Mma<E>::KPL;
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
      const int ct = wv * CPW + c, kr = ct * 16 + (lane & 15);
      SF (&fS)[NKV] = fSk[c];
      SF fD[NKV];
      float dgp = 0.f;
#pragma unroll
      for (int s = 0; s < NKV; ++s) {
        const int v0 = s * KS + kofs<E>(lane);
        float x[KPL], y[KPL];
        ld_raw<KPL>(Sg + (size_t)kr * V + v0, x);
        ld_raw<KPL>(dSg + (size_t)kr * V + v0, y);
#pragma unroll
        for (int e = 0; e < KPL; ++e) dgp += x[e] * y[e];
        fS[s] = Mma<E>::makes([&](int e) { return x[e]; });
        fD[s] = Mma<E>::makes([&](int e) { return y[e]; });
      }
      // the four lane groups hold disjoint v ranges of the same row k
      dgp += __shfl_xor(dgp, 16, WAVE);
      dgp += __shfl_xor(dgp, 32, WAVE);
      if (lane < 16) s_dgam[ct * 16 + lane] = dgp;
#pragma unroll
      for (int rt = 0; rt < 4; ++rt) {
        const int ri1 = rt * 16 + (lane & 15);
        f4 aq = f4_zero(), ak = f4_zero();
#pragma unroll
        for (int s = 0; s < NKV; ++s) {
          const int v0 = s * KS + kofs<E>(lane);
          aq = Mma<E>::mma(aq, Mma<E>::ld(s_do1 + ri1 * LDO1 + v0), fS[s]);
          ak = Mma<E>::mma(ak, sVn1.get(ri1 * LDV1 + v0), fD[s]);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int i = rt * 16 + acc_row(r), k = ct * 16 + acc_col();
          wq[i * K + k] = aq[r] * s_m0[i];
          wk[i * K + k] = ak[r];
        }
      }
    }
    // this wave's rows of dAqk, tiles J <= w (lower including the diagonal)
#pragma unroll
    for (int J = 0; J < 4; ++J) {
      daq[J] = f4_zero();
      if (J <= wv) {
#pragma unroll
        for (int s = 0; s < NKV; ++s) {
          const int v0 = s * KS + kofs<E>(lane);
          daq[J] = Mma<E>::mma(daq[J], Mma<E>::ld(s_do1 + (wv * 16 + (lane & 15)) * LDO1 + v0),
                               sVn1.get((J * 16 + (lane & 15)) * LDV1 + v0));
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) daq[J][r] *= s_m0[wv * 16 + acc_row(r)];
    }
    lds_barrier();   // phase 2 reuses the space
  }

  // ---- 2. dX_u = T^T dVn, dX_w = T^T dW; wave w owns a quarter of the
  // columns of each and every row, so each wave splits the small T^T (all
  // of it) and only its quarter of dVn^T and dW^T, instead of every wave
  // splitting all of dVn^T and dW^T for its own rows
  const int ri = wv * 16 + (lane & 15);
  f4 dxw[CTK];
  {
    static_assert(CTV % 4 == 0 && CTK % 4 == 0, "column tiles split over 4 waves");
    SF tf[4][C / KS];
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      const float* tt = a.TT + cix * C * C + (size_t)(rt * 16 + (lane & 15)) * C + kofs<E>(lane);
#pragma unroll
      for (int s = 0; s < C / KS; ++s) tf[rt][s] = Mma<E>::ld(tt + s * KS);
    }
    auto product = [&](const float* srcT, int ncols, float* dst, int ldd) {
      const int cpw = ncols / 16 / 4;   // column tiles per wave
#pragma unroll
      for (int c = 0; c < cpw; ++c) {
        const int ct = wv * cpw + c;
        const float* br = srcT + (size_t)(ct * 16 + (lane & 15)) * C + kofs<E>(lane);
        SF fb[C / KS];
#pragma unroll
        for (int s = 0; s < C / KS; ++s) fb[s] = Mma<E>::ld(br + s * KS);
#pragma unroll
        for (int rt = 0; rt < 4; ++rt) {
          f4 acc = f4_zero();
#pragma unroll
          for (int s = 0; s < C / KS; ++s) acc = Mma<E>::mma(acc, tf[rt][s], fb[s]);
#pragma unroll
          for (int r = 0; r < 4; ++r) dst[(rt * 16 + acc_row(r)) * ldd + ct * 16 + acc_col()] = acc[r];
        }
      }
    };
    product(a.dVnT + cix * V * C, V, s_dXu, LXV);
    if constexpr (!FUSED) product(a.dWT + cix * K * C, K, s_dXw, LXK);
  }
  lds_barrier();
  // ---- 3. dA = -(dX_w W^T + dX_u U^T), strictly lower; tiles J <= w of this
  // wave's block-row, held until the space is free
  f4 dat[4];
  if constexpr (FUSED) {
    // With dX_w = -dX_u S^T (below) and W S = U - Vn, the sum in dA is
    // -dX_u (U - Vn)^T + dX_u U^T = dX_u Vn^T: formed from dX_u and phase 1's
    // Vn tile, with no W or U read and no cancellation of two large terms
#pragma unroll
    for (int J = 0; J < 4; ++J) {
      dat[J] = f4_zero();
      if (J <= wv) {
#pragma unroll
        for (int s = 0; s < NKV; ++s) {
          const int v0 = s * KS + kofs<E>(lane);
          dat[J] = Mma<E>::mma(dat[J], Mma<E>::ld(s_dXu + (wv * 16 + (lane & 15)) * LXV + v0),
                               sVn1.get((J * 16 + (lane & 15)) * LDV1 + v0));
        }
      }
    }
    if constexpr (OFF_XW == 0) lds_barrier();   // dX_w takes the Vn tile's space
    // dW = -dVn S^T, so dX_w = T^T dW = -(T^T dVn) S^T = -dX_u S^T: wave w
    // owns its CPW column tiles (rows k of S) over every row of the chunk,
    // the same rows it held as B fragments in phase 1 (kept, not re-read)
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
      const int ct = wv * CPW + c;
      const SF (&fS)[NKV] = fSk[c];
#pragma unroll
      for (int rt = 0; rt < 4; ++rt) {
        f4 acc = f4_zero();
#pragma unroll
        for (int s = 0; s < NKV; ++s)
          acc = Mma<E>::mma(acc, Mma<E>::ld(s_dXu + (rt * 16 + (lane & 15)) * LXV + s * KS + kofs<E>(lane)),
                            fS[s]);
#pragma unroll
        for (int r = 0; r < 4; ++r) s_dXw[(rt * 16 + acc_row(r)) * LXK + ct * 16 + acc_col()] = -acc[r];
      }
    }
    // s_dXw complete; phase 1's workspace stores complete and visible to the
    // whole workgroup (a barrier that also orders global memory)
    __syncthreads();
  }
  // this wave's rows of dX_w, kept for phase 5 (the space is reused from phase 4)
#pragma unroll
  for (int ct = 0; ct < CTK; ++ct)
#pragma unroll
    for (int r = 0; r < 4; ++r) dxw[ct][r] = s_dXw[(wv * 16 + acc_row(r)) * LXK + ct * 16 + acc_col()];

  if constexpr (!FUSED) {
    // W in split form (bf16: fragment order)
    const SplitTile<E> Ws = split_at<E>(a.W + cix * C * K, C * K);
    const float* Ug = a.U + cix * C * V;
#pragma unroll
    for (int J = 0; J < 4; ++J) {
      f4 acc = f4_zero();
      if (J <= wv) {
        // the tile's W and U rows from global first, all in flight together
        const int wr = (J * 16 + (lane & 15)) * K + kofs<E>(lane);
        const float* ur = Ug + (size_t)(J * 16 + (lane & 15)) * V + kofs<E>(lane);
        typename Mma<E>::SFrag wf[K / KS];
        float uf[V / KS][Mma<E>::KPL];
#pragma unroll
        for (int s = 0; s < K / KS; ++s)
          wf[s] = Ws.get(std::is_same<E, bf16>::value ? frag_at(J, s, K) : wr + s * KS);
#pragma unroll
        for (int s = 0; s < V / KS; ++s) ld_raw<Mma<E>::KPL>(ur + s * KS, uf[s]);
        __builtin_amdgcn_sched_barrier(0);   // keep the loads ahead of the products
        const float* xr = s_dXw + (wv * 16 + (lane & 15)) * LXK + kofs<E>(lane);
#pragma unroll
        for (int s = 0; s < K / KS; ++s) acc = Mma<E>::mma(acc, Mma<E>::ld(xr + s * KS), wf[s]);
        const float* xu = s_dXu + (wv * 16 + (lane & 15)) * LXV + kofs<E>(lane);
#pragma unroll
        for (int s = 0; s < V / KS; ++s)
          acc = Mma<E>::mma(acc, Mma<E>::ld(xu + s * KS),
                            Mma<E>::makes([&](int e) { return uf[s][e]; }));
      }
      dat[J] = acc;
    }
  }
  // dAqk, read before the dv/dw stores
  constexpr int DQE = FUSED ? 1 : C * C / 256;
  float dqv[DQE];
  if constexpr (!FUSED) {
#pragma unroll
    for (int u = 0; u < DQE; ++u) dqv[u] = a.dAqk[cix * C * C + tid + 256 * u];
  }

  // dv = dX_u * w, dw = dX_u * v: 16-byte rows, all loads of a thread ahead of its stores
  {
    constexpr int VE = ChunkIn<E, K, V>::VE;
    constexpr int PER = C * V / VE / 256;
    static_assert(C * V / VE % 256 == 0, "whole 16-byte groups per thread");
    E* dvo = static_cast<E*>(a.dv) + ((size_t)b * T * H + h) * V;
    E* dwo = static_cast<E*>(a.dw) + ((size_t)b * T * H + h) * V;
    // raw until used, so no load waits where it is issued
    typename ChunkIn<E, K, V>::R16 wr16[PER], vr16[PER];
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int e = tid + 256 * q, i = e / (V / VE), c = (e % (V / VE)) * VE;
      wr16[q] = in.raw16(in.w, in.rowV, i, c);
      vr16[q] = in.raw16(in.v, in.rowV, i, c);
    }
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int e = tid + 256 * q, i = e / (V / VE), c = (e % (V / VE)) * VE;
      float wx[VE], vx[VE];
      ChunkIn<E, K, V>::raw16_vals(wr16[q], wx);
      ChunkIn<E, K, V>::raw16_vals(vr16[q], vx);
      if (i < nvalid) {
        typedef E EV __attribute__((__vector_size__(16)));
        EV dvv, dwv;
#pragma unroll
        for (int j = 0; j < VE; ++j) {
          const float x = s_dXu[i * LXV + c + j];
          dvv[j] = from_f<E>(x * wx[j]);
          dwv[j] = from_f<E>(x * vx[j]);
        }
        *reinterpret_cast<EV*>(dvo + (size_t)(t0 + i) * H * V + c) = dvv;
        *reinterpret_cast<EV*>(dwo + (size_t)(t0 + i) * H * V + c) = dwv;
      }
    }
  }

  lds_barrier();
#pragma unroll
  for (int J = 0; J < 4; ++J) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = wv * 16 + acc_row(r), j = J * 16 + acc_col();
      s_dA[i * AT_LD + j] = (j < i) ? -dat[J][r] : 0.f;
    }
  }
  if constexpr (FUSED) {
#pragma unroll
    for (int J = 0; J < 4; ++J)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = wv * 16 + acc_row(r), j = J * 16 + acc_col();
        s_dQ[i * AT_LD + j] = (J <= wv && j <= i) ? daq[J][r] : 0.f;
      }
  } else {
#pragma unroll
    for (int u = 0; u < DQE; ++u) {
      const int e = tid + 256 * u;
      s_dQ[(e / C) * AT_LD + e % C] = dqv[u];
    }
  }

  const int R0 = 16 * wv;
  const float* dQg = (FUSED ? a.wsQ : a.dQg) + cix * C * K;
  const float* dKt = (FUSED ? a.wsK : a.dKt) + cix * C * K;
  const size_t tok = (size_t)b * T * H + h;
  E* dqo = static_cast<E*>(a.dq) + tok * a.L * K;
  E* dko = static_cast<E*>(a.dk) + tok * K;
  E* dbo = static_cast<E*>(a.db) + tok * K;
  float* dgo = a.dg + tok * K;

  // Inputs of one pass (NH columns from c0): g for the in-chunk cumulative
  // sum and, for bf16, the k, b, q columns. They are read into registers ahead
  // of their pass (the first before the loop, the next one before the current
  // pass's output stores) and written to LDS at the top of the pass.
  constexpr int TPC = 256 / NH, SEG = C / TPC;      // cumsum: threads per column, rows each
  constexpr int SEGS = NH * (int)sizeof(E) / 16;    // 16-byte groups per staged row
  constexpr int SI = STAGE ? (C * SEGS + 255) / 256 : 1;
  static_assert(!STAGE || C * SEGS % 256 == 0, "whole groups per thread");
  typedef __attribute__((__vector_size__(16))) int v4i;
  struct PassIn { float g[SEG]; v4i k[SI], b[SI], q[SI]; };
  auto pass_load = [&](int p, PassIn& x) {
    const int c0 = p * NH, col = tid / TPC, part = tid % TPC;
#pragma unroll
    for (int r = 0; r < SEG; ++r) {
      const int i = part * SEG + r;
      x.g[r] = i < nvalid ? in.g[(size_t)(t0 + i) * in.rowK + c0 + col] : 0.f;
    }
    if constexpr (STAGE) {
#pragma unroll
      for (int u = 0; u < SI; ++u) {
        const int e = tid + 256 * u, i = e / SEGS, c = (e % SEGS) * (16 / (int)sizeof(E));
        const v4i z = {0, 0, 0, 0};
        const bool live = i < nvalid;
        x.k[u] = live ? *reinterpret_cast<const v4i*>(in.k + (size_t)(t0 + i) * in.rowK + c0 + c) : z;
        x.b[u] = live ? *reinterpret_cast<const v4i*>(in.b + (size_t)(t0 + i) * in.rowK + c0 + c) : z;
        x.q[u] = live ? *reinterpret_cast<const v4i*>(in.q + (size_t)(t0 + i) * in.rowQ + c0 + c) : z;
      }
    }
  };
  auto pass_store = [&](int p, const PassIn& x) {
    const int c0 = p * NH, col = tid / TPC, part = tid % TPC;
    float y[SEG];
#pragma unroll
    for (int r = 0; r < SEG; ++r) y[r] = x.g[r];
#pragma unroll
    for (int r = 1; r < SEG; ++r) y[r] += y[r - 1];
    const int base = lane & ~(TPC - 1);
    float off = 0.f;
#pragma unroll
    for (int q = 0; q < TPC - 1; ++q) {
      const float t = __shfl(y[SEG - 1], base + q, WAVE);
      if (q < part) off += t;
    }
#pragma unroll
    for (int r = 0; r < SEG; ++r) s_g[(part * SEG + r) * GH + col] = y[r] + off;
    if (part == TPC - 1) s_gl[c0 + col] = y[SEG - 1] + off;
    if constexpr (STAGE) {
#pragma unroll
      for (int u = 0; u < SI; ++u) {
        const int e = tid + 256 * u, i = e / SEGS, c = (e % SEGS) * (16 / (int)sizeof(E));
        *reinterpret_cast<v4i*>(s_k + i * LDI + c) = x.k[u];
        *reinterpret_cast<v4i*>(s_b + i * LDI + c) = x.b[u];
        *reinterpret_cast<v4i*>(s_q + i * LDI + c) = x.q[u];
      }
    }
  };
  PassIn pin;
  pass_load(0, pin);

#pragma unroll
  for (int p = 0; p < NPASS; ++p) {
    const int c0 = p * NH;
    auto KV = [&](int i, int kl) -> float {
      if constexpr (STAGE) return to_f(s_k[i * LDI + kl]); else return in.K_(i, c0 + kl);
    };
    auto BV = [&](int i, int kl) -> float {
      if constexpr (STAGE) return to_f(s_b[i * LDI + kl]); else return in.B_(i, c0 + kl);
    };
    auto QV = [&](int i, int kl) -> float {
      if constexpr (STAGE) return to_f(s_q[i * LDI + kl]); else return in.Q_(i, c0 + kl);
    };

    // ---- 4. this pass's gc and input columns
    pass_store(p, pin);
    lds_barrier();
    const bool safe = block_safe<NH, GH>(s_g, wv);
    // the state half's dQg, dKt for phase 5, read now so that the loads overlap
    // phases 4a-4b (and precede this pass's stores: mixed outstanding loads and
    // stores would make every load wait for all of them)
    float gqa[CTH][4], gka[CTH][4];
#pragma unroll
    for (int ct = 0; ct < CTH; ++ct)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = R0 + acc_row(r), kc = c0 + ct * 16 + acc_col();
        gqa[ct][r] = dQg[i * K + kc];
        gka[ct][r] = dKt[i * K + kc];
      }

    // ---- 4a. d(bk) and dq-hat from A and Aqk, rows of block-row I = w
    //   sum_j dA_ij k_j e^(gc_i - gc_j) = e^(gc_i - gc_r) sum_j dA_ij [k_j e^(gc_r - gc_j)]
    // on fp32 MFMA: these sums cancel against those of 4b inside dg
    f4 dbk[CTH], dqa[CTH];
#pragma unroll
    for (int ct = 0; ct < CTH; ++ct) { dbk[ct] = f4_zero(); dqa[ct] = f4_zero(); }
    {
      const int jlim = safe ? R0 + 16 : R0;     // unsafe: diagonal block done exactly below
      for (int j0 = 0; j0 < jlim; j0 += MF::KS) {
        const int j = j0 + (lane >> 4);
        const float fa = s_dA[ri * AT_LD + j], fq = s_dQ[ri * AT_LD + j];
#pragma unroll
        for (int ct = 0; ct < CTH; ++ct) {
          const int kl = ct * 16 + (lane & 15);
          const float fb = KV(j, kl) * fexp(fminf(s_g[R0 * GH + kl] - s_g[j * GH + kl], 88.f));
          dbk[ct] = MF::mma(dbk[ct], fa, fb);
          dqa[ct] = MF::mma(dqa[ct], fq, fb);
        }
      }
#pragma unroll
      for (int ct = 0; ct < CTH; ++ct) {
        const int kl = ct * 16 + acc_col();
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int i = R0 + acc_row(r);
          const float f = fexp(s_g[i * GH + kl] - s_g[R0 * GH + kl]);
          float xb = dbk[ct][r] * f, xq = dqa[ct][r] * f;
          if (!safe) {
            for (int j = R0; j <= i; ++j) {
              const float d = KV(j, kl) * fexp(fminf(s_g[i * GH + kl] - s_g[j * GH + kl], 0.f));
              if (j < i) xb += s_dA[i * AT_LD + j] * d;
              xq += s_dQ[i * AT_LD + j] * d;
            }
          }
          dbk[ct][r] = xb;
          dqa[ct][r] = xq;
        }
      }
    }

    // ---- 4b. dk from A and Aqk, rows j of block J = w:
    //   sum_i (dA_ij bk_i + dAqk_ij q_i) e^(gc_i - gc_j)
    //   = e^(gc_e - gc_j) sum_i (...) e^(gc_i - gc_e),  e = last row of block J
    f4 dka[CTH];
#pragma unroll
    for (int ct = 0; ct < CTH; ++ct) dka[ct] = f4_zero();
    {
      const int RE = R0 + 15;
      const int ilo = safe ? R0 : R0 + 16;       // unsafe: diagonal block done exactly below
      const int rj = R0 + (lane & 15);
      for (int i0 = ilo; i0 < C; i0 += MF::KS) {
        const int i = i0 + (lane >> 4);
        const float fa = s_dA[i * AT_LD + rj], fq = s_dQ[i * AT_LD + rj];
#pragma unroll
        for (int ct = 0; ct < CTH; ++ct) {
          const int kl = ct * 16 + (lane & 15);
          const float d = fexp(fminf(s_g[i * GH + kl] - s_g[RE * GH + kl], 88.f));
          dka[ct] = MF::mma(dka[ct], fa, BV(i, kl) * KV(i, kl) * d);
          dka[ct] = MF::mma(dka[ct], fq, QV(i, kl) * in.scale * d);
        }
      }
#pragma unroll
      for (int ct = 0; ct < CTH; ++ct) {
        const int kl = ct * 16 + acc_col();
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int j = R0 + acc_row(r);
          float x = dka[ct][r] * fexp(s_g[RE * GH + kl] - s_g[j * GH + kl]);
          if (!safe) {
            for (int i = j; i < R0 + 16; ++i) {
              const float d = fexp(fminf(s_g[i * GH + kl] - s_g[j * GH + kl], 0.f));
              x += (s_dA[i * AT_LD + j] * BV(i, kl) * KV(i, kl) +
                    s_dQ[i * AT_LD + j] * QV(i, kl) * in.scale) * d;
            }
          }
          dka[ct][r] = x;
        }
      }
    }
    lds_barrier();   // the cumulative-decay gradient overwrites gc in place

    // ---- 5. assemble dq, dk, db and the cumulative-decay gradient
#pragma unroll
    for (int ct = 0; ct < CTH; ++ct) {
      const int kl = ct * 16 + acc_col(), kc = c0 + kl;
      const float glast = s_gl[kc];
      float colsum = 0.f;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = R0 + acc_row(r);
        const float gcv = s_g[i * GH + kl];
        const float eg = fexp(gcv), ekt = fexp(glast - gcv);
        const float bi = BV(i, kl), ki = KV(i, kl), qh = QV(i, kl) * in.scale;
        const float gq = gqa[ct][r], gk = gka[ct][r];
        const float xw = dxw[p * CTH + ct][r];
        const float dqh = dqa[ct][r] + gq * eg;
        const float db_ = dbk[ct][r] * ki + xw * ki * eg;
        const float dk_ = dka[ct][r] + dbk[ct][r] * bi + xw * bi * eg + gk * ekt;
        const float dgc = bi * ki * dbk[ct][r] + qh * dqa[ct][r] - ki * dka[ct][r] +
                          xw * bi * ki * eg + gq * qh * eg - gk * ki * ekt;
        colsum += gk * ki * ekt;
        s_g[i * GH + kl] = dgc;
        if constexpr (STAGE) {
          // in place of this element's q, k, b (read above, by this thread only)
          s_q[i * LDI + kl] = from_f<E>(dqh * in.scale);
          s_k[i * LDI + kl] = from_f<E>(dk_);
          s_b[i * LDI + kl] = from_f<E>(db_);
        } else if (i < nvalid) {
          dqo[(size_t)(t0 + i) * H * a.L * K + kc] = from_f<E>(dqh * in.scale);
          dko[(size_t)(t0 + i) * H * K + kc] = from_f<E>(dk_);
          dbo[(size_t)(t0 + i) * H * K + kc] = from_f<E>(db_);
        }
      }
      colsum += __shfl_xor(colsum, 16, WAVE);
      colsum += __shfl_xor(colsum, 32, WAVE);
      if (lane < 16) s_col[wv * K + kc] = colsum;   // one slot per wave, added in wave order
    }
    lds_barrier();
    if (p + 1 < NPASS) pass_load(p + 1, pin);   // ahead of this pass's stores
    if constexpr (STAGE) {
      // dq, dk, db leave as 16-byte rows from the k, b, q columns' space
      constexpr int VE = 16 / (int)sizeof(E), SEG = NH / VE;
      typedef E EV __attribute__((__vector_size__(16)));
      for (int e = tid; e < 3 * C * SEG; e += 256) {
        const int which = e / (C * SEG), i = (e / SEG) % C, c = (e % SEG) * VE;
        if (i < nvalid) {
          const E* src = (which == 0 ? s_q : which == 1 ? s_k : s_b) + i * LDI + c;
          E* dst = which == 0 ? dqo + (size_t)(t0 + i) * H * a.L * K
                 : (which == 1 ? dko : dbo) + (size_t)(t0 + i) * H * K;
          *reinterpret_cast<EV*>(dst + c0 + c) = *reinterpret_cast<const EV*>(src);
        }
      }
    }

    // ---- 6. dg = reverse cumsum of dgc within the chunk; gc_last also feeds
    // every Kt and gam. Column col of this pass, rows in NB blocks of RB: each
    // thread sums its block, then runs through it from the sum of the blocks
    // after it.
    {
      constexpr int NB = 256 / NH, RB = C / NB;
      static_assert(256 % NH == 0 && C % NB == 0, "whole row blocks per column");
      const int col = tid % NH, blk = tid / NH, kc = c0 + col;
      float part = 0.f;
#pragma unroll
      for (int i = 0; i < RB; ++i) part += s_g[(blk * RB + i) * GH + col];
      s_part[blk * NH + col] = part;
      lds_barrier();
      float run = ((s_col[kc] + s_col[K + kc]) + s_col[2 * K + kc]) + s_col[3 * K + kc];
      run += (FUSED ? s_dgam[kc] : a.dgam[cix * K + kc]) * fexp(s_gl[kc]);
      for (int b2 = NB - 1; b2 > blk; --b2) run += s_part[b2 * NH + col];
#pragma unroll
      for (int i = RB - 1; i >= 0; --i) {
        const int row = blk * RB + i;
        run += s_g[row * GH + col];
        if (row < nvalid) dgo[(size_t)(t0 + row) * H * K + kc] = run;
      }
    }
    lds_barrier();   // the next pass restages gc and the inputs
  }
}

template <typename E, int K, int V>
static hipError_t launch_l0_bwd_state(const L0BwdStateArgs& a, hipStream_t st) {
  // two workgroups (halves of K) per chunk-head
  const unsigned grid = (unsigned)(2 * a.B * a.H * a.NT);
  hipLaunchKernelGGL((l0_bwd_state_kernel<E, K, V>), dim3(grid), dim3(256), 0, st, a);
  return hipGetLastError();
}

template <typename E, int K, int V, bool FUSED>
static hipError_t launch_l0_bwd_intra(const L0BwdIntraArgs& a, hipStream_t st) {
  const unsigned grid = (unsigned)(a.B * a.H * (a.nn > 0 ? a.nn : a.NT));
  hipLaunchKernelGGL((l0_bwd_intra_kernel<E, K, V, FUSED>), dim3(grid), dim3(256), 0, st, a);
  return hipGetLastError();
}

hipError_t l0_bwd_state(const L0BwdStateArgs& a, int dtype, int K, int V, hipStream_t st) {
#define NGDN_BS(E, KK, VV) \
  if (K == KK && V == VV) return launch_l0_bwd_state<E, KK, VV>(a, st);
  if (dtype == NGDN_BF16) {
    NGDN_BS(bf16, 64, 64) NGDN_BS(bf16, 64, 128) NGDN_BS(bf16, 128, 64) NGDN_BS(bf16, 128, 128)
  } else {
    NGDN_BS(float, 64, 64) NGDN_BS(float, 64, 128) NGDN_BS(float, 128, 64) NGDN_BS(float, 128, 128)
  }
#undef NGDN_BS
  return hipErrorInvalidValue;
}

template <bool FUSED>
static hipError_t l0_bwd_intra_dispatch(const L0BwdIntraArgs& a, int dtype, int K, int V,
                                        hipStream_t st) {
#define NGDN_BI(E, KK, VV) \
  if (K == KK && V == VV) return launch_l0_bwd_intra<E, KK, VV, FUSED>(a, st);
  if (dtype == NGDN_BF16) {
    NGDN_BI(bf16, 64, 64) NGDN_BI(bf16, 64, 128) NGDN_BI(bf16, 128, 64) NGDN_BI(bf16, 128, 128)
  } else {
    NGDN_BI(float, 64, 64) NGDN_BI(float, 64, 128) NGDN_BI(float, 128, 64) NGDN_BI(float, 128, 128)
  }
#undef NGDN_BI
  return hipErrorInvalidValue;
}

hipError_t l0_bwd_intra(const L0BwdIntraArgs& a, int dtype, int K, int V, hipStream_t st) {
  return l0_bwd_intra_dispatch<false>(a, dtype, K, V, st);
}

hipError_t l0_bwd_fused(const L0BwdIntraArgs& a, int dtype, int K, int V, hipStream_t st) {
  return l0_bwd_intra_dispatch<true>(a, dtype, K, V, st);
}

}  // namespace ngdn
