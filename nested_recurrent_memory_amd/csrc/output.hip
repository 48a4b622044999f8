// Output of the op for one (batch, head, chunk): level 0's read from its chunk
// terms, every upper level's read with the state its group started with, and
// the per-token mix, written once (ops/chunk.py:129-156 read_level and the
// accumulation at :250-251,285-286; ops/naive.py:376-390).
//   o = mix_0 (Qg h_n + Aqk Vn) + sum_{l>=1} mix_l (scale q_l) S_l[group]
// Each product runs on MFMA with the right operand staged in LDS as a split
// tile (each value split once, by the thread that stages it) and the left
// operand's rows read from global by the wave that owns them; wave w owns
// output rows 16w..16w+15.
#include "ngdn_kernels.h"

namespace ngdn {

template <typename E, int K, int V>
__global__ __launch_bounds__(256) void output_fwd_kernel(OutputArgs a) {
  constexpr int C = CH;
  using ST = SplitTile<E>;
  // states are staged 64 rows of K at a time (a 37 KB tile)
  constexpr int KH = K > 64 ? 64 : K;
  constexpr int LD = KH + ST::PAD;
  constexpr int LDC = C + ST::PAD;
  constexpr int LDM = LD > LDC ? LD : LDC;
  constexpr int CTV = V / 16;
  constexpr int KS = Mma<E>::KS;
  __shared__ __attribute__((aligned(16))) typename ST::T s_b[ST::NPLANE * V * LDM];
  const ST sB{s_b, V * LDM};

  const int NT = a.NT, H = a.H, T = a.T, L = a.L;
  int n, bh;   // all chunks of one (batch, head) on one XCD: groups share states in its L2
  xcd_split(blockIdx.x, gridDim.x, NT, bh, n);
  const int h = bh % H, b = bh / H;
  const int t0 = n * C;
  const int nvalid = min(C, T - t0);
  const int lane = lane_id(), wv = wave_id(), tid = threadIdx.x;
  const size_t cix = ((size_t)bh * NT + n);
  const int ri = wv * 16 + (lane & 15);      // A-operand row of this lane

  // the mix weights of this lane's four rows for every level, read up front
  // and kept raw, so no level's fold waits for a load (none for a launch
  // without mix weights: level 0's read alone)
  // Rows past the sequence end and levels past L read the last valid ones
  // (the loads carry no condition, so nothing waits for them here); fold
  // drops those rows.
  E mraw[MAXL][4];
  if (a.mix != nullptr) {
    const E* mixp = static_cast<const E*>(a.mix) + ((size_t)b * T * H + h) * L;
#pragma unroll
    for (int l = 0; l < MAXL; ++l)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = min(wv * 16 + acc_row(r), nvalid - 1), lc = min(l, L - 1);
        mraw[l][r] = mixp[(size_t)(t0 + i) * H * L + lc];
      }
  } else {
#pragma unroll
    for (int l = 0; l < MAXL; ++l)
#pragma unroll
      for (int r = 0; r < 4; ++r) mraw[l][r] = E(0.f);
  }

  f4 out[CTV];
#pragma unroll
  for (int c = 0; c < CTV; ++c) out[c] = f4_zero();
  f4 acc[CTV];

  // One stage: this wave's A fragments (NKA k-steps from global, afrag(s):
  // split derived rows or exact input rows) are read first, so their loads
  // overlap the staging of the B operand; then acc[c] += A s_B[c-th 16 rows]^T.
  auto stage = [&](auto afrag, auto nka_c, const float* bsrc, int bsrc_ld, auto bcols_c, int ldb) {
    constexpr int NKA = decltype(nka_c)::value;
    using FA = decltype(afrag(0));
    FA fa[NKA];
#pragma unroll
    for (int s = 0; s < NKA; ++s) fa[s] = afrag(s);
    stage_split<256, V, decltype(bcols_c)::value>(sB, ldb, bsrc, bsrc_ld);
    lds_barrier();
#pragma unroll
    for (int s = 0; s < NKA; ++s)
#pragma unroll
      for (int c = 0; c < CTV; ++c)
        acc[c] = Mma<E>::mma(acc[c], fa[s], sB.get((c * 16 + (lane & 15)) * ldb + kofs<E>(lane) + s * KS));
    lds_barrier();
  };
  auto fold = [&](int l, float sc) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float mr = 0.f;
#pragma unroll
      for (int q = 0; q < MAXL; ++q)
        if (q == l) mr = to_f(mraw[q][r]);
      const float m = (wv * 16 + acc_row(r) < nvalid ? mr : 0.f) * sc;
#pragma unroll
      for (int c = 0; c < CTV; ++c) out[c][r] += m * acc[c][r];
    }
  };

  // ---- level 0: Qg h + Aqk Vn (its read kept for the backward, stored
  // last), or the read a level-0 pass stored
  if (a.read0_in) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = wv * 16 + acc_row(r);
      const float* rp = a.read0_in + (((size_t)b * T + t0 + min(i, nvalid - 1)) * H + h) * V;
#pragma unroll
      for (int c = 0; c < CTV; ++c) acc[c][r] = rp[c * 16 + acc_col()];
    }
  } else {
#pragma unroll
    for (int c = 0; c < CTV; ++c) acc[c] = f4_zero();
    // bf16: Qg and Aqk in fragment order, as the chunk terms write them
    constexpr bool FR = std::is_same<E, bf16>::value;
    const SplitTile<E> Qg = split_at<E>(a.Qg + cix * C * K, C * K);
    const SplitTile<E> Aqk = split_at<E>(a.Aqk + cix * C * C, C * C);
    for (int kb = 0; kb < K; kb += KH)
      stage([&](int s) { return Qg.get(FR ? frag_at(wv, kb / KS + s, K) : ri * K + kb + kofs<E>(lane) + s * KS); },
            std::integral_constant<int, KH / KS>{}, a.hT + cix * V * K + kb, K,
            std::integral_constant<int, KH>{}, LD);
    stage([&](int s) { return Aqk.get(FR ? frag_at(wv, s, C) : ri * C + kofs<E>(lane) + s * KS); },
          std::integral_constant<int, C / KS>{}, a.vnT + cix * V * C, C,
          std::integral_constant<int, C>{}, LDC);
  }
  if (a.l0_only) {   // level 0's read only: no mix, no upper levels, no o
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = wv * 16 + acc_row(r);
      if (i < nvalid) {
        float* rp = a.read0 + (((size_t)b * T + t0 + i) * H + h) * V;
#pragma unroll
        for (int c = 0; c < CTV; ++c) rp[c * 16 + acc_col()] = acc[c][r];
      }
    }
    return;
  }
  fold(0, 1.f);
  f4 read0[CTV];
#pragma unroll
  for (int c = 0; c < CTV; ++c) read0[c] = acc[c];

  // ---- upper levels: (scale q_l) S_l[group], q rows exact
  const E* qrow = static_cast<const E*>(a.q) + ((size_t)b * T * H + h) * L * K +
                  (size_t)(t0 + min(ri, nvalid - 1)) * H * L * K + kofs<E>(lane);
  for (int l = 1; l < L; ++l) {
    const int grp = n / a.f[l];
    const float* Sl = a.statesT[l] + (((size_t)b * a.NGl[l] + grp) * H + h) * V * K;
#pragma unroll
    for (int c = 0; c < CTV; ++c) acc[c] = f4_zero();
    for (int kb = 0; kb < K; kb += KH)   // rows past the end repeat the last row
      stage([&](int s) { return Mma<E>::ld(qrow + (size_t)l * K + kb + s * KS); },
            std::integral_constant<int, KH / KS>{}, Sl + kb, K,
            std::integral_constant<int, KH>{}, LD);
    fold(l, a.scale);                           // which drops them
  }

  // ---- write o
  E* op = static_cast<E*>(a.o) + ((size_t)b * T * H + h) * V;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int i = wv * 16 + acc_row(r);
    if (i < nvalid) {
#pragma unroll
      for (int c = 0; c < CTV; ++c)
        op[(size_t)(t0 + i) * H * V + c * 16 + acc_col()] = from_f<E>(out[c][r]);
    }
  }
  if (a.read0 && !a.read0_in) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = wv * 16 + acc_row(r);
      if (i < nvalid) {
        float* rp = a.read0 + (((size_t)b * T + t0 + i) * H + h) * V;
#pragma unroll
        for (int c = 0; c < CTV; ++c) rp[c * 16 + acc_col()] = read0[c][r];
      }
    }
  }
}

template <typename E, int K, int V>
static hipError_t launch_output(const OutputArgs& a, hipStream_t st) {
  const unsigned grid = (unsigned)(a.B * a.H * a.NT);
  hipLaunchKernelGGL((output_fwd_kernel<E, K, V>), dim3(grid), dim3(256), 0, st, a);
  return hipGetLastError();
}

hipError_t output_fwd(const OutputArgs& a, int dtype, int K, int V, hipStream_t st) {
#define NGDN_OU(E, KK, VV) \
  if (K == KK && V == VV) return launch_output<E, KK, VV>(a, st);
  if (dtype == NGDN_BF16) {
    NGDN_OU(bf16, 64, 64) NGDN_OU(bf16, 128, 128) NGDN_OU(bf16, 64, 128) NGDN_OU(bf16, 128, 64)
  } else {
    NGDN_OU(float, 64, 64) NGDN_OU(float, 128, 128) NGDN_OU(float, 64, 128) NGDN_OU(float, 128, 64)
  }
#undef NGDN_OU
  return hipErrorInvalidValue;
}

}  // namespace ngdn
