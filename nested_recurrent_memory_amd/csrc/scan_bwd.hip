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
// MFMAs on split operands.
#include "ngdn_kernels.h"

namespace ngdn {

template <typename E, int K, int M>
__global__ __launch_bounds__(256) void scan_bwd_kernel(ScanBwdArgs a) {
  constexpr int BV = 32;
  constexpr int CT = BV / 16;
  constexpr int RTS = K / 16;
  constexpr int TPW = RTS * CT / 4;
  constexpr int RTV = M / 16;
  constexpr int LDS_ST = K + 4;
  constexpr int LDS_VN = M + 4;
  constexpr int KS = Mma<E>::KS;
  constexpr int NSM = (M + KS - 1) / KS;
  constexpr bool PADM = (M % KS) != 0;
  typedef typename Mma<E>::SFrag SF;
  __shared__ __attribute__((aligned(16))) float s_dST[BV * LDS_ST];
  __shared__ __attribute__((aligned(16))) float s_dVnT[BV * LDS_VN];
  __shared__ __attribute__((aligned(16))) float s_dOT[BV * LDS_VN];

  const int V = a.V, S = a.S, H = a.H;
  const int nvt = V / BV;
  const int vt = blockIdx.x % nvt;
  const int bh = blockIdx.x / nvt;
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
  auto add_kv = [&](const float* src) {   // ds += src[K][V]
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      const int g = wv * TPW + i, rt = g / CT, ct = g % CT;
#pragma unroll
      for (int r = 0; r < 4; ++r)
        ds[i][r] += src[(size_t)(rt * 16 + acc_row(r)) * V + v0 + ct * 16 + acc_col()];
    }
  };
  auto dstates = [&](int j) {
    return a.d_states + (((size_t)b * a.NG + j) * H + h) * K * V;
  };
  if (a.d_states)
    for (int j = a.NG - 1; j >= S; --j) add_kv(dstates(j));

  const float* Bb = a.Bop + (size_t)bh * S * M * K;
  const float* Ab = a.AT + (size_t)bh * S * K * M;
  const float* Gb = a.gam + (size_t)bh * S * K;
  const E* dob = l0 ? static_cast<const E*>(a.dout) + ((size_t)b * a.T * H + h) * V : nullptr;
  const E* mixb = l0 ? static_cast<const E*>(a.mix) + ((size_t)b * a.T * H + h) * a.L : nullptr;

  for (int j = S - 1; j >= 0; --j) {
    if (a.inj && (j + 1) % a.inj_every == 0)
      add_kv(a.inj + ((size_t)bh * a.inj_nf + (j + 1) / a.inj_every - 1) * K * V);

    // ---- store dS' and stage it (transposed) as the B operand of Bop dS'
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      const int g = wv * TPW + i, rt = g / CT, ct = g % CT;
      const int k0 = rt * 16 + acc_row(0), vl = ct * 16 + acc_col();
      float* o = a.dSp + ((size_t)bh * S + j) * K * V + (size_t)k0 * V + v0 + vl;
#pragma unroll
      for (int r = 0; r < 4; ++r) o[(size_t)r * V] = ds[i][r];
      *reinterpret_cast<f4*>(s_dST + vl * LDS_ST + k0) = ds[i];
    }
    if (l0) {
      // dO^T for this chunk's rows and this V slice
      for (int e = tid; e < M * BV; e += 256) {
        const int c = e / BV, vl = e % BV, t = j * M + c;
        float x = 0.f;
        if (t < a.T)
          x = to_f(dob[(size_t)t * H * V + v0 + vl]) * to_f(mixb[(size_t)t * H * a.L]);
        s_dOT[vl * LDS_VN + c] = x;
      }
    }
    __syncthreads();

    // ---- dVn = Bop dS' (+ Aqk^T dO)
    const float* Bj = Bb + (size_t)j * M * K;
    for (int rt = wv; rt < RTV; rt += 4) {
      SF bf[K / KS];
      const float* brow = Bj + (size_t)(rt * 16 + (lane & 15)) * K + kofs<E>(lane);
#pragma unroll
      for (int s = 0; s < K / KS; ++s) bf[s] = Mma<E>::ld(brow + s * KS);
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        f4 acc = f4_zero();
        const float* srow = s_dST + (ct * 16 + (lane & 15)) * LDS_ST + kofs<E>(lane);
#pragma unroll
        for (int s = 0; s < K / KS; ++s) acc = Mma<E>::mma(acc, bf[s], Mma<E>::ld(srow + s * KS));
        if (l0) {
          const float* qrow = a.AqkT + ((size_t)bh * S + j) * M * M +
                              (size_t)(rt * 16 + (lane & 15)) * M + kofs<E>(lane);
          const float* orow = s_dOT + (ct * 16 + (lane & 15)) * LDS_VN + kofs<E>(lane);
#pragma unroll
          for (int s = 0; s < NSM; ++s)
            acc = Mma<E>::mma(acc, Mma<E>::ld(qrow + s * KS), Mma<E>::ld(orow + s * KS));
        }
        const int m0 = rt * 16 + acc_row(0), vl = ct * 16 + acc_col();
        float* o = a.dVn + ((size_t)bh * S + j) * M * V + (size_t)m0 * V + v0 + vl;
#pragma unroll
        for (int r = 0; r < 4; ++r) o[(size_t)r * V] = acc[r];
        *reinterpret_cast<f4*>(s_dVnT + vl * LDS_VN + m0) = acc;
        if (a.dVnT)
          *reinterpret_cast<f4*>(a.dVnT + (((size_t)bh * S + j) * V + v0 + vl) * M + m0) = acc;
      }
    }
    __syncthreads();

    // ---- dS = diag(gam) dS' - A^T dVn (+ Qg^T dO)
    const float* Aj = Ab + (size_t)j * K * M;
    const float* Gj = Gb + (size_t)j * K;
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      const int g = wv * TPW + i, rt = g / CT, ct = g % CT;
      f4 acc = f4_zero();
      const float* arow = Aj + (size_t)(rt * 16 + (lane & 15)) * M + kofs<E>(lane);
      const float* vrow = s_dVnT + (ct * 16 + (lane & 15)) * LDS_VN + kofs<E>(lane);
#pragma unroll
      for (int s = 0; s < NSM; ++s) {
        const bool live = !PADM || (s * KS + kofs<E>(lane) < M);
        SF fa = Mma<E>::szero(), fb = fa;
        if (live) {
          fa = Mma<E>::ld(arow + s * KS);
          fb = Mma<E>::ld(vrow + s * KS);
        }
        acc = Mma<E>::mma(acc, fa, fb);
      }
      f4 qacc = f4_zero();
      if (l0) {
        const float* qrow = a.QgT + ((size_t)bh * S + j) * K * M +
                            (size_t)(rt * 16 + (lane & 15)) * M + kofs<E>(lane);
        const float* orow = s_dOT + (ct * 16 + (lane & 15)) * LDS_VN + kofs<E>(lane);
#pragma unroll
        for (int s = 0; s < NSM; ++s)
          qacc = Mma<E>::mma(qacc, Mma<E>::ld(qrow + s * KS), Mma<E>::ld(orow + s * KS));
      }
#pragma unroll
      for (int r = 0; r < 4; ++r)
        ds[i][r] = Gj[rt * 16 + acc_row(r)] * ds[i][r] - acc[r] + qacc[r];
    }
    if (a.d_states) add_kv(dstates(j));
    // s_dOT and s_dVnT are rewritten by the next step
    __syncthreads();
  }
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
  const unsigned grid = (unsigned)(a.B * a.H * (a.V / 32));
  hipLaunchKernelGGL((scan_bwd_kernel<E, K, M>), dim3(grid), dim3(256), 0, st, a);
  return hipGetLastError();
}

hipError_t scan_bwd(const ScanBwdArgs& a, int dtype, int K, hipStream_t st) {
  if (a.V % 32 != 0) return hipErrorInvalidValue;
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
