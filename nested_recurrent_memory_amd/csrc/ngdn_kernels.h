// Argument blocks and launchers shared between the kernels and the C-ABI.
#pragma once

#include "ngdn_common.h"
#include "../../include/ngdn.h"

namespace ngdn {

// Level-0 intra-chunk forward. Inputs in the reference layout (contiguous):
// q [B,T,H,L,K] (level-0 slice read), k, b [B,T,H,K], v, w [B,T,H,V] in the
// working dtype, g [B,T,H,K] fp32. Outputs, per (b, h, chunk):
// W [B,H,NT,64,K], U [B,H,NT,64,V], KtT [B,H,NT,K,64], Qg [B,H,NT,64,K],
// Aqk [B,H,NT,64,64] in the working dtype; gam [B,H,NT,K] fp32.
struct L0IntraArgs {
  const void* q; const void* k; const void* v; const float* g;
  const void* b; const void* w;
  void* W; void* U; void* KtT; void* Qg; void* Aqk; float* gam;
  int B, T, H, L, NT;
  float scale;
};
hipError_t l0_intra_fwd(const L0IntraArgs& a, int dtype, int K, int V, hipStream_t st);

// A sequence of delta-rule steps per (b, h):
//   Vn = U - A S;   S <- diag(gam) S + BT Vn
// A [B*H,S,M,K], BT [B*H,S,K,M], U [B*H,S,M,V] in the working dtype, gam
// [B*H,S,K] fp32. The state entering each step is stored: mode 0 as
// hT [B,H,S,V,K] in the working dtype (level 0, chunk states), mode 1 as fp32
// [B,NG,H,K,V] (upper levels, group states; NG >= S, extra groups hold the
// final state). vnT [B,H,S,V,M] (working dtype) receives Vn when not null.
struct ScanArgs {
  const void* A; const void* BT; const void* U; const float* gam;
  const float* init; long long init_sb, init_sh;
  void* states; int state_mode; int NG;
  void* vnT;
  float* fin; long long fin_sb, fin_sh;
  int B, H, S, M, V;
};
hipError_t scan_fwd(const ScanArgs& a, int dtype, int K, hipStream_t st);

}  // namespace ngdn

namespace ngdn {

// Promotion probe for one level (ops/probe.py:34-136), one workgroup per
// (batch, firing, head). Reads the lower level's state after this level's
// firing i: stored state src = ((i+1) f_here) / f_below, or the lower final
// state when src == NGb. below_mode 0: hT [B,H,NGb,V,K] (working dtype);
// below_mode 1: fp32 [B,NGb,H,K,V]. Parameters are this level's slices in the
// working dtype: bank [H,Nmax,K], kp [H,K,V], and the transposed projections
// bpT [H,K,V] (= b_proj^T), wpT [H,V,V] (= w_proj^T), gpT [H,K,V].
// Scan-ready outputs [B,H,NF,...]: A = keys*b*e^g [N,K], KT = keys^T [K,N],
// U = vals*w [N,V] (working dtype), gam = e^g [K] fp32. Reference-format
// outputs (fp32, [B,NF,H,...]) are written when their pointers are set.
struct ProbeArgs {
  const void* below; int below_mode; int NGb;
  const float* below_fin; long long bf_sb, bf_sh;
  int f_below, f_here;
  const void* bank; int Nmax;
  const void* kp; const void* bpT; const void* wpT; const void* gpT;
  int merge;
  void* A; void* KT; void* U; float* gam;
  float* keys; float* vals; float* bo; float* wo; float* go;
  int B, H, NF, N, V;
};
hipError_t probe_fwd(const ProbeArgs& a, int dtype, int K, hipStream_t st);

}  // namespace ngdn

namespace ngdn {

constexpr int MAXL = 8;

// Output of the whole op for one chunk (ops/chunk.py:250-286; ops/naive.py:376-390):
//   o = mix_0 (Qg h_n + Aqk Vn) + sum_{l>=1} mix_l scale q_l S_l[n / f_l]
// Level-0 terms from the intra/scan kernels ([B,H,NT,...], working dtype);
// q [B,T,H,L,K], mix [B,T,H,L] (working dtype); upper states fp32
// [B,NG_l,H,K,V]. o [B,T,H,V] in the working dtype. When reads is set, each
// level's unmixed read is also written, fp32 [L,B,T,H,V].
struct OutputArgs {
  const void* Qg; const void* Aqk; const void* hT; const void* vnT;
  const void* q; const void* mix;
  const float* states[MAXL]; int NGl[MAXL]; int f[MAXL];
  void* o; float* reads;
  int B, T, H, L, NT;
  float scale;
};
hipError_t output_fwd(const OutputArgs& a, int dtype, int K, int V, hipStream_t st);

}  // namespace ngdn
