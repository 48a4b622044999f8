// Argument blocks and launchers shared between the kernels and the C-ABI.
#pragma once

#include "ngdn_common.h"
#include "../../include/ngdn.h"

namespace ngdn {

// Level-0 intra-chunk forward. Inputs in the reference layout (contiguous):
// q [B,T,H,L,K] (level-0 slice read), k, b [B,T,H,K], v, w [B,T,H,V] in the
// working dtype, g [B,T,H,K] fp32. Outputs, per (b, h, chunk):
// W [B,H,NT,64,K], U [B,H,NT,64,V], KtT [B,H,NT,K,64], Qg [B,H,NT,64,K],
// Aqk [B,H,NT,64,64], gam [B,H,NT,K]; when set, TT [B,H,NT,64,64] (= T^T)
// for the chunk backward. W, KtT, Qg and Aqk are written in split form
// (split_at), U, gam and TT as fp32.
struct L0IntraArgs {
  const void* q; const void* k; const void* v; const float* g;
  const void* b; const void* w;
  float* W; float* U; float* KtT; float* Qg; float* Aqk; float* gam;
  float* TT;
  int B, T, H, L, NT;
  float scale;
  int n0, nn;         // chunks [n0, n0 + nn) of every (batch, head) (nn 0: all NT)
};
hipError_t l0_intra_fwd(const L0IntraArgs& a, int dtype, int K, int V, hipStream_t st);

// Most levels any entry point handles.
constexpr int MAXL = 8;

// Per-row firing gate of the decoding step (ops/naive.py:101-113): when pos
// is set, batch row b runs only if the token at pos[b] completes a chunk
// (end = pos[b] + 1, end % chunk == 0) whose number end / chunk is a multiple
// of every; other rows' workgroups return before touching memory.
struct FireGate {
  const long long* pos; int chunk, every;
};
__device__ __forceinline__ bool gated_out(const FireGate& g, int b) {
  if (!g.pos) return false;
  const long long end = g.pos[b] + 1;
  return end % g.chunk != 0 || (end / g.chunk) % g.every != 0;
}

// Columns of V per scan workgroup (each step's operands are read by V / 32
// workgroups of one (batch, head)).
constexpr int SCAN_BV = 32;
// The bf16 scans take 16-column slices, twice the workgroups with half the
// products per step, when the 32-column grid has at most this many
// workgroups (a quarter of the CUs).
constexpr int SCAN_NARROW_GRID = 64;

// A sequence of delta-rule steps per (b, h):
//   Vn = U - A S;   S <- diag(gam) S + BT Vn
// A [B*H,S,M,K], BT [B*H,S,K,M] in split form (split_at), U [B*H,S,M,V] and
// gam [B*H,S,K] fp32. The
// state entering each step is stored (fp32) as S rows (st_kv, [K][V]) and/or
// S^T rows (st_vk, [V][K]), each optional: mode 0 per (b, h, step) at
// [B,H,S,...] (level 0, chunk states), mode 1 per (b, group, h) at
// [B,NG,H,...] (upper levels, group states; NG >= S, extra groups hold the
// final state). vnT [B,H,S,V,M] and vn [B,H,S,M,V] receive Vn when set.
struct ScanArgs {
  const float* A; const float* BT; const float* U; const float* gam;
  const float* init; long long init_sb, init_sh;
  float* st_kv; float* st_vk; int state_mode; int NG;
  int vk_every;       // st_vk written at steps j with j % vk_every == 0 (<= 1: every step)
  float* vnT; float* vn;
  float* fin; long long fin_sb, fin_sh;
  int B, H, S, M, V;
  FireGate gate;
  // level 0 with read0 set: the chunk's level-0 read Qg S + Aqk Vn (Qg
  // [B*H,S,64,K], Aqk [B*H,S,64,64], fp32) into read0 [B,T,H,V] fp32
  const float* Qg; const float* Aqk; float* read0; int T;
  // bf16, fragment order as the chunk terms and the probes write them:
  // 1, BT (M % 32 == 0); 3, also A, Qg, Aqk (level 0); 0, none
  int frag;
  // steps [j0, j1) from init, the state entering step j0 (j1 0: all S)
  int j0, j1;
};
hipError_t scan_fwd(const ScanArgs& a, int dtype, int K, hipStream_t st);

// Reverse of scan_fwd. Upper levels: Bop [B*H,S,M,K] (= BT^T, the keys) and
// AT [B*H,S,K,M] (= A^T), both split, and d_states (fp32 [B,NG,H,K,V], added
// after step j, and for every stored group past the last step before the
// first). Level 0 (M = 64) sets instead the forward's own split tiles W
// [B*H,S,64,K], KtT [B*H,S,K,64], Qg [B*H,S,64,K], Aqk [B*H,S,64,64] (bf16:
// in fragment order), whose transposes it takes as its operands, dout
// [B,T,H,V], mix [B,T,H,L] and inj (fp32 [B*H,inj_nf,K,V], added before step
// j when (j+1) % inj_every == 0). gam [B*H,S,K]. d_final seeds the state
// gradient. Outputs (fp32): dSp [B*H,S,K,V] (gradient of the state after
// each step), dVn [B*H,S,M,V], dVnT = dVn^T [B*H,S,V,M] (when set), dinit
// ([K][V] at strides, when set). dout and mix are in the working dtype.
struct ScanBwdArgs {
  const float* Bop; const float* AT; const float* gam;
  const float* W; const float* KtT; const float* Qg; const float* Aqk;
  const void* dout; const void* mix; int T, L;
  // level 0: injection inj[(n+1)/inj_every - 1] before the step of chunk n;
  // levels >= 1: the level above's injection inj [B,H,inj_nf,K,V] joins the
  // group j that its firing i read, j = ((i+1) inj_fa) / inj_fh (the level's
  // interval inj_fh, the level above's inj_fa)
  const float* inj; int inj_every, inj_nf, inj_fh, inj_fa;
  const float* d_states; int NG;
  const float* d_final; long long df_sb, df_sh;
  float* dSp;
  float* dVn;
  float* dVnT;
  float* dinit; long long di_sb, di_sh;
  int B, H, S, M, V;
  // bf16, fragment order: 1, AT (upper levels, M % 32 == 0); 3, the level-0
  // tiles W, KtT, Qg, Aqk
  int frag;
  // level 0: steps [j0, j1) (j1 0: all S), from d_final, the gradient of the
  // state after step j1 - 1, to dinit, the gradient of the state entering j0
  int j0, j1;
};
hipError_t scan_bwd(const ScanBwdArgs& a, int dtype, int K, hipStream_t st);

}  // namespace ngdn

namespace ngdn {

// Promotion probe for one level (ops/probe.py:34-136), one workgroup per
// (batch, firing, head). Reads the lower level's state after this level's
// firing i: stored state src = ((i+1) f_here) / f_below, or the lower final
// state when src == NGb. below_mode 0: hT [B,H,NGb,V,K]; below_mode 1:
// [B,NGb,H,K,V] (both fp32). Parameters are this level's slices in the
// working dtype: bank [H,Nmax,K], kp [H,K,V], and the transposed projections
// bpT [H,K,V] (= b_proj^T), wpT [H,V,V] (= w_proj^T), gpT [H,K,V].
// Scan-ready outputs [B,H,NF,...] (fp32): A = keys*b*e^g [N,K], KT = keys^T
// [K,N], U = vals*w [N,V], gam = e^g [K]. Reference-format outputs (fp32,
// [B,NF,H,...]) are written when their pointers are set.
struct ProbeArgs {
  const float* below; int below_mode; int NGb;
  const float* below_fin; long long bf_sb, bf_sh;
  int f_below, f_here;
  const void* bank; int Nmax;
  const void* kp; const void* bpT; const void* wpT; const void* gpT;
  int merge;
  float* A; float* KT; float* U; float* gam;
  float* keysN; float* AT;   // optional: keys [B,H,NF,N,K], A^T [B,H,NF,K,N] for the reverse scan
  float* keys; float* vals; float* bo; float* wo; float* go;
  int B, H, NF, N, V;
  FireGate gate;
  int i0, ni;         // firings [i0, i0 + ni) (ni 0: all NF)
};
hipError_t probe_fwd(const ProbeArgs& a, int dtype, int K, hipStream_t st);

// Level-0 half of one decoding token (ops/naive.py:42-100): per (b, h),
// q [B,H,L,K], k, b [B,H,K], v, w [B,H,V], mix [B,H,L] in the working dtype,
// g [B,H,K] fp32; state s_in -> s_out [B,H,L,K,V] fp32 (may be the same
// buffer; level 0 updated, levels above copied when the buffers differ);
// o [B,H,V] in the working dtype.
struct StepArgs {
  const void* q; const void* k; const void* v; const float* g;
  const void* b; const void* w; const void* mix;
  const float* s_in; float* s_out;
  void* o;
  int B, H, L;
  float scale;
};
hipError_t step_fwd(const StepArgs& a, int dtype, int K, int V, hipStream_t st);

// The promotions that follow one decoding token (ops/naive.py:101-123),
// bottom-up over levels 1..L-1 in one launch: for every row whose firing of
// level l completes at this token (position + 1 a multiple of chunk f_l), the
// probe of level l-1's state (already updated) and one firing of level l's
// update, in place on state [B,H,L,K,V]. One workgroup of 8 waves per
// (b, h); levels with up to 64 pairs per firing (PROMOTE_NMAX).
constexpr int PROMOTE_NMAX = 64;
struct PromoteArgs {
  float* state;
  const long long* pos;   // [B] positions, or null: pos_all for every row
  long long pos_all;
  int chunk;
  int f[MAXL];       // firing intervals per level
  int N[MAXL];       // pairs per firing per level (index l >= 1)
  const void* bank; int Nmax;                                  // [L-1,H,Nmax,K]
  const void* kp; const void* bpT; const void* wpT; const void* gpT;   // [L-1,H,K,V]
  int merge;
  int B, H, L;
};
hipError_t promote_fwd(const PromoteArgs& a, int dtype, int K, hipStream_t st);

// One level's promotions in the chunk op, fused (promote_chunk.hip): one
// workgroup of 8 waves per (b, h) runs the level's firings in order with the
// level's state in registers: per firing the gather of the lower snapshot,
// the probe (as probe_fwd) and the update (as one scan_fwd step), and the
// group states stored before each firing (store-then-fire; groups past the
// last firing hold the final state). below: the lower level's stored states
// as [V][K] rows, mode 0 [B,H,NGb,V,K] (level-0 chunk states) or mode 1
// [B,NGb,H,V,K] (upper group states); below_fin: the lower final state
// ([K][V] rows at strides). Parameters: this level's slices in the working
// dtype, as for probe_fwd. init: [K][V] at strides, or null (zeros).
// st_kv [B,NG,H,K,V] and st_vk [B,NG,H,V,K] fp32; fin [K][V] at strides.
// For the backward (null for inference): keysN [B,H,NF,N,K] and
// AT = (keys b e^g)^T [B,H,NF,K,N] in split form, gam = e^g [B,H,NF,K].
// Up to PROMOTE_NMAX pairs per firing; merge at K = 64 only.
struct PromoteChainArgs {
  const float* below; int below_mode; int NGb;
  const float* below_fin; long long bf_sb, bf_sh;
  int f_below, f_here;
  const void* bank; int Nmax;
  const void* kp; const void* bpT; const void* wpT; const void* gpT;
  const float* init; long long init_sb, init_sh;
  float* st_kv; float* st_vk;
  float* fin; long long fin_sb, fin_sh;
  float* keysN; float* AT; float* gam;
  int B, H, NF, NG;
};
bool promote_chain_supported(int K, int N, bool merge);
hipError_t promote_chain_fwd(const PromoteChainArgs& a, int dtype, int K, int N, bool merge,
                             hipStream_t st);

// The layer's ShortConvolution (layer_ops.hip): x, y, dy, dx [B,T,D] and the
// caches [B,D,W] in the working dtype, w and dw [D][W] fp32 (dw summed
// into), act: SiLU after the convolution.
struct ShortConvArgs {
  const void* x; const float* w; const void* cache_in; void* y; void* cache_out;
  const void* dy; void* dx; float* dw;
  float* ws;    // backward: per-workgroup partial dw [NGDN_WPARTS][D*W], or NULL
  int B, T, D, W, act;
};

// Weight gradients summed over many workgroups: each workgroup stores its
// partial sum in row p of a workspace [NGDN_WPARTS][n] (plain stores), then
// sum_parts adds the rows into the gradient with a few atomics per element.
// Device-scope float atomics are performed past the per-XCD L2s, a few
// million of them (one per workgroup and weight) cost more than the kernel.
hipError_t sum_parts(const float* ws, long long nparts, long long n, float* out, hipStream_t st);
hipError_t short_conv_fwd(const ShortConvArgs& a, int dtype, hipStream_t st);
hipError_t short_conv_bwd(ShortConvArgs a, int dtype, hipStream_t st);

// The layer's gate prologue (layer_ops.hip, layers/nested_gdn2.py:134-166):
// from the convolved projections to the op's inputs, per (b, t, h):
//   qn[b,t,h,l,:] = normalize(q[b,t, l*H*K + h*K + :])    (q "b t (l h d)")
//   kn[b,t,h,:]   = normalize(k[b,t, h*K + :])
//   g0[b,t,h,:]   = min(-exp(A_log[h]) softplus(f[b,t,h*K+:] + dt_bias[h*K+:]), cap)
//   b0 = sigmoid(bz), w0 = sigmoid(wz), mix = softmax_l (or sigmoid) of ml[b,t,h*L+:]
// normalize(x) = x / max(|x|, 1e-12) as F.normalize. Raw inputs, qn, kn, b0,
// w0, mix in the working dtype; g0 fp32; A_log [H], dt_bias [H*K] in
// pdtype (0 fp32, 1 bf16). cap = -1/max_horizon, or +inf. The backward takes
// the gradients of the six outputs and writes those of the six raw inputs;
// dpar (fp32 [H*K + H]: ddt_bias, then dA_log) is summed into through ws
// partial rows [NGDN_WPARTS][H*K + H].
struct GatePrepArgs {
  const void* q; const void* k; const void* f; const void* bz; const void* wz; const void* ml;
  const void* A_log; const void* dt_bias;
  void* qn; void* kn; float* g0; void* b0; void* w0; void* mix;
  const void* dqn; const void* dkn; const float* dg0; const void* db0; const void* dw0; const void* dmix;
  void* dq; void* dk; void* df; void* dbz; void* dwz; void* dml;
  float* dpar; float* ws;
  long long BT;
  int H, L, K, V, pdtype, sigmoid_mix;
  float cap;
};
hipError_t gate_prep_fwd(const GatePrepArgs& a, int dtype, hipStream_t st);
hipError_t gate_prep_bwd(const GatePrepArgs& a, int dtype, hipStream_t st);

// The layer's FusedRMSNormGated (layer_ops.hip) over rows of V: x, g, y, dy,
// dx, dg in the working dtype; w and dw [V] fp32 (dw summed into); rstd
// [rows] fp32 written by the forward for the backward.
struct NormGatedArgs {
  const void* x; const void* g; const float* w; void* y; float* rstd;
  const void* dy; void* dx; void* dg; float* dw;
  float* ws;    // backward: per-workgroup partial dw [NGDN_WPARTS][n], or NULL
  long long rows;
  float eps;
};
hipError_t rmsnorm_gated_fwd(const NormGatedArgs& a, int dtype, int V, hipStream_t st);
hipError_t rmsnorm_gated_bwd(const NormGatedArgs& a, int dtype, int V, hipStream_t st);

// The model's RMSNorm (model_ops.hip) over rows of D: x, y, dy, dx in the
// working dtype; w and dw [D] fp32 (dw summed into); rstd [rows] fp32 written
// by the forward for the backward.
struct RMSNormArgs {
  const void* x; const float* w; void* y; float* rstd;
  const void* r; void* h;        // forward: residual added first (h = x + r), or NULL
  const void* dy; void* dx; float* dw;
  const void* dh; void* dr;      // backward: gradient of h besides the norm, residual's copy
  float* ws;    // backward: per-workgroup partial dw [NGDN_WPARTS][n], or NULL
  long long rows;
  int D;
  float eps;
};
bool rmsnorm_supported(int D);
bool rmsnorm_types_supported(int xd, int rd, int yd);
hipError_t rmsnorm_fwd(const RMSNormArgs& a, int xd, int rd, int yd, hipStream_t st);
hipError_t rmsnorm_bwd(const RMSNormArgs& a, int xd, int rd, int yd, hipStream_t st);

// The MLP's SwiGLU (model_ops.hip): y = silu(g) u over n values, n % 8 == 0,
// all in the working dtype.
struct SwigluArgs {
  const void* g; const void* u; void* y;
  const void* dy; void* dg; void* du;
  long long n;
};
hipError_t swiglu_fwd(const SwigluArgs& a, int dtype, hipStream_t st);
hipError_t swiglu_bwd(const SwigluArgs& a, int dtype, hipStream_t st);

// Sum of up to 8 same-shaped tensors in the working dtype into fp32
// (model_ops.hip): out[i] = sum_j x_j[i], n % 8 == 0.
constexpr int SUM_MAX = 8;
struct SumArgs {
  const void* x[SUM_MAX];
  float* out;
  long long n;
  int count;
};
hipError_t sum_into_f32(const SumArgs& a, int dtype, hipStream_t st);

// Cross entropy of rows of V logits (model_ops.hip): row_loss[r] =
// (logsumexp(x_r) - x_r[label_r]) / n_valid, 0 for ignored labels; with grad
// the logits are overwritten by d(sum of row_loss)/dx = (softmax - onehot) /
// n_valid (zeros on ignored rows). n_valid: device int64, the count of labels
// that are not ignore_index.
struct XentArgs {
  void* logits; const long long* labels; const long long* n_valid; float* row_loss;
  long long rows;
  int V, ignore_index, grad;
};
bool xent_supported(int V);
hipError_t cross_entropy(const XentArgs& a, int dtype, hipStream_t st);

// Backward of one level's firings (update: ops/update_bwd.py:115-158; probe:
// the autograd replay of ops/chunk.py:339-371,486-517, derived in closed
// form). One workgroup of 8 waves per (batch, head, firing i). Inputs: the
// lower level's states as rows and transposed (below_kv / below_vk, same
// layout modes as probe_fwd's below), the parameters as for probe_fwd (plus
// kpT = key_proj^T [H,V,K] and bankT [H,K,Nmax], original bp [H,V,K], wp
// [H,V,V], gp [H,V,K]); this level's group states Sg [B,NG,H,K,V] and SgT
// [B,NG,H,V,K] (fp32); the reverse scan's dSp (fp32
// [B,H,NF,K,V], gradient of the state after firing i) and dvn (fp32
// [B,H,NF,N,V]). Workspace (fp32, [B,H,NF,N,*]): Vals, du, dxb,
// dxg [N,K-or-V], dxw, dVals [N,V]; the parameter-gradient reduction reads
// them. dbank: this firing's bank-gradient partial (fp32 [B,H,NF,N,K],
// written), summed per head in a fixed order by the parameter-gradient pass.
// The gradient of the gathered lower state goes to inj (fp32 [B,H,NF,K,V],
// written; the lower level's reverse scan adds it), except at a level >= 2
// firing that reads the lower final state: added to d_below_fin (fp32
// [K][V] at strides).
struct ProbeBwdArgs {
  ProbeArgs f;                // gather indices, params as in the forward (f.below, f.A .. unused)
  const float* below_kv;      // lower states as rows [K][V] (level 0: h, mode 0 layout)
  const float* below_vk;      // and transposed [V][K] (level 0: hT)
  const void* kpT; const void* bankT; const void* bp; const void* wp; const void* gp;
  const float* Sg; const float* SgT; int NG;   // this level's group states, rows and transposed
  const float* dSp; const float* dvn;
  float* wsV; float* wsdu; float* wsdxb; float* wsdxg; float* wsdxw; float* wsdV;
  float* dbank;
  float* inj; float* d_below_fin;
};
hipError_t probe_bwd(const ProbeBwdArgs& a, int dtype, int K, hipStream_t st);

// Partial sums over rows m = (b, i, n) of A[b,h,i,n,X] B[b,h,i,n,Y] for the
// per-head parameter gradients of a level: one workgroup per (product, head,
// slice of items) writes its X x Y partial to parts [nprod][H][split][X][Y]
// (fp32; slices without items write zeros). ordered_sum then adds the slices
// into C_p[h] in a fixed order. Up to four sums in one launch.
struct AtBArgs {
  const float* A[4]; const float* Bm[4]; float* C[4];
  float* parts;
  int nprod;
  int B, H, NF, N, X, Y;
  int split;
};
hipError_t atb_accumulate(const AtBArgs& a, int dtype, hipStream_t st);

// Fixed-order sums of partials (deterministic reductions): for w < nsum,
// g < ng, x < n[w]: out[w][g og + x] += sum_{j1 < n1, j2 < n2} (in that order)
// parts[w][g pg + j1 s1 + j2 s2 + x].
constexpr int OSUM_MAX = 5;
struct OrderedSumArgs {
  const float* parts[OSUM_MAX]; float* out[OSUM_MAX];
  long long pg[OSUM_MAX], og[OSUM_MAX], s1[OSUM_MAX], s2[OSUM_MAX], n[OSUM_MAX];
  int n1[OSUM_MAX], n2[OSUM_MAX];
  int nsum, ng;
};
hipError_t ordered_sum(const OrderedSumArgs& a, hipStream_t st);

}  // namespace ngdn

namespace ngdn {

// Output of the whole op for one chunk (ops/chunk.py:250-286; ops/naive.py:376-390):
//   o = mix_0 (Qg h_n + Aqk Vn) + sum_{l>=1} mix_l scale q_l S_l[n / f_l]
// Level-0 terms from the intra/scan kernels ([B,H,NT,...], fp32);
// q [B,T,H,L,K], mix [B,T,H,L] (working dtype); upper group states fp32, as
// S^T rows [B,NG_l,H,V,K] (statesT). o [B,T,H,V] in the working dtype. When
// read0 is set, level 0's unmixed read Qg h_n + Aqk Vn is also written, fp32
// [B,T,H,V] (the backward's dmix_0).
// Split in two passes (the first can run beside the upper levels' promotions):
// l0_only computes level 0's read into read0 and writes nothing else;
// read0_in takes that read instead of computing it and forms o.
struct OutputArgs {
  const float* Qg; const float* Aqk; const float* hT; const float* vnT;
  const void* q; const void* mix;
  const float* statesT[MAXL]; int NGl[MAXL]; int f[MAXL];
  void* o; float* read0;
  const float* read0_in; int l0_only;
  int B, T, H, L, NT;
  float scale;
};
hipError_t output_fwd(const OutputArgs& a, int dtype, int K, int V, hipStream_t st);

// dmix_0[t] = <do[t], read0[t]> (ops/chunk.py:423), one wave per 16 tokens of
// one head: read0 fp32 [B,T,H,V], do [B,T,H,V] (working dtype), dmix fp32
// [B,T,H,L] (level-0 column written).
struct Dmix0Args {
  const float* read0; const void* dout; float* dmix;
  int B, T, H, L, V;
};
hipError_t dmix0_bwd(const Dmix0Args& a, int dtype, hipStream_t st);

// fp32 arrays cast to bf16 in one launch (the op's gradients in its inputs'
// dtype): dst[w][i] = src[w][i] rounded to nearest even, w < count.
constexpr int CAST_MAX = 16;
struct CastArgs {
  const float* src[CAST_MAX]; void* dst[CAST_MAX]; long long n[CAST_MAX];
  int count;
};
hipError_t cast_bf16(const CastArgs& a, hipStream_t st);

// Batched transposes of the last two axes in one launch: array w is
// src [batch][R][C] -> dst [batch][C][R], elements of esz bytes (2 or 4);
// tiles0 holds the prefix sums of the arrays' 32 x 32 tile counts.
constexpr int TR_MAX = 8;
struct TransposeArgs {
  const void* src[TR_MAX]; void* dst[TR_MAX];
  int batch[TR_MAX], R[TR_MAX], C[TR_MAX];
  int tiles0[TR_MAX + 1];
  int count, esz;
};
hipError_t transpose(const TransposeArgs& a, hipStream_t st);

// Backward of level l's reads, per (batch, group j, head), over the group's
// chunks (read_level_bwd, ops/chunk.py:307-336, and the dq/dmix terms of
// :423-449). With S = S_l[j] (rows [K][V] fp32, staged once) and
// dO = mix_l do:
//   read_l = scale q_l S,  dmix_l[t] = <do[t], read_l[t]>,
//   dq_l   = scale dO S^T,  dS_l[j] = scale sum_t q_l[t]^T dO[t]
// d_states fp32 [B,NG,H,K,V] written; dq [B,T,H,L,K] (level-l slice, working
// dtype) and dmix [B,T,H,L] (level-l column) written.
struct ReadStateBwdArgs {
  const void* q; const void* mix; const void* dout; const float* states;
  float* d_states; void* dq; float* dmix;
  int B, T, H, L, level, f, NG;
  float scale;
};
hipError_t read_state_bwd(const ReadStateBwdArgs& a, int dtype, int K, int V, hipStream_t st);

// Level-0 chunk backward, state-dependent half, per (b, h, chunk):
//   dQg = dO S^T, dW = -dVn S^T, dKt = Vn dS'^T, dAqk = dO Vn^T (j <= i),
//   dgam_k = sum_v dS'[k][v] S[k][v]
// with S = h (rows [K][V]), Vn rows [64][V], dS' the state gradient after the
// chunk, dO = mix_0 do. Outputs (fp32) dQg, dKt [B,H,NT,64,K], dWT
// [B,H,NT,K,64], dAqk [B,H,NT,64,64], dgam [B,H,NT,K]; dout and mix in the
// working dtype.
struct L0BwdStateArgs {
  const float* h; const float* dSp; const float* vn; const float* dVn;
  const void* dout; const void* mix;
  float* dQg; float* dWT; float* dKt; float* dAqk; float* dgam;
  int B, T, H, L, NT;
};
hipError_t l0_bwd_state(const L0BwdStateArgs& a, int dtype, int K, int V, hipStream_t st);

// Level-0 chunk backward, intra-chunk half (through T = (I+A)^-1, the decay
// products and the cumulative sum), per (b, h, chunk). Reads the forward's
// W [.,64,K], U [.,64,V] and TT = T^T [.,64,64], the state half's dQg, dKt
// [.,64,K], dWT = dW^T [.,K,64], dAqk [.,64,64], dgam [.,K], and the scan's
// dVnT = dVn^T [.,V,64] (W in split form). Writes dq[..., 0, :], dk, dv, db, dw (working dtype)
// and dg (fp32).
struct L0BwdIntraArgs {
  const void* q; const void* k; const void* v; const float* g; const void* b; const void* w;
  const float* W; const float* U; const float* TT;
  const float* dQg; const float* dWT; const float* dKt; const float* dAqk; const float* dgam;
  const float* dVnT;
  void* dq; void* dk; void* dv; float* dg; void* db; void* dw;
  int B, T, H, L, NT;
  float scale;
  // the fused form (l0_bwd): the state half computed by the same workgroup
  // from the chunk states h [.,K,V], their gradients dSp [.,K,V], Vn [.,64,V],
  // do and mix; dQg and dKt pass through the workspaces wsQ, wsK [.,64,K]
  // (fp32, no initial contents) between its phases; W, U, dQg, dWT, dKt, dAqk
  // and dgam above are then unused
  const float* h; const float* dSp; const float* vn; const void* dout; const void* mix;
  float* wsQ; float* wsK;
  int n0, nn;         // chunks [n0, n0 + nn) of every (batch, head) (nn 0: all NT)
};
hipError_t l0_bwd_intra(const L0BwdIntraArgs& a, int dtype, int K, int V, hipStream_t st);
hipError_t l0_bwd_fused(const L0BwdIntraArgs& a, int dtype, int K, int V, hipStream_t st);

}  // namespace ngdn
