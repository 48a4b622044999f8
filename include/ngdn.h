/* C ABI of the MI355X nested Gated DeltaNet op (libngdn.so, gfx950).
 *
 * Plain pointers to device memory, sizes and a HIP stream (passed as void*,
 * a hipStream_t). Every entry point validates its arguments, launches
 * asynchronously on the given stream and returns 0, or a nonzero NGDN_E*
 * code with a message available from ngdn_last_error(). Nothing is allocated
 * inside the library: callers pass every output and workspace buffer.
 * Entry points are re-entrant; the error message is kept per thread.
 *
 * Tensor layouts follow the reference op (nested_gdn2/ops/chunk.py:722-766):
 *   q [B,T,H,L,K]; k, b [B,T,H,K]; v, w [B,T,H,V]; g [B,T,H,K] fp32;
 *   mix [B,T,H,L]; initial/final state [B,H,L,K,V] fp32;
 *   query_banks [L-1,H,Nmax,K]; key_projections [L-1,H,K,V];
 *   b/g_projections [L-1,H,V,K]; w_projections [L-1,H,V,V].
 * All contiguous. "dtype" is the element type of the op's inputs and
 * parameters (other than g and the states) and of its gradients: NGDN_F32 or
 * NGDN_BF16. Chunk size is 64.
 * Working tensors between the entry points ([B,H,NT,...], NT = ceil(T/64))
 * take 4 bytes per element whatever the dtype (declared float*), and are
 * described at each function. Most hold fp32 values. Those marked "split"
 * are read only as matrix-core operands: for NGDN_BF16 each per-unit tile
 * [R][C] (one chunk's, or one firing's) holds two bf16 planes, hi = bf16(x)
 * then lo = bf16(x - hi), R*C elements apart; for NGDN_F32 the fp32 values.
 */
#ifndef NGDN_H
#define NGDN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NGDN_OK 0
#define NGDN_EINVAL 1   /* bad shape, dtype, pointer or option */
#define NGDN_ELAUNCH 2  /* the HIP runtime refused a launch */

#define NGDN_F32 0
#define NGDN_BF16 1

/* rows of per-workgroup partial sums in the ws argument of the layer/model
 * backward entry points ([NGDN_WPARTS][n] fp32, n the weight's size) */
#define NGDN_WPARTS 1024

/* Sizes of one call. hold_partial (0 or 1): with 1 a partial last chunk
 * (T % 64 != 0) completes no upper level's firing, as the reference's
 * decoding step treats an incomplete chunk (nested_gdn2/ops/naive.py:101-113);
 * with 0, as the reference's chunk form (ops/chunk.py:257-290), every chunk
 * end counts, the partial last one's included. The firings of level l are
 * then NF = NTF / f_l, NTF = T / 64 (hold) or ceil(T / 64); the stored group
 * states stay NG = ceil(ceil(T / 64) / f_l) either way. */
typedef struct ngdn_dims {
  int32_t B, T, H, L, K, V;
  int32_t dtype;
  float scale;
  int32_t hold_partial;
} ngdn_dims;

/* Last error message on this thread ("" when none). */
const char* ngdn_last_error(void);
/* Version of this interface, major * 10000 + minor * 100 + patch. A caller
 * built against this header checks ngdn_version() == NGDN_VERSION before its
 * first call: the layouts of the working tensors and the meaning of some
 * arguments changed between versions while the signatures stayed the same
 * (for instance ngdn_probe_bwd's bank-gradient argument: an accumulator
 * [L-1,H,n_max,K] before 0.2.0, the per-firing workspace ws_dbank
 * [B,H,NF,N,K] since), so an older caller can link and then write past its
 * buffers. 0.4.0 added ngdn_dims.hold_partial (the struct grew by 4 bytes);
 * 0.5.0 took W and U out of ngdn_l0_bwd; 0.6.0 moved the upper levels'
 * lower-state gradients from ngdn_probe_bwd's d_below to an injection that
 * ngdn_upper_scan_bwd adds. */
#define NGDN_VERSION 1000
int32_t ngdn_version(void);
/* Offload architecture the library was built for ("gfx950"). */
const char* ngdn_arch(void);

/* Level-0 per-chunk terms: the intra-chunk half of fla's chunk_gdn2_fwd as
 * called at nested_gdn2/ops/chunk.py:236-248 (semantics ops/naive.py:329-358).
 * Outputs: W [B,H,NT,64,K], U [B,H,NT,64,V], KtT [B,H,NT,K,64],
 * Qg [B,H,NT,64,K] (scale folded in), Aqk [B,H,NT,64,64], gam [B,H,NT,K],
 * and TT [B,H,NT,64,64] = ((I + A)^-1)^T, which only the chunk backward
 * reads (may be NULL: inference). W, KtT, Qg and Aqk are split; U, gam and
 * TT fp32. For bf16 inputs the split tensors are in fragment order: in each
 * plane of a unit tile [R][C], the 16 x 32 block (rb, cb) is 512
 * consecutive elements at 512 (rb C/32 + cb), element (r, c) of the block
 * at 8 (16 (c / 8) + r) + c % 8, so one matrix-core A fragment of a row tile
 * is one contiguous 1 KB read. Only chunks [chunk0, chunk0 + nchunk) of every
 * (batch, head) are formed (1 <= nchunk, chunk0 + nchunk <= NT): a caller can
 * form later chunks while the level-0 scan runs over earlier ones. */
int32_t ngdn_l0_intra_fwd(const ngdn_dims* d, const void* q, const void* k,
                          const void* v, const float* g, const void* b,
                          const void* w, float* W, float* U, float* KtT, float* Qg,
                          float* Aqk, float* gam, float* TT, int32_t chunk0,
                          int32_t nchunk, void* stream);

/* Level-0 state recurrence over chunks: the inter-chunk half of fla's
 * chunk_gdn2_fwd (ops/chunk.py:236-248; semantics ops/naive.py:367-392).
 * Writes final_state[:, :, 0] and, each when not NULL: hT [B,H,NT,V,K] (the
 * state entering chunk j, transposed, for chunks j with j % hT_every == 0:
 * the probes of level 1 read every f1-th), vnT [B,H,NT,V,64] (the chunk's
 * new values, transposed), for the backward h [B,H,NT,K,V] (the states as
 * rows) and vn [B,H,NT,64,V], and read0 [B,T,H,V] fp32: level 0's read
 * Qg h + Aqk Vn of every token (Qg, Aqk from ngdn_l0_intra_fwd, required
 * with read0), formed while the state is on chip, which
 * ngdn_output_upper_fwd turns into o. initial_state may be NULL (zeros).
 * W, U, KtT, gam, Qg, Aqk as ngdn_l0_intra_fwd writes them (bf16: the split
 * ones in fragment order). Runs chunks [chunk0, chunk0 + nchunk) (1 <=
 * nchunk, chunk0 + nchunk <= NT): initial_state is then the state entering
 * chunk chunk0 and final_state receives the state after the last; the
 * per-chunk outputs are written at their chunks' places. initial_state may
 * be final_state itself (each workgroup reads its slice before writing it),
 * so consecutive ranges carry the state through final_state. */
int32_t ngdn_l0_scan_fwd(const ngdn_dims* d, const float* W, const float* U,
                         const float* KtT, const float* gam, const float* Qg,
                         const float* Aqk, const float* initial_state, int32_t hT_every,
                         float* hT, float* vnT, float* h, float* vn, float* read0,
                         float* final_state, int32_t chunk0, int32_t nchunk, void* stream);

/* Promotion probe of level `level` >= 1: PROBES[promotion] applied to the
 * lower level's state after each of this level's firings
 * (ops/probe.py:69-136, gathered as in ops/chunk.py:58-93).
 * below: level 0 -> hT from ngdn_l0_scan_fwd (NG_below = NT);
 *        level >= 2 -> the lower level's fp32 group states [B,NG_below,H,K,V].
 * final_state: [B,H,L,K,V] holding the lower level's final state.
 * bpT, gpT [L-1,H,K,V] and wpT [L-1,H,V,V] are the b/g/w projections with
 * their last two axes swapped. promotion: 0 learned, 1 merge (n_queries = K).
 * Outputs for firing i in [0, NF), NF = NT / f_here, laid out [B,H,NF,...]:
 * A = keys*b*e^g [N,K] (split), KT = keys^T [K,N] (split), U = values*w [N,V],
 * gam = e^g [K]; for the backward, keysN = keys [N,K] and AT = A^T
 * [K,N] (both split; may be NULL). keys/vals/bo/wo/go (fp32, [B,NF,H,N,K|V] and [B,NF,H,K])
 * receive the probe outputs in the reference layout when not NULL.
 * Fragment order: for NGDN_BF16 with N % 32 == 0, each plane of the [K][N]
 * tiles KT and AT is in the fragment order described at ngdn_l0_intra_fwd
 * (C = N); A and keysN stay row-major. ngdn_upper_scan_fwd / _bwd read KT and
 * AT that way; a caller that writes or reads them itself must use it too.
 * Only firings [firing0, firing0 + nfiring) are probed (0 <= firing0,
 * firing0 + nfiring <= NF; nfiring 0 does nothing): a caller can probe the
 * firings whose lower state is stored while the lower level still runs. */
int32_t ngdn_probe_fwd(const ngdn_dims* d, int32_t level, int32_t promotion,
                       int32_t n_queries, int32_t f_below, int32_t f_here,
                       const float* below, int32_t ng_below,
                       const float* final_state, const void* query_banks,
                       int32_t n_max, const void* key_projections,
                       const void* bpT, const void* wpT, const void* gpT,
                       float* A, float* KT, float* U, float* gam, float* keysN,
                       float* AT, float* keys, float* vals, float* bo, float* wo,
                       float* go, int32_t firing0, int32_t nfiring, void* stream);

/* Write scan of level `level` >= 1 (ops/update_fwd.py:131-204) from the
 * probe's scan-ready pairs (A row-major; KT in fragment order for NGDN_BF16
 * with n_pairs % 32 == 0, as ngdn_probe_fwd and ngdn_promote_chain_fwd write
 * it): NF firings, NG = ceil(NT / f) stored group
 * states. Writes states [B,NG,H,K,V] fp32 (state entering each group; groups
 * past the last firing hold the final state), statesT [B,NG,H,V,K] (the same,
 * transposed; may be NULL) and final_state[:, :, level]. initial_state may be
 * NULL. Runs firings [step0, step0 + nstep) (1 <= nstep, step0 + nstep <= NF;
 * with NF = 0, step0 = nstep = 0): initial_state[:, :, level] is then the
 * state entering firing step0 and final_state[:, :, level] receives the
 * state after the last; the range ending at NF also stores the groups past
 * the last firing. initial_state may be final_state itself, so consecutive
 * ranges carry the state through it. */
int32_t ngdn_upper_scan_fwd(const ngdn_dims* d, int32_t level, int32_t n_pairs,
                            int32_t nf, int32_t ng, const float* A,
                            const float* KT, const float* U, const float* gam,
                            const float* initial_state, float* states,
                            float* statesT, float* final_state, int32_t step0,
                            int32_t nstep, void* stream);

/* The promotions of level `level` >= 1, fused: the reference's per-level
 * chain gather_source -> probe_learned / probe_merge -> update_state
 * (nested_gdn2/ops/chunk.py:257-290 with ops/probe.py:34-136 and
 * ops/update_fwd.py:131-204) in one launch of B*H workgroups, each running
 * its (b, h)'s NF = NT / f_here firings in order with the level's state on
 * chip: the lower snapshot, the probe's pairs and gates and the state never
 * go to HBM between the probe's read and the update's write. below: the lower
 * level's stored states transposed, level 1 the level-0 chunk states hT
 * [B,H,NT,V,K], level >= 2 the lower statesT [B,ng_below,H,V,K]; a firing
 * whose source index is ng_below reads final_state[:, :, level-1].
 * Parameters as for ngdn_probe_fwd. Writes states [B,NG,H,K,V] and statesT
 * [B,NG,H,V,K] (NG = ceil(NT / f_here); the state entering each group,
 * groups past the last firing hold the final state) and
 * final_state[:, :, level]. For the backward (all three or none): keysN
 * [B,H,NF,N,K] and AT = (keys b e^g)^T [B,H,NF,K,N] (split; AT in fragment
 * order for NGDN_BF16 with N % 32 == 0), gam = e^g [B,H,NF,K] fp32, as
 * ngdn_probe_fwd writes them. Up to 64 pairs per firing
 * (merge: K = 64); other levels use ngdn_probe_fwd + ngdn_upper_scan_fwd. */
int32_t ngdn_promote_chain_fwd(const ngdn_dims* d, int32_t level, int32_t promotion,
                               int32_t n_queries, int32_t f_below, int32_t f_here,
                               const float* below, int32_t ng_below,
                               float* final_state, const void* query_banks,
                               int32_t n_max, const void* key_projections,
                               const void* bpT, const void* wpT, const void* gpT,
                               const float* initial_state, float* states, float* statesT,
                               float* keysN, float* AT, float* gam, void* stream);

/* Output for every token (ops/chunk.py:129-156, 250-251, 285-286):
 * o = mix_0 (Qg h + Aqk Vn) + sum_{l>=1} mix_l scale q_l S_l[group].
 * statesT[l] (l = 1..L-1) is level l's transposed group states
 * [B,ng[l],H,V,K] (from ngdn_upper_scan_fwd) with firing interval f[l];
 * entries at l = 0 are ignored. o [B,T,H,V] in the working dtype. read0, when
 * not NULL, receives level 0's unmixed read Qg h + Aqk Vn, fp32 [B,T,H,V]
 * (the backward's dmix_0). K != V only with L == 1. */
int32_t ngdn_output_fwd(const ngdn_dims* d, const float* Qg, const float* Aqk,
                        const float* hT, const float* vnT, const void* q,
                        const void* mix, const float* const* statesT,
                        const int32_t* ng, const int32_t* f, void* o,
                        float* read0, void* stream);

/* ngdn_output_fwd in two passes, so that the first can run beside the upper
 * levels' promotions (it reads level 0 only): ngdn_output_l0_fwd writes
 * level 0's read Qg h + Aqk Vn into read0 (fp32 [B,T,H,V]); then
 * ngdn_output_upper_fwd forms o = mix_0 read0 + sum_{l>=1} mix_l scale q_l
 * S_l[group] with the same arguments as ngdn_output_fwd. Same results as the
 * one-pass entry point. */
int32_t ngdn_output_l0_fwd(const ngdn_dims* d, const float* Qg, const float* Aqk,
                           const float* hT, const float* vnT, float* read0, void* stream);
int32_t ngdn_output_upper_fwd(const ngdn_dims* d, const float* read0, const void* q,
                              const void* mix, const float* const* statesT,
                              const int32_t* ng, const int32_t* f, void* o, void* stream);

/* ---------------------------------------------------------------- backward
 * The backward of ChunkNestedGDN2Function (ops/chunk.py:650-719,
 * chunk_nested_gdn2_bwd :374-564), one entry point per stage. */

/* No counterpart in the reference (whose gradients leave its autograd in the
 * inputs' dtype): `count` (at most 16) fp32 arrays src[w] of n[w] elements
 * cast to bf16 into dst[w], rounding to nearest even, in one launch; the op
 * casts its fp32 gradients (dg, dmix, the parameter sums) this way into
 * separately allocated outputs. */
int32_t ngdn_cast_bf16(int32_t count, const float* const* src, void* const* dst,
                       const int64_t* n, void* stream);

/* No counterpart in the reference (whose kernels read the parameters as they
 * are): `count` (at most 8) arrays src[w] [batch[w]][rows[w]][cols[w]] of
 * elem_bytes-byte elements (2 or 4) transposed in their last two axes into
 * dst[w] [batch[w]][cols[w]][rows[w]], in one launch (at most 2^24 - 1
 * tiles of 32 x 32 in all, one 256-thread block each); the op lays out the
 * per-level parameters this way for the promotion kernels (the projections
 * and, for the backward, the bank with its last two axes swapped). */
int32_t ngdn_transpose(int32_t count, const void* const* src, void* const* dst,
                       const int32_t* batch, const int32_t* rows, const int32_t* cols,
                       int32_t elem_bytes, void* stream);

/* dmix for level 0 (ops/chunk.py:423): dmix[..., 0] = <do, read0> per token,
 * read0 fp32 [B,T,H,V] from ngdn_output_fwd, do [B,T,H,V]; dmix fp32
 * [B,T,H,L] (level-0 column written). */
int32_t ngdn_output_bwd(const ngdn_dims* d, const float* read0, const void* dout,
                        float* dmix, void* stream);

/* Backward of level `level`'s reads (read_level_bwd, ops/chunk.py:307-336,
 * and the dq / dmix terms of :423-449), per group of f chunks: states
 * [B,ng,H,K,V] fp32 are the level's group states. Writes d_states fp32
 * [B,ng,H,K,V], dq[..., level, :] (working dtype [B,T,H,L,K]) and
 * dmix[..., level] (fp32 [B,T,H,L]). */
int32_t ngdn_read_state_bwd(const ngdn_dims* d, int32_t level, int32_t f,
                            int32_t ng, const void* q, const void* mix,
                            const void* dout, const float* states,
                            float* d_states, void* dq, float* dmix,
                            void* stream);

/* Reverse level-0 state recurrence (the vendored fla dh kernel with dh_ext,
 * ops/_vendor/common_chunk_delta_h.py:25-380). W, KtT, Qg, Aqk and gam as
 * ngdn_l0_intra_fwd writes them (split; bf16 in fragment order): the scan
 * takes their transposes (Kt, W^T, Qg^T, Aqk^T) as its operands and forms
 * them on chip; inj
 * (fp32 [B,H,nf1,K,V], may be NULL) is level 1's gradient of the state
 * entering chunk (i+1)*f1, added before that chunk's step (the reference's
 * dh_ext, ops/chunk.py:519-528). d_final [B,H,L,K,V] fp32 (level-0 slot read,
 * may be NULL). Writes dSp [B,H,NT,K,V] (gradient of the state after each
 * chunk), dVn [B,H,NT,64,V] and dVnT [B,H,NT,V,64] (either may be NULL, not
 * both; ngdn_l0_bwd reads only dVnT), and d_initial[:, :, 0] when not NULL.
 * Runs chunks [chunk0, chunk0 + nchunk) (1 <= nchunk, chunk0 + nchunk <= NT)
 * in reverse: d_final is then the gradient of the state after the range's
 * last chunk and d_initial receives that of the state entering chunk0; the
 * two may be the same buffer (each workgroup reads its slice before writing
 * it), so consecutive ranges, last first, carry the gradient through it. */
int32_t ngdn_l0_scan_bwd(const ngdn_dims* d, const float* W, const float* KtT,
                         const float* gam, const float* Qg, const float* Aqk,
                         const void* dout, const void* mix, int32_t f1,
                         const float* inj, int32_t nf1, const float* d_final,
                         float* dSp, float* dVn, float* dVnT, float* d_initial,
                         int32_t chunk0, int32_t nchunk, void* stream);

/* Reverse write scan of level `level` >= 1 (ops/update_bwd.py:19-164): keys
 * [B,H,NF,N,K] and AT = (keys*b*e^g)^T [B,H,NF,K,N] (both split; AT in
 * fragment order for NGDN_BF16 with n_pairs % 32 == 0) from ngdn_probe_fwd, gam
 * [B,H,NF,K]; d_states fp32 [B,NG,H,K,V] (the reads' gradients); inj, when
 * not NULL, the level above's injection from its ngdn_probe_bwd (fp32
 * [B,H,nf_above,K,V]; firing i of interval f_above read this level's state
 * entering group ((i+1) f_above) / f_here, f_here this level's interval,
 * and its slot joins that group's gradient); d_final [B,H,L,K,V]. Writes dSp
 * fp32 [B,H,NF,K,V], dvn fp32 [B,H,NF,N,V] and d_initial[:, :, level] when
 * not NULL. */
int32_t ngdn_upper_scan_bwd(const ngdn_dims* d, int32_t level, int32_t n_pairs,
                            int32_t nf, int32_t ng, const float* keys,
                            const float* AT, const float* gam,
                            const float* d_states, const float* inj, int32_t f_here,
                            int32_t f_above, int32_t nf_above, const float* d_final,
                            float* dSp, float* dvn, float* d_initial,
                            void* stream);

/* Level-0 chunk backward, state half, from h and vn of ngdn_l0_scan_fwd:
 * dQg, dKt [B,H,NT,64,K], dWT [B,H,NT,K,64], dAqk [B,H,NT,64,64], dgam
 * [B,H,NT,K]. */
int32_t ngdn_l0_bwd_state(const ngdn_dims* d, const float* h, const float* dSp,
                          const float* vn, const float* dVn, const void* dout,
                          const void* mix, float* dQg, float* dWT, float* dKt,
                          float* dAqk, float* dgam, void* stream);

/* Level-0 chunk backward, intra half: writes dq[..., 0, :], dk, dv, db, dw
 * (working dtype) and dg (fp32 [B,T,H,K]). W (split), U, TT from
 * ngdn_l0_intra_fwd. */
int32_t ngdn_l0_bwd_intra(const ngdn_dims* d, const void* q, const void* k,
                          const void* v, const float* g, const void* b,
                          const void* w, const float* W, const float* U,
                          const float* TT, const float* dQg, const float* dWT,
                          const float* dKt, const float* dAqk, const float* dgam,
                          const float* dVnT, void* dq, void* dk, void* dv,
                          float* dg, void* db, void* dw, void* stream);

/* The two halves above in one launch (the rest of the vendored
 * chunk_gdn2_bwd, ops/_vendor/gdn2_chunk_bwd.py:26-187): the state half is
 * computed per chunk by the workgroup that uses it, from h [B,H,NT,K,V] and
 * vn [B,H,NT,64,V] of ngdn_l0_scan_fwd, dSp [B,H,NT,K,V] and dVnT of
 * ngdn_l0_scan_bwd, do and mix; its dQg and dKt pass through the workspaces
 * ws_dQg, ws_dKt (fp32 [B,H,NT,64,K] each, no initial contents), the rest
 * stays on chip. dA = -(dX_w W^T + dX_u U^T) is formed as -dX_u Vn^T (the
 * same, since dX_w = -dX_u S^T and W S = U - Vn), so W and U are not read; TT
 * from ngdn_l0_intra_fwd. Outputs as ngdn_l0_bwd_intra. Only chunks [chunk0,
 * chunk0 + nchunk) (1 <= nchunk, chunk0 + nchunk <= NT) are formed: a
 * caller can run them as soon as ngdn_l0_scan_bwd has covered them. */
int32_t ngdn_l0_bwd(const ngdn_dims* d, const void* q, const void* k, const void* v,
                    const float* g, const void* b, const void* w,
                    const float* TT, const float* h, const float* dSp,
                    const float* vn, const float* dVnT, const void* dout, const void* mix,
                    float* ws_dQg, float* ws_dKt, void* dq, void* dk, void* dv, float* dg,
                    void* db, void* dw, int32_t chunk0, int32_t nchunk, void* stream);

/* Backward of level `level`'s firings through its update and probe.
 * The lower level's states as rows (below_kv) and transposed (below_vk):
 * level 1 -> h and hT from ngdn_l0_scan_fwd (NG_below = NT); level >= 2 ->
 * the lower level's states and statesT from ngdn_upper_scan_fwd. Parameters
 * as for ngdn_probe_fwd plus kpT [L-1,H,V,K] (key projections transposed),
 * bankT [L-1,H,K,n_max] (banks transposed), and the untransposed bp, gp
 * [L-1,H,V,K], wp [L-1,H,V,V]. states [B,ng,H,K,V] and statesT [B,ng,H,V,K]
 * are this level's group states; dSp, dvn from ngdn_upper_scan_bwd.
 * Workspace (fp32): ws_vals, ws_du, ws_dxb, ws_dxg [B,H,NF,N,K], ws_dxw,
 * ws_dvals [B,H,NF,N,V], and ws_dbank [B,H,NF,N,K] (learned only): each
 * firing's bank-gradient partial, summed by ngdn_param_grads. The gradient
 * of the lower state a firing read goes to its slot of inj (fp32
 * [B,H,NF,K,V], written), which the lower level's reverse scan adds
 * (ngdn_l0_scan_bwd for level 1, ngdn_upper_scan_bwd otherwise); a firing
 * of level >= 2 that read the lower level's final state adds it to
 * d_final[:, :, level-1] instead. */
int32_t ngdn_probe_bwd(const ngdn_dims* d, int32_t level, int32_t promotion,
                       int32_t n_queries, int32_t f_below, int32_t f_here,
                       const float* below_kv, const float* below_vk,
                       int32_t ng_below, const float* final_state,
                       const void* query_banks, int32_t n_max,
                       const void* key_projections, const void* bpT,
                       const void* wpT, const void* gpT, const void* kpT,
                       const void* bankT, const void* bp, const void* wp,
                       const void* gp, const float* states,
                       const float* statesT, int32_t ng, const float* dSp,
                       const float* dvn, float* ws_vals, float* ws_du,
                       float* ws_dxb, float* ws_dxg, float* ws_dxw,
                       float* ws_dvals, float* ws_dbank, float* inj,
                       float* d_final, void* stream);

/* Slices of firings per head in the parameter-gradient sums (the first
 * dimension of ws_parts' slices). */
#define NGDN_PARAM_SPLIT 16

/* Per-head parameter gradients of level `level` summed over all its firings
 * (the leaf gradients of the probe replay, ops/chunk.py:502-517), from the
 * workspace of ngdn_probe_bwd; accumulated into fp32 dkp [L-1,H,K,V] (learned
 * only), dbp [L-1,H,V,K], dwp [L-1,H,V,V], dgp [L-1,H,V,K], and dbank
 * [L-1,H,n_max,K] (learned only, from ws_dbank). Deterministic: every sum
 * runs in a fixed order (partials per slice of firings in ws_parts, fp32
 * [4][H][NGDN_PARAM_SPLIT][K][V], no initial contents needed, then added
 * slice by slice), so repeated calls on the same inputs give the same bits. */
int32_t ngdn_param_grads(const ngdn_dims* d, int32_t level, int32_t promotion,
                         int32_t n_pairs, int32_t nf, const float* ws_vals,
                         const float* ws_du, const float* ws_dxb,
                         const float* ws_dxg, const float* ws_dxw,
                         const float* ws_dbank, int32_t n_max, float* dbank, float* dkp,
                         float* dbp, float* dwp, float* dgp, float* ws_parts, void* stream);

/* One decoding token: naive_step_nested_gdn2 (nested_gdn2/ops/naive.py:42-134;
 * the layer's decode and ragged-tail path, layers/nested_gdn2.py:218-224).
 * Level 0 writes (k, v, b, w, g), every level is read with its q slice and
 * mixed into o, then each level whose firing this token completes promotes,
 * bottom-up (the probe of the level below, then one firing of the update).
 * d->T is ignored. q [B,H,L,K]; k, b [B,H,K]; v, w [B,H,V]; mix [B,H,L] in
 * dtype; g [B,H,K] fp32; o [B,H,V] in dtype. state_in -> state_out
 * [B,H,L,K,V] fp32: the same buffer updates in place, distinct buffers must
 * not overlap. position: device int64 [B], each row's token index (firings
 * decided per row on the device, no host synchronisation), or NULL to use
 * position_all for every row (firings decided here, no launch for levels
 * that do not fire). A token fires level l when (pos + 1) % chunk_size == 0
 * and ((pos + 1) / chunk_size) % firing_intervals[l] == 0. firing_intervals
 * [L] and n_queries [L-1] are host arrays; parameters as for ngdn_probe_fwd
 * (every level's slice). When no level has more than 64 pairs per firing
 * (K for merge), the promotions of all levels run in one launch of B*H
 * workgroups; otherwise as two launches per level (probe, then the update)
 * through ws: fp32 workspace of B*H*(3*N*K + K) floats, N the most pairs of
 * any level (K for merge). */
int32_t ngdn_step(const ngdn_dims* d, const void* q, const void* k, const void* v,
                  const float* g, const void* b, const void* w, const void* mix,
                  const float* state_in, float* state_out, const int64_t* position,
                  int64_t position_all, int32_t chunk_size,
                  const int32_t* firing_intervals, int32_t promotion,
                  const int32_t* n_queries, const void* query_banks, int32_t n_max,
                  const void* key_projections, const void* bpT, const void* wpT,
                  const void* gpT, float* ws, void* o, void* stream);

/* Bytes of the device scratch that ngdn_step_noalloc uses (one copy per GPU,
 * held from the library's load until the process ends). */
#define NGDN_STEP_SCRATCH_BYTES (32u << 20)

/* ngdn_step without a workspace argument, and without allocating anything:
 * no counterpart in the reference. For callers that cannot allocate device
 * memory (code under HIP graph capture, tight decoding loops, harnesses that
 * forbid hipMalloc). Same arguments, results and errors as ngdn_step, minus
 * ws; the caller still passes every input and output. The levels with more
 * than 64 pairs per firing (K for merge), which ngdn_step runs through ws,
 * run through a file-scope device array of NGDN_STEP_SCRATCH_BYTES, a slice
 * of batch rows at a time; one batch row needs H * (3 N K + K) * 4 bytes, N
 * the most pairs of any level, and a call whose one row needs more than the
 * scratch holds fails with NGDN_EINVAL. Nothing in the scratch needs initial
 * contents. Every call on one GPU shares that GPU's scratch: calls that
 * overlap on one GPU (on different streams, or from different threads) race.
 * The current device must be the stream's device; the first call on a device
 * looks the scratch's address up (hipGetSymbolAddress) and keeps it. */
int32_t ngdn_step_noalloc(const ngdn_dims* d, const void* q, const void* k, const void* v,
                          const float* g, const void* b, const void* w, const void* mix,
                          const float* state_in, float* state_out, const int64_t* position,
                          int64_t position_all, int32_t chunk_size,
                          const int32_t* firing_intervals, int32_t promotion,
                          const int32_t* n_queries, const void* query_banks, int32_t n_max,
                          const void* key_projections, const void* bpT, const void* wpT,
                          const void* gpT, void* o, void* stream);

/* ---- The layer around the op (NestedGDN2Attention, layers/nested_gdn2.py),
 * which takes two modules from fla; these replace them. */

/* fla's ShortConvolution with activation "silu" (layers/nested_gdn2.py:57-60,
 * 122-130): per channel d, y[b,t,d] = act(sum_{i<W} w[d][i] x[b,t-(W-1)+i,d]),
 * act = SiLU when act != 0. x, y [B,T,D] in dtype; w [D][W] fp32 (the
 * module's weight [D,1,W]); rows before t = 0 come from cache_in (NULL:
 * zeros). The cache has fla's layout, [B,D,W] in dtype, the last W inputs with
 * the newest at index W-1; cache_out (NULL: not written, must not alias
 * cache_in) receives the last W rows of [cache_in; x], the state the next
 * call continues from. D % 8 == 0, 1 <= W <= 8. */
int32_t ngdn_short_conv_fwd(int32_t dtype, int32_t B, int32_t T, int32_t D, int32_t W,
                            int32_t act, const void* x, const float* w, const void* cache_in,
                            void* y, void* cache_out, void* stream);
/* Its backward: dx [B,T,D] (dtype) written, dw [D][W] fp32 summed into
 * (callers zero it). The gradient into cache_in is not formed. ws: fp32
 * [NGDN_WPARTS][D*W] (no initial contents needed) for the per-workgroup
 * partial sums of dw, added into dw by a second pass; or NULL to add every
 * partial into dw with device-scope atomics (several times slower). */
int32_t ngdn_short_conv_bwd(int32_t dtype, int32_t B, int32_t T, int32_t D, int32_t W,
                            int32_t act, const void* x, const float* w, const void* cache_in,
                            const void* dy, void* dx, float* dw, float* ws, void* stream);

/* fla's FusedRMSNormGated with activation "sigmoid" (layers/nested_gdn2.py:100,
 * 236): per row of V values, y = x rstd w sigmoid(g), rstd = 1 / sqrt(mean(x^2)
 * + eps). x, g, y [rows,V] in dtype; w [V] fp32; rstd [rows] fp32 written for
 * the backward (NULL: not written). V in {64, 128, 256}. */
int32_t ngdn_rmsnorm_gated_fwd(int32_t dtype, int64_t rows, int32_t V, float eps,
                               const void* x, const void* g, const float* w, void* y,
                               float* rstd, void* stream);
/* Its backward from the forward's rstd: dx, dg [rows,V] (dtype) written, dw
 * [V] fp32 summed into (callers zero it); ws fp32 [NGDN_WPARTS][V] or NULL
 * (as for ngdn_short_conv_bwd). */
int32_t ngdn_rmsnorm_gated_bwd(int32_t dtype, int64_t rows, int32_t V, const void* x,
                               const void* g, const float* w, const float* rstd,
                               const void* dy, void* dx, void* dg, float* dw, float* ws,
                               void* stream);

/* The layer's gate prologue (layers/nested_gdn2.py:134-166), from the
 * convolved projections to the op's inputs, per token t and head h:
 *   qn[t,h,l,:] = normalize(q[t, l*H*K + h*K + :])   (q in "b t (l h d)" order)
 *   kn[t,h,:]   = normalize(k[t, h*K + :])
 *   g0[t,h,:]   = min(-exp(A_log[h]) softplus(f[t, h*K + :] + dt_bias[h*K + :]), cap)
 *   b0 = sigmoid(bz), w0 = sigmoid(wz), mix[t,h,:] = softmax (or sigmoid) of ml[t, h*L + :]
 * normalize(x) = x / max(|x|, 1e-12) (F.normalize), softplus with torch's
 * threshold 20. BT = B*T tokens; q, k, f, bz, wz, ml, qn, kn, b0, w0, mix in
 * dtype; g0 fp32 [BT,H,K]; A_log [H] and dt_bias [H*K] in param_dtype.
 * cap = -1/max_horizon, or +inf. K, V in {64, 128}, 1 <= L <= 8. The
 * backward reads the forward inputs and the gradients dqn, dkn, dg0 (fp32),
 * db0, dw0, dmix of the six outputs, writes dq, dk, df, dbz, dwz, dml, and
 * adds the decay parameters' gradients into dpar (fp32 [H*K + H]: dt_bias,
 * then A_log; callers zero it) through ws (fp32 [NGDN_WPARTS][H*K + H], or
 * NULL: device-scope atomics). */
typedef struct ngdn_gate_args {
  int64_t BT;
  int32_t H, L, K, V;
  int32_t param_dtype, sigmoid_mix;
  float cap;
  const void *q, *k, *f, *bz, *wz, *ml, *A_log, *dt_bias;
  void *qn, *kn;
  float* g0;
  void *b0, *w0, *mix;
  const void *dqn, *dkn;
  const float* dg0;
  const void *db0, *dw0, *dmix;
  void *dq, *dk, *df, *dbz, *dwz, *dml;
  float *dpar, *ws;
} ngdn_gate_args;
int32_t ngdn_gate_prep_fwd(int32_t dtype, const ngdn_gate_args* g, void* stream);
int32_t ngdn_gate_prep_bwd(int32_t dtype, const ngdn_gate_args* g, void* stream);

/* ---- The model around the layer (NestedGDN2ForCausalLM,
 * models/modeling_nested_gdn2.py), which takes three more modules from fla;
 * these replace their kernels (the linear maps stay GEMMs of the caller). */

/* fla's RMSNorm (models/modeling_nested_gdn2.py:16,46-49,97-99): per row of D
 * values, y = x rstd w, rstd = 1 / sqrt(mean(x^2) + eps). x, y [rows,D] in
 * dtype; w [D] fp32; rstd [rows] fp32 written for the backward (NULL: not
 * written). D = 512 n for n in 1..6, or D in {64, 128, 256, 768}. */
int32_t ngdn_rmsnorm_fwd(int32_t dtype, int64_t rows, int32_t D, float eps, const void* x,
                         const float* w, void* y, float* rstd, void* stream);
/* Its backward from the forward's rstd: dx [rows,D] (dtype) written, dw [D]
 * fp32 summed into (callers zero it); ws fp32 [NGDN_WPARTS][D] or NULL (as
 * for ngdn_short_conv_bwd). */
int32_t ngdn_rmsnorm_bwd(int32_t dtype, int64_t rows, int32_t D, const void* x, const float* w,
                         const float* rstd, const void* dy, void* dx, float* dw, float* ws,
                         void* stream);

/* The block's residual add fused into the RMSNorm after it (no counterpart
 * entry point: the reference adds in Python, models/modeling_nested_gdn2.py:
 * 59-67, then calls fla's RMSNorm; the results are the same). With r set:
 * h = x + r rounded to x's dtype (written, [rows,D]) and y = RMSNorm(h) as
 * ngdn_rmsnorm_fwd; r NULL: y = RMSNorm(x), h untouched. y in y_dtype, so a
 * norm whose consumer computes in bf16 (autocast) writes bf16 directly.
 * Dtype combinations (x, r, y): all NGDN_F32, all NGDN_BF16, or NGDN_F32 x
 * with NGDN_BF16 r and y (r's code also selects the combination when r is
 * NULL). D as for ngdn_rmsnorm_fwd. */
int32_t ngdn_add_rmsnorm_fwd(int32_t x_dtype, int32_t r_dtype, int32_t y_dtype, int64_t rows,
                             int32_t D, float eps, const void* x, const void* r, const float* w,
                             void* h, void* y, float* rstd, void* stream);
/* Its backward from h (x when r was NULL) and the forward's rstd: dx = the
 * norm's input gradient plus dh (the gradient h receives from elsewhere, the
 * residual path; NULL: none), in x_dtype; dr (NULL: not written) the same
 * values in r_dtype; dy in y_dtype; dw and ws as for ngdn_rmsnorm_bwd. */
int32_t ngdn_add_rmsnorm_bwd(int32_t x_dtype, int32_t r_dtype, int32_t y_dtype, int64_t rows,
                             int32_t D, const void* h, const float* w, const float* rstd,
                             const void* dy, const void* dh, void* dx, void* dr, float* dw,
                             float* ws, void* stream);

/* The SwiGLU of fla's GatedMLP (models/modeling_nested_gdn2.py:17,50-56):
 * y = silu(g) u elementwise over n values (n % 8 == 0), all in dtype. */
int32_t ngdn_swiglu_fwd(int32_t dtype, int64_t n, const void* g, const void* u, void* y, void* stream);
/* Its backward: dg = dy u silu'(g), du = dy silu(g). */
int32_t ngdn_swiglu_bwd(int32_t dtype, int64_t n, const void* g, const void* u, const void* dy,
                        void* dg, void* du, void* stream);

/* out[i] = sum_{j < count} xs[j][i] in fp32, xs[j] in dtype, n % 8 == 0,
 * 1 <= count <= 8 (xs a host array of device pointers). The gradient of a
 * tensor that feeds several linear maps under autocast (the layer's eight
 * projections of x): one pass instead of a cast and an addition per
 * consumer. No counterpart in fla; it replaces autograd's accumulation. */
int32_t ngdn_sum_f32(int32_t dtype, int32_t count, const void* const* xs, int64_t n, float* out,
                     void* stream);

/* The cross entropy of fla's FusedLinearCrossEntropyLoss
 * (models/modeling_nested_gdn2.py:230-239; mean over the labels that are not
 * ignore_index): row_loss[r] = (logsumexp(logits_r) - logits_r[labels_r]) /
 * n_valid, 0 where labels_r == ignore_index (row_loss fp32 [rows]; the loss is
 * their sum). n_valid points to the device int64 count of labels that are not
 * ignore_index. With grad != 0 the logits [rows,V] (dtype) are overwritten by
 * d(loss)/d(logits) = (softmax - onehot) / n_valid, zeros on ignored rows.
 * A label outside [0, V) that is not ignore_index gives NaN on its row, and
 * n_valid == 0 gives NaN (the mean over no labels).
 * V % 8 == 0, V <= 65536. */
int32_t ngdn_cross_entropy(int32_t dtype, int64_t rows, int32_t V, int32_t ignore_index,
                           void* logits, const int64_t* labels, const int64_t* n_valid,
                           float* row_loss, int32_t grad, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NGDN_H */
