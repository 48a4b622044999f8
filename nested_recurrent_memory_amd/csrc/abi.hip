// extern "C" entry points of libngdn.so: argument checks, then launches.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <mutex>

#include "ngdn_kernels.h"

namespace {

thread_local char g_err[512] = "";

int32_t fail(int32_t code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int32_t launched(hipError_t e, const char* what) {
  if (e == hipSuccess) return NGDN_OK;
  if (e == hipErrorInvalidValue)
    return fail(NGDN_EINVAL, "%s: unsupported shape combination", what);
  return fail(NGDN_ELAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
}

bool pow2_ge16(int n) { return n >= 16 && n <= 128 && (n & (n - 1)) == 0; }

int32_t check_dims(const ngdn_dims* d, const char* what) {
  if (!d) return fail(NGDN_EINVAL, "%s: dims is NULL", what);
  if (d->B <= 0 || d->T <= 0 || d->H <= 0 || d->L <= 0 || d->L > ngdn::MAXL)
    return fail(NGDN_EINVAL, "%s: bad sizes B=%d T=%d H=%d L=%d", what, d->B, d->T, d->H, d->L);
  if (!((d->K == 64 || d->K == 128) && (d->V == 64 || d->V == 128)))
    return fail(NGDN_EINVAL, "%s: K=%d V=%d unsupported (64 or 128)", what, d->K, d->V);
  if (d->dtype != NGDN_F32 && d->dtype != NGDN_BF16)
    return fail(NGDN_EINVAL, "%s: dtype %d unsupported", what, d->dtype);
  if (d->hold_partial != 0 && d->hold_partial != 1)
    return fail(NGDN_EINVAL, "%s: hold_partial %d is neither 0 nor 1", what, d->hold_partial);
  // the largest grids are one 512-thread workgroup per (batch, head, chunk):
  // their work-items must fit 32 bits
  const long long bhc = (long long)d->B * d->H * ((d->T + ngdn::CH - 1) / ngdn::CH);
  if (bhc > (1LL << 23) - 1)
    return fail(NGDN_EINVAL, "%s: B*H*chunks = %lld exceeds %lld", what, bhc, (1LL << 23) - 1);
  return NGDN_OK;
}

inline int nchunks(const ngdn_dims* d) { return (d->T + ngdn::CH - 1) / ngdn::CH; }
// chunks [chunk0, chunk0 + nchunk) inside the sequence's NT chunks
int32_t check_range(const ngdn_dims* d, int32_t chunk0, int32_t nchunk, const char* what) {
  if (chunk0 < 0 || nchunk < 1 || chunk0 > nchunks(d) - nchunk)
    return fail(NGDN_EINVAL, "%s: chunks [%d, %d + %d) outside the %d chunks of the sequence",
                what, chunk0, chunk0, nchunk, nchunks(d));
  return NGDN_OK;
}
// chunks whose end can complete an upper level's firing
inline int fire_chunks(const ngdn_dims* d) {
  return d->hold_partial ? d->T / ngdn::CH : nchunks(d);
}

}  // namespace

extern "C" {

const char* ngdn_last_error(void) { return g_err; }
int32_t ngdn_version(void) { return NGDN_VERSION; }
const char* ngdn_arch(void) { return "gfx950"; }

int32_t ngdn_l0_intra_fwd(const ngdn_dims* d, const void* q, const void* k,
                          const void* v, const float* g, const void* b,
                          const void* w, float* W, float* U, float* KtT, float* Qg,
                          float* Aqk, float* gam, float* TT, int32_t chunk0,
                          int32_t nchunk, void* stream) {
  g_err[0] = 0;
  if (int32_t r = check_dims(d, "ngdn_l0_intra_fwd")) return r;
  if (!q || !k || !v || !g || !b || !w || !W || !U || !KtT || !Qg || !Aqk || !gam)
    return fail(NGDN_EINVAL, "ngdn_l0_intra_fwd: NULL tensor");
  if (int32_t r = check_range(d, chunk0, nchunk, "ngdn_l0_intra_fwd")) return r;
  ngdn::L0IntraArgs a{q, k, v, g, b, w, W, U, KtT, Qg, Aqk, gam, TT,
                      d->B, d->T, d->H, d->L, nchunks(d), d->scale, chunk0, nchunk};
  return launched(ngdn::l0_intra_fwd(a, d->dtype, d->K, d->V, (hipStream_t)stream),
                  "ngdn_l0_intra_fwd");
}

int32_t ngdn_l0_scan_fwd(const ngdn_dims* d, const float* W, const float* U,
                         const float* KtT, const float* gam, const float* Qg,
                         const float* Aqk, const float* initial_state, int32_t hT_every,
                         float* hT, float* vnT, float* h, float* vn, float* read0,
                         float* final_state, int32_t chunk0, int32_t nchunk, void* stream) {
  g_err[0] = 0;
  if (int32_t r = check_dims(d, "ngdn_l0_scan_fwd")) return r;
  if (!W || !U || !KtT || !gam || !final_state || (read0 && (!Qg || !Aqk)))
    return fail(NGDN_EINVAL, "ngdn_l0_scan_fwd: NULL tensor");
  if (int32_t r = check_range(d, chunk0, nchunk, "ngdn_l0_scan_fwd")) return r;
  if (hT && hT_every < 1)
    return fail(NGDN_EINVAL, "ngdn_l0_scan_fwd: hT_every must be >= 1, got %d", hT_every);
  const long long skv = (long long)d->K * d->V;
  ngdn::ScanArgs a{};
  a.A = W; a.BT = KtT; a.U = U; a.gam = gam;
  a.init = initial_state; a.init_sh = d->L * skv; a.init_sb = d->H * a.init_sh;
  a.st_vk = hT; a.vk_every = hT_every; a.st_kv = h; a.state_mode = 0; a.NG = nchunks(d);
  a.vnT = vnT; a.vn = vn;
  a.Qg = Qg; a.Aqk = Aqk; a.read0 = read0; a.T = d->T;
  a.fin = final_state; a.fin_sh = d->L * skv; a.fin_sb = d->H * a.fin_sh;
  a.B = d->B; a.H = d->H; a.S = nchunks(d); a.M = ngdn::CH; a.V = d->V;
  a.frag = d->dtype == NGDN_BF16 ? 3 : 0;   // W, KtT, Qg, Aqk: fragment order
  a.j0 = chunk0; a.j1 = chunk0 + nchunk;
  return launched(ngdn::scan_fwd(a, d->dtype, d->K, (hipStream_t)stream), "ngdn_l0_scan_fwd");
}

int32_t ngdn_probe_fwd(const ngdn_dims* d, int32_t level, int32_t promotion,
                       int32_t n_queries, int32_t f_below, int32_t f_here,
                       const float* below, int32_t ng_below,
                       const float* final_state, const void* query_banks,
                       int32_t n_max, const void* key_projections,
                       const void* bpT, const void* wpT, const void* gpT,
                       float* A, float* KT, float* U, float* gam, float* keysN,
                       float* AT, float* keys, float* vals, float* bo, float* wo,
                       float* go, int32_t firing0, int32_t nfiring, void* stream) {
  g_err[0] = 0;
  if (int32_t r = check_dims(d, "ngdn_probe_fwd")) return r;
  if (level < 1 || level >= d->L)
    return fail(NGDN_EINVAL, "ngdn_probe_fwd: level %d outside [1, L=%d)", level, d->L);
  if (d->K != d->V)
    return fail(NGDN_EINVAL, "ngdn_probe_fwd: promotion needs K == V, got %d, %d", d->K, d->V);
  if (promotion != 0 && promotion != 1)
    return fail(NGDN_EINVAL, "ngdn_probe_fwd: promotion %d unknown", promotion);
  const int N = promotion == 1 ? d->K : n_queries;
  if (!pow2_ge16(N))
    return fail(NGDN_EINVAL, "ngdn_probe_fwd: pairs per firing must be a power of two >= 16 "
                "(and <= 128), got %d", N);
  if (promotion == 0 && (n_queries > n_max || !query_banks || !key_projections))
    return fail(NGDN_EINVAL, "ngdn_probe_fwd: n_queries=%d exceeds bank rows %d", n_queries, n_max);
  if (f_below <= 0 || f_here <= 0)
    return fail(NGDN_EINVAL, "ngdn_probe_fwd: firing intervals must be positive");
  if (!below || !final_state || !bpT || !wpT || !gpT || !A || !KT || !U || !gam)
    return fail(NGDN_EINVAL, "ngdn_probe_fwd: NULL tensor");
  const long long skv = (long long)d->K * d->V;
  ngdn::ProbeArgs a{};
  a.below = below; a.below_mode = level == 1 ? 0 : 1; a.NGb = ng_below;
  a.below_fin = final_state + (long long)(level - 1) * skv;
  a.bf_sh = d->L * skv; a.bf_sb = d->H * a.bf_sh;
  a.f_below = f_below; a.f_here = f_here;
  const size_t hkv = (size_t)d->H * skv;
  const size_t esz = d->dtype == NGDN_BF16 ? 2 : 4;
  auto lvl = [&](const void* p, size_t per) -> const void* {
    return p ? static_cast<const char*>(p) + (size_t)(level - 1) * per * esz : nullptr;
  };
  a.bank = lvl(query_banks, (size_t)d->H * n_max * d->K); a.Nmax = n_max;
  a.kp = lvl(key_projections, hkv);
  a.bpT = lvl(bpT, hkv); a.wpT = lvl(wpT, hkv); a.gpT = lvl(gpT, hkv);
  a.merge = promotion;
  a.A = A; a.KT = KT; a.U = U; a.gam = gam; a.keysN = keysN; a.AT = AT;
  a.keys = keys; a.vals = vals; a.bo = bo; a.wo = wo; a.go = go;
  a.B = d->B; a.H = d->H; a.NF = fire_chunks(d) / f_here; a.N = N; a.V = d->V;
  if (firing0 < 0 || nfiring < 0 || firing0 > a.NF - nfiring)
    return fail(NGDN_EINVAL, "ngdn_probe_fwd: firings [%d, %d + %d) outside the level's %d",
                firing0, firing0, nfiring, a.NF);
  if (nfiring == 0) return NGDN_OK;
  a.i0 = firing0; a.ni = nfiring;
  return launched(ngdn::probe_fwd(a, d->dtype, d->K, (hipStream_t)stream), "ngdn_probe_fwd");
}

int32_t ngdn_promote_chain_fwd(const ngdn_dims* d, int32_t level, int32_t promotion,
                               int32_t n_queries, int32_t f_below, int32_t f_here,
                               const float* below, int32_t ng_below,
                               float* final_state, const void* query_banks,
                               int32_t n_max, const void* key_projections,
                               const void* bpT, const void* wpT, const void* gpT,
                               const float* initial_state, float* states, float* statesT,
                               float* keysN, float* AT, float* gam, void* stream) {
  g_err[0] = 0;
  const char* what = "ngdn_promote_chain_fwd";
  if (int32_t r = check_dims(d, what)) return r;
  if (level < 1 || level >= d->L)
    return fail(NGDN_EINVAL, "%s: level %d outside [1, L=%d)", what, level, d->L);
  if (d->K != d->V)
    return fail(NGDN_EINVAL, "%s: promotion needs K == V, got %d, %d", what, d->K, d->V);
  if (promotion != 0 && promotion != 1)
    return fail(NGDN_EINVAL, "%s: promotion %d unknown", what, promotion);
  const int N = promotion == 1 ? d->K : n_queries;
  if (!pow2_ge16(N))
    return fail(NGDN_EINVAL, "%s: pairs per firing must be a power of two >= 16 "
                "(and <= 128), got %d", what, N);
  if (!ngdn::promote_chain_supported(d->K, N, promotion == 1))
    return fail(NGDN_EINVAL, "%s: %d pairs per firing at K=%d (%s) need the two-launch path "
                "(ngdn_probe_fwd, ngdn_upper_scan_fwd)", what, N, d->K,
                promotion == 1 ? "merge" : "learned");
  if (promotion == 0 && (n_queries > n_max || !query_banks || !key_projections))
    return fail(NGDN_EINVAL, "%s: n_queries=%d exceeds bank rows %d", what, n_queries, n_max);
  if (f_below <= 0 || f_here <= 0)
    return fail(NGDN_EINVAL, "%s: firing intervals must be positive", what);
  if (!below || !final_state || !bpT || !wpT || !gpT || !states || !statesT)
    return fail(NGDN_EINVAL, "%s: NULL tensor", what);
  if ((keysN || AT || gam) && !(keysN && AT && gam))
    return fail(NGDN_EINVAL, "%s: keys, AT and gam are written together", what);
  const int NT = nchunks(d);
  const long long skv = (long long)d->K * d->V;
  ngdn::PromoteChainArgs a{};
  a.below = below; a.below_mode = level == 1 ? 0 : 1; a.NGb = ng_below;
  a.below_fin = final_state + (long long)(level - 1) * skv;
  a.bf_sh = d->L * skv; a.bf_sb = d->H * a.bf_sh;
  a.f_below = f_below; a.f_here = f_here;
  const size_t hkv = (size_t)d->H * skv;
  const size_t esz = d->dtype == NGDN_BF16 ? 2 : 4;
  auto lvl = [&](const void* p, size_t per) -> const void* {
    return p ? static_cast<const char*>(p) + (size_t)(level - 1) * per * esz : nullptr;
  };
  a.bank = lvl(query_banks, (size_t)d->H * n_max * d->K); a.Nmax = n_max;
  a.kp = lvl(key_projections, hkv);
  a.bpT = lvl(bpT, hkv); a.wpT = lvl(wpT, hkv); a.gpT = lvl(gpT, hkv);
  a.init = initial_state ? initial_state + (long long)level * skv : nullptr;
  a.init_sh = d->L * skv; a.init_sb = d->H * a.init_sh;
  a.st_kv = states; a.st_vk = statesT;
  a.fin = final_state + (long long)level * skv; a.fin_sh = a.init_sh; a.fin_sb = a.init_sb;
  a.keysN = keysN; a.AT = AT; a.gam = gam;
  a.B = d->B; a.H = d->H; a.NF = fire_chunks(d) / f_here; a.NG = (NT + f_here - 1) / f_here;
  return launched(ngdn::promote_chain_fwd(a, d->dtype, d->K, N, promotion == 1,
                                          (hipStream_t)stream), what);
}

int32_t ngdn_upper_scan_fwd(const ngdn_dims* d, int32_t level, int32_t n_pairs,
                            int32_t nf, int32_t ng, const float* A,
                            const float* KT, const float* U, const float* gam,
                            const float* initial_state, float* states,
                            float* statesT, float* final_state, int32_t step0,
                            int32_t nstep, void* stream) {
  g_err[0] = 0;
  if (int32_t r = check_dims(d, "ngdn_upper_scan_fwd")) return r;
  if (level < 1 || level >= d->L)
    return fail(NGDN_EINVAL, "ngdn_upper_scan_fwd: level %d outside [1, L=%d)", level, d->L);
  if (!pow2_ge16(n_pairs))
    return fail(NGDN_EINVAL, "ngdn_upper_scan_fwd: pairs per firing must be a power of two >= 16 "
                "(and <= 128), got %d", n_pairs);
  if (!(ng - 1 <= nf && nf <= ng) || nf < 0)
    return fail(NGDN_EINVAL, "ngdn_upper_scan_fwd: NF=%d inconsistent with n_groups=%d", nf, ng);
  if ((nf > 0 && (!A || !KT || !U || !gam)) || !states || !final_state)
    return fail(NGDN_EINVAL, "ngdn_upper_scan_fwd: NULL tensor");
  if (nf > 0 ? (step0 < 0 || nstep < 1 || step0 > nf - nstep) : (step0 != 0 || nstep != 0))
    return fail(NGDN_EINVAL, "ngdn_upper_scan_fwd: firings [%d, %d + %d) outside the level's %d",
                step0, step0, nstep, nf);
  const long long skv = (long long)d->K * d->V;
  ngdn::ScanArgs a{};
  a.A = A; a.BT = KT; a.U = U; a.gam = gam;
  a.j0 = step0; a.j1 = step0 + nstep;
  a.init = initial_state ? initial_state + (long long)level * skv : nullptr;
  a.init_sh = d->L * skv; a.init_sb = d->H * a.init_sh;
  a.st_kv = states; a.st_vk = statesT; a.state_mode = 1; a.NG = ng;
  a.vnT = nullptr; a.vn = nullptr;
  a.fin = final_state + (long long)level * skv; a.fin_sh = d->L * skv; a.fin_sb = d->H * a.fin_sh;
  a.B = d->B; a.H = d->H; a.S = nf; a.M = n_pairs; a.V = d->V;
  a.frag = d->dtype == NGDN_BF16 && n_pairs % 32 == 0;   // KT as ngdn_probe_fwd writes it
  return launched(ngdn::scan_fwd(a, d->dtype, d->K, (hipStream_t)stream), "ngdn_upper_scan_fwd");
}

int32_t ngdn_output_fwd(const ngdn_dims* d, const float* Qg, const float* Aqk,
                        const float* hT, const float* vnT, const void* q,
                        const void* mix, const float* const* statesT,
                        const int32_t* ng, const int32_t* f, void* o,
                        float* read0, void* stream) {
  g_err[0] = 0;
  if (int32_t r = check_dims(d, "ngdn_output_fwd")) return r;
  if (d->L > 1 && d->K != d->V)
    return fail(NGDN_EINVAL, "ngdn_output_fwd: upper levels need K == V, got %d, %d", d->K, d->V);
  if (!Qg || !Aqk || !hT || !vnT || !q || !mix || !o)
    return fail(NGDN_EINVAL, "ngdn_output_fwd: NULL tensor");
  ngdn::OutputArgs a{};
  a.Qg = Qg; a.Aqk = Aqk; a.hT = hT; a.vnT = vnT; a.q = q; a.mix = mix;
  for (int l = 1; l < d->L; ++l) {
    if (!statesT || !statesT[l] || !ng || !f || f[l] <= 0)
      return fail(NGDN_EINVAL, "ngdn_output_fwd: level %d states missing", l);
    a.statesT[l] = statesT[l]; a.NGl[l] = ng[l]; a.f[l] = f[l];
  }
  a.o = o; a.read0 = read0;
  a.B = d->B; a.T = d->T; a.H = d->H; a.L = d->L; a.NT = nchunks(d); a.scale = d->scale;
  return launched(ngdn::output_fwd(a, d->dtype, d->K, d->V, (hipStream_t)stream), "ngdn_output_fwd");
}


int32_t ngdn_output_l0_fwd(const ngdn_dims* d, const float* Qg, const float* Aqk,
                           const float* hT, const float* vnT, float* read0, void* stream) {
  g_err[0] = 0;
  if (int32_t r = check_dims(d, "ngdn_output_l0_fwd")) return r;
  if (!Qg || !Aqk || !hT || !vnT || !read0)
    return fail(NGDN_EINVAL, "ngdn_output_l0_fwd: NULL tensor");
  ngdn::OutputArgs a{};
  a.Qg = Qg; a.Aqk = Aqk; a.hT = hT; a.vnT = vnT; a.read0 = read0; a.l0_only = 1;
  a.B = d->B; a.T = d->T; a.H = d->H; a.L = d->L; a.NT = nchunks(d); a.scale = d->scale;
  return launched(ngdn::output_fwd(a, d->dtype, d->K, d->V, (hipStream_t)stream),
                  "ngdn_output_l0_fwd");
}

int32_t ngdn_output_upper_fwd(const ngdn_dims* d, const float* read0, const void* q,
                              const void* mix, const float* const* statesT,
                              const int32_t* ng, const int32_t* f, void* o, void* stream) {
  g_err[0] = 0;
  if (int32_t r = check_dims(d, "ngdn_output_upper_fwd")) return r;
  if (d->L > 1 && d->K != d->V)
    return fail(NGDN_EINVAL, "ngdn_output_upper_fwd: upper levels need K == V, got %d, %d",
                d->K, d->V);
  if (!read0 || !q || !mix || !o) return fail(NGDN_EINVAL, "ngdn_output_upper_fwd: NULL tensor");
  ngdn::OutputArgs a{};
  a.q = q; a.mix = mix; a.read0_in = read0;
  for (int l = 1; l < d->L; ++l) {
    if (!statesT || !statesT[l] || !ng || !f || f[l] <= 0)
      return fail(NGDN_EINVAL, "ngdn_output_upper_fwd: level %d states missing", l);
    a.statesT[l] = statesT[l]; a.NGl[l] = ng[l]; a.f[l] = f[l];
  }
  a.o = o;
  a.B = d->B; a.T = d->T; a.H = d->H; a.L = d->L; a.NT = nchunks(d); a.scale = d->scale;
  return launched(ngdn::output_fwd(a, d->dtype, d->K, d->V, (hipStream_t)stream),
                  "ngdn_output_upper_fwd");
}

int32_t ngdn_cast_bf16(int32_t count, const float* const* src, void* const* dst,
                       const int64_t* n, void* stream) {
  g_err[0] = 0;
  if (count < 0 || count > ngdn::CAST_MAX || (count > 0 && (!src || !dst || !n)))
    return fail(NGDN_EINVAL, "ngdn_cast_bf16: %d arrays (at most %d)", count, ngdn::CAST_MAX);
  ngdn::CastArgs a{};
  a.count = count;
  for (int w = 0; w < count; ++w) {
    if (n[w] < 0 || (n[w] > 0 && (!src[w] || !dst[w])))
      return fail(NGDN_EINVAL, "ngdn_cast_bf16: array %d NULL or of negative size", w);
    a.src[w] = src[w]; a.dst[w] = dst[w]; a.n[w] = n[w];
  }
  return launched(ngdn::cast_bf16(a, (hipStream_t)stream), "ngdn_cast_bf16");
}

int32_t ngdn_transpose(int32_t count, const void* const* src, void* const* dst,
                       const int32_t* batch, const int32_t* rows, const int32_t* cols,
                       int32_t elem_bytes, void* stream) {
  g_err[0] = 0;
  if (count < 0 || count > ngdn::TR_MAX || (count > 0 && (!src || !dst || !batch || !rows || !cols)))
    return fail(NGDN_EINVAL, "ngdn_transpose: %d arrays (at most %d)", count, ngdn::TR_MAX);
  if (elem_bytes != 2 && elem_bytes != 4)
    return fail(NGDN_EINVAL, "ngdn_transpose: elements of %d bytes (2 or 4)", elem_bytes);
  ngdn::TransposeArgs a{};
  a.count = count; a.esz = elem_bytes;
  long long tiles = 0;
  for (int w = 0; w < count; ++w) {
    if (batch[w] < 0 || rows[w] < 0 || cols[w] < 0 ||
        (batch[w] > 0 && rows[w] > 0 && cols[w] > 0 && (!src[w] || !dst[w])))
      return fail(NGDN_EINVAL, "ngdn_transpose: array %d NULL or of negative size", w);
    a.src[w] = src[w]; a.dst[w] = dst[w];
    a.batch[w] = batch[w]; a.R[w] = rows[w]; a.C[w] = cols[w];
    a.tiles0[w] = (int)tiles;
    tiles += (long long)batch[w] * ((rows[w] + 31) / 32) * ((cols[w] + 31) / 32);
    // one 256-thread block per tile: the grid's work-items must fit 32 bits
    if (tiles > (1LL << 24) - 1)
      return fail(NGDN_EINVAL, "ngdn_transpose: %lld tiles of 32 x 32 (at most %lld)", tiles,
                  (1LL << 24) - 1);
  }
  a.tiles0[count] = (int)tiles;
  return launched(ngdn::transpose(a, (hipStream_t)stream), "ngdn_transpose");
}

int32_t ngdn_output_bwd(const ngdn_dims* d, const float* read0, const void* dout,
                        float* dmix, void* stream) {
  g_err[0] = 0;
  if (int32_t r = check_dims(d, "ngdn_output_bwd")) return r;
  if (!read0 || !dout || !dmix) return fail(NGDN_EINVAL, "ngdn_output_bwd: NULL tensor");
  ngdn::Dmix0Args a{read0, dout, dmix, d->B, d->T, d->H, d->L, d->V};
  return launched(ngdn::dmix0_bwd(a, d->dtype, (hipStream_t)stream), "ngdn_output_bwd");
}

int32_t ngdn_read_state_bwd(const ngdn_dims* d, int32_t level, int32_t f,
                            int32_t ng, const void* q, const void* mix,
                            const void* dout, const float* states,
                            float* d_states, void* dq, float* dmix,
                            void* stream) {
  g_err[0] = 0;
  if (int32_t r = check_dims(d, "ngdn_read_state_bwd")) return r;
  if (level < 1 || level >= d->L || f <= 0 || ng != (nchunks(d) + f - 1) / f)
    return fail(NGDN_EINVAL, "ngdn_read_state_bwd: level %d / interval %d / groups %d inconsistent",
                level, f, ng);
  if (d->K != d->V) return fail(NGDN_EINVAL, "ngdn_read_state_bwd: K == V required");
  if (!q || !mix || !dout || !states || !d_states || !dq || !dmix)
    return fail(NGDN_EINVAL, "ngdn_read_state_bwd: NULL tensor");
  ngdn::ReadStateBwdArgs a{q, mix, dout, states, d_states, dq, dmix,
                           d->B, d->T, d->H, d->L, level, f, ng, d->scale};
  return launched(ngdn::read_state_bwd(a, d->dtype, d->K, d->V, (hipStream_t)stream),
                  "ngdn_read_state_bwd");
}

int32_t ngdn_l0_scan_bwd(const ngdn_dims* d, const float* W, const float* KtT,
                         const float* gam, const float* Qg, const float* Aqk,
                         const void* dout, const void* mix, int32_t f1,
                         const float* inj, int32_t nf1, const float* d_final,
                         float* dSp, float* dVn, float* dVnT, float* d_initial,
                         int32_t chunk0, int32_t nchunk, void* stream) {
  g_err[0] = 0;
  if (int32_t r = check_dims(d, "ngdn_l0_scan_bwd")) return r;
  if (int32_t r = check_range(d, chunk0, nchunk, "ngdn_l0_scan_bwd")) return r;
  if (!W || !KtT || !gam || !Qg || !Aqk || !dout || !mix || !dSp || (!dVn && !dVnT))
    return fail(NGDN_EINVAL, "ngdn_l0_scan_bwd: NULL tensor");
  const int NT = nchunks(d);
  if (inj && (f1 <= 0 || nf1 != fire_chunks(d) / f1))
    return fail(NGDN_EINVAL, "ngdn_l0_scan_bwd: injection count %d inconsistent with f1=%d", nf1, f1);
  const long long skv = (long long)d->K * d->V;
  ngdn::ScanBwdArgs a{};
  a.W = W; a.KtT = KtT; a.Qg = Qg; a.Aqk = Aqk; a.gam = gam;
  a.dout = dout; a.mix = mix; a.T = d->T; a.L = d->L;
  a.inj = inj; a.inj_every = inj ? f1 : 1; a.inj_nf = nf1;
  a.d_states = nullptr; a.NG = NT;
  a.d_final = d_final; a.df_sh = d->L * skv; a.df_sb = d->H * a.df_sh;
  a.dSp = dSp; a.dVn = dVn; a.dVnT = dVnT;
  a.dinit = d_initial; a.di_sh = d->L * skv; a.di_sb = d->H * a.di_sh;
  a.B = d->B; a.H = d->H; a.S = NT; a.M = ngdn::CH; a.V = d->V;
  a.frag = d->dtype == NGDN_BF16 ? 3 : 0;   // W, KtT, Qg, Aqk: fragment order
  a.j0 = chunk0; a.j1 = chunk0 + nchunk;
  return launched(ngdn::scan_bwd(a, d->dtype, d->K, (hipStream_t)stream), "ngdn_l0_scan_bwd");
}

int32_t ngdn_upper_scan_bwd(const ngdn_dims* d, int32_t level, int32_t n_pairs,
                            int32_t nf, int32_t ng, const float* keys,
                            const float* AT, const float* gam,
                            const float* d_states, const float* inj, int32_t f_here,
                            int32_t f_above, int32_t nf_above, const float* d_final,
                            float* dSp, float* dvn, float* d_initial,
                            void* stream) {
  g_err[0] = 0;
  if (int32_t r = check_dims(d, "ngdn_upper_scan_bwd")) return r;
  if (level < 1 || level >= d->L)
    return fail(NGDN_EINVAL, "ngdn_upper_scan_bwd: level %d outside [1, L=%d)", level, d->L);
  if (!pow2_ge16(n_pairs))
    return fail(NGDN_EINVAL, "ngdn_upper_scan_bwd: pairs per firing must be a power of two >= 16 "
                "(and <= 128), got %d", n_pairs);
  if (!(ng - 1 <= nf && nf <= ng) || nf < 0)
    return fail(NGDN_EINVAL, "ngdn_upper_scan_bwd: NF=%d inconsistent with NG=%d", nf, ng);
  if ((nf > 0 && (!keys || !AT || !gam || !dSp || !dvn)) || !d_states)
    return fail(NGDN_EINVAL, "ngdn_upper_scan_bwd: NULL tensor");
  if (inj && (level + 1 >= d->L || f_here < 1 || f_above < f_here || nf_above < 0 ||
              nf_above > fire_chunks(d) / f_above))
    return fail(NGDN_EINVAL, "ngdn_upper_scan_bwd: injection of level %d with intervals %d / %d "
                "and %d firings inconsistent", level + 1, f_above, f_here, nf_above);
  const long long skv = (long long)d->K * d->V;
  ngdn::ScanBwdArgs a{};
  a.Bop = keys; a.AT = AT; a.gam = gam;
  a.d_states = d_states; a.NG = ng;
  a.inj = inj; a.inj_fh = f_here; a.inj_fa = f_above; a.inj_nf = inj ? nf_above : 0;
  a.d_final = d_final ? d_final + (long long)level * skv : nullptr;
  a.df_sh = d->L * skv; a.df_sb = d->H * a.df_sh;
  a.dSp = dSp; a.dVn = dvn; a.dVnT = nullptr;
  a.dinit = d_initial ? d_initial + (long long)level * skv : nullptr;
  a.di_sh = d->L * skv; a.di_sb = d->H * a.di_sh;
  a.B = d->B; a.H = d->H; a.S = nf; a.M = n_pairs; a.V = d->V;
  a.frag = d->dtype == NGDN_BF16 && n_pairs % 32 == 0;   // AT as the probes write it
  return launched(ngdn::scan_bwd(a, d->dtype, d->K, (hipStream_t)stream), "ngdn_upper_scan_bwd");
}

int32_t ngdn_l0_bwd_state(const ngdn_dims* d, const float* h, const float* dSp,
                          const float* vn, const float* dVn, const void* dout,
                          const void* mix, float* dQg, float* dWT, float* dKt,
                          float* dAqk, float* dgam, void* stream) {
  g_err[0] = 0;
  if (int32_t r = check_dims(d, "ngdn_l0_bwd_state")) return r;
  if (!h || !dSp || !vn || !dVn || !dout || !mix || !dQg || !dWT || !dKt || !dAqk || !dgam)
    return fail(NGDN_EINVAL, "ngdn_l0_bwd_state: NULL tensor");
  ngdn::L0BwdStateArgs a{h, dSp, vn, dVn, dout, mix, dQg, dWT, dKt, dAqk, dgam,
                         d->B, d->T, d->H, d->L, nchunks(d)};
  return launched(ngdn::l0_bwd_state(a, d->dtype, d->K, d->V, (hipStream_t)stream),
                  "ngdn_l0_bwd_state");
}

int32_t ngdn_l0_bwd_intra(const ngdn_dims* d, const void* q, const void* k,
                          const void* v, const float* g, const void* b,
                          const void* w, const float* W, const float* U,
                          const float* TT, const float* dQg, const float* dWT,
                          const float* dKt, const float* dAqk, const float* dgam,
                          const float* dVnT, void* dq, void* dk, void* dv,
                          float* dg, void* db, void* dw, void* stream) {
  g_err[0] = 0;
  if (int32_t r = check_dims(d, "ngdn_l0_bwd_intra")) return r;
  if (!q || !k || !v || !g || !b || !w || !W || !U || !TT || !dQg || !dWT || !dKt || !dAqk ||
      !dgam || !dVnT || !dq || !dk || !dv || !dg || !db || !dw)
    return fail(NGDN_EINVAL, "ngdn_l0_bwd_intra: NULL tensor");
  // the fused form's fields (h .. wsK) stay NULL
  ngdn::L0BwdIntraArgs a{};
  a.q = q; a.k = k; a.v = v; a.g = g; a.b = b; a.w = w; a.W = W; a.U = U; a.TT = TT;
  a.dQg = dQg; a.dWT = dWT; a.dKt = dKt; a.dAqk = dAqk; a.dgam = dgam; a.dVnT = dVnT;
  a.dq = dq; a.dk = dk; a.dv = dv; a.dg = dg; a.db = db; a.dw = dw;
  a.B = d->B; a.T = d->T; a.H = d->H; a.L = d->L; a.NT = nchunks(d); a.scale = d->scale;
  return launched(ngdn::l0_bwd_intra(a, d->dtype, d->K, d->V, (hipStream_t)stream),
                  "ngdn_l0_bwd_intra");
}

int32_t ngdn_l0_bwd(const ngdn_dims* d, const void* q, const void* k, const void* v,
                    const float* g, const void* b, const void* w,
                    const float* TT, const float* h, const float* dSp,
                    const float* vn, const float* dVnT, const void* dout, const void* mix,
                    float* ws_dQg, float* ws_dKt, void* dq, void* dk, void* dv, float* dg,
                    void* db, void* dw, int32_t chunk0, int32_t nchunk, void* stream) {
  g_err[0] = 0;
  if (int32_t r = check_dims(d, "ngdn_l0_bwd")) return r;
  if (int32_t r = check_range(d, chunk0, nchunk, "ngdn_l0_bwd")) return r;
  if (!q || !k || !v || !g || !b || !w || !TT || !h || !dSp || !vn || !dVnT ||
      !dout || !mix || !ws_dQg || !ws_dKt || !dq || !dk || !dv || !dg || !db || !dw)
    return fail(NGDN_EINVAL, "ngdn_l0_bwd: NULL tensor");
  ngdn::L0BwdIntraArgs a{};
  a.q = q; a.k = k; a.v = v; a.g = g; a.b = b; a.w = w; a.TT = TT;
  a.dVnT = dVnT; a.dq = dq; a.dk = dk; a.dv = dv; a.dg = dg; a.db = db; a.dw = dw;
  a.B = d->B; a.T = d->T; a.H = d->H; a.L = d->L; a.NT = nchunks(d); a.scale = d->scale;
  a.h = h; a.dSp = dSp; a.vn = vn; a.dout = dout; a.mix = mix; a.wsQ = ws_dQg; a.wsK = ws_dKt;
  a.n0 = chunk0; a.nn = nchunk;
  return launched(ngdn::l0_bwd_fused(a, d->dtype, d->K, d->V, (hipStream_t)stream),
                  "ngdn_l0_bwd");
}

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
                       float* d_final, void* stream) {
  g_err[0] = 0;
  if (int32_t r = check_dims(d, "ngdn_probe_bwd")) return r;
  if (level < 1 || level >= d->L || d->K != d->V || (promotion != 0 && promotion != 1))
    return fail(NGDN_EINVAL, "ngdn_probe_bwd: bad level %d / promotion %d / K,V", level, promotion);
  const int N = promotion == 1 ? d->K : n_queries;
  if (!pow2_ge16(N))
    return fail(NGDN_EINVAL, "ngdn_probe_bwd: pairs per firing must be a power of two >= 16, got %d", N);
  if (promotion == 0 && (n_queries > n_max || n_max % 8 != 0 || !query_banks || !key_projections ||
                         !kpT || !bankT || !ws_dbank))
    return fail(NGDN_EINVAL, "ngdn_probe_bwd: bank of %d rows (a multiple of 8 >= n_queries=%d) "
                "and its transposes are required", n_max, n_queries);
  if (f_below <= 0 || f_here <= 0) return fail(NGDN_EINVAL, "ngdn_probe_bwd: bad intervals");
  if (!below_kv || !below_vk || !final_state || !bpT || !wpT || !gpT || !bp || !wp || !gp ||
      !states || !statesT || !dSp || !dvn || !ws_vals || !ws_du || !ws_dxb || !ws_dxg ||
      !ws_dxw || !ws_dvals)
    return fail(NGDN_EINVAL, "ngdn_probe_bwd: NULL tensor");
  if (!inj || (level > 1 && !d_final))
    return fail(NGDN_EINVAL, "ngdn_probe_bwd: lower-level gradient destination missing");
  const long long skv = (long long)d->K * d->V;
  ngdn::ProbeBwdArgs a{};
  a.f.below = nullptr; a.f.below_mode = level == 1 ? 0 : 1; a.f.NGb = ng_below;
  a.below_kv = below_kv; a.below_vk = below_vk;
  a.f.below_fin = final_state + (long long)(level - 1) * skv;
  a.f.bf_sh = d->L * skv; a.f.bf_sb = d->H * a.f.bf_sh;
  a.f.f_below = f_below; a.f.f_here = f_here;
  const size_t hkv = (size_t)d->H * skv;
  const size_t esz = d->dtype == NGDN_BF16 ? 2 : 4;
  auto lvl = [&](const void* p, size_t per) -> const void* {
    return p ? static_cast<const char*>(p) + (size_t)(level - 1) * per * esz : nullptr;
  };
  a.f.bank = lvl(query_banks, (size_t)d->H * n_max * d->K); a.f.Nmax = n_max;
  a.f.kp = lvl(key_projections, hkv);
  a.f.bpT = lvl(bpT, hkv); a.f.wpT = lvl(wpT, hkv); a.f.gpT = lvl(gpT, hkv);
  a.f.merge = promotion;
  a.f.B = d->B; a.f.H = d->H; a.f.NF = fire_chunks(d) / f_here; a.f.N = N; a.f.V = d->V;
  a.kpT = lvl(kpT, hkv); a.bankT = lvl(bankT, (size_t)d->H * n_max * d->K);
  a.bp = lvl(bp, hkv); a.wp = lvl(wp, hkv); a.gp = lvl(gp, hkv);
  a.Sg = states; a.SgT = statesT; a.NG = ng;
  a.dSp = dSp; a.dvn = dvn;
  a.wsV = ws_vals; a.wsdu = ws_du; a.wsdxb = ws_dxb; a.wsdxg = ws_dxg; a.wsdxw = ws_dxw;
  a.wsdV = ws_dvals;
  a.dbank = ws_dbank;   // [B,H,NF,N,K], summed by ngdn_param_grads
  a.inj = inj;
  a.d_below_fin = d_final ? d_final + (long long)(level - 1) * skv : nullptr;
  if (a.f.NF == 0) return NGDN_OK;
  return launched(ngdn::probe_bwd(a, d->dtype, d->K, (hipStream_t)stream), "ngdn_probe_bwd");
}

int32_t ngdn_param_grads(const ngdn_dims* d, int32_t level, int32_t promotion,
                         int32_t n_pairs, int32_t nf, const float* ws_vals,
                         const float* ws_du, const float* ws_dxb,
                         const float* ws_dxg, const float* ws_dxw,
                         const float* ws_dbank, int32_t n_max, float* dbank, float* dkp,
                         float* dbp, float* dwp, float* dgp, float* ws_parts, void* stream) {
  g_err[0] = 0;
  if (int32_t r = check_dims(d, "ngdn_param_grads")) return r;
  if (level < 1 || level >= d->L || d->K != d->V)
    return fail(NGDN_EINVAL, "ngdn_param_grads: bad level %d or K != V", level);
  if (!ws_vals || !ws_dxb || !ws_dxg || !ws_dxw || !dbp || !dwp || !dgp || !ws_parts ||
      (promotion == 0 && (!ws_du || !dkp || !ws_dbank || !dbank)))
    return fail(NGDN_EINVAL, "ngdn_param_grads: NULL tensor");
  if (promotion == 0 && (n_max < n_pairs || n_max % 8 != 0))
    return fail(NGDN_EINVAL, "ngdn_param_grads: bank rows %d (a multiple of 8 >= %d)", n_max,
                n_pairs);
  if (nf <= 0) return NGDN_OK;
  const int H = d->H, K = d->K, V = d->V;
  const size_t off = (size_t)(level - 1) * H * K * V;
  // firings split over up to NGDN_PARAM_SPLIT workgroups per head and
  // product, at least 4 firings each; each writes its partial
  const int split = std::max(1, std::min(NGDN_PARAM_SPLIT, (d->B * nf + 3) / 4));
  hipStream_t st = (hipStream_t)stream;
  ngdn::AtBArgs a{};
  a.parts = ws_parts;
  a.B = d->B; a.H = H; a.NF = nf; a.N = n_pairs; a.X = K; a.Y = V; a.split = split;
  // the (up to) four sums in one launch
  auto add = [&](const float* A, const float* Bm, float* C) {
    a.A[a.nprod] = A; a.Bm[a.nprod] = Bm; a.C[a.nprod] = C; ++a.nprod;
  };
  if (promotion == 0) add(ws_du, ws_vals, dkp + off);    // dWk = du^T Vals
  add(ws_vals, ws_dxb, dbp + off);                       // dBp = Vals^T dxb
  add(ws_vals, ws_dxw, dwp + off);                       // dWp = Vals^T dxw
  add(ws_vals, ws_dxg, dgp + off);                       // dGp = Vals^T dxg
  if (int32_t r = launched(ngdn::atb_accumulate(a, d->dtype, st), "ngdn_param_grads")) return r;
  // the slices added in order, and the bank gradient's per-firing partials
  // in (batch row, firing) order
  ngdn::OrderedSumArgs o{};
  o.ng = H;
  const long long kv = (long long)K * V;
  for (int p = 0; p < a.nprod; ++p) {
    o.parts[o.nsum] = ws_parts + (long long)p * H * split * kv;   // as atb writes them
    o.out[o.nsum] = a.C[p];
    o.pg[o.nsum] = (long long)split * kv; o.og[o.nsum] = kv;
    o.s1[o.nsum] = kv; o.n1[o.nsum] = split; o.s2[o.nsum] = 0; o.n2[o.nsum] = 1;
    o.n[o.nsum] = kv;
    ++o.nsum;
  }
  if (promotion == 0) {
    const long long nk = (long long)n_pairs * K;
    o.parts[o.nsum] = ws_dbank;
    o.out[o.nsum] = dbank + (size_t)(level - 1) * H * n_max * K;
    o.pg[o.nsum] = (long long)nf * nk; o.og[o.nsum] = (long long)n_max * K;
    o.s1[o.nsum] = (long long)H * nf * nk; o.n1[o.nsum] = d->B;
    o.s2[o.nsum] = nk; o.n2[o.nsum] = nf;
    o.n[o.nsum] = nk;
    ++o.nsum;
  }
  return launched(ngdn::ordered_sum(o, st), "ngdn_param_grads (sums)");
}

}  // extern "C"

namespace {

// Scratch of ngdn_step_noalloc: the per-level pairs (A, KT, U, gam) of the
// promotions whose levels take more than PROMOTE_NMAX pairs per firing. Each
// GPU holds its own copy for the life of the process; host code uses only the
// per-device address from hipGetSymbolAddress, never the array's name.
static __device__ __align__(256) float scratch[NGDN_STEP_SCRATCH_BYTES / sizeof(float)];
constexpr long long kScratchFloats = NGDN_STEP_SCRATCH_BYTES / sizeof(float);
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch[kMaxDevices];

// The current device's address of `scratch`, looked up once per device.
int32_t scratch_of_current_device(float** out, const char* what) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(NGDN_ELAUNCH, "%s: hipGetDevice: %s", what, hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(NGDN_EINVAL, "%s: device %d out of range", what, dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(NGDN_ELAUNCH, "%s: hipGetSymbolAddress(scratch) on device %d: %s", what, dev,
                  hipGetErrorString(e));
    g_scratch[dev] = static_cast<float*>(p);
  }
  *out = g_scratch[dev];
  return NGDN_OK;
}

// Pairs per firing of level l (K for merge).
inline int step_pairs(int promotion, const int32_t* n_queries, int K, int l) {
  return promotion == 1 ? K : n_queries[l - 1];
}

// The body of ngdn_step and ngdn_step_noalloc. Levels with more than
// PROMOTE_NMAX pairs per firing go through ws, rows_per_slice batch rows at a
// time (probe, then one firing of the update, per slice); ws must hold
// rows_per_slice * H * (3 N K + K) floats, N the most pairs of any level.
int32_t step_run(const ngdn_dims* d, const void* q, const void* k, const void* v,
                 const float* g, const void* b, const void* w, const void* mix,
                 const float* state_in, float* state_out, const int64_t* position,
                 int64_t position_all, int32_t chunk_size, const int32_t* firing_intervals,
                 int32_t promotion, const int32_t* n_queries, const void* query_banks,
                 int32_t n_max, const void* key_projections, const void* bpT, const void* wpT,
                 const void* gpT, float* ws, int rows_per_slice, void* o, void* stream,
                 const char* what) {
  const int L = d->L, K = d->K, V = d->V;
  const long long skv = (long long)K * V;
  hipStream_t st = (hipStream_t)stream;
  ngdn::StepArgs sa{q, k, v, g, b, w, mix, state_in, state_out, o, d->B, d->H, L, d->scale};
  if (int32_t r = launched(ngdn::step_fwd(sa, d->dtype, K, V, st), what)) return r;

  const size_t hkv = (size_t)d->H * skv;
  const size_t esz = d->dtype == NGDN_BF16 ? 2 : 4;
  if (L == 1) return NGDN_OK;
  // Every level with at most 64 pairs per firing: all promotions in one
  // gated launch. With an int position the host skips it when no level fires.
  bool fused = L <= ngdn::MAXL;
  for (int l = 1; l < L; ++l)
    if (step_pairs(promotion, n_queries, K, l) > ngdn::PROMOTE_NMAX) fused = false;
  if (fused) {
    if (!position) {
      const long long end = (long long)position_all + 1;
      bool any = false;
      for (int l = 1; l < L; ++l)
        any = any || (end % chunk_size == 0 && (end / chunk_size) % firing_intervals[l] == 0);
      if (!any) return NGDN_OK;
    }
    ngdn::PromoteArgs pa{};
    pa.state = state_out;
    pa.pos = reinterpret_cast<const long long*>(position);
    pa.pos_all = position_all;
    pa.chunk = chunk_size;
    for (int l = 0; l < L; ++l) {
      pa.f[l] = firing_intervals[l];
      pa.N[l] = l == 0 ? 0 : step_pairs(promotion, n_queries, K, l);
    }
    pa.bank = query_banks; pa.Nmax = n_max;
    pa.kp = key_projections; pa.bpT = bpT; pa.wpT = wpT; pa.gpT = gpT;
    pa.merge = promotion;
    pa.B = d->B; pa.H = d->H; pa.L = L;
    return launched(ngdn::promote_fwd(pa, d->dtype, K, st), what);
  }
  const long long row = (long long)d->H * L * skv;    // one batch row of the state
  for (int l = 1; l < L; ++l) {
    if (!position) {
      const long long end = (long long)position_all + 1;
      if (end % chunk_size != 0 || (end / chunk_size) % firing_intervals[l] != 0) continue;
    }
    const int N = step_pairs(promotion, n_queries, K, l);
    auto lvl = [&](const void* p, size_t per) -> const void* {
      return p ? static_cast<const char*>(p) + (size_t)(l - 1) * per * esz : nullptr;
    };
    for (int b0 = 0; b0 < d->B; b0 += rows_per_slice) {
      const int nb = std::min(rows_per_slice, d->B - b0);
      const size_t units = (size_t)nb * d->H;
      float* A = ws;
      float* KT = A + units * N * K;
      float* U = KT + units * K * N;
      float* gam = U + units * N * V;
      float* srow = state_out + (long long)b0 * row;
      ngdn::FireGate gate{position ? reinterpret_cast<const long long*>(position) + b0 : nullptr,
                          chunk_size, firing_intervals[l]};
      // probe of the level below (already updated this token), read as a
      // "final state": one firing, source index past every stored group
      ngdn::ProbeArgs pa{};
      pa.below_fin = srow + (long long)(l - 1) * skv;
      pa.below = pa.below_fin; pa.below_mode = 1; pa.NGb = 0;
      pa.bf_sh = L * skv; pa.bf_sb = d->H * pa.bf_sh;
      pa.f_below = firing_intervals[l - 1]; pa.f_here = firing_intervals[l];
      pa.bank = lvl(query_banks, (size_t)d->H * n_max * K); pa.Nmax = n_max;
      pa.kp = lvl(key_projections, hkv);
      pa.bpT = lvl(bpT, hkv); pa.wpT = lvl(wpT, hkv); pa.gpT = lvl(gpT, hkv);
      pa.merge = promotion;
      pa.A = A; pa.KT = KT; pa.U = U; pa.gam = gam;
      pa.B = nb; pa.H = d->H; pa.NF = 1; pa.N = N; pa.V = V;
      pa.gate = gate;
      if (int32_t r = launched(ngdn::probe_fwd(pa, d->dtype, K, st), what)) return r;
      // one firing of this level's update, in place on state_out
      ngdn::ScanArgs ca{};
      ca.A = A; ca.BT = KT; ca.U = U; ca.gam = gam;
      ca.init = srow + (long long)l * skv; ca.init_sh = L * skv; ca.init_sb = d->H * ca.init_sh;
      ca.state_mode = 0; ca.NG = 1;
      ca.fin = srow + (long long)l * skv; ca.fin_sh = ca.init_sh; ca.fin_sb = ca.init_sb;
      ca.B = nb; ca.H = d->H; ca.S = 1; ca.M = N; ca.V = V;
      ca.frag = d->dtype == NGDN_BF16 && N % 32 == 0;   // KT as probe_fwd wrote it
      ca.gate = gate;
      if (int32_t r = launched(ngdn::scan_fwd(ca, d->dtype, K, st), what)) return r;
    }
  }
  return NGDN_OK;
}

// Checks shared by ngdn_step and ngdn_step_noalloc (not the workspace).
int32_t step_check(const ngdn_dims* d, const void* q, const void* k, const void* v,
                   const float* g, const void* b, const void* w, const void* mix,
                   const float* state_in, float* state_out, const int64_t* position,
                   int64_t position_all, int32_t chunk_size, const int32_t* firing_intervals,
                   int32_t promotion, const int32_t* n_queries, const void* query_banks,
                   int32_t n_max, const void* key_projections, const void* bpT, const void* wpT,
                   const void* gpT, void* o, const char* what) {
  if (int32_t r = check_dims(d, what)) return r;
  if (!q || !k || !v || !g || !b || !w || !mix || !state_in || !state_out || !o)
    return fail(NGDN_EINVAL, "%s: NULL tensor", what);
  if (chunk_size <= 0) return fail(NGDN_EINVAL, "%s: chunk_size %d", what, chunk_size);
  if (!position && position_all < 0)
    return fail(NGDN_EINVAL, "%s: position %lld is negative", what, (long long)position_all);
  const int L = d->L, K = d->K, V = d->V;
  const long long skv = (long long)K * V;
  const long long nst = (long long)d->B * d->H * L * skv;
  if (state_in != state_out && state_out < state_in + nst && state_in < state_out + nst)
    return fail(NGDN_EINVAL, "%s: state_in and state_out overlap", what);
  if (L > 1) {
    if (K != V) return fail(NGDN_EINVAL, "%s: promotion needs K == V, got %d, %d", what, K, V);
    if (promotion != 0 && promotion != 1)
      return fail(NGDN_EINVAL, "%s: promotion %d unknown", what, promotion);
    if (!firing_intervals || (promotion == 0 && !n_queries) || !bpT || !wpT || !gpT)
      return fail(NGDN_EINVAL, "%s: NULL parameter", what);
    for (int l = 0; l < L; ++l)
      if (firing_intervals[l] <= 0)
        return fail(NGDN_EINVAL, "%s: firing interval %d of level %d", what, firing_intervals[l], l);
    for (int l = 1; l < L; ++l) {
      const int N = step_pairs(promotion, n_queries, K, l);
      if (!pow2_ge16(N))
        return fail(NGDN_EINVAL, "%s: pairs per firing must be a power of two >= 16 "
                    "(and <= 128), got %d", what, N);
      if (promotion == 0 && (N > n_max || !query_banks || !key_projections))
        return fail(NGDN_EINVAL, "%s: n_queries=%d exceeds bank rows %d", what, N, n_max);
    }
  }
  return NGDN_OK;
}

}  // namespace

extern "C" {

int32_t ngdn_step(const ngdn_dims* d, const void* q, const void* k, const void* v,
                  const float* g, const void* b, const void* w, const void* mix,
                  const float* state_in, float* state_out, const int64_t* position,
                  int64_t position_all, int32_t chunk_size,
                  const int32_t* firing_intervals, int32_t promotion,
                  const int32_t* n_queries, const void* query_banks, int32_t n_max,
                  const void* key_projections, const void* bpT, const void* wpT,
                  const void* gpT, float* ws, void* o, void* stream) {
  g_err[0] = 0;
  if (int32_t r = step_check(d, q, k, v, g, b, w, mix, state_in, state_out, position,
                             position_all, chunk_size, firing_intervals, promotion, n_queries,
                             query_banks, n_max, key_projections, bpT, wpT, gpT, o, "ngdn_step"))
    return r;
  if (d->L > 1 && !ws) return fail(NGDN_EINVAL, "ngdn_step: NULL parameter");
  return step_run(d, q, k, v, g, b, w, mix, state_in, state_out, position, position_all,
                  chunk_size, firing_intervals, promotion, n_queries, query_banks, n_max,
                  key_projections, bpT, wpT, gpT, ws, d->B, o, stream, "ngdn_step");
}

int32_t ngdn_step_noalloc(const ngdn_dims* d, const void* q, const void* k, const void* v,
                          const float* g, const void* b, const void* w, const void* mix,
                          const float* state_in, float* state_out, const int64_t* position,
                          int64_t position_all, int32_t chunk_size,
                          const int32_t* firing_intervals, int32_t promotion,
                          const int32_t* n_queries, const void* query_banks, int32_t n_max,
                          const void* key_projections, const void* bpT, const void* wpT,
                          const void* gpT, void* o, void* stream) {
  g_err[0] = 0;
  const char* what = "ngdn_step_noalloc";
  if (int32_t r = step_check(d, q, k, v, g, b, w, mix, state_in, state_out, position,
                             position_all, chunk_size, firing_intervals, promotion, n_queries,
                             query_banks, n_max, key_projections, bpT, wpT, gpT, o, what))
    return r;
  // the most pairs of any level decides the scratch taken per (row, head)
  int nmax_pairs = 0;
  for (int l = 1; l < d->L; ++l)
    nmax_pairs = std::max(nmax_pairs, step_pairs(promotion, n_queries, d->K, l));
  float* ws = nullptr;
  int rows = d->B;
  if (nmax_pairs > ngdn::PROMOTE_NMAX) {
    const long long per_row = (long long)d->H * (3LL * nmax_pairs * d->K + d->K);
    if (per_row > kScratchFloats)
      return fail(NGDN_EINVAL, "%s: one batch row needs %lld bytes of scratch (H=%d, %d pairs, "
                  "K=%d); the scratch holds %lld bytes", what, per_row * 4, d->H, nmax_pairs,
                  d->K, (long long)NGDN_STEP_SCRATCH_BYTES);
    rows = (int)std::min<long long>(d->B, kScratchFloats / per_row);
    if (int32_t r = scratch_of_current_device(&ws, what)) return r;
  }
  return step_run(d, q, k, v, g, b, w, mix, state_in, state_out, position, position_all,
                  chunk_size, firing_intervals, promotion, n_queries, query_banks, n_max,
                  key_projections, bpT, wpT, gpT, ws, rows, o, stream, what);
}

int32_t ngdn_short_conv_fwd(int32_t dtype, int32_t B, int32_t T, int32_t D, int32_t W,
                            int32_t act, const void* x, const float* w, const void* cache_in,
                            void* y, void* cache_out, void* stream) {
  g_err[0] = 0;
  if (dtype != NGDN_F32 && dtype != NGDN_BF16) return fail(NGDN_EINVAL, "ngdn_short_conv_fwd: dtype %d", dtype);
  if (B < 0 || T < 0 || D <= 0 || D % 8 != 0 || W < 1 || W > 8)
    return fail(NGDN_EINVAL, "ngdn_short_conv_fwd: B=%d T=%d D=%d W=%d (D a multiple of 8, 1 <= W <= 8)", B, T, D, W);
  if ((B * T > 0 && (!x || !y)) || !w) return fail(NGDN_EINVAL, "ngdn_short_conv_fwd: NULL tensor");
  ngdn::ShortConvArgs a{};
  a.x = x; a.w = w; a.cache_in = cache_in; a.y = y; a.cache_out = cache_out;
  a.B = B; a.T = T; a.D = D; a.W = W; a.act = act != 0;
  return launched(ngdn::short_conv_fwd(a, dtype, (hipStream_t)stream), "ngdn_short_conv_fwd");
}

int32_t ngdn_short_conv_bwd(int32_t dtype, int32_t B, int32_t T, int32_t D, int32_t W,
                            int32_t act, const void* x, const float* w, const void* cache_in,
                            const void* dy, void* dx, float* dw, float* ws, void* stream) {
  g_err[0] = 0;
  if (dtype != NGDN_F32 && dtype != NGDN_BF16) return fail(NGDN_EINVAL, "ngdn_short_conv_bwd: dtype %d", dtype);
  if (B < 0 || T < 0 || D <= 0 || D % 8 != 0 || W < 1 || W > 8)
    return fail(NGDN_EINVAL, "ngdn_short_conv_bwd: B=%d T=%d D=%d W=%d (D a multiple of 8, 1 <= W <= 8)", B, T, D, W);
  if ((B * T > 0 && (!x || !dy || !dx)) || !w || !dw) return fail(NGDN_EINVAL, "ngdn_short_conv_bwd: NULL tensor");
  ngdn::ShortConvArgs a{};
  a.x = x; a.w = w; a.cache_in = cache_in; a.dy = dy; a.dx = dx; a.dw = dw; a.ws = ws;
  a.B = B; a.T = T; a.D = D; a.W = W; a.act = act != 0;
  return launched(ngdn::short_conv_bwd(a, dtype, (hipStream_t)stream), "ngdn_short_conv_bwd");
}

int32_t ngdn_rmsnorm_gated_fwd(int32_t dtype, int64_t rows, int32_t V, float eps,
                               const void* x, const void* g, const float* w, void* y,
                               float* rstd, void* stream) {
  g_err[0] = 0;
  if (dtype != NGDN_F32 && dtype != NGDN_BF16) return fail(NGDN_EINVAL, "ngdn_rmsnorm_gated_fwd: dtype %d", dtype);
  if (rows < 0 || (V != 64 && V != 128 && V != 256))
    return fail(NGDN_EINVAL, "ngdn_rmsnorm_gated_fwd: rows=%lld V=%d (V in 64, 128, 256)", (long long)rows, V);
  if (rows > 0 && (!x || !g || !w || !y)) return fail(NGDN_EINVAL, "ngdn_rmsnorm_gated_fwd: NULL tensor");
  ngdn::NormGatedArgs a{};
  a.x = x; a.g = g; a.w = w; a.y = y; a.rstd = rstd; a.rows = rows; a.eps = eps;
  return launched(ngdn::rmsnorm_gated_fwd(a, dtype, V, (hipStream_t)stream), "ngdn_rmsnorm_gated_fwd");
}

int32_t ngdn_rmsnorm_gated_bwd(int32_t dtype, int64_t rows, int32_t V, const void* x,
                               const void* g, const float* w, const float* rstd,
                               const void* dy, void* dx, void* dg, float* dw, float* ws,
                               void* stream) {
  g_err[0] = 0;
  if (dtype != NGDN_F32 && dtype != NGDN_BF16) return fail(NGDN_EINVAL, "ngdn_rmsnorm_gated_bwd: dtype %d", dtype);
  if (rows < 0 || (V != 64 && V != 128 && V != 256))
    return fail(NGDN_EINVAL, "ngdn_rmsnorm_gated_bwd: rows=%lld V=%d (V in 64, 128, 256)", (long long)rows, V);
  if (rows > 0 && (!x || !g || !w || !rstd || !dy || !dx || !dg || !dw))
    return fail(NGDN_EINVAL, "ngdn_rmsnorm_gated_bwd: NULL tensor");
  ngdn::NormGatedArgs a{};
  a.x = x; a.g = g; a.w = w; a.rstd = const_cast<float*>(rstd); a.dy = dy; a.dx = dx; a.dg = dg;
  a.dw = dw; a.ws = ws; a.rows = rows;
  return launched(ngdn::rmsnorm_gated_bwd(a, dtype, V, (hipStream_t)stream), "ngdn_rmsnorm_gated_bwd");
}

static int32_t gate_args(int32_t dtype, const ngdn_gate_args* g, ngdn::GatePrepArgs& a, const char* who) {
  if (dtype != NGDN_F32 && dtype != NGDN_BF16) return fail(NGDN_EINVAL, "%s: dtype %d", who, dtype);
  if (!g) return fail(NGDN_EINVAL, "%s: NULL arguments", who);
  if (g->BT < 0 || g->H <= 0 || g->L < 1 || g->L > 8 || (g->K != 64 && g->K != 128) ||
      (g->V != 64 && g->V != 128) || (g->param_dtype != NGDN_F32 && g->param_dtype != NGDN_BF16))
    return fail(NGDN_EINVAL, "%s: BT=%lld H=%d L=%d K=%d V=%d param_dtype=%d (K, V in 64, 128; 1 <= L <= 8)",
                who, (long long)g->BT, g->H, g->L, g->K, g->V, g->param_dtype);
  a = ngdn::GatePrepArgs{};
  a.q = g->q; a.k = g->k; a.f = g->f; a.bz = g->bz; a.wz = g->wz; a.ml = g->ml;
  a.A_log = g->A_log; a.dt_bias = g->dt_bias;
  a.qn = g->qn; a.kn = g->kn; a.g0 = g->g0; a.b0 = g->b0; a.w0 = g->w0; a.mix = g->mix;
  a.dqn = g->dqn; a.dkn = g->dkn; a.dg0 = g->dg0; a.db0 = g->db0; a.dw0 = g->dw0; a.dmix = g->dmix;
  a.dq = g->dq; a.dk = g->dk; a.df = g->df; a.dbz = g->dbz; a.dwz = g->dwz; a.dml = g->dml;
  a.dpar = g->dpar; a.ws = g->ws;
  a.BT = g->BT; a.H = g->H; a.L = g->L; a.K = g->K; a.V = g->V;
  a.pdtype = g->param_dtype; a.sigmoid_mix = g->sigmoid_mix != 0; a.cap = g->cap;
  return 0;
}

int32_t ngdn_gate_prep_fwd(int32_t dtype, const ngdn_gate_args* g, void* stream) {
  g_err[0] = 0;
  ngdn::GatePrepArgs a;
  if (int32_t r = gate_args(dtype, g, a, "ngdn_gate_prep_fwd")) return r;
  if (a.BT > 0 && (!a.q || !a.k || !a.f || !a.bz || !a.wz || !a.ml || !a.A_log || !a.dt_bias ||
                   !a.qn || !a.kn || !a.g0 || !a.b0 || !a.w0 || !a.mix))
    return fail(NGDN_EINVAL, "ngdn_gate_prep_fwd: NULL tensor");
  return launched(ngdn::gate_prep_fwd(a, dtype, (hipStream_t)stream), "ngdn_gate_prep_fwd");
}

int32_t ngdn_gate_prep_bwd(int32_t dtype, const ngdn_gate_args* g, void* stream) {
  g_err[0] = 0;
  ngdn::GatePrepArgs a;
  if (int32_t r = gate_args(dtype, g, a, "ngdn_gate_prep_bwd")) return r;
  if (a.BT > 0 && (!a.q || !a.k || !a.f || !a.bz || !a.wz || !a.ml || !a.A_log || !a.dt_bias ||
                   !a.dqn || !a.dkn || !a.dg0 || !a.db0 || !a.dw0 || !a.dmix || !a.dq || !a.dk ||
                   !a.df || !a.dbz || !a.dwz || !a.dml || !a.dpar))
    return fail(NGDN_EINVAL, "ngdn_gate_prep_bwd: NULL tensor");
  return launched(ngdn::gate_prep_bwd(a, dtype, (hipStream_t)stream), "ngdn_gate_prep_bwd");
}

int32_t ngdn_rmsnorm_fwd(int32_t dtype, int64_t rows, int32_t D, float eps, const void* x,
                         const float* w, void* y, float* rstd, void* stream) {
  g_err[0] = 0;
  if (dtype != NGDN_F32 && dtype != NGDN_BF16) return fail(NGDN_EINVAL, "ngdn_rmsnorm_fwd: dtype %d", dtype);
  if (rows < 0 || !ngdn::rmsnorm_supported(D))
    return fail(NGDN_EINVAL, "ngdn_rmsnorm_fwd: rows=%lld D=%d (D = 512 n for n in 1..6, or 64, 128, 256, 768)",
                (long long)rows, D);
  if (rows > 0 && (!x || !w || !y)) return fail(NGDN_EINVAL, "ngdn_rmsnorm_fwd: NULL tensor");
  ngdn::RMSNormArgs a{};
  a.x = x; a.w = w; a.y = y; a.rstd = rstd; a.rows = rows; a.D = D; a.eps = eps;
  return launched(ngdn::rmsnorm_fwd(a, dtype, dtype, dtype, (hipStream_t)stream), "ngdn_rmsnorm_fwd");
}

int32_t ngdn_rmsnorm_bwd(int32_t dtype, int64_t rows, int32_t D, const void* x, const float* w,
                         const float* rstd, const void* dy, void* dx, float* dw, float* ws,
                         void* stream) {
  g_err[0] = 0;
  if (dtype != NGDN_F32 && dtype != NGDN_BF16) return fail(NGDN_EINVAL, "ngdn_rmsnorm_bwd: dtype %d", dtype);
  if (rows < 0 || !ngdn::rmsnorm_supported(D))
    return fail(NGDN_EINVAL, "ngdn_rmsnorm_bwd: rows=%lld D=%d unsupported", (long long)rows, D);
  if (rows > 0 && (!x || !w || !rstd || !dy || !dx || !dw)) return fail(NGDN_EINVAL, "ngdn_rmsnorm_bwd: NULL tensor");
  ngdn::RMSNormArgs a{};
  a.x = x; a.w = w; a.rstd = const_cast<float*>(rstd); a.dy = dy; a.dx = dx; a.dw = dw;
  a.ws = ws; a.rows = rows; a.D = D;
  return launched(ngdn::rmsnorm_bwd(a, dtype, dtype, dtype, (hipStream_t)stream), "ngdn_rmsnorm_bwd");
}

int32_t ngdn_add_rmsnorm_fwd(int32_t x_dtype, int32_t r_dtype, int32_t y_dtype, int64_t rows,
                             int32_t D, float eps, const void* x, const void* r, const float* w,
                             void* h, void* y, float* rstd, void* stream) {
  g_err[0] = 0;
  if (!ngdn::rmsnorm_types_supported(x_dtype, r_dtype, y_dtype))
    return fail(NGDN_EINVAL, "ngdn_add_rmsnorm_fwd: dtypes x=%d r=%d y=%d (all fp32, all bf16, or "
                "fp32 x with bf16 r and y)", x_dtype, r_dtype, y_dtype);
  if (rows < 0 || !ngdn::rmsnorm_supported(D))
    return fail(NGDN_EINVAL, "ngdn_add_rmsnorm_fwd: rows=%lld D=%d unsupported", (long long)rows, D);
  if (rows > 0 && (!x || !w || !y || (r && !h)))
    return fail(NGDN_EINVAL, "ngdn_add_rmsnorm_fwd: NULL tensor");
  ngdn::RMSNormArgs a{};
  a.x = x; a.r = r; a.h = r ? h : nullptr; a.w = w; a.y = y; a.rstd = rstd;
  a.rows = rows; a.D = D; a.eps = eps;
  return launched(ngdn::rmsnorm_fwd(a, x_dtype, r_dtype, y_dtype, (hipStream_t)stream),
                  "ngdn_add_rmsnorm_fwd");
}

int32_t ngdn_add_rmsnorm_bwd(int32_t x_dtype, int32_t r_dtype, int32_t y_dtype, int64_t rows,
                             int32_t D, const void* h, const float* w, const float* rstd,
                             const void* dy, const void* dh, void* dx, void* dr, float* dw,
                             float* ws, void* stream) {
  g_err[0] = 0;
  if (!ngdn::rmsnorm_types_supported(x_dtype, r_dtype, y_dtype))
    return fail(NGDN_EINVAL, "ngdn_add_rmsnorm_bwd: dtypes x=%d r=%d y=%d (all fp32, all bf16, or "
                "fp32 x with bf16 r and y)", x_dtype, r_dtype, y_dtype);
  if (rows < 0 || !ngdn::rmsnorm_supported(D))
    return fail(NGDN_EINVAL, "ngdn_add_rmsnorm_bwd: rows=%lld D=%d unsupported", (long long)rows, D);
  if (rows > 0 && (!h || !w || !rstd || !dy || !dx || !dw))
    return fail(NGDN_EINVAL, "ngdn_add_rmsnorm_bwd: NULL tensor");
  ngdn::RMSNormArgs a{};
  a.x = h; a.w = w; a.rstd = const_cast<float*>(rstd); a.dy = dy; a.dh = dh; a.dx = dx; a.dr = dr;
  a.dw = dw; a.ws = ws; a.rows = rows; a.D = D;
  return launched(ngdn::rmsnorm_bwd(a, x_dtype, r_dtype, y_dtype, (hipStream_t)stream),
                  "ngdn_add_rmsnorm_bwd");
}

int32_t ngdn_swiglu_fwd(int32_t dtype, int64_t n, const void* g, const void* u, void* y, void* stream) {
  g_err[0] = 0;
  if (dtype != NGDN_F32 && dtype != NGDN_BF16) return fail(NGDN_EINVAL, "ngdn_swiglu_fwd: dtype %d", dtype);
  if (n < 0 || n % 8 != 0) return fail(NGDN_EINVAL, "ngdn_swiglu_fwd: n=%lld (a multiple of 8)", (long long)n);
  if (n > 0 && (!g || !u || !y)) return fail(NGDN_EINVAL, "ngdn_swiglu_fwd: NULL tensor");
  ngdn::SwigluArgs a{};
  a.g = g; a.u = u; a.y = y; a.n = n;
  return launched(ngdn::swiglu_fwd(a, dtype, (hipStream_t)stream), "ngdn_swiglu_fwd");
}

int32_t ngdn_swiglu_bwd(int32_t dtype, int64_t n, const void* g, const void* u, const void* dy,
                        void* dg, void* du, void* stream) {
  g_err[0] = 0;
  if (dtype != NGDN_F32 && dtype != NGDN_BF16) return fail(NGDN_EINVAL, "ngdn_swiglu_bwd: dtype %d", dtype);
  if (n < 0 || n % 8 != 0) return fail(NGDN_EINVAL, "ngdn_swiglu_bwd: n=%lld (a multiple of 8)", (long long)n);
  if (n > 0 && (!g || !u || !dy || !dg || !du)) return fail(NGDN_EINVAL, "ngdn_swiglu_bwd: NULL tensor");
  ngdn::SwigluArgs a{};
  a.g = g; a.u = u; a.dy = dy; a.dg = dg; a.du = du; a.n = n;
  return launched(ngdn::swiglu_bwd(a, dtype, (hipStream_t)stream), "ngdn_swiglu_bwd");
}

int32_t ngdn_sum_f32(int32_t dtype, int32_t count, const void* const* xs, int64_t n, float* out,
                     void* stream) {
  g_err[0] = 0;
  if (dtype != NGDN_F32 && dtype != NGDN_BF16) return fail(NGDN_EINVAL, "ngdn_sum_f32: dtype %d", dtype);
  if (count < 1 || count > ngdn::SUM_MAX || n < 0 || n % 8 != 0)
    return fail(NGDN_EINVAL, "ngdn_sum_f32: count=%d n=%lld (1 <= count <= 8, n a multiple of 8)",
                count, (long long)n);
  if (n > 0 && (!xs || !out)) return fail(NGDN_EINVAL, "ngdn_sum_f32: NULL tensor");
  ngdn::SumArgs a{};
  for (int j = 0; j < count; ++j) {
    if (n > 0 && !xs[j]) return fail(NGDN_EINVAL, "ngdn_sum_f32: NULL input %d", j);
    a.x[j] = xs[j];
  }
  a.out = out; a.n = n; a.count = count;
  return launched(ngdn::sum_into_f32(a, dtype, (hipStream_t)stream), "ngdn_sum_f32");
}

int32_t ngdn_cross_entropy(int32_t dtype, int64_t rows, int32_t V, int32_t ignore_index,
                           void* logits, const int64_t* labels, const int64_t* n_valid,
                           float* row_loss, int32_t grad, void* stream) {
  g_err[0] = 0;
  if (dtype != NGDN_F32 && dtype != NGDN_BF16) return fail(NGDN_EINVAL, "ngdn_cross_entropy: dtype %d", dtype);
  if (rows < 0 || !ngdn::xent_supported(V))
    return fail(NGDN_EINVAL, "ngdn_cross_entropy: rows=%lld V=%d (V a multiple of 8, at most 65536)",
                (long long)rows, V);
  if (rows > 0 && (!logits || !labels || !n_valid || !row_loss))
    return fail(NGDN_EINVAL, "ngdn_cross_entropy: NULL tensor");
  ngdn::XentArgs a{};
  a.logits = logits; a.labels = reinterpret_cast<const long long*>(labels);
  a.n_valid = reinterpret_cast<const long long*>(n_valid); a.row_loss = row_loss;
  a.rows = rows; a.V = V; a.ignore_index = ignore_index; a.grad = grad != 0;
  return launched(ngdn::cross_entropy(a, dtype, (hipStream_t)stream), "ngdn_cross_entropy");
}

}  // extern "C"
