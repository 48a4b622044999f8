// extern "C" entry points of libngdn.so: argument checks, then launches.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

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
  return NGDN_OK;
}

inline int nchunks(const ngdn_dims* d) { return (d->T + ngdn::CH - 1) / ngdn::CH; }

}  // namespace

extern "C" {

const char* ngdn_last_error(void) { return g_err; }
int32_t ngdn_version(void) { return 100; }
const char* ngdn_arch(void) { return "gfx950"; }

int32_t ngdn_l0_intra_fwd(const ngdn_dims* d, const void* q, const void* k,
                          const void* v, const float* g, const void* b,
                          const void* w, void* W, void* U, void* KtT, void* Qg,
                          void* Aqk, float* gam, void* stream) {
  g_err[0] = 0;
  if (int32_t r = check_dims(d, "ngdn_l0_intra_fwd")) return r;
  if (!q || !k || !v || !g || !b || !w || !W || !U || !KtT || !Qg || !Aqk || !gam)
    return fail(NGDN_EINVAL, "ngdn_l0_intra_fwd: NULL tensor");
  ngdn::L0IntraArgs a{q, k, v, g, b, w, W, U, KtT, Qg, Aqk, gam,
                      d->B, d->T, d->H, d->L, nchunks(d), d->scale};
  return launched(ngdn::l0_intra_fwd(a, d->dtype, d->K, d->V, (hipStream_t)stream),
                  "ngdn_l0_intra_fwd");
}

int32_t ngdn_l0_scan_fwd(const ngdn_dims* d, const void* W, const void* U,
                         const void* KtT, const float* gam,
                         const float* initial_state, void* hT, void* vnT,
                         float* final_state, void* stream) {
  g_err[0] = 0;
  if (int32_t r = check_dims(d, "ngdn_l0_scan_fwd")) return r;
  if (!W || !U || !KtT || !gam || !hT || !final_state)
    return fail(NGDN_EINVAL, "ngdn_l0_scan_fwd: NULL tensor");
  const long long skv = (long long)d->K * d->V;
  ngdn::ScanArgs a{};
  a.A = W; a.BT = KtT; a.U = U; a.gam = gam;
  a.init = initial_state; a.init_sh = d->L * skv; a.init_sb = d->H * a.init_sh;
  a.states = hT; a.state_mode = 0; a.NG = nchunks(d);
  a.vnT = vnT;
  a.fin = final_state; a.fin_sh = d->L * skv; a.fin_sb = d->H * a.fin_sh;
  a.B = d->B; a.H = d->H; a.S = nchunks(d); a.M = ngdn::CH; a.V = d->V;
  return launched(ngdn::scan_fwd(a, d->dtype, d->K, (hipStream_t)stream), "ngdn_l0_scan_fwd");
}

int32_t ngdn_probe_fwd(const ngdn_dims* d, int32_t level, int32_t promotion,
                       int32_t n_queries, int32_t f_below, int32_t f_here,
                       const void* below, int32_t ng_below,
                       const float* final_state, const void* query_banks,
                       int32_t n_max, const void* key_projections,
                       const void* bpT, const void* wpT, const void* gpT,
                       void* A, void* KT, void* U, float* gam, float* keys,
                       float* vals, float* bo, float* wo, float* go,
                       void* stream) {
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
  const int NT = nchunks(d);
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
  a.A = A; a.KT = KT; a.U = U; a.gam = gam;
  a.keys = keys; a.vals = vals; a.bo = bo; a.wo = wo; a.go = go;
  a.B = d->B; a.H = d->H; a.NF = NT / f_here; a.N = N; a.V = d->V;
  if (a.NF == 0) return NGDN_OK;
  return launched(ngdn::probe_fwd(a, d->dtype, d->K, (hipStream_t)stream), "ngdn_probe_fwd");
}

int32_t ngdn_upper_scan_fwd(const ngdn_dims* d, int32_t level, int32_t n_pairs,
                            int32_t nf, int32_t ng, const void* A,
                            const void* KT, const void* U, const float* gam,
                            const float* initial_state, float* states,
                            float* final_state, void* stream) {
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
  const long long skv = (long long)d->K * d->V;
  ngdn::ScanArgs a{};
  a.A = A; a.BT = KT; a.U = U; a.gam = gam;
  a.init = initial_state ? initial_state + (long long)level * skv : nullptr;
  a.init_sh = d->L * skv; a.init_sb = d->H * a.init_sh;
  a.states = states; a.state_mode = 1; a.NG = ng;
  a.vnT = nullptr;
  a.fin = final_state + (long long)level * skv; a.fin_sh = d->L * skv; a.fin_sb = d->H * a.fin_sh;
  a.B = d->B; a.H = d->H; a.S = nf; a.M = n_pairs; a.V = d->V;
  return launched(ngdn::scan_fwd(a, d->dtype, d->K, (hipStream_t)stream), "ngdn_upper_scan_fwd");
}

int32_t ngdn_output_fwd(const ngdn_dims* d, const void* Qg, const void* Aqk,
                        const void* hT, const void* vnT, const void* q,
                        const void* mix, const float* const* states,
                        const int32_t* ng, const int32_t* f, void* o,
                        float* reads, void* stream) {
  g_err[0] = 0;
  if (int32_t r = check_dims(d, "ngdn_output_fwd")) return r;
  if (d->K != d->V)
    return fail(NGDN_EINVAL, "ngdn_output_fwd: K == V required, got %d, %d", d->K, d->V);
  if (!Qg || !Aqk || !hT || !vnT || !q || !mix || !o)
    return fail(NGDN_EINVAL, "ngdn_output_fwd: NULL tensor");
  ngdn::OutputArgs a{};
  a.Qg = Qg; a.Aqk = Aqk; a.hT = hT; a.vnT = vnT; a.q = q; a.mix = mix;
  for (int l = 1; l < d->L; ++l) {
    if (!states || !states[l] || !ng || !f || f[l] <= 0)
      return fail(NGDN_EINVAL, "ngdn_output_fwd: level %d states missing", l);
    a.states[l] = states[l]; a.NGl[l] = ng[l]; a.f[l] = f[l];
  }
  a.o = o; a.reads = reads;
  a.B = d->B; a.T = d->T; a.H = d->H; a.L = d->L; a.NT = nchunks(d); a.scale = d->scale;
  return launched(ngdn::output_fwd(a, d->dtype, d->K, d->V, (hipStream_t)stream), "ngdn_output_fwd");
}

}  // extern "C"
