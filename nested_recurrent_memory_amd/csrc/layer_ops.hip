// The two elementwise modules the layer takes from fla (layers/nested_gdn2.py:
// 17-18,57-60,100): ShortConvolution (a causal depthwise convolution over
// time with a SiLU) and FusedRMSNormGated (RMS normalisation per head, times
// a learned weight and a sigmoid gate). Both are HBM-bound: every kernel reads
// its inputs once with 16-byte accesses and accumulates in fp32.
//
// ShortConvolution, per channel d of D, taps W:
//   a[t] = sum_{i<W} w[d][i] x[t - (W-1) + i],   y[t] = silu(a[t])
// rows before t = 0 come from the cache or are zero. The cache is fla's:
// [B][D][W], the last W inputs of the previous call with the newest last; a
// call with a cache output writes the last W inputs of [cache; x] there.
// FusedRMSNormGated, per row of V values:
//   y = x rstd w sigmoid(g),   rstd = 1 / sqrt(mean(x^2) + eps)
#include <numeric>

#include "ngdn_kernels.h"

namespace ngdn {

namespace {

__device__ __forceinline__ float silu_(float a) { return a * sigmoid_fast(a); }
__device__ __forceinline__ float dsilu_(float a) {
  const float s = sigmoid_fast(a);
  return s * (1.f + a * (1.f - s));
}

// input row s of batch b, channels d..d+7. Rows s < 0 (down to -W) come from
// the cache, [B][D][W] with the newest input last (entry W + s), or are zero.
template <typename E>
__device__ __forceinline__ void conv_row(const ShortConvArgs& a, int b, int s, int d, float* out) {
  if (s >= 0) {
    load8f(static_cast<const E*>(a.x) + ((size_t)b * a.T + s) * a.D + d, out);
  } else if (a.cache_in) {
    const E* c = static_cast<const E*>(a.cache_in) + ((size_t)b * a.D + d) * a.W + (a.W + s);
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = (float)c[(size_t)e * a.W];
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = 0.f;
  }
}

// N (4 or 8) consecutive values of a row as loaded (bf16: 8 or 16 bytes in
// 2 or 4 registers; fp32: one or two 16-byte quads), converted to float where
// used, so that rows held for a whole time block cost half the registers in
// bf16
template <typename E, int N> struct Raw;
template <int N> struct Raw<bf16, N> {
  typedef __attribute__((__vector_size__(N * sizeof(bf16)))) bf16 V;
  V v;
  __device__ __forceinline__ void load(const bf16* p) { v = *reinterpret_cast<const V*>(p); }
  __device__ __forceinline__ float operator[](int e) const { return (float)v[e]; }
  __device__ __forceinline__ void set(int e, float x) { v[e] = (bf16)x; }
  __device__ __forceinline__ void store(bf16* p) const { *reinterpret_cast<V*>(p) = v; }
};
template <int N> struct Raw<float, N> {
  f4 q[N / 4];
  __device__ __forceinline__ void load(const float* p) {
#pragma unroll
    for (int j = 0; j < N / 4; ++j) q[j] = *reinterpret_cast<const f4*>(p + 4 * j);
  }
  __device__ __forceinline__ float operator[](int e) const { return q[e / 4][e % 4]; }
  __device__ __forceinline__ void set(int e, float x) { q[e / 4][e % 4] = x; }
  __device__ __forceinline__ void store(float* p) const {
#pragma unroll
    for (int j = 0; j < N / 4; ++j) *reinterpret_cast<f4*>(p + 4 * j) = q[j];
  }
};

// input row s of batch b, channels d..d+N-1, into a raw row: rows s < 0 (down
// to -W) from the cache ([B][D][W], entry W + s) or zeros, rows past the end
// of the sequence zeros
template <typename E, int N>
__device__ __forceinline__ void conv_raw(const ShortConvArgs& a, int b, int s, int d, Raw<E, N>& out) {
  if (s >= 0 && s < a.T) {
    out.load(static_cast<const E*>(a.x) + ((size_t)b * a.T + s) * a.D + d);
  } else if (s < 0 && a.cache_in) {
    const E* c = static_cast<const E*>(a.cache_in) + ((size_t)b * a.D + d) * a.W + (a.W + s);
#pragma unroll
    for (int e = 0; e < N; ++e) out.set(e, (float)c[(size_t)e * a.W]);
  } else {
#pragma unroll
    for (int e = 0; e < N; ++e) out.set(e, 0.f);
  }
}

}  // namespace

// ---------------------------------------------------------------- ShortConvolution

// Work split of both kernels: a thread owns one group of CPT channels over
// RT consecutive time steps of one sequence (a "time block"); a workgroup is
// 64 channel groups (consecutive threads, so each row access of a wave is
// contiguous) by 4 time-block slots. The taps of the thread's channels are
// loaded once (CPT W fp32, contiguous) and the W - 1 rows before the block
// are the only rows read twice. The forward holds 8 channels, the backward
// (which keeps more rows live) 4.
constexpr int SC_CG = 64, SC_SLOTS = 4;

template <typename E> struct ScRT { static constexpr int f = sizeof(E) == 2 ? 8 : 4, b = sizeof(E) == 2 ? 8 : 4; };
constexpr int SC_CPT_F = 8, SC_CPT_B = 4;

template <int CPT, int W>
__device__ __forceinline__ void load_taps(const float* w, int d, float (&tw)[CPT][W]) {
  const f4* p = reinterpret_cast<const f4*>(w + (size_t)d * W);   // 4 CPT W bytes, 16-byte aligned
#pragma unroll
  for (int j = 0; j < CPT * W / 4; ++j) {
    const f4 v = p[j];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int f = 4 * j + e;
      tw[f / W][f % W] = v[e];
    }
  }
}

template <typename E, int W>
__global__ __launch_bounds__(256) void short_conv_fwd_kernel(ShortConvArgs a) {
  constexpr int RT = ScRT<E>::f, CPT = SC_CPT_F;
  const int DG = a.D / CPT, NTB = (a.T + RT - 1) / RT;
  const int ctiles = (DG + SC_CG - 1) / SC_CG;
  const int cg = (blockIdx.x % ctiles) * SC_CG + threadIdx.x % SC_CG;
  const long long q = (long long)(blockIdx.x / ctiles) * SC_SLOTS + threadIdx.x / SC_CG;
  if (cg >= DG || q >= (long long)a.B * NTB) return;
  const int d = cg * CPT, b = (int)(q / NTB), t0 = (int)(q % NTB) * RT;
  Raw<E, CPT> x[RT + W - 1];
#pragma unroll
  for (int r = 0; r < RT + W - 1; ++r) conv_raw<E, CPT>(a, b, t0 - (W - 1) + r, d, x[r]);
  float tw[CPT][W];
  load_taps<CPT, W>(a.w, d, tw);
#pragma unroll
  for (int r = 0; r < RT; ++r) {
    if (t0 + r >= a.T) break;
    Raw<E, CPT> y;
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      float acc = 0.f;
#pragma unroll
      for (int i = 0; i < W; ++i) acc += tw[c][i] * x[r + i][c];
      y.set(c, a.act ? silu_(acc) : acc);
    }
    y.store(static_cast<E*>(a.y) + ((size_t)b * a.T + t0 + r) * a.D + d);
  }
}

template <typename E>
__global__ __launch_bounds__(256) void short_conv_cache_kernel(ShortConvArgs a) {
  // new cache entry j of [B][D][W] = row T - W + j of the sequence [cache; x]
  const int D8 = a.D / 8;
  const long long e = (long long)blockIdx.x * 256 + threadIdx.x;
  if (e >= (long long)a.B * a.W * D8) return;
  const int d = (int)(e % D8) * 8;
  const long long bj = e / D8;
  const int j = (int)(bj % a.W), b = (int)(bj / a.W);
  float x[8];
  conv_row<E>(a, b, a.T - a.W + j, d, x);
  E* c = static_cast<E*>(a.cache_out) + ((size_t)b * a.D + d) * a.W + j;
#pragma unroll
  for (int k = 0; k < 8; ++k) c[(size_t)k * a.W] = (E)x[k];
}

// dx and dw, time blocks as in the forward. For the block's rows t0..t0+RT-1
// a thread forms the pre-activations a[s], s in t0 .. t0+RT+W-2 (the rows
// whose da its dx needs), da = dy silu'(a); then dx[t] = sum_u w[W-1-u]
// da[t+u] and dw[i] += da[t] x[t-(W-1)+i]. Each workgroup walks a range of
// time blocks (its 4 slots interleaved), keeps dw in registers, sums its
// slots in LDS and adds to dw with one atomic per weight.
template <typename E, int W>
__global__ __launch_bounds__(256) void short_conv_bwd_kernel(ShortConvArgs a) {
  constexpr int RT = ScRT<E>::b, CPT = SC_CPT_B;
  __shared__ float s_dw[SC_SLOTS][SC_CG][CPT * W + 1];
  const int DG = a.D / CPT, NTB = (a.T + RT - 1) / RT;
  const int ctiles = (DG + SC_CG - 1) / SC_CG;
  const int cl = threadIdx.x % SC_CG, slot = threadIdx.x / SC_CG;
  const int cg = (blockIdx.x % ctiles) * SC_CG + cl;
  const long long nq = (long long)a.B * NTB;
  const long long rg = blockIdx.x / ctiles, nrg = gridDim.x / ctiles;
  const bool live = cg < DG;
  const int d = cg * CPT;
  float dw[CPT][W];
#pragma unroll
  for (int c = 0; c < CPT; ++c)
#pragma unroll
    for (int i = 0; i < W; ++i) dw[c][i] = 0.f;
  if (live) {
    float tw[CPT][W];
    load_taps<CPT, W>(a.w, d, tw);
    for (long long q = rg * SC_SLOTS + slot; q < nq; q += nrg * SC_SLOTS) {
      const int b = (int)(q / NTB), t0 = (int)(q % NTB) * RT;
      // every load of the block first: input rows t0-(W-1) .. t0+RT+W-2 and
      // output-gradient rows t0 .. t0+RT+W-2 (zeros past the end)
      Raw<E, CPT> x[RT + 2 * W - 2], dyr[RT + W - 1];
#pragma unroll
      for (int r = 0; r < RT + 2 * W - 2; ++r) conv_raw<E, CPT>(a, b, t0 - (W - 1) + r, d, x[r]);
#pragma unroll
      for (int u = 0; u < RT + W - 1; ++u) {
        if (t0 + u < a.T) {
          dyr[u].load(static_cast<const E*>(a.dy) + ((size_t)b * a.T + t0 + u) * a.D + d);
        } else {
#pragma unroll
          for (int c = 0; c < CPT; ++c) dyr[u].set(c, 0.f);
        }
      }
      // da[u] at s = t0 + u, formed in order; dx of row r = u - (W-1) once
      // da[r .. r+W-1] exist, so only a window of W rows of da is live
      float da[RT + W - 1][CPT];
#pragma unroll
      for (int u = 0; u < RT + W - 1; ++u) {
#pragma unroll
        for (int c = 0; c < CPT; ++c) {
          float pre = 0.f;
#pragma unroll
          for (int i = 0; i < W; ++i) pre += tw[c][i] * x[u + i][c];
          da[u][c] = a.act ? dyr[u][c] * dsilu_(pre) : dyr[u][c];
        }
        if (u < RT) {
#pragma unroll
          for (int c = 0; c < CPT; ++c)
#pragma unroll
            for (int i = 0; i < W; ++i) dw[c][i] += da[u][c] * x[u + i][c];
        }
        const int r = u - (W - 1);
        if (r >= 0 && r < RT && t0 + r < a.T) {
          Raw<E, CPT> dx;
#pragma unroll
          for (int c = 0; c < CPT; ++c) {
            float acc = 0.f;
#pragma unroll
            for (int v = 0; v < W; ++v) acc += tw[c][W - 1 - v] * da[r + v][c];
            dx.set(c, acc);
          }
          dx.store(static_cast<E*>(a.dx) + ((size_t)b * a.T + t0 + r) * a.D + d);
        }
      }
    }
  }
#pragma unroll
  for (int c = 0; c < CPT; ++c)
#pragma unroll
    for (int i = 0; i < W; ++i) s_dw[slot][cl][c * W + i] = dw[c][i];
  __syncthreads();
  if (slot == 0 && live) {
#pragma unroll
    for (int k = 0; k < CPT * W; ++k) {
      float sum = 0.f;
#pragma unroll
      for (int sl = 0; sl < SC_SLOTS; ++sl) sum += s_dw[sl][cl][k];
      if (a.ws) a.ws[(size_t)rg * a.D * W + (size_t)d * W + k] = sum;
      else atomicAdd(&a.dw[(size_t)d * W + k], sum);
    }
  }
}

static unsigned sc_ctiles(const ShortConvArgs& a, int cpt) { return (unsigned)((a.D / cpt + SC_CG - 1) / SC_CG); }

hipError_t short_conv_fwd(const ShortConvArgs& a, int dtype, hipStream_t st) {
  if (a.D % 8 != 0 || a.W < 1 || a.W > 8) return hipErrorInvalidValue;
  if ((long long)a.B * a.T > 0) {
    const int RT = dtype == NGDN_BF16 ? ScRT<bf16>::f : ScRT<float>::f;
    const long long nq = (long long)a.B * ((a.T + RT - 1) / RT);
    const unsigned grid = sc_ctiles(a, SC_CPT_F) * (unsigned)((nq + SC_SLOTS - 1) / SC_SLOTS);
#define NGDN_CF(WW)                                                                              \
    if (a.W == WW) {                                                                             \
      if (dtype == NGDN_BF16) hipLaunchKernelGGL((short_conv_fwd_kernel<bf16, WW>), dim3(grid), dim3(256), 0, st, a); \
      else hipLaunchKernelGGL((short_conv_fwd_kernel<float, WW>), dim3(grid), dim3(256), 0, st, a); \
    }
    NGDN_CF(1) NGDN_CF(2) NGDN_CF(3) NGDN_CF(4) NGDN_CF(5) NGDN_CF(6) NGDN_CF(7) NGDN_CF(8)
#undef NGDN_CF
    if (hipError_t e = hipGetLastError()) return e;
  }
  if (a.cache_out) {
    const long long m = (long long)a.B * a.W * (a.D / 8);
    const unsigned grid = (unsigned)((m + 255) / 256);
    if (dtype == NGDN_BF16) hipLaunchKernelGGL(short_conv_cache_kernel<bf16>, dim3(grid), dim3(256), 0, st, a);
    else hipLaunchKernelGGL(short_conv_cache_kernel<float>, dim3(grid), dim3(256), 0, st, a);
    return hipGetLastError();
  }
  return hipSuccess;
}

hipError_t short_conv_bwd(ShortConvArgs a, int dtype, hipStream_t st) {
  if (a.D % 8 != 0 || a.W < 1 || a.W > 8) return hipErrorInvalidValue;
  if ((long long)a.B * a.T == 0) return hipSuccess;
  const int RT = dtype == NGDN_BF16 ? ScRT<bf16>::b : ScRT<float>::b;
  const long long nq = (long long)a.B * ((a.T + RT - 1) / RT);
  const unsigned ct = sc_ctiles(a, SC_CPT_B);
  // about 2048 workgroups, each walking its share of the time blocks; at
  // most NGDN_WPARTS rows of partial sums
  long long rgs = 2048 / ct;
  const long long most = (nq + SC_SLOTS - 1) / SC_SLOTS;
  rgs = rgs < 1 ? 1 : (rgs > most ? most : rgs);
  if (rgs > NGDN_WPARTS) rgs = NGDN_WPARTS;
  const unsigned grid = ct * (unsigned)rgs;
#define NGDN_CB(WW)                                                                              \
  if (a.W == WW) {                                                                               \
    if (dtype == NGDN_BF16) hipLaunchKernelGGL((short_conv_bwd_kernel<bf16, WW>), dim3(grid), dim3(256), 0, st, a); \
    else hipLaunchKernelGGL((short_conv_bwd_kernel<float, WW>), dim3(grid), dim3(256), 0, st, a); \
  }
  NGDN_CB(1) NGDN_CB(2) NGDN_CB(3) NGDN_CB(4) NGDN_CB(5) NGDN_CB(6) NGDN_CB(7) NGDN_CB(8)
#undef NGDN_CB
  if (hipError_t e = hipGetLastError()) return e;
  return a.ws ? sum_parts(a.ws, rgs, (long long)a.D * a.W, a.dw, st) : hipSuccess;
}

// ---------------------------------------------------------------- gate prologue

namespace {

// max and sum over the first 8 lanes (the mix weights of one head, L <= 8)
__device__ __forceinline__ float max8(float v) {
#pragma unroll
  for (int o = 4; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, WAVE));
  return v;
}
__device__ __forceinline__ float sum8(float v) {
#pragma unroll
  for (int o = 4; o > 0; o >>= 1) v += __shfl_xor(v, o, WAVE);
  return v;
}
template <typename P> __device__ __forceinline__ float ldp(const void* p, size_t i) {
  return to_f(static_cast<const P*>(p)[i]);
}
// torch's softplus (beta 1, threshold 20) and its derivative. log1p(e^z) as
// max(z, 0) + log1p(t), t = e^-|z| in (0, 1], from the hardware exp and log;
// log1p(t) = log(u) t / (u - 1) with u = 1 + t rounded (the quotient undoes
// the rounding of u; Goldberg, "What every computer scientist should know
// about floating-point arithmetic", 1991, theorem 4), a few ulp. The library
// log1pf was several times the instructions of the rest of the prologue.
__device__ __forceinline__ float softplus20(float z) {
  if (z > 20.f) return z;
  const float t = __expf(-fabsf(z));
  const float u = 1.f + t;
  const float l = u == 1.f ? t : __logf(u) * (t * __builtin_amdgcn_rcpf(u - 1.f));
  return fmaxf(z, 0.f) + l;
}
__device__ __forceinline__ float dsoftplus20(float z) { return z > 20.f ? 1.f : sigmoid_fast(z); }

}  // namespace

// One wave per (b, t, h), heads fastest, so a workgroup's 4 waves read
// neighbouring parts of the same token's rows. Every access is 16 bytes: a K row is
// VK = K/8 lanes, so the L + 1 rows to normalise (q's levels, then k) take
// (L+1) VK lanes (one pass for L = 3, K = 128), and the f, bz, wz rows sit
// side by side in lanes [0, VK), [VK, 2 VK), [2 VK, 2 VK + V/8).
template <int G>
__device__ __forceinline__ float gsum(float v) {   // sum over aligned groups of G lanes
#pragma unroll
  for (int o = G / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, WAVE);
  return v;
}

// A wave takes GP_TPW consecutive token-heads and issues every load of all
// of them before the first use (each lane's row vectors to normalise, NP
// passes of 64 vectors; its gate vector; its mix logit): one token-head per
// wave left each wave two dependent memory round trips for 4 KB and ran at
// under half the copy rate.
constexpr int GP_TPW = 4;

template <typename E, typename P, int K, int V, int NP>
__global__ __launch_bounds__(256) void gate_prep_fwd_kernel(GatePrepArgs a) {
  constexpr int VK = K / 8, VV = V / 8;
  const int H = a.H, L = a.L, lane = lane_id();
  const long long th0 = ((long long)blockIdx.x * 4 + wave_id()) * GP_TPW, nth = a.BT * H;
  if (th0 >= nth) return;
  const bool isf = lane < VK, isb = !isf && lane < 2 * VK, isw = !isf && !isb && lane < 2 * VK + VV;
  // token and head of the wave's first token-head (one division), then by
  // steps: a 64-bit division per token-head was most of the scalar work
  const long long bt0 = th0 / H;
  const int h0 = (int)(th0 - bt0 * H);
  float x[GP_TPW][NP][8], z[GP_TPW][8], zm[GP_TPW];
#pragma unroll
  for (int j = 0; j < GP_TPW; ++j) {
    const long long th = th0 + j;
    const int hj = h0 + j;
    const long long bt = bt0 + hj / H;
    const int h = hj % H;
    const bool live = th < nth;
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const int r = (p * WAVE + lane) / VK, c = (p * WAVE + lane) % VK * 8;
      if (live && r <= L) {
        const E* src = r < L ? static_cast<const E*>(a.q) + (bt * L + r) * H * K + (size_t)h * K
                             : static_cast<const E*>(a.k) + th * K;
        load8f(src + c, x[j][p]);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) x[j][p][e] = 0.f;
      }
    }
    const size_t go = isf ? th * K + (size_t)lane * 8
                    : isb ? th * K + (size_t)(lane - VK) * 8 : th * V + (size_t)(lane - 2 * VK) * 8;
    if (live && (isf || isb || isw)) {
      load8f(static_cast<const E*>(isf ? a.f : isb ? a.bz : a.wz) + go, z[j]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) z[j][e] = 0.f;
    }
    zm[j] = live && lane < L ? to_f(static_cast<const E*>(a.ml)[th * L + lane]) : -INFINITY;
  }
#pragma unroll
  for (int j = 0; j < GP_TPW; ++j) {
    const long long th = th0 + j;
    if (th >= nth) break;
    const int h = (h0 + j) % H;
    // q's L rows, transposed from (l h) to (h l), and k: x / max(|x|, eps)
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const int r = (p * WAVE + lane) / VK, c = (p * WAVE + lane) % VK * 8;
      float ss = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += x[j][p][e] * x[j][p][e];
      const float inv = 1.f / fmaxf(sqrtf(gsum<VK>(ss)), 1e-12f);
      if (r <= L) {
        E* dst = r < L ? static_cast<E*>(a.qn) + (th * L + r) * K : static_cast<E*>(a.kn) + th * K;
#pragma unroll
        for (int e = 0; e < 8; ++e) x[j][p][e] *= inv;
        store8f(dst + c, x[j][p]);
      }
    }
    // decay (lanes [0, VK)), b gate ([VK, 2 VK)), w gate ([2 VK, 2 VK + VV))
    const size_t go = isf ? th * K + (size_t)lane * 8
                    : isb ? th * K + (size_t)(lane - VK) * 8 : th * V + (size_t)(lane - 2 * VK) * 8;
    if (isf) {
      const int c = lane * 8;
      const float A = __expf(ldp<P>(a.A_log, h));
      float dtv[8];
      load8f(static_cast<const P*>(a.dt_bias) + (size_t)h * K + c, dtv);
      f4 g[2];
#pragma unroll
      for (int e = 0; e < 8; ++e)
        g[e / 4][e % 4] = fminf(-A * softplus20(z[j][e] + dtv[e]), a.cap);
      *reinterpret_cast<f4*>(a.g0 + go) = g[0];
      *reinterpret_cast<f4*>(a.g0 + go + 4) = g[1];
    } else if (isb || isw) {
#pragma unroll
      for (int e = 0; e < 8; ++e) z[j][e] = sigmoid_fast(z[j][e]);
      store8f(static_cast<E*>(isb ? a.b0 : a.w0) + go, z[j]);
    }
    // mix over the L levels in lanes 0..7 (all 8 take part in the shuffles)
    if (lane < 8) {
      const float mx = max8(zm[j]);
      const float e = lane < L ? __expf(zm[j] - mx) : 0.f;
      const float den = sum8(e);
      const float m = a.sigmoid_mix ? sigmoid_fast(zm[j]) : e / den;
      if (lane < L) static_cast<E*>(a.mix)[th * L + lane] = from_f<E>(m);
    }
  }
}

// Backward, same mapping; waves walk token-heads grid-stride with a stride
// that is a multiple of H, so each wave keeps one head and its decay
// parameters' gradients collect in registers; then one partial row per
// workgroup (zeros for the heads none of its waves had).
template <typename E, typename P, int K, int V>
__global__ __launch_bounds__(256) void gate_prep_bwd_kernel(GatePrepArgs a) {
  constexpr int VK = K / 8, VV = V / 8;
  __shared__ float s_dt[4][K], s_da[4];
  const int H = a.H, L = a.L, lane = lane_id(), wv = wave_id();
  const long long th0 = (long long)blockIdx.x * 4 + wv, stride = (long long)gridDim.x * 4;
  const int h = (int)(th0 % H);
  const float A = __expf(ldp<P>(a.A_log, h));
  float ddt[8], dA = 0.f, dtb[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) ddt[e] = dtb[e] = 0.f;
  if (lane < VK) load8f(static_cast<const P*>(a.dt_bias) + (size_t)h * K + lane * 8, dtb);
  const long long bstep = stride / H;          // the stride is a multiple of H
  long long bt = th0 / H;
  for (long long th = th0; th < a.BT * H; th += stride, bt += bstep) {
    for (int base = 0; base < (L + 1) * VK; base += WAVE) {
      const int r = (base + lane) / VK, c = (base + lane) % VK * 8;
      const bool live = r <= L;
      const size_t xo = r < L ? (bt * L + r) * H * K + (size_t)h * K : th * K;
      const size_t yo = r < L ? (th * L + r) * K : th * K;
      float x[8], g[8], ss = 0.f, xg = 0.f;
      if (live) {
        load8f(static_cast<const E*>(r < L ? a.q : a.k) + xo + c, x);
        load8f(static_cast<const E*>(r < L ? a.dqn : a.dkn) + yo + c, g);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = g[e] = 0.f;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) { ss += x[e] * x[e]; xg += x[e] * g[e]; }
      const float n = sqrtf(gsum<VK>(ss));
      xg = gsum<VK>(xg);
      // y = x / max(n, eps): dx = dy / n - x <x, dy> / n^3 above eps, dy / eps below
      const float inv = 1.f / fmaxf(n, 1e-12f);
      const float cc = n > 1e-12f ? xg * inv * inv * inv : 0.f;
      if (live) {
#pragma unroll
        for (int e = 0; e < 8; ++e) g[e] = g[e] * inv - x[e] * cc;
        store8f(static_cast<E*>(r < L ? a.dq : a.dk) + xo + c, g);
      }
    }
    if (lane < VK) {
      const int c = lane * 8;
      float f[8], df[8];
      load8f(static_cast<const E*>(a.f) + th * K + c, f);
      const f4 d0 = *reinterpret_cast<const f4*>(a.dg0 + th * K + c);
      const f4 d1 = *reinterpret_cast<const f4*>(a.dg0 + th * K + c + 4);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float z = f[e] + dtb[e];
        const float gu = -A * softplus20(z);
        const float dg = gu <= a.cap ? (e < 4 ? d0[e] : d1[e - 4]) : 0.f;   // clamp(max) passes at equality
        dA += dg * gu;
        df[e] = -A * dg * dsoftplus20(z);
        ddt[e] += df[e];
      }
      store8f(static_cast<E*>(a.df) + th * K + c, df);
    } else if (lane < 2 * VK + VV) {
      const bool isb = lane < 2 * VK;
      const size_t o = isb ? th * K + (size_t)(lane - VK) * 8 : th * V + (size_t)(lane - 2 * VK) * 8;
      float z[8], d[8];
      load8f(static_cast<const E*>(isb ? a.bz : a.wz) + o, z);
      load8f(static_cast<const E*>(isb ? a.db0 : a.dw0) + o, d);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float sg = sigmoid_fast(z[e]);
        d[e] *= sg * (1.f - sg);
      }
      store8f(static_cast<E*>(isb ? a.dbz : a.dwz) + o, d);
    }
    if (lane < 8) {
      const float z = lane < L ? to_f(static_cast<const E*>(a.ml)[th * L + lane]) : -INFINITY;
      const float dm = lane < L ? to_f(static_cast<const E*>(a.dmix)[th * L + lane]) : 0.f;
      const float mx = max8(z);
      const float e = lane < L ? __expf(z - mx) : 0.f;
      const float ms = e / sum8(e);
      const float dot = sum8(ms * dm);
      const float sg = sigmoid_fast(z);
      const float dz = a.sigmoid_mix ? dm * sg * (1.f - sg) : ms * (dm - dot);
      if (lane < L) static_cast<E*>(a.dml)[th * L + lane] = from_f<E>(dz);
    }
  }
  // the decay parameters: waves -> LDS -> one partial row per workgroup
  dA = wave_sum(dA);
  if (lane < VK) {
#pragma unroll
    for (int e = 0; e < 8; ++e) s_dt[wv][lane * 8 + e] = ddt[e];
  }
  if (lane == 0) s_da[wv] = dA;
  __syncthreads();
  const int n = H * K + H;
  int hw[4];
#pragma unroll
  for (int w = 0; w < 4; ++w) hw[w] = (int)(((long long)blockIdx.x * 4 + w) % H);
  float* row = a.ws ? a.ws + (size_t)blockIdx.x * n : nullptr;
  for (int j = threadIdx.x; j < n; j += 256) {
    const int hh = j < H * K ? j / K : j - H * K;
    float v = 0.f;
    bool any = false;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      if (hw[w] != hh) continue;
      v += j < H * K ? s_dt[w][j % K] : s_da[w];
      any = true;
    }
    if (row) row[j] = v;
    else if (any) atomicAdd(&a.dpar[j], v);
  }
}

#define NGDN_GP_DISPATCH(KERNEL, GRID)                                                         \
  do {                                                                                         \
    const dim3 grid_ = (GRID);                                                                 \
    auto go = [&](auto e, auto p, auto kk, auto vv) {                                          \
      hipLaunchKernelGGL((KERNEL<decltype(e), decltype(p), decltype(kk)::value,                \
                                 decltype(vv)::value>), grid_, dim3(256), 0, st, a);           \
    };                                                                                         \
    using I64 = std::integral_constant<int, 64>;                                               \
    using I128 = std::integral_constant<int, 128>;                                             \
    auto pick_kv = [&](auto e, auto p) {                                                       \
      if (a.K == 64 && a.V == 64) go(e, p, I64{}, I64{});                                      \
      else if (a.K == 64 && a.V == 128) go(e, p, I64{}, I128{});                               \
      else if (a.K == 128 && a.V == 64) go(e, p, I128{}, I64{});                               \
      else go(e, p, I128{}, I128{});                                                           \
    };                                                                                         \
    auto pick_p = [&](auto e) {                                                                \
      if (a.pdtype == NGDN_BF16) pick_kv(e, bf16{}); else pick_kv(e, float{});                 \
    };                                                                                         \
    if (dtype == NGDN_BF16) pick_p(bf16{}); else pick_p(float{});                              \
  } while (0)

static bool gate_prep_ok(const GatePrepArgs& a) {
  return (a.K == 64 || a.K == 128) && (a.V == 64 || a.V == 128) && a.L >= 1 && a.L <= 8 && a.H > 0;
}

hipError_t gate_prep_fwd(const GatePrepArgs& a, int dtype, hipStream_t st) {
  if (!gate_prep_ok(a)) return hipErrorInvalidValue;
  if (a.BT == 0) return hipSuccess;
  const dim3 grid((unsigned)((a.BT * a.H + 4 * GP_TPW - 1) / (4 * GP_TPW)));
  const int np = ((a.L + 1) * (a.K / 8) + WAVE - 1) / WAVE;
  auto go = [&](auto e, auto p, auto kk, auto vv, auto npc) {
    hipLaunchKernelGGL((gate_prep_fwd_kernel<decltype(e), decltype(p), decltype(kk)::value,
                                             decltype(vv)::value, decltype(npc)::value>),
                       grid, dim3(256), 0, st, a);
  };
  using I64 = std::integral_constant<int, 64>;
  using I128 = std::integral_constant<int, 128>;
  auto pick_np = [&](auto e, auto p, auto kk, auto vv) {
    if (np == 1) go(e, p, kk, vv, std::integral_constant<int, 1>{});
    else if (np == 2) go(e, p, kk, vv, std::integral_constant<int, 2>{});
    else go(e, p, kk, vv, std::integral_constant<int, 3>{});
  };
  auto pick_kv = [&](auto e, auto p) {
    if (a.K == 64 && a.V == 64) pick_np(e, p, I64{}, I64{});
    else if (a.K == 64 && a.V == 128) pick_np(e, p, I64{}, I128{});
    else if (a.K == 128 && a.V == 64) pick_np(e, p, I128{}, I64{});
    else pick_np(e, p, I128{}, I128{});
  };
  auto pick_p = [&](auto e) {
    if (a.pdtype == NGDN_BF16) pick_kv(e, bf16{}); else pick_kv(e, float{});
  };
  if (dtype == NGDN_BF16) pick_p(bf16{}); else pick_p(float{});
  return hipGetLastError();
}

hipError_t gate_prep_bwd(const GatePrepArgs& a, int dtype, hipStream_t st) {
  if (!gate_prep_ok(a)) return hipErrorInvalidValue;
  if (a.BT == 0) return hipSuccess;
  // about 8 token-heads per wave, at most NGDN_WPARTS partial rows, and a
  // wave stride (4 nb) that is a multiple of H
  const long long m = a.H / std::gcd(a.H, 4);
  long long nb = (a.BT * a.H + 31) / 32;
  if (nb > NGDN_WPARTS) nb = NGDN_WPARTS;
  nb = (nb + m - 1) / m * m;
  if (nb > NGDN_WPARTS) nb -= m;
  if (nb < m) return hipErrorInvalidValue;    // H beyond 4 NGDN_WPARTS
  NGDN_GP_DISPATCH(gate_prep_bwd_kernel, dim3((unsigned)nb));
  if (hipError_t e = hipGetLastError()) return e;
  return a.ws ? sum_parts(a.ws, nb, (long long)a.H * a.K + a.H, a.dpar, st) : hipSuccess;
}

// ---------------------------------------------------------------- FusedRMSNormGated

// 16 lanes per row (8 values each), four rows per wave, 16 rows per workgroup
template <typename E, int V>
__global__ __launch_bounds__(256) void rmsnorm_gated_fwd_kernel(NormGatedArgs a) {
  constexpr int LPR = V / 8;                          // lanes per row
  static_assert(LPR <= WAVE && WAVE % LPR == 0, "rows within a wave");
  const long long row = ((long long)blockIdx.x * 256 + threadIdx.x) / LPR;
  const int c = (threadIdx.x % LPR) * 8;
  const bool live = row < a.rows;
  float x[8], g[8];
  if (live) {
    load8f(static_cast<const E*>(a.x) + row * V + c, x);
    load8f(static_cast<const E*>(a.g) + row * V + c, g);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = g[e] = 0.f;
  }
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss += x[e] * x[e];
#pragma unroll
  for (int o = LPR / 2; o > 0; o >>= 1) ss += __shfl_xor(ss, o, WAVE);
  const float rstd = 1.f / sqrtf(ss / (float)V + a.eps);
  if (!live) return;
  float y[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) y[e] = x[e] * rstd * a.w[c + e] * sigmoid_fast(g[e]);
  store8f(static_cast<E*>(a.y) + row * V + c, y);
  if (a.rstd && c == 0) a.rstd[row] = rstd;
}

// dx, dg per row; dw summed over the rows a thread visits, then over the
// workgroup in LDS, then one atomic per weight and workgroup
template <typename E, int V>
__global__ __launch_bounds__(256) void rmsnorm_gated_bwd_kernel(NormGatedArgs a) {
  constexpr int LPR = V / 8, RPB = 256 / LPR;         // lanes per row, rows per pass
  __shared__ float s_dw[RPB][V];
  const int c = (threadIdx.x % LPR) * 8, rs = threadIdx.x / LPR;
  float dw[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) dw[e] = 0.f;
  for (long long row = (long long)blockIdx.x * RPB + rs; row < a.rows; row += (long long)gridDim.x * RPB) {
    float x[8], g[8], dy[8];
    load8f(static_cast<const E*>(a.x) + row * V + c, x);
    load8f(static_cast<const E*>(a.g) + row * V + c, g);
    load8f(static_cast<const E*>(a.dy) + row * V + c, dy);
    const float rstd = a.rstd[row];
    float xh[8], s[8], dxh[8], dot = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      xh[e] = x[e] * rstd;
      s[e] = sigmoid_fast(g[e]);
      dxh[e] = dy[e] * a.w[c + e] * s[e];
      dot += dxh[e] * xh[e];
      dw[e] += dy[e] * xh[e] * s[e];
    }
#pragma unroll
    for (int o = LPR / 2; o > 0; o >>= 1) dot += __shfl_xor(dot, o, WAVE);
    const float mean = dot / (float)V;
    float dx[8], dg[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      dx[e] = rstd * (dxh[e] - xh[e] * mean);
      dg[e] = dy[e] * xh[e] * a.w[c + e] * s[e] * (1.f - s[e]);
    }
    store8f(static_cast<E*>(a.dx) + row * V + c, dx);
    store8f(static_cast<E*>(a.dg) + row * V + c, dg);
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) s_dw[rs][c + e] = dw[e];
  __syncthreads();
  for (int v = threadIdx.x; v < V; v += 256) {
    float sum = 0.f;
    for (int r = 0; r < RPB; ++r) sum += s_dw[r][v];
    if (a.ws) a.ws[(size_t)blockIdx.x * V + v] = sum;
    else atomicAdd(&a.dw[v], sum);
  }
}

hipError_t rmsnorm_gated_fwd(const NormGatedArgs& a, int dtype, int V, hipStream_t st) {
  if (a.rows == 0) return hipSuccess;
#define NGDN_NG(VV)                                                                         \
  if (V == VV) {                                                                            \
    const unsigned grid = (unsigned)((a.rows * (VV / 8) + 255) / 256);                      \
    if (dtype == NGDN_BF16)                                                                 \
      hipLaunchKernelGGL((rmsnorm_gated_fwd_kernel<bf16, VV>), dim3(grid), dim3(256), 0, st, a); \
    else                                                                                    \
      hipLaunchKernelGGL((rmsnorm_gated_fwd_kernel<float, VV>), dim3(grid), dim3(256), 0, st, a); \
    return hipGetLastError();                                                               \
  }
  NGDN_NG(64) NGDN_NG(128) NGDN_NG(256)
#undef NGDN_NG
  return hipErrorInvalidValue;
}

hipError_t rmsnorm_gated_bwd(const NormGatedArgs& a, int dtype, int V, hipStream_t st) {
  if (a.rows == 0) return hipSuccess;
#define NGDN_NG(VV)                                                                         \
  if (V == VV) {                                                                            \
    constexpr int RPB = 256 / (VV / 8);                                                     \
    const long long want = (a.rows + RPB * 16 - 1) / (RPB * 16);   /* ~16 rows per thread */ \
    const unsigned grid = (unsigned)(want < NGDN_WPARTS ? (want > 0 ? want : 1) : NGDN_WPARTS); \
    if (dtype == NGDN_BF16)                                                                 \
      hipLaunchKernelGGL((rmsnorm_gated_bwd_kernel<bf16, VV>), dim3(grid), dim3(256), 0, st, a); \
    else                                                                                    \
      hipLaunchKernelGGL((rmsnorm_gated_bwd_kernel<float, VV>), dim3(grid), dim3(256), 0, st, a); \
    if (hipError_t e = hipGetLastError()) return e;                                         \
    return a.ws ? sum_parts(a.ws, grid, VV, a.dw, st) : hipSuccess;                         \
  }
  NGDN_NG(64) NGDN_NG(128) NGDN_NG(256)
#undef NGDN_NG
  return hipErrorInvalidValue;
}

}  // namespace ngdn
