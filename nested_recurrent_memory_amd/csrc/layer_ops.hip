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
#include "ngdn_kernels.h"

namespace ngdn {

namespace {

__device__ __forceinline__ float silu_(float a) { return a / (1.f + expf(-a)); }
__device__ __forceinline__ float dsilu_(float a) {
  const float s = 1.f / (1.f + expf(-a));
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

}  // namespace

// ---------------------------------------------------------------- ShortConvolution

template <typename E, int W>
__global__ __launch_bounds__(256) void short_conv_fwd_kernel(ShortConvArgs a) {
  // thread: 8 channels of one (b, t); the W input rows are 16-byte loads
  const int D8 = a.D / 8;
  const long long e = (long long)blockIdx.x * 256 + threadIdx.x;
  if (e >= (long long)a.B * a.T * D8) return;
  const int d = (int)(e % D8) * 8;
  const long long bt = e / D8;
  const int t = (int)(bt % a.T), b = (int)(bt / a.T);
  float acc[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) acc[c] = 0.f;
#pragma unroll
  for (int i = 0; i < W; ++i) {
    float x[8];
    conv_row<E>(a, b, t - (W - 1) + i, d, x);
#pragma unroll
    for (int c = 0; c < 8; ++c) acc[c] += a.w[(size_t)(d + c) * W + i] * x[c];
  }
  float y[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) y[c] = a.act ? silu_(acc[c]) : acc[c];
  store8f(static_cast<E*>(a.y) + ((size_t)b * a.T + t) * a.D + d, y);
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

// dx and dw. A workgroup owns 32 groups of 8 channels and a block of rows;
// each thread walks rows r = lane-row, lane-row + 8, ...: it recomputes the
// pre-activation a[s] of the rows s = t .. t+W-1 its dx needs and adds
// da[t] x[t-(W-1)+i] to its dw partials; the 8 row lanes of a channel group
// are summed in LDS and added to dw with one atomic per weight.
template <typename E, int W>
__global__ __launch_bounds__(256) void short_conv_bwd_kernel(ShortConvArgs a) {
  constexpr int CG = 32, RL = 8, MAXW = W;
  __shared__ float s_dw[RL][CG][8 * MAXW];
  const int D8 = a.D / 8;
  const int cg = threadIdx.x % CG, rl = threadIdx.x / CG;
  const int dgrp = blockIdx.x % ((D8 + CG - 1) / CG) * CG + cg;
  const int rb = blockIdx.x / ((D8 + CG - 1) / CG);
  const int d = dgrp * 8;
  const bool live = dgrp < D8;
  float dw[8 * MAXW];
#pragma unroll
  for (int k = 0; k < 8 * MAXW; ++k) dw[k] = 0.f;
  const long long rows = (long long)a.B * a.T;
  const long long r0 = (long long)rb * a.rows_per_block;
  const long long r1 = min(rows, r0 + a.rows_per_block);
  if (live) {
    for (long long r = r0 + rl; r < r1; r += RL) {
      const int t = (int)(r % a.T), b = (int)(r / a.T);
      // inputs x[t - (W-1) .. t + W-1]: 2W - 1 rows
      float xs[2 * MAXW - 1][8];
#pragma unroll
      for (int q = 0; q < 2 * W - 1; ++q) {
        const int s = t - (W - 1) + q;
        if (s < a.T) {
          conv_row<E>(a, b, s, d, xs[q]);
        } else {
#pragma unroll
          for (int c = 0; c < 8; ++c) xs[q][c] = 0.f;
        }
      }
      float dx[8];
#pragma unroll
      for (int c = 0; c < 8; ++c) dx[c] = 0.f;
      // da at s = t + u (u < W), each a pre-activation over xs[u .. u+W-1]
#pragma unroll
      for (int u = 0; u < W; ++u) {
        if (t + u >= a.T) continue;
        float dy[8];
        load8f(static_cast<const E*>(a.dy) + ((size_t)b * a.T + t + u) * a.D + d, dy);
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          float pre = 0.f;
#pragma unroll
          for (int i = 0; i < W; ++i) pre += a.w[(size_t)(d + c) * W + i] * xs[u + i][c];
          const float da = a.act ? dy[c] * dsilu_(pre) : dy[c];
          // x[t] enters a[t + u] through tap W-1-u
          dx[c] += a.w[(size_t)(d + c) * W + (W - 1 - u)] * da;
          if (u == 0) {
#pragma unroll
            for (int i = 0; i < W; ++i) dw[c * MAXW + i] += da * xs[i][c];
          }
        }
      }
      store8f(static_cast<E*>(a.dx) + ((size_t)b * a.T + t) * a.D + d, dx);
    }
  }
#pragma unroll
  for (int k = 0; k < 8 * MAXW; ++k) s_dw[rl][cg][k] = dw[k];
  __syncthreads();
  if (rl == 0 && live) {
#pragma unroll
    for (int c = 0; c < 8; ++c)
#pragma unroll
      for (int i = 0; i < W; ++i) {
        float s = 0.f;
#pragma unroll
        for (int q = 0; q < RL; ++q) s += s_dw[q][cg][c * MAXW + i];
        atomicAdd(&a.dw[(size_t)(d + c) * W + i], s);
      }
  }
}

hipError_t short_conv_fwd(const ShortConvArgs& a, int dtype, hipStream_t st) {
  if (a.D % 8 != 0 || a.W < 1 || a.W > 8) return hipErrorInvalidValue;
  const long long n = (long long)a.B * a.T * (a.D / 8);
  if (n > 0) {
    const unsigned grid = (unsigned)((n + 255) / 256);
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
  const long long rows = (long long)a.B * a.T;
  if (rows == 0) return hipSuccess;
  a.rows_per_block = 256;
  const int cblocks = (a.D / 8 + 31) / 32;
  const long long rblocks = (rows + a.rows_per_block - 1) / a.rows_per_block;
  const unsigned grid = (unsigned)(cblocks * rblocks);
#define NGDN_CB(WW)                                                                              \
  if (a.W == WW) {                                                                               \
    if (dtype == NGDN_BF16) hipLaunchKernelGGL((short_conv_bwd_kernel<bf16, WW>), dim3(grid), dim3(256), 0, st, a); \
    else hipLaunchKernelGGL((short_conv_bwd_kernel<float, WW>), dim3(grid), dim3(256), 0, st, a); \
  }
  NGDN_CB(1) NGDN_CB(2) NGDN_CB(3) NGDN_CB(4) NGDN_CB(5) NGDN_CB(6) NGDN_CB(7) NGDN_CB(8)
#undef NGDN_CB
  return hipGetLastError();
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
  for (int e = 0; e < 8; ++e) y[e] = x[e] * rstd * a.w[c + e] / (1.f + expf(-g[e]));
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
      s[e] = 1.f / (1.f + expf(-g[e]));
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
    atomicAdd(&a.dw[v], sum);
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
    const unsigned grid = (unsigned)(want < 2048 ? (want > 0 ? want : 1) : 2048);           \
    if (dtype == NGDN_BF16)                                                                 \
      hipLaunchKernelGGL((rmsnorm_gated_bwd_kernel<bf16, VV>), dim3(grid), dim3(256), 0, st, a); \
    else                                                                                    \
      hipLaunchKernelGGL((rmsnorm_gated_bwd_kernel<float, VV>), dim3(grid), dim3(256), 0, st, a); \
    return hipGetLastError();                                                               \
  }
  NGDN_NG(64) NGDN_NG(128) NGDN_NG(256)
#undef NGDN_NG
  return hipErrorInvalidValue;
}

}  // namespace ngdn
