// The three modules the model takes from fla around the layer
// (models/modeling_nested_gdn2.py:15-17,44-56,97-99,230-239): RMSNorm,
// the SwiGLU of GatedMLP and the cross entropy of FusedLinearCrossEntropyLoss
// (the linear parts are hipBLASLt GEMMs on the host side). All HBM-bound:
// each kernel reads its inputs once with 16-byte accesses, computes in fp32
// and writes its outputs once.
//
// RMSNorm, per row of D:      y = x rstd w,   rstd = 1 / sqrt(mean(x^2) + eps)
// SwiGLU, elementwise:        y = silu(g) u
// Cross entropy, per row r:   loss_r = logsumexp(x_r) - x_r[label_r]
//   (a row's logits are held in registers between the statistics and the
//   gradient, so the row is read from HBM once and written once)
#include "ngdn_kernels.h"

namespace ngdn {

namespace {

__device__ __forceinline__ float sigm(float a) { return sigmoid_fast(a); }

// sum over the G lanes of a row group (G a power of two <= 64, groups aligned)
template <int G>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int o = G / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, WAVE);
  return v;
}

}  // namespace

// ---------------------------------------------------------------- RMSNorm

// G lanes per row, each holding VPL runs of 8 values: D = 8 G VPL. Lane l of
// a row owns columns (v G + l) 8 .. +7, so a wave's 16-byte accesses are
// contiguous. X is the dtype of x (and of h), R of the residual r, Y of y.
// With r set the row is first h = x + r, rounded to X and written to a.h,
// and normalised from that rounded value (as a separate add would store it).
template <typename X, typename R, typename Y, int G, int VPL>
__global__ __launch_bounds__(256) void rmsnorm_fwd_kernel(RMSNormArgs a) {
  constexpr int D = 8 * G * VPL;
  const long long row = ((long long)blockIdx.x * 256 + threadIdx.x) / G;
  const int li = threadIdx.x % G;
  const bool live = row < a.rows;
  const bool add = a.r != nullptr;
  const X* xr = static_cast<const X*>(a.x) + row * D;
  const R* rr = static_cast<const R*>(a.r) + row * D;
  float x[VPL][8], t[VPL][8];
#pragma unroll
  for (int v = 0; v < VPL; ++v) {
    if (live) {
      load8f(xr + (v * G + li) * 8, x[v]);
      if (add) load8f(rr + (v * G + li) * 8, t[v]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) x[v][e] = t[v][e] = 0.f;
    }
  }
  if (add) {
#pragma unroll
    for (int v = 0; v < VPL; ++v) {
#pragma unroll
      for (int e = 0; e < 8; ++e) x[v][e] = to_f(from_f<X>(x[v][e] + t[v][e]));
      if (live) store8f(static_cast<X*>(a.h) + row * D + (v * G + li) * 8, x[v]);
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int v = 0; v < VPL; ++v)
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += x[v][e] * x[v][e];
  ss = group_sum<G>(ss);
  const float rstd = 1.f / sqrtf(ss / (float)D + a.eps);
  if (!live) return;
  Y* yr = static_cast<Y*>(a.y) + row * D;
#pragma unroll
  for (int v = 0; v < VPL; ++v) {
    const int c = (v * G + li) * 8;
    float y[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) y[e] = x[v][e] * rstd * a.w[c + e];
    store8f(yr + c, y);
  }
  if (a.rstd && li == 0) a.rstd[row] = rstd;
}

// dx = rstd (dy w - xh mean(dy w xh)) (+ dh, the gradient h receives besides
// the norm, when set), dw += dy xh with xh = x rstd; with dr set, dx is also
// written in R's dtype (the residual's gradient). x is h when the forward
// added a residual. Rows are visited grid-stride; a thread's dw partials are
// summed over the workgroup's row slots in LDS, then written as the
// workgroup's partial row (or added to dw with one atomic per column).
template <typename X, typename R, typename Y, int G, int VPL>
__global__ __launch_bounds__(256) void rmsnorm_bwd_kernel(RMSNormArgs a) {
  constexpr int D = 8 * G * VPL, RPB = 256 / G;
  __shared__ float s_dw[RPB][D];
  const int li = threadIdx.x % G, rs = threadIdx.x / G;
  const bool res = a.dh != nullptr;
  float dw[VPL][8];
#pragma unroll
  for (int v = 0; v < VPL; ++v)
#pragma unroll
    for (int e = 0; e < 8; ++e) dw[v][e] = 0.f;
  for (long long row = (long long)blockIdx.x * RPB + rs; row < a.rows;
       row += (long long)gridDim.x * RPB) {
    const X* xr = static_cast<const X*>(a.x) + row * D;
    const Y* dyr = static_cast<const Y*>(a.dy) + row * D;
    const X* dhr = static_cast<const X*>(a.dh) + row * D;
    float x[VPL][8], dy[VPL][8], dh[VPL][8];
#pragma unroll
    for (int v = 0; v < VPL; ++v) {
      load8f(xr + (v * G + li) * 8, x[v]);
      load8f(dyr + (v * G + li) * 8, dy[v]);
      if (res) load8f(dhr + (v * G + li) * 8, dh[v]);
    }
    const float rstd = a.rstd[row];
    float dot = 0.f;
#pragma unroll
    for (int v = 0; v < VPL; ++v) {
      const int c = (v * G + li) * 8;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        x[v][e] *= rstd;                         // xh
        dw[v][e] += dy[v][e] * x[v][e];
        dy[v][e] *= a.w[c + e];                  // dxh
        dot += dy[v][e] * x[v][e];
      }
    }
    const float mean = group_sum<G>(dot) / (float)D;
    X* dxr = static_cast<X*>(a.dx) + row * D;
    R* drr = static_cast<R*>(a.dr) + row * D;
#pragma unroll
    for (int v = 0; v < VPL; ++v) {
      float dx[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) dx[e] = rstd * (dy[v][e] - x[v][e] * mean) + (res ? dh[v][e] : 0.f);
      store8f(dxr + (v * G + li) * 8, dx);
      if (a.dr) store8f(drr + (v * G + li) * 8, dx);
    }
  }
#pragma unroll
  for (int v = 0; v < VPL; ++v)
#pragma unroll
    for (int e = 0; e < 8; ++e) s_dw[rs][(v * G + li) * 8 + e] = dw[v][e];
  __syncthreads();
  for (int c = threadIdx.x; c < D; c += 256) {
    float sum = 0.f;
#pragma unroll
    for (int r = 0; r < RPB; ++r) sum += s_dw[r][c];
    if (a.ws) a.ws[(size_t)blockIdx.x * D + c] = sum;
    else atomicAdd(&a.dw[c], sum);
  }
}

// Supported widths: D = 512 VPL for VPL in 1..6 (up to 3072; the backward's
// registers run out beyond), and 64, 128, 256, 768 (fewer lanes per row).
#define NGDN_RMS_SHAPES(X) \
  X(8, 1) X(16, 1) X(32, 1) X(32, 3) X(64, 1) X(64, 2) X(64, 3) X(64, 4) X(64, 5) X(64, 6)

bool rmsnorm_supported(int D) {
#define NGDN_RMS_OK(GG, VV) if (D == 8 * GG * VV) return true;
  NGDN_RMS_SHAPES(NGDN_RMS_OK)
#undef NGDN_RMS_OK
  return false;
}

// dtype combinations (x, r, y): all fp32, all bf16, or fp32 x with bf16 r and
// y (an fp32 residual stream under bf16 autocast)
bool rmsnorm_types_supported(int xd, int rd, int yd) {
  return (xd == rd && rd == yd && (xd == NGDN_F32 || xd == NGDN_BF16)) ||
         (xd == NGDN_F32 && rd == NGDN_BF16 && yd == NGDN_BF16);
}

#define NGDN_RMS_TYPED(KERNEL, GG, VV, grid, xd, rd)                                          \
  if (xd == NGDN_BF16)                                                                        \
    hipLaunchKernelGGL((KERNEL<bf16, bf16, bf16, GG, VV>), dim3(grid), dim3(256), 0, st, a);  \
  else if (rd == NGDN_BF16)                                                                   \
    hipLaunchKernelGGL((KERNEL<float, bf16, bf16, GG, VV>), dim3(grid), dim3(256), 0, st, a); \
  else                                                                                        \
    hipLaunchKernelGGL((KERNEL<float, float, float, GG, VV>), dim3(grid), dim3(256), 0, st, a);

hipError_t rmsnorm_fwd(const RMSNormArgs& a, int xd, int rd, int yd, hipStream_t st) {
  if (!rmsnorm_types_supported(xd, rd, yd)) return hipErrorInvalidValue;
  if (a.rows == 0) return hipSuccess;
#define NGDN_RMS_F(GG, VV)                                                   \
  if (a.D == 8 * GG * VV) {                                                  \
    const unsigned grid = (unsigned)((a.rows * GG + 255) / 256);             \
    NGDN_RMS_TYPED(rmsnorm_fwd_kernel, GG, VV, grid, xd, rd)                 \
    return hipGetLastError();                                                \
  }
  NGDN_RMS_SHAPES(NGDN_RMS_F)
#undef NGDN_RMS_F
  return hipErrorInvalidValue;
}

hipError_t rmsnorm_bwd(const RMSNormArgs& a, int xd, int rd, int yd, hipStream_t st) {
  if (!rmsnorm_types_supported(xd, rd, yd)) return hipErrorInvalidValue;
  if (a.rows == 0) return hipSuccess;
#define NGDN_RMS_B(GG, VV)                                                                   \
  if (a.D == 8 * GG * VV) {                                                                  \
    constexpr long long RPB = 256 / GG;                                                      \
    const long long want = (a.rows + RPB * 16 - 1) / (RPB * 16);   /* ~16 rows per slot */   \
    const unsigned grid = (unsigned)(want < NGDN_WPARTS ? want : NGDN_WPARTS);               \
    NGDN_RMS_TYPED(rmsnorm_bwd_kernel, GG, VV, grid, xd, rd)                                 \
    if (hipError_t e = hipGetLastError()) return e;                                          \
    return a.ws ? sum_parts(a.ws, grid, a.D, a.dw, st) : hipSuccess;                         \
  }
  NGDN_RMS_SHAPES(NGDN_RMS_B)
#undef NGDN_RMS_B
  return hipErrorInvalidValue;
}
#undef NGDN_RMS_TYPED

// ---------------------------------------------------------------- partial sums

// out[j] += sum_p ws[p][j]: a workgroup takes 64 columns and a range of at
// most 64 rows (4 slices of 16), sums in LDS and adds with one atomic per
// column, so no address sees more than nparts / 64 atomics
constexpr int SP_COLS = 64, SP_ROWS = 64;

__global__ __launch_bounds__(256) void sum_parts_kernel(const float* ws, long long nparts, long long n,
                                                        float* out) {
  __shared__ float s_part[4][SP_COLS];
  const long long j = (long long)blockIdx.x * SP_COLS + threadIdx.x % SP_COLS;
  const int slice = threadIdx.x / SP_COLS;
  const long long p0 = (long long)blockIdx.y * SP_ROWS + slice * (SP_ROWS / 4);
  float acc = 0.f;
  if (j < n) {
#pragma unroll
    for (int r = 0; r < SP_ROWS / 4; ++r) {
      const long long p = p0 + r;
      if (p < nparts) acc += ws[(size_t)p * n + j];
    }
  }
  s_part[slice][threadIdx.x % SP_COLS] = acc;
  __syncthreads();
  if (slice == 0 && j < n)
    atomicAdd(&out[j], s_part[0][threadIdx.x] + s_part[1][threadIdx.x] + s_part[2][threadIdx.x] +
                       s_part[3][threadIdx.x]);
}

hipError_t sum_parts(const float* ws, long long nparts, long long n, float* out, hipStream_t st) {
  if (n == 0 || nparts == 0) return hipSuccess;
  const dim3 grid((unsigned)((n + SP_COLS - 1) / SP_COLS), (unsigned)((nparts + SP_ROWS - 1) / SP_ROWS));
  hipLaunchKernelGGL(sum_parts_kernel, grid, dim3(256), 0, st, ws, nparts, n, out);
  return hipGetLastError();
}

// ---------------------------------------------------------------- SwiGLU

template <typename E>
__global__ __launch_bounds__(256) void swiglu_fwd_kernel(SwigluArgs a) {
  const long long n8 = a.n / 8;
  for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n8;
       i += (long long)gridDim.x * 256) {
    float g[8], u[8], y[8];
    load8f(static_cast<const E*>(a.g) + i * 8, g);
    load8f(static_cast<const E*>(a.u) + i * 8, u);
#pragma unroll
    for (int e = 0; e < 8; ++e) y[e] = g[e] * sigm(g[e]) * u[e];
    store8f(static_cast<E*>(a.y) + i * 8, y);
  }
}

template <typename E>
__global__ __launch_bounds__(256) void swiglu_bwd_kernel(SwigluArgs a) {
  const long long n8 = a.n / 8;
  for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n8;
       i += (long long)gridDim.x * 256) {
    float g[8], u[8], dy[8], dg[8], du[8];
    load8f(static_cast<const E*>(a.g) + i * 8, g);
    load8f(static_cast<const E*>(a.u) + i * 8, u);
    load8f(static_cast<const E*>(a.dy) + i * 8, dy);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float s = sigm(g[e]);
      du[e] = dy[e] * g[e] * s;
      dg[e] = dy[e] * u[e] * s * (1.f + g[e] * (1.f - s));
    }
    store8f(static_cast<E*>(a.dg) + i * 8, dg);
    store8f(static_cast<E*>(a.du) + i * 8, du);
  }
}

static unsigned elementwise_grid(long long n8) {
  const long long want = (n8 + 255) / 256;
  return (unsigned)(want < 8192 ? (want > 0 ? want : 1) : 8192);   // 32 waves per CU, grid-stride
}

hipError_t swiglu_fwd(const SwigluArgs& a, int dtype, hipStream_t st) {
  if (a.n == 0) return hipSuccess;
  const unsigned grid = elementwise_grid(a.n / 8);
  if (dtype == NGDN_BF16) hipLaunchKernelGGL(swiglu_fwd_kernel<bf16>, dim3(grid), dim3(256), 0, st, a);
  else hipLaunchKernelGGL(swiglu_fwd_kernel<float>, dim3(grid), dim3(256), 0, st, a);
  return hipGetLastError();
}

hipError_t swiglu_bwd(const SwigluArgs& a, int dtype, hipStream_t st) {
  if (a.n == 0) return hipSuccess;
  const unsigned grid = elementwise_grid(a.n / 8);
  if (dtype == NGDN_BF16) hipLaunchKernelGGL(swiglu_bwd_kernel<bf16>, dim3(grid), dim3(256), 0, st, a);
  else hipLaunchKernelGGL(swiglu_bwd_kernel<float>, dim3(grid), dim3(256), 0, st, a);
  return hipGetLastError();
}

// ---------------------------------------------------------------- sum into fp32

template <typename E, int C>
__global__ __launch_bounds__(256) void sum_f32_kernel(SumArgs a) {
  const long long n8 = a.n / 8;
  for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n8;
       i += (long long)gridDim.x * 256) {
    float v[C][8];
#pragma unroll
    for (int j = 0; j < C; ++j) load8f(static_cast<const E*>(a.x[j]) + i * 8, v[j]);
    f4 o[2];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float acc = 0.f;
#pragma unroll
      for (int j = 0; j < C; ++j) acc += v[j][e];
      o[e / 4][e % 4] = acc;
    }
    *reinterpret_cast<f4*>(a.out + i * 8) = o[0];
    *reinterpret_cast<f4*>(a.out + i * 8 + 4) = o[1];
  }
}

hipError_t sum_into_f32(const SumArgs& a, int dtype, hipStream_t st) {
  if (a.n == 0) return hipSuccess;
  if (a.count < 1 || a.count > SUM_MAX || a.n % 8 != 0) return hipErrorInvalidValue;
  const long long want = (a.n / 8 + 255) / 256;
  const dim3 grid((unsigned)(want < 8192 ? want : 8192));
#define NGDN_SUM(CC)                                                                           \
  if (a.count == CC) {                                                                         \
    if (dtype == NGDN_BF16) hipLaunchKernelGGL((sum_f32_kernel<bf16, CC>), grid, dim3(256), 0, st, a); \
    else hipLaunchKernelGGL((sum_f32_kernel<float, CC>), grid, dim3(256), 0, st, a);         \
    return hipGetLastError();                                                                  \
  }
  NGDN_SUM(1) NGDN_SUM(2) NGDN_SUM(3) NGDN_SUM(4) NGDN_SUM(5) NGDN_SUM(6) NGDN_SUM(7) NGDN_SUM(8)
#undef NGDN_SUM
  return hipErrorInvalidValue;
}

// ---------------------------------------------------------------- cross entropy

// One workgroup of NTH threads per row; thread t holds the row's runs of 8
// logits t, t + NTH, ... (NV of them, the last ones partly past V/8 and
// masked). Statistics: a running max and a sum of exponentials rescaled to
// it, merged across the workgroup; then the gradient from the registers.
template <typename E, int NTH, int NV>
__global__ __launch_bounds__(NTH) void xent_kernel(XentArgs a) {
  constexpr int NW = NTH / WAVE;
  __shared__ float s_m[NW], s_s[NW];
  const long long row = blockIdx.x;
  const int tid = threadIdx.x, V8 = a.V / 8;
  E* xr = static_cast<E*>(a.logits) + row * a.V;
  const long long label = a.labels[row];
  const bool ignored = label == a.ignore_index;
  // a label outside [0, V) that is not ignore_index gives NaN (loss and row
  // gradient) instead of a read out of the row
  const bool bad = !ignored && (label < 0 || label >= a.V);
  float x[NV][8];
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int i = v * NTH + tid;
    if (i < V8) {
      load8f(xr + (size_t)i * 8, x[v]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) x[v][e] = -INFINITY;
    }
  }
  float m = -INFINITY;
#pragma unroll
  for (int v = 0; v < NV; ++v)
#pragma unroll
    for (int e = 0; e < 8; ++e) m = fmaxf(m, x[v][e]);
  float s = 0.f;
  if (m > -INFINITY) {
#pragma unroll
    for (int v = 0; v < NV; ++v)
#pragma unroll
      for (int e = 0; e < 8; ++e) s += __expf(x[v][e] - m);
  }
  // merge (m, s) over the wave, then over the waves
#pragma unroll
  for (int o = WAVE / 2; o > 0; o >>= 1) {
    const float mo = __shfl_xor(m, o, WAVE), so = __shfl_xor(s, o, WAVE);
    const float mn = fmaxf(m, mo);
    s = (m > -INFINITY ? s * __expf(m - mn) : 0.f) + (mo > -INFINITY ? so * __expf(mo - mn) : 0.f);
    m = mn;
  }
  if (lane_id() == 0) { s_m[wave_id()] = m; s_s[wave_id()] = s; }
  __syncthreads();
  float M = s_m[0];
#pragma unroll
  for (int w = 1; w < NW; ++w) M = fmaxf(M, s_m[w]);
  float S = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) S += s_s[w] * __expf(s_m[w] - M);
  const float lse = M + __logf(S);
  const long long nv = a.n_valid[0];
  const float inv_n = 1.f / (float)nv;
  if (tid == 0) {
    // with no label left the mean is 0/0, as torch's: NaN
    const float xl = (ignored || bad) ? 0.f : to_f(xr[label]);
    a.row_loss[row] = ignored ? (nv == 0 ? NAN : 0.f) : (bad ? NAN : (lse - xl) * inv_n);
  }
  if (!a.grad) return;
  __syncthreads();   // thread 0's read of the label's logit precedes the overwrite
  const float sc = ignored ? 0.f : (bad ? NAN : inv_n);
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int i = v * NTH + tid;
    if (i < V8) {
      float d[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const long long col = (long long)i * 8 + e;
        d[e] = (__expf(x[v][e] - lse) - (col == label ? 1.f : 0.f)) * sc;
      }
      store8f(xr + (size_t)i * 8, d);
    }
  }
}

bool xent_supported(int V) { return V > 0 && V % 8 == 0 && V <= 8 * 1024 * 8; }

hipError_t cross_entropy(const XentArgs& a, int dtype, hipStream_t st) {
  if (a.rows == 0) return hipSuccess;
  if (!xent_supported(a.V)) return hipErrorInvalidValue;
  const int V8 = a.V / 8;
  const dim3 grid((unsigned)a.rows);
#define NGDN_XE(NTH, NV)                                                                      \
  if (V8 <= NTH * NV) {                                                                       \
    if (dtype == NGDN_BF16) hipLaunchKernelGGL((xent_kernel<bf16, NTH, NV>), grid, dim3(NTH), 0, st, a); \
    else hipLaunchKernelGGL((xent_kernel<float, NTH, NV>), grid, dim3(NTH), 0, st, a);      \
    return hipGetLastError();                                                                 \
  }
  NGDN_XE(256, 1) NGDN_XE(256, 2) NGDN_XE(256, 4) NGDN_XE(256, 8) NGDN_XE(256, 16)
  NGDN_XE(1024, 8)
#undef NGDN_XE
  return hipErrorInvalidValue;
}

}  // namespace ngdn
