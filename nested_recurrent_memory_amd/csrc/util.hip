// Small whole-op utilities, each one launch in place of several framework
// kernels: the casts of the op's fp32 gradients to bf16, and the transposes
// of the per-level parameters into the layouts the promotion kernels read.
#include "ngdn_kernels.h"

namespace ngdn {

// One launch for every cast: blockIdx.y picks the array, the blocks along x
// stride over it.
__global__ __launch_bounds__(256) void cast_bf16_kernel(CastArgs a) {
  const int w = blockIdx.y;
  const long long n = a.n[w];
  const float* s = a.src[w];
  bf16* d = static_cast<bf16*>(a.dst[w]);
  for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long long)gridDim.x * 256)
    d[i] = from_f<bf16>(s[i]);
}

hipError_t cast_bf16(const CastArgs& a, hipStream_t st) {
  long long nmax = 0;
  for (int w = 0; w < a.count; ++w) nmax = a.n[w] > nmax ? a.n[w] : nmax;
  if (a.count == 0 || nmax == 0) return hipSuccess;
  const long long bx = (nmax + 255) / 256;
  const dim3 grid((unsigned)(bx < 2048 ? bx : 2048), (unsigned)a.count);
  hipLaunchKernelGGL(cast_bf16_kernel, grid, dim3(256), 0, st, a);
  return hipGetLastError();
}

// Batched transposes of the last two axes, 32 x 32 tiles through LDS (reads
// and writes both along rows). Block x: tile t of array w, where
// tiles0[w] <= x < tiles0[w + 1]; the array's tiles run batch-major.
template <typename T>
__global__ __launch_bounds__(256) void transpose_kernel(TransposeArgs a) {
  __shared__ T tile[32][33];
  int w = 0;
  while (w + 1 < a.count && (int)blockIdx.x >= a.tiles0[w + 1]) ++w;
  const int t = blockIdx.x - a.tiles0[w];
  const int R = a.R[w], C = a.C[w];
  const int tr = (R + 31) / 32, tc = (C + 31) / 32;
  const int b = t / (tr * tc), rt = (t / tc) % tr, ct = t % tc;
  const T* s = static_cast<const T*>(a.src[w]) + (size_t)b * R * C;
  T* d = static_cast<T*>(a.dst[w]) + (size_t)b * R * C;
  const int tx = threadIdx.x % 32, ty = threadIdx.x / 32;
  for (int i = ty; i < 32; i += 8) {
    const int r = rt * 32 + i, c = ct * 32 + tx;
    if (r < R && c < C) tile[i][tx] = s[(size_t)r * C + c];
  }
  __syncthreads();
  for (int i = ty; i < 32; i += 8) {
    const int c = ct * 32 + i, r = rt * 32 + tx;
    if (r < R && c < C) d[(size_t)c * R + r] = tile[tx][i];
  }
}

hipError_t transpose(const TransposeArgs& a, hipStream_t st) {
  const int tiles = a.tiles0[a.count];
  if (a.count == 0 || tiles == 0) return hipSuccess;
  if (a.esz == 2)
    hipLaunchKernelGGL(transpose_kernel<unsigned short>, dim3(tiles), dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL(transpose_kernel<float>, dim3(tiles), dim3(256), 0, st, a);
  return hipGetLastError();
}

}  // namespace ngdn
