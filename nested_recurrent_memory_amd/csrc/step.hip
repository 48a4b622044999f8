// One decoding token (nested_gdn2/ops/naive.py:42-134), level-0 half:
//   S0 <- e^g S0 - k ((k*b)^T (e^g S0)) + k (v*w)^T      (ops/naive.py:7-39 with N = 1)
//   read_l = (scale q_l)^T S_l  for every level, S0 already updated
//   o = sum_l mix_l read_l
// The promotions that follow at chunk boundaries reuse the probe and the
// firing scan (one firing), gated per row on the device by the position.
//
// Columns of V never interact here either: a workgroup owns SV = 32 columns
// of one (batch, head), the grid is B*H*(V/32), and the slices of one
// (batch, head) sit on one XCD. Each thread holds 4 adjacent columns (one
// 16-byte load per row) of K/32 rows of every level's state; the two sums over
// K (the erase projection and the reads) go through wave shuffles and a
// 4-wave LDS exchange. The work is one pass over the state: HBM-bound.
#include "ngdn_kernels.h"

namespace ngdn {

template <typename E, int K, int V>
__global__ __launch_bounds__(256) void step_kernel(StepArgs a) {
  constexpr int SV = 32;                 // columns per workgroup
  constexpr int CQ = SV / 4;             // threads across one row (4 columns each)
  constexpr int RG = 256 / CQ;           // row groups
  constexpr int RPT = K / RG;            // rows per thread
  constexpr int NW = 256 / WAVE;
  static_assert(RPT >= 1 && K % RG == 0, "K must be a multiple of 32");
  __shared__ __attribute__((aligned(16))) float s_red[NW][SV];
  __shared__ __attribute__((aligned(16))) float s_rd[NW][MAXL][SV];

  const int H = a.H, L = a.L;
  int bh, vs;
  xcd_split(blockIdx.x, gridDim.x, V / SV, bh, vs);
  const int h = bh % H, b = bh / H;
  const int tid = threadIdx.x, lane = lane_id(), wv = wave_id();
  const int cq = tid % CQ, rg = tid / CQ;
  const int col = vs * SV + cq * 4;

  const E* q = static_cast<const E*>(a.q) + (size_t)bh * L * K;
  const E* kk = static_cast<const E*>(a.k) + (size_t)bh * K;
  const E* bb = static_cast<const E*>(a.b) + (size_t)bh * K;
  const float* gg = a.g + (size_t)bh * K;
  const size_t sbase = (size_t)bh * L * K * V;
  const float* Sin = a.s_in + sbase;
  float* Sout = a.s_out + sbase;
  const bool copy_up = a.s_out != a.s_in;

  // ---- level 0: decay, erase projection r = (k*b)^T (e^g S0)
  f4 s0[RPT];
  float key[RPT];
  f4 part = f4_zero();
#pragma unroll
  for (int r = 0; r < RPT; ++r) {
    const int k = rg * RPT + r;
    s0[r] = *reinterpret_cast<const f4*>(Sin + (size_t)k * V + col);
    const float gam = expf(gg[k]);
    key[r] = to_f(kk[k]);
    const float kb = key[r] * to_f(bb[k]);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      s0[r][c] *= gam;
      part[c] += kb * s0[r][c];
    }
  }
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    part[c] += __shfl_xor(part[c], 8, WAVE);
    part[c] += __shfl_xor(part[c], 16, WAVE);
    part[c] += __shfl_xor(part[c], 32, WAVE);
  }
  if (lane < CQ) *reinterpret_cast<f4*>(&s_red[wv][cq * 4]) = part;

  // reads of the upper levels (unchanged by this token)
  f4 rd[MAXL];
#pragma unroll
  for (int l = 0; l < MAXL; ++l) rd[l] = f4_zero();
#pragma unroll
  for (int l = 1; l < MAXL; ++l) {
    if (l < L) {
      const float* Sl = Sin + (size_t)l * K * V;
#pragma unroll
      for (int r = 0; r < RPT; ++r) {
        const int k = rg * RPT + r;
        const f4 x = *reinterpret_cast<const f4*>(Sl + (size_t)k * V + col);
        const float ql = to_f(q[(size_t)l * K + k]) * a.scale;
#pragma unroll
        for (int c = 0; c < 4; ++c) rd[l][c] += ql * x[c];
      }
    }
  }
  lds_barrier();
  f4 u;
  {
    const E* vv = static_cast<const E*>(a.v) + (size_t)bh * V + col;
    const E* ww = static_cast<const E*>(a.w) + (size_t)bh * V + col;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float r = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) r += s_red[w][cq * 4 + c];
      u[c] = to_f(vv[c]) * to_f(ww[c]) - r;
    }
  }

  // ---- S0 += k u^T, written; reads of every level (the upper levels were
  // read above, before any store)
#pragma unroll
  for (int r = 0; r < RPT; ++r) {
    const int k = rg * RPT + r;
#pragma unroll
    for (int c = 0; c < 4; ++c) s0[r][c] += key[r] * u[c];
    *reinterpret_cast<f4*>(Sout + (size_t)k * V + col) = s0[r];
    const float ql = to_f(q[k]) * a.scale;
#pragma unroll
    for (int c = 0; c < 4; ++c) rd[0][c] += ql * s0[r][c];
  }
#pragma unroll
  for (int l = 0; l < MAXL; ++l) {
    if (l < L) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        rd[l][c] += __shfl_xor(rd[l][c], 8, WAVE);
        rd[l][c] += __shfl_xor(rd[l][c], 16, WAVE);
        rd[l][c] += __shfl_xor(rd[l][c], 32, WAVE);
      }
      if (lane < CQ) *reinterpret_cast<f4*>(&s_rd[wv][l][cq * 4]) = rd[l];
    }
  }
  lds_barrier();

  // ---- o = sum_l mix_l read_l
  if (tid < CQ) {
    const E* mix = static_cast<const E*>(a.mix) + (size_t)bh * L;
    E* o = static_cast<E*>(a.o) + (size_t)bh * V + col;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float acc = 0.f;
      for (int l = 0; l < L; ++l) {
        float r = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) r += s_rd[w][l][cq * 4 + c];
        acc += r * to_f(mix[l]);
      }
      o[c] = from_f<E>(acc);
    }
  }
  // out of place: the upper levels are copied last (after every load)
  if (copy_up) {
    for (int l = 1; l < L; ++l) {
#pragma unroll
      for (int r = 0; r < RPT; ++r) {
        const size_t off = (size_t)l * K * V + (size_t)(rg * RPT + r) * V + col;
        *reinterpret_cast<f4*>(Sout + off) = *reinterpret_cast<const f4*>(Sin + off);
      }
    }
  }
}

template <typename E, int K, int V>
static hipError_t launch_step(const StepArgs& a, hipStream_t st) {
  const unsigned grid = (unsigned)(a.B * a.H * (V / 32));
  hipLaunchKernelGGL((step_kernel<E, K, V>), dim3(grid), dim3(256), 0, st, a);
  return hipGetLastError();
}

hipError_t step_fwd(const StepArgs& a, int dtype, int K, int V, hipStream_t st) {
#define NGDN_ST(E, KK, VV) \
  if (K == KK && V == VV) return launch_step<E, KK, VV>(a, st);
  if (dtype == NGDN_BF16) {
    NGDN_ST(bf16, 64, 64) NGDN_ST(bf16, 64, 128) NGDN_ST(bf16, 128, 64) NGDN_ST(bf16, 128, 128)
  } else {
    NGDN_ST(float, 64, 64) NGDN_ST(float, 64, 128) NGDN_ST(float, 128, 64) NGDN_ST(float, 128, 128)
  }
#undef NGDN_ST
  return hipErrorInvalidValue;
}

}  // namespace ngdn
