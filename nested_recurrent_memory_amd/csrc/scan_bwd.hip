// Reverse of the delta-rule step chain (scan.hip), run per (batch, head,
// 32-column slice of V) with the fp32 state gradient in registers.
//
// Forward step: Vn = U - A S;  S' = diag(gam) S + BT Vn.  Given dS' (the
// gradient of the state after the step):
//   dVn = Bop dS'             (Bop = BT^T)
//   dS  = diag(gam) dS' - AT dVn      (AT = A^T)
// Level 0 (the reverse dh recurrence of the reference's vendored fla
// backward, nested_gdn2/ops/_vendor/common_chunk_delta_h.py:25-380) also
// carries the chunk's output o = Qg S + Aqk Vn with dO = mix_0 * do:
//   dVn += Aqk^T dO,   dS += Qg^T dO,
// and takes the promotion gradient of level 1 at every firing chunk: before
// the step of chunk n with (n+1) % f1 == 0 the injection inj[(n+1)/f1 - 1] is
// added -- the gradient of the state entering chunk n+1, which the reference
// hands to fla as dh_ext (ops/chunk.py:519-528).
// Levels >= 1 (ops/update_bwd.py:93-158): after group j's firing, the read
// gradient of the state entering group j joins: dS += d_states[j], plus, when
// a firing i of the level above read that state (j = ((i+1) f_above) /
// f_here), that firing's injection inj[i] (the level above's probe gradient).
//
// Stores, per step (fp32): dS' (the gradient of the state after it) and dVn.
// Every operand but do is derived; for bf16 inputs each product is three bf16
// MFMAs on split operands. As in the forward scan, the slices of one (batch,
// head) share an XCD and each step's operands (which do not depend on the
// state gradient) are read one step ahead.
#include "ngdn_kernels.h"

namespace ngdn {

// ---------------------------------------------------------------- levels >= 1
//
// FRB (bf16, M % 32 == 0): AT in fragment order, as the probes write it.
template <typename E, int K, int M, bool FRB, int BV>
__global__ __launch_bounds__(256) void scan_bwd_kernel(ScanBwdArgs a) {
  constexpr int CT = BV / 16;
  constexpr int RTS = K / 16;
  constexpr int TPW = RTS * CT / 4;
  constexpr int TRT = TPW / CT;               // distinct state row tiles per wave
  constexpr int RTV = M / 16;
  constexpr int RPW = (RTV + 3) / 4;          // dVn row tiles per wave (at most)
  using ST = SplitTile<E>;
  constexpr int LDS_ST = K + ST::PAD;
  constexpr int LDS_VN = M + ST::PAD;
  constexpr int KS = Mma<E>::KS;
  constexpr int NSK = K / KS;
  constexpr int NSM = (M + KS - 1) / KS;
  constexpr bool PADM = (M % KS) != 0;
  static_assert(TPW % CT == 0, "state tiles of a wave come in whole rows");
  // dS'^T and dVn^T, split once by their writers
  __shared__ __attribute__((aligned(16))) typename ST::T s_dst[ST::NPLANE * BV * LDS_ST];
  __shared__ __attribute__((aligned(16))) typename ST::T s_dvn[ST::NPLANE * BV * LDS_VN];
  const ST sdS{s_dst, BV * LDS_ST}, sdV{s_dvn, BV * LDS_VN};

  const int V = a.V, S = a.S, H = a.H;
  const int nvt = V / BV;
  int vt, bh;
  xcd_split(blockIdx.x, gridDim.x, nvt, bh, vt);
  const int h = bh % H, b = bh / H;
  const int v0 = vt * BV;
  const int lane = lane_id(), wv = wave_id();

  f4 ds[TPW];
#pragma unroll
  for (int i = 0; i < TPW; ++i) {
    const int g = wv * TPW + i, rt = g / CT, ct = g % CT;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int k = rt * 16 + acc_row(r), v = v0 + ct * 16 + acc_col();
      ds[i][r] = a.d_final ? a.d_final[b * a.df_sb + h * a.df_sh + (long long)k * V + v] : 0.f;
    }
  }
  // values of a [K][V] fp32 array at this wave's state tiles
  auto read_kv = [&](const float* src, f4* out) {
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      const int g = wv * TPW + i, rt = g / CT, ct = g % CT;
#pragma unroll
      for (int r = 0; r < 4; ++r)
        out[i][r] = src[(size_t)(rt * 16 + acc_row(r)) * V + v0 + ct * 16 + acc_col()];
    }
  };
  auto dstates = [&](int j) {
    return a.d_states + (((size_t)b * a.NG + j) * H + h) * K * V;
  };
  // the injection of the firing i of the level above that read the state
  // entering group j, if any: i + 1 = m = ceil(j f_here / f_above) when
  // (m f_above) / f_here == j (intervals f_above >= f_here: at most one m)
  auto inj_tile = [&](int j) -> const float* {
    if (!a.inj || j < 1) return nullptr;
    const int m = (j * a.inj_fh + a.inj_fa - 1) / a.inj_fa;
    if (m < 1 || m > a.inj_nf || (m * a.inj_fa) / a.inj_fh != j) return nullptr;
    return a.inj + ((size_t)bh * a.inj_nf + m - 1) * K * V;
  };
  for (int j = a.NG - 1; j >= S; --j) {
    f4 x[TPW];
    read_kv(dstates(j), x);
    if (const float* p = inj_tile(j)) {
      f4 y[TPW];
      read_kv(p, y);
#pragma unroll
      for (int i = 0; i < TPW; ++i) x[i] += y[i];
    }
#pragma unroll
    for (int i = 0; i < TPW; ++i) ds[i] += x[i];
  }

  const float* Bb = a.Bop + (size_t)bh * S * M * K;
  const float* Ab = a.AT + (size_t)bh * S * K * M;
  const float* Gb = a.gam + (size_t)bh * S * K;

  // Operands of one step, read a step ahead: they do not depend on the state gradient.
  typedef typename Mma<E>::SFrag SF;
  struct Ops {
    SF bop[RPW][NSK];           // Bop rows of this wave's dVn tiles
    SF at[TRT][NSM];            // A^T rows of this wave's state tiles
    float g[TRT][4];
    f4 add[TPW];                // the read gradient of the group the step starts
    f4 inj[TPW];                // and, when has_inj, the injection into it
    bool has_inj;
  };
  auto load = [&](int j, Ops& o) {
    const SplitTile<E> Bj = split_at<E>(Bb + (size_t)j * M * K, M * K);
    const SplitTile<E> Aj = split_at<E>(Ab + (size_t)j * K * M, K * M);
    const float* Gj = Gb + (size_t)j * K;
#pragma unroll
    for (int p = 0; p < RPW; ++p) {
      const int rt = wv + 4 * p;
      if (rt < RTV) {
        const int brow = (rt * 16 + (lane & 15)) * K + kofs<E>(lane);
#pragma unroll
        for (int s = 0; s < NSK; ++s) o.bop[p][s] = Bj.get(brow + s * KS);
      }
    }
#pragma unroll
    for (int t = 0; t < TRT; ++t) {
      const int rt = (wv * TPW) / CT + t;
      const int arow = (rt * 16 + (lane & 15)) * M + kofs<E>(lane);
#pragma unroll
      for (int s = 0; s < NSM; ++s)
        o.at[t][s] = FRB ? Aj.get(frag_at(rt, s, M))
                        : (!PADM || s * KS + kofs<E>(lane) < M) ? Aj.get(arow + s * KS)
                                                                : Mma<E>::szero();
#pragma unroll
      for (int r = 0; r < 4; ++r) o.g[t][r] = Gj[rt * 16 + acc_row(r)];
    }
    read_kv(dstates(j), o.add);
    const float* ip = inj_tile(j);
    o.has_inj = ip != nullptr;
    if (o.has_inj) read_kv(ip, o.inj);
  };

  // dVn of a step is stored at the start of the step after it, beside dS',
  // ahead of that step's operand loads: the vector memory pipe is in order,
  // so stores issued after the loads would wait for them to drain and hold
  // the wave up mid-step. (M = K = 128 keeps the stores in place: its
  // registers are already short.)
  constexpr bool DEFER = !(K == 128 && M == 128);
  f4 pdv[RPW][CT];
  auto store_dv = [&](int jj, int p, int ct) {
    const int rt = wv + 4 * p;
    const int m0 = rt * 16 + acc_row(0), vl = ct * 16 + acc_col();
    if (a.dVn) {
      float* o = a.dVn + ((size_t)bh * S + jj) * M * V + (size_t)m0 * V + v0 + vl;
#pragma unroll
      for (int r = 0; r < 4; ++r) o[(size_t)r * V] = pdv[p][ct][r];
    }
    if (a.dVnT)
      *reinterpret_cast<f4*>(a.dVnT + (((size_t)bh * S + jj) * V + v0 + vl) * M + m0) = pdv[p][ct];
  };
  auto flush_dv = [&](int jj) {
#pragma unroll
    for (int p = 0; p < RPW; ++p) {
      if (wv + 4 * p < RTV) {
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) store_dv(jj, p, ct);
      }
    }
  };

  Ops nxt;
  if (S > 0) load(S - 1, nxt);
  for (int j = S - 1; j >= 0; --j) {
    const Ops cur = nxt;

    // ---- dS' (and the previous step's dVn) to global, then the next step's
    // operand loads
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      const int g = wv * TPW + i, rt = g / CT, ct = g % CT;
      const int k0 = rt * 16 + acc_row(0), vl = ct * 16 + acc_col();
      float* o = a.dSp + ((size_t)bh * S + j) * K * V + (size_t)k0 * V + v0 + vl;
#pragma unroll
      for (int r = 0; r < 4; ++r) o[(size_t)r * V] = ds[i][r];
    }
    if (DEFER && j + 1 < S) flush_dv(j + 1);
    if (j > 0) load(j - 1, nxt);

    // ---- dS' staged (transposed) as the B operand of Bop dS'
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      const int g = wv * TPW + i, rt = g / CT, ct = g % CT;
      const int k0 = rt * 16 + acc_row(0), vl = ct * 16 + acc_col();
      sdS.put4(vl * LDS_ST + k0, ds[i]);
    }
    lds_barrier();

    // ---- dVn = Bop dS'
#pragma unroll
    for (int p = 0; p < RPW; ++p) {
      const int rt = wv + 4 * p;
      if (rt < RTV) {
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
          f4 acc = f4_zero();
          const int srow = (ct * 16 + (lane & 15)) * LDS_ST + kofs<E>(lane);
#pragma unroll
          for (int s = 0; s < NSK; ++s)
            acc = Mma<E>::mma(acc, cur.bop[p][s], sdS.get(srow + s * KS));
          const int m0 = rt * 16 + acc_row(0), vl = ct * 16 + acc_col();
          sdV.put4(vl * LDS_VN + m0, acc);
          pdv[p][ct] = acc;
          if constexpr (!DEFER) store_dv(j, p, ct);
        }
      }
    }
    lds_barrier();

    // ---- dS = diag(gam) dS' - A^T dVn, then the group's read gradient
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      const int t = i / CT, ct = i % CT;
      f4 acc = f4_zero();
      const int vrow = (ct * 16 + (lane & 15)) * LDS_VN + kofs<E>(lane);
#pragma unroll
      for (int s = 0; s < NSM; ++s) {
        const bool live = !PADM || (s * KS + kofs<E>(lane) < M);
        typename Mma<E>::SFrag fb = Mma<E>::szero();
        if (live) fb = sdV.get(vrow + s * KS);
        acc = Mma<E>::mma(acc, cur.at[t][s], fb);
      }
      f4 add = cur.add[i];
      if (cur.has_inj) add += cur.inj[i];
#pragma unroll
      for (int r = 0; r < 4; ++r) ds[i][r] = cur.g[t][r] * ds[i][r] - acc[r] + add[r];
    }
    // no barrier here: the next step's writes of s_dst follow this step's
    // second barrier, after every read of s_dst, and its writes of s_dvn
    // follow the next step's first barrier, after every read of s_dvn
  }
  if (DEFER && S > 0) flush_dv(0);
  if (a.dinit) {
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      const int g = wv * TPW + i, rt = g / CT, ct = g % CT;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int k = rt * 16 + acc_row(r), v = v0 + ct * 16 + acc_col();
        a.dinit[b * a.di_sb + h * a.di_sh + (long long)k * V + v] = ds[i][r];
      }
    }
  }
}

// ---------------------------------------------------------------- level 0
//
// The reverse scan's matrix-core operands are the transposes of the forward's
// split tiles: Kt = (KtT)^T, Aqk^T, W^T and Qg^T, all read with the
// reduction index contiguous. The scan reads the forward tiles themselves
// and transposes on chip:
//
// bf16 (fragment order): wave w's products read only column slices of the
// tiles: KtT[:, 16w .. +16] (the rows of Kt of its dVn row tile), Aqk[:, 16w
// .. +16], and W, Qg [:, NCW w .. +NCW], NCW = K / 4 (the rows of W^T and Qg^T
// of its state row tiles). In fragment order each 16-row block of such a
// slice is a run of 16 NCW contiguous elements per plane, in 16-byte
// segments (row r, columns 8 cq .. + 7 of the slice). Each wave copies its
// slices' segments (one 16-byte global load and one 16-byte LDS store per
// lane and segment) into a private LDS region and forms the transposed
// fragments with ds_read_b64_tr_b16: in each group of 16 lanes, lane q reads
// 8 bytes, the 4 values at row q / 4 and columns 4 (q % 4) .. + 3 of a 4 x 16
// block, and lane p receives column p of the block (4 consecutive rows).
// With the block's rows the 4 consecutive reduction indices 32 s + 8 (l / 16)
// + 4 h .. + 3 of a k-step and its columns the 16 operand rows of a tile, two
// such reads (h = 0, 1) give a lane the 8 values of its bf16 A fragment. No
// other wave reads a wave's region, so the copy needs no workgroup barrier;
// a wave's LDS accesses run in its program order, which keeps a step's reads
// of the region ahead of the next step's copy into it.
//
// fp32: each operand element is one 4-byte load of the transposed position,
// 16 consecutive lanes reading 64 contiguous bytes.

// Position of segment (r, cq) inside a 16-row run of a wave's copy, NCW / 8
// segments per row: rows r and r + 8 (read by the two 16-lane groups of one
// half-wave) are placed in opposite bank halves.
template <int NCW>
struct Slice {
  static constexpr int NCQ = NCW / 8;         // segments per row
  static constexpr int RUN = 16 * NCQ;        // segments per 16-row run
  static_assert(NCW == 16 || NCW == 32, "slices of 16 or 32 columns");
  __device__ __forceinline__ static int pos(int r, int cq) {
    if constexpr (NCW == 16) return (2 * r + cq) ^ (((r >> 3) & 1) << 3);
    else return 4 * r + (cq ^ (((r >> 3) & 1) << 1));
  }
};

typedef __attribute__((__vector_size__(16))) int R16;
typedef short v4s __attribute__((ext_vector_type(4)));

// The bf16 A fragment of X^T for column tile ctl of a wave's slice of X and
// k-step s (rows 32 s .. + 31 of X), from one plane of the slice's copy.
template <int NCW>
__device__ __forceinline__ bf16x8 tr_frag(const bf16* pl, int ctl, int s) {
  const int l = lane_id();
  bf16x8 f;
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    const int xr = 32 * s + 8 * (l >> 4) + 4 * hh + ((l & 15) >> 2);
    const int cq = 2 * ctl + ((l & 3) >> 1);
    const bf16* p = pl + ((xr >> 4) * Slice<NCW>::RUN + Slice<NCW>::pos(xr & 15, cq)) * 8 + 4 * (l & 1);
    const v4s x = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)(p));
    const bf16x4 y = __builtin_bit_cast(bf16x4, x);
#pragma unroll
    for (int e = 0; e < 4; ++e) f[4 * hh + e] = y[e];
  }
  return f;
}

// Segment i * 64 + lane of one plane of a wave's slice [R][c0 .. c0 + NCW) of
// a fragment-order tile with C columns: its run rb, row r and segment column
// cq. A load instruction covers whole runs (NCW = 32) or two (NCW = 16), and
// its lanes take the segments row by row, so that the LDS stores of a
// quarter-wave are 256 contiguous bytes.
template <int NCW>
__device__ __forceinline__ void seg_of(int i, int& rb, int& r, int& cq) {
  const int l = lane_id();
  if constexpr (NCW == 16) {
    rb = 2 * i + (l >> 5); r = (l & 31) >> 1; cq = l & 1;
  } else {
    rb = i; r = l >> 2; cq = l & 3;
  }
}
template <int R, int NCW>
struct SliceCopy {
  static constexpr int NL = R * NCW / 512;             // loads per plane
  static constexpr int PLANE = (R / 16) * Slice<NCW>::RUN * 8;   // LDS elements per plane
  // 16-byte segments of both planes of the slice of tile X (the chunk's tile
  // as split_at lays it out: R * C elements per plane)
  template <int C>
  __device__ __forceinline__ static void load(const bf16* X, int c0, R16* out) {
#pragma unroll
    for (int pl = 0; pl < 2; ++pl)
#pragma unroll
      for (int i = 0; i < NL; ++i) {
        int rb, r, cq;
        seg_of<NCW>(i, rb, r, cq);
        const int off = pl * R * C + (rb * (C / 32) + c0 / 32) * 512 + (c0 % 32) * 16 + (16 * cq + r) * 8;
        out[pl * NL + i] = *reinterpret_cast<const R16*>(X + off);
      }
  }
  __device__ __forceinline__ static void store(bf16* dst, const R16* in) {
#pragma unroll
    for (int pl = 0; pl < 2; ++pl)
#pragma unroll
      for (int i = 0; i < NL; ++i) {
        int rb, r, cq;
        seg_of<NCW>(i, rb, r, cq);
        *reinterpret_cast<R16*>(dst + pl * PLANE + (rb * Slice<NCW>::RUN + Slice<NCW>::pos(r, cq)) * 8) =
            in[pl * NL + i];
      }
  }
  __device__ __forceinline__ static Mma<bf16>::SFrag frag(const bf16* src, int ctl, int s) {
    return Mma<bf16>::SFrag{tr_frag<NCW>(src, ctl, s), tr_frag<NCW>(src + PLANE, ctl, s)};
  }
};

template <typename E, int K, int BV>
__global__ __launch_bounds__(256) void scan_bwd_l0_kernel(ScanBwdArgs a) {
  constexpr int M = CH;
  constexpr int CT = BV / 16;
  constexpr int RTS = K / 16;
  constexpr int TPW = RTS * CT / 4;           // state tiles per wave
  constexpr int TRT = TPW / CT;               // state row tiles per wave
  constexpr int NCW = 16 * TRT;               // columns of W and Qg a wave reads
  using ST = SplitTile<E>;
  constexpr int LDS_ST = K + ST::PAD;
  constexpr int LDS_VN = M + ST::PAD;
  constexpr int KS = Mma<E>::KS;
  constexpr int NSK = K / KS;
  constexpr int NSM = M / KS;
  constexpr int DOE = M * BV / 256;           // dO elements staged per thread
  constexpr bool BF = std::is_same<E, bf16>::value;
  static_assert(BV % DOE == 0 && 256 / (BV / DOE) == M && DOE % 4 == 0,
                "one token row slice per thread");
  static_assert(TPW % CT == 0 && (NCW == 16 || NCW == 32), "state tiles of a wave in whole rows");
  typedef typename Mma<E>::SFrag SF;
  // dS'^T, dVn^T and (mix_0 dO)^T, split once by their writers
  __shared__ __attribute__((aligned(16))) typename ST::T s_dst[ST::NPLANE * BV * LDS_ST];
  __shared__ __attribute__((aligned(16))) typename ST::T s_dvn[ST::NPLANE * BV * LDS_VN];
  __shared__ __attribute__((aligned(16))) typename ST::T s_dot[ST::NPLANE * BV * LDS_VN];
  const ST sdS{s_dst, BV * LDS_ST}, sdV{s_dvn, BV * LDS_VN}, sdO{s_dot, BV * LDS_VN};
  // bf16: every wave's copy of its slices of KtT, Aqk, W and Qg
  using CK = SliceCopy<K, 16>;
  using CQ = SliceCopy<M, 16>;
  using CW = SliceCopy<M, NCW>;
  constexpr int OPW = 2 * (CK::PLANE + CQ::PLANE + 2 * CW::PLANE);   // elements per wave
  constexpr int NSEG = 2 * (CK::NL + CQ::NL + 2 * CW::NL);           // loads per lane
  __shared__ __attribute__((aligned(16))) bf16 s_op[BF ? 4 * OPW : 8];

  const int V = a.V, S = a.S, H = a.H;
  const int nvt = V / BV;
  int vt, bh;
  xcd_split(blockIdx.x, gridDim.x, nvt, bh, vt);
  const int h = bh % H, b = bh / H;
  const int v0 = vt * BV;
  const int lane = lane_id(), wv = wave_id(), tid = threadIdx.x;
  bf16* const opw = s_op + (BF ? wv * OPW : 0);
  bf16* const oK = opw;
  bf16* const oQ = oK + 2 * CK::PLANE;
  bf16* const oW = oQ + 2 * CQ::PLANE;
  bf16* const oG = oW + 2 * CW::PLANE;

  f4 ds[TPW];
#pragma unroll
  for (int i = 0; i < TPW; ++i) {
    const int g = wv * TPW + i, rt = g / CT, ct = g % CT;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int k = rt * 16 + acc_row(r), v = v0 + ct * 16 + acc_col();
      ds[i][r] = a.d_final ? a.d_final[b * a.df_sb + h * a.df_sh + (long long)k * V + v] : 0.f;
    }
  }
  auto read_kv = [&](const float* src, f4* out) {
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      const int g = wv * TPW + i, rt = g / CT, ct = g % CT;
#pragma unroll
      for (int r = 0; r < 4; ++r)
        out[i][r] = src[(size_t)(rt * 16 + acc_row(r)) * V + v0 + ct * 16 + acc_col()];
    }
  };

  const float* Gb = a.gam + (size_t)bh * S * K;
  const E* dob = static_cast<const E*>(a.dout) + ((size_t)b * a.T * H + h) * V;
  const E* mixb = static_cast<const E*>(a.mix) + ((size_t)b * a.T * H + h) * a.L;
  // the chunk's tile of a [B*H,S,R,C] split tensor
  auto tile = [&](const float* X, int j, int RC) { return X + ((size_t)bh * S + j) * RC; };

  typedef E DV __attribute__((__vector_size__(DOE * sizeof(E))));
  constexpr int FK = BF ? 1 : NSK, FM = BF ? 1 : NSM, FT = BF ? 1 : TRT;
  struct Ops {
    float kt[FK];               // fp32: Kt rows of this wave's dVn tile, transposed reads
    float aq[FM];               // fp32: Aqk^T rows
    float wt[FT][FM];           // fp32: W^T rows of this wave's state tiles
    float qg[FT][FM];           // fp32: Qg^T rows
    float g[TRT][4];
    DV dor;                     // do at this thread's staging slots, raw
    E dm;                       // and mix_0 of its token, raw (converted when staged)
    f4 add[TPW];                // injection of the step
    bool has_add;
  };
  R16 pre[BF ? NSEG : 1];       // bf16: the next step's slice segments, raw
  auto load = [&](int j, Ops& o) {
    if constexpr (BF) {
      const bf16* kt = reinterpret_cast<const bf16*>(tile(a.KtT, j, K * M));
      const bf16* aq = reinterpret_cast<const bf16*>(tile(a.Aqk, j, M * M));
      const bf16* wq = reinterpret_cast<const bf16*>(tile(a.W, j, M * K));
      const bf16* qq = reinterpret_cast<const bf16*>(tile(a.Qg, j, M * K));
      CK::template load<M>(kt, 16 * wv, pre);
      CQ::template load<M>(aq, 16 * wv, pre + 2 * CK::NL);
      CW::template load<K>(wq, NCW * wv, pre + 2 * (CK::NL + CQ::NL));
      CW::template load<K>(qq, NCW * wv, pre + 2 * (CK::NL + CQ::NL + CW::NL));
    } else {
      // element (row tile rt of X^T, k = 4 s + lane / 16) = X[4 s + lane / 16][16 rt + lane % 16]
      const float* kt = tile(a.KtT, j, K * M);
      const float* aq = tile(a.Aqk, j, M * M);
      const float* wq = tile(a.W, j, M * K);
      const float* qq = tile(a.Qg, j, M * K);
      const int lr = lane >> 4, lc = lane & 15;
#pragma unroll
      for (int s = 0; s < FK; ++s) o.kt[s] = kt[(4 * s + lr) * M + 16 * wv + lc];
#pragma unroll
      for (int s = 0; s < FM; ++s) o.aq[s] = aq[(4 * s + lr) * M + 16 * wv + lc];
#pragma unroll
      for (int t = 0; t < FT; ++t)
#pragma unroll
        for (int s = 0; s < FM; ++s) {
          o.wt[t][s] = wq[(4 * s + lr) * K + NCW * wv + 16 * t + lc];
          o.qg[t][s] = qq[(4 * s + lr) * K + NCW * wv + 16 * t + lc];
        }
    }
    const float* Gj = Gb + (size_t)j * K;
#pragma unroll
    for (int t = 0; t < TRT; ++t) {
      const int rt = wv * TRT + t;
#pragma unroll
      for (int r = 0; r < 4; ++r) o.g[t][r] = Gj[rt * 16 + acc_row(r)];
    }
    // DOE consecutive columns of one token per thread: one vector load
    const int c = tid / (BV / DOE), vl = (tid % (BV / DOE)) * DOE, t = j * M + c;
    if (t < a.T) {
      o.dor = *reinterpret_cast<const DV*>(dob + (size_t)t * H * V + v0 + vl);
      o.dm = mixb[(size_t)t * H * a.L];
    } else {
      o.dor = DV{};
      o.dm = E(0.f);
    }
    o.has_add = a.inj && (j + 1) % a.inj_every == 0 && (j + 1) / a.inj_every <= a.inj_nf;
    if (o.has_add) read_kv(a.inj + ((size_t)bh * a.inj_nf + (j + 1) / a.inj_every - 1) * K * V, o.add);
  };
  // the operand fragments of the current step
  auto f_kt = [&](const Ops& o, int s) -> SF {
    if constexpr (BF) return CK::frag(oK, 0, s); else return o.kt[s];
  };
  auto f_aq = [&](const Ops& o, int s) -> SF {
    if constexpr (BF) return CQ::frag(oQ, 0, s); else return o.aq[s];
  };
  auto f_wt = [&](const Ops& o, int t, int s) -> SF {
    if constexpr (BF) return CW::frag(oW, t, s); else return o.wt[t][s];
  };
  auto f_qg = [&](const Ops& o, int t, int s) -> SF {
    if constexpr (BF) return CW::frag(oG, t, s); else return o.qg[t][s];
  };

  // dVn of a step, stored after the step's dVn products
  f4 pdv[CT];
  auto flush_dv = [&](int jj) {
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      const int m0 = wv * 16 + acc_row(0), vl = ct * 16 + acc_col();
      if (a.dVn) {
        float* o = a.dVn + ((size_t)bh * S + jj) * M * V + (size_t)m0 * V + v0 + vl;
#pragma unroll
        for (int r = 0; r < 4; ++r) o[(size_t)r * V] = pdv[ct][r];
      }
      if (a.dVnT)
        *reinterpret_cast<f4*>(a.dVnT + (((size_t)bh * S + jj) * V + v0 + vl) * M + m0) = pdv[ct];
    }
  };

  Ops nxt;
  // steps [j0, j1) in reverse, from the state gradient after step j1 - 1
  const int j0 = a.j0, j1 = a.j1 > 0 ? a.j1 : S;
  if (j1 > j0) load(j1 - 1, nxt);
  for (int j = j1 - 1; j >= j0; --j) {
    // ---- this step's slices into the wave's region (bf16; the previous
    // step's reads of the region were issued before, in this wave's order)
    if constexpr (BF) {
      CK::store(oK, pre);
      CQ::store(oQ, pre + 2 * CK::NL);
      CW::store(oW, pre + 2 * (CK::NL + CQ::NL));
      CW::store(oG, pre + 2 * (CK::NL + CQ::NL + CW::NL));
    }
    const Ops cur = nxt;
    if (cur.has_add) {
#pragma unroll
      for (int i = 0; i < TPW; ++i) ds[i] += cur.add[i];
    }

    // ---- the next step's operand loads (the last step reloads its own, so
    // that no branch guards them); this step's dS' and dVn are stored after
    // its dVn products, while those loads are in flight
    load(j > j0 ? j - 1 : j0, nxt);

    // ---- dS' and mix_0 dO staged (transposed) as B operands
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      const int g = wv * TPW + i, rt = g / CT, ct = g % CT;
      const int k0 = rt * 16 + acc_row(0), vl = ct * 16 + acc_col();
      sdS.put4(vl * LDS_ST + k0, ds[i]);
    }
    {
      const int c = tid / (BV / DOE), vl = (tid % (BV / DOE)) * DOE;
      const float m = to_f(cur.dm);
#pragma unroll
      for (int q = 0; q < DOE; ++q) sdO.put1((vl + q) * LDS_VN + c, to_f(cur.dor[q]) * m);
    }
    lds_barrier();

    // ---- dVn = Kt dS' + Aqk^T dO on this wave's row tile
    {
      SF fk[NSK], fq[NSM];
#pragma unroll
      for (int s = 0; s < NSK; ++s) fk[s] = f_kt(cur, s);
#pragma unroll
      for (int s = 0; s < NSM; ++s) fq[s] = f_aq(cur, s);
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        f4 acc = f4_zero();
        const int srow = (ct * 16 + (lane & 15)) * LDS_ST + kofs<E>(lane);
#pragma unroll
        for (int s = 0; s < NSK; ++s) acc = Mma<E>::mma(acc, fk[s], sdS.get(srow + s * KS));
        const int orow = (ct * 16 + (lane & 15)) * LDS_VN + kofs<E>(lane);
#pragma unroll
        for (int s = 0; s < NSM; ++s) acc = Mma<E>::mma(acc, fq[s], sdO.get(orow + s * KS));
        const int m0 = wv * 16 + acc_row(0), vl = ct * 16 + acc_col();
        sdV.put4(vl * LDS_VN + m0, acc);
        pdv[ct] = acc;
      }
    }
    lds_barrier();

    // ---- dS' (the state gradient still holds it) and dVn to global
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      const int g = wv * TPW + i, rt = g / CT, ct = g % CT;
      const int k0 = rt * 16 + acc_row(0), vl = ct * 16 + acc_col();
      float* o = a.dSp + ((size_t)bh * S + j) * K * V + (size_t)k0 * V + v0 + vl;
#pragma unroll
      for (int r = 0; r < 4; ++r) o[(size_t)r * V] = ds[i][r];
    }
    flush_dv(j);

    // ---- dS = diag(gam) dS' - W^T dVn + Qg^T dO
#pragma unroll
    for (int t = 0; t < TRT; ++t) {
      SF fw[NSM], fg[NSM];
#pragma unroll
      for (int s = 0; s < NSM; ++s) {
        fw[s] = f_wt(cur, t, s);
        fg[s] = f_qg(cur, t, s);
      }
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        const int i = t * CT + ct;
        f4 acc = f4_zero(), qacc = f4_zero();
        const int vrow = (ct * 16 + (lane & 15)) * LDS_VN + kofs<E>(lane);
#pragma unroll
        for (int s = 0; s < NSM; ++s) {
          acc = Mma<E>::mma(acc, fw[s], sdV.get(vrow + s * KS));
          qacc = Mma<E>::mma(qacc, fg[s], sdO.get(vrow + s * KS));
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) ds[i][r] = cur.g[t][r] * ds[i][r] - acc[r] + qacc[r];
      }
    }
    // s_dot and s_dvn are rewritten by the next step
    lds_barrier();
  }
  if (a.dinit) {
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      const int g = wv * TPW + i, rt = g / CT, ct = g % CT;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int k = rt * 16 + acc_row(r), v = v0 + ct * 16 + acc_col();
        a.dinit[b * a.di_sb + h * a.di_sh + (long long)k * V + v] = ds[i][r];
      }
    }
  }
}

template <typename E, int K, int M, int BV>
static hipError_t launch_scan_bwd_bv(const ScanBwdArgs& a, hipStream_t st) {
  const unsigned grid = (unsigned)(a.B * a.H * (a.V / BV));
  constexpr bool BF = std::is_same<E, bf16>::value;
  if (a.Qg) {
    // level 0: the forward's tiles, in fragment order for bf16
    if constexpr (M == CH) {
      if (a.frag != (BF ? 3 : 0) || !a.W || !a.KtT || !a.Aqk || !a.dout || !a.mix)
        return hipErrorInvalidValue;
      hipLaunchKernelGGL((scan_bwd_l0_kernel<E, K, BV>), dim3(grid), dim3(256), 0, st, a);
      return hipGetLastError();
    }
    return hipErrorInvalidValue;
  }
  constexpr bool CAN = M % 32 == 0 && BF;
  if (a.frag && !(CAN && a.frag == 1)) return hipErrorInvalidValue;
  if (CAN && a.frag == 1)
    hipLaunchKernelGGL((scan_bwd_kernel<E, K, M, CAN, BV>), dim3(grid), dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((scan_bwd_kernel<E, K, M, false, BV>), dim3(grid), dim3(256), 0, st, a);
  return hipGetLastError();
}

template <typename E, int K, int M>
static hipError_t launch_scan_bwd(const ScanBwdArgs& a, hipStream_t st) {
  // few (batch, head) pairs: the bf16 reverse scans take 16-column slices,
  // as the forward scans do
  if constexpr (std::is_same<E, bf16>::value) {
    if (a.B * a.H * (a.V / SCAN_BV) <= SCAN_NARROW_GRID) return launch_scan_bwd_bv<E, K, M, 16>(a, st);
  }
  return launch_scan_bwd_bv<E, K, M, SCAN_BV>(a, st);
}

hipError_t scan_bwd(const ScanBwdArgs& a, int dtype, int K, hipStream_t st) {
  if (a.V % SCAN_BV != 0) return hipErrorInvalidValue;
  if (a.Qg && a.M != CH) return hipErrorInvalidValue;
  if (!a.Qg && !a.d_states) return hipErrorInvalidValue;
#define NGDN_SB(E, KK, MM) \
  if (K == KK && a.M == MM) return launch_scan_bwd<E, KK, MM>(a, st);
#define NGDN_SB_K(E, KK) NGDN_SB(E, KK, 16) NGDN_SB(E, KK, 32) NGDN_SB(E, KK, 64) NGDN_SB(E, KK, 128)
  if (dtype == NGDN_BF16) {
    NGDN_SB_K(bf16, 64) NGDN_SB_K(bf16, 128)
  } else {
    NGDN_SB_K(float, 64) NGDN_SB_K(float, 128)
  }
#undef NGDN_SB_K
#undef NGDN_SB
  return hipErrorInvalidValue;
}

}  // namespace ngdn
