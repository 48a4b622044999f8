"""Chunkwise nested Gated DeltaNet on MI355X: the drop-in for the reference's
``nested_gdn2.ops.chunk.chunk_nested_gdn2`` (nested_gdn2/ops/chunk.py:722-766).

Same signature, argument conventions, errors and autograd contract as the
reference op; every arithmetic step runs in the HIP kernels of libngdn.so
(``csrc/``), reached through its C ABI. Python only validates, allocates
outputs and working buffers, and sequences the launches on torch's current
stream. There is no CPU or PyTorch fallback: without the built library or a
GPU the op raises.

Forward, per call (reference composition ops/chunk.py:159-304):
  ngdn_l0_intra_fwd    per-chunk level-0 terms, all chunks in parallel
  ngdn_l0_scan_fwd     level-0 state recurrence, states h per chunk
  for each level l >= 1:
    ngdn_probe_fwd       probe the level below at this level's firings
    ngdn_upper_scan_fwd  this level's write scan, one state per group
  ngdn_output_fwd      level-0 read + every upper read + mix, o written once
"""

from __future__ import annotations

import ctypes
import math

import torch

from . import _lib
from .schedule import n_firings, n_groups

__all__ = ["chunk_nested_gdn2", "ChunkNestedGDN2Function", "PROMOTIONS"]

PROMOTIONS = ("learned", "merge")
_SUPPORTED_KV = (64, 128)


def _as_ints(x, n):
    vals = [int(v) for v in (x.tolist() if torch.is_tensor(x) else list(x))]
    if len(vals) != n:
        raise ValueError(f"expected {n} entries, got {len(vals)}")
    return vals


def _working_dtype(q):
    if q.dtype == torch.bfloat16:
        return torch.bfloat16, _lib.NGDN_BF16
    # fp32 and fp16 run the fp32 kernels (fp16 -> fp32 is exact)
    return torch.float32, _lib.NGDN_F32


def _validate(q, k, v, L, chunk_size, promotion, n_queries, intervals, query_banks):
    if chunk_size != 64:
        raise ValueError(f"chunk_size must be 64 for GDN-2, got {chunk_size}")
    if promotion not in PROMOTIONS:
        raise ValueError(f"unknown promotion {promotion!r}; expected one of {PROMOTIONS}")
    if q.dim() != 5 or q.shape[3] != L:
        raise ValueError(f"q must be [B, T, H, L={L}, K], got {tuple(q.shape)}")
    B, T, H, _, K = q.shape
    V = v.shape[-1]
    if k.shape != (B, T, H, K) or v.shape[:3] != (B, T, H):
        raise ValueError("k must be [B, T, H, K] and v [B, T, H, V] matching q")
    if K not in _SUPPORTED_KV or V not in _SUPPORTED_KV:
        raise ValueError(f"head dims K={K}, V={V} unsupported; K and V must be 64 or 128")
    if L > 1 and K != V:
        raise ValueError(f"promotion needs K == V, got K={K}, V={V}")
    if L > 8:
        raise ValueError(f"at most 8 levels supported, got L={L}")
    if intervals[0] != 1:
        raise ValueError(f"firing_intervals[0] must be 1, got {intervals[0]}")
    if any(f <= 0 for f in intervals):
        raise ValueError(f"firing intervals must be positive, got {intervals}")
    for lvl in range(1, L):
        n = K if promotion == "merge" else n_queries[lvl - 1]
        if n < 16 or n & (n - 1) or n > 128:
            raise ValueError(f"pairs per firing must be a power of two >= 16, got {n}")
        if promotion == "learned" and n > query_banks.shape[2]:
            raise ValueError(
                f"n_queries={n} exceeds the {query_banks.shape[2]} rows of query_banks")


def _forward(q, k, v, g, b, w, mix, qb, kp, bp, wp, gp, nq, f, L, scale,
             init, promotion):
    """Runs the forward kernels. Returns (o, final_state [B,H,L,K,V] fp32,
    saved working tensors)."""
    B, T, H, _, K = q.shape
    V = v.shape[-1]
    dev = q.device
    wd, code = _working_dtype(q)
    NT = -(-T // 64)
    cvt = lambda x: x.to(wd).contiguous()  # noqa: E731
    q_, k_, v_, b_, w_, mix_ = (cvt(x) for x in (q, k, v, b, w, mix))
    g_ = g.to(torch.float32).contiguous()
    init_ = init.to(torch.float32).contiguous() if init is not None else None
    d = _lib.dims(B, T, H, L, K, V, code, scale)
    st = _lib.stream_of(q_)
    P = _lib.ptr
    e = lambda *s, dt=wd: torch.empty(*s, device=dev, dtype=dt)  # noqa: E731

    W, U, Qg = e(B, H, NT, 64, K), e(B, H, NT, 64, V), e(B, H, NT, 64, K)
    KtT, Aqk = e(B, H, NT, K, 64), e(B, H, NT, 64, 64)
    gam = e(B, H, NT, K, dt=torch.float32)
    _lib.call("ngdn_l0_intra_fwd", ctypes.byref(d), P(q_), P(k_), P(v_), P(g_), P(b_), P(w_),
              P(W), P(U), P(KtT), P(Qg), P(Aqk), P(gam), st)
    hT, vnT = e(B, H, NT, V, K), e(B, H, NT, V, 64)
    final = torch.empty(B, H, L, K, V, device=dev, dtype=torch.float32)
    _lib.call("ngdn_l0_scan_fwd", ctypes.byref(d), P(W), P(U), P(KtT), P(gam), P(init_),
              P(hT), P(vnT), P(final), st)

    states = [None] * L
    merge = promotion == "merge"
    if L > 1:
        qb_, kp_ = cvt(qb), cvt(kp)
        bpT = bp.to(wd).transpose(-1, -2).contiguous()
        wpT = wp.to(wd).transpose(-1, -2).contiguous()
        gpT = gp.to(wd).transpose(-1, -2).contiguous()
    for lvl in range(1, L):
        fh, fb = f[lvl], f[lvl - 1]
        nf, ng = n_firings(NT, fh), n_groups(NT, fh)
        N = K if merge else nq[lvl - 1]
        A_ = e(B, H, max(nf, 1), N, K)
        KT_ = e(B, H, max(nf, 1), K, N)
        U_ = e(B, H, max(nf, 1), N, V)
        gm_ = e(B, H, max(nf, 1), K, dt=torch.float32)
        below, ngb = (hT, NT) if lvl == 1 else (states[lvl - 1], n_groups(NT, fb))
        if nf > 0:
            _lib.call("ngdn_probe_fwd", ctypes.byref(d), lvl, int(merge), N, fb, fh,
                      P(below), ngb, P(final), P(qb_), qb_.shape[2], P(kp_),
                      P(bpT), P(wpT), P(gpT), P(A_), P(KT_), P(U_), P(gm_),
                      None, None, None, None, None, st)
        S_l = torch.empty(B, ng, H, K, V, device=dev, dtype=torch.float32)
        _lib.call("ngdn_upper_scan_fwd", ctypes.byref(d), lvl, N, nf, ng, P(A_), P(KT_),
                  P(U_), P(gm_), P(init_), P(S_l), P(final), st)
        states[lvl] = S_l

    o = e(B, T, H, V)
    sp = (ctypes.c_void_p * L)(*([None] + [s.data_ptr() for s in states[1:]]))
    ngs = (ctypes.c_int32 * L)(*([0] + [n_groups(NT, f[l]) for l in range(1, L)]))
    fs = (ctypes.c_int32 * L)(*f)
    _lib.call("ngdn_output_fwd", ctypes.byref(d), P(Qg), P(Aqk), P(hT), P(vnT), P(q_),
              P(mix_), sp, ngs, fs, P(o), None, st)
    saved = dict(W=W, U=U, Qg=Qg, KtT=KtT, Aqk=Aqk, gam=gam, hT=hT, vnT=vnT, states=states)
    return o, final, saved


class ChunkNestedGDN2Function(torch.autograd.Function):
    """Autograd node for the whole op (ops/chunk.py:567-719)."""

    @staticmethod
    def forward(ctx, q, k, v, g, b, w, mix_weights, query_banks, key_projections,
                b_projections, w_projections, g_projections, n_queries_per_level,
                firing_intervals, L, scale, initial_state, output_final_state,
                chunk_size, promotion):
        L = int(L)
        f = _as_ints(firing_intervals, L)
        nq = _as_ints(n_queries_per_level, L - 1) if L > 1 else []
        _validate(q, k, v, L, chunk_size, promotion, nq, f, query_banks)
        if not q.is_cuda:
            raise RuntimeError("chunk_nested_gdn2 runs on the GPU only; got CPU tensors")
        K = q.shape[-1]
        if scale is None:
            scale = K ** -0.5
        o, final, saved = _forward(q, k, v, g, b, w, mix_weights, query_banks,
                                   key_projections, b_projections, w_projections,
                                   g_projections, nq, f, L, scale, initial_state,
                                   promotion)
        o = o.to(q.dtype)
        ctx.meta = (L, scale, f, nq, initial_state is not None, promotion)
        ctx.save_for_backward(q, k, v, g, b, w, mix_weights, query_banks,
                              key_projections, b_projections, w_projections,
                              g_projections, initial_state)
        ctx.saved_fwd = saved
        return o, (final if output_final_state else None)

    @staticmethod
    def backward(ctx, do, dfinal):
        raise NotImplementedError("backward kernels are not built yet")


def chunk_nested_gdn2(q, k, v, g, b, w, mix_weights, query_banks, key_projections,
                      b_projections, w_projections, g_projections, n_queries_per_level,
                      firing_intervals, L, scale=None, initial_state=None,
                      output_final_state=False, chunk_size=64, promotion="learned"):
    """Differentiable chunkwise NestedGDN-2. Signature matches the reference op
    (nested_gdn2/ops/chunk.py:722-743) and its naive twin (ops/naive.py:226-247).

    Returns (o [B, T, H, V] in q's dtype, final_state [B, H, L, K, V] fp32 or None).
    """
    return ChunkNestedGDN2Function.apply(
        q, k, v, g, b, w, mix_weights, query_banks, key_projections, b_projections,
        w_projections, g_projections, n_queries_per_level, firing_intervals, L,
        scale, initial_state, output_final_state, chunk_size, promotion)


def default_scale(K: int) -> float:
    return 1.0 / math.sqrt(K)
