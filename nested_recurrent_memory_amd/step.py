"""One decoding token of the nested GDN memory on the GPU.

Drop-in for ``nested_gdn2.ops.naive.naive_step_nested_gdn2``
(nested_gdn2/ops/naive.py:42-134), the step the layer runs for generation
and for a ragged tail after the chunked prefill
(layers/nested_gdn2.py:218-224): same arguments, same return convention
(o in q's dtype, the new state fp32), computed by ``ngdn_step`` of
libngdn.so. Forward only (decoding); there is no CPU path.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from .chunk import PROMOTIONS, _SUPPORTED_KV, _as_ints, _params, _working_dtype, pad_kv

__all__ = ["step_nested_gdn2", "prepare_step_params"]


def prepare_step_params(query_banks, key_projections, b_projections, w_projections,
                        g_projections, dtype):
    """The per-level parameters in the layouts the step's kernels read (the
    bank padded to a multiple of 8 rows, the b/w/g projections transposed),
    for inputs of ``dtype``. A decoding loop prepares them once and passes
    them as ``params=``; they are a snapshot: prepare again after the
    parameters change."""
    wd, _ = _working_dtype(torch.empty(0, dtype=dtype))
    K, V = query_banks.shape[-1], w_projections.shape[-1]
    if K != V:   # laid out for the padded step (pad_kv)
        (query_banks, key_projections, b_projections, w_projections,
         g_projections) = pad_kv(K, V, query_banks=query_banks, key_projections=key_projections,
                                 b_projections=b_projections, w_projections=w_projections,
                                 g_projections=g_projections)[6:11]
    return _params(query_banks, key_projections, b_projections, w_projections,
                   g_projections, wd, False)


def _validate_step(q, k, v, L, chunk_size, promotion, nq, f, query_banks):
    if promotion not in PROMOTIONS:
        raise ValueError(f"unknown promotion {promotion!r}; expected one of {PROMOTIONS}")
    if chunk_size <= 0:
        raise ValueError(f"chunk_size must be positive, got {chunk_size}")
    if q.dim() != 4 or q.shape[2] != L:
        raise ValueError(f"q must be [B, H, L={L}, K], got {tuple(q.shape)}")
    B, H, _, K = q.shape
    V = v.shape[-1]
    if k.shape != (B, H, K) or v.shape[:2] != (B, H):
        raise ValueError("k must be [B, H, K] and v [B, H, V] matching q")
    if K not in _SUPPORTED_KV or V not in _SUPPORTED_KV:
        raise ValueError(f"head dims K={K}, V={V} unsupported; K and V must be 64 or 128")
    if L > 1 and K != V:
        raise ValueError(f"the promotion kernels need K == V, got K={K}, V={V} "
                         "(step_nested_gdn2 pads K != V to max(K, V) before this)")
    if L > 8:
        raise ValueError(f"at most 8 levels supported, got L={L}")
    if any(x <= 0 for x in f):
        raise ValueError(f"firing intervals must be positive, got {f}")
    for lvl in range(1, L):
        n = K if promotion == "merge" else nq[lvl - 1]
        if n < 16 or n & (n - 1) or n > 128:
            raise ValueError(f"pairs per firing must be a power of two >= 16, got {n}")
        if promotion == "learned" and n > query_banks.shape[2]:
            raise ValueError(
                f"n_queries={n} exceeds the {query_banks.shape[2]} rows of query_banks")


def step_nested_gdn2(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    g: torch.Tensor,
    b: torch.Tensor,
    w: torch.Tensor,
    mix_weights: torch.Tensor,
    state: torch.Tensor,
    position: int | torch.Tensor,
    query_banks: torch.Tensor,
    key_projections: torch.Tensor,
    b_projections: torch.Tensor,
    w_projections: torch.Tensor,
    g_projections: torch.Tensor,
    n_queries_per_level,
    firing_intervals,
    L: int,
    scale: float | None = None,
    chunk_size: int = 64,
    promotion: str = "learned",
    *,
    params: dict | None = None,
    inplace: bool = False,
) -> tuple[torch.Tensor, torch.Tensor]:
    """One token: level 0 writes, every level is read and mixed, then each
    level whose firing this token completes promotes, bottom-up
    (ops/naive.py:42-134).

    q [B,H,L,K]; k, g, b [B,H,K]; v, w [B,H,V]; mix_weights [B,H,L];
    state [B,H,L,K,V] (fp32); position: this token's index from 0, an int or
    a [B] tensor when rows sit at different positions (a CUDA tensor keeps
    the firing decision on the GPU: no host synchronisation). Returns o
    [B,H,V] in q's dtype and the new state [B,H,L,K,V] fp32; the state passed
    in is not modified.

    Beyond the reference's arguments: ``params`` takes the output of
    prepare_step_params (else the parameters are laid out on every call), and
    ``inplace=True`` updates ``state`` (fp32, contiguous, on the GPU) in place
    and returns it, which saves writing the upper levels and keeps the buffer
    fixed for graph capture.
    """
    L = int(L)
    K, V = q.shape[-1], v.shape[-1]
    if L > 1 and K != V:
        # the K = V kernels at max(K, V) on zero-padded tensors (pad_kv)
        if promotion == "merge" and K < V:
            raise ValueError(f"merge promotion with K < V (K={K}, V={V}) is not supported: "
                             "its decay is a mean over K pairs")
        if state.shape[-2:] != (K, V):
            raise ValueError(f"state must be [B, H, L, {K}, {V}], got {tuple(state.shape)}")
        padded = pad_kv(K, V, q=q, k=k, v=v, g=g, b=b, w=w, query_banks=query_banks,
                        key_projections=key_projections, b_projections=b_projections,
                        w_projections=w_projections, g_projections=g_projections,
                        state=state.to(torch.float32))
        qp, kp_, vp, gp, bp, wp, qbp, kpp, bpp, wpp, gpp, _, sp = padded
        o, s_new = step_nested_gdn2(
            qp, kp_, vp, gp, bp, wp, mix_weights, sp, position, qbp, kpp, bpp, wpp, gpp,
            n_queries_per_level, firing_intervals, L, K ** -0.5 if scale is None else scale,
            chunk_size, promotion, params=params, inplace=False)
        o, s_new = o[..., :V], s_new[..., :K, :V]
        if inplace:
            state.copy_(s_new)
            return o, state
        return o, s_new.contiguous()
    f = _as_ints(firing_intervals, L)
    nq = _as_ints(n_queries_per_level, L - 1) if L > 1 else []
    _validate_step(q, k, v, L, chunk_size, promotion, nq, f, query_banks)
    if not q.is_cuda:
        raise RuntimeError("step_nested_gdn2 runs on the GPU only; got CPU tensors")
    leaves = (q, k, v, g, b, w, mix_weights, state, query_banks, key_projections,
              b_projections, w_projections, g_projections)
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in leaves):
        raise RuntimeError("step_nested_gdn2 is forward-only (decoding); call it under "
                           "torch.no_grad() or on tensors that do not require grad")
    B, H, _, K = q.shape
    V = v.shape[-1]
    if scale is None:
        scale = K ** -0.5
    dev = q.device
    wd, code = _working_dtype(q)
    cvt = lambda x: x.to(wd).contiguous()  # noqa: E731
    q_, k_, v_, b_, w_, mix_ = (cvt(x) for x in (q, k, v, b, w, mix_weights))
    g_ = g.to(torch.float32).contiguous()
    if state.shape != (B, H, L, K, V):
        raise ValueError(f"state must be [B, H, L, K, V] = {(B, H, L, K, V)}, "
                         f"got {tuple(state.shape)}")
    if inplace:
        if state.dtype != torch.float32 or not state.is_contiguous() or state.device != dev:
            raise ValueError("inplace=True needs a contiguous fp32 state on q's device")
        s_in = s_out = state
    else:
        s_in = state.to(device=dev, dtype=torch.float32).contiguous()
        s_out = torch.empty_like(s_in)
    o = torch.empty(B, H, V, device=dev, dtype=wd)

    pos_t, pos_all = None, 0
    if torch.is_tensor(position) and position.dim() > 0:
        if position.shape != (B,):
            raise ValueError(f"position must be an int or a [B] tensor, got {tuple(position.shape)}")
        pos_t = position.to(device=dev, dtype=torch.int64).contiguous()
    else:
        pos_all = int(position)
        if pos_all < 0:
            raise ValueError(f"position must be >= 0, got {pos_all}")

    merge = promotion == "merge"
    par, ws = {}, None
    P = _lib.ptr
    fs = (ctypes.c_int32 * L)(*f)
    nqs = (ctypes.c_int32 * max(L - 1, 1))(*(nq or [0]))
    if L > 1:
        par = params if params is not None else _params(
            query_banks, key_projections, b_projections, w_projections, g_projections, wd,
            False)
        if par["qb"].dtype != wd:
            raise ValueError(f"params were prepared for {par['qb'].dtype}, inputs are {wd}")
        n_pairs = K if merge else max(nq)
        ws = torch.empty(B * H * (3 * n_pairs * K + K), device=dev, dtype=torch.float32)
    d = _lib.dims(B, 1, H, L, K, V, code, scale)
    _lib.call("ngdn_step", ctypes.byref(d), P(q_), P(k_), P(v_), P(g_), P(b_), P(w_), P(mix_),
              P(s_in), P(s_out), P(pos_t), pos_all, int(chunk_size), fs, int(merge), nqs,
              P(par.get("qb")), par.get("nmax", 0), P(par.get("kp")), P(par.get("bpT")),
              P(par.get("wpT")), P(par.get("gpT")), P(ws), P(o), _lib.stream_of(q_))
    return o.to(q.dtype), s_out
