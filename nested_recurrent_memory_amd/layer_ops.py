"""The two modules NestedGDN2Attention takes from fla
(nested_gdn2/layers/nested_gdn2.py:17-18,57-60,100), on the HIP kernels of
libngdn.so (csrc/layer_ops.hip, entry points in include/ngdn.h):

* ``ShortConvolution``: causal depthwise convolution over time with a SiLU,
  y[b,t,d] = silu(sum_{i<W} w[d,0,i] x[b,t-(W-1)+i,d]), as fla's module with
  activation "silu" and no bias. Its cache is fla's: the last W inputs,
  [B,D,W] with the newest last; a cache passed in is updated in place, as
  fla's is, and returned when ``output_final_state``.
* ``FusedRMSNormGated``: y = x / sqrt(mean(x^2) + eps) * weight * sigmoid(g)
  over the last dimension, as fla's module with activation "sigmoid".

Inputs in bfloat16 or float32 run on the kernels as they are; float16 runs in
float32 and returns float16. There is no fallback: without the library (or
on tensors off the GPU) the calls raise.
"""

from __future__ import annotations

import ctypes

import torch
import torch.nn as nn

from . import _lib

__all__ = ["ShortConvolution", "FusedRMSNormGated", "short_conv", "rmsnorm_gated", "gate_prep",
           "fanout"]


def _code(t):
    return _lib.NGDN_BF16 if t.dtype == torch.bfloat16 else _lib.NGDN_F32


def _work(t):
    return t if t.dtype in (torch.bfloat16, torch.float32) else t.float()


def _on_gpu(name, *ts):
    # the kernels take raw device pointers: a host tensor must never reach them
    dev = ts[0].device
    for t in ts:
        if t is not None and (not t.is_cuda or t.device != dev):
            raise ValueError(f"{name}: every tensor must be on one GPU (got {t.device}); "
                             "there is no CPU path")


class _ShortConvFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, cache, act, want_cache):
        B, T, D = x.shape
        W = weight.shape[-1]
        xw = _work(x).contiguous()
        w = weight.reshape(D, W).float().contiguous()
        # a copy: the cache is updated in place below and the backward reads the old one
        c = cache.to(xw.dtype, copy=True).contiguous() if cache is not None else None
        y = torch.empty_like(xw)
        new = xw.new_empty(B, D, W) if (want_cache or cache is not None) else None
        _lib.call("ngdn_short_conv_fwd", _code(xw), B, T, D, W, int(act), _lib.ptr(xw),
                  _lib.ptr(w), _lib.ptr(c), _lib.ptr(y), _lib.ptr(new), _lib.stream_of(xw))
        ctx.save_for_backward(xw, w, c)
        ctx.act, ctx.in_dtype, ctx.w_shape, ctx.w_dtype = act, x.dtype, weight.shape, weight.dtype
        cache_out = None
        if new is not None:
            if cache is not None:          # fla updates a given cache in place
                cache.copy_(new)
                new = cache
            if want_cache:
                cache_out = new
                ctx.mark_non_differentiable(cache_out)
        return y.to(x.dtype), cache_out

    @staticmethod
    def backward(ctx, dy, _dcache):
        xw, w, c = ctx.saved_tensors
        B, T, D = xw.shape
        W = w.shape[1]
        dyw = dy.to(xw.dtype).contiguous()
        dx = torch.empty_like(xw)
        dw = torch.zeros(D, W, device=xw.device, dtype=torch.float32)
        ws = torch.empty(_lib.WPARTS, D * W, device=xw.device, dtype=torch.float32)
        _lib.call("ngdn_short_conv_bwd", _code(xw), B, T, D, W, int(ctx.act), _lib.ptr(xw),
                  _lib.ptr(w), _lib.ptr(c), _lib.ptr(dyw), _lib.ptr(dx), _lib.ptr(dw),
                  _lib.ptr(ws), _lib.stream_of(xw))
        return dx.to(ctx.in_dtype), dw.reshape(ctx.w_shape).to(ctx.w_dtype), None, None, None


def short_conv(x, weight, cache=None, activation=True, output_final_state=False):
    """x [B,T,D]; weight [D,1,W] (or [D,W]); cache [B,D,W] or None (updated
    in place). Returns (y [B,T,D], the new cache [B,D,W] or None)."""
    if x.dim() != 3:
        raise ValueError(f"short_conv: x must be [B,T,D], got {tuple(x.shape)}")
    if weight.shape[0] != x.shape[-1]:
        raise ValueError(f"short_conv: weight {tuple(weight.shape)} does not match D={x.shape[-1]}")
    _on_gpu("short_conv", x, weight, cache)
    W = weight.shape[-1]
    if cache is not None and tuple(cache.shape) != (x.shape[0], x.shape[-1], W):
        raise ValueError(f"short_conv: cache {tuple(cache.shape)}, expected "
                         f"{(x.shape[0], x.shape[-1], W)} ([B,D,W])")
    return _ShortConvFn.apply(x, weight, cache, bool(activation), bool(output_final_state))


class _NormGatedFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, g, weight, eps):
        V = x.shape[-1]
        xw = _work(x).contiguous()
        gw = g.to(xw.dtype).contiguous()
        w = weight.float().contiguous()
        rows = xw.numel() // V
        y = torch.empty_like(xw)
        rstd = torch.empty(rows, device=xw.device, dtype=torch.float32)
        _lib.call("ngdn_rmsnorm_gated_fwd", _code(xw), rows, V, float(eps), _lib.ptr(xw),
                  _lib.ptr(gw), _lib.ptr(w), _lib.ptr(y), _lib.ptr(rstd), _lib.stream_of(xw))
        ctx.save_for_backward(xw, gw, w, rstd)
        ctx.dtypes = (x.dtype, g.dtype, weight.dtype)
        return y.to(x.dtype)

    @staticmethod
    def backward(ctx, dy):
        xw, gw, w, rstd = ctx.saved_tensors
        V = xw.shape[-1]
        rows = xw.numel() // V
        dyw = dy.to(xw.dtype).contiguous()
        dx, dg = torch.empty_like(xw), torch.empty_like(gw)
        dw = torch.zeros(V, device=xw.device, dtype=torch.float32)
        ws = torch.empty(_lib.WPARTS, V, device=xw.device, dtype=torch.float32)
        _lib.call("ngdn_rmsnorm_gated_bwd", _code(xw), rows, V, _lib.ptr(xw), _lib.ptr(gw),
                  _lib.ptr(w), _lib.ptr(rstd), _lib.ptr(dyw), _lib.ptr(dx), _lib.ptr(dg),
                  _lib.ptr(dw), _lib.ptr(ws), _lib.stream_of(xw))
        xd, gd, wd = ctx.dtypes
        return dx.to(xd), dg.to(gd), dw.to(wd), None


def rmsnorm_gated(x, g, weight, eps=1e-5):
    """x, g [..., V]; weight [V]. y = x rstd weight sigmoid(g)."""
    if x.shape != g.shape or weight.shape != (x.shape[-1],):
        raise ValueError(f"rmsnorm_gated: x {tuple(x.shape)}, g {tuple(g.shape)}, "
                         f"weight {tuple(weight.shape)}")
    _on_gpu("rmsnorm_gated", x, g, weight)
    return _NormGatedFn.apply(x, g, weight, eps)


class _GatePrepFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, f, bz, wz, ml, A_log, dt_bias, L, H, K, V, cap, sigmoid_mix):
        B, T = q.shape[:2]
        wd = q.dtype if q.dtype in (torch.bfloat16, torch.float32) else torch.float32
        ins = [t.to(wd).contiguous() for t in (q, k, f, bz, wz, ml)]
        pd = A_log.dtype if A_log.dtype in (torch.bfloat16, torch.float32) else torch.float32
        A, dt = A_log.to(pd).contiguous(), dt_bias.to(pd).contiguous()
        dev = q.device
        qn = torch.empty(B, T, H, L, K, device=dev, dtype=wd)
        kn = torch.empty(B, T, H, K, device=dev, dtype=wd)
        g0 = torch.empty(B, T, H, K, device=dev, dtype=torch.float32)
        b0 = torch.empty(B, T, H, K, device=dev, dtype=wd)
        w0 = torch.empty(B, T, H, V, device=dev, dtype=wd)
        mix = torch.empty(B, T, H, L, device=dev, dtype=wd)
        ga = _gate_args(B * T, H, L, K, V, pd, sigmoid_mix, cap, ins, A, dt)
        for n, t in zip(("qn", "kn", "g0", "b0", "w0", "mix"), (qn, kn, g0, b0, w0, mix)):
            setattr(ga, n, t.data_ptr())
        _lib.call("ngdn_gate_prep_fwd", _code(qn), ctypes.byref(ga), _lib.stream_of(qn))
        ctx.save_for_backward(*ins, A, dt)
        ctx.cfg = (L, H, K, V, cap, sigmoid_mix)
        ctx.dtypes = [t.dtype for t in (q, k, f, bz, wz, ml, A_log, dt_bias)]
        return qn, kn, g0, b0, w0, mix

    @staticmethod
    def backward(ctx, dqn, dkn, dg0, db0, dw0, dmix):
        *ins, A, dt = ctx.saved_tensors
        L, H, K, V, cap, sigmoid_mix = ctx.cfg
        q = ins[0]
        B, T = q.shape[:2]
        wd, dev = q.dtype, q.device

        def grad(g, shape, dtype):
            return (g.to(dtype).contiguous() if g is not None
                    else torch.zeros(shape, device=dev, dtype=dtype))
        outs = [grad(dqn, (B, T, H, L, K), wd), grad(dkn, (B, T, H, K), wd),
                grad(dg0, (B, T, H, K), torch.float32), grad(db0, (B, T, H, K), wd),
                grad(dw0, (B, T, H, V), wd), grad(dmix, (B, T, H, L), wd)]
        dins = [torch.empty_like(t) for t in ins]
        dpar = torch.zeros(H * K + H, device=dev, dtype=torch.float32)
        ws = torch.empty(_lib.WPARTS, H * K + H, device=dev, dtype=torch.float32)
        ga = _gate_args(B * T, H, L, K, V, A.dtype, sigmoid_mix, cap, ins, A, dt)
        for n, t in zip(("dqn", "dkn", "dg0", "db0", "dw0", "dmix"), outs):
            setattr(ga, n, t.data_ptr())
        for n, t in zip(("dq", "dk", "df", "dbz", "dwz", "dml"), dins):
            setattr(ga, n, t.data_ptr())
        ga.dpar, ga.ws = dpar.data_ptr(), ws.data_ptr()
        _lib.call("ngdn_gate_prep_bwd", _code(q), ctypes.byref(ga), _lib.stream_of(q))
        dt_d, A_d = ctx.dtypes[7], ctx.dtypes[6]
        res = [d.to(t) for d, t in zip(dins, ctx.dtypes[:6])]
        return (*res, dpar[H * K:].to(A_d), dpar[:H * K].to(dt_d),
                None, None, None, None, None, None)


class _Fanout(torch.autograd.Function):
    """x cast once to the autocast dtype for n consumers (aliases of one
    tensor); their gradients summed in fp32 and returned in x's dtype. The
    same values and the same fp32 sum as n autocast casts of x, without the
    n casts forward, n casts back and n - 1 separate additions."""

    @staticmethod
    def forward(ctx, x, n, dtype):
        ctx.xdtype = x.dtype
        y = x.to(dtype)
        return tuple(y.view_as(y) for _ in range(n))

    @staticmethod
    def backward(ctx, *grads):
        gs = [g.contiguous() for g in grads if g is not None]
        if not gs:
            return None, None, None
        dt = gs[0].dtype
        if (len(gs) > 8 or any(g.dtype != dt for g in gs) or dt not in (torch.bfloat16, torch.float32)
                or gs[0].numel() % 8):
            acc = gs[0].float()
            for g in gs[1:]:
                acc.add_(g)
        else:       # one pass over every gradient (ngdn_sum_f32)
            acc = torch.empty(gs[0].shape, device=gs[0].device, dtype=torch.float32)
            ptrs = (ctypes.c_void_p * len(gs))(*[g.data_ptr() for g in gs])
            _lib.call("ngdn_sum_f32", _code(gs[0]), len(gs), ptrs, acc.numel(), _lib.ptr(acc),
                      _lib.stream_of(acc))
        return acc.to(ctx.xdtype), None, None


def fanout(x, n):
    """n inputs for n linear maps of x: under autocast with x in fp32, one
    cast shared (see _Fanout); otherwise x itself, n times."""
    if (x.is_cuda and x.dtype == torch.float32 and torch.is_autocast_enabled("cuda")
            and torch.get_autocast_dtype("cuda") != torch.float32):
        return _Fanout.apply(x, n, torch.get_autocast_dtype("cuda"))
    return (x,) * n


def _gate_args(BT, H, L, K, V, pd, sigmoid_mix, cap, ins, A, dt):
    ga = _lib.GateArgs()
    ga.BT, ga.H, ga.L, ga.K, ga.V = BT, H, L, K, V
    ga.param_dtype = _lib.NGDN_BF16 if pd == torch.bfloat16 else _lib.NGDN_F32
    ga.sigmoid_mix, ga.cap = int(sigmoid_mix), float(cap)
    for n, t in zip(("q", "k", "f", "bz", "wz", "ml"), ins):
        setattr(ga, n, t.data_ptr())
    ga.A_log, ga.dt_bias = A.data_ptr(), dt.data_ptr()
    return ga


def gate_prep(q, k, f, bz, wz, ml, A_log, dt_bias, L, H, K, V, max_horizon=None,
              sigmoid_mix=False):
    """The layer's prologue (layers/nested_gdn2.py:134-166) in one kernel:
    q [B,T,L*H*K] and k [B,T,H*K] (after the convolution), f = f_proj x
    [B,T,H*K], bz = b_proj x, wz = w_proj x, ml = mix_proj x [B,T,H*L].
    Returns qn [B,T,H,L,K], kn [B,T,H,K] (L2-normalised), g0 [B,T,H,K] fp32
    (-exp(A_log) softplus(f + dt_bias), clamped at -1/max_horizon), b0, w0
    (sigmoid) and mix [B,T,H,L] (softmax over levels, or sigmoid)."""
    _on_gpu("gate_prep", q, k, f, bz, wz, ml, A_log, dt_bias)
    B, T = q.shape[:2]
    want = {"q": (B, T, L * H * K), "k": (B, T, H * K), "f": (B, T, H * K),
            "bz": (B, T, H * K), "wz": (B, T, H * V), "ml": (B, T, H * L)}
    for (n, shape), t in zip(want.items(), (q, k, f, bz, wz, ml)):
        if tuple(t.shape) != shape:
            raise ValueError(f"gate_prep: {n} {tuple(t.shape)}, expected {shape}")
    cap = -1.0 / max_horizon if max_horizon else float("inf")
    return _GatePrepFn.apply(q, k, f, bz, wz, ml, A_log, dt_bias, L, H, K, V, cap,
                             bool(sigmoid_mix))


class ShortConvolution(nn.Module):
    """fla's ``ShortConvolution(hidden_size, kernel_size, activation="silu")``
    (no bias): parameter ``weight`` [D,1,W] as nn.Conv1d holds it."""

    def __init__(self, hidden_size, kernel_size, activation="silu", bias=False):
        super().__init__()
        if bias:
            raise ValueError("ShortConvolution: bias is not supported (the layer builds it without)")
        if activation not in ("silu", "swish", None):
            raise ValueError(f"ShortConvolution: activation {activation!r}")
        self.hidden_size, self.kernel_size = hidden_size, kernel_size
        self.activation = activation
        self.weight = nn.Parameter(torch.empty(hidden_size, 1, kernel_size))
        nn.init.kaiming_uniform_(self.weight, a=5 ** 0.5)   # nn.Conv1d's default

    def forward(self, x, cache=None, output_final_state=False):
        return short_conv(x, self.weight, cache, self.activation is not None, output_final_state)


class FusedRMSNormGated(nn.Module):
    """fla's ``FusedRMSNormGated(hidden_size, activation="sigmoid", eps)``:
    parameter ``weight`` [V] (ones at init)."""

    def __init__(self, hidden_size, activation="sigmoid", eps=1e-5):
        super().__init__()
        if activation != "sigmoid":
            raise ValueError(f"FusedRMSNormGated: activation {activation!r} (the layer uses sigmoid)")
        self.hidden_size, self.eps = hidden_size, eps
        self.weight = nn.Parameter(torch.ones(hidden_size))

    def forward(self, x, g):
        return rmsnorm_gated(x, g, self.weight, self.eps)
