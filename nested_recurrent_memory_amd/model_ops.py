"""The three modules NestedGDN2ForCausalLM takes from fla
(nested_gdn2/models/modeling_nested_gdn2.py:15-17), on the HIP kernels of
libngdn.so (csrc/model_ops.hip, entry points in include/ngdn.h):

* ``RMSNorm``: y = x / sqrt(mean(x^2) + eps) * weight over the last dimension.
* ``GatedMLP``: down_proj(silu(gate_proj x) * up_proj x), the SwiGLU on a
  kernel, the three projections nn.Linear (hipBLASLt GEMMs), fla's parameter
  names and its intermediate size rule.
* ``FusedLinearCrossEntropyLoss``: mean cross entropy of (x W^T + b) against
  targets with ignore_index, without keeping the logits: the forward forms the
  logits a block of rows at a time, the cross-entropy kernel turns them into
  their gradient in place, and dx, dW (and db) are formed right there; the
  backward only scales them by the incoming gradient.

Under autocast the GEMMs run in the autocast dtype (bfloat16), as
nn.Linear's would; the kernels compute in fp32. There is no fallback: without
the library, or on tensors off the GPU, the calls raise.
"""

from __future__ import annotations

import torch
import torch.nn as nn

from . import _lib
from .layer_ops import fanout

__all__ = ["RMSNorm", "GatedMLP", "FusedLinearCrossEntropyLoss", "rms_norm", "add_rms_norm",
           "swiglu", "fused_linear_cross_entropy"]


def _code(t):
    return _lib.NGDN_BF16 if t.dtype == torch.bfloat16 else _lib.NGDN_F32


def _work(t):
    return t if t.dtype in (torch.bfloat16, torch.float32) else t.float()


def _on_gpu(name, *ts):
    dev = ts[0].device
    for t in ts:
        if t is not None and (not t.is_cuda or t.device != dev):
            raise ValueError(f"{name}: every tensor must be on one GPU (got {t.device}); "
                             "there is no CPU path")


def _compute_dtype(x):
    if torch.is_autocast_enabled("cuda"):
        return torch.get_autocast_dtype("cuda")
    return x.dtype


# ---------------------------------------------------------------- RMSNorm

class _RMSNormFn(torch.autograd.Function):
    """y = RMSNorm(x + r) (r optional) in y's dtype; with r also h = x + r.
    Dtype combinations (x, r, y) run on the kernel: all fp32, all bf16, or
    an fp32 x (a residual stream) with bf16 r and y (bf16 autocast)."""

    @staticmethod
    def forward(ctx, x, r, weight, eps, ydt):
        D = x.shape[-1]
        xw = _work(x).contiguous()
        want = torch.bfloat16 if ydt == torch.bfloat16 else x.dtype
        if xw.dtype == torch.bfloat16:
            rdt = torch.bfloat16                      # all bf16 (r is bf16: add_rms_norm)
        elif want == torch.bfloat16 and (r is None or r.dtype == torch.bfloat16):
            rdt = torch.bfloat16                      # fp32 x, bf16 r and y
        else:
            rdt = torch.float32                       # all fp32 (a bf16 r widens exactly)
        ydt = rdt
        rw = r.to(rdt).contiguous() if r is not None else None
        w = weight.float().contiguous()
        rows = xw.numel() // D
        y = torch.empty(xw.shape, device=xw.device, dtype=ydt)
        h = torch.empty_like(xw) if r is not None else None
        rstd = torch.empty(rows, device=xw.device, dtype=torch.float32)
        c = _lib.NGDN_BF16 if rdt == torch.bfloat16 else _lib.NGDN_F32
        _lib.call("ngdn_add_rmsnorm_fwd", _code(xw), c, c, rows, D, float(eps), _lib.ptr(xw),
                  _lib.ptr(rw), _lib.ptr(w), _lib.ptr(h), _lib.ptr(y), _lib.ptr(rstd),
                  _lib.stream_of(xw))
        ctx.save_for_backward(h if r is not None else xw, w, rstd)
        ctx.codes = (_code(xw), c)
        ctx.dtypes = (x.dtype, r.dtype if r is not None else None, weight.dtype, rdt)
        y = y.to(want)
        if r is None:
            return y
        return h.to(x.dtype), y

    @staticmethod
    def backward(ctx, *grads):
        hx, w, rstd = ctx.saved_tensors
        xd, rd, wd, rdt = ctx.dtypes
        if rd is None:
            dy, dh = grads[0], None
        else:
            dh, dy = grads
        D = hx.shape[-1]
        rows = hx.numel() // D
        dyw = (dy.to(rdt) if dy is not None else torch.zeros(hx.shape, device=hx.device, dtype=rdt)).contiguous()
        dhw = dh.to(hx.dtype).contiguous() if dh is not None else None
        dx = torch.empty_like(hx)
        dr = torch.empty(hx.shape, device=hx.device, dtype=rdt) if (rd is not None and ctx.needs_input_grad[1]) else None
        dw = torch.zeros(D, device=hx.device, dtype=torch.float32)
        ws = torch.empty(_lib.WPARTS, D, device=hx.device, dtype=torch.float32)
        xc, c = ctx.codes
        _lib.call("ngdn_add_rmsnorm_bwd", xc, c, c, rows, D, _lib.ptr(hx), _lib.ptr(w),
                  _lib.ptr(rstd), _lib.ptr(dyw), _lib.ptr(dhw), _lib.ptr(dx), _lib.ptr(dr),
                  _lib.ptr(dw), _lib.ptr(ws), _lib.stream_of(hx))
        return (dx.to(xd), dr.to(rd) if dr is not None else None, dw.to(wd), None, None)


def rms_norm(x, weight, eps=1e-5, out_dtype=None):
    """x [..., D]; weight [D]. y = x rstd weight, in x's dtype, or bf16 when
    out_dtype is bf16 and x fp32 (the cast a bf16 consumer would make)."""
    if weight.shape != (x.shape[-1],):
        raise ValueError(f"rms_norm: x {tuple(x.shape)}, weight {tuple(weight.shape)}")
    _on_gpu("rms_norm", x, weight)
    return _RMSNormFn.apply(x, None, weight, eps, out_dtype)


def add_rms_norm(x, r, weight, eps=1e-5, out_dtype=None):
    """h = x + r and y = RMSNorm(h) weight in one pass: returns (h, y), h in
    x's dtype (a pre-norm block's residual stream: x + sublayer(x) followed
    by the next norm), y as for rms_norm."""
    if weight.shape != (x.shape[-1],) or r.shape != x.shape:
        raise ValueError(f"add_rms_norm: x {tuple(x.shape)}, r {tuple(r.shape)}, weight {tuple(weight.shape)}")
    _on_gpu("add_rms_norm", x, r, weight)
    if (x.dtype, r.dtype) not in _ADD_FORMS:
        h = x + r                  # other dtype pairs: the add on its own, then the norm
        return h, rms_norm(h, weight, eps, out_dtype)
    return _RMSNormFn.apply(x, r, weight, eps, out_dtype)


# (x, r) dtype pairs whose sum keeps x's dtype and runs inside the norm kernel
_ADD_FORMS = {(torch.float32, torch.float32), (torch.float32, torch.bfloat16),
              (torch.bfloat16, torch.bfloat16)}


class RMSNorm(nn.Module):
    """fla's ``RMSNorm(hidden_size, eps)`` (elementwise affine, no bias):
    parameter ``weight`` [D], ones at init."""

    def __init__(self, hidden_size, elementwise_affine=True, bias=False, eps=1e-5):
        super().__init__()
        if not elementwise_affine or bias:
            raise ValueError("RMSNorm: only the affine form without bias (as the model builds it)")
        self.hidden_size, self.eps = hidden_size, eps
        self.weight = nn.Parameter(torch.ones(hidden_size))

    def forward(self, x):
        return rms_norm(x, self.weight, self.eps)


# ---------------------------------------------------------------- SwiGLU MLP

class _SwigluFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, g, u):
        gw = _work(g).contiguous()
        uw = u.to(gw.dtype).contiguous()
        y = torch.empty_like(gw)
        _lib.call("ngdn_swiglu_fwd", _code(gw), gw.numel(), _lib.ptr(gw), _lib.ptr(uw), _lib.ptr(y),
                  _lib.stream_of(gw))
        ctx.save_for_backward(gw, uw)
        ctx.dtypes = (g.dtype, u.dtype)
        return y.to(g.dtype)

    @staticmethod
    def backward(ctx, dy):
        gw, uw = ctx.saved_tensors
        dyw = dy.to(gw.dtype).contiguous()
        dg, du = torch.empty_like(gw), torch.empty_like(uw)
        _lib.call("ngdn_swiglu_bwd", _code(gw), gw.numel(), _lib.ptr(gw), _lib.ptr(uw),
                  _lib.ptr(dyw), _lib.ptr(dg), _lib.ptr(du), _lib.stream_of(gw))
        return dg.to(ctx.dtypes[0]), du.to(ctx.dtypes[1])


def swiglu(g, u):
    """silu(g) * u elementwise (g, u of one shape, numel % 8 == 0)."""
    if g.shape != u.shape or g.numel() % 8:
        raise ValueError(f"swiglu: g {tuple(g.shape)}, u {tuple(u.shape)} (same shape, numel % 8 == 0)")
    _on_gpu("swiglu", g, u)
    return _SwigluFn.apply(g, u)


class GatedMLP(nn.Module):
    """fla's ``GatedMLP`` with hidden_act "swish": parameters
    ``gate_proj``, ``up_proj``, ``down_proj`` (no bias); the intermediate size
    is ``intermediate_size`` or ``hidden_size * hidden_ratio * 2/3`` rounded up
    to a multiple of 256."""

    def __init__(self, hidden_size, hidden_ratio=None, intermediate_size=None,
                 hidden_act="swish", fuse_swiglu=True):
        super().__init__()
        if hidden_act not in ("swish", "silu"):
            raise ValueError(f"GatedMLP: hidden_act {hidden_act!r} (the model uses swish)")
        if hidden_ratio is None:
            hidden_ratio = 4
        if intermediate_size is None:
            intermediate_size = int(hidden_size * hidden_ratio * 2 / 3)
            intermediate_size = 256 * ((intermediate_size + 255) // 256)
        self.hidden_size, self.intermediate_size = hidden_size, intermediate_size
        self.gate_proj = nn.Linear(hidden_size, intermediate_size, bias=False)
        self.up_proj = nn.Linear(hidden_size, intermediate_size, bias=False)
        self.down_proj = nn.Linear(intermediate_size, hidden_size, bias=False)

    def forward(self, x):
        xg, xu = fanout(x, 2)      # one autocast cast of x for both maps
        return self.down_proj(swiglu(self.gate_proj(xg), self.up_proj(xu)))


# ---------------------------------------------------------------- linear + cross entropy

_BLOCK_BYTES = 4 << 30     # logits held at once


class _LinearCEFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, target, weight, bias, ignore_index):
        N, d = x.shape
        V = weight.shape[0]
        cdt = _compute_dtype(x)
        if cdt not in (torch.bfloat16, torch.float32):
            cdt = torch.float32
        xc = x.to(cdt).contiguous()
        wc = weight.to(cdt).contiguous()
        bc = bias.to(cdt) if bias is not None else None
        tgt = target.reshape(-1).to(torch.long).contiguous()
        grad = any(ctx.needs_input_grad[i] for i in (0, 2, 3))
        n_valid = (tgt != ignore_index).sum()
        row_loss = torch.empty(N, device=x.device, dtype=torch.float32)
        dx = torch.empty_like(xc) if grad else None
        dw = db = None
        rows = max(1, min(N, _BLOCK_BYTES // (V * xc.element_size())))
        for r0 in range(0, N, rows):
            r1 = min(N, r0 + rows)
            logits = xc[r0:r1] @ wc.t()
            if bc is not None:
                logits += bc
            _lib.call("ngdn_cross_entropy", _code(logits), r1 - r0, V, int(ignore_index),
                      _lib.ptr(logits), _lib.ptr(tgt[r0:r1]), _lib.ptr(n_valid),
                      _lib.ptr(row_loss[r0:r1]), int(grad), _lib.stream_of(logits))
            if grad:       # logits now hold d(loss)/d(logits)
                dx[r0:r1] = logits @ wc
                part = (logits.t() @ xc[r0:r1]).float()
                dw = part if dw is None else dw.add_(part)
                if bc is not None:
                    pb = logits.float().sum(0)
                    db = pb if db is None else db.add_(pb)
        ctx.dtypes = (x.dtype, weight.dtype, bias.dtype if bias is not None else None)
        if grad:
            ctx.save_for_backward(dx, dw, db)
        return row_loss.sum()

    @staticmethod
    def backward(ctx, dloss):
        dx, dw, db = ctx.saved_tensors
        xd, wd, bd = ctx.dtypes
        gx = (dx * dloss).to(xd) if ctx.needs_input_grad[0] else None
        gw = (dw * dloss).to(wd) if ctx.needs_input_grad[2] else None
        gb = (db * dloss).to(bd) if (db is not None and ctx.needs_input_grad[3]) else None
        return gx, None, gw, gb, None


def fused_linear_cross_entropy(x, target, weight, bias=None, ignore_index=-100):
    """Mean over the targets that are not ignore_index of the cross entropy of
    logits x W^T + b. x [N, d], target [N] (int), weight [V, d], bias [V]."""
    if x.dim() != 2 or weight.dim() != 2 or x.shape[1] != weight.shape[1]:
        raise ValueError(f"fused_linear_cross_entropy: x {tuple(x.shape)}, weight {tuple(weight.shape)}")
    if target.numel() != x.shape[0]:
        raise ValueError(f"fused_linear_cross_entropy: {target.numel()} targets for {x.shape[0]} rows")
    _on_gpu("fused_linear_cross_entropy", x, target, weight, bias)
    return _LinearCEFn.apply(x, target, weight, bias, ignore_index)


class FusedLinearCrossEntropyLoss(nn.Module):
    """fla's ``FusedLinearCrossEntropyLoss()`` as the model calls it
    (reduction "mean", no label smoothing): ``loss(x, target, weight, bias)``."""

    def __init__(self, ignore_index=-100, label_smoothing=0.0, reduction="mean"):
        super().__init__()
        if label_smoothing != 0.0 or reduction != "mean":
            raise ValueError("FusedLinearCrossEntropyLoss: mean reduction without label smoothing only")
        self.ignore_index = ignore_index

    def forward(self, x, target, weight, bias=None):
        return fused_linear_cross_entropy(x, target, weight, bias, self.ignore_index)
