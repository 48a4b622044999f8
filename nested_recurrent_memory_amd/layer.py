"""NestedGDN2Attention without fla: the reference's token-mixing layer
(nested_gdn2/layers/nested_gdn2.py:27-237) on this package's op, decoding
step and layer kernels.

Same parameters under the same names (so a reference layer's state_dict
loads as it is), same arguments and the same forward:
projections -> ShortConvolution + SiLU (or a plain SiLU) -> per-head L2
normalisation of q and k -> decay g0 = -exp(A_log) softplus(f_proj x + dt_bias)
(clamped at -1/max_horizon when set), gates b0 = sigmoid(b_proj x),
w0 = sigmoid(w_proj x), mix = softmax (or sigmoid) of mix_proj x -> the op
from an aligned position (its partial last chunk firing no upper level, as
the reference's stepped tail does not) and the decoding step from any other
-> FusedRMSNormGated(o, g_proj x) -> o_proj.

The matrix products of the projections are torch.nn.Linear (hipBLASLt); the
convolution, the prologue from the normalisation to the mix (one kernel
forward, one backward), the gated norm, the op and the step are HIP kernels
of libngdn.so.

Cache (``past_key_values``): a dict keyed by ``layer_idx`` whose entries hold
``"recurrent_state": (state [B,H,L,K,V] fp32, position [B] int64)`` (the
reference's format, layers/nested_gdn2.py:190-194,227-234) and
``"conv_state": (q, k, v)`` convolution caches in fla's layout, each
[B, D, conv_size] in the activation dtype (the last conv_size inputs of each
convolution, newest last), updated in place as fla's are.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch
import torch.nn as nn
import torch.nn.functional as F

from .chunk import chunk_nested_gdn2
from .layer_ops import FusedRMSNormGated, ShortConvolution, fanout, gate_prep
from .step import step_nested_gdn2

__all__ = ["NestedGDN2LayerConfig", "NestedGDN2Attention"]


class _nullcontext:
    def __enter__(self):
        return None

    def __exit__(self, *exc):
        return False


class _ForwardOnlyTail(torch.autograd.Function):
    """The stepped tokens' output joined to the graph of ``anchor``: forward
    returns it as is; a backward that carries a nonzero gradient into it
    raises (the decoding step has no backward)."""

    @staticmethod
    def forward(ctx, o, anchor):
        ctx.set_materialize_grads(False)
        return o.clone()

    @staticmethod
    def backward(ctx, grad):
        if grad is None or not bool(grad.ne(0).any()):
            return None, None
        raise RuntimeError("NestedGDN2Attention: a call continuing a cache from a position "
                           "that is not a multiple of the chunk size (64) is stepped, and the "
                           "decoding step has no backward; train from an aligned position")


@dataclass
class NestedGDN2LayerConfig:
    """The fields of the reference's NestedGDN2Config
    (models/configuration_nested_gdn2.py:14-49) that the layer reads, with
    the same defaults."""
    hidden_size: int = 1024
    num_heads: int = 16
    head_dim: int = 64
    expand_v: float = 1.0
    use_short_conv: bool = True
    conv_size: int = 4
    norm_eps: float = 1e-5
    num_levels: int = 2
    firing_intervals: tuple = (1, 4)
    n_queries_per_level: tuple = (64,)
    promotion: str = "learned"
    read_mix: str = "softmax"
    max_horizon: int | None = None
    op_chunk_size: int = 64
    read_levels: tuple | None = field(default=None)


class NestedGDN2Attention(nn.Module):
    def __init__(self, cfg, layer_idx=None):
        super().__init__()
        self.cfg = cfg
        self.layer_idx = layer_idx
        self.L = L = cfg.num_levels
        H, K = cfg.num_heads, cfg.head_dim
        V = int(cfg.head_dim * cfg.expand_v)
        self.H, self.K, self.V = H, K, V
        self.key_dim, self.value_dim = H * K, H * V
        d = cfg.hidden_size
        if len(cfg.firing_intervals) != L or cfg.firing_intervals[0] != 1:
            raise ValueError(f"firing_intervals {cfg.firing_intervals} for {L} levels "
                             "(length L, first entry 1)")
        if len(cfg.n_queries_per_level) != L - 1:
            raise ValueError(f"n_queries_per_level {cfg.n_queries_per_level} for {L} levels")
        if cfg.op_chunk_size != 64:
            raise ValueError(f"op_chunk_size must be 64, got {cfg.op_chunk_size}")
        for n in cfg.n_queries_per_level:
            if n < 16 or n & (n - 1):
                raise ValueError(f"n_queries_per_level entries must be powers of two >= 16, got {n}")

        self.q_proj = nn.Linear(d, L * self.key_dim, bias=False)
        self.k_proj = nn.Linear(d, self.key_dim, bias=False)
        self.v_proj = nn.Linear(d, self.value_dim, bias=False)
        if cfg.use_short_conv:
            self.q_conv1d = ShortConvolution(L * self.key_dim, cfg.conv_size, activation="silu")
            self.k_conv1d = ShortConvolution(self.key_dim, cfg.conv_size, activation="silu")
            self.v_conv1d = ShortConvolution(self.value_dim, cfg.conv_size, activation="silu")
        self.f_proj = nn.Sequential(nn.Linear(d, V, bias=False), nn.Linear(V, self.key_dim, bias=False))
        self.b_proj = nn.Linear(d, self.key_dim, bias=False)
        self.w_proj = nn.Linear(d, self.value_dim, bias=False)
        self.A_log = nn.Parameter(torch.log(torch.empty(H, dtype=torch.float32).uniform_(1, 16)))
        self.A_log._no_weight_decay = True
        dt = torch.exp(torch.rand(self.key_dim, dtype=torch.float32)
                       * (math.log(0.1) - math.log(0.001)) + math.log(0.001)).clamp(min=1e-4)
        self.dt_bias = nn.Parameter(dt + torch.log(-torch.expm1(-dt)))
        self.dt_bias._no_weight_decay = True
        if L > 1:
            self.b_projections = nn.Parameter(torch.randn(L - 1, H, V, K) * V ** -0.5)
            self.w_projections = nn.Parameter(torch.randn(L - 1, H, V, V) * V ** -0.5)
            self.g_projections = nn.Parameter(torch.randn(L - 1, H, V, K) * V ** -0.5)
            n_max = max(cfg.n_queries_per_level)
            if cfg.promotion == "learned":
                self.query_banks = nn.Parameter(torch.randn(L - 1, H, n_max, K) * K ** -0.5)
                self.key_projections = nn.Parameter(torch.randn(L - 1, H, K, V) * V ** -0.5)
            else:
                self.register_buffer("query_banks", torch.zeros(L - 1, H, n_max, K), persistent=False)
                self.register_buffer("key_projections", torch.zeros(L - 1, H, K, V), persistent=False)
        self.n_queries_per_level = tuple(cfg.n_queries_per_level)
        self.firing_intervals = tuple(cfg.firing_intervals)
        self.mix_proj = nn.Linear(d, H * L, bias=False)
        self.g_proj = nn.Sequential(nn.Linear(d, V, bias=False), nn.Linear(V, self.value_dim, bias=True))
        self.o_norm = FusedRMSNormGated(V, activation="sigmoid", eps=cfg.norm_eps)
        self.o_proj = nn.Linear(self.value_dim, d, bias=False)

    def _promo(self, x):
        H, K, V, L = self.H, self.K, self.V, self.L
        if L > 1:
            return dict(query_banks=self.query_banks, key_projections=self.key_projections,
                        b_projections=self.b_projections, w_projections=self.w_projections,
                        g_projections=self.g_projections)
        return dict(query_banks=x.new_empty(0, H, 1, K), key_projections=x.new_empty(0, H, K, V),
                    b_projections=x.new_empty(0, H, V, K), w_projections=x.new_empty(0, H, V, V),
                    g_projections=x.new_empty(0, H, V, K))

    def forward(self, x, past_key_values=None, use_cache=False, **kwargs):
        """Returns (output, None, past_key_values)."""
        B, T, _ = x.shape
        H, K, V, L = self.H, self.K, self.V, self.L
        cfg = self.cfg
        last = past_key_values.get(self.layer_idx) if past_key_values is not None else None
        conv = last.get("conv_state") if last is not None else None
        conv_q, conv_k, conv_v = conv if conv is not None else (None, None, None)
        # x feeds eight linear maps: one autocast cast of it for all of them
        xq, xk, xv, xf, xb, xw, xm, xg = fanout(x, 8)
        if cfg.use_short_conv:
            q, conv_q = self.q_conv1d(self.q_proj(xq), cache=conv_q, output_final_state=use_cache)
            k, conv_k = self.k_conv1d(self.k_proj(xk), cache=conv_k, output_final_state=use_cache)
            v, conv_v = self.v_conv1d(self.v_proj(xv), cache=conv_v, output_final_state=use_cache)
        else:
            q, k, v = (F.silu(p(xi)) for p, xi in ((self.q_proj, xq), (self.k_proj, xk),
                                                    (self.v_proj, xv)))
        v = v.reshape(B, T, H, V)
        # q -> [B,T,H,L,K] and k L2-normalised, the decay g0 (fp32), gates b0,
        # w0 and the level mix, in one kernel (layers/nested_gdn2.py:134-166)
        gated = cfg.read_mix == "sigmoid"
        wd = v.dtype
        q, k, g0, b0, w0, mix = gate_prep(
            q.to(wd), k.to(wd), self.f_proj(xf).to(wd), self.b_proj(xb).to(wd),
            self.w_proj(xw).to(wd), self.mix_proj(xm).to(wd), self.A_log, self.dt_bias,
            L, H, K, V, max_horizon=cfg.max_horizon, sigmoid_mix=gated)
        keep = getattr(cfg, "read_levels", None)   # eval-time read ablation (not a config field)
        if keep is not None:
            masked = torch.zeros_like(mix)
            masked[..., list(keep)] = mix[..., list(keep)]
            mix = masked if gated else masked / masked.sum(-1, keepdim=True)

        promo = dict(self._promo(x), n_queries_per_level=self.n_queries_per_level,
                     firing_intervals=self.firing_intervals, L=L, promotion=cfg.promotion)
        state, position = (last["recurrent_state"] if last is not None
                           else (None, x.new_zeros(B, dtype=torch.long)))
        BT = cfg.op_chunk_size
        # From an aligned position the whole call runs chunkwise, its partial
        # last chunk firing nothing: the reference's composition (whole chunks
        # chunkwise, the rest stepped, the step firing only at a chunk's end,
        # layers/nested_gdn2.py:196-224) in one differentiable op. From an
        # unaligned position every token steps. The position is read back to
        # the host only when it matters: without a cache it is 0, and a call
        # shorter than a chunk with no gradient to carry (a decoding step)
        # steps whatever it is; a host synchronisation per layer would stall
        # the launch queue
        grad = torch.is_grad_enabled() and q.requires_grad
        aligned = last is None or ((T >= BT or grad) and bool((position % BT == 0).all()))
        n_chunked = T if aligned else 0
        parts = []
        if n_chunked:
            o_chunk, state = chunk_nested_gdn2(
                q=q, k=k, v=v, g=g0, b=b0, w=w0, mix_weights=mix, initial_state=state,
                output_final_state=True, chunk_size=BT, fire_partial_chunk=False, **promo)
            parts.append(o_chunk)
            position = position + n_chunked
        elif state is None:
            state = x.new_zeros(B, H, L, K, V, dtype=torch.float32)
        # The step is forward-only: a stepped call that is part of a graph
        # runs on detached values and joins the graph through
        # _ForwardOnlyTail, whose backward raises, so only an actual backward
        # through it fails (the reference's step is differentiable,
        # ops/naive.py:42-134)
        anchor = q if (n_chunked < T and grad) else None
        tail = []
        with torch.no_grad() if anchor is not None else _nullcontext():
            if anchor is not None and state is not None:
                state = state.detach()
            for t in range(n_chunked, T):
                o_t, state = step_nested_gdn2(
                    q[:, t], k[:, t], v[:, t], g0[:, t], b0[:, t], w0[:, t], mix[:, t], state,
                    position, chunk_size=BT, **promo)
                tail.append(o_t.unsqueeze(1))
                position = position + 1
        if tail:
            o_tail = tail[0] if len(tail) == 1 else torch.cat(tail, dim=1)
            parts.append(_ForwardOnlyTail.apply(o_tail, anchor) if anchor is not None else o_tail)
        o = parts[0] if len(parts) == 1 else torch.cat(parts, dim=1)
        if use_cache:
            if past_key_values is None:
                past_key_values = {}
            past_key_values[self.layer_idx] = {
                "recurrent_state": (state, position),
                "conv_state": (conv_q, conv_k, conv_v) if cfg.use_short_conv else None,
            }
        o = self.o_norm(o, self.g_proj(xg).reshape(B, T, H, V))
        return self.o_proj(o.reshape(B, T, H * V)), None, past_key_values
