"""CPU restatement of the reference's NestedGDN2Attention layer -- TEST INFRASTRUCTURE.

This module is the checker, never the product. Only ``tests/`` may import it;
the shipped layer (``nested_recurrent_memory_amd.layer``) never imports it and
has no CPU fallback.

Plain PyTorch on the CPU in any float dtype (the tests use float64), written
from the reference's layer (``nested_gdn2/layers/nested_gdn2.py``) and the
published behaviour of the two fla 0.5.2 modules it uses (fla is not
installed here, so their code is not read or run):

  * ``short_conv``     -- fla ``ShortConvolution(D, W, activation="silu")``
                          without bias: a causal depthwise convolution over
                          time (weight [D,1,W]) followed by SiLU, with fla's
                          cache: the last W inputs, [B,D,W]. Pinned against
                          ``torch.nn.functional.conv1d`` with ``groups=D`` and
                          left padding (a library routine), cache continuation
                          == one pass (tests/test_layer.py).
  * ``rmsnorm_gated``  -- fla ``FusedRMSNormGated(V, activation="sigmoid")``:
                          x / sqrt(mean(x^2) + eps) * weight * sigmoid(g).
                          Pinned against ``torch.nn.functional.rms_norm``.
  * ``layer_forward``  -- the layer's forward (nested_gdn2/layers/
                          nested_gdn2.py:104-237) with the op and step of
                          ``ngdn_oracle``: the composition is restated line by
                          line; its parts are pinned as above and in
                          ``ngdn_oracle``'s own checks.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

import ngdn_oracle as ref

__all__ = ["short_conv", "rmsnorm_gated", "layer_forward"]


def short_conv(x, weight, cache=None, activation=True):
    """x [B,T,D], weight [D,1,W], cache [B,D,W] or None (fla's layout: the
    last W inputs, newest last). Returns (act(conv), new cache [B,D,W])
    (fla ShortConvolution, silu, no bias)."""
    B, T, D = x.shape
    W = weight.shape[-1]
    prev = cache.transpose(1, 2) if cache is not None else x.new_zeros(B, W, D)
    full = torch.cat([prev.to(x.dtype), x], dim=1)         # [B, W+T, D], row W is x[0]
    y = x.new_zeros(B, T, D)
    for i in range(W):
        y = y + weight[:, 0, i] * full[:, 1 + i:1 + i + T]
    if activation:
        y = F.silu(y)
    return y, full[:, T:].transpose(1, 2).contiguous()


def rmsnorm_gated(x, g, weight, eps):
    """fla FusedRMSNormGated with activation "sigmoid"."""
    rstd = torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)
    return x * rstd * weight * torch.sigmoid(g)


def layer_forward(p, x, cfg, cache=None):
    """The layer's forward (nested_gdn2/layers/nested_gdn2.py:104-237).

    p: dict of the layer's parameters by state_dict name; cfg: an object with
    the config fields the layer reads. cache: None or {"recurrent_state":
    (state, position), "conv_state": (q, k, v)}. Returns (o, new cache)."""
    B, T, d = x.shape
    L, H, K = cfg.num_levels, cfg.num_heads, cfg.head_dim
    V = int(cfg.head_dim * cfg.expand_v)
    lin = lambda name, t: t @ p[name].t()   # noqa: E731   (nn.Linear, no bias)
    conv = cache["conv_state"] if cache is not None and cache.get("conv_state") is not None else (None,) * 3
    if cfg.use_short_conv:                                              # :122-130
        q, cq = short_conv(lin("q_proj.weight", x), p["q_conv1d.weight"], conv[0])
        k, ck = short_conv(lin("k_proj.weight", x), p["k_conv1d.weight"], conv[1])
        v, cv = short_conv(lin("v_proj.weight", x), p["v_conv1d.weight"], conv[2])
    else:                                                               # :131-132
        q, k, v = (F.silu(lin(n, x)) for n in ("q_proj.weight", "k_proj.weight", "v_proj.weight"))
        cq = ck = cv = None
    q = q.reshape(B, T, L, H, K).transpose(2, 3)                        # :134
    k = k.reshape(B, T, H, K)
    v = v.reshape(B, T, H, V)
    q = F.normalize(q, dim=-1)                                          # :138-139
    k = F.normalize(k, dim=-1)
    f = lin("f_proj.1.weight", lin("f_proj.0.weight", x))
    g0 = F.softplus(f + p["dt_bias"]).reshape(B, T, H, K)               # :141-143
    g0 = -p["A_log"].exp().unsqueeze(-1) * g0
    if cfg.max_horizon:                                                 # :146-147
        g0 = g0.clamp(max=-1.0 / cfg.max_horizon)
    b0 = torch.sigmoid(lin("b_proj.weight", x)).reshape(B, T, H, K)     # :148-149
    w0 = torch.sigmoid(lin("w_proj.weight", x)).reshape(B, T, H, V)
    logits = lin("mix_proj.weight", x).reshape(B, T, H, L)              # :164-166
    mix = torch.sigmoid(logits) if cfg.read_mix == "sigmoid" else logits.softmax(-1)
    if L > 1:
        promo = [p["query_banks"], p["key_projections"], p["b_projections"],
                 p["w_projections"], p["g_projections"]]
    else:
        promo = [x.new_zeros(0, H, 1, K), x.new_zeros(0, H, K, V), x.new_zeros(0, H, V, K),
                 x.new_zeros(0, H, V, V), x.new_zeros(0, H, V, K)]
    nq, fi = tuple(cfg.n_queries_per_level), tuple(cfg.firing_intervals)
    if cache is not None and cache.get("recurrent_state") is not None:
        state, position = cache["recurrent_state"]
    else:
        state, position = None, torch.zeros(B, dtype=torch.long)
    BT = cfg.op_chunk_size                                              # :195-199
    aligned = bool((position % BT == 0).all())
    n_chunked = (T // BT) * BT if aligned else 0
    parts = []
    if n_chunked:                                                       # :201-214
        o_chunk, state = ref.chunk_forward(
            q[:, :n_chunked], k[:, :n_chunked], v[:, :n_chunked], g0[:, :n_chunked],
            b0[:, :n_chunked], w0[:, :n_chunked], mix[:, :n_chunked], *promo, nq, fi, L=L,
            initial_state=state, output_final_state=True, promotion=cfg.promotion,
            out_dtype=x.dtype)
        parts.append(o_chunk)
        position = position + n_chunked
    elif state is None:
        state = x.new_zeros(B, H, L, K, V)
    for t in range(n_chunked, T):                                       # :216-222
        o_t, state = ref.step_forward(q[:, t], k[:, t], v[:, t], g0[:, t], b0[:, t], w0[:, t],
                                      mix[:, t], state, position, *promo, nq, fi, L=L,
                                      promotion=cfg.promotion)
        parts.append(o_t.unsqueeze(1))
        position = position + 1
    o = parts[0] if len(parts) == 1 else torch.cat(parts, dim=1)
    gg = (lin("g_proj.1.weight", lin("g_proj.0.weight", x)) + p["g_proj.1.bias"]).reshape(B, T, H, V)
    o = rmsnorm_gated(o, gg, p["o_norm.weight"], cfg.norm_eps)          # :236
    out = lin("o_proj.weight", o.reshape(B, T, H * V))
    return out, {"recurrent_state": (state, position), "conv_state": (cq, ck, cv)}
