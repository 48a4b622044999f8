"""CPU restatement of the reference's NestedGDN2ForCausalLM -- TEST INFRASTRUCTURE.

This module is the checker, never the product. Only ``tests/`` may import it;
the shipped model (``nested_recurrent_memory_amd.model``) never imports it
and has no CPU fallback.

Plain PyTorch in any float dtype (the tests use float64), from the reference's
``nested_gdn2/models/modeling_nested_gdn2.py``: embeddings, blocks of
[RMSNorm -> layer -> residual, RMSNorm -> SwiGLU MLP -> residual]
(:44-68), final RMSNorm (:97-99,151), lm_head and the mean cross entropy on
labels shifted by one with ignore index -100 (:225-243). The fla modules are
restated by library routines: RMSNorm = ``F.rms_norm``, fla's GatedMLP with
swish = down(silu(gate x) * up x), the fused linear cross entropy =
``F.cross_entropy`` of the full logits. The layer is
``ngdn_layer_oracle.layer_forward``. Pinned in tests/test_model.py: the
uniform-logit loss is log V exactly, the label shift against a per-position
loop, and the residual structure (zero projections leave the embeddings).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

import ngdn_layer_oracle as lref

__all__ = ["model_forward"]


def model_forward(p, input_ids, cfg, labels=None, cache=None):
    """p: the model's state_dict values by name (float64); input_ids [B, T].
    Returns (logits [B,T,V], loss or None, new cache); cache as the layer
    oracle's, a dict from layer index to its entry."""
    d = cfg.hidden_size
    h = p["model.embeddings.weight"][input_ids]
    new_cache = {}
    for i in range(cfg.num_hidden_layers):
        pre = f"model.layers.{i}."
        x = F.rms_norm(h, (d,), p[pre + "attn_norm.weight"], cfg.norm_eps)
        lp = {k[len(pre + "attn."):]: v for k, v in p.items() if k.startswith(pre + "attn.")}
        a, new_cache[i] = lref.layer_forward(lp, x, cfg, None if cache is None else cache[i])
        h = h + a
        x = F.rms_norm(h, (d,), p[pre + "mlp_norm.weight"], cfg.norm_eps)
        gate = x @ p[pre + "mlp.gate_proj.weight"].t()
        up = x @ p[pre + "mlp.up_proj.weight"].t()
        h = h + (F.silu(gate) * up) @ p[pre + "mlp.down_proj.weight"].t()
    h = F.rms_norm(h, (d,), p["model.norm.weight"], cfg.norm_eps)
    logits = h @ p["lm_head.weight"].t()
    loss = None
    if labels is not None:
        shifted = torch.cat((labels[..., 1:], labels.new_full((labels.shape[0], 1), -100)), dim=-1)
        loss = F.cross_entropy(logits.reshape(-1, logits.shape[-1]), shifted.reshape(-1),
                               ignore_index=-100)
    return logits, loss, new_cache
