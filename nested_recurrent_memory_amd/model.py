"""NestedGDN2 language model without fla: the reference's
``nested_gdn2/models`` (configuration_nested_gdn2.py, modeling_nested_gdn2.py)
on this package's layer and kernels.

Same config fields and validation, same module tree and parameter names (a
reference checkpoint's state_dict loads as it is), same forward: embeddings ->
blocks of [RMSNorm -> NestedGDN2Attention -> residual, RMSNorm -> GatedMLP ->
residual] -> RMSNorm -> lm_head, the loss on labels shifted by one with
ignore index -100, through the fused linear cross entropy when training.
Registered with transformers' Auto classes under model_type "nested_gdn2",
as the reference registers itself (nested_gdn2/__init__.py:17-23).

Decoding cache: ``NestedGDN2Cache``, a dict from layer index to the layer's
entry (``recurrent_state`` = (state [B,H,L,K,V] fp32, position [B] int64),
``conv_state`` = fla-layout convolution caches) that also counts the tokens
seen, standing in for fla's ``Cache``.
"""

from __future__ import annotations

import torch
import torch.nn as nn
from transformers import AutoConfig, AutoModel, AutoModelForCausalLM, GenerationMixin
from transformers.configuration_utils import PretrainedConfig
from transformers.modeling_layers import GradientCheckpointingLayer
from transformers.modeling_outputs import BaseModelOutputWithPast, CausalLMOutputWithPast
from transformers.modeling_utils import PreTrainedModel

from .layer import NestedGDN2Attention
from .layer_ops import FusedRMSNormGated, ShortConvolution
from .model_ops import FusedLinearCrossEntropyLoss, GatedMLP, RMSNorm, add_rms_norm, rms_norm

__all__ = ["NestedGDN2Config", "NestedGDN2Cache", "NestedGDN2Block", "NestedGDN2Model",
           "NestedGDN2ForCausalLM", "NestedGDN2PreTrainedModel"]


class NestedGDN2Config(PretrainedConfig):
    """The reference's config (models/configuration_nested_gdn2.py:10-133):
    same fields, defaults and checks."""
    model_type = "nested_gdn2"
    keys_to_ignore_at_inference = ["past_key_values"]

    def __init__(self, vocab_size=32000, hidden_size=1024, num_hidden_layers=12, num_heads=16,
                 head_dim=64, expand_v=1.0, use_short_conv=True, conv_size=4, hidden_ratio=4,
                 intermediate_size=None, hidden_act="swish", fuse_swiglu=True, fuse_norm=True,
                 fuse_cross_entropy=True, use_cache=True, norm_eps=1e-5, initializer_range=0.02,
                 tie_word_embeddings=False, num_levels=2, firing_intervals=(1, 4),
                 n_queries_per_level=(64,), promotion="learned", read_mix="softmax",
                 max_horizon=None, op_chunk_size=64, use_triton=True, **kwargs):
        self.vocab_size = vocab_size
        self.hidden_size = hidden_size
        self.num_hidden_layers = num_hidden_layers
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.expand_v = expand_v
        self.use_short_conv = use_short_conv
        self.conv_size = conv_size
        self.hidden_ratio = hidden_ratio
        self.intermediate_size = intermediate_size
        self.hidden_act = hidden_act
        self.fuse_swiglu = fuse_swiglu
        self.fuse_norm = fuse_norm
        self.fuse_cross_entropy = fuse_cross_entropy
        self.use_cache = use_cache
        self.norm_eps = norm_eps
        self.initializer_range = initializer_range
        self.num_levels = num_levels
        self.firing_intervals = tuple(firing_intervals)
        self.n_queries_per_level = tuple(n_queries_per_level)
        self.promotion = promotion
        self.read_mix = read_mix
        self.max_horizon = max_horizon
        self.op_chunk_size = op_chunk_size
        self.use_triton = use_triton
        if len(self.firing_intervals) != num_levels:
            raise ValueError(f"firing_intervals must have length num_levels={num_levels}, "
                             f"got {len(self.firing_intervals)}")
        if self.firing_intervals[0] != 1:
            raise ValueError(f"firing_intervals[0] must be 1, got {self.firing_intervals[0]}")
        if any(b < a for a, b in zip(self.firing_intervals, self.firing_intervals[1:])):
            raise ValueError(f"firing_intervals must be non-decreasing, got {self.firing_intervals}")
        if max_horizon is not None and max_horizon < 1:
            raise ValueError(f"max_horizon must be >= 1 or None, got {max_horizon}")
        if read_mix not in ("softmax", "sigmoid"):
            raise ValueError(f"read_mix must be 'softmax' or 'sigmoid', got {read_mix!r}")
        if promotion not in ("learned", "merge"):
            raise ValueError(f"promotion must be 'learned' or 'merge', got {promotion!r}")
        if len(self.n_queries_per_level) != num_levels - 1:
            raise ValueError(f"n_queries_per_level must have length num_levels-1={num_levels - 1}, "
                             f"got {len(self.n_queries_per_level)}")
        if use_triton:
            if op_chunk_size != 64:
                raise ValueError(f"op_chunk_size must be 64 on the triton path, got {op_chunk_size}")
            for n in self.n_queries_per_level:
                if n < 16 or n & (n - 1):
                    raise ValueError(f"n_queries_per_level entries must be powers of two >= 16, got {n}")
        super().__init__(tie_word_embeddings=tie_word_embeddings, **kwargs)


class NestedGDN2Cache(dict):
    """Per-layer decoding state keyed by layer index, plus the count of tokens
    seen (``get_seq_length``)."""

    # generate() reads this of any cache it is handed: a recurrent state is
    # updated in place, so a compiled decoding loop would gain nothing
    is_compileable = False

    def __init__(self):
        super().__init__()
        self.seen_tokens = 0

    def get_seq_length(self, layer_idx=0):
        return self.seen_tokens

    @classmethod
    def from_legacy_cache(cls, past_key_values=None):
        cache = cls()
        if past_key_values:
            for i, entry in (past_key_values.items() if isinstance(past_key_values, dict)
                             else enumerate(past_key_values)):
                cache[i] = entry
        return cache


class NestedGDN2Block(GradientCheckpointingLayer):
    """Pre-norm token mixing with a residual, then pre-norm channel mixing
    with a residual (models/modeling_nested_gdn2.py:44-68). A
    GradientCheckpointingLayer: after gradient_checkpointing_enable() a
    training forward keeps only the block's inputs and recomputes the rest in
    the backward (caching is switched off for it, as the base class does)."""

    def __init__(self, config, layer_idx):
        super().__init__()
        # fuse_norm=False: torch's nn.RMSNorm and plain residual adds, as the
        # reference selects (models/modeling_nested_gdn2.py:46); the parameter
        # names are the same either way
        self.fused = config.fuse_norm
        norm = RMSNorm if config.fuse_norm else nn.RMSNorm
        self.attn_norm = norm(config.hidden_size, eps=config.norm_eps)
        self.attn = NestedGDN2Attention(config, layer_idx=layer_idx)
        self.mlp_norm = norm(config.hidden_size, eps=config.norm_eps)
        self.mlp = GatedMLP(hidden_size=config.hidden_size, hidden_ratio=config.hidden_ratio,
                            intermediate_size=config.intermediate_size,
                            hidden_act=config.hidden_act, fuse_swiglu=config.fuse_swiglu)

    def forward(self, hidden_states, residual=None, past_key_values=None, use_cache=False,
                defer_residual=False):
        """Same values as norm -> attn -> add -> norm -> mlp -> add. The norms
        write the dtype their consumers compute in (bf16 under autocast: the
        cast the projections would make) and each residual add runs inside
        the norm after it: the attention's in the second norm; with
        ``residual`` (the previous block's deferred MLP output) the input is
        hidden_states + residual, added inside the first norm; with
        ``defer_residual`` the block returns (h, mlp_out, cache) for the next
        norm to add instead of h + mlp_out."""
        if not self.fused:
            if residual is not None:
                hidden_states = hidden_states + residual
            attn_out, _, past_key_values = self.attn(self.attn_norm(hidden_states),
                                                     past_key_values=past_key_values,
                                                     use_cache=use_cache)
            hidden_states = hidden_states + attn_out
            mlp_out = self.mlp(self.mlp_norm(hidden_states))
            if defer_residual:
                return hidden_states, mlp_out, past_key_values
            return hidden_states + mlp_out, past_key_values
        cdt = (torch.get_autocast_dtype("cuda") if torch.is_autocast_enabled("cuda")
               else hidden_states.dtype)
        an, mn = self.attn_norm, self.mlp_norm
        if residual is None:
            y = rms_norm(hidden_states, an.weight, an.eps, cdt)
        else:
            hidden_states, y = add_rms_norm(hidden_states, residual, an.weight, an.eps, cdt)
        attn_out, _, past_key_values = self.attn(y, past_key_values=past_key_values,
                                                 use_cache=use_cache)
        hidden_states, y = add_rms_norm(hidden_states, attn_out, mn.weight, mn.eps, cdt)
        mlp_out = self.mlp(y)
        if defer_residual:
            return hidden_states, mlp_out, past_key_values
        return hidden_states + mlp_out, past_key_values


class NestedGDN2PreTrainedModel(PreTrainedModel):
    config_class = NestedGDN2Config
    base_model_prefix = "model"
    supports_gradient_checkpointing = True
    _no_split_modules = ["NestedGDN2Block"]

    def _init_weights(self, module):
        """As models/modeling_nested_gdn2.py:74-90: the attention layer keeps
        its own A_log, dt_bias and promotion parameters; linear and
        convolution weights and embeddings ~ N(0, initializer_range)."""
        if isinstance(module, NestedGDN2Attention):
            for p in (module.A_log, module.dt_bias):
                p._no_weight_decay = True
            return
        if isinstance(module, (nn.Linear, nn.Conv1d, ShortConvolution)):
            nn.init.normal_(module.weight, mean=0.0, std=self.config.initializer_range)
            if getattr(module, "bias", None) is not None:
                nn.init.zeros_(module.bias)
        elif isinstance(module, nn.Embedding):
            nn.init.normal_(module.weight, mean=0.0, std=self.config.initializer_range)
        elif isinstance(module, (RMSNorm, nn.RMSNorm, FusedRMSNormGated)):
            nn.init.ones_(module.weight)


class NestedGDN2Model(NestedGDN2PreTrainedModel):
    def __init__(self, config):
        super().__init__(config)
        self.embeddings = nn.Embedding(config.vocab_size, config.hidden_size)
        self.layers = nn.ModuleList(NestedGDN2Block(config, i) for i in range(config.num_hidden_layers))
        self.norm = (RMSNorm if config.fuse_norm else nn.RMSNorm)(config.hidden_size,
                                                                  eps=config.norm_eps)
        self.gradient_checkpointing = False
        self.post_init()

    def get_input_embeddings(self):
        return self.embeddings

    def set_input_embeddings(self, value):
        self.embeddings = value

    def forward(self, input_ids=None, inputs_embeds=None, output_hidden_states=None,
                return_dict=None, past_key_values=None, use_cache=None, **kwargs):
        """models/modeling_nested_gdn2.py:111-161."""
        use_cache = use_cache if use_cache is not None else (
            self.config.use_cache if not self.training else False)
        if (input_ids is None) == (inputs_embeds is None):
            raise ValueError("Pass exactly one of input_ids or inputs_embeds.")
        output_hidden_states = (output_hidden_states if output_hidden_states is not None
                                else self.config.output_hidden_states)
        return_dict = return_dict if return_dict is not None else self.config.return_dict
        hidden_states = self.embeddings(input_ids) if inputs_embeds is None else inputs_embeds
        if use_cache and not isinstance(past_key_values, NestedGDN2Cache):
            past_key_values = NestedGDN2Cache.from_legacy_cache(past_key_values)
        all_hidden_states = () if output_hidden_states else None
        residual = None     # each block's MLP output, added inside the next norm
        for layer in self.layers:
            if output_hidden_states:
                if residual is not None:
                    hidden_states, residual = hidden_states + residual, None
                all_hidden_states += (hidden_states,)
            # the tensors positionally, as checkpointing with use_reentrant
            # needs them
            hidden_states, residual, past_key_values = layer(
                hidden_states, residual, past_key_values=past_key_values, use_cache=use_cache,
                defer_residual=True)
        if use_cache:
            past_key_values.seen_tokens += hidden_states.shape[1]
        if residual is not None and self.config.fuse_norm:
            _, hidden_states = add_rms_norm(hidden_states, residual, self.norm.weight, self.norm.eps)
        else:
            if residual is not None:
                hidden_states = hidden_states + residual
            hidden_states = self.norm(hidden_states)
        if output_hidden_states:
            all_hidden_states += (hidden_states,)
        if not return_dict:
            return tuple(x for x in (hidden_states, past_key_values, all_hidden_states) if x is not None)
        return BaseModelOutputWithPast(last_hidden_state=hidden_states, past_key_values=past_key_values,
                                       hidden_states=all_hidden_states)


class NestedGDN2ForCausalLM(NestedGDN2PreTrainedModel, GenerationMixin):
    _tied_weights_keys = {"lm_head.weight": "model.embeddings.weight"}
    # the recurrent state cannot be rewound (no assisted decoding)
    _is_stateful = True

    @classmethod
    def _supports_default_dynamic_cache(cls):
        """generate() does not build a key/value cache: the first forward
        returns a NestedGDN2Cache and the later steps pass it back (the
        reference's FLAUnsupportedCacheGenerationMixin, imported by
        models/modeling_nested_gdn2.py:15)."""
        return False

    def __init__(self, config):
        super().__init__(config)
        self.model = NestedGDN2Model(config)
        self.vocab_size = config.vocab_size
        self.lm_head = nn.Linear(config.hidden_size, config.vocab_size, bias=False)
        self.criterion = None
        self.post_init()

    def get_input_embeddings(self):
        return self.model.embeddings

    def set_input_embeddings(self, value):
        self.model.embeddings = value

    def get_output_embeddings(self):
        return self.lm_head

    def set_output_embeddings(self, value):
        self.lm_head = value

    def prepare_inputs_for_generation(self, input_ids, past_key_values=None, use_cache=True, **kwargs):
        """The whole prompt on the first call, only the new tokens after
        (models/modeling_nested_gdn2.py:184-199)."""
        seen = past_key_values.get_seq_length() if past_key_values is not None else 0
        if seen:
            input_ids = input_ids[:, seen:]
        return {"input_ids": input_ids, "past_key_values": past_key_values, "use_cache": use_cache}

    def forward(self, input_ids=None, attention_mask=None, inputs_embeds=None, labels=None,
                output_hidden_states=None, return_dict=None, past_key_values=None, use_cache=None,
                **kwargs):
        """models/modeling_nested_gdn2.py:201-268. With ``fuse_cross_entropy``
        and labels in training mode the logits are not returned."""
        if attention_mask is not None and not bool(attention_mask.all()):
            raise ValueError("padded batches are not supported; run with batch_size 1 or "
                             "pack sequences to equal length")
        return_dict = return_dict if return_dict is not None else self.config.return_dict
        outputs = self.model(input_ids=input_ids, inputs_embeds=inputs_embeds,
                             output_hidden_states=output_hidden_states, return_dict=True,
                             past_key_values=past_key_values, use_cache=use_cache)
        hidden_states = outputs.last_hidden_state
        fuse = self.config.fuse_cross_entropy and labels is not None and self.training
        logits = None if fuse else self.lm_head(hidden_states)
        loss = None
        if labels is not None:
            labels = torch.cat((labels[..., 1:], labels.new_full((labels.shape[0], 1), -100)), dim=-1)
            if fuse:
                if self.criterion is None:
                    self.criterion = FusedLinearCrossEntropyLoss()
                loss = self.criterion(hidden_states.reshape(-1, self.config.hidden_size),
                                      labels.reshape(-1), self.lm_head.weight, self.lm_head.bias)
            else:
                loss = nn.functional.cross_entropy(logits.reshape(-1, self.vocab_size).float(),
                                                   labels.reshape(-1))
        if not return_dict:
            return tuple(x for x in (loss, logits, outputs.hidden_states) if x is not None)
        return CausalLMOutputWithPast(loss=loss, logits=logits,
                                      past_key_values=outputs.past_key_values,
                                      hidden_states=outputs.hidden_states)


def _register():
    for fn in (lambda: AutoConfig.register(NestedGDN2Config.model_type, NestedGDN2Config),
               lambda: AutoModel.register(NestedGDN2Config, NestedGDN2Model),
               lambda: AutoModelForCausalLM.register(NestedGDN2Config, NestedGDN2ForCausalLM)):
        try:
            fn()
        except ValueError:      # already registered (the reference's own package, or a reload)
            pass


_register()
