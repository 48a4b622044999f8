"""CPU checks of the model: the model oracle pinned by closed forms and a
per-position loop, the product model's config checks, parameter names and
Auto registration, and that its kernels refuse host tensors."""

import math

import pytest
import torch
import torch.nn.functional as F

import ngdn_model_oracle as mref
from nested_recurrent_memory_amd.model import (NestedGDN2Config, NestedGDN2ForCausalLM,
                                               NestedGDN2Model)
from nested_recurrent_memory_amd.model_ops import (GatedMLP, fused_linear_cross_entropy,
                                                   rms_norm, swiglu)

D64 = torch.float64


def _tiny(**kw):
    base = dict(vocab_size=64, hidden_size=32, num_hidden_layers=2, num_heads=2, head_dim=16,
                num_levels=2, firing_intervals=(1, 2), n_queries_per_level=(16,),
                intermediate_size=48)
    base.update(kw)
    return NestedGDN2Config(**base)


def _params(model):
    return {k: v.detach().to(D64) for k, v in model.state_dict().items()}


def test_oracle_uniform_logits_give_log_vocab():
    cfg = _tiny()
    torch.manual_seed(0)
    p = _params(NestedGDN2ForCausalLM(cfg))
    p["lm_head.weight"] = torch.zeros_like(p["lm_head.weight"])
    ids = torch.randint(0, cfg.vocab_size, (2, 20))
    _, loss, _ = mref.model_forward(p, ids, cfg, labels=ids)
    assert abs(loss.item() - math.log(cfg.vocab_size)) < 1e-12


def test_oracle_label_shift_matches_per_position_loop():
    cfg = _tiny()
    torch.manual_seed(1)
    p = _params(NestedGDN2ForCausalLM(cfg))
    ids = torch.randint(0, cfg.vocab_size, (2, 20))
    labels = ids.clone()
    labels[0, 5] = -100                       # ignored target of position 4
    logits, loss, _ = mref.model_forward(p, ids, cfg, labels=labels)
    terms = []
    for b in range(2):
        for t in range(19):
            if labels[b, t + 1] != -100:
                lp = torch.log_softmax(logits[b, t], -1)
                terms.append(-lp[labels[b, t + 1]])
    assert abs(loss.item() - torch.stack(terms).mean().item()) < 1e-12


def test_oracle_residual_stream_without_mixing():
    """Zero output projections of the layer and the MLP leave the embeddings:
    the logits are rms_norm(embedding) @ lm_head^T."""
    cfg = _tiny()
    torch.manual_seed(2)
    p = _params(NestedGDN2ForCausalLM(cfg))
    for k in p:
        if k.endswith("attn.o_proj.weight") or k.endswith("mlp.down_proj.weight"):
            p[k] = torch.zeros_like(p[k])
    ids = torch.randint(0, cfg.vocab_size, (1, 9))
    logits, _, _ = mref.model_forward(p, ids, cfg)
    h = F.rms_norm(p["model.embeddings.weight"][ids], (cfg.hidden_size,), p["model.norm.weight"],
                   cfg.norm_eps)
    torch.testing.assert_close(logits, h @ p["lm_head.weight"].t(), rtol=1e-12, atol=1e-12)


def test_config_checks_match_reference():
    with pytest.raises(ValueError, match="firing_intervals must have length"):
        NestedGDN2Config(num_levels=3, firing_intervals=(1, 4))
    with pytest.raises(ValueError, match="non-decreasing"):
        NestedGDN2Config(num_levels=3, firing_intervals=(1, 4, 2), n_queries_per_level=(64, 64))
    with pytest.raises(ValueError, match="powers of two"):
        NestedGDN2Config(n_queries_per_level=(48,))
    with pytest.raises(ValueError, match="read_mix"):
        NestedGDN2Config(read_mix="max")
    assert NestedGDN2Config(use_triton=False, n_queries_per_level=(48,)).n_queries_per_level == (48,)


def test_model_parameter_names_match_reference():
    """Names of the reference's module tree (models/modeling_nested_gdn2.py:
    44-56,93-99,164-170) and fla's GatedMLP / RMSNorm parameters."""
    cfg = _tiny(num_hidden_layers=1)
    names = set(NestedGDN2ForCausalLM(cfg).state_dict())
    want = {"model.embeddings.weight", "model.norm.weight", "lm_head.weight",
            "model.layers.0.attn_norm.weight", "model.layers.0.mlp_norm.weight",
            "model.layers.0.mlp.gate_proj.weight", "model.layers.0.mlp.up_proj.weight",
            "model.layers.0.mlp.down_proj.weight"}
    assert want <= names
    attn = {n for n in names if ".attn." in n}
    assert len(attn) == 23 and "model.layers.0.attn.q_conv1d.weight" in attn
    assert names == want | attn


def test_gated_mlp_intermediate_size_rule():
    assert GatedMLP(1024, hidden_ratio=4).intermediate_size == 2816     # 2730 -> multiple of 256
    assert GatedMLP(1024, intermediate_size=4096).intermediate_size == 4096


def test_init_and_auto_registration():
    from transformers import AutoConfig, AutoModel, AutoModelForCausalLM
    cfg = AutoConfig.for_model("nested_gdn2", vocab_size=64, hidden_size=32, num_hidden_layers=1,
                               num_heads=2, head_dim=16)
    assert isinstance(cfg, NestedGDN2Config)
    m = AutoModelForCausalLM.from_config(cfg)
    assert isinstance(m, NestedGDN2ForCausalLM)
    assert isinstance(AutoModel.from_config(cfg), NestedGDN2Model)
    w = m.model.layers[0].attn.q_proj.weight
    assert abs(w.std().item() - cfg.initializer_range) < 0.005
    assert (m.model.norm.weight == 1).all()


def test_model_ops_refuse_host_tensors():
    with pytest.raises(ValueError, match="no CPU path"):
        rms_norm(torch.randn(2, 64), torch.ones(64))
    with pytest.raises(ValueError, match="no CPU path"):
        swiglu(torch.randn(16), torch.randn(16))
    with pytest.raises(ValueError, match="no CPU path"):
        fused_linear_cross_entropy(torch.randn(4, 8), torch.zeros(4, dtype=torch.long),
                                   torch.randn(16, 8))


def test_save_pretrained_round_trip(tmp_path):
    """save_pretrained / from_pretrained and AutoModelForCausalLM give back the
    same config and parameters (the checkpoint format of the reference:
    config.json with model_type nested_gdn2 + safetensors weights)."""
    import json

    from transformers import AutoModelForCausalLM
    cfg = _tiny(num_levels=3, firing_intervals=(1, 2, 4), n_queries_per_level=(16, 32))
    torch.manual_seed(3)
    m = NestedGDN2ForCausalLM(cfg)
    m.save_pretrained(tmp_path)
    meta = json.loads((tmp_path / "config.json").read_text())
    assert meta["model_type"] == "nested_gdn2" and meta["firing_intervals"] == [1, 2, 4]
    for loaded in (NestedGDN2ForCausalLM.from_pretrained(tmp_path),
                   AutoModelForCausalLM.from_pretrained(tmp_path)):
        assert isinstance(loaded, NestedGDN2ForCausalLM)
        assert loaded.config.firing_intervals == (1, 2, 4)
        sd, sd2 = m.state_dict(), loaded.state_dict()
        assert set(sd) == set(sd2)
        for k in sd:
            assert torch.equal(sd[k], sd2[k]), k


def test_tied_embeddings():
    """tie_word_embeddings shares the embedding matrix with the LM head, as
    the reference declares (_tied_weights_keys, modeling_nested_gdn2.py:165)."""
    m = NestedGDN2ForCausalLM(_tiny(tie_word_embeddings=True))
    assert m.lm_head.weight.data_ptr() == m.model.embeddings.weight.data_ptr()
    untied = NestedGDN2ForCausalLM(_tiny())
    assert untied.lm_head.weight.data_ptr() != untied.model.embeddings.weight.data_ptr()
