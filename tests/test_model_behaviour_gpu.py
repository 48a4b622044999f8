"""Model-level behaviours the reference's own model tests check, run on this
package's model (the reference's tests need fla and CUDA, so they are
restated here against the same expectations):

* untrained loss near ln(vocab), every parameter gets a finite gradient
  (tests/models/test_modeling.py:38-59);
* the upper levels' decay and erase gates stay dead until the level has two
  read firings, T >= (2 f + 1) 64; the write gate, the bank and the key
  projections never are (tests/models/test_modeling.py:127-154);
* the promotion arms: learned trains the bank and key projections, merge
  keeps them as buffers with no gradient, and the two arms' outputs differ
  (tests/models/test_modeling.py:157-189);
* read ablation (``cfg.read_levels``, an eval-time attribute): keeping every
  level changes nothing, keeping level 0 alone changes a nested model, and
  the chunked and stepped read paths agree under it
  (tests/models/test_read_levels.py:38-75);
* the read mix: sigmoid gates are independent (they may sum past 1),
  softmax weights sum to 1; under ablation the sigmoid arm passes the kept
  gate through unchanged while the softmax arm rescales the survivors to 1
  (tests/models/test_read_mix.py:46-117).
"""

import math

import pytest
import torch

from nested_recurrent_memory_amd import layer as layer_mod
from nested_recurrent_memory_amd.model import NestedGDN2Config, NestedGDN2ForCausalLM

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
VOCAB = 512

CASES = [
    # num_levels, firing_intervals, n_queries_per_level, T
    (1, (1,), (), 256),
    (2, (1, 2), (16,), 384),
    (2, (1, 4), (32,), 640),
    (3, (1, 2, 4), (16, 16), 704),
]
IDS = ["L{}-fire{}-q{}-T{}".format(*c) for c in CASES]


def _config(num_levels, firing, n_queries, **kw):
    return NestedGDN2Config(
        vocab_size=VOCAB, hidden_size=128, num_hidden_layers=2, num_heads=2, head_dim=64,
        num_levels=num_levels, firing_intervals=firing, n_queries_per_level=n_queries,
        fuse_cross_entropy=False, **kw)


def _model(num_levels, firing, n_queries, seed=0, **kw):
    torch.manual_seed(seed)
    return NestedGDN2ForCausalLM(_config(num_levels, firing, n_queries, **kw)).to(DEV)


def _ids(B, T, seed=1):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return torch.randint(0, VOCAB, (B, T), device=DEV, generator=g)


def _set_read_levels(model, keep):
    for m in model.modules():
        if hasattr(m, "cfg") and hasattr(m.cfg, "num_levels"):
            m.cfg.read_levels = keep


def _logits(model, ids, keep):
    _set_read_levels(model, keep)
    with torch.no_grad():
        return model(input_ids=ids).logits


@pytest.mark.parametrize(("num_levels", "firing", "n_queries", "T"), CASES, ids=IDS)
def test_forward_backward_at_init(num_levels, firing, n_queries, T):
    model = _model(num_levels, firing, n_queries)
    ids = _ids(2, T)
    out = model(input_ids=ids, labels=ids)
    assert abs(out.loss.item() - math.log(VOCAB)) < 0.5, out.loss.item()
    assert out.logits.shape == (2, T, VOCAB)
    out.loss.backward()
    missing = [n for n, p in model.named_parameters() if p.requires_grad and p.grad is None]
    assert not missing, f"no gradient reached: {missing}"
    for n, p in model.named_parameters():
        assert torch.isfinite(p.grad).all(), n


@pytest.mark.parametrize(("T", "trained"), [(256, False), (384, True)])
def test_upper_gates_need_two_read_firings(T, trained):
    """Level 1 fires at chunks 1 and 3 with f = 2: at T = 256 (4 chunks) its
    first firing meets an empty state and the second lands on the last
    chunk, whose result reaches the loss only through the discarded final
    state, so the decay and erase gates get exactly zero gradient."""
    model = _model(2, (1, 2), (16,))
    ids = _ids(2, T)
    model(input_ids=ids, labels=ids).loss.backward()
    attn = model.model.layers[0].attn
    for name in ("g_projections", "b_projections"):
        got = getattr(attn, name).grad.abs().max().item()
        if trained:
            assert got > 0, f"{name} should receive gradient at T={T}"
        else:
            assert got == 0, f"{name} should be dead at T={T}, got {got}"
    for name in ("w_projections", "query_banks", "key_projections"):
        assert getattr(attn, name).grad.abs().max() > 0, name


@pytest.mark.parametrize("promotion", ["learned", "merge"])
def test_promotion_arm_wiring(promotion):
    model = _model(3, (1, 2, 4), (16, 16), promotion=promotion)
    ids = _ids(2, 640)
    model(input_ids=ids, labels=ids).loss.backward()
    attn = model.model.layers[0].attn
    for name in ("g_projections", "b_projections", "w_projections"):
        assert getattr(attn, name).grad.abs().max() > 0, name
    for name in ("query_banks", "key_projections"):
        t = getattr(attn, name)
        if promotion == "learned":
            assert isinstance(t, torch.nn.Parameter) and t.grad.abs().max() > 0, name
        else:
            assert not isinstance(t, torch.nn.Parameter) and t.grad is None, name


def test_promotion_arms_differ():
    outs = []
    for promotion in ("learned", "merge"):
        model = _model(3, (1, 2, 4), (16, 16), promotion=promotion)
        with torch.no_grad():
            outs.append(model(input_ids=_ids(2, 640)).logits)
    assert (outs[0] - outs[1]).abs().max() > 1e-3


@pytest.mark.parametrize(("num_levels", "firing", "n_queries", "T"), CASES, ids=IDS)
def test_keeping_all_levels_is_a_noop(num_levels, firing, n_queries, T):
    """Under softmax the kept weights are divided by their sum, as the
    reference does (layers/nested_gdn2.py:172-176). Each softmax weight is
    correctly rounded, but their fp32 sum can be 1 +- 1 ulp, so the division
    may move a weight by an ulp: the logits agree to rounding (the reference
    test asks for equal bits, which holds for it only where its softmax's sums
    round to exactly 1). The sigmoid arm divides nothing and is checked bit
    for bit below."""
    model = _model(num_levels, firing, n_queries)
    ids = _ids(2, T)
    base = _logits(model, ids, None)
    allk = _logits(model, ids, tuple(range(num_levels)))
    torch.testing.assert_close(allk, base, rtol=1e-5, atol=1e-5)


def test_ablation_changes_a_nested_model():
    model = _model(4, (1, 2, 4, 8), (16, 32, 64))
    ids = _ids(2, 1152)
    assert not torch.equal(_logits(model, ids, None), _logits(model, ids, (0,)))


def test_step_path_matches_chunked_under_ablation():
    """The ablation is applied to the mix before the chunked / stepped split,
    so a prefill and token-by-token decoding agree under it."""
    model = _model(4, (1, 2, 4, 8), (16, 32, 64))
    ids = _ids(1, 640)
    chunked = _logits(model, ids, (0,))
    _set_read_levels(model, (0,))
    out, cache = [], None
    with torch.no_grad():
        for t in range(ids.shape[1]):
            o = model(input_ids=ids[:, t:t + 1], past_key_values=cache, use_cache=True)
            cache = o.past_key_values
            out.append(o.logits)
    stepped = torch.cat(out, dim=1)
    torch.testing.assert_close(chunked, stepped, rtol=2e-2, atol=2e-2)


def _op_mix(monkeypatch, model, ids, keep):
    """The mix weights the layer hands the op (after the ablation mask)."""
    seen = []
    real = layer_mod.chunk_nested_gdn2

    def spy(*a, mix_weights, **kw):
        seen.append(mix_weights.detach().float().clone())
        return real(*a, mix_weights=mix_weights, **kw)

    monkeypatch.setattr(layer_mod, "chunk_nested_gdn2", spy)
    _set_read_levels(model, keep)
    with torch.no_grad():
        model(input_ids=ids)
    monkeypatch.setattr(layer_mod, "chunk_nested_gdn2", real)
    return seen[0]


def test_sigmoid_gates_are_independent(monkeypatch):
    model = _model(3, (1, 2, 4), (16, 16), read_mix="sigmoid")
    w = _op_mix(monkeypatch, model, _ids(2, 704), None)
    assert w.shape[-1] == 3
    assert w.min() >= 0.0 and w.max() <= 1.0
    assert w.sum(-1).max() > 1.0


def test_softmax_weights_sum_to_one(monkeypatch):
    model = _model(3, (1, 2, 4), (16, 16), read_mix="softmax")
    w = _op_mix(monkeypatch, model, _ids(2, 704), None)
    assert torch.allclose(w.sum(-1), torch.ones_like(w.sum(-1)), atol=1e-5)


def test_keeping_all_levels_is_a_noop_when_gated():
    model = _model(3, (1, 2, 4), (16, 16), read_mix="sigmoid")
    ids = _ids(2, 704)
    assert torch.equal(_logits(model, ids, None), _logits(model, ids, (0, 1, 2)))


def test_gated_ablation_leaves_the_kept_gate_alone(monkeypatch):
    model = _model(3, (1, 2, 4), (16, 16), read_mix="sigmoid")
    ids = _ids(2, 704)
    full = _op_mix(monkeypatch, model, ids, None)
    kept = _op_mix(monkeypatch, model, ids, (0,))
    assert torch.equal(kept[..., 0], full[..., 0])
    assert kept[..., 1:].abs().max() == 0.0
    assert kept[..., 0].max() < 1.0


def test_softmax_ablation_rescales_to_one(monkeypatch):
    model = _model(3, (1, 2, 4), (16, 16), read_mix="softmax")
    kept = _op_mix(monkeypatch, model, _ids(2, 704), (0,))
    assert torch.allclose(kept[..., 0], torch.ones_like(kept[..., 0]), atol=1e-5)
