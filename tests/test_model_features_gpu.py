"""Model features around the op (tests/models/test_modeling.py of the
reference: gradient checkpointing :85-99, autocast :102-110, generate
:222-243).

* Gradient checkpointing: after gradient_checkpointing_enable() a training
  step gives the same loss (bit for bit: the recomputed forward is the same
  launches on the same values) and the same parameter gradients (the layer's
  weight-gradient reductions add in any order: 1e-5 relative, norm-wise),
  while the memory held between the forward and the backward falls to the
  blocks' inputs (asserted: at most half of the non-checkpointed figure).
* generate(): each step's scores equal the logits of a full forward over the
  same prefix (the reference's bar: rtol = atol = 2e-2).
* fp16 autocast through the model: finite loss and gradients, and the loss
  within 2e-2 of the fp32 model's.
"""

import pytest
import torch

from nested_recurrent_memory_amd.model import NestedGDN2Config, NestedGDN2ForCausalLM

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _config(num_levels, firing, n_queries, **kw):
    base = dict(vocab_size=512, hidden_size=128, num_hidden_layers=2, num_heads=2, head_dim=64,
                num_levels=num_levels, firing_intervals=firing, n_queries_per_level=n_queries,
                fuse_cross_entropy=False)
    base.update(kw)
    return NestedGDN2Config(**base)


def _rel(a, b):
    return ((a.double() - b.double()).norm() / b.double().norm().clamp_min(1e-30)).item()


@pytest.mark.parametrize("autocast", [False, True], ids=["f32", "bf16_autocast"])
@pytest.mark.parametrize("promotion", ["learned", "merge"])
def test_gradient_checkpointing_matches(promotion, autocast):
    torch.manual_seed(0)
    model = NestedGDN2ForCausalLM(_config(3, (1, 2, 4), (16, 32), promotion=promotion,
                                          num_hidden_layers=3)).to(DEV).train()
    ids = torch.randint(0, 512, (2, 1024), device=DEV)
    params = [p for p in model.parameters() if p.requires_grad]

    def step():
        torch.cuda.synchronize()
        before = torch.cuda.memory_allocated()
        with torch.autocast("cuda", dtype=torch.bfloat16, enabled=autocast):
            loss = model(input_ids=ids, labels=ids).loss
        torch.cuda.synchronize()
        held = torch.cuda.memory_allocated() - before
        grads = torch.autograd.grad(loss, params)
        return loss.detach(), grads, held

    loss_a, grads_a, held_a = step()
    model.gradient_checkpointing_enable()
    assert all(b.gradient_checkpointing for b in model.model.layers)
    loss_b, grads_b, held_b = step()
    model.gradient_checkpointing_disable()
    print(f"  held between forward and backward: {held_a / 2**20:.1f} MiB plain, "
          f"{held_b / 2**20:.1f} MiB checkpointed", flush=True)
    assert torch.equal(loss_a, loss_b)
    for (name, _), a, b in zip([(n, p) for n, p in model.named_parameters() if p.requires_grad],
                               grads_a, grads_b):
        assert _rel(b, a) <= 1e-5, f"d{name}: rel {_rel(b, a):.3e}"
    assert held_b <= 0.5 * held_a


@pytest.mark.parametrize("promotion", ["learned", "merge"])
def test_generate_matches_brute_force(promotion):
    """Scores, not token ids: an untrained model's top candidates are closer
    together than the two paths' numerical difference."""
    torch.manual_seed(0)
    model = NestedGDN2ForCausalLM(_config(2, (1, 2), (16,), promotion=promotion)).to(DEV).eval()
    prompt = torch.randint(0, 512, (1, 96), device=DEV)
    P = prompt.shape[1]
    with torch.no_grad():
        out = model.generate(prompt, max_new_tokens=8, do_sample=False, use_cache=True,
                             output_scores=True, return_dict_in_generate=True)
        assert out.sequences.shape == (1, P + 8)
        assert len(out.scores) == 8
        ids = prompt
        for step, scores in enumerate(out.scores):
            logits = model(input_ids=ids, use_cache=False).logits[:, -1]
            torch.testing.assert_close(scores, logits, rtol=2e-2, atol=2e-2)
            ids = torch.cat([ids, out.sequences[:, P + step:P + step + 1]], dim=1)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
def test_autocast(dtype):
    torch.manual_seed(0)
    model = NestedGDN2ForCausalLM(_config(2, (1, 2), (16,))).to(DEV)
    ids = torch.randint(0, 512, (2, 256), device=DEV)
    ref = model(input_ids=ids, labels=ids).loss.detach()
    with torch.autocast("cuda", dtype=dtype):
        out = model(input_ids=ids, labels=ids)
    assert torch.isfinite(out.loss)
    out.loss.backward()
    for name, p in model.named_parameters():
        if p.grad is not None:
            assert torch.isfinite(p.grad).all(), name
    assert abs(out.loss.item() - ref.item()) <= 2e-2 * abs(ref.item())


def test_unfused_norms_match_fused():
    """fuse_norm=False builds torch's nn.RMSNorm with plain residual adds
    (models/modeling_nested_gdn2.py:46,100); with the same parameters the
    model gives the fused path's loss and gradients (fp32, norm-wise 1e-5)."""
    torch.manual_seed(0)
    fused = NestedGDN2ForCausalLM(_config(2, (1, 2), (16,))).to(DEV)
    plain = NestedGDN2ForCausalLM(_config(2, (1, 2), (16,), fuse_norm=False)).to(DEV)
    assert isinstance(plain.model.layers[0].attn_norm, torch.nn.RMSNorm)
    assert isinstance(plain.model.norm, torch.nn.RMSNorm)
    with torch.no_grad():
        for p in fused.parameters():
            p.add_(0.01 * torch.randn_like(p))
    plain.load_state_dict(fused.state_dict())
    ids = torch.randint(0, 512, (2, 256), device=DEV)
    la = fused(input_ids=ids, labels=ids).loss
    lb = plain(input_ids=ids, labels=ids).loss
    la.backward()
    lb.backward()
    assert abs(la.item() - lb.item()) <= 1e-5 * abs(la.item())
    named = dict(plain.named_parameters())
    for name, p in fused.named_parameters():
        if p.grad is not None:
            assert _rel(named[name].grad, p.grad) <= 1e-5, name
