"""The model without fla on the GPU against the CPU model oracle (float64).

* RMSNorm, SwiGLU and the fused linear cross entropy (csrc/model_ops.hip,
  through the C ABI) against torch's rms_norm / silu / cross_entropy in
  float64 on the same values. Bar as for the op: fp32 1e-5; bf16 max-abs
  2e-3 / rel 1e-2, the absolute part scaled by max(1, max|ref|); the
  cross entropy's GEMM outputs (logits, dx, dW) round to the compute dtype,
  so its bf16 inputs are compared norm-wise at 2e-2.
* NestedGDN2ForCausalLM: loss, logits and every parameter gradient against
  the oracle model with the same parameter values: fp32 (norm-wise 1e-4)
  and bf16 autocast, the fused-loss training path and the logits path;
  prefill + decoding with the cache against one pass of the oracle. Under
  autocast every GEMM output rounds to bf16 (2^-8 relative), forward and
  backward, a dozen times in sequence from the loss to the first layer's
  parameters: the bar is norm-wise 2e-2 for outputs and 5e-2 for gradients
  (observed 1.5e-2 .. 2.8e-2), 0.15 for the decay parameters (see below).
  A dropped term or a wrong gate is O(1).
"""

import pytest
import torch
import torch.nn.functional as F

import ngdn_model_oracle as mref
from nested_recurrent_memory_amd.model import NestedGDN2Config, NestedGDN2ForCausalLM
from nested_recurrent_memory_amd.model_ops import (add_rms_norm, fused_linear_cross_entropy,
                                                   rms_norm, swiglu)

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
TOL = {torch.float32: (1e-5, 1e-5), torch.bfloat16: (2e-3, 1e-2)}
NORM_TOL = {torch.float32: 1e-4, torch.bfloat16: 2e-2}


def _close(name, got, want, dtype):
    atol, rtol = TOL[dtype]
    got, want = got.detach().double().cpu(), want.detach().double()
    m = max(1.0, want.abs().max().item())
    err = (got - want).abs()
    bad = err > atol * m + rtol * want.abs()
    assert not bad.any(), (f"{name}: {int(bad.sum())} of {bad.numel()} out of bound, max err "
                           f"{err.max().item():.3e} (scale {m:.3e})")


def _near(name, got, want, tol):
    assert got is not None and want is not None, f"{name}: gradient on one side only"
    got, want = got.detach().double().cpu(), want.detach().double()
    rel = ((got - want).norm() / want.norm().clamp_min(1e-30)).item()
    print(f"  {name}: rel {rel:.2e}", flush=True)
    assert rel <= tol, f"{name}: norm-wise relative error {rel:.3e} > {tol}"


def _gen(seed):
    return torch.Generator().manual_seed(seed)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("D,rows", [(64, 33), (256, 1000), (768, 70), (1024, 40000), (3072, 129)])
def test_rms_norm_matches_torch(dtype, D, rows):
    print(f"rms_norm dtype={dtype} D={D} rows={rows}", flush=True)
    g = _gen(D + rows)
    x = (torch.randn(rows, D, generator=g) * 3).to(dtype)
    w = 1 + 0.3 * torch.randn(D, generator=g)
    dy = torch.randn(rows, D, generator=g).to(dtype)
    x64, w64 = x.double().requires_grad_(), w.double().requires_grad_()
    y64 = F.rms_norm(x64, (D,), w64, 1e-5)
    (y64 * dy.double()).sum().backward()
    xd, wd = x.to(DEV).requires_grad_(), w.to(DEV).requires_grad_()
    y = rms_norm(xd, wd, 1e-5)
    y.backward(dy.to(DEV))
    torch.cuda.synchronize()
    _close("y", y, y64, dtype)
    _close("dx", xd.grad, x64.grad, dtype)
    _close("dw", wd.grad, w64.grad, torch.float32 if rows < 10000 else torch.bfloat16)


@pytest.mark.parametrize("xdt,rdt,ydt", [
    (torch.float32, torch.bfloat16, torch.bfloat16),     # fp32 residual stream, bf16 autocast
    (torch.float32, torch.float32, None),
    (torch.bfloat16, torch.bfloat16, None),
    (torch.float32, torch.bfloat16, None),               # bf16 r widened, fp32 y
    (torch.float32, torch.float32, torch.bfloat16),      # fp32 r, y cast to bf16
], ids=["f32-bf16-bf16", "f32", "bf16", "f32-bf16-f32", "f32-f32-bf16"])
@pytest.mark.parametrize("D,rows", [(256, 1000), (1024, 40000)])
def test_add_rms_norm_matches_torch(xdt, rdt, ydt, D, rows):
    """h = x + r and y = RMSNorm(h) w in one kernel against the separate add
    and norm in float64: h, y, and the gradients of x (the residual path's dh
    plus the norm's), r and w."""
    print(f"add_rms_norm x={xdt} r={rdt} y={ydt} D={D} rows={rows}", flush=True)
    g = _gen(3 * D + rows)
    x = (torch.randn(rows, D, generator=g) * 2).to(xdt)
    r = torch.randn(rows, D, generator=g).to(rdt)
    w = 1 + 0.3 * torch.randn(D, generator=g)
    ydt_eff = ydt if ydt is not None else xdt
    dy = torch.randn(rows, D, generator=g).to(ydt_eff)
    dh = torch.randn(rows, D, generator=g).to(xdt)
    x64, r64, w64 = (t.double().requires_grad_() for t in (x, r, w))
    h64 = x64 + r64
    # the sum as stored in x's dtype is what gets normalised (as after a separate add)
    hs = h64 + (h64.detach().to(xdt).double() - h64.detach())
    y64 = F.rms_norm(hs, (D,), w64, 1e-5)
    ((y64 * dy.double()).sum() + (h64 * dh.double()).sum()).backward()
    xd, rd, wd = (t.to(DEV).requires_grad_() for t in (x, r, w))
    h, y = add_rms_norm(xd, rd, wd, 1e-5, ydt)
    assert h.dtype == xdt and y.dtype == ydt_eff
    torch.autograd.backward([h, y], [dh.to(DEV), dy.to(DEV)])
    torch.cuda.synchronize()
    _close("h", h, h64, xdt)
    _close("y", y, y64, torch.bfloat16 if torch.bfloat16 in (xdt, ydt_eff) else torch.float32)
    _close("dx", xd.grad, x64.grad, xdt)
    _close("dr", rd.grad, r64.grad, rdt)
    _close("dw", wd.grad, w64.grad, torch.float32 if rows < 10000 else torch.bfloat16)


def test_rms_norm_bf16_output_from_fp32():
    """The block's first norm: fp32 x, bf16 y equal to the fp32 norm cast."""
    g = _gen(7)
    x = torch.randn(300, 1024, generator=g).to(DEV)
    w = (1 + 0.3 * torch.randn(1024, generator=g)).to(DEV)
    y32 = rms_norm(x, w, 1e-5)
    y16 = rms_norm(x, w, 1e-5, torch.bfloat16)
    assert y16.dtype == torch.bfloat16
    assert torch.equal(y16, y32.to(torch.bfloat16))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("n", [8, 4096 * 3 + 8, 3_000_000])
def test_swiglu_matches_torch(dtype, n):
    g = _gen(n)
    a = (torch.randn(n, generator=g) * 4).to(dtype)
    b = torch.randn(n, generator=g).to(dtype)
    dy = torch.randn(n, generator=g).to(dtype)
    a64, b64 = a.double().requires_grad_(), b.double().requires_grad_()
    y64 = F.silu(a64) * b64
    (y64 * dy.double()).sum().backward()
    ad, bd = a.to(DEV).requires_grad_(), b.to(DEV).requires_grad_()
    y = swiglu(ad, bd)
    y.backward(dy.to(DEV))
    torch.cuda.synchronize()
    _close("y", y, y64, dtype)
    _close("dg", ad.grad, a64.grad, dtype)
    _close("du", bd.grad, b64.grad, dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("N,V,bias", [(300, 1000, False), (513, 32000, True), (64, 50000, False)])
def test_fused_linear_cross_entropy_matches_torch(dtype, N, V, bias):
    print(f"linear CE dtype={dtype} N={N} V={V} bias={bias}", flush=True)
    g = _gen(N + V)
    d = 128
    x = torch.randn(N, d, generator=g).to(dtype)
    w = (torch.randn(V, d, generator=g) * 0.2).to(dtype)
    b = (torch.randn(V, generator=g) * 0.5).to(dtype) if bias else None
    t = torch.randint(0, V, (N,), generator=g)
    t[::7] = -100
    x64, w64 = x.double().requires_grad_(), w.double().requires_grad_()
    b64 = b.double().requires_grad_() if bias else None
    logits64 = x64 @ w64.t() + (b64 if bias else 0)
    loss64 = F.cross_entropy(logits64, t, ignore_index=-100)
    (loss64 * 1.7).backward()
    xd, wd = x.to(DEV).requires_grad_(), w.to(DEV).requires_grad_()
    bd = b.to(DEV).requires_grad_() if bias else None
    loss = fused_linear_cross_entropy(xd, t.to(DEV), wd, bd)
    (loss * 1.7).backward()
    torch.cuda.synchronize()
    if dtype == torch.float32:
        _close("loss", loss, loss64, dtype)
        _close("dx", xd.grad, x64.grad, dtype)
        _close("dw", wd.grad, w64.grad, dtype)
        if bias:
            _close("db", bd.grad, b64.grad, dtype)
    else:
        _near("loss", loss, loss64, 2e-3)
        _near("dx", xd.grad, x64.grad, 2e-2)
        _near("dw", wd.grad, w64.grad, 2e-2)
        if bias:
            _near("db", bd.grad, b64.grad, 2e-2)


def test_cross_entropy_all_ignored_and_bad_label():
    x = torch.randn(4, 16, device=DEV)
    w = torch.randn(64, 16, device=DEV)
    loss = fused_linear_cross_entropy(x, torch.full((4,), -100, device=DEV), w)
    assert torch.isnan(loss)          # as torch's mean over no targets
    loss = fused_linear_cross_entropy(x, torch.tensor([1, 2, 64, 3], device=DEV), w)
    assert torch.isnan(loss)          # label out of range: NaN, no read out of the row


def _cfg(**kw):
    base = dict(vocab_size=1024, hidden_size=256, num_hidden_layers=2, num_heads=4, head_dim=64,
                num_levels=3, firing_intervals=(1, 1, 2), n_queries_per_level=(16, 32),
                intermediate_size=512)
    base.update(kw)
    return NestedGDN2Config(**base)


def _model(cfg, seed):
    torch.manual_seed(seed)
    m = NestedGDN2ForCausalLM(cfg)
    with torch.no_grad():      # off the identity so that the norms' weights matter
        for name, p in m.named_parameters():
            if name.endswith("norm.weight"):
                p.add_(0.2 * torch.randn_like(p))
            if name.endswith("conv1d.weight"):
                p.mul_(20)       # N(0, 0.02) init makes the convolution nearly zero
    p64 = {k: v.detach().double().cpu().requires_grad_()
           for k, v in list(m.named_parameters()) + list(m.named_buffers())}
    return m.to(DEV), p64


@pytest.mark.parametrize("mode", ["f32", "bf16_autocast"])
@pytest.mark.parametrize("promotion", ["learned", "merge"])
def test_model_training_step_matches_oracle(mode, promotion):
    print(f"model train {mode} {promotion}", flush=True)
    cfg = _cfg(promotion=promotion)
    m, p64 = _model(cfg, 3)
    m.train()
    ids = torch.randint(0, cfg.vocab_size, (2, 256), generator=_gen(4))
    ids[1, 100] = 7
    logits64, loss64, _ = mref.model_forward(p64, ids, cfg, labels=ids)
    loss64.backward()
    tol = NORM_TOL[torch.float32 if mode == "f32" else torch.bfloat16]
    with torch.autocast("cuda", dtype=torch.bfloat16, enabled=mode != "f32"):
        out = m(input_ids=ids.to(DEV), labels=ids.to(DEV))
    assert out.logits is None                  # fused loss: logits not formed
    out.loss.backward()
    torch.cuda.synchronize()
    _near("loss", out.loss, loss64, tol)
    for name, p in m.named_parameters():
        # A_log's gradient per head sums B*T*K terms dg0 * g0 that largely
        # cancel, which multiplies the bf16 roundings of the projections
        # feeding g0; the fp32 run holds it to 1e-4.
        decay = mode != "f32" and name.endswith(("attn.A_log", "attn.dt_bias"))
        gtol = tol if mode == "f32" else 5e-2
        _near(f"d{name}", p.grad, p64[name].grad, 0.15 if decay else gtol)


@pytest.mark.parametrize("mode", ["f32", "bf16_autocast"])
def test_model_at_config4_shapes_matches_oracle(mode):
    """Two layers of config 4 (hidden 1024, 8 heads of 128, three levels at
    1/4/16 chunks with 64 queries each, SwiGLU 4096, vocab 32000), B=1,
    T=1024 so that level 2 fires: loss and every parameter gradient."""
    print(f"model at config 4 shapes {mode}", flush=True)
    torch.set_num_threads(min(16, torch.get_num_threads()))
    cfg = _cfg(vocab_size=32000, hidden_size=1024, num_heads=8, head_dim=128,
               firing_intervals=(1, 4, 16), n_queries_per_level=(64, 64),
               intermediate_size=4096)
    m, p64 = _model(cfg, 31)
    m.train()
    ids = torch.randint(0, cfg.vocab_size, (1, 1024), generator=_gen(32))
    _, loss64, _ = mref.model_forward(p64, ids, cfg, labels=ids)
    loss64.backward()
    tol = NORM_TOL[torch.float32 if mode == "f32" else torch.bfloat16]
    with torch.autocast("cuda", dtype=torch.bfloat16, enabled=mode != "f32"):
        out = m(input_ids=ids.to(DEV), labels=ids.to(DEV))
    out.loss.backward()
    torch.cuda.synchronize()
    _near("loss", out.loss, loss64, tol)
    for name, p in m.named_parameters():
        decay = mode != "f32" and name.endswith(("attn.A_log", "attn.dt_bias"))
        gtol = tol if mode == "f32" else 5e-2
        _near(f"d{name}", p.grad, p64[name].grad, 0.15 if decay else gtol)


def test_model_options_match_oracle():
    """No short convolution, sigmoid level mix, a decay horizon, tied
    embeddings off, 2 levels firing every other chunk: fp32 loss and every
    gradient."""
    cfg = _cfg(num_levels=2, firing_intervals=(1, 2), n_queries_per_level=(32,),
               use_short_conv=False, read_mix="sigmoid", max_horizon=64, promotion="merge")
    m, p64 = _model(cfg, 13)
    m.train()
    ids = torch.randint(0, cfg.vocab_size, (2, 256), generator=_gen(14))
    _, loss64, _ = mref.model_forward(p64, ids, cfg, labels=ids)
    loss64.backward()
    out = m(input_ids=ids.to(DEV), labels=ids.to(DEV))
    out.loss.backward()
    torch.cuda.synchronize()
    _near("loss", out.loss, loss64, 1e-4)
    for name, p in m.named_parameters():
        _near(f"d{name}", p.grad, p64[name].grad, 1e-4)


def test_model_eval_logits_and_loss_path():
    cfg = _cfg(num_levels=2, firing_intervals=(1, 2), n_queries_per_level=(16,))
    m, p64 = _model(cfg, 5)
    m.eval()
    ids = torch.randint(0, cfg.vocab_size, (2, 192), generator=_gen(6))
    logits64, loss64, _ = mref.model_forward(p64, ids, cfg, labels=ids)
    with torch.no_grad():
        out = m(input_ids=ids.to(DEV), labels=ids.to(DEV), use_cache=False)
    _near("logits", out.logits, logits64, 1e-4)
    _near("loss", out.loss, loss64, 1e-4)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_model_prefill_and_decode_match_one_pass(dtype):
    """Prefill 100 tokens with the cache, then three single-token steps: the
    logits of every call equal the oracle's one pass over all 103 tokens
    (the layer runs the first 64 chunkwise and steps the rest either way)."""
    cfg = _cfg()
    m, p64 = _model(cfg, 7)
    m = m.to(dtype).eval()
    p64 = {k: v.detach().to(dtype).double() for k, v in p64.items()}
    ids = torch.randint(0, cfg.vocab_size, (2, 103), generator=_gen(8))
    logits64, _, _ = mref.model_forward(p64, ids, cfg)
    tol = NORM_TOL[dtype]
    with torch.no_grad():
        out = m(input_ids=ids[:, :100].to(DEV), use_cache=True)
        _near("prefill", out.logits, logits64[:, :100], tol)
        cache = out.past_key_values
        assert cache.get_seq_length() == 100
        for t in range(100, 103):
            out = m(input_ids=ids[:, t:t + 1].to(DEV), past_key_values=cache, use_cache=True)
            cache = out.past_key_values
            _near(f"decode[{t}]", out.logits[:, 0], logits64[:, t], tol)
    assert cache.get_seq_length() == 103


@pytest.mark.parametrize("cut", [64, 200])
def test_model_is_causal(cut):
    """Logits before position ``cut`` do not depend on the tokens from ``cut``
    on (all levels, whole chunks and a partial one)."""
    cfg = _cfg(num_levels=3, firing_intervals=(1, 2, 4), n_queries_per_level=(16, 32))
    m, _ = _model(cfg, 10)
    m.eval()
    ids = torch.randint(0, cfg.vocab_size, (2, 512), generator=_gen(11)).to(DEV)
    other = ids.clone()
    other[:, cut:] = torch.randint(0, cfg.vocab_size, (2, 512 - cut), generator=_gen(12)).to(DEV)
    with torch.no_grad():
        a = m(input_ids=ids, use_cache=False).logits
        b = m(input_ids=other, use_cache=False).logits
    assert torch.equal(a[:, :cut], b[:, :cut])
    assert not torch.equal(a[:, cut:], b[:, cut:])


def test_model_refuses_padded_batches():
    cfg = _cfg(num_hidden_layers=1)
    m, _ = _model(cfg, 9)
    ids = torch.randint(0, cfg.vocab_size, (2, 64), device=DEV)
    mask = torch.ones(2, 64, device=DEV, dtype=torch.long)
    mask[0, :3] = 0
    with pytest.raises(ValueError, match="padded batches"):
        m(input_ids=ids, attention_mask=mask)


@pytest.mark.parametrize("n", [2, 8])
def test_fanout_gradient_sum(n):
    """x shared by n linear maps under autocast: one cast forward, the input
    gradient summed in fp32 in one pass (ngdn_sum_f32); equals the fp64 sum of
    the per-map gradients (each a bf16 GEMM output, rounded once)."""
    from nested_recurrent_memory_amd.layer_ops import fanout
    g = _gen(n)
    x = torch.randn(3, 50, 64, generator=g).to(DEV).requires_grad_()
    ws = [torch.randn(32, 64, generator=g).to(DEV) for _ in range(n)]
    cots = [torch.randn(3, 50, 32, generator=g).to(DEV) for _ in range(n)]
    with torch.autocast("cuda", dtype=torch.bfloat16):
        xs = fanout(x, n)
        assert all(t.dtype == torch.bfloat16 for t in xs)
        ys = [torch.nn.functional.linear(xi, w) for xi, w in zip(xs, ws)]
    sum((y.float() * c).sum() for y, c in zip(ys, cots)).backward()
    # each map's input gradient is the bf16 product c_j W_j; their sum in fp64
    want = sum((c.to(torch.bfloat16) @ w.to(torch.bfloat16)).double() for c, w in zip(cots, ws))
    assert x.grad.dtype == torch.float32
    _near("dx", x.grad, want.cpu(), 1e-2)
