"""The layer without fla on the GPU against the CPU layer oracle (float64).

* ShortConvolution and FusedRMSNormGated kernels (csrc/layer_ops.hip, through
  the C ABI): outputs, the convolution cache (fla's [B,D,W] layout) and the
  gradients against oracle/ngdn_layer_oracle.py, itself pinned against
  torch's conv1d and rms_norm (tests/test_layer.py). Bar as for the op:
  fp32 1e-5; bf16 max-abs 2e-3 / rel 1e-2, the absolute part scaled by
  max(1, max|ref|).
* NestedGDN2Attention: output and every gradient (input and parameters)
  against the oracle layer with the same parameter values, for training
  (whole chunks, and ragged lengths through the op with a held partial
  chunk), prefill, and decoding with the cache.
  The layer's projections are torch Linear layers whose outputs round to the
  activation dtype between the kernels, so the bar here is norm-wise:
  ||got - ref|| <= tol ||ref|| with tol 1e-4 in fp32 and 2e-2 in bf16 (one
  bf16 rounding is 2^-9 = 2e-3 relative; a handful of them in sequence stay
  well under 2e-2, while a dropped term or wrong gate is O(1)).
"""

import pytest
import torch
import torch.nn.functional as F

import ngdn_layer_oracle as lref
from nested_recurrent_memory_amd.layer import NestedGDN2Attention, NestedGDN2LayerConfig
from nested_recurrent_memory_amd.layer_ops import rmsnorm_gated, short_conv

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
D64 = torch.float64
TOL = {torch.float32: (1e-5, 1e-5), torch.bfloat16: (2e-3, 1e-2)}
LAYER_TOL = {torch.float32: 1e-4, torch.bfloat16: 2e-2}


def _close(name, got, want, dtype):
    atol, rtol = TOL[dtype]
    got, want = got.detach().double().cpu(), want.detach().double()
    m = max(1.0, want.abs().max().item())
    err = (got - want).abs()
    bad = err > atol * m + rtol * want.abs()
    assert not bad.any(), (f"{name}: {int(bad.sum())} of {bad.numel()} out of bound, max err "
                           f"{err.max().item():.3e} (scale {m:.3e})")


def _near(name, got, want, dtype, tol=None):
    if got is None and want is None:    # no path from this parameter to the output
        print(f"  {name}: no gradient on either side", flush=True)
        return
    assert got is not None and want is not None, f"{name}: gradient on one side only"
    got, want = got.detach().double().cpu(), want.detach().double()
    rel = ((got - want).norm() / want.norm().clamp_min(1e-30)).item()
    print(f"  {name}: rel {rel:.2e}", flush=True)
    tol = tol or LAYER_TOL[dtype]
    assert rel <= tol, f"{name}: norm-wise relative error {rel:.3e} > {tol}"


def _gen(seed):
    return torch.Generator().manual_seed(seed)


# ----------------------------------------------------------------- ShortConvolution

@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("W", [1, 4, 8])
@pytest.mark.parametrize("T", [1, 3, 130])
@pytest.mark.parametrize("with_cache", [False, True], ids=["nocache", "cache"])
def test_short_conv_matches_oracle(dtype, W, T, with_cache):
    print(f"short_conv dtype={dtype} W={W} T={T} cache={with_cache}", flush=True)
    g = _gen(100 * W + T)
    B, D = 3, 136
    x = torch.randn(B, T, D, generator=g).to(dtype)
    w = (torch.randn(D, 1, W, generator=g) * 0.5).float()
    cache = torch.randn(B, D, W, generator=g).to(dtype) if with_cache else None
    dy = torch.randn(B, T, D, generator=g).to(dtype)

    x64 = x.double().requires_grad_()
    w64 = w.double().requires_grad_()
    y64, c64 = lref.short_conv(x64, w64, cache.double() if with_cache else None)
    (y64 * dy.double()).sum().backward()

    xd = x.to(DEV).requires_grad_()
    wd = w.to(DEV).requires_grad_()
    cd = cache.to(DEV) if with_cache else None
    y, c = short_conv(xd, wd, cd, activation=True, output_final_state=True)
    y.backward(dy.to(DEV))
    torch.cuda.synchronize()
    _close("y", y, y64, dtype)
    _close("cache", c, c64, dtype)
    if with_cache:
        assert c.data_ptr() == cd.data_ptr()          # updated in place, as fla's
    _close("dx", xd.grad, x64.grad, dtype)
    _close("dw", wd.grad, w64.grad, torch.float32)


def test_short_conv_no_activation_and_no_cache_output():
    g = _gen(5)
    x = torch.randn(2, 70, 64, generator=g)
    w = torch.randn(64, 1, 4, generator=g)
    y, c = short_conv(x.to(DEV), w.to(DEV), activation=False)
    assert c is None
    y64, _ = lref.short_conv(x.double(), w.double(), activation=False)
    _close("y", y, y64, torch.float32)


# ----------------------------------------------------------------- FusedRMSNormGated

@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("V,rows", [(64, 1), (64, 70001), (128, 1000), (256, 333)])
def test_rmsnorm_gated_matches_oracle(dtype, V, rows):
    print(f"rmsnorm_gated dtype={dtype} V={V} rows={rows}", flush=True)
    g = _gen(V + rows)
    x = (torch.randn(rows, V, generator=g) * 2).to(dtype)
    gate = torch.randn(rows, V, generator=g).to(dtype)
    w = 1 + 0.3 * torch.randn(V, generator=g)
    dy = torch.randn(rows, V, generator=g).to(dtype)

    x64, g64, w64 = (t.double().requires_grad_() for t in (x, gate, w))
    y64 = lref.rmsnorm_gated(x64, g64, w64, 1e-5)
    (y64 * dy.double()).sum().backward()

    xd, gd, wd = (t.to(DEV).requires_grad_() for t in (x, gate, w))
    y = rmsnorm_gated(xd, gd, wd, 1e-5)
    y.backward(dy.to(DEV))
    torch.cuda.synchronize()
    _close("y", y, y64, dtype)
    _close("dx", xd.grad, x64.grad, dtype)
    _close("dg", gd.grad, g64.grad, dtype)
    # dw sums over every row in fp32
    _close("dw", wd.grad, w64.grad, torch.float32 if rows < 10000 else torch.bfloat16)


# ----------------------------------------------------------------- gate prologue

def _prologue_ref(q, k, f, bz, wz, ml, A_log, dt_bias, L, H, K, V, max_horizon, gated):
    """The reference's expressions (layers/nested_gdn2.py:134-166) in float64."""
    B, T = q.shape[:2]
    qn = F.normalize(q.reshape(B, T, L, H, K).transpose(2, 3), dim=-1)
    kn = F.normalize(k.reshape(B, T, H, K), dim=-1)
    g0 = F.softplus(f + dt_bias).reshape(B, T, H, K)
    g0 = -A_log.exp().unsqueeze(-1) * g0
    if max_horizon:
        g0 = g0.clamp(max=-1.0 / max_horizon)
    b0 = bz.sigmoid().reshape(B, T, H, K)
    w0 = wz.sigmoid().reshape(B, T, H, V)
    lg = ml.reshape(B, T, H, L)
    mix = lg.sigmoid() if gated else lg.softmax(-1)
    return qn, kn, g0, b0, w0, mix


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("L,K,V,horizon,gated", [(3, 128, 128, None, False), (2, 64, 64, 16, True),
                                                 (1, 64, 128, None, False), (4, 128, 64, 8, False),
                                                 (8, 128, 128, 32, True), (7, 64, 64, None, False)])
def test_gate_prologue_matches_torch(dtype, L, K, V, horizon, gated):
    from nested_recurrent_memory_amd.layer_ops import gate_prep
    print(f"gate_prep dtype={dtype} L={L} K={K} V={V} horizon={horizon} gated={gated}", flush=True)
    g = _gen(L * K + V)
    B, T, H = 2, 37, 3
    raw = [torch.randn(B, T, n, generator=g).to(dtype) for n in
           (L * H * K, H * K, H * K, H * K, H * V, H * L)]
    raw[2] = raw[2] * 3                     # f: reach both softplus branches and the cap
    raw[2][0, 0, :5] = 25.0
    A_log = torch.log(torch.empty(H).uniform_(1, 16, generator=g))
    dt_bias = torch.randn(H * K, generator=g) * 0.5
    cots = [torch.randn(s, generator=g) for s in
            ((B, T, H, L, K), (B, T, H, K), (B, T, H, K), (B, T, H, K), (B, T, H, V), (B, T, H, L))]

    r64 = [t.double().requires_grad_() for t in raw]
    p64 = [A_log.double().requires_grad_(), dt_bias.double().requires_grad_()]
    outs64 = _prologue_ref(*r64, *p64, L, H, K, V, horizon, gated)
    sum((o * c.double()).sum() for o, c in zip(outs64, cots)).backward()

    rd = [t.to(DEV).requires_grad_() for t in raw]
    pd = [A_log.to(DEV).requires_grad_(), dt_bias.to(DEV).requires_grad_()]
    outs = gate_prep(*rd, *pd, L, H, K, V, max_horizon=horizon, sigmoid_mix=gated)
    sum((o.float() * c.to(DEV)).sum() for o, c in zip(outs, cots)).backward()
    torch.cuda.synchronize()
    names = ("qn", "kn", "g0", "b0", "w0", "mix")
    for n, o, o64 in zip(names, outs, outs64):
        _close(n, o, o64, dtype if n != "g0" else torch.float32)
    for n, t, t64 in zip(("dq", "dk", "df", "dbz", "dwz", "dml"), rd, r64):
        _close(n, t.grad, t64.grad, dtype)
    _close("dA_log", pd[0].grad, p64[0].grad, torch.float32)
    _close("ddt_bias", pd[1].grad, p64[1].grad, torch.float32)


# ----------------------------------------------------------------- the layer

LAYER_CASES = [
    # name, overrides. Level 1 fires after every chunk where it can, so that a
    # firing from a nonzero state reaches the output and every promotion
    # parameter has a gradient.
    ("L2learned", dict(num_levels=2, firing_intervals=(1, 1), n_queries_per_level=(16,))),
    ("L3merge", dict(num_levels=3, firing_intervals=(1, 1, 2), n_queries_per_level=(16, 32),
                     promotion="merge")),
    ("L1noconv_v2", dict(num_levels=1, firing_intervals=(1,), n_queries_per_level=(),
                         use_short_conv=False, expand_v=2.0)),
    ("L2sigmoid_horizon", dict(num_levels=2, firing_intervals=(1, 1), n_queries_per_level=(32,),
                               read_mix="sigmoid", max_horizon=64)),
    # expand_v 2 with an upper level: K = 64, V = 128 (layers/nested_gdn2.py:34)
    ("L2learned_v2", dict(num_levels=2, firing_intervals=(1, 1), n_queries_per_level=(16,),
                          expand_v=2.0)),
]
# The decay parameters' gradients sum B*T*K terms that cancel, and with
# max_horizon the clamp at -1/max_horizon flips for channels near it when the
# projection is rounded to bf16: their bf16 bar is wider.
DECAY_BF16_TOL = 6e-2


def _layer(dtype, seed, **kw):
    cfg = NestedGDN2LayerConfig(hidden_size=256, num_heads=4, head_dim=64, conv_size=4)
    for k, v in kw.items():
        setattr(cfg, k, v)
    torch.manual_seed(seed)
    layer = NestedGDN2Attention(cfg, 0)
    with torch.no_grad():       # so that the convolution and the norm weight matter
        for name, p in layer.named_parameters():
            if name.endswith("conv1d.weight"):
                p.mul_(2)
            if name == "o_norm.weight":
                p.add_(0.3 * torch.randn_like(p))
    layer = layer.to(DEV, dtype)
    # the oracle's parameters: the same values, float64 on the CPU
    p64 = {k: v.detach().double().cpu().requires_grad_()
           for k, v in list(layer.named_parameters()) + list(layer.named_buffers())}
    return cfg, layer, p64


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("case", LAYER_CASES, ids=[c[0] for c in LAYER_CASES])
def test_layer_training_step_matches_oracle(dtype, case):
    name, kw = case
    print(f"layer train dtype={dtype} case={name}", flush=True)
    cfg, layer, p64 = _layer(dtype, 11, **kw)
    g = _gen(12)
    x = torch.randn(2, 256, cfg.hidden_size, generator=g).to(dtype)
    dy = torch.randn(2, 256, cfg.hidden_size, generator=g).to(dtype)

    x64 = x.double().requires_grad_()
    o64, _ = lref.layer_forward(p64, x64, cfg)
    (o64 * dy.double()).sum().backward()

    xd = x.to(DEV).requires_grad_()
    o, _, _ = layer(xd)
    o.backward(dy.to(DEV))
    torch.cuda.synchronize()
    _near("o", o, o64, dtype)
    _near("dx", xd.grad, x64.grad, dtype)
    for pname, p in layer.named_parameters():
        wide = dtype == torch.bfloat16 and pname in ("A_log", "dt_bias")
        _near(f"d{pname}", p.grad, p64[pname].grad, dtype, DECAY_BF16_TOL if wide else None)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("case", LAYER_CASES[:2], ids=[c[0] for c in LAYER_CASES[:2]])
def test_layer_prefill_and_decode_match_oracle(dtype, case):
    """Prefill of 100 tokens (through the op, its partial second chunk firing
    nothing), then three single-token calls with the cache (stepped from
    position 100), as generation runs the layer."""
    name, kw = case
    print(f"layer decode dtype={dtype} case={name}", flush=True)
    cfg, layer, p64 = _layer(dtype, 21, **kw)
    x = torch.randn(2, 103, cfg.hidden_size, generator=_gen(22)).to(dtype)
    x64 = x.double()
    with torch.no_grad():
        pkv = {}
        o, _, pkv = layer(x[:, :100].to(DEV), past_key_values=pkv, use_cache=True)
        o64, c64 = lref.layer_forward(p64, x64[:, :100], cfg)
        _near("prefill o", o, o64, dtype)
        for t in range(100, 103):
            o, _, pkv = layer(x[:, t:t + 1].to(DEV), past_key_values=pkv, use_cache=True)
            o64, c64 = lref.layer_forward(p64, x64[:, t:t + 1], cfg, c64)
            _near(f"decode o[{t}]", o, o64, dtype)
    state, pos = pkv[0]["recurrent_state"]
    assert pos.tolist() == [103, 103]
    _near("state", state, c64["recurrent_state"][0], dtype)
    if cfg.use_short_conv:
        for got, want in zip(pkv[0]["conv_state"], c64["conv_state"]):
            _near("conv_state", got, want, dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("T", [70, 100])
@pytest.mark.parametrize("case", LAYER_CASES[:2], ids=[c[0] for c in LAYER_CASES[:2]])
def test_layer_ragged_training_matches_oracle(dtype, T, case):
    """T not a multiple of the chunk: the layer runs the whole call through
    the op with its partial last chunk firing nothing, differentiably; the
    oracle layer composes the reference's way (whole chunks chunkwise, the
    rest stepped, layers/nested_gdn2.py:196-224). Output, the cached state
    and every gradient."""
    name, kw = case
    print(f"layer ragged train dtype={dtype} T={T} case={name}", flush=True)
    cfg, layer, p64 = _layer(dtype, 13, **kw)
    g = _gen(14)
    x = torch.randn(2, T, cfg.hidden_size, generator=g).to(dtype)
    dy = torch.randn(2, T, cfg.hidden_size, generator=g).to(dtype)

    x64 = x.double().requires_grad_()
    o64, c64 = lref.layer_forward(p64, x64, cfg)
    (o64 * dy.double()).sum().backward()

    xd = x.to(DEV).requires_grad_()
    o, _, pkv = layer(xd, past_key_values={}, use_cache=True)
    o.backward(dy.to(DEV))
    torch.cuda.synchronize()
    _near("o", o, o64, dtype)
    state, pos = pkv[0]["recurrent_state"]
    assert pos.tolist() == [T, T]
    _near("state", state, c64["recurrent_state"][0], dtype)
    _near("dx", xd.grad, x64.grad, dtype)
    for pname, p in layer.named_parameters():
        wide = dtype == torch.bfloat16 and pname in ("A_log", "dt_bias")
        _near(f"d{pname}", p.grad, p64[pname].grad, dtype, DECAY_BF16_TOL if wide else None)


def test_layer_unaligned_continuation_with_grad_raises_in_backward():
    """A call continuing a cache from position 70 (not a multiple of 64) is
    stepped: with grad enabled it gives the no-grad output, and only a
    backward through the stepped tokens raises (the decoding step has no
    backward)."""
    cfg, layer, _ = _layer(torch.float32, 31, num_levels=2, firing_intervals=(1, 2),
                           n_queries_per_level=(16,))
    x = torch.randn(1, 80, cfg.hidden_size, device=DEV)
    with torch.no_grad():
        _, _, pkv = layer(x[:, :70], past_key_values={}, use_cache=True)
    snap = {0: {"recurrent_state": tuple(t.clone() for t in pkv[0]["recurrent_state"]),
                "conv_state": tuple(t.clone() for t in pkv[0]["conv_state"])}}
    with torch.no_grad():
        want, _, _ = layer(x[:, 70:], past_key_values=snap, use_cache=True)
    xg = x[:, 70:].clone().requires_grad_()
    o, _, _ = layer(xg, past_key_values=pkv, use_cache=True)
    assert o.requires_grad
    assert torch.equal(o.detach(), want)
    with pytest.raises(RuntimeError, match="no backward"):
        o.sum().backward()


def test_layer_at_model_config_shape_matches_oracle():
    """One layer at config 4's shape (hidden 1024, 8 heads of 128, three
    levels at 1/4/16 chunks with 64 queries each), bf16, T = 2048 so that
    level 2 fires twice: output and every gradient against the oracle layer."""
    dtype = torch.bfloat16
    print("layer at the model config's shape, bf16, T=2048", flush=True)
    torch.set_num_threads(min(16, torch.get_num_threads()))
    cfg, layer, p64 = _layer(dtype, 41, hidden_size=1024, num_heads=8, head_dim=128,
                             num_levels=3, firing_intervals=(1, 4, 16),
                             n_queries_per_level=(64, 64))
    g = _gen(42)
    x = torch.randn(1, 2048, cfg.hidden_size, generator=g).to(dtype)
    dy = torch.randn(1, 2048, cfg.hidden_size, generator=g).to(dtype)

    x64 = x.double().requires_grad_()
    o64, _ = lref.layer_forward(p64, x64, cfg)
    (o64 * dy.double()).sum().backward()

    xd = x.to(DEV).requires_grad_()
    o, _, _ = layer(xd)
    o.backward(dy.to(DEV))
    torch.cuda.synchronize()
    _near("o", o, o64, dtype)
    _near("dx", xd.grad, x64.grad, dtype)
    for pname, p in layer.named_parameters():
        wide = pname in ("A_log", "dt_bias")
        _near(f"d{pname}", p.grad, p64[pname].grad, dtype, DECAY_BF16_TOL if wide else None)
