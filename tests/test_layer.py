"""CPU checks of the layer: the layer oracle pinned against library routines
and its own invariants, the product layer's parameter names and shapes (a
reference layer's state_dict loads as it is), and that the product has no CPU
path (host tensors raise before any launch)."""

import pytest
import torch
import torch.nn.functional as F

import ngdn_layer_oracle as lref
from nested_recurrent_memory_amd.layer import NestedGDN2Attention, NestedGDN2LayerConfig
from nested_recurrent_memory_amd.layer_ops import rmsnorm_gated, short_conv

D64 = torch.float64


def _gen(seed):
    return torch.Generator().manual_seed(seed)


@pytest.mark.parametrize("W", [1, 2, 4, 5])
@pytest.mark.parametrize("act", [True, False])
def test_short_conv_oracle_is_causal_depthwise_conv1d(W, act):
    g = _gen(W)
    B, T, D = 2, 11, 6
    x = torch.randn(B, T, D, generator=g, dtype=D64)
    w = torch.randn(D, 1, W, generator=g, dtype=D64)
    y, cache = lref.short_conv(x, w, activation=act)
    want = F.conv1d(F.pad(x.transpose(1, 2), (W - 1, 0)), w, groups=D).transpose(1, 2)
    if act:
        want = F.silu(want)
    torch.testing.assert_close(y, want, rtol=1e-12, atol=1e-12)
    # fla's cache: the last W inputs, [B, D, W], newest last
    torch.testing.assert_close(cache, x[:, -W:].transpose(1, 2), rtol=0, atol=0)


@pytest.mark.parametrize("W", [2, 4])
@pytest.mark.parametrize("split", [1, 2, 3, 7])
def test_short_conv_oracle_cache_continues_one_pass(W, split):
    g = _gen(10 + W)
    B, T, D = 2, 9, 5
    x = torch.randn(B, T, D, generator=g, dtype=D64)
    w = torch.randn(D, 1, W, generator=g, dtype=D64)
    y, c = lref.short_conv(x, w)
    y1, c1 = lref.short_conv(x[:, :split], w)
    y2, c2 = lref.short_conv(x[:, split:], w, c1)
    torch.testing.assert_close(torch.cat([y1, y2], 1), y, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(c2, c, rtol=0, atol=0)
    # a first call shorter than the window pads its cache with zeros on the left
    if split < W:
        assert (c1[..., :W - split] == 0).all()


def test_rmsnorm_gated_oracle_matches_rms_norm():
    g = _gen(3)
    x = torch.randn(4, 3, 16, generator=g, dtype=D64)
    gate = torch.randn(4, 3, 16, generator=g, dtype=D64)
    w = torch.randn(16, generator=g, dtype=D64)
    got = lref.rmsnorm_gated(x, gate, w, 1e-5)
    want = F.rms_norm(x, (16,), w, 1e-5) * torch.sigmoid(gate)
    torch.testing.assert_close(got, want, rtol=1e-12, atol=1e-12)


def _small_cfg(**kw):
    cfg = NestedGDN2LayerConfig(hidden_size=24, num_heads=2, head_dim=8, expand_v=1.0,
                                conv_size=4, num_levels=2, firing_intervals=(1, 2),
                                n_queries_per_level=(16,), promotion="learned",
                                op_chunk_size=64)
    for k, v in kw.items():
        setattr(cfg, k, v)
    return cfg


def _oracle_params(cfg, seed):
    """The layer's parameters, drawn at the shapes the layer declares."""
    torch.manual_seed(seed)
    layer = NestedGDN2Attention(cfg, 0)
    p = {k: v.detach().to(D64) for k, v in layer.state_dict().items()}
    # bigger than the init so that the convolution and gates matter
    for k in p:
        if k.endswith("conv1d.weight"):
            p[k] = p[k] * 2
    p["o_norm.weight"] = p["o_norm.weight"] + 0.3 * torch.randn(p["o_norm.weight"].shape, dtype=D64)
    if "query_banks" not in p and cfg.num_levels > 1:
        H, K, V = cfg.num_heads, cfg.head_dim, int(cfg.head_dim * cfg.expand_v)
        p["query_banks"] = torch.zeros(cfg.num_levels - 1, H, max(cfg.n_queries_per_level), K, dtype=D64)
        p["key_projections"] = torch.zeros(cfg.num_levels - 1, H, K, V, dtype=D64)
    return p


@pytest.mark.parametrize("use_short_conv", [True, False])
@pytest.mark.parametrize("T", [128, 100])
def test_layer_oracle_chunk_and_step_forms_agree(use_short_conv, T):
    """From position 0 the chunk form over whole chunks plus steps for the
    tail equals stepping every token, and a split call with the cache equals
    one call (the layer's composition, layers/nested_gdn2.py:195-222)."""
    cfg = _small_cfg(use_short_conv=use_short_conv)
    p = _oracle_params(cfg, 7)
    x = torch.randn(2, T, cfg.hidden_size, generator=_gen(T), dtype=D64)
    o, cache = lref.layer_forward(p, x, cfg)
    assert int(cache["recurrent_state"][1][0]) == T
    # every token through the step form: T calls of one token
    c, outs = None, []
    for t in range(T):
        o_t, c = lref.layer_forward(p, x[:, t:t + 1], cfg, c)
        outs.append(o_t)
    torch.testing.assert_close(torch.cat(outs, 1), o, rtol=1e-9, atol=1e-10)
    torch.testing.assert_close(c["recurrent_state"][0], cache["recurrent_state"][0],
                               rtol=1e-9, atol=1e-10)
    # a whole first chunk, then the rest with the cache
    o1, c1 = lref.layer_forward(p, x[:, :64], cfg)
    o2, c2 = lref.layer_forward(p, x[:, 64:], cfg, c1)
    torch.testing.assert_close(torch.cat([o1, o2], 1), o, rtol=1e-9, atol=1e-10)


def test_layer_oracle_gates_matter():
    """The output gate enters the output: shifting its bias changes it, so a
    slip that drops the gate fails the GPU comparison."""
    cfg = _small_cfg()
    p = _oracle_params(cfg, 8)
    x = torch.randn(1, 64, cfg.hidden_size, generator=_gen(1), dtype=D64)
    o, _ = lref.layer_forward(p, x, cfg)
    p2 = dict(p)
    p2["g_proj.1.bias"] = p["g_proj.1.bias"] + 1.0
    o2, _ = lref.layer_forward(p2, x, cfg)
    assert (o - o2).abs().max() > 1e-3


# parameter names and shapes of the reference's layer (layers/nested_gdn2.py:
# 53-101) for hidden 64, 2 heads of 16, expand_v 2, conv 4, L=3, N=(16, 32)
REF_SHAPES = {
    "q_proj.weight": (96, 64), "k_proj.weight": (32, 64), "v_proj.weight": (64, 64),
    "q_conv1d.weight": (96, 1, 4), "k_conv1d.weight": (32, 1, 4), "v_conv1d.weight": (64, 1, 4),
    "f_proj.0.weight": (32, 64), "f_proj.1.weight": (32, 32),
    "b_proj.weight": (32, 64), "w_proj.weight": (64, 64),
    "A_log": (2,), "dt_bias": (32,),
    "b_projections": (2, 2, 32, 16), "w_projections": (2, 2, 32, 32),
    "g_projections": (2, 2, 32, 16), "query_banks": (2, 2, 32, 16),
    "key_projections": (2, 2, 16, 32),
    "mix_proj.weight": (6, 64), "g_proj.0.weight": (32, 64), "g_proj.1.weight": (64, 32),
    "g_proj.1.bias": (64,), "o_norm.weight": (32,), "o_proj.weight": (64, 64),
}


def test_layer_parameters_match_reference_names_and_shapes():
    cfg = NestedGDN2LayerConfig(hidden_size=64, num_heads=2, head_dim=16, expand_v=2.0,
                                num_levels=3, firing_intervals=(1, 2, 4),
                                n_queries_per_level=(16, 32))
    layer = NestedGDN2Attention(cfg, 0)
    got = {k: tuple(v.shape) for k, v in layer.state_dict().items()}
    assert got == REF_SHAPES
    # merge keeps query_banks/key_projections as non-persistent buffers
    cfg.promotion = "merge"
    merge = NestedGDN2Attention(cfg, 0)
    names = set(merge.state_dict())
    assert names == set(REF_SHAPES) - {"query_banks", "key_projections"}
    assert layer.A_log._no_weight_decay and layer.dt_bias._no_weight_decay


def test_layer_config_is_validated():
    with pytest.raises(ValueError):
        NestedGDN2Attention(_small_cfg(firing_intervals=(2, 2)))
    with pytest.raises(ValueError):
        NestedGDN2Attention(_small_cfg(n_queries_per_level=(24,)))
    with pytest.raises(ValueError):
        NestedGDN2Attention(_small_cfg(op_chunk_size=32))


def test_layer_ops_refuse_host_tensors():
    x = torch.randn(1, 4, 8)
    with pytest.raises(ValueError, match="no CPU path"):
        short_conv(x, torch.randn(8, 1, 4))
    with pytest.raises(ValueError, match="no CPU path"):
        rmsnorm_gated(torch.randn(2, 64), torch.randn(2, 64), torch.ones(64))
