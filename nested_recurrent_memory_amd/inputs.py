"""Seeded synthetic inputs for the op, drawn on the CPU so every consumer
(the GPU kernels, the CPU checker, the benchmark) sees identical bits.

Two distributions are offered:

``baseline``  the benchmark configurations' inputs: q, k ~ N(0,1) then
              L2-normalised over the head dim (q per level); v ~ N(0,1);
              b = sigmoid(N(0,1)); w = sigmoid(N(0,1));
              g = -softplus(N(0,1)) * g_scale (float32); mix = softmax(N(0,1))
              over levels; bank ~ N(0,1) K^-1/2; projections ~ N(0,1) V^-1/2.
``reftest``   the reference test helper's inputs (tests/ops/_op_inputs.py:11-77):
              q ~ N(0,1) (not normalised), k L2-normalised, v = 0.5 N(0,1),
              g = logsigmoid(N(0,1)) cast to the input dtype, b, w ~ U(0,1).

Float inputs are drawn in float32 and cast to ``dtype``; g stays float32 in
``baseline`` (the layer hands the op float32 decay, layers/nested_gdn2.py:142).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

NAMES = (
    "q", "k", "v", "g", "b", "w", "mix_weights", "query_banks",
    "key_projections", "b_projections", "w_projections", "g_projections",
    "n_queries_per_level", "firing_intervals",
)
LEAVES = NAMES[:12]


def make_inputs(B, T, H, K, V, L, N, intervals, n_queries=None, *,
                dtype=torch.float32, g_scale=0.1, seed=0, style="baseline"):
    """Returns a dict keyed by the op's argument names (CPU tensors)."""
    gen = torch.Generator().manual_seed(seed)

    def randn(*shape):
        return torch.randn(*shape, generator=gen, dtype=torch.float32)

    def rand(*shape):
        return torch.rand(*shape, generator=gen, dtype=torch.float32)

    if style == "baseline":
        q = F.normalize(randn(B, T, H, L, K), dim=-1)
        k = F.normalize(randn(B, T, H, K), dim=-1)
        v = randn(B, T, H, V)
        b = torch.sigmoid(randn(B, T, H, K))
        w = torch.sigmoid(randn(B, T, H, V))
        g = -F.softplus(randn(B, T, H, K)) * g_scale
        mix = torch.softmax(randn(B, T, H, L), dim=-1)
        g_dtype = torch.float32
    elif style == "reftest":
        q = randn(B, T, H, L, K)
        k = F.normalize(randn(B, T, H, K), dim=-1)
        v = randn(B, T, H, V) * 0.5
        g = F.logsigmoid(randn(B, T, H, K))
        b = rand(B, T, H, K)
        w = rand(B, T, H, V)
        mix = torch.softmax(randn(B, T, H, L), dim=-1)
        g_dtype = dtype
    else:
        raise ValueError(f"unknown input style {style!r}")

    n_up = max(L - 1, 0)
    nmax = max(N, 1)
    bank = randn(n_up, H, nmax, K) * K ** -0.5
    kp = randn(n_up, H, K, V) * V ** -0.5
    bp = randn(n_up, H, V, K) * V ** -0.5
    wp = randn(n_up, H, V, V) * V ** -0.5
    gp = randn(n_up, H, V, K) * V ** -0.5
    if n_queries is None:
        n_queries = (N,) * n_up
    out = dict(
        q=q.to(dtype), k=k.to(dtype), v=v.to(dtype), g=g.to(g_dtype),
        b=b.to(dtype), w=w.to(dtype), mix_weights=mix.to(dtype),
        query_banks=bank.to(dtype), key_projections=kp.to(dtype),
        b_projections=bp.to(dtype), w_projections=wp.to(dtype),
        g_projections=gp.to(dtype),
        n_queries_per_level=torch.tensor(list(n_queries), dtype=torch.int32),
        firing_intervals=torch.tensor(list(intervals), dtype=torch.int32),
    )
    return out


def make_cotangent(shape, seed=1, dtype=torch.float32):
    """Seeded output gradient ``do``."""
    gen = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=gen, dtype=torch.float32).to(dtype)


# The benchmark configurations (BASELINE.json "configs"): name -> kwargs.
CONFIGS = {
    "c0": dict(B=1, T=512, H=2, K=64, V=64, L=1, N=16, intervals=(1,),
               dtype=torch.float32, g_scale=0.1),
    "c1": dict(B=2, T=2048, H=8, K=128, V=128, L=2, N=32, intervals=(1, 4),
               dtype=torch.bfloat16, g_scale=0.1),
    "c2": dict(B=4, T=8192, H=16, K=128, V=128, L=3, N=64, intervals=(1, 4, 16),
               dtype=torch.bfloat16, g_scale=0.1),
    "c3": dict(B=1, T=65536, H=16, K=128, V=128, L=3, N=64, intervals=(1, 8, 64),
               dtype=torch.bfloat16, g_scale=1.0),
}
