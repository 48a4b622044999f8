"""Loads the golden vectors written by tests/golden/make_golden.py and
regenerates their inputs, checking the recorded input digest."""

from __future__ import annotations

import hashlib
import os

import numpy as np
import torch

from nested_recurrent_memory_amd.inputs import CONFIGS, make_cotangent, make_inputs

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")

# Mirrors the case table of make_golden.py (which needs the reference to run).
CASES = {
    "c0": (dict(CONFIGS["c0"]), "learned", False, False),
    "l3_learned": (dict(B=1, T=320, H=2, K=64, V=64, L=3, N=16, intervals=(1, 2, 4),
                        dtype=torch.float32, g_scale=1.0), "learned", True, False),
    "l3_merge": (dict(B=1, T=320, H=2, K=64, V=64, L=3, N=16, intervals=(1, 2, 4),
                      dtype=torch.float32, g_scale=1.0), "merge", True, False),
    "l2_bf16": (dict(B=1, T=512, H=2, K=128, V=128, L=2, N=32, intervals=(1, 4),
                     dtype=torch.bfloat16, g_scale=0.1), "learned", False, False),
    "grad_l2": (dict(B=1, T=256, H=1, K=64, V=64, L=2, N=16, intervals=(1, 2),
                     dtype=torch.float32, g_scale=0.5, style="reftest"),
                "learned", True, True),
    "grad_l3_merge": (dict(B=1, T=256, H=1, K=64, V=64, L=3, N=16, intervals=(1, 2, 4),
                           dtype=torch.float32, g_scale=0.5, style="reftest"),
                      "merge", False, True),
}

LEAVES = ("q", "k", "v", "g", "b", "w", "mix_weights", "query_banks",
          "key_projections", "b_projections", "w_projections", "g_projections")


def _digest(inp, init):
    h = hashlib.sha256()
    for name in sorted(inp):
        t = inp[name].contiguous()
        h.update(name.encode())
        h.update(t.view(torch.uint8).numpy().tobytes() if t.dtype == torch.bfloat16
                 else t.numpy().tobytes())
    if init is not None:
        h.update(init.numpy().tobytes())
    return h.hexdigest()


def load(name):
    """Returns (cfg, inputs, init, promotion, expected dict of torch tensors)."""
    cfg, promotion, with_init, with_grads = CASES[name]
    cfg = dict(cfg)
    inp = make_inputs(**cfg)
    init = None
    if with_init:
        gen = torch.Generator().manual_seed(123)
        init = torch.randn(cfg["B"], cfg["H"], cfg["L"], cfg["K"], cfg["V"],
                           generator=gen) * 0.1
    data = np.load(os.path.join(HERE, f"{name}.npz"))
    assert str(data["digest"]) == _digest(inp, init), (
        f"golden case {name}: regenerated inputs differ from the recorded ones")
    assert str(data["promotion"]) == promotion
    exp = {}
    for key in data.files:
        if key in ("digest", "promotion"):
            continue
        if key == "o_bf16_bits":
            exp["o"] = torch.from_numpy(data[key]).view(torch.bfloat16)
        else:
            exp[key] = torch.from_numpy(data[key])
    do = make_cotangent(exp["o"].shape, seed=1) if with_grads else None
    return cfg, inp, init, promotion, exp, do


def probe_update():
    data = np.load(os.path.join(HERE, "probe_update.npz"))
    return {k: torch.from_numpy(data[k]) for k in data.files}
