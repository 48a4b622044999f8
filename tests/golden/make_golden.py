"""Write golden vectors from the reference's own naive PyTorch op.

Run in the build container only (the reference is not present on the GPU box):

    python tests/golden/make_golden.py /root/reference

It loads ``nested_gdn2/ops/probe.py`` and ``nested_gdn2/ops/naive.py`` by file
path under a stub package (the real package __init__ pulls in transformers and
fla), runs them on the CPU in float32 on the seeded inputs of
``nested_recurrent_memory_amd.inputs.make_inputs``, and stores the outputs --
plus, for the gradient case, autograd gradients through the reference -- in
``tests/golden/*.npz``. Inputs are not stored: each case records a SHA-256 of
its regenerated input bytes, so a change in the input generator fails loudly.

These vectors pin the parts of the reference that only running it can pin:
cast placement, read-before-fire ordering in the composition, and the probe's
normalisation (F.normalize eps) as the reference executes them.
"""

from __future__ import annotations

import hashlib
import importlib.util
import os
import sys
import types

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from nested_recurrent_memory_amd.inputs import CONFIGS, make_cotangent, make_inputs  # noqa: E402

# name: (make_inputs kwargs, promotion, with_init, with_grads)
CASES = {
    # BASELINE config 0, whole.
    "c0": (dict(CONFIGS["c0"]), "learned", False, False),
    # Three levels, ragged groups (NT=5 with f=(1,2,4)), learned and merge.
    "l3_learned": (dict(B=1, T=320, H=2, K=64, V=64, L=3, N=16, intervals=(1, 2, 4),
                        dtype=torch.float32, g_scale=1.0), "learned", True, False),
    "l3_merge": (dict(B=1, T=320, H=2, K=64, V=64, L=3, N=16, intervals=(1, 2, 4),
                      dtype=torch.float32, g_scale=1.0), "merge", True, False),
    # bf16 inputs, fp32 g, the config-1 firing pattern on a short sequence.
    "l2_bf16": (dict(B=1, T=512, H=2, K=128, V=128, L=2, N=32, intervals=(1, 4),
                     dtype=torch.bfloat16, g_scale=0.1), "learned", False, False),
    # Gradients through the reference (float32 autograd).
    "grad_l2": (dict(B=1, T=256, H=1, K=64, V=64, L=2, N=16, intervals=(1, 2),
                     dtype=torch.float32, g_scale=0.5, style="reftest"),
                "learned", True, True),
    "grad_l3_merge": (dict(B=1, T=256, H=1, K=64, V=64, L=3, N=16, intervals=(1, 2, 4),
                           dtype=torch.float32, g_scale=0.5, style="reftest"),
                      "merge", False, True),
}

LEAVES = ("q", "k", "v", "g", "b", "w", "mix_weights", "query_banks",
          "key_projections", "b_projections", "w_projections", "g_projections")


def input_digest(inp: dict, init) -> str:
    h = hashlib.sha256()
    for name in sorted(inp):
        t = inp[name].contiguous()
        h.update(name.encode())
        h.update(t.view(torch.uint8).numpy().tobytes() if t.dtype == torch.bfloat16
                 else t.numpy().tobytes())
    if init is not None:
        h.update(init.numpy().tobytes())
    return h.hexdigest()


def case_init(cfg):
    B, H, L, K, V = cfg["B"], cfg["H"], cfg["L"], cfg["K"], cfg["V"]
    gen = torch.Generator().manual_seed(123)
    return torch.randn(B, H, L, K, V, generator=gen) * 0.1


def load_reference(ref_root: str):
    pkg = types.ModuleType("nested_gdn2")
    pkg.__path__ = []
    ops = types.ModuleType("nested_gdn2.ops")
    ops.__path__ = []
    sys.modules["nested_gdn2"] = pkg
    sys.modules["nested_gdn2.ops"] = ops
    mods = {}
    for name in ("probe", "naive"):
        path = os.path.join(ref_root, "nested_gdn2", "ops", f"{name}.py")
        spec = importlib.util.spec_from_file_location(f"nested_gdn2.ops.{name}", path)
        mod = importlib.util.module_from_spec(spec)
        sys.modules[spec.name] = mod
        spec.loader.exec_module(mod)
        mods[name] = mod
    return mods["probe"], mods["naive"]


def main(ref_root: str):
    probe, naive = load_reference(ref_root)
    torch.set_num_threads(min(8, os.cpu_count() or 1))
    for name, (cfg, promotion, with_init, with_grads) in CASES.items():
        cfg = dict(cfg)
        inp = make_inputs(**cfg)
        init = case_init(cfg) if with_init else None
        digest = input_digest(inp, init)
        kw = dict(L=cfg["L"], chunk_size=64, promotion=promotion,
                  output_final_state=True)
        store = {"digest": np.array(digest), "promotion": np.array(promotion)}
        if with_grads:
            leaves = {k: (inp[k].detach().clone().requires_grad_(True) if k in LEAVES
                          else inp[k]) for k in inp}
            i0 = init.clone().requires_grad_(True) if init is not None else None
            o, fin = naive.naive_chunk_nested_gdn2(**leaves, initial_state=i0, **kw)
            do = make_cotangent(o.shape, seed=1)
            (o.float() * do).sum().backward()
            for k in LEAVES:
                gr = leaves[k].grad
                store["grad_" + k] = (np.zeros(leaves[k].shape, np.float32) if gr is None
                                      else gr.float().numpy())
            if i0 is not None:
                store["grad_initial_state"] = i0.grad.float().numpy()
        else:
            with torch.no_grad():
                o, fin = naive.naive_chunk_nested_gdn2(**inp, initial_state=init, **kw)
        if o.dtype == torch.bfloat16:
            # bf16 output is stored as its exact bit pattern
            store["o_bf16_bits"] = o.detach().contiguous().view(torch.int16).numpy()
        else:
            store["o"] = o.detach().float().numpy()
        store["final_state"] = fin.detach().float().numpy()
        np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **store)
        print(name, tuple(o.shape), digest[:12])

    # Probe and update-step vectors on their own.
    gen = torch.Generator().manual_seed(7)
    B, NF, H, K, V, N = 1, 2, 1, 64, 64, 16
    S = torch.randn(B, NF, H, K, V, generator=gen) * K ** -0.5
    bank = torch.randn(H, 2 * N, K, generator=gen) * K ** -0.5
    kp = torch.randn(H, K, V, generator=gen) * V ** -0.5
    bp = torch.randn(H, V, K, generator=gen) * V ** -0.5
    wp = torch.randn(H, V, V, generator=gen) * V ** -0.5
    gp = torch.randn(H, V, K, generator=gen) * V ** -0.5
    store = dict(S=S.numpy(), bank=bank.numpy(), kp=kp.numpy(), bp=bp.numpy(),
                 wp=wp.numpy(), gp=gp.numpy(), n=np.array(N))
    for arm in ("learned", "merge"):
        keys, vals, b, w, g = probe.PROBES[arm](S, bank, kp, bp, wp, gp, N, torch.float32)
        for tag, t in zip(("keys", "vals", "b", "w", "g"), (keys, vals, b, w, g)):
            store[f"{arm}_{tag}"] = t.contiguous().numpy()
    # One firing of the update, on the learned pairs.
    st = torch.randn(B, H, K, V, generator=gen) * 0.3
    k0, v0, b0, w0, g0 = (store[f"learned_{t}"] for t in ("keys", "vals", "b", "w", "g"))
    upd = naive.naive_update_step(
        st, *(torch.from_numpy(x)[:, 0] for x in (k0, v0, b0, w0, g0)))
    store["update_state_in"] = st.numpy()
    store["update_state_out"] = upd.numpy()
    np.savez_compressed(os.path.join(HERE, "probe_update.npz"), **store)
    print("probe_update")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
