"""Gradient parity of the HIP backward against float64 autograd through the
CPU oracle, on identical seeded inputs.

Bar (tests/_parity.py), elementwise: bf16 inputs |got - ref| <= 2e-3 +
1e-2 |ref| for every gradient; fp32 inputs |got - ref| <= 1e-5 m + 1e-5 |ref|
with m = max(1, max|ref|) (gradients that sum summands of up to tens). The
unscaled errors are printed with every run.
"""

import pytest
import torch

import _golden
import _parity
import ngdn_oracle as ref
from nested_recurrent_memory_amd import chunk_nested_gdn2
from nested_recurrent_memory_amd.inputs import LEAVES, NAMES, make_cotangent, make_inputs

pytestmark = pytest.mark.gpu



def _run(inp, L, promotion, dtype, init=None, with_dfinal=False, seed=1):
    """(ours, oracle) dicts of gradients for every leaf (+ initial_state)."""
    gpu = {n: (inp[n].cuda().requires_grad_(True) if n in LEAVES else inp[n].cuda())
           for n in NAMES}
    i_g = init.cuda().requires_grad_(True) if init is not None else None
    o, s = chunk_nested_gdn2(**gpu, L=L, initial_state=i_g, output_final_state=True,
                             promotion=promotion)
    do = make_cotangent(o.shape, seed=seed).to(o.dtype)
    ds = make_cotangent(s.shape, seed=seed + 7) if with_dfinal else None
    loss = (o.float() * do.cuda().float()).sum()
    if ds is not None:
        loss = loss + (s * ds.cuda()).sum()
    loss.backward()
    ours = {n: gpu[n].grad for n in LEAVES}
    if i_g is not None:
        ours["initial_state"] = i_g.grad

    leaves = {n: inp[n].double().requires_grad_(True) for n in LEAVES}
    i_r = init.double().requires_grad_(True) if init is not None else None
    args = [leaves[n] for n in LEAVES] + [inp["n_queries_per_level"], inp["firing_intervals"]]
    o_r, s_r = ref.chunk_forward(*args, L=L, initial_state=i_r, output_final_state=True,
                                 promotion=promotion, out_dtype=torch.float64)
    loss_r = (o_r * do.double()).sum()
    if ds is not None:
        loss_r = loss_r + (s_r * ds.double()).sum()
    loss_r.backward()
    want = {n: (leaves[n].grad if leaves[n].grad is not None else torch.zeros_like(leaves[n]))
            for n in LEAVES}
    if i_r is not None:
        want["initial_state"] = i_r.grad
    for n in ours:
        if ours[n] is None:
            ours[n] = torch.zeros_like(want[n])
    return ours, want


def _check(ours, want, dtype, test=""):
    _parity.check_all([(n, ours[n], want[n]) for n in want], dtype, test=test)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("T,K,V", [(128, 64, 64), (192, 128, 128), (100, 64, 64),
                                   (128, 64, 128), (100, 128, 64)])
def test_level0_gradients(dtype, T, K, V):
    print(f"level0 grads T={T} K={K} V={V} {dtype}", flush=True)
    inp = make_inputs(B=2, T=T, H=2, K=K, V=V, L=1, N=16, intervals=(1,), dtype=dtype,
                      g_scale=1.0, style="reftest")
    ours, want = _run(inp, 1, "learned", dtype, with_dfinal=True)
    _check(ours, want, dtype, test=f"level0 T{T} K{K} V{V}")


#  B,   T, H,   K, L,  N, firing,    n_queries
CASES = [
    (1, 128, 2, 64, 2, 16, (1, 2), None),
    (2, 256, 2, 64, 2, 16, (1, 2), None),
    (1, 256, 4, 64, 2, 32, (1, 4), None),
    (2, 512, 2, 64, 3, 16, (1, 2, 4), None),
    (1, 512, 2, 64, 3, 32, (1, 2, 4), (32, 16)),
    (1, 256, 2, 128, 2, 16, (1, 2), None),
    (1, 256, 2, 64, 2, 16, (1, 1), None),
    (1, 320, 2, 64, 3, 16, (1, 2, 3), None),
    (1, 200, 2, 64, 3, 16, (1, 2, 4), None),
    # 64 pairs per firing with the headline schedule: level 2 fires at chunk 16
    (1, 1024, 2, 64, 3, 64, (1, 4, 16), None),
    (1, 1024, 2, 128, 3, 64, (1, 4, 16), None),
    # the reference's experiment arm (configs/nested-learned.yaml): four
    # levels at 1/2/4/8 chunks with 16/32/64 queries, head_dim 64
    (1, 1024, 2, 64, 4, 64, (1, 2, 4, 8), (16, 32, 64)),
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("promotion", ["learned", "merge"])
@pytest.mark.parametrize("B,T,H,K,L,N,firing,nq", CASES)
def test_gradients_match_oracle(B, T, H, K, L, N, firing, nq, promotion, dtype):
    print(f"grads B={B} T={T} H={H} K={K} L={L} N={N} f={firing} nq={nq} "
          f"{promotion} {dtype}", flush=True)
    inp = make_inputs(B=B, T=T, H=H, K=K, V=K, L=L, N=N, intervals=firing, n_queries=nq,
                      dtype=dtype, g_scale=1.0, style="reftest")
    ours, want = _run(inp, L, promotion, dtype)
    _check(ours, want, dtype, test=f"grads B{B} T{T} H{H} K{K} L{L} N{N} f{firing} nq{nq} "
                                   f"{promotion}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("promotion", ["learned", "merge"])
def test_initial_state_and_final_state_gradients(dtype, promotion):
    inp = make_inputs(B=2, T=256, H=2, K=64, V=64, L=3, N=16, intervals=(1, 2, 4),
                      dtype=dtype, g_scale=0.5)
    gen = torch.Generator().manual_seed(5)
    init = torch.randn(2, 2, 3, 64, 64, generator=gen) * 0.1
    ours, want = _run(inp, 3, promotion, dtype, init=init, with_dfinal=True)
    _check(ours, want, dtype, test=f"init+final {promotion}")


@pytest.mark.parametrize("name", ["grad_l2", "grad_l3_merge"])
def test_gradients_golden(name):
    """Against autograd through the reference's own naive op (float32)."""
    cfg, inp, init, promotion, exp, do = _golden.load(name)
    gpu = {n: (inp[n].cuda().requires_grad_(True) if n in LEAVES else inp[n].cuda())
           for n in NAMES}
    i_g = init.cuda().requires_grad_(True) if init is not None else None
    o, _ = chunk_nested_gdn2(**gpu, L=cfg["L"], initial_state=i_g, output_final_state=True,
                             promotion=promotion)
    (o * do.cuda()).sum().backward()
    for n in LEAVES:
        got = gpu[n].grad if gpu[n].grad is not None else torch.zeros_like(gpu[n])
        # the reference itself ran in float32: allow its rounding on top of ours
        want = exp["grad_" + n]
        m = max(1.0, want.abs().max().item())
        err = (got.cpu() - want).abs()
        assert (err <= 1e-4 * m + 1e-4 * want.abs()).all(), (n, err.max().item())
    if i_g is not None:
        want = exp["grad_initial_state"]
        err = (i_g.grad.cpu() - want).abs()
        assert (err <= 1e-4 * max(1.0, want.abs().max().item()) + 1e-4 * want.abs()).all()


# the fused promotion ladder (chunk.FUSED_PROMOTION) in the forward, with the
# backward reading its keys, (keys b e^g)^T and e^g
FUSED_CASES = [
    (1, 1024, 2, 128, 3, 64, (1, 4, 16), None, "learned"),
    (2, 512, 2, 64, 3, 32, (1, 2, 4), None, "learned"),
    (1, 512, 2, 64, 3, 16, (1, 2, 4), None, "merge"),
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("B,T,H,K,L,N,firing,nq,promotion", FUSED_CASES)
def test_gradients_with_fused_promotion(B, T, H, K, L, N, firing, nq, promotion, dtype):
    from nested_recurrent_memory_amd import chunk as chunk_mod
    print(f"fused grads B={B} T={T} K={K} L={L} N={N} f={firing} {promotion} {dtype}", flush=True)
    inp = make_inputs(B=B, T=T, H=H, K=K, V=K, L=L, N=N, intervals=firing, n_queries=nq,
                      dtype=dtype, g_scale=1.0, style="reftest")
    try:
        chunk_mod.FUSED_PROMOTION = True
        ours, want = _run(inp, L, promotion, dtype)
    finally:
        chunk_mod.FUSED_PROMOTION = False
    _check(ours, want, dtype, test=f"fused grads B{B} T{T} K{K} L{L} N{N} f{firing} {promotion}")


# K != V with upper levels (the layer's expand_v != 1): the op runs its K = V
# kernels at max(K, V) on zero-padded tensors; the results are the unpadded
# op's, against the oracle at K != V
KV_CASES = [
    (2, 320, 2, 128, 64, 3, 16, (1, 2, 4), "learned"),
    (2, 320, 2, 128, 64, 3, 16, (1, 2, 4), "merge"),
    (2, 320, 2, 64, 128, 3, 16, (1, 2, 4), "learned"),
    (1, 256, 2, 64, 128, 2, 32, (1, 1), "learned"),
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("B,T,H,K,V,L,N,firing,promotion", KV_CASES)
def test_gradients_k_ne_v(B, T, H, K, V, L, N, firing, promotion, dtype):
    print(f"grads K={K} V={V} L={L} N={N} f={firing} {promotion} {dtype}", flush=True)
    inp = make_inputs(B=B, T=T, H=H, K=K, V=V, L=L, N=N, intervals=firing, dtype=dtype,
                      g_scale=1.0, style="reftest")
    gen = torch.Generator().manual_seed(6)
    init = torch.randn(B, H, L, K, V, generator=gen) * 0.1
    ours, want = _run(inp, L, promotion, dtype, init=init, with_dfinal=True)
    _check(ours, want, dtype, test=f"grads K{K} V{V} L{L} N{N} f{firing} {promotion}")


# the level-0 chunk backward as two launches (ngdn_l0_bwd_state, then
# ngdn_l0_bwd_intra) instead of the fused ngdn_l0_bwd
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("K,V,L", [(128, 128, 3), (64, 128, 1)])
def test_gradients_with_two_launch_level0_backward(K, V, L, dtype):
    from nested_recurrent_memory_amd import chunk as chunk_mod
    print(f"two-launch l0 bwd K={K} V={V} L={L} {dtype}", flush=True)
    inp = make_inputs(B=2, T=320, H=2, K=K, V=V, L=L, N=16, intervals=(1, 2, 4)[:L],
                      dtype=dtype, g_scale=1.0, style="reftest")
    try:
        chunk_mod.FUSED_L0_BWD = False
        ours, want = _run(inp, L, "learned", dtype, with_dfinal=True)
    finally:
        chunk_mod.FUSED_L0_BWD = True
    _check(ours, want, dtype, test=f"two-launch l0 bwd K{K} V{V} L{L}")
