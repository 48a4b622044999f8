"""Input forms the op accepts besides contiguous bf16 / fp32 tensors
(ops/chunk.py:237-244 makes its inputs contiguous; tests/ops/test_chunk.py:
135-144 runs it under fp16 and bf16 autocast).

* float16 inputs (what fp16 autocast hands the op): they run the fp32
  kernels (fp16 -> fp32 is exact) and the output and gradients return in
  float16. Against the float64 oracle on the same fp16 values, bar
  |err| <= 2e-3 + 1e-2 |ref| for the output, final state and every gradient.
* Non-contiguous inputs (transposed or strided views of every tensor
  argument): output, final state and every gradient equal those of
  contiguous copies bit for bit.
"""

import pytest
import torch

import _parity
import ngdn_oracle as ref
from nested_recurrent_memory_amd import chunk_nested_gdn2
from nested_recurrent_memory_amd.inputs import LEAVES, NAMES, make_cotangent, make_inputs

pytestmark = pytest.mark.gpu

SEQ = ("q", "k", "v", "b", "w", "mix_weights")


def _run(gpu, L, promotion, init=None, seed=2):
    o, s = chunk_nested_gdn2(**gpu, L=L, initial_state=init, output_final_state=True,
                             promotion=promotion)
    do = make_cotangent(o.shape, seed=seed).cuda().to(o.dtype)
    ds = make_cotangent(s.shape, seed=seed + 1).cuda()
    torch.autograd.backward([o, s], [do, ds])
    torch.cuda.synchronize()
    return o, s, do, ds


@pytest.mark.parametrize("promotion", ["learned", "merge"])
def test_float16_inputs_match_oracle(promotion):
    inp = make_inputs(B=2, T=320, H=2, K=64, V=64, L=3, N=16, intervals=(1, 2, 4),
                      dtype=torch.float32, g_scale=0.5)
    for n in SEQ:
        inp[n] = inp[n].to(torch.float16)
    gpu = {n: (inp[n].cuda().requires_grad_(True) if n in LEAVES else inp[n].cuda())
           for n in NAMES}
    o, s, do, ds = _run(gpu, 3, promotion)
    assert o.dtype == torch.float16
    for n in SEQ:
        assert gpu[n].grad.dtype == torch.float16, n

    leaves = {n: inp[n].double().requires_grad_(True) for n in LEAVES}
    args = [leaves[n] for n in LEAVES] + [inp["n_queries_per_level"], inp["firing_intervals"]]
    o_r, s_r = ref.chunk_forward(*args, L=3, output_final_state=True, promotion=promotion,
                                 out_dtype=torch.float64)
    ((o_r * do.double().cpu()).sum() + (s_r * ds.double().cpu()).sum()).backward()
    pairs = [("o", o, o_r), ("final_state", s, s_r)]
    for n in LEAVES:
        want = leaves[n].grad if leaves[n].grad is not None else torch.zeros_like(leaves[n])
        got = gpu[n].grad if gpu[n].grad is not None else torch.zeros_like(gpu[n])
        pairs.append((n, got, want))
    _parity.check_all(pairs, torch.float16, test=f"fp16 inputs {promotion}")


def _strided(x):
    """A non-contiguous view with x's values: stored with the last two axes
    swapped (or, for 1-D-like tails, every other element of a wider buffer)."""
    if x.dim() >= 2 and x.shape[-1] > 1 and x.shape[-2] > 1:
        return x.transpose(-1, -2).contiguous().transpose(-1, -2)
    wide = torch.zeros(*x.shape[:-1], 2 * x.shape[-1], dtype=x.dtype, device=x.device)
    wide[..., ::2] = x
    return wide[..., ::2]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_non_contiguous_inputs_equal_contiguous(dtype):
    inp = make_inputs(B=2, T=256, H=2, K=64, V=64, L=3, N=16, intervals=(1, 2, 4),
                      dtype=dtype, g_scale=0.5)
    init = torch.randn(2, 2, 3, 64, 64, generator=torch.Generator().manual_seed(4)) * 0.1
    outs = []
    for view in (False, True):
        leaves = {n: inp[n].cuda() for n in LEAVES}
        if view:
            leaves = {n: _strided(x) for n, x in leaves.items()}
            assert not any(x.is_contiguous() for x in leaves.values())
        for x in leaves.values():
            x.requires_grad_(True)
        i_g = init.cuda()
        i_g = (_strided(i_g) if view else i_g).requires_grad_(True)
        gpu = dict(leaves, n_queries_per_level=inp["n_queries_per_level"],
                   firing_intervals=inp["firing_intervals"])
        o, s, _, _ = _run(gpu, 3, "learned", init=i_g)
        outs.append([o, s] + [leaves[n].grad for n in LEAVES] + [i_g.grad])
    for i, (a, b) in enumerate(zip(*outs)):
        assert torch.equal(a, b), f"tensor {i}: max |diff| {(a.float() - b.float()).abs().max()}"
