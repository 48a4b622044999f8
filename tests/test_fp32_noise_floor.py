"""How close the fp32 bar sits to fp32 rounding itself: the oracle's chunk
form (the reference's naive chunk op, ops/naive.py:226-420) evaluated in
float32 on the CPU, the precision the reference itself runs in, against the
same oracle in float64, on the four-level case of the GPU gradient tests
(tests/test_backward_gpu.py CASES: B = 1, T = 1024, H = 2, K = 64, firings
1/2/4/8 with 16/32/64 queries, the reference test's input distributions).

The unscaled fp32 bar |err| <= 1e-5 + 1e-5 |ref| is met by this fp32
evaluation of the reference's own algorithm with little room: its gradients
of k and of the query banks reach about 0.8 of the bound. The GPU's fp32
gradients on the same case reach 1.2 (dk) and 1.6 (query banks) of it, and
stay within the bar scaled by max(1, max|ref|) (tests/_parity.py). CPU only:
these figures need no GPU."""

import torch

import ngdn_oracle as ref
from nested_recurrent_memory_amd.inputs import LEAVES, make_cotangent, make_inputs


def _grads(inp, dtype, do):
    leaves = {n: inp[n].to(dtype).requires_grad_(True) for n in LEAVES}
    o, _ = ref.chunk_forward(*[leaves[n] for n in LEAVES], inp["n_queries_per_level"],
                             inp["firing_intervals"], L=4, output_final_state=True,
                             promotion="learned", dtype=dtype, out_dtype=dtype)
    (o * do.to(dtype)).sum().backward()
    return {n: leaves[n].grad for n in LEAVES if leaves[n].grad is not None}


def test_fp32_reference_reaches_the_unscaled_bar():
    torch.manual_seed(0)
    inp = make_inputs(B=1, T=1024, H=2, K=64, V=64, L=4, N=64, intervals=(1, 2, 4, 8),
                      n_queries=(16, 32, 64), dtype=torch.float32, g_scale=1.0,
                      style="reftest")
    do = make_cotangent((1, 1024, 2, 64), seed=1)
    g64 = _grads(inp, torch.float64, do)
    g32 = _grads(inp, torch.float32, do)
    ratio = {}
    for n in g64:
        err = (g32[n].double() - g64[n]).abs()
        ratio[n] = (err / (1e-5 + 1e-5 * g64[n].abs())).max().item()
        print(f"  {n:>16}: fp32 evaluation at {ratio[n]:.3f} of the unscaled bound")
    # the fp32 evaluation passes the unscaled bar, with at most a factor 2.5
    # to spare on the two gradients the GPU's fp32 path exceeds it on
    assert max(ratio.values()) <= 1.0
    assert ratio["k"] >= 0.4 and ratio["query_banks"] >= 0.4, ratio
