"""The op with ``fire_partial_chunk=False`` (ngdn_dims.hold_partial = 1): a
partial last chunk completes no upper level's firing, as the reference's
decoding step treats an incomplete chunk (ops/naive.py:101-113). Expected
values: the oracle's token-by-token pass (oracle/ngdn_oracle.py
recurrent_forward, the reference's naive recurrence ops/naive.py:137-223),
which tests/test_oracle.py pins against the chunk form at whole chunks and
against the reference's step vectors; through autograd in float64 for the
gradients. Bar as for the op (tests/_parity.py).

The cases put the partial chunk where the held and the firing forms differ:
it would complete a firing of level 1 (f1 = 1, and f1 = 2 at T = 250), of
level 2 at the start of a new group (T = 257 with f = (1, 2, 4): the
level's last stored group holds the final state without a firing), and
where no level fires at all (T < 64).
The loss reads the final state too: the output alone does not see a firing
at the very end of the sequence."""

import pytest
import torch

import _parity
import ngdn_oracle as ref
from nested_recurrent_memory_amd import chunk_nested_gdn2
from nested_recurrent_memory_amd.inputs import LEAVES, NAMES, make_cotangent, make_inputs

pytestmark = pytest.mark.gpu

#  B,   T, H,   K, L,  N, firing
CASES = [
    (1, 100, 2, 64, 2, 16, (1, 1)),
    (2, 200, 2, 64, 3, 16, (1, 1, 2)),
    (1, 257, 2, 64, 3, 16, (1, 2, 4)),
    (1, 250, 2, 128, 2, 32, (1, 2)),
    (2, 40, 2, 64, 3, 16, (1, 1, 1)),
]


def _grads(inp, L, promotion, init, do, ds, dtype):
    gpu = {n: (inp[n].cuda().requires_grad_(True) if n in LEAVES else inp[n].cuda())
           for n in NAMES}
    i_g = init.cuda().requires_grad_(True)
    o, s = chunk_nested_gdn2(**gpu, L=L, initial_state=i_g, output_final_state=True,
                             promotion=promotion, fire_partial_chunk=False)
    ((o.float() * do.cuda()).sum() + (s * ds.cuda()).sum()).backward()
    ours = {n: gpu[n].grad if gpu[n].grad is not None else torch.zeros_like(gpu[n])
            for n in LEAVES}
    ours.update(o=o, final_state=s, initial_state=i_g.grad)

    leaves = {n: inp[n].double().requires_grad_(True) for n in LEAVES}
    i_r = init.double().requires_grad_(True)
    o_r, s_r = ref.recurrent_forward(*[leaves[n] for n in LEAVES], inp["n_queries_per_level"],
                                     inp["firing_intervals"], L, initial_state=i_r,
                                     promotion=promotion)
    ((o_r * do.double()).sum() + (s_r * ds.double()).sum()).backward()
    want = {n: leaves[n].grad if leaves[n].grad is not None else torch.zeros_like(leaves[n])
            for n in LEAVES}
    want.update(o=o_r, final_state=s_r, initial_state=i_r.grad)
    return ours, want


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16],
                         ids=["f32", "bf16", "f16"])
@pytest.mark.parametrize("K,V", [(64, 128), (128, 64)])
def test_held_partial_chunk_k_ne_v(K, V, dtype):
    """K != V (the layer's expand_v): the op pads to max(K, V) and slices
    back; the held partial chunk goes through the padding unchanged. fp16
    inputs compute in fp32 and return fp16 (bar of their input precision,
    the bf16 one)."""
    B, T, H, L, N, firing = 1, 150, 2, 2, 16, (1, 1)
    print(f"held partial K={K} V={V} {dtype}", flush=True)
    inp = make_inputs(B=B, T=T, H=H, K=K, V=V, L=L, N=N, intervals=firing, dtype=dtype,
                      g_scale=1.0, style="reftest")
    gen = torch.Generator().manual_seed(T)
    init = torch.randn(B, H, L, K, V, generator=gen) * 0.1
    do = make_cotangent((B, T, H, V), seed=3).to(dtype).float()
    ds = make_cotangent((B, H, L, K, V), seed=4)
    ours, want = _grads(inp, L, "learned", init, do, ds, dtype)
    _parity.check_all([(n, ours[n], want[n]) for n in want], dtype,
                      test=f"held K{K} V{V} {dtype}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("promotion", ["learned", "merge"])
@pytest.mark.parametrize("B,T,H,K,L,N,firing", CASES)
def test_held_partial_chunk_matches_recurrence(B, T, H, K, L, N, firing, promotion, dtype):
    print(f"held partial B={B} T={T} H={H} K={K} L={L} N={N} f={firing} {promotion} {dtype}",
          flush=True)
    inp = make_inputs(B=B, T=T, H=H, K=K, V=K, L=L, N=N, intervals=firing, dtype=dtype,
                      g_scale=1.0, style="reftest")
    gen = torch.Generator().manual_seed(T)
    init = torch.randn(B, H, L, K, K, generator=gen) * 0.1
    # the output's cotangent in the output's dtype, as autograd hands it to
    # the op, so that both sides see the same values
    do = make_cotangent((B, T, H, K), seed=3).to(dtype).float()
    ds = make_cotangent((B, H, L, K, K), seed=4)
    ours, want = _grads(inp, L, promotion, init, do, ds, dtype)
    _parity.check_all([(n, ours[n], want[n]) for n in want], dtype,
                      test=f"held B{B} T{T} K{K} L{L} f{firing} {promotion}")


def test_held_and_firing_forms_differ_only_in_the_final_state():
    """The same kernels either way: at whole chunks the two forms give the
    same bits; with a partial last chunk the output is the same (a firing at
    the sequence's end reaches no token) and the upper levels' final states
    differ, level 0's not."""
    inp = make_inputs(B=1, T=200, H=2, K=64, V=64, L=3, N=16, intervals=(1, 1, 2),
                      g_scale=1.0, style="reftest")
    gpu = {n: inp[n].cuda() for n in NAMES}
    for T in (192, 200):
        cut = {n: (x[:, :T] if n in NAMES[:7] else x) for n, x in gpu.items()}
        o1, s1 = chunk_nested_gdn2(**cut, L=3, output_final_state=True)
        o2, s2 = chunk_nested_gdn2(**cut, L=3, output_final_state=True, fire_partial_chunk=False)
        assert torch.equal(o1, o2)
        assert torch.equal(s1[:, :, 0], s2[:, :, 0])
        assert torch.equal(s1, s2) == (T % 64 == 0), T
