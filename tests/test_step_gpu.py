"""Decoding step (ngdn_step) against the CPU oracle's step (float64).

The oracle's step (oracle/ngdn_oracle.py:step_forward, restating
ops/naive.py:42-134) is pinned by prefill + step == one pass in
tests/test_oracle.py. Bar (tests/_parity.py), elementwise and unscaled:
fp32 inputs |err| <= 1e-5 + 1e-5 |ref|; bf16 inputs |err| <= 2e-3 +
1e-2 |ref|, for the output and every level's state.
"""

import pytest
import torch

import _parity
import ngdn_oracle as ref
from nested_recurrent_memory_amd import chunk_nested_gdn2, step_nested_gdn2
from nested_recurrent_memory_amd.inputs import NAMES, make_inputs

pytestmark = pytest.mark.gpu

STEP_IN = ("q", "k", "v", "g", "b", "w", "mix_weights")
PARAMS = ("query_banks", "key_projections", "b_projections", "w_projections",
          "g_projections", "n_queries_per_level", "firing_intervals")


def _close(name, got, want, dtype):
    _parity.check(name, got, want, dtype, scaled=False, test="step")


def _state(B, H, L, K, V, seed):
    gen = torch.Generator().manual_seed(seed)
    return torch.randn(B, H, L, K, V, generator=gen) * 0.5


def _token(inp, t):
    return {n: inp[n][:, t] for n in STEP_IN}


CASES = [
    # L, K, V, N, intervals, promotion
    (1, 64, 128, 16, (1,), "learned"),
    (2, 64, 64, 16, (1, 1), "learned"),
    (3, 128, 128, 64, (1, 1, 2), "learned"),
    (3, 64, 64, 32, (1, 2, 4), "merge"),
    (2, 128, 128, 128, (1, 1), "merge"),
    # K != V with upper levels: the K = V kernels at max(K, V), zero-padded
    (2, 64, 128, 16, (1, 1), "learned"),
    (3, 128, 64, 32, (1, 1, 2), "merge"),
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("case", CASES, ids=lambda c: f"L{c[0]}K{c[1]}V{c[2]}N{c[3]}{c[5][0]}")
@pytest.mark.parametrize("position", [5, 63, 127, 255, "rows"])
def test_step_matches_oracle(dtype, case, position):
    L, K, V, N, f, promotion = case
    print(f"step dtype={dtype} case={case} position={position}", flush=True)
    B, H = 3, 2
    inp = make_inputs(B=B, T=1, H=H, K=K, V=V, L=L, N=N, intervals=f, dtype=dtype,
                      g_scale=0.5, seed=7)
    state = _state(B, H, L, K, V, seed=3)
    pos = torch.tensor([63, 64, 255]) if position == "rows" else position
    tok = _token(inp, 0)
    gpu_pos = pos.cuda() if torch.is_tensor(pos) else pos
    s_dev = state.cuda()
    o, s = step_nested_gdn2(**{n: x.cuda() for n, x in tok.items()}, state=s_dev,
                            position=gpu_pos, **{n: inp[n].cuda() for n in PARAMS},
                            L=L, promotion=promotion)
    torch.cuda.synchronize()
    assert o.dtype == dtype and s.dtype == torch.float32
    assert torch.equal(s_dev.cpu(), state), "the state passed in must not change"

    o_ref, s_ref = ref.step_forward(*[tok[n].double() for n in STEP_IN], state.double(), pos,
                                    *[inp[n].double() for n in PARAMS[:5]],
                                    inp["n_queries_per_level"], inp["firing_intervals"],
                                    L=L, promotion=promotion)
    _close("o", o, o_ref, dtype)
    _close("state", s, s_ref, dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("promotion", ["learned", "merge"])
def test_prefill_then_step_handoff(dtype, promotion):
    """The chunk op's final state feeds the step (tests/ops/test_chunk.py:161-197):
    prefill 128 tokens, step 128 more through firings of level 1 at tokens 191
    and 255 and of level 2 at 191; every output and the final state match one
    oracle pass. (The sequence ends on a chunk boundary: over a ragged end the
    chunk form counts the partial chunk as a firing, the step form does not,
    which is why the layer chunks only whole chunks, layers/nested_gdn2.py:198-214.)"""
    print(f"handoff dtype={dtype} promotion={promotion}", flush=True)
    B, H, K, L, T, pre = 2, 2, 64, 3, 256, 128
    f = (1, 1, 3)
    inp = make_inputs(B=B, T=T, H=H, K=K, V=K, L=L, N=16, intervals=f, dtype=dtype,
                      g_scale=0.5, seed=11)
    gpu = {n: inp[n].cuda() for n in NAMES}
    with torch.no_grad():
        o_pre, state = chunk_nested_gdn2(**{n: (gpu[n][:, :pre] if n in STEP_IN else gpu[n])
                                            for n in NAMES}, L=L, output_final_state=True,
                                         promotion=promotion)
        outs = [o_pre]
        for t in range(pre, T):
            o_t, state = step_nested_gdn2(**{n: gpu[n][:, t] for n in STEP_IN}, state=state,
                                          position=t, **{n: gpu[n] for n in PARAMS}, L=L,
                                          promotion=promotion)
            outs.append(o_t.unsqueeze(1))
    torch.cuda.synchronize()
    o_ref, s_ref = ref.chunk_forward(*[inp[n].double() if n not in PARAMS[5:] else inp[n]
                                       for n in NAMES], L=L, output_final_state=True,
                                     promotion=promotion, out_dtype=torch.float64)
    _close("o", torch.cat(outs, 1), o_ref, dtype)
    _close("final state", state, s_ref, dtype)


def test_step_rows_fire_on_device():
    """Per-row positions on the GPU: only the rows whose token ends a firing
    promote; the others keep their upper levels bit for bit."""
    B, H, K, L = 4, 2, 64, 2
    inp = make_inputs(B=B, T=1, H=H, K=K, V=K, L=L, N=16, intervals=(1, 1), seed=5)
    state = _state(B, H, L, K, K, seed=9).cuda()
    pos = torch.tensor([63, 62, 127, 0], device="cuda")
    o, s = step_nested_gdn2(**{n: x.cuda() for n, x in _token(inp, 0).items()}, state=state,
                            position=pos, **{n: inp[n].cuda() for n in PARAMS}, L=L)
    torch.cuda.synchronize()
    up_same = (s[:, :, 1] == state[:, :, 1]).flatten(1).all(1).cpu()
    assert up_same.tolist() == [False, True, False, True]


def test_step_graph_replays_match_eager():
    """One token captured in a HIP graph (in-place state, device position,
    position += 1 inside the graph) and replayed across firings of both upper
    levels: every replay equals the eager step bit for bit."""
    from nested_recurrent_memory_amd import prepare_step_params

    B, H, K, L, f = 2, 2, 64, 3, (1, 1, 2)
    inp = make_inputs(B=B, T=1, H=H, K=K, V=K, L=L, N=16, intervals=f, seed=21)
    tok = {n: x.cuda() for n, x in _token(inp, 0).items()}
    # schedule sizes as host values, as the layer passes them (tuples): a
    # device tensor would need a host read inside the capture
    par_in = {n: (inp[n].cuda() if n in PARAMS[:5] else tuple(inp[n].tolist())) for n in PARAMS}
    par = prepare_step_params(*(par_in[n] for n in PARAMS[:5]), torch.float32)
    init = _state(B, H, L, K, K, seed=4).cuda()
    state_g = init.clone()
    pos = torch.full((B,), 126, dtype=torch.int64, device="cuda")
    with torch.no_grad():
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):   # warm-up outside capture, then restore
            step_nested_gdn2(**tok, state=state_g.clone(), position=pos.clone(), **par_in,
                             L=L, params=par, inplace=True)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            o_g, _ = step_nested_gdn2(**tok, state=state_g, position=pos, **par_in, L=L,
                                      params=par, inplace=True)
            pos.add_(1)
        state_e = init.clone()
        for r in range(5):
            graph.replay()
            torch.cuda.synchronize()
            o_e, state_e = step_nested_gdn2(**tok, state=state_e, position=126 + r, **par_in,
                                            L=L)
            torch.cuda.synchronize()
            assert torch.equal(o_g, o_e), f"replay {r}: o differs"
            assert torch.equal(state_g, state_e), f"replay {r}: state differs"
    assert not torch.equal(state_e[:, :, 2], init[:, :, 2]), "level 2 should have fired"
