"""Parity at the headline configuration c2 itself (B=4, T=8192, H=16,
K=V=128, three levels at 1/4/16 chunks, 64 queries per level, bf16, the
benchmark's inputs), through the same launch the benchmark times.

* Two (batch, head) slices against the float64 oracle: the full c2 forward
  and backward run on the GPU with the output gradient nonzero on batch row
  0 only, so that each head's parameter gradients are that row's alone; the
  oracle runs the (row 0, head h) slice. Output, final state, every
  per-token gradient of the slice and the head's parameter gradients are
  compared. Rows 1-3 of every per-token gradient must be exactly zero.
* Batch rows are independent: row 2 of the B=4 forward equals a B=1 forward
  of that row bit for bit (the kernels' arithmetic per (batch, head) does not
  depend on the batch size).
* The split-sequence handoff: the first half's final state given to the
  second half as its initial state equals one pass (T/2 = 64 chunks
  completes a firing of every level).

Bar (tests/_parity.py): bf16 |err| <= 2e-3 + 1e-2 |ref| elementwise for
every tensor (outputs, states and every gradient).
"""

import pytest
import torch

import _parity
import ngdn_oracle as ref
from nested_recurrent_memory_amd import chunk_nested_gdn2
from nested_recurrent_memory_amd.inputs import CONFIGS, LEAVES, NAMES, make_cotangent, make_inputs

pytestmark = pytest.mark.gpu

SEQ = ("q", "k", "v", "g", "b", "w", "mix_weights")
PARAMS = LEAVES[7:]
HEADS = (0, 13)


@pytest.fixture(scope="module")
def c2():
    c = CONFIGS["c2"]
    inp = make_inputs(**{k: c[k] for k in ("B", "T", "H", "K", "V", "L", "N", "intervals")},
                      dtype=c["dtype"], g_scale=c["g_scale"])
    return inp, c["L"]


def _slice(inp, b, h):
    """The (b, h) slice as a B=1, H=1 problem (per-token tensors and the head's
    parameters)."""
    out = {}
    for n in NAMES:
        x = inp[n]
        if n in SEQ:
            x = x[b:b + 1, :, h:h + 1]
        elif n in PARAMS:
            x = x[:, h:h + 1]
        out[n] = x.contiguous()
    return out


def test_c2_slices_forward_backward_match_oracle(c2):
    torch.set_num_threads(min(16, torch.get_num_threads()))
    inp, L = c2
    print("c2 full forward+backward on the GPU", flush=True)
    gpu = {n: (inp[n].cuda().requires_grad_(True) if n in LEAVES else inp[n]) for n in NAMES}
    o, s = chunk_nested_gdn2(**gpu, L=L, output_final_state=True)
    do = make_cotangent(o.shape, seed=3).to(o.dtype)
    do[1:] = 0
    (o.float() * do.cuda().float()).sum().backward()
    torch.cuda.synchronize()
    for n in SEQ:
        rest = gpu[n].grad[1:]
        assert torch.count_nonzero(rest).item() == 0, f"d{n}: rows without a gradient are nonzero"
    for h in HEADS:
        print(f"c2 slice (0, {h}) against the oracle", flush=True)
        sl = _slice(inp, 0, h)
        lv = {n: sl[n].double().requires_grad_(True) for n in LEAVES}
        o_r, s_r = ref.chunk_forward(*[lv[n] for n in LEAVES], sl["n_queries_per_level"],
                                     sl["firing_intervals"], L=L, output_final_state=True,
                                     out_dtype=torch.float64)
        (o_r * do[0:1, :, h:h + 1].double()).sum().backward()
        pairs = [("o", o[0:1, :, h:h + 1], o_r), ("final_state", s[0:1, h:h + 1], s_r)]
        for n in SEQ:
            pairs.append(("d" + n, gpu[n].grad[0:1, :, h:h + 1], lv[n].grad))
        for n in PARAMS:
            pairs.append(("d" + n, gpu[n].grad[:, h:h + 1], lv[n].grad))
        _parity.check_all(pairs, torch.bfloat16, test=f"c2 slice (0,{h})")


def test_c2_batch_rows_are_independent(c2):
    inp, L = c2
    print("c2 forward B=4 against B=1 of row 2", flush=True)
    with torch.no_grad():
        g = {n: (inp[n].cuda() if n in LEAVES else inp[n]) for n in NAMES}
        o4, s4 = chunk_nested_gdn2(**g, L=L, output_final_state=True)
        one = {n: (g[n][2:3].contiguous() if n in SEQ else g[n]) for n in NAMES}
        o1, s1 = chunk_nested_gdn2(**one, L=L, output_final_state=True)
    torch.cuda.synchronize()
    assert torch.equal(o4[2:3], o1), "o of row 2 depends on the other rows"
    assert torch.equal(s4[2:3], s1), "final state of row 2 depends on the other rows"


def test_c2_split_sequence_equals_one_pass(c2):
    inp, L = c2
    print("c2 split at T/2 against one pass", flush=True)
    T = inp["q"].shape[1]
    half = T // 2
    assert (half // 64) % int(inp["firing_intervals"][-1]) == 0
    g = {n: (inp[n].cuda() if n in LEAVES else inp[n]) for n in NAMES}
    with torch.no_grad():
        o_full, s_full = chunk_nested_gdn2(**g, L=L, output_final_state=True)
        a = {n: (g[n][:, :half] if n in SEQ else g[n]) for n in NAMES}
        o1, s1 = chunk_nested_gdn2(**a, L=L, output_final_state=True)
        b = {n: (g[n][:, half:] if n in SEQ else g[n]) for n in NAMES}
        o2, s2 = chunk_nested_gdn2(**b, L=L, initial_state=s1, output_final_state=True)
    torch.cuda.synchronize()
    _parity.check_all([("o first half", o1, o_full[:, :half]),
                       ("o second half", o2, o_full[:, half:]),
                       ("final_state", s2, s_full)], torch.bfloat16, test="c2 split")
    assert torch.isfinite(o_full.float()).all() and torch.isfinite(s_full).all()
