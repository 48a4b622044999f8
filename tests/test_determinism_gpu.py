"""Run-to-run determinism of the op's backward.

Every cross-row sum in the backward (the bank and projection gradients over
all firings, the norms, gates and mixing-weight sums inside the kernels) runs
in a fixed order, so two forward+backward passes on the same inputs give the
same bits, and so does a pass whose rows are launched in two groups on two
streams. Compared with torch.equal: no tolerance.
"""

import pytest
import torch

import nested_recurrent_memory_amd.chunk as chunk_mod
from nested_recurrent_memory_amd import chunk_nested_gdn2
from nested_recurrent_memory_amd.inputs import CONFIGS, LEAVES, NAMES, make_cotangent, make_inputs

pytestmark = pytest.mark.gpu


def _grads(inp, L, promotion, seed=3, fire_partial=True):
    gpu = {n: (inp[n].cuda().requires_grad_(True) if n in LEAVES else inp[n].cuda())
           for n in NAMES}
    o, s = chunk_nested_gdn2(**gpu, L=L, output_final_state=True, promotion=promotion,
                             fire_partial_chunk=fire_partial)
    do = make_cotangent(o.shape, seed=seed).cuda().to(o.dtype)
    ds = make_cotangent(s.shape, seed=seed + 1).cuda()
    torch.autograd.backward([o, s], [do, ds])
    torch.cuda.synchronize()
    out = {"o": o.detach(), "final": s.detach()}
    out.update({n: gpu[n].grad for n in LEAVES if gpu[n].grad is not None})
    return out


def _assert_equal(a, b):
    assert a.keys() == b.keys()
    for n in a:
        assert torch.equal(a[n], b[n]), f"{n}: max |diff| {(a[n] - b[n]).abs().max().item()}"


def test_c1_two_runs_are_bit_identical():
    c = CONFIGS["c1"]
    inp = make_inputs(**{k: c[k] for k in ("B", "T", "H", "K", "V", "L", "N", "intervals")},
                      dtype=c["dtype"], g_scale=c["g_scale"])
    first = _grads(inp, c["L"], "learned")
    second = _grads(inp, c["L"], "learned")
    _assert_equal(first, second)
    assert "query_banks" in first and first["query_banks"].abs().sum() > 0


@pytest.mark.parametrize("promotion", ["learned", "merge"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_three_levels_two_runs_and_two_row_groups_are_bit_identical(promotion, dtype):
    inp = make_inputs(B=3, T=1024, H=2, K=64, V=64, L=3, N=32,
                      intervals=(1, 2, 4), dtype=dtype, g_scale=0.1)
    first = _grads(inp, 3, promotion)
    second = _grads(inp, 3, promotion)
    _assert_equal(first, second)
    try:
        chunk_mod.STREAM_GROUPS = 2
        grouped = _grads(inp, 3, promotion)
    finally:
        chunk_mod.STREAM_GROUPS = 1
    _assert_equal(first, grouped)


@pytest.mark.parametrize("T,K,L,promotion,fire_partial,fused", [
    (64 * 256, 64, 3, "learned", True, False), (64 * 200 + 17, 64, 3, "learned", True, False),
    (64 * 200 + 17, 64, 3, "merge", True, False), (64 * 200 + 17, 64, 3, "learned", False, False),
    (64 * 200 + 17, 64, 3, "learned", True, True), (64 * 256, 128, 3, "learned", True, False),
    (64 * 200 + 17, 64, 2, "learned", True, False), (64 * 200 + 17, 64, 1, "learned", True, False)])
def test_level0_chunk_ranges_equal_one_launch(T, K, L, promotion, fire_partial, fused):
    """On small grids the forward forms the level-0 chunk terms and runs the
    level-0 scan over consecutive ranges of chunks, the chunk terms of a range
    on a side stream beside the scan of the range before, the state carried
    from range to range through the final state; the upper levels' probes and
    scans follow one range behind on a second side stream. Outputs, final
    states and every gradient equal those of one launch over all chunks, bit
    for bit: with a partial last chunk, firings that read a lower final state
    (T = 64 * 256), merge promotion, a held partial chunk, and the fused
    promotion ladder (whose levels then run after the level-0 ranges)."""
    NT = -(-T // 64)
    from nested_recurrent_memory_amd import _lib
    assert len(chunk_mod._l0_ranges(1, 2, K, NT, _lib.NGDN_BF16)) > 1
    inp = make_inputs(B=1, T=T, H=2, K=K, V=K, L=L, N=32,
                      intervals=(1, 4, 16)[:L], dtype=torch.bfloat16, g_scale=0.1)
    saved = chunk_mod.L0_PARTS, chunk_mod.FUSED_PROMOTION
    try:
        chunk_mod.FUSED_PROMOTION = fused
        ranged = _grads(inp, L, promotion, fire_partial=fire_partial)
        chunk_mod.L0_PARTS = 1
        single = _grads(inp, L, promotion, fire_partial=fire_partial)
    finally:
        chunk_mod.L0_PARTS, chunk_mod.FUSED_PROMOTION = saved
    _assert_equal(ranged, single)
