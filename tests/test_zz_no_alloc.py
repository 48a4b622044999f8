"""ngdn_step_noalloc against ngdn_step, through the C ABI.

The allocation-free variant runs the same kernels; the levels with more
than 64 pairs per firing go through the library's file-scope scratch a slice
of batch rows at a time instead of through a workspace argument. Bar
(integer-exact agreement is expected from identical kernels on identical
inputs): o and the new state equal ngdn_step's bit for bit, on two calls in a
row, the second with a smaller batch. The first call's batch needs two
slices of the scratch (one row of H=2 heads at 128 pairs and K=128 takes
2 x (3 x 128 x 128 + 128) x 4 bytes, so 85 rows fit in 32 MiB) and mixes
rows that fire with rows that do not (per-row device positions).
"""

import ctypes

import pytest
import torch

from nested_recurrent_memory_amd import _lib, prepare_step_params
from nested_recurrent_memory_amd.inputs import make_inputs

pytestmark = pytest.mark.gpu

STEP_IN = ("q", "k", "v", "g", "b", "w", "mix_weights")
PARAMS = ("query_banks", "key_projections", "b_projections", "w_projections", "g_projections")


def _call(name, B, H, L, K, N, f, tok, par, state, pos, dtype_code):
    """One token through entry point ``name`` on a copy of ``state``; returns (o, state)."""
    dev = "cuda"
    s_out = state.clone()
    o = torch.empty(B, H, K, device=dev, dtype=tok["q"].dtype)
    fs = (ctypes.c_int32 * L)(*f)
    nqs = (ctypes.c_int32 * (L - 1))(*([N] * (L - 1)))
    d = _lib.dims(B, 1, H, L, K, K, dtype_code, K ** -0.5)
    P = _lib.ptr
    args = [ctypes.byref(d), *(P(tok[n]) for n in STEP_IN), P(s_out), P(s_out), P(pos), 0, 64,
            fs, 0, nqs, P(par["qb"]), par["nmax"], P(par["kp"]), P(par["bpT"]), P(par["wpT"]),
            P(par["gpT"])]
    if name == "ngdn_step":
        ws = torch.empty(B * H * (3 * N * K + K), device=dev, dtype=torch.float32)
        args.append(P(ws))
    args += [P(o), _lib.stream_of(s_out)]
    _lib.call(name, *args)
    torch.cuda.synchronize()
    return o, s_out


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "f32"])
def test_step_noalloc_matches_step_twice(dtype):
    H, L, K, N, f = 2, 3, 128, 128, (1, 1, 2)
    code = _lib.NGDN_BF16 if dtype == torch.bfloat16 else _lib.NGDN_F32
    for B, seed in ((100, 1), (3, 2)):
        print(f"step_noalloc B={B} {dtype}", flush=True)
        inp = make_inputs(B=B, T=1, H=H, K=K, V=K, L=L, N=N, intervals=f, dtype=dtype, seed=seed)
        tok = {n: inp[n][:, 0].contiguous().cuda() for n in STEP_IN}
        tok["g"] = tok["g"].float()
        par = prepare_step_params(*(inp[n].cuda() for n in PARAMS), dtype)
        gen = torch.Generator().manual_seed(seed + 10)
        state = (torch.randn(B, H, L, K, K, generator=gen) * 0.5).cuda()
        # position 127 ends chunk 2: levels 1 and 2 fire; 126 fires nothing
        pos = torch.tensor([127 if b % 3 != 1 else 126 for b in range(B)], device="cuda")
        o_ref, s_ref = _call("ngdn_step", B, H, L, K, N, f, tok, par, state, pos, code)
        o, s = _call("ngdn_step_noalloc", B, H, L, K, N, f, tok, par, state, pos, code)
        assert torch.equal(o, o_ref), f"B={B}: o differs from ngdn_step"
        assert torch.equal(s, s_ref), f"B={B}: state differs from ngdn_step"
        fired = (s[:, :, 2] != state[:, :, 2]).flatten(1).any(1).cpu()
        assert fired.tolist() == [b % 3 != 1 for b in range(B)]


def test_step_noalloc_rejects_rows_larger_than_the_scratch():
    # H=200 heads at 128 pairs and K=128: one row needs 39.4 MB > 32 MiB
    B, H, L, K, N = 1, 200, 2, 128, 128
    t = torch.zeros(B * H * L * K * K + 8, device="cuda")
    fs = (ctypes.c_int32 * L)(1, 1)
    nqs = (ctypes.c_int32 * 1)(N)
    d = _lib.dims(B, 1, H, L, K, K, _lib.NGDN_F32, 0.1)
    P = ctypes.c_void_p(t.data_ptr())
    s_out = ctypes.c_void_p(t.data_ptr())
    rc = _lib.lib().ngdn_step_noalloc(ctypes.byref(d), *([P] * 7), P, s_out, None, 63, 64, fs, 0,
                                      nqs, P, N, P, P, P, P, P, _lib.stream_of(t))
    assert rc == 1
    assert b"scratch" in _lib.lib().ngdn_last_error()
