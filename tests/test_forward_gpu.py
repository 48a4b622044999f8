"""Forward parity of the HIP path against the CPU oracle (float64).

Tolerances (written into every assertion): fp32 inputs 1e-5; bf16 inputs
max-abs 2e-3 / rel 1e-2 against the fp32-or-better oracle on identical inputs.
"""

import ctypes

import pytest
import torch

import _golden
import ngdn_oracle as ref
from nested_recurrent_memory_amd import _lib, chunk_nested_gdn2
from nested_recurrent_memory_amd.inputs import NAMES, make_inputs

pytestmark = pytest.mark.gpu

TOL = {torch.float32: dict(rtol=1e-5, atol=1e-5),
       torch.bfloat16: dict(rtol=1e-2, atol=2e-3)}


# working tensors read as matrix-core operands only: for bf16 inputs each
# per-chunk tile [R][C] holds two bf16 planes (hi, then lo) in the bytes of
# the fp32 tile
SPLIT = ("W", "KtT", "Qg", "Aqk")
# for bf16 every split tile is stored in fragment order: per plane, block
# (rb, cb) of 16 rows x 32 columns at 512 (rb C/32 + cb), element (r, c) of
# the block at 8 (16 (c // 8) + r) + c % 8
FRAG = SPLIT


def _unfrag(p, R, C):
    """[..., R*C] in fragment order -> [..., R, C] row-major."""
    x = p.reshape(*p.shape[:-1], R // 16, C // 32, 4, 16, 8)
    n = x.dim()
    x = x.permute(*range(n - 5), n - 5, n - 2, n - 4, n - 3, n - 1)
    return x.reshape(*p.shape[:-1], R, C)


def _unsplit(t, frag=False):
    R, C = t.shape[-2:]
    planes = t.contiguous().view(torch.bfloat16).reshape(*t.shape[:-2], 2, R * C)
    planes = _unfrag(planes, R, C) if frag else planes.reshape(*t.shape[:-2], 2, R, C)
    planes = planes.float()
    return planes[..., 0, :, :] + planes[..., 1, :, :]


def _gpu(inp):
    return {n: inp[n].to("cuda") for n in NAMES}


def _oracle(inp, L, promotion="learned", init=None):
    return ref.chunk_forward(*[inp[n] for n in NAMES], L=L, initial_state=init,
                             output_final_state=True, promotion=promotion,
                             out_dtype=torch.float64)


# ------------------------------------------------------------- level-0 chunk terms

@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("K,V,T,g_scale", [(64, 64, 192, 0.1), (128, 128, 130, 1.0),
                                           (64, 128, 128, 30.0), (128, 64, 64, 2.0)])
def test_l0_intra_terms(dtype, K, V, T, g_scale):
    print(f"l0_intra dtype={dtype} K={K} V={V} T={T} g_scale={g_scale}", flush=True)
    B, H, L = 2, 2, 1
    inp = make_inputs(B=B, T=T, H=H, K=K, V=V, L=L, N=16, intervals=(1,), dtype=dtype,
                      g_scale=g_scale)
    NT = -(-T // 64)
    scale = K ** -0.5
    code = _lib.NGDN_BF16 if dtype == torch.bfloat16 else _lib.NGDN_F32
    g = {n: inp[n].to("cuda").contiguous() for n in ("q", "k", "v", "g", "b", "w")}
    # the per-chunk terms are fp32 working tensors whatever the input dtype
    e = lambda *s: torch.empty(*s, device="cuda", dtype=torch.float32)  # noqa: E731
    out = dict(W=e(B, H, NT, 64, K), U=e(B, H, NT, 64, V), KtT=e(B, H, NT, K, 64),
               Qg=e(B, H, NT, 64, K), Aqk=e(B, H, NT, 64, 64), gam=e(B, H, NT, K),
               TT=e(B, H, NT, 64, 64))
    d = _lib.dims(B, T, H, L, K, V, code, scale)
    P = _lib.ptr
    _lib.call("ngdn_l0_intra_fwd", ctypes.byref(d), *(P(g[n]) for n in ("q", "k", "v", "g", "b", "w")),
              *(P(out[n]) for n in ("W", "U", "KtT", "Qg", "Aqk", "gam")),
              P(out["TT"]), 0, NT, _lib.stream_of(g["q"]))
    torch.cuda.synchronize()

    pad = NT * 64 - T

    def prep(x):
        x = x.double().transpose(1, 2)
        if pad:
            x = torch.nn.functional.pad(x, (0, 0) * (x.dim() - 3) + (0, pad))
        return x.reshape(B, H, NT, 64, *x.shape[3:])
    t = ref.l0_chunk_terms(prep(inp["q"])[..., 0, :], prep(inp["k"]), prep(inp["v"]),
                           prep(inp["g"]), prep(inp["b"]), prep(inp["w"]), scale)
    tol = TOL[dtype]
    got = {n: (_unsplit(out[n], n in FRAG) if dtype == torch.bfloat16 and n in SPLIT else out[n])
           .double().cpu() for n in out}
    torch.testing.assert_close(got["gam"], t["gam"], rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(got["Aqk"], t["Aqk"], **tol)
    torch.testing.assert_close(got["Qg"], t["Qg"], **tol)
    torch.testing.assert_close(got["KtT"], t["Kt"].transpose(-1, -2), **tol)
    torch.testing.assert_close(got["W"], t["W"], **tol)
    torch.testing.assert_close(got["U"], t["U"], **tol)
    torch.testing.assert_close(got["TT"], t["T"].transpose(-1, -2), **tol)
    # the split form is hi = bf16(x), lo = bf16(x - hi), both round-to-nearest-
    # even: lo is at most half an ulp of hi
    if dtype == torch.bfloat16:
        for n in SPLIT:
            R, C = out[n].shape[-2:]
            pl = out[n].contiguous().view(torch.bfloat16).reshape(*out[n].shape[:-2], 2, R, C)
            hi, lo = pl[..., 0, :, :].float().cpu(), pl[..., 1, :, :].float().cpu()
            assert (lo.abs() <= 2.0 ** -8 * hi.abs()).all(), n


# ------------------------------------------------------------- whole forward

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
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("promotion", ["learned", "merge"])
@pytest.mark.parametrize("B,T,H,K,L,N,firing,nq", CASES)
def test_forward_matches_oracle(B, T, H, K, L, N, firing, nq, promotion, dtype):
    print(f"forward B={B} T={T} H={H} K={K} L={L} N={N} f={firing} nq={nq} "
          f"{promotion} {dtype}", flush=True)
    inp = make_inputs(B=B, T=T, H=H, K=K, V=K, L=L, N=N, intervals=firing, n_queries=nq,
                      dtype=dtype, g_scale=1.0, style="reftest")
    o, s = chunk_nested_gdn2(**_gpu(inp), L=L, output_final_state=True, promotion=promotion)
    o_ref, s_ref = _oracle(inp, L, promotion)
    torch.testing.assert_close(o.double().cpu(), o_ref, **TOL[dtype])
    torch.testing.assert_close(s.double().cpu(), s_ref, **TOL[dtype])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("K,V,T", [(64, 128, 192), (128, 64, 100)])
def test_forward_single_level_k_ne_v(dtype, K, V, T):
    """One level with value width != key width (the layer's expand_v != 1)."""
    print(f"forward L=1 K={K} V={V} T={T} {dtype}", flush=True)
    inp = make_inputs(B=2, T=T, H=2, K=K, V=V, L=1, N=16, intervals=(1,), dtype=dtype,
                      g_scale=1.0, style="reftest")
    gen = torch.Generator().manual_seed(9)
    init = torch.randn(2, 2, 1, K, V, generator=gen) * 0.1
    o, s = chunk_nested_gdn2(**_gpu(inp), L=1, initial_state=init.cuda(), output_final_state=True)
    o_ref, s_ref = _oracle(inp, 1, init=init.double())
    torch.testing.assert_close(o.double().cpu(), o_ref, **TOL[dtype])
    torch.testing.assert_close(s.double().cpu(), s_ref, **TOL[dtype])


def _nan_tailed(x):
    """x on the GPU at the start of a buffer whose remaining 64 KiB hold NaN:
    a kernel that reads past the end of the sequence picks them up."""
    n = x.numel()
    pad = 65536 // x.element_size()
    buf = torch.full((n + pad,), float("nan"), dtype=x.dtype, device="cuda")
    buf[:n].copy_(x.reshape(-1).cuda())
    return buf[:n].view(x.shape)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("T,K", [(200, 64), (100, 128), (80, 64)])
def test_partial_last_chunk_reads_nothing_past_the_end(dtype, T, K):
    """Every input ends exactly at the sequence end (B=1) with NaN after it:
    the forward and backward must not read past the last token."""
    print(f"past-the-end T={T} K={K} {dtype}", flush=True)
    inp = make_inputs(B=1, T=T, H=2, K=K, V=K, L=3, N=16, intervals=(1, 1, 2), dtype=dtype,
                      g_scale=1.0, style="reftest")
    leaves = ("q", "k", "v", "g", "b", "w", "mix_weights")
    dev = {n: (_nan_tailed(inp[n]) if n in leaves else inp[n].cuda()) for n in NAMES}
    for n in leaves:
        dev[n].requires_grad_(True)
    o, s = chunk_nested_gdn2(**dev, L=3, output_final_state=True)
    o_ref, s_ref = _oracle(inp, 3)
    torch.testing.assert_close(o.double().cpu(), o_ref, **TOL[dtype])
    torch.testing.assert_close(s.double().cpu(), s_ref, **TOL[dtype])
    # the backward over the same buffers gives what it gives on plain copies
    do = torch.randn(o.shape, generator=torch.Generator().manual_seed(3)).to(o.dtype).cuda()
    (o.float() * do.float()).sum().backward()
    plain = {n: (inp[n].cuda().requires_grad_(True) if n in leaves else inp[n].cuda())
             for n in NAMES}
    o2, _ = chunk_nested_gdn2(**plain, L=3, output_final_state=True)
    (o2.float() * do.float()).sum().backward()
    for n in leaves:
        assert torch.isfinite(dev[n].grad).all(), n
        torch.testing.assert_close(dev[n].grad, plain[n].grad, **TOL[dtype])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("promotion", ["learned", "merge"])
def test_forward_with_initial_state(dtype, promotion):
    inp = make_inputs(B=2, T=256, H=2, K=64, V=64, L=3, N=16, intervals=(1, 2, 4),
                      dtype=dtype, g_scale=0.5)
    gen = torch.Generator().manual_seed(5)
    init = torch.randn(2, 2, 3, 64, 64, generator=gen) * 0.1
    o, s = chunk_nested_gdn2(**_gpu(inp), L=3, initial_state=init.cuda(),
                             output_final_state=True, promotion=promotion)
    o_ref, s_ref = _oracle(inp, 3, promotion, init=init.double())
    torch.testing.assert_close(o.double().cpu(), o_ref, **TOL[dtype])
    torch.testing.assert_close(s.double().cpu(), s_ref, **TOL[dtype])


@pytest.mark.parametrize("name", ["c0", "l3_learned", "l3_merge", "l2_bf16"])
def test_forward_golden(name):
    """Against the vectors the reference's own naive op produced (float32)."""
    cfg, inp, init, promotion, exp, _ = _golden.load(name)
    o, s = chunk_nested_gdn2(**_gpu(inp), L=cfg["L"],
                             initial_state=init.cuda() if init is not None else None,
                             output_final_state=True, promotion=promotion)
    tol = TOL[cfg["dtype"]]
    if exp["o"].dtype == torch.bfloat16:
        # both sides round to bf16 once; allow one bf16 ulp beyond the tolerance
        torch.testing.assert_close(o.float().cpu(), exp["o"].float(), rtol=1.5e-2, atol=2e-3)
    else:
        torch.testing.assert_close(o.float().cpu(), exp["o"], **tol)
    torch.testing.assert_close(s.cpu(), exp["final_state"], **tol)


def test_l1_config0_and_large_decay():
    """Config 0 (single level, fp32) and the reference's large-decay regime."""
    for g_scale in (0.1, 16.0):
        inp = make_inputs(B=1, T=512, H=2, K=64, V=64, L=1, N=16, intervals=(1,),
                          dtype=torch.float32, g_scale=g_scale)
        o, s = chunk_nested_gdn2(**_gpu(inp), L=1, output_final_state=True)
        o_ref, s_ref = _oracle(inp, 1)
        assert torch.isfinite(o).all() and torch.isfinite(s).all()
        torch.testing.assert_close(o.double().cpu(), o_ref, **TOL[torch.float32])
        torch.testing.assert_close(s.double().cpu(), s_ref, **TOL[torch.float32])


# ------------------------------------------------------------- fused promotion

@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("K,L,N,firing,promotion,T", [
    (64, 3, 16, (1, 2, 4), "learned", 320), (128, 3, 64, (1, 4, 16), "learned", 1100),
    (64, 2, 32, (1, 1), "learned", 200), (64, 3, 64, (1, 2, 3), "merge", 450),
    (128, 2, 32, (1, 3), "learned", 512)])
def test_fused_promotion_matches_two_launch_path(dtype, K, L, N, firing, promotion, T):
    """ngdn_promote_chain_fwd (the level's firings in one launch, on chip)
    against ngdn_probe_fwd + ngdn_upper_scan_fwd on the same inputs, with an
    initial state: outputs and final state within the op's bar (the two
    paths round differently: the fused one scales the state by e^g first)."""
    from nested_recurrent_memory_amd import chunk as chunk_mod
    print(f"fused promotion K={K} L={L} N={N} f={firing} {promotion} T={T} {dtype}", flush=True)
    inp = make_inputs(B=2, T=T, H=2, K=K, V=K, L=L, N=N, intervals=firing, dtype=dtype,
                      g_scale=0.5)
    gen = torch.Generator().manual_seed(3)
    init = (torch.randn(2, 2, L, K, K, generator=gen) * 0.2).cuda()
    g = _gpu(inp)
    outs = {}
    try:
        for fused in (True, False):
            chunk_mod.FUSED_PROMOTION = fused
            with torch.no_grad():
                outs[fused] = chunk_nested_gdn2(**g, L=L, initial_state=init,
                                                output_final_state=True, promotion=promotion)
    finally:
        chunk_mod.FUSED_PROMOTION = False
    torch.cuda.synchronize()
    tol = TOL[dtype]
    torch.testing.assert_close(outs[True][0].float(), outs[False][0].float(), **tol)
    torch.testing.assert_close(outs[True][1], outs[False][1], **tol)
    o_ref, s_ref = _oracle(inp, L, promotion, init=init.double().cpu())
    torch.testing.assert_close(outs[True][0].double().cpu(), o_ref, **tol)
    torch.testing.assert_close(outs[True][1].double().cpu(), s_ref, **tol)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_two_row_groups_equal_one(dtype):
    """The batch rows launched in two groups on two streams give the one-group
    result bit for bit (every kernel's arithmetic per (batch, head) is the
    same)."""
    from nested_recurrent_memory_amd import chunk as chunk_mod
    inp = make_inputs(B=2, T=700, H=2, K=128, V=128, L=3, N=64, intervals=(1, 2, 4),
                      dtype=dtype, g_scale=0.5)
    g = _gpu(inp)
    outs = []
    try:
        for groups in (1, 2):
            chunk_mod.STREAM_GROUPS = groups
            with torch.no_grad():
                outs.append(chunk_nested_gdn2(**g, L=3, output_final_state=True))
    finally:
        chunk_mod.STREAM_GROUPS = 1
    torch.cuda.synchronize()
    assert torch.equal(outs[0][0], outs[1][0])
    assert torch.equal(outs[0][1], outs[1][1])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("L", [1, 3])
def test_output_entry_points_agree(dtype, L):
    """The op forms level 0's read inside the level-0 scan and adds the upper
    levels' in ngdn_output_upper_fwd. The stand-alone output kernels
    (ngdn_output_fwd, and ngdn_output_l0_fwd + ngdn_output_upper_fwd) read the
    chunk states and Vn from HBM instead: called through the C ABI on the
    op's own working tensors they give the op's o within the bar."""
    from nested_recurrent_memory_amd import chunk as chunk_mod
    B, T, H, K = 2, 320, 2, 64
    inp = make_inputs(B=B, T=T, H=H, K=K, V=K, L=L, N=16, intervals=(1, 2, 4)[:L],
                      dtype=dtype, g_scale=0.5)
    g = _gpu(inp)
    leaves = {n: g[n] for n in NAMES}
    wd, code = chunk_mod._working_dtype(g["q"])
    f = (1, 2, 4)[:L]
    nq = [16] * (L - 1)
    with torch.no_grad():
        o, _ = chunk_nested_gdn2(**leaves, L=L, output_final_state=True)
        # the forward's working tensors, with every chunk's state and Vn^T stored
        q_, k_, v_, b_, w_, mix_ = (leaves[n].to(wd).contiguous() for n in
                                    ("q", "k", "v", "b", "w", "mix_weights"))
        g_ = leaves["g"].float().contiguous()
        NT = -(-T // 64)
        e = lambda *sh: torch.empty(*sh, device="cuda", dtype=torch.float32)  # noqa: E731
        W, U, KtT, Qg, Aqk, gam = (e(B, H, NT, 64, K), e(B, H, NT, 64, K), e(B, H, NT, K, 64),
                                   e(B, H, NT, 64, K), e(B, H, NT, 64, 64), e(B, H, NT, K))
        hT, vnT, read0 = e(B, H, NT, K, K), e(B, H, NT, K, 64), e(B, T, H, K)
        final = e(B, H, L, K, K)
        d = _lib.dims(B, T, H, L, K, K, code, K ** -0.5)
        P = _lib.ptr
        st = _lib.stream_of(q_)
        _lib.call("ngdn_l0_intra_fwd", ctypes.byref(d), *(P(x) for x in (
            q_, k_, v_, g_, b_, w_, W, U, KtT, Qg, Aqk, gam)), None, 0, NT, st)
        _lib.call("ngdn_l0_scan_fwd", ctypes.byref(d), *(P(x) for x in (W, U, KtT, gam, None, None,
                  None)), 1, P(hT), P(vnT), None, None, None, P(final), 0, NT, st)
        # upper levels' group states: from the op's own path (states of levels >= 1)
        saved = chunk_mod._forward(*(leaves[n] for n in NAMES[:12]), nq, list(f), L,
                                   K ** -0.5, None, "learned", True)[2]
        statesT = saved["statesT"]
        spT, ngs, fs = chunk_mod._level_arrays(statesT, NT, list(f), L)
        o1 = torch.empty_like(o)
        _lib.call("ngdn_output_fwd", ctypes.byref(d), *(P(x) for x in (Qg, Aqk, hT, vnT, q_, mix_)),
                  spT, ngs, fs, P(o1), None, st)
        _lib.call("ngdn_output_l0_fwd", ctypes.byref(d), *(P(x) for x in (Qg, Aqk, hT, vnT, read0)), st)
        o2 = torch.empty_like(o)
        _lib.call("ngdn_output_upper_fwd", ctypes.byref(d), P(read0), P(q_), P(mix_), spT, ngs, fs,
                  P(o2), st)
    torch.cuda.synchronize()
    tol = TOL[dtype]
    torch.testing.assert_close(o1.float(), o.float(), **tol)
    torch.testing.assert_close(o2.float(), o.float(), **tol)
