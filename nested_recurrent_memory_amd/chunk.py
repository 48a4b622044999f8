"""Chunkwise nested Gated DeltaNet on MI355X: the drop-in for the reference's
``nested_gdn2.ops.chunk.chunk_nested_gdn2`` (nested_gdn2/ops/chunk.py:722-766).

Same signature, argument conventions, errors and autograd contract as the
reference op; every arithmetic step runs in the HIP kernels of libngdn.so
(``csrc/``), reached through its C ABI. Python only validates, allocates
outputs and working buffers, and sequences the launches on torch's current
stream. There is no CPU or PyTorch fallback: without the built library or a
GPU the op raises.

Forward, per call (reference composition ops/chunk.py:159-304):
  ngdn_l0_intra_fwd    per-chunk level-0 terms, all chunks in parallel (on
                       small grids range by range, beside the scan)
  ngdn_l0_scan_fwd     level-0 state recurrence: states h per chunk, and
                       the level-0 read (Qg h + Aqk Vn) per row; the states
                       the level above reads (every f_1-th) when L > 1
  for each level l >= 1:
    ngdn_promote_chain_fwd  the level's firings in order per (batch, head):
                            gather, probe and update on chip, one state per
                            group stored (up to 64 pairs per firing), or
    ngdn_probe_fwd          probe the level below at this level's firings,
    ngdn_upper_scan_fwd     then this level's write scan (128 pairs)
  ngdn_output_upper_fwd  every upper read + mix over the scan's level-0
                       read, o written once
"""

from __future__ import annotations

import ctypes
import math

import torch

from . import _lib
from .schedule import n_firings, n_groups

__all__ = ["chunk_nested_gdn2", "ChunkNestedGDN2Function", "PROMOTIONS"]

PROMOTIONS = ("learned", "merge")
_SUPPORTED_KV = (64, 128)


def _as_ints(x, n):
    vals = [int(v) for v in (x.tolist() if torch.is_tensor(x) else list(x))]
    if len(vals) != n:
        raise ValueError(f"expected {n} entries, got {len(vals)}")
    return vals


def _working_dtype(q):
    if q.dtype == torch.bfloat16:
        return torch.bfloat16, _lib.NGDN_BF16
    # fp32 and fp16 run the fp32 kernels (fp16 -> fp32 is exact)
    return torch.float32, _lib.NGDN_F32


def _validate(q, k, v, L, chunk_size, promotion, n_queries, intervals, query_banks):
    if chunk_size != 64:
        raise ValueError(f"chunk_size must be 64 for GDN-2, got {chunk_size}")
    if promotion not in PROMOTIONS:
        raise ValueError(f"unknown promotion {promotion!r}; expected one of {PROMOTIONS}")
    if q.dim() != 5 or q.shape[3] != L:
        raise ValueError(f"q must be [B, T, H, L={L}, K], got {tuple(q.shape)}")
    B, T, H, _, K = q.shape
    V = v.shape[-1]
    if k.shape != (B, T, H, K) or v.shape[:3] != (B, T, H):
        raise ValueError("k must be [B, T, H, K] and v [B, T, H, V] matching q")
    if K not in _SUPPORTED_KV or V not in _SUPPORTED_KV:
        raise ValueError(f"head dims K={K}, V={V} unsupported; K and V must be 64 or 128")
    if L > 1 and K != V:
        raise ValueError(f"the promotion kernels need K == V, got K={K}, V={V} "
                         "(chunk_nested_gdn2 pads K != V to max(K, V) before this)")
    if L > 8:
        raise ValueError(f"at most 8 levels supported, got L={L}")
    if intervals[0] != 1:
        raise ValueError(f"firing_intervals[0] must be 1, got {intervals[0]}")
    if any(f <= 0 for f in intervals):
        raise ValueError(f"firing intervals must be positive, got {intervals}")
    for lvl in range(1, L):
        n = K if promotion == "merge" else n_queries[lvl - 1]
        if n < 16 or n & (n - 1) or n > 128:
            raise ValueError(f"pairs per firing must be a power of two >= 16, got {n}")
        if promotion == "learned" and n > query_banks.shape[2]:
            raise ValueError(
                f"n_queries={n} exceeds the {query_banks.shape[2]} rows of query_banks")


# Two forms of a level's promotions in the forward. Two launches (the
# default): a probe launch with one workgroup per (batch, head, firing), every
# firing at once, then the level's scan of updates per (batch, head, 32
# columns of V). Fused (True; levels with at most 64 pairs per firing, merge
# at K = 64): one launch per level (ngdn_promote_chain_fwd), one workgroup
# per (batch, head) running its firings in order with the probe and the
# update on chip. The fused form keeps the pairs off HBM but runs B H
# workgroups through a serial chain of firings; at the benchmark shapes the
# two-launch form is faster (c2: 6.67 against 6.91 ms per fwd+bwd step).
FUSED_PROMOTION = False

# The level-0 chunk backward as one launch (ngdn_l0_bwd: the state half per
# chunk in the same workgroup) or two (ngdn_l0_bwd_state, ngdn_l0_bwd_intra);
# read by the forward, which keeps U for the two-launch form only.
FUSED_L0_BWD = True
# dmix_0 (a bandwidth pass over do and the stored read) on the second side
# stream: at the fork, beside the reads' backward (False), or after the
# level-1 probe backward, beside the level-0 reverse scan (True: the reads'
# backward, which the top level's probe backward waits for, then shares the
# GPU with one kernel less; 6.14 -> 6.08 ms at c2)
DMIX0_LATE = True
# The reads' backward of the levels below the top one on the first side
# stream: beside the top level's (False), or after it, beside the top level's
# reverse scan and probe backward (True: the top level's reads backward,
# which starts the chain, then has the GPU to itself; at c2 0.234 -> 0.162
# ms, step 5.32-5.33 -> 5.30-5.31 ms)
READS_AFTER_TOP = True


# Small grids (a long sequence in a small batch: the bf16 level-0 scan then
# runs at most 128 workgroups of 16 columns, half the CUs or fewer): the
# level-0 chunk terms and scan run over L0_PARTS consecutive ranges of
# chunks (at least 64 chunks each), the chunk terms of a range on a side
# stream while the scan works through the range before it; the scan carries
# its state from range to range through the final state, so every chunk's
# arithmetic is that of one launch over all chunks. "Small" is the C
# library's own test for 16-column scan slices (a 32-column grid of at most
# 64 workgroups). Config 3 (T = 65536, B H = 16): 5.47 -> 5.01 ms per forward
# (4 ranges 5.16, 16 ranges 5.08).
L0_PARTS = 8


def _l0_ranges(B, H, V, NT, code):
    """Chunk ranges (c0, n) of the level-0 forward: one for a grid that
    fills the GPU, else up to L0_PARTS of at least 64 chunks."""
    narrow = code == _lib.NGDN_BF16 and B * H * (V // 32) <= 64
    parts = max(1, min(int(L0_PARTS), NT // 64)) if narrow else 1
    bounds = [NT * p // parts for p in range(parts + 1)]
    return [(bounds[p], bounds[p + 1] - bounds[p]) for p in range(parts)]


def _chain_ok(K, N, merge):
    if merge:
        return K == 64 and N == 64
    return K in (64, 128) and N in (16, 32, 64)


# Batch rows are independent all the way through the op, so the kernels run
# per group of batch rows, each group on its own stream: the sequential scans
# of one group (a few workgroups per CU, latency-bound) overlap the chunk
# kernels of another (throughput-bound) instead of leaving most of the GPU idle.
STREAM_GROUPS = 1
_STREAMS = {}


def _side_streams(dev, n):
    key = (dev.index if dev.index is not None else torch.cuda.current_device(), n)
    if key not in _STREAMS:
        _STREAMS[key] = [torch.cuda.Stream(device=dev) for _ in range(n)]   # default priority
    return _STREAMS[key]


def _aux_streams(dev):
    """Two streams (default priority) for independent launches inside one
    backward: the reads' backward next to the top level's scan, and the
    parameter-gradient sums next to the rest of the chain."""
    key = (dev.index if dev.index is not None else torch.cuda.current_device(), "aux")
    if key not in _STREAMS:
        _STREAMS[key] = [torch.cuda.Stream(device=dev) for _ in range(2)]
    return _STREAMS[key]


def _run_groups(B, dev, launch):
    """Calls launch(b0, nb, stream) for each group of batch rows: on the
    current stream when there is one group, else on side streams forked from
    and joined back into the current stream. Returns the number of groups."""
    n = max(1, min(STREAM_GROUPS, B))
    main = torch.cuda.current_stream(dev)
    if n == 1:
        launch(0, B, main)
        return 1
    size = -(-B // n)
    spans = [(b0, min(size, B - b0)) for b0 in range(0, B, size)]
    side = _side_streams(dev, len(spans))
    fork = main.record_event()
    for (b0, nb), st in zip(spans, side):
        st.wait_event(fork)
        with torch.cuda.stream(st):
            launch(b0, nb, st)
    for st in side[:len(spans)]:
        main.wait_stream(st)
    return len(spans)


def _rows(b0, nb):
    """View of batch rows [b0, b0 + nb) of a batch-leading tensor (None stays None)."""
    return lambda t: None if t is None else t[b0:b0 + nb]


def _fire_chunks(T, fire_partial):
    """Chunks whose end can complete an upper level's firing: every chunk,
    or (fire_partial False) the whole ones only, so that a partial last
    chunk fires nothing, as the decoding step treats an incomplete chunk
    (the library's ngdn_dims.hold_partial)."""
    NT = -(-T // 64)
    return NT if fire_partial else T // 64


def _forward(q, k, v, g, b, w, mix, qb, kp, bp, wp, gp, nq, f, L, scale,
             init, promotion, train, fire_partial=True):
    """Runs the forward kernels. Returns (o, final_state [B,H,L,K,V] fp32,
    working tensors kept for the backward when ``train``)."""
    B, T, H, _, K = q.shape
    V = v.shape[-1]
    dev = q.device
    wd, code = _working_dtype(q)
    NT = -(-T // 64)
    NTF = _fire_chunks(T, fire_partial)
    cvt = lambda x: x.to(wd).contiguous()  # noqa: E731
    q_, k_, v_, b_, w_, mix_ = (cvt(x) for x in (q, k, v, b, w, mix))
    g_ = g.to(torch.float32).contiguous()
    init_ = init.to(torch.float32).contiguous() if init is not None else None
    e = lambda *s, dt=wd: torch.empty(*s, device=dev, dtype=dt)  # noqa: E731
    # working tensors between the kernels are fp32 whatever the input dtype
    f32 = lambda *s: e(*s, dt=torch.float32)  # noqa: E731
    opt = lambda *s: f32(*s) if train else None  # noqa: E731

    # everything is allocated here, on the current stream, before any launch
    W, U, Qg = f32(B, H, NT, 64, K), f32(B, H, NT, 64, V), f32(B, H, NT, 64, K)
    KtT, Aqk = f32(B, H, NT, K, 64), f32(B, H, NT, 64, 64)
    gam = f32(B, H, NT, K)
    TT = opt(B, H, NT, 64, 64)
    # the state entering each chunk, transposed: read by level 1's probes at
    # every f1-th chunk only, so only those are written
    hT = f32(B, H, NT, V, K) if L > 1 else None
    h_, vn_ = opt(B, H, NT, K, V), opt(B, H, NT, 64, V)
    final = torch.empty(B, H, L, K, V, device=dev, dtype=torch.float32)
    states = [None] * L       # group states as rows [B,NG,H,K,V]
    statesT = [None] * L      # and transposed [B,NG,H,V,K]
    levels = [None] * L
    merge = promotion == "merge"
    par = {}
    if L > 1:
        par = _params(qb, kp, bp, wp, gp, wd, train)
    for lvl in range(1, L):
        nf, ng = n_firings(NTF, f[lvl]), n_groups(NT, f[lvl])
        N = K if merge else nq[lvl - 1]
        nf1 = max(nf, 1)
        if FUSED_PROMOTION and _chain_ok(K, N, merge):
            # one launch: probes and updates on chip; the backward's keys,
            # (keys b e^g)^T and e^g only when training
            levels[lvl] = dict(N=N, nf=nf, ng=ng, chain=True, gam=opt(B, H, nf1, K),
                               keys=opt(B, H, nf1, N, K), AT=opt(B, H, nf1, K, N))
        else:
            levels[lvl] = dict(N=N, nf=nf, ng=ng, chain=False, A=f32(B, H, nf1, N, K),
                               KT=f32(B, H, nf1, K, N), U=f32(B, H, nf1, N, V),
                               gam=f32(B, H, nf1, K), keys=opt(B, H, nf1, N, K),
                               AT=opt(B, H, nf1, K, N))
        states[lvl], statesT[lvl] = f32(B, ng, H, K, V), f32(B, ng, H, V, K)
    o = e(B, T, H, V)
    # level 0's read of every token, formed by the level-0 scan while each
    # chunk's state is on chip; the output pass adds the upper levels' reads
    # and the mix (and the backward's dmix_0 reads it again)
    read0 = f32(B, T, H, V)
    P = _lib.ptr

    def param_grads(d, lvl, sp, st):
        lv, wk = levels[lvl], work[lvl]
        ws = wk["ws"]
        _lib.call("ngdn_param_grads", ctypes.byref(d), lvl, int(merge), lv["N"], lv["nf"],
                  *(P(x) for x in ws[:5]), P(wk["dbank"]), par["nmax"], P(dqb), P(dkp),
                  P(dbp), P(dwp), P(dgp), P(parts), sp, tag=f"ngdn_param_grads.{lvl}",
                  stream=st)

    def launch(b0, nb, st):
        R = _rows(b0, nb)
        sp = _lib.ptr_of_stream(st)
        d = _lib.dims(nb, T, H, L, K, V, code, scale, hold_partial=NTF < NT)
        ranges = _l0_ranges(nb, H, V, NT, code) if nb == B else [(0, NT)]
        ts = _aux_streams(dev)[0] if len(ranges) > 1 else st
        if ts is not st:
            ts.wait_event(st.record_event())
        # every range's chunk terms queued at once on the side stream (holding
        # them to one or two ranges ahead of the scan measured slower)
        ready = []
        for c0, n in ranges:
            _lib.call("ngdn_l0_intra_fwd", ctypes.byref(d), *(P(R(x)) for x in (
                q_, k_, v_, g_, b_, w_, W, U, KtT, Qg, Aqk, gam, TT)), c0, n,
                _lib.ptr_of_stream(ts), stream=ts)
            ready.append(ts.record_event() if ts is not st else None)
        # with several ranges and unfused promotions, the upper levels follow
        # on a second side stream, one range behind: after level-0 range p,
        # each level probes and scans the firings whose lower state is stored
        tu = (_aux_streams(dev)[1] if len(ranges) > 1 and L > 1
              and not any(levels[lvl]["chain"] for lvl in range(1, L)) else None)
        done = [0] * L          # firings of each level probed and scanned so far
        for p, (c0, n) in enumerate(ranges):
            if ready[p] is not None:
                st.wait_event(ready[p])
            # a range after the first starts from the state the one before left in final
            _lib.call("ngdn_l0_scan_fwd", ctypes.byref(d), *(P(R(x)) for x in (
                W, U, KtT, gam, Qg, Aqk, init_ if p == 0 else final)), f[1] if L > 1 else 1,
                *(P(R(x)) for x in (hT, None, h_, vn_, read0, final)), c0, n, sp)
            if tu is not None:
                tu.wait_event(st.record_event())
                upper_batch(d, R, done, c0 + n, p == len(ranges) - 1, tu)
        if tu is not None:
            st.wait_event(tu.record_event())
        else:
            upper_batch(d, R, done, NT, True, st)
        spT, ngs, fs = _level_arrays([R(x) for x in statesT], NT, f, L)
        _lib.call("ngdn_output_upper_fwd", ctypes.byref(d), P(R(read0)), P(R(q_)),
                  P(R(mix_)), spT, ngs, fs, P(R(o)), sp)

    def upper_batch(d, R, done, avail, last, su):
        """Probes and scans of every upper level for the firings whose lower
        state is stored: level 0 has stored the states entering chunks
        [0, avail); each level then has stored the groups entering its firings
        so far. A firing i reads the lower level's stored state
        ((i + 1) f_here) / f_below, so the firings with (i + 1) f_here <
        avail f_below are ready; the last batch takes the rest (including
        those that read the lower final state) and stores every level's
        trailing groups. d and R: the launch's dims and batch rows; su: the
        stream."""
        sp = _lib.ptr_of_stream(su)
        for lvl in range(1, L):
            lv = levels[lvl]
            fh, fb = f[lvl], f[lvl - 1]
            nf = lv["nf"]
            upto = nf if last else min(nf, max(0, (avail * fb - 1) // fh))
            i0 = done[lvl]
            if lv["chain"]:
                belowT, ngb = (hT, NT) if lvl == 1 else (statesT[lvl - 1], n_groups(NT, fb))
                _lib.call("ngdn_promote_chain_fwd", ctypes.byref(d), lvl, int(merge), lv["N"], fb,
                          fh, P(R(belowT)), ngb, P(R(final)), P(par["qb"]), par["nmax"],
                          P(par["kp"]), P(par["bpT"]), P(par["wpT"]), P(par["gpT"]), P(R(init_)),
                          P(R(states[lvl])), P(R(statesT[lvl])),
                          *(P(R(lv[x])) for x in ("keys", "AT", "gam")), sp,
                          tag=f"ngdn_promote_chain_fwd.{lvl}")
                continue
            below, ngb = (hT, NT) if lvl == 1 else (states[lvl - 1], n_groups(NT, fb))
            if upto > i0:
                _lib.call("ngdn_probe_fwd", ctypes.byref(d), lvl, int(merge), lv["N"], fb, fh,
                          P(R(below)), ngb, P(R(final)), P(par["qb"]), par["nmax"],
                          P(par["kp"]), P(par["bpT"]), P(par["wpT"]), P(par["gpT"]),
                          *(P(R(lv[x])) for x in ("A", "KT", "U", "gam", "keys", "AT")),
                          None, None, None, None, None, i0, upto - i0, sp,
                          tag=f"ngdn_probe_fwd.{lvl}", stream=su)
            if upto > i0 or (last and nf == 0):
                # a range after the level's first starts from the state in final
                _lib.call("ngdn_upper_scan_fwd", ctypes.byref(d), lvl, lv["N"], nf, lv["ng"],
                          *(P(R(lv[x])) for x in ("A", "KT", "U", "gam")),
                          P(R(init_ if i0 == 0 else final)),
                          P(R(states[lvl])), P(R(statesT[lvl])), P(R(final)), i0, upto - i0, sp,
                          tag=f"ngdn_upper_scan_fwd.{lvl}", stream=su)
            done[lvl] = upto
            # the groups of this level stored so far bound the level above's firings
            avail = upto

    _run_groups(B, dev, launch)
    saved = None
    if train:
        # U only for the two-launch chunk backward (the fused one forms dA
        # from Vn instead)
        saved = dict(q=q_, k=k_, v=v_, b=b_, w=w_, mix=mix_, g=g_, W=W,
                     U=None if FUSED_L0_BWD else U, Qg=Qg,
                     KtT=KtT, Aqk=Aqk, gam=gam, TT=TT, NTF=NTF,
                     hT=hT, h=h_, vn=vn_, read0=read0, states=states,
                     statesT=statesT, levels=levels, final=final, par=par,
                     code=code, wd=wd)
    return o, final, saved


def _params(qb, kp, bp, wp, gp, wd, train):
    """Per-level parameters in the layouts the kernels read: originals, the
    projections with their last two axes swapped, and (for the backward) the
    bank and key projections transposed. The bank is padded to a multiple of
    8 rows so every row start is 16-byte aligned."""
    nmax = qb.shape[2]
    nmax8 = -(-nmax // 8) * 8
    qb_ = qb.to(wd)
    if nmax8 != nmax:
        qb_ = torch.nn.functional.pad(qb_, (0, 0, 0, nmax8 - nmax))
    c = lambda x: x.to(wd).contiguous()  # noqa: E731
    qb_, kp_, bp_, wp_, gp_ = (c(x) for x in (qb_, kp, bp, wp, gp))
    # the transposes in one launch
    tr = _transpose_last2([bp_, wp_, gp_] + ([kp_, qb_] if train else []))
    par = dict(qb=qb_, nmax=nmax8, kp=kp_, bpT=tr[0], wpT=tr[1], gpT=tr[2])
    if train:
        par.update(kpT=tr[3], bankT=tr[4], bp=bp_, wp=wp_, gp=gp_)
    return par


def _transpose_last2(xs):
    """Contiguous tensors of one dtype transposed in their last two axes
    (ngdn_transpose: one launch on the current stream)."""
    if any(not x.is_contiguous() or x.dtype != xs[0].dtype or x.dim() < 2 for x in xs):
        raise ValueError("_transpose_last2: contiguous tensors of one dtype, at least 2-D")
    outs = [torch.empty(x.shape[:-2] + (x.shape[-1], x.shape[-2]), device=x.device, dtype=x.dtype)
            for x in xs]
    n = len(xs)
    _lib.call("ngdn_transpose", n, (ctypes.c_void_p * n)(*(x.data_ptr() for x in xs)),
              (ctypes.c_void_p * n)(*(y.data_ptr() for y in outs)),
              (ctypes.c_int32 * n)(*(x.numel() // max(1, x.shape[-1] * x.shape[-2]) for x in xs)),
              (ctypes.c_int32 * n)(*(x.shape[-2] for x in xs)),
              (ctypes.c_int32 * n)(*(x.shape[-1] for x in xs)),
              xs[0].element_size(), _lib.stream_of(xs[0]))
    return outs


def _level_arrays(states, NT, f, L):
    sp = (ctypes.c_void_p * L)(*([None] + [s.data_ptr() for s in states[1:]]))
    ngs = (ctypes.c_int32 * L)(*([0] + [n_groups(NT, f[l]) for l in range(1, L)]))
    fs = (ctypes.c_int32 * L)(*f)
    return sp, ngs, fs


def _backward(sv, do, dfinal, L, scale, f, nq, has_init, promotion):
    """Runs the backward kernels (ops/chunk.py:374-564, mirrored). Returns the
    gradients in the working dtype (fp32 for g, the states and parameters)."""
    q_, k_, v_, b_, w_, mix_, g_ = (sv[n] for n in ("q", "k", "v", "b", "w", "mix", "g"))
    B, T, H, _, K = q_.shape
    V = v_.shape[-1]
    dev = q_.device
    wd, code = sv["wd"], sv["code"]
    NT = -(-T // 64)
    P = _lib.ptr
    e = lambda *s, dt=wd: torch.empty(*s, device=dev, dtype=dt)  # noqa: E731
    f32 = lambda *s: e(*s, dt=torch.float32)  # noqa: E731
    z32 = lambda *s: torch.zeros(*s, device=dev, dtype=torch.float32)  # noqa: E731
    do_ = do.to(wd).contiguous()
    merge = promotion == "merge"
    states, levels, par, final = sv["states"], sv["levels"], sv["par"], sv["final"]

    # everything is allocated (and zeroed) here, on the current stream; the
    # buffers that start at zero share one allocation and one fill
    zshapes = ([] if dfinal is not None else [(B, H, L, K, V)]) + \
        ([(B, H, L, K, V)] if has_init else []) + \
        ([(L - 1, H, par["nmax"], K), (L - 1, H, K, V), (L - 1, H, V, K), (L - 1, H, V, V),
          (L - 1, H, V, K)] if L > 1 else [])
    zsizes = [math.prod(sh) for sh in zshapes]
    zbuf = z32(sum(zsizes)) if zshapes else None
    zviews, off = [], 0
    for sh, n in zip(zshapes, zsizes):
        zviews.append(zbuf[off:off + n].view(sh))
        off += n
    zit = iter(zviews)
    dq = e(B, T, H, L, K)
    dmix = f32(B, T, H, L)
    d_final = (dfinal.to(torch.float32).contiguous().clone() if dfinal is not None
               else next(zit))
    d_init = next(zit) if has_init else None
    d_states = [None] + [f32(B, n_groups(NT, f[lvl]), H, K, V) for lvl in range(1, L)]
    dqb = dkp = dbp = dwp = dgp = None
    work = [None] * L
    if L > 1:
        dqb, dkp, dbp, dwp, dgp = (next(zit) for _ in range(5))
    for lvl in range(1, L):
        lv = levels[lvl]
        N, nf = lv["N"], lv["nf"]
        nfa = max(nf, 1)
        work[lvl] = dict(dSp=f32(B, H, nfa, K, V), dvn=f32(B, H, nfa, N, V),
                         ws=[f32(B, H, nfa, N, K) for _ in range(4)]
                         + [f32(B, H, nfa, N, V) for _ in range(2)],
                         dbank=None if merge else f32(B, H, nfa, N, K),
                         inj=f32(B, H, nfa, K, V))
    # per-slice partials of the parameter-gradient sums, shared by the levels
    # (their sums run one after another on one stream)
    parts = f32(4, H, _lib.PARAM_SPLIT, K, V) if L > 1 else None
    dSp0, dVnT0 = f32(B, H, NT, K, V), f32(B, H, NT, V, 64)
    # dQg, dKt: the fused chunk backward's workspaces; the rest only for the
    # two-launch form
    dQg, dKt = f32(B, H, NT, 64, K), f32(B, H, NT, 64, K)
    dVn0 = dWT = dAqk = dgam = None
    # the form the forward saved for (U is kept only for the two-launch form)
    fused_l0 = sv["U"] is None
    # small grids, one group of rows, the fused chunk backward: the level-0
    # reverse scan runs the chunk ranges of the forward last first, the
    # gradient of the state between ranges carried in l0_carry, and each
    # range's chunk backward runs on a side stream beside the scan of the
    # range before it
    l0_ranges = (_l0_ranges(B, H, V, NT, code)
                 if fused_l0 and max(1, min(STREAM_GROUPS, B)) == 1 else [(0, NT)])
    l0_carry = f32(B, H, L, K, V) if len(l0_ranges) > 1 else None
    if not fused_l0:
        dVn0, dWT = f32(B, H, NT, 64, V), f32(B, H, NT, K, 64)
        dAqk, dgam = f32(B, H, NT, 64, 64), f32(B, H, NT, K)
    dk, dv, db, dw = e(B, T, H, K), e(B, T, H, V), e(B, T, H, K), e(B, T, H, V)
    dg = f32(B, T, H, K)

    def param_grads(d, lvl, sp, st):
        lv, wk = levels[lvl], work[lvl]
        ws = wk["ws"]
        _lib.call("ngdn_param_grads", ctypes.byref(d), lvl, int(merge), lv["N"], lv["nf"],
                  *(P(x) for x in ws[:5]), P(wk["dbank"]), par["nmax"], P(dqb), P(dkp),
                  P(dbp), P(dwp), P(dgp), P(parts), sp, tag=f"ngdn_param_grads.{lvl}",
                  stream=st)

    def launch(b0, nb, st):
        R = _rows(b0, nb)
        sp = _lib.ptr_of_stream(st)
        d = _lib.dims(nb, T, H, L, K, V, code, scale, hold_partial=sv["NTF"] < NT)
        # With one group of rows, independent launches go to two side streams:
        # (a) the reads' backward of the levels below the top one
        # (each writes its own columns of dmix and dq and its own d_states)
        # beside the top level's reverse scan and probe backward (after the
        # top level's read, or beside it when READS_AFTER_TOP is off; the
        # probe backward's lower-state gradient goes to an injection, not
        # into d_states),
        # joined before the first reverse scan that reads those d_states; (b) each
        # level's parameter-gradient sums (reading only that level's
        # workspaces) and dmix_0 (before level 1's sums, or at the fork when
        # DMIX0_LATE is off) beside the rest of the chain, joined at the end. With
        # several groups of rows the sums run once over all rows after the
        # groups join, so every row group's partials are in place and the
        # result does not depend on the grouping.
        aux = _aux_streams(dev) if (L > 1 and nb == B) else None
        if aux is not None:
            fork = st.record_event()
            for a in aux:
                a.wait_event(fork)
        ta, tb = (aux[0], aux[1]) if aux else (st, st)
        sa, sb = _lib.ptr_of_stream(ta), _lib.ptr_of_stream(tb)
        # reads: dmix for every level (level 0 from the stored read, on the
        # second side stream), dq and the group-state gradients for levels >= 1
        dmix0_done = []

        def dmix0():
            _lib.call("ngdn_output_bwd", ctypes.byref(d), P(R(sv["read0"])), P(R(do_)),
                      P(R(dmix)), sb, stream=tb)
            dmix0_done.append(True)
        if not (DMIX0_LATE and aux is not None):
            dmix0()
        late = READS_AFTER_TOP and aux is not None
        for lvl in ([L - 1] + list(range(1, L - 1)) if late else range(1, L)):
            ng = n_groups(NT, f[lvl])
            top = lvl == L - 1
            _lib.call("ngdn_read_state_bwd", ctypes.byref(d), lvl, f[lvl], ng,
                      *(P(R(x)) for x in (q_, mix_, do_, states[lvl], d_states[lvl], dq, dmix)),
                      sp if top else sa, tag=f"ngdn_read_state_bwd.{lvl}", stream=st if top else ta)
            if late and top:
                aux[0].wait_stream(st)
        joined = aux is None
        inj, nf1 = None, 0
        for lvl in range(L - 1, 0, -1):
            lv, wk = levels[lvl], work[lvl]
            N, nf, ng = lv["N"], lv["nf"], lv["ng"]
            if not joined and lvl < L - 1:
                st.wait_stream(aux[0])
                joined = True
            # the level above's injection (its probe backward's lower-state
            # gradients), added by this level's reverse scan
            up = lvl + 1 < L and levels[lvl + 1]["nf"] > 0
            _lib.call("ngdn_upper_scan_bwd", ctypes.byref(d), lvl, N, nf, ng,
                      *(P(R(x)) for x in (lv["keys"], lv["AT"], lv["gam"], d_states[lvl])),
                      P(R(work[lvl + 1]["inj"])) if up else None, f[lvl],
                      f[lvl + 1] if up else 1, levels[lvl + 1]["nf"] if up else 0,
                      *(P(R(x)) for x in (d_final, wk["dSp"], wk["dvn"], d_init)),
                      sp, tag=f"ngdn_upper_scan_bwd.{lvl}")
            if nf == 0:
                continue
            fh, fb = f[lvl], f[lvl - 1]
            if lvl == 1:
                inj, nf1 = wk["inj"], nf
                b_kv, b_vk, ngb = sv["h"], sv["hT"], NT
            else:
                b_kv, b_vk = states[lvl - 1], sv["statesT"][lvl - 1]
                ngb = n_groups(NT, fb)
            ws = wk["ws"]
            _lib.call("ngdn_probe_bwd", ctypes.byref(d), lvl, int(merge), N, fb, fh,
                      P(R(b_kv)), P(R(b_vk)), ngb, P(R(final)), P(par["qb"]), par["nmax"],
                      P(par["kp"]), P(par["bpT"]), P(par["wpT"]), P(par["gpT"]),
                      P(par["kpT"]), P(par["bankT"]), P(par["bp"]), P(par["wp"]),
                      P(par["gp"]), P(R(states[lvl])), P(R(sv["statesT"][lvl])), ng,
                      P(R(wk["dSp"])), P(R(wk["dvn"])), *(P(R(x)) for x in ws),
                      P(R(wk["dbank"])), P(R(wk["inj"])), P(R(d_final)), sp,
                      tag=f"ngdn_probe_bwd.{lvl}")
            if nb == B:
                if aux is not None:
                    aux[1].wait_stream(st)
                if DMIX0_LATE and aux is not None and lvl == 1:
                    dmix0()
                param_grads(d, lvl, sb, tb)
        if not joined:
            st.wait_stream(aux[0])
        if not dmix0_done:
            # (late placement) after the upper levels' parameter-gradient sums
            dmix0()
        # level 0
        ranges = l0_ranges if nb == B else [(0, NT)]
        tl = _aux_streams(dev)[0] if len(ranges) > 1 else st
        for p in reversed(range(len(ranges))):
            c0, n = ranges[p]
            last = p == len(ranges) - 1
            _lib.call("ngdn_l0_scan_bwd", ctypes.byref(d), *(P(R(sv[x])) for x in (
                "W", "KtT", "gam", "Qg", "Aqk")), P(R(do_)), P(R(mix_)), f[1] if L > 1 else 1,
                P(R(inj)), nf1, P(R(d_final if last else l0_carry)), P(R(dSp0)), P(R(dVn0)),
                P(R(dVnT0)), P(R(d_init if p == 0 else l0_carry)), c0, n, sp)
            if fused_l0:
                # the chunk backward in one launch: the state half per chunk
                if tl is not st:
                    tl.wait_event(st.record_event())
                _lib.call("ngdn_l0_bwd", ctypes.byref(d), *(P(R(x)) for x in (
                    q_, k_, v_, g_, b_, w_, sv["TT"], sv["h"], dSp0, sv["vn"],
                    dVnT0, do_, mix_, dQg, dKt, dq, dk, dv, dg, db, dw)), c0, n,
                    _lib.ptr_of_stream(tl), stream=tl)
        if tl is not st:
            st.wait_stream(tl)
        if not fused_l0:
            _lib.call("ngdn_l0_bwd_state", ctypes.byref(d), P(R(sv["h"])), P(R(dSp0)),
                      P(R(sv["vn"])), P(R(dVn0)), P(R(do_)), P(R(mix_)),
                      *(P(R(x)) for x in (dQg, dWT, dKt, dAqk, dgam)), sp)
            _lib.call("ngdn_l0_bwd_intra", ctypes.byref(d), *(P(R(x)) for x in (
                q_, k_, v_, g_, b_, w_, sv["W"], sv["U"], sv["TT"], dQg, dWT, dKt, dAqk, dgam,
                dVnT0, dq, dk, dv, dg, db, dw)), sp)
        if aux is not None:
            st.wait_stream(aux[1])

    groups = _run_groups(B, dev, launch)
    if groups > 1:
        st = torch.cuda.current_stream(dev)
        d = _lib.dims(B, T, H, L, K, V, code, scale, hold_partial=sv["NTF"] < NT)
        for lvl in range(L - 1, 0, -1):
            if levels[lvl]["nf"] > 0:
                param_grads(d, lvl, _lib.ptr_of_stream(st), st)
    return dq, dk, dv, dg, db, dw, dmix, dqb, dkp, dbp, dwp, dgp, d_init


def _flatten(x, tensors):
    """x with every tensor replaced by its index in ``tensors`` (appended)."""
    if isinstance(x, torch.Tensor):
        tensors.append(x)
        return _Slot(len(tensors) - 1)
    if isinstance(x, dict):
        return {k: _flatten(v, tensors) for k, v in x.items()}
    if isinstance(x, list):
        return [_flatten(v, tensors) for v in x]
    return x


def _unflatten(x, tensors):
    if isinstance(x, _Slot):
        return tensors[x.i]
    if isinstance(x, dict):
        return {k: _unflatten(v, tensors) for k, v in x.items()}
    if isinstance(x, list):
        return [_unflatten(v, tensors) for v in x]
    return x


class _Slot:
    __slots__ = ("i",)

    def __init__(self, i):
        self.i = i


class ChunkNestedGDN2Function(torch.autograd.Function):
    """Autograd node for the whole op (ops/chunk.py:567-719)."""

    @staticmethod
    def forward(ctx, q, k, v, g, b, w, mix_weights, query_banks, key_projections,
                b_projections, w_projections, g_projections, n_queries_per_level,
                firing_intervals, L, scale, initial_state, output_final_state,
                chunk_size, promotion, fire_partial_chunk=True):
        L = int(L)
        f = _as_ints(firing_intervals, L)
        nq = _as_ints(n_queries_per_level, L - 1) if L > 1 else []
        _validate(q, k, v, L, chunk_size, promotion, nq, f, query_banks)
        if not q.is_cuda:
            raise RuntimeError("chunk_nested_gdn2 runs on the GPU only; got CPU tensors")
        K = q.shape[-1]
        if scale is None:
            scale = K ** -0.5
        # the backward's extra layouts are written only when a gradient is wanted
        train = any(ctx.needs_input_grad)
        o, final, saved = _forward(q, k, v, g, b, w, mix_weights, query_banks,
                                   key_projections, b_projections, w_projections,
                                   g_projections, nq, f, L, scale, initial_state,
                                   promotion, train, fire_partial_chunk)
        o = o.to(q.dtype)
        ctx.meta = (L, scale, f, nq, initial_state is not None, promotion)
        ctx.dtypes = [None if t is None else t.dtype
                      for t in (q, k, v, g, b, w, mix_weights, query_banks, key_projections,
                                b_projections, w_projections, g_projections, initial_state)]
        ctx.nmax = query_banks.shape[2] if L > 1 else 0
        # the working tensors go through save_for_backward, so that activation
        # checkpointing (torch.utils.checkpoint) can drop them after the
        # forward and have them recomputed for the backward
        tensors = []
        ctx.skeleton = _flatten(saved, tensors)
        ctx.save_for_backward(*tensors)
        return o, (final if output_final_state else None)

    @staticmethod
    def backward(ctx, do, dfinal):
        L, scale, f, nq, has_init, promotion = ctx.meta
        sv = _unflatten(ctx.skeleton, ctx.saved_tensors)
        if sv is None:
            raise RuntimeError("chunk_nested_gdn2: no saved state for the backward")
        grads = _backward(sv, do, dfinal, L, scale, f, nq, has_init, promotion)
        (dq, dk, dv, dg, db, dw, dmix, dqb, dkp, dbp, dwp, dgp, dinit) = grads
        dts = ctx.dtypes
        grads = [dq, dk, dv, dg, db, dw, dmix] + ([dqb, dkp, dbp, dwp, dgp] if L > 1 else [])
        out = _cast_grads(grads, dts[:len(grads)])
        if L > 1:
            if out[7].shape[2] != ctx.nmax:
                out[7] = out[7][:, :, :ctx.nmax]      # drop the alignment padding rows
        else:
            out += [None] * 5
        return (*out, None, None, None, None,
                dinit.to(dts[12]) if dinit is not None else None, None, None, None, None)


def _cast_grads(grads, dtypes):
    """The gradients in their inputs' dtypes. The fp32 -> bf16 casts (dg,
    dmix, the parameter sums for bf16 inputs) run in one launch into
    separately allocated tensors, which autograd takes as the leaves'
    gradients without copying them (views of one shared buffer it copies);
    the rest cast with torch."""
    out = list(grads)
    batch = [i for i, (x, dt) in enumerate(zip(grads, dtypes))
             if x is not None and x.dtype == torch.float32 and dt == torch.bfloat16
             and x.is_contiguous()]
    if len(batch) > 1:
        for i in batch:
            out[i] = torch.empty(grads[i].shape, device=grads[i].device, dtype=torch.bfloat16)
        n = len(batch)
        srcs = (ctypes.c_void_p * n)(*(grads[i].data_ptr() for i in batch))
        dsts = (ctypes.c_void_p * n)(*(out[i].data_ptr() for i in batch))
        cnt = (ctypes.c_int64 * n)(*(grads[i].numel() for i in batch))
        _lib.call("ngdn_cast_bf16", n, srcs, dsts, cnt, _lib.stream_of(grads[batch[0]]))
    else:
        batch = []
    return [x if x is None or i in batch else x.to(dt)
            for i, (x, dt) in enumerate(zip(out, dtypes))]


def chunk_nested_gdn2(q, k, v, g, b, w, mix_weights, query_banks, key_projections,
                      b_projections, w_projections, g_projections, n_queries_per_level,
                      firing_intervals, L, scale=None, initial_state=None,
                      output_final_state=False, chunk_size=64, promotion="learned",
                      fire_partial_chunk=True):
    """Differentiable chunkwise NestedGDN-2. Signature matches the reference op
    (nested_gdn2/ops/chunk.py:722-743) and its naive twin (ops/naive.py:226-247).

    Returns (o [B, T, H, V] in q's dtype, final_state [B, H, L, K, V] fp32 or None).

    ``fire_partial_chunk`` (an addition; the reference's chunk form always
    fires): with False, a partial last chunk completes no upper level's
    firing, as the reference's decoding step treats an incomplete chunk
    (ops/naive.py:101-113). The op then gives, for any T, what the reference
    layer computes by running whole chunks through the chunk op and stepping
    the rest (layers/nested_gdn2.py:196-224), differentiable throughout.

    K != V with upper levels (the layer's expand_v != 1) runs the K = V
    kernels at D = max(K, V) on zero-padded inputs and parameters: the padded
    channels stay exactly zero through every level and carry no gradient into
    the real ones, so the results are those of the unpadded op (see
    ``pad_kv``).
    """
    K, V = q.shape[-1], v.shape[-1]
    if int(L) > 1 and K != V:
        if promotion == "merge" and K < V:
            raise ValueError(f"merge promotion with K < V (K={K}, V={V}) is not supported: "
                             "its decay is a mean over K pairs")
        (q, k, v, g, b, w, query_banks, key_projections, b_projections, w_projections,
         g_projections, initial_state) = pad_kv(
            K, V, q=q, k=k, v=v, g=g, b=b, w=w, query_banks=query_banks,
            key_projections=key_projections, b_projections=b_projections,
            w_projections=w_projections, g_projections=g_projections,
            initial_state=initial_state)
        o, fin = ChunkNestedGDN2Function.apply(
            q, k, v, g, b, w, mix_weights, query_banks, key_projections, b_projections,
            w_projections, g_projections, n_queries_per_level, firing_intervals, L,
            K ** -0.5 if scale is None else scale, initial_state, output_final_state,
            chunk_size, promotion, fire_partial_chunk)
        return o[..., :V], (fin[..., :K, :V] if fin is not None else None)
    return ChunkNestedGDN2Function.apply(
        q, k, v, g, b, w, mix_weights, query_banks, key_projections, b_projections,
        w_projections, g_projections, n_queries_per_level, firing_intervals, L,
        scale, initial_state, output_final_state, chunk_size, promotion, fire_partial_chunk)


def pad_kv(K, V, *, q=None, k=None, v=None, g=None, b=None, w=None, query_banks=None,
           key_projections=None, b_projections=None, w_projections=None, g_projections=None,
           initial_state=None, state=None):
    """The op's tensors zero-padded to D = max(K, V) in their K and V axes
    (None stays None), in the order of the keywords. With K < V the key axis
    grows: q, k, b, g and the bank get zero channels, so those channels of
    the decay-masked products, of W, Kt, Qg and of every state row stay zero
    (their decay e^0 = 1 keeps a zero row zero), and the write keys
    u = Vals Wk^T get zero columns (the norm is unchanged). With V < K the
    value axis grows: v and w get zero channels, so U, Vn, the states'
    columns and Vals stay zero there, and the zero rows of the b, g, w
    projections keep the gates of the real channels unchanged. Gradients
    reaching the padded channels are zero or are dropped by the padding's
    backward. (Merge with K < V would average its decay over D pairs instead
    of K: refused by the caller.)"""
    D = max(K, V)
    pk, pv = D - K, D - V
    F = torch.nn.functional

    def last(t, p):
        return t if t is None or p == 0 else F.pad(t, (0, p))

    def last2(t, p_row, p_col):
        return t if t is None or (p_row == 0 and p_col == 0) else F.pad(t, (0, p_col, 0, p_row))

    out = [last(q, pk), last(k, pk), last(v, pv), last(g, pk), last(b, pk), last(w, pv),
           last(query_banks, pk), last2(key_projections, pk, pv),
           last2(b_projections, pv, pk), last2(w_projections, pv, pv),
           last2(g_projections, pv, pk), last2(initial_state, pk, pv)]
    if state is not None:
        out.append(last2(state, pk, pv))
    return out


def default_scale(K: int) -> float:
    return 1.0 / math.sqrt(K)
