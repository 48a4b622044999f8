"""CPU restatement of the reference's Nested Gated DeltaNet op -- TEST INFRASTRUCTURE.

This module is the checker, never the product. Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it. The shipped op (``nested_recurrent_memory_amd``) never imports it and
has no CPU fallback.

Everything here is plain PyTorch on the CPU, written from the mathematics of
the reference (awehrs/nested_recurrent_memory, ``nested_gdn2/ops``), and runs
in any float dtype; the tests use float64 so that a comparison measures the
HIP kernels, not this file. Each function cites the reference lines whose
behaviour it restates.

Pinning (how each function is checked, see ``tests/test_oracle.py``):
  * schedule            -- hand-enumerated tables, exact integers.
  * update_step         -- N=1 closed form (rank-one delta rule), pair-order
                           invariance, merge losslessness, golden vectors.
  * probe_learned/merge -- gate offsets with zero projections (sigma(-4),
                           sigma(0), -softplus(-4)), unit-norm keys, mean-over-
                           pairs decay, bank permutation, ignored rows, golden
                           vectors.
  * chunk_forward       -- token-by-token recurrence (``recurrent_forward``)
                           in float64, L=1 against an independent dense rank-one
                           loop, prefill + step == one pass, golden vectors.
  * l0_chunk_terms      -- rebuilt token-by-token inside the chunk (brute force)
                           and against ``chunk_forward``'s level-0 output.
  * gradients           -- float64 autograd through these functions plus
                           ``torch.autograd.gradcheck`` at tiny shapes.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

__all__ = [
    "B_LOGIT_INIT", "W_LOGIT_INIT", "G_LOGIT_INIT",
    "n_groups", "n_firings", "source_index",
    "update_step", "update_scan", "gates", "probe_learned", "probe_merge",
    "PROBES", "step_forward", "recurrent_forward", "chunk_forward",
    "l0_chunk_terms",
]

# Gate logit offsets (ops/probe.py:28-31).
B_LOGIT_INIT = -4.0
W_LOGIT_INIT = 0.0
G_LOGIT_INIT = -4.0


# --------------------------------------------------------------------------
# Integer schedule (ops/chunk.py:26-55)
# --------------------------------------------------------------------------

def n_groups(n_chunks: int, interval: int) -> int:
    """Groups of ``interval`` chunks covering ``n_chunks``; the last may be
    short and never fires (ops/chunk.py:26-31)."""
    return -(-n_chunks // interval)


def n_firings(n_chunks: int, interval: int) -> int:
    """One firing per complete group (ops/chunk.py:34-36)."""
    return n_chunks // interval


def source_index(f_below: int, f_here: int, n_chunks: int) -> list[int]:
    """Group of the level below whose entering state the i-th firing of this
    level reads; an index equal to the lower level's group count means its
    final state (ops/chunk.py:39-55, gather at :58-93)."""
    return [(i + 1) * f_here // f_below for i in range(n_firings(n_chunks, f_here))]


# --------------------------------------------------------------------------
# One firing of the delta rule (ops/naive.py:7-39)
# --------------------------------------------------------------------------

def update_step(S, keys, vals, b, w, g):
    """All N pairs act on the decayed pre-firing state at once.

    S [..., K, V]; keys, b [..., N, K]; vals, w [..., N, V]; g [..., K].
    S' = e^g*S - keys^T ((keys*b) (e^g*S)) + keys^T (vals*w).
    """
    Sd = S * torch.exp(g).unsqueeze(-1)
    kt = keys.transpose(-1, -2)
    erased = kt @ ((keys * b) @ Sd)
    written = kt @ (vals * w)
    return Sd - erased + written


def update_scan(keys, vals, g, b, w, groups: int, init=None):
    """One level's write scan (ops/update_fwd.py:131-204 contract; the test
    helper tests/ops/_update_ref.py:111-128): the state entering each group is
    stored, then the group's firing (if any) is applied.

    keys, b [B, NF, H, N, K]; vals, w [B, NF, H, N, V]; g [B, NF, H, K].
    Returns states [B, NG, H, K, V] and the final state [B, H, K, V].
    """
    B, NF, H, _, K = keys.shape
    V = vals.shape[-1]
    S = init if init is not None else vals.new_zeros(B, H, K, V)
    out = []
    for j in range(groups):
        out.append(S)
        if j < NF:
            S = update_step(S, keys[:, j], vals[:, j], b[:, j], w[:, j], g[:, j])
    return torch.stack(out, 1), S


# --------------------------------------------------------------------------
# Promotion probes (ops/probe.py:34-142)
# --------------------------------------------------------------------------

def gates(vals, b_proj, w_proj, g_proj):
    """b, w per pair and g per firing, projected from the values written
    (ops/probe.py:34-66). vals [B, NF, H, N, V]; b_proj, g_proj [H, V, K];
    w_proj [H, V, V]. g is the mean over pairs of -softplus."""
    dt = vals.dtype
    xb = torch.einsum("bfhnv,hvk->bfhnk", vals, b_proj.to(dt))
    xw = torch.einsum("bfhnv,hvu->bfhnu", vals, w_proj.to(dt))
    xg = torch.einsum("bfhnv,hvk->bfhnk", vals, g_proj.to(dt))
    b = torch.sigmoid(xb + B_LOGIT_INIT)
    w = torch.sigmoid(xw + W_LOGIT_INIT)
    g = -F.softplus(xg + G_LOGIT_INIT).mean(dim=-2)
    return b, w, g


def probe_learned(S_below, bank, key_proj, b_proj, w_proj, g_proj, n_queries):
    """Read the lower state with the first ``n_queries`` bank rows, derive
    unit-norm keys from the values read (ops/probe.py:69-102).

    S_below [B, NF, H, K, V]; bank [H, Nmax, K]; key_proj [H, K, V].
    """
    dt = S_below.dtype
    Q = bank[:, :n_queries].to(dt)
    vals = torch.einsum("hnk,bfhkv->bfhnv", Q, S_below)
    u = torch.einsum("bfhnv,hkv->bfhnk", vals, key_proj.to(dt))
    keys = u / u.norm(dim=-1, keepdim=True).clamp_min(1e-12)
    b, w, g = gates(vals, b_proj, w_proj, g_proj)
    return keys, vals, b, w, g


def probe_merge(S_below, bank, key_proj, b_proj, w_proj, g_proj, n_queries=None):
    """Carry the lower state up row by row: identity keys, values = the state
    (ops/probe.py:105-136). bank and key_proj are not read."""
    B, NF, H, K, _ = S_below.shape
    eye = torch.eye(K, dtype=S_below.dtype)
    b, w, g = gates(S_below, b_proj, w_proj, g_proj)
    return eye.expand(B, NF, H, K, K), S_below, b, w, g


PROBES = {"learned": probe_learned, "merge": probe_merge}


# --------------------------------------------------------------------------
# Token form (ops/naive.py:42-223)
# --------------------------------------------------------------------------

def step_forward(q, k, v, g, b, w, mix, state, position, bank, key_proj,
                 b_proj, w_proj, g_proj, n_queries, intervals, L,
                 scale=None, chunk_size=64, promotion="learned"):
    """One token (ops/naive.py:42-134): level 0 writes, all levels are read
    and mixed, then every level whose firing this token completes promotes,
    bottom-up, in rows whose position ends such a firing.

    q [B, H, L, K]; k, g, b [B, H, K]; v, w [B, H, V]; mix [B, H, L];
    state [B, H, L, K, V]; position int or [B] long.
    Returns o [B, H, V] and the new state, both in the working dtype.
    """
    if scale is None:
        scale = q.shape[-1] ** -0.5
    dt = state.dtype
    q, k, v, g, b, w, mix = (x.to(dt) for x in (q, k, v, g, b, w, mix))
    S = list(state.unbind(2))
    S[0] = update_step(S[0], k.unsqueeze(2), v.unsqueeze(2), b.unsqueeze(2),
                       w.unsqueeze(2), g)
    reads = torch.stack(
        [torch.einsum("bhk,bhkv->bhv", q[:, :, l] * scale, S[l]) for l in range(L)],
        dim=2,
    )
    o = (reads * mix.unsqueeze(-1)).sum(2)

    Bsz = k.shape[0]
    pos = (position if torch.is_tensor(position)
           else torch.full((Bsz,), int(position), dtype=torch.long))
    end = pos + 1
    boundary = (end % chunk_size) == 0
    chunk_no = end // chunk_size
    probe = PROBES[promotion]
    for lvl in range(1, L):
        rows = torch.nonzero(boundary & (chunk_no % int(intervals[lvl]) == 0)).flatten()
        if rows.numel() == 0:
            continue
        keys, vals, bp, wp, gp = probe(
            S[lvl - 1][rows].unsqueeze(1), bank[lvl - 1], key_proj[lvl - 1],
            b_proj[lvl - 1], w_proj[lvl - 1], g_proj[lvl - 1],
            int(n_queries[lvl - 1]),
        )
        new = update_step(S[lvl][rows], keys[:, 0], vals[:, 0], bp[:, 0],
                          wp[:, 0], gp[:, 0])
        S[lvl] = S[lvl].index_copy(0, rows, new)
    return o, torch.stack(S, 2)


def recurrent_forward(q, k, v, g, b, w, mix, bank, key_proj, b_proj, w_proj,
                      g_proj, n_queries, intervals, L, scale=None,
                      initial_state=None, chunk_size=64, promotion="learned",
                      dtype=torch.float64):
    """Token-by-token pass over [B, T, H, ...] inputs (ops/naive.py:137-223).
    Returns o [B, T, H, V] and the final state [B, H, L, K, V] in ``dtype``."""
    cast = lambda x: x.to(dtype)  # noqa: E731
    q, k, v, g, b, w, mix = map(cast, (q, k, v, g, b, w, mix))
    B, T, H, K = k.shape
    V = v.shape[-1]
    state = (cast(initial_state).clone() if initial_state is not None
             else torch.zeros(B, H, L, K, V, dtype=dtype))
    outs = []
    for t in range(T):
        o_t, state = step_forward(
            q[:, t], k[:, t], v[:, t], g[:, t], b[:, t], w[:, t], mix[:, t],
            state, t, bank, key_proj, b_proj, w_proj, g_proj, n_queries,
            intervals, L, scale=scale, chunk_size=chunk_size, promotion=promotion)
        outs.append(o_t)
    return torch.stack(outs, 1), state


# --------------------------------------------------------------------------
# Chunk form (ops/naive.py:226-420; composition ops/chunk.py:159-304)
# --------------------------------------------------------------------------

def l0_chunk_terms(q0, k, v, g, b, w, scale):
    """Per-chunk level-0 quantities of the chunk form (ops/naive.py:329-358).

    Inputs carry any leading dims followed by [NT, C, K] (q0, k, g, b) or
    [NT, C, V] (v, w), already zero-padded to whole chunks; q0 is unscaled.
    Returns a dict of
      gc   [.., NT, C, K]  in-chunk cumulative log decay
      A    [.., NT, C, C]  strictly lower sum_k b_i k_i k_j e^(gc_i - gc_j)
      T    [.., NT, C, C]  (I + A)^-1
      W    [.., NT, C, K]  T (b * k * e^gc)
      U    [.., NT, C, V]  T (w * v)
      Kt   [.., NT, C, K]  k * e^(gc_last - gc)
      Qg   [.., NT, C, K]  scale * q0 * e^gc
      Aqk  [.., NT, C, C]  causal (diagonal included) sum_k scale q_i k_j e^(gc_i - gc_j)
      gam  [.., NT, K]     e^gc_last
    Exponents are clamped at 0 before exp, as the reference does (:335-336,354);
    with g <= 0 the clamp only touches entries the masks discard.
    """
    C = k.shape[-2]
    gc = torch.cumsum(g, dim=-2)
    diff = (gc.unsqueeze(-2) - gc.unsqueeze(-3)).clamp(max=0.0)   # [.., i, j, K]
    dec = torch.exp(diff)
    strict = torch.tril(torch.ones(C, C, dtype=torch.bool), -1)
    causal = torch.tril(torch.ones(C, C, dtype=torch.bool), 0)
    A = torch.einsum("...ik,...jk,...ijk->...ij", b * k, k, dec) * strict
    qs = q0 * scale
    Aqk = torch.einsum("...ik,...jk,...ijk->...ij", qs, k, dec) * causal
    eye = torch.eye(C, dtype=k.dtype)
    T = torch.linalg.inv(eye + A)
    W = T @ (b * k * torch.exp(gc))
    U = T @ (w * v)
    last = gc[..., -1:, :]
    Kt = k * torch.exp(last - gc)
    Qg = qs * torch.exp(gc)
    return dict(gc=gc, A=A, T=T, W=W, U=U, Kt=Kt, Qg=Qg, Aqk=Aqk,
                gam=torch.exp(last[..., 0, :]))


def chunk_forward(q, k, v, g, b, w, mix, bank, key_proj, b_proj, w_proj,
                  g_proj, n_queries, intervals, L, scale=None,
                  initial_state=None, output_final_state=False, chunk_size=64,
                  promotion="learned", dtype=torch.float64, out_dtype=None):
    """The whole op in chunk form (ops/naive.py:226-420).

    Per chunk n: level 0's output from its chunk closed form, every level >= 1
    read with the state it held entering the chunk, the mix, level 0's state
    update, then each level with (n+1) % f == 0 fires bottom-up reading the
    level below as it now stands. T is zero-padded to whole chunks and a
    partial last chunk fires like a full one (ops/chunk.py:232).

    Computes in ``dtype``; o is returned in ``out_dtype`` (default: q's dtype),
    the final state in ``dtype``.
    """
    if out_dtype is None:
        out_dtype = q.dtype
    if scale is None:
        scale = q.shape[-1] ** -0.5
    C = chunk_size
    B, T, H, K = k.shape
    V = v.shape[-1]
    NT = -(-T // C)
    pad = NT * C - T

    def prep(x):
        # [B, T, H, ...] -> [B, H, NT, C, ...] in the working dtype
        x = x.to(dtype).transpose(1, 2)
        if pad:
            x = F.pad(x, (0, 0) * (x.dim() - 3) + (0, pad))
        return x.reshape(B, H, NT, C, *x.shape[3:])

    q, k, v, g, b, w, mix = map(prep, (q, k, v, g, b, w, mix))
    t = l0_chunk_terms(q[..., 0, :], k, v, g, b, w, scale)
    S = [(initial_state[:, :, l].to(dtype).clone() if initial_state is not None
          else torch.zeros(B, H, K, V, dtype=dtype)) for l in range(L)]
    probe = PROBES[promotion]
    chunks = []
    for n in range(NT):
        vn = t["U"][:, :, n] - t["W"][:, :, n] @ S[0]
        reads = [t["Aqk"][:, :, n] @ vn + t["Qg"][:, :, n] @ S[0]]
        for l in range(1, L):
            reads.append((q[:, :, n, :, l] * scale) @ S[l])
        mixn = mix[:, :, n]                                   # [B, H, C, L]
        chunks.append(sum(mixn[..., l:l + 1] * reads[l] for l in range(L)))
        S[0] = (t["gam"][:, :, n].unsqueeze(-1) * S[0]
                + t["Kt"][:, :, n].transpose(-1, -2) @ vn)
        for l in range(1, L):
            if (n + 1) % int(intervals[l]) != 0:
                continue
            keys, vals, bp, wp, gp = probe(
                S[l - 1].unsqueeze(1), bank[l - 1], key_proj[l - 1],
                b_proj[l - 1], w_proj[l - 1], g_proj[l - 1], int(n_queries[l - 1]))
            S[l] = update_step(S[l], keys[:, 0], vals[:, 0], bp[:, 0], wp[:, 0],
                               gp[:, 0])
    o = torch.stack(chunks, 2).reshape(B, H, NT * C, V)[:, :, :T]
    o = o.transpose(1, 2).to(out_dtype)
    final = torch.stack(S, 2) if output_final_state else None
    return o, final


def default_scale(K: int) -> float:
    return 1.0 / math.sqrt(K)
