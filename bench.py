"""Benchmark of the nested GDN op, forward + backward, on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c2]

A step is one forward and one backward of ``chunk_nested_gdn2`` over one
batch of synthetic inputs at the configuration BASELINE.json quotes its
metric on (c2: B=4, T=8192, H=16, K=V=128, 3 levels firing every 1/4/16
chunks, 64 queries per level, bf16 inputs, fp32 state). Inputs are already
resident in HBM when the timed region starts. Prints one JSON line.

The line carries:
  roofline      the dominant kernel (entry point) of the step: its algorithmic
                bytes or flops per launch divided by its average launch time,
                timed with events on the launch stream over the timed region;
                ``traffic`` is its measured HBM bytes per launch from the
                committed counter profile of the configuration
                (profiles/ngdn_fwd_bwd_<config>_traffic.md), null without one;
  cpu_baseline  the CPU restatement (oracle/ngdn_oracle.py, float32 PyTorch)
                timed on a bounded sample of the same workload, extrapolated.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from nested_recurrent_memory_amd import _lib, chunk_nested_gdn2  # noqa: E402
from nested_recurrent_memory_amd.inputs import CONFIGS, LEAVES  # noqa: E402
from nested_recurrent_memory_amd.schedule import n_firings, n_groups  # noqa: E402

HBM_PEAK_GBS = 8000.0            # MI355X HBM3E, GB/s
MFMA_BF16_TFLOPS = 2500.0        # dense bf16
MFMA_FP32_TFLOPS = 157.3


# The reference's published rows (benchmarks/bench_matched.py:49-52,77-110,
# results/h100/depth.csv): firings 1, 2, 4 ..., queries min(8 * 2^l, d) per
# level, the harness's own input distributions. "ref3" is its depth row at
# d=128, L=3 (H100: forward 10.40 ms, forward+backward 44.46 ms, 13.42 GB).
REF_SHAPES = {
    "ref3": dict(B=4, T=8192, H=16, K=128, V=128, L=3, N=32, n_queries=(16, 32),
                 intervals=(1, 2, 4), dtype=torch.bfloat16, g_scale=1.0, style="reftest"),
}


def gpu_inputs(cfg, seed=0):
    """Inputs of the configuration's distributions, drawn on the GPU: the
    benchmark configurations' (``baseline``), or the reference harness's
    (``reftest``: q ~ N(0,1), v = 0.5 N(0,1), g = logsigmoid(N(0,1)) in the
    input dtype, b, w ~ U(0,1); bench_matched.py:77-110)."""
    B, T, H, K, V, L, N = (cfg[x] for x in ("B", "T", "H", "K", "V", "L", "N"))
    dt = cfg["dtype"]
    g = torch.Generator(device="cuda").manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g, device="cuda", dtype=torch.float32)  # noqa: E731
    u = lambda *s: torch.rand(*s, generator=g, device="cuda", dtype=torch.float32)  # noqa: E731
    F = torch.nn.functional
    nq = tuple(cfg.get("n_queries") or [N] * (L - 1))
    inp = dict(
        q=F.normalize(r(B, T, H, L, K), dim=-1).to(dt),
        k=F.normalize(r(B, T, H, K), dim=-1).to(dt),
        v=r(B, T, H, V).to(dt),
        g=-F.softplus(r(B, T, H, K)) * cfg["g_scale"],
        b=torch.sigmoid(r(B, T, H, K)).to(dt),
        w=torch.sigmoid(r(B, T, H, V)).to(dt),
        mix_weights=torch.softmax(r(B, T, H, L), dim=-1).to(dt),
        query_banks=(r(L - 1, H, max(nq, default=1), K) * K ** -0.5).to(dt),
        key_projections=(r(L - 1, H, K, V) * V ** -0.5).to(dt),
        b_projections=(r(L - 1, H, V, K) * V ** -0.5).to(dt),
        w_projections=(r(L - 1, H, V, V) * V ** -0.5).to(dt),
        g_projections=(r(L - 1, H, V, K) * V ** -0.5).to(dt),
        n_queries_per_level=nq,
        firing_intervals=tuple(cfg["intervals"]),
    )
    if cfg.get("style") == "reftest":
        inp.update(q=r(B, T, H, L, K).to(dt), v=(r(B, T, H, V) * 0.5).to(dt),
                   g=F.logsigmoid(r(B, T, H, K)).to(dt).float(),
                   b=u(B, T, H, K).to(dt), w=u(B, T, H, V).to(dt))
    return inp


def work_model(cfg):
    """Work per launch of each entry point at cfg (one fwd+bwd step), as
    (algorithmic bytes, design bytes, flops).

    Algorithmic bytes count only op-level tensors, each once at its op-level
    size: the op's inputs and parameters, its outputs (o, final state), the
    output gradient do, the gradients it returns, and the state sequences
    the op saves for its backward (level-0 chunk states h and upper group
    states, fp32) with their gradients (dh, d_states). Tensors that exist only
    between this build's kernels (W, U, T, Qg, Aqk, Kt, Vn and their
    gradients, transposed copies, per-firing pairs) are not counted there.
    Design bytes count every tensor the kernel reads and writes once, as this
    kernel split lays it out. Flops are dense tile products, 2 m n k."""
    B, T, H, K, V, L, N = (cfg[x] for x in ("B", "T", "H", "K", "V", "L", "N"))
    f = cfg["intervals"]
    es = 2 if cfg["dtype"] == torch.bfloat16 else 4   # inputs, parameters, gradients
    C = 64
    NT = -(-T // C)
    units = B * H * NT                       # chunk-heads
    ck, cv, cc = C * K * es, C * V * es, C * C * es   # input tiles of one chunk
    gk = C * K * 4                                    # g and dg (fp32) of one chunk
    wk, wv, wc = C * K * 4, C * V * 4, C * C * 4      # fp32 working tiles
    kv = K * V * 4                                    # one state
    cm = C * L * es                                   # mix of one chunk
    m = {}
    tok = B * T * H                                   # token-heads
    fin0 = B * H * kv                                 # one level's final state
    # level-0 intra: reads q0,k,b,v,w + g (fp32); writes W,U,KtT,Qg,Aqk,gam
    # and, for the backward, TT
    m["ngdn_l0_intra_fwd"] = (
        units * (3 * ck + 2 * cv + gk),
        units * (3 * ck + 2 * cv + gk + 3 * wk + wv + wc + K * 4 + wc),
        units * (2 * 2 * C * C * K + 2 * C * C * (K + V) + C ** 3 // 3))
    # level-0 scan: reads W, U, KtT, gam; writes hT, vnT and (training) h, vn; + final
    m["ngdn_l0_scan_fwd"] = (units * kv + fin0,
                             units * (2 * wk + wv + K * 4 + 2 * kv + 2 * wv) + fin0,
                             units * 2 * 2 * C * K * V)
    # output: Qg, hT, Aqk, vnT, q of upper levels, mix; upper states once per
    # group; writes o and (training) level 0's read
    up_states = sum(B * H * n_groups(NT, f[lvl]) * kv for lvl in range(1, L))
    m["ngdn_output_fwd"] = (
        units * (L * ck + cm + kv + cv) + up_states,
        units * (wk + kv + wc + wv + (L - 1) * ck + cm + cv + wv) + up_states,
        units * (2 * C * K * V + 2 * C * C * V + (L - 1) * 2 * C * K * V))
    # the same output in two passes beside the fused promotion ladder: level
    # 0's share (Qg, hT, Aqk, vnT -> its read, fp32), then the upper levels'
    # reads added to it with the mix (read_0, q of upper levels, mix, upper
    # states once per group -> o)
    m["ngdn_output_l0_fwd"] = (units * (ck + kv),
                               units * (wk + kv + wc + wv + wv),
                               units * (2 * C * K * V + 2 * C * C * V))
    m["ngdn_output_upper_fwd"] = (units * ((L - 1) * ck + cm + cv) + up_states,
                                  units * (wv + (L - 1) * ck + cm + cv) + up_states,
                                  units * (L - 1) * 2 * C * K * V)
    # dmix_0 = <do, read_0>: reads read_0 (fp32), do; writes dmix
    m["ngdn_output_bwd"] = (tok * (V * es + 4), tok * (V * 4 + V * es + L * 4), tok * 2 * V)
    # level-0 reverse scan: reads the forward's W, KtT, Qg, Aqk (transposed on
    # chip), gam, do, mix; writes dSp and dVnT (and dVn for the two-launch
    # chunk backward)
    m["ngdn_l0_scan_bwd"] = (units * (cv + cm + kv),
                             units * (3 * wk + wc + K * 4 + cv + C * es + kv + wv),
                             units * (2 * C * K * V * 3 + 2 * C * C * V))
    # level-0 chunk backward, state half: h, dSp, vn, dVn, do, mix -> dQg, dWT, dKt, dAqk, dgam
    m["ngdn_l0_bwd_state"] = (units * (2 * kv + cv + cm),
                              units * (2 * kv + 2 * wv + cv + C * es + 3 * wk + wc + K * 4),
                              units * (3 * 2 * C * K * V + 2 * C * C * V))
    # level-0 chunk backward, intra half: q0,k,b,v,w,g, W,U,TT, dQg,dWT,dKt,dAqk,dgam,dVnT
    # -> dq0,dk,dv,dg,db,dw
    m["ngdn_l0_bwd_intra"] = (
        units * 2 * (3 * ck + 2 * cv + gk),
        units * (3 * ck + 2 * cv + gk + wk + wv + wc + 3 * wk + wc + K * 4 + wv
                 + 3 * ck + 2 * cv + gk),
        units * (2 * C * C * (K + V) + 2 * 2 * C * C * K + 4 * 2 * C * C * K))
    # level-0 chunk backward in one launch (the default): the state half per
    # chunk in the same workgroup, dQg and dKt through a workspace;
    # dX_w = -dX_u S^T replaces T^T dW, dA = -dX_u Vn^T (no W, U read)
    m["ngdn_l0_bwd"] = (
        units * (2 * (3 * ck + 2 * cv + gk) + 2 * kv + cv + cm),
        units * (3 * ck + 2 * cv + gk + wc + 2 * kv + 2 * wv + cv + C * es
                 + 2 * 2 * wk + 3 * ck + 2 * cv + gk),
        units * (2 * 2 * C * K * V + 2 * C * C * V + 2 * C * K * V
                 + 2 * C * C * V + 2 * 2 * C * C * K + 4 * 2 * C * C * K))
    for lvl in range(1, L):
        nf, ng = n_firings(NT, f[lvl]), n_groups(NT, f[lvl])
        fu = B * H * nf
        nk, nv_ = N * K * 4, N * V * 4
        par_f = H * (N * K + 4 * K * V) * es          # the level's bank and projections
        m[f"ngdn_probe_fwd.{lvl}"] = (fu * kv + par_f,
                                      fu * (kv + 3 * nk + 4 * K) + par_f,
                                      fu * 5 * 2 * N * K * V)
        m[f"ngdn_upper_scan_fwd.{lvl}"] = (B * H * ng * kv + fin0,
                                           fu * 3 * nk + B * H * ng * 2 * kv,
                                           fu * 2 * 2 * N * K * V)
        # the fused ladder (probe + update per firing, on chip): the gathered
        # lower states and the parameters in; group states (both layouts), the
        # final state and, for the backward, keys, (keys b e^g)^T and e^g out
        m[f"ngdn_promote_chain_fwd.{lvl}"] = (fu * kv + par_f + B * H * ng * kv + fin0,
                                              fu * (kv + 2 * nk + 4 * K) + par_f
                                              + B * H * ng * 2 * kv + fin0,
                                              fu * 7 * 2 * N * K * V)
        # reads of level lvl, per group: q_l, do, mix, the group state ->
        # d_states, dq_l, dmix_l (read, dq and dS products: 3 x 2 K V per token)
        m[f"ngdn_read_state_bwd.{lvl}"] = (tok * (K * es + V * es + es + K * es + 4)
                                           + B * H * ng * 2 * kv,
                                           tok * (K * es + V * es + K * es + 2 * 4)
                                           + B * H * ng * 2 * kv, tok * 3 * 2 * K * V)
        # reverse firing scan: keys, A^T, gam, d_states -> dSp, dvn
        m[f"ngdn_upper_scan_bwd.{lvl}"] = (B * H * ng * kv,
                                           fu * (2 * nk + K * 4 + kv + nv_) + B * H * ng * kv,
                                           fu * 2 * 2 * N * K * V)
        # firing backward: lower states (rows and transposed), this level's
        # states (both), dSp, dvn, parameters -> six workspaces, the lower
        # state's gradient; 14 N K V products
        m[f"ngdn_probe_bwd.{lvl}"] = (fu * 3 * kv + H * (N * K + 8 * K * V) * es,
                                      fu * (4 * kv + kv + nv_ + 6 * nk + kv)
                                      + H * (N * K + 8 * K * V) * es, fu * 14 * 2 * N * K * V)
        # parameter gradients: four A^T B sums over every firing's N rows,
        # written as per-slice partials (16 slices per head and product) and
        # added in order; the bank gradient from its per-firing partials
        split = max(1, min(16, (B * nf + 3) // 4))
        m[f"ngdn_param_grads.{lvl}"] = (4 * H * K * V * 4 + H * N * K * 4,
                                        fu * 6 * nk + 2 * 4 * H * split * K * V * 4
                                        + 2 * (4 * H * K * V * 4 + H * N * K * 4),
                                        4 * fu * 2 * N * K * V)
    return m, units


# entry points whose work is matrix products (intra-chunk, output, probe):
# the benchmark reports their achieved fraction of the dense MFMA peak
MFMA_KERNELS = ("ngdn_l0_intra_fwd", "ngdn_output_fwd", "ngdn_output_l0_fwd",
                "ngdn_output_upper_fwd", "ngdn_l0_bwd_state", "ngdn_l0_bwd_intra", "ngdn_l0_bwd",
                "ngdn_probe_fwd", "ngdn_promote_chain_fwd", "ngdn_probe_bwd")


def step_totals(cfg, fwd_only=False):
    """Algorithmic HBM bytes and flops of one fwd+bwd step of the op as a
    whole. Flops are the dense tile products of the op's mathematics with
    C = 64: forward, per chunk-head 2C^2(3K+2V) + 6CKV + C^3/3 for level 0,
    per token-head and upper level 2KV for its read, per firing-head 14NKV
    for a promotion; backward 2C^2(6K+4V) + 12CKV + 4C^3, 4KV and 28NKV.
    Bytes are the op-level tensors once: the
    forward reads the inputs and parameters and writes o, the final state and
    the fp32 state sequences it saves; the backward reads the inputs,
    parameters, saved states and do and writes every gradient."""
    B, T, H, K, V, L, N = (cfg[x] for x in ("B", "T", "H", "K", "V", "L", "N"))
    f = cfg["intervals"]
    es = 2 if cfg["dtype"] == torch.bfloat16 else 4
    NT = -(-T // 64)
    tok = B * T * H
    kv = K * V * 4
    inputs = tok * ((L + 2) * K * es + 2 * V * es + K * 4 + L * es)
    params = (L - 1) * H * (N * K + 4 * K * V) * es
    states = B * H * (NT + sum(n_groups(NT, f[l]) for l in range(1, L))) * kv
    fwd = inputs + params + tok * V * es + B * H * L * kv + states
    bwd = inputs + params + states + tok * V * es + (inputs + params)
    C = 64
    units = B * H * NT
    fires = sum(B * H * n_firings(NT, f[l]) for l in range(1, L))
    flops_f = (units * (2 * C * C * (3 * K + 2 * V) + 6 * C * K * V + C ** 3 // 3)
               + tok * (L - 1) * 2 * K * V + fires * 14 * N * K * V)
    flops_b = (units * (2 * C * C * (6 * K + 4 * V) + 12 * C * K * V + 4 * C ** 3)
               + tok * (L - 1) * 4 * K * V + fires * 28 * N * K * V)
    if fwd_only:
        # without a backward nothing is saved: inputs in, o and the final state out
        return fwd - states, flops_f
    return fwd + bwd, flops_f + flops_b


def profiled_traffic(config, entry):
    """HBM bytes per launch of ``entry`` as the committed counter profile of
    this configuration reports them (FETCH_SIZE and WRITE_SIZE, calibrated on
    a copy kernel), or None when no profile covers it."""
    path = os.path.join(ROOT, "profiles", f"ngdn_fwd_bwd_{config}_traffic.md")
    if not os.path.exists(path):
        return None
    for row in open(path):
        cells = [c.strip().strip("`") for c in row.strip().strip("|").split("|")]
        if len(cells) >= 5 and cells[0] == entry:
            return round(float(cells[4]) * 1e9)
    return None


def fwd_fn(inp, L):
    """The op's forward alone, on inputs that need no gradient (nothing is
    kept for a backward)."""
    def fwd():
        with torch.no_grad():
            chunk_nested_gdn2(**inp, L=L)
    return fwd


def step_fn(inp, leaves, L, do):
    def step():
        o, _ = chunk_nested_gdn2(**{**inp, **leaves}, L=L)
        o.backward(do)
    return step


def cpu_baseline(cfg, budget_s=20.0, backward=True):
    """The CPU restatement (float32 PyTorch) on one-head slices of the
    workload, forward (+ backward), extrapolated to the whole step."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import ngdn_oracle

    from nested_recurrent_memory_amd.inputs import make_cotangent, make_inputs

    cores = len(os.sched_getaffinity(0))
    threads = min(16, cores)
    torch.set_num_threads(threads)
    B, T, H = cfg["B"], cfg["T"], cfg["H"]
    one = dict(cfg)
    one.update(B=1, H=1)
    done, t_total, slices = 0, 0.0, 0
    while t_total < budget_s and slices < B * H:
        inp = make_inputs(**one, seed=slices)
        lv = {n: inp[n].float().requires_grad_(True) for n in LEAVES}
        args = [lv[n] for n in LEAVES] + [inp["n_queries_per_level"], inp["firing_intervals"]]
        t0 = time.perf_counter()
        with torch.enable_grad() if backward else torch.no_grad():
            o, _ = ngdn_oracle.chunk_forward(*args, L=cfg["L"], output_final_state=True,
                                             dtype=torch.float32, out_dtype=torch.float32)
            if backward:
                o.backward(make_cotangent(o.shape))
        t_total += time.perf_counter() - t0
        slices += 1
        done += T
    per_slice = t_total / slices
    full = per_slice * B * H
    return {"value": B * T / full, "unit": "tokens/s", "cores": cores,
            "threads": torch.get_num_threads(), "torch": torch.__version__, "kind": "port",
            "sample": f"{slices} of the {B * H} (batch, head) slices (T={T}) "
                      f"{'forward+backward' if backward else 'forward'}, "
                      f"{t_total:.1f} s, scaled by {B * H}/{slices}"}


# Decoding: one token for a batch of sequences, the c2 layer shape (H=16,
# d=128, 3 levels firing every 1/4/16 chunks, 64 queries) at a serving batch.
DECODE = dict(B=64, H=16, K=128, V=128, L=3, N=64, intervals=(1, 4, 16),
              dtype=torch.bfloat16, g_scale=0.1)


def decode_bench(args):
    """Tokens/s of the decoding step (ngdn_step): one HIP graph per token
    (the step with device-side positions, then position += 1), replayed over
    ``steps`` tokens from position 0, so every firing of the window is
    included. The step kernel's own duration is timed separately on tokens
    that fire nothing."""
    from nested_recurrent_memory_amd import prepare_step_params, step_nested_gdn2

    cfg = dict(DECODE, B=args.decode_batch or DECODE["B"])
    B, H, K, V, L, N = (cfg[x] for x in ("B", "H", "K", "V", "L", "N"))
    inp = gpu_inputs(dict(cfg, T=1))
    tok = {n: inp[n][:, 0].contiguous() for n in ("q", "k", "v", "g", "b", "w", "mix_weights")}
    rest = {n: inp[n] for n in ("query_banks", "key_projections", "b_projections",
                                "w_projections", "g_projections", "n_queries_per_level",
                                "firing_intervals")}
    par = prepare_step_params(*(rest[n] for n in list(rest)[:5]), cfg["dtype"])
    state = torch.zeros(B, H, L, K, V, device="cuda")
    pos = torch.zeros(B, dtype=torch.int64, device="cuda")

    def token(p):
        return step_nested_gdn2(**tok, state=state, position=p, **rest, L=L, params=par,
                                inplace=True)

    with torch.no_grad():
        token(pos)                                   # load the library, warm the pool
        pos.zero_()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            token(pos)
            pos.add_(1)
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            token(pos)
            pos.add_(1)
        for _ in range(args.warmup):
            graph.replay()
        pos.zero_()
        state.zero_()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            graph.replay()
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0

        # the step kernel alone: host positions that fire nothing launch only it
        _lib.TIMING = {}
        for i in range(20):
            token(1 + 64 * i)
        torch.cuda.synchronize()
        timing, _lib.TIMING = _lib.TIMING, None
    evs = timing["ngdn_step"]
    k_ms = sum(a.elapsed_time(b) for a, b in evs) / len(evs)
    es = 2
    # reads every level's state and the token's inputs, writes level 0 and o
    nbytes = B * H * ((L + 1) * K * V * 4 + (L * K + 3 * K + 2 * V + L) * es + K * 4 + V * es)
    gbs = nbytes / (k_ms * 1e-3) / 1e9
    line = {
        "metric": f"tokens/s decoding step nested GDN op (B{B},H{H},d{K},{L} lvl)",
        "value": round(B * args.steps / elapsed, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(elapsed / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "decode: step_nested_gdn2, one token per sequence per step, "
                               f"positions 0..{args.steps - 1}, HIP graph per token",
                   "B": B, "H": H, "K": K, "V": V, "L": L,
                   "firing_intervals": list(cfg["intervals"]), "n_queries": N,
                   "state": "fp32", "state_bytes": B * H * L * K * V * 4},
        # a state below the 256 MB last-level cache can be served from it
        # between tokens; the HBM figure needs B * H * L * K * V * 4 well
        # above that (B = 256: 805 MB)
        "roofline": {"kernel": "ngdn_step (step_kernel)", "bound": "hbm",
                     "cache_resident": B * H * L * K * V * 4 <= 256 * 2**20,
                     "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "algorithmic_bytes": nbytes, "avg_ms": round(k_ms, 4)},
        "cpu_baseline": None,
    }
    print(json.dumps(line))


# config 4: the full model, 12 layers, hidden 1024, 8 heads of 128, 3 levels
# firing every 1/4/16 chunks with 64 queries, SwiGLU 4096, vocab 32000
MODEL = dict(vocab_size=32000, hidden_size=1024, num_hidden_layers=12, num_heads=8, head_dim=128,
             num_levels=3, firing_intervals=(1, 4, 16), n_queries_per_level=(64, 64),
             intermediate_size=4096)
MODEL_BATCH = dict(B=8, T=4096)


def model_bench(args):
    """Tokens/s of one training step of NestedGDN2ForCausalLM at config 4:
    forward with the fused loss, backward, gradient clipping at 1.0 and an
    AdamW step, fp32 parameters under bf16 autocast (the reference's
    training loop, train/pretrain.py:208-219), on uniform random token ids.
    The roofline is the step's model flops (the GEMMs, 6 flops per weight per
    token, plus the op's dense tile products) over the step time, against the
    dense bf16 peak."""
    from nested_recurrent_memory_amd.model import NestedGDN2Config, NestedGDN2ForCausalLM

    cfg = NestedGDN2Config(**MODEL)
    B, T = MODEL_BATCH["B"], MODEL_BATCH["T"]
    torch.manual_seed(0)
    model = NestedGDN2ForCausalLM(cfg).cuda().train()
    opt = torch.optim.AdamW(model.parameters(), lr=3e-4, betas=(0.9, 0.95), weight_decay=0.1,
                            fused=True)
    g = torch.Generator(device="cuda").manual_seed(1)
    ids = torch.randint(0, cfg.vocab_size, (B, T), generator=g, device="cuda")

    def step():
        with torch.autocast("cuda", dtype=torch.bfloat16):
            loss = model(input_ids=ids, labels=ids, use_cache=False).loss
        loss.backward()
        torch.nn.utils.clip_grad_norm_(model.parameters(), 1.0)
        opt.step()
        opt.zero_grad(set_to_none=True)
        return loss

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        loss = step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    # this library's entry points, timed with events in a second pass
    _lib.TIMING = {}
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    timing, _lib.TIMING = _lib.TIMING, None
    ms = elapsed / args.steps * 1e3
    ours = {n: sum(a.elapsed_time(b) for a, b in evs) / args.steps for n, evs in timing.items()}

    linear = sum(m.weight.numel() for m in model.modules() if isinstance(m, torch.nn.Linear))
    opcfg = dict(B=B, T=T, H=cfg.num_heads, K=cfg.head_dim, V=cfg.head_dim, L=cfg.num_levels,
                 N=cfg.n_queries_per_level[0], intervals=cfg.firing_intervals, dtype=torch.bfloat16)
    op_flops = sum(w[2] for w in work_model(opcfg)[0].values()) * cfg.num_hidden_layers
    flops = 6 * linear * B * T + op_flops
    tflops = flops / (ms * 1e-3) / 1e12
    if args.kernel_table:
        for n, t in sorted(ours.items(), key=lambda kv: -kv[1]):
            print(f"{n:32s} {t:8.3f} ms/step", file=sys.stderr)
    line = {
        "metric": "tokens/s training step NestedGDN2ForCausalLM (config 4)",
        "value": round(B * T / (ms * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "model: NestedGDN2ForCausalLM fwd (fused loss) + bwd + clip + "
                               "AdamW, fp32 params under bf16 autocast",
                   "B": B, "T": T, **{k: (list(v) if isinstance(v, tuple) else v)
                                      for k, v in MODEL.items()},
                   "params": sum(p.numel() for p in model.parameters()),
                   "loss": round(float(loss.detach()), 4)},
        "roofline": {"kernel": "whole step (hipBLASLt GEMMs + this library's kernels)",
                     "bound": "mfma", "achieved": round(tflops, 1), "peak": MFMA_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tflops / MFMA_BF16_TFLOPS, 4),
                     "traffic": None, "flops_per_step": flops,
                     "library_kernels_ms": round(sum(ours.values()), 3)},
        "cpu_baseline": None,
    }
    print(json.dumps(line))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="c2",
                    help="c0..c3 (BASELINE.json configs) or ref3 (the reference's published "
                         "depth row at d=128, L=3)")
    ap.add_argument("--mode", default=None, choices=("fwdbwd", "fwd"),
                    help="a step is forward+backward (default) or forward only (default for "
                         "c3, which BASELINE.json quotes forward only)")
    ap.add_argument("--stream-groups", type=int, default=None,
                    help="groups of batch rows run on their own streams (default: the "
                         "package's STREAM_GROUPS)")
    ap.add_argument("--workload", default="train", choices=("train", "decode", "model"),
                    help="train: forward+backward at --config (the headline); "
                         "decode: the decoding step; model: a training step of the "
                         "model at config 4")
    ap.add_argument("--decode-batch", type=int, default=None,
                    help="sequences per decoding step (default 64)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--kernel-table", action="store_true",
                    help="also print per-entry-point times to stderr")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(the op shards by batch or head with no communication inside it)",
              file=sys.stderr)
        sys.exit(2)
    if args.stream_groups is not None:
        from nested_recurrent_memory_amd import chunk as _chunk
        _chunk.STREAM_GROUPS = args.stream_groups
    if args.workload == "decode":
        decode_bench(args)
        return
    if args.workload == "model":
        model_bench(args)
        return

    cfg = dict(CONFIGS[args.config] if args.config in CONFIGS else REF_SHAPES[args.config])
    fwd_only = (args.mode or ("fwd" if args.config == "c3" else "fwdbwd")) == "fwd"
    L = cfg["L"]
    inp = gpu_inputs(cfg)
    leaves = {n: inp[n].detach().clone().requires_grad_(True) for n in LEAVES}
    B, T, H, V = cfg["B"], cfg["T"], cfg["H"], cfg["V"]
    gen = torch.Generator(device="cuda").manual_seed(1)
    do = torch.randn(B, T, H, V, generator=gen, device="cuda").to(cfg["dtype"])
    fwd = fwd_fn(inp, L)
    step = fwd if fwd_only else step_fn(inp, leaves, L, do)

    for _ in range(args.warmup):
        step()
        for t in leaves.values():
            t.grad = None
    torch.cuda.synchronize()

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
        for t in leaves.values():
            t.grad = None
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0

    # per-entry-point durations from a second pass of as many steps, each
    # call bracketed by two timing events (which add about 0.1 ms to a step,
    # so they stay out of the pass above)
    _lib.TIMING = {}
    for _ in range(args.steps):
        step()
        for t in leaves.values():
            t.grad = None
    torch.cuda.synchronize()
    timing, _lib.TIMING = _lib.TIMING, None

    # the reference harness's columns (bench_matched.py:124-149): forward
    # alone (inputs that need no gradient), forward+backward, and the peak of
    # allocated memory over one forward+backward (inputs included)
    cols = None
    if not fwd_only:
        fwd()
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        for _ in range(args.steps):
            fwd()
        torch.cuda.synchronize()
        fwd_ms = (time.perf_counter() - t1) / args.steps * 1e3
        torch.cuda.reset_peak_memory_stats()
        step()
        for t in leaves.values():
            t.grad = None
        torch.cuda.synchronize()
        cols = {"nested_fwd_ms": round(fwd_ms, 3),
                "nested_fb_ms": round(elapsed / args.steps * 1e3, 3),
                "nested_gb": round(torch.cuda.max_memory_allocated() / 1e9, 3)}

    ms = {}
    for name, evs in timing.items():
        ms[name] = sum(s.elapsed_time(e) for s, e in evs) / len(evs)
    per_step = {n: sum(s.elapsed_time(e) for s, e in evs) / args.steps for n, evs in timing.items()}

    model, units = work_model(cfg)
    # per-launch algorithmic work of each entry point; upper levels keyed by
    # level, in call order within a step
    # the op runs each entry point once per group of batch rows (one stream
    # per group), so a launch does 1/launches-per-step of the step's work
    per_launch = {n: args.steps / len(evs) for n, evs in timing.items()}
    # the dominant kernel among those on the launch stream (side-stream
    # intervals include the time they share the GPU with it)
    dom = max((n for n in per_step if n not in _lib.SIDE), key=per_step.get)
    peak_f = MFMA_BF16_TFLOPS if cfg["dtype"] == torch.bfloat16 else MFMA_FP32_TFLOPS

    def launch_work(n):
        return tuple(x * per_launch[n] for x in model[n])

    roof = None
    if dom in model:
        nbytes, dbytes, flops = launch_work(dom)
        t = ms[dom] * 1e-3
        gbs, dgbs, tfs = nbytes / t / 1e9, dbytes / t / 1e9, flops / t / 1e12
        hbm_bound = (nbytes / (HBM_PEAK_GBS * 1e9)) >= (flops / (peak_f * 1e12))
        roof = {"kernel": dom, "bound": "hbm" if hbm_bound else "mfma",
                "achieved": round(gbs if hbm_bound else tfs, 2),
                "peak": HBM_PEAK_GBS if hbm_bound else peak_f,
                "unit": "GB/s" if hbm_bound else "TFLOP/s",
                "frac": round((gbs / HBM_PEAK_GBS) if hbm_bound else (tfs / peak_f), 4),
                "traffic": profiled_traffic(args.config, dom),
                "algorithmic_bytes": nbytes, "algorithmic_flops": flops,
                "design_bytes": dbytes, "design_frac": round(dgbs / HBM_PEAK_GBS, 4),
                "avg_ms": round(ms[dom], 4)}
        # the matrix-product kernels' achieved fraction of the dense MFMA peak
        mf = {}
        for n in sorted(per_step, key=per_step.get, reverse=True):
            if n.split(".")[0] in MFMA_KERNELS and n in model:
                fl = launch_work(n)[2]
                tf = fl / (ms[n] * 1e-3) / 1e12
                mf[n] = {"tflops": round(tf, 2), "frac": round(tf / peak_f, 4),
                         "avg_ms": round(ms[n], 4)}
        roof["mfma_kernels"] = mf
        sb, sf = step_totals(cfg, fwd_only)
        st = elapsed / args.steps
        roof["step"] = {"algorithmic_bytes": sb, "hbm_frac": round(sb / st / 1e9 / HBM_PEAK_GBS, 4),
                        "algorithmic_flops": sf,
                        "mfma_frac": round(sf / st / 1e12 / peak_f, 4)}
    if args.kernel_table:
        for n in sorted(per_step, key=per_step.get, reverse=True):
            extra = ""
            if n in model:
                t = ms[n] * 1e-3
                a, d, fl = launch_work(n)
                extra = (f"  alg {a / t / 1e9:7.1f} GB/s  design {d / t / 1e9:7.1f} GB/s"
                         f"  {fl / t / 1e12:7.2f} TFLOP/s")
            side = "  (side stream)" if n in _lib.SIDE else ""
            print(f"{n:28s} {per_step[n]:8.3f} ms/step  {ms[n]:8.3f} ms/launch{extra}{side}",
                  file=sys.stderr)

    ms_step = elapsed / args.steps * 1e3
    tokens = B * T * args.steps
    cpu = None if args.no_cpu_baseline else cpu_baseline(cfg, backward=not fwd_only)
    what = "fwd" if fwd_only else "fwd+bwd"
    metric = ("tokens/s fwd+bwd nested GDN op (B4,T8192,H16,d128,3 lvl)" if args.config == "c2"
              and not fwd_only else f"tokens/s {what} nested GDN op ({args.config}: B{B},T{T},"
              f"H{H},d{cfg['K']},{L} lvl)")
    line = {
        "metric": metric,
        "value": round(tokens / elapsed, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if cfg["dtype"] == torch.bfloat16 else "fp32",
        "data": "synthetic",
        "config": {"workload": f"{args.config}: chunk_nested_gdn2 "
                               f"{'forward' if fwd_only else 'forward+backward'}", "B": B,
                   "T": T, "H": H, "K": cfg["K"], "V": V, "L": L,
                   "firing_intervals": list(cfg["intervals"]),
                   "n_queries": list(inp["n_queries_per_level"]),
                   "inputs": cfg.get("style", "baseline"), "chunk": 64, "state": "fp32"},
        "reference_columns": cols,
        "roofline": roof,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
