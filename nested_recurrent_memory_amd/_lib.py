"""ctypes binding of libngdn.so (the C ABI declared in include/ngdn.h).

torch is imported first so that the HIP runtime torch ships with is the one
the library binds to (both carry the soname libamdhip64.so.7); device
pointers and streams then pass between them unchanged.
"""

from __future__ import annotations

import ctypes
import os

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libngdn.so")

NGDN_F32 = 0
NGDN_BF16 = 1
# NGDN_VERSION of include/ngdn.h: the interface the signatures below describe.
# The loader refuses a library of another version (working-tensor layouts and
# argument meanings changed between versions under unchanged signatures).
VERSION = 1000


class Dims(ctypes.Structure):
    _fields_ = [("B", ctypes.c_int32), ("T", ctypes.c_int32), ("H", ctypes.c_int32),
                ("L", ctypes.c_int32), ("K", ctypes.c_int32), ("V", ctypes.c_int32),
                ("dtype", ctypes.c_int32), ("scale", ctypes.c_float),
                ("hold_partial", ctypes.c_int32)]


P = ctypes.c_void_p
I32 = ctypes.c_int32
I64 = ctypes.c_int64
WPARTS = 1024         # NGDN_WPARTS: rows of partial weight-gradient sums in the ws arguments
PARAM_SPLIT = 16      # NGDN_PARAM_SPLIT: slices of firings per head in ngdn_param_grads
PD = ctypes.POINTER(Dims)

# name -> argtypes (all return an int32 status unless listed in _RESTYPES)
SIGNATURES = {
    "ngdn_last_error": [],
    "ngdn_version": [],
    "ngdn_arch": [],
    "ngdn_l0_intra_fwd": [PD] + [P] * 6 + [P] * 6 + [P] + [I32, I32] + [P],
    "ngdn_l0_scan_fwd": [PD, P, P, P, P, P, P, P, I32, P, P, P, P, P, P, I32, I32, P],
    "ngdn_probe_fwd": [PD, I32, I32, I32, I32, I32, P, I32, P, P, I32, P, P, P, P]
                      + [P] * 11 + [I32, I32, P],
    "ngdn_upper_scan_fwd": [PD, I32, I32, I32, I32, P, P, P, P, P, P, P, P, I32, I32, P],
    "ngdn_promote_chain_fwd": [PD, I32, I32, I32, I32, I32, P, I32, P, P, I32, P, P, P, P]
                              + [P] * 6 + [P],
    "ngdn_output_fwd": [PD, P, P, P, P, P, P, P, P, P, P, P, P],
    "ngdn_output_l0_fwd": [PD, P, P, P, P, P, P],
    "ngdn_output_upper_fwd": [PD, P, P, P, P, P, P, P, P],
    "ngdn_output_bwd": [PD, P, P, P, P],
    "ngdn_cast_bf16": [I32, P, P, P, P],
    "ngdn_transpose": [I32, P, P, P, P, P, I32, P],
    "ngdn_read_state_bwd": [PD, I32, I32, I32, P, P, P, P, P, P, P, P],
    "ngdn_l0_scan_bwd": [PD, P, P, P, P, P, P, P, I32, P, I32, P, P, P, P, P, I32, I32, P],
    "ngdn_upper_scan_bwd": [PD, I32, I32, I32, I32, P, P, P, P, P, I32, I32, I32, P, P, P, P, P],
    "ngdn_l0_bwd_state": [PD] + [P] * 6 + [P] * 5 + [P],
    "ngdn_l0_bwd_intra": [PD] + [P] * 6 + [P] * 3 + [P] * 6 + [P] * 6 + [P],
    "ngdn_l0_bwd": [PD] + [P] * 6 + [P] + [P] * 4 + [P] * 2 + [P] * 2 + [P] * 6 + [I32, I32, P],
    "ngdn_probe_bwd": [PD, I32, I32, I32, I32, I32, P, P, I32, P, P, I32, P, P, P, P,
                       P, P, P, P, P, P, P, I32, P, P] + [P] * 6 + [P, P, P] + [P],
    "ngdn_param_grads": [PD, I32, I32, I32, I32, P, P, P, P, P, P, I32, P, P, P, P, P, P, P],
    "ngdn_step": [PD] + [P] * 7 + [P, P, P, I64, I32, P, I32, P, P, I32] + [P] * 4 + [P, P, P],
    "ngdn_step_noalloc": [PD] + [P] * 7 + [P, P, P, I64, I32, P, I32, P, P, I32] + [P] * 4
                         + [P, P],
    "ngdn_short_conv_fwd": [I32, I32, I32, I32, I32, I32, P, P, P, P, P, P],
    "ngdn_short_conv_bwd": [I32, I32, I32, I32, I32, I32, P, P, P, P, P, P, P, P],
    "ngdn_rmsnorm_gated_fwd": [I32, I64, I32, ctypes.c_float, P, P, P, P, P, P],
    "ngdn_rmsnorm_gated_bwd": [I32, I64, I32, P, P, P, P, P, P, P, P, P, P],
    "ngdn_gate_prep_fwd": [I32, P, P],
    "ngdn_gate_prep_bwd": [I32, P, P],
    "ngdn_rmsnorm_fwd": [I32, I64, I32, ctypes.c_float, P, P, P, P, P],
    "ngdn_rmsnorm_bwd": [I32, I64, I32] + [P] * 8,
    "ngdn_add_rmsnorm_fwd": [I32, I32, I32, I64, I32, ctypes.c_float] + [P] * 7,
    "ngdn_add_rmsnorm_bwd": [I32, I32, I32, I64, I32] + [P] * 10,
    "ngdn_swiglu_fwd": [I32, I64] + [P] * 4,
    "ngdn_swiglu_bwd": [I32, I64] + [P] * 6,
    "ngdn_sum_f32": [I32, I32, P, I64, P, P],
    "ngdn_cross_entropy": [I32, I64, I32, I32, P, P, P, P, I32, P],
}
_RESTYPES = {"ngdn_last_error": ctypes.c_char_p, "ngdn_arch": ctypes.c_char_p}

_lib = None


class NgdnError(RuntimeError):
    pass


def lib():
    """The loaded library. Raises if it has not been built: there is no
    fallback path."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise NgdnError(
                f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; "
                f"g.build()'` (or make -C nested_recurrent_memory_amd/csrc)")
        so = ctypes.CDLL(LIB_PATH)
        for name, args in SIGNATURES.items():
            fn = getattr(so, name)
            fn.argtypes = args
            fn.restype = _RESTYPES.get(name, ctypes.c_int32)
        if so.ngdn_version() != VERSION:
            raise NgdnError(f"{LIB_PATH} implements interface version {so.ngdn_version()}, "
                            f"this package calls version {VERSION}: rebuild the library")
        _lib = so
    return _lib


# When set to a dict, every entry point call is bracketed by two timing events
# recorded on the stream it launches on: TIMING[name] collects (start, end)
# event pairs. SIDE collects the names launched on a side stream (their
# intervals overlap the main stream's kernels).
TIMING = None
SIDE = set()


def call(name, *args, tag=None, stream=None):
    """Calls entry point ``name``; raises NgdnError on a nonzero status.
    ``tag`` names the call in TIMING (default: the entry point); ``stream``
    is the torch stream the call launches on when it is not the current one
    (the timing events go on that stream)."""
    if TIMING is not None:
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record(stream)
        rc = getattr(lib(), name)(*args)
        end.record(stream)
        if stream is not None and stream != torch.cuda.current_stream():
            SIDE.add(tag or name)
        TIMING.setdefault(tag or name, []).append((start, end))
    else:
        rc = getattr(lib(), name)(*args)
    if rc != 0:
        msg = lib().ngdn_last_error().decode()
        raise NgdnError(f"{name} failed ({rc}): {msg}")


def ptr(t):
    """Device pointer of a tensor (or NULL for None)."""
    if t is None:
        return None
    return ctypes.c_void_p(t.data_ptr())


def stream_of(t):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def ptr_of_stream(st):
    return ctypes.c_void_p(st.cuda_stream)


class GateArgs(ctypes.Structure):
    """ngdn_gate_args (include/ngdn.h)."""
    _fields_ = ([("BT", ctypes.c_int64)] + [(n, ctypes.c_int32) for n in
                ("H", "L", "K", "V", "param_dtype", "sigmoid_mix")] + [("cap", ctypes.c_float)] +
                [(n, ctypes.c_void_p) for n in (
                    "q", "k", "f", "bz", "wz", "ml", "A_log", "dt_bias", "qn", "kn", "g0", "b0",
                    "w0", "mix", "dqn", "dkn", "dg0", "db0", "dw0", "dmix", "dq", "dk", "df",
                    "dbz", "dwz", "dml", "dpar", "ws")])


def dims(B, T, H, L, K, V, dtype_code, scale, hold_partial=False):
    return Dims(B, T, H, L, K, V, dtype_code, float(scale), int(hold_partial))
