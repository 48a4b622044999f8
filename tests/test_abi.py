"""CPU-side checks of the C ABI: the library loads and exports every entry
point include/ngdn.h declares; argument validation runs before any launch."""

import ctypes
import os
import re

import pytest
import torch

from nested_recurrent_memory_amd import _lib, chunk_nested_gdn2, step_nested_gdn2
from nested_recurrent_memory_amd.inputs import NAMES, make_inputs

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    text = open(os.path.join(ROOT, "include", "ngdn.h")).read()
    return sorted(set(re.findall(r"\b(ngdn_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = _declared()
    assert "ngdn_last_error" in names and "ngdn_l0_intra_fwd" in names
    # every declared symbol has a ctypes signature on the Python side
    assert set(names) <= set(_lib.SIGNATURES), set(names) - set(_lib.SIGNATURES)


def _declarations():
    """name -> parameter type strings of every function the header declares
    (comments and preprocessor lines dropped)."""
    text = open(os.path.join(ROOT, "include", "ngdn.h")).read()
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    text = "\n".join(line for line in text.splitlines() if not line.lstrip().startswith("#"))
    out = {}
    for m in re.finditer(r"\b[a-z0-9_]+\s*\**\s*\b(ngdn_[a-z0-9_]+)\s*\(([^;{]*?)\)\s*;", text):
        args = " ".join(m.group(2).split())
        parts = [] if args in ("", "void") else [a.strip() for a in args.split(",")]
        # drop the parameter name, keep the type
        out[m.group(1)] = [re.sub(r"\s*\b[A-Za-z_][A-Za-z0-9_]*$", "", a) if not a.endswith("*")
                           else a for a in parts]
    return out


def _ctype_of(decl):
    d = decl.replace(" ", "")
    if d.endswith("*"):
        return "ptr"
    return {"int32_t": "i32", "int64_t": "i64", "float": "f32"}[d]


def test_signature_table_matches_header():
    """Every declaration's parameters, one by one, against the ctypes table
    the package calls through: a pointer where the header has a pointer, the
    same integer width, the same count."""
    kind = {_lib.P: "ptr", _lib.PD: "ptr", _lib.I32: "i32", _lib.I64: "i64", ctypes.c_float: "f32"}
    decls = _declarations()
    assert set(decls) == set(_declared())
    for name, params in decls.items():
        want = [_ctype_of(re.sub(r"\b(const|struct)\b", "", p)) for p in params]
        got = [kind[t] for t in _lib.SIGNATURES[name]]
        assert got == want, (name, got, want)


def test_library_exports_every_declared_symbol():
    so = _lib.lib()
    for name in _declared():
        assert hasattr(so, name), name
    assert so.ngdn_arch() == b"gfx950"


def test_interface_version_matches_header_and_loader():
    """The header's NGDN_VERSION, the library's ngdn_version() and the version
    the Python signatures describe are one number."""
    text = open(os.path.join(ROOT, "include", "ngdn.h")).read()
    macro = int(re.search(r"#define NGDN_VERSION (\d+)", text).group(1))
    assert _lib.lib().ngdn_version() == macro == _lib.VERSION


def test_invalid_arguments_return_error_without_launch():
    so = _lib.lib()
    d = _lib.dims(1, 64, 1, 1, 96, 64, _lib.NGDN_BF16, 0.1)   # K=96 unsupported
    rc = so.ngdn_l0_intra_fwd(ctypes.byref(d), *([None] * 13), 0, 1, None)
    assert rc == 1
    assert b"K=96" in so.ngdn_last_error()
    d = _lib.dims(1, 64, 1, 2, 64, 64, _lib.NGDN_BF16, 0.1)
    rc = so.ngdn_probe_fwd(ctypes.byref(d), 1, 0, 24, 1, 2, None, 0, None, None, 32,
                           *([None] * 15), 0, 0, None)
    assert rc == 1 and b"power of two" in so.ngdn_last_error()
    d = _lib.dims(1, 64, 1, 2, 64, 64, _lib.NGDN_BF16, 0.1)
    d.hold_partial = 2
    rc = so.ngdn_l0_intra_fwd(ctypes.byref(d), *([None] * 13), 0, 1, None)
    assert rc == 1 and b"hold_partial 2" in so.ngdn_last_error()


def test_dims_struct_matches_header():
    """The ctypes mirror of ngdn_dims has the header's fields, in order and
    with the header's types, so the library reads hold_partial where the
    caller wrote it."""
    text = open(os.path.join(ROOT, "include", "ngdn.h")).read()
    body = re.search(r"typedef struct ngdn_dims \{(.*?)\} ngdn_dims;", text, re.S).group(1)
    fields = []
    for ty, names in re.findall(r"(int32_t|float)\s+([^;]+);", body):
        fields += [(n.strip(), ty) for n in names.split(",")]
    ct = {"int32_t": ctypes.c_int32, "float": ctypes.c_float}
    assert [(n, ct[t]) for n, t in fields] == list(_lib.Dims._fields_)
    assert ctypes.sizeof(_lib.Dims) == 36


def test_step_noalloc_validates_before_any_hip_call():
    """Shape errors, and a batch row larger than the scratch, are refused
    before the entry point touches the GPU (the pointers here are never
    dereferenced)."""
    so = _lib.lib()
    fake = [ctypes.c_void_p(4096 * (i + 1)) for i in range(12)]
    fs = (ctypes.c_int32 * 2)(1, 1)
    nqs = (ctypes.c_int32 * 1)(128)
    d = _lib.dims(1, 1, 2, 2, 96, 96, _lib.NGDN_F32, 0.1)      # K=96 unsupported
    rc = so.ngdn_step_noalloc(ctypes.byref(d), *fake[:7], fake[7], fake[7], None, 63, 64, fs, 0,
                              nqs, fake[8], 128, fake[9], fake[10], fake[11], fake[11],
                              fake[11], None)
    assert rc == 1 and b"K=96" in so.ngdn_last_error()
    # one row of 200 heads at 128 pairs and K=128 needs 39.4 MB > 32 MiB
    d = _lib.dims(1, 1, 200, 2, 128, 128, _lib.NGDN_F32, 0.1)
    rc = so.ngdn_step_noalloc(ctypes.byref(d), *fake[:7], fake[7], fake[7], None, 63, 64, fs, 0,
                              nqs, fake[8], 128, fake[9], fake[10], fake[11], fake[11],
                              fake[11], None)
    assert rc == 1 and b"scratch" in so.ngdn_last_error()


def _base(**kw):
    cfg = dict(B=1, T=256, H=2, K=64, V=64, L=2, N=32, intervals=(1, 2))
    cfg.update(kw)
    inp = make_inputs(**cfg)
    return {n: inp[n] for n in NAMES}, cfg["L"]


@pytest.mark.parametrize("bad_bt", [16, 32, 128])
def test_rejects_non_64_chunk_size(bad_bt):
    inp, L = _base()
    with pytest.raises((ValueError, AssertionError)):
        chunk_nested_gdn2(**inp, L=L, chunk_size=bad_bt)


@pytest.mark.parametrize("bad", [4, 8, 24])
def test_rejects_bad_n_queries(bad):
    inp, L = _base(n_queries=(bad,))
    with pytest.raises(ValueError, match="power of two"):
        chunk_nested_gdn2(**inp, L=L, chunk_size=64)


def test_cpu_tensors_raise_instead_of_falling_back():
    inp, L = _base()
    with pytest.raises(RuntimeError, match="GPU"):
        chunk_nested_gdn2(**inp, L=L)


def _step_args(L=2, K=64):
    inp = make_inputs(B=2, T=1, H=2, K=K, V=K, L=L, N=16, intervals=(1,) * L)
    args = {n: inp[n][:, 0] for n in ("q", "k", "v", "g", "b", "w", "mix_weights")}
    args.update({n: inp[n] for n in NAMES[7:]})
    args["state"] = torch.zeros(2, 2, L, K, K)
    return args, L


def test_step_cpu_tensors_raise_instead_of_falling_back():
    args, L = _step_args()
    with pytest.raises(RuntimeError, match="GPU"):
        step_nested_gdn2(**args, position=63, L=L)


def test_step_validates_before_launch():
    args, L = _step_args()
    with pytest.raises(ValueError, match="chunk_size"):
        step_nested_gdn2(**args, position=0, L=L, chunk_size=0)
    with pytest.raises(ValueError, match="promotion"):
        step_nested_gdn2(**args, position=0, L=L, promotion="sum")
    args["n_queries_per_level"] = torch.tensor([24], dtype=torch.int32)
    with pytest.raises(ValueError, match="power of two"):
        step_nested_gdn2(**args, position=0, L=L)
    so = _lib.lib()
    d = _lib.dims(1, 1, 1, 2, 64, 64, _lib.NGDN_F32, 0.1)
    rc = so.ngdn_step(ctypes.byref(d), *([None] * 9), None, -1, 64, None, 0, None, None, 16,
                      *([None] * 7))
    assert rc == 1 and b"NULL" in so.ngdn_last_error()


def test_layer_op_entry_points_validate_before_launch():
    so = _lib.lib()
    # W=9 is beyond the unrolled tap counts; D must be a multiple of 8
    assert so.ngdn_short_conv_fwd(_lib.NGDN_BF16, 1, 4, 64, 9, 1, *([None] * 6)) == 1
    assert b"W=9" in so.ngdn_last_error()
    assert so.ngdn_short_conv_bwd(_lib.NGDN_F32, 1, 4, 60, 4, 1, *([None] * 8)) == 1
    assert b"D=60" in so.ngdn_last_error()
    assert so.ngdn_rmsnorm_gated_fwd(_lib.NGDN_F32, 4, 96, 1e-5, *([None] * 6)) == 1
    assert b"V=96" in so.ngdn_last_error()
    assert so.ngdn_rmsnorm_gated_bwd(_lib.NGDN_BF16, 4, 64, *([None] * 10)) == 1
    assert b"NULL" in so.ngdn_last_error()


def test_add_rmsnorm_entry_points_validate_before_launch():
    so = _lib.lib()
    F32, BF16 = _lib.NGDN_F32, _lib.NGDN_BF16
    # bf16 x with an fp32 residual is not one of the kernel's dtype combinations
    assert so.ngdn_add_rmsnorm_fwd(BF16, F32, BF16, 4, 1024, 1e-5, *([None] * 7)) == 1
    assert b"dtypes" in so.ngdn_last_error()
    assert so.ngdn_add_rmsnorm_bwd(F32, F32, BF16, 4, 1024, *([None] * 10)) == 1
    assert b"dtypes" in so.ngdn_last_error()
    # unsupported width, then a residual without the buffer for h
    assert so.ngdn_add_rmsnorm_fwd(F32, BF16, BF16, 4, 1000, 1e-5, *([None] * 7)) == 1
    assert b"D=1000" in so.ngdn_last_error()
    assert so.ngdn_add_rmsnorm_fwd(F32, BF16, BF16, 4, 1024, 1e-5, 8, 8, 8, None, 8, None, None) == 1
    assert b"NULL" in so.ngdn_last_error()
    # zero rows: nothing to do, nothing launched
    assert so.ngdn_add_rmsnorm_fwd(F32, F32, F32, 0, 1024, 1e-5, *([None] * 7)) == 0


def test_merge_with_k_below_v_is_refused():
    """K != V runs the K = V kernels on zero-padded tensors, except merge with
    K < V, whose decay would average over max(K, V) pairs: refused before any
    launch (on CPU tensors the op would otherwise raise for the device)."""
    inp = make_inputs(B=1, T=64, H=2, K=64, V=128, L=2, N=16, intervals=(1, 1))
    with pytest.raises(ValueError, match="K < V"):
        chunk_nested_gdn2(**inp, L=2, promotion="merge")


def test_ranges_outside_the_sequence_are_refused_before_any_launch():
    """The chunk and firing ranges (interface 0.7.0 to 0.9.0) are checked on
    the host: a range outside the sequence returns NGDN_EINVAL with its
    message before any pointer is read (the pointers here are placeholders
    that are never dereferenced)."""
    so = _lib.lib()
    x = ctypes.c_void_p(256)
    d = _lib.dims(1, 128, 1, 2, 64, 64, _lib.NGDN_BF16, 0.125)     # NT = 2
    for c0, n in ((-1, 1), (0, 0), (1, 2), (2, 1)):
        rc = so.ngdn_l0_intra_fwd(ctypes.byref(d), *([x] * 13), c0, n, None)
        assert rc == 1 and b"outside the 2 chunks" in so.ngdn_last_error(), (c0, n)
        rc = so.ngdn_l0_scan_fwd(ctypes.byref(d), *([x] * 7), 1, *([x] * 6), c0, n, None)
        assert rc == 1 and b"outside the 2 chunks" in so.ngdn_last_error(), (c0, n)
        rc = so.ngdn_l0_scan_bwd(ctypes.byref(d), *([x] * 7), 1, None, 0, *([x] * 5), c0, n, None)
        assert rc == 1 and b"outside the 2 chunks" in so.ngdn_last_error(), (c0, n)
        rc = so.ngdn_l0_bwd(ctypes.byref(d), *([x] * 21), c0, n, None)
        assert rc == 1 and b"outside the 2 chunks" in so.ngdn_last_error(), (c0, n)
    # level 1 fires every chunk: NF = 2
    for i0, n in ((-1, 1), (1, 2), (3, 0)):
        rc = so.ngdn_probe_fwd(ctypes.byref(d), 1, 0, 16, 1, 1, x, 2, x, x, 16,
                               *([x] * 15), i0, n, None)
        assert rc == 1 and b"outside the level's 2" in so.ngdn_last_error(), (i0, n)
    for s0, n in ((0, 0), (1, 2), (-1, 1)):
        rc = so.ngdn_upper_scan_fwd(ctypes.byref(d), 1, 16, 2, 2, *([x] * 8), s0, n, None)
        assert rc == 1 and b"outside the level's 2" in so.ngdn_last_error(), (s0, n)


def test_utilities_refuse_bad_arguments():
    """ngdn_transpose and ngdn_cast_bf16 check their counts and element
    size on the host (no launch)."""
    so = _lib.lib()
    assert so.ngdn_transpose(9, None, None, None, None, None, 2, None) == 1
    assert b"at most 8" in so.ngdn_last_error()
    one = (ctypes.c_int32 * 1)(1)
    ptr = (ctypes.c_void_p * 1)(256)
    assert so.ngdn_transpose(1, ptr, ptr, one, one, one, 3, None) == 1
    assert b"2 or 4" in so.ngdn_last_error()
    # 2^24 tiles would need 2^32 work-items: refused before any launch
    big = (ctypes.c_int32 * 1)(1 << 12)     # 128 x 128 tiles per matrix
    many = (ctypes.c_int32 * 1)(1 << 10)    # 2^10 matrices
    assert so.ngdn_transpose(1, ptr, ptr, many, big, big, 2, None) == 1
    assert b"at most 16777215" in so.ngdn_last_error()
    assert so.ngdn_cast_bf16(17, None, None, None, None) == 1
    assert b"at most 16" in so.ngdn_last_error()


def test_transpose_wrapper_refuses_strided_or_mixed():
    """The host wrapper hands raw pointers to ngdn_transpose, so it refuses a
    strided view or mixed dtypes before any call."""
    from nested_recurrent_memory_amd.chunk import _transpose_last2
    x = torch.zeros(4, 6)
    with pytest.raises(ValueError):
        _transpose_last2([x.t()])
    with pytest.raises(ValueError):
        _transpose_last2([x, x.double()])


def test_grid_bound_is_checked_before_any_launch():
    """B*H*chunks at most 2^23 - 1 (one 512-thread workgroup per (batch, head,
    chunk) must keep the grid within 32-bit work-items): the bound itself
    passes the size check and fails only on its empty range, one more is
    refused as too large. Placeholder pointers are never dereferenced."""
    so = _lib.lib()
    x = ctypes.c_void_p(256)
    d = _lib.dims(128, 1024 * 64, 64, 1, 64, 64, _lib.NGDN_BF16, 0.125)   # 2^23
    assert so.ngdn_l0_intra_fwd(ctypes.byref(d), *([x] * 13), 0, 1, None) == 1
    assert b"exceeds 8388607" in so.ngdn_last_error()
    d = _lib.dims((1 << 23) - 1, 64, 1, 1, 64, 64, _lib.NGDN_BF16, 0.125)
    assert so.ngdn_l0_intra_fwd(ctypes.byref(d), *([x] * 13), 0, 0, None) == 1
    assert b"outside the 1 chunks" in so.ngdn_last_error()
