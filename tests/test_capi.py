"""The C ABI library loads, exports every symbol include/mtp_glora_amd.h declares,
and rejects bad arguments with the documented error codes before any device
work (so these run without a GPU)."""
import ctypes
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "mtp_glora_amd.h"


def declared_symbols():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(mga_\w+)\s*\(", text, re.M)))


def test_header_declares_entry_points():
    syms = declared_symbols()
    for s in ["mga_version", "mga_last_error", "mga_kv_append", "mga_regular_index",
              "mga_mtp_block_mask", "mga_attn_fwd", "mga_attn_bwd"]:
        assert s in syms


def test_library_exports_every_declared_symbol(mga):
    lib = mga.load_library()
    out = subprocess.run(["nm", "-D", "--defined-only", mga.library_path()], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (mga_\w+)", out))
    for s in declared_symbols():
        assert s in exported, s
        assert hasattr(lib, s)
    assert set(mga._lib.SIGNATURES) == set(declared_symbols())


def test_version_and_empty_error(mga):
    lib = mga.load_library()
    assert lib.mga_version() == 100
    assert isinstance(lib.mga_last_error(), bytes)


def _append(lib, **kw):
    a = dict(src_k=16, src_v=16, sh=1024, ss=128, src_rows=8, idx=None, n=4, dk=16, dv=16, dsh=1024,
             dss=128, off=0, cap=8, heads=2, hd=128, dtype=0, stream=None)
    a.update(kw)
    return lib.mga_kv_append(a["src_k"], a["src_v"], a["sh"], a["ss"], a["src_rows"], a["idx"], a["n"], a["dk"],
                             a["dv"], a["dsh"], a["dss"], a["off"], a["cap"], a["heads"], a["hd"],
                             a["dtype"], a["stream"])


def test_append_capacity_error(mga):
    lib = mga.load_library()
    assert _append(lib, off=6, n=4, cap=8) == mga._lib.MGA_ERR_CAPACITY
    assert b"capacity" in lib.mga_last_error()


@pytest.mark.parametrize("kw", [dict(dtype=7), dict(hd=48), dict(src_k=None), dict(src_k=8),
                                dict(ss=3), dict(heads=0), dict(n=-1),
                                dict(src_rows=3), dict(src_rows=-1)])
def test_append_invalid_arguments(mga, kw):
    lib = mga.load_library()
    assert _append(lib, **kw) == mga._lib.MGA_ERR_INVALID
    assert lib.mga_last_error() != b""


def test_attention_invalid_arguments(mga):
    lib = mga.load_library()
    P = ctypes.c_void_p(16)
    base = [P, 128, 4096, P, 128 * 64, 128, P, 128 * 64, 128, P, 128, 4096, P, P, P, P, P, P]
    # L != P + S
    rc = lib.mga_attn_fwd(*base, 100, 150, 10, 32, 8, 128, 0, 0.1, None)
    assert rc == mga._lib.MGA_ERR_INVALID and b"L == P + S" in lib.mga_last_error()
    # Hq not a multiple of Hkv
    rc = lib.mga_attn_fwd(*base, 100, 110, 10, 30, 8, 128, 0, 0.1, None)
    assert rc == mga._lib.MGA_ERR_INVALID
    # unsupported head_dim
    rc = lib.mga_attn_fwd(*base, 100, 110, 10, 32, 8, 96, 0, 0.1, None)
    assert rc == mga._lib.MGA_ERR_INVALID and b"head_dim" in lib.mga_last_error()
    # the kernels take a positive, finite scale (the reference's head_dim ** -0.5)
    for bad in (0.0, -0.1, float("inf"), float("nan")):
        rc = lib.mga_attn_fwd(*base, 100, 110, 10, 32, 8, 128, 0, bad, None)
        assert rc == mga._lib.MGA_ERR_INVALID and b"scale" in lib.mga_last_error()


def test_python_errors_are_raised(mga):
    with pytest.raises(mga._lib.CapacityError):
        mga._lib.call("mga_kv_append", 16, 16, 1024, 128, 8, None, 4, 16, 16, 1024, 128, 6, 8, 2, 128, 0, None)


def test_noalloc_rejects_oversized_calls_before_device_work(mga):
    """Hq * S above mga_attn_bwd_noalloc's fixed workspace is rejected before
    the library touches a device."""
    lib = mga.load_library()
    P = ctypes.c_void_p(16)
    rc = lib.mga_attn_bwd_noalloc(P, 128, 4096, P, 128, 128, P, 128, 128, P, 128, 4096, P, 128, 4096, P,
                                  P, 128, 4096, P, 128, 1024, P, 128, 1024, 0, P, P, P, P, P, P, P, P, P,
                                  1 << 20, 1 << 20, 0, 32, 8, 128, 0, 0.1, 3, None)
    assert rc == mga._lib.MGA_ERR_INVALID and b"workspace" in lib.mga_last_error()


def _stage(lib, **kw):
    P = ctypes.c_void_p(16)
    a = dict(q=P, k=P, v=P, qw=P, kw=P, cos=P, sin=P, rows=None, src_rows=0, S=8, Hq=4, Hkv=2, D=128, dtype=0,
             qo=P, ko=P, vo=P, rstd=P)
    a.update(kw)
    return lib.mga_qk_norm_rope_stage_fwd(a["q"], 512, 128, a["k"], 256, 128, a["v"], 256, 128, a["qw"], a["kw"],
                                          a["cos"], a["sin"], 128, ctypes.c_float(1e-6), a["rows"], a["src_rows"],
                                          a["S"], a["Hq"], a["Hkv"], a["D"], a["dtype"], a["qo"], 512, 128,
                                          a["ko"], 128, 1024, a["vo"], 128, 1024, a["rstd"], None)


@pytest.mark.parametrize("kw", [dict(v=None), dict(vo=None), dict(k=None), dict(ko=None), dict(dtype=9),
                                dict(D=130), dict(D=7), dict(Hkv=0), dict(q=None),
                                dict(q=None, qo=None), dict(qw=None), dict(qo=None),
                                dict(rows=ctypes.c_void_p(64), src_rows=0)])
def test_stage_invalid_arguments(mga, kw):
    """mga_qk_norm_rope_stage_fwd: a missing value operand or output, a query
    output / rstd without a query (the query-less form passes neither), a
    query without weight or output, bad sizes or a row gather without its
    source-row count are rejected before any launch."""
    lib = mga.load_library()
    assert _stage(lib, **kw) == mga._lib.MGA_ERR_INVALID
    assert lib.mga_last_error() != b""
