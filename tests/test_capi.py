"""The C-ABI library: loads, exports every entry point include/gdn_mi355x.h
declares, the Python bindings match the header, and argument validation
rejects bad calls before any device work.  CPU only (no kernel launches)."""
import ctypes
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "gdn_mi355x.h"


def _declared():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    decls = {}
    for m in re.finditer(r"\b(?:int|int64_t)\s+(gdn_\w+)\s*\(([^)]*)\)\s*;", text, flags=re.S):
        args = [a.strip() for a in m.group(2).split(",") if a.strip() and a.strip() != "void"]
        decls[m.group(1)] = len(args)
    return decls


def test_header_declares_entry_points():
    d = _declared()
    for name in ("gdn_abi_version", "gdn_g_beta", "gdn_conv_varlen", "gdn_conv_decode", "gdn_conv_padded",
                 "gdn_chunk_prefill", "gdn_chunk_prefill_workspace_size", "gdn_recurrent", "gdn_state_commit",
                 "gdn_rmsnorm_gated", "gdn_conv_chunk_prefill", "gdn_recurrent_decode_fused"):
        assert name in d


def test_library_exports_every_declared_symbol(pkg):
    lib = pkg._lib.load()
    d = _declared()
    out = subprocess.run(["nm", "-D", "--defined-only", str(pkg._lib.LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    for name in d:
        assert name in exported, f"{name} declared but not exported"
        assert getattr(lib, name) is not None
    assert lib.gdn_abi_version() == pkg._lib.ABI_VERSION


def test_bindings_match_header(pkg):
    d = _declared()
    assert set(pkg._lib.SIGNATURES) == set(d)
    for name, n in d.items():
        assert len(pkg._lib.SIGNATURES[name]) == n, name


def test_library_has_no_rpath_to_system_rocm(pkg):
    out = subprocess.run(["readelf", "-d", str(pkg._lib.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    assert "RPATH" not in out and "RUNPATH" not in out
    assert "libamdhip64.so" in out


def test_argument_validation_before_launch(pkg):
    """Rejected shapes return error codes without touching the device."""
    lib = pkg._lib.load()
    _lib = pkg._lib
    # unsupported head dim
    assert lib.gdn_chunk_prefill(None, 0, None, 0, None, 0, None, None, None, None, None, 0, None, None, 0, 1, 64,
                                 1, 1, 96, 1.0, 1, None, None, 0, None) == _lib.GDN_ERR_UNSUPPORTED
    assert lib.gdn_recurrent(None, 0, 0, None, 0, 0, None, 0, 0, None, None, None, 0, None, 0, None, None,
                             None, 1, 1, 1, 1, 32, 1.0, 1, None) == _lib.GDN_ERR_UNSUPPORTED
    assert lib.gdn_rmsnorm_gated(None, 0, None, 0, None, None, 4, 1, 256, 1e-6, None) == _lib.GDN_ERR_UNSUPPORTED
    # head grouping must divide
    assert lib.gdn_chunk_prefill(None, 0, None, 0, None, 0, None, None, None, None, None, 0, None, None, 0, 1, 64,
                                 3, 4, 128, 1.0, 1, None, None, 0, None) == _lib.GDN_ERR_INVALID_ARG
    # a negative segment count is rejected
    assert lib.gdn_chunk_prefill(None, 0, None, 0, None, 0, None, None, None, None, None, 0, None, None, -1, 1, 64,
                                 4, 4, 128, 1.0, 1, None, None, 0, None) == _lib.GDN_ERR_INVALID_ARG
    # conv width other than 4, and misaligned channel counts
    assert lib.gdn_conv_decode(None, 0, None, 0, 0, None, None, None, 0, 1, 64, 3, None) == _lib.GDN_ERR_UNSUPPORTED
    assert lib.gdn_conv_varlen(None, 0, None, 0, 0, None, None, None, 8, None, None, 1, 4, 30, 4,
                               None) == _lib.GDN_ERR_INVALID_ARG
    # NULL operands with real work are rejected
    assert lib.gdn_g_beta(None, None, None, None, 0, None, None, None, 32, 16, None) == _lib.GDN_ERR_INVALID_ARG
    # the fused decode step: unsupported head dim, NULL operands, grouped heads that do not divide
    fd = lib.gdn_recurrent_decode_fused
    assert fd(None, 0, None, 0, None, 0, None, 0, 3, None, None, None, None, None, 0, None, 0, None, None,
              4, 2, 4, 96, 1.0, 1, None) == _lib.GDN_ERR_UNSUPPORTED
    assert fd(None, 0, None, 0, None, 0, None, 0, 3, None, None, None, None, None, 0, None, 0, None, None,
              4, 2, 4, 128, 1.0, 1, None) == _lib.GDN_ERR_INVALID_ARG
    assert fd(None, 0, None, 0, None, 0, None, 0, 3, None, None, None, None, None, 0, None, 0, None, None,
              4, 3, 4, 128, 1.0, 1, None) == _lib.GDN_ERR_INVALID_ARG
    assert fd(None, 0, None, 0, None, 0, None, 0, 3, None, None, None, None, None, 0, None, 0, None, None,
              0, 2, 4, 128, 1.0, 1, None) == _lib.GDN_OK
    # empty work is a no-op success
    assert lib.gdn_g_beta(None, None, None, None, 0, None, None, None, 0, 16, None) == _lib.GDN_OK
    with pytest.raises(_lib.GDNKernelError):
        _lib.check("gdn_chunk_prefill", _lib.GDN_ERR_UNSUPPORTED)
