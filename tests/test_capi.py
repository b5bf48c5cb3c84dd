"""The C-ABI library: loads, exports every entry point include/gdn_mi355x.h
declares, the Python bindings match the header, and argument validation
rejects bad calls before any device work.  CPU only (no kernel launches)."""
import ctypes
import re
import subprocess
from pathlib import Path

import pytest
import torch

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


def test_ops_reject_short_id_lists(pkg, monkeypatch):
    """The wrappers check the ids / accepted lengths against the batch before
    the launch.  The device check and the launch are stubbed (CPU only): a
    short list must fail the length check, a full one reach the launch."""
    ops = pkg.ops

    class Launched(Exception):
        pass

    def fake_call(*a, **k):
        raise Launched()

    monkeypatch.setattr(ops, "_check_cuda", lambda *ts: torch.device("cpu"))
    monkeypatch.setattr(ops, "_stream", lambda dev: 0)
    monkeypatch.setattr(ops._lib, "call", fake_call)
    bf = torch.bfloat16
    Hk = Hv = 2
    D = 64
    C = 2 * Hk * D + Hv * D
    B = 4
    x = torch.zeros(B, C, dtype=bf)
    pool = torch.zeros(8, C, 3, dtype=bf)
    w = torch.zeros(C, 4, dtype=bf)
    for n_ids in (B - 1, B):
        ids = torch.arange(n_ids)
        exc = AssertionError if n_ids < B else Launched
        with pytest.raises(exc):
            ops.conv_decode_step(x, pool, ids, w)
        s_pool = torch.zeros(8, Hv, D, D)
        qk = torch.zeros(B, 2 * Hk * D, dtype=bf)
        ab = torch.zeros(B, Hv, dtype=bf)
        with pytest.raises(exc):
            ops.recurrent_decode_fused(qk, x, pool, w, ab, ab, torch.zeros(Hv, dtype=bf), torch.zeros(Hv, dtype=bf),
                                       s_pool, ids, Hk, Hv, D)
        inter = torch.zeros(B, 2, Hv, D, D)
        with pytest.raises(exc):
            ops.commit_states(s_pool, ids, inter, torch.ones(n_ids, dtype=torch.int32))
        if n_ids == B:
            with pytest.raises(AssertionError):   # a short accepted list alone
                ops.commit_states(s_pool, ids, inter, torch.ones(B - 1, dtype=torch.int32))


def test_argument_validation_before_launch(pkg):
    """Rejected shapes return error codes without touching the device."""
    lib = pkg._lib.load()
    _lib = pkg._lib
    # unsupported head dim
    assert lib.gdn_chunk_prefill(None, 0, None, 0, None, 0, None, None, None, None, None, 0, None, None, 0, 1, 64,
                                 1, 1, 96, 1.0, 1, None, None, 0, None) == _lib.GDN_ERR_UNSUPPORTED
    assert lib.gdn_recurrent(None, 0, 0, None, 0, 0, None, 0, 0, None, None, None, 0, None, 0, None, None,
                             None, 1, 1, 1, 1, 32, 1.0, 1, None, None, 1, None) == _lib.GDN_ERR_UNSUPPORTED
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
              4, 2, 4, 96, 1.0, 1, None, 0, None, 1e-6, None) == _lib.GDN_ERR_UNSUPPORTED
    assert fd(None, 0, None, 0, None, 0, None, 0, 3, None, None, None, None, None, 0, None, 0, None, None,
              4, 2, 4, 128, 1.0, 1, None, 0, None, 1e-6, None) == _lib.GDN_ERR_INVALID_ARG
    assert fd(None, 0, None, 0, None, 0, None, 0, 3, None, None, None, None, None, 0, None, 0, None, None,
              4, 3, 4, 128, 1.0, 1, None, 0, None, 1e-6, None) == _lib.GDN_ERR_INVALID_ARG
    assert fd(None, 0, None, 0, None, 0, None, 0, 3, None, None, None, None, None, 0, None, 0, None, None,
              0, 2, 4, 128, 1.0, 1, None, 0, None, 1e-6, None) == _lib.GDN_OK
    # empty work is a no-op success
    assert lib.gdn_g_beta(None, None, None, None, 0, None, None, None, 0, 16, None) == _lib.GDN_OK
    with pytest.raises(_lib.GDNKernelError):
        _lib.check("gdn_chunk_prefill", _lib.GDN_ERR_UNSUPPORTED)


def test_column_split_control(pkg):
    """gdn_set_column_split takes modes 0-2 only (a host setting, no device work)."""
    lib = pkg._lib.load()
    _lib = pkg._lib
    try:
        for bad in (-1, 3, 100):
            assert lib.gdn_set_column_split(bad) == _lib.GDN_ERR_INVALID_ARG
        for mode in (1, 2, 0):
            assert lib.gdn_set_column_split(mode) == _lib.GDN_OK
    finally:
        lib.gdn_set_column_split(0)


def test_stride_validation_before_launch(pkg):
    """Strides too short for the shapes return error codes without touching the device."""
    lib = pkg._lib.load()
    _lib = pkg._lib
    fd = lib.gdn_recurrent_decode_fused
    # slot strides shorter than a slot's states (rows of the pool would
    # overlap) and short raw rows are rejected before any launch; the dummy
    # pointers are aligned and never dereferenced.  Only where no GPU is
    # visible: a check moved behind a launch then fails with a HIP error
    # instead of touching the dummy address on a device.
    if torch.cuda.device_count() > 0:
        pytest.skip("dummy device addresses are passed only where no GPU is visible")
    P = ctypes.c_void_p(1 << 20)
    Hv, D = 4, 128
    slot = Hv * D * D
    rec = lambda s_in_stride, s_out_stride, src=None, idx=None: lib.gdn_recurrent(
        P, 0, 0, P, 0, 0, P, 0, 0, P, P, P, s_in_stride, P, s_out_stride, P, None, P, 2, 1, 4, Hv, D, 1.0, 1,
        src, idx, 4, None)
    assert rec(slot - 4, slot) == _lib.GDN_ERR_INVALID_ARG
    assert rec(slot, slot - 4) == _lib.GDN_ERR_INVALID_ARG
    # the deferred-commit source: both pointers or neither
    assert rec(slot, slot, src=P) == _lib.GDN_ERR_INVALID_ARG
    assert rec(slot, slot, idx=P) == _lib.GDN_ERR_INVALID_ARG
    commit = lambda stride: lib.gdn_state_commit(P, stride, P, P, P, 2, 4, Hv, D, None)
    assert commit(slot - 4) == _lib.GDN_ERR_INVALID_ARG
    C = 3 * Hv * D
    fdec = lambda sx_row, s_stride, cp_slot, z=None, sz=0, nw=None: fd(
        P, C, P, C, P, sx_row, P, cp_slot, 3, P, P, P, P, P, 0, P, s_stride, P, P, 2, Hv, Hv, D, 1.0, 1,
        z, sz, nw, 1e-6, None)
    assert fdec(C - 4, slot, 3 * C) == _lib.GDN_ERR_INVALID_ARG          # raw row shorter than C
    assert fdec(C, slot - 4, 3 * C) == _lib.GDN_ERR_INVALID_ARG          # state slot stride
    assert fdec(C, slot, 3 * C - 3) == _lib.GDN_ERR_INVALID_ARG          # conv slot stride
    assert fdec(C, slot, 3 * C, z=P, sz=Hv * D) == _lib.GDN_ERR_INVALID_ARG       # fused norm without its weight
    assert fdec(C, slot, 3 * C, z=P, sz=Hv * D - 4, nw=P) == _lib.GDN_ERR_INVALID_ARG  # gate rows too short


def test_column_part_gemm_validation_before_launch(pkg):
    """gdn_gemm_bf16_cols rejects part counts outside 1..4, a missing part
    table, boundaries off the 16-column grid, out of order or not ending at N,
    and parts narrower than their row stride allows, before any launch.  NULL
    operands where the part checks come first; dummy (aligned, never
    dereferenced) ones only where no GPU is visible."""
    lib = pkg._lib.load()
    _lib = pkg._lib
    M, N, K = 4, 96, 64

    def call(ends, lds=None, A=None, n_parts=None, table=True):
        n = len(ends) if n_parts is None else n_parts
        c = (ctypes.c_void_p * 5)(*([1 << 20] * 5))
        ld = (ctypes.c_int64 * 5)(*(lds or [128] * 5))
        e = (ctypes.c_int * 5)(*(list(ends) + [0] * (5 - len(ends))))
        return lib.gdn_gemm_bf16_cols(A, K, A, K, M, N, K, n, c if table else None, ld, e, None, None, None, None,
                                      0, 0, 0, None)

    assert call((96,), n_parts=0) == _lib.GDN_ERR_INVALID_ARG
    assert call((16, 32, 48, 64, 96)) == _lib.GDN_ERR_INVALID_ARG                 # five parts
    assert call((96,), table=False) == _lib.GDN_ERR_INVALID_ARG
    if torch.cuda.device_count() > 0:
        pytest.skip("dummy device addresses are passed only where no GPU is visible")
    P = ctypes.c_void_p(1 << 20)
    for ends in ((40, 96), (64, 100), (96, 64), (64, 64), (8, 48, 64, 96)):
        assert call(ends, A=P) == _lib.GDN_ERR_INVALID_ARG, ends
    assert call((64, 96), lds=[32, 128, 128, 128, 128], A=P) == _lib.GDN_ERR_INVALID_ARG   # ld < part width
