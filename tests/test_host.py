"""Host-side logic of the package: slot bookkeeping, varlen metadata, A/B
switches, the reference-module install hook, and the no-CPU-path rule.
CPU only."""
import os
import subprocess
import sys
import types
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]


def test_linear_state_pool_alloc_free_reuse(pkg):
    pool = pkg.LinearStatePool(3)
    a, b, c = pool.alloc(), pool.alloc(), pool.alloc()
    assert (a, b, c) == (0, 1, 2) and pool.num_free == 0
    with pytest.raises(AssertionError):
        pool.alloc()
    pool.free(b)
    assert pool.num_free == 1 and pool.alloc() == b       # freed slot is reused


def test_state_pools_layout_dummy_slot_and_reset(pkg):
    pools = pkg.allocate_state_pools(4, L=3, H=2, K=8, V=8, conv_dim=24, conv_kernel=4, device="cpu")
    assert pools.s_pool.shape == (5, 3, 2, 8, 8) and pools.s_pool.dtype == torch.float32
    assert pools.conv_pool.shape == (5, 3, 24, 3) and pools.conv_pool.dtype == torch.bfloat16
    assert pools.dummy_slot == 4
    s1, c1 = pools.layer(1)
    # per-layer views: slot stride spans all layers, heads/rows dense
    assert s1.stride(0) == 3 * 2 * 8 * 8 and s1.stride(1) == 64 and s1.stride(3) == 1
    assert c1.stride(0) == 3 * 24 * 3 and c1.stride(1) == 3
    pools.s_pool.fill_(1.0)
    pools.conv_pool.fill_(1.0)
    pkg.reset_linear_states(pools, torch.tensor([2]))
    assert torch.all(pools.s_pool[2] == 0) and torch.all(pools.conv_pool[2] == 0)
    assert torch.all(pools.s_pool[[0, 1, 3, 4]] == 1)


def test_varlen_meta_cached(pkg):
    m1 = pkg.varlen_meta([3, 5, 2], "cpu")
    cu, lens, cu64_cpu, cu64 = m1
    assert cu.tolist() == [0, 3, 8, 10] and lens.tolist() == [3, 5, 2]
    assert cu.dtype == torch.int32 and cu64.dtype == torch.int64 and cu64_cpu.tolist() == [0, 3, 8, 10]
    assert pkg.varlen_meta([3, 5, 2], "cpu") is m1        # reused by every layer of the step


def test_switches_from_env(pkg, monkeypatch):
    monkeypatch.setenv("NANOVLLM_GDN_GBETA", "0")
    monkeypatch.setenv("NANOVLLM_GDN_VARLEN", "0")
    sw = pkg.Switches.from_env()
    assert not sw.gbeta and not sw.varlen and sw.inplace and sw.conv_kernel
    monkeypatch.setenv("FLA_CHUNK", "0")
    w = torch.zeros(3 * 2 * 64, 4, dtype=torch.bfloat16)
    with pytest.raises(NotImplementedError):
        pkg.GatedDeltaNetCore(2, 2, 64, w, torch.zeros(2), torch.zeros(2), torch.ones(64))


def test_install_rebinds_reference_call_sites(pkg):
    mod = types.ModuleType("qwen3_5_stub")
    mod.fused_g_beta = mod.conv_decode_step = lambda *a: None
    mod._HAS_FLA = False
    prev = pkg.integration.install(mod)
    assert mod.fused_g_beta is pkg.ops.fused_g_beta
    assert mod.causal_conv_silu_varlen is pkg.ops.causal_conv_silu_varlen
    assert mod.recurrent_gdn_inplace is pkg.ops.recurrent_gdn_inplace
    assert mod._fla_chunk is pkg.ops.chunk_gated_delta_rule and mod._HAS_FLA
    assert mod._rms_gated_forward is pkg.ops.rms_norm_gated
    pkg.integration.uninstall(mod, prev)
    assert mod._HAS_FLA is False


_STUB_DISPATCH = """
def chunk_gated_delta_rule(query, key, value, g, beta, chunk_size=64, initial_state=None):
    if _USE_FLA_CHUNK:
        return _fla_chunk(query, key, value, g=g, beta=beta, initial_state=initial_state,
                          output_final_state=True, use_qk_l2norm_in_kernel=True)
    return _torch_chunk_gated_delta_rule(query, key, value, g, beta, chunk_size, initial_state)


def recurrent_gated_delta_rule(query, key, value, g, beta, initial_state=None):
    if _USE_FLA_RECURRENT:
        return _fla_recurrent(query, key, value, g=g, beta=beta, initial_state=initial_state,
                              output_final_state=True, use_qk_l2norm_in_kernel=True)
    return _torch_recurrent_gated_delta_rule(query, key, value, g, beta, initial_state)


def _torch_chunk_gated_delta_rule(*args):
    return "torch chunk port"


def _torch_recurrent_gated_delta_rule(*args):
    return "torch recurrent port"
"""


def _stub_module():
    """A module with the reference's dispatch structure for the two fla
    entry points (module globals read at call time, qwen3_5.py:140-149,
    :230-238) and fla absent."""
    mod = types.ModuleType("qwen3_5_stub")
    mod._HAS_FLA = False
    mod._fla_chunk = mod._fla_recurrent = None
    mod._USE_FLA_CHUNK = mod._USE_FLA_RECURRENT = mod._USE_GDN_VARLEN = False
    exec(_STUB_DISPATCH, mod.__dict__)
    return mod


@pytest.mark.parametrize("fla_chunk,fla_rec", [("1", "1"), ("0", "1"), ("1", "0"), ("0", "0")])
def test_install_keeps_fla_switch_semantics(pkg, monkeypatch, fla_chunk, fla_rec):
    """FLA_CHUNK / FLA_RECURRENT keep the reference's meaning after install:
    "1" routes the module's dispatcher to the HIP entry point, "0" to the
    module's own pure-torch port."""
    monkeypatch.setenv("FLA_CHUNK", fla_chunk)
    monkeypatch.setenv("FLA_RECURRENT", fla_rec)
    mod = _stub_module()
    disp_chunk, disp_rec = mod.chunk_gated_delta_rule, mod.recurrent_gated_delta_rule
    prev = pkg.integration.install(mod)
    # the dispatchers themselves are never rebound
    assert mod.chunk_gated_delta_rule is disp_chunk and mod.recurrent_gated_delta_rule is disp_rec
    assert mod._fla_chunk is pkg.ops.chunk_gated_delta_rule
    assert mod._fla_recurrent is pkg.ops.recurrent_gated_delta_rule
    assert mod._USE_GDN_VARLEN == (fla_chunk == "1")
    assert mod._HAS_FLA == (fla_chunk == "1" or fla_rec == "1")
    x = torch.zeros(1, 2, 2, 64, dtype=torch.bfloat16)
    g = torch.zeros(1, 2, 2)
    if fla_chunk == "1":
        with pytest.raises(ValueError, match="GPU only"):   # the HIP op (CPU tensors are refused)
            mod.chunk_gated_delta_rule(x, x, x, g, g.bfloat16())
    else:
        assert mod.chunk_gated_delta_rule(x, x, x, g, g.bfloat16()) == "torch chunk port"
    if fla_rec == "1":
        with pytest.raises(ValueError, match="GPU only"):
            mod.recurrent_gated_delta_rule(x[:, :1], x[:, :1], x[:, :1], g[:, :1], g[:, :1].bfloat16())
    else:
        assert mod.recurrent_gated_delta_rule(x, x, x, g, g) == "torch recurrent port"
    pkg.integration.uninstall(mod, prev)
    assert mod._HAS_FLA is False and mod._fla_chunk is None and mod._USE_FLA_CHUNK is False


def test_install_replaces_varlen_prefill_method(pkg, monkeypatch):
    mod = types.ModuleType("qwen3_5_stub")

    class Qwen3_5GatedDeltaNet:
        def _gdn_prefill_varlen(self, hidden, lens_q, ids):
            return "original"

    mod.Qwen3_5GatedDeltaNet = Qwen3_5GatedDeltaNet
    orig = Qwen3_5GatedDeltaNet.__dict__["_gdn_prefill_varlen"]
    prev = pkg.integration.install(mod)
    assert Qwen3_5GatedDeltaNet.__dict__["_gdn_prefill_varlen"] is not orig
    layer = Qwen3_5GatedDeltaNet()
    layer.conv_kernel = 3                     # other widths keep the original method
    assert layer._gdn_prefill_varlen(None, [1], None) == "original"
    pkg.integration.uninstall(mod, prev)
    assert Qwen3_5GatedDeltaNet.__dict__["_gdn_prefill_varlen"] is orig
    assert "_gdn_padded" not in Qwen3_5GatedDeltaNet.__dict__   # no such method on the stub: left alone
    monkeypatch.setenv("NANOVLLM_GDN_FUSED_PREFILL", "0")
    prev = pkg.integration.install(mod)
    assert Qwen3_5GatedDeltaNet.__dict__["_gdn_prefill_varlen"] is orig
    pkg.integration.uninstall(mod, prev)


def test_install_replaces_padded_method(pkg, monkeypatch):
    mod = types.ModuleType("qwen3_5_stub")

    class Qwen3_5GatedDeltaNet:
        def _gdn_padded(self, x, lens, ids, T):
            return "original"

    mod.Qwen3_5GatedDeltaNet = Qwen3_5GatedDeltaNet
    orig = Qwen3_5GatedDeltaNet.__dict__["_gdn_padded"]
    prev = pkg.integration.install(mod)
    assert Qwen3_5GatedDeltaNet.__dict__["_gdn_padded"] is not orig
    layer = Qwen3_5GatedDeltaNet()
    layer.conv_kernel = 4
    assert layer._gdn_padded(None, None, None, 5) == "original"   # T > 1 keeps the original method
    layer.conv_kernel = 3
    assert layer._gdn_padded(None, None, None, 1) == "original"   # other widths too
    pkg.integration.uninstall(mod, prev)
    assert Qwen3_5GatedDeltaNet.__dict__["_gdn_padded"] is orig
    monkeypatch.setenv("NANOVLLM_GDN_FUSED_DECODE", "0")
    prev = pkg.integration.install(mod)
    assert Qwen3_5GatedDeltaNet.__dict__["_gdn_padded"] is orig
    pkg.integration.uninstall(mod, prev)


@pytest.mark.parametrize("flag", ["_USE_GDN_GBETA", "_USE_CONV_TRITON", "_USE_GDN_INPLACE"])
def test_installed_methods_read_switches_at_call_time(pkg, monkeypatch, flag):
    """The reference's layer reads _USE_GDN_GBETA, _USE_CONV_TRITON and
    _USE_GDN_INPLACE on every call (qwen3_5.py:933, :978, :1011, :1024).
    Flipped on the module after install, the installed fused methods run the
    original methods (which read the flags themselves); flipped back, the
    fused path runs again.  The prefill method follows the gate and conv
    switches (its reference form reads no in-place switch)."""
    import types as _types

    mod = _types.ModuleType("qwen3_5_stub")
    mod._USE_GDN_GBETA = mod._USE_CONV_TRITON = mod._USE_GDN_INPLACE = True
    calls = []

    class Qwen3_5GatedDeltaNet:
        def _gdn_prefill_varlen(self, hidden, lens_q, ids):
            return "original prefill"

        def _gdn_padded(self, x, lens, ids, T):
            return "original padded"

    mod.Qwen3_5GatedDeltaNet = Qwen3_5GatedDeltaNet
    mod._varlen_meta = lambda lens_q: (None, None, None, None)

    class _Stop(Exception):
        pass

    def fused(*a, **k):
        calls.append("fused")
        raise _Stop

    monkeypatch.setattr(pkg.ops, "conv_chunk_prefill_varlen", fused)
    monkeypatch.setattr(pkg.ops, "recurrent_decode_fused", fused)
    monkeypatch.setattr(pkg.ops, "conv_decode_step", lambda *a, **k: None)
    prev = pkg.integration.install(mod)
    try:
        layer = Qwen3_5GatedDeltaNet()
        layer.conv_kernel, layer.num_k_heads, layer.num_v_heads = 4, 2, 4
        layer.head_k_dim = layer.head_v_dim = 8
        layer.key_dim, layer.value_dim, layer.conv_dim = 16, 32, 64
        layer.A_log = layer.dt_bias = torch.zeros(4)
        layer._v_head_slice = slice(0, 4)
        layer.in_proj_b = layer.in_proj_a = lambda h: torch.zeros(*h.shape[:-1], 4)
        layer.in_proj_z = lambda h: torch.zeros(*h.shape[:-1], 32)
        layer.in_proj_qkv = lambda h: h
        layer.conv1d = _types.SimpleNamespace(weight=torch.zeros(64, 1, 4))
        layer.conv_cache, layer.s_cache = torch.zeros(3, 64, 3), None
        layer.norm = _types.SimpleNamespace(weight=torch.ones(8), eps=1e-6)
        x = torch.zeros(2, 64)

        def run():
            out = []
            for fn, args in ((layer._gdn_prefill_varlen, (x, [1, 1], None)),
                             (layer._gdn_padded, (x.view(2, 1, 64), None, None, 1))):
                try:
                    out.append(fn(*args))
                except _Stop:
                    out.append("fused")
            return out

        assert run() == ["fused", "fused"]
        setattr(mod, flag, False)
        expect_prefill = "fused" if flag == "_USE_GDN_INPLACE" else "original prefill"
        assert run() == [expect_prefill, "original padded"]
        setattr(mod, flag, True)
        assert run() == ["fused", "fused"]
    finally:
        pkg.integration.uninstall(mod, prev)


def test_ops_have_no_cpu_path(pkg):
    a = torch.zeros(4, 2, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU only"):
        pkg.ops.fused_g_beta(a, a, torch.zeros(2), torch.zeros(2), None)
    x = torch.zeros(2, 1, 2, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU only"):
        pkg.ops.recurrent_gated_delta_rule(x, x, x, g=torch.zeros(2, 1, 2), beta=torch.zeros(2, 1, 2,
                                           dtype=torch.bfloat16))


def test_bench_refuses_multi_gpu():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr


def test_missing_library_fails_loudly(tmp_path):
    code = ("import os, sys; sys.path.insert(0, %r); os.environ['GDN_MI355X_LIB'] = %r\n"
            "import __graft_entry__ as ge\npkg = ge.load_package()\n"
            "try:\n    pkg._lib.load()\nexcept pkg._lib.GDNLibraryError as e:\n    print('LOUD', e)\n"
            % (str(ROOT), str(tmp_path / "missing.so")))
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert "LOUD" in r.stdout, r.stderr


def test_fp16_range_violation_bounds(pkg):
    """The opt-in input check of the prefill wrappers: raw rows times the
    conv's largest tap gain, the raw rows themselves without the conv, and
    the initial states must stay below the fp16 maximum (65504); non-finite
    inputs are rejected.  Pinned against hand-computed bounds."""
    f = pkg.ops.fp16_range_violation
    rows = torch.zeros(4, 6, dtype=torch.bfloat16)
    rows[1, 2] = -200.0
    w = torch.zeros(6, 4, dtype=torch.bfloat16)
    w[3] = torch.tensor([100.0, -100.0, 50.0, 50.0])          # channel gain 300
    assert f(rows=rows) is None
    assert f(rows=rows, conv_weight=w) is None                # 200 * 300 = 60000 < 65504
    w[3, 0] = 120.0                                           # gain 320 -> 64000
    assert f(rows=rows, conv_weight=w) is None
    w[3, 0] = 130.0                                           # gain 330 -> 66000
    assert "after the conv" in f(rows=rows, conv_weight=w)
    rows[0, 0] = 70000.0
    assert "input rows reach" in f(rows=rows)
    rows[0, 0] = float("nan")
    assert f(rows=rows) == "non-finite input rows"
    st = torch.zeros(2, 1, 4, 4)
    assert f(states=st) is None
    st[1, 0, 2, 3] = -65504.0
    assert "initial states" in f(states=st)
    st[1, 0, 2, 3] = float("inf")
    assert "initial states" in f(states=st)


def test_fp16_range_switch(pkg, monkeypatch):
    monkeypatch.delenv("NANOVLLM_GDN_CHECK_RANGE", raising=False)
    assert not pkg.ops.range_check_enabled()
    monkeypatch.setenv("NANOVLLM_GDN_CHECK_RANGE", "1")
    assert pkg.ops.range_check_enabled()
