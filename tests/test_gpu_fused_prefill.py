"""GPU parity of the fused prefill entry point (gates + conv1d/SiLU + chunked
delta rule in two kernels): bit-equal to the three separate entry points
called in the order of _gdn_prefill_varlen (nanovllm/models/qwen3_5.py:934-961),
whose own parity with the CPU oracle the kernel tests establish, and within
the oracle bars itself on one case."""
import pytest
import torch

from helpers import BF16, assert_out, assert_state, cu_of
from oracle import gdn_ref

pytestmark = pytest.mark.gpu


def _case(seed, Hk, Hv, D, lens, slots):
    gen = torch.Generator().manual_seed(seed)
    C = 2 * Hk * D + Hv * D
    N = sum(lens)
    mixed = torch.randn(N, C, generator=gen).to(BF16)
    if N:
        mixed[0, :8] = -0.0                                     # -0 inputs roll to +0
    conv_w = (torch.randn(C, 4, generator=gen) * 0.5).to(BF16)
    A_log = (torch.rand(Hv, generator=gen) * 2.7).to(BF16)
    dt_bias = (torch.rand(Hv, generator=gen) * 2 - 1).to(BF16)
    a = torch.randn(N, Hv, generator=gen).to(BF16)
    b = torch.randn(N, Hv, generator=gen).to(BF16)
    conv_pool = torch.randn(slots, C, 3, generator=gen).to(BF16)
    conv_pool[0, :4, 1] = -0.0
    s_pool = torch.randn(slots, Hv, D, D, generator=gen) * 0.1
    ids = torch.randperm(slots, generator=gen)[:len(lens)]
    return C, mixed, conv_w, A_log, dt_bias, a, b, conv_pool, s_pool, ids


def _cu(lens, dev):
    return torch.tensor(cu_of(lens), dtype=torch.int64, device=dev)


def _unfused(pkg, dev, Hk, Hv, D, lens, mixed, conv_w, A_log, dt_bias, a, b, conv_pool, s_pool, ids):
    ops = pkg.ops
    N = sum(lens)
    g, beta = ops.fused_g_beta(b, a, A_log, dt_bias, None)
    cu = torch.tensor(cu_of(lens), dtype=torch.int64)
    cu32 = cu.to(torch.int32).to(dev)
    lens32 = torch.tensor(lens, dtype=torch.int32, device=dev)
    q, k, v = ops.causal_conv_silu_varlen_parts(mixed, conv_pool, conv_w, lens32, cu32[:-1], Hk * D,
                                                state_ids=ids)
    o, _ = ops.chunk_gated_delta_rule_varlen(q.view(N, Hk, D), k.view(N, Hk, D), v.view(N, Hv, D), g, beta,
                                             cu.to(dev), s_pool, state_ids=ids, final_state=s_pool)
    return o


CASES = [
    # Hk, Hv, D, lens
    (4, 4, 128, [1, 2, 3, 70, 200, 64, 0, 129]),
    (2, 4, 128, [300, 5, 64, 1]),
    (4, 4, 64, [3, 150, 66, 0, 2]),
    (2, 8, 64, [97, 1, 200]),
]


@pytest.mark.parametrize("param_f32", [False, True])
@pytest.mark.parametrize("Hk,Hv,D,lens", CASES, ids=lambda c: str(c))
def test_fused_equals_separate_calls(pkg, dev, Hk, Hv, D, lens, param_f32):
    slots = len(lens) + 3
    C, mixed, conv_w, A_log, dt_bias, a, b, conv_pool, s_pool, ids = _case(41, Hk, Hv, D, lens, slots)
    if param_f32:
        A_log, dt_bias = A_log.float(), dt_bias.float()
    mixed, conv_w, A_log, dt_bias, a, b, ids = (t.to(dev) for t in (mixed, conv_w, A_log, dt_bias, a, b, ids))
    cp_u, sp_u = conv_pool.to(dev), s_pool.to(dev)
    cp_f, sp_f = conv_pool.to(dev), s_pool.to(dev)
    o_u = _unfused(pkg, dev, Hk, Hv, D, lens, mixed, conv_w, A_log, dt_bias, a, b, cp_u, sp_u, ids)
    o_f = pkg.ops.conv_chunk_prefill_varlen(mixed, cp_f, conv_w, b, a, A_log, dt_bias, _cu(lens, dev), sp_f,
                                            ids, Hk, Hv, D)
    torch.cuda.synchronize()
    assert torch.equal(o_f.view(torch.int16), o_u.view(torch.int16)), "outputs differ"
    assert torch.equal(sp_f, sp_u), "state pool differs"
    assert torch.equal(cp_f.view(torch.int16), cp_u.view(torch.int16)), "conv pool differs"
    # slots outside ids untouched in both pools
    untouched = [i for i in range(slots) if i not in ids.tolist()]
    assert torch.equal(sp_f.cpu()[untouched], s_pool[untouched])
    assert torch.equal(cp_f.cpu()[untouched].view(torch.int16), conv_pool[untouched].view(torch.int16))


def test_fused_against_oracle(pkg, dev):
    """The fused call against the CPU oracle's layer prefill chain directly."""
    Hk, Hv, D = 2, 4, 128
    lens = [130, 3, 64]
    slots = 5
    C, mixed, conv_w, A_log, dt_bias, a, b, conv_pool, s_pool, ids = _case(42, Hk, Hv, D, lens, slots)
    N = sum(lens)
    g, beta = gdn_ref.g_beta(b, a, A_log, dt_bias, None)
    y, new_conv = gdn_ref.conv_varlen(mixed, conv_pool[ids], conv_w, lens)
    kd = Hk * D
    q, k, v = y[:, :kd].reshape(N, Hk, D), y[:, kd:2 * kd].reshape(N, Hk, D), y[:, 2 * kd:].reshape(N, Hv, D)
    ro, rs = gdn_ref.chunk_varlen(q, k, v, g, beta.float(), cu_of(lens), s_pool[ids])
    cp, sp = conv_pool.to(dev), s_pool.to(dev)
    o = pkg.ops.conv_chunk_prefill_varlen(mixed.to(dev), cp, conv_w.to(dev), b.to(dev), a.to(dev), A_log.to(dev),
                                          dt_bias.to(dev), _cu(lens, dev), sp, ids.to(dev), Hk, Hv, D)
    assert_out(o.cpu(), ro.to(BF16), "fused prefill output")
    assert_state(sp.cpu()[ids], rs, "fused prefill state")
    assert torch.equal(cp.cpu()[ids].view(torch.int16), new_conv.view(torch.int16)), "conv pool"


@pytest.mark.parametrize("Hk,Hv,D,lens", [(4, 4, 128, [1, 2, 70, 3, 0, 129]), (2, 4, 64, [66, 2, 130])],
                         ids=lambda c: str(c))
def test_fresh_flags_equal_zeroed_slots(pkg, dev, Hk, Hv, D, lens):
    """Sequences flagged fresh start from zero states without reading their
    pool rows: the same results, bit for bit, as zeroing those slots first."""
    slots = len(lens) + 2
    C, mixed, conv_w, A_log, dt_bias, a, b, conv_pool, s_pool, ids = _case(43, Hk, Hv, D, lens, slots)
    fresh = torch.tensor([i % 2 == 0 for i in range(len(lens))])
    mixed, conv_w, A_log, dt_bias, a, b, ids = (t.to(dev) for t in (mixed, conv_w, A_log, dt_bias, a, b, ids))
    cp_f, sp_f = conv_pool.to(dev), s_pool.to(dev)               # stale contents in the fresh slots
    o_f = pkg.ops.conv_chunk_prefill_varlen(mixed, cp_f, conv_w, b, a, A_log, dt_bias, _cu(lens, dev), sp_f,
                                            ids, Hk, Hv, D, fresh=fresh)
    cp_z, sp_z = conv_pool.to(dev), s_pool.to(dev)
    zero = ids[fresh.to(dev)]
    cp_z[zero] = 0
    sp_z[zero] = 0
    o_z = pkg.ops.conv_chunk_prefill_varlen(mixed, cp_z, conv_w, b, a, A_log, dt_bias, _cu(lens, dev), sp_z,
                                            ids, Hk, Hv, D)
    torch.cuda.synchronize()
    assert torch.equal(o_f.view(torch.int16), o_z.view(torch.int16)), "outputs differ"
    assert torch.equal(sp_f, sp_z), "state pool differs"
    assert torch.equal(cp_f.view(torch.int16), cp_z.view(torch.int16)), "conv pool differs"


def test_range_check_rejects_before_launch(pkg, dev, monkeypatch):
    """NANOVLLM_GDN_CHECK_RANGE=1: inputs that could leave the fp16 operand
    range raise before any kernel runs (pools untouched); in-range inputs
    run as usual."""
    Hk, Hv, D, lens = 2, 2, 64, [70, 5]
    C, mixed, conv_w, A_log, dt_bias, a, b, conv_pool, s_pool, ids = _case(5, Hk, Hv, D, lens, 4)
    args = [t.to(dev) for t in (mixed, conv_pool, conv_w, b, a, A_log, dt_bias)]
    cu = _cu(lens, dev)
    pool = s_pool.to(dev)
    idd = ids.to(dev)
    monkeypatch.setenv("NANOVLLM_GDN_CHECK_RANGE", "1")
    pkg.ops.conv_chunk_prefill_varlen(*args, cu, pool, idd, Hk, Hv, D)      # in range: runs
    torch.cuda.synchronize()
    big = args[0].clone()
    big[3, 7] = 3.0e4                                 # times the taps' gain: beyond fp16
    snap = (pool.clone(), args[1].clone())
    with pytest.raises(ValueError, match="fp16"):
        pkg.ops.conv_chunk_prefill_varlen(big, *args[1:], cu, pool, idd, Hk, Hv, D)
    torch.cuda.synchronize()
    assert torch.equal(pool, snap[0]) and torch.equal(args[1], snap[1])   # rejected before any launch
    hot = pool.clone()
    hot[idd[1], 0, 5, 5] = 7.0e4
    with pytest.raises(ValueError, match="initial states"):
        pkg.ops.conv_chunk_prefill_varlen(*args, cu, hot, idd, Hk, Hv, D)
    fresh = torch.tensor([0, 1], dtype=torch.uint8, device=dev)   # the hot row is fresh: not read
    pkg.ops.conv_chunk_prefill_varlen(*args, cu, hot, idd, Hk, Hv, D, fresh=fresh)
    torch.cuda.synchronize()
    q = torch.randn(10, Hk, D, device=dev).to(BF16)
    k = torch.randn(10, Hk, D, device=dev).to(BF16)
    v = torch.randn(10, Hv, D, device=dev).to(BF16)
    v[2, 1, 3] = float("inf")
    g = torch.zeros(10, Hv, device=dev)
    beta = torch.full((10, Hv), 0.5, device=dev).to(BF16)
    with pytest.raises(ValueError, match="non-finite"):
        pkg.ops.chunk_gated_delta_rule_varlen(q, k, v, g, beta, _cu([10], dev))
