"""Seeded sweeps of random shapes.  The fused varlen prefill
(gdn_conv_chunk_prefill): key heads, value heads per key head, head dim,
sequence count and ragged lengths (empty, one-token, chunk multiples, longer),
fresh slots, bf16 or fp32 gate parameters, the column-split mode, with and
without host offsets.  Each case is held to the three separate calls
(fused_g_beta -> causal_conv_silu_varlen_parts -> chunk_gated_delta_rule_varlen)
bit for bit, outputs and both pools, and to the CPU oracle's prefill chain
(nanovllm/models/qwen3_5.py:922-961) at the suite's output and state bars.
The fused decode step likewise (test_random_shape_decode), and long sequences
cut into segments (test_random_shape_segments)."""
import pytest
import torch

from helpers import BF16, assert_out, assert_state, cu_of
from oracle import gdn_ref
from test_gpu_fused_prefill import _case, _unfused

pytestmark = pytest.mark.gpu


def _draw(i):
    gen = torch.Generator().manual_seed(1000 + i)
    pick = lambda xs: xs[int(torch.randint(len(xs), (1,), generator=gen))]
    Hk = pick([1, 2, 4])
    Hv = Hk * pick([1, 2, 4])
    D = pick([64, 128])
    n = int(torch.randint(1, 11, (1,), generator=gen))
    lens = []
    for _ in range(n):
        kind = int(torch.randint(5, (1,), generator=gen))
        if kind == 0:
            lens.append(pick([0, 1, 2, 3]))
        elif kind == 1:
            lens.append(64 * int(torch.randint(1, 6, (1,), generator=gen)))
        elif kind == 2:
            lens.append(64 * int(torch.randint(1, 6, (1,), generator=gen)) + pick([-1, 1]))
        else:
            lens.append(int(torch.randint(4, 700, (1,), generator=gen)))
    if sum(lens) == 0:
        lens[0] = 5
    fresh = [bool(torch.rand(1, generator=gen) < 0.3) for _ in lens]
    return dict(Hk=Hk, Hv=Hv, D=D, lens=lens, fresh=fresh, param_f32=bool(torch.rand(1, generator=gen) < 0.5),
                split=pick([0, 0, 1, 2]), host_cu=bool(torch.rand(1, generator=gen) < 0.7))


CASES = list(range(24))


@pytest.fixture
def split(pkg):
    lib = pkg._lib.load()
    yield lib.gdn_set_column_split
    lib.gdn_set_column_split(0)


@pytest.mark.parametrize("i", CASES)
def test_random_shape_prefill(pkg, dev, split, i):
    c = _draw(i)
    Hk, Hv, D, lens = c["Hk"], c["Hv"], c["D"], c["lens"]
    print(f"random prefill case {i}: {c}", flush=True)
    slots = len(lens) + 2
    C, mixed, conv_w, A_log, dt_bias, a, b, conv_pool, s_pool, ids = _case(500 + i, Hk, Hv, D, lens, slots)
    if c["param_f32"]:
        A_log, dt_bias = A_log.float(), dt_bias.float()
    fresh = torch.tensor(c["fresh"])
    N = sum(lens)
    cu_h = torch.tensor(cu_of(lens), dtype=torch.int64)
    d = [t.to(dev) for t in (mixed, conv_w, A_log, dt_bias, a, b, ids)]
    mixed_d, conv_w_d, A_log_d, dt_bias_d, a_d, b_d, ids_d = d
    assert split(c["split"]) == 0
    cp_f, sp_f = conv_pool.to(dev), s_pool.to(dev)
    o_f = pkg.ops.conv_chunk_prefill_varlen(mixed_d, cp_f, conv_w_d, b_d, a_d, A_log_d, dt_bias_d, cu_h.to(dev), sp_f,
                                            ids_d, Hk, Hv, D, fresh=fresh,
                                            cu_seqlens_cpu=cu_h if c["host_cu"] else None)
    # the separate calls, on pools whose fresh slots are zeroed first
    cp_u, sp_u = conv_pool.clone(), s_pool.clone()
    zero = ids[fresh]
    cp_u[zero] = 0
    sp_u[zero] = 0
    cp_u, sp_u = cp_u.to(dev), sp_u.to(dev)
    o_u = _unfused(pkg, dev, Hk, Hv, D, lens, mixed_d, conv_w_d, A_log_d, dt_bias_d, a_d, b_d, cp_u, sp_u, ids_d)
    torch.cuda.synchronize()
    assert torch.equal(o_f.view(torch.int16), o_u.view(torch.int16)), "fused output differs from the separate calls"
    assert torch.equal(sp_f, sp_u), "state pool differs from the separate calls"
    assert torch.equal(cp_f.view(torch.int16), cp_u.view(torch.int16)), "conv pool differs from the separate calls"
    # the oracle's chain from the same zeroed rows
    h0 = s_pool[ids].clone()
    h0[fresh] = 0
    conv0 = conv_pool[ids].clone()
    conv0[fresh] = 0
    g, beta = gdn_ref.g_beta(b, a, A_log, dt_bias, None)
    y, new_conv = gdn_ref.conv_varlen(mixed, conv0, conv_w, lens)
    kd = Hk * D
    q, k, v = y[:, :kd].reshape(N, Hk, D), y[:, kd:2 * kd].reshape(N, Hk, D), y[:, 2 * kd:].reshape(N, Hv, D)
    ro, rs = gdn_ref.chunk_varlen(q, k, v, g, beta.float(), cu_of(lens), h0)
    assert_out(o_f.cpu(), ro.to(BF16), f"case {i} output")
    assert_state(sp_f.cpu()[ids], rs, f"case {i} state")
    assert torch.equal(cp_f.cpu()[ids].view(torch.int16), new_conv.view(torch.int16)), "conv pool vs oracle"


def _draw_decode(i):
    gen = torch.Generator().manual_seed(2000 + i)
    pick = lambda xs: xs[int(torch.randint(len(xs), (1,), generator=gen))]
    Hk = pick([1, 2, 4, 8, 16])
    Hv = Hk * pick([1, 1, 2, 4]) if Hk < 16 else pick([16, 32])
    D = pick([64, 128])
    B = pick([1, 2, 3, 7, 33, 100, 129, 256])
    return dict(Hk=Hk, Hv=Hv, D=D, B=B, slots=B + int(torch.randint(0, 9, (1,), generator=gen)),
                param_f32=bool(torch.rand(1, generator=gen) < 0.5), norm=bool(torch.rand(1, generator=gen) < 0.5))


@pytest.mark.parametrize("i", list(range(16)))
def test_random_shape_decode(pkg, dev, i):
    """Decode steps of random shapes: the fused step against fused_g_beta ->
    conv_decode_step -> recurrent_gdn_inplace (-> the gated norm) bit for bit;
    with one key head per value head also the one-launch form that runs the
    q/k conv too (bit for bit where both run whole heads per workgroup, else
    against the two-launch whole-head form); each against the CPU oracle's
    decode chain (nanovllm/models/qwen3_5.py:1008-1030, :1083-1085)."""
    from test_gpu_fused_decode import _case as _dcase
    c = _draw_decode(i)
    Hk, Hv, D, B, slots = c["Hk"], c["Hv"], c["D"], c["B"], c["slots"]
    print(f"random decode case {i}: {c}", flush=True)
    ops = pkg.ops
    host = _dcase(700 + i, Hk, Hv, D, B, slots, c["param_f32"])
    mixed, conv_w, A_log, dt_bias, a, b, conv_pool, s_pool, ids = (t.to(dev) for t in host)
    gen = torch.Generator().manual_seed(800 + i)
    z = torch.randn(B, Hv * D, generator=gen).to(BF16).to(dev) if c["norm"] else None
    w = (1 + 0.05 * torch.randn(D, generator=gen)).to(BF16).to(dev) if c["norm"] else None
    kd = Hk * D
    # the separate calls
    cp1, sp1 = conv_pool.clone(), s_pool.clone()
    g, beta = ops.fused_g_beta(b, a, A_log, dt_bias, None)
    y = ops.conv_decode_step(mixed, cp1, ids, conv_w)
    q, k, v = y[:, :kd].view(B, 1, Hk, D), y[:, kd:2 * kd].view(B, 1, Hk, D), y[:, 2 * kd:].view(B, 1, Hv, D)
    o1 = ops.recurrent_gdn_inplace(q, k, v, g.view(B, 1, Hv), beta.view(B, 1, Hv), sp1, ids).view(B, Hv, D)
    if z is not None:
        o1 = ops.rms_norm_gated(o1, z.view(B, Hv, D), w, 1e-6)
    kw = dict(z=z, norm_weight=w, eps=1e-6) if z is not None else {}
    whole = B * Hv >= ops.WHOLE_HEAD_TILES  # the separate calls' kernel runs whole heads per workgroup

    def step(one, **extra):
        cp2, sp2 = conv_pool.clone(), s_pool.clone()
        qk = None if one else ops.conv_decode_step(mixed[:, :2 * kd], cp2[:, :2 * kd], ids, conv_w[:2 * kd])
        o2 = ops.recurrent_decode_fused(qk, mixed, cp2, conv_w, b, a, A_log, dt_bias, sp2, ids, Hk, Hv, D, **kw,
                                        **extra)
        torch.cuda.synchronize()
        return o2.reshape(B, Hv, D), sp2, cp2

    def same(x, y, name):
        for what, u, r in zip(("output", "state pool", "conv pool"), x, y):
            assert torch.equal(u.view(torch.int16) if u.dtype == BF16 else u,
                               r.view(torch.int16) if r.dtype == BF16 else r), f"{name}: {what}"

    same(step(False), (o1, sp1, cp1), "q/k conv first")
    one = step(True) if Hk == Hv else None
    if one is not None and whole:
        same(one, (o1, sp1, cp1), "one launch")
    elif one is not None and z is not None:
        # (with fewer rows the separate calls split a head's columns over
        # workgroups, whose sums over the rows group differently: the same
        # results within the bars, other bits; the two-launch form with the
        # norm in its kernel runs whole heads, as the one launch does)
        same(one, step(False, fuse_norm=True), "one launch vs two launches with whole heads")
    # the oracle's decode chain
    mixed_h, conv_w_h, A_log_h, dt_bias_h, a_h, b_h, conv_pool_h, s_pool_h, ids_h = host
    rg, rbeta = gdn_ref.g_beta(b_h, a_h, A_log_h, dt_bias_h, None)
    ry, rpool = gdn_ref.conv_decode(mixed_h, conv_pool_h.clone(), ids_h.tolist(), conv_w_h)
    rq, rk, rv = (ry[:, :kd].reshape(B, 1, Hk, D), ry[:, kd:2 * kd].reshape(B, 1, Hk, D),
                  ry[:, 2 * kd:].reshape(B, 1, Hv, D))
    ro, rs, _ = gdn_ref.recurrent_rule(rq, rk, rv, rg.view(B, 1, Hv), rbeta.float().view(B, 1, Hv), s_pool_h[ids_h])
    for name, res in (("separate calls", (o1, sp1, cp1)), ("one launch", one)):
        if res is None:
            continue
        assert_state(res[1].cpu()[ids_h], rs, f"case {i} {name} state")
        assert torch.equal(res[2].cpu().view(torch.int16), rpool.view(torch.int16)), f"{name}: conv pool vs oracle"
        if z is None:
            assert_out(res[0].cpu(), ro.reshape(B, Hv, D).to(BF16), f"case {i} {name} output")


def _draw_segments(i):
    gen = torch.Generator().manual_seed(3000 + i)
    pick = lambda xs: xs[int(torch.randint(len(xs), (1,), generator=gen))]
    Hk = pick([1, 2, 4])
    Hv = Hk * pick([1, 2])
    D = pick([64, 128])
    n = int(torch.randint(1, 6, (1,), generator=gen))
    lens = [int(torch.randint(1, 400, (1,), generator=gen)) for _ in range(n)]
    lens[int(torch.randint(n, (1,), generator=gen))] = int(torch.randint(600, 3000, (1,), generator=gen))
    return dict(Hk=Hk, Hv=Hv, D=D, lens=lens, segs=pick([2, 3, 4, 6, 8, 12]),
                h0=bool(torch.rand(1, generator=gen) < 0.6), fused=bool(torch.rand(1, generator=gen) < 0.5))


@pytest.mark.parametrize("i", list(range(12)))
def test_random_shape_segments(pkg, dev, i):
    """Long sequences cut into segments (max_segments) at random shapes: the
    chunk rule alone or the fused prefill, against the CPU oracle at the
    output and state bars, and against the same call in one pass."""
    from helpers import STATE_REL, rule_inputs, state_rel
    c = _draw_segments(i)
    Hk, Hv, D, lens, segs = c["Hk"], c["Hv"], c["D"], c["lens"], c["segs"]
    print(f"random segments case {i}: {c}", flush=True)
    N = sum(lens)
    cu = cu_of(lens)
    cu_h = torch.tensor(cu, dtype=torch.int64)
    n = len(lens)
    if not c["fused"]:
        gen = torch.Generator().manual_seed(900 + i)
        q, k, v, g, beta = rule_inputs(gen, N, Hk, Hv, D)
        h0 = torch.randn(n, Hv, D, D, generator=gen) * 0.1 if c["h0"] else None
        ro, rS = gdn_ref.chunk_varlen(q, k, v, g, beta.float(), cu, h0)
        args = (q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev), cu_h.to(dev),
                None if h0 is None else h0.to(dev))
        o_s, S_s = pkg.ops.chunk_gated_delta_rule_varlen(*args, cu_seqlens_cpu=cu_h, max_segments=segs)
        o_1, S_1 = pkg.ops.chunk_gated_delta_rule_varlen(*args, cu_seqlens_cpu=cu_h, max_segments=1)
        torch.cuda.synchronize()
        S_s, S_1 = S_s.cpu(), S_1.cpu()
    else:
        slots = n + 2
        C, mixed, conv_w, A_log, dt_bias, a, b, conv_pool, s_pool, ids = _case(950 + i, Hk, Hv, D, lens, slots)
        if not c["h0"]:
            s_pool.zero_()
        g, beta = gdn_ref.g_beta(b, a, A_log, dt_bias, None)
        y, _ = gdn_ref.conv_varlen(mixed, conv_pool[ids], conv_w, lens)
        kd = Hk * D
        q, k, v = y[:, :kd].reshape(N, Hk, D), y[:, kd:2 * kd].reshape(N, Hk, D), y[:, 2 * kd:].reshape(N, Hv, D)
        ro, rS = gdn_ref.chunk_varlen(q, k, v, g, beta.float(), cu, s_pool[ids])
        d = [t.to(dev) for t in (mixed, conv_w, A_log, dt_bias, a, b, ids)]
        res = []
        for ms in (segs, 1):
            cp, sp = conv_pool.to(dev), s_pool.to(dev)
            o = pkg.ops.conv_chunk_prefill_varlen(d[0], cp, d[1], d[5], d[4], d[2], d[3], cu_h.to(dev), sp, d[6], Hk,
                                                  Hv, D, cu_seqlens_cpu=cu_h, max_segments=ms)
            torch.cuda.synchronize()
            res.append((o, sp.cpu()[ids]))
        (o_s, S_s), (o_1, S_1) = res
    assert_out(o_s.cpu(), ro.to(BF16), f"case {i} segmented output")
    assert_state(S_s, rS, f"case {i} segmented state")
    assert_out(o_s.cpu(), o_1.cpu(), f"case {i} segmented vs one pass")
    assert state_rel(S_s, S_1) < STATE_REL
