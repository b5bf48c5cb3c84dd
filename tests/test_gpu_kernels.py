"""GPU parity of every HIP kernel against the CPU oracle on seeded inputs.

Bars: bf16 outputs max-abs 2e-2 / mean-rel 1e-3; fp32 states rel 1e-3;
conv-state rolls and untouched pool slots bit-exact."""
import math

import pytest
import torch

from helpers import (BF16, assert_out, assert_state, cu_of, gates, max_abs, mean_rel, rule_inputs,
                     state_rel)
from oracle import gdn_ref

pytestmark = pytest.mark.gpu


def _gen(seed):
    return torch.Generator().manual_seed(seed)


# ------------------------------------------------------------------ g / beta --
@pytest.mark.parametrize("param_f32", [False, True])
@pytest.mark.parametrize("with_mask", [False, True])
def test_g_beta(pkg, dev, param_f32, with_mask):
    gen = _gen(11)
    n, T, Hv = 7, 37, 16
    a, b, A_log, dt_bias = gates(gen, n * T, Hv)
    a, b = a.view(n, T, Hv), b.view(n, T, Hv)
    a[0, 0, 0] = 25.0          # softplus threshold branch
    b[0, 0, 1] = 0.0           # sigmoid(0) = 0.5
    if param_f32:
        A_log, dt_bias = A_log.float(), dt_bias.float()
    mask = (torch.rand(n, T, generator=gen) > 0.3) if with_mask else None
    g, beta = pkg.ops.fused_g_beta(b.to(dev), a.to(dev), A_log.to(dev), dt_bias.to(dev),
                                   None if mask is None else mask.to(dev))
    rg, rb = gdn_ref.g_beta(b, a, A_log, dt_bias, mask)
    torch.testing.assert_close(g.cpu(), rg, rtol=2e-6, atol=1e-7)
    # beta: at most one bf16 ulp apart (exp implementations differ in the last bit)
    d = (beta.cpu().view(torch.int16).int() - rb.view(torch.int16).int()).abs().max().item()
    assert d <= 1
    assert beta.dtype == BF16 and g.dtype == torch.float32
    if mask is not None:
        assert torch.all(g.cpu()[~mask] == 0)
    assert beta.cpu()[0, 0, 1].item() == 0.5


# ---------------------------------------------------------------------- conv --
@pytest.mark.parametrize("Hk,Hv,D", [(4, 4, 64), (2, 4, 128)])
def test_conv_varlen(pkg, dev, Hk, Hv, D):
    gen = _gen(12)
    C = 2 * Hk * D + Hv * D
    lens = [1, 2, 3, 64, 65, 200, 0, 130]
    N = sum(lens)
    x = torch.randn(N, C, generator=gen).to(BF16)
    x[0, :8] = -0.0                               # -0 inputs roll to +0 (reference add)
    state = torch.randn(len(lens), C, 3, generator=gen).to(BF16)
    w = (torch.randn(C, 4, generator=gen) * 0.5).to(BF16)
    cu = cu_of(lens)
    ry, rstate = gdn_ref.conv_varlen(x, state, w, lens)
    sd = state.to(dev)
    lens_d = torch.tensor(lens, dtype=torch.int32, device=dev)
    cu_d = torch.tensor(cu[:-1], dtype=torch.int32, device=dev)
    q, k, v = pkg.ops.causal_conv_silu_varlen_parts(x.to(dev), sd, w.to(dev), lens_d, cu_d, Hk * D)
    y = torch.cat([q, k, v], dim=1).cpu()
    assert_out(y, ry, "conv varlen")
    assert torch.equal(sd.cpu().view(torch.int16), rstate.view(torch.int16)), "conv state roll not bit-exact"


def test_conv_varlen_reference_layout_and_pool(pkg, dev):
    """[3, N, C/3] output layout, and the in-place pool form (state_ids)."""
    gen = _gen(13)
    Hk = Hv = 2
    D = 128
    C = 3 * Hk * D
    lens = [5, 70, 129]
    N = sum(lens)
    x = torch.randn(N, C, generator=gen).to(BF16)
    w = (torch.randn(C, 4, generator=gen) * 0.5).to(BF16)
    pool = torch.randn(9, C, 3, generator=gen).to(BF16)
    ids = [7, 2, 4]
    ry, rstate = gdn_ref.conv_varlen(x, pool[ids], w, lens)
    lens_d = torch.tensor(lens, dtype=torch.int32, device=dev)
    cu_d = torch.tensor(cu_of(lens)[:-1], dtype=torch.int32, device=dev)
    gathered = pool[ids].to(dev)
    y3 = pkg.ops.causal_conv_silu_varlen(x.to(dev), gathered, w.to(dev), lens_d, cu_d)
    assert y3.shape == (3, N, C // 3) and y3.is_contiguous()
    assert_out(torch.cat([y3[0], y3[1], y3[2]], dim=1), ry, "conv [3,N,C/3]")
    assert torch.equal(gathered.cpu(), rstate)
    pool_d = pool.to(dev)
    pkg.ops.causal_conv_silu_varlen_parts(x.to(dev), pool_d, w.to(dev), lens_d, cu_d, Hk * D,
                                          state_ids=torch.tensor(ids, device=dev))
    exp = pool.clone()
    exp[ids] = rstate
    assert torch.equal(pool_d.cpu(), exp)


@pytest.mark.parametrize("C", [6144, 8192, 776])
def test_conv_decode(pkg, dev, C):
    gen = _gen(14)
    B, slots = 37, 64
    x = torch.randn(B, C, generator=gen).to(BF16)
    x[0, :4] = -0.0
    pool = torch.randn(slots, C, 3, generator=gen).to(BF16)
    w = (torch.randn(C, 4, generator=gen) * 0.5).to(BF16)
    ids = torch.randperm(slots, generator=gen)[:B]
    ry, rpool = gdn_ref.conv_decode(x, pool, ids.tolist(), w)
    pool_d = pool.to(dev)
    y = pkg.ops.conv_decode_step(x.to(dev), pool_d, ids.to(dev), w.to(dev))
    assert_out(y.cpu(), ry, "conv decode")
    assert torch.equal(pool_d.cpu().view(torch.int16), rpool.view(torch.int16))


def test_conv_decode_strided_pool_view(pkg, dev):
    """Per-layer view of a [slots, L, C, 3] pool (slot stride L*C*3)."""
    gen = _gen(15)
    B, slots, L, C = 16, 20, 3, 6144
    full = torch.randn(slots, L, C, 3, generator=gen).to(BF16)
    x = torch.randn(B, C, generator=gen).to(BF16)
    w = (torch.randn(C, 4, generator=gen) * 0.5).to(BF16)
    ids = torch.randperm(slots, generator=gen)[:B]
    ry, rlayer = gdn_ref.conv_decode(x, full[:, 1].clone(), ids.tolist(), w)
    full_d = full.to(dev)
    y = pkg.ops.conv_decode_step(x.to(dev), full_d[:, 1], ids.to(dev), w.to(dev))
    assert_out(y.cpu(), ry, "conv decode strided")
    exp = full.clone()
    exp[:, 1] = rlayer
    assert torch.equal(full_d.cpu(), exp)


@pytest.mark.parametrize("layout,n,C,T", [
    ("chan", 5, 6144, 100),     # [n, T, C] rows seen as [n, C, T] (the reference's layout); 4-byte stores
    ("chan", 3, 200, 128),      # partial channel tile, 16-byte loads and stores
    ("chan", 2, 100, 50),       # C not a multiple of 8: the element-wise kernel
    ("tok", 3, 192, 128),       # [n, C, T] contiguous: 16-byte accesses
    ("tok", 4, 96, 70),         # T not a multiple of 8: 4-byte accesses, a partial last group
    ("tok", 2, 136, 600),       # many 8-token groups per channel (halo from the previous group)
    ("tok_odd", 3, 100, 66),    # token stride 1, odd sequence stride: 2-byte accesses
    ("strided", 2, 72, 90),     # neither stride 1: the element-wise kernel
])
def test_conv_padded(pkg, dev, layout, n, C, T):
    """The padded conv (a6) against the oracle for each input layout the
    kernels load differently, with end positions at, inside and before the
    tokens."""
    gen = _gen(16)
    if layout == "chan":
        xm = torch.randn(n, T, C, generator=gen).to(BF16)
        x, xd = xm.transpose(1, 2), xm.to(dev).transpose(1, 2)       # [n, C, T], channel stride 1
    elif layout == "tok":
        x = torch.randn(n, C, T, generator=gen).to(BF16)
        xd = x.to(dev)
    elif layout == "tok_odd":
        big = torch.randn(n, 2 * C + 1, T + 3, generator=gen).to(BF16)
        x = big[:, 1::2, 3:]                                        # channel stride 2 (T + 3), token stride 1
        xd = big.to(dev)[:, 1::2, 3:]
    else:
        big = torch.randn(n, 2 * C, 2 * T, generator=gen).to(BF16)
        x = big[:, ::2, ::2]                                        # channel stride 4 T, token stride 2
        xd = big.to(dev)[:, ::2, ::2]
    state = torch.randn(n, C, 3, generator=gen).to(BF16)
    w = (torch.randn(C, 4, generator=gen) * 0.5).to(BF16)
    endp = ([T, 2, -1, 0, min(57, T)] * 2)[:n]
    ry, rstate = gdn_ref.conv_padded(x, state, w, endp)
    sd = state.to(dev)
    y = pkg.ops.causal_conv_silu(xd, sd, w.to(dev), torch.tensor(endp, dtype=torch.int32, device=dev))
    assert y.shape == (n, C, T) and y.is_contiguous()
    assert_out(y.cpu(), ry, f"conv padded {layout}")
    assert torch.equal(sd.cpu(), rstate)


# ---------------------------------------------------------------- gated norm --
@pytest.mark.parametrize("D", [64, 128])
def test_rmsnorm_gated(pkg, dev, D):
    gen = _gen(17)
    N, H = 333, 16
    x = torch.randn(N, H, D, generator=gen).to(BF16)
    z = torch.randn(N, H, D, generator=gen).to(BF16)
    w = (1 + 0.02 * torch.randn(D, generator=gen)).to(BF16)
    ref = gdn_ref.rms_norm_gated(x, z, w, 1e-6)
    y = pkg.ops.rms_norm_gated(x.to(dev), z.to(dev), w.to(dev), 1e-6)
    assert_out(y.cpu(), ref, "rmsnorm gated")
    # same rounding order: all but a handful of elements are bit-identical
    diff = (y.cpu().view(torch.int16) != ref.view(torch.int16)).float().mean().item()
    assert diff < 1e-3, f"{diff:.2e} of elements differ"


# ----------------------------------------------------------- recurrent rule --
@pytest.mark.parametrize("B,Hk,Hv,D", [(9, 4, 4, 128), (300, 2, 4, 128), (5, 4, 8, 64), (700, 16, 16, 128)])
def test_recurrent_inplace(pkg, dev, B, Hk, Hv, D):
    gen = _gen(18)
    slots = B + 11
    C = 2 * Hk * D + Hv * D
    mixed = torch.randn(B, C, generator=gen).to(BF16)      # strided q/k/v views of one buffer
    a, b, A_log, dt_bias = gates(gen, B, Hv)
    g, beta = gdn_ref.g_beta(b, a, A_log, dt_bias)
    pool = torch.randn(slots, Hv, D, D, generator=gen) * 0.1
    ids = torch.randperm(slots, generator=gen)[:B]
    kd = Hk * D
    q = mixed[:, :kd].view(B, 1, Hk, D)
    k = mixed[:, kd:2 * kd].view(B, 1, Hk, D)
    v = mixed[:, 2 * kd:].view(B, 1, Hv, D)
    ro, rS, _ = gdn_ref.recurrent_rule(q, k, v, g.view(B, 1, Hv), beta.float().view(B, 1, Hv), pool[ids])
    md = mixed.to(dev)
    pool_d = pool.to(dev)
    o = pkg.ops.recurrent_gdn_inplace(md[:, :kd].view(B, 1, Hk, D), md[:, kd:2 * kd].view(B, 1, Hk, D),
                                      md[:, 2 * kd:].view(B, 1, Hv, D), g.view(B, 1, Hv).to(dev),
                                      beta.view(B, 1, Hv).to(dev), pool_d, ids.to(dev))
    assert o.shape == (B, 1, Hv, D)
    assert_out(o.cpu(), ro.to(BF16), "decode out")
    pool_out = pool_d.cpu()
    assert_state(pool_out[ids], rS, "decode state")
    untouched = torch.ones(slots, dtype=torch.bool)
    untouched[ids] = False
    assert torch.equal(pool_out[untouched], pool[untouched]), "untouched slots changed"


def test_recurrent_dummy_slot_duplicates(pkg, dev):
    """Graph pad rows all write the dummy slot: real slots stay exact."""
    gen = _gen(19)
    B, H, D, real = 64, 16, 128, 16
    slots = 33
    dummy = 32
    q = torch.randn(B, 1, H, D, generator=gen).to(BF16)
    k = torch.randn(B, 1, H, D, generator=gen).to(BF16)
    v = torch.randn(B, 1, H, D, generator=gen).to(BF16)
    a, b, A_log, dt_bias = gates(gen, B, H)
    g, beta = gdn_ref.g_beta(b, a, A_log, dt_bias)
    pool = torch.randn(slots, H, D, D, generator=gen) * 0.1
    ids = torch.full((B,), dummy, dtype=torch.int64)
    ids[:real] = torch.randperm(dummy, generator=gen)[:real]
    ro, rS, _ = gdn_ref.recurrent_rule(q[:real], k[:real], v[:real], g[:real].view(real, 1, H),
                                       beta[:real].float().view(real, 1, H), pool[ids[:real]])
    pool_d = pool.to(dev)
    o = pkg.ops.recurrent_gdn_inplace(q.to(dev), k.to(dev), v.to(dev), g.view(B, 1, H).to(dev),
                                      beta.view(B, 1, H).to(dev), pool_d, ids.to(dev))
    torch.cuda.synchronize()
    assert_out(o[:real].cpu(), ro.to(BF16), "real rows")
    assert_state(pool_d.cpu()[ids[:real]], rS, "real slots")


@pytest.mark.parametrize("T", [2, 4])
def test_recurrent_multitoken_and_commit(pkg, dev, T):
    """Spec-verify decode (GVA 16/32 at D=128): per-token states and rollback."""
    gen = _gen(20)
    B, Hk, Hv, D, slots = 12, 4, 8, 128, 20
    q = torch.randn(B, T, Hk, D, generator=gen).to(BF16)
    k = torch.randn(B, T, Hk, D, generator=gen).to(BF16)
    v = torch.randn(B, T, Hv, D, generator=gen).to(BF16)
    a, b, A_log, dt_bias = gates(gen, B * T, Hv)
    g, beta = gdn_ref.g_beta(b, a, A_log, dt_bias)
    g, beta = g.view(B, T, Hv), beta.view(B, T, Hv)
    pool = torch.randn(slots, Hv, D, D, generator=gen) * 0.1
    ids = torch.randperm(slots, generator=gen)[:B]
    ro, rS, rstates = gdn_ref.recurrent_rule(q, k, v, g, beta.float(), pool[ids], keep_states=True)
    pool_d = pool.to(dev)
    inter = torch.empty(B, T, Hv, D, D, device=dev)
    o = pkg.ops.recurrent_gdn_multitoken(q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev), pool_d,
                                         ids.to(dev), intermediate_states=inter)
    assert_out(o.cpu(), ro.to(BF16), "multitoken out")
    assert torch.equal(pool_d.cpu(), pool), "pool must be untouched when intermediates are requested"
    assert_state(inter.cpu(), rstates, "intermediate states")
    accepted = torch.randint(0, T + 1, (B,), generator=gen)
    pkg.ops.commit_states(pool_d, ids.to(dev), inter, accepted.to(dev))
    exp = pool.clone()
    for i in range(B):
        if accepted[i] > 0:
            exp[ids[i]] = inter.cpu()[i, accepted[i] - 1]
    assert torch.equal(pool_d.cpu(), exp)
    # without intermediates the pool advances by all T tokens
    pool_d2 = pool.to(dev)
    o2 = pkg.ops.recurrent_gdn_multitoken(q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev), pool_d2,
                                          ids.to(dev))
    assert_out(o2.cpu(), ro.to(BF16), "multitoken out (in place)")
    assert_state(pool_d2.cpu()[ids], rS, "multitoken final")


def test_recurrent_gathered_api(pkg, dev):
    """recurrent_gated_delta_rule(q, k, v, g, beta, initial_state): out-of-place T >= 1."""
    gen = _gen(21)
    B, T, H, D = 6, 3, 16, 128
    q = torch.randn(B, T, H, D, generator=gen).to(BF16)
    k = torch.randn(B, T, H, D, generator=gen).to(BF16)
    v = torch.randn(B, T, H, D, generator=gen).to(BF16)
    a, b, A_log, dt_bias = gates(gen, B * T, H)
    g, beta = gdn_ref.g_beta(b, a, A_log, dt_bias)
    g, beta = g.view(B, T, H), beta.view(B, T, H)
    h0 = torch.randn(B, H, D, D, generator=gen) * 0.1
    ro, rS, _ = gdn_ref.recurrent_rule(q, k, v, g, beta.float(), h0)
    h0d = h0.to(dev)
    o, S = pkg.ops.recurrent_gated_delta_rule(q.to(dev), k.to(dev), v.to(dev), g=g.to(dev), beta=beta.to(dev),
                                              initial_state=h0d)
    assert_out(o.cpu(), ro.to(BF16), "gathered out")
    assert_state(S.cpu(), rS, "gathered state")
    assert torch.equal(h0d.cpu(), h0), "initial state must not be modified"


# --------------------------------------------------------------- chunk rule --
@pytest.mark.parametrize("Hk,Hv,D", [(2, 2, 128), (2, 4, 128), (4, 4, 64)])
@pytest.mark.parametrize("with_h0", [False, True])
def test_chunk_varlen(pkg, dev, Hk, Hv, D, with_h0):
    gen = _gen(22)
    lens = [1, 63, 64, 65, 200, 7, 130]
    N = sum(lens)
    q, k, v, g, beta = rule_inputs(gen, N, Hk, Hv, D)
    cu = cu_of(lens)
    h0 = torch.randn(len(lens), Hv, D, D, generator=gen) * 0.1 if with_h0 else None
    ro, rS = gdn_ref.chunk_varlen(q, k, v, g, beta.float(), cu, h0)
    o, S = pkg.ops.chunk_gated_delta_rule_varlen(q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev),
                                                 torch.tensor(cu, device=dev),
                                                 None if h0 is None else h0.to(dev))
    assert_out(o.cpu(), ro.to(BF16), "chunk out")
    assert_state(S.cpu(), rS, "chunk final")


def test_chunk_slow_decay_long(pkg, dev):
    """Slow decay (memory spans many chunks): precision of the state chain."""
    gen = _gen(23)
    Hk = Hv = 2
    D = 128
    lens = [1500, 333]
    N = sum(lens)
    q, k, v, g, beta = rule_inputs(gen, N, Hk, Hv, D, slow_decay=True)
    cu = cu_of(lens)
    h0 = torch.randn(len(lens), Hv, D, D, generator=gen) * 0.1
    ro, rS = gdn_ref.chunk_varlen(q, k, v, g, beta.float(), cu, h0)
    o, S = pkg.ops.chunk_gated_delta_rule_varlen(q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev),
                                                 torch.tensor(cu, device=dev), h0.to(dev))
    assert_out(o.cpu(), ro.to(BF16), "chunk slow-decay out")
    assert_state(S.cpu(), rS, "chunk slow-decay final")


def test_chunk_pool_inplace_and_padded_api(pkg, dev):
    """State pool read / written in place at slot ids; batched [B, T, H, D] API."""
    gen = _gen(24)
    H, D = 4, 128
    lens = [100, 64, 30]
    N = sum(lens)
    q, k, v, g, beta = rule_inputs(gen, N, H, H, D)
    cu = cu_of(lens)
    pool = torch.randn(6, H, D, D, generator=gen) * 0.1
    ids = [5, 0, 3]
    ro, rS = gdn_ref.chunk_varlen(q, k, v, g, beta.float(), cu, pool[ids])
    pool_d = pool.to(dev)
    o, _ = pkg.ops.chunk_gated_delta_rule_varlen(q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev),
                                                 torch.tensor(cu, device=dev), pool_d,
                                                 state_ids=torch.tensor(ids, device=dev), final_state=pool_d)
    assert_out(o.cpu(), ro.to(BF16), "pool chunk out")
    assert_state(pool_d.cpu()[ids], rS, "pool chunk final")
    untouched = [i for i in range(6) if i not in ids]
    assert torch.equal(pool_d.cpu()[untouched], pool[untouched])
    # batched API: 3 rows of T = 64
    Bn, T = 3, 64
    qb, kb, vb, gb, bb = rule_inputs(gen, Bn * T, H, H, D)
    ro2, rS2 = gdn_ref.chunk_varlen(qb, kb, vb, gb, bb.float(), [0, 64, 128, 192], None)
    o2, S2 = pkg.ops.chunk_gated_delta_rule_ref_api(
        qb.view(Bn, T, H, D).to(dev), kb.view(Bn, T, H, D).to(dev), vb.view(Bn, T, H, D).to(dev),
        gb.view(Bn, T, H).to(dev), bb.view(Bn, T, H).to(dev))
    assert_out(o2.view(-1, H, D).cpu(), ro2.to(BF16), "batched chunk out")
    assert_state(S2.cpu(), rS2, "batched chunk final")


def test_rmsnorm_gated_token_ranges(pkg, dev):
    """The range form normalises exactly the selected tokens, as the full form
    does, and leaves the other rows of the output alone."""
    gen = _gen(61)
    N, H, D = 300, 4, 128
    x = torch.randn(N, H, D, generator=gen).to(BF16).to(dev)
    z = torch.randn(N, H, D, generator=gen).to(BF16).to(dev)
    w = (1 + 0.02 * torch.randn(D, generator=gen)).to(BF16).to(dev)
    full = pkg.ops.rms_norm_gated(x, z, w, 1e-6)
    sel = [(0, 10), (50, 1), (120, 100), (299, 1)]
    rows, before = [], 0
    for st, cnt in sel:
        rows += [st, cnt, before]
        before += cnt
    out = torch.full((N, H, D), 7.0, dtype=BF16, device=dev)
    pkg.ops.rms_norm_gated_ranges(x, z, w, 1e-6, out, torch.tensor(rows, device=dev), before)
    torch.cuda.synchronize()
    mask = torch.zeros(N, dtype=torch.bool)
    for st, cnt in sel:
        mask[st:st + cnt] = True
    assert torch.equal(out.cpu()[mask].view(torch.int16), full.cpu()[mask].view(torch.int16))
    assert torch.all(out.cpu()[~mask] == 7.0)


def test_rmsnorm_gated_token_ranges_bounded(pkg, dev):
    """Range entries that point past the rows are skipped by the kernel's own
    bounds (the in-range tokens still normalised exactly), and a range table
    larger than the rows is refused on the host."""
    gen = _gen(62)
    N, H, D = 64, 2, 128
    x = torch.randn(N, H, D, generator=gen).to(BF16).to(dev)
    z = torch.randn(N, H, D, generator=gen).to(BF16).to(dev)
    w = (1 + 0.02 * torch.randn(D, generator=gen)).to(BF16).to(dev)
    full = pkg.ops.rms_norm_gated(x, z, w, 1e-6)
    # (first token, count, before): tokens 60..63 valid, 64..67 past the rows
    rows = torch.tensor([60, 8, 0], device=dev)
    out = torch.full((N, H, D), 7.0, dtype=BF16, device=dev)
    pkg.ops.rms_norm_gated_ranges(x, z, w, 1e-6, out, rows, 8)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu()[60:].view(torch.int16), full.cpu()[60:].view(torch.int16))
    assert torch.all(out.cpu()[:60] == 7.0)
    with pytest.raises(pkg._lib.GDNKernelError):
        pkg.ops.rms_norm_gated_ranges(x, z, w, 1e-6, out, rows, N + 1)


def test_state_tile_pass_leaves_pool_unchanged(pkg, dev):
    """The measurement pass reads and writes back the selected state tiles of a
    per-layer pool view: every bit of the pool (other layers, other slots,
    duplicated ids included) is as before."""
    gen = _gen(63)
    slots, L, Hv, D = 12, 3, 4, 128
    pool = torch.randn(slots, L, Hv, D, D, generator=gen).to(dev)
    before = pool.clone()
    ids = torch.tensor([5, 0, 11, 5], device=dev)
    pkg.ops.state_tile_pass(pool[:, 1], ids)
    torch.cuda.synchronize()
    assert torch.equal(pool.cpu().view(torch.int32), before.cpu().view(torch.int32))
