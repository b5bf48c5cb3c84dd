"""Pins the CPU oracle (oracle/gdn_ref.py), which the GPU parity tests trust.

Each oracle function is checked against something it is not a restatement
of: the golden vectors written by tests/golden/make_golden.py from the
upstream transformers functions the reference ports; the fp64 brute-force
recurrence (oracle/recurrence.c); F.conv1d; closed forms and invariants.
CPU only."""
import math
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from helpers import cu_of, rule_inputs, state_rel
from oracle import gdn_ref

GOLDEN = Path(__file__).resolve().parent / "golden"


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a))


@pytest.fixture(scope="module")
def c0():
    return dict(np.load(GOLDEN / "config0.npz"))


@pytest.fixture(scope="module")
def edge():
    return dict(np.load(GOLDEN / "edge.npz"))


# ------------------------------------------------------------ golden vectors --
def test_golden_conv(c0):
    x, w = _t(c0["x"]), _t(c0["w"])
    T, C = x.shape
    y, st = gdn_ref.conv_varlen(x, torch.zeros(1, C, 3), w, [T])
    torch.testing.assert_close(y, _t(c0["conv_y"]), rtol=1e-5, atol=1e-6)
    # the new state is the last 3 raw inputs
    assert torch.equal(st[0], x[-3:].t())


def test_golden_g_beta(c0):
    g, beta = gdn_ref.g_beta(_t(c0["b"]), _t(c0["a"]), _t(c0["A_log"]), _t(c0["dt_bias"]))
    # log(1 + exp(z)) (the reference's Triton form) vs F.softplus's log1p: a few ulp
    torch.testing.assert_close(g, _t(c0["g"]), rtol=3e-6, atol=1e-7)
    torch.testing.assert_close(beta.float(), _t(c0["beta"]), rtol=4e-3, atol=0)   # oracle rounds beta to bf16


def test_golden_chunk_rule(c0):
    y = _t(c0["conv_y"])
    T, C = y.shape
    H, D = 4, 64
    q, k, v = (y[:, i * H * D:(i + 1) * H * D].reshape(T, H, D) for i in range(3))
    o, S = gdn_ref.chunk_rule(q, k, v, _t(c0["g"]), _t(c0["beta"]))
    torch.testing.assert_close(o, _t(c0["o_chunk"]), rtol=1e-4, atol=1e-6)
    assert state_rel(S, _t(c0["state_chunk"])) < 1e-5


def test_golden_recurrent_rule(c0):
    y = _t(c0["conv_y"])
    T, C = y.shape
    H, D = 4, 64
    q, k, v = (y[:, i * H * D:(i + 1) * H * D].reshape(1, T, H, D) for i in range(3))
    o, S, _ = gdn_ref.recurrent_rule(q, k, v, _t(c0["g"])[None], _t(c0["beta"])[None])
    torch.testing.assert_close(o[0, -64:], _t(c0["o_rec_tail"]), rtol=1e-4, atol=1e-6)
    assert state_rel(S[0], _t(c0["state_rec"])) < 1e-5


def test_golden_gated_norm_fp32(c0):
    o = _t(c0["o_chunk"])[:32]
    y = gdn_ref.rms_norm_gated(o, _t(c0["z"]), _t(c0["norm_w"]))
    torch.testing.assert_close(y, _t(c0["y_norm"]), rtol=1e-5, atol=1e-6)


def test_golden_gated_norm_bf16_rounding(edge):
    nx, nz = _t(edge["nx"]).view(torch.bfloat16), _t(edge["nz"]).view(torch.bfloat16)
    nw = _t(edge["nw"]).view(torch.bfloat16)
    ny = _t(edge["ny"]).view(torch.bfloat16)
    y = gdn_ref.rms_norm_gated(nx, nz, nw)
    # same eager rounding order: bit-identical
    assert torch.equal(y.view(torch.int16), ny.view(torch.int16))


def test_golden_edge_chunk_gva_h0(edge):
    q, k, v = _t(edge["q"]), _t(edge["k"]), _t(edge["v"])
    g, beta, h0 = _t(edge["g"]), _t(edge["beta"]), _t(edge["h0"])
    o, S = gdn_ref.chunk_varlen(q, k, v, g, beta, [0, q.shape[0]], h0[None])
    torch.testing.assert_close(o, _t(edge["o_chunk"]), rtol=1e-4, atol=1e-6)
    assert state_rel(S[0], _t(edge["state_chunk"])) < 1e-5
    o2, S2, _ = gdn_ref.recurrent_rule(q[None], k[None], v[None], g[None], beta[None], h0[None])
    torch.testing.assert_close(o2[0], _t(edge["o_rec"]), rtol=1e-4, atol=1e-6)
    assert state_rel(S2[0], _t(edge["state_rec"])) < 1e-5


def test_golden_conv_update(edge):
    cx, cstate, cw = _t(edge["cx"]), _t(edge["cstate"]), _t(edge["cw"])
    y, pool = gdn_ref.conv_decode(cx, cstate, [0, 1, 2], cw)
    torch.testing.assert_close(y, _t(edge["cy"]), rtol=1e-5, atol=1e-6)
    assert torch.equal(pool, _t(edge["cstate_after"]))


# ------------------------------------------------- fp64 brute-force recurrence --
@pytest.mark.parametrize("Hk,Hv,D,lens,slow", [
    (2, 2, 64, [1, 63, 64, 65, 130], False),
    (1, 2, 32, [200], True),
    (2, 4, 16, [7, 70], False),
])
def test_chunk_matches_f64_recurrence(Hk, Hv, D, lens, slow):
    gen = torch.Generator().manual_seed(3)
    N = sum(lens)
    q, k, v, g, beta = rule_inputs(gen, N, Hk, Hv, D, slow_decay=slow)
    cu = cu_of(lens)
    h0 = torch.randn(len(lens), Hv, D, D, generator=gen) * 0.1
    o, S = gdn_ref.chunk_varlen(q, k, v, g, beta.float(), cu, h0)
    for r in range(len(lens)):
        a, b = cu[r], cu[r + 1]
        o64, s64 = oracle.recurrence_f64(q[a:b].float(), k[a:b].float(), v[a:b].float(), g[a:b],
                                         beta[a:b].float(), h0[r])
        assert (o[a:b].double() - o64).abs().max().item() < 1e-5
        assert state_rel(S[r], s64) < 1e-5


def test_recurrent_matches_f64_recurrence():
    gen = torch.Generator().manual_seed(4)
    q, k, v, g, beta = rule_inputs(gen, 40, 2, 4, 32)
    h0 = torch.randn(4, 32, 32, generator=gen) * 0.1
    o, S, states = gdn_ref.recurrent_rule(q[None], k[None], v[None], g[None], beta.float()[None], h0[None],
                                          keep_states=True)
    o64, s64 = oracle.recurrence_f64(q.float(), k.float(), v.float(), g, beta.float(), h0)
    assert (o[0].double() - o64).abs().max().item() < 1e-5
    assert state_rel(S[0], s64) < 1e-5
    # per-token states are the recurrence prefixes (rollback semantics)
    for t in (0, 9, 39):
        _, s_t = oracle.recurrence_f64(q[:t + 1].float(), k[:t + 1].float(), v[:t + 1].float(), g[:t + 1],
                                       beta[:t + 1].float(), h0)
        assert state_rel(states[0, t], s_t) < 1e-5


# ------------------------------------------------------------- closed forms --
def test_beta0_g0_leaves_state_and_reads_it():
    gen = torch.Generator().manual_seed(6)
    T, H, D = 70, 2, 16
    q = torch.randn(T, H, D, generator=gen)
    k = torch.randn(T, H, D, generator=gen)
    v = torch.randn(T, H, D, generator=gen)
    h0 = torch.randn(H, D, D, generator=gen)
    z = torch.zeros(T, H)
    o, S = gdn_ref.chunk_rule(q, k, v, z, z, h0)
    assert torch.allclose(S, h0, atol=1e-6)
    qn = q / torch.sqrt((q * q).sum(-1, keepdim=True) + 1e-6) * D ** -0.5
    torch.testing.assert_close(o, torch.einsum("thk,hkv->thv", qn, h0), rtol=1e-5, atol=1e-6)


def test_single_token_from_zero_state():
    gen = torch.Generator().manual_seed(7)
    H, D = 3, 16
    q = torch.randn(1, H, D, generator=gen)
    k = torch.randn(1, H, D, generator=gen)
    v = torch.randn(1, H, D, generator=gen)
    beta = torch.rand(1, H, generator=gen)
    o, S = gdn_ref.chunk_rule(q, k, v, torch.zeros(1, H), beta)
    kn = k[0] / torch.sqrt((k[0] ** 2).sum(-1, keepdim=True) + 1e-6)
    qn = q[0] / torch.sqrt((q[0] ** 2).sum(-1, keepdim=True) + 1e-6) * D ** -0.5
    S_exp = beta[0][:, None, None] * kn[:, :, None] * v[0][:, None, :]
    torch.testing.assert_close(S, S_exp, rtol=1e-5, atol=1e-6)
    o_exp = (beta[0] * (qn * kn).sum(-1))[:, None] * v[0]
    torch.testing.assert_close(o[0], o_exp, rtol=1e-5, atol=1e-6)


def test_strong_decay_resets_memory():
    """exp(g) -> 0 at token t: the final state only depends on tokens >= t.
    (g = -60: e^g ~ 1e-26; far larger |g| only adds fp32 cancellation in the
    in-chunk cumsum differences, shared by the reference's formulation.)"""
    gen = torch.Generator().manual_seed(8)
    q, k, v, g, beta = rule_inputs(gen, 100, 2, 2, 16)
    g = g.clone()
    g[60] = -60.0
    h0a = torch.randn(2, 16, 16, generator=gen)
    _, Sa = gdn_ref.chunk_rule(q, k, v, g, beta.float(), h0a)
    _, Sb = gdn_ref.chunk_rule(q, k, v, g, beta.float(), None)
    _, Sc = gdn_ref.chunk_rule(q[60:], k[60:], v[60:], g[60:], beta[60:].float(), None)
    assert state_rel(Sa, Sc) < 2e-5 and state_rel(Sb, Sc) < 2e-5


def test_linear_in_v_and_affine_in_h0():
    gen = torch.Generator().manual_seed(9)
    q, k, v, g, beta = rule_inputs(gen, 90, 2, 2, 16)
    v2 = torch.randn_like(v.float())
    o1, S1 = gdn_ref.chunk_rule(q, k, v.float(), g, beta.float())
    o2, S2 = gdn_ref.chunk_rule(q, k, v2, g, beta.float())
    o3, S3 = gdn_ref.chunk_rule(q, k, 2.0 * v.float() - 3.0 * v2, g, beta.float())
    torch.testing.assert_close(o3, 2 * o1 - 3 * o2, rtol=1e-4, atol=1e-5)
    torch.testing.assert_close(S3, 2 * S1 - 3 * S2, rtol=1e-4, atol=1e-5)
    # affine in h0: S(h0a + h0b) - S(0) = [S(h0a) - S(0)] + [S(h0b) - S(0)]
    h0a = torch.randn(2, 16, 16, generator=gen)
    h0b = torch.randn(2, 16, 16, generator=gen)
    _, Sa = gdn_ref.chunk_rule(q, k, v.float(), g, beta.float(), h0a)
    _, Sb = gdn_ref.chunk_rule(q, k, v.float(), g, beta.float(), h0b)
    _, Sab = gdn_ref.chunk_rule(q, k, v.float(), g, beta.float(), h0a + h0b)
    torch.testing.assert_close(Sab - S1, (Sa - S1) + (Sb - S1), rtol=1e-4, atol=1e-5)


def test_segmented_prefill_equals_one_call():
    """Threading the final state into the next segment equals one call
    (the reference's in-layer segmentation, qwen3_5.py:853-862)."""
    gen = torch.Generator().manual_seed(10)
    q, k, v, g, beta = rule_inputs(gen, 300, 2, 2, 32)
    o, S = gdn_ref.chunk_rule(q, k, v, g, beta.float())
    o1, S1 = gdn_ref.chunk_rule(q[:111], k[:111], v[:111], g[:111], beta[:111].float())
    o2, S2 = gdn_ref.chunk_rule(q[111:], k[111:], v[111:], g[111:], beta[111:].float(), S1)
    torch.testing.assert_close(torch.cat([o1, o2]), o, rtol=1e-4, atol=1e-5)
    assert state_rel(S2, S) < 1e-5


def test_decode_equals_chunk_with_one_token():
    gen = torch.Generator().manual_seed(11)
    q, k, v, g, beta = rule_inputs(gen, 5, 2, 2, 32)
    h0 = torch.randn(5, 2, 32, 32, generator=gen) * 0.1
    o, S, _ = gdn_ref.recurrent_rule(q[:, None], k[:, None], v[:, None], g[:, None], beta.float()[:, None], h0)
    for b in range(5):
        oc, Sc = gdn_ref.chunk_rule(q[b:b + 1], k[b:b + 1], v[b:b + 1], g[b:b + 1], beta[b:b + 1].float(), h0[b])
        torch.testing.assert_close(o[b], oc, rtol=1e-5, atol=1e-6)
        assert state_rel(S[b], Sc) < 1e-5


# ----------------------------------------------------------------- g / beta --
def test_g_beta_special_cases():
    a = torch.tensor([[25.0, -3.0, 0.0]])
    b = torch.tensor([[0.0, 3.0, -3.0]])
    A_log = torch.tensor([0.5, 1.0, 2.0])
    dt = torch.tensor([0.0, 0.5, -0.5])
    g, beta = gdn_ref.g_beta(b, a, A_log, dt)
    assert g[0, 0].item() == pytest.approx(-math.exp(0.5) * 25.0, rel=1e-6)          # threshold branch
    assert g[0, 1].item() == pytest.approx(-math.exp(1.0) * math.log1p(math.exp(-2.5)), rel=1e-5)
    assert beta[0, 0].item() == 0.5
    mask = torch.tensor([False])
    g2, _ = gdn_ref.g_beta(b, a, A_log, dt, mask)
    assert torch.all(g2 == 0)


# --------------------------------------------------------------------- conv --
def test_conv_varlen_equals_conv1d_and_rolls_state():
    gen = torch.Generator().manual_seed(12)
    C, lens = 24, [5, 1, 2, 9]
    x = torch.randn(sum(lens), C, generator=gen).to(torch.bfloat16)
    x[0, 0] = -0.0
    state = torch.randn(len(lens), C, 3, generator=gen).to(torch.bfloat16)
    w = (torch.randn(C, 4, generator=gen) * 0.5).to(torch.bfloat16)
    y, st = gdn_ref.conv_varlen(x, state, w, lens)
    off = 0
    for r, T in enumerate(lens):
        win = torch.cat([state[r].float(), x[off:off + T].float().t()], dim=1)[None]
        ref = F.silu(F.conv1d(win, w.float()[:, None, :], groups=C))[0].t()
        torch.testing.assert_close(y[off:off + T].float(), ref, rtol=1e-2, atol=1e-2)
        raw = torch.cat([state[r], x[off:off + T].t()], dim=1)[:, -3:]
        exp = torch.where(raw.float() == 0, torch.zeros_like(raw), raw)          # -0 rolls to +0
        assert torch.equal(st[r].view(torch.int16), exp.view(torch.int16))
        off += T


def test_conv_segmented_equals_one_call_and_padded_matches_varlen():
    gen = torch.Generator().manual_seed(13)
    C, T = 16, 20
    x = torch.randn(T, C, generator=gen).to(torch.bfloat16)
    st0 = torch.randn(1, C, 3, generator=gen).to(torch.bfloat16)
    w = (torch.randn(C, 4, generator=gen) * 0.5).to(torch.bfloat16)
    y, st = gdn_ref.conv_varlen(x, st0, w, [T])
    y1, s1 = gdn_ref.conv_varlen(x[:7], st0, w, [7])
    y2, s2 = gdn_ref.conv_varlen(x[7:], s1, w, [T - 7])
    assert torch.equal(torch.cat([y1, y2]), y) and torch.equal(s2, st)
    yp, sp = gdn_ref.conv_padded(x.t()[None], st0, w, [T])
    assert torch.equal(yp[0].t(), y) and torch.equal(sp, st)
    # endp = -1 keeps the state; endp = 0 re-writes the old state
    _, keep = gdn_ref.conv_padded(x.t()[None], st0, w, [-1])
    assert torch.equal(keep, st0)


def test_decode_conv_is_one_token_varlen():
    gen = torch.Generator().manual_seed(14)
    C = 32
    pool = torch.randn(4, C, 3, generator=gen).to(torch.bfloat16)
    x = torch.randn(2, C, generator=gen).to(torch.bfloat16)
    w = (torch.randn(C, 4, generator=gen) * 0.5).to(torch.bfloat16)
    y, newp = gdn_ref.conv_decode(x, pool, [3, 1], w)
    yv, sv = gdn_ref.conv_varlen(x, pool[[3, 1]], w, [1, 1])
    assert torch.equal(y, yv)
    # decode roll is a pure copy: compare bits of the copied entries
    assert torch.equal(newp[[3, 1]][:, :, :2], pool[[3, 1]][:, :, 1:])
    assert torch.equal(newp[[3, 1]][:, :, 2], x)
    assert torch.equal(newp[[0, 2]], pool[[0, 2]])
