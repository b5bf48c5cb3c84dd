"""The state pass's column split (gdn_set_column_split): each sequence's heads
in 64-column workgroups, in 32-column ones, or the automatic mix (the longest
sequences in 32-column ones when that shortens the pass) give the same
outputs, final states and conv states bit for bit, since a state's value
columns evolve independently.  Covered for the fused prefill and for the
chunk rule alone, with initial states, grouped heads, D = 64 and ragged and
empty sequences; the all-narrow pass of the chunk rule is also held to the
CPU oracle."""
import pytest
import torch

from helpers import BF16, assert_out, assert_state, cu_of, rule_inputs
from oracle import gdn_ref
from test_gpu_fused_prefill import _case

pytestmark = pytest.mark.gpu

MODES = (1, 2, 0)  # all 64-column, all 32-column, automatic


@pytest.fixture
def split(pkg):
    lib = pkg._lib.load()
    yield lib.gdn_set_column_split
    lib.gdn_set_column_split(0)


def _same(x, y):
    if x.dtype == torch.bfloat16:
        return torch.equal(x.view(torch.int16), y.view(torch.int16))
    return torch.equal(x.view(torch.int32), y.view(torch.int32))


FUSED = [
    # Hk, Hv, D, lens
    (4, 4, 128, [1, 2, 3, 70, 200, 64, 0, 129, 1500]),
    (2, 4, 128, [3000, 5, 640, 1]),
    (4, 4, 64, [3, 1150, 66, 0, 2]),
    (16, 16, 128, [1374, 3778, 2225, 3022, 3204, 498, 2641, 259]),  # config 1's lengths
]


@pytest.mark.parametrize("Hk,Hv,D,lens", FUSED, ids=lambda c: str(c))
def test_fused_prefill_modes_bit_equal(pkg, dev, split, Hk, Hv, D, lens):
    slots = len(lens) + 2
    C, mixed, conv_w, A_log, dt_bias, a, b, conv_pool, s_pool, ids = _case(61, Hk, Hv, D, lens, slots)
    mixed, conv_w, A_log, dt_bias, a, b, ids = (t.to(dev) for t in (mixed, conv_w, A_log, dt_bias, a, b, ids))
    cu_h = torch.tensor(cu_of(lens), dtype=torch.int64)
    cu_d = cu_h.to(dev)
    res = {}
    for m in MODES:
        assert split(m) == 0
        cp, sp = conv_pool.to(dev), s_pool.to(dev)
        o = pkg.ops.conv_chunk_prefill_varlen(mixed, cp, conv_w, b, a, A_log, dt_bias, cu_d, sp, ids, Hk, Hv, D,
                                              cu_seqlens_cpu=cu_h)
        torch.cuda.synchronize()
        res[m] = (o.cpu(), sp.cpu(), cp.cpu())
    for m in (2, 0):
        for what, x, y in zip(("outputs", "state pool", "conv pool"), res[m], res[1]):
            assert _same(x, y), f"mode {m}: {what} differ from the 64-column pass"


RULE = [
    # Hk, Hv, D, lens
    (2, 4, 128, [1000, 3, 450, 2000]),
    (4, 4, 64, [129, 900, 0, 5]),
    (2, 2, 128, [64, 65, 1]),
]


@pytest.mark.parametrize("Hk,Hv,D,lens", RULE, ids=lambda c: str(c))
def test_chunk_rule_modes_bit_equal_and_oracle(pkg, dev, split, Hk, Hv, D, lens):
    gen = torch.Generator().manual_seed(62)
    N = sum(lens)
    q, k, v, g, beta = rule_inputs(gen, N, Hk, Hv, D)
    cu = cu_of(lens)
    h0 = torch.randn(len(lens), Hv, D, D, generator=gen) * 0.1
    cu_h = torch.tensor(cu, dtype=torch.int64)
    args = (q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev), cu_h.to(dev), h0.to(dev))
    res = {}
    for m in MODES:
        assert split(m) == 0
        # one pass (no segments), so the column split decides the launch
        o, S = pkg.ops.chunk_gated_delta_rule_varlen(*args, cu_seqlens_cpu=cu_h, max_segments=1)
        torch.cuda.synchronize()
        res[m] = (o.cpu(), S.cpu())
    for m in (2, 0):
        assert _same(res[m][0], res[1][0]), f"mode {m}: outputs differ from the 64-column pass"
        assert _same(res[m][1], res[1][1]), f"mode {m}: final states differ from the 64-column pass"
    ro, rS = gdn_ref.chunk_varlen(q, k, v, g, beta.float(), cu, h0)
    assert_out(res[2][0], ro.to(BF16), "32-column pass out")
    assert_state(res[2][1], rS, "32-column pass final")
