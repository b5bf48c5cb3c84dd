"""GPU parity of the segmented state pass: long sequences cut into segments
that run in parallel (first segment from h0; middle segments as their
zero-start result R and transition P; scan S_{s+1} = P_s S_s + R_s; later
segments again with outputs).  Checked against the CPU oracle and against the
unsegmented kernel on the same inputs."""
import pytest
import torch

from helpers import BF16, assert_out, assert_state, cu_of, rule_inputs, state_rel, STATE_REL
from oracle import gdn_ref

pytestmark = pytest.mark.gpu


CASES = [
    # Hk, Hv, D, lens, max_segments
    (2, 2, 128, [1000], 2),
    (2, 2, 128, [1000], 3),
    (2, 2, 128, [1000], 5),
    (2, 4, 128, [700, 3, 450], 4),
    (4, 4, 64, [129, 900], 12),
    (2, 2, 128, [130], 3),          # 3 chunks into 3 one-chunk segments, the last partial
]


@pytest.mark.parametrize("with_h0", [False, True])
@pytest.mark.parametrize("Hk,Hv,D,lens,segs", CASES, ids=lambda c: str(c))
def test_segmented_chunk_rule(pkg, dev, Hk, Hv, D, lens, segs, with_h0):
    gen = torch.Generator().manual_seed(51)
    N = sum(lens)
    q, k, v, g, beta = rule_inputs(gen, N, Hk, Hv, D)
    cu = cu_of(lens)
    n = len(lens)
    h0 = torch.randn(n, Hv, D, D, generator=gen) * 0.1 if with_h0 else None
    ro, rS = gdn_ref.chunk_varlen(q, k, v, g, beta.float(), cu, h0)
    cu_d = torch.tensor(cu, device=dev)
    cu_h = torch.tensor(cu, dtype=torch.int64)
    args = (q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev), cu_d, None if h0 is None else h0.to(dev))
    o_s, S_s = pkg.ops.chunk_gated_delta_rule_varlen(*args, cu_seqlens_cpu=cu_h, max_segments=segs)
    o_1, S_1 = pkg.ops.chunk_gated_delta_rule_varlen(*args, cu_seqlens_cpu=cu_h, max_segments=1)
    assert_out(o_s.cpu(), ro.to(BF16), "segmented out")
    assert_state(S_s.cpu(), rS, "segmented final")
    # against the unsegmented kernel: the same up to rounding
    assert_out(o_s.cpu(), o_1.cpu(), "segmented vs one pass")
    assert state_rel(S_s.cpu(), S_1.cpu()) < STATE_REL


def test_segmented_pool_in_place(pkg, dev):
    """Pool-indexed in-place states (h0 == hT at the slot ids): the first segment
    reads the slot, the last writes it, other slots untouched."""
    gen = torch.Generator().manual_seed(52)
    Hk = Hv = 2
    D = 128
    lens = [800, 64]
    N = sum(lens)
    q, k, v, g, beta = rule_inputs(gen, N, Hk, Hv, D)
    cu = cu_of(lens)
    pool = torch.randn(5, Hv, D, D, generator=gen) * 0.1
    ids = [3, 1]
    ro, rS = gdn_ref.chunk_varlen(q, k, v, g, beta.float(), cu, pool[ids])
    pd = pool.to(dev)
    o, _ = pkg.ops.chunk_gated_delta_rule_varlen(q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev),
                                                 torch.tensor(cu, device=dev), pd,
                                                 state_ids=torch.tensor(ids, device=dev), final_state=pd,
                                                 cu_seqlens_cpu=torch.tensor(cu), max_segments=4)
    assert_out(o.cpu(), ro.to(BF16), "pool segmented out")
    assert_state(pd.cpu()[ids], rS, "pool segmented final")
    assert torch.equal(pd.cpu()[[0, 2, 4]], pool[[0, 2, 4]])


def test_segmented_fused_prefill(pkg, dev):
    """The fused gates + conv + chunk call with segments equals the one-pass
    fused call up to rounding, with the conv states rolled once."""
    gen = torch.Generator().manual_seed(53)
    Hk, Hv, D = 2, 4, 128
    lens = [900, 5]
    N = sum(lens)
    C = 2 * Hk * D + Hv * D
    mixed = torch.randn(N, C, generator=gen).to(BF16).to(dev)
    conv_w = (torch.randn(C, 4, generator=gen) * 0.5).to(BF16).to(dev)
    A_log = (torch.rand(Hv, generator=gen) * 2.7).to(BF16).to(dev)
    dt_bias = (torch.rand(Hv, generator=gen) * 2 - 1).to(BF16).to(dev)
    a = torch.randn(N, Hv, generator=gen).to(BF16).to(dev)
    b = torch.randn(N, Hv, generator=gen).to(BF16).to(dev)
    conv0 = torch.randn(4, C, 3, generator=gen).to(BF16).to(dev)
    s0 = (torch.randn(4, Hv, D, D, generator=gen) * 0.1).to(dev)
    ids = torch.tensor([2, 0], device=dev)
    cu = torch.tensor(cu_of(lens), dtype=torch.int64)
    outs = []
    for segs in (1, 6):
        cp, sp = conv0.clone(), s0.clone()
        o = pkg.ops.conv_chunk_prefill_varlen(mixed, cp, conv_w, b, a, A_log, dt_bias, cu.to(dev), sp, ids,
                                              Hk, Hv, D, cu_seqlens_cpu=cu, max_segments=segs)
        outs.append((o.cpu(), cp.cpu(), sp.cpu()))
    (o1, c1, s1), (o6, c6, s6) = outs
    assert_out(o6, o1, "fused segmented vs one pass")
    assert state_rel(s6, s1) < STATE_REL
    assert torch.equal(c6.view(torch.int16), c1.view(torch.int16)), "conv states"
