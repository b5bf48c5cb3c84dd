"""Speculative-verify decode with the rollback folded into the next step
(ops.SpecVerify): the T-token kernel writes every per-token state, accept()
records the accepted lengths, and the next verify() starts each row from its
accepted state in place of the pool row -- no commit copy between steps.
Checked against the token-by-token oracle over several steps, against the
commit-copy path bit for bit, and at BASELINE config 4 (B = 64, T = 4,
Hk = 16, Hv = 32, pool [128, 32, 128, 128]).  (No reference counterpart: spec
decode is disabled for qwen3_5, nanovllm/config.py:84.)"""
import pytest
import torch

import bench
from helpers import BF16, assert_out, assert_state
from oracle import gdn_ref

pytestmark = pytest.mark.gpu


def _step_inputs(gen, B, T, Hk, Hv, D):
    q = torch.randn(B, T, Hk, D, generator=gen).to(BF16)
    k = torch.randn(B, T, Hk, D, generator=gen).to(BF16)
    v = torch.randn(B, T, Hv, D, generator=gen).to(BF16)
    a = torch.randn(B * T, Hv, generator=gen).to(BF16)
    b = torch.randn(B * T, Hv, generator=gen).to(BF16)
    return q, k, v, a, b


@pytest.mark.parametrize("B,T,Hk,Hv,D,slots", [(5, 4, 2, 4, 128, 9), (3, 3, 4, 4, 64, 6), (64, 4, 16, 32, 128, 128)])
def test_spec_verify_steps_without_commit(pkg, dev, B, T, Hk, Hv, D, slots):
    gen = torch.Generator().manual_seed(71)
    A_log = (torch.rand(Hv, generator=gen) * 2.7).to(BF16)
    dt_bias = (torch.rand(Hv, generator=gen) * 2 - 1).to(BF16)
    pool0 = torch.randn(slots, Hv, D, D, generator=gen) * 0.1
    ids = torch.randperm(slots, generator=gen)[:B]
    pool = pool0.to(dev)
    pool_commit = pool0.clone().to(dev)              # the same steps with a commit copy after each
    spec = pkg.ops.SpecVerify(pool)
    ref_state = pool0[ids].clone()                   # the oracle's logical state per row
    idd = ids.to(dev)
    inter_c = torch.empty(B, T, Hv, D, D, device=dev)
    for step in range(3):
        q, k, v, a, b = _step_inputs(gen, B, T, Hk, Hv, D)
        g, beta = gdn_ref.g_beta(b, a, A_log, dt_bias)
        g, beta = g.view(B, T, Hv), beta.view(B, T, Hv)
        acc = torch.randint(1, T + 1, (B,), generator=gen, dtype=torch.int64)
        if step == 1:
            acc[0] = T                                   # all kept
            acc[-1] = 1                                  # only the first
        args = (q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev))
        out = spec.verify(*args, idd)
        spec.accept(acc.to(dev))
        # commit-copy path on its own pool
        out_c = pkg.ops.recurrent_gdn_multitoken(*args, pool_commit, idd, inter_c)
        pkg.ops.commit_states(pool_commit, idd, inter_c, acc.to(dev))
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), out_c.view(torch.int16)), f"step {step}: outputs vs commit path"
        # oracle: token by token from the logical state, keeping the accepted prefix
        ro, _, states = gdn_ref.recurrent_rule(q, k, v, g, beta.float(), ref_state, keep_states=True)
        assert_out(out.cpu(), ro.to(BF16), f"step {step} outputs")
        ref_state = torch.stack([states[r, acc[r] - 1] for r in range(B)])
    # the pool still holds the initial states (nothing was committed), then commit()
    assert torch.equal(pool.cpu(), pool0), "pool written before commit()"
    spec.commit()
    torch.cuda.synchronize()
    assert torch.equal(pool, pool_commit), "committed pool vs commit-copy path"
    assert_state(pool.cpu()[ids], ref_state, "committed states vs oracle")
    untouched = [i for i in range(slots) if i not in ids.tolist()]
    assert torch.equal(pool.cpu()[untouched], pool0[untouched])


def test_spec_verify_accepted_out_of_range_reads_pool_row(pkg, dev):
    """An accepted count outside 1..T (0, or T + 1 from a caller that counts the
    bonus token) makes the next verify start that row from its pool row, as the
    commit copy leaves such a row untouched: both paths agree bit for bit, and
    no state past the [B, T] buffer is read."""
    gen = torch.Generator().manual_seed(72)
    B, T, Hk, Hv, D, slots = 6, 3, 2, 4, 128, 9
    A_log = (torch.rand(Hv, generator=gen) * 2.7).to(BF16)
    dt_bias = (torch.rand(Hv, generator=gen) * 2 - 1).to(BF16)
    pool0 = torch.randn(slots, Hv, D, D, generator=gen) * 0.1
    ids = torch.randperm(slots, generator=gen)[:B].to(dev)
    pool = pool0.to(dev)
    pool_commit = pool0.clone().to(dev)
    spec = pkg.ops.SpecVerify(pool)
    inter_c = torch.empty(B, T, Hv, D, D, device=dev)
    acc = torch.tensor([0, T + 1, 1, T, 0, T + 1], dtype=torch.int64, device=dev)
    for step in range(2):
        q, k, v, a, b = _step_inputs(gen, B, T, Hk, Hv, D)
        g, beta = gdn_ref.g_beta(b, a, A_log, dt_bias)
        args = (q.to(dev), k.to(dev), v.to(dev), g.view(B, T, Hv).to(dev), beta.view(B, T, Hv).to(dev))
        out = spec.verify(*args, ids)
        spec.accept(acc)
        out_c = pkg.ops.recurrent_gdn_multitoken(*args, pool_commit, ids, inter_c)
        pkg.ops.commit_states(pool_commit, ids, inter_c, acc)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), out_c.view(torch.int16)), f"step {step}: outputs vs commit path"
    spec.commit()
    torch.cuda.synchronize()
    assert torch.equal(pool, pool_commit), "committed pool vs commit-copy path"
    rows = [0, 1, 4, 5]
    assert torch.equal(pool.cpu()[ids.cpu()[rows]], pool0[ids.cpu()[rows]]), "out-of-range rows keep their pool rows"
