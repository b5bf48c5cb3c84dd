"""GPU parity of the fused decode step: the q/k conv, then the gates, the v
channels' conv (with its state roll) and the in-place recurrent update in one
kernel.  Bit-equal to fused_g_beta -> conv_decode_step -> recurrent_gdn_inplace
as the layer's T == 1 branch calls them (nanovllm/models/qwen3_5.py:1008-1030),
whose own parity with the CPU oracle the kernel tests establish, and within the
oracle bars itself on one case."""
import pytest
import torch

from helpers import BF16, assert_out, assert_state
from oracle import gdn_ref

pytestmark = pytest.mark.gpu


def _case(seed, Hk, Hv, D, B, slots, param_f32):
    gen = torch.Generator().manual_seed(seed)
    C = 2 * Hk * D + Hv * D
    mixed = torch.randn(B, C, generator=gen).to(BF16)
    mixed[0, -8:] = -0.0                                         # -0 inputs roll as bits
    conv_w = (torch.randn(C, 4, generator=gen) * 0.5).to(BF16)
    A_log = (torch.rand(Hv, generator=gen) * 2.7).to(BF16)
    dt_bias = (torch.rand(Hv, generator=gen) * 2 - 1).to(BF16)
    if param_f32:
        A_log, dt_bias = A_log.float(), dt_bias.float()
    a = torch.randn(B, Hv, generator=gen).to(BF16)
    b = torch.randn(B, Hv, generator=gen).to(BF16)
    conv_pool = torch.randn(slots, C, 3, generator=gen).to(BF16)
    s_pool = torch.randn(slots, Hv, D, D, generator=gen) * 0.1
    ids = torch.randperm(slots, generator=gen)[:B]
    return mixed, conv_w, A_log, dt_bias, a, b, conv_pool, s_pool, ids


CASES = [
    # Hk, Hv, D, B, slots
    (4, 4, 128, 6, 9),          # four v-blocks per head
    (2, 4, 128, 130, 140),      # GVA, two v-blocks
    (16, 16, 128, 160, 170),    # one v-block per head
    (4, 4, 64, 7, 10),
    (2, 8, 64, 3, 5),
]


@pytest.mark.parametrize("param_f32", [False, True])
@pytest.mark.parametrize("Hk,Hv,D,B,slots", CASES, ids=lambda c: str(c))
def test_fused_decode_equals_separate_calls(pkg, dev, Hk, Hv, D, B, slots, param_f32):
    ops = pkg.ops
    mixed, conv_w, A_log, dt_bias, a, b, conv_pool, s_pool, ids = (
        t.to(dev) for t in _case(61, Hk, Hv, D, B, slots, param_f32))
    kd = Hk * D
    cp1, sp1 = conv_pool.clone(), s_pool.clone()
    g, beta = ops.fused_g_beta(b, a, A_log, dt_bias, None)
    y = ops.conv_decode_step(mixed, cp1, ids, conv_w)
    q, k, v = y[:, :kd].view(B, 1, Hk, D), y[:, kd:2 * kd].view(B, 1, Hk, D), y[:, 2 * kd:].view(B, 1, Hv, D)
    o1 = ops.recurrent_gdn_inplace(q, k, v, g.view(B, 1, Hv), beta.view(B, 1, Hv), sp1, ids)
    cp2, sp2 = conv_pool.clone(), s_pool.clone()
    qk = ops.conv_decode_step(mixed[:, :2 * kd], cp2[:, :2 * kd], ids, conv_w[:2 * kd])
    o2 = ops.recurrent_decode_fused(qk, mixed, cp2, conv_w, b, a, A_log, dt_bias, sp2, ids, Hk, Hv, D)
    torch.cuda.synchronize()
    assert torch.equal(o2.view(torch.int16), o1.view(torch.int16)), "outputs differ"
    assert torch.equal(sp2, sp1), "state pool differs"
    assert torch.equal(cp2.view(torch.int16), cp1.view(torch.int16)), "conv pool differs"
    untouched = [i for i in range(slots) if i not in ids.tolist()]
    assert torch.equal(sp2[untouched], s_pool[untouched])


def test_fused_decode_against_oracle(pkg, dev):
    """The fused step against the CPU oracle's decode chain directly."""
    Hk, Hv, D, B, slots = 2, 4, 128, 5, 8
    mixed, conv_w, A_log, dt_bias, a, b, conv_pool, s_pool, ids = _case(62, Hk, Hv, D, B, slots, False)
    kd = Hk * D
    g, beta = gdn_ref.g_beta(b, a, A_log, dt_bias, None)
    ry, rpool = gdn_ref.conv_decode(mixed, conv_pool.clone(), ids.tolist(), conv_w)
    q, k, v = ry[:, :kd].reshape(B, 1, Hk, D), ry[:, kd:2 * kd].reshape(B, 1, Hk, D), ry[:, 2 * kd:].reshape(B, 1, Hv, D)
    ro, rs, _ = gdn_ref.recurrent_rule(q, k, v, g.view(B, 1, Hv), beta.float().view(B, 1, Hv), s_pool[ids])
    cp, sp = conv_pool.to(dev), s_pool.to(dev)
    idd = ids.to(dev)
    qk = pkg.ops.conv_decode_step(mixed[:, :2 * kd].to(dev), cp[:, :2 * kd], idd, conv_w[:2 * kd].to(dev))
    o = pkg.ops.recurrent_decode_fused(qk, mixed.to(dev), cp, conv_w.to(dev), b.to(dev), a.to(dev), A_log.to(dev),
                                       dt_bias.to(dev), sp, idd, Hk, Hv, D)
    assert_out(o.cpu(), ro.to(BF16), "fused decode output")
    assert_state(sp.cpu()[ids], rs, "fused decode state")
    assert torch.equal(cp.cpu().view(torch.int16), rpool.view(torch.int16)), "conv pool"


@pytest.mark.parametrize("Hk,Hv,D,B,slots", CASES + [(16, 16, 128, 256, 300)], ids=lambda c: str(c))
def test_fused_decode_norm_equals_separate_norm(pkg, dev, Hk, Hv, D, B, slots):
    """With the gate rows and the norm weight the decode step also applies the
    layer's gated RMSNorm (qwen3_5.py:1083-1085): bit-equal to
    recurrent_decode_fused followed by rms_norm_gated, states and conv pool
    as without the norm.  From B * Hv >= 2048 the norm runs in the decode
    kernel itself (the last two cases), below it as a second launch."""
    ops = pkg.ops
    mixed, conv_w, A_log, dt_bias, a, b, conv_pool, s_pool, ids = (
        t.to(dev) for t in _case(63, Hk, Hv, D, B, slots, False))
    gen = torch.Generator().manual_seed(64)
    z = torch.randn(B, Hv * D, generator=gen).to(BF16)
    z[0, :D] *= 40.0                                   # gates far out on the silu tails
    z = z.to(dev)
    w = (1 + 0.02 * torch.randn(D, generator=gen)).to(BF16).to(dev)
    mixed[1, 2 * Hk * D:] *= 1e-4                      # a row with a tiny mean square
    kd = Hk * D
    cp1, sp1 = conv_pool.clone(), s_pool.clone()
    qk = ops.conv_decode_step(mixed[:, :2 * kd], cp1[:, :2 * kd], ids, conv_w[:2 * kd])
    o1 = ops.recurrent_decode_fused(qk, mixed, cp1, conv_w, b, a, A_log, dt_bias, sp1, ids, Hk, Hv, D)
    y1 = ops.rms_norm_gated(o1.view(B, Hv, D), z.view(B, Hv, D), w, 1e-6)
    cp2, sp2 = conv_pool.clone(), s_pool.clone()
    qk2 = ops.conv_decode_step(mixed[:, :2 * kd], cp2[:, :2 * kd], ids, conv_w[:2 * kd])
    y2 = ops.recurrent_decode_fused(qk2, mixed, cp2, conv_w, b, a, A_log, dt_bias, sp2, ids, Hk, Hv, D,
                                    z=z, norm_weight=w, eps=1e-6)
    torch.cuda.synchronize()
    assert torch.equal(y2.view(B, Hv, D).view(torch.int16), y1.view(torch.int16)), "fused norm differs"
    assert torch.equal(sp2, sp1), "state pool differs"
    assert torch.equal(cp2.view(torch.int16), cp1.view(torch.int16)), "conv pool differs"


def test_fused_decode_norm_epilogue_small_batch_vs_oracle(pkg, dev):
    """The in-kernel norm forced at a small batch (whole heads per workgroup
    where the plain kernel would split them): against the oracle's decode
    chain and gated norm."""
    Hk, Hv, D, B, slots = 2, 4, 128, 5, 8
    mixed, conv_w, A_log, dt_bias, a, b, conv_pool, s_pool, ids = _case(65, Hk, Hv, D, B, slots, False)
    gen = torch.Generator().manual_seed(66)
    z = torch.randn(B, Hv * D, generator=gen).to(BF16)
    w = (1 + 0.02 * torch.randn(D, generator=gen)).to(BF16)
    kd = Hk * D
    g, beta = gdn_ref.g_beta(b, a, A_log, dt_bias, None)
    ry, rpool = gdn_ref.conv_decode(mixed, conv_pool.clone(), ids.tolist(), conv_w)
    q, k, v = ry[:, :kd].reshape(B, 1, Hk, D), ry[:, kd:2 * kd].reshape(B, 1, Hk, D), ry[:, 2 * kd:].reshape(B, 1, Hv, D)
    ro, rs, _ = gdn_ref.recurrent_rule(q, k, v, g.view(B, 1, Hv), beta.float().view(B, 1, Hv), s_pool[ids])
    ref = gdn_ref.rms_norm_gated(ro.to(BF16).view(B, Hv, D), z.view(B, Hv, D), w)
    cp, sp = conv_pool.to(dev), s_pool.to(dev)
    idd = ids.to(dev)
    qk = pkg.ops.conv_decode_step(mixed[:, :2 * kd].to(dev), cp[:, :2 * kd], idd, conv_w[:2 * kd].to(dev))
    y = pkg.ops.recurrent_decode_fused(qk, mixed.to(dev), cp, conv_w.to(dev), b.to(dev), a.to(dev), A_log.to(dev),
                                       dt_bias.to(dev), sp, idd, Hk, Hv, D, z=z.to(dev), norm_weight=w.to(dev),
                                       fuse_norm=True)
    assert_out(y.cpu().view(B, Hv, D), ref, "in-kernel norm output", ulps=4)
    assert_state(sp.cpu()[ids], rs, "fused decode state")
    assert torch.equal(cp.cpu().view(torch.int16), rpool.view(torch.int16)), "conv pool"


# (B * Hv below the whole-head threshold only with the norm: the reference
# call then runs whole heads too, as the qk=None kernel always does)
@pytest.mark.parametrize("Hk,Hv,D,B,slots,with_norm",
                         [(16, 16, 128, 130, 140, False), (16, 16, 128, 130, 140, True),
                          (8, 8, 64, 260, 270, False), (8, 8, 64, 260, 270, True), (4, 4, 128, 3, 6, True)],
                         ids=lambda c: str(c))
def test_fused_decode_with_qk_conv(pkg, dev, Hk, Hv, D, B, slots, with_norm):
    """qk=None: the q/k channels' decode conv and roll run in the decode kernel
    too (one launch for the whole step).  Bit-equal to conv_decode_step on the
    q/k channels followed by the fused call with its output, in the whole-head
    form the kernel then runs; conv pools equal over all channels, other
    slots untouched."""
    ops = pkg.ops
    mixed, conv_w, A_log, dt_bias, a, b, conv_pool, s_pool, ids = (
        t.to(dev) for t in _case(63, Hk, Hv, D, B, slots, False))
    kd = Hk * D
    gen = torch.Generator().manual_seed(64)
    z = torch.randn(B, Hv * D, generator=gen).to(BF16).to(dev) if with_norm else None
    nw = (1.0 + 0.1 * torch.randn(D, generator=gen)).to(BF16).to(dev) if with_norm else None
    cp1, sp1 = conv_pool.clone(), s_pool.clone()
    qk = ops.conv_decode_step(mixed[:, :2 * kd], cp1[:, :2 * kd], ids, conv_w[:2 * kd])
    o1 = ops.recurrent_decode_fused(qk, mixed, cp1, conv_w, b, a, A_log, dt_bias, sp1, ids, Hk, Hv, D, z=z,
                                    norm_weight=nw, fuse_norm=True)
    cp2, sp2 = conv_pool.clone(), s_pool.clone()
    o2 = ops.recurrent_decode_fused(None, mixed, cp2, conv_w, b, a, A_log, dt_bias, sp2, ids, Hk, Hv, D, z=z,
                                    norm_weight=nw)
    torch.cuda.synchronize()
    assert torch.equal(o2.view(torch.int16), o1.view(torch.int16)), "outputs differ"
    assert torch.equal(sp2, sp1), "state pool differs"
    assert torch.equal(cp2.view(torch.int16), cp1.view(torch.int16)), "conv pool differs"
    untouched = [i for i in range(slots) if i not in ids.tolist()]
    assert torch.equal(cp2[untouched].view(torch.int16), conv_pool[untouched].view(torch.int16))
    assert torch.equal(sp2[untouched], s_pool[untouched])


def test_fused_decode_qk_conv_needs_one_key_head_per_value_head(pkg, dev):
    """qk=None with GVA (Hk < Hv) is refused before any launch."""
    Hk, Hv, D, B, slots = 2, 4, 64, 3, 5
    mixed, conv_w, A_log, dt_bias, a, b, conv_pool, s_pool, ids = (
        t.to(dev) for t in _case(65, Hk, Hv, D, B, slots, False))
    with pytest.raises(AssertionError):
        pkg.ops.recurrent_decode_fused(None, mixed, conv_pool, conv_w, b, a, A_log, dt_bias, s_pool, ids, Hk, Hv, D)
