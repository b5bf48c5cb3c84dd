"""The state kernels on the engine's per-layer pool views.

The runner allocates one pool for all GDN layers, s_pool [S+1, L, Hv, D, D]
fp32 and conv_pool [S+1, L, C, 3] bf16, and binds each layer to the views
s_pool[:, l] / conv_pool[:, l], whose slot strides are L*Hv*D*D and L*C*3
elements (nanovllm/engine/model_runner.py:265-303).  Every kernel that reads
or writes the pools runs here on the middle layer's views of L = 3 pools:
  * against the same kernel on dense pools holding the same slots (bit for
    bit, at the BASELINE config 1 and 2 shapes, and the segmented pass of a
    long sequence);
  * against the oracle at the same head geometry with shorter sequences;
  * every other layer and every other slot stays bit-identical.
"""
import pytest
import torch

import bench
from helpers import BF16, assert_out, assert_state
from oracle import gdn_ref

pytestmark = pytest.mark.gpu

L, LAYER = 3, 1


def _pools(pkg, gen, slots, Hv, D, C, dev):
    pools = pkg.allocate_state_pools(slots, L, Hv, D, D, C, 4, "cpu")
    pools.s_pool.copy_(torch.randn(pools.s_pool.shape, generator=gen) * 0.1)
    pools.conv_pool.copy_(torch.randn(pools.conv_pool.shape, generator=gen).to(BF16))
    host = (pools.s_pool.clone(), pools.conv_pool.clone())
    pools.s_pool = pools.s_pool.to(dev)
    pools.conv_pool = pools.conv_pool.to(dev)
    return pools, host


def _check_untouched(pools, host, ids, layer=LAYER):
    """Other layers entirely, and this layer's other slots, bit-identical."""
    s_now, c_now = pools.s_pool.cpu(), pools.conv_pool.cpu()
    s0, c0 = host
    others = [l for l in range(L) if l != layer]
    assert torch.equal(s_now[:, others], s0[:, others]), "state pool: another layer changed"
    assert torch.equal(c_now[:, others].view(torch.int16), c0[:, others].view(torch.int16)), \
        "conv pool: another layer changed"
    keep = torch.ones(s_now.shape[0], dtype=torch.bool)
    keep[torch.as_tensor(ids)] = False
    assert torch.equal(s_now[keep, layer], s0[keep, layer]), "state pool: an untouched slot changed"
    assert torch.equal(c_now[keep, layer].view(torch.int16), c0[keep, layer].view(torch.int16)), \
        "conv pool: an untouched slot changed"


def _decode_inputs(gen, B, C, Hv):
    return (torch.randn(B, C, generator=gen).to(BF16), torch.randn(B, Hv, generator=gen).to(BF16),
            torch.randn(B, Hv, generator=gen).to(BF16))


@pytest.mark.parametrize("fused", ["separate", "two_launch", "one_launch", "one_launch_norm"])
def test_decode_on_layer_views_config2(pkg, dev, fused):
    """Config 2 geometry (B = 256 of 512 slots, 16 heads, D = 128): the
    in-place decode (conv kernel + recurrent kernel), the fused decode after
    the q/k conv (fused gates / v conv / update), or the one-launch step the
    layer runs at this batch (q = k = NULL: the q/k conv and its roll in the
    same kernel, with or without the fused gated norm), on s_pool[:, l] /
    conv_pool[:, l] equals the same calls on dense copies of that layer."""
    c = bench.make_decode()
    Hk, Hv, D = c["Hk"], c["Hv"], c["D"]
    C = 2 * Hk * D + Hv * D
    gen = torch.Generator().manual_seed(61)
    slots = 512
    pools, host = _pools(pkg, gen, slots, Hv, D, C, dev)
    s_view, c_view = pools.layer(LAYER)
    assert s_view.stride(0) == L * Hv * D * D and c_view.stride(0) == L * C * 3
    s_dense = s_view.contiguous().clone()
    c_dense = c_view.contiguous().clone()
    x, a, b = (t.to(dev) for t in (c["x"], c["a"], c["b"]))
    ids = c["ids"].to(dev)
    w, A_log, dt_bias = c["conv_w"].to(dev), c["A_log"].to(dev), c["dt_bias"].to(dev)
    kd = Hk * D

    z = torch.randn(x.shape[0], Hv * D, generator=gen).to(BF16).to(dev)
    nw = (1 + 0.02 * torch.randn(D, generator=gen)).to(BF16).to(dev)
    assert x.shape[0] * Hv >= pkg.ops.WHOLE_HEAD_TILES and Hk == Hv   # the one-launch form applies

    def step(sp, cp):
        if fused == "two_launch":
            qk = pkg.ops.conv_decode_step(x[:, :2 * kd], cp[:, :2 * kd], ids, w[:2 * kd])
            return pkg.ops.recurrent_decode_fused(qk, x, cp, w, b, a, A_log, dt_bias, sp, ids, Hk, Hv, D)
        if fused == "one_launch":
            return pkg.ops.recurrent_decode_fused(None, x, cp, w, b, a, A_log, dt_bias, sp, ids, Hk, Hv, D)
        if fused == "one_launch_norm":
            return pkg.ops.recurrent_decode_fused(None, x, cp, w, b, a, A_log, dt_bias, sp, ids, Hk, Hv, D, z=z,
                                                  norm_weight=nw, eps=1e-6)
        g, beta = pkg.ops.fused_g_beta(b, a, A_log, dt_bias, None)
        y = pkg.ops.conv_decode_step(x, cp, ids, w)
        q = y[:, :kd].view(-1, 1, Hk, D)
        k = y[:, kd:2 * kd].view(-1, 1, Hk, D)
        v = y[:, 2 * kd:].view(-1, 1, Hv, D)
        return pkg.ops.recurrent_gdn_inplace(q, k, v, g.view(-1, 1, Hv), beta.view(-1, 1, Hv), sp, ids)

    o_view = step(s_view, c_view)
    o_dense = step(s_dense, c_dense)
    torch.cuda.synchronize()
    assert torch.equal(o_view.cpu().view(torch.int16), o_dense.cpu().view(torch.int16)), "output: view vs dense"
    assert torch.equal(s_view.cpu(), s_dense.cpu()), "state: view vs dense"
    assert torch.equal(c_view.cpu().view(torch.int16), c_dense.cpu().view(torch.int16)), "conv state: view vs dense"
    _check_untouched(pools, host, c["ids"])
    # oracle on the touched slots
    idl = c["ids"].tolist()
    ref, ref_conv, ref_s = gdn_ref.gdn_core_decode(
        c["x"], torch.zeros(len(idl), Hv * D, dtype=BF16), c["b"], c["a"], idl, host[1][:, LAYER].clone(),
        host[0][:, LAYER].clone(), c["conv_w"], c["A_log"], c["dt_bias"], torch.ones(D, dtype=BF16), Hk, Hv, D)
    s_now = pools.s_pool.cpu()[:, LAYER]
    assert_state(s_now[idl], ref_s[idl], "decoded slots vs oracle")
    assert torch.equal(pools.conv_pool.cpu()[:, LAYER].view(torch.int16), ref_conv.view(torch.int16))


def _prefill_case(gen, lens, Hk, Hv, D):
    N = sum(lens)
    C = 2 * Hk * D + Hv * D
    x = torch.randn(N, C, generator=gen).to(BF16)
    a = torch.randn(N, Hv, generator=gen).to(BF16)
    b = torch.randn(N, Hv, generator=gen).to(BF16)
    return N, C, x, a, b


@pytest.mark.parametrize("lens,slots,ids,segments", [
    ("config1", 16, [9, 2, 14, 0, 7, 11, 5, 12], 0),   # BASELINE config 1 lengths (seed 1), 16 heads
    ([4096], 4, [2], 6),                                 # one long sequence, segmented state pass
])
def test_prefill_on_layer_views_bitwise(pkg, dev, lens, slots, ids, segments):
    """The pool-form chunk rule and the fused prefill on the layer views
    equal the same calls on dense copies of the layer, bit for bit."""
    gen = torch.Generator().manual_seed(62)
    if lens == "config1":
        lens = bench.make_prefill(1, None)["lens"]
    Hk = Hv = 16
    D = 128
    N, C, x, a, b = _prefill_case(gen, lens, Hk, Hv, D)
    cfg = bench.make_prefill(1, [64])          # layer parameters of config 1's distributions
    w, A_log, dt_bias = cfg["conv_w"].to(dev), cfg["A_log"].to(dev), cfg["dt_bias"].to(dev)
    pools, host = _pools(pkg, gen, slots, Hv, D, C, dev)
    s_view, c_view = pools.layer(LAYER)
    s_dense, c_dense = s_view.contiguous().clone(), c_view.contiguous().clone()
    ids_d = torch.tensor(ids, device=dev)
    cu = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int64)
    cu_d = cu.to(dev)
    xd, ad, bd = x.to(dev), a.to(dev), b.to(dev)
    fresh = torch.tensor([r % 3 == 0 for r in range(len(lens))], device=dev)

    def fused(sp, cp):
        return pkg.ops.conv_chunk_prefill_varlen(xd, cp, w, bd, ad, A_log, dt_bias, cu_d, sp, ids_d, Hk, Hv, D,
                                                 fresh=fresh, cu_seqlens_cpu=cu, max_segments=segments)

    o_v = fused(s_view, c_view)
    o_d = fused(s_dense, c_dense)
    torch.cuda.synchronize()
    assert torch.equal(o_v.cpu().view(torch.int16), o_d.cpu().view(torch.int16)), "fused output: view vs dense"
    assert torch.equal(s_view.cpu(), s_dense.cpu()), "fused final states: view vs dense"
    assert torch.equal(c_view.cpu().view(torch.int16), c_dense.cpu().view(torch.int16)), "fused conv roll"
    _check_untouched(pools, host, ids)
    # the pool-form chunk rule alone (post-conv inputs), on the views
    q = torch.randn(N, Hk, D, generator=gen).to(BF16).to(dev)
    k = torch.randn(N, Hk, D, generator=gen).to(BF16).to(dev)
    v = torch.randn(N, Hv, D, generator=gen).to(BF16).to(dev)
    g, beta = pkg.ops.fused_g_beta(bd, ad, A_log, dt_bias, None)

    def chunk(sp):
        return pkg.ops.chunk_gated_delta_rule_varlen(q, k, v, g, beta, cu_d, sp, state_ids=ids_d, final_state=sp,
                                                     cu_seqlens_cpu=cu, max_segments=segments)[0]

    o_v = chunk(s_view)
    o_d = chunk(s_dense)
    torch.cuda.synchronize()
    assert torch.equal(o_v.cpu().view(torch.int16), o_d.cpu().view(torch.int16)), "chunk output: view vs dense"
    assert torch.equal(s_view.cpu(), s_dense.cpu()), "chunk final states: view vs dense"
    _check_untouched(pools, host, ids)


def test_prefill_on_layer_views_vs_oracle(pkg, dev):
    """Config 1 head geometry (16 / 16 heads, D = 128, 8 sequences, some
    fresh) with shorter sequences: the fused prefill on the layer views
    against the oracle, other layers and slots untouched."""
    gen = torch.Generator().manual_seed(63)
    lens = [300, 1, 64, 129, 0, 257, 90, 3]
    Hk = Hv = 16
    D = 128
    N, C, x, a, b = _prefill_case(gen, lens, Hk, Hv, D)
    cfg = bench.make_prefill(1, [64])
    pools, host = _pools(pkg, gen, 12, Hv, D, C, dev)
    s_view, c_view = pools.layer(LAYER)
    ids = [11, 3, 0, 7, 5, 9, 1, 4]
    fresh = [False, True, False, False, True, False, True, False]
    cu = [0]
    for t in lens:
        cu.append(cu[-1] + t)
    o = pkg.ops.conv_chunk_prefill_varlen(x.to(dev), c_view, cfg["conv_w"].to(dev), b.to(dev), a.to(dev),
                                          cfg["A_log"].to(dev), cfg["dt_bias"].to(dev),
                                          torch.tensor(cu, device=dev), s_view, torch.tensor(ids, device=dev),
                                          Hk, Hv, D, fresh=torch.tensor(fresh, device=dev),
                                          cu_seqlens_cpu=torch.tensor(cu))
    torch.cuda.synchronize()
    conv0 = host[1][ids, LAYER].clone()
    h0 = host[0][ids, LAYER].clone()
    for r, fr in enumerate(fresh):
        if fr:
            conv0[r].zero_()
            h0[r].zero_()
    g, beta = gdn_ref.g_beta(b, a, cfg["A_log"], cfg["dt_bias"])
    y, new_conv = gdn_ref.conv_varlen(x, conv0, cfg["conv_w"], lens)
    kd = Hk * D
    ro, rS = gdn_ref.chunk_varlen(y[:, :kd].reshape(N, Hk, D), y[:, kd:2 * kd].reshape(N, Hk, D),
                                  y[:, 2 * kd:].reshape(N, Hv, D), g, beta.float(), cu, h0)
    assert_out(o.cpu(), ro.to(BF16), "fused prefill on layer views")
    s_now = pools.s_pool.cpu()[:, LAYER]
    for r, slot in enumerate(ids):
        assert_state(s_now[slot], rS[r], f"final state of sequence {r} (slot {slot})")
    assert torch.equal(pools.conv_pool.cpu()[ids, LAYER].view(torch.int16), new_conv.view(torch.int16))
    _check_untouched(pools, host, ids)
