"""GPU parity of the whole GDN mixer with its projections (GatedDeltaNetLayer:
in_proj GEMM over the concatenated qkv / z / b / a weights -> layer core ->
out_proj GEMM; Qwen3_5GatedDeltaNet, nanovllm/models/qwen3_5.py:864-1087 at
tp = 1) against the CPU oracle: fp32 matmuls of the same bf16 weights around
the oracle's layer core.  Config 1's head geometry (16 / 16 heads, D = 128)
with a 2048 hidden size, a varlen prefill step with a decode prefix and an
all-decode step on the same pools."""
import math

import pytest
import torch

from helpers import BF16, assert_layer_out, assert_out, assert_state, bf16_step, mean_rel
from oracle import gdn_ref

pytestmark = pytest.mark.gpu


def _weights(gen, hidden, Hk, Hv, D):
    C = 2 * Hk * D + Hv * D
    s = 1 / math.sqrt(hidden)
    w_qkv = (torch.randn(C, hidden, generator=gen) * s).to(BF16)
    w_z = (torch.randn(Hv * D, hidden, generator=gen) * s).to(BF16)
    w_b = (torch.randn(Hv, hidden, generator=gen) * s).to(BF16)
    w_a = (torch.randn(Hv, hidden, generator=gen) * s).to(BF16)
    w_out = (torch.randn(hidden, Hv * D, generator=gen) / math.sqrt(Hv * D)).to(BF16)
    conv_w = (torch.randn(C, 4, generator=gen) * 0.5).to(BF16)
    A_log = (torch.rand(Hv, generator=gen) * math.log(16)).to(BF16)
    dt_bias = (torch.rand(Hv, generator=gen) * 2 - 1).to(BF16)
    norm_w = (1 + 0.02 * torch.randn(D, generator=gen)).to(BF16)
    return C, w_qkv, w_z, w_b, w_a, w_out, conv_w, A_log, dt_bias, norm_w


def _matmul_bf16(x, w):
    return (x.float() @ w.float().t()).to(BF16)


def test_layer_with_projections(pkg, dev):
    gen = torch.Generator().manual_seed(81)
    Hk = Hv = 16
    D, hidden = 128, 2048
    C, w_qkv, w_z, w_b, w_a, w_out, conv_w, A_log, dt_bias, norm_w = _weights(gen, hidden, Hk, Hv, D)
    layer = pkg.GatedDeltaNetLayer(*(t.to(dev) for t in (w_qkv, w_z, w_b, w_a, w_out)), Hk, Hv, D,
                                   conv_w.to(dev), A_log.to(dev), dt_bias.to(dev), norm_w.to(dev))
    lens = [1, 1, 300, 129, 64, 700]                  # a decode prefix, then prefills
    N = sum(lens)
    n = len(lens)
    slots = 9
    ids = torch.tensor([7, 2, 0, 5, 8, 3])
    conv0 = torch.randn(slots, C, 3, generator=gen).to(BF16)
    s0 = torch.randn(slots, Hv, D, D, generator=gen) * 0.1
    x = torch.randn(N, hidden, generator=gen).to(BF16)
    cu = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32)
    cp, sp = conv0.to(dev), s0.to(dev)
    out = layer.forward(x.to(dev), cu.to(dev), max(lens), ids.to(dev), cp, sp, lens_q=lens)
    torch.cuda.synchronize()
    # (1) in_proj against fp32 matmuls (the GEMM's own bar: one bf16 step plus summation-order slack)
    y_in = layer.project_in(x.to(dev))[:4]
    w_all = torch.cat([w_qkv, w_z, w_b, w_a])
    ref_in = x.float() @ w_all.float().t()
    got_in = torch.cat([t.cpu() for t in y_in], 1).float()
    bound = bf16_step(ref_in) + (x.float().abs() @ w_all.float().abs().t()) * 2.0 ** -16
    assert bool(((got_in - ref_in).abs() <= bound).all()), "in_proj"
    mixed, z, b, a = (t.cpu() for t in y_in)
    # (2) the oracle's layer core on the GPU's projections: the decode prefix as two decode rows, then
    # the prefill group, on the same pools; then out_proj as an fp32 matmul
    conv_r, s_r = conv0.clone(), s0.clone()
    dec_ids = ids[:2].tolist()
    core_dec, conv_r, s_r = gdn_ref.gdn_core_decode(mixed[:2], z[:2], b[:2], a[:2], dec_ids, conv_r, s_r, conv_w,
                                                    A_log, dt_bias, norm_w, Hk, Hv, D)
    pre_ids = ids[2:]
    core_pre, new_conv, fin = gdn_ref.gdn_core_varlen(mixed[2:], z[2:], b[2:], a[2:], lens[2:], conv_r[pre_ids],
                                                      s_r[pre_ids], conv_w, A_log, dt_bias, norm_w, Hk, Hv, D)
    core_ref = torch.cat([core_dec.reshape(2, Hv * D), core_pre.reshape(N - 2, Hv * D)])
    ref = _matmul_bf16(core_ref, w_out)
    assert_out(out.cpu(), ref, "layer output (out_proj)")
    s_now = sp.cpu()
    for r, slot in enumerate(pre_ids.tolist()):
        assert_state(s_now[slot], fin[r], f"prefill state, slot {slot}")
    assert_state(s_now[dec_ids], s_r[dec_ids], "decode-prefix states")
    conv_r[pre_ids] = new_conv
    assert torch.equal(cp.cpu().view(torch.int16), conv_r.view(torch.int16)), "conv pool"
    # (3) an all-decode step through the layer on the same pools
    xd = torch.randn(n, hidden, generator=gen).to(BF16)
    cu1 = torch.arange(n + 1, dtype=torch.int32)
    out_d = layer.forward(xd.to(dev), cu1.to(dev), 1, ids.to(dev), cp, sp)
    md, zd, bd, ad = (t.cpu() for t in layer.project_in(xd.to(dev))[:4])
    core_d, _, s_d = gdn_ref.gdn_core_decode(md, zd, bd, ad, ids.tolist(), conv_r, s_now.clone(), conv_w, A_log,
                                             dt_bias, norm_w, Hk, Hv, D)
    assert_out(out_d.cpu(), _matmul_bf16(core_d.reshape(n, Hv * D), w_out), "decode step output")
    assert_state(sp.cpu()[ids], s_d[ids], "decode step states")


@pytest.mark.parametrize("sw", [{"fused_prefill": False, "fused_decode": False}, {"varlen": False, "fused_decode": False}],
                         ids=["unfused", "padded"])
def test_layer_gates_from_in_proj_epilogue(pkg, dev, sw):
    """With the fused prefill / decode switched off, the layer's paths run on
    g and beta from in_proj's GEMM epilogue instead of the gate kernel: the
    same results bit for bit as the core computing them itself from the b and
    a columns (qwen3_5.py:933-934, :978-979)."""
    gen = torch.Generator().manual_seed(82)
    Hk, Hv, D, hidden = 2, 4, 128, 512
    C, w_qkv, w_z, w_b, w_a, w_out, conv_w, A_log, dt_bias, norm_w = _weights(gen, hidden, Hk, Hv, D)
    switches = pkg.Switches(**sw)
    layer = pkg.GatedDeltaNetLayer(*(t.to(dev) for t in (w_qkv, w_z, w_b, w_a, w_out)), Hk, Hv, D,
                                   conv_w.to(dev), A_log.to(dev), dt_bias.to(dev), norm_w.to(dev), switches=switches)
    assert layer.gates_in_gemm()
    lens = [1, 1, 90, 3, 130]
    N = sum(lens)
    ids = torch.tensor([4, 1, 6, 0, 3], device=dev)
    conv0 = torch.randn(8, C, 3, generator=gen).to(BF16).to(dev)
    s0 = (torch.randn(8, Hv, D, D, generator=gen) * 0.1).to(dev)
    x = torch.randn(N, hidden, generator=gen).to(BF16).to(dev)
    cu = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32, device=dev)
    cp1, sp1 = conv0.clone(), s0.clone()
    out1 = layer.forward(x, cu, max(lens), ids, cp1, sp1, lens_q=lens)
    # the same step with the core's own gate kernel
    mixed, z, b, a, gb = layer.project_in(x)
    assert gb is None
    cp2, sp2 = conv0.clone(), s0.clone()
    core = layer.core.forward(mixed, z, b.contiguous(), a.contiguous(), cu, max(lens), ids, cp2, sp2, lens_q=lens)
    out2 = pkg.ops.linear(core, layer.w_out)
    torch.cuda.synchronize()
    assert torch.equal(out1.view(torch.int16), out2.view(torch.int16)), "outputs differ"
    assert torch.equal(sp1, sp2), "state pools differ"
    assert torch.equal(cp1.view(torch.int16), cp2.view(torch.int16)), "conv pools differ"
