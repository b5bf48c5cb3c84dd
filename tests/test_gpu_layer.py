"""GPU parity of the GDN layer core (GatedDeltaNetCore) and of the BASELINE
configs at full size, against the CPU oracle; plus the reference's stress
invariants restated at kernel level (nanovllm tests/stress_qwen35.py:63-78):
graph == eager, chunked prefill == one-shot, batched == solo, and
prefill-then-decode == a longer prefill."""
import pytest
import torch

import bench
from helpers import (BF16, OUT_MEAN_REL, STATE_REL, assert_layer_out, assert_layer_out_propagated, assert_out,
                     assert_state, mean_rel, state_rel)
from oracle import gdn_ref

pytestmark = pytest.mark.gpu


def _layer(gen, Hk, Hv, D):
    import math
    C = 2 * Hk * D + Hv * D
    conv_w = (torch.randn(C, 4, generator=gen) * 0.5).to(BF16)
    A_log = (torch.rand(Hv, generator=gen) * math.log(16)).to(BF16)
    dt_bias = (torch.rand(Hv, generator=gen) * 2 - 1).to(BF16)
    norm_w = (1 + 0.02 * torch.randn(D, generator=gen)).to(BF16)
    return C, conv_w, A_log, dt_bias, norm_w


def _rows(gen, N, C, Hv, D):
    return (torch.randn(N, C, generator=gen).to(BF16), torch.randn(N, Hv * D, generator=gen).to(BF16),
            torch.randn(N, Hv, generator=gen).to(BF16), torch.randn(N, Hv, generator=gen).to(BF16))


def _core(pkg, dev, Hk, Hv, D, conv_w, A_log, dt_bias, norm_w, **sw):
    switches = pkg.Switches(**sw) if sw else pkg.Switches()
    return pkg.GatedDeltaNetCore(Hk, Hv, D, conv_w.to(dev), A_log.to(dev), dt_bias.to(dev), norm_w.to(dev),
                                 switches=switches)


SWITCH_SETS = [
    {},
    {"gbeta": False},
    {"conv_kernel": False},
    {"inplace": False},
    {"varlen": False},
    {"fused_prefill": False},
    {"fused_decode": False},
]


@pytest.mark.parametrize("sw", SWITCH_SETS, ids=lambda s: ",".join(f"{k}={v}" for k, v in s.items()) or "default")
@pytest.mark.parametrize("Hk,Hv", [(4, 4), (2, 4)])
def test_layer_forward_mixed_batch(pkg, dev, sw, Hk, Hv):
    """Decode prefix (lens == 1) + varlen prefill rows in one step, pools indexed by slot."""
    gen = torch.Generator().manual_seed(31)
    D = 128
    C, conv_w, A_log, dt_bias, norm_w = _layer(gen, Hk, Hv, D)
    lens = [1, 1, 1, 70, 3, 200, 64]
    N = sum(lens)
    mixed, z, b, a = _rows(gen, N, C, Hv, D)
    slots = 12
    conv_pool = torch.randn(slots, C, 3, generator=gen).to(BF16)
    s_pool = torch.randn(slots, Hv, D, D, generator=gen) * 0.1
    ids = torch.tensor([9, 2, 7, 0, 5, 11, 3])
    # oracle: decode rows, then the varlen prefill group, each on its slots
    ref_conv, ref_s = conv_pool.clone(), s_pool.clone()
    eager = sw.get("conv_kernel") is False        # eager F.conv1d chain: bf16 rounding before SiLU
    core_d, ref_conv, ref_s = gdn_ref.gdn_core_decode(mixed[:3], z[:3], b[:3], a[:3], ids[:3].tolist(), ref_conv,
                                                      ref_s, conv_w, A_log, dt_bias, norm_w, Hk, Hv, D,
                                                      conv_eager=eager)
    pids = ids[3:]
    core_p, new_conv, new_s = gdn_ref.gdn_core_varlen(mixed[3:], z[3:], b[3:], a[3:], lens[3:], ref_conv[pids],
                                                      ref_s[pids], conv_w, A_log, dt_bias, norm_w, Hk, Hv, D,
                                                      conv_eager=eager)
    ref_conv[pids], ref_s[pids] = new_conv, new_s
    ref = torch.cat([core_d.reshape(3, -1), core_p.reshape(N - 3, -1)])

    core = _core(pkg, dev, Hk, Hv, D, conv_w, A_log, dt_bias, norm_w, **sw)
    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0).tolist()), dtype=torch.int32, device=dev)
    cp, sp = conv_pool.to(dev), s_pool.to(dev)
    out = core.forward(mixed.to(dev), z.to(dev), b.to(dev), a.to(dev), cu, max(lens), ids.to(dev), cp, sp,
                       lens_q=lens)
    assert out.shape == (N, Hv * D)
    assert_out(out.cpu(), ref, "layer forward", ulps=4)
    assert torch.equal(cp.cpu(), ref_conv), "conv pool bookkeeping"
    assert_state(sp.cpu(), ref_s, "state pool")
    untouched = [i for i in range(slots) if i not in ids.tolist()]
    assert torch.equal(sp.cpu()[untouched], s_pool[untouched])


def test_decode_graph_replay_equals_eager(pkg, dev):
    """The decode step captured in a HIP graph and replayed, with eager work
    in between, matches the eager step bit for bit on every replay."""
    gen = torch.Generator().manual_seed(32)
    Hk = Hv = 16
    D, B, slots = 128, 48, 64
    C, conv_w, A_log, dt_bias, norm_w = _layer(gen, Hk, Hv, D)
    mixed, z, b, a = (t.to(dev) for t in _rows(gen, B, C, Hv, D))
    ids = torch.full((B,), slots - 1, dtype=torch.int64)         # pad rows -> dummy slot
    ids[:-8] = torch.randperm(slots - 1, generator=gen)[:B - 8]  # real rows: distinct live slots
    ids = ids.to(dev)
    conv0 = torch.randn(slots, C, 3, generator=gen).to(BF16).to(dev)
    s0 = (torch.randn(slots, Hv, D, D, generator=gen) * 0.1).to(dev)
    core = _core(pkg, dev, Hk, Hv, D, conv_w, A_log, dt_bias, norm_w)
    cg, sg = conv0.clone(), s0.clone()
    ce, se = conv0.clone(), s0.clone()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        core.decode(mixed, z, b, a, ids, cg, sg)                  # warm-up (also on the eager copy)
    torch.cuda.current_stream().wait_stream(stream)
    core.decode(mixed, z, b, a, ids, ce, se)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        out_g = core.decode(mixed, z, b, a, ids, cg, sg)
    real = ids[:-8]
    for rep in range(3):
        graph.replay()
        torch.cuda.synchronize()
        out_e = core.decode(mixed, z, b, a, ids, ce, se)
        _ = (mixed.float() * 2).sum()                            # unrelated eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(out_g[:-8], out_e[:-8]), f"replay {rep}: outputs differ"
        assert torch.equal(sg[real], se[real]), f"replay {rep}: state pool differs"
        assert torch.equal(cg[real], ce[real]), f"replay {rep}: conv pool differs"


def test_decode_graph_one_launch_with_pad_rows_equals_eager(pkg, dev):
    """The decode step config 2 runs (Hk == Hv = 16, whole heads per
    workgroup: q/k/v conv and roll, gates, update and gated norm in one
    kernel), captured in a HIP graph the way the runner captures it
    (nanovllm/engine/model_runner.py:1584-1611): static input buffers of the
    graph's batch size, the real rows copied in before each replay and the
    pad rows pointed at the dummy slot (:289-299, :824-826), several of
    whose workgroups then write that slot's states and conv taps in one
    launch.  Three replays with new inputs and eager work in between: the
    real rows' outputs, states and conv taps equal the eager step on the
    unpadded batch bit for bit, and every slot but the dummy one is equal."""
    gen = torch.Generator().manual_seed(37)
    Hk = Hv = 16
    D, B, pad, slots = 128, 256, 16, 512
    Bg, dummy = B + pad, slots
    assert Bg * Hv >= pkg.ops.WHOLE_HEAD_TILES
    C, conv_w, A_log, dt_bias, norm_w = _layer(gen, Hk, Hv, D)
    conv0 = torch.randn(slots + 1, C, 3, generator=gen).to(BF16).to(dev)
    s0 = (torch.randn(slots + 1, Hv, D, D, generator=gen) * 0.1).to(dev)
    real = torch.randperm(slots, generator=gen)[:B].to(dev)
    core = _core(pkg, dev, Hk, Hv, D, conv_w, A_log, dt_bias, norm_w)
    cg, sg = conv0.clone(), s0.clone()
    ce, se = conv0.clone(), s0.clone()
    # the graph's static inputs; pad rows hold stale data and the dummy slot
    st_mixed, st_z, st_b, st_a = (t.to(dev) for t in _rows(gen, Bg, C, Hv, D))
    st_ids = torch.full((Bg,), dummy, dtype=torch.int64, device=dev)
    st_ids[:B] = real
    warm_c, warm_s = conv0.clone(), s0.clone()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        core.decode(st_mixed, st_z, st_b, st_a, st_ids, warm_c, warm_s)   # warm-up on a throwaway copy
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    del warm_c, warm_s
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        out_g = core.decode(st_mixed, st_z, st_b, st_a, st_ids, cg, sg)
    for rep in range(3):
        mixed, z, b, a = (t.to(dev) for t in _rows(gen, B, C, Hv, D))
        st_mixed[:B].copy_(mixed)
        st_z[:B].copy_(z)
        st_b[:B].copy_(b)
        st_a[:B].copy_(a)
        graph.replay()
        torch.cuda.synchronize()
        out_e = core.decode(mixed, z, b, a, real, ce, se)
        _ = (mixed.float() * 2).sum()                            # unrelated eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(out_g[:B].view(torch.int16), out_e.view(torch.int16)), f"replay {rep}: outputs differ"
        assert torch.equal(sg[:slots], se[:slots]), f"replay {rep}: state pool differs"
        assert torch.equal(cg[:slots].view(torch.int16), ce[:slots].view(torch.int16)), \
            f"replay {rep}: conv pool differs"
    assert not torch.equal(sg[real], s0[real]), "the replays updated the real rows' states"


def test_chunked_prefill_equals_one_shot_and_batched_equals_solo(pkg, dev):
    gen = torch.Generator().manual_seed(33)
    Hk = Hv = 4
    D = 128
    C, conv_w, A_log, dt_bias, norm_w = _layer(gen, Hk, Hv, D)
    lens = [300, 77, 129]
    N = sum(lens)
    mixed, z, b, a = (t.to(dev) for t in _rows(gen, N, C, Hv, D))
    core = _core(pkg, dev, Hk, Hv, D, conv_w, A_log, dt_bias, norm_w)
    slots = 4
    ids = torch.tensor([2, 0, 3], device=dev)
    # one shot, batched
    cp1 = torch.zeros(slots, C, 3, dtype=BF16, device=dev)
    sp1 = torch.zeros(slots, Hv, D, D, device=dev)
    out1 = core.prefill_varlen(mixed, z, b, a, lens, ids, cp1, sp1)
    # solo, each sequence alone
    cp2, sp2 = torch.zeros_like(cp1), torch.zeros_like(sp1)
    outs, off = [], 0
    for r, T in enumerate(lens):
        outs.append(core.prefill_varlen(mixed[off:off + T], z[off:off + T], b[off:off + T], a[off:off + T], [T],
                                        ids[r:r + 1], cp2, sp2))
        off += T
    assert torch.equal(torch.cat(outs), out1) and torch.equal(cp1, cp2) and torch.equal(sp1, sp2)
    # chunked: the first sequence prefilled in two calls (split inside a chunk)
    cp3, sp3 = torch.zeros_like(cp1), torch.zeros_like(sp1)
    o_a = core.prefill_varlen(mixed[:100], z[:100], b[:100], a[:100], [100], ids[:1], cp3, sp3)
    o_b = core.prefill_varlen(mixed[100:300], z[100:300], b[100:300], a[100:300], [200], ids[:1], cp3, sp3)
    assert_out(torch.cat([o_a, o_b]).cpu(), out1[:300].cpu(), "chunked == one-shot", ulps=4)
    assert torch.equal(cp3[2], cp1[2])
    # both sides carry the chunk kernel's fp16-operand error (~2e-4 each)
    assert state_rel(sp3[2].cpu(), sp1[2].cpu()) < STATE_REL


def test_prefill_then_decode_equals_longer_prefill(pkg, dev):
    gen = torch.Generator().manual_seed(34)
    Hk = Hv = 4
    D = 128
    C, conv_w, A_log, dt_bias, norm_w = _layer(gen, Hk, Hv, D)
    T = 150
    mixed, z, b, a = (t.to(dev) for t in _rows(gen, T + 1, C, Hv, D))
    core = _core(pkg, dev, Hk, Hv, D, conv_w, A_log, dt_bias, norm_w)
    ids = torch.tensor([1], device=dev)
    cp = torch.zeros(2, C, 3, dtype=BF16, device=dev)
    sp = torch.zeros(2, Hv, D, D, device=dev)
    core.prefill_varlen(mixed[:T], z[:T], b[:T], a[:T], [T], ids, cp, sp)
    o_dec = core.decode(mixed[T:], z[T:], b[T:], a[T:], ids, cp, sp)
    cp2, sp2 = torch.zeros_like(cp), torch.zeros_like(sp)
    o_all = core.prefill_varlen(mixed, z, b, a, [T + 1], ids, cp2, sp2)
    assert_out(o_dec.cpu(), o_all[T:].cpu(), "decode after prefill", ulps=4)
    assert torch.equal(cp, cp2)
    # both sides carry the chunk kernel's fp16-operand error (~2e-4 each)
    assert state_rel(sp[1].cpu(), sp2[1].cpu()) < STATE_REL


# --------------------------------------------------------- BASELINE configs --
def _prefill_config(pkg, dev, cfg):
    """Layer prefill at a BASELINE config, checked in stages:
    (1) the conv outputs against the oracle's, each within one bf16 ulp and
    flips rare;
    (2) the fused prefill call's core output (before the norm) against the
    oracle run on the GPU's own conv outputs, to the kernel bar, plus the
    final states; the GPU's gated norm on that core output against the
    oracle's norm on the same input (bit-identical but for rare flips);
    (3) the layer output against the oracle on the GPU's conv outputs, and
    (4) end to end against the pure oracle: the core output to the kernel
    bar, and the layer output to the layer bar (assert_layer_out: the
    per-element bound everywhere but for at most 1e-6 of the elements, which
    may be rounding cascades of up to four steps through the norm, each
    printed) widened in (4) by the norm's first-order propagation of the two
    core outputs' difference (helpers.norm_propagation_bound: rows whose mean
    square is near or below eps scale a conv-output flip upstream by up to
    1/sqrt(eps)), with no row left out."""
    Hk, Hv, D = cfg["Hk"], cfg["Hv"], cfg["D"]
    core = _core(pkg, dev, Hk, Hv, D, cfg["conv_w"], cfg["A_log"], cfg["dt_bias"], cfg["norm_w"])
    n = len(cfg["lens"])
    N = sum(cfg["lens"])
    cp, sp = cfg["conv_state"].to(dev), cfg["h0"].to(dev)
    out = core.prefill_varlen(cfg["x"].to(dev), cfg["z"].to(dev), cfg["b"].to(dev), cfg["a"].to(dev), cfg["lens"],
                              torch.arange(n, device=dev), cp, sp)
    # the same conv through the standalone kernel (bit-equal to the fused
    # path's conv, test_gpu_fused_prefill)
    lens32 = torch.tensor(cfg["lens"], dtype=torch.int32, device=dev)
    starts = torch.tensor(([0] + torch.tensor(cfg["lens"]).cumsum(0).tolist())[:-1], dtype=torch.int32, device=dev)
    q, k, v = pkg.ops.causal_conv_silu_varlen_parts(cfg["x"].to(dev), cfg["conv_state"].to(dev), cfg["conv_w"].to(dev),
                                                    lens32, starts, Hk * D)
    y_gpu = torch.cat([q, k, v], 1).cpu()
    torch.cuda.synchronize()
    torch.set_num_threads(min(16, torch.get_num_threads()))
    # (1) conv
    y_ref, ref_conv = gdn_ref.conv_varlen(cfg["x"], cfg["conv_state"], cfg["conv_w"], cfg["lens"])
    ulp_diff = (y_gpu.view(torch.int16).int() - y_ref.view(torch.int16).int()).abs()
    assert int(ulp_diff.max()) <= 1, "conv output more than one bf16 ulp from the oracle"
    assert float((ulp_diff > 0).float().mean()) < 1e-4, "conv rounding flips not rare"
    assert torch.equal(cp.cpu(), ref_conv), "conv state"
    # the oracle's gates, chunk rule and norm on the GPU's conv outputs
    g, beta = gdn_ref.g_beta(cfg["b"], cfg["a"], cfg["A_log"], cfg["dt_bias"])
    kd = Hk * D
    cu = [0]
    for t in cfg["lens"]:
        cu.append(cu[-1] + t)
    o_ref, ref_s = gdn_ref.chunk_varlen(y_gpu[:, :kd].reshape(N, Hk, D), y_gpu[:, kd:2 * kd].reshape(N, Hk, D),
                                        y_gpu[:, 2 * kd:].reshape(N, Hv, D), g, beta.float(), cu, cfg["h0"])
    ref = gdn_ref.rms_norm_gated(o_ref.to(BF16), cfg["z"].reshape(N, Hv, D), cfg["norm_w"])
    # (2) the core output of the fused call (fresh copies of the input pools)
    cp2, sp2 = cfg["conv_state"].to(dev), cfg["h0"].to(dev)
    o_gpu = pkg.ops.conv_chunk_prefill_varlen(cfg["x"].to(dev), cp2, cfg["conv_w"].to(dev), cfg["b"].to(dev),
                                              cfg["a"].to(dev), cfg["A_log"].to(dev), cfg["dt_bias"].to(dev),
                                              torch.tensor(cu, device=dev), sp2, None, Hk, Hv, D,
                                              cu_seqlens_cpu=torch.tensor(cu))
    zz = cfg["z"].reshape(N, Hv, D)
    y_gpu_norm = pkg.ops.rms_norm_gated(o_gpu, zz.to(dev), cfg["norm_w"].to(dev), 1e-6).cpu()
    o_gpu = o_gpu.cpu()
    assert_out(o_gpu, o_ref.to(BF16), "core output")
    for r in range(n):
        assert_state(sp[r].cpu(), ref_s[r], f"final state of sequence {r}")
    assert torch.equal(sp2.cpu(), sp.cpu()), "fused call == layer call (states)"
    y_orc_norm = gdn_ref.rms_norm_gated(o_gpu, zz, cfg["norm_w"])
    assert_layer_out(y_gpu_norm, y_orc_norm, "gated norm on the GPU's core output",
                     ms_rows=o_gpu.float().pow(2).mean(-1))
    flips = (y_gpu_norm.view(torch.int16) != y_orc_norm.view(torch.int16)).float().mean().item()
    assert flips < 1e-3, f"gated norm: {flips:.2e} of elements differ in bits"
    assert torch.equal(out.cpu().view(torch.int16), y_gpu_norm.view(torch.int16)), "layer == fused call + norm"
    # (3) the layer output against the oracle on the GPU's conv outputs
    ms = o_ref.to(BF16).float().pow(2).mean(-1)
    assert_layer_out(out.cpu(), ref, "prefill output", ms_rows=ms)
    # (4) end to end against the pure oracle
    o_e2e, _ = gdn_ref.chunk_varlen(y_ref[:, :kd].reshape(N, Hk, D), y_ref[:, kd:2 * kd].reshape(N, Hk, D),
                                    y_ref[:, 2 * kd:].reshape(N, Hv, D), g, beta.float(), cu, cfg["h0"])
    o_e2e = o_e2e.to(BF16)
    assert_out(o_gpu, o_e2e, "end-to-end core output")
    ref_e2e = gdn_ref.rms_norm_gated(o_e2e, cfg["z"].reshape(N, Hv, D), cfg["norm_w"])
    assert_layer_out_propagated(out.cpu(), ref_e2e, o_gpu, o_e2e, cfg["z"].reshape(N, Hv, D), cfg["norm_w"],
                                "end-to-end prefill output")


def test_config1_varlen_prefill_full(pkg, dev):
    print("config 1: 8 seqs ~U[128,4096] seed 1", flush=True)
    _prefill_config(pkg, dev, bench.make_prefill(1, None))


def test_config3_long_prefill_full(pkg, dev):
    print("config 3: 1 x 65536 tokens, h0 ~ N(0, 0.1^2), conv prefix", flush=True)
    _prefill_config(pkg, dev, bench.make_prefill(4, [65536], h0_std=0.1, conv_std=1.0))


def test_config2_decode_full(pkg, dev):
    print("config 2: B=256 over 512 slots", flush=True)
    c = bench.make_decode()
    core = _core(pkg, dev, c["Hk"], c["Hv"], c["D"], c["conv_w"], c["A_log"], c["dt_bias"], c["norm_w"])
    cp, sp = c["conv_pool"].to(dev), c["s_pool"].to(dev)
    out = core.decode(c["x"].to(dev), c["z"].to(dev), c["b"].to(dev), c["a"].to(dev), c["ids"].to(dev), cp, sp)
    torch.cuda.synchronize()
    ref, ref_conv, ref_s = gdn_ref.gdn_core_decode(c["x"], c["z"], c["b"], c["a"], c["ids"].tolist(),
                                                   c["conv_pool"], c["s_pool"], c["conv_w"], c["A_log"],
                                                   c["dt_bias"], c["norm_w"], c["Hk"], c["Hv"], c["D"])
    assert_out(out.cpu(), ref, "decode output", ulps=4)
    assert torch.equal(cp.cpu().view(torch.int16), ref_conv.view(torch.int16)), "conv pool roll"
    spc = sp.cpu()
    ids = c["ids"]
    assert_state(spc[ids], ref_s[ids], "decoded slots")
    untouched = torch.ones(spc.shape[0], dtype=torch.bool)
    untouched[ids] = False
    assert torch.equal(spc[untouched], c["s_pool"][untouched]), "untouched slots must be bit-identical"


def test_config4_spec_verify_full(pkg, dev):
    print("config 4: 64 seqs x 4 draft tokens, Hk=16 Hv=32", flush=True)
    c = bench.make_spec()
    B, T, Hv, D = c["B"], c["T"], c["Hv"], c["D"]
    g, beta = gdn_ref.g_beta(c["b"], c["a"], c["A_log"], c["dt_bias"])
    pool = c["s_pool"].to(dev)
    inter = torch.empty(B, T, Hv, D, D, device=dev)
    o = pkg.ops.recurrent_gdn_multitoken(c["q"].to(dev), c["k"].to(dev), c["v"].to(dev), g.to(dev), beta.to(dev),
                                         pool, c["ids"].to(dev), intermediate_states=inter)
    pkg.ops.commit_states(pool, c["ids"].to(dev), inter, c["accepted"].to(dev))
    torch.cuda.synchronize()
    ids = c["ids"]
    ro, _, rstates = gdn_ref.recurrent_rule(c["q"], c["k"], c["v"], g, beta.float(), c["s_pool"][ids],
                                            keep_states=True)
    assert_out(o.cpu(), ro.to(BF16), "spec-verify outputs")
    interc = inter.cpu()
    for t in range(T):
        assert_state(interc[:, t], rstates[:, t], f"intermediate state {t}")
    poolc = pool.cpu()
    for i in range(B):
        acc = int(c["accepted"][i])
        assert torch.equal(poolc[ids[i]], interc[i, acc - 1]), "rollback restores the accepted prefix state"


def test_installed_prefill_method_equals_layer_core(pkg, dev):
    """integration.install's fused _gdn_prefill_varlen on a stand-in layer with
    the reference's attribute names gives the layer core's prefill bit for bit
    and updates the same pools."""
    import types

    gen = torch.Generator().manual_seed(35)
    Hk, Hv, D = 2, 4, 128
    C, conv_w, A_log, dt_bias, norm_w = _layer(gen, Hk, Hv, D)
    lens = [70, 3, 130]
    N = sum(lens)
    mixed, z, b, a = (t.to(dev) for t in _rows(gen, N, C, Hv, D))
    slots = 6
    conv0 = torch.randn(slots, C, 3, generator=gen).to(BF16).to(dev)
    s0 = (torch.randn(slots, Hv, D, D, generator=gen) * 0.1).to(dev)
    ids = torch.tensor([4, 0, 2], device=dev)

    core = _core(pkg, dev, Hk, Hv, D, conv_w, A_log, dt_bias, norm_w)
    cp1, sp1 = conv0.clone(), s0.clone()
    ref = core.prefill_varlen(mixed, z, b, a, lens, ids, cp1, sp1).reshape(N, Hv * D)

    mod = types.ModuleType("qwen3_5_stub")

    def _varlen_meta(lens_q):
        cu = torch.tensor([0] + torch.tensor(lens_q).cumsum(0).tolist(), dtype=torch.int64, device=dev)
        return cu.int(), torch.tensor(lens_q, dtype=torch.int32, device=dev), cu.cpu(), cu

    class Qwen3_5GatedDeltaNet:
        def _gdn_prefill_varlen(self, hidden, lens_q, ids):
            raise AssertionError("the original method must not run")

    mod._varlen_meta = _varlen_meta
    mod.Qwen3_5GatedDeltaNet = Qwen3_5GatedDeltaNet
    prev = pkg.integration.install(mod)
    try:
        layer = Qwen3_5GatedDeltaNet()
        layer.num_k_heads, layer.num_v_heads, layer.head_k_dim, layer.head_v_dim = Hk, Hv, D, D
        layer.value_dim, layer.conv_dim, layer.conv_kernel = Hv * D, C, 4
        layer.in_proj_b, layer.in_proj_a = (lambda h: b), (lambda h: a)
        layer.in_proj_z, layer.in_proj_qkv = (lambda h: z), (lambda h: mixed)
        layer.A_log, layer.dt_bias, layer._v_head_slice = A_log.to(dev), dt_bias.to(dev), slice(0, Hv)
        layer.conv1d = types.SimpleNamespace(weight=conv_w.to(dev).view(C, 1, 4))
        norm = pkg.ops.Qwen3_5RMSNormGated(D)
        norm.weight.data = norm_w.to(dev)
        layer.norm = norm
        layer.out_proj = lambda x: x
        layer.conv_cache, layer.s_cache = conv0.clone(), s0.clone()
        out = layer._gdn_prefill_varlen(None, lens, ids)
    finally:
        pkg.integration.uninstall(mod, prev)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    assert torch.equal(layer.s_cache, sp1)
    assert torch.equal(layer.conv_cache.view(torch.int16), cp1.view(torch.int16))


@pytest.mark.parametrize("Hk,Hv,B,slots", [(2, 4, 5, 8), (16, 16, 136, 160)],
                         ids=["gva-two-launch", "one-launch"])
def test_installed_decode_method_equals_layer_core(pkg, dev, Hk, Hv, B, slots):
    """integration.install's fused _gdn_padded (T == 1) on a stand-in layer
    with the reference's attribute names gives the layer core's decode (with
    the fused decode switched off: fused_g_beta -> conv_decode_step ->
    recurrent_gdn_inplace) bit for bit, and updates the same pools.  Both of
    the installed method's branches: GVA (the q/k conv as its own launch) and
    one key head per value head with B * Hv >= WHOLE_HEAD_TILES (the whole
    step, gated norm included, in one kernel)."""
    import types

    gen = torch.Generator().manual_seed(36)
    D = 128
    C, conv_w, A_log, dt_bias, norm_w = _layer(gen, Hk, Hv, D)
    assert (Hk == Hv and B * Hv >= pkg.ops.WHOLE_HEAD_TILES) == (Hk == 16)
    mixed, z, b, a = (t.to(dev) for t in _rows(gen, B, C, Hv, D))
    conv0 = torch.randn(slots, C, 3, generator=gen).to(BF16).to(dev)
    s0 = (torch.randn(slots, Hv, D, D, generator=gen) * 0.1).to(dev)
    ids = torch.randperm(slots, generator=gen)[:B].to(dev)

    core = _core(pkg, dev, Hk, Hv, D, conv_w, A_log, dt_bias, norm_w, fused_decode=False)
    cp1, sp1 = conv0.clone(), s0.clone()
    ref = core.decode(mixed, z, b, a, ids, cp1, sp1).reshape(B, 1, Hv * D)

    mod = types.ModuleType("qwen3_5_stub")

    class Qwen3_5GatedDeltaNet:
        def _gdn_padded(self, x, lens, ids, T):
            raise AssertionError("the original method must not run")

    mod.Qwen3_5GatedDeltaNet = Qwen3_5GatedDeltaNet
    prev = pkg.integration.install(mod)
    try:
        layer = Qwen3_5GatedDeltaNet()
        layer.num_k_heads, layer.num_v_heads, layer.head_k_dim, layer.head_v_dim = Hk, Hv, D, D
        layer.key_dim, layer.value_dim, layer.conv_dim, layer.conv_kernel = Hk * D, Hv * D, C, 4
        layer.in_proj_b = lambda h: b.view(B, 1, Hv)
        layer.in_proj_a = lambda h: a.view(B, 1, Hv)
        layer.in_proj_z = lambda h: z.view(B, 1, Hv * D)
        layer.in_proj_qkv = lambda h: mixed.view(B, 1, C)
        layer.A_log, layer.dt_bias, layer._v_head_slice = A_log.to(dev), dt_bias.to(dev), slice(0, Hv)
        layer.conv1d = types.SimpleNamespace(weight=conv_w.to(dev).view(C, 1, 4))
        norm = pkg.ops.Qwen3_5RMSNormGated(D)
        norm.weight.data = norm_w.to(dev)
        layer.norm = norm
        layer.out_proj = lambda x: x
        layer.conv_cache, layer.s_cache = conv0.clone(), s0.clone()
        out = layer._gdn_padded(torch.empty(B, 1, 8, device=dev), None, ids, 1)
    finally:
        pkg.integration.uninstall(mod, prev)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    assert torch.equal(layer.s_cache, sp1)
    assert torch.equal(layer.conv_cache.view(torch.int16), cp1.view(torch.int16))


def test_split_state_pass_equals_one_stream(pkg, dev):
    """Config 1 with the state pass split over two streams (the long sequences
    on the current stream, the rest and their gated norm on a side stream)
    gives the one-stream results bit for bit, pools included."""
    cfg = bench.make_prefill(1, None)
    assert pkg.gdn_layer.late_split(cfg["lens"], cfg["Hv"]) is not None, "config 1 should split"
    n = len(cfg["lens"])
    outs = []
    for split in (False, True):
        core = _core(pkg, dev, cfg["Hk"], cfg["Hv"], cfg["D"], cfg["conv_w"], cfg["A_log"], cfg["dt_bias"],
                     cfg["norm_w"], split_state=split)
        cp, sp = cfg["conv_state"].to(dev), cfg["h0"].to(dev)
        for rep in range(2):      # twice: the second call reuses cached split metadata and allocator blocks
            out = core.prefill_varlen(cfg["x"].to(dev), cfg["z"].to(dev), cfg["b"].to(dev), cfg["a"].to(dev),
                                      cfg["lens"], torch.arange(n, device=dev), cp, sp)
        torch.cuda.synchronize()
        outs.append((out.cpu(), cp.cpu(), sp.cpu()))
    (o1, c1, s1), (o2, c2, s2) = outs
    assert torch.equal(o1.view(torch.int16), o2.view(torch.int16)), "outputs differ"
    assert torch.equal(c1.view(torch.int16), c2.view(torch.int16)), "conv pool differs"
    assert torch.equal(s1, s2), "state pool differs"
