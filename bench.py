#!/usr/bin/env python3
"""Benchmark of the GDN layer path on one MI355X.

Headline (`value`): config 1 -- varlen prefill of one GDN layer core
(fused g/beta + varlen conv + chunked gated delta rule + gated RMSNorm, the
path between the projections) over 8 sequences with lengths ~U[128, 4096]
(seed 1; 17,001 tokens), Hk = Hv = 16, d = 128, chunk 64, tokens/s.
`roofline` is the dominant kernel of that step (the chunk prefill, MFMA
bound); `cpu_baseline` is this repo's CPU oracle of the same path on a
bounded slice of the same workload.  Extra objects carry config 2 (batched
decode, HBM bound), config 3 (65,536-token prefill) and config 4
(speculative-verify multi-token decode).

Inputs are synthetic, generated with one seeded CPU torch.Generator per
config in a fixed order, then moved to HBM before the timed region.  Every
kernel runs inside the timed steps; per-kernel durations come from HIP
events recorded on the stream the kernels are launched on.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--configs 1,2,3,4]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import platform
import statistics
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

METRIC = "GDN prefill tokens/s (MFMA util); decode state GB/s vs HBM peak, 1 GPU"
HBM_PEAK_GBPS = 8000.0          # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0       # MI355X dense bf16 MFMA
BF16 = torch.bfloat16


def prefill_compulsory_bytes(cfg) -> int:
    """HBM bytes the fused prefill call cannot avoid: the conv input rows
    (bf16 [N, C]), the b / a gate inputs (bf16 [N, Hv] each), the output
    (bf16 [N, Hv*D]), each sequence's state read and written (fp32
    [Hv, D, D]) and its conv state read and written (bf16 [C, 3])."""
    N, C, Hv, D, n = cfg["N"], cfg["C"], cfg["Hv"], cfg["D"], len(cfg["lens"])
    return N * (2 * C + 4 * Hv + 2 * Hv * D) + n * (2 * 4 * Hv * D * D + 2 * 2 * C * 3)


def chunk_flops(n_tokens: int, Hv: int, D: int, C: int = 64) -> float:
    """Algorithmic chunk-prefill FLOPs per call: N*Hv*[2C(3D+2D) + 6D^2 + (2/3)C^2]
    (full QK^T/KK^T tiles, W, U, intra-chunk O, three state GEMMs, the solve)."""
    return float(n_tokens) * Hv * (2 * C * (3 * D + 2 * D) + 6 * D * D + (2.0 / 3.0) * C * C)


# ------------------------------------------------------------------ inputs --
def _params(gen, Hv, D, C):
    A_log = (torch.rand(Hv, generator=gen) * math.log(16)).to(BF16)
    dt_bias = (torch.rand(Hv, generator=gen) * 2 - 1).to(BF16)
    conv_w = (torch.randn(C, 4, generator=gen) * 0.5).to(BF16)
    norm_w = (1 + 0.02 * torch.randn(D, generator=gen)).to(BF16)
    return A_log, dt_bias, conv_w, norm_w


def make_prefill(seed: int, lens: list[int] | None, Hk=16, Hv=16, D=128, h0_std=0.0, conv_std=0.0):
    """Config 1 (seed 1, lens ~U[128,4096] x 8) / config 3 (seed 4, 1 x 65536,
    h0 ~ N(0, 0.1^2), conv prefix ~ N(0,1)).  Draw order: lens, x, z, a, b,
    A_log, dt_bias, conv_w, norm_w, h0, conv state."""
    gen = torch.Generator().manual_seed(seed)
    if lens is None:
        lens = torch.randint(128, 4097, (8,), generator=gen).tolist()
    N = sum(lens)
    C = 2 * Hk * D + Hv * D
    x = torch.randn(N, C, generator=gen).to(BF16)
    z = torch.randn(N, Hv * D, generator=gen).to(BF16)
    a = torch.randn(N, Hv, generator=gen).to(BF16)
    b = torch.randn(N, Hv, generator=gen).to(BF16)
    A_log, dt_bias, conv_w, norm_w = _params(gen, Hv, D, C)
    n = len(lens)
    h0 = torch.randn(n, Hv, D, D, generator=gen) * h0_std if h0_std else torch.zeros(n, Hv, D, D)
    cs = (torch.randn(n, C, 3, generator=gen) * conv_std).to(BF16) if conv_std else torch.zeros(n, C, 3, dtype=BF16)
    return dict(lens=lens, N=N, Hk=Hk, Hv=Hv, D=D, C=C, x=x, z=z, a=a, b=b, A_log=A_log, dt_bias=dt_bias,
                conv_w=conv_w, norm_w=norm_w, h0=h0, conv_state=cs)


def make_decode(seed=2, B=256, slots=512, Hk=16, Hv=16, D=128):
    """Config 2: ids = randperm(512)[:256], s_pool ~ N(0, 0.1^2) [512,16,128,128],
    conv_pool ~ N(0,1) [512, 6144, 3]; one token per sequence.
    Draw order: ids, s_pool, conv_pool, x, z, a, b, A_log, dt_bias, conv_w, norm_w."""
    gen = torch.Generator().manual_seed(seed)
    C = 2 * Hk * D + Hv * D
    ids = torch.randperm(slots, generator=gen)[:B]
    s_pool = torch.randn(slots, Hv, D, D, generator=gen) * 0.1
    conv_pool = torch.randn(slots, C, 3, generator=gen).to(BF16)
    x = torch.randn(B, C, generator=gen).to(BF16)
    z = torch.randn(B, Hv * D, generator=gen).to(BF16)
    a = torch.randn(B, Hv, generator=gen).to(BF16)
    b = torch.randn(B, Hv, generator=gen).to(BF16)
    A_log, dt_bias, conv_w, norm_w = _params(gen, Hv, D, C)
    return dict(B=B, Hk=Hk, Hv=Hv, D=D, C=C, ids=ids, s_pool=s_pool, conv_pool=conv_pool, x=x, z=z, a=a, b=b,
                A_log=A_log, dt_bias=dt_bias, conv_w=conv_w, norm_w=norm_w)


def make_spec(seed=3, B=64, T=4, slots=128, Hk=16, Hv=32, D=128):
    """Config 4: 64 sequences x 4 draft tokens, Hk=16 / Hv=32, pool [128,32,128,128]
    ~ N(0, 0.1^2), ids = randperm(128)[:64], accepted ~ U{1..4}.
    Draw order: ids, s_pool, q, k, v, a, b, A_log, dt_bias, accepted."""
    gen = torch.Generator().manual_seed(seed)
    ids = torch.randperm(slots, generator=gen)[:B]
    s_pool = torch.randn(slots, Hv, D, D, generator=gen) * 0.1
    q = torch.randn(B, T, Hk, D, generator=gen).to(BF16)
    k = torch.randn(B, T, Hk, D, generator=gen).to(BF16)
    v = torch.randn(B, T, Hv, D, generator=gen).to(BF16)
    a = torch.randn(B, T, Hv, generator=gen).to(BF16)
    b = torch.randn(B, T, Hv, generator=gen).to(BF16)
    A_log = (torch.rand(Hv, generator=gen) * math.log(16)).to(BF16)
    dt_bias = (torch.rand(Hv, generator=gen) * 2 - 1).to(BF16)
    accepted = torch.randint(1, T + 1, (B,), generator=gen)
    return dict(B=B, T=T, Hk=Hk, Hv=Hv, D=D, ids=ids, s_pool=s_pool, q=q, k=k, v=v, a=a, b=b, A_log=A_log,
                dt_bias=dt_bias, accepted=accepted)


def _profiled_traffic(name: str):
    """HBM bytes per launch of a kernel, as measured by the rocprofv3 PMC runs
    (FETCH_SIZE + WRITE_SIZE, scaled by a plain copy's counters) recorded in
    profiles/<name>_traffic.md on a line `traffic_bytes_per_launch: <int>`;
    None when no such measurement is committed."""
    import re

    f = ROOT / "profiles" / f"{name}_traffic.md"
    try:
        m = re.search(r"traffic_bytes_per_launch:\s*([0-9]+)", f.read_text())
    except OSError:
        return None
    return int(m.group(1)) if m else None


# ------------------------------------------------------------------ timing --
class EventTimer:
    """HIP events around named kernels on torch's current stream (the stream
    the kernels are launched on).  `only`: record just these names (each
    event pair costs the stream a few microseconds, so the timed steps carry
    events around the measured kernel only)."""

    def __init__(self, only=None):
        self.open: dict[str, torch.cuda.Event] = {}
        self.pairs: dict[str, list] = {}
        self.only = only

    def start(self, name):
        if self.only is not None and name not in self.only:
            return
        e = torch.cuda.Event(enable_timing=True)
        e.record()
        self.open[name] = e

    def stop(self, name):
        if self.only is not None and name not in self.only:
            return
        e = torch.cuda.Event(enable_timing=True)
        e.record()
        self.pairs.setdefault(name, []).append((self.open.pop(name), e))

    def reset(self):
        self.pairs.clear()

    def avg_us(self) -> dict[str, float]:
        return {k: 1e3 * statistics.fmean(s.elapsed_time(e) for s, e in v) for k, v in self.pairs.items()}


# Untimed load before every timed leg, whatever --warmup says: the GPU's
# clock settles only after some tenths of a second of sustained work (config
# 1 measured 0.297 ms per step after 5 warm-up steps, 0.260 ms after 2000).
SETTLE_S = 1.0


def settle(step, W: int, seconds: float = SETTLE_S) -> int:
    """Run `step` untimed at least W times and for at least `seconds` of wall
    time, synchronising after each call so the wall time is device time.
    Returns the number of calls."""
    torch.cuda.synchronize()
    t_end = time.perf_counter() + seconds
    n = 0
    while n < W or time.perf_counter() < t_end:
        step()
        torch.cuda.synchronize()
        n += 1
    return n


def timed_steps(step, K: int) -> float:
    """Wall-clock seconds of exactly K steps, synchronised on both sides."""
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(K):
        step()
    torch.cuda.synchronize()
    return time.perf_counter() - t0


def burst_us(fn, R: int = 20, blocks: int = 3) -> float:
    """Average duration of one call of `fn` (a fixed sequence of launches on
    the current stream): the median over `blocks` of R back-to-back calls
    between one event pair (an event pair around every call would add its own
    few microseconds to each)."""
    fn()
    torch.cuda.synchronize()
    per = []
    for _ in range(blocks):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(R):
            fn()
        e1.record()
        torch.cuda.synchronize()
        per.append(1e3 * e0.elapsed_time(e1) / R)
    return statistics.median(per)


# -------------------------------------------------------------- workloads --
def prefill_bench(pkg, cfg, dev, K, W, rule_only=False):
    """Config 1 / 3 layer-core prefill.  Returns (seconds per step, kernel us):
    after a settling period, K timed steps of the whole core (the fused launch
    pair, then the gated norm); then the fused launch pair and the norm each
    timed on their own as bursts of back-to-back calls (burst_us), the pair
    being the launches the steps run.  rule_only: also the chunk rule alone
    (gdn_chunk_prefill on the conv outputs, q / k / v / g / beta precomputed
    by the standalone kernels), as "chunk_prefill"."""
    core = pkg.GatedDeltaNetCore(cfg["Hk"], cfg["Hv"], cfg["D"], cfg["conv_w"].to(dev), cfg["A_log"].to(dev),
                                 cfg["dt_bias"].to(dev), cfg["norm_w"].to(dev))
    x, z, a, b = (cfg[k].to(dev) for k in ("x", "z", "a", "b"))
    n = len(cfg["lens"])
    s_pool = cfg["h0"].to(dev)
    conv_pool = cfg["conv_state"].to(dev)
    ids = torch.arange(n, device=dev)
    lens = cfg["lens"]
    Hk, Hv, D, N = cfg["Hk"], cfg["Hv"], cfg["D"], cfg["N"]

    def step():
        core.prefill_varlen(x, z, b, a, lens, ids, conv_pool, s_pool)

    settle(step, W)
    t = timed_steps(step, K)
    _, _, cu64_cpu, cu64_gpu = pkg.state_pool.varlen_meta(lens, dev)
    assert core.sw.fused_prefill and core.sw.gbeta and core.sw.conv_kernel, "the bench times the fused prefill"

    def pair():
        return pkg.ops.conv_chunk_prefill_varlen(x, conv_pool, core.conv_w, b, a, core.A_log, core.dt_bias, cu64_gpu,
                                                 s_pool, ids, Hk, Hv, D, cu_seqlens_cpu=cu64_cpu)

    o = pair()
    zz = z.view(N, Hv, D)
    us = {"conv_chunk_prefill": burst_us(pair),
          "rmsnorm_gated": burst_us(lambda: pkg.ops.rms_norm_gated(o, zz, core.norm_w, core.eps))}
    if rule_only:
        lens32 = torch.tensor(lens, dtype=torch.int32, device=dev)
        starts = torch.tensor([0] + torch.tensor(lens).cumsum(0)[:-1].tolist(), dtype=torch.int32, device=dev)
        cstate = conv_pool.clone()
        q, k, v = pkg.ops.causal_conv_silu_varlen_parts(x, cstate, core.conv_w, lens32, starts, Hk * D,
                                                        state_ids=ids)
        g, beta = pkg.ops.fused_g_beta(b, a, core.A_log, core.dt_bias, None)
        qv, kv, vv = q.view(N, Hk, D), k.view(N, Hk, D), v.view(N, Hv, D)

        def rule():
            pkg.ops.chunk_gated_delta_rule_varlen(qv, kv, vv, g, beta, cu64_gpu, s_pool, state_ids=ids,
                                                  final_state=s_pool, cu_seqlens_cpu=cu64_cpu)
        settle(rule, 1, 0.3)
        us["chunk_prefill"] = burst_us(rule)
    return t / K, us


def layer_bench(pkg, cfg, dev, K, W, hidden=2048):
    """Config 1 through the whole GDN mixer (GatedDeltaNetLayer): in_proj GEMM
    over the concatenated qkv / z / b / a weights, the layer core, out_proj
    GEMM.  Random-init weights of a 2048 hidden size (the configs do not name
    one).  Also times the same two GEMM shapes through torch.matmul (hipBLASLt)
    for comparison."""
    import math
    gen = torch.Generator().manual_seed(11)
    Hk, Hv, D = cfg["Hk"], cfg["Hv"], cfg["D"]
    C = cfg["C"]
    s = 1 / math.sqrt(hidden)
    ws = [(torch.randn(r, hidden, generator=gen) * s).to(BF16).to(dev) for r in (C, Hv * D, Hv, Hv)]
    w_out = (torch.randn(hidden, Hv * D, generator=gen) / math.sqrt(Hv * D)).to(BF16).to(dev)
    layer = pkg.GatedDeltaNetLayer(*ws, w_out, Hk, Hv, D, cfg["conv_w"].to(dev), cfg["A_log"].to(dev),
                                   cfg["dt_bias"].to(dev), cfg["norm_w"].to(dev))
    N = cfg["N"]
    x = torch.randn(N, hidden, generator=gen).to(BF16).to(dev)
    n = len(cfg["lens"])
    cu = torch.tensor([0] + torch.tensor(cfg["lens"]).cumsum(0).tolist(), dtype=torch.int32, device=dev)
    ids = torch.arange(n, device=dev)
    s_pool, conv_pool = cfg["h0"].to(dev), cfg["conv_state"].to(dev)
    lens = cfg["lens"]

    def step():
        layer.forward(x, cu, max(lens), ids, conv_pool, s_pool, lens_q=lens)

    settle(step, W)
    t = timed_steps(step, K)
    timer = EventTimer()
    layer.timer = timer
    for _ in range(min(K, 20)):
        step()
    torch.cuda.synchronize()
    layer.timer = None
    layer.core.timer = None
    us = timer.avg_us()
    # the same GEMM shapes through torch.matmul (hipBLASLt)
    y_in = torch.empty(N, layer.n_in, dtype=BF16, device=dev)
    core_out = torch.randn(N, Hv * D, generator=gen).to(BF16).to(dev)
    y_out = torch.empty(N, hidden, dtype=BF16, device=dev)
    ref = EventTimer()
    settle(lambda: (torch.matmul(x, layer.w_in.t(), out=y_in), torch.matmul(core_out, layer.w_out.t(), out=y_out)),
           3, 0.3)
    for _ in range(10):
        ref.start("in_proj_hipblaslt")
        torch.matmul(x, layer.w_in.t(), out=y_in)
        ref.stop("in_proj_hipblaslt")
        ref.start("out_proj_hipblaslt")
        torch.matmul(core_out, layer.w_out.t(), out=y_out)
        ref.stop("out_proj_hipblaslt")
    torch.cuda.synchronize()
    return t / K, us, ref.avg_us(), layer.n_in, hidden


def layer_decode_bench(pkg, cfg, dev, K, W, hidden=2048):
    """Config 2 (256 one-token rows, slots of a 512-slot pool) through the
    whole GDN mixer (GatedDeltaNetLayer, decode path): in_proj GEMM, the fused
    decode kernel with its gated norm, out_proj GEMM.  Random-init weights of
    a 2048 hidden size.  Also times the same two GEMM shapes through
    torch.matmul (hipBLASLt)."""
    import math
    gen = torch.Generator().manual_seed(12)
    Hk, Hv, D, C, B = cfg["Hk"], cfg["Hv"], cfg["D"], cfg["C"], cfg["B"]
    s = 1 / math.sqrt(hidden)
    ws = [(torch.randn(r, hidden, generator=gen) * s).to(BF16).to(dev) for r in (C, Hv * D, Hv, Hv)]
    w_out = (torch.randn(hidden, Hv * D, generator=gen) / math.sqrt(Hv * D)).to(BF16).to(dev)
    layer = pkg.GatedDeltaNetLayer(*ws, w_out, Hk, Hv, D, cfg["conv_w"].to(dev), cfg["A_log"].to(dev),
                                   cfg["dt_bias"].to(dev), cfg["norm_w"].to(dev))
    x = torch.randn(B, hidden, generator=gen).to(BF16).to(dev)
    cu = torch.arange(B + 1, dtype=torch.int32, device=dev)
    ids = cfg["ids"].to(dev)
    s_pool, conv_pool = cfg["s_pool"].to(dev), cfg["conv_pool"].to(dev)
    lens = [1] * B

    def step():
        layer.forward(x, cu, 1, ids, conv_pool, s_pool, lens_q=lens)

    settle(step, W)
    t = timed_steps(step, K)
    # the same step replayed from a captured HIP graph (how the engine runs decode)
    g = torch.cuda.CUDAGraph()
    gs = torch.cuda.Stream()
    gs.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(gs):
        step()
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=gs):
            step()
    torch.cuda.current_stream().wait_stream(gs)
    settle(g.replay, W)
    t_graph = timed_steps(g.replay, K)
    timer = EventTimer()
    layer.timer = timer
    for _ in range(min(K, 20)):
        step()
    torch.cuda.synchronize()
    layer.timer = None
    layer.core.timer = None
    us = timer.avg_us()
    y_in = torch.empty(B, layer.n_in, dtype=BF16, device=dev)
    core_out = torch.randn(B, Hv * D, generator=gen).to(BF16).to(dev)
    y_out = torch.empty(B, hidden, dtype=BF16, device=dev)
    ref = EventTimer()
    settle(lambda: (torch.matmul(x, layer.w_in.t(), out=y_in), torch.matmul(core_out, layer.w_out.t(), out=y_out)),
           3, 0.3)
    for _ in range(10):
        ref.start("in_proj_hipblaslt")
        torch.matmul(x, layer.w_in.t(), out=y_in)
        ref.stop("in_proj_hipblaslt")
        ref.start("out_proj_hipblaslt")
        torch.matmul(core_out, layer.w_out.t(), out=y_out)
        ref.stop("out_proj_hipblaslt")
    torch.cuda.synchronize()
    return t / K, t_graph / K, us, ref.avg_us(), layer.n_in


def decode_bench(pkg, cfg, dev, K, W):
    """Config 2 decode step of one layer core.  The timed steps alternate the
    batch's 256 slots with the pool's other 256 (the same inputs), so no step
    finds its states in the last-level cache from the step before -- as in
    the engine, where a layer's states come back after every other layer's
    have streamed through.  Also the same steps on one slot set ("hot": each
    step re-reads the states the previous one wrote), and both forms replayed
    from HIP graphs (how the engine runs decode)."""
    core = pkg.GatedDeltaNetCore(cfg["Hk"], cfg["Hv"], cfg["D"], cfg["conv_w"].to(dev), cfg["A_log"].to(dev),
                                 cfg["dt_bias"].to(dev), cfg["norm_w"].to(dev))
    x, z, a, b = (cfg[k].to(dev) for k in ("x", "z", "a", "b"))
    s_pool = cfg["s_pool"].to(dev)
    conv_pool = cfg["conv_pool"].to(dev)
    ids = cfg["ids"].to(dev)
    used = set(ids.tolist())
    other = torch.tensor([i for i in range(s_pool.shape[0]) if i not in used][:ids.numel()], device=dev)
    sets = [ids, other] if other.numel() == ids.numel() else [ids]
    turn = [0]

    def step_on(sl):
        core.decode(x, z, b, a, sl, conv_pool, s_pool)

    def step():
        step_on(sets[turn[0] % len(sets)])
        turn[0] += 1

    settle(step, W)
    timer = EventTimer()
    core.timer = timer
    t = timed_steps(step, K)
    core.timer = None
    t_hot = timed_steps(lambda: step_on(ids), K)
    # the same steps replayed from captured HIP graphs, one per slot set
    graphs = []
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for sl in sets:
            step_on(sl)
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=s):
                step_on(sl)
            graphs.append(g)
    torch.cuda.current_stream().wait_stream(s)
    gturn = [0]

    def replay():
        graphs[gturn[0] % len(graphs)].replay()
        gturn[0] += 1

    settle(replay, W)
    t_graph = timed_steps(replay, K)
    t_graph_hot = timed_steps(graphs[0].replay, K)
    rec_us, pass_us, copy_us = recurrent_burst_us(pkg, cfg, core, x, a, b, ids, conv_pool, s_pool, z)
    return t / K, t_graph / K, timer.avg_us(), rec_us, pass_us, copy_us, t_hot / K, t_graph_hot / K


def decode_gva_bench(pkg, dev, K, W):
    """Config 2's decode step at Qwen3.5's grouped geometry (16 key heads, 32
    value heads; pool [512, 32, 128, 128]), B = 256.  Two heads share each key
    head, so the step is two launches: the q/k decode conv, then the fused
    kernel (gates, v conv with its roll, state update, gated norm).  Returns
    (s per step cold, fused kernel us, tile pass us).  (The q/k conv is not
    burst-timed on its own: at 16 MB a launch it is shorter than a call's
    host overhead, so back-to-back calls would time the host.)"""
    cfg = make_decode(Hk=16, Hv=32)
    core = pkg.GatedDeltaNetCore(cfg["Hk"], cfg["Hv"], cfg["D"], cfg["conv_w"].to(dev), cfg["A_log"].to(dev),
                                 cfg["dt_bias"].to(dev), cfg["norm_w"].to(dev))
    x, z, a, b = (cfg[k].to(dev) for k in ("x", "z", "a", "b"))
    s_pool = cfg["s_pool"].to(dev)
    conv_pool = cfg["conv_pool"].to(dev)
    ids = cfg["ids"].to(dev)
    del cfg["s_pool"]
    used = set(ids.tolist())
    other = torch.tensor([i for i in range(s_pool.shape[0]) if i not in used][:ids.numel()], device=dev)
    sets = [ids, other]
    turn = [0]

    def step():
        core.decode(x, z, b, a, sets[turn[0] % 2], conv_pool, s_pool)
        turn[0] += 1

    settle(step, W)
    t = timed_steps(step, K)
    rec_us, pass_us, _ = recurrent_burst_us(pkg, cfg, core, x, a, b, ids, conv_pool, s_pool, z)
    return t / K, rec_us, pass_us


def recurrent_burst_us(pkg, cfg, core, x, a, b, ids, conv_pool, s_pool, z_rows, R=20):
    """Average duration of the in-place recurrent kernel over R back-to-back
    launches between one event pair (an event pair around each launch adds a
    few microseconds to what it measures).  Launches alternate the batch's
    slots with the pool's other slots, so no launch finds its states cached
    from the one before (the pool is larger than the last-level cache).
    Also times, the same way, the state tile pass: the same state tiles read
    and written back in place with no arithmetic (the ceiling of this access
    pattern), and its out-of-place form (the tiles written to a second pool at
    the same offsets).  Returns (kernel us, tile pass us, tile copy us)."""
    B, Hk, Hv, D = x.shape[0], cfg["Hk"], cfg["Hv"], cfg["D"]
    kd = Hk * D
    used = set(ids.tolist())
    other = [i for i in range(s_pool.shape[0]) if i not in used][:B]
    sets = [ids, torch.tensor(other, device=ids.device)] if len(other) == B else [ids]
    if core.sw.fused_decode:
        # the kernel the decode step runs: the whole step (q/k/v conv, gates,
        # state update, norm) with one key head per value head and whole heads
        # per workgroup, else gates + v conv + state update after the q/k conv
        whole = Hk == Hv and B * Hv >= pkg.ops.WHOLE_HEAD_TILES
        qk = None if whole else pkg.ops.conv_decode_step(x[:, :2 * kd], conv_pool[:, :2 * kd], ids,
                                                           core.conv_w[:2 * kd])

        zz = z_rows

        def launch(sl):
            pkg.ops.recurrent_decode_fused(qk, x, conv_pool, core.conv_w, b, a, core.A_log, core.dt_bias, s_pool,
                                           sl, Hk, Hv, D, z=zz, norm_weight=core.norm_w, eps=core.eps)
    else:
        g, beta = pkg.ops.fused_g_beta(b, a, core.A_log, core.dt_bias, None)
        y = pkg.ops.conv_decode_step(x, conv_pool, ids, core.conv_w)
        q, k, v = y[:, :kd].view(B, 1, Hk, D), y[:, kd:2 * kd].view(B, 1, Hk, D), y[:, 2 * kd:].view(B, 1, Hv, D)
        g1, b1 = g.view(B, 1, Hv), beta.view(B, 1, Hv)

        def launch(sl):
            pkg.ops.recurrent_gdn_inplace(q, k, v, g1, b1, s_pool, sl)
    rec = _burst_us(launch, sets, R)
    tile = _burst_us(lambda sl: pkg.ops.state_tile_pass(s_pool, sl), sets, R)
    dst = torch.empty_like(s_pool)
    copy = _burst_us(lambda sl: pkg.ops.state_tile_copy(s_pool, dst, sl), sets, R)
    del dst
    return rec, tile, copy


def _burst_us(launch, sets, R):
    """Average duration of one launch: the median over three blocks of R
    back-to-back launches over the slot sets in turn, each block between one
    event pair (after an untimed launch)."""
    i = [0]

    def one():
        launch(sets[i[0] % len(sets)])
        i[0] += 1
    return burst_us(lambda: [one() for _ in range(len(sets))], max(1, R // len(sets))) / len(sets)


def spec_bench(pkg, cfg, dev, K, W):
    """Config 4 in steady state: each step verifies T draft tokens per row
    starting from the previous step's accepted states (ops.SpecVerify: the
    rollback folded into the next step, no commit copy), then records the
    accepted lengths.  Kernel times are bursts of back-to-back steps:
    "recurrent_multitoken" as the steps run (each verify reads the states the
    previous one wrote, partly still in the last-level cache), and
    "recurrent_multitoken_cold" alternating two verifiers on the pool's two
    disjoint halves of rows, so that a verify's start states were written two
    steps (1.2 GB of traffic) earlier.  The commit-copy kernel is timed on its
    own for comparison."""
    B, T, Hv, D = cfg["B"], cfg["T"], cfg["Hv"], cfg["D"]
    q, k, v, a, b = (cfg[n].to(dev) for n in ("q", "k", "v", "a", "b"))
    g, beta = pkg.ops.fused_g_beta(b, a, cfg["A_log"].to(dev), cfg["dt_bias"].to(dev), None)
    s_pool = cfg["s_pool"].to(dev)
    ids = cfg["ids"].to(dev)
    acc = cfg["accepted"].to(device=dev, dtype=torch.int64)
    spec = pkg.ops.SpecVerify(s_pool)

    def step(sp=spec, rows=ids):
        sp.verify(q, k, v, g, beta, rows)
        sp.accept(acc)          # no device work: the next verify reads the accepted states

    settle(step, W)
    t = timed_steps(step, K)
    us = {"recurrent_multitoken": burst_us(step)}
    spec.commit()
    # the other half of the pool's rows, with a verifier of its own
    used = set(ids.tolist())
    other = torch.tensor([i for i in range(s_pool.shape[0]) if i not in used][:B], device=dev)
    if other.numel() == B:
        spec2 = pkg.ops.SpecVerify(s_pool)
        us["recurrent_multitoken_cold"] = burst_us(lambda: (step(), step(spec2, other)), max(1, 10)) / 2
        spec2.commit()
        spec.commit()
    # the commit copy the deferred scheme avoids (for comparison only)
    us["state_commit_copy"] = burst_us(lambda: pkg.ops.commit_states(s_pool, ids, spec.inter, acc), 5)
    return t / K, us


def gemm_shapes(pkg, dev, R=10):
    """gdn_gemm_bf16 (ops.linear) against torch.matmul (hipBLASLt) on the
    mixer's projection shapes (hidden 2048, config 1's 17,001 tokens and a
    decode batch of 256) and a square 8192^3.  Each side's R back-to-back
    launches are captured in a HIP graph (as a graph-captured decode step runs
    them: no host launch cost between the kernels, which at the decode shapes
    is longer than the kernels), and a replay is timed between one event pair,
    three times for each side in turn after about a second of untimed replays
    (the clock settles under load), the median kept; random operands."""
    out = {}
    gen = torch.Generator().manual_seed(13)
    shapes = [(17001, 8224, 2048, "in_proj_config1"), (17001, 2048, 2048, "out_proj_config1"),
              (256, 8224, 2048, "in_proj_decode256"), (256, 2048, 2048, "out_proj_decode256"),
              (8192, 8192, 8192, "square_8192")]
    graphs = {}
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for M, N, K, tag in shapes:
            a = torch.randn(M, K, generator=gen).to(BF16).to(dev)
            w = (torch.randn(N, K, generator=gen) / math.sqrt(K)).to(BF16).to(dev)
            c = torch.empty(M, N, dtype=BF16, device=dev)
            pair = []
            for fn in (lambda: pkg.ops.linear(a, w, out=c), lambda: torch.matmul(a, w.t(), out=c)):
                fn()
                torch.cuda.synchronize()
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g, stream=side):
                    for _ in range(R):
                        fn()
                pair.append(g)
            graphs[tag] = (pair, a, w, c)
    torch.cuda.current_stream().wait_stream(side)
    t_end = time.time() + 1.0
    while time.time() < t_end:
        for (g_ours, _), *_ in graphs.values():
            g_ours.replay()
        torch.cuda.synchronize()

    def t(g):
        g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        g.replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / R * 1e3
    for M, N, K, tag in shapes:
        (g_ours, g_lib), *_ = graphs[tag]
        ts, th = [], []
        for _ in range(3):
            ts.append(t(g_ours))
            th.append(t(g_lib))
        us, us_h = statistics.median(ts), statistics.median(th)
        fl = 2.0 * M * N * K
        out[tag] = {"M": M, "N": N, "K": K, "us": round(us, 1), "TFLOPs": round(fl / us / 1e6, 1),
                    "hipblaslt_us": round(us_h, 1), "hipblaslt_TFLOPs": round(fl / us_h / 1e6, 1)}
    return out


def standalone_kernels(pkg, cfg, dev, K, W):
    """The kernels the fused prefill replaces, each launched on its own at
    config 1's shapes (the path the unfused switches select): the gates, the
    varlen conv, the padded conv (sequences padded to the longest; input both
    [n, C, T] contiguous and the reference's [n, T, C] rows seen as [n, C, T]),
    the gated norm.  Returns {kernel: (average us over K launches, compulsory
    bytes)}."""
    N, C, Hv, D = cfg["N"], cfg["C"], cfg["Hv"], cfg["D"]
    lens = cfg["lens"]
    n, T = len(lens), max(lens)
    x, z, a, b = (cfg[k].to(dev) for k in ("x", "z", "a", "b"))
    A_log, dt_bias, w = cfg["A_log"].to(dev), cfg["dt_bias"].to(dev), cfg["conv_w"].to(dev)
    lens32 = torch.tensor(lens, dtype=torch.int32, device=dev)
    starts = torch.tensor([0] + torch.tensor(lens).cumsum(0)[:-1].tolist(), dtype=torch.int32, device=dev)
    st_v = torch.zeros(n, C, 3, dtype=BF16, device=dev)
    xp = torch.zeros(n, C, T, dtype=BF16, device=dev)
    for i, (s0, l) in enumerate(zip(starts.tolist(), lens)):
        xp[i, :, :l] = x[s0:s0 + l].t()
    st_p = torch.zeros(n, C, 3, dtype=BF16, device=dev)
    # the reference's own padded layout: [n, T, C] rows seen as [n, C, T] (channel stride 1)
    xt = torch.zeros(n, T, C, dtype=BF16, device=dev)
    for i, (s0, l) in enumerate(zip(starts.tolist(), lens)):
        xt[i, :l] = x[s0:s0 + l]
    st_t = torch.zeros(n, C, 3, dtype=BF16, device=dev)
    endp = lens32 - 1
    core = torch.randn(N, Hv, D, device=dev).to(BF16)
    zz = z.view(N, Hv, D)
    nw = cfg["norm_w"].to(dev)
    kd = cfg["Hk"] * D
    launches = {
        "g_beta_kernel": (lambda: pkg.ops.fused_g_beta(b, a, A_log, dt_bias, None), N * Hv * (2 + 2 + 4 + 2)),
        "conv_varlen_kernel": (lambda: pkg.ops.causal_conv_silu_varlen_parts(x, st_v, w, lens32, starts, kd),
                               2 * N * C * 2),
        "conv_padded_kernel": (lambda: pkg.ops.causal_conv_silu(xp, st_p, w, endp), 2 * n * C * T * 2),
        "conv_padded_kernel (channel-stride-1 input)": (lambda: pkg.ops.causal_conv_silu(xt.transpose(1, 2), st_t, w, endp),
                                                        2 * n * C * T * 2),
        "rmsnorm_gated_kernel": (lambda: pkg.ops.rms_norm_gated(core, zz, nw, 1e-6), 3 * N * Hv * D * 2),
    }
    out = {}
    for name, (fn, nbytes) in launches.items():
        for _ in range(W):
            fn()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(K):
            fn()
        e1.record()
        torch.cuda.synchronize()
        out[name] = (1e3 * e0.elapsed_time(e1) / K, nbytes)
    return out


CPU_SHARE = 16


def _usable_cpus() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        return os.cpu_count() or 1


def cpu_baseline(cfg, n_seq: int, threads: int):
    """CPU oracle (fp32 torch restatement of the reference path) on the first
    n_seq sequences of config 1 (the bench passes all of them: the whole
    workload): 1 warm-up on a 256-token slice, median of 3."""
    from oracle import gdn_ref

    torch.set_num_threads(threads)
    lens = cfg["lens"][:n_seq]
    N = sum(lens)
    Hk, Hv, D = cfg["Hk"], cfg["Hv"], cfg["D"]
    args = (cfg["x"][:N], cfg["z"][:N], cfg["b"][:N], cfg["a"][:N])
    common = (cfg["conv_w"], cfg["A_log"], cfg["dt_bias"], cfg["norm_w"], Hk, Hv, D)
    gdn_ref.gdn_core_varlen(*(t[:256] for t in args), [256], cfg["conv_state"][:1], cfg["h0"][:1], *common)
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        gdn_ref.gdn_core_varlen(*args, lens, cfg["conv_state"][:n_seq], cfg["h0"][:n_seq], *common)
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    cpu_name = platform.processor() or ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu_name = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"value": N / t, "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"config 1 GDN core (g/beta+conv+chunk rule+gated norm) on {n_seq} of its "
                      f"{len(cfg['lens'])} sequences "
                      f"({N} tokens, lens {lens}), fp32 torch oracle, median of 3 reps ({t:.2f} s each), "
                      f"{threads} threads (os.cpu_count()={os.cpu_count()}, usable CPUs {_usable_cpus()}, at most "
                      f"{CPU_SHARE}: one GPU's CPU share on the box), cpu='{cpu_name}'"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--configs", default="1,2,3,4,5",
                    help="1-4: BASELINE configs; 5: config 1 through the whole mixer with its projections")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB K times (the reference kernel for "
                         "scaling rocprofv3 FETCH_SIZE / WRITE_SIZE to bytes)")
    ap.add_argument("--gemm-shapes", action="store_true",
                    help="time the projection GEMM against hipBLASLt on the mixer's shapes and exit")
    ap.add_argument("--standalone-kernels", action="store_true",
                    help="only time the gate, varlen-conv, padded-conv and gated-norm kernels on their own at "
                         "config 1's shapes, K launches each")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the GDN path shards by value head / by sequence with no "
              "exchange inside the kernels, so this build reports the single-GPU figure (--gpus 1).",
              file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        sys.exit(2)
    if args.copy_calibration:
        nbytes = args.copy_calibration << 20
        src = torch.ones(nbytes // 4, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes_read": nbytes, "bytes_written": nbytes, "launches": args.steps}))
        return
    import __graft_entry__ as ge

    pkg = ge.load_package()
    pkg._lib.load()
    dev = torch.device("cuda:0")
    K, W = args.steps, args.warmup
    if args.gemm_shapes:
        print(json.dumps({"gemm_shapes": gemm_shapes(pkg, dev)}))
        return
    if args.standalone_kernels:
        res = standalone_kernels(pkg, make_prefill(1, None), dev, K, W)
        print(json.dumps({"standalone_kernels_config1": {
            k: {"us": round(t, 2), "compulsory_bytes": nb, "GBps": round(nb / (t * 1e-6) / 1e9, 1),
                "hbm_frac": round(nb / (t * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4)} for k, (t, nb) in res.items()}}))
        return
    configs = {int(c) for c in args.configs.split(",") if c}
    extra = {}

    cfg1 = make_prefill(1, None)
    N1 = cfg1["N"]
    t1, k1 = prefill_bench(pkg, cfg1, dev, K, W, rule_only=True)
    fused = True
    chunk_us = k1["conv_chunk_prefill"]
    flops = chunk_flops(N1, cfg1["Hv"], cfg1["D"])
    achieved = flops / (chunk_us * 1e-6) / 1e12
    floor1 = prefill_compulsory_bytes(cfg1)
    roofline = {"bound": "mfma", "achieved": round(achieved, 2), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": round(achieved / BF16_PEAK_TFLOPS, 4),
                "hbm_floor_frac": round(floor1 / (chunk_us * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4),
                "compulsory_bytes_per_launch": floor1,
                "traffic": _profiled_traffic("conv_chunk_prefill_config1" if fused else "chunk_prefill_config1"),
                "kernel": ("gates + conv1d/SiLU + chunk rule = chunk_prep_kernel<128, true> + "
                           "chunk_state_kernel<128, true> (one launch pair per call; the time includes the conv and "
                           "gates, the flop count is the chunk rule's matrix products)" if fused else
                           "chunk prefill = chunk_prep_kernel<128, false> + chunk_state_kernel<128, false> "
                           "(one launch pair per call)"),
                "kernel_us": round(chunk_us, 2), "algorithmic_flop_per_launch": flops,
                "timing": "median of 3 blocks of 20 back-to-back calls, each block between one event pair, after "
                          f"{SETTLE_S:.1f} s of untimed steps"}
    rule_us = k1["chunk_prefill"]
    a_rule = flops / (rule_us * 1e-6) / 1e12
    roofline_rule = {"bound": "mfma", "achieved": round(a_rule, 2), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(a_rule / BF16_PEAK_TFLOPS, 4),
                     "traffic": _profiled_traffic("chunk_prefill_config1"),
                     "kernel": "chunk rule alone = chunk_prep_kernel<128, false> + chunk_state_kernel<128, false> on "
                               "the conv outputs (q, k, v, g, beta precomputed; the varlen fla call's boundary)",
                     "kernel_us": round(rule_us, 2), "algorithmic_flop_per_launch": flops,
                     "timing": "as roofline"}
    kernels1 = {k: round(v, 2) for k, v in k1.items()}

    if 5 in configs:
        t5, k5, r5, n_in, hidden = layer_bench(pkg, cfg1, dev, max(2, K // 4), 2)
        fl_in = 2.0 * N1 * n_in * hidden
        fl_out = 2.0 * N1 * hidden * cfg1["Hv"] * cfg1["D"]
        extra["layer_with_projections_config1"] = {
            "tokens_per_s": round(N1 / t5, 1), "ms_per_step": round(t5 * 1e3, 4), "hidden": hidden,
            "kernels_us": {k: round(v, 2) for k, v in k5.items()},
            "in_proj_TFLOPs": round(fl_in / (k5["in_proj"] * 1e-6) / 1e12, 1),
            "out_proj_TFLOPs": round(fl_out / (k5["out_proj"] * 1e-6) / 1e12, 1),
            "hipblaslt_same_shapes_us": {k: round(v, 2) for k, v in r5.items()},
            "note": "in_proj = one GEMM over the concatenated qkv/z/b/a weights [N, 2048] x [8224, 2048]^T; "
                    "out_proj [N, 2048] x [2048, 2048]^T; random-init weights"}
        c2l = make_decode()
        t6, t6g, k6, r6, n_in6 = layer_decode_bench(pkg, c2l, dev, max(2, K // 4), 2)
        B6 = c2l["B"]
        extra["layer_with_projections_decode_config2"] = {
            "tokens_per_s": round(B6 / t6, 1), "ms_per_step": round(t6 * 1e3, 4),
            "tokens_per_s_graph": round(B6 / t6g, 1), "ms_per_step_graph": round(t6g * 1e3, 4), "hidden": hidden,
            "kernels_us": {k: round(v, 2) for k, v in k6.items()},
            "in_proj_TFLOPs": round(2.0 * B6 * n_in6 * hidden / (k6["in_proj"] * 1e-6) / 1e12, 1),
            "out_proj_TFLOPs": round(2.0 * B6 * hidden * c2l["Hv"] * c2l["D"] / (k6["out_proj"] * 1e-6) / 1e12, 1),
            "hipblaslt_same_shapes_us": {k: round(v, 2) for k, v in r6.items()},
            "note": "config 2's 256 one-token rows through the mixer, eager and replayed from a HIP graph; "
                    "kernels_us from an event pair around each launch (eager: includes launch gaps at this "
                    "size): in_proj [256, 2048] x [8224, 2048]^T, q/k conv, fused decode kernel, out_proj "
                    "[256, 2048] x [2048, 2048]^T; random-init weights"}
    if 2 in configs:
        c2 = make_decode()
        t2, t2g, k2, rec_us, pass_us, copy_us, t2h, t2gh = decode_bench(pkg, c2, dev, K, W)
        state_bytes = 2 * c2["B"] * c2["Hv"] * c2["D"] * c2["D"] * 4
        gbps = state_bytes / (rec_us * 1e-6) / 1e9
        extra["decode_config2"] = {
            "ms_per_step": round(t2 * 1e3, 4), "ms_per_step_graph": round(t2g * 1e3, 4),
            "ms_per_step_hot": round(t2h * 1e3, 4), "ms_per_step_graph_hot": round(t2gh * 1e3, 4),
            "steps": "alternating the batch's 256 slots with the pool's other 256 (states cold, as in a model whose "
                     "other layers stream between two calls of one layer); _hot: the same 256 slots every step",
            "kernels_us": {k: round(v, 2) for k, v in k2.items()},
            "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                         "frac": round(gbps / HBM_PEAK_GBPS, 4),
                         "traffic": _profiled_traffic("recurrent_decode_config2"),
                         "kernel": "recurrent_kernel<128,1,8,true> (the decode step's one kernel: gates, q/k/v "
                                   "conv with its state roll, state update, gated norm)",
                         "kernel_us": round(rec_us, 2),
                         "timing": "20 back-to-back launches between one event pair, alternating two disjoint "
                                   "slot sets of the pool",
                         "algorithmic_bytes_per_launch": state_bytes,
                         "inplace_tile_ceiling": {
                             "kernel_us": round(pass_us, 2),
                             "GBps": round(state_bytes / (pass_us * 1e-6) / 1e9, 1),
                             "kernel_frac_of_ceiling": round(pass_us / rec_us, 4),
                             "what": "gdn_state_tile_pass: the same state tiles read and written back in place "
                                     "with the decode kernel's layout, launch shape and cache policy, no "
                                     "arithmetic, timed the same way"},
                         "out_of_place_tile_copy": {
                             "kernel_us": round(copy_us, 2),
                             "GBps": round(state_bytes / (copy_us * 1e-6) / 1e9, 1),
                             "inplace_over_copy": round(pass_us / copy_us, 4),
                             "what": "gdn_state_tile_copy: the same pass with each tile written to a second pool "
                                     "at the same offsets (out of place), timed the same way"}}}
        del c2
        tg, rec_g, pass_g = decode_gva_bench(pkg, dev, K, W)
        sb_g = 2 * 256 * 32 * 128 * 128 * 4
        extra["decode_gva_16_32_b256"] = {
            "ms_per_step": round(tg * 1e3, 4),
            "what": "config 2's step at Hk = 16, Hv = 32 (Qwen3.5's grouped geometry), B = 256, pool "
                    "[512, 32, 128, 128], slot sets alternating as in decode_config2: two launches (the q/k decode "
                    "conv, then the fused kernel)",
            "kernels_us": {"recurrent_decode_fused": round(rec_g, 2)},
            "roofline": {"bound": "hbm", "achieved": round(sb_g / (rec_g * 1e-6) / 1e9, 1), "peak": HBM_PEAK_GBPS,
                         "unit": "GB/s", "frac": round(sb_g / (rec_g * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4),
                         "kernel_us": round(rec_g, 2), "algorithmic_bytes_per_launch": sb_g,
                         "step_frac": round(sb_g / tg / 1e9 / HBM_PEAK_GBPS, 4),
                         "inplace_tile_ceiling_us": round(pass_g, 2),
                         "timing": "as decode_config2's roofline"}}
    if 1 in configs:
        # config 1's lengths and inputs at Qwen3.5's grouped geometry (16 key
        # heads, 32 value heads): twice the value heads' state work
        cg = make_prefill(1, None, Hk=16, Hv=32)
        tgp, kgp = prefill_bench(pkg, cg, dev, max(2, K // 4), 1)
        fg = chunk_flops(cg["N"], cg["Hv"], cg["D"])
        ug = kgp["conv_chunk_prefill"]
        extra["prefill_gva_16_32_config1_lengths"] = {
            "tokens_per_s": round(cg["N"] / tgp, 1), "ms_per_step": round(tgp * 1e3, 4),
            "kernels_us": {k: round(v, 2) for k, v in kgp.items()},
            "roofline": {"bound": "mfma", "achieved": round(fg / (ug * 1e-6) / 1e12, 2), "peak": BF16_PEAK_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(fg / (ug * 1e-6) / 1e12 / BF16_PEAK_TFLOPS, 4),
                         "kernel_us": round(ug, 2), "algorithmic_flop_per_launch": fg},
            "what": "config 1's 8 sequences (17,001 tokens, seed 1) at Hk = 16, Hv = 32, D = 128: the fused launch "
                    "pair and the gated norm, timed as config 1"}
        del cg
    if 3 in configs:
        c3 = make_prefill(4, [65536], h0_std=0.1, conv_std=1.0)
        K3 = max(2, K // 4)
        t3, k3 = prefill_bench(pkg, c3, dev, K3, 1)
        f3 = chunk_flops(c3["N"], c3["Hv"], c3["D"])
        us3 = k3["conv_chunk_prefill"]
        a3 = f3 / (us3 * 1e-6) / 1e12
        floor3 = prefill_compulsory_bytes(c3)
        extra["long_prefill_config3"] = {
            "tokens_per_s": round(c3["N"] / t3, 1), "ms_per_step": round(t3 * 1e3, 3), "steps": K3,
            "kernels_us": {k: round(v, 2) for k, v in k3.items()},
            "roofline": {"bound": "mfma", "achieved": round(a3, 2), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(a3 / BF16_PEAK_TFLOPS, 4),
                         "hbm_floor_frac": round(floor3 / (us3 * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4),
                         "compulsory_bytes_per_launch": floor3,
                         "traffic": _profiled_traffic("conv_chunk_prefill_config3"), "kernel_us": round(us3, 2),
                         "algorithmic_flop_per_launch": f3}}
        del c3
    if 4 in configs:
        c4 = make_spec()
        t4, k4 = spec_bench(pkg, c4, dev, K, W)
        rb = (1 + c4["T"]) * c4["B"] * c4["Hv"] * c4["D"] * c4["D"] * 4
        g4 = rb / (k4["recurrent_multitoken"] * 1e-6) / 1e9
        extra["spec_verify_config4"] = {
            "ms_per_step": round(t4 * 1e3, 4), "kernels_us": {k: round(v, 2) for k, v in k4.items()},
            "roofline": {"bound": "hbm", "achieved": round(g4, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                         "frac": round(g4 / HBM_PEAK_GBPS, 4),
                         "traffic": _profiled_traffic("recurrent_multitoken_config4"),
                         "kernel": "recurrent_kernel multi-token form (reads the accepted state, writes T "
                                   "intermediate states per row)",
                         "kernel_us": round(k4["recurrent_multitoken"], 2),
                         "algorithmic_bytes_per_launch": rb,
                         "timing": "median of 3 blocks of 20 back-to-back steps after a settling period; each "
                                   "verify reads the start states the previous step wrote"}}
        if "recurrent_multitoken_cold" in k4:
            gc = rb / (k4["recurrent_multitoken_cold"] * 1e-6) / 1e9
            extra["spec_verify_config4"]["roofline_cold"] = {
                "bound": "hbm", "achieved": round(gc, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                "frac": round(gc / HBM_PEAK_GBPS, 4), "kernel_us": round(k4["recurrent_multitoken_cold"], 2),
                "algorithmic_bytes_per_launch": rb,
                "timing": "two verifiers on disjoint halves of the pool's rows, alternating: a verify's start "
                          "states were written two steps (1.2 GB of traffic) before it"}
        del c4

    cpu = None
    if not args.no_cpu_baseline:
        # the host cores this process may use, at most 16: the CPU share of one
        # GPU on the box, whatever os.cpu_count() reports for the whole host
        cpu = cpu_baseline(cfg1, len(cfg1["lens"]), threads=min(CPU_SHARE, _usable_cpus()))

    out = {
        "metric": METRIC, "value": round(N1 / t1, 1), "unit": "tokens/s", "n_gpus": 1, "steps": K, "warmup": W,
        "ms_per_step": round(t1 * 1e3, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "config1: varlen GDN layer-core prefill (fused g/beta + varlen conv1d+SiLU + "
                               "chunked gated delta rule + gated RMSNorm), 8 seqs lens~U[128,4096] seed 1",
                   "tokens": N1, "lens": cfg1["lens"], "Hk": 16, "Hv": 16, "head_dim": 128, "chunk": 64,
                   "conv_channels": cfg1["C"], "state": "fp32, slot pool updated in place",
                   "precision": "bf16 in/out; fp16 matrix-core operands with fp32 accumulation; fp32 state and "
                                "triangular solve",
                   "parallelism": "single GPU"},
        "kernels_us": kernels1,
        "roofline": roofline,
        "roofline_chunk_rule": roofline_rule,
        "cpu_baseline": cpu,
    }
    out.update(extra)
    print(json.dumps(out))


if __name__ == "__main__":
    main()
