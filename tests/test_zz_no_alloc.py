"""The allocation-free prefill entry point (gdn_conv_chunk_prefill_noalloc)
against the workspace entry point (gdn_conv_chunk_prefill), bit for bit, on
two calls in a row (the second smaller, so it runs on what the first left in
the shared scratch array), both through the C ABI: calls that fit the array,
calls that run as sequence groups, and a sequence that
runs as token ranges; and a larger call without host offsets, refused."""
import pytest
import torch

import bench

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16


def _inputs(dev, lens, Hk, Hv, D, seed):
    cfg = bench.make_prefill(seed, lens, Hk=Hk, Hv=Hv, D=D, h0_std=0.1, conv_std=1.0)
    n = len(lens)
    slots = n + 3
    gen = torch.Generator().manual_seed(seed + 100)
    pool_s = torch.randn(slots, Hv, D, D, generator=gen) * 0.1
    pool_c = torch.randn(slots, cfg["C"], 3, generator=gen).to(BF16)
    ids = torch.randperm(slots, generator=gen)[:n]
    fresh = torch.tensor([r % 3 == 1 for r in range(n)], dtype=torch.uint8)
    cu = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int64)
    d = {k: cfg[k].to(dev) for k in ("x", "a", "b", "A_log", "dt_bias")}
    d["w"] = cfg["conv_w"].to(dev).contiguous()
    return d, pool_s, pool_c, ids.to(dev), fresh.to(dev), cu


def _both(pkg, dev, lens, Hk, Hv, D, seed, segments=0):
    d, pool_s, pool_c, ids, fresh, cu = _inputs(dev, lens, Hk, Hv, D, seed)
    N = sum(lens)
    s1, c1 = pool_s.to(dev), pool_c.to(dev)
    o1 = pkg.ops.conv_chunk_prefill_varlen(d["x"], c1, d["w"], d["b"], d["a"], d["A_log"], d["dt_bias"], cu.to(dev),
                                           s1, ids, Hk, Hv, D, fresh=fresh, cu_seqlens_cpu=cu, max_segments=segments)
    s2, c2 = pool_s.to(dev), pool_c.to(dev)
    o2 = torch.empty(N, Hv, D, dtype=BF16, device=dev)
    pkg.ops.conv_chunk_prefill_varlen_noalloc(d["x"], c2, d["w"], d["b"], d["a"], d["A_log"], d["dt_bias"],
                                              cu.to(dev), s2, ids, Hk, Hv, D, o2, fresh=fresh, cu_seqlens_cpu=cu,
                                              max_segments=segments)
    torch.cuda.synchronize()
    assert torch.equal(o2.view(torch.int16), o1.view(torch.int16)), "outputs differ"
    assert torch.equal(s2, s1), "state pools differ"
    assert torch.equal(c2.view(torch.int16), c1.view(torch.int16)), "conv pools differ"


def test_noalloc_equals_workspace_entry_two_calls(pkg, dev):
    print("no-alloc prefill: 8 seqs, 16/16 heads, then a smaller call", flush=True)
    _both(pkg, dev, [700, 1, 0, 333, 1500, 64, 900, 129], 16, 16, 128, 7)
    _both(pkg, dev, [200, 65, 3], 16, 16, 128, 8)


def test_noalloc_segmented_and_gva(pkg, dev):
    print("no-alloc prefill: one long segmented sequence, then GVA at D = 64", flush=True)
    _both(pkg, dev, [2048], 4, 4, 128, 9, segments=4)
    _both(pkg, dev, [300, 77], 2, 4, 64, 10)


def test_noalloc_pieces_config1_then_smaller(pkg, dev):
    print("no-alloc prefill: config 1 (241 MB of records: sequence groups), then a call that fits", flush=True)
    lens = bench.make_prefill(1, None)["lens"]
    lib = pkg._lib.load()
    assert lib.gdn_conv_chunk_prefill_workspace_size(sum(lens), len(lens), 16, 128) > pkg._lib.NOALLOC_SCRATCH_BYTES
    _both(pkg, dev, lens, 16, 16, 128, 11, segments=1)
    _both(pkg, dev, [900, 64, 1], 16, 16, 128, 12, segments=1)


def test_noalloc_pieces_long_sequence_in_ranges(pkg, dev):
    print("no-alloc prefill: a 12,000-token sequence beside a short one (token ranges), then GVA, then D = 64",
          flush=True)
    lib = pkg._lib.load()
    for lens, Hk, Hv, D, seed in (([300, 12000], 16, 16, 128, 13), ([20000, 70], 4, 8, 128, 14),
                                  ([7000], 16, 32, 64, 15)):
        assert lib.gdn_conv_chunk_prefill_workspace_size(sum(lens), len(lens), Hv, D) > \
            pkg._lib.NOALLOC_SCRATCH_BYTES
        _both(pkg, dev, lens, Hk, Hv, D, seed, segments=1)


def test_noalloc_rejects_calls_beyond_the_array(pkg, dev):
    """A call whose records would exceed the array, without host offsets to
    plan pieces from, fails before any launch."""
    Hk = Hv = 16
    D = 128
    lib = pkg._lib.load()
    need = lib.gdn_conv_chunk_prefill_workspace_size(40000, 8, Hv, D)
    assert need > pkg._lib.NOALLOC_SCRATCH_BYTES
    # every pointer NULL: the size check comes first; were it moved behind the
    # launch path, the NULL operands would be rejected there instead
    st = lib.gdn_conv_chunk_prefill_noalloc(None, 6144, None, 18432, 3, None, None, None, None,
                                            None, 0, None, None, None, None, Hv * D * D, None, None, 0,
                                            8, 40000, Hk, Hv, D, 1.0, 1, None, None)
    assert st == pkg._lib.GDN_ERR_SCRATCH
