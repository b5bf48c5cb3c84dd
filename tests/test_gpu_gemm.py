"""GPU parity of the projection GEMM (gdn_gemm_bf16): C = A B^T with bf16
operands and fp32 accumulation against an fp32 CPU matmul of the same bf16
values, on the GDN layer's projection shapes (in_proj over the concatenated
qkv / z / b / a weights, out_proj) and ragged edges; the fused gate epilogue
against fused_g_beta on the b / a columns."""
import math

import pytest
import torch

from helpers import BF16, bf16_step

pytestmark = pytest.mark.gpu


def _check(c, ref, scale, tag):
    """Each element within one bf16 step of the fp32 reference plus the fp32
    summation-order slack 2^-16 (|A| |B|^T) (the reference and the kernel add
    the K products in different orders; near-zero results carry that absolute
    error), and elements that are not the rounded reference rare."""
    c, ref = c.float().cpu(), ref.float()
    d = (c - ref).abs()
    bound = bf16_step(ref) + scale * 2.0 ** -16
    assert bool((d <= bound).all()), f"{tag}: max |diff| / bound {float((d / bound).max()):.2f}"
    flips = (c != ref.to(BF16).float()).float().mean().item()
    assert flips < 2e-2, f"{tag}: {flips:.2e} of elements are not the rounded reference"


def _ref(a, w):
    return a.float() @ w.float().t(), a.float().abs() @ w.float().abs().t()


# The tile is 256 x 256, or 192 x 256 when ceil(tiles / 256 CUs) x rows is
# smaller with it, or 64 x 128 when fewer than 128 tiles of 256 x 256 would
# run, or 64 x 64 when fewer than 128 of 64 x 128 would.  The 64-row tiles run
# the deeper load pipeline (gemm_tn_deep_kernel) when K >= 1024.  64 x 64:
# (256, 256), (300, 200); deep: (1, 8224), (17, 2048), (256, 2048) (the decode
# out_proj), (100, 2000, 1088) (17 steps: a partial last round of stages);
# 64 x 128: (1000, 2080), (4111, 333); deep: (256, 8224) (the decode in_proj),
# (300, 8224, 1024) (16 steps, ragged rows);
# 192 x 256: (17000, 2048) = 712 tiles of 192 rows (3 waves) against 536 of 256
# (3 waves); 256 x 256: (8190, 2047) is exactly 256 tiles of 256 rows (344 of
# 192) and (17000, 8224) ties at 9 waves.
@pytest.mark.parametrize("M,N,K", [(256, 256, 64), (300, 200, 128), (1, 8224, 2048), (17, 2048, 2048), (256, 2048, 2048),
                                   (100, 2000, 1088), (1000, 2080, 512), (4111, 333, 192), (256, 8224, 2048),
                                   (300, 8224, 1024), (17000, 2048, 256), (8190, 2047, 128), (17000, 8224, 128)])
def test_gemm_against_fp32_matmul(pkg, dev, M, N, K):
    gen = torch.Generator().manual_seed(M * 7 + N)
    a = torch.randn(M, K, generator=gen).to(BF16)
    w = (torch.randn(N, K, generator=gen) / math.sqrt(K)).to(BF16)
    ref, sc = _ref(a, w)
    c = pkg.ops.linear(a.to(dev), w.to(dev))
    _check(c, ref, sc, f"gemm {M}x{N}x{K}")


@pytest.mark.parametrize("pad,off", [(40, 8), (41, 3)])
def test_gemm_strided_operands_and_out(pkg, dev, pad, off):
    """Row strides larger than K (views of wider buffers) and an output view;
    pad 41 / offset 3 gives an output row stride that is not a multiple of 4
    and rows at 2-byte alignment (element-by-element stores)."""
    gen = torch.Generator().manual_seed(5)
    M, N, K = 333, 264, 256
    abuf = torch.randn(M, K + 64, generator=gen).to(BF16)
    wbuf = (torch.randn(N, K + 128, generator=gen) / 16).to(BF16)
    a, w = abuf[:, 32:32 + K], wbuf[:, :K]
    out = torch.zeros(M, N + pad, dtype=BF16, device=dev)
    pkg.ops.linear(abuf.to(dev)[:, 32:32 + K], wbuf.to(dev)[:, :K], out=out[:, off:off + N])
    _check(out[:, off:off + N], *_ref(a, w), "strided gemm")
    assert torch.equal(out[:, :off].cpu(), torch.zeros(M, off, dtype=BF16))
    assert torch.equal(out[:, off + N:].cpu(), torch.zeros(M, pad - off, dtype=BF16))


@pytest.mark.parametrize("M", [100, 777, 1790])
def test_in_proj_with_gate_epilogue(pkg, dev, M):
    """The layer's in_proj over [W_qkv; W_z; W_b; W_a] (config 1 widths, a
    2048 hidden size): the projections, and g / beta from the b and a columns
    equal to fused_g_beta on them.  M = 100 runs 64 x 128 tiles, M = 777
    192 x 256 tiles, M = 1790 (231 tiles of 256 rows, 330 of 192) 256 x 256
    tiles."""
    gen = torch.Generator().manual_seed(6)
    Hk = Hv = 16
    D, hidden = 128, 2048
    C = 2 * Hk * D + Hv * D
    N = C + Hv * D + 2 * Hv
    x = torch.randn(M, hidden, generator=gen).to(BF16)
    w = (torch.randn(N, hidden, generator=gen) / math.sqrt(hidden)).to(BF16)
    A_log = (torch.rand(Hv, generator=gen) * math.log(16)).to(BF16)
    dt_bias = (torch.rand(Hv, generator=gen) * 2 - 1).to(BF16)
    y, g, beta = pkg.ops.linear(x.to(dev), w.to(dev), gates={"gate_col": C + Hv * D, "A_log": A_log.to(dev),
                                                             "dt_bias": dt_bias.to(dev)})
    _check(y, *_ref(x, w), "in_proj")
    b = y[:, C + Hv * D:C + Hv * D + Hv].contiguous()
    a = y[:, C + Hv * D + Hv:].contiguous()
    g2, beta2 = pkg.ops.fused_g_beta(b, a, A_log.to(dev), dt_bias.to(dev), None)
    torch.cuda.synchronize()
    assert torch.equal(g, g2) and torch.equal(beta.view(torch.int16), beta2.view(torch.int16))


def _layouts(C, V, Hv):
    # (the layer's three- and four-part in_proj; boundaries off the 32-column
    # grid, where one 32-column block's pieces go to two parts)
    return {"3": [C, V, 2 * Hv], "4": [C, V, Hv, Hv], "16": [48, C - 48, V + 16, 2 * Hv - 16]}


@pytest.mark.parametrize("layout", ["3", "4", "16"])
@pytest.mark.parametrize("with_gates", [False, True])
@pytest.mark.parametrize("M", [64, 100, 777, 1790])
def test_in_proj_column_parts_equal_one_output(pkg, dev, M, with_gates, layout):
    """gdn_gemm_bf16_cols (the layer's in_proj into separate qkv, z, b and a
    tensors): every part bit-equal to the same columns of the one-output GEMM,
    and the gate outputs too, for each tile shape (M = 64: 64 x 64 tiles with
    the deeper pipeline, 100: 64 x 128, 777: 192 x 256, 1790: 256 x 256)."""
    gen = torch.Generator().manual_seed(7)
    Hk, Hv = 16, 32
    D, hidden = 128, 2048
    C = 2 * Hk * D + Hv * D
    V = Hv * D
    N = C + V + 2 * Hv
    x = torch.randn(M, hidden, generator=gen).to(BF16).to(dev)
    w = (torch.randn(N, hidden, generator=gen) / math.sqrt(hidden)).to(BF16).to(dev)
    A_log = (torch.rand(Hv, generator=gen) * math.log(16)).to(BF16).to(dev)
    dt_bias = (torch.rand(Hv, generator=gen) * 2 - 1).to(BF16).to(dev)
    gates = {"gate_col": C + V, "A_log": A_log, "dt_bias": dt_bias} if with_gates else None
    widths = _layouts(C, V, Hv)[layout]
    one = pkg.ops.linear(x, w, gates=gates)
    parts = pkg.ops.linear_cols(x, w, widths, gates=gates)
    torch.cuda.synchronize()
    if with_gates:
        (y, g, beta), (ps, g2, beta2) = one, parts
        assert torch.equal(g, g2) and torch.equal(beta.view(torch.int16), beta2.view(torch.int16))
    else:
        y, ps = one, parts
    c0 = 0
    for p, wd in zip(ps, widths):
        assert p.is_contiguous() and p.shape == (M, wd)
        assert torch.equal(p.view(torch.int16), y[:, c0:c0 + wd].contiguous().view(torch.int16)), (c0, wd)
        c0 += wd


def test_column_parts_rejected_shapes(pkg, dev):
    """Part boundaries off the 16-column grid, out of order, a last boundary
    other than N, or more than four parts are rejected before any launch.
    Real (small) buffers, each part's wide enough for every column, so even a
    launch that the checks had wrongly let through would stay in bounds."""
    import ctypes
    lib = pkg._lib.load()
    _lib = pkg._lib
    M, N, K = 4, 96, 64
    a = torch.zeros(M, K, dtype=BF16, device=dev)
    b = torch.zeros(N, K, dtype=BF16, device=dev)
    outs = [torch.zeros(M, 128, dtype=BF16, device=dev) for _ in range(5)]
    c = (ctypes.c_void_p * 5)(*[o.data_ptr() for o in outs])
    ld = (ctypes.c_int64 * 5)(*([128] * 5))
    stream = torch.cuda.current_stream(dev).cuda_stream

    def call(ends):
        e = (ctypes.c_int * len(ends))(*ends)
        return lib.gdn_gemm_bf16_cols(a.data_ptr(), K, b.data_ptr(), K, M, N, K, len(ends), c, ld, e, None, None,
                                      None, None, 0, 0, 0, stream)

    for ends in ((40, 96), (64, 100), (96, 64), (64, 64), (16, 32, 48, 64, 96), (8, 48, 64, 96)):
        assert call(ends) == _lib.GDN_ERR_INVALID_ARG, ends
    for ends in ((64, 96), (16, 48, 64, 96)):
        assert call(ends) == _lib.GDN_OK, ends
    torch.cuda.synchronize()
