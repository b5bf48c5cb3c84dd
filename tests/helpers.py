"""Comparison metrics and seeded input builders shared by the tests."""
from __future__ import annotations

import math

import torch

BF16 = torch.bfloat16

# Tolerances of the north-star contract: bf16 outputs max-abs 2e-2 and
# mean-rel 1e-3; fp32 final states rel (Frobenius) 1e-3; bookkeeping exact.
# The max-abs bound is applied per element as max(2e-2, `ulps` bf16 ulps of
# the reference value): for |y| >= 2.56 a single rounding flip of a bf16
# output already exceeds 2e-2, whatever computed it.  Kernel outputs use one
# ulp.  Gated-norm (layer) outputs use four: one from a flip of the norm's
# bf16 input plus the norm's own three roundings (n, w*n, y); such elements
# must also stay rare (fraction beyond one ulp < 1e-3), so a systematic error
# cannot hide in the budget.  The chunk kernel's single-pass fp16 operands
# leave ~3e-4 relative error in the core output before its bf16 rounding, so
# a few elements in 1e4 of the gated-norm output land one ulp further out.
OUT_MAX_ABS = 2e-2
OUT_MEAN_REL = 1e-3
STATE_REL = 1e-3
BF16_ULP_REL = 2.0 ** -7


def max_abs(a, b) -> float:
    return (a.float().cpu() - b.float().cpu()).abs().max().item() if a.numel() else 0.0


def mean_rel(a, b) -> float:
    a, b = a.float().cpu(), b.float().cpu()
    den = b.abs().mean().item()
    return (a - b).abs().mean().item() / den if den > 0 else (a - b).abs().mean().item()


def state_rel(a, b) -> float:
    a, b = a.double().cpu(), b.double().cpu()
    den = b.norm().item()
    return (a - b).norm().item() / den if den > 0 else (a - b).norm().item()


def excess_abs(a, b, ulps: int = 1) -> float:
    """Largest |a - b| beyond the per-element bound max(2e-2, ulps * bf16 ulp of b)."""
    a, b = a.float().cpu(), b.float().cpu()
    if not a.numel():
        return 0.0
    bound = torch.clamp(b.abs() * (ulps * BF16_ULP_REL), min=OUT_MAX_ABS)
    return ((a - b).abs() - bound).max().item()


def assert_out(a, b, tag="", ulps: int = 1):
    ma, mr, ex = max_abs(a, b), mean_rel(a, b), excess_abs(a, b, ulps)
    assert ex <= 0 and mr <= OUT_MEAN_REL, f"{tag}: max-abs {ma:.3e} (excess over bound {ex:.3e}), mean-rel {mr:.3e}"
    if ulps > 1:
        af, bf = a.float().cpu(), b.float().cpu()
        far = ((af - bf).abs() > torch.clamp(bf.abs() * BF16_ULP_REL, min=OUT_MAX_ABS)).float().mean().item()
        assert far < 1e-3, f"{tag}: {far:.2e} of elements beyond one ulp"


def assert_state(a, b, tag=""):
    r = state_rel(a, b)
    assert r <= STATE_REL, f"{tag}: state rel {r:.3e}"


def gates(gen, n, Hv):
    """a, b ~ N(0,1) bf16; A_log ~ U(0, ln 16), dt_bias ~ U(-1, 1) as bf16 params."""
    a = torch.randn(n, Hv, generator=gen).to(BF16)
    b = torch.randn(n, Hv, generator=gen).to(BF16)
    A_log = (torch.rand(Hv, generator=gen) * math.log(16)).to(BF16)
    dt_bias = (torch.rand(Hv, generator=gen) * 2 - 1).to(BF16)
    return a, b, A_log, dt_bias


def rule_inputs(gen, N, Hk, Hv, D, slow_decay=False):
    """Post-conv q, k, v (bf16, ~N(0,1)), g (fp32) and beta (bf16)."""
    from oracle import gdn_ref

    q = torch.randn(N, Hk, D, generator=gen).to(BF16)
    k = torch.randn(N, Hk, D, generator=gen).to(BF16)
    v = torch.randn(N, Hv, D, generator=gen).to(BF16)
    a, b, A_log, dt_bias = gates(gen, N, Hv)
    g, beta = gdn_ref.g_beta(b, a, A_log, dt_bias)
    if slow_decay:
        g = g * 0.02
    return q, k, v, g, beta


def cu_of(lens):
    cu = [0]
    for t in lens:
        cu.append(cu[-1] + t)
    return cu
