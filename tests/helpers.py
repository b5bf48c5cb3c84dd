"""Comparison metrics and seeded input builders shared by the tests."""
from __future__ import annotations

import math

import torch

BF16 = torch.bfloat16

# Tolerances of the north-star contract: bf16 outputs max-abs 2e-2 and
# mean-rel 1e-3; fp32 final states rel (Frobenius) 1e-3; bookkeeping exact.
# The max-abs bound is the literal 2e-2 on every element whose reference
# value is below 2.56 in magnitude.  From 2.56 up one bf16 rounding step
# (|y| * 2^-7 or more) exceeds 2e-2 whatever computed the value, so there the
# bound is `ulps` such steps: one for kernel outputs, four for gated-norm
# (layer) outputs, whose value chain rounds to bf16 three times after the
# core output's own rounding.  Elements beyond one step (or 2e-2) must also
# be rarer than 1e-4, so a systematic error cannot hide in the budget.
OUT_MAX_ABS = 2e-2
OUT_MEAN_REL = 1e-3
STATE_REL = 1e-3
BF16_ULP_REL = 2.0 ** -7
LITERAL_BELOW = OUT_MAX_ABS / BF16_ULP_REL   # 2.56
FAR_FRACTION = 1e-4


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


def elem_bound(b, ulps: int = 1):
    """Per-element bound: 2e-2 where |b| < 2.56, else `ulps` bf16 steps of b."""
    b = b.float().cpu().abs()
    return torch.where(b < LITERAL_BELOW, torch.full_like(b, OUT_MAX_ABS), b * (ulps * BF16_ULP_REL))


def excess_abs(a, b, ulps: int = 1) -> float:
    """Largest |a - b| beyond the per-element bound (elem_bound)."""
    a, b = a.float().cpu(), b.float().cpu()
    if not a.numel():
        return 0.0
    return ((a - b).abs() - elem_bound(b, ulps)).max().item()


def far_fraction(a, b) -> float:
    """Fraction of elements beyond max(2e-2, one bf16 step of b)."""
    a, b = a.float().cpu(), b.float().cpu()
    if not a.numel():
        return 0.0
    return ((a - b).abs() > torch.clamp(b.abs() * BF16_ULP_REL, min=OUT_MAX_ABS)).float().mean().item()


def assert_out(a, b, tag="", ulps: int = 1):
    ma, mr, ex = max_abs(a, b), mean_rel(a, b), excess_abs(a, b, ulps)
    far = far_fraction(a, b)
    assert ex <= 0 and mr <= OUT_MEAN_REL and far < FAR_FRACTION, (
        f"{tag}: max-abs {ma:.3e} (excess over bound {ex:.3e}), mean-rel {mr:.3e}, "
        f"{far:.2e} of elements beyond one step")


def bf16_step(b):
    """Spacing of bf16 values at |b| (2^(e - 7) for |b| in [2^e, 2^(e+1)))."""
    b = b.float().abs().clamp(min=2.0 ** -126)
    return torch.exp2(torch.floor(torch.log2(b)) - 7)


CASCADE_FRACTION = 1e-6


def assert_layer_out(a, b, tag="", ms_rows=None):
    """Gated-norm (layer) outputs at full size.  The bar of assert_out with
    four steps above |b| = 2.56, except that at most CASCADE_FRACTION of the
    elements (and none below a million elements) may instead be a rounding
    cascade: one bf16 flip of the core output carried through the norm's
    three bf16 roundings (n, w n, y), at most four bf16 steps of the
    reference value.  At BASELINE configs 1 and 3 the core output's rows have
    mean squares near eps (median 7e-6 at config 1), so the norm multiplies
    them by ~350 and a single flip in a core-output element, or a last-bit
    difference in the norm's own fp32 arithmetic, can move an output by two
    or three steps; a CPU simulation of the kernels' error level (1e-5 of the
    typical core-output magnitude) gives ~14 such elements in 35M at config
    1, and none only at 1e-6.  Each allowed element is printed with its
    (row) index and, given ms_rows, its row's mean square.  (Outputs whose
    core outputs differ upstream: assert_layer_out_propagated.)"""
    af, bf = a.float().cpu(), b.float().cpu()
    ma, mr, far = max_abs(af, bf), mean_rel(af, bf), far_fraction(af, bf)
    d = (af - bf).abs()
    over = d > elem_bound(bf, 4)
    n_over = int(over.sum())
    allowed = int(CASCADE_FRACTION * af.numel())
    msg = (f"{tag}: max-abs {ma:.3e}, mean-rel {mr:.3e}, {far:.2e} of elements beyond one step, "
           f"{n_over} elements beyond the per-element bound (cascades allowed: {allowed})")
    if n_over:
        idx = over.nonzero()
        steps = (d[over] / bf16_step(bf[over])).tolist()
        order = sorted(range(len(steps)), key=lambda j: -steps[j])
        lines = []
        for ix in [idx[j].tolist() for j in order[:40]]:
            t = tuple(ix)
            row = f", row mean square {ms_rows[t[:-1]].item():.2e}" if ms_rows is not None else ""
            lines.append(f"    {t}: ref {bf[t].item():.6g} got {af[t].item():.6g}{row}")
        print(msg + "\n" + "\n".join(lines), flush=True)
    assert mr <= OUT_MEAN_REL and far < FAR_FRACTION, msg
    assert n_over <= allowed, msg
    if n_over:
        assert bool((d[over] <= 4 * bf16_step(bf[over]) + 1e-12).all()), msg + " (a cascade beyond four steps)"


def norm_propagation_bound(o_a, o_b, z, w, eps=1e-6):
    """Per-element bound on how far the gated norm (qwen3_5.py:546-554:
    y = w * x / sqrt(mean(x^2) + eps) * silu(z)) moves apart when its input
    rows differ by o_a - o_b: first order in the difference, the element's own
    term |w silu(z)| r |do| plus the row-scale term |w silu(z)| |o| r
    sum(|o| |do|) / (D (ms + eps)), r = 1 / sqrt(ms + eps), with a factor 2 for
    the second order.  Rows whose mean square is near or below eps have r up
    to 1 / sqrt(eps) = 1000, so a difference far below one step of their own
    values can be several steps of the output."""
    oa, ob = o_a.float().cpu(), o_b.float().cpu()
    do = (oa - ob).abs()
    ms = ob.pow(2).mean(-1, keepdim=True)
    r = torch.rsqrt(ms + eps)
    zf = z.float().cpu()
    gate = (w.float().cpu() * zf * torch.sigmoid(zf)).abs()
    row = (ob.abs() * do).mean(-1, keepdim=True) / (ms + eps)
    return 2.0 * gate * r * (do + ob.abs() * row)


def assert_layer_out_propagated(a, b, o_a, o_b, z, w, tag=""):
    """End-to-end gated-norm outputs whose core outputs differ upstream (o_a
    for a, o_b for b): every element within assert_layer_out's bar widened by
    norm_propagation_bound(o_a, o_b, ...), with no row left out; mean-rel and
    the one-step fraction as assert_layer_out.  (The norm kernel itself is held
    to assert_layer_out on identical inputs.)"""
    af, bf = a.float().cpu(), b.float().cpu()
    ma, mr, far = max_abs(af, bf), mean_rel(af, bf), far_fraction(af, bf)
    d = (af - bf).abs()
    prop = norm_propagation_bound(o_a, o_b, z, w)
    bound = elem_bound(bf, 4) + prop
    ratio = d / bound
    n_prop = int(((d > elem_bound(bf, 4)) & (d <= bound)).sum())
    n_over = int((d > bound).sum())
    allowed = int(CASCADE_FRACTION * af.numel())
    msg = (f"{tag}: max-abs {ma:.3e}, mean-rel {mr:.3e}, {far:.2e} of elements beyond one step; "
           f"{n_prop} elements beyond four steps within the norm's propagation of the core-output difference, "
           f"{n_over} beyond that (cascades allowed: {allowed}); worst |diff| / bound {float(ratio.max()):.3f}")
    print(msg, flush=True)
    assert mr <= OUT_MEAN_REL and far < FAR_FRACTION, msg
    assert n_over <= allowed, msg
    if n_over:
        over = d > bound
        assert bool((d[over] <= 4 * bf16_step(bf[over]) + prop[over] + 1e-12).all()), msg


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
