"""The HIP path against the upstream golden vectors directly (not only through
the oracle).

tests/golden/config0.npz holds BASELINE config 0 run through the upstream
transformers torch functions the reference ports (causal_conv1d_fn,
torch_chunk_gated_delta_rule, Qwen3_5RMSNormGated) in fp32; edge.npz holds the
bf16 gated norm and a single-token conv update.  The kernels take bf16
inputs, so the fp32 fixture inputs are cast to bf16 first.  Each HIP output
is then held to two bars:
  * against the oracle run on the same bf16 inputs: the parity bar of the
    other tests (tests/helpers.py);
  * against the fixture: within the distance that the bf16 input cast alone
    puts between the oracle and the fixture, plus the parity bar.  For the
    conv output the cast's effect is bounded per element in closed form.
"""
from pathlib import Path

import numpy as np
import pytest
import torch

from helpers import (BF16, OUT_MAX_ABS, OUT_MEAN_REL, STATE_REL, assert_out, assert_state, max_abs, mean_rel,
                     state_rel)
from oracle import gdn_ref

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"


def _fix(name):
    return {k: torch.from_numpy(v) for k, v in np.load(GOLDEN / name).items()}


def _near_fixture(hip, orc, fix, tag, state=False):
    """hip is no further from the fixture than the oracle on the same bf16
    inputs is, plus the parity bar."""
    if state:
        d_h, d_o = state_rel(hip, fix), state_rel(orc, fix)
        assert d_h <= d_o + STATE_REL, f"{tag}: state rel to fixture {d_h:.3e} vs oracle's {d_o:.3e}"
        return
    mr_h, mr_o = mean_rel(hip, fix), mean_rel(orc, fix)
    ma_h, ma_o = max_abs(hip, fix), max_abs(orc, fix)
    assert mr_h <= mr_o + OUT_MEAN_REL, f"{tag}: mean-rel to fixture {mr_h:.3e} vs oracle's {mr_o:.3e}"
    assert ma_h <= ma_o + OUT_MAX_ABS, f"{tag}: max-abs to fixture {ma_h:.3e} vs oracle's {ma_o:.3e}"


def test_config0_through_hip_path(pkg, dev):
    """BASELINE config 0 (T=256, H=4, d=64, one sequence, zero states)
    through the gate, varlen conv, chunk and gated-norm kernels, and through
    the fused prefill call, against the oracle and the upstream fixture."""
    f = _fix("config0.npz")
    T, C = f["x"].shape
    H, D = 4, 64
    kd = H * D
    x, w = f["x"].to(BF16), f["w"].to(BF16)
    a, b = f["a"].to(BF16), f["b"].to(BF16)
    A_log, dt_bias = f["A_log"].to(BF16), f["dt_bias"].to(BF16)
    z = f["z"].to(BF16)                     # [32, H, D]: the fixture normalises the first 32 tokens
    norm_w = f["norm_w"].to(BF16)
    lens = [T]

    # ---- HIP, separate kernels
    g_h, beta_h = pkg.ops.fused_g_beta(b.to(dev), a.to(dev), A_log.to(dev), dt_bias.to(dev), None)
    cstate = torch.zeros(1, C, 3, dtype=BF16, device=dev)
    lens32 = torch.tensor(lens, dtype=torch.int32, device=dev)
    starts = torch.zeros(1, dtype=torch.int32, device=dev)
    q_h, k_h, v_h = pkg.ops.causal_conv_silu_varlen_parts(x.to(dev), cstate, w.to(dev), lens32, starts, kd)
    cu = torch.tensor([0, T], dtype=torch.int64, device=dev)
    o_h, s_h = pkg.ops.chunk_gated_delta_rule_varlen(q_h.view(T, H, D), k_h.view(T, H, D), v_h.view(T, H, D),
                                                     g_h, beta_h, cu, None)
    y_h = pkg.ops.rms_norm_gated(o_h[:32], z.to(dev), norm_w.to(dev), 1e-6)
    # ---- HIP, the fused prefill call (the layer's product path): bit-equal
    cpool = torch.zeros(1, C, 3, dtype=BF16, device=dev)
    spool = torch.zeros(1, H, D, D, device=dev)
    o_f = pkg.ops.conv_chunk_prefill_varlen(x.to(dev), cpool, w.to(dev), b.to(dev), a.to(dev), A_log.to(dev),
                                            dt_bias.to(dev), cu, spool, None, H, H, D)
    torch.cuda.synchronize()
    assert torch.equal(o_f.cpu().view(torch.int16), o_h.cpu().view(torch.int16)), "fused == separate calls"
    assert torch.equal(spool.cpu(), s_h.cpu()), "fused final state == separate calls"
    assert torch.equal(cpool.cpu(), cstate.cpu()), "fused conv-state roll == separate calls"
    y_conv = torch.cat([q_h, k_h, v_h], 1).cpu()

    # ---- oracle on the same bf16 inputs: the parity bar
    g_o, beta_o = gdn_ref.g_beta(b, a, A_log, dt_bias)
    yc_o, cst_o = gdn_ref.conv_varlen(x, torch.zeros(1, C, 3, dtype=BF16), w, lens)
    o_o, s_o = gdn_ref.chunk_varlen(yc_o[:, :kd].reshape(T, H, D), yc_o[:, kd:2 * kd].reshape(T, H, D),
                                    yc_o[:, 2 * kd:].reshape(T, H, D), g_o, beta_o.float(), [0, T], None)
    yn_o = gdn_ref.rms_norm_gated(o_o[:32].to(BF16), z, norm_w)
    torch.testing.assert_close(g_h.cpu(), g_o, rtol=2e-6, atol=1e-6)
    assert torch.equal(beta_h.cpu().view(torch.int16), beta_o.view(torch.int16))
    assert_out(y_conv, yc_o, "config 0 conv")
    assert torch.equal(cstate.cpu(), cst_o), "config 0 conv-state roll"
    assert_out(o_h.cpu(), o_o.to(BF16), "config 0 chunk output")
    assert_state(s_h.cpu()[0], s_o[0], "config 0 final state")
    assert_out(y_h.cpu(), yn_o, "config 0 gated norm", ulps=4)

    # ---- against the upstream fixture
    # conv: |y(bf16 inputs) - y(fp32 inputs)| <= L * sum_i |w_i dx_i| + |x_i dw_i| + |dx_i dw_i| plus the
    # bf16 output rounding (half a step, 2^-9 |y|, relative), with L = max |silu'| < 1.1
    xf, wf = f["x"], f["w"]
    dx, dw = (xf - x.float()).abs(), (wf - w.float()).abs()
    win = lambda t: torch.cat([torch.zeros(3, C), t], 0).unfold(0, 4, 1)   # [T, C, 4] causal windows
    bound = 1.1 * (win(dx) * wf.abs() + win(xf.abs()) * dw + win(dx) * dw).sum(-1) \
        + f["conv_y"].abs() * (2.0 ** -8 + 1e-6) + 1e-5          # + fp32 arithmetic slack
    excess = ((y_conv.float() - f["conv_y"]).abs() - bound).max().item()
    assert excess <= 0, f"config 0 conv beyond the input-cast bound by {excess:.3e}"
    _near_fixture(g_h.cpu(), g_o, f["g"], "config 0 g")
    _near_fixture(beta_h.cpu().float(), beta_o.float(), f["beta"], "config 0 beta")
    _near_fixture(o_h.cpu().float(), o_o, f["o_chunk"], "config 0 chunk output")
    _near_fixture(s_h.cpu()[0], s_o[0], f["state_chunk"], "config 0 final state", state=True)
    _near_fixture(y_h.cpu().float(), yn_o.float(), f["y_norm"], "config 0 gated norm")
    # the upstream token-by-token form of the same rule ends in the same state
    _near_fixture(s_h.cpu()[0], s_o[0], f["state_rec"], "config 0 state vs recurrent form", state=True)
    _near_fixture(o_h.cpu().float()[-64:], o_o[-64:], f["o_rec_tail"], "config 0 output tail vs recurrent form")


def test_gated_norm_bits_vs_upstream_fixture(pkg, dev):
    """edge.npz: the upstream Qwen3_5RMSNormGated module on bf16 inputs
    (its rounding order).  Inputs need no cast; almost every output bit
    matches."""
    f = np.load(GOLDEN / "edge.npz")
    nx = torch.from_numpy(f["nx"]).view(BF16)
    nz = torch.from_numpy(f["nz"]).view(BF16)
    nw = torch.from_numpy(f["nw"]).view(BF16)
    ny = torch.from_numpy(f["ny"]).view(BF16)
    y = pkg.ops.rms_norm_gated(nx.to(dev), nz.to(dev), nw.to(dev), 1e-6).cpu()
    assert_out(y, ny, "gated norm vs upstream module")
    diff = (y.view(torch.int16) != ny.view(torch.int16)).float().mean().item()
    assert diff < 1e-3, f"{diff:.2e} of elements differ in bits from the upstream module"


def test_conv_update_vs_upstream_fixture(pkg, dev):
    """edge.npz: upstream causal_conv1d_update, one token against a non-zero
    state, fp32.  Through gdn_conv_decode on bf16-cast inputs: the state roll
    is bit-exact on the cast values, the output within the cast bound."""
    f = _fix("edge.npz")
    cx, cst, cw = f["cx"].to(BF16), f["cstate"].to(BF16), f["cw"].to(BF16)
    n, C = cx.shape
    pool = cst.clone().to(dev)
    y = pkg.ops.conv_decode_step(cx.to(dev), pool, torch.arange(n, device=dev), cw.to(dev)).cpu()
    roll = torch.cat([cst[:, :, 1:], cx.unsqueeze(-1)], -1)
    assert torch.equal(pool.cpu().view(torch.int16), roll.view(torch.int16)), "conv update roll"
    assert torch.equal(roll.float(), f["cstate_after"].to(BF16).float()), "roll == the fixture's state, cast"
    y_o, _ = gdn_ref.conv_decode(cx, cst.clone(), list(range(n)), cw)
    assert_out(y, y_o, "conv update vs oracle")
    win = torch.cat([f["cstate"], f["cx"].unsqueeze(-1)], -1)            # [n, C, 4]
    wwin = torch.cat([cst.float(), cx.float().unsqueeze(-1)], -1)
    dx, dw = (win - wwin).abs(), (f["cw"] - cw.float()).abs()
    bound = 1.1 * (dx * f["cw"].abs() + win.abs() * dw + dx * dw).sum(-1) + f["cy"].abs() * (2.0 ** -8 + 1e-6) + 1e-5
    excess = ((y.float() - f["cy"]).abs() - bound).max().item()
    assert excess <= 0, f"conv update beyond the input-cast bound by {excess:.3e}"
