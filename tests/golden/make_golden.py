"""Writes the golden vectors that pin the CPU oracle (tests/test_oracle.py).

The reference's GDN torch path is a port of the upstream transformers
functions (nanovllm/models/qwen3_5.py:18-19, :154, :619); this script runs
those upstream functions from the installed transformers package
(models/qwen3_5/modeling_qwen3_5.py: causal_conv1d_fn / causal_conv1d_update,
torch_chunk_gated_delta_rule, torch_recurrent_gated_delta_rule,
Qwen3_5RMSNormGated) on BASELINE config 0 and a few edge shapes, and stores
inputs and outputs as .npz.  It never imports the reference repository.

  python tests/golden/make_golden.py      (writes tests/golden/*.npz)
"""
from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F
from transformers.models.qwen3_5 import modeling_qwen3_5 as up

OUT = Path(__file__).resolve().parent


def _np(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().numpy()


def config0(seed: int = 0):
    """T=256, H=4, d=64, fp32; raw qkv ~ N(0,1) -> conv
    (width 4, w ~ N(0, 0.5^2)) + SiLU -> split -> rule with q,k L2-normalised
    in the rule; a, b ~ N(0,1); A_log ~ U(0, ln 16); dt_bias ~ U(-1, 1);
    zero initial state.  Draw order: x, w, a, b, A_log, dt_bias, z, norm_w."""
    gen = torch.Generator().manual_seed(seed)
    T, H, D = 256, 4, 64
    C = 3 * H * D
    x = torch.randn(T, C, generator=gen)
    w = torch.randn(C, 4, generator=gen) * 0.5
    a = torch.randn(T, H, generator=gen)
    b = torch.randn(T, H, generator=gen)
    A_log = torch.rand(H, generator=gen) * math.log(16)
    dt_bias = torch.rand(H, generator=gen) * 2 - 1
    z = torch.randn(T, H, D, generator=gen)
    norm_w = 1 + 0.02 * torch.randn(D, generator=gen)

    y = up.causal_conv1d_fn(x.t()[None], w, None, activation="silu")[0].t()      # [T, C]
    q = y[:, :H * D].reshape(1, T, H, D)
    k = y[:, H * D:2 * H * D].reshape(1, T, H, D)
    v = y[:, 2 * H * D:].reshape(1, T, H, D)
    beta = b.sigmoid()[None]
    g = (-A_log.exp() * F.softplus(a + dt_bias))[None]
    o_chunk, s_chunk = up.torch_chunk_gated_delta_rule(q, k, v, g, beta, chunk_size=64, initial_state=None,
                                                       output_final_state=True, use_qk_l2norm_in_kernel=True)
    o_rec, s_rec = up.torch_recurrent_gated_delta_rule(q, k, v, g, beta, initial_state=None,
                                                       output_final_state=True, use_qk_l2norm_in_kernel=True)
    norm = up.Qwen3_5RMSNormGated(D, eps=1e-6)
    with torch.no_grad():
        norm.weight.copy_(norm_w)
        y_norm = norm(o_chunk[0].reshape(-1, D), z.reshape(-1, D)).reshape(T, H, D)
    # kept small: the norm and recurrent outputs are stored for a token subset
    np.savez_compressed(OUT / "config0.npz", x=_np(x), w=_np(w), a=_np(a), b=_np(b), A_log=_np(A_log),
                        dt_bias=_np(dt_bias), z=_np(z[:32]), norm_w=_np(norm_w), conv_y=_np(y), g=_np(g[0]),
                        beta=_np(beta[0]), o_chunk=_np(o_chunk[0]), state_chunk=_np(s_chunk[0]),
                        o_rec_tail=_np(o_rec[0, -64:]), state_rec=_np(s_rec[0]), y_norm=_np(y_norm[:32]))


def edge_cases(seed: int = 5):
    """Small edge shapes: ragged T (65, with a tail chunk of 1), a non-zero
    initial state, grouped value heads (Hk=2 -> Hv=4 via repeat_interleave
    as the reference layer does), single-token conv update with a state,
    and the bf16 gated norm."""
    gen = torch.Generator().manual_seed(seed)
    T, Hk, Hv, D = 65, 2, 4, 32
    q = torch.randn(1, T, Hk, D, generator=gen)
    k = torch.randn(1, T, Hk, D, generator=gen)
    v = torch.randn(1, T, Hv, D, generator=gen)
    a = torch.randn(1, T, Hv, generator=gen)
    b = torch.randn(1, T, Hv, generator=gen)
    A_log = torch.rand(Hv, generator=gen) * math.log(16)
    dt_bias = torch.rand(Hv, generator=gen) * 2 - 1
    h0 = torch.randn(1, Hv, D, D, generator=gen) * 0.1
    g = -A_log.exp() * F.softplus(a + dt_bias)
    beta = b.sigmoid()
    qr, kr = q.repeat_interleave(Hv // Hk, dim=2), k.repeat_interleave(Hv // Hk, dim=2)
    o_chunk, s_chunk = up.torch_chunk_gated_delta_rule(qr, kr, v, g, beta, chunk_size=64, initial_state=h0.clone(),
                                                       output_final_state=True, use_qk_l2norm_in_kernel=True)
    o_rec, s_rec = up.torch_recurrent_gated_delta_rule(qr, kr, v, g, beta, initial_state=h0.clone(),
                                                       output_final_state=True, use_qk_l2norm_in_kernel=True)
    # single-token conv update against a non-zero state
    C = 48
    cx = torch.randn(3, C, 1, generator=gen)
    cstate = torch.randn(3, C, 3, generator=gen)
    cw = torch.randn(C, 4, generator=gen) * 0.5
    cstate_after = cstate.clone()
    cy = up.causal_conv1d_update(cx, cstate_after, cw, None, activation="silu")
    # bf16 gated norm (rounding order of the module)
    nx = torch.randn(40, 16, 128, generator=gen).to(torch.bfloat16)
    nz = torch.randn(40, 16, 128, generator=gen).to(torch.bfloat16)
    nw = (1 + 0.02 * torch.randn(128, generator=gen))
    norm = up.Qwen3_5RMSNormGated(128, eps=1e-6).to(torch.bfloat16)
    with torch.no_grad():
        norm.weight.copy_(nw.to(torch.bfloat16))
        ny = norm(nx.reshape(-1, 128), nz.reshape(-1, 128)).reshape(40, 16, 128)
    np.savez_compressed(OUT / "edge.npz", q=_np(q[0]), k=_np(k[0]), v=_np(v[0]), g=_np(g[0]), beta=_np(beta[0]),
                        h0=_np(h0[0]), o_chunk=_np(o_chunk[0]), state_chunk=_np(s_chunk[0]), o_rec=_np(o_rec[0]),
                        state_rec=_np(s_rec[0]), cx=_np(cx[:, :, 0]), cstate=_np(cstate), cw=_np(cw),
                        cy=_np(cy[:, :, 0]), cstate_after=_np(cstate_after),
                        nx=_np(nx.view(torch.int16)), nz=_np(nz.view(torch.int16)),
                        nw=_np(nw.to(torch.bfloat16).view(torch.int16)), ny=_np(ny.view(torch.int16)))


if __name__ == "__main__":
    torch.set_num_threads(4)
    config0()
    edge_cases()
    for f in sorted(OUT.glob("*.npz")):
        print(f.name, f.stat().st_size)
