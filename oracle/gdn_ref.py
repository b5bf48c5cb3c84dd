"""CPU restatement of the reference GDN layer path -- TEST INFRASTRUCTURE ONLY.

This module is the parity oracle: only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg import it, and only as the checker / CPU
baseline.  The product package (nano-vllm-extend_amd/) never imports it.

It restates, in fp32 torch on the CPU, the functions of
nanovllm/models/qwen3_5.py that the HIP kernels replace (file:line per
function).  Each function is pinned by tests/test_oracle.py against golden
vectors made with the upstream transformers torch functions the reference
ports (tests/golden/), against the fp64 brute-force recurrence in
oracle/recurrence.c, and against closed forms.  Deliberate choices:
  * q/k L2 norm in fp32 (the fla kernel and the reference's Triton decode
    kernel, qwen3_5.py:581-583; the torch port applies it in the input dtype);
  * softplus as log(1 + exp(z)) with threshold 20 (the default Triton path,
    qwen3_5.py:336);
  * gated norm in the eager rounding order (qwen3_5.py:121-131).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

BF16 = torch.bfloat16


def _bf(x: torch.Tensor) -> torch.Tensor:
    """Round to bf16 and back to fp32."""
    return x.to(BF16).to(torch.float32)


# ----------------------------------------------------------------- g / beta --
def g_beta(b: torch.Tensor, a: torch.Tensor, A_log: torch.Tensor, dt_bias: torch.Tensor,
           mask: torch.Tensor | None = None):
    """g = -exp(A_log) * softplus(a + dt_bias), beta = sigmoid(b) -> bf16.
    Follows _gdn_g_beta_kernel, nanovllm/models/qwen3_5.py:320-342."""
    z = a.float() + dt_bias.float()
    sp = torch.where(z > 20.0, z, torch.log(1.0 + torch.exp(z)))
    g = -torch.exp(A_log.float()) * sp
    if mask is not None:
        g = torch.where(mask.reshape(*mask.shape, *([1] * (g.dim() - mask.dim()))), g, torch.zeros_like(g))
    beta = torch.sigmoid(b.float()).to(BF16)
    return g, beta


# --------------------------------------------------------------------- conv --
def _roll_bits(x: torch.Tensor) -> torch.Tensor:
    """The reference's state writeback computes (x + s) with the other term
    masked to +0 (qwen3_5.py:293-297, :452-456): a bit copy except -0 -> +0."""
    return (x.float() + 0.0).to(x.dtype)


def conv_silu_window(window: torch.Tensor, w: torch.Tensor, eager_dtype=None) -> torch.Tensor:
    """window [C, K-1+T] fp32 (state then inputs), w [C, K] -> silu(conv) [C, T].
    y[c,t] = silu(sum_i w[c,i] * window[c, t+i]) (qwen3_5.py:286-292).
    eager_dtype (e.g. bf16) restates the eager F.silu(F.conv1d(...)) chain of
    the NANOVLLM_CONV_TRITON=0 path (qwen3_5.py:1020-1024, :1057-1065): the
    conv sum is rounded to that dtype before the SiLU."""
    C, L = window.shape
    K = w.shape[1]
    T = L - (K - 1)
    acc = torch.zeros(C, T, dtype=torch.float32)
    for i in range(K):
        acc += window[:, i:i + T] * w[:, i:i + 1].float()
    if eager_dtype is not None:
        acc = acc.to(eager_dtype).float()
    return acc * torch.sigmoid(acc)


def conv_varlen(x: torch.Tensor, state: torch.Tensor, w: torch.Tensor, lens: list[int], eager: bool = False):
    """Varlen causal conv + SiLU (nanovllm/models/qwen3_5.py:402-456).
    x [N, C], state [n, C, K-1], w [C, K] (bf16 in the model; any float dtype).
    Returns (y [N, C] in x's dtype, new_state [n, C, K-1])."""
    N, C = x.shape
    K = w.shape[-1]
    y = torch.empty(N, C, dtype=x.dtype)
    new_state = state.clone()
    off = 0
    for r, T in enumerate(lens):
        xs = x[off:off + T].float().t()                              # [C, T]
        window = torch.cat([state[r].float(), xs], dim=1)            # [C, K-1+T]
        y[off:off + T] = conv_silu_window(window, w.float(), x.dtype if eager else None).t().to(x.dtype)
        raw = torch.cat([state[r], x[off:off + T].t()], dim=1)       # bf16 bits
        new_state[r] = raw[:, T:T + K - 1] if eager else _roll_bits(raw[:, T:T + K - 1])
        off += T
    return y, new_state


def conv_decode(x: torch.Tensor, pool: torch.Tensor, ids: list[int], w: torch.Tensor, eager: bool = False):
    """Single-token conv + SiLU with in-place roll (qwen3_5.py:515-543):
    y = silu(x*w[K-1] + sum_i s[i]*w[i]); s <- [s1, s2, x] (bit copies).
    Returns (y [B, C] in x's dtype, new_pool)."""
    B, C = x.shape
    K = w.shape[-1]
    pool = pool.clone()
    y = torch.empty(B, C, dtype=x.dtype)
    for b, slot in enumerate(ids):
        s = pool[slot].float()                                        # [C, K-1]
        acc = x[b].float() * w[:, K - 1].float()
        for i in range(K - 1):
            acc = acc + s[:, i] * w[:, i].float()
        if eager:
            acc = acc.to(x.dtype).float()
        y[b] = (acc * torch.sigmoid(acc)).to(x.dtype)
        pool[slot] = torch.cat([pool[slot][:, 1:], x[b].unsqueeze(1)], dim=1)
    return y, pool


def conv_padded(x: torch.Tensor, state: torch.Tensor, w: torch.Tensor, endp: list[int]):
    """Padded conv + SiLU with per-row writeback at endp (qwen3_5.py:249-297).
    x [n, C, T].  Returns (y [n, C, T] in x's dtype, new_state)."""
    n, C, T = x.shape
    K = w.shape[-1]
    y = torch.empty(n, C, T, dtype=x.dtype)
    new_state = state.clone()
    for r in range(n):
        window = torch.cat([state[r].float(), x[r].float()], dim=1)
        y[r] = conv_silu_window(window, w.float()).to(x.dtype)
        e = endp[r]
        if e >= 0:
            raw = torch.cat([state[r], x[r]], dim=1)
            new_state[r] = _roll_bits(raw[:, e:e + K - 1])
    return y, new_state


# -------------------------------------------------------------- delta rule --
def l2norm(x: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """x * rsqrt(sum(x^2) + eps) (qwen3_5.py:134-137), in fp32."""
    x = x.float()
    return x * torch.rsqrt((x * x).sum(-1, keepdim=True) + eps)


def chunk_rule(q, k, v, g, beta, h0=None, chunk_size: int = 64, scale: float | None = None,
               use_l2norm: bool = True):
    """One sequence, chunked gated delta rule, fp32 (qwen3_5.py:152-227).
    q, k [T, Hv, Dk] (already grouped to value heads), v [T, Hv, Dv],
    g, beta [T, Hv]; h0 [Hv, Dk, Dv] or None.
    Returns (o [T, Hv, Dv] fp32, final [Hv, Dk, Dv] fp32)."""
    T, H, Dk = k.shape
    Dv = v.shape[-1]
    if use_l2norm:
        q, k = l2norm(q), l2norm(k)
    q, k, v, beta, g = [t.transpose(0, 1).contiguous().float() for t in (q, k, v, beta, g)]
    pad = (chunk_size - T % chunk_size) % chunk_size
    q = F.pad(q, (0, 0, 0, pad))
    k = F.pad(k, (0, 0, 0, pad))
    v = F.pad(v, (0, 0, 0, pad))
    beta = F.pad(beta, (0, pad))
    g = F.pad(g, (0, pad))
    L = T + pad
    q = q * (Dk ** -0.5 if scale is None else scale)
    v_beta = v * beta.unsqueeze(-1)
    k_beta = k * beta.unsqueeze(-1)
    nc = L // chunk_size
    q, k, v, k_beta, v_beta = [t.reshape(H, nc, chunk_size, t.shape[-1]) for t in (q, k, v, k_beta, v_beta)]
    g = g.reshape(H, nc, chunk_size).cumsum(-1)
    decay = (g.unsqueeze(-1) - g.unsqueeze(-2)).tril().exp().tril()
    upper = torch.triu(torch.ones(chunk_size, chunk_size, dtype=torch.bool), 0)
    attn = -((k_beta @ k.transpose(-1, -2)) * decay).masked_fill(upper, 0)
    for i in range(1, chunk_size):                                   # forward substitution
        row = attn[..., i, :i].clone()
        sub = attn[..., :i, :i].clone()
        attn[..., i, :i] = row + (row.unsqueeze(-1) * sub).sum(-2)
    attn = attn + torch.eye(chunk_size)
    u = attn @ v_beta
    w = attn @ (k_beta * g.exp().unsqueeze(-1))
    S = torch.zeros(H, Dk, Dv) if h0 is None else h0.float().clone()
    o = torch.zeros(H, nc, chunk_size, Dv)
    for i in range(nc):
        qi, ki = q[:, i], k[:, i]
        a = qi @ ki.transpose(-1, -2) * decay[:, i]
        v_new = u[:, i] - w[:, i] @ S
        o[:, i] = (qi * g[:, i, :, None].exp()) @ S + a @ v_new
        S = S * g[:, i, -1, None, None].exp() + (ki * (g[:, i, -1, None] - g[:, i]).exp()[..., None]).transpose(-1, -2) @ v_new
    o = o.reshape(H, L, Dv)[:, :T].transpose(0, 1).contiguous()
    return o, S


def expand_heads(x: torch.Tensor, hv: int) -> torch.Tensor:
    """Value head h reads key head h // (Hv // Hk) (repeat_interleave, qwen3_5.py:1002-1005)."""
    hk = x.shape[-2]
    return x if hk == hv else x.repeat_interleave(hv // hk, dim=-2)


def chunk_varlen(q, k, v, g, beta, cu: list[int], h0=None, scale=None, use_l2norm=True):
    """Varlen chunk rule over packed rows: q, k [N, Hk, D], v [N, Hv, D],
    g, beta [N, Hv], cu [n+1], h0 [n, Hv, D, D] or None.
    Returns (o [N, Hv, D] fp32, final [n, Hv, D, D])."""
    Hv = v.shape[1]
    qe, ke = expand_heads(q.float(), Hv), expand_heads(k.float(), Hv)
    o = torch.zeros(v.shape[0], Hv, v.shape[2])
    finals = []
    for r in range(len(cu) - 1):
        a, b = cu[r], cu[r + 1]
        o_r, s_r = chunk_rule(qe[a:b], ke[a:b], v[a:b].float(), g[a:b].float(), beta[a:b].float(),
                              None if h0 is None else h0[r], scale=scale, use_l2norm=use_l2norm)
        o[a:b] = o_r
        finals.append(s_r)
    return o, torch.stack(finals) if finals else torch.zeros(0, Hv, v.shape[2], v.shape[2])


def recurrent_rule(q, k, v, g, beta, h0=None, scale=None, use_l2norm=True, keep_states=False):
    """Token-by-token gated delta rule, fp32 (qwen3_5.py:575-594, :616-651;
    upstream T >= 1 loop).  q, k [B, T, Hk, D], v [B, T, Hv, D], g/beta
    [B, T, Hv]; h0 [B, Hv, D, D] or None.
    Returns (o [B, T, Hv, D], final [B, Hv, D, D], states [B, T, Hv, D, D] or None)."""
    Bsz, T, _, D = k.shape
    Hv = v.shape[2]
    qe, ke = expand_heads(q.float(), Hv), expand_heads(k.float(), Hv)
    if use_l2norm:
        qe, ke = l2norm(qe), l2norm(ke)
    qe = qe * (D ** -0.5 if scale is None else scale)
    S = torch.zeros(Bsz, Hv, D, v.shape[3]) if h0 is None else h0.float().clone()
    o = torch.zeros(Bsz, T, Hv, v.shape[3])
    states = torch.zeros(Bsz, T, Hv, D, v.shape[3]) if keep_states else None
    for t in range(T):
        S = S * g[:, t].float().exp()[..., None, None]
        kv = (S * ke[:, t, :, :, None]).sum(-2)
        delta = (v[:, t].float() - kv) * beta[:, t].float()[..., None]
        S = S + ke[:, t, :, :, None] * delta[:, :, None, :]
        o[:, t] = (S * qe[:, t, :, :, None]).sum(-2)
        if keep_states:
            states[:, t] = S
    return o, S, states


# -------------------------------------------------------------- gated norm --
def rms_norm_gated(x: torch.Tensor, z: torch.Tensor, w: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """Eager order of _rms_gated_forward (qwen3_5.py:121-131) in the input
    dtype (bf16 in the model): fp32 norm rounded to the input dtype, weight
    product in the input dtype, fp32 silu gate, output in the input dtype."""
    dt = x.dtype
    xf = x.float()
    var = xf.pow(2).mean(-1, keepdim=True)
    n = (xf * torch.rsqrt(var + eps)).to(dt)
    wn = w.to(dt) * n
    return (wn.float() * F.silu(z.float())).to(dt)


# ------------------------------------------------------------ layer core --
def gdn_core_varlen(mixed, z, b, a, lens, conv_state, h0, conv_w, A_log, dt_bias, norm_w,
                    Hk, Hv, D, eps=1e-6, conv_eager=False):
    """The GDN layer between its projections for one varlen prefill group
    (qwen3_5.py:922-965 without in_proj / out_proj): g/beta, conv + SiLU,
    chunk rule with initial states, gated norm.
    Returns (core [N, Hv, D] bf16, new conv states, final states)."""
    N = mixed.shape[0]
    g, beta = g_beta(b, a, A_log, dt_bias)
    y, new_conv = conv_varlen(mixed, conv_state, conv_w, lens, eager=conv_eager)
    kd = Hk * D
    qh = y[:, :kd].reshape(N, Hk, D)
    kh = y[:, kd:2 * kd].reshape(N, Hk, D)
    vh = y[:, 2 * kd:].reshape(N, Hv, D)
    cu = [0]
    for t in lens:
        cu.append(cu[-1] + t)
    o, final = chunk_varlen(qh, kh, vh, g, beta.float(), cu, h0)
    core = rms_norm_gated(o.to(BF16), z.reshape(N, Hv, D), norm_w, eps)
    return core, new_conv, final


def gdn_core_decode(mixed, z, b, a, ids, conv_pool, s_pool, conv_w, A_log, dt_bias, norm_w,
                    Hk, Hv, D, eps=1e-6, conv_eager=False):
    """One decode step of the GDN layer core against the slot pools
    (qwen3_5.py:967-1030, T = 1, in-place path).
    Returns (core [B, Hv, D] bf16, new conv pool, new state pool)."""
    B = mixed.shape[0]
    g, beta = g_beta(b, a, A_log, dt_bias)
    y, conv_pool = conv_decode(mixed, conv_pool, ids, conv_w, eager=conv_eager)
    kd = Hk * D
    q = y[:, :kd].reshape(B, 1, Hk, D)
    k = y[:, kd:2 * kd].reshape(B, 1, Hk, D)
    v = y[:, 2 * kd:].reshape(B, 1, Hv, D)
    s_pool = s_pool.clone()
    h0 = s_pool[ids]
    o, final, _ = recurrent_rule(q, k, v, g.reshape(B, 1, Hv), beta.float().reshape(B, 1, Hv), h0)
    s_pool[ids] = final
    core = rms_norm_gated(o[:, 0].to(BF16), z.reshape(B, Hv, D), norm_w, eps)
    return core, conv_pool, s_pool


def flops_chunk(n_tokens: int, Hv: int, D: int, C: int = 64) -> float:
    """Algorithmic chunk-prefill FLOPs: N*Hv*[2C(3D+2D) + 6D^2 + (2/3)C^2]."""
    return float(n_tokens) * Hv * (2 * C * (3 * D + 2 * D) + 6 * D * D + (2.0 / 3.0) * C * C)

