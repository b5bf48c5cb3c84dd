"""GDN operators with the reference's Python signatures, backed by the gfx950
HIP kernels of libgdn_mi355x.so.

Each function mirrors a module-level function of
nanovllm/models/qwen3_5.py (cited per function): same argument meaning,
same output allocation (torch.empty on the input's device), same in-place
mutation of the state pools, and the reference's shape asserts.  There is no
CPU or eager fallback: a CPU tensor or a missing library raises.
"""
from __future__ import annotations

import ctypes
import os

import torch

from . import _lib


def _check_cuda(*ts: torch.Tensor | None) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError("GDN ops run on the GPU only (got a CPU tensor; there is no CPU path)")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} vs {t.device}")
    return dev


def _bf16(t: torch.Tensor, name: str) -> None:
    if t.dtype != torch.bfloat16:
        raise TypeError(f"{name} must be bfloat16, got {t.dtype}")


def _stream(dev: torch.device) -> int:
    return _lib.stream_handle(dev)


# ------------------------------------------------------- fp16 operand range --
# The chunk kernels run their state-path products on fp16 matrix cores: the
# raw k and v rows (after the conv), Q', the block inverses, A, the state S
# and Vn = U - W S become fp16 operands, so each must stay below the fp16
# maximum.  Q' and A are bounded by the L2 norm (|Q'| <= scale, |A| <= scale);
# the inputs a caller controls are checked here on request.
FP16_MAX = 65504.0


def range_check_enabled() -> bool:
    """NANOVLLM_GDN_CHECK_RANGE=1 turns on the input range check of the
    prefill wrappers (a device reduction and a host sync per call)."""
    return os.environ.get("NANOVLLM_GDN_CHECK_RANGE", "0") == "1"


def fp16_range_violation(rows: torch.Tensor | None = None, conv_weight: torch.Tensor | None = None,
                         states: torch.Tensor | None = None) -> str | None:
    """Why a prefill call's inputs could leave the fp16 operand range, or None.

    rows: the rows that feed the kernels -- raw q|k|v rows when conv_weight
    [C, 4] is given (the conv output of channel c is at most
    sum_i |w[c, i]| * max |x| in magnitude, SiLU not increasing it), else the
    q, k, v rows themselves; states: the initial states that will be read.
    Non-finite values count as violations.  Works on any device."""
    if rows is not None and rows.numel():
        m = rows.detach().float().abs().amax()
        if not torch.isfinite(m):
            return "non-finite input rows"
        bound = float(m)
        if conv_weight is not None:
            gain = float(conv_weight.detach().float().reshape(conv_weight.shape[0], -1).abs().sum(1).amax())
            bound *= gain
        if bound >= FP16_MAX:
            return (f"input rows reach {bound:.4g} after the conv" if conv_weight is not None
                    else f"input rows reach {bound:.4g}") + f" (fp16 operands must stay below {FP16_MAX:g})"
    if states is not None and states.numel():
        m = float(states.detach().abs().amax())
        if not m < FP16_MAX:  # also catches NaN / inf
            return f"initial states reach {m:.4g} (fp16 operands must stay below {FP16_MAX:g})"
    return None


def _check_range(**kw) -> None:
    why = fp16_range_violation(**kw)
    if why is not None:
        raise ValueError(f"GDN chunk prefill: {why}")


# ----------------------------------------------------------------- g / beta --
def fused_g_beta(b: torch.Tensor, a: torch.Tensor, a_log: torch.Tensor, dt_bias: torch.Tensor,
                 mask: torch.Tensor | None):
    """g = -exp(A_log) * softplus(a + dt_bias) (fp32, 0 on padding rows),
    beta = sigmoid(b) (bf16).  b/a [.., Vh] bf16 contiguous; a_log/dt_bias
    [Vh] (bf16 or fp32); mask [n, T] bool or None.
    Reference: fused_g_beta, nanovllm/models/qwen3_5.py:345-360."""
    dev = _check_cuda(b, a, a_log, dt_bias, mask)
    _bf16(a, "a")
    _bf16(b, "b")
    assert a.is_contiguous() and b.is_contiguous() and a.shape == b.shape
    vh = a.shape[-1]
    if a_log.dtype != dt_bias.dtype or a_log.dtype not in (torch.bfloat16, torch.float32):
        a_log = a_log.float()
        dt_bias = dt_bias.float()
    a_log = a_log.contiguous()
    dt_bias = dt_bias.contiguous()
    assert a_log.numel() == vh and dt_bias.numel() == vh
    g = torch.empty_like(a, dtype=torch.float32)
    beta = torch.empty_like(a)
    flat_mask = None
    if mask is not None:
        flat_mask = mask.reshape(-1).contiguous()
        if flat_mask.dtype != torch.bool:
            flat_mask = flat_mask.to(torch.bool)
        assert flat_mask.numel() * vh == a.numel()
    _lib.call("gdn_g_beta", _lib.ptr(b), _lib.ptr(a), _lib.ptr(a_log), _lib.ptr(dt_bias),
              int(a_log.dtype == torch.float32), _lib.ptr(flat_mask), _lib.ptr(g), _lib.ptr(beta),
              a.numel(), vh, _stream(dev))
    return g, beta


# --------------------------------------------------------------------- conv --
def _conv_varlen(x, state, weight, lens, cuseq, key_dim, state_ids):
    dev = _check_cuda(x, state, weight, lens, cuseq, state_ids)
    _bf16(x, "x")
    _bf16(state, "state")
    N, C = x.shape
    K = weight.shape[-1]
    w = weight.reshape(C, K)
    _bf16(w, "weight")
    w = w.contiguous()
    assert x.stride(1) == 1 and state.stride(2) == 1 and tuple(state.shape[1:]) == (C, K - 1)
    n = lens.shape[0]
    lens32 = lens.to(torch.int32).contiguous()
    cu32 = cuseq.to(torch.int32).contiguous()
    assert cu32.shape[0] >= n
    ids = None
    if state_ids is not None:
        ids = state_ids.to(torch.int64).contiguous()
        assert ids.shape[0] == n
    y = torch.empty(N * C, dtype=x.dtype, device=x.device)
    _lib.call("gdn_conv_varlen", _lib.ptr(x), x.stride(0), _lib.ptr(state), state.stride(0),
              state.stride(1), _lib.ptr(ids), _lib.ptr(w), _lib.ptr(y), key_dim, _lib.ptr(lens32),
              _lib.ptr(cu32), n, N, C, K, _stream(dev))
    return y


def causal_conv_silu_varlen_parts(x: torch.Tensor, state: torch.Tensor, weight: torch.Tensor,
                                  lens: torch.Tensor, cuseq: torch.Tensor, key_dim: int,
                                  state_ids: torch.Tensor | None = None):
    """Varlen conv + SiLU returning the (q, k, v) parts [N, key_dim],
    [N, key_dim], [N, C - 2*key_dim], each contiguous (one allocation), so
    grouped-value layouts (C != 3*key_dim) are covered.  state: conv states
    [n, C, K-1], or with state_ids the slot pool [slots, C, K-1] updated in
    place at those rows."""
    N, C = x.shape
    y = _conv_varlen(x, state, weight, lens, cuseq, key_dim, state_ids)
    q = y[: N * key_dim].view(N, key_dim)
    k = y[N * key_dim: 2 * N * key_dim].view(N, key_dim)
    v = y[2 * N * key_dim:].view(N, C - 2 * key_dim)
    return q, k, v


def causal_conv_silu_varlen(x: torch.Tensor, state: torch.Tensor, weight: torch.Tensor,
                            lens: torch.Tensor, cuseq: torch.Tensor) -> torch.Tensor:
    """x [N, C] bf16 contiguous varlen; state [n, C, K-1] (updated in place);
    lens int32 [n]; cuseq int32 [n] (per-row starts).  Returns [3, N, C//3]:
    the q/k/v thirds, each contiguous.
    Reference: causal_conv_silu_varlen, nanovllm/models/qwen3_5.py:459-473."""
    N, C = x.shape
    d3 = C // 3
    assert d3 * 3 == C and d3 % 64 == 0
    return _conv_varlen(x, state, weight, lens, cuseq, d3, None).view(3, N, d3)


def conv_decode_step(x: torch.Tensor, state_pool: torch.Tensor, ids: torch.Tensor,
                     weight: torch.Tensor) -> torch.Tensor:
    """x [n, C] (decode rows); state_pool [slots, C, K-1] rolled in place at
    rows `ids`; weight [C, K] (or [C, 1, K]).  Returns y [n, C].
    Reference: conv_decode_step, nanovllm/models/qwen3_5.py:546-558."""
    dev = _check_cuda(x, state_pool, ids, weight)
    _bf16(x, "x")
    _bf16(state_pool, "state_pool")
    n, C = x.shape
    K = weight.shape[-1]
    w = weight.reshape(C, K).contiguous()
    assert x.stride(1) == 1 and state_pool.stride(2) == 1
    ids64 = ids.to(torch.int64).contiguous()
    assert ids64.shape == (n,), "one slot id per row"
    y = torch.empty(n, C, dtype=x.dtype, device=x.device)
    _lib.call("gdn_conv_decode", _lib.ptr(x), x.stride(0), _lib.ptr(state_pool), state_pool.stride(0),
              state_pool.stride(1), _lib.ptr(ids64), _lib.ptr(w), _lib.ptr(y), y.stride(0), n, C, K,
              _stream(dev))
    return y


def causal_conv_silu(x: torch.Tensor, state: torch.Tensor, weight: torch.Tensor,
                     endp: torch.Tensor) -> torch.Tensor:
    """x [n, C, T] (arbitrary strides), state [n, C, K-1] (updated in place
    at each row's endp), weight [C, K].  Returns y [n, C, T] contiguous;
    endp int32 [n] (-1 = skip writeback).
    Reference: causal_conv_silu, nanovllm/models/qwen3_5.py:300-317."""
    dev = _check_cuda(x, state, weight, endp)
    _bf16(x, "x")
    _bf16(state, "state")
    n, C, T = x.shape
    K = weight.shape[-1]
    w = weight.reshape(C, K).contiguous()
    assert state.stride(2) == 1
    e32 = endp.to(torch.int32).contiguous()
    y = torch.empty(n, C, T, dtype=x.dtype, device=x.device)
    _lib.call("gdn_conv_padded", _lib.ptr(x), x.stride(0), x.stride(1), x.stride(2), _lib.ptr(state),
              state.stride(0), state.stride(1), _lib.ptr(w), _lib.ptr(y), _lib.ptr(e32), n, C, T, K,
              _stream(dev))
    return y


# -------------------------------------------------------------- chunk rule --
def _host_offsets(cu_cpu, n: int):
    """int64 host copy of the sequence offsets [n + 1], or None."""
    if cu_cpu is None:
        return None
    t = torch.as_tensor(cu_cpu)
    if t.device.type != "cpu":
        raise ValueError("cu_seqlens_cpu must be in host memory")
    t = t.to(torch.int64).contiguous()
    assert t.shape == (n + 1,)
    return t


def _host_ptr(t):
    """Host pointer of a CPU tensor (the caller keeps the tensor alive)."""
    return None if t is None else t.data_ptr()


def _state_view_ok(s: torch.Tensor, H: int, D: int) -> bool:
    return (s.dtype == torch.float32 and s.dim() == 4 and tuple(s.shape[1:]) == (H, D, D)
            and s.stride(1) == D * D and s.stride(2) == D and s.stride(3) == 1)


def _rows16(t: torch.Tensor, D: int) -> torch.Tensor:
    if t.stride(2) != 1 or t.stride(1) != D or t.stride(0) % 8 or t.data_ptr() % 16:
        return t.contiguous() if not t.is_contiguous() else t.clone()
    return t


def chunk_gated_delta_rule_varlen(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, g: torch.Tensor,
                                  beta: torch.Tensor, cu_seqlens: torch.Tensor,
                                  initial_state: torch.Tensor | None = None, *,
                                  output_final_state: bool = True,
                                  use_qk_l2norm_in_kernel: bool = True, scale: float | None = None,
                                  state_ids: torch.Tensor | None = None,
                                  final_state: torch.Tensor | None = None,
                                  cu_seqlens_cpu: torch.Tensor | None = None, max_segments: int = 0):
    """Varlen chunked gated delta rule (chunk 64) on packed rows.

    q, k [N, Hk, D]; v [N, Hv, D] (bf16, head dim contiguous, any token
    stride); g [N, Hv] fp32; beta [N, Hv] bf16; cu_seqlens [n+1] (device).
    Value head h uses key head h // (Hv // Hk).
    initial_state: [n, Hv, D, D] fp32, or with state_ids a slot pool
    [slots, Hv, D, D] (any slot stride) read at rows state_ids.
    Final states go to `final_state` (same indexing; may be the pool itself
    for an in-place update) or to a new [n, Hv, D, D] tensor.
    cu_seqlens_cpu: the offsets on the host (as the fla call passes them);
    with them a call of few long sequences is cut into segments that run in
    parallel (max_segments: 0 automatic, 1 never, k up to k per sequence).
    Returns (o [N, Hv, D] bf16, final or None)."""
    dev = _check_cuda(q, k, v, g, beta, cu_seqlens, initial_state, state_ids, final_state)
    for t, nm in ((q, "q"), (k, "k"), (v, "v"), (beta, "beta")):
        _bf16(t, nm)
    N, Hk, D = k.shape
    Hv = v.shape[1]
    assert q.shape == k.shape and v.shape[0] == N and v.shape[2] == D and Hv % Hk == 0
    # the kernels read 16-byte row pieces: head-contiguous rows, 16-byte
    # aligned, token stride a multiple of 8 elements (else copy once)
    q, k, v = (_rows16(t, D) for t in (q, k, v))
    g = g.float().contiguous() if g.dtype != torch.float32 else g.contiguous()
    beta = beta.contiguous()
    assert g.shape == (N, Hv) and beta.shape == (N, Hv)
    cu = cu_seqlens.to(torch.int64).contiguous()
    n = cu.shape[0] - 1
    ids = None
    if state_ids is not None:
        ids = state_ids.to(torch.int64).contiguous()
        assert ids.shape[0] == n
    h0 = initial_state
    if h0 is not None and not _state_view_ok(h0, Hv, D):
        assert state_ids is None, "pool-indexed initial state must be an fp32 [slots, H, D, D] view"
        h0 = h0.float().contiguous()
    hT = None
    if output_final_state:
        if final_state is not None:
            assert _state_view_ok(final_state, Hv, D)
            hT = final_state
        else:
            assert state_ids is None or h0 is not None
            hT = torch.empty(n, Hv, D, D, dtype=torch.float32, device=q.device)
    if ids is not None and hT is not None and final_state is None:
        raise ValueError("state_ids requires final_state (the pool) for the output state")
    sstride = 0
    for st in (h0, hT):
        if st is not None:
            sstride = st.stride(0)
    if h0 is not None and hT is not None:
        assert h0.stride(0) == hT.stride(0), "initial and final state must share the slot stride"
    if range_check_enabled():
        read = None
        if h0 is not None:
            read = h0.index_select(0, ids) if ids is not None else h0
        _check_range(rows=torch.cat([q.reshape(N, -1), k.reshape(N, -1), v.reshape(N, -1)], 1), states=read)
    if scale is None:
        scale = D ** -0.5
    o = torch.empty(N, Hv, D, dtype=v.dtype, device=v.device)
    # per-(chunk, head) records of the chunk-local phase; the caching
    # allocator's blocks are 512-byte aligned, the kernels need 256
    ws_bytes = _lib.load().gdn_chunk_prefill_workspace_size(N, n, Hv, D)
    if ws_bytes < 0:
        raise ValueError(f"unsupported chunk shape N={N} n_seqs={n} Hv={Hv} D={D}")
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=q.device)
    cu_host = _host_offsets(cu_seqlens_cpu, n)
    _lib.call("gdn_chunk_prefill", _lib.ptr(q), q.stride(0), _lib.ptr(k), k.stride(0), _lib.ptr(v),
              v.stride(0), _lib.ptr(g), _lib.ptr(beta), _lib.ptr(h0), _lib.ptr(hT), _lib.ptr(ids),
              sstride, _lib.ptr(cu), _host_ptr(cu_host), int(max_segments), n, N, Hk, Hv, D, float(scale),
              int(bool(use_qk_l2norm_in_kernel)), _lib.ptr(o), _lib.ptr(ws), ws_bytes, _stream(dev))
    return o, hT


def conv_chunk_prefill_varlen(mixed: torch.Tensor, conv_state: torch.Tensor, conv_weight: torch.Tensor,
                              b: torch.Tensor, a: torch.Tensor, a_log: torch.Tensor, dt_bias: torch.Tensor,
                              cu_seqlens: torch.Tensor, state: torch.Tensor, state_ids: torch.Tensor | None,
                              num_k_heads: int, num_v_heads: int, head_dim: int,
                              scale: float | None = None, fresh: torch.Tensor | None = None,
                              cu_seqlens_cpu: torch.Tensor | None = None, max_segments: int = 0,
                              late: list[bool] | None = None, side_stream=None, keep: list | None = None):
    """Gates, varlen causal conv1d + SiLU and the chunked gated delta rule in
    one call (two kernels), the prefill sequence of _gdn_prefill_varlen
    (nanovllm/models/qwen3_5.py:934-961): the same results as fused_g_beta ->
    causal_conv_silu_varlen_parts -> chunk_gated_delta_rule_varlen (q/k L2
    norm on), bit for bit.

    mixed [N, C] bf16 raw q|k|v rows (C = 2*Hk*D + Hv*D, channel stride 1);
    conv_state [slots, C, 3] bf16 and state [slots, Hv, D, D] fp32 slot pools,
    both read and updated in place at rows state_ids (the sequence index if
    None); conv_weight [C, 4] (or [C, 1, 4]); b, a [N, Hv] bf16; a_log,
    dt_bias [Hv]; cu_seqlens [n+1] (device).  fresh: optional bool/uint8 [n]:
    those sequences start from zero recurrent and conv states and their pool
    rows are not read (the slot zeroing of a fresh prefill,
    model_runner.py:305-322, folded into the call).  cu_seqlens_cpu /
    max_segments: as chunk_gated_delta_rule_varlen.

    late / side_stream (split state pass): after the prep kernel on the
    current stream, the state pass of the sequences with late[r] runs on the
    current stream and that of the others on side_stream, concurrently.  The
    caller orders later work on side_stream's results itself (e.g. the current
    stream waits for side_stream) and keeps the tensors appended to `keep`
    alive until then.  Returns o [N, Hv, D] bf16, and with `late` also an
    event recorded on side_stream after its state pass."""
    dev = _check_cuda(mixed, conv_state, conv_weight, b, a, a_log, dt_bias, cu_seqlens, state, state_ids)
    _bf16(mixed, "mixed")
    _bf16(conv_state, "conv_state")
    _bf16(a, "a")
    _bf16(b, "b")
    Hk, Hv, D = num_k_heads, num_v_heads, head_dim
    N, C = mixed.shape
    assert C == 2 * Hk * D + Hv * D and Hv % Hk == 0
    w = conv_weight.reshape(C, -1)
    _bf16(w, "conv_weight")
    assert w.shape[1] == 4, "the fused path is built for conv width 4"
    w = w.contiguous()
    if mixed.stride(1) != 1 or mixed.stride(0) % 8 or mixed.data_ptr() % 16:
        mixed = mixed.contiguous()
    assert conv_state.stride(2) == 1 and tuple(conv_state.shape[1:]) == (C, 3)
    a = a.contiguous()
    b = b.contiguous()
    assert a.shape == (N, Hv) and b.shape == (N, Hv)
    if a_log.dtype != dt_bias.dtype or a_log.dtype not in (torch.bfloat16, torch.float32):
        a_log = a_log.float()
        dt_bias = dt_bias.float()
    a_log = a_log.contiguous()
    dt_bias = dt_bias.contiguous()
    assert _state_view_ok(state, Hv, D), "state must be an fp32 [slots, Hv, D, D] view"
    cu = cu_seqlens.to(torch.int64).contiguous()
    n = cu.shape[0] - 1
    ids = None
    if state_ids is not None:
        ids = state_ids.to(torch.int64).contiguous()
        assert ids.shape[0] == n
    fr = None
    if fresh is not None:
        fr = fresh.to(device=mixed.device, dtype=torch.uint8).contiguous()
        assert fr.shape == (n,)
    if range_check_enabled():
        rows_read = torch.arange(n, device=mixed.device) if ids is None else ids
        if fr is not None:
            rows_read = rows_read[fr == 0]
        _check_range(rows=mixed, conv_weight=w, states=state.index_select(0, rows_read))
    if scale is None:
        scale = D ** -0.5
    o = torch.empty(N, Hv, D, dtype=torch.bfloat16, device=mixed.device)
    ws_bytes = _lib.load().gdn_conv_chunk_prefill_workspace_size(N, n, Hv, D)
    if ws_bytes < 0:
        raise ValueError(f"unsupported chunk shape N={N} n_seqs={n} Hv={Hv} D={D}")
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=mixed.device)
    cu_host = _host_offsets(cu_seqlens_cpu, n)

    def launch(phase, select, stream):
        _lib.call("gdn_conv_chunk_prefill", _lib.ptr(mixed), mixed.stride(0), _lib.ptr(conv_state),
                  conv_state.stride(0), conv_state.stride(1), _lib.ptr(w), _lib.ptr(b), _lib.ptr(a),
                  _lib.ptr(a_log), _lib.ptr(dt_bias), int(a_log.dtype == torch.float32), _lib.ptr(state),
                  _lib.ptr(state), _lib.ptr(ids), _lib.ptr(fr), state.stride(0), _lib.ptr(cu),
                  _host_ptr(cu_host), int(max_segments), phase, _host_ptr(select), n, N, Hk, Hv, D, float(scale),
                  1, _lib.ptr(o), _lib.ptr(ws), ws_bytes, stream)

    if late is None:
        launch(3, None, _stream(dev))
        return o
    assert side_stream is not None and cu_host is not None and len(late) == n
    sel_late = torch.tensor([bool(x) for x in late], dtype=torch.uint8)
    sel_early = 1 - sel_late
    cur = torch.cuda.current_stream(dev)
    launch(1, None, cur.cuda_stream)                       # prep
    ev = torch.cuda.Event()
    ev.record(cur)
    side_stream.wait_event(ev)
    launch(2, sel_late, cur.cuda_stream)                   # the long sequences
    launch(2, sel_early, side_stream.cuda_stream)          # the others, concurrently
    side_done = torch.cuda.Event()
    side_done.record(side_stream)
    if keep is not None:
        keep.extend([mixed, w, a, b, a_log, dt_bias, cu, ids, fr, o, ws, conv_state, state])
    return o, side_done


def conv_chunk_prefill_varlen_noalloc(mixed: torch.Tensor, conv_state: torch.Tensor, conv_weight: torch.Tensor,
                                      b: torch.Tensor, a: torch.Tensor, a_log: torch.Tensor, dt_bias: torch.Tensor,
                                      cu_seqlens: torch.Tensor, state: torch.Tensor, state_ids: torch.Tensor | None,
                                      num_k_heads: int, num_v_heads: int, head_dim: int, out: torch.Tensor,
                                      scale: float | None = None, fresh: torch.Tensor | None = None,
                                      cu_seqlens_cpu: torch.Tensor | None = None, max_segments: int = 0) -> None:
    """conv_chunk_prefill_varlen through the allocation-free entry point: the
    records live in the library's fixed per-GPU scratch array (no workspace
    allocation), and the output goes to the caller's `out` [N, Hv, D] bf16.
    Nothing here allocates device memory or copies: the inputs must already
    have the layouts the kernels read (checked).  Calls that overlap on one
    GPU race on the shared array.  A call whose records do not fit the array
    runs in pieces (sequence groups, and long sequences as token ranges), the
    same bits as max_segments=1; that needs cu_seqlens_cpu, without which such
    a call raises GDNKernelError."""
    dev = _check_cuda(mixed, conv_state, conv_weight, b, a, a_log, dt_bias, cu_seqlens, state, state_ids, out, fresh)
    Hk, Hv, D = num_k_heads, num_v_heads, head_dim
    N, C = mixed.shape
    for t, nm in ((mixed, "mixed"), (conv_state, "conv_state"), (a, "a"), (b, "b"), (out, "out"),
                  (conv_weight, "conv_weight")):
        _bf16(t, nm)
    assert C == 2 * Hk * D + Hv * D and Hv % Hk == 0
    assert mixed.stride(1) == 1 and mixed.stride(0) % 8 == 0
    assert conv_weight.is_contiguous() and conv_weight.numel() == 4 * C
    assert conv_state.stride(2) == 1 and tuple(conv_state.shape[1:]) == (C, 3)
    assert a.is_contiguous() and b.is_contiguous() and a.shape == (N, Hv) and b.shape == (N, Hv)
    assert a_log.dtype == dt_bias.dtype and a_log.dtype in (torch.bfloat16, torch.float32)
    assert a_log.is_contiguous() and dt_bias.is_contiguous()
    assert _state_view_ok(state, Hv, D), "state must be an fp32 [slots, Hv, D, D] view"
    assert cu_seqlens.dtype == torch.int64 and cu_seqlens.is_contiguous()
    n = cu_seqlens.shape[0] - 1
    if state_ids is not None:
        assert state_ids.dtype == torch.int64 and state_ids.is_contiguous() and state_ids.shape == (n,)
    if fresh is not None:
        assert fresh.dtype == torch.uint8 and fresh.is_contiguous() and fresh.shape == (n,)
    assert out.shape == (N, Hv, D) and out.is_contiguous()
    cu_host = _host_offsets(cu_seqlens_cpu, n)
    if scale is None:
        scale = D ** -0.5
    _lib.call("gdn_conv_chunk_prefill_noalloc", _lib.ptr(mixed), mixed.stride(0), _lib.ptr(conv_state),
              conv_state.stride(0), conv_state.stride(1), _lib.ptr(conv_weight), _lib.ptr(b), _lib.ptr(a),
              _lib.ptr(a_log), _lib.ptr(dt_bias), int(a_log.dtype == torch.float32), _lib.ptr(state),
              _lib.ptr(state), _lib.ptr(state_ids), _lib.ptr(fresh), state.stride(0), _lib.ptr(cu_seqlens),
              _host_ptr(cu_host), int(max_segments), n, N, Hk, Hv, D, float(scale), 1, _lib.ptr(out), _stream(dev))


def chunk_gated_delta_rule(query, key, value, g=None, beta=None, scale=None, initial_state=None,
                           output_final_state=False, use_qk_l2norm_in_kernel=False,
                           cu_seqlens=None, cu_seqlens_cpu=None, chunk_size=64, **kwargs):
    """Drop-in for the chunk GDN entry point the reference calls.

    Covers both reference call forms:
      * chunk_gated_delta_rule(q, k, v, g, beta, chunk_size=64, initial_state=...)
        (nanovllm/models/qwen3_5.py:140-149): batched [B, T, H, D], always
        returns the final state, L2-norm in kernel;
      * the fla varlen call (qwen3_5.py:956-960): q[None] [1, N, H, D],
        cu_seqlens int64 [n+1], initial_state [n, H, D, D].
    Returns (o [B, T, Hv, D] bf16, final [B or n, Hv, D, D] fp32 or None)."""
    if chunk_size != 64:
        raise ValueError("only chunk_size=64 is built (the reference's value)")
    if "cu_seqlens" in kwargs:
        cu_seqlens = kwargs.pop("cu_seqlens")
    B, T, Hq, D = query.shape
    Hv = value.shape[2]
    if cu_seqlens is not None:
        assert B == 1, "varlen mode takes a single packed batch row"
        cu = cu_seqlens
        qf, kf, vf = query[0], key[0], value[0]
        gf, bf = g[0], beta[0]
    else:
        cu = torch.arange(B + 1, device=query.device, dtype=torch.int64) * T
        qf = query.reshape(B * T, Hq, D)
        kf = key.reshape(B * T, Hq, D)
        vf = value.reshape(B * T, Hv, D)
        gf = g.reshape(B * T, Hv)
        bf = beta.reshape(B * T, Hv)
    o, final = chunk_gated_delta_rule_varlen(qf, kf, vf, gf, bf, cu, initial_state,
                                             output_final_state=output_final_state,
                                             use_qk_l2norm_in_kernel=use_qk_l2norm_in_kernel,
                                             scale=scale, cu_seqlens_cpu=cu_seqlens_cpu)
    return o.view(B, T, Hv, D), final


def chunk_gated_delta_rule_ref_api(query, key, value, g, beta, chunk_size=64, initial_state=None):
    """The reference module's own signature (nanovllm/models/qwen3_5.py:140-149):
    final state always returned, q/k L2-normalised in kernel."""
    return chunk_gated_delta_rule(query, key, value, g=g, beta=beta, initial_state=initial_state,
                                  output_final_state=True, use_qk_l2norm_in_kernel=True,
                                  chunk_size=chunk_size)


# ---------------------------------------------------------- recurrent rule --
def _recurrent(q, k, v, g, beta, s_in, s_out, ids, inter, scale, l2norm, src_states=None, src_accepted=None):
    dev = _check_cuda(q, k, v, g, beta, s_in, s_out, ids, inter, src_states, src_accepted)
    for t, nm in ((q, "q"), (k, "k"), (v, "v"), (beta, "beta")):
        _bf16(t, nm)
    Bsz, T, Hk, D = k.shape
    Hv = v.shape[2]
    assert q.shape == k.shape and v.shape[:2] == (Bsz, T) and v.shape[3] == D and Hv % Hk == 0
    assert q.stride(2) == D and k.stride(2) == D and v.stride(2) == D
    assert q.stride(3) == 1 and k.stride(3) == 1 and v.stride(3) == 1
    g = g.float() if g.dtype != torch.float32 else g
    assert g.is_contiguous() and beta.is_contiguous()
    assert g.numel() == Bsz * T * Hv and beta.numel() == Bsz * T * Hv
    assert _state_view_ok(s_in, Hv, D)
    if s_out is not None:
        assert _state_view_ok(s_out, Hv, D)
    ids64 = None
    if ids is not None:
        ids64 = ids.to(torch.int64).contiguous()
        assert ids64.shape[0] == Bsz
    if inter is not None:
        assert inter.is_contiguous() and inter.dtype == torch.float32
        assert inter.shape == (Bsz, T, Hv, D, D)
    src_acc, src_T = None, 1
    if src_accepted is not None:
        assert src_states is not None and src_states.is_contiguous() and src_states.dtype == torch.float32
        assert src_states.dim() == 5 and src_states.shape[0] == Bsz and src_states.shape[2:] == (Hv, D, D)
        src_T = src_states.shape[1]
        src_acc = src_accepted if src_accepted.dtype == torch.int64 else src_accepted.to(torch.int64)
        assert src_acc.shape == (Bsz,) and src_acc.is_contiguous()
    out = torch.empty(Bsz, T, Hv, D, dtype=v.dtype, device=v.device)
    if scale is None:
        scale = D ** -0.5
    _lib.call("gdn_recurrent", _lib.ptr(q), q.stride(0), q.stride(1), _lib.ptr(k), k.stride(0),
              k.stride(1), _lib.ptr(v), v.stride(0), v.stride(1), _lib.ptr(g), _lib.ptr(beta),
              _lib.ptr(s_in), s_in.stride(0), _lib.ptr(s_out), s_out.stride(0) if s_out is not None else 0,
              _lib.ptr(ids64), _lib.ptr(inter), _lib.ptr(out), Bsz, T, Hk, Hv, D, float(scale),
              int(bool(l2norm)), _lib.ptr(src_states if src_acc is not None else None), _lib.ptr(src_acc),
              src_T, _stream(dev))
    return out


def recurrent_gdn_inplace(q, k, v, g, beta, s_pool, ids):
    """q/k/v [bs, 1, H, D] bf16, g/beta [bs, 1, H]; updates s_pool rows `ids`
    in place, returns out [bs, 1, H, DV] bf16.  q/k/v may be strided views
    of the conv output; s_pool a per-layer view of the state pool.
    Reference: recurrent_gdn_inplace, nanovllm/models/qwen3_5.py:597-613."""
    bs, _, H, DK = k.shape
    DV = v.shape[-1]
    assert q.stride(2) == DK and k.stride(2) == DK and v.stride(2) == DV
    assert g.is_contiguous() and beta.is_contiguous()
    assert s_pool.stride(1) == DK * DV and s_pool.stride(2) == DV and s_pool.stride(3) == 1
    return _recurrent(q, k, v, g, beta, s_pool, s_pool, ids, None, None, True)


# The decode kernel splits each head's columns over NVB workgroups when the
# batch has few (sequence, head) tiles (NVB 1 from B * Hv >= 2048); the split
# changes the summation order of S^T k, so whole-head and split runs differ
# in the last bits.  Its fused norm epilogue needs whole heads.
WHOLE_HEAD_TILES = 2048


def recurrent_decode_fused(qk, mixed, conv_pool, conv_weight, b, a, a_log, dt_bias, s_pool, ids, Hk, Hv, D,
                           scale=None, z=None, norm_weight=None, eps=1e-6, fuse_norm=None):
    """The decode step after the q/k conv, in one kernel: the gates from a, b,
    the v channels' conv1d + SiLU (their conv state rolled in place at `ids`)
    and the in-place recurrent update.  qk [B, 2*Hk*D] is conv_decode_step's
    output for the q and k channels; mixed [B, C] the raw rows; conv_pool
    [slots, C, 3] and s_pool [slots, Hv, D, D] per-layer pool views; b, a
    [B, Hv] bf16.  Returns out [B, 1, Hv, D] bf16, the same bits as
    fused_g_beta -> conv_decode_step -> recurrent_gdn_inplace
    (nanovllm/models/qwen3_5.py:1008-1030).  With z ([B, Hv*D] bf16, head
    dim contiguous) and norm_weight ([D]) `out` is the layer's gated RMSNorm
    of it (qwen3_5.py:1083-1085), the same bits as rms_norm_gated on the core
    output: in the same kernel when B * Hv >= WHOLE_HEAD_TILES (the kernel
    runs whole heads then anyway), else as a second launch (fuse_norm=True
    forces the one-kernel form, whose core output is then the whole-head
    kernel's).

    qk=None (Hk == Hv only): the q and k channels' decode conv runs in the
    kernel as well, their conv states rolled there (the whole step in one
    launch, whole heads per workgroup); the same bits as conv_decode_step on
    those channels followed by the call above with its output."""
    dev = _check_cuda(qk, mixed, conv_pool, conv_weight, b, a, a_log, dt_bias, s_pool, ids, z, norm_weight)
    for t, nm in ((qk, "qk"), (mixed, "mixed"), (conv_pool, "conv_pool"), (b, "b"), (a, "a")):
        if t is not None:
            _bf16(t, nm)
    B, C = mixed.shape
    kd = Hk * D
    assert C == 2 * kd + Hv * D
    if qk is None:
        assert Hk == Hv, "the q/k conv runs in the decode kernel only with one key head per value head"
        fuse_norm = True   # whole heads per workgroup in any case
    else:
        assert qk.shape == (B, 2 * kd) and qk.stride(1) == 1
    assert mixed.stride(1) == 1 and conv_pool.stride(2) == 1
    w = conv_weight.reshape(C, -1)
    assert w.shape[1] == 4
    w = w.contiguous()
    b, a = b.contiguous(), a.contiguous()
    assert b.shape == (B, Hv) and a.shape == (B, Hv)
    assert a_log.dtype == dt_bias.dtype and a_log.dtype in (torch.bfloat16, torch.float32)
    a_log, dt_bias = a_log.contiguous(), dt_bias.contiguous()
    assert a_log.numel() == Hv and dt_bias.numel() == Hv
    assert _state_view_ok(s_pool, Hv, D)
    ids64 = ids.to(torch.int64).contiguous()
    assert ids64.shape == (B,), "one slot id per row"
    if z is not None and not (fuse_norm if fuse_norm is not None else B * Hv >= WHOLE_HEAD_TILES):
        core = recurrent_decode_fused(qk, mixed, conv_pool, conv_weight, b, a, a_log, dt_bias, s_pool, ids, Hk, Hv,
                                      D, scale)
        return rms_norm_gated(core, z.reshape(B, 1, Hv, D), norm_weight, eps)
    nw = None
    if z is not None:
        _bf16(z, "z")
        z = z.reshape(B, Hv * D)
        if z.stride(1) != 1 or z.stride(0) % 4:
            z = z.contiguous()
        assert norm_weight is not None and norm_weight.numel() == D
        nw = norm_weight.to(torch.bfloat16).contiguous()
    out = torch.empty(B, 1, Hv, D, dtype=mixed.dtype, device=mixed.device)
    if scale is None:
        scale = D ** -0.5
    q_ptr, k_ptr, sqk = (None, None, 0) if qk is None else (_lib.ptr(qk), _lib.ptr(qk[:, kd:]), qk.stride(0))
    _lib.call("gdn_recurrent_decode_fused", q_ptr, sqk, k_ptr, sqk,
              _lib.ptr(mixed), mixed.stride(0), _lib.ptr(conv_pool), conv_pool.stride(0), conv_pool.stride(1),
              _lib.ptr(w), _lib.ptr(a), _lib.ptr(b), _lib.ptr(a_log), _lib.ptr(dt_bias),
              int(a_log.dtype == torch.float32), _lib.ptr(s_pool), s_pool.stride(0), _lib.ptr(ids64),
              _lib.ptr(out), B, Hk, Hv, D, float(scale), 1, _lib.ptr(z), z.stride(0) if z is not None else 0,
              _lib.ptr(nw), float(eps), _stream(dev))
    return out


def recurrent_gated_delta_rule(query, key, value, g=None, beta=None, initial_state=None, scale=None,
                               output_final_state=True, use_qk_l2norm_in_kernel=True, **kwargs):
    """Gathered-state recurrent rule (T >= 1 tokens per row).
    query/key [B, T, Hk, D], value [B, T, Hv, D], g/beta [B, T, Hv];
    initial_state [B, Hv, D, D] fp32 or None (zeros).  Returns
    (out [B, T, Hv, D], final [B, Hv, D, D] or None).
    Reference: recurrent_gated_delta_rule / _torch_recurrent_gated_delta_rule,
    nanovllm/models/qwen3_5.py:230-238, :616-651."""
    Bsz, T, Hk, D = key.shape
    Hv = value.shape[2]
    if initial_state is None:
        s_in = torch.zeros(Bsz, Hv, D, D, dtype=torch.float32, device=value.device)
    else:
        s_in = initial_state if _state_view_ok(initial_state, Hv, D) else initial_state.float().contiguous()
    s_out = torch.empty(Bsz, Hv, D, D, dtype=torch.float32, device=value.device) if output_final_state else None
    out = _recurrent(query, key, value, g.contiguous(), beta.contiguous(), s_in, s_out, None, None, scale,
                     use_qk_l2norm_in_kernel)
    return out, s_out


def recurrent_gdn_multitoken(q, k, v, g, beta, s_pool, ids, intermediate_states=None, src_states=None,
                             src_accepted=None):
    """Speculative-verify decode: T draft tokens per sequence against the
    slot pool.  q/k [B, T, Hk, D], v [B, T, Hv, D], g/beta [B, T, Hv].
    With intermediate_states ([B, T, Hv, D, D] fp32) the per-token states
    are written there and the pool is left untouched (commit_states picks
    the accepted prefix); without it the pool is advanced by all T tokens.
    src_states / src_accepted: row b starts from src_states[b,
    src_accepted[b] - 1] where src_accepted[b] >= 1 instead of its pool row
    (the previous verify's accepted state, not yet committed; see
    SpecVerify).
    Returns out [B, T, Hv, D].  (No reference counterpart: spec decode is
    disabled for qwen3_5, nanovllm/config.py:84.)"""
    s_out = None if intermediate_states is not None else s_pool
    return _recurrent(q, k, v, g, beta, s_pool, s_out, ids, intermediate_states, None, True, src_states,
                      src_accepted)


class SpecVerify:
    """Speculative-verify steps of one GDN layer with the rollback folded
    into the next step instead of a commit copy.

    verify() runs the T-token kernel and keeps every per-token state in an
    [B, T, Hv, D, D] buffer; accept(accepted) records how many of them each
    row keeps (device int64 tensor, values 1..T: the first token of a draft
    block is the target model's own and always kept).  The next verify()
    starts row b from state [b, accepted[b] - 1] directly (the kernel reads it
    where the pool row would be read, and each state is read before the step
    overwrites it in place), so nothing runs between steps.  commit() writes
    the accepted states into the pool, for any other user of the slots (a
    plain decode, a prefill, or a sequence that leaves the batch).  The rows
    keep their order across steps (ids the same); a different batch must
    commit() first.  (No reference counterpart: spec decode is disabled for
    qwen3_5, nanovllm/config.py:84.)"""

    def __init__(self, s_pool: torch.Tensor):
        self.s_pool = s_pool
        self.inter = None
        self.ids = None
        self.accepted = None      # [B] int64 of the last verify, until the next verify or commit()

    def verify(self, q, k, v, g, beta, ids):
        Bsz, T = k.shape[:2]
        Hv, D = v.shape[2], v.shape[3]
        if self.accepted is not None:
            assert self.ids is not None and torch.equal(self.ids, ids), "the batch changed: commit() first"
        if self.inter is None or self.inter.shape != (Bsz, T, Hv, D, D):
            assert self.accepted is None, "the draft length changed: commit() first"
            self.inter = torch.empty(Bsz, T, Hv, D, D, dtype=torch.float32, device=v.device)
        out = recurrent_gdn_multitoken(q, k, v, g, beta, self.s_pool, ids, self.inter,
                                       self.inter if self.accepted is not None else None, self.accepted)
        self.ids = ids
        self.accepted = None      # the pool plus this step's states, until accept()
        return out

    def accept(self, accepted: torch.Tensor) -> None:
        """accepted [B] int64 (device): tokens kept per row, 1..T.  A row
        whose count lies outside 1..T starts the next verify from its pool
        row (the last committed state), as commit() leaves it untouched."""
        assert self.inter is not None and self.accepted is None, "accept() follows one verify()"
        assert accepted.dtype == torch.int64 and accepted.shape == (self.inter.shape[0],)
        assert accepted.device == self.inter.device and accepted.is_contiguous()
        self.accepted = accepted

    def commit(self) -> None:
        """Write the accepted states into the pool rows (a no-op when
        nothing is pending)."""
        if self.accepted is None:
            return
        commit_states(self.s_pool, self.ids, self.inter, self.accepted)
        self.accepted = None


def commit_states(s_pool, ids, intermediate_states, accepted):
    """s_pool[ids[b]] <- intermediate_states[b, accepted[b] - 1]
    (accepted in [1, T]; 0 leaves the slot unchanged)."""
    dev = _check_cuda(s_pool, ids, intermediate_states, accepted)
    Bsz, T, Hv, D, _ = intermediate_states.shape
    assert _state_view_ok(s_pool, Hv, D) and intermediate_states.is_contiguous()
    ids64 = ids.to(torch.int64).contiguous()
    acc = accepted.to(torch.int32).contiguous()
    assert ids64.shape == (Bsz,) and acc.shape == (Bsz,), "one slot id and one accepted length per row"
    _lib.call("gdn_state_commit", _lib.ptr(s_pool), s_pool.stride(0), _lib.ptr(ids64),
              _lib.ptr(intermediate_states), _lib.ptr(acc), Bsz, T, Hv, D, _stream(dev))


def state_tile_pass(s_pool: torch.Tensor, ids: torch.Tensor) -> None:
    """Measurement pass (no reference counterpart): reads every state tile
    s_pool[ids[b], h] and writes it back unchanged, with the one-token decode
    kernel's tile layout and cache policy -- that step's state traffic without
    its arithmetic.  s_pool [slots, Hv, D, D] fp32 (any slot stride)."""
    dev = _check_cuda(s_pool, ids)
    assert _state_view_ok(s_pool, s_pool.shape[1], s_pool.shape[-1])
    ids64 = ids.to(torch.int64).contiguous()
    _lib.call("gdn_state_tile_pass", _lib.ptr(s_pool), s_pool.stride(0), _lib.ptr(ids64), ids64.numel(),
              s_pool.shape[1], s_pool.shape[-1], _stream(dev))


def state_tile_copy(src_pool: torch.Tensor, dst_pool: torch.Tensor, ids: torch.Tensor) -> None:
    """Measurement pass (no reference counterpart): state_tile_pass with each
    tile written to dst_pool[ids[b], h] instead of back in place (the same
    launch shape, layout and cache policy).  Both pools [slots, Hv, D, D]
    fp32 with the same slot stride, not overlapping."""
    dev = _check_cuda(src_pool, dst_pool, ids)
    assert src_pool.shape == dst_pool.shape and src_pool.stride(0) == dst_pool.stride(0)
    assert _state_view_ok(src_pool, src_pool.shape[1], src_pool.shape[-1])
    assert _state_view_ok(dst_pool, dst_pool.shape[1], dst_pool.shape[-1])
    ids64 = ids.to(torch.int64).contiguous()
    _lib.call("gdn_state_tile_copy", _lib.ptr(src_pool), _lib.ptr(dst_pool), src_pool.stride(0), _lib.ptr(ids64),
              ids64.numel(), src_pool.shape[1], src_pool.shape[-1], _stream(dev))


# ------------------------------------------------------------- projections --
def linear(x: torch.Tensor, weight: torch.Tensor, out: torch.Tensor | None = None,
           gates: dict | None = None) -> torch.Tensor:
    """F.linear(x, weight) without bias on the bf16 matrix cores (fp32
    accumulation): x [..., K] bf16 (last dim contiguous), weight [N, K] bf16
    (nn.Linear layout).  Returns [..., N] bf16 (or writes `out`, a [M, N]
    view with contiguous rows).  gates: {"gate_col", "A_log", "dt_bias"}
    (and the Hv of A_log): the columns [gate_col, gate_col + Hv) are the b
    projection and the next Hv the a projection; beta (bf16) and g (fp32)
    [M, Hv] of them are also computed and returned as (y, g, beta), equal to
    fused_g_beta on those columns.
    Reference: ColumnParallelLinear / RowParallelLinear.forward,
    nanovllm/layers/linear.py:74-75, :154-158 (tp = 1)."""
    dev = _check_cuda(x, weight, out)
    _bf16(x, "x")
    _bf16(weight, "weight")
    K = x.shape[-1]
    N = weight.shape[0]
    assert weight.shape[1] == K
    x2 = x.reshape(-1, K)
    if x2.stride(1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    w = weight if (weight.stride(1) == 1 and weight.stride(0) % 8 == 0 and weight.data_ptr() % 16 == 0) \
        else weight.contiguous()
    M = x2.shape[0]
    if out is None:
        y = torch.empty(M, N, dtype=torch.bfloat16, device=x.device)
    else:
        _bf16(out, "out")
        assert out.shape == (M, N) and out.stride(1) == 1
        y = out
    g = beta = None
    a_log = dt_bias = None
    gate_col = Hv = 0
    if gates is not None:
        a_log, dt_bias = gates["A_log"], gates["dt_bias"]
        if a_log.dtype != dt_bias.dtype or a_log.dtype not in (torch.bfloat16, torch.float32):
            a_log, dt_bias = a_log.float(), dt_bias.float()
        a_log, dt_bias = a_log.contiguous(), dt_bias.contiguous()
        Hv = a_log.numel()
        gate_col = int(gates["gate_col"])
        g = torch.empty(M, Hv, dtype=torch.float32, device=x.device)
        beta = torch.empty(M, Hv, dtype=torch.bfloat16, device=x.device)
    _lib.call("gdn_gemm_bf16", _lib.ptr(x2), x2.stride(0), _lib.ptr(w), w.stride(0), _lib.ptr(y), y.stride(0),
              M, N, K, _lib.ptr(g), _lib.ptr(beta), _lib.ptr(a_log), _lib.ptr(dt_bias),
              int(a_log is not None and a_log.dtype == torch.float32), gate_col, Hv, _stream(dev))
    y = y.view(*x.shape[:-1], N) if out is None else y
    return y if gates is None else (y, g, beta)


def linear_cols(x: torch.Tensor, weight: torch.Tensor, widths: list[int],
                gates: dict | None = None):
    """linear(x, weight) with the output's columns split into len(widths)
    (1-4) contiguous tensors [M, widths[s]] (sum(widths) == weight rows;
    every boundary a multiple of 16): the same values as linear's columns.
    For the GDN layer's in_proj over its four concatenated weights, so that
    the qkv, z, b and a parts come out as tensors of their own, as the
    reference's separate projections produce them
    (nanovllm/models/qwen3_5.py:929-939).  gates: as in linear (gate_col
    counts the concatenated columns).  Returns the list of parts, and with
    gates (parts, g, beta)."""
    dev = _check_cuda(x, weight)
    _bf16(x, "x")
    _bf16(weight, "weight")
    K = x.shape[-1]
    N = weight.shape[0]
    assert weight.shape[1] == K and sum(widths) == N and 1 <= len(widths) <= 4
    x2 = x.reshape(-1, K)
    if x2.stride(1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    w = weight if (weight.stride(1) == 1 and weight.stride(0) % 8 == 0 and weight.data_ptr() % 16 == 0) \
        else weight.contiguous()
    M = x2.shape[0]
    parts = [torch.empty(M, wd, dtype=torch.bfloat16, device=x.device) for wd in widths]
    ends, e = [], 0
    for wd in widths:
        e += wd
        ends.append(e)
    n = len(widths)
    c_arr = (ctypes.c_void_p * n)(*[p.data_ptr() for p in parts])
    ld_arr = (ctypes.c_int64 * n)(*[p.stride(0) for p in parts])
    end_arr = (ctypes.c_int * n)(*ends)
    g = beta = None
    a_log = dt_bias = None
    gate_col = Hv = 0
    if gates is not None:
        a_log, dt_bias = gates["A_log"], gates["dt_bias"]
        if a_log.dtype != dt_bias.dtype or a_log.dtype not in (torch.bfloat16, torch.float32):
            a_log, dt_bias = a_log.float(), dt_bias.float()
        a_log, dt_bias = a_log.contiguous(), dt_bias.contiguous()
        Hv = a_log.numel()
        gate_col = int(gates["gate_col"])
        g = torch.empty(M, Hv, dtype=torch.float32, device=x.device)
        beta = torch.empty(M, Hv, dtype=torch.bfloat16, device=x.device)
    _lib.call("gdn_gemm_bf16_cols", _lib.ptr(x2), x2.stride(0), _lib.ptr(w), w.stride(0), M, N, K, n, c_arr,
              ld_arr, end_arr, _lib.ptr(g), _lib.ptr(beta), _lib.ptr(a_log), _lib.ptr(dt_bias),
              int(a_log is not None and a_log.dtype == torch.float32), gate_col, Hv, _stream(dev))
    parts = [p.view(*x.shape[:-1], p.shape[1]) for p in parts]
    return parts if gates is None else (parts, g, beta)


# -------------------------------------------------------------- gated norm --
def rms_norm_gated(hidden_states: torch.Tensor, gate: torch.Tensor, weight: torch.Tensor,
                   eps: float) -> torch.Tensor:
    """y = bf16(float(bf16(w * bf16(x * rsqrt(mean(x^2) + eps)))) * silu(float(z)))
    over the last dim.  hidden_states / gate [..., H, D] bf16 (head dim
    contiguous, rows of a token contiguous).
    Reference: _rms_gated_forward, nanovllm/models/qwen3_5.py:121-131."""
    dev = _check_cuda(hidden_states, gate, weight)
    _bf16(hidden_states, "hidden_states")
    _bf16(gate, "gate")
    D = hidden_states.shape[-1]
    assert hidden_states.dim() >= 2 and gate.shape == hidden_states.shape
    w = weight.to(torch.bfloat16).contiguous()
    assert w.numel() == D
    H = hidden_states.shape[-2]
    x2 = hidden_states.reshape(-1, H, D)
    z2 = gate.reshape(-1, H, D)
    if x2.stride(2) != 1 or x2.stride(1) != D:
        x2 = x2.contiguous()
    if z2.stride(2) != 1 or z2.stride(1) != D:
        z2 = z2.contiguous()
    n_tok, H, _ = x2.shape
    y = torch.empty(n_tok, H, D, dtype=hidden_states.dtype, device=hidden_states.device)
    _lib.call("gdn_rmsnorm_gated", _lib.ptr(x2), x2.stride(0), _lib.ptr(z2), z2.stride(0), _lib.ptr(w),
              _lib.ptr(y), n_tok, H, D, float(eps), _stream(dev))
    return y.view(hidden_states.shape)


def rms_norm_gated_ranges(hidden_states: torch.Tensor, gate: torch.Tensor, weight: torch.Tensor, eps: float,
                          out: torch.Tensor, ranges: torch.Tensor, n_sel_tok: int) -> None:
    """rms_norm_gated on the tokens of some ranges only, into `out` (the same
    arithmetic, rows at the tokens' positions).  hidden_states / gate / out
    [N, H, D] bf16 with head-contiguous rows; ranges int64 [3 * n] on the
    device: (first token, token count, selected tokens before it)."""
    dev = _check_cuda(hidden_states, gate, weight, out, ranges)
    _bf16(hidden_states, "hidden_states")
    _bf16(gate, "gate")
    N, H, D = hidden_states.shape
    assert gate.shape == hidden_states.shape and out.shape == hidden_states.shape and out.is_contiguous()
    assert hidden_states.stride(2) == 1 and hidden_states.stride(1) == D
    assert gate.stride(2) == 1 and gate.stride(1) == D
    w = weight.to(torch.bfloat16).contiguous()
    _lib.call("gdn_rmsnorm_gated_ranges", _lib.ptr(hidden_states), hidden_states.stride(0), _lib.ptr(gate),
              gate.stride(0), _lib.ptr(w), _lib.ptr(out), N, _lib.ptr(ranges), ranges.numel() // 3, n_sel_tok, H,
              D, float(eps), _stream(dev))


class Qwen3_5RMSNormGated(torch.nn.Module):
    """Delta-net output norm on the value head dim, gated by silu(z).
    Reference: Qwen3_5RMSNormGated, nanovllm/models/qwen3_5.py:697-709."""

    def __init__(self, hidden_size: int, eps: float = 1e-6):
        super().__init__()
        self.weight = torch.nn.Parameter(torch.ones(hidden_size))
        self.eps = eps

    def forward(self, hidden_states: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
        return rms_norm_gated(hidden_states, gate, self.weight, self.eps)
