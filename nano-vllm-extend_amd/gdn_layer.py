"""Host-side mirror of the Qwen3.5 GDN layer between its projections.

GatedDeltaNetCore reproduces the dispatch and data flow of
Qwen3_5GatedDeltaNet.forward / _gdn_prefill_varlen / _gdn_padded
(nanovllm/models/qwen3_5.py:864-1087) from the projection outputs
(mixed qkv, z, b, a) to the gated-norm output that feeds out_proj, on the
HIP kernels of this package.  The in/out projection GEMMs are the caller's.

A/B switches (read from the environment at construction, as the reference
reads them at import; "1" = HIP kernel):
  NANOVLLM_GDN_GBETA    fused g/beta kernel  | "0": eager torch chain (:936-937)
  NANOVLLM_CONV_TRITON  conv kernels         | "0": F.conv1d chain (:1020-1024, :1057-1065)
  NANOVLLM_GDN_INPLACE  in-place decode      | "0": gather -> recurrent kernel -> scatter (:1028-1030)
  NANOVLLM_GDN_VARLEN   varlen prefill       | "0": padded prefill path (:1032-1077)
  FLA_CHUNK, FLA_RECURRENT                   | "0" selects the reference's own pure-torch ports
                                               (qwen3_5.py:152-227, :616-651).  This core is
                                               the package's own and carries no copy of them,
                                               so here "0" raises; installed into the reference
                                               module (integration.install) the switches keep
                                               their meaning and run the module's ports.
The varlen prefill reads and writes the state pools at the slot ids
directly (no gather / scatter copies).
"""
from __future__ import annotations

import contextlib
import os
from dataclasses import dataclass

import torch
import torch.nn.functional as F

from . import ops
from .state_pool import varlen_meta


@dataclass
class Switches:
    gbeta: bool = True
    conv_kernel: bool = True
    inplace: bool = True
    varlen: bool = True
    fla_chunk: bool = True
    fla_recurrent: bool = True
    fused_prefill: bool = True
    split_state: bool = False
    fused_decode: bool = True

    @classmethod
    def from_env(cls) -> "Switches":
        e = os.environ.get
        return cls(gbeta=e("NANOVLLM_GDN_GBETA", "1") == "1",
                   conv_kernel=e("NANOVLLM_CONV_TRITON", "1") == "1",
                   inplace=e("NANOVLLM_GDN_INPLACE", "1") == "1",
                   varlen=e("NANOVLLM_GDN_VARLEN", "1") == "1",
                   fla_chunk=e("FLA_CHUNK", "1") == "1",
                   fla_recurrent=e("FLA_RECURRENT", "1") == "1",
                   fused_prefill=e("NANOVLLM_GDN_FUSED_PREFILL", "1") == "1",
                   split_state=e("NANOVLLM_GDN_SPLIT_STATE", "0") == "1",
                   fused_decode=e("NANOVLLM_GDN_FUSED_DECODE", "1") == "1")


# State-pass split policy (off by default: measured at config 1 the split
# costs more than it saves -- each event between the prep and the state
# launches delays the stream by ~6 us, the long sequence's chain slows under
# the concurrent traffic, and the bandwidth-bound norm overlaps only the last
# ~18 us of the state pass).  The state pass of a varlen group lasts as long
# as its longest sequence's chain (~1.9 us per 64-token chunk when the GPU is
# full); the gated norm streams ~768 B per token and head (~5.4 TB/s).  With
# the k longest sequences on one stream and the rest on another, the rest's
# norm overlaps the long sequences' chains; k is chosen to minimise
# max(T_long, T_rest + norm_rest) + norm_long.
_CHUNK_US = 1.9
_NORM_US_PER_TOKEN_HEAD = 768 / 5.4e6

# the last plan only (its pinned host tensors are reused while the batch
# composition repeats, as by the layers of one step; nothing accumulates)
_SPLIT_CACHE: dict = {}


def late_split(lens_q: list[int], Hv: int):
    """(late flags per sequence, (early token ranges, count), (late ranges,
    count)) with the ranges as host int64 [3 * n] (first token, tokens,
    selected tokens before), or None when splitting gains under 5 us."""
    key = (tuple(lens_q), Hv)
    if key in _SPLIT_CACHE:
        return _SPLIT_CACHE[key]
    _SPLIT_CACHE.clear()
    n = len(lens_q)
    res = None
    if 2 <= n <= 64 and sum(lens_q) >= 4096:
        ch = [(l + 63) // 64 for l in lens_q]
        order = sorted(range(n), key=lambda r: -ch[r])
        norm = lambda toks: toks * Hv * _NORM_US_PER_TOKEN_HEAD
        whole = ch[order[0]] * _CHUNK_US + norm(sum(lens_q))
        best, best_k = whole - 5.0, 0
        for k in range(1, n):
            long_toks = sum(lens_q[r] for r in order[:k])
            t = max(ch[order[0]] * _CHUNK_US, ch[order[k]] * _CHUNK_US + norm(sum(lens_q) - long_toks)) \
                + norm(long_toks)
            if t < best:
                best, best_k = t, k
        if best_k:
            late = [False] * n
            for r in order[:best_k]:
                late[r] = True
            starts = [0]
            for l in lens_q:
                starts.append(starts[-1] + l)

            def ranges(flag):
                rows, before = [], 0
                for r in range(n):
                    if late[r] == flag and lens_q[r]:
                        rows += [starts[r], lens_q[r], before]
                        before += lens_q[r]
                t = torch.tensor(rows, dtype=torch.int64)
                return (t.pin_memory() if torch.cuda.is_available() else t), before

            res = (late, ranges(False), ranges(True))
    _SPLIT_CACHE[key] = res
    return res


class GatedDeltaNetCore:
    """GDN layer core for one layer's parameters.

    conv_weight [C, K] (or [C, 1, K]) bf16 with C = 2*Hk*D + Hv*D;
    A_log, dt_bias [Hv]; norm_weight [D]; eps = rms_norm_eps."""

    # Prefill segment budget (tokens per padded chunk-kernel call), as the
    # reference uses with its fused chunk kernel (qwen3_5.py:853-862).
    PREFILL_SEGMENT_TOKENS = 16384

    def __init__(self, num_k_heads: int, num_v_heads: int, head_dim: int, conv_weight: torch.Tensor,
                 A_log: torch.Tensor, dt_bias: torch.Tensor, norm_weight: torch.Tensor,
                 eps: float = 1e-6, switches: Switches | None = None):
        assert num_v_heads % num_k_heads == 0
        self.Hk, self.Hv, self.D = num_k_heads, num_v_heads, head_dim
        self.key_dim = num_k_heads * head_dim
        self.value_dim = num_v_heads * head_dim
        self.conv_dim = 2 * self.key_dim + self.value_dim
        self.K = conv_weight.shape[-1]
        self.conv_w = conv_weight.reshape(self.conv_dim, self.K)
        self.A_log, self.dt_bias, self.norm_w, self.eps = A_log, dt_bias, norm_weight, eps
        self.sw = switches or Switches.from_env()
        # Optional per-kernel timer: an object with start(name) / stop(name)
        # that records device events on the current stream (bench.py).
        self.timer = None
        if not self.sw.fla_chunk:
            raise NotImplementedError("FLA_CHUNK=0 selects the reference's pure-torch chunk port, "
                                      "which is not part of this build")
        if not self.sw.inplace and not self.sw.fla_recurrent:
            raise NotImplementedError("FLA_RECURRENT=0 selects the reference's pure-torch recurrent "
                                      "port, which is not part of this build")

    @contextlib.contextmanager
    def _timed(self, name: str):
        if self.timer is None:
            yield
            return
        self.timer.start(name)
        yield
        self.timer.stop(name)

    def _to(self, dev):
        if self.conv_w.device != dev:
            self.conv_w = self.conv_w.to(dev)
            self.A_log = self.A_log.to(dev)
            self.dt_bias = self.dt_bias.to(dev)
            self.norm_w = self.norm_w.to(dev)

    # ---------------------------------------------------------------- gates --
    def _g_beta(self, b, a, mask, gb=None):
        """g (fp32), beta (bf16) of the rows b, a; gb: the same already
        computed (the in_proj GEMM's gate epilogue, bit-equal to the gate
        kernel), padded rows of g zero under mask."""
        if gb is not None:
            g, beta = gb
            return (g if mask is None else g.masked_fill(~mask.unsqueeze(-1), 0.0)), beta
        if self.sw.gbeta:
            with self._timed("g_beta"):
                return ops.fused_g_beta(b, a, self.A_log, self.dt_bias, mask)
        beta = b.sigmoid()
        g = -self.A_log.float().exp() * F.softplus(a.float() + self.dt_bias.float())
        if mask is not None:
            g = g.masked_fill(~mask.unsqueeze(-1), 0.0)
        return g, beta

    def _norm(self, core, z):
        with self._timed("rmsnorm_gated"):
            return ops.rms_norm_gated(core, z, self.norm_w, self.eps)

    # --------------------------------------------------------------- decode --
    def decode(self, mixed, z, b, a, ids, conv_cache, s_cache, gb=None):
        """One token per row (the T == 1 branch of _gdn_padded, qwen3_5.py:1008-1030).
        mixed [B, C], z [B, Hv*D], b/a [B, Hv]; pools are per-layer views.
        Returns core [B, Hv, D] bf16."""
        self._to(mixed.device)
        B = mixed.shape[0]
        Hk, Hv, D = self.Hk, self.Hv, self.D
        kd = self.key_dim
        if self.sw.fused_decode and self.sw.gbeta and self.sw.conv_kernel and self.sw.inplace and self.K == 4:
            if Hk == Hv and B * Hv >= ops.WHOLE_HEAD_TILES:
                # the whole step in one kernel: q/k/v conv, gates, recurrent
                # update and gated norm (the same results as the calls below)
                with self._timed("recurrent_decode"):
                    out = ops.recurrent_decode_fused(None, mixed, conv_cache, self.conv_w, b, a, self.A_log,
                                                     self.dt_bias, s_cache, ids, Hk, Hv, D, z=z,
                                                     norm_weight=self.norm_w, eps=self.eps)
                return out.view(B, Hv, D)
            # q/k conv, then gates + v conv + recurrent update + gated norm in
            # one kernel (the same results as the calls below)
            with self._timed("conv_decode"):
                qk = ops.conv_decode_step(mixed[:, :2 * kd], conv_cache[:, :2 * kd], ids, self.conv_w[:2 * kd])
            with self._timed("recurrent_decode"):
                out = ops.recurrent_decode_fused(qk, mixed, conv_cache, self.conv_w, b, a, self.A_log, self.dt_bias,
                                                 s_cache, ids, Hk, Hv, D, z=z, norm_weight=self.norm_w, eps=self.eps)
            return out.view(B, Hv, D)
        g, beta = self._g_beta(b.contiguous(), a.contiguous(), None, gb)
        if self.sw.conv_kernel:
            with self._timed("conv_decode"):
                y = ops.conv_decode_step(mixed, conv_cache, ids, self.conv_w)
        else:
            window = torch.cat([conv_cache[ids], mixed.unsqueeze(-1)], dim=-1)
            conv_cache[ids] = window[..., 1:]
            y = F.silu(F.conv1d(window, self.conv_w.unsqueeze(1), groups=self.conv_dim))[..., 0]
        q = y[:, :kd].view(B, 1, Hk, D)
        k = y[:, kd:2 * kd].view(B, 1, Hk, D)
        v = y[:, 2 * kd:].view(B, 1, Hv, D)
        g1, b1 = g.view(B, 1, Hv), beta.view(B, 1, Hv)
        if self.sw.inplace:
            with self._timed("recurrent_decode"):
                out = ops.recurrent_gdn_inplace(q, k, v, g1, b1, s_cache, ids)
        else:
            out, new_s = ops.recurrent_gated_delta_rule(q, k, v, g1, b1, s_cache[ids])
            s_cache[ids] = new_s
        return self._norm(out.view(B, Hv, D), z.view(B, Hv, D))

    # ------------------------------------------------------- varlen prefill --
    def prefill_varlen(self, mixed, z, b, a, lens_q, ids, conv_cache, s_cache, fresh=None, gb=None):
        """Varlen prefill group (_gdn_prefill_varlen, qwen3_5.py:922-965) with the
        conv and recurrent states read / written in the pools at `ids`.
        mixed [N, C], z [N, Hv*D], b/a [N, Hv].  fresh: optional bool [n],
        sequences that start from zero states (their slots need no zeroing
        beforehand, model_runner.py:305-322).  Returns core [N, Hv, D] bf16."""
        self._to(mixed.device)
        N = mixed.shape[0]
        Hk, Hv, D = self.Hk, self.Hv, self.D
        if self.sw.fused_prefill and self.sw.gbeta and self.sw.conv_kernel and self.K == 4:
            # gates + conv + chunk rule in one call (the same results as the
            # three calls below)
            _, _, cu64_cpu, cu64_gpu = varlen_meta(lens_q, mixed.device)
            split = late_split(lens_q, Hv) if self.sw.split_state else None
            if split is not None:
                return self._prefill_split(mixed, z, b, a, lens_q, ids, conv_cache, s_cache, fresh, cu64_cpu,
                                           cu64_gpu, split)
            with self._timed("conv_chunk_prefill"):
                o = ops.conv_chunk_prefill_varlen(mixed, conv_cache, self.conv_w, b, a, self.A_log, self.dt_bias,
                                                  cu64_gpu, s_cache, ids, Hk, Hv, D, fresh=fresh,
                                                  cu_seqlens_cpu=cu64_cpu)
            return self._norm(o, z.view(N, Hv, D))
        if fresh is not None:
            zero = ids[fresh.to(device=ids.device, dtype=torch.bool)]
            conv_cache[zero] = 0
            s_cache[zero] = 0
        g, beta = self._g_beta(b.contiguous(), a.contiguous(), None, gb)
        cu_gpu, lens_gpu, cu64_cpu, cu64_gpu = varlen_meta(lens_q, mixed.device)
        if self.sw.conv_kernel:
            with self._timed("conv_varlen"):
                q, k, v = ops.causal_conv_silu_varlen_parts(mixed, conv_cache, self.conv_w, lens_gpu, cu_gpu[:-1],
                                                            self.key_dim, state_ids=ids)
        else:
            q, k, v = self._conv_varlen_eager(mixed, lens_q, ids, conv_cache)
        with self._timed("chunk_prefill"):
            o, _ = ops.chunk_gated_delta_rule_varlen(q.view(N, Hk, D), k.view(N, Hk, D), v.view(N, Hv, D),
                                                     g, beta, cu64_gpu, s_cache, state_ids=ids,
                                                     final_state=s_cache, cu_seqlens_cpu=cu64_cpu)
        return self._norm(o, z.view(N, Hv, D))

    def _prefill_split(self, mixed, z, b, a, lens_q, ids, conv_cache, s_cache, fresh, cu64_cpu, cu64_gpu, split):
        """Fused prefill with the state pass split over two streams: the longest
        sequences on the current stream, the others on a side stream where
        their gated norm then runs while the long ones are still in the state
        kernel.  The same results as the one-stream path, bit for bit."""
        late, (r_early, n_early), (r_late, n_late) = split
        N = mixed.shape[0]
        Hk, Hv, D = self.Hk, self.Hv, self.D
        dev = mixed.device
        side = self._side_stream(dev)
        cur = torch.cuda.current_stream(dev)
        keep = []
        # The side stream's norm reads the output and the range tables: both are
        # allocated, and the tables copied, on the current stream before the
        # prep launch, whose completion the side stream waits for.
        y = torch.empty(N, Hv, D, dtype=torch.bfloat16, device=dev)
        zz = z.view(N, Hv, D)
        r_e = r_early.to(dev, non_blocking=True)
        r_l = r_late.to(dev, non_blocking=True)
        with self._timed("conv_chunk_prefill"):
            o, side_done = ops.conv_chunk_prefill_varlen(mixed, conv_cache, self.conv_w, b, a, self.A_log,
                                                         self.dt_bias, cu64_gpu, s_cache, ids, Hk, Hv, D,
                                                         fresh=fresh, cu_seqlens_cpu=cu64_cpu, late=late,
                                                         side_stream=side, keep=keep)
            cur.wait_event(side_done)   # (the long sequences' state pass is the longer one)
        with torch.cuda.stream(side):
            ops.rms_norm_gated_ranges(o, zz, self.norm_w, self.eps, y, r_e, n_early)
        with self._timed("rmsnorm_gated"):
            ops.rms_norm_gated_ranges(o, zz, self.norm_w, self.eps, y, r_l, n_late)
            cur.wait_stream(side)
        keep.extend([y, zz, r_e, r_l])
        return y

    def _side_stream(self, dev):
        if getattr(self, "_side", None) is None or self._side.device != dev:
            self._side = torch.cuda.Stream(dev)   # default priority
        return self._side

    def _conv_varlen_eager(self, mixed, lens_q, ids, conv_cache):
        """F.conv1d chain per sequence (the reference's NANOVLLM_CONV_TRITON=0 form)."""
        outs = []
        off = 0
        w = self.conv_w.unsqueeze(1)
        K = self.K
        for r, T in enumerate(lens_q):
            slot = ids[r:r + 1]
            window = torch.cat([conv_cache[slot], mixed[off:off + T].t().unsqueeze(0)], dim=-1)
            outs.append(F.silu(F.conv1d(window, w, groups=self.conv_dim))[0].t())
            conv_cache[slot] = window[..., -(K - 1):]
            off += T
        y = torch.cat(outs, dim=0)
        kd = self.key_dim
        return y[:, :kd].contiguous(), y[:, kd:2 * kd].contiguous(), y[:, 2 * kd:].contiguous()

    # ------------------------------------------------------- padded prefill --
    def prefill_padded(self, x, z, b, a, lens, ids, conv_cache, s_cache, gb=None):
        """Padded prefill over [n, T, .] rows (T > 1 branch of _gdn_padded,
        qwen3_5.py:1032-1077): T-segments thread the conv and recurrent
        states; padding rows are exact no-ops (g = 0, masked conv output).
        x [n, T, C], z [n, T, Hv*D], b/a [n, T, Hv], lens [n] (device).
        Returns core [n, T, Hv, D] bf16."""
        self._to(x.device)
        n, T, C = x.shape
        Hk, Hv, D, K = self.Hk, self.Hv, self.D, self.K
        mask = torch.arange(T, device=x.device) < lens.unsqueeze(1)
        g, beta = self._g_beta(b.contiguous(), a.contiguous(), mask, gb)
        seg = max(1, self.PREFILL_SEGMENT_TOKENS // n)
        conv_states = conv_cache[ids]
        state = s_cache[ids]
        outs = []
        kd = self.key_dim
        for t0 in range(0, T, seg):
            t1 = min(t0 + seg, T)
            m = t1 - t0
            mixed = x[:, t0:t1].transpose(1, 2)                       # [n, C, m] strided view
            r = lens - t0
            valid = r > 0
            if self.sw.conv_kernel:
                endp = r.clamp(min=-1, max=m).to(torch.int32)
                mixed = ops.causal_conv_silu(mixed, conv_states, self.conv_w, endp)
                conv_cache[ids[valid]] = conv_states[valid]
            else:
                window = torch.cat([conv_states, mixed], dim=-1)
                mixed = F.silu(F.conv1d(window, self.conv_w.unsqueeze(1), groups=self.conv_dim))
                starts = r.clamp(min=0, max=m)
                cols = starts.view(n, 1, 1) + torch.arange(K - 1, device=x.device, dtype=torch.int64)
                sel = window.gather(-1, cols.expand(n, window.size(1), K - 1))
                conv_cache[ids[valid]] = sel[valid]
                conv_states = window[..., -(K - 1):]
            mixed = mixed * mask[:, t0:t1].unsqueeze(1).to(mixed.dtype)
            q = mixed[:, :kd].transpose(1, 2).reshape(n, m, Hk, D)
            k = mixed[:, kd:2 * kd].transpose(1, 2).reshape(n, m, Hk, D)
            v = mixed[:, 2 * kd:].transpose(1, 2).reshape(n, m, Hv, D)
            o, state = ops.chunk_gated_delta_rule(q, k, v, g=g[:, t0:t1].contiguous(),
                                                  beta=beta[:, t0:t1].contiguous(), initial_state=state,
                                                  output_final_state=True, use_qk_l2norm_in_kernel=True)
            outs.append(o)
        s_cache[ids] = state
        out = torch.cat(outs, dim=1)                                  # [n, T, Hv, D]
        return self._norm(out, z.view(n, T, Hv, D))

    # ------------------------------------------------------------- dispatch --
    def forward(self, mixed, z, b, a, cu_seqlens_q, max_seqlen_q, ids, conv_cache, s_cache,
                lens_q: list[int] | None = None, gb=None):
        """Dispatch of Qwen3_5GatedDeltaNet.forward (qwen3_5.py:864-920) over a
        varlen step: all-decode -> decode; a contiguous decode prefix goes to
        the decode path and the rest to the varlen (or padded) prefill.
        mixed [N, C], z [N, Hv*D], b/a [N, Hv]; gb: optional (g [N, Hv] fp32,
        beta [N, Hv] bf16) already computed from b, a (used by the paths that
        would run the gate kernel).  Returns [N, Hv*D] bf16."""
        rows = (lambda i, j: None) if gb is None else (lambda i, j: (gb[0][i:j], gb[1][i:j]))
        N = mixed.shape[0]
        T = int(max_seqlen_q)
        if T == 1:
            return self.decode(mixed, z, b, a, ids, conv_cache, s_cache, gb=gb).view(N, self.value_dim)
        # per-sequence lengths on the device, formed only where a path reads
        # them (a decode step or a varlen prefill given lens_q launches nothing
        # for them)
        lens_dev = lambda: cu_seqlens_q[1:] - cu_seqlens_q[:-1]
        bs = cu_seqlens_q.shape[0] - 1
        if lens_q is None:
            lens_q = lens_dev().tolist()
        n1 = 0
        while n1 < bs and lens_q[n1] == 1:
            n1 += 1
        pre_ok = 0 < n1 < bs and min(lens_q[n1:]) > 1
        if n1 == 0 or pre_ok:
            parts = []
            off = 0
            if n1:
                parts.append(self.decode(mixed[:n1], z[:n1], b[:n1], a[:n1], ids[:n1], conv_cache,
                                         s_cache, gb=rows(0, n1)).view(n1, self.value_dim))
                off = n1
            if self.sw.varlen:
                parts.append(self.prefill_varlen(mixed[off:], z[off:], b[off:], a[off:], lens_q[off:],
                                                 ids[off:], conv_cache, s_cache,
                                                 gb=rows(off, N)).view(-1, self.value_dim))
            else:
                lens_p = lens_dev()[off:]
                Tp = T if off == 0 else max(lens_q[off:])
                parts.append(self._padded_varlen(mixed[off:], z[off:], b[off:], a[off:], lens_p, Tp, ids[off:],
                                                 conv_cache, s_cache, gb=rows(off, N)))
            # (one part: no concatenation, which would copy the whole output)
            return parts[0] if len(parts) == 1 else torch.cat(parts, dim=0)
        # len-1 rows that are not a contiguous prefix: one padded pass
        return self._padded_varlen(mixed, z, b, a, lens_dev(), T, ids, conv_cache, s_cache, gb=gb)

    def _padded_varlen(self, mixed, z, b, a, lens, T, ids, conv_cache, s_cache, gb=None):
        n = lens.shape[0]
        mask = torch.arange(T, device=mixed.device) < lens.unsqueeze(1)

        def pad(t):
            p = t.new_zeros(n, T, t.shape[-1])
            p[mask] = t
            return p

        gbp = None
        if gb is not None:
            # the gate kernel on padded rows: g = 0 there (mask), beta = sigmoid(0) = 0.5
            beta_p = gb[1].new_full((n, T, gb[1].shape[-1]), 0.5)
            beta_p[mask] = gb[1]
            gbp = (pad(gb[0]), beta_p)
        core = self.prefill_padded(pad(mixed), pad(z), pad(b), pad(a), lens, ids, conv_cache, s_cache, gb=gbp)
        return core.reshape(n, T, self.value_dim)[mask]


class GatedDeltaNetLayer:
    """The whole GDN mixer of one layer, projections included
    (Qwen3_5GatedDeltaNet, nanovllm/models/qwen3_5.py:786-1087, tp = 1):

      hidden [N, hidden] --in_proj--> mixed | z | b | a --core--> [N, Hv, D]
      --out_proj--> [N, hidden]

    in_proj is one GEMM over the four projection weights concatenated
    (in_proj_qkv [C, hidden], in_proj_z [Hv*D, hidden], in_proj_b [Hv, hidden],
    in_proj_a [Hv, hidden], :811-822), whose output rows hold mixed, z, b and a
    side by side; the core reads them as strided views (the fused prefill and
    decode kernels take the raw b and a and compute g / beta themselves; when a
    path would run the gate kernel instead, the GEMM's epilogue computes g and
    beta from the b and a columns and that path uses them).
    out_proj [hidden, Hv*D] (:838-839) runs on the gated norm's output.  Both
    GEMMs are ops.linear (bf16 matrix cores, fp32 accumulation)."""

    def __init__(self, w_qkv, w_z, w_b, w_a, w_out, num_k_heads: int, num_v_heads: int, head_dim: int,
                 conv_weight, A_log, dt_bias, norm_weight, eps: float = 1e-6, switches: Switches | None = None):
        self.core = GatedDeltaNetCore(num_k_heads, num_v_heads, head_dim, conv_weight, A_log, dt_bias, norm_weight,
                                      eps=eps, switches=switches)
        c = self.core
        assert w_qkv.shape[0] == c.conv_dim and w_z.shape[0] == c.value_dim
        assert w_b.shape[0] == num_v_heads and w_a.shape[0] == num_v_heads
        self.hidden = w_qkv.shape[1]
        self.w_in = torch.cat([w_qkv, w_z, w_b, w_a], dim=0).contiguous()
        self.w_out = w_out.contiguous()
        assert self.w_out.shape == (self.hidden, c.value_dim)
        self.timer = None

    @property
    def n_in(self) -> int:
        return self.w_in.shape[0]

    def _timed(self, name):
        t = self.timer
        if t is None:
            return contextlib.nullcontext()

        @contextlib.contextmanager
        def cm():
            t.start(name)
            yield
            t.stop(name)

        return cm()

    def gates_in_gemm(self) -> bool:
        """Whether a path of the core would run the gate kernel on in_proj's b
        and a columns (the fused prefill and decode compute the gates from the
        raw columns themselves); then in_proj's epilogue yields them instead."""
        sw, c = self.core.sw, self.core
        fused_ok = sw.gbeta and sw.conv_kernel and c.K == 4
        return sw.gbeta and not (fused_ok and sw.fused_prefill and sw.varlen and sw.fused_decode and sw.inplace)

    def project_in(self, hidden, gates: bool = False):
        """hidden [N, hidden] -> (mixed, z, b, a): one GEMM over the four
        concatenated weights whose output goes to four contiguous tensors,
        mixed [N, C], z [N, Hv*D], b and a [N, Hv] (rows of contiguous tensors
        read faster than columns of one wide buffer, and the gate readers take
        them without a copy); with gates, also (g, beta) of the b and a
        columns from the GEMM's epilogue (bit-equal to the gate kernel on
        them, qwen3_5.py:933-934), else None."""
        c = self.core
        C, V, Hv = c.conv_dim, c.value_dim, c.Hv
        widths = [C, V, Hv, Hv]
        with self._timed("in_proj"):
            if all(w % 16 == 0 for w in widths[:-1]):
                if gates:
                    (mixed, z, b, a), g, beta = ops.linear_cols(hidden, self.w_in, widths,
                                                                gates={"gate_col": C + V, "A_log": c.A_log,
                                                                       "dt_bias": c.dt_bias})
                    gb = (g, beta)
                else:
                    (mixed, z, b, a), gb = ops.linear_cols(hidden, self.w_in, widths), None
                return mixed, z, b, a, gb
            if gates:
                y, g, beta = ops.linear(hidden, self.w_in, gates={"gate_col": C + V, "A_log": c.A_log,
                                                                  "dt_bias": c.dt_bias})
                gb = (g, beta)
            else:
                y, gb = ops.linear(hidden, self.w_in), None
        return y[:, :C], y[:, C:C + V], y[:, C + V:C + V + Hv], y[:, C + V + Hv:], gb

    def forward(self, hidden, cu_seqlens_q, max_seqlen_q, ids, conv_cache, s_cache, lens_q=None):
        """Qwen3_5GatedDeltaNet.forward for one varlen step (qwen3_5.py:864-920):
        hidden [N, hidden] bf16 -> [N, hidden] bf16."""
        mixed, z, b, a, gb = self.project_in(hidden, gates=self.gates_in_gemm())
        self.core.timer = self.timer
        core = self.core.forward(mixed, z, b.contiguous(), a.contiguous(), cu_seqlens_q, max_seqlen_q, ids,
                                 conv_cache, s_cache, lens_q=lens_q, gb=gb)
        with self._timed("out_proj"):
            return ops.linear(core, self.w_out)
