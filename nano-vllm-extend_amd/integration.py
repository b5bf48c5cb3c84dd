"""Install the HIP kernels behind the reference model's own call sites.

`install(mod)` takes the already-imported reference module
`nanovllm.models.qwen3_5` and rebinds the module-level names its GDN layer
calls (nanovllm/models/qwen3_5.py:56-78, 345-365, 459-479, 546-613, 697-709)
so that Qwen3_5GatedDeltaNet runs on this package without any edit to the
layer code:

  fused_g_beta                 -> ops.fused_g_beta
  causal_conv_silu_varlen      -> ops.causal_conv_silu_varlen
  conv_decode_step             -> ops.conv_decode_step
  causal_conv_silu             -> ops.causal_conv_silu
  recurrent_gdn_inplace        -> ops.recurrent_gdn_inplace
  _fla_chunk / _fla_recurrent  -> ops.chunk_gated_delta_rule / ops.recurrent_gated_delta_rule
  _rms_gated_forward           -> ops.rms_norm_gated

and sets the feature flags the layer reads (_USE_FLA_CHUNK,
_USE_FLA_RECURRENT, _USE_GDN_VARLEN) from the same environment switches
(FLA_CHUNK, FLA_RECURRENT, NANOVLLM_GDN_VARLEN) the reference reads
(qwen3_5.py:74-75, :478-479).  The module's own dispatchers
chunk_gated_delta_rule / recurrent_gated_delta_rule (qwen3_5.py:140-149,
:230-238) stay bound: with a switch at "1" they call the rebound _fla_*
entry point (the HIP kernels), with FLA_CHUNK=0 / FLA_RECURRENT=0 they run
the module's own pure-torch ports, exactly as in the reference.  _HAS_FLA is
set only when one of the two switches is on (this package then provides the
fla entry points); with both off it keeps the module's value.

With NANOVLLM_GDN_FUSED_PREFILL=1 (the default) it further replaces the
method Qwen3_5GatedDeltaNet._gdn_prefill_varlen (qwen3_5.py:922-965) with
one whose gates, conv and chunk rule are the single fused call
ops.conv_chunk_prefill_varlen (the same results as the three calls the
method makes, bit for bit), on the layer's own pools and slot ids.

With NANOVLLM_GDN_FUSED_DECODE=1 (the default) it replaces
Qwen3_5GatedDeltaNet._gdn_padded (qwen3_5.py:967-1085) with one whose
T == 1 branch runs ops.recurrent_decode_fused (gates, the conv with its
roll, the in-place recurrent update and the gated norm self.norm in one
kernel, after the q/k decode conv's own launch when the heads are grouped;
the same results bit for bit); other T keep the original method.

Both methods read the module's _USE_GDN_GBETA and _USE_CONV_TRITON (and the
decode method _USE_GDN_INPLACE) on every call, as the reference's layer
does, and run the original method when one of them is off, so the
reference's A/B switches keep their meaning when flipped at run time; conv
widths other than 4 also keep the original method.
"""
from __future__ import annotations

import os

from . import ops

PATCHED_NAMES = (
    "fused_g_beta", "causal_conv_silu_varlen", "conv_decode_step", "causal_conv_silu",
    "recurrent_gdn_inplace", "_fla_chunk", "_fla_recurrent", "_rms_gated_forward",
)
FLAG_NAMES = ("_HAS_FLA", "_USE_FLA_CHUNK", "_USE_FLA_RECURRENT", "_USE_GDN_VARLEN")


def _on(mod, name: str) -> bool:
    """A module-level switch of the reference module, read at call time (the
    layer reads _USE_GDN_GBETA, _USE_CONV_TRITON and _USE_GDN_INPLACE on every
    call, qwen3_5.py:933, :978, :1011, :1024); absent means on."""
    return bool(getattr(mod, name, True))


def _fused_prefill_method(mod, orig):
    def _gdn_prefill_varlen(self, hidden, lens_q, ids):
        """Fused form of Qwen3_5GatedDeltaNet._gdn_prefill_varlen
        (nanovllm/models/qwen3_5.py:922-965).  Other conv widths, and the
        module's _USE_GDN_GBETA or _USE_CONV_TRITON switched off at the time of
        the call, run the original method."""
        if self.conv_kernel != 4 or not (_on(mod, "_USE_GDN_GBETA") and _on(mod, "_USE_CONV_TRITON")):
            return orig(self, hidden, lens_q, ids)
        b = self.in_proj_b(hidden)
        a = self.in_proj_a(hidden)
        A_log = self.A_log[self._v_head_slice]
        dt_bias = self.dt_bias[self._v_head_slice]
        z = self.in_proj_z(hidden)
        mixed = self.in_proj_qkv(hidden)
        _, _, cu64_cpu, cu64_gpu = mod._varlen_meta(lens_q)
        core = ops.conv_chunk_prefill_varlen(
            mixed, self.conv_cache, self.conv1d.weight.view(self.conv_dim, self.conv_kernel), b, a, A_log, dt_bias,
            cu64_gpu, self.s_cache, ids, self.num_k_heads, self.num_v_heads, self.head_k_dim,
            cu_seqlens_cpu=cu64_cpu)
        core = self.norm(core, z.view(-1, self.num_v_heads, self.head_v_dim))
        return self.out_proj(core.reshape(-1, self.value_dim))

    return _gdn_prefill_varlen


def _fused_decode_method(mod, orig):
    def _gdn_padded(self, x, lens, ids, T):
        """Fused T == 1 branch of Qwen3_5GatedDeltaNet._gdn_padded
        (nanovllm/models/qwen3_5.py:967-1030, :1079-1085).  Other T and conv
        widths, and any of the module's _USE_GDN_GBETA, _USE_CONV_TRITON,
        _USE_GDN_INPLACE switched off at the time of the call, run the
        original method."""
        if T != 1 or self.conv_kernel != 4 or not (
                _on(mod, "_USE_GDN_GBETA") and _on(mod, "_USE_CONV_TRITON") and _on(mod, "_USE_GDN_INPLACE")):
            return orig(self, x, lens, ids, T)
        n = x.size(0)
        Hv, Dv = self.num_v_heads, self.head_v_dim
        b = self.in_proj_b(x).reshape(n, Hv)
        a = self.in_proj_a(x).reshape(n, Hv)
        A_log = self.A_log[self._v_head_slice]
        dt_bias = self.dt_bias[self._v_head_slice]
        z = self.in_proj_z(x)
        proj = self.in_proj_qkv(x).reshape(-1, self.conv_dim)
        w = self.conv1d.weight.view(self.conv_dim, 4)
        kd = self.key_dim
        # one key head per value head and whole heads per workgroup: the q/k
        # conv runs in the decode kernel too; else as its own launch first
        qk = None
        if not (self.num_k_heads == Hv and n * Hv >= ops.WHOLE_HEAD_TILES):
            qk = ops.conv_decode_step(proj[:, :2 * kd], self.conv_cache[:, :2 * kd], ids, w[:2 * kd])
        # gates + v conv + in-place update + the gated norm (self.norm's
        # weight and eps) in one kernel
        core = ops.recurrent_decode_fused(qk, proj, self.conv_cache, w, b, a, A_log, dt_bias, self.s_cache, ids,
                                          self.num_k_heads, Hv, self.head_k_dim, z=z.reshape(n, Hv * Dv),
                                          norm_weight=self.norm.weight, eps=self.norm.eps)
        return self.out_proj(core.reshape(n, 1, self.value_dim))

    return _gdn_padded


# The fused methods are installed under this package's own switches; the
# reference's kernel switches are checked by the methods on every call.
def _fused_decode_enabled() -> bool:
    return os.environ.get("NANOVLLM_GDN_FUSED_DECODE", "1") == "1"


def _fused_prefill_enabled() -> bool:
    return os.environ.get("NANOVLLM_GDN_FUSED_PREFILL", "1") == "1"


def install(mod) -> dict:
    """Rebind the GDN kernel entry points of a loaded qwen3_5 module.
    Returns the previous bindings (for uninstall)."""
    prev = {name: getattr(mod, name, None) for name in PATCHED_NAMES + FLAG_NAMES}
    mod.fused_g_beta = ops.fused_g_beta
    mod.causal_conv_silu_varlen = ops.causal_conv_silu_varlen
    mod.conv_decode_step = ops.conv_decode_step
    mod.causal_conv_silu = ops.causal_conv_silu
    mod.recurrent_gdn_inplace = ops.recurrent_gdn_inplace
    mod._fla_chunk = ops.chunk_gated_delta_rule
    mod._fla_recurrent = ops.recurrent_gated_delta_rule
    mod._rms_gated_forward = ops.rms_norm_gated
    use_chunk = os.environ.get("FLA_CHUNK", "1") == "1"
    use_rec = os.environ.get("FLA_RECURRENT", "1") == "1"
    if use_chunk or use_rec:
        mod._HAS_FLA = True
    mod._USE_FLA_CHUNK = use_chunk
    mod._USE_FLA_RECURRENT = use_rec
    mod._USE_GDN_VARLEN = use_chunk and os.environ.get("NANOVLLM_GDN_VARLEN", "1") == "1"
    cls = getattr(mod, "Qwen3_5GatedDeltaNet", None)
    if cls is not None and _fused_prefill_enabled() and hasattr(cls, "_gdn_prefill_varlen"):
        prev["Qwen3_5GatedDeltaNet._gdn_prefill_varlen"] = cls.__dict__.get("_gdn_prefill_varlen")
        cls._gdn_prefill_varlen = _fused_prefill_method(mod, cls._gdn_prefill_varlen)
    if cls is not None and _fused_decode_enabled() and hasattr(cls, "_gdn_padded"):
        prev["Qwen3_5GatedDeltaNet._gdn_padded"] = cls.__dict__.get("_gdn_padded")
        cls._gdn_padded = _fused_decode_method(mod, cls._gdn_padded)
    return prev


def uninstall(mod, prev: dict) -> None:
    for name, val in prev.items():
        if name.startswith("Qwen3_5GatedDeltaNet."):
            cls, attr = mod.Qwen3_5GatedDeltaNet, name.split(".", 1)[1]
            if val is None:
                delattr(cls, attr)
            else:
                setattr(cls, attr, val)
            continue
        setattr(mod, name, val)
