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
  chunk_gated_delta_rule       -> ops.chunk_gated_delta_rule_ref_api
  recurrent_gated_delta_rule   -> fla-style gathered recurrent on HIP
  _rms_gated_forward           -> ops.rms_norm_gated

and sets the feature flags the layer reads (_HAS_FLA, _USE_FLA_CHUNK,
_USE_FLA_RECURRENT, _USE_GDN_VARLEN) from the same environment switches
(FLA_CHUNK, FLA_RECURRENT, NANOVLLM_GDN_VARLEN) the reference reads.
"""
from __future__ import annotations

import os

from . import ops

PATCHED_NAMES = (
    "fused_g_beta", "causal_conv_silu_varlen", "conv_decode_step", "causal_conv_silu",
    "recurrent_gdn_inplace", "_fla_chunk", "_fla_recurrent", "chunk_gated_delta_rule",
    "recurrent_gated_delta_rule", "_rms_gated_forward",
)


def _recurrent_ref_api(query, key, value, g, beta, initial_state=None):
    return ops.recurrent_gated_delta_rule(query, key, value, g=g, beta=beta, initial_state=initial_state,
                                          output_final_state=True, use_qk_l2norm_in_kernel=True)


def install(mod) -> dict:
    """Rebind the GDN kernel entry points of a loaded qwen3_5 module.
    Returns the previous bindings (for uninstall)."""
    prev = {name: getattr(mod, name, None) for name in PATCHED_NAMES}
    prev.update({f: getattr(mod, f, None) for f in ("_HAS_FLA", "_USE_FLA_CHUNK", "_USE_FLA_RECURRENT",
                                                     "_USE_GDN_VARLEN")})
    mod.fused_g_beta = ops.fused_g_beta
    mod.causal_conv_silu_varlen = ops.causal_conv_silu_varlen
    mod.conv_decode_step = ops.conv_decode_step
    mod.causal_conv_silu = ops.causal_conv_silu
    mod.recurrent_gdn_inplace = ops.recurrent_gdn_inplace
    mod._fla_chunk = ops.chunk_gated_delta_rule
    mod._fla_recurrent = ops.recurrent_gated_delta_rule
    mod.chunk_gated_delta_rule = ops.chunk_gated_delta_rule_ref_api
    mod.recurrent_gated_delta_rule = _recurrent_ref_api
    mod._rms_gated_forward = ops.rms_norm_gated
    mod._HAS_FLA = True
    mod._USE_FLA_CHUNK = os.environ.get("FLA_CHUNK", "1") == "1"
    mod._USE_FLA_RECURRENT = os.environ.get("FLA_RECURRENT", "1") == "1"
    mod._USE_GDN_VARLEN = mod._USE_FLA_CHUNK and os.environ.get("NANOVLLM_GDN_VARLEN", "1") == "1"
    return prev


def uninstall(mod, prev: dict) -> None:
    for name, val in prev.items():
        setattr(mod, name, val)
