"""MI355X-native (gfx950) Gated DeltaNet layer path of nano-vllm-extend.

The GDN kernels of the Qwen3.5 hybrid model -- varlen / decode / padded
causal conv + SiLU, fused g/beta, chunked gated delta rule, recurrent
decode (single- and multi-token), gated RMSNorm, the projection GEMMs -- as
hand-written HIP for
gfx950 behind the C ABI of include/gdn_mi355x.h, with Python wrappers that
keep the reference's call signatures (ops), a host mirror of the layer
dispatch (gdn_layer), the slot-pool bookkeeping (state_pool) and the hook
that installs the kernels into the reference model module (integration).
"""
from . import _lib, ops, state_pool, gdn_layer, integration  # noqa: F401
from .ops import (  # noqa: F401
    Qwen3_5RMSNormGated,
    causal_conv_silu,
    causal_conv_silu_varlen,
    causal_conv_silu_varlen_parts,
    chunk_gated_delta_rule,
    chunk_gated_delta_rule_varlen,
    commit_states,
    conv_decode_step,
    fused_g_beta,
    linear,
    recurrent_gated_delta_rule,
    recurrent_gdn_inplace,
    recurrent_gdn_multitoken,
    rms_norm_gated,
)
from .gdn_layer import GatedDeltaNetCore, GatedDeltaNetLayer, Switches  # noqa: F401
from .state_pool import LinearStatePool, allocate_state_pools, reset_linear_states, varlen_meta  # noqa: F401
