"""MI355X-native packed varlen PrefixLM attention (HRM-Text hot path).

Public names follow the reference module models/flash_attention_prefixlm_v2.py.
"""
from .metadata import compute_aux_seq_tensors_scalars, useful_entries, useful_flops
from .op import FlashAttnVarlenPrefixLM, flash_attn_varlen_prefixlm
from .plan import build_plan, plan_ds_blocks, plan_inputs, plan_size
from .layer import fused_attention_layer
from .kvcache import flash_attn_with_kvcache
from .norm_mlp import rms_norm, swiglu

__all__ = [
    "build_plan",
    "compute_aux_seq_tensors_scalars",
    "flash_attn_varlen_prefixlm",
    "flash_attn_with_kvcache",
    "fused_attention_layer",
    "FlashAttnVarlenPrefixLM",
    "useful_entries",
    "useful_flops",
    "plan_ds_blocks",
    "plan_inputs",
    "plan_size",
    "rms_norm",
    "swiglu",
]
