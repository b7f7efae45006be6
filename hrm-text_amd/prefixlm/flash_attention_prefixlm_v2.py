"""Drop-in module for ``models/flash_attention_prefixlm_v2.py`` of the reference.

Exposes the names the reference's callers import from that module:
``flash_attn_varlen_prefixlm`` (models/layers.py:10) and
``compute_aux_seq_tensors_scalars`` (dataset_new.py:13), plus the operator and
autograd classes under the reference's class name.
"""
from .metadata import compute_aux_seq_tensors_scalars
from .op import FlashAttnVarlenPrefixLM, flash_attn_varlen_prefixlm

__all__ = ["compute_aux_seq_tensors_scalars", "flash_attn_varlen_prefixlm", "FlashAttnVarlenPrefixLM"]
