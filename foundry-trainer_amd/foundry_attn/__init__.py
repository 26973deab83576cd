"""foundry_attn — MI355X (gfx950) attention hot path for foundry-spike.

Host-side mirror of the reference's op surface over libfoundry_attn.so; see
ops.py.  Importing this package loads nothing; the first op call loads the
library and fails loudly if it is missing.
"""
from ._abi import FoundryAttnError, LIB_PATH, lib
from .ops import (AttnBwd, attention, attn_bwd, attn_fwd, attn_workspace_bytes, lora_bwd, lora_down, lora_fwd,
                  lora_grad, lora_grad_many, lora_up,
                  qk_prologue, qk_prologue_bwd, qk_prologue_bwd_multi, qk_prologue_multi, rope_tables)

__all__ = ["AttnBwd", "attention", "attn_fwd", "attn_bwd", "attn_workspace_bytes", "qk_prologue", "qk_prologue_bwd",
           "qk_prologue_multi", "qk_prologue_bwd_multi",
           "rope_tables", "lora_fwd", "lora_bwd", "lora_down", "lora_up", "lora_grad", "lora_grad_many",
           "FoundryAttnError",
           "LIB_PATH", "lib"]
