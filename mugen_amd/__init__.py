"""mugen_amd -- MI355X (gfx950) attention subsystem for the Mugen engine.

GQA decode / causal prefill and MLA absorbed decode / verify as hand-written
HIP kernels behind the C ABI in include/mugen_attn.h (libmugen_attn.so).
"""
from . import _capi
from .attention import (attention_decode, flash_prefill_attention, mla_absorb, mla_attention,
                        mla_attention_full, mla_latent_write, mla_project, scatter_kv)

__all__ = ["attention_decode", "flash_prefill_attention", "mla_absorb", "mla_attention", "mla_attention_full",
           "mla_latent_write", "mla_project", "scatter_kv", "_capi"]
__version__ = "0.1.0"
