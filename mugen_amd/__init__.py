"""mugen_amd -- MI355X (gfx950) attention subsystem for the Mugen engine.

GQA decode (f16/bf16 caches and the reference's 4-bit group KV store),
causal prefill, MLA absorbed decode / verify with its absorption,
up-projection and latent-cache writer, as hand-written HIP kernels behind the
C ABI in include/mugen_attn.h (libmugen_attn.so).
"""
from . import _capi
from .attention import (attention_decode, flash_prefill_attention, kv_append, prefill_workspace, mla_absorb, mla_attention,
                        mla_attention_full, mla_latent_write, mla_prepare, mla_project, scatter_kv, seq_advance)
from .kv_store import KVCacheQ4

__all__ = ["KVCacheQ4", "attention_decode", "flash_prefill_attention", "kv_append", "prefill_workspace", "mla_absorb", "mla_attention",
           "mla_attention_full", "mla_latent_write", "mla_prepare", "mla_project", "scatter_kv", "seq_advance", "_capi"]
__version__ = "0.1.0"
