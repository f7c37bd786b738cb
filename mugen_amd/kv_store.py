"""Device-resident 4-bit group KV store (the reference's KVCache format,
src/core/memory/kv_cache.cpp) and GQA decode straight from it.

KVCacheQ4 mirrors KVCache's configuration (n_layers, n_kv_heads, head_dim,
max_seq_len, fp16_preserve_last) and append semantics for a batch of
sequences: every token older than the newest fp16_preserve_last is held as
20-byte groups of 32 values (f16 scale, f16 min, 16 bytes of nibbles), the
newest ones in an f16 ring.  Appends run the quantisation on the GPU
(kv_cache.cpp:21-56 bit for bit); attention_decode reads the store without
materialising f16 K/V.  Torch holds the memory; the work is in
libmugen_attn.so.
"""
from __future__ import annotations

import ctypes
import math

import numpy as np
import torch

from . import _capi
from .attention import _dt, _need_cuda, _ptr, _stream


class KVCacheQ4:
    """Per-layer 4-bit stores for n_seq sequences.

    seq_lens / n_q4 are kept on the device (int32 [n_seq]) and on the host
    (the planner hint); append() advances both after every layer of a step
    has been appended (advance())."""

    def __init__(self, n_layers: int, n_seq: int, n_kv_heads: int, head_dim: int, max_seq_len: int = 8192,
                 fp16_preserve_last: int = 256, max_new: int = 64, device="cuda"):
        if n_layers <= 0 or n_seq <= 0 or n_kv_heads <= 0 or head_dim <= 0 or max_seq_len <= 0:
            raise ValueError("n_layers, n_seq, n_kv_heads, head_dim and max_seq_len must be > 0")
        self.n_layers, self.n_seq, self.Hk, self.D = n_layers, n_seq, n_kv_heads, head_dim
        self.vpt = n_kv_heads * head_dim
        if self.vpt % 32:
            raise ValueError("n_kv_heads * head_dim must be a multiple of 32")
        self.max_seq_len, self.preserve, self.max_new = max_seq_len, fp16_preserve_last, max_new
        self.ring = 1 << max(0, (fp16_preserve_last + max_new - 1).bit_length())  # a power of two
        self.row_bytes = self.vpt // 32 * 20
        dev = torch.device(device)
        self.q4_k = [torch.zeros((n_seq, max_seq_len, self.row_bytes), dtype=torch.uint8, device=dev)
                     for _ in range(n_layers)]
        self.q4_v = [torch.zeros_like(t) for t in self.q4_k]
        self.ring_k = [torch.zeros((n_seq, self.ring, self.vpt), dtype=torch.float16, device=dev)
                       for _ in range(n_layers)]
        self.ring_v = [torch.zeros_like(t) for t in self.ring_k]
        self.seq_lens = torch.zeros(n_seq, dtype=torch.int32, device=dev)
        self.n_q4 = torch.zeros(n_seq, dtype=torch.int32, device=dev)
        self._n_q4_next = torch.zeros_like(self.n_q4)
        self.seq_lens_host = np.zeros(n_seq, np.int32)
        self._pending = 0

    def store(self, layer: int) -> _capi.KvQ4Store:
        s = _capi.KvQ4Store()
        s.q4_k, s.q4_v = self.q4_k[layer].data_ptr(), self.q4_v[layer].data_ptr()
        s.ring_k, s.ring_v = self.ring_k[layer].data_ptr(), self.ring_v[layer].data_ptr()
        s.q4_seq_stride = self.max_seq_len * self.row_bytes
        s.ring_seq_stride = self.ring * self.vpt
        s.ring, s.fp16_preserve_last = self.ring, self.preserve
        return s

    def append(self, layer: int, k_new: torch.Tensor, v_new: torch.Tensor) -> None:
        """KVCache::append of n_new tokens per sequence to one layer:
        k_new / v_new f16 [n_seq, n_new, n_kv_heads*head_dim] (or
        [n_seq, n_new, n_kv_heads, head_dim])."""
        _need_cuda(k_new, v_new)
        n_new = k_new.shape[1]
        if k_new.dtype != torch.float16 or k_new.shape != v_new.shape or k_new.numel() != self.n_seq * n_new * self.vpt:
            raise ValueError("k_new / v_new must be float16 [n_seq, n_new, n_kv_heads*head_dim]")
        if n_new > self.max_new:
            raise ValueError(f"n_new {n_new} > max_new {self.max_new}")
        if self._pending and self._pending != n_new:
            raise ValueError("every layer of a step appends the same number of tokens")
        a = _capi.KvQ4AppendArgs()
        a.store = self.store(layer)
        a.k_new, a.v_new = k_new.data_ptr(), v_new.data_ptr()
        a.seq_lens, a.n_q4, a.n_q4_out = self.seq_lens.data_ptr(), self.n_q4.data_ptr(), self._n_q4_next.data_ptr()
        a.n_seq, a.n_new, a.n_kv_heads, a.head_dim, a.max_seq_len = self.n_seq, n_new, self.Hk, self.D, self.max_seq_len
        _capi.check(_capi.lib().mugen_attn_kv_q4_append(ctypes.byref(a), _stream(k_new.device)))
        self._pending = n_new

    def advance(self) -> None:
        """Commit the step's appends: seq_lens += n_new, n_q4 = the
        appends' result (the same for every layer)."""
        if not self._pending:
            return
        self.n_q4.copy_(self._n_q4_next)
        self.seq_lens_host = np.minimum(self.seq_lens_host + self._pending, self.max_seq_len).astype(np.int32)
        self.seq_lens.copy_(torch.from_numpy(self.seq_lens_host))
        self._pending = 0

    def attention_decode(self, layer: int, q: torch.Tensor, *, scale: float = 0.0,
                         out: torch.Tensor | None = None, out_dtype: torch.dtype = torch.float16,
                         num_splits: int = 0, workspace: torch.Tensor | None = None) -> torch.Tensor:
        """cpu_attention over this layer's store (q f16 [n_seq, H, head_dim])."""
        _need_cuda(q)
        B, H, D = q.shape
        if q.dtype != torch.float16 or B != self.n_seq or D != self.D:
            raise ValueError("q must be float16 [n_seq, n_heads, head_dim]")
        if out is None:
            out = torch.empty((B, H, D), dtype=out_dtype, device=q.device)
        a = _capi.GqaDecodeQ4Args()
        a.q, a.store, a.seq_lens, a.n_q4, a.out = q.data_ptr(), self.store(layer), self.seq_lens.data_ptr(), \
            self.n_q4.data_ptr(), out.data_ptr()
        a.batch, a.n_heads, a.n_kv_heads, a.head_dim = B, H, self.Hk, D
        a.max_seq_len, a.num_splits = self.max_seq_len, int(num_splits)
        a.scale, a.out_dtype = float(scale) if scale > 0 else 1.0 / math.sqrt(D), _dt(out.dtype)
        a.seq_lens_host = self.seq_lens_host.ctypes.data
        L = _capi.lib()
        need = L.mugen_attn_gqa_decode_q4_workspace_size(ctypes.byref(a))
        if need and (workspace is None or workspace.numel() * workspace.element_size() < need):
            workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
        ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
        _capi.check(L.mugen_attn_gqa_decode_q4(ctypes.byref(a), _ptr(workspace), ws_bytes, _stream(q.device)))
        return out
