"""Torch-tensor front end of the gfx950 attention operators.

Thin wrappers that pass device pointers of torch tensors, plus torch's
current HIP stream, through the C ABI (include/mugen_attn.h).  Torch is
used only for device memory and streams; all compute is in
libmugen_attn.so.  Operator names follow the reference's seams:

  attention_decode         <- cpu_attention / flash_attention_decode
                              (transformer.cpp:2441-2485, kernel_sources.h:2900-2999)
  flash_prefill_attention  <- flash_prefill_attention (kernel_sources.h:2769-2896)
  mla_attention            <- cpu_mla_attention latent core (transformer.cpp:2576-2608)
  mla_absorb / mla_project <- cpu_mla_attention absorption and up-projection
                              (transformer.cpp:2556-2573, 2610-2620)
  mla_attention_full       <- cpu_mla_attention (transformer.cpp:2539-2623)
  mla_latent_write         <- c_kv RMSNorm + k_rope RoPE + latent append
                              (transformer.cpp:3930-3987)
  scatter_kv               <- scatter_kv (kernel_sources.h:3018-3028)
"""
from __future__ import annotations

import ctypes
import math

import torch

from . import _capi

_DT = {torch.float32: _capi.F32, torch.float16: _capi.F16, torch.bfloat16: _capi.BF16}


def _dt(t: torch.dtype) -> int:
    try:
        return _DT[t]
    except KeyError:
        raise TypeError(f"unsupported dtype {t}") from None


def _ptr(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(device: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _host_lens(seq_lens_host):
    """int32 host array for the planner hint (or None)."""
    if seq_lens_host is None:
        return None
    import numpy as np
    return np.ascontiguousarray(seq_lens_host, dtype=np.int32)


def _need_cuda(*ts: torch.Tensor):
    for t in ts:
        if not t.is_cuda:
            raise ValueError("mugen_amd operators take device tensors (no CPU path)")
        if not t.is_contiguous():
            raise ValueError("mugen_amd operators take contiguous tensors")


# ------------------------------------------------------------------ GQA decode

def gqa_decode_args(q, k_cache, v_cache, seq_lens, out, max_seq_len, scale=0.0, num_splits=0):
    B, H, D = q.shape
    Hk = k_cache.shape[-2]
    seq_stride = k_cache[0].numel() if k_cache.dim() == 4 else 0
    a = _capi.GqaDecodeArgs()
    a.q, a.k_cache, a.v_cache = q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr()
    a.seq_lens, a.out = seq_lens.data_ptr(), out.data_ptr()
    a.batch, a.n_heads, a.n_kv_heads, a.head_dim = B, H, Hk, D
    a.max_seq_len, a.num_splits, a.seq_stride, a.scale = int(max_seq_len), int(num_splits), seq_stride, float(scale)
    a.kv_dtype, a.out_dtype = _dt(k_cache.dtype), _dt(out.dtype)
    return a


def attention_decode(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                     seq_lens: torch.Tensor, max_seq_len: int | None = None, *,
                     out: torch.Tensor | None = None, out_dtype: torch.dtype | None = None,
                     scale: float = 0.0, num_splits: int = 0,
                     workspace: torch.Tensor | None = None, seq_lens_host=None) -> torch.Tensor:
    """GQA decode.  q [B,H,D]; k/v cache [B,max_T,Hk,D] (token-major per
    sequence); seq_lens int32 [B] on device; seq_lens_host: optional host
    copy used only to balance the context splits.  Returns out [B,H,D]."""
    _need_cuda(q, k_cache, v_cache, seq_lens)
    if k_cache.dim() != 4 or v_cache.shape != k_cache.shape:
        raise ValueError("k_cache/v_cache must be [B, max_T, Hk, D] and equal shapes")
    if seq_lens.dtype != torch.int32:
        raise TypeError("seq_lens must be int32")
    if max_seq_len is None:
        max_seq_len = k_cache.shape[1]
    if out is None:
        out = torch.empty(q.shape, dtype=out_dtype or q.dtype, device=q.device)
    a = gqa_decode_args(q, k_cache, v_cache, seq_lens, out, max_seq_len, scale, num_splits)
    hl = _host_lens(seq_lens_host)
    if hl is not None:
        a.seq_lens_host = hl.ctypes.data
    L = _capi.lib()
    need = L.mugen_attn_gqa_decode_workspace_size(ctypes.byref(a))
    if need and (workspace is None or workspace.numel() * workspace.element_size() < need):
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    _capi.check(L.mugen_attn_gqa_decode(ctypes.byref(a), _ptr(workspace), ws_bytes, _stream(q.device)))
    return out


# ------------------------------------------------------------------ GQA prefill

def _prefill_args(q, k, v, start_pos, causal, out, scale=0.0, kernel=0):
    N, H, D = q.shape
    kv_len, Hk, Dk = k.shape
    if Dk != D or v.shape != k.shape:
        raise ValueError("k/v must be [kv_len, Hk, D] matching q's head_dim")
    a = _capi.GqaPrefillArgs()
    a.q, a.k, a.v, a.out = q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr()
    a.n_tokens, a.n_heads, a.n_kv_heads, a.head_dim = N, H, Hk, D
    a.kv_len, a.start_pos, a.causal, a.scale = kv_len, int(start_pos), 1 if causal else 0, float(scale)
    a.dtype, a.out_dtype, a.kernel = _dt(q.dtype), _dt(out.dtype), int(kernel)
    return a


def prefill_workspace(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, start_pos: int = 0, *,
                      causal: bool = True, out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """The optional prefill workspace for this shape
    (mugen_attn_gqa_prefill_workspace_size bytes; empty when none helps)."""
    out = torch.empty((0,), dtype=out_dtype or q.dtype, device=q.device)
    a = _prefill_args(q, k, v, start_pos, causal, out)
    a.out = q.data_ptr()  # a placeholder: only the shape matters for the size
    need = _capi.lib().mugen_attn_gqa_prefill_workspace_size(ctypes.byref(a))
    return torch.empty(need, dtype=torch.uint8, device=q.device)

def flash_prefill_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, start_pos: int = 0, *,
                            causal: bool = True, out: torch.Tensor | None = None,
                            out_dtype: torch.dtype | None = None, scale: float = 0.0,
                            kernel: int = 0, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """Causal GQA prefill.  q [N,H,D]; k/v [kv_len,Hk,D] (cache incl. the new
    tokens); token i sees keys [0, start_pos+i].  Returns out [N,H,D].
    kernel: 0 automatic, PREFILL_KERNEL_BLOCK / _WS / _SHORT force one (_SHORT
    only for head_dim 64, <= 4 heads per kv head and <= 512 visible keys).
    workspace: the optional buffer for the fp16 copy of V (bf16 prompts of
    1024+ tokens) and for the partials of split key ranges (short chunks
    over long contexts, merged by a second launch); None allocates one when
    the library asks for it, an empty tensor passes none (the call then runs
    unsplit, same result to rounding)."""
    _need_cuda(q, k, v)
    if out is None:
        out = torch.empty(q.shape, dtype=out_dtype or q.dtype, device=q.device)
    a = _prefill_args(q, k, v, start_pos, causal, out, scale, kernel)
    if workspace is None:
        need = _capi.lib().mugen_attn_gqa_prefill_workspace_size(ctypes.byref(a))
        if need:
            workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    if workspace is not None and workspace.numel():
        a.workspace, a.workspace_bytes = workspace.data_ptr(), workspace.numel() * workspace.element_size()
    _capi.check(_capi.lib().mugen_attn_gqa_prefill(ctypes.byref(a), _stream(q.device)))
    return out


# ------------------------------------------------------------------ MLA

def mla_args(q, latent, seq_lens, out, max_seq_len, scale, num_splits=0, kernel=0):
    B, q_len, H, C = q.shape
    a = _capi.MlaDecodeArgs()
    a.q, a.latent, a.seq_lens, a.out = q.data_ptr(), latent.data_ptr(), seq_lens.data_ptr(), out.data_ptr()
    a.batch, a.q_len, a.n_heads, a.kv_rank, a.rope_dim = B, q_len, H, 512, C - 512
    a.max_seq_len, a.num_splits = int(max_seq_len), int(num_splits)
    a.seq_stride = latent[0].numel()
    a.scale = float(scale)
    a.q_dtype, a.latent_dtype, a.out_dtype = _dt(q.dtype), _dt(latent.dtype), _dt(out.dtype)
    a.kernel = int(kernel)
    return a


def mla_attention(q: torch.Tensor, latent: torch.Tensor, seq_lens: torch.Tensor,
                  max_seq_len: int | None = None, *, scale: float = 1.0 / math.sqrt(192.0),
                  out: torch.Tensor | None = None, out_dtype: torch.dtype = torch.float32,
                  num_splits: int = 0, workspace: torch.Tensor | None = None,
                  seq_lens_host=None, kernel: int = 0) -> torch.Tensor:
    """MLA absorbed attention (decode: q_len 1; verify: q_len > 1, causal).

    q [B,q_len,H,576] (q_nope.W_UK ++ q_rope); latent [B,max_T,576];
    seq_lens int32 [B] = cache length incl. the q_len new tokens.
    kernel: 0 automatic, MLA_KERNEL_ROWS / MLA_KERNEL_WS force one.
    Returns out [B,q_len,H,512]."""
    _need_cuda(q, latent, seq_lens)
    if q.dim() != 4 or latent.dim() != 3 or latent.shape[-1] != q.shape[-1]:
        raise ValueError("q must be [B,q_len,H,576] and latent [B,max_T,576]")
    if seq_lens.dtype != torch.int32:
        raise TypeError("seq_lens must be int32")
    if max_seq_len is None:
        max_seq_len = latent.shape[1]
    B, q_len, H, _ = q.shape
    if out is None:
        out = torch.empty((B, q_len, H, 512), dtype=out_dtype, device=q.device)
    a = mla_args(q, latent, seq_lens, out, max_seq_len, scale, num_splits, kernel)
    hl = _host_lens(seq_lens_host)
    if hl is not None:
        a.seq_lens_host = hl.ctypes.data
    L = _capi.lib()
    need = L.mugen_attn_mla_decode_workspace_size(ctypes.byref(a))
    if need and (workspace is None or workspace.numel() * workspace.element_size() < need):
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    _capi.check(L.mugen_attn_mla_decode(ctypes.byref(a), _ptr(workspace), ws_bytes, _stream(q.device)))
    return out


_WT = {"f16": _capi.W_F16, "q8_0": _capi.W_Q8_0, "q4_0": _capi.W_Q4_0}


def _wtype(w: torch.Tensor, w_type) -> int:
    if w_type is None:
        if w.dtype != torch.float16:
            raise TypeError("block-encoded weights need w_type ('q8_0' / 'q4_0')")
        return _capi.W_F16
    return _WT[w_type] if isinstance(w_type, str) else int(w_type)


def _rope(rope) -> _capi.RopeParams:
    """(theta, factor, original_ctx) -> RopeParams; factor <= 1: plain RoPE."""
    theta, factor, ctx = rope
    return _capi.RopeParams(float(theta), float(factor), int(ctx))


def _absorb_args(q, w_kb, w_type, out, out_dtype, positions, rope, seq_base, rows_per_seq):
    """The absorb call's ABI arguments (validated) and its output tensor."""
    _need_cuda(q, w_kb)
    if q.dtype != torch.float16 or q.shape[-1] != 192:
        raise ValueError("q must be float16 [..., H, 192]")
    H = q.shape[-2]
    rows = q.numel() // (H * 192)
    if out is None:
        out = torch.empty((*q.shape[:-1], 576), dtype=out_dtype, device=q.device)
    a = _capi.MlaAbsorbArgs()
    a.q, a.w_kb, a.q_abs = q.data_ptr(), w_kb.data_ptr(), out.data_ptr()
    a.rows, a.n_heads, a.nope_dim, a.rope_dim, a.kv_rank = rows, H, 128, 64, 512
    a.w_type, a.out_dtype = _wtype(w_kb, w_type), _dt(out.dtype)
    if positions is not None:
        _need_cuda(positions)
        if positions.dtype != torch.int32 or positions.numel() != rows:
            raise ValueError("positions must be int32 with one entry per row of q")
        a.positions, a.rope = positions.data_ptr(), _rope(rope)
    elif seq_base is not None:
        _need_cuda(seq_base)
        if seq_base.dtype != torch.int32:
            raise TypeError("seq_base must be int32")
        a.seq_base, a.rows_per_seq, a.rope = seq_base.data_ptr(), int(rows_per_seq), _rope(rope)
    return a, out


def mla_absorb(q: torch.Tensor, w_kb: torch.Tensor, w_type=None, *, out: torch.Tensor | None = None,
               out_dtype: torch.dtype = torch.float32, positions: torch.Tensor | None = None,
               rope=(10000.0, 0.0, 0), seq_base: torch.Tensor | None = None, rows_per_seq: int = 1) -> torch.Tensor:
    """q_abs = [q_nope . k_b | q_rope] per head (transformer.cpp:2556-2573).

    q f16 [..., H, 192]; w_kb = attn_k_b, H*128 rows of 512 in the GGML
    encoding w_type ('f16' as a float16 tensor, 'q8_0' / 'q4_0' as uint8
    bytes).  Returns [..., H, 576] in out_dtype (F32 or BF16).  With
    positions (int32, one per row of q), q_rope is first rotated by the
    reference's q RoPE stage (transformer.cpp:3882-3921) with
    rope = (theta, yarn factor, original ctx).  With seq_base (int32
    [n_seq]) instead of positions, row r is rotated at
    seq_base[r // rows_per_seq] + r % rows_per_seq."""
    a, out = _absorb_args(q, w_kb, w_type, out, out_dtype, positions, rope, seq_base, rows_per_seq)
    _capi.check(_capi.lib().mugen_attn_mla_absorb(ctypes.byref(a), _stream(q.device)))
    return out


def mla_project(o: torch.Tensor, w_vb: torch.Tensor, w_type=None, *, out: torch.Tensor | None = None,
                out_dtype: torch.dtype = torch.float16) -> torch.Tensor:
    """out = o . v_b^T per head (transformer.cpp:2610-2620).

    o f32 [..., H, 512]; w_vb = attn_v_b, H*128 rows of 512 (w_type as in
    mla_absorb).  Returns [..., H, 128] in out_dtype (F16 or F32)."""
    _need_cuda(o, w_vb)
    if o.dtype != torch.float32 or o.shape[-1] != 512:
        raise ValueError("o must be float32 [..., H, 512]")
    H = o.shape[-2]
    rows = o.numel() // (H * 512)
    if out is None:
        out = torch.empty((*o.shape[:-1], 128), dtype=out_dtype, device=o.device)
    a = _capi.MlaProjectArgs()
    a.o, a.w_vb, a.out = o.data_ptr(), w_vb.data_ptr(), out.data_ptr()
    a.rows, a.n_heads, a.kv_rank, a.v_head_dim = rows, H, 512, 128
    a.w_type, a.out_dtype = _wtype(w_vb, w_type), _dt(out.dtype)
    _capi.check(_capi.lib().mugen_attn_mla_project(ctypes.byref(a), _stream(o.device)))
    return out


def mla_attention_full(q: torch.Tensor, w_kb: torch.Tensor, w_vb: torch.Tensor, latent: torch.Tensor,
                       seq_lens: torch.Tensor, max_seq_len: int | None = None, w_type=None, *,
                       scale: float = 1.0 / math.sqrt(192.0), num_splits: int = 0,
                       seq_lens_host=None) -> torch.Tensor:
    """cpu_mla_attention end to end (transformer.cpp:2539-2623): f16 q
    [B,q_len,H,192] and f16 latent [B,max_T,576] in, f16 [B,q_len,H,128]
    out, fp32 arithmetic throughout (the latent core runs with an fp32 q)."""
    qa = mla_absorb(q, w_kb, w_type)
    o = mla_attention(qa, latent, seq_lens, max_seq_len, scale=scale, num_splits=num_splits,
                      seq_lens_host=seq_lens_host)
    return mla_project(o, w_vb, w_type)


def _latent_args(kv_a, norm_w, positions, latent, rows_per_seq, eps, rope, max_seq_len, seq_base):
    """The latent write's ABI arguments (validated)."""
    _need_cuda(kv_a, norm_w, latent)
    if kv_a.dtype != torch.float16 or norm_w.dtype != torch.float16 or kv_a.shape[-1] != 576:
        raise ValueError("kv_a must be float16 [rows, 576] and norm_w float16 [512]")
    pos = positions if positions is not None else seq_base
    if pos is None:
        raise ValueError("positions or seq_base is required")
    _need_cuda(pos)
    if pos.dtype != torch.int32:
        raise TypeError("positions / seq_base must be int32")
    rows = kv_a.numel() // 576
    if (positions is not None and positions.numel() != rows) or latent.dim() != 3 or latent.shape[-1] != 576:
        raise ValueError("positions must hold one entry per kv_a row; latent must be [n_seq, max_T, 576]")
    a = _capi.MlaLatentWriteArgs()
    a.kv_a, a.norm_w, a.latent = kv_a.data_ptr(), norm_w.data_ptr(), latent.data_ptr()
    if positions is not None:
        a.positions = positions.data_ptr()
    else:
        a.seq_base = seq_base.data_ptr()
    a.rows, a.rows_per_seq = rows, int(rows_per_seq)
    a.max_seq_len = int(latent.shape[1] if max_seq_len is None else max_seq_len)
    a.kv_rank, a.rope_dim, a.latent_dtype = 512, 64, _dt(latent.dtype)
    a.seq_stride, a.eps, a.rope = latent[0].numel(), float(eps), _rope(rope)
    if (rows + a.rows_per_seq - 1) // a.rows_per_seq > latent.shape[0]:
        raise ValueError("more sequences than latent has")
    return a


def mla_latent_write(kv_a: torch.Tensor, norm_w: torch.Tensor, positions: torch.Tensor | None, latent: torch.Tensor,
                     *, rows_per_seq: int = 1, eps: float = 1e-6, rope=(10000.0, 0.0, 0),
                     max_seq_len: int | None = None, seq_base: torch.Tensor | None = None) -> torch.Tensor:
    """Latent-cache writer (transformer.cpp:3930-3987): RMSNorm(c_kv) * norm_w
    and RoPE(k_rope) of each kv_a row [rows, 576] (f16), written to row
    positions[r] of sequence r // rows_per_seq of latent [n_seq, max_T, 576]
    (f16 or bf16).  rope = (theta, yarn factor, original ctx).  With
    positions None, row r goes to seq_base[r // rows_per_seq] +
    r % rows_per_seq."""
    a = _latent_args(kv_a, norm_w, positions, latent, rows_per_seq, eps, rope, max_seq_len, seq_base)
    _capi.check(_capi.lib().mugen_attn_mla_latent_write(ctypes.byref(a), _stream(kv_a.device)))
    return latent


def mla_prepare(kv_a: torch.Tensor, norm_w: torch.Tensor, positions: torch.Tensor, latent: torch.Tensor,
                q: torch.Tensor, w_kb: torch.Tensor, w_type=None, *, q_abs: torch.Tensor | None = None,
                rows_per_seq: int = 1, eps: float = 1e-6, rope=(10000.0, 0.0, 0)) -> torch.Tensor:
    """mla_latent_write(kv_a, norm_w, positions, latent) and mla_absorb(q,
    w_kb, positions=positions) in one call (one kernel launch at decode
    sizes; results identical to the two calls).  Returns q_abs (F32)."""
    lw = _latent_args(kv_a, norm_w, positions, latent, rows_per_seq, eps, rope, None, None)
    ab, q_abs = _absorb_args(q, w_kb, w_type, q_abs, torch.float32, positions, rope, None, 1)
    _capi.check(_capi.lib().mugen_attn_mla_prepare(ctypes.byref(lw), ctypes.byref(ab), _stream(q.device)))
    return q_abs


# ------------------------------------------------------------------ decode-step helpers

def kv_append(k_new: torch.Tensor, v_new: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
              seq_lens: torch.Tensor) -> None:
    """Write row j of each sequence's new K / V ([B, n_new, Hk, d] or
    [B, n_new, Hk*d]) at position seq_lens[b] + j of the caches
    ([B, max_T, Hk, d]): the two scatter_kv dispatches of a decode step
    (transformer.cpp:3749-3754) with the offset read on the device."""
    _need_cuda(k_new, v_new, k_cache, v_cache, seq_lens)
    B, n_new = k_new.shape[0], k_new.shape[1]
    row = k_new[0, 0].numel()
    if k_cache[0, 0].numel() != row or v_new.shape != k_new.shape or k_cache.shape != v_cache.shape:
        raise ValueError("k_new / v_new rows must match the caches' rows")
    a = _capi.KvAppendArgs()
    a.k_new, a.v_new, a.k_cache, a.v_cache = k_new.data_ptr(), v_new.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr()
    a.seq_lens, a.seq_stride = seq_lens.data_ptr(), k_cache[0].numel()
    a.n_seq, a.n_new, a.row, a.max_seq_len = B, n_new, row, k_cache.shape[1]
    _capi.check(_capi.lib().mugen_attn_kv_append(ctypes.byref(a), _stream(k_new.device)))


def seq_advance(seq_lens: torch.Tensor, n: int, max_seq_len: int, n_q4: torch.Tensor | None = None,
                n_q4_next: torch.Tensor | None = None) -> None:
    """seq_lens += n on the device, capped at max_seq_len (and n_q4 = n_q4_next)."""
    _need_cuda(seq_lens)
    if seq_lens.dtype != torch.int32:
        raise TypeError("seq_lens must be int32")
    _capi.check(_capi.lib().mugen_attn_seq_advance(_ptr(seq_lens), int(n), seq_lens.numel(), int(max_seq_len),
                                                    _ptr(n_q4), _ptr(n_q4_next), _stream(seq_lens.device)))


# ------------------------------------------------------------------ scatter_kv

def scatter_kv(src: torch.Tensor, dst: torch.Tensor, offset: int) -> torch.Tensor:
    """dst.view(-1)[offset : offset+src.numel()] = src (16-bit elements)."""
    _need_cuda(src, dst)
    if src.element_size() != 2 or dst.element_size() != 2:
        raise TypeError("scatter_kv copies 16-bit elements")
    if offset < 0 or offset + src.numel() > dst.numel():
        raise ValueError("scatter_kv: destination range out of bounds")
    _capi.check(_capi.lib().mugen_attn_scatter_kv(_ptr(src), _ptr(dst), int(offset), src.numel(),
                                                  _stream(src.device)))
    return dst
