"""ctypes binding of libmugen_attn.so (the C ABI in include/mugen_attn.h).

The library is loaded from this package directory only; a missing library
raises immediately -- there is no fallback implementation.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmugen_attn.so")

OK = 0
E_INVALID = -1
E_UNSUPPORTED = -2
E_WORKSPACE = -3
E_HIP = -4

F32, F16, BF16 = 0, 1, 2
W_F16, W_Q4_0, W_Q8_0 = 1, 2, 8  # weight encodings (GGML type ids)
MLA_KERNEL_ROWS, MLA_KERNEL_WS = 1, 2  # mugen_attn_mla_decode_args.kernel
PREFILL_KERNEL_AUTO, PREFILL_KERNEL_BLOCK, PREFILL_KERNEL_WS, PREFILL_KERNEL_SHORT = 0, 1, 2, 3  # mugen_attn_gqa_prefill_args.kernel
MLA_SCRATCH_BYTES = 32 << 20  # MUGEN_ATTN_MLA_SCRATCH_BYTES: the fixed scratch of mugen_attn_mla_decode_noalloc

# every symbol include/mugen_attn.h declares
EXPORTS = (
    "mugen_attn_gqa_decode_workspace_size",
    "mugen_attn_gqa_decode",
    "mugen_attn_gqa_prefill",
    "mugen_attn_gqa_prefill_workspace_size",
    "mugen_attn_kv_q4_append",
    "mugen_attn_gqa_decode_q4_workspace_size",
    "mugen_attn_gqa_decode_q4",
    "mugen_attn_mla_decode_workspace_size",
    "mugen_attn_mla_decode",
    "mugen_attn_mla_decode_noalloc",
    "mugen_attn_mla_absorb",
    "mugen_attn_mla_project",
    "mugen_attn_mla_latent_write",
    "mugen_attn_mla_prepare",
    "mugen_attn_kv_append",
    "mugen_attn_seq_advance",
    "mugen_attn_scatter_kv",
    "mugen_attn_last_error",
    "mugen_attn_version",
    "mugen_attn_timing_enable",
    "mugen_attn_timing_read",
    "mugen_attn_timing_reset",
)

_vp = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float


class GqaDecodeArgs(ctypes.Structure):
    _fields_ = [
        ("q", _vp), ("k_cache", _vp), ("v_cache", _vp), ("seq_lens", _vp), ("out", _vp),
        ("batch", _i32), ("n_heads", _i32), ("n_kv_heads", _i32), ("head_dim", _i32),
        ("max_seq_len", _i32), ("num_splits", _i32), ("seq_stride", _i64), ("scale", _f32),
        ("kv_dtype", _i32), ("out_dtype", _i32), ("seq_lens_host", _vp),
    ]


class KvQ4Store(ctypes.Structure):
    _fields_ = [
        ("q4_k", _vp), ("q4_v", _vp), ("ring_k", _vp), ("ring_v", _vp),
        ("q4_seq_stride", _i64), ("ring_seq_stride", _i64), ("ring", _i32), ("fp16_preserve_last", _i32),
    ]


class KvQ4AppendArgs(ctypes.Structure):
    _fields_ = [
        ("store", KvQ4Store), ("k_new", _vp), ("v_new", _vp), ("seq_lens", _vp), ("n_q4", _vp), ("n_q4_out", _vp),
        ("n_seq", _i32), ("n_new", _i32), ("n_kv_heads", _i32), ("head_dim", _i32), ("max_seq_len", _i32),
    ]


class GqaDecodeQ4Args(ctypes.Structure):
    _fields_ = [
        ("q", _vp), ("store", KvQ4Store), ("seq_lens", _vp), ("n_q4", _vp), ("out", _vp),
        ("batch", _i32), ("n_heads", _i32), ("n_kv_heads", _i32), ("head_dim", _i32), ("max_seq_len", _i32),
        ("num_splits", _i32), ("scale", _f32), ("out_dtype", _i32), ("seq_lens_host", _vp),
    ]


class KvAppendArgs(ctypes.Structure):
    _fields_ = [
        ("k_new", _vp), ("v_new", _vp), ("k_cache", _vp), ("v_cache", _vp), ("seq_lens", _vp),
        ("seq_stride", _i64), ("n_seq", _i32), ("n_new", _i32), ("row", _i32), ("max_seq_len", _i32),
    ]


class GqaPrefillArgs(ctypes.Structure):
    _fields_ = [
        ("q", _vp), ("k", _vp), ("v", _vp), ("out", _vp),
        ("n_tokens", _i32), ("n_heads", _i32), ("n_kv_heads", _i32), ("head_dim", _i32),
        ("kv_len", _i32), ("start_pos", _i32), ("causal", _i32), ("scale", _f32),
        ("dtype", _i32), ("out_dtype", _i32), ("kernel", _i32),
        ("workspace", _vp), ("workspace_bytes", ctypes.c_size_t),
    ]


class MlaDecodeArgs(ctypes.Structure):
    _fields_ = [
        ("q", _vp), ("latent", _vp), ("seq_lens", _vp), ("out", _vp),
        ("batch", _i32), ("q_len", _i32), ("n_heads", _i32), ("kv_rank", _i32), ("rope_dim", _i32),
        ("max_seq_len", _i32), ("num_splits", _i32), ("seq_stride", _i64), ("scale", _f32),
        ("q_dtype", _i32), ("latent_dtype", _i32), ("out_dtype", _i32), ("seq_lens_host", _vp),
        ("kernel", _i32),
    ]


class RopeParams(ctypes.Structure):
    _fields_ = [("theta", _f32), ("factor", _f32), ("original_ctx", _i32)]


class MlaAbsorbArgs(ctypes.Structure):
    _fields_ = [
        ("q", _vp), ("w_kb", _vp), ("q_abs", _vp),
        ("rows", _i32), ("n_heads", _i32), ("nope_dim", _i32), ("rope_dim", _i32), ("kv_rank", _i32),
        ("w_type", _i32), ("out_dtype", _i32), ("positions", _vp), ("rope", RopeParams),
        ("seq_base", _vp), ("rows_per_seq", _i32),
    ]


class MlaLatentWriteArgs(ctypes.Structure):
    _fields_ = [
        ("kv_a", _vp), ("norm_w", _vp), ("positions", _vp), ("latent", _vp),
        ("rows", _i32), ("rows_per_seq", _i32), ("max_seq_len", _i32), ("kv_rank", _i32), ("rope_dim", _i32),
        ("latent_dtype", _i32), ("seq_stride", _i64), ("eps", _f32), ("rope", RopeParams),
        ("seq_base", _vp),
    ]


class MlaProjectArgs(ctypes.Structure):
    _fields_ = [
        ("o", _vp), ("w_vb", _vp), ("out", _vp),
        ("rows", _i32), ("n_heads", _i32), ("kv_rank", _i32), ("v_head_dim", _i32),
        ("w_type", _i32), ("out_dtype", _i32),
    ]


class MugenAttnError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


_lib = None


def load(path: str) -> ctypes.CDLL:
    """Load the library from an explicit path instead of the in-tree build
    (side-by-side comparisons of two builds); must precede any other call."""
    global _lib
    if _lib is not None:
        raise RuntimeError("libmugen_attn is already loaded")
    return lib(path)


def lib(path: str | None = None) -> ctypes.CDLL:
    """Load libmugen_attn.so; raise if it has not been built."""
    global _lib
    if _lib is None:
        path = LIB_PATH if path is None else path
        if not os.path.exists(path):
            raise ImportError(
                f"{path} not found: build it with `python -m mugen_amd.build` "
                "(or __graft_entry__.build()); mugen_amd has no CPU fallback")
        L = ctypes.CDLL(path)
        L.mugen_attn_gqa_decode_workspace_size.argtypes = [ctypes.POINTER(GqaDecodeArgs)]
        L.mugen_attn_gqa_decode_workspace_size.restype = ctypes.c_size_t
        L.mugen_attn_gqa_decode.argtypes = [ctypes.POINTER(GqaDecodeArgs), _vp, ctypes.c_size_t, _vp]
        L.mugen_attn_gqa_decode.restype = ctypes.c_int
        L.mugen_attn_kv_q4_append.argtypes = [ctypes.POINTER(KvQ4AppendArgs), _vp]
        L.mugen_attn_kv_q4_append.restype = ctypes.c_int
        L.mugen_attn_gqa_decode_q4_workspace_size.argtypes = [ctypes.POINTER(GqaDecodeQ4Args)]
        L.mugen_attn_gqa_decode_q4_workspace_size.restype = ctypes.c_size_t
        L.mugen_attn_gqa_decode_q4.argtypes = [ctypes.POINTER(GqaDecodeQ4Args), _vp, ctypes.c_size_t, _vp]
        L.mugen_attn_gqa_decode_q4.restype = ctypes.c_int
        L.mugen_attn_gqa_prefill.argtypes = [ctypes.POINTER(GqaPrefillArgs), _vp]
        L.mugen_attn_gqa_prefill_workspace_size.argtypes = [ctypes.POINTER(GqaPrefillArgs)]
        L.mugen_attn_gqa_prefill_workspace_size.restype = ctypes.c_size_t
        L.mugen_attn_gqa_prefill.restype = ctypes.c_int
        L.mugen_attn_mla_decode_workspace_size.argtypes = [ctypes.POINTER(MlaDecodeArgs)]
        L.mugen_attn_mla_decode_workspace_size.restype = ctypes.c_size_t
        L.mugen_attn_mla_decode.argtypes = [ctypes.POINTER(MlaDecodeArgs), _vp, ctypes.c_size_t, _vp]
        L.mugen_attn_mla_decode.restype = ctypes.c_int
        L.mugen_attn_mla_decode_noalloc.argtypes = [ctypes.POINTER(MlaDecodeArgs), _vp]
        L.mugen_attn_mla_decode_noalloc.restype = ctypes.c_int
        L.mugen_attn_mla_absorb.argtypes = [ctypes.POINTER(MlaAbsorbArgs), _vp]
        L.mugen_attn_mla_absorb.restype = ctypes.c_int
        L.mugen_attn_mla_project.argtypes = [ctypes.POINTER(MlaProjectArgs), _vp]
        L.mugen_attn_mla_project.restype = ctypes.c_int
        L.mugen_attn_mla_latent_write.argtypes = [ctypes.POINTER(MlaLatentWriteArgs), _vp]
        L.mugen_attn_mla_latent_write.restype = ctypes.c_int
        L.mugen_attn_mla_prepare.argtypes = [ctypes.POINTER(MlaLatentWriteArgs), ctypes.POINTER(MlaAbsorbArgs), _vp]
        L.mugen_attn_mla_prepare.restype = ctypes.c_int
        L.mugen_attn_kv_append.argtypes = [ctypes.POINTER(KvAppendArgs), _vp]
        L.mugen_attn_kv_append.restype = ctypes.c_int
        L.mugen_attn_seq_advance.argtypes = [_vp, _i32, _i32, _i32, _vp, _vp, _vp]
        L.mugen_attn_seq_advance.restype = ctypes.c_int
        L.mugen_attn_scatter_kv.argtypes = [_vp, _vp, ctypes.c_uint64, ctypes.c_uint64, _vp]
        L.mugen_attn_scatter_kv.restype = ctypes.c_int
        L.mugen_attn_last_error.restype = ctypes.c_char_p
        L.mugen_attn_version.restype = ctypes.c_char_p
        L.mugen_attn_timing_enable.argtypes = [ctypes.c_int]
        L.mugen_attn_timing_read.argtypes = [ctypes.c_char_p, ctypes.POINTER(ctypes.c_double),
                                             ctypes.POINTER(_i64)]
        L.mugen_attn_timing_reset.restype = None
        _lib = L
    return _lib


def check(rc: int) -> None:
    if rc != OK:
        raise MugenAttnError(rc, lib().mugen_attn_last_error().decode())


def version() -> str:
    return lib().mugen_attn_version().decode()


def timing_enable(on: bool) -> None:
    check(lib().mugen_attn_timing_enable(1 if on else 0))


def timing_read(kernel: str) -> tuple[float, int]:
    ms = ctypes.c_double(0.0)
    n = _i64(0)
    check(lib().mugen_attn_timing_read(kernel.encode(), ctypes.byref(ms), ctypes.byref(n)))
    return ms.value, n.value


def timing_reset() -> None:
    lib().mugen_attn_timing_reset()
