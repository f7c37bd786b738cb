"""C-ABI library checks that need no GPU: it loads, exports every function
include/mugen_attn.h declares, and rejects bad arguments before touching
the device (validation runs on the host)."""
import ctypes
import os
import re

import pytest

from mugen_amd import _capi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    src = open(os.path.join(ROOT, "include", "mugen_attn.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(mugen_attn_\w+)\s*\(", src)))


def test_library_loads_and_exports_every_declared_symbol():
    L = _capi.lib()
    declared = header_functions()
    assert len(declared) >= 11
    for name in declared:
        assert hasattr(L, name), f"{name} declared in mugen_attn.h but not exported"
    assert sorted(declared) == sorted(_capi.EXPORTS)
    assert "gfx950" in _capi.version()


def _gqa_args(**kw):
    a = _capi.GqaDecodeArgs()
    a.q = a.k_cache = a.v_cache = a.seq_lens = a.out = 0x1000
    a.batch, a.n_heads, a.n_kv_heads, a.head_dim, a.max_seq_len = 1, 28, 4, 128, 4096
    a.seq_stride, a.kv_dtype, a.out_dtype = 0, _capi.F16, _capi.F16
    for k, v in kw.items():
        setattr(a, k, v)
    return a


def _call_gqa(a, ws=None, nbytes=0):
    return _capi.lib().mugen_attn_gqa_decode(ctypes.byref(a), ws, nbytes, None)


@pytest.mark.parametrize("kw,code", [
    (dict(q=0), _capi.E_INVALID),
    (dict(n_heads=30), _capi.E_INVALID),          # not a multiple of n_kv_heads
    (dict(head_dim=100), _capi.E_UNSUPPORTED),    # not a multiple of 8
    (dict(head_dim=264), _capi.E_UNSUPPORTED),    # above 256
    (dict(n_heads=68, n_kv_heads=4), _capi.E_UNSUPPORTED),  # G = 17 > 16
    (dict(kv_dtype=_capi.F32), _capi.E_UNSUPPORTED),
    (dict(batch=2, seq_stride=10), _capi.E_INVALID),
    (dict(q=0x1002), _capi.E_INVALID),            # misaligned
])
def test_gqa_decode_rejects_bad_args(kw, code):
    assert _call_gqa(_gqa_args(**kw)) == code
    assert _capi.lib().mugen_attn_last_error().decode()


def test_gqa_workspace_size_and_missing_workspace():
    a = _gqa_args()
    need = _capi.lib().mugen_attn_gqa_decode_workspace_size(ctypes.byref(a))
    assert need > 0
    assert _call_gqa(a) == _capi.E_WORKSPACE
    assert "workspace" in _capi.lib().mugen_attn_last_error().decode()
    a1 = _gqa_args(num_splits=1)
    assert _capi.lib().mugen_attn_gqa_decode_workspace_size(ctypes.byref(a1)) == 0


def _gqa_splits(a):
    # the workspace holds B * H * splits fp32 partials of padded head_dim plus (m, l)
    ws = _capi.lib().mugen_attn_gqa_decode_workspace_size(ctypes.byref(a))
    return 1 if ws == 0 else (ws - 256) // (a.batch * a.n_heads * (4 * 128 + 8))


def _host_lens(lens):
    arr = (ctypes.c_int32 * len(lens))(*lens)
    return arr, ctypes.addressof(arr)


@pytest.mark.parametrize("B,T,splits", [(1, 512, 8), (1, 2048, 32), (1, 4096, 32), (1, 8192, 32), (2, 8192, 32),
                                         (4, 8192, 32), (8, 8192, 16)])
def test_gqa_decode_plan(B, T, splits):
    # the longest sequence in at most 32 splits of 64+ tokens, one round of
    # 512 workgroups (B * Hk * splits): the measured optimum at 1-2
    # sequences, where the smallest chunk that fits the round gave 64 splits
    # at T = 8192 and 16 at T = 2048
    a = _gqa_args(batch=B, max_seq_len=T, seq_stride=T * 4 * 128)
    keep, a.seq_lens_host = _host_lens([T] * B)  # exact plan sizes
    assert _gqa_splits(a) == splits


def test_decode_workspace_without_host_lengths_covers_every_plan():
    # a workspace sized once without host lengths serves every call that
    # passes them (short batches in a long cache plan finer chunks)
    import random
    rnd = random.Random(5)
    for _ in range(200):
        B = rnd.randint(1, 16)
        T = rnd.choice([256, 1024, 4096, 8192, 32768])
        lens = [rnd.randint(0, T) for _ in range(B)]
        a = _gqa_args(batch=B, max_seq_len=T, seq_stride=T * 4 * 128)
        size = _capi.lib().mugen_attn_gqa_decode_workspace_size
        bound = size(ctypes.byref(a))
        keep, a.seq_lens_host = _host_lens(lens)
        assert size(ctypes.byref(a)) <= bound, (B, T, lens)
        m = _mla_args(batch=B, n_heads=rnd.choice([16, 128]), q_len=rnd.choice([1, 5]), max_seq_len=T,
                      seq_stride=T * 576)
        msize = _capi.lib().mugen_attn_mla_decode_workspace_size
        mbound = msize(ctypes.byref(m))
        keep2, m.seq_lens_host = _host_lens([max(v, m.q_len) for v in lens])
        assert msize(ctypes.byref(m)) <= mbound, (B, T, lens)


def _mla_args(**kw):
    a = _capi.MlaDecodeArgs()
    a.q = a.latent = a.seq_lens = a.out = 0x1000
    a.batch, a.q_len, a.n_heads, a.kv_rank, a.rope_dim = 8, 1, 128, 512, 64
    a.max_seq_len, a.seq_stride, a.scale = 8192, 8192 * 576, 0.0721
    a.q_dtype = a.latent_dtype = _capi.BF16
    a.out_dtype = _capi.F32
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("kw,code", [
    (dict(latent=0), _capi.E_INVALID),
    (dict(kv_rank=256), _capi.E_UNSUPPORTED),
    (dict(scale=0.0), _capi.E_INVALID),
    (dict(q_dtype=_capi.F16), _capi.E_UNSUPPORTED),  # neither f32 nor the latent dtype
    (dict(seq_stride=100), _capi.E_INVALID),
])
def test_mla_rejects_bad_args(kw, code):
    a = _mla_args(**kw)
    assert _capi.lib().mugen_attn_mla_decode(ctypes.byref(a), None, 0, None) == code


def _mla_splits(a):
    # fp16 O blocks of 16 rows plus fp32 (m, l) per row, per (sequence, split)
    ws = _capi.lib().mugen_attn_mla_decode_workspace_size(ctypes.byref(a))
    R = a.q_len * a.n_heads
    return (ws - 256) // (a.batch * ((R + 15) // 16 * 16 * 512 * 2 + R * 8))


@pytest.mark.parametrize("B,H,q_len,T,splits", [(1, 16, 1, 1024, 32), (1, 16, 1, 8192, 32), (1, 128, 1, 8192, 32),
                                                 (8, 128, 1, 8192, 16), (4, 128, 5, 32768, 6)])
def test_mla_decode_plan(B, H, q_len, T, splits):
    # the longest sequence in at most 32 splits, one round of 256 workgroups
    # (row blocks x splits): V2-Lite heads at T = 8192 once took 256
    # one-tile splits (36.5 us against 16.9 with 32)
    a = _mla_args(batch=B, n_heads=H, q_len=q_len, max_seq_len=T, seq_stride=T * 576)
    keep, a.seq_lens_host = _host_lens([T] * B)  # exact plan sizes
    assert _mla_splits(a) == splits


def test_mla_workspace():
    a = _mla_args()
    need = _capi.lib().mugen_attn_mla_decode_workspace_size(ctypes.byref(a))
    assert need >= 8 * 128 * 512 * 4
    assert _capi.lib().mugen_attn_mla_decode(ctypes.byref(a), None, 0, None) == _capi.E_WORKSPACE


def test_prefill_rejects_bad_args():
    a = _capi.GqaPrefillArgs()
    a.q = a.k = a.v = a.out = 0x1000
    a.n_tokens, a.n_heads, a.n_kv_heads, a.head_dim, a.kv_len, a.start_pos, a.causal = 512, 32, 8, 64, 100, 0, 1
    a.dtype = a.out_dtype = _capi.BF16
    assert _capi.lib().mugen_attn_gqa_prefill(ctypes.byref(a), None) == _capi.E_INVALID  # kv_len < N
    a.kv_len, a.head_dim = 512, 84   # not a multiple of 8
    assert _capi.lib().mugen_attn_gqa_prefill(ctypes.byref(a), None) == _capi.E_UNSUPPORTED
    a.head_dim = 264  # above 256
    assert _capi.lib().mugen_attn_gqa_prefill(ctypes.byref(a), None) == _capi.E_UNSUPPORTED
    a.head_dim, a.n_tokens = 64, 0
    assert _capi.lib().mugen_attn_gqa_prefill(ctypes.byref(a), None) == _capi.OK  # nothing to do
    a.n_heads, a.n_kv_heads = 32, 1  # 32 heads per kv head
    assert _capi.lib().mugen_attn_gqa_prefill(ctypes.byref(a), None) == _capi.E_UNSUPPORTED
    a.n_kv_heads, a.kernel = 2, _capi.PREFILL_KERNEL_BLOCK  # 16 per kv head: the per-block kernel cannot
    assert _capi.lib().mugen_attn_gqa_prefill(ctypes.byref(a), None) == _capi.E_UNSUPPORTED
    a.kernel = 0
    assert _capi.lib().mugen_attn_gqa_prefill(ctypes.byref(a), None) == _capi.OK
    a.kernel = 4
    assert _capi.lib().mugen_attn_gqa_prefill(ctypes.byref(a), None) == _capi.E_INVALID


@pytest.mark.parametrize("n_tokens,start,kv_len,causal,H,Hk,hd", [
    (512, 1, 513, 1, 32, 8, 64),   # 513 visible keys
    (100, 0, 513, 0, 32, 8, 64),   # non-causal: all of kv_len is visible
    (64, 0, 64, 1, 32, 4, 64),     # 8 heads per kv head
    (64, 0, 64, 1, 32, 8, 128),    # head_dim 128
    (64, 0, 64, 1, 32, 8, 56),     # padded head_dim
])
def test_prefill_short_kernel_refused_outside_its_range(n_tokens, start, kv_len, causal, H, Hk, hd):
    # forcing the short kernel where it does not apply is refused before any
    # launch (the pointers are placeholders)
    a = _capi.GqaPrefillArgs()
    a.q = a.k = a.v = a.out = 0x1000
    a.n_tokens, a.n_heads, a.n_kv_heads, a.head_dim = n_tokens, H, Hk, hd
    a.kv_len, a.start_pos, a.causal = kv_len, start, causal
    a.dtype = a.out_dtype = _capi.BF16
    a.kernel = _capi.PREFILL_KERNEL_SHORT
    assert _capi.lib().mugen_attn_gqa_prefill(ctypes.byref(a), None) == _capi.E_UNSUPPORTED


def test_scatter_kv_validation():
    assert _capi.lib().mugen_attn_scatter_kv(None, None, 0, 0, None) == _capi.OK
    assert _capi.lib().mugen_attn_scatter_kv(None, None, 0, 5, None) == _capi.E_INVALID


def test_python_front_end_refuses_cpu_tensors():
    import torch
    import mugen_amd
    q = torch.zeros(1, 4, 64, dtype=torch.float16)
    k = torch.zeros(1, 8, 1, 64, dtype=torch.float16)
    with pytest.raises(ValueError, match="device tensors"):
        mugen_amd.attention_decode(q, k, k, torch.ones(1, dtype=torch.int32))


ADAPTER_PROGRAM = r"""
#include "mugen_attn.hpp"
#include <cstdio>
int main() {
    mugen_attn_gqa_decode_args a{};                // null pointers: rejected on the host
    auto r = mugen_attn::gqa_decode(a, nullptr, 0, nullptr);
    if (r || r.has_value() || r.error().empty()) return 1;
    auto ok = mugen_attn::check(MUGEN_ATTN_OK);
    if (!ok) return 2;
    std::printf("%s\n", r.error().c_str());
    return 0;
}
"""


def test_cpp_adapter_maps_status_to_expected(tmp_path):
    """include/mugen_attn.hpp compiles as C++20 and C++23 and turns a
    rejected call into a failed Status carrying the library's message."""
    import shutil
    import subprocess
    cxx = shutil.which("g++")
    if cxx is None:
        pytest.skip("no host C++ compiler")
    src = tmp_path / "adapter.cpp"
    src.write_text(ADAPTER_PROGRAM)
    libdir = os.path.join(ROOT, "mugen_amd")
    for std in ("c++20", "c++23"):
        exe = tmp_path / f"adapter_{std}"
        subprocess.run([cxx, f"-std={std}", "-Wall", "-Werror", str(src), "-I", os.path.join(ROOT, "include"),
                        "-L", libdir, "-lmugen_attn", f"-Wl,-rpath,{libdir}", "-Wl,-rpath,/opt/rocm/lib",
                        "-o", str(exe)], check=True)
        out = subprocess.run([str(exe)], capture_output=True, text=True)
        assert out.returncode == 0, out
        assert out.stdout.strip()


def test_mla_absorb_project_validation():
    L = _capi.lib()
    a = _capi.MlaAbsorbArgs()
    a.q = a.w_kb = a.q_abs = 0x1000
    a.rows, a.n_heads, a.nope_dim, a.rope_dim, a.kv_rank = 4, 16, 128, 64, 512
    a.w_type, a.out_dtype = _capi.W_Q8_0, _capi.F32
    for field, val, code in [("nope_dim", 64, _capi.E_UNSUPPORTED), ("w_type", 3, _capi.E_UNSUPPORTED),
                             ("out_dtype", _capi.F16, _capi.E_UNSUPPORTED), ("q", 0, _capi.E_INVALID),
                             ("q", 0x1001, _capi.E_INVALID), ("n_heads", 0, _capi.E_INVALID)]:
        b = _capi.MlaAbsorbArgs.from_buffer_copy(a)
        setattr(b, field, val)
        assert L.mugen_attn_mla_absorb(ctypes.byref(b), None) == code, field
    b = _capi.MlaAbsorbArgs.from_buffer_copy(a)
    b.w_type, b.w_kb = _capi.W_F16, 0x1002          # f16 rows are read 16 bytes at a time
    assert L.mugen_attn_mla_absorb(ctypes.byref(b), None) == _capi.E_INVALID
    b.rows = 0
    assert L.mugen_attn_mla_absorb(ctypes.byref(b), None) == _capi.OK
    b = _capi.MlaAbsorbArgs.from_buffer_copy(a)      # device seq_base positions need tokens per sequence
    b.seq_base, b.rows_per_seq = 0x1000, 0
    assert L.mugen_attn_mla_absorb(ctypes.byref(b), None) == _capi.E_INVALID
    p = _capi.MlaProjectArgs()
    p.o = p.w_vb = p.out = 0x1000
    p.rows, p.n_heads, p.kv_rank, p.v_head_dim, p.w_type, p.out_dtype = 4, 16, 512, 128, _capi.W_Q4_0, _capi.F16
    for field, val, code in [("v_head_dim", 64, _capi.E_UNSUPPORTED), ("out_dtype", _capi.BF16, _capi.E_UNSUPPORTED),
                             ("o", 0x1008, _capi.E_INVALID), ("w_vb", 0, _capi.E_INVALID)]:
        b = _capi.MlaProjectArgs.from_buffer_copy(p)
        setattr(b, field, val)
        assert L.mugen_attn_mla_project(ctypes.byref(b), None) == code, field


def test_latent_write_validation():
    L = _capi.lib()
    a = _capi.MlaLatentWriteArgs()
    a.kv_a = a.norm_w = a.positions = a.latent = 0x1000
    a.rows, a.rows_per_seq, a.max_seq_len, a.kv_rank, a.rope_dim = 4, 1, 64, 512, 64
    a.latent_dtype, a.seq_stride, a.eps = _capi.F16, 64 * 576, 1e-6
    a.rope = _capi.RopeParams(10000.0, 40.0, 4096)
    for field, val, code in [("kv_rank", 256, _capi.E_UNSUPPORTED), ("latent_dtype", _capi.F32, _capi.E_UNSUPPORTED),
                             ("rows_per_seq", 0, _capi.E_INVALID), ("seq_stride", 100, _capi.E_INVALID),
                             ("latent", 0x1008, _capi.E_INVALID), ("positions", 0, _capi.E_INVALID),
                             ("eps", float("nan"), _capi.E_INVALID)]:
        b = _capi.MlaLatentWriteArgs.from_buffer_copy(a)
        setattr(b, field, val)
        assert L.mugen_attn_mla_latent_write(ctypes.byref(b), None) == code, field
    b = _capi.MlaLatentWriteArgs.from_buffer_copy(a)
    b.rope = _capi.RopeParams(10000.0, 40.0, 0)     # YaRN needs the original context
    assert L.mugen_attn_mla_latent_write(ctypes.byref(b), None) == _capi.E_INVALID
    b.rope, b.rows = _capi.RopeParams(10000.0, 0.0, 0), 0
    assert L.mugen_attn_mla_latent_write(ctypes.byref(b), None) == _capi.OK
    b = _capi.MlaLatentWriteArgs.from_buffer_copy(a)  # seq_base replaces positions; one of them is needed
    b.positions, b.seq_base = 0, 0x1000
    b.rows = 0
    assert L.mugen_attn_mla_latent_write(ctypes.byref(b), None) == _capi.OK
    b.seq_base, b.rows = 0, 4
    assert L.mugen_attn_mla_latent_write(ctypes.byref(b), None) == _capi.E_INVALID


def test_kv_q4_validation():
    L = _capi.lib()
    st = _capi.KvQ4Store(0x1000, 0x1000, 0x1000, 0x1000, 64 * 320, 512 * 512, 512, 256)
    a = _capi.KvQ4AppendArgs()
    a.store = st
    a.k_new = a.v_new = a.seq_lens = a.n_q4 = 0x1000
    a.n_q4_out = 0x2000
    a.n_seq, a.n_new, a.n_kv_heads, a.head_dim, a.max_seq_len = 2, 8, 4, 128, 64
    # every case below fails validation on the host (nothing is launched)
    for field, val in [("n_q4_out", 0x1000), ("k_new", 0x1004), ("n_new", 257)]:
        b = _capi.KvQ4AppendArgs.from_buffer_copy(a)
        setattr(b, field, val)
        assert L.mugen_attn_kv_q4_append(ctypes.byref(b), None) == _capi.E_INVALID, field
    b = _capi.KvQ4AppendArgs.from_buffer_copy(a)
    b.n_kv_heads, b.head_dim = 3, 10                                              # 30 values: not whole groups
    assert L.mugen_attn_kv_q4_append(ctypes.byref(b), None) == _capi.E_UNSUPPORTED
    d = _capi.GqaDecodeQ4Args()
    d.q, d.store, d.seq_lens, d.n_q4, d.out = 0x1000, st, 0x1000, 0, 0x1000
    d.batch, d.n_heads, d.n_kv_heads, d.head_dim, d.max_seq_len, d.out_dtype = 2, 28, 4, 128, 64, _capi.F16
    assert L.mugen_attn_gqa_decode_q4(ctypes.byref(d), None, 0, None) == _capi.E_INVALID   # null n_q4
    d.n_q4 = 0x1000
    d.store.q4_k = 0x1002
    assert L.mugen_attn_gqa_decode_q4(ctypes.byref(d), None, 0, None) == _capi.E_INVALID   # misaligned store
    d.store.q4_k, d.store.ring = 0x1000, 300
    assert L.mugen_attn_gqa_decode_q4(ctypes.byref(d), None, 0, None) == _capi.E_INVALID   # ring not a power of two
    d.store.ring, d.head_dim = 512, 96
    assert L.mugen_attn_gqa_decode_q4(ctypes.byref(d), None, 0, None) == _capi.E_UNSUPPORTED  # 4-bit store: 64/128


def test_engine_header_compiles(tmp_path):
    """include/mugen_attn_engine.hpp (the C++ provider) compiles as C++20 and
    C++23 host code against the HIP runtime headers."""
    import shutil
    import subprocess
    cxx = shutil.which("g++")
    if cxx is None or not os.path.isdir("/opt/rocm/include"):
        pytest.skip("no host C++ compiler / ROCm headers")
    src = tmp_path / "engine.cpp"
    src.write_text('#include "mugen_attn_engine.hpp"\n'
                   "int main() { mugen_attn::GqaShape s; mugen_attn::StepGraph g; return s.n_layers; }\n")
    for std in ("c++20", "c++23"):
        subprocess.run([cxx, f"-std={std}", "-Wall", "-Werror", "-D__HIP_PLATFORM_AMD__", "-c", str(src),
                        "-I", os.path.join(ROOT, "include"), "-I", "/opt/rocm/include", "-o",
                        str(tmp_path / f"engine_{std}.o")], check=True)


def test_kv_append_and_seq_advance_validation():
    L = _capi.lib()
    a = _capi.KvAppendArgs()
    a.k_new = a.v_new = a.k_cache = a.v_cache = a.seq_lens = 0x1000
    a.seq_stride, a.n_seq, a.n_new, a.row, a.max_seq_len = 64 * 512, 2, 1, 512, 64
    for field, val in [("row", 12), ("seq_stride", 100), ("k_cache", 0x1004), ("seq_lens", 0)]:
        b = _capi.KvAppendArgs.from_buffer_copy(a)
        setattr(b, field, val)
        assert L.mugen_attn_kv_append(ctypes.byref(b), None) in (_capi.E_INVALID, _capi.E_UNSUPPORTED), field
    assert L.mugen_attn_seq_advance(None, 1, 4, 64, None, None, None) == _capi.E_INVALID
    assert L.mugen_attn_seq_advance(None, 1, 0, 64, None, None, None) == _capi.OK


def test_prefill_workspace_size():
    a = _capi.GqaPrefillArgs()
    a.q = a.k = a.v = a.out = 0x1000
    a.n_tokens, a.n_heads, a.n_kv_heads, a.head_dim, a.kv_len, a.start_pos, a.causal = 2048, 28, 4, 128, 2048, 0, 1
    a.dtype = a.out_dtype = _capi.BF16
    size = _capi.lib().mugen_attn_gqa_prefill_workspace_size
    assert size(ctypes.byref(a)) == 2048 * 4 * 128 * 2 + 256     # the fp16 copy of V
    a.n_tokens, a.start_pos = 1000, 1048                         # a short prompt: no copy
    assert size(ctypes.byref(a)) == 0
    a.n_tokens, a.start_pos, a.dtype = 2048, 0, _capi.F16        # f16 inputs need none
    assert size(ctypes.byref(a)) == 0
    a.dtype, a.head_dim = _capi.BF16, 84                         # invalid args: 0
    assert size(ctypes.byref(a)) == 0
    # a 256-token chunk after 7900 cached tokens: 64 workgroups unsplit, so
    # each block's 8156 keys go to 4 ranges of 2048 (32 steps of 64 keys);
    # the partials are fp16 O / l plus fp32 (max, sum) per row and range
    a.n_tokens, a.start_pos, a.kv_len, a.head_dim, a.dtype = 256, 7900, 8156, 128, _capi.F16
    assert size(ctypes.byref(a)) == 256 * 28 * 4 * (128 * 2 + 8) + 512
    a.causal = 0                                                 # non-causal: the same key range here
    assert size(ctypes.byref(a)) == 256 * 28 * 4 * (128 * 2 + 8) + 512
    a.dtype = _capi.BF16                                         # BF16: the fp16 V copy first
    assert size(ctypes.byref(a)) == 8156 * 4 * 128 * 2 + 256 + 256 * 28 * 4 * (128 * 2 + 8) + 512
    a.dtype = _capi.F16
    a.causal, a.kernel = 1, _capi.PREFILL_KERNEL_BLOCK            # a forced non-split kernel: none
    assert size(ctypes.byref(a)) == 0
    a.kernel, a.start_pos, a.kv_len = 0, 0, 256                  # a short range: no split
    assert size(ctypes.byref(a)) == 0
    # the size never falls as the range grows (an engine sizes one workspace
    # at the end of its cache for every shorter context)
    for n, H, Hk, dt in [(64, 28, 4, _capi.F16), (256, 8, 1, _capi.F16), (48, 32, 2, _capi.F16),
                         (100, 32, 8, _capi.F16), (64, 28, 4, _capi.BF16), (256, 28, 4, _capi.BF16),
                         (16, 8, 1, _capi.BF16), (100, 32, 8, _capi.BF16), (256, 32, 8, _capi.F16)]:
        a.n_tokens, a.n_heads, a.n_kv_heads, a.dtype = n, H, Hk, dt
        last = 0
        for start in range(0, 20000, 37):
            a.start_pos, a.kv_len = start, start + n
            got = size(ctypes.byref(a))
            assert got >= last, (n, H, Hk, start)
            last = got
        assert last > 0
