"""Which attention provider replaces the reference's use_gpu_attention_
switch (include/mugen_attn_path.hpp), checked on the CPU for the
reference's model configurations.

Reference rule (src/core/model/transformer.cpp): use_gpu_attention_ =
!is_mla() && n_kv_heads >= 4 (:3430), overridable (:2637); GQA models
without GPU attention run cpu_attention over the 4-bit KVCache (:3701-3731);
MLA models always run cpu_mla_attention (:3988-3995)."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def choices(tmp_path_factory):
    cxx = shutil.which("g++") or shutil.which("c++")
    if cxx is None:
        pytest.skip("no host C++ compiler")
    exe = str(tmp_path_factory.mktemp("path") / "path_select_check")
    subprocess.run([cxx, "-std=c++17", "-O1", "-I", os.path.join(ROOT, "include"),
                    os.path.join(ROOT, "tests", "cpp", "path_select_check.cpp"), "-o", exe], check=True)
    out = subprocess.run([exe], check=True, capture_output=True, text=True).stdout
    return {name: (path, sup == "1") for name, path, sup in (line.split() for line in out.splitlines())}


@pytest.mark.parametrize("name,path,supported", [
    ("llama1b", "GqaAttention", True),       # 8 KV heads: the reference attends on the GPU
    ("qwen7b", "GqaAttention", True),        # 4 KV heads: GPU
    ("v2lite", "MlaAttention", True),        # MLA: cpu_mla_attention, replaced by the latent kernels
    ("v3", "MlaAttention", True),
    ("tiny", "GqaAttentionQ4", False),       # 2 KV heads -> the reference's CPU path; the 4-bit store needs d 64/128
    ("tiny_on", "GqaAttention", True),       # the same model forced onto f16 caches: d 16 runs padded to 64
    ("small_kv", "GqaAttentionQ4", True),    # 2 KV heads at d 64: the 4-bit store provider
    ("moe", "GqaAttention", True),           # MoE layers attend like dense ones
    ("wide", "GqaAttention", True),          # head_dim 256: the f16-cache kernels' 256 build
    ("wide_kv2", "GqaAttentionQ4", True),    # head_dim 256, 2 KV heads: the 4-bit store at 256
    ("odd", "GqaAttention", True),           # head_dim 160: runs padded to 256
    ("odd_kv_off", "GqaAttentionQ4", False), # the 4-bit store keeps whole 32-value groups per head: 64/128/256
    ("huge", "GqaAttention", False),         # head_dim 512: beyond every kernel -> the reference's CPU path
    ("qwen7b_off", "GqaAttentionQ4", True),  # set_use_gpu_attention(false)
    ("small_kv_on", "GqaAttention", True),   # set_use_gpu_attention(true)
    ("v2lite_on", "MlaAttention", True),     # MLA ignores the override
    ("v2lite_off", "MlaAttention", True),
])
def test_provider_choice(choices, name, path, supported):
    assert choices[name] == (path, supported)
