"""create_attention_provider end to end (include/mugen_attn_engine.hpp): the
factory that replaces the reference's use_gpu_attention_ choice at load
(transformer.cpp:3430, override :2637) creates the provider for each of the
reference's model shapes, and what that provider computes -- prompt chunks
through prefill_layer, then two replays of one captured decode step -- is
compared with the CPU oracle.

tests/cpp/factory_check.cpp drives the providers (built by
__graft_entry__.build() next to the library) and writes every input and
output; this file rebuilds the caches from those inputs and runs the oracle:
  * Llama-3.2-1B (32/8, d64) and Qwen2.5-7B (28/4, d128) -> GqaAttention:
    causal prefill over the f16 cache, decode over prompt + steps;
  * 16/2 heads, d64 -> GqaAttentionQ4 (the reference's cpu_attention over
    its 4-bit KVCache): the same, decode reading tokens older than the
    newest 256 through the 4-bit groups (kv_cache.cpp:218-278);
  * 16/8 heads at head_dim 256 -> GqaAttention (the 256-wide kernels);
  * DeepSeek-V2-Lite (MLA, 16 heads) -> MlaAttention: the latent rows written
    by the prompt chunks and steps (RMSNorm + YaRN RoPE), then
    cpu_mla_attention (absorb, core, project) for each decode step."""
import os
import subprocess

import numpy as np
import pytest

from oracle import oracle as O
from tests import cases as C

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "tests", "cpp", "factory_check")
CONFIGS = {"llama1b": "GqaAttention", "qwen7b": "GqaAttention", "hk2_d64": "GqaAttentionQ4",
           "v2lite": "MlaAttention", "wide_d256": "GqaAttention"}
PRESERVE = 256  # ProviderLimits::fp16_preserve_last, the reference's KVCacheConfig value


@pytest.fixture(scope="module")
def dumps(tmp_path_factory, device):
    assert os.path.exists(EXE), "tests/cpp/factory_check is built by __graft_entry__.build()"
    out = str(tmp_path_factory.mktemp("factory"))
    C.say("factory_check " + " ".join(CONFIGS))
    r = subprocess.run([EXE, out, *CONFIGS], capture_output=True, text=True, timeout=120)
    print(r.stdout[-3000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0 and r.stdout.strip().endswith("PASS"), r.stdout[-2000:]
    return out


def load(dirname):
    arrays, meta = {}, {}
    with open(os.path.join(dirname, "manifest.txt")) as f:
        for line in f:
            parts = line.split()
            if parts[0].startswith("#"):
                meta[parts[0][1:]] = parts[1:]
                continue
            name, dt, dims = parts[0], parts[1], [int(x) for x in parts[2:]]
            raw = np.fromfile(os.path.join(dirname, name + ".bin"), np.uint16)
            arrays[name] = raw.reshape(dims)
    return arrays, meta


def f16(bits):
    return O.bits_to_f32(bits, C.F16)


@pytest.mark.parametrize("name", ["llama1b", "qwen7b", "hk2_d64", "wide_d256"])
def test_gqa_providers(dumps, name):
    a, meta = load(os.path.join(dumps, name))
    assert meta["path"] == [CONFIGS[name]]
    H, Hk, D, layers, B, steps, _ = (int(x) for x in meta["shape"])
    prompt = [int(x) for x in meta["prompt"]]
    row = Hk * D
    for L in range(layers):
        for b in range(B):
            P = prompt[b]
            q, k, v = (f16(a[f"prompt_{x}_s{b}_L{L}"]) for x in "qkv")
            ref = O.gqa_prefill(q, k, v, P, H, Hk, D, P, 0, nthreads=8)
            C.assert_close(f16(a[f"prompt_out_s{b}_L{L}"]), ref, f"{name} prompt seq {b} layer {L}")
        for t in range(steps):
            T = max(prompt) + t + 1
            kc = np.zeros((B, T, row), np.uint16)
            vc = np.zeros((B, T, row), np.uint16)
            lens = []
            for b in range(B):
                ks = [a[f"prompt_k_s{b}_L{L}"]] + [a[f"step_k_t{s}_L{L}"][b:b + 1] for s in range(t + 1)]
                vs = [a[f"prompt_v_s{b}_L{L}"]] + [a[f"step_v_t{s}_L{L}"][b:b + 1] for s in range(t + 1)]
                kb, vb = np.concatenate(ks), np.concatenate(vs)
                n = kb.shape[0]
                if CONFIGS[name] == "GqaAttentionQ4":  # tokens older than the newest 256 read from the groups
                    kb, vb = O.kvq4_read(kb, max(0, n - PRESERVE)), O.kvq4_read(vb, max(0, n - PRESERVE))
                kc[b, :n], vc[b, :n] = kb, vb
                lens.append(n)
            ref = O.gqa_attention(f16(a[f"step_q_t{t}_L{L}"]), f16(kc), f16(vc), lens, H, Hk, D, T * row,
                                  nthreads=8)
            C.assert_close(f16(a[f"step_out_t{t}_L{L}"]), ref, f"{name} decode step {t} layer {L} lens {lens}")


def test_mla_provider(dumps):
    a, meta = load(os.path.join(dumps, "v2lite"))
    assert meta["path"] == ["MlaAttention"]
    H, _, _, layers, B, steps, max_T = (int(x) for x in meta["shape"])
    prompt = [int(x) for x in meta["prompt"]]
    theta, factor, orig, chunk = float(meta["rope"][0]), float(meta["rope"][1]), int(meta["rope"][2]), \
        int(meta["rope"][3])
    freqs = O.yarn_freqs(64, factor, orig, theta)
    eps = 1e-6
    for L in range(layers):
        norm = a[f"norm_w_L{L}"]
        w_kb = a[f"w_kb_L{L}"].view(np.uint8)
        w_vb = a[f"w_vb_L{L}"].view(np.uint8)
        lat = np.zeros((B, max_T, 576), np.uint16)
        for b in range(B):
            for t0 in range(0, prompt[b], chunk):
                kva = a[f"prompt_kva_s{b}_c{t0}_L{L}"]
                pos = np.arange(t0, t0 + kva.shape[0], dtype=np.int32)
                lat[b:b + 1] = O.mla_latent_write(kva, norm, pos, lat[b:b + 1], kva.shape[0], max_T, freqs, eps)
        for t in range(steps):
            pos = np.array([p + t for p in prompt], np.int32)
            lat = O.mla_latent_write(a[f"step_kva_t{t}_L{L}"], norm, pos, lat, 1, max_T, freqs, eps)
            q = O.rope_q_f16(a[f"step_q_t{t}_L{L}"], pos, freqs).reshape(B, 1, H, 192)
            ref = O.mla_full(f16(q), w_kb, w_vb, O.W_F16, f16(lat), pos + 1, 1, H, C.MLA_SCALE, nthreads=8)
            got = f16(a[f"step_out_t{t}_L{L}"]).reshape(B, 1, H, 128)
            C.assert_close(got, ref, f"v2lite decode step {t} layer {L} lens {list(pos + 1)}")
