"""The engine hook: a decode step's attention calls captured once into a
HIP graph and replayed step after step, every per-step value (positions,
lengths) read from device memory -- the counterpart of the reference's
cached mega-chain (transformer.cpp:3734-3833), which patches pos /
kv_offset / seq_len into its cached dispatches before each step.

* test_cpp_provider_selftest: the C++ provider (include/mugen_attn_engine.hpp)
  replays captured multi-layer GQA, 4-bit-store GQA and MLA (decode and
  verify) steps bit-identically to eager calls; prompt chunks through
  prefill_layer (one sequence of a batch, both GQA providers) match a direct
  prefill; an MLA prompt in one call matches the token-by-token path; and
  lengths past the caches are refused (mugen_amd/engine_selftest.cpp);
* test_step_graph_replays_match_oracle: a captured step (kv_append +
  decode per layer + seq_advance) replayed several times, with eager uploads
  and synchronisations between replays, each replay checked against the
  oracle at that step's lengths."""
import os
import subprocess

import numpy as np
import pytest
import torch

import mugen_amd
from oracle import oracle as O
from tests import cases as C

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_cpp_provider_selftest(device):
    exe = os.path.join(ROOT, "mugen_amd", "engine_selftest")
    assert os.path.exists(exe), "engine_selftest is built by mugen_amd/build.py"
    C.say("engine_selftest (C++ provider, captured step vs eager)")
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    print(r.stdout[-4000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0 and r.stdout.strip().endswith("PASS"), r.stdout[-2000:]
    for part in ("gqa provider done", "mla provider done", "gqa prefill provider done", "gqa q4 provider done",
                 "prompt in a batch done", "mla prompt done", "length bounds done"):
        assert part in r.stdout, part


def test_step_graph_replays_match_oracle(device):
    n_layers, B, H, Hk, D, max_T = 2, 3, 28, 4, 128, 600
    lens = np.array([400, 1, 77], np.int32)
    steps = 4
    row = Hk * D
    K = [O.round_to(O.randn(300 + l, (B, max_T, row)), C.F16)[1] for l in range(n_layers)]
    V = [O.round_to(O.randn(400 + l, (B, max_T, row)), C.F16)[1] for l in range(n_layers)]
    kc = [C.to_dev(k, C.F16, device).view(B, max_T, Hk, D) for k in K]
    vc = [C.to_dev(v, C.F16, device).view(B, max_T, Hk, D) for v in V]
    seq = torch.from_numpy(np.concatenate([lens, lens + 1])).to(device)   # [before | after] the append
    q_in = [torch.empty((B, H, D), dtype=torch.float16, device=device) for _ in range(n_layers)]
    k_in = [torch.empty((B, 1, row), dtype=torch.float16, device=device) for _ in range(n_layers)]
    v_in = [torch.empty((B, 1, row), dtype=torch.float16, device=device) for _ in range(n_layers)]
    out = [torch.empty((B, H, D), dtype=torch.float32, device=device) for _ in range(n_layers)]
    ws = [torch.empty(1 << 24, dtype=torch.uint8, device=device) for _ in range(n_layers)]

    def step():
        for l in range(n_layers):
            mugen_amd.kv_append(k_in[l], v_in[l], kc[l], vc[l], seq[:B])
            mugen_amd.attention_decode(q_in[l], kc[l], vc[l], seq[B:], max_T, out=out[l], workspace=ws[l])
        mugen_amd.seq_advance(seq, 1, max_T)

    C.say(f"captured GQA step: layers {n_layers} batch {B} lens {list(lens)}")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    torch.cuda.synchronize()
    assert seq.cpu().tolist() == list(lens) + list(lens + 1)  # capture ran nothing
    for t in range(steps):
        qs, ks, vs = [], [], []
        for l in range(n_layers):   # this step's inputs, uploaded eagerly
            qb = O.round_to(O.randn(500 + 10 * t + l, (B, H, D)), C.F16)[1]
            kb = O.round_to(O.randn(600 + 10 * t + l, (B, 1, row)), C.F16)[1]
            vb = O.round_to(O.randn(700 + 10 * t + l, (B, 1, row)), C.F16)[1]
            q_in[l].copy_(C.to_dev(qb, C.F16, device))
            k_in[l].copy_(C.to_dev(kb, C.F16, device))
            v_in[l].copy_(C.to_dev(vb, C.F16, device))
            qs.append(qb)
            for b in range(B):      # the host mirror of the append
                K[l][b, lens[b]] = kb[b, 0]
                V[l][b, lens[b]] = vb[b, 0]
        torch.cuda.synchronize()
        C.say(f"replay {t}: lens after append {list(lens + 1)}")
        g.replay()
        torch.cuda.synchronize()
        lens = lens + 1
        assert seq.cpu().tolist() == list(lens) + list(lens + 1)
        f = lambda x: x.view(np.float16).astype(np.float32)
        for l in range(n_layers):
            ref = O.gqa_attention(f(qs[l]), f(K[l]), f(V[l]), lens, H, Hk, D, max_T * row, nthreads=8)
            C.assert_close(out[l].cpu().numpy(), ref, f"replay {t} layer {l}")


@pytest.mark.parametrize("q_len", [1, 3])
def test_mla_step_graph_replays_match_oracle(device, q_len):
    # a captured MLA step (latent write -> absorb with q RoPE -> fp32-q core
    # -> projection, then the device-side length advance), replayed with
    # fresh inputs and checked against the oracle's chain.  q_len 1 is a
    # decode step; q_len 3 a speculative verify step, whose token j of
    # sequence b sits at seq_base[b] + j (the before-lengths on the device).
    B, H, max_T, w_type = 2, 16, 256, O.W_Q8_0
    rope = (10000.0, 40.0, 4096)
    freqs = O.yarn_freqs(64, rope[1], rope[2], rope[0])
    lens = np.array([100, 7], np.int32)
    _, latb = O.round_to(O.randn(800, (B, max_T, 576), 0.0, 0.5), C.F16)
    w_kb = C.make_weights(801, H * 128, 512, w_type)
    w_vb = C.make_weights(802, H * 128, 512, w_type)
    norm = O.round_to(1.0 + O.randn(803, (512,), 0.0, 0.1), C.F16)[1]
    lat = C.to_dev(latb, C.F16, device)
    wk, wv = torch.from_numpy(w_kb).to(device), torch.from_numpy(w_vb).to(device)
    nd = C.to_dev(norm, C.F16, device)
    seq = torch.from_numpy(np.concatenate([lens, lens + q_len])).to(device)   # [before | after]
    q_in = torch.empty((B, q_len, H, 192), dtype=torch.float16, device=device)
    kv_in = torch.empty((B * q_len, 576), dtype=torch.float16, device=device)
    qa = torch.empty((B, q_len, H, 576), dtype=torch.float32, device=device)
    o = torch.empty((B, q_len, H, 512), dtype=torch.float32, device=device)
    out = torch.empty((B, q_len, H, 128), dtype=torch.float16, device=device)
    ws = torch.empty(1 << 24, dtype=torch.uint8, device=device)

    def step():
        mugen_amd.mla_latent_write(kv_in, nd, None, lat, rope=rope, rows_per_seq=q_len, seq_base=seq[:B])
        mugen_amd.mla_absorb(q_in, wk, "q8_0", out=qa, rope=rope, seq_base=seq[:B], rows_per_seq=q_len)
        mugen_amd.mla_attention(qa, lat, seq[B:], max_T, scale=C.MLA_SCALE, out=o, workspace=ws)
        mugen_amd.mla_project(o, wv, "q8_0", out=out)
        mugen_amd.seq_advance(seq, q_len, max_T)

    C.say(f"captured MLA step: batch {B} q_len {q_len} H {H} lens {list(lens)}")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    torch.cuda.synchronize()
    cache = latb.copy()
    for t in range(3):
        qb = O.round_to(O.randn(810 + t, (B, q_len, H, 192)), C.F16)[1]
        kvb = O.round_to(O.randn(820 + t, (B * q_len, 576)), C.F16)[1]
        q_in.copy_(C.to_dev(qb, C.F16, device))
        kv_in.copy_(C.to_dev(kvb, C.F16, device))
        torch.cuda.synchronize()
        C.say(f"MLA replay {t}: positions {list(lens)} + [0, {q_len})")
        g.replay()
        torch.cuda.synchronize()
        pos = (lens[:, None] + np.arange(q_len, dtype=np.int32)[None, :]).reshape(-1).astype(np.int32)
        cache = O.mla_latent_write(kvb, norm, pos, cache, q_len, max_T, freqs, 1e-6)
        qr = O.rope_q_f16(qb.reshape(B * q_len, H, 192), pos, freqs).reshape(B, q_len, H, 192)
        lens = lens + q_len
        f = lambda x: x.view(np.float16).astype(np.float32)
        ref = O.mla_full(f(qr), w_kb, w_vb, w_type, f(cache), lens, q_len, H, C.MLA_SCALE, nthreads=8)
        C.assert_close(out.float().cpu().numpy(), ref, f"MLA replay {t}")
        assert seq.cpu().tolist() == list(lens) + list(lens + q_len)
