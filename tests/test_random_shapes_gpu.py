"""Seeded random shape sweeps against the CPU oracle: MLA decode / verify /
prompt (both kernels, fp32 and 16-bit q, forced split counts), GQA decode
(head groups 1..16, both head dims, ragged and empty sequences), causal
prefill (both kernels, offsets) and short prompt chunks after long contexts
(the key-split path).  Every case draws its shape from its own
seed, so a failure names a reproducible case; sizes are bounded so the
oracle stays fast."""
import numpy as np
import pytest
import torch

import mugen_amd
from mugen_amd import _capi
from tests import cases as C

pytestmark = pytest.mark.gpu

MLA_H = [1, 3, 16, 20, 64, 128]
MLA_QLEN = [1, 1, 1, 2, 5, 9, 33, 64]


def mla_shape(seed):
    r = np.random.default_rng(1000 + seed)
    while True:
        H = int(r.choice(MLA_H))
        q_len = int(r.choice(MLA_QLEN))
        B = int(r.integers(1, 5))
        if q_len * H <= 4096:
            break
    max_T = int(r.integers(q_len, 2049))
    lens = r.integers(q_len, max_T + 1, size=B).astype(np.int32)
    lat_dt = C.F16 if r.random() < 0.5 else C.BF16
    q_dt = C.F32 if r.random() < 0.5 else lat_dt
    kernel = int(r.choice([0, _capi.MLA_KERNEL_ROWS, _capi.MLA_KERNEL_WS]))
    splits = int(r.choice([0, 0, 1, int(r.integers(2, 9))]))
    return B, q_len, H, max_T, lens, q_dt, lat_dt, kernel, splits


@pytest.mark.parametrize("seed", range(24))
def test_mla_random(device, seed):
    B, q_len, H, max_T, lens, q_dt, lat_dt, kernel, splits = mla_shape(seed)
    C.say(f"mla random seed={seed}: B={B} q_len={q_len} H={H} max_T={max_T} lens={list(lens)} q={q_dt} "
          f"lat={lat_dt} kernel={kernel} splits={splits} hint={seed % 2}")
    c = C.mla_case(2000 + seed, B, q_len, H, lens, max_T=max_T, q_dtype=q_dt, lat_dtype=lat_dt)
    q = C.to_dev(c["q"] if q_dt == C.F32 else c["qb"], q_dt, device)
    lat = C.to_dev(c["latb"], lat_dt, device)
    sl = torch.from_numpy(lens).to(device)
    # odd seeds pass the host length hint (the planner's exact unit count)
    hint = lens if seed % 2 else None
    out = mugen_amd.mla_attention(q, lat, sl, max_T, scale=C.MLA_SCALE, num_splits=splits, kernel=kernel,
                                  seq_lens_host=hint)
    torch.cuda.synchronize()
    C.assert_close(out.cpu().numpy(), C.mla_ref(c, nthreads=16), f"mla random seed={seed}")


GQA_HEADS = [(28, 4), (32, 8), (16, 16), (12, 3), (8, 1), (32, 2), (14, 2)]


@pytest.mark.parametrize("seed", range(16))
def test_gqa_decode_random(device, seed):
    r = np.random.default_rng(3000 + seed)
    H, Hk = GQA_HEADS[int(r.integers(len(GQA_HEADS)))]
    D = int(r.choice([64, 128]))
    B = int(r.integers(1, 7))
    max_T = int(r.integers(1, 3001))
    lens = r.integers(0, max_T + 1, size=B).astype(np.int32)
    dt = C.F16 if r.random() < 0.5 else C.BF16
    splits = int(r.choice([0, 0, 1, int(r.integers(2, 17))]))
    C.say(f"gqa decode random seed={seed}: B={B} H={H} Hk={Hk} D={D} max_T={max_T} lens={list(lens)} "
          f"dt={dt} splits={splits}")
    c = C.gqa_decode_case(4000 + seed, B, H, Hk, D, lens, max_T=max_T, dtype=dt)
    q = C.to_dev(c["qb"], dt, device)
    k = C.to_dev(c["kb"], dt, device)
    v = C.to_dev(c["vb"], dt, device)
    sl = torch.from_numpy(lens).to(device)
    out = mugen_amd.attention_decode(q, k, v, sl, max_T, out_dtype=torch.float32, num_splits=splits)
    torch.cuda.synchronize()
    C.assert_close(out.cpu().numpy(), C.gqa_decode_ref(c, nthreads=16), f"gqa decode random seed={seed}")


@pytest.mark.parametrize("seed", range(12))
def test_prefill_random(device, seed):
    r = np.random.default_rng(5000 + seed)
    H, Hk = GQA_HEADS[int(r.integers(len(GQA_HEADS)))]
    D = int(r.choice([64, 128]))
    N = int(r.integers(1, 1301))
    start = int(r.choice([0, int(r.integers(0, 400))]))
    dt = C.F16 if r.random() < 0.5 else C.BF16
    kernel = int(r.choice([0, _capi.PREFILL_KERNEL_BLOCK, _capi.PREFILL_KERNEL_WS]))
    C.say(f"prefill random seed={seed}: N={N} H={H} Hk={Hk} D={D} start={start} dt={dt} kernel={kernel}")
    c = C.prefill_case(6000 + seed, N, H, Hk, D, start, dt)
    q = C.to_dev(c["qb"], dt, device)
    k = C.to_dev(c["kb"], dt, device)
    v = C.to_dev(c["vb"], dt, device)
    out = mugen_amd.flash_prefill_attention(q, k, v, start, out_dtype=torch.float32, kernel=kernel)
    torch.cuda.synchronize()
    C.assert_close(out.cpu().numpy(), C.prefill_ref(c, nthreads=16), f"prefill random seed={seed}")


@pytest.mark.parametrize("seed", range(12))
def test_prefill_chunk_random(device, seed):
    # short chunks after long contexts (the key-split path when the
    # workspace is given: None allocates the size the library asks for),
    # head dims padded or not, causal or not
    r = np.random.default_rng(7000 + seed)
    H, Hk = GQA_HEADS[int(r.integers(len(GQA_HEADS)))]
    D = int(r.choice([64, 96, 128]))
    N = int(r.integers(1, 300))
    start = int(r.integers(500, 6000))
    dt = C.F16 if r.random() < 0.5 else C.BF16
    causal = r.random() < 0.8
    out_dt = [torch.float32, None][int(r.integers(2))]
    C.say(f"prefill chunk random seed={seed}: N={N} H={H} Hk={Hk} D={D} start={start} dt={dt} causal={causal} "
          f"out={out_dt}")
    c = C.prefill_case(8000 + seed, N, H, Hk, D, start, dt)
    q = C.to_dev(c["qb"], dt, device)
    k = C.to_dev(c["kb"], dt, device)
    v = C.to_dev(c["vb"], dt, device)
    out = mugen_amd.flash_prefill_attention(q, k, v, start, causal=causal, out_dtype=out_dt)
    torch.cuda.synchronize()
    if causal:
        ref = C.prefill_ref(c, nthreads=16)
    else:
        kv = c["kv_len"]
        ref = C.O.gqa_attention(c["q"], c["k"].reshape(1, kv, Hk, D).repeat(N, 0),
                                c["v"].reshape(1, kv, Hk, D).repeat(N, 0), [kv] * N, H, Hk, D, kv * Hk * D,
                                nthreads=16)
    C.assert_close(out.float().cpu().numpy(), ref, f"prefill chunk random seed={seed}")
