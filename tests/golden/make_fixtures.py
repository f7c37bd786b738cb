"""Generate the small committed fixtures under tests/golden/.

Inputs: mt19937_64 + Box-Muller (oracle generator), rounded to the storage
dtype.  Outputs: the CPU oracle in fp32 (the reference's arithmetic) and in
fp64 (the tolerance anchor).  The reference ships no attention fixtures of
its own, so these are the build's pinned vectors; each is cross-checked
against the independent fp64 numpy formulation before it is written.

Run:  python tests/golden/make_fixtures.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import oracle as O  # noqa: E402
from tests import cases as C  # noqa: E402


def save(name, **kw):
    path = os.path.join(HERE, name)
    np.savez_compressed(path, **kw)
    print(f"{name}: {os.path.getsize(path)} bytes")


def main():
    # GQA decode: Qwen-like head grouping, ragged lengths incl. 0 and 1
    lens = np.array([0, 1, 17, 90], np.int32)
    c = C.gqa_decode_case(1001, 4, 14, 2, 64, lens, dtype=C.F16)
    o32, o64 = C.gqa_decode_ref(c), C.gqa_decode_ref(c, f64=True)
    np64 = O.gqa_attention_np64(c["q"], c["k"], c["v"], lens, 14, 2, 64, c["seq_stride"])
    assert np.allclose(o64, np64, atol=1e-12)
    save("gqa_decode_small.npz", B=4, H=14, Hk=2, D=64, max_T=c["max_T"], dtype=C.F16, seq_lens=lens,
         qb=c["qb"], kb=c["kb"], vb=c["vb"], out_f32=o32, out_f64=o64)

    # causal prefill, Llama-1B head grouping, with a cache offset
    p = C.prefill_case(1002, 12, 16, 4, 64, start=9, dtype=C.BF16)
    o32, o64 = C.prefill_ref(p), C.prefill_ref(p, f64=True)
    assert np.allclose(o64, O.gqa_prefill_np64(p["q"], p["k"], p["v"], 12, 16, 4, 64, p["kv_len"], 9), atol=1e-12)
    save("prefill_small.npz", N=12, H=16, Hk=4, D=64, start=9, dtype=C.BF16, qb=p["qb"], kb=p["kb"], vb=p["vb"],
         out_f32=o32, out_f64=o64)

    # MLA verify: q_len 3, ragged, fp32 query over an fp16 latent cache
    m = C.mla_case(1003, 2, 3, 4, [40, 2], max_T=40, q_dtype=C.F32, lat_dtype=C.F16)
    o32, o64 = C.mla_ref(m), C.mla_ref(m, f64=True)
    assert np.allclose(o64, O.mla_attention_np64(m["q"], m["lat"], m["seq_lens"], 3, 4, C.MLA_SCALE), atol=1e-12)
    save("mla_verify_small.npz", B=2, q_len=3, H=4, max_T=40, q_dtype=C.F32, lat_dtype=C.F16,
         seq_lens=m["seq_lens"], q=m["q"], qb=np.zeros(1, np.uint16), latb=m["latb"], out_f32=o32, out_f64=o64)


if __name__ == "__main__":
    main()
