"""Prompt chunks over a long cache: the key-split form of the warp-specialised
prefill kernel (partials per key range, then gqa_prefill_combine) against the
CPU oracle's flash_prefill_attention restatement, and against the same call
without the workspace (one workgroup walks each block's whole key range).

The reference serves such a chunk through flash_prefill_attention with
start_pos > 0 (transformer.cpp chunked prompt; attention.cpp flash prefill):
token i sees keys [0, start_pos + i]."""
import ctypes

import pytest
import torch

import mugen_amd
from mugen_amd import _capi
from tests import cases as C

pytestmark = pytest.mark.gpu


def split_bytes(c, out_dtype, causal=True):
    """> 0 when the call splits keys."""
    a = _capi.GqaPrefillArgs()
    a.q = a.k = a.v = a.out = 0x1000
    a.n_tokens, a.n_heads, a.n_kv_heads, a.head_dim = c["N"], c["H"], c["Hk"], c["D"]
    a.kv_len, a.start_pos, a.causal = c["kv_len"], c["start"], int(causal)
    a.dtype, a.out_dtype = c["dtype"], out_dtype
    need = _capi.lib().mugen_attn_gqa_prefill_workspace_size(ctypes.byref(a))
    # the fp16 V copy of BF16 prompts of 1024+ tokens is there with or
    # without a split; below 1024 tokens anything at all means a split
    # (partials, and for 8-head blocks over long ranges the copy as well)
    long_v16 = c["kv_len"] * c["Hk"] * c["D"] * 2 + 256 if (c["dtype"] == C.BF16 and c["N"] >= 1024) else 0
    return need - long_v16


def run(c, device, out_dtype, causal=True, workspace=None, kernel=0):
    C.say(f"prefill split N={c['N']} H={c['H']} Hk={c['Hk']} D={c['D']} start={c['start']} "
          f"dtype={c['dtype']} out={out_dtype} causal={causal} ws={'auto' if workspace is None else workspace.numel()}")
    q = C.to_dev(c["qb"], c["dtype"], device)
    k = C.to_dev(c["kb"], c["dtype"], device)
    v = C.to_dev(c["vb"], c["dtype"], device)
    out = mugen_amd.flash_prefill_attention(q, k, v, c["start"], causal=causal, out_dtype=C.torch_dtype(out_dtype),
                                            workspace=workspace, kernel=kernel)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


@pytest.mark.parametrize("N,H,Hk,D,start,dtype", [
    (256, 8, 1, 128, 7900, C.F16),    # 8-head blocks, 64-key steps, 16 splits
    (100, 28, 4, 128, 4000, C.BF16),  # Qwen2.5-7B heads (G = 7), 32-key bf16 steps, ragged last block
    (64, 32, 8, 64, 3000, C.BF16),    # Llama-3.2-1B heads: 4-head blocks
    (48, 32, 2, 64, 2000, C.F16),     # G = 16: two 8-head slices per kv head
    (40, 16, 2, 96, 1500, C.F16),     # head_dim 96 in 128-wide tiles
    (300, 8, 1, 64, 1000, C.BF16),    # a split boundary inside some blocks' causal tail
    (1100, 8, 1, 64, 3000, C.BF16),   # with the fp16 V copy in front of the partials
    (256, 32, 4, 64, 6000, C.BF16),   # a short chunk whose 1600-key ranges take the fp16 V copy
])
@pytest.mark.parametrize("out_dtype", ["same", C.F32])
def test_split_chunk_vs_oracle(device, N, H, Hk, D, start, dtype, out_dtype):
    out_dtype = dtype if out_dtype == "same" else out_dtype
    c = C.prefill_case(300 + N + start, N, H, Hk, D, start, dtype)
    assert split_bytes(c, out_dtype) > 0, "the planner splits this chunk's keys"
    ref = C.prefill_ref(c, nthreads=16)
    C.assert_close(run(c, device, out_dtype), ref, f"split prefill N={N} start={start} out={out_dtype}")


def test_split_equals_unsplit(device):
    # the same chunk without a workspace runs unsplit: both within the
    # oracle's tolerance of each other
    c = C.prefill_case(311, 200, 28, 4, 128, 6000, C.F16)
    assert split_bytes(c, C.F32) > 0
    split = run(c, device, C.F32)
    unsplit = run(c, device, C.F32, workspace=torch.empty(0, dtype=torch.uint8, device=device))
    ref = C.prefill_ref(c, nthreads=16)
    C.assert_close(split, ref, "split")
    C.assert_close(unsplit, ref, "unsplit")
    C.assert_close(split, unsplit, "split vs unsplit")


def test_split_workspace_too_small(device):
    # a workspace that holds the V copy but not the partials: the call runs
    # unsplit over the copy and is still correct
    c = C.prefill_case(312, 1100, 8, 1, 64, 3000, C.BF16)
    v16 = c["kv_len"] * 1 * 64 * 2 + 256
    ws = torch.empty(v16, dtype=torch.uint8, device=device)
    C.assert_close(run(c, device, C.F32, workspace=ws), C.prefill_ref(c, nthreads=16), "v16 only")


def test_split_forced_block_kernel(device):
    # a forced kernel other than the warp-specialised one never splits
    c = C.prefill_case(313, 64, 8, 1, 128, 5000, C.BF16)
    C.assert_close(run(c, device, C.F32, kernel=_capi.PREFILL_KERNEL_BLOCK), C.prefill_ref(c, nthreads=16),
                   "forced block kernel")


def test_split_non_causal(device):
    # every row sees all kv_len keys: each split's range is whole for every row
    N, H, Hk, D, start = 33, 8, 1, 64, 4000
    c = C.prefill_case(314, N, H, Hk, D, start, C.F16)
    assert split_bytes(c, C.F32, causal=False) > 0
    kv = c["kv_len"]
    ref = C.O.gqa_attention(c["q"], c["k"].reshape(1, kv, Hk, D).repeat(N, 0), c["v"].reshape(1, kv, Hk, D).repeat(N, 0),
                            [kv] * N, H, Hk, D, kv * Hk * D)
    C.assert_close(run(c, device, C.F32, causal=False), ref, "non-causal split")


def test_split_large_scores(device):
    # scores far apart across splits: the merge re-bases each partial on the
    # largest reference max (one split's weights underflow against another's)
    N, H, Hk, D, start = 64, 8, 1, 128, 3000
    c = C.prefill_case(315, N, H, Hk, D, start, C.F16)
    kb = c["k"].copy()
    kb[100:140] *= 8.0  # a band of keys with large scores, in the first split only
    k, kbits = C.O.round_to(kb, C.F16)
    c["k"], c["kb"] = k, kbits
    assert split_bytes(c, C.F32) > 0
    C.assert_close(run(c, device, C.F32), C.prefill_ref(c, nthreads=16), "split with a dominant key band")


def test_split_graph_replays(device):
    # the split call (fp16 V copy, partials, merge) captured in a graph and
    # replayed with eager work between the replays: every replay equals the
    # eager result bit for bit
    c = C.prefill_case(316, 256, 28, 4, 128, 7936, C.BF16)
    assert split_bytes(c, C.BF16) > 0
    q = C.to_dev(c["qb"], C.BF16, device)
    k = C.to_dev(c["kb"], C.BF16, device)
    v = C.to_dev(c["vb"], C.BF16, device)
    ws = mugen_amd.prefill_workspace(q, k, v, c["start"])
    eager = mugen_amd.flash_prefill_attention(q, k, v, c["start"], workspace=ws)
    torch.cuda.synchronize()
    out = torch.empty_like(eager)
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            mugen_amd.flash_prefill_attention(q, k, v, c["start"], out=out, workspace=ws)
    torch.cuda.synchronize()
    for i in range(3):
        out.fill_(float("nan"))
        ws.fill_(0x7f)
        g.replay()
        torch.cuda.synchronize()
        C.say(f"split graph replay {i}")
        assert torch.equal(out, eager), f"replay {i} differs from the eager call"
