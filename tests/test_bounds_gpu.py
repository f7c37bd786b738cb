"""Every entry point writes only inside its buffers, also when a device
length is bad: outputs, workspaces and caches sit between canary-filled
guard bands, and a device sequence length above max_seq_len must give the
oracle's result at the clamped length (the ABI clamps device lengths to
[0, max_seq_len]) without touching a guard byte."""
import ctypes

import numpy as np
import pytest
import torch

import mugen_amd
from mugen_amd import _capi
from mugen_amd import attention as A
from oracle import oracle as O
from tests import cases as C

pytestmark = pytest.mark.gpu

GUARD = 4096   # bytes of canary on each side (keeps 256-byte alignment)
CANARY = 0xA5


class Guarded:
    """A device tensor of `shape`/`dtype` inside a canary-filled buffer."""

    def __init__(self, shape, dtype, device, fill=None):
        n = int(np.prod(shape)) * torch.empty((), dtype=dtype).element_size()
        self.n = n
        self.buf = torch.full((GUARD + n + GUARD,), CANARY, dtype=torch.uint8, device=device)
        self.t = self.buf[GUARD:GUARD + n].view(dtype).view(shape)
        if fill is not None:
            self.t.copy_(fill)

    def intact(self):
        torch.cuda.synchronize()
        head = self.buf[:GUARD].cpu().numpy()
        tail = self.buf[GUARD + self.n:].cpu().numpy()
        return bool(np.all(head == CANARY) and np.all(tail == CANARY))


def guarded_ws(need, device):
    return Guarded((max(int(need), 1),), torch.uint8, device)


@pytest.mark.parametrize("lens", [[700, 1000, 33], [700, 5000, 33], [-7, 1024, 2**30]])
def test_gqa_decode_guarded(device, lens):
    max_T = 1024
    c = C.gqa_decode_case(501, 3, 28, 4, 128, np.clip(lens, 0, max_T), max_T=max_T, dtype=C.F16)
    C.say(f"guarded gqa_decode lens={lens} max_T={max_T}")
    q = C.to_dev(c["qb"], C.F16, device)
    k = C.to_dev(c["kb"], C.F16, device)
    v = C.to_dev(c["vb"], C.F16, device)
    sl = torch.tensor(lens, dtype=torch.int32, device=device)
    for splits in (0, 3):
        out = Guarded((3, 28, 128), torch.float32, device)
        a = A.gqa_decode_args(q, k, v, sl, out.t, max_T, 0.0, splits)
        ws = guarded_ws(_capi.lib().mugen_attn_gqa_decode_workspace_size(ctypes.byref(a)), device)
        mugen_amd.attention_decode(q, k, v, sl, max_T, out=out.t, num_splits=splits, workspace=ws.t)
        assert out.intact() and ws.intact(), f"guard band overwritten (splits={splits})"
        C.assert_close(out.t.cpu().numpy(), C.gqa_decode_ref(c), f"clamped lens {lens} splits={splits}")


@pytest.mark.parametrize("q_len,lens", [(1, [300, 9999]), (1, [512, 0]), (3, [3, 2**31 - 1]), (5, [100, 513])])
def test_mla_decode_guarded(device, q_len, lens):
    max_T = 512
    clamped = np.clip(lens, 0, max_T)
    c = C.mla_case(502 + q_len, 2, q_len, 16, clamped, max_T=max_T, q_dtype=C.F32, lat_dtype=C.F16)
    C.say(f"guarded mla_decode q_len={q_len} lens={lens} max_T={max_T}")
    q = C.to_dev(c["q"], C.F32, device)
    lat = C.to_dev(c["latb"], C.F16, device)
    sl = torch.tensor(lens, dtype=torch.int32, device=device)
    for kernel in (_capi.MLA_KERNEL_ROWS, _capi.MLA_KERNEL_WS):
        out = Guarded((2, q_len, 16, 512), torch.float32, device)
        a = A.mla_args(q, lat, sl, out.t, max_T, C.MLA_SCALE, 0, kernel)
        ws = guarded_ws(_capi.lib().mugen_attn_mla_decode_workspace_size(ctypes.byref(a)), device)
        mugen_amd.mla_attention(q, lat, sl, max_T, scale=C.MLA_SCALE, out=out.t, workspace=ws.t, kernel=kernel)
        assert out.intact() and ws.intact(), f"guard band overwritten (kernel {kernel})"
        C.assert_close(out.t.cpu().numpy(), C.mla_ref(c), f"clamped lens {lens} kernel {kernel}")


def test_decode_short_host_copy_guarded(device):
    # host lengths below the device ones: the plan (grid, workspace, the
    # partials' stride) follows the host copy, and the splits it has no
    # room for are skipped -- the result is not defined, but nothing is
    # written outside the output or the workspace sized for that plan
    T = 4096
    dev_lens, host_lens = [4000, 3000], np.array([200, 100], np.int32)
    c = C.gqa_decode_case(530, 2, 28, 4, 128, dev_lens, max_T=T, dtype=C.F16)
    C.say(f"guarded gqa_decode, host lengths {list(host_lens)} below device {dev_lens}")
    q = C.to_dev(c["qb"], C.F16, device)
    k = C.to_dev(c["kb"], C.F16, device)
    v = C.to_dev(c["vb"], C.F16, device)
    sl = torch.tensor(dev_lens, dtype=torch.int32, device=device)
    out = Guarded((2, 28, 128), torch.float32, device)
    a = A.gqa_decode_args(q, k, v, sl, out.t, T, 0.0, 0)
    a.seq_lens_host = host_lens.ctypes.data
    ws = guarded_ws(_capi.lib().mugen_attn_gqa_decode_workspace_size(ctypes.byref(a)), device)
    mugen_amd.attention_decode(q, k, v, sl, T, out=out.t, workspace=ws.t, seq_lens_host=host_lens)
    assert out.intact() and ws.intact(), "guard band overwritten (gqa decode, short host copy)"
    m = C.mla_case(531, 2, 1, 16, dev_lens, max_T=T, q_dtype=C.F32, lat_dtype=C.F16)
    C.say(f"guarded mla_decode, host lengths {list(host_lens)} below device {dev_lens}")
    mq = C.to_dev(m["q"], C.F32, device)
    lat = C.to_dev(m["latb"], C.F16, device)
    mout = Guarded((2, 1, 16, 512), torch.float32, device)
    ma = A.mla_args(mq, lat, sl, mout.t, T, C.MLA_SCALE, 0, 0)
    ma.seq_lens_host = host_lens.ctypes.data
    mws = guarded_ws(_capi.lib().mugen_attn_mla_decode_workspace_size(ctypes.byref(ma)), device)
    mugen_amd.mla_attention(mq, lat, sl, T, scale=C.MLA_SCALE, out=mout.t, workspace=mws.t, seq_lens_host=host_lens)
    assert mout.intact() and mws.intact(), "guard band overwritten (mla decode, short host copy)"


def test_gqa_prefill_guarded(device):
    c = C.prefill_case(503, 77, 28, 4, 128, 30, C.BF16)
    C.say("guarded gqa_prefill N=77 start=30")
    q = C.to_dev(c["qb"], C.BF16, device)
    k = C.to_dev(c["kb"], C.BF16, device)
    v = C.to_dev(c["vb"], C.BF16, device)
    ref = C.prefill_ref(c)
    for kernel in (_capi.PREFILL_KERNEL_BLOCK, _capi.PREFILL_KERNEL_WS):
        out = Guarded((77, 28, 128), torch.bfloat16, device)
        mugen_amd.flash_prefill_attention(q, k, v, 30, out=out.t, kernel=kernel)
        assert out.intact(), f"guard band overwritten (kernel {kernel})"
        C.assert_close(out.t.float().cpu().numpy(), ref, f"guarded prefill kernel {kernel}")


@pytest.mark.parametrize("N,start", [(77, 30), (300, 212)])
def test_gqa_prefill_short_guarded(device, N, start):
    # the short-prompt kernel (head_dim 64, G = 4) with a last query block of
    # fewer than 16 tokens and a kv range ending at 512 keys
    c = C.prefill_case(505 + N, N, 32, 8, 64, start, C.BF16)
    C.say(f"guarded gqa_prefill short N={N} start={start}")
    q = C.to_dev(c["qb"], C.BF16, device)
    k = C.to_dev(c["kb"], C.BF16, device)
    v = C.to_dev(c["vb"], C.BF16, device)
    ref = C.prefill_ref(c)
    out = Guarded((N, 32, 64), torch.bfloat16, device)
    mugen_amd.flash_prefill_attention(q, k, v, start, out=out.t, kernel=_capi.PREFILL_KERNEL_SHORT)
    assert out.intact(), "guard band overwritten (short kernel)"
    C.assert_close(out.t.float().cpu().numpy(), ref, f"guarded short prefill N={N}")


@pytest.mark.parametrize("N,H,Hk,D,start,dt", [(77, 28, 4, 128, 6000, C.BF16), (5, 32, 8, 96, 3000, C.F16),
                                               (200, 32, 2, 64, 2500, C.BF16)])
def test_gqa_prefill_split_guarded(device, N, H, Hk, D, start, dt):
    # the key-split path: the fp16 V copy, the partials and the merge write
    # only inside the workspace and the output (a ragged last query block,
    # padded head_dim, two 8-head slices)
    c = C.prefill_case(520 + N, N, H, Hk, D, start, dt)
    C.say(f"guarded gqa_prefill split N={N} H={H} Hk={Hk} D={D} start={start} dt={dt}")
    q = C.to_dev(c["qb"], dt, device)
    k = C.to_dev(c["kb"], dt, device)
    v = C.to_dev(c["vb"], dt, device)
    out = Guarded((N, H, D), torch.float32, device)
    need = mugen_amd.prefill_workspace(q, k, v, start, out_dtype=torch.float32).numel()
    assert need > 0
    ws = guarded_ws(need, device)
    mugen_amd.flash_prefill_attention(q, k, v, start, out=out.t, workspace=ws.t)
    assert out.intact() and ws.intact(), "guard band overwritten (split prefill)"
    C.assert_close(out.t.cpu().numpy(), C.prefill_ref(c, nthreads=16), f"guarded split prefill N={N}")


def test_kv_append_guarded(device):
    # rows at positions >= max_seq_len are dropped, negative lengths too
    B, max_T, row = 3, 64, 512
    C.say("guarded kv_append")
    kc = Guarded((B, max_T, 4, 128), torch.float16, device, fill=torch.zeros(B, max_T, 4, 128))
    vc = Guarded((B, max_T, 4, 128), torch.float16, device, fill=torch.zeros(B, max_T, 4, 128))
    kn = torch.randn((B, 5, row), device=device).half()
    vn = torch.randn((B, 5, row), device=device).half()
    sl = torch.tensor([10, 62, 1000], dtype=torch.int32, device=device)
    mugen_amd.kv_append(kn, vn, kc.t, vc.t, sl)
    assert kc.intact() and vc.intact()
    kg = kc.t.view(B, max_T, row).cpu()
    assert torch.equal(kg[0, 10:15], kn[0].cpu())
    assert torch.equal(kg[1, 62:64], kn[1, :2].cpu())   # the rest past the cache: dropped
    assert torch.count_nonzero(kg[2]) == 0              # the whole append past the cache


def test_kv_q4_append_guarded(device):
    # a store whose device length is past max_seq_len: nothing outside it is
    # written, and the quantised count never exceeds max_seq_len
    C.say("guarded kv_q4_append")
    st = mugen_amd.KVCacheQ4(1, 2, 4, 128, max_seq_len=64, fp16_preserve_last=8, max_new=16, device=device)
    qk = Guarded(st.q4_k[0].shape, torch.uint8, device, fill=st.q4_k[0])
    rk = Guarded(st.ring_k[0].shape, torch.float16, device, fill=st.ring_k[0])
    st.q4_k[0], st.ring_k[0] = qk.t, rk.t
    st.seq_lens.copy_(torch.tensor([60, 5000], dtype=torch.int32))
    st.n_q4.copy_(torch.tensor([52, 5000], dtype=torch.int32))
    a = _capi.KvQ4AppendArgs()
    a.store = st.store(0)
    kn = torch.randn((2, 16, 512), device=device).half()
    a.k_new, a.v_new = kn.data_ptr(), kn.data_ptr()
    a.seq_lens, a.n_q4, a.n_q4_out = st.seq_lens.data_ptr(), st.n_q4.data_ptr(), st._n_q4_next.data_ptr()
    a.n_seq, a.n_new, a.n_kv_heads, a.head_dim, a.max_seq_len = 2, 16, 4, 128, 64
    _capi.check(_capi.lib().mugen_attn_kv_q4_append(ctypes.byref(a), A._stream(device)))
    assert qk.intact() and rk.intact()
    nq = st._n_q4_next.cpu().numpy()
    assert nq[0] == 64 and nq[1] == 64, nq  # 60 + 16 - 8 = 68 tokens leave the window; 64 fit


def test_latent_write_guarded(device):
    # positions outside [0, max_seq_len) are skipped
    C.say("guarded mla_latent_write")
    lat = Guarded((2, 32, 576), torch.float16, device, fill=torch.zeros(2, 32, 576))
    kv_a = torch.randn((4, 576), device=device).half()
    norm_w = torch.ones(512, device=device).half()
    pos = torch.tensor([0, 31, 32, -1], dtype=torch.int32, device=device)
    mugen_amd.mla_latent_write(kv_a, norm_w, pos, lat.t, rows_per_seq=2)
    assert lat.intact()
    got = lat.t.cpu()
    assert torch.count_nonzero(got[0, 0]) > 0 and torch.count_nonzero(got[0, 31]) > 0
    assert torch.count_nonzero(got[1]) == 0  # both rows of sequence 1 were out of range
