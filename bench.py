"""Benchmark of the MI355X attention subsystem (one GPU).

Headline workload (the metric's north-star case): MLA absorbed decode at
DeepSeek-V3 shape -- batch 8, 128 heads, q_len 1, bf16 absorbed queries
~N(0,1), bf16 latent cache of 576 dims per token ~N(0,0.5), context
lengths uniform in [1024, 8192], scale 1/sqrt(192), split-K with fp32
log-sum-exp combine, fp32 output.  One step = one layer's attention call
(main kernel + combine) with all inputs resident in HBM.

value = algorithmic HBM bytes of the step / step time (GB/s):
  sum_b T_b*576*2 (latent) + B*H*576*2 (q) + B*H*512*4 (out).
The other BASELINE configs are measured the same way and reported under
"configs" (us per layer-step plus GB/s or TFLOP/s).

  python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu] [--only NAME]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import mugen_amd  # noqa: E402
from mugen_amd import _capi  # noqa: E402

PEAK_HBM_GBS = 8000.0     # MI355X HBM3E
PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
METRIC = json.load(open(os.path.join(ROOT, "BASELINE.json")))["metric"]
MLA_SCALE = 1.0 / math.sqrt(192.0)
GRAPH_STEPS = 20  # steps per captured HIP graph in the timed region


def seeded_lens(seed, n, lo, hi):
    g = np.random.default_rng(seed)
    return g.integers(lo, hi + 1, n).astype(np.int32)


def randn(shape, std, dtype, gen, dev):
    return (torch.randn(shape, generator=gen, device=dev, dtype=torch.float32) * std).to(dtype)


class Case:
    name = ""
    kernel = ""          # dominant kernel's timing name
    profile = None       # (kernel, workload) of its summaries under profiles/
    bound = "hbm"
    unit = "GB/s"

    def step(self):
        raise NotImplementedError


class MlaDecode(Case):
    bound = "hbm"
    kernel = "mla_decode"

    def __init__(self, dev, B, H, q_len, lens, max_T, q_dtype, lat_dtype, seed, name, fallback_rows=0, layers=1):
        self.name = name
        g = torch.Generator(device=dev).manual_seed(seed)
        self.B, self.H, self.q_len = B, H, q_len
        self.lens = np.asarray(lens, np.int32)
        self.q = randn((B, q_len, H, 576), 1.0, q_dtype, g, dev)
        self.lat = randn((B, max_T, 576), 0.5, lat_dtype, g, dev)
        # layers > 1: consecutive steps read the latent caches of `layers`
        # different layers in turn, as a model's decode step does, so that
        # a cache is not still resident in the last-level cache (256 MB)
        # when its layer comes round again
        self.lats = [self.lat] + [randn((B, max_T, 576), 0.5, lat_dtype, g, dev) for _ in range(layers - 1)]
        self.layer = 0
        if fallback_rows:
            # the exact-fallback cost: every 64-token block of each sequence
            # carries a spike token (latent dim 0 = 1000, its other dims 0)
            # 40 tokens in, and `fallback_rows` of the H query rows score it
            # +72 nats above the rest (q dim 0 = 1; the other rows' q dim 0 is
            # 0, so the spike scores 0 for them).  A split whose first tile
            # does not hold its largest score overshoots the bf16 headroom
            # (2^64) for exactly those rows: fallback_rows / H of the
            # (row, split) pairs go through the fp32 recompute.
            self.q[..., 0] = 0.0
            self.q[:, :, :fallback_rows, 0] = 1.0
            spikes = torch.arange(40, max_T, 64, device=dev)
            self.lat[:, spikes, :] = 0.0
            self.lat[:, spikes, 0] = 1000.0
        self.sl = torch.from_numpy(self.lens).to(dev)
        self.max_T = max_T
        self.out = torch.empty((B, q_len, H, 512), dtype=torch.float32, device=dev)
        self.profile = ("mla_decode", {"mla_decode_v3": "v3_b8_h128", "mla_decode_v2lite": "v2lite_b1_h16",
                                       "mla_verify_v3": "verify_b4_q5_t32768",
                                       "mla_prefill_v2lite_n512": "prefill_v2lite_n512"}.get(name, name))
        self.ws = torch.empty(1 << 28, dtype=torch.uint8, device=dev)
        esz_q = self.q.element_size()
        self.bytes = float(self.lens.sum()) * 576 * self.lat.element_size() + B * q_len * H * (576 * esz_q + 512 * 4)
        vis = sum(int(T) - q_len + i + 1 for T in self.lens for i in range(q_len))
        self.flops = 2.0 * H * (576 + 512) * vis
        if q_len > 1:
            self.bound, self.unit = "mfma", "TFLOP/s"

    def step(self):
        lat = self.lats[self.layer]
        self.layer = (self.layer + 1) % len(self.lats)
        mugen_amd.mla_attention(self.q, lat, self.sl, self.max_T, scale=MLA_SCALE, out=self.out,
                                workspace=self.ws, seq_lens_host=self.lens)

    def cpu_sample(self, seconds_target=10.0):
        """Time the oracle (single-thread C port of cpu_mla_attention's core)
        on whole sequences of this workload until ~seconds_target of work;
        returns (bytes_per_s_equivalent, description)."""
        from oracle import oracle as O
        done_rows_tok = 0.0
        elapsed = 0.0
        nseq = 0
        for b in range(self.B):
            q = self.q[b:b + 1].float().cpu().numpy()
            T = int(self.lens[b])
            lat = self.lat[b:b + 1, :T].float().cpu().numpy()
            t0 = time.perf_counter()
            O.mla_attention(q, lat, [T], self.q_len, self.H, MLA_SCALE, seq_stride=T * 576, nthreads=1)
            elapsed += time.perf_counter() - t0
            done_rows_tok += self.H * sum(T - self.q_len + i + 1 for i in range(self.q_len))
            nseq += 1
            if elapsed > seconds_target:
                break
        total_rows_tok = self.H * sum(int(T) - self.q_len + i + 1 for T in self.lens for i in range(self.q_len))
        full_s = elapsed * total_rows_tok / done_rows_tok
        return full_s, f"{nseq} of {self.B} sequences (all {self.H} heads), scaled by row-tokens"

    def cpu_extras(self, threads):
        """Context for the single-thread baseline: (i) the same core with
        `threads` workers over (sequence, head), timed on the first two
        sequences and scaled by row-tokens; (ii) the per-head q_nope
        absorption of cpu_mla_attention (transformer.cpp:2563-2573) for all
        B*H rows against f16 W_UK, single thread."""
        from oracle import oracle as O
        elapsed, done = 0.0, 0.0
        for b in range(min(2, self.B)):
            q = self.q[b:b + 1].float().cpu().numpy()
            T = int(self.lens[b])
            lat = self.lat[b:b + 1, :T].float().cpu().numpy()
            t0 = time.perf_counter()
            O.mla_attention(q, lat, [T], self.q_len, self.H, MLA_SCALE, seq_stride=T * 576, nthreads=threads)
            elapsed += time.perf_counter() - t0
            done += self.H * sum(T - self.q_len + i + 1 for i in range(self.q_len))
        total = self.H * sum(int(T) - self.q_len + i + 1 for T in self.lens for i in range(self.q_len))
        mt_s = elapsed * total / done
        rng = np.random.default_rng(7)
        w = (rng.standard_normal((self.H * 128, 512)) * 0.05).astype(np.float16).view(np.uint8)
        qn = rng.standard_normal((self.B, self.q_len, self.H, 192)).astype(np.float16).astype(np.float32)
        t0 = time.perf_counter()
        O.mla_absorb(qn, w, O.W_F16, self.H)
        absorb_s = time.perf_counter() - t0
        return mt_s, absorb_s


class GqaDecode(Case):
    bound = "hbm"
    kernel = "gqa_decode"

    def __init__(self, dev, B, H, Hk, D, lens, max_T, seed, name):
        self.name = name
        g = torch.Generator(device=dev).manual_seed(seed)
        self.lens = np.asarray(lens, np.int32)
        self.q = randn((B, H, D), 1.0, torch.float16, g, dev)
        self.k = randn((B, max_T, Hk, D), 1.0, torch.float16, g, dev)
        self.v = randn((B, max_T, Hk, D), 1.0, torch.float16, g, dev)
        self.sl = torch.from_numpy(self.lens).to(dev)
        self.max_T = max_T
        self.out = torch.empty((B, H, D), dtype=torch.float16, device=dev)
        self.profile = ("gqa_decode", "qwen7b_b16_ragged" if B == 16 else "qwen7b_b1_t4096")
        self.ws = torch.empty(1 << 26, dtype=torch.uint8, device=dev)
        self.bytes = float(self.lens.sum()) * Hk * D * 2 * 2 + B * H * D * 2 * 2
        self.flops = 4.0 * H * D * float(self.lens.sum())

    def step(self):
        mugen_amd.attention_decode(self.q, self.k, self.v, self.sl, self.max_T, out=self.out, workspace=self.ws,
                                   seq_lens_host=self.lens)


class GqaDecodeQ4(Case):
    """GQA decode straight from the 4-bit group KV store (the reference's
    KVCache format, kv_cache.cpp): tokens older than the newest 256 as
    20-byte groups of 32 values, the newest 256 f16.  Bytes: the Q4 groups
    and f16 rows actually read, q and out."""
    bound = "hbm"
    kernel = "gqa_decode"

    def __init__(self, dev, B, H, Hk, D, lens, max_T, seed, name):
        self.name = name
        self.lens = np.asarray(lens, np.int32)
        self.cache = mugen_amd.KVCacheQ4(1, B, Hk, D, max_seq_len=max_T, fp16_preserve_last=256, max_new=64,
                                         device=dev)
        c = self.cache
        g = torch.Generator(device=dev).manual_seed(seed)
        # fill the store directly: random groups with valid f16 scale / min
        # for the quantised tokens, random f16 ring rows
        q4 = torch.randint(0, 256, c.q4_k[0].shape, generator=g, device=dev, dtype=torch.int32).to(torch.uint8)
        sm = (torch.rand(c.q4_k[0].shape[:2] + (c.vpt // 32, 2), generator=g, device=dev) * 0.1).to(torch.float16)
        q4 = q4.view(B, max_T, c.vpt // 32, 20)
        q4[..., 0:4] = sm.view(torch.uint8).view(B, max_T, c.vpt // 32, 4)
        c.q4_k[0].copy_(q4.view_as(c.q4_k[0]))
        c.q4_v[0].copy_(q4.view_as(c.q4_v[0]).flip(1))
        c.ring_k[0].copy_(randn(c.ring_k[0].shape, 1.0, torch.float16, g, dev))
        c.ring_v[0].copy_(randn(c.ring_v[0].shape, 1.0, torch.float16, g, dev))
        c.seq_lens_host = self.lens.copy()
        c.seq_lens.copy_(torch.from_numpy(self.lens))
        nq = np.maximum(self.lens - 256, 0).astype(np.int32)
        c.n_q4.copy_(torch.from_numpy(nq))
        self.q = randn((B, H, D), 1.0, torch.float16, g, dev)
        self.out = torch.empty((B, H, D), dtype=torch.float16, device=dev)
        self.ws = torch.empty(1 << 26, dtype=torch.uint8, device=dev)
        self.profile = ("gqa_decode_q4", "qwen7b_b16_ragged")
        nf = self.lens - nq
        self.bytes = 2.0 * (float(nq.sum()) * c.row_bytes + float(nf.sum()) * c.vpt * 2) + B * H * D * 2 * 2
        self.flops = 4.0 * H * D * float(self.lens.sum())

    def step(self):
        self.cache.attention_decode(0, self.q, out=self.out, workspace=self.ws)


class Prefill(Case):
    bound = "mfma"
    unit = "TFLOP/s"
    kernel = "gqa_prefill"
    # the fp16 copy of V (long bf16 prompts); the merge of split key ranges
    # (short chunks over a long context)
    extra_kernels = ("gqa_prefill_v16", "gqa_prefill_combine")

    def __init__(self, dev, N, H, Hk, D, seed, name, start=0):
        """N prompt tokens at start_pos `start` (a chunk after `start` cached
        tokens: the cache holds start + N rows, token i sees start + i + 1)."""
        self.name = name
        self.start = start
        kv = start + N
        g = torch.Generator(device=dev).manual_seed(seed)
        self.q = randn((N, H, D), 1.0, torch.bfloat16, g, dev)
        self.k = randn((kv, Hk, D), 1.0, torch.bfloat16, g, dev)
        self.v = randn((kv, Hk, D), 1.0, torch.bfloat16, g, dev)
        self.out = torch.empty((N, H, D), dtype=torch.bfloat16, device=dev)
        self.profile = ("gqa_prefill", "llama1b_n512" if N == 512 else
                        f"qwen7b_n{N}" + (f"_at{start}" if start else ""))
        self.flops = 4.0 * H * D * N * (start + (N + 1) / 2)
        self.bytes = (N * H * D * 2) * 2 + kv * Hk * D * 2 * 2
        self.ws = mugen_amd.prefill_workspace(self.q, self.k, self.v, start)

    def step(self):
        mugen_amd.flash_prefill_attention(self.q, self.k, self.v, self.start, out=self.out, workspace=self.ws)


class MlaFull(Case):
    """The attention part of one MLA decode layer (transformer.cpp:3882-3995,
    from the q / kv_a projections to the attention output): latent-cache
    write of the new token (c_kv RMSNorm, k_rope YaRN RoPE, append) and q
    RoPE fused into absorption by attn_k_b (one launch at decode sizes), the latent core with the fp32
    absorbed q over the f16 latent cache, up-projection by attn_v_b to f16,
    weights in a GGML block encoding.  Bytes: both weight matrices, the
    latent rows read and written, q in, q_abs and o out and back, out."""
    bound = "hbm"
    kernel = "mla_decode"
    extra_kernels = ("mla_prepare", "mla_latent_write", "mla_absorb", "mla_project")

    def __init__(self, dev, B, H, lens, max_T, w_type, seed, name, q_len=1, profile=("mla_layer", "v3_b8_q8_0")):
        self.name = name
        g = torch.Generator(device=dev).manual_seed(seed)
        self.lens = np.asarray(lens, np.int32)
        self.w_type = w_type
        self.q_len = q_len
        self.q = randn((B, q_len, H, 192), 1.0, torch.float16, g, dev)
        self.lat = randn((B, max_T, 576), 0.5, torch.float16, g, dev)
        self.sl = torch.from_numpy(self.lens).to(dev)
        self.max_T = max_T
        rb = {"f16": 1024, "q8_0": 544, "q4_0": 288}[w_type]
        # weights as a quantiser writes them: random bytes with valid f16 block scales
        wb = torch.randint(0, 256, (2, H * 128, rb), generator=g, device=dev, dtype=torch.int32).to(torch.uint8)
        if w_type == "f16":
            wf = randn((2, H * 128, 512), 0.05, torch.float16, g, dev)
            wb = wf.view(torch.uint8).reshape(2, H * 128, rb).contiguous()
        else:
            bb = 34 if w_type == "q8_0" else 18
            sc = (torch.rand((2, H * 128, 16), generator=g, device=dev) * 1e-3 + 5e-4).to(torch.float16)
            wb = wb.view(2, H * 128, 16, bb)
            wb[..., 0:2] = sc.view(torch.uint8).view(2, H * 128, 16, 2)
            wb = wb.reshape(2, H * 128, rb).contiguous()
        self.w_kb = wb[0] if w_type != "f16" else wb[0].view(torch.float16)
        self.w_vb = wb[1] if w_type != "f16" else wb[1].view(torch.float16)
        self.qa = torch.empty((B, q_len, H, 576), dtype=torch.float32, device=dev)
        self.o = torch.empty((B, q_len, H, 512), dtype=torch.float32, device=dev)
        self.out = torch.empty((B, q_len, H, 128), dtype=torch.float16, device=dev)
        self.ws = torch.empty(1 << 28, dtype=torch.uint8, device=dev)
        self.kv_a = randn((B * q_len, 576), 1.0, torch.float16, g, dev)
        self.norm_w = randn((512,), 0.1, torch.float16, g, dev) + 1.0
        # the step's new tokens sit at the end of each sequence
        pos = (self.lens[:, None] - q_len + np.arange(q_len)[None, :]).astype(np.int32).reshape(-1)
        self.pos = torch.from_numpy(pos).to(dev)
        self.rope = (10000.0, 40.0, 4096)
        self.profile = profile
        rows = B * q_len * H
        self.bytes = (2.0 * H * 128 * rb + float(self.lens.sum()) * 576 * 2 + rows * 192 * 2
                      + 2 * rows * 576 * 4 + 2 * rows * 512 * 4 + rows * 128 * 2 + 2 * B * q_len * 576 * 2)
        vis = sum(int(T) - q_len + i + 1 for T in self.lens for i in range(q_len))
        self.flops = 2.0 * rows * 128 * 512 * 2 + 2.0 * H * (576 + 512) * vis
        if q_len > 1:
            self.bound, self.unit = "mfma", "TFLOP/s"

    def step(self):
        # latent write + absorption: one launch at decode sizes
        mugen_amd.mla_prepare(self.kv_a, self.norm_w, self.pos, self.lat, self.q, self.w_kb, self.w_type,
                              q_abs=self.qa, rows_per_seq=self.q_len, rope=self.rope)
        mugen_amd.mla_attention(self.qa, self.lat, self.sl, self.max_T, scale=MLA_SCALE, out=self.o,
                                workspace=self.ws, seq_lens_host=self.lens)
        mugen_amd.mla_project(self.o, self.w_vb, self.w_type, out=self.out)


def capture(case, n):
    """HIP graph of n consecutive steps (captured on a side stream, as torch requires)."""
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(n):
            case.step()
    return g


WARMUP_MIN_S = 0.5  # untimed GPU work before timing: clocks settle


def time_case(case, steps, warmup, dev):
    """Warm-up, then EXACTLY `steps` steps timed with events between two
    synchronisations.  Warm-up is `warmup` untimed steps, continued (still
    untimed, as back-to-back replays of the captured graphs that keep the GPU
    busy) until at least WARMUP_MIN_S of wall time has passed: the first
    workload measured in a fresh process otherwise runs ~8% slower than the
    same kernels a second later (the GPU's clocks ramp up).  The steps run as
    replays of captured HIP graphs (up to GRAPH_STEPS steps each): the GPU
    executes the same kernels on the same resident inputs as an eager call,
    without the per-call Python/ctypes launch cost (~13 us), which would
    otherwise be what the small cases measure."""
    t_w = time.perf_counter()
    for _ in range(warmup):
        case.step()
    torch.cuda.synchronize(dev)
    per = min(GRAPH_STEPS, steps)
    full, rest = divmod(steps, per)
    graphs = [(capture(case, per), full)] + ([(capture(case, rest), 1)] if rest else [])
    for g, _ in graphs:  # one untimed replay each (graph upload)
        g.replay()
    torch.cuda.synchronize(dev)
    while time.perf_counter() - t_w < WARMUP_MIN_S:
        for _ in range(4):
            graphs[0][0].replay()
        torch.cuda.synchronize(dev)
    t0 = time.perf_counter()
    # an event between consecutive replays (recording one does not stall
    # the stream): the total over all `steps` and each replay's own duration
    ev = [torch.cuda.Event(enable_timing=True)]
    ev[0].record()
    per_rep = []
    for g, reps in graphs:
        for _ in range(reps):
            g.replay()
            ev.append(torch.cuda.Event(enable_timing=True))
            ev[-1].record()
            per_rep.append(per if len(per_rep) < full else rest)
    torch.cuda.synchronize(dev)
    wall_ms = (time.perf_counter() - t0) * 1e3
    ms = ev[0].elapsed_time(ev[-1]) / steps
    rep_ms = [ev[i].elapsed_time(ev[i + 1]) / per_rep[i] for i in range(len(per_rep))]
    median_ms = float(np.median(rep_ms))
    # per-kernel durations: the library launches each kernel with a start /
    # stop event pair stamped at the kernel's own start and end, on the
    # launch stream (hipExtLaunchKernelGGL)
    _capi.timing_reset()
    _capi.timing_enable(True)
    for _ in range(steps):
        case.step()
    torch.cuda.synchronize(dev)
    _capi.timing_enable(False)
    k_ms, k_n = _capi.timing_read(case.kernel)
    c_ms, c_n = _capi.timing_read(case.kernel + "_combine")
    extra = {}
    extra_ms = 0.0
    for name in getattr(case, "extra_kernels", ()):
        e_ms, e_n = _capi.timing_read(name)
        extra[name + "_us"] = round(e_ms / max(e_n, 1) * 1e3, 3)
        extra_ms += e_ms / steps
    # every kernel of a step, back to back: the roofline's denominator
    kernels_ms = (k_ms + c_ms) / steps + extra_ms
    return dict(ms_per_step=ms, median_ms=median_ms, wall_ms=wall_ms, kernel_ms=k_ms / max(k_n, 1),
                combine_ms=(c_ms / c_n) if c_n else 0.0, kernels_ms=kernels_ms, extra=extra)


def rate(case, ms):
    if case.unit == "TFLOP/s":
        return case.flops / (ms * 1e-3) / 1e12
    return case.bytes / (ms * 1e-3) / 1e9


def load_traffic(kernel, workload):
    path = os.path.join(ROOT, "profiles", f"{kernel}__{workload}.traffic.json")
    if os.path.exists(path):
        try:
            return json.load(open(path)).get("hbm_bytes_per_launch")
        except (OSError, ValueError):
            return None
    return None


def measured_peaks(dev):
    """Practical ceilings next to the datasheet peaks, measured in this run:
    a library bf16 GEMM (8192^3, hipBLASLt through torch.matmul) and a 1 GiB
    device-to-device copy (read + write bytes), event-timed after warm-up."""
    def timed(fn, reps):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / 1e3 / reps
    n = 8192
    a = torch.randn((n, n), dtype=torch.bfloat16, device=dev)
    b = torch.randn((n, n), dtype=torch.bfloat16, device=dev)
    c = torch.empty((n, n), dtype=torch.bfloat16, device=dev)
    gemm_s = timed(lambda: torch.matmul(a, b, out=c), 20)
    del a, b, c
    x = torch.empty(1 << 29, dtype=torch.float16, device=dev)
    y = torch.empty_like(x)
    copy_s = timed(lambda: y.copy_(x), 20)
    del x, y
    return {"gemm_bf16_tflops": round(2.0 * n ** 3 / gemm_s / 1e12, 1), "gemm_shape": [n, n, n],
            "copy_gbs": round(2.0 * (1 << 30) / copy_s / 1e9, 1), "copy_bytes": 1 << 30}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", default=None, help="run only the named workload")
    ap.add_argument("--headline-only", action="store_true")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="first run 5 plain device copies of MIB MiB (reference kernel for HBM counter scaling)")
    ap.add_argument("--calibrate-scatter", type=int, default=0, metavar="MIB",
                    help="first run the library's scatter_kv over MIB MiB 5 times: a kernel of this library whose "
                         "HBM bytes are known exactly (MIB read + MIB written), for HBM counter scaling")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU; multi-GPU runs are not part of it "
                          "(sharding the path over GPUs is a design note, not a measured mode)", "n_gpus": args.gpus}))
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    if args.calibrate_scatter > 0:
        n = args.calibrate_scatter << 19  # 16-bit elements
        src = torch.ones(n, dtype=torch.float16, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            mugen_amd.scatter_kv(src, dst, 0)
        torch.cuda.synchronize(dev)
        del src, dst
    if args.calibrate_copy > 0:
        n = args.calibrate_copy << 20
        src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize(dev)
        del src, dst

    head = MlaDecode(dev, 8, 128, 1, seeded_lens(45, 8, 1024, 8192), 8192, torch.bfloat16, torch.bfloat16, 45,
                     "mla_decode_v3")
    cases = [head]
    if not args.headline_only:
        cases += [
            MlaDecode(dev, 1, 16, 1, [1024], 1024, torch.float32, torch.float16, 42, "mla_decode_v2lite"),
            GqaDecode(dev, 1, 28, 4, 128, [4096], 4096, 43, "gqa_decode_qwen7b_b1"),
            GqaDecode(dev, 16, 28, 4, 128, seeded_lens(44, 16, 256, 4096), 4096, 44, "gqa_decode_qwen7b_b16"),
            GqaDecodeQ4(dev, 16, 28, 4, 128, seeded_lens(44, 16, 256, 4096), 4096, 44, "gqa_decode_q4_qwen7b_b16"),
            Prefill(dev, 512, 32, 8, 64, 46, "gqa_prefill_llama1b"),
            Prefill(dev, 2048, 28, 4, 128, 50, "gqa_prefill_qwen7b_n2048"),
            Prefill(dev, 8192, 28, 4, 128, 49, "gqa_prefill_qwen7b_n8192"),
            # a 256-token prompt chunk after 7936 cached tokens (the key
            # ranges split across workgroups, then merged)
            Prefill(dev, 256, 28, 4, 128, 53, "gqa_prefill_qwen7b_chunk256_at7936", start=7936),
            # a speculative-verify step of the 7B model: a 4-token draft plus
            # one through the prompt path after 8000 held tokens
            # (forward_prefill_all_logits, transformer.cpp:3499-3514, runs the
            # verify tokens through forward_prefill_layers at start_position)
            Prefill(dev, 5, 28, 4, 128, 54, "gqa_prefill_qwen7b_verify5_at8000", start=8000),
            MlaDecode(dev, 4, 128, 5, [32768] * 4, 32768, torch.bfloat16, torch.bfloat16, 47, "mla_verify_v3"),
            # a 512-token prompt of V2-Lite in one verify-shaped call (the
            # reference runs cpu_mla_attention once per prompt token)
            MlaDecode(dev, 1, 16, 512, [512], 512, torch.float32, torch.float16, 51, "mla_prefill_v2lite_n512"),
            MlaFull(dev, 8, 128, seeded_lens(45, 8, 1024, 8192), 8192, "q8_0", 48, "mla_layer_v3_q8_0"),
            # the same layer over a 512-token V2-Lite prompt in one step
            MlaFull(dev, 1, 16, [512], 512, "q8_0", 52, "mla_layer_prefill_v2lite_n512", q_len=512,
                    profile=("mla_layer", "prefill_v2lite_n512_q8_0")),
            MlaDecode(dev, 8, 128, 1, seeded_lens(45, 8, 1024, 8192), 8192, torch.bfloat16, torch.bfloat16, 45,
                      "mla_decode_v3_fallback_1pct", fallback_rows=1),
            MlaDecode(dev, 8, 128, 1, seeded_lens(45, 8, 1024, 8192), 8192, torch.bfloat16, torch.bfloat16, 45,
                      "mla_decode_v3_fallback_10pct", fallback_rows=13),
            # the headline step over 5 layers' caches in turn (277 MB read per
            # 5 steps, more than the 256 MB last-level cache holds)
            MlaDecode(dev, 8, 128, 1, seeded_lens(45, 8, 1024, 8192), 8192, torch.bfloat16, torch.bfloat16, 45,
                      "mla_decode_v3_5layers", layers=5),
        ]
    if args.only:
        cases = [c for c in cases if c.name == args.only]
    results = {}
    for c in cases:
        print(f"# timing {c.name}", file=sys.stderr, flush=True)
        t = time_case(c, args.steps, args.warmup, dev)
        peak = PEAK_HBM_GBS if c.unit == "GB/s" else PEAK_BF16_TFLOPS
        # the kernels' own start/stop stamps pad launches of a few us (each
        # stamped launch carries its event bookkeeping): a step's kernels
        # cannot take longer than the step, so the roofline denominator is
        # the smaller of the two
        kern_ms = min(t["kernels_ms"], t["ms_per_step"])
        results[c.name] = dict(
            us_per_step=round(t["ms_per_step"] * 1e3, 3),
            median_us_per_step=round(t["median_ms"] * 1e3, 3),
            kernel_us=round(t["kernel_ms"] * 1e3, 3),
            combine_us=round(t["combine_ms"] * 1e3, 3),
            kernels_us=round(t["kernels_ms"] * 1e3, 3),
            rate=round(rate(c, t["ms_per_step"]), 2), unit=c.unit,
            # roofline: the step's algorithmic bytes (flops) over the summed
            # durations of all its kernels (main + combine + any others)
            roofline_rate=round(rate(c, kern_ms), 2),
            frac_of_peak=round(rate(c, kern_ms) / peak, 4),
            kernel_frac=round(rate(c, min(t["kernel_ms"], kern_ms)) / peak, 4),
            algorithmic_bytes=c.bytes, algorithmic_flops=c.flops,
            traffic=load_traffic(*c.profile) if c.profile else None, **t["extra"])

    h = results.get(head.name) if head in cases else None
    line = {"metric": METRIC, "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic (seeded torch.randn: q ~N(0,1), latent ~N(0,0.5); ctx lens seeded U[1024,8192])",
            "config": {"workload": "mla_absorbed_decode_deepseek_v3", "batch": 8, "n_heads": 128, "q_len": 1,
                       "latent_dim": 576, "kv_rank": 512, "ctx_lens": [int(x) for x in head.lens],
                       "max_ctx": 8192, "split_k": "auto", "out_dtype": "f32",
                       "timing": f"HIP-graph replays of {GRAPH_STEPS}-step captures, events on the launch stream; "
                                 "ms_per_step = total / steps, median_us_per_step = median over replays"}}
    if h:
        line["value"] = h["rate"]
        line["ms_per_step"] = round(h["us_per_step"] / 1e3, 6)
        line["us_per_layer_step"] = h["us_per_step"]
        kb = head.bytes
        # achieved: algorithmic bytes / (main kernel + split-K combine), the
        # kernels' own stamped durations capped by the step time;
        # kernel_frac: main kernel alone
        ach = kb / (min(h["kernels_us"], h["us_per_step"]) * 1e-6) / 1e9
        line["roofline"] = {"bound": "hbm", "kernel": "mla_decode + mla_decode_combine", "achieved": round(ach, 1),
                            "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(ach / PEAK_HBM_GBS, 4),
                            "traffic": h["traffic"], "kernel_us": h["kernel_us"], "combine_us": h["combine_us"],
                            "kernel_frac": h["kernel_frac"],
                            "definition": "algorithmic bytes per step / (main kernel + combine) duration, "
                                          "capped by the replayed step time"}
        if not args.no_cpu:
            full_s, sample = head.cpu_sample()
            line["cpu_baseline"] = {"value": round(head.bytes / full_s / 1e9, 4), "unit": "GB/s", "cores": 1,
                                    "kind": "port", "us_per_layer_step": round(full_s * 1e6, 1),
                                    "sample": sample, "host_cores_available": os.cpu_count()}
            threads = min(16, os.cpu_count() or 1)  # the GPU box's CPU share
            mt_s, absorb_s = head.cpu_extras(threads)
            line["cpu_baseline"]["threaded"] = {"value": round(head.bytes / mt_s / 1e9, 4), "unit": "GB/s",
                                                "cores": threads, "us_per_layer_step": round(mt_s * 1e6, 1),
                                                "sample": "sequences 0-1, scaled by row-tokens"}
            line["cpu_baseline"]["absorb_us_per_layer_step"] = round(absorb_s * 1e6, 1)
    line["measured_peaks"] = mp = measured_peaks(dev)
    if h:
        # the same achieved rate against this run's own device-copy rate:
        # the practical ceiling of a streaming read on this box
        line["roofline"]["frac_measured"] = round(line["roofline"]["achieved"] / mp["copy_gbs"], 4)
        line["median_us_per_step"] = h["median_us_per_step"]
    for name, r in results.items():
        ceil = mp["copy_gbs"] if r["unit"] == "GB/s" else mp["gemm_bf16_tflops"]
        r["frac_of_measured"] = round(r["roofline_rate"] / ceil, 4)
    line["configs"] = results
    print(json.dumps(line))


if __name__ == "__main__":
    main()
