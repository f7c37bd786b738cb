// capi.hip -- extern "C" entry points of libmugen_attn (see include/mugen_attn.h).
//
// Validation, split-K planning, workspace carving and optional event timing
// live here; the kernels are in gqa_decode.hip, gqa_prefill.hip and
// mla_decode.hip.  Nothing here allocates device memory or synchronises
// the host (except mugen_attn_timing_read, which waits on its own events).
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <climits>
#include <cmath>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "common.h"
#include "kernels.h"

namespace mugen_attn {

// ------------------------------------------------------------------ errors

static thread_local std::string g_last_error;

static int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

static int hip_status(hipError_t e, const char* what) {
    if (e == hipSuccess) return MUGEN_ATTN_OK;
    return fail(MUGEN_ATTN_E_HIP, "%s: %s", what, hipGetErrorString(e));
}

// ------------------------------------------------------------------ timing

struct KernelTimer {
    std::mutex mu;
    bool enabled = false;
    struct Pending { std::string name; hipEvent_t a, b; };
    std::vector<Pending> pending;
    std::vector<hipEvent_t> pool;
    std::unordered_map<std::string, std::pair<double, int64_t>> totals;

    hipEvent_t get() {
        if (!pool.empty()) { hipEvent_t e = pool.back(); pool.pop_back(); return e; }
        hipEvent_t e = nullptr;
        if (hipEventCreate(&e) != hipSuccess) return nullptr;
        return e;
    }
    void drain() {  // caller holds mu
        for (auto& p : pending) {
            float ms = 0.f;
            if (hipEventSynchronize(p.b) == hipSuccess && hipEventElapsedTime(&ms, p.a, p.b) == hipSuccess) {
                auto& t = totals[p.name];
                t.first += ms;
                t.second += 1;
            }
            pool.push_back(p.a);
            pool.push_back(p.b);
        }
        pending.clear();
    }
};

static KernelTimer g_timer;

KernelTimer* active_timer() { return g_timer.enabled ? &g_timer : nullptr; }

bool timer_pair(KernelTimer* t, hipEvent_t* start, hipEvent_t* stop) {
    if (!t) return false;
    std::lock_guard<std::mutex> lk(t->mu);
    *start = t->get();
    *stop = t->get();
    if (*start && *stop) return true;
    if (*start) t->pool.push_back(*start);
    if (*stop) t->pool.push_back(*stop);
    return false;
}

void timer_push(KernelTimer* t, const char* name, hipEvent_t start, hipEvent_t stop) {
    std::lock_guard<std::mutex> lk(t->mu);
    t->pending.push_back({name, start, stop});
    if (t->pending.size() > 4096) t->drain();
}

// ------------------------------------------------------------------ scatter_kv

__global__ void scatter_kv_kernel(const uint16_t* __restrict__ src, uint16_t* __restrict__ dst,
                                  uint64_t offset, uint64_t count) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) dst[offset + i] = src[i];
}

// 16-byte vector copy when both ends are 16-byte aligned
__global__ void scatter_kv16_kernel(const u32x4_t* __restrict__ src, u32x4_t* __restrict__ dst,
                                    uint64_t n16) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n16) dst[i] = src[i];
}

hipError_t launch_scatter_kv(const uint16_t* src, uint16_t* dst, uint64_t offset, uint64_t count,
                             hipStream_t st, KernelTimer* t) {
    if (count == 0) return hipSuccess;
    uint16_t* d = dst + offset;
    if ((((uintptr_t)src | (uintptr_t)d) & 15) == 0 && (count & 7) == 0) {
        const uint64_t n16 = count / 8;
        return launch_k(t, "scatter_kv", scatter_kv16_kernel, dim3((unsigned)((n16 + 255) / 256)), dim3(256), st,
                        reinterpret_cast<const u32x4_t*>(src), reinterpret_cast<u32x4_t*>(d), n16);
    }
    return launch_k(t, "scatter_kv", scatter_kv_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256), st,
                    static_cast<const uint16_t*>(src), dst, offset, count);
}

// ------------------------------------------------------------------ planning

static inline int ceil_div(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }

static bool is16(int dt) { return dt == DT_F16 || dt == DT_BF16; }
static bool is_out(int dt) { return dt == DT_F32 || dt == DT_F16 || dt == DT_BF16; }

// Tokens per split for a workgroup count target; rounded to `quantum`, and
// large enough that no more than kMaxSplits splits cover max_seq_len.
static int plan_chunk(int64_t tokens_x_groups, int target_wgs, int quantum, int max_seq_len,
                      int max_splits = kMaxSplits) {
    int64_t c = (tokens_x_groups + target_wgs - 1) / target_wgs;
    c = ((c + quantum - 1) / quantum) * quantum;
    if (c < quantum) c = quantum;
    const int64_t min_c = ((int64_t)(max_seq_len > 0 ? max_seq_len : 1) + max_splits - 1) / max_splits;
    if (c < min_c) c = ((min_c + quantum - 1) / quantum) * quantum;
    return (int)c;
}

static int explicit_chunk(int max_seq_len, int num_splits, int quantum, int max_splits = kMaxSplits) {
    const int maxT = max_seq_len > 0 ? max_seq_len : 1;
    int64_t c = ((int64_t)maxT + num_splits - 1) / num_splits;
    c = ((c + quantum - 1) / quantum) * quantum;
    const int64_t min_c = ((int64_t)maxT + max_splits - 1) / max_splits;
    if (c < min_c) c = ((min_c + quantum - 1) / quantum) * quantum;
    return (int)c;
}

// GQA decode work items for a chunk: sum over sequences of max(1,
// ceil(T_b / chunk)) splits times the kv heads -- exact from the host length
// hint, else the batch * max_seq_len upper bound.
// extra: splits per sequence beyond ceil(T / chunk) (the 4-bit store splits
// its f16 ring tokens separately: at most one more)
static int64_t gqa_items(const mugen_attn_gqa_decode_args* a, int chunk, int extra = 0) {
    const int maxT = a->max_seq_len > 0 ? a->max_seq_len : 1;
    int64_t n = 0;
    if (!a->seq_lens_host) {
        n = (int64_t)a->batch * (ceil_div(maxT, chunk) + extra);
    } else {
        for (int b = 0; b < a->batch; b++) {
            const int T = std::min(a->seq_lens_host[b], maxT);  // the kernels clamp to max_seq_len too
            n += T > 0 ? ceil_div(T, chunk) + extra : 1;
        }
    }
    return n * a->n_kv_heads;
}

// automatic split plans: the longest sequence in at most kPlanSplitCap
// splits; GQA decode chunks of at least kGqaChunkMin tokens
constexpr int kPlanSplitCap = 32, kGqaChunkMin = 64;

// GQA decode: a workgroup's 4 waves take 32-token blocks round-robin, so
// chunks are multiples of 32 tokens, at least 64.  The kernel holds two
// 256-thread workgroups per CU; the plan is the smallest chunk whose work
// list fits ONE dispatch round of 512 workgroups (every CU streaming, no
// second round) and splits the longest sequence at most 32 ways.  The
// 32-token step keeps the round fuller than 128-token steps would (the CUs
// holding two workgroups set the time): Qwen2.5-7B B16 ragged decode 19.0
// -> 18.2 us.  The 32-way cap (with the floor lowered from 128 to 64
// tokens): B1 T2048 7.38 -> 6.87 us, T8192 10.83 -> 9.17, B2 T8192 12.98
// -> 10.0; B16 and B1 T4096 unchanged (their plans were ~32 splits).
static int gqa_chunk(const mugen_attn_gqa_decode_args* a, int extra = 0) {
    constexpr int q = 32, qmin = kGqaChunkMin, kSplitCap = kPlanSplitCap;
    const int maxT = a->max_seq_len > 0 ? a->max_seq_len : 1;
    if (a->num_splits > 0) return explicit_chunk(maxT, a->num_splits, q, kMaxSplits - 1);
    const int cmax = ceil_div(maxT, q) * q;
    // the longest sequence (host lengths when given) in at most kSplitCap
    // splits: more, shorter splits cost the merge more than they shorten
    // the tile chains
    int tlong = maxT;
    if (a->seq_lens_host) {
        tlong = 1;
        for (int b = 0; b < a->batch; b++) tlong = std::max(tlong, std::min(a->seq_lens_host[b], maxT));
    }
    const int cmin = std::max(ceil_div(ceil_div(maxT, kMaxSplits - 1), q), ceil_div(ceil_div(tlong, kSplitCap), q)) * q;
    // one dispatch round: two workgroups per CU, one at head_dim 256 (one
    // wave per SIMD)
    const int64_t budget = a->head_dim > 128 ? 256 : 512;
    if (gqa_items(a, cmax, extra) > budget) return cmax;  // one split per sequence already fills a round
    int lo = cmin < qmin ? qmin : cmin, hi = cmax;        // items(c) is non-increasing in c
    while (lo < hi) {
        const int mid = ((lo + hi) / 2) / q * q;
        if (mid <= lo) break;
        if (gqa_items(a, mid, extra) <= budget) hi = mid;
        else lo = mid + q;
    }
    if (gqa_items(a, lo, extra) > budget) lo = hi;
    return lo;
}

static int gqa_validate(const mugen_attn_gqa_decode_args* a, bool ring_store = false) {
    if (!a) return fail(MUGEN_ATTN_E_INVALID, "gqa_decode: null args");
    if (!a->q || !a->k_cache || !a->v_cache || !a->seq_lens || !a->out)
        return fail(MUGEN_ATTN_E_INVALID, "gqa_decode: null tensor pointer");
    if (a->batch <= 0 || a->n_heads <= 0 || a->n_kv_heads <= 0 || a->max_seq_len <= 0 || a->num_splits < 0)
        return fail(MUGEN_ATTN_E_INVALID, "gqa_decode: batch/heads/max_seq_len must be > 0, num_splits >= 0");
    if (a->n_heads % a->n_kv_heads)
        return fail(MUGEN_ATTN_E_INVALID, "gqa_decode: n_heads %d not a multiple of n_kv_heads %d", a->n_heads,
                    a->n_kv_heads);
    if (a->n_heads / a->n_kv_heads > 16)
        return fail(MUGEN_ATTN_E_UNSUPPORTED, "gqa_decode: n_heads/n_kv_heads = %d > 16",
                    a->n_heads / a->n_kv_heads);
    if (ring_store ? (a->head_dim != 64 && a->head_dim != 128 && a->head_dim != 256)
                   : (a->head_dim < 8 || a->head_dim > 256 || a->head_dim % 8))
        return fail(MUGEN_ATTN_E_UNSUPPORTED, "%s: head_dim %d (supported: %s)", ring_store ? "gqa_decode_q4" : "gqa_decode",
                    a->head_dim, ring_store ? "64, 128, 256" : "multiples of 8 up to 256");
    if (!is16(a->kv_dtype)) return fail(MUGEN_ATTN_E_UNSUPPORTED, "gqa_decode: kv_dtype must be F16 or BF16");
    if (!is_out(a->out_dtype)) return fail(MUGEN_ATTN_E_UNSUPPORTED, "gqa_decode: bad out_dtype");
    if (!ring_store && a->batch > 1 && a->seq_stride < (int64_t)a->max_seq_len * a->n_kv_heads * a->head_dim)
        return fail(MUGEN_ATTN_E_INVALID, "gqa_decode: seq_stride %lld smaller than max_seq_len*Hk*D",
                    (long long)a->seq_stride);
    if (((uintptr_t)a->q | (uintptr_t)a->k_cache | (uintptr_t)a->v_cache) & 15)
        return fail(MUGEN_ATTN_E_INVALID, "gqa_decode: q/k/v must be 16-byte aligned");
    if (a->batch > 1 && (a->seq_stride % 8))
        return fail(MUGEN_ATTN_E_INVALID, "gqa_decode: seq_stride must be a multiple of 8 elements");
    return MUGEN_ATTN_OK;
}

// The decode and prefill kernels are built for head_dim 64 and 128 (decode
// also 256); a smaller head_dim (a multiple of 8) runs on the next one up,
// its extra dims masked (q zero, outputs not stored).
static int padded_head_dim(int head_dim) { return head_dim <= 64 ? 64 : head_dim <= 128 ? 128 : 256; }

// workspace: fp32 partials [B][H][splits][D] and (m, l) [B][H][splits][2]
// (D = the padded head_dim)
// The split-K partials' stride (splits per (sequence, head) slot): the
// plan's largest split count.  With host lengths that is the longest
// sequence's (the automatic plans split it at most 32 ways, plus the 4-bit
// store's separate ring split: `extra`), so a short batch in a long cache
// needs no more than its plan; the kernels skip any split index past the
// stride, so a device length above its host copy never writes past it.
// Without host lengths every length up to max_seq_len may come.
static int plan_stride(int max_seq_len, int chunk, const int32_t* host, int batch, int extra) {
    const int maxT = max_seq_len > 0 ? max_seq_len : 1;
    if (!host) return ceil_div(maxT, chunk) + extra;
    int s = 1;
    for (int b = 0; b < batch; b++) {
        const int T = std::min(std::max(host[b], 0), maxT);
        if (T > 0) s = std::max(s, ceil_div(T, chunk) + extra);
    }
    return s;
}

// A workspace sized without host lengths (a caller sizing once, then
// passing host lengths per call) must cover every plan those lengths can
// give: the automatic plans keep the longest sequence within kPlanSplitCap
// splits of at least `qmin` tokens
static int stride_bound(int max_seq_len, int qmin, int extra) {
    const int maxT = max_seq_len > 0 ? max_seq_len : 1;
    return std::min(kPlanSplitCap, ceil_div(maxT, qmin)) + extra;
}

static size_t gqa_ws(const mugen_attn_gqa_decode_args* a, int chunk, int* splits_out, int min_splits = 0) {
    const int splits = std::max(plan_stride(a->max_seq_len, chunk, a->seq_lens_host, a->batch, 0), min_splits);
    if (splits_out) *splits_out = splits;
    if (splits <= 1) return 0;
    const size_t slots = (size_t)a->batch * a->n_heads * splits;
    return slots * (size_t)padded_head_dim(a->head_dim) * 4 + slots * 2 * 4 + 256;
}

// MLA kernel (mla_decode.hip): 16-bit q with at most 64 query rows -> the
// "rows" kernel (4 waves of 16 rows, one per SIMD); everything else -> the
// warp-specialised kernel (two waves per SIMD), which measures faster for
// fp32 q and for the wide decode / verify shapes.  args->kernel forces one.
static int mla_kernel(const mugen_attn_mla_decode_args* a) {
    if (a->kernel == MUGEN_ATTN_MLA_KERNEL_ROWS || a->kernel == MUGEN_ATTN_MLA_KERNEL_WS) return a->kernel;
    const int R = a->q_len * a->n_heads;
    return (R <= 64 && a->q_dtype != DT_F32) ? MUGEN_ATTN_MLA_KERNEL_ROWS : MUGEN_ATTN_MLA_KERNEL_WS;
}

// Work units of the MLA kernels for a chunk (mla_map in mla_decode.hip):
// the (sequence, split, 64-row block) triples that see at least one key --
// every block of every split for decode steps, of a causal multi-token
// step's split s the blocks whose last row sees past s * chunk.  Exact from
// the host length hint, else an upper bound from max_seq_len (the count
// grows with the length).
static int64_t mla_units(const mugen_attn_mla_decode_args* a, int chunk, int64_t nrb) {
    int64_t u = 0;
    for (int b = 0; b < a->batch; b++) {
        // the kernels clamp device lengths to [0, max_seq_len] too
        const int T = a->seq_lens_host ? std::min(std::max(a->seq_lens_host[b], 0), a->max_seq_len)
                                       : std::max(a->max_seq_len, 1);
        const int ns = T > 0 ? ceil_div(T, chunk) : 0;
        if (a->q_len == 1) {
            u += ns * nrb;
            continue;
        }
        for (int s = 0; s < ns; s++) {
            const int64_t x = (int64_t)s * chunk - T + a->q_len;
            u += nrb - (x <= 0 ? 0 : std::min<int64_t>(a->n_heads * x / 64, nrb - 1));
        }
    }
    return u;
}

// The MLA kernel runs one 256-thread workgroup per CU (~480 registers per
// lane, 108 KiB LDS), and each workgroup pays a fixed cost (Q fragments,
// ring fill, partial store) on top of ~1.8 us per 32-token tile.  The plan:
// the smallest chunk (multiple of 32) whose nrb * active groups fit ONE
// dispatch round of 256 CUs -- maximum parallelism, no second round -- with
// the longest sequence split at most 32 ways.
static int mla_chunk(const mugen_attn_mla_decode_args* a, int kernel) {
    const int q = mla_tile_tokens(kernel);  // chunks are whole tiles
    if (a->num_splits > 0) return explicit_chunk(a->max_seq_len, a->num_splits, q, kMaxMlaSplits);
    const int R = a->q_len * a->n_heads;
    const int64_t nrb = ceil_div(R, mla_rows_per_block(kernel));
    const int maxT = a->max_seq_len > 0 ? a->max_seq_len : 1;
    const int cmax = ceil_div(maxT, q) * q;
    // the longest sequence (host lengths when given) in at most kSplitCap
    // splits: small batches otherwise fill the round with one-tile splits
    // whose merge costs more than the tiles (DeepSeek-V2-Lite heads, B1
    // T8192: 256 splits 36.5 us, 32 splits 16.9; one V3 sequence at T8192
    // 26.0 -> 17.3 us)
    constexpr int kSplitCap = kPlanSplitCap;
    int tlong = maxT;
    if (a->seq_lens_host) {
        tlong = 1;
        for (int b = 0; b < a->batch; b++) tlong = std::max(tlong, std::min(a->seq_lens_host[b], maxT));
    }
    const int cmin = std::max(ceil_div(ceil_div(maxT, kMaxMlaSplits), q), ceil_div(ceil_div(tlong, kSplitCap), q)) * q;
    const int64_t wg_budget = 256;
    if (mla_units(a, cmax, nrb) > wg_budget) return cmax;  // one split per sequence already fills a round
    int lo = cmin < q ? q : cmin, hi = cmax;               // units(c) is non-increasing in c
    while (lo < hi) {
        const int mid = ((lo + hi) / 2) / q * q;
        if (mid <= lo) break;
        if (mla_units(a, mid, nrb) <= wg_budget) hi = mid;
        else lo = mid + q;
    }
    if (mla_units(a, lo, nrb) > wg_budget) lo = hi;
    return lo;
}

static int mla_validate(const mugen_attn_mla_decode_args* a) {
    if (!a) return fail(MUGEN_ATTN_E_INVALID, "mla_decode: null args");
    if (!a->q || !a->latent || !a->seq_lens || !a->out)
        return fail(MUGEN_ATTN_E_INVALID, "mla_decode: null tensor pointer");
    if (a->batch <= 0 || a->q_len <= 0 || a->n_heads <= 0 || a->max_seq_len <= 0 || a->num_splits < 0)
        return fail(MUGEN_ATTN_E_INVALID, "mla_decode: batch/q_len/n_heads/max_seq_len must be > 0");
    if (a->kv_rank != 512 || a->rope_dim != 64)
        return fail(MUGEN_ATTN_E_UNSUPPORTED, "mla_decode: kv_rank %d / rope_dim %d (supported: 512 / 64)",
                    a->kv_rank, a->rope_dim);
    if (!(a->scale > 0.f) || !isfinite(a->scale))
        return fail(MUGEN_ATTN_E_INVALID, "mla_decode: scale must be finite and > 0");
    if (!is16(a->latent_dtype)) return fail(MUGEN_ATTN_E_UNSUPPORTED, "mla_decode: latent dtype must be F16/BF16");
    if (a->q_dtype != DT_F32 && a->q_dtype != a->latent_dtype)
        return fail(MUGEN_ATTN_E_UNSUPPORTED, "mla_decode: q dtype must be F32 or the latent dtype");
    if (!is_out(a->out_dtype)) return fail(MUGEN_ATTN_E_UNSUPPORTED, "mla_decode: bad out_dtype");
    if (a->batch > 1 && a->seq_stride < (int64_t)a->max_seq_len * 576)
        return fail(MUGEN_ATTN_E_INVALID, "mla_decode: seq_stride smaller than max_seq_len*576");
    if (((uintptr_t)a->q | (uintptr_t)a->latent) & 15)
        return fail(MUGEN_ATTN_E_INVALID, "mla_decode: q/latent must be 16-byte aligned");
    if (a->batch > 1 && (a->seq_stride % 8))
        return fail(MUGEN_ATTN_E_INVALID, "mla_decode: seq_stride must be a multiple of 8 elements");
    if ((int64_t)a->q_len * a->n_heads > (1 << 20))
        return fail(MUGEN_ATTN_E_UNSUPPORTED, "mla_decode: q_len*n_heads too large");
    if (a->kernel < 0 || a->kernel > MUGEN_ATTN_MLA_KERNEL_WS)
        return fail(MUGEN_ATTN_E_INVALID, "mla_decode: kernel %d (0 auto, 1 rows, 2 warp-specialised)", a->kernel);
    return MUGEN_ATTN_OK;
}

static size_t mla_ws(const mugen_attn_mla_decode_args* a, int chunk, int* splits_out, int min_splits = 0) {
    const int splits = std::max(plan_stride(a->max_seq_len, chunk, a->seq_lens_host, a->batch, 0), min_splits);
    if (splits_out) *splits_out = splits;
    // every split (a single one included) writes an fp32 (m, l, o) partial
    const size_t R = (size_t)a->q_len * a->n_heads;
    const size_t rows16 = (R + 15) / 16 * 16;  // O partials are stored per 16-row block
    const size_t sb = (size_t)a->batch * splits;
    return sb * rows16 * 512 * 2 + sb * R * 2 * 4 + 256;
}

static float* align256(void* p) {
    return reinterpret_cast<float*>((reinterpret_cast<uintptr_t>(p) + 255) & ~uintptr_t(255));
}

}  // namespace mugen_attn

using namespace mugen_attn;

extern "C" {

const char* mugen_attn_last_error(void) { return g_last_error.c_str(); }

const char* mugen_attn_version(void) { return "mugen_attn 0.3.0 (gfx950, abi 3)"; }

// ------------------------------------------------------------------ 4-bit store

static int q4_store_validate(const mugen_attn_kv_q4_store& st, int n_seq, int vpt, int max_seq_len, const char* who) {
    if (!st.q4_k || !st.q4_v || !st.ring_k || !st.ring_v) return fail(MUGEN_ATTN_E_INVALID, "%s: null store pointer", who);
    if (st.ring <= 0 || (st.ring & (st.ring - 1)) || st.fp16_preserve_last < 0)
        return fail(MUGEN_ATTN_E_INVALID, "%s: ring must be a power of two, fp16_preserve_last >= 0", who);
    if (vpt % 32) return fail(MUGEN_ATTN_E_UNSUPPORTED, "%s: n_kv_heads*head_dim must be a multiple of 32", who);
    const int64_t q4_row = (int64_t)vpt / 32 * 20;
    if (n_seq > 1 && (st.q4_seq_stride < q4_row * max_seq_len || st.ring_seq_stride < (int64_t)st.ring * vpt))
        return fail(MUGEN_ATTN_E_INVALID, "%s: sequence strides smaller than one store", who);
    if ((((uintptr_t)st.q4_k | (uintptr_t)st.q4_v) & 3) || (st.q4_seq_stride & 3))
        return fail(MUGEN_ATTN_E_INVALID, "%s: Q4 stores must be 4-byte aligned", who);
    if ((((uintptr_t)st.ring_k | (uintptr_t)st.ring_v) & 15) || (st.ring_seq_stride % 8))
        return fail(MUGEN_ATTN_E_INVALID, "%s: rings must be 16-byte aligned, strides multiples of 8", who);
    return MUGEN_ATTN_OK;
}

int mugen_attn_kv_q4_append(const mugen_attn_kv_q4_append_args* a, void* stream) {
    if (!a) return fail(MUGEN_ATTN_E_INVALID, "kv_q4_append: null args");
    if (a->n_seq < 0 || a->n_new < 0 || a->n_kv_heads <= 0 || a->head_dim <= 0 || a->max_seq_len <= 0)
        return fail(MUGEN_ATTN_E_INVALID, "kv_q4_append: bad sizes");
    if (a->n_seq == 0 || a->n_new == 0) return MUGEN_ATTN_OK;
    const int vpt = a->n_kv_heads * a->head_dim;
    if (int rc = q4_store_validate(a->store, a->n_seq, vpt, a->max_seq_len, "kv_q4_append")) return rc;
    if (!a->k_new || !a->v_new || !a->seq_lens || !a->n_q4 || !a->n_q4_out)
        return fail(MUGEN_ATTN_E_INVALID, "kv_q4_append: null pointer");
    if (a->n_q4_out == a->n_q4) return fail(MUGEN_ATTN_E_INVALID, "kv_q4_append: n_q4_out aliases n_q4");
    if (a->store.ring < a->store.fp16_preserve_last + a->n_new)
        return fail(MUGEN_ATTN_E_INVALID, "kv_q4_append: ring %d < fp16_preserve_last + n_new", a->store.ring);
    if (((uintptr_t)a->k_new | (uintptr_t)a->v_new) & 15)
        return fail(MUGEN_ATTN_E_INVALID, "kv_q4_append: k_new/v_new must be 16-byte aligned");
    if ((int64_t)a->n_new * 2 > INT32_MAX || a->n_seq > 65535)
        return fail(MUGEN_ATTN_E_UNSUPPORTED, "kv_q4_append: too many tokens / sequences");
    KvQ4AppendParams p{};
    p.k_new = static_cast<const uint16_t*>(a->k_new);
    p.v_new = static_cast<const uint16_t*>(a->v_new);
    p.q4k = static_cast<uint8_t*>(a->store.q4_k);
    p.q4v = static_cast<uint8_t*>(a->store.q4_v);
    p.ring_k = static_cast<uint16_t*>(a->store.ring_k);
    p.ring_v = static_cast<uint16_t*>(a->store.ring_v);
    p.seq_lens = a->seq_lens;
    p.n_q4 = a->n_q4;
    p.n_q4_out = a->n_q4_out;
    p.q4_seq_stride = a->store.q4_seq_stride;
    p.ring_seq_stride = a->store.ring_seq_stride;
    p.n_new = a->n_new;
    p.vpt = vpt;
    p.ring = a->store.ring;
    p.preserve = a->store.fp16_preserve_last;
    p.max_seq_len = a->max_seq_len;
    return hip_status(launch_kv_q4_append(p, a->n_seq, static_cast<hipStream_t>(stream), active_timer()),
                      "kv_q4_append launch");
}

// the f16 view of a 4-bit store decode for the shared planner / validation
static mugen_attn_gqa_decode_args q4_as_gqa(const mugen_attn_gqa_decode_q4_args* a) {
    mugen_attn_gqa_decode_args g{};
    g.q = a->q;
    g.k_cache = a->store.ring_k;
    g.v_cache = a->store.ring_v;
    g.seq_lens = a->seq_lens;
    g.out = a->out;
    g.batch = a->batch;
    g.n_heads = a->n_heads;
    g.n_kv_heads = a->n_kv_heads;
    g.head_dim = a->head_dim;
    g.max_seq_len = a->max_seq_len;
    g.num_splits = a->num_splits;
    g.seq_stride = a->store.ring_seq_stride;
    g.scale = a->scale;
    g.kv_dtype = DT_F16;
    g.out_dtype = a->out_dtype;
    g.seq_lens_host = a->seq_lens_host;
    return g;
}

static int gqa_q4_validate(const mugen_attn_gqa_decode_q4_args* a) {
    if (!a) return fail(MUGEN_ATTN_E_INVALID, "gqa_decode_q4: null args");
    const mugen_attn_gqa_decode_args g = q4_as_gqa(a);
    if (int rc = gqa_validate(&g, true)) return rc;
    if (!a->n_q4) return fail(MUGEN_ATTN_E_INVALID, "gqa_decode_q4: null n_q4");
    return q4_store_validate(a->store, a->batch, a->n_kv_heads * a->head_dim, a->max_seq_len, "gqa_decode_q4");
}

// 4-bit store decode: the Q4 and f16-ring tokens of a sequence are split
// separately (at most one split more than the f16 plan), and the partials
// always go through the workspace and the combine
static size_t gqa_q4_ws(const mugen_attn_gqa_decode_q4_args* a, int chunk, int* splits_out, int min_splits = 0) {
    const int splits = std::max(plan_stride(a->max_seq_len, chunk, a->seq_lens_host, a->batch, 1), min_splits);
    if (splits_out) *splits_out = splits;
    const size_t slots = (size_t)a->batch * a->n_heads * splits;
    return slots * (size_t)padded_head_dim(a->head_dim) * 4 + slots * 2 * 4 + 256;
}

size_t mugen_attn_gqa_decode_q4_workspace_size(const mugen_attn_gqa_decode_q4_args* a) {
    if (gqa_q4_validate(a) != MUGEN_ATTN_OK) return 0;
    const mugen_attn_gqa_decode_args g = q4_as_gqa(a);
    const int bound = (!a->seq_lens_host && a->num_splits <= 0) ? stride_bound(a->max_seq_len, kGqaChunkMin, 1) : 0;
    return gqa_q4_ws(a, gqa_chunk(&g, 1), nullptr, bound);
}

int mugen_attn_gqa_decode_q4(const mugen_attn_gqa_decode_q4_args* a, void* ws, size_t ws_bytes, void* stream) {
    if (int rc = gqa_q4_validate(a)) return rc;
    const mugen_attn_gqa_decode_args g = q4_as_gqa(a);
    const int chunk = gqa_chunk(&g, 1);
    int splits = 2;
    const size_t need = gqa_q4_ws(a, chunk, &splits);
    if (!ws || ws_bytes < need)
        return fail(MUGEN_ATTN_E_WORKSPACE, "gqa_decode_q4: workspace of %zu bytes required, %zu given", need,
                    ws_bytes);
    GqaDecodeParams p{};
    p.B = a->batch;
    p.Hk = a->n_kv_heads;
    p.q = static_cast<const uint16_t*>(a->q);
    p.k = static_cast<const uint16_t*>(a->store.ring_k);
    p.v = static_cast<const uint16_t*>(a->store.ring_v);
    p.seq_lens = a->seq_lens;
    p.out = a->out;
    p.H = a->n_heads;
    p.G = a->n_heads / a->n_kv_heads;
    p.hd = a->head_dim;
    p.row_stride = a->n_kv_heads * a->head_dim;
    p.chunk = chunk;
    p.num_splits = splits;
    p.seq_stride = a->store.ring_seq_stride;
    const float scale = a->scale > 0.f ? a->scale : 1.f / sqrtf((float)a->head_dim);
    p.scale_log2 = scale * kLog2e;
    p.q4k = static_cast<const uint8_t*>(a->store.q4_k);
    p.q4v = static_cast<const uint8_t*>(a->store.q4_v);
    p.n_q4 = a->n_q4;
    p.q4_seq_stride = a->store.q4_seq_stride;
    p.q4_row_bytes = a->n_kv_heads * a->head_dim / 32 * 20;
    p.ring = a->store.ring;
    p.max_T = a->max_seq_len;
    {
        float* base = align256(ws);
        const size_t slots = (size_t)a->batch * a->n_heads * splits;
        p.ws_o = base;
        p.ws_ml = base + slots * padded_head_dim(a->head_dim);
    }
    const int64_t nwg = gqa_items(&g, chunk, 1);  // + the ring splits
    if (nwg > INT32_MAX / 2) return fail(MUGEN_ATTN_E_UNSUPPORTED, "gqa_decode_q4: too many work items");
    p.per_xcd = (int)ceil_div(nwg, (int64_t)8);
    return hip_status(launch_gqa_decode_q4(p, (int)nwg, a->head_dim, a->out_dtype, static_cast<hipStream_t>(stream),
                                           active_timer()),
                      "gqa_decode_q4 launch");
}

size_t mugen_attn_gqa_decode_workspace_size(const mugen_attn_gqa_decode_args* a) {
    if (gqa_validate(a) != MUGEN_ATTN_OK) return 0;
    const int bound = (!a->seq_lens_host && a->num_splits <= 0) ? stride_bound(a->max_seq_len, kGqaChunkMin, 0) : 0;
    return gqa_ws(a, gqa_chunk(a), nullptr, bound);
}

int mugen_attn_gqa_decode(const mugen_attn_gqa_decode_args* a, void* ws, size_t ws_bytes, void* stream) {
    int rc = gqa_validate(a);
    if (rc) return rc;
    const int chunk = gqa_chunk(a);
    int splits = 1;
    const size_t need = gqa_ws(a, chunk, &splits);
    if (need > 0 && (!ws || ws_bytes < need))
        return fail(MUGEN_ATTN_E_WORKSPACE, "gqa_decode: workspace of %zu bytes required, %zu given", need,
                    ws_bytes);
    GqaDecodeParams p{};
    p.B = a->batch;
    p.Hk = a->n_kv_heads;
    p.q = static_cast<const uint16_t*>(a->q);
    p.k = static_cast<const uint16_t*>(a->k_cache);
    p.v = static_cast<const uint16_t*>(a->v_cache);
    p.seq_lens = a->seq_lens;
    p.out = a->out;
    p.H = a->n_heads;
    p.G = a->n_heads / a->n_kv_heads;
    p.hd = a->head_dim;
    p.row_stride = a->n_kv_heads * a->head_dim;
    p.chunk = chunk;
    p.num_splits = splits;
    p.seq_stride = a->seq_stride;
    const float scale = a->scale > 0.f ? a->scale : 1.f / sqrtf((float)a->head_dim);
    p.scale_log2 = scale * kLog2e;
    p.max_T = a->max_seq_len;
    if (splits > 1) {
        float* base = align256(ws);
        const size_t slots = (size_t)a->batch * a->n_heads * splits;
        p.ws_o = base;
        p.ws_ml = base + slots * padded_head_dim(a->head_dim);
    }
    const int64_t nwg = gqa_items(a, chunk);
    if (nwg > INT32_MAX) return fail(MUGEN_ATTN_E_UNSUPPORTED, "gqa_decode: too many work items");
    hipError_t e = launch_gqa_decode(p, (int)nwg, padded_head_dim(a->head_dim), a->kv_dtype, a->out_dtype,
                                     static_cast<hipStream_t>(stream), active_timer());
    return hip_status(e, "gqa_decode launch");
}

static int gqa_prefill_validate(const mugen_attn_gqa_prefill_args* a) {
    if (!a) return fail(MUGEN_ATTN_E_INVALID, "gqa_prefill: null args");
    if (!a->q || !a->k || !a->v || !a->out) return fail(MUGEN_ATTN_E_INVALID, "gqa_prefill: null tensor pointer");
    if (a->n_tokens < 0 || a->n_heads <= 0 || a->n_kv_heads <= 0 || a->kv_len < 0 || a->start_pos < 0)
        return fail(MUGEN_ATTN_E_INVALID, "gqa_prefill: negative size");
    if (a->n_heads % a->n_kv_heads) return fail(MUGEN_ATTN_E_INVALID, "gqa_prefill: n_heads % n_kv_heads != 0");
    if (a->n_heads / a->n_kv_heads > 16)
        return fail(MUGEN_ATTN_E_UNSUPPORTED, "gqa_prefill: n_heads/n_kv_heads > 16");
    if (a->n_heads / a->n_kv_heads > 8 && a->kernel == MUGEN_ATTN_PREFILL_KERNEL_BLOCK)
        return fail(MUGEN_ATTN_E_UNSUPPORTED, "gqa_prefill: the per-block kernel serves at most 8 heads per kv head");
    if (a->head_dim < 8 || a->head_dim > 256 || a->head_dim % 8)
        return fail(MUGEN_ATTN_E_UNSUPPORTED, "gqa_prefill: head_dim %d (supported: multiples of 8 up to 256)",
                    a->head_dim);
    if (!is16(a->dtype) || !is_out(a->out_dtype)) return fail(MUGEN_ATTN_E_UNSUPPORTED, "gqa_prefill: dtype");
    if (a->kernel < 0 || a->kernel > MUGEN_ATTN_PREFILL_KERNEL_SHORT)
        return fail(MUGEN_ATTN_E_INVALID, "gqa_prefill: kernel %d (0 auto, 1 per-block, 2 warp-specialised, 3 short)",
                    a->kernel);
    if (((uintptr_t)a->q | (uintptr_t)a->k | (uintptr_t)a->v | (uintptr_t)a->out) & 15)
        return fail(MUGEN_ATTN_E_INVALID, "gqa_prefill: q/k/v/out must be 16-byte aligned");
    if (a->n_tokens == 0) return MUGEN_ATTN_OK;
    if (a->kv_len == 0) return fail(MUGEN_ATTN_E_INVALID, "gqa_prefill: kv_len == 0 with n_tokens > 0");
    if (a->causal && a->start_pos + a->n_tokens > a->kv_len)
        return fail(MUGEN_ATTN_E_INVALID, "gqa_prefill: start_pos + n_tokens (%d) > kv_len (%d)",
                    a->start_pos + a->n_tokens, a->kv_len);
    if ((int64_t)a->kv_len * a->n_kv_heads * a->head_dim * 2 > INT32_MAX)
        return fail(MUGEN_ATTN_E_UNSUPPORTED, "gqa_prefill: K/V cache larger than 2 GiB per tensor");
    return MUGEN_ATTN_OK;
}

// the optional fp16 copy of V (BF16 prompts from kPrefillV16MinTokens on:
// measured where the extra launch pays for itself)
constexpr int kPrefillV16MinTokens = 1024;
static size_t gqa_prefill_ws(const mugen_attn_gqa_prefill_args* a) {
    return (size_t)a->kv_len * a->n_kv_heads * a->head_dim * 2 + 256;
}

static bool gqa_prefill_v16_capable(const mugen_attn_gqa_prefill_args* a) {
    return a->head_dim <= 128 && a->dtype == DT_BF16;
}

// The automatic choice of the short-prompt kernel: the whole kv range fits
// on chip, from 384 visible keys on (below that the per-block kernel's
// shorter load phase wins: Llama-3.2-1B N = 128 4.4 against 4.9 us; N = 256
// 5.55 against 5.6, N = 512 7.9 against 7.5)
static bool gqa_prefill_short_default(const mugen_attn_gqa_prefill_args* a) {
    GqaPrefillParams p{};
    p.N = a->n_tokens;
    p.G = a->n_heads / a->n_kv_heads;
    p.hd = a->head_dim;
    p.kv_len = a->kv_len;
    p.start_pos = a->start_pos;
    p.causal = a->causal ? 1 : 0;
    const int kv_range = a->causal ? a->start_pos + a->n_tokens : a->kv_len;
    return gqa_prefill_short_fits(p, padded_head_dim(a->head_dim)) && kv_range >= 384;
}

// Key splits for the warp-specialised kernel.  A prompt chunk that
// continues a long context has few 16-token query blocks over a long key
// range: unsplit, workgroups for fewer than half the CUs walk the whole
// range each.  Each block's keys are then split into ranges of whole steps
// (at least kMinKeys, so that the partials' merge stays a small part of the
// call) until the work list fills about one round; the partials (fp16
// O / l, fp32 max and sum) go to the workspace after the fp16 V copy, and
// gqa_prefill_combine merges them.  The plan depends on the arguments only,
// so the workspace size function and the call agree.
struct PrefillSplit {
    int ksplit = 1, kchunk = 0;
    size_t bytes = 0;  // partial O and (max, sum) of every row and split
};
static PrefillSplit gqa_prefill_split(const mugen_attn_gqa_prefill_args* a) {
    PrefillSplit r;
    if (a->head_dim > 128 || a->n_tokens <= 0 || a->kv_len <= 0) return r;
    if (a->kernel && a->kernel != MUGEN_ATTN_PREFILL_KERNEL_WS) return r;
    if (!a->kernel && gqa_prefill_short_default(a)) return r;  // every key on chip already
    const int G = a->n_heads / a->n_kv_heads;
    const int D = padded_head_dim(a->head_dim);
    // a split call with BF16 inputs also takes the fp16 V copy
    const int dt = gqa_prefill_v16_capable(a) ? kDtBf16V16 : a->dtype;
    const int64_t units = (int64_t)ceil_div(a->n_tokens, 16) * a->n_kv_heads * gqa_prefill_ws_slices(G);
    const int64_t target = 256 * (int64_t)gqa_prefill_ws_blocks_per_cu(G, D);
    // half the CUs or more busy unsplit: the partials' round trip costs
    // more than the idle CUs would add (4-head blocks at 256 units, one per
    // CU: 39.6 us split against 34.1 unsplit)
    if (units * 2 > 256) return r;
    const int step = gqa_prefill_ws_step_keys(G, dt);
    const int kend = a->causal ? std::min(a->kv_len, a->start_pos + a->n_tokens) : a->kv_len;
    // 4-head blocks on more than a quarter of the CUs (each running alone on
    // its CU, faster per step than the 2-3 a split puts there) gain only
    // over long ranges: H32 Hk8 d64, 256 tokens after 1024 measured 15.0
    // split against 13.9 us, after 2048 19.3 against 23.4
    if (G <= 4 && units * 4 > 256 && kend < 2048) return r;
    const int steps = ceil_div(kend, step);
    // ranges of at least 256 keys (4 steps of 64, 8 of 32): verify-sized
    // chunks (5 tokens after 4000, 7B shape) 18.1 -> 13.8 us against 512
    // keys; 4-head blocks at 128 keys measured slower (9.2 -> 10.3 us)
    constexpr int kMinKeys = 256;
    const int64_t want =
        std::min<int64_t>({ceil_div(target, units), (int64_t)steps / (kMinKeys / step), (int64_t)kPrefillMaxSplits});
    if (want < 2) return r;
    const int kchunk = ceil_div(steps, (int)want) * step;
    const int ks = ceil_div(kend, kchunk);
    if (ks < 2) return r;
    r.ksplit = ks;
    r.kchunk = kchunk;
    // sized for `want` ranges (ks <= want): want never falls as the key
    // range grows, so the size at the longest range covers every shorter one
    r.bytes = (size_t)a->n_tokens * a->n_heads * want * (a->head_dim * 2 + 2 * sizeof(float)) + 512;
    return r;
}

// The fp16 copy of V (one extra launch over kv_len rows): for long BF16
// prompts, and for split chunks of 8-head blocks with ranges of 1024+ keys.
// Those otherwise convert V in LDS at 32 keys a step (256 tokens after
// 7936: 0.85 us per 32-key step against ~0.6 with the copy; 64.6 -> 55.7 us
// for the call).  4-head blocks keep 32-key steps either way, and 512-key
// ranges (64 tokens after 8000) gain less than the launch costs.  kchunk
// grows with the key range once the split count is capped, so the choice
// never turns off as kv_len grows.
static bool gqa_prefill_uses_v16(const mugen_attn_gqa_prefill_args* a) {
    if (!gqa_prefill_v16_capable(a)) return false;
    if (a->n_tokens >= kPrefillV16MinTokens) return true;
    const PrefillSplit s = gqa_prefill_split(a);
    return s.ksplit > 1 && a->n_heads / a->n_kv_heads > 4 && s.kchunk >= 1024;
}

size_t mugen_attn_gqa_prefill_workspace_size(const mugen_attn_gqa_prefill_args* a) {
    if (gqa_prefill_validate(a) != MUGEN_ATTN_OK) return 0;
    return (gqa_prefill_uses_v16(a) ? gqa_prefill_ws(a) : 0) + gqa_prefill_split(a).bytes;
}

int mugen_attn_gqa_prefill(const mugen_attn_gqa_prefill_args* a, void* stream) {
    if (int rc = gqa_prefill_validate(a)) return rc;
    if (a->n_tokens == 0) return MUGEN_ATTN_OK;
    if (a->head_dim > 128) {
        // head_dim 129..256: the per-token rule of the reference's CPU path
        // (query i of the prompt attends over start_pos + i + 1 keys,
        // transformer.cpp:1334-1335) on the decode kernel's prompt mode, one
        // (token, kv head) per workgroup over the shared cache
        if (a->kernel) return fail(MUGEN_ATTN_E_UNSUPPORTED, "gqa_prefill: head_dim > 128 has one kernel (kernel 0)");
        GqaDecodeParams d{};
        d.B = a->n_tokens;
        d.Hk = a->n_kv_heads;
        d.q = static_cast<const uint16_t*>(a->q);
        d.k = static_cast<const uint16_t*>(a->k);
        d.v = static_cast<const uint16_t*>(a->v);
        d.out = a->out;
        d.H = a->n_heads;
        d.G = a->n_heads / a->n_kv_heads;
        d.hd = a->head_dim;
        d.row_stride = a->n_kv_heads * a->head_dim;
        d.chunk = a->kv_len;
        d.num_splits = 1;
        d.seq_stride = 0;
        d.scale_log2 = (a->scale > 0.f ? a->scale : 1.f / sqrtf((float)a->head_dim)) * kLog2e;
        d.max_T = a->kv_len;
        d.pf_start = a->start_pos;
        d.pf_causal = a->causal ? 1 : 0;
        if ((int64_t)a->n_tokens * a->n_kv_heads > INT32_MAX)
            return fail(MUGEN_ATTN_E_UNSUPPORTED, "gqa_prefill: n_tokens * n_kv_heads too large");
        return hip_status(launch_gqa_prefill_wide(d, a->dtype, a->out_dtype, static_cast<hipStream_t>(stream),
                                                  active_timer()),
                          "gqa_prefill launch");
    }
    GqaPrefillParams p{};
    p.q = static_cast<const uint16_t*>(a->q);
    p.k = static_cast<const uint16_t*>(a->k);
    p.v = static_cast<const uint16_t*>(a->v);
    p.out = a->out;
    p.N = a->n_tokens;
    p.H = a->n_heads;
    p.G = a->n_heads / a->n_kv_heads;
    p.hd = a->head_dim;
    p.row_stride = a->n_kv_heads * a->head_dim;
    p.kv_len = a->kv_len;
    p.start_pos = a->start_pos;
    p.causal = a->causal ? 1 : 0;
    const float scale = a->scale > 0.f ? a->scale : 1.f / sqrtf((float)a->head_dim);
    p.scale_log2 = scale * kLog2e;
    // the warp-specialised kernel where it measured faster: every prompt
    // above head_dim 64 (graph replays: Qwen2.5-7B shape N = 16 / 256 / 768
    // 5.9 / 10.7 / 21.6 against 7.5 / 11.9 / 22.4 us, H32 Hk8 d128 N = 768
    // 18.0 against 26.5; eager: N = 8192 603 against 690 us, 32768 8.76
    // against 8.86 ms), at head_dim 64 from 1024 to 4096 tokens (Llama-3.2-1B
    // shape N = 4096 114 against 116 us, N = 8192 423 against 381; below 1024
    // the per-block and short-prompt kernels lead: N = 512 7.7 against 9.2);
    // args->kernel forces one.  At head_dim 64 the limits above are the
    // 4-head blocks' (G <= 4); its 8-head blocks (G > 4) lead at every length
    // (H28 Hk4 d64 N = 6144 203 against 245 us, H16 Hk2 N = 256 7.4 against
    // 8.0; within 1 us either way at N = 512)
    const bool ws_default =
        a->head_dim > 64 || p.G > 4 || (a->n_tokens >= 1024 && a->n_tokens <= 4096);
    int kernel = ws_default ? MUGEN_ATTN_PREFILL_KERNEL_WS : MUGEN_ATTN_PREFILL_KERNEL_BLOCK;
    // prompts whose whole kv range fits on chip: the short-prompt kernel
    const bool short_fits = gqa_prefill_short_fits(p, padded_head_dim(a->head_dim));
    if (gqa_prefill_short_default(a)) kernel = MUGEN_ATTN_PREFILL_KERNEL_SHORT;
    if (a->kernel == MUGEN_ATTN_PREFILL_KERNEL_SHORT && !short_fits)
        return fail(MUGEN_ATTN_E_UNSUPPORTED,
                    "gqa_prefill: the short kernel serves head_dim 64, n_heads/n_kv_heads <= 4 and <= 512 keys");
    if (a->kernel) kernel = a->kernel;
    int dt = a->dtype;
    const size_t v16_bytes = gqa_prefill_uses_v16(a) ? gqa_prefill_ws(a) : 0;
    const PrefillSplit split = gqa_prefill_split(a);  // none for the short kernel (default or forced)
    p.ksplit = 1;
    if (split.ksplit > 1 && a->workspace && a->workspace_bytes >= v16_bytes + split.bytes) {
        // key splits (the warp-specialised kernel): partials after the V copy
        kernel = MUGEN_ATTN_PREFILL_KERNEL_WS;
        p.ksplit = split.ksplit;
        p.kchunk = split.kchunk;
        p.ws_ml = align256(static_cast<char*>(a->workspace) + v16_bytes);
        p.ws_o = reinterpret_cast<uint16_t*>(p.ws_ml + (size_t)a->n_tokens * a->n_heads * split.ksplit * 2);
    }
    if (kernel != MUGEN_ATTN_PREFILL_KERNEL_SHORT && v16_bytes && a->workspace && a->workspace_bytes >= v16_bytes) {
        // V -> fp16 once for the whole call (the kernels then skip their
        // per-workgroup conversion)
        uint16_t* v16 = reinterpret_cast<uint16_t*>(align256(a->workspace));
        hipError_t e = launch_v_to_f16(p.v, v16, (int64_t)a->kv_len * p.row_stride, static_cast<hipStream_t>(stream),
                                       active_timer());
        if (e != hipSuccess) return hip_status(e, "gqa_prefill V conversion launch");
        p.v = v16;
        dt = kDtBf16V16;
    }
    hipError_t e = launch_gqa_prefill(p, a->n_kv_heads, padded_head_dim(a->head_dim), dt, a->out_dtype, kernel,
                                      static_cast<hipStream_t>(stream), active_timer());
    return hip_status(e, "gqa_prefill launch");
}

size_t mugen_attn_mla_decode_workspace_size(const mugen_attn_mla_decode_args* a) {
    if (mla_validate(a) != MUGEN_ATTN_OK) return 0;
    const int bound = (!a->seq_lens_host && a->num_splits <= 0)
                          ? stride_bound(a->max_seq_len, mla_tile_tokens(mla_kernel(a)), 0)
                          : 0;
    return mla_ws(a, mla_chunk(a, mla_kernel(a)), nullptr, bound);
}

}  // extern "C"

// The MLA decode call behind both entry points: `ws` is the caller's
// workspace or the library's fixed scratch.
static int mla_decode_impl(const mugen_attn_mla_decode_args* a, void* ws, size_t ws_bytes, void* stream,
                           KernelTimer* timer) {
    const int kernel = mla_kernel(a);
    const int chunk = mla_chunk(a, kernel);
    int splits = 1;
    const size_t need = mla_ws(a, chunk, &splits);
    if (!ws || ws_bytes < need)
        return fail(MUGEN_ATTN_E_WORKSPACE, "mla_decode: workspace of %zu bytes required, %zu given", need,
                    ws_bytes);
    MlaParams p{};
    p.q = a->q;
    p.lat = static_cast<const uint16_t*>(a->latent);
    p.seq_lens = a->seq_lens;
    p.out = a->out;
    p.q_len = a->q_len;
    p.H = a->n_heads;
    p.B = a->batch;
    p.R = a->q_len * a->n_heads;
    p.nrb = ceil_div(p.R, mla_rows_per_block(kernel));
    p.nq = ceil_div(p.R, 16);
    const int64_t units = mla_units(a, chunk, p.nrb);
    // the kernels number the work units and the grid in 32 bits
    if (units > (int64_t)1 << 30)
        return fail(MUGEN_ATTN_E_UNSUPPORTED, "mla_decode: batch * splits * row blocks too large");
    p.units = (int)units;
    p.chunk = chunk;
    p.num_splits = splits;
    p.max_T = a->max_seq_len;
    p.seq_stride = a->seq_stride;
    p.scale_log2 = a->scale * kLog2e;
    {
        float* base = align256(ws);
        const size_t sb = (size_t)a->batch * splits;
        p.ws_o = base;
        p.ws_ml = base + sb * (size_t)p.nq * 16 * 512 / 2;  // after the fp16 O blob
    }
    hipError_t e = launch_mla_decode(p, kernel, a->q_dtype, a->latent_dtype, a->out_dtype,
                                     static_cast<hipStream_t>(stream), timer);
    return hip_status(e, "mla_decode launch");
}

// Fixed device scratch of mugen_attn_mla_decode_noalloc: every GPU the
// library runs on holds its own copy of this array until the process ends.
// Host code must not use the array's name as a device address (it is a
// host-side stand-in): the per-device address comes from
// hipGetSymbolAddress, taken once per device with that device current.
static __device__ __align__(256) char mla_scratch[MUGEN_ATTN_MLA_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};
}  // namespace

static int scratch_for_current_device(void** out) {
    int dev = -1;
    if (int rc = hip_status(hipGetDevice(&dev), "mla_decode_noalloc: hipGetDevice")) return rc;
    if (dev < 0 || dev >= kMaxDevices) return fail(MUGEN_ATTN_E_UNSUPPORTED, "mla_decode_noalloc: device %d", dev);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* ptr = nullptr;
        if (int rc = hip_status(hipGetSymbolAddress(&ptr, HIP_SYMBOL(mla_scratch)),
                                "mla_decode_noalloc: hipGetSymbolAddress"))
            return rc;
        if (!ptr) return fail(MUGEN_ATTN_E_HIP, "mla_decode_noalloc: no scratch address");
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    return MUGEN_ATTN_OK;
}

extern "C" {

int mugen_attn_mla_decode(const mugen_attn_mla_decode_args* a, void* ws, size_t ws_bytes, void* stream) {
    if (int rc = mla_validate(a)) return rc;
    return mla_decode_impl(a, ws, ws_bytes, stream, active_timer());
}

int mugen_attn_mla_decode_noalloc(const mugen_attn_mla_decode_args* a, void* stream) {
    if (int rc = mla_validate(a)) return rc;
    const size_t need = mla_ws(a, mla_chunk(a, mla_kernel(a)), nullptr);
    if (need > (size_t)MUGEN_ATTN_MLA_SCRATCH_BYTES)
        return fail(MUGEN_ATTN_E_WORKSPACE,
                    "mla_decode_noalloc: the call needs %zu bytes of scratch, the fixed scratch holds %zu "
                    "(use mugen_attn_mla_decode with a workspace)",
                    need, (size_t)MUGEN_ATTN_MLA_SCRATCH_BYTES);
    void* ws = nullptr;
    if (int rc = scratch_for_current_device(&ws)) return rc;
    // no event timing here: this entry point creates nothing
    return mla_decode_impl(a, ws, MUGEN_ATTN_MLA_SCRATCH_BYTES, stream, nullptr);
}

// yarn_rope_freq (transformer.cpp:41-70) in the same float operations, so
// the table matches the reference's frequencies bit for bit
static RopeFreqs yarn_freqs(const mugen_attn_rope_params& r) {
#pragma clang fp contract(off)
    RopeFreqs out{};
    constexpr int RD = 64;
    const float pi_f = 3.14159265358979323846f;
    for (int i = 0; i < RD / 2; i++) {
        float freq = 1.0f / std::pow(r.theta, 2.0f * (float)i / (float)RD);
        if (r.factor > 1.0f) {
            const float log_base = std::log(r.theta);
            const float ctx_f = (float)r.original_ctx;
            float low = std::floor((float)RD * std::log(ctx_f / (32.0f * 2.0f * pi_f)) / (2.0f * log_base));
            float high = std::ceil((float)RD * std::log(ctx_f / (1.0f * 2.0f * pi_f)) / (2.0f * log_base));
            low = std::max(low, 0.0f);
            high = std::min(high, (float)(RD / 2 - 1));
            const float idx = (float)i;
            if (idx > high) {
                freq = freq / r.factor;
            } else if (idx >= low) {
                float ramp = (idx - low) / std::max(0.001f, high - low);
                ramp = std::max(0.0f, std::min(1.0f, ramp));
                freq = freq * (1.0f - ramp) + (freq / r.factor) * ramp;
            }
        }
        out.f[i] = freq;
    }
    return out;
}

static bool rope_ok(const mugen_attn_rope_params& r) {
    return std::isfinite(r.theta) && r.theta > 0.f && std::isfinite(r.factor) && (r.factor <= 1.f || r.original_ctx > 0);
}

static bool is_wtype(int w) { return w == W_F16 || w == W_Q8_0 || w == W_Q4_0; }

// weight rows: F16 rows are read 16 bytes at a time, block rows 2 at a time
static bool w_aligned(const void* w, int w_type) {
    return ((uintptr_t)w & (w_type == W_F16 ? 15 : 1)) == 0;
}

// validation and kernel parameters of an absorption (rows == 0: nothing to do)
static int absorb_params(const mugen_attn_mla_absorb_args* a, MlaProjParams* p) {
    if (!a) return fail(MUGEN_ATTN_E_INVALID, "mla_absorb: null args");
    if (a->rows < 0 || a->n_heads <= 0) return fail(MUGEN_ATTN_E_INVALID, "mla_absorb: bad rows/n_heads");
    if (a->nope_dim != 128 || a->rope_dim != 64 || a->kv_rank != 512)
        return fail(MUGEN_ATTN_E_UNSUPPORTED, "mla_absorb: nope/rope/kv_rank %d/%d/%d (supported: 128/64/512)",
                    a->nope_dim, a->rope_dim, a->kv_rank);
    if (!is_wtype(a->w_type)) return fail(MUGEN_ATTN_E_UNSUPPORTED, "mla_absorb: w_type %d", a->w_type);
    if (a->out_dtype != DT_F32 && a->out_dtype != DT_BF16)
        return fail(MUGEN_ATTN_E_UNSUPPORTED, "mla_absorb: out_dtype must be F32 or BF16");
    *p = MlaProjParams{};
    if (a->rows == 0) return MUGEN_ATTN_OK;
    if (!a->q || !a->w_kb || !a->q_abs) return fail(MUGEN_ATTN_E_INVALID, "mla_absorb: null pointer");
    if (((uintptr_t)a->q & 1) || ((uintptr_t)a->q_abs & 3) || !w_aligned(a->w_kb, a->w_type))
        return fail(MUGEN_ATTN_E_INVALID, "mla_absorb: misaligned q/q_abs/w_kb");
    if ((int64_t)a->rows * a->n_heads > (1 << 24))
        return fail(MUGEN_ATTN_E_UNSUPPORTED, "mla_absorb: rows*n_heads too large");
    const bool rope = a->positions || a->seq_base;
    if (rope && !rope_ok(a->rope)) return fail(MUGEN_ATTN_E_INVALID, "mla_absorb: bad rope parameters");
    if (!a->positions && a->seq_base && a->rows_per_seq <= 0)
        return fail(MUGEN_ATTN_E_INVALID, "mla_absorb: rows_per_seq must be > 0 with seq_base");
    *p = MlaProjParams{a->q, a->w_kb, a->q_abs, a->rows, a->n_heads, a->positions, {},
                       a->positions ? nullptr : a->seq_base, a->rows_per_seq > 0 ? a->rows_per_seq : 1};
    if (rope) p->freqs = yarn_freqs(a->rope);
    return MUGEN_ATTN_OK;
}

int mugen_attn_mla_absorb(const mugen_attn_mla_absorb_args* a, void* stream) {
    MlaProjParams p;
    if (int rc = absorb_params(a, &p)) return rc;
    if (p.rows == 0) return MUGEN_ATTN_OK;
    return hip_status(launch_mla_absorb(p, a->w_type, a->out_dtype, static_cast<hipStream_t>(stream), active_timer()),
                      "mla_absorb launch");
}

int mugen_attn_mla_project(const mugen_attn_mla_project_args* a, void* stream) {
    if (!a) return fail(MUGEN_ATTN_E_INVALID, "mla_project: null args");
    if (a->rows < 0 || a->n_heads <= 0) return fail(MUGEN_ATTN_E_INVALID, "mla_project: bad rows/n_heads");
    if (a->kv_rank != 512 || a->v_head_dim != 128)
        return fail(MUGEN_ATTN_E_UNSUPPORTED, "mla_project: kv_rank/v_head_dim %d/%d (supported: 512/128)",
                    a->kv_rank, a->v_head_dim);
    if (!is_wtype(a->w_type)) return fail(MUGEN_ATTN_E_UNSUPPORTED, "mla_project: w_type %d", a->w_type);
    if (a->out_dtype != DT_F32 && a->out_dtype != DT_F16)
        return fail(MUGEN_ATTN_E_UNSUPPORTED, "mla_project: out_dtype must be F16 or F32");
    if (a->rows == 0) return MUGEN_ATTN_OK;
    if (!a->o || !a->w_vb || !a->out) return fail(MUGEN_ATTN_E_INVALID, "mla_project: null pointer");
    if (((uintptr_t)a->o & 15) || ((uintptr_t)a->out & 3) || !w_aligned(a->w_vb, a->w_type))
        return fail(MUGEN_ATTN_E_INVALID, "mla_project: misaligned o/out/w_vb");
    if ((int64_t)a->rows * a->n_heads > (1 << 24))
        return fail(MUGEN_ATTN_E_UNSUPPORTED, "mla_project: rows*n_heads too large");
    MlaProjParams p{a->o, a->w_vb, a->out, a->rows, a->n_heads, nullptr, {}, nullptr, 1};
    return hip_status(launch_mla_project(p, a->w_type, a->out_dtype, static_cast<hipStream_t>(stream), active_timer()),
                      "mla_project launch");
}

// validation and kernel parameters of a latent write (rows == 0: nothing to do)
static int latent_params(const mugen_attn_mla_latent_write_args* a, LatentWriteParams* p) {
    if (!a) return fail(MUGEN_ATTN_E_INVALID, "mla_latent_write: null args");
    if (a->kv_rank != 512 || a->rope_dim != 64)
        return fail(MUGEN_ATTN_E_UNSUPPORTED, "mla_latent_write: kv_rank/rope_dim %d/%d (supported: 512/64)",
                    a->kv_rank, a->rope_dim);
    if (!is16(a->latent_dtype)) return fail(MUGEN_ATTN_E_UNSUPPORTED, "mla_latent_write: latent dtype must be F16/BF16");
    if (a->rows < 0 || a->rows_per_seq <= 0 || a->max_seq_len <= 0)
        return fail(MUGEN_ATTN_E_INVALID, "mla_latent_write: bad rows/rows_per_seq/max_seq_len");
    if (!(a->eps >= 0.f) || !std::isfinite(a->eps)) return fail(MUGEN_ATTN_E_INVALID, "mla_latent_write: bad eps");
    if (!rope_ok(a->rope)) return fail(MUGEN_ATTN_E_INVALID, "mla_latent_write: bad rope parameters");
    *p = LatentWriteParams{};
    if (a->rows == 0) return MUGEN_ATTN_OK;
    if (!a->kv_a || !a->norm_w || (!a->positions && !a->seq_base) || !a->latent)
        return fail(MUGEN_ATTN_E_INVALID, "mla_latent_write: null pointer");
    const int n_seq = (a->rows + a->rows_per_seq - 1) / a->rows_per_seq;
    if (n_seq > 1 && a->seq_stride < (int64_t)a->max_seq_len * 576)
        return fail(MUGEN_ATTN_E_INVALID, "mla_latent_write: seq_stride smaller than max_seq_len*576");
    if ((((uintptr_t)a->kv_a | (uintptr_t)a->norm_w | (uintptr_t)a->latent) & 15) || (a->seq_stride % 8))
        return fail(MUGEN_ATTN_E_INVALID, "mla_latent_write: kv_a/norm_w/latent must be 16-byte aligned, "
                    "seq_stride a multiple of 8");
    p->kv_a = static_cast<const uint16_t*>(a->kv_a);
    p->norm_w = static_cast<const uint16_t*>(a->norm_w);
    p->positions = a->positions;
    p->seq_base = a->positions ? nullptr : a->seq_base;
    p->latent = static_cast<uint16_t*>(a->latent);
    p->rows = a->rows;
    p->rows_per_seq = a->rows_per_seq;
    p->max_seq_len = a->max_seq_len;
    p->seq_stride = a->seq_stride;
    p->eps = a->eps;
    p->freqs = yarn_freqs(a->rope);
    return MUGEN_ATTN_OK;
}

int mugen_attn_mla_latent_write(const mugen_attn_mla_latent_write_args* a, void* stream) {
    LatentWriteParams p;
    if (int rc = latent_params(a, &p)) return rc;
    if (p.rows == 0) return MUGEN_ATTN_OK;
    return hip_status(launch_mla_latent_write(p, a->latent_dtype, static_cast<hipStream_t>(stream), active_timer()),
                      "mla_latent_write launch");
}

int mugen_attn_mla_prepare(const mugen_attn_mla_latent_write_args* lw, const mugen_attn_mla_absorb_args* ab,
                           void* stream) {
    LatentWriteParams pl;
    MlaProjParams pa;
    if (int rc = latent_params(lw, &pl)) return rc;
    if (int rc = absorb_params(ab, &pa)) return rc;
    if (pl.rows == 0 && pa.rows == 0) return MUGEN_ATTN_OK;
    return hip_status(launch_mla_prepare(pa, pl, ab->w_type, ab->out_dtype, lw->latent_dtype,
                                         static_cast<hipStream_t>(stream), active_timer()),
                      "mla_prepare launch");
}

int mugen_attn_kv_append(const mugen_attn_kv_append_args* a, void* stream) {
    if (!a) return fail(MUGEN_ATTN_E_INVALID, "kv_append: null args");
    if (a->n_seq < 0 || a->n_new < 0 || a->row <= 0 || a->max_seq_len <= 0)
        return fail(MUGEN_ATTN_E_INVALID, "kv_append: bad sizes");
    if (a->n_seq == 0 || a->n_new == 0) return MUGEN_ATTN_OK;
    if (!a->k_new || !a->v_new || !a->k_cache || !a->v_cache || !a->seq_lens)
        return fail(MUGEN_ATTN_E_INVALID, "kv_append: null pointer");
    if (a->row % 8) return fail(MUGEN_ATTN_E_UNSUPPORTED, "kv_append: row must be a multiple of 8");
    if (a->n_seq > 1 && a->seq_stride < (int64_t)a->max_seq_len * a->row)
        return fail(MUGEN_ATTN_E_INVALID, "kv_append: seq_stride smaller than max_seq_len*row");
    if ((((uintptr_t)a->k_new | (uintptr_t)a->v_new | (uintptr_t)a->k_cache | (uintptr_t)a->v_cache) & 15) ||
        (a->seq_stride % 8))
        return fail(MUGEN_ATTN_E_INVALID, "kv_append: buffers must be 16-byte aligned, seq_stride a multiple of 8");
    if (a->n_seq > 65535) return fail(MUGEN_ATTN_E_UNSUPPORTED, "kv_append: too many sequences");
    KvAppendParams p{};
    p.k_new = static_cast<const uint16_t*>(a->k_new);
    p.v_new = static_cast<const uint16_t*>(a->v_new);
    p.k_cache = static_cast<uint16_t*>(a->k_cache);
    p.v_cache = static_cast<uint16_t*>(a->v_cache);
    p.seq_lens = a->seq_lens;
    p.seq_stride = a->seq_stride;
    p.row = a->row;
    p.n_new = a->n_new;
    p.max_seq_len = a->max_seq_len;
    return hip_status(launch_kv_append(p, a->n_seq, static_cast<hipStream_t>(stream), active_timer()),
                      "kv_append launch");
}

int mugen_attn_seq_advance(int32_t* seq_lens, int32_t n, int32_t count, int32_t max_seq_len, int32_t* n_q4,
                           const int32_t* n_q4_next, void* stream) {
    if (count == 0) return MUGEN_ATTN_OK;
    if (!seq_lens || count < 0 || max_seq_len <= 0 || (n_q4 && !n_q4_next) || (n_q4 && n_q4 == n_q4_next))
        return fail(MUGEN_ATTN_E_INVALID, "seq_advance: bad arguments");
    return hip_status(launch_seq_advance(seq_lens, n, count, max_seq_len, n_q4, n_q4_next,
                                         static_cast<hipStream_t>(stream), active_timer()),
                      "seq_advance launch");
}

int mugen_attn_scatter_kv(const void* src, void* dst, uint64_t offset, uint64_t count, void* stream) {
    if (count == 0) return MUGEN_ATTN_OK;
    if (!src || !dst) return fail(MUGEN_ATTN_E_INVALID, "scatter_kv: null pointer");
    hipError_t e = launch_scatter_kv(static_cast<const uint16_t*>(src), static_cast<uint16_t*>(dst), offset, count,
                                     static_cast<hipStream_t>(stream), active_timer());
    return hip_status(e, "scatter_kv launch");
}

int mugen_attn_timing_enable(int enable) {
    std::lock_guard<std::mutex> lk(g_timer.mu);
    g_timer.enabled = enable != 0;
    return MUGEN_ATTN_OK;
}

int mugen_attn_timing_read(const char* kernel, double* total_ms, int64_t* launches) {
    if (!kernel) return fail(MUGEN_ATTN_E_INVALID, "timing_read: null kernel name");
    std::lock_guard<std::mutex> lk(g_timer.mu);
    g_timer.drain();
    auto it = g_timer.totals.find(kernel);
    if (total_ms) *total_ms = it == g_timer.totals.end() ? 0.0 : it->second.first;
    if (launches) *launches = it == g_timer.totals.end() ? 0 : it->second.second;
    return MUGEN_ATTN_OK;
}

void mugen_attn_timing_reset(void) {
    std::lock_guard<std::mutex> lk(g_timer.mu);
    g_timer.drain();
    g_timer.totals.clear();
}

}  // extern "C"
