// Token sampling on the device (gfx950): Sampler::sample
// (src/model/sampler.rs:133-196), bit-identical to the reference on the same
// logits, parameters and xorshift64 state, with two cases the reference
// leaves open: its top-k and top-p sorts are unstable, so equal values that
// straddle the cut may come in any order there (here: index order, equal to
// the reference whenever no such tie straddles the cut), and with NaN values
// their comparator is not an order at all, so the kept set is unspecified
// (here: an error, under top-k and top-p alike).
//
// The reference, on a copy of the logits:
//   repetition penalty (:151-164)   each distinct history id once:
//                                   l > 0 ? l / r : l * r
//   temperature (:166-176)          l *= 1 / t
//   top-k (:201-223)                l < (k-th largest) -> -inf
//   softmax_to_probs (:225-252)     max; e = exp(l - max); Σe left to right;
//                                   e *= 1 / Σ
//   top-p (:254-311)                descending order, running f32 sum until
//                                   it reaches p, the rest zeroed; Σ left to
//                                   right; p *= 1 / Σ
//   multinomial (:178-196)          total = Σp left to right; r = u * total;
//                                   the first i whose running sum reaches r
// Here one 1024-thread workgroup runs each phase; the element-wise work is
// spread over the threads, every left-to-right sum is the exact one
// (wm::seq_sum_nonneg, the same f32 bits as the sequential loop), the
// "first index whose running sum reaches r" is found by narrowing over exact
// partial sums (monotone: the terms are non-negative), and the two orders
// (the k-th largest logit, the descending probabilities) come from a stable
// device radix sort (rocPRIM) of order-preserving integer keys.  Equal
// probabilities at the top-p cut are taken in index order; the reference's
// unstable sort leaves that order open.  exp is glibc's expf, restated in
// wm_expf.h.
#include <rocprim/device/device_radix_sort.hpp>

#include <cmath>
#include <cstdio>
#include <vector>

#include "wm_internal.h"
#include "wm_seqsum.h"

namespace {

constexpr int kSampleThreads = 1024;

enum : uint32_t {
    SAMPLE_RUNNING = 0,
    SAMPLE_DONE = 1,         // id valid
    SAMPLE_NOT_POSITIVE = 2, // multinomial: total <= 0 or not finite (total valid)
    SAMPLE_NAN_ORDER = 3,    // NaN values to sort: top-k's logits, or top-p's probabilities
};

struct sample_state {
    uint32_t status;
    uint32_t id;
    float total;
    uint32_t pad;
};

enum { TOPK_NONE = 0, TOPK_ALL = 1, TOPK_THRESHOLD = 2 };
enum { TOPP_NONE = 0, TOPP_ONE_HOT = 1, TOPP_CUT = 2, TOPP_KEEP_ALL = 3 };

struct sample_args {
    const float *logits;
    uint32_t n;
    float *work, *probs;
    uint32_t *keys, *vals;          // sort inputs
    const uint32_t *skeys, *svals;  // sort outputs
    uint8_t *keep;
    const uint32_t *hist;
    uint32_t n_hist;
    int greedy;
    int use_rep;
    float rep;
    int use_temp;
    float inv_t;
    int topk_mode;
    uint32_t k;
    int topp_mode;
    float top_p;
    float unit;  // the xorshift64 draw in [0, 1)
    sample_state *st;
};

// Order-preserving keys: key(a) < key(b) iff a < b for non-NaN floats
// (-0 below +0, which no phase distinguishes).
__device__ __forceinline__ uint32_t order_key(float v) {
    const uint32_t b = __float_as_uint(v);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float key_value(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// argmax as lm_head.rs:161-174 (`if v > best`, starting from a[0]): index 0
// when a[0] is NaN, else the first index of the maximum over the non-NaN
// values (a NaN never compares greater).  Every thread gets the result.
__device__ uint32_t block_argmax_first(const float *a, uint32_t n, float *rv, uint32_t *ri) {
    const uint32_t tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    float bv = -INFINITY;
    uint32_t bi = 0xffffffffu;
    for (uint32_t i = tid; i < n; i += kSampleThreads) {
        const float v = a[i];
        if (!isnan(v) && (bi == 0xffffffffu || v > bv)) {
            bv = v;
            bi = i;
        }
    }
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o, 64);
        const uint32_t oi = __shfl_xor(bi, o, 64);
        const bool take = oi != 0xffffffffu && (bi == 0xffffffffu || ov > bv || (ov == bv && oi < bi));
        bv = take ? ov : bv;
        bi = take ? oi : bi;
    }
    wm_sync_lds();
    if (lane == 0) {
        rv[wid] = bv;
        ri[wid] = bi;
    }
    wm_sync_lds();
    bv = rv[0];
    bi = ri[0];
    for (int w = 1; w < kSampleThreads / 64; w++) {
        const float ov = rv[w];
        const uint32_t oi = ri[w];
        if (oi != 0xffffffffu && (bi == 0xffffffffu || ov > bv || (ov == bv && oi < bi))) {
            bv = ov;
            bi = oi;
        }
    }
    return isnan(a[0]) || bi == 0xffffffffu ? 0u : bi;
}

// The first i in [0, n) at which the left-to-right f32 sum a[0] + ... + a[i]
// reaches r (>= r), or n if it never does; a[] non-negative and finite, so
// the running sum never decreases.  One wave (all 64 lanes, same result):
// exact partial sums over 4096-term chunks locate the chunk where the sum
// first reaches r, then 512-, 64- and 8-term pieces of it, then the terms
// one by one, always continuing from the exact sum before the piece.
__device__ uint32_t seq_first_reach(const float *a, uint32_t n, float r) {
    uint32_t lo = 0, hi = n;
    float s = 0.0f;
    for (uint32_t w = 4096;; w >>= 3) {
        if (w < 8) {
            for (uint32_t i = lo; i < hi; i++) {
                s = s + a[i];
                if (s >= r) return i;
            }
            return n;
        }
        uint32_t pos = lo;
        bool found = false;
        while (pos < hi) {
            const uint32_t len = min(w, hi - pos);
            const float s2 = wm::seq_sum_nonneg_from(s, a + pos, len);
            if (s2 >= r) {
                lo = pos;
                hi = pos + len;
                found = true;
                break;
            }
            s = s2;
            pos += len;
        }
        if (!found) return n;
    }
}

// Greedy: the argmax.  Otherwise: copy, repetition penalty, temperature,
// and the keys of the top-k sort.
__global__ __launch_bounds__(kSampleThreads) void k_sample_pre(sample_args a) {
    __shared__ float rv[16];
    __shared__ uint32_t ri[16];
    const uint32_t n = a.n, tid = threadIdx.x;
    if (a.greedy) {
        const uint32_t id = block_argmax_first(a.logits, n, rv, ri);
        if (tid == 0) {
            a.st->id = id;
            a.st->status = SAMPLE_DONE;
        }
        return;
    }
    if (tid == 0) a.st->status = SAMPLE_RUNNING;
    for (uint32_t i = tid; i < n; i += kSampleThreads) a.work[i] = a.logits[i];
    if (a.use_rep) {
        __syncthreads();
        for (uint32_t h = tid; h < a.n_hist; h += kSampleThreads) {
            const uint32_t id = a.hist[h];
            if (id >= n) continue;
            bool first = true;
            for (uint32_t j = 0; j < h && first; j++) first = a.hist[j] != id;
            if (first) {  // one thread per distinct id: no two threads touch one logit
                const float l = a.work[id];
                a.work[id] = l > 0.0f ? l / a.rep : l * a.rep;
            }
        }
        __syncthreads();
    }
    int bad = 0;
    for (uint32_t i = tid; i < n; i += kSampleThreads) {
        float v = a.work[i];
        if (a.use_temp) v = v * a.inv_t;
        a.work[i] = v;
        if (a.topk_mode == TOPK_THRESHOLD) {
            a.keys[i] = order_key(v);
            bad |= isnan(v);
        }
    }
    // a NaN among the values top-k sorts leaves the k-th largest unspecified
    if (__syncthreads_or(bad) && tid == 0) a.st->status = SAMPLE_NAN_ORDER;
}

// Top-k mask, softmax_to_probs, and top-p's one-hot case or its sort keys.
__global__ __launch_bounds__(kSampleThreads) void k_sample_probs(sample_args a) {
    __shared__ float rv[16];
    __shared__ uint32_t ri[16];
    __shared__ float bcast;
    if (a.st->status != SAMPLE_RUNNING) return;
    const uint32_t n = a.n, tid = threadIdx.x, wid = tid >> 6, lane = tid & 63;
    const float thr = a.topk_mode == TOPK_THRESHOLD ? key_value(a.skeys[a.k - 1]) : 0.0f;
    float m = -INFINITY;
    for (uint32_t i = tid; i < n; i += kSampleThreads) {
        float v = a.work[i];
        if (a.topk_mode == TOPK_ALL || (a.topk_mode == TOPK_THRESHOLD && v < thr)) v = -INFINITY;
        a.work[i] = v;
        m = wm_max_nonan(m, v);
    }
    m = wm_block_max_nonan(m, rv);
    if (!isfinite(m)) {
        for (uint32_t i = tid; i < n; i += kSampleThreads) a.probs[i] = 0.0f;
    } else {
        for (uint32_t i = tid; i < n; i += kSampleThreads) a.probs[i] = wm_expf(a.work[i] - m);
        __syncthreads();
        if (wid == 0) {
            const float s = wm::seq_sum_nonneg(a.probs, n);
            if (lane == 0) bcast = s;
        }
        __syncthreads();
        const float sum = bcast;
        if (sum > 0.0f) {
            const float inv = 1.0f / sum;
            for (uint32_t i = tid; i < n; i += kSampleThreads) a.probs[i] *= inv;
        }
    }
    if (a.topp_mode == TOPP_ONE_HOT) {
        __syncthreads();
        const uint32_t am = block_argmax_first(a.probs, n, rv, ri);
        for (uint32_t i = tid; i < n; i += kSampleThreads) a.probs[i] = i == am ? 1.0f : 0.0f;
    } else if (a.topp_mode == TOPP_CUT) {
        int bad = 0;
        for (uint32_t i = tid; i < n; i += kSampleThreads) {
            const float v = a.probs[i];
            bad |= isnan(v);
            a.keys[i] = order_key(v);
            a.vals[i] = i;
        }
        if (__syncthreads_or(bad) && tid == 0) a.st->status = SAMPLE_NAN_ORDER;
    }
}

// Top-p's cut and renormalisation, then the multinomial draw.
__global__ __launch_bounds__(kSampleThreads) void k_sample_finish(sample_args a) {
    __shared__ float bcast;
    __shared__ uint32_t bcast_u;
    if (a.st->status != SAMPLE_RUNNING) return;
    const uint32_t n = a.n, tid = threadIdx.x, wid = tid >> 6, lane = tid & 63;
    if (a.topp_mode == TOPP_CUT) {
        // the probabilities in descending order (equal ones in index order)
        for (uint32_t s = tid; s < n; s += kSampleThreads) a.work[s] = key_value(a.skeys[s]);
        for (uint32_t i = tid; i < n; i += kSampleThreads) a.keep[i] = 0;
        __syncthreads();
        if (wid == 0) {
            const uint32_t j = seq_first_reach(a.work, n, a.top_p);
            if (lane == 0) bcast_u = j;
        }
        __syncthreads();
        const uint32_t cut = bcast_u == n ? n : bcast_u + 1;  // the entry that reaches p is kept
        for (uint32_t s = tid; s < cut; s += kSampleThreads) a.keep[a.svals[s]] = 1;
        __syncthreads();
        for (uint32_t i = tid; i < n; i += kSampleThreads)
            if (!a.keep[i]) a.probs[i] = 0.0f;
    }
    if (a.topp_mode == TOPP_CUT || a.topp_mode == TOPP_KEEP_ALL) {
        __syncthreads();
        if (wid == 0) {
            const float s = wm::seq_sum_nonneg(a.probs, n);
            if (lane == 0) bcast = s;
        }
        __syncthreads();
        const float sum = bcast;
        if (sum > 0.0f) {
            const float inv = 1.0f / sum;
            for (uint32_t i = tid; i < n; i += kSampleThreads) a.probs[i] *= inv;
        }
    }
    __syncthreads();
    if (wid == 0) {
        const float total = wm::seq_sum_nonneg(a.probs, n);
        if (total <= 0.0f || !isfinite(total)) {
            if (lane == 0) {
                a.st->total = total;
                a.st->status = SAMPLE_NOT_POSITIVE;
            }
        } else {
            const float r = a.unit * total;
            const uint32_t j = seq_first_reach(a.probs, n, r);
            if (lane == 0) {
                a.st->total = total;
                a.st->id = j == n ? n - 1 : j;
                a.st->status = SAMPLE_DONE;
            }
        }
    }
}

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

// Rust's `{}` of an f32 for the values the multinomial error can show.
void rust_f32(float v, char *buf, size_t len) {
    if (std::isnan(v)) snprintf(buf, len, "NaN");
    else if (std::isinf(v)) snprintf(buf, len, v > 0 ? "inf" : "-inf");
    else if (v == 0.0f) snprintf(buf, len, std::signbit(v) ? "-0" : "0");
    else snprintf(buf, len, "%.9g", (double)v);
}

}  // namespace

struct wm_sampler {
    wm_ctx *ctx = nullptr;
    int device = 0;
    wm_sampling_params p{};
    uint64_t state = 0;
    std::vector<uint32_t> hist;
    // device workspace for n values (grown on demand)
    void *ws = nullptr;
    size_t ws_bytes = 0;
    uint32_t *d_hist = nullptr;
    size_t d_hist_cap = 0, d_hist_synced = 0;
};

namespace {

uint64_t xorshift_next(uint64_t &s) {  // XorShift64::next_u64 (sampler.rs:26-33)
    uint64_t x = s;
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    s = x;
    return x;
}

bool is_greedy(const wm_sampling_params &p) {  // SamplingParams::is_greedy (sampler.rs:71-78)
    return std::fabs(p.temperature) < 1e-9f && !p.has_top_k && !p.has_top_p &&
           !p.has_repetition_penalty;
}

size_t sort_temp_bytes(uint32_t n, hipStream_t s) {
    size_t a = 0, b = 0;
    rocprim::radix_sort_keys_desc(nullptr, a, (uint32_t *)nullptr, (uint32_t *)nullptr, n, 0, 32, s);
    rocprim::radix_sort_pairs_desc(nullptr, b, (uint32_t *)nullptr, (uint32_t *)nullptr,
                                   (uint32_t *)nullptr, (uint32_t *)nullptr, n, 0, 32, s);
    return a > b ? a : b;
}

}  // namespace

// Sample from n logits at d_logits (device).  Called with the sampler's
// context current.
wm_status wm_sampler_run(wm_sampler *sp, const float *d_logits, uint32_t n, uint32_t *out_id) {
    wm_ctx *ctx = sp->ctx;
    hipStream_t s = ctx->stream;
    const wm_sampling_params &p = sp->p;
    const bool greedy = is_greedy(p);
    if (n == 0) {
        if (greedy) return wm_set_error(ctx, WM_E_PARSE, "sample: empty logits");
        return wm_set_error(ctx, WM_E_PARSE,
                            "multinomial: probabilities do not sum to a positive finite value (0)");
    }
    const size_t tmp_bytes = sort_temp_bytes(n, s);
    const size_t f = align256((size_t)n * 4);
    const size_t need = 6 * f + align256(n) + 256 + align256(tmp_bytes) + f;
    if (need > sp->ws_bytes) {
        WM_HIP(ctx, hipStreamSynchronize(s));
        if (sp->ws) WM_HIP(ctx, hipFree(sp->ws));
        sp->ws = nullptr;
        sp->ws_bytes = 0;
        WM_HIP(ctx, hipMalloc(&sp->ws, need));
        sp->ws_bytes = need;
    }
    uint8_t *b = (uint8_t *)sp->ws;
    sample_args a{};
    a.logits = d_logits;
    a.n = n;
    a.work = (float *)b;
    a.probs = (float *)(b + f);
    a.keys = (uint32_t *)(b + 2 * f);
    a.vals = (uint32_t *)(b + 3 * f);
    uint32_t *skeys = (uint32_t *)(b + 4 * f), *svals = (uint32_t *)(b + 5 * f);
    a.skeys = skeys;
    a.svals = svals;
    a.keep = b + 6 * f;
    a.st = (sample_state *)(b + 6 * f + align256(n));
    void *tmp = b + 6 * f + align256(n) + 256;
    a.greedy = greedy;
    // repetition penalty (sampler.rs:151-164): history on the device
    const float r = p.repetition_penalty;
    a.use_rep = !greedy && p.has_repetition_penalty && !(r <= 0.0f || std::fabs(r - 1.0f) < 1e-9f);
    a.rep = r;
    if (a.use_rep && !sp->hist.empty()) {
        if (sp->hist.size() > sp->d_hist_cap) {
            WM_HIP(ctx, hipStreamSynchronize(s));
            if (sp->d_hist) WM_HIP(ctx, hipFree(sp->d_hist));
            sp->d_hist = nullptr;
            sp->d_hist_cap = sp->d_hist_synced = 0;
            const size_t cap = sp->hist.size() * 2 + 256;
            WM_HIP(ctx, hipMalloc((void **)&sp->d_hist, cap * 4));
            sp->d_hist_cap = cap;
        }
        if (sp->d_hist_synced < sp->hist.size()) {
            // the copy reads host memory now (pageable): the vector may grow later
            WM_HIP(ctx, hipMemcpy(sp->d_hist + sp->d_hist_synced, sp->hist.data() + sp->d_hist_synced,
                                  (sp->hist.size() - sp->d_hist_synced) * 4, hipMemcpyHostToDevice));
            sp->d_hist_synced = sp->hist.size();
        }
    }
    a.hist = sp->d_hist;
    a.n_hist = a.use_rep ? (uint32_t)sp->hist.size() : 0;
    // temperature (sampler.rs:166-176)
    const float t = p.temperature;
    a.use_temp = !greedy && !(t <= 0.0f || std::fabs(t - 1.0f) < 1e-9f);
    a.inv_t = 1.0f / t;
    // top-k (sampler.rs:201-223), k clamped to n
    a.topk_mode = TOPK_NONE;
    if (!greedy && p.has_top_k) {
        const uint64_t k = p.top_k < n ? p.top_k : n;
        a.topk_mode = k == 0 ? TOPK_ALL : (k == n ? TOPK_NONE : TOPK_THRESHOLD);
        a.k = (uint32_t)k;
    }
    // top-p (sampler.rs:254-311)
    a.topp_mode = TOPP_NONE;
    a.top_p = p.top_p;
    if (!greedy && p.has_top_p) {
        const float tp = p.top_p;
        if (tp <= 0.0f) a.topp_mode = TOPP_ONE_HOT;
        else if (tp >= 1.0f) a.topp_mode = TOPP_NONE;
        else if (std::isnan(tp)) a.topp_mode = TOPP_KEEP_ALL;  // never reached: every entry kept
        else a.topp_mode = TOPP_CUT;
    }
    // the draw the multinomial would consume (the state advances only if it runs)
    uint64_t next_state = sp->state;
    a.unit = (float)(xorshift_next(next_state) >> 40) / (float)(1ull << 24);

    WM_HIP(ctx, hipSetDevice(sp->device));
    hipLaunchKernelGGL(k_sample_pre, dim3(1), dim3(kSampleThreads), 0, s, a);
    if (!greedy) {
        size_t tb = tmp_bytes;
        if (a.topk_mode == TOPK_THRESHOLD)
            WM_HIP(ctx, rocprim::radix_sort_keys_desc(tmp, tb, a.keys, skeys, n, 0, 32, s));
        hipLaunchKernelGGL(k_sample_probs, dim3(1), dim3(kSampleThreads), 0, s, a);
        if (a.topp_mode == TOPP_CUT)
            WM_HIP(ctx, rocprim::radix_sort_pairs_desc(tmp, tb, a.keys, skeys, a.vals, svals, n, 0, 32, s));
        hipLaunchKernelGGL(k_sample_finish, dim3(1), dim3(kSampleThreads), 0, s, a);
    }
    WM_HIP(ctx, hipGetLastError());
    sample_state st{};
    WM_HIP(ctx, hipMemcpyAsync(&st, a.st, sizeof(st), hipMemcpyDeviceToHost, s));
    WM_HIP(ctx, hipStreamSynchronize(s));
    if (st.status == SAMPLE_NOT_POSITIVE) {
        char v[32];
        rust_f32(st.total, v, sizeof v);
        return wm_set_error(ctx, WM_E_PARSE,
                            "multinomial: probabilities do not sum to a positive finite value (%s)", v);
    }
    if (st.status == SAMPLE_NAN_ORDER)
        return wm_set_error(ctx, WM_E_NONFINITE,
                            a.topp_mode == TOPP_CUT && a.topk_mode != TOPK_THRESHOLD
                                ? "sample: NaN probabilities under top-p (their order is unspecified)"
                                : "sample: NaN values under top-k or top-p (their order is unspecified)");
    if (st.status != SAMPLE_DONE) return wm_set_error(ctx, WM_E_STATE, "sample: did not finish");
    if (!greedy) sp->state = next_state;
    *out_id = st.id;
    return WM_OK;
}

wm_ctx *wm_sampler_ctx(const wm_sampler *sp) { return sp ? sp->ctx : nullptr; }

extern "C" {

wm_status wm_sampler_create(wm_ctx *ctx, const wm_sampling_params *params, uint64_t seed,
                            wm_sampler **out) {
    if (!ctx || !params || !out) return WM_E_ARG;
    wm_sampler *sp = new wm_sampler();
    sp->ctx = ctx;
    sp->device = ctx->device;
    sp->p = *params;
    sp->state = seed ? seed : 0xdeadbeefcafebabeull;  // XorShift64::new (sampler.rs:18-25)
    *out = sp;
    return WM_OK;
}

void wm_sampler_destroy(wm_sampler *sp) {
    if (!sp) return;
    if (hipSetDevice(sp->device) == hipSuccess) {
        if (sp->ws) (void)hipFree(sp->ws);
        if (sp->d_hist) (void)hipFree(sp->d_hist);
    }
    delete sp;
}

wm_status wm_sampler_observe(wm_sampler *sp, uint32_t id) {
    if (!sp) return WM_E_ARG;
    sp->hist.push_back(id);
    return WM_OK;
}

wm_status wm_sampler_checkpoint(const wm_sampler *sp, uint64_t *rng_state, uint64_t *history_len) {
    if (!sp || !rng_state || !history_len) return WM_E_ARG;
    *rng_state = sp->state;
    *history_len = sp->hist.size();
    return WM_OK;
}

wm_status wm_sampler_rollback(wm_sampler *sp, uint64_t rng_state, uint64_t history_len) {
    if (!sp) return WM_E_ARG;
    if (history_len > sp->hist.size())
        return wm_set_error(sp->ctx, WM_E_ARG, "sampler rollback: history length %llu beyond %zu",
                            (unsigned long long)history_len, sp->hist.size());
    sp->state = rng_state;
    sp->hist.resize(history_len);
    if (sp->d_hist_synced > history_len) sp->d_hist_synced = history_len;
    return WM_OK;
}

wm_status wm_sampler_sample_dev(wm_sampler *sp, const float *d_logits, size_t n, uint32_t *out_id) {
    if (!sp || !out_id || (n && !d_logits)) return WM_E_ARG;
    if (n > 0xffffffffull) return wm_set_error(sp->ctx, WM_E_SHAPE, "sample: %zu logits", n);
    return wm_sampler_run(sp, d_logits, (uint32_t)n, out_id);
}

wm_status wm_sampler_sample(wm_sampler *sp, const float *logits, size_t n, uint32_t *out_id) {
    if (!sp || !out_id || (n && !logits)) return WM_E_ARG;
    if (n > 0xffffffffull) return wm_set_error(sp->ctx, WM_E_SHAPE, "sample: %zu logits", n);
    wm_ctx *ctx = sp->ctx;
    void *d = nullptr;
    if (n) {
        wm_status st = wm_ctx_scratch(ctx, n * 4, &d);
        if (st) return st;
        WM_HIP(ctx, hipSetDevice(sp->device));
        WM_HIP(ctx, hipMemcpyAsync(d, logits, n * 4, hipMemcpyHostToDevice, ctx->stream));
    }
    return wm_sampler_run(sp, (const float *)d, (uint32_t)n, out_id);
}

}  // extern "C"
