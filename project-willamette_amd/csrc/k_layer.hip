// Per-layer kernels of the BitNet b1.58 decode step (gfx950): the RMSNorms
// (with the residual add and the int8 quantiser fused in) and the KV prefill.
// RoPE and relu²·up run in the matvec epilogues (k_i2s.hip), attention in
// k_attn.hip.
//
// Reference: src/model/cached_forward.rs:308-502 (forward_one_layer,
// apply_ffn_block), with
//   rms_norm_f32      src/model/primitives.rs:227-255
//   KV quantisation   src/model/kv_cache.rs:245-259, dequant :192-219
//
// The reference evaluates every f32 reduction left to right in one
// accumulator.  Reproducing its results bit for bit requires the same
// order, so each such sum runs as one sequential chain here: Σx² of every
// RMSNorm, the 128-term q·k dot of every score, the softmax denominator and
// the per-dimension Σ_p w_p·v_p.  Everything around a chain (the squares, the
// products, exp, the quantisation) runs across all lanes; only the adds of
// the chain are serial.  Maxima and integer sums are order-free.
#include "wm_internal.h"
#include "wm_q6k_xprep.h"
#include "wm_seqsum.h"

namespace {

constexpr int kNormThreads = 1024;

// Residual source for k_rmsnorm_quant: y_j = (w_scale*act_scale)*(Σ_s partial[s][row0+j] - asum)
struct residual_src {
    const int32_t *partial;  // K-split i32 partials of the producing matvec, or
    uint32_t split, rows_total, row0;
    float w_scale;
    const wm_act_meta *meta;
    const float *y;  // its finished f32 output (then partial is null)
};

// One workgroup.  x[n] (optionally x += residual first, written back),
// then y = (x * rsqrt) * w with rsqrt = 1/sqrt(Σx²/n + eps), then either
// y -> y_out (f32) or y -> per-vector absmax int8 (permuted layout) + meta.
// err_flag: set to layer_tag if x (after the residual) is not all finite.
// Element-wise work uses element j = tid + i * kNormThreads (coalesced
// loads: the residual's K-split partials are the kernel's largest read, and
// one CU's L1 bandwidth bounds it); the exact sum takes the squares back
// from LDS with each thread owning consecutive terms.  Five barriers in all.
constexpr int kMaxSplit = 16;  // K splits a residual source may carry

// NT threads, values per thread: n <= PER * NT; RES: a residual source is
// given (res.partial or res.y).  Only RES kernels hold the partials'
// registers, so the others keep their register budget.
template <int PER, int NT, bool RES>
__global__ __launch_bounds__(NT) void k_rmsnorm_quant(
    float *__restrict__ x, residual_src res, const float *__restrict__ w, uint32_t n, float eps,
    uint8_t *__restrict__ act, wm_act_meta *__restrict__ meta_out, float *__restrict__ y_out,
    uint32_t *__restrict__ err_flag, uint32_t layer_tag, uint8_t *__restrict__ q6k_prep,
    uint32_t *__restrict__ clear2) {
    constexpr int NW = NT / 64;
    if (clear2 && threadIdx.x < 2) clear2[threadIdx.x] = 0;  // slots the next kernel accumulates into
    extern __shared__ __align__(16) float sq[];  // x[j]*x[j], n entries
    __shared__ float red_f[NW];
    __shared__ int red_i[NW], red_nf[NW];
    __shared__ wm::seq_block_scratch seq_scratch;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    float xv[PER], wv[PER], rv[PER];
    int nonfinite = 0;
    const bool has_res = RES;
    const bool res_vec = RES && res.y != nullptr;
    // Every load below is issued before any is used (indices clamped to
    // n - 1); out-of-range values are masked after.
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const uint32_t j = min(tid + (uint32_t)i * NT, n - 1);
        xv[i] = x[j];
        wv[i] = w[j];
        rv[i] = res_vec ? res.y[j] : 0.0f;
    }
    if (res_vec) {
        // hidden += wo_out / down as finished f32 vectors; the producing
        // kernel computed them as (w_scale * act_scale) * (float)dot, the
        // same value the partial path below forms
#pragma unroll
        for (int i = 0; i < PER; i++) {
            const uint32_t j = tid + (uint32_t)i * NT;
            const float v = xv[i] + rv[i];
            xv[i] = v;
            if (j < n) {
                x[j] = v;
                nonfinite |= !isfinite(v);
            }
        }
    } else if (has_res) {
        // hidden += wo_out / down (cached_forward.rs:405-408, :496-500)
        const float combined = res.w_scale * res.meta->scale;
        const int asum = res.meta->asum;
        const int32_t *p = res.partial + res.row0;
        int dot[PER];
        if constexpr (PER <= 4) {
            // every split's loads issued before any is used (split indices
            // clamped, the copies masked after): the partials come from other
            // XCDs' caches, and one round trip per split would serialise them
            int pv[kMaxSplit][PER];
#pragma unroll
            for (int s = 0; s < kMaxSplit; s++) {
                const uint32_t sc = min((uint32_t)s, res.split - 1);
#pragma unroll
                for (int i = 0; i < PER; i++) {
                    const uint32_t j = min(tid + (uint32_t)i * NT, n - 1);
                    pv[s][i] = p[(uint64_t)sc * res.rows_total + j];
                }
            }
#pragma unroll
            for (int i = 0; i < PER; i++) {
                dot[i] = -asum;
#pragma unroll
                for (int s = 0; s < kMaxSplit; s++) dot[i] += (uint32_t)s < res.split ? pv[s][i] : 0;
            }
        } else {  // wider vectors: not enough registers to hold every partial
#pragma unroll
            for (int i = 0; i < PER; i++) dot[i] = -asum;
#pragma unroll
            for (int s = 0; s < kMaxSplit; s++) {
                const uint32_t sc = min((uint32_t)s, res.split - 1);
#pragma unroll
                for (int i = 0; i < PER; i++) {
                    const uint32_t j = min(tid + (uint32_t)i * NT, n - 1);
                    const int v = p[(uint64_t)sc * res.rows_total + j];
                    dot[i] += (uint32_t)s < res.split ? v : 0;
                }
            }
        }
#pragma unroll
        for (int i = 0; i < PER; i++) {
            const uint32_t j = tid + (uint32_t)i * NT;
            const float v = xv[i] + combined * (float)dot[i];
            xv[i] = v;
            if (j < n) {
                x[j] = v;
                nonfinite |= !isfinite(v);
            }
        }
    }
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const uint32_t j = tid + (uint32_t)i * NT;
        if (j < n) sq[j] = xv[i] * xv[i];
        else xv[i] = 0.0f;
    }
    if (err_flag && lane == 0) red_nf[wid] = __builtin_amdgcn_ballot_w64(nonfinite != 0) != 0;
    wm_sync_lds();
    // sum_sq over x in order (primitives.rs:243-246), exactly, by the workgroup
    float v2[PER];
    {
        const uint32_t m = (n + NT - 1) / NT, k0 = tid * m;
#pragma unroll
        for (int i = 0; i < PER; i++)
            v2[i] = ((uint32_t)i < m && k0 + (uint32_t)i < n) ? sq[k0 + i] : 0.0f;
    }
    const float sum_sq = wm::seq_sum_block_owned<PER, NT>(v2, n, sq, &seq_scratch);
    if (err_flag && tid == 0) {
        int any = 0;
#pragma unroll
        for (int i = 0; i < NW; i++) any |= red_nf[i];
        if (any && *err_flag == 0) *err_flag = layer_tag;
    }
    const float mean = sum_sq / (float)n;
    const float rs = 1.0f / sqrtf(mean + eps);
    float mx = 0.0f;
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const uint32_t j = tid + (uint32_t)i * NT;
        xv[i] = xv[i] * rs * wv[i];  // out[i] = x[i] * rsqrt * weight[i]
        if (j < n) {
            if (y_out) y_out[j] = xv[i];
            mx = wm_max_nonan(mx, fabsf(xv[i]));
        }
    }
    if (y_out) {
        // output_norm: also the fixed-point copy the id-only lm-head reads
        if (q6k_prep) {
            __syncthreads();  // y_out complete
            const q6k_xhdr h = q6k_xprep_block(y_out, n / Q6K_VALUES,
                                               reinterpret_cast<q6k_xq *>(q6k_prep), red_f, red_i);
            if (tid == 0) *reinterpret_cast<q6k_xhdr *>(q6k_prep + q6k_xq_bytes(n / Q6K_VALUES)) = h;
        }
        return;
    }
    // per-vector absmax int8 (src/model/bitlinear_sse2.rs:285-304)
    mx = wm_wave_max_nonneg(mx);
    if (lane == 0) red_f[wid] = mx;
    wm_sync_lds();
    float max_abs = red_f[0];
#pragma unroll
    for (int i = 1; i < NW; i++) max_abs = wm_max_nonan(max_abs, red_f[i]);
    int sum = 0;
    const float inv = 127.0f / max_abs;
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const uint32_t j = tid + (uint32_t)i * NT;
        if (j < n) {
            const int q = max_abs == 0.0f ? 0 : wm_round_clamp_i8(xv[i] * inv);
            act[wm_act_perm(j)] = (uint8_t)(int8_t)q;
            sum += q;
        }
    }
    sum = wm_wave_total_i32(sum);
    if (lane == 0) red_i[wid] = sum;
    wm_sync_lds();
    if (tid == 0) {
        int t = 0;
#pragma unroll
        for (int i = 0; i < NW; i++) t += red_i[i];
        meta_out->scale = max_abs == 0.0f ? 1.0f : max_abs / 127.0f;
        meta_out->asum = t;
    }
}

// KVCache::append for n_pos positions x n_layers (prefill from host f32).
// Grid (n_layers, n_pos); k/v are [pos][layer][kv_dim].
__global__ __launch_bounds__(256) void k_kv_append(const float *__restrict__ k,
                                                   const float *__restrict__ v, uint32_t kv_dim,
                                                   uint32_t n_layers, uint32_t pos0,
                                                   uint32_t max_seq, int8_t *k_cache,
                                                   float *k_scales, int8_t *v_cache,
                                                   float *v_scales) {
    __shared__ float red[16];
    const uint32_t l = blockIdx.x, p = blockIdx.y;
    const uint64_t src = ((uint64_t)p * n_layers + l) * kv_dim;
    const uint64_t dst = ((uint64_t)l * max_seq + pos0 + p);
    wm_kv_quantise_store(k + src, kv_dim, k_cache + dst * kv_dim, k_scales + dst, red);
    wm_sync_lds();
    wm_kv_quantise_store(v + src, kv_dim, v_cache + dst * kv_dim, v_scales + dst, red);
}

// Test hook: terms that fit in LDS (as every caller holds them) are summed
// by the workgroup algorithm, longer arrays by the one-wave algorithm straight
// from global memory.
constexpr uint32_t kDebugSeqLds = 32768;
__global__ __launch_bounds__(1024) void k_debug_seq_sum(const float *__restrict__ a, uint32_t n,
                                                        float *__restrict__ out) {
    extern __shared__ __align__(16) float terms[];
    __shared__ wm::seq_block_scratch scratch;
    constexpr int M = kDebugSeqLds / 1024;
    if (n <= kDebugSeqLds) {
        const uint32_t m = (n + 1023) / 1024, k0 = threadIdx.x * m;
        float v[M];
#pragma unroll
        for (int j = 0; j < M; j++) {
            const uint32_t k = k0 + (uint32_t)j;
            v[j] = ((uint32_t)j < m && k < n) ? a[k] : 0.0f;
            if ((uint32_t)j < m && k < n) terms[k] = v[j];
        }
        const float s = wm::seq_sum_block_owned<M, 1024>(v, n, terms, &scratch);
        if (threadIdx.x == 0) *out = s;
    } else if (threadIdx.x < 64) {
        const float s = wm::seq_sum_nonneg(a, n);
        if (threadIdx.x == 0) *out = s;
    }
}

}  // namespace

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------

void wm_launch_debug_seq_sum(const float *a, uint32_t n, float *out, hipStream_t s) {
    const size_t lds = n <= kDebugSeqLds ? (size_t)n * sizeof(float) : 0;
    hipLaunchKernelGGL(k_debug_seq_sum, dim3(1), dim3(1024), lds, s, a, n, out);
}

void wm_launch_rmsnorm_quant(float *x, const int32_t *partial, uint32_t split, uint32_t rows_total,
                             uint32_t row0, float w_scale, const wm_act_meta *meta_in,
                             const float *res_y, const float *w, uint32_t n, float eps,
                             uint8_t *act, wm_act_meta *meta_out, float *y_out,
                             uint32_t *err_flag, uint32_t layer_tag, void *q6k_prep,
                             uint32_t *clear2, hipStream_t s) {
    residual_src res{partial, split, rows_total, row0, w_scale, meta_in, res_y};
    size_t lds = (size_t)wm::seq_sum_padded(n) * sizeof(float);
    const int per = (int)((n + kNormThreads - 1) / kNormThreads);
#define WM_NORM_CASE(P, R)                                                                         \
    hipLaunchKernelGGL((k_rmsnorm_quant<P, kNormThreads, R>), dim3(1), dim3(kNormThreads), lds, s,  \
                       x, res, w, n, eps, act, meta_out, y_out, err_flag, layer_tag,                \
                       (uint8_t *)q6k_prep, clear2)
    if (partial || res_y) {
        switch (per) {  // residual sources: the hidden state, n_embd <= 8192
            case 1: WM_NORM_CASE(1, true); break;
            case 2: WM_NORM_CASE(2, true); break;
            case 3: WM_NORM_CASE(3, true); break;
            case 4: WM_NORM_CASE(4, true); break;
            case 5: WM_NORM_CASE(5, true); break;
            case 6: WM_NORM_CASE(6, true); break;
            case 7: WM_NORM_CASE(7, true); break;
            case 8: WM_NORM_CASE(8, true); break;
            default: break;
        }
        return;
    }
    switch (per) {
        case 1: WM_NORM_CASE(1, false); break;
        case 2: WM_NORM_CASE(2, false); break;
        case 3: WM_NORM_CASE(3, false); break;
        case 4: WM_NORM_CASE(4, false); break;
        case 5: WM_NORM_CASE(5, false); break;
        case 6: WM_NORM_CASE(6, false); break;
        case 7: WM_NORM_CASE(7, false); break;
        case 8: WM_NORM_CASE(8, false); break;
        case 9: WM_NORM_CASE(9, false); break;
        case 10: WM_NORM_CASE(10, false); break;
        case 11: WM_NORM_CASE(11, false); break;
        case 12: WM_NORM_CASE(12, false); break;
        case 13: WM_NORM_CASE(13, false); break;
        case 14: WM_NORM_CASE(14, false); break;
        case 15: WM_NORM_CASE(15, false); break;
        case 16: WM_NORM_CASE(16, false); break;
        default: break;
    }
#undef WM_NORM_CASE
}

void wm_launch_kv_append(const float *k, const float *v, uint32_t kv_dim, uint32_t n_layers,
                         uint32_t pos0, uint32_t n_pos, uint32_t max_seq, int8_t *k_cache,
                         float *k_scales, int8_t *v_cache, float *v_scales, hipStream_t s) {
    hipLaunchKernelGGL(k_kv_append, dim3(n_layers, n_pos), dim3(256), 0, s, k, v, kv_dim, n_layers,
                       pos0, max_seq, k_cache, k_scales, v_cache, v_scales);
}
