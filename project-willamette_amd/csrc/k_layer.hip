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
#include "wm_norm.h"
#include "wm_seqsum.h"

namespace {

constexpr int kNormThreads = 1024;

// One workgroup: x (+ res_y, the producing matvec's f32 output, written back
// to x), then y = (x * rsqrt) * w with rsqrt = 1/sqrt(Σx²/n + eps), then
// either y -> y_out (f32, plus the lm-head's fixed-point copy when q6k_prep
// is given) or y -> per-vector absmax int8 (permuted layout) + meta.
// err_flag: set to layer_tag if x + res_y is not all finite.  clear2: two
// slots the next kernel accumulates into, zeroed here.
template <int PER, int NT>
__global__ __launch_bounds__(NT) void k_rmsnorm_quant(
    float *x, const float *__restrict__ res_y, const float *__restrict__ w, uint32_t n,
    float eps, uint8_t *__restrict__ act, wm_act_meta *__restrict__ meta_out,
    float *__restrict__ y_out, uint32_t *__restrict__ err_flag, uint32_t layer_tag,
    uint8_t *__restrict__ q6k_prep, uint32_t *__restrict__ clear2) {
    if (clear2 && threadIdx.x < 2) clear2[threadIdx.x] = 0;
    extern __shared__ __align__(16) float sq[];  // x[j]*x[j], n entries
    __shared__ wm::norm_lds<NT / 64> L;
    const uint32_t tid = threadIdx.x;
    float xv[PER], wv[PER];
    const float rs = wm::norm_rsqrt<PER, NT>(x, res_y, w, n, eps, res_y ? x : nullptr, err_flag,
                                              layer_tag, sq, L, xv, wv);
    if (y_out) {
#pragma unroll
        for (int i = 0; i < PER; i++) {
            const uint32_t j = tid + (uint32_t)i * NT;
            if (j < n) y_out[j] = xv[i] * rs * wv[i];  // out[i] = x[i] * rsqrt * weight[i]
        }
        // output_norm: also the fixed-point copy the id-only lm-head reads
        if (q6k_prep) {
            __syncthreads();  // y_out complete
            const q6k_xhdr h = q6k_xprep_block(y_out, n / Q6K_VALUES,
                                               reinterpret_cast<q6k_xq *>(q6k_prep), L.red_f, L.red_i);
            if (tid == 0) *reinterpret_cast<q6k_xhdr *>(q6k_prep + q6k_xq_bytes(n / Q6K_VALUES)) = h;
        }
        return;
    }
    float scale;
    int asum;
    wm::norm_quant<PER, NT>(rs, n, xv, wv, act, L, scale, asum);
    if (tid == 0) {
        meta_out->scale = scale;
        meta_out->asum = asum;
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

bool wm_launch_rmsnorm_quant(float *x, const float *res_y, const float *w, uint32_t n, float eps,
                             uint8_t *act, wm_act_meta *meta_out, float *y_out,
                             uint32_t *err_flag, uint32_t layer_tag, void *q6k_prep,
                             uint32_t *clear2, hipStream_t s) {
    const size_t lds = (size_t)wm::seq_sum_padded(n) * sizeof(float);
    const int per = (int)((n + kNormThreads - 1) / kNormThreads);
#define WM_NORM_CASE(P)                                                                            \
    case P:                                                                                        \
        hipLaunchKernelGGL((k_rmsnorm_quant<P, kNormThreads>), dim3(1), dim3(kNormThreads), lds, s, \
                           x, res_y, w, n, eps, act, meta_out, y_out, err_flag, layer_tag,          \
                           (uint8_t *)q6k_prep, clear2);                                            \
        return true;
    switch (per) {  // n <= 16384
        WM_NORM_CASE(1) WM_NORM_CASE(2) WM_NORM_CASE(3) WM_NORM_CASE(4)
        WM_NORM_CASE(5) WM_NORM_CASE(6) WM_NORM_CASE(7) WM_NORM_CASE(8)
        WM_NORM_CASE(9) WM_NORM_CASE(10) WM_NORM_CASE(11) WM_NORM_CASE(12)
        WM_NORM_CASE(13) WM_NORM_CASE(14) WM_NORM_CASE(15) WM_NORM_CASE(16)
        default: break;
    }
#undef WM_NORM_CASE
    return false;  // n above 16384: no instantiation
}

// KVCache::read_into (src/model/kv_cache.rs:192-219) for one layer: rows
// [0, n_pos) of K and V as f32, q as f32 * the row's scale.
__global__ __launch_bounds__(256) void k_kv_dequant(const int8_t *__restrict__ k_cache,
                                                    const float *__restrict__ k_scales,
                                                    const int8_t *__restrict__ v_cache,
                                                    const float *__restrict__ v_scales,
                                                    uint64_t n, uint32_t kv_dim,
                                                    float *__restrict__ k_out,
                                                    float *__restrict__ v_out) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t p = i / kv_dim;
        k_out[i] = (float)k_cache[i] * k_scales[p];
        v_out[i] = (float)v_cache[i] * v_scales[p];
    }
}

void wm_launch_kv_dequant(const int8_t *k_cache, const float *k_scales, const int8_t *v_cache,
                          const float *v_scales, uint32_t n_pos, uint32_t kv_dim, float *k_out,
                          float *v_out, hipStream_t s) {
    const uint64_t n = (uint64_t)n_pos * kv_dim;
    if (!n) return;
    const uint32_t blocks = (uint32_t)((n + 255) / 256 < 4096 ? (n + 255) / 256 : 4096);
    hipLaunchKernelGGL(k_kv_dequant, dim3(blocks), dim3(256), 0, s, k_cache, k_scales, v_cache,
                       v_scales, n, kv_dim, k_out, v_out);
}

void wm_launch_kv_append(const float *k, const float *v, uint32_t kv_dim, uint32_t n_layers,
                         uint32_t pos0, uint32_t n_pos, uint32_t max_seq, int8_t *k_cache,
                         float *k_scales, int8_t *v_cache, float *v_scales, hipStream_t s) {
    hipLaunchKernelGGL(k_kv_append, dim3(n_layers, n_pos), dim3(256), 0, s, k, v, kv_dim, n_layers,
                       pos0, max_seq, k_cache, k_scales, v_cache, v_scales);
}
