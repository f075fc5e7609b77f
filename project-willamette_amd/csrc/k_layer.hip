// Per-layer kernels of the BitNet b1.58 decode step (gfx950).
//
// Reference: src/model/cached_forward.rs:308-502 (forward_one_layer,
// scaled_dot_product_attention_into, apply_ffn_block), with
//   rms_norm_f32      src/model/primitives.rs:227-255
//   RoPE (NEOX)       src/model/primitives.rs:285-345
//   softmax_inplace   src/model/attention.rs:45-73
//   KV quantisation   src/model/kv_cache.rs:245-259, dequant :192-219
//   relu_square, mul  src/model/ffn.rs:37-65
//
// The reference evaluates every f32 reduction left to right in one
// accumulator.  Reproducing its results bit for bit requires the same
// order, so each such sum runs as one sequential chain here: Σx² of every
// RMSNorm, the 128-term q·k dot of every score, the softmax denominator and
// the per-dimension Σ_p w_p·v_p.  Everything around a chain (the squares, the
// products, exp, the quantisation) runs across all lanes; only the adds of
// the chain are serial.  Maxima and integer sums are order-free.
#include "wm_internal.h"

namespace {

constexpr int kNormThreads = 1024;

// Sequential f32 sum of x[i]*x[i], i = 0..n-1, one accumulator, as
// `for &xi in x { sum_sq += xi * xi }`.  Executed by every lane of the
// calling wave on the same LDS data (broadcast reads), so the value is
// uniform; the multiplies do not depend on the accumulator and issue ahead.
__device__ __forceinline__ float seq_sum_squares(const float *__restrict__ xs, uint32_t n) {
    float s = 0.0f;
    uint32_t i = 0;
    for (; i + 8 <= n; i += 8) {
        float4 a = *reinterpret_cast<const float4 *>(xs + i);
        float4 b = *reinterpret_cast<const float4 *>(xs + i + 4);
        float p0 = a.x * a.x, p1 = a.y * a.y, p2 = a.z * a.z, p3 = a.w * a.w;
        float p4 = b.x * b.x, p5 = b.y * b.y, p6 = b.z * b.z, p7 = b.w * b.w;
        s = s + p0; s = s + p1; s = s + p2; s = s + p3;
        s = s + p4; s = s + p5; s = s + p6; s = s + p7;
    }
    for (; i < n; i++) s = s + xs[i] * xs[i];
    return s;
}

__device__ __forceinline__ float block_max_nonan(float v, float *red) {
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    v = wm_wave_max_nonan(v);
    __syncthreads();
    if (lane == 0) red[wid] = v;
    __syncthreads();
    float m = red[0];
    for (int w = 1; w < (int)(blockDim.x >> 6); w++) m = wm_max_nonan(m, red[w]);
    return m;
}

__device__ __forceinline__ int block_sum_i32(int v, int *red) {
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    v = wm_wave_sum_i32(v);
    __syncthreads();
    if (lane == 0) red[wid] = v;
    __syncthreads();
    int t = 0;
    for (int w = 0; w < (int)(blockDim.x >> 6); w++) t += red[w];
    return t;
}

// Residual source for k_rmsnorm_quant: y_j = (w_scale*act_scale)*(Σ_s partial[s][row0+j] - asum)
struct residual_src {
    const int32_t *partial;
    uint32_t split, rows_total, row0;
    float w_scale;
    const wm_act_meta *meta;
};

// One workgroup.  x[n] (optionally x += residual first, written back),
// then y = (x * rsqrt) * w with rsqrt = 1/sqrt(Σx²/n + eps), then either
// y -> y_out (f32) or y -> per-vector absmax int8 (permuted layout) + meta.
// err_flag: set to layer_tag if x (after the residual) is not all finite.
__global__ __launch_bounds__(kNormThreads) void k_rmsnorm_quant(
    float *__restrict__ x, residual_src res, const float *__restrict__ w, uint32_t n, float eps,
    uint8_t *__restrict__ act, wm_act_meta *__restrict__ meta_out, float *__restrict__ y_out,
    uint32_t *__restrict__ err_flag, uint32_t layer_tag) {
    extern __shared__ float xs[];
    __shared__ float red_f[16];
    __shared__ int red_i[16];
    __shared__ float s_rsqrt;
    const uint32_t tid = threadIdx.x;
    int nonfinite = 0;
    if (res.partial) {
        const float combined = res.w_scale * res.meta->scale;
        const int asum = res.meta->asum;
        for (uint32_t j = tid; j < n; j += blockDim.x) {
            int dot = -asum;
            for (uint32_t s = 0; s < res.split; s++)
                dot += res.partial[(uint64_t)s * res.rows_total + res.row0 + j];
            float v = x[j] + combined * (float)dot;
            x[j] = v;
            xs[j] = v;
            nonfinite |= !isfinite(v);
        }
    } else {
        for (uint32_t j = tid; j < n; j += blockDim.x) xs[j] = x[j];
    }
    if (err_flag) {
        int any = block_sum_i32(nonfinite, red_i);
        if (any && tid == 0 && *err_flag == 0) *err_flag = layer_tag;
    }
    __syncthreads();
    if (tid < 64) {
        float sum_sq = seq_sum_squares(xs, n);
        if (tid == 0) {
            float mean = sum_sq / (float)n;
            s_rsqrt = 1.0f / sqrtf(mean + eps);
        }
    }
    __syncthreads();
    const float rs = s_rsqrt;
    if (y_out) {
        for (uint32_t j = tid; j < n; j += blockDim.x) y_out[j] = xs[j] * rs * w[j];
        return;
    }
    // per-vector absmax int8 (src/model/bitlinear_sse2.rs:285-304)
    float m = 0.0f;
    for (uint32_t j = tid; j < n; j += blockDim.x) m = wm_max_nonan(m, fabsf(xs[j] * rs * w[j]));
    const float max_abs = block_max_nonan(m, red_f);
    int sum = 0;
    if (max_abs == 0.0f) {
        for (uint32_t j = tid; j < n; j += blockDim.x) act[wm_act_perm(j)] = 0;
    } else {
        const float inv = 127.0f / max_abs;
        for (uint32_t j = tid; j < n; j += blockDim.x) {
            int q = wm_round_clamp_i8((xs[j] * rs * w[j]) * inv);
            act[wm_act_perm(j)] = (uint8_t)(int8_t)q;
            sum += q;
        }
    }
    sum = block_sum_i32(sum, red_i);
    if (tid == 0) {
        meta_out->scale = max_abs == 0.0f ? 1.0f : max_abs / 127.0f;
        meta_out->asum = sum;
    }
}

// KV quantisation of one token vector in LDS (src/model/kv_cache.rs:245-259):
// absmax (NaN never raises it), zero/non-finite absmax -> zeros + scale 0.
__device__ void kv_quantise_store(const float *__restrict__ v, uint32_t n, int8_t *__restrict__ q,
                                  float *__restrict__ scale_out, float *red) {
    float m = 0.0f;
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) m = wm_max_nonan(m, fabsf(v[i]));
    const float absmax = block_max_nonan(m, red);
    if (absmax == 0.0f || !isfinite(absmax)) {
        for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) q[i] = 0;
        if (threadIdx.x == 0) *scale_out = 0.0f;
        return;
    }
    const float inv = 127.0f / absmax;
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) q[i] = (int8_t)wm_round_clamp_i8(v[i] * inv);
    if (threadIdx.x == 0) *scale_out = absmax / 127.0f;
}

struct qkv_args {
    const int32_t *partial;
    uint32_t split, rows_total;
    uint32_t q_row0, k_row0, v_row0;
    uint32_t n_q, n_kv;  // n_embd, kv_dim
    float q_scale, k_scale, v_scale;
    const wm_act_meta *meta;
    const float *rope_cos, *rope_sin;  // [pos][n_rot/2]
    uint32_t head_dim, n_rot, pos;
    float *q_out;
    int8_t *k_cache, *v_cache;  // this layer, this position
    float *k_scale_out, *v_scale_out;
};

// QKV epilogue (one workgroup): finalise the three BitLinear outputs, apply
// NEOX RoPE to Q and K at `pos`, write Q (f32) and append the quantised K,V
// to the cache.
__global__ __launch_bounds__(1024) void k_qkv_rope_kv(qkv_args a) {
    extern __shared__ float sm[];
    float *qs = sm, *ks = sm + a.n_q, *vs = ks + a.n_kv;
    __shared__ float red[16];
    const float in_scale = a.meta->scale;
    const int asum = a.meta->asum;
    const uint32_t total = a.n_q + 2 * a.n_kv;
    for (uint32_t i = threadIdx.x; i < total; i += blockDim.x) {
        uint32_t row;
        float ws;
        if (i < a.n_q) { row = a.q_row0 + i; ws = a.q_scale; }
        else if (i < a.n_q + a.n_kv) { row = a.k_row0 + (i - a.n_q); ws = a.k_scale; }
        else { row = a.v_row0 + (i - a.n_q - a.n_kv); ws = a.v_scale; }
        int dot = -asum;
        for (uint32_t s = 0; s < a.split; s++) dot += a.partial[(uint64_t)s * a.rows_total + row];
        sm[i] = (ws * in_scale) * (float)dot;
    }
    __syncthreads();
    // RoPE pairs (j, j + n_rot/2) in every head of Q and K
    const uint32_t half = a.n_rot / 2;
    const float *cs = a.rope_cos + (uint64_t)a.pos * half, *sn = a.rope_sin + (uint64_t)a.pos * half;
    const uint32_t n_pairs_q = (a.n_q / a.head_dim) * half, n_pairs_k = (a.n_kv / a.head_dim) * half;
    for (uint32_t p = threadIdx.x; p < n_pairs_q + n_pairs_k; p += blockDim.x) {
        float *base = p < n_pairs_q ? qs : ks;
        uint32_t pp = p < n_pairs_q ? p : p - n_pairs_q;
        uint32_t h = pp / half, j = pp % half;
        float *xh = base + h * a.head_dim;
        float c = cs[j], s = sn[j];
        float x0 = xh[j], x1 = xh[j + half];
        xh[j] = x0 * c - x1 * s;
        xh[j + half] = x0 * s + x1 * c;
    }
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < a.n_q; i += blockDim.x) a.q_out[i] = qs[i];
    kv_quantise_store(ks, a.n_kv, a.k_cache, a.k_scale_out, red);
    __syncthreads();
    kv_quantise_store(vs, a.n_kv, a.v_cache, a.v_scale_out, red);
}

struct attn_args {
    const float *q;          // [n_heads][head_dim]
    const int8_t *k_cache;   // this layer: [max_seq][kv_dim]
    const float *k_scales;   // [max_seq]
    const int8_t *v_cache;
    const float *v_scales;
    float *scores;           // [n_heads][score_stride]
    float *out;              // [n_heads][head_dim]
    uint32_t n_past, kv_dim, head_dim, group, score_stride;
    float scale;
};

// scores[h][p] = (Σ_i q_h[i] * k_p[i]) * scale, the sum sequential over i
// (cached_forward.rs:425-431); k_p[i] = (q8 as f32) * k_scale[p]
// (kv_cache.rs:213-215).  One lane per position.
__global__ __launch_bounds__(64) void k_attn_scores(attn_args a) {
    const uint32_t h = blockIdx.x, p = blockIdx.y * 64 + threadIdx.x;
    if (p >= a.n_past) return;
    const uint32_t kvh = h / a.group;
    const float *qh = a.q + (uint64_t)h * a.head_dim;
    const int8_t *kp = a.k_cache + (uint64_t)p * a.kv_dim + kvh * a.head_dim;
    const float ksc = a.k_scales[p];
    float s = 0.0f;
    for (uint32_t i = 0; i < a.head_dim; i += 16) {
        int4 raw = *reinterpret_cast<const int4 *>(kp + i);
        const int8_t *b = reinterpret_cast<const int8_t *>(&raw);
#pragma unroll
        for (int t = 0; t < 16; t++) {
            float kd = (float)b[t] * ksc;
            s = s + qh[i + t] * kd;
        }
    }
    a.scores[(uint64_t)h * a.score_stride + p] = s * a.scale;
}

constexpr int kAttnThreads = 256;
constexpr int kAttnTile = 128;  // positions per product tile
constexpr int kAttnDims = 64;   // head dims per workgroup

// softmax over scores[h][0..n_past) (attention.rs:45-73) then
// out[h][d] = Σ_p w_p * v_p[d], sequential over p (cached_forward.rs:440-447),
// for the 64 dimensions d0..d0+63 of head h.  Grid (n_heads, head_dim/64).
__global__ __launch_bounds__(kAttnThreads) void k_attn_softmax_v(attn_args a) {
    extern __shared__ float sm[];
    float *wts = sm;                         // [n_past]
    float *prod = sm + ((a.n_past + 3) & ~3u);  // [kAttnTile][kAttnDims]
    __shared__ float red[16];
    __shared__ float s_inv;
    __shared__ int s_mode;
    const uint32_t h = blockIdx.x, d0 = blockIdx.y * kAttnDims, tid = threadIdx.x;
    const uint32_t n = a.n_past;
    const float *sc = a.scores + (uint64_t)h * a.score_stride;
    float m = -INFINITY;
    for (uint32_t p = tid; p < n; p += blockDim.x) {
        float v = sc[p];
        wts[p] = v;
        m = wm_max_nonan(m, v);
    }
    const float mx = block_max_nonan(m, red);
    float *out = a.out + (uint64_t)h * a.head_dim + d0;
    if (!isfinite(mx)) {  // every weight becomes 0 -> output stays 0
        for (uint32_t d = tid; d < kAttnDims; d += blockDim.x) out[d] = 0.0f;
        return;
    }
    for (uint32_t p = tid; p < n; p += blockDim.x) wts[p] = wm_expf(wts[p] - mx);
    __syncthreads();
    if (tid < 64) {
        float sum = 0.0f;
        uint32_t p = 0;
        for (; p + 4 <= n; p += 4) {
            float4 e = *reinterpret_cast<const float4 *>(wts + p);
            sum = sum + e.x; sum = sum + e.y; sum = sum + e.z; sum = sum + e.w;
        }
        for (; p < n; p++) sum = sum + wts[p];
        if (tid == 0) {
            s_mode = sum > 0.0f;
            s_inv = 1.0f / sum;
        }
    }
    __syncthreads();
    if (s_mode) {
        const float inv = s_inv;
        for (uint32_t p = tid; p < n; p += blockDim.x) wts[p] = wts[p] * inv;
    }
    __syncthreads();
    const uint32_t kvh = h / a.group;
    const int8_t *vbase = a.v_cache + kvh * a.head_dim + d0;
    float acc = 0.0f;  // lane d of wave 0
    for (uint32_t t0 = 0; t0 < n; t0 += kAttnTile) {
        const uint32_t tn = n - t0 < (uint32_t)kAttnTile ? n - t0 : (uint32_t)kAttnTile;
        for (uint32_t idx = tid; idx < tn * kAttnDims; idx += blockDim.x) {
            uint32_t pl = idx / kAttnDims, d = idx % kAttnDims, p = t0 + pl;
            float vd = (float)vbase[(uint64_t)p * a.kv_dim + d] * a.v_scales[p];
            prod[pl * kAttnDims + d] = wts[p] * vd;
        }
        __syncthreads();
        if (tid < kAttnDims)
            for (uint32_t pl = 0; pl < tn; pl++) acc = acc + prod[pl * kAttnDims + tid];
        __syncthreads();
    }
    if (tid < kAttnDims) out[tid] = acc;
}

// relu(g)^2 * u over the gate/up BitLinear outputs (ffn.rs:37-65).
__global__ void k_gateup_relu2(const int32_t *__restrict__ partial, uint32_t split,
                               uint32_t rows_total, uint32_t gate_row0, uint32_t up_row0,
                               uint32_t n_ff, float gate_scale, float up_scale,
                               const wm_act_meta *__restrict__ meta, float *__restrict__ h) {
    const uint32_t j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= n_ff) return;
    const int asum = meta->asum;
    int dg = -asum, du = -asum;
    for (uint32_t s = 0; s < split; s++) {
        dg += partial[(uint64_t)s * rows_total + gate_row0 + j];
        du += partial[(uint64_t)s * rows_total + up_row0 + j];
    }
    const float g = (gate_scale * meta->scale) * (float)dg;
    const float u = (up_scale * meta->scale) * (float)du;
    const float r = g > 0.0f ? g : 0.0f;
    h[j] = (r * r) * u;
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
    kv_quantise_store(k + src, kv_dim, k_cache + dst * kv_dim, k_scales + dst, red);
    __syncthreads();
    kv_quantise_store(v + src, kv_dim, v_cache + dst * kv_dim, v_scales + dst, red);
}

}  // namespace

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------

void wm_launch_rmsnorm_quant(float *x, const int32_t *partial, uint32_t split, uint32_t rows_total,
                             uint32_t row0, float w_scale, const wm_act_meta *meta_in,
                             const float *w, uint32_t n, float eps, uint8_t *act,
                             wm_act_meta *meta_out, float *y_out, uint32_t *err_flag,
                             uint32_t layer_tag, hipStream_t s) {
    residual_src res{partial, split, rows_total, row0, w_scale, meta_in};
    size_t lds = ((size_t)n + 8) * sizeof(float);
    hipLaunchKernelGGL(k_rmsnorm_quant, dim3(1), dim3(kNormThreads), lds, s, x, res, w, n, eps, act,
                       meta_out, y_out, err_flag, layer_tag);
}

void wm_launch_qkv_rope_kv(const int32_t *partial, uint32_t split, uint32_t rows_total,
                           uint32_t q_row0, uint32_t k_row0, uint32_t v_row0, uint32_t n_q,
                           uint32_t n_kv, float q_scale, float k_scale, float v_scale,
                           const wm_act_meta *meta, const float *rope_cos, const float *rope_sin,
                           uint32_t head_dim, uint32_t n_rot, uint32_t pos, float *q_out,
                           int8_t *k_cache, int8_t *v_cache, float *k_scale_out,
                           float *v_scale_out, hipStream_t s) {
    qkv_args a{partial, split, rows_total, q_row0, k_row0, v_row0, n_q, n_kv, q_scale, k_scale,
               v_scale, meta, rope_cos, rope_sin, head_dim, n_rot, pos, q_out, k_cache, v_cache,
               k_scale_out, v_scale_out};
    size_t lds = (size_t)(n_q + 2 * n_kv) * sizeof(float);
    hipLaunchKernelGGL(k_qkv_rope_kv, dim3(1), dim3(1024), lds, s, a);
}

void wm_launch_attention(const float *q, const int8_t *k_cache, const float *k_scales,
                         const int8_t *v_cache, const float *v_scales, float *scores,
                         uint32_t score_stride, float *out, uint32_t n_heads, uint32_t n_kv_heads,
                         uint32_t head_dim, uint32_t n_past, float scale, hipStream_t s) {
    attn_args a{q, k_cache, k_scales, v_cache, v_scales, scores, out, n_past,
                n_kv_heads * head_dim, head_dim, n_heads / n_kv_heads, score_stride, scale};
    hipLaunchKernelGGL(k_attn_scores, dim3(n_heads, (n_past + 63) / 64), dim3(64), 0, s, a);
    size_t lds = (((size_t)n_past + 3) & ~(size_t)3) * 4 + (size_t)kAttnTile * kAttnDims * 4;
    hipLaunchKernelGGL(k_attn_softmax_v, dim3(n_heads, head_dim / kAttnDims), dim3(kAttnThreads), lds,
                       s, a);
}

void wm_launch_gateup_relu2(const int32_t *partial, uint32_t split, uint32_t rows_total,
                            uint32_t gate_row0, uint32_t up_row0, uint32_t n_ff, float gate_scale,
                            float up_scale, const wm_act_meta *meta, float *h, hipStream_t s) {
    hipLaunchKernelGGL(k_gateup_relu2, dim3((n_ff + 255) / 256), dim3(256), 0, s, partial, split,
                       rows_total, gate_row0, up_row0, n_ff, gate_scale, up_scale, meta, h);
}

void wm_launch_kv_append(const float *k, const float *v, uint32_t kv_dim, uint32_t n_layers,
                         uint32_t pos0, uint32_t n_pos, uint32_t max_seq, int8_t *k_cache,
                         float *k_scales, int8_t *v_cache, float *v_scales, hipStream_t s) {
    hipLaunchKernelGGL(k_kv_append, dim3(n_layers, n_pos), dim3(256), 0, s, k, v, kv_dim, n_layers,
                       pos0, max_seq, k_cache, k_scales, v_cache, v_scales);
}
