// Decode attention over the int8 KV cache (gfx950), in the reference's order.
//
// Reference: scaled_dot_product_attention_into
// (src/model/cached_forward.rs:417-449) on the window dequantised by
// KVCache::read_into (src/model/kv_cache.rs:192-219), softmax_inplace
// (src/model/attention.rs:45-73):
//   for each head h (kv head h / group):
//     s_p = (Σ_i q_h[i] * k_p[i]) * scale       sum over i left to right
//     w = softmax(s)                             max, exp, Σ left to right, * (1/Σ)
//     out_h[d] = Σ_p w_p * v_p[d]                sum over p left to right
//   with k_p[i] = (q8 as f32) * k_scale[p] (same for v).
//
// Every chain above is evaluated in exactly that order (the softmax
// denominator through wm::seq_sum_nonneg), so the output is bit-identical.
#include "wm_internal.h"
#include "wm_seqsum.h"

namespace {

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

// scores[h][p] = (Σ_i q_h[i] * k_p[i]) * scale.  One lane per position.
__global__ __launch_bounds__(64) void k_attn_scores(attn_args a) {
    const uint32_t h = blockIdx.x, p = blockIdx.y * 64 + threadIdx.x;
    if (p >= a.n_past) return;
    const uint32_t kvh = h / a.group;
    const float *qh = a.q + (uint64_t)h * a.head_dim;
    const int8_t *kp = a.k_cache + (uint64_t)p * a.kv_dim + kvh * a.head_dim;
    const float ksc = a.k_scales[p];
    float s = 0.0f;
    for (uint32_t i0 = 0; i0 < a.head_dim; i0 += 128) {  // head_dim is a multiple of 64
        const uint32_t nb = a.head_dim - i0 >= 128 ? 8 : 4;
        int4 raw[8];
#pragma unroll
        for (int b = 0; b < 8; b++)  // all 16-byte loads in flight together
            raw[b] = *reinterpret_cast<const int4 *>(kp + i0 + (b < (int)nb ? b : 0) * 16);
#pragma unroll
        for (int b = 0; b < 8; b++) {
            if (b < (int)nb) {
                const int8_t *kb = reinterpret_cast<const int8_t *>(&raw[b]);
#pragma unroll
                for (int t = 0; t < 16; t++) {
                    const float kd = (float)kb[t] * ksc;  // read_into: q as f32 * scale
                    s = s + qh[i0 + b * 16 + t] * kd;
                }
            }
        }
    }
    a.scores[(uint64_t)h * a.score_stride + p] = s * a.scale;
}

constexpr int kThreads = 192;   // wave 0: the 16 chains; waves 1-2: products
constexpr int kDims = 16;       // head dims per workgroup (one 16-byte V segment)
constexpr int kTile = 64;       // positions per product tile
constexpr int kPStride = 68;    // floats per dim row of a product tile

// softmax over scores[h][0..n_past) then out[h][d] = Σ_p w_p * v_p[d] for
// the 16 dimensions d0..d0+15 of head h.  Grid (n_heads, head_dim / 16).
//
// The workgroup first pulls its whole V slice (n_past x 16 int8, 64 KB at
// 4096 positions), the scores and the V scales into LDS with all loads in
// flight at once; the softmax denominator is the exact sequential sum; then
// waves 1-2 write tiles of products w_p * v_p[d] while wave 0 adds the
// previous tile, one chain per dimension.
__global__ __launch_bounds__(kThreads) void k_attn_softmax_v(attn_args a) {
    extern __shared__ __align__(16) float sm[];
    const uint32_t n = a.n_past;
    const uint32_t npad = (n + 3) & ~3u;
    float *wts = sm;                                        // [seq_sum_padded(n)]
    float *vsc = wts + wm::seq_sum_padded(n);               // [npad]
    int4 *vq = reinterpret_cast<int4 *>(vsc + npad);        // [npad] x 16 int8
    float *prod = reinterpret_cast<float *>(vq + npad);     // [2][kDims][kPStride]
    __shared__ float red[16];
    __shared__ float s_inv;
    __shared__ int s_mode;
    const uint32_t h = blockIdx.x, d0 = blockIdx.y * kDims, tid = threadIdx.x;
    const uint32_t kvh = h / a.group;
    const int8_t *vseg = a.v_cache + kvh * a.head_dim + d0;
    const float *sc = a.scores + (uint64_t)h * a.score_stride;
    __shared__ uint64_t exp_tab[32];
    if (tid < 32) exp_tab[tid] = wm::kExp2Tab[tid];
    // 1. the loads, 4 per thread per round with clamped indices so none is
    //    conditional and all 12 of a round are in flight together
    float m = -INFINITY;
    for (uint32_t base = 0; base < n; base += 4 * kThreads) {
        int4 vr[4];
        float sv[4], ss[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t p = min(base + tid + (uint32_t)i * kThreads, n - 1);
            vr[i] = *reinterpret_cast<const int4 *>(vseg + (uint64_t)p * a.kv_dim);
            sv[i] = sc[p];
            ss[i] = a.v_scales[p];
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t p = base + tid + (uint32_t)i * kThreads;
            if (p < n) {
                vq[p] = vr[i];
                wts[p] = sv[i];
                vsc[p] = ss[i];
                m = wm_max_nonan(m, sv[i]);
            }
        }
    }
    // 2. softmax (attention.rs:45-73)
    const float mx = wm_block_max_nonan(m, red);
    float *out = a.out + (uint64_t)h * a.head_dim + d0;
    if (!isfinite(mx)) {  // every weight becomes 0 -> output stays 0
        if (tid < kDims) out[tid] = 0.0f;
        return;
    }
    // exp(v - max) (attention.rs:62), 4 independent evaluations per round
    for (uint32_t base = 0; base < n; base += 4 * kThreads) {
        float e[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t p = min(base + tid + (uint32_t)i * kThreads, n - 1);
            e[i] = wm::expf_glibc(wts[p] - mx, exp_tab);
        }
        __syncthreads();  // every read of this round before any write
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t p = base + tid + (uint32_t)i * kThreads;
            if (p < n) wts[p] = e[i];
        }
    }
    __syncthreads();
    if (tid < 64) {
        const float sum = wm::seq_sum_nonneg(wts, n);
        if (tid == 0) {
            s_mode = sum > 0.0f;
            s_inv = 1.0f / sum;
        }
    }
    __syncthreads();
    if (s_mode) {
        const float inv = s_inv;
        for (uint32_t p = tid; p < n; p += kThreads) wts[p] = wts[p] * inv;
    }
    __syncthreads();
    // 3. products of tile t (waves 1-2) while wave 0 adds tile t - 1
    const uint32_t n_tiles = (n + kTile - 1) / kTile;
    const uint32_t pt = tid - 64, pl = pt >> 1, dh = (pt & 1) * 8;
    float acc = 0.0f;
    for (uint32_t t = 0; t <= n_tiles; t++) {
        if (tid >= 64) {
            if (t < n_tiles) {
                const uint32_t p = t * kTile + pl;
                float *dst = prod + (t & 1) * (kDims * kPStride) + dh * kPStride + pl;
                if (p < n) {
                    const int4 v4 = vq[p];
                    // this thread's 8 bytes, selected by register (no byte-indexed stack copy)
                    const uint32_t lo = dh ? (uint32_t)v4.z : (uint32_t)v4.x;
                    const uint32_t hi = dh ? (uint32_t)v4.w : (uint32_t)v4.y;
                    const float w = wts[p], s = vsc[p];
#pragma unroll
                    for (int i = 0; i < 8; i++) {
                        const uint32_t word = i < 4 ? lo : hi;
                        const float vd = (float)(int8_t)(word >> (8 * (i & 3))) * s;  // read_into: q * scale
                        dst[i * kPStride] = w * vd;                                    // w * v_h[d]
                    }
                }
            }
        } else if (tid < kDims && t > 0) {
            const float *src = prod + ((t - 1) & 1) * (kDims * kPStride) + tid * kPStride;
            const uint32_t p0 = (t - 1) * kTile;
            const uint32_t tn = n - p0 < (uint32_t)kTile ? n - p0 : (uint32_t)kTile;
            if (tn == (uint32_t)kTile) {
                float4 f[kTile / 4];  // the whole tile row first: one LDS latency, then the chain
#pragma unroll
                for (int i = 0; i < kTile / 4; i++) f[i] = *reinterpret_cast<const float4 *>(src + 4 * i);
#pragma unroll
                for (int i = 0; i < kTile / 4; i++) {
                    acc = acc + f[i].x; acc = acc + f[i].y; acc = acc + f[i].z; acc = acc + f[i].w;
                }
            } else {
                for (uint32_t q = 0; q < tn; q++) acc = acc + src[q];
            }
        }
        __syncthreads();
    }
    if (tid < kDims) out[tid] = acc;
}

}  // namespace

void wm_launch_attention(const float *q, const int8_t *k_cache, const float *k_scales,
                         const int8_t *v_cache, const float *v_scales, float *scores,
                         uint32_t score_stride, float *out, uint32_t n_heads, uint32_t n_kv_heads,
                         uint32_t head_dim, uint32_t n_past, float scale, hipStream_t s) {
    attn_args a{q, k_cache, k_scales, v_cache, v_scales, scores, out, n_past,
                n_kv_heads * head_dim, head_dim, n_heads / n_kv_heads, score_stride, scale};
    hipLaunchKernelGGL(k_attn_scores, dim3(n_heads, (n_past + 63) / 64), dim3(64), 0, s, a);
    const size_t npad = ((size_t)n_past + 3) & ~(size_t)3;
    const size_t lds = (size_t)wm::seq_sum_padded(n_past) * 4 + npad * (4 + 16) +
                       (size_t)2 * kDims * kPStride * 4;
    hipLaunchKernelGGL(k_attn_softmax_v, dim3(n_heads, head_dim / kDims), dim3(kThreads), lds, s, a);
}
