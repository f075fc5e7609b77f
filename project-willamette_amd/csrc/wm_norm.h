// RMSNorm with the residual add and the absmax int8 quantiser, as workgroup
// device functions (gfx950).  The stand-alone norm kernel (k_layer.hip) and
// the matvecs that start from their input's norm (k_i2s.hip) share them, so
// every copy of a norm evaluates the same operations in the same order.
//
// Reference: rms_norm_f32 (src/model/primitives.rs:227-255),
// quantize_input_absmax_i8 (src/model/bitlinear_sse2.rs:285-304), the
// residual adds of forward_one_layer (src/model/cached_forward.rs:405-408,
// :496-500).
#pragma once

#include "wm_internal.h"
#include "wm_seqsum.h"

namespace wm {

// The LDS a norm needs besides the squares (seq_sum_padded(n) floats, which
// the caller provides): NW = threads / 64.
template <int NW>
struct norm_lds {
    seq_block_scratch seq;
    float red_f[NW];
    int red_i[NW], red_nf[NW];
};

// The loads of a norm: element j = t + i*NT of x, of the weight and of y
// (the producing matvec's f32 output, nullable) into xv, wv, rv.  A caller
// with other loads to issue puts these first, so that waiting for them
// waits for nothing else.
template <int PER, int NT>
__device__ __forceinline__ void norm_load(const float *x, const float *__restrict__ y,
                                          const float *__restrict__ w, uint32_t n,
                                          float (&xv)[PER], float (&wv)[PER], float (&rv)[PER]) {
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const uint32_t j = min(threadIdx.x + (uint32_t)i * NT, n - 1);
        xv[i] = x[j];
        wv[i] = w[j];
        rv[i] = y ? y[j] : 0.0f;
    }
}

// From the loaded values: x + y (hidden += the producing matvec's output,
// when has_y; with relu2, relu(x)^2 * y: the FFN's gate x and up y,
// ffn.rs:37-65), written back to x_out when given, and the squares into sq.
// Thread t then holds element j = t + i*NT in xv[i] and its weight in wv[i]
// (0 past n).  Returns whether any of its x + y is not finite.
template <int PER, int NT>
__device__ __forceinline__ bool norm_prep(bool has_y, uint32_t n, float *x_out, float *sq,
                                          float (&xv)[PER], float (&wv)[PER],
                                          const float (&rv)[PER], bool relu2 = false) {
    const uint32_t tid = threadIdx.x;
    int nonfinite = 0;
    if (has_y) {
#pragma unroll
        for (int i = 0; i < PER; i++) {
            const uint32_t j = tid + (uint32_t)i * NT;
            const float r = xv[i] > 0.0f ? xv[i] : 0.0f;
            const float v = relu2 ? (r * r) * rv[i] : xv[i] + rv[i];
            xv[i] = v;
            if (j < n) {
                if (x_out) x_out[j] = v;
                nonfinite |= !isfinite(v);
            }
        }
    }
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const uint32_t j = tid + (uint32_t)i * NT;
        if (j < n) {
            sq[j] = xv[i] * xv[i];
        } else {
            xv[i] = 0.0f;
            wv[i] = 0.0f;
        }
    }
    return nonfinite != 0;
}

// After norm_prep: Σx² exactly, in order (primitives.rs:243-246); returns
// 1/sqrt(Σx²/n + eps).  before_walk: see seq_sum_block_owned.  err_flag (nullable): set to layer_tag when some
// thread's x + y was not finite and the flag is still clear.
template <int PER, int NT, typename Hook = seq_no_hook>
__device__ __forceinline__ float norm_sum_rsqrt(bool nonfinite, uint32_t n, float eps,
                                                uint32_t *err_flag, uint32_t layer_tag,
                                                float *sq, norm_lds<NT / 64> &L,
                                                const Hook &before_walk = Hook()) {
    constexpr int NW = NT / 64;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    if (err_flag && lane == 0) L.red_nf[wid] = __builtin_amdgcn_ballot_w64(nonfinite) != 0;
    wm_sync_lds();
    float v2[PER];
    {
        const uint32_t m = (n + NT - 1) / NT, k0 = tid * m;
#pragma unroll
        for (int i = 0; i < PER; i++)
            v2[i] = ((uint32_t)i < m && k0 + (uint32_t)i < n) ? sq[k0 + i] : 0.0f;
    }
    const float sum_sq = seq_sum_block_owned<PER, NT>(v2, n, sq, &L.seq, before_walk);
    if (err_flag && tid == 0) {
        int any = 0;
#pragma unroll
        for (int i = 0; i < NW; i++) any |= L.red_nf[i];
        if (any && *err_flag == 0) *err_flag = layer_tag;
    }
    const float mean = sum_sq / (float)n;
    return 1.0f / sqrtf(mean + eps);
}

// norm_load, norm_prep and norm_sum_rsqrt in one (x may be x_out itself:
// every load is issued before any store).
template <int PER, int NT>
__device__ __forceinline__ float norm_rsqrt(const float *x, const float *__restrict__ y,
                                            const float *__restrict__ w, uint32_t n, float eps,
                                            float *x_out, uint32_t *err_flag, uint32_t layer_tag,
                                            float *sq, norm_lds<NT / 64> &L, float (&xv)[PER],
                                            float (&wv)[PER]) {
    float rv[PER];
    norm_load<PER, NT>(x, y, w, n, xv, wv, rv);
    const bool nf = norm_prep<PER, NT>(y != nullptr, n, x_out, sq, xv, wv, rv);
    return norm_sum_rsqrt<PER, NT>(nf, n, eps, err_flag, layer_tag, sq, L);
}

// y = x * rsqrt * w (primitives.rs:249-252) into xv, then the absmax int8
// quantiser: the int8 codes to act[wm_act_perm(j)] (LDS or global memory),
// and to every thread the act scale (max_abs / 127, 1 for an all-zero
// vector) and Σq.  Ends with a barrier, so act is complete on return.
template <int PER, int NT>
__device__ __forceinline__ void norm_quant(float rsqrt_, uint32_t n, float (&xv)[PER],
                                           const float (&wv)[PER], uint8_t *act,
                                           norm_lds<NT / 64> &L, float &scale, int &asum) {
    constexpr int NW = NT / 64;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    float mx = 0.0f;
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const uint32_t j = tid + (uint32_t)i * NT;
        xv[i] = xv[i] * rsqrt_ * wv[i];  // out[i] = x[i] * rsqrt * weight[i]
        if (j < n) mx = wm_max_nonan(mx, fabsf(xv[i]));
    }
    mx = wm_wave_max_nonneg(mx);
    if (lane == 0) L.red_f[wid] = mx;
    wm_sync_lds();
    float max_abs = L.red_f[0];
#pragma unroll
    for (int i = 1; i < NW; i++) max_abs = wm_max_nonan(max_abs, L.red_f[i]);
    int sum = 0;
    const float inv = 127.0f / max_abs;
    // with NT a multiple of 128, element tid + i*NT sits at perm(tid) + i*NT
    const uint32_t pb = wm_act_perm(tid);
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const uint32_t j = tid + (uint32_t)i * NT;
        if (j < n) {
            const int q = max_abs == 0.0f ? 0 : wm_round_clamp_i8_fast(xv[i] * inv);
            act[NT % 128 == 0 ? pb + (uint32_t)i * NT : wm_act_perm(j)] = (uint8_t)(int8_t)q;
            sum += q;
        }
    }
    sum = wm_wave_total_i32(sum);
    if (lane == 0) L.red_i[wid] = sum;
    wm_sync_lds();
    int t = 0;
#pragma unroll
    for (int i = 0; i < NW; i++) t += L.red_i[i];
    scale = max_abs == 0.0f ? 1.0f : max_abs / 127.0f;
    asum = t;
}

}  // namespace wm
