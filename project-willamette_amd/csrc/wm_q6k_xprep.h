// Fixed-point copy of the hidden vector for the id-only Q6_K lm-head, shared
// by the lm-head kernels and the output-norm kernel that produces the vector.
#pragma once

#include "wm_internal.h"

// The hidden vector as 16-bit fixed point, x_i ~ 2^e * X_i with
// X_i = rint(x_i * 2^-e), |X_i| <= 32639, split X = 256*xh + xl into two int8
// (xh = (X + 128) >> 8, xl = X - 256*xh in [-128, 127]).  Entry (b, p) holds,
// for lane position p = 4k + l of block b and group hn, the four values that
// meet byte c of that lane's U[hn]: xh and xl packed as int8x4 and
// c[hn] = -32 * sum_c X (which folds the quants' offset of 32 into the dot).
struct alignas(16) q6k_xq {
    int xh[4], xl[4], c[4];
};
struct q6k_xhdr {
    int e;          // scale exponent
    uint32_t ok;    // 0: the hidden vector holds a NaN or an infinity
    float bound_k;  // row bound = bound_k * sigma_r, sigma_r = sum_j |d * sc_j|
    float mag_k;    // row magnitude bound factor (overflow guard)
};

// The prep area: xq[n_blocks*16] then, 256 bytes aligned, the header.
__host__ __device__ inline size_t q6k_xq_bytes(uint32_t n_blocks) {
    return ((size_t)n_blocks * 16 * 48 + 255) & ~(size_t)255;
}
__host__ __device__ inline size_t q6k_prep_bytes(uint32_t n_blocks) {
    return q6k_xq_bytes(n_blocks) + 256;
}

// Build the fixed-point copy of hidden[n_blocks*256] (xq[n_blocks*16], any
// address space) and return the bound factors, by the whole workgroup (red /
// redi: one slot per wave).  `hidden` may have been written by this
// workgroup before a barrier.
__device__ inline q6k_xhdr q6k_xprep_block(const float *__restrict__ hidden, uint32_t n_blocks, q6k_xq *xq,
                                float *red, int *redi) {
    const uint32_t n = n_blocks * 256, tid = threadIdx.x;
    float m = 0.0f;
    int bad = 0;
    for (uint32_t i = tid; i < n; i += blockDim.x) {
        const float v = hidden[i];
        bad |= !isfinite(v);
        m = fmaxf(m, fabsf(v));
    }
    const float maxabs = wm_block_max_nonan(m, red);
    bad = wm_block_sum_i32(bad, redi);
    // smallest e with maxabs * 2^-e <= 32639, kept >= -140 so 2^e stays representable
    int e = 0;
    if (maxabs > 0.0f && !bad) {
        int E;
        frexpf(maxabs, &E);  // maxabs < 2^E
        e = E - 15;
        if (ldexpf(maxabs, -e) > 32639.0f) e++;
        if (e < -140) e = -140;
    }
    for (uint32_t idx = tid; idx < n_blocks * 64; idx += blockDim.x) {
        const uint32_t b = idx >> 6, p = (idx >> 2) & 15, hn = idx & 3;
        const uint32_t k = p >> 2, l = p & 3, h = hn >> 1, band = hn & 1;
        const float *src = hidden + b * 256 + h * 128 + k * 32 + band * 16 + l;
        uint32_t ph = 0, pl = 0;
        int sum = 0;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const int v = bad ? 0 : (int)rintf(ldexpf(src[c * 4], -e));
            const int xh = (v + 128) >> 8, xl = v - 256 * xh;
            ph |= (uint32_t)(xh & 0xFF) << (8 * c);
            pl |= (uint32_t)(xl & 0xFF) << (8 * c);
            sum += v;
        }
        q6k_xq &o = xq[b * 16 + p];
        o.xh[hn] = (int)ph;
        o.xl[hn] = (int)pl;
        o.c[hn] = -32 * sum;
    }
    // Distance between the bounded pass and the reference's f32 dot, per
    // unit of sigma_r = sum_j |S_j| (S_j = d * sc_j, 16 values per sub-block,
    // |q - 32| <= 32, so a row's sum_i |(q-32) * S * y_i| <= 512 * max|y| * sigma_r):
    //  - fixed point: |x - 2^e X| <= 2^(e-1): 2^(e+8) * sigma_r;
    //  - this pass's f32 work (i32 -> f32, n_blocks fmas, 4 tree adds), on
    //    terms |d * T| with |2^e X| <= maxabs + 2^(e-1):
    //    gamma_(nb+5) * 512 * (maxabs + 2^(e-1)) * sigma_r;
    //  - the reference's f32 work (one product rounding, 16*nb - 1
    //    sequential adds, 4 combine adds): gamma_(16nb+5) * 512 * maxabs * sigma_r.
    const double u = 0x1p-24;
    const double gA = (n_blocks + 6) * u * 1.01, gB = (16.0 * n_blocks + 6) * u * 1.01;
    const double half_ulp = ldexp(1.0, e - 1);
    const double k = ldexp(1.0, e + 8) + 512.0 * (gA * ((double)maxabs + half_ulp) + gB * (double)maxabs);
    q6k_xhdr hd;
    hd.e = e;
    hd.ok = bad ? 0u : 1u;
    hd.bound_k = (float)(k * (1.0 + 0x1p-16));
    hd.mag_k = (float)(512.0 * ((double)maxabs + half_ulp) * (1.0 + 0x1p-16));
    return hd;
}

