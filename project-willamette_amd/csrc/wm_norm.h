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
    const float sum_sq = seq_sum_block_owned<PER, NT>(v2, n, sq, &L.seq, 0, before_walk);
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

// ---------------------------------------------------------------------------
// The norm a fused matvec starts from (k_i2s_fused), with the quantiser split
// by wave.
//
// Each wave of the matvec owns a slice of K: chunks [c0, c1) of the
// activation layout (chunk c: the 64 columns one 16-byte weight chunk
// covers; its byte l is column chunk_col(c, l)).  Here each wave also
// quantises exactly those columns, so its codes never leave it: the codes
// need no workgroup barrier, and Σq (the matvec subtracts Σ a) is a wave
// sum.  The only workgroup-wide quantities are Σx² (the exact sum) and
// max|y|.  max|y| needs the rsqrt, which comes from the sum, so it is found
// without a reduction after the sum: y = (v * r) * w rounds each exact
// product |v * w| * r twice, so an element whose f32 |v * w| lies more than
// 2^-19 (relative) below the largest cannot be the maximum (nor tie it), as
// long as nothing is subnormal (proof at fused_max_candidates).  Each wave
// lists its elements within 2^-19 of its own largest |v * w| (usually one),
// and wave 0 evaluates the list once it has the rsqrt.  When the conditions
// of that argument fail (a tiny maximum, huge weights, more than
// kCandSlots near-equal elements in a wave) every wave takes its own
// maximum and one LDS exchange follows.
// ---------------------------------------------------------------------------

// column of byte l of chunk c (the inverse of wm_act_perm: wm_act_perm(chunk_col(c, l)) == 64c + l)
__device__ __forceinline__ uint32_t chunk_col(uint32_t c, uint32_t l) {
    return 128u * (c >> 1) + 32u * (l >> 4) + 16u * (c & 1u) + (l & 15u);
}

// NP (a multiple of 4, or below 4) consecutive f32 values from byte offset
// `off` of a buffer, in 16-byte loads (zeros past the buffer's end; the
// callers' runs lie wholly inside or wholly past it)
template <int NP>
__device__ __forceinline__ void buf_run(__amdgpu_buffer_rsrc_t rs, uint32_t off, float (&out)[NP]) {
    if constexpr (NP >= 4) {
#pragma unroll
        for (int j = 0; j < NP; j += 4) {
            const wm_v4u v = __builtin_bit_cast(wm_v4u, __builtin_amdgcn_raw_buffer_load_b128(rs, off + 4 * j, 0, 0));
            out[j] = __uint_as_float(v.x);
            out[j + 1] = __uint_as_float(v.y);
            out[j + 2] = __uint_as_float(v.z);
            out[j + 3] = __uint_as_float(v.w);
        }
    } else {
#pragma unroll
        for (int j = 0; j < NP; j++) out[j] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, off + 4 * j, 0, 0));
    }
}

constexpr int kCandSlots = 4;

template <int NW>
struct fused_norm_lds {
    seq_block_scratch seq;
    float cand_v[NW][kCandSlots], cand_w[NW][kCandSlots];
    float cand_m[NW];  // the wave's largest f32 |v * w| (NaN never counted)
    int cand_n[NW];    // candidates listed; kCandSlots + 1: too many to list
    int cand_bad[NW];  // the wave holds a weight that breaks the bound (|w| > 2^60, NaN)
    float red_f[NW];   // fallback exchange of the wave maxima of |y|
    float rsq, maxabs;  // wave 0 -> all: the rsqrt and max|y| (maxabs < 0: fallback)
    float spec_rsq, spec_max;  // the speculation's rsqrt and max|y| (spec_max < 0: none)
};

// The quantiser's elements of one lane: round r covers chunk
// c0 + 4r + lane/16 (when below c1) and, in it, the four consecutive
// columns of byte quad lane % 16.  vq/wq hold them; valid() says which
// rounds hold a chunk of the wave.
template <int NR>
struct fused_quads {
    float v[NR][4], w[NR][4];
    __device__ __forceinline__ bool valid(int r, uint32_t c0, uint32_t nc) const {
        return 4u * (uint32_t)r + ((threadIdx.x & 63) >> 4) < nc;
    }
};
__device__ __forceinline__ uint32_t quad_chunk(int r, uint32_t c0) {
    return c0 + 4u * (uint32_t)r + ((threadIdx.x & 63) >> 4);
}
__device__ __forceinline__ uint32_t quad_col(int r, uint32_t c0) {
    return chunk_col(quad_chunk(r, c0), 4u * (threadIdx.x & 15));
}

// Before the sum: this wave's candidate list for max|y|.
template <int NR, int NW>
__device__ __forceinline__ void fused_max_candidates(const fused_quads<NR> &Q, uint32_t c0, uint32_t nc,
                                                     fused_norm_lds<NW> &L) {
    const uint32_t lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    float p[NR][4];
    float mx = 0.0f;
    bool bad = false;
#pragma unroll
    for (int r = 0; r < NR; r++) {
        const bool ok = Q.valid(r, c0, nc);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            p[r][i] = ok ? fabsf(Q.v[r][i]) * fabsf(Q.w[r][i]) : 0.0f;
            mx = p[r][i] > mx ? p[r][i] : mx;
            bad |= ok && !(fabsf(Q.w[r][i]) <= 0x1p60f);
        }
    }
    const float M = wm_wave_max_nonneg(mx);
    const float thr = M * (1.0f - 0x1p-19f);
    int cnt = 0;
#pragma unroll
    for (int r = 0; r < NR; r++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const bool c = p[r][i] >= thr && M > 0.0f;
            const uint64_t m = __builtin_amdgcn_ballot_w64(c);
            const int pos = cnt + __builtin_popcountll(m & ((1ull << lane) - 1ull));
            if (c && pos < kCandSlots) {
                L.cand_v[wid][pos] = Q.v[r][i];
                L.cand_w[wid][pos] = Q.w[r][i];
            }
            cnt += __builtin_popcountll(m);
        }
    const bool any_bad = __builtin_amdgcn_ballot_w64(bad) != 0;
    if (lane == 0) {
        L.cand_m[wid] = M;
        L.cand_n[wid] = cnt > kCandSlots ? kCandSlots + 1 : cnt;
        L.cand_bad[wid] = any_bad;
    }
}

// What wave 0 reads of the candidate lists, fetched while it walks the sum.
// Lane l: wave l's maximum and flags (l < NW), and candidate slot l % 4 of
// wave l / 4.
struct fused_cand_regs {
    float m, cv, cw, cm;
    int n, bad, cn;
    // what does not depend on the rsqrt (fused_cand_prep): the largest p, the
    // lists' flags, and whether this lane's slot is a candidate
    float M;
    bool flags, use;
};
template <int NW>
__device__ __forceinline__ fused_cand_regs fused_cand_fetch(const fused_norm_lds<NW> &L) {
    const int lane = (int)(threadIdx.x & 63), w = lane / kCandSlots, j = lane % kCandSlots;
    fused_cand_regs c;
    const int l = lane < NW ? lane : 0, wq = w < NW ? w : 0;
    c.m = lane < NW ? L.cand_m[l] : 0.0f;
    c.n = lane < NW ? L.cand_n[l] : 0;
    c.bad = lane < NW ? L.cand_bad[l] : 0;
    c.cv = L.cand_v[wq][j];
    c.cw = L.cand_w[wq][j];
    c.cm = w < NW ? L.cand_m[wq] : 0.0f;
    c.cn = w < NW ? L.cand_n[wq] - j : 0;  // > 0: slot j holds a candidate
    c.M = 0.0f;
    c.flags = true;
    c.use = false;
    return c;
}

// The part of fused_cand_max that does not depend on the rsqrt, ahead of it.
__device__ __forceinline__ void fused_cand_prep(fused_cand_regs &c) {
    c.M = wm_wave_max_nonneg(c.m);
    c.flags = __builtin_amdgcn_ballot_w64(c.n > kCandSlots || c.bad != 0) != 0;
    c.use = c.cn > 0 && c.cm >= c.M * (1.0f - 0x1p-19f);
}

// max|y| for a given rsqrt from the candidate lists (every lane gets it),
// and whether the bound below holds for it (false: every wave must take its
// own maximum).
//
// Why the candidates suffice.  Let M be the largest f32 p = RN(|v * w|) and
// k an element attaining it; an element i outside the lists has
// p_i < M (1 - 2^-19).  With u = 2^-24 and every rounding relative (no
// subnormal result): |v_i w_i| <= p_i (1 + u), |y_i| <= |v_i w_i| r (1 + u)^2,
// |y_k| >= M r (1 - u)^3, and (1 - 2^-19)(1 + u)^3 < (1 - u)^3, so
// |y_i| < |y_k|.  Subnormals add absolute errors of at most 2^-150 per
// rounding, times |w| <= 2^60 at most: below 2^-88, against a gap of at
// least 2^-20 |y_k| >= 2^-80 once max|y| >= 2^-60 and M >= 2^-100.  Those
// are the conditions checked.
// (c has been through fused_cand_prep)
__device__ __forceinline__ float fused_cand_max(const fused_cand_regs &c, float rsq, bool &ok) {
    const float yy = c.cv * rsq * c.cw;  // out = x * rsqrt * weight
    const float ya = wm_wave_max_nonneg(c.use ? fabsf(yy) : 0.0f);
    ok = !c.flags && c.M >= 0x1p-100f && ya >= 0x1p-60f;
    return ya;
}

// rsqrt = 1/sqrt(Σx²/n + eps) (primitives.rs:247-248)
__device__ __forceinline__ float norm_rsq(float sum_sq, uint32_t n, float eps) {
    const float mean = sum_sq / (float)n;
    return 1.0f / sqrtf(mean + eps);
}

// Wave 0, after the sum: the rsqrt and max|y| to LDS (maxabs = -1: the
// candidate bound does not hold).
template <int NW>
__device__ __forceinline__ void fused_publish(float sum_sq, uint32_t n, float eps, const fused_cand_regs &c,
                                              fused_norm_lds<NW> &L, bool no_candidates = false) {
    const float rsq = norm_rsq(sum_sq, n, eps);
    bool ok;
    const float ya = fused_cand_max(c, rsq, ok);
    ok = ok && !no_candidates;
    if ((threadIdx.x & 63) == 0) {
        L.rsq = rsq;
        L.maxabs = ok ? ya : -1.0f;
    }
}

// max|y| over the workgroup when the candidates cannot settle it: every wave
// takes its own maximum, one LDS exchange (all waves call this together).
template <int NR, int NW>
__device__ __forceinline__ float fused_block_max(const fused_quads<NR> &Q, uint32_t c0, uint32_t nc, float rsq,
                                                 fused_norm_lds<NW> &L) {
    float mx = 0.0f;
#pragma unroll
    for (int r = 0; r < NR; r++) {
        const bool ok = Q.valid(r, c0, nc);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float y = Q.v[r][i] * rsq * Q.w[r][i];  // out[i] = x[i] * rsqrt * weight[i]
            if (ok) mx = wm_max_nonan(mx, fabsf(y));
        }
    }
    const float m = wm_wave_max_nonneg(mx);
    if ((threadIdx.x & 63) == 0) L.red_f[threadIdx.x >> 6] = m;
    wm_sync_lds();
    float max_abs = L.red_f[0];
#pragma unroll
    for (int i = 1; i < NW; i++) max_abs = wm_max_nonan(max_abs, L.red_f[i]);
    return max_abs;
}

// This wave's int8 codes for a given rsqrt and max|y| (absmax quantiser,
// bitlinear_sse2.rs:285-304) into act bytes [64 c0, 64 c1), four codes per
// dword, the dwords also to qw; returns the wave's Σq.  With DIST, each
// element's distance from |y * inv| to the nearest rounding boundary (k +
// 1/2), or -1 where RN(x * rsqrt) is nonzero and below 2^-125 (its rounding
// may be absolute): what decides whether a slightly different rsqrt or
// max|y| can change the element's code.
template <int NR, bool DIST>
__device__ __forceinline__ int fused_codes(const fused_quads<NR> &Q, uint32_t c0, uint32_t nc, float rsq,
                                           float max_abs, uint8_t *act, uint32_t (&qw)[NR],
                                           float (&dist)[NR][4]) {
    const uint32_t lane = threadIdx.x & 63;
    const float inv = 127.0f / max_abs;
    int sum = 0;
#pragma unroll
    for (int r = 0; r < NR; r++) {
        qw[r] = 0;
        if (Q.valid(r, c0, nc)) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float xr = Q.v[r][i] * rsq;
                const float p = (xr * Q.w[r][i]) * inv;  // out[i] = x[i] * rsqrt * weight[i], then * inv
                const int q = max_abs == 0.0f ? 0 : wm_round_clamp_i8_fast(p);
                qw[r] |= ((uint32_t)q & 0xFFu) << (8 * i);
                sum += q;
                if (DIST) {
                    const float d = fabsf(__builtin_amdgcn_fractf(fabsf(p)) - 0.5f);
                    dist[r][i] = xr != 0.0f && fabsf(xr) < 0x1p-125f ? -1.0f : d;
                }
            }
            *reinterpret_cast<uint32_t *>(act + 64u * quad_chunk(r, c0) + 4u * (lane & 15)) = qw[r];
        }
    }
    return __builtin_amdgcn_readlane(wm_wave_scan_i32(sum), 63);
}

}  // namespace wm
