// Q6_K kernels for gfx950: repack, row dequantisation (embedding gather) and
// the tied lm-head (logits + argmax).
//
// Reference semantics (project-willamette):
//   block layout   src/model/q6_k.rs:25-57   ql[0..128] qh[128..192] sc i8[192..208] d f16[208..210]
//   dequant        src/model/q6_k.rs:59-69   value = (d*sc)*q, q = 6-bit - 32 (exact in f32)
//   row dot (x86)  src/model/q6_k_sse2.rs:46-116
//   logits         src/model/lm_head.rs:29-108 (one row dot per vocab row)
//   argmax         src/model/lm_head.rs:161-174 (first index of the maximum)
//
// The x86 row dot keeps 16 f32 partial sums: quarter k (0..3) x lane l
// (0..3); partial (k,l) accumulates ((q*(d*sc))*x) for the values whose
// index within a half-block is 32k + 16*band + 4*chunk + l, in (block, half,
// band, chunk) order, and the 16 partials are combined as
//   v_l = (p0l + p1l) + (p2l + p3l);  dot = (v0 + v3) + (v1 + v2).
// The exact kernel gives each of those 16 partial sums to its own lane, so a
// wave computes 4 rows with exactly the reference's roundings.
//
// Device layout (k_q6k_repack): rows in groups of 4; a group of n_blocks
// blocks takes 840 * n_blocks bytes, the same byte count as its GGUF blocks:
//   quants   768 bytes per block b, at 768*b: lane L' = 16*row + 4k + l holds,
//            in 3 dwords A, B, C, the 16 six-bit quants it consumes in this
//            block, q(hn, c) for hn = 2*half + band, c = chunk: byte c of
//            A / B / C holds q(0, c) / q(1, c) / q(2, c) in bits 0-5, and
//            bits 6-7 of the three bytes hold q(3, c)'s bits 0-1 / 2-3 / 4-5;
//            so the quants come back as bytes (byte c of U[hn] = q(hn, c))
//            with three ANDs and six shift/AND-OR operations;
//   scales   from 768*n_blocks, one dword per (class 4*row + k, block) in
//            [class][block] order, byte hn = sc[8h + band + 2k];
//   d        from 832*n_blocks, the f16 d values in [row][block] order.
// Each class's scales and each row's d values are contiguous, so a lane
// fetches a batch of blocks' side data with a few wide loads instead of two
// narrow loads per block (the narrow loads cost about a tenth of the
// lm-head pass's time).
//
// Two lm-head paths:
//  * exact (k_q6k_logits): every logit bit-identical to the reference, one
//    lane per SSE2 partial sum.  Used whenever the caller wants the logits.
//  * argmax-only (k_q6k_bounded -> k_q6k_select): a
//    bandwidth-bound pass computes every row's dot from
//    the int8 quants with v_dot4_i32_i8 against a 16-bit fixed-point copy of
//    the hidden vector, together with a rigorous bound on its distance from
//    the reference's f32 result.  Only rows whose upper bound reaches the
//    largest lower bound are recomputed in the exact order; every other row
//    is provably below the maximum, so the argmax is the reference's.
#include <hip/hip_fp16.h>

#include "wm_internal.h"
#include "wm_q6k_xprep.h"

namespace {

constexpr int kLogitsBlock = 256;  // 4 waves
constexpr int kMaxArgBlocks = 2048;
constexpr int kBoundedBlock = 256;
constexpr uint32_t kBoundedMaxBlocks = 2048;
constexpr bool kPipelined = true;

__host__ __device__ __forceinline__ int q6_of(const uint8_t *blk, int h, int k, int l) {
    const uint8_t *ql = blk + h * 64, *qh = blk + 128 + h * 32;
    uint32_t lo = (k & 1) ? ql[l + 32] : ql[l];
    lo = (k & 2) ? (lo >> 4) : (lo & 0x0Fu);
    uint32_t hi = (qh[l] >> (2 * k)) & 3u;
    return (int)(lo | (hi << 4));
}

__global__ void k_q6k_repack(const uint8_t *__restrict__ raw, uint8_t *__restrict__ out,
                             uint32_t n_rows, uint32_t n_blocks, uint32_t n_rowgroups) {
    uint64_t total = (uint64_t)n_rowgroups * n_blocks * Q6K_GROUP_ROWS;
    for (uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (uint64_t)gridDim.x * blockDim.x) {
        uint32_t r = idx % Q6K_GROUP_ROWS;
        uint64_t gb = idx / Q6K_GROUP_ROWS;
        uint32_t b = gb % n_blocks;
        uint64_t G = gb / n_blocks;
        uint64_t row = G * Q6K_GROUP_ROWS + r;
        uint8_t *grp = out + G * q6k_group_bytes(n_blocks);
        uint32_t *q6 = reinterpret_cast<uint32_t *>(grp + b * Q6K_QUANT_BYTES);
        uint32_t *scw = reinterpret_cast<uint32_t *>(grp + q6k_sc_base(n_blocks)) + b;  // + class*n_blocks
        uint16_t *dw = reinterpret_cast<uint16_t *>(grp + q6k_d_base(n_blocks)) +
                       r * q6k_d_stride(n_blocks) + b;
        if (b + 1 == n_blocks && (n_blocks & 1)) dw[1] = 0;  // the row's padding half
        if (row >= n_rows) {
            for (int L = 0; L < 16; L++)
                for (int j = 0; j < 3; j++) q6[(r * 16 + L) * 3 + j] = 0;
            for (int k = 0; k < 4; k++) scw[(r * 4 + k) * n_blocks] = 0;
            *dw = 0;
            continue;
        }
        const uint8_t *blk = raw + (row * n_blocks + b) * Q6K_BYTES;
        for (int k = 0; k < 4; k++) {
            for (int l = 0; l < 4; l++) {
                uint32_t w[3] = {0, 0, 0};
                for (int c = 0; c < 4; c++) {
                    uint32_t q[4];
                    for (int hn = 0; hn < 4; hn++)
                        q[hn] = (uint32_t)q6_of(blk, hn >> 1, k, (hn & 1) * 16 + c * 4 + l);
                    for (int t = 0; t < 3; t++)
                        w[t] |= (q[t] | (((q[3] >> (2 * t)) & 3u) << 6)) << (8 * c);
                }
                const int L = r * 16 + k * 4 + l;
                q6[L * 3 + 0] = w[0]; q6[L * 3 + 1] = w[1]; q6[L * 3 + 2] = w[2];
            }
            uint32_t sc = 0;
            for (int hn = 0; hn < 4; hn++) {
                int h = hn >> 1, n = hn & 1;
                sc |= (uint32_t)blk[192 + h * 8 + n + 2 * k] << (8 * hn);
            }
            scw[(r * 4 + k) * n_blocks] = sc;
        }
        *dw = (uint16_t)(blk[208] | (blk[209] << 8));
    }
}

// The 16 quants of one lane as 4 dwords of bytes: byte c of U[hn] = q(hn, c).
__device__ __forceinline__ void q6_unpack(uint32_t a, uint32_t b, uint32_t c, uint32_t U[4]) {
    const uint32_t m = 0x3F3F3F3Fu;
    U[0] = a & m;
    U[1] = b & m;
    U[2] = c & m;
    U[3] = ((a >> 6) & 0x03030303u) | ((b >> 4) & 0x0C0C0C0Cu) | ((c >> 2) & 0x30303030u);
}
// One quant q(hn, c) of a lane's three dwords.
__device__ __forceinline__ uint32_t q6_get(const uint32_t *w, int hn, int c) {
    if (hn < 3) return (w[hn] >> (8 * c)) & 63u;
    const int s = 8 * c + 6;
    return ((w[0] >> s) & 3u) | (((w[1] >> s) & 3u) << 2) | (((w[2] >> s) & 3u) << 4);
}

// Dequantise row values: thread t of 256 handles value t of each block.
// Grid (n_blocks, n_rows): row blockIdx.y comes from d_row[blockIdx.y] when
// d_row is given and goes to out + blockIdx.y * ld.
__global__ void k_q6k_dequant_row(const uint8_t *__restrict__ w, uint32_t n_blocks,
                                  uint32_t row, const uint32_t *__restrict__ d_row,
                                  float *__restrict__ out, uint32_t ld) {
    if (d_row) row = d_row[blockIdx.y];
    out += (uint64_t)blockIdx.y * ld;
    const uint32_t G = row / Q6K_GROUP_ROWS, r = row % Q6K_GROUP_ROWS;
    const uint32_t b = blockIdx.x, t = threadIdx.x;
    const uint8_t *grp = w + (uint64_t)G * q6k_group_bytes(n_blocks);
    const int h = t >> 7, k = (t >> 5) & 3, n = (t >> 4) & 1, c = (t >> 2) & 3, l = t & 3;
    const int L = r * 16 + k * 4 + l, hn = h * 2 + n;
    const uint32_t *q6 = reinterpret_cast<const uint32_t *>(grp + b * Q6K_QUANT_BYTES) + L * 3;
    const uint32_t wl[3] = {q6[0], q6[1], q6[2]};
    const uint32_t q = q6_get(wl, hn, c);
    const uint32_t scw =
        reinterpret_cast<const uint32_t *>(grp + q6k_sc_base(n_blocks))[(r * 4 + k) * n_blocks + b];
    const int sc = (int)(int8_t)(scw >> (8 * hn));
    const float d = wm_f16_bits_to_f32(
        reinterpret_cast<const uint16_t *>(grp + q6k_d_base(n_blocks))[r * q6k_d_stride(n_blocks) + b]);
    out[b * Q6K_VALUES + t] = d * (float)sc * (float)((int)q - 32);
}

struct argcand {
    float v;
    uint32_t i;
};

// (v, i) ordering for the first-index-of-maximum rule; NaN never wins.
__device__ __forceinline__ bool cand_better(float v, uint32_t i, float bv, uint32_t bi) {
    return v > bv || (v == bv && i < bi);
}

// ---------------------------------------------------------------------------
// exact row dot (reference order)
// ---------------------------------------------------------------------------

// The hidden vector permuted into lane order: xs[L * stride + b*16 + s]
// holds the value lane L = 4k + l multiplies at step s of block b.
__host__ __device__ __forceinline__ uint32_t xs_stride(uint32_t n_blocks) { return n_blocks * 16 + 4; }

__device__ void build_xs(const float *__restrict__ hidden, uint32_t n_blocks, float *xs) {
    const uint32_t stride = xs_stride(n_blocks);
    for (uint32_t idx = threadIdx.x; idx < 16u * n_blocks * 16u; idx += blockDim.x) {
        uint32_t L = idx / (n_blocks * 16), rem = idx % (n_blocks * 16);
        uint32_t b = rem / 16, s = rem % 16;
        uint32_t k = L >> 2, l = L & 3, hn = s >> 2, c = s & 3, h = hn >> 1, n = hn & 1;
        xs[L * stride + b * 16 + s] = hidden[b * 256 + h * 128 + k * 32 + n * 16 + c * 4 + l];
    }
}

// One lane's data for CH consecutive blocks of a 4-row group: its quants,
// its class's scale dwords and its row's d values (two f16 per dword).
template <int CH>
struct q6_lane_blocks {
    uint32_t w0[CH], w1[CH], w2[CH], scw[CH], dw[(CH + 1) / 2];
};
template <int CH>
__device__ __forceinline__ uint32_t q6_d_bits(const q6_lane_blocks<CH> &v, int j) {
    return (v.dw[j >> 1] >> (16 * (j & 1))) & 0xFFFFu;
}

// Per-lane offsets within a group for lane (row r, lane-in-row L = 4k + l).
struct q6_lane_offs {
    uint32_t q, sc, d;
};
__device__ __forceinline__ q6_lane_offs q6_offs(uint32_t n_blocks, uint32_t r, uint32_t L) {
    return q6_lane_offs{(16 * r + L) * 12, q6k_sc_base(n_blocks) + (4 * r + (L >> 2)) * 4 * n_blocks,
                        q6k_d_base(n_blocks) + r * 2 * q6k_d_stride(n_blocks)};
}

typedef unsigned int q6_v4u __attribute__((ext_vector_type(4)));
typedef unsigned int q6_v2u __attribute__((ext_vector_type(2)));

// N consecutive dwords at voff + soff through a buffer descriptor, in 16-,
// 12-, 8- and 4-byte loads (buffer loads need dword alignment only).
template <int N>
__device__ __forceinline__ void q6_load_dwords(uint32_t *out, __amdgpu_buffer_rsrc_t rs,
                                               uint32_t voff, uint32_t soff) {
#pragma unroll
    for (int i = 0; i + 4 <= N; i += 4) {
        const q6_v4u q = __builtin_amdgcn_raw_buffer_load_b128(rs, voff, soff + 4 * i, WM_LOAD_NT);
        out[i] = q.x;
        out[i + 1] = q.y;
        out[i + 2] = q.z;
        out[i + 3] = q.w;
    }
    constexpr int i = N & ~3;
    if constexpr (N - i == 3) {
        const wm_v3u q = __builtin_amdgcn_raw_buffer_load_b96(rs, voff, soff + 4 * i, WM_LOAD_NT);
        out[i] = q.x;
        out[i + 1] = q.y;
        out[i + 2] = q.z;
    } else if constexpr (N - i == 2) {
        const q6_v2u q = __builtin_amdgcn_raw_buffer_load_b64(rs, voff, soff + 4 * i, WM_LOAD_NT);
        out[i] = q.x;
        out[i + 1] = q.y;
    } else if constexpr (N - i == 1) {
        out[i] = __builtin_amdgcn_raw_buffer_load_b32(rs, voff, soff + 4 * i, WM_LOAD_NT);
    }
}

// Loads through a buffer descriptor of a wave-uniform group base (streaming
// kernels): lane offsets are per-lane constants, block offsets uniform.  Per
// batch: the side data in a few wide loads (an even CH starts on an even
// block, so its d values start on a dword), then CH 12-byte quant loads;
// side data first, so the first block can be reduced as soon as its quants
// arrive.
template <int CH>
__device__ __forceinline__ void q6_load_uniform(q6_lane_blocks<CH> &v, __amdgpu_buffer_rsrc_t rs,
                                                uint32_t b0, const q6_lane_offs &o) {
    q6_load_dwords<CH>(v.scw, rs, o.sc, b0 * 4);
    if constexpr (CH % 2 == 0) {
        q6_load_dwords<CH / 2>(v.dw, rs, o.d, b0 * 2);
    } else {
#pragma unroll
        for (int j = 0; j < (CH + 1) / 2; j++) v.dw[j] = 0;
#pragma unroll
        for (int j = 0; j < CH; j++)
            v.dw[j >> 1] |= (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rs, o.d, (b0 + j) * 2, 0)
                            << (16 * (j & 1));
    }
#pragma unroll
    for (int j = 0; j < CH; j++) {
        const wm_v3u q =
            __builtin_amdgcn_raw_buffer_load_b96(rs, o.q, (b0 + j) * Q6K_QUANT_BYTES, WM_LOAD_NT);
        v.w0[j] = q.x;
        v.w1[j] = q.y;
        v.w2[j] = q.z;
    }
}

// Loads from a per-lane group base (rows gathered from different groups).
template <int CH>
__device__ __forceinline__ void q6_load_lane(q6_lane_blocks<CH> &v, const uint8_t *gbase,
                                             uint32_t b0, const q6_lane_offs &o) {
#pragma unroll
    for (int j = 0; j < (CH + 1) / 2; j++) v.dw[j] = 0;
#pragma unroll
    for (int j = 0; j < CH; j++) {
        const uint32_t *q6 =
            reinterpret_cast<const uint32_t *>(gbase + (b0 + j) * Q6K_QUANT_BYTES + o.q);
        v.w0[j] = q6[0];
        v.w1[j] = q6[1];
        v.w2[j] = q6[2];
        v.scw[j] = reinterpret_cast<const uint32_t *>(gbase + o.sc)[b0 + j];
        v.dw[j >> 1] |= (uint32_t)reinterpret_cast<const uint16_t *>(gbase + o.d)[b0 + j]
                        << (16 * (j & 1));
    }
}

// Accumulate blocks b0..b0+CH-1 into this lane's partial in the SSE2 order
// (xl = xs + L*stride).
template <int CH>
__device__ __forceinline__ void q6_exact_accum(const q6_lane_blocks<CH> &v, uint32_t b0,
                                               const float *xl, float &acc) {
#pragma unroll
    for (int j = 0; j < CH; j++) {
        uint32_t U[4];
        q6_unpack(v.w0[j], v.w1[j], v.w2[j], U);
        const float d = wm_f16_bits_to_f32(q6_d_bits(v, j));
        const float *xb = xl + (b0 + j) * 16;
        if (__builtin_expect(isfinite(d), 1)) {
#pragma unroll
            for (int hn = 0; hn < 4; hn++) {
                const float S = d * (float)(int)(int8_t)(v.scw[j] >> (8 * hn));
                const float nS32 = -32.0f * S;
                const float4 x4 = *reinterpret_cast<const float4 *>(xb + hn * 4);
                const float xv[4] = {x4.x, x4.y, x4.z, x4.w};
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    // (q - 32) * S is exact in f32, so the fused form equals the
                    // reference's rounded product q * (d*sc).
                    const float qf = (float)((U[hn] >> (8 * c)) & 0xFFu);
                    const float qS = __builtin_fmaf(qf, S, nS32);
                    acc = acc + qS * xv[c];
                }
            }
        } else {
            for (int hn = 0; hn < 4; hn++) {
                const float S = d * (float)(int)(int8_t)(v.scw[j] >> (8 * hn));
                for (int c = 0; c < 4; c++) {
                    const int q = (int)((U[hn] >> (8 * c)) & 0xFFu);
                    const float qS = (float)(q - 32) * S;
                    acc = acc + qS * xb[hn * 4 + c];
                }
            }
        }
    }
}

// Combine the 16 partials of a lane group: v_l = (p0l + p1l) + (p2l + p3l);
// dot = (v0 + v3) + (v1 + v2).  The dot ends up in all 16 lanes.
__device__ __forceinline__ float q6_combine(float acc) {
    float t = acc + __shfl_xor(acc, 4, 64);
    float v = t + __shfl_xor(t, 8, 64);
    float u = v + __shfl_xor(v, 3, 64);
    return u + __shfl_xor(u, 1, 64);
}

template <int CH>
__global__ __launch_bounds__(kLogitsBlock) void k_q6k_logits(
    const uint8_t *__restrict__ w, uint32_t n_blocks, uint32_t n_rows, uint32_t n_rowgroups,
    const float *__restrict__ hidden, float *__restrict__ logits, argcand *__restrict__ cands) {
    extern __shared__ float xs[];  // [16][n_blocks*16 + 4]
    build_xs(hidden, n_blocks, xs);
    __syncthreads();
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t r = lane >> 4, L = lane & 15;
    const float *xl = xs + L * xs_stride(n_blocks);
    const q6_lane_offs o = q6_offs(n_blocks, r, L);
    const uint32_t group_bytes = q6k_group_bytes(n_blocks);
    float best_v = -INFINITY;
    uint32_t best_i = 0xFFFFFFFFu;
    constexpr uint32_t kWaves = kLogitsBlock / 64;
    const uint32_t waves_total = gridDim.x * kWaves;
    for (uint32_t G = blockIdx.x * kWaves + wave; G < n_rowgroups; G += waves_total) {
        const __amdgpu_buffer_rsrc_t rs = wm_rsrc(w + (uint64_t)G * group_bytes, group_bytes);
        float acc = 0.0f;
        for (uint32_t b0 = 0; b0 < n_blocks; b0 += CH) {
            q6_lane_blocks<CH> v;
            q6_load_uniform<CH>(v, rs, b0, o);
            q6_exact_accum<CH>(v, b0, xl, acc);
        }
        const float dot = q6_combine(acc);
        const uint32_t row = G * Q6K_GROUP_ROWS + r;
        if (L == 0 && row < n_rows) {
            if (logits) logits[row] = dot;
            if (cand_better(dot, row, best_v, best_i)) {
                best_v = dot;
                best_i = row;
            }
        }
    }
    // block-wide best candidate
    for (int o = 32; o > 0; o >>= 1) {
        float ov = __shfl_xor(best_v, o, 64);
        uint32_t oi = __shfl_xor(best_i, o, 64);
        if (cand_better(ov, oi, best_v, best_i)) {
            best_v = ov;
            best_i = oi;
        }
    }
    __shared__ argcand s_c[kLogitsBlock / 64];
    if (lane == 0) s_c[wave] = argcand{best_v, best_i};
    __syncthreads();
    if (threadIdx.x == 0) {
        argcand bc = s_c[0];
        for (int i = 1; i < (int)(blockDim.x >> 6); i++)
            if (cand_better(s_c[i].v, s_c[i].i, bc.v, bc.i)) bc = s_c[i];
        cands[blockIdx.x] = bc;
    }
}

// Combine the per-block candidates; a NaN logit at index 0 wins, as the
// reference's scan starts from logits[0] and NaN compares false.
__global__ void k_argmax_final(const argcand *__restrict__ cands, uint32_t n_cands,
                               const float *__restrict__ first_logit, uint32_t *__restrict__ out) {
    float bv = -INFINITY;
    uint32_t bi = 0xFFFFFFFFu;
    for (uint32_t i = threadIdx.x; i < n_cands; i += 64)
        if (cand_better(cands[i].v, cands[i].i, bv, bi)) {
            bv = cands[i].v;
            bi = cands[i].i;
        }
    for (int o = 32; o > 0; o >>= 1) {
        float ov = __shfl_xor(bv, o, 64);
        uint32_t oi = __shfl_xor(bi, o, 64);
        if (cand_better(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
        }
    }
    if (threadIdx.x == 0) {
        float f0 = *first_logit;
        // every row's value is -inf or NaN: the scan keeps index 0
        *out = (f0 != f0 || bi == 0xFFFFFFFFu) ? 0u : bi;
    }
}

// ---------------------------------------------------------------------------
// argmax-only path
// ---------------------------------------------------------------------------

// sigma_r = sum over the row's blocks b and sub-blocks j of |d_b * sc_bj|,
// from the raw GGUF blocks, in double and rounded up to f32 (non-finite d
// gives a non-finite sigma, which makes the row a rescoring candidate).
__global__ void k_q6k_row_sigma(const uint8_t *__restrict__ raw, uint32_t n_rows,
                                uint32_t n_blocks, float *__restrict__ sigma) {
    const uint32_t row = blockIdx.x * blockDim.x + threadIdx.x;
    if (row >= n_rows) return;
    double s = 0.0;
    for (uint32_t b = 0; b < n_blocks; b++) {
        const uint8_t *blk = raw + ((uint64_t)row * n_blocks + b) * Q6K_BYTES;
        int asc = 0;
        for (int j = 0; j < 16; j++) asc += abs((int)(int8_t)blk[192 + j]);
        const double d = (double)wm_f16_bits_to_f32(blk[208] | (blk[209] << 8));
        s += fabs(d) * asc;
    }
    sigma[row] = (float)(s * (1.0 + 0x1p-20));
}

// d = a * b + c on the low 24 bits of a and b (sign-extended), low 32 bits of
// the result: one full-rate v_mad_i32_i24.  (For this use the compiler emits a
// quarter-rate 32-bit multiply.)  The operands must come from ordinary VALU
// instructions: the instruction is opaque to the compiler's hazard tracking,
// so it must not read a register a DOT instruction has just written.
__device__ __forceinline__ int mad_i24(int a, int b, int c) {
    int d;
    asm("v_mad_i32_i24 %0, %1, %2, %3" : "=v"(d) : "v"(a), "v"(b), "v"(c));
    return d;
}

// The prep area from a hidden vector in device memory (one workgroup).
__global__ __launch_bounds__(256) void k_q6k_xprep(const float *__restrict__ hidden,
                                                   uint32_t n_blocks, uint8_t *__restrict__ prep) {
    __shared__ float red[4];
    __shared__ int redi[4];
    const q6k_xhdr h = q6k_xprep_block(hidden, n_blocks, reinterpret_cast<q6k_xq *>(prep), red, redi);
    if (threadIdx.x == 0) *reinterpret_cast<q6k_xhdr *>(prep + q6k_xq_bytes(n_blocks)) = h;
}

// One lane's contribution to its row's bounded dot over blocks b0..b0+CH-1:
// per group hn two int8 dots of the bytes U[hn] with xh and xl,
// I = 256*dh + dl (exact, |I| < 2^23), T = sum_hn sc_hn * I (exact,
// |T| < 2^31), acc += d * T in f32.
template <int CH>
__device__ __forceinline__ void q6_bounded_accum(const q6_lane_blocks<CH> &v, uint32_t b0,
                                                 const q6k_xq *xq, uint32_t p, float &acc) {
#pragma unroll
    for (int j = 0; j < CH; j++) {
        uint32_t U[4];
        q6_unpack(v.w0[j], v.w1[j], v.w2[j], U);
        // the block's 48 bytes of x in three 16-byte LDS reads
        const int4 *xp = reinterpret_cast<const int4 *>(xq + (b0 + j) * 16 + p);
        const int4 h4 = xp[0], l4 = xp[1], c4 = xp[2];
        const int xh[4] = {h4.x, h4.y, h4.z, h4.w}, xl[4] = {l4.x, l4.y, l4.z, l4.w},
                  xc[4] = {c4.x, c4.y, c4.z, c4.w};
        int T = 0;
#pragma unroll
        for (int hn = 0; hn < 4; hn++) {
            const int sc = (int)(int8_t)(v.scw[j] >> (8 * hn));
            // (clamp selects the three-operand encoding, which needs no zeroed
            // accumulator register; |dh| <= 32256 never saturates)
            const int dh = __builtin_amdgcn_sdot4((int)U[hn], xh[hn], 0, true);
            const int dl = __builtin_amdgcn_sdot4((int)U[hn], xl[hn], xc[hn], false);
            const int I = (int)(((uint32_t)dh << 8) + (uint32_t)dl);  // a VALU result
            T = mad_i24(sc, I, T);
        }
        const float d = __half2float(__ushort_as_half((unsigned short)q6_d_bits(v, j)));
        acc = __builtin_fmaf(d, (float)T, acc);
    }
}

// Bounded pass.  Workgroup w takes the 4-row groups [g0, g1) (contiguous, so
// its rows form one range), its waves taking them in turn.  Lane (r, p =
// 4k + l) of a wave handles the same 16 quants per block as in the exact
// kernel (q6_bounded_accum).  Per row: logit ~ 2^e * sum of the 16 lanes'
// acc, bound = bound_k * sigma_r, widened so that rounding a +- bound in f32
// cannot cross the true interval.  The workgroup's largest lower and upper
// bounds go to wg_lb / wg_ub.  PIPE: loads go in batches of CH blocks, the
// next batch (of this group or the wave's next one) in flight while the
// current one is reduced, so every wave keeps memory busy between its
// reductions (two register sets of CH blocks).
template <int CH, bool PIPE>
__global__ __launch_bounds__(kBoundedBlock) void k_q6k_bounded(
    const uint8_t *__restrict__ w, uint32_t n_blocks, uint32_t n_rows, uint32_t n_rowgroups,
    const float *__restrict__ sigma, const uint8_t *__restrict__ prep, const float *__restrict__ hidden,
    float *__restrict__ approx, float *__restrict__ bound, float *__restrict__ wg_lb,
    float *__restrict__ wg_ub) {
    extern __shared__ __align__(16) q6k_xq xq[];  // [n_blocks][16]
    __shared__ float red[kBoundedBlock / 64], red2[kBoundedBlock / 64];
    __shared__ int redi[kBoundedBlock / 64];
    // the fixed-point copy of the hidden vector: prepared (by the output
    // norm), or made here from `hidden` by every workgroup (the same
    // operations as k_q6k_xprep, so every workgroup gets the same copy; one
    // launch fewer)
    q6k_xhdr hdr;
    if (prep) {
        for (uint32_t i = threadIdx.x; i < n_blocks * 16 * 3; i += blockDim.x)
            reinterpret_cast<int4 *>(xq)[i] = reinterpret_cast<const int4 *>(prep)[i];
        hdr = *reinterpret_cast<const q6k_xhdr *>(prep + q6k_xq_bytes(n_blocks));
    } else {
        hdr = q6k_xprep_block(hidden, n_blocks, xq, red, redi);
    }
    __syncthreads();
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t r = lane >> 4, p = lane & 15;
    const q6_lane_offs o = q6_offs(n_blocks, r, p);
    const uint32_t group_bytes = q6k_group_bytes(n_blocks);
    const uint32_t g0 = (uint32_t)((uint64_t)blockIdx.x * n_rowgroups / gridDim.x);
    const uint32_t g1 = (uint32_t)((uint64_t)(blockIdx.x + 1) * n_rowgroups / gridDim.x);
    float lb_max = -INFINITY, ub_max = -INFINITY;
    constexpr uint32_t kWaves = kBoundedBlock / 64;
    auto epilogue = [&](uint32_t row, float acc, float sg) {
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) acc = acc + __shfl_xor(acc, o, 64);
        if (p == 0 && row < n_rows) {
            float a, eb;
            if (hdr.ok) {
                a = ldexpf(acc, hdr.e);
                eb = hdr.bound_k * sg;
                eb = eb + eb * 0x1p-20f + fabsf(a) * 0x1p-22f + 1e-35f;
                // terms this large could overflow in the reference's partial sums
                if (!(hdr.mag_k * sg < 1e37f)) eb = INFINITY;
            } else {
                a = NAN;
                eb = INFINITY;
            }
            approx[row] = a;
            bound[row] = eb;
            const float lb = a - eb, ub = a + eb;
            if (lb > lb_max) lb_max = lb;                            // NaN never raises it
            if (!(ub <= ub_max)) ub_max = ub == ub ? ub : INFINITY;  // NaN counts as +inf
        }
    };
    if (PIPE) {
        // Batches (group G, blocks bi*CH ..) in the order the wave takes them;
        // batch t+1's loads are in flight while batch t is reduced, in two
        // register sets used in turn (the loop body covers two batches, so no
        // set is ever copied).  The trip count is fixed before the loop and
        // the last batch is reduced after it, so every path into the loop
        // head has the same loads in flight and the wait for a batch never
        // covers the one issued after it (an exit between the two halves
        // would make the head's waits assume the other set still pending).
        // A row's sigma goes out before its batch, so reading it waits for no
        // weight bytes.
        const uint32_t nbat = n_blocks / CH;
        const uint32_t G0 = g0 + wave;
        if (G0 < g1) {
            const uint32_t total = (g1 - G0 + kWaves - 1) / kWaves * nbat;
            uint32_t G = G0, bi = 0;   // batch being reduced
            uint32_t Gn = G0, bn = 0;  // batch last issued
            q6_lane_blocks<CH> A, B;
            float sg = sigma[min(G0 * Q6K_GROUP_ROWS + r, n_rows - 1)], sg_n = sg;
            q6_load_uniform<CH>(A, wm_rsrc(w + (uint64_t)G0 * group_bytes, group_bytes), 0, o);
            float acc = 0.0f;
            // live = false: past the wave's last batch; the descriptor then
            // holds no records, so the loads return zeros without a memory
            // access (and the group index may run past g1)
            auto issue = [&](q6_lane_blocks<CH> &nxt, bool live) {
                if (++bn == nbat) {
                    bn = 0;
                    Gn += kWaves;
                }
                const uint32_t Gs = live ? Gn : G0;
                sg_n = sigma[min(Gs * Q6K_GROUP_ROWS + r, n_rows - 1)];
                q6_load_uniform<CH>(nxt, wm_rsrc(w + (uint64_t)Gs * group_bytes, live ? group_bytes : 0u),
                                    bn * CH, o);
                // keep the whole prefetch ahead of the reduction (the
                // scheduler would otherwise sink loads into it to save
                // registers)
                __builtin_amdgcn_sched_barrier(0);
            };
            auto reduce = [&](const q6_lane_blocks<CH> &cur) {
                q6_bounded_accum<CH>(cur, bi * CH, xq, p, acc);
                if (bi + 1 == nbat) {
                    epilogue(G * Q6K_GROUP_ROWS + r, acc, sg);
                    acc = 0.0f;
                    bi = 0;
                    G += kWaves;
                } else {
                    bi++;
                }
                __builtin_amdgcn_sched_barrier(0);  // one batch's registers live at a time
            };
            uint32_t t = 1;  // batches issued
            for (; t + 1 < total; t += 2) {
                issue(B, true);
                reduce(A);
                sg = sg_n;
                issue(A, true);
                reduce(B);
                sg = sg_n;
            }
            // the last one or two batches, on one code path
            const bool two = t < total;
            issue(B, two);
            reduce(A);
            sg = sg_n;
            if (two) reduce(B);
        }
    } else {
        for (uint32_t G = g0 + wave; G < g1; G += kWaves) {
            const __amdgpu_buffer_rsrc_t rs = wm_rsrc(w + (uint64_t)G * group_bytes, group_bytes);
            const uint32_t row = G * Q6K_GROUP_ROWS + r;
            const float sg = sigma[min(row, n_rows - 1)];
            float acc = 0.0f;
            for (uint32_t b0 = 0; b0 < n_blocks; b0 += CH) {
                q6_lane_blocks<CH> v;
                q6_load_uniform<CH>(v, rs, b0, o);
                q6_bounded_accum<CH>(v, b0, xq, p, acc);
            }
            epilogue(row, acc, sg);
        }
    }
    lb_max = wm_wave_max_nonan(lb_max);
    ub_max = wm_wave_max_nonan(ub_max);
    if (lane == 0) {
        red[wave] = lb_max;
        red2[wave] = ub_max;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float m = red[0], mu = red2[0];
        for (int i = 1; i < (int)kWaves; i++) {
            m = wm_max_nonan(m, red[i]);
            mu = wm_max_nonan(mu, red2[i]);
        }
        wg_lb[blockIdx.x] = m;
        wg_ub[blockIdx.x] = mu;
    }
}

// Selection, exact rescoring and the final argmax, in one workgroup.
// A row can hold the maximum only if its upper bound reaches the largest
// lower bound LB; every other row's reference logit is below LB, which is
// at most the reference logit of the row attaining it.  So: workgroups of
// the bounded pass whose largest upper bound reaches LB (and workgroup 0,
// for row 0, whose exact value the NaN rule reads) have their rows scanned;
// the rows that qualify are recomputed in the exact order (4 per wave pass)
// and their logits overwritten with the exact values; the first index of the
// maximum among them is the reference's argmax.  When a single row qualifies
// on its own bounds (the usual case), it is the argmax and no row is
// recomputed.  The global loads come in rounds: the workgroup bounds, the
// listed workgroups' rows, and only when rows are rescored, the hidden
// vector and their weights.
constexpr int kSelectBlock = 1024;
constexpr uint32_t kSelectCap = 2048;  // candidate rows held at once

template <int CH>
__device__ __forceinline__ void q6_select(
    const uint8_t *__restrict__ w, uint32_t n_blocks, uint32_t n_rows, uint32_t n_rowgroups,
    const float *__restrict__ hidden, float *__restrict__ logits, const float *__restrict__ bound,
    const float *__restrict__ wg_lb, const float *__restrict__ wg_ub, uint32_t n_wg,
    uint32_t *__restrict__ argmax_out, const wm_step_tail &tail) {
    extern __shared__ float xs[];  // [16][n_blocks*16 + 4]
    __shared__ uint32_t wg_r0[kBoundedMaxBlocks], wg_r1[kBoundedMaxBlocks];  // listed workgroups' rows
    __shared__ uint32_t cand[kSelectCap];
    __shared__ uint32_t n_wg_list, n_cand, n_real;
    __shared__ float red[kSelectBlock / 64];
    __shared__ argcand s_c[kSelectBlock / 64];
    __shared__ float s_f0;
    __shared__ bool s_q0, s_fin0;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // The workgroup bounds first (n_wg <= kBoundedMaxBlocks = 2 per thread).
    static_assert(kBoundedMaxBlocks <= 2 * kSelectBlock, "two workgroup bounds per thread");
    const uint32_t stride = xs_stride(n_blocks);
    float lbv[2], ubv[2];
#pragma unroll
    for (int k = 0; k < 2; k++) {
        const uint32_t i = tid + (uint32_t)k * kSelectBlock;
        lbv[k] = i < n_wg ? wg_lb[i] : -INFINITY;
        ubv[k] = i < n_wg ? wg_ub[i] : -INFINITY;
    }
    bool xs_ready = false;  // the hidden vector in lane order, loaded for the first rescoring
    if (tid == 0) {
        n_wg_list = 0;
        n_cand = 0;
        n_real = 0;
    }
    const float lb_max = wm_block_max_nonan(wm_max_nonan(lbv[0], lbv[1]), red);  // (also orders the writes above)
#pragma unroll
    for (int k = 0; k < 2; k++) {
        const uint32_t i = tid + (uint32_t)k * kSelectBlock;
        if (i < n_wg && (i == 0 || !(ubv[k] < lb_max))) {
            const uint32_t li = atomicAdd(&n_wg_list, 1u);
            wg_r0[li] = (uint32_t)((uint64_t)i * n_rowgroups / n_wg) * Q6K_GROUP_ROWS;
            wg_r1[li] = min((uint32_t)((uint64_t)(i + 1) * n_rowgroups / n_wg) * Q6K_GROUP_ROWS, n_rows);
        }
    }
    __syncthreads();
    // The rows of the listed workgroups, all at once: flat index f = li *
    // rpw + j is row r0(li) + j (rpw: the most rows a workgroup of the
    // bounded pass has), in passes of kSelectCap so the list cannot overflow.
    const uint32_t n_list = n_wg_list;
    const uint32_t rpw = (n_rowgroups + n_wg - 1) / n_wg * Q6K_GROUP_ROWS;
    const uint32_t total = n_list * rpw;
    const uint32_t slot = lane >> 4, L = lane & 15;
    const float *xl = xs + L * stride;
    float best_v = -INFINITY;
    uint32_t best_i = 0xFFFFFFFFu;
    // thread 0: the id out, and the greedy loop's ring slot and position
    const auto publish = [&](uint32_t id) {
        *argmax_out = id;
        if (tail.pos) {
            const uint32_t p = *tail.pos;
            if (tail.ring) {
                uint32_t *slot = tail.ring + 2 * (p & tail.ring_mask);
                slot[0] = id;
                slot[1] = *tail.err_flag;
                __threadfence_system();
            }
            *tail.pos = p + 1;
        }
    };
    for (uint32_t f0 = 0; f0 < total; f0 += kSelectCap) {
        for (uint32_t f = f0 + tid; f < min(f0 + kSelectCap, total); f += blockDim.x) {
            const uint32_t li = f / rpw;
            const uint32_t row = wg_r0[li] + (f - li * rpw), r1 = wg_r1[li];
            if (row < r1) {
                const float a = logits[row], b = bound[row];
                const bool q = !(a + b < lb_max);  // NaN qualifies
                if (row == 0) {
                    s_q0 = q;
                    s_fin0 = isfinite(a) && isfinite(b);
                }
                if (q || row == 0) cand[atomicAdd(&n_cand, 1u)] = row;
                if (q) atomicAdd(&n_real, 1u);
            }
        }
        __syncthreads();
        const uint32_t nc = n_cand;
        // One row qualifying on its own bounds (all rows in this pass): it is
        // the row attaining LB, whose logit is at least LB, and every other
        // row's is below LB, so it is the argmax and nothing is rescored.
        // Row 0 then only matters for the NaN rule, and finite bounds rule a
        // NaN logit out.
        if (total <= kSelectCap && n_real == 1 && s_fin0) {
            if (tid == 0) publish((cand[0] == 0 && !s_q0) ? cand[nc - 1] : cand[0]);
            return;
        }
        if (!xs_ready) {  // (uniform) xs[L*stride + b*16 + s] = x at b*256 + h*128 + k*32 +
                          // band*16 + c*4 + l, L = 4k + l, s = 4*(2h+band) + c
            for (uint32_t j = tid; j < n_blocks * 256; j += blockDim.x) {
                const uint32_t b = j >> 8, h = (j >> 7) & 1, k = (j >> 5) & 3, band = (j >> 4) & 1,
                               c = (j >> 2) & 3, l = j & 3;
                xs[(4 * k + l) * stride + b * 16 + (2 * h + band) * 4 + c] = hidden[j];
            }
            xs_ready = true;
            __syncthreads();
        }
        for (uint32_t c0 = wave * 4; c0 < nc; c0 += 4 * (kSelectBlock / 64)) {
            const uint32_t ci = min(c0 + slot, nc - 1);
            const uint32_t crow = cand[ci];
            const uint8_t *gbase = w + (uint64_t)(crow / Q6K_GROUP_ROWS) * q6k_group_bytes(n_blocks);
            const uint32_t rr = crow % Q6K_GROUP_ROWS;
            const q6_lane_offs o = q6_offs(n_blocks, rr, L);
            float acc = 0.0f;
            for (uint32_t b0 = 0; b0 < n_blocks; b0 += CH) {
                q6_lane_blocks<CH> v;
                q6_load_lane<CH>(v, gbase, b0, o);
                q6_exact_accum<CH>(v, b0, xl, acc);
            }
            const float dot = q6_combine(acc);
            if (L == 0 && c0 + slot < nc) {
                logits[crow] = dot;
                if (crow == 0) s_f0 = dot;
                if (cand_better(dot, crow, best_v, best_i)) {
                    best_v = dot;
                    best_i = crow;
                }
            }
        }
        __syncthreads();
        if (tid == 0) n_cand = 0;
        __syncthreads();
    }
    for (int o = 32; o > 0; o >>= 1) {
        float ov = __shfl_xor(best_v, o, 64);
        uint32_t oi = __shfl_xor(best_i, o, 64);
        if (cand_better(ov, oi, best_v, best_i)) {
            best_v = ov;
            best_i = oi;
        }
    }
    if (lane == 0) s_c[wave] = argcand{best_v, best_i};
    __syncthreads();
    if (tid == 0) {
        argcand bc = s_c[0];
        for (int i = 1; i < kSelectBlock / 64; i++)
            if (cand_better(s_c[i].v, s_c[i].i, bc.v, bc.i)) bc = s_c[i];
        // a NaN logit at index 0 wins (the reference's scan starts from
        // logits[0] and NaN compares false); all -inf/NaN keeps index 0
        publish((s_f0 != s_f0 || bc.i == 0xFFFFFFFFu) ? 0u : bc.i);
    }
}
template <int CH>
__global__ __launch_bounds__(kSelectBlock) void k_q6k_select(
    const uint8_t *__restrict__ w, uint32_t n_blocks, uint32_t n_rows, uint32_t n_rowgroups,
    const float *__restrict__ hidden, float *__restrict__ logits, const float *__restrict__ bound,
    const float *__restrict__ wg_lb, const float *__restrict__ wg_ub, uint32_t n_wg,
    uint32_t *__restrict__ argmax_out, wm_step_tail tail) {
    q6_select<CH>(w, n_blocks, n_rows, n_rowgroups, hidden, logits, bound, wg_lb, wg_ub, n_wg,
                  argmax_out, tail);
}

// ---------------------------------------------------------------------------
// the id-only lm-head of several hidden vectors at once (the ragged batch's
// next tokens): one bounded pass reads the table once for up to
// kMultiVec vectors, then one selection workgroup per vector
// ---------------------------------------------------------------------------
constexpr int kMultiVec = 4;
struct q6_multi {
    const float *hidden[kMultiVec];
    uint8_t *prep[kMultiVec];  // each vector's fixed-point copy and header
    float *approx[kMultiVec];  // [n_rows]: the bounded values, exact on rescored rows
    float *bound[kMultiVec];   // [n_rows]
    float *wg_lb[kMultiVec], *wg_ub[kMultiVec];  // [workgroups of the bounded pass]
    uint32_t *argmax_out[kMultiVec];
    int nv;
};
// vector v's entry of one of the arrays, by selects (no dynamic index into
// the argument block)
template <typename T>
__device__ __forceinline__ T q6_pick(const T (&arr)[kMultiVec], uint32_t v) {
    T r = arr[0];
#pragma unroll
    for (int i = 1; i < kMultiVec; i++) r = v == (uint32_t)i ? arr[i] : r;
    return r;
}

__global__ __launch_bounds__(256) void k_q6k_xprep_multi(q6_multi m, uint32_t n_blocks) {
    __shared__ float red[4];
    __shared__ int redi[4];
    const uint32_t v = blockIdx.x;
    uint8_t *prep = q6_pick(m.prep, v);
    const q6k_xhdr h = q6k_xprep_block(q6_pick(m.hidden, v), n_blocks, reinterpret_cast<q6k_xq *>(prep), red, redi);
    if (threadIdx.x == 0) *reinterpret_cast<q6k_xhdr *>(prep + q6k_xq_bytes(n_blocks)) = h;
}

template <int CH>
__global__ __launch_bounds__(kSelectBlock) void k_q6k_select_multi(
    const uint8_t *__restrict__ w, uint32_t n_blocks, uint32_t n_rows, uint32_t n_rowgroups,
    q6_multi m, uint32_t n_wg) {
    const uint32_t v = blockIdx.x;
    q6_select<CH>(w, n_blocks, n_rows, n_rowgroups, q6_pick(m.hidden, v), q6_pick(m.approx, v),
                  q6_pick(m.bound, v), q6_pick(m.wg_lb, v), q6_pick(m.wg_ub, v), n_wg,
                  q6_pick(m.argmax_out, v), wm_step_tail{});
}

// q6_bounded_accum for V vectors: each block's quants are unpacked once.
template <int CH, int V>
__device__ __forceinline__ void q6_bounded_accum_multi(const q6_lane_blocks<CH> &v, uint32_t b0,
                                                       const q6k_xq *xq, uint32_t xq_stride,
                                                       uint32_t p, float (&acc)[V]) {
#pragma unroll
    for (int j = 0; j < CH; j++) {
        uint32_t U[4];
        q6_unpack(v.w0[j], v.w1[j], v.w2[j], U);
        const float d = __half2float(__ushort_as_half((unsigned short)q6_d_bits(v, j)));
#pragma unroll
        for (int k = 0; k < V; k++) {
            const int4 *xp = reinterpret_cast<const int4 *>(xq + k * xq_stride + (b0 + j) * 16 + p);
            const int4 h4 = xp[0], l4 = xp[1], c4 = xp[2];
            const int xh[4] = {h4.x, h4.y, h4.z, h4.w}, xl[4] = {l4.x, l4.y, l4.z, l4.w},
                      xc[4] = {c4.x, c4.y, c4.z, c4.w};
            int T = 0;
#pragma unroll
            for (int hn = 0; hn < 4; hn++) {
                const int sc = (int)(int8_t)(v.scw[j] >> (8 * hn));
                const int dh = __builtin_amdgcn_sdot4((int)U[hn], xh[hn], 0, true);
                const int dl = __builtin_amdgcn_sdot4((int)U[hn], xl[hn], xc[hn], false);
                const int I = (int)(((uint32_t)dh << 8) + (uint32_t)dl);  // a VALU result
                T = mad_i24(sc, I, T);
            }
            acc[k] = __builtin_fmaf(d, (float)T, acc[k]);
        }
    }
}

// The bounded pass of k_q6k_bounded (pipelined) for V vectors at once: the
// same batches, rows, bounds and per-workgroup maxima, per vector.
template <int CH, int V>
__global__ __launch_bounds__(kBoundedBlock) void k_q6k_bounded_multi(
    const uint8_t *__restrict__ w, uint32_t n_blocks, uint32_t n_rows, uint32_t n_rowgroups,
    const float *__restrict__ sigma, q6_multi m) {
    extern __shared__ __align__(16) q6k_xq xq[];  // [V][n_blocks][16]
    __shared__ float red[V][kBoundedBlock / 64], red2[V][kBoundedBlock / 64];
    const uint32_t xq_stride = n_blocks * 16;
    q6k_xhdr hdr[V];
#pragma unroll
    for (int k = 0; k < V; k++) {
        const uint8_t *prep = m.prep[k];
        for (uint32_t i = threadIdx.x; i < n_blocks * 16 * 3; i += blockDim.x)
            reinterpret_cast<int4 *>(xq + k * xq_stride)[i] = reinterpret_cast<const int4 *>(prep)[i];
        hdr[k] = *reinterpret_cast<const q6k_xhdr *>(prep + q6k_xq_bytes(n_blocks));
    }
    __syncthreads();
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t r = lane >> 4, p = lane & 15;
    const q6_lane_offs o = q6_offs(n_blocks, r, p);
    const uint32_t group_bytes = q6k_group_bytes(n_blocks);
    const uint32_t g0 = (uint32_t)((uint64_t)blockIdx.x * n_rowgroups / gridDim.x);
    const uint32_t g1 = (uint32_t)((uint64_t)(blockIdx.x + 1) * n_rowgroups / gridDim.x);
    float lb_max[V], ub_max[V];
#pragma unroll
    for (int k = 0; k < V; k++) lb_max[k] = ub_max[k] = -INFINITY;
    constexpr uint32_t kWaves = kBoundedBlock / 64;
    auto epilogue = [&](uint32_t row, float (&acc)[V], float sg) __attribute__((always_inline)) {
#pragma unroll
        for (int k = 0; k < V; k++) {
            float a_ = acc[k];
#pragma unroll
            for (int o2 = 1; o2 < 16; o2 <<= 1) a_ = a_ + __shfl_xor(a_, o2, 64);
            if (p == 0 && row < n_rows) {
                float a, eb;
                if (hdr[k].ok) {
                    a = ldexpf(a_, hdr[k].e);
                    eb = hdr[k].bound_k * sg;
                    eb = eb + eb * 0x1p-20f + fabsf(a) * 0x1p-22f + 1e-35f;
                    if (!(hdr[k].mag_k * sg < 1e37f)) eb = INFINITY;
                } else {
                    a = NAN;
                    eb = INFINITY;
                }
                m.approx[k][row] = a;
                m.bound[k][row] = eb;
                const float lb = a - eb, ub = a + eb;
                if (lb > lb_max[k]) lb_max[k] = lb;
                if (!(ub <= ub_max[k])) ub_max[k] = ub == ub ? ub : INFINITY;
            }
        }
    };
    const uint32_t nbat = n_blocks / CH;
    const uint32_t G0 = g0 + wave;
    if (G0 < g1) {
        const uint32_t total = (g1 - G0 + kWaves - 1) / kWaves * nbat;
        uint32_t G = G0, bi = 0;
        uint32_t Gn = G0, bn = 0;
        q6_lane_blocks<CH> A, B;
        float sg = sigma[min(G0 * Q6K_GROUP_ROWS + r, n_rows - 1)], sg_n = sg;
        q6_load_uniform<CH>(A, wm_rsrc(w + (uint64_t)G0 * group_bytes, group_bytes), 0, o);
        float acc[V];
#pragma unroll
        for (int k = 0; k < V; k++) acc[k] = 0.0f;
        auto issue = [&](q6_lane_blocks<CH> &nxt, bool live) __attribute__((always_inline)) {
            if (++bn == nbat) {
                bn = 0;
                Gn += kWaves;
            }
            const uint32_t Gs = live ? Gn : G0;
            sg_n = sigma[min(Gs * Q6K_GROUP_ROWS + r, n_rows - 1)];
            q6_load_uniform<CH>(nxt, wm_rsrc(w + (uint64_t)Gs * group_bytes, live ? group_bytes : 0u),
                                bn * CH, o);
            __builtin_amdgcn_sched_barrier(0);
        };
        auto reduce = [&](const q6_lane_blocks<CH> &cur) __attribute__((always_inline)) {
            q6_bounded_accum_multi<CH, V>(cur, bi * CH, xq, xq_stride, p, acc);
            if (bi + 1 == nbat) {
                epilogue(G * Q6K_GROUP_ROWS + r, acc, sg);
#pragma unroll
                for (int k = 0; k < V; k++) acc[k] = 0.0f;
                bi = 0;
                G += kWaves;
            } else {
                bi++;
            }
            __builtin_amdgcn_sched_barrier(0);
        };
        uint32_t t = 1;
        for (; t + 1 < total; t += 2) {
            issue(B, true);
            reduce(A);
            sg = sg_n;
            issue(A, true);
            reduce(B);
            sg = sg_n;
        }
        const bool two = t < total;
        issue(B, two);
        reduce(A);
        sg = sg_n;
        if (two) reduce(B);
    }
#pragma unroll
    for (int k = 0; k < V; k++) {
        const float a1 = wm_wave_max_nonan(lb_max[k]), a2 = wm_wave_max_nonan(ub_max[k]);
        if (lane == 0) {
            red[k][wave] = a1;
            red2[k][wave] = a2;
        }
    }
    __syncthreads();
    if (threadIdx.x < (uint32_t)V) {
        const uint32_t k = threadIdx.x;
        float mm = red[k][0], mu = red2[k][0];
        for (int i = 1; i < (int)kWaves; i++) {
            mm = wm_max_nonan(mm, red[k][i]);
            mu = wm_max_nonan(mu, red2[k][i]);
        }
        q6_pick(m.wg_lb, k)[blockIdx.x] = mm;
        q6_pick(m.wg_ub, k)[blockIdx.x] = mu;
    }
}

int pick_ch(uint32_t n_blocks) {
    for (int ch : {10, 8, 5, 4, 2})
        if (n_blocks % ch == 0) return ch;
    return 1;
}

// Work buffer layout (all offsets 256-aligned).
struct work_layout {
    size_t cands, bound, wg_lb, wg_ub, prep, total;
};
size_t al256(size_t v) { return (v + 255) & ~(size_t)255; }
work_layout layout_of(uint32_t n_rows, uint32_t n_blocks) {
    work_layout l;
    size_t o = 0;
    l.cands = o; o += al256(sizeof(argcand) * kMaxArgBlocks);
    l.bound = o; o += al256((size_t)n_rows * 4);
    l.wg_lb = o; o += al256(4 * kBoundedMaxBlocks);
    l.wg_ub = o; o += al256(4 * kBoundedMaxBlocks);
    l.prep = o; o += q6k_prep_bytes(n_blocks);
    l.total = o;
    return l;
}

// Workgroups of the bounded pass: as many as fit on the device at once (one
// round, each with a contiguous range of row groups), at most one per 4 groups.
template <int CH, bool PIPE>
uint32_t bounded_blocks_for(uint32_t n_rowgroups, size_t lds) {
    static int cached[16] = {0};  // per device, per instantiation
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = 0;
    int per = dev < 16 ? cached[dev] : 0;
    if (per == 0) {
        int occ = 0, cus = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, k_q6k_bounded<CH, PIPE>, kBoundedBlock, lds) != hipSuccess || occ < 1)
            occ = 1;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1)
            cus = 256;
        per = occ * cus;
        if (dev < 16) cached[dev] = per;
    }
    uint32_t blocks = (n_rowgroups + 3) / 4;
    if (blocks > (uint32_t)per) blocks = (uint32_t)per;
    if (blocks > kBoundedMaxBlocks) blocks = kBoundedMaxBlocks;
    return blocks ? blocks : 1;
}

template <int CH>
uint32_t launch_bounded_ch(const uint8_t *w, uint32_t n_blocks, uint32_t n_rows,
                           uint32_t n_rowgroups, const uint8_t *prep, const float *hidden, float *approx,
                           float *bound, float *wg_lb, float *wg_ub, hipStream_t s) {
    const size_t lds = sizeof(q6k_xq) * 16 * n_blocks;
    const float *sigma = reinterpret_cast<const float *>(w + wm_q6k_sigma_offset(n_rowgroups, n_blocks));
    if (kPipelined) {
        const uint32_t blocks = bounded_blocks_for<CH, true>(n_rowgroups, lds);
        hipLaunchKernelGGL((k_q6k_bounded<CH, true>), dim3(blocks), dim3(kBoundedBlock), lds, s, w,
                           n_blocks, n_rows, n_rowgroups, sigma, prep, hidden, approx, bound, wg_lb, wg_ub);
        return blocks;
    }
    const uint32_t blocks = bounded_blocks_for<CH, false>(n_rowgroups, lds);
    hipLaunchKernelGGL((k_q6k_bounded<CH, false>), dim3(blocks), dim3(kBoundedBlock), lds, s, w,
                       n_blocks, n_rows, n_rowgroups, sigma, prep, hidden, approx, bound, wg_lb, wg_ub);
    return blocks;
}

template <int CH>
void launch_argmax_fast_ch(const uint8_t *w, uint32_t n_blocks, uint32_t n_rows,
                           uint32_t n_rowgroups, const float *hidden, float *logits,
                           uint32_t *argmax_out, void *work, bool prepared, hipStream_t s,
                           const wm_step_tail &tail) {
    const work_layout lay = layout_of(n_rows, n_blocks);
    uint8_t *wb = (uint8_t *)work;
    float *bound = reinterpret_cast<float *>(wb + lay.bound);
    float *wg_lb = reinterpret_cast<float *>(wb + lay.wg_lb);
    float *wg_ub = reinterpret_cast<float *>(wb + lay.wg_ub);
    const uint32_t n_wg = launch_bounded_ch<CH>(w, n_blocks, n_rows, n_rowgroups,
                                                prepared ? wb + lay.prep : nullptr, hidden,
                                                logits, bound, wg_lb, wg_ub, s);
    const size_t lds = sizeof(float) * 16 * xs_stride(n_blocks);
    hipLaunchKernelGGL(k_q6k_select<CH>, dim3(1), dim3(kSelectBlock), lds, s, w, n_blocks, n_rows,
                       n_rowgroups, hidden, logits, bound, wg_lb, wg_ub, n_wg, argmax_out, tail);
}

// The multi-vector work area: per vector slot, its prep area, the bounded
// values and bounds, and the per-workgroup maxima.
struct multi_layout {
    size_t prep, approx, bound, wg_lb, wg_ub, slot;
};
multi_layout multi_layout_of(uint32_t n_rows, uint32_t n_blocks) {
    multi_layout l;
    size_t o = 0;
    l.prep = o; o += al256(q6k_prep_bytes(n_blocks));
    l.approx = o; o += al256((size_t)n_rows * 4);
    l.bound = o; o += al256((size_t)n_rows * 4);
    l.wg_lb = o; o += al256(4 * kBoundedMaxBlocks);
    l.wg_ub = o; o += al256(4 * kBoundedMaxBlocks);
    l.slot = o;
    return l;
}

template <int CH>
uint32_t bounded_multi_blocks_for(uint32_t n_rowgroups, size_t lds) {
    static int cached[16] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = 0;
    int per = dev < 16 ? cached[dev] : 0;
    if (per == 0) {
        int occ = 0, cus = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, k_q6k_bounded_multi<CH, kMultiVec>, kBoundedBlock, lds) !=
                hipSuccess || occ < 1)
            occ = 1;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1)
            cus = 256;
        per = occ * cus;
        if (dev < 16) cached[dev] = per;
    }
    uint32_t blocks = (n_rowgroups + 3) / 4;
    if (blocks > (uint32_t)per) blocks = (uint32_t)per;
    if (blocks > kBoundedMaxBlocks) blocks = kBoundedMaxBlocks;
    return blocks ? blocks : 1;
}

// Up to kMultiVec vectors per pass over the table; a group with fewer
// fills its empty slots with the last vector's prep area (their results go
// to the slots' own areas and are not read).
template <int CH>
void launch_argmax_multi_ch(const uint8_t *w, uint32_t n_blocks, uint32_t n_rows, uint32_t n_rowgroups,
                            const float *hidden, uint32_t ld, const uint32_t *rows, uint32_t n_vec,
                            uint32_t *argmax_out, void *work, hipStream_t s) {
    const multi_layout lay = multi_layout_of(n_rows, n_blocks);
    const float *sigma = reinterpret_cast<const float *>(w + wm_q6k_sigma_offset(n_rowgroups, n_blocks));
    const size_t lds = sizeof(q6k_xq) * 16 * n_blocks * kMultiVec;
    const uint32_t blocks = bounded_multi_blocks_for<CH>(n_rowgroups, lds);
    const size_t sel_lds = sizeof(float) * 16 * xs_stride(n_blocks);
    for (uint32_t v0 = 0; v0 < n_vec; v0 += kMultiVec) {
        const int nv = (int)min((uint32_t)kMultiVec, n_vec - v0);
        q6_multi m{};
        m.nv = nv;
        for (int k = 0; k < kMultiVec; k++) {
            uint8_t *slot = (uint8_t *)work + (size_t)k * lay.slot;
            const int kr = k < nv ? k : nv - 1;  // an empty slot reads the last vector
            m.hidden[k] = hidden + (size_t)rows[v0 + kr] * ld;
            m.prep[k] = (uint8_t *)work + (size_t)kr * lay.slot + lay.prep;
            m.approx[k] = reinterpret_cast<float *>(slot + lay.approx);
            m.bound[k] = reinterpret_cast<float *>(slot + lay.bound);
            m.wg_lb[k] = reinterpret_cast<float *>(slot + lay.wg_lb);
            m.wg_ub[k] = reinterpret_cast<float *>(slot + lay.wg_ub);
            m.argmax_out[k] = argmax_out + v0 + kr;
        }
        hipLaunchKernelGGL(k_q6k_xprep_multi, dim3(nv), dim3(256), 0, s, m, n_blocks);
        hipLaunchKernelGGL((k_q6k_bounded_multi<CH, kMultiVec>), dim3(blocks), dim3(kBoundedBlock), lds, s, w,
                           n_blocks, n_rows, n_rowgroups, sigma, m);
        hipLaunchKernelGGL(k_q6k_select_multi<CH>, dim3(nv), dim3(kSelectBlock), sel_lds, s, w, n_blocks,
                           n_rows, n_rowgroups, m, blocks);
    }
}

}  // namespace

size_t wm_q6k_multi_work_bytes(uint32_t n_rows, uint32_t n_blocks) {
    return (size_t)kMultiVec * multi_layout_of(n_rows, n_blocks).slot;
}

void wm_launch_q6k_argmax_multi(const uint8_t *w, uint32_t n_blocks, uint32_t n_rows, uint32_t n_rowgroups,
                                const float *hidden, uint32_t ld, const uint32_t *rows, uint32_t n_vec,
                                uint32_t *argmax_out, void *work, hipStream_t s) {
#define WM_M_CASE(C)                                                                               \
    case C:                                                                                        \
        launch_argmax_multi_ch<C>(w, n_blocks, n_rows, n_rowgroups, hidden, ld, rows, n_vec,       \
                                  argmax_out, work, s);                                            \
        break;
    switch (pick_ch(n_blocks)) {
        WM_M_CASE(10) WM_M_CASE(8) WM_M_CASE(5) WM_M_CASE(4) WM_M_CASE(2) default: WM_M_CASE(1)
    }
#undef WM_M_CASE
}

void wm_launch_q6k_repack(const uint8_t *raw, uint8_t *out, uint32_t n_rows, uint32_t n_blocks,
                          uint32_t n_rowgroups, hipStream_t s) {
    uint64_t total = (uint64_t)n_rowgroups * n_blocks * Q6K_GROUP_ROWS;
    uint32_t blocks = (uint32_t)((total + 255) / 256);
    if (blocks > 65535u * 4) blocks = 65535u * 4;
    hipLaunchKernelGGL(k_q6k_repack, dim3(blocks), dim3(256), 0, s, raw, out, n_rows, n_blocks,
                       n_rowgroups);
    float *sigma = reinterpret_cast<float *>(out + wm_q6k_sigma_offset(n_rowgroups, n_blocks));
    hipLaunchKernelGGL(k_q6k_row_sigma, dim3((n_rows + 255) / 256), dim3(256), 0, s, raw, n_rows,
                       n_blocks, sigma);
}

void wm_launch_q6k_dequant_row(const uint8_t *w, uint32_t n_blocks, uint32_t row, float *out,
                               hipStream_t s) {
    hipLaunchKernelGGL(k_q6k_dequant_row, dim3(n_blocks), dim3(256), 0, s, w, n_blocks, row,
                       (const uint32_t *)nullptr, out, 0u);
}

void wm_launch_q6k_dequant_row_dev(const uint8_t *w, uint32_t n_blocks, const uint32_t *d_row,
                                   float *out, hipStream_t s) {
    hipLaunchKernelGGL(k_q6k_dequant_row, dim3(n_blocks), dim3(256), 0, s, w, n_blocks, 0u, d_row,
                       out, 0u);
}

void wm_launch_q6k_dequant_rows_dev(const uint8_t *w, uint32_t n_blocks, const uint32_t *d_rows,
                                    uint32_t n_rows, float *out, uint32_t ld, hipStream_t s) {
    hipLaunchKernelGGL(k_q6k_dequant_row, dim3(n_blocks, n_rows), dim3(256), 0, s, w, n_blocks, 0u,
                       d_rows, out, ld);
}

size_t wm_q6k_logits_work_bytes(uint32_t n_rows, uint32_t n_blocks) {
    return layout_of(n_rows, n_blocks).total;
}

void *wm_q6k_prep_area(void *work, uint32_t n_rows, uint32_t n_blocks) {
    return (uint8_t *)work + layout_of(n_rows, n_blocks).prep;
}

// Exact logits (bit-identical to the reference) + optional argmax.  The
// logits buffer is required: the final argmax step reads logits[0] for the
// NaN rule.
void wm_launch_q6k_logits_argmax(const uint8_t *w, uint32_t n_blocks, uint32_t n_rows,
                                 uint32_t n_rowgroups, const float *hidden, float *logits,
                                 uint32_t *argmax_out, void *work, hipStream_t s) {
    uint32_t blocks = (n_rowgroups + 3) / 4;
    const uint32_t max_blocks = 256 * 6;  // 24 waves per CU
    if (blocks > max_blocks) blocks = max_blocks;
    if (blocks == 0) blocks = 1;
    const size_t lds = sizeof(float) * 16 * (n_blocks * 16 + 4);
    argcand *cands = reinterpret_cast<argcand *>((uint8_t *)work + layout_of(n_rows, n_blocks).cands);
#define WM_LOGITS_CASE(C)                                                                           \
    case C:                                                                                         \
        hipLaunchKernelGGL(k_q6k_logits<C>, dim3(blocks), dim3(kLogitsBlock), lds, s, w, n_blocks, \
                           n_rows, n_rowgroups, hidden, logits, cands);                             \
        break;
    switch (pick_ch(n_blocks)) {
        WM_LOGITS_CASE(10) WM_LOGITS_CASE(8) WM_LOGITS_CASE(5) WM_LOGITS_CASE(4)
        WM_LOGITS_CASE(2) default: WM_LOGITS_CASE(1)
    }
#undef WM_LOGITS_CASE
    if (argmax_out)
        hipLaunchKernelGGL(k_argmax_final, dim3(1), dim3(64), 0, s, cands, blocks, logits,
                           argmax_out);
}

// Argmax only: the bounded pass, then selection + exact rescoring + argmax
// in one workgroup.  `logits` (n_rows floats) receives the bounded pass's
// values, exact on the rows that were rescored (always including row 0).
// prepared: the work buffer's prep area already holds `hidden` in fixed
// point (written by the kernel that produced it).
void wm_launch_q6k_argmax_fast(const uint8_t *w, uint32_t n_blocks, uint32_t n_rows,
                               uint32_t n_rowgroups, const float *hidden, float *logits,
                               uint32_t *argmax_out, void *work, bool prepared, hipStream_t s,
                               const wm_step_tail *tail) {
    const wm_step_tail t = tail ? *tail : wm_step_tail{};
#define WM_F_CASE(C)                                                                               \
    case C:                                                                                        \
        launch_argmax_fast_ch<C>(w, n_blocks, n_rows, n_rowgroups, hidden, logits, argmax_out,    \
                                 work, prepared, s, t);                                            \
        break;
    switch (pick_ch(n_blocks)) {
        WM_F_CASE(10) WM_F_CASE(8) WM_F_CASE(5) WM_F_CASE(4) WM_F_CASE(2) default: WM_F_CASE(1)
    }
#undef WM_F_CASE
}

// Test hook / measurement: the bounded pass alone (approximate logits and
// their bounds), after the fixed-point prep of `hidden` unless `prepared`.
void wm_launch_q6k_bounded_only(const uint8_t *w, uint32_t n_blocks, uint32_t n_rows,
                                uint32_t n_rowgroups, const float *hidden, float *approx,
                                float *bound_out, void *work, bool prepared, hipStream_t s) {
    const work_layout lay = layout_of(n_rows, n_blocks);
    uint8_t *wb = (uint8_t *)work;
    float *wg_lb = reinterpret_cast<float *>(wb + lay.wg_lb);
    float *wg_ub = reinterpret_cast<float *>(wb + lay.wg_ub);
    if (!prepared)
        hipLaunchKernelGGL(k_q6k_xprep, dim3(1), dim3(256), 0, s, hidden, n_blocks, wb + lay.prep);
#define WM_B_CASE(C)                                                                               \
    case C:                                                                                        \
        launch_bounded_ch<C>(w, n_blocks, n_rows, n_rowgroups, wb + lay.prep, hidden, approx,     \
                             bound_out, wg_lb, wg_ub, s);                                          \
        break;
    switch (pick_ch(n_blocks)) {
        WM_B_CASE(10) WM_B_CASE(8) WM_B_CASE(5) WM_B_CASE(4) WM_B_CASE(2) default: WM_B_CASE(1)
    }
#undef WM_B_CASE
}

void wm_launch_q6k_xprep(const float *hidden, uint32_t n_blocks, void *work, uint32_t n_rows,
                         hipStream_t s) {
    hipLaunchKernelGGL(k_q6k_xprep, dim3(1), dim3(256), 0, s, hidden, n_blocks,
                       (uint8_t *)work + layout_of(n_rows, n_blocks).prep);
}
