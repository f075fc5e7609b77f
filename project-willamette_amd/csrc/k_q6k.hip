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
// The lm-head kernel gives each of those 16 partial sums to its own lane, so
// a wave computes 4 rows with exactly the reference's roundings.
//
// Device layout (k_q6k_repack): rows in groups of 4; per (group, block) 840
// bytes: for lane L' = 16*row + 4k + l the 16 six-bit quants it consumes in
// this block, packed into 3 dwords (step s at bits 6s..6s+5); then per row
// the 16 sub-scales as 4 dwords (dword k, byte 2h+band = sc[8h + band + 2k]);
// then the 4 f16 d values.  Same byte count as the GGUF tensor.
#include "wm_internal.h"

namespace {

constexpr int kLogitsBlock = 256;  // 4 waves
constexpr int kMaxArgBlocks = 2048;

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
        uint8_t *dst = out + gb * Q6K_GROUP_BLOCK_BYTES;
        uint32_t *q6 = reinterpret_cast<uint32_t *>(dst);
        uint32_t *scw = reinterpret_cast<uint32_t *>(dst + Q6K_SC_OFFSET);
        uint16_t *dw = reinterpret_cast<uint16_t *>(dst + Q6K_D_OFFSET);
        if (row >= n_rows) {
            for (int L = 0; L < 16; L++)
                for (int j = 0; j < 3; j++) q6[(r * 16 + L) * 3 + j] = 0;
            for (int k = 0; k < 4; k++) scw[r * 4 + k] = 0;
            dw[r] = 0;
            continue;
        }
        const uint8_t *blk = raw + (row * n_blocks + b) * Q6K_BYTES;
        for (int k = 0; k < 4; k++) {
            for (int l = 0; l < 4; l++) {
                uint32_t w[3] = {0, 0, 0};
                for (int s = 0; s < 16; s++) {
                    int hn = s >> 2, c = s & 3, h = hn >> 1, n = hn & 1;
                    uint32_t v = (uint32_t)q6_of(blk, h, k, n * 16 + c * 4 + l);
                    int bit = 6 * s;
                    w[bit >> 5] |= v << (bit & 31);
                    if ((bit & 31) > 26) w[(bit >> 5) + 1] |= v >> (32 - (bit & 31));
                }
                int L = r * 16 + k * 4 + l;
                q6[L * 3 + 0] = w[0]; q6[L * 3 + 1] = w[1]; q6[L * 3 + 2] = w[2];
            }
            uint32_t sc = 0;
            for (int hn = 0; hn < 4; hn++) {
                int h = hn >> 1, n = hn & 1;
                sc |= (uint32_t)blk[192 + h * 8 + n + 2 * k] << (8 * hn);
            }
            scw[r * 4 + k] = sc;
        }
        dw[r] = (uint16_t)(blk[208] | (blk[209] << 8));
    }
}

__device__ __forceinline__ uint32_t q6_step(uint32_t w0, uint32_t w1, uint32_t w2, int s) {
    int bit = 6 * s;
    uint32_t lo = bit < 32 ? w0 : (bit < 64 ? w1 : w2);
    uint32_t hi = bit < 32 ? w1 : w2;
    int sh = bit & 31;
    uint32_t v = sh ? ((lo >> sh) | (hi << (32 - sh))) : lo;
    return v & 63u;
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
    const uint8_t *base = w + ((uint64_t)G * n_blocks + b) * Q6K_GROUP_BLOCK_BYTES;
    const int h = t >> 7, k = (t >> 5) & 3, n = (t >> 4) & 1, c = (t >> 2) & 3, l = t & 3;
    const int L = r * 16 + k * 4 + l, s = (h * 2 + n) * 4 + c;
    const uint32_t *q6 = reinterpret_cast<const uint32_t *>(base) + L * 3;
    const uint32_t q = q6_step(q6[0], q6[1], q6[2], s);
    const uint32_t scw = reinterpret_cast<const uint32_t *>(base + Q6K_SC_OFFSET)[r * 4 + k];
    const int sc = (int)(int8_t)(scw >> (8 * (h * 2 + n)));
    const float d = wm_f16_bits_to_f32(reinterpret_cast<const uint16_t *>(base + Q6K_D_OFFSET)[r]);
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

__global__ __launch_bounds__(kLogitsBlock) void k_q6k_logits(
    const uint8_t *__restrict__ w, uint32_t n_blocks, uint32_t n_rows, uint32_t n_rowgroups,
    const float *__restrict__ hidden, float *__restrict__ logits, argcand *__restrict__ cands) {
    extern __shared__ float xs[];  // [16][n_blocks*16 + 4]
    const uint32_t stride = n_blocks * 16 + 4;
    // permute the hidden vector into lane order: lane L = 4k + l, step s of block b
    for (uint32_t idx = threadIdx.x; idx < 16u * n_blocks * 16u; idx += blockDim.x) {
        uint32_t L = idx / (n_blocks * 16), rem = idx % (n_blocks * 16);
        uint32_t b = rem / 16, s = rem % 16;
        uint32_t k = L >> 2, l = L & 3, hn = s >> 2, c = s & 3, h = hn >> 1, n = hn & 1;
        xs[L * stride + b * 16 + s] = hidden[b * 256 + h * 128 + k * 32 + n * 16 + c * 4 + l];
    }
    __syncthreads();
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t r = lane >> 4, L = lane & 15, k = L >> 2;
    const float *xl = xs + L * stride;
    float best_v = -INFINITY;
    uint32_t best_i = 0xFFFFFFFFu;
    const uint32_t waves_total = gridDim.x * (blockDim.x >> 6);
    for (uint32_t G = blockIdx.x * (blockDim.x >> 6) + wave; G < n_rowgroups; G += waves_total) {
        const uint8_t *gbase = w + (uint64_t)G * n_blocks * Q6K_GROUP_BLOCK_BYTES;
        float acc = 0.0f;
        for (uint32_t b = 0; b < n_blocks; b++) {
            const uint8_t *base = gbase + (uint64_t)b * Q6K_GROUP_BLOCK_BYTES;
            const uint32_t *q6 = reinterpret_cast<const uint32_t *>(base) + lane * 3;
            const uint32_t w0 = wm_load_stream_u32(q6), w1 = wm_load_stream_u32(q6 + 1),
                           w2 = wm_load_stream_u32(q6 + 2);
            const uint32_t scw =
                wm_load_stream_u32(reinterpret_cast<const uint32_t *>(base + Q6K_SC_OFFSET) + r * 4 + k);
            const float d =
                wm_f16_bits_to_f32(reinterpret_cast<const uint16_t *>(base + Q6K_D_OFFSET)[r]);
            const float *xb = xl + b * 16;
            if (__builtin_expect(isfinite(d), 1)) {
#pragma unroll
                for (int hn = 0; hn < 4; hn++) {
                    const float S = d * (float)(int)(int8_t)(scw >> (8 * hn));
                    const float nS32 = -32.0f * S;
#pragma unroll
                    for (int c = 0; c < 4; c++) {
                        const int s = hn * 4 + c;
                        // (q6 - 32) * S is exact in f32, so the fused form equals the
                        // reference's rounded product q * (d*sc).
                        const float qS = __builtin_fmaf((float)q6_step(w0, w1, w2, s), S, nS32);
                        acc = acc + qS * xb[s];
                    }
                }
            } else {
                for (int hn = 0; hn < 4; hn++) {
                    const float S = d * (float)(int)(int8_t)(scw >> (8 * hn));
                    for (int c = 0; c < 4; c++) {
                        const int s = hn * 4 + c;
                        const float qS = (float)((int)q6_step(w0, w1, w2, s) - 32) * S;
                        acc = acc + qS * xb[s];
                    }
                }
            }
        }
        // v_l = (p0l + p1l) + (p2l + p3l); dot = (v0 + v3) + (v1 + v2)
        float t = acc + __shfl_xor(acc, 4, 64);
        float v = t + __shfl_xor(t, 8, 64);
        float u = v + __shfl_xor(v, 3, 64);
        float dot = u + __shfl_xor(u, 1, 64);
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

}  // namespace

void wm_launch_q6k_repack(const uint8_t *raw, uint8_t *out, uint32_t n_rows, uint32_t n_blocks,
                          uint32_t n_rowgroups, hipStream_t s) {
    uint64_t total = (uint64_t)n_rowgroups * n_blocks * Q6K_GROUP_ROWS;
    uint32_t blocks = (uint32_t)((total + 255) / 256);
    if (blocks > 65535u * 4) blocks = 65535u * 4;
    hipLaunchKernelGGL(k_q6k_repack, dim3(blocks), dim3(256), 0, s, raw, out, n_rows, n_blocks,
                       n_rowgroups);
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

size_t wm_q6k_logits_work_bytes() { return sizeof(argcand) * kMaxArgBlocks + 256; }

// `work` holds the per-block candidates.  When logits == nullptr the first
// logit is still needed for the NaN rule: the caller always passes a logits
// buffer (the library keeps one per context/model).
void wm_launch_q6k_logits_argmax(const uint8_t *w, uint32_t n_blocks, uint32_t n_rows,
                                 uint32_t n_rowgroups, const float *hidden, float *logits,
                                 uint32_t *argmax_out, void *work, hipStream_t s) {
    uint32_t waves = 256 * 8;  // 8 waves per CU
    uint32_t blocks = (n_rowgroups + 3) / 4;
    uint32_t max_blocks = waves / 4;
    if (blocks > max_blocks) blocks = max_blocks;
    if (blocks > (uint32_t)kMaxArgBlocks) blocks = kMaxArgBlocks;
    if (blocks == 0) blocks = 1;
    size_t lds = sizeof(float) * 16 * (n_blocks * 16 + 4);
    argcand *cands = reinterpret_cast<argcand *>(work);
    hipLaunchKernelGGL(k_q6k_logits, dim3(blocks), dim3(kLogitsBlock), lds, s, w, n_blocks,
                       n_rows, n_rowgroups, hidden, logits, cands);
    if (argmax_out)
        hipLaunchKernelGGL(k_argmax_final, dim3(1), dim3(64), 0, s, cands, blocks, logits,
                           argmax_out);
}
