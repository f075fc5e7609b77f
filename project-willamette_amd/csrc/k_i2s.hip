// BitLinear I2_S kernels for gfx950.
//
// Reference semantics (project-willamette):
//   quantise   src/model/bitlinear_sse2.rs:285-304   (per-vector absmax int8)
//   code map   src/model/bitlinear.rs:43-50          (00->-1, 01->0, 10->+1, 11->0)
//   byte map   src/model/bitlinear_sse2.rs:183-193   (byte gp of a 32-byte block holds
//                                                     columns gp, 32+gp, 64+gp, 96+gp
//                                                     in bits 7:6, 5:4, 3:2, 1:0)
//   dot/epilog src/model/bitlinear_sse2.rs:313-342   (i32 dot; out = (w_scale*in_scale)*dot)
//
// Device weight layout (written once at upload by k_i2s_repack): rows are
// grouped 64 at a time; for group g and 16-byte chunk c (columns
// [64c, 64c+64) of the I2_S block structure) the 64 rows' chunks are
// contiguous, so one wave loads 1 KiB per instruction with lane r reading
// row 64g+r.  Code 11 is rewritten to 01 (both mean 0) so that a code can be
// used directly as the unsigned value c = ternary + 1.
//
// The matvec computes, per row, sum(c * a) with v_dot4_i32_i8 and the
// activations broadcast from SGPRs (every lane of a wave needs the same 64
// activation bytes for a chunk), then subtracts sum(a):
//   sum(ternary * a) = sum((c - 1) * a) = sum(c * a) - sum(a).
// Integer sums are exact, so the K-split, lane order and block order do not
// change the i32 result the reference produces.
#include "wm_internal.h"

namespace {

// --------------------------------------------------------------------------
// repack
// --------------------------------------------------------------------------
__device__ __forceinline__ uint32_t canon_codes(uint32_t w) {
    // per 2-bit field: 11 -> 01
    uint32_t both = w & (w >> 1) & 0x55555555u;
    return w ^ (both << 1);
}

__global__ void k_i2s_repack(const uint8_t *__restrict__ raw, uint4 *__restrict__ out,
                             uint32_t in_dim, uint32_t out_dim, uint32_t n_groups) {
    const uint32_t n_chunks = in_dim / I2S_CHUNK_COLS;
    const uint64_t total = (uint64_t)n_groups * n_chunks * I2S_GROUP_ROWS;
    for (uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (uint64_t)gridDim.x * blockDim.x) {
        uint32_t r = idx % I2S_GROUP_ROWS;
        uint64_t gc = idx / I2S_GROUP_ROWS;
        uint32_t c = gc % n_chunks;
        uint32_t g = gc / n_chunks;
        uint32_t row = g * I2S_GROUP_ROWS + r;
        uint4 v;
        if (row < out_dim) {
            const uint4 *src = reinterpret_cast<const uint4 *>(raw + (uint64_t)row * (in_dim / 4)) + c;
            v = *src;
            v.x = canon_codes(v.x); v.y = canon_codes(v.y);
            v.z = canon_codes(v.z); v.w = canon_codes(v.w);
        } else {
            v = make_uint4(0x55555555u, 0x55555555u, 0x55555555u, 0x55555555u);  // zeros
        }
        out[idx] = v;
    }
}

// --------------------------------------------------------------------------
// activation quantiser (one workgroup of 1024 threads)
// --------------------------------------------------------------------------
__global__ __launch_bounds__(1024) void k_quantize_act(const float *__restrict__ x, uint32_t n,
                                                       uint8_t *__restrict__ act,
                                                       wm_act_meta *__restrict__ meta) {
    __shared__ float s_max[16];
    __shared__ int s_sum[16];
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    float m = 0.0f;
    for (uint32_t i = tid; i < n; i += blockDim.x) m = wm_max_nonan(m, fabsf(x[i]));
    m = wm_wave_max_nonan(m);
    if (lane == 0) s_max[wid] = m;
    __syncthreads();
    float max_abs = 0.0f;
    for (int w = 0; w < (int)(blockDim.x >> 6); w++) max_abs = wm_max_nonan(max_abs, s_max[w]);
    int sum = 0;
    if (max_abs == 0.0f) {
        for (uint32_t i = tid; i < n; i += blockDim.x) act[wm_act_perm(i)] = 0;
    } else {
        const float inv_scale = 127.0f / max_abs;
        for (uint32_t i = tid; i < n; i += blockDim.x) {
            int q = wm_round_clamp_i8(x[i] * inv_scale);
            act[wm_act_perm(i)] = (uint8_t)(int8_t)q;
            sum += q;
        }
    }
    sum = wm_wave_sum_i32(sum);
    if (lane == 0) s_sum[wid] = sum;
    __syncthreads();
    if (tid == 0) {
        int t = 0;
        for (int w = 0; w < (int)(blockDim.x >> 6); w++) t += s_sum[w];
        meta->scale = max_abs == 0.0f ? 1.0f : max_abs / 127.0f;
        meta->asum = t;
    }
}

// --------------------------------------------------------------------------
// matvec: partial dots over a K split
// --------------------------------------------------------------------------
struct i2s_multi {
    const uint8_t *w[WM_I2S_MAX_MULTI];
    uint32_t group_end[WM_I2S_MAX_MULTI];  // cumulative group counts
    int n;
    uint32_t uniform_groups;  // every tensor has this many groups (0: they differ)
};

__device__ __forceinline__ void dot_chunk(const uint4 wv, const int *__restrict__ a,
                                          int &acc16, int &acc4, int &acc1) {
    // a[k*4 + wd] holds the activations of columns 32k + 4wd .. +3 of this chunk
    const uint32_t w[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
    for (int wd = 0; wd < 4; wd++) {
        acc16 = __builtin_amdgcn_sdot4((int)((w[wd] >> 2) & 0x30303030u), a[wd], acc16, false);
        acc16 = __builtin_amdgcn_sdot4((int)(w[wd] & 0x30303030u), a[4 + wd], acc16, false);
        acc4 = __builtin_amdgcn_sdot4((int)(w[wd] & 0x0C0C0C0Cu), a[8 + wd], acc4, false);
        acc1 = __builtin_amdgcn_sdot4((int)(w[wd] & 0x03030303u), a[12 + wd], acc1, false);
    }
}

// grid: x = (global group index over all tensors) / RG, y = K split.  One
// wave, owning RG consecutive 64-row groups of one tensor: lane r computes
// row r of each.  The wave's slice of the activation vector is staged in LDS
// once; every activation read (a uniform broadcast) then serves RG weight
// chunks.  Weights stream in rounds of 4 x RG 1 KiB loads, the next round in
// flight while the current one is reduced; chunk indices past the slice are
// clamped to its last chunk, so every load is in range and unconditional.
template <int RG>
__global__ __launch_bounds__(64) void k_i2s_partial(i2s_multi m, uint32_t n_chunks,
                                                    const int *__restrict__ act,
                                                    int32_t *__restrict__ partial,
                                                    uint32_t rows_total) {
    extern __shared__ __align__(16) int act_s[];  // chunks c0..c1-1, 16 ints each
    const uint32_t gg = blockIdx.x * RG;  // first global group of this wave
    int t = 0;
    uint32_t g = gg;
    if (m.uniform_groups) {
        t = (int)(gg / m.uniform_groups);
        g = gg - (uint32_t)t * m.uniform_groups;
    } else if (m.n > 1) {  // binary search over the cumulative group counts (uniform)
        int lo = 0, hi = m.n - 1;
        while (lo < hi) {
            int mid = (lo + hi) >> 1;
            if (gg < m.group_end[mid]) hi = mid; else lo = mid + 1;
        }
        t = lo;
        g = gg - (t ? m.group_end[t - 1] : 0);
    }
    const uint4 *__restrict__ W = reinterpret_cast<const uint4 *>(m.w[t]);
    const uint32_t split = gridDim.y, s = blockIdx.y;
    const uint32_t c0 = (uint32_t)(((uint64_t)n_chunks * s) / split);
    const uint32_t c1 = (uint32_t)(((uint64_t)n_chunks * (s + 1)) / split);
    const uint32_t r = threadIdx.x, nc = c1 - c0;
    const uint64_t gstride = (uint64_t)n_chunks * I2S_GROUP_ROWS;  // uint4 per group
    const uint4 *wp = W + ((uint64_t)g * n_chunks + c0) * I2S_GROUP_ROWS + r;
    uint4 cur[4][RG];
#pragma unroll
    for (int u = 0; u < 4; u++)
#pragma unroll
        for (int q = 0; q < RG; q++)
            cur[u][q] = wm_load_stream(wp + q * gstride + min((uint32_t)u, nc - 1) * I2S_GROUP_ROWS);
    const int4 *ag = reinterpret_cast<const int4 *>(act) + (uint64_t)c0 * 4;
    for (uint32_t i = r; i < nc * 4; i += 64) reinterpret_cast<int4 *>(act_s)[i] = ag[i];
    __syncthreads();
    int acc16[RG], acc4[RG], acc1[RG];
#pragma unroll
    for (int q = 0; q < RG; q++) acc16[q] = acc4[q] = acc1[q] = 0;
    uint32_t c = 0;
    for (; c + 4 <= nc; c += 4) {
        uint4 nxt[4][RG];
#pragma unroll
        for (int u = 0; u < 4; u++)
#pragma unroll
            for (int q = 0; q < RG; q++)
                nxt[u][q] = wm_load_stream(wp + q * gstride +
                                           min(c + 4 + (uint32_t)u, nc - 1) * I2S_GROUP_ROWS);
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int *a = act_s + (c + u) * 16;
#pragma unroll
            for (int q = 0; q < RG; q++) dot_chunk(cur[u][q], a, acc16[q], acc4[q], acc1[q]);
        }
#pragma unroll
        for (int u = 0; u < 4; u++)
#pragma unroll
            for (int q = 0; q < RG; q++) cur[u][q] = nxt[u][q];
    }
    // the last nc % 4 chunks are cur[0 .. nc%4-1] (loaded by the final round)
#pragma unroll
    for (int u = 0; u < 3; u++)
        if (c + u < nc)
#pragma unroll
            for (int q = 0; q < RG; q++)
                dot_chunk(cur[u][q], act_s + (c + u) * 16, acc16[q], acc4[q], acc1[q]);
#pragma unroll
    for (int q = 0; q < RG; q++)
        partial[(uint64_t)s * rows_total + (uint64_t)(gg + q) * I2S_GROUP_ROWS + r] =
            (acc16[q] >> 4) + (acc4[q] >> 2) + acc1[q];
}

__global__ void k_i2s_finalize(const int32_t *__restrict__ partial, uint32_t split,
                               uint32_t rows_total, uint32_t row0, uint32_t out_dim,
                               float w_scale, const wm_act_meta *__restrict__ meta,
                               float *__restrict__ y, int32_t *__restrict__ dot_out) {
    uint32_t j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= out_dim) return;
    int dot = -meta->asum;
#pragma unroll
    for (uint32_t s = 0; s < 16; s++) {  // split <= 16 (wm_i2s_pick_split); loads unconditional
        const int v = partial[(uint64_t)min(s, split - 1) * rows_total + row0 + j];
        dot += s < split ? v : 0;
    }
    const float combined = w_scale * meta->scale;
    if (y) y[j] = combined * (float)dot;
    if (dot_out) dot_out[j] = dot;
}

// Finalise n_copies outputs of one shape: copy c, row j in y[c*out_dim + j].
__global__ void k_i2s_finalize_multi(const int32_t *__restrict__ partial, uint32_t split,
                                     uint32_t rows_total, uint32_t rows_per_copy, uint32_t out_dim,
                                     uint32_t n_copies, const float *__restrict__ w_scales,
                                     const wm_act_meta *__restrict__ meta, float *__restrict__ y) {
    const uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (uint64_t)n_copies * out_dim) return;
    const uint32_t c = idx / out_dim, j = idx % out_dim;
    int dot = -meta->asum;
    for (uint32_t s = 0; s < split; s++) dot += partial[(uint64_t)s * rows_total + c * rows_per_copy + j];
    y[idx] = (w_scales[c] * meta->scale) * (float)dot;
}

}  // namespace

void wm_launch_i2s_finalize_multi(const int32_t *partial, uint32_t split, uint32_t rows_total,
                                  uint32_t rows_per_copy, uint32_t out_dim, uint32_t n_copies,
                                  const float *w_scales, const wm_act_meta *meta, float *y,
                                  hipStream_t s) {
    uint64_t n = (uint64_t)n_copies * out_dim;
    hipLaunchKernelGGL(k_i2s_finalize_multi, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, s,
                       partial, split, rows_total, rows_per_copy, out_dim, n_copies, w_scales, meta,
                       y);
}

void wm_launch_i2s_repack(const uint8_t *raw, uint8_t *out, uint32_t in_dim, uint32_t out_dim,
                          uint32_t n_groups, hipStream_t s) {
    uint64_t total = (uint64_t)n_groups * (in_dim / I2S_CHUNK_COLS) * I2S_GROUP_ROWS;
    uint32_t blocks = (uint32_t)((total + 255) / 256);
    if (blocks > 65535u * 4) blocks = 65535u * 4;
    hipLaunchKernelGGL(k_i2s_repack, dim3(blocks), dim3(256), 0, s, raw,
                       reinterpret_cast<uint4 *>(out), in_dim, out_dim, n_groups);
}

void wm_launch_quantize_act(const float *x, uint32_t n, uint8_t *act, wm_act_meta *meta,
                            hipStream_t s) {
    hipLaunchKernelGGL(k_quantize_act, dim3(1), dim3(1024), 0, s, x, n, act, meta);
}

uint32_t wm_i2s_pick_split(uint32_t n_groups, uint32_t n_chunks) {
    // Each wave streams its chunks four loads at a time, one memory latency
    // per round; aim for ~32 waves per CU over 256 CUs so that few rounds
    // remain per wave, with at least 4 chunks (one round) per wave.
    uint32_t split = (4096 + n_groups - 1) / n_groups;
    uint32_t max_split = n_chunks / 4 ? n_chunks / 4 : 1;
    if (split > max_split) split = max_split;
    if (split > 16) split = 16;  // consumers sum at most 16 partials per row
    if (split < 1) split = 1;
    return split;
}

void wm_launch_i2s_partial(const wm_i2s_desc *descs, int n_desc, uint32_t n_chunks,
                           const uint8_t *act, int32_t *partial, uint32_t split,
                           uint32_t rows_total, hipStream_t s) {
    i2s_multi m{};
    uint32_t acc = 0;
    m.n = n_desc;
    m.uniform_groups = descs[0].n_groups;
    for (int i = 0; i < n_desc; i++) {
        m.w[i] = descs[i].w;
        acc += descs[i].n_groups;
        m.group_end[i] = acc;
        if (descs[i].n_groups != descs[0].n_groups) m.uniform_groups = 0;
    }
    const size_t lds = (size_t)((n_chunks + split - 1) / split) * 64;  // activation slice
    // One group per wave: measured faster than two (fewer waves hide less latency).
    hipLaunchKernelGGL(k_i2s_partial<1>, dim3(acc, split), dim3(64), lds, s, m, n_chunks,
                       reinterpret_cast<const int *>(act), partial, rows_total);
}

void wm_launch_i2s_finalize(const int32_t *partial, uint32_t split, uint32_t rows_total,
                            uint32_t row0, uint32_t out_dim, float w_scale,
                            const wm_act_meta *meta, float *y, int32_t *dot_out, hipStream_t s) {
    hipLaunchKernelGGL(k_i2s_finalize, dim3((out_dim + 255) / 256), dim3(256), 0, s, partial,
                       split, rows_total, row0, out_dim, w_scale, meta, y, dot_out);
}
