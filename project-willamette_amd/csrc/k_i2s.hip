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
#include "wm_norm.h"

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
    wm_sync_lds();
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
    wm_sync_lds();
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
    const uint8_t *const *table;  // or: device array of n tensors of uniform_groups groups each
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

// One round: chunks c .. c+3 of RG row groups (chunk u of group q at
// wp[q] + u * I2S_GROUP_ROWS, uint4 units, this lane's row), the indices past
// the slice clamped to its last chunk so every load is in range.
template <int RG>
struct i2s_round {
    uint4 v[4][RG];
};
template <int RG>
__device__ __forceinline__ void i2s_issue(i2s_round<RG> &R, const uint4 *const (&wp)[RG],
                                          uint32_t c, uint32_t nc) {
#pragma unroll
    for (int u = 0; u < 4; u++)
#pragma unroll
        for (int q = 0; q < RG; q++)
            R.v[u][q] = wm_load_stream(wp[q] + min(c + (uint32_t)u, nc - 1) * I2S_GROUP_ROWS);
}
template <int RG>
__device__ __forceinline__ void i2s_reduce(const i2s_round<RG> &R, const int *act_s, uint32_t c,
                                           uint32_t cnt, int (&acc16)[RG], int (&acc4)[RG],
                                           int (&acc1)[RG]) {
#pragma unroll
    for (int u = 0; u < 4; u++)
        if ((uint32_t)u < cnt)
#pragma unroll
            for (int q = 0; q < RG; q++)
                dot_chunk(R.v[u][q], act_s + (c + u) * 16, acc16[q], acc4[q], acc1[q]);
}
// The dots over chunks 0 .. nc-1, round 0 already issued into A (and round
// 1 into B when b_issued, nc > 4): the next round's loads go out before the
// current one is reduced, into the other register set (the loop body covers
// two rounds, so no set is copied); a round past the slice is never issued,
// and the last one is reduced on its own path.
template <int RG>
__device__ __forceinline__ void i2s_rounds(i2s_round<RG> &A, i2s_round<RG> &B,
                                           const uint4 *const (&wp)[RG], uint32_t nc, const int *act_s,
                                           int (&acc16)[RG], int (&acc4)[RG], int (&acc1)[RG],
                                           bool b_issued = false) {
    for (uint32_t c = 0;; c += 8) {
        if (c + 4 >= nc) {
            i2s_reduce<RG>(A, act_s, c, nc - c, acc16, acc4, acc1);
            return;
        }
        if (c > 0 || !b_issued) i2s_issue<RG>(B, wp, c + 4, nc);
        __builtin_amdgcn_sched_barrier(0);  // the prefetch stays ahead of the reduction
        i2s_reduce<RG>(A, act_s, c, 4, acc16, acc4, acc1);
        if (c + 8 >= nc) {
            i2s_reduce<RG>(B, act_s, c + 4, nc - c - 4, acc16, acc4, acc1);
            return;
        }
        i2s_issue<RG>(A, wp, c + 8, nc);
        __builtin_amdgcn_sched_barrier(0);
        i2s_reduce<RG>(B, act_s, c + 4, 4, acc16, acc4, acc1);
    }
}

// grid: x = (global group index over all tensors) / RG, y = K split.  One
// wave, owning RG consecutive 64-row groups of one tensor: lane r computes
// row r of each.  The wave's slice of the activation vector is staged in LDS
// once; every activation read (a uniform broadcast) then serves RG weight
// chunks.  Weights stream in rounds of 4 x RG 1 KiB loads, the next round in
// flight while the current one is reduced (i2s_rounds).
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
    typedef const uint8_t *const __attribute__((address_space(1))) table_entry;  // a global load
    const uint4 *__restrict__ W =
        reinterpret_cast<const uint4 *>(m.table ? ((table_entry *)m.table)[t] : m.w[t]);
    const uint32_t split = gridDim.y, s = blockIdx.y;
    const uint32_t c0 = (uint32_t)(((uint64_t)n_chunks * s) / split);
    const uint32_t c1 = (uint32_t)(((uint64_t)n_chunks * (s + 1)) / split);
    const uint32_t r = threadIdx.x, nc = c1 - c0;
    const uint64_t gstride = (uint64_t)n_chunks * I2S_GROUP_ROWS;  // uint4 per group
    const uint4 *wp[RG];
#pragma unroll
    for (int q = 0; q < RG; q++) wp[q] = W + ((uint64_t)g * n_chunks + c0) * I2S_GROUP_ROWS + r + q * gstride;
    i2s_round<RG> A, B;
    i2s_issue<RG>(A, wp, 0, nc);
    const int4 *ag = reinterpret_cast<const int4 *>(act) + (uint64_t)c0 * 4;
    for (uint32_t i = r; i < nc * 4; i += 64) reinterpret_cast<int4 *>(act_s)[i] = ag[i];
    wm_sync_lds();
    int acc16[RG], acc4[RG], acc1[RG];
#pragma unroll
    for (int q = 0; q < RG; q++) acc16[q] = acc4[q] = acc1[q] = 0;
    i2s_rounds<RG>(A, B, wp, nc, act_s, acc16, acc4, acc1);
#pragma unroll
    for (int q = 0; q < RG; q++)
        partial[(uint64_t)s * rows_total + (uint64_t)(gg + q) * I2S_GROUP_ROWS + r] =
            (acc16[q] >> 4) + (acc4[q] >> 2) + acc1[q];
}

// --------------------------------------------------------------------------
// matvec that starts from its input's RMSNorm, with the K split inside the
// workgroup, and fused epilogues
// --------------------------------------------------------------------------
//
// One workgroup per unit of UG 64-row groups.  It first issues its weights'
// first round, then computes the input's RMSNorm and int8 quantisation
// itself (wm_norm.h, the same operations as k_rmsnorm_quant) straight into
// LDS while those loads are in flight: every workgroup evaluates the same
// norm, so their codes agree bit for bit, and the norm costs no launch and
// no trip through memory.  Each workgroup writes its share of what the norm
// leaves behind for later kernels (x + y), workgroup 0 the cleared slots.
// Its W waves then split the chunks of K between them (wave w: chunks
// [n_chunks*w/W, n_chunks*(w+1)/W)), each computing the unit's rows over its
// slice exactly as k_i2s_partial does; the W partial dots meet in LDS (exact
// integers, so the split changes nothing) and the unit's threads finish the
// rows:
//   y = (w_scale * act_scale) * (float)(Σ c*a - Σ a)   (bitlinear_sse2.rs:327-339)
// then, by MODE,
//   WM_FUSED_PLAIN   y to out[t]
//   WM_FUSED_GATEUP  units are row groups of gate (tensor 0) and up (tensor
//                    1) together: h = relu(gate)^2 * up (ffn.rs:37-65) to out[0]
//   WM_FUSED_ROPE    units are heads (UG = head_dim / 64 groups) of Q, K, V;
//                    NEOX RoPE at `pos` on the tensors in rope_mask
//                    (primitives.rs:285-345), then to out[t]
struct i2s_fused_args {
    const uint8_t *w[WM_FUSED_MAX_TENSORS];
    float w_scale[WM_FUSED_MAX_TENSORS];
    float *out[WM_FUSED_MAX_TENSORS];
    uint32_t unit_end[WM_FUSED_MAX_TENSORS];  // cumulative units per tensor
    int n_tensors;
    uint32_t n_chunks;
    wm_fused_norm norm;                // the input's norm (n = n_chunks * 64)
    const float *rope_cos, *rope_sin;  // [pos][n_rot/2]
    uint32_t pos, n_rot, rope_mask;
    const uint32_t *pos_dev;  // nullable: the position is read here instead of `pos`
    uint32_t *absmax;  // ROPE: absmax of the outputs of tensors 1, 2 (float bits, nullable)
};

template <int MODE, int UG, int W, int NP>  // NP >= ceil(n / (W * 64)): the norm's terms per thread
__global__ __launch_bounds__(W * 64) void k_i2s_fused(i2s_fused_args a) {
    // act [n_chunks*16 ints] | red [W][UG][64] | ys [UG*64] | squares [seq_sum_padded(n)]
    extern __shared__ __align__(16) int smem[];
    __shared__ wm::norm_lds<W> nl;
    const uint32_t u = blockIdx.x;
    int t = 0;
#pragma unroll
    for (int i = 1; i < WM_FUSED_MAX_TENSORS; i++)
        if (i < a.n_tensors && u >= a.unit_end[i - 1]) t = i;
    const uint32_t lu = u - (t ? a.unit_end[t - 1] : 0u);  // unit within its tensor
    const uint32_t wid = (uint32_t)__builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t n_chunks = a.n_chunks;
    const uint32_t c0 = n_chunks * wid / W, c1 = n_chunks * (wid + 1) / W, nc = c1 - c0;
    const uint64_t gstride = (uint64_t)n_chunks * I2S_GROUP_ROWS;  // uint4 per group
    const uint4 *wp[UG];
#pragma unroll
    for (int q = 0; q < UG; q++) {
        const int tq = MODE == WM_FUSED_GATEUP ? q : t;
        const uint32_t g = MODE == WM_FUSED_GATEUP ? lu : lu * UG + q;
        wp[q] = reinterpret_cast<const uint4 *>(a.w[tq]) + g * gstride + (uint64_t)c0 * I2S_GROUP_ROWS + lane;
    }
    int *act_s = smem;
    int *red = smem + n_chunks * 16;
    float *ys = reinterpret_cast<float *>(red + W * UG * 64);
    float *sq = ys + UG * 64;
    // The norm's inputs first, alone: they come back quickly while nothing
    // else is queued (every workgroup's weight loads would otherwise be ahead
    // of them in the memory system).  The first round of weights follows
    // inside the exact sum, once its per-term work is done.
    const wm_fused_norm &nm = a.norm;
    const uint32_t n = n_chunks * 64;
    const bool first = blockIdx.x == 0;
    float xv[NP], wv[NP], rv[NP];
    wm::norm_load<NP, W * 64>(nm.x, nm.y, nm.w, n, xv, wv, rv);
    wm::norm_prep<NP, W * 64>(nm.y != nullptr, n, nullptr, sq, xv, wv, rv, nm.relu2_mul != 0);
    __builtin_amdgcn_sched_barrier(0);
    i2s_round<UG> A, B;
    // the epilogue's RoPE factors, fetched now rather than after the reduction
    const uint32_t half = a.n_rot / 2;  // ROPE: at most 64 <= W * 64 pairs, one per thread
    const bool rope = MODE == WM_FUSED_ROPE && ((a.rope_mask >> t) & 1u);
    float rc = 0.0f, rsn = 0.0f;
    if (rope && threadIdx.x < half) {
        const uint32_t pos = a.pos_dev ? *a.pos_dev : a.pos;
        rc = a.rope_cos[(uint64_t)pos * half + threadIdx.x];
        rsn = a.rope_sin[(uint64_t)pos * half + threadIdx.x];
    }
    // the input's norm and int8 codes, into LDS (the weights stay in flight;
    // no global memory access until the dots, so no wait the compiler places
    // for one can wait on the weights)
    float act_scale;
    int asum;
    {
        // the first round of weights goes out once the sum's per-term work
        // is done (data arriving during that work slows it), in flight
        // during the record walk and the quantiser
        const auto issue_first = [&]() {
            __builtin_amdgcn_sched_barrier(0);
            i2s_issue<UG>(A, wp, 0, nc);
            if (nc > 4) i2s_issue<UG>(B, wp, 4, nc);  // and the second, if the slice has one
            __builtin_amdgcn_sched_barrier(0);
        };
        const float rsq = wm::norm_sum_rsqrt<NP, W * 64>(false, n, nm.eps, nullptr, 0, sq, nl, issue_first);
        wm::norm_quant<NP, W * 64>(rsq, n, xv, wv, reinterpret_cast<uint8_t *>(act_s), nl,
                                   act_scale, asum);
    }
    // What the norm leaves for later kernels, written once this workgroup's
    // own work is done, each workgroup its contiguous share of the elements:
    // x + y (the same f32 adds as above) with the non-finite check; and by
    // workgroup 0 the cleared slots.
    const auto finish = [&]() {
        const uint32_t tid0 = threadIdx.x;
        if (first && nm.clear2 && tid0 < 2) nm.clear2[tid0] = 0;
        if (nm.x_out && nm.y) {
            const uint32_t lo = (uint32_t)((uint64_t)n * blockIdx.x / gridDim.x);
            const uint32_t hi = (uint32_t)((uint64_t)n * (blockIdx.x + 1) / gridDim.x);
            bool nonfinite = false;
            for (uint32_t j = lo + tid0; j < hi; j += W * 64) {
                const float v = nm.x[j] + nm.y[j];
                nm.x_out[j] = v;
                nonfinite |= !isfinite(v);
            }
            // every writer of this launch writes the same tag; a flag already
            // raised by an earlier layer is kept
            if (nonfinite && nm.err_flag && *nm.err_flag == 0) *nm.err_flag = nm.layer_tag;
        }
    };
    int acc16[UG], acc4[UG], acc1[UG];
#pragma unroll
    for (int q = 0; q < UG; q++) acc16[q] = acc4[q] = acc1[q] = 0;
    i2s_rounds<UG>(A, B, wp, nc, act_s + c0 * 16, acc16, acc4, acc1, nc > 4);
#pragma unroll
    for (int q = 0; q < UG; q++)
        red[(wid * UG + q) * 64 + lane] = (acc16[q] >> 4) + (acc4[q] >> 2) + acc1[q];
    wm_sync_lds();
    const uint32_t tid = threadIdx.x;
    if (MODE == WM_FUSED_GATEUP) {
        if (tid < 64) {
            int dg = -asum, du = -asum;
#pragma unroll
            for (int w = 0; w < W; w++) {
                dg += red[(w * UG + 0) * 64 + tid];
                du += red[(w * UG + 1) * 64 + tid];
            }
            const float g = (a.w_scale[0] * act_scale) * (float)dg;
            const float up = (a.w_scale[1] * act_scale) * (float)du;
            const float r = g > 0.0f ? g : 0.0f;
            a.out[0][lu * 64 + tid] = (r * r) * up;
        }
        finish();
        return;
    }
    float *out = a.out[t] + (uint64_t)lu * UG * 64;
    for (uint32_t row = tid; row < UG * 64; row += W * 64) {
        const uint32_t q = row >> 6, rr = row & 63;
        int dot = -asum;
#pragma unroll
        for (int w = 0; w < W; w++) dot += red[(w * UG + q) * 64 + rr];
        const float y = (a.w_scale[t] * act_scale) * (float)dot;
        if (MODE == WM_FUSED_PLAIN) {
            out[row] = y;
        } else {
            ys[row] = y;
        }
    }
    if (MODE == WM_FUSED_PLAIN) {
        finish();
        return;
    }
    // WM_FUSED_ROPE: pairs (j, j + n_rot/2) of this head
    wm_sync_lds();
    float mx = 0.0f;  // |output| maximum, NaN never raising it
    if (rope) {
        if (tid < half) {
            const uint32_t j = tid;
            const float x0 = ys[j], x1 = ys[j + half];
            const float r0 = x0 * rc - x1 * rsn, r1 = x0 * rsn + x1 * rc;
            out[j] = r0;
            out[j + half] = r1;
            mx = wm_max_nonan(wm_max_nonan(mx, fabsf(r0)), fabsf(r1));
        }
        for (uint32_t j = a.n_rot + tid; j < UG * 64; j += W * 64) {
            out[j] = ys[j];
            mx = wm_max_nonan(mx, fabsf(ys[j]));
        }
    } else {
        for (uint32_t j = tid; j < UG * 64; j += W * 64) {
            out[j] = ys[j];
            mx = wm_max_nonan(mx, fabsf(ys[j]));
        }
    }
    // KVCache::append needs each of K and V's absmax over all heads: the
    // units publish theirs with an integer max of the float bits (non-negative
    // floats order as their bits; the slots are cleared before the launch)
    if (t >= 1 && a.absmax) {
        mx = wm_wave_max_nonneg(mx);
        if (lane == 0) atomicMax(a.absmax + (t - 1), __float_as_uint(mx));
    }
    finish();
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

// --------------------------------------------------------------------------
// scalar f32 matvec (bitlinear_i2s_matvec_f32_scalar, src/model/bitlinear.rs:146-233)
// --------------------------------------------------------------------------
// No int8 activations: per row, two f32 accumulators, pos += x for code 10
// and neg += x for code 00, over the row's bytes in order and, in each byte,
// the codes of columns gp, gp+32, gp+64, gp+96 (bits 7:6 down to 1:0); then
// out = scale * (pos - neg).  Each accumulator is a dependent chain, so one
// lane owns one row (lane r of workgroup g: row 64g + r, its 16-byte chunks
// coalesced across the wave).  A skipped code adds +0.0 instead: pos and
// neg start at +0.0 and an f32 sum is -0.0 only when both operands are, so
// they never hold -0.0 and x + (+0.0) == x for every other value (NaN and
// inf included): the result is the reference's bit for bit.
// Chunk c of a row is bytes [16c, 16c+16): byte b of it is byte
// gp = 16(c%2) + b of block c/2, i.e. columns 128(c/2) + gp + {0,32,64,96}.
constexpr uint32_t kScalarTile = 1024;  // x columns staged in LDS per round (8 blocks, 16 chunks)

// Bytes b .. b+3 of a block (one little-endian dword; xb points at column
// gp = b of the block in LDS) in the reference's order.
__device__ __forceinline__ void scalar_dword(uint32_t wd, const float *xb, float &pos, float &neg) {
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const uint32_t byte = (wd >> (8 * e)) & 0xffu;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const uint32_t code = (byte >> (6 - 2 * q)) & 3u;
            const float xv = xb[e + 32 * q];
            pos += code == 2u ? xv : 0.0f;
            neg += code == 0u ? xv : 0.0f;
        }
    }
}

typedef uint32_t scalar_u32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(64) void k_i2s_scalar_f32(const scalar_u32x4 *__restrict__ w, uint32_t n_chunks,
                                                       uint32_t out_dim, float scale,
                                                       const float *__restrict__ x,
                                                       float *__restrict__ y) {
    __shared__ __align__(16) float xs[kScalarTile];
    const uint32_t lane = threadIdx.x, g = blockIdx.x;
    const scalar_u32x4 *wg = w + (uint64_t)g * n_chunks * I2S_GROUP_ROWS + lane;
    const uint32_t in_dim = n_chunks * I2S_CHUNK_COLS;
    float pos = 0.0f, neg = 0.0f;
    for (uint32_t base = 0; base < in_dim; base += kScalarTile) {
        const uint32_t cols = min(kScalarTile, in_dim - base);  // a multiple of 128
        __syncthreads();
        for (uint32_t i = lane; i < cols; i += 64) xs[i] = x[base + i];
        __syncthreads();
        const uint32_t c0 = base / I2S_CHUNK_COLS, c1 = c0 + cols / I2S_CHUNK_COLS;
        scalar_u32x4 cur = wg[(uint64_t)c0 * I2S_GROUP_ROWS];
        for (uint32_t c = c0; c < c1; c++) {
            const scalar_u32x4 nxt = c + 1 < c1 ? wg[(uint64_t)(c + 1) * I2S_GROUP_ROWS] : cur;
            const float *xb = xs + ((c - c0) / 2) * 128 + (c & 1) * 16;
            scalar_dword(cur.x, xb, pos, neg);
            scalar_dword(cur.y, xb + 4, pos, neg);
            scalar_dword(cur.z, xb + 8, pos, neg);
            scalar_dword(cur.w, xb + 12, pos, neg);
            cur = nxt;
        }
    }
    const uint32_t row = g * I2S_GROUP_ROWS + lane;
    if (row < out_dim) y[row] = scale * (pos - neg);
}

}  // namespace

void wm_launch_i2s_scalar_f32(const uint8_t *w, uint32_t n_groups, uint32_t n_chunks,
                              uint32_t out_dim, float scale, const float *x, float *y,
                              hipStream_t s) {
    hipLaunchKernelGGL(k_i2s_scalar_f32, dim3(n_groups), dim3(64), 0, s,
                       reinterpret_cast<const scalar_u32x4 *>(w), n_chunks, out_dim, scale, x, y);
}

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

// n_tensors tensors of groups_per groups each, their device pointers in the
// device array `table` (any count: no kernel-argument limit).
void wm_launch_i2s_partial_table(const uint8_t *const *table, uint32_t n_tensors,
                                 uint32_t groups_per, uint32_t n_chunks, const uint8_t *act,
                                 int32_t *partial, uint32_t split, uint32_t rows_total,
                                 hipStream_t s) {
    i2s_multi m{};
    m.n = (int)n_tensors;
    m.uniform_groups = groups_per;
    m.table = table;
    const size_t lds = (size_t)((n_chunks + split - 1) / split) * 64;  // activation slice
    hipLaunchKernelGGL(k_i2s_partial<1>, dim3(groups_per * n_tensors, split), dim3(64), lds, s, m,
                       n_chunks, reinterpret_cast<const int *>(act), partial, rows_total);
}

void wm_launch_i2s_finalize(const int32_t *partial, uint32_t split, uint32_t rows_total,
                            uint32_t row0, uint32_t out_dim, float w_scale,
                            const wm_act_meta *meta, float *y, int32_t *dot_out, hipStream_t s) {
    hipLaunchKernelGGL(k_i2s_finalize, dim3((out_dim + 255) / 256), dim3(256), 0, s, partial,
                       split, rows_total, row0, out_dim, w_scale, meta, y, dot_out);
}

// The fused matvec over the units of `n_tensors` tensors (see k_i2s_fused).
// Waves per workgroup: n_chunks / 4 (one 4-chunk round each), at most 16.
// Returns false (and launches nothing) when no instantiation fits the shape.
bool wm_launch_i2s_fused(int mode, const wm_i2s_desc *descs, const float *w_scales, float *const *outs,
                         int n_tensors, uint32_t n_chunks, uint32_t groups_per_unit,
                         const wm_fused_norm &norm, const float *rope_cos, const float *rope_sin,
                         uint32_t pos, uint32_t n_rot, uint32_t rope_mask, uint32_t *absmax,
                         hipStream_t s, const uint32_t *pos_dev) {
    i2s_fused_args a{};
    uint32_t acc = 0;
    a.n_tensors = n_tensors;
    for (int i = 0; i < n_tensors; i++) {
        a.w[i] = descs[i].w;
        a.w_scale[i] = w_scales[i];
        a.out[i] = outs[i];
        // units: PLAIN one per group, ROPE one per head (UG groups), GATEUP one
        // per group pair (counted on the gate tensor only)
        const uint32_t units = mode == WM_FUSED_GATEUP ? (i == 0 ? descs[0].n_groups : 0)
                                                       : descs[i].n_groups / groups_per_unit;
        acc += units;
        a.unit_end[i] = acc;
    }
    if (mode == WM_FUSED_GATEUP) a.n_tensors = 1;  // units all belong to the pair
    a.n_chunks = n_chunks;
    a.norm = norm;
    a.rope_cos = rope_cos;
    a.rope_sin = rope_sin;
    a.pos = pos;
    a.pos_dev = pos_dev;
    a.n_rot = n_rot;
    a.rope_mask = rope_mask;
    a.absmax = absmax;
    // Waves: as many as the chunks allow, up to 16 (the norm at the start is
    // latency-bound and runs best on the widest workgroup; each wave still
    // has its own chunks), rounded down to an instantiated count.
    int w = (int)(n_chunks < 16 ? n_chunks : 16);
    static const int kWs[] = {16, 12, 10, 8, 6, 4, 2, 1};
    for (int x : kWs)
        if (w >= x) { w = x; break; }
    // the norm's terms per thread, rounded up to an instantiated bound (the
    // exact sum's work grows with the bound; 3 and 7 are BitNet-2B's 2560 and
    // 6912): at most 2 below 16 waves, at most 16 with 16 (n_chunks <= 256)
    const uint32_t per = (n_chunks + (uint32_t)w - 1) / (uint32_t)w;
    const int np = w == 16 && (per == 3 || per == 7) ? (int)per
                                                     : (per <= 4 ? 4 : (per <= 8 ? 8 : 16));
    const size_t sq_bytes = (size_t)wm::seq_sum_padded(n_chunks * 64) * 4;
#define WM_FUSED_CASE(MODE, UG, W, NP)                                                             \
    if (w == W && np == NP) {                                                                      \
        const size_t lds = (size_t)n_chunks * 64 + (size_t)W * UG * 64 * 4 + (size_t)UG * 64 * 4 + \
                           sq_bytes;                                                               \
        hipLaunchKernelGGL((k_i2s_fused<MODE, UG, W, NP>), dim3(acc), dim3(W * 64), lds, s, a);    \
        return true;                                                                               \
    }
#define WM_FUSED_WS(MODE, UG)                                                                      \
    WM_FUSED_CASE(MODE, UG, 1, 4) WM_FUSED_CASE(MODE, UG, 2, 4) WM_FUSED_CASE(MODE, UG, 4, 4)      \
    WM_FUSED_CASE(MODE, UG, 6, 4) WM_FUSED_CASE(MODE, UG, 8, 4) WM_FUSED_CASE(MODE, UG, 10, 4)     \
    WM_FUSED_CASE(MODE, UG, 12, 4) WM_FUSED_CASE(MODE, UG, 16, 3) WM_FUSED_CASE(MODE, UG, 16, 4)   \
    WM_FUSED_CASE(MODE, UG, 16, 7) WM_FUSED_CASE(MODE, UG, 16, 8) WM_FUSED_CASE(MODE, UG, 16, 16)
    if (mode == WM_FUSED_PLAIN) { WM_FUSED_WS(WM_FUSED_PLAIN, 1) }
    else if (mode == WM_FUSED_GATEUP) { WM_FUSED_WS(WM_FUSED_GATEUP, 2) }
    else if (groups_per_unit == 2) { WM_FUSED_WS(WM_FUSED_ROPE, 2) }
    else if (groups_per_unit == 1) { WM_FUSED_WS(WM_FUSED_ROPE, 1) }
#undef WM_FUSED_WS
#undef WM_FUSED_CASE
    return false;
}
