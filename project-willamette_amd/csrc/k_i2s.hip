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
// The same with KS lanes per row: lane sub-slice `sub` holds chunks
// sub, sub + KS, sub + 2 KS, ... of the wave's slice (register u of round k:
// chunk sub + KS (4k + u)); loads past the slice clamp to its last chunk and
// their dots read a block of zero activations instead.  Only the first cnt
// registers (wave-uniform: the most any lane needs) are loaded, and with
// KS > 1 only by the lanes whose chunk lies in the slice (the others hold
// zeros): the CU's vector memory path moves every active lane's bytes, and
// it is what the workgroup's first loads queue on.
template <int RG, int KS>
__device__ __forceinline__ void i2s_issue_ks(i2s_round<RG> &R, const uint4 *const (&wp)[RG], uint32_t k,
                                             uint32_t nc, uint32_t sub, uint32_t cnt = 4) {
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const uint32_t j = sub + KS * (4u * k + (uint32_t)u);
#pragma unroll
        for (int q = 0; q < RG; q++) {
            R.v[u][q] = make_uint4(0u, 0u, 0u, 0u);
            if ((uint32_t)u < cnt && (KS == 1 || j < nc))
                R.v[u][q] = wm_load_stream(wp[q] + min(j, nc - 1) * I2S_GROUP_ROWS);
        }
    }
}
template <int RG, int KS>
__device__ __forceinline__ void i2s_reduce_ks(const i2s_round<RG> &R, const int *act_c0, const int *zeros,
                                              uint32_t k, uint32_t cnt, uint32_t nc, uint32_t sub,
                                              int (&acc16)[RG], int (&acc4)[RG], int (&acc1)[RG]) {
#pragma unroll
    for (int u = 0; u < 4; u++)
        if ((uint32_t)u < cnt) {
            const uint32_t j = sub + KS * (4u * k + (uint32_t)u);
            const int *a = KS == 1 || j < nc ? act_c0 + j * 16 : zeros;
#pragma unroll
            for (int q = 0; q < RG; q++) dot_chunk(R.v[u][q], a, acc16[q], acc4[q], acc1[q]);
        }
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
// One workgroup per unit of UG 64-row groups, or KS workgroups per unit
// each with 64 / KS rows of every group (KS lanes per row, below).  It first
// issues its weights' first round, then computes the input's RMSNorm and int8 quantisation
// itself (wm_norm.h, the same operations as k_rmsnorm_quant) straight into
// LDS while those loads are in flight: every workgroup evaluates the same
// norm, so their codes agree bit for bit, and the norm costs no launch and
// no trip through memory.  Each workgroup writes its share of what the norm
// leaves behind for later kernels (x + y).
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
// What the first loads of a launch need comes in the leading 14 argument
// dwords, which the hardware preloads into SGPRs at wave launch (the file is
// built with -amdgpu-kernarg-preload-count=16; the argument pointer takes
// the other two user SGPRs): the norm's inputs, the tensors' weights, where
// tensors 1 and 2 begin (units, 16 bits each), n_chunks and flags.
// Everything else is in i2s_fused_args, read once the first loads are out,
// so the norm covers that round trip.
enum : uint32_t {
    FUSED_RELU2 = 1u << 16,
    // test hooks (WM_FUSED_DEBUG_*): the speculation's max|y| skewed, the
    // candidate lists treated as failed
    FUSED_SKEW_SMALL = 1u << 17,
    FUSED_SKEW_LARGE = 1u << 18,
    FUSED_NO_CANDIDATES = 1u << 19
};
struct i2s_fused_args {
    float w_scale[WM_FUSED_MAX_TENSORS];
    float *out[WM_FUSED_MAX_TENSORS];
    float *x_out;       // nullable: x + y written here, each workgroup its share (never x itself)
    float eps;
    uint32_t *err_flag;  // nullable: set to layer_tag when x + y is not all finite
    uint32_t layer_tag;
    const float *rope_cos, *rope_sin;  // [pos][n_rot/2]
    uint32_t pos, n_rot, rope_mask;
    const uint32_t *pos_dev;  // nullable: the position is read here instead of `pos`
    uint32_t *absmax;  // ROPE: absmax slots of the outputs of tensors 1, 2 (float bits, nullable)
    uint32_t absmax_stride;  // tensor t's slots from absmax + (t - 1) * absmax_stride
};


// KS: lanes per row.  A unit's rows are then split over KS workgroups of
// R = 64 / KS rows of each of its groups, and lane l of a wave computes row
// l % R over every KS-th chunk of the wave's slice from l / R on; the KS
// partial dots of a row meet by lane exchange.
template <int MODE, int UG, int W, int NP, int KS>  // NP: a power of two >= ceil(n / (W * 64))
__global__ __launch_bounds__(W * 64) void k_i2s_fused(const float *nx, const float *ny, const float *nw,
                                                      const uint8_t *w0, const uint8_t *w1, const uint8_t *w2,
                                                      uint32_t units01, uint32_t chunks_flags, i2s_fused_args a) {
    // act [n_chunks*16 ints] | zeros [16] | red [W][UG][64] | ys [UG*64] | squares [seq_sum_padded(n)]
    extern __shared__ __align__(16) int smem[];
    __shared__ wm::fused_norm_lds<W> nl;
    constexpr int NR = (NP + 3) / 4;  // quantiser rounds: four chunks per round
    const uint32_t u = blockIdx.x;
    // this unit's tensor t (units [ue0, ue1) belong to tensor 1, from ue1 on
    // to tensor 2) and its unit within the tensor
    const uint32_t ue0 = units01 & 0xFFFFu, ue1 = units01 >> 16;
    const uint32_t n_chunks = chunks_flags & 0xFFFFu;
    const int t = u >= ue1 ? 2 : (u >= ue0 ? 1 : 0);
    const uint8_t *wt = t == 2 ? w2 : (t == 1 ? w1 : w0);
    const uint32_t lk = u - (t == 2 ? ue1 : (t == 1 ? ue0 : 0u));
    constexpr uint32_t R = 64 / KS;  // rows per group of this workgroup
    const uint32_t lu = lk / KS, h = lk % KS;  // the unit, and which R of each group's 64 rows
    const uint32_t wid = (uint32_t)__builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t sub = lane / R, row = h * R + lane % R;  // this lane's sub-slice and row
    // With SPEC, wave 0 only walks the exact sum; waves 1..W-1 own the slices
    // of K and quantise speculatively meanwhile (below).  NP bounds a wave's
    // chunks, and SPEC needs them all resident (at most two rounds).
    constexpr bool SPEC = W >= 2 && NP <= 8;
    static_assert(KS == 1 || (SPEC && NP <= 4 * KS), "KS > 1: the speculating form, one register round");
    // With SPEC the slices are NP chunks each (whole quantiser rounds, so
    // every lane of a load has a column; the workgroup's first loads queue
    // on the CU's vector memory path per instruction), from wave 1 on, as
    // many waves as n_chunks needs; otherwise n_chunks spread over all W.
    constexpr uint32_t KW = SPEC ? W - 1 : W;  // waves with a slice of K
    const uint32_t kw = SPEC ? (wid == 0 ? KW : wid - 1) : wid;
    const uint32_t c0 = SPEC ? min(kw * (uint32_t)NP, n_chunks) : n_chunks * kw / KW;
    const uint32_t nc = SPEC ? min((uint32_t)NP, n_chunks - c0) : n_chunks * (kw + 1) / KW - c0;
    const uint64_t gstride = (uint64_t)n_chunks * I2S_GROUP_ROWS;  // uint4 per group
    const uint4 *wp[UG];
#pragma unroll
    for (int q = 0; q < UG; q++) {
        const uint8_t *wq = MODE == WM_FUSED_GATEUP && q == 1 ? w1 : wt;
        const uint32_t g = MODE == WM_FUSED_GATEUP ? lu : lu * UG + q;
        wp[q] = reinterpret_cast<const uint4 *>(wq) + g * gstride + (uint64_t)c0 * I2S_GROUP_ROWS + row;
    }
    int *act_s = smem;
    int *zeros = smem + n_chunks * 16;  // the activations of a chunk past a lane's sub-slice
    int *red = zeros + 16;
    float *ys = reinterpret_cast<float *>(red + W * UG * 64);
    float *sq = ys + UG * 64;
    const uint32_t n = n_chunks * 64;
    const bool relu2 = (chunks_flags & FUSED_RELU2) != 0, has_y = ny != nullptr;
    // The norm's inputs first, once, in the quantiser's layout (fused_quads:
    // four consecutive columns per lane and round, with their norm weights;
    // the waves' slices cover the vector); the exact sum's layout (thread t:
    // terms t*NP .. t*NP+NP-1) then comes from the squares in LDS.  Then the
    // weights, whose loads are waited for only at the dots: the norm's waits
    // are for loads issued before them.
    const __amdgpu_buffer_rsrc_t rx = wm_rsrc(nx, n * 4), ry = wm_rsrc(has_y ? ny : nx, n * 4),
                                 rw = wm_rsrc(nw, n * 4);
    const uint32_t k0 = threadIdx.x * NP;
    wm::fused_quads<NR> Q;
    float yq[NR][4];
#pragma unroll
    for (int r = 0; r < NR; r++) {
        // (only the lanes whose chunk lies in the slice load)
#pragma unroll
        for (int i = 0; i < 4; i++) Q.v[r][i] = Q.w[r][i] = yq[r][i] = 0.0f;
        if (Q.valid(r, c0, nc)) {
            const uint32_t off = wm::quad_col(r, c0) * 4;
            wm::buf_run<4>(rx, off, Q.v[r]);
            wm::buf_run<4>(rw, off, Q.w[r]);
            if (has_y) wm::buf_run<4>(ry, off, yq[r]);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    if (KS > 1 && threadIdx.x < 16) zeros[threadIdx.x] = 0;
    __builtin_amdgcn_sched_barrier(0);
    // The rest of the arguments, their round trip under the norm: read
    // through their address plus a zero the compiler cannot see through, so
    // the loads stay here instead of being hoisted above the first loads.
    uint32_t zero;
    asm volatile("s_mov_b32 %0, 0" : "=s"(zero));
    const i2s_fused_args &ar =
        *reinterpret_cast<const i2s_fused_args *>(reinterpret_cast<const char *>(&a) + zero);
    float *x_out = ar.x_out, eps = ar.eps;
    uint32_t *err_flag = ar.err_flag, layer_tag = ar.layer_tag;
    float ws0 = ar.w_scale[0], w_scale1 = ar.w_scale[1], ws2 = ar.w_scale[2];
    float *o0 = ar.out[0], *o1 = ar.out[1], *o2 = ar.out[2];
    const float *rope_cos = ar.rope_cos, *rope_sin = ar.rope_sin;
    uint32_t pos_arg = ar.pos, n_rot = ar.n_rot, rope_mask = ar.rope_mask;
    const uint32_t *pos_dev = ar.pos_dev;
    uint32_t *absmax = ar.absmax;
    uint32_t absmax_stride = ar.absmax_stride;
    // Pinned in SGPRs here (a load the compiler moved to the first use would
    // stall there instead of under the norm), all by one asm: the loads go
    // out together and meet one wait (an asm per value made a chain of round
    // trips, each load issued after the previous value's wait).
    asm volatile(""
                 : "+s"(x_out), "+s"(eps), "+s"(err_flag), "+s"(layer_tag), "+s"(ws0), "+s"(w_scale1), "+s"(ws2),
                   "+s"(o0), "+s"(o1), "+s"(o2), "+s"(rope_cos), "+s"(rope_sin), "+s"(pos_arg), "+s"(n_rot),
                   "+s"(rope_mask), "+s"(pos_dev), "+s"(absmax), "+s"(absmax_stride));
    const wm_fused_norm nm = {nx, ny, x_out, nw, eps, err_flag, layer_tag, chunks_flags & FUSED_RELU2};
    const float w_scale = t == 2 ? ws2 : (t == 1 ? w_scale1 : ws0);
    float *const out_t = t == 2 ? o2 : (t == 1 ? o1 : o0);
    // the epilogue's RoPE factors
    const uint32_t half = n_rot / 2;  // ROPE: at most 64 <= W * 64 pairs, one per thread
    // this workgroup's pairs: all of the head's (KS = 1), else R, the pairs
    // (h R + i, h R + i + 64) of a 128-wide rotation over UG = 2 groups
    const uint32_t n_pairs = KS == 1 ? half : R, pair0 = KS == 1 ? 0u : h * R;
    const bool rope = MODE == WM_FUSED_ROPE && ((rope_mask >> t) & 1u);
    float rc = 0.0f, rsn = 0.0f;
    if (rope && threadIdx.x < n_pairs) {
        // (through global pointers: a flat load would also count with the
        // LDS operations, and the norm's barriers would wait for it)
        using gu32 = __attribute__((address_space(1))) const uint32_t;
        using gf32 = __attribute__((address_space(1))) const float;
        const uint32_t pos = pos_dev ? *(gu32 *)pos_dev : pos_arg;
        rc = ((gf32 *)rope_cos)[(uint64_t)pos * half + pair0 + threadIdx.x];
        rsn = ((gf32 *)rope_sin)[(uint64_t)pos * half + pair0 + threadIdx.x];
    }
    // x + y (hidden += the producing matvec's output), or with relu2
    // relu(x)^2 * y (the FFN's gate x and up y, ffn.rs:37-65), the same f32
    // operations in both layouts
    const auto combine = [&](float x, float y) {
        const float r = x > 0.0f ? x : 0.0f;
        return relu2 ? (r * r) * y : (has_y ? x + y : x);
    };
    // What the norm leaves for later kernels: x + y (the same f32 adds as
    // the norm's, never relu2's combination), each workgroup its contiguous
    // share of the elements, and whether it is all finite.
    bool nonfinite = false;
    if (nm.x_out && has_y) {
        // (n * gridDim.x fits 32 bits: the launcher rejects grids where not)
        const uint32_t lo = n * blockIdx.x / gridDim.x;
        const uint32_t hi = n * (blockIdx.x + 1) / gridDim.x;
        // the sums first, then the stores through a global pointer: a store
        // between two of them made the next wait for the inputs also wait
        // for that store (a flat store counts with the loads)
        float xs[NR][4];
#pragma unroll
        for (int r = 0; r < NR; r++) {
#pragma unroll
            for (int i = 0; i < 4; i++) xs[r][i] = Q.v[r][i] + yq[r][i];
            // (formed here, not sunk into the stores' branches below)
            asm volatile("" : "+v"(xs[r][0]), "+v"(xs[r][1]), "+v"(xs[r][2]), "+v"(xs[r][3]));
        }
        __attribute__((address_space(1))) float *const xo = (__attribute__((address_space(1))) float *)nm.x_out;
#pragma unroll
        for (int r = 0; r < NR; r++) {
            const uint32_t col = wm::quad_col(r, c0);
            if (Q.valid(r, c0, nc) && col + 4 > lo && col < hi)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    if (col + i >= lo && col + i < hi) {
                        xo[col + i] = xs[r][i];
                        nonfinite |= !isfinite(xs[r][i]);
                    }
        }
    }
    // the squares to LDS in column order: the exact sum's terms (also read
    // there by its slow paths)
#pragma unroll
    for (int r = 0; r < NR; r++) {
#pragma unroll
        for (int i = 0; i < 4; i++) Q.v[r][i] = combine(Q.v[r][i], yq[r][i]);
        if (Q.valid(r, c0, nc))
            *reinterpret_cast<float4 *>(sq + wm::quad_col(r, c0)) =
                make_float4(Q.v[r][0] * Q.v[r][0], Q.v[r][1] * Q.v[r][1], Q.v[r][2] * Q.v[r][2],
                            Q.v[r][3] * Q.v[r][3]);
    }
    wm::fused_max_candidates<NR, W>(Q, c0, nc, nl);
    wm_sync_lds();
    // The weights go out once every wave's norm inputs are in (after the
    // squares' barrier; the dots need them only during the walk): issued
    // behind each wave's own inputs, the CU's memory path served the later
    // waves' inputs behind the earlier waves' weights, and the norm waits for
    // the last of them (gate/up 7.30 -> 6.72 us, down 9.59 -> 9.32).
    // (NP bounds the chunks per wave: at most 4 chunks, one round, when NP <= 4)
    i2s_round<UG> A, B;
    if (nc > 0) i2s_issue_ks<UG, KS>(A, wp, 0, nc, sub, (nc + KS - 1) / KS);
    if constexpr (NP > 4 && KS == 1)
        if (nc > 4) i2s_issue<UG>(B, wp, 4, nc);  // and the second round, if the slice has one
    __builtin_amdgcn_sched_barrier(0);
    float v2[NP];  // this thread's run of terms (NP divides n: a run lies wholly inside or past it)
    if (k0 < n) {
        if constexpr (NP >= 4) {
#pragma unroll
            for (int j = 0; j < NP; j += 4) {
                const float4 f = *reinterpret_cast<const float4 *>(sq + k0 + j);
                v2[j] = f.x;
                v2[j + 1] = f.y;
                v2[j + 2] = f.z;
                v2[j + 3] = f.w;
            }
        } else {
#pragma unroll
            for (int j = 0; j < NP; j++) v2[j] = sq[k0 + j];
        }
    } else {
#pragma unroll
        for (int j = 0; j < NP; j++) v2[j] = 0.0f;
    }
    uint8_t *const act8 = reinterpret_cast<uint8_t *>(act_s);
    // the dots over this wave's slice, from the codes in act and the weights
    // resident in A (and B): part[q] = Σ c a over the slice for group q
    int part[UG];
    const auto dots = [&]() {
        int acc16[UG], acc4[UG], acc1[UG];
#pragma unroll
        for (int q = 0; q < UG; q++) acc16[q] = acc4[q] = acc1[q] = 0;
        if (nc > 0) {
            const uint32_t nk = (nc + KS - 1) / KS;  // chunk registers of the lanes with the most
            i2s_reduce_ks<UG, KS>(A, act_s + c0 * 16, zeros, 0, min(nk, 4u), nc, sub, acc16, acc4, acc1);
            if constexpr (NP > 4 && KS == 1)
                if (nc > 4) i2s_reduce<UG>(B, act_s + c0 * 16, 4, nc - 4, acc16, acc4, acc1);
        }
#pragma unroll
        for (int q = 0; q < UG; q++) part[q] = (acc16[q] >> 4) + (acc4[q] >> 2) + acc1[q];
    };
    // Speculation (waves 1..W-1 while wave 0 walks the exact sum): codes
    // from the rsqrt of the float64 total of the squares, which is within a
    // few ulps of the exact one, and their dots.  Afterwards only elements
    // whose |y * inv| lies within the rsqrt's possible effect of a rounding
    // boundary are redone exactly, and the difference in each such code
    // corrected in the integer dot: the result is exactly the exact codes'.
    uint32_t qw[NR];
    float dist[NR][4];
    float dmin = 1.0f;  // this lane's smallest dist (1: none)
    int wave_asum = 0;
    float rsq_s = 0.0f, max_s = 0.0f;
    bool spec_ok = false;
    wm::fused_cand_regs cand{};
    wm::seq_sum_block_owned<NP, W * 64>(
        v2, n, sq, &nl.seq, NP,
        [&]() {
            if (wid == 0) {
                if (SPEC) __builtin_amdgcn_s_setprio(3);  // the walk is the critical path
            } else if (SPEC) {
                rsq_s = nl.spec_rsq;
                max_s = nl.spec_max;
                spec_ok = max_s >= 0.0f;
                if (spec_ok) {
                    wave_asum = wm::fused_codes<NR, true>(Q, c0, nc, rsq_s, max_s, act8, qw, dist);
#pragma unroll
                    for (int r = 0; r < NR; r++)
                        if (Q.valid(r, c0, nc))
#pragma unroll
                            for (int i = 0; i < 4; i++) dmin = fminf(dmin, dist[r][i]);
                    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                    __builtin_amdgcn_wave_barrier();
                    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                    dots();
                }
            }
        },
        [&](float sum_sq) {
            wm::fused_publish<W>(sum_sq, n, nm.eps, cand, nl, (chunks_flags & FUSED_NO_CANDIDATES) != 0);
        },
        [&]() {
            // Wave 0's copy of the candidate lists (complete since before the
            // sum), read here, ahead of the other waves' dots, which keep
            // LDS busy while wave 0 walks the sum, and reduced as far as it
            // goes without the rsqrt.
            if (wid == 0) {
                cand = wm::fused_cand_fetch<W>(nl);
                wm::fused_cand_prep(cand);
            }
            // The speculation's rsqrt and max|y|, once, by the last wave (at
            // these sizes it holds no terms of the sum and waits anyway):
            // the rsqrt of the waves' float64 total, max|y| from the
            // candidates, -1 where the candidate bound does not hold.
            if (SPEC && wid == W - 1) {
                double S = 0.0;
#pragma unroll
                for (int i = 0; i < W; i++) S += nl.seq.dw[i];
                const float r = wm::norm_rsq((float)S, n, nm.eps);
                wm::fused_cand_regs c = wm::fused_cand_fetch<W>(nl);
                wm::fused_cand_prep(c);
                bool ok;
                float m = wm::fused_cand_max(c, r, ok);
                // (test hooks: a skewed max|y| moves every code's p = y * 127 / max|y|;
                // a skewed rsqrt alone would cancel in p)
                if (chunks_flags & FUSED_SKEW_SMALL) m = m * (1.0f + 0x1p-12f);
                if (chunks_flags & FUSED_SKEW_LARGE) m = m * (1.0f + 0x1p-7f);
                if (lane == 0) {
                    nl.spec_rsq = r;
                    nl.spec_max = ok && r > 0.0f && r < 0x1p100f ? m : -1.0f;
                }
            }
        });
    if (SPEC && wid == 0) __builtin_amdgcn_s_setprio(0);
    // the exact rsqrt and max|y| (wave 0); max|y| from every wave's own
    // maximum when the candidates could not settle it
    const float rsq = nl.rsq;
    float max_abs = nl.maxabs;
    const bool fallback = max_abs < 0.0f;  // the same in every wave
    if (fallback) max_abs = wm::fused_block_max<NR, W>(Q, c0, nc, rsq, nl);
    bool redo = !SPEC || !spec_ok || fallback;
    if (!redo && (rsq != rsq_s || max_abs != max_s)) {
        // |p - p'| <= |p'| (rho + 8u) with p = ((x r) w) inv, p' the same with
        // r', inv' and rho = |(r / r')(M' / M) - 1| (eight roundings of at most
        // u = 2^-24 between them), |p'| < 128; plus 2^-40 for a subnormal y.
        const double rho = fabs(((double)rsq * (double)max_s) / ((double)rsq_s * (double)max_abs) - 1.0);
        const float bound = (float)(128.0 * (rho + 9.0 * 0x1p-24) + 0x1p-40);
        const float inv = 127.0f / max_abs;
        int n_fix = 0;
        // (usually no element of the wave is that close: one test for all)
        const bool any_close = __builtin_amdgcn_ballot_w64(dmin <= bound) != 0;
#pragma unroll
        for (int r = 0; r < NR; r++) {
            if (!any_close) break;
            const bool ok = Q.valid(r, c0, nc);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                uint64_t m = __builtin_amdgcn_ballot_w64(ok && dist[r][i] <= bound);
                while (m) {
                    const int l = __builtin_ctzll(m);
                    m &= m - 1;
                    if (++n_fix > 16) break;
                    // element (r, i) of lane l: its exact code and the change
                    const float v = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(Q.v[r][i]), l));
                    const float w = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(Q.w[r][i]), l));
                    const int qs = (int)(int8_t)(uint8_t)(__builtin_amdgcn_readlane((int)qw[r], l) >> (8 * i));
                    const int qe = wm_round_clamp_i8_fast(((v * rsq) * w) * inv);
                    const int d = qe - qs;
                    if (d != 0) {
                        wave_asum += d;
                        // the weight code of that column in this lane's row:
                        // chunk u of the slice (register (u - sub) / KS of
                        // the lanes of sub-slice u % KS; the others add 0),
                        // byte b of the chunk (quarter b / 16 from the top
                        // bit pair, gp = b % 16)
                        const uint32_t u = 4u * (uint32_t)r + ((uint32_t)l >> 4), b = 4u * ((uint32_t)l & 15u) + (uint32_t)i;
                        // The dword holding it, picked with masks the
                        // compiler cannot see through (a select on u would
                        // become an indexed access and put the resident
                        // weights in scratch memory).
                        const uint32_t g = (b & 15u) >> 2;
                        constexpr int NK = NP > 4 && KS == 1 ? 8 : 4;
                        uint32_t mk[NK][4];
#pragma unroll
                        for (int k = 0; k < NK; k++)
#pragma unroll
                            for (int j = 0; j < 4; j++) {
                                mk[k][j] = u == sub + KS * (uint32_t)k && g == (uint32_t)j ? 0xFFFFFFFFu : 0u;
                                asm volatile("" : "+v"(mk[k][j]));
                            }
#pragma unroll
                        for (int q = 0; q < UG; q++) {
                            uint32_t dw = 0;
#pragma unroll
                            for (int k = 0; k < NK; k++) {
                                const uint4 ch = k < 4 ? A.v[k & 3][q] : B.v[k & 3][q];
                                dw |= (ch.x & mk[k][0]) | (ch.y & mk[k][1]) | (ch.z & mk[k][2]) | (ch.w & mk[k][3]);
                            }
                            // part holds Σ c a (c = ternary + 1); Σ a is corrected apart
                            const uint32_t code = (dw >> (8u * (b & 3u) + 6u - 2u * (b >> 4))) & 3u;
                            part[q] += (int)code * d;
                        }
                    }
                }
            }
        }
        redo = n_fix > 16;  // too many to correct one by one
    }
    if (redo) {  // the codes and dots from the exact rsqrt and max|y|
        wave_asum = wm::fused_codes<NR, false>(Q, c0, nc, rsq, max_abs, act8, qw, dist);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if constexpr (SPEC) {
            dots();
        } else {
            int acc16[UG], acc4[UG], acc1[UG];
#pragma unroll
            for (int q = 0; q < UG; q++) acc16[q] = acc4[q] = acc1[q] = 0;
            if constexpr (NP > 4)
                i2s_rounds<UG>(A, B, wp, nc, act_s + c0 * 16, acc16, acc4, acc1, nc > 4);
            else
                i2s_reduce<UG>(A, act_s + c0 * 16, 0, nc, acc16, acc4, acc1);
#pragma unroll
            for (int q = 0; q < UG; q++) part[q] = (acc16[q] >> 4) + (acc4[q] >> 2) + acc1[q];
        }
    }
    if (SPEC && wid == 0) {
#pragma unroll
        for (int q = 0; q < UG; q++) part[q] = 0;
    }
    const float act_scale = max_abs == 0.0f ? 1.0f : max_abs / 127.0f;
    // At the end: the non-finite flag of x + y (every writer of this
    // launch writes the same tag; a flag already raised by an earlier layer
    // is kept).
    const auto finish = [&]() {
        if (nonfinite && nm.err_flag && *nm.err_flag == 0) *nm.err_flag = nm.layer_tag;
    };
    // this wave's share of Σ(c - 1) a = Σ c a - Σ a over its slice, each
    // row's KS lanes summed first (lanes l, l ^ R, l ^ 2R, ...)
#pragma unroll
    for (int q = 0; q < UG; q++) {
        int p = part[q];
        if constexpr (KS >= 8) p += __shfl_xor(p, 8, 64);
        if constexpr (KS >= 4) p += __shfl_xor(p, 16, 64);
        if constexpr (KS >= 2) p += __shfl_xor(p, 32, 64);
        if (lane < R) red[(wid * UG + q) * R + lane] = p - wave_asum;
    }
    wm_sync_lds();
    const uint32_t tid = threadIdx.x;
    if (MODE == WM_FUSED_GATEUP) {
        if (tid < R) {
            int dg = 0, du = 0;
#pragma unroll
            for (int w = 0; w < W; w++) {
                dg += red[(w * UG + 0) * R + tid];
                du += red[(w * UG + 1) * R + tid];
            }
            const float g = (w_scale * act_scale) * (float)dg;
            const float up = (w_scale1 * act_scale) * (float)du;
            const float r = g > 0.0f ? g : 0.0f;
            out_t[lu * 64 + h * R + tid] = (r * r) * up;
        }
        finish();
        return;
    }
    // the unit's outputs (row i of group q at out[64 q + i]); this workgroup
    // holds rows h R .. h R + R - 1 of each group, ys[R q + i - h R]
    float *out = out_t + (uint64_t)lu * UG * 64;
    for (uint32_t idx = tid; idx < UG * R; idx += W * 64) {
        const uint32_t q = idx / R, rr = idx % R;
        int dot = 0;
#pragma unroll
        for (int w = 0; w < W; w++) dot += red[(w * UG + q) * R + rr];
        const float y = (w_scale * act_scale) * (float)dot;
        if (MODE == WM_FUSED_PLAIN) {
            out[q * 64 + h * R + rr] = y;
        } else {
            ys[idx] = y;
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
        if (tid < n_pairs) {
            const uint32_t j = pair0 + tid;  // the pair (j, j + half) of the head
            const float x0 = ys[tid], x1 = ys[tid + (KS == 1 ? half : R)];
            const float r0 = x0 * rc - x1 * rsn, r1 = x0 * rsn + x1 * rc;
            out[j] = r0;
            out[j + half] = r1;
            mx = wm_max_nonan(wm_max_nonan(mx, fabsf(r0)), fabsf(r1));
        }
        if constexpr (KS == 1)
            for (uint32_t j = n_rot + tid; j < UG * 64; j += W * 64) {
                out[j] = ys[j];
                mx = wm_max_nonan(mx, fabsf(ys[j]));
            }
    } else {
        for (uint32_t idx = tid; idx < UG * R; idx += W * 64) {
            out[(idx / R) * 64 + h * R + idx % R] = ys[idx];
            mx = wm_max_nonan(mx, fabsf(ys[idx]));
        }
    }
    // KVCache::append needs each of K and V's absmax over all heads: waves
    // 0 and 1, which hold every output (at most 128 per workgroup), store
    // their maxima to slots of their own (2 lk + wid), every launch; the
    // consumer takes the maximum over the slots (no atomics: on a launch of
    // a few hundred workgroups same-address atomics serialise)
    if (t >= 1 && absmax && wid < 2) {
        mx = wm_wave_max_nonneg(mx);
        if (lane == 0) absmax[(t - 1) * absmax_stride + 2 * lk + wid] = __float_as_uint(mx);
    }
    finish();
}

// --------------------------------------------------------------------------
// The standalone matvec in one launch (bitlinear_i2s_matvec_f32,
// src/model/bitlinear.rs:67; the quantiser of bitlinear_sse2.rs:285-304 on
// the raw input, then the ternary dots, bitlinear_sse2.rs:327-339).
//
// One workgroup per 64 / KS rows of a 64-row group (KS lanes per row, as in
// k_i2s_fused).  Its W waves split the chunks of K between them (wave w:
// chunks [n_chunks*w/W, n_chunks*(w+1)/W), at most NC); each wave loads its
// slice of x in the quantiser's layout and its slice of the weights, the
// workgroup takes max|x| (NaN never counted: an order-free maximum, so every
// workgroup gets the same one), each wave quantises its own slice into LDS
// and dots its rows over it, and the partial dots (exact integers) meet in
// LDS.  Workgroup 0 also writes the codes (the permuted layout of
// wm_act_perm) and the scale and Σq when asked.
// --------------------------------------------------------------------------
template <int W, int NC, int KS>
__global__ __launch_bounds__(W * 64) void k_i2s_matvec_one(const float *x, const uint8_t *w, uint32_t n_chunks,
                                                           uint32_t out_dim, float w_scale, float *y,
                                                           int32_t *dot_out, uint8_t *act_out,
                                                           wm_act_meta *meta_out) {
    static_assert(NC <= 4 * KS, "one register round of chunks per lane");
    // act [n_chunks*16 ints] | zeros [16] | red [W][64]
    extern __shared__ __align__(16) int smem[];
    __shared__ float wave_max[W];
    __shared__ int wave_q[W];
    constexpr int NR = (NC + 3) / 4;  // quantiser rounds: four chunks per round
    constexpr uint32_t R = 64 / KS;
    const uint32_t g = blockIdx.x / KS, h = blockIdx.x % KS;
    const uint32_t wid = (uint32_t)__builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const uint32_t lane = threadIdx.x & 63, tid = threadIdx.x;
    const uint32_t sub = lane / R, row = h * R + lane % R;
    const uint32_t c0 = n_chunks * wid / W, nc = n_chunks * (wid + 1) / W - c0;
    const uint32_t n = n_chunks * 64;
    const uint4 *wp[1] = {reinterpret_cast<const uint4 *>(w) + ((uint64_t)g * n_chunks + c0) * I2S_GROUP_ROWS + row};
    i2s_round<1> A;
    if (nc > 0) i2s_issue_ks<1, KS>(A, wp, 0, nc, sub, (nc + KS - 1) / KS);
    int *act_s = smem;
    int *zeros = smem + n_chunks * 16;
    int *red = zeros + 16;
    uint8_t *const act8 = reinterpret_cast<uint8_t *>(act_s);
    const __amdgpu_buffer_rsrc_t rx = wm_rsrc(x, n * 4);
    wm::fused_quads<NR> Q;
#pragma unroll
    for (int r = 0; r < NR; r++) {
        const uint32_t off = Q.valid(r, c0, nc) ? wm::quad_col(r, c0) * 4 : n * 4;  // past the end: zeros
        wm::buf_run<4>(rx, off, Q.v[r]);
#pragma unroll
        for (int i = 0; i < 4; i++) Q.w[r][i] = 1.0f;  // no norm: y = x exactly
    }
    if (KS > 1 && tid < 16) zeros[tid] = 0;
    float m = 0.0f;
#pragma unroll
    for (int r = 0; r < NR; r++)
        if (Q.valid(r, c0, nc))
#pragma unroll
            for (int i = 0; i < 4; i++) m = wm_max_nonan(m, fabsf(Q.v[r][i]));
    m = wm_wave_max_nonan(m);
    if (lane == 0) wave_max[wid] = m;
    wm_sync_lds();
    float max_abs = wave_max[0];
#pragma unroll
    for (int i = 1; i < W; i++) max_abs = wm_max_nonan(max_abs, wave_max[i]);
    uint32_t qw[NR];
    float dist[NR][4];
    const int wave_asum = wm::fused_codes<NR, false>(Q, c0, nc, 1.0f, max_abs, act8, qw, dist);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    int acc16[1] = {0}, acc4[1] = {0}, acc1[1] = {0};
    if (nc > 0)
        i2s_reduce_ks<1, KS>(A, act_s + c0 * 16, zeros, 0, (nc + KS - 1) / KS, nc, sub, acc16, acc4, acc1);
    int p = (acc16[0] >> 4) + (acc4[0] >> 2) + acc1[0];
    if constexpr (KS >= 8) p += __shfl_xor(p, 8, 64);
    if constexpr (KS >= 4) p += __shfl_xor(p, 16, 64);
    if constexpr (KS >= 2) p += __shfl_xor(p, 32, 64);
    if (lane < R) red[wid * R + lane] = p - wave_asum;  // Σ(c - 1) a over the wave's slice
    if (lane == 0) wave_q[wid] = wave_asum;
    wm_sync_lds();
    const float act_scale = max_abs == 0.0f ? 1.0f : max_abs / 127.0f;
    if (tid < R) {
        int dot = 0;
#pragma unroll
        for (int i = 0; i < W; i++) dot += red[i * R + tid];
        const uint32_t j = g * 64 + h * R + tid;
        if (j < out_dim) {
            y[j] = (w_scale * act_scale) * (float)dot;
            if (dot_out) dot_out[j] = dot;
        }
    }
    if (blockIdx.x == 0) {
        if (act_out)
            for (uint32_t i = tid; i < n_chunks * 16; i += W * 64)
                reinterpret_cast<int *>(act_out)[i] = act_s[i];
        if (meta_out && tid == 0) {
            int q = 0;
#pragma unroll
            for (int i = 0; i < W; i++) q += wave_q[i];
            meta_out->scale = act_scale;
            meta_out->asum = q;
        }
    }
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
bool wm_launch_i2s_matvec_one(const uint8_t *w, uint32_t n_groups, uint32_t n_chunks, uint32_t out_dim,
                              float w_scale, const float *x, float *y, int32_t *dot_out, uint8_t *act_out,
                              wm_act_meta *meta_out, hipStream_t s) {
    if (n_groups == 0 || n_chunks == 0 || n_chunks > 256) return false;
    // W: the fewest waves that keep a wave's chunks within 16 (4 waves up to
    // 64 chunks): with the input spread over fewer waves the launch starts
    // fewer of them and the workgroup's two barriers are narrower (2560
    // columns: 4.6 us with 16 waves, 4.3 with 8, 3.9-4.3 with 4).
    const int W = n_chunks <= 64 ? 4 : (n_chunks <= 128 ? 8 : 16);
    // NC: a power of two >= ceil(n_chunks / W), at most 16
    uint32_t nc = 1;
    while (nc * (uint32_t)W < n_chunks) nc *= 2;
    // KS: as many workgroups per group as keep the grid within one per CU
    // (at least NC / 4: one register round of chunks per lane)
    static const uint32_t n_cus = [] {
        int dev = 0, c = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0)
            c = 256;
        return (uint32_t)c;
    }();
    uint32_t ks = 1;
    while (ks < 8 && (uint64_t)n_groups * ks * 2 <= n_cus) ks *= 2;
    while (ks * 4 < nc) ks *= 2;
    const uint64_t grid = (uint64_t)n_groups * ks;
    if (grid > 0x7FFFFFFFu) return false;
    const size_t lds = (size_t)n_chunks * 64 + 64 + (size_t)W * 64 * 4;
#define WM_MV_CASE(WW, NC, KS)                                                                     \
    if (W == WW && nc == NC && ks == KS) {                                                         \
        hipLaunchKernelGGL((k_i2s_matvec_one<WW, NC, KS>), dim3((uint32_t)grid), dim3(WW * 64), lds, s, x, w, \
                           n_chunks, out_dim, w_scale, y, dot_out, act_out, meta_out);             \
        return true;                                                                               \
    }
    WM_MV_CASE(4, 1, 1) WM_MV_CASE(4, 1, 2) WM_MV_CASE(4, 1, 4) WM_MV_CASE(4, 1, 8)
    WM_MV_CASE(4, 2, 1) WM_MV_CASE(4, 2, 2) WM_MV_CASE(4, 2, 4) WM_MV_CASE(4, 2, 8)
    WM_MV_CASE(4, 4, 1) WM_MV_CASE(4, 4, 2) WM_MV_CASE(4, 4, 4) WM_MV_CASE(4, 4, 8)
    WM_MV_CASE(4, 8, 2) WM_MV_CASE(4, 8, 4) WM_MV_CASE(4, 8, 8)
    WM_MV_CASE(4, 16, 4) WM_MV_CASE(4, 16, 8)
    WM_MV_CASE(8, 16, 4) WM_MV_CASE(8, 16, 8)
    WM_MV_CASE(16, 16, 4) WM_MV_CASE(16, 16, 8)
#undef WM_MV_CASE
    return false;
}

bool wm_launch_i2s_fused(int mode, const wm_i2s_desc *descs, const float *w_scales, float *const *outs,
                         int n_tensors, uint32_t n_chunks, uint32_t groups_per_unit,
                         const wm_fused_norm &norm, const float *rope_cos, const float *rope_sin,
                         uint32_t pos, uint32_t n_rot, uint32_t rope_mask, const wm_fused_absmax *absmax,
                         hipStream_t s, const uint32_t *pos_dev) {
    if (n_tensors < 1 || n_tensors > WM_FUSED_MAX_TENSORS) return false;
    i2s_fused_args a{};
    const uint8_t *wts[WM_FUSED_MAX_TENSORS] = {};
    uint32_t unit_end[WM_FUSED_MAX_TENSORS] = {};
    uint32_t acc = 0;
    for (int i = 0; i < n_tensors; i++) {
        wts[i] = descs[i].w;
        a.w_scale[i] = w_scales[i];
        a.out[i] = outs[i];
        // units: PLAIN one per group, ROPE one per head (UG groups), GATEUP one
        // per group pair (counted on the gate tensor only)
        const uint32_t units = mode == WM_FUSED_GATEUP ? (i == 0 ? descs[0].n_groups : 0)
                                                       : descs[i].n_groups / groups_per_unit;
        acc += units;
        unit_end[i] = acc;
    }
    // the units of tensor 1 begin at ue0, those of tensor 2 at ue1 (past the
    // grid: no such tensor; GATEUP's units all belong to the pair)
    const bool pair = mode == WM_FUSED_GATEUP;
    if (acc >= 0xFFFFu || n_chunks > 0xFFFFu) return false;  // 16-bit unit and chunk counts (again x KS below)
    const uint32_t ue0 = !pair && n_tensors > 1 ? unit_end[0] : 0xFFFFu;
    const uint32_t ue1 = !pair && n_tensors > 2 ? unit_end[1] : 0xFFFFu;
    a.x_out = norm.x_out;
    a.eps = norm.eps;
    a.err_flag = norm.err_flag;
    a.layer_tag = norm.layer_tag;
    a.rope_cos = rope_cos;
    a.rope_sin = rope_sin;
    a.pos = pos;
    a.pos_dev = pos_dev;
    a.n_rot = n_rot;
    a.rope_mask = rope_mask;
    a.absmax = absmax ? absmax->slots : nullptr;
    a.absmax_stride = absmax ? absmax->stride : 0;
    const uint32_t chunks_flags = n_chunks | (norm.relu2_mul ? FUSED_RELU2 : 0u) |
                                  (norm.debug & WM_FUSED_DEBUG_SKEW_SMALL ? FUSED_SKEW_SMALL : 0u) |
                                  (norm.debug & WM_FUSED_DEBUG_SKEW_LARGE ? FUSED_SKEW_LARGE : 0u) |
                                  (norm.debug & WM_FUSED_DEBUG_NO_CANDIDATES ? FUSED_NO_CANDIDATES : 0u);
    // Waves: as many as the chunks allow, up to 16 (the norm at the start is
    // latency-bound and runs best on the widest workgroup; each wave still
    // has its own chunks), rounded down to an instantiated count.
    int w = (int)(n_chunks < 16 ? n_chunks : 16);
    static const int kWs[] = {16, 8, 4, 2, 1};
    for (int x : kWs)
        if (w >= x) { w = x; break; }
    // NP: the exact sum's terms per thread and the bound on a wave's chunks,
    // a power of two (it then divides n, so no thread's run straddles the
    // end).  With at least two waves and NP <= 8 the kernel speculates and
    // spreads the chunks over waves 1..w-1; otherwise over all w waves.
    const auto pow2 = [](uint32_t v) {
        int p = 1;
        while ((uint32_t)p < v) p *= 2;
        return p;
    };
    int np = w >= 2 ? pow2((n_chunks + (uint32_t)w - 2) / (uint32_t)(w - 1)) : 1;
    if (np > 8) np = 16;  // no speculation: ceil(n_chunks / w) <= 16 for n_chunks <= 256
    // KS: lanes per row.  The units of a launch are few (a layer's 64-row
    // groups), and each workgroup's dots run on one CU's four SIMDs, so a
    // unit is split over KS workgroups while the grid stays within one
    // workgroup per CU: each has 1/KS of the dots and the weight loads, and
    // the norm (the same in every workgroup) costs no more.  The 16-wave
    // speculating form only, PLAIN or whole-head ROPE (a 128-wide rotation
    // over two groups, or none): a rotation pair then lies in one workgroup.
    static const uint32_t n_cus = [] {
        int dev = 0, c = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0)
            c = 256;
        return (uint32_t)c;
    }();
    uint32_t ks = 1;
    const bool ks_form = w == 16 && np <= 8 &&
                         (mode == WM_FUSED_PLAIN ||
                          (mode == WM_FUSED_ROPE && groups_per_unit == 2 && (rope_mask == 0 || n_rot == 128)));
    if (ks_form)
        while (ks < 8 && acc * ks * 2 <= n_cus) ks *= 2;
    const uint32_t grid = acc * ks;
    if (grid >= 0xFFFFu) return false;
    // (each workgroup's share of x_out is split in 32-bit arithmetic)
    if ((uint64_t)n_chunks * I2S_CHUNK_COLS * grid >= (1ull << 32)) return false;
    const uint32_t units01 = (ue0 == 0xFFFFu ? ue0 : ue0 * ks) | (ue1 == 0xFFFFu ? ue1 : ue1 * ks) << 16;
    if (absmax) {  // two slots per workgroup of tensors 1 and 2
        uint32_t most = 0;
        for (int i = 1; i < n_tensors; i++) most = std::max(most, 2 * (unit_end[i] - unit_end[i - 1]) * ks);
        if (mode != WM_FUSED_ROPE || most > absmax->stride) return false;
        *absmax->n_slots = most;
    }
    const size_t sq_bytes = (size_t)wm::seq_sum_padded(n_chunks * 64) * 4;
#define WM_FUSED_CASE(MODE, UG, W, NP, KS)                                                         \
    if (w == W && np == NP && ks == KS) {                                                          \
        const size_t lds = (size_t)n_chunks * 64 + 64 + (size_t)W * UG * 64 * 4 +                  \
                           (size_t)UG * 64 * 4 + sq_bytes;                                         \
        hipLaunchKernelGGL((k_i2s_fused<MODE, UG, W, NP, KS>), dim3(grid), dim3(W * 64), lds, s,   \
                           norm.x, norm.y, norm.w, wts[0], wts[1], wts[2], units01, chunks_flags, a); \
        return true;                                                                               \
    }
#define WM_FUSED_WS(MODE, UG)                                                                      \
    WM_FUSED_CASE(MODE, UG, 1, 1, 1) WM_FUSED_CASE(MODE, UG, 2, 2, 1) WM_FUSED_CASE(MODE, UG, 2, 4, 1) \
    WM_FUSED_CASE(MODE, UG, 4, 2, 1) WM_FUSED_CASE(MODE, UG, 4, 4, 1) WM_FUSED_CASE(MODE, UG, 8, 2, 1) \
    WM_FUSED_CASE(MODE, UG, 8, 4, 1) WM_FUSED_CASE(MODE, UG, 16, 2, 1)                               \
    WM_FUSED_CASE(MODE, UG, 16, 4, 1) WM_FUSED_CASE(MODE, UG, 16, 8, 1)                              \
    WM_FUSED_CASE(MODE, UG, 16, 16, 1)
#define WM_FUSED_KS(MODE, UG)                                                                      \
    WM_FUSED_CASE(MODE, UG, 16, 2, 2) WM_FUSED_CASE(MODE, UG, 16, 4, 2)                              \
    WM_FUSED_CASE(MODE, UG, 16, 8, 2) WM_FUSED_CASE(MODE, UG, 16, 2, 4)                              \
    WM_FUSED_CASE(MODE, UG, 16, 4, 4) WM_FUSED_CASE(MODE, UG, 16, 8, 4)                              \
    WM_FUSED_CASE(MODE, UG, 16, 2, 8) WM_FUSED_CASE(MODE, UG, 16, 4, 8)                              \
    WM_FUSED_CASE(MODE, UG, 16, 8, 8)
    if (mode == WM_FUSED_PLAIN) { WM_FUSED_WS(WM_FUSED_PLAIN, 1) WM_FUSED_KS(WM_FUSED_PLAIN, 1) }
    else if (mode == WM_FUSED_GATEUP) { WM_FUSED_WS(WM_FUSED_GATEUP, 2) }
    else if (groups_per_unit == 2) { WM_FUSED_WS(WM_FUSED_ROPE, 2) WM_FUSED_KS(WM_FUSED_ROPE, 2) }
    else if (groups_per_unit == 1) { WM_FUSED_WS(WM_FUSED_ROPE, 1) }
#undef WM_FUSED_KS
#undef WM_FUSED_WS
#undef WM_FUSED_CASE
    return false;
}
