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
// denominator through wm::seq_sum_block_owned), so the output is
// bit-identical.
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
    // This token's K (after RoPE) and V, [kv_dim] f32: position n_past - 1
    // is not in the cache yet.  Each kernel quantises what it needs of them
    // exactly as KVCache::append does; one workgroup of each writes the
    // cache row (kv_dim bytes) and its scale.
    const float *k_new, *v_new;
    // absmax of k_new and v_new (float bits) as the QKV matvec leaves them:
    // slots whose maximum it is, k_new's [0, n), v_new's [stride, stride + n)
    const uint32_t *kv_absmax;
    uint32_t kv_absmax_n, kv_absmax_stride;
    // nullable: the token's position on the device (n_past = *pos_dev + 1,
    // for launches that are replayed at successive positions); the grid and
    // LDS are then sized for n_max, and a larger n_past launches nothing
    const uint32_t *pos_dev;
    uint32_t n_max;
};

__device__ __forceinline__ uint32_t attn_n_past(const attn_args &a) {
    return a.pos_dev ? *a.pos_dev + 1 : a.n_past;
}

constexpr uint32_t kMaxHeadDim = 128;

// KVCache::append's quantiser (src/model/kv_cache.rs:245-259) for one value,
// given the vector's absmax (NaN never raises it): a zero or non-finite
// absmax gives 0 with scale 0.
__device__ __forceinline__ bool kv_zero(float absmax) { return absmax == 0.0f || !isfinite(absmax); }
__device__ __forceinline__ int8_t kv_q(float v, float absmax) {
    return kv_zero(absmax) ? (int8_t)0 : (int8_t)wm_round_clamp_i8(v * (127.0f / absmax));
}
__device__ __forceinline__ float kv_scale(float absmax) { return kv_zero(absmax) ? 0.0f : absmax / 127.0f; }
// The absmax of k_new (which 0) or v_new (1) from its slots, in every lane
// of the calling wave (the slots hold non-negative floats, no NaN).
__device__ __forceinline__ float kv_absmax_of(const attn_args &a, uint32_t which) {
    const uint32_t *sl = a.kv_absmax + which * a.kv_absmax_stride;
    float m = 0.0f;
    for (uint32_t i = threadIdx.x & 63; i < a.kv_absmax_n; i += 64) m = fmaxf(m, __uint_as_float(sl[i]));
    return wm_wave_max_nonneg(m);
}

// scores[h][p] = (Σ_i q_h[i] * k_p[i]) * scale.  64 cached positions per
// workgroup of 256 threads; grid (n_heads, ceil((n_past - 1) / 64) + 1).
// Wave w computes the products q_i * k_i of dims [w*hd/4, (w+1)*hd/4) for
// the workgroup's 64 positions into LDS, then wave 0 adds each position's
// products in order, one lane per position (the sum is a dependent chain;
// the products are not, so four waves share them).  The last block of each
// head scores position n_past - 1, whose K row is this token's k_new
// quantised here exactly as KVCache::append does (head 0's also writes the
// row to the cache).  It runs beside the cached blocks instead of after its
// own loads.
constexpr int kScThreads = 256;
constexpr int kScStride = kMaxHeadDim + 4;  // floats per position row (16-byte rows, spread banks)
__global__ __launch_bounds__(kScThreads) void k_attn_scores(attn_args a) {
    __shared__ __align__(16) float prod[64 * kScStride];
    const uint32_t h = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const uint32_t n_past = attn_n_past(a);
    if (n_past > a.n_max) return;
    const uint32_t kvh = h / a.group, pnew = n_past - 1;
    const uint32_t n_cached_blocks = (pnew + 63) / 64;  // the block after them scores pnew
    if (blockIdx.y > n_cached_blocks) return;
    const float *qh = a.q + (uint64_t)h * a.head_dim;
    if (blockIdx.y == n_cached_blocks) {
        const float kabs = kv_absmax_of(a, 0);
        const float ksn = kv_scale(kabs);
        for (uint32_t i = tid; i < a.head_dim; i += kScThreads) {
            const float kd = (float)kv_q(a.k_new[kvh * a.head_dim + i], kabs) * ksn;  // read_into
            prod[i] = qh[i] * kd;
        }
        if (h == 0) {
            int8_t *k_row = const_cast<int8_t *>(a.k_cache) + (uint64_t)pnew * a.kv_dim;
            for (uint32_t i = tid; i < a.kv_dim; i += kScThreads) k_row[i] = kv_q(a.k_new[i], kabs);
            if (tid == 0) const_cast<float *>(a.k_scales)[pnew] = ksn;
        }
        wm_sync_lds();
        if (tid == 0) {
            float s = 0.0f;
            for (uint32_t i = 0; i < a.head_dim; i += 4) {
                const float4 f = *reinterpret_cast<const float4 *>(prod + i);
                s = s + f.x; s = s + f.y; s = s + f.z; s = s + f.w;
            }
            a.scores[(uint64_t)h * a.score_stride + pnew] = s * a.scale;
        }
        return;
    }
    const uint32_t p = blockIdx.y * 64 + lane;
    const bool live = p < pnew;
    // this wave's 16-byte segments of the K row: hd/64 of them (2 or 1)
    const uint32_t nseg = a.head_dim / 64, seg0 = wid * nseg;
    const int8_t *kp = a.k_cache + (uint64_t)(live ? p : 0) * a.kv_dim + kvh * a.head_dim;
    const float ksc = a.k_scales[live ? p : 0];
    int4 raw[2];
#pragma unroll
    for (int b = 0; b < 2; b++)  // both loads in flight together
        raw[b] = *reinterpret_cast<const int4 *>(kp + (seg0 + (b < (int)nseg ? b : 0)) * 16);
    float *row = prod + lane * kScStride;
#pragma unroll
    for (int b = 0; b < 2; b++) {
        if (b < (int)nseg) {
            const int8_t *kb = reinterpret_cast<const int8_t *>(&raw[b]);
            const uint32_t d0 = (seg0 + b) * 16;
#pragma unroll
            for (int t = 0; t < 16; t += 4) {
                float4 f;
                f.x = qh[d0 + t] * ((float)kb[t] * ksc);  // read_into: q as f32 * scale
                f.y = qh[d0 + t + 1] * ((float)kb[t + 1] * ksc);
                f.z = qh[d0 + t + 2] * ((float)kb[t + 2] * ksc);
                f.w = qh[d0 + t + 3] * ((float)kb[t + 3] * ksc);
                *reinterpret_cast<float4 *>(row + d0 + t) = f;
            }
        }
    }
    wm_sync_lds();
    if (wid == 0 && live) {
        float s = 0.0f;
        for (uint32_t i = 0; i < a.head_dim; i += 4) {
            const float4 f = *reinterpret_cast<const float4 *>(row + i);
            s = s + f.x; s = s + f.y; s = s + f.z; s = s + f.w;
        }
        a.scores[(uint64_t)h * a.score_stride + p] = s * a.scale;
    }
}

constexpr int kSvThreads = 1024;  // wave 0: the 16 chains; waves 1-15: products
constexpr int kSvDims = 16;        // head dims per workgroup (one 16-byte V segment)
constexpr int kSvTile = 240;       // positions per product tile
constexpr int kSvStride = 244;     // floats per dim row of a product tile (16-byte rows)
constexpr uint32_t kSvSerialSum = 64;  // longest exp list summed by one wave, one add at a time
static_assert(kSvTile * (kSvDims / 4) == kSvThreads - 64, "one 4-dim unit per producer thread");

// softmax over scores[h][0..n_past) then out[h][d] = Σ_p w_p * v_p[d] for
// the 16 dimensions d0..d0+15 of head h.  Grid (n_heads, head_dim / 16).
//
// The workgroup first pulls its whole V slice (n_past x 16 int8: one
// coalesced 16-byte load per position, 64 KB at 4096 positions) and the V
// scales into LDS and its head's scores into registers, all loads in flight
// at once.  All 16 waves then compute the softmax: max, exp, and the list of
// positions whose exp is not exactly 0 (kept in position order; a zero term
// changes neither the exp sum nor any output sum, so the reference's sums
// over all positions equal the sums over this list).  The exp sum runs over
// the list, left to right (one wave, one add at a time, for up to 64
// terms; the workgroup's exact sum seq_sum_block_owned beyond), then the
// normalisation.  Then,
// tile by tile, waves 1-15 write products w_p * v_p[d] (4 dims of one listed
// position per thread) while lanes 0-15 of wave 0 add the previous tile, one
// chain per dimension, in position order.  Position n_past - 1 uses this
// token's V, quantised from v_new (workgroup (0, 0) also writes the cache
// row).
// The largest of the workgroup's values (none of them NaN; -inf where a
// thread has none), in every thread: a DPP reduction per wave (-inf fills
// the lanes a shift leaves empty), one LDS exchange.  `red` is not in use
// before the call, so one barrier suffices.
__device__ __forceinline__ float sv_block_max(float v, float *red) {
    const int ninf = __float_as_int(-INFINITY);
#define SV_MAX_STEP(C, R) \
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(ninf, __float_as_int(v), C, R, 0xF, false)))
    SV_MAX_STEP(0x111, 0xF);  // row_shr:1
    SV_MAX_STEP(0x112, 0xF);  // row_shr:2
    SV_MAX_STEP(0x114, 0xF);  // row_shr:4
    SV_MAX_STEP(0x118, 0xF);  // row_shr:8
    SV_MAX_STEP(0x142, 0xA);  // row_bcast:15
    SV_MAX_STEP(0x143, 0xC);  // row_bcast:31
#undef SV_MAX_STEP
    const uint32_t lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    if (lane == 63) red[wid] = v;
    wm_sync_lds();
    float m = red[0];
#pragma unroll
    for (int w = 1; w < kSvThreads / 64; w++) m = fmaxf(m, red[w]);
    return m;
}

template <int MAXM>  // n_past <= MAXM * kSvThreads
__global__ __launch_bounds__(kSvThreads) void k_attn_softmax_v(attn_args a) {
    extern __shared__ __align__(16) float sm[];
    const uint32_t n = attn_n_past(a), pnew = n - 1;
    if (n > a.n_max) return;
    const uint32_t npad = (n + 3) & ~3u;
    float *cval = sm;                                     // [seq_sum_padded(n)] nonzero exps, then weights
    float *vsc = cval + wm::seq_sum_padded(n);            // [npad]
    int4 *vq = reinterpret_cast<int4 *>(vsc + npad);      // [npad] x 16 int8
    float *prod = reinterpret_cast<float *>(vq + npad);   // [2][kSvDims][kSvStride]
    uint16_t *cidx = reinterpret_cast<uint16_t *>(prod + 2 * kSvDims * kSvStride);  // [npad]
    __shared__ float red[16];
    __shared__ int wcnt[MAXM * 16];
    __shared__ float ssum;
    __shared__ wm::seq_block_scratch seq_scratch;
    __shared__ uint64_t exp_tab[32];
    const uint32_t h = blockIdx.x, d0 = blockIdx.y * kSvDims, tid = threadIdx.x;
    const uint32_t wid = (uint32_t)__builtin_amdgcn_readfirstlane((int)(tid >> 6)), lane = tid & 63;
    const uint32_t kvh = h / a.group;
    const int8_t *vseg = a.v_cache + kvh * a.head_dim + d0;
    const float *sc = a.scores + (uint64_t)h * a.score_stride;
    const float vabs = kv_absmax_of(a, 1);
    const bool v_writer = h == 0 && blockIdx.y == 0;
    if (tid < 32) exp_tab[tid] = wm::kExp2Tab[tid];
    // 1. the loads: thread t takes positions t + i * kSvThreads, its scores in
    //    registers, the V slice and scales into LDS; indices clamped so that
    //    every load is unconditional and all of them are in flight together
    float sv[MAXM];
    float m = -INFINITY;
    {
        int4 vr[MAXM];
        float ss[MAXM];
#pragma unroll
        for (int i = 0; i < MAXM; i++) {
            const uint32_t p = min(tid + (uint32_t)i * kSvThreads, n - 1);
            vr[i] = *reinterpret_cast<const int4 *>(vseg + (uint64_t)p * a.kv_dim);
            sv[i] = sc[p];
            ss[i] = a.v_scales[p];
        }
#pragma unroll
        for (int i = 0; i < MAXM; i++) {
            const uint32_t p = tid + (uint32_t)i * kSvThreads;
            if (p < n) m = wm_max_nonan(m, sv[i]);
            // the cache row of position n_past - 1 is stale (this token's V
            // is written below, by other threads, with no barrier between):
            // only the rows before it are copied
            if (p < pnew) {
                vq[p] = vr[i];
                vsc[p] = ss[i];
            }
        }
    }
    // this token's V (position n_past - 1 is not in the cache yet)
    if (tid < kSvDims)
        reinterpret_cast<int8_t *>(vq + pnew)[tid] = kv_q(a.v_new[kvh * a.head_dim + d0 + tid], vabs);
    if (tid == 0) vsc[pnew] = kv_scale(vabs);
    // 2. softmax (attention.rs:45-73)
    // (the thread maxima are never NaN: a NaN score never wins above; a zero
    // maximum's sign, which the reduction order could change, does not reach
    // exp(s - max))
    const float mx = sv_block_max(m, red);
    float *out = a.out + (uint64_t)h * a.head_dim + d0;
    if (!isfinite(mx)) {  // every weight becomes 0 -> output stays 0
        if (tid < kSvDims) out[tid] = 0.0f;
    } else {
        // exp(v - max) (attention.rs:62), then the positions whose exp is not
        // exactly 0, compacted in position order: a zero exp adds nothing to
        // the sum (s + 0 = s for every s the sum can hold), its weight
        // 0 * inv is 0 and its products w * v_p[d] are +-0, which leave every
        // output sum as it was (it starts at +0 and is never -0), so the
        // sum and the outputs over the compacted list are the reference's
        float e[MAXM];
        uint64_t mask[MAXM];
#pragma unroll
        for (int i = 0; i < MAXM; i++) {
            const uint32_t p = tid + (uint32_t)i * kSvThreads;
            e[i] = p < n ? wm::expf_glibc(sv[i] - mx, exp_tab) : 0.0f;
            mask[i] = __builtin_amdgcn_ballot_w64(e[i] != 0.0f);
            if (lane == 0) wcnt[i * 16 + wid] = __builtin_popcountll(mask[i]);
        }
        wm_sync_lds();
        // exclusive offsets of the (round, wave) groups, in position order
        const int c = lane < (uint32_t)(MAXM * 16) ? wcnt[lane] : 0;
        const int cinc = wm_wave_scan_i32(c);
        const uint32_t count = (uint32_t)__builtin_amdgcn_readlane(cinc, 63);
        const uint64_t below = (1ull << lane) - 1ull;
#pragma unroll
        for (int i = 0; i < MAXM; i++) {
            const int base = __builtin_amdgcn_readlane(cinc - c, i * 16 + (int)wid);
            if (e[i] != 0.0f) {
                const int k = base + __builtin_popcountll(mask[i] & below);
                cval[k] = e[i];
                cidx[k] = (uint16_t)(tid + (uint32_t)i * kSvThreads);
            }
        }
        wm_sync_lds();
        // Σ exp left to right (attention.rs:63-66) over the compacted terms:
        // up to kSvSerialSum by one wave, one add at a time; a longer list by
        // the workgroup's exact sum (thread t takes terms t*m .. t*m+m-1)
        float sum;
        if (count <= kSvSerialSum) {
            if (wid == 0) {
                // 64 terms per step, one per lane; the next step's terms are
                // read while this step's are added
                float s;
                asm volatile("v_mov_b32 %0, 0" : "=v"(s));
                float v = lane < count ? cval[lane] : 0.0f;
                for (uint32_t c = 0; c < count; c += 64) {
                    const uint32_t nx = c + 64 + lane;
                    const float vn = nx < count ? cval[nx] : 0.0f;
                    const uint32_t here = count - c < 64u ? count - c : 64u;
                    for (uint32_t k = 0; k < here; k++)
                        s = s + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), (int)k));
                    v = vn;
                }
                if (lane == 0) ssum = s;
            }
            wm_sync_lds();
            sum = ssum;
        } else {
            float ev[MAXM];
            const uint32_t mm = (count + kSvThreads - 1) / kSvThreads, k0 = tid * mm;
#pragma unroll
            for (int j = 0; j < MAXM; j++)
                ev[j] = ((uint32_t)j < mm && k0 + (uint32_t)j < count) ? cval[k0 + j] : 0.0f;
            sum = wm::seq_sum_block_owned<MAXM, kSvThreads>(ev, count, cval, &seq_scratch);
        }
        if (sum > 0.0f) {
            const float inv = 1.0f / sum;
            for (uint32_t k = tid; k < count; k += kSvThreads) cval[k] = cval[k] * inv;
        }
        wm_sync_lds();
        // 3. products of tile t (waves 1-15) while wave 0 adds tile t - 1,
        //    over the compacted positions in order
        const uint32_t n_tiles = (count + kSvTile - 1) / kSvTile;
        const uint32_t pt = tid - 64, dq = pt / kSvTile, pl = pt % kSvTile;  // producer unit
        float acc = 0.0f;
        // the chains are the critical path: wave 0's instructions go first
        // on its SIMD when a producer wave is ready at the same time
        if (wid == 0) __builtin_amdgcn_s_setprio(3);
        for (uint32_t t = 0; t <= n_tiles; t++) {
            if (wid >= 1) {
                if (t < n_tiles) {
                    const uint32_t k = t * kSvTile + pl;
                    if (k < count) {
                        const uint32_t p = cidx[k];
                        float *dst = prod + (t & 1) * (kSvDims * kSvStride) + dq * 4 * kSvStride + pl;
                        const uint32_t word = reinterpret_cast<const uint32_t *>(vq + p)[dq];
                        const float w = cval[k], s = vsc[p];
#pragma unroll
                        for (int i = 0; i < 4; i++) {
                            const float vd = (float)(int8_t)(word >> (8 * i)) * s;  // read_into: q * scale
                            dst[i * kSvStride] = w * vd;                             // w * v_h[d]
                        }
                    }
                }
            } else if (lane < kSvDims && t > 0) {
                const float *src = prod + ((t - 1) & 1) * (kSvDims * kSvStride) + lane * kSvStride;
                const uint32_t k0 = (t - 1) * kSvTile;
                const uint32_t tn = count - k0 < (uint32_t)kSvTile ? count - k0 : (uint32_t)kSvTile;
                if (tn == (uint32_t)kSvTile) {
                    // 24 products per step, the next step's reads issued before this step's adds
                    constexpr int kC = 6, kSteps = kSvTile / (4 * kC);
                    float4 f[2][kC];
#pragma unroll
                    for (int i = 0; i < kC; i++) f[0][i] = *reinterpret_cast<const float4 *>(src + 4 * i);
#pragma unroll
                    for (int c4 = 0; c4 < kSteps; c4++) {
                        if (c4 + 1 < kSteps) {
#pragma unroll
                            for (int i = 0; i < kC; i++)
                                f[(c4 + 1) & 1][i] = *reinterpret_cast<const float4 *>(src + (c4 + 1) * 4 * kC + 4 * i);
                        }
#pragma unroll
                        for (int i = 0; i < kC; i++) {
                            const float4 g = f[c4 & 1][i];
                            acc = acc + g.x; acc = acc + g.y; acc = acc + g.z; acc = acc + g.w;
                        }
                    }
                } else {
                    uint32_t q = 0;
                    for (; q + 4 <= tn; q += 4) {
                        const float4 g = *reinterpret_cast<const float4 *>(src + q);
                        acc = acc + g.x; acc = acc + g.y; acc = acc + g.z; acc = acc + g.w;
                    }
                    for (; q < tn; q++) acc = acc + src[q];
                }
            }
            wm_sync_lds();
        }
        if (wid == 0) __builtin_amdgcn_s_setprio(0);
        if (tid < kSvDims) out[tid] = acc;
    }
    if (v_writer) {  // the cache row of position n_past - 1
        int8_t *v_row = const_cast<int8_t *>(a.v_cache) + (uint64_t)pnew * a.kv_dim;
        for (uint32_t i = tid; i < a.kv_dim; i += kSvThreads) v_row[i] = kv_q(a.v_new[i], vabs);
        if (tid == 0) const_cast<float *>(a.v_scales)[pnew] = kv_scale(vabs);
    }
}

// single_token_attention_position_zero (src/model/attention.rs:135-194):
// one position, this token's K (after RoPE) and V as computed, not through
// the cache.  Per head h (one workgroup of head_dim threads): s =
// dot_f32(q_h, k_kvh) left to right, times scale; softmax of the one score
// is 1 for a finite s and 0 otherwise (attention.rs:45-73); out = w * v_kvh.
__global__ __launch_bounds__(kMaxHeadDim) void k_attn_position_zero(const float *q, const float *k,
                                                                    const float *v, float *out,
                                                                    uint32_t head_dim, uint32_t group,
                                                                    float scale) {
    __shared__ float w_s;
    const uint32_t h = blockIdx.x, kvh = h / group, tid = threadIdx.x;
    if (tid == 0) {
        const float *qh = q + (uint64_t)h * head_dim, *kh = k + (uint64_t)kvh * head_dim;
        float s = 0.0f;
        for (uint32_t i = 0; i < head_dim; i++) s = s + qh[i] * kh[i];
        const float sc = s * scale;
        // max over [sc] is sc unless sc is NaN (-inf stays); a non-finite
        // max zeroes the weights, else exp(sc - sc) / 1 = 1
        w_s = isfinite(sc) ? 1.0f : 0.0f;
    }
    wm_sync_lds();
    if (tid < head_dim) out[(uint64_t)h * head_dim + tid] = w_s * v[(uint64_t)kvh * head_dim + tid];
}

}  // namespace

// Returns false (nothing launched) for a shape the kernels do not cover:
// head_dim 64 or 128 (the scores kernel's four waves take head_dim / 64
// 16-byte segments each), n_past in [1, 4096].
bool wm_launch_attention(const float *q, const int8_t *k_cache, const float *k_scales,
                         const int8_t *v_cache, const float *v_scales, float *scores,
                         uint32_t score_stride, float *out, uint32_t n_heads, uint32_t n_kv_heads,
                         uint32_t head_dim, uint32_t n_past, float scale, const float *k_new,
                         const float *v_new, const uint32_t *kv_absmax, uint32_t kv_absmax_n,
                         uint32_t kv_absmax_stride, hipStream_t s,
                         const uint32_t *pos_dev, uint32_t n_max) {
    // with pos_dev, n_past comes from the device and n_max bounds it
    const uint32_t nb = pos_dev ? n_max : n_past;
    if ((head_dim != 64 && head_dim != 128) || nb == 0 || nb > 4 * kSvThreads ||
        nb > score_stride)
        return false;
    const uint32_t kv_dim = n_kv_heads * head_dim;
    attn_args a{q, k_cache, k_scales, v_cache, v_scales, scores, out, n_past, kv_dim, head_dim,
                n_heads / n_kv_heads, score_stride, scale, k_new, v_new, kv_absmax, kv_absmax_n,
                kv_absmax_stride, pos_dev, nb};
    hipLaunchKernelGGL(k_attn_scores, dim3(n_heads, (nb - 1 + 63) / 64 + 1), dim3(kScThreads), 0, s, a);
    const size_t npad = ((size_t)nb + 3) & ~(size_t)3;
    const size_t lds = (size_t)wm::seq_sum_padded(nb) * 4 + npad * (4 + 16) +
                       (size_t)2 * kSvDims * kSvStride * 4 + npad * 2;
    const dim3 grid(n_heads, head_dim / kSvDims);
    if (nb <= 2 * kSvThreads)
        hipLaunchKernelGGL(k_attn_softmax_v<2>, grid, dim3(kSvThreads), lds, s, a);
    else  // nb <= 4096, the models' context limit
        hipLaunchKernelGGL(k_attn_softmax_v<4>, grid, dim3(kSvThreads), lds, s, a);
    return true;
}

bool wm_launch_attention_position_zero(const float *q, const float *k_new, const float *v_new,
                                       float *out, uint32_t n_heads, uint32_t n_kv_heads,
                                       uint32_t head_dim, float scale, hipStream_t s) {
    if (head_dim == 0 || head_dim > kMaxHeadDim || n_kv_heads == 0 || n_heads % n_kv_heads) return false;
    hipLaunchKernelGGL(k_attn_position_zero, dim3(n_heads), dim3(kMaxHeadDim), 0, s, q, k_new, v_new,
                       out, head_dim, n_heads / n_kv_heads, scale);
    return true;
}
