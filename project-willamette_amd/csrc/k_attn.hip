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

// What the scores need first (the query, the K cache, this token's K, the
// geometry and the position) comes in the kernel's leading 14 argument
// dwords, which the hardware preloads into SGPRs at wave launch (the file is
// built with -amdgpu-kernarg-preload-count=16): six pointers, then
//   geom  = group | n_kv_heads << 8 | kv_absmax_n << 16
//   shape = (head_dim == 128) | sc_tile << 1 | nb << 12
// where sc_tile is the positions per score tile (group * ceil(sc_tile / 64)
// <= 16 waves) and nb the position count the launch is sized for: n_past, or
// with pos_dev the count the host expects the device word to give.  The rest
// is read from this struct once the first loads are out.
struct attn_args {
    const int8_t *v_cache;   // this layer: [max_seq][kv_dim]
    const float *v_scales;   // [max_seq]
    float *scores;           // [n_heads][score_stride]
    float *out;              // [n_heads][head_dim]
    uint32_t score_stride;
    float scale;
    // This token's V, [kv_dim] f32 (its K comes as an argument): position
    // n_past - 1 is not in the cache yet.  The kernel quantises what it needs
    // of k_new and v_new exactly as KVCache::append does and writes the cache
    // rows and scales.
    const float *v_new;
    // v_new's absmax slots begin at kv_absmax + kv_absmax_stride (k_new's at
    // kv_absmax; kv_absmax_n of each)
    uint32_t kv_absmax_stride;
    // this launch's tag on its scores (never 0, and never the tag of an
    // earlier launch whose words the scores buffer may still hold), the
    // step's error flag and the value a failed wait raises it to
    uint32_t tag;
    uint32_t *err_flag;
    uint32_t err_tag;
    uint32_t spin_limit; // polls before a wait gives up (0: at once, a test hook)
};

constexpr uint32_t kMaxHeadDim = 128;

// KVCache::append's quantiser (src/model/kv_cache.rs:245-259) for one value,
// given the vector's absmax (NaN never raises it): a zero or non-finite
// absmax gives 0 with scale 0.
__device__ __forceinline__ bool kv_zero(float absmax) { return absmax == 0.0f || !isfinite(absmax); }
__device__ __forceinline__ int8_t kv_q(float v, float absmax) {
    return kv_zero(absmax) ? (int8_t)0 : (int8_t)wm_round_clamp_i8(v * (127.0f / absmax));
}
__device__ __forceinline__ float kv_scale(float absmax) { return kv_zero(absmax) ? 0.0f : absmax / 127.0f; }
// The absmax of a vector from its n slots (as the QKV matvec leaves them:
// non-negative floats, no NaN, whose maximum it is), in every lane of the
// calling wave: the loads of the first 128 slots (kv_absmax_first, issued
// where the caller has other loads in flight), then the rest and the wave's
// maximum (kv_absmax_finish).
struct kv_absmax_part {
    float m0, m1;
};
__device__ __forceinline__ kv_absmax_part kv_absmax_first(const uint32_t *sl, uint32_t n) {
    const uint32_t l = threadIdx.x & 63;
    return {l < n ? __uint_as_float(sl[l]) : 0.0f, l + 64 < n ? __uint_as_float(sl[l + 64]) : 0.0f};
}
__device__ __forceinline__ float kv_absmax_finish(kv_absmax_part f, const uint32_t *sl, uint32_t n) {
    float m = fmaxf(f.m0, f.m1);
    for (uint32_t i = (threadIdx.x & 63) + 128; i < n; i += 64) m = fmaxf(m, __uint_as_float(sl[i]));
    return wm_wave_max_nonneg(m);
}
__device__ __forceinline__ float kv_absmax_of(const uint32_t *sl, uint32_t n) {
    return kv_absmax_finish(kv_absmax_first(sl, n), sl, n);
}

// Scores cross from the workgroups that compute them to the workgroups
// that use them inside one launch.  Each score is stored as one 64-bit word,
// (tag << 32) | bits, by an agent-scope atomic store (relaxed): on gfx950
// that goes through to the level every XCD's L2 agrees on, and a 64-bit
// aligned store is seen whole or not at all.  The tag is the launch's own
// (the host counts the launches), so a reader polls each of its scores with
// agent-scope atomic loads until it carries this launch's tag: no arrival
// counter, no fence, no L2 writeback or invalidation (__threadfence() or an
// acquire fence cost several microseconds per launch here), and no wait
// longer than the last score it needs.  A stale word can never pass for a
// fresh one, so the tags carry the correctness; the agent scope only makes
// the wait end.
__device__ __forceinline__ void st_tagged(uint64_t *p, uint32_t tag, float v) {
    __hip_atomic_store(p, ((uint64_t)tag << 32) | __float_as_uint(v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
// workgroup j of a kv head scores positions [p0_of(n, j, gs), p0_of(n, j + 1, gs))
// (n <= 4096 and j <= gs <= 256: n * j fits 32 bits, so the division is a
// 32-bit one, which the first loads' addresses wait for)
__device__ __forceinline__ uint32_t p0_of(uint32_t n, uint32_t j, uint32_t gs) {
    return n * j / gs;
}
__device__ __forceinline__ uint64_t ld_tagged(const uint64_t *p) {
    return __hip_atomic_load(const_cast<uint64_t *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

constexpr int kSvThreads = 1024;  // wave 0: the 16 chains; waves 1-15: products
constexpr int kSvDims = 16;        // head dims per workgroup (one 16-byte V segment)
constexpr int kSvTile = 240;       // positions per product tile
constexpr int kSvStride = 244;     // floats per dim row of a product tile (16-byte rows)
constexpr uint32_t kSvSerialSum = 64;  // longest exp list summed by one wave, one add at a time
static_assert(kSvTile * (kSvDims / 4) == kSvThreads - 64, "one 4-dim unit per producer thread");

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

// Decode attention for every head in one launch.  The gs = group *
// head_dim / 16 workgroups of kv head g share its K and V rows:
//
// 1. Scores.  Workgroup (g, j) takes positions [j n / gs, (j + 1) n / gs)
//    for all `group` query heads of g.  It loads those K rows once (one
//    16-byte segment per thread, with its scale), dequantises them as
//    read_into does into LDS rows, and each of its first group * np threads
//    forms one chain s = (Σ_i q_h[i] * k_p[i]) * scale, each product and add
//    in order over i (q from LDS, read by every thread of a head at once).
//    Position n - 1 is
//    this token's k_new, quantised here exactly as KVCache::append does (its
//    thread also writes the cache row segment, and kv head 0's the scale).
//    The scores go out tagged with the launch's epoch (st_tagged).
// 2. Workgroup (g, j) then serves query head g * group + j / (head_dim /
//    16) and its 16 dimensions d0 = 16 (j % (head_dim / 16)): each thread
//    polls its positions' scores until they carry this launch's tag, while
//    its V slice (n x 16 int8: one 16-byte load per position) and the V
//    scales come in.
// 3. Softmax and V.  All 16 waves compute the softmax: max, exp, and the
//    list of positions whose exp is not exactly 0 (kept in position order;
//    a zero term changes neither the exp sum nor any output sum, so the
//    reference's sums over all positions equal the sums over this list).
//    The exp sum runs over the list, left to right (one wave, one add at a
//    time, for up to 64 terms; the workgroup's exact sum
//    seq_sum_block_owned beyond), then the normalisation.  Then, tile by
//    tile, waves 1-15 write products w_p * v_p[d] (4 dims of one listed
//    position per thread) while lanes 0-15 of wave 0 add the previous tile,
//    one chain per dimension, in position order.  Position n - 1 uses this
//    token's V, quantised from v_new (workgroup j = 0 of each kv head also
//    writes the cache row segment, kv head 0's the scale).
//
// Every workgroup of the grid is resident at once (one per CU, at most 32
// per XCD, which the launcher checks), so every poll ends; it is bounded all
// the same.  K is read once per launch, and V once per XCD that serves one
// of its kv head's query heads: a query head's workgroups, which together
// read whole V lines, sit on one XCD, and the query heads are dealt to the
// 8 XCDs in turn (so that the XCDs share the work evenly).
//
// q [n_heads][head_dim], k_cache and k_scales (this layer's [max_seq][kv_dim]
// codes and [max_seq] scales), k_new (this token's K after RoPE, [kv_dim]
// f32), kv_absmax (the absmax slots) and pos_dev (nullable: the token's
// position on the device, n_past = *pos_dev + 1, for steps the host queues
// ahead; a count above nb launches nothing) lead the arguments; geom and
// shape are packed as described at attn_args.
template <int MAXM>  // n_past <= MAXM * kSvThreads
__global__ __launch_bounds__(kSvThreads) void k_attn_decode(const float *q, const int8_t *k_cache,
                                                            const float *k_scales, const float *k_new,
                                                            const uint32_t *kv_absmax, const uint32_t *pos_dev,
                                                            uint32_t geom, uint32_t shape, attn_args a) {
    extern __shared__ __align__(16) float sm[];
    __shared__ float red[16];
    __shared__ int wcnt[MAXM * 16];
    __shared__ wm::seq_block_scratch seq_scratch;
    __shared__ uint64_t exp_tab[32];
    const uint32_t group = geom & 0xFFu, n_kv_heads = (geom >> 8) & 0xFFu, kv_absmax_n = geom >> 16;
    const uint32_t hd = (shape & 1u) ? 128u : 64u, segs = hd / 16, segs_log2 = (shape & 1u) ? 3u : 2u;
    const uint32_t sc_tile = (shape >> 1) & 0x7FFu, nb = shape >> 12;
    const uint32_t gs = group * segs, kv_dim = n_kv_heads * hd;
    // Query head qh's segs workgroups (its 16-dimension slices, which
    // together read whole V lines) sit on one XCD, qh mod 8: the dispatcher
    // deals linear ids to the 8 XCDs in turn, and qh = 8k + x takes the ids
    // (k * segs + s) * 8 + x for its slices s.
    const uint32_t x8 = blockIdx.x % 8, slot = blockIdx.x / 8;
    const uint32_t qh = (slot >> segs_log2) * 8 + x8;
    if (qh >= group * n_kv_heads) return;
    const uint32_t g = qh / group, j = (qh % group) * segs + (slot & (segs - 1));
    // The position count.  Phase 1's loads go out for the launch's count nb
    // before the device word is read (each read sits where it is needed, so
    // that the wait for it comes after them); where the word gives another
    // count, phase 1 starts again with it (before any store).
    uint32_t n = nb, pnew = nb - 1;
    const auto dev_count_differs = [&]() { return pos_dev && *pos_dev + 1 != n; };
    const uint32_t tid = threadIdx.x;
    const uint32_t wid = (uint32_t)__builtin_amdgcn_readfirstlane((int)(tid >> 6)), lane = tid & 63;
    const uint32_t h = qh, d0 = (slot & (segs - 1)) * kSvDims;

    uint64_t *const scores64 = reinterpret_cast<uint64_t *>(a.scores);

    // ---- phase 1: scores of positions [p0, p1) for the group's heads ----
    const uint32_t pst = hd + 4;                  // floats per K row in LDS (spread banks)
    float *qs = sm;                               // [group][hd]
    float *kdl = sm + group * hd;                 // [sc_tile][pst] dequantised K rows
    const int8_t *kseg = k_cache + g * hd;
    const uint32_t row = tid >> segs_log2, sg = tid & (segs - 1);  // this thread's K row segment
    for (bool settled = false; !settled;) {
    settled = true;
    const uint32_t p0 = p0_of(n, j, gs), p1 = p0_of(n, j + 1, gs);
    for (uint32_t t0 = p0; t0 < p1; t0 += sc_tile) {
        const uint32_t tp = min(sc_tile, p1 - t0);
        const bool mine = row < tp, is_new = mine && t0 + row == pnew;
        // the loads, all issued together: this thread's 16-byte K segment
        // and its scale, or for the new position this token's k_new segment
        // (and, in its wave, the absmax slots); q of the group's heads
        uint32_t kw[4] = {0u, 0u, 0u, 0u};
        float ksc = 0.0f;
        float4 kn[4];
        if (mine && !is_new) {
            const int4 raw = *reinterpret_cast<const int4 *>(kseg + (uint64_t)(t0 + row) * kv_dim + sg * 16);
            kw[0] = (uint32_t)raw.x; kw[1] = (uint32_t)raw.y; kw[2] = (uint32_t)raw.z; kw[3] = (uint32_t)raw.w;
            ksc = k_scales[t0 + row];
        }
        if (is_new)
#pragma unroll
            for (int e = 0; e < 4; e++)
                kn[e] = *reinterpret_cast<const float4 *>(k_new + g * hd + sg * 16 + 4 * e);
        // (group * hd / 4 <= 512 float4 of q: one per thread at most)
        const bool q_mine = t0 == p0 && tid < group * hd / 4;
        float4 qv4;
        if (q_mine) qv4 = reinterpret_cast<const float4 *>(q + (uint64_t)g * group * hd)[tid];
        // (the wave holding the new row computes k_new's absmax: uniform)
        const bool new_wave = pnew >= t0 && pnew < t0 + tp && ((pnew - t0) << segs_log2) / 64 == wid;
        kv_absmax_part kpart{0.0f, 0.0f};
        if (new_wave) kpart = kv_absmax_first(kv_absmax, kv_absmax_n);
        if (t0 == p0 && dev_count_differs()) {  // uniform: the whole workgroup starts again
            settled = false;
            break;
        }
        // (the slots are combined only now, so that their wait is not ahead
        // of the device word's load)
        asm volatile("" : "+v"(kpart.m0), "+v"(kpart.m1));
        if (q_mine) reinterpret_cast<float4 *>(qs)[tid] = qv4;
        const float kabs = new_wave ? kv_absmax_finish(kpart, kv_absmax, kv_absmax_n) : 0.0f;
        // this thread's 16 values of k_p (read_into: q as f32 * scale; the
        // new row through KVCache::append's codes), into the tile's rows (q
        // and the rows are read after the barrier below; the rows of the
        // tile before were last read before the barrier that ends it)
        if (mine) {
            float kd[16];
            if (is_new) {
                const float ksn = kv_scale(kabs);
                const float kv[16] = {kn[0].x, kn[0].y, kn[0].z, kn[0].w, kn[1].x, kn[1].y, kn[1].z, kn[1].w,
                                      kn[2].x, kn[2].y, kn[2].z, kn[2].w, kn[3].x, kn[3].y, kn[3].z, kn[3].w};
                uint32_t cw[4] = {0u, 0u, 0u, 0u};
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    const int8_t c = kv_q(kv[e], kabs);
                    cw[e / 4] |= (uint32_t)(uint8_t)c << (8 * (e % 4));
                    kd[e] = (float)c * ksn;
                }
                // its workgroup writes the cache row segment, kv head 0's the scale
                *reinterpret_cast<int4 *>(const_cast<int8_t *>(k_cache) + (uint64_t)pnew * kv_dim + g * hd +
                                          sg * 16) = make_int4((int)cw[0], (int)cw[1], (int)cw[2], (int)cw[3]);
                if (g == 0 && sg == 0) const_cast<float *>(k_scales)[pnew] = ksn;
            } else {
#pragma unroll
                for (int e = 0; e < 16; e++) kd[e] = (float)(int8_t)(kw[e / 4] >> (8 * (e % 4))) * ksc;
            }
            float *dst = kdl + row * pst + sg * 16;
#pragma unroll
            for (int e = 0; e < 16; e += 4)
                *reinterpret_cast<float4 *>(dst + e) = make_float4(kd[e], kd[e + 1], kd[e + 2], kd[e + 3]);
        }
        wm_sync_lds();
        // (the struct's fields the stores use are in by now; taking them
        // here leaves no scalar load outstanding in the chains' loop, whose
        // waits can then count its LDS reads)
        const uint32_t sc_stride = a.score_stride, sc_tag = a.tag;
        const float sc_scale = a.scale;
        asm volatile("" ::"s"(sc_stride), "s"(sc_tag), "s"(sc_scale));
        // one chain per (head, position): s = Σ_i q_h[i] * k_p[i] in order.
        // Wave w takes head w % group and positions 64 (w / group) + lane:
        // the chains spread over the SIMDs, and a wave's q reads are one
        // address (group * ceil(sc_tile / 64) <= 16 waves).
        const uint32_t hh = wid % group, pl = (wid / group) * 64 + lane;
        if (pl < tp) {
            const float *kr = kdl + pl * pst, *qr = qs + hh * hd;
            // 16 terms per step (four float4 of k_p, four of q_h), the next
            // step's reads issued before this step's products and adds, into
            // two buffers in turn (hd is 64 or 128: 4 or 8 steps)
            float s = 0.0f;
            float4 ka[4], qa[4], kb[4], qb[4];
            const auto add16 = [&](const float4 (&k)[4], const float4 (&qq)[4]) {
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    s = s + qq[c].x * k[c].x;
                    s = s + qq[c].y * k[c].y;
                    s = s + qq[c].z * k[c].z;
                    s = s + qq[c].w * k[c].w;
                }
            };
            const auto read16 = [&](float4 (&k)[4], float4 (&qq)[4], uint32_t i) {
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    k[c] = *reinterpret_cast<const float4 *>(kr + i + 4 * c);
                    qq[c] = *reinterpret_cast<const float4 *>(qr + i + 4 * c);
                }
                __builtin_amdgcn_sched_barrier(0);  // the reads stay ahead of the adds that follow
            };
            // (a read past the row's end rereads its last 16 values, unused:
            // every read is unconditional, so each wait is for one buffer)
            read16(ka, qa, 0);
#pragma unroll 1
            for (uint32_t i = 16;; i += 32) {
                read16(kb, qb, min(i, hd - 16));
                add16(ka, qa);
                if (i >= hd) break;
                read16(ka, qa, min(i + 16, hd - 16));
                add16(kb, qb);
                if (i + 16 >= hd) break;
            }
            st_tagged(scores64 + (uint64_t)(g * group + hh) * sc_stride + t0 + pl, sc_tag, s * sc_scale);
        }
        if (t0 + sc_tile < p1) wm_sync_lds();
    }
    if (p0 >= p1 && dev_count_differs()) settled = false;  // no positions here: nothing was loaded
    if (!settled) {
        const uint32_t nd = *pos_dev + 1;
        if (nd == 0 || nd > nb) return;  // a count the launch is not sized for
        n = nd;
        pnew = nd - 1;
    }
    }

    // ---- phase 2: this head's scores, once each carries the launch's tag ----
    // The polls go out first, then the V slice and scales for phase 3
    // (thread t takes positions t + i * kSvThreads, indices clamped so every
    // load is unconditional) and this token's V.  A poll that never sees its tag gives up after
    // spin_limit rounds and raises the error flag (the step then fails and
    // is rolled back); spin_limit 0 (a test hook) gives up at once.
    const uint32_t tag = a.tag;
    const uint64_t *sc64 = scores64 + (uint64_t)h * a.score_stride;
    uint64_t sw[MAXM];
#pragma unroll
    for (int i = 0; i < MAXM; i++) sw[i] = ld_tagged(sc64 + min(tid + (uint32_t)i * kSvThreads, n - 1));
    const int8_t *vseg = a.v_cache + g * hd + d0;
    uint32_t vr0[MAXM], vr1[MAXM], vr2[MAXM], vr3[MAXM];
    float ss[MAXM];
#pragma unroll
    for (int i = 0; i < MAXM; i++) {
        const uint32_t p = min(tid + (uint32_t)i * kSvThreads, n - 1);
        const int4 t4 = *reinterpret_cast<const int4 *>(vseg + (uint64_t)p * kv_dim);
        vr0[i] = t4.x; vr1[i] = t4.y; vr2[i] = t4.z; vr3[i] = t4.w;
        ss[i] = a.v_scales[p];
    }
    // and this token's V: the workgroup's 16 values of v_new, and its absmax
    // (every wave reduces the slots itself)
    const float vnew = tid < kSvDims ? a.v_new[g * hd + d0 + tid] : 0.0f;
    // expf's table, into LDS at phase 3 (loaded here, after phase 1's loads,
    // so that no wait for it comes ahead of them)
    const uint64_t exp_word = tid < 32 ? wm::kExp2Tab[tid] : 0u;
    const float vabs = kv_absmax_of(kv_absmax + a.kv_absmax_stride, kv_absmax_n);
    {
        uint32_t pending = 0;
#pragma unroll
        for (int i = 0; i < MAXM; i++) pending |= ((uint32_t)(sw[i] >> 32) != tag ? 1u : 0u) << i;
        bool gave_up = a.spin_limit == 0;
        for (uint32_t it = 0; pending && !gave_up; it++) {
            if (it >= a.spin_limit) {
                gave_up = true;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
#pragma unroll
            for (int i = 0; i < MAXM; i++)
                if ((pending >> i) & 1u) {
                    sw[i] = ld_tagged(sc64 + min(tid + (uint32_t)i * kSvThreads, n - 1));
                    if ((uint32_t)(sw[i] >> 32) == tag) pending &= ~(1u << i);
                }
        }
        if (gave_up && a.err_flag) atomicCAS(a.err_flag, 0u, a.err_tag);
    }

    // ---- phase 3: softmax over scores[h][0..n) and the V chains ----
    const uint32_t npad = (n + 3) & ~3u;
    float *cval = sm;                                     // [seq_sum_padded(n)] nonzero exps, then weights
    float *vsc = cval + wm::seq_sum_padded(n);            // [npad]
    int4 *vq = reinterpret_cast<int4 *>(vsc + npad);      // [npad] x 16 int8
    float *prod = reinterpret_cast<float *>(vq + npad);   // [2][kSvDims][kSvStride]
    uint16_t *cidx = reinterpret_cast<uint16_t *>(prod + 2 * kSvDims * kSvStride);  // [npad]
    const bool v_writer = j == 0;
    float sv[MAXM];
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < MAXM; i++) sv[i] = __uint_as_float((uint32_t)sw[i]);
    if (tid < 32) exp_tab[tid] = exp_word;
#pragma unroll
    for (int i = 0; i < MAXM; i++)
        if (tid + (uint32_t)i * kSvThreads < n) m = wm_max_nonan(m, sv[i]);
    // softmax (attention.rs:45-73)
    // (the thread maxima are never NaN: a NaN score never wins above; a zero
    // maximum's sign, which the reduction order could change, does not reach
    // exp(s - max))
    const float mx = sv_block_max(m, red);
    float *out = a.out + (uint64_t)h * hd + d0;
    if (!isfinite(mx)) {  // every weight becomes 0 -> output stays 0
        if (tid < kSvDims) out[tid] = 0.0f;
    } else {
        // The V slice and scales into LDS.  These arrays overlap phase 1's K
        // rows: the barrier in sv_block_max is the first after which no
        // chain of this workgroup still reads them (a thread's own scores
        // can all come from other workgroups before its chains end).
#pragma unroll
        for (int i = 0; i < MAXM; i++) {
            const uint32_t p = tid + (uint32_t)i * kSvThreads;
            // the cache row of position n - 1 is stale (this token's V is
            // quantised below): only the rows before it are copied
            if (p < pnew) {
                vq[p] = make_int4(vr0[i], vr1[i], vr2[i], vr3[i]);
                vsc[p] = ss[i];
            }
        }
        // this token's V (position n - 1 is not in the cache yet)
        if (tid < kSvDims)
            reinterpret_cast<int8_t *>(vq + pnew)[tid] = kv_q(vnew, vabs);
        if (tid == 0) vsc[pnew] = kv_scale(vabs);
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
            // expf_glibc returns +0 below -0x1.9fe368p6 (its first branch), so
            // only the lanes at or above it (or NaN) evaluate it, and a wave
            // with none of them skips it (most exps underflow here)
            const float x = sv[i] - mx;
            const bool ev = p < n && !(x < -0x1.9fe368p6f);
            e[i] = 0.0f;
            if (__builtin_amdgcn_ballot_w64(ev))  // (uniform)
                if (ev) e[i] = wm::expf_glibc(x, exp_tab);
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
        // Σ exp left to right (attention.rs:63-66) over the compacted terms.
        if (count <= kSvSerialSum) {
            // Few terms (the usual case: most exps underflow to 0): wave 0
            // alone finishes, lane k holding term k.  The sum one add at a
            // time, w_k = e_k * (1 / sum), then per dimension d (lane d % 16)
            // Σ_k w_k * v_k[d] in order.
            if (wid == 0) {
                const float ev = lane < count ? cval[lane] : 0.0f;
                const uint32_t pv = lane < count ? (uint32_t)cidx[lane] : 0u;
                float s;
                asm volatile("v_mov_b32 %0, 0" : "=v"(s));
                for (uint32_t k = 0; k < count; k++)
                    s = s + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ev), (int)k));
                const float w = s > 0.0f ? ev * (1.0f / s) : ev;
                float acc;
                asm volatile("v_mov_b32 %0, 0" : "=v"(acc));
                for (uint32_t k = 0; k < count; k++) {
                    const float wk = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), (int)k));
                    const uint32_t pk = (uint32_t)__builtin_amdgcn_readlane((int)pv, (int)k);
                    const float vd = (float)reinterpret_cast<const int8_t *>(vq + pk)[lane & 15] * vsc[pk];  // read_into
                    acc = acc + wk * vd;
                }
                if (lane < kSvDims) out[lane] = acc;
            }
        } else {
        // A longer list: the workgroup's exact sum (thread t takes terms
        // t*m .. t*m+m-1), the normalisation, then the products by tiles.
        float sum;
        {
            float ev[MAXM];
            const uint32_t mm = (count + kSvThreads - 1) / kSvThreads, k0 = tid * mm;
#pragma unroll
            for (int jj = 0; jj < MAXM; jj++)
                ev[jj] = ((uint32_t)jj < mm && k0 + (uint32_t)jj < count) ? cval[k0 + jj] : 0.0f;
            sum = wm::seq_sum_block_owned<MAXM, kSvThreads>(ev, count, cval, &seq_scratch);
        }
        if (sum > 0.0f) {
            const float inv = 1.0f / sum;
            for (uint32_t k = tid; k < count; k += kSvThreads) cval[k] = cval[k] * inv;
        }
        wm_sync_lds();
        // products of tile t (waves 1-15) while wave 0 adds tile t - 1,
        // over the compacted positions in order
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
                            const float4 gg = f[c4 & 1][i];
                            acc = acc + gg.x; acc = acc + gg.y; acc = acc + gg.z; acc = acc + gg.w;
                        }
                    }
                } else {
                    uint32_t q = 0;
                    for (; q + 4 <= tn; q += 4) {
                        const float4 gg = *reinterpret_cast<const float4 *>(src + q);
                        acc = acc + gg.x; acc = acc + gg.y; acc = acc + gg.z; acc = acc + gg.w;
                    }
                    for (; q < tn; q++) acc = acc + src[q];
                }
            }
            wm_sync_lds();
        }
        if (wid == 0) __builtin_amdgcn_s_setprio(0);
        if (tid < kSvDims) out[tid] = acc;
        }
    }
    if (v_writer) {  // kv head g's segment of the cache row of position n - 1
        int8_t *v_row = const_cast<int8_t *>(a.v_cache) + (uint64_t)pnew * kv_dim + g * hd;
        for (uint32_t i = tid; i < hd; i += kSvThreads) v_row[i] = kv_q(a.v_new[g * hd + i], vabs);
        if (g == 0 && tid == 0) const_cast<float *>(a.v_scales)[pnew] = kv_scale(vabs);
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

// Returns false (nothing launched) for a shape the kernel does not cover:
// head_dim 64 or 128, n_past in [1, 4096], n_heads a multiple of n_kv_heads
// (at most 16 query heads per kv head).
// `scores`: n_heads * score_stride 64-bit words (tagged scores), zero when
// the model was created; `tag`: this launch's, 1 .. 2^32 - 1, a different
// one for every launch on the buffer (a counter of launches).
bool wm_launch_attention(const float *q, const int8_t *k_cache, const float *k_scales,
                         const int8_t *v_cache, const float *v_scales, float *scores,
                         uint32_t score_stride, float *out, uint32_t n_heads, uint32_t n_kv_heads,
                         uint32_t head_dim, uint32_t n_past, float scale, const float *k_new,
                         const float *v_new, const uint32_t *kv_absmax, uint32_t kv_absmax_n,
                         uint32_t kv_absmax_stride, uint32_t tag, uint32_t *err_flag,
                         uint32_t err_tag, bool no_wait, hipStream_t s, const uint32_t *pos_dev,
                         uint32_t n_max) {
    // with pos_dev, n_past comes from the device and n_max bounds it; the
    // score loads go out for n_max before the device word arrives, so a
    // count other than n_max costs the kernel a second start of its scores
    const uint32_t nb = pos_dev ? n_max : n_past;
    if ((head_dim != 64 && head_dim != 128) || nb == 0 || nb > 4 * kSvThreads || nb > score_stride ||
        n_kv_heads == 0 || n_heads % n_kv_heads || n_heads / n_kv_heads > 16 || tag == 0)
        return false;
    const uint32_t group = n_heads / n_kv_heads;
    // each query head's head_dim / 16 workgroups on one XCD, the heads dealt
    // to the 8 XCDs in turn; every workgroup must be resident at once (one
    // per CU, 32 CUs per XCD), since they wait for each other's scores
    const uint32_t segs = head_dim / kSvDims, per_xcd = segs * ((n_heads + 7) / 8);
    if (per_xcd > 32) return false;
    // positions per score tile: each head's chains on waves of their own
    // (64 positions a wave, 16 waves), one K segment per thread, and the
    // tile's dequantised K rows within 128 KiB of LDS
    const uint32_t pst = head_dim + 4;
    const uint32_t sc_tile = min(min(64u * (16u / group), (uint32_t)kSvThreads / (head_dim / 16)),
                                 (uint32_t)((128u * 1024u / 4u - group * head_dim) / pst));
    if (n_kv_heads > 255 || kv_absmax_n > 0xFFFFu) return false;
    const uint32_t geom = group | n_kv_heads << 8 | kv_absmax_n << 16;
    const uint32_t shape = (head_dim == 128 ? 1u : 0u) | sc_tile << 1 | nb << 12;
    attn_args a{v_cache, v_scales, scores, out, score_stride, scale, v_new, kv_absmax_stride,
                tag, err_flag, err_tag, no_wait ? 0u : (1u << 16)};
    const size_t npad = ((size_t)nb + 3) & ~(size_t)3;
    const size_t lds_sv = (size_t)wm::seq_sum_padded(nb) * 4 + npad * (4 + 16) +
                          (size_t)2 * kSvDims * kSvStride * 4 + npad * 2;
    const size_t lds_sc = ((size_t)group * head_dim + (size_t)sc_tile * pst) * 4;
    const size_t lds = lds_sv > lds_sc ? lds_sv : lds_sc;
    const dim3 grid(8 * per_xcd);
    if (nb <= 2 * kSvThreads)
        hipLaunchKernelGGL(k_attn_decode<2>, grid, dim3(kSvThreads), lds, s, q, k_cache, k_scales, k_new,
                           kv_absmax, pos_dev, geom, shape, a);
    else  // nb <= 4096, the models' context limit
        hipLaunchKernelGGL(k_attn_decode<4>, grid, dim3(kSvThreads), lds, s, q, k_cache, k_scales, k_new,
                           kv_absmax, pos_dev, geom, shape, a);
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
