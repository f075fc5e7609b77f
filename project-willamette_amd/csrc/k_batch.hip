// Kernels of the ragged multi-sequence batch (continuous batching), gfx950.
//
// Reference semantics: multi_token_forward (src/model/multi_forward.rs:49-243)
// extended with a pre-filled int8 KV cache, i.e. for every sequence the
// tokens go through forward_with_cache_into one after another
// (src/model/generate.rs:151-160; src/model/cached_forward.rs:164-502).
// Every per-token quantity is computed with the same operations, in the same
// order, as the single-token decode kernels, so a batch is bit-identical to
// that sequence of single-token steps:
//   * the BitLinear dot products are exact integers, here from int8 MFMA
//     (v_mfma_i32_16x16x64_i8) over all tokens at once;
//   * RMSNorm, the int8 quantiser, RoPE, the KV quantiser and attention run
//     per token exactly as in the decode kernels (exact sequential sums).
#include <algorithm>

#include "wm_internal.h"
#include "wm_norm.h"
#include "wm_seqsum.h"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// I2_S x int8 GEMM on MFMA
// ---------------------------------------------------------------------------
//
// One workgroup = four 64-row groups x 64 tokens: wave w owns group
// 4 * blockIdx.x + w (of whichever tensor it falls in) and all 64 tokens,
// i.e. 4 row tiles x 4 token tiles = 16 MFMAs (v_mfma_i32_16x16x64_i8) per
// 64-column chunk.  MFMA operands, lane l = 16 * seg + r:
//   A (weights): row r of a 16-row tile, dword seg of the row's 16-byte
//                chunk = 16 codes, expanded to one byte each ({0,1,2} =
//                ternary + 1);
//   B (activations): token r of a 16-token tile, the 16 bytes of the same
//                columns (the GEMM activation layout stores them
//                contiguously);
//   D: lane l holds rows 4*seg .. 4*seg+3 of token r.
// Σ_k (t_k + 1)·a_k - Σ_k a_k = Σ_k t_k·a_k is exact in i32 for any k order.
// Activations and weights go through LDS in blocks of kGemmKB chunks, in a
// ring of ST blocks: ST - 1 blocks of direct global->LDS loads are in flight
// while the waves compute the oldest one.  Each activation byte is read
// from L2 once per NG groups, and each B fragment read from LDS feeds four
// MFMAs.  Launches with few workgroups use k_i2s_gemm_kw below instead.
struct gemm_args {
    wm_gemm_desc d[WM_GEMM_MAX_DESC];
    uint32_t group_end[WM_GEMM_MAX_DESC];
    int n_desc;
    uint32_t n_groups;  // over all tensors
    uint32_t n_chunks;
    const uint8_t *act;
    uint32_t m, m_pad;
    const wm_act_meta *meta;
    float *y;
    uint32_t ldy;
};

__device__ __forceinline__ v4i expand_codes(uint32_t w) {
    // byte g of w holds the codes of columns g (bits 7:6), 32+g, 64+g, 96+g
    // of its 32-column quarter block: one shift and mask per quarter.
    const uint32_t m = 0x03030303u;
    v4i a;
    a.x = (int)((w >> 6) & m);
    a.y = (int)((w >> 4) & m);
    a.z = (int)((w >> 2) & m);
    a.w = (int)(w & m);
    return a;
}

constexpr uint32_t kGemmKB = 4;  // chunks per LDS block
constexpr uint32_t kGemmActChunk = WM_GEMM_TILE_TOKENS * 64;  // bytes of a chunk's activation tile
// LDS of a workgroup over NG 64-row groups: a ring of ST blocks of kGemmKB
// chunks (activations, then the groups' weights), later the output tile
template <int NG>
constexpr uint32_t gemm_block_bytes() { return kGemmKB * (kGemmActChunk + NG * 1024u); }
template <int NG>
constexpr uint32_t gemm_out_stride() { return NG * 64u + 4u; }  // floats per token row of the output tile
template <int NG, int ST>
constexpr size_t gemm_lds_bytes() {
    return (size_t)ST * gemm_block_bytes<NG>() > (size_t)WM_GEMM_TILE_TOKENS * gemm_out_stride<NG>() * 4
               ? (size_t)ST * gemm_block_bytes<NG>()
               : (size_t)WM_GEMM_TILE_TOKENS * gemm_out_stride<NG>() * 4;
}

// s_waitcnt vmcnt(N), the other counters left alone (gfx9 encoding: vmcnt
// in bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8)
template <uint32_t N>
__device__ __forceinline__ void gemm_vm_wait() {
    static_assert(N < 64, "vmcnt is six bits");
    __builtin_amdgcn_s_waitcnt((int)((N & 15u) | ((N >> 4) << 14) | (7u << 4) | (15u << 8)));
}
// wait until at most `blocks` blocks of this wave's loads, PER loads each,
// are still in flight (loads complete in issue order)
template <uint32_t PER>
__device__ __forceinline__ void gemm_wait_blocks(uint32_t blocks) {
    if (blocks == 0) gemm_vm_wait<0>();
    else if (blocks == 1) gemm_vm_wait<PER>();
    else if (blocks == 2) gemm_vm_wait<2 * PER>();
    else if (blocks == 3) gemm_vm_wait<3 * PER>();
    else gemm_vm_wait<4 * PER>();
}
constexpr int kGemmMaxStages = 6;  // gemm_wait_blocks covers up to 4 blocks ahead of the one waited for

// 16-byte slot of (token t, segment g) in a chunk's activation tile in LDS:
// the segment is XOR-swizzled by bits 3:2 of the token, so that the 16 lanes
// reading segment g of tokens r..r+15 hit 16 different bank groups.
__device__ __forceinline__ uint32_t gemm_act_slot(uint32_t t, uint32_t g) {
    return t * 4 + (g ^ ((t >> 2) & 3u));
}

struct gemm_group {
    const uint8_t *w;
    uint32_t g, row0, out_dim;
    float scale;
    bool live;
};

__device__ __forceinline__ gemm_group gemm_group_of(const gemm_args &a, uint32_t gid) {
    // the tensor of global group gid, by selects (no dynamic index into the argument block)
    gemm_group r{a.d[0].w, gid, a.d[0].out_row0, a.d[0].out_dim, a.d[0].scale, gid < a.n_groups};
#pragma unroll
    for (int i = 1; i < WM_GEMM_MAX_DESC; i++) {
        const bool in = i < a.n_desc && gid >= a.group_end[i - 1];
        r.w = in ? a.d[i].w : r.w;
        r.g = in ? gid - a.group_end[i - 1] : r.g;
        r.row0 = in ? a.d[i].out_row0 : r.row0;
        r.out_dim = in ? a.d[i].out_dim : r.out_dim;
        r.scale = in ? a.d[i].scale : r.scale;
    }
    return r;
}

// NG 64-row groups per workgroup of four waves: wave w works on group
// w / (4 / NG) and on TPW = NG token tiles of 16 (NG = 4: one group and all
// 64 tokens per wave; NG = 1: the workgroup's one group, 16 tokens per wave).
// ST: blocks in the LDS ring.
template <int NG, int ST>
__global__ __launch_bounds__(256) void k_i2s_gemm(gemm_args a) {
    static_assert(ST >= 2 && ST <= kGemmMaxStages, "ring size");
    constexpr uint32_t WPG = 4 / NG, TPW = 4 / WPG;  // waves per group, token tiles per wave
    constexpr uint32_t kBlock = gemm_block_bytes<NG>(), kWChunk = NG * 1024u;
    constexpr uint32_t kOutStride = gemm_out_stride<NG>();
    extern __shared__ __align__(16) uint8_t gl[];  // [ST] blocks (activations, weights), then the output tile
    const uint32_t tid = threadIdx.x;
    const uint32_t wave = (uint32_t)__builtin_amdgcn_readfirstlane((int)(tid >> 6)), lane = tid & 63;
    const uint32_t r16 = lane & 15, seg = lane >> 4;
    const uint32_t q = wave / WPG, s0 = (wave % WPG) * TPW;  // this wave's group and first token tile
    const gemm_group G = gemm_group_of(a, blockIdx.x * NG + q);
    const uint32_t n0 = blockIdx.y * WM_GEMM_TILE_TOKENS;
    const uint32_t c0 = 0, c1 = a.n_chunks;  // the chunks [c0, c1)
    // Both operands reach LDS by direct global->LDS loads (global_load_lds:
    // lane l of a wave writes 16 bytes at the wave's LDS base + 16 l), a
    // block of kGemmKB chunks at a time.  Per chunk:
    //   activations: wave w fills slots 64 w .. 64 w + 63 of the 256-slot
    //     tile; slot p holds token p / 4, segment (p % 4) ^ bits 3:2 of the
    //     token (gemm_act_slot);
    //   weights: wave w < NG copies group w's 1024-byte chunk (row r's 16
    //     bytes to slot r); a group past the last is group 0's copy, its
    //     sums discarded.
    const gemm_group GW = gemm_group_of(a, blockIdx.x * NG + (wave < NG ? wave : 0));
    const uint8_t *wsrc = (GW.live ? GW.w + (uint64_t)GW.g * a.n_chunks * 1024 : a.d[0].w) + lane * 16;
    const uint32_t p_act = wave * 64 + lane, t_act = p_act >> 2;
    const uint32_t g_act = (p_act & 3u) ^ ((t_act >> 2) & 3u);
    const uint8_t *asrc = a.act + (uint64_t)(n0 + t_act) * 64 + g_act * 16;
    const uint64_t cstride = (uint64_t)a.m_pad * 64;
    const uint32_t nblocks = (c1 - c0 + kGemmKB - 1) / kGemmKB;
#define WM_GEMM_ISSUE(BLK, BUF)                                                                  \
    do {                                                                                         \
        uint8_t *blk_ = gl + (BUF) * kBlock;                                                     \
        _Pragma("unroll") for (uint32_t kb = 0; kb < kGemmKB; kb++) {                            \
            /* past the range: its last chunk again, never read */                               \
            const uint32_t c = min(c0 + (BLK) * kGemmKB + kb, c1 - 1);                           \
            __builtin_amdgcn_global_load_lds(asrc + c * cstride,                                 \
                                             blk_ + kb * kGemmActChunk + wave * 1024, 16, 0, 0); \
            if (wave < NG)                                                                       \
                __builtin_amdgcn_global_load_lds(wsrc + (uint64_t)c * 1024,                      \
                                                 blk_ + kGemmKB * kGemmActChunk + kb * kWChunk + \
                                                     wave * 1024, 16, 0, 0);                     \
        }                                                                                        \
    } while (0)
    v4i acc[4][TPW];
#pragma unroll
    for (int rt = 0; rt < 4; rt++)
#pragma unroll
        for (uint32_t s = 0; s < TPW; s++) acc[rt][s] = v4i{0, 0, 0, 0};
    // this lane's B slots (token tile s0 + s: token 16 (s0 + s) + r16,
    // segment seg) and A words (row tile rt: row 16 rt + r16, dword seg)
    uint32_t b_off[TPW];
#pragma unroll
    for (uint32_t s = 0; s < TPW; s++) b_off[s] = gemm_act_slot((s0 + s) * 16 + r16, seg) * 16;
    const uint32_t a_off = kGemmKB * kGemmActChunk + q * 1024 + r16 * 16 + seg * 4;
    // blocks 0 .. ST - 2 in flight before the loop; block b + ST - 1 goes out
    // once every wave has finished block b - 1, whose slot it takes
#pragma unroll
    for (uint32_t b = 0; b + 1 < (uint32_t)ST; b++)
        if (b < nblocks) WM_GEMM_ISSUE(b, b);
    uint32_t slot = 0;  // b % ST
    for (uint32_t b = 0; b < nblocks; b++) {
        // this wave's loads of block b: the blocks issued after it may stay in flight
        const uint32_t ahead = min((uint32_t)ST - 2, nblocks - 1 - b);
        if (wave < NG) gemm_wait_blocks<2 * kGemmKB>(ahead);
        else gemm_wait_blocks<kGemmKB>(ahead);
        // everyone's loads of block b, and block b - 1 fully read.  A bare
        // barrier: __syncthreads()' release fence would wait for every load
        // in flight (vmcnt(0)), the later blocks' included.
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        if (b + ST - 1 < nblocks) WM_GEMM_ISSUE(b + ST - 1, slot == 0 ? ST - 1 : slot - 1);
        const uint8_t *blk = gl + slot * kBlock;
        slot = slot + 1 == (uint32_t)ST ? 0u : slot + 1;
        const uint32_t kbn = min(kGemmKB, c1 - c0 - b * kGemmKB);
        // The block's fragments first, then its MFMAs.  A chunk past the
        // range (a copy of the last one) gets zero codes, which add nothing:
        // no branch around the MFMAs, so the sums stay in their registers.
        v4i bv[kGemmKB][TPW];
        uint32_t wv[kGemmKB][4];
#pragma unroll
        for (uint32_t kb = 0; kb < kGemmKB; kb++) {
#pragma unroll
            for (uint32_t s = 0; s < TPW; s++)
                bv[kb][s] = *reinterpret_cast<const v4i *>(blk + kb * kGemmActChunk + b_off[s]);
#pragma unroll
            for (int rt = 0; rt < 4; rt++) {
                const uint32_t w = *reinterpret_cast<const uint32_t *>(blk + a_off + kb * kWChunk + rt * 256);
                wv[kb][rt] = kb < kbn ? w : 0u;
            }
        }
#pragma unroll
        for (uint32_t kb = 0; kb < kGemmKB; kb++) {
#pragma unroll
            for (int rt = 0; rt < 4; rt++) {
                const v4i av = expand_codes(wv[kb][rt]);
#pragma unroll
                for (uint32_t s = 0; s < TPW; s++)
                    acc[rt][s] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bv[kb][s], acc[rt][s], 0, 0, 0);
            }
        }
    }
#undef WM_GEMM_ISSUE
    __syncthreads();  // every wave is done with the ring before the output tile reuses it
    // epilogue: y = (w_scale * act_scale) * (dot as f32)   (bitlinear_sse2.rs:327-339),
    // through LDS so that every token's outputs of a group leave as 256
    // contiguous bytes (the MFMA layout gives each lane 4 rows of one token)
    float *ot = reinterpret_cast<float *>(gl);  // [64 tokens][kOutStride]
#pragma unroll
    for (uint32_t s = 0; s < TPW; s++) {
        const uint32_t tl = (s0 + s) * 16 + r16;
        const wm_act_meta mt = a.meta[min(n0 + tl, a.m - 1)];
        const float comb = G.scale * mt.scale;
#pragma unroll
        for (int rt = 0; rt < 4; rt++) {
            float4 o;
            o.x = comb * (float)(acc[rt][s].x - mt.asum);
            o.y = comb * (float)(acc[rt][s].y - mt.asum);
            o.z = comb * (float)(acc[rt][s].z - mt.asum);
            o.w = comb * (float)(acc[rt][s].w - mt.asum);
            *reinterpret_cast<float4 *>(ot + tl * kOutStride + q * 64 + rt * 16 + seg * 4) = o;
        }
    }
    __syncthreads();
    // the 64 x 64 outputs of group g: 1024 float4, four per thread
#pragma unroll
    for (uint32_t g = 0; g < (uint32_t)NG; g++) {
        const gemm_group Q = gemm_group_of(a, blockIdx.x * NG + g);
        if (!Q.live) break;
        const uint32_t base = Q.g * 64;
        const bool vec = ((Q.row0 | a.ldy) & 3u) == 0;
#pragma unroll
        for (uint32_t k = 0; k < 4; k++) {
            const uint32_t idx = tid + k * 256, tl = idx >> 4, c4 = (idx & 15) * 4;
            const uint32_t t = n0 + tl;
            if (t >= a.m) continue;
            const float4 o = *reinterpret_cast<const float4 *>(ot + tl * kOutStride + g * 64 + c4);
            float *dst = a.y + (uint64_t)t * a.ldy + Q.row0 + base + c4;
            if (vec && base + c4 + 4 <= Q.out_dim) {
                *reinterpret_cast<float4 *>(dst) = o;
            } else {
                const float ov[4] = {o.x, o.y, o.z, o.w};
#pragma unroll
                for (int r = 0; r < 4; r++)
                    if (base + c4 + r < Q.out_dim) dst[r] = ov[r];
            }
        }
    }
}

// The same GEMM with the K dimension split over the four waves instead of
// the tokens: every wave computes the workgroup's whole NG*64-row x 64-token
// tile over chunks w, w + 4, w + 8, ..., so each code word is expanded once
// per workgroup and feeds 4 MFMAs.  A wave's operands are its own: each
// wave keeps a private ring of ST chunk slots in LDS, filled by direct
// global->LDS loads, and needs no barrier in the K loop.  While the MFMAs of
// chunk j run, chunk j + 1's fragments are read from LDS and chunk j + ST
// is in flight.  The four partial tiles are added through LDS at the end
// (exact: integers).
template <int NG>
constexpr uint32_t gemm_kw_slot_bytes() { return 4096u + NG * 1024u; }  // B tile, then NG groups' codes
template <int NG, int ST>
constexpr size_t gemm_kw_lds_bytes() {
    constexpr size_t ring = (size_t)4 * ST * gemm_kw_slot_bytes<NG>();
    constexpr size_t red = (size_t)4 * 16 * 64 * 16;  // one group's four partial tiles
    constexpr size_t out = (size_t)WM_GEMM_TILE_TOKENS * gemm_out_stride<NG>() * 4;
    return ring > red ? (ring > out ? ring : out) : (red > out ? red : out);
}
template <int NG, int ST>
__global__ __launch_bounds__(256) void k_i2s_gemm_kw(gemm_args a) {
    static_assert(ST >= 2 && ST <= kGemmMaxStages, "ring size");
    constexpr uint32_t kOutStride = gemm_out_stride<NG>();
    constexpr uint32_t kSlot = gemm_kw_slot_bytes<NG>();
    constexpr uint32_t kLoads = 4 + NG;  // global->LDS loads per chunk and wave
    extern __shared__ __align__(16) uint8_t gl[];
    const uint32_t tid = threadIdx.x;
    const uint32_t wave = (uint32_t)__builtin_amdgcn_readfirstlane((int)(tid >> 6)), lane = tid & 63;
    const uint32_t r16 = lane & 15, seg = lane >> 4;
    const uint32_t n0 = blockIdx.y * WM_GEMM_TILE_TOKENS;
    const uint32_t nc = a.n_chunks;
    uint8_t *ring = gl + wave * ST * kSlot;
    // Loads, lane l: B tile s: LDS slot l of 16 bytes holds token 16 s + l / 4,
    // segment (l % 4) ^ bits 3:2 of the token (gemm_act_slot, so that the
    // MFMA reads below hit distinct banks); A of group g: row l's 16 bytes.
    const uint32_t t_act = lane >> 2, g_act = (lane & 3u) ^ ((t_act >> 2) & 3u);
    const uint8_t *bsrc = a.act + (uint64_t)(n0 + t_act) * 64 + g_act * 16;
    const uint64_t cstride = (uint64_t)a.m_pad * 64;
    const uint8_t *wsrc[NG];
#pragma unroll
    for (int g = 0; g < NG; g++) {
        const gemm_group Gg = gemm_group_of(a, blockIdx.x * NG + g);
        // a group past the last reads group 0's codes; its sums are discarded
        wsrc[g] = (Gg.live ? Gg.w + (uint64_t)Gg.g * nc * 1024 : a.d[0].w) + lane * 16;
    }
    // this wave's chunk j is wave + 4 j; past the end: the last chunk again
    // (its codes are zeroed before use)
#define WM_KW_ISSUE(J, SLOT)                                                                      \
    do {                                                                                          \
        const uint32_t c_ = min(wave + 4u * (J), nc - 1);                                         \
        uint8_t *d_ = ring + (SLOT) * kSlot;                                                      \
        _Pragma("unroll") for (int s_ = 0; s_ < 4; s_++)                                          \
            __builtin_amdgcn_global_load_lds(bsrc + c_ * cstride + s_ * 1024, d_ + s_ * 1024, 16, 0, 0); \
        /* (the source through a local: an array element passed to the builtin                   \
           makes the host pass drop the kernel's launch stub) */                                  \
        _Pragma("unroll") for (int g_ = 0; g_ < NG; g_++) {                                       \
            const uint8_t *w_ = wsrc[g_] + (uint64_t)c_ * 1024;                                   \
            __builtin_amdgcn_global_load_lds(w_, d_ + 4096 + g_ * 1024, 16, 0, 0);                \
        }                                                                                         \
    } while (0)
    // this lane's fragments in a slot: B of token tile s (token 16 s + r16,
    // segment seg), A of group g, row tile rt (row 16 rt + r16, dword seg)
    const uint32_t b_off = gemm_act_slot(r16, seg) * 16;
    const uint32_t a_off = 4096u + r16 * 16 + seg * 4;
#define WM_KW_READ(SLOT, BV, AV)                                                                  \
    do {                                                                                          \
        const uint8_t *q_ = ring + (SLOT) * kSlot;                                                \
        _Pragma("unroll") for (int s_ = 0; s_ < 4; s_++)                                          \
            BV[s_] = *reinterpret_cast<const v4i *>(q_ + s_ * 1024 + b_off);                      \
        _Pragma("unroll") for (int g_ = 0; g_ < NG; g_++)                                         \
            _Pragma("unroll") for (int rt_ = 0; rt_ < 4; rt_++)                                   \
                AV[g_][rt_] = *reinterpret_cast<const uint32_t *>(q_ + a_off + g_ * 1024 + rt_ * 256); \
    } while (0)
    v4i acc[NG][4][4];
#pragma unroll
    for (int g = 0; g < NG; g++)
#pragma unroll
        for (int rt = 0; rt < 4; rt++)
#pragma unroll
            for (int s = 0; s < 4; s++) acc[g][rt][s] = v4i{0, 0, 0, 0};
    const uint32_t J = (nc + 3) / 4;  // steps (the waves with fewer chunks zero their last codes)
    // chunks 0 .. ST - 1 in flight, chunk 0 read
#pragma unroll
    for (int u = 0; u < ST; u++)
        if ((uint32_t)u < J) WM_KW_ISSUE((uint32_t)u, (uint32_t)u);
    if (J > 1) gemm_wait_blocks<kLoads>(min((uint32_t)ST - 1, J - 1));
    else gemm_vm_wait<0>();
    // two register sets, used alternately (no copies between steps)
    v4i b0[4], b1[4];
    uint32_t a0[NG][4], a1[NG][4];
    WM_KW_READ(0u, b0, a0);
    uint32_t slot = 0;  // j % ST
#define WM_KW_STEP(JJ, BC, AC, BN, AN)                                                            \
    do {                                                                                          \
        const uint32_t j_ = (JJ);                                                                 \
        const uint32_t nslot_ = slot + 1 == (uint32_t)ST ? 0u : slot + 1;                         \
        /* chunk j + 1 has landed when at most the chunks issued after it are in                 \
           flight: j + 2 .. min(j + ST - 1, J - 1).  Past the last chunk the read                \
           is of a stale slot, never used. */                                                     \
        gemm_wait_blocks<kLoads>(j_ + 1 < J ? min((uint32_t)ST - 2, J - 2 - j_) : 0u);            \
        asm volatile("" ::: "memory");                                                            \
        WM_KW_READ(nslot_, BN, AN);                                                               \
        __builtin_amdgcn_sched_barrier(0); /* the reads go out before this chunk's MFMAs */       \
        const bool live_ = wave + 4u * j_ < nc;                                                   \
        _Pragma("unroll") for (int g = 0; g < NG; g++)                                            \
            _Pragma("unroll") for (int rt = 0; rt < 4; rt++) {                                    \
                const v4i av = expand_codes(live_ ? AC[g][rt] : 0u);                              \
                _Pragma("unroll") for (int s = 0; s < 4; s++)                                     \
                    acc[g][rt][s] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, BC[s], acc[g][rt][s], 0, 0, 0); \
            }                                                                                     \
        /* slot j is free once its fragments are in registers (the MFMAs above                   \
           have them); chunk j + ST takes it.  The wait is for chunk j + 1's reads               \
           too, which had this chunk's MFMAs to land. */                                          \
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");                                        \
        if (j_ + ST < J) WM_KW_ISSUE(j_ + ST, slot);                                              \
        slot = nslot_;                                                                            \
    } while (0)
    // an even number of steps: a step past J has zero codes and adds nothing
    // (no branch around the MFMAs, so the sums stay in place)
    for (uint32_t j = 0; j < J; j += 2) {
        WM_KW_STEP(j, b0, a0, b1, a1);
        WM_KW_STEP(j + 1, b1, a1, b0, a0);
    }
#undef WM_KW_STEP
#undef WM_KW_ISSUE
#undef WM_KW_READ
    __syncthreads();  // every wave is done with its ring
    // the four waves' tiles through LDS, one group at a time; wave w then
    // owns row tile w
    v4i *red = reinterpret_cast<v4i *>(gl);  // [4 waves][4 rt][4 s][64 lanes]
    v4i sum[NG][4];
#pragma unroll
    for (int g = 0; g < NG; g++) {
        if (g > 0) __syncthreads();  // the previous group's sums are read
#pragma unroll
        for (int rt = 0; rt < 4; rt++)
#pragma unroll
            for (int s = 0; s < 4; s++) red[((wave * 4 + rt) * 4 + s) * 64 + lane] = acc[g][rt][s];
        __syncthreads();
#pragma unroll
        for (int s = 0; s < 4; s++) {
            v4i t = red[((0 * 4 + wave) * 4 + s) * 64 + lane];
#pragma unroll
            for (uint32_t v = 1; v < 4; v++) t += red[((v * 4 + wave) * 4 + s) * 64 + lane];
            sum[g][s] = t;
        }
    }
    __syncthreads();  // the output tile reuses the reduction area
    // epilogue: y = (w_scale * act_scale) * (dot as f32)   (bitlinear_sse2.rs:327-339)
    float *ot = reinterpret_cast<float *>(gl);  // [64 tokens][kOutStride]
#pragma unroll
    for (int s = 0; s < 4; s++) {
        const uint32_t tl = (uint32_t)s * 16 + r16;
        const wm_act_meta mt = a.meta[min(n0 + tl, a.m - 1)];
#pragma unroll
        for (int g = 0; g < NG; g++) {
            const float comb = gemm_group_of(a, blockIdx.x * NG + g).scale * mt.scale;
            float4 o;
            o.x = comb * (float)(sum[g][s].x - mt.asum);
            o.y = comb * (float)(sum[g][s].y - mt.asum);
            o.z = comb * (float)(sum[g][s].z - mt.asum);
            o.w = comb * (float)(sum[g][s].w - mt.asum);
            *reinterpret_cast<float4 *>(ot + tl * kOutStride + g * 64 + wave * 16 + seg * 4) = o;
        }
    }
    __syncthreads();
    // the 64 x 64 outputs of group g: 1024 float4, four per thread
#pragma unroll
    for (uint32_t g = 0; g < (uint32_t)NG; g++) {
        const gemm_group Q = gemm_group_of(a, blockIdx.x * NG + g);
        if (!Q.live) break;
        const uint32_t base = Q.g * 64;
        const bool vec = ((Q.row0 | a.ldy) & 3u) == 0;
#pragma unroll
        for (uint32_t k = 0; k < 4; k++) {
            const uint32_t idx = tid + k * 256, tl = idx >> 4, c4 = (idx & 15) * 4;
            const uint32_t t = n0 + tl;
            if (t >= a.m) continue;
            const float4 o = *reinterpret_cast<const float4 *>(ot + tl * kOutStride + g * 64 + c4);
            float *dst = a.y + (uint64_t)t * a.ldy + Q.row0 + base + c4;
            if (vec && base + c4 + 4 <= Q.out_dim) {
                *reinterpret_cast<float4 *>(dst) = o;
            } else {
                const float ov[4] = {o.x, o.y, o.z, o.w};
#pragma unroll
                for (int r = 0; r < 4; r++)
                    if (base + c4 + r < Q.out_dim) dst[r] = ov[r];
            }
        }
    }
}

// ---------------------------------------------------------------------------
// per-row absmax int8 (bitlinear_sse2.rs:285-304) into the GEMM layout
// ---------------------------------------------------------------------------
// 512 threads per row: two rows per CU (at up to 128 VGPRs a thread), so
// that a batch of up to 512 rows runs in one round over the 256 CUs
constexpr int kRowThreads = 512;

__global__ __launch_bounds__(kRowThreads) void k_quantize_rows(const float *__restrict__ x,
                                                               uint32_t ldx, uint32_t n,
                                                               uint32_t m_pad,
                                                               uint8_t *__restrict__ act,
                                                               wm_act_meta *__restrict__ meta) {
    __shared__ float red_f[16];
    __shared__ int red_i[16];
    const uint32_t t = blockIdx.x;
    const float *xr = x + (uint64_t)t * ldx;
    float m = 0.0f;
    for (uint32_t j = threadIdx.x; j < n; j += kRowThreads) m = wm_max_nonan(m, fabsf(xr[j]));
    const float max_abs = wm_block_max_nonan(m, red_f);
    const float inv = 127.0f / max_abs;
    int sum = 0;
    for (uint32_t j = threadIdx.x; j < n; j += kRowThreads) {
        const int q = max_abs == 0.0f ? 0 : wm_round_clamp_i8(xr[j] * inv);
        act[wm_gemm_act_offset(j, t, m_pad)] = (uint8_t)(int8_t)q;
        sum += q;
    }
    sum = wm_block_sum_i32(sum, red_i);
    if (threadIdx.x == 0) {
        meta[t].scale = max_abs == 0.0f ? 1.0f : max_abs / 127.0f;
        meta[t].asum = sum;
    }
}

// ---------------------------------------------------------------------------
// RMSNorm per row (primitives.rs:227-255), one workgroup per token
// ---------------------------------------------------------------------------
// The decode norms' building blocks (wm_norm.h): the exact Σx² by the
// workgroup (seq_sum_block_owned), then y = x * rsqrt * w and the absmax
// int8 quantiser, here into the GEMM activation layout.
template <int PER, bool GU>
__global__ __launch_bounds__(kRowThreads) void k_rmsnorm_rows(wm_norm_rows a) {
    extern __shared__ __align__(16) float sq[];  // x[j]^2, seq_sum_padded(n) entries
    __shared__ wm::norm_lds<kRowThreads / 64> nl;
    const uint32_t t = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wid = tid >> 6, n = a.n;
    float xv[PER], wv[PER], rv[PER];
    bool nonfinite = false;
    if (GU) {
        // relu_square(gate) * up (ffn.rs:37-65)
        const float *g = a.gu + (uint64_t)t * a.ldgu;
#pragma unroll
        for (int i = 0; i < PER; i++) {
            const uint32_t j = min(tid + (uint32_t)i * kRowThreads, n - 1);
            xv[i] = g[j];
            rv[i] = g[n + j];
            wv[i] = a.w[j];
        }
        wm::norm_prep<PER, kRowThreads>(true, n, nullptr, sq, xv, wv, rv, true);
    } else {
        float *xr = a.x + (uint64_t)t * a.ldx;
        wm::norm_load<PER, kRowThreads>(xr, a.res ? a.res + (uint64_t)t * a.ldr : nullptr, a.w, n,
                                        xv, wv, rv);
        // hidden += BitLinear output (cached_forward.rs:405-408, :496-500)
        nonfinite = wm::norm_prep<PER, kRowThreads>(a.res != nullptr, n, a.res ? xr : nullptr, sq,
                                                    xv, wv, rv);
    }
    const float rs = wm::norm_sum_rsqrt<PER, kRowThreads>(nonfinite, n, a.eps, a.err_flag, a.tag,
                                                          sq, nl);
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const uint32_t j = tid + (uint32_t)i * kRowThreads;
        xv[i] = xv[i] * rs * wv[i];
        if (j < n) {
            if (a.y_out) a.y_out[(uint64_t)t * a.ldo + j] = xv[i];
            m = wm_max_nonan(m, fabsf(xv[i]));
        }
    }
    if (!a.act) return;
    m = wm_wave_max_nonneg(m);
    if (lane == 0) nl.red_f[wid] = m;
    wm_sync_lds();
    float max_abs = nl.red_f[0];
#pragma unroll
    for (int i = 1; i < kRowThreads / 64; i++) max_abs = wm_max_nonan(max_abs, nl.red_f[i]);
    const float inv = 127.0f / max_abs;
    int sum = 0;
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const uint32_t j = tid + (uint32_t)i * kRowThreads;
        if (j < n) {
            const int q = max_abs == 0.0f ? 0 : wm_round_clamp_i8_fast(xv[i] * inv);
            a.act[wm_gemm_act_offset(j, t, a.m_pad)] = (uint8_t)(int8_t)q;
            sum += q;
        }
    }
    sum = wm_wave_total_i32(sum);
    if (lane == 0) nl.red_i[wid] = sum;
    wm_sync_lds();
    if (tid == 0) {
        int tot = 0;
#pragma unroll
        for (int i = 0; i < kRowThreads / 64; i++) tot += nl.red_i[i];
        a.meta[t].scale = max_abs == 0.0f ? 1.0f : max_abs / 127.0f;
        a.meta[t].asum = tot;
    }
}

// ---------------------------------------------------------------------------
// RoPE (NEOX) + K/V append per token (cached_forward.rs:340-404)
// ---------------------------------------------------------------------------
struct qkv_rows_args {
    const float *y;
    uint32_t ldy;
    const float *cos, *sin;
    const wm_batch_tok *tok;
    uint32_t layer, n_q, n_kv, head_dim, n_rot;
    float *q_out;
};

__global__ __launch_bounds__(256) void k_qkv_rows(qkv_rows_args a) {
    extern __shared__ float sm[];  // q | k | v of this token
    __shared__ float red[16];
    const uint32_t t = blockIdx.x;
    const wm_batch_tok tk = a.tok[t];
    const uint32_t total = a.n_q + 2 * a.n_kv;
    const float *src = a.y + (uint64_t)t * a.ldy;
    for (uint32_t i = threadIdx.x; i < total; i += blockDim.x) sm[i] = src[i];
    __syncthreads();
    float *qs = sm, *ks = sm + a.n_q, *vs = ks + a.n_kv;
    const uint32_t half = a.n_rot / 2;
    const float *cs = a.cos + (uint64_t)tk.pos * half, *sn = a.sin + (uint64_t)tk.pos * half;
    const uint32_t n_pairs_q = (a.n_q / a.head_dim) * half, n_pairs_k = (a.n_kv / a.head_dim) * half;
    for (uint32_t p = threadIdx.x; p < n_pairs_q + n_pairs_k; p += blockDim.x) {
        float *base = p < n_pairs_q ? qs : ks;
        const uint32_t pp = p < n_pairs_q ? p : p - n_pairs_q;
        const uint32_t h = pp / half, j = pp % half;
        float *xh = base + h * a.head_dim;
        const float c = cs[j], s = sn[j];
        const float x0 = xh[j], x1 = xh[j + half];
        xh[j] = x0 * c - x1 * s;
        xh[j + half] = x0 * s + x1 * c;
    }
    __syncthreads();
    float *qo = a.q_out + (uint64_t)t * a.n_q;
    for (uint32_t i = threadIdx.x; i < a.n_q; i += blockDim.x) qo[i] = qs[i];
    const uint64_t row = (uint64_t)a.layer * tk.max_seq + tk.pos;
    wm_kv_quantise_store(ks, a.n_kv, tk.k + row * a.n_kv, tk.ks + row, red);
    __syncthreads();
    wm_kv_quantise_store(vs, a.n_kv, tk.v + row * a.n_kv, tk.vs + row, red);
}

// ---------------------------------------------------------------------------
// causal GQA attention of every token over its own sequence
// (cached_forward.rs:417-449, attention.rs:45-73), in two kernels
// ---------------------------------------------------------------------------
//
// Scores: one thread per (position, KV head) computes the G query heads'
// 128-term dots from one K row, each in order with k = q8 * scale, then
// * (1/sqrt(head_dim)), into scores[t][h][p].
// Softmax + V: one workgroup per (token, head): max, exp (glibc expf), exact
// sequential sum, * (1/sum), then one thread per output dimension runs
// Σ_p w_p * v_p[d] in position order.
struct attn_rows_args {
    const float *q;  // [t][n_heads * head_dim]
    const wm_batch_tok *tok;
    float *scores;   // [t][n_heads][score_stride]: the scores, then exp(s - max)
    float *out;      // [t][n_heads * head_dim]
    uint32_t layer, kv_dim, n_heads, score_stride, n_max;
    float scale;
    float *row_scale;  // [t][n_heads]: 1 / Σexp (1 when Σ is not positive)
    uint8_t *live;     // [t][n_heads][kAttnTiles]: the tile of kSvPos positions holds a non-zero exp
    const wm_attn_item *sc_items, *sv_items;  // work items of the scores and V kernels
};

constexpr int kScoreThreads = 256;  // positions per scores item, one per thread
constexpr int kScoreTok = 8;        // tokens (of one sequence) per scores item

// scores[t][h][p] for the NT tokens t0 .. t0+NT-1 of one sequence (item
// it), the G query heads of the item's KV head and position p (this thread):
// the thread loads its K row once, dequantises it (read_into: q8 * scale) and
// runs the NT*G chains Σ_i q[i] * k[i], each in dimension order, then
// * (1/sqrt(head_dim)).  The query values are the same for every lane and
// are read as scalars.  Positions past a token's own are computed from rows
// other tokens of the batch have written and never read.
// Memory that no thread writes while the kernel runs, addressed so that the
// compiler may read it through the scalar unit wherever the address is the
// same for every lane.
typedef const float __attribute__((address_space(4))) wm_const_f32;

template <int HD, int G, int NT>
__device__ __forceinline__ void scores_item(const int8_t *kp, float kscale, const float *qb,
                                            uint64_t qstride, float *dst, uint64_t sstride,
                                            float scale) {
    float s[NT][G];
#pragma unroll
    for (int tt = 0; tt < NT; tt++)
#pragma unroll
        for (int g = 0; g < G; g++) s[tt][g] = 0.0f;
    // the next 16 codes are in flight while the current ones are used
    int4 raw = *reinterpret_cast<const int4 *>(kp);
#pragma unroll 1
    for (int b = 0; b < HD / 16; b++) {
        const int4 cur = raw;
        if (b + 1 < HD / 16) raw = *reinterpret_cast<const int4 *>(kp + (b + 1) * 16);
        float kd[16];
#pragma unroll
        for (int e = 0; e < 16; e++) {
            const uint32_t wd = e < 4 ? (uint32_t)cur.x : e < 8 ? (uint32_t)cur.y : e < 12 ? (uint32_t)cur.z : (uint32_t)cur.w;
            kd[e] = (float)(int8_t)(wd >> (8 * (e & 3))) * kscale;  // read_into
        }
#pragma unroll
        for (int tt = 0; tt < NT; tt++) {
            const wm_const_f32 *qt = (const wm_const_f32 *)qb + (uint64_t)tt * qstride + b * 16;
#pragma unroll
            for (int g = 0; g < G; g++)
#pragma unroll
                for (int e = 0; e < 16; e++) s[tt][g] = s[tt][g] + qt[g * HD + e] * kd[e];
        }
    }
    // token tt, head g: dst[(tt * G + g) * sstride] (the token's rows follow
    // its G heads' rows: n_heads rows per token, G of them this KV head's)
#pragma unroll
    for (int tt = 0; tt < NT; tt++)
#pragma unroll
        for (int g = 0; g < G; g++) dst[(uint64_t)tt * qstride / HD * sstride + (uint64_t)g * sstride] = s[tt][g] * scale;
}

// One item per workgroup (blockIdx.x): its nt (1 .. kScoreTok) tokens and
// positions p0 .. p0+255 below p1, one position per thread.
template <int HD, int G>
__global__ __launch_bounds__(kScoreThreads) void k_attn_scores_rows(attn_rows_args a) {
    static_assert(kScoreTok == 8, "one case per token count");
    const wm_attn_item it = a.sc_items[blockIdx.x];
    const uint32_t p = it.p0 + threadIdx.x;
    if (it.nt == 0 || p >= it.p1) return;
    const uint32_t kvh = it.unit;
    const wm_batch_tok tk = a.tok[it.t0];  // every token of the item: the same cache
    const uint64_t lay = (uint64_t)a.layer * tk.max_seq;
    const int8_t *kp = tk.k + (lay + p) * a.kv_dim + kvh * HD;
    const float kscale = tk.ks[lay + p];
    const float *qb = a.q + (uint64_t)it.t0 * a.n_heads * HD + (uint64_t)kvh * G * HD;
    const uint64_t qstride = (uint64_t)a.n_heads * HD;
    float *dst = a.scores + ((uint64_t)it.t0 * a.n_heads + kvh * G) * a.score_stride + p;
    const uint64_t ss = a.score_stride;
    switch (it.nt) {
        case 1: scores_item<HD, G, 1>(kp, kscale, qb, qstride, dst, ss, a.scale); break;
        case 2: scores_item<HD, G, 2>(kp, kscale, qb, qstride, dst, ss, a.scale); break;
        case 3: scores_item<HD, G, 3>(kp, kscale, qb, qstride, dst, ss, a.scale); break;
        case 4: scores_item<HD, G, 4>(kp, kscale, qb, qstride, dst, ss, a.scale); break;
        case 5: scores_item<HD, G, 5>(kp, kscale, qb, qstride, dst, ss, a.scale); break;
        case 6: scores_item<HD, G, 6>(kp, kscale, qb, qstride, dst, ss, a.scale); break;
        case 7: scores_item<HD, G, 7>(kp, kscale, qb, qstride, dst, ss, a.scale); break;
        default: scores_item<HD, G, 8>(kp, kscale, qb, qstride, dst, ss, a.scale); break;
    }
}

// out[t][h][d] = Σ_p w_h[p] * v_p[d] in position order (cached_forward.rs:
// 417-449; v_p[d] = q8 * scale, read_into) for kSvTok tokens of one sequence
// (item blockIdx.x) and G query heads of one KV head, on the exps
// k_attn_softmax_rows left in place of the scores times each row's 1/sum.
// Thread d runs the kSvTok * G chains: they share every V value.  Tiles of
// kSvPos positions go through LDS: the V codes and scales (the next tile's
// loads in flight while the current one is summed) and the rows' weights; a
// token's positions past its own get weight 0 (exact: a zero term leaves
// the sum unchanged), so every tile runs in full.
// The pass ends when its longest rows do (heads whose exps are non-zero
// over the whole context, while most rows have one live tile), and what
// such a row waits on is its waves' own work per tile; so each workgroup
// takes one query head, although the heads of a KV group could share the
// V dequantisation (BitNet-2B, 16 sequences: 133 us per layer with four
// heads per workgroup, 99 with two, 90 with one).
constexpr uint32_t kSvPos = 64;
constexpr uint32_t kSvHeads = 1;  // query heads per workgroup (of one KV head's group)
constexpr uint32_t kSvTok = 1;    // tokens per V item
constexpr uint32_t kAttnTiles = 64;  // tiles of kSvPos positions per row (contexts <= 4096)

// The loads of V tile rows p0 .. p0 + kSvPos - 1 (indices clamped to n - 1):
// thread tid takes 16-byte pieces tid, tid + HD, tid + 2HD, tid + 3HD
// (piece = row * HD/16 + column) and their rows' scales, in named registers
// (an array would be kept in scratch memory).
struct sv_regs {
    int4 v0, v1, v2, v3;
    float s0, s1, s2, s3;
};
template <int HD>
__device__ __forceinline__ uint32_t sv_row(uint32_t i) { return (i * HD + threadIdx.x) / (HD / 16); }
template <int HD>
__device__ __forceinline__ uint32_t sv_col(uint32_t i) { return ((i * HD + threadIdx.x) % (HD / 16)) * 16; }
template <int HD>
__device__ __forceinline__ void sv_fetch(sv_regs &r, const int8_t *vg, const float *vsg, uint32_t kv_dim,
                                         uint32_t p0, uint32_t n) {
    static_assert(kSvPos * HD / 16 == 4 * HD, "four pieces per thread");
    const auto piece = [&](uint32_t i) {
        return *reinterpret_cast<const int4 *>(vg + (uint64_t)min(p0 + sv_row<HD>(i), n - 1) * kv_dim +
                                               sv_col<HD>(i));
    };
    r.v0 = piece(0);
    r.v1 = piece(1);
    r.v2 = piece(2);
    r.v3 = piece(3);
    r.s0 = vsg[min(p0 + sv_row<HD>(0), n - 1)];
    r.s1 = vsg[min(p0 + sv_row<HD>(1), n - 1)];
    r.s2 = vsg[min(p0 + sv_row<HD>(2), n - 1)];
    r.s3 = vsg[min(p0 + sv_row<HD>(3), n - 1)];
}
// the tile's codes into vt[row][col] as loaded, and each row's scale into vst[row]
template <int HD>
__device__ __forceinline__ void sv_stage(const sv_regs &r, int8_t (*vt)[HD], float *vst) {
    *reinterpret_cast<int4 *>(&vt[sv_row<HD>(0)][sv_col<HD>(0)]) = r.v0;
    *reinterpret_cast<int4 *>(&vt[sv_row<HD>(1)][sv_col<HD>(1)]) = r.v1;
    *reinterpret_cast<int4 *>(&vt[sv_row<HD>(2)][sv_col<HD>(2)]) = r.v2;
    *reinterpret_cast<int4 *>(&vt[sv_row<HD>(3)][sv_col<HD>(3)]) = r.v3;
    if (sv_col<HD>(0) == 0) vst[sv_row<HD>(0)] = r.s0;
    if (sv_col<HD>(1) == 0) vst[sv_row<HD>(1)] = r.s1;
    if (sv_col<HD>(2) == 0) vst[sv_row<HD>(2)] = r.s2;
    if (sv_col<HD>(3) == 0) vst[sv_row<HD>(3)] = r.s3;
}

// Softmax of one (token, head) row of scores per wave (attention.rs:45-73):
// max, exp (glibc expf) in place, the exact sequential sum of the exps by the
// one-wave algorithm (512 exps per step, summed from the registers that
// computed them) and the row's scale 1/sum (1 when the sum is not positive:
// the reference leaves the row unnormalised); the V pass forms each weight as
// exp * scale, the same f32 product the reference's `*= inv` makes.  Tiles of
// kSvPos positions whose exps are all exactly zero are flagged dead: their
// weights are zero, and a zero term leaves each of the V pass's sums
// unchanged (those sums start at +0 and can never be -0), so it skips them.
// A row whose maximum is not finite becomes all zero (its output is then 0).
// The rows of a workgroup are heads of one token, so its waves have equal
// work; a row's sum has no barrier and no idle wave, and the many rows of a
// batch keep every SIMD busy.
constexpr uint32_t kSmRows = 4;  // rows per workgroup, one per wave
static_assert(kSvPos % 8 == 0 && wm::kSeqBatch / kSvPos == 8, "a step's tiles are 8-lane groups");
__global__ __launch_bounds__(kSmRows * 64) void k_attn_softmax_rows(attn_rows_args a) {
    __shared__ uint64_t exp_tab[32];
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wid = (uint32_t)__builtin_amdgcn_readfirstlane((int)(tid >> 6));
    if (tid < 32) exp_tab[tid] = wm::kExp2Tab[tid];
    __syncthreads();
    const uint32_t h = blockIdx.x * kSmRows + wid, t = blockIdx.y;
    if (h >= a.n_heads) return;
    const uint32_t n = a.tok[t].pos + 1, n_tiles = (n + kSvPos - 1) / kSvPos;  // n_tiles <= 64
    const uint64_t row = (uint64_t)t * a.n_heads + h;
    float *w = a.scores + row * a.score_stride;
    uint8_t *live = a.live + row * kAttnTiles;
    // The row's float4s below n4 = ceil(n / 4) lie inside it (rows start
    // 16-byte aligned and score_stride >= n rounded up to 4); indices are
    // clamped to n4 - 1 and components at n and beyond are masked.
    const float4 *w4 = reinterpret_cast<const float4 *>(w);
    const uint32_t n4 = (n + 3) / 4;
    float mx = -INFINITY;
    for (uint32_t q0 = 0; q0 < n4; q0 += 256) {  // lane l: float4s q0 + l + 64i
        float4 x[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t q = q0 + lane + 64 * i;
            x[i] = w4[min(q, n4 - 1)];
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t p = 4 * (q0 + lane + 64 * i);
            mx = wm_max_nonan(mx, p < n ? x[i].x : -INFINITY);
            mx = wm_max_nonan(mx, p + 1 < n ? x[i].y : -INFINITY);
            mx = wm_max_nonan(mx, p + 2 < n ? x[i].z : -INFINITY);
            mx = wm_max_nonan(mx, p + 3 < n ? x[i].w : -INFINITY);
        }
    }
    mx = wm_wave_max_nonan(mx);
    if (!isfinite(mx)) {  // every weight becomes 0 (or the row held a NaN)
        for (uint32_t k = lane; k < n; k += 64) w[k] = 0.0f;
        if (lane < n_tiles) live[lane] = 0;
        if (lane == 0) a.row_scale[row] = 0.0f;
        return;
    }
    // steps of 512: lane l takes positions k + 8l .. k + 8l + 7; the next
    // step's scores are loaded before this step's sum
    float4 c0 = w4[min(2 * lane, n4 - 1)], c1 = w4[min(2 * lane + 1, n4 - 1)];
    float sum = 0.0f;
    for (uint32_t k = 0; k < n; k += wm::kSeqBatch) {
        const uint32_t base = k + 8 * lane;
        float4 n0 = c0, n1 = c1;
        if (k + wm::kSeqBatch < n) {
            const uint32_t nq = (base + wm::kSeqBatch) / 4;
            n0 = w4[min(nq, n4 - 1)];
            n1 = w4[min(nq + 1, n4 - 1)];
        }
        float v[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
        bool nz = false;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            v[j] = base + j < n ? wm::expf_glibc(v[j] - mx, exp_tab) : 0.0f;
            nz = nz || v[j] != 0.0f;
        }
        if (base + 8 <= n) {
            *reinterpret_cast<float4 *>(w + base) = make_float4(v[0], v[1], v[2], v[3]);
            *reinterpret_cast<float4 *>(w + base + 4) = make_float4(v[4], v[5], v[6], v[7]);
        } else {
#pragma unroll
            for (int j = 0; j < 8; j++)
                if (base + j < n) w[base + j] = v[j];
        }
        // lanes 8i .. 8i+7 hold tile k / kSvPos + i
        const uint64_t nzm = __ballot(nz);
        const uint32_t tile = k / kSvPos + lane;
        if (lane < 8 && tile < n_tiles) live[tile] = ((nzm >> (8 * lane)) & 0xFFu) != 0 ? 1 : 0;
        sum = wm::seq_sum_step(sum, v, k == 0);
        c0 = n0;
        c1 = n1;
    }
    if (lane == 0) a.row_scale[row] = sum > 0.0f ? 1.0f / sum : 1.0f;
}

// One group of 8 positions of a staged tile, as thread d reads it: the V
// codes vt[q][d], the rows' scales and the C chains' weights.
template <uint32_t C>
struct sv_group {
    int code[8];
    float4 sc[2];
    float4 w[C][2];
};
template <int HD, uint32_t C>
__device__ __forceinline__ void sv_read(sv_group<C> &g, const int8_t (*vt)[HD], const float *vst,
                                        const float (*wt)[kSvPos], uint32_t q0) {
#pragma unroll
    for (uint32_t j = 0; j < 8; j++) g.code[j] = vt[q0 + j][threadIdx.x];
    g.sc[0] = *reinterpret_cast<const float4 *>(&vst[q0]);
    g.sc[1] = *reinterpret_cast<const float4 *>(&vst[q0 + 4]);
#pragma unroll
    for (uint32_t c = 0; c < C; c++) {
        g.w[c][0] = *reinterpret_cast<const float4 *>(&wt[c][q0]);
        g.w[c][1] = *reinterpret_cast<const float4 *>(&wt[c][q0 + 4]);
    }
}
// acc[c] += w * v for the group's positions in order (v = q8 * scale: read_into)
template <uint32_t C>
__device__ __forceinline__ void sv_sum(float (&acc)[C], const sv_group<C> &g) {
    const float sc[8] = {g.sc[0].x, g.sc[0].y, g.sc[0].z, g.sc[0].w, g.sc[1].x, g.sc[1].y, g.sc[1].z, g.sc[1].w};
    float v[8];
#pragma unroll
    for (uint32_t j = 0; j < 8; j++) v[j] = (float)g.code[j] * sc[j];
#pragma unroll
    for (uint32_t c = 0; c < C; c++) {
        const float w[8] = {g.w[c][0].x, g.w[c][0].y, g.w[c][0].z, g.w[c][0].w,
                            g.w[c][1].x, g.w[c][1].y, g.w[c][1].z, g.w[c][1].w};
#pragma unroll
        for (uint32_t j = 0; j < 8; j++) acc[c] = acc[c] + w[j] * v[j];
    }
}

// G: query heads per workgroup, HG: per KV head (item unit = kv head * HG/G + part)
template <int HD, int G, int HG>
__global__ __launch_bounds__(HD) void k_attn_sv_rows(attn_rows_args a) {
    constexpr uint32_t C = kSvTok * G;  // chains per thread: c = token * G + head
    __shared__ __align__(16) int8_t vt[kSvPos][HD];
    __shared__ __align__(16) float vst[kSvPos];
    __shared__ __align__(16) float wt[C][kSvPos];
    __shared__ uint64_t live_mask;
    const wm_attn_item it = a.sv_items[blockIdx.x];
    if (it.nt == 0) return;
    const uint32_t kvh = it.unit / (HG / G), h0 = it.unit * G;  // first query head
    const uint32_t tid = threadIdx.x;
    const wm_batch_tok tk = a.tok[it.t0];  // the item's tokens share this cache
    const uint32_t n = it.p1;              // the last token's context: every tile any chain needs
    uint32_t nt_ctx[kSvTok];
#pragma unroll
    for (uint32_t tt = 0; tt < kSvTok; tt++) nt_ctx[tt] = tt < it.nt ? a.tok[it.t0 + tt].pos + 1 : 0u;
    // the tiles where any chain has a non-zero exp, in position order
    const uint32_t n_tiles = (n + kSvPos - 1) / kSvPos;
    if (tid < 64) {
        bool lv = false;
        if (tid < n_tiles)
#pragma unroll
            for (uint32_t c = 0; c < C; c++)
                if (c / G < it.nt && tid * kSvPos < nt_ctx[c / G])
                    lv = lv || a.live[((uint64_t)(it.t0 + c / G) * a.n_heads + h0 + c % G) * kAttnTiles + tid];
        const uint64_t mask = __ballot(lv);
        if (tid == 0) live_mask = mask;
    }
    const uint64_t lay = (uint64_t)a.layer * tk.max_seq;
    const int8_t *vg = tk.v + lay * a.kv_dim + kvh * HD;
    const float *vsg = tk.vs + lay;
    float acc[C];
#pragma unroll
    for (uint32_t c = 0; c < C; c++) acc[c] = 0.0f;
    // this thread's weight slots e = tid + k * HD of a tile: chain e / kSvPos,
    // position e % kSvPos; the row's exps and its 1/sum
    constexpr uint32_t WK = (C * kSvPos + HD - 1) / HD;
    const float *wrow[WK];
    float wscale[WK];
    uint32_t wlim[WK];
#pragma unroll
    for (uint32_t k = 0; k < WK; k++) {
        const uint32_t e = min(tid + k * HD, C * kSvPos - 1), c = e / kSvPos, tt = c / G;
        const uint64_t row = (uint64_t)(it.t0 + min(tt, it.nt - 1)) * a.n_heads + h0 + c % G;
        wrow[k] = a.scores + row * a.score_stride + e % kSvPos;
        wscale[k] = a.row_scale[row];
        // positions below this one count (none for a slot past the tile)
        wlim[k] = tt < it.nt && tid + k * HD < C * kSvPos ? nt_ctx[tt] : 0u;
    }
    float wr[WK];  // the next tile's exps, loaded with its V codes
    const auto wfetch = [&](uint32_t p0) {
#pragma unroll
        for (uint32_t k = 0; k < WK; k++)
            wr[k] = p0 + (tid + k * HD) % kSvPos < wlim[k] ? wrow[k][p0] : 0.0f;
    };
    __syncthreads();
    uint64_t mask = live_mask;
    sv_regs pr{};
    if (mask) {
        sv_fetch<HD>(pr, vg, vsg, a.kv_dim, (uint32_t)__builtin_ctzll(mask) * kSvPos, n);
        wfetch((uint32_t)__builtin_ctzll(mask) * kSvPos);
    }
    while (mask) {
        mask &= mask - 1;
        __syncthreads();  // the previous tile is summed
        sv_stage<HD>(pr, vt, vst);
#pragma unroll
        for (uint32_t k = 0; k < WK; k++)
            if (tid + k * HD < C * kSvPos) (&wt[0][0])[tid + k * HD] = wr[k] * wscale[k];  // exp * (1/sum)
        __syncthreads();
        if (mask) {
            sv_fetch<HD>(pr, vg, vsg, a.kv_dim, (uint32_t)__builtin_ctzll(mask) * kSvPos, n);
            wfetch((uint32_t)__builtin_ctzll(mask) * kSvPos);
        }
        // groups of 8 positions; a group's LDS reads are issued before the
        // previous group is summed, so their latency overlaps that work
        sv_group<C> ga, gb;
        sv_read<HD, C>(ga, vt, vst, wt, 0);
#pragma unroll
        for (uint32_t q = 0; q < kSvPos; q += 16) {
            sv_read<HD, C>(gb, vt, vst, wt, q + 8);
            sv_sum<C>(acc, ga);
            if (q + 16 < kSvPos) sv_read<HD, C>(ga, vt, vst, wt, q + 16);
            sv_sum<C>(acc, gb);
        }
    }
#pragma unroll
    for (uint32_t c = 0; c < C; c++)
        if (c / G < it.nt)
            a.out[(uint64_t)(it.t0 + c / G) * a.n_heads * HD + (uint64_t)(h0 + c % G) * HD + tid] = acc[c];
}

}  // namespace

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------

namespace {
constexpr uint32_t kGemmCus = 256;
}  // namespace

wm_gemm_plan wm_gemm_make_plan(uint32_t groups, uint32_t n_chunks, uint32_t m) {
    (void)n_chunks;
    wm_gemm_plan p;
    p.tiles = (m + WM_GEMM_TILE_TOKENS - 1) / WM_GEMM_TILE_TOKENS;
    // Up to two 64 x 64 output tiles per CU: the waves split K
    // (k_i2s_gemm_kw, 3 chunks in flight per wave; two workgroups fit a
    // CU's LDS).  More: the waves split the tokens of two groups per
    // workgroup (k_i2s_gemm, double-buffered).  These were the faster
    // choices in a sweep of both kernels, NG and ring depth over the
    // BitNet-2B shapes at M = 257.
    if (groups * p.tiles <= 2 * kGemmCus) {
        p.kw = true;
        p.ng = 1;
        p.st = 3;
    } else {  // more than 512 tiles: at least 256 workgroups of two groups
        p.ng = 2;
        p.st = 2;
    }
    p.gx = (groups + p.ng - 1) / p.ng;
    return p;
}

bool wm_launch_i2s_gemm(const wm_gemm_desc *d, int n_desc, uint32_t n_chunks, const uint8_t *act,
                        uint32_t m, uint32_t m_pad, const wm_act_meta *meta, float *y,
                        uint32_t ldy, hipStream_t s) {
    gemm_args a{};
    uint32_t groups = 0;
    for (int i = 0; i < n_desc; i++) {
        a.d[i] = d[i];
        groups += d[i].n_groups;
        a.group_end[i] = groups;
    }
    a.n_desc = n_desc;
    a.n_groups = groups;
    a.n_chunks = n_chunks;
    a.act = act;
    a.m = m;
    a.m_pad = m_pad;
    a.meta = meta;
    a.y = y;
    a.ldy = ldy;
    const wm_gemm_plan p = wm_gemm_make_plan(groups, n_chunks, m);
    const dim3 grid(p.gx, p.tiles);
#define WM_GEMM_CASE(KW, NG, ST)                                                                 \
    if (p.kw == KW && p.ng == NG && p.st == ST) {                                                \
        if (KW)                                                                                  \
            hipLaunchKernelGGL((k_i2s_gemm_kw<NG, ST>), grid, dim3(256), (gemm_kw_lds_bytes<NG, ST>()), s, a); \
        else                                                                                     \
            hipLaunchKernelGGL((k_i2s_gemm<NG, ST>), grid, dim3(256), (gemm_lds_bytes<NG, ST>()), s, a); \
        return true;                                                                             \
    }
    WM_GEMM_CASE(true, 1, 3)
    WM_GEMM_CASE(false, 2, 2)
#undef WM_GEMM_CASE
    return false;  // a plan with no instantiation: nothing launched
}

void wm_launch_quantize_rows(const float *x, uint32_t ldx, uint32_t n, uint32_t m, uint32_t m_pad,
                             uint8_t *act, wm_act_meta *meta, hipStream_t s) {
    hipLaunchKernelGGL(k_quantize_rows, dim3(m), dim3(kRowThreads), 0, s, x, ldx, n, m_pad, act,
                       meta);
}

bool wm_launch_rmsnorm_rows(const wm_norm_rows &a, uint32_t m, hipStream_t s) {
    const size_t lds = (size_t)wm::seq_sum_padded(a.n) * sizeof(float);
    const int per = (int)((a.n + kRowThreads - 1) / kRowThreads);
    const bool gu = a.gu != nullptr;
#define WM_ROWS_CASE(P)                                                                          \
    case P:                                                                                      \
        if (gu) hipLaunchKernelGGL((k_rmsnorm_rows<P, true>), dim3(m), dim3(kRowThreads), lds, s, a); \
        else hipLaunchKernelGGL((k_rmsnorm_rows<P, false>), dim3(m), dim3(kRowThreads), lds, s, a);   \
        return true;
    switch (per) {
        WM_ROWS_CASE(1) WM_ROWS_CASE(2) WM_ROWS_CASE(3) WM_ROWS_CASE(4)
        WM_ROWS_CASE(5) WM_ROWS_CASE(6) WM_ROWS_CASE(7) WM_ROWS_CASE(8)
        WM_ROWS_CASE(9) WM_ROWS_CASE(10) WM_ROWS_CASE(11) WM_ROWS_CASE(12)
        WM_ROWS_CASE(13) WM_ROWS_CASE(14) WM_ROWS_CASE(15) WM_ROWS_CASE(16)
        default: break;
    }
#undef WM_ROWS_CASE
    return false;  // n above 8192: no instantiation
}

void wm_launch_qkv_rows(const float *y, uint32_t ldy, const float *rope_cos, const float *rope_sin,
                        const wm_batch_tok *tok, uint32_t m, uint32_t layer, uint32_t n_q,
                        uint32_t n_kv, uint32_t head_dim, uint32_t n_rot, float *q_out,
                        hipStream_t s) {
    qkv_rows_args a{y, ldy, rope_cos, rope_sin, tok, layer, n_q, n_kv, head_dim, n_rot, q_out};
    const size_t lds = (size_t)(n_q + 2 * n_kv) * sizeof(float);
    hipLaunchKernelGGL(k_qkv_rows, dim3(m), dim3(256), lds, s, a);
}

bool wm_attn_rows_supported(uint32_t head_dim, uint32_t group) {
    return (head_dim == 64 || head_dim == 128) &&
           (group == 1 || group == 2 || group == 4 || group == 8);
}

// scores [m][n_heads][stride] | row scales [m][n_heads] | live tiles [m][n_heads][kAttnTiles]
static size_t attn_scores_part(uint32_t m, uint32_t n_heads, uint32_t n_max) {
    return ((size_t)m * n_heads * ((n_max + 3u) & ~3u) * sizeof(float) + 255) & ~(size_t)255;
}
static size_t attn_scale_part(uint32_t m, uint32_t n_heads) {
    return ((size_t)m * n_heads * sizeof(float) + 255) & ~(size_t)255;
}
static size_t attn_live_part(uint32_t m, uint32_t n_heads) {
    return ((size_t)m * n_heads * kAttnTiles + 255) & ~(size_t)255;
}
size_t wm_attn_rows_scores_bytes(uint32_t m, uint32_t n_heads, uint32_t n_max, uint32_t n_items) {
    return attn_scores_part(m, n_heads, n_max) + attn_scale_part(m, n_heads) +
           attn_live_part(m, n_heads) + (size_t)n_items * sizeof(wm_attn_item);
}
wm_attn_item *wm_attn_rows_items(float *scores, uint32_t m, uint32_t n_heads, uint32_t n_max) {
    return reinterpret_cast<wm_attn_item *>(reinterpret_cast<uint8_t *>(scores) +
                                            attn_scores_part(m, n_heads, n_max) +
                                            attn_scale_part(m, n_heads) + attn_live_part(m, n_heads));
}

uint32_t wm_attn_rows_sv_parts(uint32_t group) { return group < kSvHeads ? 1u : group / kSvHeads; }

// Items in launch order.  Workgroup i runs on XCD i % 8, so the items of one
// (sequence, unit) group, which read the same K or V rows, are all given
// the same i % 8 and share that XCD's L2; groups go to the least-loaded XCD,
// largest first, and the shorter lists are padded with empty items.
static void attn_place(std::vector<std::vector<wm_attn_item>> &groups, std::vector<uint64_t> &work,
                       std::vector<wm_attn_item> &out) {
    constexpr uint32_t kXcds = 8;
    std::vector<uint32_t> order(groups.size());
    for (uint32_t i = 0; i < order.size(); i++) order[i] = i;
    std::sort(order.begin(), order.end(), [&](uint32_t x, uint32_t y) { return work[x] > work[y]; });
    std::vector<std::vector<wm_attn_item>> lists(kXcds);
    uint64_t load[kXcds] = {};
    for (uint32_t g : order) {
        uint32_t x = 0;
        for (uint32_t k = 1; k < kXcds; k++)
            if (load[k] < load[x]) x = k;
        load[x] += work[g];
        lists[x].insert(lists[x].end(), groups[g].begin(), groups[g].end());
    }
    size_t len = 0;
    for (auto &l : lists) len = std::max(len, l.size());
    out.assign(len * kXcds, wm_attn_item{0, 0, 0, 0, 0, 0});
    for (uint32_t x = 0; x < kXcds; x++)
        for (size_t k = 0; k < lists[x].size(); k++) out[k * kXcds + x] = lists[x][k];
}

void wm_attn_rows_plan(const wm_batch_tok *tok, uint32_t m, uint32_t sc_units, uint32_t sv_units,
                       std::vector<wm_attn_item> &sc, std::vector<wm_attn_item> &sv) {
    std::vector<std::vector<wm_attn_item>> sc_groups, sv_groups;
    std::vector<uint64_t> sc_work, sv_work;
    for (uint32_t t = 0; t < m;) {
        uint32_t e = t + 1;  // the sequence's tokens: same cache, consecutive positions
        while (e < m && tok[e].k == tok[t].k && tok[e].pos == tok[e - 1].pos + 1) e++;
        for (uint32_t u = 0; u < sc_units; u++) {
            std::vector<wm_attn_item> g;
            uint64_t w = 0;
            for (uint32_t b = t; b < e; b += kScoreTok) {
                const uint32_t nt = std::min<uint32_t>(kScoreTok, e - b), p1 = tok[b + nt - 1].pos + 1;
                for (uint32_t p0 = 0; p0 < p1; p0 += kScoreThreads) g.push_back({b, nt, p0, p1, u, 0});
                w += (uint64_t)nt * p1;
            }
            sc_groups.push_back(g);
            sc_work.push_back(w);
        }
        for (uint32_t u = 0; u < sv_units; u++) {
            std::vector<wm_attn_item> g;
            uint64_t w = 0;
            for (uint32_t b = t; b < e; b += kSvTok) {
                const uint32_t nt = std::min<uint32_t>(kSvTok, e - b), p1 = tok[b + nt - 1].pos + 1;
                g.push_back({b, nt, 0, p1, u, 0});
                w += (uint64_t)nt * p1;
            }
            sv_groups.push_back(g);
            sv_work.push_back(w);
        }
        t = e;
    }
    attn_place(sc_groups, sc_work, sc);
    attn_place(sv_groups, sv_work, sv);
}

void wm_launch_attn_rows(const float *q, const wm_batch_tok *tok, uint32_t m, uint32_t n_max,
                         uint32_t layer, uint32_t n_kv_heads, uint32_t head_dim, uint32_t group,
                         float scale, float *scores, float *out, uint32_t n_sc, uint32_t n_sv,
                         hipStream_t s) {
    const uint32_t n_heads = n_kv_heads * group;
    uint8_t *base = reinterpret_cast<uint8_t *>(scores);
    float *row_scale = reinterpret_cast<float *>(base + attn_scores_part(m, n_heads, n_max));
    uint8_t *live = base + attn_scores_part(m, n_heads, n_max) + attn_scale_part(m, n_heads);
    const wm_attn_item *items = wm_attn_rows_items(scores, m, n_heads, n_max);
    attn_rows_args a{q, tok, scores, out, layer, n_kv_heads * head_dim, n_heads,
                     (n_max + 3u) & ~3u, n_max, scale, row_scale, live, items, items + n_sc};
    const dim3 sgrid(n_sc);
#define WM_SCORES_CASE(HD, G)                                                                  \
    if (head_dim == HD && group == G)                                                          \
        hipLaunchKernelGGL((k_attn_scores_rows<HD, G>), sgrid, dim3(kScoreThreads), 0, s, a);
    WM_SCORES_CASE(128, 1) WM_SCORES_CASE(128, 2) WM_SCORES_CASE(128, 4) WM_SCORES_CASE(128, 8)
    WM_SCORES_CASE(64, 1) WM_SCORES_CASE(64, 2) WM_SCORES_CASE(64, 4) WM_SCORES_CASE(64, 8)
#undef WM_SCORES_CASE
    hipLaunchKernelGGL(k_attn_softmax_rows, dim3((n_heads + kSmRows - 1) / kSmRows, m), dim3(kSmRows * 64),
                       0, s, a);
#define WM_SV_CASE(HD, G)                                                                      \
    if (head_dim == HD && group == G)                                                          \
        hipLaunchKernelGGL((k_attn_sv_rows<HD, (G < kSvHeads ? G : kSvHeads), G>),             \
                           dim3(n_sv), dim3(HD), 0, s, a);
    WM_SV_CASE(128, 1) WM_SV_CASE(128, 2) WM_SV_CASE(128, 4) WM_SV_CASE(128, 8)
    WM_SV_CASE(64, 1) WM_SV_CASE(64, 2) WM_SV_CASE(64, 4) WM_SV_CASE(64, 8)
#undef WM_SV_CASE
}
