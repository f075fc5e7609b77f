// Internal definitions shared by the HIP translation units of
// libwillamette_hip.so.  gfx950 (CDNA4) only.
//
// Every f32 expression on the decode path is evaluated as the reference's
// Rust code evaluates it: one IEEE round-to-nearest-even rounding per `+`,
// `*`, `/`, `sqrt`, never contracted (the library is built with
// -ffp-contract=off; fused multiply-adds appear only where written as
// __builtin_fma* and are exact there), IEEE denormals, and reductions in the
// reference's sequential order wherever the reference's order fixes the
// rounding.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

#include "willamette_hip.h"
#define WM_HD __host__ __device__
#include "wm_expf.h"

// ---------------------------------------------------------------------------
// host-side plumbing
// ---------------------------------------------------------------------------

struct wm_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    std::string last_error;
    // Scratch used by the host-pointer entry points (grown on demand).
    void *scratch = nullptr;
    size_t scratch_bytes = 0;
    void *pinned = nullptr;  // pinned host staging
    size_t pinned_bytes = 0;
    // Multi-tensor matvec: device copies of the last call's weight pointers
    // and scales (re-sent only when they change).
    void *multi_dev = nullptr;
    size_t multi_bytes = 0;
    std::vector<const void *> multi_ptrs;
    std::vector<float> multi_scales;
    // Device address, on this context's device, of the file-scope scratch
    // array of wm_bitlinear_i2s_matvec_f32_dev_noalloc (wm_noalloc.hip).
    void *noalloc_scratch = nullptr;
    // test hook: WM_FUSED_DEBUG_* bits for every fused matvec launched here
    uint32_t fused_debug = 0;
};

// Objects created on a context keep their own device id: destroying them
// never touches the context (which may already be gone); hipFree
// synchronises the device itself.
struct wm_tensor {
    wm_ctx *ctx = nullptr;
    int device = 0;
    int type = 0;
    uint64_t in_dim = 0;   // I2_S: columns; Q6_K: row_len
    uint64_t out_dim = 0;  // I2_S: rows;    Q6_K: n_rows
    float scale = 1.0f;    // I2_S per-tensor scale
    void *d = nullptr;     // device data in the library's layout
    size_t bytes = 0;
    // I2_S layout: 64-row groups x (in_dim/64) 16-byte chunks x 64 rows.
    uint32_t n_groups = 0, n_chunks = 0;
    // Q6_K layout: 4-row groups x blocks, 840 bytes per (group, block).
    uint32_t n_rowgroups = 0, n_blocks = 0;
};

wm_status wm_set_error(wm_ctx *ctx, wm_status st, const char *fmt, ...);
wm_status wm_hip_error(wm_ctx *ctx, hipError_t e, const char *what);
#define WM_HIP(ctx, expr)                                          \
    do {                                                           \
        hipError_t e_ = (expr);                                    \
        if (e_ != hipSuccess) return wm_hip_error((ctx), e_, #expr); \
    } while (0)

// Looks up ctx->noalloc_scratch (called by wm_ctx_create, device current).
wm_status wm_noalloc_setup(wm_ctx *ctx);
// Grows ctx->scratch to at least `bytes` and returns it.
wm_status wm_ctx_scratch(wm_ctx *ctx, size_t bytes, void **out);
wm_status wm_ctx_pinned(wm_ctx *ctx, size_t bytes, void **out);

// ---------------------------------------------------------------------------
// constants of the I2_S / Q6_K formats (src/gguf/tensor.rs:86-105)
// ---------------------------------------------------------------------------
constexpr int QK_I2S = 128;        // values per packed block
constexpr int I2S_BLOCK_BYTES = 32;
constexpr int I2S_GROUP_ROWS = 64;  // rows per group of the device layout
constexpr int I2S_CHUNK_COLS = 64;  // columns covered by one 16-byte chunk
#define WM_I2S_MAX_MULTI 64
constexpr int Q6K_VALUES = 256;
constexpr int Q6K_BYTES = 210;
constexpr int Q6K_GROUP_ROWS = 4;         // rows per wave in the device layout
constexpr int Q6K_GROUP_BLOCK_BYTES = 840;  // 4 rows x 210 bytes
constexpr int Q6K_QUANT_BYTES = 768;        // six-bit quants of one (group, block)
// Within a group of n_blocks blocks: the quants of block b at 768*b, then the
// sub-scale dwords of class c = 4*row + quarter as [c][b] from 768*n_blocks,
// then the f16 d values as [row][b] from 832*n_blocks, each row's run padded
// to an even count (so an even run of blocks starts on a dword).
__host__ __device__ inline uint32_t q6k_sc_base(uint32_t n_blocks) { return 768u * n_blocks; }
__host__ __device__ inline uint32_t q6k_d_base(uint32_t n_blocks) { return 832u * n_blocks; }
__host__ __device__ inline uint32_t q6k_d_stride(uint32_t n_blocks) { return (n_blocks + 1) & ~1u; }
__host__ __device__ inline uint32_t q6k_group_bytes(uint32_t n_blocks) {
    return 832u * n_blocks + 8u * q6k_d_stride(n_blocks);
}
// After the 4-row-group layout, 256-aligned: one f32 per row holding
// sum_j |d * sc_j| rounded up (x-independent part of the id-only lm-head's
// error bound).  Part of the same allocation, so copies of the tensor carry it.
__host__ __device__ inline size_t wm_q6k_sigma_offset(uint32_t n_rowgroups, uint32_t n_blocks) {
    return ((size_t)n_rowgroups * q6k_group_bytes(n_blocks) + 255) & ~(size_t)255;
}

// ---------------------------------------------------------------------------
// device helpers
// ---------------------------------------------------------------------------

// Rust `(v).round().clamp(-127.0, 127.0) as i8`: round half away from zero,
// a clamp that lets NaN through, and a saturating cast that maps NaN to 0
// (src/model/bitlinear_sse2.rs:300, src/model/kv_cache.rs:255).
__device__ __forceinline__ int wm_round_clamp_i8(float v) {
    float r = roundf(v);
    r = r < -127.0f ? -127.0f : r;
    r = r > 127.0f ? 127.0f : r;
    return (r != r) ? 0 : (int)r;
}
// The same value in fewer operations: round half away from zero of |v| is
// trunc(|v|) + (fract(|v|) >= 0.5), both exact (floor(|v| + 0.5) is not: the
// add rounds 0.5 - 2^-25 up to 1); v_cvt_u32_f32 truncates, gives 0 for NaN
// and saturates (a C cast would leave NaN and overflow undefined), and the
// fraction of inf, NaN or anything at or above 2^23 is not >= 0.5, so one
// min makes the clamp.
__device__ __forceinline__ int wm_round_clamp_i8_fast(float v) {
    const float a = fabsf(v);
    uint32_t t;
    asm("v_cvt_u32_f32 %0, %1" : "=v"(t) : "v"(a));
    const uint32_t m = min(t + (__builtin_amdgcn_fractf(a) >= 0.5f ? 1u : 0u), 127u);
    return __float_as_int(v) < 0 ? -(int)m : (int)m;
}

// Exact IEEE binary16 -> binary32 in integer arithmetic
// (src/model/primitives.rs:61-88); no dependence on the FP unit's
// denormal mode.
__device__ __forceinline__ float wm_f16_bits_to_f32(uint32_t bits) {
    uint32_t sign = (bits >> 15) & 1u, exp = (bits >> 10) & 0x1Fu, man = bits & 0x3FFu;
    uint32_t out;
    if (exp == 0) {
        if (man == 0) {
            out = sign << 31;
        } else {
            // normalise the subnormal: value = man * 2^-24
            int sh = __clz(man) - 21;  // leading zeros within 10 bits, +1 to hide the MSB
            man = (man << sh) & 0x3FFu;
            out = (sign << 31) | ((uint32_t)(127 - 15 + 1 - sh) << 23) | (man << 13);
        }
    } else if (exp == 0x1F) {
        out = (sign << 31) | (0xFFu << 23) | (man << 13);
    } else {
        out = (sign << 31) | ((exp + (127 - 15)) << 23) | (man << 13);
    }
    return __uint_as_float(out);
}

// glibc-identical expf (host/device, see wm_expf.h)
__device__ __forceinline__ float wm_expf(float x) { return wm::expf_glibc(x); }

// Streaming (non-temporal) 16-byte load for data read exactly once, such as
// matvec weights: it keeps them from displacing reused lines in the caches.
typedef unsigned int wm_v4u __attribute__((ext_vector_type(4)));
// The pointer is taken as global memory: a generic (flat) load would also
// count against the LDS wait counter, tying every LDS wait to the weights.
typedef const wm_v4u __attribute__((address_space(1))) wm_global_v4u;
typedef const uint32_t __attribute__((address_space(1))) wm_global_u32;
__device__ __forceinline__ uint4 wm_load_stream(const void *p) {
    const wm_v4u v = __builtin_nontemporal_load((wm_global_v4u *)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint32_t wm_load_stream_u32(const void *p) {
    return __builtin_nontemporal_load((wm_global_u32 *)p);
}

// Buffer resource for raw (unformatted) loads from `bytes` bytes at `base`;
// base must be wave-uniform (the descriptor lives in SGPRs).  Loads take a
// per-lane 32-bit offset plus a wave-uniform one, so streaming kernels spend
// no vector instructions on addresses; a lane offset at or past `bytes`
// reads zeros.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t wm_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes,
                                             0x00020000);
}
constexpr int WM_LOAD_NT = 2;  // cache policy bits of a buffer load: non-temporal
typedef unsigned int wm_v3u __attribute__((ext_vector_type(3)));

// DPP lane moves of the wave64 GFX9 family: row_shr:n (lane i of a 16-lane
// row reads lane i-n of the same row), row_bcast:15 (lane 15 of each row to
// every lane of the next row), row_bcast:31 (lane 31 to rows 2 and 3).
// Lanes with no source, and rows outside ROW_MASK, read 0.  The whole wave
// must be active.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ int wm_dpp(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, ROW_MASK, 0xF, true);
}
constexpr int WM_DPP_ROW_SHR1 = 0x111, WM_DPP_ROW_SHR2 = 0x112, WM_DPP_ROW_SHR4 = 0x114,
              WM_DPP_ROW_SHR8 = 0x118, WM_DPP_ROW_BCAST15 = 0x142, WM_DPP_ROW_BCAST31 = 0x143;

// Inclusive wave scans (Hillis-Steele inside rows, then the two row
// broadcasts).  Integer scans are exact; the float64 scan is a tree of
// depth 6 over its inputs.
template <int CTRL, int RM>
__device__ __forceinline__ long long wm_dpp_i64(long long x) {
    const int lo = wm_dpp<CTRL, RM>((int)(unsigned long long)x);
    const int hi = wm_dpp<CTRL, RM>((int)((unsigned long long)x >> 32));
    return (long long)(((unsigned long long)(unsigned)hi << 32) | (unsigned)lo);
}
__device__ __forceinline__ int wm_wave_scan_i32(int x) {
    x += wm_dpp<WM_DPP_ROW_SHR1, 0xF>(x);
    x += wm_dpp<WM_DPP_ROW_SHR2, 0xF>(x);
    x += wm_dpp<WM_DPP_ROW_SHR4, 0xF>(x);
    x += wm_dpp<WM_DPP_ROW_SHR8, 0xF>(x);
    x += wm_dpp<WM_DPP_ROW_BCAST15, 0xA>(x);
    x += wm_dpp<WM_DPP_ROW_BCAST31, 0xC>(x);
    return x;
}
__device__ __forceinline__ long long wm_wave_scan_i64(long long x) {
    x += wm_dpp_i64<WM_DPP_ROW_SHR1, 0xF>(x);
    x += wm_dpp_i64<WM_DPP_ROW_SHR2, 0xF>(x);
    x += wm_dpp_i64<WM_DPP_ROW_SHR4, 0xF>(x);
    x += wm_dpp_i64<WM_DPP_ROW_SHR8, 0xF>(x);
    x += wm_dpp_i64<WM_DPP_ROW_BCAST15, 0xA>(x);
    x += wm_dpp_i64<WM_DPP_ROW_BCAST31, 0xC>(x);
    return x;
}
__device__ __forceinline__ double wm_wave_scan_f64(double x) {
#define WM_F64_STEP(C, R) x += __longlong_as_double(wm_dpp_i64<C, R>(__double_as_longlong(x)))
    WM_F64_STEP(WM_DPP_ROW_SHR1, 0xF);
    WM_F64_STEP(WM_DPP_ROW_SHR2, 0xF);
    WM_F64_STEP(WM_DPP_ROW_SHR4, 0xF);
    WM_F64_STEP(WM_DPP_ROW_SHR8, 0xF);
    WM_F64_STEP(WM_DPP_ROW_BCAST15, 0xA);
    WM_F64_STEP(WM_DPP_ROW_BCAST31, 0xC);
#undef WM_F64_STEP
    return x;
}
// Wave totals, returned wave-uniform (lane 63 of an inclusive scan).
__device__ __forceinline__ int wm_wave_total_i32(int x) {
    return __builtin_amdgcn_readlane(wm_wave_scan_i32(x), 63);
}
// Largest of non-negative values, NaN never winning (a NaN input counts as 0).
__device__ __forceinline__ float wm_wave_max_nonneg(float v) {
    v = v > 0.0f ? v : 0.0f;
#define WM_MAX_STEP(C, R)                                                                          \
    {                                                                                              \
        const float o = __int_as_float(wm_dpp<C, R>(__float_as_int(v)));                           \
        v = o > v ? o : v;                                                                         \
    }
    WM_MAX_STEP(WM_DPP_ROW_SHR1, 0xF);
    WM_MAX_STEP(WM_DPP_ROW_SHR2, 0xF);
    WM_MAX_STEP(WM_DPP_ROW_SHR4, 0xF);
    WM_MAX_STEP(WM_DPP_ROW_SHR8, 0xF);
    WM_MAX_STEP(WM_DPP_ROW_BCAST15, 0xA);
    WM_MAX_STEP(WM_DPP_ROW_BCAST31, 0xC);
#undef WM_MAX_STEP
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Workgroup barrier for LDS traffic: waits for this wave's LDS (and scalar)
// operations, then s_barrier.  Unlike __syncthreads it does not wait for the
// wave's global loads and stores, so a store issued before it stays in
// flight; use it only where the waves exchange data through LDS alone.
__device__ __forceinline__ void wm_sync_lds() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Wave-level helpers (wave64).
__device__ __forceinline__ int wm_wave_sum_i32(int v) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
// max that never lets a NaN win (`if a > m { m = a }`)
__device__ __forceinline__ float wm_max_nonan(float m, float a) { return a > m ? a : m; }
__device__ __forceinline__ float wm_wave_max_nonan(float v) {
    for (int o = 32; o > 0; o >>= 1) v = wm_max_nonan(v, __shfl_xor(v, o, 64));
    return v;
}

// Block-wide reductions (red: >= blockDim/64 slots of LDS).  Both are
// order-free: a NaN-ignoring max and an integer sum.
__device__ __forceinline__ float wm_block_max_nonan(float v, float *red) {
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    v = wm_wave_max_nonan(v);
    wm_sync_lds();
    if (lane == 0) red[wid] = v;
    wm_sync_lds();
    float m = red[0];
    for (int w = 1; w < (int)(blockDim.x >> 6); w++) m = wm_max_nonan(m, red[w]);
    return m;
}
__device__ __forceinline__ int wm_block_sum_i32(int v, int *red) {
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    v = wm_wave_sum_i32(v);
    wm_sync_lds();
    if (lane == 0) red[wid] = v;
    wm_sync_lds();
    int t = 0;
    for (int w = 0; w < (int)(blockDim.x >> 6); w++) t += red[w];
    return t;
}

// KV quantisation of one token vector (src/model/kv_cache.rs:245-259), by
// the whole workgroup: absmax (NaN never raises it); a zero or non-finite
// absmax stores zeros with scale 0.
__device__ inline void wm_kv_quantise_store(const float *__restrict__ v, uint32_t n,
                                            int8_t *__restrict__ q, float *__restrict__ scale_out,
                                            float *red) {
    float m = 0.0f;
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) m = wm_max_nonan(m, fabsf(v[i]));
    const float absmax = wm_block_max_nonan(m, red);
    if (absmax == 0.0f || !isfinite(absmax)) {
        for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) q[i] = 0;
        if (threadIdx.x == 0) *scale_out = 0.0f;
        return;
    }
    const float inv = 127.0f / absmax;
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) q[i] = (int8_t)wm_round_clamp_i8(v[i] * inv);
    if (threadIdx.x == 0) *scale_out = absmax / 127.0f;
}

// Position of activation element i (0 <= i < in_dim) in the chunk-permuted
// layout the I2_S matvec reads: chunk c = 16-byte weight chunk index along
// the row, 64 bytes per chunk ordered [quarter k][gp].
__host__ __device__ __forceinline__ uint32_t wm_act_perm(uint32_t i) {
    uint32_t bk = i >> 7, rem = i & 127u, k = rem >> 5, rem32 = rem & 31u;
    uint32_t half = rem32 >> 4, gp = rem32 & 15u;
    return (bk * 2 + half) * 64 + k * 16 + gp;
}

// ---------------------------------------------------------------------------
// kernel launchers (defined in the .hip files)
// ---------------------------------------------------------------------------

// Activation record written by every quantising kernel and read by the
// matvec epilogues: the per-vector absmax scale and the sum of the int8
// activations (the matvec computes sum(code * a) with code in {0,1,2} and
// subtracts sum(a) to obtain sum(ternary * a)).
struct wm_act_meta {
    float scale;
    int32_t asum;
};

// I2_S repack: raw TensorView bytes (device) -> library layout (device).
void wm_launch_i2s_repack(const uint8_t *raw, uint8_t *out, uint32_t in_dim, uint32_t out_dim,
                          uint32_t n_groups, hipStream_t s);
// Quantise f32 x[n] -> permuted int8 act + meta (one workgroup).
void wm_launch_quantize_act(const float *x, uint32_t n, uint8_t *act, wm_act_meta *meta,
                            hipStream_t s);
// The whole standalone matvec in one launch (k_i2s_matvec_one): y, and when
// non-null the integer dots, the codes in the permuted layout and the
// quantiser's scale and Σq.  False (nothing launched) for n_chunks > 256.
bool wm_launch_i2s_matvec_one(const uint8_t *w, uint32_t n_groups, uint32_t n_chunks, uint32_t out_dim,
                              float w_scale, const float *x, float *y, int32_t *dot_out, uint8_t *act_out,
                              wm_act_meta *meta_out, hipStream_t s);
// Fused matvec modes (k_i2s_fused).
constexpr int WM_FUSED_MAX_TENSORS = 3;
enum { WM_FUSED_PLAIN = 0, WM_FUSED_GATEUP = 1, WM_FUSED_ROPE = 2 };

// Partial dots over K splits (one launch covers up to WM_I2S_MAX_MULTI
// tensors sharing one input): partial[split][row], rows = n_groups*64.
struct wm_i2s_desc {
    const uint8_t *w;  // library layout
    uint32_t n_groups;
};
// The RMSNorm a fused matvec starts from (see k_i2s_fused); its length is
// the matvec's in_dim.
struct wm_fused_norm {
    const float *x;         // the norm's input
    const float *y;         // nullable: residual, the norm runs on x + y
    float *x_out;           // nullable: x + y written here, each workgroup its contiguous share
                            // (never x itself)
    const float *w;         // norm weight
    float eps;
    uint32_t *err_flag;     // nullable: set to layer_tag when x + y is not all finite
    uint32_t layer_tag;
    // nonzero: x is the gate projection and y the up projection of the FFN,
    // and the norm runs on relu(x)^2 * y (ffn.rs:37-65) instead of x + y
    uint32_t relu2_mul;
    uint32_t debug;  // WM_FUSED_DEBUG_* (test hook), 0 normally
};
// Matvec that starts from its input's norm, with the K split inside each
// workgroup and a fused epilogue (mode WM_FUSED_*): rows of tensor i go to
// outs[i] as f32; see k_i2s_fused.  groups_per_unit: 1, or head_dim / 64
// for WM_FUSED_ROPE.
// ROPE: where the launch leaves the absmax of tensors 1 and 2's outputs (K
// and V), as slots whose maximum it is (float bits; every launch of one
// shape writes the same slots): tensor t's at slots[(t - 1) * stride + i],
// i < *n_slots, which the launch sets (false when they exceed the stride).
struct wm_fused_absmax {
    uint32_t *slots;
    uint32_t stride;
    uint32_t *n_slots;
};
bool wm_launch_i2s_fused(int mode, const wm_i2s_desc *descs, const float *w_scales, float *const *outs,
                         int n_tensors, uint32_t n_chunks, uint32_t groups_per_unit,
                         const wm_fused_norm &norm, const float *rope_cos, const float *rope_sin,
                         uint32_t pos, uint32_t n_rot, uint32_t rope_mask, const wm_fused_absmax *absmax,
                         hipStream_t s, const uint32_t *pos_dev = nullptr);
void wm_launch_i2s_partial_table(const uint8_t *const *table, uint32_t n_tensors,
                                 uint32_t groups_per, uint32_t n_chunks, const uint8_t *act,
                                 int32_t *partial, uint32_t split, uint32_t rows_total,
                                 hipStream_t s);
void wm_launch_i2s_partial(const wm_i2s_desc *descs, int n_desc, uint32_t n_chunks,
                           const uint8_t *act, int32_t *partial, uint32_t split,
                           uint32_t rows_total, hipStream_t s);
// y[j] = (w_scale * act_scale) * (sum_s partial[s][j] - asum), j < out_dim.
void wm_launch_i2s_finalize(const int32_t *partial, uint32_t split, uint32_t rows_total,
                            uint32_t row0, uint32_t out_dim, float w_scale,
                            const wm_act_meta *meta, float *y, int32_t *dot_out, hipStream_t s);
uint32_t wm_i2s_pick_split(uint32_t n_groups, uint32_t n_chunks);
// Model internals the continuous-batching driver (server.cpp) uses
// (model.cpp).
struct wm_model;
struct wm_kv_cache;
wm_status batch_forward_dev(wm_model *m, wm_kv_cache *const *caches, uint32_t n_seqs,
                            const uint32_t *n_new, const uint32_t *tokens, bool want_next,
                            std::vector<uint32_t> &last_rows);
wm_ctx *wm_model_ctx(const wm_model *m);
const wm_model_config &wm_model_cfg(const wm_model *m);
bool wm_model_batch_ready(const wm_model *m);
uint32_t wm_kv_max_seq(const wm_kv_cache *kv);
wm_status wm_batch_row_logits(wm_model *m, uint32_t row, const float **d_logits);
wm_status wm_batch_next_ids(wm_model *m, uint32_t n, uint32_t *out);
// The device sampler (k_sample.hip): one Sampler::sample over n logits on
// the device, on the sampler's context stream (synchronous).
struct wm_sampler;
wm_status wm_sampler_run(wm_sampler *s, const float *d_logits, uint32_t n, uint32_t *out_id);
wm_ctx *wm_sampler_ctx(const wm_sampler *s);
// Scalar f32 matvec (no int8 activations), one lane per row:
// y[j] = scale * (pos_j - neg_j) in the reference's accumulation order.
void wm_launch_i2s_scalar_f32(const uint8_t *w, uint32_t n_groups, uint32_t n_chunks,
                              uint32_t out_dim, float scale, const float *x, float *y,
                              hipStream_t s);
void wm_launch_i2s_finalize_multi(const int32_t *partial, uint32_t split, uint32_t rows_total,
                                  uint32_t rows_per_copy, uint32_t out_dim, uint32_t n_copies,
                                  const float *w_scales, const wm_act_meta *meta, float *y,
                                  hipStream_t s);

// Q6_K
// (also writes the per-row sigma array at out + wm_q6k_sigma_offset)
void wm_launch_q6k_repack(const uint8_t *raw, uint8_t *out, uint32_t n_rows, uint32_t n_blocks,
                          uint32_t n_rowgroups, hipStream_t s);
void wm_launch_q6k_dequant_row(const uint8_t *w, uint32_t n_blocks, uint32_t row, float *out,
                               hipStream_t s);
void wm_launch_q6k_dequant_row_dev(const uint8_t *w, uint32_t n_blocks, const uint32_t *d_row,
                                   float *out, hipStream_t s);
// n_rows rows, row i = d_rows[i], written to out + i * ld
void wm_launch_q6k_dequant_rows_dev(const uint8_t *w, uint32_t n_blocks, const uint32_t *d_rows,
                                    uint32_t n_rows, float *out, uint32_t ld, hipStream_t s);
// Largest row length (in 256-value blocks) the lm-head kernels stage in LDS,
// and the most rows they take.
constexpr uint32_t WM_Q6K_LOGITS_MAX_BLOCKS = 32;
constexpr uint32_t WM_Q6K_LOGITS_MAX_ROWS = 2048u * 2048u;
// logits (exact SSE2 order, required) + per-block argmax candidates + final
// argmax (argmax_out nullable).
void wm_launch_q6k_logits_argmax(const uint8_t *w, uint32_t n_blocks, uint32_t n_rows,
                                 uint32_t n_rowgroups, const float *hidden, float *logits,
                                 uint32_t *argmax_out, void *work, hipStream_t s);
// argmax only: bounded fixed-point pass + exact rescoring of the rows that
// can still be the maximum.  logits (n_rows) receives the bounded values,
// exact on the rescored rows.
// prepared: the work buffer's prep area (wm_q6k_prep_area) already holds the
// fixed-point copy of `hidden` (the output-norm kernel writes it).
// After the argmax of a decode step whose position lives on the device:
// the id and the error flag go to ring slot (position & ring_mask) (two
// words, host memory; nullable) and the position advances by one.
struct wm_step_tail {
    uint32_t *pos;              // the step's position (device)
    uint32_t *ring;             // nullable: [ring_mask + 1][2] (id, error flag)
    const uint32_t *err_flag;   // the step's error flag (device)
    uint32_t ring_mask;
};
// The id-only lm-head of n_vec hidden vectors (hidden + rows[i] * ld), ids
// to argmax_out[i], each equal to wm_launch_q6k_argmax_fast's: one bounded
// pass over the table per four vectors.  work: wm_q6k_multi_work_bytes.
size_t wm_q6k_multi_work_bytes(uint32_t n_rows, uint32_t n_blocks);
void wm_launch_q6k_argmax_multi(const uint8_t *w, uint32_t n_blocks, uint32_t n_rows, uint32_t n_rowgroups,
                                const float *hidden, uint32_t ld, const uint32_t *rows, uint32_t n_vec,
                                uint32_t *argmax_out, void *work, hipStream_t s);
void wm_launch_q6k_argmax_fast(const uint8_t *w, uint32_t n_blocks, uint32_t n_rows,
                               uint32_t n_rowgroups, const float *hidden, float *logits,
                               uint32_t *argmax_out, void *work, bool prepared, hipStream_t s,
                               const wm_step_tail *tail = nullptr);
// test hook: the bounded pass alone (values and their error bounds)
void wm_launch_q6k_bounded_only(const uint8_t *w, uint32_t n_blocks, uint32_t n_rows,
                                uint32_t n_rowgroups, const float *hidden, float *approx,
                                float *bound_out, void *work, bool prepared, hipStream_t s);
void wm_launch_q6k_xprep(const float *hidden, uint32_t n_blocks, void *work, uint32_t n_rows,
                         hipStream_t s);
size_t wm_q6k_logits_work_bytes(uint32_t n_rows, uint32_t n_blocks);
void *wm_q6k_prep_area(void *work, uint32_t n_rows, uint32_t n_blocks);

// ---------------------------------------------------------------------------
// ragged multi-sequence batch
// ---------------------------------------------------------------------------

// Per-token record: the token's sequence cache and its position in it.
struct wm_batch_tok {
    int8_t *k, *v;   // codes [layer][max_seq][kv_dim]
    float *ks, *vs;  // scales [layer][max_seq]
    uint32_t max_seq, pos;
};

// Activation layout of the batched I2_S GEMM: per 64-column chunk c (the
// columns one 16-byte weight chunk covers), all tokens' 64 bytes, each
// ordered [dword j of the weight chunk][quarter q][byte g], so that the 16
// bytes one MFMA lane needs for weight dword j are contiguous.
__host__ __device__ __forceinline__ uint64_t wm_gemm_act_offset(uint32_t i, uint32_t t,
                                                                uint32_t m_pad) {
    const uint32_t bk = i >> 7, rem = i & 127u, q = rem >> 5, r32 = rem & 31u;
    const uint32_t half = r32 >> 4, gp = r32 & 15u;
    const uint32_t c = bk * 2 + half, j = gp >> 2, g = gp & 3u;
    return ((uint64_t)c * m_pad + t) * 64 + j * 16 + q * 4 + g;
}

#define WM_GEMM_MAX_DESC 4
#define WM_GEMM_TILE_TOKENS 64
struct wm_gemm_desc {
    const uint8_t *w;   // library I2_S layout
    uint32_t n_groups;  // 64-row groups
    uint32_t out_dim;   // rows written (the tail of the last group is padding)
    uint32_t out_row0;  // first output column of this tensor in y
    float scale;        // per-tensor weight scale
};
// How a GEMM launch is laid out: which kernel (kw: the waves split K), NG
// 64-row groups per workgroup, ST chunks or blocks in flight.
struct wm_gemm_plan {
    bool kw = false;
    int ng = 1, st = 2;
    uint32_t gx = 0, tiles = 0;  // grid: row-group sets x token tiles
};
wm_gemm_plan wm_gemm_make_plan(uint32_t groups, uint32_t n_chunks, uint32_t m);
// y[t * ldy + out_row0 + r] = (scale * meta[t].scale) * (Σ_k code·act - meta[t].asum).
// Returns false (and launches nothing) when the plan has no instantiation.
bool wm_launch_i2s_gemm(const wm_gemm_desc *d, int n_desc, uint32_t n_chunks, const uint8_t *act,
                        uint32_t m, uint32_t m_pad, const wm_act_meta *meta, float *y,
                        uint32_t ldy, hipStream_t s);
// Per-row absmax int8 of x[t * ldx + 0..n) into the GEMM layout + meta[t].
void wm_launch_quantize_rows(const float *x, uint32_t ldx, uint32_t n, uint32_t m, uint32_t m_pad,
                             uint8_t *act, wm_act_meta *meta, hipStream_t s);
// RMSNorm per row.  Source: x[t] (+ res[t], written back to x) or, with gu,
// relu(gu[t][j])^2 * gu[t][n + j].  Output: act/meta (quantised) or y_out.
struct wm_norm_rows {
    float *x; uint32_t ldx;
    const float *res; uint32_t ldr;
    const float *gu; uint32_t ldgu;
    const float *w; uint32_t n; float eps;
    uint8_t *act; uint32_t m_pad; wm_act_meta *meta;
    float *y_out; uint32_t ldo;
    uint32_t *err_flag; uint32_t tag;
};
bool wm_launch_rmsnorm_rows(const wm_norm_rows &a, uint32_t m, hipStream_t s);
// RoPE + K/V append per token of a batch for one layer.
void wm_launch_qkv_rows(const float *y, uint32_t ldy, const float *rope_cos, const float *rope_sin,
                        const wm_batch_tok *tok, uint32_t m, uint32_t layer, uint32_t n_q,
                        uint32_t n_kv, uint32_t head_dim, uint32_t n_rot, float *q_out,
                        hipStream_t s);
// Causal GQA attention of every token of a batch over its own sequence cache.
bool wm_attn_rows_supported(uint32_t head_dim, uint32_t group);
// Work items of the batch attention, one per workgroup: tokens t0 .. t0+nt-1
// of one sequence (nt = 0: nothing to do), positions [p0, p1) (scores) or
// every position below p1 (V), KV head (scores) or KV-head part (V) `unit`.
struct wm_attn_item {
    uint32_t t0, nt, p0, p1, unit, pad;
};
// From the step's tokens (host copy; a sequence's tokens are consecutive):
// scores items per (sequence, KV head, 8 tokens, 256 positions) and V items
// per (sequence, KV-head part, token), ordered so that every item of one
// (sequence, unit) runs on the same XCD.
void wm_attn_rows_plan(const wm_batch_tok *tok, uint32_t m, uint32_t sc_units, uint32_t sv_units,
                       std::vector<wm_attn_item> &sc, std::vector<wm_attn_item> &sv);
// V-kernel units per KV head for a query group size
uint32_t wm_attn_rows_sv_parts(uint32_t group);
// Device workspace of one step: scores, row scales, live-tile flags and the
// n_items work items (wm_attn_rows_items: where the items go).
size_t wm_attn_rows_scores_bytes(uint32_t m, uint32_t n_heads, uint32_t n_max, uint32_t n_items);
wm_attn_item *wm_attn_rows_items(float *scores, uint32_t m, uint32_t n_heads, uint32_t n_max);
void wm_launch_attn_rows(const float *q, const wm_batch_tok *tok, uint32_t m, uint32_t n_max,
                         uint32_t layer, uint32_t n_kv_heads, uint32_t head_dim, uint32_t group,
                         float scale, float *scores, float *out, uint32_t n_sc, uint32_t n_sv,
                         hipStream_t s);
void wm_launch_debug_seq_sum(const float *a, uint32_t n, float *out, hipStream_t s);
