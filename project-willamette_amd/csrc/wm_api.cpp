// C ABI: context, device buffers, tensors, BitLinear and Q6_K entry points.
#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <vector>

#include "wm_internal.h"

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

// ---------------------------------------------------------------------------
// errors
// ---------------------------------------------------------------------------
wm_status wm_set_error(wm_ctx *ctx, wm_status st, const char *fmt, ...) {
    if (ctx) {
        char buf[512];
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(buf, sizeof(buf), fmt, ap);
        va_end(ap);
        ctx->last_error = buf;
    }
    return st;
}

wm_status wm_hip_error(wm_ctx *ctx, hipError_t e, const char *what) {
    if (e == hipErrorOutOfMemory)
        return wm_set_error(ctx, WM_E_OOM, "%s: %s", what, hipGetErrorString(e));
    return wm_set_error(ctx, WM_E_HIP, "%s: %s", what, hipGetErrorString(e));
}

wm_status wm_ctx_scratch(wm_ctx *ctx, size_t bytes, void **out) {
    if (ctx->scratch_bytes < bytes) {
        if (ctx->scratch) WM_HIP(ctx, hipFree(ctx->scratch));
        ctx->scratch = nullptr;
        ctx->scratch_bytes = 0;
        size_t cap = bytes < (1u << 20) ? (1u << 20) : bytes;
        WM_HIP(ctx, hipMalloc(&ctx->scratch, cap));
        ctx->scratch_bytes = cap;
    }
    *out = ctx->scratch;
    return WM_OK;
}

wm_status wm_ctx_pinned(wm_ctx *ctx, size_t bytes, void **out) {
    if (ctx->pinned_bytes < bytes) {
        if (ctx->pinned) WM_HIP(ctx, hipHostFree(ctx->pinned));
        ctx->pinned = nullptr;
        ctx->pinned_bytes = 0;
        size_t cap = bytes < (1u << 20) ? (1u << 20) : bytes;
        WM_HIP(ctx, hipHostMalloc(&ctx->pinned, cap, hipHostMallocDefault));
        ctx->pinned_bytes = cap;
    }
    *out = ctx->pinned;
    return WM_OK;
}

// ---------------------------------------------------------------------------
// context
// ---------------------------------------------------------------------------
extern "C" {

const char *wm_version(void) { return "willamette-hip 0.1 (gfx950)"; }

wm_status wm_ctx_create(int device, wm_ctx **out) {
    if (!out) return WM_E_ARG;
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return WM_E_HIP;
    if (device < 0 || device >= n) return WM_E_ARG;
    if (hipSetDevice(device) != hipSuccess) return WM_E_HIP;
    wm_ctx *c = new wm_ctx();
    c->device = device;
    if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
        delete c;
        return WM_E_HIP;
    }
    if (wm_noalloc_setup(c) != WM_OK) {
        hipStreamDestroy(c->stream);
        delete c;
        return WM_E_HIP;
    }
    *out = c;
    return WM_OK;
}

void wm_ctx_destroy(wm_ctx *ctx) {
    if (!ctx) return;
    hipSetDevice(ctx->device);
    hipStreamSynchronize(ctx->stream);
    if (ctx->scratch) hipFree(ctx->scratch);
    if (ctx->multi_dev) hipFree(ctx->multi_dev);
    if (ctx->pinned) hipHostFree(ctx->pinned);
    hipStreamDestroy(ctx->stream);
    delete ctx;
}

const char *wm_last_error(const wm_ctx *ctx) { return ctx ? ctx->last_error.c_str() : ""; }

void *wm_ctx_stream(wm_ctx *ctx) { return ctx ? (void *)ctx->stream : nullptr; }

wm_status wm_ctx_synchronize(wm_ctx *ctx) {
    if (!ctx) return WM_E_ARG;
    WM_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return WM_OK;
}

wm_status wm_dev_alloc(wm_ctx *ctx, size_t bytes, void **out) {
    if (!ctx || !out) return WM_E_ARG;
    *out = nullptr;
    WM_HIP(ctx, hipSetDevice(ctx->device));
    WM_HIP(ctx, hipMalloc(out, bytes ? bytes : 1));
    return WM_OK;
}

wm_status wm_dev_free(wm_ctx *ctx, void *ptr) {
    if (!ctx) return WM_E_ARG;
    if (ptr) {
        WM_HIP(ctx, hipStreamSynchronize(ctx->stream));
        WM_HIP(ctx, hipFree(ptr));
    }
    return WM_OK;
}

wm_status wm_memcpy_h2d(wm_ctx *ctx, void *dst, const void *src, size_t bytes) {
    if (!ctx || (!dst && bytes) || (!src && bytes)) return WM_E_ARG;
    WM_HIP(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
    WM_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return WM_OK;
}

wm_status wm_memcpy_d2h(wm_ctx *ctx, void *dst, const void *src, size_t bytes) {
    if (!ctx || (!dst && bytes) || (!src && bytes)) return WM_E_ARG;
    WM_HIP(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
    WM_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return WM_OK;
}

// ---------------------------------------------------------------------------
// tensors
// ---------------------------------------------------------------------------

wm_status wm_tensor_upload_i2s(wm_ctx *ctx, const uint8_t *packed, size_t packed_len,
                               const uint8_t *scale_block, size_t scale_len, uint64_t in_dim,
                               uint64_t out_dim, wm_tensor **out) {
    if (!ctx || !out) return WM_E_ARG;
    *out = nullptr;
    // src/model/bitlinear_sse2.rs:129-177 and src/gguf/tensor.rs:278-309
    if (in_dim == 0 || in_dim % QK_I2S)
        return wm_set_error(ctx, WM_E_SHAPE,
                            "bitlinear: in_dim %llu is not a positive multiple of %d",
                            (unsigned long long)in_dim, QK_I2S);
    if (out_dim == 0 || out_dim > (1ull << 30) || in_dim > (1ull << 24))
        return wm_set_error(ctx, WM_E_SHAPE, "bitlinear: unsupported shape [%llu, %llu]",
                            (unsigned long long)in_dim, (unsigned long long)out_dim);
    uint64_t expected = in_dim / 4 * out_dim;
    if (!packed || packed_len < expected)
        return wm_set_error(ctx, WM_E_SHAPE, "bitlinear: data.len()=%zu < %llu (in_dim/4 x out_dim)",
                            packed_len, (unsigned long long)expected);
    if (!scale_block || scale_len < 4)
        return wm_set_error(ctx, WM_E_SHAPE, "i2s_scale: scale_data missing or shorter than 4 bytes");
    float scale;
    std::memcpy(&scale, scale_block, 4);
    if (!std::isfinite(scale))
        return wm_set_error(ctx, WM_E_NONFINITE, "i2s_scale: non-finite scale (%g)", (double)scale);
    WM_HIP(ctx, hipSetDevice(ctx->device));
    wm_tensor *t = new wm_tensor();
    t->ctx = ctx;
    t->device = ctx->device;
    t->type = WM_TYPE_I2S;
    t->in_dim = in_dim;
    t->out_dim = out_dim;
    t->scale = scale;
    t->n_groups = (uint32_t)((out_dim + I2S_GROUP_ROWS - 1) / I2S_GROUP_ROWS);
    t->n_chunks = (uint32_t)(in_dim / I2S_CHUNK_COLS);
    t->bytes = (size_t)t->n_groups * t->n_chunks * I2S_GROUP_ROWS * 16;
    void *raw = nullptr;
    hipError_t e = hipMalloc(&t->d, t->bytes);
    if (e == hipSuccess) e = hipMalloc(&raw, expected);
    if (e == hipSuccess) e = hipMemcpyAsync(raw, packed, expected, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess) {
        wm_launch_i2s_repack((const uint8_t *)raw, (uint8_t *)t->d, (uint32_t)in_dim,
                             (uint32_t)out_dim, t->n_groups, ctx->stream);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (raw) hipFree(raw);
    if (e != hipSuccess) {
        if (t->d) hipFree(t->d);
        delete t;
        return wm_hip_error(ctx, e, "wm_tensor_upload_i2s");
    }
    *out = t;
    return WM_OK;
}

wm_status wm_tensor_upload_q6k(wm_ctx *ctx, const uint8_t *blocks, size_t len, uint64_t row_len,
                               uint64_t n_rows, wm_tensor **out) {
    if (!ctx || !out) return WM_E_ARG;
    *out = nullptr;
    if (row_len == 0 || row_len % Q6K_VALUES || row_len > 65536)
        return wm_set_error(ctx, WM_E_SHAPE, "Q6_K value count %llu is not a multiple of 256",
                            (unsigned long long)row_len);
    if (n_rows == 0 || n_rows > (1ull << 28))
        return wm_set_error(ctx, WM_E_SHAPE, "Q6_K: unsupported row count %llu",
                            (unsigned long long)n_rows);
    uint64_t expected = n_rows * (row_len / Q6K_VALUES) * Q6K_BYTES;
    if (!blocks || len != expected)
        return wm_set_error(ctx, WM_E_SHAPE, "Q6_K tensor has %zu bytes, expected %llu", len,
                            (unsigned long long)expected);
    WM_HIP(ctx, hipSetDevice(ctx->device));
    wm_tensor *t = new wm_tensor();
    t->ctx = ctx;
    t->device = ctx->device;
    t->type = WM_TYPE_Q6K;
    t->in_dim = row_len;
    t->out_dim = n_rows;
    t->n_blocks = (uint32_t)(row_len / Q6K_VALUES);
    t->n_rowgroups = (uint32_t)((n_rows + Q6K_GROUP_ROWS - 1) / Q6K_GROUP_ROWS);
    t->bytes = wm_q6k_sigma_offset(t->n_rowgroups, t->n_blocks) + (size_t)n_rows * 4;
    void *raw = nullptr;
    hipError_t e = hipMalloc(&t->d, t->bytes);
    if (e == hipSuccess) e = hipMalloc(&raw, expected);
    if (e == hipSuccess) e = hipMemcpyAsync(raw, blocks, expected, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess) {
        wm_launch_q6k_repack((const uint8_t *)raw, (uint8_t *)t->d, (uint32_t)n_rows, t->n_blocks,
                             t->n_rowgroups, ctx->stream);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (raw) hipFree(raw);
    if (e != hipSuccess) {
        if (t->d) hipFree(t->d);
        delete t;
        return wm_hip_error(ctx, e, "wm_tensor_upload_q6k");
    }
    *out = t;
    return WM_OK;
}

void wm_tensor_destroy(wm_tensor *t) {
    if (!t) return;
    if (t->d) {
        hipSetDevice(t->device);
        hipFree(t->d);
    }
    delete t;
}

wm_status wm_tensor_info(const wm_tensor *t, uint64_t shape[2], int *type, float *scale) {
    if (!t) return WM_E_ARG;
    if (shape) {
        shape[0] = t->in_dim;
        shape[1] = t->out_dim;
    }
    if (type) *type = t->type;
    if (scale) *scale = t->scale;
    return WM_OK;
}

// ---------------------------------------------------------------------------
// BitLinear
// ---------------------------------------------------------------------------

static wm_status check_i2s(wm_ctx *ctx, const wm_tensor *w) {
    if (!ctx || !w) return WM_E_ARG;
    if (w->type != WM_TYPE_I2S)
        return wm_set_error(ctx, WM_E_UNSUPPORTED_TYPE, "bitlinear: tensor type %d is not I2_S",
                            w->type);
    if (w->ctx != ctx) return wm_set_error(ctx, WM_E_ARG, "bitlinear: tensor of another context");
    return WM_OK;
}

// Device workspace for one matvec: act (in_dim bytes, 16-aligned), meta,
// partials (split x rows).
struct mv_ws {
    uint8_t *act;
    wm_act_meta *meta;
    int32_t *partial;
    float *x, *y;
    int32_t *dot;
};


// One launch where the shape allows (k_i2s_matvec_one, in_dim <= 16384),
// else the quantiser, the split partial dots and their sum.  The codes and
// the quantiser's scale land in act and meta when want_codes (the other
// path always writes them).
static void run_matvec(wm_ctx *ctx, const wm_tensor *w, const float *d_x, float *d_y,
                       int32_t *d_dot, uint8_t *act, wm_act_meta *meta, int32_t *partial,
                       bool want_codes) {
    if (wm_launch_i2s_matvec_one((const uint8_t *)w->d, w->n_groups, w->n_chunks, (uint32_t)w->out_dim,
                                 w->scale, d_x, d_y, d_dot, want_codes ? act : nullptr,
                                 want_codes ? meta : nullptr, ctx->stream))
        return;
    uint32_t split = wm_i2s_pick_split(w->n_groups, w->n_chunks);
    uint32_t rows_total = w->n_groups * I2S_GROUP_ROWS;
    wm_launch_quantize_act(d_x, (uint32_t)w->in_dim, act, meta, ctx->stream);
    wm_i2s_desc desc{(const uint8_t *)w->d, w->n_groups};
    wm_launch_i2s_partial(&desc, 1, w->n_chunks, act, partial, split, rows_total, ctx->stream);
    wm_launch_i2s_finalize(partial, split, rows_total, 0, (uint32_t)w->out_dim, w->scale, meta, d_y,
                           d_dot, ctx->stream);
}

static size_t matvec_ws_bytes(const wm_tensor *w) {
    uint32_t split = wm_i2s_pick_split(w->n_groups, w->n_chunks);
    return align256(w->in_dim) + 256 + align256((size_t)split * w->n_groups * I2S_GROUP_ROWS * 4);
}

wm_status wm_bitlinear_i2s_matvec_f32_debug(wm_ctx *ctx, const wm_tensor *w, const float *input,
                                            size_t input_len, float *output, size_t output_len,
                                            int8_t *act_out, float *act_scale, int32_t *acc_out) {
    wm_status st = check_i2s(ctx, w);
    if (st) return st;
    if (!input || !output) return wm_set_error(ctx, WM_E_ARG, "bitlinear: null input/output");
    if (input_len != w->in_dim)
        return wm_set_error(ctx, WM_E_SHAPE, "bitlinear: input.len()=%zu != in_dim=%llu", input_len,
                            (unsigned long long)w->in_dim);
    if (output_len != w->out_dim)
        return wm_set_error(ctx, WM_E_SHAPE, "bitlinear: output.len()=%zu != out_dim=%llu",
                            output_len, (unsigned long long)w->out_dim);
    WM_HIP(ctx, hipSetDevice(ctx->device));
    const size_t in_b = align256(w->in_dim * 4), out_b = align256(w->out_dim * 4);
    const size_t ws_b = matvec_ws_bytes(w);
    void *scratch;
    if ((st = wm_ctx_scratch(ctx, in_b + 2 * out_b + ws_b, &scratch))) return st;
    uint8_t *base = (uint8_t *)scratch;
    float *d_x = (float *)base;
    float *d_y = (float *)(base + in_b);
    int32_t *d_dot = (int32_t *)(base + in_b + out_b);
    uint8_t *act = base + in_b + 2 * out_b;
    wm_act_meta *meta = (wm_act_meta *)(act + align256(w->in_dim));
    int32_t *partial = (int32_t *)((uint8_t *)meta + 256);
    WM_HIP(ctx, hipMemcpyAsync(d_x, input, w->in_dim * 4, hipMemcpyHostToDevice, ctx->stream));
    run_matvec(ctx, w, d_x, d_y, d_dot, act, meta, partial, act_out || act_scale);
    WM_HIP(ctx, hipGetLastError());
    WM_HIP(ctx, hipMemcpyAsync(output, d_y, w->out_dim * 4, hipMemcpyDeviceToHost, ctx->stream));
    if (acc_out)
        WM_HIP(ctx, hipMemcpyAsync(acc_out, d_dot, w->out_dim * 4, hipMemcpyDeviceToHost, ctx->stream));
    std::vector<uint8_t> act_perm;
    wm_act_meta meta_h{};
    if (act_out) {
        act_perm.resize(w->in_dim);
        WM_HIP(ctx, hipMemcpyAsync(act_perm.data(), act, w->in_dim, hipMemcpyDeviceToHost, ctx->stream));
    }
    if (act_scale)
        WM_HIP(ctx, hipMemcpyAsync(&meta_h, meta, sizeof(meta_h), hipMemcpyDeviceToHost, ctx->stream));
    WM_HIP(ctx, hipStreamSynchronize(ctx->stream));
    if (act_out)
        for (uint32_t i = 0; i < w->in_dim; i++) act_out[i] = (int8_t)act_perm[wm_act_perm(i)];
    if (act_scale) *act_scale = meta_h.scale;
    return WM_OK;
}

wm_status wm_bitlinear_i2s_matvec_f32(wm_ctx *ctx, const wm_tensor *w, const float *input,
                                      size_t input_len, float *output, size_t output_len) {
    return wm_bitlinear_i2s_matvec_f32_debug(ctx, w, input, input_len, output, output_len, nullptr,
                                             nullptr, nullptr);
}

wm_status wm_bitlinear_i2s_matvec_f32_scalar_dev(wm_ctx *ctx, const wm_tensor *w,
                                                 const float *d_input, float *d_output) {
    wm_status st = check_i2s(ctx, w);
    if (st) return st;
    if (!d_input || !d_output) return wm_set_error(ctx, WM_E_ARG, "bitlinear scalar: null input/output");
    WM_HIP(ctx, hipSetDevice(ctx->device));
    wm_launch_i2s_scalar_f32((const uint8_t *)w->d, w->n_groups, w->n_chunks, (uint32_t)w->out_dim,
                             w->scale, d_input, d_output, ctx->stream);
    WM_HIP(ctx, hipGetLastError());
    return WM_OK;
}

wm_status wm_bitlinear_i2s_matvec_f32_scalar(wm_ctx *ctx, const wm_tensor *w, const float *input,
                                             size_t input_len, float *output, size_t output_len) {
    wm_status st = check_i2s(ctx, w);
    if (st) return st;
    if (!input || !output) return wm_set_error(ctx, WM_E_ARG, "bitlinear scalar: null input/output");
    if (input_len != w->in_dim)
        return wm_set_error(ctx, WM_E_SHAPE, "bitlinear_i2s_matvec_f32: input.len()=%zu != in_dim=%llu",
                            input_len, (unsigned long long)w->in_dim);
    if (output_len != w->out_dim)
        return wm_set_error(ctx, WM_E_SHAPE, "bitlinear_i2s_matvec_f32: output.len()=%zu != out_dim=%llu",
                            output_len, (unsigned long long)w->out_dim);
    WM_HIP(ctx, hipSetDevice(ctx->device));
    const size_t in_b = align256(w->in_dim * 4);
    void *scratch;
    if ((st = wm_ctx_scratch(ctx, in_b + align256(w->out_dim * 4), &scratch))) return st;
    float *d_x = (float *)scratch;
    float *d_y = (float *)((uint8_t *)scratch + in_b);
    WM_HIP(ctx, hipMemcpyAsync(d_x, input, w->in_dim * 4, hipMemcpyHostToDevice, ctx->stream));
    if ((st = wm_bitlinear_i2s_matvec_f32_scalar_dev(ctx, w, d_x, d_y))) return st;
    WM_HIP(ctx, hipMemcpyAsync(output, d_y, w->out_dim * 4, hipMemcpyDeviceToHost, ctx->stream));
    WM_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return WM_OK;
}

wm_status wm_bitlinear_i2s_matvec_f32_dev(wm_ctx *ctx, const wm_tensor *w, const float *d_input,
                                          float *d_output) {
    // one tensor: its pointer and scale go in the kernels' arguments (the
    // multi-copy path keeps a device table, uploaded again whenever the
    // tensors change, which for a caller stepping through layers is every call)
    if (!ctx || !w || !d_input || !d_output) return WM_E_ARG;
    wm_status st = check_i2s(ctx, w);
    if (st) return st;
    void *scratch;
    if ((st = wm_ctx_scratch(ctx, matvec_ws_bytes(w), &scratch))) return st;
    uint8_t *act = (uint8_t *)scratch;
    wm_act_meta *meta = (wm_act_meta *)(act + align256(w->in_dim));
    int32_t *partial = (int32_t *)((uint8_t *)meta + 256);
    WM_HIP(ctx, hipSetDevice(ctx->device));
    run_matvec(ctx, w, d_input, d_output, nullptr, act, meta, partial, false);
    WM_HIP(ctx, hipGetLastError());
    return WM_OK;
}

wm_status wm_debug_set_fused_flags(wm_ctx *ctx, uint32_t flags) {
    if (!ctx) return WM_E_ARG;
    const uint32_t known = WM_FUSED_DEBUG_SKEW_SMALL | WM_FUSED_DEBUG_SKEW_LARGE | WM_FUSED_DEBUG_NO_CANDIDATES |
                           WM_FUSED_DEBUG_ATTN_NO_WAIT | WM_FUSED_DEBUG_ATTN_LOOSE_COUNT;
    if (flags & ~known) return wm_set_error(ctx, WM_E_ARG, "set_fused_flags: unknown bits 0x%x", flags & ~known);
    ctx->fused_debug = flags;
    return WM_OK;
}

// ---------------------------------------------------------------------------
// FFN block (ffn_block_forward, src/model/ffn.rs:73-136)
// ---------------------------------------------------------------------------

// The shapes the block needs: gate and up [n_embd -> n_ff], down [n_ff ->
// n_embd], all I2_S of this context.  n_embd and n_ff come from gate.
static wm_status check_ffn(wm_ctx *ctx, const wm_tensor *gate, const wm_tensor *up,
                           const wm_tensor *down) {
    wm_status st;
    if ((st = check_i2s(ctx, gate)) || (st = check_i2s(ctx, up)) || (st = check_i2s(ctx, down)))
        return st;
    const uint64_t E = gate->in_dim, F = gate->out_dim;
    if (up->in_dim != E || up->out_dim != F)
        return wm_set_error(ctx, WM_E_SHAPE, "ffn_block_forward: ffn_up shape [%llu, %llu] != [%llu, %llu]",
                            (unsigned long long)up->in_dim, (unsigned long long)up->out_dim,
                            (unsigned long long)E, (unsigned long long)F);
    if (down->in_dim != F || down->out_dim != E)
        return wm_set_error(ctx, WM_E_SHAPE,
                            "ffn_block_forward: ffn_down shape [%llu, %llu] != [%llu, %llu]",
                            (unsigned long long)down->in_dim, (unsigned long long)down->out_dim,
                            (unsigned long long)F, (unsigned long long)E);
    return WM_OK;
}

// Two launches: ffn_norm + gate and up (each workgroup evaluates the norm
// and its int8 codes itself), then relu(gate)^2 * up + ffn_sub_norm + down.
// gu: 2 * n_ff floats of device scratch for the gate and up outputs.
static wm_status run_ffn(wm_ctx *ctx, const float *d_x, const float *d_norm_w, const wm_tensor *gate,
                         const wm_tensor *up, const wm_tensor *down, const float *d_sub_w, float eps,
                         float *d_out, float *gu) {
    const uint32_t F = (uint32_t)gate->out_dim;
    wm_fused_norm fn{};
    fn.debug = ctx->fused_debug;
    fn.x = d_x;
    fn.w = d_norm_w;
    fn.eps = eps;
    const wm_i2s_desc gud[2] = {{(const uint8_t *)gate->d, gate->n_groups},
                                {(const uint8_t *)up->d, up->n_groups}};
    const float gus[2] = {gate->scale, up->scale};
    float *guo[2] = {gu, gu + F};
    wm_fused_norm dn{};
    dn.debug = ctx->fused_debug;
    dn.x = gu;
    dn.y = gu + F;
    dn.relu2_mul = 1;
    dn.w = d_sub_w;
    dn.eps = eps;
    const wm_i2s_desc dd = {(const uint8_t *)down->d, down->n_groups};
    float *dout[1] = {d_out};
    if (!wm_launch_i2s_fused(WM_FUSED_PLAIN, gud, gus, guo, 2, gate->n_chunks, 1, fn, nullptr, nullptr,
                             0, 0, 0, nullptr, ctx->stream) ||
        !wm_launch_i2s_fused(WM_FUSED_PLAIN, &dd, &down->scale, dout, 1, down->n_chunks, 1, dn, nullptr,
                             nullptr, 0, 0, 0, nullptr, ctx->stream))
        return wm_set_error(ctx, WM_E_SHAPE, "ffn_block_forward: no kernel for n_embd %llu, n_ff %llu",
                            (unsigned long long)gate->in_dim, (unsigned long long)F);
    WM_HIP(ctx, hipGetLastError());
    return WM_OK;
}

wm_status wm_ffn_block_forward_dev(wm_ctx *ctx, const float *d_x, const float *d_ffn_norm_weight,
                                   const wm_tensor *gate, const wm_tensor *up, const wm_tensor *down,
                                   const float *d_ffn_sub_norm_weight, float eps, float *d_output) {
    if (!ctx || !d_x || !d_ffn_norm_weight || !d_ffn_sub_norm_weight || !d_output) return WM_E_ARG;
    wm_status st = check_ffn(ctx, gate, up, down);
    if (st) return st;
    void *scratch;
    if ((st = wm_ctx_scratch(ctx, align256(gate->out_dim * 8), &scratch))) return st;
    WM_HIP(ctx, hipSetDevice(ctx->device));
    return run_ffn(ctx, d_x, d_ffn_norm_weight, gate, up, down, d_ffn_sub_norm_weight, eps, d_output,
                   (float *)scratch);
}

wm_status wm_ffn_block_forward(wm_ctx *ctx, const float *x, size_t x_len, const float *ffn_norm_weight,
                               size_t ffn_norm_len, const wm_tensor *gate, const wm_tensor *up,
                               const wm_tensor *down, const float *ffn_sub_norm_weight,
                               size_t ffn_sub_norm_len, float eps, float *output, size_t output_len) {
    if (!ctx || !x || !ffn_norm_weight || !ffn_sub_norm_weight || !output) return WM_E_ARG;
    wm_status st = check_ffn(ctx, gate, up, down);
    if (st) return st;
    const uint64_t E = gate->in_dim, F = gate->out_dim;
    // the reference's checks, in its order (ffn.rs:87-114)
    if (x_len != E)
        return wm_set_error(ctx, WM_E_SHAPE, "ffn_block_forward: x.len()=%zu != n_embd=%llu", x_len,
                            (unsigned long long)E);
    if (ffn_norm_len != E)
        return wm_set_error(ctx, WM_E_SHAPE, "ffn_block_forward: ffn_norm_weight.len()=%zu != n_embd=%llu",
                            ffn_norm_len, (unsigned long long)E);
    if (ffn_sub_norm_len != F)
        return wm_set_error(ctx, WM_E_SHAPE,
                            "ffn_block_forward: ffn_sub_norm_weight.len()=%zu != n_ff=%llu",
                            ffn_sub_norm_len, (unsigned long long)F);
    if (output_len != E)
        return wm_set_error(ctx, WM_E_SHAPE, "ffn_block_forward: output.len()=%zu != n_embd=%llu",
                            output_len, (unsigned long long)E);
    WM_HIP(ctx, hipSetDevice(ctx->device));
    const size_t eb = align256(E * 4), fb = align256(F * 4);
    void *scratch;
    if ((st = wm_ctx_scratch(ctx, 3 * eb + 3 * fb, &scratch))) return st;
    uint8_t *b = (uint8_t *)scratch;
    float *d_x = (float *)b, *d_nw = (float *)(b + eb), *d_out = (float *)(b + 2 * eb);
    float *d_sw = (float *)(b + 3 * eb), *gu = (float *)(b + 3 * eb + fb);
    WM_HIP(ctx, hipMemcpyAsync(d_x, x, E * 4, hipMemcpyHostToDevice, ctx->stream));
    WM_HIP(ctx, hipMemcpyAsync(d_nw, ffn_norm_weight, E * 4, hipMemcpyHostToDevice, ctx->stream));
    WM_HIP(ctx, hipMemcpyAsync(d_sw, ffn_sub_norm_weight, F * 4, hipMemcpyHostToDevice, ctx->stream));
    if ((st = run_ffn(ctx, d_x, d_nw, gate, up, down, d_sw, eps, d_out, gu))) return st;
    WM_HIP(ctx, hipMemcpyAsync(output, d_out, E * 4, hipMemcpyDeviceToHost, ctx->stream));
    WM_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return WM_OK;
}

wm_status wm_bitlinear_i2s_matvec_f32_multi_dev(wm_ctx *ctx, const wm_tensor *const *ws,
                                                uint32_t n_copies, const float *d_input,
                                                float *d_outputs) {
    if (!ctx || !ws || !n_copies || !d_input || !d_outputs) return WM_E_ARG;
    wm_status st;
    for (uint32_t i = 0; i < n_copies; i++) {
        if ((st = check_i2s(ctx, ws[i]))) return st;
        if (ws[i]->in_dim != ws[0]->in_dim || ws[i]->out_dim != ws[0]->out_dim)
            return wm_set_error(ctx, WM_E_SHAPE, "bitlinear multi: tensors differ in shape");
    }
    const wm_tensor *w0 = ws[0];
    const uint32_t per = w0->n_groups;
    // one launch over every copy: the weight pointers in a device table.  The
    // K split only until ~8K single-wave workgroups exist: a wave streaming a
    // whole row group keeps its load pipeline full (320 copies of 2560x2560:
    // 6.0 TB/s unsplit, 5.6 at split 2)
    uint32_t split = (8192 + per * n_copies - 1) / (per * n_copies);
    const uint32_t max_split = w0->n_chunks / 4 ? w0->n_chunks / 4 : 1;
    split = split > max_split ? max_split : split;
    split = split > 16 ? 16 : (split < 1 ? 1 : split);
    const size_t rows_total = (size_t)per * n_copies * I2S_GROUP_ROWS;
    const size_t need = align256(w0->in_dim) + 256 + align256((size_t)split * rows_total * 4);
    void *scratch;
    if ((st = wm_ctx_scratch(ctx, need, &scratch))) return st;
    uint8_t *act = (uint8_t *)scratch;
    wm_act_meta *meta = (wm_act_meta *)(act + align256(w0->in_dim));
    int32_t *partial = (int32_t *)((uint8_t *)meta + 256);
    WM_HIP(ctx, hipSetDevice(ctx->device));
    // weight pointers and scales on the device: kept from the last call when unchanged
    std::vector<const void *> hp(n_copies);
    std::vector<float> hs(n_copies);
    for (uint32_t i = 0; i < n_copies; i++) {
        hp[i] = ws[i]->d;
        hs[i] = ws[i]->scale;
    }
    const size_t tbytes = align256((size_t)n_copies * 8) + align256((size_t)n_copies * 4);
    if (hp != ctx->multi_ptrs || hs != ctx->multi_scales) {
        if (ctx->multi_bytes < tbytes) {
            if (ctx->multi_dev) WM_HIP(ctx, hipFree(ctx->multi_dev));
            ctx->multi_dev = nullptr;
            ctx->multi_bytes = 0;
            WM_HIP(ctx, hipMalloc(&ctx->multi_dev, tbytes));
            ctx->multi_bytes = tbytes;
        }
        // pageable host sources: the runtime stages them before the calls return
        WM_HIP(ctx, hipMemcpyAsync(ctx->multi_dev, hp.data(), n_copies * 8, hipMemcpyHostToDevice,
                                   ctx->stream));
        WM_HIP(ctx, hipMemcpyAsync((uint8_t *)ctx->multi_dev + align256((size_t)n_copies * 8),
                                   hs.data(), n_copies * 4, hipMemcpyHostToDevice, ctx->stream));
        ctx->multi_ptrs = hp;
        ctx->multi_scales = hs;
    }
    const uint8_t *const *table = (const uint8_t *const *)ctx->multi_dev;
    const float *scales = (const float *)((uint8_t *)ctx->multi_dev + align256((size_t)n_copies * 8));
    wm_launch_quantize_act(d_input, (uint32_t)w0->in_dim, act, meta, ctx->stream);
    wm_launch_i2s_partial_table(table, n_copies, per, w0->n_chunks, act, partial, split,
                                (uint32_t)rows_total, ctx->stream);
    wm_launch_i2s_finalize_multi(partial, split, (uint32_t)rows_total, per * I2S_GROUP_ROWS,
                                 (uint32_t)w0->out_dim, n_copies, scales, meta, d_outputs,
                                 ctx->stream);
    WM_HIP(ctx, hipGetLastError());
    return WM_OK;
}

wm_status wm_bitlinear_i2s_matmul_f32_dev(wm_ctx *ctx, const wm_tensor *w, const float *d_x,
                                          uint32_t m, float *d_y) {
    wm_status st = check_i2s(ctx, w);
    if (st) return st;
    if (!d_x || !d_y || m == 0) return wm_set_error(ctx, WM_E_ARG, "bitlinear matmul: empty batch");
    const uint32_t m_pad = (m + WM_GEMM_TILE_TOKENS - 1) / WM_GEMM_TILE_TOKENS * WM_GEMM_TILE_TOKENS;
    const size_t act_bytes = align256((size_t)w->in_dim * m_pad);
    void *scratch;
    if ((st = wm_ctx_scratch(ctx, act_bytes + align256((size_t)m * sizeof(wm_act_meta)), &scratch)))
        return st;
    uint8_t *act = (uint8_t *)scratch;
    wm_act_meta *meta = (wm_act_meta *)(act + act_bytes);
    WM_HIP(ctx, hipSetDevice(ctx->device));
    wm_launch_quantize_rows(d_x, (uint32_t)w->in_dim, (uint32_t)w->in_dim, m, m_pad, act, meta,
                            ctx->stream);
    wm_gemm_desc d{(const uint8_t *)w->d, w->n_groups, (uint32_t)w->out_dim, 0, w->scale};
    if (!wm_launch_i2s_gemm(&d, 1, w->n_chunks, act, m, m_pad, meta, d_y, (uint32_t)w->out_dim,
                            ctx->stream))
        return wm_set_error(ctx, WM_E_SHAPE, "bitlinear matmul: no GEMM kernel for this shape");
    WM_HIP(ctx, hipGetLastError());
    return WM_OK;
}

wm_status wm_bitlinear_i2s_matmul_f32(wm_ctx *ctx, const wm_tensor *w, const float *x,
                                      size_t x_len, uint32_t m, float *y, size_t y_len) {
    wm_status st = check_i2s(ctx, w);
    if (st) return st;
    if (!x || !y || m == 0) return wm_set_error(ctx, WM_E_ARG, "bitlinear matmul: empty batch");
    if (x_len != (size_t)m * w->in_dim)
        return wm_set_error(ctx, WM_E_SHAPE, "bitlinear_i2s_matmul: input.len()=%zu != %u x in_dim=%llu",
                            x_len, m, (unsigned long long)w->in_dim);
    if (y_len != (size_t)m * w->out_dim)
        return wm_set_error(ctx, WM_E_SHAPE, "bitlinear_i2s_matmul: output.len()=%zu != %u x out_dim=%llu",
                            y_len, m, (unsigned long long)w->out_dim);
    WM_HIP(ctx, hipSetDevice(ctx->device));
    void *dx = nullptr, *dy = nullptr;
    WM_HIP(ctx, hipMalloc(&dx, x_len * 4));
    hipError_t e = hipMalloc(&dy, y_len * 4);
    if (e == hipSuccess) e = hipMemcpyAsync(dx, x, x_len * 4, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess) {
        st = wm_bitlinear_i2s_matmul_f32_dev(ctx, w, (const float *)dx, m, (float *)dy);
        if (st == WM_OK) e = hipMemcpyAsync(y, dy, y_len * 4, hipMemcpyDeviceToHost, ctx->stream);
        if (st == WM_OK && e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    }
    hipFree(dx);
    if (dy) hipFree(dy);
    if (e != hipSuccess) return wm_hip_error(ctx, e, "bitlinear_i2s_matmul");
    return st;
}

// ---------------------------------------------------------------------------
// Q6_K
// ---------------------------------------------------------------------------

static wm_status check_q6k(wm_ctx *ctx, const wm_tensor *t) {
    if (!ctx || !t) return WM_E_ARG;
    if (t->type != WM_TYPE_Q6K)
        return wm_set_error(ctx, WM_E_UNSUPPORTED_TYPE, "Q6_K: tensor type %d is not Q6_K", t->type);
    if (t->ctx != ctx) return wm_set_error(ctx, WM_E_ARG, "Q6_K: tensor of another context");
    return WM_OK;
}

// The lm-head kernels stage one row's worth of the hidden vector in LDS.
static wm_status check_lm_head(wm_ctx *ctx, const wm_tensor *t) {
    wm_status st = check_q6k(ctx, t);
    if (st) return st;
    if (t->n_blocks > WM_Q6K_LOGITS_MAX_BLOCKS || t->out_dim > WM_Q6K_LOGITS_MAX_ROWS)
        return wm_set_error(ctx, WM_E_SHAPE,
                            "compute_logits: lm-head [%llu, %llu] above the supported [%u, %u]",
                            (unsigned long long)t->in_dim, (unsigned long long)t->out_dim,
                            WM_Q6K_LOGITS_MAX_BLOCKS * Q6K_VALUES, WM_Q6K_LOGITS_MAX_ROWS);
    return WM_OK;
}

wm_status wm_q6k_dequantize_row(wm_ctx *ctx, const wm_tensor *t, uint64_t row, float *out,
                                size_t out_len) {
    wm_status st = check_q6k(ctx, t);
    if (st) return st;
    if (!out) return WM_E_ARG;
    if (out_len != t->in_dim)
        return wm_set_error(ctx, WM_E_SHAPE, "embedding_gather: out.len()=%zu != n_embd=%llu",
                            out_len, (unsigned long long)t->in_dim);
    if (row >= t->out_dim)
        return wm_set_error(ctx, WM_E_SHAPE, "embedding_gather: token_id %llu out of range (vocab_size=%llu)",
                            (unsigned long long)row, (unsigned long long)t->out_dim);
    void *scratch;
    if ((st = wm_ctx_scratch(ctx, t->in_dim * 4, &scratch))) return st;
    WM_HIP(ctx, hipSetDevice(ctx->device));
    wm_launch_q6k_dequant_row((const uint8_t *)t->d, t->n_blocks, (uint32_t)row, (float *)scratch,
                              ctx->stream);
    WM_HIP(ctx, hipGetLastError());
    WM_HIP(ctx, hipMemcpyAsync(out, scratch, t->in_dim * 4, hipMemcpyDeviceToHost, ctx->stream));
    WM_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return WM_OK;
}

wm_status wm_logits_argmax_dev(wm_ctx *ctx, const wm_tensor *t, const float *d_hidden,
                               float *d_logits, uint32_t *d_argmax) {
    wm_status st = check_lm_head(ctx, t);
    if (st) return st;
    if (!d_hidden || (!d_logits && !d_argmax)) return WM_E_ARG;
    const size_t lb = align256(t->out_dim * 4);
    const size_t wb = wm_q6k_logits_work_bytes((uint32_t)t->out_dim, t->n_blocks);
    void *scratch;
    if ((st = wm_ctx_scratch(ctx, lb + wb, &scratch))) return st;
    void *work = (uint8_t *)scratch + lb;
    WM_HIP(ctx, hipSetDevice(ctx->device));
    if (d_logits)
        wm_launch_q6k_logits_argmax((const uint8_t *)t->d, t->n_blocks, (uint32_t)t->out_dim,
                                    t->n_rowgroups, d_hidden, d_logits, d_argmax, work, ctx->stream);
    else
        wm_launch_q6k_argmax_fast((const uint8_t *)t->d, t->n_blocks, (uint32_t)t->out_dim,
                                  t->n_rowgroups, d_hidden, (float *)scratch, d_argmax, work,
                                  false, ctx->stream);
    WM_HIP(ctx, hipGetLastError());
    return WM_OK;
}

wm_status wm_logits_argmax(wm_ctx *ctx, const wm_tensor *t, const float *hidden,
                           size_t hidden_len, float *logits, uint32_t *argmax) {
    wm_status st = check_lm_head(ctx, t);
    if (st) return st;
    if (!hidden || (!logits && !argmax)) return WM_E_ARG;
    if (hidden_len != t->in_dim)
        return wm_set_error(ctx, WM_E_SHAPE, "compute_logits: final_hidden.len()=%zu != embedding_length=%llu",
                            hidden_len, (unsigned long long)t->in_dim);
    const size_t hb = align256(t->in_dim * 4), lb = align256(t->out_dim * 4);
    const size_t need = hb + lb + 256 + wm_q6k_logits_work_bytes((uint32_t)t->out_dim, t->n_blocks);
    void *scratch;
    if ((st = wm_ctx_scratch(ctx, need, &scratch))) return st;
    uint8_t *base = (uint8_t *)scratch;
    float *d_h = (float *)base;
    float *d_l = (float *)(base + hb);
    uint32_t *d_a = (uint32_t *)(base + hb + lb);
    void *work = base + hb + lb + 256;
    WM_HIP(ctx, hipSetDevice(ctx->device));
    WM_HIP(ctx, hipMemcpyAsync(d_h, hidden, t->in_dim * 4, hipMemcpyHostToDevice, ctx->stream));
    // Logits wanted: every row in the reference's exact order.  Only the id
    // wanted: the bounded pass plus exact rescoring of the rows that can win.
    if (logits)
        wm_launch_q6k_logits_argmax((const uint8_t *)t->d, t->n_blocks, (uint32_t)t->out_dim,
                                    t->n_rowgroups, d_h, d_l, d_a, work, ctx->stream);
    else
        wm_launch_q6k_argmax_fast((const uint8_t *)t->d, t->n_blocks, (uint32_t)t->out_dim,
                                  t->n_rowgroups, d_h, d_l, d_a, work, false, ctx->stream);
    WM_HIP(ctx, hipGetLastError());
    if (logits)
        WM_HIP(ctx, hipMemcpyAsync(logits, d_l, t->out_dim * 4, hipMemcpyDeviceToHost, ctx->stream));
    uint32_t a = 0;
    WM_HIP(ctx, hipMemcpyAsync(&a, d_a, 4, hipMemcpyDeviceToHost, ctx->stream));
    WM_HIP(ctx, hipStreamSynchronize(ctx->stream));
    if (argmax) *argmax = a;
    return WM_OK;
}

wm_status wm_debug_q6k_bounded_logits_dev(wm_ctx *ctx, const wm_tensor *t, const float *d_hidden,
                                          float *d_approx, float *d_bound, int reuse_prep) {
    wm_status st = check_lm_head(ctx, t);
    if (st) return st;
    if (!d_hidden || !d_approx || !d_bound) return WM_E_ARG;
    void *work;
    if ((st = wm_ctx_scratch(ctx, wm_q6k_logits_work_bytes((uint32_t)t->out_dim, t->n_blocks), &work)))
        return st;
    WM_HIP(ctx, hipSetDevice(ctx->device));
    wm_launch_q6k_bounded_only((const uint8_t *)t->d, t->n_blocks, (uint32_t)t->out_dim,
                               t->n_rowgroups, d_hidden, d_approx, d_bound, work, reuse_prep != 0,
                               ctx->stream);
    WM_HIP(ctx, hipGetLastError());
    return WM_OK;
}

wm_status wm_debug_q6k_bounded_logits(wm_ctx *ctx, const wm_tensor *t, const float *hidden,
                                      size_t hidden_len, float *approx, float *bound) {
    wm_status st = check_lm_head(ctx, t);
    if (st) return st;
    if (!hidden || !approx || !bound) return WM_E_ARG;
    if (hidden_len != t->in_dim)
        return wm_set_error(ctx, WM_E_SHAPE, "compute_logits: final_hidden.len()=%zu != embedding_length=%llu",
                            hidden_len, (unsigned long long)t->in_dim);
    const size_t hb = align256(t->in_dim * 4), lb = align256(t->out_dim * 4);
    const size_t need = hb + 2 * lb + wm_q6k_logits_work_bytes((uint32_t)t->out_dim, t->n_blocks);
    void *scratch;
    if ((st = wm_ctx_scratch(ctx, need, &scratch))) return st;
    uint8_t *base = (uint8_t *)scratch;
    float *d_h = (float *)base, *d_a = (float *)(base + hb), *d_b = (float *)(base + hb + lb);
    WM_HIP(ctx, hipSetDevice(ctx->device));
    WM_HIP(ctx, hipMemcpyAsync(d_h, hidden, t->in_dim * 4, hipMemcpyHostToDevice, ctx->stream));
    wm_launch_q6k_bounded_only((const uint8_t *)t->d, t->n_blocks, (uint32_t)t->out_dim,
                               t->n_rowgroups, d_h, d_a, d_b, base + hb + 2 * lb, false, ctx->stream);
    WM_HIP(ctx, hipGetLastError());
    WM_HIP(ctx, hipMemcpyAsync(approx, d_a, t->out_dim * 4, hipMemcpyDeviceToHost, ctx->stream));
    WM_HIP(ctx, hipMemcpyAsync(bound, d_b, t->out_dim * 4, hipMemcpyDeviceToHost, ctx->stream));
    WM_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return WM_OK;
}

wm_status wm_compute_logits(wm_ctx *ctx, const wm_tensor *t, const float *hidden,
                            size_t hidden_len, float *logits, size_t vocab) {
    wm_status st = check_q6k(ctx, t);
    if (st) return st;
    if (!logits) return WM_E_ARG;
    if (vocab != t->out_dim)
        return wm_set_error(ctx, WM_E_SHAPE, "compute_logits: vocab %zu != %llu", vocab,
                            (unsigned long long)t->out_dim);
    return wm_logits_argmax(ctx, t, hidden, hidden_len, logits, nullptr);
}

wm_status wm_debug_seq_sum(wm_ctx *ctx, const float *values, size_t n, float *sum) {
    if (!ctx || !sum || (n && !values) || n > (1u << 26)) return WM_E_ARG;
    // terms padded to whole 512-term steps (read, never used)
    const size_t padded = (n + 511) / 512 * 512;
    void *scratch;
    wm_status st = wm_ctx_scratch(ctx, padded * 4 + 256, &scratch);
    if (st) return st;
    float *d_in = (float *)scratch, *d_out = (float *)((uint8_t *)scratch + padded * 4);
    WM_HIP(ctx, hipSetDevice(ctx->device));
    if (n) WM_HIP(ctx, hipMemcpyAsync(d_in, values, n * 4, hipMemcpyHostToDevice, ctx->stream));
    wm_launch_debug_seq_sum(d_in, (uint32_t)n, d_out, ctx->stream);
    WM_HIP(ctx, hipGetLastError());
    WM_HIP(ctx, hipMemcpyAsync(sum, d_out, 4, hipMemcpyDeviceToHost, ctx->stream));
    WM_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return WM_OK;
}

wm_status wm_argmax(const float *logits, size_t n, uint32_t *out) {
    if (!logits || !out || n == 0) return WM_E_ARG;
    size_t best = 0;
    float bv = logits[0];
    for (size_t i = 1; i < n; i++)
        if (logits[i] > bv) {
            bv = logits[i];
            best = i;
        }
    *out = (uint32_t)best;
    return WM_OK;
}

}  // extern "C"
