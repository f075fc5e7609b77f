// The allocation-free BitLinear matvec: wm_bitlinear_i2s_matvec_f32_dev
// without any device allocation, for callers that cannot allocate (code
// under HIP graph capture, tight serving loops, harnesses that forbid
// hipMalloc).
//
// Its working memory (the int8 activation codes, their scale and sum, and
// the per-split partial dots) lives in one file-scope device array of
// kScratchBytes per GPU, held until the process ends.  The array's name is
// only a host-side handle: its device address is looked up once per
// context, with the context's device current, when the context is created
// (wm_noalloc_setup, called by wm_ctx_create), and only that address is
// passed to kernels.  Every call on a GPU shares that GPU's array, so calls
// that overlap on one GPU (two streams, two contexts) race; nothing in the
// array has to start at zero (every byte a call reads was written earlier
// in the same call).
#include "wm_internal.h"

namespace wm_noalloc {

constexpr size_t kScratchBytes = size_t(4) << 20;  // 4 MiB per GPU
__device__ __align__(256) uint8_t scratch[kScratchBytes];

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

}  // namespace wm_noalloc

wm_status wm_noalloc_setup(wm_ctx *ctx) {
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(wm_noalloc::scratch));
    if (e != hipSuccess) return wm_hip_error(ctx, e, "hipGetSymbolAddress(scratch)");
    ctx->noalloc_scratch = p;
    return WM_OK;
}

extern "C" wm_status wm_bitlinear_i2s_matvec_f32_dev_noalloc(wm_ctx *ctx, const wm_tensor *w,
                                                            const float *d_input, float *d_output) {
    using namespace wm_noalloc;
    if (!ctx) return WM_E_ARG;
    if (!w || !d_input || !d_output)
        return wm_set_error(ctx, WM_E_ARG, "bitlinear noalloc: null tensor/input/output");
    if (w->ctx != ctx) return wm_set_error(ctx, WM_E_ARG, "bitlinear noalloc: tensor of another context");
    if (w->type != WM_TYPE_I2S)
        return wm_set_error(ctx, WM_E_UNSUPPORTED_TYPE, "bitlinear noalloc: tensor type %d is not I2_S",
                            w->type);
    if (!ctx->noalloc_scratch)
        return wm_set_error(ctx, WM_E_STATE, "bitlinear noalloc: scratch address not set up");
    const uint32_t split = wm_i2s_pick_split(w->n_groups, w->n_chunks);
    const uint32_t rows_total = w->n_groups * I2S_GROUP_ROWS;
    const size_t act_b = align256(w->in_dim), meta_b = 256;
    const size_t need = act_b + meta_b + align256((size_t)split * rows_total * 4);
    if (need > kScratchBytes)
        return wm_set_error(ctx, WM_E_SHAPE,
                            "bitlinear noalloc: [%llu, %llu] needs %zu bytes of scratch, above the %zu-byte limit",
                            (unsigned long long)w->in_dim, (unsigned long long)w->out_dim, need,
                            kScratchBytes);
    WM_HIP(ctx, hipSetDevice(ctx->device));
    uint8_t *base = static_cast<uint8_t *>(ctx->noalloc_scratch);
    uint8_t *act = base;
    wm_act_meta *meta = reinterpret_cast<wm_act_meta *>(base + act_b);
    int32_t *partial = reinterpret_cast<int32_t *>(base + act_b + meta_b);
    wm_launch_quantize_act(d_input, (uint32_t)w->in_dim, act, meta, ctx->stream);
    const wm_i2s_desc desc{static_cast<const uint8_t *>(w->d), w->n_groups};
    wm_launch_i2s_partial(&desc, 1, w->n_chunks, act, partial, split, rows_total, ctx->stream);
    wm_launch_i2s_finalize(partial, split, rows_total, 0, (uint32_t)w->out_dim, w->scale, meta,
                           d_output, nullptr, ctx->stream);
    WM_HIP(ctx, hipGetLastError());
    return WM_OK;
}
