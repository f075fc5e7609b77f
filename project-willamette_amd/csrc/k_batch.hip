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
#include "wm_internal.h"
#include "wm_seqsum.h"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// I2_S x int8 GEMM on MFMA
// ---------------------------------------------------------------------------
//
// One workgroup = one 64-row group of one weight tensor x 64 tokens; wave w
// owns rows 16w..16w+15 and runs four 16x16x64 MFMAs (tokens 0-15, 16-31,
// 32-47, 48-63) per 64-column chunk.  MFMA operands, lane l = 16 * seg + r:
//   A (weights): row r of the wave's 16, dword seg of the row's 16-byte chunk
//                = 16 codes, expanded to one byte each ({0,1,2} = ternary+1);
//   B (activations): token r of the 16, the 16 bytes of the same columns
//                (the GEMM activation layout stores them contiguously);
//   D: lane l holds rows 4*seg .. 4*seg+3 of token r.
// Σ_k (t_k + 1)·a_k - Σ_k a_k = Σ_k t_k·a_k is exact in i32 for any k order.
struct gemm_args {
    wm_gemm_desc d[WM_GEMM_MAX_DESC];
    uint32_t group_end[WM_GEMM_MAX_DESC];
    int n_desc;
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

__global__ __launch_bounds__(256) void k_i2s_gemm(gemm_args a) {
    const uint32_t gid = blockIdx.x;
    // tensor of this group, by selects (no dynamic index into the argument block)
    const uint8_t *w = a.d[0].w;
    uint32_t g0 = 0, row0 = a.d[0].out_row0, out_dim = a.d[0].out_dim;
    float wscale = a.d[0].scale;
#pragma unroll
    for (int i = 1; i < WM_GEMM_MAX_DESC; i++) {
        const bool in = i < a.n_desc && gid >= a.group_end[i - 1];
        w = in ? a.d[i].w : w;
        g0 = in ? a.group_end[i - 1] : g0;
        row0 = in ? a.d[i].out_row0 : row0;
        out_dim = in ? a.d[i].out_dim : out_dim;
        wscale = in ? a.d[i].scale : wscale;
    }
    const uint32_t g = gid - g0;
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const uint32_t r16 = lane & 15, seg = lane >> 4;
    const uint32_t n0 = blockIdx.y * WM_GEMM_TILE_TOKENS;
    const uint8_t *wp = w + (uint64_t)g * a.n_chunks * 1024 + (wave * 16 + r16) * 16 + seg * 4;
    const uint8_t *ap = a.act + (uint64_t)(n0 + r16) * 64 + seg * 16;
    const uint64_t cstride = (uint64_t)a.m_pad * 64;
    v4i acc[4];
#pragma unroll
    for (int s = 0; s < 4; s++) acc[s] = v4i{0, 0, 0, 0};
    uint32_t c = 0;
    for (; c + 4 <= a.n_chunks; c += 4) {
        uint32_t wv[4];
        v4i b[4][4];
#pragma unroll
        for (int u = 0; u < 4; u++) wv[u] = *reinterpret_cast<const uint32_t *>(wp + (uint64_t)(c + u) * 1024);
#pragma unroll
        for (int u = 0; u < 4; u++)
#pragma unroll
            for (int s = 0; s < 4; s++)
                b[u][s] = *reinterpret_cast<const v4i *>(ap + (c + u) * cstride + s * 1024);
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const v4i av = expand_codes(wv[u]);
#pragma unroll
            for (int s = 0; s < 4; s++)
                acc[s] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, b[u][s], acc[s], 0, 0, 0);
        }
    }
    for (; c < a.n_chunks; c++) {
        const uint32_t wv = *reinterpret_cast<const uint32_t *>(wp + (uint64_t)c * 1024);
        v4i b[4];
#pragma unroll
        for (int s = 0; s < 4; s++) b[s] = *reinterpret_cast<const v4i *>(ap + c * cstride + s * 1024);
        const v4i av = expand_codes(wv);
#pragma unroll
        for (int s = 0; s < 4; s++)
            acc[s] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, b[s], acc[s], 0, 0, 0);
    }
    // epilogue: y = (w_scale * act_scale) * (dot as f32)   (bitlinear_sse2.rs:327-339)
    const uint32_t r_local = g * 64 + wave * 16 + seg * 4;
#pragma unroll
    for (int s = 0; s < 4; s++) {
        const uint32_t t = n0 + s * 16 + r16;
        if (t >= a.m) continue;
        const wm_act_meta mt = a.meta[t];
        const float comb = wscale * mt.scale;
        float o[4];
        o[0] = comb * (float)(acc[s].x - mt.asum);
        o[1] = comb * (float)(acc[s].y - mt.asum);
        o[2] = comb * (float)(acc[s].z - mt.asum);
        o[3] = comb * (float)(acc[s].w - mt.asum);
        float *dst = a.y + (uint64_t)t * a.ldy + row0 + r_local;
        if (r_local + 4 <= out_dim && ((row0 | a.ldy) & 3u) == 0) {
            *reinterpret_cast<float4 *>(dst) = make_float4(o[0], o[1], o[2], o[3]);
        } else {
#pragma unroll
            for (int r = 0; r < 4; r++)
                if (r_local + r < out_dim) dst[r] = o[r];
        }
    }
}

// ---------------------------------------------------------------------------
// per-row absmax int8 (bitlinear_sse2.rs:285-304) into the GEMM layout
// ---------------------------------------------------------------------------
constexpr int kRowThreads = 1024;

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
template <int PER, bool GU>
__global__ __launch_bounds__(kRowThreads) void k_rmsnorm_rows(wm_norm_rows a) {
    extern __shared__ __align__(16) float sq[];  // x[j]^2, seq_sum_padded(n) entries
    __shared__ float red_f[16];
    __shared__ int red_i[16];
    __shared__ float s_sum;
    const uint32_t t = blockIdx.x, tid = threadIdx.x, n = a.n;
    float xv[PER], wv[PER];
    int nonfinite = 0;
    if (GU) {
        // relu_square(gate) * up (ffn.rs:37-65)
        const float *g = a.gu + (uint64_t)t * a.ldgu;
        float gv[PER], uv[PER];
#pragma unroll
        for (int i = 0; i < PER; i++) {
            const uint32_t j = min(tid + (uint32_t)i * kRowThreads, n - 1);
            gv[i] = g[j];
            uv[i] = g[n + j];
            wv[i] = a.w[j];
        }
#pragma unroll
        for (int i = 0; i < PER; i++) {
            const float r = gv[i] > 0.0f ? gv[i] : 0.0f;
            xv[i] = (r * r) * uv[i];
        }
    } else {
        float *xr = a.x + (uint64_t)t * a.ldx;
        float rv[PER];
#pragma unroll
        for (int i = 0; i < PER; i++) {
            const uint32_t j = min(tid + (uint32_t)i * kRowThreads, n - 1);
            xv[i] = xr[j];
            wv[i] = a.w[j];
            rv[i] = a.res ? a.res[(uint64_t)t * a.ldr + j] : 0.0f;
        }
        if (a.res) {
            // hidden += BitLinear output (cached_forward.rs:405-408, :496-500)
#pragma unroll
            for (int i = 0; i < PER; i++) {
                const uint32_t j = tid + (uint32_t)i * kRowThreads;
                const float v = xv[i] + rv[i];
                xv[i] = v;
                if (j < n) {
                    xr[j] = v;
                    nonfinite |= !isfinite(v);
                }
            }
        }
    }
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const uint32_t j = tid + (uint32_t)i * kRowThreads;
        if (j < n) sq[j] = xv[i] * xv[i];
        else xv[i] = 0.0f;
    }
    if (a.err_flag) {
        const int any = wm_block_sum_i32(nonfinite, red_i);
        if (any && tid == 0 && *a.err_flag == 0) *a.err_flag = a.tag;
    }
    __syncthreads();
    if (tid < 64) {
        const float s = wm::seq_sum_nonneg(sq, n);
        if (tid == 0) s_sum = s;
    }
    __syncthreads();
    const float mean = s_sum / (float)n;
    const float rs = 1.0f / sqrtf(mean + a.eps);
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
    const float max_abs = wm_block_max_nonan(m, red_f);
    const float inv = 127.0f / max_abs;
    int sum = 0;
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const uint32_t j = tid + (uint32_t)i * kRowThreads;
        if (j < n) {
            const int q = max_abs == 0.0f ? 0 : wm_round_clamp_i8(xv[i] * inv);
            a.act[wm_gemm_act_offset(j, t, a.m_pad)] = (uint8_t)(int8_t)q;
            sum += q;
        }
    }
    sum = wm_block_sum_i32(sum, red_i);
    if (tid == 0) {
        a.meta[t].scale = max_abs == 0.0f ? 1.0f : max_abs / 127.0f;
        a.meta[t].asum = sum;
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
    float *scores;   // [t][n_heads][score_stride]
    float *out;      // [t][n_heads * head_dim]
    uint32_t layer, kv_dim, n_heads, score_stride, n_max;
    float scale;
};

constexpr int kScoreThreads = 256;

template <int HD, int G>
__global__ __launch_bounds__(kScoreThreads) void k_attn_scores_rows(attn_rows_args a) {
    __shared__ float qs[G * HD];
    const uint32_t kvh = blockIdx.y, t = blockIdx.z, tid = threadIdx.x;
    const wm_batch_tok tk = a.tok[t];
    const uint32_t n = tk.pos + 1;
    const uint32_t p0 = blockIdx.x * kScoreThreads;
    if (p0 >= n) return;  // the whole block lies past this token's context
    const float *qsrc = a.q + (uint64_t)t * a.n_heads * HD + (uint64_t)kvh * G * HD;
    for (uint32_t i = tid; i < (uint32_t)(G * HD); i += kScoreThreads) qs[i] = qsrc[i];
    __syncthreads();
    const uint32_t p = p0 + tid;
    if (p >= n) return;
    const uint64_t lay = (uint64_t)a.layer * tk.max_seq;
    const int8_t *kp = tk.k + (lay + p) * a.kv_dim + kvh * HD;
    int4 raw[HD / 16];
#pragma unroll
    for (int b = 0; b < HD / 16; b++) raw[b] = *reinterpret_cast<const int4 *>(kp + b * 16);
    const float kscale = tk.ks[lay + p];
    float s[G];
#pragma unroll
    for (int h = 0; h < G; h++) s[h] = 0.0f;
#pragma unroll
    for (int b = 0; b < HD / 16; b++) {
        const uint32_t wd[4] = {(uint32_t)raw[b].x, (uint32_t)raw[b].y, (uint32_t)raw[b].z,
                                (uint32_t)raw[b].w};
#pragma unroll
        for (int e = 0; e < 16; e++) {
            const float kd = (float)(int8_t)(wd[e >> 2] >> (8 * (e & 3))) * kscale;  // read_into
#pragma unroll
            for (int h = 0; h < G; h++) s[h] = s[h] + qs[h * HD + b * 16 + e] * kd;
        }
    }
    float *dst = a.scores + ((uint64_t)t * a.n_heads + kvh * G) * a.score_stride + p;
#pragma unroll
    for (int h = 0; h < G; h++) dst[(uint64_t)h * a.score_stride] = s[h] * a.scale;
}

constexpr int kVTile = 64;  // V rows per LDS tile

template <int HD>
__global__ __launch_bounds__(HD) void k_attn_softmax_v_rows(attn_rows_args a) {
    // LDS: weights [seq_sum_padded(n_max)] | V tile [kVTile][HD] bytes | V scales [kVTile]
    extern __shared__ __align__(16) float wts[];
    __shared__ uint64_t exp_tab[32];
    __shared__ float red[2];
    __shared__ float s_inv;
    __shared__ int s_mode;
    const uint32_t h = blockIdx.x, t = blockIdx.y, tid = threadIdx.x;
    const uint32_t group = a.n_heads / (a.kv_dim / HD), kvh = h / group;
    const wm_batch_tok tk = a.tok[t];
    const uint32_t n = tk.pos + 1;
    int8_t *vt = reinterpret_cast<int8_t *>(wts + wm::seq_sum_padded(a.n_max));
    float *st = reinterpret_cast<float *>(vt + kVTile * HD);
    const float *sc = a.scores + ((uint64_t)t * a.n_heads + h) * a.score_stride;
    if (tid < 32) exp_tab[tid] = wm::kExp2Tab[tid];
    float m = -INFINITY;
    for (uint32_t p = tid; p < n; p += HD) {
        const float v = sc[p];
        wts[p] = v;
        m = wm_max_nonan(m, v);
    }
    m = wm_wave_max_nonan(m);
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    const float mx = HD > 64 ? wm_max_nonan(red[0], red[1]) : red[0];
    float *out = a.out + (uint64_t)t * a.n_heads * HD + (uint64_t)h * HD;
    if (!isfinite(mx)) {  // every weight is 0 or NaN: the output stays 0
        out[tid] = 0.0f;
        return;
    }
    for (uint32_t p = tid; p < n; p += HD) wts[p] = wm::expf_glibc(wts[p] - mx, exp_tab);
    __syncthreads();
    if (tid < 64) {
        const float sum = wm::seq_sum_nonneg(wts, n);
        if (tid == 0) {
            s_mode = sum > 0.0f;
            s_inv = 1.0f / sum;
        }
    }
    __syncthreads();
    if (s_mode) {
        const float inv = s_inv;
        for (uint32_t p = tid; p < n; p += HD) wts[p] = wts[p] * inv;
    }
    // V rows of this KV head go through LDS a tile at a time: every thread
    // loads 16-byte pieces (all in flight together, the next tile's while the
    // current one is consumed), then thread d runs its chain from LDS.
    const uint64_t lay = (uint64_t)a.layer * tk.max_seq;
    const int8_t *vg = tk.v + lay * a.kv_dim + kvh * HD;
    const float *vsg = tk.vs + lay;
    // Tile rows p0 .. p0+63, indices clamped to n-1 so every load is in range
    // and unconditional: thread tid takes 16-byte pieces tid, tid+HD, tid+2HD,
    // tid+3HD (piece = row * HD/16 + column) and threads < 64 one scale each.
    constexpr uint32_t kPR = HD / 16;  // pieces per row
    const uint32_t r0 = tid / kPR, c0 = (tid % kPR) * 16, rstep = HD / kPR;
    int4 pre0, pre1, pre2, pre3;
    float spre = 0.0f;
#define WM_FETCH_V(P0)                                                                       \
    do {                                                                                     \
        const uint32_t q0 = (P0) + r0;                                                       \
        pre0 = *reinterpret_cast<const int4 *>(vg + (uint64_t)min(q0, n - 1) * a.kv_dim + c0); \
        pre1 = *reinterpret_cast<const int4 *>(vg + (uint64_t)min(q0 + rstep, n - 1) * a.kv_dim + c0); \
        pre2 = *reinterpret_cast<const int4 *>(vg + (uint64_t)min(q0 + 2 * rstep, n - 1) * a.kv_dim + c0); \
        pre3 = *reinterpret_cast<const int4 *>(vg + (uint64_t)min(q0 + 3 * rstep, n - 1) * a.kv_dim + c0); \
        if (tid < (uint32_t)kVTile) spre = vsg[min((P0) + tid, n - 1)];                       \
    } while (0)
    WM_FETCH_V(0u);
    float acc = 0.0f;
    for (uint32_t p0 = 0; p0 < n; p0 += kVTile) {
        __syncthreads();  // previous tile consumed (and, first time, the weights written)
        int4 *vt4 = reinterpret_cast<int4 *>(vt);
        vt4[tid] = pre0;
        vt4[tid + HD] = pre1;
        vt4[tid + 2 * HD] = pre2;
        vt4[tid + 3 * HD] = pre3;
        if (tid < (uint32_t)kVTile) st[tid] = spre;
        __syncthreads();
        WM_FETCH_V(p0 + kVTile);  // next tile; past the end the clamped rows re-read row n-1
        const uint32_t tn = n - p0 < (uint32_t)kVTile ? n - p0 : (uint32_t)kVTile;
        const float *wp = wts + p0;
        for (uint32_t q = 0; q < tn; q++)
            acc = acc + wp[q] * ((float)vt[q * HD + tid] * st[q]);  // w * (q8 * scale)
    }
    out[tid] = acc;
#undef WM_FETCH_V
}

}  // namespace

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------

void wm_launch_i2s_gemm(const wm_gemm_desc *d, int n_desc, uint32_t n_chunks, const uint8_t *act,
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
    a.n_chunks = n_chunks;
    a.act = act;
    a.m = m;
    a.m_pad = m_pad;
    a.meta = meta;
    a.y = y;
    a.ldy = ldy;
    const uint32_t tiles = (m + WM_GEMM_TILE_TOKENS - 1) / WM_GEMM_TILE_TOKENS;
    hipLaunchKernelGGL(k_i2s_gemm, dim3(groups, tiles), dim3(256), 0, s, a);
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

size_t wm_attn_rows_scores_bytes(uint32_t m, uint32_t n_heads, uint32_t n_max) {
    return (size_t)m * n_heads * ((n_max + 3u) & ~3u) * sizeof(float);
}

void wm_launch_attn_rows(const float *q, const wm_batch_tok *tok, uint32_t m, uint32_t n_max,
                         uint32_t layer, uint32_t n_kv_heads, uint32_t head_dim, uint32_t group,
                         float scale, float *scores, float *out, hipStream_t s) {
    const uint32_t n_heads = n_kv_heads * group;
    attn_rows_args a{q, tok, scores, out, layer, n_kv_heads * head_dim, n_heads,
                     (n_max + 3u) & ~3u, n_max, scale};
    const dim3 sgrid((n_max + kScoreThreads - 1) / kScoreThreads, n_kv_heads, m);
#define WM_SCORES_CASE(HD, G)                                                                  \
    if (head_dim == HD && group == G)                                                          \
        hipLaunchKernelGGL((k_attn_scores_rows<HD, G>), sgrid, dim3(kScoreThreads), 0, s, a);
    WM_SCORES_CASE(128, 1) WM_SCORES_CASE(128, 2) WM_SCORES_CASE(128, 4) WM_SCORES_CASE(128, 8)
    WM_SCORES_CASE(64, 1) WM_SCORES_CASE(64, 2) WM_SCORES_CASE(64, 4) WM_SCORES_CASE(64, 8)
#undef WM_SCORES_CASE
    const size_t lds = (size_t)wm::seq_sum_padded(n_max) * sizeof(float) +
                       (size_t)kVTile * head_dim + kVTile * sizeof(float);
    if (head_dim == 128)
        hipLaunchKernelGGL(k_attn_softmax_v_rows<128>, dim3(n_heads, m), dim3(128), lds, s, a);
    else
        hipLaunchKernelGGL(k_attn_softmax_v_rows<64>, dim3(n_heads, m), dim3(64), lds, s, a);
}
