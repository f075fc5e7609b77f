// Exact, wave-parallel evaluation of a left-to-right f32 sum.
//
// The reference accumulates non-negative terms one at a time,
//     s = 0; for a in x { s += a }            (Σx² of rms_norm_f32,
//                                              the softmax denominator)
// with one round-to-nearest-even per step.  That order fixes the result's
// last bits, and a later int8 quantisation turns a last-bit difference into
// a different token, so the device must produce exactly this value.  Doing
// the adds one by one costs ~30 cycles per term (each step waits on the
// previous one); this routine produces the same bits with one wave working
// on 512 terms at a time:
//
//   While s stays inside one binade [2^E, 2^(E+1)) with ulp u = 2^(E-23),
//   s = N*u for an integer N in [2^23, 2^24), and
//       RN(N*u + a) = (N + RN_int(a/u)) * u
//   as long as a/u is not exactly halfway between integers (then the
//   round-half-even choice depends on N's parity) and N + a/u stays below
//   2^24 - 1/2 (past that the result rounds into the next binade, where the
//   ulp doubles).  The increment RN_int(a/u) then does not depend on s, so a
//   run of such terms is summed exactly with integer prefix sums.  The first
//   term that breaks either condition (a tie, a crossing, a huge or
//   non-finite term) ends the run: the run's prefix is accepted, that one
//   term is added with an ordinary f32 add, and scanning resumes after it.
//
// a/u is computed as ldexp(a, 23 - E): exact whenever the result is a
// normal float; when it is not, a/u < 2^-126 and the term rounds away
// (increment 0, never a tie), which the code also concludes.
//
// Called by all 64 lanes of one wave with the terms in LDS (or any memory
// readable by every lane); returns the sum in every lane.  Non-negative
// terms make every step an increase, so only upward crossings occur.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace wm {

// Inclusive prefix sum over the 64 lanes of a wave (rows of 16 via DPP
// row_shr, then the three row totals via readlane).
__device__ __forceinline__ int wave_incl_scan_i32(int x) {
    x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false);  // row_shr:1
    x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false);  // row_shr:2
    x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false);  // row_shr:4
    x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false);  // row_shr:8
    const int row = (int)(threadIdx.x & 63) >> 4;
    const int t0 = __builtin_amdgcn_readlane(x, 15);
    const int t1 = __builtin_amdgcn_readlane(x, 31);
    const int t2 = __builtin_amdgcn_readlane(x, 47);
    x += (row >= 1 ? t0 : 0) + (row >= 2 ? t1 : 0) + (row >= 3 ? t2 : 0);
    return x;
}

// Terms handled per wave step (8 per lane).
constexpr uint32_t kSeqBatch = 512;
constexpr int kSeqLead = 128;  // leading terms added one by one
__host__ __device__ constexpr uint32_t seq_sum_padded(uint32_t n) {
    return (n + kSeqBatch - 1) / kSeqBatch * kSeqBatch;
}

// Sequential f32 sum of n non-negative terms a[0..n) (as s += a[i]), by one
// wave (all 64 lanes call it; the sum comes back in every lane).
// Negative terms are not allowed (the caller's terms are squares or exp()).
//
// Per step the wave holds 512 terms in registers.  The run test works from
// s's own bits: a normal s is N * 2^(E-23) with N its 24-bit significand and
// a term's increment is RN_int(ldexp(a, 23 - E)).  The same test covers the
// other values of s through the shift alone: while s is +0 or subnormal the
// shift is +255, so every non-zero term overflows the run limit and is added
// on its own (zero terms leave s unchanged); while s is +inf it is -255, so
// finite terms add nothing and only NaN or inf terms are added on their own.
// A NaN s absorbs everything.  Terms already added are zeroed in the
// registers and the same registers are rescanned with the new s, so no term
// is loaded twice.  The first kSeqLead terms, which move s through many
// binades and (while s is small) hold most of the halfway cases, are added
// one at a time straight from the registers.
// Continues the sum from s (itself a left-to-right sum of earlier terms,
// so s >= +0 or NaN); a needs no alignment and is read only below n.
__device__ inline float seq_sum_nonneg_from(float s, const float *a, uint32_t n) {
    const uint32_t lane = threadIdx.x & 63;
    for (uint32_t k = 0; k < n; k += kSeqBatch) {
        const uint32_t base = k + 8 * lane;
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; j++) v[j] = base + j < n ? a[base + j] : 0.0f;
        if (k == 0) {
            // terms 0..127 sit in lanes 0-15; adding the zeros past n changes nothing
#pragma unroll
            for (int L = 0; L < kSeqLead / 8; L++)
#pragma unroll
                for (int j = 0; j < 8; j++)
                    s = s + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v[j]), L));
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = lane < kSeqLead / 8 ? 0.0f : v[j];
        }
        // Each restart zeroes at least one non-zero term, so a step ends after
        // at most 513 passes; the bound is explicit all the same.
        for (uint32_t pass = 0; pass <= kSeqBatch; pass++) {
            if (s != s) return s;
            const uint32_t bits = __float_as_uint(s);  // s >= +0
            const uint32_t ef = bits >> 23;
            const bool normal = ef - 1u < 254u;
            const int sh = normal ? 150 - (int)ef : (ef == 0 ? 255 : -255);
            const int N = normal ? (int)((bits & 0x7fffffu) | 0x800000u) : 0;
            int p[8], rho[8];
            bool bad[8];
            int run = 0;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const float r = ldexpf(v[j], sh);    // a / ulp(s); exact unless < 2^-126
                const bool fin = r < 0x1p22f;         // false for NaN, inf, huge
                const float rr = fin ? r : 0.0f;
                bad[j] = !fin || rr - floorf(rr) == 0.5f;  // halfway: parity decides
                rho[j] = (int)rintf(rr);
                run += rho[j];
                p[j] = run;
            }
            const int incl = wave_incl_scan_i32(run);
            const int excl = incl - run;
            const int limit = (1 << 24) - 1 - N;  // N + prefix must stay below 2^24 - 1
            int first = 8, before = 0;
#pragma unroll
            for (int j = 7; j >= 0; j--) {
                // A term with increment 0 leaves N + prefix where it was, so it
                // never crosses; hence offenders are never zero terms (a zero
                // term is neither bad nor crossing), and every restart below
                // consumes a non-zero term.
                const bool off = bad[j] || (rho[j] > 0 && excl + p[j] >= limit);
                first = off ? j : first;
                before = off ? excl + (j ? p[j - 1] : 0) : before;
            }
            const uint64_t mask = __ballot(first < 8);
            if (mask == 0) {
                if (normal) s = ldexpf((float)(N + __builtin_amdgcn_readlane(incl, 63)), -sh);
                break;
            }
            const int fl = __ffsll((unsigned long long)mask) - 1;
            const int jl = __builtin_amdgcn_readlane(first, fl);
            const int pre = __builtin_amdgcn_readlane(before, fl);
            float vo = v[0];
#pragma unroll
            for (int j = 1; j < 8; j++) vo = j == jl ? v[j] : vo;
            vo = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(vo), fl));
            if (normal) s = ldexpf((float)(N + pre), -sh);  // the run before the offender
            s = s + vo;                                      // the offender, by an ordinary add
            const uint32_t done = 8 * (uint32_t)fl + (uint32_t)jl;  // last term now in s
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = 8 * lane + j <= done ? 0.0f : v[j];
        }
    }
    return s;
}

__device__ inline float seq_sum_nonneg(const float *a, uint32_t n) {
    return seq_sum_nonneg_from(0.0f, a, n);
}

// ---------------------------------------------------------------------------
// The same sum by a whole workgroup.
//
// The one-wave algorithm spends its time on passes: every binade crossing and
// every halfway case restarts a 512-term scan.  Here the work that does not
// depend on the running value is done once, by every thread in parallel, and
// only a short sequential walk remains:
//
//  1. A float64 prefix sum P_k (sum of the terms before k) predicts the binade
//     E of the f32 running sum before term k.  (The f32 sum differs from P_k
//     by accumulated rounding, far less than the distance to a power of two
//     for almost every k; every prediction is checked in step 3.)
//  2. Term k is a break if k = 0, if P_k is not positive, if the predicted
//     binade changes at k, if a_k / ulp is halfway between integers (the
//     rounding then depends on the running significand's parity) or if it is
//     huge or not finite.  Every other term contributes the integer increment
//     RN_int(a_k / ulp(E)).  A block-wide integer prefix scan gives every
//     segment between two breaks its total increment D.
//  3. One wave walks the breaks in order.  For a segment it checks that the
//     running sum s (exact so far) is a normal number in the predicted binade
//     with significand N and N + D <= 2^24 - 2; then, as in the one-wave
//     algorithm, s + (the segment, added term by term) = (N + D) * ulp
//     exactly.  A break term is added with an ordinary f32 add.  A segment
//     whose check fails is summed by the one-wave algorithm from s instead,
//     so every outcome is the left-to-right sum.
//
// With the squares of an RMSNorm (2560 or 6912 terms) a sum has about 18
// breaks and a failed prediction in well under 1% of sums.  More than
// kSeqRecords breaks (adversarial inputs) send the whole sum to the one-wave
// algorithm.
constexpr int kSeqRecords = 512;

struct seq_block_scratch {
    double dw[16];
    long long iw[16];
    int idx[kSeqRecords];
    int eaf[kSeqRecords];
    long long pi[kSeqRecords];
    float val[kSeqRecords];
    long long total;
    float out;
};

__device__ __forceinline__ double wave_incl_scan_f64(double x) {
    const int lane = (int)(threadIdx.x & 63);
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const double y = __shfl_up(x, o, 64);
        if (lane >= o) x += y;
    }
    return x;
}
__device__ __forceinline__ long long wave_incl_scan_i64(long long x) {
    const int lane = (int)(threadIdx.x & 63);
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const long long y = __shfl_up(x, o, 64);
        if (lane >= o) x += y;
    }
    return x;
}
// floor(log2 x) of a positive, finite, normal double
__device__ __forceinline__ int exp2floor_f64(double x) {
    return (int)((__double_as_longlong(x) >> 52) & 0x7FF) - 1023;
}

// Left-to-right f32 sum of n non-negative terms a[0..n) (LDS), by every
// thread of the workgroup (blockDim.x a multiple of 64, at most 1024); the
// sum comes back in every thread.  MAXM >= ceil(n / blockDim.x).
template <int MAXM>
__device__ float seq_sum_block_nonneg(const float *a, uint32_t n, seq_block_scratch *sc) {
    const uint32_t tid = threadIdx.x, nt = blockDim.x, lane = tid & 63, wid = tid >> 6;
    if (n == 0) return 0.0f;
    const uint32_t m = (n + nt - 1) / nt;
    const uint32_t k0 = tid * m;
    float v[MAXM];
    double loc = 0.0;
#pragma unroll
    for (int j = 0; j < MAXM; j++) {
        const uint32_t k = k0 + (uint32_t)j;
        v[j] = ((uint32_t)j < m && k < n) ? a[k] : 0.0f;
        loc += (double)v[j];
    }
    // 1. P before this thread's first term
    const double inc = wave_incl_scan_f64(loc);
    if (lane == 63) sc->dw[wid] = inc;
    __syncthreads();
    double P = inc - loc;
    for (uint32_t w = 0; w < wid; w++) P += sc->dw[w];
    // 2. breaks and increments
    bool brk[MAXM];
    int incr[MAXM], eaf[MAXM];
    long long pi_loc = 0;
    int nb = 0;
#pragma unroll
    for (int j = 0; j < MAXM; j++) {
        const uint32_t k = k0 + (uint32_t)j;
        const bool valid = (uint32_t)j < m && k < n;
        const double pb = P, pa = P + (double)v[j];
        P = pa;
        const bool pb_ok = pb > 0.0 && pb < 1e300, pa_ok = pa > 0.0 && pa < 1e300;
        const int eb = pb_ok ? exp2floor_f64(pb) : 0;
        const int ea = pa_ok ? exp2floor_f64(pa) : -1000;
        bool b = k == 0 || !pb_ok || !pa_ok || ea != eb;
        int d = 0;
        if (!b) {
            const float r = ldexpf(v[j], 23 - eb);  // a_k / ulp; exact unless < 2^-126
            b = !(r < 0x1p22f) || r - floorf(r) == 0.5f;
            d = b ? 0 : (int)rintf(r);
        }
        brk[j] = valid && b;
        incr[j] = valid ? d : 0;
        eaf[j] = ea;
        nb += brk[j] ? 1 : 0;
        pi_loc += incr[j];
    }
    // block-wide exclusive scan of (break count << 48) + increment sum
    const long long packed = ((long long)nb << 48) + pi_loc;
    const long long pinc = wave_incl_scan_i64(packed);
    if (lane == 63) sc->iw[wid] = pinc;
    __syncthreads();
    long long pex = pinc - packed;
    for (uint32_t w = 0; w < wid; w++) pex += sc->iw[w];
    if (tid == nt - 1) sc->total = pex + packed;
    int pos = (int)(pex >> 48);
    long long pi = pex & ((1LL << 48) - 1);
#pragma unroll
    for (int j = 0; j < MAXM; j++) {
        if (brk[j]) {
            if (pos < kSeqRecords) {
                sc->idx[pos] = (int)(k0 + (uint32_t)j);
                sc->eaf[pos] = eaf[j];
                sc->pi[pos] = pi;
                sc->val[pos] = v[j];
            }
            pos++;
        } else {
            pi += incr[j];
        }
    }
    __syncthreads();
    // 3. the walk over the breaks (one wave)
    if (wid == 0) {
        const long long tot = sc->total;
        const int nbrk = (int)(tot >> 48);
        const long long pi_tot = tot & ((1LL << 48) - 1);
        float s = 0.0f;
        if (nbrk > kSeqRecords) {
            s = seq_sum_nonneg_from(0.0f, a, n);
        } else {
            int prev_t = -1, e_seg = -1000;
            long long prev_pi = 0;
            // records 0..nbrk-1 and a final one at index n closing the last segment
            for (int base = 0; base <= nbrk; base += 64) {
                const int r = base + (int)lane;
                int ri = (int)n, re = 0;
                long long rp = pi_tot;
                float rv = 0.0f;
                if (r < nbrk) {
                    ri = sc->idx[r];
                    re = sc->eaf[r];
                    rp = sc->pi[r];
                    rv = sc->val[r];
                }
                const int here = min(64, nbrk + 1 - base);
                for (int i = 0; i < here; i++) {
                    const int t = __builtin_amdgcn_readlane(ri, i);
                    const int rpi_lo = __builtin_amdgcn_readlane((int)(rp & 0xFFFFFFFF), i);
                    const int rpi_hi = __builtin_amdgcn_readlane((int)(rp >> 32), i);
                    const long long tpi = ((long long)rpi_hi << 32) | (unsigned int)rpi_lo;
                    const int cnt = t - prev_t - 1;
                    if (cnt > 0) {
                        const long long d = tpi - prev_pi;
                        const uint32_t bits = __float_as_uint(s);
                        const uint32_t ef = bits >> 23;  // s >= +0 or NaN
                        const long long N = (long long)((bits & 0x7FFFFFu) | 0x800000u);
                        const bool ok = ef - 1u < 254u && (int)ef - 127 == e_seg && d >= 0 &&
                                        N + d <= (1LL << 24) - 2;
                        if (ok) s = ldexpf((float)(N + d), e_seg - 23);
                        else s = seq_sum_nonneg_from(s, a + prev_t + 1, (uint32_t)cnt);
                    }
                    if (t < (int)n) {
                        s = s + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(rv), i));
                        e_seg = __builtin_amdgcn_readlane(re, i);
                    }
                    prev_t = t;
                    prev_pi = tpi;
                }
            }
        }
        if (lane == 0) sc->out = s;
    }
    __syncthreads();
    return sc->out;
}

}  // namespace wm
