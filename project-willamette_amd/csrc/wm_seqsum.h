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

#include "wm_internal.h"

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

// lane l - 1's value of x; lane 0 gets `first`
__device__ __forceinline__ int wave_shr1(int x, int first) {
    return __builtin_amdgcn_update_dpp(first, x, 0x138, 0xF, 0xF, false);  // wave_shr:1
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
// One step: adds the 512 terms v (lane l holding terms 8l .. 8l+7 of the
// step, 0 past the end) to s, which the step's first terms follow; `lead`
// on the sum's first step.  v is consumed.  Every lane gets the same s.
//
// PARITY: halfway terms do not end a run.  Round-half-even takes a halfway
// term a/u = k + 1/2 to the even one of N + k and N + k + 1, so its increment
// is k + ((N + k) & 1) and the significand after it is even; the parity of
// N before any term is therefore that of the increments since the last
// halfway term (or since the run's start, plus N's own).  A segmented scan
// of those parities over the wave (segments start at halfway terms) gives
// every term its increment at once, and a run ends only at a crossing or a
// huge or non-finite term.  For inputs with many halfway terms (squares of
// values with few significant bits); without it, each one is a restart.
template <bool PARITY = false>
__device__ inline float seq_sum_step(float s, float (&v)[8], bool lead) {
    const uint32_t lane = threadIdx.x & 63;
    if (lead) {
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
        if (!PARITY) {
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const float r = ldexpf(v[j], sh);    // a / ulp(s); exact unless < 2^-126
                const bool fin = r < 0x1p22f;         // false for NaN, inf, huge
                const float rr = fin ? r : 0.0f;
                bad[j] = !fin || rr - floorf(rr) == 0.5f;  // halfway: parity decides
                rho[j] = (int)rintf(rr);
            }
        } else {
            bool half[8];
            // the lane's parity summary: bit 1 = it holds a halfway term,
            // bit 0 = parity of the increments after its last one (of all
            // of them when it holds none)
            int x = 0;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const float r = ldexpf(v[j], sh);
                const bool fin = r < 0x1p22f;
                const float rr = fin ? r : 0.0f;
                half[j] = rr - floorf(rr) == 0.5f;
                bad[j] = !fin;
                rho[j] = half[j] ? (int)floorf(rr) : (int)rintf(rr);
                x = half[j] ? 2 : x ^ (rho[j] & 1);
            }
            // inclusive segmented scan (a summary with bit 1 replaces what
            // came before it; 0 is the identity), then one lane down
            const auto comb = [](int left, int right) {
                return (right & 2) ? right : ((left & 2) | ((left ^ right) & 1));
            };
            x = comb(wm_dpp<WM_DPP_ROW_SHR1, 0xF>(x), x);
            x = comb(wm_dpp<WM_DPP_ROW_SHR2, 0xF>(x), x);
            x = comb(wm_dpp<WM_DPP_ROW_SHR4, 0xF>(x), x);
            x = comb(wm_dpp<WM_DPP_ROW_SHR8, 0xF>(x), x);
            x = comb(wm_dpp<WM_DPP_ROW_BCAST15, 0xA>(x), x);
            x = comb(wm_dpp<WM_DPP_ROW_BCAST31, 0xC>(x), x);
            const int xe = wave_shr1(x, 0);
            // parity of the significand before the lane's first term
            int par = (xe & 2) ? (xe & 1) : ((N ^ xe) & 1);
#pragma unroll
            for (int j = 0; j < 8; j++) {
                if (half[j]) {
                    rho[j] += (par + rho[j]) & 1;  // to the even neighbour
                    par = 0;
                } else {
                    par ^= rho[j] & 1;
                }
            }
        }
#pragma unroll
        for (int j = 0; j < 8; j++) {
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
    return s;
}

// Continues the sum from s (itself a left-to-right sum of earlier terms,
// so s >= +0 or NaN); a needs no alignment and is read only below n.
template <bool PARITY = false>
__device__ inline float seq_sum_nonneg_from(float s, const float *a, uint32_t n) {
    const uint32_t lane = threadIdx.x & 63;
    for (uint32_t k = 0; k < n; k += kSeqBatch) {
        const uint32_t base = k + 8 * lane;
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; j++) v[j] = base + j < n ? a[base + j] : 0.0f;
        s = seq_sum_step<PARITY>(s, v, k == 0);
        if (s != s) return s;
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
// only a short sequential walk remains.  Thread t owns the m = ceil(n / NT)
// consecutive terms k = t*m + j and holds them in registers.
//
//  1. A float64 prefix sum P_k (sum of the terms before k) predicts the binade
//     E of the f32 running sum before term k.  (The f32 sum differs from P_k
//     by accumulated rounding, far less than the distance to a power of two
//     for almost every k; every prediction is checked in step 3.)
//  2. A non-zero term k is a break if k = 0, if P_k or P_(k+1) is not
//     positive and finite, if their binades differ, if a_k / ulp(E) is
//     halfway between integers (the rounding then depends on the running
//     significand's parity) or if it is huge; any term is one if P_k (k a
//     thread's first term) or P_(k+1) (k its last) lies close to a power of
//     two (below).  Every other term contributes the integer increment
//     RN_int(a_k / ulp(E)) (0 for a zero term, which changes no running sum;
//     the terms before the first break are therefore all zeros).
//     A wave-wide integer scan places each wave's breaks in its own record
//     list, with the increment total before each.
//  3. One wave joins the lists and walks the breaks in order.  For a segment
//     (the terms between two breaks) it checks that the running sum s, exact
//     so far, is a normal number in the segment's binade with significand N,
//     and that N + D <= 2^24 - 2 for the segment's increment total D; then
//     adding the segment term by term gives exactly (N + D) * ulp, as in the
//     one-wave algorithm.  A break term is added with an ordinary f32 add.  A
//     segment whose check fails is summed by the one-wave algorithm from s
//     instead, so every outcome is the left-to-right sum.
//
// Why the "close to a power of two" rule.  The increments of one segment
// must all be taken with the same binade.  Inside a thread P_(k+1) of term k
// is bitwise P before term k+1, but across a thread boundary the two values
// come from different additions: the owner of k adds a_k to its own prefix,
// the next thread builds its prefix from the wave scan.  Every such value is
// a sum of non-negative doubles through at most 2*MAXM + 6 + 4 + 1 < 2^7
// additions along any path (MAXM <= 32), so it lies within relative
// 2^7 * 2^-53 = 2^-46 of the exact prefix, and two computations of one
// prefix within 2^-45 of each other.  A P_(k+1) farther than 2^-36 from
// every power of two therefore shares its binade with any other computation
// of the same prefix; one within 2^-36 makes term k a break, and then the
// next thread's P_(k+1) (within 2^-36 + 2^-45 < 2^-34) makes term k+1 a
// break too, so the segment after them starts with a binade computed by the
// thread that computes its increments.
//
// With the squares of an RMSNorm (2560 or 6912 terms) a sum has about 18
// breaks and a failed check in well under 1% of sums.  Squares of values
// with few significant bits (Q6_K-dequantised embedding rows) put many
// halfway terms among the first terms: up to ~75 breaks in the first wave of
// a 512-thread sum of 2560 (a few rows in a hundred above 48).  More than
// kSeqWaveRecords breaks in one wave send the whole sum to the one-wave
// algorithm (with the parity scan, which takes halfway terms in its runs).
constexpr int kSeqWaveRecords = 96;
constexpr int kSeqMaxWaves = 16;

// Increments are counted modulo 2^32: only differences over one segment are
// used, and a segment's increments add up to less than 2^24 + n / 2 (its
// terms sum to less than its binade's width, 2^23 ulps, each rounded by at
// most half an ulp), so the modular difference is the true one.
struct seq_block_scratch {
    double dw[kSeqMaxWaves];     // per wave: float64 total of its terms
    int wcnt[kSeqMaxWaves];      // per wave: breaks
    uint32_t wpi[kSeqMaxWaves];  // per wave: increment total (mod 2^32)
    int idx[kSeqMaxWaves][kSeqWaveRecords];       // term index of the break
    int eaf[kSeqMaxWaves][kSeqWaveRecords];       // predicted binade after it
    uint32_t pi[kSeqMaxWaves][kSeqWaveRecords];   // wave's increments before it
    float val[kSeqMaxWaves][kSeqWaveRecords];     // the term
    float out;
};

// a 32-bit inclusive prefix sum (modulo 2^32) over the wave, and a running
// maximum of non-negative values
__device__ __forceinline__ uint32_t wave_scan_u32(uint32_t x) {
    x += (uint32_t)wm_dpp<WM_DPP_ROW_SHR1, 0xF>((int)x);
    x += (uint32_t)wm_dpp<WM_DPP_ROW_SHR2, 0xF>((int)x);
    x += (uint32_t)wm_dpp<WM_DPP_ROW_SHR4, 0xF>((int)x);
    x += (uint32_t)wm_dpp<WM_DPP_ROW_SHR8, 0xF>((int)x);
    x += (uint32_t)wm_dpp<WM_DPP_ROW_BCAST15, 0xA>((int)x);
    x += (uint32_t)wm_dpp<WM_DPP_ROW_BCAST31, 0xC>((int)x);
    return x;
}
__device__ __forceinline__ int wave_max_scan_nonneg(int x) {
    x = max(x, wm_dpp<WM_DPP_ROW_SHR1, 0xF>(x));
    x = max(x, wm_dpp<WM_DPP_ROW_SHR2, 0xF>(x));
    x = max(x, wm_dpp<WM_DPP_ROW_SHR4, 0xF>(x));
    x = max(x, wm_dpp<WM_DPP_ROW_SHR8, 0xF>(x));
    x = max(x, wm_dpp<WM_DPP_ROW_BCAST15, 0xA>(x));
    x = max(x, wm_dpp<WM_DPP_ROW_BCAST31, 0xC>(x));
    return x;
}

// the biased exponent field of a non-negative double: floor(log2 x) + 1023
// for a positive, finite, normal x, 0 for +0
__device__ __forceinline__ int exp2field_f64(double x) {
    return (int)((__double_as_longlong(x) >> 52) & 0x7FF);
}
// floor(log2 x) of a positive, finite, normal double
__device__ __forceinline__ int exp2floor_f64(double x) { return exp2field_f64(x) - 1023; }
// x (positive, finite, normal) within relative 2^-T of a power of two
__device__ __forceinline__ bool near_pow2_f64(double x, int T) {
    const unsigned long long mant = (unsigned long long)__double_as_longlong(x) & ((1ull << 52) - 1);
    return mant <= (1ull << (52 - T)) || (1ull << 52) - mant <= (1ull << (53 - T));
}

// Left-to-right f32 sum of n non-negative terms, by every thread of a
// workgroup of NT threads (a multiple of 64, at most 1024).  v[j] holds term
// k = threadIdx.x * m + j for j < m = ceil(n / NT) <= MAXM and k < n, and 0
// otherwise; `a` holds all n terms, readable by wave 0 after a barrier (the
// caller writes it before the call).  The sum comes back in every thread.
// No work to slot in before the walk.
struct seq_no_hook {
    __device__ void operator()() const {}
};

// `before_walk` runs in every thread once the per-term work is done, while
// wave 0 walks the records and the other waves wait.  `after_walk(s)` runs
// in wave 0 alone with the finished sum, before the barrier that hands it to
// the other waves (work that only needs s can publish its result with it).
struct seq_no_after {
    __device__ void operator()(float) const {}
};
// `after_scan` runs in every thread right after the first barrier, when the
// waves' float64 totals (sc->dw) are complete.
template <int MAXM, int NT, typename Hook = seq_no_hook, typename After = seq_no_after,
          typename Mid = seq_no_hook>
__device__ __forceinline__ float seq_sum_block_owned(const float (&v)[MAXM], uint32_t n, const float *a,
                                     seq_block_scratch *sc, uint32_t m_run = 0,
                                     const Hook &before_walk = Hook(), const After &after_walk = After(),
                                     const Mid &after_scan = Mid()) {
    static_assert(NT % 64 == 0 && NT <= 64 * kSeqMaxWaves, "workgroup size");
    static_assert(MAXM >= 1 && MAXM <= 32, "terms per thread");
    constexpr int NW = NT / 64;
    constexpr int R = kSeqWaveRecords;
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wid = (uint32_t)__builtin_amdgcn_readfirstlane((int)(tid >> 6));
    if (n == 0) return 0.0f;
    // terms per thread: ceil(n / NT), or the caller's m_run (>= that, <= MAXM)
    const uint32_t m = m_run ? m_run : (n + NT - 1) / NT;
    const uint32_t k0 = tid * m;
    // A wave whose threads hold no terms (n below its first term) only takes
    // part in the barriers: its total is 0 and it records no break.
    const bool live = (uint64_t)wid * 64u * m < n;
    // 1. float64 prefix before this thread's first term
    double inc = 0.0, ex = 0.0;
    if (live) {
        double loc = 0.0;
#pragma unroll
        for (int j = 0; j < MAXM; j++) loc += (double)v[j];
        inc = wm_wave_scan_f64(loc);
        // exclusive prefix: the inclusive scan one lane down
        ex = __shfl_up(inc, 1, 64);
        if (lane == 0) ex = 0.0;
    }
    if (lane == 63) sc->dw[wid] = inc;
    wm_sync_lds();
    after_scan();
  if (live) {
    // the waves before this one: lane w < wid holds wave w's total, and a
    // scan along row 0 (NW <= 16 lanes) leaves their sum in lane 15
    double dl = (lane < (uint32_t)NW && lane < wid) ? sc->dw[lane] : 0.0;
#define WM_ROW_STEP(C) dl += __longlong_as_double(wm_dpp_i64<C, 0xF>(__double_as_longlong(dl)))
    WM_ROW_STEP(WM_DPP_ROW_SHR1);
    WM_ROW_STEP(WM_DPP_ROW_SHR2);
    WM_ROW_STEP(WM_DPP_ROW_SHR4);
    WM_ROW_STEP(WM_DPP_ROW_SHR8);
#undef WM_ROW_STEP
    const long long offb = __double_as_longlong(dl);
    const double off = __longlong_as_double(
        (long long)(((unsigned long long)(unsigned)__builtin_amdgcn_readlane((int)(offb >> 32), 15) << 32) |
                    (unsigned)__builtin_amdgcn_readlane((int)offb, 15)));
    double P = off + ex;
    // 2. breaks and increments.  Inside a thread P after term k is bitwise P
    // before term k+1, so the closeness test is needed only where the prefix
    // comes from another thread: before the first term and after the last.
    bool brk[MAXM];
    int incr[MAXM], eaf[MAXM];
    const uint32_t nval = min(m, n > k0 ? n - k0 : 0u);  // the thread's terms
    const uint32_t last = nval - 1;                        // index of the last one
    // The prefix after the thread's last term, by the same chain of adds as
    // the per-term loop below (adding the zeros past the last term leaves it
    // as is).  Non-negative terms make the chain non-decreasing, so when it
    // ends finite every prefix is finite and >= +0, and the full test below
    // reduces to one comparison of binades: the exponent field of +0 reads
    // 0, below every positive term's (>= 874), so a non-zero term on a
    // zero prefix (k == 0 among them) differs from its prefix's binade and
    // is a break, a zero term on it is not, and its increment is 0.  Only
    // sums that reach inf or NaN take the full test.
    double Pe = P;
#pragma unroll
    for (int j = 0; j < MAXM; j++) Pe = Pe + (double)v[j];
    if (Pe < 1e300) {
        const bool close0 = P > 0.0 && near_pow2_f64(P, 34);
        const bool close1 = Pe > 0.0 && near_pow2_f64(Pe, 36);
        int eb = exp2field_f64(P);  // biased: the binade is eb - 1023
#pragma unroll
        for (int j = 0; j < MAXM; j++) {
            P = P + (double)v[j];
            const int ea = exp2field_f64(P);
            // (a zero term leaves P, and so its binade, as it was)
            bool b = ea != eb;
            if (j == 0) b = b || close0;
            b = b || ((uint32_t)j == last && close1);
            const float r = ldexpf(v[j], 1046 - eb);  // a_k / ulp; exact unless < 2^-126
            b = b || !(r < 0x1p22f) || __builtin_amdgcn_fractf(r) == 0.5f;
            brk[j] = (uint32_t)j < nval && b;
            incr[j] = (uint32_t)j < nval && !b ? (int)rintf(r) : 0;
            eaf[j] = ea;
            eb = ea;
        }
    } else {
#pragma unroll
        for (int j = 0; j < MAXM; j++) {
            const uint32_t k = k0 + (uint32_t)j;
            const bool valid = (uint32_t)j < m && k < n;
            const double pb = P, pa = P + (double)v[j];
            P = pa;
            const bool pb_ok = pb > 0.0 && pb < 1e300, pa_ok = pa > 0.0 && pa < 1e300;
            const int eb = pb_ok ? exp2floor_f64(pb) : 0;
            const int ea = pa_ok ? exp2floor_f64(pa) : -1000;
            // a zero term leaves every running sum (+0, positive, inf or NaN)
            // unchanged, so it is never a break on its own account: a run of
            // zeros (an underflowed softmax tail, a zero prefix) costs nothing
            const bool zero = v[j] == 0.0f;
            bool b = !zero && (k == 0 || !pb_ok || !pa_ok || ea != eb);
            // (a zero prefix is exact in both precisions: every term before
            // it is zero, so no computation of it can land in another binade)
            if (j == 0) b = b || (pb_ok && near_pow2_f64(pb, 34));
            b = b || ((uint32_t)j == last && pa_ok && near_pow2_f64(pa, 36));
            int d = 0;
            if (!b) {
                const float r = ldexpf(v[j], 23 - eb);  // a_k / ulp; exact unless < 2^-126
                b = !(r < 0x1p22f) || r - floorf(r) == 0.5f;
                d = b ? 0 : (int)rintf(r);
            }
            brk[j] = valid && b;
            incr[j] = valid ? d : 0;
            eaf[j] = ea + 1023;
        }
    }
    uint32_t pi_loc = 0;
    int nb = 0;
#pragma unroll
    for (int j = 0; j < MAXM; j++) {
        nb += brk[j] ? 1 : 0;
        pi_loc += (uint32_t)incr[j];
    }
    // wave-local exclusive scans of the break counts and the increments
    const int nb_inc = wm_wave_scan_i32(nb);
    const uint32_t pi_inc = wave_scan_u32(pi_loc);
    int pos = nb_inc - nb;
    uint32_t pi = pi_inc - pi_loc;
#pragma unroll
    for (int j = 0; j < MAXM; j++) {
        if (brk[j]) {
            if (pos < R) {
                sc->idx[wid][pos] = (int)(k0 + (uint32_t)j);
                sc->eaf[wid][pos] = eaf[j] - 1023;
                sc->pi[wid][pos] = pi;
                sc->val[wid][pos] = v[j];
            }
            pos++;
        } else {
            pi += (uint32_t)incr[j];
        }
    }
    if (lane == 63) {
        sc->wcnt[wid] = nb_inc;
        sc->wpi[wid] = pi_inc;
    }
  } else if (lane == 63) {
    sc->wcnt[wid] = 0;
    sc->wpi[wid] = 0u;
  }
    wm_sync_lds();
    // 3. the walk over the breaks (wave 0), its first reads issued before
    // the hook's (LDS answers a wave's reads in order)
    int wc = 0;
    uint32_t wp = 0u;
    if (wid == 0) {
        wc = (int)lane < NW ? sc->wcnt[lane] : 0;
        wp = (int)lane < NW ? sc->wpi[lane] : 0u;
    }
    before_walk();
    if (wid == 0) {
        float s = 0.0f;
        if (__builtin_amdgcn_ballot_w64(wc > R) != 0) {
            s = seq_sum_nonneg_from<true>(0.0f, a, n);
        } else {
            // every wave's inclusive record count and increment total, as
            // wave-uniform values (SGPRs)
            const int cinc = wm_wave_scan_i32(wc);
            const uint32_t winc = wave_scan_u32(wp);
            int cs[NW];
            uint32_t ps[NW];
#pragma unroll
            for (int w = 0; w < NW; w++) {
                cs[w] = __builtin_amdgcn_readlane(cinc, w);
                ps[w] = (uint32_t)__builtin_amdgcn_readlane((int)winc, w);
            }
            const int nbrk = cs[NW - 1];
            const uint32_t pi_tot = ps[NW - 1];
            const int *idx = &sc->idx[0][0], *eafp = &sc->eaf[0][0];
            const uint32_t *pis = &sc->pi[0][0];
            const float *vals = &sc->val[0][0];
            // record base - 1, carried from the previous chunk: term index,
            // binade after it, increments before it
            int c_t = -1, c_e = -1000, c_p = 0;
            for (int base = 0; base <= nbrk; base += 64) {
                // lane l prepares step r = base + l: the segment between
                // records r-1 and r, then record r's term (r == nbrk: the
                // end; r > nbrk: a step that changes nothing)
                const int r = base + (int)lane;
                // record r belongs to wave wr: the waves whose records all
                // come before r are exactly those with cs[w] <= r (counts
                // are non-decreasing), and the last of them gives the
                // records and increments before wave wr
                int wr = 0, cex = 0;
                uint32_t wo = 0;
#pragma unroll
                for (int w = 0; w < NW; w++) {
                    const bool before = cs[w] <= r;
                    wr += before ? 1 : 0;
                    cex = before ? cs[w] : cex;
                    wo = before ? ps[w] : wo;
                }
                int t1 = (int)n, e1 = -1000;
                uint32_t p1 = pi_tot;
                float v1 = 0.0f;
                if (r < nbrk) {
                    const int f = wr * R + (r - cex);
                    t1 = idx[f];
                    e1 = eafp[f];
                    p1 = wo + pis[f];
                    v1 = vals[f];
                }
                // record r - 1: the lane below's (lane 0: the carry)
                const int t0 = wave_shr1(t1, c_t), e0 = wave_shr1(e1, c_e);
                const uint32_t p0 = (uint32_t)wave_shr1((int)p1, c_p);
                c_t = __builtin_amdgcn_readlane(t1, 63);
                c_e = __builtin_amdgcn_readlane(e1, 63);
                c_p = __builtin_amdgcn_readlane((int)p1, 63);
                const int cnt = r <= nbrk ? t1 - t0 - 1 : 0;  // terms in the segment
                const uint32_t dl = p1 - p0;                   // their increments
                const int D = dl <= (1u << 24) ? (int)dl : (1 << 30);
                const int here = min(64, nbrk + 1 - base);
                // When step r's check holds (s normal in binade e, s >= 2^e,
                // s + D*ulp <= (2^24 - 2) * ulp), its segment adds exactly
                // A = D * 2^(e-23): s + A is (N + D) * ulp, representable, so
                // the f32 add is exact.  The serial part is then two f32 adds
                // per step, t = s + A; s = t + V (V: the break term, +0 past
                // the last record); every lane checks its own step afterwards
                // from the value s had on entry.
                // the terms before the first break are all zeros (a non-zero
                // term on a zero prefix is a break), so that segment adds nothing
                const bool seg = cnt > 0 && r >= 1;
                const bool e_ok = e0 >= -126 && e0 <= 127;
                const float A = seg && e_ok ? ldexpf((float)D, e0 - 23) : 0.0f;
                const float lo = seg ? (e_ok ? ldexpf(1.0f, e0) : __int_as_float(0x7F800000)) : 0.0f;
                const float hi = seg ? (e_ok ? ldexpf(16777214.0f, e0 - 23) : -1.0f)
                                     : __int_as_float(0x7F800000);
                const float s0 = s;
                // (s is kept as a per-lane value, the same in every lane,
                // so the adds run on the vector unit)
                float sv;
                asm volatile("v_mov_b32 %0, %1" : "=v"(sv) : "v"(s));
                // The chain moves across the lanes: step u runs in lane u
                // (its operands are that lane's A and V), and its output
                // goes one lane up (a DPP shift; lane 0 is fed s, the value
                // entering step 0).  Every lane recomputes its step on every
                // round, but a lane's input stops changing once the lane
                // below has run its step, and so does its output: after
                // round u, lanes 0..u hold their final outputs, and in the
                // end lane u's input is the value s had entering step u.
                // Three dependent instructions a step (two adds, the
                // shift), and no step needs a value broadcast through an
                // SGPR (v_readlane, a compare's lane mask): on this part
                // such a value reaches a VALU instruction ~35 cycles after
                // it is written, and the broadcasts cost the walk more than
                // its adds.
                // Eight steps per loop trip (a taken branch costs more than
                // a step): the lanes past `here` hold A = V = +0 and pass
                // their input on unchanged.
                const int svb = __float_as_int(sv);
                float in = sv, nxt = sv;
                for (int u0 = 0; u0 < here; u0 += 8) {
#pragma unroll
                    for (int k = 0; k < 8; k++) {
                        nxt = (in + A) + v1;  // lane u: step u, once the steps below have run
                        in = __int_as_float(wave_shr1(__float_as_int(nxt), svb));
                    }
                }
                sv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(nxt), here - 1));
                const float s_in = in;
                s = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(sv)));
                // lanes past `here` hold no step; a NaN s fails every check
                const bool ok = (int)lane >= here || !seg || (s_in >= lo && s_in + A <= hi);
                const int bad = __builtin_amdgcn_ballot_w64(!ok) != 0;
                if (__builtin_amdgcn_readfirstlane(bad) != 0) {
                    s = s0;
                    for (int i = 0; i < here; i++) {
                        const int c = base + i >= 1 ? __builtin_amdgcn_readlane(cnt, i) : 0;
                        if (c > 0) {
                            const int Di = __builtin_amdgcn_readlane(D, i);
                            const int e = __builtin_amdgcn_readlane(e0, i);
                            const uint32_t bits = (uint32_t)__builtin_amdgcn_readfirstlane(__float_as_int(s));
                            const uint32_t ef = bits >> 23;
                            const int N = (int)((bits & 0x7FFFFFu) | 0x800000u);
                            if (ef - 1u < 254u && (int)ef - 127 == e && N + Di <= (1 << 24) - 2) {
                                s = ldexpf((float)(N + Di), e - 23);
                            } else {  // the segment term by term
                                const int tp = __builtin_amdgcn_readlane(t0, i);
                                s = seq_sum_nonneg_from<true>(s, a + tp + 1, (uint32_t)c);
                            }
                        }
                        s = s + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v1), i));
                    }
                }
            }
        }
        if (lane == 0) sc->out = s;
        after_walk(s);
    }
    wm_sync_lds();
    return sc->out;
}

}  // namespace wm
