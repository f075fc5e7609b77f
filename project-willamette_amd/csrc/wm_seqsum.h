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

// Terms handled per wave step (8 per lane).  Callers allocate the term
// array 16-byte aligned and readable up to seq_sum_padded(n) entries; the
// entries past n are read but ignored.
constexpr uint32_t kSeqBatch = 512;
constexpr int kSeqLead = 128;  // leading terms added one by one
__host__ __device__ constexpr uint32_t seq_sum_padded(uint32_t n) {
    return (n + kSeqBatch - 1) / kSeqBatch * kSeqBatch;
}

// Sequential f32 sum of n non-negative terms a[0..n) (as s += a[i]).
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
__device__ inline float seq_sum_nonneg(const float *a, uint32_t n) {
    const uint32_t lane = threadIdx.x & 63;
    float s = 0.0f;
    if (n == 0) return s;
    float4 nx0 = *reinterpret_cast<const float4 *>(a + 8 * lane);
    float4 nx1 = *reinterpret_cast<const float4 *>(a + 8 * lane + 4);
    for (uint32_t k = 0; k < n; k += kSeqBatch) {
        const uint32_t base = k + 8 * lane;
        float v[8] = {nx0.x, nx0.y, nx0.z, nx0.w, nx1.x, nx1.y, nx1.z, nx1.w};
        if (k + kSeqBatch < n) {  // next step's terms, in flight during this one
            nx0 = *reinterpret_cast<const float4 *>(a + base + kSeqBatch);
            nx1 = *reinterpret_cast<const float4 *>(a + base + kSeqBatch + 4);
        }
#pragma unroll
        for (int j = 0; j < 8; j++) v[j] = base + j < n ? v[j] : 0.0f;
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

}  // namespace wm
