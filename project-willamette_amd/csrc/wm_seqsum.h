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
// on 256 terms at a time:
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
// readable by every lane); returns the sum in every lane.
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

// Sequential f32 sum of n non-negative terms a[0..n) (as s += a[i]).
// Negative terms are not allowed (the caller's terms are squares or exp()).
__device__ inline float seq_sum_nonneg(const float *a, uint32_t n) {
    const uint32_t lane = threadIdx.x & 63;
    float s = 0.0f;
    uint32_t k = 0;
    // Leading terms one at a time: the first terms move s across many
    // binades, which would end every parallel run after one term.
    const uint32_t lead = n < 32 ? n : 32;
    for (; k < lead; k++) s = s + a[k];
    while (k < n) {
        if (!(s >= 0x1p-60f && s <= 0x1p+100f)) {  // zero, tiny, huge, inf or NaN
            for (; k < n; k++) s = s + a[k];
            break;
        }
        const int E = (int)((__float_as_uint(s) >> 23) & 0xffu) - 127;
        const int sh = 23 - E;
        const int N = (int)ldexpf(s, sh);  // s / ulp, in [2^23, 2^24)
        const uint32_t base = k + 4 * lane;
        float v[4];
        // unconditional loads from clamped indices, so all four are in flight at once
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t i = base + j < n ? base + j : n - 1;
            v[j] = a[i];
        }
#pragma unroll
        for (int j = 0; j < 4; j++) v[j] = (base + j < n) ? v[j] : 0.0f;
        int rho[4];
        bool bad[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float r = ldexpf(v[j], sh);  // a / ulp
            const bool ok = r < 0x1p22f;     // false for NaN, inf, huge
            const float f = floorf(r);
            const float fr = r - f;
            bad[j] = !ok || fr == 0.5f;
            rho[j] = bad[j] ? 0 : (int)f + (fr > 0.5f ? 1 : 0);
        }
        const int p0 = rho[0], p1 = p0 + rho[1], p2 = p1 + rho[2], p3 = p2 + rho[3];
        const int incl = wave_incl_scan_i32(p3);
        const int excl = incl - p3;
        const int limit = (1 << 24) - 1 - N;  // run continues while prefix < limit
        const int pj[4] = {p0, p1, p2, p3};
        int first = 4;
#pragma unroll
        for (int j = 3; j >= 0; j--)
            if (bad[j] || excl + pj[j] >= limit) first = j;
        const uint64_t mask = __ballot(first < 4);
        if (mask == 0) {
            const int total = __builtin_amdgcn_readlane(incl, 63);
            s = ldexpf((float)(N + total), -sh);
            k = (k + 256 < n) ? k + 256 : n;
            continue;
        }
        const int fl = __ffsll((unsigned long long)mask) - 1;
        const int before = excl + (first == 0 ? 0 : (first == 1 ? p0 : (first == 2 ? p1 : p2)));
        const int jl = __builtin_amdgcn_readlane(first, fl);
        const int pre = __builtin_amdgcn_readlane(before, fl);
        const uint32_t idx = k + 4 * (uint32_t)fl + (uint32_t)jl;
        s = ldexpf((float)(N + pre), -sh);  // the run before the offending term
        s = s + a[idx];                     // that term, by an ordinary add
        k = idx + 1;
    }
    return s;
}

}  // namespace wm
