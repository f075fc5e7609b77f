// expf evaluated as the reference's f32::exp evaluates on x86_64 Linux:
// glibc's expf (>= 2.27).  Its published algorithm:
//   x * 32/ln2 = k + r (k integer, |r| <= 1/2),
//   exp(x) = 2^(k/32) * P(r),  P(r) = 1 + C2 r + C1 r^2 + C0 r^3,
// in double precision, 2^(k/32) assembled from a 32-entry table of
// 2^(i/32) (each entry the correctly rounded double, stored minus i << 47)
// plus k's high bits added into the exponent field.  With the fused
// multiply-adds placed as below (glibc's FMA build contracts the r and
// polynomial steps), the result equals glibc 2.35's expf for every float in
// [-128, 0] -- every softmax argument x - max is <= 0.  tests/test_expf.py
// re-checks that claim against the host libm.
//
// Host and device code share this function (WM_HD expands to
// __host__ __device__ under hipcc).
#pragma once
#include <cstdint>
#include <cstring>

#ifndef WM_HD
#define WM_HD
#endif

namespace wm {

constexpr uint64_t kExp2Tab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

// `tab` is kExp2Tab or a copy of it (device code passes an LDS copy so the
// per-lane table lookup does not wait on global memory).
WM_HD inline float expf_glibc(float x, const uint64_t *tab = kExp2Tab) {
    const double kInvLn2N = 0x1.71547652b82fep+0 * 32.0;
    const double kShift = 0x1.8p+52;
    const double kC0 = 0x1.c6af84b912394p-5 / (32.0 * 32.0 * 32.0);
    const double kC1 = 0x1.ebfce50fac4f3p-3 / (32.0 * 32.0);
    const double kC2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    uint32_t ux;
    std::memcpy(&ux, &x, 4);
    const uint32_t abstop = (ux >> 20) & 0x7ffu;
    if (abstop >= 0x42bu) {  // |x| >= 88 or NaN
        if (ux == 0xff800000u) return 0.0f;
        if (abstop >= 0x7f8u) return x + x;
        if (x > 0x1.62e42ep6f) {
            const uint32_t inf = 0x7f800000u;
            float r;
            std::memcpy(&r, &inf, 4);
            return r;
        }
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    const double xd = (double)x;
    double kd = __builtin_fma(kInvLn2N, xd, kShift);
    uint64_t ki;
    std::memcpy(&ki, &kd, 8);
    kd -= kShift;
    const double r = __builtin_fma(kInvLn2N, xd, -kd);
    const uint64_t t = tab[ki & 31u] + (ki << 47);
    double s;
    std::memcpy(&s, &t, 8);
    const double z = __builtin_fma(kC0, r, kC1);
    const double r2 = r * r;
    double y = __builtin_fma(kC2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    y = y * s;
    return (float)y;
}

}  // namespace wm
