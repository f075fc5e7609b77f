// Compares wm::expf_glibc (project-willamette_amd/csrc/wm_expf.h, the
// function the GPU softmax calls) with the host libm's expf over the float
// bit patterns of [-128, 0] (every `stride`-th pattern, split across
// threads).  Prints "checked N mismatches M" and exits 1 on a mismatch.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <thread>
#include <vector>

#include "wm_expf.h"

int main(int argc, char **argv) {
    const uint32_t stride = argc > 1 ? (uint32_t)strtoul(argv[1], nullptr, 0) : 1u;
    const uint32_t lo = 0x80000000u, hi = 0xC3000000u;  // -0 .. -128
    unsigned nt = std::thread::hardware_concurrency();
    if (nt == 0 || nt > 16) nt = nt ? 16 : 1;
    std::vector<long> mism(nt, 0), checked(nt, 0);
    std::vector<std::thread> th;
    for (unsigned t = 0; t < nt; t++)
        th.emplace_back([&, t] {
            uint64_t span = (uint64_t)(hi - lo) + 1;
            uint64_t b0 = lo + span * t / nt, b1 = lo + span * (t + 1) / nt;
            b0 = b0 + (stride - (b0 - lo) % stride) % stride;
            for (uint64_t b = b0; b < b1; b += stride) {
                uint32_t u = (uint32_t)b;
                float x;
                std::memcpy(&x, &u, 4);
                float g = expf(x), m = wm::expf_glibc(x);
                checked[t]++;
                if (std::memcmp(&g, &m, 4) != 0) {
                    if (mism[t]++ < 3) std::printf("mismatch x=%a libm=%a restated=%a\n", x, g, m);
                }
            }
        });
    for (auto &x : th) x.join();
    long c = 0, m = 0;
    for (unsigned t = 0; t < nt; t++) c += checked[t], m += mism[t];
    std::printf("checked %ld mismatches %ld\n", c, m);
    return m ? 1 : 0;
}
