// Exhaustive host check of the fp16 hi/lo split the prefill GEMM and
// attention feed to the matrix cores (k_gemm.hip k_gemm_xprep, k_prefill.hip
// k_prefill_khl / k_prefill_vt / the query and P parts): a row scaled so its
// maximum lies in [2^14, 2^15) is split as hi = rn16(x), lo = rn16(x - hi)
// (the fp32 subtraction is exact).  Claim: hi + lo is within 2^-22 |x| of
// x for every |x| in [2^-3, 2^15) (within 2^17 of the maximum), and within
// 2^-25 absolutely below that.  Every float in [0, 2^15) is checked (the
// split is symmetric in the sign).  Exits non-zero on a violation.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <thread>
#include <vector>

int main() {
    const uint32_t top = 0x47000000u;  // 2^15
    const unsigned nt = std::max(1u, std::thread::hardware_concurrency());
    std::vector<uint64_t> vn(nt, 0), vbr(nt, 0), vba(nt, 0);
    std::vector<double> vw(nt, 0.0);
    std::vector<std::thread> th;
    for (unsigned k = 0; k < nt; ++k)
        th.emplace_back([&, k] {
            for (uint32_t u = (uint32_t)((uint64_t)top * k / nt); u < (uint32_t)((uint64_t)top * (k + 1) / nt); ++u) {
                float x;
                std::memcpy(&x, &u, 4);
                const _Float16 hi = (_Float16)x;
                const float r = x - (float)hi;
                const _Float16 lo = (_Float16)r;
                const double err = std::fabs((double)x - ((double)(float)hi + (double)(float)lo));
                if (x >= 0.125f) {
                    ++vn[k];
                    vw[k] = std::max(vw[k], err / (double)x);
                    if (err > std::ldexp((double)x, -22)) ++vbr[k];
                } else if (err > std::ldexp(1.0, -25)) {
                    ++vba[k];
                }
            }
        });
    for (auto& t : th) t.join();
    uint64_t n_rel = 0, bad_rel = 0, bad_abs = 0;
    double worst = 0.0;
    for (unsigned k = 0; k < nt; ++k) {
        n_rel += vn[k];
        bad_rel += vbr[k];
        bad_abs += vba[k];
        worst = std::max(worst, vw[k]);
    }
    std::printf("[2^-3, 2^15): %llu values, worst relative error 2^%.3f, %llu above 2^-22\n",
                (unsigned long long)n_rel, std::log2(worst), (unsigned long long)bad_rel);
    std::printf("[0, 2^-3): %llu above 2^-25 absolute\n", (unsigned long long)bad_abs);
    return (bad_rel == 0 && bad_abs == 0) ? 0 : 1;
}
