// Host check of the GEMV's second-digit-level rule (maybe_wide/block_wide of
// project-ia_amd/csrc/qh_digits.hpp, compiled here for the host) on blocks
// quantized as the device does (k from the block maximum, A = rint(x 2^k),
// |A| <= kDigitMax), for its documented properties:
//  P1  N(0,1) blocks never take level 2;
//  P2  1..6 outliers of 1e3, 1e4 or 1e5 among N(0,1) values always do;
//  P3  a block left on level 1 keeps, whichever 6 elements are removed, a
//      magnitude sum of at least 3 * (max|A| >> 6) (the rule's guarantee);
//  P4  in a level-2 block every element within 2^21 of the block maximum is
//      exact: (A + 2^-23 B) 2^-k == x, B = rint((x 2^k - A) 2^23).  (The
//      block maximum lands at x 2^k >= 2^21.9, so elements down to 2^-21
//      of it have x 2^k >= 1; between 2^-21.9 and 2^-22 an element can
//      keep 24 bits instead of all of them.)
// Prints counts; exits non-zero on any violation.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <random>

#include "qh_digits.hpp"

struct Q {
    int A[32];
    int k, amax;
    bool wide;
};

static Q quantize(const float (&x)[32]) {
    Q q{};
    float m = 0.0f;
    for (float v : x) m = std::max(m, std::fabs(v));
    q.k = 0;
    if (m > 0.0f) {
        int E;
        std::frexp(m, &E);  // m < 2^E
        q.k = 23 - E;
        if (std::rint(std::ldexp(m, q.k)) > (float)qh::kDigitMax) q.k -= 1;
    }
    q.amax = (int)std::rint(std::ldexp(m, q.k));
    int asum = 0, c1 = 0, c2 = 0;
    for (int e = 0; e < 32; ++e) {
        q.A[e] = (int)std::rint(std::ldexp(x[e], q.k));
        const int a = std::abs(q.A[e]);
        asum += a;
        c1 += std::min(a, q.amax >> 4);
        c2 += std::min(a, q.amax >> 6);
    }
    q.wide = qh::maybe_wide(q.amax, asum) && qh::block_wide(q.amax, c1, c2);
    return q;
}

// sum of |A| over all but the 6 largest
static long long rest6(const Q& q) {
    int a[32];
    for (int e = 0; e < 32; ++e) a[e] = std::abs(q.A[e]);
    std::sort(a, a + 32);
    long long s = 0;
    for (int e = 0; e < 26; ++e) s += a[e];
    return s;
}

int main() {
    std::mt19937_64 rng(20240611);
    std::normal_distribution<float> nd(0.0f, 1.0f);
    std::student_t_distribution<float> t3(3.0f);
    std::uniform_real_distribution<float> ud(0.0f, 1.0f);
    long long p1 = 0, p2_bad = 0, p2_n = 0, p3_bad = 0, p3_n = 0, p4_bad = 0, p4_n = 0;
    float x[32];
    // P1
    for (int b = 0; b < 1000000; ++b) {
        for (auto& v : x) v = nd(rng);
        p1 += quantize(x).wide;
    }
    // P2
    for (int n = 1; n <= 6; ++n)
        for (float mag : {1e3f, 1e4f, 1e5f})
            for (int b = 0; b < 20000; ++b) {
                for (auto& v : x) v = nd(rng);
                int idx[32];
                for (int e = 0; e < 32; ++e) idx[e] = e;
                std::shuffle(idx, idx + 32, rng);
                for (int o = 0; o < n; ++o) x[idx[o]] = (ud(rng) < 0.5f ? -mag : mag);
                ++p2_n;
                p2_bad += !quantize(x).wide;
            }
    // P3 and P4 over mixed distributions
    for (int b = 0; b < 2000000; ++b) {
        const int kind = b % 5;
        for (auto& v : x) {
            switch (kind) {
                case 0: v = nd(rng); break;
                case 1: v = t3(rng); break;
                case 2: v = ud(rng) < 0.8f ? 0.0f : nd(rng); break;                    // sparse
                case 3: v = std::ldexp(nd(rng), (int)(ud(rng) * 40.0f) - 20); break;  // wide magnitudes
                default: v = nd(rng) * nd(rng) * 8.0f; break;                          // product-like tails
            }
        }
        if (kind == 4 && b % 7 == 0) x[b % 32] = 3e4f;
        const Q q = quantize(x);
        if (!q.wide) {
            ++p3_n;
            if (rest6(q) < 3LL * (q.amax >> 6)) ++p3_bad;
        } else {
            float m = 0.0f;
            for (float v : x) m = std::max(m, std::fabs(v));
            for (int e = 0; e < 32; ++e) {
                if (!(std::fabs(x[e]) >= std::ldexp(m, -21))) continue;
                const float t = std::ldexp(x[e], q.k);
                const float a = std::rint(t);
                const int B = (int)std::rint((t - a) * 8388608.0f);
                const double rec = std::ldexp((double)q.A[e] + std::ldexp((double)B, -23), -q.k);
                ++p4_n;
                p4_bad += rec != (double)x[e];
            }
        }
    }
    std::printf("P1 N(0,1) blocks on level 2: %lld of 1000000\n", p1);
    std::printf("P2 outlier blocks left on level 1: %lld of %lld\n", p2_bad, p2_n);
    std::printf("P3 level-1 blocks below the guarantee: %lld of %lld\n", p3_bad, p3_n);
    std::printf("P4 inexact elements of level-2 blocks: %lld of %lld\n", p4_bad, p4_n);
    return (p1 == 0 && p2_bad == 0 && p3_bad == 0 && p4_bad == 0 && p4_n > 0) ? 0 : 1;
}
