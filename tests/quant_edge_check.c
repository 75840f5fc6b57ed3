/* Randomized check of the ConvRot quantizer's fast quotient (fp32 values, so no exhaustive check): with
 *   sc = fl(fl(amax / 16) / 127), r = fl(1 / sc), rr = r / 16, n = rne(w * rr) (one fma against 1.5 * 2^23),
 *   d = fma(w, rr, -n),
 * every |d| <= 0.5 - 2^-16 must give n == rne(fl(fl(w / 16) / sc)), the IEEE-divide result.  The error bound
 * |w rr - y/sc| + |fl(y/sc) - y/sc| <= 2^-17 + 2^-18 plus d's own rounding (2^-25) is below 2^-16, which is the
 * margin the edge leaves.  Samples: amax over 2^-90 .. 2^90, w uniform in [-amax, amax], and w placed within
 * +-2^-14 of the points whose quotient is a half-integer, where the edge is decided.  Argument: seed.  Exits 1 on
 * a violation; prints the counts, including how many samples the edge sent to the divide. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

static uint64_t state;
static uint64_t next(void) {
    state ^= state << 13;
    state ^= state >> 7;
    state ^= state << 17;
    return state;
}
static double unit(void) { return (double)(next() >> 11) * 0x1p-53; }

int main(int argc, char** argv) {
    state = 0x9E3779B97F4A7C15ull ^ (uint64_t)(argc > 1 ? strtoull(argv[1], NULL, 0) : 1);
    const float magic = 12582912.0f, edge = 0.5f - 0x1p-16f;
    long long samples = 0, checked = 0, divide = 0, bad = 0;
    for (int a = 0; a < 20000; ++a) {
        const float amax = (float)ldexp(1.0 + unit(), (int)(unit() * 180.0) - 90);
        const float sc = (amax * 0.0625f) / 127.0f;
        const float r = 1.0f / sc;
        const float rr = r * 0.0625f;
        for (int i = 0; i < 2000; ++i) {
            float w;
            if (i & 1) {
                w = (float)((2.0 * unit() - 1.0) * amax);
            } else { /* near a half-integer quotient: y/sc = k + 0.5 + eps */
                const double k = floor(unit() * 127.0);
                const double eps = (2.0 * unit() - 1.0) * 0x1p-14;
                w = (float)((k + 0.5 + eps) * (double)sc * 16.0);
                if (fabsf(w) > amax) continue;
                if (next() & 1) w = -w;
            }
            ++samples;
            const float n = fmaf(w, rr, magic);
            const float d = fmaf(w, rr, -(n - magic));
            if (fabsf(d) > edge) { ++divide; continue; }
            ++checked;
            const float ref = fminf(fmaxf(rintf((w * 0.0625f) / sc), -127.0f), 127.0f);
            if (n - magic != ref) {
                if (bad < 10) printf("violation: amax %a w %a -> %g, divide %g (d %a)\n", amax, w, n - magic, ref, d);
                ++bad;
            }
        }
    }
    printf("samples %lld checked %lld divide %lld violations %lld\n", samples, checked, divide, bad);
    return bad != 0;
}
