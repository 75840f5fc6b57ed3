/* Exhaustive check of the per-token quantizer's quotient for bf16 inputs (the GPU kernels' quant8b):
 *   q0 = fl(e * r), rem = fma(-q0, sc, e), q1 = fma(rem, r, q0), n = rne(q1)
 * with sc = fl(amax / 127), r = fl(1 / sc), against clamp(rne(fl(e / sc)), -127, 127) computed with the IEEE
 * divide, for every positive finite bf16 amax whose sc lies in [2^-100, 2^126] (and r <= 2^126) and every bf16
 * e in [0, amax].  Every operation negates with e, so negative e needs no separate pass.  Arguments: the first
 * and one past the last amax bit pattern to cover (default: all).  Prints the pair and mismatch counts; exits 1
 * on a mismatch.  Built with -ffp-contract=off so that each operation rounds as written. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float bf16_value(uint32_t bits) {
    const uint32_t u = bits << 16;
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

int main(int argc, char** argv) {
    const uint32_t lo = argc > 1 ? (uint32_t)strtoul(argv[1], NULL, 0) : 1u;
    const uint32_t hi = argc > 2 ? (uint32_t)strtoul(argv[2], NULL, 0) : 0x7F80u;
    const float magic = 12582912.0f; /* 1.5 * 2^23: x + magic - magic = rne(x) for |x| < 2^22 */
    long long pairs = 0, bad = 0, scales = 0;
    for (uint32_t a = lo; a < hi; ++a) {
        const float amax = bf16_value(a);
        const float sc = amax / 127.0f;
        const float r = 1.0f / sc;
        if (!(sc >= 0x1p-100f && sc <= 0x1p+126f && r <= 0x1p+126f)) continue;
        ++scales;
        for (uint32_t eb = 0; eb <= a; ++eb) {
            const float e = bf16_value(eb);
            const float q0 = e * r;
            const float rem = fmaf(-q0, sc, e);
            const float q1 = fmaf(rem, r, q0);
            const float n = (q1 + magic) - magic;
            const float ref = fminf(fmaxf(rintf(e / sc), -127.0f), 127.0f);
            ++pairs;
            if (n != ref) {
                if (bad < 10) printf("mismatch: amax %a e %a -> %g, divide %g\n", amax, e, n, ref);
                ++bad;
            }
        }
    }
    printf("scales %lld pairs %lld mismatches %lld\n", scales, pairs, bad);
    return bad != 0;
}
