/*
 * div_check.c — test helper: the temperature division the HIP kernels use for exact values
 * (builderforce-inference_amd/csrc/smp_common.h, div_T_fast), checked bit-for-bit against
 * IEEE f32 division. Usage: div_check T [T ...] < (nothing); prints one line per T:
 * "T count bad". x covers a strided sample of every f32 with |x| in [2^-100, 2^100).
 * Built by tests/test_division.py with gcc -O2 -ffp-contract=off (fmaf from libm).
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float fast_div(float x, float t, float r) {
    const float q = x * r;
    const float e = fmaf(-q, t, x);
    const float s = fmaf(e, r, q);
    return e != e ? q : s;
}

int main(int argc, char **argv) {
    const uint32_t stride = argc > 1 ? (uint32_t)strtoul(argv[1], 0, 10) : 997u;
    for (int i = 2; i < argc; i++) {
        const float t = strtof(argv[i], 0), r = 1.0f / t;
        uint64_t count = 0, bad = 0;
        for (uint64_t u = 0; u < (1ull << 32); u += stride) {
            uint32_t b = (uint32_t)u;
            float x;
            memcpy(&x, &b, 4);
            const float ax = fabsf(x);
            if (!(ax >= 0x1p-100f && ax < 0x1p100f)) continue;
            const float want = x / t, got = fast_div(x, t, r);
            uint32_t wb, gb;
            memcpy(&wb, &want, 4);
            memcpy(&gb, &got, 4);
            count++;
            if (wb != gb) bad++;
        }
        printf("%.9g %llu %llu\n", t, (unsigned long long)count, (unsigned long long)bad);
    }
    return 0;
}
