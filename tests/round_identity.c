/* Exhaustive check of the device rounding used by the requantizing GEMM
 * epilogues (rpl_amd/csrc/hip/common.h, x86_round_cvt): for every float y,
 *
 *   x86cvt(roundf(y)) == in_range(t) ? (int32_t)t : INT32_MIN,
 *   t = y + copysignf(0.49999997f, y)   (rounded to nearest-even),
 *
 * where x86cvt is cvttss2si (NaN / out of range -> INT32_MIN), the
 * conversion the reference's (int32_t)roundf(...) compiles to.
 * Prints the number of mismatches; exit status 1 when there are any. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static int32_t x86cvt(float f) {
    if (!(f >= -2147483648.0f && f < 2147483648.0f)) return INT32_MIN;
    return (int32_t)f;
}

static int32_t device_form(float y) {
    volatile float t = y + copysignf(0.49999997f, y);
    return (t >= -2147483648.0f && t < 2147483648.0f) ? (int32_t)t : INT32_MIN;
}

int main(void) {
    unsigned long long bad = 0;
#pragma omp parallel for reduction(+ : bad) schedule(static)
    for (long long hi = 0; hi < 65536; hi++) {
        for (uint32_t lo = 0; lo < 65536; lo++) {
            const uint32_t b = ((uint32_t)hi << 16) | lo;
            float y;
            memcpy(&y, &b, 4);
            if (device_form(y) != x86cvt(roundf(y))) bad++;
        }
    }
    printf("mismatches %llu\n", bad);
    return bad != 0;
}
