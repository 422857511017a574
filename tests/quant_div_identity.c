/* Check of the division used by the per-channel quantizer
 * (rpl_amd/csrc/hip/quant.hip, div_scale_fast): for a row scale s with
 * 2^-100 <= s <= 2^125 and inv = 1.0f / s (correctly rounded),
 *
 *   q  = x * inv,   q' = fmaf(fmaf(-q, s, x), inv, q)
 *
 * must equal x / s bit for bit whenever |x| >= s / 4 (there the residual
 * x - q*s is a multiple of 2^-148, so it is exact and Markstein's theorem
 * applies), and the device's byte of it, q8_small(q') =
 * (int32)fminf(fmaxf(q' + copysignf(0.49999997f, q'), -128), 127), must be
 * the reference's clamp(x86cvt(roundf(x / s)), -128, 127) for every x (below
 * s / 4 both give 0).  Part 1 runs every float x with s/4 <= |x| <= 128 s (128 s bounds the
 * elements of a row whose scale is s) and every 61st float below s/4, for a
 * set of scales; part 2 runs random (x, s) pairs over the whole fast range.
 * Prints the number of mismatches; exit status 1 when there are any. */
#include <float.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float f_of(uint32_t b) {
    float f;
    memcpy(&f, &b, 4);
    return f;
}
static uint32_t b_of(float f) {
    uint32_t b;
    memcpy(&b, &f, 4);
    return b;
}

static int32_t x86cvt(float f) {
    if (!(f >= -2147483648.0f && f < 2147483648.0f)) return INT32_MIN;
    return (int32_t)f;
}
static int q8(float y) {
    int32_t v = x86cvt(roundf(y));
    return v < -128 ? -128 : (v > 127 ? 127 : v);
}
static int q8_small(float y) {
    volatile float t = y + copysignf(0.49999997f, y);
    return (int)(int8_t)(int32_t)fminf(fmaxf(t, -128.0f), 127.0f);
}
static float fast_div(float x, float s, float inv) {
    volatile float q = x * inv;
    volatile float r = fmaf(-q, s, x);
    return fmaf(r, inv, q);
}

/* 0 when x behaves, 1 on a mismatch. */
static int check(float x, float s, float inv) {
    const float want = x / s, got = fast_div(x, s, inv);
    int bad = q8(want) != q8_small(got) || (fabsf(x) >= 0.25f * s && b_of(want) != b_of(got));
    if (bad) printf("mismatch: s=%a x=%a x/s=%a fast=%a\n", s, x, want, got);
    return bad;
}

static uint64_t splitmix(uint64_t* st) {
    uint64_t z = (*st += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

int main(void) {
    unsigned long long bad = 0, n = 0;
    /* Part 1: every x with s/4 <= |x| <= 128 s, a sample below s/4. */
    const float scales[] = {1.0f / 127.0f, 5.5f / 127.0f, 0.02f * 4.9f / 127.0f, 0.1f, 3.0f, 1e-30f, 1e30f,
                            0x1p-100f,     0x1.000002p-100f, 0x1p125f, 0x1.fffffep124f, 0.9999999f};
    const int ns = sizeof(scales) / sizeof(scales[0]);
    for (int k = 0; k < ns; k++) {
        const float s = scales[k], inv = 1.0f / s;
        /* 128 s can exceed FLT_MAX: elements are finite (an infinite
           element makes the scale infinite, which divides exactly). */
        const float hi = 128.0f * s;
        const long long lo = b_of(0.25f * s), top = b_of(isinf(hi) ? FLT_MAX : hi);
#pragma omp parallel for reduction(+ : bad, n) schedule(static)
        for (long long b = 0; b <= top; b++) {
            if (b < lo && b % 61) continue;
            const float x = f_of((uint32_t)b);
            bad += check(x, s, inv) + check(-x, s, inv);
            n += 2;
        }
    }
    /* Part 2: random pairs over the whole fast range of s. */
    const long long pairs = 1ll << 25;
#pragma omp parallel for reduction(+ : bad, n) schedule(static)
    for (long long i = 0; i < pairs; i++) {
        uint64_t st = (uint64_t)i * 0x2545F4914F6CDD1Dull;
        const uint64_t r = splitmix(&st);
        const uint32_t lo = b_of(0x1p-100f), hi = b_of(0x1p125f);
        const float s = f_of(lo + (uint32_t)(r % (hi - lo + 1)));
        const float inv = 1.0f / s;
        /* |x| <= 128 s, as for the elements of a row with scale s. */
        float x = f_of((uint32_t)(splitmix(&st) >> 32) & 0x7fffffffu);
        const float hi128 = 128.0f * s;
        if (isnan(x) || isinf(x) || x > hi128) x = isinf(hi128) ? fmodf(x, FLT_MAX) : fmodf(x, hi128);
        if (isnan(x)) x = 0.5f * s;
        if (r >> 63) x = -x;
        bad += check(x, s, inv);
        n++;
    }
    printf("checked %llu mismatches %llu\n", n, bad);
    return bad != 0;
}
