/* The quantizers' quotient v / scale (csrc/common.hpp quotient_by_scale)
 * restated in C and compared bit for bit with IEEE division: y = RN(1 /
 * scale), q0 = RN(v y), then twice q <- RN(q + (v - q scale) y) with both
 * products fused (fmaf).  Cases, for the FP8 group scales max(amax, 1e-10)
 * * fl(1/448) and the INT8 row scales max(amax, 1e-12) / 127: random maxima
 * over 24 decades and values in the group, values within a few ulps of scale
 * times every E4M3 value and midpoint up to 448 and every half-integer up to
 * 127, exact products with short-mantissa scales, zeros, subnormals.  Prints
 * "ok <cases>" or the first mismatches.
 * Built with -ffp-contract=off so no product is fused behind our back. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static uint64_t state = 0x9E3779B97F4A7C15ull;
static uint64_t next(void) {
    state ^= state << 13;
    state ^= state >> 7;
    state ^= state << 17;
    return state;
}
static float unit(void) { return (float)((next() >> 40) * (1.0 / 16777216.0)); }
static uint32_t bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

static float quotient(float v, float scale, float y) {
    const float q0 = v * y;
    const float q1 = fmaf(fmaf(-q0, scale, v), y, q0);
    return fmaf(fmaf(-q1, scale, v), y, q1);
}

static long cases = 0, bad = 0;
static void check(float v, float scale) {
    const float want = v / scale;
    const float got = copysignf(quotient(v, scale, 1.0f / scale), v);
    ++cases;
    if (bits(want) != bits(got) && !(isnan(want) && isnan(got))) {
        if (bad < 8) printf("mismatch v=%a scale=%a want=%a got=%a\n", v, scale, want, got);
        ++bad;
    }
}

int main(int argc, char** argv) {
    const long n = argc > 1 ? atol(argv[1]) : 1000000;
    const float c = 1.0f / 448.0f;
    float e4m3[128];
    int ne = 0;
    for (int e = 0; e < 16; ++e)
        for (int m = 0; m < 8; ++m) {
            const float v = e == 0 ? ldexpf((float)m, -9) : ldexpf(1.0f + m / 8.0f, e - 7);
            if (v <= 448.0f) e4m3[ne++] = v;
        }
    for (long i = 0; i < n; ++i) {
        float amax = expf((unit() * 2.0f - 1.0f) * 27.6f);
        if (next() % 16 == 0) amax = 1e-10f * unit();
        const float scale = fmaxf(amax, 1e-10f) * c;  /* the group scale of an amax */
        check((unit() * 2.0f - 1.0f) * amax, scale);
        const int k = (int)(next() % (uint64_t)(ne - 1));
        const float target = (next() & 1) ? 0.5f * (e4m3[k] + e4m3[k + 1]) : e4m3[k + 1];
        float v = target * scale;
        const int steps = (int)(next() % 7) - 3;
        for (int s = 0; s < abs(steps); ++s) v = nextafterf(v, steps > 0 ? INFINITY : 0.0f);
        check((next() & 1) ? -v : v, scale);
        /* INT8 rows: rint boundaries at half-integers */
        const float sc8 = fmaxf(amax, 1e-12f) / 127.0f;
        check((unit() * 2.0f - 1.0f) * amax, sc8);
        float h = ((float)(next() % 127) + 0.5f) * sc8;
        const int steps8 = (int)(next() % 7) - 3;
        for (int s = 0; s < abs(steps8); ++s) h = nextafterf(h, steps8 > 0 ? INFINITY : 0.0f);
        check((next() & 1) ? -h : h, sc8);
        check(((float)(next() % 128)) * sc8, sc8);
        const float short_scale = ldexpf((float)(1 + next() % 64), (int)(next() % 40) - 60);
        const float exact = target * short_scale;
        check(exact, short_scale);
        check(nextafterf(exact, INFINITY), short_scale);
        check(nextafterf(exact, 0.0f), short_scale);
    }
    check(0.0f, 1.0f);
    check(-0.0f, 1.0f);
    check(-0.0f, 1e-10f * c);
    check(1e-45f, 1e-10f * c);
    check(-1e-45f, 1e-10f * c);
    check(448.0f, 1.0f);
    if (bad) {
        printf("%ld of %ld cases differ\n", bad, cases);
        return 1;
    }
    printf("ok %ld\n", cases);
    return 0;
}
