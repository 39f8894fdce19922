/* Exhaustive check of the fused W8A8 quantizer's division.
 *
 * The per-token quantizer codes x as e4m3_rne(x / s) with s = max(amax, 1e-12) / 448 in
 * fp32 (IEEE divide). The fused kernel computes y = 1 / s once per row (IEEE divide) and
 * per value q = x * y, r = fma(-q, s, x), q' = copysign(fma(r, y, q), x). This program
 * runs every positive finite 16-bit amax (bf16, or fp16 with argument "fp16") against
 * every x of the same format with |x| <= amax, both signs, and counts the values whose
 * e4m3 code differs. It prints "<mismatched codes> <mismatched fp32 quotients> <pairs>".
 * A second argument "nocorrect" drops the fma correction (q' = x * y), which must mismatch;
 * "encode" prints the e4m3 codes of the floats read from stdin, one per line. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float from_bf16(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static float from_fp16(uint16_t h) {
    const int e = (h >> 10) & 31, m = h & 1023;
    float v = e == 0 ? ldexpf((float)m, -24) : (e == 31 ? INFINITY : ldexpf((float)(m | 1024), e - 25));
    return (h >> 15) ? -v : v;
}

/* e4m3 (fn) round to nearest even, for |v| <= 464 (the quantizer's range). */
static unsigned e4m3(float v) {
    const unsigned sign = signbit(v) ? 0x80u : 0u;
    const double a = fabs((double)v);
    if (a < 0x1p-6) { /* subnormal step 2^-9 */
        const double q = nearbyint(a * 512.0); /* ties to even in the default mode */
        return sign | (unsigned)q;             /* q == 8 is the smallest normal's code */
    }
    int e;
    const double f = frexp(a, &e); /* a = f * 2^e, f in [0.5, 1) */
    double m = nearbyint((f * 2.0 - 1.0) * 8.0);
    e -= 1;
    if (m == 8.0) { m = 0.0; e += 1; }
    return sign | (unsigned)(((e + 7) << 3) | (int)m);
}

int main(int argc, char** argv) {
    if (argc > 1 && strcmp(argv[1], "encode") == 0) {
        float v;
        while (scanf("%f", &v) == 1) printf("%u\n", e4m3(v));
        return 0;
    }
    const int fp16 = argc > 1 && strcmp(argv[1], "fp16") == 0;
    const int correct = !(argc > 2 && strcmp(argv[2], "nocorrect") == 0);
    const int top = fp16 ? 0x7c00 : 0x7f80; /* first non-finite positive code */
    long long bad_code = 0, bad_q = 0, pairs = 0;
#pragma omp parallel for reduction(+ : bad_code, bad_q, pairs) schedule(dynamic, 64)
    for (int a = 1; a < top; ++a) {
        const float amax = fp16 ? from_fp16((uint16_t)a) : from_bf16((uint16_t)a);
        const float s = fmaxf(amax, 1e-12f) / 448.0f;
        const float y = 1.0f / s;
        for (int b = 0; b <= a; ++b) {
            for (int neg = 0; neg < 2; ++neg) {
                const uint16_t bits = (uint16_t)(b | (neg ? 0x8000 : 0));
                const float x = fp16 ? from_fp16(bits) : from_bf16(bits);
                const float exact = x / s;
                const float q = x * y;
                const float r = fmaf(-q, s, x);
                const float fast = copysignf(correct ? fmaf(r, y, q) : q, x);
                pairs++;
                if (memcmp(&fast, &exact, 4) != 0) bad_q++;
                if (e4m3(fast) != e4m3(exact)) bad_code++;
            }
        }
    }
    printf("%lld %lld %lld\n", bad_code, bad_q, pairs);
    return 0;
}
