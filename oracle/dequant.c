/* CPU restatement, in C with OpenMP, of the reference's int4 Marlin dequant, for the host
 * baseline timed by the benchmark. Test infrastructure only: the HIP library never links or
 * calls it.
 *
 *   W[n][k] = round_t(q[n][k] * round_t(float(scale[n / block_n][k / group_size])))
 *
 * with q the signed nibbles of packed int32 [N, K/8] (least significant first, two's
 * complement; pulsarlm-core/tests/kernels/test_marlin.cpp:42-46) and round_t round-to-
 * nearest-even to bf16 or fp16 (pulsarlm-core/src/kernels/marlin.cu:78-84,123-151). The
 * numpy oracle (oracle.py dequant_int4) states the same rule; tests check the two agree bit
 * for bit. Results are float32 holding the rounded values. */
#include <omp.h>
#include <stdint.h>
#include <string.h>

static float bits_to_f32(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}
static uint32_t f32_to_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

/* Round to bf16 (round to nearest, ties to even); finite inputs. */
static float round_bf16(float f) {
    uint32_t u = f32_to_bits(f);
    u = (u + 0x7FFFu + ((u >> 16) & 1u)) & 0xFFFF0000u;
    return bits_to_f32(u);
}

/* Round to fp16 (round to nearest, ties to even) and back to float: the significand is cut
 * to 11 bits (fewer below 2^-14, where fp16 is subnormal); overflow saturates to infinity. */
static float round_fp16(float f) {
    uint32_t u = f32_to_bits(f);
    const uint32_t sign = u & 0x80000000u;
    uint32_t a = u & 0x7FFFFFFFu;
    if (a >= 0x7F800000u) return f; /* inf / nan */
    int e = (int)(a >> 23) - 127;
    if (e >= 16) return bits_to_f32(sign | 0x7F800000u);
    int drop = 13;                   /* 23 - 10 fraction bits */
    if (e < -14) drop += -14 - e;    /* subnormal fp16: fewer significand bits */
    if (drop > 24) return bits_to_f32(sign); /* below half the smallest subnormal */
    uint64_t m = (a & 0x7FFFFFu) | (e >= -126 ? 0x800000u : 0u);
    const uint64_t half = (uint64_t)1 << (drop - 1), mask = ((uint64_t)1 << drop) - 1;
    const uint64_t rem = m & mask;
    m >>= drop;
    if (rem > half || (rem == half && (m & 1))) m += 1;
    /* back to float: value = m * 2^(e - 23 + drop) */
    float v = (float)m;
    const int sh = e - 23 + drop;
    /* multiply by 2^sh exactly through the exponent field (sh in [-24, 15]) */
    v *= bits_to_f32((uint32_t)(127 + sh) << 23);
    if (v >= 65536.0f) return bits_to_f32(sign | 0x7F800000u);
    return bits_to_f32(f32_to_bits(v) | sign);
}

/* scale_dtype: 0 fp16, 1 bf16, 2 fp32 (raw storage of the [ceil(N/bn), K/g] scales).
 * out_bf16: 1 rounds to bf16, 0 to fp16. threads: 0 = OpenMP's default count. */
int oracle_dequant_int4(const int32_t* packed, const void* scale, int scale_dtype, int64_t n, int64_t k,
                        int64_t block_n, int64_t group_size, int out_bf16, float* out, int threads) {
    if (n <= 0 || k <= 0 || k % 8 || block_n <= 0 || group_size <= 0 || k % group_size) return 1;
    const int64_t groups = k / group_size;
    const int nt = threads > 0 ? threads : omp_get_max_threads();
#pragma omp parallel for schedule(static) num_threads(nt)
    for (int64_t r = 0; r < n; ++r) {
        const int64_t srow = (r / block_n) * groups;
        for (int64_t g = 0; g < groups; ++g) {
            float s;
            if (scale_dtype == 2) {
                s = ((const float*)scale)[srow + g];
            } else {
                const uint16_t h = ((const uint16_t*)scale)[srow + g];
                if (scale_dtype == 1) {
                    s = bits_to_f32((uint32_t)h << 16);
                } else { /* fp16 -> f32, exact */
                    const uint32_t sg = (uint32_t)(h & 0x8000u) << 16;
                    const uint32_t ex = (h >> 10) & 0x1Fu, fr = h & 0x3FFu;
                    float v;
                    if (ex == 0) v = (float)fr * bits_to_f32(0x33800000u); /* fr * 2^-24 */
                    else if (ex == 31) v = bits_to_f32(0x7F800000u | (fr << 13));
                    else v = bits_to_f32(((ex + 112u) << 23) | (fr << 13));
                    s = bits_to_f32(f32_to_bits(v) | sg);
                }
            }
            const float sr = out_bf16 ? round_bf16(s) : round_fp16(s);
            for (int64_t c = g * group_size; c < (g + 1) * group_size; c += 8) {
                const uint32_t w = (uint32_t)packed[r * (k / 8) + c / 8];
                for (int j = 0; j < 8; ++j) {
                    const int q = (int)((w >> (4 * j)) & 0xFu) - (int)(((w >> (4 * j)) & 0x8u) << 1);
                    const float p = (float)q * sr;
                    out[r * k + c + j] = out_bf16 ? round_bf16(p) : round_fp16(p);
                }
            }
        }
    }
    return 0;
}
