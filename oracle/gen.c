/*
 * Oracle-side seeded weight/input generator (CPU, test infrastructure only).
 *
 * This file is part of the oracle: only tests, the smoke check and the bench's
 * CPU-baseline leg load it, and only as the checker.  The HIP library has its own
 * device implementation of the same specification; the two are compared bit for
 * bit by the test suite.
 *
 * Specification (shared with the device generator):
 *   key        = fnv1a64(tensor name) XOR splitmix64(seed)
 *   h1, h2     = splitmix64(key + 2*i), splitmix64(key + 2*i + 1)   (i = row-major
 *                index of the element in the tensor's canonical diffusers layout)
 *   u1         = ((h1 >> 11) + 1) * 2^-53          in (0, 1]
 *   u2         = (h2 >> 11) * 2^-53                in [0, 1)
 *   z          = sqrt(-2 ln u1) * cos(2 pi u2)      (Box-Muller, double)
 *   value      = half( float( mean + std * z ) )    (each conversion rounds to nearest even)
 *
 * The weights the reference engine consumes are raw fp16 files
 * (vk_engine.cpp:497-505); "fp16-representable N(0, 0.02)" random-init weights are
 * produced here instead of read from disk.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

/* float32 -> nearest fp16 value (round to nearest even, subnormals kept, overflow
 * to infinity), returned as float32.  Written out by hand because the host
 * compiler has no _Float16 on this target. */
static float round_to_half(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = x & 0x80000000u, ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return f;                       /* inf / nan */
    if (ax >= 0x477ff000u) return sign ? -INFINITY : INFINITY;
    if (ax < 0x38800000u) {                                 /* fp16 subnormal range */
        float q = nearbyintf(fabsf(f) * 16777216.0f);       /* quantum 2^-24, RNE */
        float v = q * (1.0f / 16777216.0f);
        return sign ? -v : v;
    }
    uint32_t r = (ax + 0xfffu + ((ax >> 13) & 1u)) & ~0x1fffu;
    r |= sign;
    float out;
    memcpy(&out, &r, 4);
    return out;
}

static uint64_t splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ULL;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ULL;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBULL;
    return x ^ (x >> 31);
}

uint64_t oracle_fnv1a64(const char* s) {
    uint64_t h = 0xCBF29CE484222325ULL;
    for (; *s; ++s) { h ^= (uint8_t)*s; h *= 0x100000001B3ULL; }
    return h;
}

uint64_t oracle_tensor_key(const char* name, uint64_t seed) {
    return oracle_fnv1a64(name) ^ splitmix64(seed);
}

/* Fill out[0..n) with fp16-rounded N(mean, std) values, returned as float32. */
void oracle_gauss_fill(uint64_t key, int64_t n, double mean, double stdv, float* out) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        uint64_t h1 = splitmix64(key + 2ULL * (uint64_t)i);
        uint64_t h2 = splitmix64(key + 2ULL * (uint64_t)i + 1ULL);
        double u1 = (double)((h1 >> 11) + 1ULL) * 0x1.0p-53;
        double u2 = (double)(h2 >> 11) * 0x1.0p-53;
        double z = sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
        out[i] = round_to_half((float)(mean + stdv * z));
    }
}

/* Round an fp32 buffer to fp16 values in place (same rounding as above). */
void oracle_round_half(float* buf, int64_t n) {
    for (int64_t i = 0; i < n; ++i) buf[i] = round_to_half(buf[i]);
}

/* Same stream without the fp16 rounding (fp32 inputs such as latents and contexts). */
void oracle_gauss_fill_f32(uint64_t key, int64_t n, double mean, double stdv, float* out) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        uint64_t h1 = splitmix64(key + 2ULL * (uint64_t)i);
        uint64_t h2 = splitmix64(key + 2ULL * (uint64_t)i + 1ULL);
        double u1 = (double)((h1 >> 11) + 1ULL) * 0x1.0p-53;
        double u2 = (double)(h2 >> 11) * 0x1.0p-53;
        double z = sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
        out[i] = (float)(mean + stdv * z);
    }
}
