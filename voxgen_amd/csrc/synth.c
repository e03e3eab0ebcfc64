/*
 * synth.c — deterministic synthetic inputs for the BaseLM workloads.
 *
 * Every value is a pure function of (seed, element index), so the generator is
 * parallel, order-independent and identical wherever it runs:
 *   u64(seed, k)   = k-th output of splitmix64 started at `seed`
 *                    (mix(seed + (k+1) * 0x9E3779B97F4A7C15));
 *   uniform int    = multiply-high of the top 32 bits by the range;
 *   N(0,1) pairs   = Box-Muller on u64(seed, 2p) and u64(seed, 2p+1) in double.
 * Q8_0 blocks (GGUF layout, gguf.rs:41-45): d = f16(|N(0,1)| * scale_sigma),
 * q ~ U{-127..127}; scales come from stream seed^TAG_D, quants from seed^TAG_Q.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define GOLDEN 0x9E3779B97F4A7C15ull
#define TAG_D 0xD1B54A32D192ED03ull
#define TAG_Q 0x8CB92BA72F3D8DD7ull

static inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

uint64_t vs_u64(uint64_t seed, uint64_t k) { return mix64(seed + (k + 1u) * GOLDEN); }

static inline double unit_open(uint64_t r) { return ((double)(r >> 11) + 0.5) * 0x1.0p-53; }

double vs_normal(uint64_t seed, uint64_t i) {
    const uint64_t p = i >> 1;
    const double u1 = unit_open(vs_u64(seed, 2u * p));
    const double u2 = unit_open(vs_u64(seed, 2u * p + 1u));
    const double r = sqrt(-2.0 * log(u1));
    const double th = 6.283185307179586476925 * u2;
    return (i & 1u) ? r * sin(th) : r * cos(th);
}

static uint16_t f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u, exp = (x >> 23) & 0xffu, mant = x & 0x7fffffu;
    if (exp == 0xffu) return (uint16_t)(sign | 0x7c00u | (mant ? 0x200u : 0u));
    int e = (int)exp - 112;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        uint32_t m24 = mant | 0x800000u;
        int shift = 14 - e;
        uint32_t hm = m24 >> shift, rem = m24 & ((1u << shift) - 1u), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (hm & 1u))) hm++;
        return (uint16_t)(sign | hm);
    }
    uint32_t h = sign | ((uint32_t)e << 10) | (mant >> 13), rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)h;
}

void vs_fill_u64(uint64_t *dst, uint64_t n, uint64_t seed, uint64_t start) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t)n; ++i) dst[i] = vs_u64(seed, start + (uint64_t)i);
}

void vs_fill_normal_f32(float *dst, uint64_t n, uint64_t seed, float mean, float std) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t)n; ++i) dst[i] = (float)(mean + std * vs_normal(seed, (uint64_t)i));
}

void vs_fill_normal_f16(uint16_t *dst, uint64_t n, uint64_t seed, float mean, float std) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t)n; ++i)
        dst[i] = f32_to_f16((float)(mean + std * vs_normal(seed, (uint64_t)i)));
}

void vs_fill_uniform_u32(uint32_t *dst, uint64_t n, uint64_t seed, uint32_t bound) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t)n; ++i)
        dst[i] = (uint32_t)(((vs_u64(seed, (uint64_t)i) >> 32) * (uint64_t)bound) >> 32);
}

/* n_blocks Q8_0 blocks of 34 bytes: f16 scale then 32 int8 quants. */
void vs_fill_q8_0(uint8_t *dst, uint64_t n_blocks, uint64_t seed, float scale_sigma) {
    const uint64_t sd = seed ^ TAG_D, sq = seed ^ TAG_Q;
#pragma omp parallel for schedule(static)
    for (int64_t b = 0; b < (int64_t)n_blocks; ++b) {
        uint8_t *blk = dst + (uint64_t)b * 34u;
        const float d = (float)(fabs(vs_normal(sd, (uint64_t)b)) * scale_sigma);
        const uint16_t h = f32_to_f16(d);
        blk[0] = (uint8_t)(h & 0xffu);
        blk[1] = (uint8_t)(h >> 8);
        for (int j = 0; j < 32; ++j) {
            const uint64_t r = vs_u64(sq, (uint64_t)b * 32u + (uint64_t)j);
            const int q = (int)(((r >> 32) * 255u) >> 32) - 127;
            blk[2 + j] = (uint8_t)(int8_t)q;
        }
    }
}
