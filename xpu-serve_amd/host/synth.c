/* Seeded synthetic inputs, identical on every x86-64 host: splitmix64 (Steele, Lea and Flood, "Fast splittable
 * pseudorandom number generators", 2014) as a counter-based generator, and the Box-Muller transform in f64.
 * Value i of a stream is a function of (seed, i) alone, so a stream can be filled in parallel and in pieces.
 *   u1 = (mix(seed, 2i) >> 11 + 1) * 2^-53   in (0, 1]
 *   u2 = (mix(seed, 2i + 1) >> 11) * 2^-53   in [0, 1)
 *   z  = sqrt(-2 ln u1) * cos(2 pi u2)
 * mix(seed, k) is splitmix64's output for state seed + (k + 1) * 0x9E3779B97F4A7C15. */
#include <math.h>
#include <stdint.h>

static inline uint64_t mix(uint64_t seed, uint64_t k) {
    uint64_t z = seed + (k + 1) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

double xs_synth_normal_at(uint64_t seed, uint64_t i) {
    const double u1 = (double)((mix(seed, 2 * i) >> 11) + 1) * 0x1.0p-53;
    const double u2 = (double)(mix(seed, 2 * i + 1) >> 11) * 0x1.0p-53;
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586476925286766559 * u2);
}

/* out[j] = fl32(mean + stddev * z(offset + j)), j < n. */
void xs_synth_normal_f32(uint64_t seed, uint64_t offset, int64_t n, double mean, double stddev, float* out) {
#pragma omp parallel for schedule(static)
    for (int64_t j = 0; j < n; ++j) out[j] = (float)(mean + stddev * xs_synth_normal_at(seed, offset + (uint64_t)j));
}

/* Raw 64-bit draws (for picking indices): out[j] = mix(seed, offset + j). */
void xs_synth_u64(uint64_t seed, uint64_t offset, int64_t n, uint64_t* out) {
#pragma omp parallel for schedule(static)
    for (int64_t j = 0; j < n; ++j) out[j] = mix(seed, offset + (uint64_t)j);
}
