/* seedgen.c -- seeded synthetic weights and ids for the benchmark workloads.
 *
 * The stand-in for the reference's seeded initialiser (scripts/make_init.py
 * :47-52 of 14NGiestas/autoresearch): i.i.d. N(0, std) values, here from a
 * counter-based splitmix64 stream per tensor through Box-Muller, rounded to
 * bf16 (nearest, ties to even) and stored widened to fp32, so that fp32 and
 * bf16 consumers hold identical values. Output i of a stream depends only on
 * (seed, stream, i), so the result is independent of the thread count.
 */
#include <math.h>
#include <stdint.h>

static inline uint64_t splitmix(uint64_t base, uint64_t i) {
  uint64_t z = base + (i + 1) * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

static inline double u01(uint64_t z) { /* (0, 1] */
  return ((double)(z >> 11) + 1.0) * (1.0 / 9007199254740992.0);
}

static inline float bf16_round(float f) {
  union { float f; uint32_t u; } v = {f};
  v.u = (v.u + 0x7FFFu + ((v.u >> 16) & 1u)) & 0xFFFF0000u;
  return v.f;
}

/* out[0..n): N(0, std^2) rounded to bf16; pair p uses outputs 2p, 2p+1. */
void sg_normal_bf16(uint64_t seed, uint64_t stream, int64_t n, double std, float *out) {
  const uint64_t base = seed * (1ull << 20) + stream;
  const int64_t m = (n + 1) / 2;
#pragma omp parallel for schedule(static)
  for (int64_t p = 0; p < m; ++p) {
    const double r = sqrt(-2.0 * log(u01(splitmix(base, 2 * (uint64_t)p))));
    const double th = 6.283185307179586 * u01(splitmix(base, 2 * (uint64_t)p + 1));
    out[2 * p] = bf16_round((float)(r * cos(th) * std));
    if (2 * p + 1 < n) out[2 * p + 1] = bf16_round((float)(r * sin(th) * std));
  }
}

/* n doubles in (0, 1] of stream (seed, stream). */
void sg_uniform(uint64_t seed, uint64_t stream, int64_t n, double *out) {
  const uint64_t base = seed * (1ull << 20) + stream;
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) out[i] = u01(splitmix(base, (uint64_t)i));
}
