/* tsr_synth.c -- seeded synthetic inputs for the benchmark and the tests (not part of libtsr_hip).
 *
 * normal(seed, start, n, std): value i (i = start .. start+n-1) takes uniforms 2i and 2i+1 of the
 * counter-based SplitMix64 stream of `seed` (z_k = mix(seed + (k+1) * 0x9E3779B97F4A7C15),
 * u = (z >> 11) 2^-53) and returns f32(sqrt(-2 log1p(-u0)) cos(2 pi u1) std). Every value depends only
 * on (seed, i), so any slice can be drawn alone and CPU and GPU harnesses see identical bits. */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stddef.h>

static inline uint64_t mix(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
static inline double unif(uint64_t seed, uint64_t k) {
    return (double)(mix(seed + (k + 1u) * 0x9E3779B97F4A7C15ull) >> 11) * (1.0 / 9007199254740992.0);
}

typedef struct { uint64_t seed, start, n; float std; float * out; } job_t;

static void * run(void * p) {
    const job_t * j = (const job_t *)p;
    const double two_pi = 6.283185307179586476925286766559;
    for (uint64_t i = 0; i < j->n; ++i) {
        const uint64_t k = 2u * (j->start + i);
        const double r = sqrt(-2.0 * log1p(-unif(j->seed, k)));
        j->out[i] = (float)(r * cos(two_pi * unif(j->seed, k + 1u)) * (double)j->std);
    }
    return NULL;
}

void tsr_synth_normal(uint64_t seed, uint64_t start, uint64_t n, float std, float * out) {
    enum { NT = 16 };
    job_t jobs[NT];
    pthread_t th[NT];
    const uint64_t per = (n + NT - 1u) / NT;
    int nj = 0;
    for (uint64_t s = 0; s < n; s += per, ++nj)
        jobs[nj] = (job_t){ seed, start + s, (s + per < n ? per : n - s), std, out + s };
    if (n < 65536u || nj == 1) { for (int i = 0; i < nj; ++i) run(&jobs[i]); return; }
    for (int i = 0; i < nj; ++i) pthread_create(&th[i], NULL, run, &jobs[i]);
    for (int i = 0; i < nj; ++i) pthread_join(th[i], NULL);
}
