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

/* ---- seeded weights, quantized on the host ------------------------------------------------------
 * tsr_synth_quant: rows r0 .. r0+n_rows-1 of an N(0, std^2) [*, K] matrix drawn as
 * normal(seed, r * K, K, std) and quantized exactly as tsr_synth.py's quantize_q4_k / quantize_q8_0
 * (every step a single-precision operation rounded to nearest even, fp16 by RNE), on 16 threads. */
static uint16_t f32_to_f16(float f) {
    union { float f; uint32_t u; } v = { f };
    const uint32_t u = v.u, sign = (u >> 16) & 0x8000u, a = u & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return (uint16_t)(sign | 0x7E00u);
    if (a >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);      /* rounds to >= 65520: inf */
    if (a < 0x38800000u) {                                          /* half subnormal or zero */
        if (a < 0x33000000u) return (uint16_t)sign;                 /* < 2^-25: rounds to 0 */
        const uint32_t e = a >> 23, m = (a & 0x7FFFFFu) | 0x800000u;
        const uint32_t sh = 126u - e;                               /* value = m 2^(e-150); unit 2^-24 */
        uint32_t q = m >> sh;
        const uint32_t rem = m & ((1u << sh) - 1u), half = 1u << (sh - 1u);
        if (rem > half || (rem == half && (q & 1u))) ++q;
        return (uint16_t)(sign | q);
    }
    uint32_t h = ((a >> 13) - (112u << 10));
    const uint32_t rem = a & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
    return (uint16_t)(sign | h);
}

static float f16_to_f32(uint16_t h) {                               /* exact */
    const uint32_t s = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 31u, m = h & 1023u;
    union { uint32_t u; float f; } c;
    if (e == 0u) {
        c.f = (float)m * 5.9604644775390625e-08f;                  /* m 2^-24 */
        c.u |= s;
    } else {
        c.u = s | (e == 31u ? 0x7F800000u | (m << 13) : ((e + 112u) << 23) | (m << 13));
    }
    return c.f;
}

static void q4k_block(const float * x, uint8_t * o) {
    float step[8], mins[8], smax = 0.0f, mmax = 0.0f;
    for (int j = 0; j < 8; ++j) {
        float mn = x[32 * j], mx = x[32 * j];
        for (int i = 1; i < 32; ++i) { const float v = x[32 * j + i]; mn = v < mn ? v : mn; mx = v > mx ? v : mx; }
        const float lo = mn < 0.0f ? mn : 0.0f, hi = mx > lo ? mx : lo;
        step[j] = (hi - lo) / 15.0f;
        mins[j] = -lo;
        if (j == 0 || step[j] > smax) smax = step[j];
        if (j == 0 || mins[j] > mmax) mmax = mins[j];
    }
    const uint16_t dh = f32_to_f16(smax / 63.0f), mh = f32_to_f16(mmax / 63.0f);
    const float d32 = f16_to_f32(dh), m32 = f16_to_f32(mh);
    uint8_t sc[8], mnq[8], q[256];
    for (int j = 0; j < 8; ++j) {
        float a = d32 > 0.0f ? rintf(step[j] / d32) : 0.0f;
        float b = m32 > 0.0f ? rintf(mins[j] / m32) : 0.0f;
        a = a < 0.0f ? 0.0f : (a > 63.0f ? 63.0f : a);
        b = b < 0.0f ? 0.0f : (b > 63.0f ? 63.0f : b);
        sc[j] = (uint8_t)a;
        mnq[j] = (uint8_t)b;
        const float eff = d32 * (float)sc[j], off = m32 * (float)mnq[j];
        for (int i = 0; i < 32; ++i) {
            float v = eff > 0.0f ? rintf((x[32 * j + i] + off) / eff) : 0.0f;
            v = v < 0.0f ? 0.0f : (v > 15.0f ? 15.0f : v);
            q[32 * j + i] = (uint8_t)v;
        }
    }
    o[0] = (uint8_t)dh; o[1] = (uint8_t)(dh >> 8);
    o[2] = (uint8_t)mh; o[3] = (uint8_t)(mh >> 8);
    for (int j = 0; j < 4; ++j) {
        o[4 + j] = (uint8_t)((sc[j] & 63u) | ((sc[4 + j] >> 4) << 6));
        o[8 + j] = (uint8_t)((mnq[j] & 63u) | ((mnq[4 + j] >> 4) << 6));
        o[12 + j] = (uint8_t)((sc[4 + j] & 15u) | ((mnq[4 + j] & 15u) << 4));
    }
    for (int g = 0; g < 4; ++g)
        for (int i = 0; i < 32; ++i) o[16 + 32 * g + i] = (uint8_t)(q[64 * g + i] | (q[64 * g + 32 + i] << 4));
}

static float round_half_away(float v) {
    const float t = truncf(v), fr = v - t;
    return fabsf(fr) >= 0.5f ? t + (v > 0.0f ? 1.0f : -1.0f) : t;
}

static void q80_block(const float * x, uint8_t * o) {
    float amax = 0.0f;
    for (int i = 0; i < 32; ++i) { const float a = fabsf(x[i]); amax = a > amax ? a : amax; }
    const float d = amax / 127.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
    const uint16_t h = f32_to_f16(d);
    o[0] = (uint8_t)h; o[1] = (uint8_t)(h >> 8);
    for (int i = 0; i < 32; ++i) {
        float q = round_half_away(x[i] * id);
        q = q < -128.0f ? -128.0f : (q > 127.0f ? 127.0f : q);
        o[2 + i] = (uint8_t)(int8_t)q;
    }
}

typedef struct { uint64_t seed, K, r0, n; float std; int fmt; uint8_t * out; } qjob_t;

static void * qrun(void * p) {
    const qjob_t * j = (const qjob_t *)p;
    const uint64_t bs = j->fmt ? 256u : 32u, bb = j->fmt ? 144u : 34u, row_bytes = j->K / bs * bb;
    float xs[32768];
    for (uint64_t r = 0; r < j->n; ++r) {
        job_t g = { j->seed, (j->r0 + r) * j->K, j->K, j->std, xs };
        run(&g);
        uint8_t * o = j->out + r * row_bytes;
        for (uint64_t b = 0; b < j->K / bs; ++b)
            if (j->fmt) q4k_block(xs + b * bs, o + b * bb); else q80_block(xs + b * bs, o + b * bb);
    }
    return NULL;
}

/* fmt 0 = Q8_0, 1 = Q4_K; K <= 32768 and a multiple of the block; out holds n_rows rows. */
int tsr_synth_quant(int fmt, uint64_t seed, uint64_t K, uint64_t r0, uint64_t n_rows, float std, uint8_t * out) {
    enum { NT = 16 };
    const uint64_t bs = fmt ? 256u : 32u, bb = fmt ? 144u : 34u;
    if (K == 0u || K > 32768u || K % bs) return -1;
    qjob_t jobs[NT];
    pthread_t th[NT];
    const uint64_t per = (n_rows + NT - 1u) / NT;
    int nj = 0;
    for (uint64_t s = 0; s < n_rows; s += per, ++nj)
        jobs[nj] = (qjob_t){ seed, K, r0 + s, (s + per < n_rows ? per : n_rows - s), std, fmt, out + s * (K / bs * bb) };
    for (int i = 0; i < nj; ++i) pthread_create(&th[i], NULL, qrun, &jobs[i]);
    for (int i = 0; i < nj; ++i) pthread_join(th[i], NULL);
    return 0;
}
