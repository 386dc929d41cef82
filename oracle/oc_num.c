/* oc_num.c -- oracle: spec f32 rules, fp16 conversions, QACT, Q8_0 / Q4_K row dot products,
 * MUL_MAT. TEST INFRASTRUCTURE ONLY (see oc.h). Each function names the reference lines it restates. */
#include "oc.h"

#include <float.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#if !defined(FLT_EVAL_METHOD) || FLT_EVAL_METHOD != 0
#error "the oracle needs single-precision evaluation"
#endif
#if defined(__FAST_MATH__)
#error "the oracle must not be built with fast-math"
#endif

typedef union { float f; uint32_t u; } fu32;

static inline uint32_t bits_of(float f) { fu32 v; v.f = f; return v.u; }
static inline float    flt_of(uint32_t u) { fu32 v; v.u = u; return v.f; }

/* DAZ: an encoding with a zero exponent field is a signed zero (sw/sim/tsr_ref.c:54-57). */
static inline float in_daz(float x) {
    const uint32_t u = bits_of(x);
    return (u & 0x7F800000u) ? x : flt_of(u & 0x80000000u);
}

/* Result rule: a NaN becomes 0x7FC00000, a subnormal rounded result a signed zero
 * (sw/sim/tsr_ref.c:59-71; docs/spec.md:1405-1418). */
static inline float out_fix(float r) {
    const uint32_t u = bits_of(r);
    const uint32_t e = u & 0x7F800000u;
    if (e == 0x7F800000u) return (u & 0x007FFFFFu) ? flt_of(OC_NAN_BITS) : r;
    if (e == 0) return flt_of(u & 0x80000000u);
    return r;
}

float oc_fadd(float a, float b) { return out_fix(in_daz(a) + in_daz(b)); }
float oc_fsub(float a, float b) { return out_fix(in_daz(a) - in_daz(b)); }
float oc_fmul(float a, float b) { return out_fix(in_daz(a) * in_daz(b)); }
float oc_fdiv(float a, float b) { return out_fix(in_daz(a) / in_daz(b)); }
float oc_frecip(float a)        { return out_fix(1.0f / in_daz(a)); }
float oc_fsqrt(float a)         { return out_fix(sqrtf(in_daz(a))); }

/* int32 -> f32 with round-to-nearest-even (sw/sim/tsr_ref.c:107-132). The host's conversion
 * instruction rounds with the default (RNE) mode, which the oracle never changes. */
float oc_i2f(int32_t v) { return (float)v; }

/* fp16 -> f32, exact; NaN keeps sign and payload and gets the quiet bit (sw/sim/tsr_ref.c:136-160). */
float oc_h2f(uint16_t h) {
    const uint32_t s = (uint32_t)(h >> 15) << 31;
    const uint32_t e = (h >> 10) & 31u;
    const uint32_t m = h & 1023u;
    if (e == 31u) return flt_of(s | 0x7F800000u | (m ? (0x00400000u | (m << 13)) : 0u));
    if (e == 0u) {
        /* m * 2^-24 is exact in f32 (m < 2^10) */
        const float v = (float)m * 5.9604644775390625e-08f;
        return flt_of(s | bits_of(v));
    }
    return flt_of(s | ((e + 112u) << 23) | (m << 13));
}

/* f32 -> fp16 with RNE, overflow to Inf, NaN to sign | 0x7E00 (sw/sim/tsr_ref.c:162-198). The value
 * is taken apart as sig * 2^(e-23) with sig the 24-bit significand and rounded to the fp16 grid of
 * its binade (2^-24 below 2^-14). */
uint16_t oc_f2h(float f) {
    const uint32_t u = bits_of(f);
    const uint16_t s = (uint16_t)((u >> 16) & 0x8000u);
    const uint32_t a = u & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return (uint16_t)(s | 0x7E00u);
    if (a == 0x7F800000u) return (uint16_t)(s | 0x7C00u);
    const int be = (int)(a >> 23);
    if (be == 0) return s;                       /* zero or f32 subnormal */
    const int e = be - 127;
    if (e > 15) return (uint16_t)(s | 0x7C00u);
    const uint64_t sig = 0x00800000u | (a & 0x007FFFFFu);
    /* grid exponent: the fp16 ulp is 2^(e-10) for normals, 2^-24 for subnormals */
    const int ulp_e = e >= -14 ? e - 10 : -24;
    const int sh = (e - 23) - ulp_e;             /* value / ulp = sig * 2^sh, sh < 0 */
    const int rs = -sh;                          /* right shift of sig, 13 .. 48 */
    if (rs > 40) return s;                       /* far below half an ulp */
    uint64_t q = sig >> rs;
    const uint64_t rem = sig & ((1ull << rs) - 1u);
    const uint64_t half = 1ull << (rs - 1);
    if (rem > half || (rem == half && (q & 1u))) q += 1u;
    /* q counts ulps of the binade; fold it back into an fp16 encoding */
    uint32_t out;
    if (e >= -14) out = ((uint32_t)(e + 15) << 10) + (uint32_t)(q - 1024u);   /* q in [1024, 2048] */
    else out = (uint32_t)q;                                                   /* subnormal (may reach 0x400) */
    return (uint16_t)(s | out);
}

/* QACT's f32 -> int8 (sw/sim/tsr_ref.c:200-232): NaN -> 0, saturate to [-128, 127]; A32 rounds
 * half away from zero, A256 half to even. */
static int32_t sat8(double r) { return r < -128.0 ? -128 : (r > 127.0 ? 127 : (int32_t)r); }
int32_t oc_round_away8(float x) {
    if (isnan(x)) return 0;
    if (fabsf(x) >= 256.0f) return x < 0 ? -128 : 127;
    return sat8((double)roundf(x));
}
int32_t oc_round_even8(float x) {
    if (isnan(x)) return 0;
    if (fabsf(x) >= 256.0f) return x < 0 ? -128 : 127;
    return sat8((double)nearbyintf(x));          /* default mode: nearest, ties to even */
}

/* 16 partials -> y by the fixed pairwise tree (sw/sim/tsr_ref.c:592-598; docs/spec.md:470-477). */
float oc_tree16(const float p[16]) {
    float v[16];
    memcpy(v, p, sizeof v);
    for (int w = 16; w > 1; w /= 2)
        for (int k = 0; k < w / 2; ++k) v[k] = oc_fadd(v[2 * k], v[2 * k + 1]);
    return v[0];
}

/* ---- QA image (sw/sim/tsr_ref.c:418-447; docs/spec.md:402-409) ---------------------------- */
static uint32_t cdiv(uint32_t a, uint32_t b) { return (a + b - 1u) / b; }
static uint32_t qa_bsz(uint32_t kind) { return kind == OC_QA_A32 ? 32u : 256u; }

uint32_t oc_qa_d_off(uint32_t kind, uint32_t K) { (void)kind; return cdiv(K, 64u) * 64u; }
uint32_t oc_qa_bs_off(uint32_t kind, uint32_t K) {
    return oc_qa_d_off(kind, K) + cdiv(4u * (K / qa_bsz(kind)), 64u) * 64u;
}
uint32_t oc_qa_bytes(uint32_t kind, uint32_t K) {
    return oc_qa_bs_off(kind, K) + (kind == OC_QA_A256 ? cdiv(2u * (K / 16u), 64u) * 64u : 0u);
}

static void put32(uint8_t * p, uint32_t v) { for (int i = 0; i < 4; ++i) p[i] = (uint8_t)(v >> (8 * i)); }
static uint32_t get32(const uint8_t * p) { return p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 | (uint32_t)p[3] << 24; }
static int16_t geti16(const uint8_t * p) { return (int16_t)(uint16_t)(p[0] | p[1] << 8); }

/* |DAZ(x)| as bits, and whether x enters the amax search (NaN does not). For the remaining values
 * the unsigned order of the bits is the order of the magnitudes. */
static int mag_of(float x, uint32_t * m) {
    *m = bits_of(in_daz(x)) & 0x7FFFFFFFu;
    return *m <= 0x7F800000u;
}

/* QACT (sw/sim/tsr_ref.c:456-520; docs/spec.md:411-425, 1419-1430). */
void oc_qact(uint32_t kind, const float * x, uint32_t K, uint8_t * qa) {
    const uint32_t bs = qa_bsz(kind), nb = K / bs;
    memset(qa, 0, oc_qa_bytes(kind, K));
    int8_t * q = (int8_t *)qa;
    uint8_t * dreg = qa + oc_qa_d_off(kind, K);
    uint8_t * bsreg = qa + oc_qa_bs_off(kind, K);
    for (uint32_t b = 0; b < nb; ++b) {
        const float * xb = x + (size_t)b * bs;
        int8_t * qb = q + (size_t)b * bs;
        uint32_t best = 0;
        int at = -1;
        for (uint32_t j = 0; j < bs; ++j) {
            uint32_t m;
            if (mag_of(xb[j], &m) && m > best) { best = m; at = (int)j; }   /* first largest */
        }
        if (kind == OC_QA_A32) {
            const float d = oc_fdiv(flt_of(best), 127.0f);
            const float id = (bits_of(d) & 0x7FFFFFFFu) ? oc_frecip(d) : 0.0f;
            for (uint32_t j = 0; j < bs; ++j) qb[j] = (int8_t)oc_round_away8(oc_fmul(xb[j], id));
            put32(dreg + 4u * b, bits_of(oc_h2f(oc_f2h(d))));
        } else {
            float d = 0.0f;
            if (best != 0) {
                const float iscale = oc_fdiv(-127.0f, in_daz(xb[at]));
                for (uint32_t j = 0; j < bs; ++j) qb[j] = (int8_t)oc_round_even8(oc_fmul(iscale, xb[j]));
                d = oc_frecip(iscale);
            }
            put32(dreg + 4u * b, bits_of(d));
            for (uint32_t g = 0; g < bs / 16u; ++g) {
                int32_t s = 0;
                for (uint32_t l = 0; l < 16u; ++l) s += qb[16u * g + l];
                const uint16_t v = (uint16_t)(int16_t)s;
                bsreg[2u * (b * 16u + g)] = (uint8_t)v;
                bsreg[2u * (b * 16u + g) + 1u] = (uint8_t)(v >> 8);
            }
        }
    }
}

/* ---- MVM (sw/sim/tsr_ref.c:525-635) -------------------------------------------------------- */
/* Q4_K 6-bit scale / min of sub-block j from the 12 packed bytes (sw/sim/tsr_ref.c:359-367). */
static void q4k_scale_min(const uint8_t * sc12, int j, int32_t * sc, int32_t * mn) {
    if (j < 4) {
        *sc = sc12[j] & 63;
        *mn = sc12[j + 4] & 63;
    } else {
        *sc = (sc12[j + 4] & 15) | ((sc12[j - 4] >> 6) << 4);
        *mn = (sc12[j + 4] >> 4) | ((sc12[j] >> 6) << 4);
    }
}

static int32_t q8_isum(const uint8_t * blk, const int8_t * qx) {
    const int8_t * qw = (const int8_t *)(blk + 2);
    int32_t s = 0;
    for (int l = 0; l < 32; ++l) s += (int32_t)qw[l] * qx[l];
    return s;
}

/* isum / msum of one Q4_K super-block (sw/sim/tsr_ref.c:543-567): sub-block j holds the low
 * nibbles (j even) or the high nibbles (j odd) of quant bytes [32 (j/2), 32 (j/2) + 32). */
static void q4k_isum(const uint8_t * blk, const int8_t * qx, const uint8_t * bs16, int32_t * is, int32_t * ms) {
    const uint8_t * qs = blk + 16;
    int32_t a = 0, m = 0;
    for (int j = 0; j < 8; ++j) {
        const uint8_t * qq = qs + 32 * (j / 2);
        const int shift = (j & 1) ? 4 : 0;
        int32_t s = 0;
        for (int l = 0; l < 32; ++l) s += (int32_t)((qq[l] >> shift) & 15) * qx[32 * j + l];
        int32_t sc, mn;
        q4k_scale_min(blk + 4, j, &sc, &mn);
        a += sc * s;
        m += mn * ((int32_t)geti16(bs16 + 4 * j) + (int32_t)geti16(bs16 + 4 * j + 2));
    }
    *is = a;
    *ms = m;
}

static uint16_t get16(const uint8_t * p) { return (uint16_t)(p[0] | p[1] << 8); }

float oc_dot_row(uint32_t fmt, const uint8_t * row, uint32_t K, const uint8_t * qa) {
    float p[16];
    for (int i = 0; i < 16; ++i) p[i] = 0.0f;
    const int8_t * qx = (const int8_t *)qa;
    if (fmt == OC_FMT_Q8_0) {
        const uint8_t * dreg = qa + oc_qa_d_off(OC_QA_A32, K);
        for (uint32_t i = 0; i < K / 32u; ++i) {
            const uint8_t * blk = row + 34u * i;
            const float dx = flt_of(get32(dreg + 4u * i));
            const float t = oc_fmul(oc_fmul(oc_h2f(get16(blk)), dx), oc_i2f(q8_isum(blk, qx + 32u * i)));
            p[i & 15u] = oc_fadd(p[i & 15u], t);
        }
    } else {
        const uint8_t * dreg = qa + oc_qa_d_off(OC_QA_A256, K);
        const uint8_t * bsreg = qa + oc_qa_bs_off(OC_QA_A256, K);
        for (uint32_t i = 0; i < K / 256u; ++i) {
            const uint8_t * blk = row + 144u * i;
            const float dx = flt_of(get32(dreg + 4u * i));
            int32_t is, ms;
            q4k_isum(blk, qx + 256u * i, bsreg + 32u * i, &is, &ms);
            const float t1 = oc_fmul(oc_fmul(oc_h2f(get16(blk)), dx), oc_i2f(is));
            const float t2 = oc_fmul(oc_fmul(oc_h2f(get16(blk + 2)), dx), oc_i2f(ms));
            p[i & 15u] = oc_fadd(p[i & 15u], oc_fsub(t1, t2));
        }
    }
    return oc_tree16(p);
}

void oc_row_isums(uint32_t fmt, const uint8_t * row, uint32_t K, const uint8_t * qa, int32_t * out) {
    const int8_t * qx = (const int8_t *)qa;
    if (fmt == OC_FMT_Q8_0) {
        for (uint32_t i = 0; i < K / 32u; ++i) out[i] = q8_isum(row + 34u * i, qx + 32u * i);
    } else {
        const uint8_t * bsreg = qa + oc_qa_bs_off(OC_QA_A256, K);
        for (uint32_t i = 0; i < K / 256u; ++i)
            q4k_isum(row + 144u * i, qx + 256u * i, bsreg + 32u * i, &out[2 * i], &out[2 * i + 1]);
    }
}

/* ---- MUL_MAT (sw/ctrl/ref/mulmat_ref.cpp:43-63; ACC as sw/sim/tsr_sim.c:1652-1658) --------- */
typedef struct mm_job {
    uint32_t fmt, N, K, lo, hi;
    const uint8_t * w;
    const uint8_t * qa;
    const float * add;
    float * y;
} mm_job;

static size_t row_bytes(uint32_t fmt, uint32_t K) { return fmt == OC_FMT_Q8_0 ? (size_t)K / 32u * 34u : (size_t)K / 256u * 144u; }

static void * mm_rows(void * arg) {
    const mm_job * j = (const mm_job *)arg;
    const size_t rb = row_bytes(j->fmt, j->K);
    for (uint32_t n = j->lo; n < j->hi; ++n) {
        const float v = oc_dot_row(j->fmt, j->w + (size_t)n * rb, j->K, j->qa);
        j->y[n] = j->add ? oc_fadd(j->add[n], v) : v;
    }
    return NULL;
}

void oc_mul_mat(uint32_t fmt, const uint8_t * w, uint32_t N, uint32_t K, const float * x, uint32_t T,
                uint64_t x_stride, const float * add, uint64_t add_stride, float * y, uint64_t y_stride,
                uint32_t threads) {
    const uint32_t kind = fmt == OC_FMT_Q8_0 ? OC_QA_A32 : OC_QA_A256;
    uint8_t * qa = (uint8_t *)aligned_alloc(64, oc_qa_bytes(kind, K));
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    for (uint32_t t = 0; t < T; ++t) {
        oc_qact(kind, x + (size_t)t * x_stride, K, qa);
        const float * a = add ? add + (size_t)t * add_stride : NULL;
        float * yt = y + (size_t)t * y_stride;
        mm_job jobs[256];
        pthread_t th[256];
        const uint32_t per = (N + threads - 1u) / threads;
        uint32_t nj = 0;
        for (uint32_t lo = 0; lo < N; lo += per) {
            jobs[nj] = (mm_job){ fmt, N, K, lo, lo + per < N ? lo + per : N, w, qa, a, yt };
            ++nj;
        }
        if (nj == 1) {
            mm_rows(&jobs[0]);
        } else {
            for (uint32_t i = 0; i < nj; ++i) pthread_create(&th[i], NULL, mm_rows, &jobs[i]);
            for (uint32_t i = 0; i < nj; ++i) pthread_join(th[i], NULL);
        }
    }
    free(qa);
}

/* ---- batch entry points for the Python tests (one ctypes call per array) --------------------- */
void oc_fop_n(int op, const float * a, const float * b, float * out, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        switch (op) {
            case 0: out[i] = oc_fadd(a[i], b[i]); break;
            case 1: out[i] = oc_fsub(a[i], b[i]); break;
            case 2: out[i] = oc_fmul(a[i], b[i]); break;
            case 3: out[i] = oc_fdiv(a[i], b[i]); break;
            default: out[i] = oc_frecip(a[i]); break;
        }
    }
}
void oc_f2h_n(const float * x, uint16_t * out, size_t n) { for (size_t i = 0; i < n; ++i) out[i] = oc_f2h(x[i]); }
void oc_h2f_n(const uint16_t * h, float * out, size_t n) { for (size_t i = 0; i < n; ++i) out[i] = oc_h2f(h[i]); }
void oc_i2f_n(const int32_t * v, float * out, size_t n) { for (size_t i = 0; i < n; ++i) out[i] = oc_i2f(v[i]); }
void oc_round8_n(int even, const float * x, int32_t * out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = even ? oc_round_even8(x[i]) : oc_round_away8(x[i]);
}
/* QA images of T token rows (x rows at x_stride floats), image t at qa + t * oc_qa_bytes. */
void oc_qact_n(uint32_t kind, const float * x, uint32_t K, uint32_t T, uint64_t x_stride, uint8_t * qa) {
    for (uint32_t t = 0; t < T; ++t) oc_qact(kind, x + (size_t)t * x_stride, K, qa + (size_t)t * oc_qa_bytes(kind, K));
}
/* Integer sums of N rows against one QA image: out[n][...] as oc_row_isums. */
void oc_isums_n(uint32_t fmt, const uint8_t * w, uint32_t N, uint32_t K, const uint8_t * qa, int32_t * out) {
    const size_t rb = fmt == OC_FMT_Q8_0 ? (size_t)K / 32u * 34u : (size_t)K / 256u * 144u;
    const size_t per = fmt == OC_FMT_Q8_0 ? K / 32u : 2u * (K / 256u);
    for (uint32_t n = 0; n < N; ++n) oc_row_isums(fmt, w + (size_t)n * rb, K, qa, out + (size_t)n * per);
}
