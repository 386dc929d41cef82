/* oc_attn.c -- oracle: the device EXP, the AT ops and the composite flash attention on a q8_0
 * KV cache. TEST INFRASTRUCTURE ONLY (see oc.h). Fixed configuration: C = 4, PCAP = 9344, T_MAX = 1. */
#define _GNU_SOURCE
#include "oc.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

typedef union { float f; uint32_t u; } fu32;
static inline uint32_t bits_of(float f) { fu32 v; v.f = f; return v.u; }
static inline float    flt_of(uint32_t u) { fu32 v; v.u = u; return v.f; }
static inline uint32_t daz_bits(uint32_t u) { return (u & 0x7F800000u) ? u : (u & 0x80000000u); }
static inline int      isnan_bits(uint32_t u) { return (u & 0x7FFFFFFFu) > 0x7F800000u; }
static inline int      nonfinite_bits(uint32_t u) { return (u & 0x7F800000u) == 0x7F800000u; }
static inline uint16_t get16(const uint8_t * p) { return (uint16_t)(p[0] | p[1] << 8); }
static inline uint32_t get32(const uint8_t * p) { return p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 | (uint32_t)p[3] << 24; }

/* ---- EXPK (sw/sim/tsr_ref_math.c:53-159; VU section 6.3) -----------------------------------
 * exp(v) = 2^(v log2 e). |v| log2 e is formed in fixed point with 32 fraction bits from the
 * constant LK = round(log2(e) 2^38); its fraction F picks T64[F >> 26] = round(2^(j/64) 2^30) and
 * the rest G = F mod 2^26 enters a cubic 2^(G 2^-32) - 1 with coefficients round(ln2^k / k! 2^32)
 * evaluated by truncating Horner steps; the product is rounded to 24 bits (RNE). The constants are
 * computed here from their definitions (long double, 64-bit significand; the tests compare the
 * resulting EXP against the reference library bit for bit). */
static uint64_t ek_lk, ek_c1, ek_c2, ek_c3;
static uint32_t ek_t64[64];
static pthread_once_t ek_once = PTHREAD_ONCE_INIT;

static void ek_init(void) {
    const long double ln2 = M_LN2l, log2e = M_LOG2El;
    ek_lk = (uint64_t)llroundl(ldexpl(log2e, 38));
    ek_c1 = (uint64_t)llroundl(ldexpl(ln2, 32));
    ek_c2 = (uint64_t)llroundl(ldexpl(ln2 * ln2 / 2.0L, 32));
    ek_c3 = (uint64_t)llroundl(ldexpl(ln2 * ln2 * ln2 / 6.0L, 32));
    for (int j = 0; j < 64; ++j) ek_t64[j] = (uint32_t)llroundl(ldexpl(exp2l((long double)j / 64.0L), 30));
}

float oc_expk(float v) {
    pthread_once(&ek_once, ek_init);
    const uint32_t u = daz_bits(bits_of(v));
    if (isnan_bits(u)) return flt_of(OC_NAN_BITS);
    const int neg = (int)(u >> 31);
    const uint32_t a = u & 0x7FFFFFFFu;
    const float big = neg ? 0.0f : flt_of(0x7F800000u);    /* saturated result */
    if (a == 0x7F800000u) return big;
    if (a == 0) return 1.0f;
    const uint32_t ev = a >> 23;
    if (ev > 156u) return big;
    const uint64_t mv = 0x00800000u | (a & 0x007FFFFFu);
    const uint32_t sh = 156u - ev;                          /* |v| log2(e) 2^32 = mv lk 2^(ev-156) */
    const uint64_t T = sh >= 64u ? 0u : (mv * ek_lk) >> sh;
    if (T >= (1ull << 40)) return big;
    int32_t n;
    uint32_t F;
    if (neg) { n = -(int32_t)((T + 0xFFFFFFFFull) >> 32); F = (uint32_t)(0u - (uint32_t)T); }
    else     { n = (int32_t)(T >> 32);                     F = (uint32_t)T; }
    const uint64_t G = F & 0x03FFFFFFu;
    const uint64_t pf = (G * (ek_c1 + ((G * (ek_c2 + ((G * ek_c3) >> 32))) >> 32))) >> 32;
    const uint64_t t = ek_t64[F >> 26];
    const uint64_t M = t + ((t * pf) >> 32);                /* 2^frac in Q1.30 */
    uint32_t drop = 7u;
    if (M >= (1ull << 31)) { drop = 8u; n += 1; }
    uint64_t sig = M >> drop;
    const uint64_t rem = M & ((1ull << drop) - 1u), half = 1ull << (drop - 1u);
    if (rem > half || (rem == half && (sig & 1u))) sig += 1u;
    if (sig == (1ull << 24)) { sig >>= 1; n += 1; }
    const int32_t be = n + 127;
    if (be >= 255) return flt_of(0x7F800000u);
    if (be <= 0) return 0.0f;
    return flt_of(((uint32_t)be << 23) | (uint32_t)(sig & 0x007FFFFFu));
}

/* ---- MAXT, CTREE (sw/sim/tsr_ref_at.c:286-292, 588-598) ------------------------------------ */
float oc_maxt(float a, float b) {
    const uint32_t ua = daz_bits(bits_of(a)), ub = daz_bits(bits_of(b));
    if (isnan_bits(ua) || isnan_bits(ub)) return flt_of(OC_NAN_BITS);
    /* a total order on the bit patterns: negatives reversed below the positives, -0 < +0 */
    const uint32_t ka = (ua >> 31) ? ~ua : (ua ^ 0x80000000u);
    const uint32_t kb = (ub >> 31) ? ~ub : (ub ^ 0x80000000u);
    return flt_of(ka >= kb ? ua : ub);
}

float oc_ctree(const float * x, uint32_t n) {
    float v[16];
    for (uint32_t i = 0; i < n; ++i) v[i] = x[i];
    while (n > 1u) {
        const uint32_t m = (n + 1u) / 2u;
        for (uint32_t k = 0; k < n / 2u; ++k) v[k] = oc_fadd(v[2u * k], v[2u * k + 1u]);
        if (n & 1u) v[m - 1u] = v[n - 1u];
        n = m;
    }
    return v[0];
}

/* ---- block floating point (sw/sim/tsr_ref_at.c:380-488; AT section 6.4) -------------------- */
/* RNE_int(w 2^(23-es)) of a finite w with exponent <= es; zero / subnormal w gives 0. */
int32_t oc_bf_int(float w, int32_t es) {
    const uint32_t u = bits_of(w), e = (u >> 23) & 0xFFu;
    if (e == 0u) return 0;
    const uint32_t m = 0x00800000u | (u & 0x007FFFFFu);
    const int32_t sh = es - ((int32_t)e - 127);
    uint32_t v;
    if (sh == 0) v = m;
    else if (sh >= 26) v = 0;
    else {
        v = m >> sh;
        const uint32_t r = m & ((1u << sh) - 1u), h = 1u << (sh - 1);
        v += (r > h || (r == h && (v & 1u))) ? 1u : 0u;
    }
    return (u >> 31) ? -(int32_t)v : (int32_t)v;
}

/* RNE24(A) 2^k as f32; below 2^-126 a signed zero, from 2^128 a signed Inf. */
float oc_bf_f(int64_t A, int32_t k) {
    if (A == 0) return 0.0f;
    const uint32_t s = A < 0 ? 0x80000000u : 0u;
    uint64_t mag = A < 0 ? (uint64_t)0 - (uint64_t)A : (uint64_t)A;
    int32_t msb = 63 - __builtin_clzll(mag);
    int64_t e;                                   /* value = sig 2^(e - 23), sig in [2^23, 2^24) */
    if (msb > 23) {
        const int32_t sh = msb - 23;
        uint64_t sig = mag >> sh;
        const uint64_t r = mag & ((1ull << sh) - 1u), h = 1ull << (sh - 1);
        if (r > h || (r == h && (sig & 1u))) sig += 1u;
        e = (int64_t)msb + k;
        if (sig >> 24) { sig >>= 1; e += 1; }
        mag = sig;
    } else {
        mag <<= (23 - msb);
        e = (int64_t)msb + k;
    }
    if (e < -126) return flt_of(s);
    if (e > 127) return flt_of(s | 0x7F800000u);
    return flt_of(s | ((uint32_t)(e + 127) << 23) | ((uint32_t)mag & 0x007FFFFFu));
}

/* One 64-cell segment of a V slice for one row (AT 6.4 steps 2-7; sw/sim/tsr_ref_at.c:450-488).
 * w[k][e] = p_k (*) dV of block e of cell k; q[k][e] = that block's 32 quants. */
static void pv_seg(uint32_t n, const float (*w)[2], const int8_t * const (*q)[2], float c[64]) {
    int bad[2] = { 0, 0 }, any = 0;
    int32_t es = -1000;
    for (uint32_t k = 0; k < n; ++k)
        for (int e = 0; e < 2; ++e) {
            const uint32_t u = bits_of(w[k][e]);
            if (nonfinite_bits(u)) bad[e] = 1;
            else if (u & 0x7FFFFFFFu) {
                const int32_t le = (int32_t)((u >> 23) & 0xFFu) - 127;
                if (le > es) es = le;
                any = 1;
            }
        }
    int64_t acc[64];
    memset(acc, 0, sizeof acc);
    if (any)
        for (uint32_t k = 0; k < n; ++k)
            for (int e = 0; e < 2; ++e) {
                if (bad[e]) continue;
                const int64_t W = oc_bf_int(w[k][e], es);
                for (int l = 0; l < 32; ++l) acc[32 * e + l] += W * (int64_t)q[k][e][l];
            }
    for (int l = 0; l < 64; ++l)
        c[l] = bad[l >> 5] ? flt_of(OC_NAN_BITS) : (any ? oc_bf_f(acc[l], es - 23) : 0.0f);
}

/* Row-sum value of one segment's p values (AT 6.5; sw/sim/tsr_ref_at.c:490-506). */
static float lsum_seg(const float * p, uint32_t n) {
    int bad = 0, any = 0;
    int32_t ep = -1000;
    for (uint32_t k = 0; k < n; ++k) {
        const uint32_t u = daz_bits(bits_of(p[k]));
        if (nonfinite_bits(u)) bad = 1;
        else if (u & 0x7FFFFFFFu) {
            const int32_t le = (int32_t)((u >> 23) & 0xFFu) - 127;
            if (le > ep) ep = le;
            any = 1;
        }
    }
    if (bad) return flt_of(OC_NAN_BITS);
    if (!any) return 0.0f;
    int64_t S = 0;
    for (uint32_t k = 0; k < n; ++k) S += oc_bf_int(flt_of(daz_bits(bits_of(p[k]))), ep);
    return oc_bf_f(S, ep - 23);
}

/* ---- MSUM and the f32 mask copy (sw/sim/tsr_ref_at.c:646-715; AT 7.3) ---------------------- */
uint32_t oc_msum_build(const uint16_t * mask, size_t row_stride, uint32_t n_kv, uint32_t n_q, uint32_t * words) {
    int general = 0;
    for (uint32_t q = 0; q < n_q; ++q) {
        const uint16_t * m = mask + (size_t)q * row_stride;
        uint32_t * w = words + 8u + 4u * q;
        uint32_t nrun = 0;
        w[0] = w[1] = w[2] = w[3] = 0u;
        uint32_t j = 0;
        while (j < n_kv) {
            if (m[j] == 0xFC00u) { ++j; continue; }            /* -inf: invisible */
            if (m[j] & 0x7FFFu) { general = 1; ++j; continue; } /* a value other than +-0 */
            uint32_t e = j + 1u;
            while (e < n_kv && (m[e] & 0x7FFFu) == 0u) ++e;
            if (nrun < 2u) { w[2u * nrun] = j; w[2u * nrun + 1u] = e; }
            ++nrun;
            j = e;
        }
        if (nrun > 2u) general = 1;
    }
    if (general)
        for (uint32_t q = 0; q < n_q; ++q) {                    /* rows: the hull of the non -inf cells */
            const uint16_t * m = mask + (size_t)q * row_stride;
            uint32_t * w = words + 8u + 4u * q;
            uint32_t lo = 0, hi = 0;
            int seen = 0;
            for (uint32_t j = 0; j < n_kv; ++j)
                if (m[j] != 0xFC00u) { if (!seen) lo = j; seen = 1; hi = j + 1u; }
            w[0] = lo; w[1] = hi; w[2] = 0u; w[3] = 0u;
        }
    words[0] = OC_MSUM_MAGIC;
    words[1] = n_q;
    words[2] = n_kv;
    words[3] = general ? 1u : 0u;
    words[4] = words[5] = words[6] = words[7] = 0u;
    return words[3];
}

void oc_mask_f32(const uint16_t * mask, size_t row_stride, uint32_t n_kv, uint32_t n_q, float scale, float * dst) {
    const size_t w = 16u * (size_t)((n_kv + 15u) / 16u);
    for (uint32_t q = 0; q < n_q; ++q) {
        float * d = dst + (size_t)q * w;
        for (size_t j = 0; j < w; ++j)
            d[j] = j < n_kv ? oc_fdiv(oc_h2f(mask[(size_t)q * row_stride + j]), scale) : flt_of(0xFF800000u);
    }
}

/* ---- chunk planner for a one-row tile (sw/sim/include/tsr_fa_plan.h rules 1, 2, 4, 7, 8) ---- */
static uint32_t fa_ncg(uint32_t E, uint32_t D, uint32_t n_total) {
    if (D == 0u || E % D != 0u || E < D) return 0u;
    const uint64_t pc = (uint64_t)OC_C * (OC_PCAP / (16u * (E / D)));
    const uint64_t half = ((uint64_t)n_total + 1u) / 2u, c4 = 4u * OC_C;
    const uint64_t m = half <= c4 ? c4 : (half + c4 - 1u) / c4 * c4;
    uint64_t r = 128u;
    if (pc < r) r = pc;
    if (m < r) r = m;
    return (uint32_t)r;
}

long oc_fa_plan_row(uint32_t E, uint32_t D, const uint32_t * words, uint32_t q,
                    const uint32_t (*new_runs)[2], uint32_t n_new, oc_chunk * out, size_t cap) {
    const uint32_t n_kv = words[2];
    const int general = (words[3] & 1u) != 0;
    struct { uint32_t ulo, uhi; int64_t lo, hi; } sub[2];
    uint32_t nsub = 0;
    if (general) {
        if (n_kv > 0u) { sub[0].ulo = 0; sub[0].uhi = (n_kv + 15u) / 16u; sub[0].lo = 0; sub[0].hi = 0; nsub = 1; }
    } else {
        const uint32_t * w = words + 8u + 4u * q;
        if (w[0] > w[1] || w[2] > w[3] || w[1] > n_kv || w[3] > n_kv) return -2;
        if (w[1] > w[0] && w[3] > w[2] && !(w[1] <= w[2] || w[3] <= w[0])) return -2;
        uint32_t r[2][2], nr = 0;
        if (w[1] > w[0]) { r[nr][0] = w[0]; r[nr][1] = w[1]; ++nr; }
        if (w[3] > w[2]) { r[nr][0] = w[2]; r[nr][1] = w[3]; ++nr; }
        if (nr == 2 && r[1][0] < r[0][0]) {
            const uint32_t a = r[0][0], b = r[0][1];
            r[0][0] = r[1][0]; r[0][1] = r[1][1]; r[1][0] = a; r[1][1] = b;
        }
        for (uint32_t k = 0; k < nr; ++k) {
            sub[nsub].ulo = r[k][0] / 16u;
            sub[nsub].uhi = (r[k][1] + 15u) / 16u;
            sub[nsub].lo = r[k][0];
            sub[nsub].hi = r[k][1];
            ++nsub;
        }
    }
    if (nsub == 0) {                                           /* rule 8: one empty chunk */
        if (cap > 0) out[0] = (oc_chunk){ 0u, 1u, 0u, 0u, 0u };
        return 1;
    }
    uint32_t n_total = 0;
    for (uint32_t k = 0; k < nsub; ++k) n_total += sub[k].uhi - sub[k].ulo;
    const uint32_t ncg = fa_ncg(E, D, n_total);
    if (ncg == 0u) return -1;
    /* generation order, then the chunks holding a cell written in this launch at the end */
    long count = 0;
    for (int pass = 0; pass < 2; ++pass)
        for (uint32_t k = 0; k < nsub; ++k)
            for (uint32_t a = sub[k].ulo; a < sub[k].uhi; a += ncg) {
                const uint32_t b = a + ncg < sub[k].uhi ? a + ncg : sub[k].uhi;
                int has_new = 0;
                for (uint32_t i = 0; i < n_new; ++i)
                    if (new_runs[i][1] > new_runs[i][0] && new_runs[i][0] < 16ull * b && new_runs[i][1] > 16ull * a) has_new = 1;
                if (has_new != pass) continue;
                oc_chunk c;
                c.u0 = a;
                c.n_groups = b - a;
                c.general = general ? 1u : 0u;
                if (general) { c.c_lo = 0; c.c_hi = 16u * (b - a); }
                else {
                    const int64_t A = 16 * (int64_t)a, n16 = 16 * (int64_t)(b - a);
                    c.c_lo = (uint32_t)(sub[k].lo - A > 0 ? sub[k].lo - A : 0);
                    c.c_hi = (uint32_t)(sub[k].hi - A < n16 ? sub[k].hi - A : n16);
                }
                if ((size_t)count < cap) out[count] = c;
                ++count;
            }
    return count;
}

/* ---- KV store (SET_ROWS: QACT A32, fp16 of D exact; sw/ctrl/ref/kv_ref.cpp:38-43) ----------- */
void oc_kv_store_row(const float * x, uint32_t E, uint8_t * row) {
    uint8_t * qa = (uint8_t *)aligned_alloc(64, oc_qa_bytes(OC_QA_A32, E));
    oc_qact(OC_QA_A32, x, E, qa);
    const uint8_t * dreg = qa + oc_qa_d_off(OC_QA_A32, E);
    for (uint32_t b = 0; b < E / 32u; ++b) {
        const uint16_t h = oc_f2h(flt_of(get32(dreg + 4u * b)));
        row[34u * b] = (uint8_t)h;
        row[34u * b + 1u] = (uint8_t)(h >> 8);
        memcpy(row + 34u * b + 2u, qa + 32u * b, 32);
    }
    free(qa);
}

/* ---- composite flash attention (sw/sim/tsr_ref_at.c:774-860; AT 6.6) ----------------------- */
/* Score of head row h on cell `cell` (ATTQK's SEG: sw/sim/tsr_ref_at.c:294-305). */
static float att_seg(const uint8_t * krow, uint32_t g, uint32_t D, const int8_t * qx, const float * dx) {
    float p[16];
    for (int i = 0; i < 16; ++i) p[i] = 0.0f;
    for (uint32_t k = 0; k < D / 32u; ++k) {
        const uint8_t * blk = krow + 34u * (g * (D / 32u) + k);
        int32_t is = 0;
        for (int l = 0; l < 32; ++l) is += (int32_t)(int8_t)blk[2 + l] * qx[32u * k + l];
        p[k] = oc_fadd(0.0f, oc_fmul(oc_fmul(oc_h2f(get16(blk)), dx[k]), oc_i2f(is)));
    }
    return oc_tree16(p);
}

int oc_flash_attn(const float * q, uint32_t T, uint64_t q_stride, const uint8_t * kc, const uint8_t * vc,
                  uint32_t kv_size, uint32_t D, uint32_t n_head, uint32_t n_head_kv, float scale,
                  const uint32_t * msum, const float * mask_f32, const uint32_t (*new_runs)[2], uint32_t n_new,
                  float * out, uint64_t out_stride) {
    if (!(D == 64u || D == 128u || D == 256u || D == 512u)) return -1;
    if (n_head_kv == 0u || n_head % n_head_kv != 0u || n_head / n_head_kv > 64u) return -1;
    const uint32_t sb = bits_of(scale);
    if ((sb >> 31) || (sb & 0x7F800000u) == 0u || (sb & 0x7F800000u) == 0x7F800000u) return -1;
    if (msum[0] != OC_MSUM_MAGIC || msum[1] != T) return -1;
    const uint32_t n_kv = msum[2], G = n_head / n_head_kv, E = n_head_kv * D, K = n_head * D;
    if (16u * ((n_kv + 15u) / 16u) > kv_size && (msum[3] & 1u)) return -1;
    if (n_kv > kv_size) return -1;
    const size_t rowb = (size_t)E / 32u * 34u;
    const uint32_t nsl = D / 64u, mstride = 16u * ((n_kv + 15u) / 16u);
    uint8_t * qa = (uint8_t *)aligned_alloc(64, oc_qa_bytes(OC_QA_A32, K));
    float * S = (float *)malloc(sizeof(float) * (size_t)n_head * 128u * 16u);
    float * O = (float *)malloc(sizeof(float) * (size_t)n_head * D);
    float * OC = (float *)malloc(sizeof(float) * (size_t)OC_C * n_head * D);
    float * LC = (float *)malloc(sizeof(float) * (size_t)OC_C * n_head);
    float * mrun = (float *)malloc(sizeof(float) * n_head);
    float * lrun = (float *)malloc(sizeof(float) * n_head);
    float * mk = (float *)malloc(sizeof(float) * n_head);
    oc_chunk * ch = NULL;
    int rc = 0;
    for (uint32_t t = 0; t < T && rc == 0; ++t) {
        const float * qt = q + (size_t)t * q_stride;
        oc_qact(OC_QA_A32, qt, K, qa);
        const int8_t * qx = (const int8_t *)qa;
        const float * dx = (const float *)(qa + oc_qa_d_off(OC_QA_A32, K));
        const long nch = oc_fa_plan_row(E, D, msum, t, new_runs, n_new, NULL, 0);
        if (nch < 0) { rc = -2; break; }
        free(ch);
        ch = (oc_chunk *)malloc(sizeof(oc_chunk) * (size_t)nch);
        oc_fa_plan_row(E, D, msum, t, new_runs, n_new, ch, (size_t)nch);
        for (long k = 0; k < nch; ++k)
            if (ch[k].general && mask_f32 == NULL) { rc = -3; break; }
        if (rc) break;
        for (long k = 0; k < nch; ++k) {
            const oc_chunk * c = &ch[k];
            const uint32_t ncell = 16u * c->n_groups;
            /* ATTQK (+ MAXOUT, or AMASK for a GENERAL chunk), then ASMAX in place */
            for (uint32_t h = 0; h < n_head; ++h) {
                const uint32_t g = h / G;
                float * s = S + (size_t)h * ncell;
                float m = flt_of(OC_M_FLOOR);
                for (uint32_t j = 0; j < ncell; ++j) {
                    const uint32_t cell = 16u * c->u0 + j;
                    const int vis = c->general || (j >= c->c_lo && j < c->c_hi);
                    float v = vis ? att_seg(kc + (size_t)cell * rowb, g, D, qx + (size_t)h * D, dx + (size_t)h * (D / 32u))
                                  : flt_of(0xFF800000u);
                    if (c->general) {
                        const float mm = mask_f32[(size_t)t * mstride + cell];
                        v = bits_of(mm) == 0xFF800000u ? flt_of(0xFF800000u) : oc_fadd(v, mm);
                    }
                    s[j] = v;
                    m = oc_maxt(m, v);
                }
                mk[h] = m;
                for (uint32_t j = 0; j < ncell; ++j) s[j] = oc_expk(oc_fmul(oc_fsub(s[j], m), scale));
            }
            /* ATTPV with LSUM: channel ch owns groups u = ch (mod C), in segments of 4 of them */
            for (uint32_t cc = 0; cc < OC_C; ++cc) {
                uint32_t U[128], nu = 0;
                for (uint32_t u = c->u0; u < c->u0 + c->n_groups; ++u)
                    if (u % OC_C == cc) U[nu++] = u;
                for (uint32_t h = 0; h < n_head; ++h) {
                    const uint32_t g = h / G;
                    const float * p = S + (size_t)h * ncell;
                    for (uint32_t sl = 0; sl < nsl; ++sl) {
                        const uint32_t sa = g * nsl + sl;          /* slice of the cell row */
                        float acc[64];
                        for (int l = 0; l < 64; ++l) acc[l] = 0.0f;
                        for (uint32_t k0 = 0; k0 < nu; k0 += 4u) {
                            float w[64][2];
                            const int8_t * qv[64][2];
                            uint32_t n = 0;
                            for (uint32_t k1 = k0; k1 < nu && k1 < k0 + 4u; ++k1)
                                for (uint32_t rr = 0; rr < 16u; ++rr) {
                                    const uint32_t j = 16u * (U[k1] - c->u0) + rr;
                                    if ((daz_bits(bits_of(p[j])) & 0x7FFFFFFFu) == 0u) continue;
                                    const uint8_t * vrow = vc + (size_t)(16u * U[k1] + rr) * rowb;
                                    const uint8_t * b0 = vrow + 34u * (2u * sa), * b1 = vrow + 34u * (2u * sa + 1u);
                                    w[n][0] = oc_fmul(p[j], oc_h2f(get16(b0)));
                                    w[n][1] = oc_fmul(p[j], oc_h2f(get16(b1)));
                                    qv[n][0] = (const int8_t *)(b0 + 2);
                                    qv[n][1] = (const int8_t *)(b1 + 2);
                                    ++n;
                                }
                            float cseg[64];
                            pv_seg(n, (const float (*)[2])w, (const int8_t * const (*)[2])qv, cseg);
                            for (int l = 0; l < 64; ++l) acc[l] = oc_fadd(acc[l], cseg[l]);
                        }
                        memcpy(OC + ((size_t)cc * n_head + h) * D + 64u * sl, acc, sizeof acc);
                    }
                    float l = 0.0f;
                    for (uint32_t k0 = 0; k0 < nu; k0 += 4u) {
                        float ps[64];
                        uint32_t n = 0;
                        for (uint32_t k1 = k0; k1 < nu && k1 < k0 + 4u; ++k1)
                            for (uint32_t rr = 0; rr < 16u; ++rr) ps[n++] = p[16u * (U[k1] - c->u0) + rr];
                        l = oc_fadd(l, lsum_seg(ps, n));
                    }
                    LC[(size_t)cc * n_head + h] = l;
                }
            }
            /* AMERGE: CTREE over the channel partials, then INIT or the online merge */
            for (uint32_t h = 0; h < n_head; ++h) {
                float xv[OC_C];
                for (uint32_t cc = 0; cc < OC_C; ++cc) xv[cc] = LC[(size_t)cc * n_head + h];
                const float lk = oc_ctree(xv, OC_C);
                float a = 0.0f, b = 0.0f;
                if (k == 0) { lrun[h] = lk; mrun[h] = mk[h]; }
                else {
                    const float mn = oc_maxt(mrun[h], mk[h]);
                    a = oc_expk(oc_fmul(oc_fsub(mrun[h], mn), scale));
                    b = oc_expk(oc_fmul(oc_fsub(mk[h], mn), scale));
                    lrun[h] = oc_fadd(oc_fmul(lrun[h], a), oc_fmul(lk, b));
                    mrun[h] = mn;
                }
                for (uint32_t d = 0; d < D; ++d) {
                    for (uint32_t cc = 0; cc < OC_C; ++cc) xv[cc] = OC[((size_t)cc * n_head + h) * D + d];
                    const float ok = oc_ctree(xv, OC_C);
                    float * o = O + (size_t)h * D + d;
                    *o = k == 0 ? ok : oc_fadd(oc_fmul(*o, a), oc_fmul(ok, b));
                }
            }
        }
        /* ANORM */
        float * ot = out + (size_t)t * out_stride;
        for (uint32_t h = 0; h < n_head; ++h) {
            const float rinv = oc_frecip(oc_maxt(lrun[h], flt_of(OC_L_FLOOR)));
            for (uint32_t d = 0; d < D; ++d) ot[(size_t)h * D + d] = oc_fmul(O[(size_t)h * D + d], rinv);
        }
    }
    free(ch); free(qa); free(S); free(O); free(OC); free(LC); free(mrun); free(lrun); free(mk);
    return rc;
}

/* ---- batch entry points for the Python tests ------------------------------------------------ */
void oc_expk_n(const float * v, float * out, size_t n) { for (size_t i = 0; i < n; ++i) out[i] = oc_expk(v[i]); }
void oc_maxt_n(const float * a, const float * b, float * out, size_t n) { for (size_t i = 0; i < n; ++i) out[i] = oc_maxt(a[i], b[i]); }
void oc_bf_f_n(const int64_t * A, const int32_t * k, float * out, size_t n) { for (size_t i = 0; i < n; ++i) out[i] = oc_bf_f(A[i], k[i]); }
void oc_bf_int_n(const float * w, const int32_t * es, int32_t * out, size_t n) { for (size_t i = 0; i < n; ++i) out[i] = oc_bf_int(w[i], es[i]); }
/* n_rows f32 rows (src_stride floats apart) into the q8_0 cache rows idx[i]. */
void oc_kv_set_rows(const float * src, uint32_t E, uint32_t n_rows, uint64_t src_stride, const int64_t * idx, uint8_t * cache) {
    const size_t rowb = (size_t)E / 32u * 34u;
    for (uint32_t i = 0; i < n_rows; ++i) oc_kv_store_row(src + (size_t)i * src_stride, E, cache + (size_t)idx[i] * rowb);
}
