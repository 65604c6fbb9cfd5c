/*
 * mc_oracle.c -- CPU oracle (TEST INFRASTRUCTURE ONLY; see mc_oracle.h).
 *
 * Block layouts and dequantizers restate upstream ggml @11fe0215 [not
 * vendored by the reference; its call sites are kernels/moe-cache.cu:44-70
 * and patches/trace-hook/ggml-cpu.c:249-340].  The MUL_MAT_ID driver restates
 * patches/trace-hook/ggml-cpu.c:1492-1767; the post-op order restates
 * kernels/moe-cache.cu:240-284.
 */
#include "mc_oracle.h"

#include <immintrin.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ */
/* fp16                                                                */
/* ------------------------------------------------------------------ */

uint16_t or_fp32_to_fp16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint16_t sign = (uint16_t) ((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) {                     /* inf / nan */
        return sign | (ax > 0x7F800000u ? 0x7E00u : 0x7C00u);
    }
    if (ax >= 0x477FF000u) {                     /* >= 65520 rounds to inf */
        return sign | 0x7C00u;
    }
    if (ax >= 0x38800000u) {                     /* normal half: rebias exponent by -112, RNE on 13 dropped bits */
        const uint32_t m = ax + 0xC8000FFFu + ((ax >> 13) & 1u);
        return sign | (uint16_t) (m >> 13);
    }
    /* half subnormal (or zero): unit is 2^-24; f*2^24 is exact, round to nearest even */
    float af;
    memcpy(&af, &ax, 4);
    const uint32_t q = (uint32_t) nearbyintf(af * 16777216.0f);
    return sign | (uint16_t) q;
}

float or_fp16_to_fp32(uint16_t h) {
    const uint32_t sign = (uint32_t) (h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu;
    const uint32_t m = h & 0x3FFu;
    uint32_t bits;
    if (e == 0) {
        float v = ldexpf((float) m, -24);
        memcpy(&bits, &v, 4);
        bits |= sign;
    } else if (e == 31) {
        bits = sign | 0x7F800000u | (m << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* ------------------------------------------------------------------ */
/* block layouts                                                       */
/* ------------------------------------------------------------------ */

#pragma pack(push, 1)
typedef struct { uint16_t d; uint8_t qs[16]; } blk_q4_0;                                   /* 18 */
typedef struct { uint16_t d; uint8_t qh[4]; uint8_t qs[16]; } blk_q5_0;                    /* 22 */
typedef struct { uint16_t d; int8_t qs[32]; } blk_q8_0;                                    /* 34 */
typedef struct { uint16_t d; uint16_t s; int8_t qs[32]; } blk_q8_1;                        /* 36 */
typedef struct { uint8_t scales[16]; uint8_t qs[64]; uint16_t d; uint16_t dmin; } blk_q2_K; /* 84 */
typedef struct { uint8_t hmask[32]; uint8_t qs[64]; uint8_t scales[12]; uint16_t d; } blk_q3_K; /* 110 */
typedef struct { uint16_t d; uint16_t dmin; uint8_t scales[12]; uint8_t qs[128]; } blk_q4_K; /* 144 */
typedef struct { uint16_t d; uint16_t dmin; uint8_t scales[12]; uint8_t qh[32]; uint8_t qs[128]; } blk_q5_K; /* 176 */
typedef struct { uint8_t ql[128]; uint8_t qh[64]; int8_t scales[16]; uint16_t d; } blk_q6_K; /* 210 */
typedef struct { float d; int8_t qs[256]; int16_t bsums[16]; } blk_q8_K;                   /* 292 */
#pragma pack(pop)

_Static_assert(sizeof(blk_q4_0) == 18, "q4_0");
_Static_assert(sizeof(blk_q5_0) == 22, "q5_0");
_Static_assert(sizeof(blk_q8_0) == 34, "q8_0");
_Static_assert(sizeof(blk_q8_1) == 36, "q8_1");
_Static_assert(sizeof(blk_q2_K) == 84, "q2_K");
_Static_assert(sizeof(blk_q3_K) == 110, "q3_K");
_Static_assert(sizeof(blk_q4_K) == 144, "q4_K");
_Static_assert(sizeof(blk_q5_K) == 176, "q5_K");
_Static_assert(sizeof(blk_q6_K) == 210, "q6_K");
_Static_assert(sizeof(blk_q8_K) == 292, "q8_K");

#define H2F(h) or_fp16_to_fp32(h)
#define F2H(f) or_fp32_to_fp16(f)

int or_type_supported(int t) {
    switch (t) {
        case OR_Q4_0: case OR_Q5_0: case OR_Q8_0:
        case OR_Q2_K: case OR_Q3_K: case OR_Q4_K: case OR_Q5_K: case OR_Q6_K:
            return 1;
        default:
            return 0;
    }
}

int or_block_elems(int t) {
    switch (t) {
        case OR_Q4_0: case OR_Q5_0: case OR_Q8_0: case OR_Q8_1: return 32;
        case OR_Q2_K: case OR_Q3_K: case OR_Q4_K: case OR_Q5_K: case OR_Q6_K: case OR_Q8_K: return 256;
        case OR_F32: case OR_F16: return 1;
        default: return 0;
    }
}

size_t or_block_bytes(int t) {
    switch (t) {
        case OR_Q4_0: return 18; case OR_Q5_0: return 22; case OR_Q8_0: return 34; case OR_Q8_1: return 36;
        case OR_Q2_K: return 84; case OR_Q3_K: return 110; case OR_Q4_K: return 144;
        case OR_Q5_K: return 176; case OR_Q6_K: return 210; case OR_Q8_K: return 292;
        case OR_F32: return 4; case OR_F16: return 2;
        default: return 0;
    }
}

size_t or_row_bytes(int t, int64_t k) {
    const int be = or_block_elems(t);
    if (be == 0 || k % be) return 0;
    return (size_t) (k / be) * or_block_bytes(t);
}

/* 6-bit scale/min of sub-block j (0..7) in the 12-byte Q4_K/Q5_K scale array */
static void scale_min_k4(int j, const uint8_t *q, int *d, int *m) {
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

/* 6-bit scale j (0..15) of Q3_K, already offset by -32 */
static int scale_q3_K(int j, const uint8_t *sc) {
    const int lo = j < 8 ? (sc[j] & 0xF) : (sc[j - 8] >> 4);
    const int hi = (sc[8 + (j & 3)] >> (2 * (j >> 2))) & 3;
    return (lo | (hi << 4)) - 32;
}

/* value of element i (0..255) of a K-quant block, as an integer code, and its sub-block index */
static int q2_K_code(const blk_q2_K *b, int i) {
    const int h = i >> 7, j = (i & 127) >> 5, l = i & 31;
    return (b->qs[32 * h + l] >> (2 * j)) & 3;
}
static int q3_K_code(const blk_q3_K *b, int i) {            /* -4..3 */
    const int h = i >> 7, j = (i & 127) >> 5, l = i & 31;
    const int low = (b->qs[32 * h + l] >> (2 * j)) & 3;
    const int hb = (b->hmask[l] >> (4 * h + j)) & 1;
    return low - (hb ? 0 : 4);
}
static int q4_K_code(const blk_q4_K *b, int i) {
    const int c = i >> 6, l = i & 31, hi = (i >> 5) & 1;
    const uint8_t q = b->qs[32 * c + l];
    return hi ? (q >> 4) : (q & 0xF);
}
static int q5_K_code(const blk_q5_K *b, int i) {
    const int c = i >> 6, l = i & 31, hi = (i >> 5) & 1;
    const uint8_t q = b->qs[32 * c + l];
    const int lo = hi ? (q >> 4) : (q & 0xF);
    const int hb = (b->qh[l] >> (2 * c + hi)) & 1;
    return lo | (hb << 4);
}
static int q6_K_code(const blk_q6_K *b, int i) {            /* -32..31 */
    const int n = i >> 7, quarter = (i & 127) >> 5, l = i & 31;
    const uint8_t ql = b->ql[64 * n + 32 * (quarter & 1) + l];
    const int lo = (quarter >> 1) ? (ql >> 4) : (ql & 0xF);
    const int hb = (b->qh[32 * n + l] >> (2 * quarter)) & 3;
    return (lo | (hb << 4)) - 32;
}
/* scale (and min) of the 16- or 32-element sub-block that holds element i */
static int q6_K_scale(const blk_q6_K *b, int i) {
    const int n = i >> 7, quarter = (i & 127) >> 5, l = i & 31;
    return b->scales[8 * n + 2 * quarter + (l >> 4)];
}

void or_dequantize_row(int type, const void *vx, float *y, int64_t k) {
    const int be = or_block_elems(type);
    const int64_t nb = k / be;
    for (int64_t ib = 0; ib < nb; ++ib, y += be) {
        switch (type) {
            case OR_Q4_0: {
                const blk_q4_0 *b = (const blk_q4_0 *) vx + ib;
                const float d = H2F(b->d);
                for (int j = 0; j < 16; ++j) {
                    y[j]      = ((b->qs[j] & 0xF) - 8) * d;
                    y[j + 16] = ((b->qs[j] >> 4) - 8) * d;
                }
            } break;
            case OR_Q5_0: {
                const blk_q5_0 *b = (const blk_q5_0 *) vx + ib;
                const float d = H2F(b->d);
                uint32_t qh;
                memcpy(&qh, b->qh, 4);
                for (int j = 0; j < 16; ++j) {
                    const int h0 = (qh >> j) & 1, h1 = (qh >> (j + 16)) & 1;
                    y[j]      = (((b->qs[j] & 0xF) | (h0 << 4)) - 16) * d;
                    y[j + 16] = (((b->qs[j] >> 4) | (h1 << 4)) - 16) * d;
                }
            } break;
            case OR_Q8_0: {
                const blk_q8_0 *b = (const blk_q8_0 *) vx + ib;
                const float d = H2F(b->d);
                for (int j = 0; j < 32; ++j) y[j] = b->qs[j] * d;
            } break;
            case OR_Q2_K: {
                const blk_q2_K *b = (const blk_q2_K *) vx + ib;
                const float d = H2F(b->d), dm = H2F(b->dmin);
                for (int i = 0; i < 256; ++i) {
                    const uint8_t sc = b->scales[i >> 4];
                    y[i] = d * (sc & 0xF) * q2_K_code(b, i) - dm * (sc >> 4);
                }
            } break;
            case OR_Q3_K: {
                const blk_q3_K *b = (const blk_q3_K *) vx + ib;
                const float d = H2F(b->d);
                for (int i = 0; i < 256; ++i) y[i] = d * scale_q3_K(i >> 4, b->scales) * q3_K_code(b, i);
            } break;
            case OR_Q4_K: {
                const blk_q4_K *b = (const blk_q4_K *) vx + ib;
                const float d = H2F(b->d), dm = H2F(b->dmin);
                for (int i = 0; i < 256; ++i) {
                    int sc, m;
                    scale_min_k4(i >> 5, b->scales, &sc, &m);
                    y[i] = d * sc * q4_K_code(b, i) - dm * m;
                }
            } break;
            case OR_Q5_K: {
                const blk_q5_K *b = (const blk_q5_K *) vx + ib;
                const float d = H2F(b->d), dm = H2F(b->dmin);
                for (int i = 0; i < 256; ++i) {
                    int sc, m;
                    scale_min_k4(i >> 5, b->scales, &sc, &m);
                    y[i] = d * sc * q5_K_code(b, i) - dm * m;
                }
            } break;
            case OR_Q6_K: {
                const blk_q6_K *b = (const blk_q6_K *) vx + ib;
                const float d = H2F(b->d);
                for (int i = 0; i < 256; ++i) y[i] = d * q6_K_scale(b, i) * q6_K_code(b, i);
            } break;
            case OR_Q8_K: {
                const blk_q8_K *b = (const blk_q8_K *) vx + ib;
                for (int i = 0; i < 256; ++i) y[i] = b->d * b->qs[i];
            } break;
            case OR_Q8_1: {
                const blk_q8_1 *b = (const blk_q8_1 *) vx + ib;
                const float d = H2F(b->d);
                for (int j = 0; j < 32; ++j) y[j] = b->qs[j] * d;
            } break;
            default:
                memset(y, 0, sizeof(float) * be);
        }
    }
}

/* ------------------------------------------------------------------ */
/* synthetic weight quantizers (valid blocks; not ggml's quantizer)    */
/* ------------------------------------------------------------------ */

static int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }
static int rnd(float v) { return (int) lrintf(v); }

static void qw_q4_0(const float *x, blk_q4_0 *b) {
    float amax = 0, mx = 0;
    for (int j = 0; j < 32; ++j) if (fabsf(x[j]) > amax) { amax = fabsf(x[j]); mx = x[j]; }
    const float d = mx / -8.0f, id = d ? 1.0f / d : 0.0f;
    b->d = F2H(d);
    for (int j = 0; j < 16; ++j) {
        const int q0 = clampi(rnd(x[j] * id) + 8, 0, 15), q1 = clampi(rnd(x[j + 16] * id) + 8, 0, 15);
        b->qs[j] = (uint8_t) (q0 | (q1 << 4));
    }
}
static void qw_q5_0(const float *x, blk_q5_0 *b) {
    float amax = 0, mx = 0;
    for (int j = 0; j < 32; ++j) if (fabsf(x[j]) > amax) { amax = fabsf(x[j]); mx = x[j]; }
    const float d = mx / -16.0f, id = d ? 1.0f / d : 0.0f;
    b->d = F2H(d);
    uint32_t qh = 0;
    for (int j = 0; j < 16; ++j) {
        const int q0 = clampi(rnd(x[j] * id) + 16, 0, 31), q1 = clampi(rnd(x[j + 16] * id) + 16, 0, 31);
        b->qs[j] = (uint8_t) ((q0 & 0xF) | ((q1 & 0xF) << 4));
        qh |= (uint32_t) (q0 >> 4) << j;
        qh |= (uint32_t) (q1 >> 4) << (j + 16);
    }
    memcpy(b->qh, &qh, 4);
}
static void qw_q8_0(const float *x, blk_q8_0 *b) {
    float amax = 0;
    for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(x[j]));
    const float d = amax / 127.0f, id = d ? 1.0f / d : 0.0f;
    b->d = F2H(d);
    for (int j = 0; j < 32; ++j) b->qs[j] = (int8_t) clampi(rnd(x[j] * id), -127, 127);
}
static void qw_q2_K(const float *x, blk_q2_K *b) {
    float scale[16], mn[16], smax = 0, mmax = 0;
    for (int s = 0; s < 16; ++s) {
        float lo = 0, hi = 0;
        for (int l = 0; l < 16; ++l) { lo = fminf(lo, x[16 * s + l]); hi = fmaxf(hi, x[16 * s + l]); }
        scale[s] = (hi - lo) / 3.0f;
        mn[s] = -lo;
        smax = fmaxf(smax, scale[s]);
        mmax = fmaxf(mmax, mn[s]);
    }
    const float d = smax / 15.0f, dm = mmax / 15.0f;
    b->d = F2H(d);
    b->dmin = F2H(dm);
    const float dq = H2F(b->d), dmq = H2F(b->dmin);
    memset(b->qs, 0, sizeof(b->qs));
    for (int s = 0; s < 16; ++s) {
        const int isc = d ? clampi(rnd(scale[s] / d), 0, 15) : 0;
        const int im = dm ? clampi(rnd(mn[s] / dm), 0, 15) : 0;
        b->scales[s] = (uint8_t) (isc | (im << 4));
        const float ds = dq * isc, ms = dmq * im;
        for (int l = 0; l < 16; ++l) {
            const int i = 16 * s + l;
            const int q = ds ? clampi(rnd((x[i] + ms) / ds), 0, 3) : 0;
            const int h = i >> 7, j = (i & 127) >> 5, ll = i & 31;
            b->qs[32 * h + ll] |= (uint8_t) (q << (2 * j));
        }
    }
}
static void qw_q3_K(const float *x, blk_q3_K *b) {
    float scale[16], smax = 0;
    for (int s = 0; s < 16; ++s) {
        float amax = 0, mx = 0;
        for (int l = 0; l < 16; ++l) if (fabsf(x[16 * s + l]) > amax) { amax = fabsf(x[16 * s + l]); mx = x[16 * s + l]; }
        scale[s] = mx / -4.0f;                      /* codes -4..3 */
        smax = fmaxf(smax, fabsf(scale[s]));
    }
    const float d = smax / 31.0f;
    b->d = F2H(d);
    const float dq = H2F(b->d);
    memset(b->scales, 0, sizeof(b->scales));
    memset(b->qs, 0, sizeof(b->qs));
    memset(b->hmask, 0, sizeof(b->hmask));
    for (int s = 0; s < 16; ++s) {
        const int isc = d ? clampi(rnd(scale[s] / d), -32, 31) : 0;
        const int u = isc + 32;                     /* 6-bit stored value */
        if (s < 8) b->scales[s] |= (uint8_t) (u & 0xF);
        else       b->scales[s - 8] |= (uint8_t) ((u & 0xF) << 4);
        b->scales[8 + (s & 3)] |= (uint8_t) (((u >> 4) & 3) << (2 * (s >> 2)));
        const float ds = dq * isc;
        for (int l = 0; l < 16; ++l) {
            const int i = 16 * s + l;
            const int q = ds ? clampi(rnd(x[i] / ds), -4, 3) : 0;
            const int v = q + 4;                    /* 0..7 = low2 | hbit<<2 */
            const int h = i >> 7, j = (i & 127) >> 5, ll = i & 31;
            b->qs[32 * h + ll] |= (uint8_t) ((v & 3) << (2 * j));
            if (v & 4) b->hmask[ll] |= (uint8_t) (1 << (4 * h + j));
        }
    }
}
static void put_scale_min_k4(int j, uint8_t *q, int d, int m) {
    if (j < 4) {
        q[j] = (uint8_t) ((q[j] & 0xC0) | (d & 63));
        q[j + 4] = (uint8_t) ((q[j + 4] & 0xC0) | (m & 63));
    } else {
        q[j + 4] = (uint8_t) ((d & 0xF) | ((m & 0xF) << 4));
        q[j - 4] = (uint8_t) ((q[j - 4] & 0x3F) | ((d >> 4) << 6));
        q[j] = (uint8_t) ((q[j] & 0x3F) | ((m >> 4) << 6));
    }
}
static void qw_q45_K(const float *x, uint8_t *scales12, uint16_t *dh, uint16_t *dmh, int nlev, int *codes) {
    float scale[8], mn[8], smax = 0, mmax = 0;
    for (int s = 0; s < 8; ++s) {
        float lo = 0, hi = 0;
        for (int l = 0; l < 32; ++l) { lo = fminf(lo, x[32 * s + l]); hi = fmaxf(hi, x[32 * s + l]); }
        scale[s] = (hi - lo) / (float) (nlev - 1);
        mn[s] = -lo;
        smax = fmaxf(smax, scale[s]);
        mmax = fmaxf(mmax, mn[s]);
    }
    const float d = smax / 63.0f, dm = mmax / 63.0f;
    *dh = F2H(d);
    *dmh = F2H(dm);
    const float dq = H2F(*dh), dmq = H2F(*dmh);
    memset(scales12, 0, 12);
    for (int s = 0; s < 8; ++s) {
        const int isc = d ? clampi(rnd(scale[s] / d), 0, 63) : 0;
        const int im = dm ? clampi(rnd(mn[s] / dm), 0, 63) : 0;
        put_scale_min_k4(s, scales12, isc, im);
        const float ds = dq * isc, ms = dmq * im;
        for (int l = 0; l < 32; ++l) codes[32 * s + l] = ds ? clampi(rnd((x[32 * s + l] + ms) / ds), 0, nlev - 1) : 0;
    }
}
static void qw_q4_K(const float *x, blk_q4_K *b) {
    int codes[256];
    qw_q45_K(x, b->scales, &b->d, &b->dmin, 16, codes);
    for (int c = 0; c < 4; ++c)
        for (int l = 0; l < 32; ++l)
            b->qs[32 * c + l] = (uint8_t) (codes[64 * c + l] | (codes[64 * c + 32 + l] << 4));
}
static void qw_q5_K(const float *x, blk_q5_K *b) {
    int codes[256];
    qw_q45_K(x, b->scales, &b->d, &b->dmin, 32, codes);
    memset(b->qh, 0, sizeof(b->qh));
    for (int c = 0; c < 4; ++c)
        for (int l = 0; l < 32; ++l) {
            const int a0 = codes[64 * c + l], a1 = codes[64 * c + 32 + l];
            b->qs[32 * c + l] = (uint8_t) ((a0 & 0xF) | ((a1 & 0xF) << 4));
            b->qh[l] |= (uint8_t) (((a0 >> 4) << (2 * c)) | ((a1 >> 4) << (2 * c + 1)));
        }
}
static void qw_q6_K(const float *x, blk_q6_K *b) {
    float scale[16], smax = 0;
    for (int s = 0; s < 16; ++s) {
        float amax = 0, mx = 0;
        for (int l = 0; l < 16; ++l) if (fabsf(x[16 * s + l]) > amax) { amax = fabsf(x[16 * s + l]); mx = x[16 * s + l]; }
        scale[s] = mx / -32.0f;
        smax = fmaxf(smax, fabsf(scale[s]));
    }
    const float d = smax / 127.0f;
    b->d = F2H(d);
    const float dq = H2F(b->d);
    memset(b->ql, 0, sizeof(b->ql));
    memset(b->qh, 0, sizeof(b->qh));
    for (int i = 0; i < 256; ++i) {
        const int n = i >> 7, quarter = (i & 127) >> 5, l = i & 31;
        const int s = 8 * n + 2 * quarter + (l >> 4);
        const int isc = d ? clampi(rnd(scale[i >> 4] / d), -128, 127) : 0;
        b->scales[s] = (int8_t) isc;               /* sub-block i>>4 is stored at index s (same mapping) */
        const float ds = dq * isc;
        const int q = ds ? clampi(rnd(x[i] / ds), -32, 31) : 0;
        const int v = q + 32;
        b->ql[64 * n + 32 * (quarter & 1) + l] |= (uint8_t) ((v & 0xF) << (4 * (quarter >> 1)));
        b->qh[32 * n + l] |= (uint8_t) ((v >> 4) << (2 * quarter));
    }
}

void or_quantize_row_weights(int type, const float *x, void *vy, int64_t k) {
    const int be = or_block_elems(type);
    const int64_t nb = k / be;
    for (int64_t ib = 0; ib < nb; ++ib) {
        const float *xb = x + ib * be;
        switch (type) {
            case OR_Q4_0: qw_q4_0(xb, (blk_q4_0 *) vy + ib); break;
            case OR_Q5_0: qw_q5_0(xb, (blk_q5_0 *) vy + ib); break;
            case OR_Q8_0: qw_q8_0(xb, (blk_q8_0 *) vy + ib); break;
            case OR_Q2_K: qw_q2_K(xb, (blk_q2_K *) vy + ib); break;
            case OR_Q3_K: qw_q3_K(xb, (blk_q3_K *) vy + ib); break;
            case OR_Q4_K: qw_q4_K(xb, (blk_q4_K *) vy + ib); break;
            case OR_Q5_K: qw_q5_K(xb, (blk_q5_K *) vy + ib); break;
            case OR_Q6_K: qw_q6_K(xb, (blk_q6_K *) vy + ib); break;
            default: break;
        }
    }
}

/* ------------------------------------------------------------------ */
/* activation quantizers                                               */
/* ------------------------------------------------------------------ */

/* ggml-CUDA quantize_q8_1: one 32-lane group per block; amax and sum are
 * xor-butterfly reductions (offsets 16, 8, 4, 2, 1); d = amax/127 with an
 * IEEE division; q = amax == 0 ? 0 : roundf(x/d); ds = (half(d), half(sum)). */
void or_quantize_q8_1(const float *x, void *vy, int64_t k) {
    blk_q8_1 *y = (blk_q8_1 *) vy;
    for (int64_t ib = 0; ib < k / 32; ++ib) {
        const float *xb = x + 32 * ib;
        float amax = 0.0f, s[32];
        for (int j = 0; j < 32; ++j) {
            amax = fmaxf(amax, fabsf(xb[j]));
            s[j] = xb[j];
        }
        for (int off = 16; off > 0; off >>= 1) {
            float t[32];
            for (int j = 0; j < 32; ++j) t[j] = s[j] + s[j ^ off];
            memcpy(s, t, sizeof(t));
        }
        const float d = amax / 127.0f;
        for (int j = 0; j < 32; ++j) y[ib].qs[j] = (int8_t) (amax == 0.0f ? 0 : (int) roundf(xb[j] / d));
        y[ib].d = F2H(d);
        y[ib].s = F2H(s[0]);
    }
}

/* quantize_row_q8_0_ref: d = amax/127, id = 1/d, q = roundf(x*id) */
void or_quantize_q8_0(const float *x, void *vy, int64_t k) {
    blk_q8_0 *y = (blk_q8_0 *) vy;
    for (int64_t ib = 0; ib < k / 32; ++ib) {
        float amax = 0.0f;
        for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(x[32 * ib + j]));
        const float d = amax / 127.0f, id = d ? 1.0f / d : 0.0f;
        y[ib].d = F2H(d);
        for (int j = 0; j < 32; ++j) y[ib].qs[j] = (int8_t) roundf(x[32 * ib + j] * id);
    }
}

void or_quantize_q8_0_as_q8_1(const float *x, void *vy, int64_t k) {
    blk_q8_1 *y = (blk_q8_1 *) vy;
    for (int64_t ib = 0; ib < k / 32; ++ib) {
        float amax = 0.0f;
        for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(x[32 * ib + j]));
        const float d = amax / 127.0f, id = d ? 1.0f / d : 0.0f;
        y[ib].d = F2H(d);
        y[ib].s = 0;
        for (int j = 0; j < 32; ++j) y[ib].qs[j] = (int8_t) roundf(x[32 * ib + j] * id);
    }
}

/* ggml nearest_int: round half to even through the 1.5*2^23 magic constant */
static int nearest_int(float fval) {
    float val = fval + 12582912.f;
    int i;
    memcpy(&i, &val, sizeof(int));
    return (i & 0x007fffff) - 0x00400000;
}

/* quantize_row_q8_K_ref: iscale = -127/max (max = signed value of largest |x|),
 * q = min(127, nearest_int(iscale*x)), d = 1/iscale, bsums over 16 */
void or_quantize_q8_K(const float *x, void *vy, int64_t k) {
    blk_q8_K *y = (blk_q8_K *) vy;
    for (int64_t ib = 0; ib < k / 256; ++ib, x += 256) {
        float max = 0, amax = 0;
        for (int j = 0; j < 256; ++j) {
            const float ax = fabsf(x[j]);
            if (ax > amax) { amax = ax; max = x[j]; }
        }
        if (!amax) {
            y[ib].d = 0;
            memset(y[ib].qs, 0, 256);
            memset(y[ib].bsums, 0, sizeof(y[ib].bsums));
            continue;
        }
        const float iscale = -127.f / max;
        for (int j = 0; j < 256; ++j) {
            const int v = nearest_int(iscale * x[j]);
            y[ib].qs[j] = (int8_t) (v < 127 ? v : 127);
        }
        for (int j = 0; j < 16; ++j) {
            int sum = 0;
            for (int ii = 0; ii < 16; ++ii) sum += y[ib].qs[16 * j + ii];
            y[ib].bsums[j] = (int16_t) sum;
        }
        y[ib].d = 1 / iscale;
    }
}

static int is_kquant(int t) { return t == OR_Q2_K || t == OR_Q3_K || t == OR_Q4_K || t == OR_Q5_K || t == OR_Q6_K; }

int or_act_type(int wtype, int act_kind) {
    if (act_kind == OR_ACT_CPU) return is_kquant(wtype) ? OR_Q8_K : OR_Q8_0;
    return OR_Q8_1;
}

size_t or_act_row_bytes(int wtype, int act_kind, int64_t k) { return or_row_bytes(or_act_type(wtype, act_kind), k); }

void or_quantize_act_row(int wtype, int act_kind, const float *x, void *y, int64_t k) {
    switch (act_kind) {
        case OR_ACT_CPU:
            if (is_kquant(wtype)) or_quantize_q8_K(x, y, k); else or_quantize_q8_0(x, y, k);
            break;
        case OR_ACT_Q8_1: or_quantize_q8_1(x, y, k); break;
        case OR_ACT_Q8_0_AS_Q8_1: or_quantize_q8_0_as_q8_1(x, y, k); break;
        default: break;
    }
}

/* ------------------------------------------------------------------ */
/* dot products                                                        */
/* ------------------------------------------------------------------ */

/* Per-activation-block view: int8 codes + the scale of each 32-element group. */
typedef struct { const int8_t *q; float d[8]; } act_view;

/* Integer sums of one weight block against int8 activations q8 (block_elems values):
 *   legacy types:  out[0] = sum((code - offset) * q8)       (offset 8 / 16 / 0)
 *   Q2_K:          out[2g] = sum_{sub in g} sc*sum(code*q8), out[2g+1] = sum_{sub in g} m*sum(q8)   g = 0..7
 *   Q3_K / Q6_K:   out[g]  = sum_{sub in g} sc*sum(code*q8)                               g = 0..7
 *   Q4_K / Q5_K:   out[2g] = sc_g*sum(code*q8), out[2g+1] = m_g*sum(q8)                   g = 0..7
 * Returns the number of values written. */
int or_block_isums(int t, const void *w, const int8_t *q8, int32_t *out) {
    switch (t) {
        case OR_Q4_0: {
            const blk_q4_0 *b = (const blk_q4_0 *) w;
            int32_t s = 0;
            for (int j = 0; j < 16; ++j) s += ((b->qs[j] & 0xF) - 8) * q8[j] + ((b->qs[j] >> 4) - 8) * q8[j + 16];
            out[0] = s;
            return 1;
        }
        case OR_Q5_0: {
            const blk_q5_0 *b = (const blk_q5_0 *) w;
            uint32_t qh;
            memcpy(&qh, b->qh, 4);
            int32_t s = 0;
            for (int j = 0; j < 16; ++j) {
                s += (((b->qs[j] & 0xF) | (((qh >> j) & 1) << 4)) - 16) * q8[j];
                s += (((b->qs[j] >> 4) | (((qh >> (j + 16)) & 1) << 4)) - 16) * q8[j + 16];
            }
            out[0] = s;
            return 1;
        }
        case OR_Q8_0: {
            const blk_q8_0 *b = (const blk_q8_0 *) w;
            int32_t s = 0;
            for (int j = 0; j < 32; ++j) s += b->qs[j] * q8[j];
            out[0] = s;
            return 1;
        }
        case OR_Q2_K: {
            const blk_q2_K *b = (const blk_q2_K *) w;
            for (int g = 0; g < 8; ++g) {
                int32_t is = 0, ms = 0;
                for (int h = 0; h < 2; ++h) {
                    const int sub = 2 * g + h;
                    int32_t dot = 0, sq = 0;
                    for (int l = 0; l < 16; ++l) {
                        const int i = 16 * sub + l;
                        dot += q2_K_code(b, i) * q8[i];
                        sq += q8[i];
                    }
                    is += (b->scales[sub] & 0xF) * dot;
                    ms += (b->scales[sub] >> 4) * sq;
                }
                out[2 * g] = is;
                out[2 * g + 1] = ms;
            }
            return 16;
        }
        case OR_Q3_K: {
            const blk_q3_K *b = (const blk_q3_K *) w;
            for (int g = 0; g < 8; ++g) {
                int32_t is = 0;
                for (int h = 0; h < 2; ++h) {
                    const int sub = 2 * g + h;
                    int32_t dot = 0;
                    for (int l = 0; l < 16; ++l) dot += q3_K_code(b, 16 * sub + l) * q8[16 * sub + l];
                    is += scale_q3_K(sub, b->scales) * dot;
                }
                out[g] = is;
            }
            return 8;
        }
        case OR_Q4_K:
        case OR_Q5_K: {
            const uint8_t *scales = t == OR_Q4_K ? ((const blk_q4_K *) w)->scales : ((const blk_q5_K *) w)->scales;
            for (int g = 0; g < 8; ++g) {
                int sc, m;
                scale_min_k4(g, scales, &sc, &m);
                int32_t dot = 0, sq = 0;
                for (int l = 0; l < 32; ++l) {
                    const int i = 32 * g + l;
                    const int c = t == OR_Q4_K ? q4_K_code((const blk_q4_K *) w, i) : q5_K_code((const blk_q5_K *) w, i);
                    dot += c * q8[i];
                    sq += q8[i];
                }
                out[2 * g] = sc * dot;
                out[2 * g + 1] = m * sq;
            }
            return 16;
        }
        case OR_Q6_K: {
            const blk_q6_K *b = (const blk_q6_K *) w;
            for (int g = 0; g < 8; ++g) {
                int32_t is = 0;
                for (int h = 0; h < 2; ++h) {
                    int32_t dot = 0;
                    for (int l = 0; l < 16; ++l) {
                        const int i = 32 * g + 16 * h + l;
                        dot += q6_K_code(b, i) * q8[i];
                    }
                    is += q6_K_scale(b, 32 * g + 16 * h) * dot;
                }
                out[g] = is;
            }
            return 8;
        }
        default:
            return 0;
    }
}

static float block_d(int t, const void *w) {
    switch (t) {
        case OR_Q4_0: return H2F(((const blk_q4_0 *) w)->d);
        case OR_Q5_0: return H2F(((const blk_q5_0 *) w)->d);
        case OR_Q8_0: return H2F(((const blk_q8_0 *) w)->d);
        case OR_Q2_K: return H2F(((const blk_q2_K *) w)->d);
        case OR_Q3_K: return H2F(((const blk_q3_K *) w)->d);
        case OR_Q4_K: return H2F(((const blk_q4_K *) w)->d);
        case OR_Q5_K: return H2F(((const blk_q5_K *) w)->d);
        case OR_Q6_K: return H2F(((const blk_q6_K *) w)->d);
        default: return 0.0f;
    }
}
static float block_dmin(int t, const void *w) {
    switch (t) {
        case OR_Q2_K: return H2F(((const blk_q2_K *) w)->dmin);
        case OR_Q4_K: return H2F(((const blk_q4_K *) w)->dmin);
        case OR_Q5_K: return H2F(((const blk_q5_K *) w)->dmin);
        default: return 0.0f;
    }
}

/* CPU semantics (ggml generic vec_dot_<type>_q8_0 / _q8_K): exact integer sums per
 * block, one fp32 combination per block:
 *   legacy : sumf += sumi * d_w * d_a
 *   K-quant: sumf += d_a*d_w * isum - d_a*dmin_w * msum            (Q3_K/Q6_K: no min term)
 * q8_1 semantics (the GEMV kernel's formulation): per 32-element group g with
 * activation scale d_g:
 *   legacy : sumf += sumi * d_w * d_g
 *   K-quant: sumf += d_g * (d_w * isum_g - dmin_w * msum_g)                                  */
float or_vec_dot(int wt, int act_kind, int64_t k, const void *w, const void *a) {
    const int be = or_block_elems(wt);
    const size_t bb = or_block_bytes(wt);
    const int64_t nb = k / be;
    const int legacy = !is_kquant(wt);
    float sumf = 0.0f;
    int32_t is[16];
    for (int64_t ib = 0; ib < nb; ++ib) {
        const void *wb = (const char *) w + ib * bb;
        const float dw = block_d(wt, wb), dmw = block_dmin(wt, wb);
        if (act_kind == OR_ACT_CPU) {
            if (legacy) {
                const blk_q8_0 *ab = (const blk_q8_0 *) a + ib;
                or_block_isums(wt, wb, ab->qs, is);
                sumf += (float) is[0] * dw * H2F(ab->d);
            } else {
                const blk_q8_K *ab = (const blk_q8_K *) a + ib;
                const int n = or_block_isums(wt, wb, ab->qs, is);
                int32_t isum = 0, msum = 0;
                if (n == 16) {
                    for (int g = 0; g < 8; ++g) { isum += is[2 * g]; msum += is[2 * g + 1]; }
                } else {
                    for (int g = 0; g < 8; ++g) isum += is[g];
                }
                const float dall = ab->d * dw, dmin = ab->d * dmw;
                sumf += dall * (float) isum - dmin * (float) msum;
            }
        } else {
            if (legacy) {
                const blk_q8_1 *ab = (const blk_q8_1 *) a + ib;
                or_block_isums(wt, wb, ab->qs, is);
                sumf += (float) is[0] * dw * H2F(ab->d);
            } else {
                const blk_q8_1 *ab = (const blk_q8_1 *) a + 8 * ib;
                int8_t q8[256];
                for (int g = 0; g < 8; ++g) memcpy(q8 + 32 * g, ab[g].qs, 32);
                const int n = or_block_isums(wt, wb, q8, is);
                for (int g = 0; g < 8; ++g) {
                    const float dg = H2F(ab[g].d);
                    if (n == 16) sumf += dg * (dw * (float) is[2 * g] - dmw * (float) is[2 * g + 1]);
                    else         sumf += dg * (dw * (float) is[g]);
                }
            }
        }
    }
    return sumf;
}

/* ------------------------------------------------------------------ */
/* AVX2 q8_K dots (the CPU baseline's vec_dot for Q2_K and Q4_K)        */
/* ------------------------------------------------------------------ */

/* The same integers or_block_isums forms per super-block, summed with 8-bit x 8-bit
 * products (maddubs: unsigned codes x signed activations, pairs into int16, no
 * saturation: |pair| <= 2 * 15 * 127) and int16 x int16 products (madd), then the
 * scalar combination of or_vec_dot in the same order, so the result is bit-identical
 * to the scalar path (ggml's generic vec_dot_q2_K_q8_K / vec_dot_q4_K_q8_K
 * arithmetic; patches/trace-hook/ggml-cpu.c:308-340 selects q8_K for these types). */
static int or_simd = 1;

void or_set_simd(int on) { or_simd = on != 0; }

static inline int32_t hsum_i32x8(__m256i v) {
    __m128i s = _mm_add_epi32(_mm256_castsi256_si128(v), _mm256_extracti128_si256(v, 1));
    s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0x4E));
    s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0xB1));
    return _mm_cvtsi128_si32(s);
}

static inline __m256i two_scales(int s0, int s1) {       /* int16 lanes 0..7 = s0, 8..15 = s1 */
    return _mm256_set_m128i(_mm_set1_epi16((short) s1), _mm_set1_epi16((short) s0));
}

static float vec_dot_q2_K_q8_K_avx2(int64_t k, const blk_q2_K *x, const blk_q8_K *y) {
    const int64_t nb = k / 256;
    const __m256i m3 = _mm256_set1_epi8(3);
    float sumf = 0.0f;
    for (int64_t i = 0; i < nb; ++i) {
        /* min term: sum over the 16 sub-blocks of (scales >> 4) * bsums */
        const __m128i sc8 = _mm_loadu_si128((const __m128i *) x[i].scales);
        const __m256i mins16 = _mm256_cvtepu8_epi16(_mm_and_si128(_mm_srli_epi16(sc8, 4), _mm_set1_epi8(0x0F)));
        const __m256i bsums = _mm256_loadu_si256((const __m256i *) y[i].bsums);
        const int32_t msum = hsum_i32x8(_mm256_madd_epi16(mins16, bsums));
        /* scaled codes: element 128h + 32j + l is (qs[32h + l] >> 2j) & 3, sub-block 8h + 2j + (l >= 16) */
        __m256i acc = _mm256_setzero_si256();
        for (int h = 0; h < 2; ++h) {
            const __m256i qv = _mm256_loadu_si256((const __m256i *) (x[i].qs + 32 * h));
            for (int j = 0; j < 4; ++j) {
                const __m256i codes = _mm256_and_si256(_mm256_srli_epi16(qv, 2 * j), m3);
                const __m256i yv = _mm256_loadu_si256((const __m256i *) (y[i].qs + 128 * h + 32 * j));
                const __m256i p16 = _mm256_maddubs_epi16(codes, yv);
                const int sub = 8 * h + 2 * j;
                acc = _mm256_add_epi32(acc, _mm256_madd_epi16(p16, two_scales(x[i].scales[sub] & 0x0F,
                                                                                 x[i].scales[sub + 1] & 0x0F)));
            }
        }
        const int32_t isum = hsum_i32x8(acc);
        const float dall = y[i].d * H2F(x[i].d), dmin = y[i].d * H2F(x[i].dmin);
        sumf += dall * (float) isum - dmin * (float) msum;
    }
    return sumf;
}

static float vec_dot_q4_K_q8_K_avx2(int64_t k, const blk_q4_K *x, const blk_q8_K *y) {
    const int64_t nb = k / 256;
    const __m256i m4 = _mm256_set1_epi8(0x0F);
    float sumf = 0.0f;
    for (int64_t i = 0; i < nb; ++i) {
        int sc[8], m[8];
        for (int g = 0; g < 8; ++g) scale_min_k4(g, x[i].scales, &sc[g], &m[g]);
        /* min term: m_g * (bsums[2g] + bsums[2g+1]) */
        const __m256i m16 = _mm256_setr_epi16((short) m[0], (short) m[0], (short) m[1], (short) m[1], (short) m[2],
                                              (short) m[2], (short) m[3], (short) m[3], (short) m[4], (short) m[4],
                                              (short) m[5], (short) m[5], (short) m[6], (short) m[6], (short) m[7],
                                              (short) m[7]);
        const __m256i bsums = _mm256_loadu_si256((const __m256i *) y[i].bsums);
        const int32_t msum = hsum_i32x8(_mm256_madd_epi16(m16, bsums));
        /* chunk c: low nibbles of qs[32c..] are sub-block 2c, high nibbles 2c + 1 */
        __m256i acc = _mm256_setzero_si256();
        for (int c = 0; c < 4; ++c) {
            const __m256i qv = _mm256_loadu_si256((const __m256i *) (x[i].qs + 32 * c));
            const __m256i lo = _mm256_and_si256(qv, m4), hi = _mm256_and_si256(_mm256_srli_epi16(qv, 4), m4);
            const __m256i plo = _mm256_maddubs_epi16(lo, _mm256_loadu_si256((const __m256i *) (y[i].qs + 64 * c)));
            const __m256i phi = _mm256_maddubs_epi16(hi, _mm256_loadu_si256((const __m256i *) (y[i].qs + 64 * c + 32)));
            acc = _mm256_add_epi32(acc, _mm256_madd_epi16(plo, _mm256_set1_epi16((short) sc[2 * c])));
            acc = _mm256_add_epi32(acc, _mm256_madd_epi16(phi, _mm256_set1_epi16((short) sc[2 * c + 1])));
        }
        const int32_t isum = hsum_i32x8(acc);
        const float dall = y[i].d * H2F(x[i].d), dmin = y[i].d * H2F(x[i].dmin);
        sumf += dall * (float) isum - dmin * (float) msum;
    }
    return sumf;
}

/* Q4_0 x q8_0: per 32-value block, sum((code - 8) * q8) = sum(code * q8) - 8 * sum(q8), both exact
 * integer sums, combined as (float) isum * d_w * d_a like the scalar path. */
static float vec_dot_q4_0_q8_0_avx2(int64_t k, const blk_q4_0 *x, const blk_q8_0 *y) {
    const int64_t nb = k / 32;
    const __m128i m4 = _mm_set1_epi8(0x0F);
    const __m256i ones8 = _mm256_set1_epi8(1);
    const __m256i ones16 = _mm256_set1_epi16(1);
    float sumf = 0.0f;
    for (int64_t i = 0; i < nb; ++i) {
        const __m128i q = _mm_loadu_si128((const __m128i *) x[i].qs);
        /* codes of values 0..15 (low nibbles) then 16..31 (high nibbles) */
        const __m256i codes = _mm256_set_m128i(_mm_and_si128(_mm_srli_epi16(q, 4), m4), _mm_and_si128(q, m4));
        const __m256i yv = _mm256_loadu_si256((const __m256i *) y[i].qs);
        const int32_t cy = hsum_i32x8(_mm256_madd_epi16(_mm256_maddubs_epi16(codes, yv), ones16));
        const int32_t sy = hsum_i32x8(_mm256_madd_epi16(_mm256_maddubs_epi16(ones8, yv), ones16));
        const int32_t isum = cy - 8 * sy;
        sumf += (float) isum * H2F(x[i].d) * H2F(y[i].d);
    }
    return sumf;
}

/* ggml-CPU vec_dot (q8_0 / q8_K activations): AVX2 for Q4_0, Q2_K and Q4_K when enabled,
 * the scalar restatement otherwise. */
float or_vec_dot_cpu(int wt, int64_t k, const void *w, const void *a) {
    if (or_simd && wt == OR_Q4_0) return vec_dot_q4_0_q8_0_avx2(k, (const blk_q4_0 *) w, (const blk_q8_0 *) a);
    if (or_simd && wt == OR_Q2_K) return vec_dot_q2_K_q8_K_avx2(k, (const blk_q2_K *) w, (const blk_q8_K *) a);
    if (or_simd && wt == OR_Q4_K) return vec_dot_q4_K_q8_K_avx2(k, (const blk_q4_K *) w, (const blk_q8_K *) a);
    return or_vec_dot(wt, OR_ACT_CPU, k, w, a);
}

/* ------------------------------------------------------------------ */
/* GLU                                                                 */
/* ------------------------------------------------------------------ */

static float silu(float x) { return x / (1.0f + expf(-x)); }

/* kernels/ssm-conv.cu:5-57: the reference keeps a ring buffer of the last nc inputs,
 * x[(i + j) % d_conv] = x_block[i + j]; the sum visits the same values in the same order. */
void or_ssm_conv_f32(const float *x, int64_t x_row, int64_t x_seq, const void *w, int w_f16, int64_t w_row,
                     const float *bias, int silu_on, float *dst, int64_t dst_tok, int64_t dst_seq,
                     int64_t nc, int64_t nr, int64_t n_t, int64_t n_s) {
    for (int64_t s = 0; s < n_s; ++s)
        for (int64_t r = 0; r < nr; ++r) {
            const float *xr = x + s * x_seq + r * x_row;
            float wv[16];
            for (int64_t j = 0; j < nc && j < 16; ++j)
                wv[j] = w_f16 ? H2F(((const uint16_t *) w)[r * w_row + j]) : ((const float *) w)[r * w_row + j];
            const float b = bias ? bias[r] : 0.0f;
            for (int64_t t = 0; t < n_t; ++t) {
                float sumf = 0.0f;
                for (int64_t j = 0; j < nc; ++j) sumf = fmaf(xr[t + j], wv[j], sumf);
                if (silu_on) {
                    sumf += b;
                    sumf = silu(sumf);
                }
                dst[s * dst_seq + t * dst_tok + r] = sumf;
            }
        }
}

float or_glu(int op, float g, float up, float limit) {
    switch (op) {
        case OR_GLU_REGLU: return up * (g > 0.0f ? g : 0.0f);
        case OR_GLU_GEGLU: {
            const float c = 0.79788456080286535587989211986876f;
            return up * (0.5f * g * (1.0f + tanhf(c * g * (1.0f + 0.044715f * g * g))));
        }
        case OR_GLU_SWIGLU: return up * silu(g);
        case OR_GLU_SWIGLU_OAI: {
            const float alpha = 1.702f, lim = 7.0f;
            const float x = fminf(g, lim);
            const float u = fmaxf(fminf(up, lim), -lim);
            return x / (1.0f + expf(-x * alpha)) * (1.0f + u);
        }
        case OR_GLU_GEGLU_ERF: return up * (0.5f * g * (1.0f + erff(g * 0.70710678118654752440f)));
        case OR_GLU_GEGLU_QUICK: return up * (g / (1.0f + expf(-1.702f * g)));
        case OR_GLU_SWIGLU_CLAMP: {
            const float x = fminf(g, limit);
            const float u = fmaxf(fminf(up, limit), -limit);
            return silu(x) * u;
        }
        default: return up * g;
    }
}

/* ------------------------------------------------------------------ */
/* MUL_MAT_ID + post-ops                                               */
/* ------------------------------------------------------------------ */

int or_omp_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

int or_mul_mat_id(const or_mmid_args *A) {
    if (!or_type_supported(A->type)) return -1;
    if (A->sh_up && !or_type_supported(A->sh_type)) return -1;
    const int64_t K = A->ne00, R = A->ne01;
    const int n_pairs = A->n_ids * A->n_tok;
    const int nth = A->nthreads > 0 ? A->nthreads : 1;
    /* routed experts: one dot per (pick, row); each dst element is produced by exactly one dot */
#pragma omp parallel for schedule(dynamic, 16) num_threads(nth)
    for (int64_t task = 0; task < (int64_t) n_pairs * R; ++task) {
        const int pair = (int) (task / R);
        const int64_t r = task % R;
        const int t = pair / A->n_ids, c = pair % A->n_ids;
        const int32_t e = A->ids[c + (int64_t) t * A->ids_stride];
        if (e < 0 || e >= A->n_as) continue;
        const char *arow = (const char *) A->act + (size_t) (c % A->nchannels_y) * A->act_stride_channel + (size_t) t * A->act_stride_col;
        const char *wrow = (const char *) A->src0 + (size_t) e * A->nb02 + (size_t) r * A->nb01;
        float up = or_vec_dot(A->type, A->act_kind, K, wrow, arow);
        if (A->x_scale) up *= A->x_scale[e];
        if (A->x_bias) up += A->x_bias[(int64_t) e * A->bias_stride + r];
        float out = up;
        if (A->gate) {
            const char *grow = (const char *) A->gate + (size_t) e * A->nb02 + (size_t) r * A->nb01;
            float g = or_vec_dot(A->type, A->act_kind, K, grow, arow);
            if (A->gate_scale) g *= A->gate_scale[e];
            if (A->gate_bias) g += A->gate_bias[(int64_t) e * A->bias_stride + r];
            out = or_glu(A->glu_op, g, up, A->glu_limit);
        }
        A->dst[(int64_t) t * A->dst_stride_col + (int64_t) c * A->dst_stride_channel + r] = out;
    }
    /* shared expert: same rows/columns, its own (possibly different) type; no bias/scale */
    if (A->sh_up) {
        const size_t srb = or_row_bytes(A->sh_type, K);
#pragma omp parallel for schedule(dynamic, 16) num_threads(nth)
        for (int64_t task = 0; task < (int64_t) A->n_tok * R; ++task) {
            const int t = (int) (task / R);
            const int64_t r = task % R;
            const char *arow = A->sh_act ? (const char *) A->sh_act + (size_t) t * A->sh_act_stride_col
                                         : (const char *) A->act + (size_t) t * A->act_stride_col;
            float up = or_vec_dot(A->sh_type, A->act_kind, K, (const char *) A->sh_up + r * srb, arow);
            float out = up;
            if (A->sh_gate) {
                float g = or_vec_dot(A->sh_type, A->act_kind, K, (const char *) A->sh_gate + r * srb, arow);
                out = or_glu(A->glu_op, g, up, A->glu_limit);
            }
            A->sh_dst[(int64_t) t * A->sh_stride_col_dst + r] = out;
        }
    }
    return 0;
}

/* Restatement of ggml_compute_forward_mul_mat_id (patches/trace-hook/ggml-cpu.c:1563-1767):
 *   1. src1 rows are quantized to the CPU vec_dot_type (:1662-1673);
 *   2. (slot, token) pairs are grouped by expert in slot-major order (:1677-1692);
 *   3. each expert's rows are chunked (16 rows, 64 when one side is 1; re-chunked per
 *      thread when there are fewer than 4 chunks per thread) and taken from a shared
 *      counter (:1721-1765);
 *   4. every (row, pair) is one vec_dot (:1515-1549). */
int or_cpu_mul_mat_id_f32(int type, int64_t ne00, int64_t ne01, int32_t n_as,
                          const void *src0, size_t nb01, size_t nb02,
                          const float *src1, int64_t ne11, int64_t src1_stride_row, int64_t src1_stride_tok,
                          const int32_t *ids, int32_t n_ids, int32_t n_tok, int64_t ids_stride,
                          float *dst, int64_t dst_stride_col, int64_t dst_stride_channel,
                          int32_t nthreads) {
    if (!or_type_supported(type)) return -1;
    const int nth = nthreads > 0 ? nthreads : 1;
    const size_t arb = or_act_row_bytes(type, OR_ACT_CPU, ne00);
    char *wdata = (char *) malloc(arb * (size_t) ne11 * n_tok);
    int64_t *counts = (int64_t *) calloc((size_t) n_as, sizeof(int64_t));
    int32_t *rows = (int32_t *) malloc(sizeof(int32_t) * 2 * (size_t) n_as * n_ids * n_tok);
    if (!wdata || !counts || !rows) { free(wdata); free(counts); free(rows); return -2; }
#pragma omp parallel for num_threads(nth)
    for (int64_t r = 0; r < ne11 * n_tok; ++r) {
        const int64_t i11 = r % ne11, i12 = r / ne11;
        or_quantize_act_row(type, OR_ACT_CPU, src1 + i12 * src1_stride_tok + i11 * src1_stride_row, wdata + (size_t) r * arb, ne00);
    }
    const int64_t cap = (int64_t) n_ids * n_tok;
    for (int32_t t = 0; t < n_tok; ++t) {
        for (int32_t c = 0; c < n_ids; ++c) {
            const int32_t e = ids[c + (int64_t) t * ids_stride];
            if (e < 0 || e >= n_as) continue;
            int32_t *m = rows + 2 * ((int64_t) e * cap + counts[e]);
            m[0] = c;
            m[1] = t;
            counts[e] += 1;
        }
    }
    for (int32_t e = 0; e < n_as; ++e) {
        const int64_t nr1 = counts[e];
        if (nr1 == 0) continue;
        const int64_t nr0 = ne01;
        int chunk = (nr0 == 1 || nr1 == 1) ? 64 : 16;
        int64_t nc0 = (nr0 + chunk - 1) / chunk, nc1 = (nr1 + chunk - 1) / chunk;
        if (nc0 * nc1 < nth * 4) {
            nc0 = nr0 > nr1 ? nth : 1;
            nc1 = nr0 > nr1 ? 1 : nth;
        }
        const int64_t dr0 = (nr0 + nc0 - 1) / nc0, dr1 = (nr1 + nc1 - 1) / nc1;
        const char *w = (const char *) src0 + (size_t) e * nb02;
#pragma omp parallel for schedule(dynamic, 1) num_threads(nth)
        for (int64_t ch = 0; ch < nc0 * nc1; ++ch) {
            const int64_t r0s = dr0 * (ch % nc0), r0e = r0s + dr0 < nr0 ? r0s + dr0 : nr0;
            const int64_t r1s = dr1 * (ch / nc0), r1e = r1s + dr1 < nr1 ? r1s + dr1 : nr1;
            for (int64_t i1 = r1s; i1 < r1e; ++i1) {
                const int32_t *m = rows + 2 * ((int64_t) e * cap + i1);
                const int32_t c = m[0], t = m[1];
                const char *a = wdata + (size_t) ((c % ne11) + (int64_t) t * ne11) * arb;
                float *d = dst + (int64_t) t * dst_stride_col + (int64_t) c * dst_stride_channel;
                for (int64_t r = r0s; r < r0e; ++r) d[r] = or_vec_dot_cpu(type, ne00, w + (size_t) r * nb01, a);
            }
        }
    }
    free(wdata);
    free(counts);
    free(rows);
    return 0;
}

/* RMS sum of a row in the canonical order of the GPU combine kernel: 256-value
 * chunks; in chunk j, partial l (0..63) accumulates x[256j + 4l + i]^2 (i = 0..3)
 * with fmaf from 0; the 64 partials are tree-added (l += l + off, off = 32 .. 1);
 * chunk sums are added in ascending j from 0. */
float or_rms_sum(const float *x, int64_t k) {
    float total = 0.0f;
    for (int64_t j = 0; j < k / 256; ++j) {
        float part[64];
        for (int l = 0; l < 64; ++l) {
            float a = 0.0f;
            for (int i = 0; i < 4; ++i) {
                const float v = x[256 * j + 4 * l + i];
                a = fmaf(v, v, a);
            }
            part[l] = a;
        }
        for (int off = 32; off > 0; off >>= 1)
            for (int l = 0; l < off; ++l) part[l] += part[l + off];
        total += part[0];
    }
    return total;
}

void or_combine_q8_1(const float *o, int64_t o_stride, const float *w, int32_t n_used, const float *shared,
                     int64_t shared_stride, const float *residual, float *x_out, void *y, int64_t k, int64_t n_tok,
                     int32_t rms_norm, const float *norm_weight, float eps) {
    float *v = (float *) malloc(sizeof(float) * (size_t) k);
    for (int64_t t = 0; t < n_tok; ++t) {
        float *x = x_out + t * k;
        for (int64_t i = 0; i < k; ++i) {
            float a = residual ? residual[t * k + i] : 0.0f;
            if (shared) a += shared[t * shared_stride + i];
            for (int32_t j = 0; j < n_used; ++j) a = fmaf(w[t * n_used + j], o[(t * n_used + j) * o_stride + i], a);
            x[i] = a;
        }
        const float s = rms_norm ? 1.0f / sqrtf(or_rms_sum(x, k) / (float) k + eps) : 1.0f;
        for (int64_t i = 0; i < k; ++i) {
            float a = x[i];
            if (rms_norm) a *= s;
            if (rms_norm && norm_weight) a *= norm_weight[i];
            v[i] = a;
        }
        or_quantize_q8_1(v, (char *) y + (size_t) t * (size_t) (k / 32) * 36, k);
    }
    free(v);
}

/* ------------------------------------------------------------------ */
/* deterministic generators                                            */
/* ------------------------------------------------------------------ */

uint64_t or_splitmix64(uint64_t *s) {
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static double u01(uint64_t *s) { return ((or_splitmix64(s) >> 11) + 0.5) * (1.0 / 9007199254740992.0); }

void or_fill_normal(uint64_t seed, float mean, float std, float *out, int64_t n) {
    uint64_t s = seed;
    for (int64_t i = 0; i < n; i += 2) {
        const double u1 = u01(&s), u2 = u01(&s);
        const double r = sqrt(-2.0 * log(u1));
        out[i] = (float) (mean + std * r * cos(6.283185307179586 * u2));
        if (i + 1 < n) out[i + 1] = (float) (mean + std * r * sin(6.283185307179586 * u2));
    }
}

/* k distinct experts per token, uniform without replacement (partial Fisher-Yates) */
void or_topk_uniform(uint64_t seed, int32_t n_experts, int32_t k, int32_t n_tok, int32_t *ids) {
    uint64_t s = seed;
    int32_t *perm = (int32_t *) malloc(sizeof(int32_t) * (size_t) n_experts);
    for (int32_t t = 0; t < n_tok; ++t) {
        for (int32_t i = 0; i < n_experts; ++i) perm[i] = i;
        for (int32_t i = 0; i < k; ++i) {
            const int32_t j = i + (int32_t) (or_splitmix64(&s) % (uint64_t) (n_experts - i));
            const int32_t tmp = perm[i];
            perm[i] = perm[j];
            perm[j] = tmp;
            ids[(int64_t) t * k + i] = perm[i];
        }
    }
    free(perm);
}
