/* siq_oracle: CPU oracle for Siphon's quantized matvec path.
 * TEST INFRASTRUCTURE ONLY (see siq_oracle.h for scope and pinning).
 *
 * Built with -std=c17 -ffp-contract=off: every float expression below is
 * evaluated with one rounding per operation, as the reference's -std=c17
 * build does (reference Makefile:11-15).
 */
#include "siq_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ---- small helpers ------------------------------------------------------ */

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static uint32_t rd32(const uint8_t *p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) |
           ((uint32_t)p[3] << 24);
}
static void wr16(uint8_t *p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }

/* ---- geometry (reference quant.h:92-100, kernels.c:904-919) ------------- */

int siq_geometry(uint32_t type, uint32_t *blk_elems, uint32_t *blk_bytes) {
    uint32_t e = 0, b = 0;
    switch (type) {
        case SIQ_F32:  e = 1;   b = 4;   break;
        case SIQ_F16:  e = 1;   b = 2;   break;
        case SIQ_Q4_0: e = 32;  b = 18;  break;
        case SIQ_Q5_0: e = 32;  b = 22;  break;
        case SIQ_Q8_0: e = 32;  b = 34;  break;
        case SIQ_Q2_K: e = 256; b = 84;  break;
        case SIQ_Q3_K: e = 256; b = 110; break;
        case SIQ_Q4_K: e = 256; b = 144; break;
        case SIQ_Q5_K: e = 256; b = 176; break;
        case SIQ_Q6_K: e = 256; b = 210; break;
        case SIQ_Q8_K: e = 256; b = 292; break;
        default: return 0;
    }
    if (blk_elems) *blk_elems = e;
    if (blk_bytes) *blk_bytes = b;
    return 1;
}

/* reference kernels.c:946-960 */
int siq_pair(uint32_t wtype, uint32_t *pair) {
    uint32_t p;
    switch (wtype) {
        case SIQ_F32: p = SIQ_F32; break; /* x passes through (backend.c:102-103) */
        case SIQ_F16: p = SIQ_F16; break;
        case SIQ_Q4_0: case SIQ_Q5_0: case SIQ_Q8_0: p = SIQ_Q8_0; break;
        case SIQ_Q2_K: case SIQ_Q3_K: case SIQ_Q4_K: case SIQ_Q5_K:
        case SIQ_Q6_K: p = SIQ_Q8_K; break;
        default: return 0;
    }
    if (pair) *pair = p;
    return 1;
}

/* ---- IEEE binary16 (reference kernels.c:98-176) -------------------------- */

float siq_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 31u, m = h & 0x3ffu;
    if (e == 0) {
        /* zero or subnormal: m * 2^-24 is exact in binary32 */
        const float v = (float)m * 0x1p-24f;
        return u2f(f2u(v) | sign);
    }
    if (e == 31) return u2f(sign | 0x7f800000u | (m << 13));
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

uint16_t siq_f32_to_f16(float f) {
    const uint32_t u = f2u(f);
    const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    const uint32_t a = u & 0x7fffffffu;
    if (a >= 0x7f800000u) {
        if (a == 0x7f800000u) return sign | 0x7c00u;
        /* NaN: quiet, top payload bits kept, never the infinity pattern */
        uint32_t m = (a >> 13) & 0x3ffu;
        if (m == 0) m = 1;
        return (uint16_t)(sign | 0x7c00u | 0x200u | m);
    }
    if (a >= 0x477ff000u) return sign | 0x7c00u; /* >= 65520 rounds to inf */
    if (a < 0x38800000u) {
        /* result is a binary16 subnormal (or rounds up to the smallest
         * normal): m = RNE(|f| * 2^24) */
        const int e = (int)(a >> 23) - 127;
        if (e < -25) return sign; /* below half of the smallest subnormal */
        const uint32_t mant = (a & 0x7fffffu) | 0x800000u;
        const int shift = -(e + 1); /* 14..24 */
        uint32_t m = mant >> shift;
        const uint32_t rem = mant & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (m & 1u))) m++;
        return (uint16_t)(sign | m);
    }
    /* normal: rebias the exponent and round the 13 dropped bits RNE */
    uint32_t r = a - 0x38000000u;
    r += 0xfffu + ((r >> 13) & 1u);
    return (uint16_t)(sign | (r >> 13));
}

/* ---- activation quantizers --------------------------------------------- */

/* reference kernels.c:528-533: magic-number round to nearest even */
static int nearest_int_magic(float v) {
    const float t = v + 12582912.0f;
    return (int)(f2u(t) & 0x7fffffu) - 0x400000;
}

/* Q8_K block: f32 d @0, int8 qs[256] @4, int16 bsums[16] @260 (292 B).
 * reference kernels.c:561-595. bsums of an all-zero block are left
 * unwritten by the reference (reference backend.c:105 mallocs the
 * buffer); this oracle writes 0 there and tests mask them. */
void siq_quantize_q8_K(const float *x, void *out, int64_t n) {
    uint8_t *o = out;
    for (int64_t b = 0; b < n / 256; b++, x += 256, o += 292) {
        float amax = 0.0f, vmax = 0.0f;
        for (int j = 0; j < 256; j++) {
            const float a = fabsf(x[j]);
            if (a > amax) { amax = a; vmax = x[j]; } /* first occurrence wins */
        }
        int8_t *qs = (int8_t *)(o + 4);
        if (amax == 0.0f) {
            memset(o, 0, 292);
            continue;
        }
        const float iscale = -127.0f / vmax;
        for (int j = 0; j < 256; j++) {
            const int v = nearest_int_magic(iscale * x[j]);
            const int c = v < 127 ? v : 127;
            qs[j] = (int8_t)(uint8_t)(c & 0xff);
        }
        for (int g = 0; g < 16; g++) {
            int s = 0;
            for (int k = 0; k < 16; k++) s += qs[16 * g + k];
            wr16(o + 260 + 2 * g, (uint16_t)(int16_t)s);
        }
        const float d = 1.0f / iscale;
        memcpy(o, &d, 4);
    }
}

/* SIMD max semantics: sel(a > b, a, b) (NaN in either picks b). */
static float vmaxsel(float a, float b) { return a > b ? a : b; }

/* x86 cvtps_epi32 on an already-rounded value: out-of-range or NaN gives
 * the "integer indefinite" INT32_MIN. */
static int32_t cvt_i32_indef(float r) {
    if (!(r >= -2147483648.0f && r < 2147483648.0f)) return INT32_MIN;
    return (int32_t)r;
}

/* Q8_0 block: f16 d @0, int8 qs[32] @2 (34 B).
 * reference kernels_avx2.c:594-645 (SIMD form): the abs-max reduction tree
 * (8 lanes over 4 vectors, then 8->4->2->1), d = f16(max/127),
 * id = 127/max, q = saturate_i8(cvt(rint(x*id))). */
void siq_quantize_q8_0(const float *x, void *out, int64_t n) {
    uint8_t *o = out;
    for (int64_t b = 0; b < n / 32; b++, x += 32, o += 34) {
        float lane[8];
        for (int k = 0; k < 8; k++) {
            float m = fabsf(x[k]);
            m = vmaxsel(m, fabsf(x[8 + k]));
            m = vmaxsel(m, fabsf(x[16 + k]));
            m = vmaxsel(m, fabsf(x[24 + k]));
            lane[k] = m;
        }
        float m4[4], m2[2];
        for (int k = 0; k < 4; k++) m4[k] = vmaxsel(lane[4 + k], lane[k]);
        for (int k = 0; k < 2; k++) m2[k] = vmaxsel(m4[k], m4[k + 2]);
        const float mx = vmaxsel(m2[0], m2[1]);
        wr16(o, siq_f32_to_f16(mx / 127.0f));
        const float id = (mx != 0.0f) ? 127.0f / mx : 0.0f;
        for (int j = 0; j < 32; j++) {
            const float r = rintf(x[j] * id);
            int32_t v = cvt_i32_indef(r);
            if (v > 127) v = 127;
            if (v < -128) v = -128;
            o[2 + j] = (uint8_t)(int8_t)v;
        }
    }
}

/* reference kernels.c:542-558 (portable scalar form): amax, d = amax/127,
 * id = 1/d, q = roundf(x*id) (halves away from zero). */
void siq_quantize_q8_0_scalar(const float *x, void *out, int64_t n) {
    uint8_t *o = out;
    for (int64_t b = 0; b < n / 32; b++, x += 32, o += 34) {
        float amax = 0.0f;
        for (int j = 0; j < 32; j++) {
            const float a = fabsf(x[j]);
            amax = amax > a ? amax : a;
        }
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        wr16(o, siq_f32_to_f16(d));
        for (int j = 0; j < 32; j++) o[2 + j] = (uint8_t)(int8_t)roundf(x[j] * id);
    }
}

void siq_convert_f16(const float *x, uint16_t *out, int64_t n) {
    for (int64_t i = 0; i < n; i++) out[i] = siq_f32_to_f16(x[i]);
}

int siq_quantize_pair(uint32_t pair, const float *x, void *out, int64_t n) {
    switch (pair) {
        case SIQ_F32: memcpy(out, x, (size_t)n * sizeof(float)); return 1;
        case SIQ_F16: siq_convert_f16(x, out, n); return 1;
        case SIQ_Q8_0: siq_quantize_q8_0(x, out, n); return 1;
        case SIQ_Q8_K: siq_quantize_q8_K(x, out, n); return 1;
        default: return 0;
    }
}

/* ---- block decoding ------------------------------------------------------
 * Every quantized element is decoded to integers (q, s, m) such that its
 * weight value is  d*s*q - dmin*m  (K formats) or  d*q  (32-blocks).
 * ------------------------------------------------------------------------ */

typedef struct {
    int n;                 /* elements in the block */
    int q[256];            /* signed quant after bias */
    int s[256];            /* integer sub-block scale (1 for 32-blocks) */
    int m[256];            /* integer sub-block min (0 if none) */
    float d, dmin;         /* block scales */
} blk_vals;

/* 6-bit scale/min pair of sub-block j from the 12 packed bytes of Q4_K and
 * Q5_K (reference kernels.c:648-656). */
static void k4_scale_min(const uint8_t *sc, int j, int *s, int *m) {
    if (j < 4) {
        *s = sc[j] & 63;
        *m = sc[j + 4] & 63;
    } else {
        *s = (sc[j + 4] & 15) | ((sc[j - 4] >> 6) << 4);
        *m = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4);
    }
}

/* 6-bit signed scale k of Q3_K: low nibble from bytes 0..7, high 2 bits
 * from bytes 8..11 (reference kernels.c:328-333, restated per scale). */
static int k3_scale(const uint8_t *sc, int k) {
    const int lo = k < 8 ? (sc[k] & 15) : (sc[k - 8] >> 4);
    const int hi = (sc[8 + (k & 3)] >> (2 * (k >> 2))) & 3;
    return (lo | (hi << 4)) - 32;
}

static int decode_block(uint32_t type, const uint8_t *b, blk_vals *v) {
    v->dmin = 0.0f;
    switch (type) {
        case SIQ_Q4_0: {
            v->n = 32; v->d = siq_f16_to_f32(rd16(b));
            for (int j = 0; j < 16; j++) {
                v->q[j] = (b[2 + j] & 15) - 8;
                v->q[j + 16] = (b[2 + j] >> 4) - 8;
            }
            break;
        }
        case SIQ_Q5_0: {
            v->n = 32; v->d = siq_f16_to_f32(rd16(b));
            const uint32_t qh = rd32(b + 2);
            for (int j = 0; j < 16; j++) {
                v->q[j] = ((b[6 + j] & 15) | (int)(((qh >> j) & 1u) << 4)) - 16;
                v->q[j + 16] = ((b[6 + j] >> 4) | (int)(((qh >> (j + 16)) & 1u) << 4)) - 16;
            }
            break;
        }
        case SIQ_Q8_0: {
            v->n = 32; v->d = siq_f16_to_f32(rd16(b));
            for (int j = 0; j < 32; j++) v->q[j] = (int8_t)b[2 + j];
            break;
        }
        case SIQ_Q2_K: {
            const uint8_t *sc = b, *qs = b + 16;
            v->n = 256; v->d = siq_f16_to_f32(rd16(b + 80));
            v->dmin = siq_f16_to_f32(rd16(b + 82));
            for (int i = 0; i < 256; i++) {
                const int h = i >> 7, s = (i >> 5) & 3, l = i & 31;
                v->q[i] = (qs[32 * h + l] >> (2 * s)) & 3;
                v->s[i] = sc[i >> 4] & 15;
                v->m[i] = sc[i >> 4] >> 4;
            }
            return 1;
        }
        case SIQ_Q3_K: {
            const uint8_t *hm = b, *qs = b + 32, *sc = b + 96;
            v->n = 256; v->d = siq_f16_to_f32(rd16(b + 108));
            for (int i = 0; i < 256; i++) {
                const int h = i >> 7, s = (i >> 5) & 3, l = i & 31;
                const int low = (qs[32 * h + l] >> (2 * s)) & 3;
                const int hb = (hm[l] >> (4 * h + s)) & 1;
                v->q[i] = low - (hb ? 0 : 4);
                v->s[i] = k3_scale(sc, i >> 4);
                v->m[i] = 0;
            }
            return 1;
        }
        case SIQ_Q4_K:
        case SIQ_Q5_K: {
            const int five = type == SIQ_Q5_K;
            const uint8_t *sc = b + 4, *qh = b + 16, *qs = b + (five ? 48 : 16);
            v->n = 256; v->d = siq_f16_to_f32(rd16(b));
            v->dmin = siq_f16_to_f32(rd16(b + 2));
            for (int i = 0; i < 256; i++) {
                const int c = i >> 6, r = i & 63, l = r & 31, hi = r >> 5;
                const int j = 2 * c + hi; /* 32-element sub-block */
                int q = hi ? (qs[32 * c + l] >> 4) : (qs[32 * c + l] & 15);
                if (five) q += 16 * ((qh[l] >> j) & 1);
                v->q[i] = q;
                k4_scale_min(sc, j, &v->s[i], &v->m[i]);
            }
            return 1;
        }
        case SIQ_Q6_K: {
            const uint8_t *ql = b, *qh = b + 128;
            const int8_t *sc = (const int8_t *)(b + 192);
            v->n = 256; v->d = siq_f16_to_f32(rd16(b + 208));
            for (int i = 0; i < 256; i++) {
                const int h = i >> 7, t = (i >> 5) & 3, l = i & 31;
                const uint8_t byte = ql[64 * h + l + 32 * (t & 1)];
                const int lo4 = t < 2 ? (byte & 15) : (byte >> 4);
                const int hi2 = (qh[32 * h + l] >> (2 * t)) & 3;
                v->q[i] = (lo4 | (hi2 << 4)) - 32;
                v->s[i] = sc[i >> 4];
                v->m[i] = 0;
            }
            return 1;
        }
        default: return 0;
    }
    for (int j = 0; j < v->n; j++) { v->s[j] = 1; v->m[j] = 0; }
    return 1;
}

/* ---- dequantization (reference kernels.c:599-817, float semantics) ----- */

int siq_dequant_row(uint32_t type, const void *w, float *out, int64_t n) {
    uint32_t be, bb;
    if (type == SIQ_F32) {
        memcpy(out, w, (size_t)n * sizeof(float));
        return 1;
    }
    if (type == SIQ_F16) {
        const uint8_t *p = w;
        for (int64_t i = 0; i < n; i++) out[i] = siq_f16_to_f32(rd16(p + 2 * i));
        return 1;
    }
    if (type == SIQ_F32) { memcpy(out, w, (size_t)n * 4); return 1; }
    if (!siq_geometry(type, &be, &bb) || type == SIQ_Q8_K) return 0;
    const uint8_t *p = w;
    blk_vals v;
    for (int64_t b = 0; b < n / be; b++, p += bb, out += be) {
        decode_block(type, p, &v);
        for (int i = 0; i < v.n; i++) {
            switch (type) {
                case SIQ_Q4_0: case SIQ_Q5_0: case SIQ_Q8_0:
                    out[i] = (float)v.q[i] * v.d;
                    break;
                case SIQ_Q2_K: case SIQ_Q4_K: case SIQ_Q5_K: {
                    const float dl = v.d * (float)v.s[i];
                    const float ml = v.dmin * (float)v.m[i];
                    out[i] = dl * (float)v.q[i] - ml;
                    break;
                }
                default: { /* Q3_K, Q6_K: no min term */
                    const float dl = v.d * (float)v.s[i];
                    out[i] = dl * (float)v.q[i];
                    break;
                }
            }
        }
    }
    return 1;
}

/* ---- exact dot products ------------------------------------------------- */

/* Activation element k of a pair-format row as (integer quant, scale). */
static void act_block(uint32_t pair, const uint8_t *a, int64_t blk, int *q,
                      double *d) {
    if (pair == SIQ_Q8_K) {
        const uint8_t *o = a + blk * 292;
        float df; memcpy(&df, o, 4);
        *d = df;
        for (int j = 0; j < 256; j++) q[j] = (int8_t)o[4 + j];
    } else { /* Q8_0 */
        const uint8_t *o = a + blk * 34;
        *d = siq_f16_to_f32(rd16(o));
        for (int j = 0; j < 32; j++) q[j] = (int8_t)o[2 + j];
    }
}

int siq_vec_dot(uint32_t wtype, int64_t n, const void *w, const void *a,
                double *dot, double *l1) {
    uint32_t pair, be, bb;
    if (!siq_pair(wtype, &pair)) return 0;
    double s = 0.0, m = 0.0;
    if (wtype == SIQ_F32) {
        /* reference si_dot_f32 (kernels.c:180-187) sums the float products
         * in double; here each product is exact (24 + 24 bits) */
        const float *pw = w, *pa = a;
        for (int64_t i = 0; i < n; i++) {
            const double t = (double)pw[i] * (double)pa[i];
            s += t; m += fabs(t);
        }
        *dot = s; if (l1) *l1 = m;
        return 1;
    }
    if (wtype == SIQ_F16) {
        const uint8_t *pw = w, *pa = a;
        for (int64_t i = 0; i < n; i++) {
            const double t = (double)siq_f16_to_f32(rd16(pw + 2 * i)) *
                             (double)siq_f16_to_f32(rd16(pa + 2 * i));
            s += t; m += fabs(t);
        }
        *dot = s; if (l1) *l1 = m;
        return 1;
    }
    siq_geometry(wtype, &be, &bb);
    const uint8_t *pw = w;
    blk_vals v;
    int qa[256];
    double da;
    float wf[256];
    for (int64_t b = 0; b < n / be; b++, pw += bb) {
        decode_block(wtype, pw, &v);
        act_block(pair, a, b, qa, &da);
        int64_t s1 = 0, s2 = 0;
        for (int i = 0; i < v.n; i++) {
            s1 += (int64_t)v.s[i] * v.q[i] * qa[i];
            s2 += (int64_t)v.m[i] * qa[i];
        }
        s += (double)v.d * da * (double)s1 - (double)v.dmin * da * (double)s2;
        siq_dequant_row(wtype, pw, wf, v.n);
        for (int i = 0; i < v.n; i++) m += fabs((double)wf[i] * ((double)qa[i] * da));
    }
    *dot = s; if (l1) *l1 = m;
    return 1;
}

int siq_vec_dot_dequant(uint32_t wtype, int64_t n, const void *w,
                        const void *a, double *dot, double *l1) {
    uint32_t pair, be, bb;
    if (!siq_pair(wtype, &pair)) return 0;
    if (wtype == SIQ_F16 || wtype == SIQ_F32) return siq_vec_dot(wtype, n, w, a, dot, l1);
    siq_geometry(wtype, &be, &bb);
    float *wf = malloc((size_t)n * sizeof(float));
    if (!wf) return 0;
    siq_dequant_row(wtype, w, wf, n);
    /* activations: per-element value q*d; weights: float dequant. The
     * products are summed in double; the weight value d*s*q - dmin*m is
     * rounded to float here, so this agrees with siq_vec_dot only to
     * float precision of each weight. */
    double s = 0.0, m = 0.0;
    int qa[256];
    double da;
    const int64_t ab = pair == SIQ_Q8_K ? 256 : 32;
    for (int64_t b = 0; b < n / ab; b++) {
        act_block(pair, a, b, qa, &da);
        for (int j = 0; j < ab; j++) {
            const double t = (double)wf[b * ab + j] * ((double)qa[j] * da);
            s += t; m += fabs(t);
        }
    }
    free(wf);
    *dot = s; if (l1) *l1 = m;
    return 1;
}

/* ---- gemv driver (reference backend.c:17-120: convert once, then whole
 * rows per lane in contiguous chunks, per = ceil(n_out / lanes)) --------- */

typedef struct {
    uint32_t wtype;
    const uint8_t *W;
    int64_t n_out, n_in, row_bytes;
    const void *xq;
    float *y;
    double *l1;
    int lane, lanes;
} row_task;

static void *row_task_fn(void *p) {
    row_task *t = p;
    const int64_t per = (t->n_out + t->lanes - 1) / t->lanes;
    const int64_t r0 = (int64_t)t->lane * per;
    const int64_t r1 = r0 + per < t->n_out ? r0 + per : t->n_out;
    for (int64_t r = r0; r < r1; r++) {
        double d, m;
        siq_vec_dot(t->wtype, t->n_in, t->W + r * t->row_bytes, t->xq, &d, &m);
        t->y[r] = (float)d;
        if (t->l1) t->l1[r] = m;
    }
    return NULL;
}

static size_t pair_bytes(uint32_t pair, int64_t n) {
    switch (pair) {
        case SIQ_F32: return (size_t)n * 4;
        case SIQ_F16: return (size_t)n * 2;
        case SIQ_Q8_0: return (size_t)(n / 32) * 34;
        case SIQ_Q8_K: return (size_t)(n / 256) * 292;
        default: return 0;
    }
}

static int gemv_rows(uint32_t wtype, const void *W, int64_t n_out,
                     int64_t n_in, const void *xq, float *y, double *l1,
                     int lanes) {
    uint32_t be, bb;
    if (!siq_geometry(wtype, &be, &bb) || n_in % be) return 0;
    if (lanes < 1) lanes = 1;
    if (lanes > 256) lanes = 256;
    row_task t[256];
    pthread_t th[256];
    for (int i = 0; i < lanes; i++) {
        t[i] = (row_task){ wtype, W, n_out, n_in, (n_in / be) * bb, xq, y, l1, i, lanes };
    }
    int started = 1;
    for (int i = 1; i < lanes; i++, started++) {
        if (pthread_create(&th[i], NULL, row_task_fn, &t[i]) != 0) break;
    }
    row_task_fn(&t[0]);
    for (int i = 1; i < started; i++) pthread_join(th[i], NULL);
    for (int i = started; i < lanes; i++) row_task_fn(&t[i]); /* degraded */
    return 1;
}

int siq_gemv(uint32_t wtype, const void *W, int64_t n_out, int64_t n_in,
             const float *x, float *y, double *l1, int lanes) {
    uint32_t pair;
    if (!siq_pair(wtype, &pair)) return 0;
    void *xq = malloc(pair_bytes(pair, n_in) + 1);
    if (!xq) return 0;
    siq_quantize_pair(pair, x, xq, n_in);
    const int ok = gemv_rows(wtype, W, n_out, n_in, xq, y, l1, lanes);
    free(xq);
    return ok;
}

int siq_gemm(uint32_t wtype, const void *W, int64_t n_out, int64_t n_in,
             const float *X, int64_t M, float *Y, double *L1, int lanes) {
    for (int64_t m = 0; m < M; m++) {
        if (!siq_gemv(wtype, W, n_out, n_in, X + m * n_in, Y + m * n_out,
                      L1 ? L1 + m * n_out : NULL, lanes)) {
            return 0;
        }
    }
    return 1;
}

/* ---- decode attention over an f16 KV cache ------------------------------
 * Restates reference engine.c:90-147 (attn_head) with the pieces its x86
 * build dispatches to: the f16 dot of kernels_avx2.c:118-148, the softmax
 * of kernels.c:855-885 and its exp polynomial, kernels.c:820-850. Unlike
 * the quantized dots above, these are reproduced in the reference's own
 * floating-point operation order, since their results feed an f16 rounding
 * (the probabilities) that an exact evaluation would not reproduce. */

float siq_expf_poly(float x) {
    /* x = n*ln2 + b: n from the 1.5*2^23 rounding shift, ln2 in two parts */
    const float shift = 0x1.8p23f;
    const float z = fmaf(x, 0x1.715476p+0f, shift);
    const float n = z - shift;
    const float b = fmaf(-n, 0x1.7f7d1cp-20f, fmaf(-n, 0x1.62e4p-1f, x));
    /* 2^n: the integer in z's low mantissa bits moved to the exponent */
    const uint32_t e = f2u(z) << 23;
    const float k = u2f(e + 0x3f800000u);
    const float u = b * b;
    const float p = fmaf(fmaf(fmaf(0x1.0e4020p-7f, b, 0x1.573e2ep-5f), u,
                              fmaf(0x1.555e66p-3f, b, 0x1.fffdb6p-2f)),
                         u, 0x1.ffffecp-1f * b);
    if (!(fabsf(n) > 126.0f)) return fmaf(p, k, k);
    /* |n| > 126: 2^n split over two factors; |n| > 192: over/underflow */
    const uint32_t g = n <= 0.0f ? 0x82000000u : 0u;
    const float s1 = u2f(g + 0x7f000000u);
    if (fabsf(n) > 192.0f) return s1 * s1;
    const float s2 = u2f(e - g);
    return fmaf(s2, p, s2) * s1;
}

void siq_softmax(float *y, const float *x, int64_t n, float max) {
    double total = 0.0;
    int64_t i = 0;
    for (; i + 8 <= n; i += 8) {
        float v[8];
        for (int k = 0; k < 8; k++) v[k] = y[i + k] = siq_expf_poly(x[i + k] - max);
        /* the 8-lane horizontal sum: lanes l and l+4, then pairs */
        const float a = (v[0] + v[4]) + (v[2] + v[6]);
        const float c = (v[1] + v[5]) + (v[3] + v[7]);
        total += (double)(a + c);
    }
    for (; i < n; i++) {
        const float val = expf(x[i] - max);
        total += (double)val;
        y[i] = val;
    }
    const float scale = (float)(1.0 / total);
    for (i = 0; i < n; i++) y[i] *= scale;
}

float siq_dot_f16_simd(int64_t n, const uint16_t *a, const uint16_t *b) {
    /* accumulator 8*r + l is lane l of register r: element i of every
     * 32-element step goes to accumulator i % 32 */
    float acc[32];
    for (int k = 0; k < 32; k++) acc[k] = 0.0f;
    const int64_t body = n & ~(int64_t)31;
    for (int64_t i = 0; i < body; i += 32)
        for (int k = 0; k < 32; k++)
            acc[k] = fmaf(siq_f16_to_f32(a[i + k]), siq_f16_to_f32(b[i + k]), acc[k]);
    /* registers r0 += r2, r1 += r3, r0 += r1; then lanes l + (l + 4);
     * then two pairwise rounds */
    float s[8];
    for (int l = 0; l < 8; l++) s[l] = (acc[l] + acc[16 + l]) + (acc[8 + l] + acc[24 + l]);
    float t[4];
    for (int l = 0; l < 4; l++) t[l] = s[l] + s[l + 4];
    double total = 0.0;
    total += (double)((t[0] + t[1]) + (t[2] + t[3]));
    for (int64_t i = body; i < n; i++)
        total += (double)(siq_f16_to_f32(a[i]) * siq_f16_to_f32(b[i]));
    return (float)total;
}

int siq_attn_decode(const float *q, const uint16_t *k, const uint16_t *v, int64_t n_head,
                    int64_t n_head_kv, int64_t hd, int64_t n_ctx, int64_t pos, float kq_scale,
                    float *out, float *scores, uint16_t *probs16) {
    if (n_head < 1 || n_head_kv < 1 || n_head % n_head_kv || hd < 1 || pos < 0 || pos >= n_ctx)
        return 0;
    const int64_t n = pos + 1, gqa = n_head / n_head_kv;
    float *sc = malloc((size_t)n * sizeof *sc);
    float *pr = malloc((size_t)n * sizeof *pr);
    uint16_t *p16 = malloc((size_t)n * sizeof *p16);
    uint16_t *q16 = malloc((size_t)hd * sizeof *q16);
    if (!sc || !pr || !p16 || !q16) {
        free(sc), free(pr), free(p16), free(q16);
        return 0;
    }
    for (int64_t h = 0; h < n_head; h++) {
        const int64_t hk = h / gqa;
        const uint16_t *kh = k + hk * n_ctx * hd;   /* [n_ctx][hd] */
        const uint16_t *vh = v + hk * hd * n_ctx;   /* [hd][n_ctx] */
        for (int64_t d = 0; d < hd; d++) q16[d] = siq_f32_to_f16(q[h * hd + d]);
        float max = -INFINITY;
        for (int64_t j = 0; j < n; j++) {
            sc[j] = siq_dot_f16_simd(hd, kh + j * hd, q16) * kq_scale;
            if (sc[j] > max) max = sc[j];
        }
        siq_softmax(pr, sc, n, max);
        for (int64_t j = 0; j < n; j++) p16[j] = siq_f32_to_f16(pr[j]);
        for (int64_t c = 0; c < hd; c++) out[h * hd + c] = siq_dot_f16_simd(n, vh + c * n_ctx, p16);
        if (scores) memcpy(scores + h * n_ctx, sc, (size_t)n * sizeof *sc);
        if (probs16) memcpy(probs16 + h * n_ctx, p16, (size_t)n * sizeof *p16);
    }
    free(sc), free(pr), free(p16), free(q16);
    return 1;
}
