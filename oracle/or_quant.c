/* or_quant.c - oracle restatement of the block codecs and the Q8_K integer
 * dot products (TEST INFRASTRUCTURE, see oracle.h).
 *
 * Reference: src/ornith_quant.c (codecs) and src/ornith_qdot.c (Q8_K dots).
 * Every float expression keeps the reference's evaluation order; the build
 * uses -std=c11 -ffp-contract=off so no multiply-add is fused.
 */
#include "oracle.h"
#include "ornith_iq2xxs_grid.h"
#include <math.h>
#include <string.h>
#include <stdio.h>
#include <stdarg.h>

static char g_err[256];
const char *orc_last_error(void) { return g_err; }
void orc_seterr(const char *fmt, ...) {
    va_list ap; va_start(ap, fmt); vsnprintf(g_err, sizeof g_err, fmt, ap); va_end(ap);
}

static inline uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline void wr16(uint8_t *p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }

/* ---- binary16 <-> binary32 (src/ornith_quant.c:14-65) -------------------
 * f32->f16 rounds to nearest-even, including the subnormal range; NaN keeps a
 * quiet payload bit. f16->f32 is exact. */
uint16_t orc_f32_to_f16(float f) {
    uint32_t b; memcpy(&b, &f, 4);
    const uint32_t s = (b >> 16) & 0x8000u;
    const int32_t  e = (int32_t)((b >> 23) & 0xff);
    uint32_t m = b & 0x7fffffu;
    if (e == 0xff) return (uint16_t)(s | 0x7c00u | (m ? 0x200u : 0u));
    int32_t he = e - 112;                    /* 127 - 15 */
    if (he >= 31) return (uint16_t)(s | 0x7c00u);
    if (he <= 0) {
        if (he < -10) return (uint16_t)s;
        m |= 0x800000u;
        const uint32_t sh = (uint32_t)(14 - he);
        uint32_t h = m >> sh;
        const uint32_t rem = m & ((1u << sh) - 1u), half = 1u << (sh - 1);
        if (rem > half || (rem == half && (h & 1u))) h++;
        return (uint16_t)(s | h);
    }
    uint32_t h = s | ((uint32_t)he << 10) | (m >> 13);
    const uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)h;
}

float orc_f16_to_f32(uint16_t h) {
    const uint32_t s = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu, b;
    if (e == 0) {
        if (m == 0) b = s;
        else {                                /* subnormal: renormalise */
            int32_t ex = 113;
            while (!(m & 0x400u)) { m <<= 1; ex--; }
            b = s | ((uint32_t)ex << 23) | ((m & 0x3ffu) << 13);
        }
    } else if (e == 31) b = s | 0x7f800000u | (m << 13);
    else b = s | ((e + 112) << 23) | (m << 13);
    float f; memcpy(&f, &b, 4); return f;
}

static uint16_t f32_to_bf16(float f) {
    uint32_t x; memcpy(&x, &f, 4);
    if (((x >> 23) & 0xffu) == 0xffu) return (uint16_t)(x >> 16);
    x += 0x7fffu + ((x >> 16) & 1u);
    return (uint16_t)(x >> 16);
}
static float bf16_to_f32(uint16_t v) {
    uint32_t x = (uint32_t)v << 16; float f; memcpy(&f, &x, 4); return f;
}

/* ---- geometry (src/ornith_quant.c:89-146) ------------------------------ */
size_t orc_block_elems(uint32_t t) {
    switch (t) {
    case ORC_F32: case ORC_F16: case ORC_BF16: return 1;
    case ORC_Q8_0: case ORC_Q4_0: return 32;
    case ORC_Q2_K: case ORC_Q4_K: case ORC_Q5_K: case ORC_Q6_K: case ORC_IQ2_XXS: return 256;
    default: return 0;
    }
}
size_t orc_block_bytes(uint32_t t) {
    switch (t) {
    case ORC_F32: return 4;
    case ORC_F16: case ORC_BF16: return 2;
    case ORC_Q8_0: return 34;
    case ORC_Q4_0: return 18;
    case ORC_Q2_K: return 84;
    case ORC_Q4_K: return 144;
    case ORC_Q5_K: return 176;
    case ORC_Q6_K: return 210;
    case ORC_IQ2_XXS: return 66;
    default: return 0;
    }
}
size_t orc_row_bytes(uint32_t t, size_t n) {
    const size_t be = orc_block_elems(t);
    if (!be || n % be) return 0;
    return n / be * orc_block_bytes(t);
}

/* ---- Q8_0: {f16 d; i8 q[32]} (src/ornith_quant.c:155-184) ---------------
 * d = amax/127 (stored as f16, but the reciprocal uses the f32 d);
 * q = lroundf(x/d) clamped to +-127. */
static void enc_q8_0(const float *x, uint8_t *o, size_t nblk) {
    for (size_t b = 0; b < nblk; b++, x += 32, o += 34) {
        float amax = 0.0f;
        for (int j = 0; j < 32; j++) { float a = fabsf(x[j]); if (a > amax) amax = a; }
        const float d = amax / 127.0f;
        const float id = d ? 1.0f / d : 0.0f;
        wr16(o, orc_f32_to_f16(d));
        for (int j = 0; j < 32; j++) {
            long q = lroundf(x[j] * id);
            q = q > 127 ? 127 : (q < -127 ? -127 : q);
            o[2 + j] = (uint8_t)(int8_t)q;
        }
    }
}
static void dec_q8_0(const uint8_t *o, float *y, size_t nblk) {
    for (size_t b = 0; b < nblk; b++, o += 34, y += 32) {
        const float d = orc_f16_to_f32(rd16(o));
        for (int j = 0; j < 32; j++) y[j] = (float)(int8_t)o[2 + j] * d;
    }
}

/* ---- Q4_K: {f16 d; f16 dmin; u8 scales[12]; u8 qs[128]} -----------------
 * 8 sub-blocks of 32 with 6-bit (scale, min) pairs packed as in ggml
 * (src/ornith_quant.c:230-245, 381-399, 507-561). */
static void q4k_unpack(int j, const uint8_t *q, uint8_t *sc, uint8_t *mn) {
    if (j < 4) { *sc = q[j] & 63; *mn = q[j + 4] & 63; return; }
    *sc = (uint8_t)((q[j + 4] & 0x0f) | ((q[j - 4] >> 6) << 4));
    *mn = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
}
static void q4k_pack(uint8_t *q, const uint8_t *sc, const uint8_t *mn) {
    memset(q, 0, 12);
    for (int j = 0; j < 4; j++) { q[j] = sc[j] & 63; q[j + 4] = mn[j] & 63; }
    for (int j = 4; j < 8; j++) {
        q[j + 4] = (uint8_t)((sc[j] & 0x0f) | ((mn[j] & 0x0f) << 4));
        q[j - 4] |= (uint8_t)(((sc[j] >> 4) & 3) << 6);
        q[j]     |= (uint8_t)(((mn[j] >> 4) & 3) << 6);
    }
}
static void enc_q4_k(const float *x, uint8_t *p, size_t nblk) {
    for (size_t b = 0; b < nblk; b++, x += 256, p += 144) {
        float ssc[8], smn[8];
        for (int j = 0; j < 8; j++) {
            const float *v = x + 32 * j;
            float lo = v[0], hi = v[0];
            for (int l = 1; l < 32; l++) { if (v[l] < lo) lo = v[l]; if (v[l] > hi) hi = v[l]; }
            if (lo > 0.0f) lo = 0.0f;
            ssc[j] = (hi - lo) / 15.0f;
            smn[j] = -lo;
        }
        float msc = 0.0f, mmn = 0.0f;
        for (int j = 0; j < 8; j++) { if (ssc[j] > msc) msc = ssc[j]; if (smn[j] > mmn) mmn = smn[j]; }
        const float d = msc / 63.0f, dmin = mmn / 63.0f;
        const float id = d ? 1.0f / d : 0.0f, idm = dmin ? 1.0f / dmin : 0.0f;
        uint8_t sc[8], mn[8];
        for (int j = 0; j < 8; j++) {
            long s = lroundf(ssc[j] * id), m = lroundf(smn[j] * idm);
            sc[j] = (uint8_t)(s < 0 ? 0 : (s > 63 ? 63 : s));
            mn[j] = (uint8_t)(m < 0 ? 0 : (m > 63 ? 63 : m));
        }
        wr16(p, orc_f32_to_f16(d));
        wr16(p + 2, orc_f32_to_f16(dmin));
        q4k_pack(p + 4, sc, mn);
        uint8_t *qs = p + 16;
        memset(qs, 0, 128);
        for (int j = 0; j < 8; j++) {
            /* the f32 (not f16-rounded) d/dmin set the quantisation grid */
            const float rs = d * sc[j], rm = dmin * mn[j];
            const float irs = rs ? 1.0f / rs : 0.0f;
            const float *v = x + 32 * j;
            uint8_t *dst = qs + 32 * (j / 2);
            for (int l = 0; l < 32; l++) {
                long q = lroundf((v[l] + rm) * irs);
                q = q < 0 ? 0 : (q > 15 ? 15 : q);
                dst[l] |= (uint8_t)((j & 1) ? (q << 4) : q);
            }
        }
    }
}
static void dec_q4_k(const uint8_t *p, float *y, size_t nblk) {
    for (size_t b = 0; b < nblk; b++, p += 144, y += 256) {
        const float d = orc_f16_to_f32(rd16(p)), dmin = orc_f16_to_f32(rd16(p + 2));
        const uint8_t *qs = p + 16;
        for (int pair = 0; pair < 4; pair++) {
            uint8_t sc, mn;
            q4k_unpack(2 * pair, p + 4, &sc, &mn);
            const float d1 = d * sc, m1 = dmin * mn;
            q4k_unpack(2 * pair + 1, p + 4, &sc, &mn);
            const float d2 = d * sc, m2 = dmin * mn;
            const uint8_t *q = qs + 32 * pair;
            float *o = y + 64 * pair;
            for (int l = 0; l < 32; l++) o[l] = d1 * (q[l] & 0xf) - m1;
            for (int l = 0; l < 32; l++) o[32 + l] = d2 * (q[l] >> 4) - m2;
        }
    }
}

/* ---- Q6_K: {u8 ql[128]; u8 qh[64]; i8 sc[16]; f16 d} --------------------
 * value = d * sc[g] * (q - 32), q 6-bit (src/ornith_quant.c:424-500). Within
 * each 128-half, element l+32k (k=0..3) takes its low nibble from
 * ql[l + 32*(k&1)] (k<2 low half-byte, else high) and its two high bits from
 * qh[l] bits 2k..2k+1. */
static void enc_q6_k(const float *x, uint8_t *p, size_t nblk) {
    for (size_t b = 0; b < nblk; b++, x += 256, p += 210) {
        float gs[16], maxs = 0.0f;
        for (int g = 0; g < 16; g++) {
            float amax = 0.0f;
            for (int l = 0; l < 16; l++) { float a = fabsf(x[16 * g + l]); if (a > amax) amax = a; }
            gs[g] = amax / 32.0f;
            if (gs[g] > maxs) maxs = gs[g];
        }
        const float d = maxs / 127.0f, id = d ? 1.0f / d : 0.0f;
        int8_t *sc = (int8_t *)(p + 192);
        wr16(p + 208, orc_f32_to_f16(d));
        for (int g = 0; g < 16; g++) {
            long s = lroundf(gs[g] * id);
            sc[g] = (int8_t)(s < 0 ? 0 : (s > 127 ? 127 : s));
        }
        uint8_t Q[256];
        for (int g = 0; g < 16; g++) {
            const float sg = d * sc[g], isg = sg ? 1.0f / sg : 0.0f;
            for (int l = 0; l < 16; l++) {
                long q = lroundf(x[16 * g + l] * isg) + 32;
                Q[16 * g + l] = (uint8_t)(q < 0 ? 0 : (q > 63 ? 63 : q));
            }
        }
        uint8_t *ql = p, *qh = p + 128;
        for (int h = 0; h < 2; h++) {
            const uint8_t *q = Q + 128 * h;
            for (int l = 0; l < 32; l++) {
                ql[64 * h + l]      = (uint8_t)((q[l] & 15) | ((q[l + 64] & 15) << 4));
                ql[64 * h + 32 + l] = (uint8_t)((q[l + 32] & 15) | ((q[l + 96] & 15) << 4));
                qh[32 * h + l] = (uint8_t)((q[l] >> 4) | ((q[l + 32] >> 4) << 2) |
                                           ((q[l + 64] >> 4) << 4) | ((q[l + 96] >> 4) << 6));
            }
        }
    }
}
static void dec_q6_k(const uint8_t *p, float *y, size_t nblk) {
    for (size_t b = 0; b < nblk; b++, p += 210, y += 256) {
        const float d = orc_f16_to_f32(rd16(p + 208));
        const int8_t *sc = (const int8_t *)(p + 192);
        for (int h = 0; h < 2; h++) {
            const uint8_t *ql = p + 64 * h, *qh = p + 128 + 32 * h;
            const int8_t *s = sc + 8 * h;
            float *o = y + 128 * h;
            for (int l = 0; l < 32; l++) {
                const int is = l / 16;
                const int q1 = ((ql[l] & 15) | (((qh[l] >> 0) & 3) << 4)) - 32;
                const int q2 = ((ql[l + 32] & 15) | (((qh[l] >> 2) & 3) << 4)) - 32;
                const int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                const int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                o[l]      = d * s[is + 0] * q1;
                o[l + 32] = d * s[is + 2] * q2;
                o[l + 64] = d * s[is + 4] * q3;
                o[l + 96] = d * s[is + 6] * q4;
            }
        }
    }
}

/* ---- IQ2_XXS: {f16 d; u16 qs[32]} (src/ornith_quant.c:563-789) ----------
 * Per 32-group: word0 = four 8-bit grid indices, word1 = four 7-bit sign
 * indices (bit 7 of each sign byte is the parity of the low 7) plus a 4-bit
 * scale in bits 28..31. y = d*(0.5+ls)*0.25 * grid_byte * sign. */
static const uint64_t k_grid[256] = { ORNITH_IQ2XXS_GRID_VALUES };

static inline uint8_t grid_mag(int g, int j) { return (uint8_t)(k_grid[g] >> (8 * j)); }
static inline uint8_t sign_byte(uint32_t idx7) {
    return (uint8_t)(idx7 | ((uint32_t)__builtin_popcount(idx7) & 1u) << 7);
}
static inline uint32_t rd32le(const uint8_t *p) {
    return (uint32_t)rd16(p) | ((uint32_t)rd16(p + 2) << 16);
}

static void dec_iq2_xxs(const uint8_t *p, float *y, size_t nblk) {
    for (size_t b = 0; b < nblk; b++, p += 66) {
        const float d = orc_f16_to_f32(rd16(p));
        for (int g32 = 0; g32 < 8; g32++) {
            const uint32_t w0 = rd32le(p + 2 + 8 * g32), w1 = rd32le(p + 6 + 8 * g32);
            const float db = d * (0.5f + (float)(w1 >> 28)) * 0.25f;
            for (int k = 0; k < 4; k++) {
                const int gi = (int)((w0 >> (8 * k)) & 0xff);
                const uint8_t sg = sign_byte((w1 >> (7 * k)) & 127u);
                for (int j = 0; j < 8; j++)
                    *y++ = db * grid_mag(gi, j) * ((sg >> j & 1) ? -1.0f : 1.0f);
            }
        }
    }
}

/* nearest grid point to an 8-magnitude target at scale s (unit weights) */
static int iq2_best(const float *mag, float s, float *err) {
    int best = 0; float be = 1e30f;
    for (int g = 0; g < 256; g++) {
        float e = 0.0f;
        for (int j = 0; j < 8; j++) {
            const float df = mag[j] - s * (float)grid_mag(g, j);
            e += 1.0f * df * df;
        }
        if (e < be) { be = e; best = g; }
    }
    if (err) *err = be;
    return best;
}

static void enc_iq2_xxs(const float *x, uint8_t *p, size_t nblk) {
    for (size_t b = 0; b < nblk; b++, x += 256, p += 66) {
        memset(p, 0, 66);
        float mag[8][4][8], gsc[8];
        uint8_t sgn[8][4];
        for (int g32 = 0; g32 < 8; g32++) {
            float gmax = 0.0f;
            for (int k = 0; k < 4; k++) {
                const float *v = x + 32 * g32 + 8 * k;
                uint8_t s = 0; int nneg = 0;
                for (int j = 0; j < 8; j++) {
                    const float a = v[j] < 0.0f ? -v[j] : v[j];
                    if (v[j] < 0.0f) { s |= (uint8_t)(1u << j); nneg++; }
                    mag[g32][k][j] = a;
                    if (a > gmax) gmax = a;
                }
                if (nneg & 1) {             /* odd: flip the smallest magnitude */
                    int jm = 0; float vm = mag[g32][k][0];
                    for (int j = 1; j < 8; j++) if (mag[g32][k][j] < vm) { vm = mag[g32][k][j]; jm = j; }
                    s ^= (uint8_t)(1u << jm);
                }
                sgn[g32][k] = s & 127;
            }
            if (gmax < 1e-12f) { gsc[g32] = 0.0f; continue; }
            const float base = gmax / 43.0f;
            float best_s = base, best_e = 1e30f;
            for (int t = 4; t <= 64; t++) {
                const float s = base * 43.0f / (float)t;
                float tot = 0.0f, e;
                for (int k = 0; k < 4; k++) { iq2_best(mag[g32][k], s, &e); tot += e; }
                if (tot < best_e) { best_e = tot; best_s = s; }
            }
            gsc[g32] = best_s;
        }
        float mx = 0.0f;
        for (int g32 = 0; g32 < 8; g32++) if (gsc[g32] > mx) mx = gsc[g32];
        if (mx <= 0.0f) { wr16(p, orc_f32_to_f16(0.0f)); continue; }
        float d = mx / (0.25f * 15.5f);
        wr16(p, orc_f32_to_f16(d));
        d = orc_f16_to_f32(rd16(p));
        const float qd = 0.25f * d;
        for (int g32 = 0; g32 < 8; g32++) {
            long l = 0;
            if (qd > 0.0f && gsc[g32] > 0.0f) l = lroundf(gsc[g32] / qd - 0.5f);
            l = l < 0 ? 0 : (l > 15 ? 15 : l);
            const float db = qd * (0.5f + (float)l);
            uint32_t w0 = 0, w1 = 0;
            for (int k = 0; k < 4; k++) {
                const int g = db > 0.0f ? iq2_best(mag[g32][k], db, NULL) : 0;
                w0 |= (uint32_t)g << (8 * k);
                w1 |= (uint32_t)sgn[g32][k] << (7 * k);
            }
            w1 |= (uint32_t)l << 28;
            uint8_t *q = p + 2 + 8 * g32;
            wr16(q, (uint16_t)w0); wr16(q + 2, (uint16_t)(w0 >> 16));
            wr16(q + 4, (uint16_t)w1); wr16(q + 6, (uint16_t)(w1 >> 16));
        }
    }
}

/* ---- dispatch (src/ornith_quant.c:871-1073) ----------------------------- */
int orc_quantize(uint32_t t, const float *src, void *dst, size_t n) {
    const size_t be = orc_block_elems(t);
    if (!be || t == ORC_Q4_0 || t == ORC_Q2_K || t == ORC_Q5_K) {
        orc_seterr("orc_quantize: type %u not implemented", t);
        return ORC_ERR_UNSUPPORTED;
    }
    if (n % be) { orc_seterr("type %u needs a multiple of %zu", t, be); return ORC_ERR_FORMAT; }
    uint8_t *o = dst;
    switch (t) {
    case ORC_F32: memcpy(dst, src, n * 4); break;
    case ORC_F16: for (size_t i = 0; i < n; i++) wr16(o + 2 * i, orc_f32_to_f16(src[i])); break;
    case ORC_BF16: for (size_t i = 0; i < n; i++) wr16(o + 2 * i, f32_to_bf16(src[i])); break;
    case ORC_Q8_0: enc_q8_0(src, o, n / 32); break;
    case ORC_Q4_K: enc_q4_k(src, o, n / 256); break;
    case ORC_Q6_K: enc_q6_k(src, o, n / 256); break;
    case ORC_IQ2_XXS: enc_iq2_xxs(src, o, n / 256); break;
    }
    return ORC_OK;
}

int orc_dequantize(uint32_t t, const void *src, float *dst, size_t n) {
    const size_t be = orc_block_elems(t);
    if (!be || t == ORC_Q4_0 || t == ORC_Q2_K || t == ORC_Q5_K) {
        orc_seterr("orc_dequantize: type %u not implemented", t);
        return ORC_ERR_UNSUPPORTED;
    }
    if (n % be) { orc_seterr("type %u needs a multiple of %zu", t, be); return ORC_ERR_FORMAT; }
    const uint8_t *s = src;
    switch (t) {
    case ORC_F32: memcpy(dst, src, n * 4); break;
    case ORC_F16: for (size_t i = 0; i < n; i++) dst[i] = orc_f16_to_f32(rd16(s + 2 * i)); break;
    case ORC_BF16: for (size_t i = 0; i < n; i++) dst[i] = bf16_to_f32(rd16(s + 2 * i)); break;
    case ORC_Q8_0: dec_q8_0(s, dst, n / 32); break;
    case ORC_Q4_K: dec_q4_k(s, dst, n / 256); break;
    case ORC_Q6_K: dec_q6_k(s, dst, n / 256); break;
    case ORC_IQ2_XXS: dec_iq2_xxs(s, dst, n / 256); break;
    }
    return ORC_OK;
}

/* ---- Q8_K activation quantisation (src/ornith_qdot.c:32-62) -------------
 * The signed value of the FIRST largest-magnitude element sets
 * iscale = -127/max; q = clamp(rint(iscale*x), -128, 127); d = 1/iscale. */
void orc_quantize_q8k(const float *x, orc_q8k *y, int64_t k) {
    for (int64_t b = 0; b < k / 256; b++, x += 256) {
        float amax = 0.0f, mx = 0.0f;
        for (int j = 0; j < 256; j++) {
            const float a = fabsf(x[j]);
            if (a > amax) { amax = a; mx = x[j]; }
        }
        orc_q8k *o = &y[b];
        if (amax == 0.0f) { memset(o, 0, sizeof *o); continue; }
        const float iscale = -127.0f / mx;
        for (int j = 0; j < 256; j++) {
            long v = lrintf(iscale * x[j]);
            o->qs[j] = (int8_t)(v > 127 ? 127 : (v < -128 ? -128 : v));
        }
        for (int g = 0; g < 16; g++) {
            int s = 0;
            for (int l = 0; l < 16; l++) s += o->qs[16 * g + l];
            o->bsums[g] = (int16_t)s;
        }
        o->d = 1.0f / iscale;
    }
}

int orc_qdot_can(uint32_t t, int n) {
    return n % 256 == 0 && (t == ORC_Q4_K || t == ORC_Q6_K || t == ORC_Q8_0);
}

/* Integer inner sums are exact; the per-super-block float terms are added in
 * super-block order (src/ornith_qdot.c:76-163). */
float orc_qdot(uint32_t t, int n, const void *wrow, const orc_q8k *y) {
    const uint8_t *w = wrow;
    const int nb = n / 256;
    float acc = 0.0f;
    if (t == ORC_Q4_K) {
        for (int i = 0; i < nb; i++, w += 144) {
            const float d = y[i].d * orc_f16_to_f32(rd16(w));
            const float dm = -y[i].d * orc_f16_to_f32(rd16(w + 2));
            int mins = 0, dots = 0;
            for (int j = 0; j < 8; j++) {
                uint8_t sc, mn;
                q4k_unpack(j, w + 4, &sc, &mn);
                mins += mn * (y[i].bsums[2 * j] + y[i].bsums[2 * j + 1]);
                const uint8_t *q = w + 16 + 32 * (j >> 1);
                const int sh = 4 * (j & 1);
                int s = 0;
                for (int l = 0; l < 32; l++) s += ((q[l] >> sh) & 15) * y[i].qs[32 * j + l];
                dots += s * sc;
            }
            acc += d * (float)dots + dm * (float)mins;
        }
    } else if (t == ORC_Q6_K) {
        for (int i = 0; i < nb; i++, w += 210) {
            const float d = y[i].d * orc_f16_to_f32(rd16(w + 208));
            const int8_t *sc = (const int8_t *)(w + 192);
            int dots = 0;
            for (int h = 0; h < 2; h++) {
                const uint8_t *ql = w + 64 * h, *qh = w + 128 + 32 * h;
                const int8_t *q8 = y[i].qs + 128 * h, *s = sc + 8 * h;
                for (int l = 0; l < 32; l++) {
                    const int is = l / 16;
                    dots += q8[l]      * (((ql[l] & 15) | (((qh[l] >> 0) & 3) << 4)) - 32) * s[is + 0]
                          + q8[l + 32] * (((ql[l + 32] & 15) | (((qh[l] >> 2) & 3) << 4)) - 32) * s[is + 2]
                          + q8[l + 64] * (((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32) * s[is + 4]
                          + q8[l + 96] * (((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32) * s[is + 6];
                }
            }
            acc += d * (float)dots;
        }
    } else if (t == ORC_Q8_0) {
        for (int i = 0; i < nb; i++) {
            float part = 0.0f;
            for (int sb = 0; sb < 8; sb++, w += 34) {
                const int8_t *q = (const int8_t *)(w + 2), *a = y[i].qs + 32 * sb;
                int s = 0;
                for (int l = 0; l < 32; l++) s += q[l] * a[l];
                part += orc_f16_to_f32(rd16(w)) * (float)s;
            }
            acc += y[i].d * part;
        }
    }
    return acc;
}
