// oh_mv.hip - ornith_qdot on CDNA4: Q8_K activation quantisation, the
// quant-aware matvec over Q8_0 / Q4_K / Q6_K planes, the f32-fallback matvec
// (F32/F16/BF16/IQ2_XXS rows) and plane-layout decode.
//
// Exactness contract (reference src/ornith_qdot.c, src/ornith_rforward.c:100-134):
//  * Q8_K codes, bsums and d are bit-identical to qdot_quantize_row_q8_K.
//  * Each Q8_K-path dot is bit-identical to qdot_vec_dot: the integer inner
//    sums are exact in any order; the per-super-block float term and the
//    sequential super-block sum keep the reference's operation order.
//  * The fallback dot keeps ot_dot's strictly sequential f32 accumulation
//    (one lane walks one row).
//
// Work mapping of the Q8_K path: a wave64 is 8 groups x 8 lanes; a group owns
// one 256-element super-block and each lane 32 of its weights, loaded with
// 8/16-byte vector loads from the plane layout (contiguous across the
// group). A wave unit is one row (nb >= 8 super-blocks per row, in passes of
// 8) or 8/nb rows (nb < 8).
#include "oh_common.h"
#include "oh_types.h"
#include "../../include/ornith_iq2xxs_grid.h"

__constant__ uint64_t k_iq2_grid[256] = { ORNITH_IQ2XXS_GRID_VALUES };

namespace {

constexpr int kWavesPerBlock = 4;
constexpr int kUnitsPerWave = 2;

OH_DEV uint32_t wsel(const uint4 &v, int k) {   // 32-bit word k of a uint4
    return k == 0 ? v.x : (k == 1 ? v.y : (k == 2 ? v.z : v.w));
}
OH_DEV uint32_t bsel(const uint4 &v, int k) {   // byte k of a uint4
    return (wsel(v, k >> 2) >> (8 * (k & 3))) & 0xffu;
}

// 6-bit (scale, min) of sub-block j from the 12 packed bytes that start at
// byte 4 of the Q4_K header (src/ornith_qdot.c:66-72).
OH_DEV void q4k_sm(const uint4 &hdr, int j, int &sc, int &mn) {
    if (j < 4) {
        sc = (int)(bsel(hdr, 4 + j) & 63u);
        mn = (int)(bsel(hdr, 8 + j) & 63u);
    } else {
        sc = (int)((bsel(hdr, 8 + j) & 0xfu) | ((bsel(hdr, j) >> 6) << 4));
        mn = (int)((bsel(hdr, 8 + j) >> 4) | ((bsel(hdr, 4 + j) >> 6) << 4));
    }
}

OH_DEV int group_isum(int v) {     // exact sum over the 8 lanes of a group
    v += shfl_xor(v, 1); v += shfl_xor(v, 2); v += shfl_xor(v, 4);
    return v;
}

// Float term of super-block sb for the group's row; identical in all 8 lanes.
// bi = row*nb + sb indexes the planes. c = lane within the group.
OH_DEV float term_q4k(const oh_mvseg &s, int64_t bi, int sb, int c) {
    const uint4 hdr = *(const uint4 *)(s.B + bi * 16);
    const uint4 q = *(const uint4 *)(s.A + bi * 128 + 16 * c);
    const int p = c >> 1, h = c & 1;
    const int8_t *aq = s.xqs + (int64_t)sb * 256;
    const int4 alo = *(const int4 *)(aq + 64 * p + 16 * h);
    const int4 ahi = *(const int4 *)(aq + 64 * p + 32 + 16 * h);
    int dlo = 0, dhi = 0;
    dlo = dot4((int)(q.x & 0x0f0f0f0fu), alo.x, dlo);
    dlo = dot4((int)(q.y & 0x0f0f0f0fu), alo.y, dlo);
    dlo = dot4((int)(q.z & 0x0f0f0f0fu), alo.z, dlo);
    dlo = dot4((int)(q.w & 0x0f0f0f0fu), alo.w, dlo);
    dhi = dot4((int)((q.x >> 4) & 0x0f0f0f0fu), ahi.x, dhi);
    dhi = dot4((int)((q.y >> 4) & 0x0f0f0f0fu), ahi.y, dhi);
    dhi = dot4((int)((q.z >> 4) & 0x0f0f0f0fu), ahi.z, dhi);
    dhi = dot4((int)((q.w >> 4) & 0x0f0f0f0fu), ahi.w, dhi);
    int sc0, mn0, sc1, mn1, scc, mnc;
    q4k_sm(hdr, 2 * p, sc0, mn0);
    q4k_sm(hdr, 2 * p + 1, sc1, mn1);
    q4k_sm(hdr, c, scc, mnc);
    const int16_t *bs = s.xbs + (int64_t)sb * 16;
    int isum = group_isum(sc0 * dlo + sc1 * dhi);
    int mins = group_isum(mnc * ((int)bs[2 * c] + (int)bs[2 * c + 1]));
    const float yd = s.xd[sb];
    const float d = yd * h2f((uint16_t)(hdr.x & 0xffffu));
    const float dm = -yd * h2f((uint16_t)(hdr.x >> 16));
    return d * (float)isum + dm * (float)mins;
}

OH_DEV float term_q6k(const oh_mvseg &s, int64_t bi, int sb, int c) {
    const int hh = c >> 2, m = c & 3;
    const uint8_t *a = s.A + bi * 192;
    const uint2 qa = *(const uint2 *)(a + 64 * hh + 8 * m);
    const uint2 qb = *(const uint2 *)(a + 64 * hh + 32 + 8 * m);
    const uint2 qh = *(const uint2 *)(a + 128 + 32 * hh + 8 * m);
    const uint4 scv = *(const uint4 *)(s.B + bi * 16);
    const int is = 8 * hh + (m >> 1);
    const int sc1 = (int)(int8_t)bsel(scv, is), sc2 = (int)(int8_t)bsel(scv, is + 2);
    const int sc3 = (int)(int8_t)bsel(scv, is + 4), sc4 = (int)(int8_t)bsel(scv, is + 6);
    const int8_t *aq = s.xqs + (int64_t)sb * 256 + 128 * hh + 8 * m;
    const int2 a1 = *(const int2 *)(aq), a2 = *(const int2 *)(aq + 32);
    const int2 a3 = *(const int2 *)(aq + 64), a4 = *(const int2 *)(aq + 96);
    int d1 = 0, d2 = 0, d3 = 0, d4 = 0, s1 = 0, s2 = 0, s3 = 0, s4 = 0;
#pragma unroll
    for (int w = 0; w < 2; w++) {
        const uint32_t la = w ? qa.y : qa.x, lb = w ? qb.y : qb.x, hb = w ? qh.y : qh.x;
        const int q1 = (int)((la & 0x0f0f0f0fu) | ((hb & 0x03030303u) << 4));
        const int q2 = (int)((lb & 0x0f0f0f0fu) | (((hb >> 2) & 0x03030303u) << 4));
        const int q3 = (int)(((la >> 4) & 0x0f0f0f0fu) | (((hb >> 4) & 0x03030303u) << 4));
        const int q4 = (int)(((lb >> 4) & 0x0f0f0f0fu) | (((hb >> 6) & 0x03030303u) << 4));
        const int x1 = w ? a1.y : a1.x, x2 = w ? a2.y : a2.x, x3 = w ? a3.y : a3.x, x4 = w ? a4.y : a4.x;
        d1 = dot4(q1, x1, d1); s1 = dot4(0x01010101, x1, s1);
        d2 = dot4(q2, x2, d2); s2 = dot4(0x01010101, x2, s2);
        d3 = dot4(q3, x3, d3); s3 = dot4(0x01010101, x3, s3);
        d4 = dot4(q4, x4, d4); s4 = dot4(0x01010101, x4, s4);
    }
    // sum_l q8 * (q - 32) * sc  ==  sc * (sum q8*q - 32 * sum q8), exactly
    const int part = sc1 * (d1 - 32 * s1) + sc2 * (d2 - 32 * s2) +
                     sc3 * (d3 - 32 * s3) + sc4 * (d4 - 32 * s4);
    const int isum = group_isum(part);
    const float d = s.xd[sb] * h2f(*(const uint16_t *)(s.C + bi * 2));
    return d * (float)isum;
}

OH_DEV float term_q8_0(const oh_mvseg &s, int64_t bi, int sb, int c) {
    const int8_t *w = (const int8_t *)(s.A + bi * 256 + 32 * c);
    const int4 w0 = *(const int4 *)w, w1 = *(const int4 *)(w + 16);
    const int8_t *aq = s.xqs + (int64_t)sb * 256 + 32 * c;
    const int4 a0 = *(const int4 *)aq, a1 = *(const int4 *)(aq + 16);
    int is = 0;
    is = dot4(w0.x, a0.x, is); is = dot4(w0.y, a0.y, is);
    is = dot4(w0.z, a0.z, is); is = dot4(w0.w, a0.w, is);
    is = dot4(w1.x, a1.x, is); is = dot4(w1.y, a1.y, is);
    is = dot4(w1.z, a1.z, is); is = dot4(w1.w, a1.w, is);
    const float prod = h2f(*(const uint16_t *)(s.B + bi * 16 + 2 * c)) * (float)is;
    // blk_sum += wd * isum over the 8 Q8_0 blocks in order
    const int base = lane_id() & ~7;
    float part = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; k++) part += shfl(prod, base + k);
    return s.xd[sb] * part;
}

template <int T>
OH_DEV float term(const oh_mvseg &s, int64_t bi, int sb, int c) {
    if (T == OH_Q4_K) return term_q4k(s, bi, sb, c);
    if (T == OH_Q6_K) return term_q6k(s, bi, sb, c);
    return term_q8_0(s, bi, sb, c);
}

OH_DEV void emit(const oh_mvseg &s, int row, float v) {
    if (s.mode == 1) s.y[row] = s.y[row] + v;
    else s.y[row] = v;
}

// One wave unit of a Q8_K-path segment.
template <int T>
OH_DEV void wave_unit(const oh_mvseg &s, int unit, int64_t row_base) {
    const int lane = lane_id(), g = lane >> 3, c = lane & 7, nb = s.nb;
    if (nb <= 8) {
        const int rp = 8 / nb;
        const int k = g / nb, sb = g - k * nb;
        const int row = unit * rp + k;
        const bool live = k < rp && row < s.rows;
        float t = 0.0f;
        if (live) t = term<T>(s, (row_base + row) * nb + sb, sb, c);
        float acc = 0.0f;
        for (int i = 0; i < nb; i++) acc += shfl(t, (k * nb + i) * 8);
        if (live && sb == 0 && c == 0) emit(s, row, acc);
    } else {
        const int row = unit;
        float acc = 0.0f;
        for (int p0 = 0; p0 < nb; p0 += 8) {
            const int sb = p0 + g;
            float t = 0.0f;
            if (sb < nb) t = term<T>(s, (row_base + row) * nb + sb, sb, c);
            const int cnt = nb - p0 < 8 ? nb - p0 : 8;
            for (int i = 0; i < cnt; i++) acc += shfl(t, i * 8);
        }
        if (lane == 0) emit(s, row, acc);
    }
}

// Fallback row: dequantise on the fly and accumulate w_i * x_i strictly in
// order (reference mv_run f32 path + ot_dot, src/ornith_rforward.c:119-133).
OH_DEV float row_seq(const oh_mvseg &s, int64_t r, const float *x) {
    const int in = s.in;
    float acc = 0.0f;
    if (s.type == OH_F32) {
        const float *w = (const float *)s.A + r * in;
        for (int i = 0; i < in; i++) acc += w[i] * x[i];
    } else if (s.type == OH_F16 || s.type == OH_BF16) {
        const uint16_t *w = (const uint16_t *)s.A + r * in;
        for (int i = 0; i < in; i++) {
            const float wf = s.type == OH_F16 ? h2f(w[i]) : u2f((uint32_t)w[i] << 16);
            acc += wf * x[i];
        }
    } else if (s.type == OH_IQ2_XXS) {
        const int nb = in / 256;
        for (int b = 0; b < nb; b++) {
            const int64_t bi = r * nb + b;
            const float d = h2f(*(const uint16_t *)(s.C + bi * 2));
            const uint32_t *q = (const uint32_t *)(s.A + bi * 64);
            for (int g32 = 0; g32 < 8; g32++) {
                const uint32_t w0 = q[2 * g32], w1 = q[2 * g32 + 1];
                const float db = d * (0.5f + (float)(w1 >> 28)) * 0.25f;
                for (int k = 0; k < 4; k++) {
                    const uint64_t gv = k_iq2_grid[(w0 >> (8 * k)) & 0xffu];
                    const uint32_t s7 = (w1 >> (7 * k)) & 127u;
                    const uint32_t sg = s7 | ((__popc(s7) & 1u) << 7);
                    const float *xx = x + b * 256 + g32 * 32 + k * 8;
                    for (int j = 0; j < 8; j++) {
                        const float wv = db * (float)((gv >> (8 * j)) & 0xffu) * ((sg >> j) & 1u ? -1.0f : 1.0f);
                        acc += wv * xx[j];
                    }
                }
            }
        }
    }
    return acc;
}

} // namespace

// Multi-segment matvec. Q8_K-path segments: block = 4 waves x 2 units.
// Fallback segments: block = 256 rows, one lane per row, x staged in LDS.
extern "C" __global__ void __launch_bounds__(256)
oh_k_matvec(oh_mvlaunch L) {
    extern __shared__ float xs[];   // fallback segments only: in floats
    int si = 0;
    while (si + 1 < L.n && (int)blockIdx.x >= L.s[si + 1].block0) si++;
    const oh_mvseg &s = L.s[si];
    const int blk = (int)blockIdx.x - s.block0;
    int64_t row_base = 0;
    if (s.eidx) row_base = (int64_t)s.eidx[s.eslot] * s.rows;
    if (oh_qdot_can((uint32_t)s.type, s.in) && s.xqs) {
        const int wave = (int)(threadIdx.x >> 6);
        for (int u = 0; u < kUnitsPerWave; u++) {
            const int unit = (blk * kWavesPerBlock + wave) * kUnitsPerWave + u;
            if (unit >= s.units) break;
            switch (s.type) {
            case OH_Q4_K: wave_unit<OH_Q4_K>(s, unit, row_base); break;
            case OH_Q6_K: wave_unit<OH_Q6_K>(s, unit, row_base); break;
            default: wave_unit<OH_Q8_0>(s, unit, row_base); break;
            }
        }
        return;
    }
    for (int i = (int)threadIdx.x; i < s.in; i += 256) xs[i] = s.xf[i];
    __syncthreads();
    const int row = blk * 256 + (int)threadIdx.x;
    if (row < s.rows) emit(s, row, row_seq(s, row_base + row, xs));
}

// ---- Q8_K quantisation (optionally fused with RMSNorm) ----------------------
// One block of 256 threads per vector of n <= 8192 elements (n % 256 == 0).
// norm_w != nullptr: x is first RMS-normalised (src/ornith_tensor.c:100-106):
// sum of squares in double (tree-ordered), inv = (float)(1/sqrt(ss/n+eps)),
// xn_i = x_i * inv * w_i. Then each 256-block is quantised exactly as
// qdot_quantize_row_q8_K (src/ornith_qdot.c:32-62).
OH_DEV void q8k_block_from_lds(const float *v, int qb, int8_t *qs, float *d, int16_t *bs) {
    const int lane = lane_id();
    const float *xb = v + qb * 256;
    // first element of largest magnitude (ties -> lowest index)
    float best = -1.0f; int bi = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int e = lane + 64 * k;
        const float a = fabsf(xb[e]);
        if (a > best) { best = a; bi = e; }
    }
    for (int m = 32; m >= 1; m >>= 1) {
        const float ob = shfl_xor(best, m);
        const int oi = shfl_xor(bi, m);
        if (ob > best || (ob == best && oi < bi)) { best = ob; bi = oi; }
    }
    int8_t *q = qs + (int64_t)qb * 256;
    int16_t *b = bs + (int64_t)qb * 16;
    if (best == 0.0f || !(best > 0.0f)) {
#pragma unroll
        for (int k = 0; k < 4; k++) q[lane + 64 * k] = 0;
        if (lane < 16) b[lane] = 0;
        if (lane == 0) d[qb] = 0.0f;
        return;
    }
    const float iscale = -127.0f / xb[bi];
    int sums[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int e = lane + 64 * k;
        float r = __builtin_rintf(iscale * xb[e]);
        int v = (int)r;
        v = v > 127 ? 127 : (v < -128 ? -128 : v);
        q[e] = (int8_t)v;
        sums[k] = v;
    }
#pragma unroll
    for (int k = 0; k < 4; k++) {
        int sv = sums[k];
        sv += shfl_xor(sv, 1); sv += shfl_xor(sv, 2); sv += shfl_xor(sv, 4); sv += shfl_xor(sv, 8);
        if ((lane & 15) == 0) b[4 * k + (lane >> 4)] = (int16_t)sv;
    }
    if (lane == 0) d[qb] = 1.0f / iscale;
}

extern "C" __global__ void __launch_bounds__(256)
oh_k_rmsnorm_q8k(const float *x, const float *norm_w, float eps, int n,
                 float *xn_out, int8_t *qs, float *d, int16_t *bs) {
    __shared__ float v[8192];
    __shared__ double red[4];
    const int tid = (int)threadIdx.x, wave = tid >> 6;
    for (int i = tid; i < n; i += 256) v[i] = x[i];
    __syncthreads();
    if (norm_w) {
        double ss = 0.0;
        for (int i = tid; i < n; i += 256) ss += (double)v[i] * v[i];
        ss = wave_sum_d(ss);
        if (lane_id() == 0) red[wave] = ss;
        __syncthreads();
        const double tot = (red[0] + red[1]) + (red[2] + red[3]);
        const float inv = (float)(1.0 / sqrt(tot / (double)n + (double)eps));
        __syncthreads();
        for (int i = tid; i < n; i += 256) v[i] = v[i] * inv * norm_w[i];
        __syncthreads();
    }
    if (xn_out) for (int i = tid; i < n; i += 256) xn_out[i] = v[i];
    for (int qb = wave; qb < n / 256; qb += 4) q8k_block_from_lds(v, qb, qs, d, bs);
}

// Batched Q8_K of `count` vectors of n elements at stride n (SwiGLU inputs):
// when g and u are given, v = silu(g) * u first (src/ornith_rforward.c:382).
extern "C" __global__ void __launch_bounds__(256)
oh_k_swiglu_q8k(const float *g, const float *u, int n, float *h_out,
                int8_t *qs, float *d, int16_t *bs) {
    __shared__ float v[8192];
    const int vec = (int)blockIdx.x, tid = (int)threadIdx.x, wave = tid >> 6;
    const float *gv = g + (int64_t)vec * n;
    const float *uv = u ? u + (int64_t)vec * n : nullptr;
    for (int i = tid; i < n; i += 256) v[i] = uv ? ref_silu(gv[i]) * uv[i] : gv[i];
    __syncthreads();
    if (h_out) for (int i = tid; i < n; i += 256) h_out[(int64_t)vec * n + i] = v[i];
    const int nqb = n / 256;
    for (int qb = wave; qb < nqb; qb += 4)
        q8k_block_from_lds(v, qb, qs + (int64_t)vec * n, d + (int64_t)vec * nqb, bs + (int64_t)vec * nqb * 16);
}

// ---- decode of plane-layout rows to f32 (src/ornith_quant.c decoders) -------
extern "C" __global__ void __launch_bounds__(256)
oh_k_dequant(const uint8_t *A, const uint8_t *B, const uint8_t *C, int type, int in,
             int64_t row0, int64_t nrows, float *out) {
    const int64_t n = nrows * in;
    for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < n; e += (int64_t)gridDim.x * 256) {
        const int64_t r = row0 + e / in;
        const int i = (int)(e % in);
        float y = 0.0f;
        if (type == OH_F32) y = ((const float *)A)[r * in + i];
        else if (type == OH_F16) y = h2f(((const uint16_t *)A)[r * in + i]);
        else if (type == OH_BF16) y = u2f((uint32_t)((const uint16_t *)A)[r * in + i] << 16);
        else {
            const int nb = in / 256, b = i / 256, k = i % 256;
            const int64_t bi = r * nb + b;
            if (type == OH_Q4_K) {
                const uint4 hdr = *(const uint4 *)(B + bi * 16);
                const int j = k / 32, l = k % 32;
                const uint8_t q = A[bi * 128 + 32 * (j / 2) + l];
                int sc, mn;
                q4k_sm(hdr, j, sc, mn);
                const float dd = h2f((uint16_t)(hdr.x & 0xffffu)), dmin = h2f((uint16_t)(hdr.x >> 16));
                const float d1 = dd * sc, m1 = dmin * mn;
                y = d1 * (float)((j & 1) ? (q >> 4) : (q & 15)) - m1;
            } else if (type == OH_Q6_K) {
                const uint8_t *a = A + bi * 192;
                const int hh = k / 128, kk = k % 128, qd = kk / 32, l = kk % 32;
                const uint8_t ql = a[64 * hh + l + 32 * (qd & 1)];
                const uint8_t qh = a[128 + 32 * hh + l];
                const int lo = (qd < 2) ? (ql & 15) : (ql >> 4);
                const int q = (lo | (((qh >> (2 * qd)) & 3) << 4)) - 32;
                const int8_t sc = (int8_t)B[bi * 16 + 8 * hh + l / 16 + 2 * qd];
                const float dd = h2f(*(const uint16_t *)(C + bi * 2));
                y = dd * (float)sc * (float)q;
            } else if (type == OH_Q8_0) {
                const int sbk = k / 32;
                const int8_t q = (int8_t)A[bi * 256 + k];
                y = (float)q * h2f(*(const uint16_t *)(B + bi * 16 + 2 * sbk));
            } else if (type == OH_IQ2_XXS) {
                const float dd = h2f(*(const uint16_t *)(C + bi * 2));
                const uint32_t *q = (const uint32_t *)(A + bi * 64);
                const int g32 = k / 32, kk = (k % 32) / 8, j = k % 8;
                const uint32_t w0 = q[2 * g32], w1 = q[2 * g32 + 1];
                const float db = dd * (0.5f + (float)(w1 >> 28)) * 0.25f;
                const uint64_t gv = k_iq2_grid[(w0 >> (8 * kk)) & 0xffu];
                const uint32_t s7 = (w1 >> (7 * kk)) & 127u;
                const uint32_t sg = s7 | ((__popc(s7) & 1u) << 7);
                y = db * (float)((gv >> (8 * j)) & 0xffu) * ((sg >> j) & 1u ? -1.0f : 1.0f);
            }
        }
        out[e] = y;
    }
}
