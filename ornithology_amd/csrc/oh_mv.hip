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
// 8/16-byte vector loads from the plane layout (contiguous across the group).
// A unit is one row (nb > 8 super-blocks per row, taken in passes of 8) or
// 8/nb rows (nb <= 8); a step is one unit-pass. Each wave owns a contiguous
// run of units and streams its steps in batches of OH_MV_R with the next
// batch's weight loads in flight while the current batch is reduced. The
// activation (Q8_K codes, bsums, scales) sits in LDS; the block forms it in a
// prologue (copy, RMSNorm + Q8_K, or SwiGLU + Q8_K) while the first batch of
// weights is being fetched.
#include "oh_common.h"
#include "oh_types.h"
#include "../../include/ornith_iq2xxs_grid.h"

static __constant__ uint64_t k_iq2_grid[256] = { ORNITH_IQ2XXS_GRID_VALUES };

namespace {

OH_DEV uint32_t wsel(const uint4 &v, int k) {   // 32-bit word k of a uint4
    return k == 0 ? v.x : (k == 1 ? v.y : (k == 2 ? v.z : v.w));
}
OH_DEV uint32_t bsel(const uint4 &v, int k) {   // byte k of a uint4
    return (wsel(v, k >> 2) >> (8 * (k & 3))) & 0xffu;
}

// Block barrier that orders LDS only: it does not wait for the block's
// outstanding global loads (prefetched weights).
OH_DEV void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
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

// Smallest e = lane + 64k with a[k] == best over the wave (a[k]: lane's
// element lane + 64k), from one ballot per quarter; 256 when none matches.
// Wave-uniform.
OH_DEV int first_hit(const float a[4], float best) {
    const uint64_t m0 = __ballot(a[0] == best), m1 = __ballot(a[1] == best);
    const uint64_t m2 = __ballot(a[2] == best), m3 = __ballot(a[3] == best);
    return m0 ? (int)__builtin_ctzll(m0) : m1 ? 64 + (int)__builtin_ctzll(m1)
         : m2 ? 128 + (int)__builtin_ctzll(m2) : m3 ? 192 + (int)__builtin_ctzll(m3) : 256;
}

// ---- Q8_K quantisation of one 256-element block held in LDS ------------------
// One wave; exactly qdot_quantize_row_q8_K (src/ornith_qdot.c:32-62): the first
// element of largest magnitude sets iscale = -127/x, codes = rint(iscale*x)
// clamped, bsums per 16, d = 1/iscale. G: qs/d/bs are global memory read by
// other workgroups (device-scope stores); otherwise LDS.
template <bool G = false>
OH_DEV void q8k_block_from_lds(const float *v, int qb, int8_t *qs, float *d, int16_t *bs,
                               int qstride = 256, int8_t *bp = nullptr) {
    const int lane = lane_id();
    const float *xb = v + qb * 256;
    float a[4];
#pragma unroll
    for (int k = 0; k < 4; k++) a[k] = fabsf(xb[lane + 64 * k]);
    // largest magnitude (NaN never wins), then its first index
    const float best = wave_max_fast(fmaxf(fmaxf(a[0], a[1]), fmaxf(a[2], a[3])));
    const int bi = first_hit(a, best);
    int8_t *q = qs + (int64_t)qb * qstride;
    int16_t *b = bs + (int64_t)qb * 16;
    auto put8 = [&](int8_t *p, int8_t x) { if (G) stc(p, x); else *p = x; };
    auto put16 = [&](int16_t *p, int16_t x) { if (G) stc(p, x); else *p = x; };
    auto putf = [&](float *p, float x) { if (G) stc(p, x); else *p = x; };
    if (best == 0.0f || !(best > 0.0f)) {
#pragma unroll
        for (int k = 0; k < 4; k++) put8(q + lane + 64 * k, (int8_t)0);
        if (lane < 16) put16(b + lane, (int16_t)0);
        if (bp && lane < 16) bp[(int64_t)qb * 16 + lane] = 0;
        if (lane == 0) putf(d + qb, 0.0f);
        return;
    }
    const float iscale = -127.0f / xb[bi];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int e = lane + 64 * k;
        float r = __builtin_rintf(iscale * xb[e]);
        int c = (int)r;
        c = c > 127 ? 127 : (c < -128 ? -128 : c);
        put8(q + e, (int8_t)c);
        const int sv = row16_sum_i(c);                 // codes 64k + 16g .. +15
        if ((lane & 15) == 0) put16(b + 4 * k + (lane >> 4), (int16_t)sv);
        if (bp) {
            // pair sums bsums_2j + bsums_2j+1 (j = 2k + lane/32) as 64 * bh + bl
            const int ps = sv + shfl(sv, lane ^ 16);
            if ((lane & 31) == 0) {
                const int j = 2 * k + (lane >> 5);
                bp[(int64_t)qb * 16 + j] = (int8_t)(ps & 63);
                bp[(int64_t)qb * 16 + 8 + j] = (int8_t)(ps >> 6);
            }
        }
    }
    if (lane == 0) putf(d + qb, 1.0f / iscale);
}

// Q8_K of the blocks qb0, qb0 + qstep, ... (< nb, at most N of them) of v by
// one wave, the N blocks' reductions interleaved. Same result per block as
// q8k_block_from_lds.
template <int N>
OH_DEV void q8k_blocks(const float *v, int qb0, int qstep, int nb, int8_t *qs, float *d, int16_t *bs,
                       int qstride = 256) {
    const int lane = lane_id();
    float a[N][4], best[N];
    int bi[N];
#pragma unroll
    for (int n = 0; n < N; n++) {
        const int qb = qb0 + n * qstep < nb ? qb0 + n * qstep : nb - 1;
#pragma unroll
        for (int k = 0; k < 4; k++) a[n][k] = fabsf(v[qb * 256 + lane + 64 * k]);
        best[n] = fmaxf(fmaxf(a[n][0], a[n][1]), fmaxf(a[n][2], a[n][3]));
    }
#pragma unroll
    for (int n = 0; n < N; n++) best[n] = wave_max_fast(best[n]);
    // first index of the largest magnitude: the lowest lane holding it in
    // the first quarter (elements lane + 64k) that holds it at all
#pragma unroll
    for (int n = 0; n < N; n++) bi[n] = first_hit(a[n], best[n]);
#pragma unroll
    for (int n = 0; n < N; n++) {
        const int qb = qb0 + n * qstep;
        if (qb >= nb) break;
        const float *xb = v + qb * 256;
        int8_t *q = qs + (int64_t)qb * qstride;
        int16_t *b = bs + (int64_t)qb * 16;
        if (best[n] == 0.0f || !(best[n] > 0.0f)) {
#pragma unroll
            for (int k = 0; k < 4; k++) q[lane + 64 * k] = 0;
            if (lane < 16) b[lane] = 0;
            if (lane == 0) d[qb] = 0.0f;
            continue;
        }
        const float iscale = -127.0f / xb[bi[n]];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int e = lane + 64 * k;
            float r = __builtin_rintf(iscale * xb[e]);
            int c = (int)r;
            c = c > 127 ? 127 : (c < -128 ? -128 : c);
            q[e] = (int8_t)c;
            const int sv = row16_sum_i(c);
            if ((lane & 15) == 0) b[4 * k + (lane >> 4)] = (int16_t)sv;
        }
        if (lane == 0) d[qb] = 1.0f / iscale;
    }
}

// Q8_K of all nb blocks of v by the 4 waves of a block
OH_DEV void q8k_all(const float *v, int nb, int8_t *qs, float *d, int16_t *bs, int qstride) {
    const int wave = (tid_x() >> 6);
    for (int q0 = wave; q0 < nb; q0 += 16) q8k_blocks<4>(v, q0, 4, nb, qs, d, bs, qstride);
}

// ---- one super-block per lane ----------------------------------------------------
// A lane owns one 256-element super-block of a weight row: it loads the
// block's A-plane pieces (coalesced across the wave by the tile interleave)
// and its B/C bytes, and reduces them against the activation super-block in
// LDS. Integer sums are exact in any order; the float term keeps the
// reference's operations (src/ornith_qdot.c:64-216).
struct WP { const uint8_t *A, *B, *C; };
template <int T> struct SB;
template <> struct SB<OH_Q4_K> { uint4 q[8]; uint4 h; };              // qs, d/dmin/scales
template <> struct SB<OH_Q6_K> { uint4 q[12]; uint4 sc; uint32_t d; }; // ql+qh, scales, d
template <> struct SB<OH_Q8_0> { uint4 q[16]; uint4 d; };             // 8 x qs[32], 8 x d

// piece k of super-block bi is at [k * 64] of the returned pointer
OH_DEV const uint4 *a_tile(const uint8_t *A, int pb, int64_t bi) {
    return (const uint4 *)(A + (bi >> 6) * (int64_t)(64 * pb)) + (bi & 63);
}
OH_DEV void sb_load(SB<OH_Q4_K> &r, const WP &w, int64_t bi) {
    const uint4 *a = a_tile(w.A, 128, bi);
#pragma unroll
    for (int k = 0; k < 8; k++) r.q[k] = ldg(a + k * 64);
    r.h = ldg((const uint4 *)(w.B + bi * 16));
}
OH_DEV void sb_load(SB<OH_Q6_K> &r, const WP &w, int64_t bi) {
    const uint4 *a = a_tile(w.A, 192, bi);
#pragma unroll
    for (int k = 0; k < 12; k++) r.q[k] = ldg(a + k * 64);
    r.sc = ldg((const uint4 *)(w.B + bi * 16));
    r.d = ldg((const uint16_t *)(w.C + bi * 2));
}
OH_DEV void sb_load(SB<OH_Q8_0> &r, const WP &w, int64_t bi) {
    const uint4 *a = a_tile(w.A, 256, bi);
#pragma unroll
    for (int k = 0; k < 16; k++) r.q[k] = ldg(a + k * 64);
    r.d = ldg((const uint4 *)(w.B + bi * 16));
}

OH_DEV uint32_t pword(const uint4 *q, int w) { return wsel(q[w >> 2], w & 3); }
OH_DEV int aword(const int4 *a, int w) {
    const int4 v = a[w >> 2];
    return (w & 3) == 0 ? v.x : ((w & 3) == 1 ? v.y : ((w & 3) == 2 ? v.z : v.w));
}

// Q4_K: isum = sum_j sc_j * dot_j, mins = sum_j mn_j * (bsum_2j + bsum_2j+1);
// term = yd*d * isum + (-yd*dmin) * mins
OH_DEV float sb_term(const SB<OH_Q4_K> &r, const int8_t *aq, const int16_t *bs, float yd) {
    const uint32_t y = r.h.y, z = r.h.z, w = r.h.w;
    // 6-bit scales / mins of sub-blocks 0-3 and 4-7, one per byte
    const uint32_t scl = y & 0x3f3f3f3fu, sch = (w & 0x0f0f0f0fu) | ((y >> 2) & 0x30303030u);
    const uint32_t mnl = z & 0x3f3f3f3fu, mnh = ((w >> 4) & 0x0f0f0f0fu) | ((z >> 2) & 0x30303030u);
    const int4 *a4 = (const int4 *)aq;
    const uint32_t M = 0x0f0f0f0fu;
    int isum = 0;
#pragma unroll
    for (int p = 0; p < 4; p++) {
        int dl = 0, dh = 0;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint32_t qv = pword(r.q, 8 * p + k);
            dl = dot4((int)(qv & M), aword(a4, 16 * p + k), dl);
            dh = dot4((int)((qv >> 4) & M), aword(a4, 16 * p + 8 + k), dh);
        }
        const uint32_t sw = p < 2 ? scl : sch;
        const int s0 = (int)((sw >> (8 * ((2 * p) & 3))) & 0xffu);
        const int s1 = (int)((sw >> (8 * ((2 * p + 1) & 3))) & 0xffu);
        isum += s0 * dl + s1 * dh;
    }
    int mins = 0;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int mn = (int)(((j < 4 ? mnl : mnh) >> (8 * (j & 3))) & 0xffu);
        mins += mn * ((int)bs[2 * j] + (int)bs[2 * j + 1]);
    }
    const float d = yd * h2f((uint16_t)(r.h.x & 0xffffu));
    const float dm = -yd * h2f((uint16_t)(r.h.x >> 16));
    return d * (float)isum + dm * (float)mins;
}

// Q6_K: sum over 16-element groups g of sc_g * (sum q*a - 32 * bsum_g);
// term = (yd * d) * isum
OH_DEV float sb_term(const SB<OH_Q6_K> &r, const int8_t *aq, const int16_t *bs, float yd) {
    const int4 *a4 = (const int4 *)aq;
    int isum = 0;
#pragma unroll
    for (int hh = 0; hh < 2; hh++) {
        int D[8] = {0, 0, 0, 0, 0, 0, 0, 0};       // group 8hh + t
#pragma unroll
        for (int w = 0; w < 8; w++) {
            const uint32_t la = pword(r.q, 16 * hh + w);        // ql[64hh + 4w ..]
            const uint32_t lb = pword(r.q, 16 * hh + 8 + w);    // ql[64hh + 32 + 4w ..]
            const uint32_t hb = pword(r.q, 32 + 8 * hh + w);    // qh[32hh + 4w ..]
            const int q1 = (int)((la & 0x0f0f0f0fu) | ((hb & 0x03030303u) << 4));
            const int q2 = (int)((lb & 0x0f0f0f0fu) | (((hb >> 2) & 0x03030303u) << 4));
            const int q3 = (int)(((la >> 4) & 0x0f0f0f0fu) | (((hb >> 4) & 0x03030303u) << 4));
            const int q4 = (int)(((lb >> 4) & 0x0f0f0f0fu) | (((hb >> 6) & 0x03030303u) << 4));
            const int e = 32 * hh + w;                           // activation word of element 128hh + 4w
            const int is = w >> 2;
            D[0 + is] = dot4(q1, aword(a4, e), D[0 + is]);
            D[2 + is] = dot4(q2, aword(a4, e + 8), D[2 + is]);
            D[4 + is] = dot4(q3, aword(a4, e + 16), D[4 + is]);
            D[6 + is] = dot4(q4, aword(a4, e + 24), D[6 + is]);
        }
#pragma unroll
        for (int t = 0; t < 8; t++) {
            const int g = 8 * hh + t;
            const int sc = (int)(int8_t)bsel(r.sc, g);
            isum += sc * (D[t] - 32 * (int)bs[g]);
        }
    }
    const float d = yd * h2f((uint16_t)r.d);
    return d * (float)isum;
}

// Q8_0: part = sum_b d_b * isum_b (in order); term = yd * part
OH_DEV float sb_term(const SB<OH_Q8_0> &r, const int8_t *aq, const int16_t *, float yd) {
    const int4 *a4 = (const int4 *)aq;
    float part = 0.0f;
#pragma unroll
    for (int b = 0; b < 8; b++) {
        int is = 0;
#pragma unroll
        for (int k = 0; k < 8; k++) is = dot4((int)pword(r.q, 8 * b + k), aword(a4, 8 * b + k), is);
        const uint16_t dh = (uint16_t)(wsel(r.d, b >> 1) >> (16 * (b & 1)));
        part += h2f(dh) * (float)is;
    }
    return yd * part;
}

// LDS tables of the IQ2_XXS tolerance path: the codebook and, per 7-bit
// sign field, its byte mask (0xff where the weight is negative; bit 7 the
// field's parity, the decoder's sign rule, src/ornith_quant.c:660-680)
__shared__ uint64_t s_iq2_grid[256];
__shared__ uint64_t s_iq2_sign[128];
OH_DEV void iq2_tables_load() {
    const int t = tid_x();
    for (int i = t; i < 256; i += (int)blockDim.x) s_iq2_grid[i] = k_iq2_grid[i];
    for (int i = t; i < 128; i += (int)blockDim.x) {
        const uint32_t sg = (uint32_t)i | ((uint32_t)(__popc(i) & 1) << 7);
        uint64_t m = 0;
#pragma unroll
        for (int j = 0; j < 8; j++)
            if ((sg >> j) & 1u) m |= 0xffull << (8 * j);
        s_iq2_sign[i] = m;
    }
}

// outputs are read by later phases of the step kernel (device-scope accesses)
// Output stores: device-scope (G) where a later phase of the same launch
// reads them (the persistent step kernels), plain stores in a stand-alone
// launch, whose end makes them visible to the next one.
template <bool G = true>
OH_DEV void put(float *p, float v) {
    if (G) stc(p, v);
    else stg(p, v);
}
template <bool G = true>
OH_DEV void emit(float *y, int mode, int row, float v) {
    if (mode == 1) put<G>(y + row, (G ? ldc(y + row) : ldg(y + row)) + v);
    else put<G>(y + row, v);
}

// Fallback row of an F32 / F16 / BF16 tensor: convert on the fly and
// accumulate w_i * x_i strictly in order (reference mv_run f32 path + ot_dot,
// src/ornith_rforward.c:119-133).
OH_DEV float row_seq(const oh_mvseg &s, int64_t r, const float *x) {
    const int in = s.in;
    float acc = 0.0f;
    if (s.type == OH_F32) {
        const float *w = (const float *)s.A + r * in;
        for (int i = 0; i < in; i++) acc += ldg(w + i) * x[i];
    } else if (s.type == OH_F16 || s.type == OH_BF16) {
        const uint16_t *w = (const uint16_t *)s.A + r * in;
        for (int i = 0; i < in; i++) {
            const uint16_t wr = ldg(w + i);
            const float wf = s.type == OH_F16 ? h2f(wr) : u2f((uint32_t)wr << 16);
            acc += wf * x[i];
        }
    }
    return acc;
}

// ---- MoE routing of one wave (src/ornith_moe.c:8-30) ----------------------------
// Top-k by repeated argmax (largest logit, lowest index on ties), then softmax
// over the selected logits in selection order; the optional shared-expert gate
// is sigmoid of its logit. ne <= 1024, k <= 64.
OH_DEV void route_wave(const float *logits, int ne, int k, const float *shgate_logit,
                       int32_t *idx, float *w, float *shgate) {
    const int lane = lane_id();
    float v[16];
#pragma unroll
    for (int j = 0; j < 16; j++) v[j] = lane + 64 * j < ne ? logits[lane + 64 * j] : -INFINITY;
    uint32_t taken = 0;
    float mine = 0.0f;                     // lane s keeps the s-th selected logit
    int sel = 0;
    for (int s = 0; s < k; s++) {
        float bv = -INFINITY; int bi = 0x7fffffff;
#pragma unroll
        for (int j = 0; j < 16; j++) {
            const int e = lane + 64 * j;
            if (e < ne && !(taken >> j & 1u) && v[j] > bv) { bv = v[j]; bi = e; }
        }
        for (int m = 32; m >= 1; m >>= 1) {
            const float ov = shfl_xor(bv, m); const int oi = shfl_xor(bi, m);
            if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
        }
        // (no candidate left, bi the sentinel: nothing to mark)
        if (bi != 0x7fffffff && (bi & 63) == lane) taken |= 1u << (bi >> 6);
        if (lane == s) { mine = bv; sel = bi; }
    }
    // NaN/-inf logits can leave no candidate: never hand an out-of-range
    // expert index to the gathered matvec
    if (sel < 0 || sel >= ne) sel = 0;
    if (lane < k) idx[lane] = sel;
    float mx = shfl(mine, 0);
    for (int s = 1; s < k; s++) { const float x = shfl(mine, s); if (x > mx) mx = x; }
    const float e = ref_expf(mine - mx);
    float sum = 0.0f;
    for (int s = 0; s < k; s++) sum += shfl(e, s);
    if (lane < k) w[lane] = e / sum;
    if (lane == 0 && shgate_logit) *shgate = ref_sigmoid(*shgate_logit);
}

// ---- LDS layout of a matvec block ---------------------------------------------
// [qs: nb x 272 B (256 codes + 16 B bank spread)][bsums: nb*16 int16][d: nb f32]
// [pad to 16][v: in f32 (prologue input / fallback activation)]
constexpr int kAS = 272;
OH_HD inline int mv_lds_bs_off(int nb) { return nb * kAS; }
OH_HD inline int mv_lds_d_off(int nb) { return nb * kAS + nb * 32; }
OH_HD inline int mv_lds_v_off(int nb) { return (nb * kAS + nb * 36 + 15) & ~15; }

// IQ2_XXS rows (src/ornith_quant.c:660-680 decode, then ot_dot's strictly
// sequential f32 accumulation, src/ornith_rforward.c:119-133). A row's sum is
// one chain of adds in element order; its terms are not: y_i * x_i with
// y = (db * g) * (+-1) is +-((db * g) * x) exactly.
//
// iq2_rows_lane: one lane per row walks its row in element order, forming
// each term and adding it at once (256 rows per block); each row's next
// super-block (64 code bytes and d) is in flight while the current one is
// reduced. Used when the launch has rows enough to fill the GPU this way.
//
// iq2_rows (few rows, wide inputs: the decode step's experts) takes 64 rows:
// waves 1..3 form the terms of one 32-element sub-block each per chunk (lane =
// row) into a double-buffered LDS tile [64 rows][96 + 4], and wave 0 adds a
// chunk's terms in order while the next chunk is formed; the chunk barrier
// hands a tile over. The f32 activation and the 256-entry grid sit in LDS
// (every lane reads the same activation word); each producer's next
// sub-block (two code words and d) is in flight while it forms the current.
constexpr int kIq2P = 3, kIq2E = 32 * kIq2P, kIq2S = kIq2E + 4;   // producers, terms per chunk, tile row stride
constexpr int kIq2D = 6;                                            // chunks of codes in flight per producer
static_assert(kIq2S == 100, "the host's LDS plan takes term-tile rows of 100 floats");
OH_HD inline int mv_lds_iq2_off(int nb, int in) { return (mv_lds_v_off(nb) + in * 4 + 15) & ~15; }
OH_HD inline int mv_lds_iq2t_off(int nb, int in) { return mv_lds_iq2_off(nb, in) + 2048; }
// the split form's scales d: [OH_IQ2_ROWS][nb] halves after the two term tiles
OH_HD inline int mv_lds_iq2d_off(int nb, int in) { return mv_lds_iq2t_off(nb, in) + 2 * OH_IQ2_ROWS * kIq2S * 4; }

// The 128 sign patterns of IQ2_XXS as byte masks (the eighth sign is the
// parity of the seven stored ones): entry s7 = {m_lo, m_hi, m_lo & 0x01..,
// m_hi & 0x01..}, m byte j = 0xff where sign j is negative, so that
// (g ^ m) + (m & 0x01..) negates exactly those bytes of a grid entry g.
OH_DEV void iq2_sign_table(uint4 *stab) {
    const int tid = tid_x();
    if (tid < 128) {
        const uint32_t sg = (uint32_t)tid | ((__popc((uint32_t)tid) & 1u) << 7);
        uint32_t m0 = 0, m1 = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            m0 |= ((sg >> j) & 1u) * (0xffu << (8 * j));
            m1 |= ((sg >> (j + 4)) & 1u) * (0xffu << (8 * j));
        }
        stab[tid] = make_uint4(m0, m1, m0 & 0x01010101u, m1 & 0x01010101u);
    }
}
// Eight terms of one codebook entry: (db * +-g_j) * x_j, the grid bytes of
// entry gv carrying their signs (sm: the entry's sign masks); (db * -g) * x
// is -((db * g) * x) exactly.
OH_DEV void iq2_terms8(uint64_t gv, const uint4 sm, float db, const float4 x0, const float4 x1, float (&ts)[8]) {
    const uint32_t gs[2] = {((uint32_t)gv ^ sm.x) + sm.z, ((uint32_t)(gv >> 32) ^ sm.y) + sm.w};
    const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
    for (int j = 0; j < 8; j++) ts[j] = db * (float)(int8_t)(gs[j / 4] >> (8 * (j % 4))) * xs[j];
}

OH_DEV void iq2_rows_lane(const oh_mvseg &s, int slot, int blk, int expert, uint8_t *smem) {
    const int in = s.in, nb = in / 256, tid = tid_x();
    const float *v = (const float *)(smem + mv_lds_v_off(nb));
    uint64_t *grid = (uint64_t *)(smem + mv_lds_iq2_off(nb, in));
    uint4 *stab = (uint4 *)(smem + mv_lds_iq2t_off(nb, in));      // the sign masks, after the grid
    const int row = blk * OH_IQ2_ROWS_LANE + tid;
    const int64_t bi0 = ((int64_t)expert * s.rows + (row < s.rows ? row : s.rows - 1)) * nb;
    // two super-blocks' codes and d, used in turn: a slot is refilled only
    // after its super-block was reduced, so the load lands in the slot's own
    // registers (a copy between slots would wait for the load in flight)
    uint4 qa[4], qb[4];
    uint32_t da, dbb;
    auto fetch = [&](uint4 (&q)[4], uint32_t &d, int b) {
        const int bc = b < nb ? b : nb - 1;
        const uint4 *src = (const uint4 *)(s.A + (bi0 + bc) * 64);
#pragma unroll
        for (int k = 0; k < 4; k++) q[k] = ldg(src + k);
        d = ldg((const uint16_t *)(s.C + (bi0 + bc) * 2));
    };
    const uint64_t g = k_iq2_grid[tid];
    fetch(qa, da, 0);
    grid[tid] = g;
    iq2_sign_table(stab);
    lds_barrier();
    float acc = 0.0f;
    // super-block b: each term added at once, in element order
    auto reduce = [&](int b, const uint4 (&q)[4], uint32_t d) {
        const float dd = h2f((uint16_t)d);
        const float4 *xb = (const float4 *)(v + b * 256);
#pragma unroll
        for (int g32 = 0; g32 < 8; g32++) {
            const uint32_t w0 = wsel(q[g32 >> 1], 2 * (g32 & 1)), w1 = wsel(q[g32 >> 1], 2 * (g32 & 1) + 1);
            const float db = dd * (0.5f + (float)(w1 >> 28)) * 0.25f;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                float ts[8];
                iq2_terms8(grid[(w0 >> (8 * k)) & 0xffu], stab[(w1 >> (7 * k)) & 127u], db,
                           xb[g32 * 8 + 2 * k], xb[g32 * 8 + 2 * k + 1], ts);
#pragma unroll
                for (int j = 0; j < 8; j++) acc += ts[j];
            }
        }
    };
    int b = 0;
    for (; b + 2 <= nb; b += 2) {
        fetch(qb, dbb, b + 1);
        reduce(b, qa, da);
        fetch(qa, da, b + 2);
        reduce(b + 1, qb, dbb);
    }
    if (b < nb) reduce(b, qa, da);
    if (row < s.rows) emit(s.y + (size_t)slot * s.ystride, s.mode, row, acc);
}

OH_DEV void iq2_rows(const oh_mvseg &s, int slot, int blk, int expert, uint8_t *smem) {
    const int in = s.in, nb = in / 256, nsb = in / 32, tid = tid_x(), lane = tid & 63, wave = tid >> 6;
    const float *v = (const float *)(smem + mv_lds_v_off(nb));
    uint64_t *grid = (uint64_t *)(smem + mv_lds_iq2_off(nb, in));
    float *tile = (float *)(smem + mv_lds_iq2t_off(nb, in));       // [2][OH_IQ2_ROWS][kIq2S]
    const int row = blk * OH_IQ2_ROWS + lane;
    const int64_t bi0 = ((int64_t)expert * s.rows + (row < s.rows ? row : s.rows - 1)) * nb;
    const int nch = (nsb + kIq2P - 1) / kIq2P;
    // the super-block scales d of the block's rows, [OH_IQ2_ROWS][nb] halves
    // in LDS (64 * nb * 2 contiguous bytes of the C plane; nb is even)
    uint32_t *dl = (uint32_t *)(smem + mv_lds_iq2d_off(nb, in));
    const int nh = nb / 2;
    uint32_t dv[OH_IQ2_ROWS * 32 / 2 / 256];        // up to nb = 32
    const uint32_t *dsrc = (const uint32_t *)s.C;
#pragma unroll
    for (int u = 0; u < OH_IQ2_ROWS * 32 / 2 / 256; u++) {
        const int i = tid + 256 * u, r = i / nh, rr = blk * OH_IQ2_ROWS + r;
        if (i < OH_IQ2_ROWS * nh)
            dv[u] = ldg(dsrc + ((int64_t)expert * s.rows + (rr < s.rows ? rr : s.rows - 1)) * nh + (i - r * nh));
    }
    // a producer's code words for its next kIq2D chunks (a chunk's terms
    // take well under one memory round trip). Every wave issues the same
    // loads (the adding wave those of producer 0, the same lines) so that
    // each wave's wait for a slot leaves the later slots in flight.
    uint2 wq[kIq2D];
    const int pw = wave > 0 ? wave - 1 : 0;          // producer index: sub-block pw of each chunk
    // sub-block sb of the row: byte (sb / 8) * 64 + (sb % 8) * 8 = 8 sb of
    // the row's 64-byte super-blocks, so one 8-byte word per sub-block
    const uint2 *arow = (const uint2 *)(s.A + bi0 * 64);
    auto fetch = [&](int c, uint2 &w) {
        const int sb = c * kIq2P + pw;
        w = ldg(arow + (sb < nsb ? sb : nsb - 1));
    };
    const uint64_t g = k_iq2_grid[tid];            // requested before the codes: its wait leaves them in flight
    // the sign masks in LDS below the f32 activation (the Q8_K planes'
    // place, which this form does not use: at least 2464 bytes for inputs of
    // 2048 and more)
    uint4 *stab = (uint4 *)smem;
    iq2_sign_table(stab);
#pragma unroll
    for (int i = 0; i + 1 < kIq2D; i++) fetch(i < nch ? i : nch - 1, wq[i]);
    grid[tid] = g;
#pragma unroll
    for (int u = 0; u < OH_IQ2_ROWS * 32 / 2 / 256; u++)
        if (tid + 256 * u < OH_IQ2_ROWS * nh) dl[tid + 256 * u] = dv[u];
    lds_barrier();
    const uint16_t *dh = (const uint16_t *)dl + lane * nb;
    float acc = 0.0f;
    // chunk c: every wave refills the slot that chunk c - 1 emptied (wn)
    // with chunk c + kIq2D - 1 and takes its own slot's words (wr); the
    // producers form chunk c from them, the adding wave adds chunk c - 1. A
    // slot is refilled only after its words were taken, so the refill lands
    // in the slot's own registers (no copy, which would wait for every load
    // in flight).
    auto chunk = [&](auto inner, int c, uint2 &wr, uint2 &wn) {
        fetch(c + kIq2D - 1 < nch ? c + kIq2D - 1 : nch - 1, wn);
        const uint32_t w0 = wr.x, w1 = wr.y;
        if (wave > 0 && (decltype(inner)::value || c < nch)) {
            // terms of sub-block sb into tile c & 1, columns (wave - 1) * 32 ..
            const int sb = c * kIq2P + wave - 1;
            if (sb < nsb) {
                const float dd = h2f(dh[sb / 8]);
                const float db = dd * (0.5f + (float)(w1 >> 28)) * 0.25f;
                const float4 *xb = (const float4 *)(v + sb * 32);
                float *dst = tile + ((c & 1) * OH_IQ2_ROWS + lane) * kIq2S + (wave - 1) * 32;
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    float ts[8];
                    iq2_terms8(grid[(w0 >> (8 * k)) & 0xffu], stab[(w1 >> (7 * k)) & 127u], db, xb[2 * k],
                               xb[2 * k + 1], ts);
                    *(float4 *)(dst + 8 * k) = make_float4(ts[0], ts[1], ts[2], ts[3]);
                    *(float4 *)(dst + 8 * k + 4) = make_float4(ts[4], ts[5], ts[6], ts[7]);
                }
            }
        }
        if (wave == 0 && c > 0) {
            // the previous chunk's terms of this lane's row, in element order
            const int e0 = (c - 1) * kIq2E, ne = in - e0 < kIq2E ? in - e0 : kIq2E;
            const float *src = tile + (((c - 1) & 1) * OH_IQ2_ROWS + lane) * kIq2S;
            if (ne == kIq2E) {
                // every read of the chunk issued before the first add: the
                // adds then wait on no LDS round trip
                float4 q[kIq2E / 4];
#pragma unroll
                for (int i = 0; i < kIq2E / 4; i++) q[i] = *(const float4 *)(src + 4 * i);
#pragma unroll
                for (int i = 0; i < kIq2E / 4; i++) {
                    acc += q[i].x;
                    acc += q[i].y;
                    acc += q[i].z;
                    acc += q[i].w;
                }
            } else {
                for (int e = 0; e < ne; e += 4) {
                    const float4 q = *(const float4 *)(src + e);
                    acc += q.x;
                    acc += q.y;
                    acc += q.z;
                    acc += q.w;
                }
            }
        }
        lds_barrier();                              // the producers' next codes stay in flight
    };
    // the ring indexed statically, and whole groups of kIq2D chunks before
    // c = nch without any test between them (a register shift of the slots,
    // or a chunk that may be skipped, makes each use wait for every load in
    // flight)
    int c0 = 0;
    for (; c0 + kIq2D <= nch; c0 += kIq2D) {
#pragma unroll
        for (int r = 0; r < kIq2D; r++) {
            chunk(std::true_type(), c0 + r, wq[r], wq[(r + kIq2D - 1) % kIq2D]);
        }
    }
#pragma unroll
    for (int r = 0; r < kIq2D; r++) {
        if (c0 + r <= nch) chunk(std::false_type(), c0 + r, wq[r], wq[(r + kIq2D - 1) % kIq2D]);
    }
    if (wave == 0 && row < s.rows) emit(s.y + (size_t)slot * s.ystride, s.mode, row, acc);
}

OH_DEV float4 f4_silu_mul(const float4 g, const float4 u) {
    return make_float4(ref_silu(g.x) * u.x, ref_silu(g.y) * u.y, ref_silu(g.z) * u.z, ref_silu(g.w) * u.w);
}

// Block prologue for inputs wider than the register prologue (and the
// fallback rows): form the slot's activation in LDS. q8: Q8_K planes are
// needed (integer path); otherwise only the f32 vector v. The inputs are read
// in passes of up to 4 float4 per thread (4096 floats); every load of a pass
// is issued before its first LDS store, so a pass costs one memory round trip.
// Same values and summation orders as pro_compute.
template <bool G>
OH_DEV void mv_prologue(const oh_mvseg &s, int slot, int blk, uint8_t *smem, double *red, bool q8) {
    // activations come from earlier phases: device-scope loads
    const int in = s.in, nb = in / 256, tid = tid_x(), wave = tid >> 6;
    int8_t *aqs = (int8_t *)smem;
    int16_t *abs = (int16_t *)(smem + mv_lds_bs_off(nb));
    float *ad = (float *)(smem + mv_lds_d_off(nb));
    float *v = (float *)(smem + mv_lds_v_off(nb));
    float4 *v4 = (float4 *)v;
    const size_t ao = (size_t)(s.adiv > 1 ? slot / s.adiv : slot) * s.astride;
    constexpr int PW = 4;                              // float4 per thread per pass
    if (s.pro == OH_PRO_Q8K) {
        if (q8) {
            const int4 *gq = (const int4 *)(s.xqs + ao);
            const int n16 = in / 16;
            for (int i0 = 0; i0 < n16; i0 += 256 * PW) {
                int4 r[PW];
#pragma unroll
                for (int u = 0; u < PW; u++) r[u] = ldw4<G>(gq + (i0 + tid + 256 * u < n16 ? i0 + tid + 256 * u : n16 - 1));
#pragma unroll
                for (int u = 0; u < PW; u++) {
                    const int i = i0 + tid + 256 * u;
                    if (i < n16) ((int4 *)aqs)[(i >> 4) * (kAS / 16) + (i & 15)] = r[u];
                }
            }
            for (int i = tid; i < nb * 16; i += 256) abs[i] = ldw<G>(s.xbs + ao / 16 + i);
            for (int i = tid; i < nb; i += 256) ad[i] = ldw<G>(s.xd + ao / 256 + i);
        } else {
            // any width (fallback rows): scalar passes of 16 per thread
            for (int i0 = 0; i0 < in; i0 += 256 * 16) {
                float r[16];
#pragma unroll
                for (int u = 0; u < 16; u++) r[u] = ldw<G>(s.xf + ao + (i0 + tid + 256 * u < in ? i0 + tid + 256 * u : in - 1));
#pragma unroll
                for (int u = 0; u < 16; u++)
                    if (i0 + tid + 256 * u < in) v[i0 + tid + 256 * u] = r[u];
            }
        }
        lds_barrier();
        return;
    }
    // in % 256 == 0 here (mv_add)
    const int n4 = in / 4;
    const float4 *x4 = (const float4 *)(s.xf + ao);
    if (s.pro == OH_PRO_GNORM) {
        // per head of gdim elements: inv_h = 1/sqrt(sum of the head's run
        // sums, in order / gdim + eps); v = x * inv_h * w * silu(z)
        float *hinv = v + in;                          // [in / gdim]
        const int gd = s.gdim, rpg = gd / 64, nhd = in / gd;
        for (int h = tid; h < nhd; h += 256) {
            double tot;
            if (s.runs16) {
                // 16-row partials: each 64-row run is (g0 + g1) + (g2 + g3)
                const double *g = s.xruns + ao / 16 + (size_t)h * (gd / 16);
                tot = (ldw<G>(g) + ldw<G>(g + 1)) + (ldw<G>(g + 2) + ldw<G>(g + 3));
                for (int k = 1; k < rpg; k++)
                    tot += (ldw<G>(g + 4 * k) + ldw<G>(g + 4 * k + 1)) + (ldw<G>(g + 4 * k + 2) + ldw<G>(g + 4 * k + 3));
            } else {
                const double *xr = s.xruns + ao / 64;  // the slot's run sums
                tot = ldw<G>(xr + h * rpg);
                for (int k = 1; k < rpg; k++) tot += ldw<G>(xr + h * rpg + k);
            }
            hinv[h] = (float)(1.0 / sqrt(tot / (double)gd + (double)s.eps));
        }
        lds_barrier();
        const float4 *z4 = (const float4 *)(s.xf2 + ao), *w4 = (const float4 *)s.nw;
        for (int i0 = 0; i0 < n4; i0 += 256 * PW) {
            float4 xr[PW], zr[PW], wr[PW];
#pragma unroll
            for (int u = 0; u < PW; u++) {
                const int f = i0 + tid + 256 * u < n4 ? i0 + tid + 256 * u : n4 - 1;
                xr[u] = ldw4<G>(x4 + f);
                zr[u] = ldw4<G>(z4 + f);
                wr[u] = ldg(w4 + f % (gd / 4));
            }
#pragma unroll
            for (int u = 0; u < PW; u++) {
                const int f = i0 + tid + 256 * u;
                if (f < n4) {
                    const float inv = hinv[4 * f / gd];
                    const float4 x = xr[u], z = zr[u], w = wr[u];
                    v4[f] = make_float4(x.x * inv * w.x * z.x, x.y * inv * w.y * z.y, x.z * inv * w.z * z.z,
                                        x.w * inv * w.w * z.w);
                }
            }
        }
        lds_barrier();
    } else if (s.pro == OH_PRO_SWIGLU) {
        const float4 *u4 = (const float4 *)(s.xf2 + ao);
        for (int i0 = 0; i0 < n4; i0 += 256 * PW) {
            float4 gr[PW], ur[PW];
#pragma unroll
            for (int u = 0; u < PW; u++) {
                const int f = i0 + tid + 256 * u < n4 ? i0 + tid + 256 * u : n4 - 1;
                gr[u] = ldw4<G>(x4 + f);
                ur[u] = ldw4<G>(u4 + f);
            }
#pragma unroll
            for (int u = 0; u < PW; u++)
                if (i0 + tid + 256 * u < n4) v4[i0 + tid + 256 * u] = f4_silu_mul(gr[u], ur[u]);
        }
        lds_barrier();
    } else {
        for (int i0 = 0; i0 < n4; i0 += 256 * PW) {
            float4 xr[PW];
#pragma unroll
            for (int u = 0; u < PW; u++) xr[u] = ldw4<G>(x4 + (i0 + tid + 256 * u < n4 ? i0 + tid + 256 * u : n4 - 1));
#pragma unroll
            for (int u = 0; u < PW; u++)
                if (i0 + tid + 256 * u < n4) v4[i0 + tid + 256 * u] = xr[u];
        }
        lds_barrier();
        if (s.pro == OH_PRO_NORM) {
            // the weights are requested before the reduction; the sum of
            // squares in the order of the stand-alone RMSNorm kernel
            const float4 *w4 = (const float4 *)s.nw;
            double ss = 0.0;
            for (int i = tid; i < in; i += 256) ss += (double)v[i] * v[i];
            ss = wave_sum_d(ss);
            if (lane_id() == 0) red[wave] = ss;
            lds_barrier();
            const double tot = (red[0] + red[1]) + (red[2] + red[3]);
            const float inv = (float)(1.0 / sqrt(tot / (double)in + (double)s.eps));
            for (int i0 = 0; i0 < n4; i0 += 256 * PW) {
                float4 wr[PW];
#pragma unroll
                for (int u = 0; u < PW; u++) wr[u] = ldg(w4 + (i0 + tid + 256 * u < n4 ? i0 + tid + 256 * u : n4 - 1));
#pragma unroll
                for (int u = 0; u < PW; u++) {
                    const int f = i0 + tid + 256 * u;
                    if (f < n4) {
                        const float4 x = v4[f], w = wr[u];
                        v4[f] = make_float4(x.x * inv * w.x, x.y * inv * w.y, x.z * inv * w.z, x.w * inv * w.w);
                    }
                }
            }
            lds_barrier();
        }
    }
    const bool store = blk == 0 && s.oqs != nullptr;
    if (blk == 0 && s.oxf)
        for (int f = tid; f < n4; f += 256) stc4((float4 *)(s.oxf + ao) + f, v4[f]);
    if (q8 || store) {
        for (int qb = wave; qb < nb; qb += 4) {
            q8k_block_from_lds(v, qb, aqs, ad, abs, kAS);
            if (store) q8k_block_from_lds<true>(v, qb, s.oqs + ao, s.oqd + ao / 256, s.oqb + ao / 16);
        }
    }
    lds_barrier();
}

// Prologue inputs held in registers (in <= 4096): they are loaded before the
// first weight step, and the prologue consumes them while that step is still
// in flight (vector loads complete in order, so inputs loaded after the
// weights would wait for them).
struct PIn { float4 a[4], b[4], c[4]; int4 q, bsv; float d; double r0, r1; };

template <bool G>
OH_DEV void pro_load(PIn &p, const oh_mvseg &s, int slot) {
    const int tid = tid_x(), in = s.in, nb = in / 256;
    const size_t ao = (size_t)(s.adiv > 1 ? slot / s.adiv : slot) * s.astride;
    if (s.pro == OH_PRO_Q8K) {
        const int n16 = in / 16;
        p.q = ldw4<G>((const int4 *)(s.xqs + ao) + (tid < n16 ? tid : n16 - 1));
        p.bsv = ldw4<G>((const int4 *)(s.xbs + ao / 16) + (tid < 2 * nb ? tid : 2 * nb - 1));
        p.d = ldw<G>(s.xd + ao / 256 + (tid < nb ? tid : nb - 1));
    } else {
        // activations from earlier phases (device-scope loads); the RMSNorm
        // weights are constant
        const float4 *x = (const float4 *)(s.xf + ao);
        const bool wc = s.pro == OH_PRO_NORM;
        const float4 *w = (const float4 *)(wc ? s.nw : s.pro == OH_PRO_F32 ? s.xf + ao : s.xf2 + ao);
        // nk float4 per thread cover the input (a uniform bound: no
        // duplicate requests for the unused slots)
        const int n4 = in / 4, nk = (n4 + 255) / 256;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            if (k < nk) {
                const int i = tid + 256 * k < n4 ? tid + 256 * k : n4 - 1;
                p.a[k] = ldw4<G>(x + i);
                p.b[k] = wc ? ldg(w + i) : ldw4<G>(w + i);
                if (s.pro == OH_PRO_GNORM) p.c[k] = ldg((const float4 *)s.nw + i % (s.gdim / 4));
            } else {
                p.a[k] = p.b[k] = p.c[k] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            }
        }
        if (s.pro == OH_PRO_GNORM) {
            if (s.runs16) {
                // 16-row partials (in/16 <= 256): this thread's one
                const int n16 = in / 16;
                p.r0 = ldw<G>(s.xruns + ao / 16 + (tid < n16 ? tid : n16 - 1));
            } else {
                // this thread's head (tid < in/gdim): its first two run sums
                const int rpg = s.gdim / 64, nh = in / s.gdim, h = tid < nh ? tid : nh - 1;
                const double *xr = s.xruns + ao / 64;  // the slot's run sums
                p.r0 = ldw<G>(xr + h * rpg);
                p.r1 = ldw<G>(xr + h * rpg + (rpg > 1 ? 1 : 0));
            }
        }
    }
}

// Q8_K of one 256-element block held in registers by a wave, four
// consecutive elements x per lane (lane l: elements 4l..4l+3). Same result as
// q8k_block_from_lds: the scale comes from the first element of largest
// magnitude, i.e. the first such element of the lowest lane holding one (a
// ballot, then a read of that lane). q8k_pivot forms (largest magnitude,
// signed element) and q8k_emit the codes, bsums and d, so that a wave can
// run the reductions of several blocks back to back. G: the planes are
// global memory read by other workgroups (device-scope stores).
struct Q8kPiv { float best, piv; };
OH_DEV Q8kPiv q8k_pivot(const float4 x) {
    const float a0 = fabsf(x.x), a1 = fabsf(x.y), a2 = fabsf(x.z), a3 = fabsf(x.w);
    const float best = wave_max_fast(fmaxf(fmaxf(a0, a1), fmaxf(a2, a3)));
    const float v = a0 == best ? x.x : (a1 == best ? x.y : (a2 == best ? x.z : x.w));
    const uint64_t m = __ballot(a0 == best || a1 == best || a2 == best || a3 == best);
    const int l = m ? (int)__builtin_ctzll(m) : 0;
    return {best, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l))};
}
template <bool G = false>
OH_DEV void q8k_emit(const float4 x, const Q8kPiv p, int qb, int8_t *qs, float *d, int16_t *bs, int qstride) {
    const int lane = lane_id();
    int *qw = (int *)(qs + (int64_t)qb * qstride) + lane;
    int16_t *b = bs + (int64_t)qb * 16;
    auto put32 = [&](int *p, int v) { if (G) stc(p, v); else *p = v; };
    auto put16 = [&](int16_t *p, int16_t v) { if (G) stc(p, v); else *p = v; };
    auto putf = [&](float *p, float v) { if (G) stc(p, v); else *p = v; };
    // an all-zero (or NaN-led) block has zero codes, bsums and d
    const bool zero = p.best == 0.0f || !(p.best > 0.0f);
    const float iscale = zero ? 0.0f : -127.0f / p.piv;
    int c[4];
    const float xs[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int v = (int)__builtin_rintf(iscale * xs[j]);
        c[j] = zero ? 0 : (v > 127 ? 127 : (v < -128 ? -128 : v));
    }
    put32(qw, (c[0] & 0xff) | ((c[1] & 0xff) << 8) | ((c[2] & 0xff) << 16) | ((c[3] & 0xff) << 24));
    int sv = c[0] + c[1] + c[2] + c[3];
    sv += dpp_i<0xB1>(sv);
    sv += dpp_i<0x4E>(sv);                         // codes 16*(lane/4) .. +15
    if ((lane & 3) == 0) put16(b + (lane >> 2), (int16_t)sv);
    if (lane == 0) putf(d + qb, zero ? 0.0f : 1.0f / iscale);
}

OH_DEV void pro_compute(const PIn &p, const oh_mvseg &s, int slot, int blk, uint8_t *smem, double *red) {
    const int in = s.in, nb = in / 256, tid = tid_x(), wave = tid >> 6;
    int8_t *aqs = (int8_t *)smem;
    int16_t *abs = (int16_t *)(smem + mv_lds_bs_off(nb));
    float *ad = (float *)(smem + mv_lds_d_off(nb));
    float *v = (float *)(smem + mv_lds_v_off(nb));
    float4 *v4 = (float4 *)v;
    const size_t ao = (size_t)(s.adiv > 1 ? slot / s.adiv : slot) * s.astride;
    if (s.pro == OH_PRO_Q8K) {
        if (tid < in / 16) ((int4 *)aqs)[(tid >> 4) * (kAS / 16) + (tid & 15)] = p.q;
        if (tid < 2 * nb) ((int4 *)abs)[tid] = p.bsv;
        if (tid < nb) ad[tid] = p.d;
        lds_barrier();
        return;
    }
    // the activation in registers: thread tid owns float4 tid + 256k, i.e.
    // elements 4*lane.. of super-block wave + 4k
    const int n4 = in / 4;
    float4 fv[4];
#pragma unroll
    for (int k = 0; k < 4; k++) fv[k] = s.pro == OH_PRO_SWIGLU ? f4_silu_mul(p.a[k], p.b[k]) : p.a[k];
    if (s.pro == OH_PRO_GNORM) {
        // per head of gdim elements (src/ornith_rforward.c:300-319): the runs'
        // double sums of squares added in order, inv = 1/sqrt(ss/gdim + eps),
        // v = v * inv * w * silu(z)
        float *hinv = v;                            // [in/gdim]
        const int gd = s.gdim, rpg = gd / 64;
        if (s.runs16) {
            // the 16-row partials through LDS (after hinv's at most 64
            // floats); each 64-row run is (g0 + g1) + (g2 + g3)
            double *gp = (double *)(v + 64);
            if (tid < in / 16) gp[tid] = p.r0;
            lds_barrier();
            if (tid < in / gd) {
                const double *g = gp + tid * (gd / 16);
                double tot = (g[0] + g[1]) + (g[2] + g[3]);
                for (int k = 1; k < rpg; k++) tot += (g[4 * k] + g[4 * k + 1]) + (g[4 * k + 2] + g[4 * k + 3]);
                hinv[tid] = (float)(1.0 / sqrt(tot / (double)gd + (double)s.eps));
            }
        } else if (tid < in / gd) {
            double tot = p.r0;
            if (rpg > 1) tot += p.r1;
            for (int k = 2; k < rpg; k++) tot += ldc(s.xruns + ao / 64 + tid * rpg + k);
            hinv[tid] = (float)(1.0 / sqrt(tot / (double)gd + (double)s.eps));
        }
        lds_barrier();
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int f = tid + 256 * k < n4 ? tid + 256 * k : n4 - 1;
            const float inv = hinv[4 * f / gd];
            const float4 x = p.a[k], z = p.b[k], w = p.c[k];
            fv[k] = make_float4(x.x * inv * w.x * z.x, x.y * inv * w.y * z.y, x.z * inv * w.z * z.z,
                                x.w * inv * w.w * z.w);
        }
    }
    if (s.pro == OH_PRO_NORM) {
        // same summation order as the stand-alone RMSNorm kernel
#pragma unroll
        for (int k = 0; k < 4; k++)
            if (tid + 256 * k < n4) v4[tid + 256 * k] = fv[k];
        lds_barrier();
        double ss = 0.0;
        for (int i = tid; i < in; i += 256) ss += (double)v[i] * v[i];
        ss = wave_sum_d(ss);
        if (lane_id() == 0) red[wave] = ss;
        lds_barrier();
        const double tot = (red[0] + red[1]) + (red[2] + red[3]);
        const float inv = (float)(1.0 / sqrt(tot / (double)in + (double)s.eps));
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const float4 x = p.a[k], w = p.b[k];
            fv[k] = make_float4(x.x * inv * w.x, x.y * inv * w.y, x.z * inv * w.z, x.w * inv * w.w);
        }
    }
    const bool store = blk == 0 && s.oqs != nullptr;
    // the pivots of the wave's blocks wave + 4k first (independent
    // reductions back to back), then their codes
    Q8kPiv pv[4];
#pragma unroll
    for (int k = 0; k < 4; k++)
        if (wave + 4 * k < nb) pv[k] = q8k_pivot(fv[k]);
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int qb = wave + 4 * k;
        if (qb < nb) {
            if (blk == 0 && s.oxf) stc4((float4 *)(s.oxf + ao) + tid + 256 * k, fv[k]);
            q8k_emit(fv[k], pv[k], qb, aqs, ad, abs, kAS);
            if (store) q8k_emit<true>(fv[k], pv[k], qb, s.oqs + ao, s.oqd + ao / 256, s.oqb + ao / 16, 256);
        }
    }
    lds_barrier();
}

// Integer-path segment slot: every lane reduces one super-block; a wave step
// covers 64/nb rows. Steps are double-buffered: the next step's loads are in
// flight while the current one is reduced. All loads are unconditional
// (dead lanes and steps past the end re-read an in-bounds block), so the
// compiler never has to drain the queue at a branch. expert: the slot's
// expert for stacked tensors. Inside the step kernel (W::kGrid) the first
// step's weights are requested before the grid wait: they do not depend on
// the previous phase.
// LT::kLate: the slot's expert is known only after the activation is formed
// (late() routes the block, fused router): prologue first, then late(), then
// the first weights. Otherwise `expert` is given.
struct NoLate {
    static constexpr bool kLate = false;
    OH_DEV int operator()() const { return 0; }
};
template <class F> struct LateExpert {
    static constexpr bool kLate = true;
    F f;
    OH_DEV int operator()() const { return f(); }
};
template <int T, class W, class LT = NoLate>
OH_DEV void mv_seg(const oh_mvseg &s, int slot, int blk, int expert, uint8_t *smem, double *red, W &w,
                   LT late = LT()) {
    const int lane = lane_id(), wave = __builtin_amdgcn_readfirstlane(tid_x() >> 6);
    const int nb = s.nb, rps = 64 / nb;
    const int rl = lane / nb, sb = lane - rl * nb;
    const int u0 = (blk * OH_MV_WAVES + wave) * s.upw;
    const int u1 = u0 + s.upw < s.units ? u0 + s.upw : s.units;
    // paired segments: step 2u reduces W, step 2u+1 the pair W2, same rows
    const int sps = s.pair ? 2 : 1;
    const int S = u1 > u0 ? (u1 - u0) * sps : 0;
    int64_t row_base = (int64_t)expert * s.rows;            // set by late() in the late form
    float *y = s.y + (size_t)slot * s.ystride;
    const WP wp = {s.A, s.B, s.C}, wp2 = {s.A2, s.B2, s.C2};
    const uint32_t tag = s.mode == 2 ? (uint32_t)ldw<W::kGrid>(s.tagp) + 1u : 0u;
    const int8_t *aq = (const int8_t *)smem + sb * kAS;
    const int16_t *abs = (const int16_t *)(smem + mv_lds_bs_off(nb)) + sb * 16;
    const float *adp = (const float *)(smem + mv_lds_d_off(nb)) + sb;
    SB<T> ra, rb;
    auto load = [&](SB<T> &r, int st) {
        const int sc = st < S ? st : S - 1;
        int unit = u0 + sc / sps;
        unit = unit < 0 ? 0 : (unit >= s.units ? s.units - 1 : unit);
        const int row = unit * rps + (rl < rps ? rl : rps - 1);
        const int rowc = row < s.rows ? row : s.rows - 1;
        sb_load(r, (sc & (sps - 1)) ? wp2 : wp, (row_base + rowc) * nb + sb);
    };
    float gsum = 0.0f;
    // y += dot (mode 1): the first step's output row is read together with
    // the prologue inputs rather than after the reduction
    float ypre = 0.0f;
    auto comp = [&](const SB<T> &r, int st) {
        const int row = (u0 + st / sps) * rps + rl;
        const bool live = st < S && rl < rps && row < s.rows;
        const float tw = sb_term(r, aq, abs, *adp);
        const float t = live ? tw : 0.0f;
        // the row's super-block terms in order, from 0 (lanes rl*nb .. +nb-1)
        float acc = 0.0f;
        for (int i = 0; i < nb; i++) acc += shfl(t, rl * nb + i);
        if (s.pair) {
            if ((st & 1) == 0) gsum = acc;
            else if (live && sb == 0) emit<W::kGrid>(y, 0, row, ref_silu(gsum) * acc);
        } else if (live && sb == 0) {
            if (s.mode == 2) stc((uint64_t *)y + row, (uint64_t)tag << 32 | f2u(acc));
            else if (s.mode == 1 && st == 0) put<W::kGrid>(y + row, ypre + acc);
            else emit<W::kGrid>(y, s.mode, row, acc);
        }
    };
    auto y_prefetch = [&]() {
        const int row = u0 * rps + rl;
        if (s.mode == 1 && !s.pair && S > 0 && rl < rps && row < s.rows && sb == 0) ypre = ldw<W::kGrid>(y + row);
    };
    if (LT::kLate) {
        // the activation while the routing is still being published, then
        // the routed expert's first weights
        if (!w.wait()) return;
        y_prefetch();
        if (s.in <= 4096) {
            PIn pin;
            pro_load<W::kGrid>(pin, s, slot);
            pro_compute(pin, s, slot, blk, smem, red);
        } else {
            mv_prologue<W::kGrid>(s, slot, blk, smem, red, true);
        }
        row_base = (int64_t)late() * s.rows;
        load(ra, 0);
    } else if (s.in <= 4096) {
        PIn pin;
        if (W::kGrid) {
            load(ra, 0);
            if (!w.wait()) return;
            pro_load<W::kGrid>(pin, s, slot);
            y_prefetch();
        } else {
            pro_load<W::kGrid>(pin, s, slot);
            y_prefetch();
            load(ra, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
        pro_compute(pin, s, slot, blk, smem, red);
    } else {
        load(ra, 0);
        if (!w.wait()) return;
        y_prefetch();
        mv_prologue<W::kGrid>(s, slot, blk, smem, red, true);
    }
    // ra holds step 0; a step's loads are only issued when it will be reduced
    int st = 0;
    for (; st + 2 < S; st += 2) {
        load(rb, st + 1);
        comp(ra, st);
        load(ra, st + 2);
        comp(rb, st + 1);
    }
    if (st + 1 < S) {
        load(rb, st + 1);
        comp(ra, st);
        comp(rb, st + 1);
    } else if (st < S) {
        comp(ra, st);
    }
}

// Top-k routing of one token by wave 0 of a block (ne = 64 V logits, lane l
// holding experts V l .. V l + V - 1): k rounds of a wave maximum, the
// lowest index among equal maxima taken (the reference's ascending scan with
// strict '>'), the pick removed from its lane. The softmax over the picks in
// selection order: max = the first pick, e_s = expf(l_s - max), the sum in
// order, w_s = e_s / sum. Returns false (nothing written) when a logit is NaN
// or -inf: the sequential selection handles those.
template <int V>
OH_DEV bool route_pick(float (&a)[V], int k, int *sel, float *rw) {
    const int lane = lane_id();
    bool fin = true;
#pragma unroll
    for (int j = 0; j < V; j++) fin = fin && a[j] > -INFINITY;
    if (__ballot(!fin)) return false;
    float mine = 0.0f, mx = 0.0f;
    int pick = 0;
    for (int s = 0; s < k; s++) {
        float m = a[0];
#pragma unroll
        for (int j = 1; j < V; j++) m = fmaxf(m, a[j]);
        const float M = wave_max_fast(m);
        int jl = V;
#pragma unroll
        for (int j = V - 1; j >= 0; j--) if (a[j] == M) jl = j;
        const uint64_t hm = __ballot(jl < V);
        const int L = (int)__builtin_ctzll(hm);
        const int J = __builtin_amdgcn_readlane(jl, L);
        if (lane == L) {
#pragma unroll
            for (int j = 0; j < V; j++) if (j == J) a[j] = -INFINITY;
        }
        if (s == 0) mx = M;
        if (lane == s) { mine = M; pick = V * L + J; }
    }
    const float e = lane < k ? ref_expf(mine - mx) : 0.0f;
    float sum = 0.0f;
    for (int s = 0; s < k; s++) sum += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e), s));
    if (lane < k) { sel[lane] = pick; rw[lane] = e / sum; }
    return true;
}
template <int V>
OH_DEV bool route_fast(const float *rlog, int k, int *sel, float *rw) {
    const int lane = lane_id();
    float a[V];
#pragma unroll
    for (int q = 0; q < V / 4; q++) {
        const float4 t = ldc4((const float4 *)rlog + V / 4 * lane + q);
        a[4 * q] = t.x; a[4 * q + 1] = t.y; a[4 * q + 2] = t.z; a[4 * q + 3] = t.w;
    }
    return route_pick<V>(a, k, sel, rw);
}

// Router logits published in this launch as tagged words (oh_mvlaunch.rtag):
// wave 0, lane l polling experts V l .. V l + V - 1 (and lane 0 the shared
// gate's word) with device-scope loads until every word carries `tag`; the
// values into a[] (and *shl). Returns false when the words did not arrive
// within the bound (about 10 ms).
constexpr int kRouteSpin = 1 << 14;
// Wave-uniform bounded wait until *ctr >= n (lane 0 polls, device-scope
// loads with a short sleep between them). False when it gave up.
OH_DEV bool wait_count(const int32_t *ctr, int n) {
    int ok = 1;
    if (lane_id() == 0) {
        for (int it = 0; ldc(ctr) < n; it++) {
            if (it >= kRouteSpin) { ok = 0; break; }
            __builtin_amdgcn_s_sleep(2);
        }
    }
    return __builtin_amdgcn_readfirstlane(ok) != 0;
}
// The wait of a workgroup whose inputs other workgroups of the same launch
// produce (the projection part of the delta-step launch): one thread polls
// the arrival counter until it reaches n (bounded), the block takes one
// decision (the departure is counted at the end of the workgroup's work,
// fused_depart). A wait that gives up sets the error flag. kGrid: the inputs
// are read with device-scope loads.
struct CtrWait {
    static constexpr bool kGrid = true;
    int32_t *arr;
    int n;
    int32_t *err;
    bool done, ok;
    OH_DEV bool wait() {
        if (done) return ok;
        done = true;
        __shared__ int s_ok;
        if (tid_x() == 0) {
            // polled about every 0.4 us: every projection block polls the
            // one counter the delta blocks add to
            bool got = true;
            for (int it = 0; ldc(arr) < n; it++) {
                if (it >= kRouteSpin / 4) { got = false; break; }
                __builtin_amdgcn_s_sleep(16);
            }
            s_ok = got ? 1 : 0;
            if (!got) atomicOr(err, OH_ERR_WAIT);
        }
        __syncthreads();
        ok = s_ok != 0;
        return ok;
    }
};

template <int V>
OH_DEV bool route_poll(const uint64_t *tw, uint32_t tag, bool has_sh, float (&a)[V], float *shl) {
    const int lane = lane_id(), ne = 64 * V;
    uint64_t w[V], wsh = 0;
#pragma unroll
    for (int j = 0; j < V; j++) w[j] = ldc(tw + V * lane + j);
    if (has_sh && lane == 0) wsh = ldc(tw + ne);
    for (int it = 0;; it++) {
        bool ok = true;
#pragma unroll
        for (int j = 0; j < V; j++) ok = ok && (uint32_t)(w[j] >> 32) == tag;
        if (has_sh && lane == 0) ok = ok && (uint32_t)(wsh >> 32) == tag;
        if (__ballot(!ok) == 0) break;
        if (it >= kRouteSpin) return false;
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int j = 0; j < V; j++)
            if ((uint32_t)(w[j] >> 32) != tag) w[j] = ldc(tw + V * lane + j);
        if (has_sh && lane == 0 && (uint32_t)(wsh >> 32) != tag) wsh = ldc(tw + ne);
    }
#pragma unroll
    for (int j = 0; j < V; j++) a[j] = u2f((uint32_t)w[j]);
    if (has_sh && lane == 0) *shl = u2f((uint32_t)wsh);
    return true;
}

// MoE routing of a block (src/ornith_moe.c:8-30). With 256 or 512 experts
// wave 0 selects them (route_fast). Otherwise expert e's rank is the
// number of experts that precede it in the reference's selection order
// (larger logit, or equal logit and lower index); the k experts of rank < k in
// rank order are the reference's picks. Softmax over the selected logits in
// that order by one thread. Logits that are NaN or -inf fall back to the
// sequential selection of one wave. Results in LDS (sel, w, *shg); with
// `store` the block also stores them (token tok's) for later phases.
OH_DEV void route_block(const oh_mvlaunch &L, int tok, bool store, float *lg, int *sel, float *rw, float *shg,
                        int *bad, int *cnt) {
    const int tid = tid_x(), ne = L.ne, k = L.topk;
    const int ne4 = (ne + 3) & ~3;
    const bool has_sh = L.shl != nullptr;
    const float *rlog = L.rlog + (size_t)tok * ne;
    if ((ne == 256 || ne == 512) && k <= 64) {
        // wave 0 selects; the other waves wait at the barrier
        int ok = 1;
        if (tid < 64) {
            ok = ne == 256 ? route_fast<4>(rlog, k, sel, rw) : route_fast<8>(rlog, k, sel, rw);
            if (ok && tid == 0 && has_sh) *shg = ref_sigmoid(ldc(L.shl + tok));
            if (tid == 0) *bad = !ok;
        }
        __syncthreads();
        if (*bad) {
            for (int e = tid; e < ne4; e += 256) lg[e] = e < ne ? ldc(rlog + e) : -INFINITY;
            __syncthreads();
            if (tid < 64) route_wave(lg, ne, k, nullptr, sel, rw, shg);
            if (tid == 0 && has_sh) *shg = ref_sigmoid(ldc(L.shl + tok));
            __syncthreads();
        }
        if (store) {
            if (tid < k) { stc(L.ridx + (size_t)tok * k + tid, (int32_t)sel[tid]); stc(L.rw + (size_t)tok * k + tid, rw[tid]); }
            if (tid == 0 && has_sh) stc(L.shg + tok, *shg);
        }
        return;
    }
    if (tid == 0) *bad = 0;
    if (tid < 64) cnt[tid] = 0;
    for (int e = tid; e < ne4; e += 256) lg[e] = e < ne ? ldc(rlog + e) : -INFINITY;
    __syncthreads();
    const float shl = has_sh ? ldc(L.shl + tok) : 0.0f;
    // rank by strictly larger logits; equal logits inside the top k (or a
    // NaN / -inf anywhere) send the block to the sequential selection
    const float4 *l4 = (const float4 *)lg;
    for (int e = tid; e < ne; e += 256) {
        const float v = lg[e];
        if (!(v > -INFINITY)) *bad = 1;
        int gt = 0;
#pragma unroll 8
        for (int j = 0; j < ne4 / 4; j++) {
            const float4 u = l4[j];
            gt += (int)(u.x > v) + (int)(u.y > v) + (int)(u.z > v) + (int)(u.w > v);
        }
        if (gt < k) {
            if (atomicAdd(&cnt[gt], 1) != 0) *bad = 1;
            sel[gt] = e;
        }
    }
    __syncthreads();
    if (*bad) {
        if (tid < 64) route_wave(lg, ne, k, nullptr, sel, rw, shg);
        if (tid == 0 && has_sh) *shg = ref_sigmoid(shl);
    } else if (tid < 64) {
        // lane j: e_j = exp(l_j - max) in parallel; the sum in selection
        // order, then w_j = e_j / sum
        const float lj = tid < k ? lg[sel[tid]] : -INFINITY;
        const float mx = wave_max_fast(lj);
        const float e = tid < k ? ref_expf(lj - mx) : 0.0f;
        float sum = 0.0f;
        for (int j = 0; j < k; j++) sum += shfl(e, j);
        if (tid < k) rw[tid] = e / sum;
        if (tid == 0 && has_sh) *shg = ref_sigmoid(shl);
    }
    __syncthreads();
    if (store) {
        if (tid < k) { stc(L.ridx + (size_t)tok * k + tid, (int32_t)sel[tid]); stc(L.rw + (size_t)tok * k + tid, rw[tid]); }
        if (tid == 0 && has_sh) stc(L.shg + tok, *shg);
    }
}

// MoE routing of a block from logits published in this launch (L.rtag, one
// token): wave 0 polls the tagged words (route_poll) and selects as
// route_block does, the same picks and weights; lg: LDS for the sequential
// selection when a logit is NaN or -inf. A wait that gives up sets the
// session's error word (OH_ERR_WAIT) and routes zeros.
OH_DEV void route_fused(const oh_mvlaunch &L, bool store, float *lg, int *sel, float *rw, float *shg, int *bad) {
    const int tid = tid_x(), ne = L.ne, k = L.topk;
    const bool has_sh = L.rsh != 0;
    if (tid < 64) {
        const uint32_t ser = (uint32_t)ldc(L.rio + OH_IO_SERIAL), tag = ser + 1u;
        float shl = 0.0f;
        bool got = wait_count(L.mctr + (ser & 1u), L.nrb);
        int ok = 1;
        if (ne == 256) {
            float a[4];
            got = route_poll<4>(L.rtag, tag, has_sh, a, &shl) && got;
            if (!got) {
#pragma unroll
                for (int j = 0; j < 4; j++) a[j] = 0.0f;
            }
            ok = route_pick<4>(a, k, sel, rw);
            if (!ok)
#pragma unroll
                for (int j = 0; j < 4; j++) lg[4 * tid + j] = u2f((uint32_t)ldc(L.rtag + 4 * tid + j));
        } else {
            float a[8];
            got = route_poll<8>(L.rtag, tag, has_sh, a, &shl) && got;
            if (!got) {
#pragma unroll
                for (int j = 0; j < 8; j++) a[j] = 0.0f;
            }
            ok = route_pick<8>(a, k, sel, rw);
            if (!ok)
#pragma unroll
                for (int j = 0; j < 8; j++) lg[8 * tid + j] = u2f((uint32_t)ldc(L.rtag + 8 * tid + j));
        }
        if (!got && tid == 0) atomicOr(L.rio + OH_IO_ERR, OH_ERR_WAIT);
        if (tid == 0) { *bad = !ok; if (has_sh) *shg = ref_sigmoid(shl); }
        // the sequential selection over the copy (route_pick wrote nothing)
        if (!ok) {
            wave_lds_sync();
            route_wave(lg, ne, k, nullptr, sel, rw, nullptr);
        }
    }
    __syncthreads();
    if (store) {
        if (tid < k) { stc(L.ridx + tid, (int32_t)sel[tid]); stc(L.rw + tid, rw[tid]); }
        if (tid == 0 && has_sh) stc(L.shg, *shg);
    }
}

// IQ2_XXS rows in tolerance mode (segment flag iq2tree): the reference's f32
// arithmetic (f32 activation, every weight decoded exactly, src/ornith_quant.c
// :660-680) with the dot summed as a tree instead of in element order (its f32
// fallback, src/ornith_rforward.c:119-133). Lane l of a wave owns elements
// [l E, (l + 1) E) of every row (E = in / 64, whole 8-weight codebook
// entries) and keeps that slice of x in registers; a wave walks its rows one
// per step (gate and up rows of a pair in turn), with the next rows' words in
// flight. Per row the lane adds, for each sub-block part it owns,
// db * sum_j (g_j s_j) x_j (db = d (0.5 + ls) 0.25, the decoder's scale) and
// the 64 lane sums meet in a butterfly.
template <int E, class W>
OH_DEV void iq2_tree(const oh_mvseg &s, int slot, int blk, int expert, W &w) {
    constexpr int NSB = E >= 32 ? E / 32 : 1;       // sub-blocks the lane touches
    constexpr int NGE = E >= 32 ? 4 : E / 8;        // codebook entries per touched sub-block
    const int lane = lane_id(), wave = __builtin_amdgcn_readfirstlane(tid_x() >> 6);
    const int nb = s.in / 256, e0 = lane * E;
    const int sbl = e0 / 256, sub0 = (e0 % 256) / 32, ge0 = E >= 32 ? 0 : (e0 % 32) / 8;
    const int u0 = (blk * OH_MV_WAVES + wave) * s.upw;
    const int u1 = u0 + s.upw < s.units ? u0 + s.upw : s.units;
    const int sps = s.pair ? 2 : 1;
    const int S = u1 > u0 ? (u1 - u0) * sps : 0;
    const int64_t row_base = (int64_t)expert * s.rows;
    float *y = s.y + (size_t)slot * s.ystride;
    const WP wp = {s.A, s.B, s.C}, wp2 = {s.A2, s.B2, s.C2};
    iq2_tables_load();
    struct RW { uint32_t q[2 * NSB]; uint32_t d; };
    auto load = [&](RW &r, int st) {
        int sc = st < S ? st : S - 1;
        sc = sc < 0 ? 0 : sc;
        int row = u0 + sc / sps;
        row = row < s.units ? row : s.units - 1;
        const WP &p = (sc & (sps - 1)) ? wp2 : wp;
        const int64_t bi = (row_base + row) * nb + sbl;
        const uint32_t *q = (const uint32_t *)(p.A + bi * 64) + 2 * sub0;
        if constexpr (NSB == 2) {
            const uint4 v = ldg((const uint4 *)q);
            r.q[0] = v.x; r.q[1] = v.y; r.q[2] = v.z; r.q[3] = v.w;
        } else {
            const uint2 v = ldg((const uint2 *)q);
            r.q[0] = v.x; r.q[1] = v.y;
        }
        r.d = ldg((const uint16_t *)(p.C + bi * 2));
    };
    RW ra, rb;
    load(ra, 0);
    if (!w.wait()) return;
    // this lane's slice of the f32 activation (from an earlier launch)
    const size_t ao = (size_t)(s.adiv > 1 ? slot / s.adiv : slot) * s.astride;
    float x[E];
    const float4 *x4 = (const float4 *)(s.xf + ao + e0);
#pragma unroll
    for (int i = 0; i < E / 4; i++) {
        const float4 v = ldc4(x4 + i);
        x[4 * i] = v.x; x[4 * i + 1] = v.y; x[4 * i + 2] = v.z; x[4 * i + 3] = v.w;
    }
    lds_barrier();                                   // the tables
    auto dot = [&](const RW &r) {
        const float dd = h2f((uint16_t)r.d);
        float acc = 0.0f;
#pragma unroll
        for (int b = 0; b < NSB; b++) {
            const uint32_t w0 = r.q[2 * b], w1 = r.q[2 * b + 1];
            const float db = dd * (0.5f + (float)(w1 >> 28)) * 0.25f;
            float part = 0.0f;
#pragma unroll
            for (int e = 0; e < NGE; e++) {
                const int ge = ge0 + e;
                const uint64_t g = s_iq2_grid[(w0 >> (8 * ge)) & 0xffu];
                const uint64_t m = s_iq2_sign[(w1 >> (7 * ge)) & 127u];
                const uint32_t ml = (uint32_t)m, mh = (uint32_t)(m >> 32);
                const uint32_t sl = ((uint32_t)g ^ ml) + (ml & 0x01010101u);
                const uint32_t sh = ((uint32_t)(g >> 32) ^ mh) + (mh & 0x01010101u);
                const int xo = b * 32 + e * 8;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    part = fmaf((float)(int8_t)(sl >> (8 * j)), x[xo + j], part);
                    part = fmaf((float)(int8_t)(sh >> (8 * j)), x[xo + 4 + j], part);
                }
            }
            acc = fmaf(db, part, acc);
        }
        return wave_sum_f(acc);
    };
    float gsum = 0.0f;
    auto comp = [&](const RW &r, int st) {
        const float t = dot(r);
        const int row = u0 + st / sps;
        if (s.pair) {
            if ((st & 1) == 0) gsum = t;
            else if (lane == 0) emit(y, 0, row, ref_silu(gsum) * t);
        } else if (lane == 0) {
            emit(y, s.mode, row, t);
        }
    };
    int st = 0;
    for (; st + 2 < S; st += 2) {
        load(rb, st + 1);
        comp(ra, st);
        load(ra, st + 2);
        comp(rb, st + 1);
    }
    if (st + 1 < S) {
        load(rb, st + 1);
        comp(ra, st);
        comp(rb, st + 1);
    } else if (st < S) {
        comp(ra, st);
    }
}

// Launch body. TK >= 0: every segment is an integer-path segment of type TK;
// TK == OH_MV_Q4Q6: integer-path segments of types Q4_K and Q6_K only (the GQA
// q/k/v launch), so no other segment form is compiled into the kernel;
// TK < 0: any mix, including fallback segments (one lane per row, the f32
// activation in LDS). With L.route every block first routes the MoE and
// stacked segments take their experts from that routing. vb: the virtual
// block (blockIdx.x of a standalone launch).
// a router block of the fused MoE launch counts itself in this step's parity
// once every wave's tagged stores have completed; the first gate/up block
// clears the other parity's counter for the next step
OH_DEV void fused_count(const oh_mvlaunch &L, int vb, bool router) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid_x() == 0) {
        const uint32_t ser = (uint32_t)ldc(L.rio + OH_IO_SERIAL);
        if (router)
            __hip_atomic_fetch_add(L.mctr + (ser & 1u), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else if (vb == L.pb0)
            stc(L.mctr + ((ser & 1u) ^ 1u), 0);
    }
}
// the delta-step launch's consumer departure at the end of its work: the last
// of ncons consumers, every one of them past its wait and so every producer
// arrived, sets both counters back to 0
OH_DEV void fused_depart(int32_t *arr, int32_t *dep, int ncons) {
    if (tid_x() == 0 && __hip_atomic_fetch_add(dep, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == ncons - 1) {
        stc(arr, 0);
        stc(dep, 0);
    }
}

// The block's segment: every segment's first block is read at once (a
// while loop over them is a chain of dependent kernel-argument reads).
OH_DEV int seg_index(const oh_mvlaunch &L, int vb) {
    const int n = L.n;
    int b0[OH_MAX_SEGS];
#pragma unroll
    for (int i = 1; i < OH_MAX_SEGS; i++) b0[i] = L.s[i].block0;
    int si = 0;
#pragma unroll
    for (int i = 1; i < OH_MAX_SEGS; i++) si += i < n && vb >= b0[i] ? 1 : 0;
    return si;
}

template <int TK, class W>
OH_DEV void mv_body(const oh_mvlaunch &L, int vb, W &w) {
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ double red[4];
    __shared__ int rsel[64], rbad, rcnt[64];
    __shared__ float rwt[64], rshg;
    const oh_mvseg &s = L.s[seg_index(L, vb)];
    const int bseg = vb - s.block0;
    const int slot = bseg / s.bps, blk = bseg - slot * s.bps;
    if (L.rtag) {
        // router published in this launch (one token): a stacked segment's
        // block forms its activation, then routes (the first block of slot 0
        // stores the routing for the down projection), then streams its
        // expert's weights; the router, shared-gate and shared-expert
        // segments need no routing
        if (s.eidx) {
            if constexpr (TK == -1) {
                if (s.type == OH_IQ2_XXS && !s.iq2tree) {
                    // IQ2_XXS fallback rows: the normalised f32 activation
                    // first (while the router blocks run), then the routing,
                    // then the routed expert's rows
                    mv_prologue<W::kGrid>(s, slot, blk, smem, red, false);
                    route_fused(L, slot == 0 && blk == 0, (float *)(smem + L.rlg), rsel, rwt, &rshg, &rbad);
                    if (s.iq2split) iq2_rows(s, slot, blk, rsel[slot], smem);
                    else iq2_rows_lane(s, slot, blk, rsel[slot], smem);
                    if (L.mctr && vb == L.pb0) fused_count(L, vb, false);
                    return;
                }
            }
            auto route = [&]() -> int {
                route_fused(L, slot == 0 && blk == 0, (float *)(smem + L.rlg), rsel, rwt, &rshg, &rbad);
                return rsel[slot];
            };
            const LateExpert<decltype(route)> late{route};
            if constexpr (TK >= 0) {
                mv_seg<TK < 0 ? OH_Q4_K : TK>(s, slot, blk, 0, smem, red, w, late);
            } else if constexpr (TK == OH_MV_Q4Q6) {
                if (s.type == OH_Q6_K) mv_seg<OH_Q6_K>(s, slot, blk, 0, smem, red, w, late);
                else mv_seg<OH_Q4_K>(s, slot, blk, 0, smem, red, w, late);
            } else {
                if (s.type == OH_Q6_K) mv_seg<OH_Q6_K>(s, slot, blk, 0, smem, red, w, late);
                else if (s.type == OH_Q8_0) mv_seg<OH_Q8_0>(s, slot, blk, 0, smem, red, w, late);
                else mv_seg<OH_Q4_K>(s, slot, blk, 0, smem, red, w, late);
            }
            if (L.mctr && vb == L.pb0) fused_count(L, vb, false);
            return;
        }
    } else if (L.route && L.tslots > 0) {
        // several tokens: a stacked-segment block routes its own token
        if (s.eidx) {
            if (!w.wait()) return;
            route_block(L, slot / L.tslots, blk == 0 && slot % L.tslots == 0, (float *)smem, rsel, rwt, &rshg,
                        &rbad, rcnt);
        }
    } else if (L.route) {
        if (!w.wait()) return;
        route_block(L, 0, vb == 0, (float *)smem, rsel, rwt, &rshg, &rbad, rcnt);
    } else if (s.eidx) {
        if (!w.wait()) return;                    // the routing comes from an earlier phase
    }
    const int expert = !s.eidx ? 0 : (L.route ? rsel[L.tslots > 0 ? slot % L.tslots : slot] : ldw<W::kGrid>(s.eidx + slot));
    if constexpr (TK >= 0) {
        mv_seg<TK < 0 ? OH_Q4_K : TK>(s, slot, blk, expert, smem, red, w);
        if (L.mctr && (s.mode == 2 || vb == L.pb0)) fused_count(L, vb, s.mode == 2);
    } else if constexpr (TK == OH_MV_Q4Q6) {
        if (s.type == OH_Q6_K) mv_seg<OH_Q6_K>(s, slot, blk, expert, smem, red, w);
        else mv_seg<OH_Q4_K>(s, slot, blk, expert, smem, red, w);
        if (L.mctr && (s.mode == 2 || vb == L.pb0)) fused_count(L, vb, s.mode == 2);
    } else if (s.type == OH_IQ2_XXS && s.iq2tree) {
        switch (s.in / 64) {
        case 64: iq2_tree<64>(s, slot, blk, expert, w); break;
        case 32: iq2_tree<32>(s, slot, blk, expert, w); break;
        case 16: iq2_tree<16>(s, slot, blk, expert, w); break;
        default: iq2_tree<8>(s, slot, blk, expert, w); break;
        }
    } else if (oh_qdot_can((uint32_t)s.type, s.in) && (s.xqs || s.pro != OH_PRO_Q8K)) {
        switch (s.type) {
        case OH_Q4_K: mv_seg<OH_Q4_K>(s, slot, blk, expert, smem, red, w); break;
        case OH_Q6_K: mv_seg<OH_Q6_K>(s, slot, blk, expert, smem, red, w); break;
        default: mv_seg<OH_Q8_0>(s, slot, blk, expert, smem, red, w); break;
        }
        // the router segments of a fused-router launch count themselves
        if (L.mctr && (s.mode == 2 || vb == L.pb0)) fused_count(L, vb, s.mode == 2);
    } else {
        if (!w.wait()) return;
        mv_prologue<W::kGrid>(s, slot, blk, smem, red, false);
        if (s.type == OH_IQ2_XXS) {
            if (s.iq2split) iq2_rows(s, slot, blk, expert, smem);
            else iq2_rows_lane(s, slot, blk, expert, smem);
            return;
        }
        const float *v = (const float *)(smem + mv_lds_v_off(s.in / 256));
        const int row = blk * 256 + tid_x();
        const int64_t row_base = (int64_t)expert * s.rows;
        if (row < s.rows) emit(s.y + (size_t)slot * s.ystride, s.mode, row, row_seq(s, row_base + row, v));
    }
}

// Fused MoE down projection and combine (src/ornith_rforward.c:375-409). A
// block owns 64/nb output rows; its waves take the slots (the k routed experts
// in routing order, then the shared expert) round-robin, MJ slots per wave at
// most, reducing one super-block per lane over those rows. Slot j's activation
// is Q8_K(h_j) (h_j = silu(gate) * up, emitted by the paired expert launch),
// formed in LDS by the block. Wave 0 then gives row r:
// x_r += (sum_j w_j * dot_j) + shg * dot_shared in the reference's order.
template <int T, int MJ, class W>
OH_DEV void down_body(const oh_mvdown &D, int vb, W &wt) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int HA = MJ == 1 ? 4 : 5;                   // h float4 per thread
    const int lane = lane_id(), wave = (tid_x() >> 6), nw = (int)(blockDim.x >> 6);
    const int tid = tid_x();
    const int nb = D.nb, in = D.in, ns = D.k + (D.sA ? 1 : 0), rps = 64 / nb;
    const int rl = lane / nb, sb = lane - rl * nb;
    const int sq = (nb * kAS + nb * 36 + 15) & ~15;     // one slot's Q8_K planes
    float *v = (float *)(smem + ns * sq);                // ns x in f32
    float *dots = v + ns * in;                           // ns x rps f32
    const int row0 = vb * rps;
    const int row = row0 + rl;
    const int rowc = row < D.rows ? (rl < rps ? row : row0) : D.rows - 1;
    // the routing, h and x come from earlier phases
    if (!wt.wait()) return;
    // the residual rows, routing weights and shared gate of the combine are
    // requested first (they are consumed last), then the activations (at most
    // HA float4 per thread), then the weights: vector loads complete in order
    __shared__ float cw[17];
    const bool comb = wave == 0 && lane < rps && row0 + lane < D.rows;
    const float xrow = comb ? ldc(D.x + row0 + lane) : 0.0f;
    if (tid < D.k) cw[tid] = ldc(D.w + tid);
    if (tid == 16) cw[16] = D.shg ? ldc(D.shg) : 1.0f;
    const int nf = ns * in / 4, bd = (int)blockDim.x;
    const bool hreg = nf <= HA * bd;
    float4 ha[HA];
    if (hreg) {
#pragma unroll
        for (int k = 0; k < HA; k++) {
            const int f = tid + bd * k < nf ? tid + bd * k : nf - 1;
            const int jj = 4 * f / in, e = 4 * f - jj * in;
            ha[k] = ldc4((const float4 *)((jj < D.k ? D.h + (size_t)jj * D.stride : D.hsh) + e));
        }
    }
    SB<T> r[MJ];
#pragma unroll
    for (int m = 0; m < MJ; m++) {
        const int j0 = wave + nw * m, j = j0 < ns ? j0 : ns - 1;
        const bool sh = j >= D.k;
        const WP wp = sh ? WP{D.sA, D.sB, D.sC} : WP{D.A, D.B, D.C};
        const int64_t rb = sh ? 0 : (int64_t)ldc(D.eidx + j) * D.rows;
        sb_load(r[m], wp, (rb + rowc) * nb + sb);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (hreg) {
#pragma unroll
        for (int k = 0; k < HA; k++)
            if (tid + bd * k < nf) ((float4 *)v)[tid + bd * k] = make_float4(ha[k].x, ha[k].y, ha[k].z, ha[k].w);
    } else {
        for (int i = tid; i < ns * in; i += bd) {
            const int jj = i / in, e = i - jj * in;
            v[i] = ldc((jj < D.k ? D.h + (size_t)jj * D.stride : D.hsh) + e);
        }
    }
    lds_barrier();
    for (int jj = wave; jj < ns; jj += nw) {          // wave jj quantises slot jj
        uint8_t *b = smem + (size_t)jj * sq;
        for (int q0 = 0; q0 < nb; q0 += 4)
            q8k_blocks<4>(v + (size_t)jj * in, q0, 1, nb, (int8_t *)b, (float *)(b + mv_lds_d_off(nb)),
                          (int16_t *)(b + mv_lds_bs_off(nb)), kAS);
    }
    lds_barrier();
#pragma unroll
    for (int m = 0; m < MJ; m++) {
        const int j = wave + nw * m;
        if (j < ns) {
            const uint8_t *b = smem + (size_t)j * sq;
            const float tw = sb_term(r[m], (const int8_t *)b + sb * kAS,
                                     (const int16_t *)(b + mv_lds_bs_off(nb)) + sb * 16,
                                     ((const float *)(b + mv_lds_d_off(nb)))[sb]);
            const bool live = rl < rps && row < D.rows;
            const float t = live ? tw : 0.0f;
            float acc = 0.0f;
            for (int i = 0; i < nb; i++) acc += shfl(t, rl * nb + i);
            if (rl < rps && sb == 0) dots[j * rps + rl] = acc;
        }
    }
    lds_barrier();
    if (comb) {
        float acc = 0.0f;
        for (int jj = 0; jj < D.k; jj++) acc += cw[jj] * dots[jj * rps + lane];
        if (D.sA) {
            const float so = dots[D.k * rps + lane];
            const float vv = D.shg ? so * cw[16] : so;
            acc += vv;
        }
        stc(D.x + row0 + lane, xrow + acc);
    }
}

// Fused down projection, narrow form: a block owns R = 64 / (4 nb) rows and
// every slot; wave w reduces slots 4w .. 4w + 3 (lane: slot 4w + lane / (R nb),
// row lane / nb % R, super-block lane % nb), so each block requests only its
// rows' weights (4x the blocks of down_body at the same activation work per
// block). Same arithmetic and orders as down_body.
template <int T>
OH_DEV void down_narrow(const oh_mvdown &D, int vb) {
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ float cw[17];
    constexpr int HA = 8;                                 // h float4 per thread
    const int lane = lane_id(), wave = __builtin_amdgcn_readfirstlane(tid_x() >> 6), tid = tid_x();
    const int nw = (int)(blockDim.x >> 6), bd = (int)blockDim.x;
    const int nb = D.nb, in = D.in, ns = D.k + (D.sA ? 1 : 0), R = 64 / (4 * nb);
    const int js = lane / (R * nb), rl = (lane / nb) % R, sb = lane % nb;
    const int j0 = 4 * wave + js, j = j0 < ns ? j0 : ns - 1;
    const bool act = j0 < ns;
    const int row0 = vb * R, row = row0 + rl;
    const int rowc = row < D.rows ? row : D.rows - 1;
    const int sq = (nb * kAS + nb * 36 + 15) & ~15;
    float *v = (float *)(smem + ns * sq);
    float *dots = v + ns * in;                            // [ns][R]
    const bool sh = j >= D.k;
    const int e = sh ? 0 : ldg(D.eidx + j);
    const bool comb = wave == 0 && lane < R && row0 + lane < D.rows;
    const float xrow = comb ? ldg(D.x + row0 + lane) : 0.0f;
    const float cwv = tid < D.k ? ldg(D.w + tid) : (tid == 16 && D.shg ? ldg(D.shg) : 1.0f);
    const int nf = ns * in / 4;
    const bool hreg = nf <= HA * bd;
    float4 ha[HA];
    if (hreg) {
#pragma unroll
        for (int k = 0; k < HA; k++) {
            const int f = tid + bd * k < nf ? tid + bd * k : nf - 1;
            const int jj = 4 * f / in, el = 4 * f - jj * in;
            ha[k] = ldg((const float4 *)((jj < D.k ? D.h + (size_t)jj * D.stride : D.hsh) + el));
        }
    }
    const WP wp = sh ? WP{D.sA, D.sB, D.sC} : WP{D.A, D.B, D.C};
    SB<T> r;
    sb_load(r, wp, (((int64_t)(sh ? 0 : e)) * D.rows + rowc) * nb + sb);
    __builtin_amdgcn_sched_barrier(0);
    if (tid <= 16) cw[tid] = cwv;
    if (hreg) {
#pragma unroll
        for (int k = 0; k < HA; k++)
            if (tid + bd * k < nf) ((float4 *)v)[tid + bd * k] = make_float4(ha[k].x, ha[k].y, ha[k].z, ha[k].w);
    } else {
        for (int i = tid; i < ns * in; i += bd) {
            const int jj = i / in, el = i - jj * in;
            v[i] = ldg((jj < D.k ? D.h + (size_t)jj * D.stride : D.hsh) + el);
        }
    }
    lds_barrier();
    for (int jj = wave; jj < ns; jj += nw) {              // wave jj % nw quantises slot jj
        uint8_t *b = smem + (size_t)jj * sq;
        if (nb == 2) {
            q8k_blocks<2>(v + (size_t)jj * in, 0, 1, nb, (int8_t *)b, (float *)(b + mv_lds_d_off(nb)),
                          (int16_t *)(b + mv_lds_bs_off(nb)), kAS);
        } else {
            for (int q0 = 0; q0 < nb; q0 += 4)
                q8k_blocks<4>(v + (size_t)jj * in, q0, 1, nb, (int8_t *)b, (float *)(b + mv_lds_d_off(nb)),
                              (int16_t *)(b + mv_lds_bs_off(nb)), kAS);
        }
    }
    lds_barrier();
    {
        const uint8_t *b = smem + (size_t)j * sq;
        const float tw = sb_term(r, (const int8_t *)b + sb * kAS, (const int16_t *)(b + mv_lds_bs_off(nb)) + sb * 16,
                                 ((const float *)(b + mv_lds_d_off(nb)))[sb]);
        const bool live = act && row < D.rows;
        const float t = live ? tw : 0.0f;
        const int base = lane - sb;
        float acc = 0.0f;
        for (int i = 0; i < nb; i++) acc += shfl(t, base + i);
        if (act && sb == 0) dots[j * R + rl] = acc;
    }
    lds_barrier();
    if (comb) {
        float acc = 0.0f;
        for (int jj = 0; jj < D.k; jj++) acc += cw[jj] * dots[jj * R + lane];
        if (D.sA) {
            const float so = dots[D.k * R + lane];
            const float vv = D.shg ? so * cw[16] : so;
            acc += vv;
        }
        stg(D.x + row0 + lane, xrow + acc);
    }
}

// Split form of the fused down projection for the step kernel, where a block
// has 4 waves: virtual block vb = (row group rg of 64/nb rows, slot group g);
// wave w reduces slot j = 4g + w over the row group (its activation Q8_K(h_j)
// formed in the wave's own LDS) and stores the dots with device-scope stores.
// After its stores complete the block counts itself in cnt[rg]; the last of
// the row group's blocks combines x_r += (sum_j w_j * dot_j) + shg * dot_shared
// in the reference's order and resets the counter. Same arithmetic as
// down_body.
template <int T, class W>
OH_DEV void down_split(const oh_mvdown &D, int vb, W &wt) {
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ int s_last;
    constexpr int HA = 4;                                 // h float4 per lane (in <= 1024)
    const int lane = lane_id(), wave = __builtin_amdgcn_readfirstlane(tid_x() >> 6);
    const int nb = D.nb, in = D.in, ns = D.k + (D.sA ? 1 : 0), rps = 64 / nb, ng = (ns + 3) / 4;
    const int rg = vb / ng, g = vb - rg * ng;
    const int j0 = 4 * g + wave;
    const bool act = j0 < ns;
    const int j = act ? j0 : ns - 1;
    const int rl = lane / nb, sb = lane - rl * nb;
    const int row0 = rg * rps, row = row0 + rl;
    const int rowc = row < D.rows ? (rl < rps ? row : row0) : D.rows - 1;
    const int wb = (in * 4 + nb * kAS + nb * 36 + 15) & ~15;   // one wave's LDS
    float *v = (float *)(smem + wave * wb);
    uint8_t *q = (uint8_t *)(v + in);
    if (!wt.wait()) return;
    // routing first, then this slot's activation, then (once the expert is
    // known) its weights: vector loads complete in order. (Requesting the
    // weights before the wait from a routing kept in LDS was measured slower:
    // the traffic lands in the gate/up phase still running.)
    const bool sh = j >= D.k;
    const int e = sh ? 0 : ldc(D.eidx + j);
    const int nf = in / 4;
    float4 ha[HA];
#pragma unroll
    for (int k = 0; k < HA; k++) {
        const int f = lane + 64 * k < nf ? lane + 64 * k : nf - 1;
        ha[k] = ldc4((const float4 *)(j < D.k ? D.h + (size_t)j * D.stride : D.hsh) + f);
    }
    const WP wp = sh ? WP{D.sA, D.sB, D.sC} : WP{D.A, D.B, D.C};
    SB<T> r;
    sb_load(r, wp, ((int64_t)e * D.rows + rowc) * nb + sb);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < HA; k++)
        if (lane + 64 * k < nf) ((float4 *)v)[lane + 64 * k] = make_float4(ha[k].x, ha[k].y, ha[k].z, ha[k].w);
    wave_lds_sync();
    for (int q0 = 0; q0 < nb; q0 += 4)
        q8k_blocks<4>(v, q0, 1, nb, (int8_t *)q, (float *)(q + mv_lds_d_off(nb)), (int16_t *)(q + mv_lds_bs_off(nb)), kAS);
    wave_lds_sync();
    const float tw = sb_term(r, (const int8_t *)q + sb * kAS, (const int16_t *)(q + mv_lds_bs_off(nb)) + sb * 16,
                             ((const float *)(q + mv_lds_d_off(nb)))[sb]);
    const bool live = act && rl < rps && row < D.rows;
    const float t = live ? tw : 0.0f;
    float acc = 0.0f;
    for (int i = 0; i < nb; i++) acc += shfl(t, rl * nb + i);
    if (live && sb == 0) stc(D.dots + (size_t)j * D.rows + row, acc);
    // count the block in its row group once every wave's stores completed
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid_x() == 0)
        s_last = __hip_atomic_fetch_add(D.cnt + rg, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == ng - 1;
    __syncthreads();
    if (!s_last) return;
    if (wave == 0 && lane < rps && row0 + lane < D.rows) {
        const int rr = row0 + lane;
        float dv[16], wv[16];
#pragma unroll
        for (int jj = 0; jj < 16; jj++) {
            const int jc = jj < ns ? jj : ns - 1;
            dv[jj] = ldc(D.dots + (size_t)jc * D.rows + rr);
            wv[jj] = jj < D.k ? ldc(D.w + jj) : 0.0f;
        }
        const float sg = D.shg ? ldc(D.shg) : 1.0f;
        const float xr = ldc(D.x + rr);
        float sum = 0.0f;
        for (int jj = 0; jj < D.k; jj++) sum += wv[jj] * dv[jj];
        if (D.sA) {
            const float so = dv[D.k];
            const float vv = D.shg ? so * sg : so;
            sum += vv;
        }
        stc(D.x + rr, xr + sum);
    }
    if (tid_x() == 0) stc(D.cnt + rg, 0);
}

// ---- batched matvec (prefill) --------------------------------------------------
// A block owns 4 wave steps of rows (64/nb rows each, one super-block per lane,
// its weights loaded once); the activation columns are staged in LDS tcol at
// a time (the matvec prologue's layout) and every wave reduces its
// super-blocks against each staged column: per (row, column) the matvec's dot
// (src/ornith_rforward.c:100-116 with Tn columns). Grid (row blocks, groups).
OH_HD inline int mvb_col_bytes(int nb) { return (nb * kAS + nb * 36 + 15) & ~15; }

template <int T>
OH_DEV void mvb_body(const oh_mvbatch &B) {
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ int scol[64];
    const int lane = lane_id(), wave = __builtin_amdgcn_readfirstlane(tid_x() >> 6), tid = tid_x();
    const int nb = B.nb, in = B.in, rps = 64 / nb, rl = lane / nb, sb = lane - rl * nb;
    const int g = B.list ? (int)blockIdx.y : 0;
    // dense: block y takes columns [y * cpb, (y + 1) * cpb)
    const int cbeg = B.list || !B.cpb ? 0 : (int)blockIdx.y * B.cpb;
    int ncol = B.list ? B.cnt[g] : B.ncol;
    if (!B.list && B.cpb) ncol = ncol < cbeg + B.cpb ? ncol : cbeg + B.cpb;
    if (ncol <= cbeg) return;
    const int r0 = ((int)blockIdx.x * 4 + wave) * rps, row = r0 + rl;
    const bool rlive = rl < rps && row < B.rows;
    const int rowc0 = rl < rps ? row : r0, rowc = rowc0 < B.rows ? rowc0 : B.rows - 1;
    const int64_t rbase = B.list ? (int64_t)g * B.rows : 0;
    const WP wp{B.A, B.B, B.C}, wp2{B.A2, B.B2, B.C2};
    SB<T> r, r2;
    sb_load(r, wp, (rbase + rowc) * nb + sb);
    if (B.pair) sb_load(r2, wp2, (rbase + rowc) * nb + sb);
    const int cs = mvb_col_bytes(nb), n16 = in / 16;
    for (int c0 = cbeg; c0 < ncol; c0 += B.tcol) {
        const int n = ncol - c0 < B.tcol ? ncol - c0 : B.tcol;
        __syncthreads();                              // the previous tile is consumed
        if (tid < n) scol[tid] = B.list ? ldg(B.list + (size_t)g * B.lstride + c0 + tid) : c0 + tid;
        __syncthreads();
        for (int i = tid; i < n * n16; i += 256) {
            const int c = i / n16, q = i - c * n16;
            const int a = scol[c] / B.adiv;
            ((int4 *)(smem + c * cs))[(q >> 4) * (kAS / 16) + (q & 15)] = ldg((const int4 *)(B.xqs + (size_t)a * in) + q);
        }
        for (int i = tid; i < n * 2 * nb; i += 256) {
            const int c = i / (2 * nb), q = i - c * 2 * nb;
            const int a = scol[c] / B.adiv;
            ((int4 *)(smem + c * cs + mv_lds_bs_off(nb)))[q] = ldg((const int4 *)(B.xbs + (size_t)a * nb * 16) + q);
        }
        for (int i = tid; i < n * nb; i += 256) {
            const int c = i / nb, q = i - c * nb;
            const int a = scol[c] / B.adiv;
            ((float *)(smem + c * cs + mv_lds_d_off(nb)))[q] = ldg(B.xd + (size_t)a * nb + q);
        }
        __syncthreads();
#pragma unroll 1
        for (int c = 0; c < n; c++) {
            const uint8_t *cb = smem + c * cs;
            const int8_t *aq = (const int8_t *)cb + sb * kAS;
            const int16_t *abs = (const int16_t *)(cb + mv_lds_bs_off(nb)) + sb * 16;
            const float yd = ((const float *)(cb + mv_lds_d_off(nb)))[sb];
            const float t1 = rlive ? sb_term(r, aq, abs, yd) : 0.0f;
            float acc = 0.0f;
            for (int i = 0; i < nb; i++) acc += shfl(t1, rl * nb + i);
            float out = acc;
            if (B.pair) {
                const float t2 = rlive ? sb_term(r2, aq, abs, yd) : 0.0f;
                float acc2 = 0.0f;
                for (int i = 0; i < nb; i++) acc2 += shfl(t2, rl * nb + i);
                out = ref_silu(acc) * acc2;
            }
            if (rlive && sb == 0) {
                float *yp = B.y + (size_t)scol[c] * B.ystride + row;
                if (B.mode == 1) stg(yp, ldg(yp) + out);
                else stg(yp, out);
            }
        }
    }
}

} // namespace

// The stand-alone kernels; a translation unit that only needs the bodies above
// (the persistent kernels) defines OH_BODIES_ONLY.
#ifndef OH_BODIES_ONLY
extern "C" __global__ void __launch_bounds__(256) oh_k_mv_q4k(oh_mvlaunch L) {
    NoWait w;
    mv_body<OH_Q4_K>(L, (int)blockIdx.x, w);
}
extern "C" __global__ void __launch_bounds__(256) oh_k_mv_q6k(oh_mvlaunch L) {
    NoWait w;
    mv_body<OH_Q6_K>(L, (int)blockIdx.x, w);
}
extern "C" __global__ void __launch_bounds__(256) oh_k_mv_q80(oh_mvlaunch L) {
    NoWait w;
    mv_body<OH_Q8_0>(L, (int)blockIdx.x, w);
}
extern "C" __global__ void __launch_bounds__(256) oh_k_mv_q4k6k(oh_mvlaunch L) {
    NoWait w;
    mv_body<OH_MV_Q4Q6>(L, (int)blockIdx.x, w);
}
// The descriptor is read in place from the kernel-argument segment (the
// parameter is its first and only explicit argument, at offset 0): with every
// segment form in one body, the by-value parameter indexed by the block's
// segment was otherwise copied to private memory at entry (2104 bytes per
// lane, 250 VGPRs; in place: no private memory, 168 VGPRs).
extern "C" __global__ void __launch_bounds__(256) oh_k_mv_mixed(oh_mvlaunch L0) {
    NoWait w;
    const oh_mvlaunch &L = *(const oh_mvlaunch *)__builtin_amdgcn_kernarg_segment_ptr();
    mv_body<-1>(L, (int)blockIdx.x, w);
}

// one wave per slot (blockDim = 64 * slots)
extern "C" __global__ void __launch_bounds__(256) oh_k_mv_down_narrow(oh_mvdown D) {
    switch (D.type) {
    case OH_Q4_K: down_narrow<OH_Q4_K>(D, (int)blockIdx.x); break;
    case OH_Q6_K: down_narrow<OH_Q6_K>(D, (int)blockIdx.x); break;
    default: down_narrow<OH_Q8_0>(D, (int)blockIdx.x); break;
    }
}
extern "C" __global__ void __launch_bounds__(640) oh_k_mv_down(oh_mvdown D0) {
    NoWait w;
    // token blockIdx.y of a batch (0: the only token)
    oh_mvdown D = D0;
    const int t = (int)blockIdx.y;
    D.h += t * D0.hts;
    D.hsh += t * D0.hsts;
    D.x += t * D0.xts;
    D.eidx += (size_t)t * D0.k;
    D.w += (size_t)t * D0.k;
    if (D0.shg) D.shg += t;
    switch (D.type) {
    case OH_Q4_K: down_body<OH_Q4_K, 1>(D, (int)blockIdx.x, w); break;
    case OH_Q6_K: down_body<OH_Q6_K, 1>(D, (int)blockIdx.x, w); break;
    default: down_body<OH_Q8_0, 1>(D, (int)blockIdx.x, w); break;
    }
}

// ---- Q8_K quantisation (optionally fused with RMSNorm) ----------------------
// One block of 256 threads per vector of n <= 8192 elements (n % 256 == 0).
// norm_w != nullptr: x is first RMS-normalised (src/ornith_tensor.c:100-106):
// sum of squares in double (tree-ordered), inv = (float)(1/sqrt(ss/n+eps)),
// xn_i = x_i * inv * w_i. Then each 256-block is quantised exactly as
// qdot_quantize_row_q8_K (src/ornith_qdot.c:32-62).
extern "C" __global__ void __launch_bounds__(256)
oh_k_rmsnorm_q8k(const float *x, const float *norm_w, float eps, int n,
                 float *xn_out, int8_t *qs, float *d, int16_t *bs) {
    __shared__ float v[8192];
    __shared__ double red[4];
    const int tid = tid_x(), wave = tid >> 6;
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
    const int vec = (int)blockIdx.x, tid = tid_x(), wave = tid >> 6;
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
    for (int64_t e = (int64_t)blockIdx.x * 256 + tid_x(); e < n; e += (int64_t)gridDim.x * 256) {
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
                const uint8_t q = A[oh_a_off(OH_Q4_K, bi, 32 * (j / 2) + l)];
                int sc, mn;
                q4k_sm(hdr, j, sc, mn);
                const float dd = h2f((uint16_t)(hdr.x & 0xffffu)), dmin = h2f((uint16_t)(hdr.x >> 16));
                const float d1 = dd * sc, m1 = dmin * mn;
                y = d1 * (float)((j & 1) ? (q >> 4) : (q & 15)) - m1;
            } else if (type == OH_Q6_K) {
                const int hh = k / 128, kk = k % 128, qd = kk / 32, l = kk % 32;
                const uint8_t ql = A[oh_a_off(OH_Q6_K, bi, 64 * hh + l + 32 * (qd & 1))];
                const uint8_t qh = A[oh_a_off(OH_Q6_K, bi, 128 + 32 * hh + l)];
                const int lo = (qd < 2) ? (ql & 15) : (ql >> 4);
                const int q = (lo | (((qh >> (2 * qd)) & 3) << 4)) - 32;
                const int8_t sc = (int8_t)B[bi * 16 + 8 * hh + l / 16 + 2 * qd];
                const float dd = h2f(*(const uint16_t *)(C + bi * 2));
                y = dd * (float)sc * (float)q;
            } else if (type == OH_Q8_0) {
                const int sbk = k / 32;
                const int8_t q = (int8_t)A[oh_a_off(OH_Q8_0, bi, k)];
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

extern "C" __global__ void __launch_bounds__(256) oh_k_mvb_q4k(oh_mvbatch B) { mvb_body<OH_Q4_K>(B); }
extern "C" __global__ void __launch_bounds__(256) oh_k_mvb_q6k(oh_mvbatch B) { mvb_body<OH_Q6_K>(B); }
extern "C" __global__ void __launch_bounds__(256) oh_k_mvb_q80(oh_mvbatch B) { mvb_body<OH_Q8_0>(B); }

// Q8_K (optionally after RMSNorm) of `rows` vectors of n elements, one block
// per vector; the same arithmetic as oh_k_rmsnorm_q8k (and the matvec's
// RMSNorm prologue). xn_out (optional) receives the normalised f32 vectors.
// Dynamic LDS: n floats (the launcher's), so narrow rows keep more blocks
// resident; the norm weights are requested with the row.
extern "C" __global__ void __launch_bounds__(256)
oh_k_norm_q8k_rows(const float *x, const float *norm_w, float eps, int n, float *xn_out, int8_t *qs, float *d,
                   int16_t *bs, int8_t *bp, int swiglu) {
    extern __shared__ __align__(16) float v[];
    __shared__ double red[4];
    const size_t r = blockIdx.x;
    const int tid = tid_x(), wave = tid >> 6, nqb = n / 256;
    float wn[32];                                   // this thread's norm weights (n <= 8192)
    if (norm_w) {
#pragma unroll
        for (int k = 0; k < 32; k++) {
            const int i = tid + 256 * k;
            wn[k] = i < n ? ldg(norm_w + i) : 0.0f;
        }
    }
    // (unrolled, so that a thread's row loads are requested together)
    if (swiglu) {
        // rows of [gate | up] (2n): v = silu(gate) * up, the paired matvec's h
        const float *xr = x + r * 2 * n;
#pragma unroll 8
        for (int i = tid; i < n; i += 256) v[i] = ref_silu(ldg(xr + i)) * ldg(xr + n + i);
    } else {
        const float *xr = x + r * n;
#pragma unroll 8
        for (int i = tid; i < n; i += 256) v[i] = ldg(xr + i);
    }
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
#pragma unroll
        for (int k = 0; k < 32; k++) {
            const int i = tid + 256 * k;
            if (i < n) v[i] = v[i] * inv * wn[k];
        }
        __syncthreads();
    }
    if (xn_out) for (int i = tid; i < n; i += 256) stg(xn_out + r * n + i, v[i]);
    for (int qb = wave; qb < nqb; qb += 4)
        q8k_block_from_lds(v, qb, qs + r * n, d + r * nqb, bs + r * nqb * 16, 256, bp ? bp + r * nqb * 16 : nullptr);
}

#endif // OH_BODIES_ONLY
