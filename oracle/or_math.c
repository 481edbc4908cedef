/* or_math.c - oracle restatement of the f32 helpers, the matvec dispatch, the
 * attention core and the MoE router (TEST INFRASTRUCTURE, see oracle.h).
 *
 * References: src/ornith_tensor.c:100-178, src/ornith_rforward.c:100-196,
 * src/ornith_attn.c:62-397, src/ornith_moe.c:8-30.
 */
#include "oracle.h"
#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <pthread.h>

void orc_seterr(const char *fmt, ...);

/* ---- f32 helpers (src/ornith_tensor.c) ----------------------------------- */

/* sum of squares in double, one rounding to f32 for the inverse rms
 * (src/ornith_tensor.c:100-106) */
void orc_rmsnorm(const float *x, const float *w, float *out, int n, float eps) {
    double ss = 0.0;
    for (int i = 0; i < n; i++) ss += (double)x[i] * x[i];
    const float inv = (float)(1.0 / sqrt(ss / (double)n + (double)eps));
    for (int i = 0; i < n; i++) out[i] = x[i] * inv * (w ? w[i] : 1.0f);
}

/* max-shifted exponentials, double-precision sum (src/ornith_tensor.c:108-115) */
void orc_softmax(float *x, int n) {
    float mx = x[0];
    for (int i = 1; i < n; i++) if (x[i] > mx) mx = x[i];
    double sum = 0.0;
    for (int i = 0; i < n; i++) { x[i] = expf(x[i] - mx); sum += x[i]; }
    const float inv = (float)(1.0 / sum);
    for (int i = 0; i < n; i++) x[i] *= inv;
}

float orc_sigmoid(float x)  { return 1.0f / (1.0f + expf(-x)); }
float orc_silu(float x)     { return x * orc_sigmoid(x); }
float orc_softplus(float x) { return x > 20.0f ? x : log1pf(expf(x)); }

/* strictly sequential f32 accumulation (src/ornith_tensor.c:143-147) */
float orc_dot(const float *a, const float *b, int n) {
    float acc = 0.0f;
    for (int i = 0; i < n; i++) acc += a[i] * b[i];
    return acc;
}

void orc_l2norm_eps(const float *x, float *out, int n, float eps) {
    double ss = 0.0;
    for (int i = 0; i < n; i++) ss += (double)x[i] * x[i];
    const float inv = (float)(1.0 / sqrt(ss + (double)eps));
    for (int i = 0; i < n; i++) out[i] = x[i] * inv;
}

/* NeoX rotate-half over the first `rot` dims (src/ornith_tensor.c:167-178) */
void orc_rope_partial(float *v, int hd, int rot, int pos, float theta) {
    if (rot <= 0 || rot > hd) rot = hd;
    const int half = rot / 2;
    for (int i = 0; i < half; i++) {
        const float freq = powf(theta, -2.0f * (float)i / (float)rot);
        const float ang = (float)pos * freq;
        const float c = cosf(ang), s = sinf(ang);
        const float a = v[i], b = v[i + half];
        v[i] = a * c - b * s;
        v[i + half] = a * s + b * c;
    }
}

/* ---- matvec dispatch (src/ornith_rforward.c:100-196) ---------------------- */
typedef struct {
    uint32_t type; const uint8_t *W; size_t rb; int in, o0, o1;
    const float *x; const orc_q8k *xq; float *y;
} mv_part;

static void *mv_work(void *arg) {
    mv_part *p = arg;
    if (p->xq) {
        for (int o = p->o0; o < p->o1; o++)
            p->y[o] = orc_qdot(p->type, p->in, p->W + (size_t)o * p->rb, p->xq);
        return NULL;
    }
    float *row = p->type == ORC_F32 ? NULL : malloc((size_t)p->in * sizeof(float));
    for (int o = p->o0; o < p->o1; o++) {
        const float *w;
        if (!row) w = (const float *)(p->W + (size_t)o * p->rb);
        else { orc_dequantize(p->type, p->W + (size_t)o * p->rb, row, (size_t)p->in); w = row; }
        p->y[o] = orc_dot(w, p->x, p->in);
    }
    free(row);
    return NULL;
}

void orc_matvec(uint32_t type, const void *W, int in, int out,
                const float *x, float *y, int no_qdot, int nthreads) {
    orc_q8k *xq = NULL;
    if (!no_qdot && orc_qdot_can(type, in)) {
        xq = malloc((size_t)(in / 256) * sizeof(orc_q8k));
        orc_quantize_q8k(x, xq, in);
    }
    int nth = nthreads < 1 ? 1 : (nthreads > 64 ? 64 : nthreads);
    if (nth > out) nth = out;
    const int per = (out + nth - 1) / nth;
    mv_part parts[64]; pthread_t th[64];
    int np = 0;
    for (int t = 0; t < nth; t++) {
        const int o0 = t * per;
        if (o0 >= out) break;
        const int o1 = o0 + per > out ? out : o0 + per;
        parts[np++] = (mv_part){ type, W, orc_row_bytes(type, (size_t)in), in, o0, o1, x, xq, y };
    }
    if (np == 1) mv_work(&parts[0]);
    else {
        for (int t = 0; t < np; t++) pthread_create(&th[t], NULL, mv_work, &parts[t]);
        for (int t = 0; t < np; t++) pthread_join(th[t], NULL);
    }
    free(xq);
}

/* ---- KV cache + GQA step (src/ornith_attn.c:20-149) ----------------------- */
int orc_kv_init(orc_kv *c, int cap, int nkv, int hd, int quantized) {
    memset(c, 0, sizeof *c);
    c->capacity = cap; c->n_kv_heads = nkv; c->head_dim = hd; c->quantized = quantized ? 1 : 0;
    const size_t per = (size_t)cap * nkv * hd, scl = (size_t)cap * nkv;
    if (c->quantized) {
        c->Kq = calloc(per, 1); c->Vq = calloc(per, 1);
        c->Ks = calloc(scl, 4); c->Vs = calloc(scl, 4);
        if (!c->Kq || !c->Vq || !c->Ks || !c->Vs) { orc_kv_free(c); return ORC_ERR_OOM; }
    } else {
        c->K = calloc(per, 4); c->V = calloc(per, 4);
        if (!c->K || !c->V) { orc_kv_free(c); return ORC_ERR_OOM; }
    }
    return ORC_OK;
}
void orc_kv_free(orc_kv *c) {
    free(c->K); free(c->V); free(c->Kq); free(c->Vq); free(c->Ks); free(c->Vs);
    memset(c, 0, sizeof *c);
}

/* symmetric int8: scale = amax/127, code = rint(x*127/amax) in [-127,127]
 * (src/ornith_attn.c:65-77) */
float orc_kv_quant_vec(const float *x, int n, int8_t *q) {
    float amax = 0.0f;
    for (int i = 0; i < n; i++) { const float a = fabsf(x[i]); if (a > amax) amax = a; }
    if (amax == 0.0f) { memset(q, 0, (size_t)n); return 0.0f; }
    const float scale = amax / 127.0f, inv = 127.0f / amax;
    for (int i = 0; i < n; i++) {
        long v = lrintf(x[i] * inv);
        q[i] = (int8_t)(v > 127 ? 127 : (v < -127 ? -127 : v));
    }
    return scale;
}

void orc_gqa_step(orc_kv *c, const float *q, const float *k, const float *v,
                  int n_heads, float *out, float scale) {
    const int hd = c->head_dim, nkv = c->n_kv_heads;
    if (scale <= 0.0f) scale = 1.0f / sqrtf((float)hd);
    if (c->len >= c->capacity) return;
    const int pos = c->len;
    for (int h = 0; h < nkv; h++) {
        const size_t off = (size_t)pos * nkv + h;
        if (c->quantized) {
            c->Ks[off] = orc_kv_quant_vec(k + (size_t)h * hd, hd, c->Kq + off * hd);
            c->Vs[off] = orc_kv_quant_vec(v + (size_t)h * hd, hd, c->Vq + off * hd);
        } else {
            memcpy(c->K + off * hd, k + (size_t)h * hd, (size_t)hd * 4);
            memcpy(c->V + off * hd, v + (size_t)h * hd, (size_t)hd * 4);
        }
    }
    c->len++;
    orc_gqa_attend(c, q, n_heads, out, scale);
}

/* the attention half of orc_gqa_step: every head over the c->len cached
 * positions (src/ornith_attn.c:111-149) */
void orc_gqa_attend(const orc_kv *c, const float *q, int n_heads, float *out, float scale) {
    const int hd = c->head_dim, nkv = c->n_kv_heads;
    if (scale <= 0.0f) scale = 1.0f / sqrtf((float)hd);
    const int T = c->len, group = n_heads / nkv;
    if (T <= 0) return;
    float *p = malloc((size_t)T * sizeof(float));
    for (int h = 0; h < n_heads; h++) {
        const int kvh = h / group;
        const float *qh = q + (size_t)h * hd;
        for (int t = 0; t < T; t++) {
            const size_t off = (size_t)t * nkv + kvh;
            if (c->quantized) {
                float s = 0.0f;
                if (c->Ks[off] != 0.0f) {
                    const int8_t *kc = c->Kq + off * hd;
                    for (int i = 0; i < hd; i++) s += qh[i] * (float)kc[i];
                    s = s * c->Ks[off];
                }
                p[t] = s * scale;
            } else {
                p[t] = orc_dot(qh, c->K + off * hd, hd) * scale;
            }
        }
        orc_softmax(p, T);
        float *oh = out + (size_t)h * hd;
        memset(oh, 0, (size_t)hd * 4);
        for (int t = 0; t < T; t++) {
            const size_t off = (size_t)t * nkv + kvh;
            if (c->quantized) {
                const float sv = p[t] * c->Vs[off];
                if (sv == 0.0f) continue;
                const int8_t *vc = c->Vq + off * hd;
                for (int i = 0; i < hd; i++) oh[i] += sv * (float)vc[i];
            } else {
                const float *vt = c->V + off * hd;
                for (int i = 0; i < hd; i++) oh[i] += p[t] * vt[i];
            }
        }
    }
    free(p);
}

/* ---- gated delta rule (src/ornith_attn.c:198-349) -------------------------
 * S is [dv, dk] row-major. Step: S *= alpha; per row r: u = beta*(v_r - S_r.k);
 * S_r += u k; o_r = S_r.q. */
void orc_delta_step(float *S, int dk, int dv, const float *q, const float *k,
                    const float *v, float alpha, float beta, float *o) {
    for (int i = 0; i < dk * dv; i++) S[i] *= alpha;
    for (int r = 0; r < dv; r++) {
        float *Sr = S + (size_t)r * dk;
        const float u = beta * (v[r] - orc_dot(Sr, k, dk));
        for (int c = 0; c < dk; c++) Sr[c] += u * k[c];
        o[r] = orc_dot(Sr, q, dk);
    }
}

/* One chunk of the chunked scan: all S_in projections first, then forward
 * substitution of (I + M) U = T with decay ratios accumulated as bounded
 * sub-products, outputs, and the state update (src/ornith_attn.c:244-335). */
static void delta_chunk(float *S, int dk, int dv, const float *Q, const float *K,
                        const float *V, const float *al, const float *be, int C,
                        float *O) {
    float *p = malloc((size_t)C * 4);
    float *Sk = malloc((size_t)C * dv * 4), *Sq = malloc((size_t)C * dv * 4);
    float *U = malloc((size_t)C * dv * 4);
    float *kk = malloc((size_t)C * C * 4), *kq = malloc((size_t)C * C * 4);
    for (int i = 0; i < C; i++) p[i] = i == 0 ? al[0] : p[i - 1] * al[i];
    for (int i = 0; i < C; i++) {
        const float *ki = K + (size_t)i * dk, *qi = Q + (size_t)i * dk;
        for (int r = 0; r < dv; r++) {
            Sk[(size_t)i * dv + r] = orc_dot(S + (size_t)r * dk, ki, dk);
            Sq[(size_t)i * dv + r] = orc_dot(S + (size_t)r * dk, qi, dk);
        }
        for (int j = 0; j < C; j++) {
            kk[(size_t)i * C + j] = orc_dot(K + (size_t)j * dk, ki, dk);
            kq[(size_t)i * C + j] = orc_dot(K + (size_t)j * dk, qi, dk);
        }
    }
    for (int i = 0; i < C; i++) {
        const float bi = be[i], pi = p[i];
        float *ui = U + (size_t)i * dv;
        for (int r = 0; r < dv; r++)
            ui[r] = bi * V[(size_t)i * dv + r] - bi * pi * Sk[(size_t)i * dv + r];
        float ratio = 1.0f;
        for (int j = i - 1; j >= 0; j--) {
            ratio *= al[j + 1];
            const float m = bi * ratio * kk[(size_t)i * C + j];
            if (m == 0.0f) continue;
            const float *uj = U + (size_t)j * dv;
            for (int r = 0; r < dv; r++) ui[r] -= m * uj[r];
        }
    }
    for (int i = 0; i < C; i++) {
        float *oi = O + (size_t)i * dv;
        for (int r = 0; r < dv; r++) oi[r] = p[i] * Sq[(size_t)i * dv + r];
        const float wd = kq[(size_t)i * C + i];
        for (int r = 0; r < dv; r++) oi[r] += wd * U[(size_t)i * dv + r];
        float ratio = 1.0f;
        for (int j = i - 1; j >= 0; j--) {
            ratio *= al[j + 1];
            const float w = ratio * kq[(size_t)i * C + j];
            for (int r = 0; r < dv; r++) oi[r] += w * U[(size_t)j * dv + r];
        }
    }
    const float pc = p[C - 1];
    for (int i = 0; i < dk * dv; i++) S[i] *= pc;
    float ratio = 1.0f;
    for (int j = C - 1; j >= 0; j--) {
        const float *uj = U + (size_t)j * dv, *kj = K + (size_t)j * dk;
        for (int r = 0; r < dv; r++) {
            const float ur = ratio * uj[r];
            if (ur == 0.0f) continue;
            float *Sr = S + (size_t)r * dk;
            for (int c = 0; c < dk; c++) Sr[c] += ur * kj[c];
        }
        ratio *= al[j];
    }
    free(p); free(Sk); free(Sq); free(U); free(kk); free(kq);
}

void orc_delta_prefill(float *S, int dk, int dv, const float *Q, const float *K,
                       const float *V, const float *alpha, const float *beta,
                       int T, int chunk, float *O) {
    if (chunk < 1) chunk = 1;
    if (chunk > T) chunk = T;
    for (int c0 = 0; c0 < T; c0 += chunk) {
        const int C = c0 + chunk <= T ? chunk : T - c0;
        delta_chunk(S, dk, dv, Q + (size_t)c0 * dk, K + (size_t)c0 * dk,
                    V + (size_t)c0 * dv, alpha + c0, beta + c0, C, O + (size_t)c0 * dv);
    }
}

/* depthwise causal conv over a window of the last K-1 inputs, oldest first:
 * buf[j*C + c]; weight w[c*K + j], j = K-1 weights the current input
 * (src/ornith_attn.c:370-388). */
void orc_conv_step(float *buf, int K, int C, const float *x, const float *w,
                   const float *bias, float *out) {
    for (int c = 0; c < C; c++) {
        float acc = bias ? bias[c] : 0.0f;
        const float *wc = w + (size_t)c * K;
        for (int j = 0; j < K - 1; j++) acc += wc[j] * buf[(size_t)j * C + c];
        acc += wc[K - 1] * x[c];
        out[c] = acc;
    }
    if (K >= 2) {
        memmove(buf, buf + C, (size_t)(K - 2) * C * 4);
        memcpy(buf + (size_t)(K - 2) * C, x, (size_t)C * 4);
    }
}

/* ---- router (src/ornith_moe.c:8-30) ----------------------------------------
 * top-k by repeated ascending scans with strict '>' (ties go to the lower
 * index), then softmax over the selected logits with a float sum. */
void orc_moe_route(const float *logits, int ne, int k, int *idx, float *w) {
    unsigned char *taken = calloc((size_t)ne, 1);
    for (int s = 0; s < k; s++) {
        int best = -1; float bv = -INFINITY;
        for (int e = 0; e < ne; e++)
            if (!taken[e] && logits[e] > bv) { bv = logits[e]; best = e; }
        idx[s] = best; taken[best] = 1;
    }
    free(taken);
    float mx = logits[idx[0]];
    for (int s = 1; s < k; s++) if (logits[idx[s]] > mx) mx = logits[idx[s]];
    float sum = 0.0f;
    for (int s = 0; s < k; s++) { w[s] = expf(logits[idx[s]] - mx); sum += w[s]; }
    for (int s = 0; s < k; s++) w[s] /= sum;
}

/* ---- deterministic synthetic data -------------------------------------------
 * splitmix64 is counter-based: output n of the stream seeded with key is
 * mix(key + n*gamma). Element i of a Gaussian stream sums the twelve 16-bit
 * lanes of outputs 3i+1..3i+3 (Irwin-Hall(12) ~ N(0,1)), an exact integer,
 * then scales it once; the same bits come out of any IEEE machine. */
#define GAMMA 0x9E3779B97F4A7C15ull
static inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
uint64_t orc_stream_key(uint64_t seed, const char *name) {
    uint64_t h = 0xcbf29ce484222325ull;
    for (const unsigned char *s = (const unsigned char *)name; *s; s++) { h ^= *s; h *= 0x100000001b3ull; }
    return h ^ (seed * GAMMA);
}
void orc_fill_gauss(uint64_t key, float sigma, float *dst, size_t n, size_t first) {
    const float c = sigma / 131072.0f;
    for (size_t i = 0; i < n; i++) {
        const uint64_t e = first + i;
        int64_t s = 0;
        for (int k = 1; k <= 3; k++) {
            const uint64_t r = mix64(key + (3 * e + (uint64_t)k) * GAMMA);
            s += (int64_t)(r & 0xffff) + (int64_t)((r >> 16) & 0xffff) +
                 (int64_t)((r >> 32) & 0xffff) + (int64_t)(r >> 48);
        }
        dst[i] = (float)(2 * s - 786420) * c;
    }
}
void orc_fill_uniform(uint64_t key, float lo, float hi, float *dst, size_t n, size_t first) {
    for (size_t i = 0; i < n; i++) {
        const uint64_t r = mix64(key + (first + i + 1) * GAMMA);
        const float f = (float)(uint32_t)(r >> 40) / 16777216.0f;
        dst[i] = lo + (hi - lo) * f;
    }
}
void orc_fill_ids(uint64_t key, int32_t v, int32_t *dst, size_t n) {
    for (size_t i = 0; i < n; i++)
        dst[i] = (int32_t)(mix64(key + (i + 1) * GAMMA) % (uint64_t)v);
}
