/* or_model.c - oracle restatement of the real-weight forward, sessions and
 * greedy generation (TEST INFRASTRUCTURE, see oracle.h).
 *
 * Reference: src/ornith_rforward.c. Layer math :300-503, prefill :513-682,
 * token step :686-706, shape inference :719-816, sessions :908-982.
 */
#include "oracle.h"
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

void orc_seterr(const char *fmt, ...);
const void *orc_gguf_kv(const orc_gguf *g, const char *key, uint32_t *vt, size_t *len);

typedef struct {
    const orc_tensor *attn_norm, *post_norm;
    const orc_tensor *q, *k, *v, *q_norm, *k_norm, *o;                  /* full   */
    const orc_tensor *qkv, *conv, *ssm_a, *dt_bias, *ssm_norm, *alpha,
                     *beta, *gate, *ssm_out;                             /* linear */
    const orc_tensor *router, *gate_exps, *up_exps, *down_exps,
                     *gate_sh, *up_sh, *down_sh, *gate_inp_sh;           /* moe    */
    const orc_tensor *ffn_gate, *ffn_up, *ffn_down;                      /* dense  */
} orc_layer;

struct orc_model {
    orc_gguf *g;
    orc_arch a;
    orc_layer *L;
    const orc_tensor *embd, *out_norm, *lm_head;
    int nthreads, no_qdot;
};

static const orc_tensor *blk(const orc_gguf *g, int l, const char *sfx) {
    char nm[160]; snprintf(nm, sizeof nm, "blk.%d.%s", l, sfx);
    return orc_gguf_find(g, nm);
}
static uint32_t meta_u32(const orc_gguf *g, const char *key, uint32_t def) {
    uint32_t vt; size_t len; const uint8_t *p = orc_gguf_kv(g, key, &vt, &len);
    if (p && (vt == 4 || vt == 5) && len >= 4) { uint32_t v; memcpy(&v, p, 4); return v; }
    return def;
}
static float meta_f32(const orc_gguf *g, const char *key, float def) {
    uint32_t vt; size_t len; const uint8_t *p = orc_gguf_kv(g, key, &vt, &len);
    if (p && vt == 6 && len >= 4) { float v; memcpy(&v, p, 4); return v; }
    return def;
}
static int is_full(const orc_arch *a, int l) {
    return a->full_interval > 0 && l % a->full_interval == a->full_interval - 1;
}

int orc_model_load(const char *path, orc_model **out) {
    *out = NULL;
    orc_gguf *g;
    int st = orc_gguf_load(path, &g);
    if (st) return st;
    orc_model *m = calloc(1, sizeof *m);
    m->g = g;
    orc_arch *a = &m->a;
    char pfx[64] = "qwen35";
    { uint32_t vt; size_t len; const uint8_t *p = orc_gguf_kv(g, "general.architecture", &vt, &len);
      if (p && vt == 8 && len >= 8) { uint64_t n; memcpy(&n, p, 8);
          if (n < sizeof pfx && n <= len - 8) { memcpy(pfx, p + 8, n); pfx[n] = 0; } } }
    char key[160];
#define MK(s) (snprintf(key, sizeof key, "%s.%s", pfx, s), key)
    m->embd = orc_gguf_find(g, "token_embd.weight");
    a->hidden = m->embd ? (int)m->embd->dims[0] : (int)meta_u32(g, MK("embedding_length"), 4096);
    a->vocab = m->embd ? (int)m->embd->dims[1] : 248320;
    int n = 0;
    while (blk(g, n, "attn_norm.weight")) n++;
    a->n_layers = n ? n : (int)meta_u32(g, MK("block_count"), 32);
    int ff = -1;
    for (int i = 0; i < a->n_layers; i++) if (blk(g, i, "attn_q.weight")) { ff = i; break; }
    a->full_interval = ff >= 0 ? ff + 1 : (int)meta_u32(g, MK("full_attention_interval"), 4);
    a->rope_theta = meta_f32(g, MK("rope.freq_base"), 1e7f);
    a->eps = meta_f32(g, MK("attention.layer_norm_rms_epsilon"), 1e-6f);
    a->rope_dim = (int)meta_u32(g, MK("rope.dimension_count"), 64);
    {
        const int fl = a->full_interval - 1;
        const orc_tensor *qn = blk(g, fl, "attn_q_norm.weight"), *q = blk(g, fl, "attn_q.weight"),
                         *k = blk(g, fl, "attn_k.weight");
        a->hd = qn ? (int)qn->dims[0] : 256;
        const int qout = q ? (int)q->dims[1] : a->hd * 16;
        a->nh = (qout / 2) / a->hd;
        a->nkv = k ? (int)k->dims[1] / a->hd : 4;
    }
    {
        int l0 = 0;
        while (l0 < a->n_layers && is_full(a, l0)) l0++;
        const orc_tensor *sa = blk(g, l0, "ssm_a"), *sn = blk(g, l0, "ssm_norm.weight"),
                         *qkv = blk(g, l0, "attn_qkv.weight"), *cv = blk(g, l0, "ssm_conv1d.weight");
        a->nv = sa ? (int)sa->dims[0] : 32;
        a->dv = sn ? (int)sn->dims[0] : 128;
        a->dk = a->dv;
        a->conv_k = cv ? (int)cv->dims[0] : 4;
        const int cc = qkv ? (int)qkv->dims[1] : 8192;
        const int qd = (cc - a->nv * a->dv) / 2;
        a->nk = a->dk ? qd / a->dk : 16;
    }
    const orc_tensor *ge0 = blk(g, 0, "ffn_gate_exps.weight");
    if (ge0) {
        a->ne = (int)ge0->dims[2];
        a->moe_inter = (int)ge0->dims[1];
        a->top_k = (int)meta_u32(g, MK("expert_used_count"), 8);
        const orc_tensor *sh = blk(g, 0, "ffn_gate_shexp.weight");
        a->shared_inter = sh ? (int)sh->dims[1] : 0;
    } else {
        const orc_tensor *fg = blk(g, 0, "ffn_gate.weight");
        a->shared_inter = fg ? (int)fg->dims[1] : (int)meta_u32(g, MK("feed_forward_length"), 12288);
    }
#undef MK
    {   /* the tokenizer needs tokenizer.ggml.tokens (src/ornith_tokenizer.c:189-214) */
        uint32_t vt; size_t len;
        if (!orc_gguf_kv(g, "tokenizer.ggml.tokens", &vt, &len)) {
            orc_model_free(m); orc_seterr("no tokenizer.ggml.tokens"); return ORC_ERR_FORMAT;
        }
        const uint8_t *p = orc_gguf_kv(g, "tokenizer.ggml.eos_token_id", &vt, &len);
        a->eos = -1;
        if (p && len >= 4) memcpy(&a->eos, p, 4);
    }
    m->out_norm = orc_gguf_find(g, "output_norm.weight");
    m->lm_head = orc_gguf_find(g, "output.weight");
    m->L = calloc((size_t)a->n_layers, sizeof(orc_layer));
    for (int l = 0; l < a->n_layers; l++) {
        orc_layer *y = &m->L[l];
        y->attn_norm = blk(g, l, "attn_norm.weight");
        y->post_norm = blk(g, l, "post_attention_norm.weight");
        y->q = blk(g, l, "attn_q.weight"); y->k = blk(g, l, "attn_k.weight");
        y->v = blk(g, l, "attn_v.weight"); y->o = blk(g, l, "attn_output.weight");
        y->q_norm = blk(g, l, "attn_q_norm.weight"); y->k_norm = blk(g, l, "attn_k_norm.weight");
        y->qkv = blk(g, l, "attn_qkv.weight"); y->conv = blk(g, l, "ssm_conv1d.weight");
        y->ssm_a = blk(g, l, "ssm_a"); y->dt_bias = blk(g, l, "ssm_dt.bias");
        y->ssm_norm = blk(g, l, "ssm_norm.weight"); y->alpha = blk(g, l, "ssm_alpha.weight");
        y->beta = blk(g, l, "ssm_beta.weight"); y->gate = blk(g, l, "attn_gate.weight");
        y->ssm_out = blk(g, l, "ssm_out.weight");
        y->router = blk(g, l, "ffn_gate_inp.weight");
        y->gate_exps = blk(g, l, "ffn_gate_exps.weight"); y->up_exps = blk(g, l, "ffn_up_exps.weight");
        y->down_exps = blk(g, l, "ffn_down_exps.weight");
        y->gate_sh = blk(g, l, "ffn_gate_shexp.weight"); y->up_sh = blk(g, l, "ffn_up_shexp.weight");
        y->down_sh = blk(g, l, "ffn_down_shexp.weight");
        y->gate_inp_sh = blk(g, l, "ffn_gate_inp_shexp.weight");
        y->ffn_gate = blk(g, l, "ffn_gate.weight"); y->ffn_up = blk(g, l, "ffn_up.weight");
        y->ffn_down = blk(g, l, "ffn_down.weight");
    }
    m->nthreads = 1;
    *out = m;
    return ORC_OK;
}

void orc_model_free(orc_model *m) {
    if (!m) return;
    orc_gguf_free(m->g); free(m->L); free(m);
}
const orc_arch *orc_model_arch(const orc_model *m) { return &m->a; }
void orc_model_set_threads(orc_model *m, int n) { m->nthreads = n < 1 ? 1 : (n > 64 ? 64 : n); }
void orc_model_set_no_qdot(orc_model *m, int on) { m->no_qdot = on; }

static const float *F(const orc_tensor *t) { return (const float *)t->data; }

/* y = W x with W viewed as [dims[1] rows x dims[0] inputs] */
static void mv(const orc_model *m, const orc_tensor *W, const float *x, float *y) {
    orc_matvec(W->type, W->data, (int)W->dims[0], (int)W->dims[1], x, y, m->no_qdot, m->nthreads);
}
/* one expert of a stacked [in, out, ne] tensor (src/ornith_rforward.c:341-347) */
static void mv_expert(const orc_model *m, const orc_tensor *W, int e, const float *x, float *y) {
    const int in = (int)W->dims[0], out = (int)W->dims[1];
    const uint8_t *base = (const uint8_t *)W->data + (size_t)e * out * orc_row_bytes(W->type, (size_t)in);
    orc_matvec(W->type, base, in, out, x, y, m->no_qdot, m->nthreads);
}

/* ---- per-sequence state ---------------------------------------------------- */
struct orc_session {
    orc_model *m;
    orc_kv *kv;
    float **S, **conv;
    int pos, cap, nhist, have_logits;
    int32_t *hist;
    float *logits;
};

static float *zalloc(size_t n) { return calloc(n ? n : 1, sizeof(float)); }

orc_session *orc_session_new(orc_model *m, int cap, int kv_q8) {
    const orc_arch *a = &m->a;
    if (cap < 1) cap = 1;
    orc_session *s = calloc(1, sizeof *s);
    s->m = m; s->cap = cap;
    s->kv = calloc((size_t)a->n_layers, sizeof(orc_kv));
    s->S = calloc((size_t)a->n_layers, sizeof(float *));
    s->conv = calloc((size_t)a->n_layers, sizeof(float *));
    const int cc = 2 * a->nk * a->dk + a->nv * a->dv;
    for (int l = 0; l < a->n_layers; l++) {
        if (is_full(a, l)) orc_kv_init(&s->kv[l], cap, a->nkv, a->hd, kv_q8);
        else {
            s->conv[l] = zalloc((size_t)(a->conv_k - 1) * cc + 1);
            s->S[l] = zalloc((size_t)a->nv * a->dv * a->dk);
        }
    }
    s->hist = calloc((size_t)cap, sizeof(int32_t));
    s->logits = zalloc((size_t)a->vocab);
    return s;
}
void orc_session_free(orc_session *s) {
    if (!s) return;
    for (int l = 0; l < s->m->a.n_layers; l++) { orc_kv_free(&s->kv[l]); free(s->S[l]); free(s->conv[l]); }
    free(s->kv); free(s->S); free(s->conv); free(s->hist); free(s->logits); free(s);
}
const float *orc_session_logits(const orc_session *s) { return s->have_logits ? s->logits : NULL; }
int orc_session_pos(const orc_session *s) { return s->pos; }
float *orc_session_delta(orc_session *s, int l) { return s->S[l]; }
float *orc_session_conv(orc_session *s, int l) { return s->conv[l]; }
orc_kv *orc_session_kv(orc_session *s, int l) { return is_full(&s->m->a, l) ? &s->kv[l] : NULL; }

int orc_session_seed_context(orc_session *s, int n, uint64_t seed) {
    const orc_arch *a = &s->m->a;
    if (s->pos != 0 || n < 0 || n >= s->cap) return -1;
    uint64_t x = seed * 0x9E3779B97F4A7C15ull + 1;
    for (int l = 0; l < a->n_layers; l++) {
        if (!is_full(a, l)) continue;
        orc_kv *c = &s->kv[l];
        if (!c->quantized) return -1;
        const size_t nc = (size_t)n * c->n_kv_heads * c->head_dim, ns = (size_t)n * c->n_kv_heads;
        for (size_t i = 0; i < nc; i++) {
            x = x * 6364136223846793005ull + 1442695040888963407ull;
            c->Kq[i] = (int8_t)((int)((x >> 33) % 255u) - 127);
            x = x * 6364136223846793005ull + 1442695040888963407ull;
            c->Vq[i] = (int8_t)((int)((x >> 33) % 255u) - 127);
        }
        for (size_t i = 0; i < ns; i++) {
            x = x * 6364136223846793005ull + 1442695040888963407ull;
            c->Ks[i] = (float)((x >> 40) + 1) * 0x1p-30f;
            x = x * 6364136223846793005ull + 1442695040888963407ull;
            c->Vs[i] = (float)((x >> 40) + 1) * 0x1p-30f;
        }
        c->len = n;
    }
    s->pos = n;
    s->nhist = n;
    return 0;
}

int orc_session_adopt(orc_session *s, int n, const float *logits) {
    const orc_arch *a = &s->m->a;
    if (n < 0 || n >= s->cap || !logits) return -1;
    for (int l = 0; l < a->n_layers; l++)
        if (is_full(a, l)) s->kv[l].len = n;
    memcpy(s->logits, logits, (size_t)a->vocab * sizeof(float));
    s->pos = n;
    s->nhist = n;
    s->have_logits = 1;
    return 0;
}

/* ---- layer math (src/ornith_rforward.c:282-503) ----------------------------- */
static float decay_alpha(float a_in, float a_coef, float dt_bias) {
    return expf(a_coef * orc_softplus(a_in + dt_bias));
}

/* 1/sqrt(dk) scale, per-head RMSNorm(ssm_norm), * SiLU(attn_gate xn),
 * ssm_out projection accumulated into x (src/ornith_rforward.c:300-319) */
static void linear_finish(const orc_model *m, const orc_layer *y, const float *xn,
                          float *o_all, float *x) {
    const orc_arch *a = &m->a;
    const int vd = a->nv * a->dv;
    const float sc = 1.0f / sqrtf((float)a->dk);
    for (int i = 0; i < vd; i++) o_all[i] *= sc;
    float *gate = zalloc((size_t)vd), *o = zalloc((size_t)vd), *outp = zalloc((size_t)a->hidden);
    mv(m, y->gate, xn, gate);
    for (int i = 0; i < vd; i++) gate[i] = orc_silu(gate[i]);
    for (int h = 0; h < a->nv; h++)
        orc_rmsnorm(o_all + (size_t)h * a->dv, F(y->ssm_norm), o + (size_t)h * a->dv, a->dv, a->eps);
    for (int i = 0; i < vd; i++) o[i] *= gate[i];
    mv(m, y->ssm_out, o, outp);
    for (int i = 0; i < a->hidden; i++) x[i] += outp[i];
    free(gate); free(o); free(outp);
}

static void linear_attn(orc_session *s, int l, const float *xn, float *x) {
    const orc_model *m = s->m; const orc_arch *a = &m->a; const orc_layer *y = &m->L[l];
    const int qd = a->nk * a->dk, vd = a->nv * a->dv, cc = 2 * qd + vd;
    float *cat = zalloc((size_t)cc), *cv = zalloc((size_t)cc);
    mv(m, y->qkv, xn, cat);
    orc_conv_step(s->conv[l], a->conv_k, cc, cat, F(y->conv), NULL, cv);
    for (int i = 0; i < cc; i++) cv[i] = orc_silu(cv[i]);
    float *qn = zalloc((size_t)qd), *kn = zalloc((size_t)qd);
    for (int h = 0; h < a->nk; h++) {
        orc_l2norm_eps(cv + (size_t)h * a->dk, qn + (size_t)h * a->dk, a->dk, 1e-6f);
        orc_l2norm_eps(cv + qd + (size_t)h * a->dk, kn + (size_t)h * a->dk, a->dk, 1e-6f);
    }
    float *ain = zalloc((size_t)a->nv), *bin = zalloc((size_t)a->nv), *o_all = zalloc((size_t)vd);
    mv(m, y->alpha, xn, ain);
    mv(m, y->beta, xn, bin);
    for (int hv = 0; hv < a->nv; hv++) {
        const int kh = hv % a->nk;      /* k heads tile onto v heads */
        const float al = decay_alpha(ain[hv], F(y->ssm_a)[hv], F(y->dt_bias)[hv]);
        orc_delta_step(s->S[l] + (size_t)hv * a->dv * a->dk, a->dk, a->dv,
                       qn + (size_t)kh * a->dk, kn + (size_t)kh * a->dk,
                       cv + 2 * qd + (size_t)hv * a->dv, al, orc_sigmoid(bin[hv]),
                       o_all + (size_t)hv * a->dv);
    }
    linear_finish(m, y, xn, o_all, x);
    free(cat); free(cv); free(qn); free(kn); free(ain); free(bin); free(o_all);
}

/* q/k RMSNorm + partial RoPE at `pos`, append + attend, sigmoid(gate) */
static void attn_core(orc_session *s, int l, const float *qproj, float *k,
                      const float *v, int pos, float *o) {
    const orc_model *m = s->m; const orc_arch *a = &m->a; const orc_layer *y = &m->L[l];
    const int hd = a->hd, qd = a->nh * hd;
    float *q = zalloc((size_t)qd), *g = zalloc((size_t)qd);
    for (int h = 0; h < a->nh; h++) {
        memcpy(q + (size_t)h * hd, qproj + (size_t)h * 2 * hd, (size_t)hd * 4);
        memcpy(g + (size_t)h * hd, qproj + (size_t)h * 2 * hd + hd, (size_t)hd * 4);
    }
    for (int h = 0; h < a->nh; h++) {
        float *vh = q + (size_t)h * hd;
        orc_rmsnorm(vh, F(y->q_norm), vh, hd, a->eps);
        orc_rope_partial(vh, hd, a->rope_dim, pos, a->rope_theta);
    }
    for (int h = 0; h < a->nkv; h++) {
        float *vh = k + (size_t)h * hd;
        orc_rmsnorm(vh, F(y->k_norm), vh, hd, a->eps);
        orc_rope_partial(vh, hd, a->rope_dim, pos, a->rope_theta);
    }
    orc_gqa_step(&s->kv[l], q, k, v, a->nh, o, 0.0f);
    for (int i = 0; i < qd; i++) o[i] *= orc_sigmoid(g[i]);
    free(q); free(g);
}

static void full_attn(orc_session *s, int l, const float *xn, float *x) {
    const orc_model *m = s->m; const orc_arch *a = &m->a; const orc_layer *y = &m->L[l];
    const int qd = a->nh * a->hd, kvd = a->nkv * a->hd;
    float *qp = zalloc(2 * (size_t)qd), *k = zalloc((size_t)kvd), *v = zalloc((size_t)kvd);
    float *o = zalloc((size_t)qd), *outp = zalloc((size_t)a->hidden);
    mv(m, y->q, xn, qp); mv(m, y->k, xn, k); mv(m, y->v, xn, v);
    attn_core(s, l, qp, k, v, s->pos, o);
    mv(m, y->o, o, outp);
    for (int i = 0; i < a->hidden; i++) x[i] += outp[i];
    free(qp); free(k); free(v); free(o); free(outp);
}

/* router -> top-k -> per-expert SwiGLU weighted sum -> shared expert with its
 * sigmoid gate -> residual (src/ornith_rforward.c:354-411). x is both the
 * input and the accumulator. */
static void ffn_moe(const orc_model *m, int l, float *x) {
    const orc_arch *a = &m->a; const orc_layer *y = &m->L[l];
    const int H = a->hidden, I = a->moe_inter, K = a->top_k;
    float *xn = zalloc((size_t)H), *lg = zalloc((size_t)a->ne), *w = zalloc((size_t)K);
    int *idx = calloc((size_t)K, sizeof(int));
    orc_rmsnorm(x, F(y->post_norm), xn, H, a->eps);
    mv(m, y->router, xn, lg);
    orc_moe_route(lg, a->ne, K, idx, w);
    float *g = zalloc((size_t)I), *u = zalloc((size_t)I), *o = zalloc((size_t)H), *acc = zalloc((size_t)H);
    for (int s = 0; s < K; s++) {
        mv_expert(m, y->gate_exps, idx[s], xn, g);
        mv_expert(m, y->up_exps, idx[s], xn, u);
        for (int i = 0; i < I; i++) g[i] = orc_silu(g[i]) * u[i];
        mv_expert(m, y->down_exps, idx[s], g, o);
        for (int i = 0; i < H; i++) acc[i] += w[s] * o[i];
    }
    if (y->gate_sh) {
        const int sI = a->shared_inter;
        float *sg = zalloc((size_t)sI), *su = zalloc((size_t)sI), *so = zalloc((size_t)H);
        mv(m, y->gate_sh, xn, sg);
        mv(m, y->up_sh, xn, su);
        for (int i = 0; i < sI; i++) sg[i] = orc_silu(sg[i]) * su[i];
        mv(m, y->down_sh, sg, so);
        if (y->gate_inp_sh) {
            float gl = 0.0f;
            orc_matvec(y->gate_inp_sh->type, y->gate_inp_sh->data, H, 1, xn, &gl, m->no_qdot, 1);
            const float gs = orc_sigmoid(gl);
            for (int i = 0; i < H; i++) so[i] *= gs;
        }
        for (int i = 0; i < H; i++) acc[i] += so[i];
        free(sg); free(su); free(so);
    }
    for (int i = 0; i < H; i++) x[i] += acc[i];
    free(xn); free(lg); free(w); free(idx); free(g); free(u); free(o); free(acc);
}

static void ffn_dense(const orc_model *m, int l, float *x) {
    const orc_arch *a = &m->a; const orc_layer *y = &m->L[l];
    const int H = a->hidden, I = a->shared_inter;
    float *xn = zalloc((size_t)H), *g = zalloc((size_t)I), *u = zalloc((size_t)I), *o = zalloc((size_t)H);
    orc_rmsnorm(x, F(y->post_norm), xn, H, a->eps);
    mv(m, y->ffn_gate, xn, g); mv(m, y->ffn_up, xn, u);
    for (int i = 0; i < I; i++) g[i] = orc_silu(g[i]) * u[i];
    mv(m, y->ffn_down, g, o);
    for (int i = 0; i < H; i++) x[i] += o[i];
    free(xn); free(g); free(u); free(o);
}

static void ffn(const orc_model *m, int l, float *x) {
    if (m->a.ne > 0) ffn_moe(m, l, x); else ffn_dense(m, l, x);
}

static void embed(const orc_model *m, int32_t tok, float *x) {
    const size_t in = (size_t)m->a.hidden;
    orc_dequantize(m->embd->type, (const uint8_t *)m->embd->data + (size_t)tok * orc_row_bytes(m->embd->type, in), x, in);
}

static void head(const orc_model *m, const float *x, float *logits) {
    float *xn = zalloc((size_t)m->a.hidden);
    orc_rmsnorm(x, F(m->out_norm), xn, m->a.hidden, m->a.eps);
    mv(m, m->lm_head, xn, logits);
    free(xn);
}

/* rforward_token (src/ornith_rforward.c:686-706) */
static void forward_token(orc_session *s, int32_t tok, float *logits) {
    const orc_model *m = s->m; const orc_arch *a = &m->a;
    float *x = zalloc((size_t)a->hidden), *xn = zalloc((size_t)a->hidden);
    embed(m, tok, x);
    for (int l = 0; l < a->n_layers; l++) {
        orc_rmsnorm(x, F(m->L[l].attn_norm), xn, a->hidden, a->eps);
        if (is_full(a, l)) full_attn(s, l, xn, x); else linear_attn(s, l, xn, x);
        ffn(m, l, x);
    }
    s->pos++;
    if (logits) head(m, x, logits);
    free(x); free(xn);
}

/* ---- prefill (src/ornith_rforward.c:513-682) -------------------------------- */
static void full_attn_prefill(orc_session *s, int l, const float *XN, int T, int base, float *X) {
    const orc_model *m = s->m; const orc_arch *a = &m->a; const orc_layer *y = &m->L[l];
    const int H = a->hidden, qd = a->nh * a->hd, kvd = a->nkv * a->hd;
    float *qp = zalloc(2 * (size_t)qd), *k = zalloc((size_t)kvd), *v = zalloc((size_t)kvd);
    float *O = zalloc((size_t)T * qd), *outp = zalloc((size_t)H);
    for (int t = 0; t < T; t++) {
        mv(m, y->q, XN + (size_t)t * H, qp); mv(m, y->k, XN + (size_t)t * H, k);
        mv(m, y->v, XN + (size_t)t * H, v);
        attn_core(s, l, qp, k, v, base + t, O + (size_t)t * qd);
    }
    for (int t = 0; t < T; t++) {
        mv(m, y->o, O + (size_t)t * qd, outp);
        for (int i = 0; i < H; i++) X[(size_t)t * H + i] += outp[i];
    }
    free(qp); free(k); free(v); free(O); free(outp);
}

static void linear_attn_prefill(orc_session *s, int l, const float *XN, int T, int chunk, float *X) {
    const orc_model *m = s->m; const orc_arch *a = &m->a; const orc_layer *y = &m->L[l];
    const int H = a->hidden, nk = a->nk, nv = a->nv, dk = a->dk, dv = a->dv;
    const int qd = nk * dk, vd = nv * dv, cc = 2 * qd + vd;
    float *CV = zalloc((size_t)T * cc), *cat = zalloc((size_t)cc);
    for (int t = 0; t < T; t++) {
        mv(m, y->qkv, XN + (size_t)t * H, cat);
        orc_conv_step(s->conv[l], a->conv_k, cc, cat, F(y->conv), NULL, CV + (size_t)t * cc);
    }
    for (size_t i = 0; i < (size_t)T * cc; i++) CV[i] = orc_silu(CV[i]);
    float *A = zalloc((size_t)T * nv), *B = zalloc((size_t)T * nv);
    for (int t = 0; t < T; t++) {
        mv(m, y->alpha, XN + (size_t)t * H, A + (size_t)t * nv);
        mv(m, y->beta, XN + (size_t)t * H, B + (size_t)t * nv);
    }
    float *Qh = zalloc((size_t)T * dk), *Kh = zalloc((size_t)T * dk), *Vh = zalloc((size_t)T * dv);
    float *al = zalloc((size_t)T), *be = zalloc((size_t)T), *Oh = zalloc((size_t)T * dv);
    float *OA = zalloc((size_t)T * vd);
    for (int hv = 0; hv < nv; hv++) {
        const int kh = hv % nk;
        for (int t = 0; t < T; t++) {
            const float *row = CV + (size_t)t * cc;
            orc_l2norm_eps(row + kh * dk, Qh + (size_t)t * dk, dk, 1e-6f);
            orc_l2norm_eps(row + qd + kh * dk, Kh + (size_t)t * dk, dk, 1e-6f);
            memcpy(Vh + (size_t)t * dv, row + 2 * qd + hv * dv, (size_t)dv * 4);
            al[t] = decay_alpha(A[(size_t)t * nv + hv], F(y->ssm_a)[hv], F(y->dt_bias)[hv]);
            be[t] = orc_sigmoid(B[(size_t)t * nv + hv]);
        }
        orc_delta_prefill(s->S[l] + (size_t)hv * dv * dk, dk, dv, Qh, Kh, Vh, al, be, T, chunk, Oh);
        for (int t = 0; t < T; t++)
            memcpy(OA + (size_t)t * vd + hv * dv, Oh + (size_t)t * dv, (size_t)dv * 4);
    }
    for (int t = 0; t < T; t++)
        linear_finish(m, y, XN + (size_t)t * H, OA + (size_t)t * vd, X + (size_t)t * H);
    free(CV); free(cat); free(A); free(B); free(Qh); free(Kh); free(Vh);
    free(al); free(be); free(Oh); free(OA);
}

static void forward_prefill(orc_session *s, const int32_t *toks, int T, int chunk, float *logits) {
    const orc_model *m = s->m; const orc_arch *a = &m->a;
    const int H = a->hidden, base = s->pos;
    float *X = zalloc((size_t)T * H), *XN = zalloc((size_t)T * H);
    for (int t = 0; t < T; t++) embed(m, toks[t], X + (size_t)t * H);
    for (int l = 0; l < a->n_layers; l++) {
        for (int t = 0; t < T; t++)
            orc_rmsnorm(X + (size_t)t * H, F(m->L[l].attn_norm), XN + (size_t)t * H, H, a->eps);
        if (is_full(a, l)) full_attn_prefill(s, l, XN, T, base, X);
        else linear_attn_prefill(s, l, XN, T, chunk, X);
        for (int t = 0; t < T; t++) ffn(m, l, X + (size_t)t * H);
    }
    s->pos = base + T;
    if (logits) head(m, X + (size_t)(T - 1) * H, logits);
    free(X); free(XN);
}

/* ---- sessions (src/ornith_rforward.c:838-982) ------------------------------- */
int orc_session_eval(orc_session *s, const int32_t *toks, int n, int serial) {
    if (n <= 0) return ORC_OK;
    if (s->pos + n > s->cap) {
        orc_seterr("session capacity %d exceeded (pos %d + %d tokens)", s->cap, s->pos, n);
        return ORC_ERR_UNSUPPORTED;
    }
    if (serial) for (int i = 0; i < n; i++) forward_token(s, toks[i], i == n - 1 ? s->logits : NULL);
    else forward_prefill(s, toks, n, 32, s->logits);
    s->have_logits = 1;
    for (int i = 0; i < n && s->nhist < s->cap; i++) s->hist[s->nhist++] = toks[i];
    return ORC_OK;
}

int orc_session_step(orc_session *s, int32_t tok) {
    if (s->pos >= s->cap) { orc_seterr("session full"); return ORC_ERR_UNSUPPORTED; }
    forward_token(s, tok, s->logits);
    s->have_logits = 1;
    if (s->nhist < s->cap) s->hist[s->nhist++] = tok;
    return ORC_OK;
}

static int32_t argmax(const float *v, int n) {
    int b = 0;
    for (int i = 1; i < n; i++) if (v[i] > v[b]) b = i;
    return b;
}

/* greedy: emit argmax, feed it back; stop (without emitting) on eos; the
 * last step's logits are computed even though nothing is emitted after them */
int orc_session_generate(orc_session *s, int n_predict, int32_t *out_tokens,
                         int *n_out, float *logits_trace) {
    const int V = s->m->a.vocab;
    if (!s->have_logits) { orc_seterr("session has no logits"); return ORC_ERR_FORMAT; }
    int n = 0;
    int32_t next = argmax(s->logits, V);
    for (int step = 0; step < n_predict; step++) {
        if (next == s->m->a.eos) break;
        if (s->pos >= s->cap) break;
        out_tokens[n++] = next;
        if (s->nhist < s->cap) s->hist[s->nhist++] = next;
        forward_token(s, next, s->logits);
        if (logits_trace) memcpy(logits_trace + (size_t)step * V, s->logits, (size_t)V * 4);
        next = argmax(s->logits, V);
    }
    if (n_out) *n_out = n;
    return ORC_OK;
}
