/* or_gen.c - random-init qwen35moe GGUF generator (TEST INFRASTRUCTURE).
 *
 * Writes the tensor set rmodel_load expects (src/ornith_rforward.c:719-816):
 * every projection is a quantized [in, out] (or [in, out, ne] expert stack)
 * drawn from N(0, sigma); norms, ssm_a, ssm_dt.bias and ssm_conv1d are F32
 * (read by raw pointer in the reference) with the reference fixture's
 * ranges (tests/test_session.c:93-141). Metadata: the tokens array (the
 * tokenizer requires it), expert_used_count, rope.dimension_count, and no
 * eos id so generation never stops early. The HIP engine synthesises the
 * same tensors on the device from the same counter-based streams.
 */
#include "oracle.h"
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

void orc_seterr(const char *fmt, ...);

typedef struct { void **p; size_t n; } pool;
static void *keep(pool *pl, void *p) {
    pl->p = realloc(pl->p, (pl->n + 1) * sizeof(void *));
    pl->p[pl->n++] = p;
    return p;
}

static int add_q(orc_writer *w, pool *pl, const orc_gen_cfg *c, const char *name,
                 uint32_t type, int nd, uint64_t d0, uint64_t d1, uint64_t d2) {
    const uint64_t dims[3] = { d0, d1, d2 };
    const size_t n = (size_t)d0 * d1 * (nd > 2 ? d2 : 1);
    float *f = malloc(n * sizeof(float));
    if (!f) return ORC_ERR_OOM;
    orc_fill_gauss(orc_stream_key(c->seed, name), c->sigma, f, n, 0);
    const size_t nb = orc_row_bytes(type, n);
    void *q = keep(pl, malloc(nb ? nb : 1));
    int st = orc_quantize(type, f, q, n);
    free(f);
    if (st) return st;
    return orc_w_tensor(w, name, (uint32_t)nd, dims, type, q, nb);
}

static int add_u(orc_writer *w, pool *pl, const orc_gen_cfg *c, const char *name,
                 int nd, uint64_t d0, uint64_t d1, float lo, float hi) {
    const uint64_t dims[2] = { d0, d1 };
    const size_t n = (size_t)d0 * (nd > 1 ? d1 : 1);
    float *f = keep(pl, malloc(n * sizeof(float)));
    orc_fill_uniform(orc_stream_key(c->seed, name), lo, hi, f, n, 0);
    return orc_w_tensor(w, name, (uint32_t)nd, dims, ORC_F32, f, n * 4);
}

int orc_gen_write_gguf(const orc_gen_cfg *c, const char *path) {
    orc_writer *w = orc_writer_new();
    pool pl = {0};
    char nm[160], **toks = NULL;
    const int H = c->hidden, V = c->vocab;
    const int qd = c->nk * c->dhead, vd = c->nv * c->dhead, cc = 2 * qd + vd;
    int st = 0;

    orc_w_string(w, "general.architecture", "qwen35moe");
    orc_w_string(w, "general.name", "ornith-hip-random-init");
    orc_w_u32(w, "qwen35moe.block_count", (uint32_t)c->n_layers);
    orc_w_u32(w, "qwen35moe.expert_used_count", (uint32_t)c->top_k);
    orc_w_u32(w, "qwen35moe.rope.dimension_count", 64);
    orc_w_f32(w, "qwen35moe.rope.freq_base", 1e7f);
    orc_w_f32(w, "qwen35moe.attention.layer_norm_rms_epsilon", 1e-6f);
    toks = malloc((size_t)V * sizeof(char *));
    for (int i = 0; i < V; i++) { toks[i] = malloc(16); snprintf(toks[i], 16, "t%d", i); }
    orc_w_arr_str(w, "tokenizer.ggml.tokens", (const char *const *)toks, (size_t)V);

#define CK(x) do { if ((st = (x)) != 0) goto done; } while (0)
    CK(add_q(w, &pl, c, "token_embd.weight", c->t_embd, 2, H, V, 0));
    CK(add_u(w, &pl, c, "output_norm.weight", 1, H, 0, 0.9f, 1.1f));
    CK(add_q(w, &pl, c, "output.weight", c->t_output, 2, H, V, 0));
    for (int l = 0; l < c->n_layers; l++) {
        const int full = c->full_interval > 0 && l % c->full_interval == c->full_interval - 1;
#define N(s) (snprintf(nm, sizeof nm, "blk.%d.%s", l, s), nm)
        CK(add_u(w, &pl, c, N("attn_norm.weight"), 1, H, 0, 0.9f, 1.1f));
        CK(add_u(w, &pl, c, N("post_attention_norm.weight"), 1, H, 0, 0.9f, 1.1f));
        if (full) {
            CK(add_q(w, &pl, c, N("attn_q.weight"), c->t_default, 2, H, 2 * c->nh * c->hd, 0));
            CK(add_q(w, &pl, c, N("attn_k.weight"), c->t_default, 2, H, c->nkv * c->hd, 0));
            CK(add_q(w, &pl, c, N("attn_v.weight"), c->t_attn_v, 2, H, c->nkv * c->hd, 0));
            CK(add_u(w, &pl, c, N("attn_q_norm.weight"), 1, c->hd, 0, 0.9f, 1.1f));
            CK(add_u(w, &pl, c, N("attn_k_norm.weight"), 1, c->hd, 0, 0.9f, 1.1f));
            CK(add_q(w, &pl, c, N("attn_output.weight"), c->t_default, 2, c->nh * c->hd, H, 0));
        } else {
            CK(add_q(w, &pl, c, N("attn_qkv.weight"), c->t_default, 2, H, cc, 0));
            CK(add_u(w, &pl, c, N("ssm_conv1d.weight"), 2, c->conv_k, cc, -0.2f, 0.2f));
            CK(add_u(w, &pl, c, N("ssm_a"), 1, c->nv, 0, -0.8f, -0.2f));
            CK(add_u(w, &pl, c, N("ssm_dt.bias"), 1, c->nv, 0, -0.05f, 0.05f));
            CK(add_u(w, &pl, c, N("ssm_norm.weight"), 1, c->dhead, 0, 0.9f, 1.1f));
            CK(add_q(w, &pl, c, N("ssm_alpha.weight"), c->t_default, 2, H, c->nv, 0));
            CK(add_q(w, &pl, c, N("ssm_beta.weight"), c->t_default, 2, H, c->nv, 0));
            CK(add_q(w, &pl, c, N("attn_gate.weight"), c->t_default, 2, H, vd, 0));
            CK(add_q(w, &pl, c, N("ssm_out.weight"), c->t_default, 2, vd, H, 0));
        }
        if (c->ne <= 0) {
            /* dense SwiGLU FFN of width shared_inter */
            CK(add_q(w, &pl, c, N("ffn_gate.weight"), c->t_default, 2, H, c->shared_inter, 0));
            CK(add_q(w, &pl, c, N("ffn_up.weight"), c->t_default, 2, H, c->shared_inter, 0));
            CK(add_q(w, &pl, c, N("ffn_down.weight"), c->t_ffn_down, 2, c->shared_inter, H, 0));
            continue;
        }
        CK(add_q(w, &pl, c, N("ffn_gate_inp.weight"), c->t_default, 2, H, c->ne, 0));
        CK(add_q(w, &pl, c, N("ffn_gate_exps.weight"), c->t_exps ? c->t_exps : c->t_default, 3, H, c->moe_inter, c->ne));
        CK(add_q(w, &pl, c, N("ffn_up_exps.weight"), c->t_exps ? c->t_exps : c->t_default, 3, H, c->moe_inter, c->ne));
        CK(add_q(w, &pl, c, N("ffn_down_exps.weight"), c->t_exps ? c->t_exps : c->t_ffn_down, 3, c->moe_inter, H, c->ne));
        if (c->shared_inter > 0) {
            CK(add_q(w, &pl, c, N("ffn_gate_shexp.weight"), c->t_default, 2, H, c->shared_inter, 0));
            CK(add_q(w, &pl, c, N("ffn_up_shexp.weight"), c->t_default, 2, H, c->shared_inter, 0));
            CK(add_q(w, &pl, c, N("ffn_down_shexp.weight"), c->t_ffn_down, 2, c->shared_inter, H, 0));
            CK(add_q(w, &pl, c, N("ffn_gate_inp_shexp.weight"), c->t_default, 1, H, 1, 0));
        }
#undef N
    }
#undef CK
    st = orc_writer_write(w, path);
done:
    for (size_t i = 0; i < pl.n; i++) free(pl.p[i]);
    free(pl.p);
    if (toks) { for (int i = 0; i < V; i++) free(toks[i]); free(toks); }
    orc_writer_free(w);
    return st;
}
