/* oracle.h - CPU restatement of the reference decode path (TEST INFRASTRUCTURE).
 *
 * This library is the checker for the HIP engine, never part of it. Only the
 * tests, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it. Each
 * function restates the reference algorithm at the cited file:line of
 * njbrake/ornithology and keeps its floating-point operation order, so that a
 * gcc build with -std=c11 -ffp-contract=off reproduces the reference bits.
 * tests/test_oracle_quant.py, test_oracle_attn.py and test_oracle_model.py
 * check that against oracle/_ref (the reference's own sources, compiled in
 * place by oracle/Makefile) and against the fixtures in tests/golden/, and
 * pin each function further by closed forms, brute force and known answers.
 */
#ifndef ORNITH_ORACLE_H
#define ORNITH_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml tensor type ids (numeric values of the GGUF format;
 * reference src/ornith_gguf.h:17-39). */
enum {
    ORC_F32 = 0, ORC_F16 = 1, ORC_Q4_0 = 2, ORC_Q8_0 = 8, ORC_Q2_K = 10,
    ORC_Q4_K = 12, ORC_Q5_K = 13, ORC_Q6_K = 14, ORC_Q8_K = 15,
    ORC_IQ2_XXS = 16, ORC_BF16 = 30
};

/* status codes, same numbering as ornith_status (src/ornith.h:34-41) */
enum { ORC_OK = 0, ORC_ERR_IO, ORC_ERR_FORMAT, ORC_ERR_UNSUPPORTED,
       ORC_ERR_OOM, ORC_ERR_NOTFOUND };

const char *orc_last_error(void);

/* ---- f16 / bf16 (src/ornith_quant.c:14-81) ---------------------------- */
uint16_t orc_f32_to_f16(float f);
float    orc_f16_to_f32(uint16_t h);

/* ---- block geometry (src/ornith_quant.c:89-146) ----------------------- */
size_t orc_block_elems(uint32_t type);
size_t orc_block_bytes(uint32_t type);
size_t orc_row_bytes(uint32_t type, size_t n_elems);

/* ---- codecs (src/ornith_quant.c:155-789, 871-1073) -------------------- */
int orc_quantize(uint32_t type, const float *src, void *dst, size_t n);
int orc_dequantize(uint32_t type, const void *src, float *dst, size_t n);

/* ---- Q8_K activation + integer dots (src/ornith_qdot.c) --------------- */
typedef struct {
    float   d;
    int8_t  qs[256];
    int16_t bsums[16];
} orc_q8k;                      /* 292 bytes, src/ornith_qdot.h:30-34 */

void  orc_quantize_q8k(const float *x, orc_q8k *y, int64_t k);
int   orc_qdot_can(uint32_t type, int n);
float orc_qdot(uint32_t type, int n, const void *wrow, const orc_q8k *y);

/* y[o] = W[o,:] . x for o in [0,out), reference matvec_q semantics
 * (src/ornith_rforward.c:100-196): Q8_K integer path when qdot_can, else
 * dequantize the row and run the sequential f32 dot. no_qdot forces the
 * fallback (ORNITH_NO_QDOT=1). nthreads<=1 runs inline. */
void orc_matvec(uint32_t type, const void *W, int in, int out,
                const float *x, float *y, int no_qdot, int nthreads);

/* ---- f32 helpers (src/ornith_tensor.c:100-178) ------------------------ */
void  orc_rmsnorm(const float *x, const float *w, float *out, int n, float eps);
void  orc_softmax(float *x, int n);
float orc_sigmoid(float x);
float orc_silu(float x);
float orc_softplus(float x);
float orc_dot(const float *a, const float *b, int n);
void  orc_l2norm_eps(const float *x, float *out, int n, float eps);
void  orc_rope_partial(float *v, int head_dim, int rot, int pos, float theta);

/* ---- attention core (src/ornith_attn.c) ------------------------------- */
typedef struct {
    float  *K, *V;          /* fp32 mode [cap, nkv, hd]          */
    int8_t *Kq, *Vq;        /* q8 mode   [cap, nkv, hd]          */
    float  *Ks, *Vs;        /* q8 mode   [cap, nkv]              */
    int quantized, capacity, len, n_kv_heads, head_dim;
} orc_kv;

int   orc_kv_init(orc_kv *c, int cap, int nkv, int hd, int quantized);
void  orc_kv_free(orc_kv *c);
float orc_kv_quant_vec(const float *x, int n, int8_t *q);
void  orc_gqa_step(orc_kv *c, const float *q, const float *k, const float *v,
                   int n_heads, float *out, float scale);
/* attention over the c->len cached positions without appending (the second
 * half of orc_gqa_step, src/ornith_attn.c:111-149) */
void  orc_gqa_attend(const orc_kv *c, const float *q, int n_heads, float *out, float scale);
void  orc_delta_step(float *S, int dk, int dv, const float *q, const float *k,
                     const float *v, float alpha, float beta, float *o);
void  orc_delta_prefill(float *S, int dk, int dv, const float *Q,
                        const float *K, const float *V, const float *alpha,
                        const float *beta, int T, int chunk, float *O);
void  orc_conv_step(float *buf, int K, int C, const float *x,
                    const float *w, const float *bias, float *out);

/* ---- MoE router (src/ornith_moe.c:8-30) ------------------------------- */
void orc_moe_route(const float *logits, int ne, int k, int *idx, float *w);

/* ---- deterministic synthetic data ------------------------------------- */
/* Counter-based generator shared with the HIP engine's on-device weight
 * synthesis: value i of stream `key` depends only on (key, i). */
uint64_t orc_stream_key(uint64_t seed, const char *name);
void     orc_fill_gauss(uint64_t key, float sigma, float *dst, size_t n, size_t first);
void     orc_fill_uniform(uint64_t key, float lo, float hi, float *dst, size_t n, size_t first);
void     orc_fill_ids(uint64_t key, int32_t v, int32_t *dst, size_t n);

/* ---- GGUF v3 (src/ornith_gguf_write.c:218-474) ------------------------ */
typedef struct orc_gguf orc_gguf;

typedef struct {
    char     name[256];
    uint32_t n_dims;
    uint64_t dims[4];
    uint32_t type;
    uint64_t n_elements;
    const void *data;       /* points into the mapping */
    uint64_t nbytes;
} orc_tensor;

/* writer */
typedef struct orc_writer orc_writer;
orc_writer *orc_writer_new(void);
void orc_writer_free(orc_writer *w);
int  orc_w_string(orc_writer *w, const char *key, const char *val);
int  orc_w_u32(orc_writer *w, const char *key, uint32_t v);
int  orc_w_f32(orc_writer *w, const char *key, float v);
int  orc_w_arr_str(orc_writer *w, const char *key, const char *const *vals, size_t n);
int  orc_w_tensor(orc_writer *w, const char *name, uint32_t n_dims,
                  const uint64_t *dims, uint32_t type, const void *data,
                  uint64_t nbytes);
int  orc_writer_write(orc_writer *w, const char *path);

/* mmap loader */
int  orc_gguf_load(const char *path, orc_gguf **out);
void orc_gguf_free(orc_gguf *g);
uint64_t orc_gguf_n_tensors(const orc_gguf *g);
const orc_tensor *orc_gguf_tensor(const orc_gguf *g, uint64_t i);
const orc_tensor *orc_gguf_find(const orc_gguf *g, const char *name);

/* ---- model + session (src/ornith_rforward.c:24-982) ------------------- */
typedef struct {
    int hidden, n_layers, vocab, full_interval;
    int nh, nkv, hd, rope_dim;
    int nk, nv, dk, dv, conv_k;
    int ne, top_k, moe_inter, shared_inter;
    float rope_theta, eps;
    int eos;
} orc_arch;

typedef struct orc_model orc_model;
typedef struct orc_session orc_session;

int  orc_model_load(const char *path, orc_model **out);
void orc_model_free(orc_model *m);
const orc_arch *orc_model_arch(const orc_model *m);
void orc_model_set_threads(orc_model *m, int nthreads);
void orc_model_set_no_qdot(orc_model *m, int on);

orc_session *orc_session_new(orc_model *m, int cap, int kv_q8);
void orc_session_free(orc_session *s);
/* serial != 0 is ORNITH_PREFILL_SERIAL=1 (token-by-token); else chunk 32. */
int  orc_session_eval(orc_session *s, const int32_t *toks, int n, int serial);
int  orc_session_generate(orc_session *s, int n_predict, int32_t *out_tokens,
                          int *n_out, float *logits_trace);
const float *orc_session_logits(const orc_session *s);
int  orc_session_pos(const orc_session *s);
/* one rforward_token step (logits written to the session's buffer) */
int  orc_session_step(orc_session *s, int32_t token);
/* state access for parity tests: layer L's delta state [nv*dv*dk], conv
 * window [(K-1)*Cc], or Q8 KV pointers; NULL when the layer lacks it. */
float  *orc_session_delta(orc_session *s, int L);
float  *orc_session_conv(orc_session *s, int L);
orc_kv *orc_session_kv(orc_session *s, int L);
/* Timing aid for the CPU baseline, not part of the reference's algorithm:
 * move an empty session to position n (< cap) with every full-attention
 * layer's Q8 KV cache holding n seeded positions (codes in [-127, 127],
 * scales in (0, 2^-6]), as if an n-token prompt had run, so that the next
 * token steps cost what they cost at that context. Returns 0, or -1 when the
 * session is not empty, n is out of range or the cache is not Q8. */
int orc_session_seed_context(orc_session *s, int n, uint64_t seed);
/* Test aid, not part of the reference's algorithm: take the state the caller
 * wrote through orc_session_delta / _conv / _kv (a session's state computed
 * elsewhere, e.g. by the GPU engine) as that of a session at position n whose
 * last evaluation gave `logits`, so that token steps continue from it. Every
 * full-attention layer's cache then holds n positions. Returns 0, or -1 when
 * n is out of range. */
int orc_session_adopt(orc_session *s, int n, const float *logits);

/* ---- random-init GGUF generator --------------------------------------- */
typedef struct {
    int hidden, n_layers, vocab, full_interval;
    int nh, nkv, hd;
    int nk, nv, dhead, conv_k;
    int ne, top_k, moe_inter, shared_inter;
    uint32_t t_default;     /* type of every projection weight            */
    uint32_t t_attn_v;      /* attn_v                                     */
    uint32_t t_ffn_down;    /* ffn_down_exps and ffn_down_shexp           */
    uint32_t t_output;      /* lm_head                                    */
    uint32_t t_embd;        /* token_embd                                 */
    uint64_t seed;
    float sigma;            /* N(0, sigma) for projection weights          */
    uint32_t t_exps;        /* routed experts gate/up/down; 0: t_default /
                               t_ffn_down as above                         */
} orc_gen_cfg;

int orc_gen_write_gguf(const orc_gen_cfg *cfg, const char *path);

#ifdef __cplusplus
}
#endif
#endif
