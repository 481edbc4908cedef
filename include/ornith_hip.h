/* ornith_hip.h - C ABI of the MI355X (gfx950) decode engine for
 * ornithology-format qwen35moe GGUF models.
 *
 * Plain C types only (no HIP or torch types). Host pointers passed in are
 * borrowed for the duration of the call. Every entry point returns an
 * ornith_status value (src/ornith.h:34-41) and, on failure, leaves a message
 * for ornith_hip_last_error() (the reference's global, non-thread-safe error
 * buffer convention, src/ornith_util.c:7,25-30). Nothing aborts.
 *
 * Threading: one context per device, one HIP stream per context; calls on one
 * context are not re-entrant (the reference serialises generation behind one
 * mutex, src/ornith_server.c:791).
 *
 * Citations name the reference interface each entry point replaces
 * (paths relative to the njbrake/ornithology tree).
 */
#ifndef ORNITH_HIP_H
#define ORNITH_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ornith_status numbering (src/ornith.h:34-41) */
#define ORNITH_HIP_OK              0
#define ORNITH_HIP_ERR_IO          1
#define ORNITH_HIP_ERR_FORMAT      2
#define ORNITH_HIP_ERR_UNSUPPORTED 3
#define ORNITH_HIP_ERR_OOM         4
#define ORNITH_HIP_ERR_NOTFOUND    5
#define ORNITH_HIP_ERR_DEVICE      6   /* HIP runtime error (no reference twin) */

typedef struct ornith_hip_ctx ornith_hip_ctx;
typedef struct ornith_hip_tensor ornith_hip_tensor;
typedef struct ornith_hip_model ornith_hip_model;
typedef struct ornith_hip_session ornith_hip_session;

/* Q8_K activation super-block, byte-identical to oq8k_block
 * (src/ornith_qdot.h:30-34): 292 bytes. */
typedef struct {
    float   d;
    int8_t  qs[256];
    int16_t bsums[16];
} ornith_hip_q8k;

/* The ornith_arch fields the decode path uses (src/ornith_model.h:22-64),
 * inferred from tensor shapes exactly as rmodel_load does
 * (src/ornith_rforward.c:719-816). */
typedef struct {
    int32_t hidden, n_layers, vocab, full_interval;
    int32_t nh, nkv, hd, rope_dim;
    int32_t nk, nv, dk, dv, conv_k;
    int32_t ne, top_k, moe_inter, shared_inter;
    float   rope_theta, eps;
    int32_t eos;
} ornith_hip_arch;

/* Random-init model description: the tensor set and value streams of the
 * repository's GGUF generator (N(0, sigma) projections via the counter-based
 * generator, F32 norms/ssm tensors in the reference fixture ranges). */
typedef struct {
    int32_t hidden, n_layers, vocab, full_interval;
    int32_t nh, nkv, hd;
    int32_t nk, nv, dhead, conv_k;
    int32_t ne, top_k, moe_inter, shared_inter;
    uint32_t t_default, t_attn_v, t_ffn_down, t_output, t_embd;
    uint64_t seed;
    float    sigma;
    uint32_t t_exps;   /* routed experts gate/up/down; 0: t_default / t_ffn_down */
} ornith_hip_gen_cfg;

const char *ornith_hip_last_error(void);            /* ornith_last_error, src/ornith_util.c:25-30 */

int  ornith_hip_init(int device, ornith_hip_ctx **out);
void ornith_hip_free(ornith_hip_ctx *ctx);
int  ornith_hip_sync(ornith_hip_ctx *ctx);            /* wait for all work on the device */

/* ---- ornith_qdot / codecs (kernel-level boundary) --------------------------- */

/* Copy one GGUF tensor (its raw block bytes) to the device in the engine's
 * plane layout. dims[0] = input width, the product of the remaining dims =
 * rows (GGUF {in, out[, ne]}, src/ornith_rforward.c:88-89,338-347). */
int  ornith_hip_upload(ornith_hip_ctx *ctx, const char *name, uint32_t ggml_type,
                       const void *host_bytes, uint64_t nbytes, uint32_t n_dims,
                       const uint64_t *dims, ornith_hip_tensor **out);
void ornith_hip_tensor_free(ornith_hip_tensor *t);
/* Inverse of upload: the tensor's bytes in GGUF block order (nbytes must be
 * the GGUF size), e.g. to compare a synthesised tensor with a GGUF file. */
int  ornith_hip_tensor_download(const ornith_hip_tensor *t, void *gguf_bytes, uint64_t nbytes);

/* qdot_quantize_row_q8_K (src/ornith_qdot.h:36-38): k % 256 == 0. */
int  ornith_hip_quantize_q8K(ornith_hip_ctx *ctx, const float *x, int64_t k,
                             ornith_hip_q8k *yq);

/* matmul_batch_q (src/ornith_rforward.c:138-196): Y[t*out+o] = W[o,:].X[t,:]
 * for Tn columns; Q8_K integer path for Q4_K/Q6_K/Q8_0 (qdot_can), ordered
 * f32 fallback otherwise. Host X [Tn*in], Y [Tn*out]. The first call with
 * Tn > 1 that runs a Q4_K / Q6_K tensor on the matrix cores builds that
 * tensor's prompt tiles (see ornith_hip_session_new). */
int  ornith_hip_matvec(ornith_hip_ctx *ctx, const ornith_hip_tensor *W,
                       const float *x, float *y, int Tn);

/* No counterpart in the reference. ornith_hip_matvec for callers that cannot
 * allocate device memory (tight serving loops, harnesses that forbid
 * hipMalloc): the same results, computed one column at a time in a fixed
 * 4 MiB device array per GPU (resolved by ornith_hip_init) instead of a buffer
 * the library allocates. It still copies X and Y between host and device and
 * synchronises the context's stream, so it must not be called while a stream
 * capture is active. Limit: in*5 + (in/256)*40 + out*4 + 4096 <= 4 MiB (e.g.
 * out <= 1,040,000 rows at in = 2048); larger tensors return
 * ORNITH_HIP_ERR_UNSUPPORTED. Calls that overlap on one GPU share the array
 * and race: serialise them. */
int  ornith_hip_matvec_noalloc(ornith_hip_ctx *ctx, const ornith_hip_tensor *W,
                               const float *x, float *y, int Tn);

/* oq_dequantize of rows [row0, row0+nrows) (src/ornith_quant.h:64-66). */
/* oq_quantize (src/ornith_quant.h:51-66) on the device: n floats (whole
 * 256-blocks) -> GGUF blocks of Q8_0, Q4_K, Q6_K or IQ2_XXS, byte-identical
 * to the reference's encoders (src/ornith_quant.c:155-175, 451-561, 703-789). */
int  ornith_hip_quantize(ornith_hip_ctx *ctx, uint32_t ggml_type, const float *x, uint64_t n, void *out);
int  ornith_hip_dequant(ornith_hip_ctx *ctx, const ornith_hip_tensor *W,
                        int64_t row0, int64_t nrows, float *out);

/* ---- ornith_moe -------------------------------------------------------------- */

/* ornith_moe_route (src/ornith_moe.h:35-36): top-k indices (ties to the lower
 * index) and softmax weights over the selected logits. */
int  ornith_hip_moe_route(ornith_hip_ctx *ctx, const float *logits, int ne, int k,
                          int32_t *idx, float *w);

/* ---- model and sessions (src/ornith_rforward.h:24-130) ------------------------ */

/* rmodel_load: mmap the GGUF, infer the arch from tensor shapes, upload every
 * tensor once. The mapping is released before returning. */
int  ornith_hip_model_load(ornith_hip_ctx *ctx, const char *gguf_path,
                           ornith_hip_model **out);
/* Build the random-init model of `cfg` directly in HBM (same tensors and
 * values as writing its GGUF with the generator and loading it). */
int  ornith_hip_model_synth(ornith_hip_ctx *ctx, const ornith_hip_gen_cfg *cfg,
                            ornith_hip_model **out);
void ornith_hip_model_free(ornith_hip_model *m);
int  ornith_hip_model_arch(const ornith_hip_model *m, ornith_hip_arch *out);   /* rmodel_arch */
/* weight bytes resident on the device, and the GGUF bytes of one tensor */
uint64_t ornith_hip_model_bytes(const ornith_hip_model *m);
int  ornith_hip_model_tensor_info(const ornith_hip_model *m, const char *name,
                                  uint32_t *type, uint64_t *nbytes, uint64_t *rows,
                                  uint64_t *in);
const ornith_hip_tensor *ornith_hip_model_tensor(const ornith_hip_model *m, const char *name);

/* rmodel_session_new: capacity `cap` positions, Q8 KV cache (ORNITH_KV_Q8=1
 * semantics, src/ornith_attn.h:39-68). With cap >= 64 the first such session
 * of a model also builds the model's prompt tiles (a second copy of the Q4_K /
 * Q6_K tensors the prompt runs on the matrix cores, about their GGUF size;
 * none with ORNITH_HIP_MMQ=0); they are freed with the model. */
int  ornith_hip_session_new(ornith_hip_model *m, int cap, ornith_hip_session **out);
void ornith_hip_session_free(ornith_hip_session *s);                             /* rmodel_session_free */
/* rmodel_session_eval (src/ornith_rforward.c:838-849,933-944): the prompt runs
 * layer by layer over engine chunks of up to 4096 tokens (ORNITH_HIP_PREFILL_CHUNK,
 * a multiple of 32; the chunk length changes no result bit) with batched
 * projections. As in
 * the reference, gated delta-net layers use the chunked scan of 32-token
 * chunks (src/ornith_attn.c:215-349) unless ORNITH_PREFILL_SERIAL=1 selects the
 * token recurrence; either way the results are the reference's bits for that
 * mode. Models past the batched path's limits (a projection wider than 8192,
 * a type without the integer dot) and ORNITH_HIP_PREFILL=0 run the prompt
 * through the token step, i.e. with ORNITH_PREFILL_SERIAL=1 results. */
int  ornith_hip_session_eval(ornith_hip_session *s, const int32_t *tokens, int n);
/* rmodel_session_logits: copies the V next-token logits to `out`. */
int  ornith_hip_session_logits(ornith_hip_session *s, float *out);
int  ornith_hip_session_pos(const ornith_hip_session *s);                        /* rmodel_session_pos */
/* rmodel_session_generate, greedy (sp == NULL): emits up to n_predict tokens
 * into out_tokens, stopping without emitting at the model's eos id. */
int  ornith_hip_session_generate(ornith_hip_session *s, int n_predict,
                                 int32_t *out_tokens, int *n_out);
/* rforward_token for one token (src/ornith_rforward.c:686-706). */
int  ornith_hip_session_step(ornith_hip_session *s, int32_t token);
/* One token step for each of n sessions of the same model at once: token[i]
 * goes through s[i] exactly as ornith_hip_session_step
 * would (rforward_token per session, src/ornith_rforward.c:686-706) and each
 * session's logits are left for ornith_hip_session_logits; next (n entries,
 * may be NULL) receives each session's greedy next token. The projections run
 * over the n sessions together (matmul_batch_q's Tn columns,
 * src/ornith_rforward.c:91-196), so the weights are read once per step. No
 * single reference call does this; it is the multi-sequence form of the token
 * step. Sessions must be distinct, of one KV capacity and attention setting,
 * with every context on the same attention path (all within the exact walk
 * or all past it), and HIP graphs on; other batches return
 * ORNITH_HIP_ERR_UNSUPPORTED. Calls sharing a session or a first session must
 * not overlap (the first session holds the step's buffers).
 * Currently switched off: every call returns ORNITH_HIP_ERR_UNSUPPORTED (batch
 * runs have faulted the GPU with the cause not found). */
int  ornith_hip_batch_step(ornith_hip_session **s, int n, const int32_t *tokens, int32_t *next);

/* rmodel_session_save (src/ornith_rforward.c:1019-1075): the session as an
 * ORNSESS v1 file (Q8 KV cache), byte-identical to the reference's file for
 * the same state. */
int  ornith_hip_session_save(ornith_hip_session *s, const char *path);
/* rmodel_session_load (src/ornith_rforward.c:1077-1171): a new session from
 * an ORNSESS v1 file, capacity pos + extra_cap; the same errors as the
 * reference (bad magic or version, fingerprint mismatch, truncation, prefix
 * hash), plus ORNITH_HIP_ERR_UNSUPPORTED for an f32 KV cache. */
int  ornith_hip_session_load(ornith_hip_model *m, const char *path, int extra_cap, ornith_hip_session **out);

/* Session state in the reference's host layouts (src/ornith_rforward.c:986-1171
 * snapshot contents): delta state [nv][dv][dk]; conv window [(K-1)][Cc] oldest
 * first; Q8 KV codes [len][nkv][hd] and scales [len][nkv]. */
int  ornith_hip_session_get_delta(ornith_hip_session *s, int layer, float *S);
int  ornith_hip_session_get_conv(ornith_hip_session *s, int layer, float *win);
int  ornith_hip_session_get_kv(ornith_hip_session *s, int layer, int8_t *Kq,
                               float *Ks, int8_t *Vq, float *Vs);
/* The attention of the last full-attention layer as the most recent
 * evaluation left it (a parity hook, no reference twin; the inputs and output
 * of ornith_gqa_step inside full_attn, src/ornith_rforward.c:419-455,
 * src/ornith_attn.c:87-149): row < 0, the decode step's; row >= 0, that row of
 * the most recent prompt chunk. q: query heads after q_norm + RoPE [nh*hd];
 * gate [nh*hd]; o = attention * sigmoid(gate) [nh*hd], before attn_output's
 * Q8_K; *pos: the row's position. Needs a model whose last layer is
 * full attention. */
int  ornith_hip_session_get_attn(ornith_hip_session *s, int row, float *q, float *gate, float *o,
                                 int32_t *pos);

/* ---- measurement (no reference twin) -------------------------------------------- */

/* Time n_steps greedy decode steps already resident on the device (back to
 * back, the next token chosen on the device) with HIP events on the session
 * stream; *ms = total elapsed. Advances the session. A decode step replays
 * HIP graphs of one launch per operation; with ORNITH_HIP_STEP=1 in the
 * environment it runs as two launches of the persistent step kernel (body,
 * head) instead (the same for eval and generate). */
int  ornith_hip_session_time_decode(ornith_hip_session *s, int n_steps, float *ms);
/* Run one greedy decode step eagerly with HIP events around every kernel
 * launch: kinds[i] (0 matvec with Q4_K weights, 1 rmsnorm+Q8_K, 2 SwiGLU+Q8_K,
 * 3 embed, 4 delta step, 5 attn prep, 6 attn scores (exact regime), 7 attn
 * walk (exact regime), 8 router, 9 MoE combine, 10 argmax, 11 advance, 12
 * fused MoE down + combine, 13 flash attention chunks, 14 flash merge, 15
 * matvec Q6_K, 16 matvec Q8_0, 17 matvec of mixed types, 20 attention of the
 * one-launch form, 21 matvec of Q4_K and Q6_K segments, 22 delta step and its
 * output projection in one launch), algorithmic HBM bytes[i] and ms[i].
 * Advances the session by one position. */
int  ornith_hip_session_profile_step(ornith_hip_session *s, int max_launches, int32_t *kinds,
                                     double *bytes, float *ms, int *n_launches);
/* Replay, back to back, the launches of one kind (numbering as above) that a
 * decode step makes, `reps` times, between two HIP events on the session
 * stream: *us_per_launch = mean time per launch, *bytes_per_launch = mean
 * algorithmic HBM bytes, *launches_per_step = launches of that kind per step.
 * Kinds 18 and 19 are the persistent step kernel's body and head launches
 * (all operations of a step at the current position). The other kernels of
 * the step do not run, so the session's state is meaningless afterwards:
 * measurement only, free the session after. */
int  ornith_hip_session_time_kind(ornith_hip_session *s, int kind, int reps, float *us_per_launch,
                                  double *bytes_per_launch, int *launches_per_step);
/* One step-kernel body launch at the current position (the position does not
 * advance; measurement only, like time_kind) with workgroup 0's real-time
 * clock read after every grid barrier: per phase (operation) its kind
 * (numbering as above, -1 for the second stage of a two-stage operation),
 * algorithmic bytes and us from the previous barrier to its own. */
int  ornith_hip_session_profile_phases(ornith_hip_session *s, int max_phases, int32_t *kinds,
                                       double *bytes, float *us, int *n_phases);
/* Measurement (no reference twin): one run of the decode step as a single
 * persistent launch with clocks, not advancing the session: per operation
 * its kind (0 embed, 1 matvec, 2 delta-net, 3 GQA prep, 4 attention,
 * 5 attention merge, 6 MoE down, 7 greedy token) and the earliest / latest
 * time a workgroup was done with it, in microseconds from the launch's start.
 * ORNITH_HIP_ERR_UNSUPPORTED when the model has no such launch. */
int  ornith_hip_session_profile_decode(ornith_hip_session *s, int max_ops, int32_t *kinds,
                                       float *us_first, float *us_last, int *n_ops);
/* Measurement: the sub-phase clocks of operation `op` of that launch, 8 per
 * workgroup (start, weights requested, inputs arrived, activation arrived,
 * prologue done, done; -1 where not recorded), microseconds from the start. */
int  ornith_hip_session_profile_decode_op(ornith_hip_session *s, int op, float *us, int max_groups,
                                          int *grid_out);
/* Time `iters` launches of one matvec of W (activation already quantised on
 * the device) with HIP events on the context stream; *ms = mean per launch. */
int  ornith_hip_time_matvec(ornith_hip_ctx *ctx, const ornith_hip_tensor *W, int iters,
                            float *ms);
/* Cold-cache variant: n weight tensors of one type and shape (distinct
 * copies, together larger than the device caches) take turns; `iters`
 * launches in that round-robin order are captured as one HIP graph and
 * replayed between HIP events; *ms = mean per launch. No reference twin
 * (measurement only). */
int  ornith_hip_time_matvec_set(ornith_hip_ctx *ctx, const ornith_hip_tensor *const *W, int n, int iters,
                                float *ms);

#ifdef __cplusplus
}
#endif
#endif
