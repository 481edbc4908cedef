// oh_launch.h - host-side launchers for the kernels of oh_kernels.hip.
// Every launcher enqueues on `st` and returns the launch status; none of them
// synchronises or allocates, so the engine can capture them into a HIP graph.
#pragma once
#include <hip/hip_runtime.h>
#include "oh_types.h"

extern "C" {
// tk: the integer-path type every segment has (OH_Q4_K/OH_Q6_K/OH_Q8_0), or -1
// for a launch that mixes types or has fallback segments
hipError_t oh_launch_matvec(const oh_mvlaunch *L, int tk, int lds_bytes, hipStream_t st);
hipError_t oh_launch_delta_mv(const oh_op_dmv *a, int tk, int lds_bytes, const int32_t *io, hipStream_t st);
// batched matvec (grid: row blocks x groups) and its LDS column tile
hipError_t oh_launch_mvb(const oh_mvbatch *B, int groups, hipStream_t st);
int oh_mvb_tcol(int nb);
// RMSNorm (norm_w non-null) + Q8_K of `rows` vectors of n <= 8192 elements
// bp: also the Q8_K pair-sum bytes (the matrix-core product's min term);
// swiglu: x holds rows of [gate | up] (2n) and the vector is silu(gate) * up
hipError_t oh_launch_norm_q8k_rows(const float *x, const float *norm_w, float eps, int n, int rows, float *xn_out,
                                   int8_t *qs, float *d, int16_t *bs, hipStream_t st, int8_t *bp = nullptr,
                                   int swiglu = 0);
// prefill (layer-major over T tokens)
hipError_t oh_launch_embed_rows(const oh_op_embed *a, int base, int T, hipStream_t st);
hipError_t oh_launch_conv_rows(const float *cat, const float *conv_w, float *conv_state, float *out, float *stage,
                               int T, int base, int cc, int K, hipStream_t st);
hipError_t oh_launch_qk_gates_rows(int dk, const float *conv, const float *A, const float *Bg, const float *ssm_a,
                                   const float *dt_bias, float *qn, float *kn, float *al, float *be, int T, int nk,
                                   int nv, int cc, hipStream_t st);
hipError_t oh_launch_delta_scan(int dk, const float *qn, const float *kn, const float *conv, const float *al,
                                const float *be, float *S, float *out, int T, int nk, int nv, int cc,
                                float out_scale, hipStream_t st);
// the reference's chunked delta scan (grams per key head and chunk, then the scan)
int oh_delta_grams_floats(int T, int nk);
// wy non-null: the matrix-core WY form over that scratch (oh_delta_wy_floats)
hipError_t oh_launch_delta_chunked(int dk, const float *qn, const float *kn, const float *conv, const float *al,
                                   const float *be, float *grams, float *wy, float *S, float *out, int T, int nk,
                                   int nv, int cc, float out_scale, hipStream_t st);
int oh_delta_wy_floats(int T, int nv, int dk);
// z: the raw attention gate (silu applied here)
// gated per-head RMSNorm (sums of squares per 64-element run, as the decode
// step forms them) + Q8_K of T vectors
hipError_t oh_launch_gnorm_q8k_rows(const float *x, const float *z, const float *w, float eps, int n, int gdim,
                                    int T, int8_t *qs, float *d, int16_t *bs, hipStream_t st, int8_t *bp = nullptr);
// Q4_K x Q8_K products on the matrix cores: rows % 128 == 0; dense (ncol
// columns) or grouped (items from oh_launch_mmq_items, at most max_items);
// pair: a second weight set (A2/B2) for rows [rows, 2 rows)
hipError_t oh_launch_mmq(const oh_mmq *M, int max_items, int pair, hipStream_t st);
hipError_t oh_launch_mmq_items(const int32_t *cnt, int ne, int32_t *items, hipStream_t st);
bool oh_mmq_can(uint32_t type, int rows, int in);
// the prompt tiles of a Q4_K (P = 8 code pieces) or Q6_K (P = 12) tensor of
// `rows` rows (a multiple of 64) from its A and B planes
hipError_t oh_launch_mmq_tiles(const uint8_t *A, const uint8_t *B, uint8_t *PA, uint8_t *PB, int64_t rows,
                               int nb, int P, hipStream_t st);
// decode of n sessions at once: the decode bodies, one grid row per session,
// descriptors and positions in device arrays of n
hipError_t oh_launch_delta_batch(const oh_op_delta *ops, const int32_t *pos, int n, int dk, int K, int nv,
                                 hipStream_t st);
hipError_t oh_launch_prep_batch(const oh_op_prep *ops, const int32_t *pos, int n, int nh, int nkv, hipStream_t st);
hipError_t oh_launch_attn_batch(const oh_op_attn *ops, const int32_t *pos, int n, int nvb_main, int lds, int nh,
                                int hd, hipStream_t st);
// greedy token per row; with scratch bv/bi (rows x OH_ARGMAX_BLOCKS) in two stages
hipError_t oh_launch_argmax_rows(const float *v, int n, int rows, int32_t *out, hipStream_t st,
                                 float *bv = nullptr, int *bi = nullptr);
hipError_t oh_launch_batch_tokens(int32_t *const *toks, const int32_t *pos, const int32_t *tok, const int32_t *next,
                                  int n, hipStream_t st);
hipError_t oh_launch_prep_rows(const oh_op_prep *a, int base, int T, hipStream_t st);
hipError_t oh_launch_attn_rows(const oh_op_attn *a, int base, int t0, int n, size_t po_stride, size_t pml_stride,
                               hipStream_t st);
// the exact walk alone for n rows t0.. that are all inside it (one launch)
hipError_t oh_launch_attn_exact_rows(const oh_op_attn *a, int base, int t0, int n, hipStream_t st);
hipError_t oh_launch_route_rows(const float *logits, int ne, int k, const float *shl, int32_t *idx, float *w,
                                float *shg, int T, hipStream_t st);
hipError_t oh_launch_group_pairs(const int32_t *idx, int npairs, int32_t *cnt, int ne, int32_t *list, int lstride,
                                 int32_t *err, hipStream_t st);
hipError_t oh_launch_moe_combine_rows(float *x, const float *o, const float *w, int k, int H, const float *so,
                                      const float *shgate, int T, hipStream_t st);
hipError_t oh_launch_rmsnorm_q8k(const float *x, const float *norm_w, float eps, int n,
                                 float *xn_out, int8_t *qs, float *d, int16_t *bs, hipStream_t st);
hipError_t oh_launch_swiglu_q8k(const float *g, const float *u, int n, int count, float *h_out,
                                int8_t *qs, float *d, int16_t *bs, hipStream_t st);
hipError_t oh_launch_dequant(const uint8_t *A, const uint8_t *B, const uint8_t *C, int type, int in,
                             int64_t row0, int64_t nrows, float *out, hipStream_t st);
// the fused MoE down + combine for ntok tokens (grid y = token)
hipError_t oh_launch_mv_down_rows(const oh_mvdown *D, int nvb, int ntok, int lds, hipStream_t st);
// one operation of the token step as its own launch (io: position word)
hipError_t oh_launch_op(const oh_op *op, const int32_t *io, hipStream_t st);
// flash decoding past exact_max positions: query heads per block, LDS bytes,
// chunk length
int oh_flash_hb(int nh, int nkv);
int oh_flash_form(int nh, int nkv, int hd, int mfma);
int oh_flash_nvb(int nh, int nkv, int cap, int hb);
int oh_flash_form_lds(int nh, int nkv, int hd, int hb);
int oh_flash_slots(int cap);
int oh_flash_parts(int T, int cap, int hb);
int oh_flash_lds_bytes(int nh, int nkv, int hd);
int oh_flash_chunk(void);
int oh_delta_lds_bytes(int dk);
int oh_exact_lds_bytes(int hd, int exact_max);
int oh_exact_limit(int exact_max, int hd);
int oh_delta16_lds_bytes(int dk);
// prompt attention on the matrix cores for the nt tokens tf0.. of a prefill
// chunk (positions base + t, contexts past the exact walk); supported shapes
hipError_t oh_launch_attn_mfma_rows(const oh_op_attn *a, int base, int tf0, int nt, hipStream_t st);
int oh_attn_mfma_supported(int hd, int nh, int nkv);
// persistent step kernel: resident 256-thread blocks per CU at this dynamic
// LDS size, and the cooperative launch of a program (prog in device memory)
hipError_t oh_step_blocks_per_cu(int lds_bytes, int *blocks);
hipError_t oh_launch_step(const oh_op *prog, int nops, int32_t *io, unsigned *ctrs, int epoch_slot, int advance,
                          uint64_t *ts, int grid, int lds_bytes, hipStream_t st);
// the decode step as one persistent launch (oh_decode.hip): resident
// 256-thread blocks per CU at this dynamic LDS size, and the cooperative
// launch of a program (prog in device memory)
hipError_t oh_decode_blocks_per_cu(int lds_bytes, int *blocks);
// ts (optional): per-workgroup start and end-of-operation clocks, (nops + 1) * grid;
// ts2 (optional): operation prof_op's sub-phase clocks, 8 per workgroup
hipError_t oh_launch_decode(const oh_dop *prog, int nops, int32_t *io, int advance, int grid, int lds_bytes,
                            hipStream_t st, uint64_t *ts = nullptr, int prof_op = -1, uint64_t *ts2 = nullptr);
hipError_t oh_launch_moe_route(const float *logits, int ne, int k, const float *shgate_logit,
                               int32_t *idx, float *w, float *shgate, hipStream_t st);
hipError_t oh_launch_advance(int32_t *io_pos, hipStream_t st);
hipError_t oh_launch_fill_gauss(uint64_t key, float sigma, float *dst, int64_t n, hipStream_t st);
hipError_t oh_launch_fill_uniform(uint64_t key, float lo, float hi, float *dst, int64_t n, hipStream_t st);
hipError_t oh_launch_encode(const float *x, int type, int64_t nblk, uint8_t *A, uint8_t *B, uint8_t *C,
                            hipStream_t st);
}


