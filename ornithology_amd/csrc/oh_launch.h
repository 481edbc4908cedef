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
hipError_t oh_launch_mv_down(const oh_mvdown *D, int blocks, int threads, int lds_bytes, hipStream_t st);
hipError_t oh_launch_rmsnorm_q8k(const float *x, const float *norm_w, float eps, int n,
                                 float *xn_out, int8_t *qs, float *d, int16_t *bs, hipStream_t st);
hipError_t oh_launch_swiglu_q8k(const float *g, const float *u, int n, int count, float *h_out,
                                int8_t *qs, float *d, int16_t *bs, hipStream_t st);
hipError_t oh_launch_dequant(const uint8_t *A, const uint8_t *B, const uint8_t *C, int type, int in,
                             int64_t row0, int64_t nrows, float *out, hipStream_t st);
hipError_t oh_launch_embed(const uint8_t *A, const uint8_t *B, const uint8_t *C, int type, int in,
                           const int32_t *toks, const int32_t *io_pos, float *x, hipStream_t st);
hipError_t oh_launch_delta_step(int dk, const float *cat, const float *ab, const float *gate,
                                const float *conv_w, float *conv_state, const float *ssm_a,
                                const float *dt_bias, float *S, float *out, float *out_gate, double *out_runs,
                                const int32_t *io_pos, int nk, int nv, int K, int cc, float out_scale,
                                hipStream_t st);
hipError_t oh_launch_attn_prep(const float *qproj, const float *kin, const float *vin,
                               const float *q_norm, const float *k_norm, const float2 *rope,
                               float *qr, float *gate, uint32_t *Kt, float *Ks, int8_t *Vq,
                               float *Vs, const int32_t *io_pos, int nh, int nkv, int hd,
                               int rot, int cap, float eps, hipStream_t st);
hipError_t oh_launch_attn_scores(const float *qr, const uint32_t *Kt, const float *Ks,
                                 float *scores, const int32_t *io_pos, int nh, int nkv, int hd,
                                 int cap, float scale, int exact_max, hipStream_t st);
hipError_t oh_launch_attn_out(const float *scores, const int8_t *Vq, const float *Vs, const float *gate,
                              float *out, const int32_t *io_pos, int nh, int nkv, int hd, int cap,
                              int exact_max, hipStream_t st);
// flash decoding past exact_max positions: chunk partials, then their merge
int oh_flash_lds_bytes(int nh, int nkv, int hd);
int oh_flash_chunk(void);
hipError_t oh_launch_attn_flash(const float *qr, const uint32_t *Kt, const float *Ks, const int8_t *Vq,
                                const float *Vs, float *part_o, float *part_ml, const int32_t *io_pos,
                                int nh, int nkv, int hd, int cap, float scale, int exact_max, hipStream_t st);
hipError_t oh_launch_attn_combine(const float *part_o, const float *part_ml, const float *gate, float *out,
                                  const int32_t *io_pos, int nh, int nkv, int hd, int cap, int exact_max,
                                  hipStream_t st);
hipError_t oh_launch_moe_route(const float *logits, int ne, int k, const float *shgate_logit,
                               int32_t *idx, float *w, float *shgate, hipStream_t st);
hipError_t oh_launch_moe_combine(float *x, const float *o, const float *w, int k, int H,
                                 const float *so, const float *shgate, hipStream_t st);
hipError_t oh_launch_argmax(const float *v, int n, float *tmp_v, int *tmp_i, int nblk,
                            int32_t *toks, const int32_t *io_pos, int32_t *io_best,
                            hipStream_t st);
hipError_t oh_launch_advance(int32_t *io_pos, hipStream_t st);
hipError_t oh_launch_fill_gauss(uint64_t key, float sigma, float *dst, int64_t n, hipStream_t st);
hipError_t oh_launch_fill_uniform(uint64_t key, float lo, float hi, float *dst, int64_t n, hipStream_t st);
hipError_t oh_launch_encode(const float *x, int type, int64_t nblk, uint8_t *A, uint8_t *B, uint8_t *C,
                            hipStream_t st);
}

// blocks used by the argmax's first stage (the caller sizes tmp_v/tmp_i)
#define OH_ARGMAX_BLOCKS 256
