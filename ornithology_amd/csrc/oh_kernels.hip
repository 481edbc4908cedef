// oh_kernels.hip - the single device translation unit of the engine: the
// kernels of oh_mv.hip and oh_layers.hip plus their host launchers.
#include "oh_mv.hip"
#include "oh_layers.hip"
#include "oh_synth.hip"
#include "oh_launch.h"

extern "C" {

hipError_t oh_launch_matvec(const oh_mvlaunch *L, int tk, int lds_bytes, hipStream_t st) {
    if (L->total_blocks <= 0) return hipSuccess;
    void (*k)(oh_mvlaunch) = tk == OH_Q4_K ? oh_k_mv_q4k : tk == OH_Q6_K ? oh_k_mv_q6k
                           : tk == OH_Q8_0 ? oh_k_mv_q80 : oh_k_mv_mixed;
    hipLaunchKernelGGL(k, dim3(L->total_blocks), dim3(256), (size_t)lds_bytes, st, *L);
    return hipGetLastError();
}

hipError_t oh_launch_mv_down(const oh_mvdown *D, int blocks, int threads, int lds_bytes, hipStream_t st) {
    if (blocks <= 0) return hipSuccess;
    hipLaunchKernelGGL(oh_k_mv_down, dim3(blocks), dim3(threads), (size_t)lds_bytes, st, *D);
    return hipGetLastError();
}

hipError_t oh_launch_rmsnorm_q8k(const float *x, const float *norm_w, float eps, int n,
                                 float *xn_out, int8_t *qs, float *d, int16_t *bs, hipStream_t st) {
    hipLaunchKernelGGL(oh_k_rmsnorm_q8k, dim3(1), dim3(256), 0, st, x, norm_w, eps, n, xn_out, qs, d, bs);
    return hipGetLastError();
}

hipError_t oh_launch_swiglu_q8k(const float *g, const float *u, int n, int count, float *h_out,
                                int8_t *qs, float *d, int16_t *bs, hipStream_t st) {
    hipLaunchKernelGGL(oh_k_swiglu_q8k, dim3(count), dim3(256), 0, st, g, u, n, h_out, qs, d, bs);
    return hipGetLastError();
}

hipError_t oh_launch_dequant(const uint8_t *A, const uint8_t *B, const uint8_t *C, int type, int in,
                             int64_t row0, int64_t nrows, float *out, hipStream_t st) {
    const int64_t n = nrows * in;
    int64_t blocks = (n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL(oh_k_dequant, dim3((unsigned)blocks), dim3(256), 0, st, A, B, C, type, in, row0, nrows, out);
    return hipGetLastError();
}

hipError_t oh_launch_embed(const uint8_t *A, const uint8_t *B, const uint8_t *C, int type, int in,
                           const int32_t *toks, const int32_t *io_pos, float *x, hipStream_t st) {
    hipLaunchKernelGGL(oh_k_embed, dim3((in + 255) / 256), dim3(256), 0, st, A, B, C, type, in, toks, io_pos, x);
    return hipGetLastError();
}

hipError_t oh_launch_delta_step(int dk, const float *cat, const float *ab, const float *gate,
                                const float *conv_w, float *conv_state, const float *ssm_a,
                                const float *dt_bias, float *S, float *out, float *out_gate, double *out_runs,
                                const int32_t *io_pos, int nk, int nv, int K, int cc, float out_scale,
                                hipStream_t st) {
    if (dk == 128) {
        hipLaunchKernelGGL(oh_k_delta_step<128>, dim3(nv * 2), dim3(64), 0, st, cat, ab, gate, conv_w, conv_state,
                           ssm_a, dt_bias, S, out, out_gate, out_runs, io_pos, nk, nv, K, cc, out_scale);
    } else if (dk == 64) {
        hipLaunchKernelGGL(oh_k_delta_step<64>, dim3(nv), dim3(64), 0, st, cat, ab, gate, conv_w, conv_state,
                           ssm_a, dt_bias, S, out, out_gate, out_runs, io_pos, nk, nv, K, cc, out_scale);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t oh_launch_attn_prep(const float *qproj, const float *kin, const float *vin,
                               const float *q_norm, const float *k_norm, const float2 *rope,
                               float *qr, float *gate, uint32_t *Kt, float *Ks, int8_t *Vq,
                               float *Vs, const int32_t *io_pos, int nh, int nkv, int hd,
                               int rot, int cap, float eps, hipStream_t st) {
    hipLaunchKernelGGL(oh_k_attn_prep, dim3(nh + nkv), dim3(256), 0, st, qproj, kin, vin, q_norm, k_norm,
                       rope, qr, gate, Kt, Ks, Vq, Vs, io_pos, nh, nkv, hd, rot, cap, eps);
    return hipGetLastError();
}

hipError_t oh_launch_attn_scores(const float *qr, const uint32_t *Kt, const float *Ks,
                                 float *scores, const int32_t *io_pos, int nh, int nkv, int hd,
                                 int cap, float scale, int exact_max, hipStream_t st) {
    hipLaunchKernelGGL(oh_k_attn_scores, dim3(nh, (cap + 255) / 256), dim3(256), 0, st, qr, Kt, Ks,
                       scores, io_pos, nh, nkv, hd, cap, scale, exact_max);
    return hipGetLastError();
}

hipError_t oh_launch_attn_out(const float *scores, const int8_t *Vq, const float *Vs, const float *gate,
                              float *out, const int32_t *io_pos, int nh, int nkv, int hd, int cap,
                              int exact_max, hipStream_t st) {
    hipLaunchKernelGGL(oh_k_attn_out, dim3(nh / (256 / hd)), dim3(256), 0, st, scores, Vq, Vs, gate, out,
                       io_pos, nh, nkv, hd, cap, exact_max);
    return hipGetLastError();
}

// query heads per flash block: two (one when the group has a single head)
static int flash_hb(int nh, int nkv) { return nh / nkv >= 2 ? 2 : 1; }

int oh_flash_lds_bytes(int nh, int nkv, int hd) {
    const int HB = flash_hb(nh, nkv);
    return HB * (hd + 16) * 4 + kFlashCh * (hd / 4 + 1) * 4 + 16 + (kFlashCh / 16) * hd * 16 + HB * kFlashCh * 4 +
           2 * kFlashCh * 4;
}
int oh_flash_chunk(void) { return kFlashCh; }

hipError_t oh_launch_attn_flash(const float *qr, const uint32_t *Kt, const float *Ks, const int8_t *Vq,
                                const float *Vs, float *part_o, float *part_ml, const int32_t *io_pos,
                                int nh, int nkv, int hd, int cap, float scale, int exact_max, hipStream_t st) {
    const int HB = flash_hb(nh, nkv), G = nh / nkv;
    void (*k)(const float *, const uint32_t *, const float *, const int8_t *, const float *, float *, float *,
              const int32_t *, int, int, int, int, float, int) = HB == 2 ? oh_k_attn_flash<2> : oh_k_attn_flash<1>;
    hipLaunchKernelGGL(k, dim3(nkv * (G / HB), (cap + kFlashCh - 1) / kFlashCh), dim3(256),
                       (size_t)oh_flash_lds_bytes(nh, nkv, hd), st, qr, Kt, Ks, Vq, Vs, part_o, part_ml, io_pos,
                       nh, nkv, hd, cap, scale, exact_max);
    return hipGetLastError();
}

hipError_t oh_launch_attn_combine(const float *part_o, const float *part_ml, const float *gate, float *out,
                                  const int32_t *io_pos, int nh, int nkv, int hd, int cap, int exact_max,
                                  hipStream_t st) {
    hipLaunchKernelGGL(oh_k_attn_combine, dim3(nh, hd / 64), dim3(256), 0, st, part_o, part_ml, gate, out,
                       io_pos, nh, nkv, hd, cap, exact_max);
    return hipGetLastError();
}

hipError_t oh_launch_moe_route(const float *logits, int ne, int k, const float *shgate_logit,
                               int32_t *idx, float *w, float *shgate, hipStream_t st) {
    hipLaunchKernelGGL(oh_k_moe_route, dim3(1), dim3(64), 0, st, logits, ne, k, shgate_logit, idx, w, shgate);
    return hipGetLastError();
}

hipError_t oh_launch_moe_combine(float *x, const float *o, const float *w, int k, int H,
                                 const float *so, const float *shgate, hipStream_t st) {
    hipLaunchKernelGGL(oh_k_moe_combine, dim3((H + 255) / 256), dim3(256), 0, st, x, o, w, k, H, so, shgate);
    return hipGetLastError();
}

hipError_t oh_launch_argmax(const float *v, int n, float *tmp_v, int *tmp_i, int nblk,
                            int32_t *toks, const int32_t *io_pos, int32_t *io_best,
                            hipStream_t st) {
    hipLaunchKernelGGL(oh_k_argmax1, dim3(nblk), dim3(256), 0, st, v, n, tmp_v, tmp_i);
    hipLaunchKernelGGL(oh_k_argmax2, dim3(1), dim3(64), 0, st, tmp_v, tmp_i, nblk, toks, io_pos, io_best);
    return hipGetLastError();
}

hipError_t oh_launch_fill_gauss(uint64_t key, float sigma, float *dst, int64_t n, hipStream_t st) {
    int64_t blocks = (n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(oh_k_fill_gauss, dim3((unsigned)(blocks > 0 ? blocks : 1)), dim3(256), 0, st, key, sigma, dst, n);
    return hipGetLastError();
}

hipError_t oh_launch_fill_uniform(uint64_t key, float lo, float hi, float *dst, int64_t n, hipStream_t st) {
    int64_t blocks = (n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(oh_k_fill_uniform, dim3((unsigned)(blocks > 0 ? blocks : 1)), dim3(256), 0, st, key, lo, hi, dst, n);
    return hipGetLastError();
}

hipError_t oh_launch_encode(const float *x, int type, int64_t nblk, uint8_t *A, uint8_t *B, uint8_t *C,
                            hipStream_t st) {
    if (nblk <= 0) return hipSuccess;
    hipLaunchKernelGGL(oh_k_encode, dim3((unsigned)((nblk + 255) / 256)), dim3(256), 0, st, x, type, nblk, A, B, C);
    return hipGetLastError();
}

hipError_t oh_launch_advance(int32_t *io_pos, hipStream_t st) {
    hipLaunchKernelGGL(oh_k_advance, dim3(1), dim3(1), 0, st, io_pos);
    return hipGetLastError();
}

} // extern "C"
