// oh_kernels.hip - the single device translation unit of the engine: the
// kernels of oh_mv.hip and oh_layers.hip plus their host launchers.
#include "oh_mv.hip"
#include "oh_layers.hip"
#include "oh_synth.hip"
#include "oh_step.hip"
#include "oh_launch.h"

extern "C" {

hipError_t oh_launch_matvec(const oh_mvlaunch *L, int tk, int lds_bytes, hipStream_t st) {
    if (L->total_blocks <= 0) return hipSuccess;
    void (*k)(oh_mvlaunch) = tk == OH_Q4_K ? oh_k_mv_q4k : tk == OH_Q6_K ? oh_k_mv_q6k
                           : tk == OH_Q8_0 ? oh_k_mv_q80 : oh_k_mv_mixed;
    hipLaunchKernelGGL(k, dim3(L->total_blocks), dim3(256), (size_t)lds_bytes, st, *L);
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


hipError_t oh_launch_op(const oh_op *op, const int32_t *io, hipStream_t st) {
    if (op->nvb <= 0) return hipSuccess;
    const dim3 g(op->nvb), b256(256);
    switch (op->kind) {
    case OH_OP_MV:
        return oh_launch_matvec(&op->u.mv, op->tk, op->lds, st);
    case OH_OP_MV_DOWN: {
        const int ns = op->u.down.k + (op->u.down.sA ? 1 : 0);
        hipLaunchKernelGGL(oh_k_mv_down, g, dim3(64 * ns), (size_t)op->lds, st, op->u.down);
        break;
    }
    case OH_OP_EMBED: hipLaunchKernelGGL(oh_k_embed, g, b256, 0, st, op->u.embed, io); break;
    case OH_OP_DELTA:
        if (op->u.delta.K > 8) return hipErrorInvalidValue;
        if (op->u.delta.dk == 128) {
            if (op->u.delta.K <= 4) hipLaunchKernelGGL((oh_k_delta_step<128, 4>), g, dim3(64), 0, st, op->u.delta, io);
            else hipLaunchKernelGGL((oh_k_delta_step<128, 8>), g, dim3(64), 0, st, op->u.delta, io);
        } else if (op->u.delta.dk == 64) {
            if (op->u.delta.K <= 4) hipLaunchKernelGGL((oh_k_delta_step<64, 4>), g, dim3(64), 0, st, op->u.delta, io);
            else hipLaunchKernelGGL((oh_k_delta_step<64, 8>), g, dim3(64), 0, st, op->u.delta, io);
        } else {
            return hipErrorInvalidValue;
        }
        break;
    case OH_OP_ATTN_PREP: hipLaunchKernelGGL(oh_k_attn_prep, g, b256, 0, st, op->u.prep, io); break;
    case OH_OP_ATTN_MAIN: hipLaunchKernelGGL(oh_k_attn_main, g, b256, (size_t)op->lds, st, op->u.attn, io); break;
    case OH_OP_ATTN_COMBINE: hipLaunchKernelGGL(oh_k_attn_combine, g, b256, 0, st, op->u.attn, io); break;
    case OH_OP_MOE_COMBINE: hipLaunchKernelGGL(oh_k_moe_combine, g, b256, 0, st, op->u.comb); break;
    case OH_OP_ARGMAX1: hipLaunchKernelGGL(oh_k_argmax1, g, b256, 0, st, op->u.am); break;
    case OH_OP_ARGMAX2: hipLaunchKernelGGL(oh_k_argmax2, dim3(1), dim3(64), 0, st, op->u.am, io); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// query heads per flash block: up to four of a KV head's group
int oh_flash_hb(int nh, int nkv) { return nh / nkv >= 4 ? 4 : (nh / nkv >= 2 ? 2 : 1); }

int oh_flash_lds_bytes(int nh, int nkv, int hd) {
    const int HB = oh_flash_hb(nh, nkv);
    return HB * (hd + 16) * 4 + kFlashCh * (hd / 4 + 1) * 4 + 16 + (kFlashCh / 16) * hd * 16 + HB * kFlashCh * 4 +
           2 * kFlashCh * 4;
}
int oh_flash_chunk(void) { return kFlashCh; }

// exact attention walk: the scores of a block's 256/hd heads in LDS
int oh_exact_lds_bytes(int hd, int exact_max) {
    const int lim = exact_max < kExactMax ? (exact_max > 0 ? exact_max : 0) : kExactMax;
    return (256 / hd) * lim * 4;
}

// delta step LDS of the working wave (step kernel: dynamic LDS)
int oh_delta_lds_bytes(int dk) { return (2 * dk + 64 * (dk + 4)) * 4; }

hipError_t oh_step_blocks_per_cu(int lds_bytes, int *blocks) {
    hipError_t e = hipFuncSetAttribute((const void *)oh_k_step, hipFuncAttributeMaxDynamicSharedMemorySize, lds_bytes);
    if (e != hipSuccess) return e;
    return hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks, (const void *)oh_k_step, 256, (size_t)lds_bytes);
}

hipError_t oh_launch_step(const oh_op *prog, int nops, int32_t *io, unsigned *ctrs, int epoch_slot, int advance,
                          uint64_t *ts, int grid, int lds_bytes, hipStream_t st) {
    void *args[] = {(void *)&prog, (void *)&nops, (void *)&io, (void *)&ctrs, (void *)&epoch_slot,
                    (void *)&advance, (void *)&ts};
    return hipLaunchCooperativeKernel((const void *)oh_k_step, dim3(grid), dim3(256), args, (size_t)lds_bytes, st);
}

hipError_t oh_launch_moe_route(const float *logits, int ne, int k, const float *shgate_logit,
                               int32_t *idx, float *w, float *shgate, hipStream_t st) {
    hipLaunchKernelGGL(oh_k_moe_route, dim3(1), dim3(64), 0, st, logits, ne, k, shgate_logit, idx, w, shgate);
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
