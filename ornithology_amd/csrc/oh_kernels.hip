// oh_kernels.hip - the main device translation unit of the engine: the
// per-operation kernels and their host launchers. The two persistent decode
// kernels sit in translation units of their own (oh_kernels_step.hip,
// oh_kernels_decode.hip) so that the three compile in parallel.
#include "oh_mv.hip"
#include "oh_layers.hip"
#include "oh_synth.hip"
#include "oh_prefill.hip"
#include "oh_mmq.hip"
#include "oh_batch.hip"
#include "oh_attn_mfma.hip"
#include "oh_delta_mfma.hip"
#include "oh_launch.h"

// The graph step's delta step and the projection of its output in one launch
// (oh_op_dmv): workgroups [0, nd) run the delta step and count their
// arrival once their outputs (device-scope stores) are complete; the others
// are the projection's matvec workgroups behind the arrival wait.
template <int DK, int KMAX, int TK>
__global__ void __launch_bounds__(256) oh_k_delta_mv(oh_op_dmv a, const int32_t *io) {
    const int vb = (int)blockIdx.x;
    if (vb < a.nd) {
        __shared__ __align__(16) float lds[delta16_lds_floats(DK)];
        NoWait w;
        delta16_body<DK, KMAX>(a.d, vb, io[OH_IO_POS], lds, w);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (tid_x() == 0) __hip_atomic_fetch_add(a.arr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    CtrWait w{a.arr, a.nd, a.mv.rio + OH_IO_ERR, false, true};
    mv_body<TK>(a.mv, vb - a.nd, w);
    fused_depart(a.arr, a.dep, a.mv.total_blocks);
}

extern "C" {

// delta step + projection: head dim 128, conv kernels up to 8, a Q4_K or
// Q6_K projection (the host builds the fused op only for these)
hipError_t oh_launch_delta_mv(const oh_op_dmv *a, int tk, int lds_bytes, const int32_t *io, hipStream_t st) {
    if (a->d.dk != 128 || a->d.K > 8 || (tk != OH_Q4_K && tk != OH_Q6_K) || a->mv.rio == nullptr || lds_bytes > 65536)
        return hipErrorInvalidValue;
    const dim3 g(a->nd + a->mv.total_blocks), b(256);
    if (tk == OH_Q4_K) {
        if (a->d.K <= 4) hipLaunchKernelGGL((oh_k_delta_mv<128, 4, OH_Q4_K>), g, b, (size_t)lds_bytes, st, *a, io);
        else hipLaunchKernelGGL((oh_k_delta_mv<128, 8, OH_Q4_K>), g, b, (size_t)lds_bytes, st, *a, io);
    } else {
        if (a->d.K <= 4) hipLaunchKernelGGL((oh_k_delta_mv<128, 4, OH_Q6_K>), g, b, (size_t)lds_bytes, st, *a, io);
        else hipLaunchKernelGGL((oh_k_delta_mv<128, 8, OH_Q6_K>), g, b, (size_t)lds_bytes, st, *a, io);
    }
    return hipGetLastError();
}

hipError_t oh_launch_matvec(const oh_mvlaunch *L, int tk, int lds_bytes, hipStream_t st) {
    if (L->total_blocks <= 0) return hipSuccess;
    void (*k)(oh_mvlaunch) = tk == OH_Q4_K ? oh_k_mv_q4k : tk == OH_Q6_K ? oh_k_mv_q6k
                           : tk == OH_Q8_0 ? oh_k_mv_q80 : tk == OH_MV_Q4Q6 ? oh_k_mv_q4k6k : oh_k_mv_mixed;
    if (lds_bytes > 65536) {
        // wide fallback rows (IQ2_XXS term tiles, f32 activations past 8K):
        // the kernel's dynamic LDS limit raised to what this launch needs
        // (the limit plus the kernel's static LDS stays within the CU's)
        static int raised[5];
        const int ki = tk == OH_Q4_K ? 0 : tk == OH_Q6_K ? 1 : tk == OH_Q8_0 ? 2 : tk == OH_MV_Q4Q6 ? 4 : 3;
        if (raised[ki] < lds_bytes) {
            const hipError_t e = hipFuncSetAttribute((const void *)k, hipFuncAttributeMaxDynamicSharedMemorySize, lds_bytes);
            if (e != hipSuccess) return e;
            raised[ki] = lds_bytes;
        }
    }
    hipLaunchKernelGGL(k, dim3(L->total_blocks), dim3(256), (size_t)lds_bytes, st, *L);
    return hipGetLastError();
}

hipError_t oh_launch_mvb(const oh_mvbatch *B, int groups, hipStream_t st) {
    const int rps = 64 / B->nb, blocks = (B->rows + 4 * rps - 1) / (4 * rps);
    if (blocks <= 0 || groups <= 0) return hipSuccess;
    void (*k)(oh_mvbatch) = B->type == OH_Q4_K ? oh_k_mvb_q4k : B->type == OH_Q6_K ? oh_k_mvb_q6k : oh_k_mvb_q80;
    oh_mvbatch b = *B;
    int gy = groups;
    if (!B->list && blocks < 256 && B->ncol > B->tcol) {
        // few rows: spread the columns over blocks too (about 512 blocks)
        int chunks = (512 + blocks - 1) / blocks;
        const int maxc = (B->ncol + B->tcol - 1) / B->tcol;
        chunks = chunks < maxc ? chunks : maxc;
        b.cpb = (B->ncol + chunks - 1) / chunks;
        gy = (B->ncol + b.cpb - 1) / b.cpb;
    }
    hipLaunchKernelGGL(k, dim3(blocks, gy), dim3(256), (size_t)B->tcol * mvb_col_bytes(B->nb), st, b);
    return hipGetLastError();
}

int oh_mvb_tcol(int nb) {
    const int t = 32768 / mvb_col_bytes(nb);
    return t < 1 ? 1 : (t > 64 ? 64 : t);
}

hipError_t oh_launch_norm_q8k_rows(const float *x, const float *norm_w, float eps, int n, int rows, float *xn_out,
                                   int8_t *qs, float *d, int16_t *bs, hipStream_t st, int8_t *bp, int swiglu) {
    if (rows <= 0) return hipSuccess;
    if (n > 8192 || n % 256) return hipErrorInvalidValue;     // the kernel's register and LDS sizes
    hipLaunchKernelGGL(oh_k_norm_q8k_rows, dim3(rows), dim3(256), (size_t)n * 4, st, x, norm_w, eps, n, xn_out, qs, d, bs, bp,
                       swiglu);
    return hipGetLastError();
}

// ---- prefill launchers ----
hipError_t oh_launch_embed_rows(const oh_op_embed *a, int base, int T, hipStream_t st) {
    hipLaunchKernelGGL(oh_k_embed_rows, dim3((a->in + 255) / 256, T), dim3(256), 0, st, *a, base);
    return hipGetLastError();
}
hipError_t oh_launch_conv_rows(const float *cat, const float *conv_w, float *conv_state, float *out, float *stage,
                               int T, int base, int cc, int K, hipStream_t st) {
    if (K < 2 || K > kConvKMax) return hipErrorInvalidValue;
    const dim3 g((cc + 255) / 256, (T + kConvRun - 1) / kConvRun), gw((cc + 255) / 256, K - 1);
    hipLaunchKernelGGL(oh_k_conv_rows, g, dim3(256), 0, st, cat, conv_w, conv_state, out, T, base, cc, K);
    if (((base + T) & 1) != (base & 1)) {
        hipLaunchKernelGGL(oh_k_conv_window, gw, dim3(256), 0, st, cat, conv_state, T, base, cc, K);
    } else {
        hipLaunchKernelGGL(oh_k_conv_window_stage, gw, dim3(256), 0, st, cat, conv_state, stage, T, base, cc, K);
        hipError_t e = hipMemcpyAsync(conv_state + (size_t)(base & 1) * (K - 1) * cc, stage,
                                      (size_t)(K - 1) * cc * 4, hipMemcpyDeviceToDevice, st);
        if (e != hipSuccess) return e;
    }
    return hipGetLastError();
}
hipError_t oh_launch_qk_gates_rows(int dk, const float *conv, const float *A, const float *Bg, const float *ssm_a,
                                   const float *dt_bias, float *qn, float *kn, float *al, float *be, int T, int nk,
                                   int nv, int cc, hipStream_t st) {
    const dim3 g(nk + nv, T);
    if (dk == 128) hipLaunchKernelGGL(oh_k_qk_gates_rows<128>, g, dim3(64), 0, st, conv, A, Bg, ssm_a, dt_bias, qn, kn, al, be, nk, nv, cc);
    else if (dk == 64) hipLaunchKernelGGL(oh_k_qk_gates_rows<64>, g, dim3(64), 0, st, conv, A, Bg, ssm_a, dt_bias, qn, kn, al, be, nk, nv, cc);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}
hipError_t oh_launch_delta_scan(int dk, const float *qn, const float *kn, const float *conv, const float *al,
                                const float *be, float *S, float *out, int T, int nk, int nv, int cc,
                                float out_scale, hipStream_t st) {
    if (dk == 128) hipLaunchKernelGGL(oh_k_delta_scan<128>, dim3(nv * 2), dim3(64), 0, st, qn, kn, conv, al, be, S, out, T, nk, nv, cc, out_scale);
    else if (dk == 64) hipLaunchKernelGGL(oh_k_delta_scan<64>, dim3(nv), dim3(64), 0, st, qn, kn, conv, al, be, S, out, T, nk, nv, cc, out_scale);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}
int oh_delta_grams_floats(int T, int nk) { return (T + kDeltaChunk - 1) / kDeltaChunk * nk * 2 * kDeltaChunk * kDeltaChunk; }
int oh_delta_wy_floats(int T, int nv, int dk) { return (T + kWyC - 1) / kWyC * nv * delta_wy_floats(dk); }

hipError_t oh_launch_delta_chunked(int dk, const float *qn, const float *kn, const float *conv, const float *al,
                                   const float *be, float *grams, float *wy, float *S, float *out, int T, int nk,
                                   int nv, int cc, float out_scale, hipStream_t st) {
    if (T <= 0) return hipSuccess;                // no chunk (the scan kernels read row c0 + C - 1)
    const dim3 gg(nk, (T + kDeltaChunk - 1) / kDeltaChunk);
    if (wy) {
        // the matrix-core WY form: grams, the chunks' factors, then the scan
        if (dk != 128 && dk != 64) return hipErrorInvalidValue;
        if (dk == 128) {
            hipLaunchKernelGGL(oh_k_delta_grams<128>, gg, dim3(256), 0, st, qn, kn, T, nk, grams);
            hipLaunchKernelGGL(oh_k_delta_wy<128>, dim3(nv, gg.y), dim3(256), 0, st, kn, conv, al, be, grams, wy, T, nk, nv, cc);
            hipLaunchKernelGGL(oh_k_delta_mfma<128>, dim3(nv * 8), dim3(256), 0, st, qn, kn, wy, S, out, T, nk, nv,
                               out_scale);
        } else {
            hipLaunchKernelGGL(oh_k_delta_grams<64>, gg, dim3(256), 0, st, qn, kn, T, nk, grams);
            hipLaunchKernelGGL(oh_k_delta_wy<64>, dim3(nv, gg.y), dim3(256), 0, st, kn, conv, al, be, grams, wy, T, nk, nv, cc);
            hipLaunchKernelGGL(oh_k_delta_mfma<64>, dim3(nv * 4), dim3(256), 0, st, qn, kn, wy, S, out, T, nk, nv,
                               out_scale);
        }
        return hipGetLastError();
    }
    if (dk == 128) {
        hipLaunchKernelGGL(oh_k_delta_grams<128>, gg, dim3(256), 0, st, qn, kn, T, nk, grams);
        hipLaunchKernelGGL(oh_k_delta_chunked<128>, dim3(nv * 8), dim3(256), 0, st, qn, kn, conv, al, be, grams, S, out, T, nk, nv, cc, out_scale);
    } else if (dk == 64) {
        hipLaunchKernelGGL(oh_k_delta_grams<64>, gg, dim3(256), 0, st, qn, kn, T, nk, grams);
        hipLaunchKernelGGL(oh_k_delta_chunked<64>, dim3(nv * 4), dim3(256), 0, st, qn, kn, conv, al, be, grams, S, out, T, nk, nv, cc, out_scale);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}
hipError_t oh_launch_delta_batch(const oh_op_delta *ops, const int32_t *pos, int n, int dk, int K, int nv,
                                 hipStream_t st) {
    if (K > 8) return hipErrorInvalidValue;
    if (dk == 128) {
        const dim3 g(nv * 2, n);
        if (K <= 4) hipLaunchKernelGGL((oh_k_delta_batch<128, 4>), g, dim3(64), 0, st, ops, pos);
        else hipLaunchKernelGGL((oh_k_delta_batch<128, 8>), g, dim3(64), 0, st, ops, pos);
    } else if (dk == 64) {
        const dim3 g(nv, n);
        if (K <= 4) hipLaunchKernelGGL((oh_k_delta_batch<64, 4>), g, dim3(64), 0, st, ops, pos);
        else hipLaunchKernelGGL((oh_k_delta_batch<64, 8>), g, dim3(64), 0, st, ops, pos);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}
hipError_t oh_launch_prep_batch(const oh_op_prep *ops, const int32_t *pos, int n, int nh, int nkv, hipStream_t st) {
    hipLaunchKernelGGL(oh_k_prep_batch, dim3(nh + nkv, n), dim3(256), 0, st, ops, pos);
    return hipGetLastError();
}
hipError_t oh_launch_attn_batch(const oh_op_attn *ops, const int32_t *pos, int n, int nvb_main, int lds, int nh,
                                int hd, hipStream_t st) {
    hipLaunchKernelGGL(oh_k_attn_main_batch, dim3(nvb_main, n), dim3(256), (size_t)lds, st, ops, pos);
    hipLaunchKernelGGL(oh_k_attn_combine_batch, dim3(nh * (hd / 64), n), dim3(256), 0, st, ops, pos);
    return hipGetLastError();
}
hipError_t oh_launch_batch_tokens(int32_t *const *toks, const int32_t *pos, const int32_t *tok, const int32_t *next,
                                  int n, hipStream_t st) {
    hipLaunchKernelGGL(oh_k_batch_tokens, dim3((n + 255) / 256), dim3(256), 0, st, toks, pos, tok, next, n);
    return hipGetLastError();
}
hipError_t oh_launch_argmax_rows(const float *v, int n, int rows, int32_t *out, hipStream_t st, float *bv, int *bi) {
    if (!bv || !bi) {
        hipLaunchKernelGGL(oh_k_argmax_rows, dim3(rows), dim3(256), 0, st, v, n, out);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(oh_k_argmax_rows1, dim3(OH_ARGMAX_BLOCKS, rows), dim3(256), 0, st, v, n, bv, bi);
    hipLaunchKernelGGL(oh_k_argmax_rows2, dim3(rows), dim3(64), 0, st, bv, bi, out);
    return hipGetLastError();
}
bool oh_mmq_can(uint32_t type, int rows, int in) {
    return (type == OH_Q4_K || (type == OH_Q6_K && in <= 8192)) && rows > 0 && rows % kMqRows == 0 &&
           in % 256 == 0 && in > 0;
}
hipError_t oh_launch_mmq_tiles(const uint8_t *A, const uint8_t *B, uint8_t *PA, uint8_t *PB, int64_t rows,
                               int nb, int P, hipStream_t st) {
    if (rows <= 0 || rows % 64 || nb <= 0 || (P != 8 && P != 12)) return hipErrorInvalidValue;
    const int64_t n = rows * nb * (P + 1);
    const int64_t nbk = (n + 255) / 256;
    hipLaunchKernelGGL(oh_k_mmq_tiles, dim3((unsigned)(nbk < 16384 ? nbk : 16384)), dim3(256), 0, st,
                       (const uint4 *)A, (const uint4 *)B, (uint4 *)PA, (uint4 *)PB, rows, nb, P);
    return hipGetLastError();
}
hipError_t oh_launch_mmq(const oh_mmq *M, int max_items, int pair, hipStream_t st) {
    // grouped: the item rows rounded up for the XCD runs of mq_block (rows past
    // the item count exit)
    const int ty = M->list ? (max_items + 8 * kMqRun - 1) / (8 * kMqRun) * (8 * kMqRun)
                           : (M->ncol + kMqCols - 1) / kMqCols;
    if (ty <= 0) return hipSuccess;
    const dim3 grid(M->rows / kMqRows, ty, pair ? 2 : 1);
    if (M->type == OH_Q6_K) {
        static bool lds6 = false;      // stages + the rows' d exceed the default dynamic LDS limit
        if (!lds6) {
            hipError_t e = hipFuncSetAttribute((const void *)oh_k_mmq_q6k,
                                               hipFuncAttributeMaxDynamicSharedMemorySize, m6_lds_bytes(32, 2));
            if (e == hipSuccess)
                e = hipFuncSetAttribute((const void *)oh_k_mmq_q6k_s1, hipFuncAttributeMaxDynamicSharedMemorySize,
                                        m6_lds_bytes(kM6OneBuf, 1));
            if (e != hipSuccess) return e;
            lds6 = true;
        }
        if (M->nb <= kM6OneBuf)
            hipLaunchKernelGGL(oh_k_mmq_q6k_s1, grid, dim3(256), (size_t)m6_lds_bytes(M->nb, 1), st, *M);
        else
            hipLaunchKernelGGL(oh_k_mmq_q6k, grid, dim3(256), (size_t)m6_lds_bytes(M->nb, 2), st, *M);
        return hipGetLastError();
    }
    static bool lds_set = false;   // two stages exceed the default dynamic LDS limit
    if (!lds_set) {
        const hipError_t e = hipFuncSetAttribute((const void *)oh_k_mmq_q4k,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, 2 * kMqStage);
        if (e != hipSuccess) return e;
        lds_set = true;
    }
    hipLaunchKernelGGL(oh_k_mmq_q4k, grid, dim3(256), 2 * kMqStage, st, *M);
    return hipGetLastError();
}
hipError_t oh_launch_mmq_items(const int32_t *cnt, int ne, int32_t *items, hipStream_t st) {
    if (ne > 1024) return hipErrorInvalidValue;
    hipLaunchKernelGGL(oh_k_mmq_items, dim3(1), dim3(256), 0, st, cnt, ne, items);
    return hipGetLastError();
}
hipError_t oh_launch_gnorm_q8k_rows(const float *x, const float *z, const float *w, float eps, int n, int gdim,
                                    int T, int8_t *qs, float *d, int16_t *bs, hipStream_t st, int8_t *bp) {
    if (n <= 0 || n > 8192 || gdim <= 0 || n % gdim || n / gdim > 128) return hipErrorInvalidValue;
    hipLaunchKernelGGL(oh_k_gnorm_q8k_rows, dim3(T), dim3(256), (size_t)n * 4, st, x, z, w, eps, n, gdim, qs, d, bs,
                       bp);
    return hipGetLastError();
}
hipError_t oh_launch_prep_rows(const oh_op_prep *a, int base, int T, hipStream_t st) {
    hipLaunchKernelGGL(oh_k_prep_rows, dim3(a->nh + a->nkv, T), dim3(256), 0, st, *a, base);
    return hipGetLastError();
}
// the prompt's exact rows: the scores of a block's 256/hd heads in LDS, up to
// kExactMax positions
static int pf_exact_lds_bytes(int hd, int exact_max) {
    const int lim = exact_max < kExactMax ? (exact_max > 0 ? exact_max : 0) : kExactMax;
    return (256 / hd) * lim * 4;
}
hipError_t oh_launch_attn_exact_rows(const oh_op_attn *a, int base, int t0, int n, hipStream_t st) {
    const int lim = a->exact_max < kExactMax ? a->exact_max : kExactMax;
    if (n <= 0) return hipSuccess;
    if (base + t0 + n > lim) return hipErrorInvalidValue;     // every row must be inside the exact walk
    hipLaunchKernelGGL(oh_k_attn_exact_rows, dim3(a->nh / (256 / a->hd), n), dim3(256),
                       (size_t)pf_exact_lds_bytes(a->hd, a->exact_max), st, *a, base, t0);
    return hipGetLastError();
}
hipError_t oh_launch_attn_rows(const oh_op_attn *a, int base, int t0, int n, size_t po_stride, size_t pml_stride,
                               hipStream_t st) {
    const int lim = a->exact_max < kExactMax ? a->exact_max : kExactMax;
    if (base + t0 + 1 <= lim)       // some tokens walk exactly
        hipLaunchKernelGGL(oh_k_attn_exact_rows, dim3(a->nh / (256 / a->hd), n), dim3(256),
                           (size_t)pf_exact_lds_bytes(a->hd, a->exact_max), st, *a, base, t0);
    if (base + t0 + n > lim) {      // some tokens take the flash chunks
        const int nch = (base + t0 + n + kFlashCh - 1) / kFlashCh;
        const int nvb = a->nkv * (a->nh / a->nkv / a->hb) * nch;
        const size_t lds = (size_t)oh_flash_lds_bytes(a->nh, a->nkv, a->hd);
        if (a->hb == 4)
            hipLaunchKernelGGL(oh_k_attn_flash_rows<4>, dim3(nvb), dim3(256), lds, st, *a, base, t0, n, po_stride, pml_stride);
        else if (a->hb == 2)
            hipLaunchKernelGGL(oh_k_attn_flash_rows<2>, dim3(nvb), dim3(256), lds, st, *a, base, t0, n, po_stride, pml_stride);
        else
            hipLaunchKernelGGL(oh_k_attn_flash_rows<1>, dim3(nvb), dim3(256), lds, st, *a, base, t0, n, po_stride, pml_stride);
    }
    hipLaunchKernelGGL(oh_k_attn_combine_rows, dim3(a->nh * (a->hd / 64), n), dim3(256), 0, st, *a, base, t0, po_stride, pml_stride);
    return hipGetLastError();
}
hipError_t oh_launch_route_rows(const float *logits, int ne, int k, const float *shl, int32_t *idx, float *w,
                                float *shg, int T, hipStream_t st) {
    hipLaunchKernelGGL(oh_k_route_rows, dim3(T), dim3(64), 0, st, logits, ne, k, shl, idx, w, shg);
    return hipGetLastError();
}
hipError_t oh_launch_group_pairs(const int32_t *idx, int npairs, int32_t *cnt, int ne, int32_t *list, int lstride,
                                 int32_t *err, hipStream_t st) {
    hipLaunchKernelGGL(oh_k_fill_i32, dim3((ne + 255) / 256), dim3(256), 0, st, cnt, ne, 0);
    hipLaunchKernelGGL(oh_k_group_pairs, dim3((npairs + 255) / 256), dim3(256), 0, st, idx, npairs, cnt, ne, list,
                       lstride, err);
    return hipGetLastError();
}
hipError_t oh_launch_moe_combine_rows(float *x, const float *o, const float *w, int k, int H, const float *so,
                                      const float *shgate, int T, hipStream_t st) {
    hipLaunchKernelGGL(oh_k_moe_combine_rows, dim3((H + 255) / 256, T), dim3(256), 0, st, x, o, w, k, H, so, shgate);
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


hipError_t oh_launch_mv_down_rows(const oh_mvdown *D, int nvb, int ntok, int lds, hipStream_t st) {
    if (nvb <= 0 || ntok <= 0) return hipSuccess;
    const int ns = D->k + (D->sA ? 1 : 0);
    hipLaunchKernelGGL(oh_k_mv_down, dim3(nvb, ntok), dim3(64 * ns), (size_t)lds, st, *D);
    return hipGetLastError();
}

hipError_t oh_launch_op(const oh_op *op, const int32_t *io, hipStream_t st) {
    if (op->nvb <= 0) return hipSuccess;
    const dim3 g(op->nvb), b256(256);
    switch (op->kind) {
    case OH_OP_MV:
        return oh_launch_matvec(&op->u.mv, op->tk, op->lds, st);
    case OH_OP_DELTA_MV:
        return oh_launch_delta_mv(&op->u.dmv, op->tk, op->lds, io, st);
    case OH_OP_MV_DOWN: {
        const int ns = op->u.down.k + (op->u.down.sA ? 1 : 0);
        if (op->u.down.narrow) {
            if (ns > 16 || 16 % op->u.down.nb) return hipErrorInvalidValue;
            hipLaunchKernelGGL(oh_k_mv_down_narrow, g, dim3(64 * ((ns + 3) / 4)), (size_t)op->lds, st, op->u.down);
        } else {
            hipLaunchKernelGGL(oh_k_mv_down, g, dim3(64 * ns), (size_t)op->lds, st, op->u.down);
        }
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
    case OH_OP_DELTA16:
        if (op->u.delta.K > 8) return hipErrorInvalidValue;
        if (op->u.delta.dk == 128) {
            if (op->u.delta.K <= 4) hipLaunchKernelGGL((oh_k_delta16<128, 4>), g, b256, 0, st, op->u.delta, io);
            else hipLaunchKernelGGL((oh_k_delta16<128, 8>), g, b256, 0, st, op->u.delta, io);
        } else if (op->u.delta.dk == 64) {
            if (op->u.delta.K <= 4) hipLaunchKernelGGL((oh_k_delta16<64, 4>), g, b256, 0, st, op->u.delta, io);
            else hipLaunchKernelGGL((oh_k_delta16<64, 8>), g, b256, 0, st, op->u.delta, io);
        } else {
            return hipErrorInvalidValue;
        }
        break;
    case OH_OP_ATTN_PREP: hipLaunchKernelGGL(oh_k_attn_prep, g, b256, 0, st, op->u.prep, io); break;
    case OH_OP_ATTN_MAIN: hipLaunchKernelGGL(oh_k_attn_main, g, b256, (size_t)op->lds, st, op->u.attn, io); break;
    case OH_OP_ATTN_COMBINE: hipLaunchKernelGGL(oh_k_attn_combine, g, b256, 0, st, op->u.attn, io); break;
    case OH_OP_ATTN_SCORES: hipLaunchKernelGGL(oh_k_attn_scores, g, dim3(512), (size_t)op->lds, st, op->u.attn, io); break;
    case OH_OP_ATTN_WALK: hipLaunchKernelGGL(oh_k_attn_walk, g, dim3(512), (size_t)op->lds, st, op->u.attn, io); break;
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

// flash form of a decode attention: 0 = the matrix-core chunks (every query
// head of a KV head per block), else the query heads per VALU flash block
int oh_flash_form(int nh, int nkv, int hd, int mfma) {
    if (mfma && nkv > 0 && nh % nkv == 0 && nh / nkv <= 16 && (hd == 64 || hd == 128 || hd == 256)) return 0;
    return oh_flash_hb(nh, nkv);
}
int oh_flash_nvb(int nh, int nkv, int cap, int hb) {
    return hb == 0 ? nkv * fd_blocks(cap) : nkv * (nh / nkv / hb) * ((cap + kFlashCh - 1) / kFlashCh);
}
int oh_flash_form_lds(int nh, int nkv, int hd, int hb) { return hb == 0 ? kFdLds : oh_flash_lds_bytes(nh, nkv, hd); }
int oh_flash_slots(int cap) { return fd_slots(cap); }
// partials per KV head at context T
int oh_flash_parts(int T, int cap, int hb) {
    if (hb != 0) return (T + kFlashCh - 1) / kFlashCh;
    const int tpb = fd_tpb(T, cap);
    return ((T + kFdT - 1) / kFdT + tpb - 1) / tpb;
}

// contexts up to this many positions take the exact attention walk
int oh_exact_limit(int exact_max, int hd) { return exact_lim(exact_max, hd); }

// the decode step's exact attention walk: the scores of a block's 256/hd
// heads in LDS
int oh_exact_lds_bytes(int hd, int exact_max) { return (256 / hd) * exact_lim(exact_max, hd) * 4; }

// delta step LDS of the working wave (step kernel: dynamic LDS)
int oh_delta_lds_bytes(int dk) { return (2 * dk + 64 * (dk + 4)) * 4; }
int oh_delta16_lds_bytes(int dk) { return delta16_lds_floats(dk) * 4; }

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
    if (type == OH_IQ2_XXS) {
        hipLaunchKernelGGL(oh_k_encode_iq2xxs, dim3((unsigned)((nblk + 3) / 4)), dim3(256), 0, st, x, nblk, A, C);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(oh_k_encode, dim3((unsigned)((nblk + 255) / 256)), dim3(256), 0, st, x, type, nblk, A, B, C);
    return hipGetLastError();
}

hipError_t oh_launch_advance(int32_t *io_pos, hipStream_t st) {
    hipLaunchKernelGGL(oh_k_advance, dim3(1), dim3(1), 0, st, io_pos);
    return hipGetLastError();
}

} // extern "C"
