// oh_host_kernels.cpp - kernel-level entry points of the C ABI (quantize, matvec, dequant, route, no-allocation matvec).
#include "oh_engine.h"


// ---- kernel-level entry points ---------------------------------------------------------
extern "C" int ornith_hip_quantize_q8K(ornith_hip_ctx *ctx, const float *x, int64_t k,
                                       ornith_hip_q8k *yq) {
    if (k % 256) { seterr("quantize_q8K: k=%lld not a multiple of 256", (long long)k); return ORNITH_HIP_ERR_FORMAT; }
    HCHK(hipSetDevice(ctx->device));
    const int64_t nb = k / 256;
    void *sp;
    CHK(ctx_scratch(ctx, (size_t)k * 4 + (size_t)k + (size_t)nb * 4 + (size_t)nb * 32 + 1024, &sp));
    float *dx = (float *)sp;
    int8_t *qs = (int8_t *)(dx + k);
    float *dd = (float *)up256((size_t)(qs + k));
    int16_t *bs = (int16_t *)up256((size_t)(dd + nb));
    HCHK(hipMemcpyAsync(dx, x, (size_t)k * 4, hipMemcpyHostToDevice, ctx->st));
    for (int64_t off = 0; off < k; off += 8192) {
        const int n = (int)(k - off < 8192 ? k - off : 8192);
        HCHK(oh_launch_rmsnorm_q8k(dx + off, nullptr, 0.0f, n, nullptr, qs + off, dd + off / 256,
                                   bs + off / 16, ctx->st));
    }
    std::vector<int8_t> hq((size_t)k);
    std::vector<float> hd((size_t)nb);
    std::vector<int16_t> hb((size_t)nb * 16);
    HCHK(hipMemcpyAsync(hq.data(), qs, (size_t)k, hipMemcpyDeviceToHost, ctx->st));
    HCHK(hipMemcpyAsync(hd.data(), dd, (size_t)nb * 4, hipMemcpyDeviceToHost, ctx->st));
    HCHK(hipMemcpyAsync(hb.data(), bs, (size_t)nb * 32, hipMemcpyDeviceToHost, ctx->st));
    HCHK(hipStreamSynchronize(ctx->st));
    for (int64_t b = 0; b < nb; b++) {
        yq[b].d = hd[b];
        memcpy(yq[b].qs, hq.data() + b * 256, 256);
        memcpy(yq[b].bsums, hb.data() + b * 16, 32);
    }
    return ORNITH_HIP_OK;
}

// batched Q4_K products on the matrix cores (ORNITH_HIP_MMQ=0: the vector-ALU kernels)
bool mmq_enabled() {
    const char *e = getenv("ORNITH_HIP_MMQ");
    return !(e && e[0] == '0');
}

int mmq_tiles(const ornith_hip_tensor *W, hipStream_t st) {
    if (W->PA) return ORNITH_HIP_OK;
    const int P = W->type == OH_Q4_K ? 8 : W->type == OH_Q6_K ? 12 : 0;
    if (!P || W->rows % 64 || W->in % 256) {
        seterr("tensor '%s': no prompt tiles for type %u with %lld rows", W->name.c_str(), W->type,
               (long long)W->rows);
        return ORNITH_HIP_ERR_UNSUPPORTED;
    }
    const size_t nblk = (size_t)W->rows * (size_t)(W->in / 256), a = nblk * 16 * P, b = nblk * 16;
    uint8_t *mem = nullptr;
    hipError_t e = hipMalloc(&mem, up256(a) + b);
    if (e != hipSuccess) {
        seterr("tensor '%s': prompt tiles, hipMalloc(%zu): %s", W->name.c_str(), up256(a) + b,
               hipGetErrorString(e));
        return ORNITH_HIP_ERR_OOM;
    }
    e = oh_launch_mmq_tiles(W->A, W->B, mem, mem + up256(a), W->rows, (int)(W->in / 256), P, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) {
        (void)hipFree(mem);
        seterr("tensor '%s': prompt tiles: %s", W->name.c_str(), hipGetErrorString(e));
        return ORNITH_HIP_ERR_DEVICE;
    }
    W->pmem = mem;
    W->PA = mem;
    W->PB = mem + up256(a);
    return ORNITH_HIP_OK;
}

// device bytes of matvec_cols' buffer: input, output, Q8_K planes (256-aligned)
size_t matvec_col_bytes(int64_t in, int64_t out) {
    return (size_t)in * 5 + (size_t)(in / 256) * 40 + (size_t)out * 4 + 4096;
}

extern "C" int ornith_hip_matvec(ornith_hip_ctx *ctx, const ornith_hip_tensor *W,
                                 const float *x, float *y, int Tn) {
    HCHK(hipSetDevice(ctx->device));
    const int64_t in = W->in, out = W->rows, nb = in / 256;
    const bool q = oh_qdot_can(W->type, in);
    void *sp;
    if (q && Tn > 1 && in <= 8192) {
        // Tn columns: each quantised to Q8_K, one batched launch
        const size_t T = (size_t)Tn;
        CHK(ctx_scratch(ctx, T * in * 5 + T * nb * 56 + T * out * 4 + 4096, &sp));
        float *dx = (float *)sp;
        float *dy = (float *)up256((size_t)(dx + T * in));
        int8_t *qs = (int8_t *)up256((size_t)(dy + T * out));
        float *dd = (float *)up256((size_t)(qs + T * in));
        int16_t *bs = (int16_t *)up256((size_t)(dd + T * nb + 1));
        int8_t *bp = (int8_t *)up256((size_t)(bs + T * nb * 16));
        HCHK(hipMemcpyAsync(dx, x, T * in * 4, hipMemcpyHostToDevice, ctx->st));
        HCHK(oh_launch_norm_q8k_rows(dx, nullptr, 0.0f, (int)in, Tn, nullptr, qs, dd, bs, ctx->st, bp));
        if (mmq_enabled() && oh_mmq_can(W->type, (int)out, (int)in)) {
            CHK(mmq_tiles(W, ctx->st));
            oh_mmq M;
            memset(&M, 0, sizeof M);
            M.A = W->PA; M.B = W->PB; M.C = W->C; M.type = (int)W->type;
            M.xqs = qs; M.xd = dd; M.xbp = bp; M.y = dy;
            M.nb = (int)nb; M.in = (int)in; M.rows = (int)out; M.ncol = Tn; M.adiv = 1; M.ystride = (int)out;
            HCHK(oh_launch_mmq(&M, 0, 0, ctx->st));
            HCHK(hipMemcpyAsync(y, dy, T * out * 4, hipMemcpyDeviceToHost, ctx->st));
            HCHK(hipStreamSynchronize(ctx->st));
            return ORNITH_HIP_OK;
        }
        oh_mvbatch B;
        memset(&B, 0, sizeof B);
        B.A = W->A; B.B = W->B; B.C = W->C;
        B.xqs = qs; B.xd = dd; B.xbs = bs; B.y = dy;
        B.type = (int)W->type; B.nb = (int)nb; B.in = (int)in; B.rows = (int)out;
        B.ncol = Tn; B.adiv = 1; B.ystride = (int)out; B.tcol = oh_mvb_tcol((int)nb);
        HCHK(oh_launch_mvb(&B, 1, ctx->st));
        HCHK(hipMemcpyAsync(y, dy, T * out * 4, hipMemcpyDeviceToHost, ctx->st));
        HCHK(hipStreamSynchronize(ctx->st));
        return ORNITH_HIP_OK;
    }
    CHK(ctx_scratch(ctx, matvec_col_bytes(in, out), &sp));
    return matvec_cols(ctx, W, x, y, Tn, sp);
}

// The single-column path of ornith_hip_matvec over a caller-provided device
// buffer `sp` of at least matvec_col_bytes(in, out) bytes: per column, the
// input copied in, quantised to Q8_K (integer path), one matvec launch, the
// output copied out. Allocates nothing.
int matvec_cols(ornith_hip_ctx *ctx, const ornith_hip_tensor *W, const float *x, float *y, int Tn,
                       void *sp) {
    const int64_t in = W->in, out = W->rows, nb = in / 256;
    const bool q = oh_qdot_can(W->type, in);
    float *dx = (float *)sp;
    float *dy = (float *)up256((size_t)(dx + in));
    int8_t *qs = (int8_t *)up256((size_t)(dy + out));
    float *dd = (float *)up256((size_t)(qs + in));
    int16_t *bs = (int16_t *)up256((size_t)(dd + nb + 1));
    for (int t = 0; t < Tn; t++) {
        HCHK(hipMemcpyAsync(dx, x + (size_t)t * in, (size_t)in * 4, hipMemcpyHostToDevice, ctx->st));
        Act act;
        act.xf = dx;
        if (q) {
            for (int64_t off = 0; off < in; off += 8192) {
                const int n = (int)(in - off < 8192 ? in - off : 8192);
                HCHK(oh_launch_rmsnorm_q8k(dx + off, nullptr, 0.0f, n, nullptr, qs + off,
                                           dd + off / 256, bs + off / 16, ctx->st));
            }
            act.qs = qs; act.d = dd; act.bs = bs;
        }
        MvBuild b;
        CHK(mv_add(b, W, act, dy, 0));
        CHK(mv_go(b, ctx->st));
        HCHK(hipMemcpyAsync(y + (size_t)t * out, dy, (size_t)out * 4, hipMemcpyDeviceToHost, ctx->st));
    }
    HCHK(hipStreamSynchronize(ctx->st));
    return ORNITH_HIP_OK;
}

// ornith_hip_matvec without any allocation: the single-column path over the
// device's fixed scratch array (results equal ornith_hip_matvec's; every
// column is its own launch sequence). Calls that overlap on one device share
// the array and race; the caller serialises them.
extern "C" int ornith_hip_matvec_noalloc(ornith_hip_ctx *ctx, const ornith_hip_tensor *W,
                                         const float *x, float *y, int Tn) {
    if (!ctx || !W || (Tn > 0 && (!x || !y))) {
        seterr("matvec_noalloc: null context, tensor or buffer");
        return ORNITH_HIP_ERR_FORMAT;
    }
    if (Tn <= 0) return ORNITH_HIP_OK;
    const size_t need = matvec_col_bytes(W->in, W->rows);
    if (need > OH_NOALLOC_SCRATCH_BYTES) {
        seterr("matvec_noalloc: '%s' (%lld x %lld) needs %zu scratch bytes, above the fixed %u",
               W->name.c_str(), (long long)W->in, (long long)W->rows, need, OH_NOALLOC_SCRATCH_BYTES);
        return ORNITH_HIP_ERR_UNSUPPORTED;
    }
    void *sp = ctx->device >= 0 && ctx->device < OH_MAX_DEVICES ? g_scratch_dev[ctx->device] : nullptr;
    if (!sp) {
        seterr("matvec_noalloc: device %d has no scratch address (context not from ornith_hip_init)", ctx->device);
        return ORNITH_HIP_ERR_DEVICE;
    }
    HCHK(hipSetDevice(ctx->device));
    return matvec_cols(ctx, W, x, y, Tn, sp);
}

// oq_quantize on the device: n floats (whole super-blocks) -> GGUF blocks of
// Q8_0 / Q4_K / Q6_K / IQ2_XXS, the encoders of the model synthesis
extern "C" int ornith_hip_quantize(ornith_hip_ctx *ctx, uint32_t type, const float *x, uint64_t n, void *out) {
    if (type != OH_Q8_0 && type != OH_Q4_K && type != OH_Q6_K && type != OH_IQ2_XXS) {
        seterr("quantize: type %u has no device encoder (Q8_0, Q4_K, Q6_K, IQ2_XXS)", type);
        return ORNITH_HIP_ERR_UNSUPPORTED;
    }
    if (n == 0 || n % 256) { seterr("quantize: %llu values is not a whole number of 256-blocks", (unsigned long long)n); return ORNITH_HIP_ERR_FORMAT; }
    HCHK(hipSetDevice(ctx->device));
    const uint64_t dims[2] = {256, n / 256};
    ornith_hip_tensor *t = nullptr;
    CHK(tensor_alloc(ctx, "quantize", type, 2, dims, &t));
    float *dx = nullptr;
    hipError_t e = hipMalloc(&dx, n * 4);
    if (e == hipSuccess) e = hipMemcpyAsync(dx, x, n * 4, hipMemcpyHostToDevice, ctx->st);
    if (e == hipSuccess) e = oh_launch_encode(dx, (int)type, (int64_t)(n / 256), t->A, t->B, t->C, ctx->st);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->st);
    if (dx) (void)hipFree(dx);
    int r = ORNITH_HIP_OK;
    if (e != hipSuccess) { seterr("quantize: %s", hipGetErrorString(e)); r = ORNITH_HIP_ERR_DEVICE; }
    if (r == ORNITH_HIP_OK) r = ornith_hip_tensor_download(t, out, t->gguf_bytes);
    ornith_hip_tensor_free(t);
    return r;
}

extern "C" int ornith_hip_dequant(ornith_hip_ctx *ctx, const ornith_hip_tensor *W,
                                  int64_t row0, int64_t nrows, float *out) {
    if (row0 < 0 || nrows < 0 || row0 + nrows > W->rows) {
        seterr("dequant: rows [%lld, %lld) outside [0, %lld)", (long long)row0,
               (long long)(row0 + nrows), (long long)W->rows);
        return ORNITH_HIP_ERR_FORMAT;
    }
    HCHK(hipSetDevice(ctx->device));
    const size_t n = (size_t)nrows * W->in;
    void *sp;
    CHK(ctx_scratch(ctx, n * 4 + 256, &sp));
    HCHK(oh_launch_dequant(W->A, W->B, W->C, (int)W->type, (int)W->in, row0, nrows, (float *)sp, ctx->st));
    HCHK(hipMemcpyAsync(out, sp, n * 4, hipMemcpyDeviceToHost, ctx->st));
    HCHK(hipStreamSynchronize(ctx->st));
    return ORNITH_HIP_OK;
}

extern "C" int ornith_hip_moe_route(ornith_hip_ctx *ctx, const float *logits, int ne, int k,
                                    int32_t *idx, float *w) {
    if (ne < 1 || ne > 1024 || k < 1 || k > 64 || k > ne) {
        seterr("moe_route: ne=%d k=%d unsupported", ne, k);
        return ORNITH_HIP_ERR_UNSUPPORTED;
    }
    HCHK(hipSetDevice(ctx->device));
    void *sp;
    CHK(ctx_scratch(ctx, (size_t)ne * 4 + 1024, &sp));
    float *dl = (float *)sp;
    int32_t *di = (int32_t *)up256((size_t)(dl + ne));
    float *dw = (float *)(di + 64);
    HCHK(hipMemcpyAsync(dl, logits, (size_t)ne * 4, hipMemcpyHostToDevice, ctx->st));
    HCHK(oh_launch_moe_route(dl, ne, k, nullptr, di, dw, nullptr, ctx->st));
    HCHK(hipMemcpyAsync(idx, di, (size_t)k * 4, hipMemcpyDeviceToHost, ctx->st));
    HCHK(hipMemcpyAsync(w, dw, (size_t)k * 4, hipMemcpyDeviceToHost, ctx->st));
    HCHK(hipStreamSynchronize(ctx->st));
    return ORNITH_HIP_OK;
}

extern "C" int ornith_hip_time_matvec(ornith_hip_ctx *ctx, const ornith_hip_tensor *W, int iters,
                                      float *ms) {
    HCHK(hipSetDevice(ctx->device));
    const int64_t in = W->in, out = W->rows, nb = in / 256;
    void *sp;
    CHK(ctx_scratch(ctx, (size_t)in * 5 + (size_t)nb * 40 + (size_t)out * 4 + 4096, &sp));
    float *dx = (float *)sp;
    float *dy = (float *)up256((size_t)(dx + in));
    int8_t *qs = (int8_t *)up256((size_t)(dy + out));
    float *dd = (float *)up256((size_t)(qs + in));
    int16_t *bs = (int16_t *)up256((size_t)(dd + nb + 1));
    std::vector<float> hx((size_t)in);
    for (int64_t i = 0; i < in; i++) hx[i] = (float)((i * 7919) % 255 - 127) / 64.0f;
    HCHK(hipMemcpyAsync(dx, hx.data(), (size_t)in * 4, hipMemcpyHostToDevice, ctx->st));
    Act act;
    act.xf = dx;
    if (oh_qdot_can(W->type, in)) {
        for (int64_t off = 0; off < in; off += 8192) {
            const int n = (int)(in - off < 8192 ? in - off : 8192);
            HCHK(oh_launch_rmsnorm_q8k(dx + off, nullptr, 0.0f, n, nullptr, qs + off, dd + off / 256,
                                       bs + off / 16, ctx->st));
        }
        act.qs = qs; act.d = dd; act.bs = bs;
    }
    MvBuild b;
    CHK(mv_add(b, W, act, dy, 0));
    CHK(mv_go(b, ctx->st));   // warm
    hipEvent_t e0, e1;
    HCHK(hipEventCreate(&e0));
    HCHK(hipEventCreate(&e1));
    HCHK(hipEventRecord(e0, ctx->st));
    for (int i = 0; i < iters; i++) CHK(mv_go(b, ctx->st));
    HCHK(hipEventRecord(e1, ctx->st));
    HCHK(hipEventSynchronize(e1));
    float el = 0.0f;
    HCHK(hipEventElapsedTime(&el, e0, e1));
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    *ms = iters > 0 ? el / (float)iters : 0.0f;
    return ORNITH_HIP_OK;
}

extern "C" int ornith_hip_time_matvec_set(ornith_hip_ctx *ctx, const ornith_hip_tensor *const *W, int n,
                                          int iters, float *ms) {
    if (n < 1 || iters < 1) { seterr("time_matvec_set: need n >= 1 and iters >= 1"); return ORNITH_HIP_ERR_FORMAT; }
    for (int i = 1; i < n; i++)
        if (W[i]->type != W[0]->type || W[i]->in != W[0]->in || W[i]->rows != W[0]->rows) {
            seterr("time_matvec_set: tensors differ in type or shape");
            return ORNITH_HIP_ERR_FORMAT;
        }
    HCHK(hipSetDevice(ctx->device));
    const int64_t in = W[0]->in, out = W[0]->rows, nb = in / 256;
    void *sp;
    CHK(ctx_scratch(ctx, (size_t)in * 5 + (size_t)nb * 40 + (size_t)out * 4 + 4096, &sp));
    float *dx = (float *)sp;
    float *dy = (float *)up256((size_t)(dx + in));
    int8_t *qs = (int8_t *)up256((size_t)(dy + out));
    float *dd = (float *)up256((size_t)(qs + in));
    int16_t *bs = (int16_t *)up256((size_t)(dd + nb + 1));
    std::vector<float> hx((size_t)in);
    for (int64_t i = 0; i < in; i++) hx[i] = (float)((i * 7919) % 255 - 127) / 64.0f;
    HCHK(hipMemcpyAsync(dx, hx.data(), (size_t)in * 4, hipMemcpyHostToDevice, ctx->st));
    Act act;
    act.xf = dx;
    if (oh_qdot_can(W[0]->type, in)) {
        for (int64_t off = 0; off < in; off += 8192) {
            const int k = (int)(in - off < 8192 ? in - off : 8192);
            HCHK(oh_launch_rmsnorm_q8k(dx + off, nullptr, 0.0f, k, nullptr, qs + off, dd + off / 256,
                                       bs + off / 16, ctx->st));
        }
        act.qs = qs; act.d = dd; act.bs = bs;
    }
    std::vector<MvBuild> bl((size_t)n);
    for (int i = 0; i < n; i++) {
        CHK(mv_add(bl[i], W[i], act, dy, 0));
        mv_plan(bl[i]);
    }
    HCHK(hipStreamSynchronize(ctx->st));
    hipGraph_t g = nullptr;
    hipGraphExec_t ge = nullptr;
    HCHK(hipStreamBeginCapture(ctx->st, hipStreamCaptureModeThreadLocal));
    hipError_t ce = hipSuccess;
    for (int i = 0; i < iters && ce == hipSuccess; i++) ce = oh_launch_matvec(&bl[i % n].L, bl[i % n].tk, bl[i % n].lds, ctx->st);
    const hipError_t ee = hipStreamEndCapture(ctx->st, &g);
    if (ce != hipSuccess || ee != hipSuccess) {
        if (g) (void)hipGraphDestroy(g);
        HCHK(ce != hipSuccess ? ce : ee);
    }
    hipError_t ie = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    HCHK(ie);
    hipEvent_t e0 = nullptr, e1 = nullptr;
    float el = 0.0f;
    hipError_t r = hipGraphLaunch(ge, ctx->st);                  // warm
    if (r == hipSuccess) r = hipEventCreate(&e0);
    if (r == hipSuccess) r = hipEventCreate(&e1);
    if (r == hipSuccess) r = hipEventRecord(e0, ctx->st);
    if (r == hipSuccess) r = hipGraphLaunch(ge, ctx->st);
    if (r == hipSuccess) r = hipEventRecord(e1, ctx->st);
    if (r == hipSuccess) r = hipEventSynchronize(e1);
    if (r == hipSuccess) r = hipEventElapsedTime(&el, e0, e1);
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    (void)hipGraphExecDestroy(ge);
    HCHK(r);
    *ms = el / (float)iters;
    return ORNITH_HIP_OK;
}
