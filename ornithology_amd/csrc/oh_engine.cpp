// oh_engine.cpp - host side of the MI355X decode engine, shared part: the
// error buffer, the context, the no-allocation matvec's device scratch, tensors
// in the plane layout and the matvec launch builder. The rest of the host side
// (model load, sessions and the token step, prefill, batch step, snapshots,
// synthesis, timing) is in oh_host_*.cpp, all behind the C ABI of
// include/ornith_hip.h.
//
// Reference: src/ornith_rforward.c (rmodel_* / rsession_*), src/ornith_gguf_write.c
// (GGUF v3 layout), src/ornith_model.h (arch).

#include "oh_engine.h"


// ---- errors (src/ornith_util.c:7,25-30 convention: one global buffer) ---------
static char g_err[1024];
void seterr(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
}
extern "C" const char *ornith_hip_last_error(void) { return g_err; }

int ctx_scratch(ornith_hip_ctx *c, size_t bytes, void **out) {
    if (bytes > c->scratch_bytes) {
        if (c->scratch) HCHK(hipFree(c->scratch));
        c->scratch = nullptr;
        c->scratch_bytes = 0;
        HCHK(hipMalloc(&c->scratch, bytes));
        c->scratch_bytes = bytes;
    }
    *out = c->scratch;
    return ORNITH_HIP_OK;
}
static __device__ __align__(256) uint8_t scratch[OH_NOALLOC_SCRATCH_BYTES];
void *g_scratch_dev[OH_MAX_DEVICES];
static std::mutex g_scratch_mu;

int noalloc_setup(int device) {
    if (device < 0 || device >= OH_MAX_DEVICES) {
        seterr("ornith_hip_init: device %d beyond the %d the library tracks", device, OH_MAX_DEVICES);
        return ORNITH_HIP_ERR_UNSUPPORTED;
    }
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch_dev[device]) return ORNITH_HIP_OK;
    void *p = nullptr;
    HCHK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));   // the current device's copy
    g_scratch_dev[device] = p;
    return ORNITH_HIP_OK;
}

extern "C" int ornith_hip_init(int device, ornith_hip_ctx **out) {
    *out = nullptr;
    int n = 0;
    HCHK(hipGetDeviceCount(&n));
    if (device < 0 || device >= n) {
        seterr("ornith_hip_init: device %d not present (%d visible)", device, n);
        return ORNITH_HIP_ERR_NOTFOUND;
    }
    HCHK(hipSetDevice(device));
    auto *c = new ornith_hip_ctx();
    c->device = device;
    hipError_t e = hipStreamCreateWithFlags(&c->st, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete c;
        seterr("hipStreamCreate: %s", hipGetErrorString(e));
        return ORNITH_HIP_ERR_DEVICE;
    }
    const int r = noalloc_setup(device);
    if (r != ORNITH_HIP_OK) {
        (void)hipStreamDestroy(c->st);
        delete c;
        return r;
    }
    *out = c;
    return ORNITH_HIP_OK;
}

extern "C" int ornith_hip_sync(ornith_hip_ctx *c) {
    HCHK(hipSetDevice(c->device));
    HCHK(hipDeviceSynchronize());
    return ORNITH_HIP_OK;
}

extern "C" void ornith_hip_free(ornith_hip_ctx *c) {
    if (!c) return;
    (void)hipSetDevice(c->device);
    if (c->scratch) (void)hipFree(c->scratch);
    if (c->st) (void)hipStreamDestroy(c->st);
    delete c;
}

size_t elem_block(uint32_t t, size_t *bytes) {
    switch (t) {
    case OH_F32: *bytes = 4; return 1;
    case OH_F16: case OH_BF16: *bytes = 2; return 1;
    case OH_Q8_0: *bytes = 34; return 32;
    case OH_Q4_K: *bytes = 144; return 256;
    case OH_Q6_K: *bytes = 210; return 256;
    case OH_IQ2_XXS: *bytes = 66; return 256;
    default: *bytes = 0; return 0;
    }
}

// GGUF byte size of n elements of type t; 0 if unsupported/misaligned
// (oq_row_bytes, src/ornith_quant.c:140-146)
uint64_t gguf_nbytes(uint32_t t, uint64_t n) {
    size_t bb;
    const size_t be = elem_block(t, &bb);
    if (!be || n % be) return 0;
    return n / be * bb;
}

size_t up256(size_t x) { return (x + 255) & ~(size_t)255; }

// plane sizes of a rows x in tensor
void plane_bytes(uint32_t t, int64_t rows, int64_t in, size_t *a, size_t *b, size_t *c) {
    if (oh_is_quant(t)) {
        const size_t nblk = (size_t)rows * (size_t)(in / 256);
        *a = oh_plane_a_bytes(t, nblk);
        *b = nblk * oh_plane_b(t);
        *c = nblk * oh_plane_c(t);
    } else {
        size_t eb;
        elem_block(t, &eb);
        *a = (size_t)rows * in * eb;
        *b = *c = 0;
    }
}

// GGUF blocks -> planes (same bytes, regrouped)
void repack(uint32_t t, const uint8_t *src, size_t nblk, uint8_t *A, uint8_t *B, uint8_t *C) {
    switch (t) {
    case OH_Q4_K:
        for (size_t i = 0; i < nblk; i++) {
            memcpy(B + 16 * i, src + 144 * i, 16);
            for (int k = 0; k < 128; k += 16) memcpy(A + oh_a_off(t, i, k), src + 144 * i + 16 + k, 16);
        }
        break;
    case OH_Q6_K:
        for (size_t i = 0; i < nblk; i++) {
            for (int k = 0; k < 192; k += 16) memcpy(A + oh_a_off(t, i, k), src + 210 * i + k, 16);
            memcpy(B + 16 * i, src + 210 * i + 192, 16);
            memcpy(C + 2 * i, src + 210 * i + 208, 2);
        }
        break;
    case OH_Q8_0:   // nblk counts 256-element super-blocks = 8 GGUF blocks
        for (size_t i = 0; i < nblk; i++)
            for (int k = 0; k < 8; k++) {
                memcpy(A + oh_a_off(t, i, 32 * k), src + 272 * i + 34 * k + 2, 16);
                memcpy(A + oh_a_off(t, i, 32 * k + 16), src + 272 * i + 34 * k + 18, 16);
                memcpy(B + 16 * i + 2 * k, src + 272 * i + 34 * k, 2);
            }
        break;
    case OH_IQ2_XXS:
        for (size_t i = 0; i < nblk; i++) {
            memcpy(A + 64 * i, src + 66 * i + 2, 64);
            memcpy(C + 2 * i, src + 66 * i, 2);
        }
        break;
    }
}

int tensor_alloc(ornith_hip_ctx *ctx, const char *name, uint32_t type, uint32_t nd,
                        const uint64_t *dims, ornith_hip_tensor **out) {
    *out = nullptr;
    if (nd < 1 || nd > 4) { seterr("tensor '%s': %u dims", name, nd); return ORNITH_HIP_ERR_FORMAT; }
    uint64_t n = 1;
    for (uint32_t d = 0; d < nd; d++) n *= dims[d];
    const uint64_t gb = gguf_nbytes(type, n);
    if (!gb && n) { seterr("tensor '%s': type %u cannot be sized", name, type); return ORNITH_HIP_ERR_UNSUPPORTED; }
    const int64_t in = (int64_t)dims[0];
    if (oh_is_quant(type) && in % 256) {
        seterr("tensor '%s': type %u rows of %lld elements are not 256-block aligned",
               name, type, (long long)in);
        return ORNITH_HIP_ERR_UNSUPPORTED;
    }
    auto *t = new ornith_hip_tensor();
    t->ctx = ctx;
    t->name = name;
    t->type = type;
    t->nd = nd;
    for (uint32_t d = 0; d < nd; d++) t->dims[d] = dims[d];
    t->in = in;
    t->rows = in ? (int64_t)(n / (uint64_t)in) : 0;
    t->gguf_bytes = gb;
    size_t a, b, c;
    plane_bytes(type, t->rows, in, &a, &b, &c);
    const size_t total = up256(a) + up256(b) + up256(c);
    hipError_t e = hipMalloc(&t->mem, total ? total : 256);
    if (e != hipSuccess) {
        delete t;
        seterr("tensor '%s': hipMalloc(%zu): %s", name, total, hipGetErrorString(e));
        return ORNITH_HIP_ERR_OOM;
    }
    t->A = t->mem;
    t->B = t->mem + up256(a);
    t->C = t->B + up256(b);
    *out = t;
    return ORNITH_HIP_OK;
}

extern "C" void ornith_hip_tensor_free(ornith_hip_tensor *t) {
    if (!t) return;
    if (t->mem) (void)hipFree(t->mem);
    if (t->pmem) (void)hipFree(t->pmem);
    delete t;
}

extern "C" int ornith_hip_upload(ornith_hip_ctx *ctx, const char *name, uint32_t type,
                                 const void *host, uint64_t nbytes, uint32_t nd,
                                 const uint64_t *dims, ornith_hip_tensor **out) {
    *out = nullptr;
    ornith_hip_tensor *t;
    CHK(tensor_alloc(ctx, name, type, nd, dims, &t));
    if (nbytes != t->gguf_bytes) {
        seterr("tensor '%s': %llu bytes given, %llu expected", name,
               (unsigned long long)nbytes, (unsigned long long)t->gguf_bytes);
        ornith_hip_tensor_free(t);
        return ORNITH_HIP_ERR_FORMAT;
    }
    size_t a, b, c;
    plane_bytes(type, t->rows, t->in, &a, &b, &c);
    hipError_t e;
    if (oh_is_quant(type)) {
        std::vector<uint8_t> h(up256(a) + up256(b) + up256(c));
        const size_t nblk = (size_t)t->rows * (size_t)(t->in / 256);
        repack(type, (const uint8_t *)host, nblk, h.data(), h.data() + up256(a), h.data() + up256(a) + up256(b));
        e = hipMemcpy(t->mem, h.data(), h.size(), hipMemcpyHostToDevice);
    } else {
        e = hipMemcpy(t->A, host, a, hipMemcpyHostToDevice);
    }
    if (e != hipSuccess) {
        seterr("tensor '%s': upload: %s", name, hipGetErrorString(e));
        ornith_hip_tensor_free(t);
        return ORNITH_HIP_ERR_DEVICE;
    }
    *out = t;
    return ORNITH_HIP_OK;
}

// IQ2_XXS products of the token step summed as a tree over lanes (f32
// arithmetic, each weight decoded exactly; a tolerance path) instead of the
// reference's element-order f32 fallback (src/ornith_rforward.c:119-133):
// ORNITH_HIP_IQ2_TREE=1, read when a step program is built. Off by default.
bool iq2_tree_on() {
    const char *e = getenv("ORNITH_HIP_IQ2_TREE");
    return e && e[0] == '1';
}
// the tree path takes IQ2_XXS rows of 512..4096 inputs (whole codebook
// entries per lane) against an f32 activation the segment already holds
bool iq2_tree_can(uint32_t type, int64_t in) {
    return type == OH_IQ2_XXS && (in == 512 || in == 1024 || in == 2048 || in == 4096) && iq2_tree_on();
}

bool seg_q8(const oh_mvseg &s) {
    return oh_qdot_can((uint32_t)s.type, s.in) && (s.xqs || s.pro != OH_PRO_Q8K);
}
// a segment laid out in wave steps (integer path, or IQ2_XXS tree rows: one row per step)
bool seg_steps(const oh_mvseg &s) { return seg_q8(s) || s.iq2tree; }

// rows: rows of one expert for stacked segments, else all rows of W. nsub
// slots: slot k writes y + k*ystride and reads its activation at k*astride.
int mv_add(MvBuild &b, const ornith_hip_tensor *W, const Act &act, float *y, int mode,
                  const int32_t *eidx, int nsub, int ystride, int astride) {
    if (b.L.n >= OH_MAX_SEGS) { seterr("too many matvec segments"); return ORNITH_HIP_ERR_UNSUPPORTED; }
    oh_mvseg &s = b.L.s[b.L.n];
    memset(&s, 0, sizeof s);
    s.A = W->A; s.B = W->B; s.C = W->C;
    s.xqs = act.qs; s.xd = act.d; s.xbs = act.bs; s.xf = act.xf;
    s.pro = act.pro; s.xf2 = act.xf2; s.nw = act.nw; s.eps = act.eps; s.gdim = act.gdim; s.xruns = act.xruns; s.runs16 = act.runs16;
    s.oqs = act.oqs; s.oqd = act.oqd; s.oqb = act.oqb; s.oxf = act.oxf;
    s.y = y;
    s.eidx = eidx;
    s.nsub = nsub;
    s.ystride = ystride;
    s.astride = astride;
    s.type = (int)W->type;
    s.in = (int)W->in;
    s.rows = eidx ? (int)W->dims[1] : (int)W->rows;
    s.mode = mode;
    s.nb = (int)(W->in / 256);
    if (act.pro == OH_PRO_GNORM && (W->in > 8192 || act.gdim % 64 || W->in % act.gdim || !oh_qdot_can(W->type, W->in))) {
        seterr("matvec '%s': gated-norm prologue needs an integer-path type, in <= 8192 and 64 | head | in", W->name.c_str());
        return ORNITH_HIP_ERR_UNSUPPORTED;
    }
    if (act.pro != OH_PRO_Q8K && (W->in % 256 || W->in > 8192)) {
        seterr("matvec '%s': fused prologue needs in %% 256 == 0 and in <= 8192", W->name.c_str());
        return ORNITH_HIP_ERR_UNSUPPORTED;
    }
    const bool q8 = seg_q8(s);
    s.iq2tree = !q8 && iq2_tree_can(W->type, W->in) && act.xf && (act.pro == OH_PRO_Q8K || act.pro == OH_PRO_F32);
    if (q8) {
        if (s.nb > 64) { seterr("matvec '%s': %d super-blocks per row (max 64)", W->name.c_str(), s.nb); return ORNITH_HIP_ERR_UNSUPPORTED; }
        const int rps = 64 / s.nb;                  // rows per wave step (one super-block per lane)
        s.units = (s.rows + rps - 1) / rps;
    } else if (s.iq2tree) {
        s.units = s.rows;                           // one row per wave step
    } else {
        if (!act.xf) { seterr("matvec '%s': no f32 activation for the fallback path", W->name.c_str()); return ORNITH_HIP_ERR_UNSUPPORTED; }
        if (W->in > 12288) { seterr("matvec '%s': fallback input %lld too wide", W->name.c_str(), (long long)W->in); return ORNITH_HIP_ERR_UNSUPPORTED; }
        s.units = s.rows;
    }
    b.L.n++;
    const double act_bytes = act.pro == OH_PRO_NORM ? 8.0 * W->in
                           : act.pro == OH_PRO_SWIGLU ? 8.0 * W->in
                           : q8 ? (double)W->in * (1.0 + 4.0 / 256 + 32.0 / 256) : (double)W->in * 4.0;
    b.bytes += (double)nsub * ((double)s.rows * (double)gguf_nbytes(W->type, (uint64_t)W->in) + act_bytes +
                               (double)s.rows * 4.0 * (mode == 1 ? 2.0 : 1.0));
    return ORNITH_HIP_OK;
}

// gate/up pair: one segment reducing W and W2 (same type and shape) against
// the same activation, emitting silu(W.x) * (W2.x)
bool pairable(const ornith_hip_tensor *W, const ornith_hip_tensor *W2) {
    return W && W2 && W->type == W2->type && W->in == W2->in && W->rows == W2->rows &&
           (oh_qdot_can(W->type, W->in) || iq2_tree_can(W->type, W->in)) && W->nd == W2->nd;
}
int mv_add_pair(MvBuild &b, const ornith_hip_tensor *W, const ornith_hip_tensor *W2, const Act &act,
                       float *y, const int32_t *eidx, int nsub, int ystride) {
    if (!pairable(W, W2) || (!act.qs && act.pro == OH_PRO_Q8K)) {
        seterr("matvec pair '%s': unsupported", W->name.c_str());
        return ORNITH_HIP_ERR_UNSUPPORTED;
    }
    CHK(mv_add(b, W, act, y, 0, eidx, nsub, ystride, 0));
    oh_mvseg &s = b.L.s[b.L.n - 1];
    if (!seg_steps(s)) {
        b.L.n--;
        seterr("matvec pair '%s': the pair needs the integer or the IQ2_XXS tree path", W->name.c_str());
        return ORNITH_HIP_ERR_UNSUPPORTED;
    }
    s.A2 = W2->A; s.B2 = W2->B; s.C2 = W2->C;
    s.pair = 1;
    b.bytes += (double)nsub * (double)s.rows * (double)gguf_nbytes(W2->type, (uint64_t)W2->in);
    return ORNITH_HIP_OK;
}

// Lay the segments out over blocks: every wave gets a run of whole wave
// steps sized so the launch spreads over about `waves` waves (4096, i.e. 16
// per CU, for a standalone launch; the resident waves of the step kernel).
void mv_plan(MvBuild &b, int waves, int small_waves) {
    int64_t steps = 0;
    // kernel variant: one integer-path type, the Q4_K/Q6_K pair, or any mix
    bool any = false, one = true, q46 = true;
    int t0 = -1;
    for (int i = 0; i < b.L.n; i++) {
        const oh_mvseg &s = b.L.s[i];
        if (seg_steps(s)) steps += (int64_t)s.units * s.nsub * (s.pair ? 2 : 1);
        const bool q8 = seg_q8(s) && !s.iq2tree;
        if (!any) t0 = s.type;
        any = true;
        one = one && q8 && s.type == t0;
        q46 = q46 && q8 && (s.type == OH_Q4_K || s.type == OH_Q6_K);
    }
    b.tk = any && one ? t0 : any && q46 ? OH_MV_Q4Q6 : -1;
    // launches of a few MB: fewer, longer waves (each block forms the
    // activation once, so fewer blocks put less of that traffic ahead of the
    // weights); large ones keep the full spread for bandwidth
    if (small_waves > 0 && steps <= 4 * (int64_t)waves) waves = small_waves;
    // and launches of hundreds of MB (lm_head): two steps per wave, many
    // short blocks, so the last of them finish close together (measured
    // 53.5 us for C3's 286 MB lm_head against 61.8 us at 8 steps per wave)
    int64_t spw = (steps + waves - 1) / waves;
    if (steps > 4 * (int64_t)waves && spw > 2) spw = 2;
    int blocks = 0;
    b.lds = 0;
    for (int i = 0; i < b.L.n; i++) {
        oh_mvseg &s = b.L.s[i];
        const bool q8 = seg_q8(s);
        if (seg_steps(s)) {
            s.upw = (int)(spw / (s.pair ? 2 : 1) > 0 ? spw / (s.pair ? 2 : 1) : 1);
            // a Q6_K step costs about twice a Q4_K one: half the run, so a
            // Q6_K segment beside Q4_K ones (attn_v in the q/k/v launch)
            // ends with them
            if (s.type == OH_Q6_K && s.upw > 1) s.upw = (s.upw + 1) / 2;
            s.bps = (s.units + OH_MV_WAVES * s.upw - 1) / (OH_MV_WAVES * s.upw);
        } else {
            s.upw = 1;
            // IQ2_XXS fallback rows: the split form when the inputs are wide
            // and one lane per row would leave most of the GPU idle
            // (its scale table in LDS takes an even number of super-blocks
            // per row, at most 32)
            s.iq2split = s.type == OH_IQ2_XXS && s.in >= 2048 && s.in <= 8192 && (s.in / 256) % 2 == 0 &&
                         (int64_t)(s.rows + OH_IQ2_ROWS_LANE - 1) / OH_IQ2_ROWS_LANE * s.nsub < 256;
            const int rpb = s.type != OH_IQ2_XXS ? 256 : s.iq2split ? OH_IQ2_ROWS : OH_IQ2_ROWS_LANE;
            s.bps = (s.rows + rpb - 1) / rpb;
        }
        s.block0 = blocks;
        blocks += s.bps * s.nsub;
        const int nb = s.in / 256;
        const int voff = (nb * 272 + nb * 36 + 15) & ~15;
        int need = voff + ((!q8 || s.pro != OH_PRO_Q8K) ? s.in * 4 : 0) + (s.pro == OH_PRO_GNORM ? 512 : 0);
        // + the grid, then the split form's two [OH_IQ2_ROWS][96 + 4] term
        // tiles and its [OH_IQ2_ROWS][nb] half scales (its sign masks sit in
        // the Q8_K planes' place), or the lane form's 2 KB of sign masks
        if (!q8 && s.type == OH_IQ2_XXS)
            need = ((voff + s.in * 4 + 15) & ~15) + 2048 +
                   (s.iq2split ? 2 * OH_IQ2_ROWS * 100 * 4 + OH_IQ2_ROWS * nb * 2 : 2048);
        if (s.iq2tree) need = 0;                    // x in registers, the tables in static LDS
        if (need > b.lds) b.lds = need;
    }
    if (b.L.rtag) {
        // the fused router's copy of the logits for the sequential selection:
        // past every segment's activation, or, when the routed segments are
        // IQ2_XXS fallback rows (of one width), in their term tiles / sign
        // masks, which are written only once the routing is done (the
        // launch's LDS, two blocks per CU, does not grow)
        int iq2 = -1;
        bool other = false;
        for (int i = 0; i < b.L.n; i++) {
            const oh_mvseg &g = b.L.s[i];
            if (!g.eidx) continue;
            const int gnb = g.in / 256, gv = (gnb * 272 + gnb * 36 + 15) & ~15;
            const int off = ((gv + g.in * 4 + 15) & ~15) + 2048;
            if (g.type == OH_IQ2_XXS && !g.iq2tree && (iq2 < 0 || iq2 == off)) iq2 = off;
            else other = true;
        }
        if (iq2 >= 0 && !other && b.L.ne <= 512) {
            b.L.rlg = iq2;
        } else {
            b.L.rlg = (b.lds + 15) & ~15;
            b.lds = b.L.rlg + ((b.L.ne + 3) & ~3) * 4;
        }
    } else if (b.L.route && ((b.L.ne + 3) & ~3) * 4 > b.lds) {
        b.lds = ((b.L.ne + 3) & ~3) * 4;
    }
    b.L.total_blocks = blocks;
}

int mv_go(MvBuild &b, hipStream_t st) {
    mv_plan(b);
    HCHK(oh_launch_matvec(&b.L, b.tk, b.lds, st));
    return ORNITH_HIP_OK;
}
