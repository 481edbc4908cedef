// oh_engine.cpp - host side of the MI355X decode engine: GGUF mmap loading,
// upload into the plane layout, arch inference, sessions and the per-token
// kernel sequence (captured once into HIP graphs and replayed), behind the C
// ABI of include/ornith_hip.h.
//
// Reference: src/ornith_rforward.c (rmodel_* / rsession_*), src/ornith_gguf_write.c
// (GGUF v3 layout), src/ornith_model.h (arch).
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <algorithm>
#include <atomic>
#include <mutex>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include "../../include/ornith_hip.h"
#include "oh_launch.h"
#include "oh_types.h"

// ---- errors (src/ornith_util.c:7,25-30 convention: one global buffer) ---------
static char g_err[1024];
static void seterr(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
}
extern "C" const char *ornith_hip_last_error(void) { return g_err; }

#define HCHK(call)                                                                    \
    do {                                                                              \
        hipError_t e_ = (call);                                                       \
        if (e_ != hipSuccess) {                                                       \
            seterr("%s: %s (%s:%d)", #call, hipGetErrorString(e_), __FILE__, __LINE__); \
            return e_ == hipErrorOutOfMemory ? ORNITH_HIP_ERR_OOM : ORNITH_HIP_ERR_DEVICE; \
        }                                                                             \
    } while (0)
#define CHK(expr)                     \
    do {                              \
        int st_ = (expr);             \
        if (st_ != ORNITH_HIP_OK) return st_; \
    } while (0)

// ---- context -----------------------------------------------------------------------
struct ornith_hip_ctx {
    int device = 0;
    hipStream_t st = nullptr;
    void *scratch = nullptr;
    size_t scratch_bytes = 0;
};

static int ctx_scratch(ornith_hip_ctx *c, size_t bytes, void **out) {
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

// ---- the no-allocation matvec's scratch --------------------------------------------
// ornith_hip_matvec_noalloc stages its input, output and Q8_K planes in this
// fixed device array instead of allocating. Each device holds its own copy
// until the process ends. In host code `scratch` only names the symbol:
// kernels and copies get the device address that hipGetSymbolAddress returns
// for the current device, resolved once per device by ornith_hip_init.
#define OH_NOALLOC_SCRATCH_BYTES (4u << 20)
static __device__ __align__(256) uint8_t scratch[OH_NOALLOC_SCRATCH_BYTES];
#define OH_MAX_DEVICES 64
static void *g_scratch_dev[OH_MAX_DEVICES];
static std::mutex g_scratch_mu;

static int noalloc_setup(int device) {
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

// ---- tensors in the plane layout (oh_types.h) ---------------------------------------
struct ornith_hip_tensor {
    ornith_hip_ctx *ctx = nullptr;
    std::string name;
    uint32_t type = 0, nd = 0;
    uint64_t dims[4] = {0, 0, 0, 0};
    int64_t in = 0, rows = 0;
    uint64_t gguf_bytes = 0;
    uint8_t *mem = nullptr;
    uint8_t *A = nullptr, *B = nullptr, *C = nullptr;
};

static size_t elem_block(uint32_t t, size_t *bytes) {
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
static uint64_t gguf_nbytes(uint32_t t, uint64_t n) {
    size_t bb;
    const size_t be = elem_block(t, &bb);
    if (!be || n % be) return 0;
    return n / be * bb;
}

static size_t up256(size_t x) { return (x + 255) & ~(size_t)255; }

// plane sizes of a rows x in tensor
static void plane_bytes(uint32_t t, int64_t rows, int64_t in, size_t *a, size_t *b, size_t *c) {
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
static void repack(uint32_t t, const uint8_t *src, size_t nblk, uint8_t *A, uint8_t *B, uint8_t *C) {
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

static int tensor_alloc(ornith_hip_ctx *ctx, const char *name, uint32_t type, uint32_t nd,
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

// ---- matvec launch builder ------------------------------------------------------------
// Activation of a matvec segment: Q8_K planes (+ f32 for fallback rows), or
// formed inside the launch from f32 inputs (RMSNorm or SwiGLU prologue).
struct Act {
    const int8_t *qs = nullptr;
    const float *d = nullptr;
    const int16_t *bs = nullptr;
    const float *xf = nullptr;
    int pro = OH_PRO_Q8K, gdim = 0;
    const float *xf2 = nullptr, *nw = nullptr;
    const double *xruns = nullptr;
    int runs16 = 0;            // xruns: 16-row partials (OH_OP_DELTA16) instead of 64-row run sums
    float eps = 0.0f;
    int8_t *oqs = nullptr;     // prologue result stored for later launches
    float *oqd = nullptr;
    int16_t *oqb = nullptr;
    float *oxf = nullptr;
};

struct MvBuild {
    oh_mvlaunch L;
    int lds = 0;
    int tk = -1;           // kernel variant (see oh_launch_matvec)
    double bytes = 0.0;    // algorithmic HBM bytes: weights read + activation + output
    MvBuild() { memset(&L, 0, sizeof L); }
};

// IQ2_XXS products of the token step summed as a tree over lanes (f32
// arithmetic, each weight decoded exactly; a tolerance path) instead of the
// reference's element-order f32 fallback (src/ornith_rforward.c:119-133):
// ORNITH_HIP_IQ2_TREE=1, read when a step program is built. Off by default.
static bool iq2_tree_on() {
    const char *e = getenv("ORNITH_HIP_IQ2_TREE");
    return e && e[0] == '1';
}
// the tree path takes IQ2_XXS rows of 512..4096 inputs (whole codebook
// entries per lane) against an f32 activation the segment already holds
static bool iq2_tree_can(uint32_t type, int64_t in) {
    return type == OH_IQ2_XXS && (in == 512 || in == 1024 || in == 2048 || in == 4096) && iq2_tree_on();
}

static bool seg_q8(const oh_mvseg &s) {
    return oh_qdot_can((uint32_t)s.type, s.in) && (s.xqs || s.pro != OH_PRO_Q8K);
}
// a segment laid out in wave steps (integer path, or IQ2_XXS tree rows: one row per step)
static bool seg_steps(const oh_mvseg &s) { return seg_q8(s) || s.iq2tree; }

// rows: rows of one expert for stacked segments, else all rows of W. nsub
// slots: slot k writes y + k*ystride and reads its activation at k*astride.
static int mv_add(MvBuild &b, const ornith_hip_tensor *W, const Act &act, float *y, int mode,
                  const int32_t *eidx = nullptr, int nsub = 1, int ystride = 0, int astride = 0) {
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
static bool pairable(const ornith_hip_tensor *W, const ornith_hip_tensor *W2) {
    return W && W2 && W->type == W2->type && W->in == W2->in && W->rows == W2->rows &&
           (oh_qdot_can(W->type, W->in) || iq2_tree_can(W->type, W->in)) && W->nd == W2->nd;
}
static int mv_add_pair(MvBuild &b, const ornith_hip_tensor *W, const ornith_hip_tensor *W2, const Act &act,
                       float *y, const int32_t *eidx = nullptr, int nsub = 1, int ystride = 0) {
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
static void mv_plan(MvBuild &b, int waves = 4096) {
    int64_t steps = 0;
    int tk = -2;
    for (int i = 0; i < b.L.n; i++) {
        const oh_mvseg &s = b.L.s[i];
        if (seg_steps(s)) {
            steps += (int64_t)s.units * s.nsub * (s.pair ? 2 : 1);
            tk = (tk == -2 || tk == s.type) && !s.iq2tree ? s.type : -1;
        } else {
            tk = -1;
        }
    }
    b.tk = tk < 0 ? -1 : tk;
    const int64_t spw = (steps + waves - 1) / waves;
    int blocks = 0;
    b.lds = 0;
    for (int i = 0; i < b.L.n; i++) {
        oh_mvseg &s = b.L.s[i];
        const bool q8 = seg_q8(s);
        if (seg_steps(s)) {
            s.upw = (int)(spw / (s.pair ? 2 : 1) > 0 ? spw / (s.pair ? 2 : 1) : 1);
            s.bps = (s.units + OH_MV_WAVES * s.upw - 1) / (OH_MV_WAVES * s.upw);
        } else {
            s.upw = 1;
            // IQ2_XXS fallback rows: the split form when the inputs are wide
            // and one lane per row would leave most of the GPU idle
            s.iq2split = s.type == OH_IQ2_XXS && s.in >= 2048 &&
                         (int64_t)(s.rows + OH_IQ2_ROWS_LANE - 1) / OH_IQ2_ROWS_LANE * s.nsub < 256;
            const int rpb = s.type != OH_IQ2_XXS ? 256 : s.iq2split ? OH_IQ2_ROWS : OH_IQ2_ROWS_LANE;
            s.bps = (s.rows + rpb - 1) / rpb;
        }
        s.block0 = blocks;
        blocks += s.bps * s.nsub;
        const int nb = s.in / 256;
        const int voff = (nb * 272 + nb * 36 + 15) & ~15;
        int need = voff + ((!q8 || s.pro != OH_PRO_Q8K) ? s.in * 4 : 0) + (s.pro == OH_PRO_GNORM ? 512 : 0);
        // + the grid (and the split form's two [OH_IQ2_ROWS][96 + 4] term tiles)
        if (!q8 && s.type == OH_IQ2_XXS)
            need = ((voff + s.in * 4 + 15) & ~15) + 2048 + (s.iq2split ? 2 * OH_IQ2_ROWS * 100 * 4 : 0);
        if (s.iq2tree) need = 0;                    // x in registers, the tables in static LDS
        if (need > b.lds) b.lds = need;
    }
    if (b.L.route && ((b.L.ne + 3) & ~3) * 4 > b.lds) b.lds = ((b.L.ne + 3) & ~3) * 4;
    b.L.total_blocks = blocks;
}

static int mv_go(MvBuild &b, hipStream_t st) {
    mv_plan(b);
    HCHK(oh_launch_matvec(&b.L, b.tk, b.lds, st));
    return ORNITH_HIP_OK;
}

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
static bool mmq_enabled() {
    const char *e = getenv("ORNITH_HIP_MMQ");
    return !(e && e[0] == '0');
}

// device bytes of matvec_cols' buffer: input, output, Q8_K planes (256-aligned)
static size_t matvec_col_bytes(int64_t in, int64_t out) {
    return (size_t)in * 5 + (size_t)(in / 256) * 40 + (size_t)out * 4 + 4096;
}
static int matvec_cols(ornith_hip_ctx *ctx, const ornith_hip_tensor *W, const float *x, float *y, int Tn,
                       void *sp);

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
            oh_mmq M;
            memset(&M, 0, sizeof M);
            M.A = W->A; M.B = W->B; M.C = W->C; M.type = (int)W->type;
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
static int matvec_cols(ornith_hip_ctx *ctx, const ornith_hip_tensor *W, const float *x, float *y, int Tn,
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

// ---- GGUF v3 mmap reader (format: src/ornith_gguf_write.c:1-11) --------------------------
namespace {

struct GgufKV { uint32_t vt; const uint8_t *val; size_t len; };
struct GgufT { std::string name; uint32_t nd, type; uint64_t dims[4]; uint64_t off; const uint8_t *data; uint64_t nbytes; };

struct Gguf {
    uint8_t *map = nullptr;
    size_t size = 0;
    std::unordered_map<std::string, GgufKV> kv;
    std::vector<GgufT> ts;
    ~Gguf() { if (map) munmap(map, size); }
};

struct Rd {
    const uint8_t *p, *end;
    bool take(void *dst, size_t n) {
        if ((size_t)(end - p) < n) return false;
        if (dst) memcpy(dst, p, n);
        p += n;
        return true;
    }
};

size_t gguf_scalar(uint32_t vt) {
    switch (vt) {
    case 0: case 1: case 7: return 1;
    case 2: case 3: return 2;
    case 4: case 5: case 6: return 4;
    case 10: case 11: case 12: return 8;
    default: return 0;
    }
}

bool gguf_skip(Rd &r, uint32_t vt, int depth) {
    if (vt == 8) { uint64_t n; return r.take(&n, 8) && r.take(nullptr, n); }
    if (vt == 9) {
        uint32_t et; uint64_t n;
        if (depth > 3 || !r.take(&et, 4) || !r.take(&n, 8)) return false;
        for (uint64_t i = 0; i < n; i++) if (!gguf_skip(r, et, depth + 1)) return false;
        return true;
    }
    const size_t s = gguf_scalar(vt);
    return s && r.take(nullptr, s);
}

int gguf_open(const char *path, Gguf &g) {
    const int fd = open(path, O_RDONLY);
    if (fd < 0) { seterr("cannot open %s", path); return ORNITH_HIP_ERR_IO; }
    struct stat st;
    if (fstat(fd, &st) != 0) { close(fd); seterr("fstat %s failed", path); return ORNITH_HIP_ERR_IO; }
    g.size = (size_t)st.st_size;
    void *m = g.size ? mmap(nullptr, g.size, PROT_READ, MAP_PRIVATE, fd, 0) : MAP_FAILED;
    close(fd);
    if (m == MAP_FAILED) { g.size = 0; seterr("mmap %s failed", path); return ORNITH_HIP_ERR_IO; }
    g.map = (uint8_t *)m;
    Rd r{g.map, g.map + g.size};
    char magic[4];
    uint32_t ver;
    uint64_t nt, nkv;
    if (!r.take(magic, 4) || memcmp(magic, "GGUF", 4) != 0) { seterr("not a GGUF file (bad magic)"); return ORNITH_HIP_ERR_FORMAT; }
    if (!r.take(&ver, 4) || !r.take(&nt, 8) || !r.take(&nkv, 8)) { seterr("truncated GGUF header"); return ORNITH_HIP_ERR_FORMAT; }
    if (ver < 2 || ver > 3) { seterr("unsupported GGUF version %u", ver); return ORNITH_HIP_ERR_UNSUPPORTED; }
    if (nt > (1u << 24) || nkv > (1u << 24)) { seterr("implausible GGUF counts"); return ORNITH_HIP_ERR_FORMAT; }
    uint32_t align = 32;
    for (uint64_t i = 0; i < nkv; i++) {
        uint64_t kl;
        if (!r.take(&kl, 8) || (size_t)(r.end - r.p) < kl) { seterr("bad GGUF key #%llu", (unsigned long long)i); return ORNITH_HIP_ERR_FORMAT; }
        std::string key((const char *)r.p, kl);
        r.p += kl;
        GgufKV v;
        if (!r.take(&v.vt, 4)) { seterr("bad GGUF value type for '%s'", key.c_str()); return ORNITH_HIP_ERR_FORMAT; }
        v.val = r.p;
        if (!gguf_skip(r, v.vt, 0)) { seterr("bad GGUF value for '%s'", key.c_str()); return ORNITH_HIP_ERR_FORMAT; }
        v.len = (size_t)(r.p - v.val);
        if (key == "general.alignment" && v.vt == 4 && v.len >= 4) { uint32_t a; memcpy(&a, v.val, 4); if (a) align = a; }
        g.kv[key] = v;
    }
    g.ts.resize(nt);
    for (uint64_t i = 0; i < nt; i++) {
        GgufT &t = g.ts[i];
        uint64_t nl;
        if (!r.take(&nl, 8) || (size_t)(r.end - r.p) < nl) { seterr("bad GGUF tensor record #%llu", (unsigned long long)i); return ORNITH_HIP_ERR_FORMAT; }
        t.name.assign((const char *)r.p, nl);
        r.p += nl;
        if (!r.take(&t.nd, 4) || t.nd > 4 || t.nd < 1) { seterr("tensor '%s': bad dims", t.name.c_str()); return ORNITH_HIP_ERR_FORMAT; }
        uint64_t n = 1;
        for (uint32_t d = 0; d < t.nd; d++) {
            if (!r.take(&t.dims[d], 8)) { seterr("tensor '%s': bad dims", t.name.c_str()); return ORNITH_HIP_ERR_FORMAT; }
            n *= t.dims[d];
        }
        if (!r.take(&t.type, 4) || !r.take(&t.off, 8)) { seterr("tensor '%s': bad type/offset", t.name.c_str()); return ORNITH_HIP_ERR_FORMAT; }
        t.nbytes = gguf_nbytes(t.type, n);
        if (!t.nbytes && n) { seterr("tensor '%s': cannot size type %u for load", t.name.c_str(), t.type); return ORNITH_HIP_ERR_UNSUPPORTED; }
    }
    const size_t data0 = ((size_t)(r.p - g.map) + align - 1) / align * align;
    if (data0 > g.size) { seterr("data section starts past EOF"); return ORNITH_HIP_ERR_FORMAT; }
    for (auto &t : g.ts) {
        if (t.off > g.size - data0 || t.nbytes > g.size - data0 - t.off) {
            seterr("tensor '%s' data extends past EOF", t.name.c_str());
            return ORNITH_HIP_ERR_FORMAT;
        }
        t.data = g.map + data0 + t.off;
    }
    return ORNITH_HIP_OK;
}

} // namespace

// ---- model --------------------------------------------------------------------------------
struct OhLayer {
    bool full = false;
    ornith_hip_tensor *attn_norm = nullptr, *post_norm = nullptr;
    ornith_hip_tensor *q = nullptr, *k = nullptr, *v = nullptr, *q_norm = nullptr, *k_norm = nullptr, *o = nullptr;
    ornith_hip_tensor *qkv = nullptr, *conv = nullptr, *ssm_a = nullptr, *dt_bias = nullptr, *ssm_norm = nullptr;
    ornith_hip_tensor *alpha = nullptr, *beta = nullptr, *gate = nullptr, *ssm_out = nullptr;
    ornith_hip_tensor *router = nullptr, *gate_exps = nullptr, *up_exps = nullptr, *down_exps = nullptr;
    ornith_hip_tensor *gate_sh = nullptr, *up_sh = nullptr, *down_sh = nullptr, *gate_inp_sh = nullptr;
    ornith_hip_tensor *ffn_gate = nullptr, *ffn_up = nullptr, *ffn_down = nullptr;
};

struct ornith_hip_model {
    ornith_hip_ctx *ctx = nullptr;
    ornith_hip_arch a;
    std::vector<ornith_hip_tensor *> ts;
    std::unordered_map<std::string, ornith_hip_tensor *> by;
    std::vector<OhLayer> L;
    ornith_hip_tensor *embd = nullptr, *out_norm = nullptr, *lm_head = nullptr;
    uint64_t bytes = 0;
};

extern "C" void ornith_hip_model_free(ornith_hip_model *m) {
    if (!m) return;
    for (auto *t : m->ts) ornith_hip_tensor_free(t);
    delete m;
}

static ornith_hip_tensor *mt(const ornith_hip_model *m, const std::string &n) {
    auto it = m->by.find(n);
    return it == m->by.end() ? nullptr : it->second;
}
static ornith_hip_tensor *mb(const ornith_hip_model *m, int l, const char *sfx) {
    return mt(m, "blk." + std::to_string(l) + "." + sfx);
}

// metadata view shared by the GGUF and synthetic paths
struct Meta {
    std::string arch = "qwen35";
    std::unordered_map<std::string, uint32_t> u32;
    std::unordered_map<std::string, float> f32;
    bool has_tokens = false;
    int32_t eos = -1;
};

static bool is_full(const ornith_hip_arch &a, int l) {
    return a.full_interval > 0 && l % a.full_interval == a.full_interval - 1;
}

// shape inference of rmodel_load (src/ornith_rforward.c:728-803) + the engine's
// own limits, checked loudly
static int infer_arch(ornith_hip_model *m, const Meta &md) {
    ornith_hip_arch &a = m->a;
    memset(&a, 0, sizeof a);
    auto U = [&](const char *sfx, uint32_t def) {
        auto it = md.u32.find(md.arch + "." + sfx);
        return it == md.u32.end() ? def : it->second;
    };
    auto Fl = [&](const char *sfx, float def) {
        auto it = md.f32.find(md.arch + "." + sfx);
        return it == md.f32.end() ? def : it->second;
    };
    m->embd = mt(m, "token_embd.weight");
    a.hidden = m->embd ? (int)m->embd->dims[0] : (int)U("embedding_length", 4096);
    a.vocab = m->embd ? (int)m->embd->dims[1] : 248320;
    int n = 0;
    while (mb(m, n, "attn_norm.weight")) n++;
    a.n_layers = n ? n : (int)U("block_count", 32);
    int ff = -1;
    for (int i = 0; i < a.n_layers; i++) if (mb(m, i, "attn_q.weight")) { ff = i; break; }
    a.full_interval = ff >= 0 ? ff + 1 : (int)U("full_attention_interval", 4);
    a.rope_theta = Fl("rope.freq_base", 1e7f);
    a.eps = Fl("attention.layer_norm_rms_epsilon", 1e-6f);
    a.rope_dim = (int)U("rope.dimension_count", 64);
    {
        const int fl = a.full_interval - 1;
        auto *qn = mb(m, fl, "attn_q_norm.weight"), *q = mb(m, fl, "attn_q.weight"), *k = mb(m, fl, "attn_k.weight");
        a.hd = qn ? (int)qn->dims[0] : 256;
        const int qout = q ? (int)q->dims[1] : a.hd * 16;
        a.nh = (qout / 2) / a.hd;
        a.nkv = k ? (int)k->dims[1] / a.hd : 4;
    }
    {
        int l0 = 0;
        while (l0 < a.n_layers && is_full(a, l0)) l0++;
        auto *sa = mb(m, l0, "ssm_a"), *sn = mb(m, l0, "ssm_norm.weight"), *qkv = mb(m, l0, "attn_qkv.weight"),
             *cv = mb(m, l0, "ssm_conv1d.weight");
        a.nv = sa ? (int)sa->dims[0] : 32;
        a.dv = sn ? (int)sn->dims[0] : 128;
        a.dk = a.dv;
        a.conv_k = cv ? (int)cv->dims[0] : 4;
        const int cc = qkv ? (int)qkv->dims[1] : 8192;
        const int qd = (cc - a.nv * a.dv) / 2;
        a.nk = a.dk ? qd / a.dk : 16;
    }
    auto *ge0 = mb(m, 0, "ffn_gate_exps.weight");
    if (ge0) {
        a.ne = (int)ge0->dims[2];
        a.moe_inter = (int)ge0->dims[1];
        a.top_k = (int)U("expert_used_count", 8);
        auto *sh = mb(m, 0, "ffn_gate_shexp.weight");
        a.shared_inter = sh ? (int)sh->dims[1] : 0;
    } else {
        auto *fg = mb(m, 0, "ffn_gate.weight");
        a.shared_inter = fg ? (int)fg->dims[1] : (int)U("feed_forward_length", 12288);
    }
    if (!md.has_tokens) { seterr("no tokenizer.ggml.tokens"); return ORNITH_HIP_ERR_FORMAT; }
    a.eos = md.eos;
    m->out_norm = mt(m, "output_norm.weight");
    m->lm_head = mt(m, "output.weight");
    m->L.assign((size_t)a.n_layers, OhLayer());
    for (int l = 0; l < a.n_layers; l++) {
        OhLayer &y = m->L[l];
        y.full = is_full(a, l);
        y.attn_norm = mb(m, l, "attn_norm.weight"); y.post_norm = mb(m, l, "post_attention_norm.weight");
        y.q = mb(m, l, "attn_q.weight"); y.k = mb(m, l, "attn_k.weight"); y.v = mb(m, l, "attn_v.weight");
        y.o = mb(m, l, "attn_output.weight");
        y.q_norm = mb(m, l, "attn_q_norm.weight"); y.k_norm = mb(m, l, "attn_k_norm.weight");
        y.qkv = mb(m, l, "attn_qkv.weight"); y.conv = mb(m, l, "ssm_conv1d.weight");
        y.ssm_a = mb(m, l, "ssm_a"); y.dt_bias = mb(m, l, "ssm_dt.bias"); y.ssm_norm = mb(m, l, "ssm_norm.weight");
        y.alpha = mb(m, l, "ssm_alpha.weight"); y.beta = mb(m, l, "ssm_beta.weight");
        y.gate = mb(m, l, "attn_gate.weight"); y.ssm_out = mb(m, l, "ssm_out.weight");
        y.router = mb(m, l, "ffn_gate_inp.weight");
        y.gate_exps = mb(m, l, "ffn_gate_exps.weight"); y.up_exps = mb(m, l, "ffn_up_exps.weight");
        y.down_exps = mb(m, l, "ffn_down_exps.weight");
        y.gate_sh = mb(m, l, "ffn_gate_shexp.weight"); y.up_sh = mb(m, l, "ffn_up_shexp.weight");
        y.down_sh = mb(m, l, "ffn_down_shexp.weight"); y.gate_inp_sh = mb(m, l, "ffn_gate_inp_shexp.weight");
        y.ffn_gate = mb(m, l, "ffn_gate.weight"); y.ffn_up = mb(m, l, "ffn_up.weight"); y.ffn_down = mb(m, l, "ffn_down.weight");
    }
    // ---- what this engine supports (checked, never assumed) ----
    auto bad = [&](const char *why) { seterr("unsupported model: %s", why); return ORNITH_HIP_ERR_UNSUPPORTED; };
    auto need_f32 = [&](const ornith_hip_tensor *t) { return t && t->type == OH_F32; };
    if (!m->embd || !m->out_norm || !m->lm_head) return bad("token_embd/output_norm/output missing");
    if (a.hidden % 256 || a.hidden > 8192) return bad("hidden must be a multiple of 256, <= 8192");
    if (!need_f32(m->out_norm)) return bad("output_norm must be F32 (read as raw floats)");
    for (int l = 0; l < a.n_layers; l++) {
        const OhLayer &y = m->L[l];
        if (!need_f32(y.attn_norm) || !need_f32(y.post_norm)) return bad("layer norms must be F32");
        if (y.full) {
            if (!y.q || !y.k || !y.v || !y.o || !need_f32(y.q_norm) || !need_f32(y.k_norm)) return bad("full-attention tensors missing or not F32 norms");
            if (a.hd != 64 && a.hd != 128 && a.hd != 256) return bad("head_dim must be 64, 128 or 256");
            if (a.nh % a.nkv || a.nh / a.nkv > 16 || (a.nh / a.nkv & (a.nh / a.nkv - 1)))
                return bad("query heads per KV head must be a power of two <= 16");
            if (a.nkv < 1 || a.nh % a.nkv) return bad("n_heads must be a multiple of n_kv_heads");
            if ((a.nh * a.hd) % 256 || a.nh * a.hd > 8192) return bad("n_heads*head_dim must be a multiple of 256, <= 8192");
        } else {
            if (!y.qkv || !y.alpha || !y.beta || !y.gate || !y.ssm_out) return bad("linear-attention projections missing");
            if (!need_f32(y.conv) || !need_f32(y.ssm_a) || !need_f32(y.dt_bias) || !need_f32(y.ssm_norm))
                return bad("ssm_conv1d/ssm_a/ssm_dt.bias/ssm_norm must be F32");
            if (a.dk != 64 && a.dk != 128) return bad("linear head dim must be 64 or 128");
            if (a.nv % (256 / a.dk) || a.nk < 1) return bad("linear value heads must fill 256-element blocks");
            if (a.conv_k < 2 || a.conv_k > 8) return bad("conv kernel must be in [2, 8]");
            if (a.nv * a.dv > 8192) return bad("linear value width must be <= 8192");
        }
        if (a.ne > 0) {
            if (!y.router || !y.gate_exps || !y.up_exps || !y.down_exps) return bad("MoE tensors missing");
            if (a.ne > 1024 || a.top_k < 1 || a.top_k > 16 || a.top_k > a.ne) return bad("experts <= 1024 and 1 <= top_k <= 16");
            if (a.moe_inter % 256 || a.moe_inter > 8192) return bad("expert FFN width must be a multiple of 256, <= 8192");
            if (y.gate_sh && (a.shared_inter % 256 || a.shared_inter > 8192)) return bad("shared FFN width must be a multiple of 256");
        } else {
            if (!y.ffn_gate || !y.ffn_up || !y.ffn_down) return bad("dense FFN tensors missing");
            if (a.shared_inter % 256 || a.shared_inter > 8192) return bad("FFN width must be a multiple of 256");
        }
    }
    return ORNITH_HIP_OK;
}

extern "C" int ornith_hip_model_load(ornith_hip_ctx *ctx, const char *path, ornith_hip_model **out) {
    *out = nullptr;
    HCHK(hipSetDevice(ctx->device));
    Gguf g;
    CHK(gguf_open(path, g));
    Meta md;
    auto it = g.kv.find("general.architecture");
    if (it != g.kv.end() && it->second.vt == 8 && it->second.len >= 8) {
        uint64_t n;
        memcpy(&n, it->second.val, 8);
        if (n <= it->second.len - 8 && n < 64) md.arch.assign((const char *)it->second.val + 8, n);
    }
    for (auto &kv : g.kv) {
        if ((kv.second.vt == 4 || kv.second.vt == 5) && kv.second.len >= 4) { uint32_t v; memcpy(&v, kv.second.val, 4); md.u32[kv.first] = v; }
        if (kv.second.vt == 6 && kv.second.len >= 4) { float v; memcpy(&v, kv.second.val, 4); md.f32[kv.first] = v; }
    }
    md.has_tokens = g.kv.count("tokenizer.ggml.tokens") > 0;
    auto ie = g.kv.find("tokenizer.ggml.eos_token_id");
    if (ie != g.kv.end() && ie->second.len >= 4) memcpy(&md.eos, ie->second.val, 4);
    auto *m = new ornith_hip_model();
    m->ctx = ctx;
    for (auto &t : g.ts) {
        ornith_hip_tensor *dt;
        int st = ornith_hip_upload(ctx, t.name.c_str(), t.type, t.data, t.nbytes, t.nd, t.dims, &dt);
        if (st) { ornith_hip_model_free(m); return st; }
        m->ts.push_back(dt);
        m->by[t.name] = dt;
        m->bytes += dt->gguf_bytes;
    }
    int st = infer_arch(m, md);
    if (st) { ornith_hip_model_free(m); return st; }
    *out = m;
    return ORNITH_HIP_OK;
}

extern "C" int ornith_hip_model_arch(const ornith_hip_model *m, ornith_hip_arch *out) {
    *out = m->a;
    return ORNITH_HIP_OK;
}
extern "C" uint64_t ornith_hip_model_bytes(const ornith_hip_model *m) { return m->bytes; }
extern "C" const ornith_hip_tensor *ornith_hip_model_tensor(const ornith_hip_model *m, const char *name) {
    return mt(m, name);
}
extern "C" int ornith_hip_model_tensor_info(const ornith_hip_model *m, const char *name, uint32_t *type,
                                            uint64_t *nbytes, uint64_t *rows, uint64_t *in) {
    auto *t = mt(m, name);
    if (!t) { seterr("no tensor '%s'", name); return ORNITH_HIP_ERR_NOTFOUND; }
    if (type) *type = t->type;
    if (nbytes) *nbytes = t->gguf_bytes;
    if (rows) *rows = (uint64_t)t->rows;
    if (in) *in = (uint64_t)t->in;
    return ORNITH_HIP_OK;
}

// ---- sessions -----------------------------------------------------------------------------
// Q8_K planes; bp: per super-block the pair-sum bytes of the matrix-core
// product's min term
struct Q8Buf { int8_t *qs = nullptr; float *d = nullptr; int16_t *bs = nullptr; int8_t *bp = nullptr; };

struct LayerState {
    float *S = nullptr, *conv = nullptr;                 // linear
    uint32_t *Kt = nullptr; float *Ks = nullptr;         // full (Q8 KV)
    int8_t *Vq = nullptr; float *Vs = nullptr;
};

struct ornith_hip_session {
    ornith_hip_model *m = nullptr;
    uint64_t sid = 0;             // unique per session of the process
    int cap = 0, pos = 0, kvcap = 0;
    bool have_logits = false;
    std::vector<void *> allocs;
    std::vector<size_t> asz;      // bytes requested for each of allocs
    int32_t *io = nullptr;        // [0] pos, [1] best
    int32_t *toks = nullptr;      // [cap + 1]
    float *x = nullptr, *xn = nullptr;
    Q8Buf xq;
    float *cat = nullptr, *gate = nullptr, *ab = nullptr;
    float *o = nullptr;
    Q8Buf oq;
    float *qproj = nullptr, *kb = nullptr, *vb = nullptr, *qr = nullptr, *agate = nullptr, *scores = nullptr;
    float *fpo = nullptr;         // flash attention: chunk outputs [nkv][chunks][nh/nkv][hd]
    float *fpml = nullptr;        // flash attention: chunk (max, sum) [nkv][chunks][nh/nkv][2]
    float *ddots = nullptr;       // step kernel's MoE down: slot dots [slots][hidden]
    int *dcnt = nullptr;          // step kernel's MoE down: blocks done per row group
    float *osz = nullptr;         // delta step: silu(gate) per output row
    double *oruns = nullptr;      // delta step: sum of o^2 per 16-row run (per 64 rows: the step kernel)
    int exact_max = 1024;         // contexts up to this walk the attention sum in one block
    int flash_mfma = 1;           // decode flash chunks on the matrix cores (ORNITH_HIP_FLASH_MFMA=0: VALU)
    float2 *rope = nullptr;
    float *rl = nullptr, *shl = nullptr, *shg = nullptr, *ew = nullptr;
    int32_t *eidx = nullptr;
    float *g = nullptr, *u = nullptr, *h = nullptr, *od = nullptr;
    Q8Buf hq;
    float *logits = nullptr, *amv = nullptr;
    int *ami = nullptr;
    std::vector<LayerState> ls;
    hipGraphExec_t gbody = nullptr, ghead = nullptr;
    bool graphs_tried = false;
    // per-launch timing of an eager step (profile_step): events around each launch
    bool rec = false;
    std::vector<hipEvent_t> rec_ev;
    std::vector<int> rec_kind;
    std::vector<double> rec_bytes;
    // kind replay (time_kind): launch only the kernels of one kind
    int only = -1;
    int only_n = 0;
    double only_bytes = 0.0;
    // persistent step kernel: the body and head programs in device memory,
    // their barrier counters, the grid, and (profiling) phase timestamps
    struct StepProg { oh_op *ops = nullptr; unsigned *ctrs = nullptr; int n = 0, lds = 0; double bytes = 0.0; };
    StepProg sp_body, sp_head;
    // layer-major prefill: buffers for chunks of up to pf_tc tokens
    struct Pf {
        int tc = 0;
        int32_t pos_after = 0;
        int last_base = 0, last_T = 0;   // the most recent chunk (its buffers hold the last layer's rows)
        float *X = nullptr, *CAT = nullptr, *Z = nullptr, *A = nullptr, *Bg = nullptr, *CONV = nullptr;
        float *QN = nullptr, *KN = nullptr, *AL = nullptr, *BE = nullptr, *O = nullptr;
        float *QP = nullptr, *KB = nullptr, *VB = nullptr, *QR = nullptr, *AG = nullptr, *OA = nullptr;
        float *FPO = nullptr, *FPML = nullptr, *RL = nullptr, *SHL = nullptr, *SHG = nullptr, *RW = nullptr;
        int32_t *RIDX = nullptr, *CNT = nullptr, *LIST = nullptr;
        float *Hh = nullptr, *HSH = nullptr, *OD = nullptr, *ODSH = nullptr, *STAGE = nullptr, *GR = nullptr;
        float *GU = nullptr, *GSH = nullptr;      // [gate | up] rows of the matrix-core pairs
        float *WY = nullptr;                      // WY factors of the matrix-core delta chunks (on first use)
        float *XN = nullptr;                      // f32 normalised rows for the per-token expert kernels
        int32_t *ITEMS = nullptr;
        Q8Buf XQ, OQ, OAQ, HQ, HSQ;
    } pf;
    // batch decode led by this session: buffers for up to bw_n sessions
    struct Bw {
        int n = 0;
        float *X = nullptr, *CAT = nullptr, *Z = nullptr, *AB = nullptr, *O = nullptr, *OG = nullptr;
        double *RUNS = nullptr;
        float *QP = nullptr, *KB = nullptr, *VB = nullptr, *QR = nullptr, *AG = nullptr, *OA = nullptr;
        float *RL = nullptr, *SHL = nullptr, *SHG = nullptr, *RW = nullptr, *LOGITS = nullptr;
        int32_t *RIDX = nullptr, *CNT = nullptr, *LIST = nullptr, *ITEMS = nullptr, *IDX = nullptr;
        float *Hh = nullptr, *HSH = nullptr, *OD = nullptr, *ODSH = nullptr, *GU = nullptr, *GSH = nullptr;
        float *AMV = nullptr;          // argmax stage-1 bests [n][OH_ARGMAX_BLOCKS]
        int32_t *AMI = nullptr;
        uint8_t *OPS = nullptr;
        size_t ops_bytes = 0;
        int gen = 0;                   // bumped when the buffers are reallocated
        Q8Buf XQ, OQ, OAQ, HQ, HSQ;
        hipGraphExec_t graph = nullptr;  // the captured step of the key's sessions
        std::vector<uint64_t> key;
    } bw;
    std::vector<int> sp_body_rk;
    // the decode step as one persistent launch (oh_k_decode): its program in
    // device memory, grid (0: not available for this model), LDS and bytes
    struct DecProg {
        oh_dop *ops = nullptr;
        int n = 0, lds = 0, grid = 0;
        double bytes = 0.0;
        std::vector<int> kinds;          // per operation: OH_D_* kind
        std::vector<double> obytes;      // per operation: algorithmic bytes
        uint64_t *ts = nullptr;          // profiling clocks
    };
    DecProg dec;
    bool dec_tried = false;
    int step_grid = 0;
    bool step_tried = false;
    uint64_t *ts = nullptr;
};

enum { K_MATVEC = 0, K_NORM_Q8K, K_SWIGLU_Q8K, K_EMBED, K_DELTA, K_ATTN_PREP, K_ATTN_SCORES,
       K_ATTN_OUT, K_ROUTE, K_COMBINE, K_ARGMAX, K_ADVANCE, K_MV_DOWN, K_ATTN_FLASH, K_ATTN_COMBINE,
       K_MATVEC_Q6K, K_MATVEC_Q80, K_MATVEC_MIXED, K_STEP_BODY, K_STEP_HEAD, K_ATTN_MAIN };

static int rec_begin(ornith_hip_session *s, hipStream_t st) {
    if (!s->rec) return ORNITH_HIP_OK;
    hipEvent_t e;
    HCHK(hipEventCreate(&e));
    HCHK(hipEventRecord(e, st));
    s->rec_ev.push_back(e);
    return ORNITH_HIP_OK;
}
static int rec_end(ornith_hip_session *s, hipStream_t st, int kind, double bytes) {
    if (!s->rec) return ORNITH_HIP_OK;
    hipEvent_t e;
    HCHK(hipEventCreate(&e));
    HCHK(hipEventRecord(e, st));
    s->rec_ev.push_back(e);
    s->rec_kind.push_back(kind);
    s->rec_bytes.push_back(bytes);
    return ORNITH_HIP_OK;
}
// true when the launch of this kind runs (every launch unless a kind replay
// is selecting one kind); counts the replayed launches and their bytes
static bool keep(ornith_hip_session *s, int kind, double bytes) {
    if (s->only < 0) return true;
    if (kind != s->only) return false;
    s->only_n++;
    s->only_bytes += bytes;
    return true;
}
#define LAUNCH(kind, bytes, call)                  \
    do {                                           \
        if (keep(s, (kind), (bytes))) {            \
            CHK(rec_begin(s, st));                 \
            HCHK(call);                            \
            CHK(rec_end(s, st, kind, bytes));      \
        }                                          \
    } while (0)
// matvec launches are recorded by kernel variant (see oh_launch_matvec)
static int mv_kind(int tk) {
    return tk == OH_Q4_K ? K_MATVEC : tk == OH_Q6_K ? K_MATVEC_Q6K : tk == OH_Q8_0 ? K_MATVEC_Q80 : K_MATVEC_MIXED;
}

// ---- the token step as a program of operations ----------------------------------------------
// The same list of operations runs either launch by launch (captured into HIP
// graphs; profiling) or as the phases of the persistent step kernel.
struct Prog {
    std::vector<oh_op> ops;
    std::vector<int> rk;          // record kind (profiling); -1: part of the previous record
    std::vector<double> bytes;    // algorithmic HBM bytes
    int lds = 0;                  // largest dynamic LDS of an operation
    int waves = 4096;             // matvec planning target
    bool step = false;            // built for the persistent step kernel
};
static oh_op op_new(int kind, int nvb, int lds = 0) {
    oh_op o;
    memset(&o, 0, sizeof o);
    o.kind = kind;
    o.nvb = nvb;
    o.tk = -1;
    o.lds = lds;
    return o;
}
static void prog_add(Prog &P, const oh_op &o, int rk, double bytes) {
    if (o.nvb <= 0) return;
    P.ops.push_back(o);
    P.rk.push_back(rk);
    P.bytes.push_back(bytes);
    if (o.lds > P.lds) P.lds = o.lds;
}
static void prog_mv(Prog &P, MvBuild &b) {
    mv_plan(b, P.waves);
    oh_op o = op_new(OH_OP_MV, b.L.total_blocks, b.lds);
    o.tk = b.tk;
    o.u.mv = b.L;
    prog_add(P, o, mv_kind(b.tk), b.bytes);
}

extern "C" void ornith_hip_session_free(ornith_hip_session *s) {
    if (!s) return;
    (void)hipSetDevice(s->m->ctx->device);
    if (s->gbody) (void)hipGraphExecDestroy(s->gbody);
    if (s->ghead) (void)hipGraphExecDestroy(s->ghead);
    if (s->bw.graph) (void)hipGraphExecDestroy(s->bw.graph);
    for (void *p : s->allocs) (void)hipFree(p);
    delete s;
}

template <typename T>
static int salloc(ornith_hip_session *s, T **p, size_t n) {
    void *v = nullptr;
    HCHK(hipMalloc(&v, n * sizeof(T) + 256));
    HCHK(hipMemset(v, 0, n * sizeof(T) + 256));
    s->allocs.push_back(v);
    s->asz.push_back(n * sizeof(T));
    *p = (T *)v;
    return ORNITH_HIP_OK;
}
static int q8alloc(ornith_hip_session *s, Q8Buf &q, size_t n) {
    CHK(salloc(s, &q.qs, n));
    CHK(salloc(s, &q.d, n / 256 + 1));
    CHK(salloc(s, &q.bs, n / 16 + 16));
    CHK(salloc(s, &q.bp, n / 16 + 16));
    return ORNITH_HIP_OK;
}
static Act act_of(const Q8Buf &q, const float *xf) {
    Act a; a.qs = q.qs; a.d = q.d; a.bs = q.bs; a.xf = xf; return a;
}
static Act act_norm(const float *x, const float *w, float eps) {
    Act a; a.pro = OH_PRO_NORM; a.xf = x; a.nw = w; a.eps = eps; return a;
}
static Act act_gnorm(const float *o, const float *sz, const double *runs, const float *w, float eps, int gdim,
                     int runs16 = 0) {
    Act a; a.pro = OH_PRO_GNORM; a.xf = o; a.xf2 = sz; a.xruns = runs; a.nw = w; a.eps = eps; a.gdim = gdim;
    a.runs16 = runs16;
    return a;
}
static Act act_swiglu(const float *g, const float *u) {
    Act a; a.pro = OH_PRO_SWIGLU; a.xf = g; a.xf2 = u; return a;
}

extern "C" int ornith_hip_session_new(ornith_hip_model *m, int cap, ornith_hip_session **out) {
    *out = nullptr;
    if (cap < 1) cap = 1;
    HCHK(hipSetDevice(m->ctx->device));
    const ornith_hip_arch &a = m->a;
    auto *s = new ornith_hip_session();
    static std::atomic<uint64_t> next_sid{1};
    s->sid = next_sid++;
    s->m = m;
    s->cap = cap;
    s->kvcap = (cap + 15) / 16 * 16;   // KV storage stride (V is tiled by 16 positions)
    const int H = a.hidden, qd = a.nk * a.dk, vd = a.nv * a.dv, cc = 2 * qd + vd;
    const int aq = a.nh * a.hd, kvd = a.nkv * a.hd;
    const int K = a.top_k, I = a.moe_inter > a.shared_inter ? a.moe_inter : a.shared_inter;
    const int ow = vd > aq ? vd : aq;
    int st = ORNITH_HIP_OK;
#define A_(x) do { if ((st = (x)) != ORNITH_HIP_OK) { ornith_hip_session_free(s); return st; } } while (0)
    A_(salloc(s, &s->io, 64));
    A_(salloc(s, &s->toks, (size_t)cap + 1));
    A_(salloc(s, &s->x, H)); A_(salloc(s, &s->xn, H)); A_(q8alloc(s, s->xq, H));
    A_(salloc(s, &s->cat, cc > 0 ? cc : 1)); A_(salloc(s, &s->gate, vd > 0 ? vd : 1));
    A_(salloc(s, &s->ab, 2 * (a.nv > 0 ? a.nv : 1)));
    A_(salloc(s, &s->o, ow)); A_(q8alloc(s, s->oq, ow));
    A_(salloc(s, &s->qproj, 2 * (size_t)aq)); A_(salloc(s, &s->kb, kvd)); A_(salloc(s, &s->vb, kvd));
    A_(salloc(s, &s->qr, aq)); A_(salloc(s, &s->agate, aq));
    A_(salloc(s, &s->scores, (size_t)a.nh * s->kvcap));
    {
        const size_t nch = (size_t)oh_flash_slots(s->kvcap);
        A_(salloc(s, &s->fpo, (size_t)a.nh * nch * a.hd + 64));
        A_(salloc(s, &s->fpml, (size_t)a.nh * nch * 2 + 64));
    }
    A_(salloc(s, &s->ddots, (size_t)(K + 1) * H + 64));
    A_(salloc(s, &s->dcnt, (size_t)H + 64));
    A_(salloc(s, &s->osz, (size_t)a.nv * a.dv + 64));
    A_(salloc(s, &s->oruns, (size_t)a.nv * a.dv / 16 + 64));
    {
        const char *e = getenv("ORNITH_HIP_EXACT_ATTN_MAX");
        if (e && *e) s->exact_max = atoi(e);
        const char *f = getenv("ORNITH_HIP_FLASH_MFMA");
        if (f && *f) s->flash_mfma = atoi(f) != 0;
    }
    A_(salloc(s, &s->rl, a.ne > 0 ? a.ne : 1)); A_(salloc(s, &s->shl, 1)); A_(salloc(s, &s->shg, 1));
    A_(salloc(s, &s->ew, 64)); A_(salloc(s, &s->eidx, 64));
    const size_t nvec = (size_t)(K + 1);
    A_(salloc(s, &s->g, nvec * I)); A_(salloc(s, &s->u, nvec * I)); A_(salloc(s, &s->h, nvec * I));
    A_(q8alloc(s, s->hq, nvec * I));
    A_(salloc(s, &s->od, nvec * H));
    A_(salloc(s, &s->logits, a.vocab));
    A_(salloc(s, &s->amv, OH_ARGMAX_BLOCKS)); A_(salloc(s, &s->ami, OH_ARGMAX_BLOCKS));
    s->ls.resize((size_t)a.n_layers);
    bool any_full = false;
    for (int l = 0; l < a.n_layers; l++) {
        LayerState &y = s->ls[l];
        if (m->L[l].full) {
            any_full = true;
            A_(salloc(s, &y.Kt, (size_t)a.nkv * (a.hd / 4) * s->kvcap));
            A_(salloc(s, &y.Ks, (size_t)s->kvcap * a.nkv));
            A_(salloc(s, &y.Vq, (size_t)s->kvcap * a.nkv * a.hd));
            A_(salloc(s, &y.Vs, (size_t)s->kvcap * a.nkv));
        } else {
            A_(salloc(s, &y.S, (size_t)a.nv * a.dk * a.dv));
            A_(salloc(s, &y.conv, 2 * (size_t)(a.conv_k - 1) * cc));
        }
    }
    if (any_full) {
        // RoPE cos/sin per (pos, pair) with the reference's libm calls
        // (ot_rope_partial, src/ornith_tensor.c:167-178)
        int rot = a.rope_dim;
        if (rot <= 0 || rot > a.hd) rot = a.hd;
        const int half = a.hd / 2;
        std::vector<float2> tab((size_t)cap * half);
        std::vector<float> freq((size_t)rot / 2);
        for (int i = 0; i < rot / 2; i++) freq[i] = powf(a.rope_theta, -2.0f * (float)i / (float)rot);
        for (int p = 0; p < cap; p++)
            for (int i = 0; i < half; i++) {
                float2 cs = {1.0f, 0.0f};
                if (i < rot / 2) {
                    const float ang = (float)p * freq[i];
                    cs.x = cosf(ang);
                    cs.y = sinf(ang);
                }
                tab[(size_t)p * half + i] = cs;
            }
        A_(salloc(s, &s->rope, tab.size()));
        hipError_t e = hipMemcpy(s->rope, tab.data(), tab.size() * sizeof(float2), hipMemcpyHostToDevice);
        if (e != hipSuccess) { ornith_hip_session_free(s); seterr("rope upload: %s", hipGetErrorString(e)); return ORNITH_HIP_ERR_DEVICE; }
    }
#undef A_
    *out = s;
    return ORNITH_HIP_OK;
}

// ---- the token step ------------------------------------------------------------------------
// Algorithmic bytes of the small kernels (recorded by profile_step only).
static double norm_bytes(int n, bool w) { return (double)n * (4.0 + (w ? 4.0 : 0.0) + 4.0 + 1.0 + 4.0 / 256 + 2.0 / 16); }

static int build_body(ornith_hip_session *s, Prog &P) {
    const ornith_hip_model *m = s->m;
    const ornith_hip_arch &a = m->a;
    const int H = a.hidden, qd = a.nk * a.dk, vd = a.nv * a.dv, cc = 2 * qd + vd;
    const double T = (double)(s->pos + 1);
    {
        oh_op o = op_new(OH_OP_EMBED, (H + 255) / 256);
        o.u.embed = {m->embd->A, m->embd->B, m->embd->C, s->toks, s->x, (int)m->embd->type, H};
        prog_add(P, o, K_EMBED, (double)gguf_nbytes(m->embd->type, (uint64_t)H) + 4.0 * H);
    }
    for (int l = 0; l < a.n_layers; l++) {
        const OhLayer &y = m->L[l];
        LayerState &z = s->ls[l];
        const Act an = act_norm(s->x, (const float *)y.attn_norm->A, a.eps);
        if (y.full) {
            const int aqd = a.nh * a.hd, kvd = a.nkv * a.hd;
            MvBuild b;
            CHK(mv_add(b, y.q, an, s->qproj, 0));
            CHK(mv_add(b, y.k, an, s->kb, 0));
            CHK(mv_add(b, y.v, an, s->vb, 0));
            prog_mv(P, b);
            {
                oh_op o = op_new(OH_OP_ATTN_PREP, a.nh + a.nkv);
                o.u.prep = {s->qproj, s->kb, s->vb, (const float *)y.q_norm->A, (const float *)y.k_norm->A,
                            (const float *)s->rope, s->qr, s->agate, z.Kt, z.Ks, z.Vq, z.Vs,
                            a.nh, a.nkv, a.hd, a.rope_dim, s->kvcap, a.eps};
                prog_add(P, o, K_ATTN_PREP, 4.0 * (2.0 * aqd + 2.0 * kvd + 2.0 * a.hd) + 8.0 * aqd +
                                                2.0 * (kvd + 4.0 * a.nkv));
            }
            const float scale = 1.0f / sqrtf((float)a.hd);
            // contexts up to exact_max: scores + the reference-order walk;
            // longer ones: flash chunks + merge (each pair exits for the other)
            const bool ex = s->pos + 1 <= (s->exact_max < 2048 ? s->exact_max : 2048);
            oh_op_attn at;
            memset(&at, 0, sizeof at);
            at.qr = s->qr; at.gate = s->agate; at.Kt = z.Kt; at.Ks = z.Ks; at.Vq = z.Vq; at.Vs = z.Vs;
            at.scores = s->scores; at.part_o = s->fpo; at.part_ml = s->fpml; at.out = s->o;
            at.nh = a.nh; at.nkv = a.nkv; at.hd = a.hd; at.cap = s->kvcap; at.exact_max = s->exact_max;
            at.hb = oh_flash_form(a.nh, a.nkv, a.hd, s->flash_mfma); at.scale = scale;
            const double nchd = oh_flash_parts((int)T, s->kvcap, at.hb);
            // exact walk (its scores in LDS) or flash chunks, then the merge
            // of the chunks (which exits after an exact walk)
            const int nv_ex = a.nh / (256 / a.hd), nv_fl = oh_flash_nvb(a.nh, a.nkv, s->kvcap, at.hb);
            const int lds_ex = oh_exact_lds_bytes(a.hd, s->exact_max), lds_fl = oh_flash_form_lds(a.nh, a.nkv, a.hd, at.hb);
            oh_op o3 = op_new(OH_OP_ATTN_MAIN, nv_ex > nv_fl ? nv_ex : nv_fl, lds_ex > lds_fl ? lds_ex : lds_fl);
            o3.u.attn = at;
            prog_add(P, o3, K_ATTN_MAIN,
                     ex ? 2.0 * T * a.nkv * (a.hd + 4.0) + 4.0 * T * a.nh + 12.0 * aqd
                        : T * a.nkv * (2.0 * a.hd + 8.0) + 4.0 * aqd + 8.0 * nchd * aqd);
            oh_op o4 = op_new(OH_OP_ATTN_COMBINE, a.nh * (a.hd / 64));
            o4.u.attn = at;
            prog_add(P, o4, K_ATTN_COMBINE, ex ? 0.0 : 4.0 * nchd * (aqd + 2.0 * a.nh) + 12.0 * aqd);
            MvBuild b2;
            Act af;
            af.pro = OH_PRO_F32;
            af.xf = s->o;
            CHK(mv_add(b2, y.o, af, s->x, 1));
            prog_mv(P, b2);
        } else {
            MvBuild b;
            CHK(mv_add(b, y.qkv, an, s->cat, 0));
            CHK(mv_add(b, y.gate, an, s->gate, 0));
            CHK(mv_add(b, y.alpha, an, s->ab, 0));
            CHK(mv_add(b, y.beta, an, s->ab + a.nv, 0));
            prog_mv(P, b);
            const float out_scale = 1.0f / sqrtf((float)a.dk);
            const double sb = 8.0 * a.nv * a.dk * a.dv + 8.0 * (a.conv_k - 1) * cc + 4.0 * cc * (a.conv_k + 1) +
                              12.0 * vd + 16.0 * a.nv;
            // 16 state rows per 256-thread block (nv * dk / 16 blocks)
            oh_op o = op_new(OH_OP_DELTA16, a.nv * (a.dk / 16), oh_delta16_lds_bytes(a.dk));
            o.u.delta = {s->cat, s->ab, s->gate, (const float *)y.conv->A, (const float *)y.ssm_a->A,
                         (const float *)y.dt_bias->A, z.conv, z.S, s->o, s->osz, s->oruns,
                         a.dk, a.nk, a.nv, a.conv_k, cc, out_scale};
            prog_add(P, o, K_DELTA, sb);
            // per-head gated RMSNorm of the delta output inside the projection
            MvBuild b2;
            CHK(mv_add(b2, y.ssm_out,
                       act_gnorm(s->o, s->osz, s->oruns, (const float *)y.ssm_norm->A, a.eps, a.dv, 1), s->x, 1));
            prog_mv(P, b2);
        }
        // FFN: post_attention_norm (formed inside the first FFN launch), then
        // MoE (or dense SwiGLU)
        const Act pn = act_norm(s->x, (const float *)y.post_norm->A, a.eps);
        if (a.ne > 0) {
            const int K = a.top_k, I = a.moe_inter, sI = a.shared_inter;
            const int IW = I > sI ? I : sI;   // row stride of the g/u buffers
            // router (+ shared-expert gate); its first block keeps the
            // normalised activation for the expert launch
            Act pst = pn;
            pst.oqs = s->xq.qs; pst.oqd = s->xq.d; pst.oqb = s->xq.bs; pst.oxf = s->xn;
            MvBuild b;
            CHK(mv_add(b, y.router, pst, s->rl, 0));
            if (y.gate_inp_sh) CHK(mv_add(b, y.gate_inp_sh, pn, s->shl, 0));
            prog_mv(P, b);
            const Act ax = act_of(s->xq, s->xn);
            const bool paired = pairable(y.gate_exps, y.up_exps) && (!y.gate_sh || pairable(y.gate_sh, y.up_sh));
            MvBuild b2;
            // experts gate/up: every block routes first (top-k + softmax), the
            // stacked segments then read the routed experts; gate and up rows
            // are reduced together and emit h = silu(gate) * up
            if (paired) {
                CHK(mv_add_pair(b2, y.gate_exps, y.up_exps, ax, s->h, s->eidx, K, IW));
                if (y.gate_sh) CHK(mv_add_pair(b2, y.gate_sh, y.up_sh, ax, s->h + (size_t)K * IW));
            } else {
                CHK(mv_add(b2, y.gate_exps, ax, s->g, 0, s->eidx, K, IW, 0));
                CHK(mv_add(b2, y.up_exps, ax, s->u, 0, s->eidx, K, IW, 0));
                if (y.gate_sh) {
                    CHK(mv_add(b2, y.gate_sh, ax, s->g + (size_t)K * IW, 0));
                    CHK(mv_add(b2, y.up_sh, ax, s->u + (size_t)K * IW, 0));
                }
            }
            b2.L.route = 1;
            b2.L.rlog = s->rl;
            b2.L.shl = y.gate_inp_sh ? s->shl : nullptr;
            b2.L.ne = a.ne;
            b2.L.topk = K;
            b2.L.ridx = s->eidx;
            b2.L.rw = s->ew;
            b2.L.shg = s->shg;
            b2.bytes += 4.0 * a.ne + 8.0 * K;
            prog_mv(P, b2);
            const uint32_t dt = y.down_exps->type;
            const int nbd = I / 256, ns = K + (y.gate_sh ? 1 : 0);
            const int rps = nbd >= 1 ? 64 / nbd : 1;
            const int sq = (nbd * 272 + nbd * 36 + 15) & ~15, dlds = ns * sq + ns * I * 4 + ns * rps * 4;
            const bool fuse = paired && oh_qdot_can(dt, I) && nbd >= 1 && nbd <= 64 && ns <= 10 && dlds <= 65536 &&
                              (!P.step || I <= 1024) &&
                              (!y.gate_sh || (y.down_sh->type == dt && sI == I));
            if (fuse) {
                oh_mvdown D;
                memset(&D, 0, sizeof D);
                D.A = y.down_exps->A; D.B = y.down_exps->B; D.C = y.down_exps->C;
                if (y.gate_sh) { D.sA = y.down_sh->A; D.sB = y.down_sh->B; D.sC = y.down_sh->C; }
                D.eidx = s->eidx; D.w = s->ew; D.shg = y.gate_inp_sh ? s->shg : nullptr;
                D.h = s->h; D.hsh = s->h + (size_t)K * IW; D.x = s->x;
                D.type = (int)dt; D.nb = nbd; D.in = I; D.rows = H; D.k = K; D.stride = IW;
                const double db = (double)ns * ((double)H * gguf_nbytes(dt, (uint64_t)I) + 4.0 * I) + 8.0 * H + 4.0 * K;
                oh_op o = op_new(OH_OP_MV_DOWN, (H + rps - 1) / rps, dlds);
                if (P.step) {
                    // split form: (row group, 4-slot group) blocks, last one combines
                    D.dots = s->ddots;
                    D.cnt = s->dcnt;
                    o.nvb = (H + rps - 1) / rps * ((ns + 3) / 4);
                    o.lds = 4 * ((I * 4 + nbd * 272 + nbd * 36 + 15) & ~15);
                }
                o.u.down = D;
                prog_add(P, o, K_MV_DOWN, db);
            } else {
                MvBuild b3;
                Act ah;
                ah.pro = OH_PRO_F32;
                ah.xf = s->h;
                const Act a0 = paired ? ah : act_swiglu(s->g, s->u);
                CHK(mv_add(b3, y.down_exps, a0, s->od, 0, s->eidx, K, H, IW));
                if (y.gate_sh) {
                    Act a1 = a0;
                    a1.xf = a0.xf + (size_t)K * IW;
                    if (!paired) a1.xf2 = a0.xf2 + (size_t)K * IW;
                    CHK(mv_add(b3, y.down_sh, a1, s->od + (size_t)K * H, 0));
                }
                prog_mv(P, b3);
                oh_op o = op_new(OH_OP_MOE_COMBINE, (H + 255) / 256);
                o.u.comb = {s->x, s->od, s->ew, y.gate_sh ? s->od + (size_t)K * H : nullptr,
                            y.gate_inp_sh ? s->shg : nullptr, K, H};
                prog_add(P, o, K_COMBINE, 4.0 * H * (ns + 2));
            }
        } else {
            MvBuild b;
            const bool paired = pairable(y.ffn_gate, y.ffn_up);
            if (paired) {
                CHK(mv_add_pair(b, y.ffn_gate, y.ffn_up, pn, s->h));
            } else {
                CHK(mv_add(b, y.ffn_gate, pn, s->g, 0));
                CHK(mv_add(b, y.ffn_up, pn, s->u, 0));
            }
            prog_mv(P, b);
            MvBuild b2;
            Act ah;
            ah.pro = OH_PRO_F32;
            ah.xf = s->h;
            CHK(mv_add(b2, y.ffn_down, paired ? ah : act_swiglu(s->g, s->u), s->x, 1));
            prog_mv(P, b2);
        }
    }
    return ORNITH_HIP_OK;
}

static int build_head(ornith_hip_session *s, Prog &P) {
    const ornith_hip_model *m = s->m;
    const ornith_hip_arch &a = m->a;
    MvBuild b;
    CHK(mv_add(b, m->lm_head, act_norm(s->x, (const float *)m->out_norm->A, a.eps), s->logits, 0));
    prog_mv(P, b);
    oh_op o = op_new(OH_OP_ARGMAX1, OH_ARGMAX_BLOCKS);
    o.u.am = {s->logits, s->amv, s->ami, a.vocab, OH_ARGMAX_BLOCKS, s->toks, s->io + OH_IO_BEST};
    prog_add(P, o, K_ARGMAX, 4.0 * a.vocab);
    o.kind = OH_OP_ARGMAX2;
    o.nvb = 1;
    prog_add(P, o, -1, 0.0);
    return ORNITH_HIP_OK;
}

// Launch a program operation by operation (records and kind selection as
// LAUNCH does).
static int run_prog(ornith_hip_session *s, const Prog &P, hipStream_t st) {
    for (size_t i = 0; i < P.ops.size(); i++) {
        if (P.rk[i] < 0) continue;
        size_t j = i + 1;
        while (j < P.ops.size() && P.rk[j] < 0) j++;
        if (!keep(s, P.rk[i], P.bytes[i])) continue;
        CHK(rec_begin(s, st));
        for (size_t k = i; k < j; k++) HCHK(oh_launch_op(&P.ops[k], s->io, st));
        CHK(rec_end(s, st, P.rk[i], P.bytes[i]));
    }
    return ORNITH_HIP_OK;
}

static int enqueue_body(ornith_hip_session *s, hipStream_t st) {
    Prog P;
    CHK(build_body(s, P));
    CHK(run_prog(s, P, st));
    LAUNCH(K_ADVANCE, 8.0, oh_launch_advance(s->io, st));
    return ORNITH_HIP_OK;
}

static int enqueue_head(ornith_hip_session *s, hipStream_t st) {
    Prog P;
    CHK(build_head(s, P));
    return run_prog(s, P, st);
}

// ---- the persistent step kernel -------------------------------------------------------------------
// ORNITH_HIP_STEP=1 selects the persistent step kernel for decode steps;
// otherwise each operation is its own launch (HIP graphs)
static bool step_enabled() {
    const char *e = getenv("ORNITH_HIP_STEP");
    return e && e[0] == '1';
}

static int step_upload(ornith_hip_session *s, const Prog &P, ornith_hip_session::StepProg &sp) {
    sp.n = (int)P.ops.size();
    sp.lds = P.lds;
    sp.bytes = 0.0;
    for (double b : P.bytes) sp.bytes += b;
    CHK(salloc(s, &sp.ops, P.ops.size()));
    HCHK(hipMemcpy(sp.ops, P.ops.data(), P.ops.size() * sizeof(oh_op), hipMemcpyHostToDevice));
    CHK(salloc(s, &sp.ctrs, P.ops.size() * OH_STEP_NCTR * OH_STEP_CSTRIDE));
    return ORNITH_HIP_OK;
}

// Build and upload the body and head programs once per session. The grid is
// two resident 256-thread blocks per CU (one when the LDS does not allow
// two), a multiple of OH_STEP_NCTR; matvecs are planned for its waves.
// Returns ORNITH_HIP_OK with step_grid == 0 when the device cannot run it.
static int step_prepare(ornith_hip_session *s) {
    if (s->step_tried) return ORNITH_HIP_OK;
    s->step_tried = true;
    const int dev = s->m->ctx->device;
    int coop = 0, cus = 0;
    HCHK(hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev));
    HCHK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    if (!coop || cus <= 0) return ORNITH_HIP_OK;
    for (int per = 2; per >= 1; per--) {
        const int grid = per * cus / OH_STEP_NCTR * OH_STEP_NCTR;
        if (grid < OH_STEP_NCTR) return ORNITH_HIP_OK;
        Prog B, Hd;
        B.waves = Hd.waves = grid * 4;
        B.step = Hd.step = true;
        CHK(build_body(s, B));
        CHK(build_head(s, Hd));
        const int lds = B.lds > Hd.lds ? B.lds : Hd.lds;
        int fit = 0;
        HCHK(oh_step_blocks_per_cu(lds, &fit));
        if (fit < per) continue;
        CHK(step_upload(s, B, s->sp_body));
        CHK(step_upload(s, Hd, s->sp_head));
        s->sp_body_rk = B.rk;
        s->sp_body.lds = s->sp_head.lds = lds;
        s->step_grid = grid;
        return ORNITH_HIP_OK;
    }
    return ORNITH_HIP_OK;
}

// advance: the body moves the position on (a replay for timing does not)
static int step_launch(ornith_hip_session *s, bool body, uint64_t *ts, bool advance = true) {
    const ornith_hip_session::StepProg &sp = body ? s->sp_body : s->sp_head;
    HCHK(oh_launch_step(sp.ops, sp.n, s->io, sp.ctrs, body ? OH_IO_EPOCH_BODY : OH_IO_EPOCH_HEAD,
                        body && advance ? 1 : 0, ts, s->step_grid, sp.lds, s->m->ctx->st));
    return ORNITH_HIP_OK;
}

// a grid wait of the step kernel that gave up leaves io[OH_IO_ERR] set
static int step_check(ornith_hip_session *s) {
    int32_t err = 0;
    HCHK(hipMemcpy(&err, s->io + OH_IO_ERR, 4, hipMemcpyDeviceToHost));
    if (err) {
        seterr("decode step: a wait between workgroups timed out; the session state is undefined");
        return ORNITH_HIP_ERR_DEVICE;
    }
    return ORNITH_HIP_OK;
}


// ---- the decode step as one persistent launch (oh_decode.hip) -------------------------------
// Opt-in (ORNITH_HIP_DECODE=1): on C3 it measures 3.2 ms per token against
// the per-launch HIP-graph step's 2.7 ms, so the graph step stays the default.
// The program covers models whose every projection has the integer dot
// (Q4_K / Q6_K / Q8_0, inputs <= 8192), MoE FFNs with paired gate/up and a
// down projection of one type (shared expert included), delta-net head dims
// 64 / 128 with conv kernels <= 8; other models keep the per-launch step.
static bool dec_enabled() {
    const char *e = getenv("ORNITH_HIP_DECODE");
    return e && e[0] == '1';
}

struct DecB {
    std::vector<oh_dop> ops;
    std::vector<double> obytes;   // per operation (filled by dec_note)
    uint64_t *base = nullptr;   // word arena (a dummy base while sizing)
    size_t used = 0;            // words
    int G = 0, lds = 0;
    double bytes = 0.0;
    uint64_t *alloc(size_t n) {
        uint64_t *p = base + used;
        used += (n + 31) & ~(size_t)31;
        return p;
    }
};

static bool dq(const ornith_hip_tensor *W) { return W && oh_qdot_can(W->type, W->in) && W->in <= 8192; }

static oh_dmv dmv_new(const uint64_t *x, const float *nw, int pro, int in, float eps) {
    oh_dmv M;
    memset(&M, 0, sizeof M);
    M.x = x; M.nw = nw; M.pro = pro; M.in = in; M.nb = in / 256; M.eps = eps;
    return M;
}
// one segment: W (and W2, paired) applied in nsub slots (stacked: slot k is
// the routed expert k); output slot k row r at y[k * ystride + r]
static void dmv_seg(oh_dmv &M, const ornith_hip_tensor *W, const ornith_hip_tensor *W2, uint64_t *y, int nsub,
                    int ystride, int stacked, int mode, float *yp = nullptr) {
    oh_dseg &g = M.s[M.nseg++];
    memset(&g, 0, sizeof g);
    g.A = W->A; g.B = W->B; g.C = W->C;
    if (W2) { g.A2 = W2->A; g.B2 = W2->B; g.C2 = W2->C; g.pair = 1; }
    g.y = y; g.yp = yp; g.type = (int)W->type;
    g.rows = stacked ? (int)W->dims[1] : (int)W->rows;
    g.nsub = nsub; g.ystride = ystride; g.stacked = stacked; g.mode = mode;
    const int rps = 64 / M.nb;
    g.units = (g.rows + rps - 1) / rps;
    g.step0 = M.nsteps;
    M.nsteps += g.units * nsub;
}
// The decode launch's matvec (a front wave polling the inputs, three
// stepping waves per workgroup) exists for these (type, super-blocks per
// input) pairs; mode-1 output only in one segment; routing over <= 1024.
static bool dmv_ok(const oh_dmv &M) {
    const int t = M.s[0].type, nb = M.nb;
    const bool shape = t == OH_Q4_K ? (nb == 2 || nb == 4 || nb == 8 || nb == 16)
                     : t == OH_Q6_K ? (nb == 4 || nb == 8 || nb == 16) : (nb == 2 || nb == 4 || nb == 8);
    for (int i = 0; i < M.nseg; i++)
        if (M.s[i].type != t || (M.s[i].mode == 1 && M.nseg != 1)) return false;
    return shape && M.ne <= 1024;
}
// deal the steps to `waves` of the grid's 4 G waves from wave0 on, counted
// as the three stepping waves per workgroup; dynamic LDS of the operation
static bool dmv_add(DecB &b, oh_dmv &M, int wave0, int waves, double bytes) {
    if (!dmv_ok(M)) return false;
    M.wspec = 1;
    wave0 = (int)((long long)wave0 * 3 / 4);
    waves = (int)((long long)waves * 3 / 4);
    M.wave0 = wave0;
    M.spw = (M.nsteps + waves - 1) / waves;
    if (M.spw < 1) M.spw = 1;
    // residual rows of a workgroup's steps: at most 1024 words
    if (M.s[0].mode == 1 && 3 * M.spw * (64 / M.nb) > 1024) return false;
    const int l = ((M.nb * 272 + M.nb * 36 + 15) & ~15) + (M.in + 1024 + ((M.ne + 3) & ~3)) * 4;
    if (l > b.lds) b.lds = l;
    oh_dop o;
    memset(&o, 0, sizeof o);
    o.kind = OH_D_MV;
    o.nvb = b.G;
    o.u.mv = M;
    b.ops.push_back(o);
    b.bytes += bytes;
    return true;
}
static double wbytes(const ornith_hip_tensor *W, int rows) { return (double)rows * gguf_nbytes(W->type, (uint64_t)W->in); }

// Build the program; false (with nothing built) when the model is outside it.
static bool dec_build(ornith_hip_session *s, DecB &b) {
    const ornith_hip_model *m = s->m;
    const ornith_hip_arch &a = m->a;
    const int H = a.hidden, qd = a.nk * a.dk, vd = a.nv * a.dv, cc = 2 * qd + vd, aq = a.nh * a.hd;
    const int kvd = a.nkv * a.hd, G = b.G, W4 = 4 * G;
    const double T = (double)(s->pos + 1);
    if (H % 256 || H > 8192 || !dq(m->lm_head) || a.ne <= 0 || a.top_k > 64 || a.ne > 1024) return false;
    if (m->embd->type != OH_F32 && m->embd->type != OH_F16 && m->embd->type != OH_BF16 && !oh_is_quant(m->embd->type))
        return false;
    uint64_t *x = b.alloc(H);
    {
        oh_dop o;
        memset(&o, 0, sizeof o);
        o.kind = OH_D_EMBED;
        o.nvb = (H + 255) / 256;
        o.u.emb = {m->embd->A, m->embd->B, m->embd->C, s->toks, x, (int)m->embd->type, H};
        b.ops.push_back(o);
        b.bytes += (double)gguf_nbytes(m->embd->type, (uint64_t)H);
    }
    for (int l = 0; l < a.n_layers; l++) {
        const OhLayer &y = m->L[l];
        LayerState &z = s->ls[l];
        uint64_t *xmid = b.alloc(H);
        if (y.full) {
            if (!dq(y.q) || !dq(y.k) || !dq(y.v) || !dq(y.o) || y.k->type != y.q->type) return false;
            if (a.hd > 256 || 256 % a.hd || a.nh + a.nkv > 4096) return false;
            uint64_t *qkv = b.alloc(2 * (size_t)aq + 2 * (size_t)kvd);
            oh_dmv M = dmv_new(x, (const float *)y.attn_norm->A, OH_PRO_NORM, H, a.eps);
            dmv_seg(M, y.q, nullptr, qkv, 1, 0, 0, 0);
            dmv_seg(M, y.k, nullptr, qkv + 2 * aq, 1, 0, 0, 0);
            const double qb = wbytes(y.q, 2 * aq) + wbytes(y.k, kvd);
            if (y.v->type == y.q->type) {
                dmv_seg(M, y.v, nullptr, qkv + 2 * aq + kvd, 1, 0, 0, 0);
                if (!dmv_add(b, M, 0, W4, qb + wbytes(y.v, kvd))) return false;
            } else {
                // v in its own operation on the last waves, q/k on the others
                oh_dmv V = dmv_new(x, (const float *)y.attn_norm->A, OH_PRO_NORM, H, a.eps);
                dmv_seg(V, y.v, nullptr, qkv + 2 * aq + kvd, 1, 0, 0, 0);
                int vw = (int)((double)W4 * V.nsteps / (V.nsteps + M.nsteps));
                vw = vw < 4 ? 4 : (vw > W4 - 4 ? W4 - 4 : vw);
                vw = (vw + 3) & ~3;
                if (!dmv_add(b, V, W4 - vw, vw, wbytes(y.v, kvd))) return false;
                if (!dmv_add(b, M, 0, W4 - vw, qb)) return false;
            }
            // prep (q/k norm, RoPE, KV append) -> attention -> merge
            uint64_t *pflags = b.alloc(a.nh + a.nkv);
            const int lim = s->exact_max < 2048 ? s->exact_max : 2048;
            oh_op_attn at;
            memset(&at, 0, sizeof at);
            at.qr = s->qr; at.gate = s->agate; at.Kt = z.Kt; at.Ks = z.Ks; at.Vq = z.Vq; at.Vs = z.Vs;
            at.scores = s->scores; at.part_o = s->fpo; at.part_ml = s->fpml; at.out = s->o;
            at.nh = a.nh; at.nkv = a.nkv; at.hd = a.hd; at.cap = s->kvcap; at.exact_max = s->exact_max;
            at.hb = oh_flash_form(a.nh, a.nkv, a.hd, s->flash_mfma); at.scale = 1.0f / sqrtf((float)a.hd);
            const int nv_ex = a.nh / (256 / a.hd), nv_fl = oh_flash_nvb(a.nh, a.nkv, s->kvcap, at.hb);
            const int nva = nv_ex > nv_fl ? nv_ex : nv_fl, ncb = a.nh * (a.hd / 64);
            uint64_t *aflags = b.alloc(nva + ncb), *cflags = aflags + nva;
            oh_dop o;
            memset(&o, 0, sizeof o);
            o.kind = OH_D_PREP;
            o.nvb = a.nh + a.nkv;
            o.u.at.p = {nullptr, nullptr, nullptr, (const float *)y.q_norm->A, (const float *)y.k_norm->A,
                        (const float *)s->rope, s->qr, s->agate, z.Kt, z.Ks, z.Vq, z.Vs,
                        a.nh, a.nkv, a.hd, a.rope_dim, s->kvcap, a.eps};
            o.u.at.qkv = qkv;
            o.u.at.flags = pflags;
            b.ops.push_back(o);
            o.kind = OH_D_ATTN;
            o.nvb = nva;
            o.u.at.a = at;
            o.u.at.wflags = pflags;
            o.u.at.nwait_ex = o.u.at.nwait_fl = a.nh + a.nkv;
            o.u.at.flags = aflags;
            o.u.at.lim = lim;
            b.ops.push_back(o);
            const int lds_ex = oh_exact_lds_bytes(a.hd, s->exact_max), lds_fl = oh_flash_form_lds(a.nh, a.nkv, a.hd, at.hb);
            if (lds_ex > b.lds) b.lds = lds_ex;
            if (lds_fl > b.lds) b.lds = lds_fl;
            const double nch = oh_flash_parts((int)T, s->kvcap, at.hb);
            b.bytes += T * a.nkv * (2.0 * a.hd + 8.0);
            o.kind = OH_D_COMBINE;
            o.nvb = ncb;
            o.u.at.wflags = aflags;
            o.u.at.nwait_fl = nva;
            o.u.at.flags = cflags;
            b.ops.push_back(o);
            (void)nch;
            // attn_output, x += (plain input behind the attention's flags)
            oh_dmv O = dmv_new(nullptr, nullptr, OH_PRO_F32, aq, a.eps);
            O.xp = s->o;
            O.xflags = aflags;
            O.nflags_ex = nva;
            O.nflags_fl = nva + ncb;
            O.exact_lim = lim;
            O.xres = x;
            dmv_seg(O, y.o, nullptr, xmid, 1, 0, 0, 1);
            if (O.s[0].units > 2 * 3 * G) return false;
            if (!dmv_add(b, O, 0, W4, wbytes(y.o, H))) return false;
        } else {
            if (!dq(y.qkv) || !dq(y.gate) || !dq(y.alpha) || !dq(y.beta) || !dq(y.ssm_out)) return false;
            if (y.gate->type != y.qkv->type || y.alpha->type != y.qkv->type || y.beta->type != y.qkv->type) return false;
            if ((a.dk != 64 && a.dk != 128) || a.dv != a.dk || a.conv_k < 2 || a.conv_k > 8) return false;
            if (y.conv->type != OH_F32 || y.ssm_norm->type != OH_F32) return false;
            uint64_t *cat = b.alloc(cc), *zz = b.alloc(vd), *ab = b.alloc(2 * (size_t)a.nv), *o = b.alloc(vd);
            oh_dmv M = dmv_new(x, (const float *)y.attn_norm->A, OH_PRO_NORM, H, a.eps);
            dmv_seg(M, y.qkv, nullptr, cat, 1, 0, 0, 0);
            dmv_seg(M, y.gate, nullptr, zz, 1, 0, 0, 0);
            dmv_seg(M, y.alpha, nullptr, ab, 1, 0, 0, 0);
            dmv_seg(M, y.beta, nullptr, ab + a.nv, 1, 0, 0, 0);
            if (!dmv_add(b, M, 0, W4, wbytes(y.qkv, cc) + wbytes(y.gate, vd) + wbytes(y.alpha, a.nv) + wbytes(y.beta, a.nv))) return false;
            oh_dop d;
            memset(&d, 0, sizeof d);
            d.kind = OH_D_DELTA;
            d.nvb = a.nv;
            d.u.dl = {cat, ab, zz, (const float *)y.conv->A, (const float *)y.ssm_a->A, (const float *)y.dt_bias->A,
                      (const float *)y.ssm_norm->A, z.conv, z.S, o, a.dk, a.nk, a.nv, a.conv_k, cc,
                      1.0f / sqrtf((float)a.dk), a.eps};
            b.ops.push_back(d);
            const int dl = (4 * a.dk + 4 + (a.dk / 64) * 64 * (a.dk + 4)) * 4 + 8 * 8;
            if (dl > b.lds) b.lds = dl;
            b.bytes += 8.0 * a.nv * a.dk * a.dv + 8.0 * (a.conv_k - 1) * cc;
            oh_dmv O = dmv_new(o, nullptr, OH_PRO_F32, vd, a.eps);
            O.xres = x;
            dmv_seg(O, y.ssm_out, nullptr, xmid, 1, 0, 0, 1);
            if (O.s[0].units > 2 * 3 * G) return false;
            if (!dmv_add(b, O, 0, W4, wbytes(y.ssm_out, H))) return false;
        }
        // MoE FFN: router (+ shared gate), experts gate/up, down + combine
        const int K = a.top_k, I = a.moe_inter;
        if (!dq(y.router) || !dq(y.gate_exps) || !pairable(y.gate_exps, y.up_exps) || !y.down_exps ||
            !oh_qdot_can(y.down_exps->type, I) || I % 256 || I / 256 > 64 || y.gate_exps->type != y.router->type)
            return false;
        const bool sh = y.gate_sh != nullptr;
        if (sh && (!pairable(y.gate_sh, y.up_sh) || y.gate_sh->type != y.gate_exps->type || a.shared_inter != I ||
                   !y.down_sh || y.down_sh->type != y.down_exps->type))
            return false;
        if (y.gate_inp_sh && (!dq(y.gate_inp_sh) || y.gate_inp_sh->type != y.router->type)) return false;
        uint64_t *rl = b.alloc(a.ne + 1), *shl = y.gate_inp_sh ? rl + a.ne : nullptr;
        oh_dmv R = dmv_new(xmid, (const float *)y.post_norm->A, OH_PRO_NORM, H, a.eps);
        dmv_seg(R, y.router, nullptr, rl, 1, 0, 0, 0);
        if (y.gate_inp_sh) dmv_seg(R, y.gate_inp_sh, nullptr, shl, 1, 0, 0, 0);
        if (!dmv_add(b, R, 0, W4, wbytes(y.router, a.ne) + (y.gate_inp_sh ? wbytes(y.gate_inp_sh, 1) : 0.0))) return false;
        const int ns = K + (sh ? 1 : 0);
        uint64_t *h = b.alloc((size_t)ns * I), *xout = b.alloc(H);
        oh_dmv E = dmv_new(xmid, (const float *)y.post_norm->A, OH_PRO_NORM, H, a.eps);
        E.route = 1; E.rlog = rl; E.shl = shl; E.ne = a.ne; E.topk = K;
        dmv_seg(E, y.gate_exps, y.up_exps, h, K, I, 1, 0);
        if (sh) dmv_seg(E, y.gate_sh, y.up_sh, h + (size_t)K * I, 1, 0, 0, 0);
        if (!dmv_add(b, E, 0, W4, (double)ns * 2.0 * (double)I * gguf_nbytes(y.gate_exps->type, (uint64_t)H))) return false;
        oh_dop dn;
        memset(&dn, 0, sizeof dn);
        dn.kind = OH_D_DOWN;
        const int rpb = (H + G - 1) / G, nbd = I / 256;
        // a (row, slot)'s super-blocks sit in consecutive lanes of one wave;
        // at most 4 units per stepping thread, 64 rows per workgroup
        if (rpb * ns * nbd > 768 || 64 % nbd || rpb > 64) return false;
        dn.nvb = (H + rpb - 1) / rpb;
        dn.u.dn.A = y.down_exps->A; dn.u.dn.B = y.down_exps->B; dn.u.dn.C = y.down_exps->C;
        if (sh) { dn.u.dn.sA = y.down_sh->A; dn.u.dn.sB = y.down_sh->B; dn.u.dn.sC = y.down_sh->C; }
        dn.u.dn.h = h; dn.u.dn.rlog = rl; dn.u.dn.shl = shl; dn.u.dn.xres = xmid; dn.u.dn.y = xout;
        dn.u.dn.type = (int)y.down_exps->type; dn.u.dn.nb = nbd; dn.u.dn.in = I; dn.u.dn.rows = H;
        dn.u.dn.k = K; dn.u.dn.ne = a.ne; dn.u.dn.rpb = rpb;
        b.ops.push_back(dn);
        const int sq = (nbd * 272 + nbd * 36 + 15) & ~15;
        const int ld = ns * sq + ns * I * 4 + 64 * ns * 4 + ((a.ne + 3) & ~3) * 4;
        if (ld > b.lds) b.lds = ld;
        b.bytes += (double)ns * (double)H * gguf_nbytes(y.down_exps->type, (uint64_t)I);
        x = xout;
    }
    // head: output norm, lm_head (plain logits + per-workgroup argmax), greedy token
    uint64_t *amax = b.alloc(2 * (size_t)G);
    oh_dmv Hm = dmv_new(x, (const float *)m->out_norm->A, OH_PRO_NORM, H, a.eps);
    dmv_seg(Hm, m->lm_head, nullptr, nullptr, 1, 0, 0, 0, s->logits);
    Hm.amax = amax;
    if (!dmv_add(b, Hm, 0, W4, wbytes(m->lm_head, a.vocab))) return false;
    oh_dop am;
    memset(&am, 0, sizeof am);
    am.kind = OH_D_ARGMAX;
    am.nvb = 1;
    am.u.am = {amax, G, a.vocab, s->toks};
    b.ops.push_back(am);
    return true;
}

// Size, allocate and upload the program once per session (its contents do
// not depend on the position). Leaves dec.grid = 0 when the model or the
// device cannot run it.
static int dec_prepare(ornith_hip_session *s) {
    if (s->dec_tried) return ORNITH_HIP_OK;
    s->dec_tried = true;
    const int dev = s->m->ctx->device;
    int coop = 0, cus = 0;
    HCHK(hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev));
    HCHK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    if (!coop || cus <= 0) return ORNITH_HIP_OK;
    DecB sz;
    sz.G = cus;
    uint64_t dummy[1];
    sz.base = dummy;
    if (!dec_build(s, sz)) return ORNITH_HIP_OK;
    int fit = 0;
    HCHK(oh_decode_blocks_per_cu(sz.lds, &fit));
    if (fit < 1) return ORNITH_HIP_OK;
    DecB b;
    b.G = cus;
    CHK(salloc(s, &b.base, sz.used + 64));          // zeroed: tag 0 is never a live tag
    if (!dec_build(s, b)) return ORNITH_HIP_OK;
    CHK(salloc(s, &s->dec.ops, b.ops.size()));
    HCHK(hipMemcpy(s->dec.ops, b.ops.data(), b.ops.size() * sizeof(oh_dop), hipMemcpyHostToDevice));
    const int32_t one = 1;
    HCHK(hipMemcpy(s->io + OH_IO_TAG, &one, 4, hipMemcpyHostToDevice));
    s->dec.n = (int)b.ops.size();
    s->dec.kinds.clear();
    for (const oh_dop &o : b.ops) s->dec.kinds.push_back(o.kind);
    s->dec.lds = b.lds;
    s->dec.bytes = b.bytes;
    s->dec.grid = cus;
    return ORNITH_HIP_OK;
}

static int dec_launch(ornith_hip_session *s, bool advance = true) {
    HCHK(oh_launch_decode(s->dec.ops, s->dec.n, s->io, advance ? 1 : 0, s->dec.grid, s->dec.lds, s->m->ctx->st));
    return ORNITH_HIP_OK;
}


static int capture(ornith_hip_session *s, int (*fn)(ornith_hip_session *, hipStream_t), hipGraphExec_t *out) {
    hipStream_t st = s->m->ctx->st;
    hipGraph_t g = nullptr;
    HCHK(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
    int r = fn(s, st);
    hipError_t e = hipStreamEndCapture(st, &g);
    if (r != ORNITH_HIP_OK) { if (g) (void)hipGraphDestroy(g); return r; }
    if (e != hipSuccess) { seterr("graph capture: %s", hipGetErrorString(e)); return ORNITH_HIP_ERR_DEVICE; }
    e = hipGraphInstantiate(out, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) { seterr("graph instantiate: %s", hipGetErrorString(e)); return ORNITH_HIP_ERR_DEVICE; }
    return ORNITH_HIP_OK;
}

static bool graphs_enabled() {
    const char *e = getenv("ORNITH_HIP_NO_GRAPH");
    return !(e && e[0] == '1');
}

static int run_body(ornith_hip_session *s) {
    hipStream_t st = s->m->ctx->st;
    if (step_enabled()) {
        CHK(step_prepare(s));
        if (s->step_grid) return step_launch(s, true, nullptr);
    }
    if (graphs_enabled()) {
        if (!s->gbody) CHK(capture(s, enqueue_body, &s->gbody));
        HCHK(hipGraphLaunch(s->gbody, st));
        return ORNITH_HIP_OK;
    }
    return enqueue_body(s, st);
}
static int run_head(ornith_hip_session *s) {
    hipStream_t st = s->m->ctx->st;
    if (step_enabled()) {
        CHK(step_prepare(s));
        if (s->step_grid) return step_launch(s, false, nullptr);
    }
    if (graphs_enabled()) {
        if (!s->ghead) CHK(capture(s, enqueue_head, &s->ghead));
        HCHK(hipGraphLaunch(s->ghead, st));
        return ORNITH_HIP_OK;
    }
    return enqueue_head(s, st);
}

// One decode step (body and head): the persistent launch where the model
// has one, else the per-launch body and head.
static int run_step(ornith_hip_session *s) {
    if (dec_enabled() && !step_enabled()) {
        CHK(dec_prepare(s));
        if (s->dec.grid) return dec_launch(s);
    }
    CHK(run_body(s));
    return run_head(s);
}

static int sync_pos(ornith_hip_session *s) {
    HCHK(hipMemcpyAsync(s->io, &s->pos, sizeof(int32_t), hipMemcpyHostToDevice, s->m->ctx->st));
    return ORNITH_HIP_OK;
}

// ---- layer-major prefill (src/ornith_rforward.c:647-682 structure) ----------------------
// Every layer over a chunk of tokens before the next: batched matvecs for the
// projections (weights read once per chunk), the conv / delta state / KV cache
// advanced in token order with the decode step's arithmetic. Bit-identical to
// the same tokens fed through the token step.
static const int kPfChunk = 4096, kPfAttnSub = 32;

// tokens per engine chunk (ORNITH_HIP_PREFILL_CHUNK, default 2048): a multiple
// of 32, because the chunked delta scan counts its 32-token chunks from the
// start of the evaluation and an engine chunk must not split one
// prompt attention past the exact walk on the matrix cores; on unless
// ORNITH_HIP_ATTN_MFMA=0
static bool attn_mfma_enabled() {
    const char *e = getenv("ORNITH_HIP_ATTN_MFMA");
    return !(e && e[0] == '0');
}

// batch decode below the matrix-core column count through the fused slotted
// launches; on unless ORNITH_HIP_BATCH_FUSED=0
static bool batch_fused() {
    const char *e = getenv("ORNITH_HIP_BATCH_FUSED");
    return !(e && e[0] == '0');
}

// the prompt's chunked delta scan on the matrix cores in its WY form (a
// tolerance path: the chunk sums re-associated; ORNITH_HIP_DELTA_MFMA=1)
// instead of the reference-order vector-ALU scan
static bool delta_mfma_enabled() {
    const char *e = getenv("ORNITH_HIP_DELTA_MFMA");
    return e && e[0] == '1';
}

static int pf_chunk_tokens() {
    const char *e = getenv("ORNITH_HIP_PREFILL_CHUNK");
    int c = e && *e ? atoi(e) : kPfChunk;
    c = c / 32 * 32;
    return c < 32 ? 32 : (c > kPfChunk ? kPfChunk : c);
}

static bool pf_mvb_ok(const ornith_hip_tensor *W) {
    return W && oh_qdot_can(W->type, W->in) && W->in <= 8192 && W->in / 256 <= 64;
}

// routed experts the grouped batched products handle: integer-path types,
// gate and up a pair
static bool pf_moe_grouped(const OhLayer &y) {
    return pf_mvb_ok(y.gate_exps) && pf_mvb_ok(y.up_exps) && pf_mvb_ok(y.down_exps) && pairable(y.gate_exps, y.up_exps);
}

// other expert types (IQ2_XXS) run the token step's expert kernels over the
// chunk's (token, expert) slots
static bool pf_moe_slots_ok(const OhLayer &y) {
    for (const ornith_hip_tensor *W : {y.gate_exps, y.up_exps, y.down_exps})
        if (!W || W->in % 256 || W->in > 8192 || W->nd != 3) return false;
    return true;
}

static bool pf_supported(const ornith_hip_model *m) {
    const ornith_hip_arch &a = m->a;
    if (a.hidden > 8192 || a.nv * a.dv > 8192 || a.nh * a.hd > 8192) return false;
    for (int l = 0; l < a.n_layers; l++) {
        const OhLayer &y = m->L[l];
        if (y.full) {
            if (!pf_mvb_ok(y.q) || !pf_mvb_ok(y.k) || !pf_mvb_ok(y.v) || !pf_mvb_ok(y.o)) return false;
        } else {
            if (!pf_mvb_ok(y.qkv) || !pf_mvb_ok(y.gate) || !pf_mvb_ok(y.alpha) || !pf_mvb_ok(y.beta) ||
                !pf_mvb_ok(y.ssm_out))
                return false;
            if (a.dk != 64 && a.dk != 128) return false;
        }
        if (a.ne > 0) {
            if (!pf_mvb_ok(y.router) || (!pf_moe_grouped(y) && !pf_moe_slots_ok(y))) return false;
            if (a.moe_inter > 8192 || a.ne > 1024 || a.top_k > 64) return false;
            if (y.gate_sh && (!pf_mvb_ok(y.gate_sh) || !pf_mvb_ok(y.up_sh) || !pf_mvb_ok(y.down_sh) ||
                              !pairable(y.gate_sh, y.up_sh) || a.shared_inter > 8192))
                return false;
            if (y.gate_inp_sh && !pf_mvb_ok(y.gate_inp_sh)) return false;
        } else if (!pf_mvb_ok(y.ffn_gate) || !pf_mvb_ok(y.ffn_up) || !pf_mvb_ok(y.ffn_down) ||
                   !pairable(y.ffn_gate, y.ffn_up) || a.shared_inter > 8192) {
            return false;
        }
    }
    return true;
}

static int pf_alloc(ornith_hip_session *s, int tc) {
    auto &p = s->pf;
    if (p.tc >= tc) return ORNITH_HIP_OK;
    const ornith_hip_arch &a = s->m->a;
    const size_t T = (size_t)tc, H = a.hidden, qd = (size_t)a.nk * a.dk, vd = (size_t)a.nv * a.dv;
    const size_t cc = 2 * qd + vd, aq = (size_t)a.nh * a.hd, kvd = (size_t)a.nkv * a.hd;
    const size_t K = a.top_k > 0 ? a.top_k : 1, I = a.moe_inter > 0 ? a.moe_inter : 1;
    const size_t sI = a.shared_inter > 0 ? a.shared_inter : 1, ne = a.ne > 0 ? a.ne : 1;
    const size_t nch = (s->kvcap + oh_flash_chunk() - 1) / oh_flash_chunk();
    CHK(salloc(s, &p.X, T * H));
    CHK(q8alloc(s, p.XQ, T * H));
    CHK(salloc(s, &p.CAT, T * cc + 1)); CHK(salloc(s, &p.CONV, T * cc + 1));
    CHK(salloc(s, &p.Z, T * vd + 1)); CHK(salloc(s, &p.O, T * vd + 1));
    CHK(q8alloc(s, p.OQ, T * vd + 256));
    CHK(salloc(s, &p.A, T * a.nv + 1)); CHK(salloc(s, &p.Bg, T * a.nv + 1));
    CHK(salloc(s, &p.AL, T * a.nv + 1)); CHK(salloc(s, &p.BE, T * a.nv + 1));
    CHK(salloc(s, &p.QN, T * qd + 1)); CHK(salloc(s, &p.KN, T * qd + 1));
    CHK(salloc(s, &p.GR, (size_t)oh_delta_grams_floats(tc, a.nk > 0 ? a.nk : 1) + 1));
    CHK(salloc(s, &p.STAGE, (size_t)(a.conv_k > 1 ? a.conv_k - 1 : 1) * cc + 1));
    CHK(salloc(s, &p.QP, T * 2 * aq + 1)); CHK(salloc(s, &p.KB, T * kvd + 1)); CHK(salloc(s, &p.VB, T * kvd + 1));
    CHK(salloc(s, &p.QR, T * aq + 1)); CHK(salloc(s, &p.AG, T * aq + 1)); CHK(salloc(s, &p.OA, T * aq + 1));
    CHK(q8alloc(s, p.OAQ, T * aq + 256));
    CHK(salloc(s, &p.FPO, (size_t)kPfAttnSub * a.nh * nch * a.hd + 64));
    CHK(salloc(s, &p.FPML, (size_t)kPfAttnSub * a.nh * nch * 2 + 64));
    CHK(salloc(s, &p.RL, T * ne)); CHK(salloc(s, &p.SHL, T)); CHK(salloc(s, &p.SHG, T));
    CHK(salloc(s, &p.RW, T * K)); CHK(salloc(s, &p.RIDX, T * K));
    CHK(salloc(s, &p.CNT, ne)); CHK(salloc(s, &p.LIST, ne * T));
    CHK(salloc(s, &p.Hh, T * K * I)); CHK(q8alloc(s, p.HQ, T * K * I + 256));
    CHK(salloc(s, &p.HSH, T * sI)); CHK(q8alloc(s, p.HSQ, T * sI + 256));
    CHK(salloc(s, &p.OD, T * K * H)); CHK(salloc(s, &p.ODSH, T * H));
    CHK(salloc(s, &p.GU, T * K * 2 * I)); CHK(salloc(s, &p.GSH, T * 2 * sI));
    CHK(salloc(s, &p.ITEMS, (T * K + 63) / 64 + ne + 2));
    CHK(salloc(s, &p.XN, T * H));
    p.tc = tc;
    p.WY = nullptr;                       // sized for tc tokens on its first use
    return ORNITH_HIP_OK;
}

// Y[col] (+)= W . X[col]: dense columns [0, T), or grouped by expert (list/cnt)
static int pf_mvb(const ornith_hip_tensor *W, const ornith_hip_tensor *W2, const Q8Buf &x, float *y, int ystride,
                  int T, int mode, hipStream_t st, const int32_t *cnt = nullptr, const int32_t *list = nullptr,
                  int lstride = 0, int adiv = 1, int groups = 1) {
    oh_mvbatch B;
    memset(&B, 0, sizeof B);
    B.A = W->A; B.B = W->B; B.C = W->C;
    if (W2) { B.A2 = W2->A; B.B2 = W2->B; B.C2 = W2->C; B.pair = 1; }
    B.xqs = x.qs; B.xd = x.d; B.xbs = x.bs; B.y = y;
    B.type = (int)W->type; B.nb = (int)(W->in / 256); B.in = (int)W->in;
    B.rows = list ? (int)W->dims[1] : (int)W->rows;
    B.mode = mode; B.ncol = T; B.adiv = adiv; B.ystride = ystride; B.tcol = oh_mvb_tcol(B.nb);
    B.cnt = cnt; B.list = list; B.lstride = lstride;
    HCHK(oh_launch_mvb(&B, groups, st));
    return ORNITH_HIP_OK;
}

// Q4_K projections with whole 128-row tiles over at least 64 tokens run on
// the matrix cores; fewer columns (batch decode) stay on the vector-ALU kernel,
// whose whole reduction is in flight at once
static const int kMmqMinTokens = 64;
static bool pf_use_mmq(const ornith_hip_tensor *W, bool grouped, int T) {
    const int rows = grouped ? (int)W->dims[1] : (int)W->rows;
    return mmq_enabled() && T >= kMmqMinTokens && oh_mmq_can(W->type, rows, (int)W->in);
}

static int pf_mmq(const ornith_hip_tensor *W, const ornith_hip_tensor *W2, const Q8Buf &x, float *y, int ystride,
                  int T, int mode, hipStream_t st, const int32_t *cnt = nullptr, const int32_t *list = nullptr,
                  int lstride = 0, int adiv = 1, const int32_t *items = nullptr, int max_items = 0) {
    oh_mmq M;
    memset(&M, 0, sizeof M);
    M.A = W->A; M.B = W->B; M.C = W->C; M.type = (int)W->type;
    if (W2) { M.A2 = W2->A; M.B2 = W2->B; M.C2 = W2->C; }
    M.xqs = x.qs; M.xd = x.d; M.xbp = x.bp; M.y = y;
    M.cnt = cnt; M.list = list; M.items = items;
    M.nb = (int)(W->in / 256); M.in = (int)W->in; M.rows = list ? (int)W->dims[1] : (int)W->rows;
    M.mode = mode; M.ncol = T; M.lstride = lstride; M.adiv = adiv; M.ystride = ystride;
    HCHK(oh_launch_mmq(&M, max_items, W2 != nullptr, st));
    return ORNITH_HIP_OK;
}

// y (+)= W . x over T dense columns
static int pf_mm(const ornith_hip_tensor *W, const Q8Buf &x, float *y, int ystride, int T, int mode,
                 hipStream_t st) {
    if (pf_use_mmq(W, false, T)) return pf_mmq(W, nullptr, x, y, ystride, T, mode, st);
    return pf_mvb(W, nullptr, x, y, ystride, T, mode, st);
}

// h = silu(Wg . x) * (Wu . x) for `npairs` output rows (T dense columns, or the
// grouped expert pairs), quantised to Q8_K in hq
static int pf_swiglu(const ornith_hip_tensor *Wg, const ornith_hip_tensor *Wu, const Q8Buf &x, int I, int npairs,
                     int T, Q8Buf &hq, float *gu, float *hbuf, hipStream_t st, const int32_t *cnt = nullptr,
                     const int32_t *list = nullptr, int lstride = 0, int adiv = 1, int groups = 1,
                     const int32_t *items = nullptr, int max_items = 0) {
    const bool grouped = list != nullptr;
    if (pf_use_mmq(Wg, grouped, T) && pf_use_mmq(Wu, grouped, T)) {
        CHK(pf_mmq(Wg, Wu, x, gu, 2 * I, T, 0, st, cnt, list, lstride, adiv, items, max_items));
        HCHK(oh_launch_norm_q8k_rows(gu, nullptr, 0.0f, I, npairs, nullptr, hq.qs, hq.d, hq.bs, st, hq.bp, 1));
    } else {
        CHK(pf_mvb(Wg, Wu, x, hbuf, I, T, 0, st, cnt, list, lstride, adiv, groups));
        HCHK(oh_launch_norm_q8k_rows(hbuf, nullptr, 0.0f, I, npairs, nullptr, hq.qs, hq.d, hq.bs, st, hq.bp));
    }
    return ORNITH_HIP_OK;
}

static int pf_chunk(ornith_hip_session *s, int base, int T, bool chunked, hipStream_t st) {
    const ornith_hip_model *m = s->m;
    const ornith_hip_arch &a = m->a;
    auto &p = s->pf;
    const int H = a.hidden, qd = a.nk * a.dk, vd = a.nv * a.dv, cc = 2 * qd + vd, aq = a.nh * a.hd;
    const int kvd = a.nkv * a.hd;
    oh_op_embed emb = {m->embd->A, m->embd->B, m->embd->C, s->toks, p.X, (int)m->embd->type, H};
    HCHK(oh_launch_embed_rows(&emb, base, T, st));
    for (int l = 0; l < a.n_layers; l++) {
        const OhLayer &y = m->L[l];
        LayerState &z = s->ls[l];
        HCHK(oh_launch_norm_q8k_rows(p.X, (const float *)y.attn_norm->A, a.eps, H, T, nullptr, p.XQ.qs, p.XQ.d,
                                     p.XQ.bs, st, p.XQ.bp));
        if (y.full) {
            CHK(pf_mm(y.q, p.XQ, p.QP, 2 * aq, T, 0, st));
            CHK(pf_mm(y.k, p.XQ, p.KB, kvd, T, 0, st));
            CHK(pf_mm(y.v, p.XQ, p.VB, kvd, T, 0, st));
            oh_op_prep pr = {p.QP, p.KB, p.VB, (const float *)y.q_norm->A, (const float *)y.k_norm->A,
                             (const float *)s->rope, p.QR, p.AG, z.Kt, z.Ks, z.Vq, z.Vs,
                             a.nh, a.nkv, a.hd, a.rope_dim, s->kvcap, a.eps};
            HCHK(oh_launch_prep_rows(&pr, base, T, st));
            oh_op_attn at;
            memset(&at, 0, sizeof at);
            at.qr = p.QR; at.gate = p.AG; at.Kt = z.Kt; at.Ks = z.Ks; at.Vq = z.Vq; at.Vs = z.Vs;
            at.part_o = p.FPO; at.part_ml = p.FPML; at.out = p.OA;
            at.nh = a.nh; at.nkv = a.nkv; at.hd = a.hd; at.cap = s->kvcap; at.exact_max = s->exact_max;
            at.hb = oh_flash_hb(a.nh, a.nkv); at.scale = 1.0f / sqrtf((float)a.hd);
            const int nch = (s->kvcap + oh_flash_chunk() - 1) / oh_flash_chunk();
            const size_t po = (size_t)a.nh * nch * a.hd, pml = (size_t)a.nh * nch * 2;
            // tokens whose context fits the exact walk take it (sub-batches of
            // kPfAttnSub); the rest go to the matrix-core kernel in one launch
            // (ORNITH_HIP_ATTN_MFMA=0: the flash chunks of the decode step)
            const int lim = s->exact_max < 2048 ? s->exact_max : 2048;
            const int tsplit = attn_mfma_enabled() && oh_attn_mfma_supported(a.hd, a.nh, a.nkv)
                             ? (lim - base < 0 ? 0 : (lim - base > T ? T : lim - base)) : T;
            for (int t0 = 0; t0 < tsplit; t0 += kPfAttnSub)
                HCHK(oh_launch_attn_rows(&at, base, t0, tsplit - t0 < kPfAttnSub ? tsplit - t0 : kPfAttnSub, po, pml,
                                         st));
            if (tsplit < T) HCHK(oh_launch_attn_mfma_rows(&at, base, tsplit, T - tsplit, st));
            HCHK(oh_launch_norm_q8k_rows(p.OA, nullptr, 0.0f, aq, T, nullptr, p.OAQ.qs, p.OAQ.d, p.OAQ.bs, st,
                                         p.OAQ.bp));
            CHK(pf_mm(y.o, p.OAQ, p.X, H, T, 1, st));
        } else {
            CHK(pf_mm(y.qkv, p.XQ, p.CAT, cc, T, 0, st));
            CHK(pf_mm(y.gate, p.XQ, p.Z, vd, T, 0, st));
            CHK(pf_mm(y.alpha, p.XQ, p.A, a.nv, T, 0, st));
            CHK(pf_mm(y.beta, p.XQ, p.Bg, a.nv, T, 0, st));
            HCHK(oh_launch_conv_rows(p.CAT, (const float *)y.conv->A, z.conv, p.CONV, p.STAGE, T, base, cc, a.conv_k, st));
            HCHK(oh_launch_qk_gates_rows(a.dk, p.CONV, p.A, p.Bg, (const float *)y.ssm_a->A,
                                         (const float *)y.dt_bias->A, p.QN, p.KN, p.AL, p.BE, T, a.nk, a.nv, cc, st));
            if (chunked) {
                if (delta_mfma_enabled() && !p.WY)
                    CHK(salloc(s, &p.WY, (size_t)oh_delta_wy_floats(p.tc, a.nv, a.dk) + 64));
                HCHK(oh_launch_delta_chunked(a.dk, p.QN, p.KN, p.CONV, p.AL, p.BE, p.GR,
                                             delta_mfma_enabled() ? p.WY : nullptr, z.S, p.O, T, a.nk, a.nv, cc,
                                             1.0f / sqrtf((float)a.dk), st));
            } else {
                HCHK(oh_launch_delta_scan(a.dk, p.QN, p.KN, p.CONV, p.AL, p.BE, z.S, p.O, T, a.nk, a.nv, cc,
                                          1.0f / sqrtf((float)a.dk), st));
            }
            HCHK(oh_launch_gnorm_q8k_rows(p.O, p.Z, (const float *)y.ssm_norm->A, a.eps, vd, a.dv, T, p.OQ.qs,
                                          p.OQ.d, p.OQ.bs, st, p.OQ.bp));
            CHK(pf_mm(y.ssm_out, p.OQ, p.X, H, T, 1, st));
        }
        const bool slots = a.ne > 0 && !pf_moe_grouped(y);
        HCHK(oh_launch_norm_q8k_rows(p.X, (const float *)y.post_norm->A, a.eps, H, T, slots ? p.XN : nullptr, p.XQ.qs,
                                     p.XQ.d, p.XQ.bs, st, p.XQ.bp));
        if (a.ne > 0) {
            const int K = a.top_k, I = a.moe_inter, sI = a.shared_inter;
            CHK(pf_mm(y.router, p.XQ, p.RL, a.ne, T, 0, st));
            if (y.gate_inp_sh) CHK(pf_mm(y.gate_inp_sh, p.XQ, p.SHL, 1, T, 0, st));
            HCHK(oh_launch_route_rows(p.RL, a.ne, K, y.gate_inp_sh ? p.SHL : nullptr, p.RIDX, p.RW,
                                      y.gate_inp_sh ? p.SHG : nullptr, T, st));
            if (slots) {
                // experts without integer products (IQ2_XXS): the reference's
                // prompt runs the MoE per token (ffn_moe, src/ornith_rforward.c:
                // 672-673), so these are the token step's expert launches over
                // the chunk's T * K (token, expert) slots: slot t K + j is
                // token t's j-th routed expert and reads token t's normalised
                // row (and Q8_K planes) or its own silu(gate) * up
                const Act ax = act_of(p.XQ, p.XN);
                MvBuild b2, b3;
                if (pairable(y.gate_exps, y.up_exps)) {
                    CHK(mv_add_pair(b2, y.gate_exps, y.up_exps, ax, p.Hh, p.RIDX, T * K, I));
                    b2.L.s[b2.L.n - 1].astride = H;
                    b2.L.s[b2.L.n - 1].adiv = K;
                    CHK(mv_go(b2, st));
                    Act ah;
                    ah.pro = OH_PRO_F32;
                    ah.xf = p.Hh;
                    CHK(mv_add(b3, y.down_exps, ah, p.OD, 0, p.RIDX, T * K, H, I));
                } else {
                    float *G = p.GU, *U = p.GU + (size_t)T * K * I;
                    CHK(mv_add(b2, y.gate_exps, ax, G, 0, p.RIDX, T * K, I, H));
                    b2.L.s[b2.L.n - 1].adiv = K;
                    CHK(mv_add(b2, y.up_exps, ax, U, 0, p.RIDX, T * K, I, H));
                    b2.L.s[b2.L.n - 1].adiv = K;
                    CHK(mv_go(b2, st));
                    CHK(mv_add(b3, y.down_exps, act_swiglu(G, U), p.OD, 0, p.RIDX, T * K, H, I));
                }
                CHK(mv_go(b3, st));
            } else {
                HCHK(oh_launch_group_pairs(p.RIDX, T * K, p.CNT, a.ne, p.LIST, T, st));
                const int max_items = (T * K + 63) / 64 + a.ne;
                HCHK(oh_launch_mmq_items(p.CNT, a.ne, p.ITEMS, st));
                CHK(pf_swiglu(y.gate_exps, y.up_exps, p.XQ, I, T * K, T, p.HQ, p.GU, p.Hh, st, p.CNT, p.LIST, T, K,
                              a.ne, p.ITEMS, max_items));
                if (pf_use_mmq(y.down_exps, true, T))
                    CHK(pf_mmq(y.down_exps, nullptr, p.HQ, p.OD, H, T, 0, st, p.CNT, p.LIST, T, 1, p.ITEMS, max_items));
                else
                    CHK(pf_mvb(y.down_exps, nullptr, p.HQ, p.OD, H, T, 0, st, p.CNT, p.LIST, T, 1, a.ne));
            }
            if (y.gate_sh) {
                CHK(pf_swiglu(y.gate_sh, y.up_sh, p.XQ, sI, T, T, p.HSQ, p.GSH, p.HSH, st));
                CHK(pf_mm(y.down_sh, p.HSQ, p.ODSH, H, T, 0, st));
            }
            HCHK(oh_launch_moe_combine_rows(p.X, p.OD, p.RW, K, H, y.gate_sh ? p.ODSH : nullptr,
                                            y.gate_inp_sh ? p.SHG : nullptr, T, st));
        } else {
            const int I = a.shared_inter;
            CHK(pf_swiglu(y.ffn_gate, y.ffn_up, p.XQ, I, T, T, p.HSQ, p.GSH, p.HSH, st));
            CHK(pf_mm(y.ffn_down, p.HSQ, p.X, H, T, 1, st));
        }
    }
    // the last token's hidden state feeds the head
    HCHK(hipMemcpyAsync(s->x, p.X + (size_t)(T - 1) * H, (size_t)H * 4, hipMemcpyDeviceToDevice, st));
    return ORNITH_HIP_OK;
}

static bool pf_enabled() {
    const char *e = getenv("ORNITH_HIP_PREFILL");
    return !(e && e[0] == '0');
}

// the reference's prompt mode switch (src/ornith_rforward.c:838-849): default
// chunked delta scan, ORNITH_PREFILL_SERIAL=1 the token-by-token recurrence
static bool prefill_serial() {
    const char *e = getenv("ORNITH_PREFILL_SERIAL");
    return e && e[0] == '1';
}

// tokens through the layer-major prompt path (rprefill) or, with token_path,
// through the token step (rforward_token) one at a time
static int session_eval(ornith_hip_session *s, const int32_t *tokens, int n, bool token_path) {
    if (n <= 0) return ORNITH_HIP_OK;
    if (s->pos + n > s->cap) {
        seterr("session capacity %d exceeded (pos %d + %d tokens)", s->cap, s->pos, n);
        return ORNITH_HIP_ERR_UNSUPPORTED;
    }
    for (int i = 0; i < n; i++)
        if (tokens[i] < 0 || tokens[i] >= s->m->a.vocab) {
            seterr("token %d at %d outside the vocabulary (%d)", tokens[i], i, s->m->a.vocab);
            return ORNITH_HIP_ERR_FORMAT;
        }
    HCHK(hipSetDevice(s->m->ctx->device));
    hipStream_t st = s->m->ctx->st;
    CHK(sync_pos(s));
    HCHK(hipMemcpyAsync(s->toks + s->pos, tokens, (size_t)n * 4, hipMemcpyHostToDevice, st));
    const bool serial = prefill_serial();
    if (!token_path && (n > 1 || !serial) && pf_enabled() && pf_supported(s->m)) {
        // layer-major over chunks of tokens, then the head at the last one
        const int ct = pf_chunk_tokens();
        CHK(pf_alloc(s, n < ct ? n : ct));
        for (int c0 = 0; c0 < n; c0 += ct) {
            CHK(pf_chunk(s, s->pos + c0, n - c0 < ct ? n - c0 : ct, !serial, st));
            s->pf.last_base = s->pos + c0;
            s->pf.last_T = n - c0 < ct ? n - c0 : ct;
        }
        s->pf.pos_after = s->pos + n;   // outlives the asynchronous copy
        HCHK(hipMemcpyAsync(s->io + OH_IO_POS, &s->pf.pos_after, 4, hipMemcpyHostToDevice, st));
        CHK(run_head(s));
    } else if (n == 1) {
        // one token: body and head as one step (the greedy token lands at
        // toks[pos + 1], past the evaluated token)
        CHK(run_step(s));
    } else {
        for (int i = 0; i < n; i++) CHK(run_body(s));
        CHK(run_head(s));
    }
    HCHK(hipStreamSynchronize(st));
    CHK(step_check(s));
    s->pos += n;
    s->have_logits = true;
    return ORNITH_HIP_OK;
}

// ---- decode of several sessions at once -------------------------------------------------
// One token step (rforward_token, src/ornith_rforward.c:686-706) for each of n
// sessions of one model: the projections batched over the sessions
// (matmul_batch_q's Tn columns, src/ornith_rforward.c:91-196), the recurrent
// state, KV cache and attention of each session by the decode step's own
// kernels. Each column's arithmetic is its session's token step.
static int bw_alloc(ornith_hip_session *s, int n, size_t ops_bytes) {
    auto &p = s->bw;
    if (p.n >= n && p.ops_bytes >= ops_bytes) return ORNITH_HIP_OK;
    const ornith_hip_arch &a = s->m->a;
    const size_t N = (size_t)(n > p.n ? n : p.n), H = a.hidden, qd = (size_t)a.nk * a.dk, vd = (size_t)a.nv * a.dv;
    const size_t cc = 2 * qd + vd, aq = (size_t)a.nh * a.hd, kvd = (size_t)a.nkv * a.hd;
    const size_t K = a.top_k > 0 ? a.top_k : 1, I = a.moe_inter > 0 ? a.moe_inter : 1;
    const size_t sI = a.shared_inter > 0 ? a.shared_inter : 1, ne = a.ne > 0 ? a.ne : 1;
    CHK(salloc(s, &p.X, N * H)); CHK(q8alloc(s, p.XQ, N * H));
    CHK(salloc(s, &p.CAT, N * cc + 1)); CHK(salloc(s, &p.Z, N * vd + 1)); CHK(salloc(s, &p.AB, N * 2 * a.nv + 1));
    CHK(salloc(s, &p.O, N * vd + 1)); CHK(salloc(s, &p.OG, N * vd + 1)); CHK(salloc(s, &p.RUNS, N * (vd / 64) + 1));
    CHK(q8alloc(s, p.OQ, N * vd + 256));
    CHK(salloc(s, &p.QP, N * 2 * aq + 1)); CHK(salloc(s, &p.KB, N * kvd + 1)); CHK(salloc(s, &p.VB, N * kvd + 1));
    CHK(salloc(s, &p.QR, N * aq + 1)); CHK(salloc(s, &p.AG, N * aq + 1)); CHK(salloc(s, &p.OA, N * aq + 1));
    CHK(q8alloc(s, p.OAQ, N * aq + 256));
    CHK(salloc(s, &p.RL, N * ne)); CHK(salloc(s, &p.SHL, N)); CHK(salloc(s, &p.SHG, N));
    CHK(salloc(s, &p.RW, N * K)); CHK(salloc(s, &p.RIDX, N * K));
    CHK(salloc(s, &p.CNT, ne)); CHK(salloc(s, &p.LIST, ne * N));
    CHK(salloc(s, &p.ITEMS, (N * K + 63) / 64 + ne + 2));
    CHK(salloc(s, &p.Hh, N * K * I)); CHK(q8alloc(s, p.HQ, N * K * I + 256));
    CHK(salloc(s, &p.HSH, N * sI)); CHK(q8alloc(s, p.HSQ, N * sI + 256));
    CHK(salloc(s, &p.GU, N * K * 2 * I)); CHK(salloc(s, &p.GSH, N * 2 * sI));
    CHK(salloc(s, &p.OD, N * K * H)); CHK(salloc(s, &p.ODSH, N * H));
    CHK(salloc(s, &p.LOGITS, N * (size_t)a.vocab)); CHK(salloc(s, &p.IDX, 3 * N + 1));
    CHK(salloc(s, &p.AMV, N * OH_ARGMAX_BLOCKS)); CHK(salloc(s, &p.AMI, N * OH_ARGMAX_BLOCKS));
    const size_t ob = ops_bytes > p.ops_bytes ? ops_bytes : p.ops_bytes;
    CHK(salloc(s, &p.OPS, ob));
    p.ops_bytes = ob;
    p.n = (int)N;
    p.gen++;
    return ORNITH_HIP_OK;
}

// Host-side bounds check of a batch step's per-session descriptors (before
// they are uploaded): every buffer a descriptor names, with the extent the
// step's kernels reach through it at the session's position, lies inside one
// allocation of the session that owns it (the batch buffers: the leading
// session), and the attention grid and LDS cover every session's own.
// Returns a description of the first violation, or an empty string.
static bool owns(const ornith_hip_session *s, const void *p, size_t bytes) {
    const uintptr_t a = (uintptr_t)p;
    for (size_t i = 0; i < s->allocs.size(); i++) {
        const uintptr_t b = (uintptr_t)s->allocs[i];
        if (a >= b && a + bytes >= a && a + bytes <= b + s->asz[i]) return true;
    }
    return false;
}

static std::string batch_check(ornith_hip_session *const *ss, int n, const std::vector<size_t> &lofs,
                               const uint8_t *host, int nvb_main, int lds_main) {
    const ornith_hip_session *s0 = ss[0];
    const ornith_hip_model *m = s0->m;
    const ornith_hip_arch &a = m->a;
    const size_t F = sizeof(float), qd = (size_t)a.nk * a.dk, vd = (size_t)a.nv * a.dv, cc = 2 * qd + vd;
    const size_t aq = (size_t)a.nh * a.hd, kvd = (size_t)a.nkv * a.hd;
    char msg[256];
#define BC(own, ptr, bytes, what)                                                                           \
    do {                                                                                                    \
        if (!owns(own, ptr, bytes)) {                                                                       \
            snprintf(msg, sizeof msg, "layer %d session %d: %s (%zu bytes) outside its allocations", l, b,  \
                     what, (size_t)(bytes));                                                                \
            return msg;                                                                                     \
        }                                                                                                   \
    } while (0)
    for (int l = 0; l < a.n_layers; l++) {
        const uint8_t *src = host + lofs[(size_t)l];
        for (int b = 0; b < n; b++) {
            const ornith_hip_session *sb = ss[b];
            const int pos = sb->pos;
            if (m->L[l].full) {
                oh_op_prep pr;
                oh_op_attn at;
                memcpy(&pr, src + (size_t)b * sizeof(oh_op_prep), sizeof pr);
                memcpy(&at, src + (size_t)n * sizeof(oh_op_prep) + (size_t)b * sizeof(oh_op_attn), sizeof at);
                const size_t cap = (size_t)pr.cap, S = (size_t)oh_flash_slots(pr.cap);
                if (pr.cap % 16 || pos >= pr.cap || at.cap != pr.cap) {
                    snprintf(msg, sizeof msg, "layer %d session %d: position %d, KV capacity %d / %d", l, b, pos,
                             pr.cap, at.cap);
                    return msg;
                }
                BC(s0, pr.qproj, 2 * aq * F, "q projection");
                BC(s0, pr.kin, kvd * F, "k projection");
                BC(s0, pr.vin, kvd * F, "v projection");
                BC(sb, pr.rope, ((size_t)pos + 1) * (a.hd / 2) * 2 * F, "RoPE table");
                BC(s0, pr.qr, aq * F, "rotated queries");
                BC(s0, pr.gate, aq * F, "output gate");
                BC(sb, pr.Kt, kvd / 4 * cap * 4, "K codes");
                BC(sb, pr.Ks, cap * a.nkv * F, "K scales");
                BC(sb, pr.Vq, cap * kvd, "V codes");
                BC(sb, pr.Vs, cap * a.nkv * F, "V scales");
                if (at.qr != pr.qr || at.gate != pr.gate || at.Kt != pr.Kt || at.Ks != pr.Ks || at.Vq != pr.Vq ||
                    at.Vs != pr.Vs) {
                    snprintf(msg, sizeof msg, "layer %d session %d: attention and prep name different buffers", l, b);
                    return msg;
                }
                BC(sb, at.scores, (size_t)a.nh * cap * F, "scores");
                BC(sb, at.part_o, (size_t)a.nh * S * a.hd * F, "flash partial outputs");
                BC(sb, at.part_ml, (size_t)a.nh * S * 2 * F, "flash partial max/sum");
                BC(s0, at.out, aq * F, "attention output");
                const int nv_ex = a.nh / (256 / a.hd), nv_fl = oh_flash_nvb(a.nh, a.nkv, at.cap, at.hb);
                const int lds_ex = oh_exact_lds_bytes(a.hd, at.exact_max);
                const int lds_fl = oh_flash_form_lds(a.nh, a.nkv, a.hd, at.hb);
                if (nvb_main < nv_ex || nvb_main < nv_fl || lds_main < lds_ex || lds_main < lds_fl ||
                    lds_main > 65536) {
                    snprintf(msg, sizeof msg, "layer %d session %d: attention grid %d / LDS %d below %d, %d / %d, %d",
                             l, b, nvb_main, lds_main, nv_ex, nv_fl, lds_ex, lds_fl);
                    return msg;
                }
            } else {
                oh_op_delta d;
                memcpy(&d, src + (size_t)b * sizeof(oh_op_delta), sizeof d);
                if (d.cc != (int)cc || d.nv != a.nv || d.dk != a.dk || d.K != a.conv_k) {
                    snprintf(msg, sizeof msg, "layer %d session %d: delta shape", l, b);
                    return msg;
                }
                BC(s0, d.cat, cc * F, "qkv mix");
                BC(s0, d.ab, 2 * (size_t)a.nv * F, "alpha/beta");
                BC(s0, d.gate, vd * F, "z gate");
                BC(sb, d.conv_state, 2 * (size_t)(a.conv_k - 1) * cc * F, "conv window (two parities)");
                BC(sb, d.S, vd * a.dk * F, "delta state");
                BC(s0, d.out, vd * F, "delta output");
                BC(s0, d.out_gate, vd * F, "delta output gate");
                BC(s0, d.out_runs, vd / 64 * sizeof(double), "delta output runs");
            }
        }
    }
#undef BC
    for (int b = 0; b < n; b++)
        if (ss[b]->pos + 1 > ss[b]->cap || !owns(ss[b], ss[b]->toks, ((size_t)ss[b]->pos + 2) * 4)) {
            snprintf(msg, sizeof msg, "session %d: token history at position %d of %d", b, ss[b]->pos, ss[b]->cap);
            return msg;
        }
    return std::string();
}

// the device work of one batch step (its descriptors, tokens and positions
// already in p.OPS): everything but the host copies, so that it can be
// captured once and replayed for the same sessions
struct BatchPlan {
    ornith_hip_session **ss;
    int n;
    std::vector<size_t> lofs;
    size_t tok_ofs;
    int nvb_main, lds_main;
};

static int batch_enqueue(const BatchPlan &B, hipStream_t st) {
    ornith_hip_session **ss = B.ss;
    const int n = B.n;
    ornith_hip_session *s0 = ss[0];
    const ornith_hip_model *m = s0->m;
    const ornith_hip_arch &a = m->a;
    auto &p = s0->bw;
    const int H = a.hidden, qd = a.nk * a.dk, vd = a.nv * a.dv, cc = 2 * qd + vd, aq = a.nh * a.hd;
    const int kvd = a.nkv * a.hd;
    const int32_t *dtok = (const int32_t *)(p.OPS + B.tok_ofs), *dpos = dtok + n;
    int32_t *const *dtoks = (int32_t *const *)(p.OPS + B.tok_ofs + (((size_t)n * 8 + 15) & ~(size_t)15));
    oh_op_embed emb = {m->embd->A, m->embd->B, m->embd->C, dtok, p.X, (int)m->embd->type, H};
    HCHK(oh_launch_embed_rows(&emb, 0, n, st));
    // below the matrix-core column count the dense projections run as the
    // token step's fused multi-segment launches with one slot per session
    // (the normalisation / gated norm / f32 activation formed in the launch's
    // prologue, weights re-read per slot from the caches); the expert and
    // head products keep the column-streaming batched kernels
    const bool fused = n < kMmqMinTokens && batch_fused();
    for (int l = 0; l < a.n_layers; l++) {
        const OhLayer &y = m->L[l];
        const uint8_t *dops = p.OPS + B.lofs[l];
        const Act an = act_norm(p.X, (const float *)y.attn_norm->A, a.eps);
        if (!fused)
            HCHK(oh_launch_norm_q8k_rows(p.X, (const float *)y.attn_norm->A, a.eps, H, n, nullptr, p.XQ.qs, p.XQ.d,
                                         p.XQ.bs, st, p.XQ.bp));
        if (y.full) {
            if (fused) {
                MvBuild b;
                CHK(mv_add(b, y.q, an, p.QP, 0, nullptr, n, 2 * aq, H));
                CHK(mv_add(b, y.k, an, p.KB, 0, nullptr, n, kvd, H));
                CHK(mv_add(b, y.v, an, p.VB, 0, nullptr, n, kvd, H));
                CHK(mv_go(b, st));
            } else {
                CHK(pf_mm(y.q, p.XQ, p.QP, 2 * aq, n, 0, st));
                CHK(pf_mm(y.k, p.XQ, p.KB, kvd, n, 0, st));
                CHK(pf_mm(y.v, p.XQ, p.VB, kvd, n, 0, st));
            }
            const oh_op_prep *pops = (const oh_op_prep *)dops;
            const oh_op_attn *aops = (const oh_op_attn *)(dops + (size_t)n * sizeof(oh_op_prep));
            HCHK(oh_launch_prep_batch(pops, dpos, n, a.nh, a.nkv, st));
            HCHK(oh_launch_attn_batch(aops, dpos, n, B.nvb_main, B.lds_main, a.nh, a.hd, st));
            if (fused) {
                MvBuild b;
                Act af;
                af.pro = OH_PRO_F32;
                af.xf = p.OA;
                CHK(mv_add(b, y.o, af, p.X, 1, nullptr, n, H, aq));
                CHK(mv_go(b, st));
            } else {
                HCHK(oh_launch_norm_q8k_rows(p.OA, nullptr, 0.0f, aq, n, nullptr, p.OAQ.qs, p.OAQ.d, p.OAQ.bs, st,
                                             p.OAQ.bp));
                CHK(pf_mm(y.o, p.OAQ, p.X, H, n, 1, st));
            }
        } else {
            if (fused) {
                MvBuild b;
                CHK(mv_add(b, y.qkv, an, p.CAT, 0, nullptr, n, cc, H));
                CHK(mv_add(b, y.gate, an, p.Z, 0, nullptr, n, vd, H));
                CHK(mv_add(b, y.alpha, an, p.AB, 0, nullptr, n, 2 * a.nv, H));
                CHK(mv_add(b, y.beta, an, p.AB + a.nv, 0, nullptr, n, 2 * a.nv, H));
                CHK(mv_go(b, st));
            } else {
                CHK(pf_mm(y.qkv, p.XQ, p.CAT, cc, n, 0, st));
                CHK(pf_mm(y.gate, p.XQ, p.Z, vd, n, 0, st));
                CHK(pf_mm(y.alpha, p.XQ, p.AB, 2 * a.nv, n, 0, st));
                CHK(pf_mm(y.beta, p.XQ, p.AB + a.nv, 2 * a.nv, n, 0, st));
            }
            HCHK(oh_launch_delta_batch((const oh_op_delta *)dops, dpos, n, a.dk, a.conv_k, a.nv, st));
            if (fused) {
                MvBuild b;
                CHK(mv_add(b, y.ssm_out, act_gnorm(p.O, p.OG, p.RUNS, (const float *)y.ssm_norm->A, a.eps, a.dv),
                           p.X, 1, nullptr, n, H, vd));
                CHK(mv_go(b, st));
            } else {
                HCHK(oh_launch_gnorm_q8k_rows(p.O, p.Z, (const float *)y.ssm_norm->A, a.eps, vd, a.dv, n, p.OQ.qs,
                                              p.OQ.d, p.OQ.bs, st, p.OQ.bp));
                CHK(pf_mm(y.ssm_out, p.OQ, p.X, H, n, 1, st));
            }
        }
        const Act pn = act_norm(p.X, (const float *)y.post_norm->A, a.eps);
        if (!fused || a.ne <= 0)
            HCHK(oh_launch_norm_q8k_rows(p.X, (const float *)y.post_norm->A, a.eps, H, n, nullptr, p.XQ.qs, p.XQ.d,
                                         p.XQ.bs, st, p.XQ.bp));
        if (a.ne > 0) {
            const int K = a.top_k, I = a.moe_inter, sI = a.shared_inter;
            if (fused) {
                // router + shared gate; each slot's first block stores its
                // Q8_K activation (p.XQ) for the expert products
                Act pst = pn;
                pst.oqs = p.XQ.qs; pst.oqd = p.XQ.d; pst.oqb = p.XQ.bs;
                MvBuild b;
                CHK(mv_add(b, y.router, pst, p.RL, 0, nullptr, n, a.ne, H));
                if (y.gate_inp_sh) CHK(mv_add(b, y.gate_inp_sh, pn, p.SHL, 0, nullptr, n, 1, H));
                CHK(mv_go(b, st));
            } else {
                CHK(pf_mm(y.router, p.XQ, p.RL, a.ne, n, 0, st));
                if (y.gate_inp_sh) CHK(pf_mm(y.gate_inp_sh, p.XQ, p.SHL, 1, n, 0, st));
            }
            // the token step's two MoE launches for all n tokens: the experts
            // gate/up with each (token, expert) slot routing its own token,
            // then the fused down projection + combine with a grid row per
            // token (same conditions as the token step's fused down)
            const bool paired = pairable(y.gate_exps, y.up_exps) && (!y.gate_sh || pairable(y.gate_sh, y.up_sh));
            const uint32_t dt = y.down_exps->type;
            const int nbd = I / 256, ns = K + (y.gate_sh ? 1 : 0);
            const int rps = nbd >= 1 ? 64 / nbd : 1;
            const int dlds = ns * ((nbd * 272 + nbd * 36 + 15) & ~15) + ns * I * 4 + ns * rps * 4;
            if (fused && paired && oh_qdot_can(dt, I) && nbd >= 1 && nbd <= 64 && ns <= 10 && dlds <= 65536 &&
                y.gate_exps->type == y.router->type && (!y.gate_sh || (y.down_sh->type == dt && sI == I))) {
                MvBuild b2;
                const Act ax = act_of(p.XQ, nullptr);
                CHK(mv_add_pair(b2, y.gate_exps, y.up_exps, ax, p.Hh, p.RIDX, n * K, I));
                b2.L.s[b2.L.n - 1].astride = H;
                b2.L.s[b2.L.n - 1].adiv = K;
                if (y.gate_sh) {
                    CHK(mv_add_pair(b2, y.gate_sh, y.up_sh, ax, p.HSH, nullptr, n, sI));
                    b2.L.s[b2.L.n - 1].astride = H;
                }
                b2.L.route = 1;
                b2.L.tslots = K;
                b2.L.rlog = p.RL;
                b2.L.shl = y.gate_inp_sh ? p.SHL : nullptr;
                b2.L.ne = a.ne;
                b2.L.topk = K;
                b2.L.ridx = p.RIDX;
                b2.L.rw = p.RW;
                b2.L.shg = p.SHG;
                CHK(mv_go(b2, st));
                oh_mvdown D;
                memset(&D, 0, sizeof D);
                D.A = y.down_exps->A; D.B = y.down_exps->B; D.C = y.down_exps->C;
                if (y.gate_sh) { D.sA = y.down_sh->A; D.sB = y.down_sh->B; D.sC = y.down_sh->C; }
                D.eidx = p.RIDX; D.w = p.RW; D.shg = y.gate_inp_sh ? p.SHG : nullptr;
                D.h = p.Hh; D.hsh = p.HSH; D.x = p.X;
                D.hts = (size_t)K * I; D.hsts = (size_t)sI; D.xts = (size_t)H;
                D.type = (int)dt; D.nb = nbd; D.in = I; D.rows = H; D.k = K; D.stride = I;
                HCHK(oh_launch_mv_down_rows(&D, (H + rps - 1) / rps, n, dlds, st));
                continue;
            }
            HCHK(oh_launch_route_rows(p.RL, a.ne, K, y.gate_inp_sh ? p.SHL : nullptr, p.RIDX, p.RW,
                                      y.gate_inp_sh ? p.SHG : nullptr, n, st));
            HCHK(oh_launch_group_pairs(p.RIDX, n * K, p.CNT, a.ne, p.LIST, n, st));
            const int max_items = (n * K + 63) / 64 + a.ne;
            HCHK(oh_launch_mmq_items(p.CNT, a.ne, p.ITEMS, st));
            CHK(pf_swiglu(y.gate_exps, y.up_exps, p.XQ, I, n * K, n, p.HQ, p.GU, p.Hh, st, p.CNT, p.LIST, n, K, a.ne,
                          p.ITEMS, max_items));
            if (pf_use_mmq(y.down_exps, true, n))
                CHK(pf_mmq(y.down_exps, nullptr, p.HQ, p.OD, H, n, 0, st, p.CNT, p.LIST, n, 1, p.ITEMS, max_items));
            else
                CHK(pf_mvb(y.down_exps, nullptr, p.HQ, p.OD, H, n, 0, st, p.CNT, p.LIST, n, 1, a.ne));
            if (y.gate_sh) {
                CHK(pf_swiglu(y.gate_sh, y.up_sh, p.XQ, sI, n, n, p.HSQ, p.GSH, p.HSH, st));
                CHK(pf_mm(y.down_sh, p.HSQ, p.ODSH, H, n, 0, st));
            }
            HCHK(oh_launch_moe_combine_rows(p.X, p.OD, p.RW, K, H, y.gate_sh ? p.ODSH : nullptr,
                                            y.gate_inp_sh ? p.SHG : nullptr, n, st));
        } else {
            CHK(pf_swiglu(y.ffn_gate, y.ffn_up, p.XQ, a.shared_inter, n, n, p.HSQ, p.GSH, p.HSH, st));
            CHK(pf_mm(y.ffn_down, p.HSQ, p.X, H, n, 1, st));
        }
    }
    // head: output norm, lm_head over the n columns, each session's logits and
    // greedy token; the token history of each session gets this step's token
    // and, at the next position, the greedy one (where the token step's head
    // leaves it for session_generate)
    HCHK(oh_launch_norm_q8k_rows(p.X, (const float *)m->out_norm->A, a.eps, H, n, nullptr, p.XQ.qs, p.XQ.d,
                                 p.XQ.bs, st, p.XQ.bp));
    CHK(pf_mm(m->lm_head, p.XQ, p.LOGITS, a.vocab, n, 0, st));
    HCHK(oh_launch_argmax_rows(p.LOGITS, a.vocab, n, p.IDX, st, p.AMV, p.AMI));
    for (int b = 0; b < n; b++)
        HCHK(hipMemcpyAsync(ss[b]->logits, p.LOGITS + (size_t)b * a.vocab, (size_t)a.vocab * 4,
                            hipMemcpyDeviceToDevice, st));
    HCHK(oh_launch_batch_tokens(dtoks, dpos, dtok, p.IDX, n, st));
    return ORNITH_HIP_OK;
}

extern "C" int ornith_hip_batch_step(ornith_hip_session **ss, int n, const int32_t *tokens, int32_t *next) {
    if (n <= 0) return ORNITH_HIP_OK;
    if (!ss || !tokens) { seterr("batch_step: null sessions or tokens"); return ORNITH_HIP_ERR_FORMAT; }
    ornith_hip_session *s0 = ss[0];
    const ornith_hip_model *m = s0->m;
    const ornith_hip_arch &a = m->a;
    for (int b = 0; b < n; b++) {
        if (!ss[b] || ss[b]->m != m) { seterr("batch_step: session %d is not of the first session's model", b); return ORNITH_HIP_ERR_FORMAT; }
        for (int c = 0; c < b; c++)
            if (ss[c] == ss[b]) { seterr("batch_step: session %d appears twice", b); return ORNITH_HIP_ERR_FORMAT; }
        if (ss[b]->pos + 1 > ss[b]->cap) {
            seterr("session capacity %d exceeded (pos %d + 1 token) in batch slot %d", ss[b]->cap, ss[b]->pos, b);
            return ORNITH_HIP_ERR_UNSUPPORTED;
        }
        if (tokens[b] < 0 || tokens[b] >= a.vocab) {
            seterr("token %d in batch slot %d outside the vocabulary (%d)", tokens[b], b, a.vocab);
            return ORNITH_HIP_ERR_FORMAT;
        }
    }
    // one KV capacity, exact_max and flash form across the batch, and every
    // context on the same attention path (all within exact_max or all past
    // it): the only mixes the batch step is run with; others are refused
    for (int b = 1; b < n; b++) {
        const ornith_hip_session *x = ss[b], *y = ss[0];
        const int lim = oh_exact_limit(y->exact_max);
        if (x->kvcap != y->kvcap || x->exact_max != y->exact_max || x->flash_mfma != y->flash_mfma ||
            (x->pos + 1 <= lim) != (y->pos + 1 <= lim)) {
            seterr("batch_step: session %d differs from session 0 in KV capacity (%d / %d), attention settings or "
                   "attention path (position %d / %d); a batch takes sessions of one capacity on one path",
                   b, x->kvcap, y->kvcap, x->pos, y->pos);
            return ORNITH_HIP_ERR_UNSUPPORTED;
        }
    }
    if (!pf_supported(m) || !oh_qdot_can(m->lm_head->type, m->lm_head->in) || m->lm_head->in > 8192) {
        seterr("batch_step: the model is outside the batched projection path (widths <= 8192, integer dot types)");
        return ORNITH_HIP_ERR_UNSUPPORTED;
    }
    if (!graphs_enabled()) {
        // the batch step runs as one captured HIP graph; its eager form is
        // switched off (a GPU fault in an eager batch run is not explained)
        seterr("batch_step: needs HIP graphs (unset ORNITH_HIP_NO_GRAPH)");
        return ORNITH_HIP_ERR_UNSUPPORTED;
    }
    HCHK(hipSetDevice(m->ctx->device));
    hipStream_t st = m->ctx->st;
    const int qd = a.nk * a.dk, vd = a.nv * a.dv, cc = 2 * qd + vd, aq = a.nh * a.hd;
    const int kvd = a.nkv * a.hd;
    // per-layer descriptors of every session: delta ops (linear layers) or
    // prep + attention ops (full layers), n of each; then tokens, positions
    // and the sessions' token histories
    BatchPlan B;
    B.ss = ss;
    B.n = n;
    B.lofs.resize((size_t)a.n_layers);
    size_t ob = 0;
    for (int l = 0; l < a.n_layers; l++) {
        B.lofs[l] = ob;
        ob += m->L[l].full ? (size_t)n * (sizeof(oh_op_prep) + sizeof(oh_op_attn)) : (size_t)n * sizeof(oh_op_delta);
        ob = (ob + 15) & ~(size_t)15;
    }
    B.tok_ofs = ob;
    ob += (((size_t)n * 8 + 15) & ~(size_t)15) + (size_t)n * sizeof(int32_t *) + 16;
    CHK(bw_alloc(s0, n, ob));
    auto &p = s0->bw;
    std::vector<uint8_t> host(ob, 0);
    B.nvb_main = 1;
    B.lds_main = 0;
    for (int l = 0; l < a.n_layers; l++) {
        const OhLayer &y = m->L[l];
        uint8_t *dst = host.data() + B.lofs[l];
        for (int b = 0; b < n; b++) {
            ornith_hip_session *sb = ss[b];
            const LayerState &z = sb->ls[l];
            if (y.full) {
                oh_op_prep pr = {p.QP + (size_t)b * 2 * aq, p.KB + (size_t)b * kvd, p.VB + (size_t)b * kvd,
                                 (const float *)y.q_norm->A, (const float *)y.k_norm->A, (const float *)sb->rope,
                                 p.QR + (size_t)b * aq, p.AG + (size_t)b * aq, z.Kt, z.Ks, z.Vq, z.Vs,
                                 a.nh, a.nkv, a.hd, a.rope_dim, sb->kvcap, a.eps};
                memcpy(dst + (size_t)b * sizeof(oh_op_prep), &pr, sizeof pr);
                oh_op_attn at;
                memset(&at, 0, sizeof at);
                at.qr = p.QR + (size_t)b * aq; at.gate = p.AG + (size_t)b * aq;
                at.Kt = z.Kt; at.Ks = z.Ks; at.Vq = z.Vq; at.Vs = z.Vs;
                at.scores = sb->scores; at.part_o = sb->fpo; at.part_ml = sb->fpml; at.out = p.OA + (size_t)b * aq;
                at.nh = a.nh; at.nkv = a.nkv; at.hd = a.hd; at.cap = sb->kvcap; at.exact_max = sb->exact_max;
                at.hb = oh_flash_form(a.nh, a.nkv, a.hd, sb->flash_mfma); at.scale = 1.0f / sqrtf((float)a.hd);
                memcpy(dst + (size_t)n * sizeof(oh_op_prep) + (size_t)b * sizeof(oh_op_attn), &at, sizeof at);
                const int nv_ex = a.nh / (256 / a.hd), nv_fl = oh_flash_nvb(a.nh, a.nkv, sb->kvcap, at.hb);
                const int lds_ex = oh_exact_lds_bytes(a.hd, sb->exact_max), lds_fl = oh_flash_form_lds(a.nh, a.nkv, a.hd, at.hb);
                B.nvb_main = std::max(B.nvb_main, std::max(nv_ex, nv_fl));
                B.lds_main = std::max(B.lds_main, std::max(lds_ex, lds_fl));
            } else {
                oh_op_delta d = {p.CAT + (size_t)b * cc, p.AB + (size_t)b * 2 * a.nv, p.Z + (size_t)b * vd,
                                 (const float *)y.conv->A, (const float *)y.ssm_a->A, (const float *)y.dt_bias->A,
                                 z.conv, z.S, p.O + (size_t)b * vd, p.OG + (size_t)b * vd,
                                 p.RUNS + (size_t)b * (vd / 64), a.dk, a.nk, a.nv, a.conv_k, cc,
                                 1.0f / sqrtf((float)a.dk)};
                memcpy(dst + (size_t)b * sizeof(oh_op_delta), &d, sizeof d);
            }
        }
    }
    // the full bounds check runs whenever a plan is captured (the descriptors
    // of the same sessions do not change between replays; the positions are
    // checked against the capacities above on every step)
    auto check = [&]() -> int {
        const std::string bad = batch_check(ss, n, B.lofs, host.data(), B.nvb_main, B.lds_main);
        if (!bad.empty()) { seterr("batch_step plan: %s", bad.c_str()); return ORNITH_HIP_ERR_DEVICE; }
        return ORNITH_HIP_OK;
    };
    int32_t *htp = (int32_t *)(host.data() + B.tok_ofs);
    int32_t **htk = (int32_t **)(host.data() + B.tok_ofs + (((size_t)n * 8 + 15) & ~(size_t)15));
    for (int b = 0; b < n; b++) { htp[b] = tokens[b]; htp[n + b] = ss[b]->pos; htk[b] = ss[b]->toks; }
    HCHK(hipMemcpyAsync(p.OPS, host.data(), ob, hipMemcpyHostToDevice, st));
    if (graphs_enabled()) {
        // one captured step per set of sessions (ids, not addresses), buffer
        // generation, product path, batch plan and attention grid
        std::vector<uint64_t> key;
        key.push_back((uint64_t)n);
        key.push_back((uint64_t)p.gen);
        key.push_back(mmq_enabled() ? 1u : 0u);
        key.push_back(batch_fused() ? 1u : 0u);
        key.push_back((uint64_t)B.nvb_main << 32 | (uint32_t)B.lds_main);
        for (int b = 0; b < n; b++) key.push_back(ss[b]->sid);
        if (!p.graph || p.key != key) {
            CHK(check());
            if (p.graph) { (void)hipGraphExecDestroy(p.graph); p.graph = nullptr; }
            hipGraph_t g = nullptr;
            HCHK(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
            const int r = batch_enqueue(B, st);
            hipError_t e = hipStreamEndCapture(st, &g);
            if (r != ORNITH_HIP_OK) { if (g) (void)hipGraphDestroy(g); return r; }
            if (e != hipSuccess) { seterr("batch graph capture: %s", hipGetErrorString(e)); return ORNITH_HIP_ERR_DEVICE; }
            e = hipGraphInstantiate(&p.graph, g, nullptr, nullptr, 0);
            (void)hipGraphDestroy(g);
            if (e != hipSuccess) { p.graph = nullptr; seterr("batch graph instantiate: %s", hipGetErrorString(e)); return ORNITH_HIP_ERR_DEVICE; }
            p.key = key;
        }
        HCHK(hipGraphLaunch(p.graph, st));
    } else {
        CHK(check());
        CHK(batch_enqueue(B, st));
    }
    std::vector<int32_t> hn((size_t)n);
    HCHK(hipMemcpyAsync(hn.data(), p.IDX, (size_t)n * 4, hipMemcpyDeviceToHost, st));
    HCHK(hipStreamSynchronize(st));
    for (int b = 0; b < n; b++) {
        ss[b]->pos += 1;
        ss[b]->have_logits = true;
        if (next) next[b] = hn[b];
    }
    return ORNITH_HIP_OK;
}

extern "C" int ornith_hip_session_eval(ornith_hip_session *s, const int32_t *tokens, int n) {
    return session_eval(s, tokens, n, false);
}

// rforward_token whatever the prompt mode (a one-token evaluation in the
// chunked mode is a one-token delta chunk, which rounds differently)
extern "C" int ornith_hip_session_step(ornith_hip_session *s, int32_t token) {
    return session_eval(s, &token, 1, true);
}

extern "C" int ornith_hip_session_logits(ornith_hip_session *s, float *out) {
    if (!s->have_logits) { seterr("session has no logits; eval a prompt first"); return ORNITH_HIP_ERR_FORMAT; }
    HCHK(hipSetDevice(s->m->ctx->device));
    HCHK(hipMemcpyAsync(out, s->logits, (size_t)s->m->a.vocab * 4, hipMemcpyDeviceToHost, s->m->ctx->st));
    HCHK(hipStreamSynchronize(s->m->ctx->st));
    return ORNITH_HIP_OK;
}

extern "C" int ornith_hip_session_pos(const ornith_hip_session *s) { return s->pos; }

extern "C" int ornith_hip_session_generate(ornith_hip_session *s, int n_predict, int32_t *out_tokens,
                                           int *n_out) {
    if (n_out) *n_out = 0;
    if (!s->have_logits) { seterr("session has no logits; eval a prompt first"); return ORNITH_HIP_ERR_FORMAT; }
    HCHK(hipSetDevice(s->m->ctx->device));
    hipStream_t st = s->m->ctx->st;
    int n = n_predict < 0 ? 0 : n_predict;
    if (n > s->cap - s->pos) n = s->cap - s->pos;
    CHK(sync_pos(s));
    const int32_t eos = s->m->a.eos;
    int emitted = 0;
    if (eos < 0) {
        // no stop token: the whole loop stays on the device
        for (int i = 0; i < n; i++) CHK(run_step(s));
        HCHK(hipMemcpyAsync(out_tokens, s->toks + s->pos, (size_t)n * 4, hipMemcpyDeviceToHost, st));
        HCHK(hipStreamSynchronize(st));
        CHK(step_check(s));
        emitted = n;
    } else {
        for (int i = 0; i < n; i++) {
            int32_t next;
            HCHK(hipMemcpyAsync(&next, s->toks + s->pos + i, 4, hipMemcpyDeviceToHost, st));
            HCHK(hipStreamSynchronize(st));
            CHK(step_check(s));
            if (next == eos) break;
            out_tokens[emitted++] = next;
            CHK(run_step(s));
        }
        HCHK(hipStreamSynchronize(st));
    }
    s->pos += emitted;
    if (n_out) *n_out = emitted;
    return ORNITH_HIP_OK;
}

extern "C" int ornith_hip_session_time_decode(ornith_hip_session *s, int n_steps, float *ms) {
    if (!s->have_logits) { seterr("session has no logits; eval a prompt first"); return ORNITH_HIP_ERR_FORMAT; }
    if (n_steps < 0 || s->pos + n_steps > s->cap) { seterr("time_decode: %d steps exceed capacity", n_steps); return ORNITH_HIP_ERR_UNSUPPORTED; }
    HCHK(hipSetDevice(s->m->ctx->device));
    hipStream_t st = s->m->ctx->st;
    CHK(sync_pos(s));
    if (step_enabled()) CHK(step_prepare(s));
    if (dec_enabled() && !step_enabled()) CHK(dec_prepare(s));
    if (!s->step_grid && !s->dec.grid && graphs_enabled()) {
        if (!s->gbody) CHK(capture(s, enqueue_body, &s->gbody));
        if (!s->ghead) CHK(capture(s, enqueue_head, &s->ghead));
    }
    hipEvent_t e0, e1;
    HCHK(hipEventCreate(&e0));
    HCHK(hipEventCreate(&e1));
    HCHK(hipEventRecord(e0, st));
    for (int i = 0; i < n_steps; i++) CHK(run_step(s));
    HCHK(hipEventRecord(e1, st));
    HCHK(hipEventSynchronize(e1));
    float el = 0.0f;
    HCHK(hipEventElapsedTime(&el, e0, e1));
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    CHK(step_check(s));
    s->pos += n_steps;
    *ms = el;
    return ORNITH_HIP_OK;
}

// ---- state download in the reference layouts -------------------------------------------------
extern "C" int ornith_hip_session_get_delta(ornith_hip_session *s, int l, float *S) {
    const ornith_hip_arch &a = s->m->a;
    if (l < 0 || l >= a.n_layers || s->m->L[l].full) { seterr("layer %d has no delta state", l); return ORNITH_HIP_ERR_NOTFOUND; }
    HCHK(hipSetDevice(s->m->ctx->device));
    const size_t per = (size_t)a.dk * a.dv;
    HCHK(hipMemcpy(S, s->ls[l].S, (size_t)a.nv * per * 4, hipMemcpyDeviceToHost));   // [h][r][c] on both sides
    return ORNITH_HIP_OK;
}

extern "C" int ornith_hip_session_get_conv(ornith_hip_session *s, int l, float *win) {
    const ornith_hip_arch &a = s->m->a;
    if (l < 0 || l >= a.n_layers || s->m->L[l].full) { seterr("layer %d has no conv state", l); return ORNITH_HIP_ERR_NOTFOUND; }
    HCHK(hipSetDevice(s->m->ctx->device));
    const size_t cc = (size_t)(2 * a.nk * a.dk + a.nv * a.dv), wsz = (size_t)(a.conv_k - 1) * cc;
    // the window written by the last step lives in parity (pos & 1)
    HCHK(hipMemcpy(win, s->ls[l].conv + (size_t)(s->pos & 1) * wsz, wsz * 4, hipMemcpyDeviceToHost));
    return ORNITH_HIP_OK;
}

extern "C" int ornith_hip_session_get_kv(ornith_hip_session *s, int l, int8_t *Kq, float *Ks,
                                         int8_t *Vq, float *Vs) {
    const ornith_hip_arch &a = s->m->a;
    if (l < 0 || l >= a.n_layers || !s->m->L[l].full) { seterr("layer %d has no KV cache", l); return ORNITH_HIP_ERR_NOTFOUND; }
    HCHK(hipSetDevice(s->m->ctx->device));
    const int len = s->pos, cap = s->kvcap, hd = a.hd, nkv = a.nkv;
    std::vector<uint32_t> kt((size_t)nkv * (hd / 4) * cap);
    HCHK(hipMemcpy(kt.data(), s->ls[l].Kt, kt.size() * 4, hipMemcpyDeviceToHost));
    std::vector<int8_t> vt((size_t)nkv * cap * hd);
    HCHK(hipMemcpy(vt.data(), s->ls[l].Vq, vt.size(), hipMemcpyDeviceToHost));
    for (int t = 0; t < len; t++)
        for (int h = 0; h < nkv; h++)
            for (int i = 0; i < hd; i++) {
                const uint32_t w = kt[((size_t)h * (hd / 4) + i / 4) * cap + t];
                Kq[((size_t)t * nkv + h) * hd + i] = (int8_t)((w >> (8 * (i & 3))) & 0xff);
                Vq[((size_t)t * nkv + h) * hd + i] = vt[(((size_t)h * (cap / 16) + t / 16) * hd + i) * 16 + (t & 15)];
            }
    HCHK(hipMemcpy(Ks, s->ls[l].Ks, (size_t)len * nkv * 4, hipMemcpyDeviceToHost));
    HCHK(hipMemcpy(Vs, s->ls[l].Vs, (size_t)len * nkv * 4, hipMemcpyDeviceToHost));
    return ORNITH_HIP_OK;
}

// The last full-attention layer's attention inputs and output as the most
// recent evaluation left them: row < 0, the decode step's (the query heads
// after q_norm and RoPE, the output gate, and o = attention * sigmoid(gate)
// before attn_output's Q8_K, src/ornith_rforward.c:419-455); row >= 0, that
// row of the most recent prompt chunk. Only meaningful when the model's last
// layer is a full-attention layer (later linear layers reuse o). *pos: the
// position the row attended from.
extern "C" int ornith_hip_session_get_attn(ornith_hip_session *s, int row, float *q, float *gate, float *o,
                                           int32_t *pos) {
    const ornith_hip_arch &a = s->m->a;
    const size_t aq = (size_t)a.nh * a.hd;
    if (a.n_layers < 1 || !s->m->L[a.n_layers - 1].full) {
        seterr("get_attn: the last layer is not a full-attention layer");
        return ORNITH_HIP_ERR_UNSUPPORTED;
    }
    HCHK(hipSetDevice(s->m->ctx->device));
    HCHK(hipStreamSynchronize(s->m->ctx->st));
    const float *dq, *dg, *dout;
    if (row < 0) {
        if (s->pos < 1) { seterr("get_attn: no decode step yet"); return ORNITH_HIP_ERR_UNSUPPORTED; }
        dq = s->qr; dg = s->agate; dout = s->o;
        *pos = s->pos - 1;
    } else {
        if (row >= s->pf.last_T || !s->pf.QR) {
            seterr("get_attn: row %d outside the last prompt chunk (%d rows)", row, s->pf.last_T);
            return ORNITH_HIP_ERR_FORMAT;
        }
        dq = s->pf.QR + (size_t)row * aq; dg = s->pf.AG + (size_t)row * aq; dout = s->pf.OA + (size_t)row * aq;
        *pos = s->pf.last_base + row;
    }
    HCHK(hipMemcpy(q, dq, aq * 4, hipMemcpyDeviceToHost));
    HCHK(hipMemcpy(gate, dg, aq * 4, hipMemcpyDeviceToHost));
    HCHK(hipMemcpy(o, dout, aq * 4, hipMemcpyDeviceToHost));
    return ORNITH_HIP_OK;
}

// ---- session snapshots (rmodel_session_save / rmodel_session_load, src/ornith_rforward.c:986-1171) ----
// The reference's ORNSESS v1 file, byte for byte: magic, version, the
// architecture fingerprint (13 int32), pos, nhist, the FNV-1a 64 hash of the
// token history, have_logits; per layer the Q8 KV cache (quantized, len, nkv,
// hd, K codes, V codes [len][nkv][hd], K and V scales [len][nkv]) or the delta
// state [nv][dv][dk] and the conv window (K, C, [(K-1)][C] oldest first); the
// token history; the logits.
static const char kSessMagic[8] = {'O', 'R', 'N', 'S', 'E', 'S', 'S', '\0'};
static const uint32_t kSessVersion = 1;

static void sess_fp(const ornith_hip_arch &a, int32_t fp[13]) {
    const int32_t v[13] = {a.hidden, a.n_layers, a.nh, a.nkv, a.hd, a.full_interval, a.nk, a.nv, a.dk, a.dv,
                           a.conv_k, a.ne, a.vocab};
    memcpy(fp, v, sizeof v);
}

static uint64_t sess_prefix_hash(const int32_t *t, int n) {
    uint64_t h = 1469598103934665603ULL;
    const uint8_t *p = (const uint8_t *)t;
    for (size_t i = 0; i < (size_t)n * 4; i++) {
        h ^= p[i];
        h *= 1099511628211ULL;
    }
    return h;
}

extern "C" int ornith_hip_session_save(ornith_hip_session *s, const char *path) {
    const ornith_hip_arch &a = s->m->a;
    HCHK(hipSetDevice(s->m->ctx->device));
    HCHK(hipStreamSynchronize(s->m->ctx->st));
    const int pos = s->pos, cc = 2 * a.nk * a.dk + a.nv * a.dv;
    std::vector<int32_t> hist((size_t)pos + 1);
    if (pos > 0) HCHK(hipMemcpy(hist.data(), s->toks, (size_t)pos * 4, hipMemcpyDeviceToHost));
    std::vector<uint8_t> out;
    auto put = [&](const void *p, size_t n) { out.insert(out.end(), (const uint8_t *)p, (const uint8_t *)p + n); };
    auto put32 = [&](int32_t v) { put(&v, 4); };
    put(kSessMagic, 8);
    put(&kSessVersion, 4);
    int32_t fp[13];
    sess_fp(a, fp);
    put(fp, sizeof fp);
    const int32_t hl = s->have_logits ? 1 : 0;
    const uint64_t ph = sess_prefix_hash(hist.data(), pos);
    put32(pos);
    put32(pos);                                   // nhist: every token fed so far
    put(&ph, 8);
    put32(hl);
    for (int l = 0; l < a.n_layers; l++) {
        if (s->m->L[l].full) {
            const size_t hv = (size_t)pos * a.nkv * a.hd, sc = (size_t)pos * a.nkv;
            std::vector<int8_t> kq(hv + 1), vq(hv + 1);
            std::vector<float> ks(sc + 1), vs(sc + 1);
            CHK(ornith_hip_session_get_kv(s, l, kq.data(), ks.data(), vq.data(), vs.data()));
            put32(1); put32(pos); put32(a.nkv); put32(a.hd);
            put(kq.data(), hv); put(vq.data(), hv); put(ks.data(), sc * 4); put(vs.data(), sc * 4);
        } else {
            std::vector<float> S((size_t)a.nv * a.dv * a.dk), w((size_t)(a.conv_k - 1) * cc + 1);
            CHK(ornith_hip_session_get_delta(s, l, S.data()));
            CHK(ornith_hip_session_get_conv(s, l, w.data()));
            put(S.data(), S.size() * 4);
            put32(a.conv_k); put32(cc);
            put(w.data(), (size_t)(a.conv_k - 1) * cc * 4);
        }
    }
    put(hist.data(), (size_t)pos * 4);
    if (hl) {
        std::vector<float> lg((size_t)a.vocab);
        CHK(ornith_hip_session_logits(s, lg.data()));
        put(lg.data(), lg.size() * 4);
    }
    FILE *f = fopen(path, "wb");
    if (!f) { seterr("session save: cannot open %s", path); return ORNITH_HIP_ERR_IO; }
    const bool ok = fwrite(out.data(), 1, out.size(), f) == out.size();
    if (fclose(f) != 0 || !ok) { seterr("session save: write to %s failed", path); return ORNITH_HIP_ERR_IO; }
    return ORNITH_HIP_OK;
}

extern "C" int ornith_hip_session_load(ornith_hip_model *m, const char *path, int extra_cap,
                                       ornith_hip_session **out) {
    *out = nullptr;
    const ornith_hip_arch &a = m->a;
    FILE *f = fopen(path, "rb");
    if (!f) { seterr("session load: cannot open %s", path); return ORNITH_HIP_ERR_IO; }
    std::vector<uint8_t> buf;
    {
        uint8_t tmp[1 << 16];
        size_t n;
        while ((n = fread(tmp, 1, sizeof tmp, f)) > 0) buf.insert(buf.end(), tmp, tmp + n);
        fclose(f);
    }
    size_t at = 0;
    auto get = [&](void *p, size_t n) {
        if (at + n > buf.size()) return false;
        memcpy(p, buf.data() + at, n);
        at += n;
        return true;
    };
    char magic[8];
    uint32_t ver = 0;
    if (!get(magic, 8) || memcmp(magic, kSessMagic, 8) != 0) { seterr("session load: not a session file"); return ORNITH_HIP_ERR_FORMAT; }
    if (!get(&ver, 4) || ver != kSessVersion) { seterr("session load: unsupported version"); return ORNITH_HIP_ERR_FORMAT; }
    int32_t fp[13], cur[13];
    sess_fp(a, cur);
    if (!get(fp, sizeof fp)) { seterr("session load: truncated header"); return ORNITH_HIP_ERR_FORMAT; }
    if (memcmp(fp, cur, sizeof fp) != 0) {
        seterr("session load: arch fingerprint mismatch (snapshot is for a different model)");
        return ORNITH_HIP_ERR_FORMAT;
    }
    int32_t pos = 0, nhist = 0, hl = 0;
    uint64_t ph = 0;
    if (!get(&pos, 4) || !get(&nhist, 4) || !get(&ph, 8) || !get(&hl, 4)) { seterr("session load: truncated body"); return ORNITH_HIP_ERR_FORMAT; }
    if (pos < 0 || nhist != pos) {
        seterr("session load: %d history tokens for position %d (this engine keeps one per position)", nhist, pos);
        return ORNITH_HIP_ERR_UNSUPPORTED;
    }
    int cap = pos + (extra_cap > 0 ? extra_cap : 0);
    if (cap < 1) cap = 1;
    ornith_hip_session *s = nullptr;
    CHK(ornith_hip_session_new(m, cap, &s));
    auto fail = [&](int st, const char *msg) { ornith_hip_session_free(s); seterr("session load: %s", msg); return st; };
    const int cc = 2 * a.nk * a.dk + a.nv * a.dv, kc = s->kvcap, hd = a.hd, nkv = a.nkv;
    for (int l = 0; l < a.n_layers; l++) {
        LayerState &z = s->ls[l];
        if (m->L[l].full) {
            int32_t q, len, snkv, shd;
            if (!get(&q, 4) || !get(&len, 4) || !get(&snkv, 4) || !get(&shd, 4)) return fail(ORNITH_HIP_ERR_FORMAT, "truncated/corrupt");
            if (snkv != nkv || shd != hd || len > cap) return fail(ORNITH_HIP_ERR_FORMAT, "truncated/corrupt");
            if (!q) return fail(ORNITH_HIP_ERR_UNSUPPORTED, "an f32 KV cache (this engine keeps the Q8 cache)");
            if (len != pos) return fail(ORNITH_HIP_ERR_UNSUPPORTED, "a KV cache shorter than the position");
            const size_t hv = (size_t)len * nkv * hd, sc = (size_t)len * nkv;
            std::vector<int8_t> kq(hv + 1), vq(hv + 1);
            std::vector<float> ks(sc + 1), vs(sc + 1);
            if (!get(kq.data(), hv) || !get(vq.data(), hv) || !get(ks.data(), sc * 4) || !get(vs.data(), sc * 4))
                return fail(ORNITH_HIP_ERR_FORMAT, "truncated/corrupt");
            // into the device layouts: K words [kvh][hd/4][cap], V tiles [kvh][cap/16][hd][16]
            std::vector<uint32_t> kt((size_t)nkv * (hd / 4) * kc, 0u);
            std::vector<int8_t> vt((size_t)nkv * kc * hd, 0);
            for (int t = 0; t < len; t++)
                for (int h = 0; h < nkv; h++)
                    for (int i = 0; i < hd; i++) {
                        const size_t src = ((size_t)t * nkv + h) * hd + i;
                        kt[((size_t)h * (hd / 4) + i / 4) * kc + t] |= (uint32_t)(uint8_t)kq[src] << (8 * (i & 3));
                        vt[(((size_t)h * (kc / 16) + t / 16) * hd + i) * 16 + (t & 15)] = vq[src];
                    }
            if (hipMemcpy(z.Kt, kt.data(), kt.size() * 4, hipMemcpyHostToDevice) != hipSuccess ||
                hipMemcpy(z.Vq, vt.data(), vt.size(), hipMemcpyHostToDevice) != hipSuccess ||
                (sc && hipMemcpy(z.Ks, ks.data(), sc * 4, hipMemcpyHostToDevice) != hipSuccess) ||
                (sc && hipMemcpy(z.Vs, vs.data(), sc * 4, hipMemcpyHostToDevice) != hipSuccess))
                return fail(ORNITH_HIP_ERR_DEVICE, "upload failed");
        } else {
            const size_t ds = (size_t)a.nv * a.dv * a.dk;
            std::vector<float> S(ds);
            int32_t K, C;
            if (!get(S.data(), ds * 4) || !get(&K, 4) || !get(&C, 4)) return fail(ORNITH_HIP_ERR_FORMAT, "truncated/corrupt");
            if (K != a.conv_k || C != cc) return fail(ORNITH_HIP_ERR_FORMAT, "truncated/corrupt");
            const size_t wsz = (size_t)(K - 1) * C;
            std::vector<float> w(wsz + 1);
            if (!get(w.data(), wsz * 4)) return fail(ORNITH_HIP_ERR_FORMAT, "truncated/corrupt");
            // the window the next step reads lives in parity (pos & 1)
            if (hipMemcpy(z.S, S.data(), ds * 4, hipMemcpyHostToDevice) != hipSuccess ||
                hipMemcpy(z.conv + (size_t)(pos & 1) * wsz, w.data(), wsz * 4, hipMemcpyHostToDevice) != hipSuccess)
                return fail(ORNITH_HIP_ERR_DEVICE, "upload failed");
        }
    }
    std::vector<int32_t> hist((size_t)nhist + 1);
    if (!get(hist.data(), (size_t)nhist * 4)) return fail(ORNITH_HIP_ERR_FORMAT, "truncated/corrupt");
    std::vector<float> lg;
    if (hl) {
        lg.resize((size_t)a.vocab);
        if (!get(lg.data(), lg.size() * 4)) return fail(ORNITH_HIP_ERR_FORMAT, "truncated/corrupt");
    }
    if (sess_prefix_hash(hist.data(), nhist) != ph) return fail(ORNITH_HIP_ERR_FORMAT, "prefix hash mismatch (corrupt snapshot)");
    for (int i = 0; i < nhist; i++)
        if (hist[i] < 0 || hist[i] >= a.vocab) return fail(ORNITH_HIP_ERR_FORMAT, "history token outside the vocabulary");
    if (nhist > 0 && hipMemcpy(s->toks, hist.data(), (size_t)nhist * 4, hipMemcpyHostToDevice) != hipSuccess)
        return fail(ORNITH_HIP_ERR_DEVICE, "upload failed");
    if (hl) {
        // the logits, and their greedy token where the token step's head leaves
        // it (session_generate continues from there)
        hipStream_t st = m->ctx->st;
        if (hipMemcpy(s->logits, lg.data(), lg.size() * 4, hipMemcpyHostToDevice) != hipSuccess ||
            oh_launch_argmax_rows(s->logits, a.vocab, 1, s->toks + pos, st) != hipSuccess ||
            hipStreamSynchronize(st) != hipSuccess)
            return fail(ORNITH_HIP_ERR_DEVICE, "upload failed");
    }
    s->pos = pos;
    s->have_logits = hl != 0;
    *out = s;
    return ORNITH_HIP_OK;
}

// ---- GGUF-order download of a tensor (planes -> GGUF blocks) -------------------------------------
extern "C" int ornith_hip_tensor_download(const ornith_hip_tensor *t, void *out, uint64_t nbytes) {
    if (nbytes != t->gguf_bytes) {
        seterr("tensor '%s': %llu bytes requested, %llu held", t->name.c_str(), (unsigned long long)nbytes,
               (unsigned long long)t->gguf_bytes);
        return ORNITH_HIP_ERR_FORMAT;
    }
    HCHK(hipSetDevice(t->ctx->device));
    size_t a, b, c;
    plane_bytes(t->type, t->rows, t->in, &a, &b, &c);
    if (!oh_is_quant(t->type)) {
        HCHK(hipMemcpy(out, t->A, a, hipMemcpyDeviceToHost));
        return ORNITH_HIP_OK;
    }
    std::vector<uint8_t> h(up256(a) + up256(b) + up256(c));
    HCHK(hipMemcpy(h.data(), t->mem, h.size(), hipMemcpyDeviceToHost));
    const uint8_t *A = h.data(), *B = A + up256(a), *C = B + up256(b);
    uint8_t *o = (uint8_t *)out;
    const size_t nblk = (size_t)t->rows * (size_t)(t->in / 256);
    for (size_t i = 0; i < nblk; i++) {
        switch (t->type) {
        case OH_Q4_K:
            memcpy(o + 144 * i, B + 16 * i, 16);
            for (int k = 0; k < 128; k += 16) memcpy(o + 144 * i + 16 + k, A + oh_a_off(t->type, i, k), 16);
            break;
        case OH_Q6_K:
            for (int k = 0; k < 192; k += 16) memcpy(o + 210 * i + k, A + oh_a_off(t->type, i, k), 16);
            memcpy(o + 210 * i + 192, B + 16 * i, 16);
            memcpy(o + 210 * i + 208, C + 2 * i, 2);
            break;
        case OH_Q8_0:
            for (int k = 0; k < 8; k++) {
                memcpy(o + 272 * i + 34 * k, B + 16 * i + 2 * k, 2);
                memcpy(o + 272 * i + 34 * k + 2, A + oh_a_off(t->type, i, 32 * k), 16);
                memcpy(o + 272 * i + 34 * k + 18, A + oh_a_off(t->type, i, 32 * k + 16), 16);
            }
            break;
        case OH_IQ2_XXS: memcpy(o + 66 * i, C + 2 * i, 2); memcpy(o + 66 * i + 2, A + 64 * i, 64); break;
        }
    }
    return ORNITH_HIP_OK;
}

// ---- on-device random init ----------------------------------------------------------------------
// Stream key of a tensor: FNV-1a of its name xor seed*golden-gamma; element i
// of the stream depends only on (key, i) (counter-based splitmix64).
static uint64_t stream_key(uint64_t seed, const std::string &name) {
    uint64_t h = 0xcbf29ce484222325ull;
    for (unsigned char ch : name) { h ^= ch; h *= 0x100000001b3ull; }
    return h ^ (seed * 0x9E3779B97F4A7C15ull);
}

extern "C" int ornith_hip_model_synth(ornith_hip_ctx *ctx, const ornith_hip_gen_cfg *c,
                                      ornith_hip_model **out) {
    *out = nullptr;
    HCHK(hipSetDevice(ctx->device));
    auto enc_ok = [](uint32_t t) {
        return t == OH_Q8_0 || t == OH_Q4_K || t == OH_Q6_K || t == OH_IQ2_XXS || t == OH_F32;
    };
    if (!enc_ok(c->t_default) || !enc_ok(c->t_attn_v) || !enc_ok(c->t_ffn_down) || !enc_ok(c->t_output) ||
        !enc_ok(c->t_embd) || (c->t_exps && !enc_ok(c->t_exps))) {
        seterr("model_synth: on-device encoders cover F32/Q8_0/Q4_K/Q6_K/IQ2_XXS");
        return ORNITH_HIP_ERR_UNSUPPORTED;
    }
    if (c->hidden <= 0 || c->n_layers <= 0 || c->vocab <= 0 || c->dhead <= 0 || c->conv_k < 2 || c->conv_k > 8) {
        seterr("model_synth: bad config");
        return ORNITH_HIP_ERR_FORMAT;
    }
    const int H = c->hidden, V = c->vocab, qd = c->nk * c->dhead, vd = c->nv * c->dhead, cc = 2 * qd + vd;
    // largest tensor (elements) sizes the f32 staging buffer
    uint64_t mx = (uint64_t)H * V;
    auto upd = [&](uint64_t n) { if (n > mx) mx = n; };
    upd((uint64_t)H * cc); upd((uint64_t)H * 2 * c->nh * c->hd); upd((uint64_t)H * c->moe_inter * c->ne);
    upd((uint64_t)c->nh * c->hd * H); upd((uint64_t)vd * H); upd((uint64_t)H * c->shared_inter);
    float *tmp = nullptr;
    HCHK(hipMalloc(&tmp, mx * 4 + 256));
    auto *m = new ornith_hip_model();
    m->ctx = ctx;
    hipStream_t st = ctx->st;
    int status = ORNITH_HIP_OK;
    auto add_q = [&](const std::string &name, uint32_t type, int nd, uint64_t d0, uint64_t d1, uint64_t d2) {
        if (status) return;
        const uint64_t dims[3] = {d0, d1, d2};
        ornith_hip_tensor *t;
        if ((status = tensor_alloc(ctx, name.c_str(), type, (uint32_t)nd, dims, &t))) return;
        m->ts.push_back(t); m->by[name] = t; m->bytes += t->gguf_bytes;
        const int64_t n = t->rows * t->in;
        float *dst = type == OH_F32 ? (float *)t->A : tmp;
        hipError_t e = oh_launch_fill_gauss(stream_key(c->seed, name), c->sigma, dst, n, st);
        if (e == hipSuccess && type != OH_F32) e = oh_launch_encode(tmp, (int)type, n / 256, t->A, t->B, t->C, st);
        if (e == hipSuccess) e = hipStreamSynchronize(st);   // tmp is reused by the next tensor
        if (e != hipSuccess) { seterr("synth '%s': %s", name.c_str(), hipGetErrorString(e)); status = ORNITH_HIP_ERR_DEVICE; }
    };
    auto add_u = [&](const std::string &name, int nd, uint64_t d0, uint64_t d1, float lo, float hi) {
        if (status) return;
        const uint64_t dims[2] = {d0, d1};
        ornith_hip_tensor *t;
        if ((status = tensor_alloc(ctx, name.c_str(), OH_F32, (uint32_t)nd, dims, &t))) return;
        m->ts.push_back(t); m->by[name] = t; m->bytes += t->gguf_bytes;
        hipError_t e = oh_launch_fill_uniform(stream_key(c->seed, name), lo, hi, (float *)t->A, t->rows * t->in, st);
        if (e != hipSuccess) { seterr("synth '%s': %s", name.c_str(), hipGetErrorString(e)); status = ORNITH_HIP_ERR_DEVICE; }
    };
    // ORNITH_HIP_VERBOSE=1: one line per synthesised layer on stderr (a large
    // model with IQ2_XXS experts takes minutes)
    const char *vb = getenv("ORNITH_HIP_VERBOSE");
    const bool verbose = vb && vb[0] == '1';
    // same tensor set and order as the GGUF generator
    add_q("token_embd.weight", c->t_embd, 2, H, V, 0);
    add_u("output_norm.weight", 1, H, 0, 0.9f, 1.1f);
    add_q("output.weight", c->t_output, 2, H, V, 0);
    for (int l = 0; l < c->n_layers; l++) {
        const bool full = c->full_interval > 0 && l % c->full_interval == c->full_interval - 1;
        const std::string b = "blk." + std::to_string(l) + ".";
        add_u(b + "attn_norm.weight", 1, H, 0, 0.9f, 1.1f);
        add_u(b + "post_attention_norm.weight", 1, H, 0, 0.9f, 1.1f);
        if (full) {
            add_q(b + "attn_q.weight", c->t_default, 2, H, 2 * c->nh * c->hd, 0);
            add_q(b + "attn_k.weight", c->t_default, 2, H, c->nkv * c->hd, 0);
            add_q(b + "attn_v.weight", c->t_attn_v, 2, H, c->nkv * c->hd, 0);
            add_u(b + "attn_q_norm.weight", 1, c->hd, 0, 0.9f, 1.1f);
            add_u(b + "attn_k_norm.weight", 1, c->hd, 0, 0.9f, 1.1f);
            add_q(b + "attn_output.weight", c->t_default, 2, c->nh * c->hd, H, 0);
        } else {
            add_q(b + "attn_qkv.weight", c->t_default, 2, H, cc, 0);
            add_u(b + "ssm_conv1d.weight", 2, c->conv_k, cc, -0.2f, 0.2f);
            add_u(b + "ssm_a", 1, c->nv, 0, -0.8f, -0.2f);
            add_u(b + "ssm_dt.bias", 1, c->nv, 0, -0.05f, 0.05f);
            add_u(b + "ssm_norm.weight", 1, c->dhead, 0, 0.9f, 1.1f);
            add_q(b + "ssm_alpha.weight", c->t_default, 2, H, c->nv, 0);
            add_q(b + "ssm_beta.weight", c->t_default, 2, H, c->nv, 0);
            add_q(b + "attn_gate.weight", c->t_default, 2, H, vd, 0);
            add_q(b + "ssm_out.weight", c->t_default, 2, vd, H, 0);
        }
        if (c->ne <= 0) {
            // dense SwiGLU FFN of width shared_inter
            add_q(b + "ffn_gate.weight", c->t_default, 2, H, c->shared_inter, 0);
            add_q(b + "ffn_up.weight", c->t_default, 2, H, c->shared_inter, 0);
            add_q(b + "ffn_down.weight", c->t_ffn_down, 2, c->shared_inter, H, 0);
            continue;
        }
        add_q(b + "ffn_gate_inp.weight", c->t_default, 2, H, c->ne, 0);
        add_q(b + "ffn_gate_exps.weight", c->t_exps ? c->t_exps : c->t_default, 3, H, c->moe_inter, c->ne);
        add_q(b + "ffn_up_exps.weight", c->t_exps ? c->t_exps : c->t_default, 3, H, c->moe_inter, c->ne);
        add_q(b + "ffn_down_exps.weight", c->t_exps ? c->t_exps : c->t_ffn_down, 3, c->moe_inter, H, c->ne);
        if (c->shared_inter > 0) {
            add_q(b + "ffn_gate_shexp.weight", c->t_default, 2, H, c->shared_inter, 0);
            add_q(b + "ffn_up_shexp.weight", c->t_default, 2, H, c->shared_inter, 0);
            add_q(b + "ffn_down_shexp.weight", c->t_ffn_down, 2, c->shared_inter, H, 0);
            add_q(b + "ffn_gate_inp_shexp.weight", c->t_default, 1, H, 1, 0);
        }
        if (verbose && !status) {
            fprintf(stderr, "model_synth: layer %d/%d done, %.2f GB\n", l + 1, c->n_layers, (double)m->bytes / 1e9);
            fflush(stderr);
        }
    }
    (void)hipStreamSynchronize(st);
    (void)hipFree(tmp);
    if (status) { ornith_hip_model_free(m); return status; }
    Meta md;
    md.arch = "qwen35moe";
    md.u32["qwen35moe.block_count"] = (uint32_t)c->n_layers;
    md.u32["qwen35moe.expert_used_count"] = (uint32_t)c->top_k;
    md.u32["qwen35moe.rope.dimension_count"] = 64;
    md.f32["qwen35moe.rope.freq_base"] = 1e7f;
    md.f32["qwen35moe.attention.layer_norm_rms_epsilon"] = 1e-6f;
    md.has_tokens = true;
    md.eos = -1;
    const int st2 = infer_arch(m, md);
    if (st2) { ornith_hip_model_free(m); return st2; }
    *out = m;
    return ORNITH_HIP_OK;
}

// ---- one eager step with per-launch timing (HIP events around every launch) ------------------------
extern "C" int ornith_hip_session_time_kind(ornith_hip_session *s, int kind, int reps, float *us_per_launch,
                                            double *bytes_per_launch, int *launches_per_step) {
    *us_per_launch = 0.0f;
    *bytes_per_launch = 0.0;
    *launches_per_step = 0;
    if (!s->have_logits) { seterr("session has no logits; eval a prompt first"); return ORNITH_HIP_ERR_FORMAT; }
    if (kind < 0 || reps < 1) { seterr("time_kind: kind %d reps %d", kind, reps); return ORNITH_HIP_ERR_FORMAT; }
    HCHK(hipSetDevice(s->m->ctx->device));
    hipStream_t st = s->m->ctx->st;
    CHK(sync_pos(s));
    HCHK(hipStreamSynchronize(st));
    if (kind == K_STEP_BODY || kind == K_STEP_HEAD) {
        // back-to-back launches of one step-kernel program at the current
        // position (the body does not advance); bytes at this position
        const bool body = kind == K_STEP_BODY;
        CHK(step_prepare(s));
        if (!s->step_grid) { seterr("time_kind: the step kernel is not available"); return ORNITH_HIP_ERR_UNSUPPORTED; }
        Prog P;
        P.step = true;
        P.waves = s->step_grid * 4;
        CHK(body ? build_body(s, P) : build_head(s, P));
        double by = 0.0;
        for (double b : P.bytes) by += b;
        CHK(step_launch(s, body, nullptr, false));
        hipEvent_t a0 = nullptr, a1 = nullptr;
        HCHK(hipEventCreate(&a0));
        HCHK(hipEventCreate(&a1));
        HCHK(hipEventRecord(a0, st));
        for (int i = 0; i < reps; i++) CHK(step_launch(s, body, nullptr, false));
        HCHK(hipEventRecord(a1, st));
        HCHK(hipEventSynchronize(a1));
        float el = 0.0f;
        HCHK(hipEventElapsedTime(&el, a0, a1));
        (void)hipEventDestroy(a0);
        (void)hipEventDestroy(a1);
        CHK(step_check(s));
        *us_per_launch = el * 1000.0f / (float)reps;
        *bytes_per_launch = by;
        *launches_per_step = 1;
        return ORNITH_HIP_OK;
    }
    hipEvent_t e0 = nullptr, e1 = nullptr;
    HCHK(hipEventCreate(&e0));
    HCHK(hipEventCreate(&e1));
    s->only = kind;
    s->only_n = 0;
    s->only_bytes = 0.0;
    int r = enqueue_body(s, st);                   // warm-up pass: counts launches and bytes
    if (r == ORNITH_HIP_OK) r = enqueue_head(s, st);
    const int n = s->only_n;
    const double by = s->only_bytes;
    hipError_t e = hipEventRecord(e0, st);
    for (int i = 0; i < reps && r == ORNITH_HIP_OK && e == hipSuccess; i++) {
        r = enqueue_body(s, st);
        if (r == ORNITH_HIP_OK) r = enqueue_head(s, st);
    }
    if (e == hipSuccess) e = hipEventRecord(e1, st);
    if (e == hipSuccess) e = hipEventSynchronize(e1);
    s->only = -1;
    float el = 0.0f;
    if (r == ORNITH_HIP_OK && e == hipSuccess) e = hipEventElapsedTime(&el, e0, e1);
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    if (r) return r;
    HCHK(e);
    if (n > 0) {
        *us_per_launch = el * 1000.0f / (float)(reps * n);
        *bytes_per_launch = by / n;
    }
    *launches_per_step = n;
    return ORNITH_HIP_OK;
}

extern "C" int ornith_hip_session_profile_step(ornith_hip_session *s, int max_launches, int32_t *kinds,
                                               double *bytes, float *ms, int *n_launches) {
    *n_launches = 0;
    if (!s->have_logits) { seterr("session has no logits; eval a prompt first"); return ORNITH_HIP_ERR_FORMAT; }
    if (s->pos + 1 > s->cap) { seterr("profile_step: session full"); return ORNITH_HIP_ERR_UNSUPPORTED; }
    HCHK(hipSetDevice(s->m->ctx->device));
    hipStream_t st = s->m->ctx->st;
    CHK(sync_pos(s));
    HCHK(hipStreamSynchronize(st));
    s->rec = true;
    s->rec_ev.clear(); s->rec_kind.clear(); s->rec_bytes.clear();
    int r = enqueue_body(s, st);
    if (r == ORNITH_HIP_OK) r = enqueue_head(s, st);
    s->rec = false;
    hipError_t e = hipStreamSynchronize(st);
    const size_t n = s->rec_kind.size();
    if (r == ORNITH_HIP_OK && e == hipSuccess) {
        for (size_t i = 0; i < n && (int)i < max_launches; i++) {
            float el = 0.0f;
            (void)hipEventElapsedTime(&el, s->rec_ev[2 * i], s->rec_ev[2 * i + 1]);
            kinds[i] = s->rec_kind[i];
            bytes[i] = s->rec_bytes[i];
            ms[i] = el;
        }
        *n_launches = (int)(n < (size_t)max_launches ? n : (size_t)max_launches);
        s->pos += 1;
    }
    for (hipEvent_t ev : s->rec_ev) (void)hipEventDestroy(ev);
    s->rec_ev.clear();
    if (r) return r;
    HCHK(e);
    return ORNITH_HIP_OK;
}

// ---- phases of one step-kernel body launch (block 0's clock after each barrier) --------------------
extern "C" int ornith_hip_session_profile_phases(ornith_hip_session *s, int max_phases, int32_t *kinds,
                                                 double *bytes, float *us, int *n_phases) {
    *n_phases = 0;
    if (!s->have_logits) { seterr("session has no logits; eval a prompt first"); return ORNITH_HIP_ERR_FORMAT; }
    HCHK(hipSetDevice(s->m->ctx->device));
    hipStream_t st = s->m->ctx->st;
    CHK(sync_pos(s));
    CHK(step_prepare(s));
    if (!s->step_grid) { seterr("profile_phases: the step kernel is not available"); return ORNITH_HIP_ERR_UNSUPPORTED; }
    if (!s->ts) CHK(salloc(s, &s->ts, (size_t)s->sp_body.n + 8));
    Prog P;
    P.step = true;
    P.waves = s->step_grid * 4;
    CHK(build_body(s, P));
    CHK(step_launch(s, true, nullptr, false));        // warm
    CHK(step_launch(s, true, s->ts, false));
    HCHK(hipStreamSynchronize(st));
    CHK(step_check(s));
    const int n = s->sp_body.n;
    std::vector<uint64_t> t((size_t)n + 1);
    HCHK(hipMemcpy(t.data(), s->ts, t.size() * 8, hipMemcpyDeviceToHost));
    const int m = n < max_phases ? n : max_phases;
    for (int i = 0; i < m; i++) {
        kinds[i] = i < (int)P.rk.size() ? P.rk[i] : -1;
        bytes[i] = i < (int)P.bytes.size() ? P.bytes[i] : 0.0;
        us[i] = (float)((double)(t[i + 1] - t[i]) / 100.0);   // 100 MHz real-time clock
    }
    *n_phases = m;
    return ORNITH_HIP_OK;
}

// One decode launch with clocks (after a warm-up launch; neither advances the
// position): per operation its kind and, over the workgroups, the earliest and
// the latest time it was done (microseconds from the earliest start).
extern "C" int ornith_hip_session_profile_decode(ornith_hip_session *s, int max_ops, int32_t *kinds,
                                                 float *us_first, float *us_last, int *n_ops) {
    *n_ops = 0;
    if (!s->have_logits) { seterr("session has no logits; eval a prompt first"); return ORNITH_HIP_ERR_FORMAT; }
    HCHK(hipSetDevice(s->m->ctx->device));
    hipStream_t st = s->m->ctx->st;
    CHK(sync_pos(s));
    CHK(dec_prepare(s));
    if (!s->dec.grid) { seterr("profile_decode: the decode launch is not available for this model"); return ORNITH_HIP_ERR_UNSUPPORTED; }
    const int G = s->dec.grid, n = s->dec.n;
    if (!s->dec.ts) CHK(salloc(s, &s->dec.ts, (size_t)(n + 1) * G));
    HCHK(oh_launch_decode(s->dec.ops, n, s->io, 0, G, s->dec.lds, st));
    HCHK(oh_launch_decode(s->dec.ops, n, s->io, 0, G, s->dec.lds, st, s->dec.ts));
    HCHK(hipStreamSynchronize(st));
    CHK(step_check(s));
    std::vector<uint64_t> t((size_t)(n + 1) * G);
    HCHK(hipMemcpy(t.data(), s->dec.ts, t.size() * 8, hipMemcpyDeviceToHost));
    uint64_t t0 = t[0];
    for (int b = 1; b < G; b++) t0 = t[b] < t0 ? t[b] : t0;
    const int m = n < max_ops ? n : max_ops;
    for (int i = 0; i < m; i++) {
        uint64_t lo = ~0ull, hi = 0;
        for (int b = 0; b < G; b++) {
            const uint64_t v = t[(size_t)(i + 1) * G + b];
            lo = v < lo ? v : lo;
            hi = v > hi ? v : hi;
        }
        kinds[i] = s->dec.kinds[i];
        us_first[i] = (float)((double)(lo - t0) / 100.0);
        us_last[i] = (float)((double)(hi - t0) / 100.0);
    }
    *n_ops = m;
    return ORNITH_HIP_OK;
}

// Sub-phase clocks of one operation of the decode launch (measurement): per
// workgroup 8 stamps (0 start, 1 weights requested, 2 inputs arrived, 3 the
// activation arrived, 4 prologue done, 5 done; unused ones 0) in microseconds
// from the launch's earliest start, -1 where not recorded. grid_out: workgroups.
extern "C" int ornith_hip_session_profile_decode_op(ornith_hip_session *s, int op, float *us, int max_groups,
                                                    int *grid_out) {
    *grid_out = 0;
    if (!s->have_logits) { seterr("session has no logits; eval a prompt first"); return ORNITH_HIP_ERR_FORMAT; }
    HCHK(hipSetDevice(s->m->ctx->device));
    hipStream_t st = s->m->ctx->st;
    CHK(sync_pos(s));
    CHK(dec_prepare(s));
    if (!s->dec.grid) { seterr("profile_decode_op: the decode launch is not available for this model"); return ORNITH_HIP_ERR_UNSUPPORTED; }
    const int G = s->dec.grid, n = s->dec.n;
    if (op < 0 || op >= n) { seterr("profile_decode_op: operation %d outside [0, %d)", op, n); return ORNITH_HIP_ERR_FORMAT; }
    if (!s->dec.ts) CHK(salloc(s, &s->dec.ts, (size_t)(n + 1) * G));
    uint64_t *ts2 = nullptr;
    CHK(salloc(s, &ts2, (size_t)G * 8));
    HCHK(oh_launch_decode(s->dec.ops, n, s->io, 0, G, s->dec.lds, st));
    HCHK(oh_launch_decode(s->dec.ops, n, s->io, 0, G, s->dec.lds, st, s->dec.ts, op, ts2));
    HCHK(hipStreamSynchronize(st));
    CHK(step_check(s));
    std::vector<uint64_t> t((size_t)G), t2((size_t)G * 8);
    HCHK(hipMemcpy(t.data(), s->dec.ts, (size_t)G * 8, hipMemcpyDeviceToHost));
    HCHK(hipMemcpy(t2.data(), ts2, t2.size() * 8, hipMemcpyDeviceToHost));
    uint64_t t0 = t[0];
    for (int b = 1; b < G; b++) t0 = t[b] < t0 ? t[b] : t0;
    const int m = G < max_groups ? G : max_groups;
    for (int b = 0; b < m; b++)
        for (int k = 0; k < 8; k++) {
            const uint64_t v = t2[(size_t)b * 8 + k];
            us[b * 8 + k] = v == 0 ? -1.0f : (float)((double)(v - t0) / 100.0);
        }
    *grid_out = m;
    return ORNITH_HIP_OK;
}
