// oh_engine.h - internal header of the engine's host side: the shared
// types (context, tensors, model, session, launch builders), error
// macros and the functions the host source files call across files.
// Not part of the C ABI (include/ornith_hip.h).
//
// Reference: src/ornith_rforward.c (rmodel_* / rsession_*), src/ornith_gguf_write.c
// (GGUF v3 layout), src/ornith_model.h (arch).
#pragma once
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

// ---- the no-allocation matvec's scratch --------------------------------------------
// ornith_hip_matvec_noalloc stages its input, output and Q8_K planes in a
// fixed device array (`scratch`, oh_engine.cpp) instead of allocating. Each
// device holds its own copy until the process ends. In host code `scratch`
// only names the symbol: kernels and copies get the device address that
// hipGetSymbolAddress returns for the current device, resolved once per
// device by ornith_hip_init into g_scratch_dev.
#define OH_NOALLOC_SCRATCH_BYTES (4u << 20)
#define OH_MAX_DEVICES 64
// each device's address of the no-allocation scratch array (set by ornith_hip_init)
extern void *g_scratch_dev[OH_MAX_DEVICES];

void seterr(const char *fmt, ...);
#define LAUNCH(kind, bytes, call)                  \
    do {                                           \
        if (keep(s, (kind), (bytes))) {            \
            CHK(rec_begin(s, st));                 \
            HCHK(call);                            \
            CHK(rec_end(s, st, kind, bytes));      \
        }                                          \
    } while (0)


// ---- context -----------------------------------------------------------------------
struct ornith_hip_ctx {
    int device = 0;
    hipStream_t st = nullptr;
    void *scratch = nullptr;
    size_t scratch_bytes = 0;
};

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
    // Q4_K / Q6_K prompt tiles (the matrix-core prompt kernels' copy of A and
    // B, in 64-row tiles), built on the tensor's first such launch
    mutable uint8_t *pmem = nullptr, *PA = nullptr, *PB = nullptr;
};

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
    bool any_full = false;        // a full-attention (GQA) layer exists
    ornith_hip_tensor *embd = nullptr, *out_norm = nullptr, *lm_head = nullptr;
    uint64_t bytes = 0;
};

// metadata view shared by the GGUF and synthetic paths
struct Meta {
    std::string arch = "qwen35";
    std::unordered_map<std::string, uint32_t> u32;
    std::unordered_map<std::string, float> f32;
    bool has_tokens = false;
    int32_t eos = -1;
};

// ---- sessions -----------------------------------------------------------------------------
// Q8_K planes; bp: per super-block the pair-sum bytes of the matrix-core
// product's min term
struct Q8Buf { int8_t *qs = nullptr; float *d = nullptr; int16_t *bs = nullptr; int8_t *bp = nullptr; };

struct LayerState {
    float *S = nullptr, *conv = nullptr;                 // linear
    uint32_t *Kt = nullptr; float *Ks = nullptr;         // full (Q8 KV)
    int8_t *Vq = nullptr; float *Vs = nullptr;
    uint16_t *Vh = nullptr;       // the V codes as f16 bits in the same tiles (the exact walk's operand)
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
    uint64_t *rtag = nullptr;     // MoE layers: router logits as tagged words [n_layers][ne + 1] (fused router)
    int32_t *mctr = nullptr;      // MoE layers: router completion counters of the fused MoE launch [n_layers][2]
    int32_t *dmctr = nullptr;     // delta-net layers: arrival and departure counters of the delta-step launch [n_layers][2]
    // decode contexts up to this (at most the walk's cap for the head dim:
    // 8192 positions at hd 256) take the attention sum in the reference's
    // order; longer ones the flash chunks
    int exact_max = 8192;
    int pf_exact_max = 1024;      // prompt rows up to this context take the exact row walk
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
    hipGraphExec_t gbody_x = nullptr;   // the body graph of the exact-attention regime
    int qpos = 0;                       // position of the next body launch (host side)
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
       K_ATTN_WALK, K_ROUTE, K_COMBINE, K_ARGMAX, K_ADVANCE, K_MV_DOWN, K_ATTN_FLASH, K_ATTN_COMBINE,
       K_MATVEC_Q6K, K_MATVEC_Q80, K_MATVEC_MIXED, K_STEP_BODY, K_STEP_HEAD, K_ATTN_MAIN, K_MATVEC_Q4Q6,
       K_DELTA_MV };

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

// ---- layer-major prefill (src/ornith_rforward.c:647-682 structure) ----------------------
// Every layer over a chunk of tokens before the next: batched matvecs for the
// projections (weights read once per chunk), the conv / delta state / KV cache
// advanced in token order with the decode step's arithmetic. Bit-identical to
// the same tokens fed through the token step.
static const int kPfChunk = 4096, kPfAttnSub = 32;

// Q4_K projections with whole 128-row tiles over at least 64 tokens run on
// the matrix cores; fewer columns (batch decode) stay on the vector-ALU kernel,
// whose whole reduction is in flight at once
static const int kMmqMinTokens = 64;

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

// ---- host functions shared across the engine's source files ----
void seterr(const char *fmt, ...);
int ctx_scratch(ornith_hip_ctx *c, size_t bytes, void **out);
int noalloc_setup(int device);
size_t elem_block(uint32_t t, size_t *bytes);
uint64_t gguf_nbytes(uint32_t t, uint64_t n);
size_t up256(size_t x);
void plane_bytes(uint32_t t, int64_t rows, int64_t in, size_t *a, size_t *b, size_t *c);
void repack(uint32_t t, const uint8_t *src, size_t nblk, uint8_t *A, uint8_t *B, uint8_t *C);
int tensor_alloc(ornith_hip_ctx *ctx, const char *name, uint32_t type, uint32_t nd,
                        const uint64_t *dims, ornith_hip_tensor **out);
bool iq2_tree_on();
bool iq2_tree_can(uint32_t type, int64_t in);
bool seg_q8(const oh_mvseg &s);
bool seg_steps(const oh_mvseg &s);
int mv_add(MvBuild &b, const ornith_hip_tensor *W, const Act &act, float *y, int mode,
                  const int32_t *eidx = nullptr, int nsub = 1, int ystride = 0, int astride = 0);
bool pairable(const ornith_hip_tensor *W, const ornith_hip_tensor *W2);
int mv_add_pair(MvBuild &b, const ornith_hip_tensor *W, const ornith_hip_tensor *W2, const Act &act,
                       float *y, const int32_t *eidx = nullptr, int nsub = 1, int ystride = 0);
// Lay a launch's segments out over blocks for about `waves` waves; with
// small_waves > 0, launches of at most 4 * waves wave steps are laid out for
// small_waves instead.
void mv_plan(MvBuild &b, int waves = 4096, int small_waves = 0);
int mv_go(MvBuild &b, hipStream_t st);
bool mmq_enabled();
// The prompt tiles of a Q4_K / Q6_K tensor (PA, PB), built once on stream st
// and waited for; a no-op when they exist
int mmq_tiles(const ornith_hip_tensor *W, hipStream_t st);
size_t matvec_col_bytes(int64_t in, int64_t out);
int matvec_cols(ornith_hip_ctx *ctx, const ornith_hip_tensor *W, const float *x, float *y, int Tn,
                       void *sp);
ornith_hip_tensor *mt(const ornith_hip_model *m, const std::string &n);
ornith_hip_tensor *mb(const ornith_hip_model *m, int l, const char *sfx);
bool is_full(const ornith_hip_arch &a, int l);
int infer_arch(ornith_hip_model *m, const Meta &md);
int rec_begin(ornith_hip_session *s, hipStream_t st);
int rec_end(ornith_hip_session *s, hipStream_t st, int kind, double bytes);
bool keep(ornith_hip_session *s, int kind, double bytes);
int mv_kind(int tk);
oh_op op_new(int kind, int nvb, int lds = 0);
void prog_add(Prog &P, const oh_op &o, int rk, double bytes);
void prog_mv(Prog &P, MvBuild &b);
int q8alloc(ornith_hip_session *s, Q8Buf &q, size_t n);
Act act_of(const Q8Buf &q, const float *xf);
Act act_norm(const float *x, const float *w, float eps);
Act act_gnorm(const float *o, const float *sz, const double *runs, const float *w, float eps, int gdim,
                     int runs16 = 0);
Act act_swiglu(const float *g, const float *u);
double norm_bytes(int n, bool w);
int build_body(ornith_hip_session *s, Prog &P);
int build_head(ornith_hip_session *s, Prog &P);
int run_prog(ornith_hip_session *s, const Prog &P, hipStream_t st);
int enqueue_body(ornith_hip_session *s, hipStream_t st);
int enqueue_head(ornith_hip_session *s, hipStream_t st);
bool step_enabled();
int step_upload(ornith_hip_session *s, const Prog &P, ornith_hip_session::StepProg &sp);
int step_prepare(ornith_hip_session *s);
int step_launch(ornith_hip_session *s, bool body, uint64_t *ts, bool advance = true);
int step_check(ornith_hip_session *s);
bool dec_enabled();
bool dq(const ornith_hip_tensor *W);
oh_dmv dmv_new(const uint64_t *x, const float *nw, int pro, int in, float eps);
void dmv_seg(oh_dmv &M, const ornith_hip_tensor *W, const ornith_hip_tensor *W2, uint64_t *y, int nsub,
                    int ystride, int stacked, int mode, float *yp = nullptr);
bool dmv_ok(const oh_dmv &M);
bool dmv_add(DecB &b, oh_dmv &M, int wave0, int waves, double bytes);
double wbytes(const ornith_hip_tensor *W, int rows);
bool dec_build(ornith_hip_session *s, DecB &b);
int dec_prepare(ornith_hip_session *s);
int dec_launch(ornith_hip_session *s, bool advance = true);
int capture(ornith_hip_session *s, int (*fn)(ornith_hip_session *, hipStream_t), hipGraphExec_t *out);
bool graphs_enabled();
int run_body(ornith_hip_session *s);
int run_head(ornith_hip_session *s);
int run_step(ornith_hip_session *s);
int sync_pos(ornith_hip_session *s);
// the next body launch takes the exact-attention program
bool body_exact(const ornith_hip_session *s);
bool attn_mfma_enabled();
bool batch_fused();
bool router_fused();
bool delta_fused();
bool delta_mfma_enabled();
int pf_chunk_tokens();
bool pf_mvb_ok(const ornith_hip_tensor *W);
bool pf_moe_grouped(const OhLayer &y);
bool pf_moe_slots_ok(const OhLayer &y);
bool pf_supported(const ornith_hip_model *m);
int pf_alloc(ornith_hip_session *s, int tc);
int pf_mvb(const ornith_hip_tensor *W, const ornith_hip_tensor *W2, const Q8Buf &x, float *y, int ystride,
                  int T, int mode, hipStream_t st, const int32_t *cnt = nullptr, const int32_t *list = nullptr,
                  int lstride = 0, int adiv = 1, int groups = 1);
bool pf_use_mmq(const ornith_hip_tensor *W, bool grouped, int T);
int pf_tiles(const ornith_hip_model *m, hipStream_t st);
int pf_mmq(const ornith_hip_tensor *W, const ornith_hip_tensor *W2, const Q8Buf &x, float *y, int ystride,
                  int T, int mode, hipStream_t st, const int32_t *cnt = nullptr, const int32_t *list = nullptr,
                  int lstride = 0, int adiv = 1, const int32_t *items = nullptr, int max_items = 0);
int pf_mm(const ornith_hip_tensor *W, const Q8Buf &x, float *y, int ystride, int T, int mode,
                 hipStream_t st);
int pf_swiglu(const ornith_hip_tensor *Wg, const ornith_hip_tensor *Wu, const Q8Buf &x, int I, int npairs,
                     int T, Q8Buf &hq, float *gu, float *hbuf, hipStream_t st, const int32_t *cnt = nullptr,
                     const int32_t *list = nullptr, int lstride = 0, int adiv = 1, int groups = 1,
                     const int32_t *items = nullptr, int max_items = 0);
int pf_chunk(ornith_hip_session *s, int base, int T, bool chunked, hipStream_t st);
bool pf_enabled();
bool prefill_serial();
int session_eval(ornith_hip_session *s, const int32_t *tokens, int n, bool token_path);
int bw_alloc(ornith_hip_session *s, int n, size_t ops_bytes);
bool owns(const ornith_hip_session *s, const void *p, size_t bytes);
std::string batch_check(ornith_hip_session *const *ss, int n, const std::vector<size_t> &lofs,
                               const uint8_t *host, int nvb_main, int lds_main);
int batch_enqueue(const BatchPlan &B, hipStream_t st);
void sess_fp(const ornith_hip_arch &a, int32_t fp[13]);
uint64_t sess_prefix_hash(const int32_t *t, int n);
uint64_t stream_key(uint64_t seed, const std::string &name);
