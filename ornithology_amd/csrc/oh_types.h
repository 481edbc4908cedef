// oh_types.h - host/device shared descriptors of the HIP engine.
//
// Weights live in HBM in a "plane" layout derived from the GGUF blocks. For a
// tensor of R rows and nb blocks per row (block = 256 elements, or 32 for
// Q8_0 handled as 8 sub-blocks of a 256-element super-block), block b = r*nb+i
// is split into up to three planes so that every wave load is 16-byte aligned
// and contiguous across lanes (A planes of the integer-path types are
// additionally tile-interleaved, see oh_a_off):
//   Q4_K    A: qs[128]            B: d,dmin,scales[12] (16 B)
//   Q6_K    A: ql[128] qh[64]     B: scales[16]          C: d (f16)
//   Q8_0    A: 8 x qs[32]         B: 8 x d (f16)
//   IQ2_XXS A: qs[64]                                     C: d (f16)
//   F32/F16/BF16: A holds the raw row-major values.
// The byte count equals the GGUF byte count (plus the A-plane tile padding);
// decoding a plane-layout block gives the same floats as decoding the GGUF
// block.
//
// Q8_K activations use planes as well: qs[nb*256] int8, d[nb] f32,
// bsums[nb*16] int16 (the 292-byte oq8k_block fields, split).
#pragma once
#include <stdint.h>

#if defined(__HIPCC__)
#define OH_HD __host__ __device__
#else
#define OH_HD
#endif

enum {
    OH_F32 = 0, OH_F16 = 1, OH_Q8_0 = 8, OH_Q4_K = 12, OH_Q6_K = 14,
    OH_IQ2_XXS = 16, OH_BF16 = 30
};

// plane bytes per 256-element super-block
OH_HD static inline int oh_plane_a(uint32_t t) {
    switch (t) { case OH_Q4_K: return 128; case OH_Q6_K: return 192; case OH_Q8_0: return 256;
                 case OH_IQ2_XXS: return 64; default: return 0; }
}
OH_HD static inline int oh_plane_b(uint32_t t) {
    switch (t) { case OH_Q4_K: case OH_Q6_K: case OH_Q8_0: return 16; default: return 0; }
}
OH_HD static inline int oh_plane_c(uint32_t t) {
    switch (t) { case OH_Q6_K: case OH_IQ2_XXS: return 2; default: return 0; }
}
OH_HD static inline int oh_is_quant(uint32_t t) {
    return t == OH_Q4_K || t == OH_Q6_K || t == OH_Q8_0 || t == OH_IQ2_XXS;
}
// The A plane of Q4_K / Q6_K / Q8_0 is tile-interleaved: super-blocks form
// tiles of 64 (bi / 64) and inside a tile the 16-byte piece k of super-block
// j = bi % 64 sits at (k*64 + j)*16. Sixty-four lanes that each load piece k
// of one of 64 consecutive super-blocks then read 1 KB contiguously. The
// plane is padded to whole tiles.
OH_HD static inline int oh_a_tiled(uint32_t t) {
    return t == OH_Q4_K || t == OH_Q6_K || t == OH_Q8_0;
}
OH_HD static inline uint64_t oh_a_off(uint32_t t, uint64_t bi, int byte) {
    const int pb = oh_plane_a(t);
    if (!oh_a_tiled(t)) return bi * (uint64_t)pb + (uint64_t)byte;
    return (bi >> 6) * (uint64_t)(64 * pb) +
           (uint64_t)((((byte >> 4) * 64) + (int)(bi & 63)) * 16 + (byte & 15));
}
// A-plane bytes of nblk super-blocks (tiles rounded up)
OH_HD static inline uint64_t oh_plane_a_bytes(uint32_t t, uint64_t nblk) {
    const uint64_t n = oh_a_tiled(t) ? (nblk + 63) / 64 * 64 : nblk;
    return n * (uint64_t)oh_plane_a(t);
}

// integer Q8_K path exists (reference qdot_can, src/ornith_qdot.c:218-228)
OH_HD static inline int oh_qdot_can(uint32_t t, int64_t in) {
    return in % 256 == 0 && (t == OH_Q4_K || t == OH_Q6_K || t == OH_Q8_0);
}

// One matvec segment of a multi-segment launch. A segment is one weight
// tensor applied in `nsub` slots: slot k uses rows [eidx[k]*rows, +rows) of a
// stacked expert tensor (or the whole tensor when eidx is null), writes
// y + k*ystride and reads its activation at slot offset k*astride.
enum { OH_PRO_Q8K = 0, OH_PRO_NORM = 1, OH_PRO_SWIGLU = 2, OH_PRO_GNORM = 3, OH_PRO_F32 = 4 };
typedef struct {
    const uint8_t *A, *B, *C;      // weight planes (expert 0 for a stacked tensor)
    // pair != 0: a second tensor of the same type and shape (A2/B2/C2, e.g. the
    // up projection next to the gate) is reduced against the same activation
    // and the segment emits silu(W.x) * (W2.x) per row (mode 0)
    const uint8_t *A2, *B2, *C2;
    int pair;
    // activation: OH_PRO_Q8K reads Q8_K planes (and xf for the f32 fallback);
    // OH_PRO_NORM RMS-normalises xf with nw/eps; OH_PRO_SWIGLU forms
    // silu(xf)*xf2; OH_PRO_GNORM RMS-normalises each gdim-element head of xf
    // (sum of squares from xruns: one double per 64-element run) with nw/eps
    // and multiplies by xf2 (= silu(gate)); slot k's run sums start at
    // xruns + k*astride/64; OH_PRO_F32 takes xf as is; all
    // four then quantise to Q8_K inside the block.
    const int8_t *xqs;
    const float *xd;
    const int16_t *xbs;
    const float *xf, *xf2, *nw;
    const double *xruns;
    // runs16: xruns holds one double per 16-element run instead (slot k's at
    // xruns + k*astride/16) and a 64-element run sum is (g0 + g1) + (g2 + g3)
    // of its four
    // OH_PRO_NORM / OH_PRO_SWIGLU: the segment's first block also stores the
    // activation it formed (Q8_K planes and f32) for later launches
    int8_t *oqs;
    float *oqd;
    int16_t *oqb;
    float *oxf;
    float *y;                      // output, row o of slot k -> y[k*ystride + o]
    const int32_t *eidx;           // stacked experts: slot k uses expert eidx[k]
    float eps;
    int pro, gdim, runs16;
    int iq2tree;                   // IQ2_XXS rows summed as a tree (tolerance; else the f32 fallback's order)
    int iq2split;                  // IQ2_XXS fallback rows: adding wave + term-forming waves (else one lane per row)
    // mode 2: y holds 64-bit tagged words, row o's word = (*tagp + 1) << 32 |
    // float bits of the dot (a value that readers in the same launch poll for)
    const int32_t *tagp;
    int type, nb, in, rows, mode;  // mode 0: y = dot, 1: y += dot, 2: tagged word
    int nsub, ystride, astride;
    int adiv;                      // slot k reads the activation of slot k / adiv (0, 1: its own)
    int units;                     // wave work units per slot
    int upw;                       // units per wave
    int bps;                       // blocks per slot
    int block0;                    // first block of the segment in the launch
} oh_mvseg;

#define OH_MAX_SEGS 8
// kernel variant of a launch whose segments are all integer-path Q4_K and Q6_K
// ones (the others: the segment type, or -1 for any mix)
#define OH_MV_Q4Q6 (-2)
// the graph step's two-launch exact attention takes at most this many query
// heads per KV head
#define OH_EXACT2_GMAX 32
// blocks used by the argmax's first stage (the caller sizes its scratch)
#define OH_ARGMAX_BLOCKS 256
// IQ2_XXS rows of the f32 fallback per 256-thread block: one lane per row,
// or (segment flag iq2split) a lane of the adding wave per row with three
// waves forming the terms
#define OH_IQ2_ROWS_LANE 256
#define OH_IQ2_ROWS 64
#define OH_MV_WAVES 4              // waves per matvec block
#define OH_MV_R 4                  // steps per prefetch batch of a wave
// Fused MoE down projection + combine (one block per row range, every slot).
typedef struct {
    const uint8_t *A, *B, *C;      // stacked down experts
    const uint8_t *sA, *sB, *sC;   // shared-expert down (sA null: none)
    const int32_t *eidx;
    const float *w;                // routing weights [k]
    const float *shg;              // sigmoid shared gate (null: ungated)
    const float *h;                // silu(gate)*up of routed slot k at +k*stride
    const float *hsh;              // silu(gate)*up of the shared expert
    float *x;                      // residual, += combine
    // several tokens (grid y = token t): h + t*hts, hsh + t*hsts, x + t*xts,
    // eidx / w + t*k, shg + t
    size_t hts, hsts, xts;
    // split form (step kernel): a virtual block is (row group, group of 4
    // slots); slot dots go to dots[slot*rows + row], the last block of a row
    // group (counted in cnt[row group]) combines
    float *dots;
    int *cnt;
    int type, nb, in, rows, k, stride;
    // narrow form (stand-alone token-step launch): a block owns 16 / nb rows
    // and every slot (oh_k_mv_down_narrow, 64 * ceil(slots / 4) threads)
    int narrow;
} oh_mvdown;

// A launch with `route` set first routes the MoE in every block: top-k over
// the ne router logits rlog (plus the shared-expert gate logit shl, when
// non-null); stacked segments then use the routed experts, and block 0 stores
// the routing (ridx, rw, shg) for later launches. tslots > 0 (several tokens):
// stacked slot k belongs to token k / tslots and is its expert k % tslots;
// only stacked-segment blocks route (their token's logits at rlog + t*ne,
// shl + t), and the first block of a token's first slot stores its routing
// at ridx + t*topk, rw + t*topk, shg + t.
// rtag (one token): the router logits come from this launch's own router
// segments (mode 2, before the stacked ones): ne tagged words, then the
// shared-expert gate logit's word when rsh is set. A stacked segment's block
// forms its activation first, then polls the words until they carry this
// step's tag (rio[OH_IO_SERIAL] + 1), routes and only then requests its
// expert's weights; rlg is the LDS byte offset of the logits' copy for the
// sequential selection (NaN / -inf logits), past the activation.
typedef struct {
    oh_mvseg s[OH_MAX_SEGS];
    int n;
    int total_blocks;
    int route;
    const float *rlog, *shl;
    int ne, topk;
    int32_t *ridx;
    float *rw, *shg;
    int tslots;
    const uint64_t *rtag;
    int32_t *rio;
    int rsh, rlg;
    // mctr[parity] (parity = the step serial's low bit) counts the router
    // segments' blocks (nrb of them) whose tagged words are stored; a gate/up
    // block polls it, then reads the words once. The first gate/up block
    // (pb0) clears the other parity's counter for the next step. (A replay
    // of one kind's launches for timing zeroes both counters before each
    // pass, so its blocks wait as in a decode step.)
    int32_t *mctr;
    int nrb, pb0;
} oh_mvlaunch;


// ---- operations of the token step -------------------------------------------
// The decode step is a fixed list of operations. Each one runs either as its
// own kernel launch (captured into a HIP graph) or as one phase of the
// persistent step kernel, where grid barriers separate consecutive phases. An
// operation is split into nvb virtual blocks of 256 threads (one wave for the
// delta step); the current position is read from device memory at the start
// of each kernel.
enum {
    OH_OP_MV = 0,          // u.mv, kernel variant tk
    OH_OP_MV_DOWN,         // u.down
    OH_OP_EMBED,           // u.embed
    OH_OP_DELTA,           // u.delta (64 rows per virtual block, one wave; 64-row run sums)
    OH_OP_DELTA16,         // u.delta (16 rows per 256-thread virtual block; 16-row run partials)
    OH_OP_ATTN_PREP,       // u.prep
    OH_OP_ATTN_MAIN,       // u.attn: the exact walk, or flash chunks past its limit
    OH_OP_ATTN_COMBINE,    // u.attn: merge of the flash chunks
    OH_OP_MOE_COMBINE,     // u.comb
    OH_OP_ARGMAX1,         // u.am
    OH_OP_ARGMAX2,         // u.am
    OH_OP_ATTN_SCORES,     // u.attn: the exact walk's scores (the graph step's exact regime)
    OH_OP_ATTN_WALK,       // u.attn: the exact walk's softmax and output (the graph step's exact regime)
    OH_OP_DELTA_MV,        // u.dmv: the delta step and the projection of its output in one launch
    OH_OP_COUNT
};

typedef struct {
    const uint8_t *A, *B, *C;
    const int32_t *toks;
    float *x;
    int type, in;
} oh_op_embed;

typedef struct {
    const float *cat, *ab, *gate, *conv_w, *ssm_a, *dt_bias;
    float *conv_state, *S, *out, *out_gate;
    double *out_runs;
    int dk, nk, nv, K, cc;
    float out_scale;
} oh_op_delta;

typedef struct {
    const float *qproj, *kin, *vin, *q_norm, *k_norm;
    const float *rope;             // (cos, sin) per (position, pair)
    float *qr, *gate;
    uint32_t *Kt;
    float *Ks;
    int8_t *Vq;
    float *Vs;
    int nh, nkv, hd, rot, cap;
    float eps;
    uint16_t *Vh;                  // the V codes again as f16 bits, same tiles (optional)
} oh_op_prep;

// GQA scores / ordered output / flash chunks / flash merge
typedef struct {
    const float *qr, *gate;
    const uint32_t *Kt;
    const float *Ks;
    const int8_t *Vq;
    const float *Vs;
    float *scores, *part_o, *part_ml, *out;
    int nh, nkv, hd, cap, exact_max, hb;
    float scale;
    const uint16_t *Vh;            // the V codes as f16 bits (the graph step's exact walk)
} oh_op_attn;

typedef struct {
    float *x;
    const float *o, *w, *so, *shgate;
    int k, H;
} oh_op_combine;

typedef struct {
    const float *v;
    float *bv;
    int *bi;
    int n, nblk;
    int32_t *toks, *best;
} oh_op_argmax;

// The graph step's delta step and its output projection in one launch:
// workgroups [0, nd) run the delta step (16 state rows each) and add 1 to
// *arr once their outputs are stored; the projection's workgroups (the rest)
// request their first weights, wait (bounded) until *arr reaches nd, form
// the gated RMSNorm of the delta output, reduce, and at the end add 1 to
// *dep. The last of them (*dep reaching the projection's workgroup count)
// sets both counters back to 0, so every launch (replays for timing
// included) starts from zero.
typedef struct {
    oh_mvlaunch mv;
    oh_op_delta d;
    int32_t *arr, *dep;
    int nd;
} oh_op_dmv;

typedef struct {
    int kind, nvb;
    int tk;                // OH_OP_MV: OH_Q4_K / OH_Q6_K / OH_Q8_0, or -1 (mixed)
    int lds;               // dynamic LDS bytes of a standalone launch
    union {
        oh_mvlaunch mv;
        oh_mvdown down;
        oh_op_embed embed;
        oh_op_delta delta;
        oh_op_prep prep;
        oh_op_attn attn;
        oh_op_combine comb;
        oh_op_argmax am;
        oh_op_dmv dmv;
    } u;
} oh_op;

// Persistent step kernel: counters of one program phase (one per 64-byte
// line, OH_STEP_NCTR of them) and the io words it uses.
#define OH_STEP_NCTR 32
#define OH_STEP_CSTRIDE 16
enum { OH_IO_POS = 0, OH_IO_BEST = 1, OH_IO_EPOCH_BODY = 2, OH_IO_EPOCH_HEAD = 3, OH_IO_ERR = 4 };
// bits of io[OH_IO_ERR]: a bounded wait between workgroups gave up (the
// persistent kernels); an expert pair list would have overflowed
enum { OH_ERR_WAIT = 1, OH_ERR_EXPERT_LIST = 2 };

// Batched matvec (prefill): Y[col] = W . X[col] for many activation columns,
// the same integer dot per (row, column) as the matvec. Columns are dense
// [0, ncol) with activation index c and output index c, or grouped: group g
// (blockIdx.y; stacked expert g) has cnt[g] columns list[g*lstride + j] = p,
// activation index p / adiv, output index p. Activation index a: Q8_K planes
// xqs + a*in, xd + a*nb, xbs + a*nb*16. Output row o of column index p at
// y[p*ystride + o] (mode 1: +=). pair: W2 reduced too, emitting silu(W.x)*(W2.x).
typedef struct {
    const uint8_t *A, *B, *C, *A2, *B2, *C2;
    const int8_t *xqs;
    const float *xd;
    const int16_t *xbs;
    float *y;
    const int32_t *cnt, *list;
    int type, nb, in, rows, pair, mode;
    int ncol, lstride, adiv, ystride;
    int tcol;                      // columns staged in LDS at a time
    int cpb;                       // dense: columns per block along grid y (0: all)
} oh_mvbatch;

// Q4_K / Q6_K x Q8_K products of T columns on the matrix cores (prompt path): the
// same (dense | grouped) column addressing as oh_mvbatch; with A2/B2 the
// second weight set writes rows [rows, 2 rows) of each output row.
typedef struct {
    const uint8_t *A, *B, *A2, *B2;   // Q4_K / Q6_K planes (expert 0 of a stack)
    const uint8_t *C, *C2;            // Q6_K: d (f16) per super-block
    int type;                         // OH_Q4_K or OH_Q6_K
    const int8_t *xqs;                // Q8_K activation planes [a][in], [a][nb], [a][nb][16]
    const float *xd;
    const int8_t *xbp;                // per super-block: bytes bl_j, then bh_j, of the pair sums 64*bh + bl
    float *y;                         // y[p * ystride + row]
    const int32_t *cnt, *list;        // grouped columns (list != NULL)
    const int32_t *items;             // grouped: count, then (group << 16 | 64-column tile)
    int nb, in, rows, mode;           // mode 1: y += product
    int ncol, lstride, adiv, ystride;
} oh_mmq;

// ---- the decode step as one persistent launch (oh_decode.hip) ----------------
// Values that one workgroup hands to others travel as tagged words: 64 bits,
// the low 32 the value (a float's bits), the high 32 the step's tag (a
// per-session launch counter, never 0). Every operation writes its own region
// of the session's word arena, so a reader waits for exactly the words it
// needs until their tag is the current one; no barrier and no counter. Bulk
// outputs (attention partials, KV append) use plain device-scope stores
// followed by one tagged flag word per writing workgroup.
enum {
    OH_D_EMBED = 0,    // u.emb: token row -> tagged x
    OH_D_MV,           // u.mv: multi-segment matvec with prologue (+ routing, + argmax partials)
    OH_D_DELTA,        // u.dl: gated delta-net step, one workgroup per value head
    OH_D_PREP,         // u.at: q/k norm + RoPE + KV append (flags)
    OH_D_ATTN,         // u.at: exact walk (o + flags) or flash chunks (partials + flags)
    OH_D_COMBINE,      // u.at: merge of the flash chunks (o + flags)
    OH_D_DOWN,         // u.dn: MoE down projection + combine (routing recomputed)
    OH_D_ARGMAX,       // u.am: greedy token from the lm_head's per-workgroup partials
    OH_D_COUNT
};
#define OH_D_MAXSEG 6
typedef struct {
    const uint8_t *A, *B, *C, *A2, *B2, *C2;
    uint64_t *y;            // tagged output: slot k, row r at y[k * ystride + r]
    float *yp;              // optional plain copy of the output (logits)
    int type, pair, rows, nsub, ystride, stacked, mode;   // mode 1: y = xres[r] + dot
    int units;              // wave steps per slot (ceil(rows / (64 / nb)))
    int step0;              // the segment's first step in the operation
} oh_dseg;
typedef struct {
    const uint64_t *x;      // tagged activation [in]
    const float *xp;        // or a plain activation (flag-gated, pro F32)
    const uint64_t *xflags; // flags gating xp: nflags words
    int nflags_ex, nflags_fl;   // flags to wait for: exact-walk / flash contexts
    const float *nw;        // RMSNorm weight (pro NORM)
    const uint64_t *xres;   // tagged residual for mode-1 segments
    const uint64_t *rlog, *shl;   // routing: tagged router logits [ne], shared-gate logit
    uint64_t *amax;         // head: tagged (value, index) of each workgroup's best row [G][2]
    int pro, in, nb, nseg, nsteps, spw, route, ne, topk, exact_lim;
    int wave0;              // the operation's steps go to the grid's waves from wave0 on
    int wspec;              // 1: wave 0 of a workgroup forms the inputs, waves 1-3 take the steps
    float eps;
    oh_dseg s[OH_D_MAXSEG];
} oh_dmv;
typedef struct {
    const uint8_t *A, *B, *C;
    const int32_t *toks;
    uint64_t *x;
    int type, in;
} oh_demb;
typedef struct {
    const uint64_t *cat, *ab, *z;          // tagged: qkv projection [cc], alpha|beta [2 nv], gate [nv dv]
    const float *conv_w, *ssm_a, *dt_bias, *norm_w;
    float *conv_state, *S;
    uint64_t *o;                           // tagged gated-normed output [nv dv]
    int dk, nk, nv, K, cc;
    float out_scale, eps;
} oh_ddelta;
typedef struct {
    oh_op_prep p;                          // prep (qproj/kin/vin unused: the tagged inputs below)
    oh_op_attn a;                          // attention / combine
    const uint64_t *qkv;                   // tagged: q projection [nh 2hd] | k [nkv hd] | v [nkv hd]
    uint64_t *flags;                       // this operation's flag per workgroup
    const uint64_t *wflags;                // flags waited for
    int nwait_ex, nwait_fl;                // ... at exact-walk / flash contexts
    int lim;                               // exact-walk limit
} oh_datt;
typedef struct {
    const uint8_t *A, *B, *C, *sA, *sB, *sC;
    const uint64_t *h;                     // tagged silu(gate)*up: slot j at j * I, shared at k * I
    const uint64_t *rlog, *shl;            // tagged router logits (routing recomputed)
    const uint64_t *xres;                  // tagged residual [H]
    uint64_t *y;                           // tagged output [H]
    int type, nb, in, rows, k, ne, rpb;    // rpb: rows per workgroup
} oh_ddown;
typedef struct {
    const uint64_t *amax;                  // [nparts][2]
    int nparts, vocab;
    int32_t *toks;                         // the greedy token goes to toks[pos + 1]
} oh_dargmax;
typedef struct {
    int kind, nvb;
    union {
        oh_demb emb;
        oh_dmv mv;
        oh_ddelta dl;
        oh_datt at;
        oh_ddown dn;
        oh_dargmax am;
    } u;
} oh_dop;
// io words of the decode launch (after the step kernel's); OH_IO_SERIAL: the
// session's step count (advanced with the position by every token step,
// never reset), the tag source of in-launch hand-offs
enum { OH_IO_TAG = 8, OH_IO_DONE = 9, OH_IO_SERIAL = 10 };
