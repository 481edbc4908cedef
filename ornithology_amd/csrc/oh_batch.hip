// Decode of several sessions of one model in one pass: the decode step's own
// operation bodies, one grid row (blockIdx.y) per session, each with its own
// descriptor (its state, KV cache, buffers) and position. The projections of
// such a step run on the batched kernels (weights read once for all sessions).

template <int DK, int KMAX>
__global__ void __launch_bounds__(64) oh_k_delta_batch(const oh_op_delta *ops, const int32_t *pos) {
    __shared__ __align__(16) float lds[2 * DK + 64 * (DK + 4)];
    NoWait w;
    const int b = (int)blockIdx.y;
    delta_body<DK, KMAX>(ops[b], (int)blockIdx.x, pos[b], lds, w);
}

extern "C" __global__ void __launch_bounds__(256) oh_k_prep_batch(const oh_op_prep *ops, const int32_t *pos) {
    NoWait w;
    const int b = (int)blockIdx.y;
    prep_body(ops[b], (int)blockIdx.x, pos[b], w);
}

extern "C" __global__ void __launch_bounds__(256) oh_k_attn_main_batch(const oh_op_attn *ops, const int32_t *pos) {
    NoWait w;
    const int b = (int)blockIdx.y;
    attn_main_body(ops[b], (int)blockIdx.x, pos[b], w);
}

extern "C" __global__ void __launch_bounds__(256) oh_k_attn_combine_batch(const oh_op_attn *ops, const int32_t *pos) {
    NoWait w;
    const int b = (int)blockIdx.y;
    combine_body(ops[b], (int)blockIdx.x, pos[b], w, exact_lim(ops[b].exact_max, ops[b].hd));
}

// greedy token of each of the rows of v [rows][n]: the largest value, the
// lowest index among equals, NaN never chosen (0 if nothing compares), as the
// decode step's two-stage argmax
extern "C" __global__ void __launch_bounds__(256) oh_k_argmax_rows(const float *v, int n, int32_t *out) {
    __shared__ float sv[4];
    __shared__ int si[4];
    const float *vr = v + (size_t)blockIdx.x * n;
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int i = tid_x(); i < n; i += 256) {
        const float x = ldg(vr + i);
        if (x > bv || (x == bv && i < bi)) { bv = x; bi = i; }
    }
    for (int m = 32; m >= 1; m >>= 1) {
        const float ov = shfl_xor(bv, m); const int oi = shfl_xor(bi, m);
        if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
    }
    if (lane_id() == 0) { sv[tid_x() >> 6] = bv; si[tid_x() >> 6] = bi; }
    __syncthreads();
    if (tid_x() == 0) {
        bv = sv[0]; bi = si[0];
        for (int k = 1; k < 4; k++) if (sv[k] > bv || (sv[k] == bv && si[k] < bi)) { bv = sv[k]; bi = si[k]; }
        stg(out + blockIdx.x, bi == 0x7fffffff ? 0 : bi);
    }
}

// the same greedy token per row in two stages (the token step's head): stage
// 1 takes the best of one slice of a row (grid: OH_ARGMAX_BLOCKS x rows, the
// token step's argmax1), stage 2 one wave per row over the slices' bests
extern "C" __global__ void __launch_bounds__(256)
oh_k_argmax_rows1(const float *v, int n, float *bv, int *bi) {
    NoWait w;
    oh_op_argmax a;
    a.v = v + (size_t)blockIdx.y * n;
    a.bv = bv + (size_t)blockIdx.y * OH_ARGMAX_BLOCKS;
    a.bi = bi + (size_t)blockIdx.y * OH_ARGMAX_BLOCKS;
    a.n = n;
    a.nblk = OH_ARGMAX_BLOCKS;
    argmax1_body(a, (int)blockIdx.x, w);
}
extern "C" __global__ void __launch_bounds__(64)
oh_k_argmax_rows2(const float *bv, const int *bi, int32_t *out) {
    const float *rv = bv + (size_t)blockIdx.x * OH_ARGMAX_BLOCKS;
    const int *ri = bi + (size_t)blockIdx.x * OH_ARGMAX_BLOCKS;
    float b = -INFINITY;
    int k = 0x7fffffff;
    for (int i = tid_x(); i < OH_ARGMAX_BLOCKS; i += 64) {
        const float x = ldg(rv + i);
        const int xi = ldg(ri + i);
        if (x > b || (x == b && xi < k)) { b = x; k = xi; }
    }
    for (int m = 32; m >= 1; m >>= 1) {
        const float ov = shfl_xor(b, m); const int oi = shfl_xor(k, m);
        if (ov > b || (ov == b && oi < k)) { b = ov; k = oi; }
    }
    if (tid_x() == 0) stg(out + blockIdx.x, k == 0x7fffffff ? 0 : k);
}

// each session's token history: this step's token at its position and the
// greedy next one after it (toks: the sessions' history arrays)
extern "C" __global__ void __launch_bounds__(256)
oh_k_batch_tokens(int32_t *const *toks, const int32_t *pos, const int32_t *tok, const int32_t *next, int n) {
    const int b = (int)(blockIdx.x * 256 + tid_x());
    if (b >= n) return;
    int32_t *t = ldg(toks + b);
    const int p = ldg(pos + b);
    stg(t + p, ldg(tok + b));
    stg(t + p + 1, ldg(next + b));
}
