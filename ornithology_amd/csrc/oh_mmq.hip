// Exact batched Q4_K x Q8_K products on the matrix cores (prompt path).
//
// Y[p][row] = vec_dot_q4_K(W[row], X[p / adiv]) for every (row, column p), with
// the reference's arithmetic (src/ornith_qdot.c:76-105): per super-block i the
// integer sums isum = sum_j sc_j * sum_l q4 * q8 and summs = sum_j m_j *
// (bsums_2j + bsums_2j+1), then sumf += d * (float)isum + dm * (float)summs in
// super-block order, d = yd * f16(d), dm = -yd * f16(dmin).
//
// The integer sums run on v_mfma_i32_32x32x32_i8. Each 6-bit sub-block scale
// splits as sc = 8 * hi + lo (hi, lo < 8), so q4 * lo and q4 * hi (at most
// 105) stay int8 and a whole super-block accumulates exactly in int32:
// isum = 8 * (q4*hi . q8) + (q4*lo . q8). The min term is a K = 8 product of
// the 6-bit mins with the Q8_K pair sums, which split as 64 * bh + bl into
// int8 bytes (the activation quantiser emits them). Integer sums are exact in
// any order, so only the float combine needs the reference's order, and it is
// done per (row, column, super-block) exactly as the scalar dot does it.
//
// Block: 256 threads, a tile of 128 rows x 64 columns; wave w owns rows
// [32w, 32w + 32) and both 32-column halves. One super-block per stage; the
// stage's operands go global -> LDS with global_load_lds (no registers), two
// stages in flight. The weights come from the tensor's prompt tiles (below):
// one wave-load of a code piece, or of the headers, for 64 rows of one
// super-block reads 1 KB contiguously, and in LDS the 32 lanes of an MFMA
// operand read consecutive 16-byte chunks. Activation codes are loaded
// 4 columns per wave-load (16 lanes read a column's 256 bytes, whole cache
// lines) and kept column-major with the piece index XOR-swizzled by the
// column, so the operand reads (one piece of 16 consecutive columns) still
// fall in distinct LDS banks.

typedef int mq_v4i __attribute__((ext_vector_type(4)));
typedef int mq_v16i __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void mq_lds_t;

constexpr int kMqRows = 128, kMqCols = 64;
constexpr int kMqA = 0;                         // codes [8 pieces][128 rows][16 B]
constexpr int kMqB = kMqA + 8 * 128 * 16;       // activation codes [64 cols][16 slots][16 B]
constexpr int kMqH = kMqB + 16 * 64 * 16;       // weight headers [128 rows][16 B]
constexpr int kMqP = kMqH + 128 * 16;           // pair-sum bytes [64 cols][16 B]
constexpr int kMqD = kMqP + 64 * 16;            // activation d [64 cols]
constexpr int kMqStage = kMqD + 64 * 4;         // 36096 B
constexpr int kMqLoads = 16 + 16 + 2 + 1 + 1;   // wave-loads per stage (9 per wave)

// Prompt tiles: a copy of a Q4_K / Q6_K tensor's code plane A (P = 8 or 12
// pieces of 16 B per super-block) and header plane B (16 B per super-block)
// for these kernels. Row r, super-block i, piece p sits at 16-byte index
// ((r / 64 * nb + i) * P + p) * 64 + r % 64 of PA, its header at
// (r / 64 * nb + i) * 64 + r % 64 of PB. The decode planes group 64
// consecutive super-blocks of a row instead, which leaves the 64 rows of one
// stage load in 64 different cache lines. One thread per 16-byte destination.
extern "C" __global__ void __launch_bounds__(256) oh_k_mmq_tiles(const uint4 *A, const uint4 *B, uint4 *PA,
                                                                 uint4 *PB, int64_t rows, int nb, int P) {
    const int64_t na = rows * nb * P, n = na + rows * nb;
    for (int64_t d = (int64_t)blockIdx.x * 256 + threadIdx.x; d < n; d += (int64_t)gridDim.x * 256) {
        const bool code = d < na;
        const int64_t e = code ? d : d - na, q = e >> 6;
        const int p = code ? (int)(q % P) : 0;
        const int64_t ti = code ? q / P : q;
        const int i = (int)(ti % nb);
        const int64_t r = ti / nb * 64 + (e & 63), bi = r * nb + i;
        if (code) PA[e] = A[(bi >> 6) * 64 * P + p * 64 + (bi & 63)];
        else PB[e] = B[bi];
    }
}

namespace {

OH_DEV void mq_load16(const void *g, uint8_t *lds) {
    __builtin_amdgcn_global_load_lds(g, (mq_lds_t *)lds, 16, 0, 0);
}
OH_DEV void mq_load4(const void *g, uint8_t *lds) {
    __builtin_amdgcn_global_load_lds(g, (mq_lds_t *)lds, 4, 0, 0);
}

// LDS slot (16 B) of activation piece p of tile column c
OH_DEV int mq_act_slot(int c, int p) { return c * 16 + (p ^ (c & 15)); }

// The 9 wave-loads of super-block i that wave w issues into stage S (lane k
// of a wave-load writes 16 B, or 4 B, at the wave-uniform base + k * size):
// weight codes L = w + 4n (piece L / 2, rows 64 * (L & 1) + lane), activation
// codes of columns 4j .. 4j + 3 for j = w + 4n (lane k: column 4j + k / 16,
// slot k % 16), then the headers of rows 64w + lane (waves 0, 1), the pair-sum
// bytes (wave 2) or the activation d (wave 3) of column lane. acs[n]: the
// activation row of column 4(w + 4n) + lane / 16; acol: that of column lane.
OH_DEV void mq_stage_load(const oh_mmq &M, const uint8_t *A, const uint8_t *Bh, int64_t rbase, int R0, int i,
                          uint8_t *S, int w, int lane, const int (&acs)[4], int acol) {
    const int nb = M.nb;
    const int64_t rt = (rbase + R0) >> 6;          // first 64-row tile of the block
#pragma unroll
    for (int n = 0; n < 4; n++) {
        const int L = w + 4 * n, p = L >> 1, rh = L & 1;
        const uint4 *src = (const uint4 *)A + ((rt + rh) * nb + i) * (8 * 64) + p * 64 + lane;
        mq_load16(src, S + kMqA + (p * 128 + rh * 64) * 16);
    }
#pragma unroll
    for (int n = 0; n < 4; n++) {
        const int j = w + 4 * n, c = 4 * j + (lane >> 4), q = (lane & 15) ^ (c & 15);
        mq_load16(M.xqs + (size_t)acs[n] * M.in + (size_t)i * 256 + q * 16, S + kMqB + j * 64 * 16);
    }
    if (w < 2) {
        mq_load16((const uint4 *)Bh + ((rt + w) * nb + i) * 64 + lane, S + kMqH + w * 64 * 16);
    } else if (w == 2) {
        mq_load16(M.xbp + ((size_t)acol * nb + i) * 16, S + kMqP);
    } else {
        mq_load4(M.xd + (size_t)acol * nb + i, S + kMqD);
    }
}

// packed nibbles (bytes <= 15) times a factor <= 7 held in both 16-bit
// halves of f: bytes of at most 105 and halves below 2^16, so the two 16-bit
// products (one full-rate instruction) equal the 32-bit product
typedef unsigned short mq_u16x2 __attribute__((ext_vector_type(2)));
OH_DEV int mq_mul_bytes(uint32_t n, uint32_t f) {
    return __builtin_bit_cast(int, __builtin_bit_cast(mq_u16x2, n) * __builtin_bit_cast(mq_u16x2, f));
}

} // namespace

// Expert-grouped launches: blocks go to the 8 XCDs round-robin (XCD = linear
// block id % 8). Consecutive work items mostly belong to one expert (its
// column tiles), so each XCD takes runs of kMqRun consecutive items, every
// row tile of them, in turn: one expert's tiles then share an L2 and its
// weights come from HBM about once. Dense launches keep the plain order
// (a row tile's column tiles share an XCD when the row tiles are a multiple
// of 8). The launcher rounds the item rows up to a multiple of 8 * kMqRun.
constexpr int kMqRun = 8;
OH_DEV void mq_block(const oh_mmq &M, int &bx, int &by) {
    bx = (int)blockIdx.x;
    by = (int)blockIdx.y;
    const int gx = (int)gridDim.x, gy = (int)gridDim.y;
    if (!M.list || gy % (8 * kMqRun)) return;
    const int L = bx + gx * by, k = L & 7, j = L >> 3;
    const int m = j / (kMqRun * gx), r = j - m * (kMqRun * gx);
    by = (8 * m + k) * kMqRun + r / gx;
    bx = r % gx;
}

extern "C" __global__ void __launch_bounds__(256, 2) oh_k_mmq_q4k(oh_mmq M) {
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ int sact[kMqCols], sout[kMqCols];
    const int tid = tid_x(), lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int zi = (int)blockIdx.z;
    int bx, by;
    mq_block(M, bx, by);
    int g = 0, tile = by, n;
    if (M.list) {
        if (by >= ldg(M.items)) return;
        const int it = ldg(M.items + 1 + by);
        g = it >> 16;
        tile = it & 0xffff;
        n = ldg(M.cnt + g) - tile * kMqCols;
    } else {
        n = M.ncol - tile * kMqCols;
    }
    n = n < kMqCols ? n : kMqCols;
    if (n <= 0) return;
    const int R0 = bx * kMqRows;
    const uint8_t *A = zi ? M.A2 : M.A, *Bh = zi ? M.B2 : M.B;
    const int64_t rbase = M.list ? (int64_t)g * M.rows : 0;
    if (tid < kMqCols) {
        const int c = tid < n ? tid : n - 1;
        const int p = M.list ? ldg(M.list + (size_t)g * M.lstride + tile * kMqCols + c) : tile * kMqCols + c;
        sact[tid] = p / M.adiv;
        sout[tid] = p;
    }
    __syncthreads();
    const int acol = sact[lane];                    // this lane's column in activation loads
    int acs[4];
#pragma unroll
    for (int u = 0; u < 4; u++) acs[u] = sact[4 * (wave + 4 * u) + (lane >> 4)];
    auto stage = [&](int i, int buf) {
        mq_stage_load(M, A, Bh, rbase, R0, i, smem + buf * kMqStage, wave, lane, acs, acol);
    };

    const int h = lane >> 5, lr = lane & 31, arow = 32 * wave + lr;
    const uint32_t NM = 0x0f0f0f0fu;
    float acc[2][16];
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
        for (int v = 0; v < 16; v++) acc[t][v] = 0.0f;

    const int nb = M.nb;
    stage(0, 0);
    for (int i = 0; i < nb; i++) {
        const int buf = i & 1;
        if (i + 1 < nb) {
            stage(i + 1, buf ^ 1);
            // this wave's loads of stage i are the older ones; every wave
            // issued 9 for stage i + 1
            asm volatile("s_waitcnt vmcnt(9)" ::: "memory");
        } else {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
        __syncthreads();
        const uint8_t *S = smem + buf * kMqStage;
        const uint32_t *H = (const uint32_t *)(S + kMqH);
        // scales and mins of this lane's A row (sb_term's unpacking of scales[12])
        const uint4 hd = *(const uint4 *)(H + 4 * arow);
        const uint32_t hy = hd.y, hz = hd.z, hw = hd.w;
        const uint32_t scl = hy & 0x3f3f3f3fu, sch = (hw & 0x0f0f0f0fu) | ((hy >> 2) & 0x30303030u);
        const uint32_t mnl = hz & 0x3f3f3f3fu, mnh = ((hw >> 4) & 0x0f0f0f0fu) | ((hz >> 2) & 0x30303030u);
        mq_v16i ihi[2], ilo[2];
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int v = 0; v < 16; v++) { ihi[t][v] = 0; ilo[t][v] = 0; }
#pragma unroll
        for (int m = 0; m < 4; m++) {
            // piece 2m + h holds elements 16h.. of sub-blocks 2m (low nibbles)
            // and 2m + 1 (high nibbles)
            const uint4 wq = *(const uint4 *)(S + kMqA + ((2 * m + h) * 128 + arow) * 16);
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const int s = 2 * m + e;
                const uint32_t sc = ((s < 4 ? scl : sch) >> (8 * (s & 3))) & 0xffu;
                const uint32_t lo = (sc & 7u) * 0x10001u, hi = (sc >> 3) * 0x10001u;
                const uint32_t n0 = (e ? wq.x >> 4 : wq.x) & NM, n1 = (e ? wq.y >> 4 : wq.y) & NM;
                const uint32_t n2 = (e ? wq.z >> 4 : wq.z) & NM, n3 = (e ? wq.w >> 4 : wq.w) & NM;
                const mq_v4i alo = {mq_mul_bytes(n0, lo), mq_mul_bytes(n1, lo), mq_mul_bytes(n2, lo),
                                    mq_mul_bytes(n3, lo)};
                const mq_v4i ahi = {mq_mul_bytes(n0, hi), mq_mul_bytes(n1, hi), mq_mul_bytes(n2, hi),
                                    mq_mul_bytes(n3, hi)};
#pragma unroll
                for (int t = 0; t < 2; t++) {
                    const mq_v4i xb = *(const mq_v4i *)(S + kMqB + mq_act_slot(32 * t + lr, 2 * s + h) * 16);
                    ihi[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(ahi, xb, ihi[t], 0, 0, 0);
                    ilo[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(alo, xb, ilo[t], 0, 0, 0);
                }
            }
        }
        // mins: K = 8 (bytes 0..7 of the lanes of the first half), the rest zero
        const mq_v4i am = h ? mq_v4i{0, 0, 0, 0} : mq_v4i{(int)mnl, (int)mnh, 0, 0};
        mq_v16i shi[2], slo[2];
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const uint4 bp = *(const uint4 *)(S + kMqP + (32 * t + lr) * 16);
            const mq_v4i bl = h ? mq_v4i{0, 0, 0, 0} : mq_v4i{(int)bp.x, (int)bp.y, 0, 0};
            const mq_v4i bh = h ? mq_v4i{0, 0, 0, 0} : mq_v4i{(int)bp.z, (int)bp.w, 0, 0};
            mq_v16i zero;
#pragma unroll
            for (int v = 0; v < 16; v++) zero[v] = 0;
            shi[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(am, bh, zero, 0, 0, 0);
            slo[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(am, bl, zero, 0, 0, 0);
        }
        // float combine: output (row 8*(v/4) + 4h + v%4, column lr) of each
        // 32x32 tile, per super-block in order
        const float *XD = (const float *)(S + kMqD);
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const float yd = XD[32 * t + lr], nyd = -yd;
#pragma unroll
            for (int vg = 0; vg < 4; vg++) {
                const uint32_t *hr = H + 4 * (32 * wave + 8 * vg + 4 * h);
                const uint32_t dw[4] = {hr[0], hr[4], hr[8], hr[12]};
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const int v = 4 * vg + k;
                    const float d = yd * h2f((uint16_t)(dw[k] & 0xffffu));
                    const float dm = nyd * h2f((uint16_t)(dw[k] >> 16));
                    const int isum = (ihi[t][v] << 3) + ilo[t][v];
                    const int summs = (shi[t][v] << 6) + slo[t][v];
                    acc[t][v] += d * (float)isum + dm * (float)summs;
                }
            }
        }
        __syncthreads();                            // stage buf is refilled next iteration
    }
    const size_t zoff = (size_t)zi * M.rows;
#pragma unroll
    for (int t = 0; t < 2; t++) {
        const int col = 32 * t + lr;
        if (col >= n) continue;
        float *yc = M.y + (size_t)sout[col] * M.ystride + zoff + R0 + 32 * wave + 4 * h;
#pragma unroll
        for (int v = 0; v < 16; v++) {
            float *yp = yc + 8 * (v / 4) + (v % 4);
            if (M.mode == 1) stg(yp, ldg(yp) + acc[t][v]);
            else stg(yp, acc[t][v]);
        }
    }
}

// ---- Q6_K x Q8_K (src/ornith_qdot.c:109-138) --------------------------------
// Per super-block the reference's integer sum is isum = sum_g sc_g *
// sum_{i in g} (q6_i - 32) * q8_i over the 16-element groups g, and the float
// combine sumf += (yd * f16(d)) * isum in super-block order. The integer sum
// is formed exactly on v_mfma_i32_32x32x32_i8: each weight becomes
// p = sc_g * (q6 - 32) (|p| <= 4096), split as p = 64 * hi + lo with
// lo in [0, 63] and hi in [-64, 64], both int8; then isum =
// 64 * (hi . q8) + (lo . q8), exact in int32. A lane's 16 K-values of one
// MFMA are exactly one group (one scale). The transform runs on packed int16
// (two weights per instruction).
//
// Block and stage pipeline as oh_k_mmq_q4k; the stage holds the 12 code
// pieces (ql 0-7, qh 8-11) of 128 rows, the rows' 16 group scales, the 64
// columns' activation codes and d; the rows' f16 d of every super-block sit in
// LDS for the whole launch.
constexpr int kM6A = 0;                          // codes [12 pieces][128 rows][16 B]
constexpr int kM6B = kM6A + 12 * 128 * 16;       // activation codes [64 cols][16 slots][16 B]
constexpr int kM6S = kM6B + 16 * 64 * 16;        // group scales [128 rows][16 B]
constexpr int kM6X = kM6S + 128 * 16;            // activation d [64 cols]
constexpr int kM6Stage = kM6X + 64 * 4;          // 43264 B
constexpr int kM6Loads = 24 + 16 + 2 + 1;        // wave-loads per stage (10 or 11 per wave)
OH_HD inline int m6_lds_bytes(int nb, int nbuf) { return nbuf * kM6Stage + 128 * nb * 2; }
// Products of at most kM6OneBuf super-blocks (K <= 512: the expert down
// projections) are a short latency chain per block; one stage buffer (44 KB of
// LDS instead of 87 KB) lets two blocks share a CU and overlap their chains.
constexpr int kM6OneBuf = 2;

typedef short m6_s2 __attribute__((ext_vector_type(2)));

namespace {

// The wave-loads of super-block i that wave w issues into stage S: weight
// codes L = w + 4n (piece L / 2, rows 64 * (L & 1) + lane), activation codes
// as in mq_stage_load, then the group scales of rows 64w + lane (waves 0, 1)
// or the activation d of column lane (wave 2): 11, 11, 11 and 10 loads.
OH_DEV void m6_stage_load(const oh_mmq &M, const uint8_t *A, const uint8_t *Bs, int64_t rbase, int R0, int i,
                          uint8_t *S, int w, int lane, const int (&acs)[4], int acol) {
    const int nb = M.nb;
    const int64_t rt = (rbase + R0) >> 6;
#pragma unroll
    for (int n = 0; n < 6; n++) {
        const int L = w + 4 * n, p = L >> 1, rh = L & 1;
        const uint4 *src = (const uint4 *)A + ((rt + rh) * nb + i) * (12 * 64) + p * 64 + lane;
        mq_load16(src, S + kM6A + (p * 128 + rh * 64) * 16);
    }
#pragma unroll
    for (int n = 0; n < 4; n++) {
        const int j = w + 4 * n, c = 4 * j + (lane >> 4), q = (lane & 15) ^ (c & 15);
        mq_load16(M.xqs + (size_t)acs[n] * M.in + (size_t)i * 256 + q * 16, S + kM6B + j * 64 * 16);
    }
    if (w < 2) {
        mq_load16((const uint4 *)Bs + ((rt + w) * nb + i) * 64 + lane, S + kM6S + w * 64 * 16);
    } else if (w == 2) {
        mq_load4(M.xd + (size_t)acol * nb + i, S + kM6X);
    }
}

// sixteen weights of one group (bytes of q6 in [0, 63], four per word) times
// the group scale, split into the lo / hi int8 operands
OH_DEV void m6_split(const uint32_t q6[4], int sc, mq_v4i &lo, mq_v4i &hi) {
    const m6_s2 scv = {(short)sc, (short)sc}, off = {(short)(-32 * sc), (short)(-32 * sc)};
    const m6_s2 m63 = {63, 63};
#pragma unroll
    for (int k = 0; k < 4; k++) {
        // bytes 0,1 and 2,3 of the word as int16 pairs
        const uint32_t u01 = __builtin_amdgcn_perm(0u, q6[k], 0x0c010c00u);
        const uint32_t u23 = __builtin_amdgcn_perm(0u, q6[k], 0x0c030c02u);
        const m6_s2 p01 = __builtin_bit_cast(m6_s2, u01) * scv + off;
        const m6_s2 p23 = __builtin_bit_cast(m6_s2, u23) * scv + off;
        const uint32_t l01 = __builtin_bit_cast(uint32_t, p01 & m63), l23 = __builtin_bit_cast(uint32_t, p23 & m63);
        const uint32_t h01 = __builtin_bit_cast(uint32_t, p01 >> (m6_s2){6, 6});
        const uint32_t h23 = __builtin_bit_cast(uint32_t, p23 >> (m6_s2){6, 6});
        // low bytes of the four int16 values, in order
        lo[k] = (int)__builtin_amdgcn_perm(l23, l01, 0x06040200u);
        hi[k] = (int)__builtin_amdgcn_perm(h23, h01, 0x06040200u);
    }
}

// NBUF stage buffers: 2 overlaps the loads of super-block i + 1 with the
// products of i; 1 loads super-block i + 1 after the products of i.
template <int NBUF>
OH_DEV void m6_body(const oh_mmq &M, uint8_t *smem, int *sact, int *sout) {
    const int tid = tid_x(), lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int zi = (int)blockIdx.z;
    int bx, by;
    mq_block(M, bx, by);
    int g = 0, tile = by, n;
    if (M.list) {
        if (by >= ldg(M.items)) return;
        const int it = ldg(M.items + 1 + by);
        g = it >> 16;
        tile = it & 0xffff;
        n = ldg(M.cnt + g) - tile * kMqCols;
    } else {
        n = M.ncol - tile * kMqCols;
    }
    n = n < kMqCols ? n : kMqCols;
    if (n <= 0) return;
    const int R0 = bx * kMqRows;
    const uint8_t *A = zi ? M.A2 : M.A, *Bs = zi ? M.B2 : M.B, *Cd = zi ? M.C2 : M.C;
    const int64_t rbase = M.list ? (int64_t)g * M.rows : 0;
    const int nb = M.nb;
    uint16_t *Dr = (uint16_t *)(smem + NBUF * kM6Stage);   // [128 rows][nb] f16 d
    for (int k = tid; k < 128 * nb; k += 256) {
        const int r = k / nb, i = k - r * nb;
        Dr[k] = ldg((const uint16_t *)(Cd + ((rbase + R0 + r) * nb + i) * 2));
    }
    if (tid < kMqCols) {
        const int c = tid < n ? tid : n - 1;
        const int p = M.list ? ldg(M.list + (size_t)g * M.lstride + tile * kMqCols + c) : tile * kMqCols + c;
        sact[tid] = p / M.adiv;
        sout[tid] = p;
    }
    __syncthreads();
    const int acol = sact[lane];
    int acs[4];
#pragma unroll
    for (int u = 0; u < 4; u++) acs[u] = sact[4 * (wave + 4 * u) + (lane >> 4)];
    auto stage = [&](int i, int buf) {
        m6_stage_load(M, A, Bs, rbase, R0, i, smem + buf * kM6Stage, wave, lane, acs, acol);
    };

    const int h = lane >> 5, lr = lane & 31, arow = 32 * wave + lr;
    const uint32_t NM = 0x0f0f0f0fu;
    float acc[2][16];
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
        for (int v = 0; v < 16; v++) acc[t][v] = 0.0f;

    stage(0, 0);
    for (int i = 0; i < nb; i++) {
        const int buf = NBUF == 2 ? i & 1 : 0;
        if (NBUF == 2 && i + 1 < nb) {
            stage(i + 1, buf ^ 1);
            // this wave's loads of stage i are the older ones; every wave
            // issued at least 10 for stage i + 1
            asm volatile("s_waitcnt vmcnt(10)" ::: "memory");
        } else {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
        __syncthreads();
        const uint8_t *S = smem + buf * kM6Stage;
        const int8_t *sc8 = (const int8_t *)(S + kM6S + arow * 16);
        mq_v16i ihi[2], ilo[2];
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int v = 0; v < 16; v++) { ihi[t][v] = 0; ilo[t][v] = 0; }
#pragma unroll
        for (int ks = 0; ks < 8; ks++) {
            // this lane's group gq = 2 ks + h: elements 16 gq .. + 15 of the
            // super-block (half hh, quarter qt, 16-element part pr)
            const int gq = 2 * ks + h, hh = gq >> 3, qt = (gq & 7) >> 1, pr = gq & 1;
            const uint4 wl = *(const uint4 *)(S + kM6A + ((4 * hh + 2 * (qt & 1) + pr) * 128 + arow) * 16);
            const uint4 wh = *(const uint4 *)(S + kM6A + ((8 + 2 * hh + pr) * 128 + arow) * 16);
            const uint32_t l4[4] = {wl.x, wl.y, wl.z, wl.w}, h4[4] = {wh.x, wh.y, wh.z, wh.w};
            uint32_t q6[4];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const uint32_t nib = (qt >> 1) ? (l4[k] >> 4) & NM : l4[k] & NM;
                q6[k] = nib | (((h4[k] >> (2 * qt)) & 0x03030303u) << 4);
            }
            mq_v4i alo, ahi;
            m6_split(q6, (int)sc8[gq], alo, ahi);
#pragma unroll
            for (int t = 0; t < 2; t++) {
                const mq_v4i xb = *(const mq_v4i *)(S + kM6B + mq_act_slot(32 * t + lr, 2 * ks + h) * 16);
                ihi[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(ahi, xb, ihi[t], 0, 0, 0);
                ilo[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(alo, xb, ilo[t], 0, 0, 0);
            }
        }
        // float combine: output (row 8*(v/4) + 4h + v%4, column lr) of each
        // 32x32 tile, per super-block in order
        const float *XD = (const float *)(S + kM6X);
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const float yd = XD[32 * t + lr];
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int row = 32 * wave + 8 * (v / 4) + 4 * h + (v % 4);
                const float d = yd * h2f(Dr[row * nb + i]);
                const int isum = 64 * ihi[t][v] + ilo[t][v];
                acc[t][v] += d * (float)isum;
            }
        }
        __syncthreads();                            // stage buf is refilled next
        if (NBUF == 1 && i + 1 < nb) stage(i + 1, 0);
    }
    const size_t zoff = (size_t)zi * M.rows;
#pragma unroll
    for (int t = 0; t < 2; t++) {
        const int col = 32 * t + lr;
        if (col >= n) continue;
        float *yc = M.y + (size_t)sout[col] * M.ystride + zoff + R0 + 32 * wave + 4 * h;
#pragma unroll
        for (int v = 0; v < 16; v++) {
            float *yp = yc + 8 * (v / 4) + (v % 4);
            if (M.mode == 1) stg(yp, ldg(yp) + acc[t][v]);
            else stg(yp, acc[t][v]);
        }
    }
}

} // namespace

extern "C" __global__ void __launch_bounds__(256, 1) oh_k_mmq_q6k(oh_mmq M) {
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ int sact[kMqCols], sout[kMqCols];
    m6_body<2>(M, smem, sact, sout);
}
extern "C" __global__ void __launch_bounds__(256, 2) oh_k_mmq_q6k_s1(oh_mmq M) {
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ int sact[kMqCols], sout[kMqCols];
    m6_body<1>(M, smem, sact, sout);
}

// Work items of a grouped product: (group, 64-column tile) pairs, packed as
// g << 16 | tile after the count in items[0]. One block of 256 threads.
extern "C" __global__ void __launch_bounds__(256) oh_k_mmq_items(const int32_t *cnt, int ne, int32_t *items) {
    __shared__ int pre[1025];
    const int tid = tid_x();
    for (int g = tid; g < ne; g += 256) pre[g + 1] = (ldg(cnt + g) + kMqCols - 1) / kMqCols;
    if (tid == 0) pre[0] = 0;
    __syncthreads();
    if (tid == 0)
        for (int g = 0; g < ne; g++) pre[g + 1] += pre[g];
    __syncthreads();
    for (int g = tid; g < ne; g += 256)
        for (int k = pre[g]; k < pre[g + 1]; k++) stg(items + 1 + k, (g << 16) | (k - pre[g]));
    if (tid == 0) stg(items, pre[ne]);
}
