// Chunked gated delta rule on the matrix cores (prompt path, a tolerance
// form of oh_k_delta_chunked; ORNITH_HIP_DELTA_MFMA=1). The reference's chunk
// recurrence (delta_chunk, src/ornith_attn.c:215-349), for a chunk of C <= 32
// tokens with incoming state S (dv x dk), decays p_i = prod_{l<=i} alpha_l and
// ratios r_ij = p_i / p_j = prod_{l=j+1}^{i} alpha_l:
//   (I + M) U = diag(beta) V - diag(beta p) K S^T,  M_ij = beta_i r_ij (k_j.k_i), j < i
//   O = diag(p) Q S^T + L U,                          L_ij = r_ij (k_j.q_i),  j <= i
//   S' = p_{C-1} S + U^T diag(g) K,                    g_j = r_{C-1,j}
// is split into the WY form: U = U0 - W S^T with (I + M) U0 = diag(beta) V and
// (I + M) W = diag(beta p) K, which depend only on the chunk's own inputs.
// oh_k_delta_wy forms U0, W, L, g and p for every (value head, chunk) at
// once (forward substitution on the vector ALUs, a thread per column, the
// reference's ratio and coefficient order); oh_k_delta_mfma then walks the
// chunks of one 16-row slab of S in order, each chunk as four small fp32
// products on v_mfma_f32_16x16x4_f32 (X = W S^T, Y = Q S^T, L U, U^T diag(g) K).
// Every product and decay is the reference's in fp32; the sums are
// re-associated (the matrix cores' order), so results differ from the
// reference's bits at the rounding level.

constexpr int kWyC = 32;                               // chunk length (the reference's)
// scratch floats per (chunk, value head): W [32][dk], U0 [32][dk], L [32][32], p [32], g [32]
OH_HD constexpr int delta_wy_floats(int dk) { return 2 * kWyC * dk + kWyC * kWyC + 2 * kWyC; }

typedef float dm_f4 __attribute__((ext_vector_type(4)));
// s_waitcnt immediate for vmcnt(0) with expcnt and lgkmcnt left at their
// maxima (gfx9 encoding: vmcnt [3:0] and [15:14], expcnt [6:4], lgkmcnt [11:8])
constexpr int kWaitVm0 = 0x0F70;

template <int DK>
__global__ void __launch_bounds__(256)
oh_k_delta_wy(const float *kn, const float *conv, const float *al, const float *be, const float *grams,
              float *wy, int T, int nk, int nv, int cc) {
    constexpr int CH = kWyC;
    __shared__ float alpha[CH], beta[CH], p[CH];
    __shared__ float M[CH][CH + 1], R[CH][CH + 1];
    const int hv = (int)blockIdx.x, ch = (int)blockIdx.y, kh = hv % nk, tid = tid_x();
    const int c0 = ch * CH, C = T - c0 < CH ? T - c0 : CH;
    const int qd = nk * DK;
    const float *gm = grams + ((size_t)ch * nk + kh) * 2 * CH * CH;   // kk [i][j] then kq [i][j]
    if (tid < CH) {
        alpha[tid] = tid < C ? ldg(al + (size_t)(c0 + tid) * nv + hv) : 1.0f;
        beta[tid] = tid < C ? ldg(be + (size_t)(c0 + tid) * nv + hv) : 0.0f;
    }
    __syncthreads();
    if (tid == 0) {
        float pp = 0.0f;
        for (int i = 0; i < CH; i++) {
            pp = i == 0 ? alpha[0] : pp * alpha[i];
            p[i] = i < C ? pp : 0.0f;
        }
    }
    if (tid < CH) {
        // row i's ratios and coefficients, j descending as the reference
        const int i = tid;
        for (int j = 0; j < CH; j++) { R[i][j] = 0.0f; M[i][j] = 0.0f; }
        if (i < C) {
            R[i][i] = 1.0f;
            float ratio = 1.0f;
            for (int j = i - 1; j >= 0; j--) {
                ratio *= alpha[j + 1];
                R[i][j] = ratio;
                M[i][j] = beta[i] * ratio * ldg(gm + i * CH + j);
            }
        }
    }
    __syncthreads();
    float *out = wy + ((size_t)ch * nv + hv) * delta_wy_floats(DK);
    if (tid < 2 * DK) {
        // column tid: V columns first (U0), then K columns (W)
        const bool isv = tid < DK;
        const int c = isv ? tid : tid - DK;
        float x[CH];
#pragma unroll
        for (int i = 0; i < CH; i++) {
            float b = 0.0f;
            if (i < C) {
                b = isv ? beta[i] * ldg(conv + (size_t)(c0 + i) * cc + 2 * qd + hv * DK + c)
                        : (beta[i] * p[i]) * ldg(kn + ((size_t)(c0 + i) * nk + kh) * DK + c);
#pragma unroll
                for (int j = CH - 1; j >= 0; j--)
                    if (j < i) b = b - M[i][j] * x[j];
            }
            x[i] = b;
        }
        float *dst = out + (isv ? CH * DK : 0) + c;
#pragma unroll
        for (int i = 0; i < CH; i++) stg(dst + i * DK, x[i]);
    }
    float *Lo = out + 2 * CH * DK, *po = Lo + CH * CH, *go = po + CH;
    for (int e = tid; e < CH * CH; e += 256) {
        const int i = e / CH, j = e % CH;
        stg(Lo + e, (i < C && j <= i) ? R[i][j] * ldg(gm + CH * CH + i * CH + j) : 0.0f);
    }
    if (tid < CH) {
        stg(po + tid, p[tid]);
        stg(go + tid, tid < C ? R[C - 1][tid] : 0.0f);
    }
}

// One block per 16 rows of one value head's state (nv * DK/16 blocks, 4
// waves), the chunks in order. Waves 0, 1 form X = W S^T and U = U0 - X for
// chunk rows 16 t .. (t = wave & 1), waves 2, 3 form Y = Q S^T and then
// O = diag(p) Y + L U; all four update 16-column tiles of the slab,
// S' = p_{C-1} S + U^T diag(g) K. LDS holds the slab S [16][DK+4], U
// transposed [16][36] and the chunk's K [32][DK+2] twice (chunk c in buffer
// c & 1); W, Q, L, U0, p and g are read from global memory straight into the
// lane layout of the product that uses them. Each chunk's operands are
// requested one chunk ahead, so a chunk costs its products and two barriers.
// MFMA operand layout (v_mfma_f32_16x16x4_f32, wave64): A lane l holds
// A[l % 16][k], B lane l holds B[k][l % 16], with k = (l / 16) * K/4 + s at
// step s (each lane's operands are consecutive floats); D lane l, register v
// holds D[4 (l/16) + v][l % 16].
template <int DK>
struct DmOps {
    static constexpr int KW = DK / 4, NK4 = DK / 32;
    float a[KW];              // W (waves 0, 1) or Q (waves 2, 3) row 16 t + l % 16, k = (l/16) KW ..
    float4 k4[NK4];           // K rows (tid + 256 j) / (DK/4), four columns each, for the LDS tile
    float g[8];               // g[(l/16) 8 + s]
    float lu[8];              // waves 2, 3: L[16 t + l % 16][(l/16) 8 + s]
    float x4[4];              // waves 0, 1: U0[16 t + 4 (l/16) + v][r0 + l % 16]; waves 2, 3: p[16 t + 4 (l/16) + v]
    float pl;                 // p[C - 1]
};

template <int DK>
__device__ __forceinline__ void dm_fetch(DmOps<DK> &o, const float *qn, const float *kn, const float *wy, int ch,
                                         int T, int nk, int nv, int hv, int kh, int r0, int tid) {
    constexpr int CH = kWyC, KW = DmOps<DK>::KW;
    const int lane = tid & 63, wave = tid >> 6, li = lane & 15, gq = lane >> 4, t = wave & 1;
    const int c0 = ch * CH, C = T - c0 < CH ? T - c0 : CH;
    const float *blk = wy + ((size_t)ch * nv + hv) * delta_wy_floats(DK);
    const float *Lg = blk + 2 * CH * DK, *pg = Lg + CH * CH, *gg = pg + CH;
    // rows past the chunk's end read its last row: their Q rows give outputs
    // that are not stored, their K rows meet g = 0 and U = 0
    const int i = 16 * t + li;
    const float4 *src = wave < 2 ? (const float4 *)(blk + i * DK + gq * KW)
                                 : (const float4 *)(qn + ((size_t)(c0 + (i < C ? i : C - 1)) * nk + kh) * DK + gq * KW);
#pragma unroll
    for (int s = 0; s < KW / 4; s++) {
        const float4 v = ldg(src + s);
        o.a[4 * s] = v.x; o.a[4 * s + 1] = v.y; o.a[4 * s + 2] = v.z; o.a[4 * s + 3] = v.w;
    }
    if (wave < 2) {
#pragma unroll
        for (int v = 0; v < 4; v++) o.x4[v] = ldg(blk + CH * DK + (16 * t + 4 * gq + v) * DK + r0 + li);
    } else {
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const float4 v = ldg((const float4 *)(Lg + i * CH + gq * 8) + h);
            o.lu[4 * h] = v.x; o.lu[4 * h + 1] = v.y; o.lu[4 * h + 2] = v.z; o.lu[4 * h + 3] = v.w;
        }
        const float4 v = ldg((const float4 *)(pg + 16 * t + 4 * gq));
        o.x4[0] = v.x; o.x4[1] = v.y; o.x4[2] = v.z; o.x4[3] = v.w;
    }
#pragma unroll
    for (int j = 0; j < DmOps<DK>::NK4; j++) {
        const int e = tid + 256 * j, row = e / (DK / 4);
        o.k4[j] = ldg((const float4 *)(kn + ((size_t)(c0 + (row < C ? row : C - 1)) * nk + kh) * DK) + e % (DK / 4));
    }
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const float4 v = ldg((const float4 *)(gg + gq * 8) + h);
        o.g[4 * h] = v.x; o.g[4 * h + 1] = v.y; o.g[4 * h + 2] = v.z; o.g[4 * h + 3] = v.w;
    }
    o.pl = ldg(pg + C - 1);
}

// the chunk's K rows into an LDS tile [32][DK + 2] (row stride = 2 mod 8
// floats: the update's column reads of rows 8 apart fall in distinct banks)
template <int DK>
__device__ __forceinline__ void dm_put_k(const DmOps<DK> &o, float *Kl, int tid) {
    constexpr int KLS = DK + 2;
#pragma unroll
    for (int j = 0; j < DmOps<DK>::NK4; j++) {
        const int e = tid + 256 * j, row = e / (DK / 4), col = 4 * (e % (DK / 4));
        *(float2 *)(Kl + row * KLS + col) = make_float2(o.k4[j].x, o.k4[j].y);
        *(float2 *)(Kl + row * KLS + col + 2) = make_float2(o.k4[j].z, o.k4[j].w);
    }
}

template <int DK>
__global__ void __launch_bounds__(256)
oh_k_delta_mfma(const float *qn, const float *kn, const float *wy, float *S, float *outp, int T, int nk, int nv,
                float out_scale) {
    constexpr int CH = kWyC, TS = DK + 4, LS = 36, KLS = DK + 2, KW = DK / 4, NQ = DK / 64;
    __shared__ __align__(16) float Ss[16 * TS];        // the slab
    __shared__ __align__(16) float Ut[16 * LS];        // Ut[m][k] = U[k][m]
    __shared__ __align__(16) float Kl[2][CH * KLS];    // the chunk's K rows
    const int tid = tid_x(), lane = tid & 63, wave = tid >> 6;
    // blocks go to the 8 XCDs round-robin (XCD = block % 8); with nv % 8 == 0
    // the DK/16 slabs of a head share one XCD, so its L2 holds the head's W,
    // Q, K and L once instead of every XCD pulling every head's operands
    constexpr int NS = DK / 16;
    const int x = (int)blockIdx.x;
    const int hv = (nv & 7) == 0 ? ((x >> 3) / NS) * 8 + (x & 7) : x / NS;
    const int slab = (nv & 7) == 0 ? (x >> 3) % NS : x % NS, kh = hv % nk;
    const int r0 = slab * 16;                          // first state row of the slab
    const int vd = nv * DK;
    const int li = lane & 15, gq = lane >> 4, t = wave & 1;
    float *Sg = S + ((size_t)hv * DK + r0) * DK;
    const int nch = (T + CH - 1) / CH;
    DmOps<DK> cur, nxt;
    dm_fetch<DK>(cur, qn, kn, wy, 0, T, nk, nv, hv, kh, r0, tid);
    for (int e = tid; e < 16 * DK / 4; e += 256) {
        const int m = (4 * e) / DK, n = (4 * e) % DK;
        *(float4 *)(Ss + m * TS + n) = ldg((const float4 *)Sg + e);
    }
    dm_put_k<DK>(cur, Kl[0], tid);
    __syncthreads();
    for (int ch = 0; ch < nch; ch++) {
        const int c0 = ch * CH, C = T - c0 < CH ? T - c0 : CH;
        // this chunk's operands (requested a chunk ago) are complete: say so
        // before the next chunk's requests go out, or the waits on them
        // (counted in issue order) would also wait for the new requests
        __builtin_amdgcn_s_waitcnt(kWaitVm0);
        if (ch + 1 < nch) dm_fetch<DK>(nxt, qn, kn, wy, ch + 1, T, nk, nv, hv, kh, r0, tid);
        // X = W S^T (waves 0, 1) or Y = Q S^T (waves 2, 3): the slab operand
        // read whole, then four independent accumulator chains
        float sb[KW];
#pragma unroll
        for (int s4 = 0; s4 < KW / 4; s4++) {
            const float4 v = *(const float4 *)(Ss + li * TS + gq * KW + 4 * s4);
            sb[4 * s4] = v.x; sb[4 * s4 + 1] = v.y; sb[4 * s4 + 2] = v.z; sb[4 * s4 + 3] = v.w;
        }
        dm_f4 a0 = {0.0f, 0.0f, 0.0f, 0.0f}, a1 = a0, a2 = a0, a3 = a0;
#pragma unroll
        for (int s4 = 0; s4 < KW / 4; s4++) {
            a0 = __builtin_amdgcn_mfma_f32_16x16x4f32(cur.a[4 * s4], sb[4 * s4], a0, 0, 0, 0);
            a1 = __builtin_amdgcn_mfma_f32_16x16x4f32(cur.a[4 * s4 + 1], sb[4 * s4 + 1], a1, 0, 0, 0);
            a2 = __builtin_amdgcn_mfma_f32_16x16x4f32(cur.a[4 * s4 + 2], sb[4 * s4 + 2], a2, 0, 0, 0);
            a3 = __builtin_amdgcn_mfma_f32_16x16x4f32(cur.a[4 * s4 + 3], sb[4 * s4 + 3], a3, 0, 0, 0);
        }
        const dm_f4 acc = (a0 + a1) + (a2 + a3);
        if (wave < 2) {
            // U = U0 - X, kept transposed for the two products that read it
#pragma unroll
            for (int v = 0; v < 4; v++) Ut[li * LS + 16 * t + 4 * gq + v] = cur.x4[v] - acc[v];
        }
        __syncthreads();
        const float *Kc = Kl[ch & 1];
        float ur[8], kb[NQ][8];
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const float4 v = *(const float4 *)(Ut + li * LS + gq * 8 + 4 * h);
            ur[4 * h] = v.x; ur[4 * h + 1] = v.y; ur[4 * h + 2] = v.z; ur[4 * h + 3] = v.w;
        }
#pragma unroll
        for (int q = 0; q < NQ; q++)
#pragma unroll
            for (int s = 0; s < 8; s++) kb[q][s] = Kc[(gq * 8 + s) * KLS + 16 * (wave * NQ + q) + li];
        if (wave >= 2) {
            // O = diag(p) Y + L U for chunk rows 16 t ..; B = U [k][m] = Ut[m][k]
            dm_f4 l0 = {0.0f, 0.0f, 0.0f, 0.0f}, l1 = l0;
#pragma unroll
            for (int s = 0; s < 8; s += 2) {
                l0 = __builtin_amdgcn_mfma_f32_16x16x4f32(cur.lu[s], ur[s], l0, 0, 0, 0);
                l1 = __builtin_amdgcn_mfma_f32_16x16x4f32(cur.lu[s + 1], ur[s + 1], l1, 0, 0, 0);
            }
            const dm_f4 lu = l0 + l1;
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int i = 16 * t + 4 * gq + v;
                if (i < C) stg(outp + (size_t)(c0 + i) * vd + hv * DK + r0 + li, (cur.x4[v] * acc[v] + lu[v]) * out_scale);
            }
        }
        // S' = p_{C-1} S + U^T diag(g) K: A = g_k U[k][m] (lane: Ut[m][k]),
        // B = K[k][n0 + n] from the LDS tile
        float ga[8];
#pragma unroll
        for (int s = 0; s < 8; s++) ga[s] = cur.g[s] * ur[s];
        dm_f4 d0[NQ], d1[NQ];
#pragma unroll
        for (int q = 0; q < NQ; q++) {
            d0[q] = dm_f4{0.0f, 0.0f, 0.0f, 0.0f};
            d1[q] = d0[q];
        }
#pragma unroll
        for (int s = 0; s < 8; s += 2) {
#pragma unroll
            for (int q = 0; q < NQ; q++) {
                d0[q] = __builtin_amdgcn_mfma_f32_16x16x4f32(ga[s], kb[q][s], d0[q], 0, 0, 0);
                d1[q] = __builtin_amdgcn_mfma_f32_16x16x4f32(ga[s + 1], kb[q][s + 1], d1[q], 0, 0, 0);
            }
        }
#pragma unroll
        for (int q = 0; q < NQ; q++) {
            const int n0 = 16 * (wave * NQ + q);
            const dm_f4 d = d0[q] + d1[q];
#pragma unroll
            for (int v = 0; v < 4; v++) {
                float *sp = Ss + (4 * gq + v) * TS + n0 + li;
                *sp = cur.pl * *sp + d[v];
            }
        }
        // the next chunk's K into the other tile (its last readers passed the
        // barrier that ended the previous chunk)
        if (ch + 1 < nch) dm_put_k<DK>(nxt, Kl[(ch + 1) & 1], tid);
        __syncthreads();
        if (ch + 1 < nch) cur = nxt;
    }
    for (int e = tid; e < 16 * DK / 4; e += 256) {
        const int m = (4 * e) / DK, n = (4 * e) % DK;
        stg((float4 *)Sg + e, *(const float4 *)(Ss + m * TS + n));
    }
}
