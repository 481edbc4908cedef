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
// waves), the chunks in order. LDS: the slab S [16][DK+4]; the chunk's W and
// Q [32][DK+4], K transposed [DK][36], L [32][36], U transposed [16][36], p, g.
// The MFMA k index of lane l at step s is (l/16) * K/4 + s, so each lane's
// operands are consecutive floats (b128 reads).
OH_HD constexpr int delta_mfma_lds_bytes(int dk) {
    return (16 * (dk + 4) + 2 * 32 * (dk + 4) + dk * 36 + 32 * 36 + 16 * 36 + 2 * 32) * 4;
}

template <int DK>
__global__ void __launch_bounds__(256)
oh_k_delta_mfma(const float *qn, const float *kn, const float *wy, float *S, float *outp, int T, int nk, int nv,
                float out_scale) {
    constexpr int CH = kWyC, TS = DK + 4, LS = 36, NKT = DK / 16;
    extern __shared__ __align__(16) float dml[];
    float *Ss = dml;                                   // [16][TS]
    float *Wc = Ss + 16 * TS;                          // [32][TS]
    float *Qc = Wc + 32 * TS;                          // [32][TS]
    float *Kt = Qc + 32 * TS;                          // [DK][LS]: Kt[n][k] = K[k][n]
    float *Lc = Kt + DK * LS;                          // [32][LS]
    float *Ut = Lc + 32 * LS;                          // [16][LS]: Ut[m][k] = U[k][m]
    float *pc = Ut + 16 * LS, *gc = pc + 32;
    const int tid = tid_x(), lane = tid & 63, wave = tid >> 6;
    const int hv = (int)blockIdx.x / (DK / 16), slab = (int)blockIdx.x % (DK / 16), kh = hv % nk;
    const int r0 = slab * 16;                          // first state row of the slab
    const int vd = nv * DK;
    const int li = lane & 15, gq = lane >> 4;
    float *Sg = S + ((size_t)hv * DK + r0) * DK;
    for (int e = tid; e < 16 * DK / 4; e += 256) {
        const int m = (4 * e) / DK, n = (4 * e) % DK;
        *(float4 *)(Ss + m * TS + n) = ldg((const float4 *)Sg + e);
    }
    const int nch = (T + CH - 1) / CH;
    for (int ch = 0; ch < nch; ch++) {
        const int c0 = ch * CH, C = T - c0 < CH ? T - c0 : CH;
        const float *blk = wy + ((size_t)ch * nv + hv) * delta_wy_floats(DK);
        // chunk operands to LDS: W, Q (rows >= C zero), K transposed, L, p, g
        for (int e = tid; e < CH * DK / 4; e += 256) {
            const int i = (4 * e) / DK, n = (4 * e) % DK;
            const float4 w = ldg((const float4 *)blk + e);
            const float4 q = i < C ? ldg((const float4 *)(qn + ((size_t)(c0 + i) * nk + kh) * DK) + n / 4)
                                   : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            const float4 k = i < C ? ldg((const float4 *)(kn + ((size_t)(c0 + i) * nk + kh) * DK) + n / 4)
                                   : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            *(float4 *)(Wc + i * TS + n) = w;
            *(float4 *)(Qc + i * TS + n) = q;
            Kt[(n + 0) * LS + i] = k.x;
            Kt[(n + 1) * LS + i] = k.y;
            Kt[(n + 2) * LS + i] = k.z;
            Kt[(n + 3) * LS + i] = k.w;
        }
        for (int e = tid; e < CH * CH; e += 256) Lc[(e / CH) * LS + e % CH] = ldg(blk + 2 * CH * DK + e);
        if (tid < CH) {
            pc[tid] = ldg(blk + 2 * CH * DK + CH * CH + tid);
            gc[tid] = ldg(blk + 2 * CH * DK + CH * CH + CH + tid);
        }
        __syncthreads();
        // X = W S^T (waves 0, 1: chunk rows 16 t ..) and Y = Q S^T (waves 2, 3)
        const int t = wave & 1;
        const float *Arow = (wave < 2 ? Wc : Qc) + (16 * t + li) * TS + gq * (DK / 4);
        const float *Brow = Ss + li * TS + gq * (DK / 4);
        dm_f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s4 = 0; s4 < DK / 16; s4++) {
            const float4 a = *(const float4 *)(Arow + 4 * s4), b = *(const float4 *)(Brow + 4 * s4);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.x, b.x, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.y, b.y, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.z, b.z, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.w, b.w, acc, 0, 0, 0);
        }
        // D layout: lane l holds rows 4 (l/16) + v (v < 4) of column l % 16
        if (wave < 2) {
            // U = U0 - X, kept transposed for the two products that read it
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int i = 16 * t + 4 * gq + v;
                const float u0 = ldg(blk + CH * DK + (size_t)i * DK + r0 + li);
                Ut[li * LS + i] = u0 - acc[v];
            }
        }
        __syncthreads();
        if (wave >= 2) {
            // O = diag(p) Y + L U for chunk rows 16 t ..
            const float *La = Lc + (16 * t + li) * LS + gq * 8;
            const float *Ub = Ut + li * LS + gq * 8;
            dm_f4 lu = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int s4 = 0; s4 < 2; s4++) {
                const float4 a = *(const float4 *)(La + 4 * s4), b = *(const float4 *)(Ub + 4 * s4);
                lu = __builtin_amdgcn_mfma_f32_16x16x4f32(a.x, b.x, lu, 0, 0, 0);
                lu = __builtin_amdgcn_mfma_f32_16x16x4f32(a.y, b.y, lu, 0, 0, 0);
                lu = __builtin_amdgcn_mfma_f32_16x16x4f32(a.z, b.z, lu, 0, 0, 0);
                lu = __builtin_amdgcn_mfma_f32_16x16x4f32(a.w, b.w, lu, 0, 0, 0);
            }
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int i = 16 * t + 4 * gq + v;
                if (i < C) stg(outp + (size_t)(c0 + i) * vd + hv * DK + r0 + li, (pc[i] * acc[v] + lu[v]) * out_scale);
            }
        }
        // S' = p_{C-1} S + U^T diag(g) K: output tiles of 16 columns, NKT / 4 per wave
        const float pl = pc[C - 1];
#pragma unroll
        for (int q = 0; q < NKT / 4; q++) {
            const int n0 = 16 * (wave * (NKT / 4) + q);
            const float *Ua = Ut + li * LS + gq * 8;
            const float *Kb = Kt + (n0 + li) * LS + gq * 8;
            dm_f4 d = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int s4 = 0; s4 < 2; s4++) {
                const float4 a = *(const float4 *)(Ua + 4 * s4), b = *(const float4 *)(Kb + 4 * s4);
                const float4 g = *(const float4 *)(gc + gq * 8 + 4 * s4);
                d = __builtin_amdgcn_mfma_f32_16x16x4f32(g.x * a.x, b.x, d, 0, 0, 0);
                d = __builtin_amdgcn_mfma_f32_16x16x4f32(g.y * a.y, b.y, d, 0, 0, 0);
                d = __builtin_amdgcn_mfma_f32_16x16x4f32(g.z * a.z, b.z, d, 0, 0, 0);
                d = __builtin_amdgcn_mfma_f32_16x16x4f32(g.w * a.w, b.w, d, 0, 0, 0);
            }
#pragma unroll
            for (int v = 0; v < 4; v++) {
                float *sp = Ss + (4 * gq + v) * TS + n0 + li;
                *sp = pl * *sp + d[v];
            }
        }
        __syncthreads();
    }
    for (int e = tid; e < 16 * DK / 4; e += 256) {
        const int m = (4 * e) / DK, n = (4 * e) % DK;
        stg((float4 *)Sg + e, *(const float4 *)(Ss + m * TS + n));
    }
}
