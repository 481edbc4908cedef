// oh_prefill.hip - layer-major prompt processing (src/ornith_rforward.c:513-682
// structure): every layer runs over a chunk of T tokens before the next, the
// projections as batched matvecs (oh_k_mvb_*), the recurrent parts (conv
// window, delta state, KV cache) advanced in token order. Each per-token
// computation repeats the decode step's arithmetic in the same order, and the
// delta recurrence is stepped token by token, so a prompt processed here gives
// bit-identical logits and state to the same prompt fed through the token
// step (the reference's ORNITH_PREFILL_SERIAL=1 mode). Included into
// oh_kernels.hip after the operation bodies.

// ---- embedding of T tokens: grid (H/256, T), token t at toks[base + t] -----------
extern "C" __global__ void __launch_bounds__(256) oh_k_embed_rows(oh_op_embed a, int base) {
    NoWait w;
    oh_op_embed b = a;
    b.x = a.x + (size_t)blockIdx.y * a.in;
    embed_body(b, (int)blockIdx.x, base + (int)blockIdx.y, w);
}

// ---- causal depthwise conv + SiLU over T tokens (src/ornith_attn.c:370-388) ------
// Thread per (channel, run of tokens): the K-1 inputs before token t come from the
// chunk or, for the first tokens, from the window state (row j = position
// base-(K-1)+j), summed as the decode step sums them. The window the next step
// reads (parity (base+T)&1) receives the last K-1 inputs.
constexpr int kConvRun = 16, kConvKMax = 8;      // tokens per thread, largest kernel width
extern "C" __global__ void __launch_bounds__(256)
oh_k_conv_rows(const float *cat, const float *conv_w, float *conv_state, float *out, int T, int base, int cc, int K) {
    // a thread walks kConvRun tokens of one channel, the K - 1 earlier inputs
    // in registers (K <= kConvKMax); per token the decode step's conv order
    const int c = (int)(blockIdx.x * 256 + tid_x()), t0 = (int)blockIdx.y * kConvRun;
    if (c >= cc) return;
    const int t1 = t0 + kConvRun < T ? t0 + kConvRun : T;
    const float *win = conv_state + (size_t)(base & 1) * (K - 1) * cc;
    float w[kConvKMax], xw[kConvKMax];
#pragma unroll
    for (int j = 0; j < kConvKMax; j++) {
        w[j] = j < K ? ldg(conv_w + (size_t)c * K + j) : 0.0f;
        const int tj = t0 - (K - 1) + j;
        xw[j] = j >= K - 1 ? 0.0f : tj >= 0 ? ldg(cat + (size_t)tj * cc + c) : ldg(win + (size_t)(t0 + j) * cc + c);
    }
    // the run's inputs are requested together (one memory latency per run)
    float xr[kConvRun];
#pragma unroll
    for (int u = 0; u < kConvRun; u++) xr[u] = t0 + u < t1 ? ldg(cat + (size_t)(t0 + u) * cc + c) : 0.0f;
#pragma unroll
    for (int u = 0; u < kConvRun; u++) {
        const int t = t0 + u;
        if (t >= t1) break;
        const float xt = xr[u];
        float acc = 0.0f, wl = 0.0f;
#pragma unroll
        for (int j = 0; j < kConvKMax; j++) {
            if (j < K - 1) acc += w[j] * xw[j];
            if (j == K - 1) wl = w[j];
        }
        acc += wl * xt;
        stg(out + (size_t)t * cc + c, ref_silu(acc));
#pragma unroll
        for (int j = 0; j + 1 < kConvKMax; j++)
            if (j + 1 < K - 1) xw[j] = xw[j + 1];
#pragma unroll
        for (int j = 0; j < kConvKMax; j++)
            if (j == K - 2) xw[j] = xt;
    }
}

// the window after the chunk (a separate launch: the conv above reads the old one)
extern "C" __global__ void __launch_bounds__(256)
oh_k_conv_window(const float *cat, float *conv_state, int T, int base, int cc, int K) {
    const int c = (int)(blockIdx.x * 256 + tid_x()), j = (int)blockIdx.y;   // j < K-1
    if (c >= cc) return;
    const float *win = conv_state + (size_t)(base & 1) * (K - 1) * cc;
    float *nwin = conv_state + (size_t)((base + T) & 1) * (K - 1) * cc;
    const int tj = T - (K - 1) + j;
    const float v = tj >= 0 ? ldg(cat + (size_t)tj * cc + c) : ldg(win + (size_t)(T + j) * cc + c);
    if (nwin != win) stg(nwin + (size_t)j * cc + c, v);
}
// same-parity case (T even): the new window overwrites the old one in place,
// so it is staged first
extern "C" __global__ void __launch_bounds__(256)
oh_k_conv_window_stage(const float *cat, const float *conv_state, float *stage, int T, int base, int cc, int K) {
    const int c = (int)(blockIdx.x * 256 + tid_x()), j = (int)blockIdx.y;
    if (c >= cc) return;
    const float *win = conv_state + (size_t)(base & 1) * (K - 1) * cc;
    const int tj = T - (K - 1) + j;
    stg(stage + (size_t)j * cc + c, tj >= 0 ? ldg(cat + (size_t)tj * cc + c) : ldg(win + (size_t)(T + j) * cc + c));
}

// ---- per (token, key head): L2 norms of q and k; per (token, value head): gates --
// grid (nk + nv, T), one wave: blocks [0, nk) normalise q and k of key head kh
// (double sums of each 64-channel run, the runs added in order, as the decode
// step), blocks [nk, nk+nv) form alpha = exp(ssm_a * softplus(a + dt_bias)) and
// beta = sigmoid(b) of value head hv.
template <int DK>
__global__ void __launch_bounds__(64)
oh_k_qk_gates_rows(const float *conv, const float *A, const float *Bg, const float *ssm_a, const float *dt_bias,
                   float *qn, float *kn, float *al, float *be, int nk, int nv, int cc) {
    constexpr int NQ = DK / 64;
    const int t = (int)blockIdx.y, h = (int)blockIdx.x, lane = lane_id();
    if (h < nk) {
        const int qd = nk * DK;
        const float *cq = conv + (size_t)t * cc + h * DK, *ck = conv + (size_t)t * cc + qd + h * DK;
        float vq[NQ], vk[NQ];
        double tq = 0.0, tk = 0.0;
#pragma unroll
        for (int i = 0; i < NQ; i++) {
            vq[i] = ldg(cq + lane + 64 * i);
            vk[i] = ldg(ck + lane + 64 * i);
        }
#pragma unroll
        for (int i = 0; i < NQ; i++) {
            const double sq = wave_sum_d((double)vq[i] * vq[i]);
            const double sk = wave_sum_d((double)vk[i] * vk[i]);
            tq = i == 0 ? sq : tq + sq;
            tk = i == 0 ? sk : tk + sk;
        }
        const float iq = (float)(1.0 / sqrt(tq + (double)1e-6f));
        const float ik = (float)(1.0 / sqrt(tk + (double)1e-6f));
#pragma unroll
        for (int i = 0; i < NQ; i++) {
            stg(qn + ((size_t)t * nk + h) * DK + lane + 64 * i, vq[i] * iq);
            stg(kn + ((size_t)t * nk + h) * DK + lane + 64 * i, vk[i] * ik);
        }
    } else if (lane == 0) {
        const int hv = h - nk;
        const float av = ldg(A + (size_t)t * nv + hv), bv = ldg(Bg + (size_t)t * nv + hv);
        stg(al + (size_t)t * nv + hv, ref_expf(ldg(ssm_a + hv) * ref_softplus(av + ldg(dt_bias + hv))));
        stg(be + (size_t)t * nv + hv, ref_sigmoid(bv));
    }
}

// ---- the delta recurrence over T tokens (src/ornith_attn.c:198-213) ---------------
// One wave per 64 state rows of value head hv (grid nv * DK/64); each lane
// keeps its row in registers for the whole chunk and steps it token by token
// exactly as the decode step does: s = S*alpha, sk = sum s*k, u = beta(v-sk),
// s += u*k, o = sum s*q (sums in column order). Per token it writes o*scale,
// silu(gate) and the run sum of o^2 over its 64 rows (the gated norm's inputs).
template <int DK>
__global__ void __launch_bounds__(64)
oh_k_delta_scan(const float *qn, const float *kn, const float *conv, const float *al, const float *be,
                float *S, float *out, int T, int nk, int nv, int cc, float out_scale) {
    constexpr int NQ = DK / 64;
    __shared__ __align__(16) float kq[2][2 * DK];              // [buffer][k | q]
    const int lane = lane_id(), vb = (int)blockIdx.x;
    const int hv = vb / NQ, slab = vb % NQ, r = slab * 64 + lane, kh = hv % nk;
    const int qd = nk * DK, vd = nv * DK;
    float *Sr = S + ((size_t)hv * DK + r) * DK;
    float s[DK];
#pragma unroll
    for (int c = 0; c < DK / 4; c++) {
        const float4 v = ldg((const float4 *)Sr + c);
        s[4 * c] = v.x; s[4 * c + 1] = v.y; s[4 * c + 2] = v.z; s[4 * c + 3] = v.w;
    }
    // token t's k and q (uniform over the wave) through LDS, the next token's
    // already requested while t is stepped
    float pk[NQ], pq[NQ], pv, pa, pb;
    auto fetch = [&](int t) {
        const int tc = t < T ? t : T - 1;
#pragma unroll
        for (int i = 0; i < NQ; i++) {
            pk[i] = ldg(kn + ((size_t)tc * nk + kh) * DK + lane + 64 * i);
            pq[i] = ldg(qn + ((size_t)tc * nk + kh) * DK + lane + 64 * i);
        }
        pv = ldg(conv + (size_t)tc * cc + 2 * qd + hv * DK + r);
        pa = ldg(al + (size_t)tc * nv + hv);
        pb = ldg(be + (size_t)tc * nv + hv);
    };
    fetch(0);
    for (int t = 0; t < T; t++) {
        const int bf = t & 1;
#pragma unroll
        for (int i = 0; i < NQ; i++) {
            kq[bf][lane + 64 * i] = pk[i];
            kq[bf][DK + lane + 64 * i] = pq[i];
        }
        const float v = pv, alpha = pa, beta = pb;
        fetch(t + 1);
        wave_lds_sync();
        const float *kk = kq[bf], *qq = kq[bf] + DK;
#pragma unroll
        for (int c = 0; c < DK; c++) s[c] = s[c] * alpha;
        float sk = 0.0f;
#pragma unroll
        for (int c = 0; c < DK; c++) sk += s[c] * kk[c];
        const float u = beta * (v - sk);
#pragma unroll
        for (int c = 0; c < DK; c++) s[c] += u * kk[c];
        float o = 0.0f;
#pragma unroll
        for (int c = 0; c < DK; c++) o += s[c] * qq[c];
        o *= out_scale;
        stg(out + (size_t)t * vd + hv * DK + r, o);
    }
#pragma unroll
    for (int c = 0; c < DK / 4; c++) stg((float4 *)Sr + c, make_float4(s[4 * c], s[4 * c + 1], s[4 * c + 2], s[4 * c + 3]));
}

// ---- chunked delta scan (the reference's default prompt mode) --------------------
// ornith_delta_prefill / delta_chunk (src/ornith_attn.c:215-349): the prompt in
// chunks of kDeltaChunk tokens counted from the start of the evaluation; per
// chunk, with S_in the incoming state,
//   p_i = prod_{l<=i} alpha_l, Sk_i = S_in k_i, Sq_i = S_in q_i,
//   u_i = beta_i v_i - beta_i p_i Sk_i - sum_{j<i} beta_i (p_i/p_j)(k_j.k_i) u_j,
//   o_i = p_i Sq_i + sum_{j<=i} (p_i/p_j)(k_j.q_i) u_j,
//   S_out = p_{C-1} S_in + sum_j (p_{C-1}/p_j) u_j k_j^T,
// where p_i/p_j is accumulated as the running product of alpha_{j+1..i}. Every
// float is formed in the reference's order, so the result equals its bits
// (it differs from the token-by-token recurrence in rounding).
constexpr int kDeltaChunk = 32;

// the chunk Gram matrices, once per (key head, chunk): kk[i][j] = k_j.k_i and
// kq[i][j] = k_j.q_i (ot_dot order: sequential over the head dimension)
template <int DK>
__global__ void __launch_bounds__(256)
oh_k_delta_grams(const float *qn, const float *kn, int T, int nk, float *grams) {
    constexpr int CH = kDeltaChunk, LD = DK + 1;
    __shared__ float ks[CH * LD], qs[CH * LD];
    const int kh = (int)blockIdx.x, ch = (int)blockIdx.y, tid = tid_x();
    const int c0 = ch * CH, C = T - c0 < CH ? T - c0 : CH;
    for (int e = tid; e < CH * DK; e += 256) {
        const int i = e / DK, c = e - i * DK;
        const size_t src = ((size_t)(c0 + (i < C ? i : 0)) * nk + kh) * DK + c;
        ks[i * LD + c] = i < C ? ldg(kn + src) : 0.0f;
        qs[i * LD + c] = i < C ? ldg(qn + src) : 0.0f;
    }
    __syncthreads();
    // pair p < 2*CH*CH: p / (CH*CH) selects kk or kq, then (i, j) = row, column
    constexpr int NP = 2 * CH * CH / 256;
    float acc[NP];
    int ii[NP], jj[NP], wq[NP];
#pragma unroll
    for (int m = 0; m < NP; m++) {
        const int p = tid + 256 * m;
        wq[m] = p / (CH * CH);
        ii[m] = (p % (CH * CH)) / CH;
        jj[m] = p % CH;
        acc[m] = 0.0f;
    }
    for (int c = 0; c < DK; c++) {
#pragma unroll
        for (int m = 0; m < NP; m++) {
            const float a = ks[jj[m] * LD + c];
            const float b = wq[m] ? qs[ii[m] * LD + c] : ks[ii[m] * LD + c];
            acc[m] += a * b;
        }
    }
    float *g = grams + ((size_t)ch * nk + kh) * 2 * CH * CH;
#pragma unroll
    for (int m = 0; m < NP; m++) stg(g + tid + 256 * m, acc[m]);
}

// A block per 16 rows of one value head's state (256 blocks at C3). Thread
// (r, g) = (tid % 16, tid / 16) keeps state row r in registers and takes
// tokens g and g + 16 of each chunk for the S_in projections and the outputs;
// the first 16 threads run the forward substitution of their rows; for the
// state update thread (tid / 16, tid % 16) owns DK / 16 columns of one row in
// LDS (the update is independent per element). Every float is formed in
// delta_chunk's order.
template <int DK>
__global__ void __launch_bounds__(256)
oh_k_delta_chunked(const float *qn, const float *kn, const float *conv, const float *al, const float *be,
                   const float *grams, float *S, float *out, int T, int nk, int nv, int cc, float out_scale) {
    constexpr int CH = kDeltaChunk, RB = 16, KS = DK + 4, XS = DK + 4, CPL = DK / 16;
    __shared__ __align__(16) float kc[CH][KS], qc[CH][KS];
    __shared__ __align__(16) float M[CH][CH + 4], W[CH][CH + 4];   // k_j.k_i / k_j.q_i, then the coefficients
    __shared__ float U[CH][RB + 1], Sq[CH][RB + 1];      // [token][row]
    __shared__ float alpha[CH], beta[CH], p[CH], wend[CH];
    __shared__ int mz[CH];                               // row i of M holds a zero (j < i)
    __shared__ __align__(16) float xs[RB * XS];
    const int tid = tid_x();
    // blocks go to the 8 XCDs round-robin (XCD = block % 8); with nv % 8 == 0
    // the slabs of a head share one XCD and its L2 copy of the head's inputs
    constexpr int NS = DK / RB;
    const int vb = (int)blockIdx.x;
    const int hv = (nv & 7) == 0 ? ((vb >> 3) / NS) * 8 + (vb & 7) : vb / NS;
    const int slab = (nv & 7) == 0 ? (vb >> 3) % NS : vb % NS, kh = hv % nk;
    const int qd = nk * DK, vd = nv * DK, r0 = hv * DK + slab * RB;
    const int r = tid % RB, g = tid / RB;                // projections, outputs, reload
    const int ur = tid / RB, ucg = tid % RB;             // update: row, column group
    float *Srow = S + (size_t)r0 * DK;
    for (int e = tid; e < RB * DK / 4; e += 256) {
        const int row = e / (DK / 4), c4 = e - row * (DK / 4);
        *(float4 *)(xs + row * XS + 4 * c4) = ldg((const float4 *)Srow + e);
    }
    __syncthreads();
    float s[DK];
    auto reload = [&]() {
#pragma unroll
        for (int c = 0; c < DK / 4; c++) {
            const float4 v = *(const float4 *)(xs + r * XS + 4 * c);
            s[4 * c] = v.x; s[4 * c + 1] = v.y; s[4 * c + 2] = v.z; s[4 * c + 3] = v.w;
        }
    };
    // the next chunk's keys, queries, Gram matrices, values and gates are
    // requested into registers while the current chunk is computed
    constexpr int NKQ = CH * DK / 4 / 256, NG = CH * CH / 256, NU = CH * RB / 256;
    float4 rk[NKQ], rq[NKQ];
    float rm[NG], rw[NG], ru[NU], ral = 0.0f, rbe = 0.0f;
    auto fetch = [&](int cs, int chn) {
        const int Cn = T - cs < CH ? T - cs : CH;
        if (Cn <= 0) return;
#pragma unroll
        for (int m = 0; m < NKQ; m++) {
            const int e = tid + 256 * m, i = e / (DK / 4), c = e - i * (DK / 4);
            const size_t src = ((size_t)(cs + (i < Cn ? i : 0)) * nk + kh) * DK;
            rk[m] = ldg((const float4 *)(kn + src) + c);
            rq[m] = ldg((const float4 *)(qn + src) + c);
        }
        const float *gm = grams + ((size_t)chn * nk + kh) * 2 * CH * CH;
#pragma unroll
        for (int m = 0; m < NG; m++) {
            rm[m] = ldg(gm + tid + 256 * m);
            rw[m] = ldg(gm + CH * CH + tid + 256 * m);
        }
        if (tid < Cn) {
            ral = ldg(al + (size_t)(cs + tid) * nv + hv);
            rbe = ldg(be + (size_t)(cs + tid) * nv + hv);
        }
#pragma unroll
        for (int m = 0; m < NU; m++) {
            const int e = tid + 256 * m, i = e / RB, rr = e - i * RB;
            ru[m] = ldg(conv + (size_t)(cs + (i < Cn ? i : 0)) * cc + 2 * qd + r0 + rr);
        }
    };
    fetch(0, 0);
    for (int c0 = 0, ch = 0; c0 < T; c0 += CH, ch++) {
        const int C = T - c0 < CH ? T - c0 : CH;
        __syncthreads();                                 // the previous chunk is consumed
#pragma unroll
        for (int m = 0; m < NKQ; m++) {
            const int e = tid + 256 * m, i = e / (DK / 4), c = e - i * (DK / 4);
            if (i < C) {
                *(float4 *)(&kc[i][4 * c]) = rk[m];
                *(float4 *)(&qc[i][4 * c]) = rq[m];
            }
        }
#pragma unroll
        for (int m = 0; m < NG; m++) {
            const int e = tid + 256 * m;
            M[e / CH][e % CH] = rm[m];
            W[e / CH][e % CH] = rw[m];
        }
        if (tid < C) {
            alpha[tid] = ral;
            beta[tid] = rbe;
        }
#pragma unroll
        for (int m = 0; m < NU; m++) {
            const int e = tid + 256 * m, i = e / RB, rr = e - i * RB;
            if (i < C) U[i][rr] = ru[m];
        }
        fetch(c0 + CH, ch + 1);
        __syncthreads();
        // decay products: thread i owns row i of the coefficient tables, which
        // turn in place into M[i][j] = beta_i (p_i/p_j) k_j.k_i and
        // W[i][j] = (p_i/p_j) k_j.q_i
        // (the gates and row i are read into registers first, so the
        // product chains wait on no LDS read; the same products in the same
        // order as a loop over LDS)
        if (tid < C) {
            const int i = tid;
            float ag[CH], mr[CH], wr[CH];
#pragma unroll
            for (int l = 0; l < CH; l++) ag[l] = alpha[l];
#pragma unroll
            for (int q = 0; q < CH / 4; q++) {
                const float4 vm = *(const float4 *)&M[i][4 * q], vw = *(const float4 *)&W[i][4 * q];
                mr[4 * q] = vm.x; mr[4 * q + 1] = vm.y; mr[4 * q + 2] = vm.z; mr[4 * q + 3] = vm.w;
                wr[4 * q] = vw.x; wr[4 * q + 1] = vw.y; wr[4 * q + 2] = vw.z; wr[4 * q + 3] = vw.w;
            }
            float pi = ag[0];
#pragma unroll
            for (int l = 1; l < CH; l++)
                if (l <= i) pi = pi * ag[l];
            p[i] = pi;
            const float bi = beta[i];
            float ratio = 1.0f;
            int z = 0;
#pragma unroll
            for (int j = CH - 2; j >= 0; j--) {
                if (j < i) {
                    ratio *= ag[j + 1];
                    const float mij = bi * ratio * mr[j];
                    mr[j] = mij;
                    z |= mij == 0.0f;
                    wr[j] = ratio * wr[j];
                }
            }
#pragma unroll
            for (int q = 0; q < CH / 4; q++) {
                *(float4 *)&M[i][4 * q] = float4{mr[4 * q], mr[4 * q + 1], mr[4 * q + 2], mr[4 * q + 3]};
                *(float4 *)&W[i][4 * q] = float4{wr[4 * q], wr[4 * q + 1], wr[4 * q + 2], wr[4 * q + 3]};
            }
            mz[i] = z;
        }
        if (tid == 64) {
            float ag[CH];
#pragma unroll
            for (int l = 0; l < CH; l++) ag[l] = alpha[l];
            float ratio = 1.0f;
#pragma unroll
            for (int j = CH - 1; j >= 0; j--) {
                if (j < C) {
                    wend[j] = ratio;
                    ratio *= ag[j];
                }
            }
        }
        __syncthreads();
        // projections of the incoming state, tokens g and g + 16; U starts as
        // t_i = beta_i v_i - beta_i p_i (S_in k_i); the state row comes from
        // LDS here (it is live only in this phase)
        reload();
        {
            const int i0 = g, i1 = g + RB;
            const int j0 = i0 < C ? i0 : 0, j1 = i1 < C ? i1 : 0;
            float ak0 = 0.0f, aq0 = 0.0f, ak1 = 0.0f, aq1 = 0.0f;
#pragma unroll
            for (int c = 0; c < DK; c++) {
                ak0 += s[c] * kc[j0][c];
                aq0 += s[c] * qc[j0][c];
                ak1 += s[c] * kc[j1][c];
                aq1 += s[c] * qc[j1][c];
            }
            if (i0 < C) {
                U[i0][r] = beta[i0] * U[i0][r] - beta[i0] * p[i0] * ak0;
                Sq[i0][r] = aq0;
            }
            if (i1 < C) {
                U[i1][r] = beta[i1] * U[i1][r] - beta[i1] * p[i1] * ak1;
                Sq[i1][r] = aq1;
            }
        }
        __syncthreads();
        // forward substitution (I + M) U = T, a thread per row, in registers:
        // u_i = (((t_i - m_{i,i-1} u_{i-1}) - m_{i,i-2} u_{i-2}) ...), a term
        // with m = 0 skipped (subtracting an exact +0 leaves u_i's bits as
        // they are, so the zero test sits on the product, off the chain). Row
        // i's coefficients are read into registers before its chain starts.
        if (tid < RB) {
            float u[CH];
#pragma unroll
            for (int i = 0; i < CH; i++) u[i] = i < C ? U[i][tid] : 0.0f;
#pragma unroll
            for (int i = 1; i < CH; i++) {
                if (i < C) {
                    float mr[CH];
#pragma unroll
                    for (int q = 0; q < CH / 4; q++)
                        if (4 * q < i) {
                            const float4 v = *(const float4 *)&M[i][4 * q];
                            mr[4 * q] = v.x; mr[4 * q + 1] = v.y; mr[4 * q + 2] = v.z; mr[4 * q + 3] = v.w;
                        }
                    float ui = u[i];
                    if (__builtin_amdgcn_readfirstlane(mz[i]) == 0) {
#pragma unroll
                        for (int j = i - 1; j >= 0; j--) ui = ui - mr[j] * u[j];
                    } else {
#pragma unroll
                        for (int j = i - 1; j >= 0; j--) {
                            const float pr = mr[j] != 0.0f ? mr[j] * u[j] : 0.0f;
                            ui = ui - pr;
                        }
                    }
                    u[i] = ui;
                }
            }
#pragma unroll
            for (int i = 0; i < CH; i++)
                if (i < C) U[i][tid] = u[i];
        }
        __syncthreads();
        // outputs of tokens g and g + 16, scaled by 1/sqrt(dk): o_i =
        // p_i Sq_i + w_ii u_i + sum_{j<i} w_ij u_j, j descending
        {
            float u[CH];
#pragma unroll
            for (int j = 0; j < CH; j++) u[j] = j < C ? U[j][r] : 0.0f;
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int i = g + RB * h;
                if (i < C) {
                    float wr[CH];
#pragma unroll
                    for (int q = 0; q < CH / 4; q++) {
                        const float4 v = *(const float4 *)&W[i][4 * q];
                        wr[4 * q] = v.x; wr[4 * q + 1] = v.y; wr[4 * q + 2] = v.z; wr[4 * q + 3] = v.w;
                    }
                    float o = p[i] * Sq[i][r];
                    o += W[i][i] * U[i][r];
#pragma unroll
                    for (int j = CH - 1; j >= 0; j--)
                        if (j < i) o += wr[j] * u[j];
                    o *= out_scale;
                    stg(out + (size_t)(c0 + i) * vd + r0 + r, o);
                }
            }
        }
        // S_out = p_{C-1} S_in + sum_j (p_{C-1}/p_j) u_j k_j^T, j descending:
        // CPL columns of row ur
        {
            const float pc = p[C - 1];
            float x[CPL], uw[CH];
            float *xr = xs + ur * XS + ucg * CPL;
#pragma unroll
            for (int j = 0; j < CH; j++) uw[j] = j < C ? wend[j] * U[j][ur] : 0.0f;
#pragma unroll
            for (int c = 0; c < CPL; c++) x[c] = xr[c] * pc;
#pragma unroll
            for (int j = CH - 1; j >= 0; j--) {
                if (j < C) {
                    // the key segment is read whether or not the term is
                    // skipped, so the reads can run ahead of the sums
                    float kk[CPL];
#pragma unroll
                    for (int c4 = 0; c4 < CPL / 4; c4++) {
                        const float4 v = *(const float4 *)&kc[j][ucg * CPL + 4 * c4];
                        kk[4 * c4] = v.x; kk[4 * c4 + 1] = v.y; kk[4 * c4 + 2] = v.z; kk[4 * c4 + 3] = v.w;
                    }
                    const float uj = uw[j];
                    if (uj != 0.0f) {
#pragma unroll
                        for (int c = 0; c < CPL; c++) x[c] += uj * kk[c];
                    }
                }
            }
#pragma unroll
            for (int c = 0; c < CPL; c++) xr[c] = x[c];
        }
    }
    __syncthreads();                                     // every row's update is in LDS
    for (int e = tid; e < RB * DK / 4; e += 256) {
        const int row = e / (DK / 4), c4 = e - row * (DK / 4);
        stg((float4 *)Srow + e, *(const float4 *)(xs + row * XS + 4 * c4));
    }
}

// ---- gated per-head RMSNorm + Q8_K of T vectors (src/ornith_rforward.c:300-319) ---
// one block per token: per head of gdim elements the runs' sums of squares in
// order, inv = 1/sqrt(ss/gdim + eps), v = x * inv * w * silu(z); then Q8_K.
// Dynamic LDS: n floats (n <= 8192), so narrower rows keep more blocks resident.
extern "C" __global__ void __launch_bounds__(256)
oh_k_gnorm_q8k_rows(const float *x, const float *z, const float *w, float eps, int n, int gdim, int8_t *qs,
                    float *d, int16_t *bs, int8_t *bp) {
    extern __shared__ __align__(16) float v[];
    __shared__ float hinv[128];
    __shared__ double runs[128];
    const size_t t = blockIdx.x;
    const int tid = tid_x(), lane = lane_id(), wave = tid >> 6, nh = n / gdim, rpg = gdim / 64, nqb = n / 256;
    // double sums of squares of each 64-element run (the decode step's
    // butterfly over its 64 state rows), then per head the runs in order
    for (int rn = wave; rn < n / 64; rn += 4) {
        const float o = ldg(x + t * n + rn * 64 + lane);
        const double so = wave_sum_d((double)o * o);
        if (lane == 0) runs[rn] = so;
    }
    __syncthreads();
    if (tid < nh) {
        double tot = runs[tid * rpg];
        for (int k = 1; k < rpg; k++) tot += runs[tid * rpg + k];
        hinv[tid] = (float)(1.0 / sqrt(tot / (double)gdim + (double)eps));
    }
    __syncthreads();
    for (int i = tid; i < n; i += 256)
        v[i] = ldg(x + t * n + i) * hinv[i / gdim] * ldg(w + i % gdim) * ref_silu(ldg(z + t * n + i));
    __syncthreads();
    for (int qb = wave; qb < nqb; qb += 4)
        q8k_block_from_lds(v, qb, qs + t * n, d + t * nqb, bs + t * nqb * 16, 256, bp ? bp + t * nqb * 16 : nullptr);
}

// ---- GQA over T tokens: the decode operations with token t at position base+t ----
extern "C" __global__ void __launch_bounds__(256) oh_k_prep_rows(oh_op_prep a, int base) {
    NoWait w;
    const int t = (int)blockIdx.y;
    oh_op_prep b = a;
    b.qproj = a.qproj + (size_t)t * 2 * a.nh * a.hd;
    b.kin = a.kin + (size_t)t * a.nkv * a.hd;
    b.vin = a.vin + (size_t)t * a.nkv * a.hd;
    b.qr = a.qr + (size_t)t * a.nh * a.hd;
    b.gate = a.gate + (size_t)t * a.nh * a.hd;
    prep_body(b, (int)blockIdx.x, base + t, w);
}

// tokens t0 + blockIdx.y; flash partials per token at part + (blockIdx.y) * pstride
// exact walks of the sub-batch's tokens whose context is at most lim (the
// others exit): token t0 + blockIdx.y at position base + t0 + blockIdx.y
// the prompt's exact walks: many rows at once, so fewer V tiles in flight
// per thread and more resident blocks (VGPRs for 6 blocks per CU)
constexpr int kExactRowsVT = 2;
extern "C" __global__ void __launch_bounds__(256, 6) oh_k_attn_exact_rows(oh_op_attn a, int base, int t0) {
    NoWait w;
    const int t = t0 + (int)blockIdx.y, qd = a.nh * a.hd;
    const int lim = a.exact_max < kExactMax ? a.exact_max : kExactMax;
    oh_op_attn b = a;
    b.qr = a.qr + (size_t)t * qd;
    b.gate = a.gate + (size_t)t * qd;
    b.out = a.out + (size_t)t * qd;
    exact_body<NoWait, kExactRowsVT>(b, (int)blockIdx.x, base + t, lim, w);
}

// flash chunks of the n tokens t0.. of a sub-batch: each block stages its KV
// chunk once (up to the last token's context) and runs flash_token for every
// token whose context exceeds lim and reaches the chunk; the per-token
// arithmetic is the decode step's, and the tile positions a token cannot see
// score -inf (exact zeros), so each token's partials equal the decode step's
template <int HB>
__global__ void __launch_bounds__(256)
oh_k_attn_flash_rows(oh_op_attn a, int base, int t0, int n, size_t po_stride, size_t pml_stride) {
    extern __shared__ __align__(16) uint8_t fsm[];
    const int lim = a.exact_max < kExactMax ? a.exact_max : kExactMax;
    const int G = a.nh / a.nkv, ngb = G / HB, gx = a.nkv * ngb;
    const int vb = (int)blockIdx.x, bx = vb % gx, c = vb / gx;
    const int g = bx / ngb, hb0 = (bx % ngb) * HB, tc0 = c * kFlashCh;
    const int Tmax = base + t0 + n, qd = a.nh * a.hd;
    if (Tmax <= lim || tc0 >= Tmax) return;
    const FlashLds<HB> L(fsm, a.hd);
    flash_tile<HB>(a, L, g, tc0, Tmax);
    // the first token that uses this chunk; each token's queries are requested
    // into registers while the previous token computes
    int k = 0;
    while (k < n && (base + t0 + k + 1 <= lim || tc0 >= base + t0 + k + 1)) k++;
    const int tid = tid_x(), nq = HB * a.hd;
    float qv[4];
    auto qload = [&](int kk) {
        const float *src = a.qr + (size_t)(t0 + kk) * qd + ((size_t)g * G + hb0) * a.hd;
#pragma unroll
        for (int m = 0; m < 4; m++) qv[m] = tid + 256 * m < nq ? ldg(src + tid + 256 * m) : 0.0f;
    };
    if (k < n) qload(k);
    for (; k < n; k++) {
#pragma unroll
        for (int m = 0; m < 4; m++)
            if (tid + 256 * m < nq) flash_q_put<HB>(L, a.hd, tid + 256 * m, qv[m]);
        if (k + 1 < n) qload(k + 1);
        flash_token<HB, false, false>(a, L, g, hb0, c, base + t0 + k + 1, nullptr, a.part_o + (size_t)k * po_stride,
                                      a.part_ml + (size_t)k * pml_stride);
        __syncthreads();                                // q and the probabilities are reused
    }
}

extern "C" __global__ void __launch_bounds__(256)
oh_k_attn_combine_rows(oh_op_attn a, int base, int t0, size_t po_stride, size_t pml_stride) {
    NoWait w;
    const int t = t0 + (int)blockIdx.y, qd = a.nh * a.hd;
    oh_op_attn b = a;
    b.gate = a.gate + (size_t)t * qd;
    b.out = a.out + (size_t)t * qd;
    b.part_o = a.part_o + (size_t)blockIdx.y * po_stride;
    b.part_ml = a.part_ml + (size_t)blockIdx.y * pml_stride;
    combine_body(b, (int)blockIdx.x, base + t, w, a.exact_max < kExactMax ? a.exact_max : kExactMax);
}

// ---- MoE over T tokens ------------------------------------------------------------
// routing of token t (one wave): the decode route (src/ornith_moe.c:8-30)
extern "C" __global__ void __launch_bounds__(64)
oh_k_route_rows(const float *logits, int ne, int k, const float *shgate_logit, int32_t *idx, float *w,
                float *shgate) {
    const size_t t = blockIdx.x;
    // 256 / 512 experts: the expert launch's selection (route_fast), the
    // sequential one when a logit is NaN or -inf
    if ((ne == 256 || ne == 512) && k <= 64) {
        const bool ok = ne == 256 ? route_fast<4>(logits + t * ne, k, idx + t * k, w + t * k)
                                  : route_fast<8>(logits + t * ne, k, idx + t * k, w + t * k);
        if (ok) {
            if (lane_id() == 0 && shgate_logit) shgate[t] = ref_sigmoid(shgate_logit[t]);
            return;
        }
    }
    route_wave(logits + t * ne, ne, k, shgate_logit ? shgate_logit + t : nullptr, idx + t * k, w + t * k,
               shgate ? shgate + t : nullptr);
}

// expert lists: pair p = t*k + s goes to list[e*lstride + j] of expert e = idx[p]
// (the order inside a list does not matter: every pair is computed on its own)
extern "C" __global__ void __launch_bounds__(256)
oh_k_group_pairs(const int32_t *idx, int npairs, int32_t *cnt, int ne, int32_t *list, int lstride, int32_t *err) {
    const int p = (int)(blockIdx.x * 256 + tid_x());
    if (p >= npairs) return;
    const int e = ldg(idx + p);
    // an expert index outside [0, ne), or more pairs for one expert than the
    // list holds (a token routed to one expert twice: the fallback pick of a
    // router whose logits are all NaN or -inf), is reported, never written
    if (e < 0 || e >= ne) { atomicOr(err, OH_ERR_EXPERT_LIST); return; }
    const int j = atomicAdd(cnt + e, 1);
    if (j >= lstride) { atomicOr(err, OH_ERR_EXPERT_LIST); return; }
    stg(list + (size_t)e * lstride + j, (int32_t)p);
}

extern "C" __global__ void __launch_bounds__(256) oh_k_fill_i32(int32_t *p, int n, int32_t v) {
    const int i = (int)(blockIdx.x * 256 + tid_x());
    if (i < n) p[i] = v;
}

// x_t += sum_s w_ts * o_ts (s in routing order) + shared * gate_t; grid (H/256, T)
constexpr int kCombineK = 16;                    // slots whose loads are issued together
extern "C" __global__ void __launch_bounds__(256)
oh_k_moe_combine_rows(float *x, const float *o, const float *w, int k, int H, const float *so, const float *shgate) {
    const int i = (int)(blockIdx.x * 256 + tid_x());
    const size_t t = blockIdx.y;
    if (i >= H) return;
    float acc = 0.0f;
    if (k <= kCombineK) {
        // every slot's weight and output requested before the ordered sum
        float ws[kCombineK], os[kCombineK];
#pragma unroll
        for (int s = 0; s < kCombineK; s++) {
            ws[s] = s < k ? ldg(w + t * k + s) : 0.0f;
            os[s] = s < k ? ldg(o + (t * k + s) * H + i) : 0.0f;
        }
#pragma unroll
        for (int s = 0; s < kCombineK; s++)
            if (s < k) acc += ws[s] * os[s];
    } else {
        for (int s = 0; s < k; s++) acc += ldg(w + t * k + s) * ldg(o + (t * k + s) * H + i);
    }
    if (so) {
        const float sv = ldg(so + t * H + i);
        const float v = shgate ? sv * ldg(shgate + t) : sv;
        acc += v;
    }
    stg(x + t * H + i, ldg(x + t * H + i) + acc);
}
