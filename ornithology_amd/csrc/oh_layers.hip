// oh_layers.hip - per-token layer kernels of the decode step (ornith_attn and
// ornith_moe on CDNA4): token embedding, the fused gated delta-net step, GQA
// decode over the Q8 KV cache, the MoE router and combine, and the greedy
// argmax. Included into oh_kernels.hip (single device translation unit).
//
// All float arithmetic follows the reference order (see oh_common.h); the
// places where a reduction order differs from the reference are marked
// "tree-ordered" and only ever concern double-precision sums of squares or of
// softmax terms, which are rounded to float once afterwards.

namespace {

// decode element i of row r of a plane-layout tensor (src/ornith_quant.c)
OH_DEV float dec_elem(const uint8_t *A, const uint8_t *B, const uint8_t *C, int type,
                      int in, int64_t r, int i) {
    if (type == OH_F32) return ldg((const float *)A + r * in + i);
    if (type == OH_F16) return h2f(ldg((const uint16_t *)A + r * in + i));
    if (type == OH_BF16) return u2f((uint32_t)ldg((const uint16_t *)A + r * in + i) << 16);
    const int nb = in / 256, b = i / 256, k = i % 256;
    const int64_t bi = r * nb + b;
    if (type == OH_Q4_K) {
        const uint4 hdr = ldg((const uint4 *)(B + bi * 16));
        const int j = k / 32, l = k % 32;
        const uint8_t q = ldg(A + oh_a_off(OH_Q4_K, bi, 32 * (j / 2) + l));
        int sc, mn;
        q4k_sm(hdr, j, sc, mn);
        const float d1 = h2f((uint16_t)(hdr.x & 0xffffu)) * sc;
        const float m1 = h2f((uint16_t)(hdr.x >> 16)) * mn;
        return d1 * (float)((j & 1) ? (q >> 4) : (q & 15)) - m1;
    }
    if (type == OH_Q6_K) {
        const int hh = k / 128, kk = k % 128, qd = kk / 32, l = kk % 32;
        const uint8_t ql = ldg(A + oh_a_off(OH_Q6_K, bi, 64 * hh + l + 32 * (qd & 1)));
        const uint8_t qh = ldg(A + oh_a_off(OH_Q6_K, bi, 128 + 32 * hh + l));
        const int lo = (qd < 2) ? (ql & 15) : (ql >> 4);
        const int q = (lo | (((qh >> (2 * qd)) & 3) << 4)) - 32;
        const int8_t sc = (int8_t)ldg(B + bi * 16 + 8 * hh + l / 16 + 2 * qd);
        return h2f(ldg((const uint16_t *)(C + bi * 2))) * (float)sc * (float)q;
    }
    if (type == OH_Q8_0)
        return (float)(int8_t)ldg(A + oh_a_off(OH_Q8_0, bi, k)) * h2f(ldg((const uint16_t *)(B + bi * 16 + 2 * (k / 32))));
    if (type == OH_IQ2_XXS) {
        const float dd = h2f(ldg((const uint16_t *)(C + bi * 2)));
        const uint32_t *q = (const uint32_t *)(A + bi * 64);
        const int g32 = k / 32, kk = (k % 32) / 8, j = k % 8;
        const uint32_t w0 = ldg(q + 2 * g32), w1 = ldg(q + 2 * g32 + 1);
        const float db = dd * (0.5f + (float)(w1 >> 28)) * 0.25f;
        const uint64_t gv = k_iq2_grid[(w0 >> (8 * kk)) & 0xffu];
        const uint32_t s7 = (w1 >> (7 * kk)) & 127u;
        const uint32_t sg = s7 | ((__popc(s7) & 1u) << 7);
        return db * (float)((gv >> (8 * j)) & 0xffu) * ((sg >> j) & 1u ? -1.0f : 1.0f);
    }
    return 0.0f;
}

// block-wide (256 threads) double sum, tree-ordered; every thread gets it
OH_DEV double block_sum_d(double v, double *red) {
    v = wave_sum_d(v);
    const int w = (tid_x() >> 6);
    __syncthreads();
    if (lane_id() == 0) red[w] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

} // namespace

// ---- embedding (src/ornith_rforward.c:199-208) --------------------------------
// The token id at toks[pos] was written by an earlier launch (or the host).
template <class W>
OH_DEV void embed_body(const oh_op_embed &a, int vb, int pos, W &w) {
    if (!w.wait()) return;
    const int32_t tok = ldg(a.toks + pos);
    const int i = vb * 256 + tid_x();
    if (i < a.in) stc(a.x + i, dec_elem(a.A, a.B, a.C, a.type, a.in, tok, i));
}

// ---- gated delta-net decode step (src/ornith_rforward.c:457-503,300-319,
//      src/ornith_attn.c:198-213,370-388) -----------------------------------------
// One wave per 64 state rows of one value head (virtual block vb of nv * DK/64;
// in a 256-thread block only wave 0 works, the others take part in the grid
// wait). The state S of value head hv is row-major in HBM (element (r, c) at
// S[hv][r][c], the reference's layout). The wave reads its 64 x DK slab with
// contiguous 16-byte loads, issued first (the state does not depend on the
// previous phase), transposes it through LDS so each lane walks its own row
// in the reference's order, and writes it back the same way. The output is
// o * 1/sqrt(dk) per row, silu(gate) per row and the sum of o^2 over the
// wave's rows; the per-head gated RMSNorm is applied by the consumer (the
// ssm_out projection prologue). The conv window is double-buffered by position
// parity: the step reads window[p] and the channel's single owner writes
// window[1-p], so waves sharing a key head never race. lds: 2*DK + 64*(DK+4)
// floats for the working wave.
template <int DK, int KMAX, class W>
OH_DEV void delta_body(const oh_op_delta &a, int vb, int pos, float *lds, W &w) {
    // TS: LDS row stride padded by 4 floats; with 16-byte accesses every
    // 16-lane pass of a row-per-lane walk and of a coalesced row copy covers
    // all 64 banks once. KMAX >= conv_k bounds the conv taps held in registers.
    constexpr int NQ = DK / 64, TS = DK + 4;
    float *qn = lds, *kn = lds + DK, *tile = lds + 2 * DK;
    const bool act = tid_x() < 64;
    const int lane = lane_id();
    const int nk = a.nk, nv = a.nv, K = a.K, cc = a.cc;
    const int hv = vb / NQ, slab = vb % NQ;
    const int r = slab * 64 + lane, kh = hv % nk, qd = nk * DK;
    const int p = pos & 1;
    const float *win = a.conv_state + (size_t)p * (K - 1) * cc;
    float *nwin = a.conv_state + (size_t)(1 - p) * (K - 1) * cc;
    // channels of a: q channels kh*DK + lane + 64i (i < NQ), k channels
    // likewise, then this row's v channel
    constexpr int NCH = 2 * NQ + 1;
    int ch[NCH];
#pragma unroll
    for (int i = 0; i < NQ; i++) {
        ch[i] = kh * DK + lane + 64 * i;
        ch[NQ + i] = qd + kh * DK + lane + 64 * i;
    }
    ch[2 * NQ] = 2 * qd + hv * DK + r;
    // everything that does not depend on the previous phase is requested
    // before the grid wait: the state slab (rows [slab*64, +64) of head hv,
    // contiguous), the conv weights and window, ssm_a and dt_bias
    float4 st[DK / 4];
    float cw[NCH][KMAX], wv[NCH][KMAX], sa = 0.0f, dtb = 0.0f;
    if (act) {
        const float4 *Sr = (const float4 *)(a.S + ((size_t)hv * DK + slab * 64) * DK);
#pragma unroll
        for (int i = 0; i < DK / 4; i++) st[i] = ldg(Sr + lane + 64 * i);
#pragma unroll
        for (int c = 0; c < NCH; c++) {
            if (KMAX == 4 && K == 4) {
                const float4 c4 = ldg((const float4 *)(a.conv_w + (size_t)ch[c] * 4));
                cw[c][0] = c4.x; cw[c][1] = c4.y; cw[c][2] = c4.z; cw[c][3] = c4.w;
            } else {
#pragma unroll
                for (int j = 0; j < KMAX; j++) cw[c][j] = j < K ? ldg(a.conv_w + (size_t)ch[c] * K + j) : 0.0f;
            }
#pragma unroll
            for (int j = 0; j < KMAX; j++) wv[c][j] = j < K - 1 ? ldg(win + (size_t)j * cc + ch[c]) : 0.0f;
        }
        sa = ldg(a.ssm_a + hv);
        dtb = ldg(a.dt_bias + hv);
    }
    if (!w.wait() || !act) return;
    // then this step's inputs from the input projection
    float cx[NCH];
#pragma unroll
    for (int c = 0; c < NCH; c++) cx[c] = ldw<W::kGrid>(a.cat + ch[c]);
    const float av = ldw<W::kGrid>(a.ab + hv), bv = ldw<W::kGrid>(a.ab + nv + hv);
    const float gz = ldw<W::kGrid>(a.gate + (size_t)hv * DK + r);
    // slab -> LDS, row-padded (frees the slab's registers for the step)
#pragma unroll
    for (int i = 0; i < DK / 4; i++) {
        const int f = lane + 64 * i, row = (4 * f) / DK, col = (4 * f) % DK;
        *(float4 *)(tile + row * TS + col) = make_float4(st[i].x, st[i].y, st[i].z, st[i].w);
    }

    // causal depthwise conv (no bias) + SiLU
    float cv[NCH];
#pragma unroll
    for (int c = 0; c < NCH; c++) {
        float acc = 0.0f, wl = 0.0f;
#pragma unroll
        for (int j = 0; j < KMAX; j++) {
            if (j < K - 1) acc += cw[c][j] * wv[c][j];
            if (j == K - 1) wl = cw[c][j];
        }
        acc += wl * cx[c];
        cv[c] = ref_silu(acc);
        const bool owner = c == 2 * NQ || (hv < nk && slab == 0);
        if (owner) {
#pragma unroll
            for (int j = 0; j + 1 < KMAX; j++)
                if (j + 1 < K - 1) stg(nwin + (size_t)j * cc + ch[c], wv[c][j + 1]);
            stg(nwin + (size_t)(K - 2) * cc + ch[c], cx[c]);
        }
    }
    // per-head L2 normalisation of q and k (src/ornith_tensor.c:155-160):
    // double sums of each 64-channel run (butterfly), then the runs in order
    double tq = 0.0, tk = 0.0;
#pragma unroll
    for (int i = 0; i < NQ; i++) {
        const double sq = wave_sum_d((double)cv[i] * cv[i]);
        const double sk = wave_sum_d((double)cv[NQ + i] * cv[NQ + i]);
        tq = i == 0 ? sq : tq + sq;
        tk = i == 0 ? sk : tk + sk;
    }
    const float iq = (float)(1.0 / sqrt(tq + (double)1e-6f));
    const float ik = (float)(1.0 / sqrt(tk + (double)1e-6f));
#pragma unroll
    for (int i = 0; i < NQ; i++) {
        qn[lane + 64 * i] = cv[i] * iq;
        kn[lane + 64 * i] = cv[NQ + i] * ik;
    }
    const float alpha = ref_expf(sa * ref_softplus(av + dtb));
    const float beta = ref_sigmoid(bv);
    wave_lds_sync();

    // the lane's row in registers: s = S * alpha; sk = sum_c s_c k_c; then
    // s_c += u k_c and o = sum_c s_c q_c, each sum in column order
    float *tr = tile + lane * TS;
    float sr[DK];
#pragma unroll
    for (int c = 0; c < DK / 4; c++) {
        const float4 v = *(const float4 *)(tr + 4 * c);
        sr[4 * c + 0] = v.x * alpha;
        sr[4 * c + 1] = v.y * alpha;
        sr[4 * c + 2] = v.z * alpha;
        sr[4 * c + 3] = v.w * alpha;
    }
    float sk = 0.0f;
#pragma unroll
    for (int c = 0; c < DK / 4; c++) {
        const float4 kk = *(const float4 *)(kn + 4 * c);
        sk += sr[4 * c + 0] * kk.x;
        sk += sr[4 * c + 1] * kk.y;
        sk += sr[4 * c + 2] * kk.z;
        sk += sr[4 * c + 3] * kk.w;
    }
    const float u = beta * (cv[2 * NQ] - sk);
    float o = 0.0f;
#pragma unroll
    for (int c = 0; c < DK / 4; c++) {
        const float4 kk = *(const float4 *)(kn + 4 * c), qq = *(const float4 *)(qn + 4 * c);
        sr[4 * c + 0] += u * kk.x;
        sr[4 * c + 1] += u * kk.y;
        sr[4 * c + 2] += u * kk.z;
        sr[4 * c + 3] += u * kk.w;
        o += sr[4 * c + 0] * qq.x;
        o += sr[4 * c + 1] * qq.y;
        o += sr[4 * c + 2] * qq.z;
        o += sr[4 * c + 3] * qq.w;
        *(float4 *)(tr + 4 * c) = make_float4(sr[4 * c], sr[4 * c + 1], sr[4 * c + 2], sr[4 * c + 3]);
    }
    wave_lds_sync();
    float4 *Sw = (float4 *)(a.S + ((size_t)hv * DK + slab * 64) * DK);
#pragma unroll
    for (int i = 0; i < DK / 4; i++) {
        const int f = lane + 64 * i, row = (4 * f) / DK, col = (4 * f) % DK;
        stg(Sw + f, *(const float4 *)(tile + row * TS + col));
    }
    // the gated RMSNorm's inputs for the consumer: o, silu(gate) and the
    // butterfly double sum of o^2 over this wave's 64 rows
    o *= a.out_scale;
    const double so = wave_sum_d((double)o * o);
    stc(a.out + (size_t)hv * DK + r, o);
    stc(a.out_gate + (size_t)hv * DK + r, ref_silu(gz));
    if (lane == 0) stc(a.out_runs + vb, so);
}

// ---- the same decode step, 16 state rows per 256-thread block --------------------
// delta_body's arithmetic spread over four times as many blocks with four
// waves each: virtual block vb of nv * DK/16 takes rows [slab*16, +16) of
// value head hv (256 blocks at C3). Every thread loads two float4 of the
// 16 x DK state slab (contiguous, coalesced) before anything else and keeps
// them in registers. Waves 0 and 1 form the conv + SiLU + L2 norm of the key
// head's q and k channels (a lane per channel, lane + 64 i, as delta_body's
// wave), wave 2's lanes 0..15 the 16 rows' v channels and silu(gate), wave 3's
// lane 0 alpha and beta. The delta rule per row (s_c = S_c * alpha,
// sk = sum s_c k_c, u = beta (v - sk), s_c += u k_c, o = sum s_c q_c, the
// sums in column order) then runs as: every thread forms the products of its
// eight elements (s_c k_c, later s_c q_c after the update, which it also
// stores as the new state) into an LDS tile, and lanes 0..15 of wave 0 add
// their row's products in column order; the same floats as delta_body's row
// walk, with the chains reduced to adds. The sum of o^2 is left as 16-row
// partials (row16_sum_d), whose (g0 + g1) + (g2 + g3) is delta_body's 64-row
// run sum.
// The conv window is double-buffered by position parity as in delta_body;
// its q/k channels are written by slab 0 of value head kh (hv < nk).
// lds: delta16_lds_floats(DK) floats.
OH_HD constexpr int delta16_lds_floats(int dk) { return 2 * dk + 2 * 16 + 4 + 16 * (dk + 4); }

template <int DK, int KMAX, class W>
OH_DEV void delta16_body(const oh_op_delta &a, int vb, int pos, float *lds, W &w) {
    constexpr int NQ = DK / 64, TS = DK + 4, RB = 16, NF = RB * DK / 4 / 256;
    static_assert(NF >= 1 && RB * DK / 4 % 256 == 0, "16 rows of DK columns: whole float4 per thread");
    float *qn = lds, *kn = lds + DK, *vrow = lds + 2 * DK, *urow = vrow + RB, *coef = urow + RB;
    float *tile = coef + 4;                               // [RB][TS], 16-byte aligned
    const int tid = tid_x(), lane = tid & 63, wave = tid >> 6;
    const int nk = a.nk, nv = a.nv, K = a.K, cc = a.cc, qd = nk * DK;
    const int hv = vb / (DK / RB), slab = vb % (DK / RB), kh = hv % nk;
    const int r0 = slab * RB;                             // first row (within the head)
    const int p = pos & 1;
    const float *win = a.conv_state + (size_t)p * (K - 1) * cc;
    float *nwin = a.conv_state + (size_t)(1 - p) * (K - 1) * cc;
    // the state slab first (it does not depend on the previous phase)
    const float4 *Sr = (const float4 *)(a.S + ((size_t)hv * DK + r0) * DK);
    float4 st[NF];
#pragma unroll
    for (int i = 0; i < NF; i++) st[i] = ldg(Sr + tid + 256 * i);
    // this lane's conv channels: q (wave 0) or k (wave 1) channels of key
    // head kh, lane + 64 i; the v channel of row lane (wave 2, lanes < 16)
    const bool qk = wave < 2, vl = wave == 2 && lane < RB;
    int ch[NQ];
#pragma unroll
    for (int i = 0; i < NQ; i++)
        ch[i] = qk ? (wave == 0 ? 0 : qd) + kh * DK + lane + 64 * i : 2 * qd + hv * DK + r0 + (lane & (RB - 1));
    float cw[NQ][KMAX] = {}, wv[NQ][KMAX] = {}, sa = 0.0f, dtb = 0.0f;
    if (qk || vl) {
#pragma unroll
        for (int i = 0; i < NQ; i++) {
            if (i > 0 && !qk) break;
            if (KMAX == 4 && K == 4) {
                const float4 c4 = ldg((const float4 *)(a.conv_w + (size_t)ch[i] * 4));
                cw[i][0] = c4.x; cw[i][1] = c4.y; cw[i][2] = c4.z; cw[i][3] = c4.w;
            } else {
#pragma unroll
                for (int j = 0; j < KMAX; j++) cw[i][j] = j < K ? ldg(a.conv_w + (size_t)ch[i] * K + j) : 0.0f;
            }
#pragma unroll
            for (int j = 0; j < KMAX; j++) wv[i][j] = j < K - 1 ? ldg(win + (size_t)j * cc + ch[i]) : 0.0f;
        }
    }
    if (wave == 3 && lane == 0) {
        sa = ldg(a.ssm_a + hv);
        dtb = ldg(a.dt_bias + hv);
    }
    if (!w.wait()) return;
    // this step's inputs from the input projection
    float cx[NQ];
#pragma unroll
    for (int i = 0; i < NQ; i++) cx[i] = (qk || (vl && i == 0)) ? ldw<W::kGrid>(a.cat + ch[i]) : 0.0f;
    const float gz = vl ? ldw<W::kGrid>(a.gate + (size_t)hv * DK + r0 + lane) : 0.0f;
    float av = 0.0f, bv = 0.0f;
    if (wave == 3 && lane == 0) {
        av = ldw<W::kGrid>(a.ab + hv);
        bv = ldw<W::kGrid>(a.ab + nv + hv);
    }
    // causal depthwise conv (no bias) + SiLU, in delta_body's order
    float cv[NQ];
#pragma unroll
    for (int i = 0; i < NQ; i++) {
        float acc = 0.0f, wl = 0.0f;
#pragma unroll
        for (int j = 0; j < KMAX; j++) {
            if (j < K - 1) acc += cw[i][j] * wv[i][j];
            if (j == K - 1) wl = cw[i][j];
        }
        acc += wl * cx[i];
        cv[i] = ref_silu(acc);
    }
    const bool owner = vl || (qk && hv < nk && slab == 0);
    if (owner) {
#pragma unroll
        for (int i = 0; i < NQ; i++) {
            if (i > 0 && !qk) break;
#pragma unroll
            for (int j = 0; j + 1 < KMAX; j++)
                if (j + 1 < K - 1) stg(nwin + (size_t)j * cc + ch[i], wv[i][j + 1]);
            stg(nwin + (size_t)(K - 2) * cc + ch[i], cx[i]);
        }
    }
    if (qk) {
        // per-head L2 normalisation (src/ornith_tensor.c:155-160): double
        // sums of each 64-channel run, then the runs in order
        double t = 0.0;
#pragma unroll
        for (int i = 0; i < NQ; i++) {
            const double sq = wave_sum_d((double)cv[i] * cv[i]);
            t = i == 0 ? sq : t + sq;
        }
        const float inv = (float)(1.0 / sqrt(t + (double)1e-6f));
        float *dst = wave == 0 ? qn : kn;
#pragma unroll
        for (int i = 0; i < NQ; i++) dst[lane + 64 * i] = cv[i] * inv;
    } else if (vl) {
        vrow[lane] = cv[0];
        stc(a.out_gate + (size_t)hv * DK + r0 + lane, ref_silu(gz));
    } else if (wave == 3 && lane == 0) {
        coef[0] = ref_expf(sa * ref_softplus(av + dtb));
        coef[1] = ref_sigmoid(bv);
    }
    __syncthreads();
    // the products each row walk adds are formed element-parallel (every
    // thread its eight elements), so the two ordered sums are adds only:
    // pk_c = (S_c * alpha) * k_c into the tile
    const float alpha = coef[0];
    float4 sa4[NF];
#pragma unroll
    for (int i = 0; i < NF; i++) {
        const int f = tid + 256 * i, row = (4 * f) / DK, col = (4 * f) % DK;
        const float4 x = st[i], kk = *(const float4 *)(kn + col);
        sa4[i] = make_float4(x.x * alpha, x.y * alpha, x.z * alpha, x.w * alpha);
        *(float4 *)(tile + row * TS + col) =
            make_float4(sa4[i].x * kk.x, sa4[i].y * kk.y, sa4[i].z * kk.z, sa4[i].w * kk.w);
    }
    __syncthreads();
    // sk = sum_c pk_c in column order; u = beta (v - sk)
    if (wave == 0 && lane < RB) {
        const float *tr = tile + lane * TS;
        float sk = 0.0f;
#pragma unroll
        for (int c = 0; c < DK / 4; c++) {
            const float4 t = *(const float4 *)(tr + 4 * c);
            sk += t.x;
            sk += t.y;
            sk += t.z;
            sk += t.w;
        }
        urow[lane] = coef[1] * (vrow[lane] - sk);
    }
    __syncthreads();
    // s_c += u k_c (the new state, stored) and po_c = s_c q_c into the tile
    float4 *Sw = (float4 *)(a.S + ((size_t)hv * DK + r0) * DK);
#pragma unroll
    for (int i = 0; i < NF; i++) {
        const int f = tid + 256 * i, row = (4 * f) / DK, col = (4 * f) % DK;
        const float u = urow[row];
        const float4 kk = *(const float4 *)(kn + col), qq = *(const float4 *)(qn + col);
        float s0 = sa4[i].x, s1 = sa4[i].y, s2 = sa4[i].z, s3 = sa4[i].w;
        s0 += u * kk.x;
        s1 += u * kk.y;
        s2 += u * kk.z;
        s3 += u * kk.w;
        stg(Sw + f, make_float4(s0, s1, s2, s3));
        *(float4 *)(tile + row * TS + col) = make_float4(s0 * qq.x, s1 * qq.y, s2 * qq.z, s3 * qq.w);
    }
    __syncthreads();
    // o = sum_c po_c in column order
    if (wave == 0) {
        float o = 0.0f;
        if (lane < RB) {
            const float *tr = tile + lane * TS;
#pragma unroll
            for (int c = 0; c < DK / 4; c++) {
                const float4 t = *(const float4 *)(tr + 4 * c);
                o += t.x;
                o += t.y;
                o += t.z;
                o += t.w;
            }
            o *= a.out_scale;
            stc(a.out + (size_t)hv * DK + r0 + lane, o);
        }
        const double g = row16_sum_d(lane < RB ? (double)o * o : 0.0);
        if (lane == 0) stc(a.out_runs + vb, g);
    }
}

// ---- GQA decode (src/ornith_rforward.c:419-455, src/ornith_attn.c:65-149) -------
// prep: per-head RMSNorm + partial NeoX RoPE (cos/sin from a host-built table
// of the reference's powf/cosf/sinf values), Q8 append of k and v at `pos`.
// Virtual blocks [0, nh) are query heads, [nh, nh+nkv) key/value heads.
// K codes are stored as [kvh][hd/4][cap] 32-bit words (4 codes each, so a
// lane per position reads coalesced words); V codes as [kvh][cap/16][hd][16]
// tiles (a lane per element reads 16 consecutive positions in one 16-byte
// load). cap is a multiple of 16.
template <class W>
OH_DEV void prep_body(const oh_op_prep &a, int vb, int pos, W &w) {
    __shared__ float v[256];
    __shared__ double red[4];
    __shared__ float amax_s[4];
    if (!w.wait()) return;
    const int hb = vb, t = tid_x();
    const int nh = a.nh, nkv = a.nkv, hd = a.hd, cap = a.cap;
    const bool isq = hb < nh;
    const int h = isq ? hb : hb - nh;
    const int r = a.rot <= 0 || a.rot > hd ? hd : a.rot;
    const int half = r / 2;
    // every input is requested before the first reduction: the head's
    // values, its norm weight, the RoPE (cos, sin) of this element's pair,
    // and the gate (query heads) or the raw v (kv heads)
    const float *src = isq ? a.qproj + (size_t)h * 2 * hd : a.kin + (size_t)h * hd;
    const float *nw = isq ? a.q_norm : a.k_norm;
    const float2 *rope = (const float2 *)a.rope;
    const float x = t < hd ? ldw<W::kGrid>(src + t) : 0.0f;
    const float nwt = t < hd ? ldg(nw + t) : 0.0f;
    const int pi = t < half ? t : t - half;
    const float2 cs = t < 2 * half ? ldg(rope + (size_t)pos * (hd / 2) + pi) : make_float2(1.0f, 0.0f);
    const float other = t < hd ? (isq ? ldw<W::kGrid>(a.qproj + (size_t)h * 2 * hd + hd + t)
                                      : ldw<W::kGrid>(a.vin + (size_t)h * hd + t))
                               : 0.0f;
    double ss = block_sum_d((double)x * x, red);
    const float inv = (float)(1.0 / sqrt(ss / (double)hd + (double)a.eps));
    if (t < hd) v[t] = x * inv * nwt;
    __syncthreads();
    float y = t < hd ? v[t] : 0.0f;
    if (t < half) {
        y = v[t] * cs.x - v[t + half] * cs.y;
    } else if (t >= half && t < 2 * half) {
        y = v[t - half] * cs.y + v[t] * cs.x;
    }
    if (isq) {
        if (t < hd) {
            stc(a.qr + (size_t)h * hd + t, y);
            stc(a.gate + (size_t)h * hd + t, other);
        }
        return;
    }
    // Q8 encode of k (post norm/rope) and raw v (src/ornith_attn.c:65-77)
    for (int which = 0; which < 2; which++) {
        const float val = which == 0 ? y : other;
        float am = wave_max_f(fabsf(val));
        __syncthreads();
        if (lane_id() == 0) amax_s[t >> 6] = am;
        __syncthreads();
        const float amax = fmaxf(fmaxf(amax_s[0], amax_s[1]), fmaxf(amax_s[2], amax_s[3]));
        int code = 0;
        float scale = 0.0f;
        if (amax != 0.0f) {
            scale = amax / 127.0f;
            const float iv = 127.0f / amax;
            int q = (int)__builtin_rintf(val * iv);
            code = q > 127 ? 127 : (q < -127 ? -127 : q);
        }
        const size_t off = (size_t)pos * nkv + h;
        if (which == 0) {
            // pack 4 consecutive codes into one word of Kt[h][t/4][pos]
            const int c0 = shfl(code, (lane_id() & ~3) + 0), c1 = shfl(code, (lane_id() & ~3) + 1);
            const int c2 = shfl(code, (lane_id() & ~3) + 2), c3 = shfl(code, (lane_id() & ~3) + 3);
            if (t < hd && (t & 3) == 0)
                stc(a.Kt + ((size_t)h * (hd / 4) + t / 4) * cap + pos,
                    (uint32_t)(c0 & 0xff) | ((uint32_t)(c1 & 0xff) << 8) |
                    ((uint32_t)(c2 & 0xff) << 16) | ((uint32_t)(c3 & 0xff) << 24));
            if (t == 0) stc(a.Ks + off, scale);
        } else {
            // tiles of 16 positions: Vq[h][pos/16][i][pos%16], and Vh the same as f16
            const size_t vo = (((size_t)h * (cap / 16) + pos / 16) * hd + t) * 16 + (pos & 15);
            if (t < hd) stc(a.Vq + vo, (int8_t)code);
            if (t < hd && a.Vh) stc(a.Vh + vo, f16_bits_of_code(code));
            if (t == 0) stc(a.Vs + off, scale);
        }
    }
}

// KV entries at earlier positions were written by earlier launches; the one
// at `pos` by the prep phase of this launch with device-scope stores, before
// any workgroup of this launch read its cache line. Plain loads therefore see
// every entry.

// Longest context of the prompt's exact rows (their scores stay in LDS).
constexpr int kExactMax = 2048;
// Longest context of the decode step's exact walk for head dim hd: the
// scores of the block's 256/hd heads stay in LDS, at most 48 KB of it
// (8192 positions at hd 256, 6144 at 128, 3072 at 64).
OH_HD inline int exact_cap(int hd) {
    const int c = 12288 * hd / 256;
    return c < 8192 ? c : 8192;
}
// the decode step's exact-walk limit for a session's exact_max
OH_HD inline int exact_lim(int exact_max, int hd) {
    const int c = exact_cap(hd);
    return exact_max < c ? (exact_max > 0 ? exact_max : 0) : c;
}

// Exact GQA output of the block's 256/hd query heads (virtual block g):
// scores s_t = (sum_i q_i*code_i) * Ks_t * scale, sequential over i
// (src/ornith_attn.c:80-85,119-122), kept in LDS; softmax over T
// (src/ornith_tensor.c:108-115; tree-ordered double sum) and the output
// o_i = sum_t (p_t*Vs_t)*code_t,i, sequential over t, skipping zero weights
// (src/ornith_attn.c:132-140); then o *= sigmoid(gate).
// VT: tiles of 16 V positions in flight per thread (the decode step's single
// row keeps 8; the prompt's many rows keep fewer, for occupancy)
template <class W, int VT = 8>
OH_DEV void exact_body(const oh_op_attn &a, int vb, int pos, int lim, W &w) {
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ float q[256];
    __shared__ float pbuf[4][256];
    __shared__ float inv_s[4], mx_s[4];
    __shared__ double red[4];
    __shared__ float mred[4];
    const int nh = a.nh, nkv = a.nkv, hd = a.hd, cap = a.cap;
    const int hpb = 256 / hd, t = tid_x(), g = vb;
    const int T = pos + 1;
    if (T > lim || g * hpb >= nh) return;
    if (!w.wait()) return;
    float *sc = (float *)smem;                               // [hpb][lim]
    q[t] = ldc(a.qr + (size_t)g * 256 + t);                  // the block's heads are contiguous
    __syncthreads();
    for (int hl = 0; hl < hpb; hl++) {
        const int kvh = (g * hpb + hl) / (nh / nkv);
        const float *qh = q + hl * hd;
        for (int t0 = 0; t0 < T; t0 += 256) {
            const int tt = t0 + t;
            if (tt < T) {
                const uint32_t *kw = a.Kt + (size_t)kvh * (hd / 4) * cap + tt;
                float acc = 0.0f;
                for (int w0 = 0; w0 < hd / 4; w0 += 16) {
                    uint32_t wd[16];
#pragma unroll
                    for (int u = 0; u < 16; u++) wd[u] = w0 + u < hd / 4 ? ldg(kw + (size_t)(w0 + u) * cap) : 0u;
#pragma unroll
                    for (int u = 0; u < 16; u++) {
                        if (w0 + u >= hd / 4) break;
                        const int wi = w0 + u;
                        acc += qh[4 * wi + 0] * (float)(int8_t)(wd[u] & 0xff);
                        acc += qh[4 * wi + 1] * (float)(int8_t)((wd[u] >> 8) & 0xff);
                        acc += qh[4 * wi + 2] * (float)(int8_t)((wd[u] >> 16) & 0xff);
                        acc += qh[4 * wi + 3] * (float)(int8_t)(wd[u] >> 24);
                    }
                }
                const float ks = ldg(a.Ks + (size_t)tt * nkv + kvh);
                const float v = ks == 0.0f ? 0.0f : acc * ks;
                sc[hl * lim + tt] = v * a.scale;
            }
        }
    }
    __syncthreads();
    for (int hl = 0; hl < hpb; hl++) {
        const float *sh = sc + hl * lim;
        float mx = -INFINITY;
        for (int i = t; i < T; i += 256) mx = fmaxf(mx, sh[i]);
        mx = wave_max_f(mx);
        __syncthreads();
        if (lane_id() == 0) mred[t >> 6] = mx;
        __syncthreads();
        mx = fmaxf(fmaxf(mred[0], mred[1]), fmaxf(mred[2], mred[3]));
        double sum = 0.0;
        for (int i = t; i < T; i += 256) sum += ref_expf(sh[i] - mx);
        sum = block_sum_d(sum, red);
        if (t == 0) { mx_s[hl] = mx; inv_s[hl] = (float)(1.0 / sum); }
    }
    const int hl = t / hd, i = t % hd, h = g * hpb + hl;
    const int kvh = h / (nh / nkv);
    const uint4 *vt = (const uint4 *)a.Vq + (size_t)kvh * (cap / 16) * hd + i;
    float o = 0.0f;
    for (int t0 = 0; t0 < T; t0 += 256) {
        const int n = T - t0 < 256 ? T - t0 : 256;
        __syncthreads();
        for (int k = t; k < hpb * 256; k += 256) {
            const int hh = k / 256, tt = k % 256;
            const int hg = g * hpb + hh, kv2 = hg / (nh / nkv);
            if (tt < n) {
                const float p = ref_expf(sc[hh * lim + t0 + tt] - mx_s[hh]) * inv_s[hh];
                pbuf[hh][tt] = p * ldg(a.Vs + (size_t)(t0 + tt) * nkv + kv2);
            }
        }
        __syncthreads();
        // tiles of 16 positions, VT tiles in flight, adds in position order
        for (int k0 = 0; k0 < n; k0 += 16 * VT) {
            uint4 cw[VT];
#pragma unroll
            for (int u = 0; u < VT; u++) {
                const int tile = k0 + 16 * u < n ? k0 + 16 * u : ((n - 1) & ~15);
                cw[u] = ldg(vt + (size_t)((t0 + tile) / 16) * hd);
            }
#pragma unroll
            for (int u = 0; u < VT; u++) {
#pragma unroll
                for (int j = 0; j < 16; j++) {
                    const int k = k0 + 16 * u + j;
                    const int8_t c = (int8_t)(wsel(cw[u], j >> 2) >> (8 * (j & 3)));
                    // the reference skips zero weights; o starts at +0 and a
                    // round-to-nearest sum is -0 only when both addends are,
                    // so o is never -0 and adding 0 * c = +-0 leaves its bits
                    // unchanged: the plain sum equals the skipping one
                    const float sv = k < n ? pbuf[hl][k] : 0.0f;
                    o = o + sv * (float)c;
                }
            }
        }
    }
    stc(a.out + (size_t)h * hd + i, o * ref_sigmoid(ldc(a.gate + (size_t)h * hd + i)));
}

// ---- the exact walk in two launches (the decode step's graph path) ----------------
// The same arithmetic as exact_body, with the scores spread over many blocks:
// exact_scores_body writes s_t = (sum_i q_i*code_i) * Ks_t * scale of every
// query head to a.scores [nh][cap]; exact_walk_body (one block per query
// head) takes the softmax over them and the output walk in position order.

// Scores of KV head g's query heads for the 64 positions of tile c
// (vb = c * nkv + g), 512 threads: the tile's key words and the group's
// queries go to LDS; lane = position, wave w takes the HPW heads from
// w * HPW on (HPW * 8 >= nh / nkv); each dot sequential over i as in
// exact_body.
template <int HW, int HPW, class W>
OH_DEV void exact_scores_hw(const oh_op_attn &a, int vb, int pos, W &w) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int nh = a.nh, nkv = a.nkv, hd = 4 * HW, cap = a.cap, G = nh / nkv;
    const int g = vb % nkv, c = vb / nkv, T = pos + 1;
    const int tid = tid_x(), lane = lane_id(), wave = tid >> 6;
    const int t = c * 64 + lane;
    const int tc = t < T ? t : T - 1;
    if (!w.wait()) return;
    uint32_t *kt = (uint32_t *)smem;                          // [HW][64]
    float4 *q = (float4 *)(smem + HW * 64 * 4);               // [G][hd / 4]
    {
        // wave w loads words w, w + 8, ... of the tile's 64 positions; the
        // group's queries (at most OH_EXACT2_GMAX * hd floats) load at the
        // same time, every load issued before any is used
        const uint32_t *kw = a.Kt + (size_t)g * HW * cap + tc;
        uint32_t wd[HW / 8];
#pragma unroll
        for (int k = 0; k < HW / 8; k++) wd[k] = ldg(kw + (size_t)(wave + 8 * k) * cap);
        constexpr int QR = OH_EXACT2_GMAX * HW / 512;          // float4 per thread
        const int n4 = G * HW;
        const float4 *qs = (const float4 *)(a.qr + (size_t)g * G * hd);
        float4 qv[QR];
#pragma unroll
        for (int r = 0; r < QR; r++) qv[r] = ldg(qs + (tid + 512 * r < n4 ? tid + 512 * r : 0));
#pragma unroll
        for (int k = 0; k < HW / 8; k++) kt[(wave + 8 * k) * 64 + lane] = wd[k];
#pragma unroll
        for (int r = 0; r < QR; r++) if (tid + 512 * r < n4) q[tid + 512 * r] = qv[r];
    }
    const float ks = ldg(a.Ks + (size_t)tc * nkv + g);
    // the tile's f16 value codes (4 tiles of 16 positions: 2 * hd / 128
    // uint4 per thread), loaded here only so that the walk, which reads them
    // next, finds them in the caches; consumed by an empty asm at the end
    constexpr int VR = HW / 16;
    uint32_t vk[VR];
    {
        const uint4 *vt = (const uint4 *)(a.Vh + ((size_t)g * (cap / 16) + (size_t)c * 4) * hd * 16);
#pragma unroll
        for (int r = 0; r < VR; r++) {
            const int i = tid + 512 * r;                       // tile i / (2 * hd) of the 4
            vk[r] = a.Vh && c * 64 + (i / (2 * hd)) * 16 < T ? ldg(vt + i).x : 0u;
        }
    }
    __syncthreads();
    const int h0 = wave * HPW;
    if (h0 >= G) return;
    const float4 *qh[HPW];
#pragma unroll
    for (int j = 0; j < HPW; j++) qh[j] = q + (h0 + j < G ? h0 + j : G - 1) * HW;
    float acc[HPW];
#pragma unroll
    for (int j = 0; j < HPW; j++) acc[j] = 0.0f;
#pragma unroll 4
    for (int u = 0; u < HW; u++) {
        const uint32_t wv = kt[u * 64 + lane];
        const float c0 = (float)(int8_t)(wv & 0xff), c1 = (float)(int8_t)((wv >> 8) & 0xff);
        const float c2 = (float)(int8_t)((wv >> 16) & 0xff), c3 = (float)(int8_t)(wv >> 24);
#pragma unroll
        for (int j = 0; j < HPW; j++) {
            const float4 qv = qh[j][u];
            acc[j] += qv.x * c0;
            acc[j] += qv.y * c1;
            acc[j] += qv.z * c2;
            acc[j] += qv.w * c3;
        }
    }
    uint32_t keep = 0;
#pragma unroll
    for (int r = 0; r < VR; r++) keep ^= vk[r];
    asm volatile("" ::"v"(keep));
    if (t >= T) return;
#pragma unroll
    for (int j = 0; j < HPW; j++) {
        if (h0 + j >= G) break;
        const float v = ks == 0.0f ? 0.0f : acc[j] * ks;
        stc(a.scores + (size_t)(g * G + h0 + j) * cap + t, v * a.scale);
    }
}
template <int HW, class W>
OH_DEV void exact_scores_g(const oh_op_attn &a, int vb, int pos, W &w) {
    const int G = a.nh / a.nkv;
    if (G <= 8) exact_scores_hw<HW, 1>(a, vb, pos, w);
    else if (G <= 16) exact_scores_hw<HW, 2>(a, vb, pos, w);
    else exact_scores_hw<HW, 4>(a, vb, pos, w);
}
// the host takes this form only for nh / nkv <= OH_EXACT2_GMAX
template <class W>
OH_DEV void exact_scores_body(const oh_op_attn &a, int vb, int pos, int lim, W &w) {
    const int c = vb / a.nkv, T = pos + 1;
    if (T > lim || c * 64 >= T || a.nh > OH_EXACT2_GMAX * a.nkv) return;
    if (a.hd == 256) exact_scores_g<64>(a, vb, pos, w);
    else if (a.hd == 128) exact_scores_g<32>(a, vb, pos, w);
    else exact_scores_g<16>(a, vb, pos, w);
}

// Query head h = vb: softmax over its T scores (max, exps, the double sum in
// exact_body's order, inv = 1/sum) and o_i = sum_t (p_t*Vs_t)*code_t,i in
// position order (thread i < hd), then o *= sigmoid(gate). The exps, then
// the p_t*Vs_t, sit in dynamic LDS: the tiles of 16 positions up to lim and
// two zero tiles past the last. The codes are read from the f16 copy a.Vh,
// so each product is one mixed-precision fma with a zero addend: the exact
// product rounded once, as the reference's multiply (a zero product may
// come out +0 where the multiply gives -0; the running sum is never -0, so
// adding either leaves it unchanged).
template <class W>
OH_DEV void exact_walk_body(const oh_op_attn &a, int vb, int pos, int lim, W &w) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int NT = 512;                     // threads: the softmax on all, the walk on the first hd
    static_assert(NT == 512, "the block sum below adds eight wave sums");
    __shared__ double red[NT / 64];
    __shared__ float mred[NT / 64];
    __shared__ uint64_t etab[32];
    const int nh = a.nh, nkv = a.nkv, hd = a.hd, cap = a.cap;
    const int h = vb, T = pos + 1, t = tid_x();
    if (T > lim || h >= nh) return;
    if (!w.wait()) return;
    float *pb = (float *)smem;
    const int kvh = h / (nh / nkv);
    const int nt = (T + 15) / 16;
    if (t < 32) etab[t] = k_exp2_tab[t];
    // the first NB tiles of this thread's codes (the 16 f16 codes of element
    // t in two uint4) load while the softmax runs; the walk keeps NB tiles
    // in flight, reloading each slot right after its products are formed
    constexpr int NB = 16;
    const uint8_t *vbase = (const uint8_t *)a.Vh + (size_t)kvh * (cap / 16) * hd * 32;
    const uint32_t lo = (uint32_t)(t < hd ? t : 0) * 32u;
    auto ldt = [&](uint4 (&c)[2], int tile) {
        const uint8_t *p = vbase + (size_t)tile * hd * 32;
        c[0] = ldg((const uint4 *)(p + lo));
        c[1] = ldg((const uint4 *)(p + lo + 16));
    };
    // this thread's scores (positions t, t + NT, ...: at most PT of them,
    // lim <= NT * PT, requested in groups of 8 up to T) and value scales,
    // then the gate and the code ring: every load issued before any is used,
    // the softmax's first (they return in order)
    constexpr int PT = 16;
    const float *sh = a.scores + (size_t)h * cap;
    float sv[PT], vs[PT];
#pragma unroll
    for (int r0 = 0; r0 < PT; r0 += 8) {
        if (NT * r0 >= T) break;
#pragma unroll
        for (int r = r0; r < r0 + 8; r++) {
            const int i = t + NT * r < T ? t + NT * r : T - 1;
            sv[r] = ldg(sh + i);
            vs[r] = ldg(a.Vs + (size_t)i * nkv + kvh);
        }
    }
    const float gt = t < hd ? ldg(a.gate + (size_t)h * hd + t) : 0.0f;
    uint4 cw[NB][2];
    if (t < hd) {
#pragma unroll
        for (int u = 0; u < NB; u++) ldt(cw[u], u < nt ? u : nt - 1);
    }
    float mx = -INFINITY;
#pragma unroll
    for (int r0 = 0; r0 < PT; r0 += 8) {
        if (NT * r0 >= T) break;
#pragma unroll
        for (int r = r0; r < r0 + 8; r++) if (t + NT * r < T) mx = fmaxf(mx, sv[r]);
    }
    mx = wave_max_f(mx);
    if (lane_id() == 0) mred[t >> 6] = mx;
    __syncthreads();
#pragma unroll
    for (int k = 0; k < NT / 64; k++) mx = fmaxf(mx, mred[k]);
    // the exps in groups of 8 slots (a slot past T is computed on a
    // repeated score and left out of the sum), so those of a group overlap
    double sum = 0.0;
#pragma unroll
    for (int r0 = 0; r0 < PT; r0 += 8) {
        if (NT * r0 >= T) break;
#pragma unroll
        for (int r = r0; r < r0 + 8; r++) sv[r] = ref_expf_sel(sv[r] - mx, etab);
#pragma unroll
        for (int r = r0; r < r0 + 8; r++) sum += t + NT * r < T ? (double)sv[r] : 0.0;
    }
    // the double sum over the block (tree-ordered, as the walk's other
    // forms; the exps are at most 1, so the order moves only the last
    // bits of a double)
    sum = wave_sum_d(sum);
    if (lane_id() == 0) red[t >> 6] = sum;
    __syncthreads();
    sum = ((red[0] + red[1]) + (red[2] + red[3])) + ((red[4] + red[5]) + (red[6] + red[7]));
    const float inv = (float)(1.0 / sum);
#pragma unroll
    for (int r0 = 0; r0 < PT; r0 += 8) {
        if (NT * r0 >= T) break;
#pragma unroll
        for (int r = r0; r < r0 + 8; r++) if (t + NT * r < T) pb[t + NT * r] = sv[r] * inv * vs[r];
    }
    for (int i = T + t; i < 16 * (nt + 2); i += NT) pb[i] = 0.0f;
    __syncthreads();
    if (t >= hd) return;
    // adds in position order; the weights past T are +0 (the plain sum
    // equals the reference's zero-skipping one, see exact_body). While the
    // 16 adds of tile k run, each add is followed by the product of the same
    // lane position of tile k + 1 (scheduling barriers keep that order, so
    // no instruction waits on the one just before it); the weights of tile
    // k + 2 load from LDS after the second position and tile k's code slot
    // (its products were formed a step earlier) reloads with tile k + NB
    // after the fourth, inside the add chain's latency.
    const float4 *p4 = (const float4 *)pb;
    auto comp = [](const float4 (&P)[4], int j) {
        const float4 v = P[j >> 2];
        return (j & 3) == 0 ? v.x : (j & 3) == 1 ? v.y : (j & 3) == 2 ? v.z : v.w;
    };
    auto code = [](const uint4 (&c)[2], int j) {
        const uint32_t wv = wsel(c[j >> 3], (j >> 1) & 3);
        return (float)__builtin_bit_cast(_Float16, (uint16_t)((j & 1) ? (wv >> 16) : (wv & 0xffffu)));
    };
    float o = 0.0f;
    float X[16], Y[16];
    float4 P0[4], P1[4];
    // RELOAD: a step of a full group of NB tiles (slot u reloads); the
    // steps of the last, partial group load nothing
    auto step = [&](auto reload, int k, int u, const float (&A)[16], float (&B)[16], const float4 (&Pk1)[4],
                    float4 (&Pk2)[4]) {
        const int s1 = (u + 1) % NB;
#pragma unroll
        for (int j = 0; j < 16; j++) {
            o = o + A[j];
            B[j] = __builtin_fmaf(comp(Pk1, j), code(cw[s1], j), 0.0f);
            if (j == 1) {
#pragma unroll
                for (int q = 0; q < 4; q++) Pk2[q] = p4[4 * (k + 2) + q];
            }
            if (decltype(reload)::value && j == 3) ldt(cw[u], k + NB < nt ? k + NB : nt - 1);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
#pragma unroll
    for (int j = 0; j < 4; j++) P0[j] = p4[j];
#pragma unroll
    for (int j = 0; j < 16; j++) X[j] = __builtin_fmaf(comp(P0, j), code(cw[0], j), 0.0f);
#pragma unroll
    for (int j = 0; j < 4; j++) P1[j] = p4[4 + j];
    int k0 = 0;
    for (; k0 + NB <= nt; k0 += NB) {
#pragma unroll
        for (int u = 0; u < NB; u += 2) {
            step(std::true_type(), k0 + u, u, X, Y, P1, P0);
            step(std::true_type(), k0 + u + 1, u + 1, Y, X, P0, P1);
        }
    }
#pragma unroll
    for (int u = 0; u < NB; u += 2) {
        if (k0 + u < nt) step(std::false_type(), k0 + u, u, X, Y, P1, P0);
        if (k0 + u + 1 < nt) step(std::false_type(), k0 + u + 1, u + 1, Y, X, P0, P1);
    }
    stc(a.out + (size_t)h * hd + t, o * ref_sigmoid(gt));
}

// ---- flash decoding for long contexts ----------------------------------------------
// Past exact_max positions the attention of one KV head is split into chunks
// of 64 positions: all nh/nkv query heads of the group score the chunk against
// its Q8 keys once, take the chunk's softmax statistics (max m, sum l of
// exp(s - m)) and the chunk's unnormalised output
// sum_t exp(s_t - m) * Vs_t * code_t. attn_combine merges the chunks with the
// usual rescaling. This re-associates the reference's sums (tolerance, not bit
// parity), and reads each KV byte once per group instead of once per head.
constexpr int kFlashCh = 64;

// LDS of a flash block: the HB query heads (quarters padded by a float4),
// the chunk's key words, value tiles, probabilities and scales
template <int HB> struct FlashLds {
    float *q, *pp, *ks, *vs;
    uint32_t *kc;
    uint4 *vt;
    int qst, kst;
    OH_DEV FlashLds(uint8_t *fsm, int hd) {
        qst = hd + 16;
        kst = hd / 4 + 1;
        q = (float *)fsm;                                     // [HB][4][hd/4 + 4]
        kc = (uint32_t *)(q + HB * qst);                      // [64][hd/4 + 1]
        const int vto = ((HB * qst + kFlashCh * kst) * 4 + 15) & ~15;
        vt = (uint4 *)(fsm + vto);                            // [4][hd]
        pp = (float *)(vt + (kFlashCh / 16) * hd);            // [HB][64]
        ks = pp + HB * kFlashCh;                              // [64]
        vs = ks + kFlashCh;                                   // [64]
    }
};

// the chunk of KV group g starting at t0 (positions past T - 1 read T - 1's).
// Every load of the tile (at most 16 key words and 4 value pieces per thread,
// hd <= 256) is issued before the first LDS store, so the tile costs one
// memory round trip rather than one per loop pass.
template <int HB>
OH_DEV void flash_tile(const oh_op_attn &a, const FlashLds<HB> &L, int g, int t0, int T) {
    const int tid = tid_x(), hd = a.hd, hw = hd / 4, cap = a.cap, nkv = a.nkv;
    constexpr int KW = 64 * kFlashCh / 256, VW = (kFlashCh / 16) * 256 / 256;
    const int nkw = hw * kFlashCh, nvw = (kFlashCh / 16) * hd;
    uint32_t kr[KW];
    uint4 vr[VW];
#pragma unroll
    for (int u = 0; u < KW; u++) {
        const int k = tid + 256 * u < nkw ? tid + 256 * u : nkw - 1;
        const int wi = k / kFlashCh, j = k % kFlashCh;
        const int t = t0 + j < T ? t0 + j : T - 1;
        kr[u] = ldg(a.Kt + ((size_t)g * hw + wi) * cap + t);
    }
#pragma unroll
    for (int u = 0; u < VW; u++) {
        const int k = tid + 256 * u < nvw ? tid + 256 * u : nvw - 1;
        const int tt = k / hd, i = k % hd;
        const int tile = (t0 / 16 + tt) * 16 < T ? t0 / 16 + tt : (T - 1) / 16;
        vr[u] = ldg((const uint4 *)a.Vq + ((size_t)g * (cap / 16) + tile) * hd + i);
    }
    float ksv = 0.0f, vsv = 0.0f;
    if (tid < kFlashCh) {
        const int t = t0 + tid < T ? t0 + tid : T - 1;
        ksv = ldg(a.Ks + (size_t)t * nkv + g);
        vsv = ldg(a.Vs + (size_t)t * nkv + g);
    }
#pragma unroll
    for (int u = 0; u < KW; u++) {
        const int k = tid + 256 * u;
        if (k < nkw) L.kc[(k % kFlashCh) * L.kst + k / kFlashCh] = kr[u];
    }
#pragma unroll
    for (int u = 0; u < VW; u++)
        if (tid + 256 * u < nvw) L.vt[tid + 256 * u] = vr[u];
    if (tid < kFlashCh) {
        L.ks[tid] = ksv;
        L.vs[tid] = vsv;
    }
}

// element k < HB * hd of the block's query heads into the LDS layout
template <int HB>
OH_DEV void flash_q_put(const FlashLds<HB> &L, int hd, int k, float v) {
    const int h = k / hd, e = k % hd, qq = e / (hd / 4);
    L.q[h * L.qst + qq * (hd / 4 + 4) + e % (hd / 4)] = v;
}

// One query position of context T against the chunk c in LDS (positions of
// the tile at or past T score -inf, so they add exact zeros): the HB heads'
// scores, the chunk statistics (m, l) into part_ml and the unnormalised output
// into part_o. LOADQ: the queries are read from qsrc (COH: written by another
// block of the same launch); otherwise the caller has put them into LDS.
template <int HB, bool COH, bool LOADQ = true>
OH_DEV void flash_token(const oh_op_attn &a, const FlashLds<HB> &L, int g, int hb0, int c, int T, const float *qsrc,
                        float *part_o, float *part_ml) {
    const int nh = a.nh, nkv = a.nkv, hd = a.hd, cap = a.cap;
    const int G = nh / nkv;
    const int t0 = c * kFlashCh;
    const int tid = tid_x(), hw = hd / 4;
    const int nchmax = (cap + kFlashCh - 1) / kFlashCh;
    const int qst = L.qst, kst = L.kst;
    if (LOADQ) {
        for (int k = tid; k < HB * hd; k += 256) {
            const float *src = qsrc + ((size_t)g * G + hb0) * hd + k;
            flash_q_put<HB>(L, hd, k, COH ? ldc(src) : ldg(src));
        }
    }
    __syncthreads();
    // scores: thread -> (position j, quarter of the head dimension), the HB
    // heads against its key codes; the quarters are summed with DPP
    {
        const int q4 = tid & 3, j = tid >> 2, wq = hw / 4;
        const uint32_t *kj = L.kc + j * kst + q4 * wq;
        const float4 *q4p = (const float4 *)(L.q + q4 * (hd / 4 + 4));
        float acc[HB];
#pragma unroll
        for (int h = 0; h < HB; h++) acc[h] = 0.0f;
#pragma unroll 4
        for (int wi = 0; wi < wq; wi++) {
            const uint32_t wd = kj[wi];
            const float c0 = (float)(int8_t)(wd & 0xff), c1 = (float)(int8_t)((wd >> 8) & 0xff);
            const float c2 = (float)(int8_t)((wd >> 16) & 0xff), c3 = (float)(int8_t)(wd >> 24);
#pragma unroll
            for (int h = 0; h < HB; h++) {
                const float4 qv = q4p[h * (qst / 4) + wi];
                acc[h] = fmaf(qv.x, c0, acc[h]);
                acc[h] = fmaf(qv.y, c1, acc[h]);
                acc[h] = fmaf(qv.z, c2, acc[h]);
                acc[h] = fmaf(qv.w, c3, acc[h]);
            }
        }
        const float kss = L.ks[j];
        const bool valid = t0 + j < T;
#pragma unroll
        for (int h = 0; h < HB; h++) {
            float v = acc[h];
            v += dpp_f<0xB1>(v);
            v += dpp_f<0x4E>(v);
            if (q4 == 0) {
                const float sc = kss == 0.0f ? 0.0f : v * kss * a.scale;
                L.pp[h * kFlashCh + j] = valid ? sc : -INFINITY;
            }
        }
    }
    __syncthreads();
    // per-head chunk statistics: a wave per head, a lane per position
    const int wave = tid >> 6, lane = tid & 63;
#pragma unroll
    for (int h0 = 0; h0 < HB; h0 += 4) {
        const int h = h0 + wave;
        if (h < HB) {
            const float sv = L.pp[h * kFlashCh + lane];
            const float m = wave_max_fast(sv);
            const float e = sv == -INFINITY ? 0.0f : __expf(sv - m);
            float l = e;
            for (int mm = 32; mm >= 1; mm >>= 1) l += shfl_xor(l, mm);
            L.pp[h * kFlashCh + lane] = e * L.vs[lane];
            if (lane == 0) {
                float *ml = part_ml + (((size_t)g * nchmax + c) * G + hb0 + h) * 2;
                stc(ml, m);
                stc(ml + 1, l);
            }
        }
    }
    __syncthreads();
    // unnormalised outputs: thread -> (dimension i, head h1 + hs*k)
    {
        const int i = tid % hd, hs = 256 / hd, h1 = tid / hd;
        float o[HB];
#pragma unroll
        for (int k = 0; k < HB; k++) o[k] = 0.0f;
        const float4 *pp4 = (const float4 *)L.pp;
#pragma unroll 1
        for (int tt = 0; tt < kFlashCh / 16; tt++) {
            const uint4 cw = L.vt[tt * hd + i];
#pragma unroll
            for (int j4 = 0; j4 < 4; j4++) {
                const uint32_t wd = wsel(cw, j4);
                const float c0 = (float)(int8_t)(wd & 0xff), c1 = (float)(int8_t)((wd >> 8) & 0xff);
                const float c2 = (float)(int8_t)((wd >> 16) & 0xff), c3 = (float)(int8_t)(wd >> 24);
#pragma unroll
                for (int k = 0; k < HB; k++) {
                    const int h = h1 + hs * k < HB ? h1 + hs * k : HB - 1;
                    const float4 pv = pp4[(h * kFlashCh + tt * 16 + 4 * j4) / 4];
                    o[k] = fmaf(pv.x, c0, o[k]);
                    o[k] = fmaf(pv.y, c1, o[k]);
                    o[k] = fmaf(pv.z, c2, o[k]);
                    o[k] = fmaf(pv.w, c3, o[k]);
                }
            }
        }
#pragma unroll
        for (int k = 0; k < HB; k++) {
            const int h = h1 + hs * k;
            if (h < HB) stc(part_o + (((size_t)g * nchmax + c) * G + hb0 + h) * hd + i, o[k]);
        }
    }
}

// HB query heads of one KV head per virtual block (compile time: the loops
// over heads unroll); vb = chunk * (nkv * G/HB) + group-block, G = nh/nkv.
template <int HB, class W>
OH_DEV void flash_body(const oh_op_attn &a, int vb, int pos, int lim, W &w) {
    extern __shared__ __align__(16) uint8_t fsm[];
    const int nh = a.nh, nkv = a.nkv;
    const int T = pos + 1;
    const int G = nh / nkv, ngb = G / HB, gx = nkv * ngb;
    const int bx = vb % gx, c = vb / gx;
    const int g = bx / ngb, hb0 = (bx % ngb) * HB;
    const int t0 = c * kFlashCh;
    if (T <= lim || t0 >= T) return;
    if (!w.wait()) return;
    const FlashLds<HB> L(fsm, a.hd);
    // the queries (written by the prep phase) and the tile are all requested
    // before the first wait: HB * hd <= 1024 floats, at most 4 per thread
    const int tid = tid_x(), nq = HB * a.hd;
    const float *qs = a.qr + ((size_t)g * G + hb0) * a.hd;
    float qv[4];
#pragma unroll
    for (int m = 0; m < 4; m++) qv[m] = ldc(qs + (tid + 256 * m < nq ? tid + 256 * m : nq - 1));
    flash_tile<HB>(a, L, g, t0, T);
#pragma unroll
    for (int m = 0; m < 4; m++)
        if (tid + 256 * m < nq) flash_q_put<HB>(L, a.hd, tid + 256 * m, qv[m]);
    flash_token<HB, true, false>(a, L, g, hb0, c, T, nullptr, a.part_o, a.part_ml);
}

// ---- flash decoding on the matrix cores --------------------------------------------
// The same chunked form (re-associated softmax and V sums, tolerance bar) for
// the decode token, with every query head of a KV head in one block: block b
// of KV head g takes the 32-position tiles [b*tpb, (b+1)*tpb) of the context
// and its four waves take every fourth tile. Per tile a wave forms S^T = K Q^T
// (32 positions x the G <= 16 query heads of g as columns) with
// v_mfma_f32_16x16x32_f16 on the raw int8 key codes (exact in fp16) against
// the pre-scaled queries split into fp16 high and low parts (two products:
// about 22 significant bits; each head's queries and each wave's P*Vs are
// first brought to at most 1 by an exact power of two, undone in fp32), scales
// by the keys' scales in fp32, keeps a running max and sum per head, and
// accumulates O^T += V^T P^T on the raw value codes with P*Vs split the same
// way. The four waves' (m, l, O) merge in
// LDS into one partial per block; attn_combine merges the blocks.
//
// Lane layouts of v_mfma_f32_16x16x32_f16: A (16 x 32) lane l holds row l%16,
// k = 8*(l/16) + j; B (32 x 16) column l%16, the same k; D (16 x 16) column
// l%16, rows 4*(l/16) + v. Row r of the two S^T sub-tiles u = 0, 1 is position
// 8*(r/4) + 4u + r%4 of the tile, so D value v of sub-tile u in lane (c, q)
// is position 8q + 4u + v: exactly the B operand (k = 8q + j) of the tile's
// 32-position V^T P^T product.
typedef _Float16 fd_h8 __attribute__((ext_vector_type(8)));
typedef float fd_f4 __attribute__((ext_vector_type(4)));
constexpr int kFdT = 32;          // positions per wave tile
constexpr int kFdMaxBlk = 128;    // blocks per KV head

OH_HD inline int fd_blocks(int cap) {
    const int b = (cap + kFdT - 1) / kFdT;
    return b < kFdMaxBlk ? b : kFdMaxBlk;
}
// partial slots per KV head (both flash forms share the partial buffers)
OH_HD inline int fd_slots(int cap) {
    const int c = (cap + kFlashCh - 1) / kFlashCh, b = fd_blocks(cap);
    return c > b ? c : b;
}
// tiles per block for context T (the blocks holding work: ceil(tiles / tpb)):
// at least one per wave, so the merge has fewer partials at short contexts
OH_HD inline int fd_tpb(int T, int cap) {
    const int nt = (T + kFdT - 1) / kFdT, B = fd_blocks(cap);
    const int t = (nt + B - 1) / B;
    return t > 4 ? t : 4;
}
constexpr int kFdLds = 4 * 64 * 2 * 4 + 4 * 4 * 64 * 16;   // merge: (m, l) and four dim tiles per wave

template <int HD, class W>
OH_DEV void flashm_body(const oh_op_attn &a, int vb, int pos, int lim, W &w) {
    extern __shared__ __align__(16) uint8_t fsm[];
    constexpr int NS = HD / 32, ND = HD / 16, HW = HD / 4;
    const int nkv = a.nkv, G = a.nh / nkv, cap = a.cap, T = pos + 1;
    const int g = vb % nkv, b = vb / nkv;
    const int nt = (T + kFdT - 1) / kFdT, tpb = fd_tpb(T, cap), tb = b * tpb;
    if (T <= lim || tb >= nt) return;
    if (!w.wait()) return;
    const int te = tb + tpb < nt ? tb + tpb : nt;
    const int tid = tid_x(), lane = tid & 63, wave = tid >> 6;
    const int col = lane & 15, qd = lane >> 4, r = lane & 15;
    const bool cv = col < G;
    // the queries (written by the prep operation) as B operands: K-step s
    // holds dims 32 s + 8 qd .. + 7 of head col, times 1/sqrt(hd) and 2^-eq
    // (eq: the exponent of the head's largest |q|, so the fp16 halves keep
    // their precision whatever the magnitude)
    fd_h8 qh[NS], ql[NS];
    int eq = 0;
    {
        const float *qs = a.qr + (size_t)(g * G + (cv ? col : 0)) * HD + 8 * qd;
        float xv[NS][8];
        float amax = 0.0f;
#pragma unroll
        for (int s = 0; s < NS; s++) {
            const float4 x0 = ldc4((const float4 *)(qs + 32 * s)), x1 = ldc4((const float4 *)(qs + 32 * s + 4));
            const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
            for (int j = 0; j < 8; j++) {
                xv[s][j] = cv ? xs[j] * a.scale : 0.0f;
                amax = fmaxf(amax, fabsf(xv[s][j]));
            }
        }
        amax = fmaxf(amax, shfl_xor(amax, 16));
        amax = fmaxf(amax, shfl_xor(amax, 32));
        if (amax > 0.0f && amax <= 3.0e38f) frexpf(amax, &eq);
#pragma unroll
        for (int s = 0; s < NS; s++)
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const float v = ldexpf(xv[s][j], -eq);
                const _Float16 h = (_Float16)v;
                qh[s][j] = h;
                ql[s][j] = (_Float16)(v - (float)h);
            }
    }
    fd_f4 o[ND];
#pragma unroll
    for (int d = 0; d < ND; d++) o[d] = fd_f4{0.0f, 0.0f, 0.0f, 0.0f};
    // O is kept in units of 2^-ev, ev the exponent of the largest value scale
    // seen so far by this wave (P*Vs*2^-ev <= 1 keeps the fp16 halves exact)
    float m = -INFINITY, l = 0.0f, vm = 0.0f;
    int ev = 0;
    const uint32_t *kb = a.Kt + (size_t)g * HW * cap;
    const uint8_t *vq = (const uint8_t *)a.Vq + (size_t)g * (cap / 16) * HD * 16;
    for (int t = tb + wave; t < te; t += 4) {
        const int p0 = t * kFdT;
        // every load of the tile first: key words, value codes, scales
        uint32_t kw[2][NS][2];
#pragma unroll
        for (int u = 0; u < 2; u++) {
            int p = p0 + 8 * (r >> 2) + 4 * u + (r & 3);
            p = p < T ? p : T - 1;
#pragma unroll
            for (int s = 0; s < NS; s++) {
                kw[u][s][0] = ldg(kb + (size_t)(8 * s + 2 * qd) * cap + p);
                kw[u][s][1] = ldg(kb + (size_t)(8 * s + 2 * qd + 1) * cap + p);
            }
        }
        int vt = (p0 + 8 * qd) / 16;
        vt = vt <= (T - 1) / 16 ? vt : (T - 1) / 16;
        uint2 vw[ND];
#pragma unroll
        for (int d = 0; d < ND; d++)
            vw[d] = ldg((const uint2 *)(vq + ((size_t)vt * HD + 16 * d + r) * 16 + 8 * (qd & 1)));
        float ks[8], vs[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int p = p0 + 8 * qd + j, pc = p < T ? p : T - 1;
            ks[j] = ldg(a.Ks + (size_t)pc * nkv + g);
            vs[j] = ldg(a.Vs + (size_t)pc * nkv + g);
        }
        // scores of positions p0 + 8 qd + j for head col
        float sj[8];
#pragma unroll
        for (int u = 0; u < 2; u++) {
            fd_f4 sc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int s = 0; s < NS; s++) {
                fd_h8 ka;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    ka[j] = (_Float16)(float)(int8_t)(kw[u][s][0] >> (8 * j));
                    ka[4 + j] = (_Float16)(float)(int8_t)(kw[u][s][1] >> (8 * j));
                }
                sc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qh[s], sc, 0, 0, 0);
                sc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, ql[s], sc, 0, 0, 0);
            }
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int j = 4 * u + v;
                const float k = ks[j];
                const float x = k == 0.0f ? 0.0f : sc[v] * ldexpf(k, eq);
                sj[j] = p0 + 8 * qd + j < T ? x : -INFINITY;
            }
        }
        // online softmax per head (the tile's first position is < T, so the
        // new max is finite)
        float mx = sj[0];
#pragma unroll
        for (int j = 1; j < 8; j++) mx = fmaxf(mx, sj[j]);
        mx = fmaxf(mx, shfl_xor(mx, 16));
        mx = fmaxf(mx, shfl_xor(mx, 32));
        const float mn = fmaxf(m, mx);
        const float corr = m == -INFINITY ? 0.0f : __expf(m - mn);
        float vx = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; j++)
            if (p0 + 8 * qd + j < T) vx = fmaxf(vx, fabsf(vs[j]));
        vx = fmaxf(vx, shfl_xor(vx, 16));
        vx = fmaxf(vx, shfl_xor(vx, 32));
        vm = fmaxf(vm, vx);
        int en = ev;
        if (vm > 0.0f && vm <= 3.0e38f) frexpf(vm, &en);
        const float fac = corr * ldexpf(1.0f, ev - en);
        ev = en;
        float ls = 0.0f;
        fd_h8 ph, pl;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float e = sj[j] == -INFINITY ? 0.0f : __expf(sj[j] - mn);
            ls += e;
            const float pv = p0 + 8 * qd + j < T ? e * ldexpf(vs[j], -ev) : 0.0f;
            const _Float16 h = (_Float16)pv;
            ph[j] = h;
            pl[j] = (_Float16)(pv - (float)h);
        }
        ls += shfl_xor(ls, 16);
        ls += shfl_xor(ls, 32);
        l = l * corr + ls;
        m = mn;
        if (__ballot(fac != 1.0f) != 0) {
#pragma unroll
            for (int d = 0; d < ND; d++) o[d] *= fac;
        }
#pragma unroll
        for (int d = 0; d < ND; d++) {
            fd_h8 va;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                va[j] = (_Float16)(float)(int8_t)(vw[d].x >> (8 * j));
                va[4 + j] = (_Float16)(float)(int8_t)(vw[d].y >> (8 * j));
            }
            o[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, ph, o[d], 0, 0, 0);
            o[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pl, o[d], 0, 0, 0);
        }
    }
    {
        const float u = ldexpf(1.0f, ev);
#pragma unroll
        for (int d = 0; d < ND; d++) o[d] *= u;
    }
    // merge the four waves: factors exp(m_w - M) per lane, then the dim tiles
    // four at a time through LDS (thread (wave, lane) merges tile d0 + wave)
    float *sml = (float *)fsm;                                  // [4][64][2]
    fd_f4 *sob = (fd_f4 *)(fsm + 4 * 64 * 2 * 4);               // [4 waves][4 tiles][64]
    sml[(wave * 64 + lane) * 2] = m;
    sml[(wave * 64 + lane) * 2 + 1] = l;
    __syncthreads();
    float M = -INFINITY;
#pragma unroll
    for (int k = 0; k < 4; k++) M = fmaxf(M, sml[(k * 64 + lane) * 2]);
    float f[4], L = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const float mk = sml[(k * 64 + lane) * 2];
        f[k] = mk == -INFINITY ? 0.0f : __expf(mk - M);
        L += sml[(k * 64 + lane) * 2 + 1] * f[k];
    }
    const int S = fd_slots(cap);
    const size_t pb = ((size_t)g * S + b) * G + col;
    if (cv && wave == 0 && qd == 0) {
        stc(a.part_ml + pb * 2, M);
        stc(a.part_ml + pb * 2 + 1, L);
    }
#pragma unroll
    for (int d0 = 0; d0 < ND; d0 += 4) {
#pragma unroll
        for (int k = 0; k < 4; k++) sob[(wave * 4 + k) * 64 + lane] = o[d0 + k];
        __syncthreads();
        fd_f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int k = 0; k < 4; k++) acc += sob[(k * 4 + wave) * 64 + lane] * f[k];
        if (cv) stc4((float4 *)(a.part_o + pb * HD + 16 * (d0 + wave) + 4 * qd),
                     make_float4(acc[0], acc[1], acc[2], acc[3]));
        __syncthreads();
    }
}

// The attention of the current step: up to lim = min(exact_max, kExactMax)
// positions the exact walk (virtual blocks [0, nh*hd/256)), beyond that the
// flash chunks (virtual blocks as flash_body).
template <class W>
OH_DEV void attn_main_body(const oh_op_attn &a, int vb, int pos, W &w) {
    const int lim = exact_lim(a.exact_max, a.hd);
    if (pos + 1 <= lim) {
        exact_body(a, vb, pos, lim, w);
    } else if (a.hb == 0) {
        if (a.hd == 256) flashm_body<256>(a, vb, pos, lim, w);
        else if (a.hd == 128) flashm_body<128>(a, vb, pos, lim, w);
        else flashm_body<64>(a, vb, pos, lim, w);
    } else if (a.hb == 4) {
        flash_body<4>(a, vb, pos, lim, w);
    } else if (a.hb == 2) {
        flash_body<2>(a, vb, pos, lim, w);
    } else {
        flash_body<1>(a, vb, pos, lim, w);
    }
}

// Merge of the flash chunks of query head h (virtual block vb = y * nh + h,
// y < hd/64; 4 waves; wave w takes chunks w, w+4, ...; a lane per dimension):
// running max rescaling, then
// out = (sum_c o_c e^(m_c-M)) / (sum_c l_c e^(m_c-M)) * sigmoid(gate).
// lim: contexts up to it took the exact walk (nothing to merge).
template <class W>
OH_DEV void combine_body(const oh_op_attn &a, int vb, int pos, W &w, int lim) {
    __shared__ float sm[4][3][64];
    const int nh = a.nh, nkv = a.nkv, hd = a.hd, cap = a.cap;
    const int T = pos + 1;
    if (T <= lim) return;
    if (!w.wait()) return;
    const int h = vb % nh, G = nh / nkv, g = h / G, hl = h % G;
    const int wave = (tid_x() >> 6), lane = (tid_x() & 63);
    const int i = (vb / nh) * 64 + lane;
    const int nch = a.hb == 0 ? (((T + kFdT - 1) / kFdT) + fd_tpb(T, cap) - 1) / fd_tpb(T, cap)
                              : (T + kFlashCh - 1) / kFlashCh;
    const int nchmax = a.hb == 0 ? fd_slots(cap) : (cap + kFlashCh - 1) / kFlashCh;
    float M = -INFINITY, L = 0.0f, O = 0.0f;
    // chunks wave, wave+4, ... in order; their partials requested 8 at a time
    constexpr int CB = 8;
    for (int c0 = wave; c0 < nch; c0 += 4 * CB) {
        float mb[CB], lb[CB], ob[CB];
#pragma unroll
        for (int u = 0; u < CB; u++) {
            const int c = c0 + 4 * u < nch ? c0 + 4 * u : c0;
            const size_t base = ((size_t)g * nchmax + c) * G + hl;
            mb[u] = ldw<W::kGrid>(a.part_ml + base * 2);
            lb[u] = ldw<W::kGrid>(a.part_ml + base * 2 + 1);
            ob[u] = ldw<W::kGrid>(a.part_o + base * hd + i);
        }
#pragma unroll
        for (int u = 0; u < CB; u++) {
            if (c0 + 4 * u >= nch) break;
            const float m = mb[u], mn = fmaxf(M, m);
            const float e1 = M == -INFINITY ? 0.0f : __expf(M - mn), e2 = __expf(m - mn);
            O = O * e1 + ob[u] * e2;
            L = L * e1 + lb[u] * e2;
            M = mn;
        }
    }
    sm[wave][0][lane] = M; sm[wave][1][lane] = L; sm[wave][2][lane] = O;
    __syncthreads();
    if (wave == 0) {
        float Mt = -INFINITY;
        for (int k = 0; k < 4; k++) Mt = fmaxf(Mt, sm[k][0][lane]);
        float Lt = 0.0f, Ot = 0.0f;
        for (int k = 0; k < 4; k++) {
            const float mw = sm[k][0][lane];
            const float f = mw == -INFINITY ? 0.0f : __expf(mw - Mt);
            Lt += sm[k][1][lane] * f;
            Ot += sm[k][2][lane] * f;
        }
        stc(a.out + (size_t)h * hd + i, Ot / Lt * ref_sigmoid(ldw<W::kGrid>(a.gate + (size_t)h * hd + i)));
    }
}

// x += sum_s w_s * o_s (sequential in s, from 0) + shared * gate
// (src/ornith_rforward.c:375-409)
template <class W>
OH_DEV void moe_combine_body(const oh_op_combine &a, int vb, W &w) {
    if (!w.wait()) return;
    const int i = vb * 256 + tid_x();
    if (i >= a.H) return;
    float acc = 0.0f;
    for (int s = 0; s < a.k; s++) acc += ldc(a.w + s) * ldc(a.o + (size_t)s * a.H + i);
    if (a.so) {
        const float so = ldc(a.so + i);
        const float v = a.shgate ? so * ldc(a.shgate) : so;
        acc += v;
    }
    stc(a.x + i, ldc(a.x + i) + acc);
}

// ---- greedy argmax over the logits (src/ornith_rforward.c:18-22) ----------------
// stage 1: per-block best (largest value, lowest index on ties) of the
// elements vb, vb + nblk*256, ...
template <class W>
OH_DEV void argmax1_body(const oh_op_argmax &a, int vb, W &w) {
    __shared__ float sv[4];
    __shared__ int si[4];
    if (!w.wait()) return;
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int i = vb * 256 + tid_x(); i < a.n; i += a.nblk * 256) {
        const float x = ldc(a.v + i);
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
        stc(a.bv + vb, bv);
        stc(a.bi + vb, bi);
    }
}

// stage 2 (one wave): combine the per-block bests; write the next token at
// toks[pos] (pos was already advanced by the body) and keep it in *best.
template <class W>
OH_DEV void argmax2_body(const oh_op_argmax &a, int pos, W &w) {
    if (!w.wait()) return;
    if (tid_x() >= 64) return;
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int i = tid_x(); i < a.nblk; i += 64) {
        const float x = ldc(a.bv + i);
        const int xi = ldc(a.bi + i);
        if (x > bv || (x == bv && xi < bi)) { bv = x; bi = xi; }
    }
    for (int m = 32; m >= 1; m >>= 1) {
        const float ov = shfl_xor(bv, m); const int oi = shfl_xor(bi, m);
        if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
    }
    if (tid_x() == 0) {
        if (bi == 0x7fffffff) bi = 0;
        stc(a.toks + pos, (int32_t)bi);
        stc(a.best, (int32_t)bi);
    }
}

#ifndef OH_BODIES_ONLY
// ---- standalone kernels (one launch per operation, captured into HIP graphs) -------
extern "C" __global__ void __launch_bounds__(256) oh_k_embed(oh_op_embed a, const int32_t *io) {
    NoWait w;
    embed_body(a, (int)blockIdx.x, io[OH_IO_POS], w);
}

template <int DK, int KMAX>
__global__ void __launch_bounds__(64) oh_k_delta_step(oh_op_delta a, const int32_t *io) {
    __shared__ __align__(16) float lds[2 * DK + 64 * (DK + 4)];
    NoWait w;
    delta_body<DK, KMAX>(a, (int)blockIdx.x, io[OH_IO_POS], lds, w);
}

template <int DK, int KMAX>
__global__ void __launch_bounds__(256) oh_k_delta16(oh_op_delta a, const int32_t *io) {
    __shared__ __align__(16) float lds[delta16_lds_floats(DK)];
    NoWait w;
    delta16_body<DK, KMAX>(a, (int)blockIdx.x, io[OH_IO_POS], lds, w);
}

extern "C" __global__ void __launch_bounds__(256) oh_k_attn_prep(oh_op_prep a, const int32_t *io) {
    NoWait w;
    prep_body(a, (int)blockIdx.x, io[OH_IO_POS], w);
}

extern "C" __global__ void __launch_bounds__(256) oh_k_attn_main(oh_op_attn a, const int32_t *io) {
    NoWait w;
    attn_main_body(a, (int)blockIdx.x, io[OH_IO_POS], w);
}

// the graph step's exact attention in two launches (contexts up to the exact
// limit; both exit past it): the scores, then the softmax and output walk
extern "C" __global__ void __launch_bounds__(512) oh_k_attn_scores(oh_op_attn a, const int32_t *io) {
    NoWait w;
    exact_scores_body(a, (int)blockIdx.x, io[OH_IO_POS], exact_lim(a.exact_max, a.hd), w);
}
extern "C" __global__ void __launch_bounds__(512) oh_k_attn_walk(oh_op_attn a, const int32_t *io) {
    NoWait w;
    exact_walk_body(a, (int)blockIdx.x, io[OH_IO_POS], exact_lim(a.exact_max, a.hd), w);
}
extern "C" __global__ void __launch_bounds__(256) oh_k_attn_combine(oh_op_attn a, const int32_t *io) {
    NoWait w;
    combine_body(a, (int)blockIdx.x, io[OH_IO_POS], w, exact_lim(a.exact_max, a.hd));
}

extern "C" __global__ void __launch_bounds__(256) oh_k_moe_combine(oh_op_combine a) {
    NoWait w;
    moe_combine_body(a, (int)blockIdx.x, w);
}

extern "C" __global__ void __launch_bounds__(256) oh_k_argmax1(oh_op_argmax a) {
    NoWait w;
    argmax1_body(a, (int)blockIdx.x, w);
}

extern "C" __global__ void __launch_bounds__(64) oh_k_argmax2(oh_op_argmax a, const int32_t *io) {
    NoWait w;
    argmax2_body(a, io[OH_IO_POS], w);
}

// ---- MoE router (src/ornith_moe.c:8-30) ------------------------------------------
// One wave: top-k by repeated scans (strict '>', ties -> lower index), softmax
// over the selected logits with a sequential float sum; also sigmoid of the
// shared-expert gate logit.
extern "C" __global__ void __launch_bounds__(64)
oh_k_moe_route(const float *logits, int ne, int k, const float *shgate_logit,
               int32_t *idx, float *w, float *shgate) {
    route_wave(logits, ne, k, shgate_logit, idx, w, shgate);
}

// advance the stream position after a token's layers (rforward_token s->pos++)
// and the session's step serial
extern "C" __global__ void oh_k_advance(int32_t *io) {
    io[OH_IO_POS] = io[OH_IO_POS] + 1;
    io[OH_IO_SERIAL] = io[OH_IO_SERIAL] + 1;
}

#endif // OH_BODIES_ONLY
