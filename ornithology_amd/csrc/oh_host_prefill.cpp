// oh_host_prefill.cpp - the layer-major prefill (src/ornith_rforward.c:647-682 structure).
#include "oh_engine.h"


// tokens per engine chunk (ORNITH_HIP_PREFILL_CHUNK, default kPfChunk = 4096): a multiple
// of 32, because the chunked delta scan counts its 32-token chunks from the
// start of the evaluation and an engine chunk must not split one
// prompt attention past the exact walk on the matrix cores; on unless
// ORNITH_HIP_ATTN_MFMA=0
bool attn_mfma_enabled() {
    const char *e = getenv("ORNITH_HIP_ATTN_MFMA");
    return !(e && e[0] == '0');
}

// batch decode below the matrix-core column count through the fused slotted
// launches; on unless ORNITH_HIP_BATCH_FUSED=0
bool batch_fused() {
    const char *e = getenv("ORNITH_HIP_BATCH_FUSED");
    return !(e && e[0] == '0');
}
// the token step's MoE router inside the experts launch (its logits handed
// over as tagged words) instead of a launch of its own; on unless
// ORNITH_HIP_ROUTER_FUSE=0 (same bits either way)
bool router_fused() {
    const char *e = getenv("ORNITH_HIP_ROUTER_FUSE");
    return !(e && e[0] == '0');
}
// the delta step and its output projection in one launch: opt-in (on C3 it
// measures 23.8 us per layer replayed against 6.0 + 11.2 us for the two
// launches, and 334 against 374 tok/s)
bool delta_fused() {
    const char *e = getenv("ORNITH_HIP_DELTA_FUSE");
    return e && e[0] == '1';
}

// the prompt's chunked delta scan on the matrix cores in its WY form (a
// tolerance path: the chunk sums re-associated; ORNITH_HIP_DELTA_MFMA=1)
// instead of the reference-order vector-ALU scan
bool delta_mfma_enabled() {
    const char *e = getenv("ORNITH_HIP_DELTA_MFMA");
    return e && e[0] == '1';
}

int pf_chunk_tokens() {
    const char *e = getenv("ORNITH_HIP_PREFILL_CHUNK");
    int c = e && *e ? atoi(e) : kPfChunk;
    c = c / 32 * 32;
    return c < 32 ? 32 : (c > kPfChunk ? kPfChunk : c);
}

bool pf_mvb_ok(const ornith_hip_tensor *W) {
    return W && oh_qdot_can(W->type, W->in) && W->in <= 8192 && W->in / 256 <= 64;
}

// routed experts the grouped batched products handle: integer-path types,
// gate and up a pair
bool pf_moe_grouped(const OhLayer &y) {
    return pf_mvb_ok(y.gate_exps) && pf_mvb_ok(y.up_exps) && pf_mvb_ok(y.down_exps) && pairable(y.gate_exps, y.up_exps);
}

// other expert types (IQ2_XXS) run the token step's expert kernels over the
// chunk's (token, expert) slots
bool pf_moe_slots_ok(const OhLayer &y) {
    for (const ornith_hip_tensor *W : {y.gate_exps, y.up_exps, y.down_exps})
        if (!W || W->in % 256 || W->in > 8192 || W->nd != 3) return false;
    return true;
}

bool pf_supported(const ornith_hip_model *m) {
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

int pf_alloc(ornith_hip_session *s, int tc) {
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
int pf_mvb(const ornith_hip_tensor *W, const ornith_hip_tensor *W2, const Q8Buf &x, float *y, int ystride,
                  int T, int mode, hipStream_t st, const int32_t *cnt, const int32_t *list,
                  int lstride, int adiv, int groups) {
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
bool pf_use_mmq(const ornith_hip_tensor *W, bool grouped, int T) {
    const int rows = grouped ? (int)W->dims[1] : (int)W->rows;
    return mmq_enabled() && T >= kMmqMinTokens && oh_mmq_can(W->type, rows, (int)W->in);
}

// The prompt tiles of every tensor that pf_chunk runs on the matrix cores
// (the pairs of pf_swiglu only when both qualify)
int pf_tiles(const ornith_hip_model *m, hipStream_t st) {
    if (!mmq_enabled()) return ORNITH_HIP_OK;
    const int T = kMmqMinTokens;
    for (const OhLayer &y : m->L) {
        const ornith_hip_tensor *dense[] = {y.q, y.k, y.v, y.o, y.qkv, y.gate, y.alpha, y.beta, y.ssm_out,
                                            y.router, y.gate_inp_sh, y.down_sh, y.ffn_down};
        for (const ornith_hip_tensor *W : dense)
            if (W && pf_use_mmq(W, false, T)) CHK(mmq_tiles(W, st));
        const ornith_hip_tensor *pairs[][2] = {{y.gate_sh, y.up_sh}, {y.ffn_gate, y.ffn_up}};
        for (auto &pr : pairs)
            if (pr[0] && pr[1] && pf_use_mmq(pr[0], false, T) && pf_use_mmq(pr[1], false, T)) {
                CHK(mmq_tiles(pr[0], st));
                CHK(mmq_tiles(pr[1], st));
            }
        if (y.gate_exps && y.up_exps && pf_use_mmq(y.gate_exps, true, T) && pf_use_mmq(y.up_exps, true, T)) {
            CHK(mmq_tiles(y.gate_exps, st));
            CHK(mmq_tiles(y.up_exps, st));
        }
        if (y.down_exps && pf_use_mmq(y.down_exps, true, T)) CHK(mmq_tiles(y.down_exps, st));
    }
    return ORNITH_HIP_OK;
}

int pf_mmq(const ornith_hip_tensor *W, const ornith_hip_tensor *W2, const Q8Buf &x, float *y, int ystride,
                  int T, int mode, hipStream_t st, const int32_t *cnt, const int32_t *list,
                  int lstride, int adiv, const int32_t *items, int max_items) {
    CHK(mmq_tiles(W, st));
    if (W2) CHK(mmq_tiles(W2, st));
    oh_mmq M;
    memset(&M, 0, sizeof M);
    M.A = W->PA; M.B = W->PB; M.C = W->C; M.type = (int)W->type;
    if (W2) { M.A2 = W2->PA; M.B2 = W2->PB; M.C2 = W2->C; }
    M.xqs = x.qs; M.xd = x.d; M.xbp = x.bp; M.y = y;
    M.cnt = cnt; M.list = list; M.items = items;
    M.nb = (int)(W->in / 256); M.in = (int)W->in; M.rows = list ? (int)W->dims[1] : (int)W->rows;
    M.mode = mode; M.ncol = T; M.lstride = lstride; M.adiv = adiv; M.ystride = ystride;
    HCHK(oh_launch_mmq(&M, max_items, W2 != nullptr, st));
    return ORNITH_HIP_OK;
}

// y (+)= W . x over T dense columns
int pf_mm(const ornith_hip_tensor *W, const Q8Buf &x, float *y, int ystride, int T, int mode,
                 hipStream_t st) {
    if (pf_use_mmq(W, false, T)) return pf_mmq(W, nullptr, x, y, ystride, T, mode, st);
    return pf_mvb(W, nullptr, x, y, ystride, T, mode, st);
}

// h = silu(Wg . x) * (Wu . x) for `npairs` output rows (T dense columns, or the
// grouped expert pairs), quantised to Q8_K in hq
int pf_swiglu(const ornith_hip_tensor *Wg, const ornith_hip_tensor *Wu, const Q8Buf &x, int I, int npairs,
                     int T, Q8Buf &hq, float *gu, float *hbuf, hipStream_t st, const int32_t *cnt,
                     const int32_t *list, int lstride, int adiv, int groups,
                     const int32_t *items, int max_items) {
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

int pf_chunk(ornith_hip_session *s, int base, int T, bool chunked, hipStream_t st) {
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
                             a.nh, a.nkv, a.hd, a.rope_dim, s->kvcap, a.eps, z.Vh};
            HCHK(oh_launch_prep_rows(&pr, base, T, st));
            oh_op_attn at;
            memset(&at, 0, sizeof at);
            at.qr = p.QR; at.gate = p.AG; at.Kt = z.Kt; at.Ks = z.Ks; at.Vq = z.Vq; at.Vs = z.Vs;
            at.part_o = p.FPO; at.part_ml = p.FPML; at.out = p.OA;
            at.nh = a.nh; at.nkv = a.nkv; at.hd = a.hd; at.cap = s->kvcap; at.exact_max = s->pf_exact_max;
            at.hb = oh_flash_hb(a.nh, a.nkv); at.scale = 1.0f / sqrtf((float)a.hd);
            const int nch = (s->kvcap + oh_flash_chunk() - 1) / oh_flash_chunk();
            const size_t po = (size_t)a.nh * nch * a.hd, pml = (size_t)a.nh * nch * 2;
            // tokens whose context fits the exact walk take it (sub-batches of
            // kPfAttnSub); the rest go to the matrix-core kernel in one launch
            // (ORNITH_HIP_ATTN_MFMA=0: the flash chunks of the decode step)
            const int lim = s->pf_exact_max < 2048 ? s->pf_exact_max : 2048;
            const int tsplit = attn_mfma_enabled() && oh_attn_mfma_supported(a.hd, a.nh, a.nkv)
                             ? (lim - base < 0 ? 0 : (lim - base > T ? T : lim - base)) : T;
            if (tsplit < T || base + T <= lim) {
                // every row before tsplit is inside the exact walk: one launch
                HCHK(oh_launch_attn_exact_rows(&at, base, 0, tsplit, st));
            } else {
                for (int t0 = 0; t0 < tsplit; t0 += kPfAttnSub)
                    HCHK(oh_launch_attn_rows(&at, base, t0, tsplit - t0 < kPfAttnSub ? tsplit - t0 : kPfAttnSub, po,
                                             pml, st));
            }
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
                HCHK(oh_launch_group_pairs(p.RIDX, T * K, p.CNT, a.ne, p.LIST, T, s->io + OH_IO_ERR, st));
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

bool pf_enabled() {
    const char *e = getenv("ORNITH_HIP_PREFILL");
    return !(e && e[0] == '0');
}

// the reference's prompt mode switch (src/ornith_rforward.c:838-849): default
// chunked delta scan, ORNITH_PREFILL_SERIAL=1 the token-by-token recurrence
bool prefill_serial() {
    const char *e = getenv("ORNITH_PREFILL_SERIAL");
    return e && e[0] == '1';
}

// tokens through the layer-major prompt path (rprefill) or, with token_path,
// through the token step (rforward_token) one at a time
int session_eval(ornith_hip_session *s, const int32_t *tokens, int n, bool token_path) {
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
