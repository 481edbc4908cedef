// oh_host_session.cpp - sessions, the token step as a program of operations, its graph and persistent launches.
#include "oh_engine.h"


int rec_begin(ornith_hip_session *s, hipStream_t st) {
    if (!s->rec) return ORNITH_HIP_OK;
    hipEvent_t e;
    HCHK(hipEventCreate(&e));
    HCHK(hipEventRecord(e, st));
    s->rec_ev.push_back(e);
    return ORNITH_HIP_OK;
}
int rec_end(ornith_hip_session *s, hipStream_t st, int kind, double bytes) {
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
bool keep(ornith_hip_session *s, int kind, double bytes) {
    if (s->only < 0) return true;
    if (kind != s->only) return false;
    s->only_n++;
    s->only_bytes += bytes;
    return true;
}
// matvec launches are recorded by kernel variant (see oh_launch_matvec)
int mv_kind(int tk) {
    return tk == OH_Q4_K ? K_MATVEC : tk == OH_Q6_K ? K_MATVEC_Q6K : tk == OH_Q8_0 ? K_MATVEC_Q80
         : tk == OH_MV_Q4Q6 ? K_MATVEC_Q4Q6 : K_MATVEC_MIXED;
}
oh_op op_new(int kind, int nvb, int lds) {
    oh_op o;
    memset(&o, 0, sizeof o);
    o.kind = kind;
    o.nvb = nvb;
    o.tk = -1;
    o.lds = lds;
    return o;
}
void prog_add(Prog &P, const oh_op &o, int rk, double bytes) {
    if (o.nvb <= 0) return;
    P.ops.push_back(o);
    P.rk.push_back(rk);
    P.bytes.push_back(bytes);
    if (o.lds > P.lds) P.lds = o.lds;
}
void prog_mv(Prog &P, MvBuild &b) {
    // the graph step's launches of a few MB run on 1024 waves (measured
    // 0.4-0.6 us faster per 9-14 MB launch than 4096); the step kernel plans
    // for its resident waves
    mv_plan(b, P.waves, P.step ? 0 : 1024);
    oh_op o = op_new(OH_OP_MV, b.L.total_blocks, b.lds);
    o.tk = b.tk;
    o.u.mv = b.L;
    prog_add(P, o, mv_kind(b.tk), b.bytes);
}

extern "C" void ornith_hip_session_free(ornith_hip_session *s) {
    if (!s) return;
    (void)hipSetDevice(s->m->ctx->device);
    if (s->gbody) (void)hipGraphExecDestroy(s->gbody);
    if (s->gbody_x) (void)hipGraphExecDestroy(s->gbody_x);
    if (s->ghead) (void)hipGraphExecDestroy(s->ghead);
    if (s->bw.graph) (void)hipGraphExecDestroy(s->bw.graph);
    for (void *p : s->allocs) (void)hipFree(p);
    delete s;
}
int q8alloc(ornith_hip_session *s, Q8Buf &q, size_t n) {
    CHK(salloc(s, &q.qs, n));
    CHK(salloc(s, &q.d, n / 256 + 1));
    CHK(salloc(s, &q.bs, n / 16 + 16));
    CHK(salloc(s, &q.bp, n / 16 + 16));
    return ORNITH_HIP_OK;
}
Act act_of(const Q8Buf &q, const float *xf) {
    Act a; a.qs = q.qs; a.d = q.d; a.bs = q.bs; a.xf = xf; return a;
}
Act act_norm(const float *x, const float *w, float eps) {
    Act a; a.pro = OH_PRO_NORM; a.xf = x; a.nw = w; a.eps = eps; return a;
}
Act act_gnorm(const float *o, const float *sz, const double *runs, const float *w, float eps, int gdim,
                     int runs16) {
    Act a; a.pro = OH_PRO_GNORM; a.xf = o; a.xf2 = sz; a.xruns = runs; a.nw = w; a.eps = eps; a.gdim = gdim;
    a.runs16 = runs16;
    return a;
}
Act act_swiglu(const float *g, const float *u) {
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
    if (a.ne > 0) {
        A_(salloc(s, &s->rtag, (size_t)a.n_layers * (a.ne + 1)));
        A_(salloc(s, &s->mctr, (size_t)a.n_layers * 2));
        A_(salloc(s, &s->dmctr, (size_t)a.n_layers * 2));
    }
    {
        const char *e = getenv("ORNITH_HIP_EXACT_ATTN_MAX");
        if (e && *e) s->exact_max = s->pf_exact_max = atoi(e);
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
            A_(salloc(s, &y.Vh, (size_t)s->kvcap * a.nkv * a.hd));
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
    // a session long enough for matrix-core prompt chunks has the model's
    // prompt tiles built here, once per model, outside its prompts
    if (cap >= kMmqMinTokens) A_(pf_tiles(m, m->ctx->st));
#undef A_
    *out = s;
    return ORNITH_HIP_OK;
}

// ---- the token step ------------------------------------------------------------------------
// Algorithmic bytes of the small kernels (recorded by profile_step only).
double norm_bytes(int n, bool w) { return (double)n * (4.0 + (w ? 4.0 : 0.0) + 4.0 + 1.0 + 4.0 / 256 + 2.0 / 16); }

int build_body(ornith_hip_session *s, Prog &P) {
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
                            a.nh, a.nkv, a.hd, a.rope_dim, s->kvcap, a.eps, z.Vh};
                prog_add(P, o, K_ATTN_PREP, 4.0 * (2.0 * aqd + 2.0 * kvd + 2.0 * a.hd) + 8.0 * aqd +
                                                2.0 * (kvd + 4.0 * a.nkv));
            }
            const float scale = 1.0f / sqrtf((float)a.hd);
            // contexts up to exact_max: scores + the reference-order walk;
            // longer ones: flash chunks + merge (each pair exits for the other)
            const bool ex = s->qpos + 1 <= oh_exact_limit(s->exact_max, a.hd);
            oh_op_attn at;
            memset(&at, 0, sizeof at);
            at.qr = s->qr; at.gate = s->agate; at.Kt = z.Kt; at.Ks = z.Ks; at.Vq = z.Vq; at.Vs = z.Vs; at.Vh = z.Vh;
            at.scores = s->scores; at.part_o = s->fpo; at.part_ml = s->fpml; at.out = s->o;
            at.nh = a.nh; at.nkv = a.nkv; at.hd = a.hd; at.cap = s->kvcap; at.exact_max = s->exact_max;
            at.hb = oh_flash_form(a.nh, a.nkv, a.hd, s->flash_mfma); at.scale = scale;
            const double nchd = oh_flash_parts((int)T, s->kvcap, at.hb);
            // exact walk (its scores in LDS) or flash chunks, then the merge
            // of the chunks (which exits after an exact walk)
            const int nv_fl = oh_flash_nvb(a.nh, a.nkv, s->kvcap, at.hb);
            const int lds_fl = oh_flash_form_lds(a.nh, a.nkv, a.hd, at.hb);
            const double kvb = T * a.nkv * (a.hd + 4.0);          // one of K or V with its scales
            if (!P.step && ex && a.nh <= OH_EXACT2_GMAX * a.nkv) {
                // graph step, exact regime (the host picks this program
                // while the context fits the exact walk): the scores over
                // 64-position tiles of every KV head, then one block per
                // query head for the softmax and the output walk
                const int lim = oh_exact_limit(s->exact_max, a.hd);
                oh_op o3 = op_new(OH_OP_ATTN_SCORES, a.nkv * ((lim + 63) / 64), ((a.nh / a.nkv) * 4 + 64) * a.hd);
                o3.u.attn = at;
                prog_add(P, o3, K_ATTN_SCORES, kvb + 4.0 * T * a.nh + 4.0 * aqd);
                oh_op o4 = op_new(OH_OP_ATTN_WALK, a.nh, ((lim + 15) / 16 + 2) * 16 * 4);
                o4.u.attn = at;
                // the walk reads the f16 copy of the codes (2 bytes each) and the scales
                prog_add(P, o4, K_ATTN_WALK, T * a.nkv * (2.0 * a.hd + 4.0) + 4.0 * T * a.nh + 12.0 * aqd);
            } else {
                const int nv_ex = a.nh / (256 / a.hd), lds_ex = oh_exact_lds_bytes(a.hd, s->exact_max);
                oh_op o3 = op_new(OH_OP_ATTN_MAIN, nv_ex > nv_fl ? nv_ex : nv_fl, lds_ex > lds_fl ? lds_ex : lds_fl);
                o3.u.attn = at;
                prog_add(P, o3, K_ATTN_MAIN, ex ? 2.0 * kvb + 4.0 * T * a.nh + 12.0 * aqd
                                                : 2.0 * kvb + 4.0 * aqd + 8.0 * nchd * aqd);
                oh_op o4 = op_new(OH_OP_ATTN_COMBINE, a.nh * (a.hd / 64));
                o4.u.attn = at;
                prog_add(P, o4, K_ATTN_COMBINE, ex ? 0.0 : 4.0 * nchd * (aqd + 2.0 * a.nh) + 12.0 * aqd);
            }
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
            // per-head gated RMSNorm of the delta output inside the projection
            MvBuild b2;
            CHK(mv_add(b2, y.ssm_out,
                       act_gnorm(s->o, s->osz, s->oruns, (const float *)y.ssm_norm->A, a.eps, a.dv, 1), s->x, 1));
            if (!P.step && delta_fused() && a.dk == 128 && a.conv_k <= 8 && s->dmctr &&
                (y.ssm_out->type == OH_Q4_K || y.ssm_out->type == OH_Q6_K)) {
                // one launch: the delta step's blocks, then the projection's
                // blocks (first weights requested, then the arrival wait)
                mv_plan(b2, P.waves, 1024);
                if (b2.tk == (int)y.ssm_out->type && b2.lds <= 65536) {
                    oh_op f = op_new(OH_OP_DELTA_MV, o.nvb + b2.L.total_blocks, b2.lds);
                    f.tk = b2.tk;
                    f.u.dmv.mv = b2.L;
                    f.u.dmv.mv.rio = s->io;
                    f.u.dmv.d = o.u.delta;
                    f.u.dmv.arr = s->dmctr + (size_t)l * 2;
                    f.u.dmv.dep = s->dmctr + (size_t)l * 2 + 1;
                    f.u.dmv.nd = o.nvb;
                    prog_add(P, f, K_DELTA_MV, sb + b2.bytes);
                } else {
                    prog_add(P, o, K_DELTA, sb);
                    oh_op m = op_new(OH_OP_MV, b2.L.total_blocks, b2.lds);
                    m.tk = b2.tk;
                    m.u.mv = b2.L;
                    prog_add(P, m, mv_kind(b2.tk), b2.bytes);
                }
            } else {
                prog_add(P, o, K_DELTA, sb);
                prog_mv(P, b2);
            }
        }
        // FFN: post_attention_norm (formed inside the first FFN launch), then
        // MoE (or dense SwiGLU)
        const Act pn = act_norm(s->x, (const float *)y.post_norm->A, a.eps);
        if (a.ne > 0) {
            const int K = a.top_k, I = a.moe_inter, sI = a.shared_inter;
            const int IW = I > sI ? I : sI;   // row stride of the g/u buffers
            const bool paired = pairable(y.gate_exps, y.up_exps) && (!y.gate_sh || pairable(y.gate_sh, y.up_sh));
            // router in the experts launch (graph step): its segments come
            // first (the lowest blocks, dispatched first) and publish the
            // logits as tagged words; the expert blocks form the normalised
            // activation themselves, then route and stream their experts
            const bool fr = !P.step && paired && s->rtag && router_fused() && (a.ne == 256 || a.ne == 512) &&
                            K <= 64 && H <= 4096 && oh_qdot_can(y.router->type, H) &&
                            (!y.gate_inp_sh || oh_qdot_can(y.gate_inp_sh->type, H)) &&
                            oh_qdot_can(y.gate_exps->type, H) && (!y.gate_sh || oh_qdot_can(y.gate_sh->type, H));
            // the same with IQ2_XXS routed experts (their fallback rows, gate
            // and up as separate segments): each expert block forms the
            // normalised f32 activation, then routes from the tagged logits
            const bool fr2 = !fr && !P.step && s->rtag && router_fused() && (a.ne == 256 || a.ne == 512) &&
                             K <= 64 && H <= 4096 && oh_qdot_can(y.router->type, H) &&
                             (!y.gate_inp_sh || oh_qdot_can(y.gate_inp_sh->type, H)) &&
                             y.gate_exps->type == OH_IQ2_XXS && y.up_exps->type == OH_IQ2_XXS && !iq2_tree_on() &&
                             (!y.gate_sh || (oh_qdot_can(y.gate_sh->type, H) && oh_qdot_can(y.up_sh->type, H)));
            MvBuild b2;
            if (fr || fr2) {
                uint64_t *rt = s->rtag + (size_t)l * (a.ne + 1);
                CHK(mv_add(b2, y.router, pn, (float *)rt, 2));
                b2.L.s[b2.L.n - 1].tagp = s->io + OH_IO_SERIAL;
                if (y.gate_inp_sh) {
                    CHK(mv_add(b2, y.gate_inp_sh, pn, (float *)(rt + a.ne), 2));
                    b2.L.s[b2.L.n - 1].tagp = s->io + OH_IO_SERIAL;
                }
                if (fr) {
                    CHK(mv_add_pair(b2, y.gate_exps, y.up_exps, pn, s->h, s->eidx, K, IW));
                    if (y.gate_sh) CHK(mv_add_pair(b2, y.gate_sh, y.up_sh, pn, s->h + (size_t)K * IW));
                } else {
                    // the layout of the unfused launch: g and u, the shared
                    // expert's after the K routed slots (the down projection
                    // forms silu(g) * u)
                    CHK(mv_add(b2, y.gate_exps, pn, s->g, 0, s->eidx, K, IW, 0));
                    CHK(mv_add(b2, y.up_exps, pn, s->u, 0, s->eidx, K, IW, 0));
                    if (y.gate_sh) {
                        CHK(mv_add(b2, y.gate_sh, pn, s->g + (size_t)K * IW, 0));
                        CHK(mv_add(b2, y.up_sh, pn, s->u + (size_t)K * IW, 0));
                    }
                }
                b2.L.rtag = rt;
                b2.L.rio = s->io;
                b2.L.rsh = y.gate_inp_sh ? 1 : 0;
            } else {
                // router (+ shared-expert gate); its first block keeps the
                // normalised activation for the expert launch
                Act pst = pn;
                pst.oqs = s->xq.qs; pst.oqd = s->xq.d; pst.oqb = s->xq.bs; pst.oxf = s->xn;
                MvBuild b;
                CHK(mv_add(b, y.router, pst, s->rl, 0));
                if (y.gate_inp_sh) CHK(mv_add(b, y.gate_inp_sh, pn, s->shl, 0));
                prog_mv(P, b);
                const Act ax = act_of(s->xq, s->xn);
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
            const uint32_t dt = y.down_exps->type;
            const int nbd = I / 256, ns = K + (y.gate_sh ? 1 : 0);
            const int rps = nbd >= 1 ? 64 / nbd : 1;
            const int sq = (nbd * 272 + nbd * 36 + 15) & ~15, dlds = ns * sq + ns * I * 4 + ns * rps * 4;
            const bool fuse = paired && oh_qdot_can(dt, I) && nbd >= 1 && nbd <= 64 && ns <= 10 && dlds <= 65536 &&
                              (!P.step || I <= 1024) &&
                              (!y.gate_sh || (y.down_sh->type == dt && sI == I));
            if (fr || fr2) {
                // the router blocks' completion counter and the first gate/up
                // block (which clears the other parity's counter)
                b2.L.mctr = s->mctr + (size_t)l * 2;
                mv_plan(b2, P.waves, 1024);
                b2.L.pb0 = -1;
                for (int i = 0; i < b2.L.n; i++) {
                    const oh_mvseg &g = b2.L.s[i];
                    if (g.mode == 2) b2.L.nrb += g.bps * g.nsub;
                    if ((fr ? g.pair != 0 : g.eidx != nullptr) && b2.L.pb0 < 0) b2.L.pb0 = g.block0;
                }
                oh_op o = op_new(OH_OP_MV, b2.L.total_blocks, b2.lds);
                o.tk = b2.tk;
                o.u.mv = b2.L;
                prog_add(P, o, mv_kind(b2.tk), b2.bytes);
            } else {
                prog_mv(P, b2);
            }
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
                if (!P.step && 16 % nbd == 0) {
                    // narrow form: 16 / nb rows per block, four times the
                    // blocks, each requesting only its rows' weights
                    // (measured 9.3 -> 8.4 us per C3 launch, same bits)
                    const int rn = 16 / nbd;
                    D.narrow = 1;
                    o.nvb = (H + rn - 1) / rn;
                    o.lds = ns * sq + ns * I * 4 + ns * rn * 4;
                }
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

int build_head(ornith_hip_session *s, Prog &P) {
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
int run_prog(ornith_hip_session *s, const Prog &P, hipStream_t st) {
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

int enqueue_body(ornith_hip_session *s, hipStream_t st) {
    Prog P;
    CHK(build_body(s, P));
    CHK(run_prog(s, P, st));
    LAUNCH(K_ADVANCE, 8.0, oh_launch_advance(s->io, st));
    return ORNITH_HIP_OK;
}

int enqueue_head(ornith_hip_session *s, hipStream_t st) {
    Prog P;
    CHK(build_head(s, P));
    return run_prog(s, P, st);
}

// ---- the persistent step kernel -------------------------------------------------------------------
// ORNITH_HIP_STEP=1 selects the persistent step kernel for decode steps;
// otherwise each operation is its own launch (HIP graphs)
bool step_enabled() {
    const char *e = getenv("ORNITH_HIP_STEP");
    return e && e[0] == '1';
}

int step_upload(ornith_hip_session *s, const Prog &P, ornith_hip_session::StepProg &sp) {
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
int step_prepare(ornith_hip_session *s) {
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
int step_launch(ornith_hip_session *s, bool body, uint64_t *ts, bool advance) {
    const ornith_hip_session::StepProg &sp = body ? s->sp_body : s->sp_head;
    HCHK(oh_launch_step(sp.ops, sp.n, s->io, sp.ctrs, body ? OH_IO_EPOCH_BODY : OH_IO_EPOCH_HEAD,
                        body && advance ? 1 : 0, ts, s->step_grid, sp.lds, s->m->ctx->st));
    return ORNITH_HIP_OK;
}

// io[OH_IO_ERR]: a grid wait of a persistent kernel that gave up, or an
// expert pair list that would have overflowed (the list was left unwritten)
int step_check(ornith_hip_session *s) {
    int32_t err = 0;
    HCHK(hipMemcpy(&err, s->io + OH_IO_ERR, 4, hipMemcpyDeviceToHost));
    if (err & OH_ERR_WAIT) {
        seterr("decode step: a wait between workgroups timed out; the session state is undefined");
        return ORNITH_HIP_ERR_DEVICE;
    }
    if (err) {
        seterr("MoE: a token routed to one expert twice or outside the experts (router logits all NaN or -inf); "
               "the session state is undefined");
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
bool dec_enabled() {
    const char *e = getenv("ORNITH_HIP_DECODE");
    return e && e[0] == '1';
}

bool dq(const ornith_hip_tensor *W) { return W && oh_qdot_can(W->type, W->in) && W->in <= 8192; }

oh_dmv dmv_new(const uint64_t *x, const float *nw, int pro, int in, float eps) {
    oh_dmv M;
    memset(&M, 0, sizeof M);
    M.x = x; M.nw = nw; M.pro = pro; M.in = in; M.nb = in / 256; M.eps = eps;
    return M;
}
// one segment: W (and W2, paired) applied in nsub slots (stacked: slot k is
// the routed expert k); output slot k row r at y[k * ystride + r]
void dmv_seg(oh_dmv &M, const ornith_hip_tensor *W, const ornith_hip_tensor *W2, uint64_t *y, int nsub,
                    int ystride, int stacked, int mode, float *yp) {
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
bool dmv_ok(const oh_dmv &M) {
    const int t = M.s[0].type, nb = M.nb;
    const bool shape = t == OH_Q4_K ? (nb == 2 || nb == 4 || nb == 8 || nb == 16)
                     : t == OH_Q6_K ? (nb == 4 || nb == 8 || nb == 16) : (nb == 2 || nb == 4 || nb == 8);
    for (int i = 0; i < M.nseg; i++)
        if (M.s[i].type != t || (M.s[i].mode == 1 && M.nseg != 1)) return false;
    return shape && M.ne <= 1024;
}
// deal the steps to `waves` of the grid's 4 G waves from wave0 on, counted
// as the three stepping waves per workgroup; dynamic LDS of the operation
bool dmv_add(DecB &b, oh_dmv &M, int wave0, int waves, double bytes) {
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
double wbytes(const ornith_hip_tensor *W, int rows) { return (double)rows * gguf_nbytes(W->type, (uint64_t)W->in); }

// Build the program; false (with nothing built) when the model is outside it.
bool dec_build(ornith_hip_session *s, DecB &b) {
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
            const int lim = oh_exact_limit(s->exact_max, a.hd);
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
                        a.nh, a.nkv, a.hd, a.rope_dim, s->kvcap, a.eps, z.Vh};
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
int dec_prepare(ornith_hip_session *s) {
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

int dec_launch(ornith_hip_session *s, bool advance) {
    HCHK(oh_launch_decode(s->dec.ops, s->dec.n, s->io, advance ? 1 : 0, s->dec.grid, s->dec.lds, s->m->ctx->st));
    return ORNITH_HIP_OK;
}


int capture(ornith_hip_session *s, int (*fn)(ornith_hip_session *, hipStream_t), hipGraphExec_t *out) {
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

bool graphs_enabled() {
    const char *e = getenv("ORNITH_HIP_NO_GRAPH");
    return !(e && e[0] == '1');
}

// the graph step's attention regime for the next body launch: contexts up
// to the exact limit take the exact-walk program (its own graph)
bool body_exact(const ornith_hip_session *s) {
    return s->m->any_full && s->qpos + 1 <= oh_exact_limit(s->exact_max, s->m->a.hd);
}

int run_body(ornith_hip_session *s) {
    hipStream_t st = s->m->ctx->st;
    if (step_enabled()) {
        CHK(step_prepare(s));
        if (s->step_grid) { s->qpos++; return step_launch(s, true, nullptr); }
    }
    if (graphs_enabled()) {
        hipGraphExec_t &g = body_exact(s) ? s->gbody_x : s->gbody;
        if (!g) CHK(capture(s, enqueue_body, &g));
        HCHK(hipGraphLaunch(g, st));
    } else {
        CHK(enqueue_body(s, st));
    }
    s->qpos++;
    return ORNITH_HIP_OK;
}
int run_head(ornith_hip_session *s) {
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
int run_step(ornith_hip_session *s) {
    if (dec_enabled() && !step_enabled()) {
        CHK(dec_prepare(s));
        if (s->dec.grid) return dec_launch(s);
    }
    CHK(run_body(s));
    return run_head(s);
}

int sync_pos(ornith_hip_session *s) {
    s->qpos = s->pos;
    HCHK(hipMemcpyAsync(s->io, &s->pos, sizeof(int32_t), hipMemcpyHostToDevice, s->m->ctx->st));
    return ORNITH_HIP_OK;
}
