// oh_host_snapshot.cpp - state download in the reference layouts, ORNSESS session snapshots, GGUF-order tensor download.
#include "oh_engine.h"


// ---- state download in the reference layouts -------------------------------------------------
extern "C" int ornith_hip_session_get_delta(ornith_hip_session *s, int l, float *S) {
    const ornith_hip_arch &a = s->m->a;
    if (l < 0 || l >= a.n_layers || s->m->L[l].full) { seterr("layer %d has no delta state", l); return ORNITH_HIP_ERR_NOTFOUND; }
    HCHK(hipSetDevice(s->m->ctx->device));
    const size_t per = (size_t)a.dk * a.dv;
    HCHK(hipMemcpy(S, s->ls[l].S, (size_t)a.nv * per * 4, hipMemcpyDeviceToHost));   // [h][r][c] on both sides
    return ORNITH_HIP_OK;
}

extern "C" int ornith_hip_session_get_conv(ornith_hip_session *s, int l, float *win) {
    const ornith_hip_arch &a = s->m->a;
    if (l < 0 || l >= a.n_layers || s->m->L[l].full) { seterr("layer %d has no conv state", l); return ORNITH_HIP_ERR_NOTFOUND; }
    HCHK(hipSetDevice(s->m->ctx->device));
    const size_t cc = (size_t)(2 * a.nk * a.dk + a.nv * a.dv), wsz = (size_t)(a.conv_k - 1) * cc;
    // the window written by the last step lives in parity (pos & 1)
    HCHK(hipMemcpy(win, s->ls[l].conv + (size_t)(s->pos & 1) * wsz, wsz * 4, hipMemcpyDeviceToHost));
    return ORNITH_HIP_OK;
}

extern "C" int ornith_hip_session_get_kv(ornith_hip_session *s, int l, int8_t *Kq, float *Ks,
                                         int8_t *Vq, float *Vs) {
    const ornith_hip_arch &a = s->m->a;
    if (l < 0 || l >= a.n_layers || !s->m->L[l].full) { seterr("layer %d has no KV cache", l); return ORNITH_HIP_ERR_NOTFOUND; }
    HCHK(hipSetDevice(s->m->ctx->device));
    const int len = s->pos, cap = s->kvcap, hd = a.hd, nkv = a.nkv;
    std::vector<uint32_t> kt((size_t)nkv * (hd / 4) * cap);
    HCHK(hipMemcpy(kt.data(), s->ls[l].Kt, kt.size() * 4, hipMemcpyDeviceToHost));
    std::vector<int8_t> vt((size_t)nkv * cap * hd);
    HCHK(hipMemcpy(vt.data(), s->ls[l].Vq, vt.size(), hipMemcpyDeviceToHost));
    for (int t = 0; t < len; t++)
        for (int h = 0; h < nkv; h++)
            for (int i = 0; i < hd; i++) {
                const uint32_t w = kt[((size_t)h * (hd / 4) + i / 4) * cap + t];
                Kq[((size_t)t * nkv + h) * hd + i] = (int8_t)((w >> (8 * (i & 3))) & 0xff);
                Vq[((size_t)t * nkv + h) * hd + i] = vt[(((size_t)h * (cap / 16) + t / 16) * hd + i) * 16 + (t & 15)];
            }
    HCHK(hipMemcpy(Ks, s->ls[l].Ks, (size_t)len * nkv * 4, hipMemcpyDeviceToHost));
    HCHK(hipMemcpy(Vs, s->ls[l].Vs, (size_t)len * nkv * 4, hipMemcpyDeviceToHost));
    return ORNITH_HIP_OK;
}

// The last full-attention layer's attention inputs and output as the most
// recent evaluation left them: row < 0, the decode step's (the query heads
// after q_norm and RoPE, the output gate, and o = attention * sigmoid(gate)
// before attn_output's Q8_K, src/ornith_rforward.c:419-455); row >= 0, that
// row of the most recent prompt chunk. Only meaningful when the model's last
// layer is a full-attention layer (later linear layers reuse o). *pos: the
// position the row attended from.
extern "C" int ornith_hip_session_get_attn(ornith_hip_session *s, int row, float *q, float *gate, float *o,
                                           int32_t *pos) {
    const ornith_hip_arch &a = s->m->a;
    const size_t aq = (size_t)a.nh * a.hd;
    if (a.n_layers < 1 || !s->m->L[a.n_layers - 1].full) {
        seterr("get_attn: the last layer is not a full-attention layer");
        return ORNITH_HIP_ERR_UNSUPPORTED;
    }
    HCHK(hipSetDevice(s->m->ctx->device));
    HCHK(hipStreamSynchronize(s->m->ctx->st));
    const float *dq, *dg, *dout;
    if (row < 0) {
        if (s->pos < 1) { seterr("get_attn: no decode step yet"); return ORNITH_HIP_ERR_UNSUPPORTED; }
        dq = s->qr; dg = s->agate; dout = s->o;
        *pos = s->pos - 1;
    } else {
        if (row >= s->pf.last_T || !s->pf.QR) {
            seterr("get_attn: row %d outside the last prompt chunk (%d rows)", row, s->pf.last_T);
            return ORNITH_HIP_ERR_FORMAT;
        }
        dq = s->pf.QR + (size_t)row * aq; dg = s->pf.AG + (size_t)row * aq; dout = s->pf.OA + (size_t)row * aq;
        *pos = s->pf.last_base + row;
    }
    HCHK(hipMemcpy(q, dq, aq * 4, hipMemcpyDeviceToHost));
    HCHK(hipMemcpy(gate, dg, aq * 4, hipMemcpyDeviceToHost));
    HCHK(hipMemcpy(o, dout, aq * 4, hipMemcpyDeviceToHost));
    return ORNITH_HIP_OK;
}

// ---- session snapshots (rmodel_session_save / rmodel_session_load, src/ornith_rforward.c:986-1171) ----
// The reference's ORNSESS v1 file, byte for byte: magic, version, the
// architecture fingerprint (13 int32), pos, nhist, the FNV-1a 64 hash of the
// token history, have_logits; per layer the Q8 KV cache (quantized, len, nkv,
// hd, K codes, V codes [len][nkv][hd], K and V scales [len][nkv]) or the delta
// state [nv][dv][dk] and the conv window (K, C, [(K-1)][C] oldest first); the
// token history; the logits.
static const char kSessMagic[8] = {'O', 'R', 'N', 'S', 'E', 'S', 'S', '\0'};

// the f16 bit pattern of an integer V code (|c| <= 127: exact), the
// device's f16_bits_of_code
static uint16_t f16_of_code(int c) {
    if (c == 0) return 0;
    const uint16_t sgn = c < 0 ? 0x8000 : 0;
    const unsigned m = (unsigned)(c < 0 ? -c : c);
    const int e = 31 - __builtin_clz(m);
    return (uint16_t)(sgn | (unsigned)(e + 15) << 10 | (m - (1u << e)) << (10 - e));
}
static const uint32_t kSessVersion = 1;

void sess_fp(const ornith_hip_arch &a, int32_t fp[13]) {
    const int32_t v[13] = {a.hidden, a.n_layers, a.nh, a.nkv, a.hd, a.full_interval, a.nk, a.nv, a.dk, a.dv,
                           a.conv_k, a.ne, a.vocab};
    memcpy(fp, v, sizeof v);
}

uint64_t sess_prefix_hash(const int32_t *t, int n) {
    uint64_t h = 1469598103934665603ULL;
    const uint8_t *p = (const uint8_t *)t;
    for (size_t i = 0; i < (size_t)n * 4; i++) {
        h ^= p[i];
        h *= 1099511628211ULL;
    }
    return h;
}

extern "C" int ornith_hip_session_save(ornith_hip_session *s, const char *path) {
    const ornith_hip_arch &a = s->m->a;
    HCHK(hipSetDevice(s->m->ctx->device));
    HCHK(hipStreamSynchronize(s->m->ctx->st));
    const int pos = s->pos, cc = 2 * a.nk * a.dk + a.nv * a.dv;
    std::vector<int32_t> hist((size_t)pos + 1);
    if (pos > 0) HCHK(hipMemcpy(hist.data(), s->toks, (size_t)pos * 4, hipMemcpyDeviceToHost));
    std::vector<uint8_t> out;
    auto put = [&](const void *p, size_t n) { out.insert(out.end(), (const uint8_t *)p, (const uint8_t *)p + n); };
    auto put32 = [&](int32_t v) { put(&v, 4); };
    put(kSessMagic, 8);
    put(&kSessVersion, 4);
    int32_t fp[13];
    sess_fp(a, fp);
    put(fp, sizeof fp);
    const int32_t hl = s->have_logits ? 1 : 0;
    const uint64_t ph = sess_prefix_hash(hist.data(), pos);
    put32(pos);
    put32(pos);                                   // nhist: every token fed so far
    put(&ph, 8);
    put32(hl);
    for (int l = 0; l < a.n_layers; l++) {
        if (s->m->L[l].full) {
            const size_t hv = (size_t)pos * a.nkv * a.hd, sc = (size_t)pos * a.nkv;
            std::vector<int8_t> kq(hv + 1), vq(hv + 1);
            std::vector<float> ks(sc + 1), vs(sc + 1);
            CHK(ornith_hip_session_get_kv(s, l, kq.data(), ks.data(), vq.data(), vs.data()));
            put32(1); put32(pos); put32(a.nkv); put32(a.hd);
            put(kq.data(), hv); put(vq.data(), hv); put(ks.data(), sc * 4); put(vs.data(), sc * 4);
        } else {
            std::vector<float> S((size_t)a.nv * a.dv * a.dk), w((size_t)(a.conv_k - 1) * cc + 1);
            CHK(ornith_hip_session_get_delta(s, l, S.data()));
            CHK(ornith_hip_session_get_conv(s, l, w.data()));
            put(S.data(), S.size() * 4);
            put32(a.conv_k); put32(cc);
            put(w.data(), (size_t)(a.conv_k - 1) * cc * 4);
        }
    }
    put(hist.data(), (size_t)pos * 4);
    if (hl) {
        std::vector<float> lg((size_t)a.vocab);
        CHK(ornith_hip_session_logits(s, lg.data()));
        put(lg.data(), lg.size() * 4);
    }
    FILE *f = fopen(path, "wb");
    if (!f) { seterr("session save: cannot open %s", path); return ORNITH_HIP_ERR_IO; }
    const bool ok = fwrite(out.data(), 1, out.size(), f) == out.size();
    if (fclose(f) != 0 || !ok) { seterr("session save: write to %s failed", path); return ORNITH_HIP_ERR_IO; }
    return ORNITH_HIP_OK;
}

extern "C" int ornith_hip_session_load(ornith_hip_model *m, const char *path, int extra_cap,
                                       ornith_hip_session **out) {
    *out = nullptr;
    const ornith_hip_arch &a = m->a;
    FILE *f = fopen(path, "rb");
    if (!f) { seterr("session load: cannot open %s", path); return ORNITH_HIP_ERR_IO; }
    std::vector<uint8_t> buf;
    {
        uint8_t tmp[1 << 16];
        size_t n;
        while ((n = fread(tmp, 1, sizeof tmp, f)) > 0) buf.insert(buf.end(), tmp, tmp + n);
        fclose(f);
    }
    size_t at = 0;
    auto get = [&](void *p, size_t n) {
        if (at + n > buf.size()) return false;
        memcpy(p, buf.data() + at, n);
        at += n;
        return true;
    };
    char magic[8];
    uint32_t ver = 0;
    if (!get(magic, 8) || memcmp(magic, kSessMagic, 8) != 0) { seterr("session load: not a session file"); return ORNITH_HIP_ERR_FORMAT; }
    if (!get(&ver, 4) || ver != kSessVersion) { seterr("session load: unsupported version"); return ORNITH_HIP_ERR_FORMAT; }
    int32_t fp[13], cur[13];
    sess_fp(a, cur);
    if (!get(fp, sizeof fp)) { seterr("session load: truncated header"); return ORNITH_HIP_ERR_FORMAT; }
    if (memcmp(fp, cur, sizeof fp) != 0) {
        seterr("session load: arch fingerprint mismatch (snapshot is for a different model)");
        return ORNITH_HIP_ERR_FORMAT;
    }
    int32_t pos = 0, nhist = 0, hl = 0;
    uint64_t ph = 0;
    if (!get(&pos, 4) || !get(&nhist, 4) || !get(&ph, 8) || !get(&hl, 4)) { seterr("session load: truncated body"); return ORNITH_HIP_ERR_FORMAT; }
    if (pos < 0 || nhist != pos) {
        seterr("session load: %d history tokens for position %d (this engine keeps one per position)", nhist, pos);
        return ORNITH_HIP_ERR_UNSUPPORTED;
    }
    int cap = pos + (extra_cap > 0 ? extra_cap : 0);
    if (cap < 1) cap = 1;
    ornith_hip_session *s = nullptr;
    CHK(ornith_hip_session_new(m, cap, &s));
    auto fail = [&](int st, const char *msg) { ornith_hip_session_free(s); seterr("session load: %s", msg); return st; };
    const int cc = 2 * a.nk * a.dk + a.nv * a.dv, kc = s->kvcap, hd = a.hd, nkv = a.nkv;
    for (int l = 0; l < a.n_layers; l++) {
        LayerState &z = s->ls[l];
        if (m->L[l].full) {
            int32_t q, len, snkv, shd;
            if (!get(&q, 4) || !get(&len, 4) || !get(&snkv, 4) || !get(&shd, 4)) return fail(ORNITH_HIP_ERR_FORMAT, "truncated/corrupt");
            if (snkv != nkv || shd != hd || len > cap) return fail(ORNITH_HIP_ERR_FORMAT, "truncated/corrupt");
            if (!q) return fail(ORNITH_HIP_ERR_UNSUPPORTED, "an f32 KV cache (this engine keeps the Q8 cache)");
            if (len != pos) return fail(ORNITH_HIP_ERR_UNSUPPORTED, "a KV cache shorter than the position");
            const size_t hv = (size_t)len * nkv * hd, sc = (size_t)len * nkv;
            std::vector<int8_t> kq(hv + 1), vq(hv + 1);
            std::vector<float> ks(sc + 1), vs(sc + 1);
            if (!get(kq.data(), hv) || !get(vq.data(), hv) || !get(ks.data(), sc * 4) || !get(vs.data(), sc * 4))
                return fail(ORNITH_HIP_ERR_FORMAT, "truncated/corrupt");
            // into the device layouts: K words [kvh][hd/4][cap], V tiles [kvh][cap/16][hd][16]
            std::vector<uint32_t> kt((size_t)nkv * (hd / 4) * kc, 0u);
            std::vector<int8_t> vt((size_t)nkv * kc * hd, 0);
            std::vector<uint16_t> vh((size_t)nkv * kc * hd, 0);
            for (int t = 0; t < len; t++)
                for (int h = 0; h < nkv; h++)
                    for (int i = 0; i < hd; i++) {
                        const size_t src = ((size_t)t * nkv + h) * hd + i;
                        kt[((size_t)h * (hd / 4) + i / 4) * kc + t] |= (uint32_t)(uint8_t)kq[src] << (8 * (i & 3));
                        const size_t vo = (((size_t)h * (kc / 16) + t / 16) * hd + i) * 16 + (t & 15);
                        vt[vo] = vq[src];
                        vh[vo] = f16_of_code(vq[src]);
                    }
            if (hipMemcpy(z.Kt, kt.data(), kt.size() * 4, hipMemcpyHostToDevice) != hipSuccess ||
                hipMemcpy(z.Vq, vt.data(), vt.size(), hipMemcpyHostToDevice) != hipSuccess ||
                hipMemcpy(z.Vh, vh.data(), vh.size() * 2, hipMemcpyHostToDevice) != hipSuccess ||
                (sc && hipMemcpy(z.Ks, ks.data(), sc * 4, hipMemcpyHostToDevice) != hipSuccess) ||
                (sc && hipMemcpy(z.Vs, vs.data(), sc * 4, hipMemcpyHostToDevice) != hipSuccess))
                return fail(ORNITH_HIP_ERR_DEVICE, "upload failed");
        } else {
            const size_t ds = (size_t)a.nv * a.dv * a.dk;
            std::vector<float> S(ds);
            int32_t K, C;
            if (!get(S.data(), ds * 4) || !get(&K, 4) || !get(&C, 4)) return fail(ORNITH_HIP_ERR_FORMAT, "truncated/corrupt");
            if (K != a.conv_k || C != cc) return fail(ORNITH_HIP_ERR_FORMAT, "truncated/corrupt");
            const size_t wsz = (size_t)(K - 1) * C;
            std::vector<float> w(wsz + 1);
            if (!get(w.data(), wsz * 4)) return fail(ORNITH_HIP_ERR_FORMAT, "truncated/corrupt");
            // the window the next step reads lives in parity (pos & 1)
            if (hipMemcpy(z.S, S.data(), ds * 4, hipMemcpyHostToDevice) != hipSuccess ||
                hipMemcpy(z.conv + (size_t)(pos & 1) * wsz, w.data(), wsz * 4, hipMemcpyHostToDevice) != hipSuccess)
                return fail(ORNITH_HIP_ERR_DEVICE, "upload failed");
        }
    }
    std::vector<int32_t> hist((size_t)nhist + 1);
    if (!get(hist.data(), (size_t)nhist * 4)) return fail(ORNITH_HIP_ERR_FORMAT, "truncated/corrupt");
    std::vector<float> lg;
    if (hl) {
        lg.resize((size_t)a.vocab);
        if (!get(lg.data(), lg.size() * 4)) return fail(ORNITH_HIP_ERR_FORMAT, "truncated/corrupt");
    }
    if (sess_prefix_hash(hist.data(), nhist) != ph) return fail(ORNITH_HIP_ERR_FORMAT, "prefix hash mismatch (corrupt snapshot)");
    for (int i = 0; i < nhist; i++)
        if (hist[i] < 0 || hist[i] >= a.vocab) return fail(ORNITH_HIP_ERR_FORMAT, "history token outside the vocabulary");
    if (nhist > 0 && hipMemcpy(s->toks, hist.data(), (size_t)nhist * 4, hipMemcpyHostToDevice) != hipSuccess)
        return fail(ORNITH_HIP_ERR_DEVICE, "upload failed");
    if (hl) {
        // the logits, and their greedy token where the token step's head leaves
        // it (session_generate continues from there)
        hipStream_t st = m->ctx->st;
        if (hipMemcpy(s->logits, lg.data(), lg.size() * 4, hipMemcpyHostToDevice) != hipSuccess ||
            oh_launch_argmax_rows(s->logits, a.vocab, 1, s->toks + pos, st) != hipSuccess ||
            hipStreamSynchronize(st) != hipSuccess)
            return fail(ORNITH_HIP_ERR_DEVICE, "upload failed");
    }
    s->pos = pos;
    s->have_logits = hl != 0;
    *out = s;
    return ORNITH_HIP_OK;
}

// ---- GGUF-order download of a tensor (planes -> GGUF blocks) -------------------------------------
extern "C" int ornith_hip_tensor_download(const ornith_hip_tensor *t, void *out, uint64_t nbytes) {
    if (nbytes != t->gguf_bytes) {
        seterr("tensor '%s': %llu bytes requested, %llu held", t->name.c_str(), (unsigned long long)nbytes,
               (unsigned long long)t->gguf_bytes);
        return ORNITH_HIP_ERR_FORMAT;
    }
    HCHK(hipSetDevice(t->ctx->device));
    size_t a, b, c;
    plane_bytes(t->type, t->rows, t->in, &a, &b, &c);
    if (!oh_is_quant(t->type)) {
        HCHK(hipMemcpy(out, t->A, a, hipMemcpyDeviceToHost));
        return ORNITH_HIP_OK;
    }
    std::vector<uint8_t> h(up256(a) + up256(b) + up256(c));
    HCHK(hipMemcpy(h.data(), t->mem, h.size(), hipMemcpyDeviceToHost));
    const uint8_t *A = h.data(), *B = A + up256(a), *C = B + up256(b);
    uint8_t *o = (uint8_t *)out;
    const size_t nblk = (size_t)t->rows * (size_t)(t->in / 256);
    for (size_t i = 0; i < nblk; i++) {
        switch (t->type) {
        case OH_Q4_K:
            memcpy(o + 144 * i, B + 16 * i, 16);
            for (int k = 0; k < 128; k += 16) memcpy(o + 144 * i + 16 + k, A + oh_a_off(t->type, i, k), 16);
            break;
        case OH_Q6_K:
            for (int k = 0; k < 192; k += 16) memcpy(o + 210 * i + k, A + oh_a_off(t->type, i, k), 16);
            memcpy(o + 210 * i + 192, B + 16 * i, 16);
            memcpy(o + 210 * i + 208, C + 2 * i, 2);
            break;
        case OH_Q8_0:
            for (int k = 0; k < 8; k++) {
                memcpy(o + 272 * i + 34 * k, B + 16 * i + 2 * k, 2);
                memcpy(o + 272 * i + 34 * k + 2, A + oh_a_off(t->type, i, 32 * k), 16);
                memcpy(o + 272 * i + 34 * k + 18, A + oh_a_off(t->type, i, 32 * k + 16), 16);
            }
            break;
        case OH_IQ2_XXS: memcpy(o + 66 * i, C + 2 * i, 2); memcpy(o + 66 * i + 2, A + 64 * i, 64); break;
        }
    }
    return ORNITH_HIP_OK;
}
