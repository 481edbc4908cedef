// oh_host_model.cpp - GGUF v3 mmap reader, model load and upload into the plane layout, arch inference.
#include "oh_engine.h"


// ---- GGUF v3 mmap reader (format: src/ornith_gguf_write.c:1-11) --------------------------
namespace {

struct GgufKV { uint32_t vt; const uint8_t *val; size_t len; };
struct GgufT { std::string name; uint32_t nd, type; uint64_t dims[4]; uint64_t off; const uint8_t *data; uint64_t nbytes; };

struct Gguf {
    uint8_t *map = nullptr;
    size_t size = 0;
    std::unordered_map<std::string, GgufKV> kv;
    std::vector<GgufT> ts;
    ~Gguf() { if (map) munmap(map, size); }
};

struct Rd {
    const uint8_t *p, *end;
    bool take(void *dst, size_t n) {
        if ((size_t)(end - p) < n) return false;
        if (dst) memcpy(dst, p, n);
        p += n;
        return true;
    }
};

size_t gguf_scalar(uint32_t vt) {
    switch (vt) {
    case 0: case 1: case 7: return 1;
    case 2: case 3: return 2;
    case 4: case 5: case 6: return 4;
    case 10: case 11: case 12: return 8;
    default: return 0;
    }
}

bool gguf_skip(Rd &r, uint32_t vt, int depth) {
    if (vt == 8) { uint64_t n; return r.take(&n, 8) && r.take(nullptr, n); }
    if (vt == 9) {
        uint32_t et; uint64_t n;
        if (depth > 3 || !r.take(&et, 4) || !r.take(&n, 8)) return false;
        for (uint64_t i = 0; i < n; i++) if (!gguf_skip(r, et, depth + 1)) return false;
        return true;
    }
    const size_t s = gguf_scalar(vt);
    return s && r.take(nullptr, s);
}

int gguf_open(const char *path, Gguf &g) {
    const int fd = open(path, O_RDONLY);
    if (fd < 0) { seterr("cannot open %s", path); return ORNITH_HIP_ERR_IO; }
    struct stat st;
    if (fstat(fd, &st) != 0) { close(fd); seterr("fstat %s failed", path); return ORNITH_HIP_ERR_IO; }
    g.size = (size_t)st.st_size;
    void *m = g.size ? mmap(nullptr, g.size, PROT_READ, MAP_PRIVATE, fd, 0) : MAP_FAILED;
    close(fd);
    if (m == MAP_FAILED) { g.size = 0; seterr("mmap %s failed", path); return ORNITH_HIP_ERR_IO; }
    g.map = (uint8_t *)m;
    Rd r{g.map, g.map + g.size};
    char magic[4];
    uint32_t ver;
    uint64_t nt, nkv;
    if (!r.take(magic, 4) || memcmp(magic, "GGUF", 4) != 0) { seterr("not a GGUF file (bad magic)"); return ORNITH_HIP_ERR_FORMAT; }
    if (!r.take(&ver, 4) || !r.take(&nt, 8) || !r.take(&nkv, 8)) { seterr("truncated GGUF header"); return ORNITH_HIP_ERR_FORMAT; }
    if (ver < 2 || ver > 3) { seterr("unsupported GGUF version %u", ver); return ORNITH_HIP_ERR_UNSUPPORTED; }
    if (nt > (1u << 24) || nkv > (1u << 24)) { seterr("implausible GGUF counts"); return ORNITH_HIP_ERR_FORMAT; }
    uint32_t align = 32;
    for (uint64_t i = 0; i < nkv; i++) {
        uint64_t kl;
        if (!r.take(&kl, 8) || (size_t)(r.end - r.p) < kl) { seterr("bad GGUF key #%llu", (unsigned long long)i); return ORNITH_HIP_ERR_FORMAT; }
        std::string key((const char *)r.p, kl);
        r.p += kl;
        GgufKV v;
        if (!r.take(&v.vt, 4)) { seterr("bad GGUF value type for '%s'", key.c_str()); return ORNITH_HIP_ERR_FORMAT; }
        v.val = r.p;
        if (!gguf_skip(r, v.vt, 0)) { seterr("bad GGUF value for '%s'", key.c_str()); return ORNITH_HIP_ERR_FORMAT; }
        v.len = (size_t)(r.p - v.val);
        if (key == "general.alignment" && v.vt == 4 && v.len >= 4) { uint32_t a; memcpy(&a, v.val, 4); if (a) align = a; }
        g.kv[key] = v;
    }
    g.ts.resize(nt);
    for (uint64_t i = 0; i < nt; i++) {
        GgufT &t = g.ts[i];
        uint64_t nl;
        if (!r.take(&nl, 8) || (size_t)(r.end - r.p) < nl) { seterr("bad GGUF tensor record #%llu", (unsigned long long)i); return ORNITH_HIP_ERR_FORMAT; }
        t.name.assign((const char *)r.p, nl);
        r.p += nl;
        if (!r.take(&t.nd, 4) || t.nd > 4 || t.nd < 1) { seterr("tensor '%s': bad dims", t.name.c_str()); return ORNITH_HIP_ERR_FORMAT; }
        uint64_t n = 1;
        for (uint32_t d = 0; d < t.nd; d++) {
            if (!r.take(&t.dims[d], 8)) { seterr("tensor '%s': bad dims", t.name.c_str()); return ORNITH_HIP_ERR_FORMAT; }
            n *= t.dims[d];
        }
        if (!r.take(&t.type, 4) || !r.take(&t.off, 8)) { seterr("tensor '%s': bad type/offset", t.name.c_str()); return ORNITH_HIP_ERR_FORMAT; }
        t.nbytes = gguf_nbytes(t.type, n);
        if (!t.nbytes && n) { seterr("tensor '%s': cannot size type %u for load", t.name.c_str(), t.type); return ORNITH_HIP_ERR_UNSUPPORTED; }
    }
    const size_t data0 = ((size_t)(r.p - g.map) + align - 1) / align * align;
    if (data0 > g.size) { seterr("data section starts past EOF"); return ORNITH_HIP_ERR_FORMAT; }
    for (auto &t : g.ts) {
        if (t.off > g.size - data0 || t.nbytes > g.size - data0 - t.off) {
            seterr("tensor '%s' data extends past EOF", t.name.c_str());
            return ORNITH_HIP_ERR_FORMAT;
        }
        t.data = g.map + data0 + t.off;
    }
    return ORNITH_HIP_OK;
}

} // namespace

extern "C" void ornith_hip_model_free(ornith_hip_model *m) {
    if (!m) return;
    for (auto *t : m->ts) ornith_hip_tensor_free(t);
    delete m;
}

ornith_hip_tensor *mt(const ornith_hip_model *m, const std::string &n) {
    auto it = m->by.find(n);
    return it == m->by.end() ? nullptr : it->second;
}
ornith_hip_tensor *mb(const ornith_hip_model *m, int l, const char *sfx) {
    return mt(m, "blk." + std::to_string(l) + "." + sfx);
}

bool is_full(const ornith_hip_arch &a, int l) {
    return a.full_interval > 0 && l % a.full_interval == a.full_interval - 1;
}

// shape inference of rmodel_load (src/ornith_rforward.c:728-803) + the engine's
// own limits, checked loudly
int infer_arch(ornith_hip_model *m, const Meta &md) {
    ornith_hip_arch &a = m->a;
    memset(&a, 0, sizeof a);
    auto U = [&](const char *sfx, uint32_t def) {
        auto it = md.u32.find(md.arch + "." + sfx);
        return it == md.u32.end() ? def : it->second;
    };
    auto Fl = [&](const char *sfx, float def) {
        auto it = md.f32.find(md.arch + "." + sfx);
        return it == md.f32.end() ? def : it->second;
    };
    m->embd = mt(m, "token_embd.weight");
    a.hidden = m->embd ? (int)m->embd->dims[0] : (int)U("embedding_length", 4096);
    a.vocab = m->embd ? (int)m->embd->dims[1] : 248320;
    int n = 0;
    while (mb(m, n, "attn_norm.weight")) n++;
    a.n_layers = n ? n : (int)U("block_count", 32);
    int ff = -1;
    for (int i = 0; i < a.n_layers; i++) if (mb(m, i, "attn_q.weight")) { ff = i; break; }
    a.full_interval = ff >= 0 ? ff + 1 : (int)U("full_attention_interval", 4);
    a.rope_theta = Fl("rope.freq_base", 1e7f);
    a.eps = Fl("attention.layer_norm_rms_epsilon", 1e-6f);
    a.rope_dim = (int)U("rope.dimension_count", 64);
    {
        const int fl = a.full_interval - 1;
        auto *qn = mb(m, fl, "attn_q_norm.weight"), *q = mb(m, fl, "attn_q.weight"), *k = mb(m, fl, "attn_k.weight");
        a.hd = qn ? (int)qn->dims[0] : 256;
        const int qout = q ? (int)q->dims[1] : a.hd * 16;
        a.nh = (qout / 2) / a.hd;
        a.nkv = k ? (int)k->dims[1] / a.hd : 4;
    }
    {
        int l0 = 0;
        while (l0 < a.n_layers && is_full(a, l0)) l0++;
        auto *sa = mb(m, l0, "ssm_a"), *sn = mb(m, l0, "ssm_norm.weight"), *qkv = mb(m, l0, "attn_qkv.weight"),
             *cv = mb(m, l0, "ssm_conv1d.weight");
        a.nv = sa ? (int)sa->dims[0] : 32;
        a.dv = sn ? (int)sn->dims[0] : 128;
        a.dk = a.dv;
        a.conv_k = cv ? (int)cv->dims[0] : 4;
        const int cc = qkv ? (int)qkv->dims[1] : 8192;
        const int qd = (cc - a.nv * a.dv) / 2;
        a.nk = a.dk ? qd / a.dk : 16;
    }
    auto *ge0 = mb(m, 0, "ffn_gate_exps.weight");
    if (ge0) {
        a.ne = (int)ge0->dims[2];
        a.moe_inter = (int)ge0->dims[1];
        a.top_k = (int)U("expert_used_count", 8);
        auto *sh = mb(m, 0, "ffn_gate_shexp.weight");
        a.shared_inter = sh ? (int)sh->dims[1] : 0;
    } else {
        auto *fg = mb(m, 0, "ffn_gate.weight");
        a.shared_inter = fg ? (int)fg->dims[1] : (int)U("feed_forward_length", 12288);
    }
    if (!md.has_tokens) { seterr("no tokenizer.ggml.tokens"); return ORNITH_HIP_ERR_FORMAT; }
    a.eos = md.eos;
    m->out_norm = mt(m, "output_norm.weight");
    m->lm_head = mt(m, "output.weight");
    m->L.assign((size_t)a.n_layers, OhLayer());
    for (int l = 0; l < a.n_layers; l++) {
        OhLayer &y = m->L[l];
        y.full = is_full(a, l);
        m->any_full = m->any_full || y.full;
        y.attn_norm = mb(m, l, "attn_norm.weight"); y.post_norm = mb(m, l, "post_attention_norm.weight");
        y.q = mb(m, l, "attn_q.weight"); y.k = mb(m, l, "attn_k.weight"); y.v = mb(m, l, "attn_v.weight");
        y.o = mb(m, l, "attn_output.weight");
        y.q_norm = mb(m, l, "attn_q_norm.weight"); y.k_norm = mb(m, l, "attn_k_norm.weight");
        y.qkv = mb(m, l, "attn_qkv.weight"); y.conv = mb(m, l, "ssm_conv1d.weight");
        y.ssm_a = mb(m, l, "ssm_a"); y.dt_bias = mb(m, l, "ssm_dt.bias"); y.ssm_norm = mb(m, l, "ssm_norm.weight");
        y.alpha = mb(m, l, "ssm_alpha.weight"); y.beta = mb(m, l, "ssm_beta.weight");
        y.gate = mb(m, l, "attn_gate.weight"); y.ssm_out = mb(m, l, "ssm_out.weight");
        y.router = mb(m, l, "ffn_gate_inp.weight");
        y.gate_exps = mb(m, l, "ffn_gate_exps.weight"); y.up_exps = mb(m, l, "ffn_up_exps.weight");
        y.down_exps = mb(m, l, "ffn_down_exps.weight");
        y.gate_sh = mb(m, l, "ffn_gate_shexp.weight"); y.up_sh = mb(m, l, "ffn_up_shexp.weight");
        y.down_sh = mb(m, l, "ffn_down_shexp.weight"); y.gate_inp_sh = mb(m, l, "ffn_gate_inp_shexp.weight");
        y.ffn_gate = mb(m, l, "ffn_gate.weight"); y.ffn_up = mb(m, l, "ffn_up.weight"); y.ffn_down = mb(m, l, "ffn_down.weight");
    }
    // ---- what this engine supports (checked, never assumed) ----
    auto bad = [&](const char *why) { seterr("unsupported model: %s", why); return ORNITH_HIP_ERR_UNSUPPORTED; };
    auto need_f32 = [&](const ornith_hip_tensor *t) { return t && t->type == OH_F32; };
    if (!m->embd || !m->out_norm || !m->lm_head) return bad("token_embd/output_norm/output missing");
    if (a.hidden % 256 || a.hidden > 8192) return bad("hidden must be a multiple of 256, <= 8192");
    if (!need_f32(m->out_norm)) return bad("output_norm must be F32 (read as raw floats)");
    for (int l = 0; l < a.n_layers; l++) {
        const OhLayer &y = m->L[l];
        if (!need_f32(y.attn_norm) || !need_f32(y.post_norm)) return bad("layer norms must be F32");
        if (y.full) {
            if (!y.q || !y.k || !y.v || !y.o || !need_f32(y.q_norm) || !need_f32(y.k_norm)) return bad("full-attention tensors missing or not F32 norms");
            if (a.hd != 64 && a.hd != 128 && a.hd != 256) return bad("head_dim must be 64, 128 or 256");
            if (a.nh % a.nkv || a.nh / a.nkv > 16 || (a.nh / a.nkv & (a.nh / a.nkv - 1)))
                return bad("query heads per KV head must be a power of two <= 16");
            if (a.nkv < 1 || a.nh % a.nkv) return bad("n_heads must be a multiple of n_kv_heads");
            if ((a.nh * a.hd) % 256 || a.nh * a.hd > 8192) return bad("n_heads*head_dim must be a multiple of 256, <= 8192");
        } else {
            if (!y.qkv || !y.alpha || !y.beta || !y.gate || !y.ssm_out) return bad("linear-attention projections missing");
            if (!need_f32(y.conv) || !need_f32(y.ssm_a) || !need_f32(y.dt_bias) || !need_f32(y.ssm_norm))
                return bad("ssm_conv1d/ssm_a/ssm_dt.bias/ssm_norm must be F32");
            if (a.dk != 64 && a.dk != 128) return bad("linear head dim must be 64 or 128");
            if (a.nv % (256 / a.dk) || a.nk < 1) return bad("linear value heads must fill 256-element blocks");
            if (a.conv_k < 2 || a.conv_k > 8) return bad("conv kernel must be in [2, 8]");
            if (a.nv * a.dv > 8192) return bad("linear value width must be <= 8192");
        }
        if (a.ne > 0) {
            if (!y.router || !y.gate_exps || !y.up_exps || !y.down_exps) return bad("MoE tensors missing");
            if (a.ne > 1024 || a.top_k < 1 || a.top_k > 16 || a.top_k > a.ne) return bad("experts <= 1024 and 1 <= top_k <= 16");
            if (a.moe_inter % 256 || a.moe_inter > 8192) return bad("expert FFN width must be a multiple of 256, <= 8192");
            if (y.gate_sh && (a.shared_inter % 256 || a.shared_inter > 8192)) return bad("shared FFN width must be a multiple of 256");
        } else {
            if (!y.ffn_gate || !y.ffn_up || !y.ffn_down) return bad("dense FFN tensors missing");
            if (a.shared_inter % 256 || a.shared_inter > 8192) return bad("FFN width must be a multiple of 256");
        }
    }
    return ORNITH_HIP_OK;
}

extern "C" int ornith_hip_model_load(ornith_hip_ctx *ctx, const char *path, ornith_hip_model **out) {
    *out = nullptr;
    HCHK(hipSetDevice(ctx->device));
    Gguf g;
    CHK(gguf_open(path, g));
    Meta md;
    auto it = g.kv.find("general.architecture");
    if (it != g.kv.end() && it->second.vt == 8 && it->second.len >= 8) {
        uint64_t n;
        memcpy(&n, it->second.val, 8);
        if (n <= it->second.len - 8 && n < 64) md.arch.assign((const char *)it->second.val + 8, n);
    }
    for (auto &kv : g.kv) {
        if ((kv.second.vt == 4 || kv.second.vt == 5) && kv.second.len >= 4) { uint32_t v; memcpy(&v, kv.second.val, 4); md.u32[kv.first] = v; }
        if (kv.second.vt == 6 && kv.second.len >= 4) { float v; memcpy(&v, kv.second.val, 4); md.f32[kv.first] = v; }
    }
    md.has_tokens = g.kv.count("tokenizer.ggml.tokens") > 0;
    auto ie = g.kv.find("tokenizer.ggml.eos_token_id");
    if (ie != g.kv.end() && ie->second.len >= 4) memcpy(&md.eos, ie->second.val, 4);
    auto *m = new ornith_hip_model();
    m->ctx = ctx;
    for (auto &t : g.ts) {
        ornith_hip_tensor *dt;
        int st = ornith_hip_upload(ctx, t.name.c_str(), t.type, t.data, t.nbytes, t.nd, t.dims, &dt);
        if (st) { ornith_hip_model_free(m); return st; }
        m->ts.push_back(dt);
        m->by[t.name] = dt;
        m->bytes += dt->gguf_bytes;
    }
    int st = infer_arch(m, md);
    if (st) { ornith_hip_model_free(m); return st; }
    *out = m;
    return ORNITH_HIP_OK;
}

extern "C" int ornith_hip_model_arch(const ornith_hip_model *m, ornith_hip_arch *out) {
    *out = m->a;
    return ORNITH_HIP_OK;
}
extern "C" uint64_t ornith_hip_model_bytes(const ornith_hip_model *m) { return m->bytes; }
extern "C" const ornith_hip_tensor *ornith_hip_model_tensor(const ornith_hip_model *m, const char *name) {
    return mt(m, name);
}
extern "C" int ornith_hip_model_tensor_info(const ornith_hip_model *m, const char *name, uint32_t *type,
                                            uint64_t *nbytes, uint64_t *rows, uint64_t *in) {
    auto *t = mt(m, name);
    if (!t) { seterr("no tensor '%s'", name); return ORNITH_HIP_ERR_NOTFOUND; }
    if (type) *type = t->type;
    if (nbytes) *nbytes = t->gguf_bytes;
    if (rows) *rows = (uint64_t)t->rows;
    if (in) *in = (uint64_t)t->in;
    return ORNITH_HIP_OK;
}
