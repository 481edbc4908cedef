// oh_host_synth.cpp - on-device random model synthesis (the generator's model on the device).
#include "oh_engine.h"


// ---- on-device random init ----------------------------------------------------------------------
// Stream key of a tensor: FNV-1a of its name xor seed*golden-gamma; element i
// of the stream depends only on (key, i) (counter-based splitmix64).
uint64_t stream_key(uint64_t seed, const std::string &name) {
    uint64_t h = 0xcbf29ce484222325ull;
    for (unsigned char ch : name) { h ^= ch; h *= 0x100000001b3ull; }
    return h ^ (seed * 0x9E3779B97F4A7C15ull);
}

extern "C" int ornith_hip_model_synth(ornith_hip_ctx *ctx, const ornith_hip_gen_cfg *c,
                                      ornith_hip_model **out) {
    *out = nullptr;
    HCHK(hipSetDevice(ctx->device));
    auto enc_ok = [](uint32_t t) {
        return t == OH_Q8_0 || t == OH_Q4_K || t == OH_Q6_K || t == OH_IQ2_XXS || t == OH_F32;
    };
    if (!enc_ok(c->t_default) || !enc_ok(c->t_attn_v) || !enc_ok(c->t_ffn_down) || !enc_ok(c->t_output) ||
        !enc_ok(c->t_embd) || (c->t_exps && !enc_ok(c->t_exps))) {
        seterr("model_synth: on-device encoders cover F32/Q8_0/Q4_K/Q6_K/IQ2_XXS");
        return ORNITH_HIP_ERR_UNSUPPORTED;
    }
    if (c->hidden <= 0 || c->n_layers <= 0 || c->vocab <= 0 || c->dhead <= 0 || c->conv_k < 2 || c->conv_k > 8) {
        seterr("model_synth: bad config");
        return ORNITH_HIP_ERR_FORMAT;
    }
    const int H = c->hidden, V = c->vocab, qd = c->nk * c->dhead, vd = c->nv * c->dhead, cc = 2 * qd + vd;
    // largest tensor (elements) sizes the f32 staging buffer
    uint64_t mx = (uint64_t)H * V;
    auto upd = [&](uint64_t n) { if (n > mx) mx = n; };
    upd((uint64_t)H * cc); upd((uint64_t)H * 2 * c->nh * c->hd); upd((uint64_t)H * c->moe_inter * c->ne);
    upd((uint64_t)c->nh * c->hd * H); upd((uint64_t)vd * H); upd((uint64_t)H * c->shared_inter);
    float *tmp = nullptr;
    HCHK(hipMalloc(&tmp, mx * 4 + 256));
    auto *m = new ornith_hip_model();
    m->ctx = ctx;
    hipStream_t st = ctx->st;
    int status = ORNITH_HIP_OK;
    auto add_q = [&](const std::string &name, uint32_t type, int nd, uint64_t d0, uint64_t d1, uint64_t d2) {
        if (status) return;
        const uint64_t dims[3] = {d0, d1, d2};
        ornith_hip_tensor *t;
        if ((status = tensor_alloc(ctx, name.c_str(), type, (uint32_t)nd, dims, &t))) return;
        m->ts.push_back(t); m->by[name] = t; m->bytes += t->gguf_bytes;
        const int64_t n = t->rows * t->in;
        float *dst = type == OH_F32 ? (float *)t->A : tmp;
        hipError_t e = oh_launch_fill_gauss(stream_key(c->seed, name), c->sigma, dst, n, st);
        if (e == hipSuccess && type != OH_F32) e = oh_launch_encode(tmp, (int)type, n / 256, t->A, t->B, t->C, st);
        if (e == hipSuccess) e = hipStreamSynchronize(st);   // tmp is reused by the next tensor
        if (e != hipSuccess) { seterr("synth '%s': %s", name.c_str(), hipGetErrorString(e)); status = ORNITH_HIP_ERR_DEVICE; }
    };
    auto add_u = [&](const std::string &name, int nd, uint64_t d0, uint64_t d1, float lo, float hi) {
        if (status) return;
        const uint64_t dims[2] = {d0, d1};
        ornith_hip_tensor *t;
        if ((status = tensor_alloc(ctx, name.c_str(), OH_F32, (uint32_t)nd, dims, &t))) return;
        m->ts.push_back(t); m->by[name] = t; m->bytes += t->gguf_bytes;
        hipError_t e = oh_launch_fill_uniform(stream_key(c->seed, name), lo, hi, (float *)t->A, t->rows * t->in, st);
        if (e != hipSuccess) { seterr("synth '%s': %s", name.c_str(), hipGetErrorString(e)); status = ORNITH_HIP_ERR_DEVICE; }
    };
    // ORNITH_HIP_VERBOSE=1: one line per synthesised layer on stderr (a large
    // model with IQ2_XXS experts takes minutes)
    const char *vb = getenv("ORNITH_HIP_VERBOSE");
    const bool verbose = vb && vb[0] == '1';
    // same tensor set and order as the GGUF generator
    add_q("token_embd.weight", c->t_embd, 2, H, V, 0);
    add_u("output_norm.weight", 1, H, 0, 0.9f, 1.1f);
    add_q("output.weight", c->t_output, 2, H, V, 0);
    for (int l = 0; l < c->n_layers; l++) {
        const bool full = c->full_interval > 0 && l % c->full_interval == c->full_interval - 1;
        const std::string b = "blk." + std::to_string(l) + ".";
        add_u(b + "attn_norm.weight", 1, H, 0, 0.9f, 1.1f);
        add_u(b + "post_attention_norm.weight", 1, H, 0, 0.9f, 1.1f);
        if (full) {
            add_q(b + "attn_q.weight", c->t_default, 2, H, 2 * c->nh * c->hd, 0);
            add_q(b + "attn_k.weight", c->t_default, 2, H, c->nkv * c->hd, 0);
            add_q(b + "attn_v.weight", c->t_attn_v, 2, H, c->nkv * c->hd, 0);
            add_u(b + "attn_q_norm.weight", 1, c->hd, 0, 0.9f, 1.1f);
            add_u(b + "attn_k_norm.weight", 1, c->hd, 0, 0.9f, 1.1f);
            add_q(b + "attn_output.weight", c->t_default, 2, c->nh * c->hd, H, 0);
        } else {
            add_q(b + "attn_qkv.weight", c->t_default, 2, H, cc, 0);
            add_u(b + "ssm_conv1d.weight", 2, c->conv_k, cc, -0.2f, 0.2f);
            add_u(b + "ssm_a", 1, c->nv, 0, -0.8f, -0.2f);
            add_u(b + "ssm_dt.bias", 1, c->nv, 0, -0.05f, 0.05f);
            add_u(b + "ssm_norm.weight", 1, c->dhead, 0, 0.9f, 1.1f);
            add_q(b + "ssm_alpha.weight", c->t_default, 2, H, c->nv, 0);
            add_q(b + "ssm_beta.weight", c->t_default, 2, H, c->nv, 0);
            add_q(b + "attn_gate.weight", c->t_default, 2, H, vd, 0);
            add_q(b + "ssm_out.weight", c->t_default, 2, vd, H, 0);
        }
        if (c->ne <= 0) {
            // dense SwiGLU FFN of width shared_inter
            add_q(b + "ffn_gate.weight", c->t_default, 2, H, c->shared_inter, 0);
            add_q(b + "ffn_up.weight", c->t_default, 2, H, c->shared_inter, 0);
            add_q(b + "ffn_down.weight", c->t_ffn_down, 2, c->shared_inter, H, 0);
            continue;
        }
        add_q(b + "ffn_gate_inp.weight", c->t_default, 2, H, c->ne, 0);
        add_q(b + "ffn_gate_exps.weight", c->t_exps ? c->t_exps : c->t_default, 3, H, c->moe_inter, c->ne);
        add_q(b + "ffn_up_exps.weight", c->t_exps ? c->t_exps : c->t_default, 3, H, c->moe_inter, c->ne);
        add_q(b + "ffn_down_exps.weight", c->t_exps ? c->t_exps : c->t_ffn_down, 3, c->moe_inter, H, c->ne);
        if (c->shared_inter > 0) {
            add_q(b + "ffn_gate_shexp.weight", c->t_default, 2, H, c->shared_inter, 0);
            add_q(b + "ffn_up_shexp.weight", c->t_default, 2, H, c->shared_inter, 0);
            add_q(b + "ffn_down_shexp.weight", c->t_ffn_down, 2, c->shared_inter, H, 0);
            add_q(b + "ffn_gate_inp_shexp.weight", c->t_default, 1, H, 1, 0);
        }
        if (verbose && !status) {
            fprintf(stderr, "model_synth: layer %d/%d done, %.2f GB\n", l + 1, c->n_layers, (double)m->bytes / 1e9);
            fflush(stderr);
        }
    }
    (void)hipStreamSynchronize(st);
    (void)hipFree(tmp);
    if (status) { ornith_hip_model_free(m); return status; }
    Meta md;
    md.arch = "qwen35moe";
    md.u32["qwen35moe.block_count"] = (uint32_t)c->n_layers;
    md.u32["qwen35moe.expert_used_count"] = (uint32_t)c->top_k;
    md.u32["qwen35moe.rope.dimension_count"] = 64;
    md.f32["qwen35moe.rope.freq_base"] = 1e7f;
    md.f32["qwen35moe.attention.layer_norm_rms_epsilon"] = 1e-6f;
    md.has_tokens = true;
    md.eos = -1;
    const int st2 = infer_arch(m, md);
    if (st2) { ornith_hip_model_free(m); return st2; }
    *out = m;
    return ORNITH_HIP_OK;
}
