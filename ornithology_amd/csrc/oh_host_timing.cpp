// oh_host_timing.cpp - per-launch timing of one eager step and phase clocks of the persistent kernels.
#include "oh_engine.h"


// ---- one eager step with per-launch timing (HIP events around every launch) ------------------------
extern "C" int ornith_hip_session_time_kind(ornith_hip_session *s, int kind, int reps, float *us_per_launch,
                                            double *bytes_per_launch, int *launches_per_step) {
    *us_per_launch = 0.0f;
    *bytes_per_launch = 0.0;
    *launches_per_step = 0;
    if (!s->have_logits) { seterr("session has no logits; eval a prompt first"); return ORNITH_HIP_ERR_FORMAT; }
    if (kind < 0 || reps < 1) { seterr("time_kind: kind %d reps %d", kind, reps); return ORNITH_HIP_ERR_FORMAT; }
    HCHK(hipSetDevice(s->m->ctx->device));
    hipStream_t st = s->m->ctx->st;
    CHK(sync_pos(s));
    HCHK(hipStreamSynchronize(st));
    if (kind == K_STEP_BODY || kind == K_STEP_HEAD) {
        // back-to-back launches of one step-kernel program at the current
        // position (the body does not advance); bytes at this position
        const bool body = kind == K_STEP_BODY;
        CHK(step_prepare(s));
        if (!s->step_grid) { seterr("time_kind: the step kernel is not available"); return ORNITH_HIP_ERR_UNSUPPORTED; }
        Prog P;
        P.step = true;
        P.waves = s->step_grid * 4;
        CHK(body ? build_body(s, P) : build_head(s, P));
        double by = 0.0;
        for (double b : P.bytes) by += b;
        CHK(step_launch(s, body, nullptr, false));
        hipEvent_t a0 = nullptr, a1 = nullptr;
        HCHK(hipEventCreate(&a0));
        HCHK(hipEventCreate(&a1));
        HCHK(hipEventRecord(a0, st));
        for (int i = 0; i < reps; i++) CHK(step_launch(s, body, nullptr, false));
        HCHK(hipEventRecord(a1, st));
        HCHK(hipEventSynchronize(a1));
        float el = 0.0f;
        HCHK(hipEventElapsedTime(&el, a0, a1));
        (void)hipEventDestroy(a0);
        (void)hipEventDestroy(a1);
        CHK(step_check(s));
        *us_per_launch = el * 1000.0f / (float)reps;
        *bytes_per_launch = by;
        *launches_per_step = 1;
        return ORNITH_HIP_OK;
    }
    hipEvent_t e0 = nullptr, e1 = nullptr;
    HCHK(hipEventCreate(&e0));
    HCHK(hipEventCreate(&e1));
    s->only = kind;
    s->only_n = 0;
    s->only_bytes = 0.0;
    // the fused MoE launch's router counters are cleared step by step by the
    // launch itself, keyed on the step serial, which replays do not advance:
    // zero them before every pass (eager, not captured) so that its routed
    // blocks wait for the router blocks as in a decode step
    const size_t mb = (size_t)s->m->a.n_layers * 2 * sizeof(int32_t);
    hipError_t e = s->mctr ? hipMemsetAsync(s->mctr, 0, mb, st) : hipSuccess;
    int r = e == hipSuccess ? enqueue_body(s, st) : ORNITH_HIP_ERR_DEVICE;   // warm-up pass: counts launches and bytes
    if (r == ORNITH_HIP_OK) r = enqueue_head(s, st);
    const int n = s->only_n;
    const double by = s->only_bytes;
    if (e == hipSuccess) e = hipEventRecord(e0, st);
    for (int i = 0; i < reps && r == ORNITH_HIP_OK && e == hipSuccess; i++) {
        if (s->mctr) e = hipMemsetAsync(s->mctr, 0, mb, st);
        if (e == hipSuccess) r = enqueue_body(s, st);
        if (r == ORNITH_HIP_OK && e == hipSuccess) r = enqueue_head(s, st);
    }
    if (e == hipSuccess) e = hipEventRecord(e1, st);
    // and after the last pass, for the next decode step (its parity's counter
    // holds the replay's arrivals)
    if (e == hipSuccess && s->mctr) e = hipMemsetAsync(s->mctr, 0, mb, st);
    if (e == hipSuccess) e = hipEventSynchronize(e1);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    s->only = -1;
    float el = 0.0f;
    if (r == ORNITH_HIP_OK && e == hipSuccess) e = hipEventElapsedTime(&el, e0, e1);
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    if (r) return r;
    HCHK(e);
    if (n > 0) {
        *us_per_launch = el * 1000.0f / (float)(reps * n);
        *bytes_per_launch = by / n;
    }
    *launches_per_step = n;
    return ORNITH_HIP_OK;
}

extern "C" int ornith_hip_session_profile_step(ornith_hip_session *s, int max_launches, int32_t *kinds,
                                               double *bytes, float *ms, int *n_launches) {
    *n_launches = 0;
    if (!s->have_logits) { seterr("session has no logits; eval a prompt first"); return ORNITH_HIP_ERR_FORMAT; }
    if (s->pos + 1 > s->cap) { seterr("profile_step: session full"); return ORNITH_HIP_ERR_UNSUPPORTED; }
    HCHK(hipSetDevice(s->m->ctx->device));
    hipStream_t st = s->m->ctx->st;
    CHK(sync_pos(s));
    HCHK(hipStreamSynchronize(st));
    s->rec = true;
    s->rec_ev.clear(); s->rec_kind.clear(); s->rec_bytes.clear();
    int r = enqueue_body(s, st);
    if (r == ORNITH_HIP_OK) r = enqueue_head(s, st);
    s->rec = false;
    hipError_t e = hipStreamSynchronize(st);
    const size_t n = s->rec_kind.size();
    if (r == ORNITH_HIP_OK && e == hipSuccess) {
        for (size_t i = 0; i < n && (int)i < max_launches; i++) {
            float el = 0.0f;
            (void)hipEventElapsedTime(&el, s->rec_ev[2 * i], s->rec_ev[2 * i + 1]);
            kinds[i] = s->rec_kind[i];
            bytes[i] = s->rec_bytes[i];
            ms[i] = el;
        }
        *n_launches = (int)(n < (size_t)max_launches ? n : (size_t)max_launches);
        s->pos += 1;
    }
    for (hipEvent_t ev : s->rec_ev) (void)hipEventDestroy(ev);
    s->rec_ev.clear();
    if (r) return r;
    HCHK(e);
    return ORNITH_HIP_OK;
}

// ---- phases of one step-kernel body launch (block 0's clock after each barrier) --------------------
extern "C" int ornith_hip_session_profile_phases(ornith_hip_session *s, int max_phases, int32_t *kinds,
                                                 double *bytes, float *us, int *n_phases) {
    *n_phases = 0;
    if (!s->have_logits) { seterr("session has no logits; eval a prompt first"); return ORNITH_HIP_ERR_FORMAT; }
    HCHK(hipSetDevice(s->m->ctx->device));
    hipStream_t st = s->m->ctx->st;
    CHK(sync_pos(s));
    CHK(step_prepare(s));
    if (!s->step_grid) { seterr("profile_phases: the step kernel is not available"); return ORNITH_HIP_ERR_UNSUPPORTED; }
    if (!s->ts) CHK(salloc(s, &s->ts, (size_t)s->sp_body.n + 8));
    Prog P;
    P.step = true;
    P.waves = s->step_grid * 4;
    CHK(build_body(s, P));
    CHK(step_launch(s, true, nullptr, false));        // warm
    CHK(step_launch(s, true, s->ts, false));
    HCHK(hipStreamSynchronize(st));
    CHK(step_check(s));
    const int n = s->sp_body.n;
    std::vector<uint64_t> t((size_t)n + 1);
    HCHK(hipMemcpy(t.data(), s->ts, t.size() * 8, hipMemcpyDeviceToHost));
    const int m = n < max_phases ? n : max_phases;
    for (int i = 0; i < m; i++) {
        kinds[i] = i < (int)P.rk.size() ? P.rk[i] : -1;
        bytes[i] = i < (int)P.bytes.size() ? P.bytes[i] : 0.0;
        us[i] = (float)((double)(t[i + 1] - t[i]) / 100.0);   // 100 MHz real-time clock
    }
    *n_phases = m;
    return ORNITH_HIP_OK;
}

// One decode launch with clocks (after a warm-up launch; neither advances the
// position): per operation its kind and, over the workgroups, the earliest and
// the latest time it was done (microseconds from the earliest start).
extern "C" int ornith_hip_session_profile_decode(ornith_hip_session *s, int max_ops, int32_t *kinds,
                                                 float *us_first, float *us_last, int *n_ops) {
    *n_ops = 0;
    if (!s->have_logits) { seterr("session has no logits; eval a prompt first"); return ORNITH_HIP_ERR_FORMAT; }
    HCHK(hipSetDevice(s->m->ctx->device));
    hipStream_t st = s->m->ctx->st;
    CHK(sync_pos(s));
    CHK(dec_prepare(s));
    if (!s->dec.grid) { seterr("profile_decode: the decode launch is not available for this model"); return ORNITH_HIP_ERR_UNSUPPORTED; }
    const int G = s->dec.grid, n = s->dec.n;
    if (!s->dec.ts) CHK(salloc(s, &s->dec.ts, (size_t)(n + 1) * G));
    HCHK(oh_launch_decode(s->dec.ops, n, s->io, 0, G, s->dec.lds, st));
    HCHK(oh_launch_decode(s->dec.ops, n, s->io, 0, G, s->dec.lds, st, s->dec.ts));
    HCHK(hipStreamSynchronize(st));
    CHK(step_check(s));
    std::vector<uint64_t> t((size_t)(n + 1) * G);
    HCHK(hipMemcpy(t.data(), s->dec.ts, t.size() * 8, hipMemcpyDeviceToHost));
    uint64_t t0 = t[0];
    for (int b = 1; b < G; b++) t0 = t[b] < t0 ? t[b] : t0;
    const int m = n < max_ops ? n : max_ops;
    for (int i = 0; i < m; i++) {
        uint64_t lo = ~0ull, hi = 0;
        for (int b = 0; b < G; b++) {
            const uint64_t v = t[(size_t)(i + 1) * G + b];
            lo = v < lo ? v : lo;
            hi = v > hi ? v : hi;
        }
        kinds[i] = s->dec.kinds[i];
        us_first[i] = (float)((double)(lo - t0) / 100.0);
        us_last[i] = (float)((double)(hi - t0) / 100.0);
    }
    *n_ops = m;
    return ORNITH_HIP_OK;
}

// Sub-phase clocks of one operation of the decode launch (measurement): per
// workgroup 8 stamps (0 start, 1 weights requested, 2 inputs arrived, 3 the
// activation arrived, 4 prologue done, 5 done; unused ones 0) in microseconds
// from the launch's earliest start, -1 where not recorded. grid_out: workgroups.
extern "C" int ornith_hip_session_profile_decode_op(ornith_hip_session *s, int op, float *us, int max_groups,
                                                    int *grid_out) {
    *grid_out = 0;
    if (!s->have_logits) { seterr("session has no logits; eval a prompt first"); return ORNITH_HIP_ERR_FORMAT; }
    HCHK(hipSetDevice(s->m->ctx->device));
    hipStream_t st = s->m->ctx->st;
    CHK(sync_pos(s));
    CHK(dec_prepare(s));
    if (!s->dec.grid) { seterr("profile_decode_op: the decode launch is not available for this model"); return ORNITH_HIP_ERR_UNSUPPORTED; }
    const int G = s->dec.grid, n = s->dec.n;
    if (op < 0 || op >= n) { seterr("profile_decode_op: operation %d outside [0, %d)", op, n); return ORNITH_HIP_ERR_FORMAT; }
    if (!s->dec.ts) CHK(salloc(s, &s->dec.ts, (size_t)(n + 1) * G));
    uint64_t *ts2 = nullptr;
    CHK(salloc(s, &ts2, (size_t)G * 8));
    HCHK(oh_launch_decode(s->dec.ops, n, s->io, 0, G, s->dec.lds, st));
    HCHK(oh_launch_decode(s->dec.ops, n, s->io, 0, G, s->dec.lds, st, s->dec.ts, op, ts2));
    HCHK(hipStreamSynchronize(st));
    CHK(step_check(s));
    std::vector<uint64_t> t((size_t)G), t2((size_t)G * 8);
    HCHK(hipMemcpy(t.data(), s->dec.ts, (size_t)G * 8, hipMemcpyDeviceToHost));
    HCHK(hipMemcpy(t2.data(), ts2, t2.size() * 8, hipMemcpyDeviceToHost));
    uint64_t t0 = t[0];
    for (int b = 1; b < G; b++) t0 = t[b] < t0 ? t[b] : t0;
    const int m = G < max_groups ? G : max_groups;
    for (int b = 0; b < m; b++)
        for (int k = 0; k < 8; k++) {
            const uint64_t v = t2[(size_t)b * 8 + k];
            us[b * 8 + k] = v == 0 ? -1.0f : (float)((double)(v - t0) / 100.0);
        }
    *grid_out = m;
    return ORNITH_HIP_OK;
}
