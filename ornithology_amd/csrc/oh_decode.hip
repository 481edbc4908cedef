// oh_decode.hip - the decode step (rforward_token, src/ornith_rforward.c:686-706)
// as ONE persistent launch: every workgroup walks the same program of
// operations (embedding, per layer: input projections, delta-net step or GQA,
// output projection, router, experts, down projection; then lm_head and the
// greedy token) and hands activations to the next operation as tagged words.
//
// Hand-off. A tagged word is 64 bits: the value's 32 bits and the step's tag
// (a per-session launch counter). An operation writes its outputs into its
// own region of the session's word arena with device-scope stores and goes
// on; a reader loads the words it needs (all requests issued at once) and
// re-polls only those whose tag is not yet the current step's. The load that
// delivers the value is the wait: no counter and no second round trip. A word
// is written by one lane in one 64-bit store, so a reader sees either the old
// word or the new one, never a mix.
//
// Roles inside a workgroup. Vector memory operations complete in order
// within a wave, and a workgroup barrier that orders global memory waits for
// all of them. So wave 0 (the front wave) never holds weight loads or output
// stores: it polls the operation's inputs into LDS. Waves 1-3 (the back waves)
// request their weights as soon as the operation starts and write the
// outputs. All four waves form the activation (RMSNorm, Q8_K) and the MoE
// routing from LDS in parallel; the barriers between these stages order LDS
// only, so the weight stream keeps flowing underneath them.
//
// Bulk outputs that are not per-element words (the GQA prep's queries and KV
// append, the attention partials and output) use the device-scope stores of
// the operation bodies shared with the per-launch path; the writer then waits
// for their completion and stores one tagged flag word, which readers poll.
//
// Arithmetic is the same as the per-launch kernels' (the same helpers, the
// same orders), so results are bit-identical to them.
//
// Every wait is bounded: after about 200 ms, or once another workgroup has
// given up (io[OH_IO_ERR] != 0), a workgroup records the failure and leaves
// at the end of the operation; every other workgroup then gives up at its
// next wait, so the grid drains.

namespace {

constexpr uint64_t kDecTicks = 20000000;   // 200 ms of the 100 MHz real-time clock
constexpr int kDecPF = 2;                  // matvec steps per wave whose weights are in registers

// The decode launch keeps expf's 32-entry table in LDS (filled at the start):
// a lookup is then an LDS read instead of a global load in the middle of a
// dependent chain. Same values, same results as ref_expf.
__shared__ uint64_t g_dexp[32];
OH_DEV float dexpf(float x) { return ref_expf_tab(x, g_dexp); }
OH_DEV float dsigmoid(float x) { return 1.0f / (1.0f + dexpf(-x)); }
OH_DEV float dsilu(float x) { return x * dsigmoid(x); }
OH_DEV float dsoftplus(float x) { return x > 20.0f ? x : ref_log1pf(dexpf(x)); }

struct Dctl {
    uint32_t tag;
    int32_t *err;
    int pos;
    int *dead;              // LDS [2]: a wait of the workgroup gave up during an operation of that parity
    int par;                // the current operation's parity
    uint64_t *st;           // profiling: this workgroup's sub-phase clocks of one operation (or null)
    OH_DEV void fail() const { dead[par] = 1; }
    OH_DEV void stamp(int k) const {
        if (st && tid_x() == 0) st[k] = __builtin_amdgcn_s_memrealtime();
    }
};

OH_DEV uint64_t llw(float v, uint32_t tag) { return ((uint64_t)tag << 32) | (uint64_t)f2u(v); }
OH_DEV uint64_t llw_i(int v, uint32_t tag) { return ((uint64_t)tag << 32) | (uint64_t)(uint32_t)v; }
OH_DEV bool ll_ok(uint64_t w, uint32_t tag) { return (uint32_t)(w >> 32) == tag; }
OH_DEV float ll_f(uint64_t w) { return u2f((uint32_t)w); }
OH_DEV uint64_t dec_now() { return __builtin_amdgcn_s_memrealtime(); }
OH_DEV uint64_t ll_ready(const Dctl &c) { return (uint64_t)c.tag << 32; }

// Re-poll the words of v that do not carry the tag yet (addr(k): address of
// word k) until all do. False: the wait gave up (and io[OH_IO_ERR] is set).
template <int N, class F>
OH_DEV bool ll_settle(uint64_t (&v)[N], F addr, const Dctl &c) {
    uint64_t t0 = 0;
    for (int it = 0;; it++) {
        bool stale = false;
#pragma unroll
        for (int k = 0; k < N; k++) stale |= !ll_ok(v[k], c.tag);
        if (!stale) return true;
        if (it == 0) {
            t0 = dec_now();
        } else if ((it & 7) == 0 && (ldc(c.err) != 0 || dec_now() - t0 > kDecTicks)) {
            stc(c.err, (int32_t)1);
            c.fail();
            return false;
        }
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int k = 0; k < N; k++)
            if (!ll_ok(v[k], c.tag)) v[k] = ldc(addr(k));
    }
}

// One wave: words [0, n) of src into the float array dst (LDS), lane l
// taking words l + 64 k, PB per lane per pass, every load of a pass issued at
// once.
template <int PB>
OH_DEV void ll_fetch_wave(float *dst, const uint64_t *src, int n, const Dctl &c) {
    const int l = lane_id();
    for (int i0 = 0; i0 < n; i0 += 64 * PB) {
        uint64_t v[PB];
#pragma unroll
        for (int k = 0; k < PB; k++) {
            const int i = i0 + l + 64 * k;
            v[k] = i < n ? ldc(src + i) : ll_ready(c);
        }
        if (!ll_settle<PB>(v, [&](int k) { return src + i0 + l + 64 * k; }, c)) return;
#pragma unroll
        for (int k = 0; k < PB; k++) {
            const int i = i0 + l + 64 * k;
            if (i < n) dst[i] = ll_f(v[k]);
        }
    }
}

// One wave: wait until the n flag words of f carry the tag
OH_DEV void flags_wait_wave(const uint64_t *f, int n, const Dctl &c) {
    const int l = lane_id();
    for (int i0 = 0; i0 < n; i0 += 64 * 4) {
        uint64_t v[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int i = i0 + l + 64 * k;
            v[k] = i < n ? ldc(f + i) : ll_ready(c);
        }
        if (!ll_settle<4>(v, [&](int k) { return f + i0 + l + 64 * k; }, c)) return;
    }
}
// the whole workgroup waits for the flags (no weights in flight: the GQA
// operations); ends with a full barrier
OH_DEV void flags_wait(const uint64_t *f, int n, const Dctl &c) {
    if (tid_x() < 64) flags_wait_wave(f, n, c);
    __syncthreads();
}

// this workgroup's device-scope stores are complete: publish its flag
OH_DEV void flag_set(uint64_t *f, const Dctl &c) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid_x() == 0) stc(f, llw_i(0, c.tag));
}

// ---- embedding (src/ornith_rforward.c:199-208) ---------------------------------
OH_DEV void dop_embed(const oh_demb &a, int vb, const Dctl &c) {
    const int32_t tok = ldg(a.toks + c.pos);
    const int i = vb * 256 + tid_x();
    if (i < a.in) stc(a.x + i, llw(dec_elem(a.A, a.B, a.C, a.type, a.in, tok, i), c.tag));
}

// ---- MoE routing (src/ornith_moe.c:8-30) -----------------------------------------
// route_wave's selection (repeated strict-'>' scans, ties to the lower index;
// softmax in selection order) with the LDS expf table: the rare path.
OH_DEV void dec_route_wave(const float *logits, int ne, int k, int32_t *idx, float *w) {
    const int lane = lane_id();
    float v[16];
#pragma unroll
    for (int j = 0; j < 16; j++) v[j] = lane + 64 * j < ne ? logits[lane + 64 * j] : -INFINITY;
    uint32_t taken = 0;
    float mine = 0.0f;
    int sel = 0;
    for (int s = 0; s < k; s++) {
        float bv = -INFINITY; int bi = 0x7fffffff;
#pragma unroll
        for (int j = 0; j < 16; j++) {
            const int e = lane + 64 * j;
            if (e < ne && !(taken >> j & 1u) && v[j] > bv) { bv = v[j]; bi = e; }
        }
        for (int m = 32; m >= 1; m >>= 1) {
            const float ov = shfl_xor(bv, m); const int oi = shfl_xor(bi, m);
            if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
        }
        if ((bi & 63) == lane) taken |= 1u << (bi >> 6);
        if (lane == s) { mine = bv; sel = bi; }
    }
    if (sel < 0 || sel >= ne) sel = 0;
    if (lane < k) idx[lane] = sel;
    float mx = shfl(mine, 0);
    for (int s = 1; s < k; s++) { const float x = shfl(mine, s); if (x > mx) mx = x; }
    const float e = dexpf(mine - mx);
    float sum = 0.0f;
    for (int s = 0; s < k; s++) sum += shfl(e, s);
    if (lane < k) w[lane] = e / sum;
}

// LDS state of a routing (the front wave fills lg and resets bad/cnt)
struct DRoute {
    float *lg;              // ne logits, padded with -inf to a multiple of 4
    int *sel, *bad, *cnt;
    float *rw, *shg, *sl;
};
// The routing of route_block, by the whole workgroup from the logits in LDS:
// expert e's rank is the number of experts ahead of it in the reference's
// order (larger logit, or equal logit and lower index); equal logits in the
// top k, NaN or -inf take the sequential selection. Ends with an LDS barrier.
OH_DEV void dec_route(const DRoute &R, int ne, int k, bool has_sh) {
    const int tid = tid_x(), ne4 = (ne + 3) & ~3;
    const float4 *l4 = (const float4 *)R.lg;
    for (int e = tid; e < ne; e += 256) {
        const float v = R.lg[e];
        if (!(v > -INFINITY)) *R.bad = 1;
        int gt = 0;
#pragma unroll 8
        for (int j = 0; j < ne4 / 4; j++) {
            const float4 u = l4[j];
            gt += (int)(u.x > v) + (int)(u.y > v) + (int)(u.z > v) + (int)(u.w > v);
        }
        if (gt < k) {
            if (atomicAdd(&R.cnt[gt], 1) != 0) *R.bad = 1;
            R.sel[gt] = e;
        }
    }
    lds_barrier();
    if (*R.bad) {
        if (tid < 64) dec_route_wave(R.lg, ne, k, R.sel, R.rw);
    } else if (tid < 64) {
        const float lj = tid < k ? R.lg[R.sel[tid]] : -INFINITY;
        const float mx = wave_max_fast(lj);
        const float e = tid < k ? dexpf(lj - mx) : 0.0f;
        float sum = 0.0f;
        for (int j = 0; j < k; j++) sum += shfl(e, j);
        if (tid < k) R.rw[tid] = e / sum;
    }
    if (tid == 0) *R.shg = has_sh ? dsigmoid(*R.sl) : 1.0f;
    lds_barrier();
}
// the front wave: the tagged logits (and shared-gate logit) into LDS, the
// rank counters cleared
OH_DEV void route_fetch(const DRoute &R, const uint64_t *rlog, const uint64_t *shl, int ne, const Dctl &c) {
    const int l = lane_id(), ne4 = (ne + 3) & ~3;
    ll_fetch_wave<4>(R.lg, rlog, ne, c);
    for (int e = ne + l; e < ne4; e += 64) R.lg[e] = -INFINITY;
    if (shl) {
        uint64_t w1[1] = {ldc(shl)};
        ll_settle<1>(w1, [&](int) { return shl; }, c);
        if (l == 0) *R.sl = ll_f(w1[0]);
    }
    if (l == 0) *R.bad = 0;
    R.cnt[l] = 0;
}

// ---- the activation of a matvec: Q8_K of the input (after RMSNorm) ----------------
// in = 256 NB floats in LDS v (published); all four waves. Thread t's sum of
// squares over elements t + 256 k, the tree of the per-launch prologue, x *
// inv * w; then wave w quantises blocks w, w + 4, ... interleaved
// (qdot_quantize_row_q8_K per block). nw: the RMSNorm weights of elements
// t + 256 k (registers), or null (no norm).
template <int NB>
OH_DEV void dec_act(float *v, const float *nw, float eps, uint8_t *smem, double *red) {
    const int tid = tid_x(), wave = tid >> 6;
    if (nw) {
        float x[NB];
#pragma unroll
        for (int k = 0; k < NB; k++) x[k] = v[tid + 256 * k];
        double ss = 0.0;
#pragma unroll
        for (int k = 0; k < NB; k++) ss += (double)x[k] * x[k];
        ss = wave_sum_d(ss);
        if (lane_id() == 0) red[wave] = ss;
        lds_barrier();
        const double tot = (red[0] + red[1]) + (red[2] + red[3]);
        const float inv = (float)(1.0 / sqrt(tot / (double)(256 * NB) + (double)eps));
#pragma unroll
        for (int k = 0; k < NB; k++) v[tid + 256 * k] = x[k] * inv * nw[k];
        lds_barrier();
    }
    constexpr int QN = (NB + 3) / 4;
    q8k_blocks<QN>(v, wave, 4, NB, (int8_t *)smem, (float *)(smem + mv_lds_d_off(NB)),
                   (int16_t *)(smem + mv_lds_bs_off(NB)), kAS);
    lds_barrier();
}

// ---- multi-segment matvec ---------------------------------------------------------
// The steps of all segments (a step: 64/nb rows of one slot, one super-block
// per lane; a paired step reduces W and W2 for the same rows) are dealt to
// the back waves of the grid (three per workgroup) in contiguous runs of
// M.spw. A back wave's first kDecPF steps are requested when the operation
// starts (stacked-expert steps once the routing is known); longer runs
// stream with two steps in flight. The dot of a row is the per-launch
// matvec's (sb_term per super-block, the terms summed in order). Outputs:
// tagged words (mode 1: the residual word plus the dot), an optional plain
// copy, and (head) the workgroup's best (value, index) for the greedy token.
struct DStep { int seg, slot, unit; };
// the step -> (segment, slot, unit) map from segment tables in registers
struct DSegTab {
    int n, step0[OH_D_MAXSEG], units[OH_D_MAXSEG];
    OH_DEV DStep at(int gs) const {
        int si = 0;
#pragma unroll
        for (int k = 1; k < OH_D_MAXSEG; k++)
            if (k < n && gs >= step0[k]) si = k;
        int s0 = step0[0], u = units[0];
#pragma unroll
        for (int k = 1; k < OH_D_MAXSEG; k++)
            if (k == si) { s0 = step0[k]; u = units[k]; }
        const int loc = gs - s0;
        return DStep{si, loc / u, loc - (loc / u) * u};
    }
};

template <int T>
struct DBuf { SB<T> a, b; };

template <int T, int NB>
OH_DEV void dec_load(DBuf<T> &r, const oh_dmv &M, const DSegTab &tab, int gs, int rl, int sb, const int *sel) {
    const DStep d = tab.at(gs);
    const oh_dseg &s = M.s[d.seg];
    constexpr int RPS = 64 / NB;
    const int row = d.unit * RPS + (rl < RPS ? rl : RPS - 1);
    const int rowc = row < s.rows ? row : s.rows - 1;
    const int64_t rb = s.stacked ? (int64_t)sel[d.slot] * s.rows : 0;
    sb_load(r.a, WP{s.A, s.B, s.C}, (rb + rowc) * NB + sb);
    if (s.pair) sb_load(r.b, WP{s.A2, s.B2, s.C2}, (rb + rowc) * NB + sb);
}

// LDS: [Q8_K planes of NB blocks][v: the input, 256 NB floats][residual rows:
// 1024 floats][router logits]
template <int T, int NB>
OH_DEV void dop_mv(const oh_dmv &M, int vb, uint8_t *smem, const Dctl &c) {
    __shared__ double red[4];
    __shared__ int rsel[64], rbad, rcnt[64];
    __shared__ float rwt[64], rshg, rsl;
    __shared__ float bestv[4];
    __shared__ int besti[4];
    constexpr int IN = 256 * NB, RPS = 64 / NB;
    const int tid = tid_x(), lane = lane_id(), wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nsteps = M.nsteps, spw = M.spw;
    const int rl = lane / NB, sb = lane - rl * NB;
    // back wave b (1..3) of workgroup vb is stepping wave vb * 3 + b - 1 - wave0
    const int g0 = vb * 3 - M.wave0;
    if (g0 + 2 < 0 || (g0 > 0 ? g0 : 0) * spw >= nsteps) {
        if (M.amax && tid == 0) {
            stc(M.amax + 2 * vb, llw(-INFINITY, c.tag));
            stc(M.amax + 2 * vb + 1, llw_i(0x7fffffff, c.tag));
        }
        return;
    }
    DSegTab tab;
    tab.n = M.nseg;
#pragma unroll
    for (int k = 0; k < OH_D_MAXSEG; k++) { tab.step0[k] = M.s[k].step0; tab.units[k] = M.s[k].units; }
    float *v = (float *)(smem + mv_lds_v_off(NB));
    float *xres = v + IN;
    DRoute R{xres + 1024, rsel, &rbad, rcnt, rwt, &rshg, &rsl};
    const bool route = M.route != 0, norm = M.pro == OH_PRO_NORM;
    const int bs0 = (g0 > 0 ? g0 : 0) * spw, bs1 = (g0 + 3) * spw < nsteps ? (g0 + 3) * spw : nsteps;
    // the RMSNorm weights of this thread's elements: the first requests of every wave
    float nw[NB];
    if (norm) {
#pragma unroll
        for (int k = 0; k < NB; k++) nw[k] = ldg(M.nw + tid + 256 * k);
    }
    c.stamp(0);
    const int gw = g0 + wave - 1;
    const int s0 = gw * spw;
    const int S = wave > 0 && gw >= 0 && s0 < nsteps ? (nsteps - s0 < spw ? nsteps - s0 : spw) : 0;
    DBuf<T> b0, b1;
    bool pre0 = false, pre1 = false;
    if (wave == 0) {
        // front: routing logits, the input, the residual rows
        if (route) route_fetch(R, M.rlog, M.shl, M.ne, c);
        if (M.x) {
            ll_fetch_wave<32>(v, M.x, IN, c);
        } else {
            flags_wait_wave(M.xflags, c.pos + 1 <= M.exact_lim ? M.nflags_ex : M.nflags_fl, c);
            for (int i0 = 0; i0 < IN; i0 += 64 * 16) {
                float r[16];
#pragma unroll
                for (int u = 0; u < 16; u++) r[u] = i0 + lane + 64 * u < IN ? ldc(M.xp + i0 + lane + 64 * u) : 0.0f;
#pragma unroll
                for (int u = 0; u < 16; u++)
                    if (i0 + lane + 64 * u < IN) v[i0 + lane + 64 * u] = r[u];
            }
        }
        if (M.s[0].mode == 1) {
            const int rows = M.s[0].rows;
            const int r0 = bs0 * RPS, r1 = bs1 * RPS < rows ? bs1 * RPS : rows;
            if (r1 > r0) ll_fetch_wave<4>(xres, M.xres + r0, r1 - r0, c);
        }
        c.stamp(1);
    } else {
        // back: the weights that do not depend on the routing
        auto stacked = [&](int st) { return M.s[tab.at(s0 + st).seg].stacked != 0; };
        pre0 = S > 0 && !stacked(0);
        pre1 = S > 1 && !stacked(1);
        if (pre0) dec_load<T, NB>(b0, M, tab, s0, rl, sb, rsel);
        if (pre1) dec_load<T, NB>(b1, M, tab, s0 + 1, rl, sb, rsel);
    }
    lds_barrier();                            // the front wave's inputs are in LDS
    c.stamp(2);
    if (route) {
        dec_route(R, M.ne, M.topk, M.shl != nullptr);
        if (S > 0 && !pre0) dec_load<T, NB>(b0, M, tab, s0, rl, sb, rsel);
        if (S > 1 && !pre1) dec_load<T, NB>(b1, M, tab, s0 + 1, rl, sb, rsel);
    }
    dec_act<NB>(v, norm ? nw : nullptr, M.eps, smem, red);
    c.stamp(4);
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    if (S > 0) {
        const int8_t *aq = (const int8_t *)smem + sb * kAS;
        const int16_t *abs = (const int16_t *)(smem + mv_lds_bs_off(NB)) + sb * 16;
        const float yd = ((const float *)(smem + mv_lds_d_off(NB)))[sb];
        auto comp = [&](const DBuf<T> &r, int st) {
            const DStep d = tab.at(s0 + st);
            const oh_dseg &s = M.s[d.seg];
            const int row = d.unit * RPS + rl;
            const bool live = rl < RPS && row < s.rows;
            const float t1 = live ? sb_term(r.a, aq, abs, yd) : 0.0f;
            float acc = 0.0f;
#pragma unroll
            for (int i = 0; i < NB; i++) acc += shfl(t1, rl * NB + i);
            float out = acc;
            if (s.pair) {
                const float t2 = live ? sb_term(r.b, aq, abs, yd) : 0.0f;
                float acc2 = 0.0f;
#pragma unroll
                for (int i = 0; i < NB; i++) acc2 += shfl(t2, rl * NB + i);
                out = dsilu(acc) * acc2;
            }
            if (live && sb == 0) {
                const float val = s.mode == 1 ? xres[row - bs0 * RPS] + out : out;
                const size_t o = (size_t)d.slot * s.ystride + row;
                if (s.y) stc(s.y + o, llw(val, c.tag));
                if (s.yp) stg(s.yp + o, val);
                if (val > bv || (val == bv && row < bi)) { bv = val; bi = row; }
            }
        };
        int st = 0;
        for (; st + 1 < S; st += 2) {
            comp(b0, st);
            if (st + 2 < S) dec_load<T, NB>(b0, M, tab, s0 + st + 2, rl, sb, rsel);
            comp(b1, st + 1);
            if (st + 3 < S) dec_load<T, NB>(b1, M, tab, s0 + st + 3, rl, sb, rsel);
        }
        if (st < S) comp(b0, st);
    }
    c.stamp(5);
    if (M.amax) {
        for (int m = 32; m >= 1; m >>= 1) {
            const float ov = shfl_xor(bv, m);
            const int oi = shfl_xor(bi, m);
            if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
        }
        if (lane == 0) { bestv[wave] = bv; besti[wave] = bi; }
        lds_barrier();
        if (tid == 0) {
            bv = bestv[0]; bi = besti[0];
            for (int k = 1; k < 4; k++)
                if (bestv[k] > bv || (bestv[k] == bv && besti[k] < bi)) { bv = bestv[k]; bi = besti[k]; }
            stc(M.amax + 2 * vb, llw(bv, c.tag));
            stc(M.amax + 2 * vb + 1, llw_i(bi, c.tag));
        }
    }
}

// ---- gated delta-net step (src/ornith_rforward.c:457-503,300-319,
//      src/ornith_attn.c:198-213,370-388), one workgroup per value head -----------
// The row waves (wave w < DK/64) own state rows [64 w, +64) of value head hv
// = vb: they request their slab when the operation starts and move it into a
// row-padded LDS tile while the front waves (the others) poll this step's
// inputs and form the conv + SiLU of the head's q, k and v channels, the L2
// norms of q and k (double sums of each 64-channel run, the runs added in
// order), the decay and beta, and silu(gate) per row. Then each row lane walks
// its row in the reference's column order (decay, S.k, rank-1 update, S.q).
// The per-head gated RMSNorm follows in the workgroup: the double sums of o^2
// of the 64-row runs added in order, o * inv * w * silu(gate). The conv window
// is double-buffered by position parity, each channel written by one owner.
template <int DK, int KMAX>
OH_DEV void dop_delta(const oh_ddelta &a, int vb, float *lds, const Dctl &c) {
    constexpr int NQ = DK / 64, TS = DK + 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid_x() >> 6), lane = lane_id();
    const bool row = wave < NQ;
    float *qn = lds, *kn = qn + DK, *vv = kn + DK, *zs = vv + DK, *ab = zs + DK;   // front -> rows
    float *tile = ab + 4 + (row ? wave : 0) * 64 * TS;
    double *runs = (double *)(lds + 4 * DK + 4 + NQ * 64 * TS);
    const int nk = a.nk, nv = a.nv, K = a.K, cc = a.cc;
    const int hv = vb, kh = hv % nk, qd = nk * DK;
    const int p = c.pos & 1;
    const float *win = a.conv_state + (size_t)p * (K - 1) * cc;
    float *nwin = a.conv_state + (size_t)(1 - p) * (K - 1) * cc;
    c.stamp(0);
    float4 st[DK / 4];
    float nw = 0.0f;
    if (row) {
        const float4 *Sr = (const float4 *)(a.S + ((size_t)hv * DK + wave * 64) * DK);
#pragma unroll
        for (int i = 0; i < DK / 4; i++) st[i] = ldg(Sr + lane + 64 * i);
        nw = ldg(a.norm_w + wave * 64 + lane);
    } else {
        // front wave f = wave - NQ of NF: channels of its share; q runs and k
        // runs each go to one wave so its L2 norm is that wave's butterfly sums
        const int NF = 4 - NQ, f = wave - NQ;
        // q channel runs i (i < NQ) on front wave i % NF, k runs on (NQ + i) % NF,
        // v runs and gate runs on (2 NQ + i) % NF
        for (int job = f; job < 3 * NQ; job += NF) {
            const int kind = job / NQ, i = job % NQ;       // 0 q, 1 k, 2 v (+ gate)
            const int chl = 64 * i + lane;
            const int ch = kind == 0 ? kh * DK + chl : kind == 1 ? qd + kh * DK + chl : 2 * qd + hv * DK + chl;
            float cw[KMAX], wv[KMAX];
            if (KMAX == 4 && K == 4) {
                const float4 c4 = ldg((const float4 *)(a.conv_w + (size_t)ch * 4));
                cw[0] = c4.x; cw[1] = c4.y; cw[2] = c4.z; cw[3] = c4.w;
            } else {
#pragma unroll
                for (int j = 0; j < KMAX; j++) cw[j] = j < K ? ldg(a.conv_w + (size_t)ch * K + j) : 0.0f;
            }
#pragma unroll
            for (int j = 0; j < KMAX; j++) wv[j] = j < K - 1 ? ldg(win + (size_t)j * cc + ch) : 0.0f;
            uint64_t w[2] = {ldc(a.cat + ch), kind == 2 ? ldc(a.z + (size_t)hv * DK + chl) : ll_ready(c)};
            ll_settle<2>(w, [&](int k) { return k == 0 ? a.cat + ch : a.z + (size_t)hv * DK + chl; }, c);
            const float cx = ll_f(w[0]);
            float acc = 0.0f, wl = 0.0f;
#pragma unroll
            for (int j = 0; j < KMAX; j++) {
                if (j < K - 1) acc += cw[j] * wv[j];
                if (j == K - 1) wl = cw[j];
            }
            acc += wl * cx;
            const float cv = dsilu(acc);
            // the conv window: v channels always ours, q / k channels by the
            // key head's first value head
            if (kind == 2 || hv < nk) {
#pragma unroll
                for (int j = 0; j + 1 < KMAX; j++)
                    if (j + 1 < K - 1) stg(nwin + (size_t)j * cc + ch, wv[j + 1]);
                stg(nwin + (size_t)(K - 2) * cc + ch, cx);
            }
            if (kind == 2) {
                vv[chl] = cv;
                zs[chl] = dsilu(ll_f(w[1]));
            } else {
                // this run's butterfly double sum of squares, added to the runs before it
                const double sq = wave_sum_d((double)cv * cv);
                (kind == 0 ? qn : kn)[chl] = cv;
                if (lane == 0) ((double *)(ab + 4 + NQ * 64 * TS) + 4)[kind * NQ + i] = sq;
            }
        }
        if (f == 0) {
            uint64_t w[2] = {ldc(a.ab + hv), ldc(a.ab + nv + hv)};
            ll_settle<2>(w, [&](int k) { return a.ab + (k == 0 ? hv : nv + hv); }, c);
            if (lane == 0) {
                ab[0] = dexpf(ldg(a.ssm_a + hv) * dsoftplus(ll_f(w[0]) + ldg(a.dt_bias + hv)));
                ab[1] = dsigmoid(ll_f(w[1]));
            }
        }
    }
    if (row) {
        // the slab into the row-padded tile while the front waves work
#pragma unroll
        for (int i = 0; i < DK / 4; i++) {
            const int f = lane + 64 * i, r = (4 * f) / DK, col = (4 * f) % DK;
            *(float4 *)(tile + r * TS + col) = make_float4(st[i].x, st[i].y, st[i].z, st[i].w);
        }
    }
    lds_barrier();                            // the front waves' values are in LDS
    c.stamp(2);
    float o = 0.0f;
    if (row) {
        // the L2 norms from the runs' sums (in order), then the row walk
        const double *rs = (const double *)(ab + 4 + NQ * 64 * TS) + 4;
        double tq = rs[0], tk = rs[NQ];
        for (int i = 1; i < NQ; i++) { tq += rs[i]; tk += rs[NQ + i]; }
        const float iq = (float)(1.0 / sqrt(tq + (double)1e-6f));
        const float ik = (float)(1.0 / sqrt(tk + (double)1e-6f));
        const float alpha = ab[0], beta = ab[1];
        float *tr = tile + lane * TS;
        float sr[DK];
#pragma unroll
        for (int cI = 0; cI < DK / 4; cI++) {
            const float4 v = *(const float4 *)(tr + 4 * cI);
            sr[4 * cI + 0] = v.x * alpha;
            sr[4 * cI + 1] = v.y * alpha;
            sr[4 * cI + 2] = v.z * alpha;
            sr[4 * cI + 3] = v.w * alpha;
        }
        float sk = 0.0f;
#pragma unroll
        for (int cI = 0; cI < DK / 4; cI++) {
            const float4 kk = *(const float4 *)(kn + 4 * cI);
            sk += sr[4 * cI + 0] * (kk.x * ik);
            sk += sr[4 * cI + 1] * (kk.y * ik);
            sk += sr[4 * cI + 2] * (kk.z * ik);
            sk += sr[4 * cI + 3] * (kk.w * ik);
        }
        const float u = beta * (vv[wave * 64 + lane] - sk);
#pragma unroll
        for (int cI = 0; cI < DK / 4; cI++) {
            const float4 kk = *(const float4 *)(kn + 4 * cI), qq = *(const float4 *)(qn + 4 * cI);
            sr[4 * cI + 0] += u * (kk.x * ik);
            sr[4 * cI + 1] += u * (kk.y * ik);
            sr[4 * cI + 2] += u * (kk.z * ik);
            sr[4 * cI + 3] += u * (kk.w * ik);
            o += sr[4 * cI + 0] * (qq.x * iq);
            o += sr[4 * cI + 1] * (qq.y * iq);
            o += sr[4 * cI + 2] * (qq.z * iq);
            o += sr[4 * cI + 3] * (qq.w * iq);
            *(float4 *)(tr + 4 * cI) = make_float4(sr[4 * cI], sr[4 * cI + 1], sr[4 * cI + 2], sr[4 * cI + 3]);
        }
        wave_lds_sync();
        float4 *Sw = (float4 *)(a.S + ((size_t)hv * DK + wave * 64) * DK);
#pragma unroll
        for (int i = 0; i < DK / 4; i++) {
            const int f = lane + 64 * i, r = (4 * f) / DK, col = (4 * f) % DK;
            stg(Sw + f, *(const float4 *)(tile + r * TS + col));
        }
        o *= a.out_scale;
        const double so = wave_sum_d((double)o * o);
        if (lane == 0) runs[wave] = so;
    }
    c.stamp(4);
    lds_barrier();
    if (row) {
        double tot = runs[0];
        for (int k = 1; k < NQ; k++) tot += runs[k];
        const float inv = (float)(1.0 / sqrt(tot / (double)DK + (double)a.eps));
        stc(a.o + (size_t)hv * DK + wave * 64 + lane, llw(o * inv * nw * zs[wave * 64 + lane], c.tag));
    }
    c.stamp(5);
}

// ---- MoE down projection + combine (src/ornith_rforward.c:375-409) ---------------
// Workgroup vb owns rows [vb * rpb, +rpb) of the hidden state. The front wave
// polls the router logits; the workgroup routes (the same selection as the
// experts operation); the back waves then request the down weights of the
// routed experts and the shared expert for their units (a unit: one
// super-block of one (row, slot), UPT per back thread) while the front wave
// polls h and the residual rows; every slot's h is quantised to Q8_K
// (q8k_blocks), the units reduced, and each row combined x_r + ((sum_j w_j *
// dot_j) + shg * dot_shared) in the reference's order.
// LDS: [ns slots' Q8_K planes][v: ns * in floats][dots: rpb * ns][logits]
template <int T, int UPT>
OH_DEV void dop_down(const oh_ddown &D, int vb, uint8_t *smem, const Dctl &c) {
    __shared__ int rsel[64], rbad, rcnt[64];
    __shared__ float rwt[64], rshg, rsl;
    __shared__ float xrow[64];
    const int tid = tid_x(), lane = lane_id(), wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nb = D.nb, in = D.in, ns = D.k + (D.sA ? 1 : 0);
    const int row0 = vb * D.rpb;
    const int nrow = D.rows - row0 < D.rpb ? (D.rows - row0 > 0 ? D.rows - row0 : 0) : D.rpb;
    const int U = nrow * ns * nb;
    const int sq = (nb * kAS + nb * 36 + 15) & ~15;
    float *v = (float *)(smem + ns * sq);
    float *dots = v + ns * in;
    DRoute R{dots + 64 * ns, rsel, &rbad, rcnt, rwt, &rshg, &rsl};
    c.stamp(0);
    if (wave == 0) route_fetch(R, D.rlog, D.shl, D.ne, c);
    lds_barrier();
    dec_route(R, D.ne, D.k, D.shl != nullptr);
    c.stamp(1);
    SB<T> r[UPT];
    const int bt = tid - 64;                  // back thread
    if (wave > 0) {
#pragma unroll
        for (int k = 0; k < UPT; k++) {
            const int u0 = bt + 192 * k, u = u0 < U ? u0 : (U > 0 ? U - 1 : 0);
            const int sbi = u % nb, j = (u / nb) % ns, rl = u / (nb * ns);
            const bool sh = j >= D.k;
            const WP wp = sh ? WP{D.sA, D.sB, D.sC} : WP{D.A, D.B, D.C};
            const int64_t rb = sh ? 0 : (int64_t)rsel[j] * D.rows;
            const int rr = row0 + rl < D.rows ? row0 + rl : D.rows - 1;
            if (192 * k < U) sb_load(r[k], wp, (rb + rr) * nb + sbi);
        }
    } else {
        ll_fetch_wave<32>(v, D.h, ns * in, c);
        if (nrow > 0) ll_fetch_wave<1>(xrow, D.xres + row0, nrow, c);
    }
    lds_barrier();                            // h and the residual rows are in LDS
    c.stamp(2);
    for (int jj = wave; jj < ns; jj += 4) {
        uint8_t *b = smem + (size_t)jj * sq;
        for (int q0 = 0; q0 < nb; q0 += 4)
            q8k_blocks<4>(v + (size_t)jj * in, q0, 1, nb, (int8_t *)b, (float *)(b + mv_lds_d_off(nb)),
                          (int16_t *)(b + mv_lds_bs_off(nb)), kAS);
    }
    lds_barrier();
    c.stamp(4);
    if (wave > 0) {
#pragma unroll
        for (int k = 0; k < UPT; k++) {
            if (192 * k >= U) break;
            const int u = bt + 192 * k;
            const int uc = u < U ? u : U - 1;
            const int sbi = uc % nb, j = (uc / nb) % ns, rl = uc / (nb * ns);
            const uint8_t *b = smem + (size_t)j * sq;
            const float tw = sb_term(r[k], (const int8_t *)b + sbi * kAS,
                                     (const int16_t *)(b + mv_lds_bs_off(nb)) + sbi * 16,
                                     ((const float *)(b + mv_lds_d_off(nb)))[sbi]);
            const float t = u < U ? tw : 0.0f;
            // the (row, slot)'s nb terms sit in nb consecutive lanes: added in order
            float acc = 0.0f;
            const int base = lane - sbi;
            for (int i = 0; i < nb; i++) acc += shfl(t, base + i);
            if (u < U && sbi == 0) dots[rl * ns + j] = acc;
        }
    }
    lds_barrier();
    if (tid < nrow) {
        float acc = 0.0f;
        for (int jj = 0; jj < D.k; jj++) acc += rwt[jj] * dots[tid * ns + jj];
        if (D.sA) {
            const float so = dots[tid * ns + D.k];
            const float vv = D.shl ? so * rshg : so;
            acc += vv;
        }
        stc(D.y + row0 + tid, llw(xrow[tid] + acc, c.tag));
    }
    c.stamp(5);
}

// ---- GQA (src/ornith_rforward.c:419-455, src/ornith_attn.c:65-149) --------------
// prep: prep_body's arithmetic on the tagged q/k/v projection (per-head RMSNorm,
// partial NeoX RoPE, Q8 append of k and v at pos); queries, gate and the KV
// entry go out with device-scope stores, then the workgroup's flag.
OH_DEV void dop_prep(const oh_datt &d, int vb, const Dctl &c) {
    __shared__ float v[256];
    __shared__ double red[4];
    __shared__ float amax_s[4];
    const oh_op_prep &a = d.p;
    const int pos = c.pos, hb = vb, t = tid_x();
    const int nh = a.nh, nkv = a.nkv, hd = a.hd, cap = a.cap;
    const bool isq = hb < nh;
    const int h = isq ? hb : hb - nh;
    const int r = a.rot <= 0 || a.rot > hd ? hd : a.rot;
    const int half = r / 2;
    const float *nw = isq ? a.q_norm : a.k_norm;
    const float2 *rope = (const float2 *)a.rope;
    const float nwt = t < hd ? ldg(nw + t) : 0.0f;
    const int pi = t < half ? t : t - half;
    const float2 cs = t < 2 * half ? ldg(rope + (size_t)pos * (hd / 2) + pi) : make_float2(1.0f, 0.0f);
    // the head's value and its gate (query heads) or raw v (kv heads)
    const size_t kofs = (size_t)nh * 2 * hd, vofs = kofs + (size_t)nkv * hd;
    const uint64_t *wa[2];
    wa[0] = t < hd ? (isq ? d.qkv + (size_t)h * 2 * hd + t : d.qkv + kofs + (size_t)h * hd + t) : nullptr;
    wa[1] = t < hd ? (isq ? d.qkv + (size_t)h * 2 * hd + hd + t : d.qkv + vofs + (size_t)h * hd + t) : nullptr;
    uint64_t w[2];
#pragma unroll
    for (int k = 0; k < 2; k++) w[k] = wa[k] ? ldc(wa[k]) : ((uint64_t)c.tag << 32);
    if (!ll_settle<2>(w, [&](int k) { return wa[k]; }, c)) c.fail();
    const float x = t < hd ? ll_f(w[0]) : 0.0f;
    const float other = t < hd ? ll_f(w[1]) : 0.0f;
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
    } else {
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
                const int c0 = shfl(code, (lane_id() & ~3) + 0), c1 = shfl(code, (lane_id() & ~3) + 1);
                const int c2 = shfl(code, (lane_id() & ~3) + 2), c3 = shfl(code, (lane_id() & ~3) + 3);
                if (t < hd && (t & 3) == 0)
                    stc(a.Kt + ((size_t)h * (hd / 4) + t / 4) * cap + pos,
                        (uint32_t)(c0 & 0xff) | ((uint32_t)(c1 & 0xff) << 8) |
                        ((uint32_t)(c2 & 0xff) << 16) | ((uint32_t)(c3 & 0xff) << 24));
                if (t == 0) stc(a.Ks + off, scale);
            } else {
                const size_t vo = (((size_t)h * (cap / 16) + pos / 16) * hd + t) * 16 + (pos & 15);
                if (t < hd) stc(a.Vq + vo, (int8_t)code);
                if (t < hd && a.Vh) stc(a.Vh + vo, f16_bits_of_code(code));
                if (t == 0) stc(a.Vs + off, scale);
            }
        }
    }
    flag_set(d.flags + vb, c);
}


// attention body of the per-launch path (exact walk or flash chunks) once
// every prep workgroup has published; then this workgroup's flag
OH_DEV void dop_attn(const oh_datt &d, int vb, const Dctl &c) {
    flags_wait(d.wflags, d.nwait_ex, c);
    NoWait w;
    attn_main_body(d.a, vb, c.pos, w);
    flag_set(d.flags + vb, c);
}

// merge of the flash chunks (nothing to do inside the exact walk)
OH_DEV void dop_combine(const oh_datt &d, int vb, const Dctl &c) {
    if (c.pos + 1 <= d.lim) return;
    flags_wait(d.wflags, d.nwait_fl, c);
    NoWait w;
    combine_body(d.a, vb, c.pos, w, d.lim);
    flag_set(d.flags + vb, c);
}

// ---- greedy token (src/ornith_rforward.c:18-22): the largest logit, the lowest
// index among equals, from the lm_head workgroups' partials (workgroup 0)
OH_DEV void dop_argmax(const oh_dargmax &a, int32_t *io, const Dctl &c) {
    __shared__ float sv[4];
    __shared__ int si[4];
    const int t = tid_x();
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int p0 = 0; p0 < a.nparts; p0 += 256) {
        const int p = p0 + t;
        uint64_t w[2];
        w[0] = p < a.nparts ? ldc(a.amax + 2 * p) : ll_ready(c);
        w[1] = p < a.nparts ? ldc(a.amax + 2 * p + 1) : ll_ready(c);
        if (!ll_settle<2>(w, [&](int k) { return a.amax + 2 * p + k; }, c)) break;
        if (p < a.nparts) {
            const float x = ll_f(w[0]);
            const int xi = (int)(uint32_t)w[1];
            if (x > bv || (x == bv && xi < bi)) { bv = x; bi = xi; }
        }
    }
    for (int m = 32; m >= 1; m >>= 1) {
        const float ov = shfl_xor(bv, m);
        const int oi = shfl_xor(bi, m);
        if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
    }
    if (lane_id() == 0) { sv[t >> 6] = bv; si[t >> 6] = bi; }
    __syncthreads();
    if (t == 0) {
        bv = sv[0]; bi = si[0];
        for (int k = 1; k < 4; k++) if (sv[k] > bv || (sv[k] == bv && si[k] < bi)) { bv = sv[k]; bi = si[k]; }
        if (bi == 0x7fffffff) bi = 0;
        stc(a.toks + c.pos + 1, (int32_t)bi);
        stc(io + OH_IO_BEST, (int32_t)bi);
    }
}

} // namespace

// The decode step: every workgroup walks the program (nops operations in
// device memory, their descriptors double-buffered in LDS); operation i's
// virtual blocks go to workgroups round-robin. The position and the tag come
// from io. At the end the last workgroup to finish advances the position
// (advance != 0) and the tag (never 0), so the next launch's words are told
// apart from this one's.
// ts (profiling, optional): each workgroup's real-time clock at its start
// (ts[b]) and when it is done with operation i (ts[(i + 1) * grid + b]);
// ts2: operation prof_op's sub-phase clocks, 8 per workgroup.
extern "C" __global__ void __launch_bounds__(256, 1)
oh_k_decode(const oh_dop *__restrict__ prog, int nops, int32_t *io, int advance, uint64_t *ts, int prof_op,
            uint64_t *ts2) {
    extern __shared__ __align__(16) uint8_t smem[];
    // s_dead[p]: a wait gave up during an operation of parity p. It is read
    // after that operation's closing barrier; a thread that fails in the next
    // operation writes the other word, so every thread reads the same value.
    __shared__ int s_dead[2];
    Dctl c;
    c.pos = ldc(io + OH_IO_POS);
    c.tag = (uint32_t)ldc(io + OH_IO_TAG);
    c.err = io + OH_IO_ERR;
    c.dead = s_dead;
    c.par = 0;
    c.st = nullptr;
    if (ts && tid_x() == 0) ts[blockIdx.x] = dec_now();
    if (tid_x() < 32) g_dexp[tid_x()] = k_exp2_tab[tid_x()];
    if (tid_x() == 0) { s_dead[0] = 0; s_dead[1] = 0; }
    // operation descriptors in LDS, double-buffered: operation i + 1's words
    // are requested when operation i starts and stored when it ends
    constexpr int DW = (int)((sizeof(oh_dop) + 3) / 4);
    static_assert(DW <= 512, "descriptor larger than two words per thread");
    __shared__ __align__(16) uint32_t dbuf[2][DW];
    {
        const uint32_t *src = (const uint32_t *)prog;
        const int t = tid_x();
        if (t < DW) dbuf[0][t] = ldg(src + t);
        if (t + 256 < DW) dbuf[0][t + 256] = ldg(src + t + 256);
        __syncthreads();
    }
    for (int i = 0; i < nops; i++) {
        uint32_t nx0 = 0, nx1 = 0;
        if (i + 1 < nops) {
            const uint32_t *src = (const uint32_t *)(prog + i + 1);
            const int t = tid_x();
            nx0 = t < DW ? ldg(src + t) : 0u;
            nx1 = t + 256 < DW ? ldg(src + t + 256) : 0u;
        }
        const oh_dop &op = *(const oh_dop *)dbuf[i & 1];
        c.st = ts2 && i == prof_op ? ts2 + (size_t)blockIdx.x * 8 : nullptr;
        c.par = i & 1;
        const int kind = op.kind, nvb = op.nvb;
        for (int vb = (int)blockIdx.x; vb < nvb; vb += (int)gridDim.x) {
            switch (kind) {
            case OH_D_EMBED: dop_embed(op.u.emb, vb, c); break;
            case OH_D_MV: {
                const oh_dmv &M = op.u.mv;
                const int t = M.s[0].type, nb = M.nb;
                if (t == OH_Q4_K) {
                    if (nb == 2) dop_mv<OH_Q4_K, 2>(M, vb, smem, c);
                    else if (nb == 4) dop_mv<OH_Q4_K, 4>(M, vb, smem, c);
                    else if (nb == 8) dop_mv<OH_Q4_K, 8>(M, vb, smem, c);
                    else dop_mv<OH_Q4_K, 16>(M, vb, smem, c);
                } else if (t == OH_Q6_K) {
                    if (nb == 4) dop_mv<OH_Q6_K, 4>(M, vb, smem, c);
                    else if (nb == 8) dop_mv<OH_Q6_K, 8>(M, vb, smem, c);
                    else dop_mv<OH_Q6_K, 16>(M, vb, smem, c);
                } else {
                    if (nb == 2) dop_mv<OH_Q8_0, 2>(M, vb, smem, c);
                    else if (nb == 4) dop_mv<OH_Q8_0, 4>(M, vb, smem, c);
                    else dop_mv<OH_Q8_0, 8>(M, vb, smem, c);
                }
                break;
            }
            case OH_D_DELTA:
                if (op.u.dl.dk == 128) {
                    if (op.u.dl.K <= 4) dop_delta<128, 4>(op.u.dl, vb, (float *)smem, c);
                    else dop_delta<128, 8>(op.u.dl, vb, (float *)smem, c);
                } else {
                    if (op.u.dl.K <= 4) dop_delta<64, 4>(op.u.dl, vb, (float *)smem, c);
                    else dop_delta<64, 8>(op.u.dl, vb, (float *)smem, c);
                }
                break;
            case OH_D_PREP: dop_prep(op.u.at, vb, c); break;
            case OH_D_ATTN: dop_attn(op.u.at, vb, c); break;
            case OH_D_COMBINE: dop_combine(op.u.at, vb, c); break;
            case OH_D_DOWN: {
                const oh_ddown &D = op.u.dn;
                const bool one = D.rpb * (D.k + (D.sA ? 1 : 0)) * D.nb <= 192;
                if (D.type == OH_Q4_K) { if (one) dop_down<OH_Q4_K, 1>(D, vb, smem, c); else dop_down<OH_Q4_K, 4>(D, vb, smem, c); }
                else if (D.type == OH_Q6_K) { if (one) dop_down<OH_Q6_K, 1>(D, vb, smem, c); else dop_down<OH_Q6_K, 4>(D, vb, smem, c); }
                else { if (one) dop_down<OH_Q8_0, 1>(D, vb, smem, c); else dop_down<OH_Q8_0, 4>(D, vb, smem, c); }
                break;
            }
            case OH_D_ARGMAX: dop_argmax(op.u.am, io, c); break;
            default: break;
            }
            lds_barrier();                    // LDS is reused by the next virtual block
        }
        if (ts && tid_x() == 0) ts[(size_t)(i + 1) * gridDim.x + blockIdx.x] = dec_now();
        if (i + 1 < nops) {
            const int t = tid_x();
            if (t < DW) dbuf[(i + 1) & 1][t] = nx0;
            if (t + 256 < DW) dbuf[(i + 1) & 1][t + 256] = nx1;
        }
        lds_barrier();
        if (s_dead[i & 1]) break;            // a wait gave up: leave (io[OH_IO_ERR] is set)
    }
    if (tid_x() == 0) {
        const int done = __hip_atomic_fetch_add(io + OH_IO_DONE, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        if (done == (int)gridDim.x - 1) {
            stc(io + OH_IO_DONE, (int32_t)0);
            if (advance) stc(io + OH_IO_POS, (int32_t)(c.pos + 1));
            const uint32_t nt = c.tag + 1u;
            stc(io + OH_IO_TAG, (int32_t)(nt == 0u ? 1u : nt));
        }
    }
}
