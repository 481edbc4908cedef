// oh_attn_mfma.hip - GQA prompt attention on the matrix cores (prefill tokens
// whose context exceeds the exact walk's limit). Included into oh_kernels.hip.
//
// Reference: ornith_gqa_step over the Q8 KV cache (src/ornith_attn.c:87-149)
// for every prompt token (src/ornith_rforward.c:513-556): score_t =
// (q . code_t) * Ks_t / sqrt(hd), softmax over t <= position, output
// sum_t p_t * Vs_t * code_t, then o *= sigmoid(gate). Past the exact walk the
// engine already re-associates these sums (flash chunks, tolerance-checked);
// this kernel computes the same quantities in a flash-attention form on
// v_mfma_f32_32x32x16_f16: fp16 operands (queries pre-scaled by 1/sqrt(hd),
// K and V codes times their per-position scale), fp32 accumulation, online
// softmax in fp32. Tolerance bar as for the flash chunks (logits within 1e-2
// relative L2 of the reference order).
//
// fp16 range: each per-position scale s = m * 2^e (m in [1, 2)) enters the
// fp16 operands only as its significand, code * m (|.| < 254, so every
// operand is a normal fp16 or zero, whatever the scales are); the exponents
// are applied in fp32, exactly: a score is multiplied by its key's 2^e after
// the product, and the output accumulator is held in units of 2^E, E the
// largest V exponent of the tiles seen so far (rescaled exactly when E
// grows), so a probability enters P as p * 2^(e - E) <= 1.
//
// Work: a block of 4 waves takes one KV head g and TPB prompt tokens; wave w
// owns 32 query rows = (32 / G) tokens x the G query heads of g. Per KV tile of
// 64 positions the block converts the Q8 codes to fp16 in LDS once; each wave
// then forms S^T = K Q^T (64 positions x its 32 queries: the positions of a
// query land in one lane, so its row max and sum are lane-local plus one lane
// exchange), the probabilities P^T, and O^T += V^T P^T (hd x 32, in
// accumulator registers). The next tile's codes are in flight during the
// current tile's products.

typedef _Float16 fa_h8 __attribute__((ext_vector_type(8)));
typedef _Float16 fa_h4 __attribute__((ext_vector_type(4)));
typedef float fa_f32x16 __attribute__((ext_vector_type(16)));

constexpr int kFaT = 64;                  // KV positions per tile
constexpr int kFaPS = kFaT + 8;           // P^T and V^T row stride (fp16): 144 B, bank-conflict free

OH_HD inline int fa_ks(int hd) { return hd + 8; }     // K row stride (fp16)
OH_HD inline int fa_lds_bytes(int hd) {
    return (kFaT * fa_ks(hd) + hd * kFaPS + 4 * 32 * kFaPS) * 2 + 4 * kFaT * 4 + 16;
}

namespace {

template <int HD, int G>
__global__ void __launch_bounds__(256, 1)
oh_k_attn_mfma_rows(oh_op_attn a, int base, int tf0, int nt) {
    extern __shared__ __align__(16) uint8_t fsm[];
    constexpr int TPW = 32 / G, TPB = 4 * TPW;         // tokens per wave / block
    constexpr int NKS = HD / 16, NDT = HD / 32;         // K-steps of S, dim tiles of O
    constexpr int KS = HD + 8;
    _Float16 *K16 = (_Float16 *)fsm;                    // [64 positions][KS]
    _Float16 *V16 = K16 + kFaT * KS;                    // [HD dims][kFaPS]
    _Float16 *P16 = V16 + HD * kFaPS;                   // [4 waves][32 queries][kFaPS]
    float *sKs = (float *)(P16 + 4 * 32 * kFaPS);       // [64] K scale significands
    float *sVs = sKs + kFaT;                            // [64] V scale significands
    int *sKe = (int *)(sVs + kFaT);                     // [64] K scale exponents
    int *sVe = sKe + kFaT;                              // [64] V scale exponents
    int *sVE = sVe + kFaT;                              // the tile's largest V exponent
    const int tid = tid_x(), lane = lane_id(), wave = tid >> 6;
    const int lq = lane & 31, hf = lane >> 5;           // query column, K half
    const int g = (int)blockIdx.y, nkv = a.nkv, cap = a.cap;
    const int qd = a.nh * HD;
    const int tb0 = tf0 + (int)blockIdx.x * TPB;        // first token of the block
    const int tend = tf0 + nt;
    const int tlast = (tb0 + TPB < tend ? tb0 + TPB : tend) - 1;
    const int ctx = base + tlast + 1;                   // positions the block reads
    const int ntiles = (ctx + kFaT - 1) / kFaT;
    // this lane's query: token tq, head g*G + hi
    const int tq = tb0 + wave * TPW + lq / G, hi = lq % G;
    const bool qvalid = tq < tend;
    const int tqc = qvalid ? tq : tend - 1;
    const int qpos = base + tqc;                        // attends to positions <= qpos
    const int wlast = base + (tb0 + wave * TPW + TPW - 1 < tend ? tb0 + wave * TPW + TPW - 1 : tend - 1);

    // queries (pre-scaled) as the B operand of S^T: K-step s holds dims
    // 16 s + 8 hf .. + 7 of this lane's query
    fa_h8 qf[NKS];
    {
        const float *qsrc = a.qr + (size_t)tqc * qd + (size_t)(g * G + hi) * HD;
#pragma unroll
        for (int s = 0; s < NKS; s++) {
            const float4 x0 = ldg((const float4 *)(qsrc + 16 * s + 8 * hf));
            const float4 x1 = ldg((const float4 *)(qsrc + 16 * s + 8 * hf + 4));
            const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
            for (int j = 0; j < 8; j++) qf[s][j] = (_Float16)(xs[j] * a.scale);
        }
    }
    fa_f32x16 o[NDT];
#pragma unroll
    for (int d = 0; d < NDT; d++)
#pragma unroll
        for (int v = 0; v < 16; v++) o[d][v] = 0.0f;
    float m = -INFINITY, l = 0.0f;
    int E = -1000;                                      // o is held in units of 2^E

    // raw codes of a tile: K words [HD/4][64 positions] as uint4 of four
    // positions, V tiles [4][HD][16 positions] as uint4, and the scales
    constexpr int NKU = HD / 64, NVU = HD / 64;         // uint4 per thread
    uint4 kr[NKU], vr[NVU];
    float scl = 0.0f;
    auto fetch = [&](int tile) {
        const int t0 = tile * kFaT;
#pragma unroll
        for (int i = 0; i < NKU; i++) {
            const int idx = tid + 256 * i, w = idx >> 4;
            int t = t0 + 4 * (idx & 15);
            t = t < cap ? t : cap - 4;
            kr[i] = ldg((const uint4 *)(a.Kt + ((size_t)g * (HD / 4) + w) * cap + t));
        }
#pragma unroll
        for (int i = 0; i < NVU; i++) {
            const int idx = tid + 256 * i, j = idx / HD, d = idx % HD;
            int tj = t0 / 16 + j;
            tj = tj < cap / 16 ? tj : cap / 16 - 1;
            vr[i] = ldg((const uint4 *)a.Vq + ((size_t)g * (cap / 16) + tj) * HD + d);
        }
        if (tid < 2 * kFaT) {
            int t = t0 + (tid & (kFaT - 1));
            t = t < cap ? t : cap - 1;
            scl = ldg((tid < kFaT ? a.Ks : a.Vs) + (size_t)t * nkv + g);
        }
    };
    fetch(0);
    for (int tile = 0; tile < ntiles; tile++) {
        const int t0 = tile * kFaT;
        // scales as significand and exponent, then the codes times the
        // significand as fp16 (positions past the block's context are zero)
        if (tid < 2 * kFaT) {
            const int p = t0 + (tid & (kFaT - 1));
            const float sc = p < ctx ? scl : 0.0f;
            const bool nz = sc != 0.0f && isfinite(sc);
            const int ex = nz ? ilogbf(sc) : -1000;
            (tid < kFaT ? sKs : sVs)[tid & (kFaT - 1)] = nz ? ldexpf(sc, -ex) : (isfinite(sc) ? 0.0f : sc);
            (tid < kFaT ? sKe : sVe)[tid & (kFaT - 1)] = nz ? ex : 0;
            if (tid >= kFaT) {
                const int em = wave_max_i(ex);          // wave 1 holds the V scales
                if (tid == kFaT) *sVE = em;
            }
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < NKU; i++) {
            const int idx = tid + 256 * i, w = idx >> 4, pq = 4 * (idx & 15);
            const uint32_t wd[4] = {kr[i].x, kr[i].y, kr[i].z, kr[i].w};
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const float sc = sKs[pq + u];
                fa_h4 h;
#pragma unroll
                for (int b = 0; b < 4; b++) h[b] = (_Float16)((float)(int8_t)(wd[u] >> (8 * b)) * sc);
                *(fa_h4 *)(K16 + (pq + u) * KS + 4 * w) = h;
            }
        }
#pragma unroll
        for (int i = 0; i < NVU; i++) {
            const int idx = tid + 256 * i, j = idx / HD, d = idx % HD;
            const uint32_t wd[4] = {vr[i].x, vr[i].y, vr[i].z, vr[i].w};
            fa_h8 h0, h1;
#pragma unroll
            for (int b = 0; b < 8; b++) {
                h0[b] = (_Float16)((float)(int8_t)(wd[b >> 2] >> (8 * (b & 3))) * sVs[16 * j + b]);
                h1[b] = (_Float16)((float)(int8_t)(wd[2 + (b >> 2)] >> (8 * (b & 3))) * sVs[16 * j + 8 + b]);
            }
            *(fa_h8 *)(V16 + d * kFaPS + 16 * j) = h0;
            *(fa_h8 *)(V16 + d * kFaPS + 16 * j + 8) = h1;
        }
        __syncthreads();
        if (tile + 1 < ntiles) fetch(tile + 1);
        // a wave whose tokens all precede this tile has nothing to add
        if (t0 <= wlast) {
            // S^T for the two 32-position halves of the tile
            fa_f32x16 sc[2];
#pragma unroll
            for (int pt = 0; pt < 2; pt++) {
#pragma unroll
                for (int v = 0; v < 16; v++) sc[pt][v] = 0.0f;
#pragma unroll
                for (int s = 0; s < NKS; s++) {
                    const fa_h8 ka = *(const fa_h8 *)(K16 + (32 * pt + lq) * KS + 16 * s + 8 * hf);
                    sc[pt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka, qf[s], sc[pt], 0, 0, 0);
                }
            }
            // each key's scale exponent, then the causal mask and the online
            // softmax of this lane's query (its 32 positions here, the other
            // 32 in lane ^ 32)
            float mx = -INFINITY;
#pragma unroll
            for (int pt = 0; pt < 2; pt++)
#pragma unroll
                for (int vg = 0; vg < 4; vg++) {
                    const int4 ke = *(const int4 *)(sKe + 32 * pt + 8 * vg + 4 * hf);
                    const int kes[4] = {ke.x, ke.y, ke.z, ke.w};
#pragma unroll
                    for (int k = 0; k < 4; k++) {
                        const int v = 4 * vg + k, p = t0 + 32 * pt + 8 * vg + 4 * hf + k;
                        sc[pt][v] = p > qpos ? -INFINITY : ldexpf(sc[pt][v], kes[k]);
                        mx = fmaxf(mx, sc[pt][v]);
                    }
                }
            mx = fmaxf(mx, __shfl_xor(mx, 32));
            const float mn = fmaxf(m, mx);
            const float corr = mn == -INFINITY ? 1.0f : __expf(m - mn);
            const int En = E > *sVE ? E : *sVE;         // the output's new unit 2^En
            float ls = 0.0f;
            _Float16 *pw = P16 + (wave * 32 + lq) * kFaPS;
#pragma unroll
            for (int pt = 0; pt < 2; pt++)
#pragma unroll
                for (int vg = 0; vg < 4; vg++) {
                    fa_h4 h;
                    const int4 ve = *(const int4 *)(sVe + 32 * pt + 8 * vg + 4 * hf);
                    const int ves[4] = {ve.x, ve.y, ve.z, ve.w};
#pragma unroll
                    for (int k = 0; k < 4; k++) {
                        const float x = sc[pt][4 * vg + k];
                        const float e = x == -INFINITY ? 0.0f : __expf(x - mn);
                        ls += e;
                        h[k] = (_Float16)ldexpf(e, ves[k] - En);
                    }
                    *(fa_h4 *)(pw + 32 * pt + 8 * vg + 4 * hf) = h;
                }
            ls += __shfl_xor(ls, 32);
            l = l * corr + ls;
            m = mn;
            const float co = ldexpf(corr, E - En);
            E = En;
#pragma unroll
            for (int d = 0; d < NDT; d++)
#pragma unroll
                for (int v = 0; v < 16; v++) o[d][v] *= co;
            wave_lds_sync();
            // O^T += V^T P^T over the tile's 64 positions
#pragma unroll
            for (int ks = 0; ks < kFaT / 16; ks++) {
                const fa_h8 pb = *(const fa_h8 *)(pw + 16 * ks + 8 * hf);
#pragma unroll
                for (int d = 0; d < NDT; d++) {
                    const fa_h8 va = *(const fa_h8 *)(V16 + (32 * d + lq) * kFaPS + 16 * ks + 8 * hf);
                    o[d] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pb, o[d], 0, 0, 0);
                }
            }
        }
        __syncthreads();                                // K16 / V16 / P16 are refilled
    }
    if (!qvalid) return;
    // out = O / l * sigmoid(gate) for this lane's query: dims 32 d + 8 (v/4)
    // + 4 hf + v % 4
    const float inv = 1.0f / l;
    const size_t ob = (size_t)tq * qd + (size_t)(g * G + hi) * HD;
#pragma unroll
    for (int d = 0; d < NDT; d++)
#pragma unroll
        for (int vg = 0; vg < 4; vg++) {
            const int dim = 32 * d + 8 * vg + 4 * hf;
            const float4 gt = ldg((const float4 *)(a.gate + ob + dim));
            const float4 r = make_float4(ldexpf(o[d][4 * vg], E) * inv * ref_sigmoid(gt.x),
                                         ldexpf(o[d][4 * vg + 1], E) * inv * ref_sigmoid(gt.y),
                                         ldexpf(o[d][4 * vg + 2], E) * inv * ref_sigmoid(gt.z),
                                         ldexpf(o[d][4 * vg + 3], E) * inv * ref_sigmoid(gt.w));
            stg((float4 *)(a.out + ob + dim), r);
        }
}

} // namespace

extern "C" hipError_t oh_launch_attn_mfma_rows(const oh_op_attn *a, int base, int tf0, int nt, hipStream_t st) {
    if (nt <= 0) return hipSuccess;
    const int G = a->nh / a->nkv, hd = a->hd;
    void (*k)(oh_op_attn, int, int, int) = nullptr;
#define FA_CASE(H, GG) if (hd == H && G == GG) k = oh_k_attn_mfma_rows<H, GG>;
    FA_CASE(64, 4) FA_CASE(64, 8) FA_CASE(64, 16)
    FA_CASE(128, 4) FA_CASE(128, 8) FA_CASE(128, 16)
    FA_CASE(256, 4) FA_CASE(256, 8) FA_CASE(256, 16)
#undef FA_CASE
    if (!k) return hipErrorNotSupported;
    const int lds = fa_lds_bytes(hd);
    const hipError_t e = hipFuncSetAttribute((const void *)k, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (e != hipSuccess) return e;
    const int tpb = 4 * (32 / G);
    hipLaunchKernelGGL(k, dim3((nt + tpb - 1) / tpb, a->nkv), dim3(256), (size_t)lds, st, *a, base, tf0, nt);
    return hipGetLastError();
}

extern "C" int oh_attn_mfma_supported(int hd, int nh, int nkv) {
    const int G = nkv > 0 ? nh / nkv : 0;
    return (hd == 64 || hd == 128 || hd == 256) && (G == 4 || G == 8 || G == 16) && nh % nkv == 0;
}
