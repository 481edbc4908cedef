// oh_synth.hip - on-device random-init weights: the counter-based value
// streams of the repository's GGUF generator and the reference's block
// encoders (src/ornith_quant.c:155-175 Q8_0, :451-500 Q6_K, :507-561 Q4_K),
// writing straight into the plane layout. The encoders keep the reference's
// float operation order, lroundf (half away from zero) and the binary16
// round-to-nearest-even conversion, so a synthesised tensor equals the GGUF
// tensor the oracle generator writes, byte for byte.
// Included into oh_kernels.hip.

namespace {

constexpr uint64_t kGamma = 0x9E3779B97F4A7C15ull;

OH_DEV uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// lroundf semantics: nearest, halfway cases away from zero
OH_DEV long round_away(float x) {
    float r = truncf(x);
    if (fabsf(x - r) >= 0.5f) r += copysignf(1.0f, x);
    return (long)r;
}

// binary32 -> binary16, nearest-even incl. subnormals (src/ornith_quant.c:14-41)
OH_DEV uint16_t f2h_rne(float f) {
    const uint32_t b = f2u(f);
    const uint32_t s = (b >> 16) & 0x8000u;
    const int32_t e = (int32_t)((b >> 23) & 0xff);
    uint32_t m = b & 0x7fffffu;
    if (e == 0xff) return (uint16_t)(s | 0x7c00u | (m ? 0x200u : 0u));
    const int32_t he = e - 112;
    if (he >= 31) return (uint16_t)(s | 0x7c00u);
    if (he <= 0) {
        if (he < -10) return (uint16_t)s;
        m |= 0x800000u;
        const uint32_t sh = (uint32_t)(14 - he);
        uint32_t h = m >> sh;
        const uint32_t rem = m & ((1u << sh) - 1u), half = 1u << (sh - 1);
        if (rem > half || (rem == half && (h & 1u))) h++;
        return (uint16_t)(s | h);
    }
    uint32_t h = s | ((uint32_t)he << 10) | (m >> 13);
    const uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)h;
}

} // namespace

// value i of a Gaussian stream: Irwin-Hall(12) of 16-bit lanes, one scaling
extern "C" __global__ void __launch_bounds__(256)
oh_k_fill_gauss(uint64_t key, float sigma, float *dst, int64_t n) {
    const float c = sigma / 131072.0f;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
        int64_t s = 0;
        for (int k = 1; k <= 3; k++) {
            const uint64_t r = mix64(key + (3 * (uint64_t)i + (uint64_t)k) * kGamma);
            s += (int64_t)(r & 0xffff) + (int64_t)((r >> 16) & 0xffff) + (int64_t)((r >> 32) & 0xffff) +
                 (int64_t)(r >> 48);
        }
        dst[i] = (float)(2 * s - 786420) * c;
    }
}

extern "C" __global__ void __launch_bounds__(256)
oh_k_fill_uniform(uint64_t key, float lo, float hi, float *dst, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
        const uint64_t r = mix64(key + ((uint64_t)i + 1) * kGamma);
        const float f = (float)(uint32_t)(r >> 40) / 16777216.0f;
        dst[i] = lo + (hi - lo) * f;
    }
}

// one thread per 256-element super-block of x -> planes
extern "C" __global__ void __launch_bounds__(256)
oh_k_encode(const float *x, int type, int64_t nblk, uint8_t *A, uint8_t *B, uint8_t *C) {
    const int64_t b = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (b >= nblk) return;
    const float *v = x + b * 256;
    if (type == OH_Q8_0) {
        for (int sb = 0; sb < 8; sb++) {
            const float *w = v + 32 * sb;
            float amax = 0.0f;
            for (int j = 0; j < 32; j++) { const float a = fabsf(w[j]); if (a > amax) amax = a; }
            const float d = amax / 127.0f;
            const float id = d != 0.0f ? 1.0f / d : 0.0f;
            *(uint16_t *)(B + b * 16 + 2 * sb) = f2h_rne(d);
            for (int j = 0; j < 32; j++) {
                long r = round_away(w[j] * id);
                A[oh_a_off(OH_Q8_0, b, 32 * sb + j)] = (uint8_t)(int8_t)(r > 127 ? 127 : (r < -127 ? -127 : r));
            }
        }
    } else if (type == OH_Q4_K) {
        float ssc[8], smn[8];
        for (int j = 0; j < 8; j++) {
            const float *w = v + 32 * j;
            float lo = w[0], hi = w[0];
            for (int l = 1; l < 32; l++) { if (w[l] < lo) lo = w[l]; if (w[l] > hi) hi = w[l]; }
            if (lo > 0.0f) lo = 0.0f;
            ssc[j] = (hi - lo) / 15.0f;
            smn[j] = -lo;
        }
        float msc = 0.0f, mmn = 0.0f;
        for (int j = 0; j < 8; j++) { if (ssc[j] > msc) msc = ssc[j]; if (smn[j] > mmn) mmn = smn[j]; }
        const float d = msc / 63.0f, dmin = mmn / 63.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f, idm = dmin != 0.0f ? 1.0f / dmin : 0.0f;
        uint8_t sc[8], mn[8];
        for (int j = 0; j < 8; j++) {
            long s = round_away(ssc[j] * id), m = round_away(smn[j] * idm);
            sc[j] = (uint8_t)(s < 0 ? 0 : (s > 63 ? 63 : s));
            mn[j] = (uint8_t)(m < 0 ? 0 : (m > 63 ? 63 : m));
        }
        uint8_t hdr[16];
        const uint16_t dh = f2h_rne(d), mh = f2h_rne(dmin);
        hdr[0] = (uint8_t)dh; hdr[1] = (uint8_t)(dh >> 8); hdr[2] = (uint8_t)mh; hdr[3] = (uint8_t)(mh >> 8);
        uint8_t *ps = hdr + 4;
        for (int i = 0; i < 12; i++) ps[i] = 0;
        for (int j = 0; j < 4; j++) { ps[j] = sc[j] & 63; ps[j + 4] = mn[j] & 63; }
        for (int j = 4; j < 8; j++) {
            ps[j + 4] = (uint8_t)((sc[j] & 0x0f) | ((mn[j] & 0x0f) << 4));
            ps[j - 4] |= (uint8_t)(((sc[j] >> 4) & 3) << 6);
            ps[j] |= (uint8_t)(((mn[j] >> 4) & 3) << 6);
        }
        for (int i = 0; i < 16; i++) B[b * 16 + i] = hdr[i];
        for (int j = 0; j < 8; j += 2) {
            const float rs0 = d * sc[j], rm0 = dmin * mn[j], irs0 = rs0 != 0.0f ? 1.0f / rs0 : 0.0f;
            const float rs1 = d * sc[j + 1], rm1 = dmin * mn[j + 1], irs1 = rs1 != 0.0f ? 1.0f / rs1 : 0.0f;
            for (int l = 0; l < 32; l++) {
                long q0 = round_away((v[32 * j + l] + rm0) * irs0);
                long q1 = round_away((v[32 * (j + 1) + l] + rm1) * irs1);
                q0 = q0 < 0 ? 0 : (q0 > 15 ? 15 : q0);
                q1 = q1 < 0 ? 0 : (q1 > 15 ? 15 : q1);
                A[oh_a_off(OH_Q4_K, b, 16 * j + l)] = (uint8_t)(q0 | (q1 << 4));
            }
        }
    } else if (type == OH_Q6_K) {
        float gs[16], maxs = 0.0f;
        for (int g = 0; g < 16; g++) {
            float amax = 0.0f;
            for (int l = 0; l < 16; l++) { const float a = fabsf(v[16 * g + l]); if (a > amax) amax = a; }
            gs[g] = amax / 32.0f;
            if (gs[g] > maxs) maxs = gs[g];
        }
        const float d = maxs / 127.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
        int8_t sc[16];
        for (int g = 0; g < 16; g++) {
            long s = round_away(gs[g] * id);
            sc[g] = (int8_t)(s < 0 ? 0 : (s > 127 ? 127 : s));
            B[b * 16 + g] = (uint8_t)sc[g];
        }
        *(uint16_t *)(C + b * 2) = f2h_rne(d);
        uint8_t Q[256];
        for (int g = 0; g < 16; g++) {
            const float sg = d * sc[g], isg = sg != 0.0f ? 1.0f / sg : 0.0f;
            for (int l = 0; l < 16; l++) {
                long q = round_away(v[16 * g + l] * isg) + 32;
                Q[16 * g + l] = (uint8_t)(q < 0 ? 0 : (q > 63 ? 63 : q));
            }
        }
        for (int h = 0; h < 2; h++) {
            const uint8_t *q = Q + 128 * h;
            for (int l = 0; l < 32; l++) {
                A[oh_a_off(OH_Q6_K, b, 64 * h + l)] = (uint8_t)((q[l] & 15) | ((q[l + 64] & 15) << 4));
                A[oh_a_off(OH_Q6_K, b, 64 * h + 32 + l)] = (uint8_t)((q[l + 32] & 15) | ((q[l + 96] & 15) << 4));
                A[oh_a_off(OH_Q6_K, b, 128 + 32 * h + l)] =
                    (uint8_t)((q[l] >> 4) | ((q[l + 32] >> 4) << 2) | ((q[l + 64] >> 4) << 4) | ((q[l + 96] >> 4) << 6));
            }
        }
    }
}

// IQ2_XXS (src/ornith_quant.c:703-789, quantize_iq2_xxs_core without
// importance weights): one wave per 256-element super-block. Lanes 0..31 take
// the 32 sub-groups of 8 (group lane / 4, sub-group lane % 4): magnitudes and
// the sign bits, an odd count fixed by flipping the smallest magnitude. Per
// group of 32 the scale search over trial magnitudes t = 4..64: for each
// trial the four sub-groups' smallest error over the 256 grid points (lane l
// holds points l + 64q), added in sub-group order, a strictly smaller total
// replacing the best as in the reference's loop. Then d (binary16), the 4-bit
// group scales and the grid picks (the lowest index among equal errors).
extern "C" __global__ void __launch_bounds__(256)
oh_k_encode_iq2xxs(const float *x, int64_t nblk, uint8_t *A, uint8_t *C) {
    __shared__ float smag[4][32][8];
    __shared__ uint32_t ssgn[4][32];
    const int wave = tid_x() >> 6, lane = lane_id();
    const int64_t b = (int64_t)blockIdx.x * 4 + wave;
    if (b >= nblk) return;
    const float *v = x + b * 256;
    float (*mag)[8] = smag[wave];
    if (lane < 32) {
        const float *xk = v + 8 * lane;
        uint32_t s = 0;
        int nneg = 0;
        float m[8];
        for (int j = 0; j < 8; j++) {
            const float val = xk[j];
            if (val < 0.0f) { m[j] = -val; s |= 1u << j; nneg++; }
            else m[j] = val;
        }
        if (nneg & 1) {
            int imin = 0;
            float vmin = m[0];
            for (int j = 1; j < 8; j++)
                if (m[j] < vmin) { vmin = m[j]; imin = j; }
            s ^= 1u << imin;
        }
        for (int j = 0; j < 8; j++) mag[lane][j] = m[j];
        ssgn[wave][lane] = s & 127u;
    }
    wave_lds_sync();
    float gm[4][8];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const uint64_t gw = k_iq2_grid[lane + 64 * q];
#pragma unroll
        for (int j = 0; j < 8; j++) gm[q][j] = (float)((gw >> (8 * j)) & 0xff);
    }
    // the smallest sum_j (mag_j - s * grid_j)^2 over the grid and its first index
    auto best = [&](const float *mg, float s, int *gidx) -> float {
        float tm[8];
#pragma unroll
        for (int j = 0; j < 8; j++) tm[j] = mg[j];
        float be = 1e30f;
        int bg = 0;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            float e = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const float df = tm[j] - s * gm[q][j];
                e += df * df;
            }
            if (e < be) { be = e; bg = lane + 64 * q; }
        }
        for (int m = 32; m >= 1; m >>= 1) {
            const float oe = shfl_xor(be, m);
            const int og = shfl_xor(bg, m);
            if (oe < be || (oe == be && og < bg)) { be = oe; bg = og; }
        }
        if (gidx) *gidx = bg;
        return be;
    };
    float gsc[8];
    for (int g32 = 0; g32 < 8; g32++) {
        float gmax = 0.0f;
        for (int k = 0; k < 4; k++)
            for (int j = 0; j < 8; j++)
                if (mag[4 * g32 + k][j] > gmax) gmax = mag[4 * g32 + k][j];
        if (gmax < 1e-12f) { gsc[g32] = 0.0f; continue; }
        const float base = gmax / 43.0f;
        float best_s = base, best_e = 1e30f;
        for (int t = 4; t <= 64; t++) {
            const float s = base * 43.0f / (float)t;
            float tot = 0.0f;
            for (int k = 0; k < 4; k++) tot += best(mag[4 * g32 + k], s, nullptr);
            if (tot < best_e) { best_e = tot; best_s = s; }
        }
        gsc[g32] = best_s;
    }
    float mx = 0.0f;
    for (int g32 = 0; g32 < 8; g32++) if (gsc[g32] > mx) mx = gsc[g32];
    uint32_t *qw = (uint32_t *)(A + b * 64);
    if (mx <= 0.0f) {                          // all-zero block
        if (lane < 16) stg(qw + lane, 0u);
        if (lane == 0) stg((uint16_t *)C + b, f2h_rne(0.0f));
        return;
    }
    const uint16_t dh = f2h_rne(mx / (0.25f * 15.5f));
    const float qd = 0.25f * h2f(dh);
    uint32_t words[16];
    for (int g32 = 0; g32 < 8; g32++) {
        long l = 0;
        if (qd > 0.0f && gsc[g32] > 0.0f) l = round_away(gsc[g32] / qd - 0.5f);
        l = l < 0 ? 0 : (l > 15 ? 15 : l);
        const float db = qd * (0.5f + (float)l);
        uint32_t a0 = 0, a1 = 0;
        for (int k = 0; k < 4; k++) {
            int g = 0;
            if (db > 0.0f) best(mag[4 * g32 + k], db, &g);
            a0 |= (uint32_t)(g & 0xff) << (8 * k);
            a1 |= (ssgn[wave][4 * g32 + k] & 127u) << (7 * k);
        }
        a1 |= (uint32_t)l << 28;
        words[2 * g32] = a0;
        words[2 * g32 + 1] = a1;
    }
    if (lane < 16) {
        uint32_t w = words[0];
#pragma unroll
        for (int k = 1; k < 16; k++) if (lane == k) w = words[k];
        stg(qw + lane, w);
    }
    if (lane == 0) stg((uint16_t *)C + b, dh);
}
