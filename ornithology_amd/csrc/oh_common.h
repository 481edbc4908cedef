// oh_common.h - device helpers shared by the HIP kernels (gfx950 / CDNA4).
//
// Everything here is exact: the scalar float functions reproduce the
// reference CPU path bit for bit (the reference's libm is glibc; its expf and
// log1pf are restated below from their published algorithms and were checked
// against glibc on every float input). All kernels are compiled with
// -ffp-contract=off, so a*b+c is two roundings unless fma() is written.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define OH_DEV __device__ __forceinline__

// ---- bit casts / f16 -------------------------------------------------------
OH_DEV uint32_t f2u(float f) { return __float_as_uint(f); }
OH_DEV float u2f(uint32_t u) { return __uint_as_float(u); }
// the f16 bit pattern of an integer code (exact for |c| <= 2048)
OH_DEV uint16_t f16_bits_of_code(int c) { return __builtin_bit_cast(uint16_t, (_Float16)(float)c); }

// exact binary16 -> binary32 (hardware conversion is exact for every input)
OH_DEV float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

// ---- glibc-compatible expf --------------------------------------------------
// Algorithm of glibc 2.35 sysdeps/ieee754/flt-32/e_expf.c (ARM
// optimized-routines, MIT): x*N/ln2 = k + r with |r| <= 1/2, N = 32;
// 2^(k/N) from a 32-entry table of 2^(i/32) (correctly rounded doubles, exponent
// bias folded in), degree-3 polynomial for 2^(r/N), one rounding to float. The
// reduction r = x*N/ln2 - k and the polynomial are fused multiply-adds, which is
// how the x86-64 FMA build of glibc evaluates them; that form matched glibc's
// expf on every float input.
static __constant__ uint64_t k_exp2_tab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

// tab: the 32 table entries (k_exp2_tab, or a copy of it in LDS)
template <typename TabT>
OH_DEV float ref_expf_tab(float x, const TabT *tab) {
    const uint32_t ax = f2u(x) & 0x7fffffffu;
    if (ax >= 0x42b00000u) {                       // |x| >= 88
        if (f2u(x) == 0xff800000u) return 0.0f;    // -inf
        if (ax >= 0x7f800000u) return x + x;       // nan, +inf
        if (x > 0x1.62e42ep6f) return u2f(0x7f800000u);   // overflow
        if (x < -0x1.9fe368p6f) return 0.0f;              // underflow
    }
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32.0;
    const double shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
    const double c1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    const double xd = (double)x;
    const double z = inv_ln2_n * xd;
    double kd = z + shift;
    const uint64_t ki = (uint64_t)__double_as_longlong(kd);
    kd -= shift;
    const double r = fma(inv_ln2_n, xd, -kd);
    uint64_t t = tab[ki % 32];
    t += ki << 47;
    const double s = __longlong_as_double((long long)t);
    const double p = fma(c0, r, c1);
    const double r2 = r * r;
    double y = fma(c2, r, 1.0);
    y = fma(p, r2, y);
    y = y * s;
    return (float)y;
}
OH_DEV float ref_expf(float x) { return ref_expf_tab(x, k_exp2_tab); }
// The same function without branches: the table path runs for every input
// and the special cases (|x| >= 88: -inf, NaN/+inf, overflow, underflow)
// replace its value by selects, so that several of these in a row overlap
// (the branches of ref_expf_tab keep each one in a block of its own).
template <typename TabT>
OH_DEV float ref_expf_sel(float x, const TabT *tab) {
    const uint32_t ax = f2u(x) & 0x7fffffffu;
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32.0;
    const double shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
    const double c1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    const double xd = (double)x;
    const double z = inv_ln2_n * xd;
    double kd = z + shift;
    const uint64_t ki = (uint64_t)__double_as_longlong(kd);
    kd -= shift;
    const double r = fma(inv_ln2_n, xd, -kd);
    uint64_t t = tab[ki % 32];
    t += ki << 47;
    const double s = __longlong_as_double((long long)t);
    const double p = fma(c0, r, c1);
    const double r2 = r * r;
    double y = fma(c2, r, 1.0);
    y = fma(p, r2, y);
    y = y * s;
    // every candidate formed first, then chosen by masks (a conditional
    // operand would be turned back into a branch)
    const uint32_t v = f2u((float)y), xx = f2u(x + x);
    const uint32_t m_big = 0u - (uint32_t)(ax >= 0x42b00000u);
    const uint32_t m_ninf = m_big & (0u - (uint32_t)(f2u(x) == 0xff800000u));
    const uint32_t m_nan = m_big & ~m_ninf & (0u - (uint32_t)(ax >= 0x7f800000u));
    const uint32_t m_over = m_big & ~m_ninf & ~m_nan & (0u - (uint32_t)(x > 0x1.62e42ep6f));
    const uint32_t m_under = m_big & ~m_ninf & ~m_nan & ~m_over & (0u - (uint32_t)(x < -0x1.9fe368p6f));
    const uint32_t m_keep = ~(m_ninf | m_nan | m_over | m_under);
    return u2f((v & m_keep) | (xx & m_nan) | (0x7f800000u & m_over));
}

// ---- glibc-compatible log1pf ------------------------------------------------
// fdlibm s_log1pf.c (Sun Microsystems, freely redistributable), the
// implementation glibc 2.35 uses: reduce 1+x = 2^k (1+f), log1p(f) via
// s = f/(2+f) and a degree-7 polynomial in s^2, with a correction term c for
// the rounding of 1+x. Matched glibc on all 2^32 inputs.
OH_DEV float ref_log1pf(float x) {
    const float ln2_hi = 6.9313812256e-01f, ln2_lo = 9.0580006145e-06f;
    const float Lp1 = 6.6666668653e-01f, Lp2 = 4.0000000596e-01f, Lp3 = 2.8571429849e-01f,
                Lp4 = 2.2222198546e-01f, Lp5 = 1.8183572590e-01f, Lp6 = 1.5313838422e-01f,
                Lp7 = 1.4798198640e-01f;
    float hfsq, f = 0.0f, c = 0.0f, s, z, R, u;
    int32_t k, hx, hu = 0, ax;
    hx = (int32_t)f2u(x);
    ax = hx & 0x7fffffff;
    k = 1;
    if (hx < 0x3ed413d7) {                         // x < 0.41422
        if (ax >= 0x3f800000) {                    // x <= -1
            if (x == -1.0f) return u2f(0xff800000u);
            return u2f(0x7fc00000u);
        }
        if (ax < 0x31000000) {                     // |x| < 2^-29
            if (ax < 0x24800000) return x;         // |x| < 2^-54
            return x - x * x * 0.5f;
        }
        if (hx > 0 || hx <= (int32_t)0xbe95f61f) { k = 0; f = x; hu = 1; }
    } else if (hx >= 0x7f800000) {
        return x + x;
    }
    if (k != 0) {
        if (hx < 0x5a000000) {
            u = 1.0f + x;
            hu = (int32_t)f2u(u);
            k = (hu >> 23) - 127;
            c = (k > 0) ? 1.0f - (u - x) : x - (u - 1.0f);
            c /= u;
        } else {
            u = x;
            hu = (int32_t)f2u(u);
            k = (hu >> 23) - 127;
            c = 0.0f;
        }
        hu &= 0x007fffff;
        if (hu < 0x3504f7) {
            u = u2f((uint32_t)hu | 0x3f800000u);
        } else {
            k += 1;
            u = u2f((uint32_t)hu | 0x3f000000u);
            hu = (0x00800000 - hu) >> 2;
        }
        f = u - 1.0f;
    }
    hfsq = 0.5f * f * f;
    if (hu == 0) {                                  // |f| < 2^-20
        if (f == 0.0f) {
            if (k == 0) return 0.0f;
            c += (float)k * ln2_lo;
            return (float)k * ln2_hi + c;
        }
        R = hfsq * (1.0f - 0.66666666666666666f * f);
        if (k == 0) return f - R;
        return (float)k * ln2_hi - ((R - ((float)k * ln2_lo + c)) - f);
    }
    s = f / (2.0f + f);
    z = s * s;
    R = z * (Lp1 + z * (Lp2 + z * (Lp3 + z * (Lp4 + z * (Lp5 + z * (Lp6 + z * Lp7))))));
    if (k == 0) return f - (hfsq - s * (hfsq + R));
    return (float)k * ln2_hi - ((hfsq - (s * (hfsq + R) + ((float)k * ln2_lo + c))) - f);
}

// reference activation helpers (src/ornith_tensor.c:117-123)
OH_DEV float ref_sigmoid(float x) { return 1.0f / (1.0f + ref_expf(-x)); }
OH_DEV float ref_silu(float x) { return x * ref_sigmoid(x); }
OH_DEV float ref_softplus(float x) { return x > 20.0f ? x : ref_log1pf(ref_expf(x)); }

// ---- wave helpers (wave64) --------------------------------------------------
// The thread index through an empty volatile asm: inside the persistent step
// kernel every operation body computes its thread-dependent addresses afresh
// instead of the compiler hoisting all of them out of the phase loop (where
// they would stay live, and spill, across every phase).
OH_DEV int tid_x() {
    int t = (int)threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}
OH_DEV int lane_id() { return tid_x() & 63; }

// lane shuffles over the whole wave (ds_bpermute), with the lane index taken
// from tid_x() so that no index computation is hoisted out of the step loop
OH_DEV int bperm(int v, int src) { return __builtin_amdgcn_ds_bpermute(src << 2, v); }
OH_DEV int shfl(int v, int src) { return bperm(v, src & 63); }
OH_DEV float shfl(float v, int src) { return __int_as_float(bperm(__float_as_int(v), src & 63)); }
OH_DEV double shfl(double v, int src) {
    const long long b = __double_as_longlong(v);
    const int lo = bperm((int)b, src & 63), hi = bperm((int)(b >> 32), src & 63);
    return __longlong_as_double(((long long)hi << 32) | (unsigned)lo);
}
template <typename T>
OH_DEV T shfl_xor(T v, int m) { return shfl(v, lane_id() ^ m); }

// DPP all-reduce within each 16-lane row (xor 1, xor 2, half-mirror, mirror:
// after each step every lane holds the combined value of a group twice as
// large). Only for order-independent operations (integer sums, max, min).
template <int CTRL>
OH_DEV int dpp_i(int v) { return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false); }
template <int CTRL>
OH_DEV float dpp_f(float v) { return __int_as_float(dpp_i<CTRL>(__float_as_int(v))); }
template <int CTRL>
OH_DEV double dpp_d(double v) {
    const long long b = __double_as_longlong(v);
    const int lo = dpp_i<CTRL>((int)b), hi = dpp_i<CTRL>((int)(b >> 32));
    return __longlong_as_double(((long long)hi << 32) | (unsigned)lo);
}
OH_DEV double readlane_d(double v, int l) {
    const long long b = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_readlane((int)b, l), hi = __builtin_amdgcn_readlane((int)(b >> 32), l);
    return __longlong_as_double(((long long)hi << 32) | (unsigned)lo);
}
// Wave-wide double sum in a fixed tree (pairs, quads, eights and sixteens of
// a row by DPP, then (row0 + row1) + (row2 + row3)); every lane gets it. Used
// for sums of squares that the reference adds sequentially in double and
// rounds to float afterwards.
// sum over each 16-lane row (every lane of the row holds it): the first four
// levels of wave_sum_d, so a 64-lane wave_sum_d equals (g0 + g1) + (g2 + g3)
// over the four rows' g
OH_DEV double row16_sum_d(double v) {
    v += dpp_d<0xB1>(v);
    v += dpp_d<0x4E>(v);
    v += dpp_d<0x141>(v);
    v += dpp_d<0x140>(v);
    return v;
}
OH_DEV double wave_sum_d(double v) {
    v += dpp_d<0xB1>(v);
    v += dpp_d<0x4E>(v);
    v += dpp_d<0x141>(v);
    v += dpp_d<0x140>(v);
    return (readlane_d(v, 0) + readlane_d(v, 16)) + (readlane_d(v, 32) + readlane_d(v, 48));
}
// float sum over the wave: DPP within each 16-lane row, then the rows
OH_DEV float wave_sum_f(float v) {
    v += __int_as_float(dpp_i<0xB1>(__float_as_int(v)));
    v += __int_as_float(dpp_i<0x4E>(__float_as_int(v)));
    v += __int_as_float(dpp_i<0x141>(__float_as_int(v)));
    v += __int_as_float(dpp_i<0x140>(__float_as_int(v)));
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return (r0 + r1) + (r2 + r3);
}
OH_DEV int wave_sum_i(int v) {
    for (int m = 32; m >= 1; m >>= 1) v += shfl_xor(v, m);
    return v;
}
OH_DEV float wave_max_f(float v) {
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, shfl_xor(v, m));
    return v;
}

OH_DEV int row16_sum_i(int v) {
    v += dpp_i<0xB1>(v); v += dpp_i<0x4E>(v); v += dpp_i<0x141>(v); v += dpp_i<0x140>(v);
    return v;
}
// wave-wide max / min: DPP within each 16-lane row, then the four rows'
// results read out as scalars (uniform in every lane)
// integer max over the wave (every lane active)
OH_DEV int wave_max_i(int v) {
    v = max(v, dpp_i<0xB1>(v)); v = max(v, dpp_i<0x4E>(v));
    v = max(v, dpp_i<0x141>(v)); v = max(v, dpp_i<0x140>(v));
    const int r0 = __builtin_amdgcn_readlane(v, 0), r1 = __builtin_amdgcn_readlane(v, 16);
    const int r2 = __builtin_amdgcn_readlane(v, 32), r3 = __builtin_amdgcn_readlane(v, 48);
    return max(max(r0, r1), max(r2, r3));
}
OH_DEV float wave_max_fast(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v)); v = fmaxf(v, dpp_f<0x4E>(v));
    v = fmaxf(v, dpp_f<0x141>(v)); v = fmaxf(v, dpp_f<0x140>(v));
    const int iv = __float_as_int(v);
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(iv, 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(iv, 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(iv, 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(iv, 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}
OH_DEV int wave_min_fast(int v) {
    v = min(v, dpp_i<0xB1>(v)); v = min(v, dpp_i<0x4E>(v));
    v = min(v, dpp_i<0x141>(v)); v = min(v, dpp_i<0x140>(v));
    const int r0 = __builtin_amdgcn_readlane(v, 0), r1 = __builtin_amdgcn_readlane(v, 16);
    const int r2 = __builtin_amdgcn_readlane(v, 32), r3 = __builtin_amdgcn_readlane(v, 48);
    return min(min(r0, r1), min(r2, r3));
}

// signed 8-bit dot of four packed bytes, accumulated into c (exact integers)
OH_DEV int dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

// ---- data shared between workgroups of one launch ----------------------------
// The L2 caches of the XCDs are not coherent with each other, and a CU's L1 is
// not coherent with other CUs. Values that one workgroup writes and another
// reads later in the same launch (the persistent token-step kernel, whose
// phases are separated by grid barriers) therefore use device-scope accesses:
// relaxed device-scope atomic loads and stores, i.e. ordinary loads and stores
// with the sc1 scope bit. A device-scope store is acknowledged once it is
// visible at device scope, and a device-scope load does not return a
// non-coherent cached copy. The grid barrier waits for the stores' completion
// before it signals. Weights and other data that no launch writes use plain
// accesses.
#define OH_GLOBAL __attribute__((address_space(1)))
template <typename T>
OH_DEV T ldc(const T *p) {
    return __hip_atomic_load((const OH_GLOBAL T *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
OH_DEV void stc(T *p, T v) { __hip_atomic_store((OH_GLOBAL T *)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
// Plain loads and stores of global memory through pointers taken from an
// operation descriptor: the explicit address space makes them global_load /
// global_store (a pointer read from memory would otherwise be accessed with
// flat instructions, which also count against the LDS wait counter).
template <typename T>
OH_DEV T ldg(const T *p) { return *(const OH_GLOBAL T *)p; }
template <typename T>
OH_DEV void stg(T *p, const T &v) { *(OH_GLOBAL T *)p = v; }
// HIP's vector types copy through a generic reference: load and store their
// raw vector form instead
typedef unsigned oh_u4 __attribute__((ext_vector_type(4)));
typedef float oh_f4 __attribute__((ext_vector_type(4)));
typedef float oh_f2 __attribute__((ext_vector_type(2)));
template <>
OH_DEV uint4 ldg(const uint4 *p) {
    const oh_u4 v = *(const OH_GLOBAL oh_u4 *)p;
    return make_uint4(v.x, v.y, v.z, v.w);
}
template <>
OH_DEV int4 ldg(const int4 *p) {
    const oh_u4 v = *(const OH_GLOBAL oh_u4 *)p;
    return make_int4((int)v.x, (int)v.y, (int)v.z, (int)v.w);
}
template <>
OH_DEV float4 ldg(const float4 *p) {
    const oh_f4 v = *(const OH_GLOBAL oh_f4 *)p;
    return make_float4(v.x, v.y, v.z, v.w);
}
template <>
OH_DEV float2 ldg(const float2 *p) {
    const oh_f2 v = *(const OH_GLOBAL oh_f2 *)p;
    return make_float2(v.x, v.y);
}
typedef unsigned oh_u2 __attribute__((ext_vector_type(2)));
template <>
OH_DEV uint2 ldg(const uint2 *p) {
    const oh_u2 v = *(const OH_GLOBAL oh_u2 *)p;
    return make_uint2(v.x, v.y);
}
template <>
OH_DEV void stg(float4 *p, const float4 &v) {
    oh_f4 r;
    r.x = v.x; r.y = v.y; r.z = v.z; r.w = v.w;
    *(OH_GLOBAL oh_f4 *)p = r;
}
OH_DEV float4 ldc4(const float4 *p) {
    const double *q = (const double *)p;
    const double a = ldc(q), b = ldc(q + 1);
    const uint64_t ua = (uint64_t)__double_as_longlong(a), ub = (uint64_t)__double_as_longlong(b);
    return make_float4(u2f((uint32_t)ua), u2f((uint32_t)(ua >> 32)), u2f((uint32_t)ub), u2f((uint32_t)(ub >> 32)));
}
OH_DEV int4 ldc4(const int4 *p) {
    const float4 v = ldc4((const float4 *)p);
    return make_int4((int)f2u(v.x), (int)f2u(v.y), (int)f2u(v.z), (int)f2u(v.w));
}
OH_DEV void stc4(float4 *p, const float4 v) {
    double *q = (double *)p;
    stc(q, __longlong_as_double((long long)(((uint64_t)f2u(v.y) << 32) | f2u(v.x))));
    stc(q + 1, __longlong_as_double((long long)(((uint64_t)f2u(v.w) << 32) | f2u(v.z))));
}

// A load of another launch's (or phase's) output: device-scope inside the
// persistent kernels (G: the phases of one launch), a plain load in a
// stand-alone kernel, whose start is ordered after the earlier launches'
// writes (a plain load may then hit in this XCD's L2, which a device-scope
// one skips).
template <bool G, typename T>
OH_DEV T ldw(const T *p) {
    if constexpr (G) return ldc(p);
    else return ldg(p);
}
template <bool G>
OH_DEV float4 ldw4(const float4 *p) {
    if constexpr (G) return ldc4(p);
    else return ldg(p);
}
template <bool G>
OH_DEV int4 ldw4(const int4 *p) {
    if constexpr (G) return ldc4(p);
    else return ldg(p);
}

// LDS ordering between the lanes of one wave (no workgroup barrier): waits for
// the wave's LDS operations and keeps the compiler from moving LDS accesses
// across it.
OH_DEV void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// A no-op grid wait: the bodies of the token-step operations call wait()
// before their first read of another phase's output; a standalone kernel has
// nothing to wait for (the kernel boundary orders it).
struct NoWait {
    static constexpr bool kGrid = false;
    OH_DEV bool wait() { return true; }
};
