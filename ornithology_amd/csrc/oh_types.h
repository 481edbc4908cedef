// oh_types.h - host/device shared descriptors of the HIP engine.
//
// Weights live in HBM in a "plane" layout derived from the GGUF blocks. For a
// tensor of R rows and nb blocks per row (block = 256 elements, or 32 for
// Q8_0 handled as 8 sub-blocks of a 256-element super-block), block b = r*nb+i
// is split into up to three planes so that every wave load is 16-byte aligned
// and contiguous across lanes:
//   Q4_K    A: qs[128]            B: d,dmin,scales[12] (16 B)
//   Q6_K    A: ql[128] qh[64]     B: scales[16]          C: d (f16)
//   Q8_0    A: 8 x qs[32]         B: 8 x d (f16)
//   IQ2_XXS A: qs[64]                                     C: d (f16)
//   F32/F16/BF16: A holds the raw row-major values.
// The byte count equals the GGUF byte count; decoding a plane-layout block
// gives the same floats as decoding the GGUF block.
//
// Q8_K activations use planes as well: qs[nb*256] int8, d[nb] f32,
// bsums[nb*16] int16 (the 292-byte oq8k_block fields, split).
#pragma once
#include <stdint.h>

#if defined(__HIPCC__)
#define OH_HD __host__ __device__
#else
#define OH_HD
#endif

enum {
    OH_F32 = 0, OH_F16 = 1, OH_Q8_0 = 8, OH_Q4_K = 12, OH_Q6_K = 14,
    OH_IQ2_XXS = 16, OH_BF16 = 30
};

// plane bytes per 256-element super-block
OH_HD static inline int oh_plane_a(uint32_t t) {
    switch (t) { case OH_Q4_K: return 128; case OH_Q6_K: return 192; case OH_Q8_0: return 256;
                 case OH_IQ2_XXS: return 64; default: return 0; }
}
OH_HD static inline int oh_plane_b(uint32_t t) {
    switch (t) { case OH_Q4_K: case OH_Q6_K: case OH_Q8_0: return 16; default: return 0; }
}
OH_HD static inline int oh_plane_c(uint32_t t) {
    switch (t) { case OH_Q6_K: case OH_IQ2_XXS: return 2; default: return 0; }
}
OH_HD static inline int oh_is_quant(uint32_t t) {
    return t == OH_Q4_K || t == OH_Q6_K || t == OH_Q8_0 || t == OH_IQ2_XXS;
}
// integer Q8_K path exists (reference qdot_can, src/ornith_qdot.c:218-228)
OH_HD static inline int oh_qdot_can(uint32_t t, int64_t in) {
    return in % 256 == 0 && (t == OH_Q4_K || t == OH_Q6_K || t == OH_Q8_0);
}

// One matvec segment of a multi-segment launch.
typedef struct {
    const uint8_t *A, *B, *C;      // weight planes (expert 0 for a stacked tensor)
    const int8_t *xqs;             // Q8_K activation planes
    const float *xd;
    const int16_t *xbs;
    const float *xf;               // f32 activation (f32/IQ2_XXS fallback rows)
    float *y;                      // output, row o -> y[o]
    const int32_t *eidx;           // gathered expert: rows += eidx[eslot]*rows
    int type, nb, in, rows, mode;  // mode 0: y = dot, 1: y += dot
    int eslot;
    int units;                     // wave work units in this segment
    int block0;                    // first block of the segment in the launch
} oh_mvseg;

#define OH_MAX_SEGS 24
typedef struct {
    oh_mvseg s[OH_MAX_SEGS];
    int n;
    int total_blocks;
} oh_mvlaunch;
