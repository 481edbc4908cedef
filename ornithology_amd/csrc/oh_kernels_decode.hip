// oh_kernels_decode.hip - the translation unit of the persistent tagged-word
// decode kernel (oh_decode.hip) and its launchers. It needs only the operation
// bodies, so the stand-alone kernels of oh_mv.hip and oh_layers.hip are left out.
#define OH_BODIES_ONLY
#include "oh_mv.hip"
#include "oh_layers.hip"
#include "oh_decode.hip"
#include "oh_launch.h"

extern "C" {

hipError_t oh_decode_blocks_per_cu(int lds_bytes, int *blocks) {
    hipError_t e = hipFuncSetAttribute((const void *)oh_k_decode, hipFuncAttributeMaxDynamicSharedMemorySize, lds_bytes);
    if (e != hipSuccess) return e;
    return hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks, (const void *)oh_k_decode, 256, (size_t)lds_bytes);
}

hipError_t oh_launch_decode(const oh_dop *prog, int nops, int32_t *io, int advance, int grid, int lds_bytes,
                            hipStream_t st, uint64_t *ts, int prof_op, uint64_t *ts2) {
    void *args[] = {(void *)&prog, (void *)&nops, (void *)&io, (void *)&advance, (void *)&ts, (void *)&prof_op,
                    (void *)&ts2};
    return hipLaunchCooperativeKernel((const void *)oh_k_decode, dim3(grid), dim3(256), args, (size_t)lds_bytes, st);
}

} // extern "C"
