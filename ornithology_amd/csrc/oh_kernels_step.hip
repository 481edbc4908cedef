// oh_kernels_step.hip - the translation unit of the persistent token-step
// kernel (oh_step.hip) and its launchers. It needs only the operation bodies,
// so the stand-alone kernels of oh_mv.hip and oh_layers.hip are left out.
#define OH_BODIES_ONLY
#include "oh_mv.hip"
#include "oh_layers.hip"
#include "oh_step.hip"
#include "oh_launch.h"

extern "C" {

hipError_t oh_step_blocks_per_cu(int lds_bytes, int *blocks) {
    hipError_t e = hipFuncSetAttribute((const void *)oh_k_step, hipFuncAttributeMaxDynamicSharedMemorySize, lds_bytes);
    if (e != hipSuccess) return e;
    return hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks, (const void *)oh_k_step, 256, (size_t)lds_bytes);
}

hipError_t oh_launch_step(const oh_op *prog, int nops, int32_t *io, unsigned *ctrs, int epoch_slot, int advance,
                          uint64_t *ts, int grid, int lds_bytes, hipStream_t st) {
    void *args[] = {(void *)&prog, (void *)&nops, (void *)&io, (void *)&ctrs, (void *)&epoch_slot,
                    (void *)&advance, (void *)&ts};
    return hipLaunchCooperativeKernel((const void *)oh_k_step, dim3(grid), dim3(256), args, (size_t)lds_bytes, st);
}

} // extern "C"
