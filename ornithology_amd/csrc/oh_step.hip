// oh_step.hip - the persistent token-step kernel: one cooperative launch runs
// every operation of a decode step (a program of oh_op descriptors) as phases
// separated by grid barriers, instead of one kernel launch per operation.
// Included into oh_kernels.hip after the operation bodies.
//
// Grid barrier. Every phase i has OH_STEP_NCTR arrival counters, one per
// 64-byte line; workgroup b adds 1 to counter b % OH_STEP_NCTR when it is done
// with phase i (after its stores have completed). The counters only grow: in
// the e-th launch of a program (e from 0, kept in io[epoch slot]) phase i is
// complete when every counter of phase i holds (e+1) * gridDim/OH_STEP_NCTR.
// Lanes 0..31 of wave 0 poll the 32 counters with device-scope loads.
//
// A workgroup that has no virtual block in a phase does not wait for the
// previous phase: it arrives at once and goes on to the next phase, where it
// requests its first weights before it waits. Workgroup 0 always has virtual
// block 0 of every phase (phases without blocks are not emitted) and always
// waits, so phase i complete implies phase i-1 complete.
//
// Every wait is bounded: after about a second, or as soon as another
// workgroup has given up (io[OH_IO_ERR] != 0), the workgroup records the
// failure and leaves the kernel, so the grid always drains; the host reports
// the error. Cooperative launch guarantees that all workgroups are resident.

namespace {

constexpr int kSpinMax = 1 << 20;

struct GridWait {
    static constexpr bool kGrid = true;
    const unsigned *ctr;        // the previous phase's counters, null for phase 0
    unsigned target;
    int32_t *err;
    uint64_t *ts;               // block 0 records when the wait was passed (or null)
    bool pending, dead;
    OH_DEV bool wait() {
        if (!pending) return !dead;
        pending = false;
        __shared__ int s_fail;
        if (tid_x() < OH_STEP_NCTR) {
            const unsigned *c = ctr + tid_x() * OH_STEP_CSTRIDE;
            int n = 0;
            bool fail = false;
            while ((int)(ldc(c) - target) < 0) {
                __builtin_amdgcn_s_sleep(1);
                if ((++n & 255) == 0 && (ldc(err) != 0 || n > kSpinMax)) {
                    fail = true;
                    break;
                }
            }
            const bool any = __ballot(fail) != 0;
            if (threadIdx.x == 0) {
                s_fail = any ? 1 : 0;
                if (any) stc(err, (int32_t)1);
                if (ts && blockIdx.x == 0) stg(ts, (uint64_t)__builtin_amdgcn_s_memrealtime());
            }
        }
        __syncthreads();
        dead = s_fail != 0;
        return !dead;
    }
};

// End of a phase for this workgroup: every wave waits for its own memory
// operations (device-scope stores are complete once acknowledged), then one
// thread adds the arrival.
OH_DEV void grid_arrive(unsigned *ctr) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0)
        __hip_atomic_fetch_add(ctr + (blockIdx.x % OH_STEP_NCTR) * OH_STEP_CSTRIDE, 1u, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
}

// Values passed to a non-inlined function arrive in vector registers; these
// put them back in scalar registers. The descriptor pointer becomes a
// constant-address-space pointer: its fields are read with scalar loads and
// the pointers stored in it are known to be global.
OH_DEV int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }
template <typename T>
OH_DEV T *uni_ptr(T *p) {
    const uint64_t a = (uint64_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
    return (T *)(((uint64_t)hi << 32) | lo);
}
template <typename T>
OH_DEV const T *uni_const(const T *p) {
    return (const T *)(const __attribute__((address_space(4))) T *)(uintptr_t)uni_ptr(p);
}

template <class W>
OH_DEV void run_vb(const oh_op &op, int vb, int pos, W &w) {
    extern __shared__ __align__(16) uint8_t smem[];
    switch (op.kind) {
    case OH_OP_MV:
        if (op.tk == OH_Q4_K) mv_body<OH_Q4_K>(op.u.mv, vb, w);
        else if (op.tk == OH_Q6_K) mv_body<OH_Q6_K>(op.u.mv, vb, w);
        else if (op.tk == OH_Q8_0) mv_body<OH_Q8_0>(op.u.mv, vb, w);
        else mv_body<-1>(op.u.mv, vb, w);
        break;
    case OH_OP_MV_DOWN:
        if (op.u.down.type == OH_Q4_K) down_split<OH_Q4_K>(op.u.down, vb, w);
        else if (op.u.down.type == OH_Q6_K) down_split<OH_Q6_K>(op.u.down, vb, w);
        else down_split<OH_Q8_0>(op.u.down, vb, w);
        break;
    case OH_OP_EMBED: embed_body(op.u.embed, vb, pos, w); break;
    case OH_OP_DELTA:
        if (op.u.delta.dk == 128) {
            if (op.u.delta.K <= 4) delta_body<128, 4>(op.u.delta, vb, pos, (float *)smem, w);
            else delta_body<128, 8>(op.u.delta, vb, pos, (float *)smem, w);
        } else {
            if (op.u.delta.K <= 4) delta_body<64, 4>(op.u.delta, vb, pos, (float *)smem, w);
            else delta_body<64, 8>(op.u.delta, vb, pos, (float *)smem, w);
        }
        break;
    case OH_OP_DELTA16:
        if (op.u.delta.dk == 128) {
            if (op.u.delta.K <= 4) delta16_body<128, 4>(op.u.delta, vb, pos, (float *)smem, w);
            else delta16_body<128, 8>(op.u.delta, vb, pos, (float *)smem, w);
        } else {
            if (op.u.delta.K <= 4) delta16_body<64, 4>(op.u.delta, vb, pos, (float *)smem, w);
            else delta16_body<64, 8>(op.u.delta, vb, pos, (float *)smem, w);
        }
        break;
    case OH_OP_ATTN_PREP: prep_body(op.u.prep, vb, pos, w); break;
    case OH_OP_ATTN_MAIN: attn_main_body(op.u.attn, vb, pos, w); break;
    case OH_OP_ATTN_COMBINE: combine_body(op.u.attn, vb, pos, w, exact_lim(op.u.attn.exact_max, op.u.attn.hd)); break;
    case OH_OP_MOE_COMBINE: moe_combine_body(op.u.comb, vb, w); break;
    case OH_OP_ARGMAX1: argmax1_body(op.u.am, vb, w); break;
    case OH_OP_ARGMAX2: argmax2_body(op.u.am, pos, w); break;
    default: w.wait(); break;
    }
}

} // namespace

// prog: nops operations in device memory; ctrs: nops * OH_STEP_NCTR *
// OH_STEP_CSTRIDE counters of this program; epoch_slot: the io word counting
// this program's launches; advance: write io[OH_IO_POS] = pos + 1 at the end
// (the body program). ts (optional, nops + 1 entries): block 0's real-time
// clock at the start, after each barrier, and at the end.
extern "C" __global__ void __launch_bounds__(256, 2)
oh_k_step(const oh_op *__restrict__ prog, int nops, int32_t *io, unsigned *ctrs, int epoch_slot, int advance,
          uint64_t *ts) {
    const int pos = io[OH_IO_POS];
    const unsigned epoch = (unsigned)io[epoch_slot];
    const unsigned target = (epoch + 1u) * (gridDim.x / OH_STEP_NCTR);
    int32_t *err = io + OH_IO_ERR;
    const bool rec = ts && blockIdx.x == 0 && threadIdx.x == 0;
    if (rec) ts[0] = __builtin_amdgcn_s_memrealtime();
    for (int i = 0; i < nops; i++) {
        // the descriptor through a uniform constant-address-space pointer
        // (scalar loads; the pointers it holds are global); the position
        // through an opaque copy, so nothing derived from it is hoisted out
        // of this loop
        const oh_op &op = *uni_const(prog + i);
        int posi = pos;
        asm volatile("" : "+s"(posi));
        GridWait w{i > 0 ? ctrs + (size_t)(i - 1) * OH_STEP_NCTR * OH_STEP_CSTRIDE : nullptr, target, err,
                   ts ? ts + i : nullptr, i > 0, false};
        for (int vb = (int)blockIdx.x; vb < op.nvb; vb += (int)gridDim.x) {
            run_vb(op, vb, posi, w);
            if (w.dead) return;
            __syncthreads();                  // LDS is reused by the next virtual block
        }
        if (blockIdx.x == 0 && !w.wait()) return;
        if (i + 1 < nops) grid_arrive(ctrs + (size_t)i * OH_STEP_NCTR * OH_STEP_CSTRIDE);
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        if (rec) ts[nops] = __builtin_amdgcn_s_memrealtime();
        if (advance) io[OH_IO_POS] = pos + 1;
        io[epoch_slot] = (int32_t)(epoch + 1u);
    }
}
