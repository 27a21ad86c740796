// Q4_K streaming matvec (Q8 input) and the Q4_K gate/up kernel.
#include "launch.h"

namespace fl {

#define C(FMT, F32IN, RR, SS)                                                                         \
    if (p.r == RR && p.su == SS) {                                                                    \
        hipLaunchKernelGGL((k_mvs<FMT, F32IN, RR, SS>),                                                  \
                           dim3(resident_grid(k_mvs<FMT, F32IN, RR, SS>, kMvsThreads, p.lds, p.grid)), \
                           dim3(kMvsThreads), p.lds, st, a);                                       \
        return hipSuccess;                                                                            \
    }

// Reference-order (SEQ) instantiations of the plans mvs_plan picks.
#define SX(RR, SS)                                                                                      \
    if (p.r == RR && p.su == SS) {                                                                      \
        const size_t lds = align16(p.lds) + seq_lds_bytes(kMvsThreads / 64, RR, SS);                   \
        hipLaunchKernelGGL((k_mvs<F_Q4K, false, RR, SS, 0, true>),                                     \
                           dim3(resident_grid(k_mvs<F_Q4K, false, RR, SS, 0, true>, kMvsThreads, lds, p.grid)), \
                           dim3(kMvsThreads), lds, st, a);                                              \
        return hipSuccess;                                                                              \
    }

hipError_t launch_mvs_q4k(const MvsPlan &p, hipStream_t st, const MvsArgs &a) {
    if (a.seq) {
        SX(4, 1) SX(2, 1) SX(2, 2) SX(1, 2)
        return hipErrorNotSupported;
    }
    // pre-quantized input whose row fits one unit: the lane's activation runs
    // in registers (RegX4L, no LDS staging or workgroup barrier)
    static const bool noregx = measure_env("FLARE_NO_REGX") != nullptr;
    if (!noregx && a.pro == PRO_LOADQ && mvs_steps(F_Q4K, a.W.cols) <= p.su) {
#define CR(RR, SS)                                                                                        \
    if (p.r == RR && p.su == SS) {                                                                        \
        hipLaunchKernelGGL((k_mvs<F_Q4K, false, RR, SS, 2>),                                               \
                           dim3(resident_grid(k_mvs<F_Q4K, false, RR, SS, 2>, kMvsThreads, p.lds, p.grid)), \
                           dim3(kMvsThreads), p.lds, st, a);                                            \
        return hipSuccess;                                                                                \
    }
        CR(1, 2) CR(2, 2) CR(4, 2)
#undef CR
    }
    C(F_Q4K, false, 4, 1) C(F_Q4K, false, 2, 1) C(F_Q4K, false, 2, 2) C(F_Q4K, false, 1, 2) C(F_Q4K, false, 1, 4)
    return hipErrorNotSupported;
}
#undef C
#undef SX

hipError_t launch_mvs_gu_q4k(const MvsPlan &p, hipStream_t st, const MvsArgs &a) {
    if (a.seq) {
#define GS(SS, NW)                                                                                    \
    if (p.su == SS && p.r == NW) {                                                                    \
        const size_t lds = align16(p.lds) + seq_lds_bytes(NW, 4, SS);                                 \
        hipLaunchKernelGGL((k_mvs_gu<F_Q4K, SS, NW, 0, true>),                                       \
                           dim3(resident_grid(k_mvs_gu<F_Q4K, SS, NW, 0, true>, NW * 64, lds, p.grid)), \
                           dim3(NW * 64), lds, st, a);                                                \
        return hipSuccess;                                                                            \
    }
        GS(1, 8) GS(2, 8)
#undef GS
        return hipErrorNotSupported;
    }
#define G(SS, NW)                                                                               \
    if (p.su == SS && p.r == NW) {                                                              \
        hipLaunchKernelGGL((k_mvs_gu<F_Q4K, SS, NW>),                                         \
                           dim3(resident_grid(k_mvs_gu<F_Q4K, SS, NW>, NW * 64, p.lds, p.grid)),      \
                           dim3(NW * 64), p.lds, st, a);                                        \
        return hipSuccess;                                                                      \
    }
    G(1, 8) G(1, 4) G(2, 8) G(2, 4) G(1, 16) G(2, 16) G(1, 2) G(2, 2)
#undef G
    return hipErrorNotSupported;
}

}  // namespace fl
