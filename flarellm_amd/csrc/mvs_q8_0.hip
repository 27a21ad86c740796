// Q8_0 streaming matvecs (Q8 and f32 input) and the Q8_0 gate/up kernel.
#include "launch.h"

namespace fl {

#define C(FMT, F32IN, RR, SS)                                                                         \
    if (p.r == RR && p.su == SS) {                                                                    \
        hipLaunchKernelGGL((k_mvs<FMT, F32IN, RR, SS>),                                                  \
                           dim3(resident_grid(k_mvs<FMT, F32IN, RR, SS>, kMvsThreads, p.lds, p.grid)), \
                           dim3(kMvsThreads), p.lds, st, a);                                       \
        return hipSuccess;                                                                            \
    }

hipError_t launch_mvs_q8_0(bool f32in, const MvsPlan &p, hipStream_t st, const MvsArgs &a) {
    if (f32in) {
        C(F_Q8_0, true, 2, 1) C(F_Q8_0, true, 4, 1) C(F_Q8_0, true, 2, 2) C(F_Q8_0, true, 4, 2)
    } else {
        C(F_Q8_0, false, 4, 1) C(F_Q8_0, false, 4, 2) C(F_Q8_0, false, 2, 1) C(F_Q8_0, false, 2, 2) C(F_Q8_0, false, 2, 4) C(F_Q8_0, false, 1, 4) C(F_Q8_0, false, 1, 8)
    }
    return hipErrorNotSupported;
}
#undef C

hipError_t launch_mvs_gu_q8_0(const MvsPlan &p, hipStream_t st, const MvsArgs &a) {
#define G(SS, NW)                                                                                \
    if (p.su == SS && p.r == NW) {                                                               \
        hipLaunchKernelGGL((k_mvs_gu<F_Q8_0, SS, NW>),                                         \
                           dim3(resident_grid(k_mvs_gu<F_Q8_0, SS, NW>, NW * 64, p.lds, p.grid)),      \
                           dim3(NW * 64), p.lds, st, a);                                        \
        return hipSuccess;                                                                       \
    }
    G(1, 8) G(2, 8) G(1, 4) G(2, 4) G(1, 16) G(2, 16) G(1, 2) G(2, 2)
#undef G
    return hipErrorNotSupported;
}

}  // namespace fl
