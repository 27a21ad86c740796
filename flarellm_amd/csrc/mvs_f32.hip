// f32-input streaming matvecs over Q6_K and f32 weights (logits path).
#include "launch.h"

namespace fl {

#define C(FMT, F32IN, RR, SS)                                                                         \
    if (p.r == RR && p.su == SS) {                                                                    \
        hipLaunchKernelGGL((k_mvs<FMT, F32IN, RR, SS>),                                                  \
                           dim3(resident_grid(k_mvs<FMT, F32IN, RR, SS>, kMvsThreads, p.lds, p.grid)), \
                           dim3(kMvsThreads), p.lds, st, a);                                       \
        return hipSuccess;                                                                            \
    }

hipError_t launch_mvs_f32(int fmt, const MvsPlan &p, hipStream_t st, const MvsArgs &a) {
    if (fmt == F_Q6K) {
        C(F_Q6K, true, 4, 1) C(F_Q6K, true, 2, 1) C(F_Q6K, true, 2, 2)
#ifdef FLARE_MEASURE
        C(F_Q6K, true, 1, 1) C(F_Q6K, true, 1, 2) C(F_Q6K, true, 4, 2) C(F_Q6K, true, 8, 1)
#endif
    } else if (fmt == F_F32) {
        C(F_F32, true, 4, 1) C(F_F32, true, 4, 2) C(F_F32, true, 2, 1) C(F_F32, true, 2, 2) C(F_F32, true, 2, 4)
    }
    return hipErrorNotSupported;
}
#undef C

}  // namespace fl
