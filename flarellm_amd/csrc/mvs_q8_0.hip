// Q8_0 streaming matvecs (Q8 and f32 input) and the Q8_0 gate/up kernel.
#include "launch.h"

namespace fl {

// (RXX false matches either way: a plan with no register variant falls back)
#define CX(FMT, F32IN, RR, SS, RXX)                                                                      \
    if (p.r == RR && p.su == SS && (rx || !RXX)) {                                                          \
        hipLaunchKernelGGL((k_mvs<FMT, F32IN, RR, SS, RXX>),                                               \
                           dim3(resident_grid(k_mvs<FMT, F32IN, RR, SS, RXX>, kMvsThreads, p.lds, p.grid)), \
                           dim3(kMvsThreads), p.lds, st, a);                                          \
        return hipSuccess;                                                                               \
    }
#define C(FMT, F32IN, RR, SS) CX(FMT, F32IN, RR, SS, false)

// Norm prologues whose whole row fits one unit keep the quantized activation
// in registers (RegX8, no workgroup barrier).
static bool use_regx(const MvsPlan &p, const MvsArgs &a) {
    static const bool off = getenv("FLARE_NO_REGX") != nullptr;
    return !off && (a.pro == PRO_NORMQ0 || a.pro == PRO_NORMQ1) && mvs_steps(F_Q8_0, a.W.cols) <= p.su;
}

hipError_t launch_mvs_q8_0(bool f32in, const MvsPlan &p, hipStream_t st, const MvsArgs &a) {
    const bool rx = !f32in && use_regx(p, a);
    if (!f32in) {
        if (rx) {
            CX(F_Q8_0, false, 4, 1, true) CX(F_Q8_0, false, 4, 2, true) CX(F_Q8_0, false, 2, 1, true)
            CX(F_Q8_0, false, 2, 2, true) CX(F_Q8_0, false, 2, 4, true)
        }
    }
    if (f32in) {
        C(F_Q8_0, true, 2, 1) C(F_Q8_0, true, 4, 1) C(F_Q8_0, true, 2, 2) C(F_Q8_0, true, 4, 2)
    } else {
        C(F_Q8_0, false, 4, 1) C(F_Q8_0, false, 4, 2) C(F_Q8_0, false, 2, 1) C(F_Q8_0, false, 2, 2) C(F_Q8_0, false, 2, 4) C(F_Q8_0, false, 1, 4) C(F_Q8_0, false, 1, 8)
    }
    return hipErrorNotSupported;
}
#undef C
#undef CX

hipError_t launch_mvs_gu_q8_0(const MvsPlan &p, hipStream_t st, const MvsArgs &a) {
    const bool rx = use_regx(p, a);
#define GX(SS, NW, RXX)                                                                              \
    if (p.su == SS && p.r == NW && (rx || !RXX)) {                                                      \
        hipLaunchKernelGGL((k_mvs_gu<F_Q8_0, SS, NW, RXX>),                                        \
                           dim3(resident_grid(k_mvs_gu<F_Q8_0, SS, NW, RXX>, NW * 64, p.lds, p.grid)),     \
                           dim3(NW * 64), p.lds, st, a);                                         \
        return hipSuccess;                                                                        \
    }
#define G(SS, NW) GX(SS, NW, false)
    if (rx) { GX(1, 4, true) GX(2, 4, true) GX(1, 8, true) GX(2, 8, true) }
    G(1, 8) G(2, 8) G(1, 4) G(2, 4) G(1, 16) G(2, 16) G(1, 2) G(2, 2)
#undef G
#undef GX
    return hipErrorNotSupported;
}

}  // namespace fl
