// Q8_0 streaming matvecs (Q8 and f32 input) and the Q8_0 gate/up kernel.
#include "launch.h"

namespace fl {

// (RXX false matches either way: a plan with no register variant falls back)
#define CX(FMT, F32IN, RR, SS, RXX)                                                                      \
    if (p.r == RR && p.su == SS && (rx == RXX || !RXX)) {                                                          \
        hipLaunchKernelGGL((k_mvs<FMT, F32IN, RR, SS, RXX>),                                               \
                           dim3(resident_grid(k_mvs<FMT, F32IN, RR, SS, RXX>, kMvsThreads, p.lds, p.grid)), \
                           dim3(kMvsThreads), p.lds, st, a);                                          \
        return hipSuccess;                                                                               \
    }
#define C(FMT, F32IN, RR, SS) CX(FMT, F32IN, RR, SS, 0)

// Norm prologues whose whole row fits one unit keep the quantized activation
// in registers (RegX8, no workgroup barrier).
// 1: norm prologue (RegX8), 2: pre-quantized input (RegX8L), 0: LDS staging
static int use_regx(const MvsPlan &p, const MvsArgs &a) {
    static const bool off = measure_env("FLARE_NO_REGX") != nullptr;
    if (off || mvs_steps(F_Q8_0, a.W.cols) > p.su) return 0;
    if (a.pro == PRO_NORMQ0 || a.pro == PRO_NORMQ1) return 1;
    return a.pro == PRO_LOADQ ? 2 : 0;
}

// Reference-order (SEQ) instantiations of the plans mvs_plan picks.
#define SX(RR, SS, RXX)                                                                                  \
    if (p.r == RR && p.su == SS && rx == RXX) {                                                          \
        const size_t lds = align16(p.lds) + seq_lds_bytes(kMvsThreads / 64, RR, SS);                    \
        hipLaunchKernelGGL((k_mvs<F_Q8_0, false, RR, SS, RXX, true>),                                   \
                           dim3(resident_grid(k_mvs<F_Q8_0, false, RR, SS, RXX, true>, kMvsThreads, lds, p.grid)), \
                           dim3(kMvsThreads), lds, st, a);                                               \
        return hipSuccess;                                                                               \
    }

hipError_t launch_mvs_q8_0(bool f32in, const MvsPlan &p, hipStream_t st, const MvsArgs &a) {
    const int rx = f32in ? 0 : use_regx(p, a);
    if (a.seq) {
        if (f32in) return hipErrorNotSupported;
        SX(4, 1, 1) SX(4, 2, 1) SX(2, 1, 1) SX(2, 2, 1) SX(2, 4, 1)
        SX(4, 1, 2) SX(4, 2, 2) SX(2, 1, 2) SX(2, 2, 2) SX(1, 4, 2) SX(1, 8, 2)
        SX(4, 1, 0) SX(4, 2, 0) SX(2, 1, 0) SX(2, 2, 0) SX(1, 4, 0)
        return hipErrorNotSupported;
    }
    if (!f32in) {
        if (rx == 1) {
            CX(F_Q8_0, false, 4, 1, 1) CX(F_Q8_0, false, 4, 2, 1) CX(F_Q8_0, false, 2, 1, 1)
            CX(F_Q8_0, false, 2, 2, 1) CX(F_Q8_0, false, 2, 4, 1)
        } else if (rx == 2) {
            CX(F_Q8_0, false, 4, 1, 2) CX(F_Q8_0, false, 4, 2, 2) CX(F_Q8_0, false, 2, 2, 2)
            CX(F_Q8_0, false, 1, 4, 2) CX(F_Q8_0, false, 1, 8, 2)
        }
    }
    if (f32in) {
        C(F_Q8_0, true, 2, 1) C(F_Q8_0, true, 4, 1) C(F_Q8_0, true, 2, 2) C(F_Q8_0, true, 4, 2)
#ifdef FLARE_MEASURE
        C(F_Q8_0, true, 1, 2) C(F_Q8_0, true, 1, 4) C(F_Q8_0, true, 2, 4)
#endif
    } else {
        C(F_Q8_0, false, 4, 1) C(F_Q8_0, false, 4, 2) C(F_Q8_0, false, 2, 1) C(F_Q8_0, false, 2, 2) C(F_Q8_0, false, 2, 4) C(F_Q8_0, false, 1, 4) C(F_Q8_0, false, 1, 8)
    }
    return hipErrorNotSupported;
}
#undef C
#undef CX
#undef SX

hipError_t launch_mvs_gu_q8_0(const MvsPlan &p, hipStream_t st, const MvsArgs &a) {
    const int rx = use_regx(p, a);
    if (a.seq) {
#define GS(SS, NW, RXX)                                                                               \
    if (p.su == SS && p.r == NW && rx == RXX) {                                                       \
        const size_t lds = align16(p.lds) + seq_lds_bytes(NW, 4, SS);                                 \
        hipLaunchKernelGGL((k_mvs_gu<F_Q8_0, SS, NW, RXX, true>),                                    \
                           dim3(resident_grid(k_mvs_gu<F_Q8_0, SS, NW, RXX, true>, NW * 64, lds, p.grid)), \
                           dim3(NW * 64), lds, st, a);                                                \
        return hipSuccess;                                                                            \
    }
        GS(1, 8, 1) GS(2, 8, 1) GS(1, 8, 0) GS(2, 8, 0)
#undef GS
        return hipErrorNotSupported;
    }
#define GX(SS, NW, RXX)                                                                              \
    if (p.su == SS && p.r == NW && (rx == RXX || !RXX)) {                                                      \
        hipLaunchKernelGGL((k_mvs_gu<F_Q8_0, SS, NW, RXX>),                                        \
                           dim3(resident_grid(k_mvs_gu<F_Q8_0, SS, NW, RXX>, NW * 64, p.lds, p.grid)),     \
                           dim3(NW * 64), p.lds, st, a);                                         \
        return hipSuccess;                                                                        \
    }
#define G(SS, NW) GX(SS, NW, 0)
    if (rx == 1) { GX(1, 4, 1) GX(2, 4, 1) GX(1, 8, 1) GX(2, 8, 1) }
    G(1, 8) G(2, 8) G(1, 4) G(2, 4) G(1, 16) G(2, 16) G(1, 2) G(2, 2)
#undef G
#undef GX
    return hipErrorNotSupported;
}

}  // namespace fl
