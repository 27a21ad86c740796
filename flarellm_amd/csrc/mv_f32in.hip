// f32-input matvecs (logits path): Q8_0 (tied embedding), Q6_K, F32.
#include "launch.h"

namespace fl {

template <int FMT>
static hipError_t launch_f32in_fmt(const MvPlan &p, hipStream_t st, const F32Args &a) {
#define C(L, UU, RR)                                                                                 \
    if (p.lpr == L && p.u == UU && p.r == RR) {                                                      \
        hipLaunchKernelGGL((k_mv_f32in<FMT, L, UU, RR>), dim3(p.grid), dim3(kThreads), p.lds, st, a); \
        return hipSuccess;                                                                           \
    }
#define CL(L) C(L, 1, 8) C(L, 1, 4) C(L, 1, 2) C(L, 1, 1) C(L, 2, 4) C(L, 2, 2) C(L, 2, 1) C(L, 4, 2) C(L, 4, 1)
    CL(64) CL(32) CL(16)
#undef CL
#undef C
    return hipErrorNotSupported;
}

hipError_t launch_mv_f32in(int fmt, const MvPlan &p, hipStream_t st, const F32Args &a) {
    switch (fmt) {
    case F_Q8_0: return launch_f32in_fmt<F_Q8_0>(p, st, a);
    case F_Q6K: return launch_f32in_fmt<F_Q6K>(p, st, a);
    case F_F32: return launch_f32in_fmt<F_F32>(p, st, a);
    }
    return hipErrorNotSupported;
}

}  // namespace fl
