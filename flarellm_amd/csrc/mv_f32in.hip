// f32-input matvecs (logits path): Q8_0 (tied embedding), Q6_K, F32.
#include "launch.h"

namespace fl {

template <int FMT>
static hipError_t launch_f32in_fmt(const MvPlan &p, hipStream_t st, const F32Args &a) {
#define C(L, RR, UU)                                                                                \
    if (p.lpr == L && p.r == RR && p.u == UU) {                                                     \
        hipLaunchKernelGGL((k_mv_f32in<FMT, L, RR, UU>), dim3(p.grid), dim3(kThreads), p.lds, st, a); \
        return hipSuccess;                                                                          \
    }
    C(64, 1, 1) C(64, 2, 1) C(64, 4, 1) C(64, 8, 1) C(64, 1, 2) C(64, 2, 2) C(64, 4, 2) C(64, 1, 4) C(64, 2, 4)
    C(32, 1, 1) C(32, 2, 1) C(32, 4, 1) C(32, 8, 1) C(32, 1, 2) C(32, 2, 2) C(32, 4, 2)
    C(16, 1, 1) C(16, 2, 1) C(16, 4, 1) C(16, 8, 1) C(16, 1, 2) C(16, 2, 2) C(16, 4, 2)
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
