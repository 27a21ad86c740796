// MFMA output projection (f32 input) launcher.
#include "launch.h"
#include "mvo_kernels.h"

namespace fl {

hipError_t launch_mvo(int fmt, hipStream_t st, const MvoArgs &a) {
    if (a.M < 1 || a.M > kMvoMaxTokens) return hipErrorInvalidValue;
    const size_t lds = (size_t)2 * a.M * a.W.cols * 2 + 64;
    const int ntiles = (a.W.rows + 15) / 16;
    const int want = std::max(1, (ntiles + kMvoThreads / 64 - 1) / (kMvoThreads / 64));
    if (fmt == F_Q6K) {
        if (a.W.cols % 256) return hipErrorInvalidValue;
        hipLaunchKernelGGL(k_mvo<F_Q6K>, dim3(resident_grid(k_mvo<F_Q6K>, kMvoThreads, lds, want)),
                           dim3(kMvoThreads), lds, st, a);
    } else if (fmt == F_Q8_0) {
        if (a.W.cols % 32) return hipErrorInvalidValue;
        hipLaunchKernelGGL(k_mvo<F_Q8_0>, dim3(resident_grid(k_mvo<F_Q8_0>, kMvoThreads, lds, want)),
                           dim3(kMvoThreads), lds, st, a);
    } else {
        return hipErrorNotSupported;
    }
    return hipGetLastError();
}

}  // namespace fl
