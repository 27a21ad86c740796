// Decode attention launchers.
#include "launch.h"

namespace fl {

template <typename KT>
static hipError_t launch_attn_t(int D, int G, hipStream_t st, const AttnArgs &a) {
#define C(DD, GG)                                                                                  \
    if (D == DD && G == GG) {                                                                      \
        hipLaunchKernelGGL((k_attn<KT, DD, GG>), dim3(a.nsplit, a.nkv), dim3(kAttnThreads), 0, st, a); \
        return hipSuccess;                                                                         \
    }
    C(64, 1) C(64, 2) C(64, 3) C(64, 4) C(64, 8)
    C(128, 1) C(128, 2) C(128, 3) C(128, 4) C(128, 8)
#undef C
    return hipErrorNotSupported;
}

hipError_t launch_attn(bool f16, int D, int G, hipStream_t st, const AttnArgs &a) {
    if (a.nsplit < 1 || a.nsplit > kAttnMaxSplit) return hipErrorInvalidValue;
    return f16 ? launch_attn_t<__half>(D, G, st, a) : launch_attn_t<float>(D, G, st, a);
}

}  // namespace fl
