// Decode attention launchers.
#include "launch.h"

namespace fl {

template <typename KT, int DD, int GG>
static hipError_t launch_one(hipStream_t st, const AttnArgs &a) {
    const size_t lds = ((size_t)(kAttnThreads / 64) * GG * DD + (size_t)2 * a.nsplit * GG) * 4;
    static bool attr_set = false;  // allow > 64 KiB of dynamic LDS (160 KiB per CU on gfx950)
    if (!attr_set) {
        const hipError_t e = hipFuncSetAttribute((const void *)k_attn<KT, DD, GG>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024 - 16384);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    hipLaunchKernelGGL((k_attn<KT, DD, GG>), dim3(a.nsplit, a.nkv), dim3(kAttnThreads), lds, st, a);
    return hipSuccess;
}

template <typename KT>
static hipError_t launch_attn_t(int D, int G, hipStream_t st, const AttnArgs &a) {
#define C(DD, GG) \
    if (D == DD && G == GG) return launch_one<KT, DD, GG>(st, a);
    C(64, 1) C(64, 2) C(64, 3) C(64, 4) C(64, 8)
    C(128, 1) C(128, 2) C(128, 3) C(128, 4) C(128, 8)
#undef C
    return hipErrorNotSupported;
}

hipError_t launch_attn(bool f16, int D, int G, hipStream_t st, const AttnArgs &a) {
    return f16 ? launch_attn_t<__half>(D, G, st, a) : launch_attn_t<float>(D, G, st, a);
}

}  // namespace fl
