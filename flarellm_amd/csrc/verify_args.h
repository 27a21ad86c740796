// Arguments of the speculative-verify GEMM (kernels in verify_kernels.h,
// included by verify.hip only).
#pragma once

#include "kernels.h"

namespace fl {

constexpr int kVerifyMaxTokens = 16;  // the MFMA tile's token side

typedef long long i64x1_t;
typedef int v4i32_t __attribute__((ext_vector_type(4)));

struct VgArgs {
    WDesc W;          // weight planes (Q8_0: int8 quants + f16 scales; Q4_K: qs + 16-B headers)
    const int8_t *xq; // [M][K] Q8_0-quantized activations
    const float *xs;  // [M][K/32] block scales
    const int *xsum;  // [M][K/32] block sums of the quants
    int M;
    int ksplit;       // K chunks (grid y); chunk = ceil(units / ksplit) units
    float *part;      // [ksplit][M][rows] fp32 partial sums
};

// Plain (F32 / F16) cache of one layer, for K / V written straight from the
// QKV partials.
struct KvDst {
    void *kc, *vc;
    long long head_stride;  // elements between kv heads
    int v_tblk;             // V in 32-slot transposed blocks
};

}  // namespace fl
