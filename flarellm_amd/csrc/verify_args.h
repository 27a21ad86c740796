// Arguments of the speculative-verify GEMM (kernels in verify_kernels.h,
// included by verify.hip only).
#pragma once

#include "kernels.h"

namespace fl {

constexpr int kVerifyMaxTokens = 16;  // the MFMA tile's token side (fl_verify batches)
constexpr int kPrefillTokens = 64;    // prefill passes: four token tiles per weight fragment
constexpr int kPrefillMaxKsplit = 32;

typedef long long i64x1_t;
typedef int v4i32_t __attribute__((ext_vector_type(4)));
typedef float v4f32_t __attribute__((ext_vector_type(4)));

struct VgArgs {
    WDesc W;          // weight planes (Q8_0: int8 quants + f16 scales; Q4_K: qs + 16-B headers)
    const int8_t *xq; // [M][K] Q8_0-quantized activations
    const float *xs;  // [M][K/32] block scales
    const int *xsum;  // [M][K/32] block sums of the quants
    int M;
    int ksplit;       // K chunks (grid y)
    int chunk;        // units (Q8_0 blocks / Q4_K super-blocks) per K chunk; ksplit = ceil(units / chunk)
    float *part;      // [ksplit][M][rows] fp32 partial sums
    int *dots;        // testing (nullptr otherwise): the per-block integer dots the MFMAs form,
                      // [M][rows][K/32] (Q4_K: block 8*sb + j = sub-block j of super-block sb)
    // k_vgemm_q4k8 only (rows % 64 == 0): the last-arriving K split of each
    // workgroup column sums the partials of its 64 rows and applies
    // post 1 = SiLU(gate)*up + Q8_0 (gate/up weight; a column holds 32 gate
    // and the matching 32 up rows), post 2 = the QKV post (qp); 0 = none
    int post;
    int *counters;    // [gridDim.x] arrival counters, zero between launches
    int8_t *hq;       // post 1: Q8_0 of h, [M][F] codes, [M][F/32] scales and sums
    float *hs;
    int *hsum;
    int F;
    struct QkvPost {
        int nq, nk, D;
        const float *rope;
        long long sin_off;
        const int *pos0p;
        float *Q, *Kst, *Vst;
        void *kc, *vc;          // KVW 1 / 2: the layer's F16 / F32 cache
        long long head_stride;
        int v_tblk;
        int kvw;                // 0 staging rows, 1 F16 cache, 2 F32 cache
    } qp;
};

}  // namespace fl
