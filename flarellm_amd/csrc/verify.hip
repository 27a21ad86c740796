// Speculative-verify launchers (kernels in verify_kernels.h).
#include "launch.h"
#include "verify_kernels.h"

namespace fl {

hipError_t launch_vgemm(int fmt, hipStream_t st, const VgArgs &a) {
    const int tiles = (a.W.rows + 15) / 16;
    const dim3 grid((tiles + 3) / 4, a.ksplit);
    if (a.M < 1 || a.M > kPrefillTokens || a.ksplit < 1 || a.chunk < 1) return hipErrorInvalidValue;
    const int nt = (a.M + 15) / 16;  // token tiles of the M > 8 kernels
    if (a.M > kVerifyMaxTokens && a.W.cols % 256 == 0 && !a.post) {
        // prefill batches: activations staged per 256-value step (chunk = steps)
        // Q4_K: the int8-MFMA form, whose MFMAs form the reference's exact
        // per-block integer dots (C3 4096-token prefill 336 ms).
        // FLARE_PGEMM_H: the f16-MFMA form (sub-block scales folded into the
        // weight operand, activation scales into the activation operand, so
        // the MFMAs apply the block terms; 381 ms), whose MFMAs accumulate
        // scaled products rather than integer dots; a measurement switch
        static const bool f16 = measure_env("FLARE_PGEMM_H") != nullptr;
        if (fmt == F_Q4K && f16 && !a.dots) {
            const dim3 gh((tiles + 7) / 8, a.ksplit);
            static const bool db = measure_env("FLARE_PGEMM_DB") != nullptr;  // measurement switch
            if (db) hipLaunchKernelGGL((k_pgemm_h<8, 2>), gh, dim3(512), 0, st, a);
            else hipLaunchKernelGGL((k_pgemm_h<8, 1>), gh, dim3(512), 0, st, a);
        } else if (fmt == F_Q4K) {
            // 8-wave workgroups (128 rows per staged activation tile, 16
            // waves per CU): C3 4096-token prefill 358 -> 336 ms against 4 waves
            const dim3 g8((tiles + 7) / 8, a.ksplit);
            if (a.dots) hipLaunchKernelGGL((k_pgemm<F_Q4K, true, 8>), g8, dim3(512), 0, st, a);
            else hipLaunchKernelGGL((k_pgemm<F_Q4K, false, 8>), g8, dim3(512), 0, st, a);
        } else if (fmt == F_Q8_0) {
            // 4 waves: 8 measured alike on Llama-3.2-1B (C2 512 tokens 12.2-12.4 ms)
            if (a.dots) hipLaunchKernelGGL((k_pgemm<F_Q8_0, true>), grid, dim3(256), 0, st, a);
            else hipLaunchKernelGGL((k_pgemm<F_Q8_0, false>), grid, dim3(256), 0, st, a);
        } else {
            return hipErrorNotSupported;
        }
        return hipGetLastError();
    }
    if (a.W.cols % 32) return hipErrorInvalidValue;
    size_t kn;
    if (fmt == F_Q4K) {
        if (a.W.cols % 256) return hipErrorInvalidValue;
        const int nsb = a.W.cols >> 8;
        kn = (size_t)a.chunk * 256;
        if (a.post) {
            // fused epilogues: 8-token kernel, whole 64-row columns
            if (a.M > 8 || a.W.rows % 64 || !a.counters) return hipErrorInvalidValue;
            if (a.post == 1 && (a.F % 32 || a.W.rows != 2 * a.F || !a.hq)) return hipErrorInvalidValue;
        }
        if (a.M <= 8) {
            // activations of 8 token rows, then 8 (scale, sum) pairs per block
            // one super-block in flight per wave: 2 or 3 measured slower on
            // MI355X (Llama-3-8B shapes; VGPRs 112 / 132 against 85)
            const size_t lds = 8 * (kn + 32) + 8 * (kn / 32) * 8;
            hipLaunchKernelGGL(k_vgemm_q4k8<1>, grid, dim3(256), lds, st, a);
        } else {
            if (a.post) return hipErrorInvalidValue;
            const size_t lds = (((size_t)a.M * (kn + 32) + 15) & ~(size_t)15) + (size_t)a.M * (kn / 32) * 8;
            switch (nt) {
            case 1: hipLaunchKernelGGL(k_vgemm_q4k<1>, grid, dim3(256), lds, st, a); break;
            case 2: hipLaunchKernelGGL(k_vgemm_q4k<2>, grid, dim3(256), lds, st, a); break;
            case 3: hipLaunchKernelGGL(k_vgemm_q4k<3>, grid, dim3(256), lds, st, a); break;
            default: hipLaunchKernelGGL(k_vgemm_q4k<4>, grid, dim3(256), lds, st, a); break;
            }
        }
    } else {
        if (fmt != F_Q8_0 || a.post) return hipErrorNotSupported;
        const int nb = a.W.cols >> 5;
        kn = (size_t)a.chunk * 32;
        if (a.M <= 8) {
            hipLaunchKernelGGL(k_vgemm_q8_08, grid, dim3(256), 8 * (kn + 32) + 8 * (kn / 32) * 8, st, a);
        } else {
            const size_t lds = (((size_t)a.M * (kn + 32) + 15) & ~(size_t)15) + (size_t)a.M * (kn / 32) * 8;
            switch (nt) {
            case 1: hipLaunchKernelGGL(k_vgemm_q8_0<1>, grid, dim3(256), lds, st, a); break;
            case 2: hipLaunchKernelGGL(k_vgemm_q8_0<2>, grid, dim3(256), lds, st, a); break;
            case 3: hipLaunchKernelGGL(k_vgemm_q8_0<3>, grid, dim3(256), lds, st, a); break;
            default: hipLaunchKernelGGL(k_vgemm_q8_0<4>, grid, dim3(256), lds, st, a); break;
            }
        }
    }
    return hipGetLastError();
}

hipError_t launch_v_embed(int fmt, hipStream_t st, const WDesc &E, const int *tokens, int M, float *x) {
    switch (fmt) {
    case F_Q8_0: hipLaunchKernelGGL(k_v_embed<F_Q8_0>, dim3(M), dim3(256), 0, st, E, tokens, x); break;
    case F_Q6K: hipLaunchKernelGGL(k_v_embed<F_Q6K>, dim3(M), dim3(256), 0, st, E, tokens, x); break;
    case F_Q4K: hipLaunchKernelGGL(k_v_embed<F_Q4K>, dim3(M), dim3(256), 0, st, E, tokens, x); break;
    default: hipLaunchKernelGGL(k_v_embed<F_F32>, dim3(M), dim3(256), 0, st, E, tokens, x); break;
    }
    return hipGetLastError();
}

hipError_t launch_v_resnorm(int pro, hipStream_t st, const float *part, int ksplit, int M, int H, float *x,
                            const float *w, float eps, int8_t *q, float *s, int *sum) {
    if (H % 32 || H > kResnormMaxH || M < 1) return hipErrorInvalidValue;
    if (pro == PRO_NORMQ0)
        hipLaunchKernelGGL(k_v_resnorm<PRO_NORMQ0>, dim3(M), dim3(kResnormThreads), 0, st, part, ksplit, M, H, x, w,
                           eps, q, s, sum);
    else
        hipLaunchKernelGGL(k_v_resnorm<PRO_NORMQ1>, dim3(M), dim3(kResnormThreads), 0, st, part, ksplit, M, H, x, w,
                           eps, q, s, sum);
    return hipGetLastError();
}

// P.kvw 1 / 2: K / V go straight into the F16 / F32 cache slots; 0: to the
// f32 staging rows
hipError_t launch_v_qkv_post(hipStream_t st, const float *part, int ksplit, int M, int rows,
                             const VgArgs::QkvPost &P) {
    const dim3 grid((rows / 2 + 255) / 256, M);
    if (P.kvw == 1) hipLaunchKernelGGL(k_v_qkv_post<1>, grid, dim3(256), 0, st, part, ksplit, M, rows, P);
    else if (P.kvw == 2) hipLaunchKernelGGL(k_v_qkv_post<2>, grid, dim3(256), 0, st, part, ksplit, M, rows, P);
    else hipLaunchKernelGGL(k_v_qkv_post<0>, grid, dim3(256), 0, st, part, ksplit, M, rows, P);
    return hipGetLastError();
}

hipError_t launch_v_store(hipStream_t st, const float *part, int ksplit, int M, int rows, float *out) {
    hipLaunchKernelGGL(k_v_store, dim3((rows + 255) / 256, M), dim3(256), 0, st, part, ksplit, M, rows, out);
    return hipGetLastError();
}

hipError_t launch_v_residual(hipStream_t st, const float *part, int ksplit, int M, int H, float *x) {
    hipLaunchKernelGGL(k_v_residual, dim3((H + 255) / 256, M), dim3(256), 0, st, part, ksplit, M, H, x);
    return hipGetLastError();
}

hipError_t launch_v_silu_quant(hipStream_t st, const float *part, int ksplit, int M, int F, int8_t *q, float *s,
                               int *sum) {
    if (F % 32) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_v_silu_quant, dim3((F + 255) / 256, M), dim3(256), 0, st, part, ksplit, M, F, q, s, sum);
    return hipGetLastError();
}

}  // namespace fl
