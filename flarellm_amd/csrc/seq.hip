// Reference-order kernels of the decode step (FL_OPT_EXACT).
//
// With FL_OPT_EXACT the decode step computes every floating-point value in
// the order of the x86-64 reference, so its logits are bit-identical to the
// CPU restatement.  The quantized matvecs are the streaming kernels of
// mvs_kernels.h with their SEQ instantiation (same tiles, loads, integer dots
// and per-block terms; row sums folded in block order).  Attention and the
// f32 output projection are sequential in the reference and get the kernels
// below: they are simple, not fast.
#include "launch.h"

namespace fl {

// grouped-query attention of one query head over slots 0..pos (model.rs:
// 9849-9905, fused_attention_head_scalar 9914-9966): scores
// (sum_d q k sequential) * (1/sqrt(D)), then the online softmax in token
// order.  One workgroup per query head; the scores go through `scores`.
template <bool F16>
__global__ __launch_bounds__(256) void k_attn_seq(SeqAttnArgs a) {
    const int h = blockIdx.x, kvh = h / a.group, D = a.D;
    const int T = *a.posp + 1;
    const float *qh = a.q + (size_t)h * D;
    float *sc = a.scores + (size_t)h * a.slots;
    const size_t hbase = (size_t)kvh * a.head_stride;
    const float scale = 1.0f / sqrtf((float)D);
    for (int t = threadIdx.x; t < T; t += blockDim.x) {
        float dot = 0.0f;
        for (int d = 0; d < D; d++) {
            const size_t o = hbase + (size_t)t * D + d;
            const float k = F16 ? h2f(((const uint16_t *)a.kc)[o]) : ((const float *)a.kc)[o];
            dot += qh[d] * k;
        }
        sc[t] = dot * scale;
    }
    __syncthreads();
    if ((int)threadIdx.x < D) {
        const int d = threadIdx.x;
        float m = -INFINITY, sum = 0.0f, o = 0.0f;
        for (int t = 0; t < T; t++) {
            const float s = sc[t];
            // F16 caches keep V in 32-slot transposed blocks [slot/32][D][32]
            const float v = F16 ? h2f(((const uint16_t *)a.vc)[hbase + ((size_t)(t >> 5) * D + d) * 32 + (t & 31)])
                                : ((const float *)a.vc)[hbase + (size_t)t * D + d];
            const float nm = fmaxf(m, s);
            const float old_scale = fl_expf(m - nm);
            const float w = fl_expf(s - nm);
            sum = sum * old_scale + w;
            o = o * old_scale + w * v;
            m = nm;
        }
        if (sum > 0.0f) {
            const float inv = 1.0f / sum;
            o *= inv;
        }
        a.out[(size_t)h * D + d] = o;
    }
}

// rmsnorm_into (model.rs:7456-7477): (x * inv_rms) * w with the sequential
// sum of squares.  One workgroup.
__global__ __launch_bounds__(256) void k_rmsnorm_seq(const float *x, const float *w, int n, float eps, float *out) {
    __shared__ float ess[kEssLdsWords + 1];
    const float inv = wg_inv_rms<true>(x, n, eps, nullptr, ess);
    for (int i = threadIdx.x; i < n; i += blockDim.x) out[i] = (x[i] * inv) * w[i];
}

// Output projection over the dequantized weight with an f32 input, one row
// per thread: matvec_argmax_f32 (model.rs:8668-8689, sum += row[j] * vec[j]
// in order, first maximum) and, with `logits`, the matvec_into values.
// Weights dequantized as dequantize_tensor does (quantize.rs:189-197,
// 343-384).
template <int FMT>
__global__ __launch_bounds__(256) void k_out_seq(WDesc W, const float *xn, float *logits, unsigned long long *slot) {
    extern __shared__ float lx[];
    const int K = W.cols;
    for (int i = threadIdx.x; i < K; i += blockDim.x) lx[i] = xn[i];
    __syncthreads();
    const int row = blockIdx.x * blockDim.x + threadIdx.x;
    unsigned long long best = 0;
    if (row < W.rows) {
        float s = 0.0f;
        if (FMT == F_Q8_0) {
            const int nb = K >> 5;
            for (int b = 0; b < nb; b++) {
                const float scale = h2f(W.s[(size_t)row * nb + b]);
                const int8_t *q = (const int8_t *)W.q + (size_t)row * K + 32 * b;
                for (int k = 0; k < 32; k++) s += ((float)q[k] * scale) * lx[32 * b + k];
            }
        } else if (FMT == F_Q6K) {
            for (int j = 0; j < K; j++) s += q6k_elem(W, row, j) * lx[j];
        } else if (FMT == F_Q4K) {
            for (int j = 0; j < K; j++) s += q4k_elem(W, row, j) * lx[j];
        } else {
            const float *r = (const float *)W.q + (size_t)row * K;
            for (int j = 0; j < K; j++) s += r[j] * lx[j];
        }
        if (logits) logits[row] = s;
        best = argmax_key(s, (uint32_t)row);
    }
    if (!slot) return;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) best = umax64(best, __shfl_xor(best, o, 64));
    if ((threadIdx.x & 63) == 0 && best) atomicMax(slot, best);
}

hipError_t launch_attn_seq(bool f16, hipStream_t st, const SeqAttnArgs &a, int num_heads) {
    if (f16) hipLaunchKernelGGL(k_attn_seq<true>, dim3(num_heads), dim3(256), 0, st, a);
    else hipLaunchKernelGGL(k_attn_seq<false>, dim3(num_heads), dim3(256), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_rmsnorm_seq(hipStream_t st, const float *x, const float *w, int n, float eps, float *out) {
    hipLaunchKernelGGL(k_rmsnorm_seq, dim3(1), dim3(256), 0, st, x, w, n, eps, out);
    return hipGetLastError();
}

hipError_t launch_out_seq(int fmt, hipStream_t st, const WDesc &W, const float *xn, float *logits,
                          unsigned long long *slot) {
    const dim3 grid((W.rows + 255) / 256);
    const size_t lds = (size_t)W.cols * 4;
    switch (fmt) {
    case F_Q8_0: hipLaunchKernelGGL(k_out_seq<F_Q8_0>, grid, dim3(256), lds, st, W, xn, logits, slot); break;
    case F_Q6K: hipLaunchKernelGGL(k_out_seq<F_Q6K>, grid, dim3(256), lds, st, W, xn, logits, slot); break;
    case F_Q4K: hipLaunchKernelGGL(k_out_seq<F_Q4K>, grid, dim3(256), lds, st, W, xn, logits, slot); break;
    case F_F32: hipLaunchKernelGGL(k_out_seq<F_F32>, grid, dim3(256), lds, st, W, xn, logits, slot); break;
    default: return hipErrorNotSupported;
    }
    return hipGetLastError();
}

}  // namespace fl
