// Quantized matvec kernels (batch-1 decode), gfx950 wave64.
//
// Work split: a workgroup of 256 threads is divided into groups of LPR lanes;
// each group owns R consecutive output rows.  Lane gl of a group walks the
// row's "units" gl, gl+LPR, ... and issues the weight loads of U units x R
// rows before consuming any of them, so every lane keeps U*R*32 bytes of
// HBM reads in flight.  The activation is staged once per workgroup in LDS
// (loaded, or computed by a fused RMSNorm+Q8 prologue).  Row partial sums
// are reduced within the group with a fixed butterfly (deterministic).
#pragma once

#include "kernels.h"

namespace fl {

enum Epi { EPI_STORE = 0, EPI_ADD = 1, EPI_ARGMAX = 2 };

struct Q8inArgs {
    WDesc W;
    int pro, epi;
    const float *x, *nw;  // prologue input / norm weight (PRO_NORMQ*)
    float eps;
    const int8_t *gq;     // PRO_LOADQ input
    const float *gs;
    const int *gsum;
    float *out;
    unsigned long long *slot;  // EPI_ARGMAX
};

struct F32Args {
    WDesc W;
    int pro, epi;  // pro 0: load x; 1: rmsnorm_into(x, nw) (model.rs:7469-7477)
    const float *x, *nw;
    float eps;
    float *out;
    unsigned long long *slot;
};

struct GuArgs {
    WDesc W;  // [w_gate; w_up], 2F rows
    int F, pro;
    const float *x, *nw;
    float eps;
    const int8_t *gq;
    const float *gs;
    const int *gsum;
    int8_t *hq;
    float *hs;
    int *hsum;
    float *hout;  // optional f32 SiLU*up output
};

// ---------------------------------------------------------------------------
// row dot bodies
// ---------------------------------------------------------------------------
template <int LPR, int R, int U>
__device__ __forceinline__ void rows_q8_0(const WDesc &W, const int *rix, const int8_t *lq,
                                          const float *ls, int gl, float *acc) {
    const int bpr = W.cols >> 5;
    for (int b0 = gl; b0 < bpr; b0 += LPR * U) {
        int4 w0[U][R], w1[U][R];
        uint16_t sc[U][R];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int b = min(b0 + u * LPR, bpr - 1);
#pragma unroll
            for (int r = 0; r < R; r++) {
                const int4 *p = (const int4 *)(W.q + (size_t)rix[r] * W.cols + b * 32);
                w0[u][r] = ld_stream(p);
                w1[u][r] = ld_stream(p + 1);
                sc[u][r] = W.s[(size_t)rix[r] * bpr + b];
            }
        }
        __builtin_amdgcn_sched_barrier(0);  // keep all loads above issued back to back
        // branch-free consume (a branch would let the compiler sink the loads
        // above into it and serialize them); out-of-range units add 0
#pragma unroll
        for (int u = 0; u < U; u++) {
            const bool valid = b0 + u * LPR < bpr;
            const int b = valid ? b0 + u * LPR : bpr - 1;
            const int4 x0 = *(const int4 *)(lq + b * 32), x1 = *(const int4 *)(lq + b * 32 + 16);
            const float xs = ls[b];
#pragma unroll
            for (int r = 0; r < R; r++) {
                const int d = dot16(w1[u][r], x1, dot16(w0[u][r], x0, 0));
                const float combined = h2f(sc[u][r]) * xs;
                const float t = combined * (float)d;
                acc[r] += valid ? t : 0.0f;
            }
        }
    }
}

template <int LPR, int R, int U>
__device__ __forceinline__ void rows_q4k(const WDesc &W, const int *rix, const int8_t *lq,
                                         const float *ls, const int *lsum, int gl, float *acc) {
    const int nsb = W.cols >> 8;
    const int units = nsb * 4;
    const size_t rstride = (size_t)nsb * 144;
    for (int u0 = gl; u0 < units; u0 += LPR * U) {
        int4 hd[U][R], q0[U][R], q1[U][R];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int uu = min(u0 + u * LPR, units - 1);
            const int sb = uu >> 2, sub = uu & 3;
#pragma unroll
            for (int r = 0; r < R; r++) {
                const uint8_t *blk = W.q + (size_t)rix[r] * rstride + (size_t)sb * 144;
                hd[u][r] = ld_stream((const void *)blk);
                q0[u][r] = ld_stream((const void *)(blk + 16 + 32 * sub));
                q1[u][r] = ld_stream((const void *)(blk + 32 + 32 * sub));
            }
        }
        __builtin_amdgcn_sched_barrier(0);  // keep all loads above issued back to back
#pragma unroll
        for (int u = 0; u < U; u++) {
            const bool valid = u0 + u * LPR < units;
            const int uu = valid ? u0 + u * LPR : units - 1;
            const int sb = uu >> 2, sub = uu & 3;
            const int blo = sb * 8 + sub, bhi = blo + 4;
            const int4 xl0 = *(const int4 *)(lq + blo * 32), xl1 = *(const int4 *)(lq + blo * 32 + 16);
            const int4 xh0 = *(const int4 *)(lq + bhi * 32), xh1 = *(const int4 *)(lq + bhi * 32 + 16);
            const float s_lo = ls[blo], s_hi = ls[bhi];
            const float qsum_lo = (float)lsum[blo], qsum_hi = (float)lsum[bhi];
#pragma unroll
            for (int r = 0; r < R; r++) {
                const uint32_t h0 = (uint32_t)hd[u][r].x;
                const float d = h2f((uint16_t)(h0 & 0xFFFF)), dmin = h2f((uint16_t)(h0 >> 16));
                // unpack_q4k_scales (model.rs:8709-8719) for sub and sub+4
                const uint32_t s_a = byte_of((uint32_t)hd[u][r].y, sub);  // scales[sub]
                const uint32_t s_b = byte_of((uint32_t)hd[u][r].z, sub);  // scales[sub+4]
                const uint32_t s_c = byte_of((uint32_t)hd[u][r].w, sub);  // scales[sub+8]
                const uint32_t sc_lo = s_a & 63, mn_lo = s_b & 63;
                const uint32_t sc_hi = (s_a >> 6) | ((s_c & 0xF) << 2);
                const uint32_t mn_hi = (s_b >> 6) | ((s_c >> 4) << 2);
                const int4 a = q0[u][r], c = q1[u][r];
                const int4 lo0 = make_int4(a.x & 0x0F0F0F0F, a.y & 0x0F0F0F0F, a.z & 0x0F0F0F0F, a.w & 0x0F0F0F0F);
                const int4 lo1 = make_int4(c.x & 0x0F0F0F0F, c.y & 0x0F0F0F0F, c.z & 0x0F0F0F0F, c.w & 0x0F0F0F0F);
                const int4 hi0 = make_int4((a.x >> 4) & 0x0F0F0F0F, (a.y >> 4) & 0x0F0F0F0F,
                                           (a.z >> 4) & 0x0F0F0F0F, (a.w >> 4) & 0x0F0F0F0F);
                const int4 hi1 = make_int4((c.x >> 4) & 0x0F0F0F0F, (c.y >> 4) & 0x0F0F0F0F,
                                           (c.z >> 4) & 0x0F0F0F0F, (c.w >> 4) & 0x0F0F0F0F);
                const int dl = dot16(lo1, xl1, dot16(lo0, xl0, 0));
                const int dh = dot16(hi1, xh1, dot16(hi0, xh0, 0));
                // per-term arithmetic of dot_q4k_q8_0_scalar (model.rs:9016-9022)
                const float d_sc_lo = d * (float)sc_lo, dmin_mn_lo = dmin * (float)mn_lo;
                const float d_sc_hi = d * (float)sc_hi, dmin_mn_hi = dmin * (float)mn_hi;
                const float t_lo = s_lo * (d_sc_lo * (float)dl - dmin_mn_lo * qsum_lo);
                const float t_hi = s_hi * (d_sc_hi * (float)dh - dmin_mn_hi * qsum_hi);
                acc[r] += valid ? t_lo : 0.0f;
                acc[r] += valid ? t_hi : 0.0f;
            }
        }
    }
}

// f32-input bodies (logits path: dequantized weight times the unquantized
// final_normed, matvec_argmax_f32 model.rs:8668-8689)
template <int LPR, int R, int U>
__device__ __forceinline__ void rows_f32in_q8_0(const WDesc &W, const int *rix, const float *lx, int gl,
                                                float *acc) {
    const int bpr = W.cols >> 5;
    for (int b0 = gl; b0 < bpr; b0 += LPR * U) {
        int4 w0[U][R], w1[U][R];
        uint16_t sc[U][R];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int b = min(b0 + u * LPR, bpr - 1);
#pragma unroll
            for (int r = 0; r < R; r++) {
                const int4 *p = (const int4 *)(W.q + (size_t)rix[r] * W.cols + b * 32);
                w0[u][r] = ld_stream(p);
                w1[u][r] = ld_stream(p + 1);
                sc[u][r] = W.s[(size_t)rix[r] * bpr + b];
            }
        }
        __builtin_amdgcn_sched_barrier(0);  // keep all loads above issued back to back
#pragma unroll
        for (int u = 0; u < U; u++) {
            const bool valid = b0 + u * LPR < bpr;
            const int b = valid ? b0 + u * LPR : bpr - 1;
            float xv[32];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const float4 t = *(const float4 *)(lx + b * 32 + 4 * j);
                xv[4 * j] = t.x; xv[4 * j + 1] = t.y; xv[4 * j + 2] = t.z; xv[4 * j + 3] = t.w;
            }
#pragma unroll
            for (int r = 0; r < R; r++) {
                const float scale = h2f(sc[u][r]);
                const int ws[8] = {w0[u][r].x, w0[u][r].y, w0[u][r].z, w0[u][r].w,
                                   w1[u][r].x, w1[u][r].y, w1[u][r].z, w1[u][r].w};
                float a = 0.0f;
#pragma unroll
                for (int j = 0; j < 8; j++)
#pragma unroll
                    for (int k = 0; k < 4; k++) {
                        // dequant_q8_0_block: (q as f32) * scale (quantize.rs:194)
                        const float wv = (float)(int8_t)(ws[j] >> (8 * k)) * scale;
                        a += wv * xv[4 * j + k];
                    }
                acc[r] += valid ? a : 0.0f;
            }
        }
    }
}

template <int LPR, int R, int U>
__device__ __forceinline__ void rows_f32in_q6k(const WDesc &W, const int *rix, const float *lx, int gl,
                                               float *acc) {
    const int nsb = W.cols >> 8;
    const int units = nsb * 4;  // unit = (superblock, half, l0 in {0,16}) -> 64 weights
    for (int u0 = gl; u0 < units; u0 += LPR * U) {
        int4 qa[U][R], qb[U][R], qh[U][R], scv[U][R];
        uint16_t dd[U][R];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int uu = min(u0 + u * LPR, units - 1);
            const int sb = uu >> 2, hf = (uu >> 1) & 1, l0 = (uu & 1) * 16;
#pragma unroll
            for (int r = 0; r < R; r++) {
                const uint8_t *body = W.q + ((size_t)rix[r] * nsb + sb) * 208;
                qa[u][r] = ld_stream((const void *)(body + 64 * hf + l0));
                qb[u][r] = ld_stream((const void *)(body + 64 * hf + 32 + l0));
                qh[u][r] = ld_stream((const void *)(body + 128 + 32 * hf + l0));
                scv[u][r] = *(const int4 *)(body + 192);
                dd[u][r] = W.s[(size_t)rix[r] * nsb + sb];
            }
        }
        __builtin_amdgcn_sched_barrier(0);  // keep all loads above issued back to back
#pragma unroll
        for (int u = 0; u < U; u++) {
            const bool valid = u0 + u * LPR < units;
            const int uu = valid ? u0 + u * LPR : units - 1;
            const int sb = uu >> 2, hf = (uu >> 1) & 1, l0 = (uu & 1) * 16;
            const int ebase = sb * 256 + hf * 128 + l0;
            const int so = hf * 8 + (l0 >> 4);
#pragma unroll
            for (int r = 0; r < R; r++) {
                const float d = h2f(dd[u][r]);
                const uint32_t scw[4] = {(uint32_t)scv[u][r].x, (uint32_t)scv[u][r].y, (uint32_t)scv[u][r].z,
                                         (uint32_t)scv[u][r].w};
                // dequant_q6k_block (quantize.rs:366-378): w = d * sc * q
                const float ds1 = d * (float)(int8_t)byte_of(scw[so >> 2], so & 3);
                const float ds2 = d * (float)(int8_t)byte_of(scw[(so + 2) >> 2], (so + 2) & 3);
                const float ds3 = d * (float)(int8_t)byte_of(scw[(so + 4) >> 2], (so + 4) & 3);
                const float ds4 = d * (float)(int8_t)byte_of(scw[(so + 6) >> 2], (so + 6) & 3);
                const uint32_t A[4] = {(uint32_t)qa[u][r].x, (uint32_t)qa[u][r].y, (uint32_t)qa[u][r].z,
                                       (uint32_t)qa[u][r].w};
                const uint32_t B[4] = {(uint32_t)qb[u][r].x, (uint32_t)qb[u][r].y, (uint32_t)qb[u][r].z,
                                       (uint32_t)qb[u][r].w};
                const uint32_t Hh[4] = {(uint32_t)qh[u][r].x, (uint32_t)qh[u][r].y, (uint32_t)qh[u][r].z,
                                        (uint32_t)qh[u][r].w};
                float a = 0.0f;
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const uint32_t la = byte_of(A[i >> 2], i & 3), lb = byte_of(B[i >> 2], i & 3);
                    const uint32_t hh = byte_of(Hh[i >> 2], i & 3);
                    const int q1 = (int)((la & 0xF) | ((hh & 3) << 4)) - 32;
                    const int q2 = (int)((lb & 0xF) | (((hh >> 2) & 3) << 4)) - 32;
                    const int q3 = (int)((la >> 4) | (((hh >> 4) & 3) << 4)) - 32;
                    const int q4 = (int)((lb >> 4) | (((hh >> 6) & 3) << 4)) - 32;
                    a += (ds1 * (float)q1) * lx[ebase + i];
                    a += (ds2 * (float)q2) * lx[ebase + 32 + i];
                    a += (ds3 * (float)q3) * lx[ebase + 64 + i];
                    a += (ds4 * (float)q4) * lx[ebase + 96 + i];
                }
                acc[r] += valid ? a : 0.0f;
            }
        }
    }
}

template <int LPR, int R, int U>
__device__ __forceinline__ void rows_f32in_f32(const WDesc &W, const int *rix, const float *lx, int gl,
                                               float *acc) {
    const int units = W.cols >> 2;
    const float *wf = (const float *)W.q;
    for (int u0 = gl; u0 < units; u0 += LPR * U) {
        float4 wv[U][R];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int uu = min(u0 + u * LPR, units - 1);
#pragma unroll
            for (int r = 0; r < R; r++)
                wv[u][r] = ld_stream_f((const void *)(wf + (size_t)rix[r] * W.cols + 4 * uu));
        }
        __builtin_amdgcn_sched_barrier(0);  // keep all loads above issued back to back
#pragma unroll
        for (int u = 0; u < U; u++) {
            const bool valid = u0 + u * LPR < units;
            const int uu = valid ? u0 + u * LPR : units - 1;
            const float4 xv = *(const float4 *)(lx + 4 * uu);
#pragma unroll
            for (int r = 0; r < R; r++) {
                const float t = wv[u][r].x * xv.x + wv[u][r].y * xv.y + wv[u][r].z * xv.z + wv[u][r].w * xv.w;
                acc[r] += valid ? t : 0.0f;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// epilogue helpers
// ---------------------------------------------------------------------------
template <int R>
__device__ __forceinline__ void group_argmax_commit(const float *acc, int row0, int rows,
                                                    unsigned long long *slot, unsigned long long *lred) {
    unsigned long long best = 0;
#pragma unroll
    for (int r = 0; r < R; r++) {
        if (row0 + r < rows) {
            const unsigned long long k = argmax_key(acc[r], (uint32_t)(row0 + r));
            best = k > best ? k : best;
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const unsigned long long t = __shfl_xor(best, o, 64);
        best = t > best ? t : best;
    }
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) lred[w] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long b = lred[0];
        for (int i = 1; i < (int)(blockDim.x >> 6); i++) b = lred[i] > b ? lred[i] : b;
        atomicMax(slot, b);
    }
}

template <int R>
__device__ __forceinline__ void store_rows(const float *acc, int row0, int rows, int gl, int epi, float *out) {
    if (gl < R && row0 + gl < rows) {
        float v = acc[0];
#pragma unroll
        for (int r = 1; r < R; r++) v = (gl == r) ? acc[r] : v;
        if (epi == EPI_ADD) out[row0 + gl] += v;  // residual add (model.rs:2305-2311, 2537-2543)
        else out[row0 + gl] = v;
    }
}

__host__ __device__ inline size_t q8_lds_bytes(int K) { return (size_t)K + (size_t)(K / 32) * 8 + 64 * 4 + 64; }

// ---------------------------------------------------------------------------
// kernels
// ---------------------------------------------------------------------------
template <int FMT, int LPR, int R, int U>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 4))) void k_mv_q8in(Q8inArgs a) {
    extern __shared__ __align__(16) char smem[];
    const WDesc &W = a.W;
    const int K = W.cols;
    int8_t *lq = (int8_t *)smem;
    float *ls = (float *)(smem + K);
    int *lsum = (int *)(ls + (K >> 5));
    float *red = (float *)(lsum + (K >> 5));
    if (a.pro == PRO_LOADQ) stage_q8<PRO_LOADQ>(a.x, a.nw, a.eps, K, a.gq, a.gs, a.gsum, lq, ls, lsum, red);
    else if (a.pro == PRO_NORMQ0) stage_q8<PRO_NORMQ0>(a.x, a.nw, a.eps, K, a.gq, a.gs, a.gsum, lq, ls, lsum, red);
    else stage_q8<PRO_NORMQ1>(a.x, a.nw, a.eps, K, a.gq, a.gs, a.gsum, lq, ls, lsum, red);
    constexpr int G = kThreads / LPR;
    const int grp = threadIdx.x / LPR, gl = threadIdx.x % LPR;
    const int row0 = (blockIdx.x * G + grp) * R;
    int rix[R];
#pragma unroll
    for (int r = 0; r < R; r++) rix[r] = min(row0 + r, W.rows - 1);
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;
    if (row0 < W.rows) {
        if (FMT == F_Q8_0) rows_q8_0<LPR, R, U>(W, rix, lq, ls, gl, acc);
        else rows_q4k<LPR, R, U>(W, rix, lq, ls, lsum, gl, acc);
    }
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = group_sum<LPR>(acc[r]);
    if (a.epi == EPI_ARGMAX) group_argmax_commit<R>(acc, row0, W.rows, a.slot, (unsigned long long *)red);
    else store_rows<R>(acc, row0, W.rows, gl, a.epi, a.out);
}

template <int FMT, int LPR, int R, int U>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 4))) void k_mv_f32in(F32Args a) {
    extern __shared__ __align__(16) char smem[];
    const WDesc &W = a.W;
    const int K = W.cols;
    float *lx = (float *)smem;
    float *red = lx + K;
    if (a.pro == 1) {
        const float inv = wg_inv_rms(a.x, K, a.eps, red);
        for (int i = threadIdx.x; i < K; i += blockDim.x) lx[i] = (a.x[i] * inv) * a.nw[i];
    } else {
        for (int i = threadIdx.x; i < K; i += blockDim.x) lx[i] = a.x[i];
    }
    __syncthreads();
    constexpr int G = kThreads / LPR;
    const int grp = threadIdx.x / LPR, gl = threadIdx.x % LPR;
    const int row0 = (blockIdx.x * G + grp) * R;
    int rix[R];
#pragma unroll
    for (int r = 0; r < R; r++) rix[r] = min(row0 + r, W.rows - 1);
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;
    if (row0 < W.rows) {
        if (FMT == F_Q8_0) rows_f32in_q8_0<LPR, R, U>(W, rix, lx, gl, acc);
        else if (FMT == F_Q6K) rows_f32in_q6k<LPR, R, U>(W, rix, lx, gl, acc);
        else rows_f32in_f32<LPR, R, U>(W, rix, lx, gl, acc);
    }
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = group_sum<LPR>(acc[r]);
    if (a.epi == EPI_ARGMAX) group_argmax_commit<R>(acc, row0, W.rows, a.slot, (unsigned long long *)red);
    else store_rows<R>(acc, row0, W.rows, gl, EPI_STORE, a.out);
}

// Fused gate/up matvec over W = [w_gate; w_up] with the SiLU(gate)*up
// (model.rs:9788-9795) and quantize_input_q8_0 (5557-5570) epilogue.
// Workgroup b (NT threads) produces hidden block b (32 values): NT/LPR groups
// each own RH gate rows and the matching RH up rows.
template <int FMT, int LPR, int U, int NT>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(1, 4))) void k_gateup(GuArgs a) {
    extern __shared__ __align__(16) char smem[];
    const WDesc &W = a.W;
    const int K = W.cols;
    int8_t *lq = (int8_t *)smem;
    float *ls = (float *)(smem + K);
    int *lsum = (int *)(ls + (K >> 5));
    float *red = (float *)(lsum + (K >> 5));
    float *gu = red + 16;  // [64]: gate[32], up[32]
    if (a.pro == PRO_LOADQ) stage_q8<PRO_LOADQ>(a.x, a.nw, a.eps, K, a.gq, a.gs, a.gsum, lq, ls, lsum, red);
    else if (a.pro == PRO_NORMQ0) stage_q8<PRO_NORMQ0>(a.x, a.nw, a.eps, K, a.gq, a.gs, a.gsum, lq, ls, lsum, red);
    else stage_q8<PRO_NORMQ1>(a.x, a.nw, a.eps, K, a.gq, a.gs, a.gsum, lq, ls, lsum, red);
    constexpr int G = NT / LPR;
    constexpr int R = 64 / G;
    constexpr int RH = R / 2;
    static_assert(RH >= 1, "gate_up needs >= 2 rows per group");
    const int grp = threadIdx.x / LPR, gl = threadIdx.x % LPR;
    const int i0 = blockIdx.x * 32 + grp * RH;
    int rix[R];
#pragma unroll
    for (int r = 0; r < R; r++) rix[r] = (r < RH) ? (i0 + r) : (a.F + i0 + r - RH);
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;
    if (FMT == F_Q8_0) rows_q8_0<LPR, R, U>(W, rix, lq, ls, gl, acc);
    else rows_q4k<LPR, R, U>(W, rix, lq, ls, lsum, gl, acc);
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = group_sum<LPR>(acc[r]);
    if (gl == 0) {
#pragma unroll
        for (int r = 0; r < RH; r++) {
            gu[grp * RH + r] = acc[r];
            gu[32 + grp * RH + r] = acc[RH + r];
        }
    }
    __syncthreads();
    if (threadIdx.x < 32) {
        // lanes 0..31 of wave 0: one hidden value each, then the block quantizer
        const int j = threadIdx.x;
        const float g = gu[j];
        const float h = (g / (1.0f + expf(-g))) * gu[32 + j];
        if (a.hout) a.hout[blockIdx.x * 32 + j] = h;
        gu[j] = h;
    }
    __syncthreads();
    if (threadIdx.x == 0) quant_block32(gu, a.hq + blockIdx.x * 32, a.hs + blockIdx.x, a.hsum + blockIdx.x);
}

}  // namespace fl
