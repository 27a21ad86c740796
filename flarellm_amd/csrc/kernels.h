// Device kernels of the MI355X decode backend (gfx950, wave64).
//
// Numerics contract (checked by tests against the CPU oracle):
//  * activation quantization (quantize_input_q8_0_into, model.rs:5557-5570)
//    is reproduced bit-exactly from identical f32 inputs: IEEE division,
//    round-half-away, saturating int8 cast;
//  * per-block integer dots are exact (v_dot4_i32_i8 on the same int8/nibble
//    operands as model.rs:8082-8099 / 8997-9014);
//  * every per-block float term is formed with the reference's operation
//    order (built with -ffp-contract=off); only the order in which the
//    per-block terms of a row are summed differs (wave tree instead of a
//    sequential loop), which the north-star tolerance (1e-3 rel) covers.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fl {

constexpr int kThreads = 256;  // 4 wave64 per workgroup

enum Fmt { F_F32 = 0, F_Q8_0 = 1, F_Q4K = 2, F_Q6K = 3 };

// ------------------------------------------------------------------------
// small helpers
// ------------------------------------------------------------------------
__device__ __forceinline__ float h2f(uint16_t h) { return __half2float(__ushort_as_half(h)); }
__device__ __forceinline__ uint16_t f2h(float f) { return __half_as_ushort(__float2half(f)); }

__device__ __forceinline__ int dot16(const int4 &a, const int4 &b, int c) {
    c = __builtin_amdgcn_sdot4(a.x, b.x, c, false);
    c = __builtin_amdgcn_sdot4(a.y, b.y, c, false);
    c = __builtin_amdgcn_sdot4(a.z, b.z, c, false);
    c = __builtin_amdgcn_sdot4(a.w, b.w, c, false);
    return c;
}

template <int W>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int o = W / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
template <int W>
__device__ __forceinline__ int group_sum_i(int v) {
#pragma unroll
    for (int o = W / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
template <int W>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
    for (int o = W / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// Workgroup-wide sum with a fixed combination order (deterministic).
__device__ __forceinline__ float wg_sum(float v, float *red) {
    v = group_sum<64>(v);
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    __syncthreads();
    if (lane == 0) red[w] = v;
    __syncthreads();
    float t = 0.0f;
    for (int i = 0; i < (int)(blockDim.x >> 6); i++) t += red[i];
    return t;
}

__device__ __forceinline__ int8_t sat_i8(float v) {
    v = fminf(fmaxf(v, -128.0f), 127.0f);
    return (int8_t)(int)v;
}

// quantize_input_q8_0_into for one 32-block (model.rs:5557-5570).
__device__ __forceinline__ void quant_block32(const float *v, int8_t *q, float *s, int *sum) {
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(v[j]));
    const float d = amax / 127.0f;
    const float id = (d != 0.0f) ? 127.0f / amax : 0.0f;
    int acc = 0;
    int packed[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        uint32_t p = 0;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            int8_t qq = sat_i8(roundf(v[4 * j + k] * id));
            acc += qq;
            p |= (uint32_t)(uint8_t)qq << (8 * k);
        }
        packed[j] = (int)p;
    }
    int4 *qd = (int4 *)q;
    qd[0] = make_int4(packed[0], packed[1], packed[2], packed[3]);
    qd[1] = make_int4(packed[4], packed[5], packed[6], packed[7]);
    *s = d;
    *sum = acc;
}

// ------------------------------------------------------------------------
// Input staging (prologues).  Every workgroup builds the activation it needs
// in LDS.  ORDER 0 = rmsnorm_quantize_q8_0_scalar ((x*w)*inv, model.rs:5615);
// ORDER 1 = rmsnorm_scalar_into ((x*inv)*w, model.rs:7474) then quantize.
// ------------------------------------------------------------------------
enum Pro { PRO_LOADQ = 0, PRO_NORMQ0 = 1, PRO_NORMQ1 = 2 };

__device__ __forceinline__ float wg_inv_rms(const float *x, int n, float eps, float *red) {
    float ss = 0.0f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) ss += x[i] * x[i];
    ss = wg_sum(ss, red);
    const float rms = sqrtf(ss / (float)n + eps);
    return 1.0f / rms;
}

template <int PRO>
__device__ __forceinline__ void stage_q8(const float *x, const float *w, float eps, int n,
                                         const int8_t *gq, const float *gs, const int *gsum,
                                         int8_t *lq, float *ls, int *lsum, float *red) {
    const int nb = n >> 5;
    if (PRO == PRO_LOADQ) {
        const int4 *src = (const int4 *)gq;
        int4 *dst = (int4 *)lq;
        for (int i = threadIdx.x; i < (n >> 4); i += blockDim.x) dst[i] = src[i];
        for (int i = threadIdx.x; i < nb; i += blockDim.x) {
            ls[i] = gs[i];
            lsum[i] = gsum[i];
        }
    } else {
        const float inv = wg_inv_rms(x, n, eps, red);
        for (int b = threadIdx.x; b < nb; b += blockDim.x) {
            float v[32];
            const float4 *xs = (const float4 *)(x + b * 32), *ws = (const float4 *)(w + b * 32);
#pragma unroll
            for (int j = 0; j < 8; j++) {
                float4 a = xs[j], c = ws[j];
                if (PRO == PRO_NORMQ0) {
                    v[4 * j + 0] = a.x * c.x * inv; v[4 * j + 1] = a.y * c.y * inv;
                    v[4 * j + 2] = a.z * c.z * inv; v[4 * j + 3] = a.w * c.w * inv;
                } else {
                    v[4 * j + 0] = (a.x * inv) * c.x; v[4 * j + 1] = (a.y * inv) * c.y;
                    v[4 * j + 2] = (a.z * inv) * c.z; v[4 * j + 3] = (a.w * inv) * c.w;
                }
            }
            quant_block32(v, lq + b * 32, ls + b, lsum + b);
        }
    }
    __syncthreads();
}

// ------------------------------------------------------------------------
// Row dots over a Q8-quantized input held in LDS.
// A "group" of LPR lanes cooperates on R rows; lane gl walks the row's units.
//   Q8_0 (re-laid-out): unit = one 32-block; weights int8 [rows][K] plus
//        f16 scales [rows][K/32].
//   Q4_K (GGUF bytes):  unit = one (superblock, sub) pair = 32 qs bytes,
//        i.e. 32 low-nibble weights of sub-block `sub` and 32 high-nibble
//        weights of sub-block `sub+4`.
// ------------------------------------------------------------------------
struct WDesc {
    const uint8_t *q;   // Q8_0: int8 quants; Q4_K: raw blocks; Q6_K: 208-B bodies; F32: floats
    const uint16_t *s;  // Q8_0: f16 block scales; Q6_K: f16 super-block d
    int rows, cols;
};

template <int LPR, int R>
__device__ __forceinline__ void rows_q8_0(const WDesc &W, const int *rix, const int8_t *lq,
                                          const float *ls, int gl, float *acc) {
    const int bpr = W.cols >> 5;
    for (int b = gl; b < bpr; b += LPR) {
        const int4 x0 = *(const int4 *)(lq + b * 32), x1 = *(const int4 *)(lq + b * 32 + 16);
        const float xs = ls[b];
        int4 w0[R], w1[R];
        uint16_t sc[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int4 *p = (const int4 *)(W.q + (size_t)rix[r] * W.cols + b * 32);
            w0[r] = p[0];
            w1[r] = p[1];
            sc[r] = W.s[(size_t)rix[r] * bpr + b];
        }
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int d = dot16(w1[r], x1, dot16(w0[r], x0, 0));
            const float combined = h2f(sc[r]) * xs;
            acc[r] += combined * (float)d;
        }
    }
}

__device__ __forceinline__ uint32_t byte_of(uint32_t w, int i) { return (w >> (8 * i)) & 0xFFu; }

template <int LPR, int R>
__device__ __forceinline__ void rows_q4k(const WDesc &W, const int *rix, const int8_t *lq,
                                         const float *ls, const int *lsum, int gl, float *acc) {
    const int nsb = W.cols >> 8;
    const int units = nsb * 4;
    const size_t rstride = (size_t)nsb * 144;
    for (int u = gl; u < units; u += LPR) {
        const int sb = u >> 2, sub = u & 3;
        const int blo = sb * 8 + sub, bhi = blo + 4;
        const int4 xl0 = *(const int4 *)(lq + blo * 32), xl1 = *(const int4 *)(lq + blo * 32 + 16);
        const int4 xh0 = *(const int4 *)(lq + bhi * 32), xh1 = *(const int4 *)(lq + bhi * 32 + 16);
        const float s_lo = ls[blo], s_hi = ls[bhi];
        const float qsum_lo = (float)lsum[blo], qsum_hi = (float)lsum[bhi];
        int4 hd[R], q0[R], q1[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint8_t *blk = W.q + (size_t)rix[r] * rstride + (size_t)sb * 144;
            hd[r] = *(const int4 *)blk;
            q0[r] = *(const int4 *)(blk + 16 + 32 * sub);
            q1[r] = *(const int4 *)(blk + 32 + 32 * sub);
        }
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint32_t h0 = (uint32_t)hd[r].x;
            const float d = h2f((uint16_t)(h0 & 0xFFFF)), dmin = h2f((uint16_t)(h0 >> 16));
            const uint32_t s_a = byte_of((uint32_t)hd[r].y, sub);   // scales[sub]
            const uint32_t s_b = byte_of((uint32_t)hd[r].z, sub);   // scales[sub+4]
            const uint32_t s_c = byte_of((uint32_t)hd[r].w, sub);   // scales[sub+8]
            const uint32_t sc_lo = s_a & 63, mn_lo = s_b & 63;
            const uint32_t sc_hi = (s_a >> 6) | ((s_c & 0xF) << 2);
            const uint32_t mn_hi = (s_b >> 6) | ((s_c >> 4) << 2);
            const int4 a = q0[r], c = q1[r];
            const int4 lo0 = make_int4(a.x & 0x0F0F0F0F, a.y & 0x0F0F0F0F, a.z & 0x0F0F0F0F, a.w & 0x0F0F0F0F);
            const int4 lo1 = make_int4(c.x & 0x0F0F0F0F, c.y & 0x0F0F0F0F, c.z & 0x0F0F0F0F, c.w & 0x0F0F0F0F);
            const int4 hi0 = make_int4((a.x >> 4) & 0x0F0F0F0F, (a.y >> 4) & 0x0F0F0F0F,
                                       (a.z >> 4) & 0x0F0F0F0F, (a.w >> 4) & 0x0F0F0F0F);
            const int4 hi1 = make_int4((c.x >> 4) & 0x0F0F0F0F, (c.y >> 4) & 0x0F0F0F0F,
                                       (c.z >> 4) & 0x0F0F0F0F, (c.w >> 4) & 0x0F0F0F0F);
            const int dl = dot16(lo1, xl1, dot16(lo0, xl0, 0));
            const int dh = dot16(hi1, xh1, dot16(hi0, xh0, 0));
            const float d_sc_lo = d * (float)sc_lo, dmin_mn_lo = dmin * (float)mn_lo;
            const float d_sc_hi = d * (float)sc_hi, dmin_mn_hi = dmin * (float)mn_hi;
            acc[r] += s_lo * (d_sc_lo * (float)dl - dmin_mn_lo * qsum_lo);
            acc[r] += s_hi * (d_sc_hi * (float)dh - dmin_mn_hi * qsum_hi);
        }
    }
}

template <int FMT, int LPR, int R>
__device__ __forceinline__ void rows_q8in(const WDesc &W, const int *rix, const int8_t *lq,
                                          const float *ls, const int *lsum, int gl, float *acc) {
    if (FMT == F_Q8_0)
        rows_q8_0<LPR, R>(W, rix, lq, ls, gl, acc);
    else
        rows_q4k<LPR, R>(W, rix, lq, ls, lsum, gl, acc);
}

// ------------------------------------------------------------------------
// Row dots over an f32 input in LDS (logits path: dequantized weight times
// the unquantized final_normed vector, matvec_argmax_f32 model.rs:8668).
//   Q8_0: w = (float)q * scale  (dequant_q8_0_block, quantize.rs:194)
//   Q6_K: unit = (superblock, half, l0) -> 64 weights;
//         w = d * sc * q       (dequant_q6k_block, quantize.rs:375-378)
//   F32 : unit = 32 floats
// ------------------------------------------------------------------------
template <int LPR, int R>
__device__ __forceinline__ void rows_f32in_q8_0(const WDesc &W, const int *rix, const float *lx,
                                                int gl, float *acc) {
    const int bpr = W.cols >> 5;
    for (int b = gl; b < bpr; b += LPR) {
        float xv[32];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            float4 t = *(const float4 *)(lx + b * 32 + 4 * j);
            xv[4 * j] = t.x; xv[4 * j + 1] = t.y; xv[4 * j + 2] = t.z; xv[4 * j + 3] = t.w;
        }
        int4 w0[R], w1[R];
        uint16_t sc[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int4 *p = (const int4 *)(W.q + (size_t)rix[r] * W.cols + b * 32);
            w0[r] = p[0];
            w1[r] = p[1];
            sc[r] = W.s[(size_t)rix[r] * bpr + b];
        }
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float scale = h2f(sc[r]);
            const int ws[8] = {w0[r].x, w0[r].y, w0[r].z, w0[r].w, w1[r].x, w1[r].y, w1[r].z, w1[r].w};
            float a = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; j++) {
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const float wv = (float)(int8_t)(ws[j] >> (8 * k)) * scale;
                    a += wv * xv[4 * j + k];
                }
            }
            acc[r] += a;
        }
    }
}

template <int LPR, int R>
__device__ __forceinline__ void rows_f32in_q6k(const WDesc &W, const int *rix, const float *lx,
                                               int gl, float *acc) {
    const int nsb = W.cols >> 8;
    const int units = nsb * 4;
    for (int u = gl; u < units; u += LPR) {
        const int sb = u >> 2, hf = (u >> 1) & 1, l0 = (u & 1) * 16;
        const int ebase = sb * 256 + hf * 128 + l0;
        int4 qa[R], qb[R], qh[R], scv[R];
        uint16_t dd[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint8_t *body = W.q + ((size_t)rix[r] * nsb + sb) * 208;
            qa[r] = *(const int4 *)(body + 64 * hf + l0);
            qb[r] = *(const int4 *)(body + 64 * hf + 32 + l0);
            qh[r] = *(const int4 *)(body + 128 + 32 * hf + l0);
            scv[r] = *(const int4 *)(body + 192);
            dd[r] = W.s[(size_t)rix[r] * nsb + sb];
        }
        const int is = l0 >> 4;
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float d = h2f(dd[r]);
            const uint32_t scw[4] = {(uint32_t)scv[r].x, (uint32_t)scv[r].y, (uint32_t)scv[r].z,
                                     (uint32_t)scv[r].w};
            const int so = hf * 8 + is;
            const float sc1 = (float)(int8_t)byte_of(scw[so >> 2], so & 3);
            const float sc2 = (float)(int8_t)byte_of(scw[(so + 2) >> 2], (so + 2) & 3);
            const float sc3 = (float)(int8_t)byte_of(scw[(so + 4) >> 2], (so + 4) & 3);
            const float sc4 = (float)(int8_t)byte_of(scw[(so + 6) >> 2], (so + 6) & 3);
            const float ds1 = d * sc1, ds2 = d * sc2, ds3 = d * sc3, ds4 = d * sc4;
            const uint32_t A[4] = {(uint32_t)qa[r].x, (uint32_t)qa[r].y, (uint32_t)qa[r].z, (uint32_t)qa[r].w};
            const uint32_t B[4] = {(uint32_t)qb[r].x, (uint32_t)qb[r].y, (uint32_t)qb[r].z, (uint32_t)qb[r].w};
            const uint32_t Hh[4] = {(uint32_t)qh[r].x, (uint32_t)qh[r].y, (uint32_t)qh[r].z, (uint32_t)qh[r].w};
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
            acc[r] += a;
        }
    }
}

template <int LPR, int R>
__device__ __forceinline__ void rows_f32in_f32(const WDesc &W, const int *rix, const float *lx,
                                               int gl, float *acc) {
    const int units = W.cols >> 2;
    const float *wf = (const float *)W.q;
    for (int u = gl; u < units; u += LPR) {
        const float4 xv = *(const float4 *)(lx + 4 * u);
        float4 wv[R];
#pragma unroll
        for (int r = 0; r < R; r++) wv[r] = *(const float4 *)(wf + (size_t)rix[r] * W.cols + 4 * u);
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] += wv[r].x * xv.x + wv[r].y * xv.y + wv[r].z * xv.z + wv[r].w * xv.w;
    }
}

template <int FMT, int LPR, int R>
__device__ __forceinline__ void rows_f32in(const WDesc &W, const int *rix, const float *lx, int gl,
                                           float *acc) {
    if (FMT == F_Q8_0)
        rows_f32in_q8_0<LPR, R>(W, rix, lx, gl, acc);
    else if (FMT == F_Q6K)
        rows_f32in_q6k<LPR, R>(W, rix, lx, gl, acc);
    else
        rows_f32in_f32<LPR, R>(W, rix, lx, gl, acc);
}

// Packed (value, index) key whose unsigned max is the first maximum:
// order-preserving float bits in the high word, ~index in the low word.
__device__ __forceinline__ unsigned long long argmax_key(float v, uint32_t idx) {
    uint32_t u = __float_as_uint(v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)u << 32) | (unsigned long long)(0xFFFFFFFFu - idx);
}

}  // namespace fl
