// Output projection with an f32 input on f16 MFMA (the logits path of
// forward_greedy, flare-core/src/model.rs:1917-1931: matvec_argmax_f32 over
// the dequantized Q6_K output / tied Q8_0 embedding, model.rs:8668-8689).
//
// The RMS-normed input of up to 8 tokens (rmsnorm_into, model.rs:7456-7477)
// sits in LDS as f16 high parts and f16 residuals (x = hi + lo to ~22 bits);
// weight codes are exact in f16 (Q6_K: q - 32 in -32..31; Q8_0: int8), so
// every MFMA product is exact in fp32 and the per-block scale (Q6_K d*sc per
// 16 values, Q8_0 d per 32) multiplies the block's MFMA sum in fp32.
//   Q6_K: v_mfma_f32_16x16x16_f16, one 16-value sub-block of 16 rows.
//   Q8_0: v_mfma_f32_16x16x32_f16, one 32-value block of 16 rows.
// Tile rows: lane l owns weight row l%16 of the tile; MFMA rows are
// (token, hi / lo), so lane group l/16 collects tokens 2(l/16), 2(l/16)+1.
// Epilogue: logits store, or first-max argmax per token (packed u64 max).
#pragma once

#include "mv_kernels.h"

namespace fl {

typedef _Float16 v4h_t __attribute__((ext_vector_type(4)));
typedef _Float16 v8h2_t __attribute__((ext_vector_type(8)));
typedef float v4fm_t __attribute__((ext_vector_type(4)));

constexpr int kMvoThreads = 512;  // 8 waves
constexpr int kMvoMaxTokens = 8;

struct MvoArgs {
    WDesc W;
    const float *x;   // [M][K] input rows (before the norm)
    const float *nw;  // norm weight [K] (nullptr: no norm, x used as is)
    float eps;
    int M;
    int epi;          // EPI_STORE or EPI_ARGMAX
    float *out;       // EPI_STORE: [M][rows]
    unsigned long long *slots;  // EPI_ARGMAX: [M] packed (value, index) keys
};

__device__ __forceinline__ v4fm_t mfma_k16(const v4h_t &a, const v4h_t &b, const v4fm_t &c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ v4fm_t mfma_k32(const v8h2_t &a, const v8h2_t &b, const v4fm_t &c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// 4 six-bit Q6_K codes (bytes of w, 0..63) -> f16 (code - 32), exact:
// binary16 0x6400 | c is 1024 + c; subtracting 1056 leaves c - 32.
__device__ __forceinline__ v4h_t q6_codes_to_h4(uint32_t w) {
    const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, w, 0x07010700u);  // bytes c0, 0x64, c1, 0x64
    const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, w, 0x07030702u);  // bytes c2, 0x64, c3, 0x64
    v4h_t r;
    uint32_t u[2] = {lo, hi};
    __builtin_memcpy(&r, u, 8);
    const v4h_t bias = {(_Float16)1056.0f, (_Float16)1056.0f, (_Float16)1056.0f, (_Float16)1056.0f};
    return r - bias;
}

// 8 int8 codes -> f16, exact
__device__ __forceinline__ v8h2_t i8_codes_to_h8(uint32_t w0, uint32_t w1) {
    v8h2_t r;
#pragma unroll
    for (int i = 0; i < 8; i++) r[i] = (_Float16)(int8_t)(((i < 4 ? w0 : w1) >> (8 * (i & 3))) & 0xFFu);
    return r;
}

// Q6_K super-block data of one lane: row n, value group kg (4 values of each
// 16-value sub-block).  Llama.cpp layout (quantize.rs:343-384): value
// e = 128 hf + 32 g + l: ql byte 64 hf + 32 (g & 1) + l (low nibble g < 2),
// qh byte 32 hf + l (bits 2g), scale sc[8 hf + l / 16 + 2 g].
struct Q6Lane {
    uint32_t ql[2][2][2];  // [hf][g & 1][l0 half] 4 bytes
    uint32_t qh[2][2];     // [hf][l0 half]
    v4i_t sc;              // 16 int8 scales of the row's super-block
    uint16_t d;
    __device__ __forceinline__ void load(const WDesc &W, int row, int sb, int kg) {
        const int nsb = W.cols >> 8;
        const size_t rs = (size_t)row * nsb + sb;
        const uint8_t *qlp = W.q + rs * 128 + 4 * kg, *qhp = W.h + rs * 64 + 4 * kg;
#pragma unroll
        for (int hf = 0; hf < 2; hf++)
#pragma unroll
            for (int h16 = 0; h16 < 2; h16++) {
                qh[hf][h16] = *(const uint32_t *)(qhp + 32 * hf + 16 * h16);
#pragma unroll
                for (int g1 = 0; g1 < 2; g1++) ql[hf][g1][h16] = *(const uint32_t *)(qlp + 64 * hf + 32 * g1 + 16 * h16);
            }
        sc = *(const v4i_t *)(W.h2 + rs * 16);
        d = W.s[rs];
    }
};

template <int FMT>
__global__ __launch_bounds__(kMvoThreads) void k_mvo(MvoArgs a) {
    extern __shared__ __align__(16) char smem[];
    const WDesc &W = a.W;
    const int K = W.cols, M = a.M;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, kg = lane >> 4, r16 = lane & 15;
    constexpr int NW = kMvoThreads / 64;
    // LDS: rows m = 2t + (hi / lo) of the normed input as f16, [2*M][K]
    _Float16 *xa = (_Float16 *)smem;
    float *red = (float *)(smem + (size_t)2 * M * K * 2);  // [NW]
    // ---- prologue: rmsnorm_into per token, split into f16 hi / lo ----------
    for (int t = 0; t < M; t++) {
        const float *x = a.x + (size_t)t * K;
        float inv = 1.0f;
        if (a.nw) inv = wg_inv_rms(x, K, a.eps, red);
        for (int i = threadIdx.x; i < K; i += blockDim.x) {
            const float v = a.nw ? (x[i] * inv) * a.nw[i] : x[i];
            // high part rounded toward zero by v_cvt_pkrtz (the compiler
            // cannot re-form it from the product, so hi and the residual
            // come from the same fp32 v)
            const auto h2 = __builtin_amdgcn_cvt_pkrtz(v, 0.0f);
            _Float16 h;
            __builtin_memcpy(&h, &h2, 2);
            xa[(size_t)(2 * t) * K + i] = h;
            xa[(size_t)(2 * t + 1) * K + i] = (_Float16)(v - (float)h);
        }
        __syncthreads();  // red is reused by the next token
    }
    // A operand row of this lane: m = r16 (token m/2, hi/lo m%2); rows >= 2M are zero
    const bool arow = r16 < 2 * M;
    const _Float16 *xrow = xa + (size_t)(arow ? r16 : 0) * K;

    const int ntiles = (W.rows + 15) / 16;
    const int gw = blockIdx.x * NW + wave, tw = gridDim.x * NW;
    unsigned long long best[2] = {0ull, 0ull};
    for (int tile = gw; tile < ntiles; tile += tw) {
        const int n = tile * 16 + r16, row = min(n, W.rows - 1);
        float acc[2] = {0.0f, 0.0f};  // tokens 2kg, 2kg+1
        if constexpr (FMT == F_Q6K) {
            const int nsb = K >> 8;
            Q6Lane ta, tb;
            ta.load(W, row, 0, kg);
            pingpong(
                nsb, ta, tb, [&](Q6Lane &T, int sb) { T.load(W, row, sb, kg); },
                [&](Q6Lane &cur, int sb) {
                    const float d = h2f(cur.d);
                    const uint32_t scw[4] = {(uint32_t)cur.sc.x, (uint32_t)cur.sc.y, (uint32_t)cur.sc.z,
                                             (uint32_t)cur.sc.w};
#pragma unroll
                    for (int hf = 0; hf < 2; hf++)
#pragma unroll
                        for (int g = 0; g < 4; g++)
#pragma unroll
                            for (int h16 = 0; h16 < 2; h16++) {
                                const uint32_t qlw = cur.ql[hf][g & 1][h16], qhw = cur.qh[hf][h16];
                                const uint32_t codes = ((qlw >> (4 * (g >> 1))) & 0x0F0F0F0Fu) |
                                                       (((qhw >> (2 * g)) & 0x03030303u) << 4);
                                const v4h_t b = q6_codes_to_h4(codes);
                                const int col = sb * 256 + hf * 128 + g * 32 + h16 * 16 + 4 * kg;
                                v4h_t av = {(_Float16)0.0f, (_Float16)0.0f, (_Float16)0.0f, (_Float16)0.0f};
                                if (arow) av = *(const v4h_t *)(xrow + col);
                                const v4fm_t dd = mfma_k16(av, b, v4fm_t{0.f, 0.f, 0.f, 0.f});
                                const int si = hf * 8 + h16 + 2 * g;
                                const float s = d * (float)(int8_t)((scw[si >> 2] >> (8 * (si & 3))) & 0xFFu);
                                acc[0] += s * (dd[0] + dd[1]);
                                acc[1] += s * (dd[2] + dd[3]);
                            }
                });
        } else {  // Q8_0
            const int nb = K >> 5;
            const int8_t *wq = (const int8_t *)W.q + (size_t)row * K + 8 * kg;
            const uint16_t *ws = W.s + (size_t)row * nb;
            struct Q8Blk {
                v2i_t w;
                uint16_t s;
            } ta, tb;
            auto ld = [&](Q8Blk &T, int b) {
                T.w = *(const v2i_t *)(wq + 32 * b);
                T.s = ws[b];
            };
            ld(ta, 0);
            pingpong(nb, ta, tb, ld, [&](Q8Blk &T, int b) {
                const v8h2_t bv = i8_codes_to_h8((uint32_t)T.w.x, (uint32_t)T.w.y);
                v8h2_t av;
#pragma unroll
                for (int i = 0; i < 8; i++) av[i] = (_Float16)0.0f;
                if (arow) av = *(const v8h2_t *)(xrow + 32 * b + 8 * kg);
                const v4fm_t dd = mfma_k32(av, bv, v4fm_t{0.f, 0.f, 0.f, 0.f});
                const float s = h2f(T.s);
                acc[0] += s * (dd[0] + dd[1]);
                acc[1] += s * (dd[2] + dd[3]);
            });
        }
        // epilogue for row n, tokens 2kg + e
#pragma unroll
        for (int e = 0; e < 2; e++) {
            const int t = 2 * kg + e;
            if (t < M && n < W.rows) {
                if (a.epi == EPI_STORE) a.out[(size_t)t * W.rows + n] = acc[e];
                else best[e] = umax64(best[e], argmax_key(acc[e], (uint32_t)n));
            }
        }
    }
    if (a.epi == EPI_ARGMAX) {
        // per token: max over the 16 rows (lanes of one kg group), then the
        // workgroup, then one device atomic per token
        __shared__ unsigned long long lb[NW][kMvoMaxTokens];
#pragma unroll
        for (int e = 0; e < 2; e++) {
#pragma unroll
            for (int o = 1; o < 16; o <<= 1) best[e] = umax64(best[e], __shfl_xor(best[e], o, 64));
            if (r16 == 0 && 2 * kg + e < kMvoMaxTokens) lb[wave][2 * kg + e] = best[e];
        }
        __syncthreads();
        if (threadIdx.x < M) {
            unsigned long long b = lb[0][threadIdx.x];
            for (int w = 1; w < NW; w++) b = umax64(b, lb[w][threadIdx.x]);
            atomicMax(a.slots + threadIdx.x, b);
        }
    }
}

}  // namespace fl
