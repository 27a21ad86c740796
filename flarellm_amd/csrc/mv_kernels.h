// Quantized matvec kernels (batch-1 decode), gfx950 wave64.
//
// Work split: a workgroup of 256 threads is divided into groups of LPR lanes.
// A group works on "items" = (row group of R rows, unit chunk); lane gl owns
// units gl, gl+LPR, ..., gl+(U-1)*LPR of the chunk.  Workgroups stride over
// the items (persistent grid), keeping the next item's weights in flight
// while the current one is consumed.  Load order inside a workgroup:
//   1. the activation loads of the prologue (x / norm weight, or the
//      pre-quantized input),
//   2. the first weight tile,
//   3. prologue arithmetic (waits only for 1: vmcnt completes in order),
// so weight streaming starts before the prologue's RMSNorm/quantize runs.
// Row partial sums are reduced within the group with a fixed butterfly
// (deterministic); every per-block float term keeps the reference's operation
// order (built with -ffp-contract=off).
#pragma once

#include "kernels.h"

namespace fl {

enum Epi { EPI_STORE = 0, EPI_ADD = 1, EPI_ARGMAX = 2, EPI_QKV = 3 };

// EPI_QKV: the fused QKV matvec stores q (after RoPE) and writes the new
// token's K (after RoPE) and V straight into the KV cache.  The weight rows
// of every q / k head are uploaded pair-interleaved (row 2i = original row i,
// row 2i+1 = original row i + D/2), so each rotate-half pair of
// apply_rope_with_table (model.rs:7283-7296) lands in one tile.
struct QkvEpi {
    const float *rope;  // cos table [max_pos][D/2]; sin table at rope + sin_off
    long long sin_off;
    const int *posp;    // token position (device)
    void *kc, *vc;      // this layer's head-major cache [kv_head][slot][D]
    long long head_stride;  // elements between kv heads (max_seq * D)
    int nq, nk;         // q rows (Nq*D) and k rows (Nkv*D); v rows follow
    int hd;             // head_dim
    int kv_f16;         // cache element: 1 = binary16 (RNE), 0 = f32
};

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
    QkvEpi qkv;                // EPI_QKV
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
    long long *trace;  // FLARE_MV_TRACE builds: phase timestamps of workgroup 0
};

#ifdef FLARE_MV_TRACE
#define MV_TS(i)                                                                          \
    do {                                                                                  \
        if (a.trace && blockIdx.x == 0 && threadIdx.x == 0)                              \
            a.trace[i] = (long long)__builtin_amdgcn_s_memrealtime();                     \
    } while (0)
#else
#define MV_TS(i) \
    do {         \
    } while (0)
#endif

// ---------------------------------------------------------------------------
// Two-phase activation prologue.  Phase 1 (issue) loads this thread's share
// of the input into registers; phase 2 (finish) computes and writes LDS.
// NT = threads of the workgroup; E = elements per thread of the norm input
// (n == NT*E with E in {8, 16}); other n take the generic loop of stage_q8.
// ---------------------------------------------------------------------------
template <int NT>
struct StageQ8 {
    v4i_t qv[4];  // PRO_LOADQ: int8 quants (16 B each), scales, sums
    float sv[2];
    int sumv[2];
    v4f_t xv[4], wv[4];  // PRO_NORMQ*: x and norm weight

    // Loads are unconditional (indices clamped into range) so that they stay
    // in registers and in flight; finish() discards the clamped duplicates.
    __device__ __forceinline__ void issue(int pro, int n, const float *x, const float *w, const int8_t *gq,
                                          const float *gs, const int *gsum) {
        const int t = threadIdx.x;
        if (pro == PRO_LOADQ) {
            const int n16 = n >> 4, nb = n >> 5;
#pragma unroll
            for (int k = 0; k < 4; k++) qv[k] = ((const v4i_t *)gq)[min(t + k * NT, n16 - 1)];
#pragma unroll
            for (int k = 0; k < 2; k++) {
                const int j = min(t + k * NT, nb - 1);
                sv[k] = gs[j];
                sumv[k] = gsum[j];
            }
        } else {
            const int E = n / NT;
            if (n == NT * E && (E == 8 || E == 16)) {
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const int o = min(t * E + 4 * k, n - 4);
                    xv[k] = *(const v4f_t *)(x + o);
                    wv[k] = *(const v4f_t *)(w + o);
                }
            }
        }
    }

    __device__ __forceinline__ void finish(int pro, int n, float eps, const float *x, const float *w,
                                           int8_t *lq, float *ls, int *lsum, float *red) {
        const int t = threadIdx.x;
        if (pro == PRO_LOADQ) {
            const int n16 = n >> 4, nb = n >> 5;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int i = t + k * NT;
                if (i < n16) ((v4i_t *)lq)[i] = qv[k];
            }
#pragma unroll
            for (int k = 0; k < 2; k++) {
                const int j = t + k * NT;
                if (j < nb) {
                    ls[j] = sv[k];
                    lsum[j] = sumv[k];
                }
            }
            __syncthreads();
            return;
        }
        const int E = n / NT;
        if (!(n == NT * E && (E == 8 || E == 16))) {
            if (pro == PRO_NORMQ0) stage_q8<PRO_NORMQ0>(x, w, eps, n, nullptr, nullptr, nullptr, lq, ls, lsum, red);
            else stage_q8<PRO_NORMQ1>(x, w, eps, n, nullptr, nullptr, nullptr, lq, ls, lsum, red);
            return;
        }
        float xs[16], ws[16];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            xs[4 * k] = xv[k].x; xs[4 * k + 1] = xv[k].y; xs[4 * k + 2] = xv[k].z; xs[4 * k + 3] = xv[k].w;
            ws[4 * k] = wv[k].x; ws[4 * k + 1] = wv[k].y; ws[4 * k + 2] = wv[k].z; ws[4 * k + 3] = wv[k].w;
        }
        // sum of squares: per-thread sequential, then the workgroup tree
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < 16; j++)
            if (j < E) ss += xs[j] * xs[j];
        ss = wg_sum(ss, red);
        const float rms = sqrtf(ss / (float)n + eps);
        const float inv = 1.0f / rms;
        float v[16];
        float amax = 0.0f;
#pragma unroll
        for (int j = 0; j < 16; j++) {
            v[j] = 0.0f;
            if (j < E) {
                // rmsnorm_quantize_q8_0_scalar (x*w)*inv (model.rs:5615) or
                // rmsnorm_scalar_into (x*inv)*w (model.rs:7474)
                v[j] = (pro == PRO_NORMQ0) ? xs[j] * ws[j] * inv : (xs[j] * inv) * ws[j];
                amax = fmaxf(amax, fabsf(v[j]));
            }
        }
        // a 32-block spans 32/E consecutive lanes of one row
        if (E == 8) amax = row_max<4>(amax);
        else amax = row_max<2>(amax);
        const float d = amax / 127.0f;
        const float id = (d != 0.0f) ? 127.0f / amax : 0.0f;
        int qsum = 0;
        uint32_t packed[4] = {0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < 16; j++) {
            if (j < E) {
                const int8_t qq = sat_i8(roundf(v[j] * id));
                qsum += qq;
                packed[j >> 2] |= (uint32_t)(uint8_t)qq << (8 * (j & 3));
            }
        }
        if (E == 8) {
            ((v2i_t *)lq)[t] = v2i_t{(int)packed[0], (int)packed[1]};
            qsum += __shfl_xor(qsum, 1, 64);
            qsum += __shfl_xor(qsum, 2, 64);
            if ((t & 3) == 0) {
                ls[t >> 2] = d;
                lsum[t >> 2] = qsum;
            }
        } else {
            ((v4i_t *)lq)[t] = v4i_t{(int)packed[0], (int)packed[1], (int)packed[2], (int)packed[3]};
            qsum += __shfl_xor(qsum, 1, 64);
            if ((t & 1) == 0) {
                ls[t >> 1] = d;
                lsum[t >> 1] = qsum;
            }
        }
        __syncthreads();
    }
};

// f32 input staging (logits path): pro 0 copies x, pro 1 is rmsnorm_into.
template <int NT>
struct StageF32 {
    v4f_t xv[4], wv[4];
    __device__ __forceinline__ void issue(int pro, int n, const float *x, const float *w) {
        const int t = threadIdx.x, E = n / NT;
        if (n == NT * E && (E == 8 || E == 16)) {
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int o = min(t * E + 4 * k, n - 4);
                xv[k] = *(const v4f_t *)(x + o);
                wv[k] = *(const v4f_t *)((pro == 1 ? w : x) + o);  // w may be null for pro 0
            }
        }
    }
    __device__ __forceinline__ void finish(int pro, int n, float eps, const float *x, const float *w, float *lx,
                                           float *red) {
        const int t = threadIdx.x, E = n / NT;
        if (!(n == NT * E && (E == 8 || E == 16))) {
            if (pro == 1) {
                const float inv = wg_inv_rms(x, n, eps, red);
                for (int i = t; i < n; i += NT) lx[i] = (x[i] * inv) * w[i];
            } else {
                for (int i = t; i < n; i += NT) lx[i] = x[i];
            }
            __syncthreads();
            return;
        }
        float xs[16], ws[16];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            xs[4 * k] = xv[k].x; xs[4 * k + 1] = xv[k].y; xs[4 * k + 2] = xv[k].z; xs[4 * k + 3] = xv[k].w;
            ws[4 * k] = wv[k].x; ws[4 * k + 1] = wv[k].y; ws[4 * k + 2] = wv[k].z; ws[4 * k + 3] = wv[k].w;
        }
        float inv = 1.0f;
        if (pro == 1) {
            float ss = 0.0f;
#pragma unroll
            for (int j = 0; j < 16; j++)
                if (j < E) ss += xs[j] * xs[j];
            ss = wg_sum(ss, red);
            const float rms = sqrtf(ss / (float)n + eps);
            inv = 1.0f / rms;
        }
#pragma unroll
        for (int j = 0; j < 16; j++)
            if (j < E) lx[t * E + j] = (pro == 1) ? (xs[j] * inv) * ws[j] : xs[j];
        __syncthreads();
    }
};

// ---------------------------------------------------------------------------
// Weight tiles: U units x R rows of one lane, loaded with streaming 16-byte
// loads.  Out-of-range units are clamped to a valid address (their terms are
// masked at consume time, so no branch can sink the loads).
// ---------------------------------------------------------------------------
template <int FMT, int LPR, int U, int R>
struct Tile;

// Q8_0 (re-laid-out): unit = one 32-block; int8 quants [rows][K] + f16 scales.
template <int LPR, int U, int R>
struct Tile<F_Q8_0, LPR, U, R> {
    v4i_t w0[U][R], w1[U][R];
    uint16_t sc[U][R];
    __device__ __forceinline__ void load(const WDesc &W, const int *rix, int ubase) {
        const int bpr = W.cols >> 5;
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int b = min(ubase + u * LPR, bpr - 1);
#pragma unroll
            for (int r = 0; r < R; r++) {
                const v4i_t *p = (const v4i_t *)(W.q + (size_t)rix[r] * W.cols + b * 32);
                w0[u][r] = ld_stream(p);
                w1[u][r] = ld_stream(p + 1);
                sc[u][r] = W.s[(size_t)rix[r] * bpr + b];
            }
        }
    }
};

// matvec_q8_0_preq_into per-block term (model.rs:8082-8099)
template <int LPR, int U, int R>
__device__ __forceinline__ void tile_dot_q8(const Tile<F_Q8_0, LPR, U, R> &T, const WDesc &W, const int8_t *lq,
                                            const float *ls, const int *, int ubase, float *acc) {
    const int bpr = W.cols >> 5;
#pragma unroll
    for (int u = 0; u < U; u++) {
        const bool valid = ubase + u * LPR < bpr;
        const int b = valid ? ubase + u * LPR : bpr - 1;
        const v4i_t x0 = *(const v4i_t *)(lq + b * 32), x1 = *(const v4i_t *)(lq + b * 32 + 16);
        const float xs = ls[b];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int d = dot16(T.w1[u][r], x1, dot16(T.w0[u][r], x0, 0));
            const float combined = h2f(T.sc[u][r]) * xs;
            const float t = combined * (float)d;
            acc[r] += valid ? t : 0.0f;
        }
    }
}

template <int LPR, int U, int R>
__device__ __forceinline__ void tile_dot_f32(const Tile<F_Q8_0, LPR, U, R> &T, const WDesc &W, const float *lx,
                                             int ubase, float *acc) {
    const int bpr = W.cols >> 5;
#pragma unroll
    for (int u = 0; u < U; u++) {
        const bool valid = ubase + u * LPR < bpr;
        const int b = valid ? ubase + u * LPR : bpr - 1;
        // dequant_q8_0_block: (q as f32) * scale (quantize.rs:194), then the
        // f32 dot of matvec_argmax_f32; x is read from LDS one 16-B quarter
        // at a time (keeps the live register set small)
        float a[R];
#pragma unroll
        for (int r = 0; r < R; r++) a[r] = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const v4f_t xq = *(const v4f_t *)(lx + b * 32 + 4 * j);
#pragma unroll
            for (int r = 0; r < R; r++) {
                const float scale = h2f(T.sc[u][r]);
                const int wj = j < 4 ? T.w0[u][r][j] : T.w1[u][r][j - 4];
#pragma unroll
                for (int k = 0; k < 4; k++) a[r] += ((float)(int8_t)(wj >> (8 * k)) * scale) * xq[k];
            }
        }
#pragma unroll
        for (int r = 0; r < R; r++) {
            acc[r] += valid ? a[r] : 0.0f;
        }
    }
}

// Q4_K (GGUF bytes): unit = (superblock, sub) = 32 qs bytes holding the low
// nibbles of sub-block `sub` and the high nibbles of sub-block `sub+4`.
template <int LPR, int U, int R>
struct Tile<F_Q4K, LPR, U, R> {
    v4i_t hd[U][R], q0[U][R], q1[U][R];
    __device__ __forceinline__ void load(const WDesc &W, const int *rix, int ubase) {
        const int nsb = W.cols >> 8, units = nsb * 4;
        const size_t rstride = (size_t)nsb * 144;
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int uu = min(ubase + u * LPR, units - 1);
            const int sb = uu >> 2, sub = uu & 3;
#pragma unroll
            for (int r = 0; r < R; r++) {
                const uint8_t *blk = W.q + (size_t)rix[r] * rstride + (size_t)sb * 144;
                hd[u][r] = ld_stream(blk);
                q0[u][r] = ld_stream(blk + 16 + 32 * sub);
                q1[u][r] = ld_stream(blk + 32 + 32 * sub);
            }
        }
    }
};

// dot_q4k_q8_0_scalar per-sub-block terms (model.rs:8969-9025)
template <int LPR, int U, int R>
__device__ __forceinline__ void tile_dot_q8(const Tile<F_Q4K, LPR, U, R> &T, const WDesc &W, const int8_t *lq,
                                            const float *ls, const int *lsum, int ubase, float *acc) {
    const int units = (W.cols >> 8) * 4;
#pragma unroll
    for (int u = 0; u < U; u++) {
        const bool valid = ubase + u * LPR < units;
        const int uu = valid ? ubase + u * LPR : units - 1;
        const int sb = uu >> 2, sub = uu & 3;
        const int blo = sb * 8 + sub, bhi = blo + 4;
        const v4i_t xl0 = *(const v4i_t *)(lq + blo * 32), xl1 = *(const v4i_t *)(lq + blo * 32 + 16);
        const v4i_t xh0 = *(const v4i_t *)(lq + bhi * 32), xh1 = *(const v4i_t *)(lq + bhi * 32 + 16);
        const float s_lo = ls[blo], s_hi = ls[bhi];
        const float qsum_lo = (float)lsum[blo], qsum_hi = (float)lsum[bhi];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint32_t h0 = (uint32_t)T.hd[u][r].x;
            const float d = h2f((uint16_t)(h0 & 0xFFFF)), dmin = h2f((uint16_t)(h0 >> 16));
            // unpack_q4k_scales (model.rs:8709-8719) for sub and sub+4
            const uint32_t s_a = byte_of((uint32_t)T.hd[u][r].y, sub);  // scales[sub]
            const uint32_t s_b = byte_of((uint32_t)T.hd[u][r].z, sub);  // scales[sub+4]
            const uint32_t s_c = byte_of((uint32_t)T.hd[u][r].w, sub);  // scales[sub+8]
            const uint32_t sc_lo = s_a & 63, mn_lo = s_b & 63;
            const uint32_t sc_hi = (s_a >> 6) | ((s_c & 0xF) << 2);
            const uint32_t mn_hi = (s_b >> 6) | ((s_c >> 4) << 2);
            const v4i_t a = T.q0[u][r], c = T.q1[u][r];
            const v4i_t lo0 = v4i_t{a.x & 0x0F0F0F0F, a.y & 0x0F0F0F0F, a.z & 0x0F0F0F0F, a.w & 0x0F0F0F0F};
            const v4i_t lo1 = v4i_t{c.x & 0x0F0F0F0F, c.y & 0x0F0F0F0F, c.z & 0x0F0F0F0F, c.w & 0x0F0F0F0F};
            const v4i_t hi0 = v4i_t{(a.x >> 4) & 0x0F0F0F0F, (a.y >> 4) & 0x0F0F0F0F,
                                       (a.z >> 4) & 0x0F0F0F0F, (a.w >> 4) & 0x0F0F0F0F};
            const v4i_t hi1 = v4i_t{(c.x >> 4) & 0x0F0F0F0F, (c.y >> 4) & 0x0F0F0F0F,
                                       (c.z >> 4) & 0x0F0F0F0F, (c.w >> 4) & 0x0F0F0F0F};
            const int dl = dot16(lo1, xl1, dot16(lo0, xl0, 0));
            const int dh = dot16(hi1, xh1, dot16(hi0, xh0, 0));
            const float d_sc_lo = d * (float)sc_lo, dmin_mn_lo = dmin * (float)mn_lo;
            const float d_sc_hi = d * (float)sc_hi, dmin_mn_hi = dmin * (float)mn_hi;
            const float t_lo = s_lo * (d_sc_lo * (float)dl - dmin_mn_lo * qsum_lo);
            const float t_hi = s_hi * (d_sc_hi * (float)dh - dmin_mn_hi * qsum_hi);
            acc[r] += valid ? t_lo : 0.0f;
            acc[r] += valid ? t_hi : 0.0f;
        }
    }
}

// Q6_K (re-laid-out: 208-byte bodies + f16 d): unit = (superblock, half,
// l0 in {0,16}) -> 64 weights.
template <int LPR, int U, int R>
struct Tile<F_Q6K, LPR, U, R> {
    v4i_t qa[U][R], qb[U][R], qh[U][R], scv[U][R];
    uint16_t dd[U][R];
    __device__ __forceinline__ void load(const WDesc &W, const int *rix, int ubase) {
        const int nsb = W.cols >> 8, units = nsb * 4;
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int uu = min(ubase + u * LPR, units - 1);
            const int sb = uu >> 2, hf = (uu >> 1) & 1, l0 = (uu & 1) * 16;
#pragma unroll
            for (int r = 0; r < R; r++) {
                const uint8_t *body = W.q + ((size_t)rix[r] * nsb + sb) * 208;
                qa[u][r] = ld_stream(body + 64 * hf + l0);
                qb[u][r] = ld_stream(body + 64 * hf + 32 + l0);
                qh[u][r] = ld_stream(body + 128 + 32 * hf + l0);
                scv[u][r] = *(const v4i_t *)(body + 192);
                dd[u][r] = W.s[(size_t)rix[r] * nsb + sb];
            }
        }
    }
};

template <int LPR, int U, int R>
__device__ __forceinline__ void tile_dot_f32(const Tile<F_Q6K, LPR, U, R> &T, const WDesc &W, const float *lx,
                                             int ubase, float *acc) {
    const int units = (W.cols >> 8) * 4;
#pragma unroll
    for (int u = 0; u < U; u++) {
        const bool valid = ubase + u * LPR < units;
        const int uu = valid ? ubase + u * LPR : units - 1;
        const int sb = uu >> 2, hf = (uu >> 1) & 1, l0 = (uu & 1) * 16;
        const int ebase = sb * 256 + hf * 128 + l0;
        const int so = hf * 8 + (l0 >> 4);
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float d = h2f(T.dd[u][r]);
            const uint32_t scw[4] = {(uint32_t)T.scv[u][r].x, (uint32_t)T.scv[u][r].y, (uint32_t)T.scv[u][r].z,
                                     (uint32_t)T.scv[u][r].w};
            // dequant_q6k_block (quantize.rs:366-378): w = d * sc * q
            const float ds1 = d * (float)(int8_t)byte_of(scw[so >> 2], so & 3);
            const float ds2 = d * (float)(int8_t)byte_of(scw[(so + 2) >> 2], (so + 2) & 3);
            const float ds3 = d * (float)(int8_t)byte_of(scw[(so + 4) >> 2], (so + 4) & 3);
            const float ds4 = d * (float)(int8_t)byte_of(scw[(so + 6) >> 2], (so + 6) & 3);
            const uint32_t A[4] = {(uint32_t)T.qa[u][r].x, (uint32_t)T.qa[u][r].y, (uint32_t)T.qa[u][r].z,
                                   (uint32_t)T.qa[u][r].w};
            const uint32_t B[4] = {(uint32_t)T.qb[u][r].x, (uint32_t)T.qb[u][r].y, (uint32_t)T.qb[u][r].z,
                                   (uint32_t)T.qb[u][r].w};
            const uint32_t Hh[4] = {(uint32_t)T.qh[u][r].x, (uint32_t)T.qh[u][r].y, (uint32_t)T.qh[u][r].z,
                                    (uint32_t)T.qh[u][r].w};
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

// F32: unit = 4 floats.
template <int LPR, int U, int R>
struct Tile<F_F32, LPR, U, R> {
    v4f_t wv[U][R];
    __device__ __forceinline__ void load(const WDesc &W, const int *rix, int ubase) {
        const int units = W.cols >> 2;
        const float *wf = (const float *)W.q;
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int uu = min(ubase + u * LPR, units - 1);
#pragma unroll
            for (int r = 0; r < R; r++) wv[u][r] = ld_stream_f(wf + (size_t)rix[r] * W.cols + 4 * uu);
        }
    }
};

template <int LPR, int U, int R>
__device__ __forceinline__ void tile_dot_f32(const Tile<F_F32, LPR, U, R> &T, const WDesc &W, const float *lx,
                                             int ubase, float *acc) {
    const int units = W.cols >> 2;
#pragma unroll
    for (int u = 0; u < U; u++) {
        const bool valid = ubase + u * LPR < units;
        const int uu = valid ? ubase + u * LPR : units - 1;
        const v4f_t xv = *(const v4f_t *)(lx + 4 * uu);
#pragma unroll
        for (int r = 0; r < R; r++) {
            const v4f_t w = T.wv[u][r];
            const float t = w.x * xv.x + w.y * xv.y + w.z * xv.z + w.w * xv.w;
            acc[r] += valid ? t : 0.0f;
        }
    }
}

__host__ __device__ inline int fmt_units_per_row(int fmt, int cols) {
    return fmt == F_Q8_0 ? cols / 32 : (fmt == F_F32 ? cols / 4 : cols / 64);
}

// ---------------------------------------------------------------------------
// epilogue helpers
// ---------------------------------------------------------------------------
__device__ __forceinline__ unsigned long long umax64(unsigned long long a, unsigned long long b) {
    return a > b ? a : b;
}

template <int R>
__device__ __forceinline__ unsigned long long rows_best(const float *acc, int row0, int rows) {
    unsigned long long best = 0;
#pragma unroll
    for (int r = 0; r < R; r++)
        if (row0 + r < rows) best = umax64(best, argmax_key(acc[r], (uint32_t)(row0 + r)));
    return best;
}

// wave max -> workgroup max -> one device atomic (first maximum on ties)
__device__ __forceinline__ void wg_argmax_commit(unsigned long long best, unsigned long long *slot,
                                                 unsigned long long *lred) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) best = umax64(best, __shfl_xor(best, o, 64));
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) lred[w] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long b = lred[0];
        for (int i = 1; i < (int)(blockDim.x >> 6); i++) b = umax64(b, lred[i]);
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

// EPI_QKV store of a finished row group (R even, rows row0.. row0+R-1 in
// the pair-interleaved order); lane gl < R/2 handles pair gl.
template <int R>
__device__ __forceinline__ void store_qkv(const float *acc, int row0, int rows, int gl, const QkvEpi &e, int pos,
                                          float *q) {
    static_assert(R % 2 == 0, "EPI_QKV needs row pairs");
    if (gl >= R / 2) return;
    const int n = row0 + 2 * gl;  // first row of the pair (even)
    if (n >= rows) return;
    float x0 = acc[0], x1 = acc[1];
#pragma unroll
    for (int r = 2; r < R; r += 2) {
        x0 = (gl == r / 2) ? acc[r] : x0;
        x1 = (gl == r / 2) ? acc[r + 1] : x1;
    }
    const int D = e.hd, half = D >> 1;
    const int j = n % D, i = j >> 1;  // pair index within the head
    if (n < e.nq + e.nk) {
        const float c = e.rope[(size_t)pos * half + i], sn = e.rope[e.sin_off + (size_t)pos * half + i];
        const float y0 = x0 * c - x1 * sn, y1 = x0 * sn + x1 * c;
        if (n < e.nq) {
            const int h = n / D;
            q[h * D + i] = y0;
            q[h * D + i + half] = y1;
        } else {
            const int kvh = (n - e.nq) / D;
            const size_t off = (size_t)kvh * e.head_stride + (size_t)pos * D;
            if (e.kv_f16) {
                ((uint16_t *)e.kc)[off + i] = f2h(y0);
                ((uint16_t *)e.kc)[off + i + half] = f2h(y1);
            } else {
                ((float *)e.kc)[off + i] = y0;
                ((float *)e.kc)[off + i + half] = y1;
            }
        }
    } else {
        // v rows keep their original order
        const int vi = n - e.nq - e.nk, kvh = vi / D, d = vi % D;
        const size_t off = (size_t)kvh * e.head_stride + (size_t)pos * D + d;
        if (e.kv_f16) {
            ((uint16_t *)e.vc)[off] = f2h(x0);
            ((uint16_t *)e.vc)[off + 1] = f2h(x1);
        } else {
            ((float *)e.vc)[off] = x0;
            ((float *)e.vc)[off + 1] = x1;
        }
    }
}

__host__ __device__ inline size_t q8_lds_bytes(int K) { return (size_t)K + (size_t)(K / 32) * 8 + 64 * 4 + 64; }

// ---------------------------------------------------------------------------
// Persistent matvecs.  Items = (row group of R rows) x (unit chunk of
// LPR*U units); group grp of workgroup b walks items b*G+grp + k*stride and
// keeps the next item's tile in flight (ping-pong tiles ta / tb).
// ---------------------------------------------------------------------------
template <int FMT, int LPR, int U, int R>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 4))) void k_mv_q8in(Q8inArgs a) {
    extern __shared__ __align__(16) char smem[];
    const WDesc &W = a.W;
    const int K = W.cols;
    int8_t *lq = (int8_t *)smem;
    float *ls = (float *)(smem + K);
    int *lsum = (int *)(ls + (K >> 5));
    float *red = (float *)(lsum + (K >> 5));
    constexpr int G = kThreads / LPR;
    const int grp = threadIdx.x / LPR, gl = threadIdx.x % LPR;
    // local item li of this group = (row group gid + (li / nchunk) * stride,
    // chunk li % nchunk): all chunks of a row group stay in one group
    const int nchunk = (fmt_units_per_row(FMT, K) + LPR * U - 1) / (LPR * U);
    const int ngrp = (W.rows + R - 1) / R;
    const int gid = blockIdx.x * G + grp, stride = gridDim.x * G;
    const int nitems = gid < ngrp ? ((ngrp - 1 - gid) / stride + 1) * nchunk : 0;
    int it = 0;
    int rix[R];
    auto rows_of = [&](int li, int &rg, int &chunk) {
        const int k = li / nchunk;
        chunk = li - k * nchunk;
        rg = min(gid + k * stride, ngrp - 1);
#pragma unroll
        for (int r = 0; r < R; r++) rix[r] = min(rg * R + r, W.rows - 1);
    };

    const int qpos = a.epi == EPI_QKV ? *a.qkv.posp : 0;
    StageQ8<kThreads> stg;
    stg.issue(a.pro, K, a.x, a.nw, a.gq, a.gs, a.gsum);  // 1. activation loads
    Tile<FMT, LPR, U, R> ta, tb;
    int rg, ch;
    rows_of(0, rg, ch);
    ta.load(W, rix, ch * LPR * U + gl);                          // 2. first weight tile
    stg.finish(a.pro, K, a.eps, a.x, a.nw, lq, ls, lsum, red);  // 3. prologue arithmetic

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;
    unsigned long long best = 0;
    auto consume = [&](const Tile<FMT, LPR, U, R> &T, int item) {
        int rgc, chc;
        rows_of(item, rgc, chc);
        tile_dot_q8(T, W, lq, ls, lsum, chc * LPR * U + gl, acc);
        if (chc == nchunk - 1) {
#pragma unroll
            for (int r = 0; r < R; r++) acc[r] = group_sum<LPR>(acc[r]);
            if (a.epi == EPI_ARGMAX) best = umax64(best, rows_best<R>(acc, rgc * R, W.rows));
            else if constexpr (R % 2 == 0) {
                if (a.epi == EPI_QKV) store_qkv<R>(acc, rgc * R, W.rows, gl, a.qkv, qpos, a.out);
                else store_rows<R>(acc, rgc * R, W.rows, gl, a.epi, a.out);
            } else store_rows<R>(acc, rgc * R, W.rows, gl, a.epi, a.out);
#pragma unroll
            for (int r = 0; r < R; r++) acc[r] = 0.0f;
        }
    };
    // (a group with no next item must not prefetch: the clamped index would
    // stream the current tile a second time)
    while (it < nitems) {
        if (it + 1 < nitems) {
            rows_of(it + 1, rg, ch);
            tb.load(W, rix, ch * LPR * U + gl);
        }
        consume(ta, it);
        it += 1;
        if (it >= nitems) break;
        if (it + 1 < nitems) {
            rows_of(it + 1, rg, ch);
            ta.load(W, rix, ch * LPR * U + gl);
        }
        consume(tb, it);
        it += 1;
    }
    if (a.epi == EPI_ARGMAX) wg_argmax_commit(best, a.slot, (unsigned long long *)red);
}

template <int FMT, int LPR, int U, int R>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 4))) void k_mv_f32in(F32Args a) {
    extern __shared__ __align__(16) char smem[];
    const WDesc &W = a.W;
    const int K = W.cols;
    float *lx = (float *)smem;
    float *red = lx + K;
    constexpr int G = kThreads / LPR;
    const int grp = threadIdx.x / LPR, gl = threadIdx.x % LPR;
    // local item li of this group = (row group gid + (li / nchunk) * stride,
    // chunk li % nchunk): all chunks of a row group stay in one group
    const int nchunk = (fmt_units_per_row(FMT, K) + LPR * U - 1) / (LPR * U);
    const int ngrp = (W.rows + R - 1) / R;
    const int gid = blockIdx.x * G + grp, stride = gridDim.x * G;
    const int nitems = gid < ngrp ? ((ngrp - 1 - gid) / stride + 1) * nchunk : 0;
    int it = 0;
    int rix[R];
    auto rows_of = [&](int li, int &rg, int &chunk) {
        const int k = li / nchunk;
        chunk = li - k * nchunk;
        rg = min(gid + k * stride, ngrp - 1);
#pragma unroll
        for (int r = 0; r < R; r++) rix[r] = min(rg * R + r, W.rows - 1);
    };

    StageF32<kThreads> stg;
    stg.issue(a.pro, K, a.x, a.nw);
    Tile<FMT, LPR, U, R> ta, tb;
    int rg, ch;
    rows_of(0, rg, ch);
    ta.load(W, rix, ch * LPR * U + gl);
    stg.finish(a.pro, K, a.eps, a.x, a.nw, lx, red);

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;
    unsigned long long best = 0;
    auto consume = [&](const Tile<FMT, LPR, U, R> &T, int item) {
        int rgc, chc;
        rows_of(item, rgc, chc);
        tile_dot_f32(T, W, lx, chc * LPR * U + gl, acc);
        if (chc == nchunk - 1) {
#pragma unroll
            for (int r = 0; r < R; r++) acc[r] = group_sum<LPR>(acc[r]);
            if (a.epi == EPI_ARGMAX) best = umax64(best, rows_best<R>(acc, rgc * R, W.rows));
            else store_rows<R>(acc, rgc * R, W.rows, gl, EPI_STORE, a.out);
#pragma unroll
            for (int r = 0; r < R; r++) acc[r] = 0.0f;
        }
    };
    // (a group with no next item must not prefetch: the clamped index would
    // stream the current tile a second time)
    while (it < nitems) {
        if (it + 1 < nitems) {
            rows_of(it + 1, rg, ch);
            tb.load(W, rix, ch * LPR * U + gl);
        }
        consume(ta, it);
        it += 1;
        if (it >= nitems) break;
        if (it + 1 < nitems) {
            rows_of(it + 1, rg, ch);
            ta.load(W, rix, ch * LPR * U + gl);
        }
        consume(tb, it);
        it += 1;
    }
    if (a.epi == EPI_ARGMAX) wg_argmax_commit(best, a.slot, (unsigned long long *)red);
}

// Fused gate/up matvec over W = [w_gate; w_up] with the SiLU(gate)*up
// (model.rs:9788-9795) and quantize_input_q8_0 (5557-5570) epilogue.
// Block b (32 hidden values) = gate rows [32b, 32b+32) and up rows
// [F+32b, F+32b+32): NT/LPR groups each own RH gate rows and the matching RH
// up rows (R = 2*RH).  Workgroups stride over the F/32 blocks, prefetching
// the next block's tile; the trip count is uniform within a workgroup.
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
    constexpr int G = NT / LPR;
    constexpr int R = 64 / G;
    constexpr int RH = R / 2;
    static_assert(RH >= 1, "gate_up needs >= 2 rows per group");
    const int grp = threadIdx.x / LPR, gl = threadIdx.x % LPR;
    const int nblk = a.F / 32;
    int blk = blockIdx.x;
    int rix[R];
    auto rows_of = [&](int b) {
        const int i0 = b * 32 + grp * RH;
#pragma unroll
        for (int r = 0; r < R; r++) rix[r] = (r < RH) ? (i0 + r) : (a.F + i0 + r - RH);
    };

    MV_TS(0);
    StageQ8<NT> stg;
    stg.issue(a.pro, K, a.x, a.nw, a.gq, a.gs, a.gsum);
    Tile<FMT, LPR, U, R> ta, tb;
    rows_of(min(blk, nblk - 1));
    ta.load(W, rix, gl);
    MV_TS(1);
    stg.finish(a.pro, K, a.eps, a.x, a.nw, lq, ls, lsum, red);
    MV_TS(2);

    int nround = 0;
    auto consume = [&](const Tile<FMT, LPR, U, R> &T, int b) {
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] = 0.0f;
        tile_dot_q8(T, W, lq, ls, lsum, gl, acc);
        if (nround == 0) MV_TS(3);
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
            if (a.hout) a.hout[b * 32 + j] = h;
            quant_block32_lanes(h, a.hq + b * 32, a.hs + b, a.hsum + b);
        }
        __syncthreads();  // gu reused by the next block
        if (nround == 0) MV_TS(4);
        nround++;
    };
    while (blk < nblk) {
        if (blk + (int)gridDim.x < nblk) {
            rows_of(blk + (int)gridDim.x);
            tb.load(W, rix, gl);
        }
        consume(ta, blk);
        blk += gridDim.x;
        if (blk >= nblk) break;
        if (blk + (int)gridDim.x < nblk) {
            rows_of(blk + (int)gridDim.x);
            ta.load(W, rix, gl);
        }
        consume(tb, blk);
        blk += gridDim.x;
    }
    MV_TS(5);
}

}  // namespace fl
