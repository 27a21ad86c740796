// Speculative-verify batch (M <= 16 draft tokens through the model in one
// pass): quantized GEMMs on int8 MFMA plus the per-token glue kernels.
//
// The reference verifies drafts one forward pass at a time
// (Generator::speculative_step, flare-core/src/generate.rs:244-312) and runs
// batched projections as one quantized matvec per token
// (CpuBackend::batched_dequant_matmul, flare-core/src/model.rs:740-1036: each
// row quantized by quantize_input_q8_0_into, then the single-token
// per-block integer dots).  Here the M tokens share each weight read: one
// v_mfma_i32_16x16x32_i8 forms the exact 32-value block dot of 16 weight rows
// with all M tokens at once, and the fp32 block terms follow the reference's
// per-block formulas.
#pragma once

#include "verify_args.h"
#include "attm_kernels.h"  // split8, mfma16 (f16 MFMA helpers)

namespace fl {

// LDS staging of one K chunk: int8 activations of the M tokens, then
// (scale, block sum as float) pairs.
// Every load of a round goes out before the first LDS store, so a round
// costs one L2 round trip.
// T8: (scale, sum) pairs block-major, 8 tokens per block ([b][8]); else
// token-major ([t][nb]).  SQ: the second member is scale * sum instead.
template <int FMT, bool T8 = false, bool SQ = false>
__device__ __forceinline__ void vg_stage(const VgArgs &a, int k0, int kn, int8_t *lx, float2 *lsc, int xs = 0) {
    if (!xs) xs = kn;  // LDS row stride of the activations
    constexpr int U = 8;
    const int K = a.W.cols, nb = kn >> 5, b0 = k0 >> 5;
    const int nx = a.M * (kn >> 3), ns = a.M * nb;
    for (int base = threadIdx.x; base < nx; base += U * blockDim.x) {
        i64x1_t v[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int i = base + u * blockDim.x;
            const int t = i / (kn >> 3), o = (i % (kn >> 3)) * 8;
            if (i < nx) v[u] = *(const i64x1_t *)(a.xq + (size_t)t * K + k0 + o);
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int i = base + u * blockDim.x;
            const int t = i / (kn >> 3), o = (i % (kn >> 3)) * 8;
            if (i < nx) *(i64x1_t *)(lx + t * xs + o) = v[u];
        }
    }
    for (int base = threadIdx.x; base < ns; base += 4 * blockDim.x) {
        float sv[4];
        int mv[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int i = base + u * blockDim.x;
            const int t = i / nb, b = i % nb;
            if (i < ns) {
                sv[u] = a.xs[(size_t)t * (K >> 5) + b0 + b];
                mv[u] = a.xsum[(size_t)t * (K >> 5) + b0 + b];
            }
        }
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int i = base + u * blockDim.x;
            if (i < ns) lsc[T8 ? (i % nb) * 8 + i / nb : i] = make_float2(sv[u], SQ ? sv[u] * (float)mv[u] : (float)mv[u]);
        }
    }
    __syncthreads();
}

// D[token][row] = sum_k X[token][k] * W[row][k] for one 32-value block.
// Lane l: A = X[t = l%16][8*(l/16) .. +8], B = W[row = l%16][8*(l/16) .. +8],
// D[i] = token 4*(l/16)+i, row l%16.
__device__ __forceinline__ v4i32_t vg_mfma(i64x1_t a, i64x1_t b) {
    const v4i32_t z = {0, 0, 0, 0};
    return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, z, 0, 0, 0);
}

// Testing readback of one per-block integer dot (VgArgs::dots).
__device__ __forceinline__ void vg_dot_out(const VgArgs &a, int t, int n, int blk, int v) {
    if (t < a.M && n < a.W.rows) a.dots[((size_t)t * a.W.rows + n) * (a.W.cols >> 5) + blk] = v;
}

// Q8_0 weights: unit = one 32-block.  Block term of matvec_q8_0_preq_into
// (model.rs:8082-8099): (f16(w_scale) * x_scale) * (int dot as f32).
// NT token tiles of 16 (M <= 16 NT): each weight fragment feeds NT MFMAs.
// Activation rows sit xst = kn + 32 bytes apart in LDS (the 16 lanes of a
// tile read distinct banks).
template <int NT>
__global__ __launch_bounds__(256) void k_vgemm_q8_0(VgArgs a) {
    extern __shared__ __align__(16) char smem[];
    const WDesc &W = a.W;
    const int K = W.cols, nbk = K >> 5;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int chunk = a.chunk;
    const int b0 = blockIdx.y * chunk, b1 = min(nbk, b0 + chunk);
    if (b0 >= b1) return;
    const int kn = (b1 - b0) * 32, xst = a.chunk * 32 + 32;
    int8_t *lx = (int8_t *)smem;
    float2 *lsc = (float2 *)(smem + ((a.M * xst + 15) & ~15));
    vg_stage<F_Q8_0>(a, b0 * 32, kn, lx, lsc, xst);
    const int tile = blockIdx.x * 4 + wave;
    if (tile * 16 >= W.rows) return;
    const int n = tile * 16 + (lane & 15), kg = lane >> 4, tA = lane & 15;
    const int row = min(n, W.rows - 1);
    const int nbc = b1 - b0;
    float acc[NT][4];
#pragma unroll
    for (int tt = 0; tt < NT; tt++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[tt][i] = 0.f;
    const int8_t *wq = (const int8_t *)W.q + (size_t)row * K + 8 * kg;
    const uint16_t *ws = W.s + (size_t)row * nbk;
    i64x1_t wn = *(const i64x1_t *)(wq + 32 * b0);
    uint16_t sn = ws[b0];
    for (int b = b0; b < b1; b++) {
        const i64x1_t wcur = wn;
        const uint16_t scur = sn;
        if (b + 1 < b1) {
            wn = *(const i64x1_t *)(wq + 32 * (b + 1));
            sn = ws[b + 1];
        }
        const int bl = b - b0;
        const float wsc = h2f(scur);
#pragma unroll
        for (int tt = 0; tt < NT; tt++) {
            const int tx = tA + 16 * tt;
            const i64x1_t x = tx < a.M ? *(const i64x1_t *)(lx + tx * xst + 32 * bl + 8 * kg) : 0;
            const v4i32_t d = vg_mfma(x, wcur);
            if (a.dots)
#pragma unroll
                for (int i = 0; i < 4; i++) vg_dot_out(a, 16 * tt + 4 * kg + i, n, b, d[i]);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int t = 16 * tt + 4 * kg + i;
                if (t < a.M) acc[tt][i] = __builtin_fmaf(wsc * lsc[t * nbc + bl].x, (float)d[i], acc[tt][i]);
            }
        }
    }
    if (n < W.rows) {
#pragma unroll
        for (int tt = 0; tt < NT; tt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int t = 16 * tt + 4 * kg + i;
                if (t < a.M) a.part[((size_t)blockIdx.y * a.M + t) * W.rows + n] = acc[tt][i];
            }
    }
}

// Q4_K weights (flarellm layout): unit = one 256-value super-block, 8 MFMAs
// per token tile (sub-block j: low nibbles of qs[32j..32j+32) for j < 4,
// high nibbles of qs[32(j-4)..] for j >= 4).  Block term of
// dot_q4k_q8_0_scalar (model.rs:8969-9025): s_x * (d*sc*dot - dmin*mn*sum(q_x)).
// NT token tiles of 16 as in k_vgemm_q8_0.
template <int NT>
__global__ __launch_bounds__(256) void k_vgemm_q4k(VgArgs a) {
    extern __shared__ __align__(16) char smem[];
    const WDesc &W = a.W;
    const int K = W.cols, nsb = K >> 8;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int chunk = a.chunk;
    const int s0 = blockIdx.y * chunk, s1 = min(nsb, s0 + chunk);
    if (s0 >= s1) return;
    const int kn = (s1 - s0) * 256, nbc = kn >> 5, xst = a.chunk * 256 + 32;
    int8_t *lx = (int8_t *)smem;
    float2 *lsc = (float2 *)(smem + ((a.M * xst + 15) & ~15));
    const int tile = blockIdx.x * 4 + wave;
    const int n = tile * 16 + (lane & 15), kg = lane >> 4, tA = lane & 15;
    const int row = min(n, W.rows - 1);
    float acc[NT][4];
#pragma unroll
    for (int tt = 0; tt < NT; tt++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[tt][i] = 0.f;
    const uint8_t *qs = W.q + (size_t)row * nsb * 128 + 8 * kg;
    const uint8_t *hd = W.h + (size_t)row * nsb * 16;
    auto load = [&](int sb, i64x1_t *w, v4i_t &h) {
#pragma unroll
        for (int jj = 0; jj < 4; jj++) w[jj] = *(const i64x1_t *)(qs + (size_t)sb * 128 + 32 * jj);
        h = *(const v4i_t *)(hd + (size_t)sb * 16);
    };
    i64x1_t wn[4];
    v4i_t hn;
    load(s0, wn, hn);
    vg_stage<F_Q4K>(a, s0 * 256, kn, lx, lsc, xst);
    if (tile * 16 >= W.rows) return;
    for (int sb = s0; sb < s1; sb++) {
        i64x1_t w[4];
        const v4i_t h = hn;
#pragma unroll
        for (int jj = 0; jj < 4; jj++) w[jj] = wn[jj];
        if (sb + 1 < s1) load(sb + 1, wn, hn);
        const uint32_t h0 = (uint32_t)h.x;
        const float d = h2f((uint16_t)(h0 & 0xFFFF)), dmin = h2f((uint16_t)(h0 >> 16));
        const int sl = sb - s0;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int jj = j & 3;
            const i64x1_t m4 = 0x0F0F0F0F0F0F0F0FLL;
            const i64x1_t wb = j < 4 ? (w[jj] & m4) : ((w[jj] >> 4) & m4);
            // unpack_q4k_scales (model.rs:8709-8719), flare packing
            const uint32_t sa = byte_of((uint32_t)h.y, jj), sbb = byte_of((uint32_t)h.z, jj),
                           scc = byte_of((uint32_t)h.w, jj);
            const uint32_t sc = j < 4 ? (sa & 63) : ((sa >> 6) | ((scc & 0xF) << 2));
            const uint32_t mn = j < 4 ? (sbb & 63) : ((sbb >> 6) | ((scc >> 4) << 2));
            const float dsc = d * (float)sc, dmn = dmin * (float)mn;
            const int bl = sl * 8 + j;
#pragma unroll
            for (int tt = 0; tt < NT; tt++) {
                const int tx = tA + 16 * tt;
                const i64x1_t x = tx < a.M ? *(const i64x1_t *)(lx + tx * xst + sl * 256 + 32 * j + 8 * kg) : 0;
                const v4i32_t dd = vg_mfma(x, wb);
                if (a.dots)
#pragma unroll
                    for (int i = 0; i < 4; i++) vg_dot_out(a, 16 * tt + 4 * kg + i, n, sb * 8 + j, dd[i]);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int t = 16 * tt + 4 * kg + i;
                    if (t < a.M) {
                        const float2 xs = lsc[t * nbc + bl];
                        acc[tt][i] += xs.x * (dsc * (float)dd[i] - dmn * xs.y);
                    }
                }
            }
        }
    }
    if (n < W.rows) {
#pragma unroll
        for (int tt = 0; tt < NT; tt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int t = 16 * tt + 4 * kg + i;
                if (t < a.M) a.part[((size_t)blockIdx.y * a.M + t) * W.rows + n] = acc[tt][i];
            }
    }
}

// ---------------------------------------------------------------------------
// Prefill GEMM, 17..64 tokens (kPrefillTokens): each wave owns 16 weight rows
// and all four 16-token tiles, so every weight fragment read from HBM feeds
// four MFMAs.  K is walked in 256-value steps (one Q4_K super-block, or eight
// Q8_0 blocks); the 64 activation rows of a step (16 KB of codes plus the
// (scale, sum) pairs) are staged through a double-buffered LDS slot, the next
// step's loads in flight while this one is consumed, so the LDS footprint
// does not grow with K.  Same per-block terms as k_vgemm_q8_0 / k_vgemm_q4k.
// ---------------------------------------------------------------------------
// LDS row stride of one step's codes: 68 dwords, so the 8-byte MFMA operand
// reads of 16 token rows (dword 68 t + 2 kg) fall on distinct banks
constexpr int kPgStride = 256 + 16;
// plane stride of the [block][token] scale arrays: 80 floats, so the min-term
// reads (block kg, token tA) and the staging stores spread over the banks
constexpr int kPgPlane = 80;

// One step's activation pieces in registers, staged by NT threads: 1024
// pieces of 16 code bytes (token i / 16, bytes 16 (i % 16)) and 512
// (scale, scale * code sum) pairs (token i / 8, block i % 8).
template <int NT>
struct PgStage {
    static constexpr int QN = 1024 / NT, SN = 512 / NT;
    v4i_t q[QN];
    float2 sc[SN];
};

template <int NT>
__device__ __forceinline__ void pg_load(const VgArgs &a, int k0, PgStage<NT> &r) {
    const int K = a.W.cols, t = threadIdx.x;
#pragma unroll
    for (int u = 0; u < PgStage<NT>::QN; u++) {
        const int i = t + NT * u;
        const int tok = min(i >> 4, a.M - 1);
        r.q[u] = *(const v4i_t *)(a.xq + (size_t)tok * K + k0 + 16 * (i & 15));
    }
#pragma unroll
    for (int u = 0; u < PgStage<NT>::SN; u++) {
        const int i = t + NT * u;
        const int tok = min(i >> 3, a.M - 1);
        const size_t o = (size_t)tok * (K >> 5) + (k0 >> 5) + (i & 7);
        r.sc[u] = make_float2(a.xs[o], (float)a.xsum[o]);
    }
}

// codes [token][kPgStride]; scales and scale * code sums as [block][token]
// planes, so the four tokens of an MFMA output lane are one 16-B read each
template <int NT>
__device__ __forceinline__ void pg_store(const PgStage<NT> &r, int8_t *lx, float *ls, float *lq) {
    const int t = threadIdx.x;
#pragma unroll
    for (int u = 0; u < PgStage<NT>::QN; u++) {
        const int i = t + NT * u;
        *(v4i_t *)(lx + (i >> 4) * kPgStride + 16 * (i & 15)) = r.q[u];
    }
#pragma unroll
    for (int u = 0; u < PgStage<NT>::SN; u++) {
        const int i = t + NT * u, o = (i & 7) * kPgPlane + (i >> 3);
        ls[o] = r.sc[u].x;
        lq[o] = r.sc[u].x * r.sc[u].y;
    }
}

// Prefill GEMM, 17..64 tokens (kPrefillTokens): each wave owns 16 weight rows
// and all four 16-token tiles, so every weight fragment read from HBM feeds
// four MFMAs.  K is walked in 256-value steps (one Q4_K super-block, or eight
// Q8_0 blocks); the 64 activation rows of a step (16 KB of codes plus the
// per-block scale terms) are staged through a double-buffered LDS slot, the
// next step's loads in flight while this one is consumed, so the LDS
// footprint does not grow with K.  Per 32-block the four token tiles' MFMAs
// issue back to back, then their outputs take the block term of
// k_vgemm_q8_0 / k_vgemm_q4k with fused multiply-adds:
//   Q4_K  acc += (s * d*sc) * dot, then per step the min terms
//         - sum_j (d_min*mn_j) * (s * sum q)_j as one K = 8 f32 MFMA per tile
//   Q8_0  acc += (s * d_w) * dot
// (the same terms as the reference's s * (d*sc*dot - dmin*mn*sum q), in
// another rounding order).
// DOTS: also write each per-block integer dot to a.dots (the readback of
// fl_op_batched_block_dots; a separate instantiation, so the product's has
// no trace of it)
// NW waves (16 rows each) share the staged activations; NW = 8 runs with at
// most 128 VGPRs, so two workgroups (16 waves) fit on a CU beside their LDS.
template <int FMT, bool DOTS = false, int NW = 4>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(NW == 8 ? 4 : 1)))
void k_pgemm(VgArgs a) {
    __shared__ __align__(16) int8_t lx[2][64 * kPgStride];
    __shared__ __align__(16) float lsc[2][8 * kPgPlane];  // [block][token] activation scales
    __shared__ __align__(16) float lsq[2][8 * kPgPlane];  // [block][token] scale * code sum
    const WDesc &W = a.W;
    const int K = W.cols, nst = K >> 8;  // 256-value steps
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int s0 = blockIdx.y * a.chunk, s1 = min(nst, s0 + a.chunk);
    if (s0 >= s1) return;
    const int tile = blockIdx.x * NW + wave;
    const int n = tile * 16 + (lane & 15), kg = lane >> 4, tA = lane & 15;
    const int row = min(n, W.rows - 1);
    float acc[4][4];
#pragma unroll
    for (int tt = 0; tt < 4; tt++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[tt][i] = 0.f;
    // weights of one step for this lane: Q4_K qs 4 x 8 B + the 16-B header;
    // Q8_0 8 blocks x 8 B + 8 scales
    i64x1_t wn[8];
    v4i_t hn;
    uint16_t sn[8];
    auto wload = [&](int st) {
        if constexpr (FMT == F_Q4K) {
            const uint8_t *qs = W.q + ((size_t)row * nst + st) * 128 + 8 * kg;
#pragma unroll
            for (int jj = 0; jj < 4; jj++) wn[jj] = *(const i64x1_t *)(qs + 32 * jj);
            hn = *(const v4i_t *)(W.h + ((size_t)row * nst + st) * 16);
        } else {
            const int8_t *wq = (const int8_t *)W.q + (size_t)row * K + 256 * st + 8 * kg;
#pragma unroll
            for (int jj = 0; jj < 8; jj++) wn[jj] = *(const i64x1_t *)(wq + 32 * jj);
#pragma unroll
            for (int jj = 0; jj < 8; jj++) sn[jj] = W.s[(size_t)row * (K >> 5) + 8 * st + jj];
        }
    };
    PgStage<NW * 64> xr;
    wload(s0);
    pg_load(a, s0 * 256, xr);
    pg_store(xr, lx[0], lsc[0], lsq[0]);
    __syncthreads();
    for (int st = s0; st < s1; st++) {
        const int cur = (st - s0) & 1;
        i64x1_t w[8];
        v4i_t h = hn;
        uint16_t sc8[8];
#pragma unroll
        for (int jj = 0; jj < 8; jj++) {
            w[jj] = wn[jj];
            sc8[jj] = sn[jj];
        }
        if (st + 1 < s1) {
            wload(st + 1);
            pg_load(a, (st + 1) * 256, xr);
        }
        const int8_t *bx = lx[cur];
        if (tile * 16 < W.rows) {
            float d = 0.f, dmin = 0.f;
            if constexpr (FMT == F_Q4K) {
                const uint32_t h0 = (uint32_t)h.x;
                d = h2f((uint16_t)(h0 & 0xFFFF));
                dmin = h2f((uint16_t)(h0 >> 16));
            }
#pragma unroll
            for (int j = 0; j < 8; j++) {
                i64x1_t wb;
                float dsc;
                if constexpr (FMT == F_Q4K) {
                    const int jj = j & 3;
                    const i64x1_t m4 = 0x0F0F0F0F0F0F0F0FLL;
                    wb = j < 4 ? (w[jj] & m4) : ((w[jj] >> 4) & m4);
                    // unpack_q4k_scales (model.rs:8709-8719), flare packing
                    const uint32_t sa = byte_of((uint32_t)h.y, jj), scc = byte_of((uint32_t)h.w, jj);
                    const uint32_t sc = j < 4 ? (sa & 63) : ((sa >> 6) | ((scc & 0xF) << 2));
                    dsc = d * (float)sc;
                } else {
                    wb = w[j];
                    dsc = h2f(sc8[j]);
                }
                // Q4_K sub-block j: low nibbles pair with activation bytes 32j of
                // the step for j < 4 (qs bytes 32jj..), high nibbles with 32j
                v4i32_t dd[4];
#pragma unroll
                for (int tt = 0; tt < 4; tt++)
                    dd[tt] = vg_mfma(*(const i64x1_t *)(bx + (tA + 16 * tt) * kPgStride + 32 * j + 8 * kg), wb);
                if constexpr (DOTS)
#pragma unroll
                    for (int tt = 0; tt < 4; tt++)
#pragma unroll
                        for (int i = 0; i < 4; i++) vg_dot_out(a, 16 * tt + 4 * kg + i, n, st * 8 + j, dd[tt][i]);
#pragma unroll
                for (int tt = 0; tt < 4; tt++) {
                    const int t0 = 16 * tt + 4 * kg;  // tokens t0 .. t0+3 of this lane
                    const v4f_t xs = *(const v4f_t *)&lsc[cur][j * kPgPlane + t0];
                    const float xv[4] = {xs.x, xs.y, xs.z, xs.w};
#pragma unroll
                    for (int i = 0; i < 4; i++) acc[tt][i] = __builtin_fmaf(xv[i] * dsc, (float)dd[tt][i], acc[tt][i]);
                }
            }
            if constexpr (FMT == F_Q4K) {
                // the min terms of the step's 8 sub-blocks, as a K = 8 f32 MFMA
                // per token tile: A = s * sum q [token][sub-block], B = -d_min*mn
                // [sub-block][row]; lane (row, kg) supplies sub-blocks kg, 4 + kg
                const uint32_t sbb = byte_of((uint32_t)h.z, kg), scc = byte_of((uint32_t)h.w, kg);
                const float nm0 = -(dmin * (float)(sbb & 63));
                const float nm1 = -(dmin * (float)((sbb >> 6) | ((scc >> 4) << 2)));
#pragma unroll
                for (int tt = 0; tt < 4; tt++) {
                    v4f32_t c = {acc[tt][0], acc[tt][1], acc[tt][2], acc[tt][3]};
                    c = __builtin_amdgcn_mfma_f32_16x16x4f32(lsq[cur][kg * kPgPlane + tA + 16 * tt], nm0, c, 0, 0, 0);
                    c = __builtin_amdgcn_mfma_f32_16x16x4f32(lsq[cur][(4 + kg) * kPgPlane + tA + 16 * tt], nm1, c, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; i++) acc[tt][i] = c[i];
                }
            }
        }
        if (st + 1 < s1) pg_store(xr, lx[cur ^ 1], lsc[cur ^ 1], lsq[cur ^ 1]);
        __syncthreads();
    }
    if (n < W.rows) {
#pragma unroll
        for (int tt = 0; tt < 4; tt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int t = 16 * tt + 4 * kg + i;
                if (t < a.M) a.part[((size_t)blockIdx.y * a.M + t) * W.rows + n] = acc[tt][i];
            }
    }
}

// Prefill GEMM for Q4_K weights on f16 MFMA (v_mfma_f32_16x16x32_f16), 17..64
// tokens.  The int8 form above pays fp32 block terms per output and 32-block;
// here the MFMA applies them:
//  * B = sc * q of the lane's row: a 4-bit code times its 6-bit sub-block
//    scale is an integer below 1024, exact in f16 (nibble -> 1024 + q by a
//    byte permute under 0x64, then one packed f16 fma: (1024 + q) * sc -
//    1024 * sc, exact);
//  * A = the token's dequantized Q8 activation s * q in f16 high part +
//    f16 residual (~22 bits), staged once per workgroup and step in LDS;
//  * so one super-block's MFMAs accumulate sum_j s_j * sc_j * dot_j in fp32
//    and the step ends with acc += d * C - d_min * Cmin, where Cmin =
//    sum_j mn_j * (s * sum q)_j is a K = 8 f32 MFMA as in k_pgemm.
// Each wave owns 16 weight rows and the four 16-token tiles (NW waves: NW x
// 16 rows per workgroup share the staged activations); the next step's
// activation codes and weights are in flight while the current one is consumed.
constexpr int kPhStride = 256 + 8;  // halves per staged activation row

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));

// 8 nibbles (low or high half of the bytes of w) of a row times the
// sub-block scale, as 8 exact binary16 values
__device__ __forceinline__ h8_t q4_scaled_h8(const i64x1_t w, bool high, h2_t sc2, h2_t bias2) {
    const uint32_t w0 = (uint32_t)w, w1 = (uint32_t)((uint64_t)w >> 32);
    const uint32_t n0 = (high ? w0 >> 4 : w0) & 0x0F0F0F0Fu, n1 = (high ? w1 >> 4 : w1) & 0x0F0F0F0Fu;
    constexpr uint32_t m = 0x64646464u;
    uint32_t d[4];
    d[0] = __builtin_amdgcn_perm(m, n0, 0x04010400u);  // bytes: n0.b0, 0x64, n0.b1, 0x64
    d[1] = __builtin_amdgcn_perm(m, n0, 0x04030402u);
    d[2] = __builtin_amdgcn_perm(m, n1, 0x04010400u);
    d[3] = __builtin_amdgcn_perm(m, n1, 0x04030402u);
    h8_t r;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        h2_t v;
        __builtin_memcpy(&v, &d[k], 4);
        v = __builtin_elementwise_fma(v, sc2, bias2);  // (1024 + q) * sc - 1024 * sc = q * sc, one rounding: exact
        r[2 * k] = v[0];
        r[2 * k + 1] = v[1];
    }
    return r;
}

// NB: activation buffers in LDS (2: the next step is staged while this one is
// consumed, one barrier per step; 1: two barriers per step, half the LDS, so
// two workgroups fit a CU)
template <int NW, int NB>
__global__ __launch_bounds__(NW * 64) void k_pgemm_h(VgArgs a) {
    constexpr int NTH = NW * 64, NPC = 1024 / NTH;  // 16-code pieces per thread and step
    __shared__ __align__(16) _Float16 lxh[NB][64 * kPhStride];  // high parts [token][k]
    __shared__ __align__(16) _Float16 lxl[NB][64 * kPhStride];  // residuals
    __shared__ __align__(16) float lsq[NB][8 * 64];             // [block][token] s * sum q
    const WDesc &W = a.W;
    const int K = W.cols, nst = K >> 8;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, t = threadIdx.x;
    const int s0 = blockIdx.y * a.chunk, s1 = min(nst, s0 + a.chunk);
    if (s0 >= s1) return;
    const int tile = blockIdx.x * NW + wave;
    const int n = tile * 16 + (lane & 15), kg = lane >> 4, tA = lane & 15;
    const int row = min(n, W.rows - 1);
    const bool live = tile * 16 < W.rows;  // wave-uniform
    // activation staging: pieces of 16 codes (token i / 16, bytes 16 (i % 16))
    v4i_t xc[NPC];
    float xsc[NPC];
    float usq = 0.0f;  // (token t / 8, block t % 8): s * sum q (t < 512)
    auto xload = [&](int st) {
        const int k0 = st * 256;
#pragma unroll
        for (int u = 0; u < NPC; u++) {
            const int i = t + NTH * u, tok = min(i >> 4, a.M - 1);
            xc[u] = *(const v4i_t *)(a.xq + (size_t)tok * K + k0 + 16 * (i & 15));
            // token rows >= M stay zero in the MFMA: their scale is taken as 0
            xsc[u] = (i >> 4) < a.M ? a.xs[(size_t)tok * (K >> 5) + (k0 >> 5) + ((i & 15) >> 1)] : 0.0f;
        }
        if (t < 512) {
            const int tok = min(t >> 3, a.M - 1);
            const size_t o = (size_t)tok * (K >> 5) + (k0 >> 5) + (t & 7);
            usq = a.xs[o] * (float)a.xsum[o];
        }
    };
    auto xstore = [&](int buf) {
#pragma unroll
        for (int u = 0; u < NPC; u++) {
            const int i = t + NTH * u, tok = i >> 4;
            float v[16];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const uint32_t wd = (uint32_t)xc[u][k];
#pragma unroll
                for (int e = 0; e < 4; e++) v[4 * k + e] = (float)(int8_t)(wd >> (8 * e));
            }
            h8_t hi[2], lo[2];
#pragma unroll
            for (int h = 0; h < 2; h++) {
                float x[8];
#pragma unroll
                for (int k = 0; k < 8; k++) x[k] = v[8 * h + k] * xsc[u];
                v8h_t a8, b8;
                split8(x, a8, b8);
                hi[h] = a8;
                lo[h] = b8;
            }
            _Float16 *ph = &lxh[buf][tok * kPhStride + 16 * (i & 15)];
            _Float16 *pl = &lxl[buf][tok * kPhStride + 16 * (i & 15)];
            *(h8_t *)ph = hi[0];
            *(h8_t *)(ph + 8) = hi[1];
            *(h8_t *)pl = lo[0];
            *(h8_t *)(pl + 8) = lo[1];
        }
        if (t < 512) lsq[buf][(t & 7) * 64 + (t >> 3)] = (t >> 3) < a.M ? usq : 0.0f;
    };
    // weights of one step for this lane: qs 4 x 8 B + the 16-B header; two
    // steps in flight (sets alternate by step parity)
    i64x1_t wn[2][4];
    v4i_t hn[2];
    auto wload = [&](int st, int set) {
        const int sc = min(st, s1 - 1);
        const uint8_t *qs = W.q + ((size_t)row * nst + sc) * 128 + 8 * kg;
#pragma unroll
        for (int jj = 0; jj < 4; jj++) wn[set][jj] = *(const i64x1_t *)(qs + 32 * jj);
        hn[set] = *(const v4i_t *)(W.h + ((size_t)row * nst + sc) * 16);
    };
    float acc[4][4];
#pragma unroll
    for (int tt = 0; tt < 4; tt++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[tt][i] = 0.f;
    wload(s0, 0);
    wload(s0 + 1, 1);
    xload(s0);
    xstore(0);
    if (s0 + 1 < s1) xload(s0 + 1);
    __syncthreads();
    auto step = [&](int st, int cur) {
        i64x1_t w[4];
        const v4i_t h = hn[cur];
#pragma unroll
        for (int jj = 0; jj < 4; jj++) w[jj] = wn[cur][jj];
        if (st + 2 < s1) wload(st + 2, cur);
        if (live) {
            const uint32_t h0 = (uint32_t)h.x;
            const float d = h2f((uint16_t)(h0 & 0xFFFF)), dmin = h2f((uint16_t)(h0 >> 16));
            v4f32_t cm[4];
#pragma unroll
            for (int tt = 0; tt < 4; tt++) cm[tt] = v4f32_t{0.f, 0.f, 0.f, 0.f};
            const _Float16 *bh = lxh[NB == 2 ? cur : 0], *bl = lxl[NB == 2 ? cur : 0];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int jj = j & 3;
                // unpack_q4k_scales (model.rs:8709-8719), flare packing
                const uint32_t sa = byte_of((uint32_t)h.y, jj), scc = byte_of((uint32_t)h.w, jj);
                const uint32_t sc = j < 4 ? (sa & 63) : ((sa >> 6) | ((scc & 0xF) << 2));
                const _Float16 scf = (_Float16)(float)sc;
                const h2_t sc2 = {scf, scf}, bias2 = {(_Float16)(-1024.0f * (float)sc), (_Float16)(-1024.0f * (float)sc)};
                const h8_t b = q4_scaled_h8(w[jj], j >= 4, sc2, bias2);
                v8h_t bv;
                __builtin_memcpy(&bv, &b, 16);
#pragma unroll
                for (int tt = 0; tt < 4; tt++) {
                    const int o = (tA + 16 * tt) * kPhStride + 32 * j + 8 * kg;
                    cm[tt] = mfma16(*(const v8h_t *)(bh + o), bv, cm[tt]);
                    cm[tt] = mfma16(*(const v8h_t *)(bl + o), bv, cm[tt]);
                }
            }
            // min terms: K = 8 f32 MFMA per tile (A = s * sum q, B = mn of
            // sub-blocks kg and 4 + kg of this lane's row)
            const uint32_t sbb = byte_of((uint32_t)h.z, kg), scc = byte_of((uint32_t)h.w, kg);
            const float mn0 = (float)(sbb & 63), mn1 = (float)((sbb >> 6) | ((scc >> 4) << 2));
#pragma unroll
            for (int tt = 0; tt < 4; tt++) {
                v4f32_t c = {0.f, 0.f, 0.f, 0.f};
                const float *lq = lsq[NB == 2 ? cur : 0];
                c = __builtin_amdgcn_mfma_f32_16x16x4f32(lq[kg * 64 + tA + 16 * tt], mn0, c, 0, 0, 0);
                c = __builtin_amdgcn_mfma_f32_16x16x4f32(lq[(4 + kg) * 64 + tA + 16 * tt], mn1, c, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; i++) acc[tt][i] = __builtin_fmaf(d, cm[tt][i], __builtin_fmaf(-dmin, c[i], acc[tt][i]));
            }
        }
        if (st + 1 < s1) {
            if constexpr (NB == 1) __syncthreads();  // every wave is done with the buffer
            xstore(NB == 2 ? cur ^ 1 : 0);
            if (st + 2 < s1) xload(st + 2);
        }
        __syncthreads();
    };
    // the register set and LDS buffer of step st are (st - s0) & 1
    for (int st = s0; st < s1; st += 2) {
        step(st, 0);
        if (st + 1 < s1) step(st + 1, 1);
    }
    if (n < W.rows) {
#pragma unroll
        for (int tt = 0; tt < 4; tt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int tk = 16 * tt + 4 * kg + i;
                if (tk < a.M) a.part[((size_t)blockIdx.y * a.M + tk) * W.rows + n] = acc[tt][i];
            }
    }
}

// Q8_0, M <= 8 tokens: blocks b and b+1 share one accumulating MFMA pair,
// as the sub-block pairs of k_vgemm_q4k8 (token slots 0-7 carry block b's
// activations in k 0-15, slots 8-15 block b+1's in k 16-31; weight lanes of
// k 0-15 hold block b, those of k 16-31 block b+1).  Lane (n, kg) loads 16
// bytes at 16*(kg&1) of its block; eight blocks per round.  Block term of
// matvec_q8_0_preq_into (model.rs:8082-8099).
__global__ __launch_bounds__(256) void k_vgemm_q8_08(VgArgs a) {
    extern __shared__ __align__(16) char smem[];
    const WDesc &W = a.W;
    const int K = W.cols, nbk = K >> 5;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int chunk = a.chunk;
    const int b0 = blockIdx.y * chunk, b1 = min(nbk, b0 + chunk);
    if (b0 >= b1) return;
    const int kn = (b1 - b0) * 32, xst = kn + 32;
    int8_t *lx = (int8_t *)smem;
    float2 *lsc = (float2 *)(smem + 8 * xst);
    const int tile = blockIdx.x * 4 + wave;
    const bool live = tile * 16 < W.rows;  // wave-uniform
    const int n = tile * 16 + (lane & 15), kg = lane >> 4, tA = lane & 15;
    const int h = kg & 1, hi = kg >> 1;    // weight lane: byte half, block b + hi
    const int tx = tA & 7, xhi = tA >> 3;  // activation lane: token tx of block b + xhi
    const bool xon = xhi == hi && tx < a.M;
    const int row = min(n, W.rows - 1);
    const int8_t *wq = (const int8_t *)W.q + (size_t)row * K + 16 * h;
    const uint16_t *ws = W.s + (size_t)row * nbk;
    v4i_t wn[4];
    uint16_t sn[4];
    auto load = [&](int g0) {  // pair p: blocks g0+2p, g0+2p+1 (clamped into the chunk)
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const int bb = min(g0 + 2 * p + hi, b1 - 1);
            wn[p] = *(const v4i_t *)(wq + 32 * (size_t)bb);
            sn[p] = ws[bb];
        }
    };
    if (live) load(b0);
    vg_stage<F_Q8_0, true>(a, b0 * 32, kn, lx, lsc, xst);
    if (!live) return;
    const int8_t *xo = lx + tx * xst + 16 * h + 32 * xhi;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    for (int g0 = b0; g0 < b1; g0 += 8) {
        v4i_t w[4];
        uint16_t sc[4];
#pragma unroll
        for (int p = 0; p < 4; p++) {
            w[p] = wn[p];
            sc[p] = sn[p];
        }
        if (g0 + 8 < b1) load(g0 + 8);
        v4i32_t dd[4];
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const int bl = g0 - b0 + 2 * p;
            const bool xok = xon && g0 + 2 * p + xhi < b1;
            const v4i_t xv = xok ? *(const v4i_t *)(xo + 32 * bl) : v4i_t{0, 0, 0, 0};
            const i64x1_t w1 = ((i64x1_t)(uint32_t)w[p].y << 32) | (uint32_t)w[p].x;
            const i64x1_t w2 = ((i64x1_t)(uint32_t)w[p].w << 32) | (uint32_t)w[p].z;
            const i64x1_t x1 = ((i64x1_t)(uint32_t)xv.y << 32) | (uint32_t)xv.x;
            const i64x1_t x2 = ((i64x1_t)(uint32_t)xv.w << 32) | (uint32_t)xv.z;
            dd[p] = __builtin_amdgcn_mfma_i32_16x16x32_i8(x2, w2, vg_mfma(x1, w1), 0, 0, 0);
        }
        if (a.dots)
#pragma unroll
            for (int p = 0; p < 4; p++)
#pragma unroll
                for (int e = 0; e < 4; e++)
                    if (g0 + 2 * p + hi < b1) vg_dot_out(a, 4 * h + e, n, g0 + 2 * p + hi, dd[p][e]);
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const int bb = g0 + 2 * p + hi;
            if (bb < b1) {
                const float wsc = h2f(sc[p]);
                const float4 *ls = (const float4 *)(lsc + (bb - b0) * 8 + 4 * h);
                const float4 l0 = ls[0], l1 = ls[1];
                const float xs[4] = {l0.x, l0.z, l1.x, l1.z};
#pragma unroll
                for (int e = 0; e < 4; e++) acc[e] = __builtin_fmaf(wsc * xs[e], (float)dd[p][e], acc[e]);
            }
        }
    }
    // lanes kg and kg+2 hold the even and odd blocks of the same outputs
#pragma unroll
    for (int e = 0; e < 4; e++) acc[e] += __shfl_xor(acc[e], 32, 64);
    if (n < W.rows && hi == 0) {
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int t = 4 * h + e;
            if (t < a.M) a.part[((size_t)blockIdx.y * a.M + t) * W.rows + n] = acc[e];
        }
    }
}

template <int KVW>
__device__ __forceinline__ void qkv_post_pair(const VgArgs::QkvPost &P, int t, int n, float x0, float x1);

// Q4_K, M <= 8 tokens.  Sub-blocks j and j+4 are the low and high nibbles
// of the same 32 qs bytes, so one pair of accumulating MFMAs forms both:
// token slots 0-7 carry sub-block j's activations in k 0-15 of each MFMA
// (zeros in k 16-31), slots 8-15 sub-block j+4's in k 16-31; the weight
// lanes of k 0-15 hold the low nibbles, those of k 16-31 the high ones.  Lane
// (n, kg) loads 16 qs bytes at 16*(kg&1): the first MFMA takes bytes 0-7, the
// second 8-15.  Every output slot is then a live (token, sub-block) term, so
// the per-block fp32 work per MFMA halves against k_vgemm_q4k.
// PD super-blocks of weights in flight per wave.
template <int PD>
__global__ __launch_bounds__(256) void k_vgemm_q4k8(VgArgs a) {
    extern __shared__ __align__(16) char smem[];
    const WDesc &W = a.W;
    const int K = W.cols, nsb = K >> 8;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int chunk = a.chunk;
    const int s0 = blockIdx.y * chunk, s1 = min(nsb, s0 + chunk);
    if (s0 >= s1) return;
    const int kn = (s1 - s0) * 256;
    // activation rows kn + 32 bytes apart: the 16-byte reads of the 8 token
    // rows land on distinct LDS banks
    const int xst = kn + 32;
    int8_t *lx = (int8_t *)smem;
    float2 *lsc = (float2 *)(smem + 8 * xst);
    // post 1: waves 0-1 take gate rows 32x .. 32x+31, waves 2-3 the up rows F
    // further on
    const int tile = a.post == 1 ? (wave < 2 ? 2 * (int)blockIdx.x + wave : a.F / 16 + 2 * (int)blockIdx.x + wave - 2)
                                 : (int)blockIdx.x * 4 + wave;
    const bool live = tile * 16 < W.rows;  // wave-uniform (always, with post)
    const int n = tile * 16 + (lane & 15), kg = lane >> 4, tA = lane & 15;
    const int h = kg & 1, hi = kg >> 1;     // weight lane: byte half, nibble (sub-block j + 4*hi)
    const int tx = tA & 7, xhi = tA >> 3;   // activation lane: token tx of sub-block j + 4*xhi
    const bool xon = xhi == hi && tx < a.M;
    const int row = min(n, W.rows - 1);
    const uint8_t *qs = W.q + (size_t)row * nsb * 128 + 16 * h;
    const uint8_t *hd = W.h + (size_t)row * nsb * 16;
    v4i_t wb[PD][4], hb[PD];
    auto load = [&](int u, int sb) {
#pragma unroll
        for (int p = 0; p < 4; p++) wb[u][p] = *(const v4i_t *)(qs + (size_t)sb * 128 + 32 * p);
        hb[u] = *(const v4i_t *)(hd + (size_t)sb * 16);
    };
    if (live) {
#pragma unroll
        for (int u = 0; u < PD; u++) load(u, min(s0 + u, s1 - 1));
    }
    vg_stage<F_Q4K, true, true>(a, s0 * 256, kn, lx, lsc, xst);
    if (!live) return;
    const int sh = 4 * hi;
    const i64x1_t m4 = 0x0F0F0F0F0F0F0F0FLL;
    const int8_t *xo = lx + tx * xst + 16 * h + 128 * xhi;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    for (int sb0 = s0; sb0 < s1; sb0 += PD)
#pragma unroll
    for (int u = 0; u < PD; u++) {
        const int sb = sb0 + u;
        if (sb >= s1) break;
        v4i_t w[4];
        const v4i_t hh = hb[u];
#pragma unroll
        for (int p = 0; p < 4; p++) w[p] = wb[u][p];
        if (sb + PD < s1) load(u, sb + PD);
        const int sl = sb - s0;
        v4i32_t dd[4];
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const v4i_t xv = xon ? *(const v4i_t *)(xo + sl * 256 + 32 * p) : v4i_t{0, 0, 0, 0};
            const i64x1_t w1 = ((((i64x1_t)(uint32_t)w[p].y << 32) | (uint32_t)w[p].x) >> sh) & m4;
            const i64x1_t w2 = ((((i64x1_t)(uint32_t)w[p].w << 32) | (uint32_t)w[p].z) >> sh) & m4;
            const i64x1_t x1 = ((i64x1_t)(uint32_t)xv.y << 32) | (uint32_t)xv.x;
            const i64x1_t x2 = ((i64x1_t)(uint32_t)xv.w << 32) | (uint32_t)xv.z;
            dd[p] = __builtin_amdgcn_mfma_i32_16x16x32_i8(x2, w2, vg_mfma(x1, w1), 0, 0, 0);
        }
        if (a.dots)
#pragma unroll
            for (int p = 0; p < 4; p++)
#pragma unroll
                for (int e = 0; e < 4; e++) vg_dot_out(a, 4 * h + e, n, sb * 8 + p + 4 * hi, dd[p][e]);
        const uint32_t h0 = (uint32_t)hh.x;
        const float d = h2f((uint16_t)(h0 & 0xFFFF)), dmin = h2f((uint16_t)(h0 >> 16));
        // unpack_q4k_scales (model.rs:8709-8719), flare packing: the 6-bit
        // scale / min of sub-block p + 4*hi in byte p, all four at once
        const uint32_t sa = (uint32_t)hh.y, sbb = (uint32_t)hh.z, scc = (uint32_t)hh.w;
        const uint32_t scw = hi ? (((sa >> 6) & 0x03030303u) | ((scc & 0x0F0F0F0Fu) << 2)) : (sa & 0x3F3F3F3Fu);
        const uint32_t mnw =
            hi ? (((sbb >> 6) & 0x03030303u) | (((scc >> 4) & 0x0F0F0F0Fu) << 2)) : (sbb & 0x3F3F3F3Fu);
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const float dsc = d * (float)byte_of(scw, p), dmn = dmin * (float)byte_of(mnw, p);
            const float4 *ls = (const float4 *)(lsc + (sl * 8 + p + 4 * hi) * 8 + 4 * h);
            const float4 l0 = ls[0], l1 = ls[1];
            const float xs[4] = {l0.x, l0.z, l1.x, l1.z}, xm[4] = {l0.y, l0.w, l1.y, l1.w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                // s * (d*sc*dot - dmin*mn*sum q) as (s * d*sc) * dot - (dmin*mn) * (s * sum q)
                const float a1 = __builtin_fmaf(xs[e] * dsc, (float)dd[p][e], acc[e]);
                acc[e] = __builtin_fmaf(-dmn, xm[e], a1);
            }
        }
    }
    // lanes kg and kg+2 hold sub-blocks 0-3 and 4-7 of the same outputs
#pragma unroll
    for (int e = 0; e < 4; e++) acc[e] += __shfl_xor(acc[e], 32, 64);
    if (n < W.rows && hi == 0) {
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int t = 4 * h + e;
            float *dst = a.part + ((size_t)blockIdx.y * a.M + t) * W.rows + n;
            if (t < a.M) {
                if (a.post) st_agent(dst, acc[e]);  // read by another workgroup
                else *dst = acc[e];
            }
        }
    }
    if (!a.post) return;
    // ---- the last-arriving K split of this column finishes its rows -------
    __shared__ int is_last;
    if (!split_arrive_last<true>(&a.counters[blockIdx.x], a.ksplit, &is_last)) return;
    const int t = threadIdx.x >> 5, u = threadIdx.x & 31;  // token, unit (post 1) / row pair (post 2)
    const int tc = min(t, a.M - 1);
    auto psum = [&](int row) {
        float v = 0.0f;
        for (int k0 = 0; k0 < a.ksplit; k0 += 8) {  // 8 loads in flight, added in split order
            float pv[8];
#pragma unroll
            for (int u = 0; u < 8; u++) pv[u] = ld_agent(a.part + ((size_t)min(k0 + u, a.ksplit - 1) * a.M + tc) * W.rows + row);
#pragma unroll
            for (int u = 0; u < 8; u++)
                if (k0 + u < a.ksplit) v += pv[u];
        }
        return v;
    };
    if (a.post == 1) {
        // silu_mul_into (model.rs:9783-9796), then quantize_input_q8_0_into:
        // one 32-block of h per token
        const int j = 32 * (int)blockIdx.x + u;
        const float g = psum(j), up = psum(a.F + j);
        const float hv = (g / (1.0f + fl_expf(-g))) * up;
        if (t < a.M) {  // uniform per 32-lane group
            const size_t b = (size_t)t * (a.F >> 5) + blockIdx.x;
            quant_block32_lanes(hv, a.hq + (size_t)t * a.F + 32 * blockIdx.x, a.hs + b, a.hsum + b);
        }
    } else {
        const int n2 = 64 * (int)blockIdx.x + 2 * u;
        const float x0 = psum(n2), x1 = psum(n2 + 1);
        if (t < a.M) {
            if (a.qp.kvw == 1) qkv_post_pair<1>(a.qp, t, n2, x0, x1);
            else if (a.qp.kvw == 2) qkv_post_pair<2>(a.qp, t, n2, x0, x1);
            else qkv_post_pair<0>(a.qp, t, n2, x0, x1);
        }
    }
}

// ---- per-token glue ------------------------------------------------------

// Sum of the K-split partials of one output, in split order (loads issued 8
// at a time, all in flight, then added in order: the same sum as a loop).
__device__ __forceinline__ float vsum_part(const float *part, int ksplit, int M, int rows, int t, int n) {
    float v = 0.0f;
    for (int k0 = 0; k0 < ksplit; k0 += 8) {
        float pv[8];
#pragma unroll
        for (int u = 0; u < 8; u++) pv[u] = part[((size_t)min(k0 + u, ksplit - 1) * M + t) * rows + n];
#pragma unroll
        for (int u = 0; u < 8; u++)
            if (k0 + u < ksplit) v += pv[u];
    }
    return v;
}
__device__ __forceinline__ float4 vsum_part4(const float *part, int ksplit, int M, int rows, int t, int e) {
    float4 p = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int k0 = 0; k0 < ksplit; k0 += 8) {
        float4 pv[8];
#pragma unroll
        for (int u = 0; u < 8; u++) pv[u] = *(const float4 *)(part + ((size_t)min(k0 + u, ksplit - 1) * M + t) * rows + e);
#pragma unroll
        for (int u = 0; u < 8; u++)
            if (k0 + u < ksplit) {
                p.x += pv[u].x;
                p.y += pv[u].y;
                p.z += pv[u].z;
                p.w += pv[u].w;
            }
    }
    return p;
}

// Embedding rows of the M tokens (token_embedding lookup, model.rs:1964).
template <int FMT>
__global__ __launch_bounds__(256) void k_v_embed(WDesc E, const int *tokens, float *x) {
    const int t = blockIdx.x, H = E.cols;
    const int row = min(max(tokens[t], 0), E.rows - 1);
    for (int i = threadIdx.x; i < H; i += blockDim.x) {
        float v;
        if (FMT == F_Q8_0) v = (float)((const int8_t *)E.q)[(size_t)row * H + i] * h2f(E.s[(size_t)row * (H >> 5) + (i >> 5)]);
        else if (FMT == F_Q6K) v = q6k_elem(E, row, i);
        else if (FMT == F_Q4K) v = q4k_elem(E, row, i);
        else v = ((const float *)E.q)[(size_t)row * H + i];
        x[(size_t)t * H + i] = v;
    }
}

// QKV post of one rotate-half pair (rows n, n+1) of token t: RoPE
// (apply_rope_with_table, model.rs:7283-7296) on the pair-interleaved q / k
// rows at position pos0 + t; q to Q[t].  K / V: KVW 0 = f32 staging rows
// (quantized into the cache afterwards), 1 / 2 = stored into the F16 / F32
// cache slot pos0 + t (cpu_kv_write's layout, model.rs:9810-9846).
template <int KVW>
__device__ __forceinline__ void qkv_post_pair(const VgArgs::QkvPost &P, int t, int n, float x0, float x1) {
    const int D = P.D, half = D >> 1, pos = *P.pos0p + t;
    const int nq = P.nq, nk = P.nk;
    auto put = [&](bool isv, int e, float v) {  // element e of this token's K or V row
        if constexpr (KVW == 0) {
            (isv ? P.Vst : P.Kst)[(size_t)t * nk + e] = v;
        } else {
            const int kvh = e / D, ch = e % D;
            const size_t o = (size_t)kvh * P.head_stride +
                             ((isv && P.v_tblk) ? vt_off(pos, ch, D) : (size_t)pos * D + ch);
            if constexpr (KVW == 1) ((__half *)(isv ? P.vc : P.kc))[o] = __float2half(v);
            else ((float *)(isv ? P.vc : P.kc))[o] = v;
        }
    };
    if (n < nq + nk) {
        const int j = n % D, i = j >> 1;
        const float c = P.rope[(size_t)pos * half + i], sn = P.rope[P.sin_off + (size_t)pos * half + i];
        const float y0 = x0 * c - x1 * sn, y1 = x0 * sn + x1 * c;
        if (n < nq) {
            const int h = n / D;
            P.Q[(size_t)t * nq + h * D + i] = y0;
            P.Q[(size_t)t * nq + h * D + i + half] = y1;
        } else {
            const int k0 = (n - nq) - j;
            put(false, k0 + i, y0);
            put(false, k0 + i + half, y1);
        }
    } else {
        const int vi = n - nq - nk;
        put(true, vi, x0);
        put(true, vi + 1, x1);
    }
}

// QKV partials -> qkv_post_pair for every (token, row pair).
template <int KVW>
__global__ __launch_bounds__(256) void k_v_qkv_post(const float *part, int ksplit, int M, int rows,
                                                    VgArgs::QkvPost P) {
    const int t = blockIdx.y;
    const int pair = blockIdx.x * blockDim.x + threadIdx.x;  // rows 2*pair, 2*pair+1
    if (2 * pair >= rows) return;
    const int n = 2 * pair;
    qkv_post_pair<KVW>(P, t, n, vsum_part(part, ksplit, M, rows, t, n), vsum_part(part, ksplit, M, rows, t, n + 1));
}

// out[t] = partials (plain store, fl_op_batched_matvec_q8in)
__global__ __launch_bounds__(256) void k_v_store(const float *part, int ksplit, int M, int rows, float *out) {
    const int t = blockIdx.y, i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < rows) out[(size_t)t * rows + i] = vsum_part(part, ksplit, M, rows, t, i);
}

// Residual add + RMSNorm + Q8_0 quantization for M tokens, one workgroup per
// token: x[t] += partials (the residual add, model.rs:2305-2311 / 2537-2543;
// part == nullptr: none), then the decode prologue's arithmetic on the
// updated row (rmsnorm_quantize_q8_0 / rmsnorm_into + quantize, model.rs:
// 5581-5640 / 7456-7477).  Thread i holds elements 4i..4i+3 of every
// 4096-element chunk in registers (H <= kResnormMaxH), so 8 lanes form one
// 32-block; the norm weights load before the reduction.
constexpr int kResnormThreads = 1024;
constexpr int kResnormChunks = 4;
constexpr int kResnormMaxH = 4 * kResnormThreads * kResnormChunks;
template <int PRO>
__global__ __launch_bounds__(kResnormThreads) void k_v_resnorm(const float *part, int ksplit, int M, int H, float *x,
                                                                const float *w, float eps, int8_t *q, float *s,
                                                                int *sum) {
    __shared__ float red[kResnormThreads / 64];
    const int t = blockIdx.x, tid = threadIdx.x;
    float *xt = x + (size_t)t * H;
    float4 v[kResnormChunks], wv[kResnormChunks];
    float ss = 0.0f;
#pragma unroll
    for (int c = 0; c < kResnormChunks; c++) {
        const int e = 4 * (tid + c * kResnormThreads);
        v[c] = wv[c] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (e < H) {
            v[c] = *(const float4 *)(xt + e);
            wv[c] = *(const float4 *)(w + e);
            if (part) {
                const float4 p = vsum_part4(part, ksplit, M, H, t, e);
                v[c].x += p.x;
                v[c].y += p.y;
                v[c].z += p.z;
                v[c].w += p.w;
                *(float4 *)(xt + e) = v[c];
            }
        }
        ss += v[c].x * v[c].x + v[c].y * v[c].y + v[c].z * v[c].z + v[c].w * v[c].w;
    }
    ss = wave_sum(ss);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    ss = 0.0f;
#pragma unroll
    for (int i = 0; i < kResnormThreads / 64; i++) ss += red[i];
    const float inv = 1.0f / sqrtf(ss / (float)H + eps);
#pragma unroll
    for (int c = 0; c < kResnormChunks; c++) {
        const int e = 4 * (tid + c * kResnormThreads);
        if (c * 4 * kResnormThreads >= H) break;  // uniform: shuffles below
        const bool in = e < H;  // H % 32 == 0: a 32-block is wholly in or out
        float y[4] = {v[c].x, v[c].y, v[c].z, v[c].w}, wi[4] = {wv[c].x, wv[c].y, wv[c].z, wv[c].w};
        float amax = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            y[j] = (PRO == PRO_NORMQ0) ? y[j] * wi[j] * inv : (y[j] * inv) * wi[j];
            amax = fmaxf(amax, fabsf(y[j]));
        }
#pragma unroll
        for (int o = 1; o < 8; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
        const float d = amax / 127.0f;
        const float id = (d != 0.0f) ? 127.0f / amax : 0.0f;
        int cs = 0;
        int8_t qq[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            qq[j] = q8_code(y[j] * id);
            cs += qq[j];
        }
        char4 cq;
        cq.x = qq[0];
        cq.y = qq[1];
        cq.z = qq[2];
        cq.w = qq[3];
#pragma unroll
        for (int o = 1; o < 8; o <<= 1) cs += __shfl_xor(cs, o, 64);
        if (in) {
            *(char4 *)(q + (size_t)t * H + e) = cq;
            if ((tid & 7) == 0) {
                s[(size_t)t * (H >> 5) + (e >> 5)] = d;
                sum[(size_t)t * (H >> 5) + (e >> 5)] = cs;
            }
        }
    }
}

// x[t] += partials (residual add, model.rs:2305-2311 / 2537-2543)
__global__ __launch_bounds__(256) void k_v_residual(const float *part, int ksplit, int M, int H, float *x) {
    const int t = blockIdx.y, i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < H) x[(size_t)t * H + i] += vsum_part(part, ksplit, M, H, t, i);
}

// gate/up partials -> SiLU(g) * u (silu_mul_into, model.rs:9783-9796) ->
// Q8_0 quantization per 32-block (the down projection's input).
__global__ __launch_bounds__(256) void k_v_silu_quant(const float *part, int ksplit, int M, int F, int8_t *q, float *s,
                                                      int *sum) {
    const int t = blockIdx.y, i = blockIdx.x * blockDim.x + threadIdx.x;  // F % 256 == 0 not required:
    const int rows = 2 * F;
    const int ic = min(i, F - 1);
    const float g = vsum_part(part, ksplit, M, rows, t, ic), u = vsum_part(part, ksplit, M, rows, t, F + ic);
    const float h = (g / (1.0f + fl_expf(-g))) * u;
    // 32 lanes per block (F % 32 == 0, so a block never straddles the end)
    if (i - (threadIdx.x & 31) < F)
        quant_block32_lanes(h, q + (size_t)t * F + (i & ~31), s + (size_t)t * (F >> 5) + (i >> 5),
                            sum + (size_t)t * (F >> 5) + (i >> 5));
}

}  // namespace fl
