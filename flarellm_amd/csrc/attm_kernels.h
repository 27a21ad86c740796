// Split-K GQA decode attention on f16 MFMA (fp16 and Q8 KV caches).
//
// Same semantics as k_attn (cpu_grouped_query_attention_into,
// flare-core/src/model.rs:9849-9966; online softmax of
// fused_attention_head_scalar 9914-9966), restructured for CDNA4:
//  * every wave walks its own 32-token blocks with a wave-private online
//    softmax (no workgroup barrier inside the token loop);
//  * scores S = Q K^T: v_mfma_f32_16x16x32_f16 with the G query heads as
//    rows, each q split into an f16 high part and an f16 residual
//    (q = hi + lo to ~22 bits, every product exact in fp32), K rows as the
//    B operand straight from the token-major cache;
//  * output O += P V: the same MFMA with P (hi / lo) as rows and V as the B
//    operand, which needs 8 consecutive tokens of one channel per lane: the
//    model's V cache is stored in 32-token transposed blocks
//    [kv head][slot / 32][channel][32 slots].
// Q8 caches: K block scale applied per (token, 32-channel block) to each
// block's MFMA result; V scales folded into P per block.
#pragma once

#include "attn_kernels.h"

namespace fl {

typedef _Float16 v8h_t __attribute__((ext_vector_type(8)));
typedef float v4f32_t __attribute__((ext_vector_type(4)));

constexpr int kAttmThreads = 512;  // 8 waves, each walking 32-token blocks
constexpr int kAttmBlock = 32;
constexpr int kAttmMaxSplit = 64;
constexpr int kAttmSingle = 1024;  // contexts up to this many tokens run as one split

// Offset of (slot t, channel d) in one kv head's transposed V store.
__host__ __device__ inline size_t vt_off(int t, int d, int D) {
    return ((size_t)(t >> 5) * D + d) * 32 + (t & 31);
}

__device__ __forceinline__ v4f32_t mfma16(const v8h_t &a, const v8h_t &b, const v4f32_t &c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// 8 floats -> f16 high parts and f16 residuals
__device__ __forceinline__ void split8(const float *x, v8h_t &hi, v8h_t &lo) {
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const _Float16 h = (_Float16)x[i];
        hi[i] = h;
        lo[i] = (_Float16)(x[i] - (float)h);
    }
}

__device__ __forceinline__ v8h_t as_h8(const v4i_t &v) {
    v8h_t r;
    __builtin_memcpy(&r, &v, 16);
    return r;
}

// int8 codes -> exact f16 values
__device__ __forceinline__ v8h_t i8x8_to_h8(const v2i_t &c) {
    v8h_t r;
#pragma unroll
    for (int i = 0; i < 8; i++) r[i] = (_Float16)(int8_t)(((uint32_t)(i < 4 ? c.x : c.y) >> (8 * (i & 3))) & 0xFF);
    return r;
}

template <typename KT, int D>
struct AttmTile;

// fp16: K rows (B operand of S), transposed V (B operand of O)
template <int D>
struct AttmTile<__half, D> {
    static constexpr int DT = D / 32, NT = D / 16;
    v4i_t k[2][DT];  // [token half][32-channel tile]
    v4i_t v[NT];     // [16-channel tile]
    __device__ __forceinline__ void load(const AttnArgs &a, int kvh, int tb, int tlast, int lane) {
        const __half *kc = (const __half *)a.kc + (size_t)kvh * a.head_stride;
        const __half *vc = (const __half *)a.vc + (size_t)kvh * a.head_stride;
        const int kg = lane >> 4, r = lane & 15;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int t = min(tb + 16 * h + r, tlast);
#pragma unroll
            for (int dt = 0; dt < DT; dt++) k[h][dt] = *(const v4i_t *)(kc + (size_t)t * D + 32 * dt + 8 * kg);
        }
        // the 8 slots tb + 8kg .. +8 of channel 16nt + r (one 32-slot block)
#pragma unroll
        for (int nt = 0; nt < NT; nt++) v[nt] = *(const v4i_t *)(vc + vt_off(tb, 16 * nt + r, D) + 8 * kg);
    }
};

// Q8: int8 codes + f16 scale per (slot, 32-channel block)
template <int D>
struct AttmTile<KvQ8, D> {
    static constexpr int DT = D / 32, NT = D / 16;
    v2i_t k[2][DT];
    v2i_t v[NT];
    uint32_t ksc[2][(DT + 1) / 2];  // this lane's slot: K scales (2 per word)
    __device__ __forceinline__ void load(const AttnArgs &a, int kvh, int tb, int tlast, int lane) {
        const int8_t *kc = (const int8_t *)a.kc + (size_t)kvh * a.head_stride;
        const int8_t *vc = (const int8_t *)a.vc + (size_t)kvh * a.head_stride;
        const int kg = lane >> 4, r = lane & 15;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int t = min(tb + 16 * h + r, tlast);
#pragma unroll
            for (int dt = 0; dt < DT; dt++) k[h][dt] = *(const v2i_t *)(kc + (size_t)t * D + 32 * dt + 8 * kg);
            const uint32_t *sp = (const uint32_t *)(a.ks + ((size_t)kvh * a.S + t) * DT);
#pragma unroll
            for (int w = 0; w < (DT + 1) / 2; w++) ksc[h][w] = sp[w];
        }
#pragma unroll
        for (int nt = 0; nt < NT; nt++) v[nt] = *(const v2i_t *)(vc + vt_off(tb, 16 * nt + r, D) + 8 * kg);
    }
};

// One workgroup = (split s, kv head kvh, query z); waves take 32-token
// blocks of the split's chunk round-robin.
template <typename KT, int D, int G>
__global__ __launch_bounds__(kAttmThreads) void k_attm(AttnArgs a0) {
    constexpr int DT = D / 32, NT = D / 16, NW = kAttmThreads / 64;
    constexpr int OPT = (G * D + kAttmThreads - 1) / kAttmThreads;
    static_assert(2 * G <= 16, "query heads (hi/lo rows) exceed the MFMA tile");
    __shared__ float sp[NW][G][kAttmBlock];  // p of the current block (per wave)
    __shared__ float vsc[NW][kAttmBlock][DT];  // Q8: V scales of the block's slots
    __shared__ float vmax[NW][DT];             // Q8: their maximum per 32-channel block
    __shared__ float red[NW][G * D];         // per-wave O, then the workgroup output
    __shared__ float wm[NW][G], wl[NW][G];
    __shared__ float Mx[G], Lx[G];
    __shared__ int is_last;
    __shared__ int8_t nk[D], nv[D];              // Q8 decode step: the new token's codes
    __shared__ uint16_t nks[D / 32], nvs[D / 32];  // and scales

    AttnArgs a = a0;
    const int zq = (int)blockIdx.z;
    if (zq) {
        a.q += (size_t)zq * a.qstride;
        if (a.out) a.out += (size_t)zq * a.ostride;
        if (a.oq) {
            a.oq += (size_t)zq * a.ostride;
            a.os += (size_t)zq * (a.ostride / 32);
            a.osum += (size_t)zq * (a.ostride / 32);
        }
        a.part += (size_t)zq * a.nkv * a.nsplit * G * (D + 2);
        a.counters += (size_t)zq * a.nkv;
    }
    const int kvh = blockIdx.y, s = blockIdx.x, tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6, kg = lane >> 4, r = lane & 15;
    ATTN_TS(0);
    const int pos = *a.posp + zq, T = pos + 1;
    // up to kAttmSingle tokens: one split (no cross-workgroup merge);
    // beyond: chunks of at least chmin slots over the nsplit workgroups
    int CH = T <= kAttmSingle ? T : max(a.chmin, (T + a.nsplit - 1) / a.nsplit);
    CH = (CH + kAttmBlock * NW - 1) / (kAttmBlock * NW) * (kAttmBlock * NW);
    const int t0 = s * CH;
    if (t0 >= T) return;
    const int t1 = min(T, t0 + CH);
    const int nact = (T + CH - 1) / CH;

    // the new token (Q8 decode step): quantize, store, and use its codes
    NewRow<KT> nrow;
    const bool has_new = a.knew != nullptr;

    // the first block's K / V loads go out before the query setup
    const int nblk = (t1 - t0 + kAttmBlock - 1) / kAttmBlock;
    AttmTile<KT, D> tile;
    if (wave < nblk) tile.load(a, kvh, t0 + wave * kAttmBlock, t1 - 1, lane);

    // A operand of S: row m = 2g + (hi / lo) of head g (rows >= 2G zero)
    v8h_t aq[DT];
    {
        const int m = r, g = min(m >> 1, G - 1);
        const v4f_t *qp = (const v4f_t *)(a.q + (size_t)(kvh * G + g) * D + 8 * kg);
#pragma unroll
        for (int dt = 0; dt < DT; dt++) {
            const v4f_t q0 = qp[8 * dt], q1 = qp[8 * dt + 1];
            float x[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
            if ((m >> 1) >= G) {
#pragma unroll
                for (int i = 0; i < 8; i++) x[i] = 0.0f;
            }
            v8h_t hi, lo;
            split8(x, hi, lo);
            aq[dt] = (m & 1) ? lo : hi;
        }
    }
    const float scale = 1.0f / sqrtf((float)D);
    ATTN_TS(1);

    // wave-private online softmax state; lane group kg holds heads 2kg, 2kg+1
    float m_run[2] = {-INFINITY, -INFINITY}, l_run[2] = {0.0f, 0.0f};
    v4f32_t oacc[NT];
#pragma unroll
    for (int nt = 0; nt < NT; nt++) oacc[nt] = v4f32_t{0.f, 0.f, 0.f, 0.f};

    // one 32-slot block (slots tb .. tb+31) with its tile in registers
    auto process = [&](AttmTile<KT, D> &tile, int bi) {
        const int tb = t0 + bi * kAttmBlock;
        if constexpr (std::is_same<KT, KvQ8>::value) {
            // Q8 decode step: the block holding slot pos quantizes the new
            // token, stores it, and patches its K row / V column in registers
            if (has_new && pos >= tb && pos < tb + kAttmBlock) {
                const int c = lane % (D / 8);  // lanes >= D/8 duplicate a chunk
                nrow.build(a, kvh, c);
                if (lane < D / 8) {
                    nrow.store(a, kvh, pos, c);
                    *(v2i_t *)(nk + 8 * c) = nrow.k;
                    *(v2i_t *)(nv + 8 * c) = nrow.v;
                    if ((c & 3) == 0) {
                        nks[c >> 2] = (uint16_t)(nrow.sc & 0xFFFF);
                        nvs[c >> 2] = (uint16_t)(nrow.sc >> 16);
                    }
                }
                __builtin_amdgcn_s_waitcnt(0);
                __builtin_amdgcn_wave_barrier();
                const int pi = pos - tb, th = pi >> 4;
                if ((pi & 15) == r) {
#pragma unroll
                    for (int h = 0; h < 2; h++)
                        if (h == th) {
#pragma unroll
                            for (int dt = 0; dt < DT; dt++) tile.k[h][dt] = *(const v2i_t *)(nk + 32 * dt + 8 * kg);
#pragma unroll
                            for (int w = 0; w < (DT + 1) / 2; w++)
                                tile.ksc[h][w] = (uint32_t)nks[2 * w] |
                                                 ((2 * w + 1 < DT ? (uint32_t)nks[2 * w + 1] : 0u) << 16);
                        }
                }
                // V: byte (pi & 7) of the 8 slots lane group kg holds
                if ((pi >> 3) == kg) {
                    const int sh = 8 * (pi & 3);
#pragma unroll
                    for (int nt = 0; nt < NT; nt++) {
                        const uint32_t b = (uint32_t)(uint8_t)nv[16 * nt + r];
                        if ((pi & 7) < 4) tile.v[nt].x = (int)(((uint32_t)tile.v[nt].x & ~(0xFFu << sh)) | (b << sh));
                        else tile.v[nt].y = (int)(((uint32_t)tile.v[nt].y & ~(0xFFu << sh)) | (b << sh));
                    }
                }
            }
        }
        // ---- scores: two 16-slot halves -------------------------------------
        float sc[2][2];  // [half][head parity] for slot tb + 16h + r
#pragma unroll
        for (int h = 0; h < 2; h++) {
            v4f32_t acc = v4f32_t{0.f, 0.f, 0.f, 0.f};
            if constexpr (std::is_same<KT, __half>::value) {
#pragma unroll
                for (int dt = 0; dt < DT; dt++) acc = mfma16(aq[dt], as_h8(tile.k[h][dt]), acc);
            } else {
#pragma unroll
                for (int dt = 0; dt < DT; dt++) {
                    const v4f32_t part = mfma16(aq[dt], i8x8_to_h8(tile.k[h][dt]), v4f32_t{0.f, 0.f, 0.f, 0.f});
                    const uint32_t w = tile.ksc[h][dt >> 1];
                    const float ks = h2f((uint16_t)((dt & 1) ? (w >> 16) : (w & 0xFFFF)));
#pragma unroll
                    for (int i = 0; i < 4; i++) acc[i] += part[i] * ks;
                }
            }
            const int t = tb + 16 * h + r;
            const bool ok = t < t1;
            sc[h][0] = ok ? (acc[0] + acc[1]) * scale : -INFINITY;
            sc[h][1] = ok ? (acc[2] + acc[3]) * scale : -INFINITY;
        }
        if (bi == wave) ATTN_TS(2);
        // ---- online softmax per head (rows of 16 lanes hold one head pair) --
        float alpha[2];
#pragma unroll
        for (int e = 0; e < 2; e++) {
            float bm = row_max<16>(fmaxf(sc[0][e], sc[1][e]));
            const float mn = fmaxf(m_run[e], bm);
            alpha[e] = (m_run[e] == -INFINITY) ? 0.0f : __expf(m_run[e] - mn);
            const float p0 = sc[0][e] == -INFINITY ? 0.0f : __expf(sc[0][e] - mn);
            const float p1 = sc[1][e] == -INFINITY ? 0.0f : __expf(sc[1][e] - mn);
            l_run[e] = l_run[e] * alpha[e] + row_sum<16>(p0 + p1);
            m_run[e] = mn;
            const int g = 2 * kg + e;
            if (g < G) {
                sp[wave][g][r] = p0;
                sp[wave][g][16 + r] = p1;
            }
        }
        if constexpr (std::is_same<KT, KvQ8>::value) {
            // V scales of the block's 32 slots (lane = slot, one word per 2 blocks)
            if (lane < kAttmBlock) {
                const int t = min(tb + lane, t1 - 1);
#pragma unroll
                for (int b = 0; b < DT; b++) {
                    uint16_t sv = a.vs[((size_t)kvh * a.S + t) * DT + b];
                    if (has_new && tb + lane == pos) sv = nvs[b];
                    const float v = (tb + lane < t1) ? h2f(sv) : 0.0f;
                    vsc[wave][lane][b] = v;
                    float mx = row_max<16>(v);
                    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
                    if (lane == 0) vmax[wave][b] = mx;
                }
            }
        }
        __builtin_amdgcn_wave_barrier();
        // ---- rescale O (rows 4kg+i: heads 2kg + i/2) and accumulate P V -----
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            oacc[nt][0] *= alpha[0];
            oacc[nt][1] *= alpha[0];
            oacc[nt][2] *= alpha[1];
            oacc[nt][3] *= alpha[1];
        }
        {
            const int m = r, g = m >> 1;
            float p[8];
#pragma unroll
            for (int i = 0; i < 8; i++) p[i] = g < G ? sp[wave][g][8 * kg + i] : 0.0f;
            if constexpr (std::is_same<KT, __half>::value) {
                v8h_t hi, lo;
                split8(p, hi, lo);
                const v8h_t ap = (m & 1) ? lo : hi;
#pragma unroll
                for (int nt = 0; nt < NT; nt++) oacc[nt] = mfma16(ap, as_h8(tile.v[nt]), oacc[nt]);
            } else {
                // V scales folded into P relative to the block's largest
                // scale (keeps the f16 residual out of the subnormal range),
                // which multiplies the block's MFMA result
#pragma unroll
                for (int b = 0; b < DT; b++) {
                    const float vref = vmax[wave][b];
                    const float inv = vref > 0.0f ? 1.0f / vref : 0.0f;
                    float pb[8];
#pragma unroll
                    for (int i = 0; i < 8; i++) pb[i] = p[i] * (vsc[wave][8 * kg + i][b] * inv);
                    v8h_t hi, lo;
                    split8(pb, hi, lo);
                    const v8h_t ap = (m & 1) ? lo : hi;
#pragma unroll
                    for (int u = 0; u < 2; u++) {
                        const v4f32_t part =
                            mfma16(ap, i8x8_to_h8(tile.v[2 * b + u]), v4f32_t{0.f, 0.f, 0.f, 0.f});
#pragma unroll
                        for (int i = 0; i < 4; i++) oacc[2 * b + u][i] += part[i] * vref;
                    }
                }
            }
        }
        __builtin_amdgcn_wave_barrier();
    };
    if constexpr (std::is_same<KT, __half>::value) {
        // ping-pong: the wave's next block is in flight while this one computes
        AttmTile<KT, D> tile2;
        for (int bi = wave; bi < nblk; bi += 2 * NW) {
            if (bi + NW < nblk) tile2.load(a, kvh, t0 + (bi + NW) * kAttmBlock, t1 - 1, lane);
            process(tile, bi);
            if (bi + NW >= nblk) break;
            if (bi + 2 * NW < nblk) tile.load(a, kvh, t0 + (bi + 2 * NW) * kAttmBlock, t1 - 1, lane);
            process(tile2, bi + NW);
        }
    } else {
        // Q8 (more registers per block): one tile, loaded at the top
        for (int bi = wave; bi < nblk; bi += NW) {
            if (bi != wave) tile.load(a, kvh, t0 + bi * kAttmBlock, t1 - 1, lane);
            process(tile, bi);
        }
    }

    ATTN_TS(3);
    // ---- combine the 4 waves: O_w (relative to m_w), m_w, l_w ---------------
#pragma unroll
    for (int e = 0; e < 2; e++) {
        const int g = 2 * kg + e;
        if (g < G && r == 0) {
            wm[wave][g] = m_run[e];
            wl[wave][g] = l_run[e];
        }
    }
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
#pragma unroll
        for (int e = 0; e < 2; e++) {
            const int g = 2 * kg + e;
            if (g < G) red[wave][g * D + 16 * nt + r] = oacc[nt][2 * e] + oacc[nt][2 * e + 1];
        }
    }
    __syncthreads();
    if (tid < G) {
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < NW; w++) M = fmaxf(M, wm[w][tid]);
        float L = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; w++) L += wm[w][tid] == -INFINITY ? 0.0f : wl[w][tid] * __expf(wm[w][tid] - M);
        Mx[tid] = M;
        Lx[tid] = L;
    }
    __syncthreads();
    float res[OPT];
#pragma unroll
    for (int k = 0; k < OPT; k++) {
        const int i = tid + k * kAttmThreads;
        float O = 0.0f;
        if (i < G * D) {
            const int g = i / D;
#pragma unroll
            for (int w = 0; w < NW; w++)
                if (wm[w][g] != -INFINITY) O += red[w][i] * __expf(wm[w][g] - Mx[g]);
        }
        res[k] = O;
    }
    float *mo = &red[0][0];  // final output of this kv head (for the Q8 copy)
    if (nact == 1) {
        __syncthreads();  // red is overwritten below
#pragma unroll
        for (int k = 0; k < OPT; k++) {
            const int i = tid + k * kAttmThreads;
            if (i < G * D) {
                const float v = res[k] * (1.0f / Lx[i / D]);
                mo[i] = v;
                if (a.out) a.out[(size_t)kvh * G * D + i] = v;
            }
        }
    } else {
        // publish (unnormalised o, m, l) with agent-scope stores, then count in
        constexpr int P = G * (D + 2);
        float *mypart = a.part + ((size_t)kvh * a.nsplit + s) * P;
#pragma unroll
        for (int k = 0; k < OPT; k++) {
            const int i = tid + k * kAttmThreads;
            if (i < G * D) st_agent(mypart + i, res[k]);
        }
        if (tid < G) {
            st_agent(mypart + G * D + 2 * tid, Mx[tid]);
            st_agent(mypart + G * D + 2 * tid + 1, Lx[tid]);
        }
        ATTN_TS(4);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        ATTN_TS(5);
        if (tid == 0) {
            const int old = __hip_atomic_fetch_add(&a.counters[kvh], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            is_last = (old == nact - 1);
        }
        __syncthreads();
        if (!is_last) return;
        // last workgroup of the kv head: each thread merges its OPT outputs
        // (one head each) over the nact partials, MB splits per round trip
        // (all loads of a batch independent), online rescale between batches:
        // out = sum_j o_j e^(m_j - M) / sum_j l_j e^(m_j - M)
        ATTN_TSL(6);
        constexpr int MB = OPT == 1 ? 32 : 16;
        const float *pb = a.part + (size_t)kvh * a.nsplit * P;
        float M[OPT], L[OPT], O[OPT];
#pragma unroll
        for (int k = 0; k < OPT; k++) {
            M[k] = -INFINITY;
            L[k] = 0.0f;
            O[k] = 0.0f;
        }
        for (int j0 = 0; j0 < nact; j0 += MB) {
#pragma unroll
            for (int k = 0; k < OPT; k++) {
                const int i = min(tid + k * kAttmThreads, G * D - 1), g = i / D;
                float mv[MB], lv[MB], ov[MB];
#pragma unroll
                for (int k2 = 0; k2 < MB; k2++) {
                    const float *pj = pb + (size_t)min(j0 + k2, nact - 1) * P;
                    mv[k2] = ld_agent(pj + G * D + 2 * g);
                    lv[k2] = ld_agent(pj + G * D + 2 * g + 1);
                    ov[k2] = ld_agent(pj + i);
                }
                float Mb = M[k];
#pragma unroll
                for (int k2 = 0; k2 < MB; k2++)
                    if (j0 + k2 < nact) Mb = fmaxf(Mb, mv[k2]);
                const float rr = (M[k] == -INFINITY) ? 0.0f : __expf(M[k] - Mb);
                L[k] *= rr;
                O[k] *= rr;
#pragma unroll
                for (int k2 = 0; k2 < MB; k2++) {
                    if (j0 + k2 < nact) {
                        const float w = (mv[k2] == -INFINITY) ? 0.0f : __expf(mv[k2] - Mb);
                        L[k] += lv[k2] * w;
                        O[k] += ov[k2] * w;
                    }
                }
                M[k] = Mb;
            }
        }
        ATTN_TSL(7);
#pragma unroll
        for (int k = 0; k < OPT; k++) O[k] *= 1.0f / L[k];
        __syncthreads();  // red (mo) is rewritten below
#pragma unroll
        for (int k = 0; k < OPT; k++) {
            const int i = tid + k * kAttmThreads;
            if (i < G * D) {
                const float v = O[k];
                mo[i] = v;
                if (a.out) a.out[(size_t)kvh * G * D + i] = v;
            }
        }
        if (tid == 0) __hip_atomic_store(&a.counters[kvh], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        ATTN_TSL(8);
    }
    __syncthreads();
    if (a.oq) {
        // Q8_0 copy of this kv head's G*D outputs (quantize_input_q8_0_into), 32 lanes per block
        const int nb = G * D / 32;
        for (int b = tid >> 5; b < nb; b += kAttmThreads / 32) {
            const int gb = kvh * nb + b;
            quant_block32_lanes(mo[b * 32 + (tid & 31)], a.oq + gb * 32, a.os + gb, a.osum + gb);
        }
    }
    if (nact > 1) ATTN_TSL(9);
}

}  // namespace fl
