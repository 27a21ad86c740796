// Split-K GQA decode attention kernel (gfx950 wave64).
#pragma once

#include "kernels.h"

namespace fl {

// ---------------------------------------------------------------------------
// Split-K GQA decode attention (cpu_grouped_query_attention_into semantics,
// model.rs:9849-9966).  Grid (nsplit, num_kv_heads); workgroup (s, kvh)
// handles the G query heads sharing kv head kvh over token chunk s, then the
// last workgroup of each kv head merges the chunk partials (flash-decode
// rescale) and writes the f32 output plus its Q8_0 quantization.
// When `knew` is set, q/k arrive un-rotated (QKV matvec output): RoPE is
// applied here and the chunk holding slot `pos` stores the new K/V.
// ---------------------------------------------------------------------------
struct AttnArgs {
    const float *q;      // [nh*D], RoPE already applied
    const void *kc, *vc; // this layer's cache
    long long tok_stride, head_stride;  // elements between slots / kv heads
    const int *posp;     // attends slots 0..*posp
    int nkv, nsplit;     // grid = (nsplit, nkv)
    int chmin;           // minimum tokens per split (a multiple of attn_tpp(D))
    float *part;         // [nkv][nsplit][G][D+2] split partials
    int *counters;       // [nkv] arrival counters (zero between launches)
    float *out;          // [nh*D]
    int8_t *oq;          // optional Q8_0 copy of out (the wo matvec input)
    float *os;
    int *osum;
    long long *trace;    // FLARE_ATTN_TRACE builds: per-phase timestamps of workgroup (0,0)
};



#ifdef FLARE_ATTN_TRACE
#define ATTN_TS(i)                                                                          \
    do {                                                                                    \
        if (a.trace && blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0)             \
            a.trace[i] = (long long)__builtin_amdgcn_s_memrealtime();                       \
    } while (0)
// same, recorded by the workgroup that merges kv head 0
#define ATTN_TSL(i)                                                                         \
    do {                                                                                    \
        if (a.trace && blockIdx.y == 0 && threadIdx.x == 0)                                 \
            a.trace[i] = (long long)__builtin_amdgcn_s_memrealtime();                       \
    } while (0)
#else
#define ATTN_TS(i) \
    do {           \
    } while (0)
#define ATTN_TSL(i) \
    do {            \
    } while (0)
#endif

template <typename KT>
__device__ __forceinline__ void load8(const KT *p, float *v);
template <>
__device__ __forceinline__ void load8<__half>(const __half *p, float *v) {
    const v4i_t t = *(const v4i_t *)p;
    const uint32_t w[4] = {(uint32_t)t.x, (uint32_t)t.y, (uint32_t)t.z, (uint32_t)t.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        v[2 * i] = h2f((uint16_t)(w[i] & 0xFFFF));
        v[2 * i + 1] = h2f((uint16_t)(w[i] >> 16));
    }
}
template <>
__device__ __forceinline__ void load8<float>(const float *p, float *v) {
    const v4f_t a = ((const v4f_t *)p)[0], b = ((const v4f_t *)p)[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}
// Agent-scope relaxed atomic float store / load (cross-XCD visible without
// a cache write-back fence).
__device__ __forceinline__ void st_agent(float *p, float v) {
    __hip_atomic_store((unsigned *)p, __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_agent(const float *p) {
    return __uint_as_float(__hip_atomic_load((const unsigned *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}

// K/V rows kept raw in registers (8 elements) and converted at use.
template <typename KT>
struct KVRaw;
template <>
struct KVRaw<__half> {
    v4i_t v;
    __device__ __forceinline__ void load(const __half *p) { v = *(const v4i_t *)p; }
    __device__ __forceinline__ void get(float *o) const {
        const uint32_t w[4] = {(uint32_t)v.x, (uint32_t)v.y, (uint32_t)v.z, (uint32_t)v.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            o[2 * i] = h2f((uint16_t)(w[i] & 0xFFFF));
            o[2 * i + 1] = h2f((uint16_t)(w[i] >> 16));
        }
    }
};
template <>
struct KVRaw<float> {
    v4f_t a, b;
    __device__ __forceinline__ void load(const float *p) {
        a = ((const v4f_t *)p)[0];
        b = ((const v4f_t *)p)[1];
    }
    __device__ __forceinline__ void get(float *o) const {
        o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w; o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
    }
};

constexpr int kAttnThreads = 256;  // 4 waves per workgroup
constexpr int kAttnMaxSplit = 256; // splits per kv head

// lanes per token row (8 elements each), tokens per pass, passes per round
__host__ __device__ constexpr int attn_lpt(int D) { return D / 8; }
__host__ __device__ constexpr int attn_tpp(int D) { return kAttnThreads / attn_lpt(D); }
__host__ __device__ constexpr int attn_np(int D) { return D == 64 ? 4 : 8; }
__host__ __device__ constexpr int attn_round(int D) { return attn_tpp(D) * attn_np(D); }  // 128 tokens

// One workgroup = (split s, kv head kvh): tokens [t0, t1) for the G query
// heads of the group (cpu_grouped_query_attention_into, model.rs:9849-9905;
// fused_attention_head_scalar 9914-9966).  Thread (tk, c) holds elements
// [8c, 8c+8) of the K and V rows of tokens tk + p*TPP.  Per round of NP
// passes: scores -> LDS; per head one wave takes the round max into a
// workgroup-uniform running max M, writes p = exp(s - M) and keeps the
// denominator; every thread then accumulates p * v for its rows and
// elements.  The partial o is reduced over token slices at the end.
// nsplit > 1: (m, l, o) partials are published with agent-scope stores and
// the last workgroup of the kv head merges them (flash-decode rescale).
template <typename KT, int D, int G>
__global__ __launch_bounds__(kAttnThreads) void k_attn(AttnArgs a) {
    constexpr int LPT = attn_lpt(D), TPP = attn_tpp(D), NP = attn_np(D), CR = TPP * NP;
    constexpr int NW = kAttnThreads / 64, WPT = 64 / LPT;  // token rows per wave per pass
    __shared__ float sc[G][CR];
    __shared__ float Mx[G], al[G], Lx[G];
    __shared__ float red[NW][G * D];  // per-wave o partials, then the final output
    __shared__ int is_last;

    const int kvh = blockIdx.y, s = blockIdx.x, tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int tk = tid / LPT, c = tid % LPT;
    ATTN_TS(0);
    // the query rows and the position are independent loads: issue both first
    float qr[G][8];
#pragma unroll
    for (int g = 0; g < G; g++) {
        const v4f_t *qp = (const v4f_t *)(a.q + (size_t)(kvh * G + g) * D + c * 8);
        const v4f_t q0 = qp[0], q1 = qp[1];
        qr[g][0] = q0.x; qr[g][1] = q0.y; qr[g][2] = q0.z; qr[g][3] = q0.w;
        qr[g][4] = q1.x; qr[g][5] = q1.y; qr[g][6] = q1.z; qr[g][7] = q1.w;
    }
    const int T = *a.posp + 1;
    int CH = max(a.chmin, (T + a.nsplit - 1) / a.nsplit);
    CH = (CH + TPP - 1) / TPP * TPP;
    const int t0 = s * CH;
    if (t0 >= T) return;
    const int t1 = min(T, t0 + CH);
    const int nact = (T + CH - 1) / CH;
    const KT *kc = (const KT *)a.kc + (size_t)kvh * a.head_stride + c * 8;
    const KT *vc = (const KT *)a.vc + (size_t)kvh * a.head_stride + c * 8;

    KVRaw<KT> kb[NP], vb[NP];
    auto fetch = [&](int tb) {
#pragma unroll
        for (int p = 0; p < NP; p++) {
            const int t = min(tb + tk + p * TPP, t1 - 1);
            kb[p].load(kc + (size_t)t * a.tok_stride);
            vb[p].load(vc + (size_t)t * a.tok_stride);
        }
    };
    fetch(t0);
    if (tid < G) {
        Mx[tid] = -INFINITY;
        Lx[tid] = 0.0f;
    }
    ATTN_TS(1);
    const float scale = 1.0f / sqrtf((float)D);
    float o[G][8];
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int e = 0; e < 8; e++) o[g][e] = 0.0f;

    for (int tb = t0; tb < t1; tb += CR) {
        const int n = min(CR, t1 - tb);
        // scores s = (q . k) / sqrt(D), reduced over the LPT lanes of the row
#pragma unroll
        for (int p = 0; p < NP; p++) {
            float kk[8];
            kb[p].get(kk);
#pragma unroll
            for (int g = 0; g < G; g++) {
                float d = 0.0f;
#pragma unroll
                for (int e = 0; e < 8; e++) d += qr[g][e] * kk[e];
                d = row_sum<LPT>(d);
                if (c == 0) sc[g][tk + p * TPP] = d * scale;
            }
        }
        if (tb == t0) ATTN_TS(2);
        __syncthreads();
        // per head: round max -> running max, probabilities, denominator
        for (int g = wave; g < G; g += NW) {
            float m = -INFINITY;
            for (int i = lane; i < n; i += 64) m = fmaxf(m, sc[g][i]);
            m = wave_max(m);
            const float Mo = Mx[g], Mn = fmaxf(Mo, m);
            float l = 0.0f;
            for (int i = lane; i < CR; i += 64) {
                const float pv = i < n ? __expf(sc[g][i] - Mn) : 0.0f;
                sc[g][i] = pv;
                l += pv;
            }
            l = wave_sum(l);
            if (lane == 0) {
                const float alpha = (Mo == -INFINITY) ? 0.0f : __expf(Mo - Mn);
                al[g] = alpha;
                Lx[g] = Lx[g] * alpha + l;
                Mx[g] = Mn;
            }
        }
        __syncthreads();
        if (tb == t0) ATTN_TS(3);
        // o = o * alpha + sum_p p * v over this thread's rows
#pragma unroll
        for (int g = 0; g < G; g++) {
            const float alpha = al[g];
#pragma unroll
            for (int e = 0; e < 8; e++) o[g][e] *= alpha;
        }
#pragma unroll
        for (int p = 0; p < NP; p++) {
            float vv[8];
            vb[p].get(vv);
#pragma unroll
            for (int g = 0; g < G; g++) {
                const float pr = sc[g][tk + p * TPP];
#pragma unroll
                for (int e = 0; e < 8; e++) o[g][e] += pr * vv[e];
            }
        }
        if (tb + CR < t1) {
            __syncthreads();  // sc is rewritten by the next round
            fetch(tb + CR);
        }
    }
    ATTN_TS(4);
    // reduce o over the WPT token rows of the wave, then over the waves
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int e = 0; e < 8; e++) {
            float v = o[g][e];
#pragma unroll
            for (int m = LPT; m < 64; m <<= 1) v += __shfl_xor(v, m, 64);
            o[g][e] = v;
        }
    if (lane < LPT) {
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
            for (int e = 0; e < 8; e++) red[wave][g * D + c * 8 + e] = o[g][e];
    }
    __syncthreads();
    constexpr int OPT = (G * D + kAttnThreads - 1) / kAttnThreads;
    float res[OPT];
#pragma unroll
    for (int k = 0; k < OPT; k++) {
        const int i = tid + k * kAttnThreads;
        float O = 0.0f;
        if (i < G * D) {
#pragma unroll
            for (int w = 0; w < NW; w++) O += red[w][i];
        }
        res[k] = O;
    }
    ATTN_TS(5);
    float *mo = &red[0][0];  // final output of this kv head (for the Q8 copy)
    if (nact == 1) {
        __syncthreads();  // red is overwritten below
#pragma unroll
        for (int k = 0; k < OPT; k++) {
            const int i = tid + k * kAttnThreads;
            if (i < G * D) {
                const float v = res[k] * (1.0f / Lx[i / D]);
                mo[i] = v;
                if (a.out) a.out[(size_t)kvh * G * D + i] = v;
            }
        }
    } else {
        // publish (unnormalised o, m, l) with agent-scope stores, wait for
        // their completion, then count this split in
        constexpr int P = G * (D + 2);
        float *mypart = a.part + ((size_t)kvh * a.nsplit + s) * P;
#pragma unroll
        for (int k = 0; k < OPT; k++) {
            const int i = tid + k * kAttnThreads;
            if (i < G * D) st_agent(mypart + i, res[k]);
        }
        if (tid < G) {
            st_agent(mypart + G * D + 2 * tid, Mx[tid]);
            st_agent(mypart + G * D + 2 * tid + 1, Lx[tid]);
        }
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (tid == 0) {
            const int old = __hip_atomic_fetch_add(&a.counters[kvh], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            is_last = (old == nact - 1);
        }
        __syncthreads();
        if (!is_last) return;
        ATTN_TSL(6);
        // last workgroup of the kv head: thread t merges outputs
        // [t*OPT, t*OPT+OPT) (one head g) from the split partials, 16 splits
        // per round trip, with an online rescale between batches:
        // out = sum_j o_j e^(m_j - M) / sum_j l_j e^(m_j - M)
        const float *pb = a.part + (size_t)kvh * a.nsplit * P;
        const int i0 = min(tid * OPT, G * D - OPT), g = i0 / D;
        float M = -INFINITY, L = 0.0f, O[OPT];
#pragma unroll
        for (int k = 0; k < OPT; k++) O[k] = 0.0f;
        for (int j0 = 0; j0 < nact; j0 += 16) {
            float mv[16], lv[16], ov[16][OPT];
#pragma unroll
            for (int k2 = 0; k2 < 16; k2++) {
                const float *pj = pb + (size_t)min(j0 + k2, nact - 1) * P;
                mv[k2] = ld_agent(pj + G * D + 2 * g);
                lv[k2] = ld_agent(pj + G * D + 2 * g + 1);
#pragma unroll
                for (int k = 0; k < OPT; k++) ov[k2][k] = ld_agent(pj + i0 + k);
            }
            float Mb = M;
#pragma unroll
            for (int k2 = 0; k2 < 16; k2++)
                if (j0 + k2 < nact) Mb = fmaxf(Mb, mv[k2]);
            const float r = (M == -INFINITY) ? 0.0f : __expf(M - Mb);
            L *= r;
#pragma unroll
            for (int k = 0; k < OPT; k++) O[k] *= r;
#pragma unroll
            for (int k2 = 0; k2 < 16; k2++) {
                if (j0 + k2 < nact) {
                    const float w = (mv[k2] == -INFINITY) ? 0.0f : __expf(mv[k2] - Mb);
                    L += lv[k2] * w;
#pragma unroll
                    for (int k = 0; k < OPT; k++) O[k] += ov[k2][k] * w;
                }
            }
            M = Mb;
        }
        __syncthreads();  // red (mo) is rewritten below
        if (tid * OPT < G * D) {
#pragma unroll
            for (int k = 0; k < OPT; k++) {
                const float v = O[k] * (1.0f / L);
                mo[i0 + k] = v;
                if (a.out) a.out[(size_t)kvh * G * D + i0 + k] = v;
            }
        }
        ATTN_TSL(9);
        if (tid == 0) __hip_atomic_store(&a.counters[kvh], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (nact == 1) ATTN_TS(7); else ATTN_TSL(7);
    if (a.oq) {
        // Q8_0 copy of this kv head's G*D outputs (quantize_input_q8_0_into), 32 lanes per block
        const int nb = G * D / 32;
        for (int b = tid >> 5; b < nb; b += kAttnThreads / 32) {
            const int gb = kvh * nb + b;
            quant_block32_lanes(mo[b * 32 + (tid & 31)], a.oq + gb * 32, a.os + gb, a.osum + gb);
        }
    }
    if (nact == 1) ATTN_TS(8); else ATTN_TSL(8);
}

}  // namespace fl
