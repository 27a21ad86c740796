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
    const float *q;      // [nh*D]
    const float *knew;   // [nkv*D] un-rotated new key (or null)
    const float *vnew;   // [nkv*D]
    const float *rope;   // rope table base: cos [maxpos][D/2] then sin at +sin_off
    long long sin_off;
    void *kc, *vc;       // cache for this layer
    long long tok_stride, head_stride;  // elements between slots / kv heads
    const int *posp;     // attends slots 0..*posp
    int nkv, nsplit, chmax;
    int chmin;           // minimum tokens per split (a multiple of the batch size)
    float *part;         // [nkv][nsplit][G][D+2]
    int *counters;       // [nkv]
    float *out;          // [nh*D]
    int8_t *oq;          // optional Q8 output
    float *os;
    int *osum;
    int skip_merge;      // timing experiments only
    long long *trace;    // FLARE_ATTN_TRACE builds: per-phase timestamps of workgroup (0,0)
};

#ifdef FLARE_ATTN_TRACE
#define ATTN_TS(i)                                                                          \
    do {                                                                                    \
        if (a.trace && blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0)             \
            a.trace[i] = (long long)__builtin_amdgcn_s_memrealtime();                       \
    } while (0)
#else
#define ATTN_TS(i) \
    do {           \
    } while (0)
#endif

template <typename KT>
__device__ __forceinline__ void load8(const KT *p, float *v);
template <>
__device__ __forceinline__ void load8<__half>(const __half *p, float *v) {
    const int4 t = *(const int4 *)p;
    const uint32_t w[4] = {(uint32_t)t.x, (uint32_t)t.y, (uint32_t)t.z, (uint32_t)t.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        v[2 * i] = h2f((uint16_t)(w[i] & 0xFFFF));
        v[2 * i + 1] = h2f((uint16_t)(w[i] >> 16));
    }
}
template <>
__device__ __forceinline__ void load8<float>(const float *p, float *v) {
    const float4 a = ((const float4 *)p)[0], b = ((const float4 *)p)[1];
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
    int4 v;
    __device__ __forceinline__ void load(const __half *p) { v = *(const int4 *)p; }
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
    float4 a, b;
    __device__ __forceinline__ void load(const float *p) {
        a = ((const float4 *)p)[0];
        b = ((const float4 *)p)[1];
    }
    __device__ __forceinline__ void get(float *o) const {
        o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w; o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
    }
};

__device__ __forceinline__ float kv_to_f32(__half v) { return __half2float(v); }
__device__ __forceinline__ float kv_to_f32(float v) { return v; }
__device__ __forceinline__ float kv_round(float v, const __half *) { return h2f(f2h(v)); }
__device__ __forceinline__ float kv_round(float v, const float *) { return v; }
__device__ __forceinline__ void kv_store(__half *p, float v) { *p = __ushort_as_half(f2h(v)); }
__device__ __forceinline__ void kv_store(float *p, float v) { *p = v; }

// Online-softmax state merge (flash-decode rescale): (m1,l1,o1) += (m2,l2,o2).
template <int G, int EPL>
__device__ __forceinline__ void ms_merge(float *m, float *l, float (*o)[EPL], const float *m2, const float *l2,
                                         const float (*o2)[EPL]) {
#pragma unroll
    for (int g = 0; g < G; g++) {
        const float M = fmaxf(m[g], m2[g]);
        const float a1 = (m[g] == -INFINITY) ? 0.0f : expf(m[g] - M);
        const float a2 = (m2[g] == -INFINITY) ? 0.0f : expf(m2[g] - M);
        l[g] = l[g] * a1 + l2[g] * a2;
#pragma unroll
        for (int e = 0; e < EPL; e++) o[g][e] = o[g][e] * a1 + o2[g][e] * a2;
        m[g] = M;
    }
}

constexpr int kAttnThreads = 1024;  // 16 waves per workgroup (4 per SIMD)
constexpr int kAttnNB = 2;          // tokens per thread per batch (K/V loads issued together)

// Tokens covered per batch, and the minimum chunk per split: contexts up to
// 4 batches run one workgroup per kv head and need no cross-workgroup merge.
__host__ __device__ constexpr int attn_tpp(int D) { return kAttnThreads / (D / 8); }
__host__ __device__ constexpr int attn_batch(int D) { return attn_tpp(D) * kAttnNB; }
__host__ __device__ constexpr int attn_chmin(int D) { return attn_batch(D); }

// Workgroup (s, kvh) covers tokens [t0, t1) of kv head kvh for its G query
// heads.  Per batch of NB*TPP tokens: scores -> LDS, per-head batch max ->
// workgroup-uniform running max M, p = exp(s - M) once per (head, token),
// o += p * v with the thread's V registers.  Since M is shared by all
// threads, the final cross-thread reduction of o and l is a plain sum.
template <typename KT, int D, int G>
__global__ __launch_bounds__(kAttnThreads) __attribute__((amdgpu_waves_per_eu(1, 4))) void k_attn(AttnArgs a) {
    constexpr int EPL = 8;                  // elements per lane per token row
    constexpr int LPT = D / EPL;            // lanes per token row (8 or 16): one DPP row group
    constexpr int TPP = kAttnThreads / LPT; // tokens per pass
    constexpr int NB = kAttnNB;
    constexpr int TB = TPP * NB;            // tokens per batch
    constexpr int NW = kAttnThreads / 64;
    __shared__ float kn[D], vn[D];
    __shared__ float sc[G][TB];             // scores, then probabilities
    __shared__ float Mx[G], bmax[G];
    __shared__ float lpart[NW][G];
    __shared__ float lchunk[G * (kAttnThreads / 8 * kAttnNB) / 64 + 1];
    __shared__ float linv[G];
    __shared__ int is_last;
    // dynamic: per-wave o partials [NW][G*D] (then the final output), then the
    // merge buffers m / weights [nsplit*G] and l [nsplit*G]
    extern __shared__ float dyn[];
    float(*ow)[G * D] = (float(*)[G * D])dyn;

    const int kvh = blockIdx.y, s = blockIdx.x, tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    ATTN_TS(0);
    const int pos = *a.posp;
    const int T = pos + 1;
    const int CH = max(a.chmin, (T + a.nsplit - 1) / a.nsplit);
    const int t0 = s * CH;
    if (t0 >= T) return;
    const int t1 = min(T, t0 + CH);
    const int nact = (T + CH - 1) / CH;
    const int half = D / 2;
    const int tk = tid / LPT, c = tid % LPT;
    KT *kc = (KT *)a.kc, *vc = (KT *)a.vc;

    // q and the rope row go out first; the first K/V batch right after
    const bool rot = a.knew != nullptr;
    const float *cs = a.rope + (size_t)pos * half;
    const float *sn = cs + a.sin_off;
    float qr[G][EPL];
#pragma unroll
    for (int g = 0; g < G; g++) {
        const float4 *qp = (const float4 *)(a.q + (size_t)(kvh * G + g) * D + c * EPL);
        const float4 q0 = qp[0], q1 = qp[1];
        qr[g][0] = q0.x; qr[g][1] = q0.y; qr[g][2] = q0.z; qr[g][3] = q0.w;
        qr[g][4] = q1.x; qr[g][5] = q1.y; qr[g][6] = q1.z; qr[g][7] = q1.w;
    }
    const bool lo = c < LPT / 2;
    const int d0 = (lo ? c : c - LPT / 2) * EPL;
    float co[EPL], si[EPL];
    if (rot) {
#pragma unroll
        for (int e = 0; e < EPL; e++) { co[e] = cs[d0 + e]; si[e] = sn[d0 + e]; }
    }
    // K: token-parallel (LPT lanes per row, NB tokens per thread per batch).
    // V: wave-parallel by dimension: wave w owns batch tokens [w*TPW, w*TPW+TPW)
    // and lane l holds elements [l*EPV, l*EPV+EPV) of those rows.
    constexpr int TPW = TB / NW;   // tokens per wave per batch
    constexpr int EPV = D / 64;    // V elements per lane (1 or 2)
    KVRaw<KT> kb[NB];
    KT vb[TPW][EPV];
    auto fetch_batch = [&](int tb) {
#pragma unroll
        for (int j = 0; j < NB; j++) {
            const int tt = min(tb + tk + j * TPP, t1 - 1);
            kb[j].load(kc + (size_t)tt * a.tok_stride + (size_t)kvh * a.head_stride + c * EPL);
        }
#pragma unroll
        for (int j = 0; j < TPW; j++) {
            const int tt = min(tb + wave * TPW + j, t1 - 1);
            const KT *vp = vc + (size_t)tt * a.tok_stride + (size_t)kvh * a.head_stride + lane * EPV;
#pragma unroll
            for (int e = 0; e < EPV; e++) vb[j][e] = vp[e];
        }
    };
    fetch_batch(t0);
    ATTN_TS(1);
    if (rot) {
        // rotate-half: lane c's partner (element d +- D/2) is lane c ^ (LPT/2)
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
            for (int e = 0; e < EPL; e++) {
                const float own = qr[g][e], other = __shfl_xor(own, LPT / 2, 64);
                qr[g][e] = lo ? (own * co[e] - other * si[e]) : (other * si[e] + own * co[e]);
            }
    }
    ATTN_TS(2);
    const bool has_new = rot && (t1 == T);
    if (has_new && tid < D) {
        // RoPE the new key (apply_rope_with_table) and store K/V at slot pos
        const int d = tid;
        const float *kh = a.knew + (size_t)kvh * D, *vh = a.vnew + (size_t)kvh * D;
        float kr;
        if (d < half) kr = kh[d] * cs[d] - kh[d + half] * sn[d];
        else kr = kh[d - half] * sn[d - half] + kh[d] * cs[d - half];
        kr = kv_round(kr, (const KT *)nullptr);
        const float vr = kv_round(vh[d], (const KT *)nullptr);
        kn[d] = kr;
        vn[d] = vr;
        const size_t off = (size_t)pos * a.tok_stride + (size_t)kvh * a.head_stride + d;
        kv_store(kc + off, kr);
        kv_store(vc + off, vr);
    }
    if (tid < G) Mx[tid] = -INFINITY;
    __syncthreads();
    ATTN_TS(3);

    const float scale = 1.0f / sqrtf((float)D);
    float o[G][EPV], lp = 0.0f;
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int e = 0; e < EPV; e++) o[g][e] = 0.0f;
    for (int tb0 = t0; tb0 < t1; tb0 += TB) {
        const int nb_tok = min(TB, t1 - tb0);
        KT vx[TPW][EPV];
        // scores of this batch (token tb0 + tk + j*TPP), reduced over the row group
#pragma unroll
        for (int j = 0; j < NB; j++) {
            const int t = tb0 + tk + j * TPP;
            float kk[EPL];
            kb[j].get(kk);
            if (has_new && t == pos) {
#pragma unroll
                for (int e = 0; e < EPL; e++) kk[e] = kn[c * EPL + e];
            }
#pragma unroll
            for (int g = 0; g < G; g++) {
                float p = 0.0f;
#pragma unroll
                for (int e = 0; e < EPL; e++) p += qr[g][e] * kk[e];
                p = row_sum<LPT>(p);
                if (c == 0 && t < t1) sc[g][tk + j * TPP] = p * scale;
            }
        }
#pragma unroll
        for (int j = 0; j < TPW; j++)
#pragma unroll
            for (int e = 0; e < EPV; e++) vx[j][e] = vb[j][e];
        if (tb0 == t0) ATTN_TS(10);
        if (tb0 + TB < t1) fetch_batch(tb0 + TB);  // next batch in flight during the softmax
        __syncthreads();
        if (tb0 == t0) ATTN_TS(11);
        // per-head max of the batch (one wave per head)
        for (int g = wave; g < G; g += NW) {
            float mv = -INFINITY;
            for (int i = lane; i < nb_tok; i += 64) mv = fmaxf(mv, sc[g][i]);
            mv = wave_max(mv);
            if (lane == 0) bmax[g] = mv;
        }
        if (tb0 == t0) ATTN_TS(12);
        __syncthreads();
        if (tb0 == t0) ATTN_TS(13);
        // workgroup-uniform running max; rescale the accumulators
        float Mn[G];
#pragma unroll
        for (int g = 0; g < G; g++) {
            const float Mo = Mx[g];
            Mn[g] = fmaxf(Mo, bmax[g]);
            const float al = (Mo == -INFINITY) ? 0.0f : expf(Mo - Mn[g]);
#pragma unroll
            for (int e = 0; e < EPV; e++) o[g][e] *= al;
            if (tid == g) lp *= al;  // thread g keeps head g's partial denominator
        }
        // probabilities once per (head, token); each 64-token chunk of a head
        // is one wave, whose sum goes to lchunk (TB is a multiple of 64)
        for (int i = tid; i < G * TB; i += kAttnThreads) {
            const int g = i / TB, j = i % TB;
            float p = 0.0f;
            if (j < nb_tok) {
                p = expf(sc[g][j] - Mn[g]);
                sc[g][j] = p;
            }
            p = wave_sum(p);
            if (lane == 0) lchunk[i >> 6] = p;
        }
        if (tb0 == t0) ATTN_TS(14);
        __syncthreads();
        if (tb0 == t0) ATTN_TS(15);
        if (tid < G) {
            float l = 0.0f;
            for (int k = 0; k < TB / 64; k++) l += lchunk[tid * (TB / 64) + k];
            lp += l;
            Mx[tid] = Mn[tid];
        }
        // o += p * v over this wave's tokens
#pragma unroll
        for (int j = 0; j < TPW; j++) {
            const int jj = wave * TPW + j;
            if (jj < nb_tok) {
                float vv[EPV];
#pragma unroll
                for (int e = 0; e < EPV; e++)
                    vv[e] = (has_new && tb0 + jj == pos) ? vn[lane * EPV + e] : kv_to_f32(vx[j][e]);
#pragma unroll
                for (int g = 0; g < G; g++) {
                    const float p = sc[g][jj];
#pragma unroll
                    for (int e = 0; e < EPV; e++) o[g][e] += p * vv[e];
                }
            }
        }
        if (tb0 == t0) ATTN_TS(16);
        __syncthreads();  // sc / Mx reused by the next batch
        if (tb0 == t0) ATTN_TS(17);
    }
    ATTN_TS(4);
    // o: one row of G*D per wave in LDS, summed over the waves below
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int e = 0; e < EPV; e++) ow[wave][g * D + lane * EPV + e] = o[g][e];
    if (tid < G) lpart[0][tid] = lp;
    ATTN_TS(5);
    __syncthreads();
    ATTN_TS(6);
    float res[(G * D + kAttnThreads - 1) / kAttnThreads];
    {
        int k = 0;
        for (int i = tid; i < G * D; i += kAttnThreads, k++) {
            float O = 0.0f;
#pragma unroll
            for (int w = 0; w < NW; w++) O += ow[w][i];
            res[k] = O;
        }
    }
    float Lg[G];
#pragma unroll
    for (int g = 0; g < G; g++) Lg[g] = lpart[0][g];
    __syncthreads();  // ow is overwritten with the final output below
    float *mo = &ow[0][0];
    if (nact == 1) {
        int k = 0;
        for (int i = tid; i < G * D; i += kAttnThreads, k++) {
            const float v = res[k] * (1.0f / Lg[i / D]);
            mo[i] = v;
            a.out[(size_t)kvh * G * D + i] = v;
        }
    } else {
        // publish this split's partial (m, l, unnormalised o)
        // Publish this split's partial (m, l, unnormalised o) with agent-scope
        // atomic stores (written through to the device coherence point, so no
        // L2 write-back fence is needed), wait for their completion, then count
        // the split in.  The last split reads the partials back with
        // agent-scope atomic loads.
        const int P = G * (D + 2);
        float *mypart = a.part + ((size_t)kvh * a.nsplit + s) * P;
        {
            int k = 0;
            for (int i = tid; i < G * D; i += kAttnThreads, k++) st_agent(mypart + i, res[k]);
        }
        if (tid < G) {
            st_agent(mypart + G * D + 2 * tid, Mx[tid]);
            st_agent(mypart + G * D + 2 * tid + 1, Lg[tid]);
        }
        __builtin_amdgcn_s_waitcnt(0);  // all stores of this thread acknowledged
        __syncthreads();
        if (tid == 0) {
            const int old = __hip_atomic_fetch_add(&a.counters[kvh], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            is_last = (old == nact - 1);
        }
        __syncthreads();
        if (!is_last || a.skip_merge) return;
        // last workgroup of this kv head: merge the nact split partials
        float *mw = dyn + NW * G * D;    // [nact*G] m, then weights
        float *lw = mw + a.nsplit * G;   // [nact*G] l
        const float *pbase = a.part + (size_t)kvh * a.nsplit * P;
        for (int i = tid; i < nact * G; i += kAttnThreads) {
            const int j = i / G, g = i % G;
            mw[i] = ld_agent(pbase + (size_t)j * P + G * D + 2 * g);
            lw[i] = ld_agent(pbase + (size_t)j * P + G * D + 2 * g + 1);
        }
        __syncthreads();
        for (int g = wave; g < G; g += NW) {
            float M = -INFINITY;
            for (int j = lane; j < nact; j += 64) M = fmaxf(M, mw[j * G + g]);
            M = wave_max(M);
            float L = 0.0f;
            for (int j = lane; j < nact; j += 64) {
                const float mj = mw[j * G + g];
                const float w = (mj == -INFINITY) ? 0.0f : expf(mj - M);
                mw[j * G + g] = w;
                L += lw[j * G + g] * w;
            }
            L = wave_sum(L);
            if (lane == 0) linv[g] = 1.0f / L;
        }
        __syncthreads();
        for (int i = tid; i < G * D; i += kAttnThreads) {
            const int g = i / D;
            float O = 0.0f;
            int j = 0;
            for (; j + 4 <= nact; j += 4) {
                const float o0 = ld_agent(pbase + (size_t)j * P + i);
                const float o1 = ld_agent(pbase + (size_t)(j + 1) * P + i);
                const float o2 = ld_agent(pbase + (size_t)(j + 2) * P + i);
                const float o3 = ld_agent(pbase + (size_t)(j + 3) * P + i);
                O += o0 * mw[j * G + g];
                O += o1 * mw[(j + 1) * G + g];
                O += o2 * mw[(j + 2) * G + g];
                O += o3 * mw[(j + 3) * G + g];
            }
            for (; j < nact; j++) O += ld_agent(pbase + (size_t)j * P + i) * mw[j * G + g];
            const float v = O * linv[g];
            mo[i] = v;
            a.out[(size_t)kvh * G * D + i] = v;
        }
        if (tid == 0) __hip_atomic_store(&a.counters[kvh], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    ATTN_TS(7);
    if (a.oq) {
        // Q8_0 quantization of this kv head's G*D outputs: 32 lanes per block
        const int nb = G * D / 32;
        for (int b = tid >> 5; b < nb; b += kAttnThreads / 32) {
            const int gb = kvh * nb + b;
            quant_block32_lanes(mo[b * 32 + (tid & 31)], a.oq + gb * 32, a.os + gb, a.osum + gb);
        }
    }
    ATTN_TS(8);
}

}  // namespace fl
