// Split-K GQA decode attention kernel (gfx950 wave64).
#pragma once

#include <type_traits>

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
    const void *kc, *vc; // this layer's cache (F32/F16 values, Q8 int8 codes, KIVI 2-bit codes)
    long long tok_stride, head_stride;  // elements between slots / kv heads (F32/F16/Q8)
    const int *posp;     // attends slots 0..*posp
    int nkv, nsplit;     // grid = (nsplit, nkv)
    int chmin;           // minimum tokens per split (a multiple of attn_tpp(D))
    int single;          // MFMA kernel: contexts up to this many tokens run as one split
    int waves;           // MFMA kernel: waves per workgroup (4 or 8; other values mean 8)
    float *part;         // [nkv][nsplit][G][D+2] split partials
    int *counters;       // [nkv] arrival counters (zero between launches)
    float *out;          // [nh*D]
    int8_t *oq;          // optional Q8_0 copy of out (the wo matvec input)
    float *os;
    int *osum;
    long long *trace;    // FLARE_ATTN_TRACE builds: per-phase timestamps of workgroup (0,0)
    // Q8 / KIVI caches (head-major, max_seq slots per kv head)
    int S;               // slots per kv head (a multiple of 32)
    uint16_t *ks, *vs;   // Q8: f16 scale per 32 values [kvh][S][D/32]
    uint32_t *kp, *vp;   // KIVI: (scale, min) f16 pairs; K [kvh][S/32][D], V [kvh][S][D/32]
    __half *rk, *rv;     // KIVI: fp16 residual ring [kvh][kKiviRing][D]
    // new token (Q8 / KIVI decode step): K / V rows [nkv*D] as f32 from the
    // QKV epilogue; quantized (Q8) or rounded (KIVI ring) and stored into the
    // cache slot *posp by the workgroup whose chunk holds it.  nullptr when
    // the cache was written beforehand (fl_kv_write).
    const float *knew, *vnew;
    // several query tokens (speculative verify): grid z = query index; query
    // z sits at position *posp + z and attends slots 0..*posp+z (causal).
    // q / out / oq advance by qstride / ostride floats per query; split
    // partials and counters have one set per query.
    int qstride, ostride;
    int v_tblk;  // F16 / Q8 model caches: V stored in 32-slot transposed blocks [slot/32][D][32]
    // MFMA kernel, several queries: grid z = query pairs; the model's G/2
    // query heads of queries 2z and 2z+1 (kernel G = 2 x the model's) share
    // each K/V block, query 2z masking slot *posp + 2z + 1
    int qpair;
    int nq;  // k_attq: queries of the pass (even)
};

// Fused QKV + attention launch (k_qkv_attm): the attention workgroups of kv
// head h wait until count[h] reaches target (the QKV workgroups of h have
// published q and the new K / V rows), with a bounded spin that sets *err
// and proceeds on timeout, so every wave exits.
struct FuseWait {
    int *count;
    int target;
    int *err;
};
constexpr int kFuseSpinLimit = 1 << 22;

// Offset of (slot t, channel d) in one kv head's transposed V store.
__host__ __device__ inline size_t vt_off(int t, int d, int D) {
    return ((size_t)(t >> 5) * D + d) * 32 + (t & 31);
}

// KIVI 2-bit cache constants: groups of 32 (K per channel over 32 tokens, V
// per token over 32 channels); the newest tokens stay in an fp16 ring.
constexpr int kKiviGroup = 32;
constexpr int kKiviResidual = 128;  // at least this many newest tokens are fp16
// ring slots per kv head: the window plus two groups, so a verify batch of up
// to 32 tokens still finds every query's window tokens in the ring
constexpr int kKiviRing = kKiviResidual + 2 * kKiviGroup;
static_assert(kKiviRing % 32 == 0, "ring blocks of 32 slots");
// Tokens [0, kivi_qlen(T)) of a T-token cache are read from the 2-bit groups,
// [kivi_qlen(T), T) from the ring (between 129 and 160 tokens once T > 128).
__host__ __device__ inline int kivi_qlen(int T) {
    return T - 1 - kKiviResidual > 0 ? kKiviGroup * ((T - 1 - kKiviResidual) / kKiviGroup) : 0;
}

// KV storage tags for the attention kernel
struct KvQ8 {};
struct KvKivi {};



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

__device__ __forceinline__ void h8_to_f32(const v4i_t &v, float *o) {
    const uint32_t w[4] = {(uint32_t)v.x, (uint32_t)v.y, (uint32_t)v.z, (uint32_t)v.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        o[2 * i] = h2f((uint16_t)(w[i] & 0xFFFF));
        o[2 * i + 1] = h2f((uint16_t)(w[i] >> 16));
    }
}
__device__ __forceinline__ v4i_t f32_to_h8(const float *x) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; i++) w[i] = (uint32_t)f2h(x[2 * i]) | ((uint32_t)f2h(x[2 * i + 1]) << 16);
    return v4i_t{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
}

// KIVI 2-bit group quantizer (quantize_to_packed arithmetic,
// flare-core/src/kv_cache.rs:336-371): min / max of the group, scale =
// (max - min) / 3 (0 for a range below f32::EPSILON), code =
// clamp(round((v - min) * 3 / range), 0, 3).  The (scale, min) pair is kept
// as two binary16 values; dequantization is code * scale + min.
struct KiviQ {
    float mn, inv, scale;
    __device__ __forceinline__ void init(float lo, float hi) {
        const float range = hi - lo;
        scale = fabsf(range) < 1.1920929e-7f ? 0.0f : range / 3.0f;
        inv = fabsf(scale) < 1.1920929e-7f ? 0.0f : 3.0f / range;
        mn = lo;
    }
    __device__ __forceinline__ uint32_t code(float v) const {
        if (scale == 0.0f) return 0u;
        return (uint32_t)fminf(fmaxf(roundf((v - mn) * inv), 0.0f), 3.0f);
    }
    __device__ __forceinline__ uint32_t packed() const { return (uint32_t)f2h(scale) | ((uint32_t)f2h(mn) << 16); }
};

// One token's K and V elements [8c, 8c+8) for kv head kvh, kept raw in
// registers and decoded at use.
template <typename KT>
struct KVRow;
template <>
struct KVRow<float> {
    v4f_t k0, k1, v0, v1;
    __device__ __forceinline__ void load(const AttnArgs &a, int kvh, int t, int c) {
        const size_t o = (size_t)kvh * a.head_stride + (size_t)t * a.tok_stride + 8 * c;
        const v4f_t *kp = (const v4f_t *)((const float *)a.kc + o), *vp = (const v4f_t *)((const float *)a.vc + o);
        k0 = kp[0]; k1 = kp[1]; v0 = vp[0]; v1 = vp[1];
    }
    __device__ __forceinline__ void getk(float *o) const {
        o[0] = k0.x; o[1] = k0.y; o[2] = k0.z; o[3] = k0.w; o[4] = k1.x; o[5] = k1.y; o[6] = k1.z; o[7] = k1.w;
    }
    __device__ __forceinline__ void getv(float *o) const {
        o[0] = v0.x; o[1] = v0.y; o[2] = v0.z; o[3] = v0.w; o[4] = v1.x; o[5] = v1.y; o[6] = v1.z; o[7] = v1.w;
    }
};
template <>
struct KVRow<__half> {
    v4i_t k, v;
    __device__ __forceinline__ void load(const AttnArgs &a, int kvh, int t, int c) {
        const size_t o = (size_t)kvh * a.head_stride + (size_t)t * a.tok_stride + 8 * c;
        k = *(const v4i_t *)((const __half *)a.kc + o);
        v = *(const v4i_t *)((const __half *)a.vc + o);
    }
    __device__ __forceinline__ void getk(float *o) const { h8_to_f32(k, o); }
    __device__ __forceinline__ void getv(float *o) const { h8_to_f32(v, o); }
};
// The new token's row for the Q8 / KIVI decode step: every thread builds the
// stored form of elements [8c, 8c+8) from the f32 QKV output (Q8: the four
// lanes of a 32-block agree on its scale through DPP; KIVI: binary16), so the
// thread that meets slot pos uses exactly what it stores.
template <typename KT>
struct NewRow {
    __device__ __forceinline__ void build(const AttnArgs &, int, int) {}
    __device__ __forceinline__ void store(const AttnArgs &, int, int, int) const {}
};
__device__ __forceinline__ void q8_block8(const float *x, v2i_t &q, uint16_t &s) {
    // quantize_input_q8_0_into arithmetic (model.rs:5557-5570) over a 32-block
    // spread across 4 adjacent lanes (8 values each); scale stored as binary16
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) amax = fmaxf(amax, fabsf(x[i]));
    amax = row_max<4>(amax);
    const float d = amax / 127.0f;
    const float id = (d != 0.0f) ? 127.0f / amax : 0.0f;
    uint32_t w[2] = {0u, 0u};
#pragma unroll
    for (int i = 0; i < 8; i++) w[i >> 2] |= (uint32_t)(uint8_t)q8_code(x[i] * id) << (8 * (i & 3));
    q = v2i_t{(int)w[0], (int)w[1]};
    s = f2h(d);
}
template <>
struct NewRow<KvQ8> {
    v2i_t k, v;
    uint32_t sc;  // K scale | V scale << 16 (binary16) of this lane's 32-block
    __device__ __forceinline__ void build(const AttnArgs &a, int kvh, int c) {
        const int D = (int)a.tok_stride;
        float kx[8], vx[8];
        const v4f_t *kp = (const v4f_t *)(a.knew + kvh * D + 8 * c), *vp = (const v4f_t *)(a.vnew + kvh * D + 8 * c);
        const v4f_t k0 = kp[0], k1 = kp[1], v0 = vp[0], v1 = vp[1];
        kx[0] = k0.x; kx[1] = k0.y; kx[2] = k0.z; kx[3] = k0.w; kx[4] = k1.x; kx[5] = k1.y; kx[6] = k1.z; kx[7] = k1.w;
        vx[0] = v0.x; vx[1] = v0.y; vx[2] = v0.z; vx[3] = v0.w; vx[4] = v1.x; vx[5] = v1.y; vx[6] = v1.z; vx[7] = v1.w;
        uint16_t sk, sv;
        q8_block8(kx, k, sk);
        q8_block8(vx, v, sv);
        sc = (uint32_t)sk | ((uint32_t)sv << 16);
    }
    // K row-major, V into the 32-slot transposed blocks
    __device__ __forceinline__ void store(const AttnArgs &a, int kvh, int t, int c) const {
        const int D = (int)a.tok_stride;
        int8_t *kc = (int8_t *)a.kc + (size_t)kvh * a.head_stride;
        int8_t *vc = (int8_t *)a.vc + (size_t)kvh * a.head_stride;
        *(v2i_t *)(kc + (size_t)t * D + 8 * c) = k;
#pragma unroll
        for (int i = 0; i < 8; i++)
            vc[((size_t)(t >> 5) * D + 8 * c + i) * 32 + (t & 31)] =
                (int8_t)(((uint32_t)(i < 4 ? v.x : v.y) >> (8 * (i & 3))) & 0xFF);
        if ((c & 3) == 0) {
            const size_t so = ((size_t)kvh * a.S + t) * (D >> 5) + (c >> 2);
            a.ks[so] = (uint16_t)(sc & 0xFFFF);
            a.vs[so] = (uint16_t)(sc >> 16);
        }
    }
};
// KIVI code placement: 32-bit words of 16 codes, two runs of 8 (run A, run
// B); code j of run A at bit 8 + 2(j/2) + 16(j%2), of run B at bit 2(j/2) +
// 16(j%2), so that code pair (2k, 2k+1) of a run reaches bits 8 and 24 (the
// units of 1/4 under binary16 1.0 in each half-word) with a single shift.
//  K (token rows of D/16 words): word kg*(D/64) + w holds channels
//    64w + 8kg + j (run A, 32-channel tile 2w) and 64w + 32 + 8kg + j (run B,
//    tile 2w+1): the codes an MFMA lane group kg needs for one token.
//  V (2D words per 32-token group): word (kg*16 + r)*(D/32) + w holds group
//    tokens 8kg + j of channel 32w + r (run A, 16-channel tile 2w) and of
//    channel 32w + 16 + r (run B, tile 2w+1): what lane (kg, r) reads.
__host__ __device__ inline int kivi_bit(int j, int run) { return (run ? 0 : 8) + 2 * (j >> 1) + 16 * (j & 1); }
// ring slot of token t; the ring V is stored in 32-slot transposed blocks
__host__ __device__ inline size_t kivi_ring_k(int kvh, int t, int c, int D) {
    return ((size_t)kvh * kKiviRing + (size_t)(t % kKiviRing)) * D + c;
}
__host__ __device__ inline size_t kivi_ring_v(int kvh, int t, int c, int D) {
    const int sl = t % kKiviRing;
    return (size_t)kvh * kKiviRing * D + ((size_t)(sl >> 5) * D + c) * 32 + (sl & 31);
}

template <>
struct NewRow<KvKivi> {
    v4i_t k, v;  // binary16 K / V of channels [8c, 8c+8)
    __device__ __forceinline__ void build(const AttnArgs &a, int kvh, int c) {
        const int D = (int)a.tok_stride;
        float kx[8], vx[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            kx[i] = a.knew[kvh * D + 8 * c + i];
            vx[i] = a.vnew[kvh * D + 8 * c + i];
        }
        k = f32_to_h8(kx);
        v = f32_to_h8(vx);
    }
    __device__ __forceinline__ void store(const AttnArgs &a, int kvh, int t, int c) const {
        const int D = (int)a.tok_stride;
        *(v4i_t *)(a.rk + kivi_ring_k(kvh, t, 8 * c, D)) = k;
        const uint32_t w[4] = {(uint32_t)v.x, (uint32_t)v.y, (uint32_t)v.z, (uint32_t)v.w};
#pragma unroll
        for (int i = 0; i < 8; i++)
            ((uint16_t *)a.rv)[kivi_ring_v(kvh, t, 8 * c + i, D)] = (uint16_t)((w[i >> 1] >> (16 * (i & 1))) & 0xFFFF);
    }
};

// Quantize KIVI group gi of kv head kvh (tokens [32gi, 32gi+32)) into the
// 2-bit store.  src(t, ch, is_v) returns the binary16-rounded value of token
// t, channel ch.  Every thread of the workgroup must call it (it holds
// barriers); lds: 3 * 32 * (D/32) floats of workgroup scratch.
//  K: per channel over the 32 tokens (4 channels = one code byte per thread).
//  V: per token over each 32-channel group, then one code byte (4 tokens of
//     one channel) per thread.
template <typename Src>
__device__ __forceinline__ void kivi_quantize_group(const AttnArgs &a, int D, int kvh, int gi, Src src, float *lds) {
    const int tid = threadIdx.x, nt = blockDim.x, DT = D >> 5;
    const int t0 = gi * kKiviGroup;
    // K parameters per channel over the group's 32 tokens
    for (int c = tid; c < D; c += nt) {
        float lo = INFINITY, hi = -INFINITY;
        for (int t = 0; t < kKiviGroup; t++) {
            const float v = src(t0 + t, c, false);
            lo = v < lo ? v : lo;
            hi = v > hi ? v : hi;
        }
        KiviQ qz;
        qz.init(lo, hi);
        a.kp[((size_t)kvh * (a.S >> 5) + gi) * D + c] = qz.packed();
        lds[3 * c] = qz.mn;
        lds[3 * c + 1] = qz.inv;
        lds[3 * c + 2] = qz.scale;
    }
    __syncthreads();
    // K codes: one word (16 channels of one token) per thread
    const int KWR = D / 16;
    for (int idx = tid; idx < kKiviGroup * KWR; idx += nt) {
        const int t = idx / KWR, wi = idx % KWR, kg = wi / (D / 64), w = wi % (D / 64);
        uint32_t word = 0;
#pragma unroll
        for (int run = 0; run < 2; run++)
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int c = 64 * w + 32 * run + 8 * kg + j;
                KiviQ qz;
                qz.mn = lds[3 * c];
                qz.inv = lds[3 * c + 1];
                qz.scale = lds[3 * c + 2];
                word |= qz.code(src(t0 + t, c, false)) << kivi_bit(j, run);
            }
        ((uint32_t *)a.kc)[((size_t)kvh * a.S + t0 + t) * KWR + wi] = word;
    }
    __syncthreads();  // lds is reused for the V parameters
    // V parameters per (token, 32-channel group)
    for (int idx = tid; idx < kKiviGroup * DT; idx += nt) {
        const int tl = idx % kKiviGroup, cg = idx / kKiviGroup;
        float lo = INFINITY, hi = -INFINITY;
        for (int i = 0; i < kKiviGroup; i++) {
            const float v = src(t0 + tl, 32 * cg + i, true);
            lo = v < lo ? v : lo;
            hi = v > hi ? v : hi;
        }
        KiviQ qz;
        qz.init(lo, hi);
        a.vp[((size_t)kvh * a.S + t0 + tl) * DT + cg] = qz.packed();
        lds[3 * idx] = qz.mn;
        lds[3 * idx + 1] = qz.inv;
        lds[3 * idx + 2] = qz.scale;
    }
    __syncthreads();
    // V codes: one byte = 4 tokens of one channel
    // V codes: one word (8 tokens of two channels) per thread
    uint32_t *vg = (uint32_t *)a.vc + ((size_t)kvh * (a.S >> 5) + gi) * (size_t)(2 * D);
    for (int idx = tid; idx < 2 * D; idx += nt) {
        const int ln = idx / DT, w = idx % DT, kg = ln >> 4, r = ln & 15;
        uint32_t word = 0;
#pragma unroll
        for (int run = 0; run < 2; run++) {
            const int c = 32 * w + 16 * run + r;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int tl = 8 * kg + j, li = (c >> 5) * kKiviGroup + tl;
                KiviQ qz;
                qz.mn = lds[3 * li];
                qz.inv = lds[3 * li + 1];
                qz.scale = lds[3 * li + 2];
                word |= qz.code(src(t0 + tl, c, true)) << kivi_bit(j, run);
            }
        }
        vg[idx] = word;
    }
    __syncthreads();
}

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
__global__ __launch_bounds__(kAttnThreads) void k_attn(AttnArgs a0) {
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
    const int pos = *a.posp + zq, T = pos + 1;
    int CH = max(a.chmin, (T + a.nsplit - 1) / a.nsplit);
    CH = (CH + TPP - 1) / TPP * TPP;
    const int t0 = s * CH;
    if (t0 >= T) return;
    const int t1 = min(T, t0 + CH);
    const int nact = (T + CH - 1) / CH;
    KVRow<KT> rows[NP];
    auto fetch = [&](int tb) {
#pragma unroll
        for (int p = 0; p < NP; p++) {
            const int tu = tb + tk + p * TPP;
            const int t = min(tu, t1 - 1);
            rows[p].load(a, kvh, t, c);
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
            rows[p].getk(kk);
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
            rows[p].getv(vv);
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
        if (!split_arrive_last<false>(&a.counters[kvh], nact, &is_last)) return;
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
