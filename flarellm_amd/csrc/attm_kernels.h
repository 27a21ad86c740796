// Split-K GQA decode attention on f16 MFMA (fp16, Q8 and KIVI2 KV caches).
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
// KIVI2 caches: 2-bit codes are exact in f16; K (scale, min) per channel
// folds the scale into the query operand and adds sum(q * min) per head, V
// (scale, min) per (token, 32 channels) folds the scale into P and adds
// sum(p * min) per (head, channel group).  Tokens above the quantized prefix
// come from the fp16 ring exactly as for an fp16 cache.
#pragma once

#include "attn_kernels.h"

namespace fl {

typedef _Float16 v8h_t __attribute__((ext_vector_type(8)));
typedef float v4f32_t __attribute__((ext_vector_type(4)));

constexpr int kAttmThreads = 512;  // 8 waves, each walking 32-token blocks
constexpr int kAttmBlock = 32;
constexpr int kAttmMaxSplit = 64;
constexpr int kAttmSingle = 1024;  // contexts up to this many tokens run as one split

__device__ __forceinline__ v4f32_t mfma16(const v8h_t &a, const v8h_t &b, const v4f32_t &c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// 8 floats -> f16 high parts and f16 residuals.  The high part is rounded
// toward zero by v_cvt_pkrtz_f16_f32, an operation the compiler cannot
// re-derive from the expression that produced x: a plain conversion let it
// form the high part straight from a product (one rounding, v_fma_mix) for
// the residual while storing the conversion of the rounded fp32 product, so
// the two could differ by one f16 unit.  x - hi is exact in fp32 and leaves
// one f16 rounding for the residual (~22 bits together).
__device__ __forceinline__ void split8(const float *x, v8h_t &hi, v8h_t &lo) {
#pragma unroll
    for (int i = 0; i < 8; i += 2) {
        const auto h2 = __builtin_amdgcn_cvt_pkrtz(x[i], x[i + 1]);
        _Float16 h[2];
        __builtin_memcpy(h, &h2, 4);
        hi[i] = h[0];
        hi[i + 1] = h[1];
        lo[i] = (_Float16)(x[i] - (float)h[0]);
        lo[i + 1] = (_Float16)(x[i + 1] - (float)h[1]);
    }
}

__device__ __forceinline__ v8h_t as_h8(const v4i_t &v) {
    v8h_t r;
    __builtin_memcpy(&r, &v, 16);
    return r;
}

// int8 codes -> exact f16 values: bias each byte to unsigned (xor 0x80), make
// it the low byte of binary16 0x64XX = 1024 + XX with one byte permute per two
// codes (v_perm_b32 picks bytes of the codes and of 0x64646464), then
// subtract 1152 = 1024 + 128 in packed f16 (every value is an integer below
// 2048, so each step is exact).
__device__ __forceinline__ v8h_t i8x8_to_h8(const v2i_t &c) {
    const uint32_t u0 = (uint32_t)c.x ^ 0x80808080u, u1 = (uint32_t)c.y ^ 0x80808080u;
    constexpr uint32_t m = 0x64646464u;
    uint32_t d[4];
    d[0] = __builtin_amdgcn_perm(m, u0, 0x04010400u);  // bytes: u0.b0, 0x64, u0.b1, 0x64
    d[1] = __builtin_amdgcn_perm(m, u0, 0x04030402u);
    d[2] = __builtin_amdgcn_perm(m, u1, 0x04010400u);
    d[3] = __builtin_amdgcn_perm(m, u1, 0x04030402u);
    v8h_t r;
    __builtin_memcpy(&r, d, 16);
    const _Float16 k = (_Float16)1152.0f;
    const v8h_t bias = {k, k, k, k, k, k, k, k};
    return r - bias;
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

// Q8: int8 codes + f16 scale per (slot, 32-channel block), with the V
// scales of slot tb + lane % 32.
template <int D>
struct AttmTile<KvQ8, D> {
    static constexpr int DT = D / 32, NT = D / 16, VW = (DT + 1) / 2;
    v2i_t k[2][DT];
    v2i_t v[NT];
    uint32_t ksc[2][VW];  // this lane's slot: K scales (2 per word)
    uint32_t vsc[VW];     // slot tb + lane % 32: V scales (2 per word)
    __device__ __forceinline__ void load_k(const AttnArgs &a, int kvh, int tb, int tlast, int lane) {
        const int8_t *kc = (const int8_t *)a.kc + (size_t)kvh * a.head_stride;
        const int kg = lane >> 4, r = lane & 15;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int t = min(tb + 16 * h + r, tlast);
#pragma unroll
            for (int dt = 0; dt < DT; dt++) k[h][dt] = *(const v2i_t *)(kc + (size_t)t * D + 32 * dt + 8 * kg);
            const uint32_t *sp = (const uint32_t *)(a.ks + ((size_t)kvh * a.S + t) * DT);
#pragma unroll
            for (int w = 0; w < VW; w++) ksc[h][w] = sp[w];
        }
    }
    __device__ __forceinline__ void load_v(const AttnArgs &a, int kvh, int tb, int tlast, int lane) {
        const int8_t *vc = (const int8_t *)a.vc + (size_t)kvh * a.head_stride;
        const int kg = lane >> 4, r = lane & 15;
#pragma unroll
        for (int nt = 0; nt < NT; nt++) v[nt] = *(const v2i_t *)(vc + vt_off(tb, 16 * nt + r, D) + 8 * kg);
        const int t = min(tb + (lane & 31), tlast);
        const uint32_t *sp = (const uint32_t *)(a.vs + ((size_t)kvh * a.S + t) * DT);
#pragma unroll
        for (int w = 0; w < VW; w++) vsc[w] = sp[w];
    }
    __device__ __forceinline__ void load(const AttnArgs &a, int kvh, int tb, int tlast, int lane) {
        load_k(a, kvh, tb, tlast, lane);
        load_v(a, kvh, tb, tlast, lane);
    }
};

// N consecutive 32-bit words (N = 1, 2, 4) in one load
template <int N>
__device__ __forceinline__ void ld_words(const void *p, uint32_t *w) {
    if constexpr (N == 4) {
        const v4i_t v = *(const v4i_t *)p;
        w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
    } else if constexpr (N == 2) {
        const v2i_t v = *(const v2i_t *)p;
        w[0] = v.x; w[1] = v.y;
    } else {
        w[0] = *(const uint32_t *)p;
    }
}

// KIVI2, a block of the 2-bit prefix: the lane's codes (K: 8 channels of
// every 32-channel tile for its slot; V: 8 slots of its channel in every
// 16-channel tile) and the block's (scale, min) pairs, all in one flight.
template <int D>
struct AttmKiviQ {
    static constexpr int DT = D / 32, KW = D / 64;
    uint32_t k[2][KW];  // [slot half] word w: 32-channel tiles 2w, 2w+1 (runs A, B)
    uint32_t v[DT];     // word w: 16-channel tiles 2w, 2w+1 (runs A, B)
    uint32_t kp[KW];    // K pairs of channels lane + 64i (the block's group)
    uint32_t vp[DT];    // V pairs of slot tb + lane % 32, per 32-channel group
    __device__ __forceinline__ void load(const AttnArgs &a, int kvh, int tb, int tlast, int lane) {
        const int kg = lane >> 4, r = lane & 15;
        const uint8_t *kc = (const uint8_t *)a.kc, *vc = (const uint8_t *)a.vc;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int t = min(tb + 16 * h + r, tlast);
            ld_words<KW>(kc + ((size_t)kvh * a.S + t) * (D / 4) + kg * (D / 16), k[h]);
        }
        const size_t gi = (size_t)kvh * (a.S >> 5) + (tb >> 5);
        ld_words<DT>(vc + gi * (size_t)(D * 8) + (kg * 16 + r) * (D / 16) * 2, v);
#pragma unroll
        for (int i = 0; i < KW; i++) kp[i] = a.kp[gi * D + lane + 64 * i];
        const int t = min(tb + (lane & 31), tlast);
        ld_words<DT>(a.vp + ((size_t)kvh * a.S + t) * DT, vp);
    }
};

// KIVI2, a block of the fp16 ring: K rows and transposed V as for fp16
template <int D>
struct AttmTile<KvKivi, D> {
    static constexpr int DT = D / 32, NT = D / 16;
    v4i_t k[2][DT];
    v4i_t v[NT];
    __device__ __forceinline__ void load(const AttnArgs &a, int kvh, int tb, int tlast, int lane) {
        const int kg = lane >> 4, r = lane & 15;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int t = min(tb + 16 * h + r, tlast);
#pragma unroll
            for (int dt = 0; dt < DT; dt++) k[h][dt] = *(const v4i_t *)(a.rk + kivi_ring_k(kvh, t, 32 * dt + 8 * kg, D));
        }
#pragma unroll
        for (int nt = 0; nt < NT; nt++) v[nt] = *(const v4i_t *)(a.rv + kivi_ring_v(kvh, tb, 16 * nt + r, D) + 8 * kg);
    }
};

// Run `run` of a KIVI code word (kivi_bit placement) -> 8 x binary16
// 1 + code/4, exact: one shift moves each code pair to bits 8 and 24, which
// go under 0x3C00 (1.0).  Operands of the form 1 + c/4 keep the MFMA sums'
// magnitudes near those of the codes; the callers scale the other operand
// by 4 and subtract its sum (a bias term): sum a (1 + c/4) * 4 - 4 sum a =
// sum a c.
// m: 0x03000300 held in a vector register (kivi_mask), so that each pair is
// one v_and_or_b32 (a VOP3 instruction reads at most one scalar / constant
// operand here).
__device__ __forceinline__ uint32_t kivi_mask() {
    uint32_t m = 0x03000300u;
    asm volatile("" : "+v"(m));
    return m;
}
__device__ __forceinline__ v8h_t kivi_unpack(uint32_t w, int run, uint32_t m) {
    uint32_t d[4];
#pragma unroll
    for (int k = 0; k < 4; k++) d[k] = ((run ? w << (8 - 2 * k) : w >> (2 * k)) & m) | 0x3C003C00u;
    v8h_t r;
    __builtin_memcpy(&r, d, 16);
    return r;
}

// LDS written by other lanes of this wave becomes readable: wait for this
// wave's LDS operations only (lgkmcnt 0; vector memory loads stay in flight)
// and keep the compiler from moving LDS accesses across.
__device__ __forceinline__ void lds_wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// One workgroup = (split s, kv head kvh, query z); waves take 32-token
// blocks of the split's chunk round-robin.
// The new token's binary16 K / V row (channels [8c, 8c+8)) from the f32 rows
// the fused QKV workgroups published (agent-scope loads); the cache slot
// itself was written by those workgroups.
struct NewRowH16 {
    v4i_t k, v;
    __device__ __forceinline__ void build(const AttnArgs &a, int kvh, int c) {
        const int D = (int)a.tok_stride;
        float kx[8], vx[8];
#pragma unroll
        for (int i = 0; i < 8; i += 2) {
            const float2 kk = ld_agent2(a.knew + kvh * D + 8 * c + i), vv = ld_agent2(a.vnew + kvh * D + 8 * c + i);
            kx[i] = kk.x;
            kx[i + 1] = kk.y;
            vx[i] = vv.x;
            vx[i + 1] = vv.y;
        }
        k = f32_to_h8(kx);
        v = f32_to_h8(vx);
    }
    __device__ __forceinline__ void store(const AttnArgs &, int, int, int) const {}
};

// One workgroup = (split bx, kv head by, query bz).  FUSED (fp16 cache, one
// query): the first K / V block is issued before the wait on fw, q is read
// with agent-scope loads after it, and the block holding slot pos takes the
// new token's K / V from the published rows.
template <typename KT, int D, int G, int NTH, bool FUSED>
__device__ __forceinline__ void attm_body(const AttnArgs &a0, int bx, int by, int bz, const FuseWait &fw) {
    static_assert(!FUSED || std::is_same<KT, __half>::value, "fused launch: fp16 cache");
    constexpr int DT = D / 32, NT = D / 16, NW = NTH / 64;
    constexpr int OPT = (G * D + NTH - 1) / NTH;
    static_assert(2 * G <= 16, "query heads (hi/lo rows) exceed the MFMA tile");
    constexpr bool KIVI = std::is_same<KT, KvKivi>::value;
    constexpr bool QV = KIVI || std::is_same<KT, KvQ8>::value;  // quantized V: scales folded into P
    __shared__ __align__(16) float sp[NW][G][kAttmBlock];  // p of the current block (per wave)
    __shared__ __align__(16) float vrat[QV ? NW : 1][DT][kAttmBlock];  // V scale / block maximum per (32-ch group, slot)
    // PV A operands of the quantized-V paths, per 32-channel group: rows (head, high / residual) x slots
    __shared__ __align__(16) _Float16 apb[QV ? NW : 1][DT][2 * G][kAttmBlock];
    __shared__ float vmax[NW][DT];             // Q8: their maximum per 32-channel block
    __shared__ float red[NW][G * D];         // per-wave O, then the workgroup output
    __shared__ float wm[NW][G], wl[NW][G];
    __shared__ float Mx[G], Lx[G];
    __shared__ int is_last;
    __shared__ int8_t nk[D], nv[D];              // Q8 decode step: the new token's codes
    __shared__ uint16_t nks[D / 32], nvs[D / 32];  // and scales
    __shared__ __align__(16) uint32_t kpar[KIVI ? NW : 1][KIVI ? D : 1];   // KIVI: K (scale, min) of the block's group
    __shared__ __align__(16) float vmn[KIVI ? NW : 1][KIVI ? DT : 1][KIVI ? kAttmBlock : 1];  // KIVI: V min per (32-ch group, slot)
    // KIVI scores A operand: rows (head, high / residual) x channels of q * K scale
    __shared__ __align__(16) _Float16 akb[KIVI ? NW : 1][KIVI ? 2 * G : 1][KIVI ? D : 8];
    __shared__ float kbias[KIVI ? NW : 1][G], vbias[KIVI ? NW : 1][G][DT];
    __shared__ uint16_t nkh[KIVI || FUSED ? D : 1], nvh[KIVI || FUSED ? D : 1];  // KIVI / fused decode step: the new token in binary16
    __shared__ __align__(16) float qs[KIVI ? G : 1][KIVI ? D : 1];  // KIVI: the query rows

    AttnArgs a = a0;
    const int zq = bz;
    const bool qpair = a.qpair != 0;
    const int z0 = qpair ? 2 * zq : zq;  // first query of this workgroup
    if (zq) {
        a.q += (size_t)z0 * a.qstride;
        if (a.out) a.out += (size_t)z0 * a.ostride;
        if (a.oq) {
            a.oq += (size_t)z0 * a.ostride;
            a.os += (size_t)z0 * (a.ostride / 32);
            a.osum += (size_t)z0 * (a.ostride / 32);
        }
        a.part += (size_t)zq * a.nkv * a.nsplit * G * (D + 2);
        a.counters += (size_t)zq * a.nkv;
    }
    const int kvh = by, s = bx, tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6, kg = lane >> 4, r = lane & 15;
    ATTN_TS(0);
    using Tile0 = typename std::conditional<KIVI, AttmKiviQ<D>, AttmTile<KT, D>>::type;
    Tile0 tile;
    // Q8: the wave's first block is loaded before the position is known,
    // assuming chmin-slot chunks (exact while T <= nsplit * chmin, reloaded
    // otherwise); the unconditional early load also keeps this kernel's
    // registers below the spill threshold (measured at 128k slots).  The query
    // loads precede the position load (a vector load, so waiting for it does
    // not hold up the kernel arguments).
    const int t0s = s * a.chmin;
    constexpr bool spec = std::is_same<KT, KvQ8>::value;
    if constexpr (spec) tile.load(a, kvh, min(t0s + wave * kAttmBlock, a.S - kAttmBlock), a.S - 1, lane);
    v4f_t qv[DT][2];
    auto load_q = [&]() {
        const int g = min(r >> 1, G - 1);
        // query pairs: rows g >= G/2 are the second query's heads
        constexpr int GH = G / 2 > 0 ? G / 2 : 1;
        const size_t qo = !qpair ? (size_t)(kvh * G + g) * D
                                 : (g >= GH ? (size_t)a.qstride : 0) + (size_t)(kvh * GH + g % GH) * D;
        if constexpr (FUSED) {
            // published in this launch: agent-scope loads
            const float *qf = a.q + qo + 8 * kg;
#pragma unroll
            for (int dt = 0; dt < DT; dt++)
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const float2 u = ld_agent2(qf + 32 * dt + 4 * h), w = ld_agent2(qf + 32 * dt + 4 * h + 2);
                    qv[dt][h] = v4f_t{u.x, u.y, w.x, w.y};
                }
        } else {
            const v4f_t *qp = (const v4f_t *)(a.q + qo + 8 * kg);
#pragma unroll
            for (int dt = 0; dt < DT; dt++) {
                qv[dt][0] = qp[8 * dt];
                qv[dt][1] = qp[8 * dt + 1];
            }
        }
    };
    if constexpr (!FUSED) load_q();
    const int pos = __hip_atomic_load(a.posp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + (qpair ? z0 + 1 : zq),
              T = pos + 1;
    // query pairs: the first query's heads (rows < G/2) stop before slot pos
    const int lastA0 = (qpair && 2 * kg < G / 2) ? pos : INT_MAX;
    const int lastA1 = (qpair && 2 * kg + 1 < G / 2) ? pos : INT_MAX;
    // element i of this kv head's G*D outputs -> offset from a.out / a.oq
    auto oix = [&](int i) -> size_t {
        if (!qpair) return (size_t)kvh * G * D + i;
        constexpr int HD = (G / 2) * D;
        return (i >= HD ? (size_t)a.ostride + (i - HD) : (size_t)i) + (size_t)kvh * HD;
    };
    // up to a.single tokens: one split (no cross-workgroup merge);
    // beyond: chunks of at least chmin slots over the nsplit workgroups
    int CH = T <= a.single ? T : max(a.chmin, (T + a.nsplit - 1) / a.nsplit);
    CH = (CH + kAttmBlock * NW - 1) / (kAttmBlock * NW) * (kAttmBlock * NW);
    const int t0 = s * CH;
    if (t0 >= T) return;
    const int t1 = min(T, t0 + CH);
    const int nact = (T + CH - 1) / CH;

    // the new token (Q8 decode step): quantize, store, and use its codes
    typename std::conditional<FUSED, NewRowH16, NewRow<KT>>::type nrow;
    const bool has_new = a.knew != nullptr;

    const int nblk = (t1 - t0 + kAttmBlock - 1) / kAttmBlock;
    // KIVI: blocks [0, nqb) of the chunk come from the 2-bit prefix (qlen
    // and t0 are multiples of 32), the rest from the fp16 ring
    const int qlen = kivi_qlen(T);
    const int nqb = KIVI ? min(nblk, max(0, (qlen - t0) / kAttmBlock)) : 0;
    if constexpr (KIVI) {
        if (wave < nqb) tile.load(a, kvh, t0 + wave * kAttmBlock, t1 - 1, lane);
    } else {
        if ((!spec || t0 != t0s) && wave < nblk) tile.load(a, kvh, t0 + wave * kAttmBlock, t1 - 1, lane);
    }
    if constexpr (FUSED) {
        // the first block is in flight; wait for the QKV workgroups of this
        // kv head, then read q
        if (tid == 0) {
            int n = 0;
            while (__hip_atomic_load(fw.count + kvh, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < fw.target) {
                if (++n > kFuseSpinLimit) {
                    __hip_atomic_store(fw.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
        }
        __syncthreads();
        load_q();
    }

    // A operand of S: row m = 2g + (hi / lo) of head g (rows >= 2G zero)
    v8h_t aq[DT];
    {
        const int m = r, g = min(m >> 1, G - 1);
#pragma unroll
        for (int dt = 0; dt < DT; dt++) {
            const v4f_t q0 = qv[dt][0], q1 = qv[dt][1];
            float x[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
            if ((m >> 1) >= G) {
#pragma unroll
                for (int i = 0; i < 8; i++) x[i] = 0.0f;
            }
            if constexpr (KIVI) {
                // 4 x the f32 query in LDS (scaled per 2-bit channel in each quantized block)
                if (!(m & 1) && (m >> 1) < G) {
#pragma unroll
                    for (int i = 0; i < 8; i++) qs[g][32 * dt + 8 * kg + i] = 4.0f * x[i];  // exact
                }
            }
            v8h_t hi, lo;
            split8(x, hi, lo);
            aq[dt] = (m & 1) ? lo : hi;
        }
    }
    const float scale = 1.0f / sqrtf((float)D);
    if constexpr (KIVI) __syncthreads();  // qs
    const uint32_t kmask = KIVI ? kivi_mask() : 0u;
    ATTN_TS(1);

    // wave-private online softmax state; lane group kg holds heads 2kg, 2kg+1
    float m_run[2] = {-INFINITY, -INFINITY}, l_run[2] = {0.0f, 0.0f};
    v4f32_t oacc[NT];
#pragma unroll
    for (int nt = 0; nt < NT; nt++) oacc[nt] = v4f32_t{0.f, 0.f, 0.f, 0.f};

    // one 32-slot block (slots tb .. tb+31) with its tile in registers
    auto process = [&](auto &tile, int bi) {
        using TT = typename std::remove_reference<decltype(tile)>::type;
        constexpr bool KQ = std::is_same<TT, AttmKiviQ<D>>::value;                 // 2-bit block
        constexpr bool H16 = std::is_same<KT, __half>::value || (KIVI && !KQ);    // fp16 operands
        const int tb = t0 + bi * kAttmBlock;
        if constexpr (std::is_same<KT, KvQ8>::value) {
            // Q8 decode step: the block holding slot pos quantizes the new
            // token, stores it, and patches its K row / V column in registers
            // a wave-uniform branch (the position is a vector load: without
            // readfirstlane the compiler lowers this as a divergent region and
            // its waits land on every block)
            if (__builtin_amdgcn_readfirstlane((int)(has_new && pos >= tb && pos < tb + kAttmBlock))) {
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
                lds_wave_sync();  // the codes / halves written to LDS above (the cache stores stay in flight)
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
        v8h_t ak[KQ ? DT : 1];
        if constexpr (KIVI || FUSED) if constexpr (!KQ) {
            // a wave-uniform branch (the position is a vector load: without
            // readfirstlane the compiler lowers this as a divergent region and
            // its waits land on every block)
            if (__builtin_amdgcn_readfirstlane((int)(has_new && pos >= tb && pos < tb + kAttmBlock))) {
                // decode step: the new token goes into the ring (binary16); the
                // block holding it patches its K row / V column in registers
                const int c = lane % (D / 8);
                nrow.build(a, kvh, c);
                if (lane < D / 8) {
                    nrow.store(a, kvh, pos, c);
                    *(v4i_t *)(nkh + 8 * c) = nrow.k;
                    *(v4i_t *)(nvh + 8 * c) = nrow.v;
                }
                lds_wave_sync();  // the codes / halves written to LDS above (the cache stores stay in flight)
                const int pi = pos - tb, th = pi >> 4;
                if ((pi & 15) == r) {
#pragma unroll
                    for (int h = 0; h < 2; h++)
                        if (h == th) {
#pragma unroll
                            for (int dt = 0; dt < DT; dt++) tile.k[h][dt] = *(const v4i_t *)(nkh + 32 * dt + 8 * kg);
                        }
                }
                if ((pi >> 3) == kg) {
                    const int e = pi & 7, sh = 16 * (e & 1);
#pragma unroll
                    for (int nt = 0; nt < NT; nt++) {
                        const uint32_t hv = nvh[16 * nt + r];
#pragma unroll
                        for (int j = 0; j < 4; j++)
                            if (j == (e >> 1)) {
                                const uint32_t w = (uint32_t)tile.v[nt][j];
                                tile.v[nt][j] = (int)((w & ~(0xFFFFu << sh)) | (hv << sh));
                            }
                    }
                }
            }
        }
        if constexpr (KQ) {
            {
                // stage the group's K (scale, min) and the slots' V (scale, min)
#pragma unroll
                for (int i = 0; i < TT::KW; i++) kpar[wave][lane + 64 * i] = tile.kp[i];
                if (lane < kAttmBlock) {
                    const bool okt = tb + lane < t1;
#pragma unroll
                    for (int b = 0; b < DT; b++) {
                        const uint32_t sm = okt ? tile.vp[b] : 0u;
                        const float sv = h2f((uint16_t)(sm & 0xFFFF));
                        vmn[wave][b][lane] = h2f((uint16_t)(sm >> 16));
                        float mx = row_max<16>(sv);
                        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
                        vrat[wave][b][lane] = mx > 0.0f ? 4.0f * (sv * __builtin_amdgcn_rcpf(mx)) : 0.0f;  // 4 x ratio
                        if (lane == 0) vmax[wave][b] = mx;
                    }
                }
                lds_wave_sync();
                // scores A operand: each lane forms 8 distinct products
                // 4 q[g][c] scale[c] (channels 8j .. 8j+7 of head g), split
                // high / residual into rows 2g / 2g+1, and its part of the
                // head's bias sum_c q[g][c] min[c] - sum_c (high + residual)
                // (the B operand is 1 + code/4)
                constexpr int CJ = D / 8, KU = G * CJ;
#pragma unroll
                for (int u0 = 0; u0 < KU; u0 += 64) {
                    const int u = min(u0 + lane, KU - 1), g = u / CJ, j = u % CJ;
                    const v4f_t q0 = *(const v4f_t *)&qs[g][8 * j], q1 = *(const v4f_t *)&qs[g][8 * j + 4];
                    const v4i_t k0 = *(const v4i_t *)&kpar[wave][8 * j], k1 = *(const v4i_t *)&kpar[wave][8 * j + 4];
                    const float qv[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
                    const uint32_t sm[8] = {(uint32_t)k0.x, (uint32_t)k0.y, (uint32_t)k0.z, (uint32_t)k0.w,
                                            (uint32_t)k1.x, (uint32_t)k1.y, (uint32_t)k1.z, (uint32_t)k1.w};
                    float x[8], kb = 0.0f, hs = 0.0f;  // qs holds 4 q
#pragma unroll
                    for (int i = 0; i < 8; i++) {
                        x[i] = qv[i] * h2f((uint16_t)(sm[i] & 0xFFFF));
                        kb = __builtin_fmaf(qv[i], h2f((uint16_t)(sm[i] >> 16)), kb);
                    }
                    v8h_t hi, lo;
                    split8(x, hi, lo);
#pragma unroll
                    for (int i = 0; i < 8; i++) hs += (float)hi[i] + (float)lo[i];  // exact pair sums
                    kb = __builtin_fmaf(kb, 0.25f, -hs);
                    kb = row_sum<(CJ < 16 ? CJ : 16)>(kb);  // the CJ lanes of head g (aligned)
                    if (u0 + lane < KU) {
                        *(v8h_t *)&akb[wave][2 * g][8 * j] = hi;
                        *(v8h_t *)&akb[wave][2 * g + 1][8 * j] = lo;
                        if (j == 0) kbias[wave][g] = kb;
                    }
                }
                lds_wave_sync();
#pragma unroll
                for (int dt = 0; dt < DT; dt++)
                    ak[dt] = r < 2 * G ? *(const v8h_t *)&akb[wave][r][32 * dt + 8 * kg] : v8h_t{};
            }
        }
        // ---- scores: two 16-slot halves -------------------------------------
        float sc[2][2];  // [half][head parity] for slot tb + 16h + r
#pragma unroll
        for (int h = 0; h < 2; h++) {
            v4f32_t acc = v4f32_t{0.f, 0.f, 0.f, 0.f};
            float kbh[2] = {0.0f, 0.0f};
            if constexpr (H16) {
#pragma unroll
                for (int dt = 0; dt < DT; dt++) acc = mfma16(aq[dt], as_h8(tile.k[h][dt]), acc);
            } else if constexpr (KQ) {
                // codes of this lane's slot: word dt/2, run dt%2 per 32-channel tile
#pragma unroll
                for (int dt = 0; dt < DT; dt++)
                    acc = mfma16(ak[dt], kivi_unpack(tile.k[h][dt >> 1], dt & 1, kmask), acc);
                kbh[0] = 2 * kg < G ? kbias[wave][2 * kg] : 0.0f;
                kbh[1] = 2 * kg + 1 < G ? kbias[wave][2 * kg + 1] : 0.0f;
            } else {
#pragma unroll
                for (int dt = 0; dt < DT; dt++) {
                    const v4f32_t part = mfma16(aq[dt], i8x8_to_h8(tile.k[h][dt]), v4f32_t{0.f, 0.f, 0.f, 0.f});
                    const uint32_t w = tile.ksc[h][dt >> 1];
                    const float ks = h2f((uint16_t)((dt & 1) ? (w >> 16) : (w & 0xFFFF)));
#pragma unroll
                    for (int i = 0; i < 4; i++) acc[i] = __builtin_fmaf(part[i], ks, acc[i]);
                }
            }
            const int t = tb + 16 * h + r;
            const bool ok = t < t1;
            sc[h][0] = ok && t != lastA0 ? (acc[0] + acc[1] + kbh[0]) * scale : -INFINITY;
            sc[h][1] = ok && t != lastA1 ? (acc[2] + acc[3] + kbh[1]) * scale : -INFINITY;
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
#pragma unroll
                for (int b = 0; b < DT; b++) {
                    uint16_t sv = (uint16_t)(tile.vsc[b >> 1] >> (16 * (b & 1)));
                    if (has_new && tb + lane == pos) sv = nvs[b];
                    const float v = (tb + lane < t1) ? h2f(sv) : 0.0f;
                    float mx = row_max<16>(v);
                    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
                    vrat[wave][b][lane] = mx > 0.0f ? v * __builtin_amdgcn_rcpf(mx) : 0.0f;
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
        if constexpr (QV && !H16) {
            // quantized V: each lane forms 8 distinct products p[g][t] *
            // ratio[b][t] (slots 8kq .. 8kq+7, head g, channel group b),
            // split high / residual into rows 2g / 2g+1 of group b's A
            // operand; KIVI: its part of the bias sum_t p[g][t] min[b][t]
            constexpr int PU = G * DT * 4;
#pragma unroll
            for (int u0 = 0; u0 < PU; u0 += 64) {
                const int u = min(u0 + lane, PU - 1), kq = u & 3, b = (u >> 2) % DT, g = u / (4 * DT);
                const v4f_t p0 = *(const v4f_t *)&sp[wave][g][8 * kq], p1 = *(const v4f_t *)&sp[wave][g][8 * kq + 4];
                const v4f_t r0 = *(const v4f_t *)&vrat[wave][b][8 * kq], r1 = *(const v4f_t *)&vrat[wave][b][8 * kq + 4];
                const float pv[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
                const float rv[8] = {r0.x, r0.y, r0.z, r0.w, r1.x, r1.y, r1.z, r1.w};
                // KIVI: the B operand is 1 + code/4, so the ratios carry a
                // factor 4 and the bias also takes vref * sum_t (high + residual)
                float x[8];
#pragma unroll
                for (int i = 0; i < 8; i++) x[i] = pv[i] * rv[i];
                v8h_t hi, lo;
                split8(x, hi, lo);
                float vb = 0.0f;
                if constexpr (KIVI) {
                    const v4f_t n0 = *(const v4f_t *)&vmn[wave][b][8 * kq], n1 = *(const v4f_t *)&vmn[wave][b][8 * kq + 4];
                    const float nv8[8] = {n0.x, n0.y, n0.z, n0.w, n1.x, n1.y, n1.z, n1.w};
                    float hs = 0.0f;
#pragma unroll
                    for (int i = 0; i < 8; i++) {
                        vb = __builtin_fmaf(pv[i], nv8[i], vb);
                        hs += (float)hi[i] + (float)lo[i];  // exact pair sum
                    }
                    vb = __builtin_fmaf(-vmax[wave][b], hs, vb);
                    vb = row_sum<4>(vb);  // the 4 slot chunks of (g, b)
                }
                if (u0 + lane < PU) {
                    *(v8h_t *)&apb[wave][b][2 * g][8 * kq] = hi;
                    *(v8h_t *)&apb[wave][b][2 * g + 1][8 * kq] = lo;
                    if constexpr (KIVI)
                        if (kq == 0) vbias[wave][g][b] = vb;
                }
            }
            lds_wave_sync();
        }
        {
            const int m = r, g = m >> 1;
            if constexpr (H16) {
                float p[8];
#pragma unroll
                for (int i = 0; i < 8; i++) p[i] = g < G ? sp[wave][g][8 * kg + i] : 0.0f;
                v8h_t hi, lo;
                split8(p, hi, lo);
                const v8h_t ap = (m & 1) ? lo : hi;
#pragma unroll
                for (int nt = 0; nt < NT; nt++) oacc[nt] = mfma16(ap, as_h8(tile.v[nt]), oacc[nt]);
            } else if constexpr (KQ) {
                {
                    // codes * scale via MFMA (scales folded into P as for Q8),
                    // plus the bias sum_t p_t min_t per (head, 32-channel group)
                    const uint32_t *vw = tile.v;
#pragma unroll
                    for (int b = 0; b < DT; b++) {
                        const float vref = vmax[wave][b];
                        const v8h_t ap = m < 2 * G ? *(const v8h_t *)&apb[wave][b][m][8 * kg] : v8h_t{};
#pragma unroll
                        for (int u = 0; u < 2; u++) {
                            const int nt = 2 * b + u;
                            const v4f32_t part = mfma16(ap, kivi_unpack(vw[nt >> 1], nt & 1, kmask),
                                                        v4f32_t{0.f, 0.f, 0.f, 0.f});
#pragma unroll
                            for (int i = 0; i < 4; i++) oacc[nt][i] = __builtin_fmaf(part[i], vref, oacc[nt][i]);
                        }
                    }
                    // rows 4kg + i of oacc: head 2kg + i/2, (hi, lo); the bias goes on the hi row
#pragma unroll
                    for (int nt = 0; nt < NT; nt++) {
                        if (2 * kg < G) oacc[nt][0] += vbias[wave][2 * kg][nt >> 1];
                        if (2 * kg + 1 < G) oacc[nt][2] += vbias[wave][2 * kg + 1][nt >> 1];
                    }
                }
            } else {
                // V scales folded into P relative to the block's largest
                // scale (keeps the f16 residual out of the subnormal range),
                // which multiplies the block's MFMA result
#pragma unroll
                for (int b = 0; b < DT; b++) {
                    const float vref = vmax[wave][b];
                    const v8h_t ap = m < 2 * G ? *(const v8h_t *)&apb[wave][b][m][8 * kg] : v8h_t{};
#pragma unroll
                    for (int u = 0; u < 2; u++) {
                        const v4f32_t part =
                            mfma16(ap, i8x8_to_h8(tile.v[2 * b + u]), v4f32_t{0.f, 0.f, 0.f, 0.f});
#pragma unroll
                        for (int i = 0; i < 4; i++) oacc[2 * b + u][i] = __builtin_fmaf(part[i], vref, oacc[2 * b + u][i]);
                    }
                }
            }
        }
        __builtin_amdgcn_wave_barrier();
    };
    if constexpr (!KIVI) {
        // ping-pong: the wave's next block is in flight while this one computes
        // (Q8 at D = 128: 248 VGPRs with both tiles, no spills; 128k slots
        // 74 -> 71 us against reloading each half as it is consumed)
        AttmTile<KT, D> tile2;
        const int nbw = wave < nblk ? (nblk - wave + NW - 1) / NW : 0;  // blocks wave, wave + NW, ...
        pingpong(
            nbw, tile, tile2,
            [&](AttmTile<KT, D> &T, int j) { T.load(a, kvh, t0 + (wave + j * NW) * kAttmBlock, t1 - 1, lane); },
            [&](AttmTile<KT, D> &T, int j) { process(T, wave + j * NW); });
    } else if constexpr (KIVI) {
        // 2-bit blocks ping-pong (small tiles), then the ring blocks
        Tile0 tile2;
        const int nbw = wave < nqb ? (nqb - wave + NW - 1) / NW : 0;
        pingpong(
            nbw, tile, tile2, [&](Tile0 &T, int j) { T.load(a, kvh, t0 + (wave + j * NW) * kAttmBlock, t1 - 1, lane); },
            [&](Tile0 &T, int j) { process(T, wave + j * NW); });
        AttmTile<KvKivi, D> rt;
        const int bi0 = nqb > wave ? wave + (nqb - wave + NW - 1) / NW * NW : wave;
        for (int bi = bi0; bi < nblk; bi += NW) {
            rt.load(a, kvh, t0 + bi * kAttmBlock, t1 - 1, lane);
            process(rt, bi);
        }
    }
    if constexpr (KIVI) {
        // decode step that ages group qlen/32 out of the fp16 residual: split
        // 0 moves it from the ring into the 2-bit store (its tokens are read
        // from the ring by every split of this step, from the store after it)
        if (has_new && s == 0 && kivi_qlen(T + 1) > qlen) {
            const __half *rk = a.rk, *rv = a.rv;
            auto src = [&](int t, int ch, bool is_v) -> float {
                return __half2float(is_v ? rv[kivi_ring_v(kvh, t, ch, D)] : rk[kivi_ring_k(kvh, t, ch, D)]);
            };
            kivi_quantize_group(a, D, kvh, qlen / kKiviGroup, src, &red[0][0]);
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
        const int i = tid + k * NTH;
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
        ATTN_TS(4);
        // the only workgroup of this kv head: clear its fused-launch count
        if constexpr (FUSED)
            if (tid == 0) __hip_atomic_store(fw.count + kvh, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();  // red is overwritten below
#pragma unroll
        for (int k = 0; k < OPT; k++) {
            const int i = tid + k * NTH;
            if (i < G * D) {
                const float v = res[k] * (1.0f / Lx[i / D]);
                mo[i] = v;
                if (a.out) a.out[oix(i)] = v;
            }
        }
    } else {
        // publish (unnormalised o, m, l) with agent-scope stores, then count in
        constexpr int P = G * (D + 2);
        float *mypart = a.part + ((size_t)kvh * a.nsplit + s) * P;
#pragma unroll
        for (int k = 0; k < OPT; k++) {
            const int i = tid + k * NTH;
            if (i < G * D) st_agent(mypart + i, res[k]);
        }
        if (tid < G) {
            st_agent(mypart + G * D + 2 * tid, Mx[tid]);
            st_agent(mypart + G * D + 2 * tid + 1, Lx[tid]);
        }
        ATTN_TS(4);
        ATTN_TS(5);
        if (!split_arrive_last<false>(&a.counters[kvh], nact, &is_last)) return;
        // last workgroup of the kv head: each thread merges its OPT outputs
        // (one head each) over the nact partials, MB splits per round trip
        // (all loads of a batch independent), online rescale between batches:
        // out = sum_j o_j e^(m_j - M) / sum_j l_j e^(m_j - M)
        ATTN_TSL(6);
        // batch size from the live split count (8 / 16 / 24 / 32): every load
        // of a batch is a live partial, and up to 24-32 splits take one trip
        const float *pb = a.part + (size_t)kvh * a.nsplit * P;
        float M[OPT], L[OPT], O[OPT];
#pragma unroll
        for (int k = 0; k < OPT; k++) {
            M[k] = -INFINITY;
            L[k] = 0.0f;
            O[k] = 0.0f;
        }
        auto merge = [&](auto mbc) {
            constexpr int MB = decltype(mbc)::value;
            for (int j0 = 0; j0 < nact; j0 += MB) {
#pragma unroll
                for (int k = 0; k < OPT; k++) {
                    const int i = min(tid + k * NTH, G * D - 1), g = i / D;
                    float mv[MB], lv[MB], ov[MB];
#pragma unroll
                    for (int k2 = 0; k2 < MB; k2++) {
                        const float *pj = pb + (size_t)min(j0 + k2, nact - 1) * P;
                        if constexpr (D == 64) {
                            // (m, l) in one load: measured faster at D = 64
                            // (Llama-3.2-1B), slower at D = 128 (Llama-3-8B)
                            const float2 ml = ld_agent2(pj + G * D + 2 * g);
                            mv[k2] = ml.x;
                            lv[k2] = ml.y;
                        } else {
                            mv[k2] = ld_agent(pj + G * D + 2 * g);
                            lv[k2] = ld_agent(pj + G * D + 2 * g + 1);
                        }
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
        };
        // one output per thread (one query head per wave): lane j of every
        // wave loads split j's (m, l) and forms its weight e^(m_j - M) once;
        // each lane folds its head's o_j * w_j in split order, w_j read from
        // lane j.  Two (m, l) loads per wave instead of two per split.
        auto wmerge = [&](auto mbc) {
            constexpr int MB = decltype(mbc)::value;
            const int i = min(tid, G * D - 1), g = i / D;
            float mj = -INFINITY, lj = 0.0f;
            if (lane < nact) {
                const float *pm = pb + (size_t)lane * P + G * D + 2 * g;
                mj = ld_agent(pm);
                lj = ld_agent(pm + 1);
            }
            float ov[MB];
#pragma unroll
            for (int k2 = 0; k2 < MB; k2++) ov[k2] = ld_agent(pb + (size_t)min(k2, nact - 1) * P + i);
            const float Mw = wave_max(mj);
            const float wj = (mj == -INFINITY) ? 0.0f : __expf(mj - Mw);
            L[0] = wave_sum(lj * wj);
            float o = 0.0f;
#pragma unroll
            for (int k2 = 0; k2 < MB; k2++)
                if (k2 < nact) o = fmaf(ov[k2], __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wj), k2)), o);
            O[0] = o;
        };
        if (OPT == 1 && nact <= 64) {
            if (nact <= 8) wmerge(std::integral_constant<int, 8>{});
            else if (nact <= 16) wmerge(std::integral_constant<int, 16>{});
            else if (nact <= 24) wmerge(std::integral_constant<int, 24>{});
            else if (nact <= 32) wmerge(std::integral_constant<int, 32>{});
            else wmerge(std::integral_constant<int, 64>{});
        } else if (nact <= 8) merge(std::integral_constant<int, 8>{});
        else if (nact <= 16) merge(std::integral_constant<int, 16>{});
        else if (OPT > 1 || nact <= 24) merge(std::integral_constant<int, OPT == 1 ? 24 : 16>{});
        else merge(std::integral_constant<int, 32>{});
        ATTN_TSL(7);
#pragma unroll
        for (int k = 0; k < OPT; k++) O[k] *= 1.0f / L[k];
        if constexpr (OPT == 1) {
            // one output per thread, a 32-block in 32 consecutive lanes: the
            // Q8_0 copy straight from registers (no LDS round trip)
            if (tid == 0) {
                __hip_atomic_store(&a.counters[kvh], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if constexpr (FUSED) __hip_atomic_store(fw.count + kvh, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            if (tid < G * D) {
                if (a.out) a.out[oix(tid)] = O[0];
                if (a.oq) {
                    const size_t e0 = oix(tid & ~31);
                    quant_block32_lanes(O[0], a.oq + e0, a.os + e0 / 32, a.osum + e0 / 32);
                }
            }
            ATTN_TSL(8);
            ATTN_TSL(9);
            return;
        }
        __syncthreads();  // red (mo) is rewritten below
#pragma unroll
        for (int k = 0; k < OPT; k++) {
            const int i = tid + k * NTH;
            if (i < G * D) {
                const float v = O[k];
                mo[i] = v;
                if (a.out) a.out[oix(i)] = v;
            }
        }
        if (tid == 0) {
            __hip_atomic_store(&a.counters[kvh], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if constexpr (FUSED) __hip_atomic_store(fw.count + kvh, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        ATTN_TSL(8);
    }
    __syncthreads();
    if (nact == 1) ATTN_TS(6);
    if (a.oq) {
        // Q8_0 copy of this kv head's G*D outputs (quantize_input_q8_0_into), 32 lanes per block
        const int nb = G * D / 32;
        for (int b = tid >> 5; b < nb; b += NTH / 32) {
            const size_t e0 = oix(b * 32);
            quant_block32_lanes(mo[b * 32 + (tid & 31)], a.oq + e0, a.os + e0 / 32, a.osum + e0 / 32);
        }
    }
    if (nact > 1) ATTN_TSL(9);
    else ATTN_TS(7);
}

template <typename KT, int D, int G, int NTH = kAttmThreads>
__global__ __launch_bounds__(NTH) void k_attm(AttnArgs a0) {
    attm_body<KT, D, G, NTH, false>(a0, (int)blockIdx.x, (int)blockIdx.y, (int)blockIdx.z, FuseWait{});
}

}  // namespace fl
