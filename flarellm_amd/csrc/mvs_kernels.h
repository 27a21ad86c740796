// Streaming quantized matvecs (gfx950).
//
// Every weight row is read as contiguous 16-byte pieces: lane l of a wave
// loads bytes [16l, 16l+16) of a 1 KiB step of the row, so one load
// instruction covers 1 KiB of one row.  Per-block integer dots that span two
// lanes (a 32-value block = 2 pieces) are completed with a DPP lane-pair add,
// which is exact, so every per-block term is formed from the same integers
// as the reference.
//
// Weight planes on the device (uploaded once, see flare_hip.hip):
//   Q8_0  q = int8 quants [rows][K]        s = f16 block scales [rows][K/32]
//   Q4_K  q = qs nibbles [rows][nsb][128]  h = 16-B headers (d, dmin, scales[12]) [rows][nsb]
//   Q6_K  q = ql [rows][nsb][128]          h = qh [rows][nsb][64]
//         h2 = int8 scales [rows][nsb][16] s = f16 d [rows][nsb]
//   F32   q = floats [rows][K]
//
// Kernels:
//   k_mvs      one wave per row group of R rows; the persistent waves walk
//              (row group, round of SU steps) units with the next unit's
//              pieces in flight (ping-pong tiles).  Epilogues: store, residual
//              add, fused QKV (RoPE + KV store), first-max argmax.
//   k_mvs_gu   fused gate/up: a workgroup owns 32-hidden-unit blocks; SiLU*up
//              and the Q8_0 quantization of the block are its epilogue.
#pragma once

#include "mv_kernels.h"

namespace fl {

// The four int8 of a word as exact floats: bias to unsigned (xor 0x80),
// convert each byte in place (v_cvt_f32_ubyte0..3), subtract 128.
__device__ __forceinline__ void i8x4_to_f32(int w, float *q) {
    const uint32_t u = (uint32_t)w ^ 0x80808080u;
    q[0] = (float)(u & 0xFFu) - 128.0f;
    q[1] = (float)((u >> 8) & 0xFFu) - 128.0f;
    q[2] = (float)((u >> 16) & 0xFFu) - 128.0f;
    q[3] = (float)(u >> 24) - 128.0f;
}

#ifndef FLARE_NO_STAGE_BARRIER
#define FLARE_STAGE_BARRIER() __builtin_amdgcn_sched_barrier(0)
#else
#define FLARE_STAGE_BARRIER() \
    do {                      \
    } while (0)
#endif

// lanes l and l^1 exchange a value (quad_perm [1,0,3,2])
__device__ __forceinline__ int xpair(int v) { return __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, true); }

// bytes of one row in the streamed plane
__host__ __device__ inline int mvs_span(int fmt, int K) {
    return fmt == F_Q8_0 ? K : (fmt == F_F32 ? 4 * K : K / 2);
}
__host__ __device__ inline int mvs_steps(int fmt, int K) { return (mvs_span(fmt, K) + 1023) >> 10; }

// ---------------------------------------------------------------------------
// pieces: the 16 B (plus side data) of one lane for one (row, step)
// ---------------------------------------------------------------------------
template <int FMT>
struct Pc;

template <>
struct Pc<F_Q8_0> {
    v4i_t q;
    uint32_t sc;
    __device__ __forceinline__ void load(const WDesc &W, int row, int step, int lane) {
        const int K = W.cols;
        const int off = min(step * 1024 + 16 * lane, K - 16);
        q = ld_stream(W.q + (size_t)row * K + off);
        sc = W.s[(size_t)row * (K >> 5) + (off >> 5)];
    }
};

template <>
struct Pc<F_Q4K> {
    v4i_t q, h;
    __device__ __forceinline__ void load(const WDesc &W, int row, int step, int lane) {
        const int nsb = W.cols >> 8, span = nsb * 128;
        const int off = min(step * 1024 + 16 * lane, span - 16);
        q = ld_stream(W.q + (size_t)row * span + off);
        h = *(const v4i_t *)(W.h + ((size_t)row * nsb + (off >> 7)) * 16);  // 8 lanes share it
    }
};

template <>
struct Pc<F_Q6K> {
    v4i_t ql, qh;
    // scales of the low- and high-nibble weights, each kept as loaded: a
    // combining shift right after the loads would make the wave wait for
    // them (and, completing in order, for every load before them) when the
    // tile is issued instead of when it is consumed
    uint32_t sc0, sc1;
    uint32_t d;
    __device__ __forceinline__ void load(const WDesc &W, int row, int step, int lane) {
        const int nsb = W.cols >> 8, span = nsb * 128;
        const int off = min(step * 1024 + 16 * lane, span - 16);
        const int sb = off >> 7, o = off & 127, hf = o >> 6, q = (o >> 4) & 3;
        const size_t rs = (size_t)row * nsb + sb;
        ql = ld_stream(W.q + (size_t)row * span + off);
        qh = *(const v4i_t *)(W.h + rs * 64 + hf * 32 + (q & 1) * 16);  // 2 lanes share it
        const int si = hf * 8 + (q & 1) + 2 * (q >> 1);
        const uint8_t *scp = W.h2 + rs * 16;
        sc0 = scp[si];
        sc1 = scp[si + 4];
        d = W.s[rs];
    }
};

template <>
struct Pc<F_F32> {
    v4f_t w;
    __device__ __forceinline__ void load(const WDesc &W, int row, int step, int lane) {
        const int K = W.cols;
        const int off = min(step * 1024 + 16 * lane, 4 * K - 16);
        w = ld_stream_f(W.q + (size_t)row * K * 4 + off);
    }
};

// ---- Q8 input (int8 activations in LDS) -----------------------------------
// matvec_q8_0_preq_into per-block term (model.rs:8082-8099):
// (f16(w_scale) * x_scale) * (int dot as f32), counted once (even lane).
__device__ __forceinline__ float pc_dot_q8(const Pc<F_Q8_0> &P, const WDesc &W, const int8_t *lq, const float *ls,
                                           const int *, int step, int lane) {
    const int K = W.cols, off0 = step * 1024 + 16 * lane;
    const int off = min(off0, K - 16);
    const v4i_t x = *(const v4i_t *)(lq + off);
    int d = dot16(P.q, x, 0);
    d += xpair(d);
    const float t = mul_h16lo(P.sc, ls[off >> 5]) * (float)d;
    return (off0 < K && !(lane & 1)) ? t : 0.0f;
}

// Q4_K (scale, min) of the sub-block a lane owns after the pair add: c (even
// lane, low nibbles) or c+4 (odd lane, high nibbles), with c = (lane / 2) % 4
// (unpack_q4k_scales model.rs:8709-8719, flare packing).  Low half: sc =
// y.byte(c) & 63, mn = z.byte(c) & 63; high half: sc = y.byte(c) >> 6 |
// (w.byte(c) & 15) << 2, mn = z.byte(c) >> 6 | (w.byte(c) >> 4) << 2.  Both
// cases are bit-field extracts at lane-constant offsets and widths (a zero
// width extracts 0), so a lane spends 6 integer ops per (row, step) on them.
struct Q4Lane {
    uint32_t oa, wa, oc, wc;
    __device__ __forceinline__ explicit Q4Lane(int lane) {
        const uint32_t c = (lane >> 1) & 3, h = lane & 1;
        oa = 8 * c + 6 * h;
        wa = h ? 2 : 6;
        oc = 8 * c;
        wc = h ? 4 : 0;
    }
    __device__ __forceinline__ void scmn(const v4i_t &hd, uint32_t &sc, uint32_t &mn) const {
        const uint32_t y = (uint32_t)hd.y, z = (uint32_t)hd.z, w = (uint32_t)hd.w;
        sc = __builtin_amdgcn_ubfe(y, oa, wa) | (__builtin_amdgcn_ubfe(w, oc, wc) << 2);
        mn = __builtin_amdgcn_ubfe(z, oa, wa) | (__builtin_amdgcn_ubfe(w, oc + 4, wc) << 2);
    }
};

// dot_q4k_q8_0_scalar per-sub-block term (model.rs:8969-9025) of one lane:
// s_x * (d*sc*dot - dmin*mn*sum(q_x)).  The 16 qs bytes of a lane hold half of
// sub-block c (low nibbles, activation run xl) and half of sub-block c+4 (high
// nibbles, run xh); the pair add gives the even lane sub-block c's full dot
// and the odd lane c+4's (each lane keeps its own half-dot and passes the
// other one to its partner).  xs is the lane's block scale (0 for a lane past
// the row's end), xsum its block code sum.
__device__ __forceinline__ float q4_term(const Pc<F_Q4K> &P, const v4i_t &xl, const v4i_t &xh, float xs, float xsum,
                                         const Q4Lane &L) {
    const v4i_t lo = P.q & 0x0F0F0F0F;
    // high nibbles: one 64-bit shift per two words
    const uint64_t w01 = ((uint64_t)(uint32_t)P.q.y << 32) | (uint32_t)P.q.x;
    const uint64_t w23 = ((uint64_t)(uint32_t)P.q.w << 32) | (uint32_t)P.q.z;
    const uint64_t h01 = (w01 >> 4) & 0x0F0F0F0F0F0F0F0Full, h23 = (w23 >> 4) & 0x0F0F0F0F0F0F0F0Full;
    const v4i_t hi = {(int)(uint32_t)h01, (int)(uint32_t)(h01 >> 32), (int)(uint32_t)h23, (int)(uint32_t)(h23 >> 32)};
    const int dl = dot16(lo, xl, 0), dh = dot16(hi, xh, 0);
    const bool odd = L.wc != 0;
    const int dot = (odd ? dh : dl) + xpair(odd ? dl : dh);
    const uint32_t h0 = (uint32_t)P.h.x;
    uint32_t sc, mn;
    L.scmn(P.h, sc, mn);
    const float d_sc = mul_h16lo(h0, (float)sc), dmin_mn = mul_h16hi(h0, (float)mn);
    return xs * (d_sc * (float)dot - dmin_mn * xsum);
}

// the same term with the activation codes, scales and sums in LDS
__device__ __forceinline__ float pc_dot_q8(const Pc<F_Q4K> &P, const WDesc &W, const int8_t *lq, const float *ls,
                                           const int *lsum, int step, int lane) {
    const int K = W.cols, span = (K >> 8) * 128, off0 = step * 1024 + 16 * lane;
    // lane-constant parts of the activation offsets: the lane's low run is
    // sub-block c of super-block off0/128 (bytes blo*32 + half*16), its high
    // run 128 bytes on, its own block blo (+4 on the odd lane); the step adds
    // 2048 bytes / 64 blocks.  Lanes past the row's end read a clamped, valid
    // offset and contribute 0 through a zero activation scale.
    const Q4Lane L(lane);
    const int lo_b = min(step * 2048 + (lane >> 3) * 256 + ((lane >> 1) & 3) * 32 + (lane & 1) * 16, K - 144);
    const int own = min(step * 64 + (lane >> 3) * 8 + ((lane >> 1) & 3) + 4 * (lane & 1), (K >> 5) - 1);
    const v4i_t xl = *(const v4i_t *)(lq + lo_b);
    const v4i_t xh = *(const v4i_t *)(lq + lo_b + 128);
    const float xs = off0 < span ? ls[own] : 0.0f;
    return q4_term(P, xl, xh, xs, (float)lsum[own], L);
}

// ---- f32 input, quantized weights (logits): split activations -------------
// dequant (quantize.rs) then matvec_argmax_f32's f32 dot (model.rs:8668-8689).
// The f32 activation is held in LDS as three int8 levels per 16-element
// group, x ~= s1 a1 + s2 a2 + s3 a3: a1 quantizes x at s1 = max|x| / 127,
// a2 the remainder x - s1 a1 at its own max / 127, a3 the next remainder
// (each level gains >= 7.99 bits, so the represented x is within ~2^-24 of
// the group's largest element: fp32's own resolution).  A lane's 16 weights
// share one scale, so their dot is
//     scale * (s1 D1 + s2 D2 + s3 D3 - bias * G),  D_k = sum_j c_j a_kj
// with D_k three v_dot4_i32_i8 chains over the byte codes c_j (Q8_0: signed
// codes, bias 0; Q6_K: 6-bit codes 0..63, bias 32) and G = sum_k s_k sum_j
// a_kj, the represented group sum.  Instead of a conversion and an fp32 FMA
// per weight: 3 integer dots per 4 weights.  Equal to sum (scale * q_j) *
// x_j up to fp32 rounding (the accumulation order differs from the
// reference's sequential sum in any case; production parity is 1e-3
// relative; the reference-order mode has its own kernel).
// LDS: a1[K] | a2[K] | a3[K] | per group {s1, s2, s3, G} | red[64]
__host__ __device__ inline size_t mvs_split_lds_bytes(int K) { return (size_t)K * 3 + (size_t)(K / 16) * 16 + 64 * 4; }

struct XGrp {
    v4i_t a[3];
    v4f_t r;  // s1, s2, s3, G
    __device__ __forceinline__ void load(const char *smem, int K, int e) {
#pragma unroll
        for (int k = 0; k < 3; k++) a[k] = *(const v4i_t *)(smem + (size_t)k * K + e);
        r = *(const v4f_t *)(smem + (size_t)3 * K + (e >> 4) * 16);
    }
    // sum_j c_j x_j - BIAS * sum_j x_j over the group, codes c as 4 words
    template <int BIAS>
    __device__ __forceinline__ float dot(const uint32_t (&c)[4]) const {
        int d[3];
#pragma unroll
        for (int k = 0; k < 3; k++) {
            d[k] = __builtin_amdgcn_sdot4((int)c[0], a[k].x, 0, false);
            d[k] = __builtin_amdgcn_sdot4((int)c[1], a[k].y, d[k], false);
            d[k] = __builtin_amdgcn_sdot4((int)c[2], a[k].z, d[k], false);
            d[k] = __builtin_amdgcn_sdot4((int)c[3], a[k].w, d[k], false);
        }
        float v = r.x * (float)d[0];
        v = __builtin_fmaf(r.y, (float)d[1], v);
        v = __builtin_fmaf(r.z, (float)d[2], v);
        if (BIAS) v = __builtin_fmaf(-(float)BIAS, r.w, v);
        return v;
    }
};

// levels of one 16-element group held as NV values per thread (NV = 16: one
// thread; NV = 8: the lane pair t, t^1, t even holding the first half)
template <int NV>
__device__ __forceinline__ void split_levels(const float *v, char *smem, int K, int e0, bool lead) {
    float r[NV];
#pragma unroll
    for (int j = 0; j < NV; j++) r[j] = v[j];
    float sk[3], gs = 0.0f;
#pragma unroll
    for (int k = 0; k < 3; k++) {
        float m = 0.0f;
#pragma unroll
        for (int j = 0; j < NV; j++) m = fmaxf(m, fabsf(r[j]));
        if (NV == 8) m = fmaxf(m, __int_as_float(xpair(__float_as_int(m))));
        const float inv = m > 0.0f ? 127.0f / m : 0.0f, sc = m * (1.0f / 127.0f);
        uint32_t w[NV / 4];
        int sum = 0;
#pragma unroll
        for (int j = 0; j < NV; j++) {
            const int c = q8_code(r[j] * inv);
            r[j] = __builtin_fmaf(-sc, (float)c, r[j]);
            sum += c;
            if (j % 4 == 0) w[j / 4] = 0u;
            w[j / 4] |= ((uint32_t)c & 0xFFu) << (8 * (j % 4));
        }
        if (NV == 8) sum += xpair(sum);
        char *dst = smem + (size_t)k * K + e0;
        if constexpr (NV == 16) *(v4i_t *)dst = v4i_t{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
        else *(v2i_t *)dst = v2i_t{(int)w[0], (int)w[1]};
        sk[k] = sc;
        gs = __builtin_fmaf(sc, (float)sum, gs);
    }
    if (lead) *(v4f_t *)(smem + (size_t)3 * K + (e0 >> 4) * 16) = v4f_t{sk[0], sk[1], sk[2], gs};
}

template <int FMT>
struct XIn;

// Lane bytes of a Q8_0 piece: 16 codes of elements [off, off + 16), one group.
template <>
struct XIn<F_Q8_0> {
    XGrp g;
    bool ok;
    __device__ __forceinline__ void load(const WDesc &W, const char *smem, int step, int lane) {
        const int K = W.cols, off0 = step * 1024 + 16 * lane;
        g.load(smem, K, min(off0, K - 16));
        ok = off0 < K;
    }
};

__device__ __forceinline__ float pc_dot_f32x(const Pc<F_Q8_0> &P, const XIn<F_Q8_0> &X) {
    const uint32_t c[4] = {(uint32_t)P.q.x, (uint32_t)P.q.y, (uint32_t)P.q.z, (uint32_t)P.q.w};
    return X.ok ? mul_h16lo(P.sc, X.g.dot<0>(c)) : 0.0f;
}

// dequant_q6k_block (quantize.rs:343-384, llama.cpp layout): w = d*sc*q.
// Lane bytes: ql[hf*64 + qq*16 + i]; qq<2 -> q1 (low) / q3 (high), qq>=2 ->
// q2 / q4; the 2 qh bits sit at shift 2*(qq>>1) and +4.  The low nibbles are
// the 16 elements from e_lo, the high nibbles the 16 from e_lo + 64.
template <>
struct XIn<F_Q6K> {
    XGrp lo, hi;
    int sh;
    bool ok;
    __device__ __forceinline__ void load(const WDesc &W, const char *smem, int step, int lane) {
        const int K = W.cols, span = (K >> 8) * 128, off0 = step * 1024 + 16 * lane;
        const int off = min(off0, span - 16);
        const int sb = off >> 7, o = off & 127, hf = o >> 6, qq = (o >> 4) & 3;
        const int e_lo = sb * 256 + hf * 128 + (qq >> 1) * 32 + (qq & 1) * 16;
        lo.load(smem, K, e_lo);
        hi.load(smem, K, e_lo + 64);
        sh = 2 * (qq >> 1);
        ok = off0 < span;
    }
};

__device__ __forceinline__ float pc_dot_f32x(const Pc<F_Q6K> &P, const XIn<F_Q6K> &X) {
    uint32_t clo[4], chi[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        // four 6-bit codes per word, assembled byte-wise: nibble | 2 qh bits << 4
        const uint32_t lw = (uint32_t)P.ql[j], hw = (uint32_t)P.qh[j];
        // (the 2 bits at sh / sh + 4 of each qh byte land on bits 4-5 by one
        // shift within the byte, sh <= 2)
        clo[j] = (lw & 0x0F0F0F0Fu) | ((hw << (4 - X.sh)) & 0x30303030u);
        chi[j] = ((lw >> 4) & 0x0F0F0F0Fu) | ((hw >> X.sh) & 0x30303030u);
    }
    const float slo = X.lo.dot<32>(clo), shi = X.hi.dot<32>(chi);
    const float ds_lo = mul_h16lo(P.d, (float)(int8_t)P.sc0), ds_hi = mul_h16lo(P.d, (float)(int8_t)P.sc1);
    return X.ok ? ds_lo * slo + ds_hi * shi : 0.0f;
}

// ---- f32 input, f32 weights: x as floats in LDS ---------------------------
template <>
struct XIn<F_F32> {
    v4f_t x;
    bool ok;
    __device__ __forceinline__ void load(const WDesc &W, const char *smem, int step, int lane) {
        const float *lx = (const float *)smem;
        const int K = W.cols, off0 = step * 1024 + 16 * lane;
        const int off = min(off0, 4 * K - 16);
        x = *(const v4f_t *)(lx + (off >> 2));
        ok = off0 < 4 * K;
    }
};

__device__ __forceinline__ float pc_dot_f32x(const Pc<F_F32> &P, const XIn<F_F32> &X) {
    const float a = P.w.x * X.x.x + P.w.y * X.x.y + P.w.z * X.x.z + P.w.w * X.x.w;
    return X.ok ? a : 0.0f;
}

// ---------------------------------------------------------------------------
// arguments
// ---------------------------------------------------------------------------
struct MvsArgs {
    WDesc W;
    int pro, epi;          // prologue (PRO_* for Q8 input; 0 copy / 1 rmsnorm for f32 input), epilogue
    const float *x, *nw;   // prologue input and norm weight
    float eps;
    const int8_t *gq;      // PRO_LOADQ input
    const float *gs;
    const int *gsum;
    float *out;
    unsigned long long *slot;  // EPI_ARGMAX
    QkvEpi qkv;                // EPI_QKV
    // gate/up: F hidden units, Q8_0 output blocks, optional f32 copy
    int F;
    int8_t *hq;
    float *hs;
    int *hsum;
    float *hout;
    long long *trace;
    int seq;  // host-side: launch the reference-order (SEQ) instantiation
};

// f32 input: x[K] | gx[K/16] | red[64]; Q8 input: q[K] | scales, sums [K/32] | red
__host__ __device__ inline size_t mvs_lds_bytes(bool f32in, int K) {
    return f32in ? (size_t)K * 4 + (size_t)(K / 16) * 4 + 64 * 4 : (size_t)K + (size_t)(K / 32) * 8 + 64 * 4 + 64;
}
// gate/up: the Q8 input area, the 32 SiLU*up values of the current block,
// then one 256-byte exp table per wave
__host__ __device__ inline size_t mvs_lds_gu(int K, int nw) { return mvs_lds_bytes(false, K) + 32 * 4 + (size_t)nw * 256; }

// prologue staging shared by both kernels: x (Q8 or f32) into LDS
template <bool F32IN, int NT, bool SEQ = false, int VT = NT>
struct Stage;
template <int NT, bool SEQ, int VT>
struct Stage<false, NT, SEQ, VT> {
    StageQ8<NT, SEQ, VT> s;
    __device__ __forceinline__ void issue(const MvsArgs &a) { s.issue(a.pro, a.W.cols, a.x, a.nw, a.gq, a.gs, a.gsum); }
    __device__ __forceinline__ void finish(const MvsArgs &a, char *smem, float *ess = nullptr) {
        const int K = a.W.cols;
        int8_t *lq = (int8_t *)smem;
        float *ls = (float *)(smem + K);
        int *lsum = (int *)(ls + (K >> 5));
        float *red = (float *)(lsum + (K >> 5));
        s.finish(a.pro, K, a.eps, a.x, a.nw, lq, ls, lsum, red, a.trace, ess);
    }
};
template <int NT, bool SEQ, int VT>
struct Stage<true, NT, SEQ, VT> {
    StageF32<NT> s;
    __device__ __forceinline__ void issue(const MvsArgs &a) { s.issue(a.pro, a.W.cols, a.x, a.nw); }
    __device__ __forceinline__ void finish(const MvsArgs &a, char *smem, float * = nullptr) {
        const int K = a.W.cols;
        float *lx = (float *)smem;
        s.finish(a.pro, K, a.eps, a.x, a.nw, lx, lx + K + K / 16);
        // gx: sums of the 16-element groups of x (sequential fp32 per group)
        for (int gi = threadIdx.x; gi < K / 16; gi += NT) {
            float g = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; i++) g += lx[16 * gi + i];
            lx[K + gi] = g;
        }
        __syncthreads();
    }
};

// prologue of the split form (quantized weights, f32 input): x (pro 0) or
// rmsnorm(x) * w (pro 1, the same roundings as StageF32) -> the three int8
// levels and group records in LDS
template <int NT>
struct StageSplit {
    v4f_t xv[4], wv[4];
    __device__ __forceinline__ void issue(const MvsArgs &a) {
        const int t = threadIdx.x, n = a.W.cols, E = n / NT;
        if (n == NT * E && (E == 8 || E == 16)) {
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int o = min(t * E + 4 * k, n - 4);
                xv[k] = *(const v4f_t *)(a.x + o);
                wv[k] = *(const v4f_t *)((a.pro == 1 ? a.nw : a.x) + o);  // nw may be null for pro 0
            }
        }
    }
    __device__ __forceinline__ void finish(const MvsArgs &a, char *smem, float * = nullptr) {
        const int t = threadIdx.x, n = a.W.cols, E = n / NT;
        float *red = (float *)(smem + mvs_split_lds_bytes(n) - 64 * 4);
        if (n == NT * E && (E == 8 || E == 16)) {
            float xs[16], ws[16];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                xs[4 * k] = xv[k].x; xs[4 * k + 1] = xv[k].y; xs[4 * k + 2] = xv[k].z; xs[4 * k + 3] = xv[k].w;
                ws[4 * k] = wv[k].x; ws[4 * k + 1] = wv[k].y; ws[4 * k + 2] = wv[k].z; ws[4 * k + 3] = wv[k].w;
            }
            float inv = 1.0f;
            if (a.pro == 1) {
                float ss = 0.0f;
#pragma unroll
                for (int j = 0; j < 16; j++)
                    if (j < E) ss += xs[j] * xs[j];
                ss = wg_sum<NT>(ss, red);
                inv = 1.0f / sqrtf(ss / (float)n + a.eps);
            }
            float v[16];
#pragma unroll
            for (int j = 0; j < 16; j++) v[j] = (a.pro == 1) ? (xs[j] * inv) * ws[j] : xs[j];
            if (E == 16) split_levels<16>(v, smem, n, 16 * t, true);
            else split_levels<8>(v, smem, n, 8 * t, (t & 1) == 0);
        } else {
            const float inv = a.pro == 1 ? wg_inv_rms(a.x, n, a.eps, red) : 1.0f;
            for (int gi = t; gi < n / 16; gi += NT) {
                float v[16];
#pragma unroll
                for (int j = 0; j < 16; j++) {
                    const float xj = a.x[16 * gi + j];
                    v[j] = a.pro == 1 ? (xj * inv) * a.nw[16 * gi + j] : xj;
                }
                split_levels<16>(v, smem, n, 16 * gi, true);
            }
        }
        __syncthreads();
    }
};

// LDS of k_mvs's activation staging
template <int FMT, bool F32IN>
__host__ __device__ inline size_t mvs_lds_fmt(int K) {
    return (F32IN && FMT != F_F32) ? mvs_split_lds_bytes(K) : mvs_lds_bytes(F32IN, K);
}
__host__ __device__ inline size_t mvs_lds_fmt(int fmt, bool f32in, int K) {
    return (f32in && fmt != F_F32) ? mvs_split_lds_bytes(K) : mvs_lds_bytes(f32in, K);
}

template <int FMT, bool F32IN>
__device__ __forceinline__ float pc_dot(const Pc<FMT> &P, const WDesc &W, const char *smem, int step, int lane) {
    if constexpr (F32IN) {
        XIn<FMT> X;
        X.load(W, smem, step, lane);
        return pc_dot_f32x(P, X);
    } else {
        const int K = W.cols;
        const int8_t *lq = (const int8_t *)smem;
        const float *ls = (const float *)(smem + K);
        const int *lsum = (const int *)(ls + (K >> 5));
        return pc_dot_q8(P, W, lq, ls, lsum, step, lane);
    }
}

// ---------------------------------------------------------------------------
// Register-resident activation (Q8_0 weights, norm prologue, whole row in one
// unit: S <= SU steps).  Lane l of a wave reads exactly the activations
// [1024 s + 16 l, +16) of every step s, and a 32-block is a lane pair, so each
// wave normalizes and quantizes x itself: sum of squares by a wave reduction,
// block amax by a lane-pair exchange, codes and block scales kept in
// registers.  No LDS staging and no workgroup barrier: a wave starts on its
// weights as soon as its own activations have arrived.
// (rmsnorm_quantize_q8_0_scalar model.rs:5610-5640 / rmsnorm_scalar_into +
// quantize_input_q8_0_into 7456-7477, 5534-5571)
// ---------------------------------------------------------------------------
template <int SX, bool SEQ = false>
struct RegX8 {
    v4f_t xv[SX][4], wv[SX][4];
    v4i_t q[SX];
    float sc[SX];
    __device__ __forceinline__ void issue(const MvsArgs &a, int lane) {
        const int K = a.W.cols;
#pragma unroll
        for (int s = 0; s < SX; s++) {
            const int off = min(s * 1024 + 16 * lane, K - 16);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                xv[s][j] = *(const v4f_t *)(a.x + off + 4 * j);
                wv[s][j] = *(const v4f_t *)(a.nw + off + 4 * j);
            }
        }
    }
    // ess: this wave's kEssLdsWords floats of LDS (SEQ)
    __device__ __forceinline__ void finish(const MvsArgs &a, int lane, float *ess = nullptr) {
        const int K = a.W.cols;
        float ss = 0.0f;
        if constexpr (SEQ) {
            // the reference's sequential order, reproduced exactly (ess.h)
            float t[SX][16];
#pragma unroll
            for (int s = 0; s < SX; s++) {
                const bool ok = s * 1024 + 16 * lane < K;
#pragma unroll
                for (int i = 0; i < 16; i++) t[s][i] = ok ? xv[s][i >> 2][i & 3] * xv[s][i >> 2][i & 3] : 0.0f;
            }
            ss = ess_sumsq<SX>(t, K, lane, ess, a.x);
        } else {
#pragma unroll
            for (int s = 0; s < SX; s++) {
                if (s * 1024 + 16 * lane < K) {
#pragma unroll
                    for (int j = 0; j < 4; j++)
#pragma unroll
                        for (int k = 0; k < 4; k++) ss += xv[s][j][k] * xv[s][j][k];
                }
            }
            ss = wave_sum(ss);
        }
        const float rms = sqrtf(ss / (float)K + a.eps);
        const float inv = 1.0f / rms;
#pragma unroll
        for (int s = 0; s < SX; s++) {
            float v[16];
            // (x*w)*inv or (x*inv)*w: one branch on the uniform prologue kind
            if (a.pro == PRO_NORMQ0) {
#pragma unroll
                for (int i = 0; i < 16; i++) v[i] = xv[s][i >> 2][i & 3] * wv[s][i >> 2][i & 3] * inv;
            } else {
#pragma unroll
                for (int i = 0; i < 16; i++) v[i] = (xv[s][i >> 2][i & 3] * inv) * wv[s][i >> 2][i & 3];
            }
            float amax = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; i++) amax = fmaxf(amax, fabsf(v[i]));
            amax = fmaxf(amax, __int_as_float(xpair(__float_as_int(amax))));  // the block's other half
            const float d = amax / 127.0f;
            const float id = (d != 0.0f) ? 127.0f / amax : 0.0f;
            uint32_t pk[4] = {0, 0, 0, 0};
#pragma unroll
            for (int i = 0; i < 16; i++) pk[i >> 2] |= (uint32_t)(uint8_t)q8_code(v[i] * id) << (8 * (i & 3));
            q[s] = v4i_t{(int)pk[0], (int)pk[1], (int)pk[2], (int)pk[3]};
            sc[s] = d;
        }
    }
};

// PRO_LOADQ variant: the activation arrives quantized (the attention output,
// the SiLU*up hidden vector); each lane loads its own 16 codes and block scale
// per step straight into registers.
template <int SX>
struct RegX8L {
    v4i_t q[SX];
    float sc[SX];
    __device__ __forceinline__ void issue(const MvsArgs &a, int lane) {
        const int K = a.W.cols;
#pragma unroll
        for (int s = 0; s < SX; s++) {
            const int off = min(s * 1024 + 16 * lane, K - 16);
            q[s] = *(const v4i_t *)(a.gq + off);
            sc[s] = a.gs[off >> 5];
        }
    }
    __device__ __forceinline__ void finish(const MvsArgs &, int, float * = nullptr) {}
};

// PRO_LOADQ variant for Q4_K weights: lane l's 16 qs bytes of a step hold
// half `h` of sub-blocks c (low nibbles) and c+4 (high nibbles) of one
// super-block, so the lane loads those two 16-code runs of the pre-quantized
// activation and its own sub-block's (scale, code sum): c on the even lane,
// c+4 on the odd one (the pair add of pc_dot_q8 gives each its full block).
template <int SX>
struct RegX4L {
    v4i_t ql[SX], qh[SX];
    float sc[SX];
    int sm[SX];
    __device__ __forceinline__ void issue(const MvsArgs &a, int lane) {
        const int span = (a.W.cols >> 8) * 128;
#pragma unroll
        for (int s = 0; s < SX; s++) {
            const int off = min(s * 1024 + 16 * lane, span - 16);
            const int sb = off >> 7, c = (off >> 5) & 3, h = (off >> 4) & 1;
            const int blo = sb * 8 + c, bhi = blo + 4, own = h ? bhi : blo;
            ql[s] = *(const v4i_t *)(a.gq + blo * 32 + h * 16);
            qh[s] = *(const v4i_t *)(a.gq + bhi * 32 + h * 16);
            sc[s] = a.gs[own];
            sm[s] = a.gsum[own];
        }
    }
    __device__ __forceinline__ void finish(const MvsArgs &, int, float * = nullptr) {}
};

// dot_q4k_q8_0_scalar per-sub-block term (as pc_dot_q8) with the activation
// runs in registers
template <int SX>
__device__ __forceinline__ float pc_dot_q4x(const Pc<F_Q4K> &P, const WDesc &W, const RegX4L<SX> &X, int s,
                                            int lane) {
    const int span = (W.cols >> 8) * 128, off0 = s * 1024 + 16 * lane;
    return q4_term(P, X.ql[s], X.qh[s], off0 < span ? X.sc[s] : 0.0f, (float)X.sm[s], Q4Lane(lane));
}

// matvec_q8_0_preq_into per-block term with the activation codes in registers
__device__ __forceinline__ float pc_dot_q8x(const Pc<F_Q8_0> &P, const WDesc &W, const v4i_t &xq, float xs, int step,
                                            int lane) {
    int d = dot16(P.q, xq, 0);
    d += xpair(d);
    const float t = mul_h16lo(P.sc, xs) * (float)d;
    return (step * 1024 + 16 * lane < W.cols && !(lane & 1)) ? t : 0.0f;
}

// ---------------------------------------------------------------------------
// Reference-order row sums (SEQ kernels).  The reference adds the per-block
// terms of a row one at a time in block order (model.rs:8082-8099 for Q8_0,
// 8997-9014 for Q4_K).  Within one 1 KiB step, lane l holds the term of the
// piece at byte 16*l: Q8_0 block 32*step + l/2 on the even lane (the odd
// lane's copy is zero); Q4_K super-block l/8, sub-block c = (l/2)%4 (even
// lane, low nibbles) or c+4 (odd lane), i.e. the reference's order lo(0),
// hi(0), lo(1), hi(1), ...  A unit's terms pass through a wave-private LDS
// area and lane r adds row r's terms in that order to its running sum.  The
// tiles, loads, integer dots and per-block float terms are the ones the
// tree-order kernels use.
// ---------------------------------------------------------------------------
template <int FMT, int R, int SU>
struct SeqFold {
    float run = 0.0f;  // lane r: running sum of row r
    __device__ __forceinline__ void add(const float (&t)[R][SU], float *fs, int rr, int lane) {
#pragma unroll
        for (int r = 0; r < R; r++)
#pragma unroll
            for (int s = 0; s < SU; s++) fs[(r * SU + s) * 64 + lane] = t[r][s];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if (rr == 0) run = 0.0f;
        if (lane < R) {
            // all 64 terms of a step are read before the dependent adds; the
            // terms past the row's end are +-0 and leave the sum unchanged
            // (the running sum starts at +0 and never becomes -0)
#pragma unroll
            for (int s = 0; s < SU; s++) {
                const v4f_t *p = (const v4f_t *)(fs + (lane * SU + s) * 64);
                v4f_t v[16];
#pragma unroll
                for (int i = 0; i < 16; i++) v[i] = p[i];
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    if (FMT == F_Q8_0) {  // one term per lane pair (the even lane)
                        run += v[i].x;
                        run += v[i].z;
                    } else {
                        run += v[i].x;
                        run += v[i].y;
                        run += v[i].z;
                        run += v[i].w;
                    }
                }
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    // row r's sum, read from lane r (every lane gets it)
    __device__ __forceinline__ float row(int r) const {
        return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(run), r));
    }
};

__host__ __device__ inline size_t align16(size_t b) { return (b + 15) & ~(size_t)15; }
// LDS of the SEQ areas, per wave: the fold terms (R x SU x 64 floats) or the
// exact sum of squares' scratch (wave 0's area also serves the workgroup form)
__host__ __device__ inline int seq_wave_words(int r, int su) {
    const int f = r * su * 64, e = (kEssLdsWords + 1 + 3) & ~3;
    return f > e ? f : e;
}
__host__ __device__ inline size_t seq_lds_bytes(int waves, int r, int su) { return (size_t)waves * seq_wave_words(r, su) * 4; }

// ---------------------------------------------------------------------------
// k_mvs: generic persistent streaming matvec
// ---------------------------------------------------------------------------
constexpr int kMvsThreads = 256;

// RX: register-resident activation (Q8_0, S <= SU): 1 = norm prologue
// (RegX8), 2 = pre-quantized input (RegX8L)
// SEQ: row sums and the norm's sum of squares in the reference's sequential
// order (SeqFold, seq_sumsq); LDS grows by seq_lds_bytes(4, R, SU)
// Row groups a set of waves walks: every group of the weight (RowsAll), or
// the groups of one kv head's rows in the fused QKV weight (RowsKvGroup:
// the G*D query rows of its heads, then its D key rows, then its D value
// rows; rows are [q (nq) | k (nk) | v (nk)], R divides D).
struct RowsAll {
    int ngrp;
    __device__ __forceinline__ int rg(int i) const { return i; }
};
struct RowsKvGroup {
    int ngrp, h, qg, kg, nq, nk, R;  // qg = G*D/R, kg = D/R row groups
    __device__ __forceinline__ int rg(int i) const {
        if (i < qg) return h * qg + i;
        if (i < qg + kg) return (nq / R) + h * kg + (i - qg);
        return ((nq + nk) / R) + h * kg + (i - qg - kg);
    }
};

// The persistent matvec of one set of waves: global wave gw of tw walks row
// groups map.rg(gw), map.rg(gw + tw), ...  NT: threads per workgroup.
template <int FMT, bool F32IN, int R, int SU, int RX, bool SEQ, int NT, typename Map>
__device__ __forceinline__ void mvs_body(const MvsArgs &a, char *smem, int gw, int tw, const Map &map) {
    static_assert(!RX || ((FMT == F_Q8_0 || (FMT == F_Q4K && RX == 2)) && !F32IN),
                  "register activation: Q8_0 weights (or pre-quantized Q4_K input), Q8 input");
    static_assert(!SEQ || !F32IN, "reference-order sums: Q8 input");
    const WDesc &W = a.W;
    const int K = W.cols;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int S = mvs_steps(FMT, K), NR = (S + SU - 1) / SU;
    const int ngrp = map.ngrp;
    const int nunits = gw < ngrp ? ((ngrp - 1 - gw) / tw + 1) * NR : 0;

    Pc<FMT> ta[R][SU], tb[R][SU];
    auto load = [&](Pc<FMT>(&T)[R][SU], int u) {
        const int k = u / NR, rr = u - k * NR, rg = map.rg(min(gw + k * tw, ngrp - 1));
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int row = min(rg * R + r, W.rows - 1);
#pragma unroll
            for (int s = 0; s < SU; s++) T[r][s].load(W, row, min(rr * SU + s, S - 1), lane);
        }
    };
    MV_TS(0);
    MV_TSB(0);
    // (the Q8 staging of a wider workgroup keeps the decomposition of a
    // kMvsThreads one: the same norm sums as k_mvs)
    typename std::conditional<F32IN && FMT != F_F32, StageSplit<NT>,
                              Stage<F32IN, NT, SEQ, (NT > kMvsThreads ? kMvsThreads : NT)>>::type stg;
    typename std::conditional<RX == 2, typename std::conditional<FMT == F_Q4K, RegX4L<SU>, RegX8L<SU>>::type,
                              RegX8<RX ? SU : 1, SEQ>>::type rx;
    if constexpr (RX) rx.issue(a, lane);
    else stg.issue(a);             // 1. activation loads
    FLARE_STAGE_BARRIER();  // keep them ahead of the weight loads (loads complete in order)
    load(ta, 0);                   // 2. first weight pieces (unconditional: clamped rows are valid, and
                                   // the prologue below then waits for the activation loads only)
    const int qpos = a.epi == EPI_QKV ? ld_uniform(a.qkv.posp) : 0;
    // epilogue operands of the wave's first row group, in flight with the
    // first tile: the residual rows (EPI_ADD, lane r = row r) or lane p's
    // RoPE (cos, sin) (EPI_QKV)
    // Both loads are issued on every path (valid addresses, clamped or a
    // stand-in), so the compiler's wait counts stay static and the prologue
    // waits for the activation loads only.
    float pre0, pre1;
    {
        const int row0f = min(map.rg(min(gw, ngrp - 1)) * R, W.rows - 1);
        const float *p0 = (const float *)W.q, *p1 = (const float *)W.q;
        if (a.epi == EPI_ADD) {
            p0 = a.out + min(row0f + min(lane, R - 1), W.rows - 1);
            p1 = p0;
        }
        if (a.epi == EPI_QKV) {
            const int half = a.qkv.hd >> 1;
            const int n = min(row0f + 2 * min(lane, R / 2 - 1), W.rows - 1);
            p0 = a.qkv.rope_cur + ((n % a.qkv.hd) >> 1);  // no dependence on the position load
            p1 = p0 + half;
        }
        pre0 = *p0;
        pre1 = *p1;
    }
    MV_TS(1);
    float *seqa = (float *)(smem + align16(mvs_lds_fmt<FMT, F32IN>(K)));  // SEQ areas
    float *fs = seqa + wave * seq_wave_words(R, SU);
    if constexpr (RX) rx.finish(a, lane, fs);
    else stg.finish(a, smem, seqa);  // 3. prologue arithmetic (ends with a barrier)
    MV_TS(2);

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;
    unsigned long long best = 0;
    SeqFold<FMT, R, SU> fold;
    auto consume = [&](const Pc<FMT>(&T)[R][SU], int u) {
        const int k = u / NR, rr = u - k * NR, rg = map.rg(gw + k * tw);
        if constexpr (SEQ) {
            float t[R][SU];
#pragma unroll
            for (int r = 0; r < R; r++)
#pragma unroll
                for (int s = 0; s < SU; s++) {
                    if constexpr (RX) t[r][s] = pc_dot_q8x(T[r][s], W, rx.q[s], rx.sc[s], s, lane);
                    else t[r][s] = pc_dot<FMT, false>(T[r][s], W, smem, rr * SU + s, lane);
                }
            fold.add(t, fs, rr, lane);
        } else if constexpr (F32IN) {
            // one step at a time: the lane's activation floats are loaded
            // once and shared by the R rows (not hoisted for the whole tile)
#pragma unroll
            for (int s = 0; s < SU; s++) {
                XIn<FMT> X;
                X.load(W, smem, rr * SU + s, lane);
#pragma unroll
                for (int r = 0; r < R; r++) acc[r] += pc_dot_f32x(T[r][s], X);
                __builtin_amdgcn_sched_barrier(0);
            }
        } else if constexpr (RX) {
            // one unit covers the row (NR == 1): step s is compile-time
#pragma unroll
            for (int r = 0; r < R; r++)
#pragma unroll
                for (int s = 0; s < SU; s++) {
                    if constexpr (FMT == F_Q4K) acc[r] += pc_dot_q4x(T[r][s], W, rx, s, lane);
                    else acc[r] += pc_dot_q8x(T[r][s], W, rx.q[s], rx.sc[s], s, lane);
                }
        } else {
#pragma unroll
            for (int r = 0; r < R; r++)
#pragma unroll
                for (int s = 0; s < SU; s++) acc[r] += pc_dot<FMT, F32IN>(T[r][s], W, smem, rr * SU + s, lane);
        }
        if (u == 0) MV_TS(3);
        if (rr == NR - 1) {
#pragma unroll
            for (int r = 0; r < R; r++) acc[r] = SEQ ? fold.row(r) : wave_sum(acc[r]);
            const int row0 = rg * R;
            if (a.epi == EPI_ARGMAX) {
                best = umax64(best, rows_best<R>(acc, row0, W.rows));
            } else if (a.epi == EPI_ADD) {
                // residual add (model.rs:2305-2311, 2537-2543): lane r adds row r
                const float v = lane_row<R>(acc, lane);
                if (lane < R && row0 + lane < W.rows) a.out[row0 + lane] = (k == 0 ? pre0 : a.out[row0 + lane]) + v;
            } else if constexpr (R % 2 == 0) {
                if (a.epi == EPI_QKV) store_qkv<R>(acc, row0, W.rows, lane, a.qkv, qpos, a.out, k == 0, pre0, pre1);
                else store_rows<R>(acc, row0, W.rows, lane, a.epi, a.out);
            } else {
                store_rows<R>(acc, row0, W.rows, lane, a.epi, a.out);
            }
#pragma unroll
            for (int r = 0; r < R; r++) acc[r] = 0.0f;
        }
    };
    // ping-pong: the next unit's pieces are in flight while this one is
    // consumed
    pingpong(nunits, ta, tb, load, consume);
    MV_TS(4);
    if (a.epi == EPI_ARGMAX) {
        float *red = (float *)(smem + mvs_lds_fmt<FMT, F32IN>(K) - 64 * 4 - (F32IN ? 0 : 64));
        wg_argmax_commit(best, a.slot, (unsigned long long *)red);
    }
    MV_TSB(1);
}

template <int FMT, bool F32IN, int R, int SU, int RX = 0, bool SEQ = false>
__global__ __launch_bounds__(kMvsThreads) void k_mvs(MvsArgs a) {
    extern __shared__ __align__(16) char smem[];
    constexpr int NW = kMvsThreads / 64;
    mvs_body<FMT, F32IN, R, SU, RX, SEQ, kMvsThreads>(a, smem, (int)blockIdx.x * NW + (threadIdx.x >> 6),
                                                      (int)gridDim.x * NW, RowsAll{(a.W.rows + R - 1) / R});
}

// ---------------------------------------------------------------------------
// k_mvs_gu: fused gate/up + SiLU + Q8_0 quantization of the hidden vector
// (model.rs:2376-2416, silu_mul_into 9783-9796, quantize 2480-2522).
// Rows [0, F) are w_gate, [F, 2F) w_up.  Workgroup b owns hidden blocks
// b, b + grid, ...; wave w takes hidden units 32*blk + w*HU .. + HU, HU/2 at
// a time (item = 2 gate rows + the 2 matching up rows).
// ---------------------------------------------------------------------------
template <int FMT, int SU, int NW, int RX = 0, bool SEQ = false>
__global__ __launch_bounds__(NW * 64) void k_mvs_gu(MvsArgs a) {
    static_assert(!RX || FMT == F_Q8_0, "register activation: Q8_0 weights");
    extern __shared__ __align__(16) char smem[];
    constexpr int NT = NW * 64, HU = 32 / NW, IPB = HU / 2;  // items per wave per block
    static_assert(HU % 2 == 0, "two hidden units per item");
    constexpr int R = 4;
    const WDesc &W = a.W;
    const int K = W.cols, F = a.F;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int S = mvs_steps(FMT, K), NR = (S + SU - 1) / SU;
    const int nblk = F / 32;
    const int myblk = (int)blockIdx.x < nblk ? (nblk - 1 - (int)blockIdx.x) / (int)gridDim.x + 1 : 0;
    const int upb = IPB * NR;  // units per block per wave
    const int nunits = myblk * upb;
    float *hb = (float *)(smem + mvs_lds_bytes(false, K));  // [32] SiLU*up of the current block

    Pc<FMT> ta[R][SU], tb[R][SU];
    auto rows_of = [&](int u, int &blk, int &item, int &rr) {
        const int kb = u / upb, rem = u - kb * upb;
        item = rem / NR;
        rr = rem - item * NR;
        blk = (int)blockIdx.x + kb * (int)gridDim.x;
    };
    auto load = [&](Pc<FMT>(&T)[R][SU], int u) {
        int blk, item, rr;
        rows_of(u, blk, item, rr);
        const int f = blk * 32 + wave * HU + item * 2;
        const int rws[R] = {f, f + 1, F + f, F + f + 1};
#pragma unroll
        for (int r = 0; r < R; r++)
#pragma unroll
            for (int s = 0; s < SU; s++) T[r][s].load(W, rws[r], min(rr * SU + s, S - 1), lane);
    };
    MV_TS(0);
    MV_TSB(0);
    Stage<false, NT, SEQ> stg;
    typename std::conditional<RX == 2, RegX8L<SU>, RegX8<RX ? SU : 1, SEQ>>::type rx;
    // the SiLU's exp table, one copy per wave in LDS: a global table load in
    // the epilogue would wait for the next tile's loads (loads complete in
    // order); an LDS read does not
    uint64_t *etab = (uint64_t *)(hb + 32) + wave * 32;
    const uint64_t etv = kExp2Tab[lane & 31];
    if constexpr (RX) rx.issue(a, lane);
    else stg.issue(a);
    FLARE_STAGE_BARRIER();
    load(ta, 0);  // unconditional, so the prologue waits for the activation loads only
    if (lane < 32) etab[lane] = etv;
    MV_TS(1);
    float *seqa = (float *)(smem + align16(mvs_lds_gu(K, NW)));  // SEQ areas
    float *fs = seqa + wave * seq_wave_words(R, SU);
    if constexpr (RX) rx.finish(a, lane, fs);
    else stg.finish(a, smem, seqa);
    MV_TS(2);

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;
    SeqFold<FMT, R, SU> fold;
    auto consume = [&](const Pc<FMT>(&T)[R][SU], int u) {
        int blk, item, rr;
        rows_of(u, blk, item, rr);
        if constexpr (SEQ) {
            float t[R][SU];
#pragma unroll
            for (int r = 0; r < R; r++)
#pragma unroll
                for (int s = 0; s < SU; s++) {
                    if constexpr (RX) t[r][s] = pc_dot_q8x(T[r][s], W, rx.q[s], rx.sc[s], s, lane);
                    else t[r][s] = pc_dot<FMT, false>(T[r][s], W, smem, rr * SU + s, lane);
                }
            fold.add(t, fs, rr, lane);
        } else {
#pragma unroll
            for (int r = 0; r < R; r++)
#pragma unroll
                for (int s = 0; s < SU; s++) {
                    if constexpr (RX) acc[r] += pc_dot_q8x(T[r][s], W, rx.q[s], rx.sc[s], s, lane);
                    else acc[r] += pc_dot<FMT, false>(T[r][s], W, smem, rr * SU + s, lane);
                }
        }
        if (u == 0) MV_TS(3);
        if (rr == NR - 1) {
#pragma unroll
            for (int r = 0; r < R; r++) acc[r] = SEQ ? fold.row(r) : wave_sum(acc[r]);
            if (lane < 2) {
                // silu_mul_into: g / (1 + exp(-g)) * u
                const float g = lane ? acc[1] : acc[0], up = lane ? acc[3] : acc[2];
                hb[wave * HU + item * 2 + lane] = (g / (1.0f + fl_expf_t(-g, etab))) * up;
            }
#pragma unroll
            for (int r = 0; r < R; r++) acc[r] = 0.0f;
            if (item == IPB - 1) {
                // block complete on every wave: quantize it
                __syncthreads();
                if (threadIdx.x < 32) {
                    const float h = hb[threadIdx.x];
                    if (a.hout) a.hout[blk * 32 + threadIdx.x] = h;
                    quant_block32_lanes(h, a.hq + blk * 32, a.hs + blk, a.hsum + blk);
                }
                __syncthreads();  // hb reused by the next block
                if (u == upb - 1) MV_TS(4);
            }
        }
    };
    pingpong(nunits, ta, tb, load, consume);
    MV_TS(5);
    MV_TSB(1);
}

}  // namespace fl
