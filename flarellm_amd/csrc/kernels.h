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
#include <stdlib.h>

namespace fl {

// Measurement switches (tile shapes, split counts, rejected kernel variants,
// trace dumps) are read from the environment in FLARE_MEASURE builds only; the
// product library ignores them and runs the measured defaults.
inline const char *measure_env(const char *name) {
#ifdef FLARE_MEASURE
    return getenv(name);
#else
    (void)name;
    return nullptr;
#endif
}

constexpr int kThreads = 256;  // 4 wave64 per workgroup

enum Fmt { F_F32 = 0, F_Q8_0 = 1, F_Q4K = 2, F_Q6K = 3 };

// Native 16-/8-byte vectors.  HIP's int4/float4 are structs whose copies
// lower to memcpy through a private alloca (scratch memory); these stay in
// registers.
typedef int v4i_t __attribute__((ext_vector_type(4)));
typedef float v4f_t __attribute__((ext_vector_type(4)));
typedef int v2i_t __attribute__((ext_vector_type(2)));

// ------------------------------------------------------------------------
// small helpers
// ------------------------------------------------------------------------
__device__ __forceinline__ float h2f(uint16_t h) { return __half2float(__ushort_as_half(h)); }
__device__ __forceinline__ uint16_t f2h(float f) { return __half_as_ushort(__float2half(f)); }

// v_dot4_i32_i8 with an inline-constant zero accumulator: the builtin's
// v_dot4c form accumulates in place and first needs a v_mov of 0
__device__ __forceinline__ int dot4_z(int a, int b) {
    int r;
    asm("v_dot4_i32_i8 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
    return r;
}

__device__ __forceinline__ int dot16(const v4i_t &a, const v4i_t &b, int c) {
    if (__builtin_constant_p(c) && c == 0) c = dot4_z(a.x, b.x);
    else c = __builtin_amdgcn_sdot4(a.x, b.x, c, false);
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

// DPP reductions inside one 16-lane row: every lane of each aligned group of
// W lanes (W = 2, 4, 8, 16) ends with the group's sum/max.  Each step adds a
// lane to its partner (commutative), so all lanes of a group agree bit-wise.
#define FL_DPP(v, ctrl) __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), ctrl, 0xF, 0xF, false))
template <int W>
__device__ __forceinline__ float row_sum(float v) {
    static_assert(W == 2 || W == 4 || W == 8 || W == 16, "row_sum width");
    v += FL_DPP(v, 0xB1);                    // quad_perm [1,0,3,2]
    if (W >= 4) v += FL_DPP(v, 0x4E);        // quad_perm [2,3,0,1]
    if (W >= 8) v += FL_DPP(v, 0x141);       // row_half_mirror
    if (W >= 16) v += FL_DPP(v, 0x140);      // row_mirror
    return v;
}
template <int W>
__device__ __forceinline__ float row_max(float v) {
    static_assert(W == 2 || W == 4 || W == 8 || W == 16, "row_max width");
    v = fmaxf(v, FL_DPP(v, 0xB1));
    if (W >= 4) v = fmaxf(v, FL_DPP(v, 0x4E));
    if (W >= 8) v = fmaxf(v, FL_DPP(v, 0x141));
    if (W >= 16) v = fmaxf(v, FL_DPP(v, 0x140));
    return v;
}
// Sum over all 64 lanes, every lane with the same value: DPP sums inside the
// 16-lane rows, then the four row sums read into scalars (v_readlane: no LDS
// round trips) and added as (r0 + r1) + (r2 + r3), the order of the
// cross-row shuffle form (xor 16, then xor 32).  The whole wave must be active.
__device__ __forceinline__ float wave_sum(float v) {
    v = row_sum<16>(v);
    const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return (a + b) + (c + d);
}
// Max over all 64 lanes (DPP within rows, then two cross-row shuffles).
__device__ __forceinline__ float wave_max(float v) {
    v = row_max<16>(v);
    v = fmaxf(v, __shfl_xor(v, 16, 64));
    v = fmaxf(v, __shfl_xor(v, 32, 64));
    return v;
}

// Workgroup-wide sum with a fixed combination order (deterministic).  NT:
// the workgroup's thread count when known at compile time (0: blockDim.x,
// which is read from the dispatch packet).
template <int NT = 0>
__device__ __forceinline__ float wg_sum(float v, float *red) {
    v = wave_sum(v);
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    __syncthreads();
    if (lane == 0) red[w] = v;
    __syncthreads();
    float t = 0.0f;
    const int nw = NT ? NT / 64 : (int)(blockDim.x >> 6);
    for (int i = 0; i < nw; i++) t += red[i];
    return t;
}

// Double-buffered streaming loops: unit u + 1's loads are in flight while
// unit u is consumed (ta holds unit 0 on entry).  The steady-state loop issues its
// loads unconditionally and the last one or two units are consumed after it:
// with a load under a branch the compiler must assume the path that issued
// none, and the consume of a tile would then wait for the next tile's loads
// too (loads complete in order), losing the overlap.
template <typename T, typename L, typename C>
__device__ __forceinline__ void pingpong(int nunits, T &ta, T &tb, const L &load, const C &consume) {
    int u = 0;
    for (; u + 2 < nunits; u += 2) {
        load(tb, u + 1);
        consume(ta, u);
        load(ta, u + 2);
        consume(tb, u + 1);
    }
    if (u + 1 < nunits) {
        load(tb, u + 1);
        consume(ta, u);
        consume(tb, u + 1);
    } else if (u < nunits) {
        consume(ta, u);
    }
}

// Agent-scope relaxed atomic float store / load (cross-XCD visible without
// a cache write-back fence).
__device__ __forceinline__ void st_agent(float *p, float v) {
    __hip_atomic_store((unsigned *)p, __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_agent(const float *p) {
    return __uint_as_float(__hip_atomic_load((const unsigned *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}
// two adjacent floats (8-byte aligned) in one agent-scope load
__device__ __forceinline__ float2 ld_agent2(const float *p) {
    const unsigned long long u =
        __hip_atomic_load((const unsigned long long *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return make_float2(__uint_as_float((unsigned)u), __uint_as_float((unsigned)(u >> 32)));
}

// f32 product of the f16 in the low (high) half of w and b, rounded once as a
// plain multiply: v_fma_mix_f32 with the f16 operand selected by op_sel and a
// -0 addend (x + -0 = x for every x, signed zeros included), one op instead of
// a conversion and a multiply
__device__ __forceinline__ float mul_h16lo(uint32_t w, float b) {
    float r;
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(w), "v"(b), "v"(-0.0f));
    return r;
}
__device__ __forceinline__ float mul_h16hi(uint32_t w, float b) {
    float r;
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(w), "v"(b), "v"(-0.0f));
    return r;
}

// A uniform int read through the scalar data cache (s_load_dword): waiting
// for it does not wait for the vector loads in flight, as the wait for a
// vector load does (loads complete in order).  Only for data that no kernel
// writes while the reading kernel runs (the scalar cache is invalidated at
// each launch).
__device__ __forceinline__ int ld_uniform(const int *p) {
    return *(const __attribute__((address_space(4))) int *)p;
}

// ------------------------------------------------------------------------
// expf with the arithmetic of the x86-64 reference.  Rust's f32::exp lowers to
// the C library's expf; glibc (sysdeps/ieee754/flt-32/e_expf.c, the published
// ARM optimized-routines algorithm) computes it in double precision as
//   z = x * 32/ln2, k = round(z) (shift trick), r = z - k,
//   exp(x) = 2^(k/32) * (1 + C2 r + C1 r^2 + C0 r^3),
// with 2^(i/32) from a 32-entry table, and on FMA-capable hosts evaluates r
// and the polynomial with fused multiply-adds.  Every operation here is an
// IEEE double operation with the same rounding, so the result is bit-identical
// to the host's expf: checked for all 2^32 float inputs on the CPU, and on
// the GPU against the host library by the tests.
// kExp2Tab[i] = bits(2^(i/32) rounded to double) - (i << 47).
// ------------------------------------------------------------------------
__device__ static const uint64_t kExp2Tab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull};

// fl_expf with the table read from `tab` (a copy of kExp2Tab, e.g. in LDS)
__device__ __forceinline__ float fl_expf_t(float x, const uint64_t *tab) {
    if (x != x) return x + x;                   // NaN
    if (x == -INFINITY) return 0.0f;
    if (x > 0x1.62e42ep6f) return INFINITY;     // above log(2^128)
    if (x < -0x1.9fe368p6f) return 0.0f;        // below log(2^-150)
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32, shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32, c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32,
                 c2 = 0x1.62e42ff0c52d6p-1 / 32;
    const double xd = (double)x;
    const double z = inv_ln2_n * xd;
    double kd = z + shift;
    const uint64_t ki = (uint64_t)__double_as_longlong(kd);
    kd -= shift;
    const double r = __builtin_fma(inv_ln2_n, xd, -kd);
    const uint64_t t = tab[ki % 32] + (ki << 47);
    const double s = __longlong_as_double((long long)t);
    const double p = __builtin_fma(c0, r, c1);
    const double r2 = r * r;
    double y = __builtin_fma(c2, r, 1.0);
    y = __builtin_fma(p, r2, y);
    y = y * s;
    return (float)y;
}

__device__ __forceinline__ float fl_expf(float x) {
    if (x != x) return x + x;                   // NaN
    if (x == -INFINITY) return 0.0f;
    if (x > 0x1.62e42ep6f) return INFINITY;     // above log(2^128)
    if (x < -0x1.9fe368p6f) return 0.0f;        // below log(2^-150)
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32, shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32, c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32,
                 c2 = 0x1.62e42ff0c52d6p-1 / 32;
    const double xd = (double)x;
    const double z = inv_ln2_n * xd;
    double kd = z + shift;
    const uint64_t ki = (uint64_t)__double_as_longlong(kd);
    kd -= shift;
    const double r = __builtin_fma(inv_ln2_n, xd, -kd);
    const uint64_t t = kExp2Tab[ki % 32] + (ki << 47);
    const double s = __longlong_as_double((long long)t);
    const double p = __builtin_fma(c0, r, c1);
    const double r2 = r * r;
    double y = __builtin_fma(c2, r, 1.0);
    y = __builtin_fma(p, r2, y);
    y = y * s;
    return (float)y;
}

// ------------------------------------------------------------------------
// Arrival of a workgroup at a split-merge counter (split-K attention, fused
// verify GEMM epilogues).  The workgroup has stored its partials with
// agent-scope atomic stores; returns true (in every thread) in the workgroup
// that arrives last, after which its agent-scope loads see every other
// workgroup's partials.  RESET: the last arrival sets the counter back to 0.
//   FLARE_SPLIT_SYNC 1 (default): each wave waits for its own stores
//     (s_waitcnt 0), workgroup barrier, thread 0 counts with a relaxed
//     agent-scope RMW; the partials themselves move only through agent-scope
//     atomic stores / loads.
//   2: each wave's agent-scope release fence before the barrier, thread 0
//     counts with an acq_rel RMW, the last workgroup's waves acquire at agent
//     scope before loading (an L2 writeback + invalidate on gfx950).
//   0: barrier, thread 0's acq_rel RMW only.
// (2 and 0 exist in FLARE_MEASURE builds only.)
// Why 1 is sufficient on gfx950.  The partials are written with agent-scope
// atomic stores, which carry the device scope bits (sc1): they are written
// through to the device's point of coherence (past the per-XCD L2s), and a
// store is acknowledged -- vmcnt decremented -- only once it is there.  The
// s_waitcnt 0 of every wave therefore means all its partials are visible
// device-wide before the barrier, and thread 0's counting RMW is issued
// after the barrier.  The last arriver issues its loads after that RMW has
// returned (the flag passes through LDS and a barrier), and they are
// agent-scope atomic loads, which read from the point of coherence rather
// than a possibly stale L2 line.  A release fence would add an L2 writeback
// of non-atomic data (there is none) and an acquire fence an L2 invalidate
// for non-atomic loads (there are none): the measured 3.41 vs 4.83 ms per
// C5 verify pass is that extra cache maintenance.  The split-merge tests
// (bit-repeatable over 20 launches, forced splits, every verify test) run
// on this form.
// ------------------------------------------------------------------------
#ifndef FLARE_SPLIT_SYNC
#define FLARE_SPLIT_SYNC 1
#endif
#if FLARE_SPLIT_SYNC != 1 && !defined(FLARE_MEASURE)
#error "FLARE_SPLIT_SYNC variants other than 1 are measurement builds (define FLARE_MEASURE)"
#endif
template <bool RESET>
__device__ __forceinline__ bool split_arrive_last(int *counter, int n, int *flag) {
#if FLARE_SPLIT_SYNC == 2
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    __syncthreads();
    if (threadIdx.x == 0) {
        const int old = __hip_atomic_fetch_add(counter, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        *flag = old == n - 1;
        if (RESET && old == n - 1) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    const bool last = *flag != 0;
    if (last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    return last;
#elif FLARE_SPLIT_SYNC == 1
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
        const int old = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *flag = old == n - 1;
        if (RESET && old == n - 1) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    return *flag != 0;
#else
    __syncthreads();
    if (threadIdx.x == 0) {
        const int old = __hip_atomic_fetch_add(counter, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        *flag = old == n - 1;
        if (RESET && old == n - 1) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    return *flag != 0;
#endif
}

// Sum of squares in the reference's order: a sequential f32 fold over the
// vector (x.iter().map(|v| v * v).sum(), model.rs:5615 / 7466).  Every lane
// runs the same chain on uniform loads and holds the result.
__device__ __forceinline__ float seq_sumsq(const float *x, int n) {
    float ss = 0.0f;
    for (int j = 0; j < n; j += 4) {
        const v4f_t v = *(const v4f_t *)(x + j);
        ss += v.x * v.x;
        ss += v.y * v.y;
        ss += v.z * v.z;
        ss += v.w * v.w;
    }
    return ss;
}

__device__ __forceinline__ int8_t sat_i8(float v) {
    v = fminf(fmaxf(v, -128.0f), 127.0f);
    return (int8_t)(int)v;
}

// quantize_input_q8_0_into's code (y).round() as i8 (model.rs:5557-5570):
// round half away from zero, then saturate to [-128, 127] (a NaN gives -128,
// as sat_i8 does).  Adding the largest float below 0.5 with y's sign and
// truncating rounds exactly as roundf for every float: the sum reaches the
// next integer only when y's fraction is at least 0.5 (at a fraction just
// below 0.5 it stays at least an ulp short), and a y of 2^23 or more is
// already an integer that the addition rounds back to.  Clamping before the
// truncation does not change the result.  4 ops against roundf's 8.
__device__ __forceinline__ int8_t q8_code(float y) {
    const float s = y + __builtin_copysignf(0.49999997f, y);
    return (int8_t)(int)fminf(fmaxf(s, -128.0f), 127.0f);
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
            int8_t qq = q8_code(v[4 * j + k] * id);
            acc += qq;
            p |= (uint32_t)(uint8_t)qq << (8 * k);
        }
        packed[j] = (int)p;
    }
    v4i_t *qd = (v4i_t *)q;
    qd[0] = v4i_t{packed[0], packed[1], packed[2], packed[3]};
    qd[1] = v4i_t{packed[4], packed[5], packed[6], packed[7]};
    *s = d;
    *sum = acc;
}

// quantize_input_q8_0_into for one 32-block held one value per lane by lanes
// 0..31 (and a second block by lanes 32..63).  Same arithmetic as
// quant_block32; all 32 lanes compute the identical d / id.
__device__ __forceinline__ void quant_block32_lanes(float v, int8_t *q, float *s, int *sum) {
    const int lane = threadIdx.x & 31;
    float amax = fabsf(v);
    amax = row_max<16>(amax);
    amax = fmaxf(amax, __shfl_xor(amax, 16, 64));
    const float d = amax / 127.0f;
    const float id = (d != 0.0f) ? 127.0f / amax : 0.0f;
    const int8_t qq = q8_code(v * id);
    q[lane] = qq;
    int t = qq;
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) t += __shfl_xor(t, o, 64);
    if (lane == 0) {
        *s = d;
        *sum = t;
    }
}

// ------------------------------------------------------------------------
// Input staging (prologues).  Every workgroup builds the activation it needs
// in LDS.  ORDER 0 = rmsnorm_quantize_q8_0_scalar ((x*w)*inv, model.rs:5615);
// ORDER 1 = rmsnorm_scalar_into ((x*inv)*w, model.rs:7474) then quantize.
// ------------------------------------------------------------------------
enum Pro { PRO_LOADQ = 0, PRO_NORMQ0 = 1, PRO_NORMQ1 = 2 };

}  // namespace fl
#include "ess.h"
namespace fl {

// SEQ: the sum of squares in the reference's sequential order (ess_sumsq_wg
// with `ess` = kEssLdsWords + 1 floats of LDS, else the plain loop).
template <bool SEQ = false>
__device__ __forceinline__ float wg_inv_rms(const float *x, int n, float eps, float *red, float *ess = nullptr) {
    float ss = 0.0f;
    if (SEQ) {
        ss = ess ? ess_sumsq_wg(x, n, ess) : seq_sumsq(x, n);
    } else {
        for (int i = threadIdx.x; i < n; i += blockDim.x) ss += x[i] * x[i];
        ss = wg_sum(ss, red);
    }
    const float rms = sqrtf(ss / (float)n + eps);
    return 1.0f / rms;
}

template <int PRO, bool SEQ = false>
__device__ __forceinline__ void stage_q8(const float *x, const float *w, float eps, int n,
                                         const int8_t *gq, const float *gs, const int *gsum,
                                         int8_t *lq, float *ls, int *lsum, float *red, float *ess = nullptr) {
    const int nb = n >> 5;
    if (PRO == PRO_LOADQ) {
        const v4i_t *src = (const v4i_t *)gq;
        v4i_t *dst = (v4i_t *)lq;
        for (int i = threadIdx.x; i < (n >> 4); i += blockDim.x) dst[i] = src[i];
        for (int i = threadIdx.x; i < nb; i += blockDim.x) {
            ls[i] = gs[i];
            lsum[i] = gsum[i];
        }
    } else {
        // one element per lane; the 32 lanes of a half-wave form one block
        // (blockDim and n are multiples of 32), quantized by the lane quantizer
        const float inv = wg_inv_rms<SEQ>(x, n, eps, red, ess);
        for (int i = threadIdx.x; i < n; i += blockDim.x) {
            const float v = (PRO == PRO_NORMQ0) ? x[i] * w[i] * inv : (x[i] * inv) * w[i];
            quant_block32_lanes(v, lq + (i & ~31), ls + (i >> 5), lsum + (i >> 5));
        }
    }
    __syncthreads();
}

// A weight matrix on the device, in per-format planes (see mvs_kernels.h).
struct WDesc {
    const uint8_t *q;   // Q8_0: int8 quants; Q4_K: qs nibbles; Q6_K: ql; F32: floats
    const uint16_t *s;  // Q8_0: f16 block scales; Q6_K: f16 super-block d
    const uint8_t *h;   // Q4_K: 16-B headers (d, dmin, scales); Q6_K: qh
    const uint8_t *h2;  // Q6_K: int8 sub-block scales
    int rows, cols;
};

// Element i of row `row` of a Q4_K / Q6_K weight (dequant_q4k_block /
// dequant_q6k_block, flare-loader/src/quantize.rs:343-423).
__device__ __forceinline__ float q4k_elem(const WDesc &W, int row, int i) {
    const int nsb = W.cols >> 8, sb = i >> 8, e = i & 255, sblk = e >> 5, k = e & 31, ii = sblk & 3;
    const size_t rs = (size_t)row * nsb + sb;
    const uint8_t *hd = W.h + rs * 16;
    const float d = h2f((uint16_t)(hd[0] | (hd[1] << 8))), dmin = h2f((uint16_t)(hd[2] | (hd[3] << 8)));
    const uint8_t *s = hd + 4;
    uint32_t sc, mn;
    if (sblk < 4) {
        sc = s[ii] & 63;
        mn = s[ii + 4] & 63;
    } else {
        sc = (s[ii] >> 6) | ((s[ii + 8] & 0xF) << 2);
        mn = (s[ii + 4] >> 6) | ((s[ii + 8] >> 4) << 2);
    }
    const uint8_t qb = W.q[rs * 128 + 32 * ii + k];
    return d * (float)sc * (float)(sblk < 4 ? (qb & 0xF) : (qb >> 4)) - dmin * (float)mn;
}
__device__ __forceinline__ float q6k_elem(const WDesc &W, int row, int i) {
    const int nsb = W.cols >> 8, sb = i >> 8, e = i & 255, hf = e >> 7, r = e & 127, grp = r >> 5, l = r & 31;
    const size_t rs = (size_t)row * nsb + sb;
    const uint8_t *ql = W.q + rs * 128 + 64 * hf, *qh = W.h + rs * 64 + 32 * hf;
    const uint8_t la = ql[l], lb = ql[32 + l], hh = qh[l];
    int q;
    switch (grp) {
    case 0: q = (int)((la & 0xF) | ((hh & 3) << 4)) - 32; break;
    case 1: q = (int)((lb & 0xF) | (((hh >> 2) & 3) << 4)) - 32; break;
    case 2: q = (int)((la >> 4) | (((hh >> 4) & 3) << 4)) - 32; break;
    default: q = (int)((lb >> 4) | (((hh >> 6) & 3) << 4)) - 32; break;
    }
    const float sc = (float)(int8_t)W.h2[rs * 16 + hf * 8 + (l >> 4) + 2 * grp];
    return h2f(W.s[rs]) * sc * (float)q;
}

__device__ __forceinline__ uint32_t byte_of(uint32_t w, int i) { return (w >> (8 * i)) & 0xFFu; }

// 16-byte streaming loads (weights are read once per token: non-temporal hint)
__device__ __forceinline__ v4i_t ld_stream(const void *p) { return __builtin_nontemporal_load((const v4i_t *)p); }
__device__ __forceinline__ v4f_t ld_stream_f(const void *p) { return __builtin_nontemporal_load((const v4f_t *)p); }

// Packed (value, index) key whose unsigned max is the first maximum:
// order-preserving float bits in the high word, ~index in the low word.
__device__ __forceinline__ unsigned long long argmax_key(float v, uint32_t idx) {
    uint32_t u = __float_as_uint(v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)u << 32) | (unsigned long long)(0xFFFFFFFFu - idx);
}

}  // namespace fl
