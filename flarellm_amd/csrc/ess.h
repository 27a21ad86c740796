// Exact sequential sum of squares on one wave.
//
// The reference forms RMSNorm's sum of squares as a sequential f32 fold,
// `x.iter().map(|v| v * v).sum()` (flare-core/src/model.rs:5615, 7466):
// s_0 = t_0, s_i = fl(s_{i-1} + t_i) with t_i = fl(x_i * x_i) >= 0.  As a
// dependent chain of n adds that is n x 3.4 ns on MI355X (14 us at n = 4096).
// This routine returns the same bits from a mostly parallel computation.
//
// Why it works.  While s stays inside one binade [2^E, 2^(E+1)) the grid of
// f32 values there has spacing u = 2^(E-23), s is a multiple of u, and so
//   fl(s + t) = s + rne(t / u) * u        (t >= 0, s + t < 2^(E+1))
// unless t / u is exactly halfway between two integers (then the tie goes to
// the even neighbour and depends on s).  So the steps inside a binade add
// integers c_i = rne(t_i / u) to s's mantissa, which is associative.  Only
// the steps that leave the binade, and the ties, need the real f32 add.
//
// The algorithm.
//  1. An approximate prefix sum P (any order) predicts each element's binade:
//     element i spans [P_{i-1}, P_i]; it is "simple" when both ends lie in the
//     same normal binade E and t_i / u_E is no tie; otherwise it is an
//     "event".  Consecutive elements share their boundary values exactly, so
//     every run of simple elements uses one E: the E of the event that ends
//     the run.
//  2. Pieces of 16 elements whose ends share a binade, whose sum T is below
//     2^(E-1) and that hold no tie sum their c_i directly (6 ops per
//     element).  The other pieces ("slow") are gathered
//     into LDS and classified element by element, 16 lanes per piece.  The
//     first kEssFold pieces (where s crosses many binades) are folded
//     sequentially.
//  3. A short sequential chain walks the events in order: the pending integer
//     sum of the simple run before an event is added to s's bit pattern
//     (checked: s is in the predicted binade and its mantissa does not carry
//     out), then s = fl(s + t_event) is the reference's own add.
//  Any failed check or more than kEssSlowSlots slow pieces falls back to the
//  plain sequential loop, so the result is the reference's sum in every case; the checks make a wrong prediction
//  cost time, never bits.
//
// The elements are taken in the register layout of the decode matvecs: lane
// l holds piece (s, l) = x[1024 s + 16 l, +16) for s < SX, which is also the
// summation order (s major, then lane, then element).
#pragma once

// included by kernels.h after its helpers (v4f_t, seq_sumsq)
namespace fl {

constexpr int kEssFold = 2;        // leading pieces folded sequentially
constexpr int kEssSlowSlots = 24;  // slow pieces one pass can take
constexpr int kEssSlotWords = 20;  // t[16], Ps, Pn, Qx (u32), pad
// LDS of one wave's scratch (floats)
constexpr int kEssLdsWords = kEssSlowSlots * kEssSlotWords;

__device__ __forceinline__ uint32_t f_bits(float f) { return __float_as_uint(f); }
__device__ __forceinline__ float bits_f(uint32_t u) { return __uint_as_float(u); }

// Scans through ds_bpermute shuffles.  (A DPP form of these scans gave wrong
// sums on gfx950 in some instruction schedules and right ones in others; the
// shuffles have no such dependence.)
template <int W>
__device__ __forceinline__ float scan_f(float v, int lane) {
#pragma unroll
    for (int o = 1; o < W; o <<= 1) {
        const float n = __shfl_up(v, o, W);
        if ((lane & (W - 1)) >= o) v += n;
    }
    return v;
}
template <int W>
__device__ __forceinline__ uint32_t scan_u(uint32_t v, int lane) {
#pragma unroll
    for (int o = 1; o < W; o <<= 1) {
        const uint32_t n = __shfl_up(v, o, W);
        if ((lane & (W - 1)) >= o) v += n;
    }
    return v;
}
template <int W>
__device__ __forceinline__ uint32_t scan_max_u(uint32_t v, int lane) {
#pragma unroll
    for (int o = 1; o < W; o <<= 1) {
        const uint32_t n = __shfl_up(v, o, W);
        if ((lane & (W - 1)) >= o) v = max(v, n);
    }
    return v;
}
// lane i - 1's value within W-lane groups, 0 on a group's first lane
template <int W>
__device__ __forceinline__ float prev_f(float v, int lane) {
    const float n = __shfl_up(v, 1, W);
    return (lane & (W - 1)) ? n : 0.0f;
}
template <int W>
__device__ __forceinline__ uint32_t prev_u(uint32_t v, int lane) {
    const uint32_t n = __shfl_up(v, 1, W);
    return (lane & (W - 1)) ? n : 0u;
}

__device__ __forceinline__ float rd_lane(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
__device__ __forceinline__ uint32_t rd_lane_u(uint32_t v, int l) { return (uint32_t)__builtin_amdgcn_readlane((int)v, l); }

// Add the pending integer sum `cs` (units of the binade's spacing) to s, whose
// binade must be e; sets `bad` when the prediction does not hold.
__device__ __forceinline__ void ess_seg(float &s, uint32_t cs, uint32_t e, bool &bad) {
    if (cs == 0) return;
    const uint32_t sb = f_bits(s), es = sb >> 23;
    const uint32_t nb = sb + cs;
    if (es != e || es - 1u >= 254u || cs >= (1u << 24) || (nb >> 23) != es) bad = true;
    else s = bits_f(nb);
}

// The reference's sequential sum of t over the elements of the valid pieces
// (pieces with 1024 s + 16 l >= K hold t = 0 and are ignored).  `t` are the
// squares fl(x*x) of the lane's pieces; `lds` is this wave's kEssLdsWords
// floats; `x` (global) serves the sequential fallback.  Every lane returns
// the sum.  K must be a multiple of 16.
template <int SX>
__device__ float ess_sumsq(const float (&t)[SX][16], int K, int lane, float *lds, const float *x) {
    // 1. piece sums and the approximate exclusive prefix at piece boundaries
    float T[SX], Ps[SX], Pn[SX];
    bool slow[SX];
    float carry = 0.0f;
#pragma unroll
    for (int s = 0; s < SX; s++) {
        float a = 0.0f;
#pragma unroll
        for (int j = 0; j < 16; j++) a += t[s][j];
        T[s] = a;
        const float inc = scan_f<64>(a, lane);
        Ps[s] = carry + (inc - a);  // >= 0, exactly 0 on lane 0
        const float next_carry = carry + rd_lane(inc, 63);
        const float nb = __shfl_down(Ps[s], 1, 64);  // lane l + 1's value
        Pn[s] = lane < 63 ? nb : next_carry;
        carry = next_carry;
    }
    // 2. fast pieces: one binade, no element can tie
    bool bad = false;
    uint32_t Qx[SX];
    uint32_t qcarry = 0;
    int nslow = 0;
#pragma unroll
    for (int s = 0; s < SX; s++) {
        const bool valid = 1024 * s + 16 * lane < K && !(s == 0 && lane < kEssFold);
        const uint32_t eb = f_bits(Ps[s]) >> 23, ee = f_bits(Pn[s]) >> 23, et = f_bits(T[s]) >> 23;
        bool fast = valid && eb == ee && eb - 1u < 254u && et + 1u < eb;
        uint32_t a = 0;
        if (fast) {
            // t / u < 2^23 here (T < 2^(E-1)); a tie (fraction exactly 1/2)
            // sends the piece to the element-wise path, where it is an event
            const int k = 150 - (int)eb;
            bool tie = false;
#pragma unroll
            for (int j = 0; j < 16; j++) {
                const float y = ldexpf(t[s][j], k), r = rintf(y);
                tie = tie || fabsf(y - r) == 0.5f;
                a += (uint32_t)r;
            }
            if (tie) {
                fast = false;
                a = 0;
            }
        }
        slow[s] = valid && !fast;
        const uint32_t inc = scan_u<64>(a, lane);
        Qx[s] = qcarry + inc - a;  // contributions of the fast pieces before this one
        qcarry += rd_lane_u(inc, 63);
        nslow += __popcll(__ballot(slow[s]));
    }
    const uint32_t qtot = qcarry;
    if (nslow > kEssSlowSlots) bad = true;

    // 3. the folded leading pieces, sequentially (lanes 0 .. kEssFold-1 of s = 0)
    float S = 0.0f;
#pragma unroll
    for (int l = 0; l < kEssFold; l++)
#pragma unroll
        for (int j = 0; j < 16; j++) S = S + rd_lane(t[0][j], l);

    if (!bad) {
        // 4. gather the slow pieces into LDS slots, in order
        int base = 0;
#pragma unroll
        for (int s = 0; s < SX; s++) {
            const unsigned long long m = __ballot(slow[s]);
            if (slow[s]) {
                const int slot = base + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                                                       __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0));
                float *p = lds + slot * kEssSlotWords;
#pragma unroll
                for (int j = 0; j < 16; j++) p[j] = t[s][j];
                p[16] = Ps[s];
                p[17] = Pn[s];
                p[18] = __uint_as_float(Qx[s]);
            }
            base += __popcll(m);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

        // 5. slow pieces element by element (16 lanes per piece), then the
        //    sequential chain over their events
        uint32_t pend = 0, qlast = 0;
        const int j = lane & 15, row = lane >> 4;
        for (int it = 0; it * 4 < nslow; it++) {
            const int q = it * 4 + row;
            const bool live = q < nslow;
            const float *p = lds + min(q, kEssSlowSlots - 1) * kEssSlotWords;
            const float te = live ? p[j] : 0.0f;
            const float ps = p[16], pn = p[17];
            const uint32_t qx = __float_as_uint(p[18]);
            const float L = scan_f<16>(te, lane);
            const float Lex = prev_f<16>(L, lane);
            const float st = j == 0 ? ps : ps + Lex;
            const float en = j == 15 ? pn : ps + L;
            const uint32_t e = f_bits(st) >> 23;
            bool ev = e - 1u >= 254u || e != (f_bits(en) >> 23);
            const float y = ldexpf(te, 150 - (int)e);
            const float r = rintf(y);
            ev = ev || fabsf(y - r) == 0.5f || !(y < 16777216.0f);
            const uint32_t ce = ev ? 0u : (uint32_t)r;
            const uint32_t Qr = scan_u<16>(ce, lane);  // inclusive, within the piece
            const uint32_t Qprev = scan_max_u<16>(ev ? Qr : 0u, lane);
            const uint32_t Qpe = prev_u<16>(Qprev, lane);  // 0 on the piece's first lane
            const uint32_t before = Qr - Qpe;  // simple sum since the previous event (events: c = 0)
            const unsigned long long evm = __ballot(ev && live);
            // chain over this pass's pieces, in order (constant readlane lanes)
#pragma unroll
            for (int rr = 0; rr < 4; rr++) {
                const int qq = it * 4 + rr;
                if (qq < nslow) {
                    const int l0 = rr * 16;
                    pend += rd_lane_u(qx, l0) - qlast;  // fast pieces since the last slow piece
                    qlast = rd_lane_u(qx, l0);
                    const uint32_t m = (uint32_t)(evm >> l0) & 0xFFFFu;
#pragma unroll
                    for (int jj = 0; jj < 16; jj++) {
                        if (m & (1u << jj)) {
                            pend += rd_lane_u(before, l0 + jj);
                            ess_seg(S, pend, rd_lane_u(e, l0 + jj), bad);
                            pend = 0;
                            S = S + rd_lane(te, l0 + jj);
                        }
                    }
                    // the piece's simple tail after its last event
                    pend += rd_lane_u(Qr, l0 + 15) - rd_lane_u(Qprev, l0 + 15);
                }
            }
        }
        // 6. the final run: its binade is the one at the end boundary of the
        //    last valid piece (shared with the run's items)
        const int last = (K >> 4) - 1, s_last = last >> 6, l_last = last & 63;
        float pend_b = 0.0f;
#pragma unroll
        for (int s = 0; s < SX; s++)
            if (s == s_last) pend_b = __shfl(Pn[s], l_last, 64);  // (a bpermute: l_last is not constant)
        pend += qtot - qlast;
        ess_seg(S, pend, f_bits(pend_b) >> 23, bad);
    }
    if (bad) S = seq_sumsq(x, K);
    return S;
}

// Workgroup form for n <= 4096: wave 0 loads x in the piece layout and runs
// ess_sumsq while the other waves wait at the barrier.  `scratch` holds
// kEssLdsWords + 1 floats of LDS.  Every thread of the workgroup must call it.
__device__ __forceinline__ float ess_sumsq_wg(const float *x, int n, float *scratch) {
    if (n > 4096 || (n & 15)) return seq_sumsq(x, n);
    if (threadIdx.x < 64) {
        const int lane = threadIdx.x;
        float t[4][16];
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const int off = 1024 * s + 16 * lane;
            const bool ok = off < n;
            const int o = min(off, n - 16);
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const v4f_t v = *(const v4f_t *)(x + o + 4 * k);
                t[s][4 * k] = ok ? v.x * v.x : 0.0f;
                t[s][4 * k + 1] = ok ? v.y * v.y : 0.0f;
                t[s][4 * k + 2] = ok ? v.z * v.z : 0.0f;
                t[s][4 * k + 3] = ok ? v.w * v.w : 0.0f;
            }
        }
        const float S = ess_sumsq<4>(t, n, lane, scratch + 1, x);
        if (lane == 0) scratch[0] = S;
    }
    __syncthreads();
    const float S = scratch[0];
    __syncthreads();  // scratch may be reused by the caller
    return S;
}

}  // namespace fl
