// Shared pieces of the matvec kernels: epilogue codes and helpers, the
// activation prologues (stage x into LDS: copy, RMSNorm, Q8_0 quantization)
// and trace macros.  The kernels themselves are in mvs_kernels.h.
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
    const float *rope_cur;  // RoPE cos [D/2] then sin [D/2] of the step's position (k_embed writes them)
    const int *posp;    // token position (device)
    void *kc, *vc;      // this layer's head-major cache [kv_head][slot][D]
    long long head_stride;  // elements between kv heads (max_seq * D)
    int nq, nk;         // q rows (Nq*D) and k rows (Nkv*D); v rows follow
    int hd;             // head_dim
    int kv_f16;         // cache element: 1 = binary16 (RNE), 0 = f32
    int kv_stage;       // 1: K (after RoPE) and V go to the output after q, as f32
    int v_tblk;         // 1: V stored in 32-slot transposed blocks [slot/32][D][32]
    // 1 (fused QKV + attention launch): q, and K (after RoPE) / V as f32
    // after q, are stored with agent-scope stores for the attention
    // workgroups of the same launch; the cache rows are written as usual
    int publish;
};

#ifdef FLARE_MV_TRACE
#define MV_TS(i)                                                                          \
    do {                                                                                  \
        if (a.trace && blockIdx.x == 0 && threadIdx.x == 0)                              \
            a.trace[i] = (long long)__builtin_amdgcn_s_memrealtime();                     \
    } while (0)
// per-workgroup start / end (trace[64 + 2b], trace[65 + 2b])
#define MV_TSB(i)                                                                         \
    do {                                                                                  \
        if (a.trace && threadIdx.x == 0 && blockIdx.x < 1024)                            \
            a.trace[64 + 2 * blockIdx.x + (i)] = (long long)__builtin_amdgcn_s_memrealtime(); \
        if (a.trace && threadIdx.x == 0 && blockIdx.x < 1024 && (i) == 0)                \
            a.trace[64 + 2048 + blockIdx.x] = ((long long)__builtin_amdgcn_s_getreg((20 << 0) | (0 << 6) | (3 << 11)) << 32) | \
                (long long)__builtin_amdgcn_s_getreg((4 << 0) | (0 << 6) | (31 << 11)); \
    } while (0)
#define ST_TS(i)                                                                          \
    do {                                                                                  \
        if (tr && blockIdx.x == 0 && threadIdx.x == 0)                                    \
            tr[i] = (long long)__builtin_amdgcn_s_memrealtime();                          \
    } while (0)
#else
#define ST_TS(i) \
    do {         \
    } while (0)
#define MV_TS(i) \
    do {         \
    } while (0)
#define MV_TSB(i) \
    do {          \
    } while (0)
#endif

// ---------------------------------------------------------------------------
// Two-phase activation prologue.  Phase 1 (issue) loads this thread's share
// of the input into registers; phase 2 (finish) computes and writes LDS.
// NT = threads of the workgroup; E = elements per thread of the norm input
// (n == NT*E with E in {8, 16}); other n take the generic loop of stage_q8.
// ---------------------------------------------------------------------------
// SEQ: the sum of squares in the reference's sequential order.
// VT <= NT: only threads [0, VT) stage (the decomposition of a VT-thread
// workgroup, so the sums are those of that kernel); the others only join
// the barriers.
template <int NT, bool SEQ = false, int VT = NT>
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
        if (VT < NT && t >= VT) return;
        if (pro == PRO_LOADQ) {
            const int n16 = n >> 4, nb = n >> 5;
#pragma unroll
            for (int k = 0; k < 4; k++) qv[k] = ((const v4i_t *)gq)[min(t + k * VT, n16 - 1)];
#pragma unroll
            for (int k = 0; k < 2; k++) {
                const int j = min(t + k * VT, nb - 1);
                sv[k] = gs[j];
                sumv[k] = gsum[j];
            }
        } else {
            const int E = n / VT;
            if (n == VT * E && (E == 8 || E == 16)) {
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
                                           int8_t *lq, float *ls, int *lsum, float *red, long long *tr = nullptr,
                                           float *ess = nullptr) {
        const int t = threadIdx.x;
        const bool act = VT == NT || t < VT;
        ST_TS(7);
        if (pro == PRO_LOADQ) {
            const int n16 = n >> 4, nb = n >> 5;
            if (act) {
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const int i = t + k * VT;
                    if (i < n16) ((v4i_t *)lq)[i] = qv[k];
                }
#pragma unroll
                for (int k = 0; k < 2; k++) {
                    const int j = t + k * VT;
                    if (j < nb) {
                        ls[j] = sv[k];
                        lsum[j] = sumv[k];
                    }
                }
            }
            __syncthreads();
            return;
        }
        const int E = n / VT;
        if (!(n == VT * E && (E == 8 || E == 16))) {
            if (pro == PRO_NORMQ0) stage_q8<PRO_NORMQ0, SEQ>(x, w, eps, n, nullptr, nullptr, nullptr, lq, ls, lsum, red, ess);
            else stage_q8<PRO_NORMQ1, SEQ>(x, w, eps, n, nullptr, nullptr, nullptr, lq, ls, lsum, red, ess);
            return;
        }
        // E (8 or 16) as a compile-time constant: no per-element guards
        auto body = [&](auto ec) {
            constexpr int EC = decltype(ec)::value;
            float xs[EC], ws[EC];
#pragma unroll
            for (int k = 0; k < EC / 4; k++) {
                xs[4 * k] = xv[k].x; xs[4 * k + 1] = xv[k].y; xs[4 * k + 2] = xv[k].z; xs[4 * k + 3] = xv[k].w;
                ws[4 * k] = wv[k].x; ws[4 * k + 1] = wv[k].y; ws[4 * k + 2] = wv[k].z; ws[4 * k + 3] = wv[k].w;
            }
            // sum of squares: per-thread sequential, then the workgroup tree
            float ss = 0.0f;
#pragma unroll
            for (int j = 0; j < EC; j++) ss += xs[j] * xs[j];
            if (!act) ss = 0.0f;
            ST_TS(8);
            if (SEQ) ss = ess ? ess_sumsq_wg(x, n, ess) : seq_sumsq(x, n);
            else ss = wg_sum<VT>(ss, red);  // the first VT / 64 waves' sums
            ST_TS(9);
            const float rms = sqrtf(ss / (float)n + eps);
            const float inv = 1.0f / rms;
            float v[EC];
            // rmsnorm_quantize_q8_0_scalar (x*w)*inv (model.rs:5615) or
            // rmsnorm_scalar_into (x*inv)*w (model.rs:7474): one branch on the
            // uniform prologue kind
            if (pro == PRO_NORMQ0) {
#pragma unroll
                for (int j = 0; j < EC; j++) v[j] = xs[j] * ws[j] * inv;
            } else {
#pragma unroll
                for (int j = 0; j < EC; j++) v[j] = (xs[j] * inv) * ws[j];
            }
            float amax = 0.0f;
#pragma unroll
            for (int j = 0; j < EC; j++) amax = fmaxf(amax, fabsf(v[j]));
            // a 32-block spans 32/E consecutive lanes of one row
            if (EC == 8) amax = row_max<4>(amax);
            else amax = row_max<2>(amax);
            const float d = amax / 127.0f;
            const float id = (d != 0.0f) ? 127.0f / amax : 0.0f;
            int qsum = 0;
            uint32_t packed[EC / 4];
#pragma unroll
            for (int k = 0; k < EC / 4; k++) packed[k] = 0;
#pragma unroll
            for (int j = 0; j < EC; j++) {
                const int8_t qq = q8_code(v[j] * id);
                qsum += qq;
                packed[j >> 2] |= (uint32_t)(uint8_t)qq << (8 * (j & 3));
            }
            if constexpr (EC == 8) {
                qsum += __builtin_amdgcn_update_dpp(0, qsum, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
                qsum += __builtin_amdgcn_update_dpp(0, qsum, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
                if (act) {
                    ((v2i_t *)lq)[t] = v2i_t{(int)packed[0], (int)packed[1]};
                    if ((t & 3) == 0) {
                        ls[t >> 2] = d;
                        lsum[t >> 2] = qsum;
                    }
                }
            } else {
                qsum += __builtin_amdgcn_update_dpp(0, qsum, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
                if (act) {
                    ((v4i_t *)lq)[t] = v4i_t{(int)packed[0], (int)packed[1], (int)packed[2], (int)packed[3]};
                    if ((t & 1) == 0) {
                        ls[t >> 1] = d;
                        lsum[t >> 1] = qsum;
                    }
                }
            }
        };
        if (E == 8) body(std::integral_constant<int, 8>{});
        else body(std::integral_constant<int, 16>{});
        ST_TS(10);
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
            ss = wg_sum<NT>(ss, red);
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

// Stores of a finished row group (every lane holds all R row sums; lane 0
// writes them: a per-lane select of acc[lane] would become a dynamically
// indexed private array).
template <int R>
__device__ __forceinline__ void store_rows(const float *acc, int row0, int rows, int gl, int epi, float *out) {
    if (gl != 0) return;
#pragma unroll
    for (int r = 0; r < R; r++) {
        if (row0 + r < rows) {
            if (epi == EPI_ADD) out[row0 + r] += acc[r];  // residual add (model.rs:2305-2311, 2537-2543)
            else out[row0 + r] = acc[r];
        }
    }
}

// Lane r's row of a finished group (every lane holds all R sums), formed by
// adding masked terms: a select chain here was turned back into a private
// array indexed by the lane (scratch stores on every group).
template <int R>
__device__ __forceinline__ float lane_row(const float *acc, int gl) {
    float v = 0.0f;
#pragma unroll
    for (int r = 0; r < R; r++) v += gl == r ? acc[r] : 0.0f;
    return v;
}

// RoPE (cos, sin) of the pair that lane p < R/2 stores for rows n = row0 + 2p
// (q and k rows only).
__device__ __forceinline__ void qkv_rope_cs(const QkvEpi &e, int n, float &c, float &sn) {
    const int half = e.hd >> 1, i = (n % e.hd) >> 1;
    c = e.rope_cur[i];
    sn = e.rope_cur[half + i];
}

// EPI_QKV store of one rotate-half pair (rows n, n+1 in the pair-interleaved
// order of the fused QKV weight); (c, sn) = qkv_rope_cs of the pair.
__device__ __forceinline__ void store_qkv_pair(float x0, float x1, int n, const QkvEpi &e, int pos, float *q,
                                               float c, float sn) {
    const int D = e.hd, half = D >> 1;
    const int j = n % D, i = j >> 1;  // pair index within the head
    if (n < e.nq + e.nk) {
        const float y0 = x0 * c - x1 * sn, y1 = x0 * sn + x1 * c;
        if (n < e.nq) {
            const int h = n / D;
            if (e.publish) {
                st_agent(q + h * D + i, y0);
                st_agent(q + h * D + i + half, y1);
                return;
            }
            q[h * D + i] = y0;
            q[h * D + i + half] = y1;
        } else if (e.kv_stage) {
            const int k0 = (n - e.nq) - j;  // start of this kv head's row
            q[e.nq + k0 + i] = y0;
            q[e.nq + k0 + i + half] = y1;
        } else {
            const int kvh = (n - e.nq) / D;
            if (e.publish) {
                const int k0 = (n - e.nq) - j;
                st_agent(q + e.nq + k0 + i, y0);
                st_agent(q + e.nq + k0 + i + half, y1);
            }
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
        if (e.publish) {
            st_agent(q + e.nq + e.nk + vi, x0);
            st_agent(q + e.nq + e.nk + vi + 1, x1);
        }
        if (e.kv_stage) {
            q[e.nq + e.nk + vi] = x0;
            q[e.nq + e.nk + vi + 1] = x1;
            return;
        }
        if (e.v_tblk) {  // channels d, d+1 of slot pos: 32 elements apart
            const size_t o = (size_t)kvh * e.head_stride + ((size_t)(pos >> 5) * D + d) * 32 + (pos & 31);
            ((uint16_t *)e.vc)[o] = f2h(x0);
            ((uint16_t *)e.vc)[o + 32] = f2h(x1);
            return;
        }
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

// EPI_QKV store of a finished row group (R even); lane p < R/2 stores pair p.
// pre: lane p's (cos, sin) already loaded (pre_ok), else loaded here
template <int R>
__device__ __forceinline__ void store_qkv(const float *acc, int row0, int rows, int gl, const QkvEpi &e, int pos,
                                          float *q, bool pre_ok, float pc, float ps) {
    static_assert(R % 2 == 0, "EPI_QKV needs row pairs");
    // lane p < R/2 stores pair p: select its two rows first (constant
    // indices only), then one store path
    float x0 = acc[0], x1 = acc[1];
#pragma unroll
    for (int p = 1; p < R / 2; p++)
        if (gl == p) {
            x0 = acc[2 * p];
            x1 = acc[2 * p + 1];
        }
    if (gl < R / 2 && row0 + 2 * gl < rows) {
        const int n = row0 + 2 * gl;
        float c = pc, sn = ps;
        if (!pre_ok && n < e.nq + e.nk) qkv_rope_cs(e, n, c, sn);
        store_qkv_pair(x0, x1, n, e, pos, q, c, sn);
    }
}

}  // namespace fl
