// Reference-order kernels of the decode step (FL_OPT_EXACT).
//
// With FL_OPT_EXACT the decode step computes every floating-point value in
// the order of the x86-64 reference, so its logits are bit-identical to the
// CPU restatement.  The quantized matvecs are the streaming kernels of
// mvs_kernels.h with their SEQ instantiation (same tiles, loads, integer dots
// and per-block terms; row sums folded in block order).  Attention and the
// f32 output projection are sequential in the reference and get the kernels
// below: they are simple, not fast.
#include "launch.h"

namespace fl {

// grouped-query attention of one query head over slots 0..pos (model.rs:
// 9849-9905, fused_attention_head_scalar 9914-9966): scores
// (sum_d q k sequential) * (1/sqrt(D)), then the online softmax in token
// order.  One workgroup per query head; the scores go through `scores`.
template <bool F16>
__global__ __launch_bounds__(256) void k_attn_seq(SeqAttnArgs a) {
    const int h = blockIdx.x, kvh = h / a.group, D = a.D;
    const int T = *a.posp + 1;
    const float *qh = a.q + (size_t)h * D;
    float *sc = a.scores + (size_t)h * a.slots;
    const size_t hbase = (size_t)kvh * a.head_stride;
    const float scale = 1.0f / sqrtf((float)D);
    for (int t = threadIdx.x; t < T; t += blockDim.x) {
        float dot = 0.0f;
        for (int d = 0; d < D; d++) {
            const size_t o = hbase + (size_t)t * D + d;
            const float k = F16 ? h2f(((const uint16_t *)a.kc)[o]) : ((const float *)a.kc)[o];
            dot += qh[d] * k;
        }
        sc[t] = dot * scale;
    }
    __syncthreads();
    if ((int)threadIdx.x < D) {
        const int d = threadIdx.x;
        float m = -INFINITY, sum = 0.0f, o = 0.0f;
        for (int t = 0; t < T; t++) {
            const float s = sc[t];
            // F16 caches keep V in 32-slot transposed blocks [slot/32][D][32]
            const float v = F16 ? h2f(((const uint16_t *)a.vc)[hbase + ((size_t)(t >> 5) * D + d) * 32 + (t & 31)])
                                : ((const float *)a.vc)[hbase + (size_t)t * D + d];
            const float nm = fmaxf(m, s);
            const float old_scale = fl_expf(m - nm);
            const float w = fl_expf(s - nm);
            sum = sum * old_scale + w;
            o = o * old_scale + w * v;
            m = nm;
        }
        if (sum > 0.0f) {
            const float inv = 1.0f / sum;
            o *= inv;
        }
        a.out[(size_t)h * D + d] = o;
    }
}

// The same attention split in two kernels that keep the reference's order
// where it matters and run everything else in parallel.
//  k_attn_scores_exact: one lane per (slot, kv head) forms the G scores of
//    its slot, each dot summed over d in order, times 1/sqrt(D) (the lanes
//    of a wave read 64 consecutive K rows; q sits in LDS).
//  k_attn_chain_exact: one workgroup per query head.  The running maxima
//    m_t (a prefix max: exact in any order), the weights exp(s_t - m_t) and
//    the rescales exp(m_{t-1} - m_t) are formed in parallel into LDS; then
//    lane d walks o_d = o_d * old_t + w_t * v_td in token order and a second
//    wave walks sum = sum * old_t + w_t.  Between changes of the maximum the
//    rescale is exactly 1 and o * 1 = o, so 32-token blocks without a change
//    skip the multiply: one dependent add per token and lane.
template <bool F16, int DD>
__global__ __launch_bounds__(64) void k_attn_scores_exact(SeqAttnArgs a) {
    extern __shared__ float lq[];  // [G][D]
    const int kvh = blockIdx.y, G = a.group;
    constexpr int D = DD;
    const int T = *a.posp + 1;
    for (int i = threadIdx.x; i < G * D; i += blockDim.x) lq[i] = a.q[(size_t)kvh * G * D + i];
    __syncthreads();
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (F16 && blockIdx.x * 64 < T) {
        // the V blocks of these 64 slots, read once here so that the chain
        // kernel's V loads find them in the memory-side cache: up to 2 blocks
        // of [D][32] binary16 (4 D 16-byte pieces each), D / 8 pieces per lane
        const v4i_t *vb = (const v4i_t *)((const uint16_t *)a.vc + (size_t)kvh * a.head_stride +
                                           (size_t)blockIdx.x * 2 * D * 32);
        const int nb = min(2, (T - (int)blockIdx.x * 64 + 31) / 32);
        int acc = 0;
#pragma unroll
        for (int i = 0; i < D / 8; i++) {
            const int e = threadIdx.x + 64 * i;  // piece e of nb * D * 4 pieces
            if (e < nb * D * 4) acc ^= vb[e].x;
        }
        asm volatile("" ::"v"(acc));
    }
    if (t >= T) return;
    const size_t hbase = (size_t)kvh * a.head_stride + (size_t)t * D;
    const float scale = 1.0f / sqrtf((float)D);
    // the slot's whole K row, loaded up front
    float k[D];
    if (F16) {
#pragma unroll
        for (int d0 = 0; d0 < D; d0 += 8) {
            const v4i_t kv = *(const v4i_t *)((const uint16_t *)a.kc + hbase + d0);
#pragma unroll
            for (int e = 0; e < 8; e++) k[d0 + e] = h2f((uint16_t)((uint32_t)kv[e >> 1] >> (16 * (e & 1))));
        }
    } else {
#pragma unroll
        for (int d0 = 0; d0 < D; d0 += 4) {
            const v4f_t kv = *(const v4f_t *)((const float *)a.kc + hbase + d0);
#pragma unroll
            for (int e = 0; e < 4; e++) k[d0 + e] = kv[e];
        }
    }
    for (int g = 0; g < G; g++) {
        float acc = 0.0f;
#pragma unroll
        for (int d = 0; d < D; d++) acc += lq[g * D + d] * k[d];
        a.scores[(size_t)(kvh * G + g) * a.slots + t] = acc * scale;
    }
}

constexpr int kChainBlk = 32;
constexpr int kChainRing = 8;        // fp16 V blocks in flight per chain lane
constexpr int kChainThreads = 512;   // prologue parallelism; D chain lanes + the sum lane

// 32 fp16 V values of lane d for one 32-slot block ([slot/32][D][32] layout):
// value j in word j / 2 (q[j / 8][(j / 2) % 4]), half j % 2
struct VBlk {
    v4i_t q[4];
};

// the products w_t * v_t of one block, each one v_fma_mix (the exact binary16
// operand times w plus -0: rounded once, as (float)v * w); the weights in 8
// b128 LDS reads
__device__ __forceinline__ void chain_products(const VBlk &v, const float *w, float (&p)[kChainBlk]) {
    const v4f_t *wp = (const v4f_t *)w;
#pragma unroll
    for (int q = 0; q < kChainBlk / 4; q++) {
        const v4f_t wq = wp[q];
        const uint32_t w0 = (uint32_t)v.q[q >> 1][2 * (q & 1)], w1 = (uint32_t)v.q[q >> 1][2 * (q & 1) + 1];
        p[4 * q] = mul_h16lo(w0, wq.x);
        p[4 * q + 1] = mul_h16hi(w0, wq.y);
        p[4 * q + 2] = mul_h16lo(w1, wq.z);
        p[4 * q + 3] = mul_h16hi(w1, wq.w);
    }
}


template <bool F16>
__global__ __launch_bounds__(kChainThreads) void k_attn_chain_exact(SeqAttnArgs a) {
    extern __shared__ float sm[];  // w[slots] | old[slots] | flags[slots/32] | wave maxima[8] | sum
    __shared__ uint64_t etab[32];  // the exp table of fl_expf
    constexpr int NW = kChainThreads / 64;
    const int h = blockIdx.x, kvh = h / a.group, D = a.D;
    const int T = *a.posp + 1, nt = kChainThreads, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int nblk = (T + kChainBlk - 1) / kChainBlk;
    float *w = sm, *old = sm + a.slots;
    int *flag = (int *)(old + a.slots);
    float *wmax = (float *)(flag + (a.slots + kChainBlk - 1) / kChainBlk);
    float *ssum = wmax + NW;
    const size_t hb = (size_t)kvh * a.head_stride;
    // scores into LDS first (vector loads complete in order), flags cleared
    const float *sc = a.scores + (size_t)h * a.slots;
    for (int t = tid; t < T; t += nt) w[t] = sc[t];
    for (int b = tid; b < nblk; b += nt) flag[b] = 0;
    if (tid < 32) etab[tid] = kExp2Tab[tid];
    // then the chain lanes' first V blocks, in flight during the prologue
    VBlk ring[kChainRing];
    if (F16 && tid < D) {
#pragma unroll
        for (int r = 0; r < kChainRing; r++) {
            const v4i_t *p = (const v4i_t *)((const uint16_t *)a.vc + hb + ((size_t)min(r, nblk - 1) * D + tid) * 32);
#pragma unroll
            for (int i = 0; i < 4; i++) ring[r].q[i] = p[i];
        }
    }
    __syncthreads();
    // running maximum: contiguous chunks; exclusive max of the earlier chunks
    // by a wave scan and the wave maxima (max is exact in any order)
    const int C = (T + nt - 1) / nt, c0 = min(T, tid * C), c1 = min(T, c0 + C);
    float cm = -INFINITY;
    for (int t = c0; t < c1; t++) cm = fmaxf(cm, w[t]);
    float inc = cm;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const float n = __shfl_up(inc, o, 64);
        if (lane >= o) inc = fmaxf(inc, n);
    }
    if (lane == 63) wmax[wv] = inc;
    float m = __shfl_up(inc, 1, 64);
    if (lane == 0) m = -INFINITY;
    __syncthreads();
    for (int i = 0; i < wv; i++) m = fmaxf(m, wmax[i]);
    // the running maximum m_t of the chunk into old[] (a cheap serial pass),
    // then the weights exp(s_t - m_t) and rescales exp(m_{t-1} - m_t) as
    // independent iterations (table in LDS; exp(0) = 1 exactly); a block
    // with a rescale other than 1 is flagged
    const float m_in = m;
    for (int t = c0; t < c1; t++) {
        m = fmaxf(m, w[t]);
        old[t] = m;
    }
    float pm = m_in;
    for (int t = c0; t < c1; t++) {
        const float s = w[t], nm = old[t];
        w[t] = fl_expf_t(s - nm, etab);
        const float r = pm == nm ? 1.0f : fl_expf_t(pm - nm, etab);
        old[t] = r;
        if (r != 1.0f) flag[t / kChainBlk] = 1;
        pm = nm;
    }
    __syncthreads();
    if (tid < D) {
        float o = 0.0f;
        if (F16) {
            // per block: its 32 products first (independent), then the
            // dependent adds (between changes of the maximum the rescale is
            // exactly 1 and o * 1 = o: one dependent add per slot).  A wave64
            // VALU instruction holds the SIMD for 4 cycles, so the chain is
            // issue-bound (~26 cycles per slot measured with every schedule
            // tried: products interleaved with the adds, or formed a block
            // ahead; the V stream costs ~10 % of it).
            auto block = [&](int b, VBlk &slot) {
                const int t0 = b * kChainBlk, n = min(kChainBlk, T - t0);
                float p[kChainBlk];
                chain_products(slot, w + t0, p);
                // refill the slot with block b + kChainRing
                const v4i_t *q = (const v4i_t *)((const uint16_t *)a.vc + hb +
                                                 ((size_t)min(b + kChainRing, nblk - 1) * D + tid) * 32);
#pragma unroll
                for (int i = 0; i < 4; i++) slot.q[i] = q[i];
                if (n == kChainBlk && !flag[b]) {
#pragma unroll
                    for (int i = 0; i < kChainBlk; i++) o = o + p[i];
                } else {
#pragma unroll
                    for (int i = 0; i < kChainBlk; i++)
                        if (i < n) o = o * old[t0 + i] + p[i];
                }
            };
            // whole rounds of the ring without conditions (so the compiler's
            // wait counts stay exact: each slot waits for its own loads only),
            // then the remaining blocks
            int b0 = 0;
            for (; b0 + kChainRing <= nblk; b0 += kChainRing) {
#pragma unroll
                for (int r = 0; r < kChainRing; r++) block(b0 + r, ring[r]);
            }
#pragma unroll
            for (int r = 0; r < kChainRing; r++)
                if (b0 + r < nblk) block(b0 + r, ring[r]);
        } else {
            for (int b = 0; b < nblk; b++) {
                const int t0 = b * kChainBlk, n = min(kChainBlk, T - t0);
                float v[kChainBlk];
#pragma unroll
                for (int i = 0; i < kChainBlk; i++)
                    v[i] = ((const float *)a.vc)[hb + (size_t)min(t0 + i, T - 1) * D + tid];
                if (n == kChainBlk && !flag[b]) {
#pragma unroll
                    for (int i = 0; i < kChainBlk; i++) o = o + w[t0 + i] * v[i];
                } else {
#pragma unroll
                    for (int i = 0; i < kChainBlk; i++)
                        if (i < n) o = o * old[t0 + i] + w[t0 + i] * v[i];
                }
            }
        }
        __syncthreads();
        const float sum = *ssum;
        if (sum > 0.0f) {
            const float inv = 1.0f / sum;
            o *= inv;
        }
        a.out[(size_t)h * D + tid] = o;
    } else {
        if (tid == D) {
            // the weights' sum in the same order; the next block's weights
            // are read while this block's adds run
            float sum = 0.0f;
            v4f_t wq[kChainBlk / 4], wqn[kChainBlk / 4];
#pragma unroll
            for (int q = 0; q < kChainBlk / 4; q++) wq[q] = ((const v4f_t *)w)[q];
            for (int b = 0; b < nblk; b++) {
                const int t0 = b * kChainBlk, n = min(kChainBlk, T - t0);
                const v4f_t *wn = (const v4f_t *)(w + (size_t)min(b + 1, nblk) * kChainBlk);
#pragma unroll
                for (int q = 0; q < kChainBlk / 4; q++) wqn[q] = wn[q];
                if (n == kChainBlk && !flag[b]) {
#pragma unroll
                    for (int q = 0; q < kChainBlk / 4; q++) {
                        sum = sum + wq[q].x;
                        sum = sum + wq[q].y;
                        sum = sum + wq[q].z;
                        sum = sum + wq[q].w;
                    }
                } else {
                    for (int i = 0; i < n; i++) sum = sum * old[t0 + i] + w[t0 + i];
                }
#pragma unroll
                for (int q = 0; q < kChainBlk / 4; q++) wq[q] = wqn[q];
            }
            *ssum = sum;
        }
        __syncthreads();
    }
}

// rmsnorm_into (model.rs:7456-7477): (x * inv_rms) * w with the sequential
// sum of squares.  One workgroup.
__global__ __launch_bounds__(256) void k_rmsnorm_seq(const float *x, const float *w, int n, float eps, float *out) {
    __shared__ float ess[kEssLdsWords + 1];
    const float inv = wg_inv_rms<true>(x, n, eps, nullptr, ess);
    for (int i = threadIdx.x; i < n; i += blockDim.x) out[i] = (x[i] * inv) * w[i];
}

// Output projection over the dequantized weight with an f32 input, one row
// per thread: matvec_argmax_f32 (model.rs:8668-8689, sum += row[j] * vec[j]
// in order, first maximum) and, with `logits`, the matvec_into values.
// Weights dequantized as dequantize_tensor does (quantize.rs:189-197,
// 343-384).
template <int FMT>
__global__ __launch_bounds__(256) void k_out_seq(WDesc W, const float *xn, float *logits, unsigned long long *slot) {
    extern __shared__ float lx[];
    const int K = W.cols;
    for (int i = threadIdx.x; i < K; i += blockDim.x) lx[i] = xn[i];
    __syncthreads();
    const int row = blockIdx.x * blockDim.x + threadIdx.x;
    unsigned long long best = 0;
    if (row < W.rows) {
        float s = 0.0f;
        if (FMT == F_Q8_0) {
            const int nb = K >> 5;
            for (int b = 0; b < nb; b++) {
                const float scale = h2f(W.s[(size_t)row * nb + b]);
                const int8_t *q = (const int8_t *)W.q + (size_t)row * K + 32 * b;
                for (int k = 0; k < 32; k++) s += ((float)q[k] * scale) * lx[32 * b + k];
            }
        } else if (FMT == F_Q6K) {
            for (int j = 0; j < K; j++) s += q6k_elem(W, row, j) * lx[j];
        } else if (FMT == F_Q4K) {
            for (int j = 0; j < K; j++) s += q4k_elem(W, row, j) * lx[j];
        } else {
            const float *r = (const float *)W.q + (size_t)row * K;
            for (int j = 0; j < K; j++) s += r[j] * lx[j];
        }
        if (logits) logits[row] = s;
        best = argmax_key(s, (uint32_t)row);
    }
    if (!slot) return;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) best = umax64(best, __shfl_xor(best, o, 64));
    if ((threadIdx.x & 63) == 0 && best) atomicMax(slot, best);
}

// The same projection with one lane per row, streaming the quantized row
// from the device planes (Q8_0, Q6_K): the lane forms every dequantized
// weight as dequantize_tensor does -- Q8_0 q * d (exact), Q6_K (d * sc) * q --
// and adds w * x[j] in column order, so each row's sum is the reference's
// bit for bit.  x sits in LDS (broadcast reads); the row's next 32 (Q8_0) or
// 256 (Q6_K) weights are loaded while the current ones are consumed.  The
// time is the VALU work (about 5 operations per weight), not the stream.
template <int FMT>
__global__ __launch_bounds__(256) void k_out_exact(WDesc W, const float *xn, float *logits, unsigned long long *slot) {
    extern __shared__ float lx[];
    const int K = W.cols;
    for (int i = threadIdx.x; i < K; i += blockDim.x) lx[i] = xn[i];
    __syncthreads();
    const int row = min((int)(blockIdx.x * blockDim.x + threadIdx.x), W.rows - 1);
    float s = 0.0f;
    if constexpr (FMT == F_Q8_0) {
        const int nb = K >> 5;
        const v4i_t *q = (const v4i_t *)(W.q + (size_t)row * K);
        const uint16_t *sc = W.s + (size_t)row * nb;
        v4i_t a0 = q[0], a1 = q[1];
        uint16_t d0 = sc[0];
        for (int b = 0; b < nb; b++) {
            const int bn = min(b + 1, nb - 1);
            const v4i_t n0 = q[2 * bn], n1 = q[2 * bn + 1];
            const uint16_t dn = sc[bn];
            const float d = h2f(d0);
            const v4f_t *xb = (const v4f_t *)(lx + 32 * b);
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const v4i_t a = h ? a1 : a0;
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const v4f_t xv = xb[4 * h + k];
                    const uint32_t w4 = (uint32_t)a[k];
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const float w = (float)(int8_t)(w4 >> (8 * e)) * d;
                        s += w * xv[e];
                    }
                }
            }
            a0 = n0;
            a1 = n1;
            d0 = dn;
        }
    } else {  // Q6_K, llama.cpp layout (dequant_q6k_block)
        const int nsb = K >> 8;
        const size_t rb = (size_t)row * nsb;
        for (int sb = 0; sb < nsb; sb++) {
            const v4i_t *ql = (const v4i_t *)(W.q + (rb + sb) * 128);
            const v4i_t *qh = (const v4i_t *)(W.h + (rb + sb) * 64);
            const v4i_t scv = *(const v4i_t *)(W.h2 + (rb + sb) * 16);
            const float d = h2f(W.s[rb + sb]);
            v4i_t L[8], H[4];
#pragma unroll
            for (int i = 0; i < 8; i++) L[i] = ql[i];
#pragma unroll
            for (int i = 0; i < 4; i++) H[i] = qh[i];
            const float *xs = lx + 256 * sb;
#pragma unroll
            for (int hf = 0; hf < 2; hf++)
#pragma unroll
                for (int g = 0; g < 4; g++) {
#pragma unroll
                    for (int half16 = 0; half16 < 2; half16++) {
                        // scale of elements l = 16 * half16 .. +16 of group g
                        const int si = hf * 8 + half16 + 2 * g;
                        const float dsc = d * (float)(int8_t)((uint32_t)scv[si >> 2] >> (8 * (si & 3)));
#pragma unroll
                        for (int k = 0; k < 4; k++) {
                            const int l4 = half16 * 4 + k;  // dword of l = 4 * l4 .. + 4
                            const uint32_t lw = (uint32_t)L[hf * 4 + (g & 1) * 2 + (l4 >> 2)][l4 & 3];
                            const uint32_t hw = (uint32_t)H[hf * 2 + (l4 >> 2)][l4 & 3];
                            const uint32_t u = ((lw >> (4 * (g >> 1))) & 0x0F0F0F0Fu) | (((hw >> (2 * g)) & 0x03030303u) << 4);
                            const v4f_t xv = *(const v4f_t *)(xs + hf * 128 + g * 32 + 4 * l4);
#pragma unroll
                            for (int e = 0; e < 4; e++) {
                                const float q = (float)((int)((u >> (8 * e)) & 63u) - 32);
                                const float w = dsc * q;
                                s += w * xv[e];
                            }
                        }
                    }
                }
        }
    }
    const int r = blockIdx.x * blockDim.x + threadIdx.x;
    unsigned long long best = 0;
    if (r < W.rows) {
        if (logits) logits[r] = s;
        best = argmax_key(s, (uint32_t)r);
    }
    if (!slot) return;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) best = umax64(best, __shfl_xor(best, o, 64));
    if ((threadIdx.x & 63) == 0 && best) atomicMax(slot, best);
}

hipError_t launch_attn_seq(bool f16, hipStream_t st, const SeqAttnArgs &a0, int num_heads) {
    const SeqAttnArgs &a = a0;
    // w / old of every slot, the block flags, 8 wave maxima, the sum, and one
    // block of slack (the pipelined chain reads block nblk's weights, unused)
    const size_t chain_lds = (size_t)a.slots * 8 + (size_t)((a.slots + kChainBlk - 1) / kChainBlk) * 4 + 64 + kChainBlk * 4;
    // the chain kernel: whole waves of chain lanes (D a multiple of 64) plus
    // one wave for the sum, at most 4 waves; w / old of every slot in LDS
    if (a.group > 8 || (a.D != 64 && a.D != 128) || chain_lds > 64 * 1024) {
        // general shapes: the simple kernel
        if (f16) hipLaunchKernelGGL(k_attn_seq<true>, dim3(num_heads), dim3(256), 0, st, a);
        else hipLaunchKernelGGL(k_attn_seq<false>, dim3(num_heads), dim3(256), 0, st, a);
        return hipGetLastError();
    }
    const int nkv = num_heads / a.group;
    const dim3 sg((a.slots + 63) / 64, nkv);
    const size_t qlds = (size_t)a.group * a.D * 4;
    const int nt = kChainThreads;  // D chain lanes + the sum lane + prologue threads
    if (f16) {
        if (a.D == 64) hipLaunchKernelGGL((k_attn_scores_exact<true, 64>), sg, dim3(64), qlds, st, a);
        else hipLaunchKernelGGL((k_attn_scores_exact<true, 128>), sg, dim3(64), qlds, st, a);
        hipLaunchKernelGGL(k_attn_chain_exact<true>, dim3(num_heads), dim3(nt), chain_lds, st, a);
    } else {
        if (a.D == 64) hipLaunchKernelGGL((k_attn_scores_exact<false, 64>), sg, dim3(64), qlds, st, a);
        else hipLaunchKernelGGL((k_attn_scores_exact<false, 128>), sg, dim3(64), qlds, st, a);
        hipLaunchKernelGGL(k_attn_chain_exact<false>, dim3(num_heads), dim3(nt), chain_lds, st, a);
    }
    return hipGetLastError();
}

hipError_t launch_rmsnorm_seq(hipStream_t st, const float *x, const float *w, int n, float eps, float *out) {
    hipLaunchKernelGGL(k_rmsnorm_seq, dim3(1), dim3(256), 0, st, x, w, n, eps, out);
    return hipGetLastError();
}

hipError_t launch_out_seq(int fmt, hipStream_t st, const WDesc &W, const float *xn, float *logits,
                          unsigned long long *slot) {
    const dim3 grid((W.rows + 255) / 256);
    const size_t lds = (size_t)W.cols * 4;
    switch (fmt) {
    case F_Q8_0: hipLaunchKernelGGL(k_out_exact<F_Q8_0>, grid, dim3(256), lds, st, W, xn, logits, slot); break;
    case F_Q6K: hipLaunchKernelGGL(k_out_exact<F_Q6K>, grid, dim3(256), lds, st, W, xn, logits, slot); break;
    case F_Q4K: hipLaunchKernelGGL(k_out_seq<F_Q4K>, grid, dim3(256), lds, st, W, xn, logits, slot); break;
    case F_F32: hipLaunchKernelGGL(k_out_seq<F_F32>, grid, dim3(256), lds, st, W, xn, logits, slot); break;
    default: return hipErrorNotSupported;
    }
    return hipGetLastError();
}

}  // namespace fl
