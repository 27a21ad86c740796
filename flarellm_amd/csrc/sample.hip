// Token sampling on the device: flare-core/src/sampling.rs restated for one
// workgroup over the logits row (repeat penalty, temperature, softmax, then
// greedy / top-p / min-p / top-k), so the non-greedy path needs no logits
// readback.  Candidate sets of up to kSmallCands tokens are selected (radix
// select on the probability bits), ordered and walked in LDS; larger min-p /
// top-k sets are ordered by a device-wide radix sort and walked by a second
// kernel.
#include <hip/hip_runtime.h>
#include <hipcub/hipcub.hpp>

#include "kernels.h"
#include "sample_args.h"

namespace fl {

constexpr int kSampleThreads = 1024;
constexpr int kSmallCands = 2048;

namespace {

__device__ __forceinline__ float block_max(float v, float *red) {
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    __syncthreads();
    if (lane == 0) red[w] = v;
    __syncthreads();
    float t = red[0];
    for (int i = 1; i < kSampleThreads / 64; i++) t = fmaxf(t, red[i]);
    return t;
}

__device__ __forceinline__ int block_sum_int(int v, int *red) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    __syncthreads();
    if (lane == 0) red[w] = v;
    __syncthreads();
    int t = 0;
    for (int i = 0; i < kSampleThreads / 64; i++) t += red[i];
    return t;
}

// Exclusive rank of this thread's flag among the workgroup's set flags (in
// thread order); *total = number of set flags.
__device__ __forceinline__ int block_rank(bool f, int *wsum, int *total) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const unsigned long long bal = __ballot(f);
    const int r = __popcll(bal & ((1ull << lane) - 1ull));
    __syncthreads();
    if (lane == 0) wsum[w] = __popcll(bal);
    __syncthreads();
    int off = 0, tot = 0;
    for (int j = 0; j < kSampleThreads / 64; j++) {
        const int v = wsum[j];
        off += j < w ? v : 0;
        tot += v;
    }
    *total = tot;
    return off + r;
}

// Sequential walk of the reference over candidates ordered by descending
// probability (sample_top_p / sample_top_k / sample_min_p,
// sampling.rs:131-268): top-p cut, total, threshold u*total, first prefix
// reaching it.  Keys: probability bits << 32 | ~index.
__device__ int walk(const unsigned long long *key, int L, int mode, float top_p, float u) {
    auto prob = [&](int i) { return __uint_as_float((unsigned)(key[i] >> 32)); };
    auto index = [&](int i) { return (int)(0xFFFFFFFFu - (unsigned)(key[i] & 0xFFFFFFFFull)); };
    int cutoff = L;
    if (mode == SM_TOP_P) {
        float cum = 0.0f;
        for (int i = 0; i < L; i++) {
            cum += prob(i);
            if (cum >= top_p) {
                cutoff = i + 1;
                break;
            }
        }
    }
    float total = 0.0f;
    for (int i = 0; i < cutoff; i++) total += prob(i);
    const float thr = u * total;
    float acc = 0.0f;
    for (int i = 0; i < cutoff; i++) {
        acc += prob(i);
        if (acc >= thr) return index(i);
    }
    return index(cutoff - 1);
}

}  // namespace

__global__ __launch_bounds__(kSampleThreads) void k_sample(SampleArgs a) {
    __shared__ float redf[kSampleThreads / 64];
    __shared__ int redi[kSampleThreads / 64];
    __shared__ int wsum[kSampleThreads / 64];
    __shared__ int hist[256];
    __shared__ unsigned sel_prefix;
    __shared__ int sel_remaining;
    __shared__ unsigned long long cand[kSmallCands];
    const int tid = threadIdx.x, n = a.n;
    float *p = a.p;
    // ---- apply_repeat_penalty (sampling.rs:83-96): once per occurrence --------
    for (int i = tid; i < n; i += kSampleThreads) p[i] = a.logits[i];
    if (a.penalty != 1.0f && a.n_prev > 0) {
        __syncthreads();
        for (int j = tid; j < a.n_prev; j += kSampleThreads) {
            const int t = a.prev[j];
            if (t >= 0 && t < n) atomicAdd(&a.counts[t], 1);
        }
        __syncthreads();
        for (int j = tid; j < a.n_prev; j += kSampleThreads) {
            const int t = a.prev[j];
            if (t < 0 || t >= n) continue;
            const int c = atomicExch(&a.counts[t], 0);  // the first occurrence takes the count
            if (c > 0) {
                float v = p[t];
                for (int r = 0; r < c; r++) v = v > 0.0f ? v / a.penalty : v * a.penalty;
                p[t] = v;
            }
        }
    }
    __syncthreads();
    // ---- apply_temperature (sampling.rs:73-81), max and first-max argmax ------
    const bool scale = a.temperature != 0.0f && a.temperature != 1.0f;
    const float inv_temp = 1.0f / a.temperature;
    float mx = -INFINITY;
    int mi = 0x7FFFFFFF;
    for (int i = tid; i < n; i += kSampleThreads) {
        float v = p[i];
        if (scale) {
            v *= inv_temp;
            p[i] = v;
        }
        if (v > mx) {  // strictly greater: this thread's first maximum
            mx = v;
            mi = i;
        }
    }
    const float gmax = block_max(mx, redf);
    // first index holding the maximum (sample_greedy, sampling.rs:101-111)
    {
        int cand_i = (mx == gmax) ? mi : 0x7FFFFFFF;
        for (int o = 32; o > 0; o >>= 1) cand_i = min(cand_i, __shfl_xor(cand_i, o));
        __syncthreads();
        if ((tid & 63) == 0) redi[tid >> 6] = cand_i;
        __syncthreads();
        int best = redi[0];
        for (int i = 1; i < kSampleThreads / 64; i++) best = min(best, redi[i]);
        if (a.mode == SM_GREEDY) {
            if (tid == 0) a.state[0] = best == 0x7FFFFFFF ? 0 : best;
            return;
        }
        if (tid == 0) a.state[3] = best == 0x7FFFFFFF ? 0 : best;
    }
    // ---- softmax: exps, their sum, probabilities -----------------------------
    float part = 0.0f;
    for (int i = tid; i < n; i += kSampleThreads) {
        const float e = fl_expf(p[i] - gmax);
        p[i] = e;
        part += e;
    }
    __syncthreads();
    float sum;
    if (a.exact) {
        // the reference's sequential fold (exps.iter().sum())
        if (tid == 0) {
            float s = 0.0f;
            for (int i = 0; i < n; i++) s += p[i];
            redf[0] = s;
        }
        __syncthreads();
        sum = redf[0];
        __syncthreads();
    } else {
        sum = wg_sum(part, redf);
    }
    const float inv_sum = 1.0f / sum;
    float pmax = 0.0f;
    for (int i = tid; i < n; i += kSampleThreads) {
        // sample_top_p / sample_top_k: e * inv_sum; softmax() (min-p): e / sum
        const float q = a.mode == SM_MIN_P ? p[i] / sum : p[i] * inv_sum;
        p[i] = q;
        pmax = fmaxf(pmax, q);
    }
    __syncthreads();
    // ---- candidate set -----------------------------------------------------
    int K;                 // candidates to take
    unsigned kth = 0;      // smallest candidate key (K-limited modes)
    int need_eq = 0;       // how many keys equal to kth are taken
    float thr = 0.0f;      // min-p threshold
    if (a.mode == SM_MIN_P) {
        const float gpmax = block_max(pmax, redf);
        thr = a.min_p * gpmax;
        int c = 0;
        for (int i = tid; i < n; i += kSampleThreads) c += p[i] >= thr;
        K = block_sum_int(c, redi);
        if (K == 0) {  // no candidate: the greedy token (sampling.rs:233-236)
            if (tid == 0) a.state[0] = a.state[3];
            return;
        }
    } else {
        K = min(a.K, n);
        // radix select of the K-th largest probability (bits of p >= 0 order as unsigned)
        if (tid == 0) {
            sel_prefix = 0;
            sel_remaining = K;
        }
        unsigned mask = 0;
        for (int shift = 24; shift >= 0; shift -= 8) {
            for (int i = tid; i < 256; i += kSampleThreads) hist[i] = 0;
            __syncthreads();
            const unsigned pre = sel_prefix;
            for (int i = tid; i < n; i += kSampleThreads) {
                const unsigned b = __float_as_uint(p[i]);
                if ((b & mask) == pre) atomicAdd(&hist[(b >> shift) & 255], 1);
            }
            __syncthreads();
            if (tid == 0) {
                int cum = 0, rem = sel_remaining, d = 255;
                for (; d > 0; d--) {
                    if (cum + hist[d] >= rem) break;
                    cum += hist[d];
                }
                sel_prefix = pre | ((unsigned)d << shift);
                sel_remaining = rem - cum;
            }
            mask |= 255u << shift;
            __syncthreads();
        }
        kth = sel_prefix;
        need_eq = sel_remaining;
    }
    if (K > kSmallCands) {
        // large set: sort keys for the device-wide sort; non-candidates get
        // key 0 and sort last
        for (int i = tid; i < n; i += kSampleThreads) {
            const unsigned b = __float_as_uint(p[i]);
            const bool take = a.mode == SM_MIN_P ? p[i] >= thr : b >= kth;
            a.keys[i] = take ? b : 0u;
            a.vals[i] = i;
        }
        if (tid == 0) {
            a.state[1] = K;
            a.state[2] = 1;
        }
        return;
    }
    // ---- small set: ordered compaction into LDS --------------------------------
    int taken = 0, eq_taken = 0;
    for (int base = 0; base < n; base += kSampleThreads) {
        const int i = base + tid;
        const float q = i < n ? p[i] : 0.0f;
        const unsigned b = __float_as_uint(q);
        bool take;
        if (a.mode == SM_MIN_P) {
            take = i < n && q >= thr;
        } else {
            const bool eq = i < n && b == kth;
            int eq_tot;
            const int er = block_rank(eq, wsum, &eq_tot);
            take = i < n && (b > kth || (eq && eq_taken + er < need_eq));
            eq_taken += eq_tot;
        }
        int tot;
        const int r = block_rank(take, wsum, &tot);
        if (take && taken + r < kSmallCands)
            cand[taken + r] = ((unsigned long long)b << 32) | (unsigned long long)(0xFFFFFFFFu - (unsigned)i);
        taken += tot;
    }
    const int L = min(taken, kSmallCands);
    int S = 2;
    while (S < L) S <<= 1;
    for (int i = L + tid; i < S; i += kSampleThreads) cand[i] = 0ull;
    __syncthreads();
    // bitonic sort, descending: probability, then ascending index
    for (int k = 2; k <= S; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = tid; i < S; i += kSampleThreads) {
                const int ixj = i ^ j;
                if (ixj > i) {
                    const unsigned long long x = cand[i], y = cand[ixj];
                    const bool desc = (i & k) == 0;
                    if (desc ? (x < y) : (x > y)) {
                        cand[i] = y;
                        cand[ixj] = x;
                    }
                }
            }
            __syncthreads();
        }
    }
    if (tid == 0) {
        a.state[0] = walk(cand, L, a.mode, a.top_p, a.u);
        a.state[2] = 0;
    }
}

// Walk of a large candidate set after the device-wide sort (descending keys,
// ties in index order: the sort is stable).  Sums in the reference's
// sequential order when exact, else per-thread chunks combined in order.
__global__ __launch_bounds__(kSampleThreads) void k_sample_walk(SampleArgs a) {
    __shared__ float chunk_sum[kSampleThreads];
    __shared__ float pref[kSampleThreads + 1];
    if (a.state[2] != 1) return;
    const int L = a.state[1], tid = threadIdx.x;
    auto prob = [&](int i) { return __uint_as_float(a.skeys[i]); };
    if (a.exact) {
        if (tid == 0) {
            float total = 0.0f;
            for (int i = 0; i < L; i++) total += prob(i);
            const float thr = a.u * total;
            float acc = 0.0f;
            int out = a.svals[L - 1];
            for (int i = 0; i < L; i++) {
                acc += prob(i);
                if (acc >= thr) {
                    out = a.svals[i];
                    break;
                }
            }
            a.state[0] = out;
        }
        return;
    }
    const int per = (L + kSampleThreads - 1) / kSampleThreads;
    const int c0 = min(L, tid * per), c1 = min(L, c0 + per);
    float s = 0.0f;
    for (int i = c0; i < c1; i++) s += prob(i);
    chunk_sum[tid] = s;
    __syncthreads();
    if (tid == 0) {
        float acc = 0.0f;
        for (int t = 0; t < kSampleThreads; t++) {
            pref[t] = acc;
            acc += chunk_sum[t];
        }
        pref[kSampleThreads] = acc;
    }
    __syncthreads();
    const float thr = a.u * pref[kSampleThreads];
    // the chunk in which the running sum first reaches thr
    const bool here = c0 < c1 && pref[tid] + chunk_sum[tid] >= thr && (tid == 0 || pref[tid] < thr);
    if (here) {
        float acc = pref[tid];
        int out = a.svals[c1 - 1];
        for (int i = c0; i < c1; i++) {
            acc += prob(i);
            if (acc >= thr) {
                out = a.svals[i];
                break;
            }
        }
        a.state[0] = out;
    }
    __syncthreads();
    if (tid == 0 && !(pref[kSampleThreads] >= thr)) a.state[0] = a.svals[L - 1];
}

// Workspace bytes of the device-wide sort for n keys.
size_t sample_sort_bytes(int n) {
    size_t bytes = 0;
    (void)hipcub::DeviceRadixSort::SortPairsDescending(nullptr, bytes, (const unsigned *)nullptr, (unsigned *)nullptr,
                                                       (const int *)nullptr, (int *)nullptr, n);
    return bytes;
}

hipError_t launch_sample(hipStream_t st, const SampleArgs &a, void *sort_tmp, size_t sort_bytes) {
    if (a.n < 1 || a.K < 1) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_sample, dim3(1), dim3(kSampleThreads), 0, st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const bool large = (a.mode == SM_MIN_P) || (a.mode == SM_TOP_K && a.K > kSmallCands);
    if (!large) return hipSuccess;
    size_t bytes = sort_bytes;
    e = hipcub::DeviceRadixSort::SortPairsDescending(sort_tmp, bytes, a.keys, const_cast<unsigned *>(a.skeys),
                                                     a.vals, const_cast<int *>(a.svals), a.n, 0, 32, st);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_sample_walk, dim3(1), dim3(kSampleThreads), 0, st, a);
    return hipGetLastError();
}

}  // namespace fl
