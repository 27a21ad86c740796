// Decode attention launchers and the Q8 / KIVI cache writers.
#include "attm_kernels.h"
#include "attq_kernels.h"
#include "launch.h"

namespace fl {

template <typename KT>
static hipError_t launch_attn_t(int D, int G, hipStream_t st, const AttnArgs &a, int nq) {
#define C(DD, GG)                                                                                  \
    if (D == DD && G == GG) {                                                                      \
        hipLaunchKernelGGL((k_attn<KT, DD, GG>), dim3(a.nsplit, a.nkv, nq), dim3(kAttnThreads), 0, st, a); \
        return hipSuccess;                                                                         \
    }
    C(64, 1) C(64, 2) C(64, 3) C(64, 4) C(64, 8)
    C(128, 1) C(128, 2) C(128, 3) C(128, 4) C(128, 8)
#undef C
    return hipErrorNotSupported;
}

template <typename KT>
static hipError_t launch_attm_t(int D, int G, hipStream_t st, const AttnArgs &a, int nq) {
#define C(DD, GG)                                                                                  \
    if (D == DD && G == GG) {                                                                      \
        if (a.waves == 4)                                                                          \
            hipLaunchKernelGGL((k_attm<KT, DD, GG, 256>), dim3(a.nsplit, a.nkv, nq), dim3(256), 0, st, a); \
        else                                                                                       \
            hipLaunchKernelGGL((k_attm<KT, DD, GG>), dim3(a.nsplit, a.nkv, nq), dim3(kAttmThreads), 0, st, a); \
        return hipSuccess;                                                                         \
    }
    C(64, 1) C(64, 2) C(64, 3) C(64, 4) C(64, 8)
    C(128, 1) C(128, 2) C(128, 3) C(128, 4) C(128, 8)
#undef C
    return hipErrorNotSupported;
}

template <typename KT>
static int attm_resident_t(int D, int G, int waves) {
    int n = 0;
#define C(DD, GG)                                                                                       \
    if (D == DD && G == GG) {                                                                           \
        if (waves == 4)                                                                                 \
            (void)hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k_attm<KT, DD, GG, 256>, 256, 0);     \
        else                                                                                            \
            (void)hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k_attm<KT, DD, GG>, kAttmThreads, 0); \
        return n;                                                                                       \
    }
    C(64, 1) C(64, 2) C(64, 3) C(64, 4) C(64, 8)
    C(128, 1) C(128, 2) C(128, 3) C(128, 4) C(128, 8)
#undef C
    return 0;
}

int attm_resident_per_cu(int kvfmt, int D, int G, int waves) {
    if (kvfmt == KV_F16) return attm_resident_t<__half>(D, G, waves);
    if (kvfmt == KV_Q8) return attm_resident_t<KvQ8>(D, G, waves);
    if (kvfmt == KV_KIVI) return attm_resident_t<KvKivi>(D, G, waves);
    return 0;
}

// Several queries over an fp16 cache (V in transposed blocks): query pairs
// in groups of NW per workgroup (4 or 8 waves), K/V blocks shared in LDS.
hipError_t launch_attq(int D, int G, hipStream_t st, const AttnArgs &a) {
    const int npairs = a.nq / 2;
    if (a.nq < 2 || a.nq % 2 || !a.v_tblk || a.nsplit < 1 || a.nsplit > kAttmMaxSplit || a.S % 32 || a.chmin < 1)
        return hipErrorInvalidValue;
    // pairs per workgroup x block lanes (waves per pair, each walking every
    // BW-th block): 8 x 2 for prefill passes (C3 4096-token prefill 380 ms
    // against 388 with 8 x 1; two pairs per wave sharing each LDS fragment
    // read measured slower, 452 against 515 ms before other changes), 4 x 2 for
    // up to 8 queries (the verify batches keep k_attm, which measured faster).
    // FLARE_ATTQ_BW / FLARE_ATTQ_PBW: 1 or 2 (measurement switches)
    static const int bwe = measure_env("FLARE_ATTQ_BW") ? atoi(measure_env("FLARE_ATTQ_BW")) : 2;
    static const int pbw = measure_env("FLARE_ATTQ_PBW") ? atoi(measure_env("FLARE_ATTQ_PBW")) : 2;
    const int NPW = npairs <= 4 ? 4 : 8, BW = npairs <= 4 ? (bwe == 1 ? 1 : 2) : (pbw == 1 ? 1 : 2);
    const dim3 grid(a.nsplit, a.nkv, (npairs + NPW - 1) / NPW);
#define C(DD, GG)                                                                                     \
    if (D == DD && G == GG) {                                                                         \
        if (NPW == 8 && BW == 2) hipLaunchKernelGGL((k_attq<DD, 2 * GG, 8, 2>), grid, dim3(1024), 0, st, a); \
        else if (NPW == 8) hipLaunchKernelGGL((k_attq<DD, 2 * GG, 8, 1>), grid, dim3(512), 0, st, a); \
        else if (BW == 1) hipLaunchKernelGGL((k_attq<DD, 2 * GG, 4, 1>), grid, dim3(256), 0, st, a);  \
        else hipLaunchKernelGGL((k_attq<DD, 2 * GG, 4, 2>), grid, dim3(512), 0, st, a);               \
        return hipGetLastError();                                                                     \
    }
    C(64, 1) C(64, 2) C(64, 4) C(128, 1) C(128, 2) C(128, 4)
#undef C
    return hipErrorNotSupported;
}

hipError_t launch_attn(int kvfmt, int D, int G, hipStream_t st, const AttnArgs &a, int nq) {
    if (nq < 1) return hipErrorInvalidValue;
    if (nq > 1 && a.knew) return hipErrorInvalidValue;  // new-token stores are single-query
    if (a.qpair) {
        // query pairs: fp16 / Q8 MFMA kernel, even query count, 2G <= 8
        if (nq % 2 || !(G == 1 || G == 2 || G == 4) || !((kvfmt == KV_F16 && a.v_tblk) || kvfmt == KV_Q8))
            return hipErrorInvalidValue;
        if (a.nsplit < 1 || a.nsplit > kAttmMaxSplit || a.S % 32) return hipErrorInvalidValue;
        if (kvfmt == KV_F16) return launch_attm_t<__half>(D, 2 * G, st, a, nq / 2);
        return launch_attm_t<KvQ8>(D, 2 * G, st, a, nq / 2);
    }
    // model caches in fp16 / Q8 (V in transposed blocks): the MFMA kernel
    if ((kvfmt == KV_F16 && a.v_tblk) || kvfmt == KV_Q8 || kvfmt == KV_KIVI) {
        if ((kvfmt != KV_KIVI && !a.v_tblk) || a.nsplit < 1 || a.nsplit > kAttmMaxSplit || a.S % 32)
            return hipErrorInvalidValue;
        if (kvfmt == KV_F16) return launch_attm_t<__half>(D, G, st, a, nq);
        if (kvfmt == KV_Q8) return launch_attm_t<KvQ8>(D, G, st, a, nq);
        return launch_attm_t<KvKivi>(D, G, st, a, nq);
    }
    if (a.nsplit < 1 || a.nsplit > kAttnMaxSplit) return hipErrorInvalidValue;
    switch (kvfmt) {
    case KV_F32: return launch_attn_t<float>(D, G, st, a, nq);
    case KV_F16: return launch_attn_t<__half>(D, G, st, a, nq);
    }
    return hipErrorNotSupported;
}

// ---------------------------------------------------------------------------
// Cache writers for n new token rows (fl_kv_write / fl_kv_write_batch).
// rows: f32 [n][nkv][D] staged on the device, token p0 + i in row i.
// ---------------------------------------------------------------------------

// Q8: one thread per (token, kv head, 32-block); quantize_input_q8_0_into
// arithmetic with the scale stored as binary16.
// p0p (optional): the first position read from the device (captured verify).
__global__ __launch_bounds__(256) void k_kv_q8_write(AttnArgs a, const float *krows, const float *vrows, int p0h,
                                                     const int *p0p, int n, int D) {
    const int nb = D / 32, p0 = p0p ? *p0p : p0h;
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const long long total = (long long)n * a.nkv * nb * 2;
    if (i >= total) return;
    const int isv = (int)(i & 1);
    long long j = i >> 1;
    const int b = (int)(j % nb);
    j /= nb;
    const int kvh = (int)(j % a.nkv);
    const int r = (int)(j / a.nkv);
    const float *x = (isv ? vrows : krows) + ((size_t)r * a.nkv + kvh) * D + 32 * b;
    float amax = 0.0f;
    for (int e = 0; e < 32; e++) amax = fmaxf(amax, fabsf(x[e]));
    const float d = amax / 127.0f;
    const float id = (d != 0.0f) ? 127.0f / amax : 0.0f;
    const int t = p0 + r;
    if (isv) {  // V codes into the 32-slot transposed blocks
        int8_t *q = (int8_t *)a.vc + (size_t)kvh * a.head_stride;
        for (int e = 0; e < 32; e++) q[vt_off(t, 32 * b + e, D)] = q8_code(x[e] * id);
    } else {
        int8_t *q = (int8_t *)a.kc + (size_t)kvh * a.head_stride + (size_t)t * D + 32 * b;
        for (int e = 0; e < 32; e++) q[e] = q8_code(x[e] * id);
    }
    (isv ? a.vs : a.ks)[((size_t)kvh * a.S + t) * nb + b] = f2h(d);
}

// KIVI step 1: quantize the groups that leave the ring while rows
// [p0, p0+n) are written (grid: groups x kv heads).  Values of staged rows are
// rounded to binary16 first, as the ring would hold them.
__global__ __launch_bounds__(256) void k_kv_kivi_groups(AttnArgs a, const float *krows, const float *vrows, int p0,
                                                        int n, int D, int g0) {
    __shared__ float lds[3 * kKiviGroup * 4];
    const int gi = g0 + (int)blockIdx.x, kvh = (int)blockIdx.y;
    auto src = [&](int t, int ch, bool is_v) -> float {
        if (t >= p0) {
            const float *r = is_v ? vrows : krows;
            return __half2float(__float2half(r[((size_t)(t - p0) * a.nkv + kvh) * D + ch]));
        }
        return is_v ? __half2float(a.rv[kivi_ring_v(kvh, t, ch, D)]) : __half2float(a.rk[kivi_ring_k(kvh, t, ch, D)]);
    };
    kivi_quantize_group(a, D, kvh, gi, src, lds);
}

// KIVI step 2: the newest rows (at most kKiviRing) into the fp16 ring.
__global__ __launch_bounds__(256) void k_kv_kivi_ring(AttnArgs a, const float *krows, const float *vrows, int p0,
                                                      int n, int D, int first) {
    const int r = first + (int)blockIdx.x, kvh = (int)blockIdx.y;
    const int t = p0 + r;
    for (int e = threadIdx.x; e < 2 * D; e += blockDim.x) {
        const int isv = e >= D, ch = e % D;
        const float v = (isv ? vrows : krows)[((size_t)r * a.nkv + kvh) * D + ch];
        if (isv) a.rv[kivi_ring_v(kvh, t, ch, D)] = __float2half(v);
        else a.rk[kivi_ring_k(kvh, t, ch, D)] = __float2half(v);
    }
}

// F32 / F16: plain copy (binary16 RNE for F16, as half::f16::from_f32).
__global__ __launch_bounds__(256) void k_kv_plain_write(AttnArgs a, const float *krows, const float *vrows, int p0h,
                                                        const int *p0p, int n, int D, int f16) {
    const int p0 = p0p ? *p0p : p0h;
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const long long per = (long long)a.nkv * D;
    if (i >= (long long)n * per * 2) return;
    const int isv = (int)(i / ((long long)n * per));
    const long long j = i % ((long long)n * per);
    const int r = (int)(j / per), kvh = (int)((j % per) / D), ch = (int)(j % D);
    const float v = (isv ? vrows : krows)[j];
    const size_t o = (size_t)kvh * a.head_stride +
                     ((isv && a.v_tblk) ? vt_off(p0 + r, ch, D) : (size_t)(p0 + r) * D + ch);
    void *dst = isv ? (void *)a.vc : (void *)a.kc;
    if (f16) ((__half *)dst)[o] = __float2half(v);
    else ((float *)dst)[o] = v;
}

hipError_t launch_kv_write(int kvfmt, hipStream_t st, const AttnArgs &a, const float *krows, const float *vrows,
                           int p0, int n, int D, const int *p0p) {
    if (n <= 0) return hipSuccess;
    if (kvfmt == KV_F32 || kvfmt == KV_F16) {
        const long long total = (long long)n * a.nkv * D * 2;
        hipLaunchKernelGGL(k_kv_plain_write, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, a, krows,
                           vrows, p0, p0p, n, D, kvfmt == KV_F16 ? 1 : 0);
        return hipGetLastError();
    }
    if (kvfmt == KV_Q8) {
        const long long total = (long long)n * a.nkv * (D / 32) * 2;
        hipLaunchKernelGGL(k_kv_q8_write, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, a, krows, vrows,
                           p0, p0p, n, D);
        return hipGetLastError();
    }
    if (kvfmt != KV_KIVI) return hipErrorNotSupported;
    if (p0p) return hipErrorInvalidValue;  // KIVI group work is planned from the host position
    // groups [0, kivi_qlen(T + 1)) are quantized once T tokens are written
    const int g0 = kivi_qlen(p0 + 1) / kKiviGroup, g1 = kivi_qlen(p0 + n + 1) / kKiviGroup;
    if (g1 > g0) {
        hipLaunchKernelGGL(k_kv_kivi_groups, dim3(g1 - g0, a.nkv), dim3(256), 0, st, a, krows, vrows, p0, n, D, g0);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    const int first = n > kKiviRing ? n - kKiviRing : 0;
    hipLaunchKernelGGL(k_kv_kivi_ring, dim3(n - first, a.nkv), dim3(256), 0, st, a, krows, vrows, p0, n, D, first);
    return hipGetLastError();
}

}  // namespace fl
