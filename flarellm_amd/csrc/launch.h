// Host-side launch plans and launchers of the kernel translation units.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>
#include <map>
#include <mutex>
#include <utility>

#include "attn_kernels.h"
#include "mvs_kernels.h"
#include "verify_args.h"

namespace fl {

// Persistent kernels assume every workgroup of the grid is resident at once
// (a late second wave of workgroups would run the whole prologue again after
// the first wave drained): clamp the grid to the kernel's occupancy x CUs.
template <typename Kern>
inline int resident_grid(Kern kernel, int threads, size_t lds, int want) {
    static std::mutex mu;
    static std::map<std::pair<const void *, size_t>, int> cache;
    const std::pair<const void *, size_t> key((const void *)kernel, lds);
    std::lock_guard<std::mutex> lk(mu);
    auto it = cache.find(key);
    int cap;
    if (it != cache.end()) {
        cap = it->second;
    } else {
        int dev = 0, ncu = 0, per = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, kernel, threads, lds) != hipSuccess || per < 1)
            cap = want;
        else
            cap = per * ncu;
        cache[key] = cap;
    }
    return std::max(1, std::min(want, cap));
}

// Streaming matvec plan: R rows per wave item, SU steps (1 KiB each) per
// unit, so one tile is R*SU 16-byte pieces per lane (<= 8; two tiles in
// flight); grid = persistent workgroups (4 waves each), at most 4 per CU.
struct MvsPlan {
    int r = 2, su = 1, grid = 1;
    size_t lds = 0;
};

// (R, SU) per format and step count: tiles of 2-8 pieces, chosen so the
// kernel stays within ~160 VGPRs (>= 3 waves per SIMD)
// pairs: the epilogue needs row pairs (fused QKV + RoPE)
inline void mvs_shape(int fmt, bool f32in, int S, bool pairs, int &r, int &su) {
    // f32 input (logits), measured on MI355X: Q8_0 4 rows x 2 KiB (Llama-3.2-1B
    // tied output: 45.7 vs 48.5 us for 2 x 2 KiB), Q6_K 2 rows x 1 KiB
    if (fmt == F_Q8_0 && f32in) { r = S >= 2 ? 4 : 2; su = S >= 2 ? 2 : 1; return; }
    if (fmt == F_Q6K && f32in) { r = 2; su = 1; return; }
    if (S <= 1) { r = 4; su = 1; return; }
    // Q4_K with Q8 input, measured on MI355X (Llama-3-8B): QKV 4 rows x 1 KiB
    // (8.0 vs 8.6-8.9 us for 2-row tiles); rows of one or two steps (wo) 2 x
    // 2 KiB with the codes in registers (4.3 vs 4.7 us for 1 x 2 KiB), longer
    // rows (down) 4 x 1 KiB (7.6 vs 8.4 us for 1 x 2 KiB, 7.9 for 2 x 1 KiB)
    if (fmt == F_Q4K) {
        if (pairs) { r = 4; su = 1; }
        else if (S <= 2) { r = 2; su = 2; }
        else { r = 4; su = 1; }
        return;
    }
    if (fmt == F_Q6K) { r = 2; su = 2; return; }
    if (S == 2 || S == 3) { r = 4; su = 2; return; }
    // long Q8_0 rows (Llama-3.2-1B down, 8 KiB): 1 row x 4 KiB measured best
    r = pairs ? 2 : 1;
    su = 4;
}

inline MvsPlan mvs_plan(int fmt, int rows, int cols, bool f32in, bool pairs = false) {
    MvsPlan p;
    mvs_shape(fmt, f32in, mvs_steps(fmt, cols), pairs, p.r, p.su);
    // tuning overrides for the Q8-input kernels (experiments): FLARE_MVS_R /
    // FLARE_MVS_SU / FLARE_MVS_GRID
    // (FLARE_MVF_R / FLARE_MVF_SU for the f32-input kernels)
    const char *er = measure_env(f32in ? "FLARE_MVF_R" : pairs ? "FLARE_QKV_R" : "FLARE_MVS_R");
    if (er) p.r = atoi(er);
    if (const char *e = measure_env(f32in ? "FLARE_MVF_SU" : pairs ? "FLARE_QKV_SU" : "FLARE_MVS_SU")) p.su = atoi(e);
    // fill the chip: halve the rows per group while fewer than 256
    // workgroups (4 waves, one group each) would run; not for the fused QKV,
    // whose waves each normalise the activation (4 rows x 2 KiB measured
    // best for Llama-3.2-1B's 3072 rows: 5.7 vs 6.5 us)
    while (p.r > 2 && (rows + p.r - 1) / p.r < 4 * 256 && !er && !pairs) p.r /= 2;
    const int ngrp = (rows + p.r - 1) / std::max(1, p.r);
    p.grid = std::max(1, std::min((ngrp + 3) / 4, 1024));
    if (const char *e = measure_env("FLARE_MVS_GRID")) p.grid = std::max(1, std::min(p.grid, atoi(e)));
    p.lds = mvs_lds_fmt(fmt, f32in, cols);
    if (const char *e = measure_env("FLARE_MVS_LDSPAD")) p.lds += (size_t)atoi(e);  // placement experiments
    return p;
}

// gate/up: 32 hidden units per workgroup block, 4 rows per item, 8 waves
// per workgroup
inline MvsPlan mvs_gu_plan(int fmt, int F, int cols) {
    MvsPlan p;
    const int nblk = F / 32;
    // waves per workgroup and steps per unit, measured on MI355X: Q4_K
    // (Llama-3-8B gate/up, 448 blocks) 8 waves x 1 KiB; Q8_0 (Llama-3.2-1B,
    // 256 blocks) 8 waves x 2 KiB
    p.r = 8;
    p.su = (fmt == F_Q8_0 && mvs_steps(fmt, cols) >= 2) ? 2 : 1;
    // tuning overrides (experiments): FLARE_GU_NW / FLARE_GU_SU
    if (const char *e = measure_env("FLARE_GU_NW")) p.r = atoi(e);
    if (const char *e = measure_env("FLARE_GU_SU")) p.su = atoi(e);
    p.grid = std::max(1, std::min(nblk, 1024));
    p.lds = mvs_lds_gu(cols, p.r);
    return p;
}

// Split count for a cache of up to max_seq slots (fixed for the captured
// decode graph; the kernel derives the chunk from the live position).  A
// chunk is max(chmin, ceil(T / nsplit)) tokens rounded up to one pass, so
// about 256 workgroups run once the context is long enough.
inline void choose_splits(int max_seq, int nkv, int head_dim, int &nsplit, int &chmin) {
    chmin = attn_round(head_dim) / 2;  // 64 tokens: half a round of loads per thread
    const int cover = (max_seq + chmin - 1) / chmin;
    nsplit = std::max(1, std::min({cover, std::max(1, 256 / std::max(1, nkv)), kAttnMaxSplit}));
}

inline bool attn_supported(int D, int G) {
    return (D == 64 || D == 128) && (G == 1 || G == 2 || G == 3 || G == 4 || G == 8);
}

// launchers (return hipErrorNotSupported when no instantiation matches)
hipError_t launch_mvs_q8_0(bool f32in, const MvsPlan &p, hipStream_t st, const MvsArgs &a);
hipError_t launch_mvs_q4k(const MvsPlan &p, hipStream_t st, const MvsArgs &a);
hipError_t launch_mvs_f32(int fmt, const MvsPlan &p, hipStream_t st, const MvsArgs &a);
hipError_t launch_mvs_gu_q8_0(const MvsPlan &p, hipStream_t st, const MvsArgs &a);
hipError_t launch_mvs_gu_q4k(const MvsPlan &p, hipStream_t st, const MvsArgs &a);
enum KvFmt { KV_F32 = 0, KV_F16 = 1, KV_Q8 = 2, KV_KIVI = 3 };  // == FL_KV_*
hipError_t launch_attn(int kvfmt, int D, int G, hipStream_t st, const AttnArgs &a, int nq = 1);
hipError_t launch_attq(int D, int G, hipStream_t st, const AttnArgs &a);
// fused QKV matvec + decode attention (fused.hip): nqwg QKV workgroups (a
// multiple of a.nkv) of nt threads, then a.nsplit * a.nkv attention ones
hipError_t launch_qkv_attm(int fmt, const MvsPlan &p, int rx, int D, int G, int nt, hipStream_t st,
                           const struct MvsArgs &m, const AttnArgs &at, int nqwg, const FuseWait &fw);
// workgroups of the MFMA attention kernel (format, D, G, waves) resident on one CU at once
int attm_resident_per_cu(int kvfmt, int D, int G, int waves);
// Write n token rows (device f32 [n][nkv][D]) at positions p0.. into a Q8 or
// KIVI cache (quantizing the KIVI groups that leave the ring).
// p0p (optional, F32 / F16 / Q8): read the first position from the device instead of p0.
hipError_t launch_kv_write(int kvfmt, hipStream_t st, const AttnArgs &a, const float *krows, const float *vrows,
                           int p0, int n, int D, const int *p0p = nullptr);

// Reference-order kernels (seq.hip): sequential attention of the new token
// over slots 0..*posp of an F32 / F16 head-major cache, rmsnorm_into, and the
// f32-input output projection with first-max argmax.
struct SeqAttnArgs {
    const float *q;
    const void *kc, *vc;     // layer cache planes [kv head][slot][D] (F16: V in 32-slot transposed blocks)
    long long head_stride;   // elements between kv heads
    int D, group, slots;     // head_dim, query heads per kv head, slots per kv head
    const int *posp;         // token position (device)
    float *scores;           // [num_heads][slots] scratch
    float *out;              // [num_heads][D]
};
hipError_t launch_attn_seq(bool f16, hipStream_t st, const SeqAttnArgs &a, int num_heads);
hipError_t launch_rmsnorm_seq(hipStream_t st, const float *x, const float *w, int n, float eps, float *out);
hipError_t launch_out_seq(int fmt, hipStream_t st, const WDesc &W, const float *xn, float *logits,
                          unsigned long long *slot);

// MFMA output projection with f32 input for up to 8 tokens (mvo.hip)
struct MvoArgs;
hipError_t launch_mvo(int fmt, hipStream_t st, const MvoArgs &a);

// speculative verify (verify.hip)
hipError_t launch_vgemm(int fmt, hipStream_t st, const VgArgs &a);
hipError_t launch_v_embed(int fmt, hipStream_t st, const WDesc &E, const int *tokens, int M, float *x);
hipError_t launch_v_resnorm(int pro, hipStream_t st, const float *part, int ksplit, int M, int H, float *x,
                            const float *w, float eps, int8_t *q, float *s, int *sum);
hipError_t launch_v_qkv_post(hipStream_t st, const float *part, int ksplit, int M, int rows,
                             const VgArgs::QkvPost &P);
hipError_t launch_v_store(hipStream_t st, const float *part, int ksplit, int M, int rows, float *out);
hipError_t launch_v_residual(hipStream_t st, const float *part, int ksplit, int M, int H, float *x);
hipError_t launch_v_silu_quant(hipStream_t st, const float *part, int ksplit, int M, int F, int8_t *q, float *s,
                               int *sum);

}  // namespace fl
