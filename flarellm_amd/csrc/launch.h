// Host-side launch plans and launchers of the kernel translation units.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>

#include "attn_kernels.h"
#include "mv_kernels.h"

namespace fl {

// Matvec plan: LPR lanes per row group, R rows per group, U units unrolled
// per lane per iteration (U*R*32 B of weight loads in flight per lane).
struct MvPlan {
    int lpr = 64, r = 1, u = 1, grid = 1;
    size_t lds = 0;
};

inline int units_per_row(int fmt, int cols) {
    switch (fmt) {
    case F_Q8_0: return cols / 32;
    case F_Q4K:
    case F_Q6K: return cols / 64;
    default: return cols / 4;
    }
}

inline MvPlan mv_plan(int fmt, int rows, int cols, bool f32in) {
    MvPlan p;
    const int upr = units_per_row(fmt, cols);
    p.lpr = upr >= 64 ? 64 : (upr >= 32 ? 32 : 16);
    const int iters = (upr + p.lpr - 1) / p.lpr;
    p.u = iters >= 4 ? 4 : (iters >= 2 ? 2 : 1);
    if (p.lpr < 64 && p.u > 2) p.u = 2;
    const int groups = kThreads / p.lpr;
    p.r = 8 / p.u;
    while (p.r > 1 && (rows + groups * p.r - 1) / (groups * p.r) < 512) p.r /= 2;
    p.grid = (rows + groups * p.r - 1) / (groups * p.r);
    p.lds = f32in ? (size_t)cols * 4 + 64 * 4 : q8_lds_bytes(cols);
    return p;
}

struct GuPlan {
    int lpr = 64, u = 1;
    size_t lds = 0;
};
constexpr int kGuThreads = 512;

inline GuPlan gu_plan(int fmt, int cols) {
    GuPlan p;
    const int upr = units_per_row(fmt, cols);
    p.lpr = upr >= 64 ? 64 : (upr >= 32 ? 32 : 16);
    const int iters = (upr + p.lpr - 1) / p.lpr;
    p.u = (p.lpr < 64 && iters >= 2) ? 2 : 1;
    p.lds = q8_lds_bytes(cols) + 96 * 4;
    return p;
}

// Split count for a cache of up to max_seq slots.  The kernel covers the
// context in chunks of max(chmin, ceil(T / nsplit)) tokens (chmin = one
// batch), so each workgroup streams at most a few batches and ~T/chmin
// workgroups per kv head run in parallel (at most 256 splits).
inline void choose_splits(int max_seq, int nkv, int head_dim, int &nsplit, int &chmax) {
    const int chmin = attn_chmin(head_dim);
    const int cover = (max_seq + chmin - 1) / chmin;
    nsplit = std::max(1, std::min(cover, 256));
    chmax = std::max(chmin, (max_seq + nsplit - 1) / nsplit);
    (void)nkv;
}

inline bool attn_supported(int D, int G) {
    return (D == 64 || D == 128) && (G == 1 || G == 2 || G == 3 || G == 4 || G == 8);
}

// launchers (return hipErrorNotSupported when no instantiation matches)
hipError_t launch_mv_q8in_q8_0(const MvPlan &p, hipStream_t st, const Q8inArgs &a);
hipError_t launch_mv_q8in_q4k(const MvPlan &p, hipStream_t st, const Q8inArgs &a);
hipError_t launch_mv_f32in(int fmt, const MvPlan &p, hipStream_t st, const F32Args &a);
hipError_t launch_gateup_q8_0(const GuPlan &p, int grid, hipStream_t st, const GuArgs &a);
hipError_t launch_gateup_q4k(const GuPlan &p, int grid, hipStream_t st, const GuArgs &a);
hipError_t launch_attn(bool f16, int D, int G, hipStream_t st, const AttnArgs &a);

}  // namespace fl
