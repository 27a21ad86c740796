// Host-side launch plans and launchers of the kernel translation units.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>

#include "attn_kernels.h"
#include "mv_kernels.h"

namespace fl {

// Matvec plan: LPR lanes per row group, U units per lane per item, R rows
// per group; grid = persistent workgroup count.
struct MvPlan {
    int lpr = 64, u = 1, r = 1, grid = 1;
    size_t lds = 0;
};

inline int units_per_row(int fmt, int cols) { return fmt_units_per_row(fmt, cols); }

// rows per tile so that one lane keeps ~256 B of weights in flight
inline int tile_rows(int fmt, int u) {
    const int base = (fmt == F_Q8_0 || fmt == F_F32) ? 8 : 4;
    return std::max(1, base / u);
}

inline MvPlan mv_plan(int fmt, int rows, int cols, bool f32in) {
    MvPlan p;
    const int upr = units_per_row(fmt, cols);
    for (int lpr : {64, 32, 16}) {
        if (lpr > 16 && upr * 2 <= lpr) continue;  // more than half the lanes idle
        int u = (upr + lpr - 1) / lpr;
        u = u >= 4 ? 4 : (u >= 2 ? 2 : 1);
        int r = tile_rows(fmt, u);
        const int groups = kThreads / lpr;
        const int nchunk = (upr + lpr * u - 1) / (lpr * u);
        auto wgs = [&](int rr) { return ((rows + rr - 1) / rr * nchunk + groups - 1) / groups; };
        while (r > 1 && wgs(r) < 256) r /= 2;
        // vocab-sized outputs run persistent (grid capped at 1024): 2-row
        // tiles keep more independent loads in flight per wave (measured
        // 55 us vs 72 us for 128256 x 2048 Q8_0, 151 vs 169 us for Q6_K)
        if (rows >= 32768) r = std::min(r, 2);
        p.lpr = lpr;
        p.u = u;
        p.r = r;
        p.grid = std::max(1, std::min(wgs(r), 1024));
        if (wgs(r) >= 256) break;
    }
    p.lds = f32in ? (size_t)cols * 4 + 64 * 4 : q8_lds_bytes(cols);
    // tuning overrides (experiments): FLARE_MV_R / FLARE_MV_GRID
    if (const char *e = getenv("FLARE_MV_R")) {
        const int r = atoi(e);
        if (r == 1 || r == 2 || r == 4 || r == 8) p.r = r;
        const int groups = kThreads / p.lpr;
        const int nchunk = (upr + p.lpr * p.u - 1) / (p.lpr * p.u);
        p.grid = std::max(1, std::min(((rows + p.r - 1) / p.r * nchunk + groups - 1) / groups, 1024));
    }
    if (const char *e = getenv("FLARE_MV_GRID")) p.grid = std::max(1, std::min(p.grid, atoi(e)));
    return p;
}

// Same plan with an even row count per tile (EPI_QKV stores row pairs).
inline MvPlan mv_plan_even(MvPlan p, int fmt, int rows, int cols) {
    if (p.r % 2 == 0) return p;
    p.r = 2;
    const int upr = units_per_row(fmt, cols), groups = kThreads / p.lpr;
    const int nchunk = (upr + p.lpr * p.u - 1) / (p.lpr * p.u);
    p.grid = std::max(1, std::min(((rows + 1) / 2 * nchunk + groups - 1) / groups, 1024));
    return p;
}

struct GuPlan {
    int lpr = 64, u = 1, grid = 1;
    size_t lds = 0;
};
constexpr int kGuThreads = 512;

inline GuPlan gu_plan(int fmt, int cols, int F) {
    GuPlan p;
    const int upr = units_per_row(fmt, cols);
    p.lpr = upr >= 64 ? 64 : (upr >= 32 ? 32 : 16);
    const int u = (upr + p.lpr - 1) / p.lpr;  // the whole row in one tile
    p.u = u <= 1 ? 1 : (u <= 2 ? 2 : (u <= 4 ? 4 : 0));
    p.grid = std::max(1, std::min(F / 32, 256));
    p.lds = q8_lds_bytes(cols) + 96 * 4;
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
hipError_t launch_mv_q8in_q8_0(const MvPlan &p, hipStream_t st, const Q8inArgs &a);
hipError_t launch_mv_q8in_q4k(const MvPlan &p, hipStream_t st, const Q8inArgs &a);
hipError_t launch_mv_f32in(int fmt, const MvPlan &p, hipStream_t st, const F32Args &a);
hipError_t launch_gateup_q8_0(const GuPlan &p, hipStream_t st, const GuArgs &a);
hipError_t launch_gateup_q4k(const GuPlan &p, hipStream_t st, const GuArgs &a);
hipError_t launch_attn(bool f16, int D, int G, hipStream_t st, const AttnArgs &a);

}  // namespace fl
