// Causal GQA attention for several consecutive query tokens over an fp16
// cache (speculative-verify and prefill passes).
//
// Same semantics as k_attm's query-pair mode (cpu_grouped_query_attention_into,
// flare-core/src/model.rs:9849-9966; causal prefill attention 336-368):
// query j of the pass sits at position *posp + j and attends slots
// 0 .. *posp + j.  The difference is the data flow: k_attm gives every query
// pair its own workgroup, each streaming the whole K/V prefix of its kv head,
// so a pass of M tokens reads the cache M/2 times.  Here one workgroup holds
// NW query pairs (one per wave) and stages each 32-slot K/V block in LDS once
// for all of them:
//  * grid (split, kv head, pair group); the split's chunk of slots is walked
//    block by block, the next block's global loads in flight (registers)
//    while the waves compute on the current one (double-buffered LDS, one
//    workgroup barrier per block);
//  * per wave, the fp16 MFMA scheme of k_attm: rows (query, head, high /
//    residual) of the pair's 2G heads, S = Q K^T and O += P V on
//    v_mfma_f32_16x16x32_f16, wave-private online softmax;
//  * splits publish (o, m, l) per wave with agent-scope stores; the last
//    arriving workgroup of a (pair group, kv head) merges them (weights per
//    row formed once, then one load per partial and output) and writes the
//    f32 output and / or its Q8_0 copy.
#pragma once

#include "attm_kernels.h"

namespace fl {

constexpr int kAttqKPad = 8;  // halves of padding per staged K row
constexpr int kAttqVPad = 8;  // per staged V channel row

template <int D, int NPW>  // NPW = query pairs per workgroup
struct AttqLds {
    static constexpr int KS = D + kAttqKPad, VS = 32 + kAttqVPad;
    static constexpr int KH = 32 * KS, VH = D * VS;  // halves per staged block
    static constexpr size_t LOOP = (size_t)2 * (KH + VH) * 2;  // double-buffered K and V
    static constexpr size_t SP = (size_t)NPW * 8 * 32 * 4;      // p of the current block per pair
    static constexpr size_t RED = (size_t)NPW * 8 * D * 4;      // per-pair outputs (after the loop)
    static constexpr size_t WT = (size_t)NPW * 8 * kAttmMaxSplit * 4;  // merge weights
    static constexpr size_t BYTES = (LOOP + SP > RED + WT ? LOOP + SP : RED + WT);
};

// G2 = rows of a query pair: the model's G heads of each of its 2 queries.
// NW waves, RP query pairs per wave (each staged K / V fragment read from LDS
// once per wave feeds the RP pairs' MFMAs).
template <int D, int G2, int NW, int RP>
__global__ __launch_bounds__(NW * 64) void k_attq(AttnArgs a) {
    constexpr int DT = D / 32, NT = D / 16, NTH = NW * 64, GH = G2 / 2, NPW = NW * RP;
    using L = AttqLds<D, NPW>;
    constexpr int KS = L::KS, VS = L::VS;
    static_assert(G2 <= 8 && G2 % 2 == 0, "2G rows of a query pair (hi / lo) fill at most one MFMA tile");
    __shared__ __align__(16) char smem[L::BYTES];
    __shared__ int is_last;
    _Float16 *lk = (_Float16 *)smem;             // [2][32][KS]
    _Float16 *lv = lk + 2 * L::KH;               // [2][D][VS]
    float *sp = (float *)(smem + L::LOOP);       // [NPW][8][32]
    float *red = (float *)smem;                  // [NPW][8][D], after the loop
    float *wt = (float *)(smem + L::RED);        // [NPW][8][kAttmMaxSplit]

    const int kvh = blockIdx.y, s = blockIdx.x, zg = blockIdx.z, tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6, kg = lane >> 4, r = lane & 15;
    const int npairs = a.nq / 2, pw0 = zg * NPW + wave * RP;  // the wave's first pair
    const bool live = pw0 < npairs;                           // wave-uniform
    const int glast = 2 * min(npairs, (zg + 1) * NPW) - 1;    // last query of the group
    int q0[RP];
#pragma unroll
    for (int i = 0; i < RP; i++) q0[i] = 2 * min(pw0 + i, npairs - 1);

    // query rows first (independent of the position)
    v4f_t qv[RP][DT][2];
    {
        const int g = min(r >> 1, G2 - 1);
#pragma unroll
        for (int i = 0; i < RP; i++) {
            const size_t qo = (size_t)(q0[i] + (g >= GH ? 1 : 0)) * a.qstride + (size_t)(kvh * GH + g % GH) * D;
            const v4f_t *qp = (const v4f_t *)(a.q + qo + 8 * kg);
#pragma unroll
            for (int dt = 0; dt < DT; dt++) {
                qv[i][dt][0] = qp[8 * dt];
                qv[i][dt][1] = qp[8 * dt + 1];
            }
        }
    }
    const int base = __hip_atomic_load(a.posp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int Tg = base + glast + 1;  // slots the group's last query sees
    int CH = max(a.chmin, (Tg + a.nsplit - 1) / a.nsplit);
    CH = (CH + kAttmBlock - 1) / kAttmBlock * kAttmBlock;
    const int t0 = s * CH;
    if (t0 >= Tg) return;  // whole workgroup
    const int t1 = min(Tg, t0 + CH), nact = (Tg + CH - 1) / CH;
    const int nblk = (t1 - t0 + kAttmBlock - 1) / kAttmBlock;
    // rows of lane group kg: head rows 2kg + e; their query's last slot
    int lim[RP][2];
#pragma unroll
    for (int i = 0; i < RP; i++)
#pragma unroll
        for (int e = 0; e < 2; e++) lim[i][e] = base + q0[i] + ((2 * kg + e) >= GH ? 1 : 0);
    const int wlim = base + 2 * min(pw0 + RP - 1, npairs - 1) + 1;  // last slot any row of the wave sees

    // block staging: K rows tb..tb+31 (contiguous [slot][D]) and the transposed
    // V block ([D][32], contiguous), 16 B per thread and piece
    constexpr int NP = 32 * D / 8, PPT = (NP + NTH - 1) / NTH;
    const __half *kc = (const __half *)a.kc + (size_t)kvh * a.head_stride;
    const __half *vc = (const __half *)a.vc + (size_t)kvh * a.head_stride;
    // two register sets: block j's pieces live in set j & 1, loaded two
    // iterations before they are staged
    v4i_t kr[2][PPT], vr[2][PPT];
    auto gload = [&](v4i_t(&kk)[PPT], v4i_t(&vv)[PPT], int tb) {
        const v4i_t *ks = (const v4i_t *)(kc + (size_t)tb * D);
        const v4i_t *vs = (const v4i_t *)(vc + vt_off(tb, 0, D));
#pragma unroll
        for (int u = 0; u < PPT; u++) {
            const int i = min(tid + u * NTH, NP - 1);
            kk[u] = ks[i];
            vv[u] = vs[i];
        }
    };
    auto lstore = [&](const v4i_t(&kk)[PPT], const v4i_t(&vv)[PPT], int buf) {
#pragma unroll
        for (int u = 0; u < PPT; u++) {
            const int i = tid + u * NTH;
            if (NP % NTH == 0 || i < NP) {
                *(v4i_t *)(lk + buf * L::KH + (i / (D / 8)) * KS + 8 * (i % (D / 8))) = kk[u];
                *(v4i_t *)(lv + buf * L::VH + (i >> 2) * VS + 8 * (i & 3)) = vv[u];
            }
        }
    };
    gload(kr[0], vr[0], t0);
    if (nblk > 1) gload(kr[1], vr[1], t0 + kAttmBlock);

    // A operands of S: row m = 2g + (hi / lo) of head row g (rows >= 2 G2 zero)
    v8h_t aq[RP][DT];
#pragma unroll
    for (int i = 0; i < RP; i++)
#pragma unroll
        for (int dt = 0; dt < DT; dt++) {
            const v4f_t x0 = qv[i][dt][0], x1 = qv[i][dt][1];
            float x[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
            if ((r >> 1) >= G2) {
#pragma unroll
                for (int j = 0; j < 8; j++) x[j] = 0.0f;
            }
            v8h_t hi, lo;
            split8(x, hi, lo);
            aq[i][dt] = (r & 1) ? lo : hi;
        }
    const float scale = 1.0f / sqrtf((float)D);
    float m_run[RP][2], l_run[RP][2];
    v4f32_t oacc[RP][NT];
#pragma unroll
    for (int i = 0; i < RP; i++) {
        m_run[i][0] = m_run[i][1] = -INFINITY;
        l_run[i][0] = l_run[i][1] = 0.0f;
#pragma unroll
        for (int nt = 0; nt < NT; nt++) oacc[i][nt] = v4f32_t{0.f, 0.f, 0.f, 0.f};
    }

    lstore(kr[0], vr[0], 0);
    if (nblk > 2) gload(kr[0], vr[0], t0 + 2 * kAttmBlock);
    __syncthreads();
    // block bi: computed from LDS buffer bi & 1; then block bi + 1 (register
    // set (bi + 1) & 1) goes to the other buffer and that set loads block bi + 3
    auto block = [&](int bi, v4i_t(&kn)[PPT], v4i_t(&vn)[PPT]) {
        const int cur = bi & 1, tb = t0 + bi * kAttmBlock;
        if (live && tb <= wlim) {  // wave-uniform: some row sees the block
            const _Float16 *bk = lk + cur * L::KH, *bv = lv + cur * L::VH;
            v4f32_t acc[RP][2];
#pragma unroll
            for (int i = 0; i < RP; i++) acc[i][0] = acc[i][1] = v4f32_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int h = 0; h < 2; h++)
#pragma unroll
                for (int dt = 0; dt < DT; dt++) {
                    const v8h_t kb = *(const v8h_t *)(bk + (16 * h + r) * KS + 32 * dt + 8 * kg);
#pragma unroll
                    for (int i = 0; i < RP; i++) acc[i][h] = mfma16(aq[i][dt], kb, acc[i][h]);
                }
            v8h_t ap[RP];
#pragma unroll
            for (int i = 0; i < RP; i++) {
                float *spw = sp + (wave * RP + i) * 8 * 32;
                float sc[2][2];  // [half][head row parity] for slot tb + 16h + r
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const int t = tb + 16 * h + r;
                    sc[h][0] = t < t1 && t <= lim[i][0] ? (acc[i][h][0] + acc[i][h][1]) * scale : -INFINITY;
                    sc[h][1] = t < t1 && t <= lim[i][1] ? (acc[i][h][2] + acc[i][h][3]) * scale : -INFINITY;
                }
                float alpha[2];
#pragma unroll
                for (int e = 0; e < 2; e++) {
                    const float bm = row_max<16>(fmaxf(sc[0][e], sc[1][e]));
                    const float mn = fmaxf(m_run[i][e], bm);
                    // a row that has seen nothing yet keeps m = -inf (and p = 0)
                    alpha[e] = (m_run[i][e] == -INFINITY) ? 0.0f : __expf(m_run[i][e] - mn);
                    const float p0 = sc[0][e] == -INFINITY ? 0.0f : __expf(sc[0][e] - mn);
                    const float p1 = sc[1][e] == -INFINITY ? 0.0f : __expf(sc[1][e] - mn);
                    l_run[i][e] = l_run[i][e] * alpha[e] + row_sum<16>(p0 + p1);
                    m_run[i][e] = mn;
                    const int g = 2 * kg + e;
                    if (g < G2) {
                        spw[g * 32 + r] = p0;
                        spw[g * 32 + 16 + r] = p1;
                    }
                }
#pragma unroll
                for (int nt = 0; nt < NT; nt++) {
                    oacc[i][nt][0] *= alpha[0];
                    oacc[i][nt][1] *= alpha[0];
                    oacc[i][nt][2] *= alpha[1];
                    oacc[i][nt][3] *= alpha[1];
                }
            }
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int i = 0; i < RP; i++) {
                const float *spw = sp + (wave * RP + i) * 8 * 32;
                const int g = r >> 1;
                float pv[8];
#pragma unroll
                for (int j = 0; j < 8; j++) pv[j] = g < G2 ? spw[g * 32 + 8 * kg + j] : 0.0f;
                v8h_t hi, lo;
                split8(pv, hi, lo);
                ap[i] = (r & 1) ? lo : hi;
            }
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                const v8h_t vb = *(const v8h_t *)(bv + (16 * nt + r) * VS + 8 * kg);
#pragma unroll
                for (int i = 0; i < RP; i++) oacc[i][nt] = mfma16(ap[i], vb, oacc[i][nt]);
            }
            __builtin_amdgcn_wave_barrier();
        }
        if (bi + 1 < nblk) {
            lstore(kn, vn, cur ^ 1);
            if (bi + 3 < nblk) gload(kn, vn, tb + 3 * kAttmBlock);
        }
        __syncthreads();
    };
    for (int bi = 0; bi < nblk; bi += 2) {
        block(bi, kr[1], vr[1]);
        if (bi + 1 < nblk) block(bi + 1, kr[0], vr[0]);
    }

    // per-pair result: head row g = 2kg + e, channel 16nt + r
    // (rows 4kg + 2e / + 1 of oacc: high / residual parts of P)
    constexpr int P = G2 * (D + 2);
    float *gpart = a.part + ((size_t)zg * a.nkv + kvh) * a.nsplit * NPW * P;  // this (group, kv head)
#pragma unroll
    for (int i = 0; i < RP; i++) {
        const int slot = wave * RP + i;
        if (pw0 + i >= npairs) continue;  // wave-uniform
        float *mypart = gpart + ((size_t)s * NPW + slot) * P;
        float *rw = red + slot * 8 * D;
#pragma unroll
        for (int e = 0; e < 2; e++) {
            const int g = 2 * kg + e;
            if (g < G2) {
                const float il = nact == 1 ? 1.0f / l_run[i][e] : 1.0f;
#pragma unroll
                for (int nt = 0; nt < NT; nt++) {
                    const float o = oacc[i][nt][2 * e] + oacc[i][nt][2 * e + 1];
                    if (nact == 1) rw[g * D + 16 * nt + r] = o * il;
                    else st_agent(mypart + g * D + 16 * nt + r, o);
                }
                if (nact > 1 && r == 0) {
                    st_agent(mypart + G2 * D + 2 * g, m_run[i][e]);
                    st_agent(mypart + G2 * D + 2 * g + 1, l_run[i][e]);
                }
            }
        }
    }
    if (nact > 1) {
        if (!split_arrive_last<true>(&a.counters[(size_t)zg * a.nkv + kvh], nact, &is_last)) return;
        // last workgroup: merge weights per (pair, head row) from the (m, l)
        // of every split (loads in batches of 8 splits, all in flight), then
        // each thread's outputs in chunks of 8, all loads of a batch of 8
        // splits in flight (a handful of round trips in all, not one per output)
        float *mw = wt;  // [NPW * 8][kAttmMaxSplit]: m, then the weights
        float *lw = red; // [NPW * 8][kAttmMaxSplit]: l (red is rewritten after)
        for (int i = tid; i < NPW * G2; i += NTH) {
            const int w = i / G2, g = i % G2;
            for (int j0 = 0; j0 < nact; j0 += 8) {
                float mv[8], lv[8];
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    const float *pj = gpart + ((size_t)min(j0 + k, nact - 1) * NPW + w) * P + G2 * D + 2 * g;
                    mv[k] = ld_agent(pj);
                    lv[k] = ld_agent(pj + 1);
                }
#pragma unroll
                for (int k = 0; k < 8; k++)
                    if (j0 + k < nact) {
                        mw[(w * 8 + g) * kAttmMaxSplit + j0 + k] = mv[k];
                        lw[(w * 8 + g) * kAttmMaxSplit + j0 + k] = lv[k];
                    }
            }
            float M = -INFINITY;
            for (int j = 0; j < nact; j++) M = fmaxf(M, mw[(w * 8 + g) * kAttmMaxSplit + j]);
            float Ls = 0.0f;
            for (int j = 0; j < nact; j++) {
                const float mj = mw[(w * 8 + g) * kAttmMaxSplit + j];
                const float wj = mj == -INFINITY ? 0.0f : __expf(mj - M);
                Ls += lw[(w * 8 + g) * kAttmMaxSplit + j] * wj;
                mw[(w * 8 + g) * kAttmMaxSplit + j] = wj;
            }
            const float il = 1.0f / Ls;
            for (int j = 0; j < nact; j++) mw[(w * 8 + g) * kAttmMaxSplit + j] *= il;
        }
        __syncthreads();
        constexpr int NO = NPW * G2 * D, CK = NO / NTH < 8 ? NO / NTH : 8;  // outputs; per chunk and thread
        static_assert(NO % (NTH * CK) == 0, "whole chunks of outputs per thread");
        for (int c0 = 0; c0 < NO; c0 += NTH * CK) {
            float O[CK];
#pragma unroll
            for (int k = 0; k < CK; k++) O[k] = 0.0f;
            for (int j0 = 0; j0 < nact; j0 += 8) {
                float ov[CK][8];
#pragma unroll
                for (int k = 0; k < CK; k++) {
                    const int i = c0 + k * NTH + tid, w = i / (G2 * D), gd = i % (G2 * D);
#pragma unroll
                    for (int u = 0; u < 8; u++)
                        ov[k][u] = ld_agent(gpart + ((size_t)min(j0 + u, nact - 1) * NPW + w) * P + gd);
                }
#pragma unroll
                for (int k = 0; k < CK; k++) {
                    const int i = c0 + k * NTH + tid, w = i / (G2 * D), g = (i % (G2 * D)) / D;
                    const float *wr = wt + (w * 8 + g) * kAttmMaxSplit;
#pragma unroll
                    for (int u = 0; u < 8; u++)
                        if (j0 + u < nact) O[k] += ov[k][u] * wr[j0 + u];
                }
            }
#pragma unroll
            for (int k = 0; k < CK; k++) {
                const int i = c0 + k * NTH + tid, w = i / (G2 * D), gd = i % (G2 * D);
                if (zg * NPW + w < npairs) red[w * 8 * D + gd] = O[k];
            }
        }
        __syncthreads();
    } else {
        __syncthreads();
    }
    // outputs of head row g of pair slot w: query 2 (group base + w) + (g >= GH),
    // model head kvh * GH + g % GH; the f32 rows and / or their Q8_0 blocks
    // (32 lanes each)
    for (int b = tid >> 5; b < NPW * G2 * D / 32; b += NTH / 32) {
        const int w = b / (G2 * D / 32), gd = (b % (G2 * D / 32)) * 32, g = gd / D, c = gd % D;
        const int pw = zg * NPW + w;
        if (pw >= npairs) continue;  // 32-lane groups: uniform
        const int q = 2 * pw + (g >= GH ? 1 : 0);
        const size_t e0 = (size_t)q * a.ostride + (size_t)(kvh * GH + g % GH) * D + c;
        const float v = red[w * 8 * D + gd + (tid & 31)];
        if (a.out) a.out[e0 + (tid & 31)] = v;
        if (a.oq) quant_block32_lanes(v, a.oq + e0, a.os + e0 / 32, a.osum + e0 / 32);
    }
}

}  // namespace fl
