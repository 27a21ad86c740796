// Causal GQA attention for several consecutive query tokens over an fp16
// cache (speculative-verify and prefill passes).
//
// Same semantics as k_attm's query-pair mode (cpu_grouped_query_attention_into,
// flare-core/src/model.rs:9849-9966; causal prefill attention 336-368):
// query j of the pass sits at position *posp + j and attends slots
// 0 .. *posp + j.  The difference is the data flow: k_attm gives every query
// pair its own workgroup, each streaming the whole K/V prefix of its kv head,
// so a pass of M tokens reads the cache M/2 times.  Here one workgroup holds
// NPW query pairs and stages each 32-slot K/V block in LDS once for all of
// them:
//  * grid (split, kv head, pair group); the split's chunk of slots is walked
//    BW blocks per iteration, the next iterations' global loads in flight
//    (registers) while the waves compute on the current one (double-buffered
//    LDS, one workgroup barrier per iteration);
//  * NPW x BW waves: wave (block lane b, pair slot p) takes block b of every
//    iteration for pair p, with the fp16 MFMA scheme of k_attm (rows (query,
//    head, high / residual) of the pair's 2G heads, S = Q K^T and O += P V
//    on v_mfma_f32_16x16x32_f16, wave-private online softmax); the BW lanes
//    of a pair combine through LDS after the loop;
//  * splits publish (o, m, l) per pair with agent-scope stores; the last
//    arriving workgroup of a (pair group, kv head) merges them (weights per
//    row formed once, the loads of a batch of 8 splits all in flight) and
//    writes the f32 output and / or its Q8_0 copy.
#pragma once

#include "attm_kernels.h"

namespace fl {

constexpr int kAttqKPad = 8;  // halves of padding per staged K row
constexpr int kAttqVPad = 8;  // per staged V channel row

template <int D, int NPW, int BW>  // query pairs per workgroup, block lanes
struct AttqLds {
    static constexpr int KS = D + kAttqKPad, VS = 32 + kAttqVPad;
    static constexpr int KH = 32 * KS, VH = D * VS;  // halves per staged block
    static constexpr size_t LOOP = (size_t)2 * BW * (KH + VH) * 2;  // double-buffered K and V blocks
    static constexpr size_t SP = (size_t)NPW * BW * 8 * 32 * 4;      // p of the current block per wave
    static constexpr size_t RED = (size_t)NPW * 8 * D * 4;           // per-pair outputs (after the loop)
    static constexpr size_t WT = (size_t)NPW * 8 * kAttmMaxSplit * 4;  // merge weights
    static constexpr size_t COMB = (size_t)BW * NPW * 8 * (D + 2) * 4;  // block-lane states (after the loop)
    static constexpr size_t A = LOOP + SP > RED + WT ? LOOP + SP : RED + WT;
    static constexpr size_t BYTES = A > COMB ? A : COMB;
};

// G2 = rows of a query pair: the model's G heads of each of its 2 queries.
template <int D, int G2, int NPW, int BW>
__global__ __launch_bounds__(NPW * BW * 64) void k_attq(AttnArgs a) {
    constexpr int DT = D / 32, NT = D / 16, NW = NPW * BW, NTH = NW * 64, GH = G2 / 2;
    using L = AttqLds<D, NPW, BW>;
    constexpr int KS = L::KS, VS = L::VS;
    static_assert(G2 <= 8 && G2 % 2 == 0, "2G rows of a query pair (hi / lo) fill at most one MFMA tile");
    __shared__ __align__(16) char smem[L::BYTES];
    __shared__ int is_last;
    _Float16 *lk = (_Float16 *)smem;             // [2][BW][32][KS]
    _Float16 *lv = lk + 2 * BW * L::KH;          // [2][BW][D][VS]
    float *sp = (float *)(smem + L::LOOP);       // [NW][8][32]
    float *red = (float *)smem;                  // [NPW][8][D], after the loop
    float *wt = (float *)(smem + L::RED);        // [NPW][8][kAttmMaxSplit]
    float *comb = (float *)smem;                 // [BW][NPW][8][D + 2], after the loop

    const int kvh = blockIdx.y, s = blockIdx.x, zg = blockIdx.z, tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6, kg = lane >> 4, r = lane & 15;
    const int slot = wave % NPW, bl = wave / NPW;  // pair slot, block lane
    const int npairs = a.nq / 2, pw = zg * NPW + slot;
    const bool live = pw < npairs;                          // wave-uniform
    const int glast = 2 * min(npairs, (zg + 1) * NPW) - 1;  // last query of the group
    const int q0 = 2 * min(pw, npairs - 1);

    // query rows first (independent of the position)
    v4f_t qv[DT][2];
    {
        const int g = min(r >> 1, G2 - 1);
        const size_t qo = (size_t)(q0 + (g >= GH ? 1 : 0)) * a.qstride + (size_t)(kvh * GH + g % GH) * D;
        const v4f_t *qp = (const v4f_t *)(a.q + qo + 8 * kg);
#pragma unroll
        for (int dt = 0; dt < DT; dt++) {
            qv[dt][0] = qp[8 * dt];
            qv[dt][1] = qp[8 * dt + 1];
        }
    }
    const int base = __hip_atomic_load(a.posp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int Tg = base + glast + 1;  // slots the group's last query sees
    int CH = max(a.chmin, (Tg + a.nsplit - 1) / a.nsplit);
    CH = (CH + kAttmBlock - 1) / kAttmBlock * kAttmBlock;
    const int t0 = s * CH;
    if (t0 >= Tg) return;  // whole workgroup
    const int t1 = min(Tg, t0 + CH), nact = (Tg + CH - 1) / CH;
    const int nblk = (t1 - t0 + kAttmBlock - 1) / kAttmBlock, nit = (nblk + BW - 1) / BW;
    // rows of lane group kg: head rows 2kg + e; their query's last slot
    int lim[2];
#pragma unroll
    for (int e = 0; e < 2; e++) lim[e] = base + q0 + ((2 * kg + e) >= GH ? 1 : 0);
    const int wlim = base + q0 + 1;  // last slot any row of the wave sees

    // staging of iteration it: blocks it*BW .. it*BW + BW-1 of the chunk (K rows
    // [slot][D] and the transposed V block [D][32], both contiguous), 16 B per
    // thread and piece; block indices past the chunk are clamped (never read)
    constexpr int NP = 32 * D / 8, PPT = (NP * BW + NTH - 1) / NTH;
    const __half *kc = (const __half *)a.kc + (size_t)kvh * a.head_stride;
    const __half *vc = (const __half *)a.vc + (size_t)kvh * a.head_stride;
    v4i_t kr[2][PPT], vr[2][PPT];  // register set it & 1, loaded two iterations ahead
    auto gload = [&](v4i_t(&kk)[PPT], v4i_t(&vv)[PPT], int it) {
#pragma unroll
        for (int u = 0; u < PPT; u++) {
            const int i = min(tid + u * NTH, NP * BW - 1), bb = i / NP, j = i % NP;
            const int tb = t0 + min(it * BW + bb, nblk - 1) * kAttmBlock;
            kk[u] = ((const v4i_t *)(kc + (size_t)tb * D))[j];
            vv[u] = ((const v4i_t *)(vc + vt_off(tb, 0, D)))[j];
        }
    };
    auto lstore = [&](const v4i_t(&kk)[PPT], const v4i_t(&vv)[PPT], int buf) {
#pragma unroll
        for (int u = 0; u < PPT; u++) {
            const int i = tid + u * NTH, bb = i / NP, j = i % NP;
            if ((NP * BW) % NTH == 0 || i < NP * BW) {
                *(v4i_t *)(lk + (buf * BW + bb) * L::KH + (j / (D / 8)) * KS + 8 * (j % (D / 8))) = kk[u];
                *(v4i_t *)(lv + (buf * BW + bb) * L::VH + (j >> 2) * VS + 8 * (j & 3)) = vv[u];
            }
        }
    };
    gload(kr[0], vr[0], 0);
    if (nit > 1) gload(kr[1], vr[1], 1);

    // A operand of S: row m = 2g + (hi / lo) of head row g (rows >= 2 G2 zero)
    v8h_t aq[DT];
#pragma unroll
    for (int dt = 0; dt < DT; dt++) {
        const v4f_t x0 = qv[dt][0], x1 = qv[dt][1];
        float x[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        if ((r >> 1) >= G2) {
#pragma unroll
            for (int j = 0; j < 8; j++) x[j] = 0.0f;
        }
        v8h_t hi, lo;
        split8(x, hi, lo);
        aq[dt] = (r & 1) ? lo : hi;
    }
    const float scale = 1.0f / sqrtf((float)D);
    float m_run[2] = {-INFINITY, -INFINITY}, l_run[2] = {0.0f, 0.0f};
    v4f32_t oacc[NT];
#pragma unroll
    for (int nt = 0; nt < NT; nt++) oacc[nt] = v4f32_t{0.f, 0.f, 0.f, 0.f};
    float *spw = sp + wave * 8 * 32;

    lstore(kr[0], vr[0], 0);
    if (nit > 2) gload(kr[0], vr[0], 2);
    __syncthreads();
    // iteration it: block it*BW + bl from LDS buffer it & 1; then iteration
    // it + 1 (register set (it + 1) & 1) goes to the other buffer and that set
    // loads iteration it + 3
    auto iter = [&](int it, v4i_t(&kn)[PPT], v4i_t(&vn)[PPT]) {
        const int cur = it & 1, bi = it * BW + bl, tb = t0 + bi * kAttmBlock;
        if (live && bi < nblk && tb <= wlim) {  // wave-uniform: some row sees the block
            const _Float16 *bk = lk + (cur * BW + bl) * L::KH, *bv = lv + (cur * BW + bl) * L::VH;
            float sc[2][2];  // [half][head row parity] for slot tb + 16h + r
#pragma unroll
            for (int h = 0; h < 2; h++) {
                v4f32_t acc = v4f32_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int dt = 0; dt < DT; dt++)
                    acc = mfma16(aq[dt], *(const v8h_t *)(bk + (16 * h + r) * KS + 32 * dt + 8 * kg), acc);
                const int t = tb + 16 * h + r;
                sc[h][0] = t < t1 && t <= lim[0] ? (acc[0] + acc[1]) * scale : -INFINITY;
                sc[h][1] = t < t1 && t <= lim[1] ? (acc[2] + acc[3]) * scale : -INFINITY;
            }
            float alpha[2];
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const float bm = row_max<16>(fmaxf(sc[0][e], sc[1][e]));
                const float mn = fmaxf(m_run[e], bm);
                // a row that has seen nothing yet keeps m = -inf (and p = 0)
                alpha[e] = (m_run[e] == -INFINITY) ? 0.0f : __expf(m_run[e] - mn);
                const float p0 = sc[0][e] == -INFINITY ? 0.0f : __expf(sc[0][e] - mn);
                const float p1 = sc[1][e] == -INFINITY ? 0.0f : __expf(sc[1][e] - mn);
                l_run[e] = l_run[e] * alpha[e] + row_sum<16>(p0 + p1);
                m_run[e] = mn;
                const int g = 2 * kg + e;
                if (g < G2) {
                    spw[g * 32 + r] = p0;
                    spw[g * 32 + 16 + r] = p1;
                }
            }
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                oacc[nt][0] *= alpha[0];
                oacc[nt][1] *= alpha[0];
                oacc[nt][2] *= alpha[1];
                oacc[nt][3] *= alpha[1];
            }
            {
                const int g = r >> 1;
                float pv[8];
#pragma unroll
                for (int j = 0; j < 8; j++) pv[j] = g < G2 ? spw[g * 32 + 8 * kg + j] : 0.0f;
                v8h_t hi, lo;
                split8(pv, hi, lo);
                const v8h_t ap = (r & 1) ? lo : hi;
#pragma unroll
                for (int nt = 0; nt < NT; nt++)
                    oacc[nt] = mfma16(ap, *(const v8h_t *)(bv + (16 * nt + r) * VS + 8 * kg), oacc[nt]);
            }
            __builtin_amdgcn_wave_barrier();
        }
        if (it + 1 < nit) {
            lstore(kn, vn, cur ^ 1);
            if (it + 3 < nit) gload(kn, vn, it + 3);
        }
        __syncthreads();
    };
    for (int it = 0; it < nit; it += 2) {
        iter(it, kr[1], vr[1]);
        if (it + 1 < nit) iter(it + 1, kr[0], vr[0]);
    }

    // combine the BW block lanes of each pair (head row g = 2kg + e, channel
    // 16nt + r; rows 4kg + 2e / + 1 of oacc: high / residual parts of P)
    float o_fin[2][NT];
#pragma unroll
    for (int e = 0; e < 2; e++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++) o_fin[e][nt] = oacc[nt][2 * e] + oacc[nt][2 * e + 1];
    if constexpr (BW > 1) {
        float *cw = comb + (size_t)(bl * NPW + slot) * 8 * (D + 2);
        if (live) {
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const int g = 2 * kg + e;
                if (g < G2) {
#pragma unroll
                    for (int nt = 0; nt < NT; nt++) cw[g * (D + 2) + 16 * nt + r] = o_fin[e][nt];
                    if (r == 0) {
                        cw[g * (D + 2) + D] = m_run[e];
                        cw[g * (D + 2) + D + 1] = l_run[e];
                    }
                }
            }
        }
        __syncthreads();
        if (bl == 0 && live) {
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const int g = 2 * kg + e;
                if (g < G2) {
                    float M = -INFINITY;
#pragma unroll
                    for (int b = 0; b < BW; b++) M = fmaxf(M, comb[(size_t)((b * NPW + slot) * 8 + g) * (D + 2) + D]);
                    float Ls = 0.0f, wb[BW];
#pragma unroll
                    for (int b = 0; b < BW; b++) {
                        const float *cb = comb + (size_t)((b * NPW + slot) * 8 + g) * (D + 2);
                        wb[b] = cb[D] == -INFINITY ? 0.0f : __expf(cb[D] - M);
                        Ls += cb[D + 1] * wb[b];
                    }
#pragma unroll
                    for (int nt = 0; nt < NT; nt++) {
                        float o = 0.0f;
#pragma unroll
                        for (int b = 0; b < BW; b++)
                            o += comb[(size_t)((b * NPW + slot) * 8 + g) * (D + 2) + 16 * nt + r] * wb[b];
                        o_fin[e][nt] = o;
                    }
                    m_run[e] = M;
                    l_run[e] = Ls;
                }
            }
        }
        __syncthreads();  // comb is rewritten below (red aliases it)
    }

    // per-pair result (block lane 0 holds the combined state)
    constexpr int P = G2 * (D + 2);
    float *gpart = a.part + ((size_t)zg * a.nkv + kvh) * a.nsplit * NPW * P;  // this (group, kv head)
    if (bl == 0 && live) {
        float *mypart = gpart + ((size_t)s * NPW + slot) * P;
        float *rw = red + slot * 8 * D;
#pragma unroll
        for (int e = 0; e < 2; e++) {
            const int g = 2 * kg + e;
            if (g < G2) {
                const float il = nact == 1 ? 1.0f / l_run[e] : 1.0f;
#pragma unroll
                for (int nt = 0; nt < NT; nt++) {
                    if (nact == 1) rw[g * D + 16 * nt + r] = o_fin[e][nt] * il;
                    else st_agent(mypart + g * D + 16 * nt + r, o_fin[e][nt]);
                }
                if (nact > 1 && r == 0) {
                    st_agent(mypart + G2 * D + 2 * g, m_run[e]);
                    st_agent(mypart + G2 * D + 2 * g + 1, l_run[e]);
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
        constexpr int NO = NPW * G2 * D;  // outputs of the group
        constexpr int CK = NO / NTH < 1 ? 1 : NO / NTH < 8 ? NO / NTH : 8;  // per thread and chunk
        for (int c0 = 0; c0 < NO; c0 += NTH * CK) {
            float O[CK];
#pragma unroll
            for (int k = 0; k < CK; k++) O[k] = 0.0f;
            for (int j0 = 0; j0 < nact; j0 += 8) {
                float ov[CK][8];
#pragma unroll
                for (int k = 0; k < CK; k++) {
                    const int i = min(c0 + k * NTH + tid, NO - 1), w = i / (G2 * D), gd = i % (G2 * D);
#pragma unroll
                    for (int u = 0; u < 8; u++)
                        ov[k][u] = ld_agent(gpart + ((size_t)min(j0 + u, nact - 1) * NPW + w) * P + gd);
                }
#pragma unroll
                for (int k = 0; k < CK; k++) {
                    const int i = min(c0 + k * NTH + tid, NO - 1), w = i / (G2 * D), g = (i % (G2 * D)) / D;
                    const float *wr = wt + (w * 8 + g) * kAttmMaxSplit;
#pragma unroll
                    for (int u = 0; u < 8; u++)
                        if (j0 + u < nact) O[k] += ov[k][u] * wr[j0 + u];
                }
            }
#pragma unroll
            for (int k = 0; k < CK; k++) {
                const int i = c0 + k * NTH + tid, w = i / (G2 * D), gd = i % (G2 * D);
                if (i < NO && zg * NPW + w < npairs) red[w * 8 * D + gd] = O[k];
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
