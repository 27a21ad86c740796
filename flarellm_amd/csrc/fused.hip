// Fused QKV + attention launch of the decode step (fp16 KV cache).
//
// The attention of a decode step reads the layer's whole K / V cache, which
// does not depend on the step's new token; only q and the new token's K / V
// row do.  One launch holds both:
//  * workgroups [0, nqwg): the fused QKV matvec (norm prologue, RoPE
//    epilogue, cache store of the new K / V row), the workgroups of kv head h
//    walking the row groups of h's query, key and value rows (RowsKvGroup).
//    They publish q and the new K / V rows (f32, agent-scope stores), wait
//    for their own stores, and count one arrival on count[h];
//  * workgroups [nqwg, nqwg + nsplit * nkv): the split attention
//    (attm_body), which issues its first K / V block, waits until count[h]
//    reaches the number of QKV workgroups of h, then reads q and patches the
//    new token's K / V from the published rows.
// So the K / V stream of attention overlaps the QKV matvec, and the step
// loses one kernel boundary.  The values and their order of operations are
// those of the two separate kernels (k_mvs EPI_QKV, k_attm), so the outputs
// are identical.
//
// Forward progress: workgroups are dispatched in index order on each XCD
// (the QKV workgroups of kv head h are h, h + nkv, ..., so with nkv a
// multiple of 8 they and the attention workgroups of h share XCD h), and a
// QKV workgroup never waits, so every QKV workgroup is dispatched and
// finishes whatever the attention workgroups hold.  The attention wait is
// bounded (kFuseSpinLimit polls; on timeout it sets *err and goes on).
#include "attm_kernels.h"
#include "launch.h"
#include "mvs_kernels.h"

namespace fl {

template <int FMT, int R, int SU, int RX, int D, int G, int NT>
__global__ __launch_bounds__(NT) void k_qkv_attm(MvsArgs m, AttnArgs at, int nqwg, FuseWait fw) {
    extern __shared__ __align__(16) char smem[];
    constexpr int NW = NT / 64;
    const int b = (int)blockIdx.x, nkv = at.nkv;
    if (b < nqwg) {
        const int h = b % nkv, j = b / nkv, per = nqwg / nkv;
        RowsKvGroup map;
        map.h = h;
        map.R = R;
        map.nq = m.qkv.nq;
        map.nk = m.qkv.nk;
        map.qg = (m.qkv.nq / nkv) / R;
        map.kg = D / R;
        map.ngrp = map.qg + 2 * map.kg;
        mvs_body<FMT, false, R, SU, RX, false, NT>(m, smem, j * NW + (int)(threadIdx.x >> 6), per * NW, map);
        // every wave's agent-scope stores have completed (vmcnt counts stores
        // on gfx9), then one relaxed agent-scope arrival; the readers' loads
        // are agent-scope loads issued after they see the count
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (threadIdx.x == 0) __hip_atomic_fetch_add(fw.count + h, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    const int ab = b - nqwg;
    attm_body<__half, D, G, NT, true>(at, ab / nkv, ab % nkv, 0, fw);
}

// (FMT, R, SU, RX, D, G, NT) instantiations: the Llama-3.2-1B Q8_0 and
// Llama-3-8B Q4_K decode plans.
hipError_t launch_qkv_attm(int fmt, const MvsPlan &p, int rx, int D, int G, int nt, hipStream_t st,
                           const MvsArgs &m, const AttnArgs &at, int nqwg, const FuseWait &fw) {
    const dim3 grid(nqwg + at.nsplit * at.nkv);
#define C(FF, RR, SS, XX, DD, GG, NN)                                                                          \
    if (fmt == FF && p.r == RR && p.su == SS && rx == XX && D == DD && G == GG && nt == NN) {                 \
        hipLaunchKernelGGL((k_qkv_attm<FF, RR, SS, XX, DD, GG, NN>), grid, dim3(NN), p.lds, st, m, at, nqwg, fw); \
        return hipGetLastError();                                                                              \
    }
    C(F_Q8_0, 4, 2, 1, 64, 4, 256)
    C(F_Q4K, 4, 1, 0, 128, 4, 512)
#undef C
    return hipErrorNotSupported;
}

}  // namespace fl
