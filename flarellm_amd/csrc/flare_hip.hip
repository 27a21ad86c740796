// flare_hip.hip -- MI355X (gfx950) decode backend for flarellm: kernels and
// the C-ABI declared in include/flare_hip.h.
//
// Decode step = one HIP graph (captured once, replayed per token):
//   embed      token select (prompt or previous argmax) + embedding row dequant
//   per layer: qkv      RMSNorm+Q8 quantize prologue, fused [wq;wk;wv] matvec
//              attn     RoPE(q,k) + KV store + split-K online softmax with a
//                       last-workgroup merge that also Q8-quantizes the output
//              wo       matvec + residual add into x
//              gate_up  RMSNorm+Q8 prologue, [w_gate;w_up] matvec, SiLU*up and
//                       Q8 quantize epilogue
//              down     matvec + residual add into x
//   out        final RMSNorm prologue, output matvec with fused argmax
// Every kernel reads the token position from device memory, so replays need
// no host work.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/flare_hip.h"
#include "kernels.h"
#include "attm_kernels.h"
#include "launch.h"
#include "mvo_kernels.h"
#include "sample_args.h"

using namespace fl;

// =====================================================================
// Kernels
// =====================================================================

__global__ __launch_bounds__(kThreads) void k_quantize(const float *x, int nblk, int8_t *q,
                                                       float *s, int *sums) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblk) return;
    float v[32];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        v4f_t t = ((const v4f_t *)(x + b * 32))[j];
        v[4 * j] = t.x; v[4 * j + 1] = t.y; v[4 * j + 2] = t.z; v[4 * j + 3] = t.w;
    }
    quant_block32(v, q + b * 32, s + b, sums + b);
}

template <int PRO, bool SEQ>
__global__ __launch_bounds__(kThreads) void k_norm_quant(const float *x, const float *w, int n,
                                                         float eps, int8_t *q, float *s, int *sums) {
    __shared__ float red[8];
    __shared__ float ess[SEQ ? kEssLdsWords + 1 : 1];
    stage_q8<PRO, SEQ>(x, w, eps, n, nullptr, nullptr, nullptr, q, s, sums, red, SEQ ? ess : nullptr);
}

__global__ __launch_bounds__(kThreads) void k_rmsnorm(const float *x, const float *w, int n,
                                                      float eps, float *out) {
    __shared__ float red[8];
    const float inv = wg_inv_rms(x, n, eps, red);
    for (int i = threadIdx.x; i < n; i += blockDim.x) out[i] = (x[i] * inv) * w[i];
}

// Per-block integer dots (parity surface).  One thread per unit.
template <int FMT>
__global__ __launch_bounds__(kThreads) void k_block_dots(WDesc W, const int8_t *xq, int *dots) {
    if (FMT == F_Q8_0) {
        const int bpr = W.cols >> 5;
        const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
        if (i >= (long long)W.rows * bpr) return;
        const int row = (int)(i / bpr), b = (int)(i % bpr);
        const v4i_t *p = (const v4i_t *)(W.q + (size_t)row * W.cols + b * 32);
        const v4i_t *xp = (const v4i_t *)(xq + b * 32);
        dots[i] = dot16(p[1], xp[1], dot16(p[0], xp[0], 0));
    } else {
        const int nsb = W.cols >> 8;
        const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
        if (i >= (long long)W.rows * nsb * 4) return;
        const int sub = (int)(i & 3);
        const long long rs = i >> 2;
        const int row = (int)(rs / nsb), sb = (int)(rs % nsb);
        const uint8_t *qs = W.q + ((size_t)row * nsb + sb) * 128;
        const v4i_t a = *(const v4i_t *)(qs + 32 * sub), c = *(const v4i_t *)(qs + 16 + 32 * sub);
        const int blo = sb * 8 + sub, bhi = blo + 4;
        const v4i_t *xl = (const v4i_t *)(xq + blo * 32), *xh = (const v4i_t *)(xq + bhi * 32);
        const v4i_t lo0 = v4i_t{a.x & 0x0F0F0F0F, a.y & 0x0F0F0F0F, a.z & 0x0F0F0F0F, a.w & 0x0F0F0F0F};
        const v4i_t lo1 = v4i_t{c.x & 0x0F0F0F0F, c.y & 0x0F0F0F0F, c.z & 0x0F0F0F0F, c.w & 0x0F0F0F0F};
        const v4i_t hi0 = v4i_t{(a.x >> 4) & 0x0F0F0F0F, (a.y >> 4) & 0x0F0F0F0F,
                                   (a.z >> 4) & 0x0F0F0F0F, (a.w >> 4) & 0x0F0F0F0F};
        const v4i_t hi1 = v4i_t{(c.x >> 4) & 0x0F0F0F0F, (c.y >> 4) & 0x0F0F0F0F,
                                   (c.z >> 4) & 0x0F0F0F0F, (c.w >> 4) & 0x0F0F0F0F};
        dots[rs * 8 + 2 * sub] = dot16(lo1, xl[1], dot16(lo0, xl[0], 0));
        dots[rs * 8 + 2 * sub + 1] = dot16(hi1, xh[1], dot16(hi0, xh[0], 0));
    }
}

// Dequantize (dequantize_tensor, gguf.rs:717-880) one 32-value group per thread.
template <int FMT>
__global__ __launch_bounds__(kThreads) void k_dequant(WDesc W, float *out) {
    const long long g = (long long)blockIdx.x * blockDim.x + threadIdx.x;  // 32-value group
    const int gpr = W.cols >> 5;
    if (g >= (long long)W.rows * gpr) return;
    const int row = (int)(g / gpr), j = (int)(g % gpr);
    float *o = out + (size_t)row * W.cols + (size_t)j * 32;
    if (FMT == F_Q8_0) {
        const float scale = h2f(W.s[(size_t)row * gpr + j]);
        const int8_t *q = (const int8_t *)W.q + (size_t)row * W.cols + j * 32;
        for (int k = 0; k < 32; k++) o[k] = (float)q[k] * scale;
    } else if (FMT == F_Q4K) {
        for (int k = 0; k < 32; k++) o[k] = q4k_elem(W, row, j * 32 + k);
    } else if (FMT == F_Q6K) {
        for (int k = 0; k < 32; k++) o[k] = q6k_elem(W, row, j * 32 + k);
    } else {
        const float *src = (const float *)W.q + (size_t)row * W.cols + j * 32;
        for (int k = 0; k < 32; k++) o[k] = src[k];
    }
}

// apply_rope_with_table, x86 branch (model.rs:7283-7296).
__global__ __launch_bounds__(kThreads) void k_rope(float *data, int num_heads, int head_dim,
                                                   const float *cs, const float *sn) {
    const int half = head_dim / 2;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= num_heads * half) return;
    const int h = i / half, d = i % half;
    float *p = data + h * head_dim;
    const float c = cs[d], s = sn[d], x0 = p[d], x1 = p[d + half];
    p[d] = x0 * c - x1 * s;
    p[d + half] = x0 * s + x1 * c;
}

__global__ __launch_bounds__(kThreads) void k_silu_mul(const float *g, const float *u, int n,
                                                       float *out) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float gv = g[i];
    out[i] = (gv / (1.0f + fl_expf(-gv))) * u[i];
}

// Decode-step head: choose the token (prompt slot or previous argmax) and
// dequantize its embedding row into x (token_embedding lookup, model.rs:1964).
// d_counters: split-merge arrival counters [0, 1024), then the fused
// QKV + attention launch's per-kv-head arrival counts [1024, 1056) and its
// wait-timeout flag (1056)
constexpr int kFuseCount = 1024, kFuseErr = 1056, kCounterWords = 1088;

struct DevState {
    int step;     // next step to run
    int pos;      // position of the step in flight
    int n_prompt; // steps < n_prompt read tokens[step]
    int pad;
    unsigned long long argmax;
};

__device__ __forceinline__ uint32_t key_index(unsigned long long k) {
    return 0xFFFFFFFFu - (uint32_t)(k & 0xFFFFFFFFull);
}

// Also writes the RoPE (cos, sin) row of the step's position (RopeTable,
// model.rs:7190-7212) to rope_cur, read by the QKV epilogues of every layer.
// One workgroup of kEmbedThreads (few elements per thread: the dequant loads
// of each element are a dependent chain).
constexpr int kEmbedThreads = 1024;
template <int FMT>
// x == nullptr: the embedding row is already in the residual buffer (a caller
// that passes the f32 embedding, forward_single_token_gpu model.rs:555).
__global__ __launch_bounds__(kEmbedThreads) void k_embed(WDesc E, DevState *st, int *tokens, float *x, const float *rope,
                                                   long long sin_off, int half, float *rope_cur) {
    __shared__ int tok_s, step_s;
    if (threadIdx.x == 0) {
        const int s = st->step;
        int tok;
        if (s < st->n_prompt) {
            tok = tokens[s];
        } else {
            tok = (int)key_index(st->argmax);
            tokens[s] = tok;
        }
        tok = min(max(tok, 0), E.rows - 1);
        tok_s = tok;
        step_s = s;
    }
    __syncthreads();
    const int row = tok_s, H = E.cols;
    for (int i = threadIdx.x; x && i < H; i += blockDim.x) {
        float v;
        if (FMT == F_Q8_0) {
            v = (float)((const int8_t *)E.q)[(size_t)row * H + i] * h2f(E.s[(size_t)row * (H >> 5) + (i >> 5)]);
        } else if (FMT == F_Q6K) {
            v = q6k_elem(E, row, i);
        } else if (FMT == F_Q4K) {
            v = q4k_elem(E, row, i);
        } else {
            v = ((const float *)E.q)[(size_t)row * H + i];
        }
        x[i] = v;
    }
    for (int i = threadIdx.x; i < half; i += blockDim.x) {
        rope_cur[i] = rope[(size_t)step_s * half + i];
        rope_cur[half + i] = rope[sin_off + (size_t)step_s * half + i];
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        st->pos = step_s;
        st->step = step_s + 1;
        st->argmax = 0ull;
    }
}

// =====================================================================
// Host side
// =====================================================================

struct fl_weight {
    int format = 0, rows = 0, cols = 0;
    void *q = nullptr;      // device planes (see WDesc)
    void *s = nullptr;
    void *h = nullptr;
    void *h2 = nullptr;
    size_t plane_bytes[4] = {0, 0, 0, 0};  // q, s, h, h2
    size_t gguf_bytes = 0;  // algorithmic bytes (GGUF size)
    WDesc desc() const {
        WDesc d;
        d.q = (const uint8_t *)q;
        d.s = (const uint16_t *)s;
        d.h = (const uint8_t *)h;
        d.h2 = (const uint8_t *)h2;
        d.rows = rows;
        d.cols = cols;
        return d;
    }
};

struct Layer {
    fl_weight qkv, wo, gu, down;
    float *attn_norm = nullptr, *ffn_norm = nullptr;
};

struct fl_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    std::string err;
    // op scratch
    int *d_pos = nullptr;
    float *d_rope_row = nullptr;  // [2*256]
    float *d_part = nullptr;
    size_t part_cap = 0;
    int *d_counters = nullptr;    // [kCounterWords]: split arrivals [0, 1024), fused-launch counts and flag after
    unsigned long long *d_slot = nullptr;
    // model
    bool have_cfg = false, have_weights = false;
    fl_model_config cfg{};
    int kv_format = FL_KV_F16;
    int layer_fmt = FL_Q8_0;
    std::vector<Layer> layers;
    fl_weight embed, output;
    bool tied = true;
    float *out_norm = nullptr;
    void *kcache = nullptr, *vcache = nullptr;  // values (F32/F16) or codes (Q8/KIVI)
    size_t kv_layer_elems = 0;                  // elements (F32/F16) or code bytes (Q8/KIVI) per layer
    int kv_slots = 0;                           // slots per kv head (max_seq; a multiple of 32 for Q8/KIVI)
    uint16_t *kscale = nullptr, *vscale = nullptr;  // Q8 scales [L][nkv][S][D/32]
    uint32_t *kparam = nullptr, *vparam = nullptr;  // KIVI (scale, min): K [L][nkv][S/32][D], V [L][nkv][S][D/32]
    __half *kring = nullptr, *vring = nullptr;      // KIVI fp16 ring [L][nkv][kKiviRing][D]
    float *kvstage = nullptr;                       // host rows staged for fl_kv_write(_batch): 2 x cap x nkv*D
    size_t kvstage_rows = 0;
    float *rope = nullptr;
    int nsplit = 1, chmin = 1, single = kAttmSingle, attn_waves = 8;
    bool fuse_attn = false;  // FL_OPT_FUSE_ATTN
    int ncu = 256;  // compute units of the device (fl_model_init)
    // activations
    float *x = nullptr, *qkv = nullptr, *attn = nullptr, *logits = nullptr;
    float *bench_out = nullptr;  // output of fl_bench_layer_kernel launches
    long long *bench_trace = nullptr;  // attention phase timestamps (FLARE_ATTN_TRACE builds)
    float *rope_cur = nullptr;         // RoPE (cos, sin) of the step in flight [D]
    int8_t *aq = nullptr, *hq = nullptr;
    float *as = nullptr, *hs = nullptr;
    int *asum = nullptr, *hsum = nullptr;
    DevState *st = nullptr;
    int *tokens = nullptr;
    hipGraph_t graph = nullptr;
    std::map<int, hipGraphExec_t> vgraphs;  // captured verify passes, by batch size
    hipGraphExec_t gexec = nullptr;
    bool graph_ready = false;
    // speculative verify buffers (allocated on first fl_verify)
    bool have_verify = false;
    float *vx = nullptr, *vx2 = nullptr, *vq = nullptr, *vk = nullptr, *vv = nullptr, *vpart = nullptr;
    int8_t *vxq = nullptr, *vaq = nullptr, *vhq = nullptr;  // vhq: Q8_0 of the hidden vector (fused SiLU)
    float *vxs = nullptr, *vas = nullptr, *vhs = nullptr;
    int *vxsum = nullptr, *vasum = nullptr, *vhsum = nullptr;
    int *vcnt = nullptr;  // arrival counters of the fused verify GEMM epilogues
    int *vtok = nullptr, *vpos = nullptr;
    unsigned long long *vslots = nullptr;
    size_t vpart_floats = 0;
    // fl_set_option switches (measurement / testing)
    bool verify_fuse = true, verify_graph = true;
    // FL_OPT_EXACT: the decode step in the reference's floating-point order
    bool exact = false;
    float *scratch = nullptr;     // device address of `scratch` on this context's GPU
    float *seq_scores = nullptr;  // [num_heads][kv_slots] attention scores (exact mode)
    float *seq_xn = nullptr;      // [hidden] final-normed vector (exact mode)
    // layer probe (fl_probe_layer): intermediates of one layer of the step
    int probe_layer = -1;
    char *probe_dev = nullptr;
    void *probe_host = nullptr;
    size_t probe_bytes = 0;
    // device sampler (allocated on first use, for rows of up to sample_cap)
    int sample_cap = 0, sample_prev_cap = 0;
    float *sp = nullptr;
    int *scounts = nullptr, *sprev = nullptr, *sstate = nullptr, *svals = nullptr, *ssvals = nullptr;
    unsigned *skeys = nullptr, *sskeys = nullptr;
    void *ssort = nullptr;
    size_t ssort_bytes = 0;
};

constexpr int kVerifyMaxKsplit = 16;
constexpr int kVerifyCounters = 4096;  // workgroup columns of a fused verify GEMM

// K-split partials of fl_op_batched_matvec_q8in_noalloc: a file-scope device
// array (each GPU holds its own copy for the life of the process), 16 MiB.
// Host code uses its device address from hipGetSymbolAddress (fl_ctx::scratch),
// never the array's name.
constexpr size_t kNoAllocScratchFloats = (size_t)4 << 20;
static __device__ __align__(256) float scratch[kNoAllocScratchFloats];

static std::string g_err;
static thread_local char g_errbuf[512];

static int fail(fl_ctx *ctx, int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_errbuf, sizeof g_errbuf, fmt, ap);
    va_end(ap);
    if (ctx) ctx->err = g_errbuf;
    g_err = g_errbuf;
    return code;
}

int fl_host_fail(fl_ctx *ctx, int code, const char *msg) { return fail(ctx, code, "%s", msg); }

#define HIPCHK(ctx, expr)                                                                   \
    do {                                                                                    \
        hipError_t e_ = (expr);                                                             \
        if (e_ != hipSuccess)                                                               \
            return fail((ctx), FL_E_HIP, "%s failed: %s (%s:%d)", #expr, hipGetErrorString(e_), \
                        __FILE__, __LINE__);                                                \
    } while (0)

static int dev_alloc(fl_ctx *ctx, void **p, size_t bytes) {
    if (bytes == 0) bytes = 16;
    hipError_t e = hipMalloc(p, bytes);
    if (e != hipSuccess) return fail(ctx, FL_E_OOM, "hipMalloc(%zu) failed: %s", bytes, hipGetErrorString(e));
    return 0;
}
#define ALLOC(ctx, ptr, bytes)                                            \
    do {                                                                  \
        int rc_ = dev_alloc((ctx), (void **)&(ptr), (bytes));             \
        if (rc_) return rc_;                                              \
    } while (0)

static void weight_release(fl_weight &w) {
    for (void *p : {w.q, w.s, w.h, w.h2})
        if (p) (void)hipFree(p);
    w.q = w.s = w.h = w.h2 = nullptr;
}

static size_t row_bytes(int fmt, int cols) { return fl_format_row_bytes(fmt, (size_t)cols); }

static int weight_cols(const fl_raw_weight *w) {
    switch (w->format) {
    case FL_F32: return w->blocks_per_row;
    case FL_Q8_0: return w->blocks_per_row * 32;
    case FL_Q4K:
    case FL_Q6K: return w->blocks_per_row * 256;
    }
    return 0;
}

// Upload `n` RawWeights sharing format and cols as one row-concatenated
// device weight (Model::set_raw_weights fusion, model.rs:1411-1452).
// Pair-interleave the rows of each head (row 2i <- row i, row 2i+1 <- row
// i + D/2) so the rotate-half pairs of RoPE are adjacent rows (EPI_QKV).
static std::vector<uint8_t> pair_rows(const fl_raw_weight &w, int hd) {
    const size_t rb = row_bytes(w.format, weight_cols(&w)), rows = (size_t)w.num_rows, half = hd / 2;
    std::vector<uint8_t> out(rows * rb);
    const uint8_t *src = (const uint8_t *)w.data;
    for (size_t r = 0; r < rows; r++) {
        const size_t h = r / hd, j = r % hd;
        const size_t dst = h * hd + (j < half ? 2 * j : 2 * (j - half) + 1);
        std::memcpy(&out[dst * rb], src + r * rb, rb);
    }
    return out;
}

static int upload_concat(fl_ctx *ctx, const fl_raw_weight *const *ws_in, int n, fl_weight &out, int npair = 0,
                         int hd = 0) {
    // the first npair weights get their head rows pair-interleaved
    std::vector<std::vector<uint8_t>> keep;
    fl_raw_weight tmp[8];
    const fl_raw_weight *ws[8];
    if (n > 8) return fail(ctx, FL_E_INVALID, "too many fused weights");
    for (int i = 0; i < n; i++) {
        ws[i] = ws_in[i];
        if (i < npair && ws_in[i] && ws_in[i]->data) {
            if (ws_in[i]->num_rows % hd) return fail(ctx, FL_E_INVALID, "q/k rows not a multiple of head_dim");
            const size_t rb = row_bytes(ws_in[i]->format, weight_cols(ws_in[i]));
            if (rb == 0 || ws_in[i]->nbytes < rb * (size_t)ws_in[i]->num_rows)
                return fail(ctx, FL_E_INVALID, "weight bytes %zu < rows*row_bytes", ws_in[i]->nbytes);
            keep.push_back(pair_rows(*ws_in[i], hd));
            tmp[i] = *ws_in[i];
            tmp[i].data = keep.back().data();
            ws[i] = &tmp[i];
        }
    }
    const int fmt = ws[0]->format, cols = weight_cols(ws[0]);
    int rows = 0;
    for (int i = 0; i < n; i++) {
        if (!ws[i] || !ws[i]->data) return fail(ctx, FL_E_INVALID, "null weight");
        if (ws[i]->format != fmt || weight_cols(ws[i]) != cols)
            return fail(ctx, FL_E_INVALID, "fused weights must share format and columns");
        const size_t need = row_bytes(fmt, cols) * (size_t)ws[i]->num_rows;
        if (need == 0 || ws[i]->nbytes < need)
            return fail(ctx, FL_E_INVALID, "weight bytes %zu < rows*row_bytes %zu (format %d, cols %d)",
                        ws[i]->nbytes, need, fmt, cols);
        rows += ws[i]->num_rows;
    }
    if (fmt != FL_Q8_0 && fmt != FL_Q4K && fmt != FL_Q6K && fmt != FL_F32)
        return fail(ctx, FL_E_UNSUPPORTED, "weight format %d not supported", fmt);
    if (fmt == FL_F32 && cols % 4) return fail(ctx, FL_E_INVALID, "f32 cols must be a multiple of 4");
    out.format = fmt;
    out.rows = rows;
    out.cols = cols;
    out.gguf_bytes = row_bytes(fmt, cols) * (size_t)rows;
    const size_t R = (size_t)rows;
    // Split every GGUF block into per-field planes, each [rows][blocks][len]:
    //   Q8_0 (34 B):  s = f16 scale [0,2), q = quants [2,34)
    //   Q4_K (144 B): h = d, dmin, scales [0,16), q = qs [16,144)
    //   Q6_K (210 B): q = ql [0,128), h = qh [128,192), h2 = scales [192,208), s = d [208,210)
    //   F32:          q = the row
    struct Seg {
        void **plane;
        int off, len;
    };
    std::vector<Seg> segs;
    size_t nblk, bsz;
    if (fmt == FL_Q8_0) {
        nblk = (size_t)cols / 32, bsz = 34;
        segs = {{&out.s, 0, 2}, {&out.q, 2, 32}};
    } else if (fmt == FL_Q4K) {
        nblk = (size_t)cols / 256, bsz = 144;
        segs = {{&out.h, 0, 16}, {&out.q, 16, 128}};
    } else if (fmt == FL_Q6K) {
        nblk = (size_t)cols / 256, bsz = 210;
        segs = {{&out.q, 0, 128}, {&out.h, 128, 64}, {&out.h2, 192, 16}, {&out.s, 208, 2}};
    } else {
        nblk = 1, bsz = (size_t)cols * 4;
        segs = {{&out.q, 0, (int)bsz}};
    }
    for (const Seg &g : segs) {
        ALLOC(ctx, *g.plane, R * nblk * (size_t)g.len);
        const int pi = g.plane == &out.q ? 0 : (g.plane == &out.s ? 1 : (g.plane == &out.h ? 2 : 3));
        out.plane_bytes[pi] = R * nblk * (size_t)g.len;
    }
    std::vector<uint8_t> host;
    size_t row_base = 0;
    for (int i = 0; i < n; i++) {
        const size_t r = (size_t)ws[i]->num_rows, nb = r * nblk;
        const uint8_t *src = (const uint8_t *)ws[i]->data;
        for (const Seg &g : segs) {
            host.resize(nb * (size_t)g.len);
#pragma omp parallel for schedule(static)
            for (long long k = 0; k < (long long)nb; k++)
                std::memcpy(&host[(size_t)k * g.len], src + (size_t)k * bsz + g.off, (size_t)g.len);
            HIPCHK(ctx, hipMemcpy((uint8_t *)*g.plane + row_base * nblk * g.len, host.data(), host.size(),
                                  hipMemcpyHostToDevice));
        }
        row_base += r;
    }
    return 0;
}

// ---- launches ---------------------------------------------------------------

#ifdef FLARE_MV_TRACE
// trace builds: FLARE_MV_TRACE_LAYER = l records the QKV launch of layer l of
// the decode step only (graph replays included)
static bool g_trace_off = false;
#endif
static MvsArgs mvs_args(fl_ctx *ctx, const fl_weight &w, int pro, int epi, const float *x, const float *nw,
                        float eps, const int8_t *q, const float *s, const int *sums, float *out,
                        unsigned long long *slot) {
    MvsArgs a{};
    a.W = w.desc();
    a.pro = pro;
    a.epi = epi;
    a.x = x;
    a.nw = nw;
    a.eps = eps;
    a.gq = q;
    a.gs = s;
    a.gsum = sums;
    a.out = out;
    a.slot = slot;
    a.trace = ctx->bench_trace;
#ifdef FLARE_MV_TRACE
    if (g_trace_off) a.trace = nullptr;
#endif
    return a;
}

static int mvs_result(fl_ctx *ctx, hipError_t e, const MvsPlan &p) {
    if (e == hipErrorNotSupported)
        return fail(ctx, FL_E_UNSUPPORTED, "no matvec kernel for plan r=%d su=%d", p.r, p.su);
    HIPCHK(ctx, e);
    HIPCHK(ctx, hipGetLastError());
    return 0;
}

// Q8-input matvec (Q8_0 / Q4_K weights): prologue pro, epilogue epi.
static int launch_q8in(fl_ctx *ctx, const fl_weight &w, int pro, int epi, const float *x,
                       const float *nw, float eps, const int8_t *q, const float *s, const int *sums,
                       float *out, unsigned long long *slot, const QkvEpi *qe = nullptr) {
    if (pro == PRO_LOADQ && w.cols > 4 * 16 * kMvsThreads)
        return fail(ctx, FL_E_UNSUPPORTED, "quantized input of %d columns is too wide", w.cols);
    const MvsPlan p = mvs_plan(w.format, w.rows, w.cols, false, epi == EPI_QKV);
    MvsArgs a = mvs_args(ctx, w, pro, epi, x, nw, eps, q, s, sums, out, slot);
    a.seq = ctx->exact;
    if (epi == EPI_QKV) {
        if (!qe) return fail(ctx, FL_E_INVALID, "EPI_QKV without its arguments");
        if (w.rows != qe->nq + 2 * qe->nk || qe->nq % qe->hd || qe->nk % qe->hd)
            return fail(ctx, FL_E_INVALID, "fused QKV rows %d do not match the heads", w.rows);
        a.qkv = *qe;  // every plan has an even R
    }
    hipError_t e;
    if (w.format == FL_Q8_0) e = launch_mvs_q8_0(false, p, ctx->stream, a);
    else if (w.format == FL_Q4K) e = launch_mvs_q4k(p, ctx->stream, a);
    else return fail(ctx, FL_E_UNSUPPORTED, "no Q8-input matvec for format %d", w.format);
    return mvs_result(ctx, e, p);
}

// f32-input matvec (Q8_0 / Q6_K / f32 weights): pro 0 copies x, 1 = rmsnorm_into.
// Several tokens (speculative verify) over Q6_K / Q8_0 weights: the MFMA
// kernel (rows of M tokens at x, x + cols, ..., argmax keys at slot[0..M)),
// which dequantizes each weight once for all M tokens.  One token: the
// streaming kernel (per-block scale work dominates either way, and the
// streaming kernel keeps more bytes in flight per wave).
static int launch_f32in(fl_ctx *ctx, const fl_weight &w, int pro, int epi, const float *x,
                        const float *nw, float eps, float *out, unsigned long long *slot, int M = 1) {
    if ((w.format == FL_Q6K || w.format == FL_Q8_0) && (M > 1 || measure_env("FLARE_MVO_SINGLE"))) {
        MvoArgs a{};
        a.W = w.desc();
        a.x = x;
        a.nw = pro == 1 ? nw : nullptr;
        a.eps = eps;
        a.M = M;
        a.epi = epi;
        a.out = out;
        a.slots = slot;
        const hipError_t e = launch_mvo(w.format, ctx->stream, a);
        HIPCHK(ctx, e);
        return 0;
    }
    if (M != 1) return fail(ctx, FL_E_UNSUPPORTED, "multi-token f32-input matvec for format %d", w.format);
    const MvsPlan p = mvs_plan(w.format, w.rows, w.cols, true);
    const MvsArgs a = mvs_args(ctx, w, pro, epi, x, nw, eps, nullptr, nullptr, nullptr, out, slot);
    hipError_t e;
    if (w.format == FL_Q8_0) e = launch_mvs_q8_0(true, p, ctx->stream, a);
    else if (w.format == FL_Q6K || w.format == FL_F32) e = launch_mvs_f32(w.format, p, ctx->stream, a);
    else return fail(ctx, FL_E_UNSUPPORTED, "no f32-input matvec for format %d", w.format);
    return mvs_result(ctx, e, p);
}

static int launch_gateup(fl_ctx *ctx, const fl_weight &w, int pro, const float *x, const float *nw,
                         float eps, const int8_t *q, const float *s, const int *sums, int8_t *hq,
                         float *hs, int *hsum, float *hout) {
    const int F = w.rows / 2;
    if (w.rows % 2 || F % 32) return fail(ctx, FL_E_INVALID, "gate_up rows %d must be 2*32k", w.rows);
    if (pro == PRO_LOADQ && w.cols > 4 * 16 * 4 * 64)
        return fail(ctx, FL_E_UNSUPPORTED, "gate_up input of %d columns is too wide", w.cols);
    MvsArgs a = mvs_args(ctx, w, pro, EPI_STORE, x, nw, eps, q, s, sums, nullptr, nullptr);
    a.seq = ctx->exact;
    a.F = F;
    a.hq = hq;
    a.hs = hs;
    a.hsum = hsum;
    a.hout = hout;
    const MvsPlan p = mvs_gu_plan(w.format, F, w.cols);
    hipError_t e;
    if (w.format == FL_Q8_0) e = launch_mvs_gu_q8_0(p, ctx->stream, a);
    else if (w.format == FL_Q4K) e = launch_mvs_gu_q4k(p, ctx->stream, a);
    else return fail(ctx, FL_E_UNSUPPORTED, "no gate_up kernel for format %d", w.format);
    return mvs_result(ctx, e, p);
}

static int launch_attention(fl_ctx *ctx, int kv_format, int D, int G, AttnArgs &a) {
    const hipError_t e = launch_attn(kv_format, D, G, ctx->stream, a);
    if (e == hipErrorNotSupported)
        return fail(ctx, FL_E_UNSUPPORTED, "attention: head_dim %d / group %d not supported", D, G);
    HIPCHK(ctx, e);
    HIPCHK(ctx, hipGetLastError());
    return 0;
}

// Algorithmic K+V bytes one decode attention launch reads over T tokens.
static double attn_bytes(const fl_ctx *ctx, int T) {
    const fl_model_config &c = ctx->cfg;
    const double kvd = (double)c.num_kv_heads * c.head_dim;
    switch (ctx->kv_format) {
    case FL_KV_F32: return 2.0 * T * kvd * 4;
    case FL_KV_F16: return 2.0 * T * kvd * 2;
    case FL_KV_Q8: return 2.0 * T * (kvd + kvd / 32 * 2);
    default: {
        const int Q = kivi_qlen(T);
        // codes (2 bits) + K (scale, min) per 32 tokens x channel + V (scale, min) per token x 32 channels
        const double quant = 2.0 * Q * kvd / 4 + (Q / 32) * kvd * 4 + Q * (kvd / 32) * 4;
        return quant + 2.0 * (T - Q) * kvd * 2;
    }
    }
}

// Captured graphs hold device pointers: drop them whenever a buffer they use
// is reallocated or the model changes (they are captured again on next use).
static void drop_graphs(fl_ctx *c) {
    if (c->gexec) (void)hipGraphExecDestroy(c->gexec);
    if (c->graph) (void)hipGraphDestroy(c->graph);
    c->gexec = nullptr;
    c->graph = nullptr;
    c->graph_ready = false;
    for (auto &kv : c->vgraphs) (void)hipGraphExecDestroy(kv.second);
    c->vgraphs.clear();
}

// Split partial sets per (query, kv head) the attention kernels may publish:
// the decode split count, or up to kAttmMaxSplit for k_attq (fp16 caches).
static int part_splits(const fl_ctx *ctx) {
    return ctx->kv_format == FL_KV_F16 ? std::max(ctx->nsplit, kAttmMaxSplit) : ctx->nsplit;
}

static int ensure_part(fl_ctx *ctx, size_t floats) {
    if (ctx->part_cap >= floats) return 0;
    drop_graphs(ctx);
    if (ctx->d_part) (void)hipFree(ctx->d_part);
    ctx->d_part = nullptr;
    ctx->part_cap = 0;
    ALLOC(ctx, ctx->d_part, floats * 4);
    ctx->part_cap = floats;
    return 0;
}

// =====================================================================
// C-ABI
// =====================================================================
extern "C" {

int fl_abi_version(void) { return FL_ABI_VERSION; }
const char *fl_backend_name(void) { return "flare-hip (MI355X gfx950)"; }

const char *fl_last_error(const fl_ctx *ctx) { return ctx ? ctx->err.c_str() : g_err.c_str(); }

int fl_ctx_create(int device, fl_ctx **out) {
    if (!out) return fail(nullptr, FL_E_INVALID, "out is null");
    *out = nullptr;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n == 0) return fail(nullptr, FL_E_HIP, "no HIP device available");
    if (device < 0 || device >= n) return fail(nullptr, FL_E_INVALID, "device %d out of range", device);
    fl_ctx *c = new fl_ctx();
    c->device = device;
    e = hipSetDevice(device);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete c;
        return fail(nullptr, FL_E_HIP, "stream creation failed: %s", hipGetErrorString(e));
    }
    int rc = dev_alloc(c, (void **)&c->d_pos, 64);
    if (!rc) rc = dev_alloc(c, (void **)&c->d_rope_row, 2 * 512 * 4);
    if (!rc) rc = dev_alloc(c, (void **)&c->d_counters, kCounterWords * 4);
    if (!rc) rc = dev_alloc(c, (void **)&c->d_slot, 64);
    if (rc) {
        fl_ctx_destroy(c);
        return rc;
    }
    (void)hipMemset(c->d_counters, 0, kCounterWords * 4);
    // this device's copy of the no-alloc scratch array (device current)
    e = hipGetSymbolAddress((void **)&c->scratch, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !c->scratch) {
        fl_ctx_destroy(c);
        return fail(nullptr, FL_E_HIP, "scratch array address: %s", hipGetErrorString(e));
    }
    c->verify_fuse = measure_env("FLARE_NO_VFUSE") == nullptr;  // initial value of FL_OPT_VERIFY_FUSE
    c->fuse_attn = measure_env("FLARE_FUSE_ATTN") != nullptr;  // initial value of FL_OPT_FUSE_ATTN
    *out = c;
    return 0;
}

int fl_set_option(fl_ctx *ctx, int option, int value) {
    if (!ctx) return fail(nullptr, FL_E_INVALID, "null context");
    switch (option) {
    case FL_OPT_VERIFY_FUSE: ctx->verify_fuse = value != 0; break;
    case FL_OPT_VERIFY_GRAPH: ctx->verify_graph = value != 0; break;
    case FL_OPT_EXACT: ctx->exact = value != 0; break;
    case FL_OPT_FUSE_ATTN: ctx->fuse_attn = value != 0; break;
    default: return fail(ctx, FL_E_INVALID, "unknown option %d", option);
    }
    drop_graphs(ctx);  // captured passes bake the old choice in
    return 0;
}

static void model_release(fl_ctx *c) {
    drop_graphs(c);
    for (auto &l : c->layers) {
        weight_release(l.qkv); weight_release(l.wo); weight_release(l.gu); weight_release(l.down);
        if (l.attn_norm) (void)hipFree(l.attn_norm);
        if (l.ffn_norm) (void)hipFree(l.ffn_norm);
    }
    c->layers.clear();
    weight_release(c->embed);
    weight_release(c->output);
    void *kvp[] = {c->kscale, c->vscale, c->kparam, c->vparam, c->kring, c->vring, c->kvstage};
    for (void *p : kvp)
        if (p) (void)hipFree(p);
    c->kscale = c->vscale = nullptr; c->kparam = c->vparam = nullptr; c->kring = c->vring = nullptr;
    c->kvstage = nullptr; c->kvstage_rows = 0;
    void *ptrs[] = {c->out_norm, c->kcache, c->vcache, c->rope, c->x, c->qkv, c->attn, c->logits, c->bench_out,
                    c->bench_trace, c->rope_cur, c->seq_scores, c->seq_xn,
                    c->aq, c->hq, c->as, c->hs, c->asum, c->hsum, c->st, c->tokens};
    for (void *p : ptrs)
        if (p) (void)hipFree(p);
    c->out_norm = nullptr; c->kcache = c->vcache = nullptr; c->rope = nullptr; c->x = c->qkv = nullptr;
    c->attn = c->logits = c->bench_out = nullptr; c->bench_trace = nullptr; c->rope_cur = nullptr; c->aq = c->hq = nullptr; c->as = c->hs = nullptr;
    c->asum = c->hsum = nullptr; c->st = nullptr; c->tokens = nullptr;
    c->seq_scores = c->seq_xn = nullptr;
    if (c->probe_dev) (void)hipFree(c->probe_dev);
    c->probe_dev = nullptr;
    c->probe_bytes = 0;
    c->probe_layer = -1;
    c->probe_host = nullptr;
    void *vp[] = {c->vx, c->vx2, c->vq, c->vk, c->vv, c->vpart, c->vxq, c->vaq, c->vxs, c->vas, c->vxsum, c->vasum,
                  c->vtok, c->vpos, c->vslots, c->vhq, c->vhs, c->vhsum, c->vcnt};
    for (void *p : vp)
        if (p) (void)hipFree(p);
    c->vx = c->vx2 = c->vq = c->vk = c->vv = c->vpart = nullptr; c->vxq = c->vaq = nullptr; c->vxs = c->vas = nullptr;
    c->vxsum = c->vasum = nullptr; c->vtok = c->vpos = nullptr; c->vslots = nullptr; c->vpart_floats = 0;
    c->vhq = nullptr; c->vhs = nullptr; c->vhsum = c->vcnt = nullptr;
    c->have_verify = false;
    c->have_cfg = c->have_weights = false;
}

void fl_ctx_destroy(fl_ctx *ctx) {
    if (!ctx) return;
    (void)hipSetDevice(ctx->device);
    if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
    model_release(ctx);
    void *ptrs[] = {ctx->d_pos, ctx->d_rope_row, ctx->d_part, ctx->d_counters, ctx->d_slot,
                    ctx->sp, ctx->scounts, ctx->sprev, ctx->sstate, ctx->svals, ctx->ssvals, ctx->skeys,
                    ctx->sskeys, ctx->ssort};
    for (void *p : ptrs)
        if (p) (void)hipFree(p);
    if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
    delete ctx;
}

void *fl_ctx_stream(fl_ctx *ctx) { return ctx ? (void *)ctx->stream : nullptr; }

// The fused QKV + attention launch's wait-timeout flag (set only if its
// bounded wait ran out: the step's outputs are then invalid).
static int fuse_check(fl_ctx *ctx) {
    if (!ctx->d_counters) return 0;
    int err = 0;
    HIPCHK(ctx, hipMemcpy(&err, ctx->d_counters + kFuseErr, 4, hipMemcpyDeviceToHost));
    if (err) return fail(ctx, FL_E_HIP, "fused QKV + attention launch: wait for the QKV workgroups timed out");
    return 0;
}

int fl_sync(fl_ctx *ctx) {
    if (!ctx) return fail(nullptr, FL_E_INVALID, "null ctx");
    HIPCHK(ctx, hipStreamSynchronize(ctx->stream));
    return fuse_check(ctx);
}

int fl_weight_upload(fl_ctx *ctx, const fl_raw_weight *w, fl_weight **out) {
    if (!ctx || !w || !out) return fail(ctx, FL_E_INVALID, "null argument");
    *out = nullptr;
    if (w->num_rows <= 0 || w->blocks_per_row <= 0) return fail(ctx, FL_E_INVALID, "empty weight");
    fl_weight *fw = new fl_weight();
    const fl_raw_weight *arr[1] = {w};
    int rc = upload_concat(ctx, arr, 1, *fw);
    if (rc) {
        weight_release(*fw);
        delete fw;
        return rc;
    }
    *out = fw;
    return 0;
}

void fl_weight_free(fl_ctx *ctx, fl_weight *w) {
    (void)ctx;
    if (!w) return;
    weight_release(*w);
    delete w;
}

int fl_op_quantize_q8(fl_ctx *ctx, const float *x, int n, int8_t *q, float *scales, int32_t *sums) {
    if (!ctx || !x || !q || !scales || !sums) return fail(ctx, FL_E_INVALID, "null argument");
    if (n <= 0 || n % 32) return fail(ctx, FL_E_INVALID, "n=%d must be a positive multiple of 32", n);
    const int nb = n / 32;
    hipLaunchKernelGGL(k_quantize, dim3((nb + kThreads - 1) / kThreads), dim3(kThreads), 0, ctx->stream, x,
                       nb, q, scales, (int *)sums);
    HIPCHK(ctx, hipGetLastError());
    return 0;
}

int fl_op_rmsnorm_quantize_q8(fl_ctx *ctx, const float *x, const float *w, int n, float eps, int order,
                              int8_t *q, float *scales, int32_t *sums) {
    if (!ctx || !x || !w || !q || !scales || !sums) return fail(ctx, FL_E_INVALID, "null argument");
    if (n <= 0 || n % 32) return fail(ctx, FL_E_INVALID, "n=%d must be a positive multiple of 32", n);
    // FL_OPT_EXACT: the sum of squares in the reference's sequential order
    auto kern = order == 0 ? (ctx->exact ? k_norm_quant<PRO_NORMQ0, true> : k_norm_quant<PRO_NORMQ0, false>)
                           : (ctx->exact ? k_norm_quant<PRO_NORMQ1, true> : k_norm_quant<PRO_NORMQ1, false>);
    hipLaunchKernelGGL(kern, dim3(1), dim3(kThreads), 0, ctx->stream, x, w, n, eps, q, scales, (int *)sums);
    HIPCHK(ctx, hipGetLastError());
    return 0;
}

int fl_op_rmsnorm(fl_ctx *ctx, const float *x, const float *w, int n, float eps, float *out) {
    if (!ctx || !x || !w || !out || n <= 0) return fail(ctx, FL_E_INVALID, "bad argument");
    if (ctx->exact) HIPCHK(ctx, launch_rmsnorm_seq(ctx->stream, x, w, n, eps, out));
    else hipLaunchKernelGGL(k_rmsnorm, dim3(1), dim3(kThreads), 0, ctx->stream, x, w, n, eps, out);
    HIPCHK(ctx, hipGetLastError());
    return 0;
}

int fl_op_matvec_q8in(fl_ctx *ctx, const fl_weight *w, const int8_t *q, const float *scales,
                      const int32_t *sums, float *out) {
    if (!ctx || !w || !q || !scales || !sums || !out) return fail(ctx, FL_E_INVALID, "null argument");
    return launch_q8in(ctx, *w, PRO_LOADQ, EPI_STORE, nullptr, nullptr, 0.f, q, scales, (const int *)sums, out,
                       nullptr);
}

int fl_op_matvec_f32in(fl_ctx *ctx, const fl_weight *w, const float *x, float *out) {
    if (!ctx || !w || !x || !out) return fail(ctx, FL_E_INVALID, "null argument");
    return launch_f32in(ctx, *w, 0, EPI_STORE, x, nullptr, 0.f, out, nullptr);
}

int fl_op_block_dots(fl_ctx *ctx, const fl_weight *w, const int8_t *q, int32_t *dots) {
    if (!ctx || !w || !q || !dots) return fail(ctx, FL_E_INVALID, "null argument");
    long long n;
    if (w->format == FL_Q8_0) {
        n = (long long)w->rows * (w->cols / 32);
        hipLaunchKernelGGL(k_block_dots<F_Q8_0>, dim3((unsigned)((n + kThreads - 1) / kThreads)), dim3(kThreads),
                           0, ctx->stream, w->desc(), q, (int *)dots);
    } else if (w->format == FL_Q4K) {
        n = (long long)w->rows * (w->cols / 256) * 4;
        hipLaunchKernelGGL(k_block_dots<F_Q4K>, dim3((unsigned)((n + kThreads - 1) / kThreads)), dim3(kThreads),
                           0, ctx->stream, w->desc(), q, (int *)dots);
    } else {
        return fail(ctx, FL_E_UNSUPPORTED, "block dots need Q8_0 or Q4_K");
    }
    HIPCHK(ctx, hipGetLastError());
    return 0;
}

int fl_op_dequant(fl_ctx *ctx, const fl_weight *w, float *out) {
    if (!ctx || !w || !out) return fail(ctx, FL_E_INVALID, "null argument");
    const long long n = (long long)w->rows * (w->cols / 32);
    const dim3 grid((unsigned)((n + kThreads - 1) / kThreads));
    switch (w->format) {
    case FL_Q8_0: hipLaunchKernelGGL(k_dequant<F_Q8_0>, grid, dim3(kThreads), 0, ctx->stream, w->desc(), out); break;
    case FL_Q4K: hipLaunchKernelGGL(k_dequant<F_Q4K>, grid, dim3(kThreads), 0, ctx->stream, w->desc(), out); break;
    case FL_Q6K: hipLaunchKernelGGL(k_dequant<F_Q6K>, grid, dim3(kThreads), 0, ctx->stream, w->desc(), out); break;
    case FL_F32: hipLaunchKernelGGL(k_dequant<F_F32>, grid, dim3(kThreads), 0, ctx->stream, w->desc(), out); break;
    default: return fail(ctx, FL_E_UNSUPPORTED, "format %d", w->format);
    }
    HIPCHK(ctx, hipGetLastError());
    return 0;
}

int fl_op_matvec_argmax(fl_ctx *ctx, const fl_weight *w, const int8_t *q, const float *scales,
                        const int32_t *sums, const float *x, int64_t *out_idx, float *out_val) {
    if (!ctx || !w || !out_idx || !out_val) return fail(ctx, FL_E_INVALID, "null argument");
    HIPCHK(ctx, hipMemsetAsync(ctx->d_slot, 0, 8, ctx->stream));
    int rc;
    if (q) {
        if (!scales || !sums) return fail(ctx, FL_E_INVALID, "quantized input needs scales and sums");
        rc = launch_q8in(ctx, *w, PRO_LOADQ, EPI_ARGMAX, nullptr, nullptr, 0.f, q, scales, (const int *)sums,
                         nullptr, ctx->d_slot);
    } else {
        if (!x) return fail(ctx, FL_E_INVALID, "need q or x");
        rc = launch_f32in(ctx, *w, 0, EPI_ARGMAX, x, nullptr, 0.f, nullptr, ctx->d_slot);
    }
    if (rc) return rc;
    unsigned long long key = 0;
    HIPCHK(ctx, hipMemcpyAsync(&key, ctx->d_slot, 8, hipMemcpyDeviceToHost, ctx->stream));
    HIPCHK(ctx, hipStreamSynchronize(ctx->stream));
    const int64_t idx = (int64_t)(0xFFFFFFFFu - (uint32_t)(key & 0xFFFFFFFFull));
    uint32_t u = (uint32_t)(key >> 32);
    u = (u & 0x80000000u) ? (u & 0x7FFFFFFFu) : ~u;
    float v;
    std::memcpy(&v, &u, 4);
    HIPCHK(ctx, hipMemcpyAsync(out_idx, &idx, 8, hipMemcpyHostToDevice, ctx->stream));
    HIPCHK(ctx, hipMemcpyAsync(out_val, &v, 4, hipMemcpyHostToDevice, ctx->stream));
    HIPCHK(ctx, hipStreamSynchronize(ctx->stream));
    return 0;
}

// Host RoPE table row with the formula of RopeTable::new (model.rs:7197-7204).
static void rope_row_host(int head_dim, int pos, float theta, float *c, float *s) {
    const int half = head_dim / 2;
    for (int d = 0; d < half; d++) {
        const float freq = 1.0f / powf(theta, 2.0f * (float)d / (float)head_dim);
        const float angle = (float)pos * freq;
        s[d] = sinf(angle);
        c[d] = cosf(angle);
    }
}

int fl_op_rope(fl_ctx *ctx, float *data, int num_heads, int head_dim, int pos, float theta) {
    if (!ctx || !data || num_heads <= 0 || head_dim <= 0 || head_dim % 2 || head_dim > 512 || pos < 0)
        return fail(ctx, FL_E_INVALID, "bad rope argument");
    std::vector<float> cs(512), sn(512);
    rope_row_host(head_dim, pos, theta, cs.data(), sn.data());
    HIPCHK(ctx, hipMemcpyAsync(ctx->d_rope_row, cs.data(), 512 * 4, hipMemcpyHostToDevice, ctx->stream));
    HIPCHK(ctx, hipMemcpyAsync(ctx->d_rope_row + 512, sn.data(), 512 * 4, hipMemcpyHostToDevice, ctx->stream));
    const int n = num_heads * head_dim / 2;
    hipLaunchKernelGGL(k_rope, dim3((n + kThreads - 1) / kThreads), dim3(kThreads), 0, ctx->stream, data, num_heads,
                       head_dim, ctx->d_rope_row, ctx->d_rope_row + 512);
    HIPCHK(ctx, hipGetLastError());
    HIPCHK(ctx, hipStreamSynchronize(ctx->stream));  // host staging buffers go out of scope
    return 0;
}

int fl_op_silu_mul(fl_ctx *ctx, const float *gate, const float *up, int n, float *out) {
    if (!ctx || !gate || !up || !out || n <= 0) return fail(ctx, FL_E_INVALID, "bad argument");
    hipLaunchKernelGGL(k_silu_mul, dim3((n + kThreads - 1) / kThreads), dim3(kThreads), 0, ctx->stream, gate, up,
                       n, out);
    HIPCHK(ctx, hipGetLastError());
    return 0;
}

int fl_op_attention(fl_ctx *ctx, const float *q, const void *k_cache, const void *v_cache, int kv_format,
                    int num_heads, int num_kv_heads, int head_dim, int seq_len, int num_splits, float *out) {
    if (!ctx || !q || !k_cache || !v_cache || !out) return fail(ctx, FL_E_INVALID, "null argument");
    if (num_kv_heads <= 0 || num_heads % num_kv_heads || seq_len <= 0)
        return fail(ctx, FL_E_INVALID, "bad attention shape");
    if (num_kv_heads > 1024) return fail(ctx, FL_E_INVALID, "too many kv heads");
    if (kv_format != FL_KV_F16 && kv_format != FL_KV_F32) return fail(ctx, FL_E_UNSUPPORTED, "kv format");
    const int G = num_heads / num_kv_heads;
    int ns, chmin;
    choose_splits(seq_len, num_kv_heads, head_dim, ns, chmin);
    if (num_splits > 0) {
        ns = std::min(num_splits, kAttnMaxSplit);
        chmin = 1;
    }
    const size_t need = (size_t)num_kv_heads * ns * G * (head_dim + 2);
    int rc = ensure_part(ctx, need);
    if (rc) return rc;
    const int pos = seq_len - 1;
    HIPCHK(ctx, hipMemcpyAsync(ctx->d_pos, &pos, 4, hipMemcpyHostToDevice, ctx->stream));
    AttnArgs a{};
    a.q = q;
    a.kc = (void *)k_cache;
    a.vc = (void *)v_cache;
    a.tok_stride = (long long)num_kv_heads * head_dim;  // [slot][kv_head][head_dim]
    a.head_stride = head_dim;
    a.posp = ctx->d_pos;
    a.nkv = num_kv_heads;
    a.nsplit = ns;
    a.chmin = chmin;
    a.single = kAttmSingle;
    a.part = ctx->d_part;
    a.counters = ctx->d_counters;
    a.out = out;
    rc = launch_attention(ctx, kv_format, head_dim, G, a);
    if (rc) return rc;
    HIPCHK(ctx, hipStreamSynchronize(ctx->stream));  // pos staged from the host stack
    return 0;
}

// ---- model -------------------------------------------------------------------

int fl_model_init(fl_ctx *ctx, const fl_model_config *cfg, int kv_format) {
    if (!ctx || !cfg) return fail(ctx, FL_E_INVALID, "null argument");
    const fl_model_config &c = *cfg;
    if (c.hidden_dim <= 0 || c.hidden_dim % 32 || c.num_layers <= 0 || c.num_heads <= 0 ||
        c.num_kv_heads <= 0 || c.num_heads % c.num_kv_heads || (c.head_dim != 64 && c.head_dim != 128) ||
        c.intermediate_dim % 32 || c.vocab_size <= 0 || c.max_seq_len <= 0)
        return fail(ctx, FL_E_INVALID,
                    "unsupported config (hidden %% 32, head_dim 64/128, inter %% 32 required)");
    if (kv_format < FL_KV_F32 || kv_format > FL_KV_KIVI2) return fail(ctx, FL_E_UNSUPPORTED, "kv format %d", kv_format);
    if (!attn_supported(c.head_dim, c.num_heads / c.num_kv_heads))
        return fail(ctx, FL_E_UNSUPPORTED, "heads per kv group %d", c.num_heads / c.num_kv_heads);
    model_release(ctx);
    ctx->cfg = c;
    ctx->kv_format = kv_format;
    const size_t H = c.hidden_dim, qd = (size_t)c.num_heads * c.head_dim, kvd = (size_t)c.num_kv_heads * c.head_dim;
    const size_t F = c.intermediate_dim, L = c.num_layers, S = c.max_seq_len;
    {
        // Q8 / KIVI groups and the fp16 / Q8 transposed V blocks span 32 slots
        const bool blk32 = kv_format != FL_KV_F32;
        const size_t Sa = blk32 ? (S + 31) / 32 * 32 : S;
        ctx->kv_slots = (int)Sa;
        const size_t code_bytes = kv_format == FL_KV_F32 ? 4 * kvd : kv_format == FL_KV_F16 ? 2 * kvd
                                : kv_format == FL_KV_Q8 ? kvd : kvd / 4;  // per token
        ctx->kv_layer_elems = kv_format <= FL_KV_F16 ? Sa * kvd : Sa * code_bytes;
        ALLOC(ctx, ctx->kcache, L * Sa * code_bytes);
        ALLOC(ctx, ctx->vcache, L * Sa * code_bytes);
        HIPCHK(ctx, hipMemset(ctx->kcache, 0, L * Sa * code_bytes));
        HIPCHK(ctx, hipMemset(ctx->vcache, 0, L * Sa * code_bytes));
        if (kv_format == FL_KV_Q8) {
            const size_t n = L * Sa * (kvd / 32) * 2;
            ALLOC(ctx, ctx->kscale, n);
            ALLOC(ctx, ctx->vscale, n);
            HIPCHK(ctx, hipMemset(ctx->kscale, 0, n));
            HIPCHK(ctx, hipMemset(ctx->vscale, 0, n));
        }
        if (kv_format == FL_KV_KIVI2) {
            const size_t nk = L * (Sa / 32) * kvd * 4, nv = L * Sa * (kvd / 32) * 4, nr = L * kKiviRing * kvd * 2;
            ALLOC(ctx, ctx->kparam, nk);
            ALLOC(ctx, ctx->vparam, nv);
            ALLOC(ctx, ctx->kring, nr);
            ALLOC(ctx, ctx->vring, nr);
            HIPCHK(ctx, hipMemset(ctx->kparam, 0, nk));
            HIPCHK(ctx, hipMemset(ctx->vparam, 0, nv));
            HIPCHK(ctx, hipMemset(ctx->kring, 0, nr));
            HIPCHK(ctx, hipMemset(ctx->vring, 0, nr));
        }
    }
    // RoPE table for every position (RopeTable::new formula, host libm)
    const int half = c.head_dim / 2;
    std::vector<float> tab(2 * S * half);
#pragma omp parallel for schedule(static)
    for (long long p = 0; p < (long long)S; p++)
        rope_row_host(c.head_dim, (int)p, c.rope_theta, &tab[p * half], &tab[S * half + p * half]);
    ALLOC(ctx, ctx->rope, tab.size() * 4);
    HIPCHK(ctx, hipMemcpy(ctx->rope, tab.data(), tab.size() * 4, hipMemcpyHostToDevice));
    if (kv_format == FL_KV_F16 || kv_format == FL_KV_Q8 || kv_format == FL_KV_KIVI2) {
        // MFMA kernel: at most kAttmMaxSplit splits per kv head, chunks of at
        // least chmin slots.  Measured on MI355X (Llama-3.2-1B D=64 at ~800 tokens, Llama-3-8B
        // D=128 at ~4k): split every context longer than one block per wave,
        // 4-wave workgroups for D=64 and 8-wave ones for D=128.  More,
        // smaller splits spread the K/V stream over more CUs; the split merge
        // (publish, count, one round trip of partial loads) costs ~3-4 us.
        // The split count stops where every workgroup of a decode launch is
        // resident at once (CUs x resident workgroups per CU / kv heads):
        // beyond that, a second dispatch round repeats the whole latency
        // chain (Llama-3-8B heads at 32k / 128k: 32 splits against 64 cut
        // fp16 44 -> 32 / 109 -> 99 us, Q8 49 -> 32 / 100 -> 88 us).
        ctx->attn_waves = c.head_dim <= 64 ? 4 : 8;
        ctx->single = 0;
        if (const char *ev = measure_env("FLARE_ATTN_WAVES")) ctx->attn_waves = atoi(ev) == 4 ? 4 : 8;  // tuning override
        const int pass = kAttmBlock * ctx->attn_waves;  // tokens of one block per wave
        ctx->chmin = pass;
        if (const char *ev = measure_env("FLARE_ATTN_CHMIN")) ctx->chmin = std::max(pass, atoi(ev) / pass * pass);
        if (const char *ev = measure_env("FLARE_ATTN_SINGLE")) ctx->single = std::max(0, atoi(ev));  // tuning override
        int ncu = 0, dev = 0;
        (void)hipGetDevice(&dev);
        (void)hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev);
        const int res = attm_resident_per_cu(kv_format, c.head_dim, c.num_heads / c.num_kv_heads, ctx->attn_waves);
        if (ncu > 0) ctx->ncu = ncu;
        const int fit = ncu > 0 && res > 0 ? std::max(1, ncu * res / c.num_kv_heads) : kAttmMaxSplit;
        ctx->nsplit = std::max(1, std::min({kAttmMaxSplit, fit, (c.max_seq_len + ctx->chmin - 1) / ctx->chmin}));
    } else {
        choose_splits(c.max_seq_len, c.num_kv_heads, c.head_dim, ctx->nsplit, ctx->chmin);
        if (const char *ev = measure_env("FLARE_ATTN_CHMIN")) ctx->chmin = std::max(1, atoi(ev));  // tuning override
    }
    if (const char *ev = measure_env("FLARE_ATTN_NSPLIT")) {  // tuning override
        const int ns = atoi(ev);
        if (ns > 0 && ns <= (kv_format != FL_KV_F32 ? kAttmMaxSplit : kAttnMaxSplit))
            ctx->nsplit = ns;
    }
    const int G = c.num_heads / c.num_kv_heads;
    // split partials for up to kPrefillTokens queries (decode uses 1), so
    // a verify batch never reallocates them
    int rc = ensure_part(ctx, (size_t)kPrefillTokens * c.num_kv_heads * part_splits(ctx) * G * (c.head_dim + 2));
    if (rc) return rc;
    ALLOC(ctx, ctx->x, H * 4);
    ALLOC(ctx, ctx->qkv, (qd + 2 * kvd) * 4);
    ALLOC(ctx, ctx->attn, qd * 4);
    ALLOC(ctx, ctx->seq_scores, (size_t)c.num_heads * ctx->kv_slots * 4);
    ALLOC(ctx, ctx->seq_xn, H * 4);
    ALLOC(ctx, ctx->aq, qd);
    ALLOC(ctx, ctx->as, qd / 32 * 4);
    ALLOC(ctx, ctx->asum, qd / 32 * 4);
    ALLOC(ctx, ctx->hq, F);
    ALLOC(ctx, ctx->hs, F / 32 * 4);
    ALLOC(ctx, ctx->hsum, F / 32 * 4);
    ALLOC(ctx, ctx->logits, (size_t)c.vocab_size * 4);
    ALLOC(ctx, ctx->bench_out, std::max({(size_t)c.vocab_size, H, qd + 2 * kvd, 2 * F}) * 4);
    ALLOC(ctx, ctx->bench_trace, (64 + 3072) * 8);
    ALLOC(ctx, ctx->rope_cur, (size_t)c.head_dim * 4);
    ALLOC(ctx, ctx->st, sizeof(DevState));
    ALLOC(ctx, ctx->tokens, S * 4);
    HIPCHK(ctx, hipMemset(ctx->st, 0, sizeof(DevState)));
    HIPCHK(ctx, hipMemset(ctx->tokens, 0, S * 4));
    HIPCHK(ctx, hipMemset(ctx->d_counters, 0, kCounterWords * 4));
    ctx->have_cfg = true;
    return 0;
}

int fl_has_weights(const fl_ctx *ctx) { return ctx && ctx->have_weights ? 1 : 0; }
int fl_has_kv_cache(const fl_ctx *ctx) { return ctx && ctx->have_cfg ? 1 : 0; }

int fl_upload_weights(fl_ctx *ctx, const fl_raw_weight *layers, const float *const *attn_norms,
                      const float *const *ffn_norms, const float *output_norm, const fl_raw_weight *embedding,
                      const fl_raw_weight *output) {
    if (!ctx || !layers || !attn_norms || !ffn_norms || !output_norm || !embedding)
        return fail(ctx, FL_E_INVALID, "null argument");
    if (!ctx->have_cfg) return fail(ctx, FL_E_STATE, "fl_model_init must precede fl_upload_weights");
    const fl_model_config &c = ctx->cfg;
    const int H = c.hidden_dim, qd = c.num_heads * c.head_dim, kvd = c.num_kv_heads * c.head_dim;
    const int F = c.intermediate_dim;
    const int fmt = layers[0].format;
    if (fmt != FL_Q8_0 && fmt != FL_Q4K) return fail(ctx, FL_E_UNSUPPORTED, "layer format %d (need Q8_0/Q4_K)", fmt);
    if (fmt == FL_Q4K && (H % 256 || F % 256 || qd % 256))
        return fail(ctx, FL_E_INVALID, "Q4_K needs dims multiple of 256");
    const int exp_rows[7] = {qd, kvd, kvd, H, F, F, H};
    const int exp_cols[7] = {H, H, H, qd, H, H, F};
    for (int l = 0; l < c.num_layers; l++)
        for (int j = 0; j < 7; j++) {
            const fl_raw_weight &w = layers[l * 7 + j];
            if (w.format != fmt) return fail(ctx, FL_E_INVALID, "layer %d weight %d: mixed formats", l, j);
            if (w.num_rows != exp_rows[j] || weight_cols(&w) != exp_cols[j])
                return fail(ctx, FL_E_INVALID, "layer %d weight %d: shape %dx%d, expected %dx%d", l, j, w.num_rows,
                            weight_cols(&w), exp_rows[j], exp_cols[j]);
        }
    if (weight_cols(embedding) != H || embedding->num_rows != c.vocab_size)
        return fail(ctx, FL_E_INVALID, "embedding shape");
    if (output && (weight_cols(output) != H || output->num_rows != c.vocab_size))
        return fail(ctx, FL_E_INVALID, "output shape");
    ctx->have_weights = false;
    drop_graphs(ctx);
    for (auto &l : ctx->layers) {
        weight_release(l.qkv); weight_release(l.wo); weight_release(l.gu); weight_release(l.down);
        if (l.attn_norm) (void)hipFree(l.attn_norm);
        if (l.ffn_norm) (void)hipFree(l.ffn_norm);
    }
    ctx->layers.assign(c.num_layers, Layer());
    ctx->layer_fmt = fmt;
    for (int l = 0; l < c.num_layers; l++) {
        const fl_raw_weight *w = &layers[l * 7];
        const fl_raw_weight *qkv[3] = {&w[0], &w[1], &w[2]};
        const fl_raw_weight *wo[1] = {&w[3]};
        const fl_raw_weight *gu[2] = {&w[4], &w[5]};
        const fl_raw_weight *dn[1] = {&w[6]};
        Layer &L = ctx->layers[l];
        int rc = upload_concat(ctx, qkv, 3, L.qkv, 2, c.head_dim);
        if (!rc) rc = upload_concat(ctx, wo, 1, L.wo);
        if (!rc) rc = upload_concat(ctx, gu, 2, L.gu);
        if (!rc) rc = upload_concat(ctx, dn, 1, L.down);
        if (rc) return rc;
        ALLOC(ctx, L.attn_norm, (size_t)H * 4);
        ALLOC(ctx, L.ffn_norm, (size_t)H * 4);
        HIPCHK(ctx, hipMemcpy(L.attn_norm, attn_norms[l], (size_t)H * 4, hipMemcpyHostToDevice));
        HIPCHK(ctx, hipMemcpy(L.ffn_norm, ffn_norms[l], (size_t)H * 4, hipMemcpyHostToDevice));
    }
    weight_release(ctx->embed);
    weight_release(ctx->output);
    const fl_raw_weight *e1[1] = {embedding};
    int rc = upload_concat(ctx, e1, 1, ctx->embed);
    if (rc) return rc;
    ctx->tied = output == nullptr;
    if (!ctx->tied) {
        const fl_raw_weight *o1[1] = {output};
        rc = upload_concat(ctx, o1, 1, ctx->output);
        if (rc) return rc;
    }
    if (!ctx->out_norm) ALLOC(ctx, ctx->out_norm, (size_t)H * 4);
    HIPCHK(ctx, hipMemcpy(ctx->out_norm, output_norm, (size_t)H * 4, hipMemcpyHostToDevice));
    ctx->have_weights = true;
    return 0;
}

static void kv_layer_args(fl_ctx *ctx, int l, AttnArgs &a);

int fl_kv_write(fl_ctx *ctx, int layer, int position, const float *key, const float *value) {
    if (!ctx || !key || !value) return fail(ctx, FL_E_INVALID, "null argument");
    if (!ctx->have_cfg) return fail(ctx, FL_E_STATE, "no kv cache");
    const fl_model_config &c = ctx->cfg;
    if (layer < 0 || layer >= c.num_layers) return fail(ctx, FL_E_INVALID, "layer %d", layer);
    if (ctx->kv_format == FL_KV_Q8 || ctx->kv_format == FL_KV_KIVI2)
        return fl_kv_write_batch(ctx, layer, position, 1, key, value);
    const int slot = position % c.max_seq_len;  // ring write (GpuKvCache::write)
    const size_t hd = (size_t)c.head_dim;
    // device layout is head-major: [layer][kv_head][slot][head_dim]
    for (int h = 0; h < c.num_kv_heads; h++) {
        const size_t off = (size_t)layer * ctx->kv_layer_elems + ((size_t)h * ctx->kv_slots + slot) * hd;
        if (ctx->kv_format == FL_KV_F32) {
            HIPCHK(ctx, hipMemcpy((float *)ctx->kcache + off, key + h * hd, hd * 4, hipMemcpyHostToDevice));
            HIPCHK(ctx, hipMemcpy((float *)ctx->vcache + off, value + h * hd, hd * 4, hipMemcpyHostToDevice));
        } else {
            std::vector<__half> hk(hd), hv(hd);
            for (size_t i = 0; i < hd; i++) {
                hk[i] = __float2half(key[h * hd + i]);
                hv[i] = __float2half(value[h * hd + i]);
            }
            HIPCHK(ctx, hipMemcpy((__half *)ctx->kcache + off, hk.data(), hd * 2, hipMemcpyHostToDevice));
            // V: channel d of the slot sits in the 32-slot transposed block
            const size_t vbase = (size_t)layer * ctx->kv_layer_elems + (size_t)h * ctx->kv_slots * hd;
            for (size_t d = 0; d < hd; d++)
                HIPCHK(ctx, hipMemcpy((__half *)ctx->vcache + vbase + vt_off(slot, (int)d, (int)hd), &hv[d], 2,
                                      hipMemcpyHostToDevice));
        }
    }
    return 0;
}

int fl_kv_write_batch(fl_ctx *ctx, int layer, int pos0, int n, const float *keys, const float *values) {
    if (!ctx || !keys || !values) return fail(ctx, FL_E_INVALID, "null argument");
    if (!ctx->have_cfg) return fail(ctx, FL_E_STATE, "no kv cache");
    const fl_model_config &c = ctx->cfg;
    if (layer < 0 || layer >= c.num_layers) return fail(ctx, FL_E_INVALID, "layer %d", layer);
    if (n <= 0 || pos0 < 0 || pos0 + n > c.max_seq_len)
        return fail(ctx, FL_E_INVALID, "rows [%d, %d) outside the cache (max_seq_len %d)", pos0, pos0 + n,
                    c.max_seq_len);
    const size_t kvd = (size_t)c.num_kv_heads * c.head_dim;
    // stage the rows (at most 4096 per launch pair), then quantize on the device
    const int chunk = 4096;
    const size_t cap = (size_t)std::min(n, chunk);
    if (ctx->kvstage_rows < cap) {
        if (ctx->kvstage) (void)hipFree(ctx->kvstage);
        ctx->kvstage = nullptr;
        ctx->kvstage_rows = 0;
        ALLOC(ctx, ctx->kvstage, 2 * cap * kvd * 4);
        ctx->kvstage_rows = cap;
    }
    AttnArgs a{};
    kv_layer_args(ctx, layer, a);
    for (int r0 = 0; r0 < n; r0 += chunk) {
        const int m = std::min(chunk, n - r0);
        float *kd = ctx->kvstage, *vd = ctx->kvstage + ctx->kvstage_rows * kvd;
        HIPCHK(ctx, hipMemcpyAsync(kd, keys + (size_t)r0 * kvd, (size_t)m * kvd * 4, hipMemcpyHostToDevice, ctx->stream));
        HIPCHK(ctx, hipMemcpyAsync(vd, values + (size_t)r0 * kvd, (size_t)m * kvd * 4, hipMemcpyHostToDevice,
                                   ctx->stream));
        HIPCHK(ctx, launch_kv_write(ctx->kv_format, ctx->stream, a, kd, vd, pos0 + r0, m, c.head_dim));
        HIPCHK(ctx, hipStreamSynchronize(ctx->stream));  // the staging buffer is reused
    }
    return 0;
}

int fl_reset(fl_ctx *ctx) {
    if (!ctx || !ctx->have_cfg) return fail(ctx, FL_E_STATE, "no model");
    const fl_model_config &c = ctx->cfg;
    const size_t L = c.num_layers, Sa = ctx->kv_slots, kvd = (size_t)c.num_kv_heads * c.head_dim;
    const size_t esz = ctx->kv_format == FL_KV_F16 ? 2 : ctx->kv_format == FL_KV_F32 ? 4 : 1;
    const size_t bytes = L * ctx->kv_layer_elems * esz;
    HIPCHK(ctx, hipMemsetAsync(ctx->kcache, 0, bytes, ctx->stream));
    HIPCHK(ctx, hipMemsetAsync(ctx->vcache, 0, bytes, ctx->stream));
    if (ctx->kscale) {
        HIPCHK(ctx, hipMemsetAsync(ctx->kscale, 0, L * Sa * (kvd / 32) * 2, ctx->stream));
        HIPCHK(ctx, hipMemsetAsync(ctx->vscale, 0, L * Sa * (kvd / 32) * 2, ctx->stream));
    }
    if (ctx->kparam) {
        HIPCHK(ctx, hipMemsetAsync(ctx->kparam, 0, L * (Sa / 32) * kvd * 4, ctx->stream));
        HIPCHK(ctx, hipMemsetAsync(ctx->vparam, 0, L * Sa * (kvd / 32) * 4, ctx->stream));
        HIPCHK(ctx, hipMemsetAsync(ctx->kring, 0, L * kKiviRing * kvd * 2, ctx->stream));
        HIPCHK(ctx, hipMemsetAsync(ctx->vring, 0, L * kKiviRing * kvd * 2, ctx->stream));
    }
    HIPCHK(ctx, hipMemsetAsync(ctx->st, 0, sizeof(DevState), ctx->stream));
    // split-merge arrival counters: every launch leaves them at zero (the
    // last arriver resets its counter); cleared here too, so a launch that
    // did not complete cannot leave a stale count behind a reset
    HIPCHK(ctx, hipMemsetAsync(ctx->d_counters, 0, kCounterWords * 4, ctx->stream));
    if (ctx->vcnt) HIPCHK(ctx, hipMemsetAsync(ctx->vcnt, 0, kVerifyCounters * 4, ctx->stream));
    HIPCHK(ctx, hipStreamSynchronize(ctx->stream));
    return 0;
}

// Cache planes of layer l (every KV format), head-major with kv_slots slots
// per kv head.
static void kv_layer_args(fl_ctx *ctx, int l, AttnArgs &a) {
    const fl_model_config &c = ctx->cfg;
    const size_t D = c.head_dim, kvd = (size_t)c.num_kv_heads * D, Sa = ctx->kv_slots;
    const size_t esz = ctx->kv_format == FL_KV_F16 ? 2 : ctx->kv_format == FL_KV_F32 ? 4 : 1;
    a.kc = (uint8_t *)ctx->kcache + (size_t)l * ctx->kv_layer_elems * esz;
    a.vc = (uint8_t *)ctx->vcache + (size_t)l * ctx->kv_layer_elems * esz;
    a.tok_stride = (long long)D;
    a.head_stride = (long long)(Sa * D);
    a.nkv = c.num_kv_heads;
    a.S = (int)Sa;
    a.v_tblk = ctx->kv_format == FL_KV_F16 || ctx->kv_format == FL_KV_Q8;
    if (ctx->kscale) {
        a.ks = ctx->kscale + (size_t)l * Sa * (kvd / 32);
        a.vs = ctx->vscale + (size_t)l * Sa * (kvd / 32);
    }
    if (ctx->kparam) {
        a.kp = ctx->kparam + (size_t)l * (Sa / 32) * kvd;
        a.vp = ctx->vparam + (size_t)l * Sa * (kvd / 32);
        a.rk = ctx->kring + (size_t)l * kKiviRing * kvd;
        a.rv = ctx->vring + (size_t)l * kKiviRing * kvd;
    }
}

// Enqueue one decode step (kernels only; no host synchronisation).
// Attention of layer l over the head-major cache [kv_head][slot][head_dim]
// (q from the fused QKV output, RoPE already applied by its epilogue).
static AttnArgs layer_attn_args(fl_ctx *ctx, int l) {
    const fl_model_config &c = ctx->cfg;
    AttnArgs a{};
    kv_layer_args(ctx, l, a);
    a.q = ctx->qkv;
    a.posp = &ctx->st->pos;
    a.nsplit = ctx->nsplit;
    a.chmin = ctx->chmin;
    a.single = ctx->single;
    a.waves = ctx->attn_waves;
    a.part = ctx->d_part;
    a.counters = ctx->d_counters;
    a.out = nullptr;  // the wo matvec reads the Q8_0 copy only
    a.oq = ctx->aq;
    a.os = ctx->as;
    a.osum = ctx->asum;
    if (ctx->kv_format == FL_KV_Q8 || ctx->kv_format == FL_KV_KIVI2) {
        // the QKV epilogue leaves the new K / V rows (f32) after q
        const size_t qd = (size_t)c.num_heads * c.head_dim, kvd = (size_t)c.num_kv_heads * c.head_dim;
        a.knew = ctx->qkv + qd;
        a.vnew = ctx->qkv + qd + kvd;
    }
    return a;
}

// EPI_QKV arguments of layer l: RoPE at the live position, K/V rows into
// this layer's cache slot.
static QkvEpi layer_qkv_epi(fl_ctx *ctx, int l) {
    const fl_model_config &c = ctx->cfg;
    AttnArgs a{};
    kv_layer_args(ctx, l, a);
    QkvEpi e{};
    e.rope_cur = ctx->rope_cur;
    e.posp = &ctx->st->pos;
    e.kc = (void *)a.kc;
    e.vc = (void *)a.vc;
    e.head_stride = a.head_stride;
    e.nq = c.num_heads * c.head_dim;
    e.nk = c.num_kv_heads * c.head_dim;
    e.hd = c.head_dim;
    e.kv_f16 = ctx->kv_format == FL_KV_F16;
    e.v_tblk = ctx->kv_format == FL_KV_F16;
    // Q8 / KIVI: K (after RoPE) and V stay f32 in the output after q; the
    // attention kernel quantizes and stores them
    e.kv_stage = ctx->kv_format == FL_KV_Q8 || ctx->kv_format == FL_KV_KIVI2;
    return e;
}

// ---- layer probe ------------------------------------------------------------
// Regions (PR_*), each [kProbeTokens][per-token size], 256-byte aligned;
// byte offsets into off[], total size returned.  The decode step fills token
// 0; a verify pass its M tokens.  The norm codes (PR_XQ .. PR_FS) exist only
// in the verify pass, whose GEMMs read them from memory.
constexpr int kProbeTokens = 16;
enum {
    PR_XIN, PR_Q, PR_K, PR_V, PR_ATTN, PR_AS, PR_XMID, PR_HS, PR_XOUT, PR_XFIN, PR_AQ, PR_HQ,
    PR_XQ, PR_XS, PR_FQ, PR_FS, PR_N
};
static size_t probe_layout(const fl_model_config &c, size_t off[PR_N]) {
    const size_t H = c.hidden_dim, nq = (size_t)c.num_heads * c.head_dim, nk = (size_t)c.num_kv_heads * c.head_dim,
                 F = c.intermediate_dim;
    const size_t sz[PR_N] = {H * 4, nq * 4, nk * 4, nk * 4, nq * 4, nq / 32 * 4, H * 4, F / 32 * 4, H * 4, H * 4,
                             nq, F, H, H / 32 * 4, H, H / 32 * 4};
    size_t o = 0;
    for (int i = 0; i < PR_N; i++) {
        off[i] = o;
        o += (sz[i] * kProbeTokens + 255) / 256 * 256;
    }
    return o;
}

}  // extern "C"
// K / V rows of slots *posp .. *posp + M - 1 (cache layout of kv_layer_args)
// as f32, [M][nkv*D]
template <bool F16>
__global__ void k_probe_kv(const void *kc, const void *vc, long long head_stride, int D, int nkv, bool vt,
                           const int *posp, int M, float *k, float *v) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= M * nkv * D) return;
    const int m = i / (nkv * D), r = i % (nkv * D), h = r / D, d = r % D, t = *posp + m;
    const size_t kb = (size_t)h * head_stride;
    const size_t ko = kb + (size_t)t * D + d, vo = kb + (vt ? vt_off(t, d, D) : (size_t)t * D + d);
    if (F16) {
        k[i] = __half2float(((const __half *)kc)[ko]);
        v[i] = __half2float(((const __half *)vc)[vo]);
    } else {
        k[i] = ((const float *)kc)[ko];
        v[i] = ((const float *)vc)[vo];
    }
}
extern "C" {

static int probe_copy(fl_ctx *ctx, int region, const void *src, size_t bytes) {
    size_t off[PR_N];
    probe_layout(ctx->cfg, off);
    HIPCHK(ctx, hipMemcpyAsync(ctx->probe_dev + off[region], src, bytes, hipMemcpyDeviceToDevice, ctx->stream));
    return 0;
}

// the layer's K / V rows at *posp .. + M - 1 (F32 / F16 caches), or the f32
// staging rows the Q8 / KIVI writers quantize (`stage_k`, `stage_v`)
static int probe_kv(fl_ctx *ctx, int l, const int *posp, int M, const float *stage_k, const float *stage_v) {
    const fl_model_config &c = ctx->cfg;
    size_t off[PR_N];
    probe_layout(c, off);
    float *pk = (float *)(ctx->probe_dev + off[PR_K]), *pv = (float *)(ctx->probe_dev + off[PR_V]);
    const int n = M * c.num_kv_heads * c.head_dim;
    if (ctx->kv_format == FL_KV_F32 || ctx->kv_format == FL_KV_F16) {
        AttnArgs ka{};
        kv_layer_args(ctx, l, ka);
        if (ctx->kv_format == FL_KV_F16)
            hipLaunchKernelGGL(k_probe_kv<true>, dim3((n + 255) / 256), dim3(256), 0, ctx->stream, ka.kc, ka.vc,
                               ka.head_stride, c.head_dim, c.num_kv_heads, true, posp, M, pk, pv);
        else
            hipLaunchKernelGGL(k_probe_kv<false>, dim3((n + 255) / 256), dim3(256), 0, ctx->stream, ka.kc, ka.vc,
                               ka.head_stride, c.head_dim, c.num_kv_heads, false, posp, M, pk, pv);
        HIPCHK(ctx, hipGetLastError());
        return 0;
    }
    int rc = probe_copy(ctx, PR_K, stage_k, (size_t)n * 4);
    return rc ? rc : probe_copy(ctx, PR_V, stage_v, (size_t)n * 4);
}

// QKV matvec and decode attention of layer l as one launch (fused.hip), for
// fp16 caches with a matching instantiation.  Returns 0 when launched, 1 when
// not applicable (the caller launches the two kernels), -rc on an error.
static int launch_qkv_attention(fl_ctx *ctx, const fl_weight &w, const float *norm_w, int norm_pro, float eps,
                                int l, const QkvEpi &qe, float *attn_out) {
    const fl_model_config &c = ctx->cfg;
    const int nkv = c.num_kv_heads, D = c.head_dim, G = c.num_heads / nkv;
    if (!ctx->fuse_attn || ctx->kv_format != FL_KV_F16 || nkv < 1 || nkv > kFuseErr - kFuseCount) return 1;
    if (w.rows != qe.nq + 2 * qe.nk) return -fail(ctx, FL_E_INVALID, "fused QKV rows %d do not match the heads", w.rows);
    const MvsPlan p = mvs_plan(w.format, w.rows, w.cols, false, true);
    if (D % p.r) return 1;
    const int nt = 64 * ctx->attn_waves;  // workgroup size: the attention kernel's
    const int rx = w.format == FL_Q8_0 && mvs_steps(F_Q8_0, w.cols) <= p.su ? 1 : 0;
    MvsArgs m = mvs_args(ctx, w, norm_pro, EPI_QKV, ctx->x, norm_w, eps, nullptr, nullptr, nullptr, ctx->qkv, nullptr);
    m.qkv = qe;
    m.qkv.publish = 1;
    m.trace = nullptr;
    AttnArgs a = layer_attn_args(ctx, l);
    a.out = attn_out;
    a.knew = ctx->qkv + qe.nq;
    a.vnew = ctx->qkv + qe.nq + qe.nk;
    // one wave per row group of each kv head's query, key and value rows
    const int ngrp = (G + 2) * D / p.r, nw = nt / 64;
    const int nqwg = nkv * ((ngrp + nw - 1) / nw);
    const FuseWait fw{ctx->d_counters + kFuseCount, nqwg / nkv, ctx->d_counters + kFuseErr};
    const hipError_t e = launch_qkv_attm(w.format == FL_Q8_0 ? F_Q8_0 : F_Q4K, p, rx, D, G, nt, ctx->stream, m, a,
                                         nqwg, fw);
    if (e == hipErrorNotSupported) return 1;
    if (e != hipSuccess) return -fail(ctx, FL_E_HIP, "fused QKV + attention launch: %s", hipGetErrorString(e));
    return 0;
}

// x_given: the caller has put the step's f32 embedding row into ctx->x.
static int enqueue_step(fl_ctx *ctx, bool want_logits, bool x_given = false) {
    const fl_model_config &c = ctx->cfg;
    if (ctx->exact && ctx->kv_format != FL_KV_F32 && ctx->kv_format != FL_KV_F16)
        return fail(ctx, FL_E_UNSUPPORTED, "FL_OPT_EXACT needs an F32 or F16 KV cache (the reference's forms)");
    const int hd = c.head_dim, G = c.num_heads / c.num_kv_heads;
    const float eps = c.rms_norm_eps;
    const int norm_pro = ctx->layer_fmt == FL_Q8_0 ? PRO_NORMQ0 : PRO_NORMQ1;
    const long long sin_off = (long long)c.max_seq_len * (c.head_dim / 2);
    switch (ctx->embed.format) {
    case FL_Q8_0: hipLaunchKernelGGL(k_embed<F_Q8_0>, dim3(1), dim3(kEmbedThreads), 0, ctx->stream, ctx->embed.desc(), ctx->st, ctx->tokens, x_given ? nullptr : ctx->x, ctx->rope, sin_off, c.head_dim / 2, ctx->rope_cur); break;
    case FL_Q6K: hipLaunchKernelGGL(k_embed<F_Q6K>, dim3(1), dim3(kEmbedThreads), 0, ctx->stream, ctx->embed.desc(), ctx->st, ctx->tokens, x_given ? nullptr : ctx->x, ctx->rope, sin_off, c.head_dim / 2, ctx->rope_cur); break;
    case FL_Q4K: hipLaunchKernelGGL(k_embed<F_Q4K>, dim3(1), dim3(kEmbedThreads), 0, ctx->stream, ctx->embed.desc(), ctx->st, ctx->tokens, x_given ? nullptr : ctx->x, ctx->rope, sin_off, c.head_dim / 2, ctx->rope_cur); break;
    default: hipLaunchKernelGGL(k_embed<F_F32>, dim3(1), dim3(kEmbedThreads), 0, ctx->stream, ctx->embed.desc(), ctx->st, ctx->tokens, x_given ? nullptr : ctx->x, ctx->rope, sin_off, c.head_dim / 2, ctx->rope_cur); break;
    }
    HIPCHK(ctx, hipGetLastError());
    const size_t H = c.hidden_dim, nq = (size_t)c.num_heads * hd, nk = (size_t)c.num_kv_heads * hd;
    const size_t F = c.intermediate_dim;
    size_t poff[PR_N];
    probe_layout(c, poff);
    for (int l = 0; l < c.num_layers; l++) {
        Layer &L = ctx->layers[l];
        const bool probe = l == ctx->probe_layer && ctx->probe_dev;
        int rc;
        if (probe && (rc = probe_copy(ctx, PR_XIN, ctx->x, H * 4))) return rc;
        const QkvEpi qe = layer_qkv_epi(ctx, l);
        // one launch for QKV and attention where an instantiation fits
        float *probe_attn = probe ? (float *)(ctx->probe_dev + poff[PR_ATTN]) : nullptr;
        const int fused = ctx->exact ? 1 : launch_qkv_attention(ctx, L.qkv, L.attn_norm, norm_pro, eps, l, qe, probe_attn);
        if (fused < 0) return -fused;
        if (!fused) {
            if (probe) {
                if ((rc = probe_copy(ctx, PR_Q, ctx->qkv, nq * 4))) return rc;
                if ((rc = probe_kv(ctx, l, &ctx->st->pos, 1, ctx->qkv + nq, ctx->qkv + nq + nk))) return rc;
                if ((rc = probe_copy(ctx, PR_AQ, ctx->aq, nq))) return rc;
                if ((rc = probe_copy(ctx, PR_AS, ctx->as, nq / 32 * 4))) return rc;
            }
        } else {
        // measurement: QKV on pre-quantized codes (wrong values, the time of
        // a QKV without its norm prologue)
#ifdef FLARE_MV_TRACE
        static const int trace_layer = measure_env("FLARE_MV_TRACE_LAYER") ? atoi(measure_env("FLARE_MV_TRACE_LAYER")) : -1;
        g_trace_off = trace_layer >= 0 && l != trace_layer;
#endif
        static const bool qkv_preq = measure_env("FLARE_QKV_PREQ") != nullptr;
        if (qkv_preq && !ctx->exact)
            rc = launch_q8in(ctx, L.qkv, PRO_LOADQ, EPI_QKV, nullptr, nullptr, 0.f, ctx->hq, ctx->hs, ctx->hsum,
                             ctx->qkv, nullptr, &qe);
        else
        rc = launch_q8in(ctx, L.qkv, norm_pro, EPI_QKV, ctx->x, L.attn_norm, eps, nullptr, nullptr, nullptr,
                         ctx->qkv, nullptr, &qe);
#ifdef FLARE_MV_TRACE
        g_trace_off = trace_layer >= 0;
#endif
        if (rc) return rc;
        if (probe) {
            if ((rc = probe_copy(ctx, PR_Q, ctx->qkv, nq * 4))) return rc;
            // Q8 / KIVI: the f32 rows after q that the attention kernel quantizes
            if ((rc = probe_kv(ctx, l, &ctx->st->pos, 1, ctx->qkv + nq, ctx->qkv + nq + nk))) return rc;
        }
        if (ctx->exact) {
            // reference-order attention, then quantize_input_q8_0_into of its output
            AttnArgs a = layer_attn_args(ctx, l);
            SeqAttnArgs sa{};
            sa.q = ctx->qkv;
            sa.kc = a.kc;
            sa.vc = a.vc;
            sa.head_stride = a.head_stride;
            sa.D = hd;
            sa.group = G;
            sa.slots = ctx->kv_slots;
            sa.posp = &ctx->st->pos;
            sa.scores = ctx->seq_scores;
            sa.out = ctx->attn;
            HIPCHK(ctx, launch_attn_seq(ctx->kv_format == FL_KV_F16, ctx->stream, sa, c.num_heads));
            const int nblk = c.num_heads * hd / 32;
            hipLaunchKernelGGL(k_quantize, dim3((nblk + kThreads - 1) / kThreads), dim3(kThreads), 0, ctx->stream,
                               ctx->attn, nblk, ctx->aq, ctx->as, ctx->asum);
            HIPCHK(ctx, hipGetLastError());
            if (probe && (rc = probe_copy(ctx, PR_ATTN, ctx->attn, nq * 4))) return rc;
        } else {
            AttnArgs a = layer_attn_args(ctx, l);
            if (probe) a.out = probe_attn;  // also the f32 output
#ifdef FLARE_ATTN_TRACE
            // trace builds: FLARE_ATTN_TRACE_LAYER = l records layer l's launch
            if (measure_env("FLARE_ATTN_TRACE_LAYER") && l == atoi(measure_env("FLARE_ATTN_TRACE_LAYER")))
                a.trace = ctx->bench_trace;
#endif
            rc = launch_attention(ctx, ctx->kv_format, hd, G, a);
            if (rc) return rc;
        }
        if (probe) {
            if ((rc = probe_copy(ctx, PR_AQ, ctx->aq, nq))) return rc;
            if ((rc = probe_copy(ctx, PR_AS, ctx->as, nq / 32 * 4))) return rc;
        }
        }
        rc = launch_q8in(ctx, L.wo, PRO_LOADQ, EPI_ADD, nullptr, nullptr, 0.f, ctx->aq, ctx->as, ctx->asum, ctx->x,
                         nullptr);
        if (rc) return rc;
        if (probe && (rc = probe_copy(ctx, PR_XMID, ctx->x, H * 4))) return rc;
        static const bool gu_preq = measure_env("FLARE_GU_PREQ") != nullptr;
        if (gu_preq && !ctx->exact)
            rc = launch_gateup(ctx, L.gu, PRO_LOADQ, nullptr, nullptr, 0.f, ctx->aq, ctx->as, ctx->asum, ctx->hq,
                               ctx->hs, ctx->hsum, nullptr);
        else
        rc = launch_gateup(ctx, L.gu, norm_pro, ctx->x, L.ffn_norm, eps, nullptr, nullptr, nullptr, ctx->hq, ctx->hs,
                           ctx->hsum, nullptr);
        if (rc) return rc;
        if (probe) {
            if ((rc = probe_copy(ctx, PR_HQ, ctx->hq, F))) return rc;
            if ((rc = probe_copy(ctx, PR_HS, ctx->hs, F / 32 * 4))) return rc;
        }
        rc = launch_q8in(ctx, L.down, PRO_LOADQ, EPI_ADD, nullptr, nullptr, 0.f, ctx->hq, ctx->hs, ctx->hsum, ctx->x,
                         nullptr);
        if (rc) return rc;
        if (probe && (rc = probe_copy(ctx, PR_XOUT, ctx->x, H * 4))) return rc;
    }
    if (ctx->probe_dev && ctx->probe_layer >= 0) {
        int rc = probe_copy(ctx, PR_XFIN, ctx->x, H * 4);
        if (rc) return rc;
    }
    // output projection (forward_greedy, model.rs:1898-1932)
    const fl_weight &O = ctx->tied ? ctx->embed : ctx->output;
    const bool q8out = !ctx->tied && ((O.format == FL_Q8_0 && ctx->layer_fmt == FL_Q8_0) ||
                                      (O.format == FL_Q4K && ctx->layer_fmt == FL_Q4K));
    int rc;
    if (q8out) {
        rc = launch_q8in(ctx, O, PRO_NORMQ1, want_logits ? EPI_STORE : EPI_ARGMAX, ctx->x, ctx->out_norm, eps,
                         nullptr, nullptr, nullptr, ctx->logits, &ctx->st->argmax);
    } else if (ctx->exact) {
        // rmsnorm_into, then matvec_argmax_f32 / matvec_into over the dequantized weight
        HIPCHK(ctx, launch_rmsnorm_seq(ctx->stream, ctx->x, ctx->out_norm, c.hidden_dim, eps, ctx->seq_xn));
        HIPCHK(ctx, launch_out_seq(O.format, ctx->stream, O.desc(), ctx->seq_xn, want_logits ? ctx->logits : nullptr,
                                   &ctx->st->argmax));
        rc = 0;
    } else {
        if (O.format == FL_Q4K) return fail(ctx, FL_E_UNSUPPORTED, "Q4_K output with Q8_0 layers");
        rc = launch_f32in(ctx, O, 1, want_logits ? EPI_STORE : EPI_ARGMAX, ctx->x, ctx->out_norm, eps, ctx->logits,
                          &ctx->st->argmax);
    }
    return rc;
}

// FLARE_NO_GRAPH=1: enqueue the step's kernels directly instead of replaying a
// HIP graph (identical kernels; for profilers that cannot follow graphs).
// Graphs are also off under rocprofv3 counter collection (it sets
// ROCPROF_COUNTER_COLLECTION): the one counter run that replayed graphs
// died with a SIGSEGV in a profiler-side thread at the first capture.
static bool use_graph() {
    static const bool g = getenv("FLARE_NO_GRAPH") == nullptr && getenv("ROCPROF_COUNTER_COLLECTION") == nullptr;
    return g;
}

static int launch_step(fl_ctx *ctx) {
    if (!use_graph()) return enqueue_step(ctx, false);
    HIPCHK(ctx, hipGraphLaunch(ctx->gexec, ctx->stream));
    return 0;
}

static int ensure_graph(fl_ctx *ctx) {
    if (!use_graph()) {
        ctx->graph_ready = true;
        return 0;
    }
    if (ctx->gexec) return 0;
    HIPCHK(ctx, hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
    int rc = enqueue_step(ctx, false);
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(ctx->stream, &g);
    if (rc) {
        if (g) (void)hipGraphDestroy(g);
        return rc;
    }
    if (e != hipSuccess) return fail(ctx, FL_E_HIP, "graph capture failed: %s", hipGetErrorString(e));
    ctx->graph = g;
    HIPCHK(ctx, hipGraphInstantiate(&ctx->gexec, g, nullptr, nullptr, 0));
    ctx->graph_ready = true;
    return 0;
}

// One decode step at `pos`: the token's embedding row (embedding == nullptr)
// or the caller's f32 embedding row.
static int decode_step(fl_ctx *ctx, uint32_t token, const float *embedding, int pos, float *out_logits,
                       int32_t *out_token, float *out_val) {
    if (!ctx) return fail(nullptr, FL_E_INVALID, "null ctx");
    if (!ctx->have_weights) return fail(ctx, FL_E_STATE, "weights not uploaded");
    const fl_model_config &c = ctx->cfg;
    if (pos < 0 || pos >= c.max_seq_len)
        return fail(ctx, FL_E_INVALID, "pos %d outside the KV cache (max_seq_len %d)", pos, c.max_seq_len);
    if ((int)token >= c.vocab_size) return fail(ctx, FL_E_INVALID, "token %u >= vocab", token);
    const int tok = (int)token;
    DevState hs{};
    hs.step = pos;
    hs.pos = pos;
    hs.n_prompt = pos + 1;
    HIPCHK(ctx, hipMemcpyAsync(ctx->tokens + pos, &tok, 4, hipMemcpyHostToDevice, ctx->stream));
    HIPCHK(ctx, hipMemcpyAsync(ctx->st, &hs, sizeof hs, hipMemcpyHostToDevice, ctx->stream));
    if (embedding)
        HIPCHK(ctx, hipMemcpyAsync(ctx->x, embedding, (size_t)c.hidden_dim * 4, hipMemcpyHostToDevice, ctx->stream));
    if (out_logits || embedding || ctx->probe_layer >= 0) {
        // enqueued directly: the captured step dequantizes the token's row
        // (and carries no probe copies)
        int rc = enqueue_step(ctx, out_logits != nullptr, embedding != nullptr);
        if (rc) return rc;
    } else {
        int rc = ensure_graph(ctx);
        if (!rc) rc = launch_step(ctx);
        if (rc) return rc;
    }
    DevState out{};
    HIPCHK(ctx, hipMemcpyAsync(&out, ctx->st, sizeof out, hipMemcpyDeviceToHost, ctx->stream));
    if (out_logits)
        HIPCHK(ctx, hipMemcpyAsync(out_logits, ctx->logits, (size_t)c.vocab_size * 4, hipMemcpyDeviceToHost,
                                   ctx->stream));
    if (ctx->probe_layer >= 0 && ctx->probe_host)
        HIPCHK(ctx, hipMemcpyAsync(ctx->probe_host, ctx->probe_dev, ctx->probe_bytes, hipMemcpyDeviceToHost,
                                   ctx->stream));
    HIPCHK(ctx, hipStreamSynchronize(ctx->stream));
    if (out_logits) {
        int bi = 0;
        float bv = -INFINITY;
        for (int i = 0; i < c.vocab_size; i++)
            if (out_logits[i] > bv) { bv = out_logits[i]; bi = i; }
        if (out_token) *out_token = bi;
        if (out_val) *out_val = bv;
    } else {
        const unsigned long long k = out.argmax;
        if (out_token) *out_token = (int32_t)(0xFFFFFFFFu - (uint32_t)(k & 0xFFFFFFFFull));
        uint32_t u = (uint32_t)(k >> 32);
        u = (u & 0x80000000u) ? (u & 0x7FFFFFFFu) : ~u;
        float v;
        std::memcpy(&v, &u, 4);
        if (out_val) *out_val = v;
    }
    return 0;
}

int fl_probe_layout(const fl_ctx *ctx, size_t *offsets, int n) {
    if (!ctx || !ctx->have_cfg || !offsets || n < PR_N) return -1;
    return (int)probe_layout(ctx->cfg, offsets);
}

int fl_probe_layer(fl_ctx *ctx, int layer, void *host_buf) {
    if (!ctx || !ctx->have_cfg) return fail(ctx, FL_E_STATE, "no model");
    if (layer < 0) {
        ctx->probe_layer = -1;
        ctx->probe_host = nullptr;
        return 0;
    }
    if (layer >= ctx->cfg.num_layers || !host_buf) return fail(ctx, FL_E_INVALID, "layer %d / null buffer", layer);
    size_t off[PR_N];
    const size_t bytes = probe_layout(ctx->cfg, off);
    if (!ctx->probe_dev) {
        ALLOC(ctx, ctx->probe_dev, bytes);
        HIPCHK(ctx, hipMemset(ctx->probe_dev, 0, bytes));
        ctx->probe_bytes = bytes;
    }
    ctx->probe_layer = layer;
    ctx->probe_host = host_buf;
    return 0;
}

int fl_decode_step(fl_ctx *ctx, uint32_t token, int pos, float *out_logits, int32_t *out_token, float *out_val) {
    return decode_step(ctx, token, nullptr, pos, out_logits, out_token, out_val);
}

int fl_decode_step_embed(fl_ctx *ctx, const float *embedding, int pos, float *out_logits, int32_t *out_token,
                         float *out_val) {
    if (!embedding) return fail(ctx, FL_E_INVALID, "null embedding");
    return decode_step(ctx, 0u, embedding, pos, out_logits, out_token, out_val);
}

int fl_generate(fl_ctx *ctx, const uint32_t *prompt, int n_prompt, int n_gen, uint32_t *out_tokens) {
    if (!ctx || !prompt || !out_tokens) return fail(ctx, FL_E_INVALID, "null argument");
    if (!ctx->have_weights) return fail(ctx, FL_E_STATE, "weights not uploaded");
    const fl_model_config &c = ctx->cfg;
    if (n_prompt <= 0 || n_gen <= 0) return fail(ctx, FL_E_INVALID, "n_prompt and n_gen must be positive");
    const int steps = n_prompt + n_gen - 1;
    if (steps > c.max_seq_len)
        return fail(ctx, FL_E_INVALID, "prompt+generation (%d) exceeds max_seq_len %d", steps, c.max_seq_len);
    for (int i = 0; i < n_prompt; i++)
        if ((int)prompt[i] >= c.vocab_size) return fail(ctx, FL_E_INVALID, "prompt token %u >= vocab", prompt[i]);
    int rc = ensure_graph(ctx);
    if (rc) return rc;
    std::vector<int> toks(prompt, prompt + n_prompt);
    DevState hs{};
    hs.n_prompt = n_prompt;
    HIPCHK(ctx, hipMemcpyAsync(ctx->tokens, toks.data(), (size_t)n_prompt * 4, hipMemcpyHostToDevice, ctx->stream));
    HIPCHK(ctx, hipMemcpyAsync(ctx->st, &hs, sizeof hs, hipMemcpyHostToDevice, ctx->stream));
    for (int s = 0; s < steps; s++) {
        rc = launch_step(ctx);
        if (rc) return rc;
    }
    std::vector<int> gen((size_t)std::max(n_gen - 1, 1));
    DevState out{};
    if (n_gen > 1)
        HIPCHK(ctx, hipMemcpyAsync(gen.data(), ctx->tokens + n_prompt, (size_t)(n_gen - 1) * 4, hipMemcpyDeviceToHost,
                                   ctx->stream));
    HIPCHK(ctx, hipMemcpyAsync(&out, ctx->st, sizeof out, hipMemcpyDeviceToHost, ctx->stream));
    HIPCHK(ctx, hipStreamSynchronize(ctx->stream));
    for (int i = 0; i < n_gen - 1; i++) out_tokens[i] = (uint32_t)gen[i];
    out_tokens[n_gen - 1] = 0xFFFFFFFFu - (uint32_t)(out.argmax & 0xFFFFFFFFull);
    return 0;
}

int fl_decode_run(fl_ctx *ctx, uint32_t token, int pos, int n_steps, uint32_t *out_tokens) {
    if (!ctx || !out_tokens) return fail(ctx, FL_E_INVALID, "null argument");
    if (!ctx->have_weights) return fail(ctx, FL_E_STATE, "weights not uploaded");
    const fl_model_config &c = ctx->cfg;
    if (n_steps <= 0) return fail(ctx, FL_E_INVALID, "n_steps must be positive");
    if (pos < 0 || pos + n_steps > c.max_seq_len)
        return fail(ctx, FL_E_INVALID, "steps [%d, %d) outside the KV cache (max_seq_len %d)", pos, pos + n_steps,
                    c.max_seq_len);
    if ((int)token >= c.vocab_size) return fail(ctx, FL_E_INVALID, "token %u >= vocab", token);
    int rc = ensure_graph(ctx);
    if (rc) return rc;
    const int tok = (int)token;
    DevState hs{};
    hs.step = pos;
    hs.pos = pos;
    hs.n_prompt = pos + 1;  // step `pos` reads tokens[pos]; later steps take the previous argmax
    HIPCHK(ctx, hipMemcpyAsync(ctx->tokens + pos, &tok, 4, hipMemcpyHostToDevice, ctx->stream));
    HIPCHK(ctx, hipMemcpyAsync(ctx->st, &hs, sizeof hs, hipMemcpyHostToDevice, ctx->stream));
    for (int s = 0; s < n_steps; s++) {
        rc = launch_step(ctx);
        if (rc) return rc;
    }
    std::vector<int> gen((size_t)std::max(n_steps - 1, 1));
    DevState out{};
    if (n_steps > 1)
        HIPCHK(ctx, hipMemcpyAsync(gen.data(), ctx->tokens + pos + 1, (size_t)(n_steps - 1) * 4,
                                   hipMemcpyDeviceToHost, ctx->stream));
    HIPCHK(ctx, hipMemcpyAsync(&out, ctx->st, sizeof out, hipMemcpyDeviceToHost, ctx->stream));
    HIPCHK(ctx, hipStreamSynchronize(ctx->stream));
    for (int i = 0; i < n_steps - 1; i++) out_tokens[i] = (uint32_t)gen[i];
    out_tokens[n_steps - 1] = 0xFFFFFFFFu - (uint32_t)(out.argmax & 0xFFFFFFFFull);
    return 0;
}

int fl_decode_continue(fl_ctx *ctx, int n_steps) {
    if (!ctx) return fail(nullptr, FL_E_INVALID, "null ctx");
    if (!ctx->graph_ready) return fail(ctx, FL_E_STATE, "fl_generate must run first");
    if (n_steps < 0) return fail(ctx, FL_E_INVALID, "n_steps < 0");
    DevState st{};
    HIPCHK(ctx, hipMemcpyAsync(&st, ctx->st, sizeof st, hipMemcpyDeviceToHost, ctx->stream));
    HIPCHK(ctx, hipStreamSynchronize(ctx->stream));
    if (st.step + n_steps > ctx->cfg.max_seq_len)
        return fail(ctx, FL_E_INVALID, "continuing %d steps from %d exceeds max_seq_len %d", n_steps, st.step,
                    ctx->cfg.max_seq_len);
    for (int s = 0; s < n_steps; s++) {
        const int rc = launch_step(ctx);
        if (rc) return rc;
    }
    return 0;
}

int fl_read_tokens(fl_ctx *ctx, int start, int n, uint32_t *out) {
    if (!ctx || !out) return fail(ctx, FL_E_INVALID, "null argument");
    if (!ctx->have_cfg || start < 0 || n < 0 || start + n > ctx->cfg.max_seq_len)
        return fail(ctx, FL_E_INVALID, "token range");
    HIPCHK(ctx, hipMemcpyAsync(out, ctx->tokens + start, (size_t)n * 4, hipMemcpyDeviceToHost, ctx->stream));
    HIPCHK(ctx, hipStreamSynchronize(ctx->stream));
    return 0;
}

int fl_gqa_from_cache(fl_ctx *ctx, int layer, const float *q, int seq_len, float *out) {
    if (!ctx || !q || !out) return fail(ctx, FL_E_INVALID, "null argument");
    if (!ctx->have_cfg) return fail(ctx, FL_E_STATE, "no kv cache");
    const fl_model_config &c = ctx->cfg;
    if (layer < 0 || layer >= c.num_layers) return fail(ctx, FL_E_INVALID, "layer %d", layer);
    if (seq_len <= 0 || seq_len > c.max_seq_len) return fail(ctx, FL_E_INVALID, "seq_len %d", seq_len);
    const size_t qd = (size_t)c.num_heads * c.head_dim;
    HIPCHK(ctx, hipMemcpyAsync(ctx->qkv, q, qd * 4, hipMemcpyHostToDevice, ctx->stream));
    const int pos = seq_len - 1;
    HIPCHK(ctx, hipMemcpyAsync(ctx->d_pos, &pos, 4, hipMemcpyHostToDevice, ctx->stream));
    AttnArgs a{};
    kv_layer_args(ctx, layer, a);
    a.q = ctx->qkv;
    a.posp = ctx->d_pos;
    a.nsplit = ctx->nsplit;
    a.chmin = ctx->chmin;
    a.single = ctx->single;
    a.waves = ctx->attn_waves;
    a.part = ctx->d_part;
    a.counters = ctx->d_counters;
    a.out = ctx->attn;
    int rc = launch_attention(ctx, ctx->kv_format, c.head_dim, c.num_heads / c.num_kv_heads, a);
    if (rc) return rc;
    HIPCHK(ctx, hipMemcpyAsync(out, ctx->attn, qd * 4, hipMemcpyDeviceToHost, ctx->stream));
    HIPCHK(ctx, hipStreamSynchronize(ctx->stream));
    return 0;
}

int fl_bench_attention(fl_ctx *ctx, int seq_len, int iters, double *bytes_per_launch) {
    if (!ctx || !ctx->have_cfg) return fail(ctx, FL_E_STATE, "no kv cache");
    const fl_model_config &c = ctx->cfg;
    if (seq_len <= 0 || seq_len > c.max_seq_len) return fail(ctx, FL_E_INVALID, "seq_len %d", seq_len);
    const int pos = seq_len - 1;
    HIPCHK(ctx, hipMemcpyAsync(ctx->d_pos, &pos, 4, hipMemcpyHostToDevice, ctx->stream));
    for (int i = 0; i < iters; i++) {
        AttnArgs a{};
        kv_layer_args(ctx, i % c.num_layers, a);
        a.q = ctx->qkv;
        a.posp = ctx->d_pos;
        a.nsplit = ctx->nsplit;
        a.chmin = ctx->chmin;
        a.single = ctx->single;
        a.waves = ctx->attn_waves;
        a.part = ctx->d_part;
        a.counters = ctx->d_counters;
        a.out = ctx->attn;
        const int rc = launch_attention(ctx, ctx->kv_format, c.head_dim, c.num_heads / c.num_kv_heads, a);
        if (rc) return rc;
    }
    if (bytes_per_launch) *bytes_per_launch = attn_bytes(ctx, seq_len);
    HIPCHK(ctx, hipStreamSynchronize(ctx->stream));  // pos staged from the host stack
    return 0;
}

// ---- speculative verify -------------------------------------------------------


static int verify_alloc(fl_ctx *ctx) {
    if (ctx->have_verify) return 0;
    const fl_model_config &c = ctx->cfg;
    // sized for prefill passes (the largest batches)
    const size_t M = kPrefillTokens, H = c.hidden_dim, qd = (size_t)c.num_heads * c.head_dim;
    const size_t kvd = (size_t)c.num_kv_heads * c.head_dim, F = c.intermediate_dim;
    const size_t kmax = std::max({H, qd, F});
    const size_t rmax = std::max({qd + 2 * kvd, 2 * F, H});
    ALLOC(ctx, ctx->vx, M * H * 4);
    ALLOC(ctx, ctx->vx2, M * H * 4);
    ALLOC(ctx, ctx->vq, M * qd * 4);
    ALLOC(ctx, ctx->vk, M * kvd * 4);
    ALLOC(ctx, ctx->vv, M * kvd * 4);
    ctx->vpart_floats = (size_t)kPrefillMaxKsplit * M * rmax;
    ALLOC(ctx, ctx->vpart, ctx->vpart_floats * 4);
    ALLOC(ctx, ctx->vxq, M * kmax);
    ALLOC(ctx, ctx->vxs, M * (kmax / 32) * 4);
    ALLOC(ctx, ctx->vxsum, M * (kmax / 32) * 4);
    ALLOC(ctx, ctx->vaq, M * qd);
    ALLOC(ctx, ctx->vas, M * (qd / 32) * 4);
    ALLOC(ctx, ctx->vasum, M * (qd / 32) * 4);
    ALLOC(ctx, ctx->vtok, M * 4);
    ALLOC(ctx, ctx->vpos, 4);
    ALLOC(ctx, ctx->vslots, M * 8);
    ALLOC(ctx, ctx->vhq, M * F);
    ALLOC(ctx, ctx->vhs, M * (F / 32) * 4);
    ALLOC(ctx, ctx->vhsum, M * (F / 32) * 4);
    ALLOC(ctx, ctx->vcnt, kVerifyCounters * 4);
    HIPCHK(ctx, hipMemset(ctx->vcnt, 0, kVerifyCounters * 4));  // the kernels leave them at zero
    ctx->have_verify = true;
    return 0;
}

// K chunks of a verify GEMM for M tokens: about 2048 waves (one 16-row tile
// x one chunk each), at most kVerifyMaxKsplit.  Returns the split count and
// sets the chunk (units per split, every chunk non-empty: the reducers sum
// all ksplit partial sets).  The paired Q8_0 kernel (M <= 8) walks rounds of
// 8 blocks, so its chunks are whole rounds.
// Largest dynamic LDS one workgroup may use on this device.
static size_t max_lds_per_block() {
    static const size_t v = [] {
        int dev = 0, b = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&b, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || b <= 0)
            return (size_t)65536;
        return (size_t)b;
    }();
    return v;
}

// (The M > 16 prefill batches allow up to kPrefillMaxKsplit splits and
// shrink the chunk until the staged activations of all M rows fit in LDS.)
static int verify_split(const fl_weight &w, int M, int &chunk) {
    const int tiles = (w.rows + 15) / 16;
    const int units = w.format == FL_Q4K ? w.cols / 256 : w.cols / 32;
    const int ubytes = w.format == FL_Q4K ? 256 : 32;
    const int maxks = M > kVerifyMaxTokens ? kPrefillMaxKsplit : kVerifyMaxKsplit;
    static const int target = measure_env("FLARE_VG_WAVES") ? atoi(measure_env("FLARE_VG_WAVES")) : 2048;  // tuning
    const int want = std::max(1, std::min({units, maxks, (target + tiles - 1) / tiles}));
    if (M > kVerifyMaxTokens && w.cols % 256 == 0) {
        // the prefill kernel walks 256-value steps: chunk counts steps
        const int steps = w.cols / 256;
        const int ks = std::max(1, std::min({steps, maxks, (target + tiles - 1) / tiles}));
        chunk = (steps + ks - 1) / ks;
        return (steps + chunk - 1) / chunk;
    }
    chunk = (units + want - 1) / want;
    if (w.format == FL_Q8_0 && M <= 8) chunk = std::min(units, (chunk + 7) / 8 * 8);
    if (M > kVerifyMaxTokens) {
        auto lds = [&](int ch) {
            const size_t kn = (size_t)ch * ubytes;
            return (((size_t)M * (kn + 32) + 15) & ~(size_t)15) + (size_t)M * (kn / 32) * 8;
        };
        while (chunk > 1 && lds(chunk) > max_lds_per_block()) chunk--;
        if ((units + chunk - 1) / chunk > maxks) chunk = (units + maxks - 1) / maxks;
    }
    return (units + chunk - 1) / chunk;
}

static int verify_gemm(fl_ctx *ctx, const fl_weight &w, int M, const int8_t *xq, const float *xs, const int *xsum,
                       int &ksplit, const VgArgs *post = nullptr) {
    VgArgs a{};
    if (post) a = *post;  // fused epilogue fields
    a.W = w.desc();
    a.xq = xq;
    a.xs = xs;
    a.xsum = xsum;
    a.M = M;
    a.ksplit = ksplit = verify_split(w, M, a.chunk);
    a.part = ctx->vpart;
    if ((size_t)ksplit * M * w.rows > ctx->vpart_floats) return fail(ctx, FL_E_INVALID, "verify partials too small");
    const hipError_t e = launch_vgemm(w.format, ctx->stream, a);
    if (e == hipErrorNotSupported) return fail(ctx, FL_E_UNSUPPORTED, "no verify GEMM for format %d", w.format);
    HIPCHK(ctx, e);
    return 0;
}

int fl_op_batched_matvec_q8in(fl_ctx *ctx, const fl_weight *w, int n_tokens, const int8_t *q, const float *scales,
                               const int32_t *sums, float *out) {
    if (!ctx || !w || !q || !scales || !sums || !out) return fail(ctx, FL_E_INVALID, "null argument");
    if (n_tokens < 1 || n_tokens > kPrefillTokens)
        return fail(ctx, FL_E_INVALID, "batch of %d tokens (1..%d)", n_tokens, kPrefillTokens);
    if (w->format != FL_Q8_0 && w->format != FL_Q4K) return fail(ctx, FL_E_UNSUPPORTED, "format %d", w->format);
    // partials of this op live in their own buffer (sized for this weight)
    int chunk = 0;
    const int ks = verify_split(*w, n_tokens, chunk);
    const size_t need = (size_t)ks * n_tokens * w->rows;
    float *part = nullptr;
    ALLOC(ctx, part, need * 4);
    VgArgs a{};
    a.W = w->desc();
    a.xq = q;
    a.xs = scales;
    a.xsum = sums;
    a.M = n_tokens;
    a.ksplit = ks;
    a.chunk = chunk;
    a.part = part;
    hipError_t e = launch_vgemm(w->format, ctx->stream, a);
    if (e == hipSuccess) e = launch_v_store(ctx->stream, part, ks, n_tokens, w->rows, out);
    const hipError_t e2 = hipStreamSynchronize(ctx->stream);
    (void)hipFree(part);
    HIPCHK(ctx, e);
    HIPCHK(ctx, e2);
    return 0;
}

int fl_op_batched_block_dots(fl_ctx *ctx, const fl_weight *w, int n_tokens, const int8_t *q, const float *scales,
                             const int32_t *sums, int32_t *dots) {
    if (!ctx || !w || !q || !scales || !sums || !dots) return fail(ctx, FL_E_INVALID, "null argument");
    if (n_tokens < 1 || n_tokens > kPrefillTokens)
        return fail(ctx, FL_E_INVALID, "batch of %d tokens (1..%d)", n_tokens, kPrefillTokens);
    if (w->format != FL_Q8_0 && w->format != FL_Q4K) return fail(ctx, FL_E_UNSUPPORTED, "format %d", w->format);
    int chunk = 0;
    const int ks = verify_split(*w, n_tokens, chunk);
    float *part = nullptr;
    ALLOC(ctx, part, (size_t)ks * n_tokens * w->rows * 4);
    VgArgs a{};
    a.W = w->desc();
    a.xq = q;
    a.xs = scales;
    a.xsum = sums;
    a.M = n_tokens;
    a.ksplit = ks;
    a.chunk = chunk;
    a.part = part;
    a.dots = dots;
    const hipError_t e = launch_vgemm(w->format, ctx->stream, a);
    const hipError_t e2 = hipStreamSynchronize(ctx->stream);
    (void)hipFree(part);
    HIPCHK(ctx, e);
    HIPCHK(ctx, e2);
    return 0;
}

int fl_op_batched_matvec_q8in_noalloc(fl_ctx *ctx, const fl_weight *w, int n_tokens, const int8_t *q,
                                      const float *scales, const int32_t *sums, float *out) {
    if (!ctx || !w || !q || !scales || !sums || !out) return fail(ctx, FL_E_INVALID, "null argument");
    if (n_tokens < 1 || n_tokens > kVerifyMaxTokens)
        return fail(ctx, FL_E_INVALID, "batch of %d tokens (1..%d)", n_tokens, kVerifyMaxTokens);
    if (w->format != FL_Q8_0 && w->format != FL_Q4K) return fail(ctx, FL_E_UNSUPPORTED, "format %d", w->format);
    if (!ctx->scratch) return fail(ctx, FL_E_STATE, "no scratch array on this device");
    // same K split (and so the same kernels and summation order) as the
    // allocating entry point; partials in the device's scratch array
    int chunk = 0;
    const int ks = verify_split(*w, n_tokens, chunk);
    const size_t need = (size_t)ks * n_tokens * w->rows;
    if (need > kNoAllocScratchFloats)
        return fail(ctx, FL_E_INVALID,
                    "batched matvec needs %zu floats of K-split partials (%d splits x %d tokens x %d rows); the "
                    "no-alloc scratch holds %zu",
                    need, ks, n_tokens, w->rows, kNoAllocScratchFloats);
    VgArgs a{};
    a.W = w->desc();
    a.xq = q;
    a.xs = scales;
    a.xsum = sums;
    a.M = n_tokens;
    a.ksplit = ks;
    a.chunk = chunk;
    a.part = ctx->scratch;  // every partial is written before it is read: nothing to clear
    HIPCHK(ctx, launch_vgemm(w->format, ctx->stream, a));
    HIPCHK(ctx, launch_v_store(ctx->stream, ctx->scratch, ks, n_tokens, w->rows, out));
    return 0;
}

int fl_op_batched_dequant_matmul(fl_ctx *ctx, const fl_weight *w, const float *input, int batch, float *out) {
    if (!ctx || !w || !input || !out) return fail(ctx, FL_E_INVALID, "null argument");
    if (batch < 1) return fail(ctx, FL_E_INVALID, "batch %d", batch);
    if (w->format != FL_Q8_0 && w->format != FL_Q4K)
        return fail(ctx, FL_E_UNSUPPORTED, "batched_dequant_matmul for format %d (Q8_0 / Q4_K)", w->format);
    // quantize_input_q8_0_into of every input row (rows are contiguous and
    // cols % 32 == 0, so the blocks of all rows are one array)
    const size_t cols = (size_t)w->cols, nblk = (size_t)batch * cols / 32;
    int8_t *q = nullptr;
    float *sc = nullptr;
    int *sum = nullptr;
    int rc = dev_alloc(ctx, (void **)&q, (size_t)batch * cols);
    if (!rc) rc = dev_alloc(ctx, (void **)&sc, nblk * 4);
    if (!rc) rc = dev_alloc(ctx, (void **)&sum, nblk * 4);
    if (!rc) {
        hipLaunchKernelGGL(k_quantize, dim3((unsigned)((nblk + kThreads - 1) / kThreads)), dim3(kThreads), 0,
                           ctx->stream, input, (int)nblk, q, sc, sum);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) rc = fail(ctx, FL_E_HIP, "quantize: %s", hipGetErrorString(e));
    }
    // then the per-row quantized matvec, kVerifyMaxTokens rows per GEMM
    for (int b0 = 0; !rc && b0 < batch; b0 += kVerifyMaxTokens) {
        const int n = std::min(kVerifyMaxTokens, batch - b0);
        rc = fl_op_batched_matvec_q8in(ctx, w, n, q + (size_t)b0 * cols, sc + (size_t)b0 * (cols / 32),
                                       sum + (size_t)b0 * (cols / 32), out + (size_t)b0 * w->rows);
    }
    (void)hipStreamSynchronize(ctx->stream);
    if (q) (void)hipFree(q);
    if (sc) (void)hipFree(sc);
    if (sum) (void)hipFree(sum);
    return rc;
}

int fl_op_prefill_attention(fl_ctx *ctx, const float *q, const float *k, const float *v, int seq_len, int num_heads,
                            int num_kv_heads, int head_dim, float *out) {
    if (!ctx || !q || !k || !v || !out) return fail(ctx, FL_E_INVALID, "null argument");
    if (seq_len < 1 || num_kv_heads <= 0 || num_heads % num_kv_heads || num_kv_heads > 1024)
        return fail(ctx, FL_E_INVALID, "bad prefill attention shape");
    const int G = num_heads / num_kv_heads;
    if (!attn_supported(head_dim, G)) return fail(ctx, FL_E_UNSUPPORTED, "head_dim %d / group %d", head_dim, G);
    // queries z0 .. z0+Z-1 per launch (grid z), each attending 0..z0+z of the
    // token-major rows; one set of split partials and counters per query
    const int Z = std::min(seq_len, std::max(1, 1024 / num_kv_heads));
    int ns, chmin;
    choose_splits(seq_len, num_kv_heads, head_dim, ns, chmin);
    ns = std::min(ns, 8);
    int rc = ensure_part(ctx, (size_t)Z * num_kv_heads * ns * G * (head_dim + 2));
    if (rc) return rc;
    const int qd = num_heads * head_dim;
    std::vector<int> starts;
    for (int z0 = 0; z0 < seq_len; z0 += Z) starts.push_back(z0);
    int *dstart = nullptr;
    rc = dev_alloc(ctx, (void **)&dstart, starts.size() * 4);
    if (rc) return rc;
    hipError_t e = hipMemcpyAsync(dstart, starts.data(), starts.size() * 4, hipMemcpyHostToDevice, ctx->stream);
    for (size_t c = 0; e == hipSuccess && c < starts.size(); c++) {
        const int z0 = starts[c], nq = std::min(Z, seq_len - z0);
        AttnArgs a{};
        a.q = q + (size_t)z0 * qd;
        a.kc = k;
        a.vc = v;
        a.tok_stride = (long long)num_kv_heads * head_dim;  // [token][kv_head][head_dim]
        a.head_stride = head_dim;
        a.posp = dstart + c;
        a.nkv = num_kv_heads;
        a.nsplit = ns;
        a.chmin = chmin;
        a.single = kAttmSingle;
        a.part = ctx->d_part;
        a.counters = ctx->d_counters;
        a.out = out + (size_t)z0 * qd;
        a.qstride = qd;
        a.ostride = qd;
        e = launch_attn(FL_KV_F32, head_dim, G, ctx->stream, a, nq);
    }
    const hipError_t es = hipStreamSynchronize(ctx->stream);
    (void)hipFree(dstart);
    HIPCHK(ctx, e);
    HIPCHK(ctx, es);
    return 0;
}

int fl_op_batched_matvec_f32in(fl_ctx *ctx, const fl_weight *w, int n_tokens, const float *x, float *out) {
    if (!ctx || !w || !x || !out) return fail(ctx, FL_E_INVALID, "null argument");
    if (w->format != FL_Q6K && w->format != FL_Q8_0) return fail(ctx, FL_E_UNSUPPORTED, "format %d", w->format);
    if (n_tokens < 1 || n_tokens > kMvoMaxTokens)
        return fail(ctx, FL_E_INVALID, "batch of %d tokens (1..%d)", n_tokens, kMvoMaxTokens);
    MvoArgs a{};
    a.W = w->desc();
    a.x = x;
    a.nw = nullptr;
    a.M = n_tokens;
    a.epi = EPI_STORE;
    a.out = out;
    HIPCHK(ctx, launch_mvo(w->format, ctx->stream, a));
    return 0;
}

// The verify pass for M tokens at the device positions vpos.. (tokens in
// vtok, vslots cleared); dev_pos: the cache writers read the position from the
// device too (graph capture), pos0 is then only used for planning checks.
// What a pass of enqueue_verify produces: the greedy key of every token
// (speculative verify), nothing (prefill chunks before the last), or the key
// / the logits of the last token only (the last prefill chunk).
enum { VOUT_ALL = 0, VOUT_NONE = 1, VOUT_LAST_ARGMAX = 2, VOUT_LAST_LOGITS = 3 };

static int enqueue_verify(fl_ctx *ctx, int M, int pos0, bool dev_pos, int out_mode = VOUT_ALL) {
    const fl_model_config &c = ctx->cfg;
    int rc;
    const int H = c.hidden_dim, D = c.head_dim, G = c.num_heads / c.num_kv_heads;
    const int qd = c.num_heads * D, kvd = c.num_kv_heads * D, F = c.intermediate_dim;
    const float eps = c.rms_norm_eps;
    const int pro = ctx->layer_fmt == FL_Q8_0 ? PRO_NORMQ0 : PRO_NORMQ1;
    hipStream_t st = ctx->stream;
    float *xa = ctx->vx;
    HIPCHK(ctx, launch_v_embed(ctx->embed.format, st, ctx->embed.desc(), ctx->vtok, M, xa));
    // Q4_K layers, up to 8 tokens: the QKV post and SiLU run inside the GEMMs
    const bool fuse = ctx->verify_fuse && ctx->layer_fmt == FL_Q4K && M <= 8 &&
                      std::max(qd + 2 * kvd, 2 * F) / 64 <= kVerifyCounters;
    int ks_down = 0;
    for (int l = 0; l < c.num_layers; l++) {
        Layer &L = ctx->layers[l];
        int ks;
        // attention block (model.rs:2016-2311), M tokens at positions pos0..pos0+M-1;
        // the previous layer's down projection is added to x here
        // the previous layer's down projection is added to x here (layer 0:
        // norm only), one workgroup per token
        HIPCHK(ctx, launch_v_resnorm(pro, st, l ? ctx->vpart : nullptr, ks_down, M, H, xa, L.attn_norm, eps, ctx->vxq,
                                     ctx->vxs, ctx->vxsum));
        const bool probe = l == ctx->probe_layer && ctx->probe_dev && M <= kProbeTokens;
        if (probe) {
            if ((rc = probe_copy(ctx, PR_XIN, xa, (size_t)M * H * 4))) return rc;
            if ((rc = probe_copy(ctx, PR_XQ, ctx->vxq, (size_t)M * H))) return rc;
            if ((rc = probe_copy(ctx, PR_XS, ctx->vxs, (size_t)M * (H / 32) * 4))) return rc;
        }
        AttnArgs a{};
        kv_layer_args(ctx, l, a);
        // RoPE'd q; K and V straight into F16 / F32 cache slots, else staged
        const bool plain = ctx->kv_format == FL_KV_F16 || ctx->kv_format == FL_KV_F32;
        VgArgs pq{};
        pq.qp.nq = qd;
        pq.qp.nk = kvd;
        pq.qp.D = D;
        pq.qp.rope = ctx->rope;
        pq.qp.sin_off = (long long)c.max_seq_len * (D / 2);
        pq.qp.pos0p = ctx->vpos;
        pq.qp.Q = ctx->vq;
        pq.qp.Kst = ctx->vk;
        pq.qp.Vst = ctx->vv;
        pq.qp.kc = const_cast<void *>(a.kc);
        pq.qp.vc = const_cast<void *>(a.vc);
        pq.qp.head_stride = a.head_stride;
        pq.qp.v_tblk = a.v_tblk;
        pq.qp.kvw = !plain ? 0 : ctx->kv_format == FL_KV_F16 ? 1 : 2;
        if (fuse && L.qkv.rows % 64 == 0) {
            // the QKV post runs in the GEMM's last-arriving K split
            pq.post = 2;
            pq.counters = ctx->vcnt;
            rc = verify_gemm(ctx, L.qkv, M, ctx->vxq, ctx->vxs, ctx->vxsum, ks, &pq);
            if (rc) return rc;
        } else {
            rc = verify_gemm(ctx, L.qkv, M, ctx->vxq, ctx->vxs, ctx->vxsum, ks);
            if (rc) return rc;
            HIPCHK(ctx, launch_v_qkv_post(st, ctx->vpart, ks, M, L.qkv.rows, pq.qp));
        }
        if (probe) {
            if ((rc = probe_copy(ctx, PR_Q, ctx->vq, (size_t)M * qd * 4))) return rc;
            if ((rc = probe_kv(ctx, l, ctx->vpos, M, ctx->vk, ctx->vv))) return rc;
        }
        if (!plain)
            HIPCHK(ctx, launch_kv_write(ctx->kv_format, st, a, ctx->vk, ctx->vv, pos0, M, D,
                                        dev_pos ? ctx->vpos : nullptr));
        a.q = ctx->vq;
        a.posp = ctx->vpos;
        a.nsplit = ctx->nsplit;
        // M queries (M/2 pairs): chunks M (M/2) times the decode minimum, so
        // the launch keeps about the decode step's workgroup count (Llama-3-8B, 8 queries at
        // 4k on MI355X, unpaired: 33 vs 40 us per layer, one split per query 47 us;
        // paired: M/2 measured best against 1, 2, 6 and 8)
        // query pairs share each K/V block (fp16 / Q8, G <= 4, even M)
        static const bool no_pair = measure_env("FLARE_NO_QPAIR") != nullptr;  // measurement switch
        a.qpair = !no_pair && M % 2 == 0 && (G == 1 || G == 2 || G == 4) &&
                  (ctx->kv_format == FL_KV_F16 || ctx->kv_format == FL_KV_Q8);
        a.chmin = ctx->chmin * (a.qpair ? M / 2 : M);
        a.single = ctx->single;
        a.waves = ctx->attn_waves;
        a.part = ctx->d_part;
        a.counters = ctx->d_counters;
        size_t poff[PR_N];
        probe_layout(c, poff);
        a.out = probe ? (float *)(ctx->probe_dev + poff[PR_ATTN]) : nullptr;  // the f32 output, when probed
        a.oq = ctx->vaq;
        a.os = ctx->vas;
        a.osum = ctx->vasum;
        a.qstride = qd;
        a.ostride = qd;
        // fp16 caches, even M: the query pairs of a group share each staged
        // K/V block (k_attq), so the pass reads the cache once per group
        static const bool no_attq = measure_env("FLARE_NO_ATTQ") != nullptr;  // measurement switch
        static const int attq_chmin = measure_env("FLARE_ATTQ_CHMIN") ? std::max(32, atoi(measure_env("FLARE_ATTQ_CHMIN"))) : 64;
        // (prefill passes; the verify batches of up to 8 tokens keep k_attm's
        // query pairs, which measured faster at 8 tokens)
        static const bool attq_verify = measure_env("FLARE_ATTQ_VERIFY") != nullptr;  // measurement switch
        if (!no_attq && a.qpair && (M > kVerifyMaxTokens || attq_verify) && ctx->kv_format == FL_KV_F16 &&
            (D == 64 || D == 128)) {
            // splits: about one workgroup per CU over (kv heads x pair groups)
            static const int attq_ns = measure_env("FLARE_ATTQ_NSPLIT") ? atoi(measure_env("FLARE_ATTQ_NSPLIT")) : 0;
            const int per_wg = M / 2 <= 4 ? 4 : 8;  // pairs per workgroup (launch_attq)
            const int groups = (M / 2 + per_wg - 1) / per_wg;
            int ns = attq_ns > 0 ? attq_ns : ctx->ncu / (c.num_kv_heads * groups);
            a.nsplit = std::max(1, std::min(kAttmMaxSplit, ns));
            a.nq = M;
            a.chmin = attq_chmin;
            const hipError_t e = launch_attq(D, G, st, a);
            if (e == hipErrorNotSupported) return fail(ctx, FL_E_UNSUPPORTED, "attention shape");
            HIPCHK(ctx, e);
        } else {
            const hipError_t e = launch_attn(ctx->kv_format, D, G, st, a, M);
            if (e == hipErrorNotSupported) return fail(ctx, FL_E_UNSUPPORTED, "attention shape");
            HIPCHK(ctx, e);
        }
        if (probe) {
            if ((rc = probe_copy(ctx, PR_AQ, ctx->vaq, (size_t)M * qd))) return rc;
            if ((rc = probe_copy(ctx, PR_AS, ctx->vas, (size_t)M * (qd / 32) * 4))) return rc;
        }
        rc = verify_gemm(ctx, L.wo, M, ctx->vaq, ctx->vas, ctx->vasum, ks);
        if (rc) return rc;
        // FFN block (model.rs:2376-2543): wo residual + FFN norm in one kernel
        HIPCHK(ctx, launch_v_resnorm(pro, st, ctx->vpart, ks, M, H, xa, L.ffn_norm, eps, ctx->vxq, ctx->vxs,
                                     ctx->vxsum));
        if (probe) {
            if ((rc = probe_copy(ctx, PR_XMID, xa, (size_t)M * H * 4))) return rc;
            if ((rc = probe_copy(ctx, PR_FQ, ctx->vxq, (size_t)M * H))) return rc;
            if ((rc = probe_copy(ctx, PR_FS, ctx->vxs, (size_t)M * (H / 32) * 4))) return rc;
        }
        if (fuse && L.gu.rows == 2 * F && F % 32 == 0) {
            // SiLU(gate)*up + Q8_0 in the GEMM's last-arriving K split
            VgArgs pg{};
            pg.post = 1;
            pg.counters = ctx->vcnt;
            pg.hq = ctx->vhq;
            pg.hs = ctx->vhs;
            pg.hsum = ctx->vhsum;
            pg.F = F;
            rc = verify_gemm(ctx, L.gu, M, ctx->vxq, ctx->vxs, ctx->vxsum, ks, &pg);
        } else {
            rc = verify_gemm(ctx, L.gu, M, ctx->vxq, ctx->vxs, ctx->vxsum, ks);
            if (!rc) HIPCHK(ctx, launch_v_silu_quant(st, ctx->vpart, ks, M, F, ctx->vhq, ctx->vhs, ctx->vhsum));
        }
        if (rc) return rc;
        if (probe) {
            if ((rc = probe_copy(ctx, PR_HQ, ctx->vhq, (size_t)M * F))) return rc;
            if ((rc = probe_copy(ctx, PR_HS, ctx->vhs, (size_t)M * (F / 32) * 4))) return rc;
        }
        rc = verify_gemm(ctx, L.down, M, ctx->vhq, ctx->vhs, ctx->vhsum, ks_down);
        if (rc) return rc;
    }
    HIPCHK(ctx, launch_v_residual(st, ctx->vpart, ks_down, M, H, xa));
    if (ctx->probe_dev && ctx->probe_layer >= 0 && M <= kProbeTokens) {
        rc = probe_copy(ctx, PR_XFIN, xa, (size_t)M * H * 4);
        if (rc) return rc;
    }
    if (out_mode == VOUT_NONE) return 0;
    // output projection + fused argmax per token (forward_greedy, model.rs:1898-1932)
    const fl_weight &O = ctx->tied ? ctx->embed : ctx->output;
    const bool q8out = !ctx->tied && ((O.format == FL_Q8_0 && ctx->layer_fmt == FL_Q8_0) ||
                                      (O.format == FL_Q4K && ctx->layer_fmt == FL_Q4K));
    if (out_mode == VOUT_LAST_ARGMAX || out_mode == VOUT_LAST_LOGITS) {
        // the last token only (forward_prefill returns its logits, model.rs:2578-3040)
        const float *xt = xa + (size_t)(M - 1) * H;
        const int epi = out_mode == VOUT_LAST_LOGITS ? EPI_STORE : EPI_ARGMAX;
        if (O.format == FL_Q4K && !q8out) return fail(ctx, FL_E_UNSUPPORTED, "Q4_K output with Q8_0 layers");
        if (q8out)
            return launch_q8in(ctx, O, PRO_NORMQ1, epi, xt, ctx->out_norm, eps, nullptr, nullptr, nullptr, ctx->logits,
                               ctx->vslots + (M - 1));
        return launch_f32in(ctx, O, 1, epi, xt, ctx->out_norm, eps, ctx->logits, ctx->vslots + (M - 1));
    }
    if (!q8out && O.format != FL_F32) {
        if (O.format == FL_Q4K) return fail(ctx, FL_E_UNSUPPORTED, "Q4_K output with Q8_0 layers");
        // all M tokens in one MFMA launch (M <= 8 per launch)
        for (int t0 = 0; t0 < M; t0 += kMvoMaxTokens) {
            rc = launch_f32in(ctx, O, 1, EPI_ARGMAX, xa + (size_t)t0 * H, ctx->out_norm, eps, nullptr,
                              ctx->vslots + t0, std::min(kMvoMaxTokens, M - t0));
            if (rc) return rc;
        }
    } else {
        for (int t = 0; t < M; t++) {
            const float *xt = xa + (size_t)t * H;
            if (q8out)
                rc = launch_q8in(ctx, O, PRO_NORMQ1, EPI_ARGMAX, xt, ctx->out_norm, eps, nullptr, nullptr, nullptr,
                                 nullptr, ctx->vslots + t);
            else
                rc = launch_f32in(ctx, O, 1, EPI_ARGMAX, xt, ctx->out_norm, eps, nullptr, ctx->vslots + t);
            if (rc) return rc;
        }
    }
    return 0;
}

// Decode a packed argmax key (value bits << 32 | ~index) into (index, value).
static void unpack_key(unsigned long long k, int32_t *tok, float *val) {
    if (tok) *tok = (int32_t)(0xFFFFFFFFu - (uint32_t)(k & 0xFFFFFFFFull));
    if (val) {
        uint32_t u = (uint32_t)(k >> 32);
        u = (u & 0x80000000u) ? (u & 0x7FFFFFFFu) : ~u;
        std::memcpy(val, &u, 4);
    }
}

// Checks shared by fl_verify and fl_prefill for a pass of M tokens at pos0.
static int verify_check(fl_ctx *ctx, const uint32_t *tokens, int M, int pos0) {
    if (!ctx->have_weights) return fail(ctx, FL_E_STATE, "weights not uploaded");
    const fl_model_config &c = ctx->cfg;
    if (pos0 < 0 || pos0 + M > c.max_seq_len)
        return fail(ctx, FL_E_INVALID, "positions [%d, %d) outside the KV cache (max_seq_len %d)", pos0, pos0 + M,
                    c.max_seq_len);
    if (std::min(M, kPrefillTokens) * c.num_kv_heads > 1024)
        return fail(ctx, FL_E_INVALID, "too many kv heads for a verify batch");
    for (int i = 0; i < M; i++)
        if ((int)tokens[i] >= c.vocab_size) return fail(ctx, FL_E_INVALID, "token %u >= vocab", tokens[i]);
    return verify_alloc(ctx);
}

// One pass of M (<= kVerifyMaxTokens) tokens at pos0; the token ids are
// already in ctx->vtok.  `*pos_host` must stay valid until the stream
// reaches the pass (the position is copied to the device asynchronously).
static int run_verify_pass(fl_ctx *ctx, int M, const int *pos_host, int out_mode) {
    const fl_model_config &c = ctx->cfg;
    hipStream_t st = ctx->stream;
    const int G = c.num_heads / c.num_kv_heads;
    HIPCHK(ctx, hipMemcpyAsync(ctx->vpos, pos_host, 4, hipMemcpyHostToDevice, st));
    if (out_mode != VOUT_NONE) HIPCHK(ctx, hipMemsetAsync(ctx->vslots, 0, (size_t)M * 8, st));
    int rc = ensure_part(ctx, (size_t)M * c.num_kv_heads * part_splits(ctx) * G * (c.head_dim + 2));
    if (rc) return rc;
    // F32 / F16 / Q8 caches: one captured graph per (batch size, output
    // mode) (the positions are read from the device); KIVI plans its group
    // work from the host.  FLARE_NO_VERIFY_GRAPH (read per call): enqueue the
    // kernels directly
    const bool graph = use_graph() && ctx->verify_graph && getenv("FLARE_NO_VERIFY_GRAPH") == nullptr &&
                       ctx->probe_layer < 0;
    if (graph && ctx->kv_format != FL_KV_KIVI2) {
        const int key = M + 256 * out_mode;
        auto it = ctx->vgraphs.find(key);
        if (it == ctx->vgraphs.end()) {
            HIPCHK(ctx, hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
            rc = enqueue_verify(ctx, M, *pos_host, true, out_mode);
            hipGraph_t g = nullptr;
            const hipError_t e = hipStreamEndCapture(st, &g);
            if (rc) {
                if (g) (void)hipGraphDestroy(g);
                return rc;
            }
            if (e != hipSuccess) return fail(ctx, FL_E_HIP, "verify graph capture failed: %s", hipGetErrorString(e));
            hipGraphExec_t ge = nullptr;
            const hipError_t ei = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
            (void)hipGraphDestroy(g);
            if (ei != hipSuccess) return fail(ctx, FL_E_HIP, "verify graph instantiate: %s", hipGetErrorString(ei));
            it = ctx->vgraphs.emplace(key, ge).first;
        }
        HIPCHK(ctx, hipGraphLaunch(it->second, st));
        return 0;
    }
    return enqueue_verify(ctx, M, *pos_host, false, out_mode);
}

int fl_verify(fl_ctx *ctx, const uint32_t *tokens, int n_tokens, int pos0, int32_t *out_tokens, float *out_vals) {
    if (!ctx || !tokens || !out_tokens) return fail(ctx, FL_E_INVALID, "null argument");
    const int M = n_tokens;
    if (M < 1 || M > kVerifyMaxTokens) return fail(ctx, FL_E_INVALID, "verify batch of %d tokens (1..%d)", M, kVerifyMaxTokens);
    int rc = verify_check(ctx, tokens, M, pos0);
    if (rc) return rc;
    if (ctx->exact) {
        // reference-order mode: the reference's own sequential verification
        // (one forward_greedy per draft, generate.rs:244-312)
        for (int t = 0; t < M; t++) {
            rc = decode_step(ctx, tokens[t], nullptr, pos0 + t, nullptr, &out_tokens[t], out_vals ? &out_vals[t] : nullptr);
            if (rc) return rc;
        }
        return 0;
    }
    hipStream_t st = ctx->stream;
    std::vector<int> tk(tokens, tokens + M);
    HIPCHK(ctx, hipMemcpyAsync(ctx->vtok, tk.data(), (size_t)M * 4, hipMemcpyHostToDevice, st));
    rc = run_verify_pass(ctx, M, &pos0, VOUT_ALL);
    if (rc) return rc;
    std::vector<unsigned long long> keys(M);
    HIPCHK(ctx, hipMemcpyAsync(keys.data(), ctx->vslots, (size_t)M * 8, hipMemcpyDeviceToHost, st));
    if (ctx->probe_layer >= 0 && ctx->probe_host)
        HIPCHK(ctx, hipMemcpyAsync(ctx->probe_host, ctx->probe_dev, ctx->probe_bytes, hipMemcpyDeviceToHost, st));
    HIPCHK(ctx, hipStreamSynchronize(st));
    for (int t = 0; t < M; t++) unpack_key(keys[t], &out_tokens[t], out_vals ? &out_vals[t] : nullptr);
    return 0;
}

int fl_prefill(fl_ctx *ctx, const uint32_t *tokens, int n_tokens, int pos0, float *out_logits, int32_t *out_token,
               float *out_val) {
    if (!ctx || !tokens) return fail(ctx, FL_E_INVALID, "null argument");
    if (n_tokens < 1) return fail(ctx, FL_E_INVALID, "prefill of %d tokens", n_tokens);
    int rc = verify_check(ctx, tokens, n_tokens, pos0);
    if (rc) return rc;
    if (ctx->exact) {
        // reference-order mode: the prompt as sequential decode steps, which
        // forward_prefill equals (test_batched_prefill_matches_sequential,
        // flare-core/src/generate.rs:657)
        for (int i = 0; i + 1 < n_tokens; i++) {
            rc = decode_step(ctx, tokens[i], nullptr, pos0 + i, nullptr, nullptr, nullptr);
            if (rc) return rc;
        }
        return decode_step(ctx, tokens[n_tokens - 1], nullptr, pos0 + n_tokens - 1, out_logits, out_token, out_val);
    }
    hipStream_t st = ctx->stream;
    // FLARE_PREFILL_TOKENS: pass size (measurement switch; 1..64)
    static const int C = measure_env("FLARE_PREFILL_TOKENS")
                             ? std::max(1, std::min(kPrefillTokens, atoi(measure_env("FLARE_PREFILL_TOKENS"))))
                             : kPrefillTokens;
    const int nchunks = (n_tokens + C - 1) / C;
    // host copies stay alive until the final synchronisation
    std::vector<int> tk(tokens, tokens + n_tokens), pos(nchunks);
    for (int k = 0; k < nchunks; k++) {
        const int t0 = k * C, M = std::min(C, n_tokens - t0);
        pos[k] = pos0 + t0;
        HIPCHK(ctx, hipMemcpyAsync(ctx->vtok, tk.data() + t0, (size_t)M * 4, hipMemcpyHostToDevice, st));
        const int mode = k + 1 < nchunks ? VOUT_NONE : out_logits ? VOUT_LAST_LOGITS : VOUT_LAST_ARGMAX;
        rc = run_verify_pass(ctx, M, &pos[k], mode);
        if (rc) return rc;
    }
    const int Mlast = n_tokens - (nchunks - 1) * C;
    unsigned long long key = 0;
    HIPCHK(ctx, hipMemcpyAsync(&key, ctx->vslots + (Mlast - 1), 8, hipMemcpyDeviceToHost, st));
    if (out_logits)
        HIPCHK(ctx, hipMemcpyAsync(out_logits, ctx->logits, (size_t)ctx->cfg.vocab_size * 4, hipMemcpyDeviceToHost, st));
    HIPCHK(ctx, hipStreamSynchronize(st));
    if (out_logits) {
        int bi = 0;
        float bv = -INFINITY;
        for (int i = 0; i < ctx->cfg.vocab_size; i++)
            if (out_logits[i] > bv) { bv = out_logits[i]; bi = i; }
        if (out_token) *out_token = bi;
        if (out_val) *out_val = bv;
    } else {
        unpack_key(key, out_token, out_val);
    }
    return 0;
}

// ---- device sampling ----------------------------------------------------------

static int sample_alloc(fl_ctx *ctx, int n, int n_prev) {
    if (n > ctx->sample_cap) {
        void **bufs[] = {(void **)&ctx->sp, (void **)&ctx->scounts, (void **)&ctx->svals, (void **)&ctx->ssvals,
                         (void **)&ctx->skeys, (void **)&ctx->sskeys, &ctx->ssort};
        for (void **b : bufs) {
            if (*b) (void)hipFree(*b);
            *b = nullptr;
        }
        ctx->sample_cap = 0;
        ALLOC(ctx, ctx->sp, (size_t)n * 4);
        ALLOC(ctx, ctx->scounts, (size_t)n * 4);
        ALLOC(ctx, ctx->svals, (size_t)n * 4);
        ALLOC(ctx, ctx->ssvals, (size_t)n * 4);
        ALLOC(ctx, ctx->skeys, (size_t)n * 4);
        ALLOC(ctx, ctx->sskeys, (size_t)n * 4);
        ctx->ssort_bytes = std::max<size_t>(fl::sample_sort_bytes(n), 256);
        ALLOC(ctx, ctx->ssort, ctx->ssort_bytes);
        HIPCHK(ctx, hipMemset(ctx->scounts, 0, (size_t)n * 4));  // the sampler leaves them at zero
        ctx->sample_cap = n;
    }
    if (!ctx->sstate) ALLOC(ctx, ctx->sstate, 16);
    if (n_prev > ctx->sample_prev_cap) {
        if (ctx->sprev) (void)hipFree(ctx->sprev);
        ctx->sprev = nullptr;
        ctx->sample_prev_cap = 0;
        const int cap = std::max(n_prev, 1024);
        ALLOC(ctx, ctx->sprev, (size_t)cap * 4);
        ctx->sample_prev_cap = cap;
    }
    return 0;
}

// Enqueue the sampler over `logits` (device) and read the token back.
static int sample_logits(fl_ctx *ctx, const float *logits, int n, const fl_sampling_params *sp,
                         const uint32_t *prev, int n_prev, float u, int32_t *out) {
    if (!sp || !out || (n_prev > 0 && !prev)) return fail(ctx, FL_E_INVALID, "null argument");
    if (n < 1 || n_prev < 0) return fail(ctx, FL_E_INVALID, "sampling %d logits with %d previous tokens", n, n_prev);
    int rc = sample_alloc(ctx, n, n_prev);
    if (rc) return rc;
    fl::SampleArgs a{};
    a.logits = logits;
    a.n = n;
    a.p = ctx->sp;
    a.counts = ctx->scounts;
    a.prev = ctx->sprev;
    a.n_prev = n_prev;
    a.penalty = sp->repeat_penalty;
    a.temperature = sp->temperature;
    a.top_p = sp->top_p;
    a.min_p = sp->min_p;
    // the priority of Generator::step (generate.rs:220-230)
    if (sp->temperature == 0.0f) {
        a.mode = fl::SM_GREEDY;
        a.K = 1;
    } else if (sp->top_p < 1.0f) {
        a.mode = fl::SM_TOP_P;
        a.K = std::min(512, n);
    } else if (sp->min_p > 0.0f) {
        a.mode = fl::SM_MIN_P;
        a.K = n;
    } else if (sp->top_k > 0) {
        a.mode = fl::SM_TOP_K;
        a.K = std::max(1, std::min(sp->top_k, n));
    } else {
        a.mode = fl::SM_TOP_P;  // sample_top_p(logits, 1.0, rng_val)
        a.top_p = 1.0f;
        a.K = std::min(512, n);
    }
    a.u = u;
    a.exact = ctx->exact ? 1 : 0;
    a.keys = ctx->skeys;
    a.vals = ctx->svals;
    a.skeys = ctx->sskeys;
    a.svals = ctx->ssvals;
    a.state = ctx->sstate;
    // host copy alive until the synchronisation below
    std::vector<int> pv(prev, prev + n_prev);
    if (n_prev > 0) HIPCHK(ctx, hipMemcpyAsync(ctx->sprev, pv.data(), (size_t)n_prev * 4, hipMemcpyHostToDevice, ctx->stream));
    HIPCHK(ctx, fl::launch_sample(ctx->stream, a, ctx->ssort, ctx->ssort_bytes));
    int st[4] = {0, 0, 0, 0};
    HIPCHK(ctx, hipMemcpyAsync(st, ctx->sstate, 16, hipMemcpyDeviceToHost, ctx->stream));
    HIPCHK(ctx, hipStreamSynchronize(ctx->stream));
    *out = st[0];
    return 0;
}

int fl_op_sample(fl_ctx *ctx, const float *logits, int n, const fl_sampling_params *params, const uint32_t *prev_tokens,
                 int n_prev, float rng_val, int32_t *out_token) {
    if (!ctx || !logits) return fail(ctx, FL_E_INVALID, "null argument");
    return sample_logits(ctx, logits, n, params, prev_tokens, n_prev, rng_val, out_token);
}

int fl_decode_step_sample(fl_ctx *ctx, uint32_t token, int pos, const fl_sampling_params *params,
                          const uint32_t *prev_tokens, int n_prev, float rng_val, int32_t *out_token) {
    if (!ctx) return fail(nullptr, FL_E_INVALID, "null ctx");
    if (!ctx->have_weights) return fail(ctx, FL_E_STATE, "weights not uploaded");
    const fl_model_config &c = ctx->cfg;
    if (pos < 0 || pos >= c.max_seq_len)
        return fail(ctx, FL_E_INVALID, "pos %d outside the KV cache (max_seq_len %d)", pos, c.max_seq_len);
    if ((int)token >= c.vocab_size) return fail(ctx, FL_E_INVALID, "token %u >= vocab", token);
    const int tok = (int)token;
    DevState hs{};
    hs.step = pos;
    hs.pos = pos;
    hs.n_prompt = pos + 1;
    HIPCHK(ctx, hipMemcpyAsync(ctx->tokens + pos, &tok, 4, hipMemcpyHostToDevice, ctx->stream));
    HIPCHK(ctx, hipMemcpyAsync(ctx->st, &hs, sizeof hs, hipMemcpyHostToDevice, ctx->stream));
    int rc = enqueue_step(ctx, true);
    if (rc) return rc;
    return sample_logits(ctx, ctx->logits, c.vocab_size, params, prev_tokens, n_prev, rng_val, out_token);
}

// Launch `iters` copies of one layer kernel on the context stream, cycling
// through the layers.
int fl_bench_layer_kernel(fl_ctx *ctx, int which, int first_layer, int iters, double *bytes_per_launch) {
    if (!ctx || !ctx->have_weights) return fail(ctx, FL_E_STATE, "no model");
    const fl_model_config &c = ctx->cfg;
    const int norm_pro = ctx->layer_fmt == FL_Q8_0 ? PRO_NORMQ0 : PRO_NORMQ1;
    const fl_weight *w = nullptr;
    for (int i = 0; i < iters; i++) {
        // cycle through the layers so repeated launches stream distinct
        // weights from HBM instead of re-reading a cache-resident matrix
        const int li = (first_layer + i) % c.num_layers;
        Layer &L = ctx->layers[li];
        int rc = 0;
        switch (which) {
        case 0: {
            // writes q to the bench buffer and K/V into the cache slot of the
            // current position (the next decode step rewrites that slot)
            w = &L.qkv;
            const QkvEpi qe = layer_qkv_epi(ctx, li);
            rc = launch_q8in(ctx, L.qkv, norm_pro, EPI_QKV, ctx->x, L.attn_norm, c.rms_norm_eps, nullptr, nullptr,
                             nullptr, ctx->bench_out, nullptr, &qe);
            break;
        }
        case 1: w = &L.wo; rc = launch_q8in(ctx, L.wo, PRO_LOADQ, EPI_STORE, nullptr, nullptr, 0.f, ctx->aq, ctx->as, ctx->asum, ctx->bench_out, nullptr); break;
        case 2: w = &L.gu; rc = launch_gateup(ctx, L.gu, norm_pro, ctx->x, L.ffn_norm, c.rms_norm_eps, nullptr, nullptr, nullptr, ctx->hq, ctx->hs, ctx->hsum, nullptr); break;
        case 3: w = &L.down; rc = launch_q8in(ctx, L.down, PRO_LOADQ, EPI_STORE, nullptr, nullptr, 0.f, ctx->hq, ctx->hs, ctx->hsum, ctx->bench_out, nullptr); break;
        case 4: {
            const fl_weight &O = ctx->tied ? ctx->embed : ctx->output;
            w = &O;
            const bool q8out = !ctx->tied && (O.format == FL_Q8_0 || O.format == FL_Q4K);
            if (q8out) rc = launch_q8in(ctx, O, PRO_NORMQ1, EPI_ARGMAX, ctx->x, ctx->out_norm, c.rms_norm_eps, nullptr, nullptr, nullptr, nullptr, ctx->d_slot);
            else rc = launch_f32in(ctx, O, 1, EPI_ARGMAX, ctx->x, ctx->out_norm, c.rms_norm_eps, nullptr, ctx->d_slot);
            break;
        }
        case 5: {  // attention of layer li at the current position
            AttnArgs a = layer_attn_args(ctx, li);
            a.trace = ctx->bench_trace;
            rc = launch_attention(ctx, ctx->kv_format, c.head_dim, c.num_heads / c.num_kv_heads, a);
            break;
        }
        case 6: case 7: case 8: case 9: {  // verify GEMMs (8 tokens): qkv, wo, gate/up, down
            rc = verify_alloc(ctx);
            if (rc) return rc;
            const fl_weight *vw[4] = {&L.qkv, &L.wo, &L.gu, &L.down};
            w = vw[which - 6];
            int ks;
            rc = verify_gemm(ctx, *w, 8, ctx->vxq, ctx->vxs, ctx->vxsum, ks);
            break;
        }
        default: return fail(ctx, FL_E_INVALID, "which=%d", which);
        }
        if (rc) return rc;
    }
    if (which <= 4 && measure_env("FLARE_MV_TRACE_PRINT")) {
        // workgroup 0 phases, then the spread of workgroup start / end times
        std::vector<long long> tr(64 + 3072, 0);
        HIPCHK(ctx, hipStreamSynchronize(ctx->stream));
        HIPCHK(ctx, hipMemcpy(tr.data(), ctx->bench_trace, tr.size() * 8, hipMemcpyDeviceToHost));
        fprintf(stderr, "mv trace which=%d (10ns ticks from wg0 start):", which);
        for (int i = 1; i < 11; i++) fprintf(stderr, " %lld", tr[i] ? tr[i] - tr[0] : -1);
        long long s0 = 0, s1 = 0, e0 = 0, e1 = 0;
        int n = 0;
        for (int b = 0; b < 1024; b++) {
            const long long st = tr[64 + 2 * b], en = tr[65 + 2 * b];
            if (!st || !en || en < st) continue;
            if (!n || st < s0) s0 = st;
            if (!n || st > s1) s1 = st;
            if (!n || en < e0) e0 = en;
            if (!n || en > e1) e1 = en;
            n++;
        }
        if (n) fprintf(stderr, " | %d wgs: starts %lld..%lld ends %lld..%lld", n, s0 - tr[0], s1 - tr[0], e0 - tr[0], e1 - tr[0]);
        fprintf(stderr, "\n");
        if (const char *dump = measure_env("FLARE_MV_TRACE_DUMP")) {
            // raw per-workgroup (start, end) ticks, one line per launch
            if (FILE *f = fopen(dump, "a")) {
                fprintf(f, "%d", which);
                for (int b = 0; b < 1024; b++) fprintf(f, " %lld %lld %lld", tr[64 + 2 * b] ? tr[64 + 2 * b] - tr[0] : -1,
                                                        tr[65 + 2 * b] ? tr[65 + 2 * b] - tr[0] : -1, tr[64 + 2048 + b]);
                fprintf(f, "\n");
                fclose(f);
            }
        }
        HIPCHK(ctx, hipMemset(ctx->bench_trace, 0, tr.size() * 8));
    }
    if (which == 5 && measure_env("FLARE_ATTN_TRACE_PRINT")) {
        long long tr[24] = {0};
        HIPCHK(ctx, hipStreamSynchronize(ctx->stream));
        HIPCHK(ctx, hipMemcpy(tr, ctx->bench_trace, sizeof tr, hipMemcpyDeviceToHost));
        fprintf(stderr, "attn trace (10ns ticks from start):");
        for (int i = 1; i < 10; i++) fprintf(stderr, " %lld", tr[i] - tr[0]);
        fprintf(stderr, "\n");
    }
    if (bytes_per_launch && which == 5) {
        DevState st{};
        HIPCHK(ctx, hipMemcpy(&st, ctx->st, sizeof st, hipMemcpyDeviceToHost));
        *bytes_per_launch = attn_bytes(ctx, st.pos + 1);
    } else if (bytes_per_launch && w) {
        *bytes_per_launch = (double)w->gguf_bytes;
    }
    return 0;
}

const char *fl_bench_kernel_name(fl_ctx *ctx, int which) {
    if (!ctx || !ctx->have_weights) return "";
    switch (which) {
    case 0: return "k_mvs";
    case 1: return "k_mvs";
    case 2: return "k_mvs_gu";
    case 3: return "k_mvs";
    case 4: return "k_mvs";
    case 5: return ctx->kv_format == FL_KV_F32 ? "k_attn" : "k_attm";
    case 6: case 7: case 8: case 9: return ctx->layer_fmt == FL_Q4K ? "k_vgemm_q4k" : "k_vgemm_q8_0";
    }
    return "";
}

}  // extern "C"
