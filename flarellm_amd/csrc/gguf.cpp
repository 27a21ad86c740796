// GGUF v2/v3 reader (flare-loader/src/gguf.rs) feeding the device upload.
//
// The file is memory-mapped read-only; tensor bytes are handed to
// fl_upload_weights straight from the mapping (RawWeight::data without a
// copy: pages stream in from the file as the upload reads them).  Header
// parsing follows GgufFile::parse_header (gguf.rs:131-204): magic, version 2..3,
// the reference's sanity limits, metadata values (read_metadata_value,
// gguf.rs:917-963), tensor infos and tensor data at the next 32-byte boundary.
// Model configuration follows GgufFile::to_model_config (gguf.rs:241-346) and
// raw weights GgufFile::read_raw_weight (gguf.rs:616-653).
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cctype>
#include <climits>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <map>
#include <new>
#include <string>
#include <vector>

#include "../../include/flare_hip.h"
#include "host_api.h"

namespace {

constexpr uint32_t kMagic = 0x46554747u;  // "GGUF"
constexpr uint64_t kMaxTensors = 1000000, kMaxMetadata = 100000, kMaxString = 1 << 20;
constexpr uint64_t kAlign = 32;

// GGUF metadata value types (gguf.rs:917-963)
enum { V_U8 = 0, V_I8, V_U16, V_I16, V_U32, V_I32, V_F32, V_BOOL, V_STR, V_ARR, V_U64, V_I64, V_F64 };

struct Value {
    int type = -1;
    uint64_t u = 0;   // unsigned integers and bool
    int64_t i = 0;    // signed integers
    double f = 0.0;   // floats
    std::string s;
    std::vector<Value> arr;
};

// ggml type ids (QuantFormat::from_gguf_type, quantize.rs:32-60) -> (block elements, block bytes)
bool ggml_block(uint32_t t, uint64_t *elems, uint64_t *bytes) {
    struct B { uint32_t t; uint64_t e, b; };
    static const B tab[] = {
        {0, 1, 4},      {1, 1, 2},       {32, 1, 2},  // F32, F16, BF16 (flarellm's id)
        {2, 32, 18},    {3, 32, 20},     {6, 32, 22}, {7, 32, 24}, {8, 32, 34}, {9, 32, 36},  // Q4_0..Q8_1
        {10, 256, 84},  {11, 256, 110},  {12, 256, 144}, {13, 256, 176}, {14, 256, 210},     // Q2_K..Q6_K
    };
    for (const B &x : tab)
        if (x.t == t) {
            *elems = x.e;
            *bytes = x.b;
            return true;
        }
    return false;
}

struct Reader {
    const uint8_t *p;
    uint64_t n, off = 0;
    bool ok = true;
    bool need(uint64_t k) {
        if (!ok || off + k > n) ok = false;
        return ok;
    }
    template <class T> T get() {
        T v{};
        if (need(sizeof(T))) {
            std::memcpy(&v, p + off, sizeof(T));
            off += sizeof(T);
        }
        return v;
    }
    bool str(std::string &out, std::string &err) {
        const uint64_t len = get<uint64_t>();
        if (!ok) return false;
        if (len > kMaxString) {
            err = "string length " + std::to_string(len) + " exceeds maximum " + std::to_string(kMaxString);
            ok = false;
            return false;
        }
        if (!need(len)) return false;
        out.assign((const char *)p + off, (size_t)len);
        off += len;
        return true;
    }
};

bool read_typed(Reader &r, uint32_t type, Value &v, std::string &err, bool allow_array) {
    v.type = (int)type;
    switch (type) {
    case V_U8: v.u = r.get<uint8_t>(); break;
    case V_I8: v.i = r.get<int8_t>(); break;
    case V_U16: v.u = r.get<uint16_t>(); break;
    case V_I16: v.i = r.get<int16_t>(); break;
    case V_U32: v.u = r.get<uint32_t>(); break;
    case V_I32: v.i = r.get<int32_t>(); break;
    case V_F32: v.f = r.get<float>(); break;
    case V_BOOL: v.u = r.get<uint8_t>() != 0; break;
    case V_STR: r.str(v.s, err); break;
    case V_U64: v.u = r.get<uint64_t>(); break;
    case V_I64: v.i = r.get<int64_t>(); break;
    case V_F64: v.f = r.get<double>(); break;
    case V_ARR: {
        if (!allow_array) {
            err = "invalid metadata value type: 9";
            return false;
        }
        const uint32_t et = r.get<uint32_t>();
        const uint64_t count = r.get<uint64_t>();
        if (!r.ok) break;
        if (count > r.n) {  // every element takes at least one byte
            r.ok = false;
            break;
        }
        v.arr.resize((size_t)count);
        for (uint64_t k = 0; k < count && r.ok; k++)
            if (!read_typed(r, et, v.arr[k], err, false)) return false;
        break;
    }
    default:
        err = "invalid metadata value type: " + std::to_string(type);
        return false;
    }
    if (!r.ok && err.empty()) err = "I/O error: unexpected end of file";
    return r.ok;
}

}  // namespace

struct TensorInfo {
    std::string name;
    std::vector<uint64_t> dims;
    uint32_t type = 0;
    uint64_t offset = 0;
};

struct fl_gguf {
    // the mapping (or an owned copy for fl_gguf_open_memory)
    void *map = nullptr;
    size_t map_len = 0;
    std::vector<uint8_t> owned;
    const uint8_t *data = nullptr;
    uint64_t len = 0;
    uint32_t version = 0;
    std::map<std::string, Value> meta;
    std::vector<TensorInfo> tensors;
    uint64_t data_offset = 0;

    ~fl_gguf() {
        if (map) munmap(map, map_len);
    }
    const TensorInfo *find(const char *name) const {
        for (const TensorInfo &t : tensors)
            if (t.name == name) return &t;
        return nullptr;
    }
};

namespace {

int gg_fail(int code, const std::string &msg) { return fl_host_fail(nullptr, code, msg.c_str()); }

// GgufFile::parse_header (gguf.rs:131-204)
int parse(fl_gguf *g) {
    Reader r{g->data, g->len};
    std::string err;
    const uint32_t magic = r.get<uint32_t>();
    if (!r.ok) return gg_fail(FL_E_INVALID, "I/O error: unexpected end of file");
    if (magic != kMagic) {
        char b[96];
        std::snprintf(b, sizeof b, "invalid GGUF magic number: expected 0x%08X, got 0x%08X", kMagic, magic);
        return gg_fail(FL_E_INVALID, b);
    }
    g->version = r.get<uint32_t>();
    if (r.ok && (g->version < 2 || g->version > 3))
        return gg_fail(FL_E_INVALID, "unsupported GGUF version: " + std::to_string(g->version));
    const uint64_t ntensors = r.get<uint64_t>(), nmeta = r.get<uint64_t>();
    if (!r.ok) return gg_fail(FL_E_INVALID, "I/O error: unexpected end of file");
    if (ntensors > kMaxTensors)
        return gg_fail(FL_E_INVALID, "invalid GGUF format: tensor count " + std::to_string(ntensors) +
                                         " exceeds maximum " + std::to_string(kMaxTensors));
    if (nmeta > kMaxMetadata)
        return gg_fail(FL_E_INVALID, "invalid GGUF format: metadata count " + std::to_string(nmeta) +
                                         " exceeds maximum " + std::to_string(kMaxMetadata));
    for (uint64_t k = 0; k < nmeta; k++) {
        std::string key;
        if (!r.str(key, err)) return gg_fail(FL_E_INVALID, err.empty() ? "I/O error: unexpected end of file" : err);
        const uint32_t type = r.get<uint32_t>();
        Value v;
        if (!r.ok || !read_typed(r, type, v, err, true))
            return gg_fail(FL_E_INVALID, err.empty() ? "I/O error: unexpected end of file" : err);
        g->meta[key] = std::move(v);  // a repeated key keeps the last value (HashMap::insert)
    }
    g->tensors.resize((size_t)ntensors);
    for (uint64_t k = 0; k < ntensors; k++) {
        TensorInfo &t = g->tensors[(size_t)k];
        if (!r.str(t.name, err)) return gg_fail(FL_E_INVALID, err.empty() ? "I/O error: unexpected end of file" : err);
        const uint32_t nd = r.get<uint32_t>();
        if (!r.ok || nd > 8) return gg_fail(FL_E_INVALID, "invalid GGUF format: tensor dimensions");
        t.dims.resize(nd);
        for (uint32_t d = 0; d < nd; d++) t.dims[d] = r.get<uint64_t>();
        t.type = r.get<uint32_t>();
        t.offset = r.get<uint64_t>();
        if (!r.ok) return gg_fail(FL_E_INVALID, "I/O error: unexpected end of file");
    }
    g->data_offset = (r.off + kAlign - 1) / kAlign * kAlign;
    return 0;
}

const Value *meta(const fl_gguf *g, const std::string &key) {
    auto it = g->meta.find(key);
    return it == g->meta.end() ? nullptr : &it->second;
}

// meta_usize (gguf.rs:218-237): u32, i32, u64, i64, u16, u8
bool meta_usize(const fl_gguf *g, const std::string &key, uint64_t *out) {
    const Value *v = meta(g, key);
    if (!v) return false;
    switch (v->type) {
    case V_U32: case V_U64: case V_U16: case V_U8: *out = v->u; return true;
    case V_I32: case V_I64: *out = (uint64_t)v->i; return true;
    default: return false;
    }
}

// meta_f32 (gguf.rs:240-251): f32 or f64
bool meta_f32(const fl_gguf *g, const std::string &key, float *out) {
    const Value *v = meta(g, key);
    if (!v || (v->type != V_F32 && v->type != V_F64)) return false;
    *out = (float)v->f;
    return true;
}

// Element count (numel().max(1)); 0 when the product of the dimensions does
// not fit in 63 bits (a crafted header), which every caller rejects.
uint64_t numel(const TensorInfo &t) {
    uint64_t n = 1;
    for (uint64_t d : t.dims) {
        if (d != 0 && n > (UINT64_C(1) << 63) / d) return 0;
        n *= d;
    }
    return n ? n : 1;
}

int tensor_bytes(const TensorInfo &t, uint64_t *bytes) {
    uint64_t e, b;
    if (!ggml_block(t.type, &e, &b)) return FL_E_UNSUPPORTED;
    const uint64_t n = numel(t);
    if (n == 0) return FL_E_INVALID;
    const uint64_t blocks = n / e + (n % e != 0);
    if (blocks > UINT64_MAX / b) return FL_E_INVALID;
    *bytes = blocks * b;  // bytes_for_elements (quantize.rs:139-147)
    return 0;
}

int tensor_span(const fl_gguf *g, const TensorInfo &t, const uint8_t **p, uint64_t *bytes) {
    int rc = tensor_bytes(t, bytes);
    if (rc == FL_E_UNSUPPORTED) return gg_fail(rc, "unsupported quantization format of tensor " + t.name);
    if (rc) return gg_fail(rc, "tensor " + t.name + " has dimensions whose product overflows");
    // offset checked before the addition, so a huge offset cannot wrap
    if (g->data_offset > g->len || t.offset > g->len - g->data_offset)
        return gg_fail(FL_E_INVALID, "tensor " + t.name + " starts past the end of the file");
    const uint64_t start = g->data_offset + t.offset;
    if (*bytes > g->len - start)
        return gg_fail(FL_E_INVALID, "tensor " + t.name + " extends past the end of the file");
    *p = g->data + start;
    return 0;
}

}  // namespace

extern "C" {

int fl_gguf_open(const char *path, fl_gguf **out) {
    if (!path || !out) return gg_fail(FL_E_INVALID, "null argument");
    *out = nullptr;
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return gg_fail(FL_E_INVALID, std::string("I/O error: cannot open ") + path);
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size <= 0) {
        close(fd);
        return gg_fail(FL_E_INVALID, std::string("I/O error: cannot stat ") + path);
    }
    void *m = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (m == MAP_FAILED) return gg_fail(FL_E_INVALID, std::string("I/O error: cannot map ") + path);
    fl_gguf *g = new (std::nothrow) fl_gguf();
    if (!g) {
        munmap(m, (size_t)st.st_size);
        return gg_fail(FL_E_OOM, "out of host memory");
    }
    g->map = m;
    g->map_len = (size_t)st.st_size;
    g->data = (const uint8_t *)m;
    g->len = (uint64_t)st.st_size;
    const int rc = parse(g);
    if (rc) {
        delete g;
        return rc;
    }
    *out = g;
    return 0;
}

int fl_gguf_open_memory(const void *data, size_t len, fl_gguf **out) {
    if ((!data && len) || !out) return gg_fail(FL_E_INVALID, "null argument");
    *out = nullptr;
    fl_gguf *g = new (std::nothrow) fl_gguf();
    if (!g) return gg_fail(FL_E_OOM, "out of host memory");
    g->owned.assign((const uint8_t *)data, (const uint8_t *)data + len);
    g->data = g->owned.data();
    g->len = len;
    const int rc = parse(g);
    if (rc) {
        delete g;
        return rc;
    }
    *out = g;
    return 0;
}

void fl_gguf_close(fl_gguf *g) { delete g; }

int fl_gguf_version(const fl_gguf *g) { return g ? (int)g->version : -1; }
uint64_t fl_gguf_data_offset(const fl_gguf *g) { return g ? g->data_offset : 0; }
int fl_gguf_tensor_count(const fl_gguf *g) { return g ? (int)g->tensors.size() : -1; }

int fl_gguf_find_tensor(const fl_gguf *g, const char *name) {
    if (!g || !name) return -1;
    for (size_t i = 0; i < g->tensors.size(); i++)
        if (g->tensors[i].name == name) return (int)i;
    return -1;
}

int fl_gguf_tensor_info(const fl_gguf *g, int index, const char **name, int *n_dims, uint64_t *dims,
                        uint32_t *ggml_type, uint64_t *offset, uint64_t *nbytes) {
    if (!g || index < 0 || index >= (int)g->tensors.size()) return gg_fail(FL_E_INVALID, "tensor index");
    const TensorInfo &t = g->tensors[(size_t)index];
    if (name) *name = t.name.c_str();
    if (n_dims) *n_dims = (int)t.dims.size();
    if (dims)
        for (size_t d = 0; d < t.dims.size() && d < 8; d++) dims[d] = t.dims[d];
    if (ggml_type) *ggml_type = t.type;
    if (offset) *offset = t.offset;
    if (nbytes) {
        uint64_t b = 0;
        *nbytes = tensor_bytes(t, &b) ? 0 : b;
    }
    return 0;
}

int fl_gguf_meta_u64(const fl_gguf *g, const char *key, uint64_t *out) {
    if (!g || !key || !out) return gg_fail(FL_E_INVALID, "null argument");
    return meta_usize(g, key, out) ? 0 : gg_fail(FL_E_INVALID, std::string("missing metadata key: ") + key);
}

int fl_gguf_meta_f32(const fl_gguf *g, const char *key, float *out) {
    if (!g || !key || !out) return gg_fail(FL_E_INVALID, "null argument");
    return meta_f32(g, key, out) ? 0 : gg_fail(FL_E_INVALID, std::string("missing metadata key: ") + key);
}

const char *fl_gguf_meta_str(const fl_gguf *g, const char *key) {
    if (!g || !key) return nullptr;
    const Value *v = meta(g, key);
    return v && v->type == V_STR ? v->s.c_str() : nullptr;
}

int fl_gguf_model_config(const fl_gguf *g, fl_model_config *cfg, int *arch) {
    // GgufFile::to_model_config (gguf.rs:241-346)
    if (!g || !cfg) return gg_fail(FL_E_INVALID, "null argument");
    const char *a = fl_gguf_meta_str(g, "general.architecture");
    if (!a) return gg_fail(FL_E_INVALID, "missing metadata key: general.architecture");
    std::string prefix(a);
    for (char &ch : prefix) ch = (char)std::tolower((unsigned char)ch);
    static const char *const archs[] = {"llama", "qwen2", "mistral", "phi3", "gemma2"};
    int id = -1;
    for (int k = 0; k < 5; k++)
        if (prefix == archs[k]) id = k;
    if (id < 0) return gg_fail(FL_E_UNSUPPORTED, "unsupported architecture: " + prefix);
    uint64_t vocab = 0;
    const TensorInfo *emb = g->find("token_embd.weight");
    if (!emb) emb = g->find("model.embed_tokens.weight");
    if (emb && emb->dims.size() == 2) vocab = emb->dims[1];
    else if (!meta_usize(g, prefix + ".vocab_size", &vocab)) vocab = 32000;
    uint64_t hidden, layers, heads, kv, inter, ctxlen;
    if (!meta_usize(g, prefix + ".embedding_length", &hidden))
        return gg_fail(FL_E_INVALID, "missing metadata key: " + prefix + ".embedding_length");
    if (!meta_usize(g, prefix + ".block_count", &layers))
        return gg_fail(FL_E_INVALID, "missing metadata key: " + prefix + ".block_count");
    if (!meta_usize(g, prefix + ".attention.head_count", &heads))
        return gg_fail(FL_E_INVALID, "missing metadata key: " + prefix + ".attention.head_count");
    if (heads == 0) return gg_fail(FL_E_INVALID, "attention.head_count is 0");
    if (!meta_usize(g, prefix + ".attention.head_count_kv", &kv)) kv = heads;
    if (!meta_usize(g, prefix + ".feed_forward_length", &inter)) inter = hidden * 4;
    if (!meta_usize(g, prefix + ".context_length", &ctxlen)) ctxlen = 2048;
    float theta, eps;
    if (!meta_f32(g, prefix + ".rope.freq_base", &theta)) theta = 10000.0f;
    if (!meta_f32(g, prefix + ".attention.layer_norm_rms_epsilon", &eps)) eps = 1e-5f;
    cfg->hidden_dim = (int)hidden;
    cfg->num_layers = (int)layers;
    cfg->num_heads = (int)heads;
    cfg->num_kv_heads = (int)kv;
    cfg->head_dim = (int)(hidden / heads);
    cfg->intermediate_dim = (int)inter;
    cfg->vocab_size = (int)vocab;
    cfg->max_seq_len = (int)ctxlen;
    cfg->rms_norm_eps = eps;
    cfg->rope_theta = theta;
    if (arch) *arch = id;
    return 0;
}

int fl_gguf_raw_weight(const fl_gguf *g, const char *name, fl_raw_weight *out) {
    // GgufFile::read_raw_weight (gguf.rs:616-653), zero-copy
    if (!g || !name || !out) return gg_fail(FL_E_INVALID, "null argument");
    const TensorInfo *t = g->find(name);
    if (!t) return gg_fail(FL_E_INVALID, std::string("tensor not found: ") + name);
    int fmt;
    uint64_t wpb;
    switch (t->type) {
    case 0: fmt = FL_F32; wpb = 1; break;
    case 8: fmt = FL_Q8_0; wpb = 32; break;
    case 12: fmt = FL_Q4K; wpb = 256; break;
    case 14: fmt = FL_Q6K; wpb = 256; break;
    default:
        return gg_fail(FL_E_UNSUPPORTED, std::string("tensor ") + name + ": ggml type " + std::to_string(t->type) +
                                             " is not on this backend's path (Q8_0, Q4_K, Q6_K, F32)");
    }
    const uint8_t *p;
    uint64_t bytes;
    int rc = tensor_span(g, *t, &p, &bytes);
    if (rc) return rc;
    // dimensions are [cols, rows]: the last one is the output rows
    const uint64_t rows = t->dims.empty() ? 1 : t->dims.back();
    uint64_t cols = 1;
    for (size_t d = 0; d + 1 < t->dims.size(); d++) cols *= t->dims[d];  // bounded: numel() did not overflow
    if (rows > (uint64_t)INT_MAX || (cols + wpb - 1) / wpb > (uint64_t)INT_MAX)
        return gg_fail(FL_E_INVALID, std::string("tensor ") + name + " has more rows or blocks than an int holds");
    out->data = p;
    out->nbytes = (size_t)bytes;
    out->format = fmt;
    out->num_rows = (int)rows;
    out->blocks_per_row = (int)((cols + wpb - 1) / wpb);
    return 0;
}

int fl_gguf_tensor_f32(const fl_gguf *g, const char *name, float *out, size_t n) {
    // a 1-D F32 / F16 tensor (norm weights), dequantized as dequantize_tensor does
    if (!g || !name || !out) return gg_fail(FL_E_INVALID, "null argument");
    const TensorInfo *t = g->find(name);
    if (!t) return gg_fail(FL_E_INVALID, std::string("tensor not found: ") + name);
    if (numel(*t) != n) return gg_fail(FL_E_INVALID, std::string("tensor ") + name + " has another size");
    const uint8_t *p;
    uint64_t bytes;
    int rc = tensor_span(g, *t, &p, &bytes);
    if (rc) return rc;
    if (t->type == 0) {
        std::memcpy(out, p, n * 4);
        return 0;
    }
    if (t->type == 1) {
        for (size_t i = 0; i < n; i++) {
            uint16_t h;
            std::memcpy(&h, p + 2 * i, 2);
            // IEEE binary16 -> binary32, subnormals included (quantize.rs:505-537)
            const uint32_t sign = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31, m = h & 1023;
            uint32_t bits;
            if (e == 0) {
                if (m == 0) {
                    bits = sign;
                } else {
                    int ee = -1;
                    uint32_t mm = m;
                    do {
                        ee++;
                        mm <<= 1;
                    } while (!(mm & 1024));
                    bits = sign | ((uint32_t)(127 - 15 - ee) << 23) | ((mm & 1023) << 13);
                }
            } else if (e == 31) {
                bits = sign | 0x7F800000u | (m << 13);
            } else {
                bits = sign | ((e + 112) << 23) | (m << 13);
            }
            std::memcpy(out + i, &bits, 4);
        }
        return 0;
    }
    return gg_fail(FL_E_UNSUPPORTED, std::string("tensor ") + name + " is not F32 / F16");
}

int fl_model_load_gguf(fl_ctx *ctx, const fl_gguf *g, int kv_format, int max_seq_len) {
    // weights.rs:30-66 names + load_raw_layer_weights (gguf.rs:661-688), then
    // init_gpu_kv_cache + upload_weights_to_gpu
    if (!ctx || !g) return fl_host_fail(ctx, FL_E_INVALID, "null argument");
    fl_model_config cfg;
    int arch = -1;
    int rc = fl_gguf_model_config(g, &cfg, &arch);
    if (rc) return fl_host_fail(ctx, rc, fl_last_error(nullptr));
    if (arch != 0 && arch != 2)  // llama, mistral: the decode path's arithmetic
        return fl_host_fail(ctx, FL_E_UNSUPPORTED, "architecture has biases / soft-capping this backend does not run");
    if (max_seq_len > 0) cfg.max_seq_len = max_seq_len;
    rc = fl_model_init(ctx, &cfg, kv_format);
    if (rc) return rc;
    const int L = cfg.num_layers;
    std::vector<fl_raw_weight> layers((size_t)7 * L);
    std::vector<std::vector<float>> an((size_t)L), fn((size_t)L);
    std::vector<const float *> anp((size_t)L), fnp((size_t)L);
    static const char *const names[7] = {"attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up",
                                         "ffn_down"};
    char name[128];
    for (int l = 0; l < L; l++) {
        for (int k = 0; k < 7; k++) {
            std::snprintf(name, sizeof name, "blk.%d.%s.weight", l, names[k]);
            rc = fl_gguf_raw_weight(g, name, &layers[(size_t)7 * l + k]);
            if (rc) return fl_host_fail(ctx, rc, fl_last_error(nullptr));
        }
        an[(size_t)l].resize((size_t)cfg.hidden_dim);
        fn[(size_t)l].resize((size_t)cfg.hidden_dim);
        std::snprintf(name, sizeof name, "blk.%d.attn_norm.weight", l);
        rc = fl_gguf_tensor_f32(g, name, an[(size_t)l].data(), (size_t)cfg.hidden_dim);
        if (!rc) {
            std::snprintf(name, sizeof name, "blk.%d.ffn_norm.weight", l);
            rc = fl_gguf_tensor_f32(g, name, fn[(size_t)l].data(), (size_t)cfg.hidden_dim);
        }
        if (rc) return fl_host_fail(ctx, rc, fl_last_error(nullptr));
        anp[(size_t)l] = an[(size_t)l].data();
        fnp[(size_t)l] = fn[(size_t)l].data();
    }
    std::vector<float> onorm((size_t)cfg.hidden_dim);
    const char *on = g->find("output_norm.weight") ? "output_norm.weight" : "model.norm.weight";
    rc = fl_gguf_tensor_f32(g, on, onorm.data(), onorm.size());
    if (rc) return fl_host_fail(ctx, rc, fl_last_error(nullptr));
    fl_raw_weight emb, outw;
    rc = fl_gguf_raw_weight(g, g->find("token_embd.weight") ? "token_embd.weight" : "model.embed_tokens.weight",
                            &emb);
    if (rc) return fl_host_fail(ctx, rc, fl_last_error(nullptr));
    const char *oname = g->find("output.weight") ? "output.weight" : (g->find("lm_head.weight") ? "lm_head.weight" : nullptr);
    if (oname) {
        rc = fl_gguf_raw_weight(g, oname, &outw);
        if (rc) return fl_host_fail(ctx, rc, fl_last_error(nullptr));
    }
    // tied output when output.weight is absent (weights.rs:50-51)
    return fl_upload_weights(ctx, layers.data(), anp.data(), fnp.data(), onorm.data(), &emb, oname ? &outw : nullptr);
}

}  // extern "C"
