// Synthetic model generation: seeded N(mean, std) weights quantized into GGUF
// block bytes.  Host-only.  The reference loads real GGUF files; this exists
// so that tests and the benchmark can build Llama-shaped models offline.
//
// Block encoders write the byte layouts the reference decodes:
//   Q8_0  flare-loader/src/quantize.rs:189-197
//   Q4_K  flare-core/src/model.rs:8700-8719 + quantize.rs:386-423 (flare
//         packing of the 6-bit scales and low/high nibble = weight j / j+128)
//   Q6_K  flare-loader/src/quantize.rs:343-384 (llama.cpp layout)
#include <cmath>
#include <cstdint>
#include <cstring>

#include "../../include/flare_hip.h"

namespace {

inline uint64_t splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

inline uint16_t f32_to_f16(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u, exp = (x >> 23) & 0xFFu, man = x & 0x7FFFFFu;
    if (exp == 0xFF) return (uint16_t)(sign | 0x7C00u | (man ? 0x200u : 0u));
    int32_t e = (int32_t)exp - 112;
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        man |= 0x800000u;
        uint32_t shift = (uint32_t)(14 - e), hm = man >> shift, rem = man & ((1u << shift) - 1u);
        uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (hm & 1u))) hm++;
        return (uint16_t)(sign | hm);
    }
    uint32_t h = sign | ((uint32_t)e << 10) | (man >> 13), rem = man & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)h;
}

inline float f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31, exp = (h >> 10) & 0x1F, man = h & 0x3FF, u;
    if (exp == 0) {
        if (man == 0) {
            u = sign;
        } else {
            int e = -1;
            do { man <<= 1; e++; } while (!(man & 0x400));
            u = sign | ((uint32_t)(112 - e) << 23) | ((man & 0x3FF) << 13);
        }
    } else if (exp == 31) {
        u = sign | 0x7F800000u | (man << 13);
    } else {
        u = sign | ((exp + 112) << 23) | (man << 13);
    }
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

inline void put16(uint8_t *p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }

inline int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

void enc_q8_0(const float *x, uint8_t *blk) {
    float amax = 0.0f;
    for (int i = 0; i < 32; i++) amax = std::fmax(amax, std::fabs(x[i]));
    uint16_t dh = f32_to_f16(amax / 127.0f);
    float d = f16_to_f32(dh);
    float id = d != 0.0f ? 1.0f / d : 0.0f;
    put16(blk, dh);
    for (int i = 0; i < 32; i++) blk[2 + i] = (uint8_t)(int8_t)clampi((int)std::lround(x[i] * id), -128, 127);
}

void enc_q4k(const float *x, uint8_t *blk) {
    // Sub-block j covers weights [32j, 32j+32): j<4 are low nibbles of
    // qs[32j..], j>=4 are high nibbles of qs[32(j-4)..].
    float scale[8], mnv[8];
    float max_scale = 0.0f, max_min = 0.0f;
    for (int j = 0; j < 8; j++) {
        float lo = 0.0f, hi = -INFINITY;
        for (int k = 0; k < 32; k++) {
            lo = std::fmin(lo, x[32 * j + k]);
            hi = std::fmax(hi, x[32 * j + k]);
        }
        scale[j] = (hi - lo) / 15.0f;
        mnv[j] = -lo;
        max_scale = std::fmax(max_scale, scale[j]);
        max_min = std::fmax(max_min, mnv[j]);
    }
    uint16_t dh = f32_to_f16(max_scale / 63.0f), mh = f32_to_f16(max_min / 63.0f);
    float d = f16_to_f32(dh), dmin = f16_to_f32(mh);
    uint8_t sc[8], mn[8];
    for (int j = 0; j < 8; j++) {
        sc[j] = (uint8_t)(d > 0.0f ? clampi((int)std::lround(scale[j] / d), 0, 63) : 0);
        mn[j] = (uint8_t)(dmin > 0.0f ? clampi((int)std::lround(mnv[j] / dmin), 0, 63) : 0);
    }
    put16(blk, dh);
    put16(blk + 2, mh);
    uint8_t *s = blk + 4;
    for (int i = 0; i < 4; i++) {
        s[i] = (uint8_t)((sc[i] & 63) | ((sc[i + 4] & 3) << 6));
        s[i + 4] = (uint8_t)((mn[i] & 63) | ((mn[i + 4] & 3) << 6));
        s[i + 8] = (uint8_t)(((sc[i + 4] >> 2) & 0xF) | (((mn[i + 4] >> 2) & 0xF) << 4));
    }
    uint8_t q[256];
    for (int j = 0; j < 8; j++) {
        float ds = d * (float)sc[j], dm = dmin * (float)mn[j];
        for (int k = 0; k < 32; k++) {
            int v = ds > 0.0f ? (int)std::lround((x[32 * j + k] + dm) / ds) : 0;
            q[32 * j + k] = (uint8_t)clampi(v, 0, 15);
        }
    }
    for (int j = 0; j < 128; j++) blk[16 + j] = (uint8_t)(q[j] | (q[j + 128] << 4));
}

void enc_q6k(const float *x, uint8_t *blk) {
    float scale[16], max_abs_scale = 0.0f, max_scale = 0.0f;
    for (int j = 0; j < 16; j++) {
        float amax = 0.0f, vmax = 0.0f;
        for (int k = 0; k < 16; k++) {
            float v = x[16 * j + k];
            if (std::fabs(v) > amax) { amax = std::fabs(v); vmax = v; }
        }
        scale[j] = amax > 0.0f ? -vmax / 32.0f : 0.0f;
        if (std::fabs(scale[j]) > max_abs_scale) { max_abs_scale = std::fabs(scale[j]); max_scale = scale[j]; }
    }
    uint16_t dh = f32_to_f16(max_abs_scale > 0.0f ? -max_scale / 128.0f : 0.0f);
    float d = f16_to_f32(dh);
    int8_t sc[16];
    for (int j = 0; j < 16; j++) sc[j] = (int8_t)(d != 0.0f ? clampi((int)std::lround(scale[j] / d), -128, 127) : 0);
    uint8_t *ql = blk, *qh = blk + 128;
    std::memset(blk, 0, 210);
    for (int e = 0; e < 256; e++) {
        float ds = d * (float)sc[e / 16];
        int qv = ds != 0.0f ? clampi((int)std::lround(x[e] / ds), -32, 31) : 0;
        uint8_t u = (uint8_t)(qv + 32);
        int half = e / 128, r = e % 128, g = r / 32, l = r % 32;
        int qa = 64 * half + l, qb = 64 * half + 32 + l, hb = 32 * half + l;
        switch (g) {
        case 0: ql[qa] |= (uint8_t)(u & 0xF); qh[hb] |= (uint8_t)((u >> 4) << 0); break;
        case 1: ql[qb] |= (uint8_t)(u & 0xF); qh[hb] |= (uint8_t)((u >> 4) << 2); break;
        case 2: ql[qa] |= (uint8_t)((u & 0xF) << 4); qh[hb] |= (uint8_t)((u >> 4) << 4); break;
        default: ql[qb] |= (uint8_t)((u & 0xF) << 4); qh[hb] |= (uint8_t)((u >> 4) << 6); break;
        }
    }
    for (int j = 0; j < 16; j++) blk[192 + j] = (uint8_t)sc[j];
    put16(blk + 208, dh);
}

}  // namespace

extern "C" {

void fl_synth_normal(uint64_t seed, uint64_t offset, size_t n, float mean, float std_,
                     float *out) {
    const double two_pi = 6.283185307179586;
    uint64_t key = splitmix64(seed * 0xD1B54A32D192ED03ull + 0x632BE59BD9B4E019ull);
#pragma omp parallel for schedule(static)
    for (long long i = 0; i < (long long)n; i++) {
        uint64_t r = splitmix64(key ^ ((offset + (uint64_t)i) * 0x9E3779B97F4A7C15ull));
        double u1 = ((double)(r >> 40) + 1.0) * (1.0 / 16777217.0);
        double u2 = (double)(r & 0xFFFFFFull) * (1.0 / 16777216.0);
        double z = std::sqrt(-2.0 * std::log(u1)) * std::cos(two_pi * u2);
        out[i] = mean + std_ * (float)z;
    }
}

size_t fl_format_row_bytes(int format, size_t cols) {
    switch (format) {
    case FL_F32: return cols * 4;
    case FL_Q8_0: return cols % 32 ? 0 : cols / 32 * 34;
    case FL_Q4K: return cols % 256 ? 0 : cols / 256 * 144;
    case FL_Q6K: return cols % 256 ? 0 : cols / 256 * 210;
    }
    return 0;
}

size_t fl_synth_quantize(const float *src, size_t rows, size_t cols, int format, uint8_t *out) {
    size_t rb = fl_format_row_bytes(format, cols);
    if (rb == 0) return 0;
#pragma omp parallel for schedule(static)
    for (long long r = 0; r < (long long)rows; r++) {
        const float *x = src + (size_t)r * cols;
        uint8_t *o = out + (size_t)r * rb;
        switch (format) {
        case FL_F32: std::memcpy(o, x, cols * 4); break;
        case FL_Q8_0: for (size_t b = 0; b < cols / 32; b++) enc_q8_0(x + b * 32, o + b * 34); break;
        case FL_Q4K: for (size_t b = 0; b < cols / 256; b++) enc_q4k(x + b * 256, o + b * 144); break;
        case FL_Q6K: for (size_t b = 0; b < cols / 256; b++) enc_q6k(x + b * 256, o + b * 210); break;
        }
    }
    return rb * rows;
}

}  // extern "C"
