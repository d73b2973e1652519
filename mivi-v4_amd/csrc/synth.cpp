// Synthetic inputs: seeded normals and f32 -> Q4_K / Q6_K / Q8_0 encoders.
//
// The reference ships no K-quant quantizer (its only quantizers are Q8_0:
// crates/mivi-quant/src/q8_0.rs:31-58 and training/export/convert_to_gguf.py:135-156),
// so benchmark and test weights are produced here. These encoders only make
// inputs; every parity check runs on the packed bytes they emit.
//
// Normals: pair p of a stream draws two uniforms from SplitMix64 seeded with
// (seed, p) and applies Box-Muller in double precision. Element order does not
// depend on the thread count.
#include <math.h>
#include <string.h>

#include <algorithm>
#include <thread>
#include <vector>

#include "../../include/mivi_hip.h"

namespace {

inline uint64_t splitmix64(uint64_t& s) {
    uint64_t z = (s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

inline void normal_pair(uint64_t seed, uint64_t p, double* z0, double* z1) {
    uint64_t s = seed * 0xD1B54A32D192ED03ull + p * 0x9E3779B97F4A7C15ull + 0x632BE59BD9B4E019ull;
    double u1 = ((double)(splitmix64(s) >> 11) + 1.0) * (1.0 / 9007199254740992.0);  // (0, 1]
    double u2 = (double)(splitmix64(s) >> 11) * (1.0 / 9007199254740992.0);          // [0, 1)
    double r = sqrt(-2.0 * log(u1));
    double t = 6.283185307179586476925 * u2;
    *z0 = r * cos(t);
    *z1 = r * sin(t);
}

template <typename F>
void parallel_for(size_t n, F f) {
    unsigned nt = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    if (n < 4096 || nt == 1) {
        f((size_t)0, n);
        return;
    }
    std::vector<std::thread> th;
    size_t chunk = (n + nt - 1) / nt;
    for (unsigned t = 0; t < nt; t++) {
        size_t a = t * chunk, b = std::min(n, a + chunk);
        if (a >= b) break;
        th.emplace_back([=] { f(a, b); });
    }
    for (auto& t : th) t.join();
}

inline uint16_t f32_to_f16(float f) {
    _Float16 h = (_Float16)f;  // round to nearest even
    uint16_t b;
    memcpy(&b, &h, 2);
    return b;
}
inline float f16_to_f32(uint16_t b) {
    _Float16 h;
    memcpy(&h, &b, 2);
    return (float)h;
}

// q8_0.rs:31-58 (same arithmetic as the reference's quantizer)
void enc_q8_0(const float* x, uint8_t* o) {
    float amax = 0.0f;
    for (int i = 0; i < 32; i++) amax = std::max(amax, fabsf(x[i]));
    float d = amax / 127.0f;
    float id = d != 0.0f ? 1.0f / d : 0.0f;
    uint16_t h = f32_to_f16(d);
    o[0] = (uint8_t)h;
    o[1] = (uint8_t)(h >> 8);
    for (int i = 0; i < 32; i++) {
        float r = roundf(x[i] * id);
        r = std::min(127.0f, std::max(-128.0f, r));
        o[2 + i] = (uint8_t)(int8_t)r;
    }
}

// Q4_K: per 32-value sub-block an affine (scale, min) fit, 6-bit codes
// against the f16 super-scales, packed as q4_k_m.rs:11-22 decodes them.
void enc_q4_k(const float* x, uint8_t* o) {
    float sc[8], mn[8];
    for (int s = 0; s < 8; s++) {
        float lo = 0.0f, hi = -INFINITY;
        for (int i = 0; i < 32; i++) {
            lo = std::min(lo, x[32 * s + i]);
            hi = std::max(hi, x[32 * s + i]);
        }
        sc[s] = std::max(0.0f, (hi - lo) / 15.0f);
        mn[s] = -lo;
    }
    float msc = 0.0f, mmn = 0.0f;
    for (int s = 0; s < 8; s++) {
        msc = std::max(msc, sc[s]);
        mmn = std::max(mmn, mn[s]);
    }
    float d = msc / 63.0f, dmin = mmn / 63.0f;
    uint16_t dh = f32_to_f16(d), mh = f32_to_f16(dmin);
    float df = f16_to_f32(dh), mf = f16_to_f32(mh);
    uint8_t isc[8], imn[8];
    for (int s = 0; s < 8; s++) {
        int a = df > 0.0f ? (int)lrintf(sc[s] / df) : 0;
        int b = mf > 0.0f ? (int)lrintf(mn[s] / mf) : 0;
        isc[s] = (uint8_t)std::min(63, std::max(0, a));
        imn[s] = (uint8_t)std::min(63, std::max(0, b));
    }
    o[0] = (uint8_t)dh; o[1] = (uint8_t)(dh >> 8);
    o[2] = (uint8_t)mh; o[3] = (uint8_t)(mh >> 8);
    uint8_t* q = o + 4;
    for (int j = 0; j < 4; j++) {
        q[j] = (uint8_t)((isc[j] & 63) | ((isc[j + 4] >> 4) << 6));
        q[j + 4] = (uint8_t)((imn[j] & 63) | ((imn[j + 4] >> 4) << 6));
        q[j + 8] = (uint8_t)((isc[j + 4] & 0xF) | ((imn[j + 4] & 0xF) << 4));
    }
    uint8_t code[256];
    for (int s = 0; s < 8; s++) {
        float D = df * (float)isc[s], M = mf * (float)imn[s];
        for (int i = 0; i < 32; i++) {
            int c = D > 0.0f ? (int)lrintf((x[32 * s + i] + M) / D) : 0;
            code[32 * s + i] = (uint8_t)std::min(15, std::max(0, c));
        }
    }
    uint8_t* qs = o + 16;
    for (int g = 0; g < 4; g++)
        for (int l = 0; l < 32; l++)
            qs[32 * g + l] = (uint8_t)(code[64 * g + l] | (code[64 * g + 32 + l] << 4));
}

// Q6_K: per 16-value sub-block a symmetric scale as an int8 multiple of the
// f16 super-scale, 6-bit codes with offset 32, packed as q6_k.rs:8-38
// decodes them.
void enc_q6_k(const float* x, uint8_t* o) {
    float s16[16];
    float ms = 0.0f;
    for (int s = 0; s < 16; s++) {
        float a = 0.0f;
        for (int i = 0; i < 16; i++) a = std::max(a, fabsf(x[16 * s + i]));
        s16[s] = a / 31.0f;
        ms = std::max(ms, s16[s]);
    }
    float d = ms / 127.0f;
    uint16_t dh = f32_to_f16(d);
    float df = f16_to_f32(dh);
    int8_t isc[16];
    for (int s = 0; s < 16; s++) {
        int v = df > 0.0f ? (int)lrintf(s16[s] / df) : 0;
        isc[s] = (int8_t)std::min(127, std::max(-128, v));
    }
    uint8_t code[256];
    for (int e = 0; e < 256; e++) {
        float D = df * (float)isc[e / 16];
        int c = D != 0.0f ? (int)lrintf(x[e] / D) : 0;
        code[e] = (uint8_t)(std::min(31, std::max(-32, c)) + 32);
    }
    uint8_t* ql = o;
    uint8_t* qh = o + 128;
    for (int h = 0; h < 2; h++) {
        for (int l = 0; l < 32; l++) {
            const uint8_t* c = code + 128 * h;
            ql[64 * h + l] = (uint8_t)((c[l] & 0xF) | ((c[l + 64] & 0xF) << 4));
            ql[64 * h + 32 + l] = (uint8_t)((c[l + 32] & 0xF) | ((c[l + 96] & 0xF) << 4));
            qh[32 * h + l] = (uint8_t)((c[l] >> 4) | ((c[l + 32] >> 4) << 2) | ((c[l + 64] >> 4) << 4) |
                                       ((c[l + 96] >> 4) << 6));
        }
    }
    memcpy(o + 192, isc, 16);
    o[208] = (uint8_t)dh;
    o[209] = (uint8_t)(dh >> 8);
}

bool sizes(int32_t t, size_t* bs, size_t* ts) {
    switch (t) {
    case MIVI_GGML_Q4_K: *bs = 256; *ts = 144; return true;
    case MIVI_GGML_Q6_K: *bs = 256; *ts = 210; return true;
    case MIVI_GGML_Q8_0: *bs = 32; *ts = 34; return true;
    case MIVI_GGML_F16: *bs = 1; *ts = 2; return true;
    case MIVI_GGML_F32: *bs = 1; *ts = 4; return true;
    default: return false;
    }
}

void encode_rows(int32_t t, const float* src, size_t rows, size_t cols, uint8_t* dst, size_t bs, size_t ts) {
    size_t nb = cols / bs;
    size_t total = rows * nb;
    parallel_for(total, [&](size_t a, size_t b) {
        for (size_t i = a; i < b; i++) {
            const float* x = src + i * bs;
            uint8_t* o = dst + i * ts;
            switch (t) {
            case MIVI_GGML_Q4_K: enc_q4_k(x, o); break;
            case MIVI_GGML_Q6_K: enc_q6_k(x, o); break;
            case MIVI_GGML_Q8_0: enc_q8_0(x, o); break;
            case MIVI_GGML_F16: { uint16_t h = f32_to_f16(*x); memcpy(o, &h, 2); break; }
            default: memcpy(o, x, 4); break;
            }
        }
    });
}

}  // namespace

extern "C" void mivi_synth_normal(uint64_t seed, float mean, float std, float* out, size_t n) {
    size_t pairs = (n + 1) / 2;
    parallel_for(pairs, [&](size_t a, size_t b) {
        for (size_t p = a; p < b; p++) {
            double z0, z1;
            normal_pair(seed, p, &z0, &z1);
            out[2 * p] = (float)(mean + std * z0);
            if (2 * p + 1 < n) out[2 * p + 1] = (float)(mean + std * z1);
        }
    });
}

extern "C" int32_t mivi_synth_quantize(int32_t t, const float* src, size_t rows, size_t cols, uint8_t* dst,
                                       size_t dst_len) {
    size_t bs, ts;
    if (!sizes(t, &bs, &ts)) return MIVI_ERR_UNSUPPORTED_TYPE;
    if (cols % bs) return MIVI_ERR_DIMENSION_MISALIGNED;
    if (dst_len < rows * (cols / bs) * ts) return MIVI_ERR_BUFFER_TOO_SMALL;
    encode_rows(t, src, rows, cols, dst, bs, ts);
    return MIVI_OK;
}

extern "C" int32_t mivi_synth_random_weights(int32_t t, uint64_t seed, float std, size_t rows, size_t cols,
                                             uint8_t* dst, size_t dst_len) {
    size_t bs, ts;
    if (!sizes(t, &bs, &ts)) return MIVI_ERR_UNSUPPORTED_TYPE;
    if (cols % bs) return MIVI_ERR_DIMENSION_MISALIGNED;
    if (dst_len < rows * (cols / bs) * ts) return MIVI_ERR_BUFFER_TOO_SMALL;
    // generate and encode in row slabs to bound memory
    const size_t slab = std::max<size_t>(1, (size_t)(64u << 20) / (cols * 4));
    std::vector<float> buf;
    for (size_t r0 = 0; r0 < rows; r0 += slab) {
        size_t nr = std::min(slab, rows - r0);
        buf.resize(nr * cols);
        // element index is global (row-major), so slabs compose exactly
        size_t e0 = r0 * cols;
        size_t n = nr * cols;
        parallel_for((n + 1) / 2, [&](size_t a, size_t b) {
            for (size_t p = a; p < b; p++) {
                size_t e = e0 + 2 * p;
                // pairs are aligned to even global indices (cols is even)
                double z0, z1;
                normal_pair(seed, e / 2, &z0, &z1);
                buf[2 * p] = (float)(std * z0);
                if (2 * p + 1 < n) buf[2 * p + 1] = (float)(std * z1);
            }
        });
        encode_rows(t, buf.data(), nr, cols, dst + r0 * (cols / bs) * ts, bs, ts);
    }
    return MIVI_OK;
}
