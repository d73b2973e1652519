/*
 * Oracle restatement of crates/mivi-quant (TEST INFRASTRUCTURE ONLY).
 * See oracle.h for the pinning of each function.
 */
#include "oracle.h"

#include <immintrin.h>
#include <math.h>
#include <omp.h>
#include <stdlib.h>
#include <string.h>

static int g_threads = 1;
static int g_avx2 = 1;

void or_set_threads(int n) { g_threads = n < 1 ? 1 : n; }
int or_get_threads(void) { return g_threads; }
void or_set_avx2(int on) { g_avx2 = on ? 1 : 0; }

/* types.rs:91-101 */
int or_block_size(int32_t t, size_t* out) {
    switch (t) {
    case 0: case 26: case 28: case 27: /* F32 I32 F64 I64 */
    case 1: case 30: case 25: case 24: /* F16 BF16 I16 I8 */
        *out = 1; return 1;
    case 2: case 3: case 6: case 7: case 8: case 9:
        *out = 32; return 1;
    case 10: case 11: case 12: case 13: case 14: case 15:
        *out = 256; return 1;
    default: return 0;
    }
}

/* types.rs:110-130 */
int or_type_size(int32_t t, size_t* out) {
    switch (t) {
    case 0: case 26: *out = 4; return 1;
    case 1: case 30: case 25: *out = 2; return 1;
    case 24: *out = 1; return 1;
    case 27: case 28: *out = 8; return 1;
    case 2: *out = 18; return 1;
    case 3: *out = 20; return 1;
    case 6: *out = 22; return 1;
    case 7: *out = 24; return 1;
    case 8: *out = 34; return 1;
    case 9: *out = 36; return 1;
    case 10: *out = 84; return 1;
    case 11: *out = 110; return 1;
    case 12: *out = 144; return 1;
    case 13: *out = 176; return 1;
    case 14: *out = 210; return 1;
    case 15: *out = 292; return 1;
    default: return 0;
    }
}

/* `half` 2.7.1 f16::to_f32 is an exact widening; F16C does the same. */
float or_f16_to_f32(uint16_t h) { return _cvtsh_ss(h); }
/* `half` 2.7.1 f16::from_f32: IEEE round-to-nearest-even. */
uint16_t or_f32_to_f16(float f) { return (uint16_t)_cvtss_sh(f, _MM_FROUND_TO_NEAREST_INT); }
static inline float bf16_to_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}
static inline uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

static void set_err(or_quant_error* e, int kind) {
    if (e) { memset(e, 0, sizeof(*e)); e->kind = kind; }
}
static int err_small(or_quant_error* e, size_t expected, size_t actual) {
    set_err(e, OR_ERR_BUFFER_TOO_SMALL);
    if (e) { e->expected = expected; e->actual = actual; }
    return OR_ERR_BUFFER_TOO_SMALL;
}
static int err_misaligned(or_quant_error* e, size_t dim, size_t bs) {
    set_err(e, OR_ERR_DIMENSION_MISALIGNED);
    if (e) { e->dim = dim; e->block_size = bs; }
    return OR_ERR_DIMENSION_MISALIGNED;
}
static int err_unsupported(or_quant_error* e, int32_t t) {
    set_err(e, OR_ERR_UNSUPPORTED_TYPE);
    if (e) e->type_id = (uint32_t)t;
    return OR_ERR_UNSUPPORTED_TYPE;
}

/* ------------------------------------------------------------------ */
/* avx2.rs:12-21 */
static inline float hsum256(__m256 v) {
    __m128 lo = _mm256_castps256_ps128(v);
    __m128 hi = _mm256_extractf128_ps(v, 1);
    __m128 s128 = _mm_add_ps(lo, hi);
    __m128 shuf = _mm_movehl_ps(s128, s128);
    __m128 s64 = _mm_add_ps(s128, shuf);
    __m128 shuf2 = _mm_shuffle_ps(s64, s64, 1);
    __m128 s32 = _mm_add_ss(s64, shuf2);
    return _mm_cvtss_f32(s32);
}

/* q4_k_m.rs:11-22 */
void or_get_scale_min_k4(int j, const uint8_t* q, uint8_t* d, uint8_t* m) {
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* q4_k_m.rs:24-58 */
void or_dequantize_q4_k(const uint8_t* block, float* out) {
    float d = or_f16_to_f32(rd16(block));
    float dmin = or_f16_to_f32(rd16(block + 2));
    const uint8_t* scales = block + 4;
    const uint8_t* qs = block + 16;
    for (int j = 0; j < 4; j++) {
        uint8_t sc0, m0, sc1, m1;
        or_get_scale_min_k4(2 * j, scales, &sc0, &m0);
        or_get_scale_min_k4(2 * j + 1, scales, &sc1, &m1);
        float d1 = d * (float)sc0;
        float m1v = dmin * (float)m0;
        float d2 = d * (float)sc1;
        float m2v = dmin * (float)m1;
        const uint8_t* q = qs + j * 32;
        float* o = out + j * 64;
        for (int l = 0; l < 32; l++) {
            float q0 = (float)(q[l] & 0x0F);
            float q1 = (float)(q[l] >> 4);
            o[l] = d1 * q0 - m1v;
            o[l + 32] = d2 * q1 - m2v;
        }
    }
}

/* q6_k.rs:8-38 */
void or_dequantize_q6_k(const uint8_t* block, float* out) {
    const uint8_t* ql = block;
    const uint8_t* qh = block + 128;
    const uint8_t* sc = block + 192;
    float d = or_f16_to_f32(rd16(block + 208));
    for (int half = 0; half < 2; half++) {
        const uint8_t* qlh = ql + half * 64;
        const uint8_t* qhh = qh + half * 32;
        const int8_t* sch = (const int8_t*)(sc + half * 8);
        float* y = out + half * 128;
        for (int l = 0; l < 32; l++) {
            int is = l / 16;
            int q1 = (int)(int8_t)((qlh[l] & 0x0F) | ((qhh[l] & 3) << 4)) - 32;
            int q2 = (int)(int8_t)((qlh[l + 32] & 0x0F) | (((qhh[l] >> 2) & 3) << 4)) - 32;
            int q3 = (int)(int8_t)((qlh[l] >> 4) | (((qhh[l] >> 4) & 3) << 4)) - 32;
            int q4 = (int)(int8_t)((qlh[l + 32] >> 4) | (((qhh[l] >> 6) & 3) << 4)) - 32;
            y[l] = d * (float)sch[is] * (float)q1;
            y[l + 32] = d * (float)sch[is + 2] * (float)q2;
            y[l + 64] = d * (float)sch[is + 4] * (float)q3;
            y[l + 96] = d * (float)sch[is + 6] * (float)q4;
        }
    }
}

/* q8_0.rs:11-22 */
void or_dequantize_q8_0(const uint8_t* block, float* out) {
    float d = or_f16_to_f32(rd16(block));
    for (int i = 0; i < 32; i++) out[i] = (float)(int8_t)block[2 + i] * d;
}

/* q8_0.rs:31-58: amax/127, id from the f32 d (not the f16-rounded one),
 * round half away from zero (f32::round), clamp, saturating cast. */
void or_quantize_q8_0_block(const float* src, uint8_t* dst) {
    float amax = 0.0f;
    for (int i = 0; i < 32; i++) {
        float a = fabsf(src[i]);
        if (a > amax) amax = a;
    }
    float d = amax / 127.0f;
    float id = d != 0.0f ? 1.0f / d : 0.0f;
    uint16_t h = or_f32_to_f16(d);
    dst[0] = (uint8_t)(h & 0xFF);
    dst[1] = (uint8_t)(h >> 8);
    for (int i = 0; i < 32; i++) {
        float r = roundf(src[i] * id);
        if (r < -128.0f) r = -128.0f;
        if (r > 127.0f) r = 127.0f;
        dst[2 + i] = (uint8_t)(int8_t)r;
    }
}

/* q8_0.rs:60-124 */
float or_dot_q8_0_f32(const float* q, const uint8_t* k) {
    float d = or_f16_to_f32(rd16(k));
    if (g_avx2) {
        const uint8_t* kp = k + 2;
        __m128i k16_0 = _mm_loadu_si128((const __m128i*)kp);
        __m128i k16_1 = _mm_loadu_si128((const __m128i*)(kp + 16));
        __m256 k0 = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(k16_0));
        __m256 k1 = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_srli_si128(k16_0, 8)));
        __m256 k2 = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(k16_1));
        __m256 k3 = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_srli_si128(k16_1, 8)));
        __m256 acc = _mm256_mul_ps(_mm256_loadu_ps(q), k0);
        acc = _mm256_fmadd_ps(_mm256_loadu_ps(q + 8), k1, acc);
        acc = _mm256_fmadd_ps(_mm256_loadu_ps(q + 16), k2, acc);
        acc = _mm256_fmadd_ps(_mm256_loadu_ps(q + 24), k3, acc);
        return hsum256(acc) * d;
    }
    float sum = 0.0f;
    for (int i = 0; i < 32; i++) sum += q[i] * (float)(int8_t)k[2 + i];
    return sum * d;
}

/* ------------------------------------------------------------------ */
/* Row kernels. */

/* q4_k_m.rs:88-139 */
static float row_q4k_scalar(const uint8_t* row, const float* x, size_t nb) {
    float total = 0.0f;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t* blk = row + b * 144;
        float d = or_f16_to_f32(rd16(blk));
        float dmin = or_f16_to_f32(rd16(blk + 2));
        const uint8_t* scales = blk + 4;
        const uint8_t* qs = blk + 16;
        const float* xb = x + b * 256;
        for (int j = 0; j < 4; j++) {
            uint8_t sc0, m0, sc1, m1;
            or_get_scale_min_k4(2 * j, scales, &sc0, &m0);
            or_get_scale_min_k4(2 * j + 1, scales, &sc1, &m1);
            float d1 = d * (float)sc0, m1v = dmin * (float)m0;
            float d2 = d * (float)sc1, m2v = dmin * (float)m1;
            const uint8_t* q = qs + j * 32;
            const float* x0 = xb + j * 64;
            const float* x1 = xb + j * 64 + 32;
            float sq0 = 0, sx0 = 0, sq1 = 0, sx1 = 0;
            for (int l = 0; l < 32; l++) {
                float q0 = (float)(q[l] & 0x0F), q1 = (float)(q[l] >> 4);
                sq0 += q0 * x0[l];
                sx0 += x0[l];
                sq1 += q1 * x1[l];
                sx1 += x1[l];
            }
            total += d1 * sq0 - m1v * sx0 + d2 * sq1 - m2v * sx1;
        }
    }
    return total;
}

/* q4_k_m.rs:141-214 */
static float row_q4k_avx2(const uint8_t* row, const float* x, size_t nb) {
    float total = 0.0f;
    const __m256i mask = _mm256_set1_epi32(0x0F);
    for (size_t b = 0; b < nb; b++) {
        const uint8_t* blk = row + b * 144;
        float d = or_f16_to_f32(rd16(blk));
        float dmin = or_f16_to_f32(rd16(blk + 2));
        const uint8_t* scales = blk + 4;
        const uint8_t* qs = blk + 16;
        const float* xp = x + b * 256;
        for (int j = 0; j < 4; j++) {
            uint8_t sc0, m0, sc1, m1;
            or_get_scale_min_k4(2 * j, scales, &sc0, &m0);
            or_get_scale_min_k4(2 * j + 1, scales, &sc1, &m1);
            float d1 = d * (float)sc0, m1v = dmin * (float)m0;
            float d2 = d * (float)sc1, m2v = dmin * (float)m1;
            const uint8_t* qg = qs + j * 32;
            const float* x0p = xp + j * 64;
            const float* x1p = xp + j * 64 + 32;
            __m256 aq0 = _mm256_setzero_ps(), ax0 = _mm256_setzero_ps();
            __m256 aq1 = _mm256_setzero_ps(), ax1 = _mm256_setzero_ps();
            for (int k = 0; k < 4; k++) {
                int off = k * 8;
                __m256i bytes = _mm256_cvtepu8_epi32(_mm_loadl_epi64((const __m128i*)(qg + off)));
                __m256 q0 = _mm256_cvtepi32_ps(_mm256_and_si256(bytes, mask));
                __m256 xv0 = _mm256_loadu_ps(x0p + off);
                aq0 = _mm256_fmadd_ps(q0, xv0, aq0);
                ax0 = _mm256_add_ps(ax0, xv0);
                __m256 q1 = _mm256_cvtepi32_ps(_mm256_srli_epi32(bytes, 4));
                __m256 xv1 = _mm256_loadu_ps(x1p + off);
                aq1 = _mm256_fmadd_ps(q1, xv1, aq1);
                ax1 = _mm256_add_ps(ax1, xv1);
            }
            float sq0 = hsum256(aq0), sx0 = hsum256(ax0);
            float sq1 = hsum256(aq1), sx1 = hsum256(ax1);
            total += d1 * sq0 - m1v * sx0 + d2 * sq1 - m2v * sx1;
        }
    }
    return total;
}

/* q6_k.rs:68-111 */
static float row_q6k_scalar(const uint8_t* row, const float* x, size_t nb) {
    float total = 0.0f;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t* blk = row + b * 210;
        const uint8_t* ql = blk;
        const uint8_t* qh = blk + 128;
        const uint8_t* sc = blk + 192;
        float d = or_f16_to_f32(rd16(blk + 208));
        const float* xb = x + b * 256;
        float bsum = 0.0f;
        for (int half = 0; half < 2; half++) {
            const uint8_t* qlh = ql + half * 64;
            const uint8_t* qhh = qh + half * 32;
            const int8_t* sch = (const int8_t*)(sc + half * 8);
            const float* xh = xb + half * 128;
            for (int l = 0; l < 32; l++) {
                int is = l / 16;
                int q1 = (int)(int8_t)((qlh[l] & 0x0F) | ((qhh[l] & 3) << 4)) - 32;
                int q2 = (int)(int8_t)((qlh[l + 32] & 0x0F) | (((qhh[l] >> 2) & 3) << 4)) - 32;
                int q3 = (int)(int8_t)((qlh[l] >> 4) | (((qhh[l] >> 4) & 3) << 4)) - 32;
                int q4 = (int)(int8_t)((qlh[l + 32] >> 4) | (((qhh[l] >> 6) & 3) << 4)) - 32;
                float s0 = (float)sch[is], s1 = (float)sch[is + 2];
                float s2 = (float)sch[is + 4], s3 = (float)sch[is + 6];
                bsum += s0 * (float)q1 * xh[l] + s1 * (float)q2 * xh[l + 32] +
                        s2 * (float)q3 * xh[l + 64] + s3 * (float)q4 * xh[l + 96];
            }
        }
        total += bsum * d;
    }
    return total;
}

/* q6_k.rs:113-199 */
static float row_q6k_avx2(const uint8_t* row, const float* x, size_t nb) {
    float total = 0.0f;
    const __m256i m0f = _mm256_set1_epi32(0x0F), m03 = _mm256_set1_epi32(0x03);
    const __m256 c32 = _mm256_set1_ps(32.0f);
    for (size_t b = 0; b < nb; b++) {
        const uint8_t* blk = row + b * 210;
        const uint8_t* ql = blk;
        const uint8_t* qh = blk + 128;
        const int8_t* sc = (const int8_t*)(blk + 192);
        float d = or_f16_to_f32(rd16(blk + 208));
        const float* xp = x + b * 256;
        __m256 acc = _mm256_setzero_ps();
        for (int half = 0; half < 2; half++) {
            const uint8_t* qlh = ql + half * 64;
            const uint8_t* qhh = qh + half * 32;
            const int8_t* sch = sc + half * 8;
            const float* xh = xp + half * 128;
            for (int is = 0; is < 2; is++) {
                __m256 s0 = _mm256_set1_ps((float)sch[is]);
                __m256 s1 = _mm256_set1_ps((float)sch[is + 2]);
                __m256 s2 = _mm256_set1_ps((float)sch[is + 4]);
                __m256 s3 = _mm256_set1_ps((float)sch[is + 6]);
                for (int k = 0; k < 2; k++) {
                    int l = is * 16 + k * 8;
                    __m256i ql0 = _mm256_cvtepu8_epi32(_mm_loadl_epi64((const __m128i*)(qlh + l)));
                    __m256i ql32 = _mm256_cvtepu8_epi32(_mm_loadl_epi64((const __m128i*)(qlh + l + 32)));
                    __m256i qh0 = _mm256_cvtepu8_epi32(_mm_loadl_epi64((const __m128i*)(qhh + l)));
                    __m256i q1i = _mm256_or_si256(_mm256_and_si256(ql0, m0f),
                                                  _mm256_slli_epi32(_mm256_and_si256(qh0, m03), 4));
                    __m256 q1f = _mm256_sub_ps(_mm256_cvtepi32_ps(q1i), c32);
                    acc = _mm256_fmadd_ps(_mm256_mul_ps(s0, q1f), _mm256_loadu_ps(xh + l), acc);
                    __m256i q2i = _mm256_or_si256(
                        _mm256_and_si256(ql32, m0f),
                        _mm256_slli_epi32(_mm256_and_si256(_mm256_srli_epi32(qh0, 2), m03), 4));
                    __m256 q2f = _mm256_sub_ps(_mm256_cvtepi32_ps(q2i), c32);
                    acc = _mm256_fmadd_ps(_mm256_mul_ps(s1, q2f), _mm256_loadu_ps(xh + l + 32), acc);
                    __m256i q3i = _mm256_or_si256(
                        _mm256_srli_epi32(ql0, 4),
                        _mm256_slli_epi32(_mm256_and_si256(_mm256_srli_epi32(qh0, 4), m03), 4));
                    __m256 q3f = _mm256_sub_ps(_mm256_cvtepi32_ps(q3i), c32);
                    acc = _mm256_fmadd_ps(_mm256_mul_ps(s2, q3f), _mm256_loadu_ps(xh + l + 64), acc);
                    __m256i q4i = _mm256_or_si256(
                        _mm256_srli_epi32(ql32, 4),
                        _mm256_slli_epi32(_mm256_and_si256(_mm256_srli_epi32(qh0, 6), m03), 4));
                    __m256 q4f = _mm256_sub_ps(_mm256_cvtepi32_ps(q4i), c32);
                    acc = _mm256_fmadd_ps(_mm256_mul_ps(s3, q4f), _mm256_loadu_ps(xh + l + 96), acc);
                }
            }
        }
        total += hsum256(acc) * d;
    }
    return total;
}

/* q8_0.rs:180-197 */
static float row_q80_scalar(const uint8_t* row, const float* x, size_t nb) {
    float rs = 0.0f;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t* blk = row + b * 34;
        float d = or_f16_to_f32(rd16(blk));
        const float* xs = x + b * 32;
        float acc = 0.0f;
        for (int j = 0; j < 32; j++) acc += (float)(int8_t)blk[2 + j] * xs[j];
        rs += acc * d;
    }
    return rs;
}

/* q8_0.rs:199-240 */
static float row_q80_avx2(const uint8_t* row, const float* x, size_t nb) {
    float total = 0.0f;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t* blk = row + b * 34;
        float d = or_f16_to_f32(rd16(blk));
        const uint8_t* qs = blk + 2;
        const float* xp = x + b * 32;
        __m256 acc = _mm256_setzero_ps();
        for (int k = 0; k < 4; k++) {
            __m256 q = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_loadl_epi64((const __m128i*)(qs + 8 * k))));
            acc = _mm256_fmadd_ps(q, _mm256_loadu_ps(xp + 8 * k), acc);
        }
        total += hsum256(acc) * d;
    }
    return total;
}

/* f16.rs:42-64 (F16) and :75-97 (BF16): scalar sequential sums */
static float row_f16(const uint8_t* row, const float* x, size_t d) {
    float s = 0.0f;
    for (size_t j = 0; j < d; j++) s += or_f16_to_f32(rd16(row + 2 * j)) * x[j];
    return s;
}
static float row_bf16(const uint8_t* row, const float* x, size_t d) {
    float s = 0.0f;
    for (size_t j = 0; j < d; j++) s += bf16_to_f32(rd16(row + 2 * j)) * x[j];
    return s;
}
/* avx2.rs:30-57 matvec_f32_avx2 (aligned weights) */
static float row_f32_avx2(const float* row, const float* x, size_t d) {
    size_t chunks = d / 8;
    __m256 acc = _mm256_setzero_ps();
    for (size_t c = 0; c < chunks; c++)
        acc = _mm256_fmadd_ps(_mm256_loadu_ps(row + 8 * c), _mm256_loadu_ps(x + 8 * c), acc);
    float s = hsum256(acc);
    for (size_t r = chunks * 8; r < d; r++) s += row[r] * x[r];
    return s;
}
/* lib.rs:105-128 unaligned F32 fallback: plain sequential sum */
static float row_f32_unaligned(const uint8_t* row, const float* x, size_t d) {
    float s = 0.0f;
    for (size_t j = 0; j < d; j++) {
        float w;
        memcpy(&w, row + 4 * j, 4);
        s += w * x[j];
    }
    return s;
}

/* ------------------------------------------------------------------ */
/* types.rs:146-181 */
static int validate_matvec(size_t out_len, size_t w_len, size_t x_len, size_t n, size_t d,
                           size_t row_bytes, size_t bs, int row_bytes_overflow,
                           or_quant_error* err) {
    if (d % bs != 0) return err_misaligned(err, d, bs);
    if (out_len < n) return err_small(err, n, out_len);
    if (x_len < d) return err_small(err, d, x_len);
    size_t minw;
    if (row_bytes_overflow || __builtin_mul_overflow(n, row_bytes, &minw))
        return err_small(err, (size_t)-1, w_len);
    if (w_len < minw) return err_small(err, minw, w_len);
    return OR_OK;
}

typedef enum { K_Q4K, K_Q6K, K_Q80, K_F16, K_BF16, K_F32A, K_F32U } row_kind;

static float compute_row(row_kind k, const uint8_t* row, const float* x, size_t d) {
    switch (k) {
    case K_Q4K: return g_avx2 ? row_q4k_avx2(row, x, d / 256) : row_q4k_scalar(row, x, d / 256);
    case K_Q6K: return g_avx2 ? row_q6k_avx2(row, x, d / 256) : row_q6k_scalar(row, x, d / 256);
    case K_Q80: return g_avx2 ? row_q80_avx2(row, x, d / 32) : row_q80_scalar(row, x, d / 32);
    case K_F16: return row_f16(row, x, d);
    case K_BF16: return row_bf16(row, x, d);
    case K_F32A: return row_f32_avx2((const float*)row, x, d);
    case K_F32U: return row_f32_unaligned(row, x, d);
    }
    return 0.0f;
}

/* types.rs:240-269: 128-row chunks over the worker pool when n >= 256. */
static void parallel_row_matvec(float* out, const uint8_t* w, const float* x, size_t n,
                                size_t d, size_t row_bytes, row_kind k) {
    if (n >= 256) {
        long nchunks = (long)((n + 127) / 128);
#pragma omp parallel for schedule(dynamic, 1) num_threads(g_threads)
        for (long c = 0; c < nchunks; c++) {
            size_t r0 = (size_t)c * 128, r1 = r0 + 128 < n ? r0 + 128 : n;
            for (size_t i = r0; i < r1; i++) out[i] = compute_row(k, w + i * row_bytes, x, d);
        }
    } else {
        for (size_t i = 0; i < n; i++) out[i] = compute_row(k, w + i * row_bytes, x, d);
    }
}

/* lib.rs:75-134 */
int or_quantized_matvec(float* out, size_t out_len, int32_t t, const uint8_t* w, size_t w_len,
                        const float* x, size_t x_len, size_t n, size_t d, or_quant_error* err) {
    size_t row_bytes = 0, bs = 1;
    row_kind k;
    int ovf = 0;
    switch (t) {
    case OR_Q4_K: bs = 256; row_bytes = (d / 256) * 144; k = K_Q4K; break;  /* q4_k_m.rs:224-226 */
    case OR_Q6_K: bs = 256; row_bytes = (d / 256) * 210; k = K_Q6K; break;  /* q6_k.rs:209-211 */
    case OR_Q8_0: bs = 32; row_bytes = (d / 32) * 34; k = K_Q80; break;     /* q8_0.rs:134-136 */
    case OR_F16:
    case OR_BF16:                                                            /* f16.rs:49-52 */
        if (__builtin_mul_overflow(d, (size_t)2, &row_bytes)) {
            set_err(err, OR_ERR_ARITHMETIC_OVERFLOW);
            return OR_ERR_ARITHMETIC_OVERFLOW;
        }
        k = t == OR_F16 ? K_F16 : K_BF16;
        break;
    case OR_F32:                                                             /* lib.rs:89-94 */
        ovf = __builtin_mul_overflow(d, (size_t)4, &row_bytes);
        k = ((uintptr_t)w % 4 == 0) ? K_F32A : K_F32U;
        break;
    default: return err_unsupported(err, t);
    }
    int rc = validate_matvec(out_len, w_len, x_len, n, d, row_bytes, bs, ovf, err);
    if (rc) return rc;
    set_err(err, OR_OK);
    parallel_row_matvec(out, w, x, n, d, row_bytes, k);
    return OR_OK;
}

/* lib.rs:35-72 (the reference panics where it asserts; the oracle reports
 * BufferTooSmall for those cases instead) */
int or_dequantize_slice(int32_t t, const uint8_t* bytes, size_t bytes_len, float* out,
                        size_t out_len, or_quant_error* err) {
    size_t bb, be;
    void (*fn)(const uint8_t*, float*) = NULL;
    switch (t) {
    case OR_Q8_0: bb = 34; be = 32; fn = or_dequantize_q8_0; break;
    case OR_Q4_K: bb = 144; be = 256; fn = or_dequantize_q4_k; break;
    case OR_Q6_K: bb = 210; be = 256; fn = or_dequantize_q6_k; break;
    case OR_F16:
    case OR_BF16: {
        size_t count = bytes_len / 2;
        if (out_len < count) return err_small(err, count, out_len);
        for (size_t i = 0; i < count; i++)
            out[i] = t == OR_F16 ? or_f16_to_f32(rd16(bytes + 2 * i)) : bf16_to_f32(rd16(bytes + 2 * i));
        set_err(err, OR_OK);
        return OR_OK;
    }
    case OR_F32: {
        size_t count = bytes_len / 4;
        if (out_len < count) return err_small(err, count, out_len);
        for (size_t i = 0; i < count; i++) memcpy(out + i, bytes + 4 * i, 4);
        set_err(err, OR_OK);
        return OR_OK;
    }
    default: return err_unsupported(err, t);
    }
    size_t nblocks = out_len / be;                       /* types.rs:281-285 */
    if (bytes_len < nblocks * bb) return err_small(err, nblocks * bb, bytes_len);
    for (size_t b = 0; b < nblocks; b++) fn(bytes + b * bb, out + b * be);
    set_err(err, OR_OK);
    return OR_OK;
}

/* ------------------------------------------------------------------ */
/* simd/mod.rs:41-49 + avx2.rs:65-87 */
float or_dot_product(const float* a, const float* b, size_t len) {
    if (g_avx2) {
        size_t chunks = len / 8;
        __m256 acc = _mm256_setzero_ps();
        for (size_t c = 0; c < chunks; c++)
            acc = _mm256_fmadd_ps(_mm256_loadu_ps(a + 8 * c), _mm256_loadu_ps(b + 8 * c), acc);
        float s = hsum256(acc);
        for (size_t r = chunks * 8; r < len; r++) s += a[r] * b[r];
        return s;
    }
    float s = 0.0f;
    for (size_t i = 0; i < len; i++) s += a[i] * b[i];
    return s;
}

/* Per-lane semantics shared by avx2.rs:153-235 (pair) and :243-346 (single):
 * every output lane below floor(batch/8)*8 is a fused FMA chain over the
 * columns in order; the remaining lanes use an unfused multiply-add. The
 * reference's own test lib.rs:459-565 asserts pair == single bit for bit. */
static void accumulate_transposed(float* out, const float* wrow, const float* xt,
                                  size_t batch, size_t cols) {
    size_t vend = (batch / 8) * 8;
    size_t off = 0;
    for (; off + 8 <= vend; off += 8) {
        __m256 a = _mm256_loadu_ps(out + off);
        for (size_t c = 0; c < cols; c++)
            a = _mm256_fmadd_ps(_mm256_set1_ps(wrow[c]), _mm256_loadu_ps(xt + c * batch + off), a);
        _mm256_storeu_ps(out + off, a);
    }
    for (size_t b = vend; b < batch; b++) {
        float a = out[b];
        for (size_t c = 0; c < cols; c++) a += wrow[c] * xt[c * batch + b];
        out[b] = a;
    }
}

/* types.rs:188-235 */
static int validate_matmul(size_t out_len, size_t w_len, size_t in_len, size_t batch,
                           size_t rows, size_t cols, size_t row_bytes, size_t bs,
                           or_quant_error* err) {
    size_t e;
    if (cols % bs != 0) return err_misaligned(err, cols, bs);
    if (__builtin_mul_overflow(batch, rows, &e)) { set_err(err, OR_ERR_ARITHMETIC_OVERFLOW); return OR_ERR_ARITHMETIC_OVERFLOW; }
    if (out_len < e) return err_small(err, e, out_len);
    if (__builtin_mul_overflow(batch, cols, &e)) { set_err(err, OR_ERR_ARITHMETIC_OVERFLOW); return OR_ERR_ARITHMETIC_OVERFLOW; }
    if (in_len < e) return err_small(err, e, in_len);
    if (__builtin_mul_overflow(rows, row_bytes, &e)) { set_err(err, OR_ERR_ARITHMETIC_OVERFLOW); return OR_ERR_ARITHMETIC_OVERFLOW; }
    if (w_len < e) return err_small(err, e, w_len);
    return OR_OK;
}

/* lib.rs:254-342, one worker's row range */
static int batched_rows(float* rmo, size_t r0, size_t r1, size_t batch, size_t cols,
                        size_t row_bytes, int32_t t, const uint8_t* w, const float* in,
                        const float* xt) {
    float* dec = (float*)malloc(cols * sizeof(float));
    int rc = OR_OK;
    for (size_t r = r0; r < r1 && rc == OR_OK; r++) {
        float* o = rmo + (r - r0) * batch;
        rc = or_dequantize_slice(t, w + r * row_bytes, row_bytes, dec, cols, NULL);
        if (rc) break;
        if (batch <= 8) {
            for (size_t b = 0; b < batch; b++) o[b] = or_dot_product(dec, in + b * cols, cols);
        } else {
            memset(o, 0, batch * sizeof(float));
            if (g_avx2) {
                accumulate_transposed(o, dec, xt, batch, cols);
            } else {
                for (size_t b = 0; b < batch; b++) {
                    float a = 0.0f;
                    for (size_t c = 0; c < cols; c++) a += dec[c] * xt[c * batch + b];
                    o[b] = a;
                }
            }
        }
    }
    free(dec);
    return rc;
}

/* lib.rs:143-251 */
int or_quantized_matmul_rows(float* out, size_t out_len, int32_t t, const uint8_t* w,
                             size_t w_len, const float* in, size_t in_len, size_t batch,
                             size_t rows, size_t cols, or_quant_error* err) {
    size_t bs, ts, row_bytes;
    if (!or_block_size(t, &bs)) return err_unsupported(err, t);
    if (!or_type_size(t, &ts)) return err_unsupported(err, t);
    if (cols % bs != 0) return err_misaligned(err, cols, bs);
    if (__builtin_mul_overflow(cols / bs, ts, &row_bytes)) { set_err(err, OR_ERR_ARITHMETIC_OVERFLOW); return OR_ERR_ARITHMETIC_OVERFLOW; }
    int rc = validate_matmul(out_len, w_len, in_len, batch, rows, cols, row_bytes, bs, err);
    if (rc) return rc;
    if (batch == 1) return or_quantized_matvec(out, rows, t, w, w_len, in, cols, rows, cols, err);
    set_err(err, OR_OK);
    if (batch == 0 || rows == 0) return OR_OK;
    if (t != OR_Q8_0 && t != OR_Q4_K && t != OR_Q6_K && t != OR_F16 && t != OR_BF16 && t != OR_F32)
        return err_unsupported(err, t);

    float* xt = NULL;
    if (batch > 8) {
        xt = (float*)malloc(cols * batch * sizeof(float));
        for (size_t b = 0; b < batch; b++)
            for (size_t c = 0; c < cols; c++) xt[c * batch + b] = in[b * cols + c];
    }
    float* rmo = (float*)calloc(rows * batch, sizeof(float));
    int nt = g_threads;
    if (rows >= 256 && nt > 1) {
        size_t chunk = (rows + (size_t)nt - 1) / (size_t)nt;
        long nch = (long)((rows + chunk - 1) / chunk);
#pragma omp parallel for schedule(dynamic, 1) num_threads(nt)
        for (long c = 0; c < nch; c++) {
            size_t r0 = (size_t)c * chunk, r1 = r0 + chunk < rows ? r0 + chunk : rows;
            batched_rows(rmo + r0 * batch, r0, r1, batch, cols, row_bytes, t, w, in, xt);
        }
    } else {
        batched_rows(rmo, 0, rows, batch, cols, row_bytes, t, w, in, xt);
    }
    for (size_t r = 0; r < rows; r++)
        for (size_t b = 0; b < batch; b++) out[b * rows + r] = rmo[r * batch + b];
    free(rmo);
    free(xt);
    return OR_OK;
}
