/*
 * Oracle restatement of crates/mivi-core numerics (TEST INFRASTRUCTURE ONLY).
 */
#include "oracle.h"

#include <immintrin.h>
#include <math.h>
#include <string.h>

static inline float hsum256(__m256 v) {
    __m128 lo = _mm256_castps256_ps128(v);
    __m128 hi = _mm256_extractf128_ps(v, 1);
    __m128 s128 = _mm_add_ps(lo, hi);
    __m128 s64 = _mm_add_ps(s128, _mm_movehl_ps(s128, s128));
    __m128 s32 = _mm_add_ss(s64, _mm_shuffle_ps(s64, s64, 1));
    return _mm_cvtss_f32(s32);
}

/* norm.rs:6-32 (AVX2 branch: 8-lane FMA sum of squares, hsum, scalar tail) */
float or_compute_rms_scale(const float* x, size_t len, float eps) {
    if (len == 0) return 0.0f;
    size_t chunks = len / 8;
    __m256 acc = _mm256_setzero_ps();
    for (size_t c = 0; c < chunks; c++) {
        __m256 v = _mm256_loadu_ps(x + 8 * c);
        acc = _mm256_fmadd_ps(v, v, acc);
    }
    float s = hsum256(acc);
    for (size_t i = chunks * 8; i < len; i++) s += x[i] * x[i];
    return 1.0f / sqrtf(s / (float)len + eps);
}

/* norm.rs:38-72: out = (x * scale) * w */
void or_rms_norm(float* out, const float* x, const float* w, size_t len, float eps) {
    if (len == 0) return;
    float s = or_compute_rms_scale(x, len, eps);
    for (size_t i = 0; i < len; i++) out[i] = x[i] * s * w[i];
}

/* norm.rs:78-116 */
void or_rms_norm_in_place(float* x, const float* w, size_t len, float eps) {
    if (len == 0) return;
    float s = or_compute_rms_scale(x, len, eps);
    for (size_t i = 0; i < len; i++) x[i] = x[i] * s * w[i];
}

/* avx2.rs:95-115 */
void or_vec_add(float* out, const float* src, size_t len) {
    for (size_t i = 0; i < len; i++) out[i] += src[i];
}

/* avx2.rs:123-144: fused in 8-lane chunks, unfused scalar tail */
void or_vec_fmadd(float* out, float scale, const float* src, size_t len) {
    size_t chunks = len / 8;
    __m256 sv = _mm256_set1_ps(scale);
    for (size_t c = 0; c < chunks; c++) {
        __m256 o = _mm256_loadu_ps(out + 8 * c);
        _mm256_storeu_ps(out + 8 * c, _mm256_fmadd_ps(sv, _mm256_loadu_ps(src + 8 * c), o));
    }
    for (size_t i = chunks * 8; i < len; i++) out[i] += scale * src[i];
}

/* math.rs:76-82 */
float or_silu(float x) { return x <= -50.0f ? 0.0f : x / (1.0f + expf(-x)); }

/* math.rs:94-100 */
void or_swiglu(float* g, const float* u, size_t len) {
    for (size_t i = 0; i < len; i++) g[i] = or_silu(g[i]) * u[i];
}

/* math.rs:32-72 */
void or_softmax(float* x, size_t len) {
    if (len == 0) return;
    float mx = -INFINITY;
    for (size_t i = 0; i < len; i++)
        if (isfinite(x[i]) && x[i] > mx) mx = x[i];
    if (!isfinite(mx)) {
        float u = 1.0f / (float)len;
        for (size_t i = 0; i < len; i++) x[i] = u;
        return;
    }
    float sum = 0.0f;
    for (size_t i = 0; i < len; i++) {
        if (isfinite(x[i])) {
            x[i] = expf(x[i] - mx);
            sum += x[i];
        } else {
            x[i] = 0.0f;
        }
    }
    if (sum > 0.0f) {
        float inv = 1.0f / sum;
        for (size_t i = 0; i < len; i++) x[i] *= inv;
    } else {
        float u = 1.0f / (float)len;
        for (size_t i = 0; i < len; i++) x[i] = u;
    }
}

/* rope.rs:50-122 */
int or_rope_table(float* cos_t, float* sin_t, size_t head_dim, size_t max_seq_len,
                  float rope_base, int scaling, float scale, size_t orig_max_seq_len,
                  float beta_fast, float beta_slow) {
    if (head_dim % 2 != 0 || head_dim > 1024) return 1;
    size_t half = head_dim / 2;
    float inv_freq[512];
    for (size_t i = 0; i < half; i++) {
        float base_freq = 1.0f / powf(rope_base, (float)(2 * i) / (float)head_dim);
        float f = base_freq;
        if (scaling == 1) {
            f = scale > 0.0f ? base_freq / scale : base_freq;
        } else if (scaling == 2 && scale > 1.0f) {
            float orig_len = (float)(orig_max_seq_len > 1 ? orig_max_seq_len : 1);
            float low_rot = orig_len / (beta_slow > 0.01f ? beta_slow : 0.01f);
            float high_rot = orig_len / (beta_fast > 0.01f ? beta_fast : 0.01f);
            float wavelength = 2.0f * (float)M_PI / base_freq;
            float ramp;
            if (high_rot >= low_rot) {
                ramp = wavelength < high_rot ? 0.0f : 1.0f;
            } else if (wavelength < high_rot) {
                ramp = 0.0f;
            } else if (wavelength > low_rot) {
                ramp = 1.0f;
            } else {
                ramp = (wavelength - high_rot) / (low_rot - high_rot);
            }
            float scaled = base_freq / scale;
            f = (1.0f - ramp) * base_freq + ramp * scaled;
        }
        inv_freq[i] = f;
    }
    for (size_t pos = 0; pos < max_seq_len; pos++) {
        for (size_t i = 0; i < half; i++) {
            float angle = (float)pos * inv_freq[i];
            cos_t[pos * half + i] = cosf(angle);
            sin_t[pos * half + i] = sinf(angle);
        }
    }
    return 0;
}

/* rope.rs:452-473 */
void or_rope_rotate(float* v, size_t n_heads, size_t head_dim, const float* c, const float* s) {
    size_t half = head_dim / 2;
    for (size_t h = 0; h < n_heads; h++) {
        float* hd = v + h * head_dim;
        for (size_t i = 0; i < half; i++) {
            float v0 = hd[2 * i], v1 = hd[2 * i + 1];
            hd[2 * i] = v0 * c[i] - v1 * s[i];
            hd[2 * i + 1] = v0 * s[i] + v1 * c[i];
        }
    }
}

/* math.rs:150-182 */
void or_apply_rope_direct(float* q, size_t q_len, float* k, size_t k_len, size_t head_dim,
                          size_t pos, float rope_base) {
    for (int pass = 0; pass < 2; pass++) {
        float* v = pass == 0 ? q : k;
        size_t n = (pass == 0 ? q_len : k_len) / head_dim;
        for (size_t h = 0; h < n; h++) {
            float* hd = v + h * head_dim;
            for (size_t i = 0; i < head_dim; i += 2) {
                float freq = 1.0f / powf(rope_base, (float)i / (float)head_dim);
                float angle = (float)pos * freq;
                float sn = sinf(angle), cs = cosf(angle);
                float a = hd[i], b = hd[i + 1];
                hd[i] = a * cs - b * sn;
                hd[i + 1] = a * sn + b * cs;
            }
        }
    }
}

/* sampler.rs:305-316: first index of the strict maximum */
uint32_t or_argmax(const float* l, size_t n) {
    size_t idx = 0;
    float mx = -INFINITY;
    for (size_t i = 0; i < n; i++)
        if (l[i] > mx) { mx = l[i]; idx = i; }
    return (uint32_t)idx;
}
