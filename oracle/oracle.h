/*
 * CPU oracle for the mivi-v4 quantized-inference hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This is a plain-C restatement of the reference
 * Rust CPU path (crates/mivi-quant, crates/mivi-core, crates/mivi-kv,
 * crates/mivi-model). It is the parity checker for the HIP library and the
 * timed CPU baseline; it is never linked into or called by the product.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it.
 *
 * Every function cites the reference file:line it follows. The AVX2 row
 * kernels keep the reference's intrinsic order (the reference binary takes
 * the AVX2 path on every x86-64 host with AVX2+FMA), so results are bit-exact
 * with the reference wherever the reference itself is deterministic. The
 * library is compiled with -ffp-contract=off because Rust never contracts
 * a*b+c; FMAs appear only where the reference calls _mm256_fmadd_ps.
 *
 * Parity pinning (what checks each function; see tests/test_oracle_*.py):
 *   dequant Q4_K/Q6_K/Q8_0/F16/BF16/F32  - reference known answers
 *       (q6_k.rs:236-252, q8_0.rs:246-259), closed-form exhaustive scale/min
 *       decode, f64 brute force.
 *   row kernels / matvec / matmul_rows   - reference known answer
 *       (q8_0.rs:261-280), f64 brute force bound, batched==matvec
 *       (lib.rs:404-457), paired-order contract (lib.rs:459-565).
 *   q8_0 quantize + dot                  - q8_0.rs:282-307,
 *       tests/quantized_kv_and_prefill.rs:76-100, closed form.
 *   rope cache                           - rope.rs:238-259 (table vs direct),
 *       tests/long_context_retrieval.rs:45-91 (norm preservation).
 *   rmsnorm / silu / swiglu / softmax    - math.rs:188-241 closed forms.
 *   kv cache sizes                       - tests/quantized_kv_and_prefill.rs:4-74.
 *   forward_step (whole model)           - tests/fixtures/oracle_output.json
 *       (tiny model, tolerance 0.05 + argmax, oracle_comparison_test.rs:57-75),
 *       plus two-pass f64 attention and tile invariants.
 *   Parity unpinned: the YaRN ramp branch of RopeCache (rope.rs:71-105) is
 *       checked only for finiteness/norm preservation, as the reference is.
 */
#ifndef MIVI_ORACLE_H
#define MIVI_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GgmlType ids, crates/mivi-quant/src/types.rs:22-52 */
enum {
    OR_F32 = 0, OR_F16 = 1, OR_Q8_0 = 8, OR_Q4_K = 12, OR_Q6_K = 14, OR_BF16 = 30
};

/* QuantError variants in declaration order, types.rs:5-15 (0 = Ok). */
enum {
    OR_OK = 0,
    OR_ERR_UNSUPPORTED_TYPE = 1,
    OR_ERR_BUFFER_TOO_SMALL = 2,
    OR_ERR_DIMENSION_MISALIGNED = 3,
    OR_ERR_ARITHMETIC_OVERFLOW = 4,
};

typedef struct {
    int32_t kind;       /* one of OR_ERR_* */
    uint32_t type_id;   /* UnsupportedType(u32) */
    size_t expected;    /* BufferTooSmall */
    size_t actual;
    size_t dim;         /* DimensionMisaligned */
    size_t block_size;
} or_quant_error;

/* threading: number of OpenMP threads used by row-parallel kernels */
void or_set_threads(int n);
/* 1: attention heads one after another, as the reference's loop
 * (transformer.rs:128); 0 (default): heads over the threads for long caches */
void or_set_serial_attention(int on);
int or_get_threads(void);
/* 1 = AVX2+FMA kernels (reference default on x86-64), 0 = scalar kernels */
void or_set_avx2(int on);

/* --- mivi-quant --- */
int or_block_size(int32_t t, size_t* out);            /* types.rs:91-101 */
int or_type_size(int32_t t, size_t* out);             /* types.rs:110-130 */
float or_f16_to_f32(uint16_t h);
uint16_t or_f32_to_f16(float f);
void or_get_scale_min_k4(int j, const uint8_t* q, uint8_t* d, uint8_t* m); /* q4_k_m.rs:11-22 */
void or_dequantize_q4_k(const uint8_t* block, float* out);  /* q4_k_m.rs:24-58 */
void or_dequantize_q6_k(const uint8_t* block, float* out);  /* q6_k.rs:8-38 */
void or_dequantize_q8_0(const uint8_t* block, float* out);  /* q8_0.rs:11-22 */
void or_quantize_q8_0_block(const float* src, uint8_t* dst); /* q8_0.rs:31-58 */
float or_dot_q8_0_f32(const float* q, const uint8_t* k_block); /* q8_0.rs:60-124 */
/* lib.rs:35-72 */
int or_dequantize_slice(int32_t t, const uint8_t* bytes, size_t bytes_len,
                        float* out, size_t out_len, or_quant_error* err);
/* lib.rs:75-134 */
int or_quantized_matvec(float* out, size_t out_len, int32_t t,
                        const uint8_t* w, size_t w_len, const float* x, size_t x_len,
                        size_t n, size_t d, or_quant_error* err);
/* lib.rs:143-357 */
int or_quantized_matmul_rows(float* out, size_t out_len, int32_t t,
                             const uint8_t* w, size_t w_len, const float* in, size_t in_len,
                             size_t batch, size_t rows, size_t cols, or_quant_error* err);

/* --- mivi-core --- */
float or_compute_rms_scale(const float* x, size_t len, float eps);  /* norm.rs:6-32 */
void or_rms_norm(float* out, const float* x, const float* w, size_t len, float eps); /* norm.rs:38-72 */
void or_rms_norm_in_place(float* x, const float* w, size_t len, float eps);        /* norm.rs:78-116 */
float or_dot_product(const float* a, const float* b, size_t len);   /* simd/mod.rs:41-49 */
void or_vec_add(float* out, const float* src, size_t len);          /* avx2.rs:95-115 */
void or_vec_fmadd(float* out, float scale, const float* src, size_t len); /* avx2.rs:123-144 */
float or_silu(float x);                                              /* math.rs:76-82 */
void or_swiglu(float* gate, const float* up, size_t len);            /* math.rs:94-100 */
void or_softmax(float* x, size_t len);                               /* math.rs:32-72 */
/* rope.rs:50-122; scaling: 0 none, 1 linear, 2 yarn */
int or_rope_table(float* cos_t, float* sin_t, size_t head_dim, size_t max_seq_len,
                  float rope_base, int scaling, float scale, size_t orig_max_seq_len,
                  float beta_fast, float beta_slow);
/* rope.rs:212-231, interleaved pairs */
void or_rope_rotate(float* v, size_t n_heads, size_t head_dim, const float* cos_row,
                    const float* sin_row);
/* math.rs:150-182 (direct formula form used by the reference's own test) */
void or_apply_rope_direct(float* q, size_t q_len, float* k, size_t k_len,
                          size_t head_dim, size_t pos, float rope_base);
uint32_t or_argmax(const float* logits, size_t n);                  /* sampler.rs:305-316 */

/* sampler.rs: GenerationConfig's sampling fields (config.rs:163-174) */
typedef struct {
    float temperature, top_p, min_p, repetition_penalty, presence_penalty, frequency_penalty;
    uint32_t top_k;
} or_sampler_config;
uint64_t or_sampler_seed(uint64_t seed);                             /* sampler.rs:28-57 */
float or_random_f32(uint64_t* state);                                /* sampler.rs:70-77 */
void or_apply_penalties(float* l, size_t n, const uint32_t* recent, size_t nr, float rep,
                        float presence, float frequency);           /* sampler.rs:219-257 */
void or_apply_min_p(float* l, size_t n, float min_p);                /* sampler.rs:260-276 */
void or_apply_top_k(float* l, size_t n, size_t k);                   /* sampler.rs:287-301 */
/* sampler.rs:91-135 Sampler::sample (logits modified in place) */
uint32_t or_sample(float* l, size_t n, const uint32_t* recent, size_t nr,
                   const or_sampler_config* c, uint64_t* rng);

/* --- mivi-model + mivi-kv --- */
enum { OR_KV_F32 = 0, OR_KV_Q8_0 = 1, OR_KV_F16RT = 100 };

typedef struct or_model or_model;
typedef struct {
    size_t dim, hidden_dim, n_layers, n_heads, n_kv_heads, head_dim, kv_dim;
    size_t vocab_size, max_seq_len, ssm_conv_kernel;
    float rope_base, rms_norm_eps;
    int32_t n_attn_layers;
    int32_t yarn;           /* 1 if YaRN scaling active */
    float yarn_scale;
} or_model_info;

/* model.rs:105-233 (load from an in-memory GGUF image; the image must stay
 * alive for the model's lifetime, exactly like the reference's mmap). */
int or_model_create(const uint8_t* gguf, size_t len, size_t max_ctx, int kv_precision,
                    or_model** out, char* errbuf, size_t errlen);
void or_model_destroy(or_model* m);
void or_model_info_get(const or_model* m, or_model_info* info);
void or_model_reset(or_model* m);                                   /* model.rs:494-497 */
/* model.rs:336-433; compute_logits=0 for prefill steps. Returns 0 on success. */
int or_model_forward_step(or_model* m, uint32_t token, size_t pos, int compute_logits);
const float* or_model_logits(const or_model* m);
const float* or_model_hidden(const or_model* m);                     /* RunState.x */
/* transformer.rs:114-301 on standalone rows: K/V are [seq, kv_dim] floats
 * (OR_KV_F32) or [seq, kv_dim/32*34] bytes (OR_KV_Q8_0). */
void or_attention(const float* q, const void* kc, const void* vc, int prec, size_t n_heads, size_t n_kv_heads,
                  size_t head_dim, size_t seq, float* out);
/* State injection (cache.rs:827-914 / arena.rs:110-123 semantics, raw layouts):
 * KV: [n_attn, max_seq_len, row] where row = kv_dim floats (F32) or
 * kv_dim/32*34 bytes (Q8_0). conv: [n_layers, dim, kernel] floats. */
size_t or_model_kv_bytes(const or_model* m);
void* or_model_k_cache(or_model* m);
void* or_model_v_cache(or_model* m);
float* or_model_conv_states(or_model* m);
size_t or_model_conv_len(const or_model* m);

#ifdef __cplusplus
}
#endif
#endif
