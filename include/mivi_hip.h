/*
 * mivi-hip: MI355X (gfx950) implementation of mivi-v4's quantized-inference
 * hot path behind a plain C ABI.
 *
 * Every entry point replaces one function of the reference's Rust surface
 * (crates/mivi-quant, crates/mivi-model); the citation on each declaration
 * names it. Conventions:
 *
 *  - Buffers passed to compute entry points are GPU-accessible pointers
 *    (hipMalloc'd device memory); their lengths are given in elements (f32)
 *    or bytes (u8), exactly like the reference's slices, so the host can run
 *    the reference's validation before anything is launched.
 *  - `stream` is a hipStream_t (NULL = the default stream). Work is enqueued
 *    on it and the call returns; results are ready once the stream is
 *    synchronized. Validation errors are returned synchronously and nothing
 *    is written to `out` (reference: validate-before-write, types.rs:146-235,
 *    lib.rs:152-169).
 *  - Return value: 0 = Ok; 1..4 = the QuantError variants in declaration
 *    order (types.rs:5-15); >= 100 = HIP / model errors. Details of the last
 *    failure on the calling thread: mivi_hip_last_error().
 */
#ifndef MIVI_HIP_H
#define MIVI_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GgmlType ids (crates/mivi-quant/src/types.rs:22-52) */
#define MIVI_GGML_F32 0
#define MIVI_GGML_F16 1
#define MIVI_GGML_Q8_0 8
#define MIVI_GGML_Q4_K 12
#define MIVI_GGML_Q6_K 14
#define MIVI_GGML_BF16 30

/* status codes */
#define MIVI_OK 0
#define MIVI_ERR_UNSUPPORTED_TYPE 1      /* QuantError::UnsupportedType(u32) */
#define MIVI_ERR_BUFFER_TOO_SMALL 2      /* QuantError::BufferTooSmall{expected,actual} */
#define MIVI_ERR_DIMENSION_MISALIGNED 3  /* QuantError::DimensionMisaligned{dim,block_size} */
#define MIVI_ERR_ARITHMETIC_OVERFLOW 4   /* QuantError::ArithmeticOverflow */
#define MIVI_ERR_HIP 100                 /* a HIP runtime call failed */
#define MIVI_ERR_INVALID_ARGUMENT 101    /* null pointer / bad handle */
#define MIVI_ERR_INVALID_TOKEN 110       /* ModelError::InvalidToken (model.rs:41-42) */
#define MIVI_ERR_CONTEXT_OVERFLOW 111    /* ModelError::ContextOverflow (model.rs:43-44) */
#define MIVI_ERR_GGUF 112                /* ModelError::Gguf (model.rs:27-28) */
#define MIVI_ERR_MISSING_WEIGHT 113      /* ModelError::MissingWeight (model.rs:35-36) */
#define MIVI_ERR_INVALID_CONFIG 114      /* ModelError::InvalidConfig (model.rs:37-38) */
#define MIVI_ERR_KV_CACHE 115            /* ModelError::KvCache (model.rs:33-34) */
#define MIVI_ERR_UNSUPPORTED 116         /* a model feature this build does not run */

typedef struct mivi_error {
    int32_t code;          /* one of MIVI_* above */
    uint32_t type_id;      /* UnsupportedType payload */
    size_t expected;       /* BufferTooSmall payload */
    size_t actual;
    size_t dim;            /* DimensionMisaligned payload */
    size_t block_size;
    char message[256];     /* formatted like the reference's Display impls */
} mivi_error;

/* Details of the last non-zero status returned on this thread. */
int32_t mivi_hip_last_error(mivi_error* out);
/* Library version string. */
const char* mivi_hip_version(void);

/* ---------------------------------------------------------------------
 * mivi-quant
 * ------------------------------------------------------------------- */

/* crates/mivi-quant/src/lib.rs:75-134 quantized_matvec:
 * out[n] = W[n, d] * x[d] for W in `ggml_type` (Q4_K, Q6_K, Q8_0, F16, BF16,
 * F32). `out_len` may exceed n; the tail is left untouched (types.rs:312-328). */
int32_t mivi_hip_quantized_matvec(float* out, size_t out_len, int32_t ggml_type,
                                  const uint8_t* weights, size_t weights_len,
                                  const float* x, size_t x_len, size_t n, size_t d,
                                  void* stream);

/* crates/mivi-quant/src/q4_k_m.rs:217-237 try_matvec_q4_k_m */
int32_t mivi_hip_try_matvec_q4_k_m(float* out, size_t out_len, const uint8_t* weights,
                                   size_t weights_len, const float* x, size_t x_len,
                                   size_t n, size_t d, void* stream);
/* crates/mivi-quant/src/q6_k.rs:202-221 try_matvec_q6_k */
int32_t mivi_hip_try_matvec_q6_k(float* out, size_t out_len, const uint8_t* weights,
                                 size_t weights_len, const float* x, size_t x_len,
                                 size_t n, size_t d, void* stream);
/* crates/mivi-quant/src/q8_0.rs:127-147 try_matvec_q8_0 */
int32_t mivi_hip_try_matvec_q8_0(float* out, size_t out_len, const uint8_t* weights,
                                 size_t weights_len, const float* x, size_t x_len,
                                 size_t n, size_t d, void* stream);
/* crates/mivi-quant/src/f16.rs:42-64 try_matvec_f16 */
int32_t mivi_hip_try_matvec_f16(float* out, size_t out_len, const uint8_t* weights,
                                size_t weights_len, const float* x, size_t x_len,
                                size_t n, size_t d, void* stream);
/* crates/mivi-quant/src/f16.rs:75-97 try_matvec_bf16 */
int32_t mivi_hip_try_matvec_bf16(float* out, size_t out_len, const uint8_t* weights,
                                 size_t weights_len, const float* x, size_t x_len,
                                 size_t n, size_t d, void* stream);

/* crates/mivi-quant/src/lib.rs:143-251 quantized_matmul_rows:
 * out[batch, rows] = inputs[batch, cols] * W[rows, cols]^T. batch == 1 is the
 * matvec path (lib.rs:173-182); Q4_K with batch >= 16 and cols a multiple of
 * 2048 runs on the matrix cores, other cases one GEMV per input row. */
int32_t mivi_hip_quantized_matmul_rows(float* out, size_t out_len, int32_t ggml_type,
                                       const uint8_t* weights, size_t weights_len,
                                       const float* inputs, size_t inputs_len, size_t batch,
                                       size_t rows, size_t cols, void* stream);

/* No counterpart in the reference (its Rust kernels read the GGUF layout):
 * rewrites rows x cols weights into the layout of the packed GEMV, of the
 * same size. Q6_K (cols 2048, 4096 or 8192): with cols 2048 and rows a
 * multiple of 4, row quads (four rows' codes, scales and d interleaved for the
 * matrix-core GEMV, codes re-encoded six bits to a byte); otherwise unit
 * planes, a byte permutation of each row. Q4_K (cols 2048 or 8192, rows a
 * multiple of 4): row quads of 4608-byte sub-quads (four rows' code bytes,
 * 6-bit scales and mins, d and dmin laid out for the matrix-core GEMV). dst
 * must not overlap src. Other types/shapes return MIVI_ERR_UNSUPPORTED. For
 * callers that keep weights resident (the model loader packs the Q6_K head
 * and every Q4_K projection once). */
int32_t mivi_hip_pack_weights(int32_t ggml_type, const uint8_t* src, size_t src_len, uint8_t* dst,
                              size_t dst_len, size_t rows, size_t cols, void* stream);

/* quantized_matvec (lib.rs:75-134) over weights packed by
 * mivi_hip_pack_weights (16-byte aligned): the same result as
 * mivi_hip_quantized_matvec on the unpacked bytes, bit for bit; validation,
 * sizes and errors as there. No counterpart in the reference. */
int32_t mivi_hip_quantized_matvec_packed(float* out, size_t out_len, int32_t ggml_type,
                                         const uint8_t* packed, size_t packed_len, const float* x,
                                         size_t x_len, size_t n, size_t d, void* stream);

/* quantized_matmul_rows (lib.rs:143-251) over weights packed by
 * mivi_hip_pack_weights (16-byte aligned): out[batch, rows] = inputs[batch,
 * cols] * W^T, every input's row of outputs equal to its own
 * mivi_hip_quantized_matvec_packed bit for bit (Q6_K row quads: up to eight
 * inputs per launch, each quad read once for them); sizes and errors as
 * mivi_hip_quantized_matmul_rows. No counterpart in the reference. */
int32_t mivi_hip_quantized_matmul_rows_packed(float* out, size_t out_len, int32_t ggml_type,
                                              const uint8_t* packed, size_t packed_len, const float* inputs,
                                              size_t inputs_len, size_t batch, size_t rows, size_t cols,
                                              void* stream);

/* No counterpart in the reference (its Rust kernels read the GGUF layout):
 * the size in bytes of mivi_hip_pack_weights_gemm's copy of rows x cols
 * weights, 0 when it has none (Q4_K only, rows a multiple of 32, cols of
 * 2048): rows * cols * 2 + (rows / 32) * (cols / 256) * 640. */
size_t mivi_hip_gemm_packed_size(int32_t ggml_type, size_t rows, size_t cols);

/* No counterpart in the reference: rewrites rows x cols Q4_K weights into the
 * operand layout of the matrix-core row products (the fp16 values sc * q of
 * every weight in MFMA B-operand order, then d, dmin and the sub-block mins
 * per row and super-block), mivi_hip_gemm_packed_size bytes; src and dst
 * 16-byte aligned and distinct. For callers that run row products on
 * resident weights (the model loader packs every Q4_K projection once for
 * the chunked prefill). Other types/shapes return MIVI_ERR_UNSUPPORTED. */
int32_t mivi_hip_pack_weights_gemm(int32_t ggml_type, const uint8_t* src, size_t src_len, uint8_t* dst,
                                   size_t dst_len, size_t rows, size_t cols, void* stream);

/* quantized_matmul_rows (lib.rs:143-251) over weights with their
 * mivi_hip_pack_weights_gemm copy (wg): batch >= 16 runs the matrix cores on
 * wg, fewer inputs the GEMVs on the GGUF rows w; the results equal
 * mivi_hip_quantized_matmul_rows' bit for bit; sizes and errors as there
 * (wg_len below mivi_hip_gemm_packed_size: buffer too small). No counterpart
 * in the reference. */
int32_t mivi_hip_quantized_matmul_rows_gemm_packed(float* out, size_t out_len, int32_t ggml_type,
                                                   const uint8_t* weights, size_t weights_len,
                                                   const uint8_t* wg, size_t wg_len, const float* inputs,
                                                   size_t inputs_len, size_t batch, size_t rows, size_t cols,
                                                   void* stream);

/* crates/mivi-quant/src/lib.rs:35-72 dequantize_slice: bit-exact decode of
 * out_len / block_size blocks (Q4_K, Q6_K, Q8_0) or of bytes_len / type_size
 * elements (F16, BF16, F32). */
int32_t mivi_hip_dequantize_slice(int32_t ggml_type, const uint8_t* bytes, size_t bytes_len,
                                  float* out, size_t out_len, void* stream);

/* crates/mivi-quant/src/q8_0.rs:31-58 quantize_f32_to_q8_0_block, applied to
 * n_blocks consecutive 32-element blocks: dst holds n_blocks * 34 bytes. */
int32_t mivi_hip_quantize_q8_0(const float* src, size_t src_len, uint8_t* dst, size_t dst_len,
                               size_t n_blocks, void* stream);

/* crates/mivi-quant/src/q8_0.rs:60-124 dot_q8_0_f32, applied to n pairs:
 * out[i] = dot(q[32 i .. 32 i + 32], k_blocks[34 i .. 34 i + 34]). */
int32_t mivi_hip_dot_q8_0_f32(const float* q, size_t q_len, const uint8_t* k_blocks,
                              size_t k_len, float* out, size_t out_len, size_t n, void* stream);

/* ---------------------------------------------------------------------
 * mivi-model: one hybrid (ShortConv + GQA) model resident on the GPU
 * ------------------------------------------------------------------- */

/* KvPrecision (crates/mivi-kv/src/cache.rs:5-15) plus the half-precision
 * layout this build adds. */
#define MIVI_KV_F32 0
#define MIVI_KV_Q8_0 1
#define MIVI_KV_F16 2

typedef struct mivi_model mivi_model;

typedef struct mivi_model_info {
    size_t dim, hidden_dim, n_layers, n_heads, n_kv_heads, head_dim, kv_dim;
    size_t vocab_size, max_seq_len, ssm_conv_kernel, n_attn_layers, max_batch;
    float rope_base, rms_norm_eps;
    int32_t kv_precision, yarn;
    float yarn_scale;
    size_t weight_bytes;   /* device bytes of the weights: the GGUF tensor data plus the
                              packed copies kept beside it (Q6_K head, Q4_K and Q6_K row
                              quads; with max_batch > 1 the Q4_K projections in the batched
                              column kernels' group order and the Q6_K head in 32-row tiles;
                              the Q4_K projections' fp16 sc * q for the prefill's row
                              products); MIVI_NO_PACK=1 at create leaves the copies out,
                              MIVI_NO_COLS_PACK=1 the batched projections',
                              MIVI_NO_HEAD_T32=1 the batched head's, MIVI_NO_GEMM_PACK=1 the
                              row products' */
    size_t kv_bytes;       /* device bytes of K + V for all sequences */
} mivi_model_info;

/* crates/mivi-model/src/model.rs:105-233 Model::load_with_options, from an
 * in-memory GGUF image (host memory; copied to the device, so the image may
 * be freed afterwards). max_ctx = 0 selects the reference default (16384,
 * capped at 65536, model.rs:132-138). max_batch >= 1 independent sequences
 * (each with its own KV cache and ShortConv state). */
int32_t mivi_hip_model_create(const uint8_t* gguf, size_t gguf_len, size_t max_ctx,
                              int32_t kv_precision, size_t max_batch, mivi_model** out);
void mivi_hip_model_destroy(mivi_model* m);
int32_t mivi_hip_model_info(const mivi_model* m, mivi_model_info* out);

/* model.rs:494-497 Model::reset_context (all sequences) */
int32_t mivi_hip_model_reset(mivi_model* m);

/* model.rs:336-433 Model::forward_step for sequence `seq`. With
 * compute_logits != 0 the logits are copied to `logits_host` (vocab_size
 * floats, host memory) when it is non-NULL. Synchronous. */
int32_t mivi_hip_model_forward_step(mivi_model* m, size_t seq, uint32_t token, size_t pos,
                                    int32_t compute_logits, float* logits_host);

/* model.rs:488-491 Model::forward: forward_step with logits. */
int32_t mivi_hip_model_forward(mivi_model* m, size_t seq, uint32_t token, size_t pos,
                               float* logits_host);

/* model.rs:488-491 Model::forward of sequences 0..batch-1 (tokens[b] at
 * pos[b], host arrays) in one batched step: the batched decode's kernels
 * (each projection one GEMV over the batch's columns, one attention launch
 * with the batch's split count). logits_host (batch * vocab_size floats,
 * host, row b = sequence b) may be NULL. The reference runs one Model per
 * sequence; each row equals that sequence's forward up to float rounding.
 * Synchronous. */
int32_t mivi_hip_model_forward_batch(mivi_model* m, size_t batch, const uint32_t* tokens,
                                     const size_t* pos, float* logits_host);

/* Greedy decode loop (the argmax feedback of oracle_comparison_test.rs:37-50
 * and sampler.rs:305-316, without penalties): feeds `token` at `pos`, then
 * n_steps - 1 times the argmax of the previous logits; writes the n_steps
 * argmax tokens to tokens_out (host). All sequences 0..batch-1 advance
 * together, each from tokens[i] at pos[i] (host arrays). Runs from one
 * captured HIP graph; synchronous. */
int32_t mivi_hip_model_generate_greedy(mivi_model* m, size_t batch, const uint32_t* tokens,
                                       const size_t* pos, size_t n_steps, uint32_t* tokens_out);

/* Prompt prefill of one sequence (model.rs:499-606): with the default
 * PrefillStrategy::Token, forward_step(tokens[i], pos0 + i, false) per token;
 * after mivi_hip_model_set_prefill_tile(m, t > 1), PrefillStrategy::Chunked:
 * tiles of t tokens through every layer at once (model.rs:676-831,
 * attention_forward_tile transformer.rs:356-559, ssm_forward_tile
 * ssm.rs:174-387): row-batch products (matrix cores for Q4_K), K/V and the
 * ShortConv state left as the token path leaves them. Synchronous. */
int32_t mivi_hip_model_prefill(mivi_model* m, size_t seq, const uint32_t* tokens, size_t n,
                               size_t pos0);

/* Model::set_prefill_strategy (model.rs:260-266): tile_tokens 0 or 1 =
 * Token, t > 1 = Chunked { tile_tokens: t } (at most 4096). Tile buffers are
 * allocated by the first chunked prefill. */
int32_t mivi_hip_model_set_prefill_tile(mivi_model* m, size_t tile_tokens);

/* State export/import for one sequence (cache.rs:682-914, arena.rs:110-123
 * semantics with raw layouts): K and V are [n_attn_layers, tokens, row] with
 * row = kv_dim floats (F32), kv_dim halves (F16) or kv_dim/32*34 bytes
 * (Q8_0); conv is [n_layers, dim, ssm_conv_kernel] floats. Host buffers. */
int32_t mivi_hip_model_export_state(mivi_model* m, size_t seq, size_t tokens, void* k_out,
                                    void* v_out, size_t kv_len, float* conv_out,
                                    size_t conv_len);
int32_t mivi_hip_model_import_state(mivi_model* m, size_t seq, size_t tokens, const void* k_in,
                                    const void* v_in, size_t kv_len, const float* conv_in,
                                    size_t conv_len);

/* cache.rs:688-746 KvCache::export_state_range for sequence seq: the K and V
 * rows of positions [start, start + tokens) of every attention layer, laid
 * out as mivi_hip_model_export_state's ([n_attn_layers, tokens, row]; kv_len
 * bytes each, at least that size); with conv_out non-NULL also the
 * ShortConv state (arena.rs:110-114). An interval past max_seq_len returns
 * MIVI_ERR_KV_CACHE (KvError::ContextOverflow). Host buffers; synchronous. */
int32_t mivi_hip_model_export_state_range(mivi_model* m, size_t seq, size_t start, size_t tokens,
                                          void* k_out, void* v_out, size_t kv_len, float* conv_out,
                                          size_t conv_len);

/* cache.rs:827-914 KvCache::import_state_at: an interval export into
 * positions [start, start + tokens) of sequence seq's caches, every other
 * position left as it is; kv_len must be exactly n_attn_layers * tokens *
 * row (else MIVI_ERR_KV_CACHE, KvError::DimMismatch). With conv_in non-NULL
 * (conv_len exact) the ShortConv state is imported too (arena.rs:116-123),
 * else left as it is. The device model keeps no cache position, so this is
 * also import_state_range (cache.rs:814-822). Host buffers; synchronous. */
int32_t mivi_hip_model_import_state_at(mivi_model* m, size_t seq, size_t start, size_t tokens,
                                       const void* k_in, const void* v_in, size_t kv_len,
                                       const float* conv_in, size_t conv_len);

/* ---------------------------------------------------------------------
 * Sampling: crates/mivi-model/src/sampler.rs:91-135 (Sampler::sample) with
 * GenerationConfig's sampling fields (config.rs:163-174). top_k 0 = off.
 * ------------------------------------------------------------------- */
typedef struct {
    float temperature, top_p, min_p, repetition_penalty, presence_penalty, frequency_penalty;
    uint32_t top_k;
} mivi_sampler_config;

/* Sampler::sample on the device, asynchronous on the stream (the split path
 * of mivi_hip_sample_rows on one row, with a workspace the library keeps per
 * device: the first call on a device allocates it, so do not make that call
 * under graph capture):
 * logits (n floats, device) are modified in place as the reference modifies
 * its &mut [f32] (penalties, temperature, min-p, top-k, then the softmax
 * probabilities); recent (n_recent token ids, device) is the penalty window;
 * rng_state (device u64) is the xorshift64* state, advanced by one draw when
 * the reference draws (seed it with the reference's rule: 0 ->
 * 0x853c49e6748fea9b); token (device u32) receives the sampled id. The draw
 * is bit-exact; cumulative sums are the reference's up to float rounding,
 * and tied top-p probabilities are ordered by index. */
int32_t mivi_hip_sample(float* logits, size_t n, const uint32_t* recent, size_t n_recent,
                        const mivi_sampler_config* cfg, uint64_t* rng_state, uint32_t* token,
                        void* stream);

/* No counterpart in the reference; for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops). The same
 * computation as mivi_hip_sample, bit for bit, with the workspace in a
 * fixed-size device array of the library (513 KB per GPU, held until the
 * process ends) instead of a buffer allocated on the first call: it calls no
 * hipMalloc or hipFree. n at most 262144 logits (larger n returns
 * MIVI_ERR_INVALID_ARGUMENT before anything runs). Every call on a GPU
 * shares that GPU's array, so calls that overlap on one GPU (other streams
 * or threads) race; order them. Asynchronous on the stream. */
int32_t mivi_hip_sample_noalloc(float* logits, size_t n, const uint32_t* recent, size_t n_recent,
                                const mivi_sampler_config* cfg, uint64_t* rng_state, uint32_t* token,
                                void* stream);

/* Sampler::sample (sampler.rs:91-135) on `rows` rows at once, one sampler
 * per row (the per-sequence samplers of a batch): row b's logits at
 * logits + b * row_stride, its penalty window at recent + b * recent_stride
 * (n_recent ids each), its state rng_states[b], its token tokens[b]; the same
 * results as mivi_hip_sample on each row. Spread over the whole device (a
 * chunk kernel over 1024-logit chunks, then one workgroup per row over the
 * chunks' top-k candidates when top_k <= 128; with no top-k and top_p >= 1,
 * softmax kernels per chunk and a pick over the chunks' masses), with
 * `workspace` (device,
 * 8-byte aligned) of at least mivi_hip_sample_rows_workspace(n, rows)
 * bytes, which calls running at once must not share. Asynchronous on the
 * stream. rows <= 65535. */
size_t mivi_hip_sample_rows_workspace(size_t n, size_t rows);
int32_t mivi_hip_sample_rows(float* logits, size_t n, size_t rows, size_t row_stride,
                             const uint32_t* recent, size_t n_recent, size_t recent_stride,
                             const mivi_sampler_config* cfg, uint64_t* rng_states, uint32_t* tokens,
                             void* workspace, size_t workspace_bytes, void* stream);

/* The generation loop of model.rs:1130-1180 on the device for `batch`
 * sequences starting from tokens[b] at pos[b]: n_steps decode steps, each
 * sampling every sequence's next token with Sampler::sample (its penalty
 * window = its last 64 generated tokens, RECENT_TOKENS_WINDOW; seeds[b] per
 * sequence, 0 -> the reference's fallback seed; the eos_ids (at most 4) are
 * suppressed on the first token as the loop does). Stopping at an
 * end-of-sequence token is left to the caller: tokens_out[step * batch + b]
 * holds all n_steps tokens. Errors as mivi_hip_model_generate_greedy. */
int32_t mivi_hip_model_generate(mivi_model* m, size_t batch, const uint32_t* tokens,
                                const size_t* pos, size_t n_steps, const mivi_sampler_config* cfg,
                                const uint64_t* seeds, const uint32_t* eos_ids, size_t n_eos,
                                uint32_t* tokens_out);

/* ---------------------------------------------------------------------
 * Prefix cache: PrefixCache of crates/mivi-kv/src/prefix.rs with its
 * snapshots in device memory. A chunk node holds the KV interval it owns
 * (every attention layer, as the model's cache stores it) and the ShortConv
 * state at its boundary, copied device to device from a model sequence at
 * insert and back at restore; the bookkeeping (chained FNV-1a chunk hashes,
 * parent links of delta chunks, LRU order with the deepest chunk evicted
 * first, chunk count and byte budget) is the reference's. Errors of the
 * reference's KvError::DimMismatch / ContextOverflow are MIVI_ERR_KV_CACHE.
 * With Q8_0 caches the chunk size must be a multiple of 16 (whole groups).
 * ------------------------------------------------------------------- */
typedef struct mivi_prefix_cache mivi_prefix_cache;

/* PrefixCache::with_budget (prefix.rs:148-168); 0 takes the default (1024
 * chunks, 64 tokens, 512 MB). */
int32_t mivi_hip_prefix_cache_create(size_t max_chunks, size_t chunk_size,
                                     size_t max_memory_bytes, mivi_prefix_cache** out);
void mivi_hip_prefix_cache_destroy(mivi_prefix_cache* pc);

/* compute_chunk_hash (prefix.rs:70-87). */
uint64_t mivi_hip_prefix_chunk_hash(uint64_t prev_hash, const uint32_t* tokens, size_t n);

/* insert_delta_chunk (prefix.rs:251-303): chunk chunk_index (n_tokens ==
 * chunk size) of sequence seq of m, which has processed exactly pos =
 * (chunk_index + 1) * chunk_size tokens; chunk_index > 0 needs its parent
 * prev_hash cached at the previous boundary. *hash_out = the chunk's hash.
 * Synchronous. */
int32_t mivi_hip_prefix_cache_insert_delta(mivi_prefix_cache* pc, mivi_model* m, size_t seq,
                                           size_t pos, uint64_t prev_hash,
                                           const uint32_t* tokens, size_t n_tokens,
                                           size_t chunk_index, uint64_t* hash_out);

/* insert_chunk (prefix.rs:239-249): a full snapshot, the whole prefix
 * [0, pos) of sequence seq's KV caches and its ShortConv state in one node
 * with no parent (restoring it needs no other chunk); its hash chains the
 * chunk's tokens on prev_hash. Synchronous. */
int32_t mivi_hip_prefix_cache_insert(mivi_prefix_cache* pc, mivi_model* m, size_t seq, size_t pos,
                                     uint64_t prev_hash, const uint32_t* tokens, size_t n_tokens,
                                     size_t chunk_index, uint64_t* hash_out);

/* find_longest_suffix_match (prefix.rs:453-517): the longest suffix of
 * tokens, k whole chunks starting at an absolute position (start_pos + its
 * offset) that is a multiple of the chunk size, whose tokens equal a cached
 * chunk's (by the chunk's standalone hash). *suffix_len = the matched tokens
 * (0 if none), *match_pos = the position the chunk's state was taken at,
 * *hash_out = its hash; touches it in the LRU order. Only the tokens are
 * matched: the caller must check that its state fits the preceding context.
 * Several matching chunks: the lowest hash (the reference's order is that
 * of its hash map). */
int32_t mivi_hip_prefix_cache_find_suffix(mivi_prefix_cache* pc, size_t start_pos, const uint32_t* tokens,
                                          size_t n, size_t* suffix_len, size_t* match_pos,
                                          uint64_t* hash_out);

/* find_longest_prefix (prefix.rs:200-237): tokens matched by the deepest
 * cached chunk (0 if none) and its hash; touches it in the LRU order. */
int32_t mivi_hip_prefix_cache_find(mivi_prefix_cache* pc, const uint32_t* tokens, size_t n,
                                   size_t* matched, uint64_t* hash_out);

/* restore_longest_prefix (prefix.rs:305-358): the matched chain's KV
 * intervals into sequence seq's caches and the deepest node's ShortConv
 * state into the sequence; *matched = 0 when nothing matches. The caller
 * continues (prefill) from position *matched. Synchronous. */
int32_t mivi_hip_prefix_cache_restore(mivi_prefix_cache* pc, mivi_model* m, size_t seq,
                                      const uint32_t* tokens, size_t n, size_t* matched,
                                      uint64_t* hash_out);

/* len, memory_usage_bytes, prune_to_bytes, clear (prefix.rs:179-196,
 * 395-423); contains: whether a chunk of that hash is cached. */
size_t mivi_hip_prefix_cache_len(const mivi_prefix_cache* pc);
size_t mivi_hip_prefix_cache_memory_bytes(const mivi_prefix_cache* pc);
size_t mivi_hip_prefix_cache_prune(mivi_prefix_cache* pc, size_t target_bytes);
void mivi_hip_prefix_cache_clear(mivi_prefix_cache* pc);
int32_t mivi_hip_prefix_cache_contains(const mivi_prefix_cache* pc, uint64_t hash);

/* ---------------------------------------------------------------------
 * Measurement (no counterpart in the reference): reads `bytes` bytes at p
 * (16-byte aligned, bytes % 16 == 0) once with plain coalesced 16-byte loads
 * on the stream and discards them. Its time is the floor for any kernel that
 * reads the same bytes, against which the benchmark reports the GEMVs.
 * ------------------------------------------------------------------- */
int32_t mivi_hip_read_floor(const uint8_t* p, size_t bytes, void* stream);

/* ---------------------------------------------------------------------
 * Synthetic inputs (no counterpart in the reference, which ships no K-quant
 * quantizer): seeded SplitMix64 + Box-Muller normals and f32 -> Q4_K / Q6_K /
 * Q8_0 encoders, host side, multithreaded. Used to build test and benchmark
 * inputs; parity is always defined on the packed bytes they produce.
 * ------------------------------------------------------------------- */
/* n normals N(mean, std) from stream `seed` into out (host) */
void mivi_synth_normal(uint64_t seed, float mean, float std, float* out, size_t n);
/* rows x cols f32 (host) -> packed blocks (host); cols % block == 0 */
int32_t mivi_synth_quantize(int32_t ggml_type, const float* src, size_t rows, size_t cols,
                            uint8_t* dst, size_t dst_len);
/* seeded N(0, std) weights directly into packed blocks (host) */
int32_t mivi_synth_random_weights(int32_t ggml_type, uint64_t seed, float std, size_t rows,
                                  size_t cols, uint8_t* dst, size_t dst_len);

#ifdef __cplusplus
}
#endif
#endif
