// Arguments of the dequant-fused GEMV launcher shared by the C ABI and the
// decode step.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/mivi_hip.h"
#include "common.h"

namespace mivi {

// How a workgroup forms the activation vector it stages in LDS.
enum GemvPrologue : int {
    PRO_NONE = 0,     // x as given
    PRO_RMSNORM = 1,  // (x * 1/sqrt(mean(x^2)+eps)) * w        (norm.rs:38-72)
    PRO_SWIGLU = 2,   // silu(x) * x2                          (math.rs:76-100)
    PRO_CONV = 3,     // ShortConv gate over in_proj = [B|C|X] (ssm.rs:80-140)
};

struct GemvSeg {
    const uint8_t* W;  // rows of this segment
    float* y;          // outputs of this segment
    int n;             // rows
    // Q4_K: the same rows in the row products' operand layout
    // (launch_pack_q4k_gemm), read by the matrix-core row products, else null
    const uint8_t* wg;
};

// y_s[r] (=|+=) W_s[r, :] . prologue(x) for up to three weight matrices that
// share the input (q/k/v, gate/up).
struct GemvArgs {
    GemvSeg seg[3];
    int nseg;
    int K;                 // columns (multiple of the block size)
    const float* x;        // input (dim K; for PRO_CONV the 3K in_proj output)
    const float* x2;       // PRO_SWIGLU: up
    const float* norm_w;   // PRO_RMSNORM: weight
    float eps;
    const float* conv_w;   // PRO_CONV: [K * ksize] weights (or shared [ksize])
    int conv_mode;         // 0 full per-channel, 1 shared, 2 default 1/ksize
    int ksize;
    const float* st_in;    // PRO_CONV: previous state [K * ksize]
    float* st_out;         // PRO_CONV: next state, written by workgroup 0
    const int* phase;      // PRO_CONV: if set, st_in/st_out swap when *phase is odd
    int accumulate;        // 1: y += result (residual add, vec_add of ffn.rs:106)
    int epilogue;          // GemvEpilogue
    int packed;            // 1: Q6_K rows in the unit-plane layout of mivi_hip_pack_weights
    float* part_val;       // EPI_ARGMAX: per-wave maximum ...
    int* part_idx;         // ... and the first row holding it
    // Batched columns: ncol > 1 activation vectors (one per sequence) against
    // the same rows. Column c reads x + c*xs (x2 + c*xs; st_in / st_out +
    // c*sts; phase + c) and writes every segment's outputs at + c*ys (the
    // argmax partials at + c*ps). ncol 0 or 1: one column.
    int ncol;
    int64_t xs, sts, ys, ps;
    // Batched Q4_K columns (the column kernels): the launch's rows packed by
    // launch_pack_q4k_cols in the kernel's group order, else null (GGUF rows)
    const uint8_t* cw;
};

// Most columns one batched streaming launch takes (more are split into
// launches of at most this many; fewer at K = 8192 and on packed rows).
constexpr int kMaxGemvCols = 8;

// What the GEMV does with its row results (streaming kernel, K = 2048).
enum GemvEpilogue : int {
    EPI_STORE = 0,    // y (=|+=) result
    EPI_SWIGLU = 1,   // two segments gate|up of n rows each: y_gate[i] = silu(gate_i) * up_i (ffn.rs:84-95)
    EPI_ARGMAX = 2,   // store, and each wave's (max, first row) into part_val/part_idx
    EPI_CONV = 3,     // one segment [B|C|X] of 3D rows (the ShortConv in_proj): the gated conv of
                      // ssm.rs:80-140 per channel into y[0..D) (C * conv(window, B * X)), the next
                      // window into st_out (conv fields and ncol strides as for PRO_CONV)
};

// Number of per-wave argmax partials an EPI_ARGMAX launch of this shape
// writes (0 when the shape cannot take the epilogue); packed: the rows are in
// the layout of launch_pack_q6k.
int gemv_argmax_parts(int32_t ggml_type, int K, int n, bool packed = false);

// Packed Q6_K matrices of K = 2048 columns and a multiple of 4 rows use the
// row-quad layout (matrix-core GEMV); other packed shapes the unit-plane one.
inline bool quad_layout(size_t rows, size_t cols) { return cols == 2048 && rows % 4 == 0; }

// Workgroups of a row-quad GEMV over n rows.
int quad_grid(int n);

// Workgroups per CU of a streaming GEMV over n rows (all segments).
int stream_wg_per_cu(int n);

int32_t launch_gemv_ex(int32_t ggml_type, int prologue, const GemvArgs& a, hipStream_t s);

// Row-batch product: the a.ncol activation rows (row m at a.x + m * a.xs,
// after the prologue) against each segment's weight rows, output row m of
// segment s at a.seg[s].y + m * a.ys (=|+= with a.accumulate). Q4_K with at
// least 16 rows and K % 2048 == 0 runs on the matrix cores (fp16 hi/lo
// activations), anything else as a batched GEMV. No conv prologue, store
// epilogue only.
int32_t launch_rows(int32_t ggml_type, int prologue, const GemvArgs& a, hipStream_t s);

// rows x cols Q6_K (cols 2048/4096/8192) into the packed layout: row quads
// when quad_layout(rows, cols), unit planes otherwise
int32_t launch_pack_q6k(const uint8_t* src, uint8_t* dst, size_t rows, size_t cols, hipStream_t s);

// rows x cols Q4_K (cols 2048 or 8192, rows a multiple of 4) into row quads,
// the layout of the matrix-core GEMV for one column (packed = 1): bit-identical
// results to the streaming kernel on the GGUF rows
inline bool q4k_quad_layout(size_t rows, size_t cols) { return (cols == 2048 || cols == 8192) && rows % 4 == 0; }
int32_t launch_pack_q4k(const uint8_t* src, uint8_t* dst, size_t rows, size_t cols, hipStream_t s);

// The batched Q4_K column kernel takes 16-row groups: lane row j of group grp
// is row cols_group_row(...) of the launch's concatenated segments (n rows,
// n0 in the first), or -1 (none; its lanes then read row 0 and store
// nothing). EPI_SWIGLU groups: gate rows 8 grp .. 8 grp + 7, then the same up
// rows; EPI_CONV groups: channels 5 grp .. 5 grp + 4 of the D = n0 / 3, each
// as its B, C, X rows (j = 3i + k; row 15 repeats row 14); other epilogues:
// rows 16 grp .. 16 grp + 15.
__host__ __device__ inline int cols_group_row(int epi, int grp, int j, int n0, int n) {
    if (epi == EPI_SWIGLU) {
        const int c = 8 * grp + (j & 7);
        return c < n0 ? c + (j >> 3) * n0 : -1;
    }
    if (epi == EPI_CONV) {
        const int D3 = n0 / 3, jj = j < 15 ? j : 14, c = 5 * grp + jj / 3;
        return c < D3 ? c + (jj % 3) * D3 : -1;
    }
    const int r = 16 * grp + j;
    return r < n ? r : -1;
}
__host__ __device__ inline int cols_groups(int epi, int n0, int n) {
    return epi == EPI_SWIGLU ? (n0 + 7) / 8 : epi == EPI_CONV ? (n0 / 3 + 4) / 5 : (n + 15) / 16;
}

// Q4_K rows in the column kernel's order (launch_pack_q4k_cols): per group,
// per superblock s of the row (cols / 256 of them), kColsChunkBytes:
//   [0, 256)      the 16 rows' headers, 16 bytes at 16 j: d | dmin << 16
//                 (fp16), the sub-block scales sc0..sc7 and the mins
//                 m0..m3 as bytes (get_scale_min_k4 decoded, q4_k_m.rs:11-58)
//   [256, 320)    the mins m4..m7 of row j, 4 bytes at 256 + 4 j
//   [320, 2368)   the code bytes as two 1 KB halves, lane l = j + 16 kg
//                 holding in each 16 bytes of row j: codes [32 g + 8 kg, + 8)
//                 for g = 0, 1 (first half) and g = 2, 3 (second), the bytes
//                 of its two B operands per 64-value unit.
// Every load of the kernel is then one contiguous 256 B, 64 B or 1 KB (the
// GGUF rows give it 16 rows x 32 bytes per load instruction, bound by the
// L1's cache-line rate), and no scale needs unpacking beyond a byte select.
// rows_host[16 grp + j]: the device address of group grp's row j (any valid
// row where the group has none there).
constexpr int kColsMinsOff = 256;
constexpr int kColsCodesOff = 320;
constexpr int kColsChunkBytes = kColsCodesOff + 2048;

// rows x cols Q4_K (rows % 32 == 0, cols % 256 == 0) into the operand layout
// of the matrix-core row products (launch_rows with GemvSeg::wg): the fp16
// values sc * q in MFMA B-operand order, then d, dmin and the sub-block mins
// per row and super-block; q4k_gemm_packed_bytes(rows, cols) bytes
inline size_t q4k_gemm_packed_bytes(size_t rows, size_t cols) {
    return rows * cols * 2 + rows / 32 * (cols / 256) * 640;
}
int32_t launch_pack_q4k_gemm(const uint8_t* src, uint8_t* dst, size_t rows, size_t cols, hipStream_t s);
// Q6_K in 32-row tiles (K = 2048, rows % 32 == 0), the batched head's copy:
// each superblock of 32 rows laid out as the B operand of the 32 x 32 x 16
// int8 matrix instruction, the size of the GGUF rows (launch_pack_q6k_t32).
// launch_gemv_t32 runs ncol columns over it, eight per launch (one segment,
// no or RMSNorm prologue, store or argmax epilogue; x 16-byte aligned, xs %
// 4 == 0), every column's result equal to the one-column packed kernel's bit
// for bit; an argmax launch writes t32_argmax_parts(n) partials per column.
inline bool t32_layout(size_t rows, size_t cols) { return cols == 2048 && rows > 0 && rows % 32 == 0; }
int32_t launch_pack_q6k_t32(const uint8_t* src, uint8_t* dst, size_t rows, size_t cols, hipStream_t s);
int32_t launch_gemv_t32(int pro, const GemvArgs& a, hipStream_t s);
int t32_argmax_parts(int n);
int32_t launch_pack_q4k_cols(const uint8_t* const* rows_host, int ngroups, size_t cols, uint8_t* dst,
                             hipStream_t s);

// Row `id` of an embedding table (model.rs:358-375, the token's row
// dequantized: Q6_K, Q4_K, Q8_0, F16, BF16 or F32) into x, by threads
// t0, t0 + nt, ... of the caller.
__device__ __forceinline__ void embed_row(int32_t type, const uint8_t* table, size_t row_bytes, uint32_t id, float* x,
                                          int dim, int t0, int nt) {
    const uint8_t* row = table + (size_t)id * row_bytes;
    for (int i = t0; i < dim; i += nt) {
        float y = 0.f;
        if (type == MIVI_GGML_Q6_K) {
            const uint8_t* blk = row + (size_t)(i / 256) * 210;
            int e = i % 256, half = e / 128, r = e % 128, grp = r / 32, l = r % 32;
            const uint8_t* ql = blk + half * 64;
            const uint8_t* qh = blk + 128 + half * 32;
            const int8_t* sc = (const int8_t*)(blk + 192 + half * 8);
            float d = half_bits_to_f32(ld_u16(blk + 208));
            int lo = (grp & 1) ? ql[l + 32] : ql[l];
            int nib = grp < 2 ? (lo & 0xF) : (lo >> 4);
            int q = (nib | (((qh[l] >> (2 * grp)) & 3) << 4)) - 32;
            y = d * (float)sc[l / 16 + 2 * grp] * (float)q;
        } else if (type == MIVI_GGML_Q4_K) {
            const uint8_t* blk = row + (size_t)(i / 256) * 144;
            int e = i % 256, j = e / 64, r = e % 64, hi = r / 32, l = r % 32;
            float d = half_bits_to_f32(ld_u16(blk)), dmin = half_bits_to_f32(ld_u16(blk + 2));
            const uint8_t* sc = blk + 4;
            int jj = 2 * j + hi;
            uint32_t s, m;
            if (jj < 4) { s = sc[jj] & 63; m = sc[jj + 4] & 63; }
            else { s = (sc[jj + 4] & 0xF) | ((sc[jj - 4] >> 6) << 4); m = (sc[jj + 4] >> 4) | ((sc[jj] >> 6) << 4); }
            uint32_t qb = blk[16 + j * 32 + l];
            float dd = d * (float)s, mm = dmin * (float)m;
            y = dd * (float)(hi ? (qb >> 4) : (qb & 0xF)) - mm;
        } else if (type == MIVI_GGML_Q8_0) {
            const uint8_t* blk = row + (size_t)(i / 32) * 34;
            y = (float)(int8_t)blk[2 + i % 32] * half_bits_to_f32(ld_u16(blk));
        } else if (type == MIVI_GGML_F16) {
            y = half_bits_to_f32(ld_u16(row + 2 * (size_t)i));
        } else if (type == MIVI_GGML_BF16) {
            y = bf16_bits_to_f32(ld_u16(row + 2 * (size_t)i));
        } else {
            const uint8_t* p = row + 4 * (size_t)i;
            y = __uint_as_float(p[0] | (p[1] << 8) | (p[2] << 16) | ((uint32_t)p[3] << 24));
        }
        x[i] = y;
    }
}

// EmbedNext: with a table, the chosen token's embedding row goes to x (+ b *
// xs) for the next step, so the step needs no embedding launch of its own.
struct EmbedNext {
    const uint8_t* table;
    size_t row_bytes;
    float* x;
    int64_t xs;
    int32_t type;
    int dim;
};

// End-of-sequence ids suppressed on a generation's first token.
struct SampleEos {
    uint32_t id[4];
    int n;
};

// Sampler::sample for sequences seq0 .. seq0 + batch - 1 of a decode step
// (logits of sequence b at logits + b * lstride), penalty window = the last
// `window` tokens of history[step * hstride + seq]; writes tok[b] and the
// history at *step. rng: one xorshift64* state per sequence (rng[b]). ws:
// sample_seq_workspace(n, batch) bytes of device memory (8-byte aligned);
// the logits are left as the reference's sample() leaves its slice (the
// probabilities, or the penalised logits divided by the temperature on the
// greedy path).
// en: the sampled tokens' embeddings for the next step (EmbedNext).
size_t sample_seq_workspace(size_t n, size_t batch);
int32_t launch_sample_seq(float* logits, int64_t lstride, int n, uint32_t* history, int hstride, int seq0, int batch,
                          int window, const int* step, const SampleEos& eos, const mivi_sampler_config& cfg,
                          uint64_t* rng, uint32_t* tok, void* ws, const EmbedNext& en, hipStream_t s);

}  // namespace mivi
