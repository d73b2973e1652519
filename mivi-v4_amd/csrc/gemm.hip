// quantized_matmul_rows (crates/mivi-quant/src/lib.rs:143-357) for gfx950.
//
// batch == 1 is exactly the matvec path (lib.rs:171-182). Small batches run
// the GEMV kernels once per input row; the weight rows stay hot in L2/MALL
// across the launches.
#include "common.h"

namespace mivi {
int32_t launch_gemv(int32_t t, const uint8_t* W, const float* x, float* y, size_t n, size_t d, bool accumulate,
                    hipStream_t s);
bool format_sizes(int32_t t, size_t* bs, size_t* ts);
bool ggml_sizes(int32_t t, size_t* bs, size_t* ts);
}  // namespace mivi

using namespace mivi;

// types.rs:188-235 validate_matmul_args after lib.rs:152-166
static int32_t validate_matmul(int32_t t, size_t out_len, size_t w_len, size_t in_len, size_t batch, size_t rows,
                               size_t cols) {
    size_t bs, ts, row_bytes, e;
    if (!ggml_sizes(t, &bs, &ts)) return err_unsupported(t);
    if (cols % bs != 0) return err_misaligned(cols, bs);
    if (__builtin_mul_overflow(cols / bs, ts, &row_bytes)) return err_overflow();
    if (__builtin_mul_overflow(batch, rows, &e)) return err_overflow();
    if (out_len < e) return err_buffer_too_small(e, out_len);
    if (__builtin_mul_overflow(batch, cols, &e)) return err_overflow();
    if (in_len < e) return err_buffer_too_small(e, in_len);
    if (__builtin_mul_overflow(rows, row_bytes, &e)) return err_overflow();
    if (w_len < e) return err_buffer_too_small(e, w_len);
    return MIVI_OK;
}

extern "C" int32_t mivi_hip_quantized_matmul_rows(float* out, size_t out_len, int32_t t, const uint8_t* w,
                                                  size_t w_len, const float* in, size_t in_len, size_t batch,
                                                  size_t rows, size_t cols, void* stream) {
    int32_t rc = validate_matmul(t, out_len, w_len, in_len, batch, rows, cols);
    if (rc) return rc;
    size_t bs, ts;
    // lib.rs:173-182 (matvec) and :273-277 (dequantize_slice) both reject
    // formats outside the supported set before writing anything.
    if (batch > 0 && rows > 0 && !format_sizes(t, &bs, &ts)) return err_unsupported(t);
    if (batch == 0 || rows == 0) return clear_error();
    if (!out || !w || !in) return set_error(MIVI_ERR_INVALID_ARGUMENT, "null buffer");
    clear_error();
    hipStream_t s = (hipStream_t)stream;
    for (size_t b = 0; b < batch; b++) {
        rc = launch_gemv(t, w, in + b * cols, out + b * rows, rows, cols, false, s);
        if (rc) return rc;
    }
    return MIVI_OK;
}
