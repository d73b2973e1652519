// Thread-local error details for the C ABI (the QuantError / ModelError
// payloads of crates/mivi-quant/src/types.rs:5-15 and
// crates/mivi-model/src/model.rs:25-49, with their Display texts).
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "common.h"

namespace mivi {

static thread_local mivi_error g_err;

int32_t set_error(int32_t code, const char* fmt, ...) {
    memset(&g_err, 0, sizeof(g_err));
    g_err.code = code;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err.message, sizeof(g_err.message), fmt, ap);
    va_end(ap);
    return code;
}

int32_t err_buffer_too_small(size_t expected, size_t actual) {
    set_error(MIVI_ERR_BUFFER_TOO_SMALL, "Buffer too small: expected at least %zu bytes, got %zu",
              expected, actual);
    g_err.expected = expected;
    g_err.actual = actual;
    return MIVI_ERR_BUFFER_TOO_SMALL;
}

int32_t err_misaligned(size_t dim, size_t block_size) {
    set_error(MIVI_ERR_DIMENSION_MISALIGNED, "Dimension not a multiple of block size %zu: %zu",
              block_size, dim);
    g_err.dim = dim;
    g_err.block_size = block_size;
    return MIVI_ERR_DIMENSION_MISALIGNED;
}

int32_t err_unsupported(int32_t type_id) {
    set_error(MIVI_ERR_UNSUPPORTED_TYPE, "Unsupported GGML quantization type: %u", (uint32_t)type_id);
    g_err.type_id = (uint32_t)type_id;
    return MIVI_ERR_UNSUPPORTED_TYPE;
}

int32_t err_overflow() {
    return set_error(MIVI_ERR_ARITHMETIC_OVERFLOW, "Arithmetic overflow in quantization operation");
}

int32_t clear_error() {
    memset(&g_err, 0, sizeof(g_err));
    return MIVI_OK;
}

}  // namespace mivi

extern "C" int32_t mivi_hip_last_error(mivi_error* out) {
    if (out) *out = mivi::g_err;
    return mivi::g_err.code;
}

extern "C" const char* mivi_hip_version(void) { return "mivi-hip 0.1.0 (gfx950)"; }
