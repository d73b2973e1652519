// Shared device helpers and host error plumbing for the mivi-hip library.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>

#include "../../include/mivi_hip.h"

// ---------------------------------------------------------------- host side
namespace mivi {

// Records the details of a failing call in a thread-local slot and returns
// its code (read back through mivi_hip_last_error).
int32_t set_error(int32_t code, const char* fmt, ...);
int32_t err_buffer_too_small(size_t expected, size_t actual);
int32_t err_misaligned(size_t dim, size_t block_size);
int32_t err_unsupported(int32_t type_id);
int32_t err_overflow();
int32_t clear_error();

#define MIVI_HIP_CHECK(expr)                                                          \
    do {                                                                              \
        hipError_t e_ = (expr);                                                       \
        if (e_ != hipSuccess)                                                         \
            return ::mivi::set_error(MIVI_ERR_HIP, "%s failed: %s", #expr,            \
                                     hipGetErrorString(e_));                          \
    } while (0)

// Integer tuning knob from the environment (dflt when unset or empty).
inline int env_knob(const char* name, int dflt) {
    const char* v = getenv(name);
    return v && *v ? atoi(v) : dflt;
}

inline int num_cus() {
    static int n = 0;
    if (n == 0) {
        int dev = 0;
        hipGetDevice(&dev);
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = 256;
    }
    return n;
}

}  // namespace mivi

// -------------------------------------------------------------- device side
typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float half_bits_to_f32(uint32_t bits) {
    // exact widening (v_cvt_f32_f16)
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(bits & 0xFFFFu));
}

// silu(g) = g / (1 + exp(-g)), 0 for g <= -50 (math.rs:76-82)
__device__ __forceinline__ float silu_f(float g) { return g <= -50.0f ? 0.0f : g / (1.0f + expf(-g)); }

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits) {
    return __uint_as_float((bits & 0xFFFFu) << 16);
}

__device__ __forceinline__ uint32_t f32_to_half_bits(float f) {
    // round to nearest even (v_cvt_f16_f32 under the default rounding mode)
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);
}

__device__ __forceinline__ uint32_t ld_u16(const uint8_t* p) {
    return (uint32_t)*(const uint16_t*)p;
}

// 16 bytes starting at a 2-byte aligned address. Never touches memory past
// p + 16: reads [p - 2, p + 16) when p is 2 mod 4 (aligned dwords plus a
// 16-bit tail) and [p, p + 16) otherwise.
__device__ __forceinline__ u32x4 ld16_a2(const uint8_t* p) {
    const uintptr_t a = (uintptr_t)p;
    const uint32_t* base = (const uint32_t*)(a & ~(uintptr_t)3);
    const uint32_t sh = (uint32_t)(a & 3);
    u32x4_a4 v = *(const u32x4_a4*)base;
    const uint32_t tail16 = (uint32_t)*(const uint16_t*)(p + 14);
    const uint32_t e = sh ? tail16 : v.w;
    u32x4 r;
    r.x = __builtin_amdgcn_alignbyte(v.y, v.x, sh);
    r.y = __builtin_amdgcn_alignbyte(v.z, v.y, sh);
    r.z = __builtin_amdgcn_alignbyte(v.w, v.z, sh);
    r.w = __builtin_amdgcn_alignbyte(e, v.w, sh);
    return r;
}

__device__ __forceinline__ float ubyte_f32(uint32_t w, int k) {
    return (float)((w >> (8 * k)) & 0xFFu);
}

// byte k of w as a signed value (v_cvt_f32_i32 of the sign-extended byte)
__device__ __forceinline__ float sbyte_f32(uint32_t w, int k) {
    return (float)(int)(int8_t)(w >> (8 * k));
}

// Sum over groups of `width` consecutive lanes (width a power of two <= 64).
template <int WIDTH>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int s = WIDTH / 2; s >= 1; s >>= 1) v += __shfl_xor(v, s, 64);
    return v;
}

__device__ __forceinline__ float wave_sum(float v) { return group_sum<64>(v); }

// Cross-lane moves without LDS: DPP within rows of 16 lanes and the gfx950
// half/row swaps. CTRL is a full permutation (quad_perm, row_ror), so every
// lane reads a valid source; bound_ctrl set lets the compiler fold the move
// into the instruction that consumes it (v_add_f32_dpp and the like).
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    static_assert((CTRL & ~0xFF) == 0 || (CTRL >= 0x121 && CTRL <= 0x12F), "quad_perm or row_ror only");
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, true));
}
// (value of this lane, value of lane ^ 32) as (lower half's, upper half's)
__device__ __forceinline__ void swap32(float v, float& lo, float& hi) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    lo = __uint_as_float(p[0]);
    hi = __uint_as_float(p[1]);
}
// (value of this lane, value of lane ^ 16) as (even row's, odd row's)
__device__ __forceinline__ void swap16(float v, float& ev, float& od) {
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    ev = __uint_as_float(p[0]);
    od = __uint_as_float(p[1]);
}

// The butterfly of group_sum<W> (v += value of lane ^ o for o = W/2 .. 1, in
// that order) without LDS traffic. The xor-4 step reads lane (i + 4) mod 16,
// so the result is group_sum<W>'s bit for bit in the lanes with bit 2 clear
// (lanes 0-3, 8-11, ... of each group), the lanes that use it here; the
// other steps pair exactly (IEEE addition is commutative).
// The same butterfly (v + value of lane ^ o, o = 32 .. 1) exact in every
// lane: the xor-4 partner is lane (i + 4) mod 16 where bit 2 is clear and
// (i - 4) mod 16 where it is set.
__device__ __forceinline__ float xor4_mov(float v) {
    const float up = dpp_mov<0x12C>(v), dn = dpp_mov<0x124>(v);  // row_ror:12, row_ror:4
    return (threadIdx.x & 4) ? dn : up;
}
__device__ __forceinline__ float xsum_all64(float v) {
    float a, b;
    swap32(v, a, b);
    v = a + b;
    swap16(v, a, b);
    v = a + b;
    v += dpp_mov<0x128>(v);
    v += xor4_mov(v);
    v += dpp_mov<0x4E>(v);
    v += dpp_mov<0xB1>(v);
    return v;
}

template <int W>
__device__ __forceinline__ float xsum_desc(float v) {
    static_assert(W >= 8 && W <= 64, "groups of 8 to 64 lanes");
    float a, b;
    if constexpr (W >= 64) { swap32(v, a, b); v = a + b; }
    if constexpr (W >= 32) { swap16(v, a, b); v = a + b; }
    if constexpr (W >= 16) v += dpp_mov<0x128>(v);  // row_ror:8   (lane ^ 8)
    v += dpp_mov<0x12C>(v);                          // row_ror:12  (lane ^ 4 where bit 2 is clear)
    v += dpp_mov<0x4E>(v);                           // quad_perm [2,3,0,1] (lane ^ 2)
    v += dpp_mov<0xB1>(v);                           // quad_perm [1,0,3,2] (lane ^ 1)
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) v = fmaxf(v, __shfl_xor(v, s, 64));
    return v;
}
