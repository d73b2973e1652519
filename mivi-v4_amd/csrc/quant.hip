// K-quant dequantization and dequant-fused GEMV kernels for gfx950, plus the
// C-ABI entry points that mirror crates/mivi-quant's public functions.
//
// Layout of the packed formats (identical bytes to the reference):
//   Q4_K  144 B / 256 values: f16 d | f16 dmin | 12 B 6-bit scales+mins | 128 B nibbles
//         (crates/mivi-quant/src/q4_k_m.rs:11-58)
//   Q6_K  210 B / 256 values: 128 B ql | 64 B qh | 16 x i8 scales | f16 d
//         (crates/mivi-quant/src/q6_k.rs:8-38)
//   Q8_0   34 B /  32 values: f16 d | 32 x i8 (crates/mivi-quant/src/q8_0.rs:11-22)
//
// GEMV design (one weight row = nb superblocks): a wave owns a tile of rows
// and streams it with 16-byte loads; each lane owns one "unit" of a
// superblock (a quarter: 64 values) and keeps it for U rows at once, so the
// activation slice it reads from LDS is reused U times. Partial row sums are
// reduced across the LPR lanes that share a row. Activations are staged once
// per workgroup in LDS together with per-sub-block sums (the min term of
// Q4_K and the -32 offset of Q6_K need sum(x) per sub-block).
#include <stdlib.h>

#include <algorithm>
#include <type_traits>

#include "common.h"
#include "gemv.h"

namespace {

constexpr int kWG = 256;
constexpr size_t kMaxLdsK = 12288;  // x in LDS up to this many columns

// ------------------------------------------------------------------ dequant

// q4_k_m.rs:24-58. One thread per (block, j, l): two outputs. The products
// and the subtraction are separate roundings, like the reference.
__global__ void __launch_bounds__(kWG) dequant_q4k_kernel(const uint8_t* __restrict__ src,
                                                          float* __restrict__ out, size_t nblocks) {
    size_t t = (size_t)blockIdx.x * kWG + threadIdx.x;
    size_t b = t >> 7;
    if (b >= nblocks) return;
    int r = (int)(t & 127), j = r >> 5, l = r & 31;
    const uint8_t* blk = src + b * 144;
    float d = half_bits_to_f32(ld_u16(blk)), dmin = half_bits_to_f32(ld_u16(blk + 2));
    const uint8_t* sc = blk + 4;
    int j0 = 2 * j, j1 = 2 * j + 1;
    uint32_t s0, m0, s1, m1;
    if (j0 < 4) {
        s0 = sc[j0] & 63; m0 = sc[j0 + 4] & 63;
    } else {
        s0 = (sc[j0 + 4] & 0xF) | ((sc[j0 - 4] >> 6) << 4);
        m0 = (sc[j0 + 4] >> 4) | ((sc[j0] >> 6) << 4);
    }
    if (j1 < 4) {
        s1 = sc[j1] & 63; m1 = sc[j1 + 4] & 63;
    } else {
        s1 = (sc[j1 + 4] & 0xF) | ((sc[j1 - 4] >> 6) << 4);
        m1 = (sc[j1 + 4] >> 4) | ((sc[j1] >> 6) << 4);
    }
    float d1 = d * (float)s0, mv1 = dmin * (float)m0;
    float d2 = d * (float)s1, mv2 = dmin * (float)m1;
    uint32_t q = blk[16 + j * 32 + l];
    float* o = out + b * 256 + j * 64;
    o[l] = d1 * (float)(q & 0xF) - mv1;
    o[l + 32] = d2 * (float)(q >> 4) - mv2;
}

// q6_k.rs:8-38. One thread per (block, half, l): four outputs, y = (d*sc)*q.
__global__ void __launch_bounds__(kWG) dequant_q6k_kernel(const uint8_t* __restrict__ src,
                                                          float* __restrict__ out, size_t nblocks) {
    size_t t = (size_t)blockIdx.x * kWG + threadIdx.x;
    size_t b = t >> 6;
    if (b >= nblocks) return;
    int r = (int)(t & 63), half = r >> 5, l = r & 31;
    const uint8_t* blk = src + b * 210;
    const uint8_t* ql = blk + half * 64;
    const uint8_t* qh = blk + 128 + half * 32;
    const int8_t* sc = (const int8_t*)(blk + 192 + half * 8);
    float d = half_bits_to_f32(ld_u16(blk + 208));
    int is = l / 16;
    int q1 = (int)((ql[l] & 0xF) | ((qh[l] & 3) << 4)) - 32;
    int q2 = (int)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
    int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
    int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
    float* y = out + b * 256 + half * 128;
    y[l] = d * (float)sc[is] * (float)q1;
    y[l + 32] = d * (float)sc[is + 2] * (float)q2;
    y[l + 64] = d * (float)sc[is + 4] * (float)q3;
    y[l + 96] = d * (float)sc[is + 6] * (float)q4;
}

// q8_0.rs:11-22
__global__ void __launch_bounds__(kWG) dequant_q80_kernel(const uint8_t* __restrict__ src,
                                                          float* __restrict__ out, size_t nblocks) {
    size_t t = (size_t)blockIdx.x * kWG + threadIdx.x;
    size_t b = t >> 5;
    if (b >= nblocks) return;
    int i = (int)(t & 31);
    const uint8_t* blk = src + b * 34;
    float d = half_bits_to_f32(ld_u16(blk));
    out[b * 32 + i] = (float)(int8_t)blk[2 + i] * d;
}

// f16.rs:24-39 and lib.rs:57-69: element-wise widening (kind 0 f16, 1 bf16, 2 f32)
__global__ void __launch_bounds__(kWG) dequant_dense_kernel(const uint8_t* __restrict__ src,
                                                            float* __restrict__ out, size_t n, int kind) {
    size_t i = (size_t)blockIdx.x * kWG + threadIdx.x;
    if (i >= n) return;
    if (kind == 0) out[i] = half_bits_to_f32(src[2 * i] | (src[2 * i + 1] << 8));
    else if (kind == 1) out[i] = bf16_bits_to_f32(src[2 * i] | (src[2 * i + 1] << 8));
    else out[i] = __uint_as_float(src[4 * i] | (src[4 * i + 1] << 8) | (src[4 * i + 2] << 16) |
                                  ((uint32_t)src[4 * i + 3] << 24));
}

// -------------------------------------------------------------- x staging

// Workgroup-wide sum (all threads get the result). `red` holds >= 4 floats.
__device__ __forceinline__ float block_sum(float v, float* red) {
    v = wave_sum(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < kWG / 64; i++) s += red[i];
    __syncthreads();
    return s;
}

// Forms the activation vector for this GEMV in LDS (K floats) followed by
// per-`G`-value sums taken sequentially in element order (G = 0: none).
template <int PRO, int G>
__device__ __forceinline__ void stage_input(float* lds, const mivi::GemvArgs& a) {
    const int K = a.K;
    __shared__ float red[kWG / 64];
    if (PRO == mivi::PRO_NONE) {
        if ((K & 3) == 0 && ((uintptr_t)a.x & 15) == 0) {
            for (int i = threadIdx.x; i < K / 4; i += kWG) *(f32x4*)(lds + 4 * i) = *(const f32x4*)(a.x + 4 * i);
        } else {
            for (int i = threadIdx.x; i < K; i += kWG) lds[i] = a.x[i];
        }
    } else if (PRO == mivi::PRO_RMSNORM) {
        float ss = 0.f;
        for (int i = threadIdx.x; i < K; i += kWG) {
            float v = a.x[i];
            lds[i] = v;
            ss = fmaf(v, v, ss);
        }
        ss = block_sum(ss, red);
        const float scale = 1.0f / sqrtf(ss / (float)K + a.eps);
        for (int i = threadIdx.x; i < K; i += kWG) lds[i] = lds[i] * scale * a.norm_w[i];
    } else if (PRO == mivi::PRO_SWIGLU) {
        for (int i = threadIdx.x; i < K; i += kWG) lds[i] = silu_f(a.x[i]) * a.x2[i];
    } else {  // PRO_CONV, ssm.rs:80-140: bx = B*X; shift state; conv; gate by C
        const float* Bv = a.x;
        const float* Cv = a.x + K;
        const float* Xv = a.x + 2 * K;
        const int ks = a.ksize;
        const bool writer = blockIdx.x == 0;
        const bool swap = a.phase && ((*a.phase) & 1);
        const float* st_in = swap ? a.st_out : a.st_in;
        float* st_out = swap ? (float*)a.st_in : a.st_out;
        for (int d = threadIdx.x; d < K; d += kWG) {
            const float bx = Bv[d] * Xv[d];
            const float* old = st_in + (size_t)d * ks;
            float conv = 0.0f;
            for (int k = 0; k < ks; k++) {
                const float sv = k + 1 < ks ? old[k + 1] : bx;
                const float wv = a.conv_mode == 0 ? a.conv_w[(size_t)d * ks + k]
                               : a.conv_mode == 1 ? a.conv_w[k] : 1.0f / (float)ks;
                conv += wv * sv;
                if (writer) st_out[(size_t)d * ks + k] = sv;
            }
            lds[d] = Cv[d] * conv;
        }
    }
    __syncthreads();
    if (G > 0) {
        float* sums = lds + K;
        for (int i = threadIdx.x; i < K / G; i += kWG) {
            float s = 0.0f;
#pragma unroll
            for (int k = 0; k < G; k++) s += lds[G * i + k];
            sums[i] = s;
        }
        __syncthreads();
    }
}

// Segment table of a GemvArgs held in registers: the kernel-argument struct
// is never indexed dynamically (that would turn every row lookup into a
// dependent load from the kernarg segment).
struct Segs {
    // row r of the concatenated segments lives at
    //   W0 + r * row_bytes + (r >= n0) * dW1 + (r >= n01) * dW2
    // (and its output at y0 + r + ...): no per-row selects that the compiler
    // could turn into an indexed table in scratch memory.
    uintptr_t W0, y0;
    int64_t dW1, dW2, dy1, dy2;
    int n0, n01, n;
    size_t rb;
    __device__ __forceinline__ Segs(const mivi::GemvArgs& a, size_t row_bytes) : rb(row_bytes) {
        n0 = a.seg[0].n;
        n01 = n0 + (a.nseg > 1 ? a.seg[1].n : 0);
        n = n01 + (a.nseg > 2 ? a.seg[2].n : 0);
        W0 = (uintptr_t)a.seg[0].W;
        y0 = (uintptr_t)a.seg[0].y;
        const uintptr_t W1 = a.nseg > 1 ? (uintptr_t)a.seg[1].W : W0;
        const uintptr_t W2 = a.nseg > 2 ? (uintptr_t)a.seg[2].W : W1;
        const uintptr_t y1 = a.nseg > 1 ? (uintptr_t)a.seg[1].y : y0;
        const uintptr_t y2 = a.nseg > 2 ? (uintptr_t)a.seg[2].y : y1;
        // base of segment 1 minus where row n0 would be in segment 0, etc.
        dW1 = (int64_t)(W1 - (uintptr_t)n0 * rb) - (int64_t)W0;
        dW2 = (int64_t)(W2 - (uintptr_t)n01 * rb) - (int64_t)(W1 - (uintptr_t)n0 * rb);
        dy1 = (int64_t)(y1 - (uintptr_t)n0 * 4) - (int64_t)y0;
        dy2 = (int64_t)(y2 - (uintptr_t)n01 * 4) - (int64_t)(y1 - (uintptr_t)n0 * 4);
    }
    __device__ __forceinline__ const uint8_t* row(int r, size_t = 0) const {
        uintptr_t p = W0 + (uintptr_t)r * rb;
        p += (r >= n0 ? (uintptr_t)dW1 : 0) + (r >= n01 ? (uintptr_t)dW2 : 0);
        return (const uint8_t*)p;
    }
    __device__ __forceinline__ float* out(int r) const {
        uintptr_t p = y0 + (uintptr_t)r * 4;
        p += (r >= n0 ? (uintptr_t)dy1 : 0) + (r >= n01 ? (uintptr_t)dy2 : 0);
        return (float*)p;
    }
};

typedef __attribute__((address_space(1))) float gfloat;

// y[r] = v, or y[r] += v when accumulating. Each row has exactly one writer,
// so the accumulate is a global atomic add without return: the same single
// fp32 addition as a read-modify-write (up to denormal flushing in the atomic
// unit), but with no load whose wait would drain the weight prefetch queue.
__device__ __forceinline__ void store_out(const Segs& sg, int accumulate, int r, float v) {
    gfloat* y = (gfloat*)sg.out(r);
    if (accumulate)
        __builtin_amdgcn_global_atomic_fadd_f32(y, v);
    else
        *y = v;
}

// ------------------------------------------------------------------- Q4_K

// Scale/min pair for sub-blocks 2g and 2g+1 (q4_k_m.rs:11-22) from the 12
// scale bytes s0|s1|s2 (header dwords 1..3); g is per lane.
__device__ __forceinline__ void q4k_scales(uint32_t s0, uint32_t s1, uint32_t s2, int g,
                                           uint32_t& sc0, uint32_t& m0, uint32_t& sc1, uint32_t& m1) {
    const uint32_t sh = 16u * (uint32_t)(g & 1);
    if (g < 2) {
        uint32_t lo = s0 >> sh, bm = s1 >> sh;
        sc0 = lo & 63; sc1 = (lo >> 8) & 63;
        m0 = bm & 63; m1 = (bm >> 8) & 63;
    } else {
        uint32_t lo = s2 >> sh, hy = s0 >> sh, hz = s1 >> sh;
        sc0 = (lo & 0xF) | (((hy >> 6) & 3) << 4);
        m0 = ((lo >> 4) & 0xF) | (((hz >> 6) & 3) << 4);
        sc1 = ((lo >> 8) & 0xF) | (((hy >> 14) & 3) << 4);
        m1 = ((lo >> 12) & 0xF) | (((hz >> 14) & 3) << 4);
    }
}

// Partial dot of one Q4_K quarter (64 values: sub-blocks 2g, 2g+1) with x;
// the reference's d1*sum(q x) - m1*sum(x) + d2*... form (q4_k_m.rs:144-214).
__device__ __forceinline__ float q4k_unit(u32x4 hdr, u32x4 qa, u32x4 qb, int g, const float* xv,
                                          float X0, float X1) {
    float d = half_bits_to_f32(hdr.x), dmin = half_bits_to_f32(hdr.x >> 16);
    uint32_t sc0, m0, sc1, m1;
    q4k_scales(hdr.y, hdr.z, hdr.w, g, sc0, m0, sc1, m1);
    const uint32_t q[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
    float a0 = 0.f, a1 = 0.f, b0 = 0.f, b1 = 0.f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        uint32_t lo = q[i] & 0x0F0F0F0Fu, hi = (q[i] >> 4) & 0x0F0F0F0Fu;
        const float* x0 = xv + 4 * i;       // low nibbles: values 4i..4i+3
        const float* x1 = xv + 32 + 4 * i;  // high nibbles: values 32+4i..
        a0 = fmaf(ubyte_f32(lo, 0), x0[0], a0);
        a1 = fmaf(ubyte_f32(lo, 1), x0[1], a1);
        a0 = fmaf(ubyte_f32(lo, 2), x0[2], a0);
        a1 = fmaf(ubyte_f32(lo, 3), x0[3], a1);
        b0 = fmaf(ubyte_f32(hi, 0), x1[0], b0);
        b1 = fmaf(ubyte_f32(hi, 1), x1[1], b1);
        b0 = fmaf(ubyte_f32(hi, 2), x1[2], b0);
        b1 = fmaf(ubyte_f32(hi, 3), x1[3], b1);
    }
    float d1 = d * (float)sc0, mv1 = dmin * (float)m0;
    float d2 = d * (float)sc1, mv2 = dmin * (float)m1;
    return d1 * (a0 + a1) - mv1 * X0 + d2 * (b0 + b1) - mv2 * X1;
}

template <int LPR, int U, int PRO>
__global__ void __launch_bounds__(kWG) gemv_q4k_kernel(const mivi::GemvArgs a) {
    extern __shared__ float lds[];
    stage_input<PRO, 32>(lds, a);
    const int K = a.K, nb = K / 256;
    const size_t row_bytes = (size_t)nb * 144;
    const float* xsum = lds + K;
    const Segs sg(a, row_bytes);
    const int n = sg.n;
    constexpr int RPG = 64 / LPR;   // rows per lane group
    constexpr int RPT = RPG * U;    // rows per wave tile
    const int lane = threadIdx.x & 63, lr = lane % LPR, sub = lane / LPR;
    const int units = nb * 4;
    const int ntiles = (n + RPT - 1) / RPT;
    const int nwaves = gridDim.x * (kWG / 64);
    for (int tile = blockIdx.x * (kWG / 64) + (threadIdx.x >> 6); tile < ntiles; tile += nwaves) {
        const uint8_t* rows[U];
#pragma unroll
        for (int k = 0; k < U; k++) rows[k] = sg.row(min(tile * RPT + k * RPG + sub, n - 1), row_bytes);
        float acc[U];
#pragma unroll
        for (int k = 0; k < U; k++) acc[k] = 0.f;
        for (int u = lr; u < units; u += LPR) {
            const int b = u >> 2, g = u & 3;
            u32x4 hdr[U], qa[U], qb[U];
#pragma unroll
            for (int k = 0; k < U; k++) {
                const uint8_t* blk = rows[k] + (size_t)b * 144;
                hdr[k] = *(const u32x4_a4*)blk;
                qa[k] = *(const u32x4_a4*)(blk + 16 + 32 * g);
                qb[k] = *(const u32x4_a4*)(blk + 32 + 32 * g);
            }
            float xv[64];
            const float* xp = lds + b * 256 + g * 64;
#pragma unroll
            for (int i = 0; i < 16; i++) *(f32x4*)(xv + 4 * i) = *(const f32x4*)(xp + 4 * i);
            const float X0 = xsum[b * 8 + 2 * g], X1 = xsum[b * 8 + 2 * g + 1];
#pragma unroll
            for (int k = 0; k < U; k++) acc[k] += q4k_unit(hdr[k], qa[k], qb[k], g, xv, X0, X1);
        }
#pragma unroll
        for (int k = 0; k < U; k++) {
            float s = group_sum<LPR>(acc[k]);
            int r = tile * RPT + k * RPG + sub;
            if (lr == 0 && r < n) store_out(sg, a.accumulate, r, s);
        }
    }
}

// ------------------------------------------------------------------- Q6_K

// Partial dot of one Q6_K quarter: half h, l in [16j, 16j+16), the four
// 16-value sub-blocks l, l+32, l+64, l+96 (q6_k.rs:68-111). sum(sc*(q-32)*x)
// is formed as sc*(sum(q*x) - 32*sum(x)); both sums run over the same 16
// values in the same order, so an all-32 sub-block gives exactly 0.
__device__ __forceinline__ float q6k_unit(u32x4 ql0, u32x4 ql1, u32x4 qh, u32x4 scw, uint32_t dbits,
                                          int h, int j, const float* xv, const float* X) {
    const uint32_t L0[4] = {ql0.x, ql0.y, ql0.z, ql0.w};
    const uint32_t L1[4] = {ql1.x, ql1.y, ql1.z, ql1.w};
    const uint32_t H[4] = {qh.x, qh.y, qh.z, qh.w};
    float s[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        uint32_t q1 = (L0[i] & 0x0F0F0F0Fu) | ((H[i] << 4) & 0x30303030u);
        uint32_t q2 = (L1[i] & 0x0F0F0F0Fu) | ((H[i] << 2) & 0x30303030u);
        uint32_t q3 = ((L0[i] >> 4) & 0x0F0F0F0Fu) | (H[i] & 0x30303030u);
        uint32_t q4 = ((L1[i] >> 4) & 0x0F0F0F0Fu) | ((H[i] >> 2) & 0x30303030u);
#pragma unroll
        for (int k = 0; k < 4; k++) {
            s[0] = fmaf(ubyte_f32(q1, k), xv[4 * i + k], s[0]);
            s[1] = fmaf(ubyte_f32(q2, k), xv[16 + 4 * i + k], s[1]);
            s[2] = fmaf(ubyte_f32(q3, k), xv[32 + 4 * i + k], s[2]);
            s[3] = fmaf(ubyte_f32(q4, k), xv[48 + 4 * i + k], s[3]);
        }
    }
    // scales sc[8h + j + 2k], k = 0..3 (signed bytes)
    const uint32_t lo = h ? scw.z : scw.x, hi = h ? scw.w : scw.y;
    const int sh = 8 * j;
    float sc0 = sbyte_f32(lo >> sh, 0);
    float sc1 = sbyte_f32(lo >> sh, 2);
    float sc2 = sbyte_f32(hi >> sh, 0);
    float sc3 = sbyte_f32(hi >> sh, 2);
    float t = sc0 * (s[0] - 32.0f * X[0]);
    t = fmaf(sc1, s[1] - 32.0f * X[1], t);
    t = fmaf(sc2, s[2] - 32.0f * X[2], t);
    t = fmaf(sc3, s[3] - 32.0f * X[3], t);
    return t * half_bits_to_f32(dbits);
}

template <int LPR, int U, int PRO>
__global__ void __launch_bounds__(kWG) gemv_q6k_kernel(const mivi::GemvArgs a) {
    extern __shared__ float lds[];
    stage_input<PRO, 16>(lds, a);
    const int K = a.K, nb = K / 256;
    const size_t row_bytes = (size_t)nb * 210;
    const float* xsum = lds + K;
    const Segs sg(a, row_bytes);
    const int n = sg.n;
    constexpr int RPG = 64 / LPR;
    constexpr int RPT = RPG * U;
    const int lane = threadIdx.x & 63, lr = lane % LPR, sub = lane / LPR;
    const int units = nb * 4;
    const int ntiles = (n + RPT - 1) / RPT;
    const int nwaves = gridDim.x * (kWG / 64);
    for (int tile = blockIdx.x * (kWG / 64) + (threadIdx.x >> 6); tile < ntiles; tile += nwaves) {
        const uint8_t* rows[U];
#pragma unroll
        for (int k = 0; k < U; k++) rows[k] = sg.row(min(tile * RPT + k * RPG + sub, n - 1), row_bytes);
        float acc[U];
#pragma unroll
        for (int k = 0; k < U; k++) acc[k] = 0.f;
        for (int u = lr; u < units; u += LPR) {
            const int b = u >> 2, h = (u >> 1) & 1, j = u & 1;
            u32x4 ql0[U], ql1[U], qh[U], scw[U];
            uint32_t db[U];
#pragma unroll
            for (int k = 0; k < U; k++) {
                const uint8_t* blk = rows[k] + (size_t)b * 210;
                ql0[k] = ld16_a2(blk + 64 * h + 16 * j);
                ql1[k] = ld16_a2(blk + 64 * h + 32 + 16 * j);
                qh[k] = ld16_a2(blk + 128 + 32 * h + 16 * j);
                scw[k] = ld16_a2(blk + 192);
                db[k] = ld_u16(blk + 208);
            }
            float xv[64];
            const int e0 = b * 256 + h * 128 + 16 * j;
#pragma unroll
            for (int q = 0; q < 4; q++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    *(f32x4*)(xv + 16 * q + 4 * i) = *(const f32x4*)(lds + e0 + 32 * q + 4 * i);
            float X[4];
#pragma unroll
            for (int q = 0; q < 4; q++) X[q] = xsum[(e0 + 32 * q) / 16];
#pragma unroll
            for (int k = 0; k < U; k++) acc[k] += q6k_unit(ql0[k], ql1[k], qh[k], scw[k], db[k], h, j, xv, X);
        }
#pragma unroll
        for (int k = 0; k < U; k++) {
            float s = group_sum<LPR>(acc[k]);
            int r = tile * RPT + k * RPG + sub;
            if (lr == 0 && r < n) store_out(sg, a.accumulate, r, s);
        }
    }
}

// ------------------------------------------------------------------- Q8_0

template <int LPR, int U, int PRO>
__global__ void __launch_bounds__(kWG) gemv_q80_kernel(const mivi::GemvArgs a) {
    extern __shared__ float lds[];
    stage_input<PRO, 0>(lds, a);
    const int K = a.K, nb = K / 32;
    const size_t row_bytes = (size_t)nb * 34;
    const Segs sg(a, row_bytes);
    const int n = sg.n;
    constexpr int RPG = 64 / LPR;
    constexpr int RPT = RPG * U;
    const int lane = threadIdx.x & 63, lr = lane % LPR, sub = lane / LPR;
    const int ntiles = (n + RPT - 1) / RPT;
    const int nwaves = gridDim.x * (kWG / 64);
    for (int tile = blockIdx.x * (kWG / 64) + (threadIdx.x >> 6); tile < ntiles; tile += nwaves) {
        const uint8_t* rows[U];
#pragma unroll
        for (int k = 0; k < U; k++) rows[k] = sg.row(min(tile * RPT + k * RPG + sub, n - 1), row_bytes);
        float acc[U];
#pragma unroll
        for (int k = 0; k < U; k++) acc[k] = 0.f;
        for (int b = lr; b < nb; b += LPR) {
            u32x4 qa[U], qb[U];
            uint32_t db[U];
#pragma unroll
            for (int k = 0; k < U; k++) {
                const uint8_t* blk = rows[k] + (size_t)b * 34;
                db[k] = ld_u16(blk);
                qa[k] = ld16_a2(blk + 2);
                qb[k] = ld16_a2(blk + 18);
            }
            const float* xp = lds + b * 32;
#pragma unroll
            for (int k = 0; k < U; k++) {
                const uint32_t q[8] = {qa[k].x, qa[k].y, qa[k].z, qa[k].w, qb[k].x, qb[k].y, qb[k].z, qb[k].w};
                float s0 = 0.f, s1 = 0.f;
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    s0 = fmaf(sbyte_f32(q[i], 0), xp[4 * i], s0);
                    s1 = fmaf(sbyte_f32(q[i], 1), xp[4 * i + 1], s1);
                    s0 = fmaf(sbyte_f32(q[i], 2), xp[4 * i + 2], s0);
                    s1 = fmaf(sbyte_f32(q[i], 3), xp[4 * i + 3], s1);
                }
                acc[k] = fmaf(s0 + s1, half_bits_to_f32(db[k]), acc[k]);
            }
        }
#pragma unroll
        for (int k = 0; k < U; k++) {
            float s = group_sum<LPR>(acc[k]);
            int r = tile * RPT + k * RPG + sub;
            if (lr == 0 && r < n) store_out(sg, a.accumulate, r, s);
        }
    }
}

// -------------------------------------------------- F16 / BF16 / F32 rows

// KIND 0 f16, 1 bf16, 2 f32. One wave per row; rows of any alignment.
template <int KIND, int PRO>
__global__ void __launch_bounds__(kWG) gemv_dense_kernel(const mivi::GemvArgs a) {
    extern __shared__ float lds[];
    stage_input<PRO, 0>(lds, a);
    const int d = a.K;
    const size_t row_bytes = (size_t)d * (KIND == 2 ? 4 : 2);
    const Segs sg(a, row_bytes);
    const int n = sg.n;
    const int lane = threadIdx.x & 63;
    const int nwaves = gridDim.x * (kWG / 64);
    for (int r = blockIdx.x * (kWG / 64) + (threadIdx.x >> 6); r < n; r += nwaves) {
        const uint8_t* row = sg.row(r, row_bytes);
        float acc = 0.f;
        for (int k = lane; k < d; k += 64) {
            float w;
            if (KIND == 2) {
                const uint8_t* p = row + 4 * (size_t)k;
                w = ((uintptr_t)p & 3) ? __uint_as_float(p[0] | (p[1] << 8) | (p[2] << 16) | ((uint32_t)p[3] << 24))
                                       : *(const float*)p;
            } else {
                uint32_t bits = ld_u16(row + 2 * (size_t)k);
                w = KIND == 0 ? half_bits_to_f32(bits) : bf16_bits_to_f32(bits);
            }
            acc = fmaf(w, lds[k], acc);
        }
        acc = wave_sum(acc);
        if (lane == 0) store_out(sg, a.accumulate, r, acc);
    }
}

// ------------------------------------------------- tiled GEMV (Q4_K / Q6_K)
//
// Persistent workgroups stream tiles of RT whole rows: every thread copies
// fixed 16-byte chunks of the tile (one contiguous 4 KB span per workgroup
// instruction), holds the next tile in registers while the current one is
// reduced out of LDS, then writes it to the other LDS buffer. The compute
// layout is the per-quarter-superblock unit of the kernels above; each lane
// keeps its activation slice and sub-block sums in registers for the whole
// launch.

enum { FMT_Q4K = 0, FMT_Q6K = 1 };

template <int FMT> struct KQ;
template <> struct KQ<FMT_Q4K> { static constexpr int bytes = 144, G = 32, CPT = 5; };
template <> struct KQ<FMT_Q6K> { static constexpr int bytes = 210, G = 0, CPT = 7; };

__device__ __forceinline__ u32x4 ldg16(const uint8_t* p) {
    return *(const __attribute__((address_space(1))) u32x4*)p;
}

// Unaligned LDS/global vector types: the HSA runtime runs gfx9+ in unaligned
// access mode, so these compile to single ds_read_b128 / ds_read_b64.
typedef uint32_t u32x4_a2 __attribute__((ext_vector_type(4), aligned(2)));
typedef uint32_t u32x2_a1 __attribute__((ext_vector_type(2), aligned(1)));

// ------------------------------------------------ activations as int8 digits
//
// The tiled kernels multiply the weight codes by x in integer arithmetic.
// x is represented against one scale per launch, s = 2 max|x| / 127, as
//     x ~= s * (d0 + d1 / 256 + d2 / 256^2),   d0 in [-64, 64], d1, d2 in [-128, 127],
// the balanced base-256 digits of Y = rint(x * 127 * 2^15 / max|x|)
// (|Y| <= 127 * 2^15 < 2^22), so |x - x~| <= 1.2e-7 * max|x|. A row's dot
// product is then
//     s * sum_d 256^-d * sum_i w_i d_i,
// where every sum of code * digit is exact in int32 (v_dot4_i32_i8) and the
// per-sub-block scales are applied with exact 24-bit integer multiplies.
// The error of the whole dot is below 2.5e-7 * ||w||_1 * max|x|, i.e.
// 2.5e-7 * sqrt(K) * ||w|| * ||x|| (2.3e-5 of ||w|| ||x|| at K = 8192).
constexpr float kDig1 = 1.0f / 256.0f, kDig2 = 1.0f / 65536.0f;
constexpr float kDigMul = 4161536.0f;  // 127 * 2^15: Y = rint(x * kDigMul / max|x|)

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ float nanmax(float a, float b) { return (b > a || b != b) ? b : a; }

// The digit planes of four values: Y = rint(u * mul) for |Y| < 2^22 (adding
// 1.5 * 2^23 in the fma rounds once, ties to even, and leaves Y in the low
// mantissa bits), written as balanced base-256 digits
// Y = 65536 d0 + 256 d1 + d2 with d1, d2 in [-128, 127]: the bytes of
// Y + 0x808080 are d + 128, so a byte permute gathers each plane and an xor
// with 0x80 per byte makes the digits signed. Value e in byte e of w0 (d0),
// w1 (d1) and w2 (d2). (Non-finite inputs give a NaN digit scale, so their
// digits never matter.)
__device__ __forceinline__ void digits4_b256(const float (&u)[4], float mul, uint32_t& w0, uint32_t& w1,
                                             uint32_t& w2) {
    uint32_t z[4];
#pragma unroll
    for (int e = 0; e < 4; e++) z[e] = __float_as_uint(fmaf(u[e], mul, 12582912.0f)) - 0x4ABF7F80u;  // - bits(1.5*2^23) + 0x808080
    const uint32_t lo01 = __builtin_amdgcn_perm(z[1], z[0], 0x05010400u);  // z0.b0 z1.b0 z0.b1 z1.b1
    const uint32_t lo23 = __builtin_amdgcn_perm(z[3], z[2], 0x05010400u);  // z2.b0 z3.b0 z2.b1 z3.b1
    w2 = __builtin_amdgcn_perm(lo23, lo01, 0x05040100u) ^ 0x80808080u;
    w1 = __builtin_amdgcn_perm(lo23, lo01, 0x07060302u) ^ 0x80808080u;
    w0 = (__builtin_amdgcn_perm(z[1], z[0], 0x0c0c0602u) | __builtin_amdgcn_perm(z[3], z[2], 0x06020c0cu)) ^ 0x80808080u;
}

// Digit planes of the K floats staged at xs, written to dig[d * K / 4 + i]
// (four values per dword, value 4i + e in byte e). Returns s (NaN when x
// holds a NaN or an infinity, so the products come out NaN as in fp32).
__device__ __forceinline__ float stage_digits(const float* xs, uint32_t* dig, int K) {
    __shared__ float red[kWG / 64];
    float m = 0.f;
    for (int i = threadIdx.x; i < K; i += kWG) m = nanmax(m, fabsf(xs[i]));
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) m = nanmax(m, __shfl_xor(m, o, 64));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    m = red[0];
#pragma unroll
    for (int i = 1; i < kWG / 64; i++) m = nanmax(m, red[i]);
    const bool finite = m > 0.f && m <= 3.40282347e38f;
    const float mul = finite ? kDigMul / m : 0.0f;
    const float sc = ((m - m) + m) * (2.0f / 127.0f);
    for (int i = threadIdx.x; i < K / 4; i += kWG) {
        const f32x4 v = *(const f32x4*)(xs + 4 * i);
        uint32_t w0, w1, w2;
        const float u[4] = {v[0], v[1], v[2], v[3]};
        digits4_b256(u, mul, w0, w1, w2);
        dig[i] = w0;
        dig[K / 4 + i] = w1;
        dig[K / 2 + i] = w2;
    }
    return sc;
}

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// a * b for |a| < 2^23 and 8-bit b: the explicit 24-bit sign extension lets
// the compiler use the full-rate v_mad_i32_i24 instead of v_mul_lo_u32.
__device__ __forceinline__ int mul24(int a, int b) { return (int)__builtin_amdgcn_sbfe(a, 0, 24) * b; }
// a * b + c with the same bounds (v_mad_i32_i24)
__device__ __forceinline__ int mad24(int a, int b, int c) { return (int)__builtin_amdgcn_sbfe(a, 0, 24) * b + c; }

// One Q6_K unit (16 values of each of the sub-blocks l, l+32, l+64, l+96 of
// half h, q6_k.rs:68-111): sum over the unit of sc * (q - 32) * digits, per
// digit plane, in int32; off[k][d] = -32 * sum of the 16 digits of quad k.
// Returns d * (A0 + A1/256 + A2/256^2) in units of s.
__device__ __forceinline__ float q6k_unit_i8(u32x4 ql0, u32x4 ql1, u32x4 qh, u32x2 scw, uint32_t dbits,
                                             const uint32_t (&xd)[3][16], const int (&off)[4][3]) {
    const uint32_t L0[4] = {ql0.x, ql0.y, ql0.z, ql0.w};
    const uint32_t L1[4] = {ql1.x, ql1.y, ql1.z, ql1.w};
    const uint32_t H[4] = {qh.x, qh.y, qh.z, qh.w};
    int D[4][3];
#pragma unroll
    for (int k = 0; k < 4; k++)
#pragma unroll
        for (int d = 0; d < 3; d++) D[k][d] = off[k][d];
#pragma unroll
    for (int m = 0; m < 4; m++) {
        const uint32_t q1 = (L0[m] & 0x0F0F0F0Fu) | ((H[m] << 4) & 0x30303030u);
        const uint32_t q2 = (L1[m] & 0x0F0F0F0Fu) | ((H[m] << 2) & 0x30303030u);
        const uint32_t q3 = ((L0[m] >> 4) & 0x0F0F0F0Fu) | (H[m] & 0x30303030u);
        const uint32_t q4 = ((L1[m] >> 4) & 0x0F0F0F0Fu) | ((H[m] >> 2) & 0x30303030u);
#pragma unroll
        for (int d = 0; d < 3; d++) {
            D[0][d] = sdot4(q1, xd[d][m], D[0][d]);
            D[1][d] = sdot4(q2, xd[d][4 + m], D[1][d]);
            D[2][d] = sdot4(q3, xd[d][8 + m], D[2][d]);
            D[3][d] = sdot4(q4, xd[d][12 + m], D[3][d]);
        }
    }
    // scales sc[8h + j + 2k], k = 0..3: bytes 0, 2, 4, 6 of scw
    const int sc[4] = {(int)(int8_t)scw.x, (int)(int8_t)(scw.x >> 16), (int)(int8_t)scw.y,
                       (int)(int8_t)(scw.y >> 16)};
    int A[3];
#pragma unroll
    for (int d = 0; d < 3; d++) {
        // |D| <= 16 * 32 * 127 < 2^17, |A| < 2^26: exact 24-bit multiplies
        A[d] = mul24(D[0][d], sc[0]) + mul24(D[1][d], sc[1]) + mul24(D[2][d], sc[2]) + mul24(D[3][d], sc[3]);
    }
    const float f = fmaf((float)A[2], kDig2, fmaf((float)A[1], kDig1, (float)A[0]));
    return half_bits_to_f32(dbits) * f;
}

// One Q4_K unit (sub-blocks 2g and 2g+1, q4_k_m.rs:144-214):
// d * s * sum_d 256^-d (sc0 * sum(q xd) + sc1 * ...) - dmin * (m0 X0 + m1 X1),
// X0, X1 the fp32 sums of x over the two sub-blocks.
__device__ __forceinline__ float q4k_unit_i8(u32x4 hdr, u32x4 qa, u32x4 qb, int g, const uint32_t (&xd)[3][16],
                                             float s, float X0, float X1) {
    const float d = half_bits_to_f32(hdr.x), dmin = half_bits_to_f32(hdr.x >> 16);
    uint32_t sc0, m0, sc1, m1;
    q4k_scales(hdr.y, hdr.z, hdr.w, g, sc0, m0, sc1, m1);
    const uint32_t q[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
    int Dl[3] = {0, 0, 0}, Dh[3] = {0, 0, 0};
#pragma unroll
    for (int m = 0; m < 8; m++) {
        const uint32_t lo = q[m] & 0x0F0F0F0Fu, hi = (q[m] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
        for (int e = 0; e < 3; e++) {
            Dl[e] = sdot4(lo, xd[e][m], Dl[e]);       // values 64g + 4m + 0..3
            Dh[e] = sdot4(hi, xd[e][8 + m], Dh[e]);   // values 64g + 32 + 4m + 0..3
        }
    }
    int A[3];
#pragma unroll
    for (int e = 0; e < 3; e++) A[e] = mul24(Dl[e], (int)sc0) + mul24(Dh[e], (int)sc1);
    const float f = fmaf((float)A[2], kDig2, fmaf((float)A[1], kDig1, (float)A[0]));
    return (d * s) * f - dmin * fmaf((float)m0, X0, (float)m1 * X1);
}

// ------------------------------------------- activation staging (stream kernel)
//
// Each thread owns E = K / 256 consecutive activations. All of its input
// loads are issued in one batch (before the weight prefetch, so waiting for
// them never waits for weights), then one workgroup reduction (sum of
// squares and max together) and one barrier publish the int8 digit planes
// (and, for Q4_K, the fp32 sums of each 32-value sub-block) in LDS.

typedef __attribute__((address_space(1))) const f32x4 gf32x4;

constexpr int kConvKs = 3;  // conv window of the streaming prologue (LFM2 L_cache)

template <int PRO, int E>
struct StageIn {
    static constexpr bool kConv = PRO == mivi::PRO_CONV;
    f32x4 x[E / 4], y[E / 4];                 // NONE: x; RMSNORM: x, norm w; SWIGLU: gate, up; CONV: B, X
    f32x4 c[kConv ? E / 4 : 1];               // CONV: C
    f32x4 st[kConv ? E * kConvKs / 4 : 1];    // CONV: previous window of the E channels
    f32x4 cw[kConv ? E * kConvKs / 4 : 1];    // CONV: per-channel weights (mode 0)

    // NONE / RMSNORM / SWIGLU: chunk i of this thread is the 16 bytes at
    // 16 (threadIdx.x + kWG i), so each wave load reads 1 KB contiguous, and
    // the thread keeps them (digit dword threadIdx.x + kWG i, a 32-value
    // sub-block over eight consecutive threads). CONV: the thread's own E
    // consecutive values (its channels' windows are contiguous).
    __device__ __forceinline__ void load(const mivi::GemvArgs& a) {
        const int e0 = threadIdx.x * E;
        if constexpr (!kConv) {
#pragma unroll
            for (int i = 0; i < E / 4; i++) x[i] = *(gf32x4*)(a.x + 4 * (threadIdx.x + kWG * i));
        } else {
#pragma unroll
            for (int i = 0; i < E / 4; i++) x[i] = *(gf32x4*)(a.x + e0 + 4 * i);
        }
        if constexpr (PRO == mivi::PRO_RMSNORM) {
#pragma unroll
            for (int i = 0; i < E / 4; i++) y[i] = *(gf32x4*)(a.norm_w + 4 * (threadIdx.x + kWG * i));
        } else if constexpr (PRO == mivi::PRO_SWIGLU) {
#pragma unroll
            for (int i = 0; i < E / 4; i++) y[i] = *(gf32x4*)(a.x2 + 4 * (threadIdx.x + kWG * i));
        } else if constexpr (kConv) {
            // a.x = [B | C | X], ssm.rs:80-140
#pragma unroll
            for (int i = 0; i < E / 4; i++) {
                c[i] = *(gf32x4*)(a.x + a.K + e0 + 4 * i);
                y[i] = *(gf32x4*)(a.x + 2 * a.K + e0 + 4 * i);
            }
            const bool swap = a.phase && ((*a.phase) & 1);
            const float* st_in = swap ? a.st_out : a.st_in;
#pragma unroll
            for (int i = 0; i < E * kConvKs / 4; i++) st[i] = *(gf32x4*)(st_in + e0 * kConvKs + 4 * i);
            if (a.conv_mode == 0) {
#pragma unroll
                for (int i = 0; i < E * kConvKs / 4; i++) cw[i] = *(gf32x4*)(a.conv_w + e0 * kConvKs + 4 * i);
            }
        }
    }

    // Forms the activations, writes the digit planes dig[3][PS] (PS dwords
    // apart, K/4 when 0; and the Q4_K sub-block sums xsum[K/32] when SUMS)
    // and returns the digit scale s.
    template <bool SUMS, int PS = 0>
    __device__ __forceinline__ float finish(const mivi::GemvArgs& a, uint32_t* dig, float* xsum) {
        __shared__ float red[2][kWG / 64];
        const int K = a.K, e0 = threadIdx.x * E;
        // dword of values 4q .. 4q+3 of this thread
        auto dw = [&](int q) { return kConv ? e0 / 4 + q : (int)threadIdx.x + kWG * q; };
        float v[E];
#pragma unroll
        for (int i = 0; i < E; i++) v[i] = x[i / 4][i % 4];
        float m = 0.f, ss = 0.f;
        if constexpr (PRO == mivi::PRO_RMSNORM) {
            // ss and max|x w| in one reduction; max|x * scale * w| = scale * max|x w|
            // (a NaN or infinite x makes ss, so the scale and m, NaN)
#pragma unroll
            for (int i = 0; i < E; i++) {
                ss = fmaf(v[i], v[i], ss);
                m = fmaxf(m, fabsf(v[i] * y[i / 4][i % 4]));
            }
        } else if constexpr (PRO == mivi::PRO_SWIGLU) {
#pragma unroll
            for (int i = 0; i < E; i++) v[i] = silu_f(v[i]) * y[i / 4][i % 4];  // math.rs:87-95
        } else if constexpr (kConv) {
            const bool writer = blockIdx.x == 0;
            const bool swap = a.phase && ((*a.phase) & 1);
            float* st_out = swap ? (float*)a.st_in : a.st_out;
            float w[E * kConvKs];
#pragma unroll
            for (int i = 0; i < E * kConvKs; i++)
                w[i] = a.conv_mode == 0 ? cw[i / 4][i % 4]
                     : a.conv_mode == 1 ? a.conv_w[i % kConvKs] : 1.0f / (float)kConvKs;
            float nst[E * kConvKs];
#pragma unroll
            for (int d = 0; d < E; d++) {
                const float bx = v[d] * y[d / 4][d % 4];
                float conv = 0.0f;
#pragma unroll
                for (int k = 0; k < kConvKs; k++) {
                    const int o = d * kConvKs + k;
                    const float sv = k + 1 < kConvKs ? st[(o + 1) / 4][(o + 1) % 4] : bx;
                    conv += w[o] * sv;
                    nst[o] = sv;
                }
                v[d] = c[d / 4][d % 4] * conv;
            }
            if (writer) {
#pragma unroll
                for (int i = 0; i < E * kConvKs / 4; i++)
                    *(f32x4*)(st_out + e0 * kConvKs + 4 * i) =
                        f32x4{nst[4 * i], nst[4 * i + 1], nst[4 * i + 2], nst[4 * i + 3]};
            }
        }
        if constexpr (PRO != mivi::PRO_RMSNORM) {
            // fmaxf passes NaNs over: nn, a sum of v * 0, turns m NaN for them
            float nn = 0.f;
#pragma unroll
            for (int i = 0; i < E; i++) {
                m = fmaxf(m, fabsf(v[i]));
                nn = fmaf(v[i], 0.f, nn);
            }
            m += nn;
        }
        // one workgroup reduction of (ss, m): the xor butterfly of the wave
        // (lane 0's sums), then the waves in order
        if constexpr (PRO == mivi::PRO_RMSNORM) ss = xsum_desc<64>(ss);
        {
            float lo, hi;
            swap32(m, lo, hi);
            m = nanmax(lo, hi);
            swap16(m, lo, hi);
            m = nanmax(lo, hi);
            m = nanmax(m, dpp_mov<0x128>(m));
            m = nanmax(m, dpp_mov<0x12C>(m));
            m = nanmax(m, dpp_mov<0x4E>(m));
            m = nanmax(m, dpp_mov<0xB1>(m));
        }
        if ((threadIdx.x & 63) == 0) {
            red[0][threadIdx.x >> 6] = ss;
            red[1][threadIdx.x >> 6] = m;
        }
        __syncthreads();
        m = red[1][0];
        ss = red[0][0];
#pragma unroll
        for (int i = 1; i < kWG / 64; i++) {
            m = nanmax(m, red[1][i]);
            ss += red[0][i];
        }
        // RMSNORM: x = (v w) / rms (math.rs:7-22); the digits are those of
        // u = v w, since 1 / rms cancels in u * kDigMul / max|u|, and the
        // scale goes into s and the sub-block sums
        float scale = 1.0f;
        if constexpr (PRO == mivi::PRO_RMSNORM) {
            scale = 1.0f / sqrtf(ss / (float)K + a.eps);
#pragma unroll
            for (int i = 0; i < E; i++) v[i] = v[i] * y[i / 4][i % 4];
        }
        // digits (see the representation above)
        const bool finite = m > 0.f && m <= 3.40282347e38f;
        const float mul = finite ? kDigMul / m : 0.0f;
        const float sc = ((m - m) + m * scale) * (2.0f / 127.0f);
        uint32_t w0[E / 4], w1[E / 4], w2[E / 4];
#pragma unroll
        for (int q = 0; q < E / 4; q++) {
            const float u[4] = {v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
            digits4_b256(u, mul, w0[q], w1[q], w2[q]);
        }
        const int P = PS ? PS : K / 4;
#pragma unroll
        for (int q = 0; q < E / 4; q++) {
            dig[dw(q)] = w0[q];
            dig[P + dw(q)] = w1[q];
            dig[2 * P + dw(q)] = w2[q];
        }
        if constexpr (SUMS) {
            static_assert(E >= 4, "at least four activations per thread");
            if constexpr (!kConv) {
                // fp32 sums of each 32-value sub-block: eight consecutive
                // threads, xor 1, 2, 4 (the writers, lanes with bit 2 clear,
                // see their exact partners; row_ror:12 reads lane (i + 4) mod 16)
#pragma unroll
                for (int q = 0; q < E / 4; q++) {
                    float t = ((v[4 * q] + v[4 * q + 1]) + v[4 * q + 2]) + v[4 * q + 3];
                    t += dpp_mov<0xB1>(t);
                    t += dpp_mov<0x4E>(t);
                    t += dpp_mov<0x12C>(t);
                    if ((threadIdx.x & 7) == 0) xsum[dw(q) >> 3] = t * scale;
                }
            } else {
                // fp32 sums of each 32-value sub-block (32 / E threads share one)
#pragma unroll
                for (int b = 0; b < (E >= 32 ? E / 32 : 1); b++) {
                    float t = 0.f;
#pragma unroll
                    for (int i = 0; i < (E >= 32 ? 32 : E); i++) t += v[b * 32 + i];
                    // xor 1, 2, 4 in that order (as above)
                    if constexpr (E < 32) t += dpp_mov<0xB1>(t);
                    if constexpr (E < 16) t += dpp_mov<0x4E>(t);
                    if constexpr (E < 8) t += dpp_mov<0x12C>(t);
                    if (E >= 32 || (threadIdx.x % (32 / E)) == 0) xsum[(e0 + 32 * b) / 32] = t * scale;
                }
            }
        }
        __syncthreads();
        return sc;
    }
};

// Bytes of one 64-value unit of a row, as its lane loads them.
template <int FMT> struct Unit;
template <> struct Unit<FMT_Q6K> { u32x4 ql0, ql1, qh; u32x2 sc; uint32_t d; };
template <> struct Unit<FMT_Q4K> { u32x4 hdr, qa, qb; };

typedef __attribute__((address_space(1))) const u32x4_a2 gu32x4_a2;
typedef __attribute__((address_space(1))) const u32x2_a1 gu32x2_a1;
typedef __attribute__((address_space(1))) const uint16_t gu16;

// Packed Q6_K row of U = K/64 units (mivi_hip_pack_weights): the same bytes
// as the GGUF row, regrouped so that each load of a wave is contiguous:
//   [0, 16U)      ql bytes 64h + 16j .. +16 of unit u = (b, h, j) at 16u
//   [16U, 32U)    ql bytes 64h + 32 + 16j .. +16
//   [32U, 48U)    qh bytes 128 + 32h + 16j .. +16
//   [48U, 52U)    the unit's four scales sc[8h + j + 2k], k = 0..3, at 4u
//   [52U, 52.5U)  d of block b at 52U + 2b
__device__ __forceinline__ void load_unit_q6k_packed(Unit<FMT_Q6K>& U, const uint8_t* row, int u, int nu) {
    U.ql0 = ldg16(row + 16 * u);
    U.ql1 = ldg16(row + 16 * nu + 16 * u);
    U.qh = ldg16(row + 32 * nu + 16 * u);
    // the four scale bytes, spread by packed_q6k_scales at compute time (doing
    // it here would make the wave wait for this load as soon as it is issued)
    U.sc.x = *(const __attribute__((address_space(1))) uint32_t*)(row + 48 * nu + 4 * u);
    U.sc.y = 0;
    U.d = *(gu16*)(row + 52 * nu + 2 * (u >> 2));
}

// The packed unit's scale dword (sc[k] in byte k) as the GGUF layout's two
// dwords hold them (sc[k] in byte 2k).
__device__ __forceinline__ u32x2 packed_q6k_scales(uint32_t w) {
    return u32x2{(w & 0xFFu) | ((w & 0xFF00u) << 8), ((w >> 16) & 0xFFu) | ((w >> 24) << 16)};
}

// Unit u of the row at `row`: Q6_K unit (b, h, j) = block u/4, half h,
// l in [16j, 16j + 16); Q4_K unit (b, g) = block u/4, sub-blocks 2g, 2g+1.
template <int FMT>
__device__ __forceinline__ void load_unit(Unit<FMT>& U, const uint8_t* row, int u) {
    const int b = u >> 2;
    if constexpr (FMT == FMT_Q6K) {
        const int h = (u >> 1) & 1, j = u & 1;
        const uint8_t* p = row + b * 210;
        U.ql0 = *(gu32x4_a2*)(p + 64 * h + 16 * j);
        U.ql1 = *(gu32x4_a2*)(p + 64 * h + 32 + 16 * j);
        U.qh = *(gu32x4_a2*)(p + 128 + 32 * h + 16 * j);
        U.sc = *(gu32x2_a1*)(p + 192 + 8 * h + j);
        U.d = *(gu16*)(p + 208);
    } else {
        const int g = u & 3;
        const uint8_t* p = row + b * 144;
        U.hdr = ldg16(p);
        U.qa = ldg16(p + 16 + 32 * g);
        U.qb = ldg16(p + 32 + 32 * g);
    }
}

// Column c of a batched launch (a.ncol > 1): the same weights against the
// c-th activation vector, written to the c-th outputs (pointer + c * stride).
__device__ __forceinline__ mivi::GemvArgs gemv_column(const mivi::GemvArgs& a, int c) {
    mivi::GemvArgs v = a;
    v.x = a.x + c * a.xs;
    if (a.x2) v.x2 = a.x2 + c * a.xs;
    if (a.st_in) v.st_in = a.st_in + c * a.sts;
    if (a.st_out) v.st_out = a.st_out + c * a.sts;
    if (a.phase) v.phase = a.phase + c;
    return v;
}

// EPI_CONV: the ShortConv step of channel c of column col from its in_proj
// rows B, C, X (ssm.rs:80-140), in the operation order of the PRO_CONV
// prologue (StageIn::finish), so out_proj's input is the same bit for bit:
// bx = B * X, the window shifts in bx, conv = sum_k w_k * window_k from
// zero, y = C * conv; the window goes to the column's other ping-pong buffer.
// conv_prefetch loads what the step needs besides B, C, X (the window, the
// weights, the buffer to write), so a kernel can issue it with its weight
// loads; conv_epilogue = both.
struct ConvPre {
    float sv[kConvKs - 1];  // window values 1 .. ks-1
    float w[kConvKs];
    float* st_out;
};
__device__ __forceinline__ void conv_prefetch(const mivi::GemvArgs& a, int col, int c, ConvPre& pre) {
    const bool swap = a.phase && (a.phase[col] & 1);
    const float* st_in = (swap ? a.st_out : a.st_in) + col * a.sts + (size_t)c * kConvKs;
    pre.st_out = (swap ? (float*)a.st_in : a.st_out) + col * a.sts + (size_t)c * kConvKs;
#pragma unroll
    for (int k = 0; k + 1 < kConvKs; k++) pre.sv[k] = st_in[k + 1];
#pragma unroll
    for (int k = 0; k < kConvKs; k++)
        pre.w[k] = a.conv_mode == 0 ? a.conv_w[(size_t)c * kConvKs + k]
                 : a.conv_mode == 1 ? a.conv_w[k] : 1.0f / (float)kConvKs;
}
__device__ __forceinline__ void conv_finish(const mivi::GemvArgs& a, int col, int c, float B, float C, float X,
                                            const ConvPre& pre) {
    const float bx = B * X;
    float conv = 0.0f;
    float sv[kConvKs];
#pragma unroll
    for (int k = 0; k < kConvKs; k++) {
        sv[k] = k + 1 < kConvKs ? pre.sv[k] : bx;
        conv += pre.w[k] * sv[k];
    }
#pragma unroll
    for (int k = 0; k < kConvKs; k++) pre.st_out[k] = sv[k];
    a.seg[0].y[col * a.ys + c] = C * conv;
}
__device__ __forceinline__ void conv_epilogue(const mivi::GemvArgs& a, int col, int c, float B, float C, float X) {
    ConvPre pre;
    conv_prefetch(a, col, c, pre);
    conv_finish(a, col, c, B, C, X, pre);
}

// K-quant GEMV for the decode shapes (K = 2048/4096/8192). A persistent grid
// of waves walks groups of RPW = 64/LPR rows; in each group a row is covered
// by LPR lanes, each owning NU fixed 64-value units, so a lane's activation
// digits stay in registers for the whole launch. Every lane loads its own
// units straight from HBM into a ring of PD row groups held in registers:
// the loop has no LDS traffic and no barriers, so each wave streams at its
// own pace. After the x staging the workgroup never synchronises again.
// NC > 1: up to NC activation columns (sequences of a batched decode step)
// against the same rows. Each row is loaded once and its units are dotted
// with every column's digits (also held in registers), in the same order as
// the one-column kernel, so every column's result is bit-identical to a
// one-column launch on that column.
// XL: the digits stay in LDS and each step reads its units' digits there
// (for column counts whose digits would not fit in registers).
template <int FMT, int KT, int LPR, int NU, int PD, int PRO, int EPI, bool PACK = false, int NC = 1, bool XL = false>
__global__ void __launch_bounds__(kWG) gemv_kq_stream_kernel(const mivi::GemvArgs a) {
    static_assert(!PACK || FMT == FMT_Q6K, "only Q6_K has a packed layout");
    constexpr int RPW = 64 / LPR;
    static_assert(EPI != mivi::EPI_SWIGLU || LPR == 32, "the pair epilogue takes two rows per wave");
    static_assert(EPI != mivi::EPI_CONV || (FMT == FMT_Q4K && KT == 2048), "the conv epilogue is the Q4_K in_proj");
    constexpr int K = KT, nb = K / 256, units = nb * 4;
    constexpr int row_bytes = nb * KQ<FMT>::bytes;
    __shared__ __attribute__((aligned(16))) uint32_t dig[NC][3 * K / 4];
    __shared__ float xsum[NC][FMT == FMT_Q4K ? K / 32 : 1];
    const Segs sg(a, row_bytes);
    const int n = sg.n;
    const int ncol = NC == 1 ? 1 : a.ncol;  // workgroup-uniform, <= NC
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, lr = lane % LPR, sub = lane / LPR;
    // EPI_SWIGLU: group c is the row pair (gate c, up c) = rows c and n0 + c.
    // EPI_CONV: group g is channels RPW g .. RPW g + RPW - 1, taken in three
    // steps, their B rows, C rows, X rows (rows c, D + c, 2D + c); the conv
    // runs after the X step from the B and C sums kept in registers
    const int n0 = a.seg[0].n;
    const int D3 = n0 / 3;
    const int ngroups = EPI == mivi::EPI_SWIGLU ? n0 : EPI == mivi::EPI_CONV ? (D3 + RPW - 1) / RPW : (n + RPW - 1) / RPW;
    const int nw = gridDim.x * (kWG / 64), wid = blockIdx.x * (kWG / 64) + wave;
    const int cnt = (wid < ngroups ? (ngroups - wid + nw - 1) / nw : 0) * (EPI == mivi::EPI_CONV ? 3 : 1);  // wave-uniform

    // row of this lane in step s of this wave (steps past the end re-read
    // the wave's last row, and waves without rows read row 0; such rows are
    // never stored). Branch-free, so the waits for the activation loads stay
    // precise: a branch around the prefetch would make the compiler wait for
    // every outstanding weight load before staging x.
    auto row_of = [&](int st) {
        st = st < cnt ? st : cnt - 1;
        if constexpr (EPI == mivi::EPI_SWIGLU) {
            int c = wid + st * nw;
            c = c < 0 ? 0 : c < n0 ? c : n0 - 1;
            return c + sub * n0;
        } else if constexpr (EPI == mivi::EPI_CONV) {
            int c = (wid + (st / 3) * nw) * RPW + sub;
            c = c < 0 ? 0 : c < D3 ? c : D3 - 1;
            return c + (st % 3) * D3;
        } else {
            const int r = (wid + st * nw) * RPW + sub;
            return r < 0 ? 0 : r < n ? r : n - 1;
        }
    };
    Unit<FMT> buf[PD][NU];
    auto load_step = [&](Unit<FMT> (&B)[NU], int st) {
        const uint8_t* row = sg.row(row_of(st));
#pragma unroll
        for (int i = 0; i < NU; i++) {
            if constexpr (PACK) load_unit_q6k_packed(B[i], row, min(lr + LPR * i, units - 1), units);
            else load_unit<FMT>(B[i], row, min(lr + LPR * i, units - 1));
        }
    };
    // activation loads first, then the first PD row groups of weights, which
    // stay in flight while x is staged; with several columns the next
    // column's activations load while the current one is staged
    StageIn<PRO, K / kWG> in[NC > 1 ? 2 : 1];
    float s[NC];
    // (scheduling barriers keep this order: activation loads, weight loads,
    // then the activation math, which then waits for the activations only)
    in[0].load(NC == 1 ? a : gemv_column(a, 0));
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int p = 0; p < PD; p++) load_step(buf[p], p);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (NC == 1) {
        s[0] = in[0].template finish<FMT == FMT_Q4K>(a, dig[0], xsum[0]);
    } else {
#pragma unroll
        for (int c = 0; c < NC; c++) {
            if (c + 1 < ncol) in[(c + 1) & 1].load(gemv_column(a, c + 1));
            if (c < ncol) s[c] = in[c & 1].template finish<FMT == FMT_Q4K>(gemv_column(a, c), dig[c], xsum[c]);
            else s[c] = 0.0f;
        }
    }

    // this lane's activation digits (and their per-quad offsets / fp32
    // sub-block sums), per column, fixed for the launch
    constexpr int NCR = XL ? 1 : NC;  // columns held in registers
    uint32_t xd[NCR][NU][3][16];
    int off[NCR][NU][4][3];
    float X[NCR][NU][2];
    auto fetch_digits = [&](int cc, int i, uint32_t (&d)[3][16], int (&o)[4][3], float (&xs)[2]) {
        const int u = min(lr + LPR * i, units - 1);
        const int b = u >> 2;
        if (FMT == FMT_Q4K) {
            const int g = u & 3;
            const int w0 = (b * 256 + g * 64) / 4;
#pragma unroll
            for (int e = 0; e < 3; e++)
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const u32x4 v = *(const u32x4*)(dig[cc] + e * (K / 4) + w0 + 4 * q);
                    d[e][4 * q] = v.x; d[e][4 * q + 1] = v.y; d[e][4 * q + 2] = v.z; d[e][4 * q + 3] = v.w;
                }
            xs[0] = xsum[cc][b * 8 + 2 * g];
            xs[1] = xsum[cc][b * 8 + 2 * g + 1];
        } else {
            const int h = (u >> 1) & 1, j = u & 1;
            const int e0 = b * 256 + h * 128 + 16 * j;
#pragma unroll
            for (int e = 0; e < 3; e++)
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const u32x4 v = *(const u32x4*)(dig[cc] + e * (K / 4) + (e0 + 32 * q) / 4);
                    d[e][4 * q] = v.x; d[e][4 * q + 1] = v.y; d[e][4 * q + 2] = v.z; d[e][4 * q + 3] = v.w;
                    int t = 0;
                    t = sdot4(v.x, 0x01010101u, t);
                    t = sdot4(v.y, 0x01010101u, t);
                    t = sdot4(v.z, 0x01010101u, t);
                    t = sdot4(v.w, 0x01010101u, t);
                    o[q][e] = -32 * t;
                }
        }
    };
#pragma unroll
    for (int cc = 0; cc < NCR; cc++)
#pragma unroll
    for (int i = 0; i < NU; i++) {
        if constexpr (XL) break;
        const int u = min(lr + LPR * i, units - 1);
        const int b = u >> 2;
        if (FMT == FMT_Q4K) {
            const int g = u & 3;
            const int w0 = (b * 256 + g * 64) / 4;
#pragma unroll
            for (int e = 0; e < 3; e++)
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const u32x4 v = *(const u32x4*)(dig[cc] + e * (K / 4) + w0 + 4 * q);
                    xd[cc][i][e][4 * q] = v.x; xd[cc][i][e][4 * q + 1] = v.y;
                    xd[cc][i][e][4 * q + 2] = v.z; xd[cc][i][e][4 * q + 3] = v.w;
                }
            X[cc][i][0] = xsum[cc][b * 8 + 2 * g];
            X[cc][i][1] = xsum[cc][b * 8 + 2 * g + 1];
        } else {
            const int h = (u >> 1) & 1, j = u & 1;
            const int e0 = b * 256 + h * 128 + 16 * j;
#pragma unroll
            for (int e = 0; e < 3; e++)
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const u32x4 v = *(const u32x4*)(dig[cc] + e * (K / 4) + (e0 + 32 * q) / 4);
                    xd[cc][i][e][4 * q] = v.x; xd[cc][i][e][4 * q + 1] = v.y;
                    xd[cc][i][e][4 * q + 2] = v.z; xd[cc][i][e][4 * q + 3] = v.w;
                    int t = 0;
                    t = sdot4(v.x, 0x01010101u, t);
                    t = sdot4(v.y, 0x01010101u, t);
                    t = sdot4(v.z, 0x01010101u, t);
                    t = sdot4(v.w, 0x01010101u, t);
                    off[cc][i][q][e] = -32 * t;
                }
        }
    }
    // EPI_CONV: the channels' B and C sums between their steps
    float keepB[NC], keepC[NC];
#pragma unroll
    for (int c = 0; c < NC; c++) keepB[c] = keepC[c] = 0.f;
    // EPI_ARGMAX: per column, this lane's maximum and its first row
    float best[NC];
    int bidx[NC];
#pragma unroll
    for (int c = 0; c < NC; c++) { best[c] = -INFINITY; bidx[c] = 0x7FFFFFFF; }
    auto write_part = [&]() {
#pragma unroll
        for (int c = 0; c < NC; c++) {
            if (c >= ncol) break;
            // merge the RPW row groups of the wave (lanes 0, LPR, ...), then
            // lane 0 writes; lanes that hold no row carry (-inf, INT_MAX)
            float bv = best[c];
            int bi = bidx[c];
#pragma unroll
            for (int o = LPR; o < 64; o <<= 1) {
                const float ov = __shfl_xor(bv, o, 64);
                const int oi = __shfl_xor(bi, o, 64);
                if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
            }
            if (lane == 0) {
                a.part_val[c * a.ps + wid] = bv;
                a.part_idx[c * a.ps + wid] = bi;
            }
        }
    };
    if (cnt == 0) {  // wave-uniform; no barrier follows
        if constexpr (EPI == mivi::EPI_ARGMAX) write_part();
        return;
    }

    auto compute = [&](const Unit<FMT> (&B)[NU], int st) {
#pragma unroll
        for (int cc = 0; cc < NC; cc++) {
            if (cc >= ncol) break;
            float acc = 0.f;
#pragma unroll
            for (int i = 0; i < NU; i++) {
                if (lr + LPR * i >= units) continue;
                const int cr = XL ? 0 : cc;
                if constexpr (XL) fetch_digits(cc, i, xd[0][i], off[0][i], X[0][i]);
                if constexpr (FMT == FMT_Q4K)
                    acc += q4k_unit_i8(B[i].hdr, B[i].qa, B[i].qb, (lr + LPR * i) & 3, xd[cr][i], s[cc], X[cr][i][0],
                                       X[cr][i][1]);
                else
                    acc += q6k_unit_i8(B[i].ql0, B[i].ql1, B[i].qh, PACK ? packed_q6k_scales(B[i].sc.x) : B[i].sc,
                                       B[i].d, xd[cr][i], off[cr][i]);
            }
            float sum = xsum_desc<LPR>(acc);  // exact in the lr == 0 lanes that use it
            if (FMT == FMT_Q6K) sum *= s[cc];
            if constexpr (EPI == mivi::EPI_SWIGLU) {
                // lane 0 holds gate c, lane 32 up c (math.rs:87-95)
                const float up = __shfl(sum, 32, 64);
                const int c = wid + st * nw;
                if (lane == 0 && c < n0) *(gfloat*)(sg.out(c) + cc * a.ys) = silu_f(sum) * up;
            } else if constexpr (EPI == mivi::EPI_CONV) {
                // every lane of a row holds its sum: B and C wait in
                // registers for the X step of the same channels
                const int kind = st % 3;
                if (kind == 0) keepB[cc] = sum;
                else if (kind == 1) keepC[cc] = sum;
                else {
                    const int c = (wid + (st / 3) * nw) * RPW + sub;
                    if (lr == 0 && c < D3) conv_epilogue(a, cc, c, keepB[cc], keepC[cc], sum);
                }
            } else {
                const int r = (wid + st * nw) * RPW + sub;
                if (lr == 0 && r < n) {
                    gfloat* y = (gfloat*)(sg.out(r) + cc * a.ys);
                    if (a.accumulate) __builtin_amdgcn_global_atomic_fadd_f32(y, sum);
                    else *y = sum;
                    // sampler.rs:305-316: strictly greater wins, so NaN never does
                    if constexpr (EPI == mivi::EPI_ARGMAX)
                        if (sum > best[cc]) { best[cc] = sum; bidx[cc] = r; }
                }
            }
        }
    };
    // Step st is computed from ring slot st % PD, which is then refilled
    // with step st + PD. Whole rounds of PD steps run without early exits
    // (an exit merging into the loop header would make the compiler wait for
    // every outstanding load); the tail computes the last < PD steps.
    int st = 0;
    for (; st + PD <= cnt; st += PD) {
#pragma unroll
        for (int p = 0; p < PD; p++) {
            compute(buf[p], st + p);
            load_step(buf[p], st + p + PD);
        }
    }
#pragma unroll
    for (int p = 0; p < PD; p++)
        if (st + p < cnt) compute(buf[p], st + p);
    if constexpr (EPI == mivi::EPI_ARGMAX) write_part();
}


// --------------------------------------- batched Q4_K GEMV on the matrix cores
//
// Several activation columns (the sequences of a batched decode step, the
// input rows of a small matmul_rows batch) against Q4_K rows in their GGUF
// layout: up to 8 columns at K = 2048, up to 4 at K = 8192 (blockIdx.y picks
// a group of four columns where a launch holds more). A workgroup is eight
// waves in R = 8 / DQ teams of DQ waves; a team owns 16 rows at a time
// (EPI_SWIGLU: gate rows c..c+7 and up rows c..c+7) and its wave q the q-th
// of DQ slices of their superblocks. Per 32-value sub-block and group G of
// four columns, v_mfma_i32_16x16x32_i8 takes
//   A  row i = 4c' + p: digit plane p of column 4G + c' (a zero plane for
//      p = 3) at the sub-block's 32 k (lane l: row l % 16, k = 8 (l / 16) .. +8),
//   B  the 4-bit codes of the 16 rows (lane l: row l % 16, the low or high
//      nibbles of the 8 code bytes of k = 8 (l / 16) .. +8),
// and lane l receives C[4 (l / 16) + p][l % 16] (p = 0..2): column
// 4G + l / 16, row l % 16, plane p, the exact integer sums of code x digit.
// The lane sums sc x C over the superblock's eight sub-blocks in int32 (one
// 24-bit multiply-add a step) and the min terms m x X in f32, then takes one
// float step per superblock: d s (A0 + A1/256 + A2/65536) - dmin sum m X
// (q4_k_m.rs:144-214). The digits are those of the one-column kernels
// (ColStage), but the one-column kernels take a float step per 64-value unit,
// so a batched column agrees with its one-column GEMV to float rounding, not
// bit for bit. On rows packed by launch_pack_q4k_cols (CW) the scales and
// mins arrive decoded, the eight scales feed a single chain per plane, and
// the min terms run on v_mfma_f32_16x16x16_f16 (the columns' sub-block sums
// as fp16 hi / lo pairs against the rows' mins; see the kernel). Waves 1.. of a team hand
// their partial row sums to wave 0 through LDS. Digits sit in LDS (8 KB per
// column at K = 2048: three planes and the zero plane, padded apart against
// bank conflicts).

constexpr int kColWaves = 8;              // waves of a batched-column workgroup
constexpr int kColWG = 64 * kColWaves;

// One wave's share of the activation staging: part h of P of column c, V =
// K / P consecutive values, lane l holding values 4 (l + 64 i) .. +3 of the
// part (i < V / 256), so every load is one coalesced 1 KB wave access.
// issue() starts the loads; the kernel calls it before its weight prefetch
// so that the in-order completion of loads does not queue the activations
// behind the weights. part() applies the prologue and forms the part's
// max |u|, the NaN flag and (RMSNORM) sum x^2; finish() takes the column's
// totals and writes the digit planes (digits4_b256 of
// Y = rint(u * 127 * 2^15 / max|u|), |Y| < 2^22, so d0 lies in [-64, 64])
// and the fp32 sums of every 32-value sub-block, and returns the digit scale
// s = 2 max|x| / 127 with x ~ s (d0 + d1/256 + d2/65536) (NaN when x holds a
// NaN or an infinity, so the products come out NaN as in fp32). Under
// RMSNORM the digits are taken of u = x * norm_w: the norm's 1 / rms cancels
// in u * 127 / max|u| and only scales s and the sub-block sums. Prologues
// NONE, RMSNORM and CONV (a.x = [B | C | X], ssm.rs:80-140; issue() loads B,
// part() the rest; u = C * conv, the window written back by the column's
// first workgroup).
template <int PRO, int K, int P>
struct ColStage {
    static_assert(PRO != mivi::PRO_SWIGLU, "no SwiGLU prologue here");
    static constexpr int V = K / P, NL = V / 256;
    f32x4 u[NL];
    float t4[NL];  // sums of the lane's four values
    float m = 0.f, ss = 0.f;

    // u[i] holds chunk ch(i) = (i + blockIdx.x) mod NL of the part: the
    // workgroups of an XCD start at different chunks, so their simultaneous
    // first loads spread over the L2 channels instead of all asking one line
    __device__ __forceinline__ int ch(int i) const { return (i + (int)blockIdx.x) & (NL - 1); }
    __device__ __forceinline__ void issue(const mivi::GemvArgs& a, int h) {
        static_assert((NL & (NL - 1)) == 0, "a power of two of chunks");
        const int l = threadIdx.x & 63, o = h * V;
#pragma unroll
        for (int i = 0; i < NL; i++) u[i] = *(const gf32x4*)(a.x + o + 4 * (l + 64 * ch(i)));
    }
    // nwl: RMSNORM's weight vector in LDS (loaded once by the workgroup)
    __device__ __forceinline__ void part(const mivi::GemvArgs& a, int h, const float* nwl = nullptr) {
        const int l = threadIdx.x & 63, o = h * V;
        float nn = 0.f;  // NaN for a NaN value (fmaxf passes it over)
        if constexpr (PRO == mivi::PRO_CONV) {
            const bool swap = a.phase && ((*a.phase) & 1);
            const float* st_in = swap ? a.st_out : a.st_in;
            float* st_out = swap ? (float*)a.st_in : a.st_out;
#pragma unroll
            for (int i = 0; i < NL; i++) {
                const int d0 = o + 4 * (l + 64 * ch(i));  // channels d0 .. d0 + 3
                float st[4 * kConvKs], cw[4 * kConvKs];
#pragma unroll
                for (int q = 0; q < kConvKs; q++) {
                    const f32x4 s4 = *(const gf32x4*)(st_in + (size_t)d0 * kConvKs + 4 * q);
                    st[4 * q] = s4.x; st[4 * q + 1] = s4.y; st[4 * q + 2] = s4.z; st[4 * q + 3] = s4.w;
                    if (a.conv_mode == 0) {
                        const f32x4 w4 = *(const gf32x4*)(a.conv_w + (size_t)d0 * kConvKs + 4 * q);
                        cw[4 * q] = w4.x; cw[4 * q + 1] = w4.y; cw[4 * q + 2] = w4.z; cw[4 * q + 3] = w4.w;
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; e++)
                            cw[4 * q + e] = a.conv_mode == 1 ? a.conv_w[(4 * q + e) % kConvKs] : 1.0f / (float)kConvKs;
                    }
                }
                const f32x4 c4 = *(const gf32x4*)(a.x + a.K + d0), x4 = *(const gf32x4*)(a.x + 2 * a.K + d0);
                const float b[4] = {u[i].x, u[i].y, u[i].z, u[i].w};
                const float cv[4] = {c4.x, c4.y, c4.z, c4.w};
                const float xv[4] = {x4.x, x4.y, x4.z, x4.w};
                float y[4], nst[4 * kConvKs];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float bx = b[e] * xv[e];
                    float conv = 0.0f;
#pragma unroll
                    for (int k = 0; k < kConvKs; k++) {
                        const int q = e * kConvKs + k;
                        const float sv = k + 1 < kConvKs ? st[q + 1] : bx;
                        conv += cw[q] * sv;
                        nst[q] = sv;
                    }
                    y[e] = cv[e] * conv;
                }
                if (blockIdx.x == 0) {
#pragma unroll
                    for (int q = 0; q < kConvKs; q++)
                        *(f32x4*)(st_out + (size_t)d0 * kConvKs + 4 * q) =
                            f32x4{nst[4 * q], nst[4 * q + 1], nst[4 * q + 2], nst[4 * q + 3]};
                }
                u[i] = f32x4{y[0], y[1], y[2], y[3]};
            }
        }
#pragma unroll
        for (int i = 0; i < NL; i++) {
            float x[4] = {u[i].x, u[i].y, u[i].z, u[i].w};
            if constexpr (PRO == mivi::PRO_RMSNORM) {
                const f32x4 w4 = *(const f32x4*)&nwl[o + 4 * (l + 64 * ch(i))];
                const float nw[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    ss = fmaf(x[e], x[e], ss);  // (non-finite x: ss, so s, NaN)
                    x[e] *= nw[e];
                }
            }
#pragma unroll
            for (int e = 0; e < 4; e++) m = fmaxf(m, fabsf(x[e]));
            t4[i] = ((x[0] + x[1]) + x[2]) + x[3];
            if constexpr (PRO != mivi::PRO_RMSNORM) nn = fmaf(t4[i], 0.f, nn);  // a NaN (an infinity is in m)
            u[i] = f32x4{x[0], x[1], x[2], x[3]};
        }
        m += nn;
        if constexpr (PRO == mivi::PRO_RMSNORM) ss = xsum_all64(ss);
        float lo, hi;
        swap32(m, lo, hi);
        m = nanmax(lo, hi);
        swap16(m, lo, hi);
        m = nanmax(lo, hi);
        m = nanmax(m, dpp_mov<0x128>(m));
        m = nanmax(m, xor4_mov(m));
        m = nanmax(m, dpp_mov<0x4E>(m));
        m = nanmax(m, dpp_mov<0xB1>(m));
    }
    // mt, sst: the column's max |u| and sum x^2 over its P parts. HL: the
    // sub-block sums go out as fp16 hi / lo pairs of X / sx (the min-term
    // operands of the packed-row kernel, see gemv_q4k_cols_kernel), sx = the
    // power of two returned in *sxo with |X| / sx < 2^15
    template <int PS, bool HL = false>
    __device__ __forceinline__ float finish(const mivi::GemvArgs& a, int h, float mt, float sst, uint32_t* dig,
                                            float* xsum, float* sxo = nullptr) {
        const int l = threadIdx.x & 63, o = h * V;
        // RMSNORM: x = u / rms (math.rs:7-22); else scale 1
        const float scale = PRO == mivi::PRO_RMSNORM ? 1.0f / sqrtf(sst / (float)K + a.eps) : 1.0f;
        const bool finite = mt > 0.f && mt <= 3.40282347e38f;
        const float mul = finite ? kDigMul / mt : 0.0f;
        const float sc = ((mt - mt) + mt * scale) * (2.0f / 127.0f);
        // |X| <= 32 max|u| scale < 2^e (non-finite or zero: 1; the product
        // is then NaN through sc or zero anyway)
        float inv_sx = 1.0f;
        if constexpr (HL) {
            const float bound = 32.0f * mt * scale;
            int e = 0;
            if (bound > 0.f && bound <= 3.40282347e38f) {
                frexpf(bound, &e);
                e = e < -100 ? -100 : e;
            } else {
                e = 15;
            }
            inv_sx = ldexpf(1.0f, 15 - e);
            if (sxo) *sxo = ldexpf(1.0f, e - 15);
        }
#pragma unroll
        for (int i = 0; i < NL; i++) {
            const int w = (o >> 2) + l + 64 * ch(i);  // the dword of values 4w .. 4w + 3
            const float x[4] = {u[i].x, u[i].y, u[i].z, u[i].w};
            uint32_t w0, w1, w2;
            digits4_b256(x, mul, w0, w1, w2);
            dig[w] = w0;
            dig[PS + w] = w1;
            dig[2 * PS + w] = w2;
            // sub-block sums: eight lanes, xor 1, 2, 4 (the writers, lanes
            // with bit 2 clear, see their exact partners; row_ror:12 reads
            // lane (i + 4) mod 16)
            float t = t4[i];
            t += dpp_mov<0xB1>(t);
            t += dpp_mov<0x4E>(t);
            t += dpp_mov<0x12C>(t);
            if ((l & 7) == 0) {
                if constexpr (HL) {
                    // sub-block q = w >> 3: halves 4 (q >> 1) + (q & 1) (hi)
                    // and + 2 (lo), i.e. per superblock b and lane group kg
                    // of the products: Xhi[2kg], Xhi[2kg+1], Xlo[2kg], Xlo[2kg+1]
                    const float xs = (t * scale) * inv_sx;
                    const _Float16 hi = (_Float16)xs;
                    const _Float16 lo = (_Float16)(xs - (float)hi);
                    _Float16* xh = (_Float16*)xsum;
                    const int q = w >> 3;
                    xh[4 * (q >> 1) + (q & 1)] = hi;
                    xh[4 * (q >> 1) + 2 + (q & 1)] = lo;
                } else {
                    xsum[w >> 3] = t * scale;
                }
            }
        }
        return sc;
    }
};

// Columns [c0, c0 + 4) of a batched launch (blockIdx.y = column group).
__device__ __forceinline__ mivi::GemvArgs gemv_col_group(const mivi::GemvArgs& a, int c0) {
    mivi::GemvArgs v = gemv_column(a, c0);
#pragma unroll
    for (int i = 0; i < 3; i++)  // static indices: the arguments stay in registers
        if (i < a.nseg) v.seg[i].y = a.seg[i].y + c0 * a.ys;
    v.ncol = min(4, a.ncol - c0);
    return v;
}

typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

// WPE: waves per SIMD the launch places (2: one workgroup per CU, whose
// waves may then take up to 256 registers; 4: two workgroups per CU)
template <int PRO, int EPI, int KT, int NG, int DQ, int KS = 1, bool CW = false, int WPE = 2>
__global__ void __launch_bounds__(kColWG) __attribute__((amdgpu_waves_per_eu(2, WPE))) gemv_q4k_cols_kernel(const mivi::GemvArgs a0) {
    static_assert(KT == 1024 || KT == 2048 || KT == 8192, "decode depths (per K split)");
    static_assert(DQ == 4 || DQ == 8, "depth slices per team");
    // KS > 1: the depth a0.K = KS * KT in KS slices, slice blockIdx.y; the
    // workgroup stages and reads only its slice and adds its partial sums
    // into y (the residual add: other slices add theirs)
    static_assert(KS == 1 || (PRO == mivi::PRO_NONE && EPI == mivi::EPI_STORE), "K splits: products added into y");
    // NG = 1 launched with several column groups (KS = 1): column group
    // blockIdx.y, at most four columns
    const mivi::GemvArgs a = (KS == 1 && NG == 1 && gridDim.y > 1) ? gemv_col_group(a0, 4 * (int)blockIdx.y) : a0;
    const int ks = KS > 1 ? (int)blockIdx.y : 0;
    constexpr int K = KT, nb = K / 256;
    constexpr int R = kColWaves / DQ;       // teams
    constexpr int SQ = nb / DQ;             // superblocks per wave and group: 1, 2 or 4
    // U group steps' chunks in flight per wave, all of a step's SQ (more, the
    // weights then loaded whole at the start, delays the activations)
    constexpr int U = 1;
    constexpr int PD = SQ * U;
    static_assert(PD <= 4, "ring of at most four superblock chunks");
    constexpr int NCM = 4 * NG;
    constexpr int P = kColWaves / NCM;      // staging parts per column (one per wave)
    constexpr int PS = K / 4 + 4;           // digit plane stride (dwords)
    __shared__ __attribute__((aligned(16))) uint32_t dig[NCM][4 * PS];
    __shared__ __attribute__((aligned(16))) float xsum[NCM][K / 32];
    __shared__ float scol[NCM];
    __shared__ float sxc[CW ? NCM : 1];     // CW: the columns' min-term scales sx
    __shared__ float red[2][NCM][P];        // parts' max |u| and sum x^2
    __shared__ float xq[R][2][DQ - 1][NG][64];  // waves 1.. -> wave 0 of a team, by group-step parity
    // RMSNORM: the weight vector, loaded once for the workgroup's columns
    __shared__ __attribute__((aligned(16))) float nwl[PRO == mivi::PRO_RMSNORM ? K : 4];
    const Segs sg(a, (size_t)nb * KS * 144);
    const int n = sg.n, n0 = a.seg[0].n;
    const int ncol = a.ncol;  // 1..NCM, workgroup-uniform
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int team = wave / DQ, wq = wave % DQ;
    const int j = lane & 15, kg = lane >> 4;
    // EPI_CONV: a group holds channels 5g .. 5g+4, lane row j = 3i + k their
    // B, C, X rows (k = 0, 1, 2); lane row 15 repeats row 14 and is not stored
    static_assert(EPI != mivi::EPI_CONV || KT == 2048, "the conv epilogue is the K = 2048 in_proj");
    const int ngroups = mivi::cols_groups(EPI, n0, n);
    // group steps (workgroup-uniform): team t takes group
    // blockIdx.x + (st R + t) gridDim.x in step st
    const int stride = R * (int)gridDim.x;
    const int cnt = (int)blockIdx.x < ngroups ? (ngroups - (int)blockIdx.x + stride - 1) / stride : 0;

    // row of lane row j in group step st (-1: none; loads then use row 0)
    auto row_of = [&](int st) {
        const int grp = (int)blockIdx.x + (st * R + team) * (int)gridDim.x;
        return mivi::cols_group_row(EPI, grp, j, n0, n);
    };
    // the activations first (see ColStage), then the weight ring
    const int task_c = wave / P, task_h = wave % P;  // this wave's column and part
    const bool stager = task_c < ncol;               // wave-uniform
    ColStage<PRO, K, P> stg;
    mivi::GemvArgs ax = a;  // the staged slice
    if constexpr (KS > 1) ax.x = a.x + ks * KT;
    static_assert(PRO != mivi::PRO_RMSNORM || K == 4 * kColWG, "one norm weight quad per thread");
    f32x4 nw4;
    if constexpr (PRO == mivi::PRO_RMSNORM) nw4 = *(const gf32x4*)(a.norm_w + 4 * threadIdx.x);
    if (stager) stg.issue(gemv_column(ax, task_c), task_h);
    // ring of superblock chunks: this wave's superblock bb of step st in slot
    // (st mod U) SQ + bb. Every load is unconditional (a step past the last
    // one re-reads the last): a branch around a load makes the compiler wait
    // for it before the next chunk's use, a memory latency per superblock.
    u32x4 hdr[PD];
    uint32_t mxr[CW ? PD : 1];  // CW: mins m4..m7 of row j
    u32x2 cq[PD][4];
    auto load = [&](int slot, int st, int bb) {
        st = st < cnt ? st : cnt - 1;
        if constexpr (CW) {
            // launch_pack_q4k_cols layout: group grp's chunk of this superblock
            int grp = (int)blockIdx.x + ((st < 0 ? 0 : st) * R + team) * (int)gridDim.x;
            grp = grp < ngroups ? grp : ngroups - 1;
            const uint8_t* p = a.cw + ((size_t)grp * (nb * KS) + ks * nb + wq * SQ + bb) * mivi::kColsChunkBytes;
            hdr[slot] = ldg16(p + 16 * j);
            mxr[slot] = *(const __attribute__((address_space(1))) uint32_t*)(p + mivi::kColsMinsOff + 4 * j);
            const u32x4 c0 = ldg16(p + mivi::kColsCodesOff + 16 * lane);
            const u32x4 c1 = ldg16(p + mivi::kColsCodesOff + 1024 + 16 * lane);
            cq[slot][0] = u32x2{c0.x, c0.y};
            cq[slot][1] = u32x2{c0.z, c0.w};
            cq[slot][2] = u32x2{c1.x, c1.y};
            cq[slot][3] = u32x2{c1.z, c1.w};
        } else {
            const int r = row_of(st < 0 ? 0 : st);
            const uint8_t* p = sg.row(r < 0 ? 0 : r) + 144 * (ks * nb + wq * SQ + bb);
            hdr[slot] = ldg16(p);
#pragma unroll
            for (int g = 0; g < 4; g++)
                cq[slot][g] = *(const __attribute__((address_space(1))) u32x2*)(p + 16 + 32 * g + 8 * kg);
        }
    };
#pragma unroll
    for (int q = 0; q < PD; q++) load(q, q / SQ, q % SQ);
    // EPI_CONV: the first group step's conv windows and weights (wave 0 of a
    // team, lanes j = 3i < 15 of each column), loaded with the weights so the
    // epilogue waits for no memory
    ConvPre cpre0[EPI == mivi::EPI_CONV ? NG : 1];
    if constexpr (EPI == mivi::EPI_CONV) {
        const int r0 = row_of(0);
#pragma unroll
        for (int G = 0; G < NG; G++)
            if (wq == 0 && cnt > 0 && j < 15 && j % 3 == 0 && r0 >= 0 && 4 * G + kg < ncol)
                conv_prefetch(a, 4 * G + kg, r0, cpre0[G]);
    }
    // the zero plane of every column
#pragma unroll
    for (int c = 0; c < NCM; c++)
        for (int i = threadIdx.x; i < PS / 4; i += kColWG) *(u32x4*)&dig[c][3 * PS + 4 * i] = u32x4{0u, 0u, 0u, 0u};
    if constexpr (PRO == mivi::PRO_RMSNORM) {
        *(f32x4*)&nwl[4 * threadIdx.x] = nw4;
        __syncthreads();
    }
    if (stager) stg.part(gemv_column(ax, task_c), task_h, nwl);
    if constexpr (P > 1) {
        if (stager && lane == 0) {
            red[0][task_c][task_h] = stg.m;
            red[1][task_c][task_h] = stg.ss;
        }
        __syncthreads();
    }
    if (stager) {
        float mt = stg.m, sst = stg.ss;
        if constexpr (P > 1) {
            mt = red[0][task_c][0];
            sst = red[1][task_c][0];
#pragma unroll
            for (int h = 1; h < P; h++) {
                mt = nanmax(mt, red[0][task_c][h]);
                sst += red[1][task_c][h];
            }
        }
        const float sc = stg.template finish<PS, CW>(gemv_column(ax, task_c), task_h, mt, sst, dig[task_c],
                                                      xsum[task_c], (lane == 0 && task_h == 0) ? &sxc[task_c] : nullptr);
        if (lane == 0 && task_h == 0) scol[task_c] = sc;
    }
    __syncthreads();
    if (cnt == 0) return;  // workgroup-uniform
    float s[NG], sx[NG];
#pragma unroll
    for (int G = 0; G < NG; G++) {
        s[G] = scol[min(4 * G + kg, ncol - 1)];
        sx[G] = CW ? sxc[min(4 * G + kg, ncol - 1)] : 0.f;
    }
    // CW min-term product (v_mfma_f32_16x16x16_f16): A row i = j = 4q + t is
    // column 4t + q (rows of t >= NG or past ncol repeat a column; their
    // outputs are not used), its k-group kg the fp16 pairs
    // Xhi[2kg], Xhi[2kg+1], Xlo[2kg], Xlo[2kg+1] of a superblock; B column j
    // the mins m[2kg], m[2kg+1], m[2kg], m[2kg+1] of row j. Lane (j, kg)
    // receives D[4kg + G][j] = sum over the superblock of m X / sx for row j
    // and column 4G + kg. msel picks bytes 2kg, 2kg+1 of {mins m4..m7 : m0..m3}.
    const _Float16* xhA = (const _Float16*)xsum[min(4 * (j & 3) + (j >> 2), ncol - 1)] + 4 * kg;
    const uint32_t msel = (uint32_t)(2 * kg) | (uint32_t)(2 * kg + 1) << 8 | 0x0C0C0000u;
    const int ci = j >> 2, pi = j & 3;  // A operand of this lane: column 4G + ci, plane pi
    const uint32_t* dA[NG];
#pragma unroll
    for (int G = 0; G < NG; G++) dA[G] = dig[min(4 * G + ci, ncol - 1)] + pi * PS + 2 * kg;

    // group step st from slots s0 .. s0 + SQ - 1; REFILL: reload them with
    // step st + U's chunks
    auto step = [&](const int st, const int s0, auto refill) {
        // this wave's superblocks of the group, each summed in int32 over its
        // four units before the float steps
        float part[NG], pm[NG];
#pragma unroll
        for (int G = 0; G < NG; G++) part[G] = pm[G] = 0.f;
#pragma unroll
        for (int bb = 0; bb < SQ; bb++) {
            const int slot = s0 + bb, b = wq * SQ + bb;
            const u32x4 h = hdr[slot];
            u32x2 q[4];
#pragma unroll
            for (int g = 0; g < 4; g++) q[g] = cq[slot][g];
            if constexpr (CW) {
                // packed header: h.x = d | dmin << 16, h.y, h.z the scales
                // sc0..sc7 as bytes, h.w and mxr the mins m0..m7 as bytes
                const uint32_t mx = mxr[slot];
                if constexpr (decltype(refill)::value) load(slot, st + U, bb);
                const float d = half_bits_to_f32(h.x), dmin = half_bits_to_f32(h.x >> 16);
                const uint32_t mp = __builtin_amdgcn_perm(mx, h.w, msel);
                const float ma = (float)(mp & 0xFFu), mb = (float)((mp >> 8) & 0xFFu);
                const f16x4 Bm = {(_Float16)ma, (_Float16)mb, (_Float16)ma, (_Float16)mb};
                const f16x4 Ax = *(const f16x4*)(xhA + 16 * b);
                const f32x4 Dm = __builtin_amdgcn_mfma_f32_16x16x16f16(Ax, Bm, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                // the eight 6-bit scales, each extracted once (a byte select
                // folded into every multiply costs a multiply and an add per
                // product instead of one v_mad_i32_i24)
                int scs[8];
#pragma unroll
                for (int k = 0; k < 8; k++) scs[k] = (int)(((k < 4 ? h.y : h.z) >> (8 * (k & 3))) & 63u);
                // every digit operand of the superblock from LDS, then every
                // product, then the scale chains: the LDS and matrix-core
                // latencies overlap instead of adding up per sub-block pair
                long Al[4][NG], Ah[4][NG];
#pragma unroll
                for (int g = 0; g < 4; g++)
#pragma unroll
                    for (int G = 0; G < NG; G++) {
                        const int w0 = (256 * b + 64 * g) / 4;
                        const u32x2 alo = *(const u32x2*)(dA[G] + w0);
                        const u32x2 ahi = *(const u32x2*)(dA[G] + w0 + 8);
                        Al[g][G] = (long)(((uint64_t)alo.y << 32) | alo.x);
                        Ah[g][G] = (long)(((uint64_t)ahi.y << 32) | ahi.x);
                    }
                i32x4 Dl[4][NG], Dh[4][NG];
#pragma unroll
                for (int g = 0; g < 4; g++) {
                    const long blo = (long)(((uint64_t)(q[g].y & 0x0F0F0F0Fu) << 32) | (q[g].x & 0x0F0F0F0Fu));
                    const long bhi = (long)(((uint64_t)((q[g].y >> 4) & 0x0F0F0F0Fu) << 32) | ((q[g].x >> 4) & 0x0F0F0F0Fu));
                    const i32x4 z = {0, 0, 0, 0};
#pragma unroll
                    for (int G = 0; G < NG; G++) {
                        Dl[g][G] = __builtin_amdgcn_mfma_i32_16x16x32_i8(Al[g][G], blo, z, 0, 0, 0);
                        Dh[g][G] = __builtin_amdgcn_mfma_i32_16x16x32_i8(Ah[g][G], bhi, z, 0, 0, 0);
                    }
                }
                // one chain per plane over the superblock's eight sub-blocks:
                // |D| < 2^16, sc < 64, below 2^31 (exact)
                int Ac[NG][3];
#pragma unroll
                for (int g = 0; g < 4; g++)
#pragma unroll
                    for (int G = 0; G < NG; G++)
#pragma unroll
                        for (int e = 0; e < 3; e++) {
                            Ac[G][e] = g == 0 ? mul24(Dl[g][G][e], scs[2 * g]) : mad24(Dl[g][G][e], scs[2 * g], Ac[G][e]);
                            asm("" : "+v"(Ac[G][e]));
                            Ac[G][e] = mad24(Dh[g][G][e], scs[2 * g + 1], Ac[G][e]);
                            asm("" : "+v"(Ac[G][e]));
                        }
#pragma unroll
                for (int G = 0; G < NG; G++) {
                    // q4_k_m.rs:144-214 per superblock: d s sum sc (q . x~/s),
                    // and the min term dmin sum m X / sx, taken off at the end
                    const float f = fmaf((float)Ac[G][2], kDig2, fmaf((float)Ac[G][1], kDig1, (float)Ac[G][0]));
                    part[G] = fmaf(d * s[G], f, part[G]);
                    pm[G] = fmaf(dmin, Dm[G], pm[G]);
                }
                continue;
            }
            if constexpr (decltype(refill)::value) load(slot, st + U, bb);
            const float d = half_bits_to_f32(h.x), dmin = half_bits_to_f32(h.x >> 16);
            int AL[NG][3], AH[NG][3];  // low- and high-nibble sub-blocks, one product per step
            float Mac[NG];
#pragma unroll
            for (int G = 0; G < NG; G++) {
                AL[G][0] = AL[G][1] = AL[G][2] = AH[G][0] = AH[G][1] = AH[G][2] = 0;
                Mac[G] = 0.f;
            }
#pragma unroll
            for (int g = 0; g < 4; g++) {
                uint32_t sc0, m0, sc1, m1;
                q4k_scales(h.y, h.z, h.w, g, sc0, m0, sc1, m1);
                const float m0f = (float)m0, m1f = (float)m1;
                const long blo = (long)(((uint64_t)(q[g].y & 0x0F0F0F0Fu) << 32) | (q[g].x & 0x0F0F0F0Fu));
                const long bhi = (long)(((uint64_t)((q[g].y >> 4) & 0x0F0F0F0Fu) << 32) | ((q[g].x >> 4) & 0x0F0F0F0Fu));
#pragma unroll
                for (int G = 0; G < NG; G++) {
                    const int w0 = (256 * b + 64 * g) / 4;
                    const u32x2 alo = *(const u32x2*)(dA[G] + w0);
                    const u32x2 ahi = *(const u32x2*)(dA[G] + w0 + 8);
                    long al = (long)(((uint64_t)alo.y << 32) | alo.x);
                    long ah = (long)(((uint64_t)ahi.y << 32) | ahi.x);
                    const i32x4 z = {0, 0, 0, 0};
                    const i32x4 Dl = __builtin_amdgcn_mfma_i32_16x16x32_i8(al, blo, z, 0, 0, 0);
                    const i32x4 Dh = __builtin_amdgcn_mfma_i32_16x16x32_i8(ah, bhi, z, 0, 0, 0);
                    // |D| <= 32 * 15 * 128 < 2^16, sc < 64: the superblock sum
                    // stays below 8 * 2^22 < 2^31 (exact)
#pragma unroll
                    for (int e = 0; e < 3; e++) {
                        AL[G][e] = mad24(Dl[e], (int)sc0, AL[G][e]);
                        AH[G][e] = mad24(Dh[e], (int)sc1, AH[G][e]);
                        // keep each step one v_mad_i32_i24 (not re-associated
                        // into multiplies and three-input adds)
                        asm("" : "+v"(AL[G][e]), "+v"(AH[G][e]));
                    }
                    const int cl = min(4 * G + kg, ncol - 1);
                    const float2 X = *(const float2*)&xsum[cl][b * 8 + 2 * g];
                    Mac[G] = fmaf(m1f, X.y, fmaf(m0f, X.x, Mac[G]));
                }
            }
#pragma unroll
            for (int G = 0; G < NG; G++) {
                // q4_k_m.rs:144-214 per superblock: d * s * sum sc * (q . x~/s) - dmin * sum m * X
                const float f = fmaf((float)(AL[G][2] + AH[G][2]), kDig2,
                                     fmaf((float)(AL[G][1] + AH[G][1]), kDig1, (float)(AL[G][0] + AH[G][0])));
                part[G] += (d * s[G]) * f - dmin * Mac[G];
            }
        }
        if constexpr (CW) {
#pragma unroll
            for (int G = 0; G < NG; G++) part[G] = fmaf(-sx[G], pm[G], part[G]);
        }
        // the team's DQ slices of the depth, summed by its wave 0 in slice
        // order (one LDS exchange; the buffer alternates with the step's parity)
        if (wq > 0) {
#pragma unroll
            for (int G = 0; G < NG; G++) xq[team][st & 1][wq - 1][G][lane] = part[G];
        }
        __syncthreads();
        if (wq == 0) {
            const int r = row_of(st);
#pragma unroll
            for (int G = 0; G < NG; G++) {
                float v = part[G];
#pragma unroll
                for (int i = 0; i < DQ - 1; i++) v += xq[team][st & 1][i][G][lane];
                const int cc = 4 * G + kg;
                if constexpr (EPI == mivi::EPI_SWIGLU) {
                    // lanes j < 8: gate c; lanes j + 8: up c (math.rs:87-95)
                    const float up = __shfl(v, lane + 8, 64);
                    if (j < 8 && r >= 0 && cc < ncol) *(gfloat*)(sg.out(r) + cc * a.ys) = silu_f(v) * up;
                } else if constexpr (EPI == mivi::EPI_CONV) {
                    // lanes j = 3i hold B of channel 5g + i, j + 1 its C, j + 2 its X
                    const float cv = __shfl(v, lane + 1, 64), xv = __shfl(v, lane + 2, 64);
                    if (j < 15 && j % 3 == 0 && r >= 0 && cc < ncol) {
                        if (st == 0) conv_finish(a, cc, r, v, cv, xv, cpre0[G]);
                        else conv_epilogue(a, cc, r, v, cv, xv);
                    }
                } else {
                    if (r >= 0 && cc < ncol) {
                        gfloat* y = (gfloat*)(sg.out(r) + cc * a.ys);
                        if (KS > 1 || a.accumulate) __builtin_amdgcn_global_atomic_fadd_f32(y, v);
                        else *y = v;
                    }
                }
            }
        }
    };
    // blocks of U steps: every block but the last refills the ring with the
    // next block's chunks; the last one (its steps up to cnt) loads nothing
    const int nblk = (cnt + U - 1) / U;
    for (int blk = 0; blk + 1 < nblk; blk++) {
#pragma unroll
        for (int u = 0; u < U; u++) step(blk * U + u, u * SQ, std::true_type{});
    }
#pragma unroll
    for (int u = 0; u < U; u++) {
        const int st = (nblk - 1) * U + u;
        if (st < cnt) step(st, u * SQ, std::false_type{});  // workgroup-uniform
    }
}

// Launch of the batched kernel over ngr row groups and gy column groups:
// two teams of four waves a workgroup (DQ = 4) where the groups fill 1.5
// workgroups per CU at K = 2048, else one team of eight (DQ = 8); at most one
// workgroup per CU and column group, whose staging its waves then share
// (two column groups may then place two workgroups on a CU).
template <int PRO, int EPI, int KT, int NG>
void launch_cols(const mivi::GemvArgs& a, int ngr, int gy, hipStream_t s) {
    const int cus = mivi::num_cus();
    auto go = [&](auto dq, int gc) {
        constexpr int DQ = decltype(dq)::value;
        const dim3 grid(gc, gy);
        if (NG == 1 && (size_t)gc * gy > (size_t)cus) {
            if constexpr (NG == 1) {
                if (a.cw)
                    hipLaunchKernelGGL((gemv_q4k_cols_kernel<PRO, EPI, KT, NG, DQ, 1, true, 4>), grid, dim3(kColWG), 0, s, a);
                else
                    hipLaunchKernelGGL((gemv_q4k_cols_kernel<PRO, EPI, KT, NG, DQ, 1, false, 4>), grid, dim3(kColWG), 0, s, a);
            }
        } else if (a.cw) {
            hipLaunchKernelGGL((gemv_q4k_cols_kernel<PRO, EPI, KT, NG, DQ, 1, true>), grid, dim3(kColWG), 0, s, a);
        } else {
            hipLaunchKernelGGL((gemv_q4k_cols_kernel<PRO, EPI, KT, NG, DQ>), grid, dim3(kColWG), 0, s, a);
        }
    };
    if constexpr (KT == 2048) {
        if (2 * ngr >= 3 * cus) {
            go(std::integral_constant<int, 4>{}, std::max(1, std::min((ngr + 1) / 2, cus)));
            return;
        }
    }
    go(std::integral_constant<int, 8>{}, std::max(1, std::min(ngr, cus)));
}

// Products added into y (the residual adds: the FFN down projection at K =
// 8192, the attention and ShortConv output projections at K = 2048) in KS
// slices of the depth KFULL: KS workgroups per row group, each staging only
// its slice of the columns (at KS = 8 one eighth of the activation bytes,
// which bound the unsplit launch) and adding its partial sums into y. Two
// teams of four waves a workgroup; gc row-group workgroups per slice, a
// multiple of 8, so that a row group's slices share an XCD.
template <int KFULL, int KS, int NG>
void launch_cols_ksplit(const mivi::GemvArgs& a, int ngr, hipStream_t s) {
    constexpr int KT = KFULL / KS;
    const int cus = mivi::num_cus();
    int gc = std::min((ngr + 1) / 2, std::max(8, cus / KS));
    gc = std::max(8, gc / 8 * 8);
    if (a.cw)
        hipLaunchKernelGGL((gemv_q4k_cols_kernel<mivi::PRO_NONE, mivi::EPI_STORE, KT, NG, 4, KS, true>), dim3(gc, KS),
                           dim3(kColWG), 0, s, a);
    else
        hipLaunchKernelGGL((gemv_q4k_cols_kernel<mivi::PRO_NONE, mivi::EPI_STORE, KT, NG, 4, KS>), dim3(gc, KS),
                           dim3(kColWG), 0, s, a);
}

// ------------------------------------------ Q6_K row quads on the matrix cores
//
// Packed Q6_K matrices with K = 2048 and a multiple of 4 rows
// (mivi_hip_pack_weights) are stored as row quads: quad Q (rows 4Q .. 4Q+3)
// is 6720 contiguous bytes laid out for the 64 lanes l = 4b + j of one wave
// (j = row of the quad, b = 0..15). Lane (b, j) owns units b and b + 16 of row
// j, the units a lane of the unit-plane kernel owns at 16 lanes per row (unit
// u: superblock u/4, half (u/2)&1, values 16(u&1) .. +16 of each quarter
// q = 0..3 of the half, q6_k.rs:8-43). Slot g = 4i + q is quarter q of the
// lane's unit i: sixteen 6-bit codes c_0..c_15 with scale sc[8h + (u&1) + 2q].
// Offsets below are from o = 64 for odd Q (0 for even Q):
//   [0, 6144)     codes, 16 B per lane at 1024 k + 16 l (k = 0..5). Slot g is
//                 dwords 3g .. 3g+2 of the lane's 24: byte e of dword 3g+m
//                 holds c_{4m+e} in bits 0-5 and bits 2m, 2m+1 of c_{12+e} in
//                 bits 6-7, so the four dwords of codes unpack in 9 operations.
//   [6144, 6656)  8 B per lane at 6144 + 8 l: the scale of slot g in byte g
// and the 64 bytes of d, 4 B per (row j, superblock s < 4) at 4 (4 j + s) (the
// fp16 d of superblock s, then of superblock s + 4), follow at 6656 for even
// Q and lead at 0 for odd Q. A quad is 4 x 1680 = 52.5 lines of 128 B, so the
// odd quads start half a line in; with their d first, every 1 KB wave load of
// codes and every scale load is line-aligned, and the d regions of quads 2P
// and 2P + 1 share one line. A packed matrix keeps the GGUF matrix's size.
//
// The products run on v_mfma_i32_4x4x4_16b_i8 (16 independent 4 x 4 x 4
// blocks; block b is lanes 4b .. 4b+3): lane 4b+v supplies row v of A, the
// digit plane v of x (v = 0..2; zeros for v = 3) at the block's four k, and
// lane 4b+j supplies column j of B, four codes of row j, so lane 4b+j
// receives D[v] = sum over k of digit_v * code for its own row. Four
// instructions cover a slot; the chain starts from T = -32 * (sum of the
// slot's digits of plane v), the Q6_K offset. The integer sums are those of
// the sdot4 kernel, the per-unit float steps and the cross-lane reduction run
// in the same order, so the result equals the unit-plane kernel's bit for bit.

constexpr int kQuadBytes = 6720;

// v summed over b for lanes 4b + j: b xor 8, 4, 2, 1 in that order (lane xor
// 32, 16, 8, 4), exact in lanes 0-3, which hold the four rows' sums
__device__ __forceinline__ float quad_lane_sum(float v) {
    float a, b;
    swap32(v, a, b);
    v = a + b;
    swap16(v, a, b);
    v = a + b;
    v += dpp_mov<0x128>(v);  // row_ror:8   (lane ^ 8)
    v += dpp_mov<0x12C>(v);  // row_ror:12  (lane ^ 4 for lanes 0-3)
    return v;
}


__device__ __forceinline__ i32x4 mfma4x4(uint32_t a, uint32_t b, i32x4 c) {
    return __builtin_amdgcn_mfma_i32_4x4x4i8((int)a, (int)b, c, 0, 0, 0);
}

// (through a global-address-space pointer: a flat load would also count
// against the LDS counter, so every LDS wait would wait for it)
__device__ __forceinline__ u32x4 ldg16_nt(const uint8_t* p) {
    return __builtin_nontemporal_load((const __attribute__((address_space(1))) u32x4*)p);
}

// the 6-bit code of value 128h + 32q + l of the Q6_K superblock at blk (q6_k.rs:8-43, before the -32)
__device__ __forceinline__ uint32_t q6_code(const uint8_t* blk, int h, int q, int l) {
    const uint8_t* ql = blk + 64 * h;
    const uint8_t* qh = blk + 128 + 32 * h;
    uint32_t lo = (q & 1) ? ql[l + 32] : ql[l];
    lo = (q & 2) ? (lo >> 4) : (lo & 0xFu);
    return lo | (((uint32_t)(qh[l] >> (2 * q)) & 3u) << 4);
}

// NC columns (sequences) against the same quads, as the stream kernel's
// batched columns; PD row quads in flight per wave.
template <int PRO, int EPI, int NC, int PD>
__global__ void __launch_bounds__(kWG) gemv_q6k_quad_kernel(const mivi::GemvArgs a) {
    constexpr int K = 2048;
    __shared__ __attribute__((aligned(16))) uint32_t dig[NC][3 * K / 4];
    __shared__ i32x4 tl[NC > 1 ? NC : 1][8][16];  // NC > 1: offset tuples per column, slot, block
    const int nquads = a.seg[0].n / 4;
    const uint8_t* W = a.seg[0].W;
    const int ncol = NC == 1 ? 1 : a.ncol;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int b = lane >> 2, jv = lane & 3;
    const int nw = gridDim.x * (kWG / 64), wid = blockIdx.x * (kWG / 64) + wave;
    const int cnt = wid < nquads ? (nquads - wid + nw - 1) / nw : 0;  // wave-uniform

    u32x4 w[PD][6];
    u32x2 scw[PD];
    uint32_t dw[PD];
    // quad of step st (steps past the end re-read the wave's last quad and
    // waves without quads read quad 0; nothing is stored for them)
    auto load = [&](int p, int st) {
        st = st < cnt ? st : cnt - 1;
        int q = wid + st * nw;
        q = q < 0 ? 0 : q < nquads ? q : nquads - 1;
        const uint8_t* base = W + (size_t)q * kQuadBytes;
        const uint8_t* cb = base + 64 * (q & 1);  // codes and scales
        const uint8_t* db = base + ((q & 1) ? 0 : 6656);
#pragma unroll
        for (int k = 0; k < 6; k++) w[p][k] = ldg16_nt(cb + 1024 * k + 16 * lane);
        scw[p] = *(const __attribute__((address_space(1))) u32x2*)(cb + 6144 + 8 * lane);
        dw[p] = *(const __attribute__((address_space(1))) uint32_t*)(db + 4 * (4 * jv + (b >> 2)));
    };
    // activation loads, then the first PD quads, then the activation math
    StageIn<PRO, K / kWG> in[NC > 1 ? 2 : 1];
    float s[NC];
    in[0].load(NC == 1 ? a : gemv_column(a, 0));
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int p = 0; p < PD; p++) load(p, p);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (NC == 1) {
        s[0] = in[0].template finish<false>(a, dig[0], nullptr);
    } else {
#pragma unroll
        for (int c = 0; c < NC; c++) {
            if (c + 1 < ncol) in[(c + 1) & 1].load(gemv_column(a, c + 1));
            if (c < ncol) s[c] = in[c & 1].template finish<false>(gemv_column(a, c), dig[c], nullptr);
            else s[c] = 0.0f;
        }
    }
    // A operands: plane jv of the digits at the slot's k (lanes jv = 3: zeros)
    uint32_t A[NC][32];
#pragma unroll
    for (int c = 0; c < NC; c++)
#pragma unroll
        for (int g = 0; g < 8; g++) {
            const int u = b + 16 * (g >> 2), q = g & 3;
            const int base = 64 * (u >> 2) + 32 * ((u >> 1) & 1) + 8 * q + 4 * (u & 1);
            u32x4 t = *(const u32x4*)(dig[c] + (jv < 3 ? jv : 0) * (K / 4) + base);
            if (jv == 3) t = u32x4{0, 0, 0, 0};
            A[c][4 * g] = t.x; A[c][4 * g + 1] = t.y; A[c][4 * g + 2] = t.z; A[c][4 * g + 3] = t.w;
        }
    // offset tuples T[g] = -32 * (sum of the slot's 16 digits of plane v), by
    // the same instruction against codes of -32 (0xE0)
    i32x4 T[NC == 1 ? 8 : 1];
#pragma unroll
    for (int c = 0; c < NC; c++)
#pragma unroll
        for (int g = 0; g < 8; g++) {
            i32x4 t = {0, 0, 0, 0};
#pragma unroll
            for (int m = 0; m < 4; m++) t = mfma4x4(A[c][4 * g + m], 0xE0E0E0E0u, t);
            if constexpr (NC == 1) T[g] = t;
            else if (wave == 0 && jv == 0) tl[c][g][b] = t;
        }
    if constexpr (NC > 1) __syncthreads();

    float best[NC];
    int bidx[NC];
#pragma unroll
    for (int c = 0; c < NC; c++) { best[c] = -INFINITY; bidx[c] = 0x7FFFFFFF; }
    auto write_part = [&]() {
#pragma unroll
        for (int c = 0; c < NC; c++) {
            if (c >= ncol) break;
            // rows of the wave's steps sit in lanes 0..3; others carry (-inf, INT_MAX)
            float bv = best[c];
            int bi = bidx[c];
#pragma unroll
            for (int o = 1; o < 4; o <<= 1) {
                const float ov = __shfl_xor(bv, o, 64);
                const int oi = __shfl_xor(bi, o, 64);
                if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
            }
            if (lane == 0) {
                a.part_val[c * a.ps + wid] = bv;
                a.part_idx[c * a.ps + wid] = bi;
            }
        }
    };
    if (cnt == 0) {  // wave-uniform; no barrier follows
        if constexpr (EPI == mivi::EPI_ARGMAX) write_part();
        return;
    }

    auto compute = [&](int p, int st) {
        int acc[NC][2][3];
#pragma unroll
        for (int g = 0; g < 8; g++) {
            const int D0 = 3 * g;
            const uint32_t W0 = w[p][D0 >> 2][D0 & 3];
            const uint32_t W1 = w[p][(D0 + 1) >> 2][(D0 + 1) & 3];
            const uint32_t W2 = w[p][(D0 + 2) >> 2][(D0 + 2) & 3];
            const uint32_t B0 = W0 & 0x3F3F3F3Fu, B1 = W1 & 0x3F3F3F3Fu, B2 = W2 & 0x3F3F3F3Fu;
            const uint32_t B3 = ((W0 >> 6) & 0x03030303u) | ((W1 >> 4) & 0x0C0C0C0Cu) | ((W2 >> 2) & 0x30303030u);
            const int scv = __builtin_amdgcn_sbfe((int)(g < 4 ? scw[p].x : scw[p].y), 8 * (g & 3), 8);
#pragma unroll
            for (int c = 0; c < NC; c++) {
                if (c >= ncol) break;
                i32x4 D;
                if constexpr (NC == 1) D = T[g];
                else D = tl[c][g][b];
                D = mfma4x4(A[c][4 * g], B0, D);
                D = mfma4x4(A[c][4 * g + 1], B1, D);
                D = mfma4x4(A[c][4 * g + 2], B2, D);
                D = mfma4x4(A[c][4 * g + 3], B3, D);
                // |D| < 2^18, |A| < 2^26: exact 24-bit multiplies (as q6k_unit_i8)
                const int i = g >> 2;
                if ((g & 3) == 0) {
                    acc[c][i][0] = mul24(D[0], scv);
                    acc[c][i][1] = mul24(D[1], scv);
                    acc[c][i][2] = mul24(D[2], scv);
                } else {
                    acc[c][i][0] += mul24(D[0], scv);
                    acc[c][i][1] += mul24(D[1], scv);
                    acc[c][i][2] += mul24(D[2], scv);
                }
            }
        }
        const int r = 4 * (wid + st * nw) + jv;
#pragma unroll
        for (int c = 0; c < NC; c++) {
            if (c >= ncol) break;
            // per unit d * s-less value, units b then b + 16, as the unit-plane kernel sums them
            float v = 0.f;
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const float f = fmaf((float)acc[c][i][2], kDig2, fmaf((float)acc[c][i][1], kDig1, (float)acc[c][i][0]));
                v += half_bits_to_f32(i ? dw[p] >> 16 : dw[p]) * f;
            }
            // sum over the row's 16 lanes (b), in group_sum<16>'s order
            v = quad_lane_sum(v);
            v *= s[c];
            if (lane < 4) {
                gfloat* y = (gfloat*)(a.seg[0].y + r + c * a.ys);
                if (a.accumulate) __builtin_amdgcn_global_atomic_fadd_f32(y, v);
                else *y = v;
                // sampler.rs:305-316: strictly greater wins, so NaN never does
                if constexpr (EPI == mivi::EPI_ARGMAX)
                    if (v > best[c]) { best[c] = v; bidx[c] = r; }
            }
        }
    };
    // Rounds whose refills all stay in range run branch-free; the last full
    // round refills only the steps that exist (a refill of an earlier quad
    // would go back to memory: the code loads are non-temporal), and the
    // tail computes the last < PD steps.
    int st = 0;
    for (; st + 2 * PD <= cnt; st += PD) {
#pragma unroll
        for (int p = 0; p < PD; p++) {
            compute(p, st + p);
            load(p, st + p + PD);
        }
    }
    if (st + PD <= cnt) {
#pragma unroll
        for (int p = 0; p < PD; p++) {
            compute(p, st + p);
            if (st + p + PD < cnt) load(p, st + p + PD);
        }
        st += PD;
    }
#pragma unroll
    for (int p = 0; p < PD; p++)
        if (st + p < cnt) compute(p, st + p);
    if constexpr (EPI == mivi::EPI_ARGMAX) write_part();
}

// One column of the eight-column kernels' activations (K = 2048) as
// base-256 digit planes, formed in the one-column kernel's order so that
// every column's sums are that kernel's: load() issues the column's loads
// (chunk i is values 4 (lane + 64 i) .. + 3, which thread lane + 64 (i & 3)
// of the one-column kernel holds), finish() forms each chunk's three plane
// dwords, hands them to put(i, d) and returns the column's scale s.
template <int PRO>
struct ColB256 {
    static constexpr int K = 2048, NL = K / 256;
    f32x4 u[NL];
    f32x4 nwt[PRO == mivi::PRO_RMSNORM ? NL : 1];
    __device__ __forceinline__ void load(const mivi::GemvArgs& a, int col, int lane) {
        const float* x = a.x + (size_t)col * a.xs;
#pragma unroll
        for (int i = 0; i < NL; i++) u[i] = *(const gf32x4*)(x + 4 * (lane + 64 * i));
        if constexpr (PRO == mivi::PRO_RMSNORM) {
#pragma unroll
            for (int i = 0; i < NL; i++) nwt[i] = *(const gf32x4*)(a.norm_w + 4 * (lane + 64 * i));
        }
    }
    template <class Put>
    __device__ __forceinline__ float finish(const mivi::GemvArgs& a, Put put) {
        float v[NL][4];
#pragma unroll
        for (int i = 0; i < NL; i++) { v[i][0] = u[i].x; v[i][1] = u[i].y; v[i][2] = u[i].z; v[i][3] = u[i].w; }
        float m = 0.f, scale = 1.0f;
        if constexpr (PRO == mivi::PRO_RMSNORM) {
            // the one-column kernel's order: thread lane + 64 h sums its
            // chunks h, h + 4 in turn, each wave's sum is lane 0's butterfly
            // sum, and the four waves add in order
            float pw[4];
#pragma unroll
            for (int h = 0; h < 4; h++) {
                float t = 0.f;
#pragma unroll
                for (int e = 0; e < 4; e++) t = fmaf(v[h][e], v[h][e], t);
#pragma unroll
                for (int e = 0; e < 4; e++) t = fmaf(v[h + 4][e], v[h + 4][e], t);
                pw[h] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(xsum_desc<64>(t)), 0));
            }
            const float ss = ((pw[0] + pw[1]) + pw[2]) + pw[3];
            scale = 1.0f / sqrtf(ss / (float)K + a.eps);
            // digits of u = v w (math.rs:7-22; 1 / rms goes into s)
#pragma unroll
            for (int i = 0; i < NL; i++)
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    v[i][e] = v[i][e] * nwt[i][e];
                    m = fmaxf(m, fabsf(v[i][e]));
                }
        } else {
            float nn = 0.f;  // NaN for a NaN or infinite value (fmaxf passes NaNs over)
#pragma unroll
            for (int i = 0; i < NL; i++)
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    m = fmaxf(m, fabsf(v[i][e]));
                    nn = fmaf(v[i][e], 0.f, nn);
                }
            m += nn;
        }
        {
            float lo, hi;
            swap32(m, lo, hi);
            m = nanmax(lo, hi);
            swap16(m, lo, hi);
            m = nanmax(lo, hi);
            m = nanmax(m, dpp_mov<0x128>(m));
            m = nanmax(m, xor4_mov(m));
            m = nanmax(m, dpp_mov<0x4E>(m));
            m = nanmax(m, dpp_mov<0xB1>(m));
        }
        const bool finite = m > 0.f && m <= 3.40282347e38f;
        const float mul = finite ? kDigMul / m : 0.0f;
#pragma unroll
        for (int i = 0; i < NL; i++) {
            uint32_t d[3];
            digits4_b256(v[i], mul, d[0], d[1], d[2]);
            put(i, d);
        }
        return ((m - m) + m * scale) * (2.0f / 127.0f);
    }
};

// Up to eight columns (sequences) against the same row quads, so a batched
// head reads its quads once per step. Eight waves per workgroup, wave c
// forming column c's digits; each wave then takes its own quads as above.
// The 3 ncol digit planes (plane 3c + p = plane p of column c) sit in LDS in
// groups of four, laid out for the 4 x 4 x 4 instruction: entry (G, g,
// lane 4b + v) is the 16 digits of plane 4G + v at slot g of the lane's
// unit, so one 1 KB read gives a group's A operands for a slot, and lane
// 4b + j receives the four planes' sums for row j. The codes enter as
// c - 32 (signed bytes: (c + 0x60) ^ 0x80), which adds the Q6_K offset in
// the instruction; the integer sums are the one-column kernel's. The float
// steps run in its order, and the cross-lane sum of the eight columns is a
// reduce-scatter over the same butterfly (lane bits 5, 4, 3, then 2), after
// which lane l with bit 2 clear holds column (l >> 3) & 7, row l & 3: every
// column's result equals the one-column kernel's bit for bit.
// NGR groups (3: up to four columns, 6: up to eight); planes past 3 ncol are
// zeros.
constexpr int kQuad8Waves = 8, kQuad8WG = 64 * kQuad8Waves;

template <int PRO, int EPI, int PD, int NGR>
__global__ void __launch_bounds__(kQuad8WG) gemv_q6k_quad8_kernel(const mivi::GemvArgs a) {
    constexpr int NCM = 4 * NGR / 3;
    static_assert(NGR == 3 || NGR == 6, "four or eight columns");
    __shared__ u32x4 Ab[NGR][8][64];  // [group][slot][lane]
    __shared__ float scol[kQuad8Waves];
    const int nquads = a.seg[0].n / 4;
    const uint8_t* W = a.seg[0].W;
    const int ncol = a.ncol;  // 1..NCM, workgroup-uniform
    const int npl = 3 * ncol;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int jv = lane & 3;
    const int nw = gridDim.x * kQuad8Waves, wid = blockIdx.x * kQuad8Waves + wave;
    const int cnt = wid < nquads ? (nquads - wid + nw - 1) / nw : 0;  // wave-uniform

    u32x4 w[PD][6];
    u32x2 scw[PD];
    uint32_t dw[PD];
    auto load = [&](int p, int st) {  // as gemv_q6k_quad_kernel's
        st = st < cnt ? st : cnt - 1;
        int q = wid + st * nw;
        q = q < 0 ? 0 : q < nquads ? q : nquads - 1;
        const uint8_t* base = W + (size_t)q * kQuadBytes;
        const uint8_t* cb = base + 64 * (q & 1);
        const uint8_t* db = base + ((q & 1) ? 0 : 6656);
#pragma unroll
        for (int k = 0; k < 6; k++) w[p][k] = ldg16_nt(cb + 1024 * k + 16 * lane);
        scw[p] = *(const __attribute__((address_space(1))) u32x2*)(cb + 6144 + 8 * lane);
        dw[p] = *(const __attribute__((address_space(1))) uint32_t*)(db + 4 * (4 * jv + (lane >> 4)));
    };
    const bool stager = wave < ncol && wave < NCM;  // wave-uniform
    ColB256<PRO> col;
    if (stager) col.load(a, wave, lane);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int p = 0; p < PD; p++) load(p, p);
    __builtin_amdgcn_sched_barrier(0);
    // planes 3 ncol .. 4 NGR - 1 read zeros
#pragma unroll
    for (int G = 0; G < NGR; G++)
        if (4 * G + (int)(threadIdx.x & 3) >= npl) Ab[G][threadIdx.x >> 6][threadIdx.x & 63] = u32x4{0, 0, 0, 0};
    if (stager) {
        // dword lane + 64 i of a plane: 16 B chunk k = lane / 4 + 16 i of
        // unit 4 i + kb, quarter q (chunk k of a plane is unit
        // 4 (k >> 4) + 2 ((k >> 3) & 1) + (k & 1), quarter (k >> 1) & 3),
        // dword e of the chunk
        uint32_t* A32 = (uint32_t*)&Ab[0][0][0];
        const int kb = 2 * ((lane >> 5) & 1) + ((lane >> 2) & 1), q = (lane >> 3) & 3, e = lane & 3;
        const float sc = col.finish(a, [&](int i, const uint32_t (&d)[3]) {
            const int g = 4 * (i >> 2) + q, bb = 4 * (i & 3) + kb;
#pragma unroll
            for (int p = 0; p < 3; p++) {
                const int pl = 3 * wave + p;
                A32[(((pl >> 2) * 8 + g) * 64 + 4 * bb + (pl & 3)) * 4 + e] = d[p];
            }
        });
        if (lane == 0) scol[wave] = sc;
    }
    __syncthreads();

    const int cl = (lane >> 3) & 7;  // this lane's column after the cross-lane sum
    const float s_l = scol[cl < ncol ? cl : 0];
    float best = -INFINITY;
    int bidx = 0x7FFFFFFF;
    auto write_part = [&]() {
        // lanes 8c .. 8c + 3 hold column c's rows; lanes with bit 2 set carry (-inf, INT_MAX)
        float bv = best;
        int bi = bidx;
#pragma unroll
        for (int o = 1; o < 4; o <<= 1) {
            const float ov = __shfl_xor(bv, o, 64);
            const int oi = __shfl_xor(bi, o, 64);
            if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
        }
        if ((lane & 7) == 0 && cl < ncol) {
            a.part_val[cl * a.ps + wid] = bv;
            a.part_idx[cl * a.ps + wid] = bi;
        }
    };
    if (cnt == 0) {  // wave-uniform; no barrier follows
        if constexpr (EPI == mivi::EPI_ARGMAX) write_part();
        return;
    }

    auto compute = [&](int p, int st) {
        int acc[4 * NGR][2];
#pragma unroll
        for (int g = 0; g < 8; g++) {
            const int D0 = 3 * g;
            const uint32_t W0 = w[p][D0 >> 2][D0 & 3];
            const uint32_t W1 = w[p][(D0 + 1) >> 2][(D0 + 1) & 3];
            const uint32_t W2 = w[p][(D0 + 2) >> 2][(D0 + 2) & 3];
            uint32_t B[4] = {W0 & 0x3F3F3F3Fu, W1 & 0x3F3F3F3Fu, W2 & 0x3F3F3F3Fu,
                             ((W0 >> 6) & 0x03030303u) | ((W1 >> 4) & 0x0C0C0C0Cu) | ((W2 >> 2) & 0x30303030u)};
#pragma unroll
            for (int m = 0; m < 4; m++) B[m] = (B[m] + 0x60606060u) ^ 0x80808080u;  // c - 32 per byte
            const int scv = __builtin_amdgcn_sbfe((int)(g < 4 ? scw[p].x : scw[p].y), 8 * (g & 3), 8);
#pragma unroll
            for (int G = 0; G < NGR; G++) {
                // (volatile: read at each step, not held in registers across the loop)
                const u32x4 A = *(volatile __attribute__((address_space(3))) u32x4*)&Ab[G][g][lane];
                i32x4 D = {0, 0, 0, 0};
                D = mfma4x4(A.x, B[0], D);
                D = mfma4x4(A.y, B[1], D);
                D = mfma4x4(A.z, B[2], D);
                D = mfma4x4(A.w, B[3], D);
                const int i = g >> 2;
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    if ((g & 3) == 0) acc[4 * G + v][i] = mul24(D[v], scv);
                    else acc[4 * G + v][i] += mul24(D[v], scv);
                }
            }
        }
        float vc[8];
#pragma unroll
        for (int c = 0; c < 8; c++) {
            vc[c] = 0.f;
            if (c < NCM) {  // (columns past ncol sum zeros)
#pragma unroll
                for (int i = 0; i < 2; i++) {
                    const float f = fmaf((float)acc[3 * c + 2][i], kDig2, fmaf((float)acc[3 * c + 1][i], kDig1, (float)acc[3 * c][i]));
                    vc[c] += half_bits_to_f32(i ? dw[p] >> 16 : dw[p]) * f;
                }
            }
        }
        // reduce-scatter: lane bit 5 keeps columns 4 (bit 5) + 0..3, bit 4
        // then halves them, bit 3 picks one; bit 2 finishes the sum
        float r4[4], r2[2];
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const auto t = __builtin_amdgcn_permlane32_swap(__float_as_uint(vc[c]), __float_as_uint(vc[c + 4]), false, false);
            r4[c] = __uint_as_float(t[0]) + __uint_as_float(t[1]);
        }
#pragma unroll
        for (int c = 0; c < 2; c++) {
            const auto t = __builtin_amdgcn_permlane16_swap(__float_as_uint(r4[c]), __float_as_uint(r4[c + 2]), false, false);
            r2[c] = __uint_as_float(t[0]) + __uint_as_float(t[1]);
        }
        const bool b3 = lane & 8;
        float y = (b3 ? r2[1] : r2[0]) + dpp_mov<0x128>(b3 ? r2[0] : r2[1]);  // row_ror:8 (lane ^ 8)
        y += dpp_mov<0x12C>(y);                                               // row_ror:12 (lane ^ 4 where bit 2 is clear)
        y *= s_l;
        if (!(lane & 4) && cl < ncol) {
            const int r = 4 * (wid + st * nw) + jv;
            gfloat* yp = (gfloat*)(a.seg[0].y + r + cl * a.ys);
            if (a.accumulate) __builtin_amdgcn_global_atomic_fadd_f32(yp, y);
            else *yp = y;
            // sampler.rs:305-316: strictly greater wins, so NaN never does
            if constexpr (EPI == mivi::EPI_ARGMAX)
                if (y > best) { best = y; bidx = r; }
        }
    };
    int st = 0;
    for (; st + 2 * PD <= cnt; st += PD) {
#pragma unroll
        for (int p = 0; p < PD; p++) {
            compute(p, st + p);
            load(p, st + p + PD);
        }
    }
    if (st + PD <= cnt) {
#pragma unroll
        for (int p = 0; p < PD; p++) {
            compute(p, st + p);
            if (st + p + PD < cnt) load(p, st + p + PD);
        }
        st += PD;
    }
#pragma unroll
    for (int p = 0; p < PD; p++)
        if (st + p < cnt) compute(p, st + p);
    if constexpr (EPI == mivi::EPI_ARGMAX) write_part();
}

// ------------------------------------ Q6_K 32-row tiles for batched columns
//
// The batched head's copy of a Q6_K matrix with K = 2048 and a multiple of 32
// rows (launch_pack_q6k_t32, the model loader for max_batch > 1): chunk
// c = 8 T + s holds superblock s of rows 32 T .. 32 T + 31 in 6720 bytes at
// 6720 c, laid out as the B operand of v_mfma_i32_32x32x16_i8: lane
// l = n + 32 hh supplies row 32 T + n at values 8 hh .. 8 hh + 7 of every
// 16-value sub-block. Offsets from o = 64 for odd c (0 for even c):
//   [0, 6144)     codes, 16 B per lane at 1024 k + 16 l (k = 0..5). Sub-blocks
//                 2P and 2P + 1 are dwords 3P .. 3P + 2 of the lane's 24:
//                 sixteen 6-bit codes, c_0..c_7 of sub-block 2P and
//                 c_8..c_15 of 2P + 1, packed as the row quads pack a slot
//                 (byte e of dword 3P + m: c_{4m+e} in bits 0-5, bits 2m,
//                 2m + 1 of c_{12+e} in bits 6-7)
//   [6144, 6656)  row n's sixteen sub-block scales at 6144 + 16 n
// and the 64 bytes of d (row n's fp16 at 2 n) follow at 6656 for even c and
// lead at 0 for odd c, so every 1 KB wave load of codes is line-aligned (as
// in the row quads). The copy has the GGUF matrix's size.
constexpr int kT32Bytes = 6720;

// f(std::integral_constant<int, I>) for I = I0 .. N - 1, unrolled at compile
// time (register arrays indexed by I stay in registers)
template <int I0, int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (I0 < N) {
        f(std::integral_constant<int, I0>{});
        static_for<I0 + 1, N>(f);
    }
}

// Superblock of step j of a tile: 0, 4, 2, 6, 1, 5, 3, 7 (j's bits reversed),
// the order in which the row's unit values fold into the one-column
// kernel's cross-lane sum.
__host__ __device__ constexpr int t32_superblock(int j) { return ((j & 1) << 2) | (j & 2) | (j >> 2); }

// Up to eight columns against 32-row tiles on v_mfma_i32_32x32x16_i8, one
// 16-value sub-block per instruction. A row m = 8 p + c is digit plane p of
// column c (staged into LDS as the eight-column quad kernel stages them; rows
// 24-31 and columns past ncol are zeros), B the tile's codes as c - 32 (signed
// bytes (c + 0x60) ^ 0x80), so lane l = n + 32 hh receives, for row n of the
// tile, the plane sums of columns 4 hh .. 4 hh + 3 (register 4 p + j: plane
// p, column 4 hh + j). Each sum is scaled by its sub-block's scale with exact
// 24-bit multiplies and summed over the four sub-blocks of a unit of the
// one-column kernel (half h, sub-blocks 8 h + jj + 2 q of one superblock), so
// the unit sums are that kernel's integers; each unit's float step, and the
// sum of the row's 32 unit values in the order of that kernel's butterfly
// over its 16 lanes (units b and b + 16 in lane b; b xor 8, 4, 2, 1), run
// in registers as superblocks arrive in t32_superblock order. Every column's
// result therefore equals the one-column kernel's bit for bit. PD
// superblocks in flight per wave; the waves take tiles wid, wid + nw, ...
template <int PRO, int EPI, int PD>
__global__ void __launch_bounds__(kQuad8WG) gemv_q6k_t32_kernel(const mivi::GemvArgs a) {
    constexpr int K = 2048, NS = K / 256, NSB = K / 16;
    constexpr int AROW = 65;  // u32x2 per sub-block row of A in LDS (64 lanes and one of padding)
    static_assert(NS % PD == 0, "ring slots at fixed superblock steps");
    __shared__ u32x2 Ab[NSB * AROW];  // A operands: [sub-block][lane], eight digits each
    __shared__ float scol[kQuad8Waves];
    const int ntiles = a.seg[0].n / 32;
    const uint8_t* W = a.seg[0].W;
    const int ncol = a.ncol;  // 1..8, workgroup-uniform
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n = lane & 31, hh = lane >> 5;
    const int nw = gridDim.x * kQuad8Waves, wid = blockIdx.x * kQuad8Waves + wave;
    const int cnt = wid < ntiles ? (ntiles - wid + nw - 1) / nw : 0;  // tiles, wave-uniform

    u32x4 w[PD][6];
    u32x4 scw[PD];
    uint32_t dbits[PD];
    // step t = 8 i + j: tile wid + i nw, superblock t32_superblock(j)
    auto load = [&](int p, int i, int j) __attribute__((always_inline)) {
        const size_t c = (size_t)(wid + i * nw) * NS + t32_superblock(j);
        const uint8_t* base = W + c * kT32Bytes;
        const uint8_t* cb = base + 64 * (c & 1);
        const uint8_t* db = base + ((c & 1) ? 0 : 6656);
#pragma unroll
        for (int k = 0; k < 6; k++) w[p][k] = ldg16_nt(cb + 1024 * k + 16 * lane);
        scw[p] = *(const __attribute__((address_space(1))) u32x4*)(cb + 6144 + 16 * n);
        dbits[p] = *(const __attribute__((address_space(1))) uint16_t*)(db + 2 * n);
    };
    const bool stager = wave < ncol;  // wave-uniform
    ColB256<PRO> col;
    if (stager) col.load(a, wave, lane);
    __builtin_amdgcn_sched_barrier(0);
    if (cnt > 0) {
#pragma unroll
        for (int p = 0; p < PD; p++) load(p, 0, p);
    }
    __builtin_amdgcn_sched_barrier(0);
    // rows without a column (m >= 24, or column m % 8 >= ncol) read zeros
    for (int idx = threadIdx.x; idx < NSB * 64; idx += kQuad8WG) {
        const int m = idx & 31;
        if (m >= 24 || (m & 7) >= ncol) Ab[(idx >> 6) * AROW + (idx & 63)] = u32x2{0, 0};
    }
    if (stager) {
        // chunk i, dword j4 = lane + 64 i of the column: values 4 j4 .. + 3,
        // sub-block j4 / 4, lane half (j4 >> 1) & 1, dword j4 & 1 of the 8 B
        uint32_t* A32 = (uint32_t*)Ab;
        const float sc = col.finish(a, [&](int i, const uint32_t (&d)[3]) {
            const int j4 = lane + 64 * i;
            const int base = ((j4 >> 2) * AROW + wave + 32 * ((j4 >> 1) & 1)) * 2 + (j4 & 1);
#pragma unroll
            for (int p = 0; p < 3; p++) A32[base + 16 * p] = d[p];  // row 8 p + wave
        });
        if (lane == 0) scol[wave] = sc;
    }
    __syncthreads();

    float s_c[4];
#pragma unroll
    for (int cc = 0; cc < 4; cc++) s_c[cc] = scol[4 * hh + cc < ncol ? 4 * hh + cc : 0];
    float best[4];
    int bidx[4];
#pragma unroll
    for (int cc = 0; cc < 4; cc++) { best[cc] = -INFINITY; bidx[cc] = 0x7FFFFFFF; }
    auto write_part = [&]() {
#pragma unroll
        for (int cc = 0; cc < 4; cc++) {
            float bv = best[cc];
            int bi = bidx[cc];
#pragma unroll
            for (int o = 1; o < 32; o <<= 1) {
                const float ov = __shfl_xor(bv, o, 64);
                const int oi = __shfl_xor(bi, o, 64);
                if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
            }
            const int cl = 4 * hh + cc;
            if (n == 0 && cl < ncol) {
                a.part_val[cl * a.ps + wid] = bv;
                a.part_idx[cl * a.ps + wid] = bi;
            }
        }
    };
    if (cnt == 0) {  // wave-uniform; no barrier follows
        if constexpr (EPI == mivi::EPI_ARGMAX) write_part();
        return;
    }

    // unit values of the row (per column cc): W the first superblock's term,
    // V a unit's value v_b (b < 8), A4 the first level of the sum
    float Wu[4][4], Vu[4][4], A4[4][4];
    auto compute = [&](auto J, int tile) __attribute__((always_inline)) {
        constexpr int j = decltype(J)::value, p = j % PD, sb = t32_superblock(j);
        const float d = half_bits_to_f32(dbits[p]);
        const i32x16 zero = {};
#pragma unroll
        for (int uu = 0; uu < 4; uu++) {
            const int h = uu >> 1, jj = uu & 1;
            // (opaque from here: this unit's code and scale decode is not
            // hoisted above it, which would hold every unit's decoded
            // codes and scales at once)
#pragma unroll
            for (int k = 0; k < 6; k++) asm volatile("" : "+v"(w[p][k]));
            asm volatile("" : "+v"(scw[p]));
            i32x16 D[4];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                // sub-block isl = 8 h + 2 q + jj: pair P = 4 h + q, codes c_0..c_7
                // (jj = 0) or c_8..c_15 (jj = 1) of its three dwords, as c - 32
                const int isl = 8 * h + 2 * q + jj, D0 = 3 * (isl >> 1);
                const uint32_t W0 = w[p][D0 >> 2][D0 & 3];
                const uint32_t W1 = w[p][(D0 + 1) >> 2][(D0 + 1) & 3];
                const uint32_t W2 = w[p][(D0 + 2) >> 2][(D0 + 2) & 3];
                uint32_t b0, b1;
                if (jj == 0) {
                    b0 = W0 & 0x3F3F3F3Fu;
                    b1 = W1 & 0x3F3F3F3Fu;
                } else {
                    b0 = W2 & 0x3F3F3F3Fu;
                    b1 = ((W0 >> 6) & 0x03030303u) | ((W1 >> 4) & 0x0C0C0C0Cu) | ((W2 >> 2) & 0x30303030u);
                }
                b0 = (b0 + 0x60606060u) ^ 0x80808080u;
                b1 = (b1 + 0x60606060u) ^ 0x80808080u;
                // (volatile: read at each step, not hoisted out of the tile loop)
                const u32x2 A = *(volatile __attribute__((address_space(3))) u32x2*)&Ab[(16 * sb + isl) * AROW + lane];
                D[q] = __builtin_amdgcn_mfma_i32_32x32x16_i8((long)(((uint64_t)A.y << 32) | A.x),
                                                             (long)(((uint64_t)b1 << 32) | b0), zero, 0, 0, 0);
            }
            int acc[3][4];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int isl = 8 * h + 2 * q + jj;
                const int scv = __builtin_amdgcn_sbfe((int)scw[p][isl >> 2], 8 * (isl & 3), 8);
                // |D| < 2^17, |sc| <= 128: exact 24-bit multiplies (as the quad
                // kernels); each sum passes an empty asm so the four steps stay
                // a chain of multiply-adds (v_mad_i32_i24) instead of separate
                // multiplies and three-way adds
#pragma unroll
                for (int pl = 0; pl < 3; pl++)
#pragma unroll
                    for (int cc = 0; cc < 4; cc++) {
                        if (q == 0) acc[pl][cc] = mul24(D[q][4 * pl + cc], scv);
                        else acc[pl][cc] += mul24(D[q][4 * pl + cc], scv);
                        asm volatile("" : "+v"(acc[pl][cc]));
                    }
            }
#pragma unroll
            for (int cc = 0; cc < 4; cc++) {
                const float f = fmaf((float)acc[2][cc], kDig2, fmaf((float)acc[1][cc], kDig1, (float)acc[0][cc]));
                // unit b = 4 (sb & 3) + uu of the one-column kernel, term i = sb >> 2
                // (each result passes an empty volatile asm, which keeps this
                // unit's arithmetic ahead of the next unit's loads and products:
                // the products would otherwise all be issued first and spilled)
                if ((j & 1) == 0) {  // superblock sb < 4: the first term of v_b
                    float v = 0.f;
                    v += d * f;
                    asm volatile("" : "+v"(v));
                    Wu[uu][cc] = v;
                } else {  // sb + 4: v_b complete
                    float v = Wu[uu][cc];
                    v += d * f;
                    if (j == 1 || j == 5) v = v;                        // v_b, b = uu or 4 + uu
                    else if (j == 3) v = Vu[uu][cc] + v;                // a_b = v_b + v_(b+8), b = uu
                    else v = A4[uu][cc] + (Vu[uu][cc] + v);             // j = 7: a_(4+uu), then + a_uu
                    asm volatile("" : "+v"(v));
                    if (j == 3) A4[uu][cc] = v;
                    else Vu[uu][cc] = v;
                }
            }
            // one unit's four results live at a time (hoisting the next
            // unit's products spills)
            __builtin_amdgcn_sched_barrier(0);
        }
        if (j == NS - 1) {
            // Vu[b][cc] = a_b + a_(b+4) (b < 4); then b xor 2, b xor 1
            const int r = 32 * tile + n;
#pragma unroll
            for (int cc = 0; cc < 4; cc++) {
                float y = (Vu[0][cc] + Vu[2][cc]) + (Vu[1][cc] + Vu[3][cc]);
                y *= s_c[cc];
                const int cl = 4 * hh + cc;
                if (cl < ncol) {
                    gfloat* yp = (gfloat*)(a.seg[0].y + r + cl * a.ys);
                    if (a.accumulate) __builtin_amdgcn_global_atomic_fadd_f32(yp, y);
                    else *yp = y;
                    // sampler.rs:305-316: strictly greater wins, so NaN never does
                    if constexpr (EPI == mivi::EPI_ARGMAX)
                        if (y > best[cc]) { best[cc] = y; bidx[cc] = r; }
                }
            }
        }
    };
    // Tiles with a successor refill every slot branch-free; the last tile
    // refills only the steps that exist.
    for (int i = 0; i < cnt; i++) {
        const int tile = wid + i * nw;
        if (i + 1 < cnt) {  // wave-uniform
            static_for<0, NS>([&](auto J) __attribute__((always_inline)) {
                constexpr int j = decltype(J)::value;
                compute(J, tile);
                load(j % PD, i + (j + PD) / NS, (j + PD) % NS);
            });
        } else {
            static_for<0, NS>([&](auto J) __attribute__((always_inline)) {
                constexpr int j = decltype(J)::value;
                compute(J, tile);
                if constexpr (j + PD < NS) load(j % PD, i, j + PD);
            });
        }
    }
    if constexpr (EPI == mivi::EPI_ARGMAX) write_part();
}

// ------------------------------------------ Q4_K row quads on the matrix cores
//
// Packed Q4_K matrices with K = 2048 S (S = 1 or 4) columns and a multiple of
// 4 rows (mivi_hip_pack_weights) are stored as row quads: quad Q (rows 4Q ..
// 4Q+3) is S sub-quads of 4608 contiguous bytes, sub-quad s holding values
// [2048 s, 2048 s + 2048) of the four rows, laid out for the 64 lanes
// l = 4b + j of one wave (j = row of the quad, b = 0..15). Lane (b, j) owns
// units t = 32 s + b and t + 16 of row j, where unit t is sub-blocks 2g and
// 2g + 1 of superblock t / 4 (g = t & 3, q4_k_m.rs:24-63): the units lanes
// b and b + 16 (K = 2048), or b + 16 i (K = 8192), of the streaming kernel own.
//   [0, 4096)     the units' 32 code bytes each, 16 B per lane at
//                 1024 k + 16 l: k = 0, 1 unit t (its bytes 0-15, 16-31),
//                 k = 2, 3 unit t + 16; byte e holds value 64 g + e (low
//                 nibble) and 64 g + 32 + e (high nibble) of the unit
//   [4096, 4480)  6 B per lane at 6 l: the 6-bit scales of sub-blocks
//                 (2g, 2g + 1) of unit t, then of unit t + 16, in bits 0-23,
//                 their 6-bit mins in bits 24-47
//   [4480, 4608)  f16 d | f16 dmin of the superblocks of units t and t + 16
//                 of row j, 8 B per (j, b / 4) at 4480 + 8 (4 j + b / 4)
// A sub-quad is 36 lines of 128 B and every 1 KB wave load of codes is
// contiguous; a packed matrix keeps the GGUF matrix's size.
//
// The products run on v_mfma_i32_4x4x4_16b_i8 as in the Q6_K quad kernel:
// in block b, lane 4b + v supplies digit plane v of x (zeros for v = 3) at
// four values and lane 4b + j four codes of row j at the same values, and
// lane 4b + j receives the plane sums of its row. Eight instructions cover a
// 32-value sub-block; the integer sums are the sdot4 kernel's, the per-unit
// float steps are q4k_unit_i8's, and the unit values are summed in the
// streaming kernel's butterfly order (units t, t + 16 first at K = 2048;
// t + 64, then t + 32, then t + 16 at K = 8192; then the lanes), so every
// row equals the streaming kernel's result on the GGUF rows bit for bit.

constexpr int kQ4SubQuadBytes = 4608;

typedef uint32_t u32x2_a4 __attribute__((ext_vector_type(2), aligned(4)));

// One sub-quad's bytes as lane l loads them.
struct Q4Item {
    u32x4 c[4];          // code bytes of unit t (c[0], c[1]) and t + 16 (c[2], c[3])
    uint32_t slo, shi;   // 8 B at (6 l) & ~3: the lane's six scale bytes at bit 16 (l & 1)
    u32x2 dp;            // d | dmin << 16 of the superblocks of units t and t + 16
};

__device__ __forceinline__ void load_q4_item(Q4Item& it, const uint8_t* sub, int lane) {
#pragma unroll
    for (int k = 0; k < 4; k++) it.c[k] = ldg16_nt(sub + 1024 * k + 16 * lane);
    const u32x2_a4 sw = *(const __attribute__((address_space(1))) u32x2_a4*)(sub + 4096 + ((6 * lane) & ~3));
    it.slo = sw.x;
    it.shi = sw.y;
    it.dp = *(const __attribute__((address_space(1))) u32x2*)(sub + 4480 + 8 * (4 * (lane & 3) + (lane >> 4)));
}

// The lane's two unit values of one sub-quad (q4k_unit_i8's steps), from its
// digit operands A[i][h][m] (unit i, sub-block 2g + h, values 4m .. 4m + 3)
// and fp32 sub-block sums X[i][h].
__device__ __forceinline__ void q4_item_units(const Q4Item& it, const uint32_t (&A)[2][2][8], const float (&X)[2][2],
                                              float s, int lane, float (&u)[2]) {
    const uint32_t sh = 16u * (uint32_t)(lane & 1);
    const uint32_t lo = __builtin_amdgcn_alignbit(it.shi, it.slo, sh), hi = it.shi >> sh;
    const uint32_t scf[2][2] = {{lo & 63u, (lo >> 6) & 63u}, {(lo >> 12) & 63u, (lo >> 18) & 63u}};
    const uint32_t mf[2][2] = {{(lo >> 24) & 63u, __builtin_amdgcn_alignbit(hi, lo, 30) & 63u},
                               {(hi >> 4) & 63u, (hi >> 10) & 63u}};
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const uint32_t w[8] = {it.c[2 * i].x, it.c[2 * i].y, it.c[2 * i].z, it.c[2 * i].w,
                               it.c[2 * i + 1].x, it.c[2 * i + 1].y, it.c[2 * i + 1].z, it.c[2 * i + 1].w};
        i32x4 Dl = {0, 0, 0, 0}, Dh = {0, 0, 0, 0};
#pragma unroll
        for (int m = 0; m < 8; m++) {
            Dl = mfma4x4(A[i][0][m], w[m] & 0x0F0F0F0Fu, Dl);
            Dh = mfma4x4(A[i][1][m], (w[m] >> 4) & 0x0F0F0F0Fu, Dh);
        }
        int Ae[3];
#pragma unroll
        for (int e = 0; e < 3; e++) Ae[e] = mul24(Dl[e], (int)scf[i][0]) + mul24(Dh[e], (int)scf[i][1]);
        const float f = fmaf((float)Ae[2], kDig2, fmaf((float)Ae[1], kDig1, (float)Ae[0]));
        const uint32_t dpv = i ? it.dp.y : it.dp.x;
        const float d = half_bits_to_f32(dpv), dmin = half_bits_to_f32(dpv >> 16);
        u[i] = (d * s) * f - dmin * fmaf((float)mf[i][0], X[i][0], (float)mf[i][1] * X[i][1]);
    }
}

// One column; a step is one quad (store), the gate and up quads of the same
// rows (EPI_SWIGLU: seg[0] gate, seg[1] up), or the B, C and X quads of four
// channels (EPI_CONV: one segment [B | C | X]); PD steps in flight per wave.
template <int PRO, int EPI, int S, int PD>
__global__ void __launch_bounds__(kWG) gemv_q4k_quad_kernel(const mivi::GemvArgs a) {
    constexpr int K = 2048 * S;
    constexpr int G = EPI == mivi::EPI_SWIGLU ? 2 : EPI == mivi::EPI_CONV ? 3 : 1;
    static_assert(EPI != mivi::EPI_ARGMAX, "the argmax epilogue is the Q6_K head's");
    __shared__ __attribute__((aligned(16))) uint32_t dig[3 * K / 4];
    __shared__ __attribute__((aligned(16))) float xsum[K / 32];
    const Segs sg(a, (size_t)S * 1152);
    const int n0 = a.seg[0].n, D3 = n0 / 3;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int b = lane >> 2, jv = lane & 3;
    const int nw = gridDim.x * (kWG / 64), wid = blockIdx.x * (kWG / 64) + wave;
    const int nsteps = EPI == mivi::EPI_SWIGLU ? n0 / 4 : EPI == mivi::EPI_CONV ? D3 / 4 : sg.n / 4;
    const int cnt = wid < nsteps ? (nsteps - wid + nw - 1) / nw : 0;  // wave-uniform

    // first row of quad g of step st (steps past the end re-read the wave's
    // last step and waves without steps read step 0; nothing is stored for them)
    auto quad_row = [&](int st, int g) {
        st = st < cnt ? st : cnt - 1;
        int q = wid + st * nw;
        q = q < 0 ? 0 : q < nsteps ? q : nsteps - 1;
        return 4 * q + g * (EPI == mivi::EPI_SWIGLU ? n0 : EPI == mivi::EPI_CONV ? D3 : 0);
    };
    Q4Item buf[PD][G][S];
    ConvPre cpre[EPI == mivi::EPI_CONV ? PD : 1];  // lanes < 4: the step's channel's conv inputs
    auto load = [&](int p, int st) {
#pragma unroll
        for (int g = 0; g < G; g++) {
            const uint8_t* base = sg.row(quad_row(st, g));
#pragma unroll
            for (int q = 0; q < S; q++) load_q4_item(buf[p][g][q], base + q * kQ4SubQuadBytes, lane);
        }
        if constexpr (EPI == mivi::EPI_CONV) {
            if (lane < 4) conv_prefetch(a, 0, quad_row(st, 0) + jv, cpre[p]);  // channel 4q + jv
        }
    };
    // activation loads, then the first PD steps, then the activation math
    StageIn<PRO, K / kWG> in;
    in.load(a);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int p = 0; p < PD; p++) load(p, p);
    __builtin_amdgcn_sched_barrier(0);
    const float s = in.template finish<true>(a, dig, xsum);

    // digit operands and sub-block sums of sub-quad q for this lane
    auto fetch = [&](int q, uint32_t (&Ao)[2][2][8], float (&Xo)[2][2]) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int t = 32 * q + b + 16 * i;
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const uint32_t* src = dig + (jv < 3 ? jv : 0) * (K / 4) + 16 * t + 8 * h;
                u32x4 v0 = *(const u32x4*)src, v1 = *(const u32x4*)(src + 4);
                if (jv == 3) v0 = v1 = u32x4{0, 0, 0, 0};
                Ao[i][h][0] = v0.x; Ao[i][h][1] = v0.y; Ao[i][h][2] = v0.z; Ao[i][h][3] = v0.w;
                Ao[i][h][4] = v1.x; Ao[i][h][5] = v1.y; Ao[i][h][6] = v1.z; Ao[i][h][7] = v1.w;
            }
            Xo[i][0] = xsum[2 * t];
            Xo[i][1] = xsum[2 * t + 1];
        }
    };
    uint32_t A1[2][2][8];
    float X1[2][2];
    if constexpr (S == 1) fetch(0, A1, X1);
    if (cnt == 0) return;  // wave-uniform; no barrier follows

    auto compute = [&](int p, int st) {
        float rv[G];
#pragma unroll
        for (int g = 0; g < G; g++) {
            float u[S][2];
#pragma unroll
            for (int q = 0; q < S; q++) {
                if constexpr (S == 1) {
                    q4_item_units(buf[p][g][q], A1, X1, s, lane, u[q]);
                } else {
                    uint32_t Ao[2][2][8];
                    float Xo[2][2];
                    fetch(q, Ao, Xo);
                    q4_item_units(buf[p][g][q], Ao, Xo, s, lane, u[q]);
                }
            }
            float v;
            if constexpr (S == 1) {
                v = (0.f + u[0][0]) + (0.f + u[0][1]);
            } else {
                const float a00 = (0.f + u[0][0]) + u[2][0], a01 = (0.f + u[0][1]) + u[2][1];
                const float a10 = (0.f + u[1][0]) + u[3][0], a11 = (0.f + u[1][1]) + u[3][1];
                v = (a00 + a10) + (a01 + a11);
            }
            // the remaining butterfly levels over b (lanes 4b + j)
            rv[g] = quad_lane_sum(v);
        }
        const int r = 4 * (wid + st * nw) + jv;
        if (lane < 4) {
            if constexpr (EPI == mivi::EPI_SWIGLU) {
                *(gfloat*)sg.out(r) = silu_f(rv[0]) * rv[1];  // math.rs:87-95
            } else if constexpr (EPI == mivi::EPI_CONV) {
                conv_finish(a, 0, r, rv[0], rv[1], rv[2], cpre[p]);
            } else {
                store_out(sg, a.accumulate, r, rv[0]);
            }
        }
    };
    // the ring as in the Q6_K quad kernel: the last full round refills only
    // steps that exist (the code loads are non-temporal)
    int st = 0;
    for (; st + 2 * PD <= cnt; st += PD) {
#pragma unroll
        for (int p = 0; p < PD; p++) {
            compute(p, st + p);
            load(p, st + p + PD);
        }
    }
    if (st + PD <= cnt) {
#pragma unroll
        for (int p = 0; p < PD; p++) {
            compute(p, st + p);
            if (st + p + PD < cnt) load(p, st + p + PD);
        }
        st += PD;
    }
#pragma unroll
    for (int p = 0; p < PD; p++)
        if (st + p < cnt) compute(p, st + p);
}

// K = 8192 (S = 4): the workgroup's waves take the four sub-quads of the
// same quads (wave w sub-quad w, its digit operands fixed for the launch)
// and hand their unit values to wave 0 through LDS, which sums them in the
// streaming kernel's order (t + 64, t + 32, t + 16, then the lanes).
template <int PRO, int PD>
__global__ void __launch_bounds__(kWG) gemv_q4k_quad8k_kernel(const mivi::GemvArgs a) {
    constexpr int K = 8192;
    __shared__ __attribute__((aligned(16))) uint32_t dig[3 * K / 4];
    __shared__ __attribute__((aligned(16))) float xsum[K / 32];
    __shared__ float xch[2][4][2][64];  // [step parity][sub-quad][unit][lane]
    const Segs sg(a, (size_t)4 * 1152);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int b = lane >> 2, jv = lane & 3;
    const int nsteps = sg.n / 4;
    const int cnt = (int)blockIdx.x < nsteps ? (nsteps - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x : 0;
    auto load = [&](Q4Item& it, int st) {
        st = st < cnt ? st : cnt - 1;
        int q = (int)blockIdx.x + st * (int)gridDim.x;
        q = q < 0 ? 0 : q < nsteps ? q : nsteps - 1;
        load_q4_item(it, sg.row(4 * q) + wave * kQ4SubQuadBytes, lane);
    };
    Q4Item buf[PD];
    StageIn<PRO, K / kWG> in;
    in.load(a);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int p = 0; p < PD; p++) load(buf[p], p);
    __builtin_amdgcn_sched_barrier(0);
    const float s = in.template finish<true>(a, dig, xsum);
    uint32_t A[2][2][8];
    float X[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int t = 32 * wave + b + 16 * i;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const uint32_t* src = dig + (jv < 3 ? jv : 0) * (K / 4) + 16 * t + 8 * h;
            u32x4 v0 = *(const u32x4*)src, v1 = *(const u32x4*)(src + 4);
            if (jv == 3) v0 = v1 = u32x4{0, 0, 0, 0};
            A[i][h][0] = v0.x; A[i][h][1] = v0.y; A[i][h][2] = v0.z; A[i][h][3] = v0.w;
            A[i][h][4] = v1.x; A[i][h][5] = v1.y; A[i][h][6] = v1.z; A[i][h][7] = v1.w;
        }
        X[i][0] = xsum[2 * t];
        X[i][1] = xsum[2 * t + 1];
    }
    if (cnt == 0) return;  // workgroup-uniform

    auto compute = [&](const Q4Item& it, int st) {
        float u[2];
        q4_item_units(it, A, X, s, lane, u);
        xch[st & 1][wave][0][lane] = u[0];
        xch[st & 1][wave][1][lane] = u[1];
        __syncthreads();
        if (wave == 0) {
            float w[4][2];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                w[q][0] = xch[st & 1][q][0][lane];
                w[q][1] = xch[st & 1][q][1][lane];
            }
            const float a00 = (0.f + w[0][0]) + w[2][0], a01 = (0.f + w[0][1]) + w[2][1];
            const float a10 = (0.f + w[1][0]) + w[3][0], a11 = (0.f + w[1][1]) + w[3][1];
            const float v = quad_lane_sum((a00 + a10) + (a01 + a11));
            if (lane < 4) store_out(sg, a.accumulate, 4 * ((int)blockIdx.x + st * (int)gridDim.x) + jv, v);
        }
    };
    int st = 0;
    for (; st + 2 * PD <= cnt; st += PD) {
#pragma unroll
        for (int p = 0; p < PD; p++) {
            compute(buf[p], st + p);
            load(buf[p], st + p + PD);
        }
    }
    if (st + PD <= cnt) {
#pragma unroll
        for (int p = 0; p < PD; p++) {
            compute(buf[p], st + p);
            if (st + p + PD < cnt) load(buf[p], st + p + PD);
        }
        st += PD;
    }
#pragma unroll
    for (int p = 0; p < PD; p++)
        if (st + p < cnt) compute(buf[p], st + p);
}

// One thread per (quad, sub-quad, lane): the lane's code bytes and scale
// bytes, and (lanes with b % 4 == 0) the d pairs of its row.
__global__ void __launch_bounds__(kWG) pack_q4k_quad_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                                            size_t nquads, int S) {
    const size_t i = (size_t)blockIdx.x * kWG + threadIdx.x;
    if (i >= nquads * (size_t)S * 64) return;
    const size_t Q = i / (64 * (size_t)S);
    const int sq = (int)((i >> 6) % (size_t)S), l = (int)(i & 63), b = l >> 2, j = l & 3;
    const uint8_t* row = src + (4 * Q + j) * ((size_t)S * 1152);
    uint8_t* o = dst + (Q * S + sq) * kQ4SubQuadBytes;
    uint64_t w = 0;
    for (int ii = 0; ii < 2; ii++) {
        const int t = 32 * sq + b + 16 * ii, g = t & 3;
        const uint8_t* blk = row + (t >> 2) * 144;
        for (int k = 0; k < 32; k++) o[1024 * (2 * ii + (k >> 4)) + 16 * l + (k & 15)] = blk[16 + 32 * g + k];
        uint32_t sd[3];
        for (int k = 0; k < 3; k++)
            sd[k] = blk[4 + 4 * k] | (blk[5 + 4 * k] << 8) | (blk[6 + 4 * k] << 16) | ((uint32_t)blk[7 + 4 * k] << 24);
        uint32_t sc0, m0, sc1, m1;
        q4k_scales(sd[0], sd[1], sd[2], g, sc0, m0, sc1, m1);
        w |= (uint64_t)(sc0 | (sc1 << 6)) << (12 * ii);
        w |= (uint64_t)(m0 | (m1 << 6)) << (24 + 12 * ii);
        if ((b & 3) == 0)
            for (int k = 0; k < 4; k++) o[4480 + 8 * (4 * j + (b >> 2)) + 4 * ii + k] = blk[k];
    }
    for (int k = 0; k < 6; k++) o[4096 + 6 * l + k] = (uint8_t)(w >> (8 * k));
}

// One thread per (quad, lane): writes the lane's codes, scales and (lanes
// with b % 4 == 0) the d pair of its row.
__global__ void __launch_bounds__(kWG) pack_q6k_quad_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                                            size_t nquads) {
    const size_t i = (size_t)blockIdx.x * kWG + threadIdx.x;
    if (i >= nquads * 64) return;
    const size_t Q = i >> 6;
    const int l = (int)(i & 63), b = l >> 2, j = l & 3;
    const uint8_t* row = src + (4 * Q + j) * 1680;
    uint8_t* o = dst + Q * kQuadBytes + 64 * (Q & 1);  // codes and scales
    uint8_t* od = dst + Q * kQuadBytes + ((Q & 1) ? 0 : 6656);
    for (int g = 0; g < 8; g++) {
        const int u = b + 16 * (g >> 2), q = g & 3, h = (u >> 1) & 1, jj = u & 1;
        const uint8_t* blk = row + (u >> 2) * 210;
        uint32_t c[16];
        for (int e = 0; e < 16; e++) c[e] = q6_code(blk, h, q, 16 * jj + e);
        for (int m = 0; m < 3; m++) {
            uint32_t word = 0;
            for (int e = 0; e < 4; e++) word |= (c[4 * m + e] | (((c[12 + e] >> (2 * m)) & 3u) << 6)) << (8 * e);
            const int D = 3 * g + m;
            *(uint32_t*)(o + 1024 * (D >> 2) + 16 * l + 4 * (D & 3)) = word;
        }
        o[6144 + 8 * l + g] = blk[192 + 8 * h + jj + 2 * q];
    }
    if ((b & 3) == 0) {
        const int s = b >> 2;
        uint8_t* dp = od + 4 * (4 * j + s);
        dp[0] = row[s * 210 + 208];
        dp[1] = row[s * 210 + 209];
        dp[2] = row[(s + 4) * 210 + 208];
        dp[3] = row[(s + 4) * 210 + 209];
    }
}

// ------------------------------------------------------- Q8_0 quantize/dot

// q8_0.rs:31-58, one wave per two blocks (32 lanes per block).
__global__ void __launch_bounds__(kWG) quantize_q80_kernel(const float* __restrict__ src,
                                                           uint8_t* __restrict__ dst, size_t nblocks) {
    size_t t = (size_t)blockIdx.x * kWG + threadIdx.x;
    size_t b = t >> 5;
    int i = (int)(t & 31);
    bool valid = b < nblocks;
    float v = valid ? src[b * 32 + i] : 0.f;
    float a = fabsf(v);
#pragma unroll
    for (int s = 16; s >= 1; s >>= 1) a = fmaxf(a, __shfl_xor(a, s, 32));
    if (!valid) return;
    float d = a / 127.0f;
    float id = d != 0.0f ? 1.0f / d : 0.0f;
    float q = roundf(v * id);
    q = fminf(fmaxf(q, -128.0f), 127.0f);
    uint8_t* blk = dst + b * 34;
    blk[2 + i] = (uint8_t)(int8_t)q;
    if (i == 0) {
        uint32_t h = f32_to_half_bits(d);
        blk[0] = (uint8_t)(h & 0xFF);
        blk[1] = (uint8_t)(h >> 8);
    }
}

// q8_0.rs:60-124: sum of q*k over 32 values, times d
__global__ void __launch_bounds__(kWG) dot_q80_kernel(const float* __restrict__ q, const uint8_t* __restrict__ k,
                                                      float* __restrict__ out, size_t n) {
    size_t t = (size_t)blockIdx.x * kWG + threadIdx.x;
    size_t b = t >> 5;
    int i = (int)(t & 31);
    bool valid = b < n;
    float p = valid ? q[b * 32 + i] * (float)(int8_t)k[b * 34 + 2 + i] : 0.f;
#pragma unroll
    for (int s = 16; s >= 1; s >>= 1) p += __shfl_xor(p, s, 32);
    if (valid && i == 0) out[b] = p * half_bits_to_f32(k[b * 34] | (k[b * 34 + 1] << 8));
}

int pow2_ceil(int v) {
    int p = 1;
    while (p < v) p <<= 1;
    return p;
}

// Launch-shape knobs (defaults tuned on MI355X; the environment variables
// MIVI_GEMV_WG_PER_CU and MIVI_GEMV_U override them for sweeps).
int env_int(const char* name, int dflt) {
    const char* v = getenv(name);
    return v && *v ? atoi(v) : dflt;
}

int grid_for(int waves) {
    static const int per_cu = env_int("MIVI_GEMV_WG_PER_CU", 8);
    int wgs = (waves + 3) / 4;
    int cap = mivi::num_cus() * per_cu;
    return std::max(1, std::min(wgs, cap));
}

template <int PRO>
int32_t launch_pro(int32_t t, const mivi::GemvArgs& a, int n, hipStream_t s) {
    const int K = a.K;
    static const int u_env = env_int("MIVI_GEMV_U", 0);
    const int U = u_env ? u_env : (n >= 16384 ? 4 : 2);
#define L3(KER, LPR, UU) hipLaunchKernelGGL((KER<LPR, UU, PRO>), dim3(grid), dim3(kWG), lds, s, a)
#define BY_U(KER, LPR) \
    if (U == 4) L3(KER, LPR, 4); else L3(KER, LPR, 2)
#define BY_LPR(KER)                          \
    switch (lpr) {                           \
    case 1: BY_U(KER, 1); break;             \
    case 2: BY_U(KER, 2); break;             \
    case 4: BY_U(KER, 4); break;             \
    case 8: BY_U(KER, 8); break;             \
    case 16: BY_U(KER, 16); break;           \
    case 32: BY_U(KER, 32); break;           \
    default: BY_U(KER, 64); break;           \
    }
    // streaming kernel for the decode shapes, the generic kernel otherwise
    bool stream_ok = (t == MIVI_GGML_Q4_K || t == MIVI_GGML_Q6_K) && (K == 2048 || K == 4096 || K == 8192) &&
                     !env_int("MIVI_GEMV_V1", 0);
    // its staging loads activations as 16-byte vectors; the conv prologue is
    // specialised for the 3-tap window
    auto a16 = [](const void* p) { return p == nullptr || (uintptr_t)p % 16 == 0; };
    stream_ok = stream_ok && a16(a.x) && a16(a.x2) && a16(a.norm_w);
    if (PRO == mivi::PRO_CONV)
        stream_ok = stream_ok && K == 2048 && a.ksize == kConvKs && a16(a.st_in) && a16(a.st_out) &&
                    (a.conv_mode != 0 || a16(a.conv_w));
    if (a.ncol > 1 && !stream_ok) return mivi::set_error(MIVI_ERR_UNSUPPORTED, "no batched GEMV for this shape");
    if (stream_ok) {
        const int lpr = K == 2048 ? 32 : 64;
        const int ngroups = (n + 64 / lpr - 1) / (64 / lpr);
        // 2 workgroups per CU measured best for the head GEMV (24.7 us vs 26.2 at 3)
        const int per_cu = mivi::stream_wg_per_cu(n);
        const int grid = std::max(1, std::min((ngroups + 3) / 4, mivi::num_cus() * per_cu));
        if (a.packed && t == MIVI_GGML_Q4_K) {
            // packed Q4_K row quads on the matrix cores (one column)
            if constexpr (PRO == mivi::PRO_NONE || PRO == mivi::PRO_RMSNORM) {
                const int ep = a.epilogue;
                bool ok = (K == 2048 || K == 8192) && a.ncol <= 1 && ep != mivi::EPI_ARGMAX;
                for (int i = 0; i < a.nseg; i++) ok = ok && a.seg[i].n % 4 == 0;
                if (ep == mivi::EPI_SWIGLU) ok = ok && K == 2048 && a.nseg == 2 && a.seg[1].n == a.seg[0].n;
                if (ep == mivi::EPI_CONV)
                    ok = ok && K == 2048 && a.nseg == 1 && a.seg[0].n % 12 == 0 && a.ksize == kConvKs && a.st_in &&
                         a.st_out && (a.conv_mode == 2 || a.conv_w);
                if (!ok) return mivi::set_error(MIVI_ERR_UNSUPPORTED, "no Q4_K row-quad GEMV for this shape");
                const int nsteps = ep == mivi::EPI_SWIGLU ? a.seg[0].n / 4 : ep == mivi::EPI_CONV ? a.seg[0].n / 12 : n / 4;
                // one workgroup per CU at most (two for gate|up), each wave a
                // whole number of steps; PD: steps in flight, no more than a wave has
                // (gate|up: two workgroups per CU, one step of two quads per
                // wave: 2391 against 2365 tok/s on config 4; a store GEMV of
                // the same step count is slower so: config 1 4.53 against 4.02 us)
                const int qf = ep == mivi::EPI_SWIGLU ? 2 : 1;
                const int qg = std::max(1, std::min((nsteps + 3) / 4, mivi::num_cus() * qf));
                const int cmax = (nsteps + qg * 4 - 1) / (qg * 4);
                const int pd = (cmax >= 4 && K == 2048) ? 4 : cmax >= 2 ? 2 : 1;  // K = 8192: 2 (registers)
#define LQ4(EPI, S, PD) hipLaunchKernelGGL((gemv_q4k_quad_kernel<PRO, EPI, S, PD>), dim3(qg), dim3(kWG), 0, s, a)
#define LQ4P(EPI, S) \
    if (pd == 4) LQ4(EPI, S, 4); else if (pd == 2) LQ4(EPI, S, 2); else LQ4(EPI, S, 1)
                if (ep == mivi::EPI_SWIGLU) { LQ4P(mivi::EPI_SWIGLU, 1); }
                else if (ep == mivi::EPI_CONV) { LQ4P(mivi::EPI_CONV, 1); }
                else if (K == 2048) { LQ4P(mivi::EPI_STORE, 1); }
                else {
                    // K = 8192: the four waves of a workgroup split each quad
                    const int g8 = std::max(1, std::min(n / 4, mivi::num_cus()));
                    const int c8 = (n / 4 + g8 - 1) / g8;
#define LQ8(PD) hipLaunchKernelGGL((gemv_q4k_quad8k_kernel<PRO, PD>), dim3(g8), dim3(kWG), 0, s, a)
                    if (c8 >= 4) LQ8(4); else if (c8 >= 2) LQ8(2); else LQ8(1);
#undef LQ8
                }
#undef LQ4P
#undef LQ4
                MIVI_HIP_CHECK(hipGetLastError());
                return MIVI_OK;
            } else {
                return mivi::set_error(MIVI_ERR_UNSUPPORTED, "packed rows take no conv or SwiGLU prologue");
            }
        }
        if (a.epilogue == mivi::EPI_CONV) {
            // the ShortConv in_proj with the gated conv in its epilogue: Q4_K
            // rows at K = 2048, one segment of 3D rows [B|C|X]
            if constexpr (PRO == mivi::PRO_NONE || PRO == mivi::PRO_RMSNORM) {
                if (t != MIVI_GGML_Q4_K || K != 2048 || a.packed || a.nseg != 1 || a.seg[0].n % 3 != 0 ||
                    a.ksize != kConvKs || !a.st_in || !a.st_out || (a.conv_mode != 2 && !a.conv_w) ||
                    a.ncol > mivi::kMaxGemvCols)
                    return mivi::set_error(MIVI_ERR_UNSUPPORTED, "no conv epilogue for this shape");
                const int D3 = a.seg[0].n / 3;
                if (a.ncol > 2) {
                    if (a.ncol > 4) launch_cols<PRO, mivi::EPI_CONV, 2048, 2>(a, (D3 + 4) / 5, 1, s);
                    else launch_cols<PRO, mivi::EPI_CONV, 2048, 1>(a, (D3 + 4) / 5, 1, s);
                } else {
                    // in_proj's own mapping (two rows per wave), the channels'
                    // three row steps a ring round of three
                    const int gcv = std::max(1, std::min(((D3 + 1) / 2 + 3) / 4, mivi::num_cus() * per_cu));
                    if (a.ncol == 2)
                        hipLaunchKernelGGL((gemv_kq_stream_kernel<FMT_Q4K, 2048, 32, 1, 3, PRO, mivi::EPI_CONV, false, 2>),
                                           dim3(gcv), dim3(kWG), 0, s, a);
                    else
                        hipLaunchKernelGGL((gemv_kq_stream_kernel<FMT_Q4K, 2048, 32, 1, 3, PRO, mivi::EPI_CONV>),
                                           dim3(gcv), dim3(kWG), 0, s, a);
                }
                MIVI_HIP_CHECK(hipGetLastError());
                return MIVI_OK;
            } else {
                return mivi::set_error(MIVI_ERR_UNSUPPORTED, "the conv epilogue takes no conv or SwiGLU prologue");
            }
        }
        if (a.packed && mivi::quad_layout(n, K)) {
            // packed Q6_K row quads on the matrix cores (one segment: the quads span the matrix)
            if (t != MIVI_GGML_Q6_K || a.nseg != 1 || a.epilogue == mivi::EPI_SWIGLU)
                return mivi::set_error(MIVI_ERR_UNSUPPORTED, "packed row quads take one Q6_K segment, store or argmax");
            if constexpr (PRO == mivi::PRO_NONE || PRO == mivi::PRO_RMSNORM) {
                const int qgrid = mivi::quad_grid(n);  // even: as many waves in eight-wave workgroups
#define LQ(EPI, NC, PD) hipLaunchKernelGGL((gemv_q6k_quad_kernel<PRO, EPI, NC, PD>), dim3(qgrid), dim3(kWG), 0, s, a)
#define LQ8(EPI, PD, NGR) \
    hipLaunchKernelGGL((gemv_q6k_quad8_kernel<PRO, EPI, PD, NGR>), dim3(qgrid / 2), dim3(kQuad8WG), 0, s, a)
                if (a.ncol > 4) {
                    if (a.epilogue == mivi::EPI_ARGMAX) LQ8(mivi::EPI_ARGMAX, 3, 6); else LQ8(mivi::EPI_STORE, 3, 6);
                } else if (a.ncol > 2) {
                    if (a.epilogue == mivi::EPI_ARGMAX) LQ8(mivi::EPI_ARGMAX, 3, 3); else LQ8(mivi::EPI_STORE, 3, 3);
                } else if (a.epilogue == mivi::EPI_ARGMAX) {
                    if (a.ncol > 1) LQ(mivi::EPI_ARGMAX, 2, 2); else LQ(mivi::EPI_ARGMAX, 1, 3);
                } else {
                    if (a.ncol > 1) LQ(mivi::EPI_STORE, 2, 2); else LQ(mivi::EPI_STORE, 1, 3);
                }
#undef LQ
#undef LQ8
                MIVI_HIP_CHECK(hipGetLastError());
                return MIVI_OK;
            } else {
                return mivi::set_error(MIVI_ERR_UNSUPPORTED, "packed rows take no conv or SwiGLU prologue");
            }
        }
#define LSE(FMT, KT, LPR, NU, PD, EPI) \
    hipLaunchKernelGGL((gemv_kq_stream_kernel<FMT, KT, LPR, NU, PD, PRO, EPI>), dim3(grid), dim3(kWG), 0, s, a)
#define LS(FMT, KT, LPR, NU, PD) LSE(FMT, KT, LPR, NU, PD, mivi::EPI_STORE)
#define LSP(KT, LPR, NU, PD, EPI) \
    hipLaunchKernelGGL((gemv_kq_stream_kernel<FMT_Q6K, KT, LPR, NU, PD, PRO, EPI, true>), dim3(grid), dim3(kWG), 0, s, a)
        if (a.ncol > 1) {
            // batched columns (launch_gemv_ex passes at most gemv_max_cols):
            // the one-column kernel's mapping, so each column's result is
            // bit-identical to a one-column launch. Two columns at K = 2048
            // keep their digits in registers (PD 2 leaves room for them);
            // more columns (up to 8 at K = 2048, 4 at K = 8192) read them
            // from LDS each step (XL), so one launch reads each weight row
            // once for all of them.
#define LB(FMT, KT, LPR, NU, PD, EPI, PACK, NC)                                                                 \
    hipLaunchKernelGGL((gemv_kq_stream_kernel<FMT, KT, LPR, NU, PD, PRO, EPI, PACK, NC>), dim3(grid), dim3(kWG), 0, \
                       s, a)
#define LBX(FMT, EPI, G)                                                                                          \
    hipLaunchKernelGGL((gemv_kq_stream_kernel<FMT, 2048, 32, 1, 2, PRO, EPI, false, mivi::kMaxGemvCols, true>),   \
                       dim3(G), dim3(kWG), 0, s, a)
            const int ep = a.epilogue;
            const bool wide = a.ncol > 2 && !a.packed;
            // Q4_K, 3+ columns at K = 2048 or 2+ at K = 8192, store or SwiGLU
            // epilogue: the matrix-core kernel (same results, bit for bit)
            if (PRO != mivi::PRO_SWIGLU && t == MIVI_GGML_Q4_K && !a.packed && ep != mivi::EPI_ARGMAX &&
                ((K == 2048 && a.ncol > 2) || (K == 8192 && ep == mivi::EPI_STORE && PRO == mivi::PRO_NONE)) &&
                !env_int("MIVI_GEMV_COLS_SDOT", 0)) {
                if (ep == mivi::EPI_SWIGLU && (a.nseg != 2 || a.seg[1].n != a.seg[0].n))
                    return mivi::set_error(MIVI_ERR_INVALID_ARGUMENT, "SwiGLU epilogue needs gate|up of equal rows");
                // 16-row groups (8 gate|up channel pairs)
                const int ngr = ep == mivi::EPI_SWIGLU ? (a.seg[0].n + 7) / 8 : (n + 15) / 16;
                const int gy = (a.ncol + 3) / 4;
                if constexpr (PRO == mivi::PRO_SWIGLU) {
                } else if (K == 8192) {
                    // added into y: eight slices of the depth (config 5: 8320
                    // tok/s, 8300 at four slices, 7735 unsplit)
                    if constexpr (PRO == mivi::PRO_NONE) {
                        if (a.accumulate) {
                            if (a.ncol > 4) launch_cols_ksplit<8192, 8, 2>(a, ngr, s);
                            else launch_cols_ksplit<8192, 8, 1>(a, ngr, s);
                        } else {
                            launch_cols<PRO, mivi::EPI_STORE, 8192, 1>(a, ngr, gy, s);
                        }
                    }
                } else if (ep == mivi::EPI_SWIGLU) {
                    if (a.ncol > 4 && PRO != mivi::PRO_CONV) {
                        if constexpr (PRO != mivi::PRO_CONV) launch_cols<PRO, mivi::EPI_SWIGLU, 2048, 2>(a, ngr, 1, s);
                    } else {
                        launch_cols<PRO, mivi::EPI_SWIGLU, 2048, 1>(a, ngr, gy, s);
                    }
                } else if (PRO == mivi::PRO_NONE && a.accumulate && a.ncol > 4) {
                    // added into y, five or more columns: all of them in one
                    // workgroup over half the depth (8430 tok/s, 8390 as two
                    // groups of four columns over the whole depth)
                    if constexpr (PRO == mivi::PRO_NONE) launch_cols_ksplit<2048, 2, 2>(a, ngr, s);
                } else if (a.ncol > 4 && (ngr < mivi::num_cus() || PRO == mivi::PRO_CONV)) {
                    // fewer row groups than CUs (the 2048-row projections), or
                    // the conv prologue (whose eight columns at once would not
                    // fit the registers): the two groups of four columns side by side
                    launch_cols<PRO, mivi::EPI_STORE, 2048, 1>(a, ngr, gy, s);
                } else if (a.ncol > 4) {
                    if constexpr (PRO != mivi::PRO_CONV) launch_cols<PRO, mivi::EPI_STORE, 2048, 2>(a, ngr, 1, s);
                } else {
                    launch_cols<PRO, mivi::EPI_STORE, 2048, 1>(a, ngr, 1, s);
                }
                MIVI_HIP_CHECK(hipGetLastError());
                return MIVI_OK;
            }
            // the packed unit-plane kernel keeps two columns in registers
            if (a.packed && a.ncol > 2) return MIVI_ERR_UNSUPPORTED;
            if (K == 2048) {
                if (ep == mivi::EPI_STORE) {
                    if (a.packed) {
                        if constexpr (PRO == mivi::PRO_NONE || PRO == mivi::PRO_RMSNORM)
                            LB(FMT_Q6K, 2048, 32, 1, 2, mivi::EPI_STORE, true, 2);
                        else
                            return mivi::set_error(MIVI_ERR_UNSUPPORTED, "packed rows take no conv or SwiGLU prologue");
                    } else if (wide) {
                        if (t == MIVI_GGML_Q4_K) LBX(FMT_Q4K, mivi::EPI_STORE, grid); else LBX(FMT_Q6K, mivi::EPI_STORE, grid);
                    } else if (t == MIVI_GGML_Q4_K) LB(FMT_Q4K, 2048, 32, 1, 2, mivi::EPI_STORE, false, 2);
                    else LB(FMT_Q6K, 2048, 32, 1, 2, mivi::EPI_STORE, false, 2);
                } else if constexpr (PRO == mivi::PRO_NONE || PRO == mivi::PRO_RMSNORM) {
                    if (ep == mivi::EPI_SWIGLU) {
                        if (a.nseg != 2 || a.seg[1].n != a.seg[0].n)
                            return mivi::set_error(MIVI_ERR_INVALID_ARGUMENT, "SwiGLU epilogue needs gate|up of equal rows");
                        const int g1 = std::max(1, std::min((a.seg[0].n + 3) / 4, mivi::num_cus() * per_cu));
                        if (wide) {
                            if (t == MIVI_GGML_Q4_K) LBX(FMT_Q4K, mivi::EPI_SWIGLU, g1); else LBX(FMT_Q6K, mivi::EPI_SWIGLU, g1);
                        } else if (t == MIVI_GGML_Q4_K)
                            hipLaunchKernelGGL((gemv_kq_stream_kernel<FMT_Q4K, 2048, 32, 1, 2, PRO, mivi::EPI_SWIGLU, false, 2>),
                                               dim3(g1), dim3(kWG), 0, s, a);
                        else
                            hipLaunchKernelGGL((gemv_kq_stream_kernel<FMT_Q6K, 2048, 32, 1, 2, PRO, mivi::EPI_SWIGLU, false, 2>),
                                               dim3(g1), dim3(kWG), 0, s, a);
                    } else {
                        if (a.packed) LB(FMT_Q6K, 2048, 32, 1, 2, mivi::EPI_ARGMAX, true, 2);
                        else if (wide) {
                            if (t == MIVI_GGML_Q4_K) LBX(FMT_Q4K, mivi::EPI_ARGMAX, grid); else LBX(FMT_Q6K, mivi::EPI_ARGMAX, grid);
                        } else if (t == MIVI_GGML_Q4_K) LB(FMT_Q4K, 2048, 32, 1, 2, mivi::EPI_ARGMAX, false, 2);
                        else LB(FMT_Q6K, 2048, 32, 1, 2, mivi::EPI_ARGMAX, false, 2);
                    }
                } else {
                    return mivi::set_error(MIVI_ERR_UNSUPPORTED, "batched GEMV epilogue %d with this prologue", ep);
                }
            } else if (K == 8192 && ep == mivi::EPI_STORE && !a.packed) {
                // two units per lane: the columns' digits stay in LDS
                if constexpr (PRO == mivi::PRO_NONE) {
                    if (t == MIVI_GGML_Q4_K)
                        hipLaunchKernelGGL((gemv_kq_stream_kernel<FMT_Q4K, 8192, 64, 2, 2, PRO, mivi::EPI_STORE, false, 4, true>),
                                           dim3(grid), dim3(kWG), 0, s, a);
                    else
                        hipLaunchKernelGGL((gemv_kq_stream_kernel<FMT_Q6K, 8192, 64, 2, 2, PRO, mivi::EPI_STORE, false, 4, true>),
                                           dim3(grid), dim3(kWG), 0, s, a);
                } else {
                    return mivi::set_error(MIVI_ERR_UNSUPPORTED, "batched d=8192 GEMV takes no prologue");
                }
            } else {
                return mivi::set_error(MIVI_ERR_UNSUPPORTED, "no batched GEMV for d=%d", K);
            }
#undef LBX
#undef LB
            MIVI_HIP_CHECK(hipGetLastError());
            return MIVI_OK;
        }
        if (a.packed) {
            // packed Q6_K rows (store or argmax epilogue, no conv/SwiGLU prologue)
            if (t != MIVI_GGML_Q6_K || a.epilogue == mivi::EPI_SWIGLU)
                return mivi::set_error(MIVI_ERR_UNSUPPORTED, "packed rows are Q6_K with the store or argmax epilogue");
            if constexpr (PRO == mivi::PRO_NONE || PRO == mivi::PRO_RMSNORM) {
                // K = 2048: two units per lane, four rows per wave (about 4 %
                // faster than one unit per lane on the 65536-row head)
                if (a.epilogue == mivi::EPI_ARGMAX) {
                    if (K != 2048) return mivi::set_error(MIVI_ERR_UNSUPPORTED, "argmax epilogue needs K = 2048");
                    LSP(2048, 16, 2, 3, mivi::EPI_ARGMAX);
                } else if (K == 2048) LSP(2048, 16, 2, 3, mivi::EPI_STORE);
                else if (K == 4096) LSP(4096, 64, 1, 4, mivi::EPI_STORE);
                else LSP(8192, 64, 2, 2, mivi::EPI_STORE);
                MIVI_HIP_CHECK(hipGetLastError());
                return MIVI_OK;
            } else {
                return mivi::set_error(MIVI_ERR_UNSUPPORTED, "packed rows take no conv or SwiGLU prologue");
            }
        }
#undef LSP
        if (a.epilogue != mivi::EPI_STORE) {
            // the fused epilogues run at K = 2048 (two rows per wave)
            if (K != 2048 || PRO == mivi::PRO_SWIGLU || PRO == mivi::PRO_CONV)
                return mivi::set_error(MIVI_ERR_UNSUPPORTED, "GEMV epilogue %d needs K = 2048", a.epilogue);
            if constexpr (PRO == mivi::PRO_NONE || PRO == mivi::PRO_RMSNORM) {
                if (a.epilogue == mivi::EPI_SWIGLU) {
                    if (a.nseg != 2 || a.seg[1].n != a.seg[0].n)
                        return mivi::set_error(MIVI_ERR_INVALID_ARGUMENT, "SwiGLU epilogue needs gate|up of equal rows");
                    const int g1 = std::max(1, std::min((a.seg[0].n + 3) / 4, mivi::num_cus() * per_cu));
                    if (t == MIVI_GGML_Q4_K)
                        hipLaunchKernelGGL((gemv_kq_stream_kernel<FMT_Q4K, 2048, 32, 1, 4, PRO, mivi::EPI_SWIGLU>),
                                           dim3(g1), dim3(kWG), 0, s, a);
                    else
                        hipLaunchKernelGGL((gemv_kq_stream_kernel<FMT_Q6K, 2048, 32, 1, 4, PRO, mivi::EPI_SWIGLU>),
                                           dim3(g1), dim3(kWG), 0, s, a);
                } else {
                    if (t == MIVI_GGML_Q4_K) LSE(FMT_Q4K, 2048, 32, 1, 4, mivi::EPI_ARGMAX);
                    else if (n >= 32768) LSE(FMT_Q6K, 2048, 16, 2, 3, mivi::EPI_ARGMAX);
                    else LSE(FMT_Q6K, 2048, 32, 1, 4, mivi::EPI_ARGMAX);
                }
            }
            MIVI_HIP_CHECK(hipGetLastError());
            return MIVI_OK;
        }
        if (K == 2048) {
            // Q6_K heads (n >= 32768): two units per lane, four rows per wave,
            // about 1 us faster at 65536 rows; slower on the small Q4_K shapes
            if (t == MIVI_GGML_Q4_K) LS(FMT_Q4K, 2048, 32, 1, 4);
            else if (n >= 32768) LS(FMT_Q6K, 2048, 16, 2, 3);
            else LS(FMT_Q6K, 2048, 32, 1, 4);
        }
        if constexpr (PRO != mivi::PRO_CONV) {  // the conv prologue only runs at K = 2048
            if (K == 4096) {
                if (t == MIVI_GGML_Q4_K) LS(FMT_Q4K, 4096, 64, 1, 4); else LS(FMT_Q6K, 4096, 64, 1, 4);
            } else if (K == 8192) {
                if (t == MIVI_GGML_Q4_K) LS(FMT_Q4K, 8192, 64, 2, 2); else LS(FMT_Q6K, 8192, 64, 2, 2);
            }
        }
#undef LS
#undef LSE
        MIVI_HIP_CHECK(hipGetLastError());
        return MIVI_OK;
    }
    if (a.epilogue != mivi::EPI_STORE)
        return mivi::set_error(MIVI_ERR_UNSUPPORTED, "GEMV epilogue %d needs the streaming kernel", a.epilogue);
    if (a.packed) return mivi::set_error(MIVI_ERR_UNSUPPORTED, "packed rows need the streaming kernel (K = 2048/4096/8192)");
    switch (t) {
    case MIVI_GGML_Q4_K:
    case MIVI_GGML_Q6_K: {
        const int nb = K / 256;
        const int lpr = std::min(64, pow2_ceil(nb * 4));
        const size_t lds = (size_t)K * 4 + (size_t)K / (t == MIVI_GGML_Q4_K ? 32 : 16) * 4;
        const int grid = grid_for((n + (64 / lpr) * U - 1) / ((64 / lpr) * U));
        if (t == MIVI_GGML_Q4_K) {
            BY_LPR(gemv_q4k_kernel)
        } else {
            BY_LPR(gemv_q6k_kernel)
        }
        break;
    }
    case MIVI_GGML_Q8_0: {
        const int nb = K / 32;
        const int lpr = std::min(64, pow2_ceil(nb));
        const size_t lds = (size_t)K * 4;
        const int grid = grid_for((n + (64 / lpr) * U - 1) / ((64 / lpr) * U));
        BY_LPR(gemv_q80_kernel)
        break;
    }
    case MIVI_GGML_F16:
    case MIVI_GGML_BF16:
    case MIVI_GGML_F32: {
        const size_t lds = (size_t)K * 4;
        const int grid = grid_for(n);
        if (t == MIVI_GGML_F16) hipLaunchKernelGGL((gemv_dense_kernel<0, PRO>), dim3(grid), dim3(kWG), lds, s, a);
        else if (t == MIVI_GGML_BF16) hipLaunchKernelGGL((gemv_dense_kernel<1, PRO>), dim3(grid), dim3(kWG), lds, s, a);
        else hipLaunchKernelGGL((gemv_dense_kernel<2, PRO>), dim3(grid), dim3(kWG), lds, s, a);
        break;
    }
    default: return mivi::err_unsupported(t);
    }
#undef BY_LPR
#undef BY_U
#undef L3
    MIVI_HIP_CHECK(hipGetLastError());
    return MIVI_OK;
}

}  // namespace

// ------------------------------------------------------------ host launch

namespace mivi {

int stream_wg_per_cu(int n) {
    // Below 32768 rows a launch is bound by its fixed per-workgroup work (the
    // activation staging, one to a few ring steps per wave): one workgroup
    // per CU measured 2 us faster at K = 8192 (7.8 vs 9.8 us) and 0.2-0.5 us
    // faster on the K = 2048 decode shapes. Large matrices keep two.
    static const int env = env_int("MIVI_GEMV_STREAM_WG_PER_CU", 0);
    return env ? env : n >= 32768 ? 2 : 1;
}

int quad_grid(int n) {
    // 2 workgroups per CU measured best for the 65536-row head (18.7 us vs 20.6 at 3)
    // (even, so the eight-wave batched kernel launches as many waves)
    static const int per_cu = env_int("MIVI_GEMV_QUAD_WG_PER_CU", 2);
    const int g = std::max(1, std::min((n / 4 + 3) / 4, num_cus() * per_cu));
    return g + (g & 1);
}

int gemv_argmax_parts(int32_t t, int K, int n, bool packed) {
    if ((t != MIVI_GGML_Q4_K && t != MIVI_GGML_Q6_K) || K != 2048 || env_int("MIVI_GEMV_V1", 0)) return 0;
    if (packed && t == MIVI_GGML_Q6_K && quad_layout(n, K)) return 4 * quad_grid(n);
    const int per_cu = stream_wg_per_cu(n);
    const int ngroups = (n + 1) / 2;
    return 4 * std::max(1, std::min((ngroups + 3) / 4, num_cus() * per_cu));
}

// Most columns one batched streaming launch takes at depth K for n rows, 1
// where there is no batched kernel: 8 at K = 2048 (digits in LDS: 6 KB per
// column), 4 at K = 8192 (24 KB per column); packed Q6_K row quads take 8
// (the eight-wave quad kernel), packed unit planes (rows not a multiple of
// four) 2 (the streaming kernel with both columns in registers).
static int gemv_max_cols(int32_t t, int K, int n, bool packed, int pro = PRO_NONE, int epilogue = EPI_STORE) {
    if ((t != MIVI_GGML_Q4_K && t != MIVI_GGML_Q6_K) || env_int("MIVI_GEMV_V1", 0)) return 1;
    if (packed) return (t == MIVI_GGML_Q6_K && K == 2048) ? (quad_layout(n, K) ? kMaxGemvCols : 2) : 1;
    // Q4_K at K = 8192 on the matrix cores: column groups of four run side by
    // side in one launch (one workgroup per CU each)
    if (K == 8192 && t == MIVI_GGML_Q4_K && pro == PRO_NONE && epilogue == EPI_STORE &&
        !env_int("MIVI_GEMV_COLS_SDOT", 0))
        return kMaxGemvCols;
    return K == 2048 ? kMaxGemvCols : K == 8192 ? 4 : 1;
}

// Columns [c0, c0 + nc) of a batched GEMV as one launch's arguments.
static GemvArgs column_args(const GemvArgs& a, int c0, int nc) {
    GemvArgs v = a;
    v.x = a.x + c0 * a.xs;
    if (a.x2) v.x2 = a.x2 + c0 * a.xs;
    if (a.st_in) v.st_in = a.st_in + c0 * a.sts;
    if (a.st_out) v.st_out = a.st_out + c0 * a.sts;
    if (a.phase) v.phase = a.phase + c0;
    for (int i = 0; i < a.nseg; i++) v.seg[i].y = a.seg[i].y + c0 * a.ys;
    if (a.part_val) v.part_val = a.part_val + c0 * a.ps;
    if (a.part_idx) v.part_idx = a.part_idx + c0 * a.ps;
    v.ncol = nc;
    return v;
}

// one eight-wave workgroup per CU at most (64 KB of LDS each)
int t32_grid(int n) { return std::max(1, std::min((n / 32 + kQuad8Waves - 1) / kQuad8Waves, num_cus())); }
int t32_argmax_parts(int n) { return kQuad8Waves * t32_grid(n); }

int32_t launch_gemv_t32(int pro, const GemvArgs& a, hipStream_t s) {
    const int ncol = std::max(1, a.ncol);
    if (a.nseg != 1 || !t32_layout((size_t)a.seg[0].n, (size_t)a.K) || (a.epilogue != EPI_STORE && a.epilogue != EPI_ARGMAX) ||
        (pro != PRO_NONE && pro != PRO_RMSNORM) || (pro == PRO_RMSNORM && !a.norm_w) || ((uintptr_t)a.seg[0].W % 16) ||
        ((uintptr_t)a.x % 16) || (ncol > 1 && a.xs % 4) ||
        (a.epilogue == EPI_ARGMAX && (!a.part_val || !a.part_idx || (ncol > 1 && a.ps < t32_argmax_parts(a.seg[0].n)))))
        return set_error(MIVI_ERR_UNSUPPORTED, "no 32-row tile GEMV for this shape");
    const dim3 grid((unsigned)t32_grid(a.seg[0].n));
    // groups of at most eight columns
    for (int c0 = 0; c0 < ncol; c0 += kMaxGemvCols) {
        const GemvArgs v = column_args(a, c0, std::min(kMaxGemvCols, ncol - c0));
#define LT(P, E) hipLaunchKernelGGL((gemv_q6k_t32_kernel<P, E, 2>), grid, dim3(kQuad8WG), 0, s, v)
        if (pro == PRO_RMSNORM) {
            if (a.epilogue == EPI_ARGMAX) LT(PRO_RMSNORM, EPI_ARGMAX); else LT(PRO_RMSNORM, EPI_STORE);
        } else {
            if (a.epilogue == EPI_ARGMAX) LT(PRO_NONE, EPI_ARGMAX); else LT(PRO_NONE, EPI_STORE);
        }
#undef LT
    }
    MIVI_HIP_CHECK(hipGetLastError());
    return MIVI_OK;
}


static int32_t launch_by_pro(int32_t t, int pro, const GemvArgs& a, int n, hipStream_t s) {
    switch (pro) {
    case PRO_NONE: return launch_pro<PRO_NONE>(t, a, n, s);
    case PRO_RMSNORM: return launch_pro<PRO_RMSNORM>(t, a, n, s);
    case PRO_SWIGLU: return launch_pro<PRO_SWIGLU>(t, a, n, s);
    default: return launch_pro<PRO_CONV>(t, a, n, s);
    }
}

int32_t launch_gemv_ex(int32_t t, int pro, const GemvArgs& a, hipStream_t s) {
    int n = 0;
    for (int i = 0; i < a.nseg; i++) n += a.seg[i].n;
    if (n == 0 || a.K == 0) return MIVI_OK;
    if (a.ncol > 1) {
        // column groups of the batched kernel; columns it cannot take run
        // one launch each
        const int cap = gemv_max_cols(t, a.K, n, a.packed != 0, pro, a.epilogue);
        for (int c0 = 0; c0 < a.ncol;) {
            const int nc = std::min(cap, a.ncol - c0);
            int32_t rc = nc > 1 ? launch_by_pro(t, pro, column_args(a, c0, nc), n, s) : MIVI_ERR_UNSUPPORTED;
            if (rc == MIVI_ERR_UNSUPPORTED) {
                for (int c = c0; c < c0 + nc; c++)
                    if ((rc = launch_gemv_ex(t, pro, column_args(a, c, 1), s))) return rc;
            } else if (rc) {
                return rc;
            }
            c0 += nc;
        }
        return MIVI_OK;
    }
    if ((size_t)a.K > kMaxLdsK)
        return set_error(MIVI_ERR_UNSUPPORTED, "GEMV with d=%d exceeds the LDS staging limit %zu", a.K, kMaxLdsK);
    GemvArgs one = a;
    one.ncol = 1;
    return launch_by_pro(t, pro, one, n, s);
}

// Enqueues y[0..n) (=|+=) W[n, d] x for a validated problem.
int32_t launch_gemv(int32_t t, const uint8_t* W, const float* x, float* y, size_t n, size_t d,
                    bool accumulate, hipStream_t s) {
    GemvArgs a = {};
    a.seg[0] = {W, y, (int)n};
    a.nseg = 1;
    a.K = (int)d;
    a.x = x;
    a.accumulate = accumulate ? 1 : 0;
    return launch_gemv_ex(t, PRO_NONE, a, s);
}

int32_t launch_dequant(int32_t t, const uint8_t* src, float* out, size_t count, hipStream_t s) {
    // count = blocks (K-quants) or elements (dense)
    if (count == 0) return MIVI_OK;
    size_t threads;
    switch (t) {
    case MIVI_GGML_Q4_K:
        threads = count * 128;
        hipLaunchKernelGGL(dequant_q4k_kernel, dim3((threads + kWG - 1) / kWG), dim3(kWG), 0, s, src, out, count);
        break;
    case MIVI_GGML_Q6_K:
        threads = count * 64;
        hipLaunchKernelGGL(dequant_q6k_kernel, dim3((threads + kWG - 1) / kWG), dim3(kWG), 0, s, src, out, count);
        break;
    case MIVI_GGML_Q8_0:
        threads = count * 32;
        hipLaunchKernelGGL(dequant_q80_kernel, dim3((threads + kWG - 1) / kWG), dim3(kWG), 0, s, src, out, count);
        break;
    case MIVI_GGML_F16:
    case MIVI_GGML_BF16:
    case MIVI_GGML_F32:
        hipLaunchKernelGGL(dequant_dense_kernel, dim3((count + kWG - 1) / kWG), dim3(kWG), 0, s, src, out, count,
                           t == MIVI_GGML_F16 ? 0 : t == MIVI_GGML_BF16 ? 1 : 2);
        break;
    default: return err_unsupported(t);
    }
    MIVI_HIP_CHECK(hipGetLastError());
    return MIVI_OK;
}

int32_t launch_quantize_q80(const float* src, uint8_t* dst, size_t nblocks, hipStream_t s) {
    if (nblocks == 0) return MIVI_OK;
    size_t threads = nblocks * 32;
    hipLaunchKernelGGL(quantize_q80_kernel, dim3((threads + kWG - 1) / kWG), dim3(kWG), 0, s, src, dst, nblocks);
    MIVI_HIP_CHECK(hipGetLastError());
    return MIVI_OK;
}

// Block size / type size of the formats this library runs
// (types.rs:91-130); false for every other GgmlType.
bool format_sizes(int32_t t, size_t* bs, size_t* ts) {
    switch (t) {
    case MIVI_GGML_Q4_K: *bs = 256; *ts = 144; return true;
    case MIVI_GGML_Q6_K: *bs = 256; *ts = 210; return true;
    case MIVI_GGML_Q8_0: *bs = 32; *ts = 34; return true;
    case MIVI_GGML_F16:
    case MIVI_GGML_BF16: *bs = 1; *ts = 2; return true;
    case MIVI_GGML_F32: *bs = 1; *ts = 4; return true;
    default: return false;
    }
}

// Every GgmlType the reference's from_u32 accepts, with its block/type size
// when it has one (types.rs:55-137).
bool ggml_sizes(int32_t t, size_t* bs, size_t* ts) {
    switch (t) {
    case 0: case 26: *bs = 1; *ts = 4; return true;
    case 1: case 30: case 25: *bs = 1; *ts = 2; return true;
    case 24: *bs = 1; *ts = 1; return true;
    case 27: case 28: *bs = 1; *ts = 8; return true;
    case 2: *bs = 32; *ts = 18; return true;
    case 3: *bs = 32; *ts = 20; return true;
    case 6: *bs = 32; *ts = 22; return true;
    case 7: *bs = 32; *ts = 24; return true;
    case 8: *bs = 32; *ts = 34; return true;
    case 9: *bs = 32; *ts = 36; return true;
    case 10: *bs = 256; *ts = 84; return true;
    case 11: *bs = 256; *ts = 110; return true;
    case 12: *bs = 256; *ts = 144; return true;
    case 13: *bs = 256; *ts = 176; return true;
    case 14: *bs = 256; *ts = 210; return true;
    case 15: *bs = 256; *ts = 292; return true;
    default: return false;
    }
}

// types.rs:146-181 validate_matvec_args, with the row-byte arithmetic of
// each format's try_matvec_* (q4_k_m.rs:224-226, q6_k.rs:209-211,
// q8_0.rs:134-136, f16.rs:49-52, lib.rs:90-93).
int32_t validate_matvec(int32_t t, size_t out_len, size_t w_len, size_t x_len, size_t n, size_t d,
                        size_t* row_bytes_out) {
    size_t bs, ts, row_bytes;
    if (!format_sizes(t, &bs, &ts)) return err_unsupported(t);
    bool ovf = false;
    if (bs == 1) {
        if (__builtin_mul_overflow(d, ts, &row_bytes)) {
            if (t != MIVI_GGML_F32) return err_overflow();  // f16.rs:49-51
            ovf = true;                                    // lib.rs:90-93 maps it to BufferTooSmall
        }
    } else {
        row_bytes = (d / bs) * ts;
    }
    if (d % bs != 0) return err_misaligned(d, bs);
    if (out_len < n) return err_buffer_too_small(n, out_len);
    if (x_len < d) return err_buffer_too_small(d, x_len);
    size_t minw;
    if (ovf || __builtin_mul_overflow(n, row_bytes, &minw)) return err_buffer_too_small(SIZE_MAX, w_len);
    if (w_len < minw) return err_buffer_too_small(minw, w_len);
    if (row_bytes_out) *row_bytes_out = row_bytes;
    return MIVI_OK;
}

}  // namespace mivi

// ------------------------------------------------------------ Q6_K packing

namespace {
// one thread per (row, unit): moves the unit's bytes into the plane layout
// of load_unit_q6k_packed (a permutation of the row's bytes)
__global__ void __launch_bounds__(kWG) pack_q6k_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                                       size_t rows, int nu, size_t row_bytes) {
    const size_t i = (size_t)blockIdx.x * kWG + threadIdx.x;
    if (i >= rows * (size_t)nu) return;
    const size_t r = i / nu;
    const int u = (int)(i % nu), b = u >> 2, h = (u >> 1) & 1, j = u & 1;
    const uint8_t* p = src + r * row_bytes + (size_t)b * 210;
    uint8_t* q = dst + r * row_bytes;
    for (int k = 0; k < 16; k++) {
        q[16 * u + k] = p[64 * h + 16 * j + k];
        q[16 * nu + 16 * u + k] = p[64 * h + 32 + 16 * j + k];
        q[32 * nu + 16 * u + k] = p[128 + 32 * h + 16 * j + k];
    }
    for (int k = 0; k < 4; k++) q[48 * nu + 4 * u + k] = p[192 + 8 * h + j + 2 * k];
    if ((u & 3) == 0) {
        q[52 * nu + 2 * b] = p[208];
        q[52 * nu + 2 * b + 1] = p[209];
    }
}

// One thread per (chunk, lane) of the 32-row tile layout (gemv_q6k_t32_kernel):
// the lane's 96 code bytes and, for lanes l < 32, its row's scales and d.
__global__ void __launch_bounds__(kWG) pack_q6k_t32_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                                           size_t nchunks) {
    const size_t i = (size_t)blockIdx.x * kWG + threadIdx.x;
    if (i >= nchunks * 64) return;
    const size_t c = i >> 6;
    const int l = (int)(i & 63), n = l & 31, hh = l >> 5;
    const size_t T = c / 8;
    const int sb = (int)(c % 8);
    const uint8_t* blk = src + (32 * T + n) * 1680 + (size_t)sb * 210;
    uint8_t* o = dst + c * kT32Bytes + 64 * (c & 1);  // codes and scales
    uint8_t* od = dst + c * kT32Bytes + ((c & 1) ? 0 : 6656);
    for (int P = 0; P < 8; P++) {
        uint32_t cd[16];
        for (int e = 0; e < 16; e++) {
            const int v = 16 * (2 * P + (e >> 3)) + 8 * hh + (e & 7);  // value of the superblock
            cd[e] = q6_code(blk, v >> 7, (v >> 5) & 3, v & 31);
        }
        for (int m = 0; m < 3; m++) {
            uint32_t word = 0;
            for (int e = 0; e < 4; e++) word |= (cd[4 * m + e] | (((cd[12 + e] >> (2 * m)) & 3u) << 6)) << (8 * e);
            const int D = 3 * P + m;
            *(uint32_t*)(o + 1024 * (D >> 2) + 16 * l + 4 * (D & 3)) = word;
        }
    }
    if (hh == 0) {
        for (int k = 0; k < 16; k++) o[6144 + 16 * n + k] = blk[192 + k];
        od[2 * n] = blk[208];
        od[2 * n + 1] = blk[209];
    }
}
}  // namespace

namespace mivi {
int32_t launch_pack_q6k(const uint8_t* src, uint8_t* dst, size_t rows, size_t cols, hipStream_t s) {
    if (quad_layout(rows, cols)) {
        const size_t threads = rows / 4 * 64;
        if (threads == 0) return MIVI_OK;
        hipLaunchKernelGGL(pack_q6k_quad_kernel, dim3((unsigned)((threads + kWG - 1) / kWG)), dim3(kWG), 0, s, src, dst,
                           rows / 4);
        MIVI_HIP_CHECK(hipGetLastError());
        return MIVI_OK;
    }
    const int nu = (int)(cols / 64);
    const size_t threads = rows * (size_t)nu;
    if (threads == 0) return MIVI_OK;
    hipLaunchKernelGGL(pack_q6k_kernel, dim3((unsigned)((threads + kWG - 1) / kWG)), dim3(kWG), 0, s, src, dst, rows,
                       nu, (cols / 256) * 210);
    MIVI_HIP_CHECK(hipGetLastError());
    return MIVI_OK;
}

// One thread per (group, superblock, lane slot l = j + 16 kg): its 32 code
// bytes, and (kg = 0) row j's header with the scales and mins decoded.
__global__ void __launch_bounds__(kWG) pack_q4k_cols_kernel(const uint64_t* __restrict__ rows, int ngroups, int nbt,
                                                            uint8_t* __restrict__ dst) {
    const size_t i = (size_t)blockIdx.x * kWG + threadIdx.x;
    if (i >= (size_t)ngroups * nbt * 64) return;
    const int l = (int)(i & 63), j = l & 15, kg = l >> 4;
    const size_t gsb = i >> 6;  // group * nbt + superblock
    const int sb = (int)(gsb % nbt);
    const uint8_t* src = (const uint8_t*)rows[(gsb / nbt) * 16 + j] + 144 * sb;
    uint8_t* d = dst + gsb * kColsChunkBytes;
    u32x2 c[4];
#pragma unroll
    for (int g = 0; g < 4; g++) c[g] = *(const u32x2*)(src + 16 + 32 * g + 8 * kg);
    *(u32x4*)(d + kColsCodesOff + 16 * l) = u32x4{c[0].x, c[0].y, c[1].x, c[1].y};
    *(u32x4*)(d + kColsCodesOff + 1024 + 16 * l) = u32x4{c[2].x, c[2].y, c[3].x, c[3].y};
    if (kg == 0) {
        const u32x4 h = *(const u32x4*)src;
        uint32_t sc[8], mn[8];
#pragma unroll
        for (int g = 0; g < 4; g++) q4k_scales(h.y, h.z, h.w, g, sc[2 * g], mn[2 * g], sc[2 * g + 1], mn[2 * g + 1]);
        auto bytes4 = [](const uint32_t* v) { return v[0] | v[1] << 8 | v[2] << 16 | v[3] << 24; };
        *(u32x4*)(d + 16 * j) = u32x4{h.x, bytes4(sc), bytes4(sc + 4), bytes4(mn)};
        *(uint32_t*)(d + kColsMinsOff + 4 * j) = bytes4(mn + 4);
    }
}

int32_t launch_pack_q6k_t32(const uint8_t* src, uint8_t* dst, size_t rows, size_t cols, hipStream_t s) {
    if (!t32_layout(rows, cols) || ((uintptr_t)dst % 16))
        return set_error(MIVI_ERR_UNSUPPORTED, "no 32-row tile layout for %zu x %zu Q6_K", rows, cols);
    const size_t nchunks = rows / 32 * (cols / 256);
    hipLaunchKernelGGL(pack_q6k_t32_kernel, dim3((unsigned)((nchunks * 64 + kWG - 1) / kWG)), dim3(kWG), 0, s, src,
                       dst, nchunks);
    MIVI_HIP_CHECK(hipGetLastError());
    return MIVI_OK;
}

int32_t launch_pack_q4k_cols(const uint8_t* const* rows_host, int ngroups, size_t cols, uint8_t* dst,
                             hipStream_t s) {
    if (ngroups <= 0) return MIVI_OK;
    if (cols % 256) return set_error(MIVI_ERR_INVALID_ARGUMENT, "Q4_K rows of %zu columns", cols);
    for (size_t i = 0; i < (size_t)ngroups * 16; i++)
        if ((uintptr_t)rows_host[i] % 16)
            return set_error(MIVI_ERR_INVALID_ARGUMENT, "Q4_K rows must be 16-byte aligned to pack");
    uint64_t* d = nullptr;
    const size_t tb = (size_t)ngroups * 16 * sizeof(uint64_t);
    MIVI_HIP_CHECK(hipMalloc(&d, tb));
    hipError_t e = hipMemcpy(d, rows_host, tb, hipMemcpyHostToDevice);
    const int nbt = (int)(cols / 256);
    const size_t threads = (size_t)ngroups * nbt * 64;
    if (e == hipSuccess) {
        hipLaunchKernelGGL(pack_q4k_cols_kernel, dim3((unsigned)((threads + kWG - 1) / kWG)), dim3(kWG), 0, s, d,
                           ngroups, nbt, dst);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    const hipError_t f = hipFree(d);
    if (e != hipSuccess) return set_error(MIVI_ERR_HIP, "packing Q4_K rows for the column kernel: %s", hipGetErrorString(e));
    if (f != hipSuccess) return set_error(MIVI_ERR_HIP, "hipFree: %s", hipGetErrorString(f));
    return MIVI_OK;
}

int32_t launch_pack_q4k(const uint8_t* src, uint8_t* dst, size_t rows, size_t cols, hipStream_t s) {
    const int S = (int)(cols / 2048);
    const size_t threads = rows / 4 * (size_t)S * 64;
    if (threads == 0) return MIVI_OK;
    hipLaunchKernelGGL(pack_q4k_quad_kernel, dim3((unsigned)((threads + kWG - 1) / kWG)), dim3(kWG), 0, s, src, dst,
                       rows / 4, S);
    MIVI_HIP_CHECK(hipGetLastError());
    return MIVI_OK;
}
}  // namespace mivi

// --------------------------------------------------------- read floor probe

// external linkage, so that the store below (and the loads feeding it) stay
__device__ uint32_t mivi_read_floor_sink;

namespace {

// The floor for any kernel that reads these bytes once: a persistent grid of
// 2 workgroups per CU reads 16 bytes per lane, four loads in flight per
// iteration, and folds them into one word per thread that is stored only
// when it equals `key`, a value known only at run time (so the compiler keeps
// the loads; a stored word is harmless).
__global__ void __launch_bounds__(kWG) read_floor_kernel(const u32x4* __restrict__ p, size_t n16, uint32_t key) {
    const size_t nt = (size_t)gridDim.x * kWG;
    size_t i = (size_t)blockIdx.x * kWG + threadIdx.x;
    uint32_t acc = 0;
    for (; i + 3 * nt < n16; i += 4 * nt) {
        u32x4 v[4];
#pragma unroll
        for (int u = 0; u < 4; u++) v[u] = __builtin_nontemporal_load(p + i + u * nt);
#pragma unroll
        for (int u = 0; u < 4; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    for (; i < n16; i += nt) {
        const u32x4 v = p[i];
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (acc == key) mivi_read_floor_sink = acc;
}

}  // namespace

// -------------------------------------------------------------------- C ABI

using namespace mivi;

extern "C" int32_t mivi_hip_read_floor(const uint8_t* p, size_t bytes, void* stream) {
    if (bytes % 16) return err_misaligned(bytes, 16);
    if (bytes && !p) return set_error(MIVI_ERR_INVALID_ARGUMENT, "null buffer");
    if ((uintptr_t)p % 16) return set_error(MIVI_ERR_INVALID_ARGUMENT, "buffer must be 16-byte aligned");
    clear_error();
    if (bytes == 0) return MIVI_OK;
    const size_t n16 = bytes / 16;
    const size_t need = (n16 + kWG - 1) / kWG;
    const int grid = (int)std::max<size_t>(1, std::min<size_t>(need, (size_t)num_cus() * 2));
    hipLaunchKernelGGL(read_floor_kernel, dim3(grid), dim3(kWG), 0, (hipStream_t)stream, (const u32x4*)p, n16,
                       0x9E3779B9u);
    MIVI_HIP_CHECK(hipGetLastError());
    return MIVI_OK;
}

// Packed rows: Q6_K with d in {2048, 4096, 8192} (the streaming kernel's
// shapes), Q4_K with d in {2048, 8192} and a multiple of 4 rows (row quads).
static bool packable(int32_t t, size_t d, size_t rows) {
    if (t == MIVI_GGML_Q6_K) return d == 2048 || d == 4096 || d == 8192;
    return t == MIVI_GGML_Q4_K && (d == 2048 || d == 8192) && rows % 4 == 0;
}

extern "C" int32_t mivi_hip_pack_weights(int32_t t, const uint8_t* src, size_t src_len, uint8_t* dst,
                                         size_t dst_len, size_t rows, size_t cols, void* stream) {
    size_t bs, ts;
    if (!format_sizes(t, &bs, &ts)) return err_unsupported(t);
    if (cols % bs != 0) return err_misaligned(cols, bs);
    size_t need;
    if (__builtin_mul_overflow(rows, (cols / bs) * ts, &need)) return err_overflow();
    if (src_len < need) return err_buffer_too_small(need, src_len);
    if (dst_len < need) return err_buffer_too_small(need, dst_len);
    if (!packable(t, cols, rows))
        return set_error(MIVI_ERR_UNSUPPORTED, "no packed layout for type %d with %zu rows of %zu columns", t, rows,
                         cols);
    if (rows && (!src || !dst)) return set_error(MIVI_ERR_INVALID_ARGUMENT, "null buffer");
    if (src == dst && rows) return set_error(MIVI_ERR_INVALID_ARGUMENT, "packing needs distinct buffers");
    clear_error();
    if (t == MIVI_GGML_Q4_K) return launch_pack_q4k(src, dst, rows, cols, (hipStream_t)stream);
    return launch_pack_q6k(src, dst, rows, cols, (hipStream_t)stream);
}

extern "C" int32_t mivi_hip_quantized_matvec_packed(float* out, size_t out_len, int32_t t, const uint8_t* packed,
                                                    size_t packed_len, const float* x, size_t x_len, size_t n,
                                                    size_t d, void* stream) {
    int32_t rc = validate_matvec(t, out_len, packed_len, x_len, n, d, nullptr);
    if (rc) return rc;
    if (!packable(t, d, n))
        return set_error(MIVI_ERR_UNSUPPORTED, "no packed layout for type %d with %zu rows of %zu columns", t, n, d);
    if (n && (!out || !packed || !x)) return set_error(MIVI_ERR_INVALID_ARGUMENT, "null buffer");
    if ((uintptr_t)packed % 16) return set_error(MIVI_ERR_INVALID_ARGUMENT, "packed rows must be 16-byte aligned");
    if (n > (size_t)INT32_MAX) return err_overflow();
    clear_error();
    if (n == 0) return MIVI_OK;
    GemvArgs a = {};
    a.seg[0] = {packed, out, (int)n};
    a.nseg = 1;
    a.K = (int)d;
    a.x = x;
    a.packed = 1;
    return launch_gemv_ex(t, PRO_NONE, a, (hipStream_t)stream);
}

extern "C" int32_t mivi_hip_quantized_matmul_rows_packed(float* out, size_t out_len, int32_t t,
                                                        const uint8_t* packed, size_t packed_len, const float* in,
                                                        size_t in_len, size_t batch, size_t rows, size_t cols,
                                                        void* stream) {
    // the sizes and errors of mivi_hip_quantized_matmul_rows (types.rs:188-235)
    size_t bs, ts, row_bytes, e;
    if (!format_sizes(t, &bs, &ts)) return err_unsupported(t);
    if (cols % bs != 0) return err_misaligned(cols, bs);
    if (__builtin_mul_overflow(cols / bs, ts, &row_bytes)) return err_overflow();
    if (__builtin_mul_overflow(batch, rows, &e)) return err_overflow();
    if (out_len < e) return err_buffer_too_small(e, out_len);
    if (__builtin_mul_overflow(batch, cols, &e)) return err_overflow();
    if (in_len < e) return err_buffer_too_small(e, in_len);
    if (__builtin_mul_overflow(rows, row_bytes, &e)) return err_overflow();
    if (packed_len < e) return err_buffer_too_small(e, packed_len);
    if (!packable(t, cols, rows))
        return set_error(MIVI_ERR_UNSUPPORTED, "no packed layout for type %d with %zu rows of %zu columns", t, rows,
                         cols);
    if (batch == 0 || rows == 0) return clear_error();
    if (!out || !packed || !in) return set_error(MIVI_ERR_INVALID_ARGUMENT, "null buffer");
    if ((uintptr_t)packed % 16) return set_error(MIVI_ERR_INVALID_ARGUMENT, "packed rows must be 16-byte aligned");
    if (rows > (size_t)INT32_MAX || batch > (size_t)INT32_MAX) return err_overflow();
    clear_error();
    // the inputs as columns of batched launches (up to eight per launch for
    // Q6_K row quads, one per launch otherwise)
    GemvArgs a = {};
    a.seg[0] = {packed, out, (int)rows};
    a.nseg = 1;
    a.K = (int)cols;
    a.x = in;
    a.packed = 1;
    a.ncol = (int)batch;
    a.xs = (int64_t)cols;
    a.ys = (int64_t)rows;
    return launch_gemv_ex(t, PRO_NONE, a, (hipStream_t)stream);
}

static int32_t matvec_typed(int32_t t, float* out, size_t out_len, const uint8_t* w, size_t w_len,
                            const float* x, size_t x_len, size_t n, size_t d, void* stream) {
    int32_t rc = validate_matvec(t, out_len, w_len, x_len, n, d, nullptr);
    if (rc) return rc;
    if (n && (!out || !w || (d && !x))) return set_error(MIVI_ERR_INVALID_ARGUMENT, "null buffer");
    clear_error();
    return launch_gemv(t, w, x, out, n, d, false, (hipStream_t)stream);
}

extern "C" int32_t mivi_hip_quantized_matvec(float* out, size_t out_len, int32_t t, const uint8_t* w,
                                             size_t w_len, const float* x, size_t x_len, size_t n, size_t d,
                                             void* stream) {
    return matvec_typed(t, out, out_len, w, w_len, x, x_len, n, d, stream);
}

#define TYPED_ENTRY(NAME, T)                                                                          \
    extern "C" int32_t NAME(float* out, size_t out_len, const uint8_t* w, size_t w_len, const float* x, \
                            size_t x_len, size_t n, size_t d, void* stream) {                        \
        return matvec_typed(T, out, out_len, w, w_len, x, x_len, n, d, stream);                      \
    }
TYPED_ENTRY(mivi_hip_try_matvec_q4_k_m, MIVI_GGML_Q4_K)
TYPED_ENTRY(mivi_hip_try_matvec_q6_k, MIVI_GGML_Q6_K)
TYPED_ENTRY(mivi_hip_try_matvec_q8_0, MIVI_GGML_Q8_0)
TYPED_ENTRY(mivi_hip_try_matvec_f16, MIVI_GGML_F16)
TYPED_ENTRY(mivi_hip_try_matvec_bf16, MIVI_GGML_BF16)
#undef TYPED_ENTRY

extern "C" int32_t mivi_hip_dequantize_slice(int32_t t, const uint8_t* bytes, size_t bytes_len, float* out,
                                             size_t out_len, void* stream) {
    size_t bs, ts;
    if (!format_sizes(t, &bs, &ts)) return err_unsupported(t);
    size_t count;
    if (bs == 1) {
        count = bytes_len / ts;  // f16.rs:17-23, lib.rs:58-63
        if (out_len < count) return err_buffer_too_small(count, out_len);
    } else {
        count = out_len / bs;    // types.rs:281-285
        if (bytes_len < count * ts) return err_buffer_too_small(count * ts, bytes_len);
    }
    if (count && (!bytes || !out)) return set_error(MIVI_ERR_INVALID_ARGUMENT, "null buffer");
    clear_error();
    return launch_dequant(t, bytes, out, count, (hipStream_t)stream);
}

extern "C" int32_t mivi_hip_quantize_q8_0(const float* src, size_t src_len, uint8_t* dst, size_t dst_len,
                                          size_t n_blocks, void* stream) {
    if (src_len < n_blocks * 32) return err_buffer_too_small(n_blocks * 32, src_len);
    if (dst_len < n_blocks * 34) return err_buffer_too_small(n_blocks * 34, dst_len);
    clear_error();
    return launch_quantize_q80(src, dst, n_blocks, (hipStream_t)stream);
}

extern "C" int32_t mivi_hip_dot_q8_0_f32(const float* q, size_t q_len, const uint8_t* k, size_t k_len, float* out,
                                         size_t out_len, size_t n, void* stream) {
    if (q_len < n * 32) return err_buffer_too_small(n * 32, q_len);
    if (k_len < n * 34) return err_buffer_too_small(n * 34, k_len);
    if (out_len < n) return err_buffer_too_small(n, out_len);
    clear_error();
    if (n == 0) return MIVI_OK;
    size_t threads = n * 32;
    hipLaunchKernelGGL(dot_q80_kernel, dim3((threads + kWG - 1) / kWG), dim3(kWG), 0, (hipStream_t)stream, q, k, out, n);
    MIVI_HIP_CHECK(hipGetLastError());
    return MIVI_OK;
}
