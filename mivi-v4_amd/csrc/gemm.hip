// quantized_matmul_rows (crates/mivi-quant/src/lib.rs:143-357) for gfx950.
//
// batch == 1 is exactly the matvec path (lib.rs:171-182). Q4_K and Q6_K with
// at least kMfmaMinBatch rows run on the matrix cores:
//
//   gemm_prep_kernel   one workgroup per input row: scales the row by a power
//                      of two 2^-e (so that |x| <= 1), splits it into fp16
//                      hi + lo (x = hi + lo to about 2^-22 relative) and forms
//                      the fp32 sums of each 32-value sub-block, also split;
//   gemm_q4k_kernel    64 x 256 output tiles (input rows x weight rows),
//                      v_mfma_f32_32x32x16_f16. The
//                      B operand is sc*q of the Q4_K sub-block, an integer
//                      <= 945 and so exact in fp16; one MFMA chain per 256-value
//                      super-block gives sum(sc q x), folded into the fp32
//                      accumulator as acc += d * C. The min term of
//                      q4_k_m.rs:24-63, dmin * sum_sub m_sub * X_sub, runs on
//                      the same MFMA shape with B = m (K = 8 sub-blocks padded
//                      to 16) and is subtracted the same way. The row scale
//                      2^e is applied at the store.
//   gemm_q6k_kernel    the same tiles for Q6_K: B = q (exact in fp16), the
//                      per-sub-block scale d * sc applied to each k-step's
//                      chain (one 32 x 32 x 16 product per 16-value
//                      sub-block).
//
// Other formats, and fewer rows, run the batched GEMV (the inputs as its
// columns).
#include <mutex>
#include <type_traits>
#include <vector>

#include "common.h"
#include "gemv.h"

namespace mivi {
bool format_sizes(int32_t t, size_t* bs, size_t* ts);
bool ggml_sizes(int32_t t, size_t* bs, size_t* ts);
}  // namespace mivi

using namespace mivi;

namespace {

constexpr int kMfmaMinBatch = 16;
constexpr int kTm = 64;             // input rows of a GEMM tile
constexpr int kTk = 64;             // k-tile: one Q4_K group (a sub-block pair)
constexpr int kXs = kTk + 8;        // padded LDS row (halves) of an x or B tile

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// ---------------------------------------------------------------- prep
// grid = Mp rows, 256 threads, K = 8 * 256 * r (thread t owns values
// [8t, 8t + 8) of each 2048-value stretch). Row m < M is v = pro(X row m)
// with X row m at X + m * ldx: PRO_NONE v = x; PRO_RMSNORM v = (x * s) * w,
// s = 1/sqrt(mean(x^2) + eps) (norm.rs:38-72); PRO_SWIGLU v = silu(x) * x2
// (math.rs:87-95, X2 row m at X2 + m * ldx). Then e = exponent with
// max|v| * 2^-e <= 1; xh/xl = fp16 hi/lo of v * 2^-e; sh/sl = fp16 hi/lo of
// each 32-value sub-block sum of v * 2^-e (fp32). Rows >= M are zero.
typedef _Float16 half8p __attribute__((ext_vector_type(8)));
// R > 0: K = 2048 R, the thread's 8 R values (and norm weights or up values)
// loaded once and held in registers through both reductions; R = 0: any K,
// each pass re-reading them. The same operations in the same order either way.
template <int R>
__global__ void __launch_bounds__(256) gemm_prep_kernel(const float* __restrict__ X, const float* __restrict__ X2,
                                                        const float* __restrict__ norm_w, float eps, int pro,
                                                        int64_t ldx, int M, int K, _Float16* __restrict__ xh,
                                                        _Float16* __restrict__ xl, _Float16* __restrict__ sh,
                                                        _Float16* __restrict__ sl, float* __restrict__ rowscale) {
    __shared__ float red[4];
    const int m = blockIdx.x;
    const bool live = m < M;
    const float* x = X + (live ? m : 0) * ldx;
    const float* x2 = pro == PRO_SWIGLU ? X2 + (live ? m : 0) * ldx : nullptr;
    auto block_red = [&](float v, bool is_max) {
        v = is_max ? wave_max(v) : wave_sum(v);
        __syncthreads();
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
        __syncthreads();
        return is_max ? fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])) : (red[0] + red[1]) + (red[2] + red[3]);
    };
    // the 8 values [i, i + 8) of a row as two 16-byte loads
    auto load8 = [&](const float* p, int i, float (&v)[8]) {
        const f32x4 a = *(const f32x4*)(p + i), b = *(const f32x4*)(p + i + 4);
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    };
    constexpr int RR = R > 0 ? R : 1;
    float xr[RR][8], wr[RR][8];  // R > 0: x and (norm w | up) of stretch r
    if constexpr (R > 0) {
#pragma unroll
        for (int r = 0; r < R; r++) {
#pragma unroll
            for (int q = 0; q < 8; q++) { xr[r][q] = 0.f; wr[r][q] = 0.f; }
            if (live) {
                load8(x, 2048 * r + 8 * threadIdx.x, xr[r]);
                if (pro == PRO_RMSNORM) load8(norm_w, 2048 * r + 8 * threadIdx.x, wr[r]);
                else if (pro == PRO_SWIGLU) load8(x2, 2048 * r + 8 * threadIdx.x, wr[r]);
            }
        }
    }
    float scale = 1.0f;
    if (pro == PRO_RMSNORM) {
        float ss = 0.f;
        if constexpr (R > 0) {
#pragma unroll
            for (int r = 0; r < R; r++)
#pragma unroll
                for (int q = 0; q < 8; q++) ss = fmaf(xr[r][q], xr[r][q], ss);
        } else if (live) {
            for (int i = 8 * threadIdx.x; i < K; i += 8 * 256) {
                float v[8];
                load8(x, i, v);
#pragma unroll
                for (int q = 0; q < 8; q++) ss = fmaf(v[q], v[q], ss);
            }
        }
        ss = block_red(ss, false);
        scale = 1.0f / sqrtf(ss / (float)K + eps);
    }
    auto values = [&](int r, int i, float (&v)[8]) {  // pro(x)[i .. i + 8), i = 2048 r + 8 t
        float w[8];
        if constexpr (R > 0) {
#pragma unroll
            for (int q = 0; q < 8; q++) { v[q] = xr[r][q]; w[q] = wr[r][q]; }
        } else {
            load8(x, i, v);
            if (pro == PRO_RMSNORM) load8(norm_w, i, w);
            else if (pro == PRO_SWIGLU) load8(x2, i, w);
        }
        if (pro == PRO_RMSNORM) {
#pragma unroll
            for (int q = 0; q < 8; q++) v[q] = v[q] * scale * w[q];
        } else if (pro == PRO_SWIGLU) {
#pragma unroll
            for (int q = 0; q < 8; q++) v[q] = silu_f(v[q]) * w[q];
        }
    };
    // stretch r of the thread: values [2048 r + 8 t, + 8)
    auto more = [&](int r) { return R > 0 ? r < R : 2048 * r + 8 * (int)threadIdx.x < K; };
    float mx = 0.f;
    if (live)
        for (int r = 0; more(r); r++) {  // (R > 0: unrolled, the registers indexed statically)
            const int i = 2048 * r + 8 * threadIdx.x;
            float v[8];
            values(r, i, v);
#pragma unroll
            for (int q = 0; q < 8; q++) mx = fmaxf(mx, fabsf(v[q]));
        }
    mx = block_red(mx, true);
    // 2^-e with max * 2^-e in [1/2, 1); e = 0 for an all-zero row
    int e = 0;
    if (mx > 0.f && mx <= 3.40282347e38f) frexpf(mx, &e);
    const float inv = ldexpf(1.0f, -e);
    if (threadIdx.x == 0) rowscale[m] = live ? ldexpf(1.0f, e) : 0.f;
    for (int r = 0; more(r); r++) {
        const int i = 2048 * r + 8 * threadIdx.x;
        float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        if (live) values(r, i, v);
#pragma unroll
        for (int q = 0; q < 8; q++) v[q] *= inv;  // exact: power-of-two scaling
        half8p hv, lv;
        float sum = 0.f;
#pragma unroll
        for (int q = 0; q < 8; q++) {
            hv[q] = (_Float16)v[q];
            lv[q] = (_Float16)(v[q] - (float)hv[q]);
            sum += v[q];
        }
        *(half8p*)(xh + (size_t)m * K + i) = hv;
        *(half8p*)(xl + (size_t)m * K + i) = lv;
        // 4 consecutive threads hold one 32-value sub-block
        sum += __shfl_xor(sum, 1, 64);
        sum += __shfl_xor(sum, 2, 64);
        if ((threadIdx.x & 3) == 0) {
            const _Float16 h = (_Float16)sum;
            sh[(size_t)m * (K / 32) + i / 32] = h;
            sl[(size_t)m * (K / 32) + i / 32] = (_Float16)(sum - (float)h);
        }
    }
}

// (scale, min) pair of sub-block j (0..7) from the 12 scale bytes held in
// hdr dwords 1..3 (get_scale_min_k4, q4_k_m.rs:11-22)
__device__ __forceinline__ void scale_min_k4(const uint8_t* q, int j, uint32_t& sc, uint32_t& m) {
    if (j < 4) {
        sc = q[j] & 63;
        m = q[j + 4] & 63;
    } else {
        sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

// The 6-bit scale of sub-block j (0..7) from a block header held in
// registers (dwords 1..3 = the 12 scale bytes), get_scale_min_k4 of
// q4_k_m.rs:11-22 with byte selects by shifts, so j may vary at run time.
__device__ __forceinline__ uint32_t scale_k4(const u32x4& hdr, int j) {
    const int sh = 8 * (j & 3);
    const uint32_t a = (hdr.y >> sh) & 0xFFu;  // q[j & 3]
    const uint32_t c = (hdr.w >> sh) & 0xFFu;  // q[8 + (j & 3)]
    return j < 4 ? (a & 63u) : ((c & 0xFu) | ((a >> 6) << 4));
}

// 8 nibbles (bytes of w0, w1; low or high nibble) times sc, as exact fp16
__device__ __forceinline__ half8 nib8_times(uint32_t w0, uint32_t w1, bool high, _Float16 sc) {
    uint32_t t0 = high ? (w0 >> 4) & 0x0F0F0F0Fu : w0 & 0x0F0F0F0Fu;
    uint32_t t1 = high ? (w1 >> 4) & 0x0F0F0F0Fu : w1 & 0x0F0F0F0Fu;
    // fp16 1024 + q has bit pattern 0x6400 | q: bytes [q, 0x64]
    const uint32_t p0 = __builtin_amdgcn_perm(0x64646464u, t0, 0x07010700u);  // q0, q1
    const uint32_t p1 = __builtin_amdgcn_perm(0x64646464u, t0, 0x07030702u);  // q2, q3
    const uint32_t p2 = __builtin_amdgcn_perm(0x64646464u, t1, 0x07010700u);
    const uint32_t p3 = __builtin_amdgcn_perm(0x64646464u, t1, 0x07030702u);
    const half2v off = {(_Float16)-1024.0f, (_Float16)-1024.0f};
    const half2v s2 = {sc, sc};
    half2v h0 = (__builtin_bit_cast(half2v, p0) + off) * s2;
    half2v h1 = (__builtin_bit_cast(half2v, p1) + off) * s2;
    half2v h2 = (__builtin_bit_cast(half2v, p2) + off) * s2;
    half2v h3 = (__builtin_bit_cast(half2v, p3) + off) * s2;
    return half8{h0.x, h0.y, h1.x, h1.y, h2.x, h2.y, h3.x, h3.y};
}

// The outputs of one lane, 2 x 16 registers: acc[i][r] is row row(i, r),
// column col(i); y (=|+=) acc * rowscale[row]. Every row scale and (with
// accumulate) every old value is loaded before the first store: the stores
// could alias later loads as far as the compiler knows, and each load would
// otherwise wait for the store before it and then for its own memory trip.
template <class RowF, class ColF>
__device__ __forceinline__ void gemm_store(float* __restrict__ Y, int64_t ldy, int M, int N,
                                           const float* __restrict__ rowscale, const f32x16 (&acc)[2], RowF row,
                                           ColF col, int accumulate) {
    float rs[2][16], old[2][16];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int n = col(i);
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int m = row(i, r);
            const bool in = m < M && n < N;
            rs[i][r] = in ? rowscale[m] : 0.f;
            old[i][r] = in && accumulate ? Y[m * ldy + n] : 0.f;
        }
    }
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int n = col(i);
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int m = row(i, r);
            if (m < M && n < N) {
                const float v = acc[i][r] * rs[i][r];
                Y[m * ldy + n] = accumulate ? old[i][r] + v : v;  // one writer per output
            }
        }
    }
}

// grid = (ceil(N / 256), Mp / 64), 512 threads = 8 waves: wave w computes
// input rows 32 (w & 1) .. +32 of the tile against weight rows 64 (w >> 1)
// .. +64 (two 32 x 32 MFMA tiles). Per 64-value k-tile the workgroup stages x
// (fp16 hi and lo, 16 KB, shared by the eight waves) and builds the fp16 B
// operand sc*q once into LDS (two threads per weight row, from qs bytes and
// scales held in registers), so no wave repeats another's conversion. LDS
// holds two k-tiles: while the waves run the products of tile t from one
// buffer they build tile t + 1 in the other, so a k-tile costs one barrier,
// and each tile's bytes are loaded two tiles ahead into one of three
// register stages. 120 KB of LDS: one workgroup (eight waves) per CU.
constexpr int kGT = 512;  // threads of a GEMM workgroup
constexpr int kGN = 256;  // weight rows of its tile

struct GemmStage {
    u32x4 xh, xl;       // x chunk of 8 values: input row tid/8, chunk tid%8
    u32x4 qs, hdr, ps;  // 16 qs bytes of weight row bn; its block header; sub-block sums (tid < 128)
};

struct GemmBuf {
    _Float16 Xh[kTm][kXs];
    _Float16 Xl[kTm][kXs];
    _Float16 Bt[kGN][kXs];  // sc * q of the k-tile, weight-row major
};

__global__ void __launch_bounds__(kGT) gemm_q4k_kernel(const uint8_t* __restrict__ W, int N, int K,
                                                       const _Float16* __restrict__ xh,
                                                       const _Float16* __restrict__ xl,
                                                       const _Float16* __restrict__ sh,
                                                       const _Float16* __restrict__ sl,
                                                       const float* __restrict__ rowscale, float* __restrict__ Y,
                                                       int M, int64_t ldy, int accumulate) {
    __shared__ __attribute__((aligned(16))) GemmBuf buf[2];
    // per super-block (by its parity): d, dmin, scales (rows 20 B apart, so
    // the 32 rows a wave reads fall in distinct banks); sub-block sums of x
    __shared__ __attribute__((aligned(16))) uint8_t Wh[2][kGN][20];
    __shared__ __attribute__((aligned(16))) _Float16 Sh[2][kTm][8];
    __shared__ __attribute__((aligned(16))) _Float16 Sl[2][kTm][8];
    const int n0 = blockIdx.x * kGN, m0 = blockIdx.y * kTm;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave & 1, wn = wave >> 1;
    const int nb = K / 256;
    const size_t rb = (size_t)nb * 144;
    const int li = lane & 31, lh = lane >> 5;
    // B building: weight row bn of the tile, qs bytes [16 bc, 16 bc + 16) of
    // the group; each 16 threads cover 8 rows x 2 halves, eight consecutive
    // lanes on eight rows (their LDS rows 144 B apart hit distinct banks)
    const int bn = 8 * (tid >> 4) + (tid & 7), bc = (tid >> 3) & 1;
    const uint8_t* brow = W + (size_t)(n0 + bn < N ? n0 + bn : N - 1) * rb;
    const int xr = tid >> 3, xc = tid & 7;  // x staging: row xr, values 8 xc .. +8 of the k-tile

    f32x16 acc[2], c1[2];
#pragma unroll
    for (int nt = 0; nt < 2; nt++) {
        acc[nt] = f32x16{};
        c1[nt] = f32x16{};
    }

    const int ntiles = K / kTk;
    auto load_tile = [&](GemmStage& S, int t) {
        const int k0 = t * kTk;
        const size_t o = (size_t)(m0 + xr) * K + k0 + 8 * xc;
        S.xh = *(const u32x4*)(xh + o);
        S.xl = *(const u32x4*)(xl + o);
        const int b = k0 / 256, g = (k0 % 256) / 64;
        S.qs = *(const u32x4*)(brow + (size_t)b * 144 + 16 + 32 * g + 16 * bc);
        if (g == 0) {
            S.hdr = *(const u32x4*)(brow + (size_t)b * 144);
            if (tid < 2 * kTm) {
                const int rr = tid >> 1, half = tid & 1;
                S.ps = half ? *(const u32x4*)(sl + (size_t)(m0 + rr) * (K / 32) + 8 * b)
                            : *(const u32x4*)(sh + (size_t)(m0 + rr) * (K / 32) + 8 * b);
            }
        }
    };
    u32x4 hdr = {};  // this thread's weight row header of the super-block being built
    auto store_tile = [&](const GemmStage& S, int t) {
        GemmBuf& B = buf[t & 1];
        *(u32x4*)&B.Xh[xr][8 * xc] = S.xh;
        *(u32x4*)&B.Xl[xr][8 * xc] = S.xl;
        const int g = t & 3, p = (t >> 2) & 1;
        if (g == 0) {
            hdr = S.hdr;
            if (bc == 0) {
                uint32_t* w = (uint32_t*)&Wh[p][bn][0];
                w[0] = S.hdr.x; w[1] = S.hdr.y; w[2] = S.hdr.z; w[3] = S.hdr.w;
            }
            if (tid < 2 * kTm) {
                if (tid & 1) *(u32x4*)&Sl[p][tid >> 1][0] = S.ps;
                else *(u32x4*)&Sh[p][tid >> 1][0] = S.ps;
            }
        }
        // values 16bc .. 16bc+15 of sub-blocks 2g (low nibbles) and 2g+1 (high)
        const _Float16 s0 = (_Float16)(float)scale_k4(hdr, 2 * g), s1 = (_Float16)(float)scale_k4(hdr, 2 * g + 1);
        *(half8*)&B.Bt[bn][16 * bc] = nib8_times(S.qs.x, S.qs.y, false, s0);
        *(half8*)&B.Bt[bn][16 * bc + 8] = nib8_times(S.qs.z, S.qs.w, false, s0);
        *(half8*)&B.Bt[bn][32 + 16 * bc] = nib8_times(S.qs.x, S.qs.y, true, s1);
        *(half8*)&B.Bt[bn][32 + 16 * bc + 8] = nib8_times(S.qs.z, S.qs.w, true, s1);
    };

    const int ar = 32 * wm + li;  // this lane's A row (input row of the tile)
    auto compute = [&](int t) {
        const GemmBuf& B = buf[t & 1];
#pragma unroll
        for (int s = 0; s < 4; s++) {
            // k-step s: values 16s .. 16s+15 of the group; lane half lh holds 8 of them
            const half8 a_h = *(const half8*)&B.Xh[ar][16 * s + 8 * lh];
            const half8 a_l = *(const half8*)&B.Xl[ar][16 * s + 8 * lh];
            half8 bq[2];
#pragma unroll
            for (int nt = 0; nt < 2; nt++) bq[nt] = *(const half8*)&B.Bt[64 * wn + 32 * nt + li][16 * s + 8 * lh];
#pragma unroll
            for (int nt = 0; nt < 2; nt++) c1[nt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a_h, bq[nt], c1[nt], 0, 0, 0);
#pragma unroll
            for (int nt = 0; nt < 2; nt++) c1[nt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a_l, bq[nt], c1[nt], 0, 0, 0);
        }
        if ((t & 3) == 3) {
            // end of super-block: acc += d * C, then the min term
            // dmin * sum_sub m_sub * X_sub on the same MFMA shape
            const int p = (t >> 2) & 1;
            float d[2], dm[2];
            half8 bm[2];
#pragma unroll
            for (int nt = 0; nt < 2; nt++) {
                const int r = 64 * wn + 32 * nt + li;
                const uint32_t w0 = *(const uint32_t*)&Wh[p][r][0];
                d[nt] = half_bits_to_f32(w0);
                dm[nt] = half_bits_to_f32(w0 >> 16);
                // B[k][n] = m of sub-block k for k < 8, 0 for k = 8..15 (lane half 1)
                half8 v = {};
                if (lh == 0) {
#pragma unroll
                    for (int j = 0; j < 8; j++) {
                        uint32_t sc, mm;
                        scale_min_k4(&Wh[p][r][4], j, sc, mm);
                        v[j] = (_Float16)(float)mm;
                    }
                }
                bm[nt] = v;
            }
#pragma unroll
            for (int nt = 0; nt < 2; nt++) {
                acc[nt] += d[nt] * c1[nt];
                c1[nt] = f32x16{};
            }
            const half8 s_h = lh == 0 ? *(const half8*)&Sh[p][ar][0] : half8{};
            const half8 s_l = lh == 0 ? *(const half8*)&Sl[p][ar][0] : half8{};
#pragma unroll
            for (int nt = 0; nt < 2; nt++) {
                f32x16 c2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(s_h, bm[nt], f32x16{}, 0, 0, 0);
                c2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(s_l, bm[nt], c2, 0, 0, 0);
                acc[nt] -= dm[nt] * c2;
            }
        }
    };
    // three register stages with fixed roles (no dynamic indexing): at step t
    // the stage holding tile t + 1 is built into LDS and tile t + 2 loads
    // into the stage tile t - 1 used
    GemmStage S0, S1, S2;
    load_tile(S0, 0);
    if (1 < ntiles) load_tile(S1, 1);
    store_tile(S0, 0);
    __syncthreads();
    auto step = [&](GemmStage& Snext, GemmStage& Sfar, int t) {
        if (t + 2 < ntiles) load_tile(Sfar, t + 2);
        compute(t);
        if (t + 1 < ntiles) store_tile(Snext, t + 1);  // the other buffer: every wave is past tile t - 1
        __syncthreads();
    };
    for (int t = 0; t < ntiles; t += 3) {
        step(S1, S2, t);
        if (t + 1 < ntiles) step(S2, S0, t + 1);
        if (t + 2 < ntiles) step(S0, S1, t + 2);
    }
    // store: D[i][j] in lane j + 32*((i/4)%2), register 4*(i/8) + i%4
    gemm_store(
        Y, ldy, M, N, rowscale, acc, [&](int, int r) { return m0 + 32 * wm + 8 * (r / 4) + 4 * lh + (r % 4); },
        [&](int nt) { return n0 + 64 * wn + 32 * nt + li; }, accumulate);
}


// ------------------------------------------------ Q4_K B operand converted once
//
// launch_pack_q4k_gemm layout of a rows x cols Q4_K matrix (rows % 32 == 0,
// cols % 256 == 0), read by gemm_q4k_b16_kernel:
//   B section: per 32-row tile nt and 64-value k-tile kt (Q4_K group g = kt %
//   4 of super-block kt / 4: sub-block 2g from the low nibbles of its 32 code
//   bytes, 2g + 1 from the high ones), per k-step s (values 16s .. 16s + 15
//   of the k-tile), the v_mfma_f32_32x32x16_f16 B operand: lane l (row 32 nt +
//   l % 32, values 16 s + 8 (l / 32) .. + 7) holds the 8 fp16 sc * q, exact
//   (<= 945), at byte ((nt * KT + kt) * 4 + s) * 1024 + 16 l (KT = cols / 64);
//   H section (after the rows * cols * 2 bytes of B): per (nt, super-block
//   sb), 640 bytes: the 32 rows' d | dmin << 16 (their header's first dword),
//   then their 8 sub-block mins as fp16 (16 bytes a row).
// The values are those gemm_q4k_kernel builds in LDS for every tile of
// input rows; here they are built once and every k-step's B is one
// contiguous 1 KB load.
constexpr int kGemmHBytes = 640;

__global__ void __launch_bounds__(256) pack_q4k_gemm_kernel(const uint8_t* __restrict__ src,
                                                            uint8_t* __restrict__ dst, int rows, int cols) {
    const int KT = cols / kTk, NB = cols / 256;
    const size_t rb = (size_t)NB * 144;
    const size_t nb16 = (size_t)rows / 32 * KT * 4 * 64;  // 16-byte B entries
    const size_t nh = (size_t)rows / 32 * NB * 32;        // (row, super-block) header entries
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i < nb16) {
        const int l = (int)(i & 63);
        size_t q = i >> 6;
        const int s = (int)(q & 3);
        q >>= 2;
        const int kt = (int)(q % KT);
        const size_t nt = q / KT;
        const int kk0 = 16 * s + 8 * (l >> 5), g = kt % 4;  // values kk0 .. kk0 + 7 of the group
        const uint8_t* blk = src + (32 * nt + (l & 31)) * rb + (size_t)(kt / 4) * 144;
        uint32_t sc, mn;
        scale_min_k4(blk + 4, 2 * g + (kk0 >= 32), sc, mn);
        half8 v;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const uint32_t byte = blk[16 + 32 * g + ((kk0 + e) & 31)];
            v[e] = (_Float16)(float)((kk0 >= 32 ? byte >> 4 : byte & 15u) * sc);
        }
        *(half8*)(dst + i * 16) = v;
    } else if (i < nb16 + nh) {
        const size_t h = i - nb16, q = h >> 5;  // q = nt * NB + sb
        const int r = (int)(h & 31), sb = (int)(q % NB);
        const size_t nt = q / NB;
        const uint8_t* blk = src + (32 * nt + r) * rb + (size_t)sb * 144;
        uint8_t* H = dst + (size_t)rows * cols * 2 + q * kGemmHBytes;
        *(uint32_t*)(H + 4 * r) = *(const uint32_t*)blk;
        half8 mv;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            uint32_t sc, mn;
            scale_min_k4(blk + 4, j, sc, mn);
            mv[j] = (_Float16)(float)mn;
        }
        *(half8*)(H + 128 + 16 * r) = mv;
    }
}

// gemm_q4k_kernel's tiles (64 input rows x 256 weight rows, 512 threads) on
// the converted B: wave w takes weight rows 32 w .. 32 w + 31 of the tile for
// all 64 input rows (two 32 x 32 MFMA tiles), its B operands loaded straight
// into registers (one 1 KB load per k-step), only x (fp16 hi and lo) staged
// in LDS. Four register stages in a ring, k-tile t + 3 loading while t
// computes, unrolled by four so that the tiles that start a super-block
// (and bring its header and sub-block sums) are known at compile time:
// every load is unconditional (the last tiles re-read tile KT - 1), so the
// compiler counts them exactly and waits only for the tile in hand. The
// same MFMA chains in the same order as gemm_q4k_kernel: the same results,
// bit for bit.
struct GemmStageB {
    u32x4 xh, xl, ps;  // x chunk of 8 values (input row tid/8, chunk tid%8); sub-block sums (super-block start)
    u32x4 b[4];        // the wave's B operand of each k-step
};

__global__ void __launch_bounds__(kGT) gemm_q4k_b16_kernel(const uint8_t* __restrict__ Wg, int N, int K,
                                                           const _Float16* __restrict__ xh,
                                                           const _Float16* __restrict__ xl,
                                                           const _Float16* __restrict__ sh,
                                                           const _Float16* __restrict__ sl,
                                                           const float* __restrict__ rowscale,
                                                           float* __restrict__ Y, int M, int64_t ldy, int accumulate) {
    __shared__ __attribute__((aligned(16))) _Float16 Xh[2][kTm][kXs];
    __shared__ __attribute__((aligned(16))) _Float16 Xl[2][kTm][kXs];
    __shared__ __attribute__((aligned(16))) _Float16 Sh[2][kTm][8];
    __shared__ __attribute__((aligned(16))) _Float16 Sl[2][kTm][8];
    const int n0 = blockIdx.x * kGN, m0 = blockIdx.y * kTm;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 31, lh = lane >> 5;
    const int KT = K / kTk, NB = K / 256;  // KT: a multiple of 32 (K % 2048 == 0)
    // this wave's 32-row tile (past N: the last one, loaded and not stored)
    const bool live = n0 + 32 * wave < N;
    const int nt = live ? (n0 >> 5) + wave : N / 32 - 1;
    const uint8_t* Bw = Wg + (size_t)nt * KT * 4096 + 16 * lane;
    const uint8_t* Hw = Wg + (size_t)N * K * 2 + (size_t)nt * NB * kGemmHBytes;
    const int xr = tid >> 3, xc = tid & 7;
    const int pr = (tid >> 1) & (kTm - 1);  // sub-block sums: row pr, hi (even) or lo (odd)
    const _Float16* ps_src = ((tid & 1) ? sl : sh) + (size_t)(m0 + pr) * (K / 32);

    f32x16 acc[2], c1[2];
#pragma unroll
    for (int mt = 0; mt < 2; mt++) {
        acc[mt] = f32x16{};
        c1[mt] = f32x16{};
    }
    uint32_t hd = 0, hd_n = 0;  // the lane's row: d | dmin << 16 of the super-block computing, of the next
    u32x4 hm = {}, hm_n = {};   // their 8 mins (fp16)
    // SB: t starts a super-block (t % 4 == 0): its sub-block sums into the
    // stage, its header into hd_n / hm_n
    auto load = [&](GemmStageB& S, int t, auto SB) {
        t = t < KT ? t : KT - 4 + (t & 3);  // (KT % 4 == 0: keeps t % 4)
        const size_t o = (size_t)(m0 + xr) * K + t * kTk + 8 * xc;
        S.xh = *(const u32x4*)(xh + o);
        S.xl = *(const u32x4*)(xl + o);
#pragma unroll
        for (int s = 0; s < 4; s++) S.b[s] = *(const u32x4*)(Bw + ((size_t)t * 4 + s) * 1024);
        if constexpr (decltype(SB)::value) {
            S.ps = *(const u32x4*)(ps_src + 8 * (t >> 2));
            const uint8_t* h = Hw + (size_t)(t >> 2) * kGemmHBytes;
            hd_n = *(const uint32_t*)(h + 4 * li);
            hm_n = *(const u32x4*)(h + 128 + 16 * li);
        }
    };
    auto store_x = [&](const GemmStageB& S, int t) {
        const int bf = t & 1;
        *(u32x4*)&Xh[bf][xr][8 * xc] = S.xh;
        *(u32x4*)&Xl[bf][xr][8 * xc] = S.xl;
        if ((t & 3) == 0 && tid < 2 * kTm) {
            const int p = (t >> 2) & 1;
            if (tid & 1) *(u32x4*)&Sl[p][pr][0] = S.ps;
            else *(u32x4*)&Sh[p][pr][0] = S.ps;
        }
    };
    auto compute = [&](const GemmStageB& S, int t) {
        const int bf = t & 1;
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const half8 bq = __builtin_bit_cast(half8, S.b[s]);
            half8 a_h[2], a_l[2];
#pragma unroll
            for (int mt = 0; mt < 2; mt++) {
                a_h[mt] = *(const half8*)&Xh[bf][32 * mt + li][16 * s + 8 * lh];
                a_l[mt] = *(const half8*)&Xl[bf][32 * mt + li][16 * s + 8 * lh];
            }
#pragma unroll
            for (int mt = 0; mt < 2; mt++) c1[mt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a_h[mt], bq, c1[mt], 0, 0, 0);
#pragma unroll
            for (int mt = 0; mt < 2; mt++) c1[mt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a_l[mt], bq, c1[mt], 0, 0, 0);
        }
        if ((t & 3) == 3) {
            // end of super-block: acc += d * C, then the min term on the same MFMA shape
            const int p = (t >> 2) & 1;
            const float d = half_bits_to_f32(hd), dm = half_bits_to_f32(hd >> 16);
            const half8 bm = lh == 0 ? __builtin_bit_cast(half8, hm) : half8{};
#pragma unroll
            for (int mt = 0; mt < 2; mt++) {
                acc[mt] += d * c1[mt];
                c1[mt] = f32x16{};
            }
#pragma unroll
            for (int mt = 0; mt < 2; mt++) {
                const half8 s_h = lh == 0 ? *(const half8*)&Sh[p][32 * mt + li][0] : half8{};
                const half8 s_l = lh == 0 ? *(const half8*)&Sl[p][32 * mt + li][0] : half8{};
                f32x16 c2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(s_h, bm, f32x16{}, 0, 0, 0);
                c2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(s_l, bm, c2, 0, 0, 0);
                acc[mt] -= dm * c2;
            }
        }
    };
    GemmStageB S0, S1, S2, S3;
    load(S0, 0, std::true_type{});
    hd = hd_n;
    hm = hm_n;
    load(S1, 1, std::false_type{});
    load(S2, 2, std::false_type{});
    store_x(S0, 0);
    __syncthreads();
    // step t: tile t computes from Sc (its x already in LDS), tile t + 1's x
    // goes into the other LDS buffer from Sn, tile t + 3 loads into Sf (the
    // stage tile t - 1 used); the step that loads a super-block's first tile
    // (t % 4 == 1) brings its header, taken over after the last k-tile of
    // the super-block before it
    auto step = [&](const GemmStageB& Sc, const GemmStageB& Sn, GemmStageB& Sf, int t, auto SB) {
        load(Sf, t + 3, SB);
        compute(Sc, t);
        if ((t & 3) == 3) {
            hd = hd_n;
            hm = hm_n;
        }
        if (t + 1 < KT) store_x(Sn, t + 1);
        __syncthreads();
    };
    for (int t = 0; t < KT; t += 4) {
        step(S0, S1, S3, t, std::false_type{});
        step(S1, S2, S0, t + 1, std::true_type{});
        step(S2, S3, S1, t + 2, std::false_type{});
        step(S3, S0, S2, t + 3, std::false_type{});
    }
    if (!live) return;
    // store: D[i][j] in lane j + 32*((i/4)%2), register 4*(i/8) + i%4
    gemm_store(
        Y, ldy, M, N, rowscale, acc, [&](int mt, int r) { return m0 + 32 * mt + 8 * (r / 4) + 4 * lh + (r % 4); },
        [&](int) { return n0 + 32 * wave + li; }, accumulate);
}


// Q6_K (q6_k.rs:8-43: y = (d * sc) * q, q = code - 32, one int8 scale per
// 16-value sub-block) on the same tiles as gemm_q4k_kernel. The B operand
// is q itself, exact in fp16; sc * q (up to 4096 in magnitude) is not
// always exact in fp16, so the scale is applied per sub-block instead: a
// 32 x 32 x 16 product is exactly one sub-block, so each k-step's chain (x
// hi, then x lo) starts from zero and is folded into the fp32 accumulator as
// acc += (d * sc) * C, the factor per weight row (lane) and sub-block.
// Blocks are 210 bytes (2-byte aligned): the code bytes of a k-tile pair
// (ql low nibbles and qh bits 0-3, then the high nibbles and bits 4-7 of the
// same bytes) are loaded once per pair with ld16_a2.
struct GemmStage6 {
    u32x4 xh, xl;             // x chunk of 8 values: input row tid/8, chunk tid%8
    u32x4 ql0, ql1, qh, scw;  // weight row bn: ql / qh bytes of the k-tile pair; the 16 scales
    uint32_t d;               // and d (first k-tile of a super-block)
};

struct GemmBuf6 {
    _Float16 Xh[kTm][kXs];
    _Float16 Xl[kTm][kXs];
    _Float16 Bq[kGN][kXs];  // q = code - 32 of the k-tile, weight-row major
};

// four 6-bit codes (nibbles of ql at bit 4p, two qh bits at 4p + 2j) as
// fp16 q = code - 32: 1024 + code has the bits 0x6400 | code
__device__ __forceinline__ void q6_codes8(uint32_t l0, uint32_t l1, uint32_t h0, uint32_t h1, int p, int j,
                                          _Float16* dst) {
    const uint32_t sn = 4u * (uint32_t)p, sh = 4u * (uint32_t)p + 2u * (uint32_t)j;
    const uint32_t c0 = ((l0 >> sn) & 0x0F0F0F0Fu) | (((h0 >> sh) & 0x03030303u) << 4);
    const uint32_t c1 = ((l1 >> sn) & 0x0F0F0F0Fu) | (((h1 >> sh) & 0x03030303u) << 4);
    const uint32_t p0 = __builtin_amdgcn_perm(0x64646464u, c0, 0x07010700u);
    const uint32_t p1 = __builtin_amdgcn_perm(0x64646464u, c0, 0x07030702u);
    const uint32_t p2 = __builtin_amdgcn_perm(0x64646464u, c1, 0x07010700u);
    const uint32_t p3 = __builtin_amdgcn_perm(0x64646464u, c1, 0x07030702u);
    const half2v off = {(_Float16)-1056.0f, (_Float16)-1056.0f};
    const half2v h0v = __builtin_bit_cast(half2v, p0) + off, h1v = __builtin_bit_cast(half2v, p1) + off;
    const half2v h2v = __builtin_bit_cast(half2v, p2) + off, h3v = __builtin_bit_cast(half2v, p3) + off;
    *(half8*)dst = half8{h0v.x, h0v.y, h1v.x, h1v.y, h2v.x, h2v.y, h3v.x, h3v.y};
}

__global__ void __launch_bounds__(kGT) gemm_q6k_kernel(const uint8_t* __restrict__ W, int N, int K,
                                                       const _Float16* __restrict__ xh,
                                                       const _Float16* __restrict__ xl,
                                                       const float* __restrict__ rowscale, float* __restrict__ Y,
                                                       int M, int64_t ldy, int accumulate) {
    __shared__ __attribute__((aligned(16))) GemmBuf6 buf[2];
    // per super-block (by its parity): the 16 int8 scales and d of each
    // weight row (rows 20 B apart, so the 32 rows a wave reads fall in
    // distinct banks)
    __shared__ __attribute__((aligned(16))) uint8_t Wh[2][kGN][20];
    const int n0 = blockIdx.x * kGN, m0 = blockIdx.y * kTm;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave & 1, wn = wave >> 1;
    const size_t rb = (size_t)(K / 256) * 210;
    const int li = lane & 31, lh = lane >> 5;
    const int bn = 8 * (tid >> 4) + (tid & 7), bc = (tid >> 3) & 1;
    const uint8_t* brow = W + (size_t)(n0 + bn < N ? n0 + bn : N - 1) * rb;
    const int xr = tid >> 3, xc = tid & 7;

    f32x16 acc[2];
#pragma unroll
    for (int nt = 0; nt < 2; nt++) acc[nt] = f32x16{};

    const int ntiles = K / kTk;
    auto load_tile = [&](GemmStage6& S, int t) {
        const int k0 = t * kTk;
        const size_t o = (size_t)(m0 + xr) * K + k0 + 8 * xc;
        S.xh = *(const u32x4*)(xh + o);
        S.xl = *(const u32x4*)(xl + o);
        const int b = k0 / 256, g = (k0 % 256) / 64, h = g >> 1;
        const uint8_t* blk = brow + (size_t)b * 210;
        // branch-free: both k-tiles of a pair load the pair's bytes, every
        // k-tile the block's scales and d (used at its first k-tile)
        S.ql0 = ld16_a2(blk + 64 * h + 16 * bc);
        S.ql1 = ld16_a2(blk + 64 * h + 32 + 16 * bc);
        S.qh = ld16_a2(blk + 128 + 32 * h + 16 * bc);
        S.scw = ld16_a2(blk + 192);
        S.d = ld_u16(blk + 208);
    };
    auto store_tile = [&](const GemmStage6& S, int t) {
        GemmBuf6& B = buf[t & 1];
        *(u32x4*)&B.Xh[xr][8 * xc] = S.xh;
        *(u32x4*)&B.Xl[xr][8 * xc] = S.xl;
        const int g = t & 3, p = g & 1, sp = (t >> 2) & 1;
        const u32x4 ql0 = S.ql0, ql1 = S.ql1, qh = S.qh;
        if (g == 0 && bc == 0) {
            uint32_t* w = (uint32_t*)&Wh[sp][bn][0];
            w[0] = S.scw.x; w[1] = S.scw.y; w[2] = S.scw.z; w[3] = S.scw.w; w[4] = S.d;
        }
        // values 16 bc .. +15 of the tile's two 32-value quarters (codes of
        // ql0 / ql1 with the qh bit pairs 2p, 2p + 1)
        q6_codes8(ql0.x, ql0.y, qh.x, qh.y, p, 0, &B.Bq[bn][16 * bc]);
        q6_codes8(ql0.z, ql0.w, qh.z, qh.w, p, 0, &B.Bq[bn][16 * bc + 8]);
        q6_codes8(ql1.x, ql1.y, qh.x, qh.y, p, 1, &B.Bq[bn][32 + 16 * bc]);
        q6_codes8(ql1.z, ql1.w, qh.z, qh.w, p, 1, &B.Bq[bn][32 + 16 * bc + 8]);
    };

    const int ar = 32 * wm + li;
    auto compute = [&](int t) {
        const GemmBuf6& B = buf[t & 1];
        const int g = t & 3, sp = (t >> 2) & 1;
        // d * sc of this lane's two weight rows for the tile's four sub-blocks
        float ds[2][4];
#pragma unroll
        for (int nt = 0; nt < 2; nt++) {
            const int r = 64 * wn + 32 * nt + li;
            const uint32_t scs = *(const uint32_t*)&Wh[sp][r][4 * g];
            const float d = half_bits_to_f32(*(const uint32_t*)&Wh[sp][r][16]);
#pragma unroll
            for (int s = 0; s < 4; s++) ds[nt][s] = d * (float)(int)(int8_t)(scs >> (8 * s));
        }
        // k-step s: sub-block 4g + s, its chain (x hi, then x lo) scaled into acc
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const half8 a_h = *(const half8*)&B.Xh[ar][16 * s + 8 * lh];
            const half8 a_l = *(const half8*)&B.Xl[ar][16 * s + 8 * lh];
            half8 bq[2];
#pragma unroll
            for (int nt = 0; nt < 2; nt++) bq[nt] = *(const half8*)&B.Bq[64 * wn + 32 * nt + li][16 * s + 8 * lh];
            f32x16 c[2];
#pragma unroll
            for (int nt = 0; nt < 2; nt++) c[nt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a_h, bq[nt], f32x16{}, 0, 0, 0);
#pragma unroll
            for (int nt = 0; nt < 2; nt++) c[nt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a_l, bq[nt], c[nt], 0, 0, 0);
#pragma unroll
            for (int nt = 0; nt < 2; nt++)
#pragma unroll
                for (int r = 0; r < 16; r++) acc[nt][r] = fmaf(ds[nt][s], c[nt][r], acc[nt][r]);
        }
    };
    // two register stages (gemm_q4k_kernel's three would not fit the
    // registers), each loaded two k-tiles ahead: at step t the stage holding
    // tile t + 1 is built into LDS and then reloaded with tile t + 3
    GemmStage6 S0, S1;
    load_tile(S0, 0);
    if (1 < ntiles) load_tile(S1, 1);
    store_tile(S0, 0);
    if (2 < ntiles) load_tile(S0, 2);
    __syncthreads();
    auto step = [&](GemmStage6& Snext, int t) {  // Snext holds tile t + 1
        compute(t);
        if (t + 1 < ntiles) store_tile(Snext, t + 1);  // the other buffer: every wave is past tile t - 1
        if (t + 3 < ntiles) load_tile(Snext, t + 3);
        __syncthreads();
    };
    for (int t = 0; t < ntiles; t += 2) {
        step(S1, t);
        if (t + 1 < ntiles) step(S0, t + 1);
    }
    gemm_store(
        Y, ldy, M, N, rowscale, acc, [&](int, int r) { return m0 + 32 * wm + 8 * (r / 4) + 4 * lh + (r % 4); },
        [&](int nt) { return n0 + 64 * wn + 32 * nt + li; }, accumulate);
}

}  // namespace

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

// Device workspace of the MFMA path: one grow-only buffer per device, reused
// across calls. Calls on different streams are ordered through an event
// recorded after each use, so they never overwrite each other's activations.
struct GemmWorkspace {
    std::mutex mu;
    void* ptr = nullptr;
    size_t bytes = 0;
    hipEvent_t done = nullptr;
};

static GemmWorkspace& gemm_workspace(int dev) {
    static std::mutex mu;
    static std::vector<GemmWorkspace*> all;
    std::lock_guard<std::mutex> lk(mu);
    if ((size_t)dev >= all.size()) all.resize(dev + 1, nullptr);
    if (!all[dev]) all[dev] = new GemmWorkspace();  // lives until the process ends
    return *all[dev];
}

// Y_s[m * ys + n] (=|+=) sum_k W_s[n, k] * pro(X)[m, k] for the segments s
// of a (Q4_K or Q6_K, K % 2048 == 0): one activation split, one GEMM per
// segment.
static int32_t rows_mfma(int32_t t, int pro, const GemvArgs& a, hipStream_t s) {
    const size_t batch = (size_t)a.ncol;
    if (batch > (size_t)INT32_MAX - kTm) return err_overflow();
    const size_t mp = (batch + kTm - 1) / kTm * kTm, K = (size_t)a.K;
    const size_t bx = mp * K * 2, bs = mp * (K / 32) * 2, bytes = 2 * bx + 2 * bs + mp * 4 + 256;
    int dev = 0;
    MIVI_HIP_CHECK(hipGetDevice(&dev));
    GemmWorkspace& ws = gemm_workspace(dev);
    std::lock_guard<std::mutex> lk(ws.mu);
    if (!ws.done) MIVI_HIP_CHECK(hipEventCreateWithFlags(&ws.done, hipEventDisableTiming));
    else MIVI_HIP_CHECK(hipStreamWaitEvent(s, ws.done, 0));  // the previous user is done with it
    if (ws.bytes < bytes) {
        if (ws.ptr) {
            MIVI_HIP_CHECK(hipEventSynchronize(ws.done));
            MIVI_HIP_CHECK(hipFree(ws.ptr));
            ws.ptr = nullptr;
            ws.bytes = 0;
        }
        MIVI_HIP_CHECK(hipMalloc(&ws.ptr, bytes));
        ws.bytes = bytes;
    }
    uint8_t* p = (uint8_t*)ws.ptr;
    _Float16* xh = (_Float16*)p;
    _Float16* xl = (_Float16*)(p + bx);
    _Float16* sh = (_Float16*)(p + 2 * bx);
    _Float16* sl = (_Float16*)(p + 2 * bx + bs);
    float* rs = (float*)(p + 2 * bx + 2 * bs);
    auto prep = K == 2048 ? gemm_prep_kernel<1> : K == 4096 ? gemm_prep_kernel<2> : K == 8192 ? gemm_prep_kernel<4>
                                                                                             : gemm_prep_kernel<0>;
    hipLaunchKernelGGL(prep, dim3((unsigned)mp), dim3(256), 0, s, a.x, a.x2, a.norm_w, a.eps, pro, a.xs,
                       (int)batch, (int)K, xh, xl, sh, sl, rs);
    for (int i = 0; i < a.nseg; i++) {
        const int rows = a.seg[i].n;
        if (rows == 0) continue;
        dim3 grid((unsigned)((rows + kGN - 1) / kGN), (unsigned)(mp / kTm));
        if (t == MIVI_GGML_Q6_K)
            hipLaunchKernelGGL(gemm_q6k_kernel, grid, dim3(kGT), 0, s, a.seg[i].W, rows, (int)K, xh, xl, rs,
                               a.seg[i].y, (int)batch, a.ys, a.accumulate);
        else if (a.seg[i].wg && rows % 32 == 0)
            hipLaunchKernelGGL(gemm_q4k_b16_kernel, grid, dim3(kGT), 0, s, a.seg[i].wg, rows, (int)K, xh, xl, sh, sl,
                               rs, a.seg[i].y, (int)batch, a.ys, a.accumulate);
        else
            hipLaunchKernelGGL(gemm_q4k_kernel, grid, dim3(kGT), 0, s, a.seg[i].W, rows, (int)K, xh, xl, sh, sl, rs,
                               a.seg[i].y, (int)batch, a.ys, a.accumulate);
    }
    MIVI_HIP_CHECK(hipGetLastError());
    MIVI_HIP_CHECK(hipEventRecord(ws.done, s));
    return MIVI_OK;
}

namespace mivi {
int32_t launch_pack_q4k_gemm(const uint8_t* src, uint8_t* dst, size_t rows, size_t cols, hipStream_t s) {
    if (rows % 32 || cols % 256 || rows > (size_t)INT32_MAX || cols > (size_t)INT32_MAX)
        return set_error(MIVI_ERR_UNSUPPORTED, "no row-product layout for %zu rows of %zu columns", rows, cols);
    const size_t n = rows / 32 * (cols / kTk) * 4 * 64 + rows / 32 * (cols / 256) * 32;
    if (n == 0) return MIVI_OK;
    hipLaunchKernelGGL(pack_q4k_gemm_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, src, dst, (int)rows,
                       (int)cols);
    MIVI_HIP_CHECK(hipGetLastError());
    return MIVI_OK;
}

int32_t launch_rows(int32_t t, int pro, const GemvArgs& a, hipStream_t s) {
    if (pro == PRO_CONV || a.epilogue != EPI_STORE)
        return set_error(MIVI_ERR_UNSUPPORTED, "row products take no conv prologue or fused epilogue");
    // the activation split reads 16-byte vectors of every row
    auto a16 = [](const void* p) { return p == nullptr || (uintptr_t)p % 16 == 0; };
    const bool aligned = a16(a.x) && a16(a.x2) && a16(a.norm_w) && a.xs % 4 == 0;
    if ((t == MIVI_GGML_Q4_K || t == MIVI_GGML_Q6_K) && a.ncol >= kMfmaMinBatch && a.K % 2048 == 0 && aligned)
        return rows_mfma(t, pro, a, s);
    return launch_gemv_ex(t, pro, a, s);
}
}  // namespace mivi

static bool gemm_packable(int32_t t, size_t rows, size_t cols) {
    return t == MIVI_GGML_Q4_K && rows % 32 == 0 && cols % 2048 == 0;
}

extern "C" size_t mivi_hip_gemm_packed_size(int32_t t, size_t rows, size_t cols) {
    return gemm_packable(t, rows, cols) ? mivi::q4k_gemm_packed_bytes(rows, cols) : 0;
}

extern "C" int32_t mivi_hip_pack_weights_gemm(int32_t t, const uint8_t* src, size_t src_len, uint8_t* dst,
                                              size_t dst_len, size_t rows, size_t cols, void* stream) {
    size_t bs, ts, need;
    if (!format_sizes(t, &bs, &ts)) return err_unsupported(t);
    if (cols % bs != 0) return err_misaligned(cols, bs);
    if (!gemm_packable(t, rows, cols))
        return set_error(MIVI_ERR_UNSUPPORTED, "no row-product layout for type %d with %zu rows of %zu columns", t,
                         rows, cols);
    if (__builtin_mul_overflow(rows, (cols / bs) * ts, &need)) return err_overflow();
    if (src_len < need) return err_buffer_too_small(need, src_len);
    const size_t out = mivi::q4k_gemm_packed_bytes(rows, cols);
    if (dst_len < out) return err_buffer_too_small(out, dst_len);
    if (rows && (!src || !dst)) return set_error(MIVI_ERR_INVALID_ARGUMENT, "null buffer");
    if ((uintptr_t)src % 16 || (uintptr_t)dst % 16)
        return set_error(MIVI_ERR_INVALID_ARGUMENT, "weights and packed copy must be 16-byte aligned");
    if (rows && src < dst + out && dst < src + need)
        return set_error(MIVI_ERR_INVALID_ARGUMENT, "packing needs distinct buffers");
    clear_error();
    return mivi::launch_pack_q4k_gemm(src, dst, rows, cols, (hipStream_t)stream);
}

extern "C" int32_t mivi_hip_quantized_matmul_rows_gemm_packed(float* out, size_t out_len, int32_t t,
                                                              const uint8_t* w, size_t w_len, const uint8_t* wg,
                                                              size_t wg_len, const float* in, size_t in_len,
                                                              size_t batch, size_t rows, size_t cols, void* stream) {
    int32_t rc = validate_matmul(t, out_len, w_len, in_len, batch, rows, cols);
    if (rc) return rc;
    if (!gemm_packable(t, rows, cols))
        return set_error(MIVI_ERR_UNSUPPORTED, "no row-product layout for type %d with %zu rows of %zu columns", t,
                         rows, cols);
    const size_t need = mivi::q4k_gemm_packed_bytes(rows, cols);
    if (wg_len < need) return err_buffer_too_small(need, wg_len);
    if (batch == 0 || rows == 0) return clear_error();
    if (!out || !w || !wg || !in) return set_error(MIVI_ERR_INVALID_ARGUMENT, "null buffer");
    if ((uintptr_t)wg % 16) return set_error(MIVI_ERR_INVALID_ARGUMENT, "packed copy must be 16-byte aligned");
    if (rows > (size_t)INT32_MAX || cols > (size_t)INT32_MAX || batch > (size_t)INT32_MAX - kTm) return err_overflow();
    clear_error();
    // batch >= kMfmaMinBatch: the matrix cores on the packed copy; fewer
    // rows: the GEMVs on the GGUF rows
    mivi::GemvArgs a = {};
    a.seg[0] = {w, out, (int)rows, wg};
    a.nseg = 1;
    a.K = (int)cols;
    a.x = in;
    a.ncol = (int)batch;
    a.xs = (int64_t)cols;
    a.ys = (int64_t)rows;
    return mivi::launch_rows(t, mivi::PRO_NONE, a, (hipStream_t)stream);
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
    if (rows > (size_t)INT32_MAX || cols > (size_t)INT32_MAX || batch > (size_t)INT32_MAX - kTm) return err_overflow();
    // Q4_K / Q6_K with batch >= kMfmaMinBatch and cols % 2048 == 0: the matrix cores;
    // otherwise one GEMV over the batch's input rows as columns: the streaming
    // kernel reads each weight row once per two inputs, with every input's
    // result bit-identical to its own matvec (lib.rs:404-457); other shapes
    // run one launch per input row
    mivi::GemvArgs a = {};
    a.seg[0] = {w, out, (int)rows};
    a.nseg = 1;
    a.K = (int)cols;
    a.x = in;
    a.ncol = (int)batch;
    a.xs = (int64_t)cols;
    a.ys = (int64_t)rows;
    return mivi::launch_rows(t, mivi::PRO_NONE, a, s);
}
