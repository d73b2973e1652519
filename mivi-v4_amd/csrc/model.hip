// The mivi-v4 hybrid (ShortConv + GQA) decode step on one MI355X.
//
// Reference: crates/mivi-model/src/{model,ssm,transformer,ffn,loader,gguf}.rs
// and crates/mivi-kv/src/cache.rs. One `mivi_model` owns the packed weights
// (the GGUF tensor-data section copied once to HBM), per-sequence run state,
// the KV caches and the RoPE table. A decode step is a fixed sequence of
// kernel launches that read the token/position of each sequence from device
// memory, so one captured HIP graph replays every greedy step.
//
// Per layer (launches):
//   ShortConv: in_proj GEMV with the RMSNorm fused into its input staging;
//              out_proj GEMV whose staging computes B*X, the causal depthwise
//              conv and the C gate (state ping-pong by a per-sequence phase)
//              and whose output accumulates into the residual.
//   GQA:       q|k|v as one 3-segment GEMV with fused RMSNorm; split-T
//              attention (QK-norm, RoPE, KV store of the current token and
//              online softmax fused); combine; wo GEMV accumulating into x.
//   FFN:       gate|up as one 2-segment GEMV with fused RMSNorm; down GEMV
//              with SwiGLU fused into its staging, accumulating into x.
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <map>
#include <string>
#include <initializer_list>
#include <vector>

#include "common.h"
#include "gemv.h"

namespace mivi {
int32_t launch_dequant(int32_t t, const uint8_t* src, float* out, size_t count, hipStream_t s);
bool ggml_sizes(int32_t t, size_t* bs, size_t* ts);
bool format_sizes(int32_t t, size_t* bs, size_t* ts);
}  // namespace mivi

using namespace mivi;

namespace {

constexpr int kWG = 256;
constexpr int kMaxHd = 128;            // head_dim supported by the attention kernel
constexpr int kMaxAttnSplits = 1024;   // 65536 tokens / 64 tokens per tile
constexpr int kMaxArgmaxParts = 16384; // per-wave argmax partials of the head GEMV
// tokens per attention workgroup (its LDS holds 8192 f32 of K and of V)
inline int attn_tile_tokens(size_t) { return 64; }

// ------------------------------------------------------------------ GGUF

struct GTensor {
    int32_t type = 0;
    std::vector<size_t> dims;
    size_t offset = 0;  // absolute offset in the image
    size_t nbytes = 0;
};

struct GMeta {
    bool is_uint = false, is_float = false, is_u32 = false, is_array = false;
    uint64_t u = 0;
    double f = 0;
    size_t n_strings = 0;       // array: number of string elements
    uint64_t max_positive = 0;  // array: largest positive integer element
};

struct Gguf {
    std::map<std::string, GMeta> meta;
    std::map<std::string, GTensor> tensors;
    size_t data_offset = 0;
};

struct Reader {
    const uint8_t* p;
    size_t n, pos = 0;
    bool bad = false;
    uint64_t u(int bytes) {
        if (pos + (size_t)bytes > n) { bad = true; return 0; }
        uint64_t v = 0;
        for (int i = 0; i < bytes; i++) v |= (uint64_t)p[pos + i] << (8 * i);
        pos += (size_t)bytes;
        return v;
    }
    bool str(std::string* out) {
        uint64_t len = u(8);
        if (bad || len > (1u << 20) || pos + len > n) { bad = true; return false; }
        if (out) out->assign((const char*)p + pos, (size_t)len);
        pos += (size_t)len;
        return true;
    }
};

// gguf.rs:264-310 value types; records the as_usize / as_f32 views
// (gguf.rs:59-84) of scalars and summaries of arrays.
bool read_value(Reader& r, uint32_t type, GMeta* m, bool top) {
    switch (type) {
    case 0: case 1: case 2: case 3: case 4: case 5: case 10: case 11: {
        static const int sz[] = {1, 1, 2, 2, 4, 4, 0, 0, 0, 0, 8, 8};
        int b = sz[type];
        uint64_t v = r.u(b);
        bool sgn = type == 1 || type == 3 || type == 5 || type == 11;
        int64_t sv = sgn ? (int64_t)(v << (64 - 8 * b)) >> (64 - 8 * b) : (int64_t)v;
        if (m && (!sgn || sv >= 0)) {
            uint64_t uv = sgn ? (uint64_t)sv : v;
            if (top) { m->is_uint = true; m->u = uv; m->is_u32 = type == 4; }
            else if (uv > m->max_positive) m->max_positive = uv;
        }
        return !r.bad;
    }
    case 6: {
        uint32_t v = (uint32_t)r.u(4);
        float f;
        memcpy(&f, &v, 4);
        if (m && top) { m->is_float = true; m->f = f; }
        return !r.bad;
    }
    case 12: {
        uint64_t v = r.u(8);
        double f;
        memcpy(&f, &v, 8);
        if (m && top) { m->is_float = true; m->f = (double)(float)f; }
        return !r.bad;
    }
    case 7: r.u(1); return !r.bad;
    case 8:
        if (m && !top) m->n_strings++;
        return r.str(nullptr);
    case 9: {
        uint32_t et = (uint32_t)r.u(4);
        uint64_t len = r.u(8);
        if (r.bad || len > 10000000ull) return false;
        if (m && top) m->is_array = true;
        for (uint64_t i = 0; i < len; i++)
            if (!read_value(r, et, top ? m : nullptr, false)) return false;
        return true;
    }
    default: return false;
    }
}

// gguf.rs:106-253
int32_t parse_gguf(const uint8_t* p, size_t n, Gguf* g) {
    Reader r{p, n};
    if (n < 16) return set_error(MIVI_ERR_GGUF, "GGUF loading error: file too small");
    uint32_t magic = (uint32_t)r.u(4);
    if (magic != 0x46554747u) return set_error(MIVI_ERR_GGUF, "GGUF loading error: invalid magic 0x%X", magic);
    uint32_t ver = (uint32_t)r.u(4);
    if (ver != 2 && ver != 3) return set_error(MIVI_ERR_GGUF, "GGUF loading error: unsupported version %u", ver);
    uint64_t nt = r.u(8), nm = r.u(8);
    if (nt > 50000 || nm > 100000) return set_error(MIVI_ERR_GGUF, "GGUF loading error: counts exceed limits");
    for (uint64_t i = 0; i < nm; i++) {
        std::string key;
        if (!r.str(&key)) break;
        GMeta m;
        uint32_t t = (uint32_t)r.u(4);
        if (!read_value(r, t, &m, true)) { r.bad = true; break; }
        g->meta[key] = m;
    }
    std::vector<std::pair<std::string, GTensor>> infos;
    for (uint64_t i = 0; i < nt && !r.bad; i++) {
        std::string name;
        r.str(&name);
        uint32_t nd = (uint32_t)r.u(4);
        GTensor t;
        for (uint32_t d = 0; d < nd && !r.bad; d++) t.dims.push_back((size_t)r.u(8));
        t.type = (int32_t)r.u(4);
        t.offset = (size_t)r.u(8);
        infos.emplace_back(name, t);
    }
    if (r.bad) return set_error(MIVI_ERR_GGUF, "GGUF loading error: malformed file");
    size_t align = 32;
    auto it = g->meta.find("general.alignment");
    if (it != g->meta.end() && it->second.is_u32 && it->second.u > 0) align = (size_t)it->second.u;
    g->data_offset = (r.pos + align - 1) / align * align;
    for (auto& kv : infos) {
        GTensor t = kv.second;
        size_t bs, ts, ne = 1;
        if (!ggml_sizes(t.type, &bs, &ts))
            return set_error(MIVI_ERR_GGUF, "GGUF loading error: unsupported type %d for tensor '%s'", t.type,
                             kv.first.c_str());
        for (size_t d : t.dims) ne *= d;
        t.offset = g->data_offset + t.offset;
        t.nbytes = (ne + bs - 1) / bs * ts;
        if (t.offset + t.nbytes > n)
            return set_error(MIVI_ERR_GGUF, "GGUF loading error: tensor '%s' exceeds the file", kv.first.c_str());
        g->tensors[kv.first] = t;
    }
    return MIVI_OK;
}

// ------------------------------------------------------------- kernels

struct AttnArgs {
    const float* q;        // [n_heads * hd] raw projections of this sequence
    const float* k;        // [kv_dim]
    const float* v;
    const float* q_norm;   // optional [hd]
    const float* k_norm;
    float eps;
    const float* rope_cos; // [max_seq * hd/2]
    const float* rope_sin;
    uint8_t* kc;           // this sequence's cache for this layer: [max_seq * row_bytes]
    uint8_t* vc;
    size_t row_bytes;
    const int* pos;        // device position of this sequence
    int n_heads, n_kv_heads, hd, nsplit;
    float scale;
    float* part_m;         // [n_heads * nsplit]
    float* part_l;
    float* part_acc;       // [n_heads * nsplit * hd]
    // sequence b of a batched launch (blockIdx.y): q/k/v + b*qkv_s,
    // kc/vc + b*kv_s bytes, pos + b, part_m/part_l + b*part_s,
    // part_acc + b*part_s*hd
    int64_t qkv_s, kv_s, part_s;
    int keep_cache;        // 1: the current token's K/V are already in the cache (not stored again)
    int packed;            // 1: Q8_0 caches in 16-token groups (q8g_* layout below)
};

// Q8_0 caches with head_dim 64 in 16-token groups, the layout the matrix-core
// attention reads with one aligned 16-byte load per lane: group g (tokens
// 16g..16g+15) of kv head h sits at (g * n_kv + h) * 1088 bytes and holds,
// for token t of the group and lane l = t + 16c,
//   bytes 16l..16l+15   K: quants 8c..8c+7 of block 0, then of block 1
//                       V: dims 16c..16c+15
//   bytes 1024 + 4t + 2b  the f16 scale of block b of token t.
// Same bytes as the reference's rows (cache.rs: 68 per kv head and token),
// rearranged; state export/import converts at the boundary.
constexpr int kQ8GroupBytes = 1088;
__host__ __device__ inline size_t q8g_base(size_t pos, int kvh, int n_kv) {
    return ((pos / 16) * (size_t)n_kv + kvh) * kQ8GroupBytes;
}
__host__ __device__ inline int q8g_k_off(int t, int d) {
    const int b = d / 32, i = d % 32;
    return 16 * (t + 16 * (i / 8)) + 8 * b + i % 8;
}
__host__ __device__ inline int q8g_v_off(int t, int d) { return 16 * (t + 16 * (d / 16)) + d % 16; }
__host__ __device__ inline int q8g_d_off(int t, int b) { return 1024 + 4 * t + 2 * b; }

__device__ __forceinline__ float block_sum256(float v, float* red) {
    v = wave_sum(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return red[0] + red[1] + red[2] + red[3];
}

// Embedding row of token tok (model.rs:355-366): bit-exact dequantization of
// one row, generic over the stored format.
// blockIdx.x = b: token tok[b] into x + b * x_stride.
__global__ void __launch_bounds__(kWG) embed_kernel(int32_t type, const uint8_t* table, size_t row_bytes,
                                                    const uint32_t* tok, float* x, int dim, int64_t x_stride) {
    embed_row(type, table, row_bytes, tok[blockIdx.x], x + blockIdx.x * x_stride, dim, threadIdx.x, kWG);
}

// Current token's head vector: optional per-head RMSNorm (transformer.rs:81-96)
// then interleaved-pair RoPE (rope.rs:452-473). One thread per pair.
__device__ __forceinline__ void prep_head(float* dst, const float* src, const float* nw, float eps, int hd,
                                          const float* cs, const float* sn, float* red) {
    // dst/src: hd values; executed by the whole workgroup
    float ss = 0.f;
    if (nw) {
        for (int i = threadIdx.x; i < hd; i += kWG) ss = fmaf(src[i], src[i], ss);
        ss = block_sum256(ss, red);
    }
    const float sc = nw ? 1.0f / sqrtf(ss / (float)hd + eps) : 1.0f;
    for (int i = threadIdx.x; i < hd / 2; i += kWG) {
        float v0 = src[2 * i], v1 = src[2 * i + 1];
        if (nw) {
            v0 = v0 * sc * nw[2 * i];
            v1 = v1 * sc * nw[2 * i + 1];
        }
        float c = cs[i], s = sn[i];
        dst[2 * i] = v0 * c - v1 * s;
        dst[2 * i + 1] = v0 * s + v1 * c;
    }
}

// ------------------------------------------------------------ attention
//
// GQA decode attention in two launches (transformer.rs:112-301):
//  attn_tile_kernel    grid (8 * ceil(nsplit / 8) * n_kv_heads, sequences):
//                      one workgroup per (kv head, split) of a sequence takes
//                      the split's tiles of that kv head for its hpk query
//                      heads and writes (max, sum, unnormalised output) per
//                      query head;
//  attn_combine_kernel grid (n_heads, sequences): merges the splits.
// The softmax is taken per tile and merged exactly (same value as the
// reference's token-by-token online form, different rounding).

typedef __attribute__((address_space(1))) const u32x4 gau32x4;
typedef uint32_t u32x4_a2m __attribute__((ext_vector_type(4), aligned(2)));
typedef __attribute__((address_space(1))) const u32x4_a2m gau32x4_a2;

// Head vector of the current token for this wave: optional per-head RMSNorm
// (transformer.rs:81-96) then interleaved-pair RoPE (rope.rs:452-473). Lane l
// holds the pair (2l, 2l+1); hd <= 128.
__device__ __forceinline__ void wave_prep_head(float* dst, const float* src, const float* nw, float eps, int hd,
                                               const float* cs, const float* sn) {
    const int l = threadIdx.x & 63;
    const bool on = 2 * l < hd;
    float v0 = on ? src[2 * l] : 0.f, v1 = on ? src[2 * l + 1] : 0.f;
    if (nw) {
        const float ss = wave_sum(fmaf(v0, v0, v1 * v1));
        const float sc = 1.0f / sqrtf(ss / (float)hd + eps);
        if (on) {
            v0 = v0 * sc * nw[2 * l];
            v1 = v1 * sc * nw[2 * l + 1];
        }
    }
    if (on) {
        const float c = cs[l], s = sn[l];
        dst[2 * l] = v0 * c - v1 * s;
        dst[2 * l + 1] = v0 * s + v1 * c;
    }
}

// wave_prep_head for heads 0 .. nh-1 (nh <= 4) of src (hd apart) into
// dst[h]: every head's loads issued before any arithmetic, so one wave pays
// one memory latency for all of them
__device__ __forceinline__ void wave_prep_heads4(float (*dst)[64], const float* src, int nh, const float* nw,
                                                 float eps, int hd, const float* cs, const float* sn) {
    const int l = threadIdx.x & 63;
    const bool on = 2 * l < hd;
    float v0[4], v1[4];
#pragma unroll
    for (int h = 0; h < 4; h++) {
        v0[h] = on && h < nh ? src[h * hd + 2 * l] : 0.f;
        v1[h] = on && h < nh ? src[h * hd + 2 * l + 1] : 0.f;
    }
    const float w0 = nw && on ? nw[2 * l] : 1.f, w1 = nw && on ? nw[2 * l + 1] : 1.f;
    const float c = on ? cs[l] : 0.f, s = on ? sn[l] : 0.f;
#pragma unroll
    for (int h = 0; h < 4; h++) {
        if (h >= nh) break;
        float x0 = v0[h], x1 = v1[h];
        if (nw) {
            const float ss = wave_sum(fmaf(x0, x0, x1 * x1));
            const float sc = 1.0f / sqrtf(ss / (float)hd + eps);
            x0 = x0 * sc * w0;
            x1 = x1 * sc * w1;
        }
        if (on) {
            dst[h][2 * l] = x0 * c - x1 * s;
            dst[h][2 * l + 1] = x0 * s + x1 * c;
        }
    }
}

// The current token's K (per-head RMSNorm, RoPE) and V of kv head kvh into
// the cache in its precision (cache.rs:395-461); kcur/vcur keep the values
// as stored, which is what attention reads back (with write false only those
// values are formed, the cache is left alone). One wave.
template <int KVP>
__device__ __forceinline__ void attn_store_current(const AttnArgs& a, int kvh, int pos, const float* cs,
                                                   const float* sn, float* kcur, float* vcur, bool write = true) {
    const int hd = a.hd, lane = threadIdx.x & 63;
    const size_t rb = a.row_bytes;
    wave_prep_head(kcur, a.k + (size_t)kvh * hd, a.k_norm, a.eps, hd, cs, sn);
    for (int i = lane; i < hd; i += 64) vcur[i] = a.v[(size_t)kvh * hd + i];
    __builtin_amdgcn_wave_barrier();
    uint8_t* krow = a.kc + (size_t)pos * rb;
    uint8_t* vrow = a.vc + (size_t)pos * rb;
    if constexpr (KVP == MIVI_KV_F32) {
        for (int i = lane; i < hd && write; i += 64) {
            ((float*)krow)[kvh * hd + i] = kcur[i];
            ((float*)vrow)[kvh * hd + i] = vcur[i];
        }
    } else if constexpr (KVP == MIVI_KV_F16) {
        for (int i = lane; i < hd; i += 64) {
            const uint32_t kb = f32_to_half_bits(kcur[i]), vb = f32_to_half_bits(vcur[i]);
            if (write) {
                ((uint16_t*)krow)[kvh * hd + i] = (uint16_t)kb;
                ((uint16_t*)vrow)[kvh * hd + i] = (uint16_t)vb;
            }
            kcur[i] = half_bits_to_f32(kb);
            vcur[i] = half_bits_to_f32(vb);
        }
    } else {
        // q8_0.rs:31-58 per 32-value block: lanes 0-31 K, 32-63 V
        const int nbk = hd / 32;
        const bool isv = lane >= 32;
        float* cur = isv ? vcur : kcur;
        uint8_t* row = isv ? vrow : krow;
        const int i = lane & 31;
        for (int bi = 0; bi < nbk; bi++) {
            const float xv = cur[bi * 32 + i];
            float am = fabsf(xv);
#pragma unroll
            for (int sh = 16; sh >= 1; sh >>= 1) am = fmaxf(am, __shfl_xor(am, sh, 32));
            const float d = am / 127.0f;
            const float id = d != 0.0f ? 1.0f / d : 0.0f;
            const float q = fminf(fmaxf(roundf(xv * id), -128.0f), 127.0f);
            const uint32_t dh = f32_to_half_bits(d);
            if (write && a.packed) {
                uint8_t* g = (isv ? a.vc : a.kc) + q8g_base((size_t)pos, kvh, a.n_kv_heads);
                const int t = pos & 15, dd = bi * 32 + i;
                g[isv ? q8g_v_off(t, dd) : q8g_k_off(t, dd)] = (uint8_t)(int8_t)q;
                if (i == 0) { g[q8g_d_off(t, bi)] = (uint8_t)dh; g[q8g_d_off(t, bi) + 1] = (uint8_t)(dh >> 8); }
            } else if (write) {
                uint8_t* blk = row + (size_t)(kvh * nbk + bi) * 34;
                blk[2 + i] = (uint8_t)(int8_t)q;
                if (i == 0) { blk[0] = (uint8_t)dh; blk[1] = (uint8_t)(dh >> 8); }
            }
            cur[bi * 32 + i] = q * half_bits_to_f32(dh);
        }
    }
}

// Tiles of TT tokens; split s of nsplit takes tiles [s * tps, s * tps + tps)
// with tps = ceil(ntiles / nsplit), looping over them with an online softmax
// (the tile max and sum merged into running ones) while the next tile's rows
// are already being loaded.
// Workgroup id -> (kv head, split): dispatch deals workgroups to the 8 XCDs
// round robin by id, and each XCD has its own L2. A cache row holds every kv
// head of its token, so the n_kv_heads workgroups of one split are placed on
// the same XCD (id % 8 = split % 8) and each row's lines come from HBM once.
__device__ __forceinline__ bool attn_tile_of(int n_kv, int nsplit, int* kvh, int* split) {
    const int id = blockIdx.x, slot = id >> 3;
    *kvh = slot % n_kv;
    *split = (slot / n_kv) * 8 + (id & 7);
    return *split < nsplit;
}

// Workgroups of one attention launch: 8 * ceil(nsplit / 8) * n_kv per
// sequence (the last ones idle when nsplit is not a multiple of 8).
inline unsigned attn_tile_grid(int n_kv, int nsplit) { return (unsigned)(8 * ((nsplit + 7) / 8) * n_kv); }

template <int KVP, int HDM>  // cache precision; LDS sized for head_dim <= HDM (64 or 128)
__global__ void __launch_bounds__(kWG) attn_tile_kernel(AttnArgs a) {
    constexpr int TT = 64;  // tokens per tile (LDS 36-67 KB: four or two workgroups per CU)
    __shared__ __attribute__((aligned(16))) float kt[TT][HDM + 4];
    __shared__ __attribute__((aligned(16))) float vt[TT][HDM];
    __shared__ __attribute__((aligned(16))) float qs[4][HDM];
    __shared__ __attribute__((aligned(16))) float sc[4][TT];
    __shared__ __attribute__((aligned(16))) float kcur[HDM], vcur[HDM];
    int kvh, split;
    if (!attn_tile_of(a.n_kv_heads, a.nsplit, &kvh, &split)) return;  // workgroup-uniform
    {
        const int b = blockIdx.y;  // sequence of a batched launch
        a.q += b * a.qkv_s; a.k += b * a.qkv_s; a.v += b * a.qkv_s;
        a.kc += b * a.kv_s; a.vc += b * a.kv_s;
        a.pos += b;
        a.part_m += b * a.part_s; a.part_l += b * a.part_s; a.part_acc += b * a.part_s * a.hd;
    }
    const int hd = a.hd, hpk = a.n_heads / a.n_kv_heads;
    const int pos = *a.pos, T = pos + 1;
    const int ntiles = (T + TT - 1) / TT;
    const int tps = (ntiles + a.nsplit - 1) / a.nsplit;
    const int tile0 = split * tps, tile1 = min(ntiles, tile0 + tps);
    if (tile0 >= tile1) return;  // workgroup-uniform: beyond the context
    const bool owner = tile1 == ntiles;  // the last tile holds the current token
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const float* cs = a.rope_cos + (size_t)pos * (hd / 2);
    const float* sn = a.rope_sin + (size_t)pos * (hd / 2);
    const size_t rb = a.row_bytes;

    // tile loads into registers (rows past the tile re-read its row 0 and are dropped)
    constexpr bool Q8 = KVP == MIVI_KV_Q8_0;
    constexpr int E = KVP == MIVI_KV_F32 ? 4 : 8;  // values per 16-byte chunk (f32/f16)
    constexpr int CPT = Q8 ? 2 : TT * HDM / E / kWG;
    u32x4 kr[CPT], vr[CPT];
    uint32_t kd = 0, vd = 0;  // Q8_0 block scales (thread = one 32-value block)
    auto load_tile = [&](int t) {
        const int t0 = t * TT, nt = min(TT, T - t0);
        const uint8_t* kb = a.kc + (size_t)t0 * rb;
        const uint8_t* vb = a.vc + (size_t)t0 * rb;
        if constexpr (Q8) {
            const int bpt = hd / 32;
            const int j = threadIdx.x / bpt, bi = threadIdx.x % bpt;
            const bool ok = j < nt && threadIdx.x < TT * bpt;
            const size_t o = (ok ? (size_t)j * rb : 0) + (size_t)(kvh * bpt + bi) * 34;
            kd = *(const __attribute__((address_space(1))) uint16_t*)(kb + o);
            vd = *(const __attribute__((address_space(1))) uint16_t*)(vb + o);
            kr[0] = *(gau32x4_a2*)(kb + o + 2);
            kr[1] = *(gau32x4_a2*)(kb + o + 18);
            vr[0] = *(gau32x4_a2*)(vb + o + 2);
            vr[1] = *(gau32x4_a2*)(vb + o + 18);
        } else {
            const int cpr = hd / E;
#pragma unroll
            for (int k = 0; k < CPT; k++) {
                const int c = threadIdx.x + k * kWG;
                const int j = c / cpr, part = c % cpr;
                const bool ok = j < nt;
                const size_t o = (ok ? (size_t)j * rb : 0) + (size_t)kvh * hd * (16 / E) + (size_t)(ok ? part : 0) * 16;
                kr[k] = *(gau32x4*)(kb + o);
                vr[k] = *(gau32x4*)(vb + o);
            }
        }
    };
    // registers -> LDS as f32 (the current token from kcur/vcur)
    auto store_tile = [&](int t) {
        const int t0 = t * TT, nt = min(TT, T - t0);
        if constexpr (Q8) {
            const int bpt = hd / 32;
            const int j = threadIdx.x / bpt, bi = threadIdx.x % bpt;
            if (j < nt && threadIdx.x < TT * bpt) {
                const bool cur = t0 + j == pos;
                const float dk = half_bits_to_f32(kd), dv = half_bits_to_f32(vd);
                const uint32_t kw[8] = {kr[0].x, kr[0].y, kr[0].z, kr[0].w, kr[1].x, kr[1].y, kr[1].z, kr[1].w};
                const uint32_t vw[8] = {vr[0].x, vr[0].y, vr[0].z, vr[0].w, vr[1].x, vr[1].y, vr[1].z, vr[1].w};
#pragma unroll
                for (int q = 0; q < 8; q++) {
                    const int d = bi * 32 + 4 * q;
                    f32x4 kk = {sbyte_f32(kw[q], 0) * dk, sbyte_f32(kw[q], 1) * dk, sbyte_f32(kw[q], 2) * dk,
                                sbyte_f32(kw[q], 3) * dk};
                    f32x4 vv = {sbyte_f32(vw[q], 0) * dv, sbyte_f32(vw[q], 1) * dv, sbyte_f32(vw[q], 2) * dv,
                                sbyte_f32(vw[q], 3) * dv};
                    if (cur) {
                        kk = *(const f32x4*)&kcur[d];
                        vv = *(const f32x4*)&vcur[d];
                    }
                    *(f32x4*)&kt[j][d] = kk;
                    *(f32x4*)&vt[j][d] = vv;
                }
            }
        } else {
            const int cpr = hd / E;
#pragma unroll
            for (int k = 0; k < CPT; k++) {
                const int c = threadIdx.x + k * kWG;
                const int j = c / cpr, part = c % cpr;
                if (j >= nt) continue;
                const bool cur = t0 + j == pos;
                const uint32_t kw[4] = {kr[k].x, kr[k].y, kr[k].z, kr[k].w};
                const uint32_t vw[4] = {vr[k].x, vr[k].y, vr[k].z, vr[k].w};
#pragma unroll
                for (int q = 0; q < E / 4; q++) {
                    const int d = part * E + 4 * q;
                    f32x4 kk, vv;
                    if constexpr (KVP == MIVI_KV_F32) {
                        kk = __builtin_bit_cast(f32x4, kr[k]);
                        vv = __builtin_bit_cast(f32x4, vr[k]);
                    } else {
                        kk = {half_bits_to_f32(kw[2 * q]), half_bits_to_f32(kw[2 * q] >> 16),
                              half_bits_to_f32(kw[2 * q + 1]), half_bits_to_f32(kw[2 * q + 1] >> 16)};
                        vv = {half_bits_to_f32(vw[2 * q]), half_bits_to_f32(vw[2 * q] >> 16),
                              half_bits_to_f32(vw[2 * q + 1]), half_bits_to_f32(vw[2 * q + 1] >> 16)};
                    }
                    if (cur) {
                        kk = *(const f32x4*)&kcur[d];
                        vv = *(const f32x4*)&vcur[d];
                    }
                    *(f32x4*)&kt[j][d] = kk;
                    *(f32x4*)&vt[j][d] = vv;
                }
            }
        }
    };

    // 1. the first tile's loads, then 2. query heads (one wave each) and, in
    // the owner split, the current K/V
    load_tile(tile0);
    if (wave < hpk) wave_prep_head(qs[wave], a.q + (size_t)(kvh * hpk + wave) * hd, a.q_norm, a.eps, hd, cs, sn);
    if (owner && wave == 3) attn_store_current<KVP>(a, kvh, pos, cs, sn, kcur, vcur, !a.keep_cache);

    // running softmax state of query head `wave`: lane holds dims lane, lane + 64
    float m_run = -INFINITY, l_run = 0.f, o0 = 0.f, o1 = 0.f;
    for (int t = tile0; t < tile1; t++) {
        const int nt = min(TT, T - t * TT);
        __syncthreads();  // previous tile's LDS reads (and the query prep) are done
        store_tile(t);
        __syncthreads();
        if (t + 1 < tile1) load_tile(t + 1);
        // scores: thread -> (token j, heads hg, hg + 256/TT, ...)
        {
            const int j = threadIdx.x % TT, hg = threadIdx.x / TT;
            for (int h = hg; h < 4; h += kWG / TT) {
                float sv = -INFINITY;
                if (h < hpk && j < nt) {
                    f32x4 d = {0.f, 0.f, 0.f, 0.f};
                    for (int i = 0; i < hd; i += 4) {
                        const f32x4 kk = *(const f32x4*)&kt[j][i];
                        const f32x4 qq = *(const f32x4*)&qs[h][i];
                        d.x = fmaf(qq.x, kk.x, d.x);
                        d.y = fmaf(qq.y, kk.y, d.y);
                        d.z = fmaf(qq.z, kk.z, d.z);
                        d.w = fmaf(qq.w, kk.w, d.w);
                    }
                    sv = ((d.x + d.y) + (d.z + d.w)) * a.scale;
                }
                sc[h][j] = sv;
            }
        }
        __syncthreads();
        if (wave < hpk) {
            float v[TT / 64];
            float mx = -INFINITY;
#pragma unroll
            for (int k = 0; k < TT / 64; k++) {
                v[k] = sc[wave][lane + 64 * k];
                mx = fmaxf(mx, v[k]);
            }
            mx = wave_max(mx);
            const float m_new = fmaxf(m_run, mx);
            const float alpha = m_run == -INFINITY ? 0.f : expf(m_run - m_new);
            float l = 0.f;
#pragma unroll
            for (int k = 0; k < TT / 64; k++) {
                const float p = lane + 64 * k < nt ? expf(v[k] - m_new) : 0.f;
                sc[wave][lane + 64 * k] = p;
                l += p;
            }
            l = wave_sum(l);
            __builtin_amdgcn_wave_barrier();  // sc[wave] is written and read by this wave only
            // whole groups of 4 tokens, then the rest (rows past nt are never
            // read: they may hold anything)
            float a0 = 0.f, a1 = 0.f;
            const int dl = lane < hd ? lane : 0;
            const int dh = lane + 64 < hd ? lane + 64 : 0;
            int j = 0;
            for (; j + 4 <= nt; j += 4) {
                const f32x4 pj = *(const f32x4*)&sc[wave][j];
                a0 = fmaf(pj.x, vt[j][dl], a0);
                a0 = fmaf(pj.y, vt[j + 1][dl], a0);
                a0 = fmaf(pj.z, vt[j + 2][dl], a0);
                a0 = fmaf(pj.w, vt[j + 3][dl], a0);
                if (HDM > 64) {
                    a1 = fmaf(pj.x, vt[j][dh], a1);
                    a1 = fmaf(pj.y, vt[j + 1][dh], a1);
                    a1 = fmaf(pj.z, vt[j + 2][dh], a1);
                    a1 = fmaf(pj.w, vt[j + 3][dh], a1);
                }
            }
            for (; j < nt; j++) {
                const float pj = sc[wave][j];
                a0 = fmaf(pj, vt[j][dl], a0);
                if (HDM > 64) a1 = fmaf(pj, vt[j][dh], a1);
            }
            o0 = o0 * alpha + a0;
            o1 = o1 * alpha + a1;
            l_run = l_run * alpha + l;
            m_run = m_new;
        }
    }
    if (wave < hpk) {
        const int h = kvh * hpk + wave;
        const size_t pi = (size_t)h * a.nsplit + split;
        if (lane == 0) {
            a.part_m[pi] = m_run;
            a.part_l[pi] = l_run;
        }
        if (lane < hd) a.part_acc[pi * hd + lane] = o0;
        if (HDM > 64 && lane + 64 < hd) a.part_acc[pi * hd + lane + 64] = o1;
    }
}

// ------------------------------------------- Q8_0 attention on the matrix cores
//
// Q8_0 caches (q8g_* group layout) with head_dim 64 and at most 4 query heads
// per kv head. One wave per (kv head, split), a workgroup = W kv heads of one
// split (all of them for 8 kv heads, so it reads whole cache rows; placed as
// attn_tile_of places its workgroups). Each wave walks its
// split's 16-token groups (1088 contiguous bytes of K and of V each, one
// 16-byte load per lane) with an online softmax of its own; no workgroup
// barriers.
//  scores  S[h][t] = q_h . k_t on v_mfma_i32_16x16x32_i8, one instruction per
//          32-value block: the query of each head as four int8 digit planes,
//          q = s_h (d0 + d1/254 + d2/254^2) (A rows 4h + p), the
//          cache's int8 K quants as stored (B operand), the block scales and
//          plane weights applied to the int32 sums (lane t + 16h, reg p);
//  values  O[h][d] += p_h(t) dv(t) v(t, d) in f32 on the VALU, lane t + 16c
//          owning token t and dims 16c..16c+15 for all four heads (the p of
//          the other heads' lanes by permlane row swaps).
// The softmax reference point moves only when a group's maximum exceeds it by
// 2^8 (p <= 256); the lane partials are summed over the 16 token lanes at the
// end. Tokens of the last group past the position get p = 0 (their bytes are
// never used).
constexpr int kQ8GroupTokens = 16;

// CTRL a full permutation within rows (quad_perm, row mirrors): every lane
// reads a valid source, and bound_ctrl set lets the compiler fold the move
// into the instruction that consumes it
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    static_assert((CTRL & ~0xFF) == 0 || CTRL == 0x140 || CTRL == 0x141, "quad_perm or row mirror only");
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, true));
}
// sum / max over each row of 16 lanes, result in every lane of the row
__device__ __forceinline__ float row_sum16(float v) {
    v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_f<0x141>(v);  // row_half_mirror
    v += dpp_f<0x140>(v);  // row_mirror
    return v;
}
__device__ __forceinline__ float row_max16(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    v = fmaxf(v, dpp_f<0x141>(v));
    v = fmaxf(v, dpp_f<0x140>(v));
    return v;
}

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_a2m __attribute__((ext_vector_type(2), aligned(2)));
typedef __attribute__((address_space(1))) const u32x2_a2m gau32x2_a2;
typedef __attribute__((address_space(1))) const uint16_t gau16;
typedef __attribute__((address_space(1))) const uint32_t gau32;

struct Q8Group {
    u32x4 k;       // B operands: 8 K quants of block 0 (xy) and of block 1 (zw), token lane & 15
    uint32_t dk;   // its block scales (f16 | f16 << 16)
    u32x4 v;       // V dims 16c..16c+15 of token lane & 15 (c = lane >> 4)
    uint32_t dv;   // their block scale (f16)
};

inline bool attn_q8_mfma_ok(int kv_precision, int hd, int n_heads, int n_kv) {
    return kv_precision == MIVI_KV_Q8_0 && hd == 64 && n_kv > 0 && n_heads % n_kv == 0 && n_heads / n_kv <= 4;
}

// x of the four lanes t, t + 16, t + 32, t + 48 (rows 0..3 at the lane's
// position t) into every lane of that position: one v_permlane16_swap
// (odd rows of one copy with even rows of the other) gives rows {2r, 2r + 1}
// of the lane's half, two v_permlane32_swap (upper half of one copy with the
// lower half of the other) spread each over both halves.
__device__ __forceinline__ void rows_all(float x, float& r0, float& r1, float& r2, float& r3) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    const auto e = __builtin_amdgcn_permlane32_swap(a[0], a[0], false, false);  // a[0]: row 2(c >> 1)
    const auto o = __builtin_amdgcn_permlane32_swap(a[1], a[1], false, false);  // a[1]: row 2(c >> 1) + 1
    r0 = __uint_as_float(e[0]); r2 = __uint_as_float(e[1]);
    r1 = __uint_as_float(o[0]); r3 = __uint_as_float(o[1]);
}

// The end of a matrix-core attention wave: lane t + 16c holds head c's
// running (m, l) and acc[h][i] = dims 16c + i of head h for token lanes t.
// Sums over the 16 token lanes of each row: l by a butterfly; the 64 (head,
// dim) values by a reduce-scatter, each level halving a lane's values while
// the partner (across bit b of t) adds the other half (row mirror, half-row
// mirror, then xor 2 and xor 1 within quads), so lane t ends with values
// 4t .. 4t + 3: head t / 4, dims 16c + 4 (t % 4) .. + 3. Writes the split's
// partials (m in natural-log units for the combine).
__device__ __forceinline__ void attn_write_partials(const AttnArgs& a, float (&acc)[4][16], float m_run,
                                                    float l_run, int kvh, int hpk, int split, int t, int c) {
    constexpr int HD = 64;
    l_run = row_sum16(l_run);
    float v[64];
#pragma unroll
    for (int k = 0; k < 4; k++)
#pragma unroll
        for (int i = 0; i < 16; i++) v[16 * k + i] = acc[k][i];
    auto level = [&](auto mov, int n, bool keep_lo) {
#pragma unroll
        for (int k = 0; k < n; k++) {
            const float lo = v[k], hi = v[k + n];
            v[k] = (keep_lo ? lo : hi) + mov(keep_lo ? hi : lo);
        }
    };
    level([](float x) { return dpp_f<0x140>(x); }, 32, (t & 8) == 0);  // row_mirror: t <-> 15 - t
    level([](float x) { return dpp_f<0x141>(x); }, 16, (t & 4) == 0);  // row_half_mirror: t <-> 7 - t (mod 8)
    level([](float x) { return dpp_f<0x4E>(x); }, 8, (t & 2) == 0);    // quad_perm [2,3,0,1]
    level([](float x) { return dpp_f<0xB1>(x); }, 4, (t & 1) == 0);    // quad_perm [1,0,3,2]
    if ((t >> 2) < hpk) {
        const size_t pi = (size_t)(kvh * hpk + (t >> 2)) * a.nsplit + split;
        *(f32x4*)(a.part_acc + pi * HD + 16 * c + 4 * (t & 3)) = f32x4{v[0], v[1], v[2], v[3]};
    }
    if (t == 0 && c < hpk) {
        const size_t pi = (size_t)(kvh * hpk + c) * a.nsplit + split;
        a.part_m[pi] = m_run * 0.69314718055994531f;
        a.part_l[pi] = l_run;
    }
}

template <int PD, int W>  // groups in flight per wave; waves (kv heads) per workgroup
__global__ void __launch_bounds__(64 * W, 2) attn_q8_mfma_kernel(AttnArgs a) {
    constexpr int HD = 64, G = kQ8GroupTokens;
    __shared__ __attribute__((aligned(16))) float qs[W][4][HD];   // [wave][head][dim]
    __shared__ __attribute__((aligned(16))) float cur[W][2][HD];  // owner: current K/V as stored
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    int kvg, split;
    if (!attn_tile_of((a.n_kv_heads + W - 1) / W, a.nsplit, &kvg, &split)) return;  // workgroup-uniform
    const int kvh = kvg * W + wave;
    if (kvh >= a.n_kv_heads) return;  // wave-uniform (no workgroup barrier below)
    {
        const int b = blockIdx.y;
        a.q += b * a.qkv_s; a.k += b * a.qkv_s; a.v += b * a.qkv_s;
        a.kc += b * a.kv_s; a.vc += b * a.kv_s;
        a.pos += b;
        a.part_m += b * a.part_s; a.part_l += b * a.part_s; a.part_acc += b * a.part_s * HD;
    }
    const int hpk = a.n_heads / a.n_kv_heads;
    const int pos = *a.pos;
    const int ng = (pos + G) / G;
    const int gps = (ng + a.nsplit - 1) / a.nsplit;
    const int g0 = split * gps, g1 = min(ng, g0 + gps);
    if (g0 >= g1) return;  // beyond the context
    const float* cs = a.rope_cos + (size_t)pos * (HD / 2);
    const float* sn = a.rope_sin + (size_t)pos * (HD / 2);

    // 1. the split holding the current token stores its K/V first (then reads
    //    it back like any cached token). Only this wave reads that row in this
    //    launch (the token's group lies in no other split, and later launches
    //    see it across the kernel boundary), so the store needs workgroup
    //    scope: an agent-scope fence would write back and invalidate the
    //    XCD's whole L2 under every other workgroup there (4 us a launch)
    if (g1 == ng && !a.keep_cache) {
        attn_store_current<MIVI_KV_Q8_0>(a, kvh, pos, cs, sn, cur[wave][0], cur[wave][1], true);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    }

    // 2. group loads, q8g_* layout: a wave-uniform group address plus fixed
    //    lane offsets (branch free: past the split's end the last group is re-read)
    const int t = lane & 15, c = lane >> 4;
    const size_t gstride = (size_t)a.n_kv_heads * kQ8GroupBytes;
    const uint8_t* kc = a.kc + (size_t)kvh * kQ8GroupBytes;
    const uint8_t* vc = a.vc + (size_t)kvh * kQ8GroupBytes;
    const int o_kv = 16 * lane, o_dk = q8g_d_off(t, 0), o_dv = q8g_d_off(t, c >> 1);
    auto load = [&](Q8Group& q, int g) {
        g = min(g, g1 - 1);
        const uint8_t* kg = kc + (size_t)g * gstride;
        const uint8_t* vg = vc + (size_t)g * gstride;
        // streamed once per step: non-temporal loads
        q.k = __builtin_nontemporal_load((gau32x4*)(kg + o_kv));
        q.dk = __builtin_nontemporal_load((gau32*)(kg + o_dk));
        q.v = __builtin_nontemporal_load((gau32x4*)(vg + o_kv));
        q.dv = __builtin_nontemporal_load((gau16*)(vg + o_dv));
    };
    Q8Group ring[PD];
#pragma unroll
    for (int i = 0; i < PD; i++) load(ring[i], g0 + i);

    // 3. query heads (QK-norm, RoPE) and their digit planes: A row 4h + p
    //    (p < 3; row 4h + 3 zero), lane = row + 16 * (k / 8)
    for (int h = 0; h < hpk; h++)
        wave_prep_head(qs[wave][h], a.q + (size_t)(kvh * hpk + h) * HD, a.q_norm, a.eps, HD, cs, sn);
    __builtin_amdgcn_wave_barrier();
    float amax[4];
#pragma unroll
    for (int h = 0; h < 4; h++) amax[h] = h < hpk ? wave_max(fabsf(qs[wave][h][lane])) : 0.f;
    long qa[2];
    {
        const int qh = t >> 2, qp = t & 3;
        const float am = qh == 0 ? amax[0] : qh == 1 ? amax[1] : qh == 2 ? amax[2] : amax[3];
        const float inv = am > 0.f ? 127.0f / am : 0.f;
#pragma unroll
        for (int b = 0; b < 2; b++) {
            uint32_t w[2] = {0u, 0u};
#pragma unroll
            for (int e = 0; e < 8; e++) {
                float y = qh < hpk && qp < 3 ? qs[wave][qh][32 * b + 8 * c + e] * inv : 0.f;
                float dg = rintf(y);
                for (int k = 0; k < qp; k++) {
                    y = (y - dg) * 254.0f;  // exact: |y - dg| <= 1/2
                    dg = rintf(y);
                }
                w[e >> 2] |= ((uint32_t)(int)dg & 0xFFu) << (8 * (e & 3));
            }
            qa[b] = (long)(((uint64_t)w[1] << 32) | w[0]);
        }
    }
    // score of lane (t, h = c) in log2 units: scale * s_h * log2(e) / 254 * sum
    const float am_c = c == 0 ? amax[0] : c == 1 ? amax[1] : c == 2 ? amax[2] : amax[3];
    const float qscale = a.scale * (am_c / 127.0f) * (1.4426950408889634f / 254.0f);

    float m_run = -INFINITY, l_run = 0.f;  // head c (lane t + 16c)
    float acc[4][16];                      // head h, dim 16c + i (lane t + 16c)
#pragma unroll
    for (int k = 0; k < 4; k++)
#pragma unroll
        for (int i = 0; i < 16; i++) acc[k][i] = 0.f;

    auto scores = [&](const Q8Group& q, i32x4* s) {
        const i32x4 z = {0, 0, 0, 0};
        const long kb0 = (long)(((uint64_t)q.k.y << 32) | q.k.x), kb1 = (long)(((uint64_t)q.k.w << 32) | q.k.z);
        s[0] = __builtin_amdgcn_mfma_i32_16x16x32_i8(qa[0], kb0, z, 0, 0, 0);
        s[1] = __builtin_amdgcn_mfma_i32_16x16x32_i8(qa[1], kb1, z, 0, 0, 0);
    };
    auto step = [&](const Q8Group& q, const i32x4* sa, int g) {
        // 254 * (d0 + d1/254 + d2/254^2) sums per block: (254 a0 + a1) + a2/254
        const float u0 = fmaf((float)sa[0].z, 1.0f / 254.0f, (float)(254 * sa[0].x + sa[0].y));
        const float u1 = fmaf((float)sa[1].z, 1.0f / 254.0f, (float)(254 * sa[1].x + sa[1].y));
        const bool valid = g * G + t <= pos;  // bytes of tokens past the position may hold anything
        float s = fmaf(half_bits_to_f32(q.dk >> 16), u1, half_bits_to_f32(q.dk) * u0) * qscale;
        s = valid ? s : -INFINITY;
        if (__builtin_amdgcn_ballot_w64(s > m_run + 8.0f)) {  // wave-uniform, rare after the first group
            const float m_new = fmaxf(m_run, row_max16(s));
            const float al = __builtin_amdgcn_exp2f(m_run - m_new);  // 0 while m_run is -inf
            m_run = m_new;
            l_run *= al;
            float a0, a1, a2, a3;
            rows_all(al, a0, a1, a2, a3);
#pragma unroll
            for (int i = 0; i < 16; i++) {
                acc[0][i] *= a0; acc[1][i] *= a1; acc[2][i] *= a2; acc[3][i] *= a3;
            }
        }
        const float p = __builtin_amdgcn_exp2f(s - m_run);  // v_exp_f32 (p <= 256)
        l_run += p;
        float p0, p1, p2, p3;  // p of token t for heads 0..3
        rows_all(p, p0, p1, p2, p3);
        const float dv = valid ? half_bits_to_f32(q.dv) : 0.f;
        const float w0 = p0 * dv, w1 = p1 * dv, w2 = p2 * dv, w3 = p3 * dv;
        const uint32_t vw[4] = {q.v.x, q.v.y, q.v.z, q.v.w};
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const float vf = sbyte_f32(vw[i >> 2], i & 3);
            acc[0][i] = fmaf(w0, vf, acc[0][i]);
            acc[1][i] = fmaf(w1, vf, acc[1][i]);
            acc[2][i] = fmaf(w2, vf, acc[2][i]);
            acc[3][i] = fmaf(w3, vf, acc[3][i]);
        }
    };

    // the score products of a group are issued one group ahead
    i32x4 sa[2];
    scores(ring[0], sa);
    for (int base = g0; base < g1; base += PD) {
#pragma unroll
        for (int i = 0; i < PD; i++) {
            if (base + i < g1) {  // wave-uniform
                const i32x4 cur_s[2] = {sa[0], sa[1]};
                scores(ring[(i + 1) % PD], sa);
                step(ring[i], cur_s, base + i);
            }
            // (unconditional, past the split's end a re-read of its last
            // group: a branch here makes the compiler wait for every load)
            load(ring[i], base + i + PD);
        }
    }

    // 4. the split's partials
    attn_write_partials(a, acc, m_run, l_run, kvh, hpk, split, t, c);
}

// The query heads of one wave, loaded before anything else the wave reads
// (lane l < 32 holds dims 2l, 2l + 1 of each head, with the per-head norm
// weights and the RoPE row), then normalised and rotated into dst[h]
// (transformer.rs:81-96, rope.rs:452-473), as wave_prep_heads4.
struct QHeads {
    float v0[4], v1[4], w0, w1, c, s;
    __device__ __forceinline__ void load(const float* src, int nh, const float* nw, const float* cs, const float* sn) {
        const int l = threadIdx.x & 63;
        const bool on = l < 32;
#pragma unroll
        for (int h = 0; h < 4; h++) {
            v0[h] = on && h < nh ? src[h * 64 + 2 * l] : 0.f;
            v1[h] = on && h < nh ? src[h * 64 + 2 * l + 1] : 0.f;
        }
        w0 = nw && on ? nw[2 * l] : 1.f;
        w1 = nw && on ? nw[2 * l + 1] : 1.f;
        c = on ? cs[l] : 0.f;
        s = on ? sn[l] : 0.f;
    }
    __device__ __forceinline__ void finish(float (*dst)[64], int nh, bool norm, float eps) const {
        const int l = threadIdx.x & 63;
#pragma unroll
        for (int h = 0; h < 4; h++) {
            if (h >= nh) break;
            float x0 = v0[h], x1 = v1[h];
            if (norm) {
                const float ss = wave_sum(fmaf(x0, x0, x1 * x1));
                const float sc = 1.0f / sqrtf(ss / 64.0f + eps);
                x0 = x0 * sc * w0;
                x1 = x1 * sc * w1;
            }
            if (l < 32) {
                dst[h][2 * l] = x0 * c - x1 * s;
                dst[h][2 * l + 1] = x0 * s + x1 * c;
            }
        }
    }
};

// ------------------------------------------- fp16 attention on the matrix cores
//
// fp16 caches (token rows of n_kv_heads x 64 halves, the tile kernel's
// layout) with head_dim 64 and at most 4 query heads per kv head. One wave
// (workgroup) per (kv head, split) of a sequence: the split holds groups
// [split * tps, ...) of 16 tokens, tps = ceil(groups / nsplit) (the rule the
// split merge reads back), walked with an online softmax. Lane t + 16c loads
// dims 16c..16c+15 of token t of a group (32 bytes of K, 32 of V; rows past
// the position read the position's row, so the last group never reads past
// it).
//  scores  v_mfma_f32_16x16x16_f16, four per group: A row 4h + i holds the
//          query of head h in log2 units (scale * log2 e folded in) as an
//          fp16 hi part (i = 0) and lo part (i = 1; q = hi + lo to about
//          2^-22), rows 4h + 2, 4h + 3 zero; B the cache's fp16 K as
//          stored. Instruction j takes dims 16c + 4j .. +3 from k-lane
//          group c (any order of k serves while A and B agree), so lane
//          t + 16h receives head h's hi and lo sums for token t: products
//          of fp16 values are exact, summed in f32;
//  values  v_mfma_f32_16x16x16_f16, four per group (dims 16j .. 16j + 15):
//          A row 4h + i is head h's p at the group's tokens as fp16 hi
//          (i = 0) and lo (i = 1) parts, B the V values as stored, both
//          passed through a per-wave LDS tile; the accumulators hold the
//          token sums across the split (lane n + 16h: dim 16j + n of head h).
// The wave loads its query heads (and the owner, the split holding the
// current token, its K and V) before its cache groups, so those small loads
// wait for no group. The owner stores the current K/V after issuing its
// group loads and patches its token's lanes with them as stored (nothing is
// read back). Tokens of the last group past the position get p = 0.
struct F16Group {
    u32x4 k0, k1;  // K dims 16c .. 16c+15 of token lane & 15 (fp16 pairs)
    u32x4 v0, v1;  // V, the same
};
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));

inline bool attn_f16_mfma_ok(int kv_precision, int hd, int n_heads, int n_kv) {
    return kv_precision == MIVI_KV_F16 && hd == 64 && n_kv > 0 && n_heads % n_kv == 0 && n_heads / n_kv <= 4;
}

template <int PD>  // groups in flight
__global__ void __launch_bounds__(64, 2) attn_f16_mfma_kernel(AttnArgs a) {
    constexpr int HD = 64, G = kQ8GroupTokens;
    __shared__ __attribute__((aligned(16))) float qs[4][HD];       // [head][dim]
    __shared__ __attribute__((aligned(16))) uint32_t curw[2][32];  // owner: current K/V as stored (fp16 pairs)
    // a group's p [head][token] and V [token][dim] (rows of 68 halves: the
    // operand reads of four rows 4 apart fall in four bank ranges)
    constexpr int VROW = 68;
    __shared__ __attribute__((aligned(16))) float pt[4][G];
    __shared__ __attribute__((aligned(16))) _Float16 vt[G][VROW];
    const int lane = threadIdx.x & 63;
    int kvh, split;
    if (!attn_tile_of(a.n_kv_heads, a.nsplit, &kvh, &split)) return;  // workgroup-uniform
    {
        const int b = blockIdx.y;
        a.q += b * a.qkv_s; a.k += b * a.qkv_s; a.v += b * a.qkv_s;
        a.kc += b * a.kv_s; a.vc += b * a.kv_s;
        a.pos += b;
        a.part_m += b * a.part_s; a.part_l += b * a.part_s; a.part_acc += b * a.part_s * HD;
    }
    const int hpk = a.n_heads / a.n_kv_heads;
    const int pos = *a.pos;
    const int ng = (pos + G) / G;
    const int tps = (ng + a.nsplit - 1) / a.nsplit;
    const int g0 = split * tps, g1 = min(ng, g0 + tps);
    if (g0 >= g1) return;  // the split is beyond the context
    const float* cs = a.rope_cos + (size_t)pos * (HD / 2);
    const float* sn = a.rope_sin + (size_t)pos * (HD / 2);
    const int t = lane & 15, c = lane >> 4;
    const bool own = g1 == ng && !a.keep_cache;  // the split holding the current token

    // 1. the small loads: query heads (+ norm weights, RoPE row); the owner's
    //    current K (pair 2l, 2l + 1 in lane l < 32, its norm weights) and V
    QHeads qh;
    qh.load(a.q + (size_t)(kvh * hpk) * HD, hpk, a.q_norm, cs, sn);
    float k0 = 0.f, k1 = 0.f, kn0 = 1.f, kn1 = 1.f, vv0 = 0.f, vv1 = 0.f;
    if (own && lane < 32) {
        const float* kp = a.k + (size_t)kvh * HD + 2 * lane;
        const float* vp = a.v + (size_t)kvh * HD + 2 * lane;
        k0 = kp[0]; k1 = kp[1]; vv0 = vp[0]; vv1 = vp[1];
        if (a.k_norm) { kn0 = a.k_norm[2 * lane]; kn1 = a.k_norm[2 * lane + 1]; }
    }

    // 2. the first PD groups (the current token's lanes read the cache's old
    //    bytes there and are patched below)
    const size_t rb = a.row_bytes;
    const uint8_t* kc = a.kc + (size_t)kvh * (HD * 2) + 32 * c;
    const uint8_t* vc = a.vc + (size_t)kvh * (HD * 2) + 32 * c;
    u32x4 ck0 = {}, ck1 = {}, cv0 = {}, cv1 = {};  // the owner's current K/V as stored (dims 16c .. +15)
    auto load = [&](F16Group& q, int g) {
        g = min(g, g1 - 1);
        const int row = g * G + t;
        if (own && row >= pos) {
            q.k0 = ck0; q.k1 = ck1; q.v0 = cv0; q.v1 = cv1;
        } else {
            const size_t o = (size_t)min(row, pos) * rb;  // streamed once per step: non-temporal
            q.k0 = __builtin_nontemporal_load((gau32x4*)(kc + o));
            q.k1 = __builtin_nontemporal_load((gau32x4*)(kc + o + 16));
            q.v0 = __builtin_nontemporal_load((gau32x4*)(vc + o));
            q.v1 = __builtin_nontemporal_load((gau32x4*)(vc + o + 16));
        }
    };
    F16Group ring[PD];
#pragma unroll
    for (int i = 0; i < PD; i++) {
        const int g = min(g0 + i, g1 - 1);
        const size_t o = (size_t)min(g * G + t, pos) * rb;
        ring[i].k0 = __builtin_nontemporal_load((gau32x4*)(kc + o));
        ring[i].k1 = __builtin_nontemporal_load((gau32x4*)(kc + o + 16));
        ring[i].v0 = __builtin_nontemporal_load((gau32x4*)(vc + o));
        ring[i].v1 = __builtin_nontemporal_load((gau32x4*)(vc + o + 16));
    }

    // 3. the owner forms its K (per-head RMSNorm, RoPE; transformer.rs:81-96,
    //    rope.rs:452-473) and V as fp16, stores them into the cache row
    //    (cache.rs:395-461) and patches its token's lanes
    if (own) {
        if (a.k_norm) {
            const float ss = wave_sum(lane < 32 ? fmaf(k0, k0, k1 * k1) : 0.f);
            const float sc = 1.0f / sqrtf(ss / (float)HD + a.eps);
            k0 = k0 * sc * kn0;
            k1 = k1 * sc * kn1;
        }
        if (lane < 32) {
            const float cc = cs[lane], ss = sn[lane];
            const float r0 = k0 * cc - k1 * ss, r1 = k0 * ss + k1 * cc;
            const uint32_t kw = f32_to_half_bits(r0) | (f32_to_half_bits(r1) << 16);
            const uint32_t vw = f32_to_half_bits(vv0) | (f32_to_half_bits(vv1) << 16);
            ((uint32_t*)(a.kc + (size_t)pos * rb))[kvh * (HD / 2) + lane] = kw;
            ((uint32_t*)(a.vc + (size_t)pos * rb))[kvh * (HD / 2) + lane] = vw;
            curw[0][lane] = kw;
            curw[1][lane] = vw;
        }
        __builtin_amdgcn_wave_barrier();
        ck0 = *(const u32x4*)&curw[0][8 * c]; ck1 = *(const u32x4*)&curw[0][8 * c + 4];
        cv0 = *(const u32x4*)&curw[1][8 * c]; cv1 = *(const u32x4*)&curw[1][8 * c + 4];
#pragma unroll
        for (int i = 0; i < PD; i++) {
            if (min(g0 + i, g1 - 1) * G + t >= pos) {
                ring[i].k0 = ck0; ring[i].k1 = ck1; ring[i].v0 = cv0; ring[i].v1 = cv1;
            }
        }
    }

    // 4. query heads in log2 units as fp16 hi / lo: A row 4h + i, lane =
    //    row + 16 * kg holds dims 16 kg + 4j .. +3 for instruction j
    qh.finish(qs, hpk, a.q_norm != nullptr, a.eps);
    __builtin_amdgcn_wave_barrier();
    half4_t qa[4];
    {
        const int qhd = t >> 2, qi = t & 3;
        const float qscale = a.scale * 1.4426950408889634f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float y = qhd < hpk && qi < 2 ? qs[qhd][16 * c + 4 * j + e] * qscale : 0.f;
                const _Float16 hi = (_Float16)y;
                const _Float16 lo = (_Float16)(y - (float)hi);
                qa[j][e] = qi == 0 ? hi : qi == 1 ? lo : (_Float16)0.0f;
            }
        }
    }

    float m_run = -INFINITY, l_run = 0.f;  // head c (lane t + 16c)
    // P.V on v_mfma_f32_16x16x16_f16, K = the group's 16 tokens: A row 4h + i
    // is head h's p as fp16 hi (i = 0) and lo (i = 1) parts (rows 4h + 2,
    // 4h + 3 zero), B the V values as stored (dims 16j .. 16j + 15 for
    // instruction j), so lane n + 16h accumulates head h's hi and lo sums
    // for dim 16j + n in pv[j][0], pv[j][1], over every group of the split
    f32x4 pv[4];
#pragma unroll
    for (int j = 0; j < 4; j++) pv[j] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int am = lane & 15, akg = lane >> 4;  // operand lane: row / column, k group

    auto scores = [&](const F16Group& q) {
        const uint32_t kw[8] = {q.k0.x, q.k0.y, q.k0.z, q.k0.w, q.k1.x, q.k1.y, q.k1.z, q.k1.w};
        f32x4 s4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint64_t kb = ((uint64_t)kw[2 * j + 1] << 32) | kw[2 * j];
            s4 = __builtin_amdgcn_mfma_f32_16x16x16f16(qa[j], __builtin_bit_cast(half4_t, kb), s4, 0, 0, 0);
        }
        return s4.x + s4.y;  // head c, token t: hi part + lo part
    };
    auto step = [&](const F16Group& q, float s, int g) {
        const bool valid = g * G + t <= pos;
        s = valid ? s : -INFINITY;
        if (__builtin_amdgcn_ballot_w64(s > m_run + 8.0f)) {  // wave-uniform, rare after the first group
            const float m_new = fmaxf(m_run, row_max16(s));
            const float al = __builtin_amdgcn_exp2f(m_run - m_new);  // 0 while m_run is -inf
            m_run = m_new;
            l_run *= al;
            // (the accumulator lanes n + 16c hold head c: the lane's own al)
#pragma unroll
            for (int j = 0; j < 4; j++) pv[j] *= al;
        }
        const float p = __builtin_amdgcn_exp2f(s - m_run);  // v_exp_f32 (p <= 256)
        l_run += p;
        // p and V to LDS, read back in operand order
        pt[c][t] = p;
        uint2* vrow = (uint2*)&vt[t][16 * c];
        vrow[0] = uint2{q.v0.x, q.v0.y}; vrow[1] = uint2{q.v0.z, q.v0.w};
        vrow[2] = uint2{q.v1.x, q.v1.y}; vrow[3] = uint2{q.v1.z, q.v1.w};
        __builtin_amdgcn_wave_barrier();
        const f32x4 p4 = *(const f32x4*)&pt[am >> 2][4 * akg];
        const int ai = am & 3;
        half4_t A;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const _Float16 hi = (_Float16)p4[r];
            const _Float16 lo = (_Float16)(p4[r] - (float)hi);  // exact: p = hi + lo to about 2^-22
            A[r] = ai == 0 ? hi : ai == 1 ? lo : (_Float16)0.0f;
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            // ds_read_b64_tr_b16: in each 16-lane group, lane 4r + q gives the
            // address of 4 halves and lane i receives half i % 4 of the
            // segments of lanes 4r + i / 4, r = 0..3 (checked on the GPU). Lane
            // 16 kg + 4r + q addresses token 4 kg + r, dims 16j + 4q .. + 3, so
            // lane n + 16 kg receives dim 16j + n of tokens 4 kg .. 4 kg + 3
            typedef short s16x4 __attribute__((ext_vector_type(4)));
            const s16x4 raw = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) s16x4*)&vt[4 * akg + (am >> 2)][16 * j + 4 * (am & 3)]);
            pv[j] = __builtin_amdgcn_mfma_f32_16x16x16f16(A, __builtin_bit_cast(half4_t, raw), pv[j], 0, 0, 0);
        }
        __builtin_amdgcn_wave_barrier();  // (the next group's writes after these reads)
    };

    // the score products of a group are issued one group ahead
    float sa = scores(ring[0]);
    for (int base = g0; base < g1; base += PD) {
#pragma unroll
        for (int i = 0; i < PD; i++) {
            if (base + i < g1) {  // wave-uniform
                const float cur_s = sa;
                sa = scores(ring[(i + 1) % PD]);
                step(ring[i], cur_s, base + i);
            }
            // only groups of the split (no re-reads past its end: the wave
            // would wait for them before it ends)
            if (base + i + PD < g1) load(ring[i], base + i + PD);
        }
    }

    // 5. the split's partials: lane n + 16h holds head h's dims 16j + n
    //    (hi + lo rows); l summed over the token lanes
    l_run = row_sum16(l_run);
    if (c < hpk) {
        const size_t pi = (size_t)(kvh * hpk + c) * a.nsplit + split;
#pragma unroll
        for (int j = 0; j < 4; j++) a.part_acc[pi * HD + 16 * j + t] = pv[j][0] + pv[j][1];
        if (t == 0) {
            a.part_m[pi] = m_run * 0.69314718055994531f;
            a.part_l[pi] = l_run;
        }
    }
}

// Prefill tile: K/V of tile row blockIdx.x (position pos0 + row, k/v at
// a.k/a.v + row * qkv_s) for kv head blockIdx.y into the cache, as the decode
// step stores its current token. One wave per (row, kv head).
template <int KVP>
__global__ void __launch_bounds__(64) kv_store_rows_kernel(AttnArgs a, int pos0) {
    __shared__ __attribute__((aligned(16))) float kcur[kMaxHd], vcur[kMaxHd];
    const int r = blockIdx.x, kvh = blockIdx.y, pos = pos0 + r;
    a.k += r * a.qkv_s;
    a.v += r * a.qkv_s;
    const float* cs = a.rope_cos + (size_t)pos * (a.hd / 2);
    const float* sn = a.rope_sin + (size_t)pos * (a.hd / 2);
    attn_store_current<KVP>(a, kvh, pos, cs, sn, kcur, vcur, true);
}

// Prefill tile ShortConv (ssm.rs:174-300, kernel size ks <= 8): out row r =
// C_r * conv_r, conv_r = sum_k w_k s_k over the window s_k = BX(r - ks + 1 +
// k), BX(j) = B_j * X_j for the tile's rows j >= 0 and the sequence's state
// (the phase's buffer) before them, st[ks + j] for j < 0; the state becomes
// BX(rows - ks + k), updated in place. proj rows are [B | C | X] (3 * dim),
// out rows dim. Thread (channel d, chunk c) computes rows 8c .. 8c + 7 with
// every load issued up front (the window of each row depends only on its
// inputs, not on the rows before); chunk 0's thread of a channel is the
// only one that reads the state (rows below ks - 1), so it writes the new
// one after. The same products and sums, in the same order, as the
// sequential window: bx = B * X, conv = w_0 s_0 + w_1 s_1 + ...
constexpr int kConvRowsChunk = 8;
__global__ void __launch_bounds__(256) conv_rows_kernel(const float* proj, float* out, int rows, int dim, int ks,
                                                        const float* conv_w, int conv_mode, float* st_a, float* st_b,
                                                        const int* phase) {
    constexpr int R = kConvRowsChunk;
    const int d = blockIdx.x * 256 + threadIdx.x;
    if (d >= dim) return;
    const int r0 = blockIdx.y * R;
    float* st = ((*phase) & 1 ? st_b : st_a) + (size_t)d * ks;
    float w[8];
    for (int k = 0; k < ks; k++)
        w[k] = conv_mode == 0 ? conv_w[(size_t)d * ks + k] : conv_mode == 1 ? conv_w[k] : 1.0f / (float)ks;
    // BX(j) for j = r0 - (ks - 1) .. r0 + R - 1: bx[j - r0 + ks - 1]
    float bx[R + 7], cv[R];
    auto BX = [&](int j) {
        if (j < 0) return st[ks + j];
        const float* p = proj + (size_t)j * 3 * dim;
        return p[d] * p[2 * dim + d];
    };
#pragma unroll
    for (int i = 0; i < R + 7; i++) {
        const int j = r0 - (ks - 1) + i;
        bx[i] = i < R + ks - 1 && j < rows ? BX(j) : 0.f;
    }
#pragma unroll
    for (int i = 0; i < R; i++) cv[i] = r0 + i < rows ? proj[(size_t)(r0 + i) * 3 * dim + dim + d] : 0.f;
#pragma unroll
    for (int i = 0; i < R; i++) {
        if (r0 + i >= rows) break;
        float conv = 0.f;
        if (ks == 3) {
            conv = w[0] * bx[i] + w[1] * bx[i + 1] + w[2] * bx[i + 2];  // ssm.rs:250-252
        } else {
            for (int k = 0; k < ks; k++) conv += w[k] * bx[i + k];
        }
        out[(size_t)(r0 + i) * dim + d] = cv[i] * conv;
    }
    if (blockIdx.y == 0) {
        float ns[8];
        for (int k = 0; k < ks; k++) ns[k] = BX(rows - ks + k);  // (reads the old state before the writes)
        for (int k = 0; k < ks; k++) st[k] = ns[k];
    }
}

__global__ void iota_kernel(int* dst, int base, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) dst[i] = base + i;
}

// Merges the nv = ceil(T / TT) splits of query head blockIdx.x:
// out = sum_s acc_s e^(m_s - M) * (1 / sum_s l_s e^(m_s - M)), the
// reciprocal multiply of transformer.rs:293-298.
// blockIdx.y: sequence of a batched launch (partials + b * part_s (m, l) and
// + b * part_s * hd (acc), out + b * out_s, position posp[b]).
// The position and every partial the launch needs (up to kCombineRegs
// splits per thread) are loaded at once, before nv is known (entries of
// splits past nv are masked, never multiplied), so the kernel waits for
// memory once; splits beyond that take a loop.
constexpr int kCombineRegs = 16;
__global__ void __launch_bounds__(kWG) attn_combine_kernel(const float* part_m, const float* part_l,
                                                           const float* part_acc, float* out, const int* posp,
                                                           int nsplit, int tt, int hd, int64_t part_s,
                                                           int64_t out_s) {
    __shared__ float w[kMaxAttnSplits];
    __shared__ float red[2][kWG / 64];
    __shared__ float part[kWG];
    const int h = blockIdx.x, b = blockIdx.y;
    part_m += b * part_s; part_l += b * part_s; part_acc += b * part_s * hd;
    out += b * out_s;
    const float* pm = part_m + (size_t)h * nsplit;
    const float* pl = part_l + (size_t)h * nsplit;
    // thread (g, d): dims d < hd, splits s = g, g + G, ...
    const int hdp = hd <= 64 ? 64 : 128, G = kWG / hdp;
    const int d = threadIdx.x % hdp, g = threadIdx.x / hdp;
    const float* acc = part_acc + (size_t)h * nsplit * hd + d;
    const int pos = posp[b];
    const bool own = (int)threadIdx.x < nsplit;
    const float m0 = own ? pm[threadIdx.x] : -INFINITY, l0 = own ? pl[threadIdx.x] : 0.f;
    float av[kCombineRegs];
#pragma unroll
    for (int k = 0; k < kCombineRegs; k++) {
        const int sk = g + k * G;
        av[k] = (d < hd && sk < nsplit) ? acc[(size_t)sk * hd] : 0.f;
    }
    const int ntiles = (pos + 1 + tt - 1) / tt;
    const int tps = (ntiles + nsplit - 1) / nsplit;
    const int nv = (ntiles + tps - 1) / tps;  // splits that hold tiles
    float M = (int)threadIdx.x < nv ? m0 : -INFINITY;
    for (int s = threadIdx.x + kWG; s < nv; s += kWG) M = fmaxf(M, pm[s]);
    M = wave_max(M);
    if ((threadIdx.x & 63) == 0) red[0][threadIdx.x >> 6] = M;
    __syncthreads();
    M = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));
    float L = 0.f;
    if ((int)threadIdx.x < nv) {
        const float ws = expf(m0 - M);
        w[threadIdx.x] = ws;
        L = l0 * ws;
    }
    for (int s = threadIdx.x + kWG; s < nv; s += kWG) {
        const float ws = expf(pm[s] - M);
        w[s] = ws;
        L = fmaf(pl[s], ws, L);
    }
    L = wave_sum(L);
    if ((threadIdx.x & 63) == 0) red[1][threadIdx.x >> 6] = L;
    __syncthreads();
    L = red[1][0] + red[1][1] + red[1][2] + red[1][3];
    float o = 0.f;
    if (d < hd) {
#pragma unroll
        for (int k = 0; k < kCombineRegs; k++)
            if (g + k * G < nv) o = fmaf(av[k], w[g + k * G], o);
        for (int s = g + kCombineRegs * G; s < nv; s += G) o = fmaf(acc[(size_t)s * hd], w[s], o);
    }
    part[threadIdx.x] = o;
    __syncthreads();
    if (g == 0 && d < hd) {
        for (int k = 1; k < G; k++) o += part[k * hdp + d];
        out[(size_t)h * hd + d] = L > 0.f ? o * (1.0f / L) : 0.f;
    }
}

// attn_combine_kernel for head_dim 64 and nsplit <= NS (16 or 32) in one wave per query
// head: lane s holds split s's (m, l), lane d sums dim d over the splits in
// the four interleaved chains of attn_combine_kernel's thread groups g =
// 0..3 (splits g, g + 4, ...) and adds them in the same order, with the same
// reductions (wave_max, wave_sum), so the output is the same bit for bit;
// without workgroup barriers or LDS the kernel waits for memory once and
// ends.
template <int NS>
__global__ void __launch_bounds__(64) attn_combine64_kernel(const float* part_m, const float* part_l,
                                                            const float* part_acc, float* out, const int* posp,
                                                            int nsplit, int tt, int64_t part_s, int64_t out_s) {
    constexpr int HD = 64;
    const int h = blockIdx.x, b = blockIdx.y, lane = threadIdx.x;
    part_m += b * part_s; part_l += b * part_s; part_acc += b * part_s * HD;
    out += b * out_s;
    const float* pm = part_m + (size_t)h * nsplit;
    const float* pl = part_l + (size_t)h * nsplit;
    const float* acc = part_acc + (size_t)h * nsplit * HD + lane;
    const int pos = posp[b];
    const bool own = lane < nsplit;
    const float m0 = own ? pm[lane] : -INFINITY, l0 = own ? pl[lane] : 0.f;
    float av[NS];
#pragma unroll
    for (int k = 0; k < NS; k++) av[k] = k < nsplit ? acc[(size_t)k * HD] : 0.f;
    const int ntiles = (pos + 1 + tt - 1) / tt;
    const int tps = (ntiles + nsplit - 1) / nsplit;
    const int nv = (ntiles + tps - 1) / tps;  // splits that hold tiles (wave-uniform)
    const float M = wave_max(lane < nv ? m0 : -INFINITY);
    float ws = 0.f, L = 0.f;
    if (lane < nv) {
        ws = expf(m0 - M);
        L = l0 * ws;
    }
    L = wave_sum(L);
    float o = 0.f;
#pragma unroll
    for (int g = 0; g < 4; g++) {
        float og = 0.f;
#pragma unroll
        for (int k = g; k < NS; k += 4)
            if (k < nv) og = fmaf(av[k], __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ws), k)), og);
        o = g == 0 ? og : o + og;
    }
    out[(size_t)h * HD + lane] = L > 0.f ? o * (1.0f / L) : 0.f;
}

// sampler.rs:305-316: index of the first strict maximum (NaN never wins).
// Writes the token for the next step, records it, advances pos and the
// ShortConv phase of the sequence.
// With part_idx set, `logits`/`n` are instead the per-wave (max, first row)
// partials of the head GEMV's argmax epilogue.
// blockIdx.x = b: sequence seq + b of a batched launch (values and indices
// + b * vstride; tok, pos, phase + b).
__global__ void __launch_bounds__(1024) argmax_advance_kernel(const float* logits, const int* part_idx, int n,
                                                              uint32_t* tok, int* pos, int* phase, uint32_t* history,
                                                              const int* pos0, int stride, int seq, int do_argmax,
                                                              int64_t vstride, EmbedNext en) {
    __shared__ float bv[16];
    __shared__ int bi[16];
    __shared__ uint32_t chosen;
    {
        const int b = blockIdx.x;
        logits += b * vstride;
        if (part_idx) part_idx += b * vstride;
        tok += b; pos += b; pos0 += b; phase += b;
        seq += b;
        en.x += b * en.xs;
    }
    if (do_argmax) {
        float best = -INFINITY;
        int idx = 0x7FFFFFFF;
        for (int i = threadIdx.x; i < n; i += blockDim.x) {
            const float v = logits[i];
            const int vi = part_idx ? part_idx[i] : i;
            if (v > best || (v == best && vi < idx)) { best = v; idx = vi; }
        }
#pragma unroll
        for (int sh = 32; sh >= 1; sh >>= 1) {
            float ov = __shfl_xor(best, sh, 64);
            int oi = __shfl_xor(idx, sh, 64);
            if (ov > best || (ov == best && oi < idx)) { best = ov; idx = oi; }
        }
        if ((threadIdx.x & 63) == 0) { bv[threadIdx.x >> 6] = best; bi[threadIdx.x >> 6] = idx; }
        __syncthreads();
        if (threadIdx.x == 0) {
            float b = bv[0];
            int id = bi[0];
            for (int w = 1; w < (int)(blockDim.x >> 6); w++)
                if (bv[w] > b || (bv[w] == b && bi[w] < id)) { b = bv[w]; id = bi[w]; }
            if (id == 0x7FFFFFFF) id = 0;
            *tok = (uint32_t)id;
            chosen = (uint32_t)id;
            // step k of a generate call runs at pos0 + k (pos advances below)
            if (history) history[(size_t)(*pos - *pos0) * stride + seq] = (uint32_t)id;
        }
        if (en.table) {
            __syncthreads();
            embed_row(en.type, en.table, en.row_bytes, chosen, en.x, en.dim, threadIdx.x, blockDim.x);
        }
    }
    if (threadIdx.x == 0) {
        *pos += 1;
        *phase += 1;
    }
}

__global__ void step_counter_kernel(int* step) { *step += 1; }

__global__ void set_ctrl_kernel(uint32_t* tok, int* pos, int* pos0, uint32_t t, int p) {
    *tok = t;
    *pos = p;
    *pos0 = p;
}

__global__ void set_int_kernel(int* dst, int v) { *dst = v; }

// --------------------------------------------------------------- model

struct Mat {
    int32_t type = 0;
    const uint8_t* w = nullptr;  // device
    size_t rows = 0, cols = 0;
    // the same rows packed for one-column GEMVs (Q4_K row quads; Q6_K row
    // quads at 2048 columns, unit planes at 4096 or 8192), else null
    const uint8_t* quad = nullptr;
    // Q4_K: the rows in the row products' operand layout (prefill tiles of
    // 16+ rows on the matrix cores; launch_pack_q4k_gemm), else null
    const uint8_t* gemm = nullptr;
};

struct Layer {
    bool attn = false;
    const float* norm = nullptr;       // attn_norm / ssm_norm (device f32)
    const float* q_norm = nullptr;
    const float* k_norm = nullptr;
    Mat wq, wk, wv, wo, in_proj, out_proj, gate, up, down;
    const float* conv = nullptr;
    size_t conv_len = 0;
    const float* ffn_norm = nullptr;
    int cache_idx = -1;
    // batched Q4_K launches' rows in the column kernel's group order
    // (launch_pack_q4k_cols; models with max_batch > 1), else null: q|k|v,
    // wo or out_proj, in_proj (conv groups), gate|up (SwiGLU groups), down
    const uint8_t *cw_qkv = nullptr, *cw_o = nullptr, *cw_in = nullptr, *cw_gu = nullptr, *cw_down = nullptr;
};

struct SeqState {
    float *x, *sc_in, *hb, *hb2, *q, *k, *v, *attn_out, *logits;
    float *conv_a, *conv_b;  // ping-pong [n_layers * dim * ksize]
    float *part_m, *part_l, *part_acc;
    float* part_val;  // head GEMV argmax partials (kMaxArgmaxParts)
    int* part_idx;
    uint8_t *kc, *vc;        // [n_attn * max_seq * row_bytes]
};

// Element strides between consecutive sequences' vectors in the per-kind
// arenas (SeqState pointers of sequence b = arena + b * stride).
struct SeqStrides {
    size_t x = 0, sc_in = 0, hb = 0, qkv = 0, logits = 0, conv = 0, parts = 0;
    size_t kv = 0;    // bytes: one sequence's K (or V) cache
    size_t part = 0;  // attention split partials (m, l) per sequence; acc: part * head_dim
};

struct Ctrl {  // device control block
    uint32_t tok[64];
    int pos[64];
    int pos0[64];  // position at the last set_ctrl: a greedy step's index is pos - pos0
    int phase[64];
    int step;      // the sampled generation's step counter
};

}  // namespace

// Waves (kv heads) per workgroup of the Q8_0 group kernel: every kv head of
// a split in one workgroup (8 for the 1.2B model), so a workgroup reads whole
// cache rows (all kv heads of 16 tokens, contiguous).
inline int attn_q8_waves(int n_kv) { return n_kv > 4 ? 8 : 4; }

// Splits per sequence of the Q8_0 group kernel for a batch of nb sequences:
// about eight waves per CU in all, at most `cap`. Fewer, longer splits keep
// each wave streaming: for config 5 (8 sequences) 8 waves per CU give 7131
// tok/s against 6607 at 16 and 6353 at 4.
int attn_q8_splits(int cap, int nb, int n_kv) {
    const int w = attn_q8_waves(n_kv);
    const int waves = std::max(1, nb * w * ((n_kv + w - 1) / w));
    return std::max(1, std::min(cap, 8 * num_cus() / waves));
}

// Attention of nseq sequences (tile rows) over their caches, then the merge of
// the splits into out (+ b * out_s).
void enqueue_attention(const mivi_model_info& c, const AttnArgs& a, unsigned nseq, float* out, int64_t out_s,
                       hipStream_t s) {
    int tt;
    if (a.packed) {  // Q8_0 group layout (attn_q8_mfma_ok shapes)
        // three groups in flight per wave: other depths measured slower
        // (config 5: 6583 tok/s at 2, 7095 at 3, 6645 at 4, 6356 at 6; at
        // one workgroup per CU and up to 256 registers 8090 at 3 and 4, 7450
        // at 6, against 8400 here). The kernel waits on memory: its score and
        // value arithmetic taken out, a launch is under 2 us shorter.
        const int w = attn_q8_waves((int)c.n_kv_heads);
        dim3 grid(attn_tile_grid(((int)c.n_kv_heads + w - 1) / w, a.nsplit), nseq);
        if (w == 8) hipLaunchKernelGGL((attn_q8_mfma_kernel<3, 8>), grid, dim3(512), 0, s, a);
        else hipLaunchKernelGGL((attn_q8_mfma_kernel<3, 4>), grid, dim3(kWG), 0, s, a);
        tt = kQ8GroupTokens;
    } else if (attn_f16_mfma_ok(c.kv_precision, (int)c.head_dim, (int)c.n_heads, (int)c.n_kv_heads)) {
        // fp16 rows in 16-token groups on the matrix cores, one wave per
        // workgroup (the XCD placement of attn_tile_of spreads them)
        dim3 grid(attn_tile_grid((int)c.n_kv_heads, a.nsplit), nseq);
        hipLaunchKernelGGL((attn_f16_mfma_kernel<4>), grid, dim3(64), 0, s, a);
        tt = kQ8GroupTokens;
    } else {
        dim3 grid(attn_tile_grid((int)c.n_kv_heads, a.nsplit), nseq);
#define ATT(KVP, HDM) hipLaunchKernelGGL((attn_tile_kernel<KVP, HDM>), grid, dim3(kWG), 0, s, a)
        if (c.head_dim <= 64) {
            if (c.kv_precision == MIVI_KV_F32) ATT(MIVI_KV_F32, 64);
            else if (c.kv_precision == MIVI_KV_F16) ATT(MIVI_KV_F16, 64);
            else ATT(MIVI_KV_Q8_0, 64);
        } else {
            if (c.kv_precision == MIVI_KV_F32) ATT(MIVI_KV_F32, 128);
            else if (c.kv_precision == MIVI_KV_F16) ATT(MIVI_KV_F16, 128);
            else ATT(MIVI_KV_Q8_0, 128);
        }
#undef ATT
        tt = attn_tile_tokens(c.head_dim);
    }
    // (at 33-64 splits, a wave's 64 + 3 loads exceed the 63 it may have in
    // flight: the 256-thread merge is faster there, 2365 against 2303 tok/s
    // on config 4 with the loads split over the wave's halves)
    if (c.head_dim == 64 && a.nsplit <= 32) {
#define CMB(NS)                                                                                                    \
    hipLaunchKernelGGL(attn_combine64_kernel<NS>, dim3((unsigned)c.n_heads, nseq), dim3(64), 0, s, a.part_m, a.part_l, \
                       a.part_acc, out, a.pos, a.nsplit, tt, a.part_s, out_s)
        if (a.nsplit <= 16) CMB(16);
        else CMB(32);
#undef CMB
        return;
    }
    hipLaunchKernelGGL(attn_combine_kernel, dim3((unsigned)c.n_heads, nseq), dim3(kWG), 0, s, a.part_m, a.part_l,
                       a.part_acc, out, a.pos, a.nsplit, tt, (int)c.head_dim, a.part_s, out_s);
}

struct mivi_model {
    mivi_model_info info{};
    hipStream_t stream = nullptr;
    uint8_t* d_weights = nullptr;
    float* d_aux = nullptr;  // decoded f32 vectors
    Mat embd, head;
    uint8_t* head_packed = nullptr;  // Q6_K head in the packed unit-plane layout (else null)
    uint8_t* head_t32 = nullptr;     // max_batch > 1: the Q6_K head in 32-row tiles for batched steps (else null)
    const float* out_norm = nullptr;
    std::vector<Layer> layers;
    float *rope_cos = nullptr, *rope_sin = nullptr;
    std::vector<SeqState> seqs;
    SeqStrides strides;
    std::vector<void*> allocs;
    Ctrl* ctrl = nullptr;
    uint32_t* history = nullptr;  // [max_seq * max_batch]
    size_t kv_row_bytes = 0;
    bool kv_packed = false;    // Q8_0 caches in the q8g_* group layout
    size_t kv_layer_bytes = 0; // one attention layer's K (or V) cache of one sequence
    int nsplit = 1;
    hipGraphExec_t graph = nullptr;
    size_t graph_batch = 0;
    // sampled generation: per-sequence xorshift64* states and the step graph
    // captured for one (batch, config, end-of-sequence ids)
    uint64_t* rng = nullptr;  // [max_batch]
    uint8_t* samp_ws = nullptr;  // the sampler's candidates, sample_seq_workspace(vocab, max_batch) bytes
    hipGraphExec_t graph_s = nullptr;
    size_t graph_s_batch = 0;
    mivi_sampler_config graph_s_cfg{};
    SampleEos graph_s_eos{};
    // chunked prefill (PrefillStrategy::Chunked, model.rs:519-536): rows per
    // tile (0 = token by token) and the tile buffers, allocated on first use
    size_t prefill_tile = 0, pf_cap = 0;
    float *pf_x = nullptr, *pf_p1 = nullptr, *pf_p2 = nullptr, *pf_ao = nullptr;
    float *pf_pm = nullptr, *pf_pl = nullptr, *pf_pa = nullptr;
    int* pf_pos = nullptr;
    uint32_t* pf_tok = nullptr;

    ~mivi_model() {
        if (graph) hipGraphExecDestroy(graph);
        if (graph_s) hipGraphExecDestroy(graph_s);
        for (void* p : allocs) hipFree(p);
        if (stream) hipStreamDestroy(stream);
    }
    template <typename T>
    int32_t alloc(T** p, size_t count) {
        void* q = nullptr;
        hipError_t e = hipMalloc(&q, std::max<size_t>(1, count * sizeof(T)));
        if (e != hipSuccess) return set_error(MIVI_ERR_HIP, "hipMalloc(%zu) failed: %s", count * sizeof(T), hipGetErrorString(e));
        // zeroed on the model's stream and waited for: the stream is
        // non-blocking, so a null-stream memset could still be running (and
        // overwrite data) when the stream's next copy or kernel touches the
        // buffer, as the first prefill does right after allocating its tiles
        e = hipMemsetAsync(q, 0, std::max<size_t>(1, count * sizeof(T)), stream);
        if (e == hipSuccess) e = hipStreamSynchronize(stream);
        if (e != hipSuccess) {
            (void)hipFree(q);
            return set_error(MIVI_ERR_HIP, "zeroing %zu bytes failed: %s", count * sizeof(T), hipGetErrorString(e));
        }
        allocs.push_back(q);
        *p = (T*)q;
        return MIVI_OK;
    }
};

namespace {

// Enqueues part of one decode step of sequences b0 .. b0+nb-1: the
// embeddings (do_embed), layers [l0, l1), then the head, argmax and position
// advance (do_head). Each projection is one GEMV over the nb sequences'
// activation columns (weights read once for all of them); attention runs per
// sequence.
// The embedding of the next token by the argmax kernel (when `on`), into the
// activation arena starting at x (sequence b at x + b * strides.x).
EmbedNext embed_next_args(mivi_model* m, float* x, bool on) {
    EmbedNext en{};
    if (!on) return en;
    size_t bs, ts;
    format_sizes(m->embd.type, &bs, &ts);
    en.table = m->embd.w;
    en.row_bytes = (m->info.dim * ts) / bs;  // model.rs:358-360
    en.x = x;
    en.xs = (int64_t)m->strides.x;
    en.type = m->embd.type;
    en.dim = (int)m->info.dim;
    return en;
}

// The segments of g (matrices ms, in order) in runs of equal weight type:
// launch(type, the run's arguments, its matrices, their count) per run.
template <class F>
int32_t by_type_runs(const GemvArgs& g, std::initializer_list<const Mat*> ms, F&& launch) {
    const Mat* const* v = ms.begin();
    for (int i = 0; i < g.nseg;) {
        int j = i + 1;
        while (j < g.nseg && v[j]->type == v[i]->type) j++;
        GemvArgs r = g;
        r.nseg = j - i;
        for (int k = i; k < j; k++) r.seg[k - i] = g.seg[k];
        const int32_t rc = launch(v[i]->type, r, v + i, j - i);
        if (rc) return rc;
        i = j;
    }
    return MIVI_OK;
}

// A decode projection over the matrices ms[0 .. g.nseg): with one column and
// every matrix held packed, the GEMV on the packed rows (the same results
// bit for bit); otherwise the GGUF rows.
int32_t launch_proj(int32_t t, int pro, const GemvArgs& g, std::initializer_list<const Mat*> ms, hipStream_t s) {
    bool quads = g.ncol <= 1 && (int)ms.size() == g.nseg;
    for (const Mat* x : ms) quads = quads && x->quad;
    if (quads) {
        GemvArgs q = g;
        int i = 0;
        for (const Mat* x : ms) q.seg[i++].W = x->quad;
        q.packed = 1;
        const int32_t rc = launch_gemv_ex(t, pro, q, s);
        if (rc != MIVI_ERR_UNSUPPORTED) return rc;
    }
    return launch_gemv_ex(t, pro, g, s);
}

int32_t enqueue_step(mivi_model* m, size_t b0, size_t nb, bool logits, bool argmax, hipStream_t s, bool do_embed,
                     size_t l0, size_t l1, bool do_head, bool embed_next) {
    const mivi_model_info& c = m->info;
    const SeqStrides& z = m->strides;
    SeqState& s0 = m->seqs[b0];
    int32_t rc;
    const int D = (int)c.dim, H = (int)c.hidden_dim, KV = (int)c.kv_dim;
    const int ncol = (int)nb;
    if (do_embed) {
        size_t bs, ts;
        format_sizes(m->embd.type, &bs, &ts);
        size_t row_bytes = (c.dim * ts) / bs;  // model.rs:358-360
        hipLaunchKernelGGL(embed_kernel, dim3((unsigned)nb), dim3(kWG), 0, s, m->embd.type, m->embd.w, row_bytes,
                           &m->ctrl->tok[b0], s0.x, D, (int64_t)z.x);
    }
    for (size_t l = l0; l < l1 && l < c.n_layers; l++) {
        const Layer& L = m->layers[l];
        GemvArgs g = {};
        if (!L.attn) {
            if (c.ssm_conv_kernel == 0) continue;  // ssm.rs:60-62
            // in_proj on rms_norm(x, ssm_norm) with the gated conv (ssm.rs:80-140)
            // in its epilogue, which writes C * conv to sc_in[0, D) and the next
            // window; shapes the epilogue does not take store [B|C|X] and run
            // the conv as out_proj's prologue instead
            const size_t ks = c.ssm_conv_kernel;
            g.seg[0] = {L.in_proj.w, s0.sc_in, 3 * D};
            g.nseg = 1; g.K = D; g.x = s0.x; g.norm_w = L.norm; g.eps = c.rms_norm_eps;
            g.ncol = ncol; g.xs = z.x; g.ys = z.sc_in;
            g.conv_w = L.conv;
            g.conv_mode = (L.conv && L.conv_len >= (size_t)D * ks) ? 0 : (L.conv && L.conv_len >= ks) ? 1 : 2;
            g.ksize = (int)ks;
            g.st_in = s0.conv_a + l * (size_t)D * ks;
            g.st_out = s0.conv_b + l * (size_t)D * ks;
            g.phase = &m->ctrl->phase[b0];
            g.sts = z.conv;
            g.epilogue = EPI_CONV;
            g.cw = ncol > 1 ? L.cw_in : nullptr;
            rc = launch_proj(L.in_proj.type, PRO_RMSNORM, g, {&L.in_proj}, s);
            const bool conv_fused = rc == MIVI_OK;
            if (rc && rc != MIVI_ERR_UNSUPPORTED) return rc;
            if (!conv_fused) {
                g.epilogue = EPI_STORE;
                g.cw = nullptr;  // packed in the conv groups' order
                if ((rc = launch_gemv_ex(L.in_proj.type, PRO_RMSNORM, g, s))) return rc;
            }
            // out_proj on the gated conv, residual add into x
            GemvArgs go = {};
            go.seg[0] = {L.out_proj.w, s0.x, D};
            go.nseg = 1; go.K = D; go.x = s0.sc_in;
            go.accumulate = 1;
            go.ncol = ncol; go.xs = z.sc_in; go.ys = z.x;
            go.cw = ncol > 1 ? L.cw_o : nullptr;
            if (!conv_fused) {
                go.conv_w = g.conv_w; go.conv_mode = g.conv_mode; go.ksize = g.ksize;
                go.st_in = g.st_in; go.st_out = g.st_out; go.phase = g.phase; go.sts = g.sts;
            }
            if ((rc = launch_proj(L.out_proj.type, conv_fused ? PRO_NONE : PRO_CONV, go, {&L.out_proj}, s))) return rc;
        } else {
            g.seg[0] = {L.wq.w, s0.q, D};
            g.seg[1] = {L.wk.w, s0.k, KV};
            g.seg[2] = {L.wv.w, s0.v, KV};
            g.nseg = 3; g.K = D; g.x = s0.x; g.norm_w = L.norm; g.eps = c.rms_norm_eps;
            g.ncol = ncol; g.xs = z.x; g.ys = z.qkv;
            g.cw = ncol > 1 ? L.cw_qkv : nullptr;  // (all three Q4_K: one run)
            // one launch per run of equal weight types (a Q4_K_M file's
            // Q6_K attn_v runs apart from q|k)
            rc = by_type_runs(g, {&L.wq, &L.wk, &L.wv}, [&](int32_t t, const GemvArgs& gr, const Mat* const* mr, int n) {
                if (n == 3) return launch_proj(t, PRO_RMSNORM, gr, {mr[0], mr[1], mr[2]}, s);
                if (n == 2) return launch_proj(t, PRO_RMSNORM, gr, {mr[0], mr[1]}, s);
                return launch_proj(t, PRO_RMSNORM, gr, {mr[0]}, s);
            });
            if (rc) return rc;
            {
                // one launch for the nb sequences (blockIdx.y = sequence)
                AttnArgs a = {};
                a.q = s0.q; a.k = s0.k; a.v = s0.v;
                a.q_norm = L.q_norm; a.k_norm = L.k_norm; a.eps = c.rms_norm_eps;
                a.rope_cos = m->rope_cos; a.rope_sin = m->rope_sin;
                a.kc = s0.kc + (size_t)L.cache_idx * m->kv_layer_bytes;
                a.vc = s0.vc + (size_t)L.cache_idx * m->kv_layer_bytes;
                a.row_bytes = m->kv_row_bytes;
                a.packed = m->kv_packed;
                a.pos = &m->ctrl->pos[b0];
                a.n_heads = (int)c.n_heads; a.n_kv_heads = (int)c.n_kv_heads; a.hd = (int)c.head_dim;
                // Q8_0 group kernel: about two workgroups per CU over the
                // batch's sequences (config 5, 8 sequences: 32 splits of
                // 1024 tokens, 4067 against 3820 tok/s with 64)
                a.nsplit = m->kv_packed || attn_f16_mfma_ok(c.kv_precision, (int)c.head_dim, (int)c.n_heads,
                                                            (int)c.n_kv_heads)
                               ? attn_q8_splits(m->nsplit, (int)nb, (int)c.n_kv_heads)
                               : m->nsplit;
                a.scale = 1.0f / sqrtf((float)c.head_dim);
                a.part_m = s0.part_m; a.part_l = s0.part_l; a.part_acc = s0.part_acc;
                a.qkv_s = (int64_t)z.qkv; a.kv_s = (int64_t)z.kv; a.part_s = (int64_t)z.part;
                enqueue_attention(c, a, (unsigned)nb, s0.attn_out, (int64_t)z.x, s);
            }
            g = {};
            g.seg[0] = {L.wo.w, s0.x, D};
            g.nseg = 1; g.K = D; g.x = s0.attn_out; g.accumulate = 1;
            g.ncol = ncol; g.xs = z.x; g.ys = z.x;
            g.cw = ncol > 1 ? L.cw_o : nullptr;
            if ((rc = launch_proj(L.wo.type, PRO_NONE, g, {&L.wo}, s))) return rc;
        }
        // ffn.rs:56-108
        g = {};
        g.seg[0] = {L.gate.w, s0.hb, H};
        g.seg[1] = {L.up.w, s0.hb2, H};
        g.nseg = 2; g.K = D; g.x = s0.x; g.norm_w = L.ffn_norm; g.eps = c.rms_norm_eps;
        g.ncol = ncol; g.xs = z.x; g.ys = z.hb;
        bool fused = false;
        if (L.gate.type == L.up.type) {
            // gate|up with the SwiGLU epilogue writes silu(gate) * up into hb
            // directly where the streaming kernel takes the shape
            g.epilogue = EPI_SWIGLU;
            g.cw = ncol > 1 ? L.cw_gu : nullptr;
            rc = launch_proj(L.gate.type, PRO_RMSNORM, g, {&L.gate, &L.up}, s);
            fused = rc == MIVI_OK;
            if (rc && rc != MIVI_ERR_UNSUPPORTED) return rc;
            g.epilogue = EPI_STORE;
            g.cw = nullptr;  // packed in the SwiGLU groups' order
        }
        if (fused) {
        } else if (L.gate.type == L.up.type) {
            if ((rc = launch_proj(L.gate.type, PRO_RMSNORM, g, {&L.gate, &L.up}, s))) return rc;
        } else {
            GemvArgs g1 = g;
            g1.nseg = 1;
            if ((rc = launch_proj(L.gate.type, PRO_RMSNORM, g1, {&L.gate}, s))) return rc;
            g1.seg[0] = g.seg[1];
            if ((rc = launch_proj(L.up.type, PRO_RMSNORM, g1, {&L.up}, s))) return rc;
        }
        g = {};
        g.seg[0] = {L.down.w, s0.x, D};
        g.nseg = 1; g.K = H; g.x = s0.hb; g.x2 = s0.hb2; g.accumulate = 1;
        g.ncol = ncol; g.xs = z.hb; g.ys = z.x;
        g.cw = ncol > 1 && fused ? L.cw_down : nullptr;
        if ((rc = launch_proj(L.down.type, fused ? PRO_NONE : PRO_SWIGLU, g, {&L.down}, s))) return rc;
    }
    if (!do_head) {
        MIVI_HIP_CHECK(hipGetLastError());
        return MIVI_OK;
    }
    int parts = 0;  // > 0: the head GEMV reduced the argmax to per-wave partials
    if (logits) {
        // model.rs:435-473
        GemvArgs g = {};
        g.seg[0] = {m->head_packed ? m->head_packed : m->head.w, s0.logits, (int)c.vocab_size};
        g.nseg = 1; g.K = D; g.x = s0.x; g.norm_w = m->out_norm; g.eps = c.rms_norm_eps;
        g.packed = m->head_packed ? 1 : 0;
        g.ncol = ncol; g.xs = z.x; g.ys = z.logits;
        const int pro = m->out_norm ? PRO_RMSNORM : PRO_NONE;
        // batched: the 32-row tile copy when there is one
        const bool t32 = ncol > 1 && m->head_t32;
        if (t32) { g.seg[0].W = m->head_t32; g.packed = 0; }
        auto launch = [&]() { return t32 ? launch_gemv_t32(pro, g, s) : launch_gemv_ex(m->head.type, pro, g, s); };
        const int np = !argmax ? 0
                       : t32   ? t32_argmax_parts((int)c.vocab_size)
                               : gemv_argmax_parts(m->head.type, D, (int)c.vocab_size, m->head_packed != nullptr);
        if (np > 0 && np <= kMaxArgmaxParts) {
            g.epilogue = EPI_ARGMAX;
            g.part_val = s0.part_val;
            g.part_idx = s0.part_idx;
            g.ps = z.parts;
            rc = launch();
            if (rc == MIVI_OK) parts = np;
            else if (rc != MIVI_ERR_UNSUPPORTED) return rc;
            g.epilogue = EPI_STORE;
        }
        if (!parts && (rc = launch())) return rc;
    }
    hipLaunchKernelGGL(argmax_advance_kernel, dim3((unsigned)nb), dim3(1024), 0, s, parts ? s0.part_val : s0.logits,
                       parts ? s0.part_idx : nullptr, parts ? parts : (int)c.vocab_size, &m->ctrl->tok[b0],
                       &m->ctrl->pos[b0], &m->ctrl->phase[b0], argmax ? m->history : nullptr, &m->ctrl->pos0[b0],
                       (int)c.max_batch, (int)b0, (argmax && logits) ? 1 : 0,
                       (int64_t)(parts ? z.parts : z.logits), embed_next_args(m, s0.x, embed_next && argmax && logits));
    MIVI_HIP_CHECK(hipGetLastError());
    return MIVI_OK;
}

int32_t enqueue_step(mivi_model* m, size_t b, bool logits, bool argmax, hipStream_t s) {
    return enqueue_step(m, b, 1, logits, argmax, s, true, 0, m->info.n_layers, true, false);
}

// One greedy step of sequences 0..batch-1, layer by layer across the
// sequences: every projection is one GEMV over all the sequences' columns.
// The step starts from x already holding the tokens' embeddings and ends by
// embedding the chosen tokens for the next step (the first step's embedding
// is the caller's).
int32_t enqueue_batch_step(mivi_model* m, size_t batch, hipStream_t s) {
    return enqueue_step(m, 0, batch, true, true, s, false, 0, m->info.n_layers, true, true);
}

constexpr int kPrefillSplits = 16;  // attention splits per tile row, at most

// Tile buffers for `rows` rows (grow-only).
int32_t prefill_buffers(mivi_model* m, size_t rows) {
    if (m->pf_cap >= rows) return MIVI_OK;
    const mivi_model_info& c = m->info;
    const size_t D = c.dim, H = c.hidden_dim, KV = c.kv_dim;
    const size_t p1 = std::max({3 * D, D + 2 * KV, H});
    const size_t parts = rows * c.n_heads * kPrefillSplits;
    int32_t rc;
    if ((rc = m->alloc(&m->pf_x, rows * D)) || (rc = m->alloc(&m->pf_p1, rows * p1)) ||
        (rc = m->alloc(&m->pf_p2, rows * H)) || (rc = m->alloc(&m->pf_ao, rows * D)) ||
        (rc = m->alloc(&m->pf_pm, parts)) || (rc = m->alloc(&m->pf_pl, parts)) ||
        (rc = m->alloc(&m->pf_pa, parts * c.head_dim)) || (rc = m->alloc(&m->pf_pos, rows)) ||
        (rc = m->alloc(&m->pf_tok, rows)))
        return rc;
    m->pf_cap = rows;
    return MIVI_OK;
}

// One prefill tile of sequence b: tokens (device) at positions p0 .. p0+rows-1
// through every layer (model.rs:608-831 with attention_forward_tile and
// ssm_forward_tile): row-batch products for the projections (matrix cores
// for Q4_K), the tile's K/V stored before attention, attention per row over
// the cache, the ShortConv window walked over the rows. Leaves the caches and
// the conv state as the token-by-token path would; the residual rows are
// dropped at the end (the next decode step embeds its own token).
int32_t enqueue_prefill_tile(mivi_model* m, size_t b, size_t p0, size_t rows, hipStream_t s) {
    const mivi_model_info& c = m->info;
    SeqState& st = m->seqs[b];
    const int D = (int)c.dim, H = (int)c.hidden_dim, KV = (int)c.kv_dim, R = (int)rows;
    const size_t ldq = (size_t)D + 2 * KV;
    int32_t rc;
    size_t bs, ts;
    format_sizes(m->embd.type, &bs, &ts);
    hipLaunchKernelGGL(embed_kernel, dim3((unsigned)R), dim3(kWG), 0, s, m->embd.type, m->embd.w,
                       (c.dim * ts) / bs, m->pf_tok, m->pf_x, D, (int64_t)D);
    hipLaunchKernelGGL(iota_kernel, dim3((unsigned)((R + 255) / 256)), dim3(256), 0, s, m->pf_pos, (int)p0, R);
    for (size_t l = 0; l < c.n_layers; l++) {
        const Layer& L = m->layers[l];
        GemvArgs g = {};
        if (!L.attn) {
            if (c.ssm_conv_kernel == 0) continue;  // ssm.rs:60-62
            g.seg[0] = {L.in_proj.w, m->pf_p1, 3 * D, L.in_proj.gemm};
            g.nseg = 1; g.K = D; g.x = m->pf_x; g.norm_w = L.norm; g.eps = c.rms_norm_eps;
            g.ncol = R; g.xs = D; g.ys = 3 * D;
            if ((rc = launch_rows(L.in_proj.type, PRO_RMSNORM, g, s))) return rc;
            const size_t ks = c.ssm_conv_kernel;
            const int mode = (L.conv && L.conv_len >= (size_t)D * ks) ? 0 : (L.conv && L.conv_len >= ks) ? 1 : 2;
            hipLaunchKernelGGL(conv_rows_kernel,
                               dim3((unsigned)((D + 255) / 256), (unsigned)((R + kConvRowsChunk - 1) / kConvRowsChunk)),
                               dim3(256), 0, s, m->pf_p1,
                               m->pf_ao, R, D, (int)ks, L.conv, mode, st.conv_a + l * (size_t)D * ks,
                               st.conv_b + l * (size_t)D * ks, &m->ctrl->phase[b]);
            g = {};
            g.seg[0] = {L.out_proj.w, m->pf_x, D, L.out_proj.gemm};
            g.nseg = 1; g.K = D; g.x = m->pf_ao; g.accumulate = 1;
            g.ncol = R; g.xs = D; g.ys = D;
            if ((rc = launch_rows(L.out_proj.type, PRO_NONE, g, s))) return rc;
        } else {
            g.seg[0] = {L.wq.w, m->pf_p1, D, L.wq.gemm};
            g.seg[1] = {L.wk.w, m->pf_p1 + D, KV, L.wk.gemm};
            g.seg[2] = {L.wv.w, m->pf_p1 + D + KV, KV, L.wv.gemm};
            g.nseg = 3; g.K = D; g.x = m->pf_x; g.norm_w = L.norm; g.eps = c.rms_norm_eps;
            g.ncol = R; g.xs = D; g.ys = (int64_t)ldq;
            rc = by_type_runs(g, {&L.wq, &L.wk, &L.wv}, [&](int32_t t, const GemvArgs& gr, const Mat* const*, int) {
                return launch_rows(t, PRO_RMSNORM, gr, s);
            });
            if (rc) return rc;
            AttnArgs a = {};
            a.q = m->pf_p1; a.k = m->pf_p1 + D; a.v = m->pf_p1 + D + KV;
            a.q_norm = L.q_norm; a.k_norm = L.k_norm; a.eps = c.rms_norm_eps;
            a.rope_cos = m->rope_cos; a.rope_sin = m->rope_sin;
            a.kc = st.kc + (size_t)L.cache_idx * m->kv_layer_bytes;
            a.vc = st.vc + (size_t)L.cache_idx * m->kv_layer_bytes;
            a.row_bytes = m->kv_row_bytes;
            a.packed = m->kv_packed;
            a.n_heads = (int)c.n_heads; a.n_kv_heads = (int)c.n_kv_heads; a.hd = (int)c.head_dim;
            a.scale = 1.0f / sqrtf((float)c.head_dim);
            a.qkv_s = (int64_t)ldq; a.kv_s = 0;
            // 1. the tile's K/V rows into the cache
            dim3 sgrid((unsigned)R, (unsigned)c.n_kv_heads);
#define KVS(KVP) hipLaunchKernelGGL((kv_store_rows_kernel<KVP>), sgrid, dim3(64), 0, s, a, (int)p0)
            if (c.kv_precision == MIVI_KV_F32) KVS(MIVI_KV_F32);
            else if (c.kv_precision == MIVI_KV_F16) KVS(MIVI_KV_F16);
            else KVS(MIVI_KV_Q8_0);
#undef KVS
            // 2. attention of every row over the cache up to its position
            const size_t tt = (size_t)attn_tile_tokens(c.head_dim);
            const int nsplit = (int)std::max<size_t>(1, std::min<size_t>(kPrefillSplits, (p0 + rows + 8 * tt - 1) / (8 * tt)));
            a.pos = m->pf_pos;
            a.nsplit = nsplit;
            a.part_m = m->pf_pm; a.part_l = m->pf_pl; a.part_acc = m->pf_pa;
            a.part_s = (int64_t)c.n_heads * nsplit;
            a.keep_cache = 1;
            enqueue_attention(c, a, (unsigned)R, m->pf_ao, (int64_t)D, s);
            g = {};
            g.seg[0] = {L.wo.w, m->pf_x, D, L.wo.gemm};
            g.nseg = 1; g.K = D; g.x = m->pf_ao; g.accumulate = 1;
            g.ncol = R; g.xs = D; g.ys = D;
            if ((rc = launch_rows(L.wo.type, PRO_NONE, g, s))) return rc;
        }
        // ffn.rs:56-108 on the rows
        g = {};
        g.seg[0] = {L.gate.w, m->pf_p1, H, L.gate.gemm};
        g.seg[1] = {L.up.w, m->pf_p2, H, L.up.gemm};
        g.nseg = 2; g.K = D; g.x = m->pf_x; g.norm_w = L.ffn_norm; g.eps = c.rms_norm_eps;
        g.ncol = R; g.xs = D; g.ys = H;
        if (L.gate.type == L.up.type) {
            if ((rc = launch_rows(L.gate.type, PRO_RMSNORM, g, s))) return rc;
        } else {
            GemvArgs g1 = g;
            g1.nseg = 1;
            if ((rc = launch_rows(L.gate.type, PRO_RMSNORM, g1, s))) return rc;
            g1.seg[0] = g.seg[1];
            if ((rc = launch_rows(L.up.type, PRO_RMSNORM, g1, s))) return rc;
        }
        g = {};
        g.seg[0] = {L.down.w, m->pf_x, D, L.down.gemm};
        g.nseg = 1; g.K = H; g.x = m->pf_p1; g.x2 = m->pf_p2; g.accumulate = 1;
        g.ncol = R; g.xs = H; g.ys = D;
        if ((rc = launch_rows(L.down.type, PRO_SWIGLU, g, s))) return rc;
    }
    MIVI_HIP_CHECK(hipGetLastError());
    return MIVI_OK;
}

void host_rope_table(std::vector<float>& cs, std::vector<float>& sn, size_t hd, size_t max_seq, float base,
                     bool yarn, float scale) {
    // rope.rs:50-122 with the YaRN parameters of model.rs:194-206
    size_t half = hd / 2;
    std::vector<float> inv(half);
    for (size_t i = 0; i < half; i++) {
        float bf = 1.0f / powf(base, (float)(2 * i) / (float)hd);
        float f = bf;
        if (yarn && scale > 1.0f) {
            float orig = 4096.0f, beta_fast = 32.0f, beta_slow = 1.0f;
            float low_rot = orig / std::max(beta_slow, 0.01f);
            float high_rot = orig / std::max(beta_fast, 0.01f);
            float wl = 2.0f * (float)M_PI / bf;
            float ramp;
            if (high_rot >= low_rot) ramp = wl < high_rot ? 0.0f : 1.0f;
            else if (wl < high_rot) ramp = 0.0f;
            else if (wl > low_rot) ramp = 1.0f;
            else ramp = (wl - high_rot) / (low_rot - high_rot);
            float sf = bf / scale;
            f = (1.0f - ramp) * bf + ramp * sf;
        }
        inv[i] = f;
    }
    cs.resize(max_seq * half);
    sn.resize(max_seq * half);
    for (size_t p = 0; p < max_seq; p++)
        for (size_t i = 0; i < half; i++) {
            float ang = (float)p * inv[i];
            cs[p * half + i] = cosf(ang);
            sn[p * half + i] = sinf(ang);
        }
}

int32_t model_error(int32_t code, const char* fmt, ...) {
    char buf[240];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    return set_error(code, "%s", buf);
}

}  // namespace

// ----------------------------------------------------------------- C ABI

extern "C" int32_t mivi_hip_model_create(const uint8_t* img, size_t len, size_t max_ctx, int32_t kv_precision,
                                         size_t max_batch, mivi_model** out) {
    if (!img || !out) return set_error(MIVI_ERR_INVALID_ARGUMENT, "null argument");
    *out = nullptr;
    if (max_batch == 0 || max_batch > 64) return set_error(MIVI_ERR_INVALID_ARGUMENT, "max_batch must be 1..64");
    if (kv_precision != MIVI_KV_F32 && kv_precision != MIVI_KV_F16 && kv_precision != MIVI_KV_Q8_0)
        return set_error(MIVI_ERR_INVALID_ARGUMENT, "unknown kv precision %d", kv_precision);
    Gguf g;
    int32_t rc = parse_gguf(img, len, &g);
    if (rc) return rc;
    auto meta_u = [&](const char* k2, const char* k1, size_t* dst) {
        for (const char* k : {k2, k1}) {
            auto it = g.meta.find(k);
            if (it != g.meta.end() && it->second.is_uint) *dst = (size_t)it->second.u;
        }
    };
    auto meta_f = [&](const char* k2, const char* k1, float* dst) {
        for (const char* k : {k2, k1}) {
            auto it = g.meta.find(k);
            if (it != g.meta.end() && it->second.is_float) *dst = (float)it->second.f;
        }
    };
    auto has = [&](const std::string& n) { return g.tensors.count(n) > 0; };
    mivi_model_info c{};
    // config.rs:123-159 defaults, loader.rs:44-177 overrides
    c.dim = 1024; c.hidden_dim = 4608; c.n_layers = 16; c.n_heads = 16; c.n_kv_heads = 8;
    c.vocab_size = 65536; c.max_seq_len = 128000; c.rope_base = 1000000.0f; c.rms_norm_eps = 1e-5f;
    c.ssm_conv_kernel = 3;
    meta_u("lfm2.context_length", "lfm.context_length", &c.max_seq_len);
    meta_u("lfm2.embedding_length", "lfm.embedding_length", &c.dim);
    meta_u("lfm2.feed_forward_length", "lfm.feed_forward_length", &c.hidden_dim);
    meta_u("lfm2.block_count", "lfm.block_count", &c.n_layers);
    meta_u("lfm2.attention.head_count", "lfm.attention.head_count", &c.n_heads);
    for (const char* k : {"lfm2.attention.head_count_kv", "lfm.attention.head_count_kv"}) {
        auto it = g.meta.find(k);
        if (it == g.meta.end()) continue;
        if (it->second.is_array) {
            if (it->second.max_positive > 0) c.n_kv_heads = (size_t)it->second.max_positive;
        } else if (it->second.is_uint) {
            c.n_kv_heads = (size_t)it->second.u;
        }
    }
    meta_f("lfm2.rope.freq_base", "lfm.rope.freq_base", &c.rope_base);
    meta_f("lfm2.attention.layer_norm_rms_epsilon", "lfm.attention.layer_norm_rms_epsilon", &c.rms_norm_eps);
    meta_u("lfm2.ssm.conv_kernel", "lfm.ssm.conv_kernel", &c.ssm_conv_kernel);
    for (size_t i = 0; i < c.n_layers; i++) {
        std::string a = "blk." + std::to_string(i) + ".ssm_conv.weight";
        std::string b = "blk." + std::to_string(i) + ".shortconv.conv.weight";
        const GTensor* t = has(a) ? &g.tensors[a] : has(b) ? &g.tensors[b] : nullptr;
        if (t) {
            size_t tot = 1;
            for (size_t d : t->dims) tot *= d;
            if (c.dim > 0 && tot >= c.dim && tot % c.dim == 0) { c.ssm_conv_kernel = tot / c.dim; break; }
        }
    }
    {
        auto it = g.meta.find("tokenizer.ggml.tokens");
        if (it != g.meta.end() && it->second.is_array && it->second.n_strings > 0) c.vocab_size = it->second.n_strings;
    }
    c.head_dim = c.n_heads ? c.dim / c.n_heads : 64;
    c.kv_dim = c.n_kv_heads * c.head_dim;
    if (!c.dim || !c.n_heads || !c.n_kv_heads || c.dim % c.n_heads || c.n_heads % c.n_kv_heads || !c.n_layers)
        return model_error(MIVI_ERR_INVALID_CONFIG, "Invalid model configuration");
    size_t cap = max_ctx ? max_ctx : 16384;
    cap = std::min<size_t>(cap, 65536);
    c.max_seq_len = std::min(c.max_seq_len, cap);
    c.max_batch = max_batch;
    c.kv_precision = kv_precision;
    if (c.head_dim > kMaxHd || c.head_dim % 8 != 0)
        return model_error(MIVI_ERR_UNSUPPORTED, "head_dim %zu not supported (max %d, multiple of 8)", c.head_dim, kMaxHd);
    if (c.n_heads / c.n_kv_heads > 4)
        return model_error(MIVI_ERR_UNSUPPORTED, "more than 4 query heads per kv head");
    if (kv_precision == MIVI_KV_Q8_0 && c.head_dim % 32 != 0)
        return model_error(MIVI_ERR_UNSUPPORTED, "Q8_0 KV needs head_dim % 32 == 0");

    mivi_model* m = new mivi_model();
    auto fail = [&](int32_t code) { delete m; return code; };
    if (hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking) != hipSuccess)
        return fail(set_error(MIVI_ERR_HIP, "hipStreamCreate failed"));

    // weights: the tensor-data section, copied once
    size_t data_len = len - g.data_offset;
    if ((rc = m->alloc(&m->d_weights, data_len))) return fail(rc);
    if (hipMemcpy(m->d_weights, img + g.data_offset, data_len, hipMemcpyHostToDevice) != hipSuccess)
        return fail(set_error(MIVI_ERR_HIP, "weight upload failed"));
    c.weight_bytes = data_len;
    auto dev = [&](const GTensor& t) { return m->d_weights + (t.offset - g.data_offset); };

    // f32 vectors: F32 tensors are used in place; others are decoded once
    std::vector<std::pair<const GTensor*, const float**>> to_decode;
    size_t aux_len = 0;
    auto vec = [&](const std::string& name, const float** dst, size_t* n_out) -> bool {
        auto it = g.tensors.find(name);
        if (it == g.tensors.end()) return false;
        const GTensor& t = it->second;
        size_t ne = 1;
        for (size_t d : t.dims) ne *= d;
        if (n_out) *n_out = ne;
        if (t.type == MIVI_GGML_F32 && t.offset % 4 == 0) {
            *dst = (const float*)dev(t);
        } else {
            size_t bs, ts;
            if (!format_sizes(t.type, &bs, &ts)) return false;
            to_decode.push_back({&t, dst});
            aux_len += (ne + bs - 1) / bs * bs;
        }
        return true;
    };
    auto mat = [&](const std::string& name, Mat* dst) -> bool {
        auto it = g.tensors.find(name);
        if (it == g.tensors.end()) return false;
        const GTensor& t = it->second;
        dst->type = t.type;
        dst->w = dev(t);
        dst->cols = t.dims.empty() ? 0 : t.dims[0];
        dst->rows = t.dims.size() > 1 ? t.dims[1] : dst->cols;
        return true;
    };
    m->layers.resize(c.n_layers);
    int n_attn = 0;
    for (size_t i = 0; i < c.n_layers; i++) {
        Layer& L = m->layers[i];
        std::string p = "blk." + std::to_string(i) + ".";
        L.attn = !(has(p + "ssm_in.weight") || has(p + "shortconv.in_proj.weight") || has(p + "shortconv.conv.weight"));
        if (L.attn) {
            L.cache_idx = n_attn++;
            if (!vec(p + "attn_norm.weight", &L.norm, nullptr))
                return fail(model_error(MIVI_ERR_MISSING_WEIGHT, "Missing model weight: %sattn_norm.weight", p.c_str()));
            vec(p + "attn_q_norm.weight", &L.q_norm, nullptr);
            vec(p + "attn_k_norm.weight", &L.k_norm, nullptr);
            for (auto& nm : {std::make_pair("attn_q", &L.wq), std::make_pair("attn_k", &L.wk),
                             std::make_pair("attn_v", &L.wv), std::make_pair("attn_output", &L.wo)})
                if (!mat(p + nm.first + ".weight", nm.second))
                    return fail(model_error(MIVI_ERR_MISSING_WEIGHT, "Missing model weight: %s%s.weight", p.c_str(), nm.first));
        } else {
            if (!vec(p + "ssm_norm.weight", &L.norm, nullptr) && !vec(p + "attn_norm.weight", &L.norm, nullptr))
                return fail(model_error(MIVI_ERR_MISSING_WEIGHT, "Missing model weight: %sssm_norm.weight", p.c_str()));
            if (!mat(p + "ssm_in.weight", &L.in_proj) && !mat(p + "shortconv.in_proj.weight", &L.in_proj))
                return fail(model_error(MIVI_ERR_MISSING_WEIGHT, "Missing model weight: %sssm_in.weight", p.c_str()));
            if (!mat(p + "ssm_out.weight", &L.out_proj) && !mat(p + "shortconv.out_proj.weight", &L.out_proj))
                return fail(model_error(MIVI_ERR_MISSING_WEIGHT, "Missing model weight: %sssm_out.weight", p.c_str()));
            if (!vec(p + "ssm_conv.weight", &L.conv, &L.conv_len)) vec(p + "shortconv.conv.weight", &L.conv, &L.conv_len);
        }
        if (!vec(p + "ffn_norm.weight", &L.ffn_norm, nullptr) || !mat(p + "ffn_gate.weight", &L.gate) ||
            !mat(p + "ffn_up.weight", &L.up) || !mat(p + "ffn_down.weight", &L.down))
            return fail(model_error(MIVI_ERR_MISSING_WEIGHT, "Missing model weight: %sffn_*", p.c_str()));
    }
    c.n_attn_layers = (size_t)n_attn;
    if (!mat("token_embd.weight", &m->embd) && !mat("model.embed_tokens.weight", &m->embd))
        return fail(model_error(MIVI_ERR_MISSING_WEIGHT, "Missing model weight: token_embd.weight"));
    if (!vec("output_norm.weight", &m->out_norm, nullptr) && !vec("token_embd_norm.weight", &m->out_norm, nullptr))
        vec("token_embd_norm", &m->out_norm, nullptr);
    if (!mat("output.weight", &m->head) && !mat("lm_head.weight", &m->head)) m->head = m->embd;  // model.rs:455-459

    // every projection must be a format the GEMV runs, with matching shapes
    auto check = [&](const Mat& M, size_t rows, size_t cols, const char* what) -> int32_t {
        size_t bs, ts;
        if (!format_sizes(M.type, &bs, &ts)) return err_unsupported(M.type);
        if (cols % bs) return err_misaligned(cols, bs);
        size_t need = rows * (cols / bs) * ts;
        (void)what;
        if (M.rows * (M.cols / bs) * ts < need) return err_buffer_too_small(need, M.rows * (M.cols / bs) * ts);
        return MIVI_OK;
    };
    for (size_t i = 0; i < c.n_layers; i++) {
        const Layer& L = m->layers[i];
        if (L.attn) {
            if ((rc = check(L.wq, c.dim, c.dim, "q")) || (rc = check(L.wk, c.kv_dim, c.dim, "k")) ||
                (rc = check(L.wv, c.kv_dim, c.dim, "v")) || (rc = check(L.wo, c.dim, c.dim, "o")))
                return fail(rc);
        } else {
            if ((rc = check(L.in_proj, 3 * c.dim, c.dim, "in")) || (rc = check(L.out_proj, c.dim, c.dim, "out")))
                return fail(rc);
        }
        if ((rc = check(L.gate, c.hidden_dim, c.dim, "gate")) || (rc = check(L.up, c.hidden_dim, c.dim, "up")) ||
            (rc = check(L.down, c.dim, c.hidden_dim, "down")))
            return fail(rc);
    }
    if ((rc = check(m->head, c.vocab_size, c.dim, "head"))) return fail(rc);
    // the head GEMV streams the largest matrix: keep a packed copy of a Q6_K
    // head (the GGUF copy stays for the embedding lookup)
    if (m->head.type == MIVI_GGML_Q6_K && (c.dim == 2048 || c.dim == 4096 || c.dim == 8192) &&
        ((uintptr_t)m->head.w % 16) == 0 && !getenv("MIVI_NO_PACK")) {
        const size_t bytes = c.vocab_size * (c.dim / 256) * 210;
        if ((rc = m->alloc(&m->head_packed, bytes))) return fail(rc);
        if ((rc = launch_pack_q6k(m->head.w, m->head_packed, c.vocab_size, c.dim, nullptr))) return fail(rc);
        if (hipDeviceSynchronize() != hipSuccess) return fail(set_error(MIVI_ERR_HIP, "packing the head failed"));
        c.weight_bytes += bytes;
        // batched steps read the head once for up to eight sequences on the
        // 32 x 32 x 16 int8 matrix instruction (same results bit for bit)
        if (max_batch > 1 && t32_layout(c.vocab_size, c.dim) && !getenv("MIVI_NO_HEAD_T32")) {
            if ((rc = m->alloc(&m->head_t32, bytes))) return fail(rc);
            if ((rc = launch_pack_q6k_t32(m->head.w, m->head_t32, c.vocab_size, c.dim, nullptr))) return fail(rc);
            if (hipDeviceSynchronize() != hipSuccess)
                return fail(set_error(MIVI_ERR_HIP, "packing the batched head failed"));
            c.weight_bytes += bytes;
        }
    }
    // one-column decode GEMVs stream the projections packed (bit-identical
    // to the GGUF rows): Q4_K as row quads (matrix cores), Q6_K (the
    // attn_v / ffn_down of a Q4_K_M file) as row quads at 2048 columns and
    // unit planes at 4096 or 8192; a packed copy of each, the GGUF rows
    // staying for the batched and prefill products
    if (!getenv("MIVI_NO_PACK")) {
        std::vector<Mat*> qm;
        for (size_t i = 0; i < c.n_layers; i++) {
            Layer& L = m->layers[i];
            Mat* all[] = {&L.wq, &L.wk, &L.wv, &L.wo, &L.in_proj, &L.out_proj, &L.gate, &L.up, &L.down};
            for (Mat* x : all)
                if (x->w && (uintptr_t)x->w % 16 == 0 &&
                    ((x->type == MIVI_GGML_Q4_K && q4k_quad_layout(x->rows, x->cols)) ||
                     (x->type == MIVI_GGML_Q6_K && (x->cols == 2048 || x->cols == 4096 || x->cols == 8192))))
                    qm.push_back(x);
        }
        auto bytes = [](const Mat* x) { return x->rows * (x->cols / 256) * (x->type == MIVI_GGML_Q6_K ? 210 : 144); };
        size_t total = 0;
        for (Mat* x : qm) total += bytes(x);  // each a multiple of 16 bytes
        uint8_t* q = nullptr;
        if (total && (rc = m->alloc(&q, total))) return fail(rc);
        for (Mat* x : qm) {
            rc = x->type == MIVI_GGML_Q6_K ? launch_pack_q6k(x->w, q, x->rows, x->cols, nullptr)
                                           : launch_pack_q4k(x->w, q, x->rows, x->cols, nullptr);
            if (rc) return fail(rc);
            x->quad = q;
            q += bytes(x);
        }
        if (total && hipDeviceSynchronize() != hipSuccess)
            return fail(set_error(MIVI_ERR_HIP, "packing the projections failed"));
        c.weight_bytes += total;
    }
    // batched decode GEMVs (max_batch > 1) stream each all-Q4_K projection
    // launch packed in the column kernel's group order: one more copy of
    // those rows (not with MIVI_NO_PACK or MIVI_NO_COLS_PACK)
    if (!getenv("MIVI_NO_PACK") && !getenv("MIVI_NO_COLS_PACK") && max_batch > 1) {
        struct Job {
            const uint8_t** dst;
            std::vector<const Mat*> ms;
            int epi;
        };
        std::vector<Job> jobs;
        auto q4 = [](const Mat& x) { return x.w && x.type == MIVI_GGML_Q4_K && x.cols % 256 == 0; };
        for (size_t i = 0; i < c.n_layers; i++) {
            Layer& L = m->layers[i];
            if (L.attn) {
                if (q4(L.wq) && q4(L.wk) && q4(L.wv)) jobs.push_back({&L.cw_qkv, {&L.wq, &L.wk, &L.wv}, EPI_STORE});
                if (q4(L.wo)) jobs.push_back({&L.cw_o, {&L.wo}, EPI_STORE});
            } else {
                if (q4(L.in_proj)) jobs.push_back({&L.cw_in, {&L.in_proj}, EPI_CONV});
                if (q4(L.out_proj)) jobs.push_back({&L.cw_o, {&L.out_proj}, EPI_STORE});
            }
            if (q4(L.gate) && q4(L.up) && L.gate.rows == L.up.rows) jobs.push_back({&L.cw_gu, {&L.gate, &L.up}, EPI_SWIGLU});
            if (q4(L.down)) jobs.push_back({&L.cw_down, {&L.down}, EPI_STORE});
        }
        auto groups = [](const Job& j) {
            size_t n = 0;
            for (const Mat* x : j.ms) n += x->rows;
            return cols_groups(j.epi, (int)j.ms[0]->rows, (int)n);
        };
        size_t total = 0;
        for (const Job& j : jobs) total += (size_t)groups(j) * (j.ms[0]->cols / 256) * kColsChunkBytes;
        uint8_t* q = nullptr;
        if (total && (rc = m->alloc(&q, total))) return fail(rc);
        std::vector<const uint8_t*> rows;
        for (const Job& j : jobs) {
            const int ng = groups(j), n0 = (int)j.ms[0]->rows;
            int n = 0;
            for (const Mat* x : j.ms) n += (int)x->rows;
            const size_t rb = j.ms[0]->cols / 256 * 144;
            rows.assign((size_t)ng * 16, nullptr);
            for (int grp = 0; grp < ng; grp++)
                for (int jj = 0; jj < 16; jj++) {
                    int r = cols_group_row(j.epi, grp, jj, n0, n);
                    r = r < 0 ? 0 : r;  // (its lanes store nothing)
                    size_t k = 0;
                    while (r >= (int)j.ms[k]->rows) r -= (int)j.ms[k++]->rows;
                    rows[(size_t)grp * 16 + jj] = j.ms[k]->w + (size_t)r * rb;
                }
            if ((rc = launch_pack_q4k_cols(rows.data(), ng, j.ms[0]->cols, q, nullptr))) return fail(rc);
            *j.dst = q;
            q += (size_t)ng * (j.ms[0]->cols / 256) * kColsChunkBytes;
        }
        c.weight_bytes += total;
    }
    // the chunked prefill's row products (tiles of 16+ rows) read each Q4_K
    // projection's B operand converted once, sc * q in fp16 in MFMA operand
    // order (3.6x the Q4_K bytes; not with MIVI_NO_PACK or MIVI_NO_GEMM_PACK)
    if (!getenv("MIVI_NO_PACK") && !getenv("MIVI_NO_GEMM_PACK")) {
        std::vector<Mat*> gm;
        for (size_t i = 0; i < c.n_layers; i++) {
            Layer& L = m->layers[i];
            Mat* all[] = {&L.wq, &L.wk, &L.wv, &L.wo, &L.in_proj, &L.out_proj, &L.gate, &L.up, &L.down};
            for (Mat* x : all)
                if (x->w && x->type == MIVI_GGML_Q4_K && x->rows % 32 == 0 && x->cols % 2048 == 0 &&
                    (uintptr_t)x->w % 16 == 0)
                    gm.push_back(x);
        }
        size_t total = 0;
        for (Mat* x : gm) total += q4k_gemm_packed_bytes(x->rows, x->cols);  // multiples of 128 bytes
        uint8_t* q = nullptr;
        if (total && (rc = m->alloc(&q, total))) return fail(rc);
        for (Mat* x : gm) {
            if ((rc = launch_pack_q4k_gemm(x->w, q, x->rows, x->cols, nullptr))) return fail(rc);
            x->gemm = q;
            q += q4k_gemm_packed_bytes(x->rows, x->cols);
        }
        if (total && hipDeviceSynchronize() != hipSuccess)
            return fail(set_error(MIVI_ERR_HIP, "packing the projections for the row products failed"));
        c.weight_bytes += total;
    }
    {
        size_t bs, ts;
        if (!format_sizes(m->embd.type, &bs, &ts) || c.dim % bs) return fail(err_unsupported(m->embd.type));
        // every token id below vocab_size must have a row (model.rs:357-364)
        if (m->embd.rows < c.vocab_size || m->embd.cols != c.dim)
            return fail(model_error(MIVI_ERR_INVALID_CONFIG, "token_embd is %zux%zu, vocab %zu x dim %zu",
                                    m->embd.rows, m->embd.cols, c.vocab_size, c.dim));
    }

    // decode non-F32 vectors
    if (aux_len) {
        if ((rc = m->alloc(&m->d_aux, aux_len))) return fail(rc);
        size_t off = 0;
        for (auto& td : to_decode) {
            const GTensor& t = *td.first;
            size_t bs, ts, ne = 1;
            format_sizes(t.type, &bs, &ts);
            for (size_t d : t.dims) ne *= d;
            size_t count = bs == 1 ? ne : (ne + bs - 1) / bs;
            if ((rc = launch_dequant(t.type, dev(t), m->d_aux + off, count, m->stream))) return fail(rc);
            *td.second = m->d_aux + off;
            off += (ne + bs - 1) / bs * bs;
        }
    }

    // RoPE table (model.rs:194-212)
    c.yarn = c.max_seq_len > 4096;
    c.yarn_scale = c.yarn ? (float)c.max_seq_len / 4096.0f : 1.0f;
    {
        std::vector<float> cs, sn;
        host_rope_table(cs, sn, c.head_dim, c.max_seq_len, c.rope_base, c.yarn, c.yarn_scale);
        if ((rc = m->alloc(&m->rope_cos, cs.size())) || (rc = m->alloc(&m->rope_sin, sn.size()))) return fail(rc);
        hipError_t e = hipMemcpyAsync(m->rope_cos, cs.data(), cs.size() * 4, hipMemcpyHostToDevice, m->stream);
        if (e == hipSuccess) e = hipMemcpyAsync(m->rope_sin, sn.data(), sn.size() * 4, hipMemcpyHostToDevice, m->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(m->stream);
        if (e != hipSuccess) return fail(set_error(MIVI_ERR_HIP, "uploading the RoPE table failed: %s", hipGetErrorString(e)));
    }

    // run state, KV caches
    m->kv_row_bytes = kv_precision == MIVI_KV_Q8_0 ? (c.kv_dim / 32) * 34
                    : kv_precision == MIVI_KV_F16 ? c.kv_dim * 2 : c.kv_dim * 4;
    m->kv_packed = attn_q8_mfma_ok(kv_precision, (int)c.head_dim, (int)c.n_heads, (int)c.n_kv_heads);
    // the group layout holds whole 16-token groups
    m->kv_layer_bytes = (m->kv_packed ? (c.max_seq_len + 15) / 16 * 16 : c.max_seq_len) * m->kv_row_bytes;
    // about two workgroups per CU over all kv heads (each split loops over
    // ceil(tiles / nsplit) tiles)
    const size_t tt = (size_t)attn_tile_tokens(c.head_dim);
    const size_t want = std::max<size_t>(1, 2 * (size_t)num_cus() / std::max<size_t>(1, c.n_kv_heads));
    m->nsplit = (int)std::max<size_t>(1, std::min((c.max_seq_len + tt - 1) / tt, want));
    size_t ks = std::max<size_t>(1, c.ssm_conv_kernel);
    // Per-sequence vectors live in one arena per kind, sequence b at
    // base + b * stride, so a batched GEMV addresses every sequence's
    // activations and outputs with one stride (q|k|v share one slot).
    m->seqs.resize(max_batch);
    {
        SeqStrides& z = m->strides;
        z.x = c.dim; z.sc_in = 3 * c.dim; z.hb = c.hidden_dim; z.qkv = c.dim + 2 * c.kv_dim;
        z.logits = c.vocab_size; z.conv = c.n_layers * c.dim * ks; z.parts = kMaxArgmaxParts;
        const size_t B = max_batch;
        float *x, *sc_in, *hb, *hb2, *qkv, *ao, *lg, *ca, *cb, *pv;
        int* pi;
        if ((rc = m->alloc(&x, B * z.x)) || (rc = m->alloc(&sc_in, B * z.sc_in)) || (rc = m->alloc(&hb, B * z.hb)) ||
            (rc = m->alloc(&hb2, B * z.hb)) || (rc = m->alloc(&qkv, B * z.qkv)) || (rc = m->alloc(&ao, B * z.x)) ||
            (rc = m->alloc(&lg, B * z.logits)) || (rc = m->alloc(&ca, B * z.conv)) || (rc = m->alloc(&cb, B * z.conv)) ||
            (rc = m->alloc(&pv, B * z.parts)) || (rc = m->alloc(&pi, B * z.parts)))
            return fail(rc);
        for (size_t b = 0; b < B; b++) {
            SeqState& st = m->seqs[b];
            st.x = x + b * z.x; st.sc_in = sc_in + b * z.sc_in;
            st.hb = hb + b * z.hb; st.hb2 = hb2 + b * z.hb;
            st.q = qkv + b * z.qkv; st.k = st.q + c.dim; st.v = st.k + c.kv_dim;
            st.attn_out = ao + b * z.x; st.logits = lg + b * z.logits;
            st.conv_a = ca + b * z.conv; st.conv_b = cb + b * z.conv;
            st.part_val = pv + b * z.parts; st.part_idx = pi + b * z.parts;
        }
    }
    {
        SeqStrides& z = m->strides;
        z.kv = c.n_attn_layers * m->kv_layer_bytes;
        z.part = c.n_heads * m->nsplit;
        const size_t B = max_batch;
        float *pm, *pl, *pa;
        uint8_t *kc, *vc;
        if ((rc = m->alloc(&pm, B * z.part)) || (rc = m->alloc(&pl, B * z.part)) ||
            (rc = m->alloc(&pa, B * z.part * c.head_dim)) || (rc = m->alloc(&kc, B * z.kv)) ||
            (rc = m->alloc(&vc, B * z.kv)))
            return fail(rc);
        for (size_t b = 0; b < B; b++) {
            SeqState& st = m->seqs[b];
            st.part_m = pm + b * z.part; st.part_l = pl + b * z.part; st.part_acc = pa + b * z.part * c.head_dim;
            st.kc = kc + b * z.kv; st.vc = vc + b * z.kv;
        }
    }
    c.kv_bytes = 2 * max_batch * m->strides.kv;
    if ((rc = m->alloc(&m->ctrl, 1)) || (rc = m->alloc(&m->history, c.max_seq_len * max_batch)) ||
        (rc = m->alloc(&m->rng, max_batch)) ||
        (rc = m->alloc(&m->samp_ws, sample_seq_workspace(c.vocab_size, max_batch))))
        return fail(rc);
    if (hipStreamSynchronize(m->stream) != hipSuccess || hipDeviceSynchronize() != hipSuccess)
        return fail(set_error(MIVI_ERR_HIP, "model setup failed"));
    m->info = c;
    *out = m;
    return clear_error();
}

extern "C" void mivi_hip_model_destroy(mivi_model* m) { delete m; }

extern "C" int32_t mivi_hip_model_info(const mivi_model* m, mivi_model_info* out) {
    if (!m || !out) return set_error(MIVI_ERR_INVALID_ARGUMENT, "null argument");
    *out = m->info;
    return MIVI_OK;
}

extern "C" int32_t mivi_hip_model_reset(mivi_model* m) {
    if (!m) return set_error(MIVI_ERR_INVALID_ARGUMENT, "null model");
    // arena.rs:90-108 clears the run state; cache.rs:287-289 only rewinds
    const mivi_model_info& c = m->info;
    size_t ks = std::max<size_t>(1, c.ssm_conv_kernel);
    for (auto& st : m->seqs) {
        MIVI_HIP_CHECK(hipMemsetAsync(st.x, 0, c.dim * 4, m->stream));
        MIVI_HIP_CHECK(hipMemsetAsync(st.conv_a, 0, c.n_layers * c.dim * ks * 4, m->stream));
        MIVI_HIP_CHECK(hipMemsetAsync(st.conv_b, 0, c.n_layers * c.dim * ks * 4, m->stream));
        MIVI_HIP_CHECK(hipMemsetAsync(st.logits, 0, c.vocab_size * 4, m->stream));
    }
    MIVI_HIP_CHECK(hipMemsetAsync(m->ctrl, 0, sizeof(Ctrl), m->stream));
    MIVI_HIP_CHECK(hipStreamSynchronize(m->stream));
    return clear_error();
}

static int32_t check_tok_pos(mivi_model* m, uint32_t token, size_t pos) {
    if ((size_t)token >= m->info.vocab_size)
        return set_error(MIVI_ERR_INVALID_TOKEN, "Invalid token ID: %u", token);  // model.rs:342-344
    if (pos >= m->info.max_seq_len)
        return set_error(MIVI_ERR_CONTEXT_OVERFLOW, "Context overflow: current pos %zu >= max_seq_len %zu", pos,
                         m->info.max_seq_len);  // model.rs:345-350
    return MIVI_OK;
}

static int32_t set_ctrl(mivi_model* m, size_t seq, uint32_t token, size_t pos) {
    // the phase counter keeps running; only token and position are set
    hipLaunchKernelGGL(set_ctrl_kernel, dim3(1), dim3(1), 0, m->stream, &m->ctrl->tok[seq], &m->ctrl->pos[seq],
                       &m->ctrl->pos0[seq],
                       token, (int)pos);
    MIVI_HIP_CHECK(hipGetLastError());
    return MIVI_OK;
}

extern "C" int32_t mivi_hip_model_forward_step(mivi_model* m, size_t seq, uint32_t token, size_t pos,
                                               int32_t compute_logits, float* logits_host) {
    if (!m || seq >= m->info.max_batch) return set_error(MIVI_ERR_INVALID_ARGUMENT, "bad model or sequence");
    int32_t rc = check_tok_pos(m, token, pos);
    if (rc) return rc;
    if ((rc = set_ctrl(m, seq, token, pos))) return rc;
    if ((rc = enqueue_step(m, seq, compute_logits != 0, false, m->stream))) return rc;
    if (compute_logits && logits_host)
        MIVI_HIP_CHECK(hipMemcpyAsync(logits_host, m->seqs[seq].logits, m->info.vocab_size * 4,
                                      hipMemcpyDeviceToHost, m->stream));
    MIVI_HIP_CHECK(hipStreamSynchronize(m->stream));
    return clear_error();
}

extern "C" int32_t mivi_hip_model_forward(mivi_model* m, size_t seq, uint32_t token, size_t pos, float* logits) {
    return mivi_hip_model_forward_step(m, seq, token, pos, 1, logits);
}

// Model::forward (model.rs:488-491) of sequences 0..batch-1 in one batched
// step: the kernels of the batched decode (every projection one GEMV over the
// batch's columns, one attention launch with the batch's split count), the
// head storing logits.
extern "C" int32_t mivi_hip_model_forward_batch(mivi_model* m, size_t batch, const uint32_t* tokens,
                                                const size_t* pos, float* logits_host) {
    if (!m || batch == 0 || batch > m->info.max_batch || !tokens || !pos)
        return set_error(MIVI_ERR_INVALID_ARGUMENT, "bad argument");
    for (size_t b = 0; b < batch; b++) {
        int32_t rc = check_tok_pos(m, tokens[b], pos[b]);
        if (rc) return rc;
    }
    for (size_t b = 0; b < batch; b++) {
        int32_t rc = set_ctrl(m, b, tokens[b], pos[b]);
        if (rc) return rc;
    }
    int32_t rc = enqueue_step(m, 0, batch, true, false, m->stream, true, 0, m->info.n_layers, true, false);
    if (rc) return rc;
    if (logits_host)
        MIVI_HIP_CHECK(hipMemcpy2DAsync(logits_host, m->info.vocab_size * 4, m->seqs[0].logits,
                                        m->strides.logits * 4, m->info.vocab_size * 4, batch,
                                        hipMemcpyDeviceToHost, m->stream));
    MIVI_HIP_CHECK(hipStreamSynchronize(m->stream));
    return clear_error();
}

extern "C" int32_t mivi_hip_model_set_prefill_tile(mivi_model* m, size_t tile_tokens) {
    if (!m) return set_error(MIVI_ERR_INVALID_ARGUMENT, "null model");
    if (tile_tokens > 4096) return set_error(MIVI_ERR_INVALID_ARGUMENT, "prefill tile of %zu tokens (at most 4096)", tile_tokens);
    // ssm.rs:174-300 walks windows of at most 8 taps here
    m->prefill_tile = m->info.ssm_conv_kernel > 8 ? 0 : tile_tokens;
    return clear_error();
}

extern "C" int32_t mivi_hip_model_prefill(mivi_model* m, size_t seq, const uint32_t* tokens, size_t n, size_t pos0) {
    if (!m || seq >= m->info.max_batch || (n && !tokens)) return set_error(MIVI_ERR_INVALID_ARGUMENT, "bad argument");
    for (size_t i = 0; i < n; i++) {
        int32_t rc = check_tok_pos(m, tokens[i], pos0 + i);
        if (rc) return rc;
    }
    if (m->prefill_tile > 1 && n > 1) {
        // chunked: tiles of prefill_tile rows (model.rs:676-831)
        const size_t tile = std::min(m->prefill_tile, n);
        int32_t rc = prefill_buffers(m, tile);
        if (rc) return rc;
        for (size_t c0 = 0; c0 < n; c0 += tile) {
            const size_t rows = std::min(tile, n - c0);
            MIVI_HIP_CHECK(hipMemcpyAsync(m->pf_tok, tokens + c0, rows * 4, hipMemcpyHostToDevice, m->stream));
            if ((rc = enqueue_prefill_tile(m, seq, pos0 + c0, rows, m->stream))) return rc;
            // the host token array is read by the copy above before it returns
            MIVI_HIP_CHECK(hipStreamSynchronize(m->stream));
        }
        return clear_error();
    }
    for (size_t i = 0; i < n; i++) {
        int32_t rc = set_ctrl(m, seq, tokens[i], pos0 + i);
        if (rc) return rc;
        if ((rc = enqueue_step(m, seq, false, false, m->stream))) return rc;
        if ((i & 255) == 255) MIVI_HIP_CHECK(hipStreamSynchronize(m->stream));
    }
    MIVI_HIP_CHECK(hipStreamSynchronize(m->stream));
    return clear_error();
}

extern "C" int32_t mivi_hip_model_generate_greedy(mivi_model* m, size_t batch, const uint32_t* tokens,
                                                  const size_t* pos, size_t n_steps, uint32_t* tokens_out) {
    if (!m || batch == 0 || batch > m->info.max_batch || !tokens || !pos || (n_steps && !tokens_out))
        return set_error(MIVI_ERR_INVALID_ARGUMENT, "bad argument");
    for (size_t b = 0; b < batch; b++) {
        int32_t rc = check_tok_pos(m, tokens[b], pos[b]);
        if (rc) return rc;
        if (pos[b] + n_steps > m->info.max_seq_len)
            return set_error(MIVI_ERR_CONTEXT_OVERFLOW, "Context overflow: current pos %zu >= max_seq_len %zu",
                             pos[b] + n_steps - 1, m->info.max_seq_len);
    }
    if (n_steps == 0) return clear_error();
    for (size_t b = 0; b < batch; b++) {
        int32_t rc = set_ctrl(m, b, tokens[b], pos[b]);  // (pos0: the step index is pos - pos0)
        if (rc) return rc;
    }
    {
        // the first step's embeddings; each step embeds the next tokens itself
        const EmbedNext en = embed_next_args(m, m->seqs[0].x, true);
        hipLaunchKernelGGL(embed_kernel, dim3((unsigned)batch), dim3(kWG), 0, m->stream, en.type, en.table,
                           en.row_bytes, &m->ctrl->tok[0], en.x, en.dim, en.xs);
    }
    if (!m->graph || m->graph_batch != batch) {
        if (m->graph) {
            hipGraphExecDestroy(m->graph);
            m->graph = nullptr;
        }
        hipGraph_t gr;
        MIVI_HIP_CHECK(hipStreamBeginCapture(m->stream, hipStreamCaptureModeThreadLocal));
        int32_t rc = MIVI_OK;
        rc = enqueue_batch_step(m, batch, m->stream);
        hipError_t e = hipStreamEndCapture(m->stream, &gr);
        if (rc) return rc;
        if (e != hipSuccess) return set_error(MIVI_ERR_HIP, "graph capture failed: %s", hipGetErrorString(e));
        e = hipGraphInstantiate(&m->graph, gr, nullptr, nullptr, 0);
        hipGraphDestroy(gr);
        if (e != hipSuccess) return set_error(MIVI_ERR_HIP, "graph instantiate failed: %s", hipGetErrorString(e));
        m->graph_batch = batch;
    }
    for (size_t i = 0; i < n_steps; i++) MIVI_HIP_CHECK(hipGraphLaunch(m->graph, m->stream));
    std::vector<uint32_t> hist(n_steps * m->info.max_batch);
    MIVI_HIP_CHECK(hipMemcpyAsync(hist.data(), m->history, hist.size() * 4, hipMemcpyDeviceToHost, m->stream));
    MIVI_HIP_CHECK(hipStreamSynchronize(m->stream));
    for (size_t i = 0; i < n_steps; i++)
        for (size_t b = 0; b < batch; b++) tokens_out[i * batch + b] = hist[i * m->info.max_batch + b];
    return clear_error();
}

// The generation loop of model.rs:1130-1180 with Sampler::sample on the
// device: each step runs the decode step of the batch and samples every
// sequence's next token from its logits (penalty window = its last 64
// generated tokens, RECENT_TOKENS_WINDOW, config.rs:11; the end-of-sequence
// ids suppressed on the first token). Stopping at an end-of-sequence token
// is the caller's: all n_steps tokens are produced.
extern "C" int32_t mivi_hip_model_generate(mivi_model* m, size_t batch, const uint32_t* tokens, const size_t* pos,
                                           size_t n_steps, const mivi_sampler_config* cfg, const uint64_t* seeds,
                                           const uint32_t* eos_ids, size_t n_eos, uint32_t* tokens_out) {
    if (!m || batch == 0 || batch > m->info.max_batch || !tokens || !pos || !cfg || !seeds ||
        (n_steps && !tokens_out) || (n_eos && !eos_ids) || n_eos > 4)
        return set_error(MIVI_ERR_INVALID_ARGUMENT, "bad argument");
    for (size_t b = 0; b < batch; b++) {
        int32_t rc = check_tok_pos(m, tokens[b], pos[b]);
        if (rc) return rc;
        if (pos[b] + n_steps > m->info.max_seq_len)
            return set_error(MIVI_ERR_CONTEXT_OVERFLOW, "Context overflow: current pos %zu >= max_seq_len %zu",
                             pos[b] + n_steps - 1, m->info.max_seq_len);
    }
    if (n_steps == 0) return clear_error();
    for (size_t b = 0; b < batch; b++) {
        int32_t rc = set_ctrl(m, b, tokens[b], pos[b]);
        if (rc) return rc;
    }
    // Sampler::with_seed / set_seed (sampler.rs:28-57): seed 0 -> FALLBACK_RNG_SEED
    std::vector<uint64_t> st(batch);
    for (size_t b = 0; b < batch; b++) st[b] = seeds[b] ? seeds[b] : 0x853c49e6748fea9bULL;
    MIVI_HIP_CHECK(hipMemcpyAsync(m->rng, st.data(), batch * 8, hipMemcpyHostToDevice, m->stream));
    hipLaunchKernelGGL(set_int_kernel, dim3(1), dim3(1), 0, m->stream, &m->ctrl->step, 0);
    {
        const EmbedNext en = embed_next_args(m, m->seqs[0].x, true);
        hipLaunchKernelGGL(embed_kernel, dim3((unsigned)batch), dim3(kWG), 0, m->stream, en.type, en.table,
                           en.row_bytes, &m->ctrl->tok[0], en.x, en.dim, en.xs);
    }
    SampleEos eos{};
    eos.n = (int)n_eos;
    for (size_t i = 0; i < n_eos; i++) eos.id[i] = eos_ids[i];
    if (!m->graph_s || m->graph_s_batch != batch || memcmp(&m->graph_s_cfg, cfg, sizeof(*cfg)) ||
        memcmp(&m->graph_s_eos, &eos, sizeof(eos))) {
        if (m->graph_s) {
            hipGraphExecDestroy(m->graph_s);
            m->graph_s = nullptr;
        }
        const mivi_model_info& c = m->info;
        hipGraph_t gr;
        MIVI_HIP_CHECK(hipStreamBeginCapture(m->stream, hipStreamCaptureModeThreadLocal));
        // x holds the tokens' embeddings when a step starts: the first step's
        // come from the launch below, each step's sampler embeds the next
        int32_t rc = enqueue_step(m, 0, batch, true, false, m->stream, false, 0, c.n_layers, true, false);
        if (!rc)
            rc = launch_sample_seq(m->seqs[0].logits, (int64_t)m->strides.logits, (int)c.vocab_size, m->history,
                                   (int)c.max_batch, 0, (int)batch, 64, &m->ctrl->step, eos, *cfg, m->rng,
                                   &m->ctrl->tok[0], m->samp_ws, embed_next_args(m, m->seqs[0].x, true), m->stream);
        if (!rc) hipLaunchKernelGGL(step_counter_kernel, dim3(1), dim3(1), 0, m->stream, &m->ctrl->step);
        hipError_t e = hipStreamEndCapture(m->stream, &gr);
        if (rc) return rc;
        if (e != hipSuccess) return set_error(MIVI_ERR_HIP, "graph capture failed: %s", hipGetErrorString(e));
        e = hipGraphInstantiate(&m->graph_s, gr, nullptr, nullptr, 0);
        hipGraphDestroy(gr);
        if (e != hipSuccess) return set_error(MIVI_ERR_HIP, "graph instantiate failed: %s", hipGetErrorString(e));
        m->graph_s_batch = batch;
        m->graph_s_cfg = *cfg;
        m->graph_s_eos = eos;
    }
    for (size_t i = 0; i < n_steps; i++) MIVI_HIP_CHECK(hipGraphLaunch(m->graph_s, m->stream));
    std::vector<uint32_t> hist(n_steps * m->info.max_batch);
    MIVI_HIP_CHECK(hipMemcpyAsync(hist.data(), m->history, hist.size() * 4, hipMemcpyDeviceToHost, m->stream));
    MIVI_HIP_CHECK(hipStreamSynchronize(m->stream));
    for (size_t i = 0; i < n_steps; i++)
        for (size_t b = 0; b < batch; b++) tokens_out[i * batch + b] = hist[i * m->info.max_batch + b];
    return clear_error();
}

// One layer's Q8_0 cache between the reference's rows (tokens x n_kv x 68
// bytes: per kv head two blocks of f16 scale + 32 quants) and the q8g_* group
// layout. `groups` holds whole groups starting with the one that contains
// the first row's position; p0 = that position mod 16. Bytes of positions
// outside the rows are left as they are.
static void q8_rows_to_groups(const uint8_t* rows, size_t p0, size_t tokens, int n_kv, bool is_v, uint8_t* groups) {
    const size_t rb = (size_t)n_kv * 68;
    for (size_t p = 0; p < tokens; p++) {
        const size_t r = p0 + p;
        const int t = (int)(r % 16);
        for (int h = 0; h < n_kv; h++) {
            const uint8_t* src = rows + p * rb + (size_t)h * 68;
            uint8_t* g = groups + q8g_base(r, h, n_kv);
            for (int b = 0; b < 2; b++) {
                memcpy(g + q8g_d_off(t, b), src + 34 * b, 2);
                for (int i = 0; i < 32; i++) g[is_v ? q8g_v_off(t, 32 * b + i) : q8g_k_off(t, 32 * b + i)] = src[34 * b + 2 + i];
            }
        }
    }
}
static void q8_groups_to_rows(const uint8_t* groups, size_t p0, size_t tokens, int n_kv, bool is_v, uint8_t* rows) {
    const size_t rb = (size_t)n_kv * 68;
    for (size_t p = 0; p < tokens; p++) {
        const size_t r = p0 + p;
        const int t = (int)(r % 16);
        for (int h = 0; h < n_kv; h++) {
            uint8_t* dst = rows + p * rb + (size_t)h * 68;
            const uint8_t* g = groups + q8g_base(r, h, n_kv);
            for (int b = 0; b < 2; b++) {
                memcpy(dst + 34 * b, g + q8g_d_off(t, b), 2);
                for (int i = 0; i < 32; i++) dst[34 * b + 2 + i] = g[is_v ? q8g_v_off(t, 32 * b + i) : q8g_k_off(t, 32 * b + i)];
            }
        }
    }
}

static size_t conv_state_len(const mivi_model* m) {
    return m->info.n_layers * m->info.dim * std::max<size_t>(1, m->info.ssm_conv_kernel);
}

// KvError::ContextOverflow of an interval [start, start + tokens)
// (cache.rs:692-697, :834-839)
static int32_t kv_interval_check(mivi_model* m, size_t seq, size_t start, size_t tokens) {
    if (!m || seq >= m->info.max_batch) return set_error(MIVI_ERR_INVALID_ARGUMENT, "bad model or sequence");
    const size_t mx = m->info.max_seq_len;
    if (start > mx || tokens > mx - start)
        return set_error(MIVI_ERR_KV_CACHE, "KV cache error: Context length exceeded: attempted pos %zu >= max_seq_len %zu",
                         start > mx ? start : start + tokens, mx);
    return MIVI_OK;
}

// K and V rows of positions [start, start + tokens) of every attention layer
// of sequence seq, to host buffers laid out [n_attn_layers, tokens, row]
// (cache.rs:688-746). The Q8_0 group layout goes through the host as the
// whole groups covering the interval.
static int32_t kv_rows_out(mivi_model* m, size_t seq, size_t start, size_t tokens, void* k_out, void* v_out) {
    const mivi_model_info& c = m->info;
    SeqState& st = m->seqs[seq];
    const size_t lb = m->kv_layer_bytes, rb = m->kv_row_bytes, tb = tokens * rb;
    if (tokens == 0) return MIVI_OK;
    if (m->kv_packed) {
        const int nkv = (int)c.n_kv_heads;
        const size_t g0 = start / 16, g1 = (start + tokens + 15) / 16, gb = (g1 - g0) * 16 * rb;
        std::vector<uint8_t> kg(gb), vg(gb);
        for (size_t l = 0; l < c.n_attn_layers; l++) {
            MIVI_HIP_CHECK(hipMemcpyAsync(kg.data(), st.kc + l * lb + g0 * 16 * rb, gb, hipMemcpyDeviceToHost, m->stream));
            MIVI_HIP_CHECK(hipMemcpyAsync(vg.data(), st.vc + l * lb + g0 * 16 * rb, gb, hipMemcpyDeviceToHost, m->stream));
            MIVI_HIP_CHECK(hipStreamSynchronize(m->stream));
            q8_groups_to_rows(kg.data(), start % 16, tokens, nkv, false, (uint8_t*)k_out + l * tb);
            q8_groups_to_rows(vg.data(), start % 16, tokens, nkv, true, (uint8_t*)v_out + l * tb);
        }
        return MIVI_OK;
    }
    for (size_t l = 0; l < c.n_attn_layers; l++) {
        MIVI_HIP_CHECK(hipMemcpyAsync((uint8_t*)k_out + l * tb, st.kc + l * lb + start * rb, tb, hipMemcpyDeviceToHost,
                                      m->stream));
        MIVI_HIP_CHECK(hipMemcpyAsync((uint8_t*)v_out + l * tb, st.vc + l * lb + start * rb, tb, hipMemcpyDeviceToHost,
                                      m->stream));
    }
    MIVI_HIP_CHECK(hipStreamSynchronize(m->stream));
    return MIVI_OK;
}

// The host rows of an interval export into positions [start, start +
// tokens) of sequence seq's caches, other positions untouched
// (cache.rs:827-914). In the Q8_0 group layout, groups only partly inside
// the interval are read back first and rewritten whole.
static int32_t kv_rows_in(mivi_model* m, size_t seq, size_t start, size_t tokens, const void* k_in, const void* v_in) {
    const mivi_model_info& c = m->info;
    SeqState& st = m->seqs[seq];
    const size_t lb = m->kv_layer_bytes, rb = m->kv_row_bytes, tb = tokens * rb;
    if (tokens == 0) return MIVI_OK;
    if (m->kv_packed) {
        const int nkv = (int)c.n_kv_heads;
        const size_t g0 = start / 16, g1 = (start + tokens + 15) / 16, gb = (g1 - g0) * 16 * rb;
        const bool partial = (start % 16) != 0 || ((start + tokens) % 16) != 0;
        std::vector<uint8_t> kg(gb, 0), vg(gb, 0);
        for (size_t l = 0; l < c.n_attn_layers; l++) {
            uint8_t* kd = st.kc + l * lb + g0 * 16 * rb;
            uint8_t* vd = st.vc + l * lb + g0 * 16 * rb;
            if (partial) {
                MIVI_HIP_CHECK(hipMemcpyAsync(kg.data(), kd, gb, hipMemcpyDeviceToHost, m->stream));
                MIVI_HIP_CHECK(hipMemcpyAsync(vg.data(), vd, gb, hipMemcpyDeviceToHost, m->stream));
            }
            MIVI_HIP_CHECK(hipStreamSynchronize(m->stream));  // and the previous layer's uploads have read kg/vg
            q8_rows_to_groups((const uint8_t*)k_in + l * tb, start % 16, tokens, nkv, false, kg.data());
            q8_rows_to_groups((const uint8_t*)v_in + l * tb, start % 16, tokens, nkv, true, vg.data());
            MIVI_HIP_CHECK(hipMemcpyAsync(kd, kg.data(), gb, hipMemcpyHostToDevice, m->stream));
            MIVI_HIP_CHECK(hipMemcpyAsync(vd, vg.data(), gb, hipMemcpyHostToDevice, m->stream));
        }
    } else {
        for (size_t l = 0; l < c.n_attn_layers; l++) {
            MIVI_HIP_CHECK(hipMemcpyAsync(st.kc + l * lb + start * rb, (const uint8_t*)k_in + l * tb, tb,
                                          hipMemcpyHostToDevice, m->stream));
            MIVI_HIP_CHECK(hipMemcpyAsync(st.vc + l * lb + start * rb, (const uint8_t*)v_in + l * tb, tb,
                                          hipMemcpyHostToDevice, m->stream));
        }
    }
    MIVI_HIP_CHECK(hipStreamSynchronize(m->stream));
    return MIVI_OK;
}

// arena.rs:110-114: the sequence's current ShortConv state (the ping-pong
// buffer its phase selects) to the host
static int32_t conv_out_host(mivi_model* m, size_t seq, float* conv_out) {
    Ctrl ctl;
    MIVI_HIP_CHECK(hipMemcpyAsync(&ctl, m->ctrl, sizeof(Ctrl), hipMemcpyDeviceToHost, m->stream));
    MIVI_HIP_CHECK(hipStreamSynchronize(m->stream));
    const SeqState& st = m->seqs[seq];
    const float* cur = (ctl.phase[seq] & 1) ? st.conv_b : st.conv_a;
    MIVI_HIP_CHECK(hipMemcpy(conv_out, cur, conv_state_len(m) * 4, hipMemcpyDeviceToHost));
    return MIVI_OK;
}

// arena.rs:116-123: the state becomes phase 0's input buffer
static int32_t conv_in_host(mivi_model* m, size_t seq, const float* conv_in) {
    MIVI_HIP_CHECK(hipMemcpyAsync(m->seqs[seq].conv_a, conv_in, conv_state_len(m) * 4, hipMemcpyHostToDevice, m->stream));
    hipLaunchKernelGGL(set_int_kernel, dim3(1), dim3(1), 0, m->stream, &m->ctrl->phase[seq], 0);
    MIVI_HIP_CHECK(hipGetLastError());
    MIVI_HIP_CHECK(hipStreamSynchronize(m->stream));
    return MIVI_OK;
}

static int32_t state_sizes(mivi_model* m, size_t seq, size_t tokens, size_t kv_len, size_t conv_len) {
    if (!m || seq >= m->info.max_batch) return set_error(MIVI_ERR_INVALID_ARGUMENT, "bad model or sequence");
    if (tokens > m->info.max_seq_len)
        return set_error(MIVI_ERR_KV_CACHE, "KV cache error: Context length exceeded: attempted pos %zu >= max_seq_len %zu",
                         tokens, m->info.max_seq_len);
    size_t need = m->info.n_attn_layers * tokens * m->kv_row_bytes;
    if (kv_len < need) return err_buffer_too_small(need, kv_len);
    size_t cl = conv_state_len(m);
    if (conv_len < cl) return err_buffer_too_small(cl, conv_len);
    return MIVI_OK;
}

extern "C" int32_t mivi_hip_model_export_state(mivi_model* m, size_t seq, size_t tokens, void* k_out, void* v_out,
                                               size_t kv_len, float* conv_out, size_t conv_len) {
    int32_t rc = state_sizes(m, seq, tokens, kv_len, conv_len);
    if (rc) return rc;
    if ((rc = kv_rows_out(m, seq, 0, tokens, k_out, v_out))) return rc;
    if ((rc = conv_out_host(m, seq, conv_out))) return rc;
    return clear_error();
}

extern "C" int32_t mivi_hip_model_import_state(mivi_model* m, size_t seq, size_t tokens, const void* k_in,
                                               const void* v_in, size_t kv_len, const float* conv_in,
                                               size_t conv_len) {
    int32_t rc = state_sizes(m, seq, tokens, kv_len, conv_len);
    if (rc) return rc;
    if ((rc = kv_rows_in(m, seq, 0, tokens, k_in, v_in))) return rc;
    if ((rc = conv_in_host(m, seq, conv_in))) return rc;
    return clear_error();
}

extern "C" int32_t mivi_hip_model_export_state_range(mivi_model* m, size_t seq, size_t start, size_t tokens,
                                                     void* k_out, void* v_out, size_t kv_len, float* conv_out,
                                                     size_t conv_len) {
    int32_t rc = kv_interval_check(m, seq, start, tokens);
    if (rc) return rc;
    const size_t need = m->info.n_attn_layers * tokens * m->kv_row_bytes;
    if ((tokens && (!k_out || !v_out)) || kv_len < need) return err_buffer_too_small(need, kv_len);
    if (conv_out && conv_len < conv_state_len(m)) return err_buffer_too_small(conv_state_len(m), conv_len);
    if ((rc = kv_rows_out(m, seq, start, tokens, k_out, v_out))) return rc;
    if (conv_out && (rc = conv_out_host(m, seq, conv_out))) return rc;
    return clear_error();
}

extern "C" int32_t mivi_hip_model_import_state_at(mivi_model* m, size_t seq, size_t start, size_t tokens,
                                                  const void* k_in, const void* v_in, size_t kv_len,
                                                  const float* conv_in, size_t conv_len) {
    int32_t rc = kv_interval_check(m, seq, start, tokens);
    if (rc) return rc;
    const size_t need = m->info.n_attn_layers * tokens * m->kv_row_bytes;
    if (kv_len != need || (tokens && (!k_in || !v_in)))  // KvError::DimMismatch (cache.rs:851-856)
        return set_error(MIVI_ERR_KV_CACHE, "KV cache error: dimension mismatch: expected %zu, got %zu", need, kv_len);
    if (conv_in && conv_len != conv_state_len(m))
        return set_error(MIVI_ERR_KV_CACHE, "KV cache error: dimension mismatch: expected %zu, got %zu",
                         conv_state_len(m), conv_len);
    if ((rc = kv_rows_in(m, seq, start, tokens, k_in, v_in))) return rc;
    if (conv_in && (rc = conv_in_host(m, seq, conv_in))) return rc;
    return clear_error();
}

// ------------------------------------------------------------ prefix cache
//
// PrefixCache (crates/mivi-kv/src/prefix.rs) with its snapshots in device
// memory. A node owns one chunk's KV interval [kv_start, pos) of every
// attention layer (K then V, as the model's cache stores them: rows, or whole
// 16-token groups of the Q8_0 group layout) and the ShortConv state at its
// boundary, copied device to device from a sequence of the model at insert
// and back at restore. The host keeps the reference's bookkeeping: chained
// chunk hashes, delta nodes with parent links, LRU order with the deepest
// chunk evicted first, a chunk count and a byte budget.

namespace {

constexpr size_t kPrefixChunkTokens = 64;          // PREFIX_CHUNK_SIZE (prefix.rs:12)
constexpr size_t kPrefixMaxChunks = 1024;          // DEFAULT_MAX_CACHED_CHUNKS (prefix.rs:15)
constexpr size_t kPrefixMaxBytes = 512ull << 20;   // DEFAULT_MAX_PREFIX_CACHE_BYTES (prefix.rs:17)

// compute_chunk_hash (prefix.rs:70-87): 64-bit FNV-1a over the tokens'
// little-endian bytes, started from the FNV offset basis for a first chunk
// and from the previous hash xor 0x9E3779B97F4A7C15 otherwise.
uint64_t prefix_chunk_hash(uint64_t prev, const uint32_t* t, size_t n) {
    uint64_t h = prev == 0 ? 0xCBF29CE484222325ull : prev ^ 0x9E3779B97F4A7C15ull;
    for (size_t i = 0; i < n; i++)
        for (int b = 0; b < 4; b++) {
            h ^= (t[i] >> (8 * b)) & 0xFFu;
            h *= 0x00000100000001B3ull;
        }
    return h;
}

struct PrefixNode {
    size_t chunk_index = 0, pos = 0, kv_start = 0;
    uint64_t hash = 0, parent = 0;
    uint64_t standalone = 0;  // compute_chunk_hash(0, tokens): the suffix search's key (prefix.rs:24-26)
    bool has_parent = false;
    std::vector<uint32_t> tokens;
    uint8_t* dev = nullptr;  // K interval of every attention layer | V interval | ShortConv state
    size_t kv_bytes = 0;     // bytes of the K (or V) part
    size_t conv_bytes = 0;
    size_t bytes() const { return sizeof(PrefixNode) + tokens.capacity() * 4 + 2 * kv_bytes + conv_bytes; }
};

// the current ShortConv buffer of a sequence (ping-pong by *phase) into dst
__global__ void conv_snapshot_kernel(float* dst, const float* a, const float* b, const int* phase, size_t n) {
    const float* src = (*phase & 1) ? b : a;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        dst[i] = src[i];
}

}  // namespace

struct mivi_prefix_cache {
    size_t chunk_size = kPrefixChunkTokens, max_chunks = kPrefixMaxChunks, max_bytes = kPrefixMaxBytes;
    std::map<uint64_t, PrefixNode> chunks;
    std::vector<uint64_t> lru;  // least recently used first
    size_t total = 0;
    // the model shape the snapshots were taken from
    size_t n_attn = 0, row_bytes = 0, conv_len = 0;
    bool shaped = false;
    ~mivi_prefix_cache() {
        for (auto& e : chunks)
            if (e.second.dev) (void)hipFree(e.second.dev);
    }
    void lru_remove(uint64_t h) {
        auto it = std::find(lru.begin(), lru.end(), h);
        if (it != lru.end()) lru.erase(it);
    }
    void touch(uint64_t h) {  // prefix.rs:440-446
        auto it = std::find(lru.begin(), lru.end(), h);
        if (it != lru.end()) {
            lru.erase(it);
            lru.push_back(h);
        }
    }
    // prefix.rs:425-437: the least recently used of the chunks with the
    // largest chunk index (leaves go before the ancestors they extend)
    bool select_eviction(uint64_t* out) const {
        bool sel = false;
        size_t idx = 0;
        for (uint64_t h : lru) {
            auto it = chunks.find(h);
            if (it == chunks.end()) continue;
            if (!sel || it->second.chunk_index > idx) {
                sel = true;
                idx = it->second.chunk_index;
                *out = h;
            }
        }
        if (!sel && !lru.empty()) {
            *out = lru.front();
            sel = true;
        }
        return sel;
    }
    void evict(uint64_t h) {
        lru_remove(h);
        auto it = chunks.find(h);
        if (it == chunks.end()) return;
        total -= std::min(total, it->second.bytes());
        if (it->second.dev) (void)hipFree(it->second.dev);
        chunks.erase(it);
    }
    size_t prune(size_t target) {  // prefix.rs:401-423
        size_t n = 0;
        uint64_t h;
        while (total > target && !lru.empty() && select_eviction(&h)) {
            const bool present = chunks.count(h) != 0;
            evict(h);
            n += present;
        }
        return n;
    }
};

static int32_t prefix_shape(mivi_prefix_cache* pc, mivi_model* m) {
    const size_t conv_len = m->info.n_layers * m->info.dim * std::max<size_t>(1, m->info.ssm_conv_kernel);
    if (m->kv_packed && pc->chunk_size % 16)
        return set_error(MIVI_ERR_INVALID_ARGUMENT, "chunk size %zu: the Q8_0 group layout needs multiples of 16",
                         pc->chunk_size);
    if (!pc->shaped) {
        pc->n_attn = m->info.n_attn_layers;
        pc->row_bytes = m->kv_row_bytes;
        pc->conv_len = conv_len;
        pc->shaped = true;
    } else if (pc->n_attn != m->info.n_attn_layers || pc->row_bytes != m->kv_row_bytes || pc->conv_len != conv_len) {
        return set_error(MIVI_ERR_INVALID_ARGUMENT, "prefix cache holds snapshots of a model of another shape");
    }
    return MIVI_OK;
}

static int32_t dim_mismatch(size_t expected, size_t got) {  // KvError::DimMismatch
    return set_error(MIVI_ERR_KV_CACHE, "KV cache error: dimension mismatch: expected %zu, got %zu", expected, got);
}

extern "C" int32_t mivi_hip_prefix_cache_create(size_t max_chunks, size_t chunk_size, size_t max_memory_bytes,
                                                mivi_prefix_cache** out) {
    if (!out) return set_error(MIVI_ERR_INVALID_ARGUMENT, "null argument");
    mivi_prefix_cache* pc = new mivi_prefix_cache();
    // PrefixCache::with_budget (prefix.rs:148-168): 0 takes the default
    if (chunk_size) pc->chunk_size = chunk_size;
    if (max_chunks) pc->max_chunks = max_chunks;
    if (max_memory_bytes) pc->max_bytes = max_memory_bytes;
    *out = pc;
    return clear_error();
}

extern "C" void mivi_hip_prefix_cache_destroy(mivi_prefix_cache* pc) { delete pc; }

extern "C" uint64_t mivi_hip_prefix_chunk_hash(uint64_t prev_hash, const uint32_t* tokens, size_t n) {
    return prefix_chunk_hash(prev_hash, tokens, tokens ? n : 0);
}

extern "C" size_t mivi_hip_prefix_cache_len(const mivi_prefix_cache* pc) { return pc ? pc->chunks.size() : 0; }
extern "C" size_t mivi_hip_prefix_cache_memory_bytes(const mivi_prefix_cache* pc) { return pc ? pc->total : 0; }
extern "C" int32_t mivi_hip_prefix_cache_contains(const mivi_prefix_cache* pc, uint64_t hash) {
    return pc && pc->chunks.count(hash) ? 1 : 0;
}
extern "C" size_t mivi_hip_prefix_cache_prune(mivi_prefix_cache* pc, size_t target_bytes) {
    return pc ? pc->prune(target_bytes) : 0;
}
extern "C" void mivi_hip_prefix_cache_clear(mivi_prefix_cache* pc) {
    if (!pc) return;
    while (!pc->chunks.empty()) pc->evict(pc->chunks.begin()->first);
    pc->lru.clear();
    pc->total = 0;
}

// insert_node (prefix.rs:360-392): a node for the chunk `tokens` (hash
// chained on prev_hash) owning positions [kv_start, pos) of sequence seq's
// KV caches and the sequence's ShortConv state, copied device to device. In
// the Q8_0 group layout the interval is stored as the whole groups covering
// it (rows past pos in the last group come along and are rewritten by the
// decode before they are read).
static int32_t prefix_insert_node(mivi_prefix_cache* pc, mivi_model* m, size_t seq, uint64_t prev_hash,
                                  const uint32_t* tokens, size_t n_tokens, size_t chunk_index, size_t kv_start,
                                  size_t pos, bool has_parent, uint64_t* hash_out) {
    const uint64_t hash = prefix_chunk_hash(prev_hash, tokens, n_tokens);
    *hash_out = hash;
    clear_error();
    if (pc->chunks.count(hash)) {  // already cached: the new snapshot is not taken
        pc->touch(hash);
        return MIVI_OK;
    }
    PrefixNode nd;
    nd.chunk_index = chunk_index;
    nd.pos = pos;
    nd.kv_start = kv_start;
    nd.hash = hash;
    nd.parent = prev_hash;
    nd.has_parent = has_parent;
    nd.standalone = prefix_chunk_hash(0, tokens, n_tokens);
    nd.tokens.assign(tokens, tokens + n_tokens);
    // the group layout copies whole 16-token groups (the layer buffer holds
    // whole groups, also past a max_seq_len that is not a multiple of 16)
    const size_t end = m->kv_packed ? (pos + 15) / 16 * 16 : pos;
    const size_t iv = (end - kv_start) * pc->row_bytes;  // one layer's interval (rows, or whole groups)
    nd.kv_bytes = pc->n_attn * iv;
    nd.conv_bytes = pc->conv_len * 4;
    MIVI_HIP_CHECK(hipMalloc(&nd.dev, std::max<size_t>(1, 2 * nd.kv_bytes + nd.conv_bytes)));
    SeqState& st = m->seqs[seq];
    const size_t lb = m->kv_layer_bytes, off = kv_start * pc->row_bytes;
    hipError_t e = hipSuccess;
    if (pc->n_attn && iv) {
        e = hipMemcpy2DAsync(nd.dev, iv, st.kc + off, lb, iv, pc->n_attn, hipMemcpyDeviceToDevice, m->stream);
        if (e == hipSuccess)
            e = hipMemcpy2DAsync(nd.dev + nd.kv_bytes, iv, st.vc + off, lb, iv, pc->n_attn, hipMemcpyDeviceToDevice,
                                 m->stream);
    }
    if (e == hipSuccess && pc->conv_len) {
        hipLaunchKernelGGL(conv_snapshot_kernel, dim3(64), dim3(256), 0, m->stream,
                           (float*)(nd.dev + 2 * nd.kv_bytes), st.conv_a, st.conv_b, &m->ctrl->phase[seq], pc->conv_len);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipStreamSynchronize(m->stream);
    if (e != hipSuccess) {
        (void)hipFree(nd.dev);
        return set_error(MIVI_ERR_HIP, "prefix snapshot copy failed: %s", hipGetErrorString(e));
    }
    const size_t nb = nd.bytes();
    pc->chunks.emplace(hash, std::move(nd));
    pc->lru.push_back(hash);
    pc->total += nb;
    uint64_t ev;
    while (pc->chunks.size() > pc->max_chunks && pc->select_eviction(&ev)) pc->evict(ev);
    pc->prune(pc->max_bytes);
    return MIVI_OK;
}

// insert_delta_chunk (prefix.rs:251-303)
extern "C" int32_t mivi_hip_prefix_cache_insert_delta(mivi_prefix_cache* pc, mivi_model* m, size_t seq, size_t pos,
                                                      uint64_t prev_hash, const uint32_t* tokens, size_t n_tokens,
                                                      size_t chunk_index, uint64_t* hash_out) {
    if (!pc || !m || !hash_out || (n_tokens && !tokens) || seq >= m->info.max_batch)
        return set_error(MIVI_ERR_INVALID_ARGUMENT, "bad argument");
    int32_t rc = prefix_shape(pc, m);
    if (rc) return rc;
    size_t start, end;
    if (__builtin_mul_overflow(chunk_index, pc->chunk_size, &start) ||
        __builtin_add_overflow(start, pc->chunk_size, &end))
        return set_error(MIVI_ERR_KV_CACHE, "KV cache error: Context length exceeded: attempted pos %zu >= max_seq_len %zu",
                         (size_t)-1, pos);
    if (n_tokens != pc->chunk_size || pos != end) return dim_mismatch(end, pos);
    if (end > m->info.max_seq_len)
        return set_error(MIVI_ERR_KV_CACHE, "KV cache error: Context length exceeded: attempted pos %zu >= max_seq_len %zu",
                         end, m->info.max_seq_len);
    bool has_parent = false;
    if (start == 0) {
        if (prev_hash != 0) return dim_mismatch(0, start);
    } else {
        auto it = pc->chunks.find(prev_hash);
        if (it == pc->chunks.end()) return dim_mismatch(start, 0);
        if (it->second.pos != start || it->second.chunk_index != chunk_index - 1)
            return dim_mismatch(start, it->second.pos);
        has_parent = true;
    }
    return prefix_insert_node(pc, m, seq, prev_hash, tokens, n_tokens, chunk_index, start, end, has_parent, hash_out);
}

// insert_chunk (prefix.rs:239-249): a full snapshot, the whole prefix
// [0, pos) of sequence seq and its ShortConv state in one node with no
// parent; restoring it needs no other node.
extern "C" int32_t mivi_hip_prefix_cache_insert(mivi_prefix_cache* pc, mivi_model* m, size_t seq, size_t pos,
                                                uint64_t prev_hash, const uint32_t* tokens, size_t n_tokens,
                                                size_t chunk_index, uint64_t* hash_out) {
    if (!pc || !m || !hash_out || (n_tokens && !tokens) || seq >= m->info.max_batch)
        return set_error(MIVI_ERR_INVALID_ARGUMENT, "bad argument");
    int32_t rc = prefix_shape(pc, m);
    if (rc) return rc;
    if (pos > m->info.max_seq_len)
        return set_error(MIVI_ERR_KV_CACHE, "KV cache error: Context length exceeded: attempted pos %zu >= max_seq_len %zu",
                         pos, m->info.max_seq_len);
    return prefix_insert_node(pc, m, seq, prev_hash, tokens, n_tokens, chunk_index, 0, pos, false, hash_out);
}

// find_longest_suffix_match (prefix.rs:453-517): for k full chunks from the
// longest down, the suffix of the last k * chunk_size tokens (its absolute
// position start_pos + offset a multiple of chunk_size) against the cached
// chunks of that many tokens by their standalone hash; the first found is
// touched in the LRU order. The reference scans its hash map in no defined
// order; here the chunks are scanned in ascending hash order.
extern "C" int32_t mivi_hip_prefix_cache_find_suffix(mivi_prefix_cache* pc, size_t start_pos, const uint32_t* tokens,
                                                     size_t n, size_t* suffix_len, size_t* match_pos,
                                                     uint64_t* hash_out) {
    if (!pc || !suffix_len || !match_pos || !hash_out || (n && !tokens))
        return set_error(MIVI_ERR_INVALID_ARGUMENT, "null argument");
    *suffix_len = 0;
    *match_pos = 0;
    *hash_out = 0;
    clear_error();
    const size_t cs = pc->chunk_size;
    if (n < cs || pc->chunks.empty()) return MIVI_OK;
    const size_t max_k = (n > start_pos ? n - start_pos : 0) / cs;
    for (size_t k = max_k; k >= 1; k--) {
        const size_t len = k * cs, s0 = n - len;
        if (s0 < start_pos || (start_pos + s0) % cs) continue;
        const uint64_t sh = prefix_chunk_hash(0, tokens + s0, len);
        for (const auto& e : pc->chunks) {
            const PrefixNode& nd = e.second;
            if (nd.tokens.size() == len && nd.standalone == sh) {
                pc->touch(e.first);
                *suffix_len = len;
                *match_pos = nd.pos;
                *hash_out = e.first;
                return MIVI_OK;
            }
        }
    }
    return MIVI_OK;
}

// find_longest_prefix (prefix.rs:200-237): the deepest cached chunk whose
// chain of hashes matches the tokens' full chunks (the chain stops at the
// first miss); touches it in the LRU order
static const PrefixNode* prefix_find(mivi_prefix_cache* pc, const uint32_t* tokens, size_t n, size_t* matched) {
    *matched = 0;
    if (n < pc->chunk_size) return nullptr;
    uint64_t h = 0, deep = 0;
    size_t deep_len = 0;
    for (size_t i = 0; i < n / pc->chunk_size; i++) {
        h = prefix_chunk_hash(h, tokens + i * pc->chunk_size, pc->chunk_size);
        if (!pc->chunks.count(h)) break;
        deep = h;
        deep_len = (i + 1) * pc->chunk_size;
    }
    if (!deep_len) return nullptr;
    pc->touch(deep);
    *matched = deep_len;
    return &pc->chunks.at(deep);
}

extern "C" int32_t mivi_hip_prefix_cache_find(mivi_prefix_cache* pc, const uint32_t* tokens, size_t n,
                                              size_t* matched, uint64_t* hash_out) {
    if (!pc || !matched || !hash_out || (n && !tokens)) return set_error(MIVI_ERR_INVALID_ARGUMENT, "null argument");
    const PrefixNode* nd = prefix_find(pc, tokens, n, matched);
    *hash_out = nd ? nd->hash : 0;
    return clear_error();
}

// restore_longest_prefix (prefix.rs:305-358): the matched chain's KV
// intervals into sequence seq's caches in causal order, then the deepest
// node's ShortConv state (as mivi_hip_model_import_state leaves it: phase 0's
// input buffer). *matched = 0 when nothing matches; the caller prefills from
// position *matched on.
extern "C" int32_t mivi_hip_prefix_cache_restore(mivi_prefix_cache* pc, mivi_model* m, size_t seq,
                                                 const uint32_t* tokens, size_t n, size_t* matched,
                                                 uint64_t* hash_out) {
    if (!pc || !m || !matched || !hash_out || (n && !tokens) || seq >= m->info.max_batch)
        return set_error(MIVI_ERR_INVALID_ARGUMENT, "bad argument");
    *matched = 0;
    *hash_out = 0;
    size_t len = 0;
    const PrefixNode* nd = prefix_find(pc, tokens, n, &len);
    if (!nd) return clear_error();
    int32_t rc = prefix_shape(pc, m);
    if (rc) return rc;
    if (nd->pos != len) return dim_mismatch(len, nd->pos);
    if (len > m->info.max_seq_len)
        return set_error(MIVI_ERR_KV_CACHE, "KV cache error: Context length exceeded: attempted pos %zu >= max_seq_len %zu",
                         len, m->info.max_seq_len);
    std::vector<const PrefixNode*> path;
    for (const PrefixNode* p = nd;;) {
        path.push_back(p);
        if (!p->has_parent) break;
        auto it = pc->chunks.find(p->parent);
        if (it == pc->chunks.end()) return dim_mismatch(len, 0);
        p = &it->second;
    }
    SeqState& st = m->seqs[seq];
    const size_t lb = m->kv_layer_bytes;
    for (auto it = path.rbegin(); it != path.rend(); ++it) {
        const PrefixNode* p = *it;
        if (!pc->n_attn || !p->kv_bytes) continue;
        const size_t iv = p->kv_bytes / pc->n_attn, off = p->kv_start * pc->row_bytes;
        MIVI_HIP_CHECK(hipMemcpy2DAsync(st.kc + off, lb, p->dev, iv, iv, pc->n_attn, hipMemcpyDeviceToDevice, m->stream));
        MIVI_HIP_CHECK(hipMemcpy2DAsync(st.vc + off, lb, p->dev + p->kv_bytes, iv, iv, pc->n_attn,
                                        hipMemcpyDeviceToDevice, m->stream));
    }
    if (pc->conv_len)
        MIVI_HIP_CHECK(hipMemcpyAsync(st.conv_a, nd->dev + 2 * nd->kv_bytes, pc->conv_len * 4, hipMemcpyDeviceToDevice,
                                      m->stream));
    hipLaunchKernelGGL(set_int_kernel, dim3(1), dim3(1), 0, m->stream, &m->ctrl->phase[seq], 0);
    MIVI_HIP_CHECK(hipStreamSynchronize(m->stream));
    *matched = len;
    *hash_out = nd->hash;
    return clear_error();
}
