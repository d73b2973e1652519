// Sampler::sample (crates/mivi-model/src/sampler.rs:91-135) on the device:
// penalties, temperature, min-p, top-k, softmax, then top-p or categorical
// sampling with the reference's xorshift64* generator, with the logits
// modified in place as the reference modifies its &mut [f32].
//
// Two paths compute the same function:
// * the whole-row path: one workgroup over the row (mivi_hip_sample, and the
//   fallback of the split path);
// * the split path (rows of a batch, the generation loop): a chunk kernel with
//   one workgroup per 1024 logits applies the penalties and the temperature,
//   writes the row back and, when top_k <= 128, hands on every logit of its
//   chunk with fewer than top_k larger ones in the chunk (the only logits the
//   global top-k can keep); a pick kernel, one workgroup per row, runs min-p,
//   top-k, softmax and top-p / categorical over those candidates. Rows whose
//   candidates do not fit (ties, top_k of 0 or above 128, all -inf) run the
//   whole-row steps from the transformed row instead.
//
// Order statistics run as radix searches over order-preserving 32-bit keys of
// the floats (four 8-bit passes, 256-bin histograms in LDS). Probability
// masses are accumulated as 2^-40 fixed-point integers, so every bin sum and
// prefix is exact and the result does not depend on thread timing. The draw r
// is bit-exact with the reference; the cumulative sums it is compared against
// are the reference's up to float rounding (its sums run sequentially), so a
// token can differ only where r falls within rounding of a boundary. Tied
// probabilities in the top-p order are taken by index (the reference's
// sort_unstable_by leaves their order unspecified).
#include <math.h>

#include <algorithm>
#include <mutex>
#include <vector>

#include "common.h"
#include "gemv.h"

namespace {

constexpr int kST = 1024;                 // threads of a row workgroup
constexpr int kSW = kST / 64;             // its waves
constexpr double kFix = 1099511627776.0;  // 2^40
constexpr int kWinLds = 1024;             // penalty-window ids staged in LDS

constexpr int kCT = 256;                  // threads of a chunk workgroup
constexpr int kCW = kCT / 64;             // its waves
constexpr int kCC = 4 * kCT;              // logits per chunk
constexpr int kCapC = 256;                // candidates a chunk may hand on
constexpr int kKMax = 128;                // largest top_k the split path selects
constexpr int kCandVPT = 8;               // candidates per thread of the pick workgroup
constexpr int kCapB = kST * kCandVPT;     // candidates a row may hold
constexpr int kMaxChunks = kST;           // chunks the pick workgroup indexes

enum { kModeRow = 0, kModeGreedy = 1, kModeTopK = 2, kModeCat = 3 };

struct SampleArgs {
    float temperature, top_p, min_p, ln_min_p, rep, presence, frequency;
    int top_k;
};

// order-preserving key of a float (non-NaN); funkey inverts it
__device__ __forceinline__ uint32_t fkey(float f) {
    const uint32_t b = __float_as_uint(f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float funkey(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}
__device__ __forceinline__ uint64_t fixp(float p) { return (uint64_t)((double)p * kFix); }

__device__ __forceinline__ bool penalties_on(const SampleArgs& c) {
    return (c.rep > 0.0f && c.rep != 1.0f) || c.presence != 0.0f || c.frequency != 0.0f;
}

// sampler.rs:219-257 for one distinct token seen `count` times
__device__ __forceinline__ float penalise(float v, int count, const SampleArgs& c) {
    if (c.rep > 0.0f && c.rep != 1.0f) v = v > 0.0f ? v / c.rep : v * c.rep;
    if (c.presence != 0.0f) v -= c.presence;
    if (c.frequency != 0.0f) v -= c.frequency * (float)count;
    return v;
}

struct Shared {
    unsigned long long hist[256];
    unsigned long long wsum[kSW];
    float wf[kSW];
    int wi[kSW];
    uint32_t bin;
    unsigned long long above;
    float r;
    int found;
    float sp[64];
    int sid[64];
    uint32_t rec[kWinLds];
    int off[kMaxChunks + 1];
};

// Adds w to hist[b] for the active lanes of a wave (called by every lane):
// one LDS atomic per wave when every active lane has the same bin (the top
// bits of a row's keys mostly agree, and per-lane atomics would serialise on
// that bin), one per lane otherwise. Integer sums: exact in any order.
template <class T>
__device__ __forceinline__ void hist_add(T* hist, uint32_t b, T w, bool act) {
    const unsigned long long m = __ballot(act);
    if (!m) return;
    const int lead = __builtin_ctzll(m);
    const uint32_t lb = __shfl(b, lead, 64);
    if (__ballot(act && b != lb) == 0) {
        T s = act ? w : (T)0;
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o, 64);
        if ((int)(threadIdx.x & 63) == lead) atomicAdd(&hist[lb], s);
    } else if (act) {
        atomicAdd(&hist[b], w);
    }
}

// Wave 0: the first bin from the top of hist where `above` plus the running
// weight reaches target (bin 0 if none does, as a full scan ends); lane l
// holds bins 255 - 4l .. 252 - 4l. Writes the bin and the weight above it.
template <class T>
__device__ __forceinline__ void select_bin(const T* hist, T above, T target, uint32_t* bin_out, T* above_out) {
    const int l = threadIdx.x;
    T hb[4], ls = 0;
#pragma unroll
    for (int q = 0; q < 4; q++) { hb[q] = hist[255 - 4 * l - q]; ls += hb[q]; }
    T inc = ls;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const T u = __shfl_up(inc, o, 64);
        if (l >= o) inc += u;
    }
    const T ex = inc - ls;
    const unsigned long long hit = __ballot(above + inc >= target);
    const int first = hit ? __builtin_ctzll(hit) : 64;
    if (first == 64) {
        if (l == 63) { *bin_out = 0; *above_out = above + inc - hb[3]; }
    } else if (l == first) {
        T a = above + ex;
        int q = 0;
        for (; q < 3; q++) {
            if (a + hb[q] >= target) break;
            a += hb[q];
        }
        *bin_out = (uint32_t)(255 - 4 * l - q);
        *above_out = a;
    }
}

// A row as the passes see it: read and written in memory on each pass
// (MemRow, element threadIdx.x + kST j in step j; the row stays in L2), or
// the candidates of the split path (CandRow). each(f) calls f(i, x) for every
// element this thread owns, x by reference; each_slot(f) calls f(i, x, valid)
// for every slot in step across the workgroup; size() counts the elements.
struct MemRow {
    float* L;
    int n;
    __device__ __forceinline__ void load(float* L_, int n_) { L = L_; n = n_; }
    __device__ __forceinline__ void store(float*) const {}
    __device__ __forceinline__ int size() const { return n; }
    template <class F>
    __device__ __forceinline__ void each(F f) {
        for (int i = threadIdx.x; i < n; i += kST) {
            float x = L[i];
            f(i, x);
            L[i] = x;
        }
    }
    template <class F>
    __device__ __forceinline__ void each_slot(F f) {
        for (int base = 0; base < n; base += kST) {
            const int i = base + threadIdx.x;
            const bool ok = i < n;
            float x = ok ? L[i] : 0.0f;
            f(i, x, ok);
            if (ok) L[i] = x;
        }
    }
};

// The candidates of one row (list position threadIdx.x + kST j in slot j),
// with their indices in the row; store() writes the whole row: zero outside
// the candidates (whose probability is zero on every path through here).
struct CandRow {
    float v[kCandVPT];
    int id[kCandVPT];
    int m, n;
    bool write;
    __device__ __forceinline__ void load(const float* cval, const int* cidx, size_t base, const int* off, int nch, int M, int n_,
                         bool write_) {
        m = M;
        n = n_;
        write = write_;
#pragma unroll
        for (int j = 0; j < kCandVPT; j++) {
            const int p = (int)threadIdx.x + kST * j;
            v[j] = -INFINITY;
            id[j] = 0;
            if (p < M) {
                int lo = 0, hi = nch;  // off[lo] <= p < off[hi]
                while (hi - lo > 1) {
                    const int mid = (lo + hi) >> 1;
                    if (off[mid] <= p) lo = mid;
                    else hi = mid;
                }
                const size_t g = base + (size_t)lo * kCapC + (p - off[lo]);
                v[j] = cval[g];
                id[j] = cidx[g];
            }
        }
    }
    __device__ __forceinline__ void store(float* L) const {
        if (!write) return;
        for (int i = 4 * threadIdx.x; i < n; i += 4 * kST) {
            if (i + 3 < n && ((uintptr_t)L & 15) == 0) {
                *(f32x4*)(L + i) = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            } else {
                for (int e = 0; e < 4 && i + e < n; e++) L[i + e] = 0.0f;
            }
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < kCandVPT; j++)
            if ((int)threadIdx.x + kST * j < m) L[id[j]] = v[j];
    }
    __device__ __forceinline__ int size() const { return m; }
    template <class F>
    __device__ __forceinline__ void each(F f) {
#pragma unroll
        for (int j = 0; j < kCandVPT; j++)
            if ((int)threadIdx.x + kST * j < m) f(id[j], v[j]);
    }
    template <class F>
    __device__ __forceinline__ void each_slot(F f) {
#pragma unroll
        for (int j = 0; j < kCandVPT; j++) f(id[j], v[j], (int)threadIdx.x + kST * j < m);
    }
};

template <class Row>
__device__ __forceinline__ float bmax_finite(Row& row, Shared& sh) {
    float m = -INFINITY;
    row.each([&](int, float& x) {
        if (isfinite(x) && x > m) m = x;
    });
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    if ((threadIdx.x & 63) == 0) sh.wf[threadIdx.x >> 6] = m;
    __syncthreads();
    m = sh.wf[0];
    for (int w = 1; w < kSW; w++) m = fmaxf(m, sh.wf[w]);
    __syncthreads();
    return m;
}

// sum of the per-thread partials, in a fixed order (wave butterfly, then waves in order)
__device__ __forceinline__ float bsum_f(float v, Shared& sh) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    if ((threadIdx.x & 63) == 0) sh.wf[threadIdx.x >> 6] = v;
    __syncthreads();
    float s = sh.wf[0];
    for (int w = 1; w < kSW; w++) s += sh.wf[w];
    __syncthreads();
    return s;
}

__device__ __forceinline__ unsigned long long bsum_u(unsigned long long v, Shared& sh) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    if ((threadIdx.x & 63) == 0) sh.wsum[threadIdx.x >> 6] = v;
    __syncthreads();
    unsigned long long s = 0;
    for (int w = 0; w < kSW; w++) s += sh.wsum[w];
    __syncthreads();
    return s;
}

// Exclusive prefix over the threads (thread order) of a per-thread value.
template <int NW, class T>
__device__ __forceinline__ T bscan_excl(T v, T* total, T* wtot) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    T inc = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const T u = __shfl_up(inc, o, 64);
        if (lane >= o) inc += u;
    }
    if (lane == 63) wtot[wave] = inc;
    __syncthreads();
    T before = 0, all = 0;
    for (int w = 0; w < NW; w++) {
        if (w < wave) before += wtot[w];
        all += wtot[w];
    }
    __syncthreads();
    *total = all;
    return before + inc - v;
}

// sampler.rs:305-316: first index of the strict maximum (0 if none)
template <class Row>
__device__ __forceinline__ int bargmax(Row& row, Shared& sh) {
    float best = -INFINITY;
    int idx = 0x7FFFFFFF;
    row.each([&](int i, float& x) {
        if (x > best || (x == best && x > -INFINITY && i < idx)) { best = x; idx = i; }
    });
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float ov = __shfl_xor(best, o, 64);
        const int oi = __shfl_xor(idx, o, 64);
        if (ov > best || (ov == best && oi < idx)) { best = ov; idx = oi; }
    }
    if ((threadIdx.x & 63) == 0) { sh.wf[threadIdx.x >> 6] = best; sh.wi[threadIdx.x >> 6] = idx; }
    __syncthreads();
    best = sh.wf[0];
    idx = sh.wi[0];
    for (int w = 1; w < kSW; w++)
        if (sh.wf[w] > best || (sh.wf[w] == best && sh.wi[w] < idx)) { best = sh.wf[w]; idx = sh.wi[w]; }
    __syncthreads();
    return best > -INFINITY && idx != 0x7FFFFFFF ? idx : 0;
}

// The largest key K whose active elements with key >= K weigh at least
// `target` (the caller guarantees the total does); *above = the weight of the
// active elements with key > K. f(i, x, key, weight) says whether element i
// (value x) is active.
template <class Row, class F>
__device__ __forceinline__ uint32_t radix_search(Row& row, F f, unsigned long long target, unsigned long long* above_out, Shared& sh) {
    uint32_t prefix = 0, pmask = 0;
    unsigned long long above = 0;
    for (int pass = 0; pass < 4; pass++) {
        const int shf = 24 - 8 * pass;
        for (int b = threadIdx.x; b < 256; b += kST) sh.hist[b] = 0;
        __syncthreads();
        row.each_slot([&](int i, float& x, bool ok) {
            uint32_t k = 0;
            unsigned long long w = 0;
            const bool act = ok && f(i, x, k, w) && w && (k & pmask) == prefix;
            hist_add(sh.hist, (k >> shf) & 255u, w, act);
        });
        __syncthreads();
        if (threadIdx.x < 64) select_bin(sh.hist, above, target, &sh.bin, &sh.above);
        __syncthreads();
        prefix |= sh.bin << shf;
        pmask |= 0xFFu << shf;
        above = sh.above;
        __syncthreads();
    }
    *above_out = above;
    return prefix;
}

// sampler.rs:70-77 (thread 0), broadcast
__device__ __forceinline__ float draw(unsigned long long* rng, Shared& sh) {
    if (threadIdx.x == 0) {
        unsigned long long s = *rng;
        s ^= s >> 12;
        s ^= s << 25;
        s ^= s >> 27;
        *rng = s;
        const unsigned long long r = (s * 0x2545F4914F6CDD1DULL) >> 32;
        sh.r = (float)(r >> 8) / 16777216.0f;
    }
    __syncthreads();
    const float r = sh.r;
    __syncthreads();
    return r;
}

// Wave 0 finishes a draw over s <= 64 elements (probability sp[l], index
// sid[l]) that hold all the fixed-point mass left: sorted by probability
// (ties by index) for top-p, by index for categorical, then the same
// fixed-point scan as the radix path, so both return the same token. r is
// the draw; returns the token in lane 0.
__device__ __forceinline__ int wave_pick(const Shared& sh, int s, bool top_p, float top_p_v, float r, int n) {
    const int l = threadIdx.x;
    const bool ok = l < s;
    const float p = ok ? sh.sp[l] : 0.0f;
    int id = ok ? sh.sid[l] : 0;
    unsigned long long w = ok ? fixp(p) : 0;
    unsigned long long key = !ok ? 0ull
                             : top_p ? ((unsigned long long)fkey(p) << 32) | (uint32_t)~(uint32_t)id
                                     : (unsigned long long)(0xFFFFFFFFu - (uint32_t)id);
    // bitonic sort, descending by key across the wave
#pragma unroll
    for (int k = 2; k <= 64; k <<= 1) {
#pragma unroll
        for (int j = k >> 1; j > 0; j >>= 1) {
            const unsigned long long ok2 = __shfl_xor(key, j, 64);
            const unsigned long long ow = __shfl_xor(w, j, 64);
            const int oid = __shfl_xor(id, j, 64);
            const bool keep_max = ((l & k) == 0) == ((l & j) == 0);
            if (keep_max ? ok2 > key : ok2 < key) { key = ok2; w = ow; id = oid; }
        }
    }
    unsigned long long cum = w;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const unsigned long long u = __shfl_up(cum, o, 64);
        if (l >= o) cum += u;
    }
    const unsigned long long total = __shfl(cum, 63, 64);
    unsigned long long tr;
    if (top_p) {
        unsigned long long tgt = (unsigned long long)ceil((double)top_p_v * kFix);
        tgt = tgt ? tgt : 1;
        unsigned long long nmass = total;
        const unsigned long long hit = __ballot(cum >= tgt);
        if (total >= tgt) nmass = __shfl(cum, __builtin_ctzll(hit), 64);
        const float rr = r * (float)((double)nmass / kFix);
        tr = (unsigned long long)ceil((double)rr * kFix);
        tr = tr ? tr : 1;
        tr = tr < nmass ? tr : nmass;
    } else {
        tr = (unsigned long long)ceil((double)r * kFix);
        if (tr == 0) return 0;
        if (total < tr) return n - 1;
    }
    const unsigned long long hit = __ballot(cum >= tr);
    return __shfl(id, __builtin_ctzll(hit), 64);
}

// Compacts the elements with match(x) (at most 64, counted by the caller
// with this thread's share `mine`, exclusive prefix `pos`) into sh.sp/sid;
// the next barrier publishes them.
template <class Row, class M>
__device__ __forceinline__ void compact_small(Row& row, M match, int pos, Shared& sh) {
    row.each([&](int i, float& x) {
        if (match(x)) {
            sh.sp[pos] = x;
            sh.sid[pos] = i;
            pos++;
        }
    });
}

// Steps 4-7 of Sampler::sample over a row already penalised and divided by
// the temperature: min-p, top-k, softmax (the probabilities written back to
// L), then top-p or categorical. n is the length of the whole row.
template <class Row>
__device__ __forceinline__ int sample_tail(Row& row, float* L, int n, const SampleArgs& c, unsigned long long* rng, Shared& sh) {
    // 4. min-p (sampler.rs:260-276); ln(min_p) comes from the host's libm
    if (c.min_p > 0.0f && c.min_p < 1.0f) {
        const float mx = bmax_finite(row, sh);
        if (isfinite(mx)) {
            const float thr = mx + c.ln_min_p;
            row.each([&](int, float& x) {
                if (x < thr) x = -INFINITY;
            });
        }
    }
    // 5. top-k: the k-th largest value is the cutoff (sampler.rs:287-301).
    // Over candidates holding fewer than k elements every finite logit is a
    // candidate and the cutoff is -inf: nothing to mask.
    if (c.top_k > 0 && c.top_k < n && c.top_k <= row.size()) {
        unsigned long long above;
        const uint32_t K = radix_search(
            row, [&](int, float x, uint32_t& k, unsigned long long& w) { k = fkey(x); w = 1; return true; },
            (unsigned long long)c.top_k, &above, sh);
        const float cutoff = funkey(K);
        row.each([&](int, float& x) {
            if (x < cutoff) x = -INFINITY;
        });
    }
    // 6. softmax (math.rs:32-72)
    {
        const float mx = bmax_finite(row, sh);
        if (!isfinite(mx)) {
            const float u = 1.0f / (float)n;
            row.each([&](int, float& x) { x = u; });
        } else {
            float s = 0.0f;
            row.each([&](int, float& x) {
                if (isfinite(x)) {
                    x = expf(x - mx);
                    s += x;
                } else {
                    x = 0.0f;
                }
            });
            const float sum = bsum_f(s, sh);
            if (sum > 0.0f) {
                const float inv = 1.0f / sum;
                row.each([&](int, float& x) { x *= inv; });
            } else {
                const float u = 1.0f / (float)n;
                row.each([&](int, float& x) { x = u; });
            }
        }
    }
    row.store(L);
    __syncthreads();
    if (c.top_p < 1.0f) {
        // 7a. top-p (sampler.rs:150-215)
        const float cutoff = n > 1 ? (1.0f - c.top_p) / ((float)n - 1.0f) : 0.0f;
        auto cand = [=](float p) { return p >= cutoff && p > 0.0f && isfinite(p); };
        auto heavy = [=](float p) { return cand(p) && fixp(p) > 0; };
        unsigned long long nc = 0, wt = 0, hv = 0;
        row.each([&](int, float& x) {
            if (cand(x)) {
                nc++;
                const unsigned long long w = fixp(x);
                wt += w;
                hv += w > 0;
            }
        });
        nc = bsum_u(nc, sh);
        wt = bsum_u(wt, sh);
        if (nc == 0) return bargmax(row, sh);
        unsigned long long nh;
        const unsigned long long ph = bscan_excl<kSW, unsigned long long>(hv, &nh, sh.wsum);
        if (nh <= 64) {
            // few candidates carry mass (top-k left few): one wave finishes
            compact_small(row, heavy, (int)ph, sh);
            const float r = draw(rng, sh);
            if (threadIdx.x < 64) {
                const int t = wave_pick(sh, (int)nh, true, c.top_p, r, n);
                if (threadIdx.x == 0) sh.found = t;
            }
            __syncthreads();
            const int t = sh.found;
            __syncthreads();
            return t;
        }
        auto fc = [&](int, float x, uint32_t& k, unsigned long long& w) {
            if (!cand(x)) return false;
            k = fkey(x);
            w = fixp(x);
            return true;
        };
        // the nucleus: candidates above K*, then the first t ties at K*
        unsigned long long tgt = (unsigned long long)ceil((double)c.top_p * kFix);
        tgt = tgt ? tgt : 1;
        unsigned long long nmass;
        if (wt < tgt) {
            nmass = wt;  // every candidate
        } else {
            unsigned long long above;
            const uint32_t Ks = radix_search(row, fc, tgt, &above, sh);
            const unsigned long long ws = fixp(funkey(Ks));
            const unsigned long long t = (tgt - above + ws - 1) / ws;
            nmass = above + t * ws;
        }
        const float mass = (float)((double)nmass / kFix);
        const float r = draw(rng, sh) * mass;
        unsigned long long tr = (unsigned long long)ceil((double)r * kFix);
        tr = tr ? tr : 1;
        tr = tr < nmass ? tr : nmass;
        unsigned long long above_r;
        const uint32_t Kr = radix_search(row, fc, tr, &above_r, sh);
        const unsigned long long wr = fixp(funkey(Kr));
        const unsigned long long j = (tr - above_r + wr - 1) / wr;
        // the j-th tie at Kr in index order: the smallest index whose count of
        // ties at or below it reaches j (keys = reversed indices)
        unsigned long long ab;
        const uint32_t Ki = radix_search(
            row,
            [&](int i, float x, uint32_t& k, unsigned long long& w) {
                if (!(cand(x) && fkey(x) == Kr)) return false;
                k = 0xFFFFFFFFu - (uint32_t)i;
                w = 1;
                return true;
            },
            j, &ab, sh);
        return (int)(0xFFFFFFFFu - Ki);
    } else {
        // 7b. categorical (sampler.rs:137-148): the first index whose
        // cumulative probability reaches r, i.e. the smallest index whose mass
        // at or below it reaches r (keys = reversed indices). r == 0 takes
        // index 0; past the total, n - 1.
        auto heavy = [](float p) { return fixp(p) > 0; };
        unsigned long long tot = 0, hv = 0;
        row.each([&](int, float& x) {
            const unsigned long long w = fixp(x);
            tot += w;
            hv += w > 0;
        });
        tot = bsum_u(tot, sh);
        unsigned long long nh;
        const unsigned long long ph = bscan_excl<kSW, unsigned long long>(hv, &nh, sh.wsum);
        if (nh <= 64) compact_small(row, heavy, (int)ph, sh);
        const float r = draw(rng, sh);
        const unsigned long long tr = (unsigned long long)ceil((double)r * kFix);
        if (tr == 0 || n == 0) return 0;
        if (tot < tr) return n - 1;
        if (nh <= 64) {
            if (threadIdx.x < 64) {
                const int t = wave_pick(sh, (int)nh, false, 1.0f, r, n);
                if (threadIdx.x == 0) sh.found = t;
            }
            __syncthreads();
            const int t = sh.found;
            __syncthreads();
            return t;
        }
        unsigned long long ab;
        const uint32_t Ki = radix_search(
            row,
            [&](int i, float x, uint32_t& k, unsigned long long& w) {
                k = 0xFFFFFFFFu - (uint32_t)i;
                w = fixp(x);
                return true;
            },
            tr, &ab, sh);
        return (int)(0xFFFFFFFFu - Ki);
    }
}

// Sampler::sample over the logits L[0, n) with the penalty window R (R::n
// ids, R::at(j) in window order); returns the token (in every thread). With
// PRE the row is already penalised and divided by the temperature (the chunk
// kernel did it). The passes run over `row` (Row::load takes L), which ends
// holding the probabilities, written back to L as the reference leaves them.
template <class Row, bool PRE, class R>
__device__ __forceinline__ int sample_body(float* L, int n, const R& recent, const SampleArgs& c, unsigned long long* rng,
                           Shared& sh) {
    const int tid = threadIdx.x;
    const int nr = recent.n;
    // 1. penalties, sampler.rs:104-118, 219-257 (each distinct token once)
    if (!PRE && nr > 0 && penalties_on(c)) {
        for (int q = tid; q < nr && q < kWinLds; q += kST) sh.rec[q] = recent.at(q);
        __syncthreads();
        auto rat = [&](int q) { return q < kWinLds ? sh.rec[q] : recent.at(q); };
        for (int q = tid; q < nr; q += kST) {
            const uint32_t t = rat(q);
            bool first = t < (uint32_t)n;
            for (int k = 0; k < q && first; k++) first = rat(k) != t;
            if (first) {
                int count = 0;
                for (int k = 0; k < nr; k++) count += rat(k) == t;
                L[t] = penalise(L[t], count, c);
            }
        }
        __syncthreads();
    }
    Row row;
    row.load(L, n);
    // 2. zero temperature: greedy, penalties honoured (sampler.rs:120-123)
    if (c.temperature <= 0.0f) return bargmax(row, sh);
    // 3. temperature (sampler.rs:279-285)
    if (!PRE) {
        const float inv_t = 1.0f / c.temperature;
        row.each([&](int, float& x) { x *= inv_t; });
    }
    return sample_tail(row, L, n, c, rng, sh);
}

template <bool PRE, class R>
__device__ __forceinline__ int sample_row(float* L, int n, const R& recent, const SampleArgs& c,
                                          unsigned long long* rng, Shared& sh) {
    return sample_body<MemRow, PRE>(L, n, recent, c, rng, sh);
}

struct FlatRecent {
    const uint32_t* p;
    int n;
    __device__ __forceinline__ uint32_t at(int j) const { return p[j]; }
};

// ------------------------------------------------------------- split path

// The last `window` tokens a sequence generated, from the step history
// (history[step * stride + seq]).
struct HistRecent {
    const uint32_t* h;
    int stride, first, n;
    __device__ __forceinline__ uint32_t at(int j) const { return h[(size_t)(first + j) * stride]; }
};

// Where a row's penalty window comes from: row b's n ids at p + b * stride
// (FlatSrc), or the last `window` generated tokens of sequence seq0 + b
// (HistSrc).
struct FlatSrc {
    const uint32_t* p;
    int n;
    int64_t stride;
    __device__ __forceinline__ FlatRecent at(int b) const { return FlatRecent{p ? p + (size_t)b * stride : p, p ? n : 0}; }
};
struct HistSrc {
    const uint32_t* history;
    int hstride, seq0, window;
    const int* step;
    __device__ __forceinline__ HistRecent at(int b) const {
        const int st = *step, nr = st < window ? st : window;
        return HistRecent{history + seq0 + b, hstride, st - nr, nr};
    }
};

struct ChunkShared {
    float x[kCC];
    uint32_t rec[kWinLds];
    unsigned hist[256];
    unsigned wtot[kCW];
    float wf[kCW];
    int wi[kCW];
    uint32_t bin;
    unsigned above;
};

// The split path's chunk kernel: chunk blockIdx.x (kCC logits) of row
// blockIdx.y. Applies the first-step end-of-sequence suppression (eos, when
// *step == 0), the penalties of the ids in the chunk and the temperature,
// writes the chunk back, then hands on (mode kModeTopK) every finite logit
// with fewer than k larger finite ones in the chunk, in index order, or
// (kModeGreedy) the chunk's first maximum. ccount = the candidates handed on,
// -1 if more than kCapC.
template <class Src>
__global__ void __launch_bounds__(kCT) sample_chunk_kernel(float* logits, int64_t lstride, int n, Src src,
                                                           mivi::SampleEos eos, const int* step, SampleArgs c,
                                                           int mode, float* cval, int* cidx, int* ccount) {
    __shared__ ChunkShared sh;
    const int t = threadIdx.x, ci = blockIdx.x, b = blockIdx.y, nch = gridDim.x;
    float* L = logits + (int64_t)b * lstride;
    const int c0 = ci * kCC, cn = min(kCC, n - c0), i0 = 4 * t;
    const bool vec = ((uintptr_t)(L + c0) & 15) == 0 && i0 + 3 < cn;
    float x[4];
    if (vec) {
        const f32x4 v = *(const f32x4*)(L + c0 + i0);
        x[0] = v.x; x[1] = v.y; x[2] = v.z; x[3] = v.w;
    } else {
#pragma unroll
        for (int e = 0; e < 4; e++) x[e] = i0 + e < cn ? L[c0 + i0 + e] : -INFINITY;
    }
    const auto recent = src.at(b);
    const int nr = recent.n;
    const bool pen = nr > 0 && penalties_on(c);
    const bool eos0 = step && eos.n > 0 && *step == 0;
    if (pen || eos0) {
#pragma unroll
        for (int e = 0; e < 4; e++) sh.x[i0 + e] = x[e];
        for (int q = t; pen && q < nr && q < kWinLds; q += kCT) sh.rec[q] = recent.at(q);
        __syncthreads();
        // the generation loop (model.rs:1141-1160) suppresses them before sampling
        if (eos0 && t < eos.n && eos.id[t] >= (uint32_t)c0 && eos.id[t] < (uint32_t)(c0 + cn))
            sh.x[eos.id[t] - c0] = -INFINITY;
        __syncthreads();
        if (pen) {
            auto rat = [&](int q) { return q < kWinLds ? sh.rec[q] : recent.at(q); };
            for (int q = t; q < nr; q += kCT) {
                const uint32_t tk = rat(q);
                bool first = tk >= (uint32_t)c0 && tk < (uint32_t)(c0 + cn);
                for (int k = 0; k < q && first; k++) first = rat(k) != tk;
                if (first) {
                    int count = 0;
                    for (int k = 0; k < nr; k++) count += rat(k) == tk;
                    sh.x[tk - c0] = penalise(sh.x[tk - c0], count, c);
                }
            }
            __syncthreads();
        }
#pragma unroll
        for (int e = 0; e < 4; e++) x[e] = i0 + e < cn ? sh.x[i0 + e] : -INFINITY;
    }
    if (c.temperature > 0.0f) {
        const float inv_t = 1.0f / c.temperature;
#pragma unroll
        for (int e = 0; e < 4; e++) x[e] *= inv_t;
    }
    if (vec) {
        *(f32x4*)(L + c0 + i0) = f32x4{x[0], x[1], x[2], x[3]};
    } else {
#pragma unroll
        for (int e = 0; e < 4; e++)
            if (i0 + e < cn) L[c0 + i0 + e] = x[e];
    }
    if (mode == kModeRow) return;
    const size_t base = ((size_t)b * nch + ci) * kCapC;
    if (mode == kModeCat) {
        // the chunk's largest finite logit (cval[base]) for the softmax maximum
        float m = -INFINITY;
#pragma unroll
        for (int e = 0; e < 4; e++)
            if (i0 + e < cn && isfinite(x[e])) m = fmaxf(m, x[e]);
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
        if ((t & 63) == 0) sh.wf[t >> 6] = m;
        __syncthreads();
        if (t == 0) {
            for (int w = 1; w < kCW; w++) m = fmaxf(m, sh.wf[w]);
            cval[base] = m;
        }
        return;
    }
    if (mode == kModeGreedy) {
        // the chunk's first maximum above -inf (sampler.rs:305-316)
        float best = -INFINITY;
        int idx = 0x7FFFFFFF;
#pragma unroll
        for (int e = 0; e < 4; e++)
            if (i0 + e < cn && x[e] > best) { best = x[e]; idx = i0 + e; }
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) {
            const float ov = __shfl_xor(best, o, 64);
            const int oi = __shfl_xor(idx, o, 64);
            if (ov > best || (ov == best && oi < idx)) { best = ov; idx = oi; }
        }
        if ((t & 63) == 0) { sh.wf[t >> 6] = best; sh.wi[t >> 6] = idx; }
        __syncthreads();
        if (t == 0) {
            for (int w = 1; w < kCW; w++)
                if (sh.wf[w] > best || (sh.wf[w] == best && sh.wi[w] < idx)) { best = sh.wf[w]; idx = sh.wi[w]; }
            const bool found = best > -INFINITY;
            if (found) { cval[base] = best; cidx[base] = c0 + idx; }
            ccount[(size_t)b * nch + ci] = found ? 1 : 0;
        }
        return;
    }
    // kModeTopK: the chunk's k-th largest finite key K (0 when at most k are finite)
    const unsigned k = (unsigned)c.top_k;
    uint32_t key[4];
    bool ok[4];
    unsigned nf = 0;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        ok[e] = i0 + e < cn && isfinite(x[e]);
        key[e] = ok[e] ? fkey(x[e]) : 0u;
        nf += ok[e];
    }
    unsigned nfin;
    bscan_excl<kCW>(nf, &nfin, sh.wtot);
    uint32_t K = 0;
    if (nfin > k) {
        uint32_t prefix = 0, pmask = 0;
        unsigned above = 0;
        for (int pass = 0; pass < 4; pass++) {
            const int shf = 24 - 8 * pass;
            sh.hist[t] = 0;
            __syncthreads();
#pragma unroll
            for (int e = 0; e < 4; e++)
                hist_add(sh.hist, (key[e] >> shf) & 255u, 1u, ok[e] && (key[e] & pmask) == prefix);
            __syncthreads();
            if (t < 64) select_bin(sh.hist, above, k, &sh.bin, &sh.above);
            __syncthreads();
            prefix |= sh.bin << shf;
            pmask |= 0xFFu << shf;
            above = sh.above;
            __syncthreads();
        }
        K = prefix;
    }
    unsigned mine = 0;
#pragma unroll
    for (int e = 0; e < 4; e++) mine += ok[e] && key[e] >= K;
    unsigned total;
    unsigned pos = bscan_excl<kCW>(mine, &total, sh.wtot);
    if (total > (unsigned)kCapC) {
        if (t == 0) ccount[(size_t)b * nch + ci] = -1;
        return;
    }
#pragma unroll
    for (int e = 0; e < 4; e++)
        if (ok[e] && key[e] >= K) {
            cval[base + pos] = x[e];
            cidx[base + pos] = c0 + i0 + e;
            pos++;
        }
    if (t == 0) ccount[(size_t)b * nch + ci] = (int)total;
}

// Categorical sampling without top-k / top-p (kModeCat), split over the
// chunks. sample_cat_exp_kernel: M = the row's largest finite logit (the
// chunks' maxima), min-p against it (sampler.rs:260-276), e = exp(x - M)
// written over the chunk and the chunk's sum (cval[base + 1]); a row with no
// finite logit takes e = 1 (the softmax's uniform branch, math.rs:43-48).
// sample_cat_prob_kernel: S = the chunk sums in chunk order, p = e * (1/S)
// written over the chunk (the probabilities the reference leaves) and the
// chunk's 2^-40 fixed-point mass (cidx[base], [base + 1] as a u64). The
// row's maximum and sum are block reductions over the chunk values with a
// fixed tree, so every workgroup of the row gets the same M and S.
template <class T, class Op>
__device__ __forceinline__ T chunk_reduce(T v, T* w, Op op) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = op(v, __shfl_xor(v, o, 64));
    if ((threadIdx.x & 63) == 0) w[threadIdx.x >> 6] = v;
    __syncthreads();
    T r = w[0];
#pragma unroll
    for (int k = 1; k < kCW; k++) r = op(r, w[k]);
    __syncthreads();
    return r;
}

__global__ void __launch_bounds__(kCT) sample_cat_exp_kernel(float* logits, int64_t lstride, int n, SampleArgs c,
                                                             float* cval) {
    __shared__ float wf[kCW];
    const int t = threadIdx.x, ci = blockIdx.x, b = blockIdx.y, nch = gridDim.x;
    float* L = logits + (int64_t)b * lstride;
    const int c0 = ci * kCC, cn = min(kCC, n - c0), i0 = 4 * t;
    auto fmax_op = [](float u, float v) { return fmaxf(u, v); };
    auto fadd_op = [](float u, float v) { return u + v; };
    float M = -INFINITY;
    for (int j = t; j < nch; j += kCT) M = fmaxf(M, cval[((size_t)b * nch + j) * kCapC]);
    M = chunk_reduce(M, wf, fmax_op);
    const bool uniform = !isfinite(M);
    const float thr = (c.min_p > 0.0f && c.min_p < 1.0f) ? M + c.ln_min_p : -INFINITY;
    float s = 0.0f;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int i = c0 + i0 + e;
        if (i0 + e < cn) {
            const float x = L[i];
            const float y = uniform ? 1.0f : (isfinite(x) && !(x < thr)) ? expf(x - M) : 0.0f;
            L[i] = y;
            s += y;
        }
    }
    s = chunk_reduce(s, wf, fadd_op);
    if (t == 0) cval[((size_t)b * nch + ci) * kCapC + 1] = s;
}

__global__ void __launch_bounds__(kCT) sample_cat_prob_kernel(float* logits, int64_t lstride, int n, float* cval,
                                                              int* cidx) {
    __shared__ unsigned long long wsum[kCW];
    __shared__ float wf[kCW];
    const int t = threadIdx.x, ci = blockIdx.x, b = blockIdx.y, nch = gridDim.x;
    float* L = logits + (int64_t)b * lstride;
    const int c0 = ci * kCC, cn = min(kCC, n - c0), i0 = 4 * t;
    float S = 0.0f;
    for (int j = t; j < nch; j += kCT) S += cval[((size_t)b * nch + j) * kCapC + 1];
    S = chunk_reduce(S, wf, [](float u, float v) { return u + v; });
    const float inv = 1.0f / S;
    unsigned long long w = 0;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int i = c0 + i0 + e;
        if (i0 + e < cn) {
            const float p = L[i] * inv;
            L[i] = p;
            w += fixp(p);
        }
    }
    w = chunk_reduce(w, wsum, [](unsigned long long u, unsigned long long v) { return u + v; });
    if (t == 0) *(unsigned long long*)(cidx + ((size_t)b * nch + ci) * kCapC) = w;
}

// Where a row's token goes: tok[b], and the step history of sequence seq0 + b
// when history is set.
struct TokOut {
    uint32_t* tok;
    uint32_t* history;
    int hstride, seq0;
    const int* step;
    mivi::EmbedNext en;  // with a table: the token's embedding for the next step
};

struct NoRecent {
    static constexpr int n = 0;
    __device__ __forceinline__ uint32_t at(int) const { return 0; }
};

// The split path's pick kernel: row blockIdx.x from its chunks' candidates
// (the whole transformed row when they do not fit), probabilities written
// back to the row when `write`.
__global__ void __launch_bounds__(kST) sample_pick_kernel(float* logits, int64_t lstride, int n, int nch,
                                                          SampleArgs c, int mode, const float* cval, const int* cidx,
                                                          const int* ccount, unsigned long long* rng, TokOut out,
                                                          int write) {
    __shared__ Shared sh;
    const int t = threadIdx.x, b = blockIdx.x;
    float* L = logits + (int64_t)b * lstride;
    if (mode == kModeCat) {
        // 7b. categorical (sampler.rs:137-148) over the probabilities the
        // chunk kernels left: the chunk where the fixed-point mass reaches
        // r, then the index inside it
        const float r = draw(rng + b, sh);
        const unsigned long long tr = (unsigned long long)ceil((double)r * kFix);
        const unsigned long long cm =
            t < nch ? *(const unsigned long long*)(cidx + ((size_t)b * nch + t) * kCapC) : 0ull;
        unsigned long long tot;
        const unsigned long long ex = bscan_excl<kSW, unsigned long long>(cm, &tot, sh.wsum);
        if (t == 0) sh.bin = 0;
        __syncthreads();
        if (t < nch && cm && ex < tr && tr <= ex + cm) {
            sh.bin = (uint32_t)t;
            sh.above = ex;
        }
        __syncthreads();
        int tok;
        if (tr == 0 || n == 0) {
            tok = 0;
        } else if (tot < tr) {
            tok = n - 1;
        } else {
            const int cc = (int)sh.bin, c0 = cc * kCC, cn = min(kCC, n - c0);
            const unsigned long long tr2 = tr - sh.above;
            const unsigned long long wv = t < cn ? fixp(L[c0 + t]) : 0ull;
            unsigned long long tot2;
            const unsigned long long ex2 = bscan_excl<kSW, unsigned long long>(wv, &tot2, sh.wsum);
            if (wv && ex2 < tr2 && tr2 <= ex2 + wv) sh.bin = (uint32_t)(c0 + t);
            __syncthreads();
            tok = (int)sh.bin;
        }
        if (t == 0) {
            out.tok[b] = (uint32_t)tok;
            if (out.history) out.history[(size_t)(*out.step) * out.hstride + out.seq0 + b] = (uint32_t)tok;
        }
        if (out.en.table)
            mivi::embed_row(out.en.type, out.en.table, out.en.row_bytes, (uint32_t)tok, out.en.x + b * out.en.xs,
                            out.en.dim, t, kST);
        return;
    }
    bool fast = mode != kModeRow;
    int M = 0;
    if (fast) {
        const int cnt = t < nch ? ccount[(size_t)b * nch + t] : 0;
        const bool ovf = __syncthreads_or(cnt < 0);
        unsigned long long tot;
        const unsigned long long ex = bscan_excl<kSW, unsigned long long>(cnt > 0 ? cnt : 0, &tot, sh.wsum);
        if (t < nch) sh.off[t] = (int)ex;
        if (t == 0) sh.off[nch] = (int)tot;
        __syncthreads();
        M = (int)tot;
        fast = !ovf && M > 0 && M <= kCapB;
    }
    int tok;
    if (!fast) {
        tok = sample_row<true>(L, n, NoRecent{}, c, rng + b, sh);
    } else {
        CandRow row;
        row.load(cval, cidx, (size_t)b * nch * kCapC, sh.off, nch, M, n, write != 0);
        tok = mode == kModeGreedy ? bargmax(row, sh) : sample_tail(row, L, n, c, rng + b, sh);
    }
    if (t == 0) {
        out.tok[b] = (uint32_t)tok;
        if (out.history) out.history[(size_t)(*out.step) * out.hstride + out.seq0 + b] = (uint32_t)tok;
    }
    if (out.en.table)  // every thread holds the token
        mivi::embed_row(out.en.type, out.en.table, out.en.row_bytes, (uint32_t)tok, out.en.x + b * out.en.xs,
                        out.en.dim, t, kST);
}

SampleArgs make_args(const mivi_sampler_config& cfg) {
    SampleArgs a;
    a.temperature = cfg.temperature;
    a.top_p = cfg.top_p;
    a.min_p = cfg.min_p;
    a.ln_min_p = (cfg.min_p > 0.0f && cfg.min_p < 1.0f) ? logf(cfg.min_p) : 0.0f;  // sampler.rs:270 min_p.ln()
    a.rep = cfg.repetition_penalty;
    a.presence = cfg.presence_penalty;
    a.frequency = cfg.frequency_penalty;
    a.top_k = cfg.top_k > (uint32_t)INT32_MAX ? INT32_MAX : (int)cfg.top_k;
    return a;
}

size_t n_chunks(size_t n) { return std::max<size_t>(1, (n + kCC - 1) / kCC); }

size_t split_workspace(size_t n, size_t rows) {
    const size_t cand = rows * n_chunks(n) * kCapC;
    return ((cand * 8 + rows * n_chunks(n) * 4) + 255) & ~(size_t)255;
}

template <class Src>
int32_t launch_split(float* logits, int64_t lstride, int n, int rows, const Src& src, const mivi::SampleEos& eos,
                     const int* step, const mivi_sampler_config& cfg, uint64_t* rng, const TokOut& out, void* ws,
                     bool write, hipStream_t s) {
    const SampleArgs a = make_args(cfg);
    const int nch = (int)n_chunks((size_t)n);
    int mode = kModeRow;
    if (nch <= kMaxChunks) {
        if (a.temperature <= 0.0f) mode = kModeGreedy;
        else if (a.top_k > 0 && a.top_k <= kKMax && a.top_k < n) mode = kModeTopK;
        else if ((a.top_k <= 0 || a.top_k >= n) && !(a.top_p < 1.0f) && n > 0) mode = kModeCat;
    }
    float* cval = (float*)ws;
    int* cidx = (int*)(cval + (size_t)rows * nch * kCapC);
    int* ccount = cidx + (size_t)rows * nch * kCapC;
    hipLaunchKernelGGL(sample_chunk_kernel<Src>, dim3((unsigned)nch, (unsigned)rows), dim3(kCT), 0, s, logits, lstride,
                       n, src, eos, step, a, mode, cval, cidx, ccount);
    MIVI_HIP_CHECK(hipGetLastError());
    if (mode == kModeCat) {
        hipLaunchKernelGGL(sample_cat_exp_kernel, dim3((unsigned)nch, (unsigned)rows), dim3(kCT), 0, s, logits, lstride,
                           n, a, cval);
        hipLaunchKernelGGL(sample_cat_prob_kernel, dim3((unsigned)nch, (unsigned)rows), dim3(kCT), 0, s, logits,
                           lstride, n, cval, cidx);
        MIVI_HIP_CHECK(hipGetLastError());
    }
    hipLaunchKernelGGL(sample_pick_kernel, dim3((unsigned)rows), dim3(kST), 0, s, logits, lstride, n, nch, a, mode,
                       cval, cidx, ccount, (unsigned long long*)rng, out, write ? 1 : 0);
    MIVI_HIP_CHECK(hipGetLastError());
    return MIVI_OK;
}

}  // namespace

namespace mivi {
size_t sample_seq_workspace(size_t n, size_t batch) { return split_workspace(n, batch); }

int32_t launch_sample_seq(float* logits, int64_t lstride, int n, uint32_t* history, int hstride, int seq0, int batch,
                          int window, const int* step, const SampleEos& eos, const mivi_sampler_config& cfg,
                          uint64_t* rng, uint32_t* tok, void* ws, const EmbedNext& en, hipStream_t s) {
    return launch_split(logits, lstride, n, batch, HistSrc{history, hstride, seq0, window, step}, eos, step, cfg, rng,
                        TokOut{tok, history, hstride, seq0, step, en}, ws, false, s);
}
}  // namespace mivi

// -------------------------------------------------------------------- C ABI

// The workspace of mivi_hip_sample (one row of the split path): one
// grow-only buffer per device, kept until the process ends; calls on
// different streams are ordered through an event recorded after each use.
struct SampleWorkspace {
    std::mutex mu;
    void* ptr = nullptr;
    size_t bytes = 0;
    hipEvent_t done = nullptr;
};

static SampleWorkspace& sample_workspace(int dev) {
    static std::mutex mu;
    static std::vector<SampleWorkspace*> all;
    std::lock_guard<std::mutex> lk(mu);
    if ((size_t)dev >= all.size()) all.resize(dev + 1, nullptr);
    if (!all[dev]) all[dev] = new SampleWorkspace();
    return *all[dev];
}

extern "C" int32_t mivi_hip_sample(float* logits, size_t n, const uint32_t* recent, size_t n_recent,
                                   const mivi_sampler_config* cfg, uint64_t* rng_state, uint32_t* token,
                                   void* stream) {
    if (!cfg || !rng_state || !token || (n && !logits) || (n_recent && !recent))
        return mivi::set_error(MIVI_ERR_INVALID_ARGUMENT, "null argument");
    if (n > (size_t)INT32_MAX || n_recent > (size_t)INT32_MAX) return mivi::err_overflow();
    mivi::clear_error();
    hipStream_t s = (hipStream_t)stream;
    int dev = 0;
    MIVI_HIP_CHECK(hipGetDevice(&dev));
    SampleWorkspace& ws = sample_workspace(dev);
    std::lock_guard<std::mutex> lk(ws.mu);
    if (!ws.done) MIVI_HIP_CHECK(hipEventCreateWithFlags(&ws.done, hipEventDisableTiming));
    else MIVI_HIP_CHECK(hipStreamWaitEvent(s, ws.done, 0));  // the previous user is done with it
    const size_t need = split_workspace(n, 1);
    if (ws.bytes < need) {
        if (ws.ptr) {
            MIVI_HIP_CHECK(hipEventSynchronize(ws.done));
            MIVI_HIP_CHECK(hipFree(ws.ptr));
            ws.ptr = nullptr;
            ws.bytes = 0;
        }
        MIVI_HIP_CHECK(hipMalloc(&ws.ptr, need));
        ws.bytes = need;
    }
    const int32_t rc = launch_split(logits, (int64_t)n, (int)n, 1,
                                    FlatSrc{n_recent ? recent : nullptr, (int)n_recent, 0}, mivi::SampleEos{},
                                    nullptr, *cfg, rng_state, TokOut{token, nullptr, 0, 0, nullptr, mivi::EmbedNext{}},
                                    ws.ptr, true, s);
    MIVI_HIP_CHECK(hipEventRecord(ws.done, s));
    return rc;
}

// mivi_hip_sample_noalloc: the split path's workspace for one row of at most
// kNoAllocMaxN logits lives in this file-scope device array, one copy per
// GPU, held until the process ends (513 KB). In host code `scratch` names a
// host-side stand-in, not device memory: the device address of each GPU's
// copy comes from hipGetSymbolAddress, resolved once per device (with that
// device current) and kept in g_scratch_dev. Every call on a GPU shares its
// copy, so calls that overlap on one GPU (different streams, threads) race.
// The kernels write every workspace word they later read within one call,
// so nothing needs clearing between calls.
constexpr size_t kNoAllocMaxN = 262144;
constexpr size_t kNoAllocScratchBytes =
    ((kNoAllocMaxN + kCC - 1) / kCC * kCapC * 8 + (kNoAllocMaxN + kCC - 1) / kCC * 4 + 255) & ~(size_t)255;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

constexpr int kNoAllocMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_dev[kNoAllocMaxDevices];  // device address of `scratch` per GPU, null until resolved

static int32_t noalloc_scratch(int dev, void** out) {
    if (dev < 0 || dev >= kNoAllocMaxDevices)
        return mivi::set_error(MIVI_ERR_INVALID_ARGUMENT, "device %d beyond the %d the scratch table holds", dev,
                               kNoAllocMaxDevices);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_dev[dev]) {
        void* p = nullptr;
        MIVI_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (!p) return mivi::set_error(MIVI_ERR_HIP, "hipGetSymbolAddress returned no address for the scratch");
        g_scratch_dev[dev] = p;
    }
    *out = g_scratch_dev[dev];
    return MIVI_OK;
}

extern "C" int32_t mivi_hip_sample_noalloc(float* logits, size_t n, const uint32_t* recent, size_t n_recent,
                                           const mivi_sampler_config* cfg, uint64_t* rng_state, uint32_t* token,
                                           void* stream) {
    if (!cfg || !rng_state || !token || (n && !logits) || (n_recent && !recent))
        return mivi::set_error(MIVI_ERR_INVALID_ARGUMENT, "null argument");
    if (n > kNoAllocMaxN)
        return mivi::set_error(MIVI_ERR_INVALID_ARGUMENT,
                               "%zu logits: mivi_hip_sample_noalloc takes at most %zu (its scratch is fixed)", n,
                               kNoAllocMaxN);
    if (n_recent > (size_t)INT32_MAX) return mivi::err_overflow();
    if (split_workspace(n, 1) > kNoAllocScratchBytes)
        return mivi::set_error(MIVI_ERR_INVALID_ARGUMENT, "scratch too small for %zu logits", n);
    mivi::clear_error();
    int dev = 0;
    MIVI_HIP_CHECK(hipGetDevice(&dev));
    void* ws = nullptr;
    int32_t rc = noalloc_scratch(dev, &ws);
    if (rc) return rc;
    return launch_split(logits, (int64_t)n, (int)n, 1, FlatSrc{n_recent ? recent : nullptr, (int)n_recent, 0},
                        mivi::SampleEos{}, nullptr, *cfg, rng_state,
                        TokOut{token, nullptr, 0, 0, nullptr, mivi::EmbedNext{}}, ws, true, (hipStream_t)stream);
}

extern "C" size_t mivi_hip_sample_rows_workspace(size_t n, size_t rows) { return split_workspace(n, rows); }

extern "C" int32_t mivi_hip_sample_rows(float* logits, size_t n, size_t rows, size_t row_stride,
                                        const uint32_t* recent, size_t n_recent, size_t recent_stride,
                                        const mivi_sampler_config* cfg, uint64_t* rng_states, uint32_t* tokens,
                                        void* workspace, size_t workspace_bytes, void* stream) {
    if (!cfg || !rng_states || !tokens || !workspace || (n && !logits) || (n_recent && !recent))
        return mivi::set_error(MIVI_ERR_INVALID_ARGUMENT, "null argument");
    if (rows == 0) return mivi::clear_error();
    if (n > (size_t)INT32_MAX || n_recent > (size_t)INT32_MAX || rows > 65535 || row_stride > (size_t)INT64_MAX ||
        recent_stride > (size_t)INT64_MAX)
        return mivi::err_overflow();
    if (rows > 1 && row_stride < n) return mivi::set_error(MIVI_ERR_INVALID_ARGUMENT, "row_stride %zu < n %zu", row_stride, n);
    if (rows > 1 && n_recent && recent_stride < n_recent)
        return mivi::set_error(MIVI_ERR_INVALID_ARGUMENT, "recent_stride %zu < n_recent %zu", recent_stride, n_recent);
    if (workspace_bytes < split_workspace(n, rows))
        return mivi::set_error(MIVI_ERR_INVALID_ARGUMENT, "workspace of %zu bytes, %zu needed", workspace_bytes,
                               split_workspace(n, rows));
    // the categorical path keeps 64-bit chunk masses in the workspace
    if ((uintptr_t)workspace & 7) return mivi::set_error(MIVI_ERR_INVALID_ARGUMENT, "workspace not 8-byte aligned");
    mivi::clear_error();
    return launch_split(logits, (int64_t)row_stride, (int)n, (int)rows,
                        FlatSrc{n_recent ? recent : nullptr, (int)n_recent, (int64_t)recent_stride}, mivi::SampleEos{},
                        nullptr, *cfg, rng_states, TokOut{tokens, nullptr, 0, 0, nullptr, mivi::EmbedNext{}}, workspace, true,
                        (hipStream_t)stream);
}
