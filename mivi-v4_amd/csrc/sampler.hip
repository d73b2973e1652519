// Sampler::sample (crates/mivi-model/src/sampler.rs:91-135) on the device:
// penalties, temperature, min-p, top-k, softmax, then top-p or categorical
// sampling with the reference's xorshift64* generator, in one workgroup, with
// the logits modified in place as the reference modifies its &mut [f32].
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

#include "common.h"

namespace {

constexpr int kST = 1024;                 // threads of the sampling workgroup
constexpr int kSW = kST / 64;             // its waves
constexpr double kFix = 1099511627776.0;  // 2^40

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

struct Shared {
    unsigned long long hist[256];
    unsigned long long wsum[kSW];
    float wf[kSW];
    int wi[kSW];
    uint32_t bin;
    unsigned long long above;
    float r;
    int found;
};

__device__ float bmax_finite_of(const float* L, int n, Shared& sh) {
    float m = -INFINITY;
    for (int i = threadIdx.x; i < n; i += kST) {
        const float v = L[i];
        if (isfinite(v) && v > m) m = v;
    }
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
__device__ float bsum_f(float v, Shared& sh) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    if ((threadIdx.x & 63) == 0) sh.wf[threadIdx.x >> 6] = v;
    __syncthreads();
    float s = sh.wf[0];
    for (int w = 1; w < kSW; w++) s += sh.wf[w];
    __syncthreads();
    return s;
}

__device__ unsigned long long bsum_u(unsigned long long v, Shared& sh) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    if ((threadIdx.x & 63) == 0) sh.wsum[threadIdx.x >> 6] = v;
    __syncthreads();
    unsigned long long s = 0;
    for (int w = 0; w < kSW; w++) s += sh.wsum[w];
    __syncthreads();
    return s;
}

// sampler.rs:305-316: first index of the strict maximum (0 if none)
__device__ int bargmax(const float* L, int n, Shared& sh) {
    float best = -INFINITY;
    int idx = 0x7FFFFFFF;
    for (int i = threadIdx.x; i < n; i += kST) {
        const float v = L[i];
        if (v > best) { best = v; idx = i; }
    }
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
    return idx == 0x7FFFFFFF ? 0 : idx;
}

// The largest key K whose active elements with key >= K weigh at least
// `target` (the caller guarantees the total does); *above = the weight of the
// active elements with key > K. f(i, key, weight) says whether i is active.
template <class F>
__device__ uint32_t radix_search(int n, F f, unsigned long long target, unsigned long long* above_out, Shared& sh) {
    uint32_t prefix = 0, pmask = 0;
    unsigned long long above = 0;
    for (int pass = 0; pass < 4; pass++) {
        const int shf = 24 - 8 * pass;
        for (int b = threadIdx.x; b < 256; b += kST) sh.hist[b] = 0;
        __syncthreads();
        for (int i = threadIdx.x; i < n; i += kST) {
            uint32_t k;
            unsigned long long w;
            if (f(i, k, w) && w && (k & pmask) == prefix) atomicAdd(&sh.hist[(k >> shf) & 255u], w);
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            unsigned long long acc = above;
            int b = 255;
            for (; b > 0; b--) {
                if (acc + sh.hist[b] >= target) break;
                acc += sh.hist[b];
            }
            sh.bin = (uint32_t)b;
            sh.above = acc;
        }
        __syncthreads();
        prefix |= sh.bin << shf;
        pmask |= 0xFFu << shf;
        above = sh.above;
        __syncthreads();
    }
    *above_out = above;
    return prefix;
}

// Exclusive prefix over the threads (thread order) of a per-thread value.
template <class T>
__device__ T bscan_excl(T v, T* total, Shared& sh, T* wtot) {
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
    for (int w = 0; w < kSW; w++) {
        if (w < wave) before += wtot[w];
        all += wtot[w];
    }
    __syncthreads();
    *total = all;
    return before + inc - v;
}

// Index of the j-th (1-based) element in index order with match(i) true;
// -1 if there are fewer. Threads own contiguous chunks.
template <class M>
__device__ int find_nth(int n, M match, unsigned long long j, Shared& sh) {
    const int chunk = (n + kST - 1) / kST, b0 = min(n, threadIdx.x * chunk), b1 = min(n, b0 + chunk);
    unsigned long long c = 0;
    for (int i = b0; i < b1; i++) c += match(i) ? 1 : 0;
    unsigned long long total;
    const unsigned long long ex = bscan_excl<unsigned long long>(c, &total, sh, sh.wsum);
    if (threadIdx.x == 0) sh.found = -1;
    __syncthreads();
    if (ex < j && j <= ex + c) {
        unsigned long long k = ex;
        for (int i = b0; i < b1; i++)
            if (match(i) && ++k == j) { sh.found = i; break; }
    }
    __syncthreads();
    const int r = sh.found;
    __syncthreads();
    return r;
}

// sampler.rs:70-77 (thread 0), broadcast
__device__ float draw(unsigned long long* rng, Shared& sh) {
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

__global__ void __launch_bounds__(kST) sample_kernel(float* L, int n, const uint32_t* recent, int nr, SampleArgs c,
                                                     unsigned long long* rng, uint32_t* tok_out) {
    __shared__ Shared sh;
    const int tid = threadIdx.x;
    // 1. penalties, sampler.rs:104-118, 219-257 (each distinct token once)
    if (nr > 0 && ((c.rep > 0.0f && c.rep != 1.0f) || c.presence != 0.0f || c.frequency != 0.0f)) {
        for (int q = tid; q < nr; q += kST) {
            const uint32_t t = recent[q];
            bool first = t < (uint32_t)n;
            for (int k = 0; k < q && first; k++) first = recent[k] != t;
            if (first) {
                int count = 0;
                for (int k = 0; k < nr; k++) count += recent[k] == t;
                float v = L[t];
                if (c.rep > 0.0f && c.rep != 1.0f) v = v > 0.0f ? v / c.rep : v * c.rep;
                if (c.presence != 0.0f) v -= c.presence;
                if (c.frequency != 0.0f) v -= c.frequency * (float)count;
                L[t] = v;
            }
        }
        __syncthreads();
    }
    // 2. zero temperature: greedy, penalties honoured (sampler.rs:120-123)
    if (c.temperature <= 0.0f) {
        const int i = bargmax(L, n, sh);
        if (tid == 0) *tok_out = (uint32_t)i;
        return;
    }
    // 3. temperature (sampler.rs:279-285)
    const float inv_t = 1.0f / c.temperature;
    for (int i = tid; i < n; i += kST) L[i] *= inv_t;
    __syncthreads();
    // 4. min-p (sampler.rs:260-276); ln(min_p) comes from the host's libm
    if (c.min_p > 0.0f && c.min_p < 1.0f) {
        const float mx = bmax_finite_of(L, n, sh);
        if (isfinite(mx)) {
            const float thr = mx + c.ln_min_p;
            for (int i = tid; i < n; i += kST)
                if (L[i] < thr) L[i] = -INFINITY;
        }
        __syncthreads();
    }
    // 5. top-k: the k-th largest value is the cutoff (sampler.rs:287-301)
    if (c.top_k > 0 && c.top_k < n) {
        unsigned long long above;
        const uint32_t K = radix_search(
            n, [&](int i, uint32_t& k, unsigned long long& w) { k = fkey(L[i]); w = 1; return true; },
            (unsigned long long)c.top_k, &above, sh);
        const float cutoff = funkey(K);
        for (int i = tid; i < n; i += kST)
            if (L[i] < cutoff) L[i] = -INFINITY;
        __syncthreads();
    }
    // 6. softmax (math.rs:32-72)
    {
        const float mx = bmax_finite_of(L, n, sh);
        if (!isfinite(mx)) {
            const float u = 1.0f / (float)n;
            for (int i = tid; i < n; i += kST) L[i] = u;
        } else {
            float s = 0.0f;
            for (int i = tid; i < n; i += kST) {
                const float v = L[i];
                if (isfinite(v)) {
                    const float e = expf(v - mx);
                    L[i] = e;
                    s += e;
                } else {
                    L[i] = 0.0f;
                }
            }
            const float sum = bsum_f(s, sh);
            if (sum > 0.0f) {
                const float inv = 1.0f / sum;
                for (int i = tid; i < n; i += kST) L[i] *= inv;
            } else {
                const float u = 1.0f / (float)n;
                for (int i = tid; i < n; i += kST) L[i] = u;
            }
        }
        __syncthreads();
    }
    if (c.top_p < 1.0f) {
        // 7a. top-p (sampler.rs:150-215)
        const float cutoff = n > 1 ? (1.0f - c.top_p) / ((float)n - 1.0f) : 0.0f;
        auto cand = [&](int i) {
            const float p = L[i];
            return p >= cutoff && p > 0.0f && isfinite(p);
        };
        unsigned long long nc = 0, wt = 0;
        for (int i = tid; i < n; i += kST)
            if (cand(i)) { nc++; wt += fixp(L[i]); }
        nc = bsum_u(nc, sh);
        wt = bsum_u(wt, sh);
        if (nc == 0) {
            const int i = bargmax(L, n, sh);
            if (tid == 0) *tok_out = (uint32_t)i;
            return;
        }
        auto fc = [&](int i, uint32_t& k, unsigned long long& w) {
            if (!cand(i)) return false;
            k = fkey(L[i]);
            w = fixp(L[i]);
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
            const uint32_t Ks = radix_search(n, fc, tgt, &above, sh);
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
        const uint32_t Kr = radix_search(n, fc, tr, &above_r, sh);
        const unsigned long long wr = fixp(funkey(Kr));
        const unsigned long long j = (tr - above_r + wr - 1) / wr;
        const int i = find_nth(n, [&](int q) { return cand(q) && fkey(L[q]) == Kr; }, j, sh);
        if (tid == 0) *tok_out = (uint32_t)(i >= 0 ? i : 0);
    } else {
        // 7b. categorical (sampler.rs:137-148): first index whose cumulative
        // probability reaches r
        const float r = draw(rng, sh);
        const unsigned long long tr = (unsigned long long)ceil((double)r * kFix);
        const int chunk = (n + kST - 1) / kST, b0 = min(n, tid * chunk), b1 = min(n, b0 + chunk);
        unsigned long long s = 0;
        for (int i = b0; i < b1; i++) s += fixp(L[i]);
        unsigned long long total;
        const unsigned long long ex = bscan_excl<unsigned long long>(s, &total, sh, sh.wsum);
        // r == 0 takes index 0 (its cumulative sum is >= 0); past the total, n - 1
        if (tid == 0) sh.found = tr == 0 ? 0 : n > 0 ? n - 1 : 0;
        __syncthreads();
        if (tr > 0 && ex < tr && tr <= ex + s) {
            unsigned long long acc = ex;
            for (int i = b0; i < b1; i++) {
                acc += fixp(L[i]);
                if (acc >= tr) { sh.found = i; break; }
            }
        }
        __syncthreads();
        if (tid == 0) *tok_out = (uint32_t)sh.found;
    }
}

}  // namespace

// -------------------------------------------------------------------- C ABI

extern "C" int32_t mivi_hip_sample(float* logits, size_t n, const uint32_t* recent, size_t n_recent,
                                   const mivi_sampler_config* cfg, uint64_t* rng_state, uint32_t* token,
                                   void* stream) {
    if (!cfg || !rng_state || !token || (n && !logits) || (n_recent && !recent))
        return mivi::set_error(MIVI_ERR_INVALID_ARGUMENT, "null argument");
    if (n > (size_t)INT32_MAX || n_recent > (size_t)INT32_MAX) return mivi::err_overflow();
    mivi::clear_error();
    SampleArgs a;
    a.temperature = cfg->temperature;
    a.top_p = cfg->top_p;
    a.min_p = cfg->min_p;
    a.ln_min_p = (cfg->min_p > 0.0f && cfg->min_p < 1.0f) ? logf(cfg->min_p) : 0.0f;  // sampler.rs:270 min_p.ln()
    a.rep = cfg->repetition_penalty;
    a.presence = cfg->presence_penalty;
    a.frequency = cfg->frequency_penalty;
    a.top_k = cfg->top_k > (uint32_t)INT32_MAX ? INT32_MAX : (int)cfg->top_k;
    hipLaunchKernelGGL(sample_kernel, dim3(1), dim3(kST), 0, (hipStream_t)stream, logits, (int)n, recent,
                       (int)n_recent, a, (unsigned long long*)rng_state, token);
    MIVI_HIP_CHECK(hipGetLastError());
    return MIVI_OK;
}
