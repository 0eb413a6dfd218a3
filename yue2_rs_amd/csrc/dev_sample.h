// dev_sample.h -- device pieces of choose() (src/sampling.rs:103-215) and of
// the MT19937 stream, shared by the sampler kernels (sampler.hip) and the
// sampler workgroup of the persistent step kernel (step.hip).
#pragma once
#include <hip/hip_runtime.h>

#include "kernels.h"
#include "runtime.h"
#include "sampler.h"
#include "y2_math.h"

namespace y2 {

constexpr int kSurvivorMax = 2048;
constexpr int kWindowMax = 128;  // penalty_window is at most 100
static_assert(kChooseChunk == 1024, "finish_kernel rescans one chunk with its 1024 threads");

__device__ __forceinline__ uint32_t ukey(float f) { return (uint32_t)total_key(f) ^ 0x80000000u; }
__device__ __forceinline__ float from_ukey(uint32_t k) {
    const int32_t b = (int32_t)(k ^ 0x80000000u);
    return u2f((uint32_t)(b < 0 ? b ^ 0x7fffffff : b));
}
__device__ __forceinline__ bool is_finite(float v) {
    return (f2u(v) & 0x7f800000u) != 0x7f800000u;
}
__device__ __forceinline__ float cast(float x, int legacy) { return legacy ? rb(x) : x; }

// Order key of entry i with score v: ascending keys run through the scores
// in descending total order, ties by ascending id (src/sampling.rs:170, 174).
__device__ __forceinline__ uint64_t order_key(float v, int i) {
    return ((uint64_t)(~ukey(v)) << 32) | (uint32_t)i;
}
__device__ __forceinline__ float key_value(uint64_t k) { return from_ukey(~(uint32_t)(k >> 32)); }

__device__ __forceinline__ uint64_t kmin(uint64_t a, uint64_t b) { return a < b ? a : b; }
__device__ __forceinline__ uint64_t shfl_xor64(uint64_t v, int m) {
    const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)v, m, 64);
    const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(v >> 32), m, 64);
    return ((uint64_t)hi << 32) | lo;
}

// compiler-rt __powisf2, which Rust's f32::powi calls for a run-time exponent.
__device__ __forceinline__ float powi_f32(float a, int b) {
    const int recip = b < 0;
    float r = 1.0f;
    for (;;) {
        if (b & 1) r *= a;
        b /= 2;
        if (b == 0) break;
        a *= a;
    }
    return recip ? 1.0f / r : r;
}

// Bitonic sort of n (power of two) 64-bit keys in LDS, ascending.
__device__ __forceinline__ void bitonic_sort(uint64_t* v, int n) {
    for (int size = 2; size <= n; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = threadIdx.x; i < n / 2; i += blockDim.x) {
                const int lo = 2 * i - (i & (stride - 1));
                const int hi = lo + stride;
                const bool up = (lo & size) == 0;
                const uint64_t a = v[lo], b = v[hi];
                if ((a > b) == up) {
                    v[lo] = b;
                    v[hi] = a;
                }
            }
            __syncthreads();
        }
    }
}

// Rank of `key` among v[0, n): the number of entries below it.  The threads
// of a wave read the same entry at each step (LDS broadcasts), four at a time.
__device__ __forceinline__ int rank_below(const uint64_t* v, int n, uint64_t key) {
    int r = 0, j = 0;
    for (; j + 4 <= n; j += 4) {
        const uint64_t a0 = v[j], a1 = v[j + 1], a2 = v[j + 2], a3 = v[j + 3];
        r += (a0 < key) + (a1 < key) + (a2 < key) + (a3 < key);
    }
    for (; j < n; ++j) r += v[j] < key;
    return r;
}

// v[0, n) in ascending order, for n distinct keys (sort keys carry the token
// id).  With at most one entry per thread, each thread moves its entry to its
// rank in tmp (n entries apart from v) and the block copies tmp back: one
// pass of n broadcast reads instead of the log2(n)^2 / 2 barrier-separated
// stages of bitonic_sort, whose order it gives.  Otherwise bitonic_sort over
// the next power of two (v must hold it; the padding is ~0).  Called by the
// whole block.
__device__ __forceinline__ void sort_distinct(uint64_t* v, int n, uint64_t* tmp) {
    const int tid = threadIdx.x, nt = blockDim.x;
    if (n <= nt) {
        const uint64_t mine = tid < n ? v[tid] : 0;
        if (tid < n) tmp[rank_below(v, n, mine)] = mine;
        __syncthreads();
        if (tid < n) v[tid] = tmp[tid];
        __syncthreads();
        return;
    }
    int n2 = 2;
    while (n2 < n) n2 <<= 1;
    for (int i = n + tid; i < n2; i += nt) v[i] = ~0ull;
    __syncthreads();
    bitonic_sort(v, n2);
}

// CFG mix (src/sampling.rs:261-266) and phase mask (:116-129) of entry i.
__device__ __forceinline__ float mixed_score(const SampleArgs& a, int i, int step) {
    const float c = a.logits[i];
    float v = c;
    if (a.rows == 2) {
        const float u = a.logits[(size_t)a.vocab + i];
        v = rb(u + rb(a.cfg_scale * rb(c - u)));
    }
    bool in = true;
    if (a.phase == YUE2_PHASE_ABC) in = i < kEod;
    else if (a.phase == YUE2_PHASE_SEMANTIC) in = i >= kCodecOffset && i < kCodecOffset + kCodecSize;
    if (a.phase != YUE2_PHASE_NONE && i == a.end_id && step >= a.min_tokens) in = true;
    return (a.mode == 0 || in) ? v : -__builtin_huge_valf();
}

// The penalty window: the last penalty_window history ids (:130-131), into
// ids; returns their number.  Ends with a barrier.
__device__ __forceinline__ int load_window(const SampleArgs& a, int step, int32_t* ids) {
    int wn = 0;
    if (a.mode == 1) {
        const int len = a.hist_len >= 0 ? a.hist_len : step;
        const int from = len > a.window ? len - a.window : 0;
        wn = len - from;
        for (int i = threadIdx.x; i < wn; i += blockDim.x) ids[i] = a.history[from + i];
    }
    __syncthreads();
    return wn;
}

// Repetition penalty (:132-144) on the ids in [lo, lo + n), whose scores are
// vals[id - lo]: the first occurrence of each id in the window applies
// alpha^count.  Needs blockDim.x >= wn; ends with a barrier.
__device__ __forceinline__ void apply_penalty(const SampleArgs& a, const int32_t* ids, int wn, float* vals, int lo,
                              int n) {
    const int t = threadIdx.x;
    if (t < wn) {
        const int id = ids[t];
        if (id >= lo && id < lo + n) {
            bool first = true;
            for (int j = 0; j < t; ++j) first &= ids[j] != id;
            if (first) {
                int count = 0;
                for (int j = t; j < wn; ++j) count += ids[j] == id;
                const float alpha = cast(powi_f32(a.repetition_penalty, count), a.legacy);
                const float s = vals[id - lo];
                vals[id - lo] = cast(s < 0.0f ? s * alpha : s / alpha, a.legacy);
            }
        }
    }
    __syncthreads();
}

// The chosen id becomes every row's next input; it is logged at [step] and
// ends the phase when it is the end token.
__device__ __forceinline__ void publish(const SampleArgs& a, int step, int32_t id) {
    StepState* st = a.st;
    for (int b = 0; b < a.rows; ++b) st->ids[b] = id;
    if (a.token_log) a.token_log[step] = id;
    if (a.phase != YUE2_PHASE_NONE && id == a.end_id) st->done = 1;
}

// v[0] + v[1] + ... + v[n-1] in f32 from -0, in order (n >= 0); the LDS
// reads go out eight at a time ahead of their adds.
__device__ __forceinline__ float seq_sum(const float* v, int n) {
    float s = -0.0f;
    int k = 0;
    for (; k + 8 <= n; k += 8) {
        float t[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) t[j] = v[k + j];
#pragma unroll
        for (int j = 0; j < 8; ++j) s = s + t[j];
    }
    for (; k < n; ++k) s = s + v[k];
    return s;
}

// Steps 6-8 over the n survivors, given as order keys in surv (each key
// carries its score; surv holds the next power of two >= n entries, e_val and p_s n each:
// LDS arrays of kSurvivorMax, or the overflow arrays in global memory for
// more survivors): sort by score descending and id ascending (:174),
// top-p (:175-190) and renormalisation (:191-197) as sequential f32 sums,
// then the exponential race in id order (:198-214), whose uniforms are
// stream positions 2 id and 2 id + 1 of this token's block.  Returns the
// chosen id in every thread.
__device__ __forceinline__ int32_t race_tail(const SampleArgs& a, int step, uint64_t* surv, float* e_val, float* p_s, int n,
                                    int* s_kept, int* s_sel) {
    const int tid = threadIdx.x, nt = blockDim.x;
    // (e_val, not yet written, lends its room to the sort: n <= the block
    // size there, at most 1024 keys in its kSurvivorMax floats)
    sort_distinct(surv, n, reinterpret_cast<uint64_t*>(e_val));
    const float max = key_value(surv[0]);
    for (int i = tid; i < n; i += nt) e_val[i] = expf_cr(key_value(surv[i]) - max);
    __syncthreads();
    // The sums and the cumulative pass are sequential (in sorted order, as in
    // the reference); the divisions are independent and run on all threads.
    __shared__ float s_sum;
    const bool nucleus = a.top_p < 1.0f;
    if (nucleus) {
        if (tid == 0) s_sum = seq_sum(e_val, n);
        __syncthreads();
        const float sum = s_sum;
        for (int i = tid; i < n; i += nt) p_s[i] = cast(e_val[i] / sum, a.legacy);
        __syncthreads();
    }
    if (tid == 0) {
        int kept = n;
        if (nucleus) {
            float cumulative = 0.0f;
            const int protect = a.legacy ? 3 : 1;
            kept = 0;
            // entries read eight at a time ahead of the sequential pass (the
            // compaction writes index kept <= i, never a later entry)
            for (int i0 = 0; i0 < n; i0 += 8) {
                float pv[8], ev[8];
                uint64_t sv[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int i = min(i0 + j, n - 1);
                    pv[j] = p_s[i];
                    ev[j] = e_val[i];
                    sv[j] = surv[i];
                }
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    if (i0 + j >= n) break;
                    cumulative += pv[j];
                    const float prior = cast(cast(cumulative, a.legacy) - pv[j], a.legacy);
                    if (prior <= a.top_p || i0 + j < protect) {
                        surv[kept] = sv[j];
                        e_val[kept] = ev[j];
                        ++kept;
                    }
                }
            }
        }
        s_sum = seq_sum(e_val, kept);
        *s_kept = kept;
    }
    __syncthreads();
    const int kept = *s_kept;
    {
        const float sum = s_sum;
        for (int i = tid; i < kept; i += nt) {
            const float p = cast(e_val[i] / sum, a.legacy);
            surv[i] = ((uint64_t)(surv[i] & 0xffffffffu) << 32) | f2u(p);
        }
    }
    __syncthreads();
    sort_distinct(surv, kept, reinterpret_cast<uint64_t*>(e_val));  // e_val is rewritten below
    const uint32_t* stream = a.stream[step & 1];
    for (int i = tid; i < kept; i += nt) {
        const uint32_t id = (uint32_t)(surv[i] >> 32);
        const float p = u2f((uint32_t)(surv[i] & 0xffffffffu));
        const uint64_t hi = stream[2 * (size_t)id], lo = stream[2 * (size_t)id + 1];
        const double u = (double)(((hi << 32) | lo) & ((1ull << 53) - 1)) / 9007199254740992.0;
        const float noise = cast((float)(-log1p_d(-u)), a.legacy);
        e_val[i] = cast(p / noise, a.legacy);
    }
    __syncthreads();
    if (tid == 0) {
        // the first maximum in id order; entries read eight at a time
        float best = -__builtin_huge_valf();
        int32_t selected = 0;
        for (int i0 = 0; i0 < kept; i0 += 8) {
            float ev[8];
            uint64_t sv[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int i = min(i0 + j, kept - 1);
                ev[j] = e_val[i];
                sv[j] = surv[i];
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                if (i0 + j < kept && ev[j] > best) {
                    best = ev[j];
                    selected = (int32_t)(sv[j] >> 32);
                }
            }
        }
        *s_sel = selected;
    }
    __syncthreads();
    return *s_sel;
}

// MT19937 (src/sampling.rs:15-55): the next `count` outputs of the stream
// whose state is *mt into out; the state is advanced in place when `save`.
// The twist of 624 words runs as three dependent phases (i < 227 reads only
// old words; 227 <= i < 454 and 454 <= i < 624 read words of the previous
// phase), each read into registers before the barrier that precedes the
// write.  s: 624 words of LDS; every thread of the block takes part
// (blockDim.x >= 227).
__device__ __forceinline__ void mt_fill(MtState* mt, uint32_t* out, size_t count, uint32_t* s, bool save) {
    const int tid = threadIdx.x, nt = blockDim.x;
    for (int i = tid; i < 624; i += nt) s[i] = mt->state[i];
    int next = mt->next;
    __syncthreads();
    size_t produced = 0;
    while (produced < count) {
        if (next == 624) {
            // phase A: i in [0, 227)
            uint32_t v = 0;
            if (tid < 227) {
                const uint32_t bits = (s[tid] & 0x80000000u) | (s[tid + 1] & 0x7fffffffu);
                v = s[tid + 397] ^ (bits >> 1) ^ ((bits & 1u) ? 0x9908b0dfu : 0u);
            }
            __syncthreads();
            if (tid < 227) s[tid] = v;
            __syncthreads();
            // phase B: i in [227, 454)
            if (tid < 227) {
                const int i = tid + 227;
                const uint32_t bits = (s[i] & 0x80000000u) | (s[i + 1] & 0x7fffffffu);
                v = s[i - 227] ^ (bits >> 1) ^ ((bits & 1u) ? 0x9908b0dfu : 0u);
            }
            __syncthreads();
            if (tid < 227) s[tid + 227] = v;
            __syncthreads();
            // phase C: i in [454, 624); i = 623 pairs with the new word 0
            if (tid < 170) {
                const int i = tid + 454;
                const uint32_t nxt = i == 623 ? s[0] : s[i + 1];
                const uint32_t bits = (s[i] & 0x80000000u) | (nxt & 0x7fffffffu);
                v = s[i - 227] ^ (bits >> 1) ^ ((bits & 1u) ? 0x9908b0dfu : 0u);
            }
            __syncthreads();
            if (tid < 170) s[tid + 454] = v;
            __syncthreads();
            next = 0;
        }
        const size_t take = min((size_t)(624 - next), count - produced);
        for (int t = tid; t < (int)take; t += nt) {
            uint32_t y = s[next + t];
            y ^= y >> 11;
            y ^= (y << 7) & 0x9d2c5680u;
            y ^= (y << 15) & 0xefc60000u;
            y ^= y >> 18;
            out[produced + t] = y;
        }
        next += (int)take;
        produced += take;
    }
    __syncthreads();
    if (save) {
        for (int i = tid; i < 624; i += nt) mt->state[i] = s[i];
        if (tid == 0) mt->next = next;
    }
}

}  // namespace y2
