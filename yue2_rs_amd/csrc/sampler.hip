// sampler.hip -- on-device CFG mix, choose() and the MT19937 stream.
//
// One workgroup selects the next token from the LM-head logits so that only
// the token id leaves the device.  It follows src/sampling.rs:103-215 step by
// step: phase mask, repetition penalty, validity check, greedy argmax or
// temperature, top-k with ties kept at the threshold, top-p with a
// sequential f32 cumulative sum, renormalisation and the exponential race
// p / -ln(1 - u) in id order.  The race reads its uniforms from the token's
// block of 2 * vocab MT19937 outputs, which choose() consumes whatever the
// logits are, so the block is generated ahead by mt_generate_kernel.
#include "kernels.h"
#include "runtime.h"
#include "sampler.h"
#include "y2_math.h"

namespace y2 {

constexpr int kSurvivorMax = 2048;

__device__ __forceinline__ uint32_t ukey(float f) { return (uint32_t)total_key(f) ^ 0x80000000u; }
__device__ __forceinline__ float from_ukey(uint32_t k) {
    const int32_t b = (int32_t)(k ^ 0x80000000u);
    return u2f((uint32_t)(b < 0 ? b ^ 0x7fffffff : b));
}
__device__ __forceinline__ bool is_finite(float v) {
    return (f2u(v) & 0x7f800000u) != 0x7f800000u;
}
__device__ __forceinline__ float cast(float x, int legacy) { return legacy ? rb(x) : x; }

// compiler-rt __powisf2, which Rust's f32::powi calls for a run-time exponent.
__device__ float powi_f32(float a, int b) {
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
__device__ void bitonic_sort(uint64_t* v, int n) {
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

__global__ __launch_bounds__(1024) void choose_kernel(const SampleArgs a) {
    __shared__ uint64_t surv[kSurvivorMax];
    __shared__ float e_val[kSurvivorMax];
    __shared__ uint32_t hist[256];
    __shared__ int32_t window_ids[128];
    __shared__ int32_t s_count, s_bad, s_selected, s_kept;
    __shared__ uint32_t s_prefix;
    __shared__ int32_t s_remaining;
    __shared__ int32_t red_key[16], red_idx[16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    StepState* st = a.st;
    if (st->error || st->done) return;
    const int V = a.vocab, step = st->step;
    float* sc = a.scores;
    if (tid == 0) {
        s_count = 0;
        s_bad = 0;
        s_kept = 0;
    }
    // 1. CFG mix (src/sampling.rs:261-266) and phase mask (:116-129).
    for (int i = tid; i < V; i += 1024) {
        const float c = a.logits[i];
        float v = c;
        if (a.rows == 2) {
            const float u = a.logits[(size_t)V + i];
            v = rb(u + rb(a.cfg_scale * rb(c - u)));
        }
        bool in = true;
        if (a.phase == YUE2_PHASE_ABC) in = i < kEod;
        else if (a.phase == YUE2_PHASE_SEMANTIC) in = i >= kCodecOffset && i < kCodecOffset + kCodecSize;
        if (a.phase != YUE2_PHASE_NONE && i == a.end_id && step >= a.min_tokens) in = true;
        sc[i] = (a.mode == 0 || in) ? v : -__builtin_huge_valf();
    }
    __syncthreads();
    // 2. Repetition penalty over the last penalty_window generated ids
    //    (:130-144).  The first occurrence of each id applies alpha^count.
    if (a.mode == 1) {
        const int from = step > a.window ? step - a.window : 0;
        const int wn = step - from;
        for (int i = tid; i < wn; i += 1024) window_ids[i] = a.token_log[from + i];
        __syncthreads();
        if (tid < wn) {
            const int id = window_ids[tid];
            bool first = true;
            for (int j = 0; j < tid; ++j) first &= window_ids[j] != id;
            if (first) {
                int count = 0;
                for (int j = tid; j < wn; ++j) count += window_ids[j] == id;
                const float alpha = cast(powi_f32(a.repetition_penalty, count), a.legacy);
                const float s = sc[id];
                sc[id] = cast(s < 0.0f ? s * alpha : s / alpha, a.legacy);
            }
        }
        __syncthreads();
    }
    // 3. NaN / +inf check (:145-147), then greedy or temperature (:148-161).
    const bool greedy = a.mode == 0 || a.temperature == 0.0f;
    int32_t bk = INT32_MIN, bi = INT32_MAX, local_count = 0;
    for (int i = tid; i < V; i += 1024) {
        float v = sc[i];
        if (v != v || v == __builtin_huge_valf()) s_bad = 1;
        if (!greedy && a.temperature != 1.0f) {
            v = cast(v / a.temperature, a.legacy);
            sc[i] = v;
        }
        if (is_finite(v)) {
            ++local_count;
            const int32_t k = total_key(v);
            if (k > bk) {
                bk = k;
                bi = i;
            }
        }
    }
    atomicAdd(&s_count, local_count);
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) {
        const int32_t ok = __shfl_xor(bk, s, 64), oi = __shfl_xor(bi, s, 64);
        if (ok > bk || (ok == bk && oi < bi)) {
            bk = ok;
            bi = oi;
        }
    }
    if (lane == 0) {
        red_key[wave] = bk;
        red_idx[wave] = bi;
    }
    __syncthreads();
    if (a.mode == 1 && s_bad) {
        if (tid == 0) atomicCAS(&st->error, 0, 4);
        return;
    }
    if (s_count == 0) {
        if (tid == 0) atomicCAS(&st->error, 0, 3);
        return;
    }
    if (greedy) {
        if (tid == 0) {
            for (int w = 1; w < 16; ++w)
                if (red_key[w] > bk || (red_key[w] == bk && red_idx[w] < bi)) {
                    bk = red_key[w];
                    bi = red_idx[w];
                }
            s_selected = bi;
        }
        __syncthreads();
    } else {
        // 4. top-k threshold: the element of rank min(k-1, n-1) in
        //    descending total order, by radix select on the order keys.
        if (tid == 0) {
            s_prefix = 0;
            s_remaining = min(a.top_k - 1, s_count - 1);
        }
        for (int shift = 24; shift >= 0; shift -= 8) {
            for (int i = tid; i < 256; i += 1024) hist[i] = 0;
            __syncthreads();
            const uint32_t prefix = s_prefix;
            for (int i = tid; i < V; i += 1024) {
                const float v = sc[i];
                if (!is_finite(v)) continue;
                const uint32_t k = ukey(v);
                if (shift == 24 || (k >> (shift + 8)) == (prefix >> (shift + 8)))
                    atomicAdd(&hist[(k >> shift) & 255u], 1u);
            }
            __syncthreads();
            if (tid == 0) {
                int cum = 0, remaining = s_remaining;
                for (int bin = 255; bin >= 0; --bin) {
                    const int hcount = (int)hist[bin];
                    if (cum + hcount > remaining) {
                        s_prefix = prefix | ((uint32_t)bin << shift);
                        s_remaining = remaining - cum;
                        break;
                    }
                    cum += hcount;
                }
            }
            __syncthreads();
        }
        const float threshold = from_ukey(s_prefix);
        // 5. Survivors: finite scores >= threshold (ties kept, :173).
        if (tid == 0) s_count = 0;
        __syncthreads();
        for (int i = tid; i < V; i += 1024) {
            const float v = sc[i];
            if (is_finite(v) && v >= threshold) {
                const int at = atomicAdd(&s_count, 1);
                if (at < kSurvivorMax) surv[at] = ((uint64_t)(~ukey(v)) << 32) | (uint32_t)i;
            }
        }
        __syncthreads();
        const int n = s_count;
        if (n > kSurvivorMax) {
            if (tid == 0) atomicCAS(&st->error, 0, 5);
            return;
        }
        int n2 = 2;
        while (n2 < n) n2 <<= 1;
        for (int i = n + tid; i < n2; i += 1024) surv[i] = ~0ull;
        __syncthreads();
        // 6. Sort by score descending, id ascending (:174).
        bitonic_sort(surv, n2);
        const float max = sc[(int32_t)(surv[0] & 0xffffffffu)];
        for (int i = tid; i < n; i += 1024) e_val[i] = expf_cr(sc[(int32_t)(surv[i] & 0xffffffffu)] - max);
        __syncthreads();
        // 7. top-p (:175-190) and renormalisation (:191-197), sequential f32.
        if (tid == 0) {
            int kept = n;
            if (a.top_p < 1.0f) {
                float sum = -0.0f;
                for (int i = 0; i < n; ++i) sum = sum + e_val[i];
                float cumulative = 0.0f;
                const int protect = a.legacy ? 3 : 1;
                kept = 0;
                for (int i = 0; i < n; ++i) {
                    const float p = cast(e_val[i] / sum, a.legacy);
                    cumulative += p;
                    const float prior = cast(cast(cumulative, a.legacy) - p, a.legacy);
                    if (prior <= a.top_p || i < protect) {
                        surv[kept] = surv[i];
                        e_val[kept] = e_val[i];
                        ++kept;
                    }
                }
            }
            float sum = -0.0f;
            for (int i = 0; i < kept; ++i) sum = sum + e_val[i];
            for (int i = 0; i < kept; ++i) {
                const float p = cast(e_val[i] / sum, a.legacy);
                surv[i] = ((uint64_t)(surv[i] & 0xffffffffu) << 32) | f2u(p);
            }
            s_kept = kept;
        }
        __syncthreads();
        const int kept = s_kept;
        int k2 = 2;
        while (k2 < kept) k2 <<= 1;
        for (int i = kept + tid; i < k2; i += 1024) surv[i] = ~0ull;
        __syncthreads();
        // 8. Exponential race in id order (:198-214): uniforms at stream
        //    positions 2 id and 2 id + 1 of this token's block.
        bitonic_sort(surv, k2);
        const uint32_t* stream = a.stream[step & 1];
        for (int i = tid; i < kept; i += 1024) {
            const uint32_t id = (uint32_t)(surv[i] >> 32);
            const float p = u2f((uint32_t)(surv[i] & 0xffffffffu));
            const uint64_t hi = stream[2 * (size_t)id], lo = stream[2 * (size_t)id + 1];
            const double u = (double)(((hi << 32) | lo) & ((1ull << 53) - 1)) / 9007199254740992.0;
            const float noise = cast((float)(-log1p_d(-u)), a.legacy);
            e_val[i] = cast(p / noise, a.legacy);
        }
        __syncthreads();
        if (tid == 0) {
            float best = -__builtin_huge_valf();
            int32_t selected = 0;
            for (int i = 0; i < kept; ++i) {
                if (e_val[i] > best) {
                    best = e_val[i];
                    selected = (int32_t)(surv[i] >> 32);
                }
            }
            s_selected = selected;
        }
        __syncthreads();
    }
    if (tid == 0) {
        const int32_t id = s_selected;
        for (int b = 0; b < a.rows; ++b) st->ids[b] = id;
        a.token_log[step] = id;
        if (a.phase != YUE2_PHASE_NONE && id == a.end_id) st->done = 1;
    }
}

// MT19937 block generation (src/sampling.rs:15-55).  The twist of 624 words
// runs as three dependent phases (i < 227 reads only old words; 227 <= i <
// 454 and 454 <= i < 624 read words of the previous phase), each read into
// registers before the barrier that precedes the write.
__global__ __launch_bounds__(256) void mt_generate_kernel(MtState* mt, uint32_t* out0,
                                                          uint32_t* out1, size_t count,
                                                          const StepState* st, int ahead) {
    __shared__ uint32_t s[624];
    const int tid = threadIdx.x;
    uint32_t* out = ((st->step + ahead) & 1) ? out1 : out0;
    for (int i = tid; i < 624; i += 256) s[i] = mt->state[i];
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
        for (int t = tid; t < (int)take; t += 256) {
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
    for (int i = tid; i < 624; i += 256) mt->state[i] = s[i];
    if (tid == 0) mt->next = next;
}

void launch_choose(hipStream_t s, const SampleArgs& a) { choose_kernel<<<1, 1024, 0, s>>>(a); }

void launch_mt_generate(hipStream_t s, MtState* mt, uint32_t* out0, uint32_t* out1, size_t count,
                        const StepState* st, int ahead) {
    mt_generate_kernel<<<1, 256, 0, s>>>(mt, out0, out1, count, st, ahead);
}

}  // namespace y2
