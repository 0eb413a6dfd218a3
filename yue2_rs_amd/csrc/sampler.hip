// sampler.hip -- on-device CFG mix, choose() and the MT19937 stream.
//
// choose() follows src/sampling.rs:103-215 step by step: phase mask,
// repetition penalty, validity check, greedy argmax or temperature, top-k
// with ties kept at the threshold, top-p with a sequential f32 cumulative
// sum, renormalisation and the exponential race p / -ln(1 - u) in id order.
// The race reads its uniforms from the token's block of 2 * vocab MT19937
// outputs, which choose() consumes whatever the logits are, so the block is
// generated ahead by mt_generate_kernel.
//
// Chunked path: score_kernel, one workgroup per kChooseChunk vocabulary
// entries, applies the mix, mask, penalty and temperature and sorts its chunk
// by (score descending, id ascending), keeping the first min(top_k, chunk)
// entries.  Every entry of the global top-k is within its own chunk's top-k,
// so finish_kernel (one workgroup) finds the top-k threshold by radix select
// over at most chunks * top_k keys.  Only a chunk whose list was cut short
// and ends at the threshold can hold further survivors (entries equal to the
// threshold); those chunks are rescanned.  Sort, top-p, renormalisation and
// the race then run over the survivors alone.
// Single-workgroup path: choose_kernel does the same over the whole
// vocabulary; it serves top-k values the chunked lists cannot hold.
#include <algorithm>

#include "dev_sample.h"
#include "kernels.h"
#include "runtime.h"
#include "sampler.h"
#include "y2_math.h"

namespace y2 {


// Single-workgroup choose() over the whole vocabulary.
__global__ __launch_bounds__(1024) void choose_kernel(const SampleArgs a) {
    __shared__ uint64_t surv[kSurvivorMax];
    __shared__ float e_val[kSurvivorMax];
    __shared__ float p_buf[kSurvivorMax];
    __shared__ uint32_t hist[256];
    __shared__ int32_t window_ids[kWindowMax];
    __shared__ int32_t s_count, s_bad, s_sel, s_kept;
    __shared__ uint32_t s_prefix;
    __shared__ int32_t s_remaining;
    __shared__ uint64_t red[16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    StepState* st = a.st;
    if (st->error || st->done) return;
    const int V = a.vocab, step = st->step + a.step_offset;
    float* sc = a.scores;
    if (tid == 0) {
        s_count = 0;
        s_bad = 0;
        s_kept = 0;
    }
    // 1-2. mix, mask and repetition penalty
    for (int i = tid; i < V; i += 1024) sc[i] = mixed_score(a, i, step);
    const int wn = load_window(a, step, window_ids);
    if (a.mode == 1) apply_penalty(a, window_ids, wn, sc, 0, V);
    // 3. NaN / +inf check (:145-147), then greedy or temperature (:148-161).
    const bool greedy = a.mode == 0 || a.temperature == 0.0f;
    uint64_t best = ~0ull;
    int local_count = 0;
    for (int i = tid; i < V; i += 1024) {
        float v = sc[i];
        if (v != v || v == __builtin_huge_valf()) s_bad = 1;
        if (!greedy && a.temperature != 1.0f) {
            v = cast(v / a.temperature, a.legacy);
            sc[i] = v;
        }
        if (is_finite(v)) {
            ++local_count;
            best = kmin(best, order_key(v, i));
        }
    }
    atomicAdd(&s_count, local_count);
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) best = kmin(best, shfl_xor64(best, s));
    if (lane == 0) red[wave] = best;
    __syncthreads();
    if (a.mode == 1 && s_bad) {
        if (tid == 0) atomicCAS(&st->error, 0, 4);
        return;
    }
    if (s_count == 0) {
        if (tid == 0) atomicCAS(&st->error, 0, 3);
        return;
    }
    int32_t selected;
    if (greedy) {
        for (int w = 0; w < 16; ++w) best = kmin(best, red[w]);
        selected = (int32_t)(best & 0xffffffffu);
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
        // 5. Survivors: finite scores >= threshold (ties kept, :173), into
        //    LDS, or (when more than it holds survive) into the overflow arrays
        uint64_t* dst = surv;
        int n = 0;
        bool overflow = false;
        for (int pass = 0; pass < 2; ++pass) {
            const int cap = pass == 0 ? kSurvivorMax : a.big_cap;
            __syncthreads();  // every thread has read the previous pass's count
            if (tid == 0) s_count = 0;
            __syncthreads();
            for (int i = tid; i < V; i += 1024) {
                const float v = sc[i];
                if (is_finite(v) && v >= threshold) {
                    const int at = atomicAdd(&s_count, 1);
                    if (at < cap) dst[at] = order_key(v, i);
                }
            }
            __syncthreads();
            n = s_count;
            if (n <= cap) break;
            if (pass == 1 || !a.big) {
                if (tid == 0) atomicCAS(&st->error, 0, 5);
                return;
            }
            dst = a.big;
            overflow = true;
        }
        selected = overflow ? race_tail(a, step, a.big, a.big_e, a.big_p, n, &s_kept, &s_sel)
                            : race_tail(a, step, surv, e_val, p_buf, n, &s_kept, &s_sel);
    }
    if (tid == 0) publish(a, step, selected);
}

// Chunked path, part 1: one workgroup of 256 threads per kChooseChunk
// entries.  Writes the tempered scores (for the survivors' exponentials and
// rescans), the chunk's {finite entries, invalid-logit flag} and its first
// `list` order keys (greedy: list 1, the chunk's best entry).
__global__ __launch_bounds__(256) void score_kernel(const SampleArgs a) {
    constexpr int PER = kChooseChunk / 256;
    __shared__ float vals[kChooseChunk];
    __shared__ uint64_t keys[kChooseChunk];
    __shared__ int32_t window_ids[kWindowMax];
    __shared__ int32_t s_finite, s_bad;
    __shared__ uint64_t s_best[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const StepState* st = a.st;
    if (st->error || st->done) return;
    const int V = a.vocab, step = st->step + a.step_offset, c = blockIdx.x, lo = c * kChooseChunk;
    if (tid == 0) {
        s_finite = 0;
        s_bad = 0;
    }
#pragma unroll
    for (int e = 0; e < PER; ++e) {
        const int j = tid + 256 * e, i = lo + j;
        vals[j] = i < V ? mixed_score(a, i, step) : -__builtin_huge_valf();
    }
    const int wn = load_window(a, step, window_ids);
    if (a.mode == 1) apply_penalty(a, window_ids, wn, vals, lo, min(kChooseChunk, V - lo));
    const bool greedy = a.mode == 0 || a.temperature == 0.0f;
    int fin = 0, bad = 0;
    uint64_t best = ~0ull;
#pragma unroll
    for (int e = 0; e < PER; ++e) {
        const int j = tid + 256 * e, i = lo + j;
        float v = vals[j];
        uint64_t key = ~0ull;
        if (i < V) {
            if (v != v || v == __builtin_huge_valf()) bad = 1;
            if (!greedy) {
                if (a.temperature != 1.0f) v = cast(v / a.temperature, a.legacy);
                a.scores[i] = v;
            }
            if (is_finite(v)) {
                ++fin;
                key = order_key(v, i);
            }
        }
        if (greedy) best = kmin(best, key);
        else keys[j] = key;
    }
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) {
        fin += __shfl_xor(fin, s, 64);
        bad |= __shfl_xor(bad, s, 64);
        if (greedy) best = kmin(best, shfl_xor64(best, s));
    }
    if (lane == 0) {
        atomicAdd(&s_finite, fin);
        if (bad) atomicOr(&s_bad, 1);
        s_best[wave] = best;
    }
    __syncthreads();
    if (greedy) {
        if (tid == 0) {
            for (int w = 1; w < 4; ++w) best = kmin(best, s_best[w]);
            a.cand[c] = kmin(best, s_best[0]);
            a.meta[c] = make_int2(s_finite, s_bad);
        }
        return;
    }
    bitonic_sort(keys, kChooseChunk);
    const int n = min(a.list, s_finite);
    for (int j = tid; j < n; j += 256) a.cand[(size_t)c * a.list + j] = keys[j];
    if (tid == 0) a.meta[c] = make_int2(s_finite, s_bad);
}

// Chunked path, part 2: one workgroup of 1024 threads.
__global__ __launch_bounds__(1024) void finish_kernel(const SampleArgs a) {
    constexpr int PER = kChooseCandMax / 1024;
    __shared__ int32_t off[kChooseChunksMax + 1];
    __shared__ int32_t rescan[kChooseChunksMax];
    __shared__ uint64_t rescan_last[kChooseChunksMax];
    __shared__ uint64_t surv[kSurvivorMax];
    __shared__ float e_val[kSurvivorMax];
    __shared__ float p_buf[kSurvivorMax];
    __shared__ uint32_t hist[256];
    __shared__ int32_t wsum[16];
    __shared__ uint64_t red[16];
    __shared__ int32_t s_count, s_bad, s_n, s_nres, s_kept, s_sel, s_remaining;
    __shared__ uint32_t s_prefix;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    StepState* st = a.st;
    if (st->error || st->done) return;
    const int V = a.vocab, step = st->step + a.step_offset, nch = a.chunks, L = a.list;
    if (tid == 0) {
        s_count = 0;
        s_bad = 0;
        s_n = 0;
        s_nres = 0;
    }
    // chunk totals, one chunk per thread, and the offsets of the lists
    // concatenated in chunk order (off[nch] = their total length)
    int fin = 0, bad = 0;
    if (tid < nch) {
        const int2 m = a.meta[tid];
        fin = m.x;
        bad = m.y;
    }
    const int nc = min(L, fin);
    int incl = nc;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int t = __shfl_up(incl, d, 64);
        if (lane >= d) incl += t;
    }
    if (lane == 63) wsum[wave] = incl;
    __syncthreads();
    if (fin) atomicAdd(&s_count, fin);
    if (bad) atomicOr(&s_bad, 1);
    int base = 0;
    for (int w = 0; w < wave; ++w) base += wsum[w];
    if (tid <= nch) off[tid] = base + incl - nc;
    __syncthreads();
    if (a.mode == 1 && s_bad) {
        if (tid == 0) atomicCAS(&st->error, 0, 4);
        return;
    }
    const int count = s_count;
    if (count == 0) {
        if (tid == 0) atomicCAS(&st->error, 0, 3);
        return;
    }
    if (a.mode == 0 || a.temperature == 0.0f) {
        uint64_t best = fin > 0 ? a.cand[tid] : ~0ull;
#pragma unroll
        for (int s = 32; s >= 1; s >>= 1) best = kmin(best, shfl_xor64(best, s));
        if (lane == 0) red[wave] = best;
        __syncthreads();
        if (tid == 0) {
            for (int w = 0; w < 16; ++w) best = kmin(best, red[w]);
            publish(a, step, (int32_t)(best & 0xffffffffu));
        }
        return;
    }
    // candidates: entry i of the concatenation lies in the last chunk whose
    // offset is <= i
    const int T = off[nch];
    uint64_t mine[PER];
#pragma unroll
    for (int q = 0; q < PER; ++q) {
        const int i = tid + 1024 * q;
        mine[q] = ~0ull;
        if (i < T) {
            int lo = 0, hi = nch;
            while (hi - lo > 1) {
                const int mid = (lo + hi) >> 1;
                if (off[mid] <= i) lo = mid;
                else hi = mid;
            }
            mine[q] = a.cand[(size_t)lo * L + (i - off[lo])];
        }
    }
    // top-k threshold: rank min(k-1, n-1) in descending order, by radix
    // select over the candidates' score keys
    if (tid == 0) {
        s_prefix = 0;
        s_remaining = min(a.top_k - 1, count - 1);
    }
    for (int shift = 24; shift >= 0; shift -= 8) {
        if (tid < 256) hist[tid] = 0;
        __syncthreads();
        const uint32_t prefix = s_prefix;
#pragma unroll
        for (int q = 0; q < PER; ++q) {
            if (tid + 1024 * q >= T) continue;
            const uint32_t k = ~(uint32_t)(mine[q] >> 32);
            if (shift == 24 || (k >> (shift + 8)) == (prefix >> (shift + 8)))
                atomicAdd(&hist[(k >> shift) & 255u], 1u);
        }
        __syncthreads();
        if (wave == 0) {
            // lane l holds bins 255 - 4 l .. 252 - 4 l, in descending order
            uint32_t h[4];
            int t = 0;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                h[q] = hist[255 - 4 * lane - q];
                t += (int)h[q];
            }
            int above = t;
#pragma unroll
            for (int d = 1; d < 64; d <<= 1) {
                const int u = __shfl_up(above, d, 64);
                if (lane >= d) above += u;
            }
            above -= t;  // entries in higher bins than this lane's
            const int remaining = s_remaining;
            if (remaining >= above && remaining < above + t) {
                int cum = above;
                for (int q = 0; q < 4; ++q) {
                    if (cum + (int)h[q] > remaining) {
                        s_prefix = prefix | ((uint32_t)(255 - 4 * lane - q) << shift);
                        s_remaining = remaining - cum;
                        break;
                    }
                    cum += (int)h[q];
                }
            }
        }
        __syncthreads();
    }
    const float threshold = from_ukey(s_prefix);
    // chunks whose list was cut at an entry equal to the threshold: the
    // entries after that one in order that equal it survive too
    if (tid < nch && fin > L) {
        const uint64_t last = a.cand[(size_t)tid * L + L - 1];
        if (key_value(last) >= threshold) {
            const int r = atomicAdd(&s_nres, 1);
            rescan[r] = tid;
            rescan_last[r] = last;
        }
    }
    __syncthreads();
    const int nres = s_nres;
    // survivors (:173), into LDS, or (when more than it holds survive) into
    // the overflow arrays: listed entries >= threshold and the rescans' ties
    uint64_t* dst = surv;
    int n = 0;
    bool overflow = false;
    for (int pass = 0; pass < 2; ++pass) {
        const int cap = pass == 0 ? kSurvivorMax : a.big_cap;
        __syncthreads();  // every thread has read the previous pass's count
        if (tid == 0) s_n = 0;
        __syncthreads();
#pragma unroll
        for (int q = 0; q < PER; ++q) {
            if (tid + 1024 * q >= T) continue;
            if (key_value(mine[q]) >= threshold) {
                const int at = atomicAdd(&s_n, 1);
                if (at < cap) dst[at] = mine[q];
            }
        }
        for (int r = 0; r < nres; ++r) {
            const int i = rescan[r] * kChooseChunk + tid;
            if (i < V) {
                const float v = a.scores[i];
                if (is_finite(v) && v >= threshold) {
                    const uint64_t k = order_key(v, i);
                    if (k > rescan_last[r]) {
                        const int at = atomicAdd(&s_n, 1);
                        if (at < cap) dst[at] = k;
                    }
                }
            }
        }
        __syncthreads();
        n = s_n;
        if (n <= cap) break;
        if (pass == 1 || !a.big) {
            if (tid == 0) atomicCAS(&st->error, 0, 5);
            return;
        }
        dst = a.big;
        overflow = true;
    }
    const int32_t selected = overflow ? race_tail(a, step, a.big, a.big_e, a.big_p, n, &s_kept, &s_sel)
                                      : race_tail(a, step, surv, e_val, p_buf, n, &s_kept, &s_sel);
    if (tid == 0) publish(a, step, selected);
}

__global__ __launch_bounds__(256) void mt_generate_kernel(MtState* mt, uint32_t* out0, uint32_t* out1,
                                                          size_t count, const StepState* st, int ahead) {
    __shared__ uint32_t s[624];
    mt_fill(mt, ((st->step + ahead) & 1) ? out1 : out0, count, s, true);
}


int survivor_capacity(int vocab) {
    int c = 2;
    while (c < vocab) c <<= 1;
    return c;
}

size_t survivor_bytes(int vocab) {
    return sizeof(uint64_t) * (size_t)survivor_capacity(vocab) + 2 * sizeof(float) * (size_t)vocab;
}

void set_survivor_buffers(SampleArgs& a, void* base, int vocab) {
    a.big_cap = survivor_capacity(vocab);
    a.big = static_cast<uint64_t*>(base);
    a.big_e = reinterpret_cast<float*>(a.big + a.big_cap);
    a.big_p = a.big_e + vocab;
}

int choose_list_len(int vocab, int mode, float temperature, int top_k) {
    const int chunks = (vocab + kChooseChunk - 1) / kChooseChunk;
    if (chunks < 1 || chunks >= kChooseChunksMax) return 0;
    const int list = (mode == 0 || temperature == 0.0f) ? 1 : std::min(top_k, kChooseChunk);
    if (list < 1 || (size_t)chunks * list > (size_t)kChooseCandMax) return 0;
    return list;
}

void launch_choose(hipStream_t s, const SampleArgs& a) {
    if (a.cand) {
        score_kernel<<<a.chunks, 256, 0, s>>>(a);
        finish_kernel<<<1, 1024, 0, s>>>(a);
    } else {
        choose_kernel<<<1, 1024, 0, s>>>(a);
    }
}

void launch_mt_generate(hipStream_t s, MtState* mt, uint32_t* out0, uint32_t* out1, size_t count,
                        const StepState* st, int ahead) {
    mt_generate_kernel<<<1, 256, 0, s>>>(mt, out0, out1, count, st, ahead);
}

}  // namespace y2
