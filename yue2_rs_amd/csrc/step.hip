// step.hip -- the persistent token-step kernel: one launch runs a whole
// decode token (embedding, every layer, final norm and LM head) for one or
// two batch rows (Model::hidden + forward, src/model.rs:452-591).
//
// Why one kernel: each phase of the step (norm -> QKV -> attention -> O ->
// norm -> gate/up -> down) depends on the complete output of the previous
// one.  A kernel per phase pays a launch, a ramp-up and a drain at every one
// of those ~140 dependencies per token (about 7 us each on this part, the
// same as a whole 16 MB read).  Here one workgroup per CU stays resident for
// the whole step.
//
// Dependencies between workgroups are dataflow, not barriers: every value a
// workgroup produces for others (q/k/v, attention output, x after O and after
// down, SwiGLU activations, the attention block statistics and partials) is a
// tagged 64-bit word (dev_flow.h), and its consumers poll for it.  A
// workgroup starts on the next phase as soon as the inputs it needs exist.
//
// Weight streaming: each wave walks its rows of a GEMV as a sequence of
// items (SEG 16-byte chunks per lane of one row, both matrices for the
// gate/up pair) through a ring of R register slots, so R-1 items are in
// flight while one is multiplied.  Before polling for the next phase's
// inputs every wave already issues the first R-1 items of the next GEMV.
//
// Work split (n rows of a GEMV over G workgroups): workgroup w owns rows
// [w*n/G, (w+1)*n/G); its 8 waves take every 8th row.  Every row's
// arithmetic is the DOT order of dev_gemv.h, and the attention is the same
// arithmetic as dev_attn.h, so the results equal the per-phase kernels' bit
// for bit.  The launch uses exactly one workgroup per CU, so all are
// co-resident (every wait is bounded all the same).
#include <algorithm>

#include "dev_attn.h"
#include "dev_flow.h"
#include "dev_sample.h"
#include "dev_gemv.h"
#include "dev_ring.h"
#include "kernels.h"
#include "runtime.h"
#include "step.h"

namespace y2 {

constexpr int kStepThreads = kRingThreads;

// Trace of the traced instantiation: thread 0 of each workgroup stamps the
// device wall clock (100 MHz) into trace[slot * gridDim.x + workgroup];
// slots past the buffer are dropped.  The untraced kernel has no code for it.
template <bool ON>
struct Tracer {
    unsigned long long* buf;
    int slots, slot;
    __device__ __forceinline__ void mark() {
        if constexpr (ON) {
            if (threadIdx.x == 0 && slot < slots) gblw(buf)[(size_t)slot * gridDim.x + blockIdx.x] = wall_clock64();
            ++slot;
        }
    }
};

// ---- staging and norms -----------------------------------------------------

// Batch rows of x, the SwiGLU activations and q/k/v are BF16-exact, so with
// two rows one packed word carries both (half the words to poll).
template <int B>
constexpr bool kPack = B == 2;
// With one row, the GEMV outputs that other workgroups gather (x, q/k/v, the
// SwiGLU activations; BF16-exact) go out two per word: rows 2p and 2p + 1.
template <int B>
constexpr bool kPair = B == 1;
constexpr int kPairRowsMax = 64;  // rows of one such GEMV per workgroup
// The generic kernels' iterations (512 inputs each): hidden and heads *
// head_dim up to 4608, intermediate up to 14336.  (Nine, not eight: a row's
// items are then three chunks per lane, as the 3B-class kernel's; with four
// the head_dim-128 kernels spilled ~35 registers, with three 8.)
constexpr int kStepAnyIth = 9, kStepAnyItq = 9, kStepAnyIti = 28;

// First row of workgroup w's share of an exchanged GEMV output of n rows:
// even for paired words (a pair never straddles two workgroups).
template <int B>
__device__ __forceinline__ int xlo(int n, int w, int parts) {
    return kPair<B> ? 2 * part_lo(n / 2, w, parts) : part_lo(n, w, parts);
}


// xs[b * k + i] = row b's value of x-like words tx (packed for two rows,
// for one row two values per word), i < k.
// (Past 16 words per thread, in passes of 16: the first pass's words are
// all in before the second's are polled.)
template <int B, int N>
__device__ __forceinline__ bool stage_rows(float* xs, const uint64_t* tx, int k, uint32_t tag, StepState* st) {
    if constexpr (kPack<B>) {
        if constexpr (N <= 16) {
            return gather_pair<kStepThreads, N>(tx, k, tag, xs, st);
        } else {
            static_assert(N <= 32, "two passes");
            constexpr int F = 16 * kStepThreads;
            const auto put = [=](int base) {
                return [=](int i, uint32_t bits) {
                    xs[base + i] = bf16_lo(bits);
                    xs[k + base + i] = bf16_hi(bits);
                };
            };
            return gather_put<kStepThreads, 16>([=](int i) { return tx + i; }, min(k, F), tag, put(0), st) &&
                   (k <= F || gather_put<kStepThreads, N - 16>([=](int i) { return tx + F + i; }, k - F, tag,
                                                               put(F), st));
        }
    } else {
        // one row: word p holds rows 2p and 2p + 1 (past 8 words per
        // thread, in passes of 8)
        static_assert(kPair<B>, "one or two rows");
        constexpr int M = (N + 1) / 2, F = 8 * kStepThreads;
        static_assert(M <= 16, "two passes");
        const auto put = [=](int base) {
            return [=](int i, uint32_t bits) {
                xs[2 * (base + i)] = bf16_lo(bits);
                xs[2 * (base + i) + 1] = bf16_hi(bits);
            };
        };
        if constexpr (M <= 8) {
            return gather_put<kStepThreads, M>([=](int i) { return tx + i; }, k / 2, tag, put(0), st);
        } else {
            return gather_put<kStepThreads, 8>([=](int i) { return tx + i; }, min(k / 2, F), tag, put(0), st) &&
                   (k / 2 <= F ||
                    gather_put<kStepThreads, M - 8>([=](int i) { return tx + F + i; }, k / 2 - F, tag, put(F), st));
        }
    }
}

// xs[b * k + i] = row b's attention output i, i < k: words tx[b * k / 2 + p]
// each hold outputs 2p (low half) and 2p + 1 (high half) of a row.
template <int B, int N>
__device__ __forceinline__ bool stage_att(float* xs, const uint64_t* tx, int k, uint32_t tag, StepState* st) {
    static_assert(B * N <= 32, "at most 16 words per thread in flight");
    const int h = k / 2;
    return gather_put<kStepThreads, (B * N + 1) / 2>([=](int i) { return tx + i; }, B * h, tag,
                                                     [=](int i, uint32_t bits) {
                                                         const int b = i >= h ? 1 : 0, p = i - b * h;
                                                         xs[b * k + 2 * p] = bf16_lo(bits);
                                                         xs[b * k + 2 * p + 1] = bf16_hi(bits);
                                                     },
                                                     st);
}

// stage_rows for x ahead of its RMSNorm, plus each thread's shares of the
// norm's sums.  With packed words (two rows) the shares are added as the
// words arrive (over the elements this thread stages, in arrival order), so
// the norm needs no pass over LDS of its own; for one row a separate pass
// measured faster (the added live registers cost the batch-1 kernel more).
template <int B, int N>
__device__ __forceinline__ bool stage_x(float* xs, const uint64_t* tx, int k, uint32_t tag, StepState* st,
                                        double* e_sum, double* w_sum) {
    if constexpr (kPack<B>) {
        static_assert(N <= 16, "at most 16 words per thread in flight");
#pragma unroll
        for (int b = 0; b < B; ++b) e_sum[b] = w_sum[b] = 0.0;
        return gather_put<kStepThreads, N>([=](int i) { return tx + i; }, k, tag,
                                           [&](int i, uint32_t bits) {
                                               const float x0 = bf16_lo(bits), x1 = bf16_hi(bits);
                                               xs[i] = x0;
                                               xs[k + i] = x1;
                                               norm_partial_add(e_sum[0], w_sum[0], x0, i, k);
                                               norm_partial_add(e_sum[B - 1], w_sum[B - 1], x1, i, k);
                                           },
                                           st);
    } else {
        return stage_rows<B, N>(xs, tx, k, tag, st);  // norm_rows adds the shares
    }
}

// res[b * n + r] = xs[b * k + h0 + r], r < n = h1 - h0 <= kResRows: this
// workgroup's rows of the residual stream, taken from the staged x before it
// is normalised, for the residual epilogue of the next O or down projection
// (whose rows [h0, h1) are this workgroup's).  The norm's first barrier
// orders these reads before its writes to xs.
template <int B>
__device__ __forceinline__ void copy_res(float* res, const float* xs, int k, int h0, int h1) {
    const int n = h1 - h0, t = threadIdx.x;
    if (t < B * n) res[t] = xs[(t / n) * k + h0 + t % n];
}

// gam[j] = g[tid + 512 j] for tid + 512 j < k: a norm's gammas, loaded
// ahead.  The loads are unconditional (entries past k re-read g[k - 1] and
// are never used): a conditional load would make the compiler wait for it,
// and so for everything issued before it, where the branches join.
template <int N>
__device__ __forceinline__ void load_gamma(const float* g, int k, float* gam) {
#pragma unroll
    for (int j = 0; j < N; ++j) gam[j] = gbl(g)[min((int)threadIdx.x + j * kStepThreads, k - 1)];
}

// xs[b] = RMSNorm(xs[b]) (Norm::apply, src/tensor.rs:1140-1157) with the
// gammas of load_gamma; the rows' scales are decided together from each
// thread's shares of the sums (stage_x's with packed words, else added here).
// Entered right after a block barrier.
template <int B, int N>
__device__ __forceinline__ void norm_rows(float* xs, int k, const float* gam, float eps, int* fallbacks,
                                          double* e_sum, double* w_sum) {
    // a thread's elements tid + 512 j, all read at once (past k: element
    // k - 1, never written back), so their LDS reads are in flight together;
    // read inside the stores' bounds test, each one was waited for before the
    // next was issued
    float v[B][N];
#pragma unroll
    for (int b = 0; b < B; ++b)
#pragma unroll
        for (int j = 0; j < N; ++j) v[b][j] = xs[b * k + min((int)threadIdx.x + j * kStepThreads, k - 1)];
    if constexpr (!kPack<B>) {
#pragma unroll
        for (int b = 0; b < B; ++b) e_sum[b] = w_sum[b] = 0.0;
#pragma unroll
        for (int j = 0; j < N; ++j) {
            const int i = threadIdx.x + j * kStepThreads;
            if (i < k)
#pragma unroll
                for (int b = 0; b < B; ++b) norm_partial_add(e_sum[b], w_sum[b], v[b][j], i, k);
        }
    }
    float s[B];
    norm_scales_from<kStepThreads, B>(e_sum, w_sum, xs, k, eps, fallbacks, s);
#pragma unroll
    for (int b = 0; b < B; ++b)
#pragma unroll
        for (int j = 0; j < N; ++j) {
            const int i = threadIdx.x + j * kStepThreads;
            const float y = rb(rb(v[b][j] * s[b]) * gam[j]);
            if (i < k) xs[b * k + i] = y;
        }
    __syncthreads();
}

// ---- the fused sampler -----------------------------------------------------

__device__ __forceinline__ void st_agent_u64(uint64_t* p, uint64_t v) {
    __hip_atomic_store(gblw(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent_f32(float* p, float v) {
    __hip_atomic_store(gblw(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_agent_f32(const float* p) {
    return __hip_atomic_load(gblw(const_cast<float*>(p)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Block reductions over the 512 threads (red: 8 words of LDS scratch per
// value); every thread gets the result.
__device__ __forceinline__ int block_sum_i(int v, int* red) {
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    int t = 0;
    for (int w = 0; w < kStepThreads / 64; ++w) t += red[w];
    return t;
}
__device__ __forceinline__ uint64_t block_min_u64(uint64_t v, uint64_t* red) {
    for (int m = 32; m >= 1; m >>= 1) v = kmin(v, shfl_xor64(v, m));
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    uint64_t t = ~0ull;
    for (int w = 0; w < kStepThreads / 64; ++w) t = kmin(t, red[w]);
    return t;
}

// The LM-head rows worker w computes (and scores): rows [lo, lo + n) split
// over the workers, plus the stop row (if any) for worker 0.  Every other
// logit is -inf, so these are the only entries choose() can pick.
struct HeadRows {
    int lo, n, stop;
    __device__ __forceinline__ int r0(int w, int nw) const { return lo + part_lo(n, w, nw); }
    __device__ __forceinline__ int r1(int w, int nw) const { return lo + part_lo(n, w + 1, nw); }
    __device__ __forceinline__ int extra(int w) const { return w == 0 ? stop : -1; }
};

// A worker's share of the fused sampler: its rows [r0, r1) (and `extra`
// when >= 0) of the step's logits, just stored by this workgroup, scored as
// choose() scores every entry -- CFG mix, phase mask, repetition penalty,
// validity, temperature (src/sampling.rs:117-161, 261-266) -- and its best
// `list` order keys (score descending, id ascending) published for the
// sampler workgroup, followed by one tagged word {finite entries | invalid
// flag << 31}.  lds: at least 13 KiB.
__device__ __forceinline__ void score_rows(const StepArgs* args, int r0, int r1, int extra, int w, uint32_t epoch,
                                           float* lds) {
    const FusedSampler& fs = args->smp;
    const SampleArgs& a = fs.a;
    StepState* st = args->st;
    const int tid = threadIdx.x, span = r1 - r0 + (extra >= 0 ? 1 : 0);
    float* vals = lds;                                                 // [kFusedRowsMax]
    uint64_t* keys = reinterpret_cast<uint64_t*>(lds + kFusedRowsMax);  // [kFusedRowsMax]
    int32_t* ids = reinterpret_cast<int32_t*>(keys + kFusedRowsMax);    // [kWindowMax]
    int* red = ids + kWindowMax;                                       // [16]
    const int step = *gbl(&st->step) + 1;  // the token this launch chooses
    // this workgroup's logit stores (lane 0 of each wave) precede the reads
    __syncthreads();
    const int wn = load_window(a, step, ids);
    const int nr = r1 - r0;  // entry j < nr is row r0 + j; entry nr is the extra row
    for (int j = tid; j < kFusedRowsMax; j += kStepThreads)
        vals[j] = j < span ? mixed_score(a, j < nr ? r0 + j : extra, step) : -__builtin_huge_valf();
    __syncthreads();
    if (a.mode == 1) {
        apply_penalty(a, ids, wn, vals, r0, nr);
        if (extra >= 0) apply_penalty(a, ids, wn, vals + nr, extra, 1);
    }
    const bool greedy = a.mode == 0 || a.temperature == 0.0f;
    int fin = 0, bad = 0;
    uint64_t best = ~0ull;
    for (int j = tid; j < kFusedRowsMax; j += kStepThreads) {
        const int i = j < nr ? r0 + j : extra;
        float v = vals[j];
        uint64_t key = ~0ull;
        if (j < span) {
            if (v != v || v == __builtin_huge_valf()) bad = 1;
            if (!greedy) {
                if (a.temperature != 1.0f) v = cast(v / a.temperature, a.legacy);
                st_agent_f32(a.scores + i, v);  // for the sampler's rescans of ties
            }
            if (is_finite(v)) {
                ++fin;
                key = order_key(v, i);
            }
        }
        best = kmin(best, key);
        keys[j] = key;
    }
    fin = block_sum_i(fin, red);
    bad = block_sum_i(bad, red + 8);
    if (greedy) {
        best = block_min_u64(best, reinterpret_cast<uint64_t*>(red));  // (red's ints are read: barrier inside)
        if (tid == 0) st_agent_u64(fs.cand + w, best);
    } else {
        // the n smallest keys in order, each stored at its rank (the keys
        // are distinct: they carry the id; the non-finite entries, ~0, rank
        // above every finite one and are not listed)
        const int n = min(fs.list, fin);
        for (int j = tid; j < span; j += kStepThreads) {
            const uint64_t k = keys[j];
            if (k == ~0ull) continue;
            const int r = rank_below(keys, span, k);
            if (r < n) st_agent_u64(fs.cand + (size_t)w * fs.list + r, k);
        }
    }
    stores_done();  // every candidate and score is stored before the word that announces them
    __syncthreads();
    if (tid == 0) st_tag_bits(args->tsmp + w, (uint32_t)fin | (bad ? 0x80000000u : 0u), flow_tag(epoch, 0, FK_SMP));
}

// The sampler workgroup of the fused sampler, for the token after the one
// this launch forwards (number st->step + 1 of the loop): the step's 2 *
// vocab MT19937 draws (src/sampling.rs:198-214 consumes exactly that many),
// then the rest of choose() over the workers' candidate lists.  Every entry
// of the global top-k is within its worker's top-k list.  LB bounds the
// top-k threshold T from below: at least k entries are >= LB, and (LB being
// no smaller than any full list's k-th entry) every entry above LB is
// listed.  So T is the k-th listed entry >= LB when k of them exceed LB,
// and LB otherwise (the k-th entry overall when there is no bound).
// Survivors are the listed entries >= T plus, from lists cut at an entry
// equal to T, the worker's further entries equal to T (rescanned); then
// race_tail.  Live: the id becomes every row's next input and the state
// advances (ids, token log, end flag, step, positions, MT state).  lds:
// kSamplerLds bytes.
__device__ __forceinline__ void sampler_wg(const StepArgs* args, const HeadRows hr, int nwork, uint32_t epoch,
                                           bool live, float* lds) {
    const FusedSampler& fs = args->smp;
    const SampleArgs& a = fs.a;
    StepState* st = args->st;
    const int tid = threadIdx.x, V = a.vocab, K = fs.list;
    const int step = *gbl(&st->step) + 1;
    const bool greedy = a.mode == 0 || a.temperature == 0.0f;
    uint32_t* mts = reinterpret_cast<uint32_t*>(lds);                     // [640]
    int32_t* finw = reinterpret_cast<int32_t*>(lds + 640);                // [512]
    int32_t* rescan = finw + 512;                                         // [512]
    uint64_t* rlast = reinterpret_cast<uint64_t*>(rescan + 512);          // [512]
    uint64_t* C = rlast + 512;                                            // [kSurvivorMax]
    float* e_val = reinterpret_cast<float*>(C + kSurvivorMax);            // [kSurvivorMax]
    float* p_buf = e_val + kSurvivorMax;                                  // [kSurvivorMax]
    int* misc = reinterpret_cast<int*>(p_buf + kSurvivorMax);             // [32]
    uint64_t* red = reinterpret_cast<uint64_t*>(misc + 32);               // [8]
    if (!greedy) mt_fill(fs.mt, fs.draws, 2 * (size_t)V, mts, live);
    if (!gather_put<kStepThreads, 1>([=](int i) { return args->tsmp + i; }, nwork, flow_tag(epoch, 0, FK_SMP),
                                     [=](int i, uint32_t bits) { finw[i] = (int32_t)bits; }, st))
        return;
    int fin_me = 0, bad_me = 0;
    if (tid < nwork) {
        fin_me = finw[tid] & 0x7fffffff;
        bad_me = ((uint32_t)finw[tid] >> 31) & 1;
    }
    const int count = block_sum_i(fin_me, misc);
    const int bad = block_sum_i(bad_me, misc + 8);
    if ((a.mode == 1 && bad) || count == 0) {
        if (tid == 0) set_error(&st->error, count == 0 && !(a.mode == 1 && bad) ? 3 : 4);
        return;
    }
    int32_t id;
    if (greedy) {
        const uint64_t k = tid < nwork && fin_me > 0 ? ld_tag(fs.cand + tid) : ~0ull;
        id = (int32_t)(block_min_u64(k, red) & 0xffffffffu);
    } else {
        // LB, the larger of two bounds each with k entries at or above it:
        // the largest k-th entry of a full list, and the k-th largest of the
        // lists' first entries (one per worker)
        const uint64_t* mine = fs.cand + (size_t)tid * K;  // thread t < nwork reads worker t's list
        const uint64_t head_me = tid < nwork && fin_me > 0 ? ld_tag(mine) : ~0ull;
        const uint64_t last_me = tid < nwork && fin_me >= K ? ld_tag(mine + K - 1) : ~0ull;
        const uint64_t lb1 = block_min_u64(last_me, red);
        // the K-th smallest head: the present heads are distinct, and the
        // absent ones (~0) rank above them, so it is the head of rank K - 1,
        // or absent when fewer than K are present
        __shared__ uint64_t s_lb2;
        if (tid == 0) s_lb2 = ~0ull;
        C[tid] = head_me;
        __syncthreads();
        if (head_me != ~0ull && rank_below(C, nwork, head_me) == K - 1) s_lb2 = head_me;
        __syncthreads();
        const uint64_t lb2 = s_lb2;
        const uint64_t lb_key = kmin(lb1, lb2);
        const bool lb_none = lb_key == ~0ull;
        const float LB = lb_none ? -__builtin_huge_valf() : key_value(lb_key);
        __syncthreads();  // C is rewritten below
        // listed entries >= LB, into C (LDS; the overflow arrays beyond it):
        // thread t walks worker t's list (values non-increasing) until an
        // entry falls below LB, four loads in flight at a time
        uint64_t* dst = C;
        int cap = kSurvivorMax, nc = 0;
        const int listed = tid < nwork ? min(K, fin_me) : 0;
        for (int pass = 0; pass < 2; ++pass) {
            __syncthreads();
            if (tid == 0) misc[16] = 0;
            __syncthreads();
            bool more = listed > 0;
            for (int j0 = 0; more && j0 < listed; j0 += 4) {
                uint64_t k4[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) k4[u] = j0 + u < listed ? ld_tag(mine + j0 + u) : ~0ull;
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    if (j0 + u < listed && key_value(k4[u]) >= LB) {
                        const int at = atomicAdd(&misc[16], 1);
                        if (at < cap) dst[at] = k4[u];
                    } else {
                        more = false;
                    }
                }
            }
            __syncthreads();
            nc = misc[16];
            if (nc <= cap) break;
            dst = a.big;
            cap = a.big_cap;
        }
        __syncthreads();
        sort_distinct(dst, nc, reinterpret_cast<uint64_t*>(e_val));  // e_val is free until race_tail
        // T, and the survivors among the listed entries: a prefix of dst
        float T;
        if (lb_none) {
            T = key_value(dst[min(K, nc) - 1]);
        } else {
            int above = 0;
            for (int i = tid; i < nc; i += kStepThreads) above += key_value(dst[i]) > LB;
            above = block_sum_i(above, misc);
            T = above >= K ? key_value(dst[K - 1]) : LB;
        }
        int ns = 0;
        for (int i = tid; i < nc; i += kStepThreads) ns += key_value(dst[i]) >= T;
        ns = block_sum_i(ns, misc + 8);
        // lists cut at an entry equal to T: the worker's later entries equal to T
        if (tid == 0) misc[17] = 0;
        __syncthreads();
        if (tid < nwork && fin_me > K) {
            const uint64_t last = ld_tag(fs.cand + (size_t)tid * K + K - 1);
            if (key_value(last) >= T) {
                const int r = atomicAdd(&misc[17], 1);
                rescan[r] = tid;
                rlast[r] = last;
            }
        }
        __syncthreads();
        const int nres = misc[17];
        int n = ns;
        for (int pass = 0; pass < 2 && nres > 0; ++pass) {
            __syncthreads();
            if (tid == 0) misc[18] = ns;
            __syncthreads();
            for (int r = 0; r < nres; ++r) {
                const int lo = hr.r0(rescan[r], nwork), hi = hr.r1(rescan[r], nwork);
                const int extra = hr.extra(rescan[r]);
                for (int q = lo + tid; q < hi + (extra >= 0 ? 1 : 0); q += kStepThreads) {
                    const int i = q < hi ? q : extra;
                    const float v = ld_agent_f32(a.scores + i);
                    if (is_finite(v) && v >= T) {
                        const uint64_t k = order_key(v, i);
                        if (k > rlast[r]) {
                            const int at = atomicAdd(&misc[18], 1);
                            if (at < cap) dst[at] = k;
                        }
                    }
                }
            }
            __syncthreads();
            n = misc[18];
            if (n <= cap) break;
            // more survivors than LDS holds: the prefix moves to the overflow arrays
            for (int i = tid; i < ns; i += kStepThreads) a.big[i] = dst[i];
            dst = a.big;
            cap = a.big_cap;
        }
        __syncthreads();
        id = dst == C ? race_tail(a, step, C, e_val, p_buf, n, &misc[20], &misc[21])
                      : race_tail(a, step, a.big, a.big_e, a.big_p, n, &misc[20], &misc[21]);
    }
    if (live && tid == 0) {
        publish(a, step, id);
        for (int b = 0; b < a.rows; ++b) st->pos[b] += 1;
        st->step = step;
    }
}

// ---- the kernel ------------------------------------------------------------

typedef const __attribute__((address_space(4))) StepArgs* ArgsPtr;
typedef const __attribute__((address_space(4))) LayerDev* LayerPtr;

// Layer l's weight and norm pointers through the constant address space:
// scalar loads, which wait on nothing but themselves.  (A generic pointer
// would be read with a vector load, and on this architecture the wait for a
// vector load also waits for every store and load issued before it.)
__device__ __forceinline__ LayerPtr layer_at(ArgsPtr a, int l) { return (LayerPtr)a->layers + l; }

// The arguments through a pointer the compiler cannot follow from one phase
// to the next: fields are re-read (scalar loads) in the phase that uses them
// instead of being kept live, in scalar registers, across the whole launch.
__device__ __forceinline__ ArgsPtr fresh(ArgsPtr p) {
    asm volatile("" : "+s"(p));
    return p;
}

// The attention arguments of layer l for batch row b (field by field: a
// struct copy cannot bind to the constant address space).
__device__ __forceinline__ FlowAttn layer_attn(ArgsPtr a, const KvView& kv, int b, int l, uint32_t epoch,
                                               int wpg, int D, bool packed) {
    FlowAttn f;
    f.qkv = a->tqkv;
    f.qkv_stride = (a->heads + 2 * a->kv_heads) * D;
    f.packed = packed;
    f.kv_base = b == 0 ? kv.base[0] : kv.base[1];  // selects: no indexed struct copy
    f.cap = b == 0 ? kv.capacity[0] : kv.capacity[1];
    f.pos = *gbl(&a->st->pos[b]);
    f.layer = l;
    f.heads = a->heads;
    f.kv_heads = a->kv_heads;
    f.blk_stride = a->blk_stride;
    f.att_stride = a->heads * D;
    f.wpg = wpg;
    f.scale = a->scale;
    f.eps = a->eps;
    f.q_norm = layer_at(a, l)->q_norm;
    f.k_norm = layer_at(a, l)->k_norm;
    f.cos_t = a->rope_cos;
    f.sin_t = a->rope_sin;
    f.bmax = a->tbmax;
    f.bsum = a->tbsum;
    f.part = a->tpart;
    f.att = a->tatt;
    f.epoch = epoch;
    f.st = a->st;
    return f;
}

// G: query heads per KV head; MASK 0: every GEMV input is exactly 512 IT
// long, 1: the intermediate size is short of 512 * ITI (the down
// projection's rows are masked), 2: any input may be short of its 512 IT
// (every GEMV masked) and G is only the most query heads a KV head has (the
// shape's own at run time); TRACE: the traced
// instantiation; OE: the O projection's first weight items are requested
// during the attention, right after its q/k/v gather, instead of after it
// (long contexts: the attention is long enough that they land before its
// later gathers, which at short contexts they delay).
template <int B, int D, int G, int ITH, int ITQ, int ITI, int MASK, bool TRACE, bool OE>
__global__ __launch_bounds__(kStepThreads) void step_kernel(const StepArgs* args_dev, const StepCall call) {
    // 16-byte aligned whatever the static LDS before it: staged inputs and K/V
    // chunks are read with 16-byte LDS reads, which are split and slow when
    // misaligned
    extern __shared__ __align__(16) float lds[];
    __shared__ float res_s[B * kResRows];  // this workgroup's rows of x (residual)
    __shared__ float pk_s[kPairRowsMax];   // one row: a GEMV's outputs before they go out in pairs
    constexpr int RMAX = std::max(std::max(Ring<ITH, false>::SIZE, Ring<ITH, true>::SIZE),
                                  std::max(Ring<ITQ, false>::SIZE, Ring<ITI, false>::SIZE));
    constexpr bool MH = MASK == 2, MQ = MASK == 2, MI = MASK >= 1;  // masked: hidden, heads * D, intermediate
    const ArgsPtr args = (ArgsPtr)args_dev;
    const int tid = threadIdx.x, wg = blockIdx.x;
    // with the fused sampler the last workgroup is the sampler and the
    // others (the workers) share the layers
    const int nwg = call.sample ? (int)gridDim.x - 1 : (int)gridDim.x;
    StepState* st = fresh(args)->st;
    // after an error, or once the sampler chose the phase's end token (the
    // reference stops before that token's forward, src/sampling.rs:268-271)
    if (ld_dev_i(&st->error) || ld_dev_i(&st->done)) return;
    const int seq = *gbl(&st->seq);
    const uint32_t epoch = ((uint32_t)seq + 1u) & 0xFFFFFu;
    const HeadRows hr{call.head_lo, call.head_n, call.head_stop};
    if (call.sample && wg == nwg) {
        sampler_wg(args_dev, hr, nwg, epoch, call.sample == 1, lds);
        // the next launch's epoch: every worker read seq before it announced
        // its candidates, which the sampler waited for
        if (tid == 0) *gblw(&st->seq) = seq + 1;
        return;
    }
    uint4 ring[RMAX];
    float gam[ITH];
    double e_sum[B], w_sum[B];  // this thread's shares of the next RMSNorm's sums
    Tracer<TRACE> tr{call.trace, call.trace_slots, 0};
    tr.mark();

    // Embedding (src/model.rs:452-464): the whole of x staged for the first
    // norm, straight from the table.
    {
        ArgsPtr a = fresh(args);
        const int H = a->hidden, qkvw = (a->heads + 2 * a->kv_heads) * D;
        int ids[B];
        for (int b = 0; b < B; ++b) {
            ids[b] = *gbl(&st->ids[b]);
            if (ids[b] < 0 || ids[b] >= a->vocab) {
                if (tid == 0) set_error(&st->error, 2);
                return;
            }
        }
        // the rows' embeddings are requested before the ring's first items
        // (loads complete in order: staging them then waits for them alone);
        // element tid + 512 j (H <= 512 ITH), unconditional loads (past the
        // end they re-read element H - 1, never staged)
        float ev[B][ITH];
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const auto* e = gbl(a->embed + (size_t)ids[b] * H);
#pragma unroll
            for (int j = 0; j < ITH; ++j) ev[b][j] = bf16(e[min(tid + j * kStepThreads, H - 1)]);
        }
        load_gamma<ITH>(layer_at(a, 0)->in_norm, H, gam);
        prefetch_ring<ITH, false, MH>(layer_at(a, 0)->wqkv, nullptr, H, xlo<B>(qkvw, wg, nwg),
                                  xlo<B>(qkvw, wg + 1, nwg), qkvw, ring);
#pragma unroll
        for (int b = 0; b < B; ++b)
#pragma unroll
            for (int j = 0; j < ITH; ++j)
                if (tid + j * kStepThreads < H) lds[b * H + tid + j * kStepThreads] = ev[b][j];
        __syncthreads();
    }

    // Layers, then (when the call asks for logits) one more pass of the
    // norm + GEMV head with the final norm and the LM head: one copy of that
    // code serves both (the per-layer code has to fit the instruction cache).
    const int layers_n = fresh(args)->layers_n;
    const int passes = layers_n + (call.head ? 1 : 0);
    for (int l = 0; l < passes; ++l) {
        const bool last = l == layers_n;
        // ---- input RMSNorm + fused QKV projection (final norm + LM head) ----
        {
            ArgsPtr a = fresh(args);
            const int lc = min(l, layers_n - 1);  // layer pointers are never read past the table
            const int H = a->hidden, n = last ? hr.n : (a->heads + 2 * a->kv_heads) * D;
            const uint16_t* w = last ? a->lm_head + (size_t)hr.lo * H : layer_at(a, lc)->wqkv;
            // (the LM head's rows are the fused sampler's HeadRows split)
            const int r0 = last ? part_lo(n, wg, nwg) : xlo<B>(n, wg, nwg);
            const int r1 = last ? part_lo(n, wg + 1, nwg) : xlo<B>(n, wg + 1, nwg);
            if (l > 0) {
                // the gammas and first weights go out before the wait
                load_gamma<ITH>(last ? a->final_norm : layer_at(a, lc)->in_norm, H, gam);
                prefetch_ring<ITH, false, MH>(w, nullptr, H, r0, r1, n, ring);
                a = fresh(args);
                if (!stage_x<B, ITH>(lds, a->tx, H, flow_tag(epoch, l - 1, FK_XD), st, e_sum, w_sum)) return;
            } else if constexpr (kPack<B>) {
                norm_partials<kStepThreads, B>(lds, H, e_sum, w_sum);  // x from the embedding
            }
            // this workgroup's rows of x: the residual of the O projection
            if (!last) copy_res<B>(res_s, lds, H, xlo<B>(H, wg, nwg), xlo<B>(H, wg + 1, nwg));
            a = fresh(args);
            norm_rows<B, ITH>(lds, H, gam, a->eps, wg == 0 && !last ? &st->norm_fallbacks : nullptr, e_sum, w_sum);
            tr.mark();
            a = fresh(args);
            gemv_ring<B, EPI_STORE, ITH, MH, kPack<B>, kPair<B>>(
                w, nullptr, lds, H, last ? a->logits + hr.lo : nullptr, last ? nullptr : a->tqkv,
                flow_tag(epoch, l, FK_QKV), last ? a->vocab : n, r0, r1, n, ring, nullptr, pk_s);
            tr.mark();
        }
        if (last) break;
        // ---- QK-norm + RoPE + KV append + attention ----
        {
            ArgsPtr a = fresh(args);
            const int groups = a->kv_heads * B, wpg = nwg / groups;
            const int group = wg / wpg, kvh = a->kv_heads;
            const int H = a->hidden, qw = a->heads * D;
            const int h0 = xlo<B>(H, wg, nwg), h1 = xlo<B>(H, wg + 1, nwg);
            auto pre_o = [&] {
                if constexpr (OE) prefetch_ring<ITQ, false, MQ>(layer_at(fresh(args), l)->wo, nullptr, qw, h0, h1, H, ring);
            };
            if (group < groups) {
                const FlowAttn fa = layer_attn(a, call.kv, group / kvh, l, epoch, wpg, D, kPack<B>);
                if (!attn_flow<kStepThreads, D, G, MASK == 2, false, OE, !OE && MASK == 0>(fa, wg % wpg, group % kvh, group / kvh, lds, [&] { tr.mark(); },
                                                   pre_o))
                    return;
            } else {
                pre_o();
                for (int i = 0; i < 6; ++i) tr.mark();  // a workgroup past the groups: no attention
            }
            tr.mark();
        }
        // ---- O projection + residual ----
        {
            ArgsPtr a = fresh(args);
            const int H = a->hidden, qw = a->heads * D;
            const int h0 = xlo<B>(H, wg, nwg), h1 = xlo<B>(H, wg + 1, nwg);
            if constexpr (!OE) prefetch_ring<ITQ, false, MQ>(layer_at(a, l)->wo, nullptr, qw, h0, h1, H, ring);
            a = fresh(args);
            if (!stage_att<B, ITQ>(lds, a->tatt, qw, flow_tag(epoch, l, FK_ATT), st)) return;
            tr.mark();
            a = fresh(args);
            gemv_ring<B, EPI_RESID, ITQ, MQ, kPack<B>, kPair<B>>(layer_at(a, l)->wo, nullptr, lds, qw, nullptr, a->tx,
                                                                   flow_tag(epoch, l, FK_XO), H, h0, h1, H, ring, res_s, pk_s);
            tr.mark();
        }
        // ---- post-attention RMSNorm + gate/up + SwiGLU ----
        {
            ArgsPtr a = fresh(args);
            const int H = a->hidden, I = a->intermediate;
            load_gamma<ITH>(layer_at(a, l)->post_norm, H, gam);
            prefetch_ring<ITH, true, MH>(layer_at(a, l)->wg, layer_at(a, l)->wu, H, xlo<B>(I, wg, nwg), xlo<B>(I, wg + 1, nwg), I, ring);
            a = fresh(args);
            if (!stage_x<B, ITH>(lds, a->tx, H, flow_tag(epoch, l, FK_XO), st, e_sum, w_sum)) return;
            // this workgroup's rows of x: the residual of the down projection
            copy_res<B>(res_s, lds, H, xlo<B>(H, wg, nwg), xlo<B>(H, wg + 1, nwg));
            a = fresh(args);
            norm_rows<B, ITH>(lds, H, gam, a->eps, wg == 0 ? &st->norm_fallbacks : nullptr, e_sum, w_sum);
            tr.mark();
            a = fresh(args);
            gemv_ring<B, EPI_SWIGLU, ITH, MH, kPack<B>, kPair<B>>(
                layer_at(a, l)->wg, layer_at(a, l)->wu, lds, H, nullptr, a->tact, flow_tag(epoch, l, FK_ACT), I,
                xlo<B>(I, wg, nwg), xlo<B>(I, wg + 1, nwg), I, ring, nullptr, pk_s);
            tr.mark();
        }
        // ---- down projection + residual ----
        {
            ArgsPtr a = fresh(args);
            const int H = a->hidden, I = a->intermediate;
            const int h0 = xlo<B>(H, wg, nwg), h1 = xlo<B>(H, wg + 1, nwg);
            prefetch_ring<ITI, false, MI>(layer_at(a, l)->wd, nullptr, I, h0, h1, H, ring);
            a = fresh(args);
            if (!stage_rows<B, ITI>(lds, a->tact, I, flow_tag(epoch, l, FK_ACT), st)) return;
            tr.mark();
            a = fresh(args);
            gemv_ring<B, EPI_RESID, ITI, MI, kPack<B>, kPair<B>>(layer_at(a, l)->wd, nullptr, lds, I, nullptr, a->tx,
                                                                   flow_tag(epoch, l, FK_XD), H, h0, h1, H, ring, res_s, pk_s);
            tr.mark();
        }
    }
    if (call.head && hr.stop >= 0) {
        // a phase's LM head (project_phase, src/model.rs:478-507): worker 0
        // computes the stop row from the normalised x still staged in LDS,
        // and every worker writes -inf to its share of the other entries
        ArgsPtr a = fresh(args);
        const int H = a->hidden, V = a->vocab;
        const uint16_t* ws = a->lm_head + (size_t)hr.stop * H;
        const int rn = wg == 0 ? 1 : 0;
        prefetch_ring<ITH, false, MH>(ws, nullptr, H, 0, rn, 1, ring);
        gemv_ring<B, EPI_STORE, ITH, MH, kPack<B>>(ws, nullptr, lds, H, a->logits + hr.stop, nullptr, 0, V, 0, rn,
                                                      1, ring);
        const int f0 = part_lo(V, wg, nwg), f1 = part_lo(V, wg + 1, nwg);
        for (int b = 0; b < B; ++b)
            for (int i = f0 + tid; i < f1; i += kStepThreads)
                if ((i < hr.lo || i >= hr.lo + hr.n) && i != hr.stop)
                    gblw(a->logits)[(size_t)b * V + i] = -__builtin_huge_valf();
    }
    // the fused sampler's share of this workgroup: its rows of the LM head
    if (call.sample && call.head) score_rows(args_dev, hr.r0(wg, nwg), hr.r1(wg, nwg), hr.extra(wg), wg, epoch, lds);
    // The next launch's epoch (the sampler workgroup's when there is one).
    // Workgroup 0 cannot get here before every workgroup has read seq: its
    // final input needs every workgroup's output.
    if (!call.sample && wg == 0 && tid == 0) *gblw(&st->seq) = seq + 1;
}

template <int B, int D, int G, int ITH, int ITQ, int ITI, int MASK>
static hipError_t launch_step_t(hipStream_t s, const StepArgs* dev, const StepCall& call, int nwg, size_t lds) {
    if (call.trace)
        step_kernel<B, D, G, ITH, ITQ, ITI, MASK, true, false><<<nwg, kStepThreads, lds, s>>>(dev, call);
    else if (call.context >= kOEarlyKeys)
        step_kernel<B, D, G, ITH, ITQ, ITI, MASK, false, true><<<nwg, kStepThreads, lds, s>>>(dev, call);
    else
        step_kernel<B, D, G, ITH, ITQ, ITI, MASK, false, false><<<nwg, kStepThreads, lds, s>>>(dev, call);
    return hipGetLastError();
}

// The compiled step kernels.  Two shapes have their own, unmasked: the
// 3B-class one (hidden 3072, 24 x 128 query heads, 3 per KV head,
// intermediate 8192) and the YuE2 one (2048, 16 x 128, 2 per KV head, 6144).
// Any other shape with head_dim 64 or 128, at most 8 query heads per KV
// head, hidden and heads * head_dim at most 4608 and intermediate at most
// 14336 (hidden and intermediate multiples of 8) runs on a generic kernel
// of its head_dim (one for up to 4 query heads per KV head, one for up to
// 8), every GEMV input masked to its length.
enum class StepShape { kNone, k3B, kYue2, kAny128, kAny64, kAny128G8, kAny64G8 };

static StepShape step_shape(int hidden, int heads, int kv_heads, int dim, int inter) {
    if (kv_heads < 1 || heads % kv_heads) return StepShape::kNone;
    const int G = heads / kv_heads, qw = heads * dim;
    if (dim == 128 && G == 3 && hidden == 3072 && qw == 3072 && inter == 8192) return StepShape::k3B;
    if (dim == 128 && G == 2 && hidden == 2048 && qw == 2048 && inter == 6144) return StepShape::kYue2;
    const bool fits = G <= 8 && hidden >= 8 && hidden <= 512 * kStepAnyIth && hidden % 8 == 0 && qw <= 512 * kStepAnyItq &&
                      inter >= 8 && inter <= 512 * kStepAnyIti && inter % 8 == 0;
    if (!fits || (dim != 128 && dim != 64)) return StepShape::kNone;
    if (G <= 4) return dim == 128 ? StepShape::kAny128 : StepShape::kAny64;
    return dim == 128 ? StepShape::kAny128G8 : StepShape::kAny64G8;
}

bool step_supported(const Yue2Config& c, int rows, int nwg) {
    if (step_shape(c.hidden_size, c.num_attention_heads, c.num_key_value_heads, c.head_dim, c.intermediate_size) ==
        StepShape::kNone)
        return false;
    const int G = c.num_attention_heads / c.num_key_value_heads;
    if (rows < 1 || rows > 2 || nwg < c.num_key_value_heads * rows) return false;
    const int wpg = nwg / (c.num_key_value_heads * rows);  // workgroups past the groups take no attention
    const int max_blocks = (c.max_position_embeddings + kBlockKeys - 1) / kBlockKeys;
    const int bpw = attn_bpw_max(max_blocks, wpg);
    // the attention's p (G x bpw blocks of f32) is staged in its K region
    // (the merge's partials, G x head_dim x bpw + blocks words at most, are
    // gathered into the K/V region with rows padded to four floats)
    const int merge_words = G * c.head_dim * bpw + 2 * max_blocks;
    // (with one row each workgroup's share of an exchanged output is even:
    // at most 2 ceil(n / 2 / nwg) rows, paired in LDS)
    auto share = [&](int n) { return std::max((n + nwg - 1) / nwg, 2 * ((n / 2 + nwg - 1) / nwg)); };
    const int qkv_rows = (c.num_attention_heads + 2 * c.num_key_value_heads) * c.head_dim;
    const bool pairs_fit = share(c.hidden_size) <= kPairRowsMax && share(c.intermediate_size) <= kPairRowsMax &&
                           share(qkv_rows) <= kPairRowsMax && c.hidden_size % 2 == 0 &&
                           c.intermediate_size % 2 == 0 && qkv_rows % 2 == 0;
    return pairs_fit && G <= 8 && share(c.hidden_size) <= kResRows && max_blocks <= 24576 / kBlockKeys &&
           (size_t)(merge_words + 3 * G * c.head_dim) * 4 <= (size_t)2 * kAttnChunk * kBlockKeys * c.head_dim * 2 &&
           G * bpw * kBlockKeys * 4 <= kAttnChunk * kBlockKeys * c.head_dim * 2;
}

size_t step_lds_bytes(const StepArgs& a, int nwg) {
    const int kmax = std::max(std::max(a.hidden, a.intermediate), a.heads * a.head_dim);
    const int G = a.heads / a.kv_heads, wpg = nwg / (a.kv_heads * a.rows);
    const int bpw = attn_bpw_max(a.max_blocks, wpg);
    // staged GEMV inputs; the attention (staged K/V chunks + scores; its
    // merge reuses the K/V region)
    return std::max((size_t)a.rows * kmax * sizeof(float), attn_flow_lds(G, a.head_dim, bpw));
}

template <int B, int D, int G, int ITH, int ITQ, int ITI, int MASK>
static int resident_t(size_t lds) {
    // every instantiation a launch may pick must fit one workgroup per CU
    int n = 0, n2 = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &n, reinterpret_cast<const void*>(step_kernel<B, D, G, ITH, ITQ, ITI, MASK, false, false>),
            kStepThreads, lds) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &n2, reinterpret_cast<const void*>(step_kernel<B, D, G, ITH, ITQ, ITI, MASK, false, true>),
            kStepThreads, lds) != hipSuccess)
        return 0;
    return std::min(n, n2);
}

size_t step_launch_lds(const StepArgs& a, int nwg, int sample) {
    const size_t lds = step_lds_bytes(a, sample ? nwg - 1 : nwg);
    return sample ? std::max(lds, kSamplerLds) : lds;
}

int step_resident_per_cu(const StepArgs& a, int nwg, int sample) {
    const size_t lds = step_launch_lds(a, nwg, sample);
    if (lds > kStepLdsMax) return 0;
    switch (step_shape(a.hidden, a.heads, a.kv_heads, a.head_dim, a.intermediate)) {
        case StepShape::k3B:
            return a.rows == 1 ? resident_t<1, 128, 3, 6, 6, 16, 0>(lds) : resident_t<2, 128, 3, 6, 6, 16, 0>(lds);
        case StepShape::kYue2:
            return a.rows == 1 ? resident_t<1, 128, 2, 4, 4, 12, 0>(lds) : resident_t<2, 128, 2, 4, 4, 12, 0>(lds);
        case StepShape::kAny128:
            return a.rows == 1 ? resident_t<1, 128, 4, kStepAnyIth, kStepAnyItq, kStepAnyIti, 2>(lds)
                               : resident_t<2, 128, 4, kStepAnyIth, kStepAnyItq, kStepAnyIti, 2>(lds);
        case StepShape::kAny64:
            return a.rows == 1 ? resident_t<1, 64, 4, kStepAnyIth, kStepAnyItq, kStepAnyIti, 2>(lds)
                               : resident_t<2, 64, 4, kStepAnyIth, kStepAnyItq, kStepAnyIti, 2>(lds);
        case StepShape::kAny128G8:
            return a.rows == 1 ? resident_t<1, 128, 8, kStepAnyIth, kStepAnyItq, kStepAnyIti, 2>(lds)
                               : resident_t<2, 128, 8, kStepAnyIth, kStepAnyItq, kStepAnyIti, 2>(lds);
        case StepShape::kAny64G8:
            return a.rows == 1 ? resident_t<1, 64, 8, kStepAnyIth, kStepAnyItq, kStepAnyIti, 2>(lds)
                               : resident_t<2, 64, 8, kStepAnyIth, kStepAnyItq, kStepAnyIti, 2>(lds);
        default:
            return 0;
    }
}

bool fused_sampler_supported(const Yue2Config& c, int rows, int nwg, int mode, float temperature, int top_k,
                             int head_n) {
    const int workers = nwg - 1;
    if (workers < 1 || !step_supported(c, rows, workers)) return false;
    if ((head_n + workers - 1) / workers + 1 > kFusedRowsMax) return false;  // a worker's rows and the stop row
    const bool greedy = mode == 0 || temperature == 0.0f;
    return greedy || (top_k >= 1 && top_k <= kFusedListMax);
}

hipError_t launch_step(hipStream_t s, const StepArgs* dev, const StepArgs& a, const StepCall& call, int nwg) {
    const size_t lds = step_launch_lds(a, nwg, call.sample);
    if (lds > kStepLdsMax) return hipErrorInvalidValue;
    switch (step_shape(a.hidden, a.heads, a.kv_heads, a.head_dim, a.intermediate)) {
        case StepShape::k3B:
            return a.rows == 1 ? launch_step_t<1, 128, 3, 6, 6, 16, 0>(s, dev, call, nwg, lds)
                               : launch_step_t<2, 128, 3, 6, 6, 16, 0>(s, dev, call, nwg, lds);
        case StepShape::kYue2:
            return a.rows == 1 ? launch_step_t<1, 128, 2, 4, 4, 12, 0>(s, dev, call, nwg, lds)
                               : launch_step_t<2, 128, 2, 4, 4, 12, 0>(s, dev, call, nwg, lds);
        case StepShape::kAny128:
            return a.rows == 1 ? launch_step_t<1, 128, 4, kStepAnyIth, kStepAnyItq, kStepAnyIti, 2>(s, dev, call, nwg, lds)
                               : launch_step_t<2, 128, 4, kStepAnyIth, kStepAnyItq, kStepAnyIti, 2>(s, dev, call, nwg, lds);
        case StepShape::kAny64:
            return a.rows == 1 ? launch_step_t<1, 64, 4, kStepAnyIth, kStepAnyItq, kStepAnyIti, 2>(s, dev, call, nwg, lds)
                               : launch_step_t<2, 64, 4, kStepAnyIth, kStepAnyItq, kStepAnyIti, 2>(s, dev, call, nwg, lds);
        case StepShape::kAny128G8:
            return a.rows == 1 ? launch_step_t<1, 128, 8, kStepAnyIth, kStepAnyItq, kStepAnyIti, 2>(s, dev, call, nwg, lds)
                               : launch_step_t<2, 128, 8, kStepAnyIth, kStepAnyItq, kStepAnyIti, 2>(s, dev, call, nwg, lds);
        case StepShape::kAny64G8:
            return a.rows == 1 ? launch_step_t<1, 64, 8, kStepAnyIth, kStepAnyItq, kStepAnyIti, 2>(s, dev, call, nwg, lds)
                               : launch_step_t<2, 64, 8, kStepAnyIth, kStepAnyItq, kStepAnyIti, 2>(s, dev, call, nwg, lds);
        default:
            return hipErrorInvalidValue;
    }
}

}  // namespace y2
