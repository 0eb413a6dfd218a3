// step.hip -- the persistent token-step kernel: one launch runs a whole
// decode token (embedding, every layer, final norm and LM head) for one or
// two batch rows (Model::hidden + forward, src/model.rs:452-591).
//
// Why one kernel: each phase of the step (norm -> QKV -> attention -> O ->
// norm -> gate/up -> down) depends on the complete output of the previous
// one, so a kernel per phase pays a launch, a ramp-up and a drain for every
// dependency -- about 5 us each, ~140 times per token.  Here one workgroup
// per CU stays resident for the whole step.  Phases are separated by grid
// barriers, and before arriving at a barrier every wave already requests the
// weights of its first row of the next GEMV, so HBM keeps streaming while the
// barrier and the next phase's RMSNorm resolve.
//
// Work split (n rows of a GEMV over G workgroups): workgroup w owns rows
// [w*n/G, (w+1)*n/G); its 8 waves take every 8th row, double-buffered.  The
// arithmetic of every row is the DOT order of dev_gemv.h, the attention is
// dev_attn.h with one (kv head, row) group per G/(kv_heads*rows) workgroups,
// so the results equal the per-phase kernels' bit for bit.
//
// Barriers: a counter per launch (two, alternating with the launch sequence
// number so the idle one can be cleared), bounded spins; a timeout sets the
// device error and every workgroup leaves, so a launch always terminates.
// The launch uses exactly one workgroup per CU, so all are co-resident.
#include <algorithm>

#include "dev_attn.h"
#include "dev_gemv.h"
#include "kernels.h"
#include "runtime.h"
#include "step.h"

namespace y2 {

constexpr int kStepThreads = 512;
constexpr int kStepWaves = kStepThreads / 64;
constexpr int kDevErrBarrier = 7;

// Optional trace: thread 0 of each workgroup stamps the device wall clock
// (100 MHz) into trace[slot * gridDim.x + workgroup]; slots past the buffer
// are dropped.
struct Tracer {
    unsigned long long* buf;
    int slots, slot;
    __device__ __forceinline__ void mark() {
        if (buf && threadIdx.x == 0 && slot < slots) buf[(size_t)slot * gridDim.x + blockIdx.x] = wall_clock64();
        ++slot;
    }
};

// Grid barrier number `epoch` of this launch.  Thread 0 arrives with a
// release add (writes this XCD's dirty L2 lines back) and spins on relaxed
// agent-scope loads, which read through to memory without touching the
// caches; one acquire fence after the spin (L1/L2 invalidate) makes the other
// workgroups' results visible, and the workgroup barrier passes that on.
__device__ bool grid_sync(int* bar, int epoch, StepState* st, Tracer& tr) {
    __shared__ int s_ok;
    __syncthreads();
    tr.mark();
    if (threadIdx.x == 0) {
        __hip_atomic_fetch_add(bar, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        const int target = epoch * (int)gridDim.x;
        int ok = 1;
        unsigned spins = 0;
        while (__hip_atomic_load(bar, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
            if (++spins > (1u << 22) ||
                __hip_atomic_load(&st->error, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
                atomicCAS(&st->error, 0, kDevErrBarrier);
                ok = 0;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        s_ok = ok;
    }
    tr.mark();
    __syncthreads();
    return s_ok != 0;
}

__device__ __forceinline__ int part_lo(int n, int w, int parts) { return (int)(((long)n * w) / parts); }

// Request this wave's first row of rows [r0, r1) (both matrices for a pair).
// The load is unconditional (a wave without a row re-reads the range's last
// row, or row 0 for an empty range) so the buffer is provably overwritten here
// and holds no live values between phases.
template <int IT, bool PAIR>
__device__ __forceinline__ void prefetch_first(const uint16_t* w, const uint16_t* w2, int k, int r0,
                                               int r1, uint4* buf) {
    const int lane = threadIdx.x & 63;
    const int row = max(min(r0 + (threadIdx.x >> 6), r1 - 1), 0);
    load_row<IT>(w, row, k, lane, buf);
    if constexpr (PAIR) load_row<IT>(w2, row, k, lane, buf + IT);
}

// Rows [r0, r1) of y = W xs with epilogue EPI; buf holds each wave's first row.
template <int B, int EPI, int IT>
__device__ __forceinline__ void gemv_rows(const uint16_t* w, const uint16_t* w2, const float* xs, int k,
                                          float* y, int y_stride, int r0, int r1, uint4* buf) {
    constexpr bool PAIR = EPI == EPI_SWIGLU;
    const int lane = threadIdx.x & 63;
    int row = r0 + (threadIdx.x >> 6);
    float acc[B], acc2[B];
    if constexpr (IT > 8) {
        // single buffer: one long row per wave is enough bytes in flight
        while (row < r1) {
            dot_rows<B, IT, PAIR>(xs, k, lane, buf, buf + IT, acc, acc2);
            if (lane == 0)
#pragma unroll
                for (int b = 0; b < B; ++b) gemv_store<EPI>(y + (size_t)b * y_stride + row, acc[b], acc2[b]);
            row += kStepWaves;
            if (row < r1) {
                load_row<IT>(w, row, k, lane, buf);
                if constexpr (PAIR) load_row<IT>(w2, row, k, lane, buf + IT);
            }
        }
        return;
    }
    uint4 nb[PAIR ? 2 * IT : IT];
    while (row < r1) {
        int next = row + kStepWaves;
        if (next < r1) {
            load_row<IT>(w, next, k, lane, nb);
            if constexpr (PAIR) load_row<IT>(w2, next, k, lane, nb + IT);
        }
        dot_rows<B, IT, PAIR>(xs, k, lane, buf, buf + IT, acc, acc2);
        if (lane == 0)
#pragma unroll
            for (int b = 0; b < B; ++b) gemv_store<EPI>(y + (size_t)b * y_stride + row, acc[b], acc2[b]);
        row = next;
        if (row >= r1) break;
        next = row + kStepWaves;
        if (next < r1) {
            load_row<IT>(w, next, k, lane, buf);
            if constexpr (PAIR) load_row<IT>(w2, next, k, lane, buf + IT);
        }
        dot_rows<B, IT, PAIR>(xs, k, lane, nb, nb + IT, acc, acc2);
        if (lane == 0)
#pragma unroll
            for (int b = 0; b < B; ++b) gemv_store<EPI>(y + (size_t)b * y_stride + row, acc[b], acc2[b]);
        row = next;
    }
}

// xs[b*k + i] = src[b*stride + i]
template <int B>
__device__ __forceinline__ void stage(float* xs, const float* src, int stride, int k) {
#pragma unroll
    for (int b = 0; b < B; ++b)
        for (int i = threadIdx.x; i < k; i += kStepThreads) xs[b * k + i] = src[(size_t)b * stride + i];
    __syncthreads();
}

// xs[b] = RMSNorm(xs[b]) with gammas g (Norm::apply, src/tensor.rs:1140-1157).
template <int B>
__device__ __forceinline__ void norm_rows(float* xs, int k, const float* g, float eps, int* fallbacks) {
#pragma unroll
    for (int b = 0; b < B; ++b) {
        float* xb = xs + b * k;
        const float s = norm_scale_block<kStepThreads>(xb, k, eps, fallbacks);
        for (int i = threadIdx.x; i < k; i += kStepThreads) xb[i] = rb(rb(xb[i] * s) * g[i]);
    }
    __syncthreads();
}

template <int B, int D, int ITH, int ITQ, int ITI>
__global__ __launch_bounds__(kStepThreads) void step_kernel(const StepArgs a) {
    extern __shared__ float lds[];
    constexpr int PMAX = std::max(std::max(2 * ITH, ITQ), ITI);
    const int tid = threadIdx.x, wg = blockIdx.x, nwg = gridDim.x;
    StepState* st = a.st;
    if (st->error) return;
    const int seq = st->seq;
    int* bar = a.bars + (seq & 1);
    if (wg == 0 && tid == 0) a.bars[(seq + 1) & 1] = 0;
    int epoch = 0;
    const int H = a.hidden, I = a.intermediate, qw = a.heads * D;
    const int qkvw = qw + 2 * a.kv_heads * D;
    int* fallbacks = wg == 0 ? &st->norm_fallbacks : nullptr;
    uint4 pre[PMAX];
    Tracer tr{a.trace, a.trace_slots, 0};
    tr.mark();

    // Embedding (src/model.rs:452-464): this workgroup's slice of x, and the
    // whole of x staged for the first norm.
    for (int b = 0; b < B; ++b) {
        const int id = st->ids[b];
        if (id < 0 || id >= a.vocab) {
            if (tid == 0) atomicCAS(&st->error, 0, 2);
            return;
        }
    }
    {
        const int lo = part_lo(H, wg, nwg), hi = part_lo(H, wg + 1, nwg);
        for (int b = 0; b < B; ++b) {
            const uint16_t* e = a.embed + (size_t)st->ids[b] * H;
            for (int i = lo + tid; i < hi; i += kStepThreads) a.x[(size_t)b * H + i] = bf16(e[i]);
        }
    }
    {
        const int r0 = part_lo(qkvw, wg, nwg), r1 = part_lo(qkvw, wg + 1, nwg);
        prefetch_first<ITH, false>(a.layers[0].wqkv, nullptr, H, r0, r1, pre);
    }
    for (int b = 0; b < B; ++b) {
        const uint16_t* e = a.embed + (size_t)st->ids[b] * H;
        for (int i = tid; i < H; i += kStepThreads) lds[b * H + i] = bf16(e[i]);
    }
    __syncthreads();

    const int groups = a.kv_heads * B, wpg = nwg / groups;
    const int group = wg / wpg, wg_in = wg % wpg;
    for (int l = 0; l < a.layers_n; ++l) {
        const LayerDev& Lw = a.layers[l];
        // ---- input RMSNorm + fused QKV projection ----
        if (l > 0) stage<B>(lds, a.x, H, H);
        norm_rows<B>(lds, H, Lw.in_norm, a.eps, fallbacks);
        tr.mark();
        {
            const int r0 = part_lo(qkvw, wg, nwg), r1 = part_lo(qkvw, wg + 1, nwg);
            gemv_rows<B, EPI_STORE, ITH>(Lw.wqkv, nullptr, lds, H, a.qkv, qkvw, r0, r1, pre);
        }
        if (!grid_sync(bar, ++epoch, st, tr)) return;
        // ---- QK-norm + RoPE + KV append + attention ----
        {
            AttnArgs at = a.attn;
            at.layer = l;
            at.q_norm = Lw.q_norm;
            at.k_norm = Lw.k_norm;
            if (!attn_group<kStepThreads, D, 4>(at, wg_in, group % a.kv_heads, group / a.kv_heads, lds)) return;
        }
        {
            const int r0 = part_lo(H, wg, nwg), r1 = part_lo(H, wg + 1, nwg);
            prefetch_first<ITQ, false>(Lw.wo, nullptr, qw, r0, r1, pre);
        }
        if (!grid_sync(bar, ++epoch, st, tr)) return;
        // ---- O projection + residual ----
        stage<B>(lds, a.att, qw, qw);
        tr.mark();
        {
            const int r0 = part_lo(H, wg, nwg), r1 = part_lo(H, wg + 1, nwg);
            gemv_rows<B, EPI_RESID, ITQ>(Lw.wo, nullptr, lds, qw, a.x, H, r0, r1, pre);
        }
        {
            const int r0 = part_lo(I, wg, nwg), r1 = part_lo(I, wg + 1, nwg);
            prefetch_first<ITH, true>(Lw.wg, Lw.wu, H, r0, r1, pre);
        }
        if (!grid_sync(bar, ++epoch, st, tr)) return;
        // ---- post-attention RMSNorm + gate/up + SwiGLU ----
        stage<B>(lds, a.x, H, H);
        norm_rows<B>(lds, H, Lw.post_norm, a.eps, fallbacks);
        tr.mark();
        {
            const int r0 = part_lo(I, wg, nwg), r1 = part_lo(I, wg + 1, nwg);
            gemv_rows<B, EPI_SWIGLU, ITH>(Lw.wg, Lw.wu, lds, H, a.act, I, r0, r1, pre);
        }
        {
            const int r0 = part_lo(H, wg, nwg), r1 = part_lo(H, wg + 1, nwg);
            prefetch_first<ITI, false>(Lw.wd, nullptr, I, r0, r1, pre);
        }
        if (!grid_sync(bar, ++epoch, st, tr)) return;
        // ---- down projection + residual ----
        stage<B>(lds, a.act, I, I);
        tr.mark();
        {
            const int r0 = part_lo(H, wg, nwg), r1 = part_lo(H, wg + 1, nwg);
            gemv_rows<B, EPI_RESID, ITI>(Lw.wd, nullptr, lds, I, a.x, H, r0, r1, pre);
        }
        if (l + 1 < a.layers_n) {
            const int r0 = part_lo(qkvw, wg, nwg), r1 = part_lo(qkvw, wg + 1, nwg);
            prefetch_first<ITH, false>(a.layers[l + 1].wqkv, nullptr, H, r0, r1, pre);
        } else if (a.head) {
            const int r0 = part_lo(a.vocab, wg, nwg), r1 = part_lo(a.vocab, wg + 1, nwg);
            prefetch_first<ITH, false>(a.lm_head, nullptr, H, r0, r1, pre);
        }
        if (!grid_sync(bar, ++epoch, st, tr)) return;
    }
    // ---- final norm + LM head (src/model.rs:465-468, 590) ----
    if (a.head) {
        stage<B>(lds, a.x, H, H);
        norm_rows<B>(lds, H, a.final_norm, a.eps, nullptr);
        const int r0 = part_lo(a.vocab, wg, nwg), r1 = part_lo(a.vocab, wg + 1, nwg);
        gemv_rows<B, EPI_STORE, ITH>(a.lm_head, nullptr, lds, H, a.logits, a.vocab, r0, r1, pre);
    }
    if (wg == 0 && tid == 0) st->seq = seq + 1;
}

template <int B, int D, int ITH, int ITQ, int ITI>
static hipError_t launch_step_t(hipStream_t s, const StepArgs& a, int nwg, size_t lds) {
    step_kernel<B, D, ITH, ITQ, ITI><<<nwg, kStepThreads, lds, s>>>(a);
    return hipGetLastError();
}

// Shapes with a compiled step kernel: {head_dim, iterations for hidden,
// for heads*head_dim, for intermediate}.
bool step_supported(const Yue2Config& c, int rows, int nwg) {
    const int ith = (c.hidden_size / 8 + 63) / 64, itq = (c.num_attention_heads * c.head_dim / 8 + 63) / 64;
    const int iti = (c.intermediate_size / 8 + 63) / 64;
    const bool shape = (c.head_dim == 128 && ith == 6 && itq == 6 && iti == 16) ||
                       (c.head_dim == 64 && ith == 2 && itq == 2 && iti == 6);
    return shape && rows >= 1 && rows <= 2 && nwg % (c.num_key_value_heads * rows) == 0 &&
           c.num_attention_heads / c.num_key_value_heads <= 4;
}

hipError_t launch_step(hipStream_t s, const StepArgs& a, int nwg) {
    const int kmax = std::max(std::max(a.hidden, a.intermediate), a.heads * a.attn.dim);
    const int G = a.heads / a.kv_heads;
    const size_t lds = std::max((size_t)a.rows * kmax, (size_t)G * a.attn.bpw * kBlockKeys) * sizeof(float);
    if (lds > 128 * 1024) return hipErrorInvalidValue;
    const int ith = (a.hidden / 8 + 63) / 64;
    if (a.attn.dim == 128 && ith == 6) {
        if (a.rows == 1) return launch_step_t<1, 128, 6, 6, 16>(s, a, nwg, lds);
        return launch_step_t<2, 128, 6, 6, 16>(s, a, nwg, lds);
    }
    if (a.attn.dim == 64 && ith == 2) {
        if (a.rows == 1) return launch_step_t<1, 64, 2, 2, 6>(s, a, nwg, lds);
        return launch_step_t<2, 64, 2, 2, 6>(s, a, nwg, lds);
    }
    return hipErrorInvalidValue;
}

}  // namespace y2
