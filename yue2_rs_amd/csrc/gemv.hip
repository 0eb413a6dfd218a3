// gemv.hip -- BF16 GEMV with FP32 accumulation in the DOT order
// (Linear::apply_range + finish, src/tensor.rs:946-1118), optionally fused
// with the RMSNorm that produces its input (Norm::apply, :1140-1157).
//
// Layout and schedule (gfx950):
//  * one 512-thread workgroup per CU; workgroup g owns the contiguous rows
//    [g n / G, (g + 1) n / G) and its 8 waves take every 8th row of them;
//  * a wave walks its rows as items through the register ring of dev_ring.h
//    (R-1 items of 16-byte loads in flight, ~100 KB per CU): lane l streams
//    chunks l, l+64, ... of a row and keeps one f32 fma chain, then the 64
//    lanes combine by an xor butterfly -- exactly the DOT order, so any batch
//    row equals the batch-1 result;
//  * the ring's first items are requested before the input vector is staged;
//  * the input rows are staged once per workgroup in LDS (f32), and for a
//    residual epilogue the workgroup's own output rows as well.  With a norm
//    prologue the workgroup computes the RMSNorm scale itself (guarded, see
//    norm_scales_block) and stages rb(rb(x * s) * gamma).
#include <algorithm>

#include "dev_gemv.h"
#include "dev_ring.h"
#include "kernels.h"
#include "y2_math.h"

namespace y2 {

constexpr int kGemvThreads = kRingThreads;

// IT chunks of 8 per lane cover k (k <= 512 IT); chunks past k are masked.
template <int B, int EPI, int IT, bool NORM>
__global__ __launch_bounds__(kGemvThreads) void gemv_kernel(const GemvArgs a) {
    // 16-byte aligned whatever the static LDS before it: the staged rows are
    // read as float4 (a misaligned 16-byte LDS read is split and slow)
    extern __shared__ __align__(16) float xs[];  // [B][k] inputs, then [B][kResRows] residual rows
    constexpr bool PAIR = EPI == EPI_SWIGLU;
    const int tid = threadIdx.x, k = a.k, n = a.n;
    const int r0 = part_lo(n, blockIdx.x, gridDim.x), r1 = part_lo(n, blockIdx.x + 1, gridDim.x);
    // The inputs, the residual rows and the gammas (all written before this
    // launch) are requested before the ring's first items: loads complete in
    // order, so staging them then waits for them alone, and the norm runs
    // while the ring's loads are in flight.  Element tid + 512 j of each row
    // (k <= 512 IT); the loads are unconditional (past the end they re-read
    // the last element, never staged), so that no branch join makes the
    // compiler wait for everything issued before them.
    float xv[B][IT], gv[NORM ? IT : 1], rv = 0.0f;
#pragma unroll
    for (int b = 0; b < B; ++b)
#pragma unroll
        for (int j = 0; j < IT; ++j) xv[b][j] = a.x[(size_t)b * a.x_stride + min(tid + j * kGemvThreads, k - 1)];
    if constexpr (NORM)
#pragma unroll
        for (int j = 0; j < IT; ++j) gv[j] = a.gamma[min(tid + j * kGemvThreads, k - 1)];
    const int span = r1 - r0;
    if constexpr (EPI == EPI_RESID) {
        const int t = min(tid, max(B * span - 1, 0));
        rv = a.y[(size_t)(t / max(span, 1)) * a.y_stride + r0 + t % max(span, 1)];
    }
    uint4 ring[Ring<IT, PAIR>::SIZE];
    prefetch_ring<IT, PAIR, true>(a.w, a.w2, k, r0, r1, n, ring);
#pragma unroll
    for (int b = 0; b < B; ++b)
#pragma unroll
        for (int j = 0; j < IT; ++j)
            if (tid + j * kGemvThreads < k) xs[b * k + tid + j * kGemvThreads] = xv[b][j];
    float* res = xs + B * k;
    if constexpr (EPI == EPI_RESID)
        if (tid < B * span) res[tid] = rv;
    __syncthreads();
    if constexpr (NORM) {
        float s[B];
        norm_scales_block<kGemvThreads, B>(xs, k, a.eps, (blockIdx.x == 0 && a.st) ? &a.st->norm_fallbacks : nullptr,
                                           s);
#pragma unroll
        for (int b = 0; b < B; ++b)
#pragma unroll
            for (int j = 0; j < IT; ++j) {
                const int i = tid + j * kGemvThreads;
                if (i < k) xs[b * k + i] = rb(rb(xs[b * k + i] * s[b]) * gv[j]);
            }
        __syncthreads();
    }
    gemv_ring<B, EPI, IT, true>(a.w, a.w2, xs, k, a.y, nullptr, 0, a.y_stride, r0, r1, n, ring, res);
}

static int g_cus = 0;

constexpr size_t kGemvLdsMax = 128 * 1024;

static int cu_count() {
    if (g_cus <= 0) {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, 0) != hipSuccess || v <= 0)
            v = 256;
        g_cus = v;
    }
    return g_cus;
}

template <int B, int EPI, bool NORM>
static hipError_t gemv_dispatch(hipStream_t s, const GemvArgs& a) {
    const int iters = (a.k / 8 + 63) / 64;
    const int blocks = std::max(1, std::min(cu_count(), a.n));
    // a residual epilogue stages the workgroup's output rows (at most kResRows)
    if (EPI == EPI_RESID && (a.n + blocks - 1) / blocks > kResRows) return hipErrorInvalidValue;
    const size_t lds = (size_t)B * (a.k + kResRows) * sizeof(float);
#define Y2_GEMV_CASE(N)                                                                               \
    if (iters <= N) {                                                                                 \
        static const hipError_t attr = hipFuncSetAttribute(                                           \
            reinterpret_cast<const void*>(&gemv_kernel<B, EPI, N, NORM>),                             \
            hipFuncAttributeMaxDynamicSharedMemorySize, (int)kGemvLdsMax);                            \
        if (attr != hipSuccess) return attr;                                                          \
        gemv_kernel<B, EPI, N, NORM><<<blocks, kGemvThreads, lds, s>>>(a);                            \
        return hipGetLastError();                                                                     \
    }
    Y2_GEMV_CASE(1)
    Y2_GEMV_CASE(2)
    Y2_GEMV_CASE(4)
    Y2_GEMV_CASE(6)
    Y2_GEMV_CASE(8)
    Y2_GEMV_CASE(12)
    Y2_GEMV_CASE(16)
    Y2_GEMV_CASE(32)
#undef Y2_GEMV_CASE
    return hipErrorInvalidValue;
}

template <int B, bool NORM>
static hipError_t gemv_epi(hipStream_t s, int epi, const GemvArgs& a) {
    switch (epi) {
        case EPI_STORE: return gemv_dispatch<B, EPI_STORE, NORM>(s, a);
        case EPI_RESID: return gemv_dispatch<B, EPI_RESID, NORM>(s, a);
        case EPI_SWIGLU: return gemv_dispatch<B, EPI_SWIGLU, NORM>(s, a);
        case EPI_RAW: return gemv_dispatch<B, EPI_RAW, NORM>(s, a);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemv(hipStream_t s, int epi, const GemvArgs& a) {
    if (a.k % 8 != 0 || a.k <= 0 || a.k > 32 * 512 || a.n <= 0 || a.rows < 1 || a.rows > kMaxRows)
        return hipErrorInvalidValue;
    // LDS holds rows * k f32 inputs and the residual rows (one workgroup per CU)
    if ((size_t)a.rows * (a.k + kResRows) * sizeof(float) > kGemvLdsMax) return hipErrorInvalidValue;
    const bool norm = a.gamma != nullptr;
    if (a.rows == 1) return norm ? gemv_epi<1, true>(s, epi, a) : gemv_epi<1, false>(s, epi, a);
    return norm ? gemv_epi<2, true>(s, epi, a) : gemv_epi<2, false>(s, epi, a);
}

}  // namespace y2
