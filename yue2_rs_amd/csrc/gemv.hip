// gemv.hip -- BF16 GEMV with FP32 accumulation in the DOT order
// (Linear::apply_range + finish, src/tensor.rs:946-1118), optionally fused
// with the RMSNorm that produces its input (Norm::apply, :1140-1157).
//
// Layout and schedule (gfx950):
//  * one 512-thread workgroup per CU; workgroup g owns a contiguous range of
//    weight rows, and its 8 waves take every 8th row of that range;
//  * a wave owns one row at a time: lane l streams chunks l, l+64, ... of the
//    row with 128-bit loads (8 BF16 values) and keeps one f32 fma chain, then
//    the 64 lanes combine by an xor butterfly -- exactly the DOT order, so any
//    batch row equals the batch-1 result;
//  * the first row's weights are requested before the input vector is staged,
//    and row r+8 is requested while row r is computed (double buffering), so
//    each CU keeps ~100 KB of weight reads in flight;
//  * the input rows are staged once per workgroup in LDS (f32).  With a norm
//    prologue the workgroup computes the RMSNorm scale itself (guarded, see
//    norm_scale_block) and stages rb(rb(x * s) * gamma).
#include <algorithm>

#include "dev_gemv.h"
#include "kernels.h"
#include "y2_math.h"

namespace y2 {

constexpr int kGemvThreads = 512;
constexpr int kGemvWaves = kGemvThreads / 64;

template <int B, int EPI, int IT>
__device__ __forceinline__ void compute_row(const GemvArgs& a, const float* xs, int row, int lane,
                                            const uint4* wv, const uint4* wv2) {
    float acc[B], acc2[B];
    dot_rows<B, IT, EPI == EPI_SWIGLU>(xs, a.k, lane, wv, wv2, acc, acc2);
    if (lane == 0) {
#pragma unroll
        for (int b = 0; b < B; ++b) gemv_store<EPI>(a.y + (size_t)b * a.y_stride + row, acc[b], acc2[b]);
    }
}

template <int B, int EPI, int IT, bool NORM>
__global__ __launch_bounds__(kGemvThreads) void gemv_kernel(const GemvArgs a) {
    extern __shared__ float xs[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int k = a.k;
    const int per = (a.n + gridDim.x - 1) / gridDim.x;
    const int r0 = blockIdx.x * per, r1 = min(a.n, r0 + per);
    constexpr int IT2 = EPI == EPI_SWIGLU ? IT : 1;
    uint4 bufA[IT], bufA2[IT2], bufB[IT], bufB2[IT2];
    int row = r0 + wave;
    if (row < r1) {
        load_row<IT>(a.w, row, k, lane, bufA);
        if constexpr (EPI == EPI_SWIGLU) load_row<IT>(a.w2, row, k, lane, bufA2);
    }
    for (int b = 0; b < B; ++b)
        for (int i = tid; i < k; i += kGemvThreads) xs[b * k + i] = a.x[(size_t)b * a.x_stride + i];
    __syncthreads();
    if constexpr (NORM) {
        for (int b = 0; b < B; ++b) {
            float* xb = xs + b * k;
            const float s = norm_scale_block<kGemvThreads>(
                xb, k, a.eps, (blockIdx.x == 0 && a.st) ? &a.st->norm_fallbacks : nullptr);
            for (int i = tid; i < k; i += kGemvThreads) xb[i] = rb(rb(xb[i] * s) * a.gamma[i]);
        }
        __syncthreads();
    }
    while (row < r1) {
        int next = row + kGemvWaves;
        if (next < r1) {
            load_row<IT>(a.w, next, k, lane, bufB);
            if constexpr (EPI == EPI_SWIGLU) load_row<IT>(a.w2, next, k, lane, bufB2);
        }
        compute_row<B, EPI, IT>(a, xs, row, lane, bufA, bufA2);
        row = next;
        if (row >= r1) break;
        next = row + kGemvWaves;
        if (next < r1) {
            load_row<IT>(a.w, next, k, lane, bufA);
            if constexpr (EPI == EPI_SWIGLU) load_row<IT>(a.w2, next, k, lane, bufA2);
        }
        compute_row<B, EPI, IT>(a, xs, row, lane, bufB, bufB2);
        row = next;
    }
}

static int g_cus = 0;

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
    const int blocks = std::max(1, std::min(cu_count(), (a.n + kGemvWaves - 1) / kGemvWaves));
    const size_t lds = (size_t)B * a.k * sizeof(float);
#define Y2_GEMV_CASE(N)                                                       \
    if (iters <= N) {                                                         \
        gemv_kernel<B, EPI, N, NORM><<<blocks, kGemvThreads, lds, s>>>(a);    \
        return hipGetLastError();                                             \
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
    // LDS holds rows * k f32 inputs (64 KiB per workgroup).
    if ((size_t)a.rows * a.k * sizeof(float) > 64 * 1024) return hipErrorInvalidValue;
    const bool norm = a.gamma != nullptr;
    if (a.rows == 1) return norm ? gemv_epi<1, true>(s, epi, a) : gemv_epi<1, false>(s, epi, a);
    return norm ? gemv_epi<2, true>(s, epi, a) : gemv_epi<2, false>(s, epi, a);
}

}  // namespace y2
