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

#include "kernels.h"
#include "y2_math.h"

namespace y2 {

constexpr int kGemvThreads = 512;
constexpr int kGemvWaves = kGemvThreads / 64;

__device__ __forceinline__ void unpack8w(const uint4 w, float* f) {
    f[0] = bf16_lo(w.x); f[1] = bf16_hi(w.x);
    f[2] = bf16_lo(w.y); f[3] = bf16_hi(w.y);
    f[4] = bf16_lo(w.z); f[5] = bf16_hi(w.z);
    f[6] = bf16_lo(w.w); f[7] = bf16_hi(w.w);
}

__device__ __forceinline__ float wave_sum_xor(float v) {
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) v = v + __shfl_xor(v, s, 64);
    return v;
}

// RMSNorm scale of the n values xs[0..n) (LDS), all threads of the block
// participating.  The reference sums the squares in one sequential f32 chain
// (src/tensor.rs:1144).  The block computes the exact sum E and the bound
// B = 2^-24 * 1.001 * sum_i t_i (n - i) on that chain's rounding error in f64;
// the scale rb(1/sqrt(S/n + eps)) is monotone in S, so if both ends of
// [E - B, E + B] map to the same BF16 scale it is the chain's scale.
// Otherwise thread 0 runs the chain.
template <int NT>
__device__ float norm_scale_block(const float* xs, int n, float eps, int* fallbacks) {
    __shared__ double red_e[NT / 64], red_w[NT / 64];
    __shared__ float s_scale;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    double e_sum = 0.0, w_sum = 0.0;
    for (int i = tid; i < n; i += NT) {
        const float t = xs[i] * xs[i];
        e_sum += (double)t;
        w_sum += (double)t * (double)(n - i);
    }
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) {
        e_sum += __shfl_xor(e_sum, s, 64);
        w_sum += __shfl_xor(w_sum, s, 64);
    }
    if (lane == 0) {
        red_e[wave] = e_sum;
        red_w[wave] = w_sum;
    }
    __syncthreads();
    if (tid == 0) {
        double e = 0.0, w = 0.0;
        for (int i = 0; i < NT / 64; ++i) {
            e += red_e[i];
            w += red_w[i];
        }
        float scale = 0.0f;
        bool done = false;
        if (e < 1e300 && w < 1e300) {
            const double bound = w * 0x1.0p-24 * 1.001 + e * 4e-12;
            const double lo = e - bound, hi = e + bound;
            float lo_f = (float)lo, hi_f = (float)hi;
            if ((double)lo_f > lo) lo_f = lo_f > 0.0f ? u2f(f2u(lo_f) - 1u) : 0.0f;
            if (lo_f < 0.0f) lo_f = 0.0f;
            if ((double)hi_f < hi) hi_f = u2f(f2u(hi_f) + 1u);
            const float s_a = norm_scale_from_sum(lo_f, n, eps);
            const float s_b = norm_scale_from_sum(hi_f, n, eps);
            if (hi_f <= 3.0e38f && s_a == s_b) {
                scale = s_a;
                done = true;
            }
        }
        if (!done) {
            float sum = -0.0f;
            for (int i = 0; i < n; ++i) sum = sum + xs[i] * xs[i];
            scale = norm_scale_from_sum(sum, n, eps);
            if (fallbacks) atomicAdd(fallbacks, 1);
        }
        s_scale = scale;
    }
    __syncthreads();
    return s_scale;
}

template <int IT>
__device__ __forceinline__ void load_row(const uint16_t* __restrict__ w, int row, int k, int nchunk,
                                         int lane, uint4* buf) {
    const uint4* wr = reinterpret_cast<const uint4*>(w + (size_t)row * k);
#pragma unroll
    for (int it = 0; it < IT; ++it) {
        const int c = lane + 64 * it;
        buf[it] = c < nchunk ? wr[c] : make_uint4(0, 0, 0, 0);
    }
}

template <int B, int EPI, int IT>
__device__ __forceinline__ void compute_row(const GemvArgs& a, const float* xs, int row, int nchunk,
                                            int lane, const uint4* wv, const uint4* wv2) {
    const int k = a.k;
    float acc[B], acc2[B];
#pragma unroll
    for (int b = 0; b < B; ++b) acc[b] = acc2[b] = 0.0f;
#pragma unroll
    for (int it = 0; it < IT; ++it) {
        const int c = lane + 64 * it;
        if (c < nchunk) {
            float wf[8], wf2[8];
            unpack8w(wv[it], wf);
            if constexpr (EPI == EPI_SWIGLU) unpack8w(wv2[it], wf2);
#pragma unroll
            for (int b = 0; b < B; ++b) {
                const float4* xp = reinterpret_cast<const float4*>(xs + b * k + 8 * c);
                const float4 x0 = xp[0], x1 = xp[1];
                const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
                float s = acc[b];
#pragma unroll
                for (int e = 0; e < 8; ++e) s = __builtin_fmaf(wf[e], xv[e], s);
                acc[b] = s;
                if constexpr (EPI == EPI_SWIGLU) {
                    float s2 = acc2[b];
#pragma unroll
                    for (int e = 0; e < 8; ++e) s2 = __builtin_fmaf(wf2[e], xv[e], s2);
                    acc2[b] = s2;
                }
            }
        }
    }
#pragma unroll
    for (int b = 0; b < B; ++b) {
        acc[b] = wave_sum_xor(acc[b]);
        if constexpr (EPI == EPI_SWIGLU) acc2[b] = wave_sum_xor(acc2[b]);
    }
    if (lane == 0) {
#pragma unroll
        for (int b = 0; b < B; ++b) {
            float* yp = a.y + (size_t)b * a.y_stride + row;
            if constexpr (EPI == EPI_RAW) {
                *yp = acc[b];
            } else if constexpr (EPI == EPI_STORE) {
                *yp = rb(acc[b]);
            } else if constexpr (EPI == EPI_RESID) {
                *yp = rb(*yp + rb(acc[b]));
            } else {
                const float g = silu_rb(rb(acc[b]));
                *yp = rb(g * rb(acc2[b]));
            }
        }
    }
}

template <int B, int EPI, int IT, bool NORM>
__global__ __launch_bounds__(kGemvThreads) void gemv_kernel(const GemvArgs a) {
    extern __shared__ float xs[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int k = a.k, nchunk = k >> 3;
    const int per = (a.n + gridDim.x - 1) / gridDim.x;
    const int r0 = blockIdx.x * per, r1 = min(a.n, r0 + per);
    constexpr int IT2 = EPI == EPI_SWIGLU ? IT : 1;
    uint4 bufA[IT], bufA2[IT2], bufB[IT], bufB2[IT2];
    int row = r0 + wave;
    if (row < r1) {
        load_row<IT>(a.w, row, k, nchunk, lane, bufA);
        if constexpr (EPI == EPI_SWIGLU) load_row<IT>(a.w2, row, k, nchunk, lane, bufA2);
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
            load_row<IT>(a.w, next, k, nchunk, lane, bufB);
            if constexpr (EPI == EPI_SWIGLU) load_row<IT>(a.w2, next, k, nchunk, lane, bufB2);
        }
        compute_row<B, EPI, IT>(a, xs, row, nchunk, lane, bufA, bufA2);
        row = next;
        if (row >= r1) break;
        next = row + kGemvWaves;
        if (next < r1) {
            load_row<IT>(a.w, next, k, nchunk, lane, bufA);
            if constexpr (EPI == EPI_SWIGLU) load_row<IT>(a.w2, next, k, nchunk, lane, bufA2);
        }
        compute_row<B, EPI, IT>(a, xs, row, nchunk, lane, bufB, bufB2);
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
