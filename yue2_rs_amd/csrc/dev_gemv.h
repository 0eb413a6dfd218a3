// dev_gemv.h -- device building blocks of the BF16 GEMV in the DOT order and
// of the RMSNorm that feeds it, shared by the standalone kernels and the
// persistent token-step kernel.
//
// DOT order (Linear::apply_range, src/tensor.rs:946-1118, Accelerate
// cblas_sgemv substitute): chunk c = 8 consecutive elements, chunk c -> lane
// c mod 64, each lane one fma chain over its chunks in ascending order from
// +0, then an xor butterfly over the 64 lanes with offsets 32..1.
#pragma once
#include <hip/hip_runtime.h>

#include "dev_mem.h"
#include "kernels.h"
#include "y2_math.h"

namespace y2 {

__device__ __forceinline__ void unpack_bf16x8(const uint4 w, float* f) {
    f[0] = bf16_lo(w.x); f[1] = bf16_hi(w.x);
    f[2] = bf16_lo(w.y); f[3] = bf16_hi(w.y);
    f[4] = bf16_lo(w.z); f[5] = bf16_hi(w.z);
    f[6] = bf16_lo(w.w); f[7] = bf16_hi(w.w);
}

// v summed over the wave by the xor butterfly 32, 16, ..., 1 (ALU lane
// exchanges, dev_mem.h).
__device__ __forceinline__ float wave_sum_xor(float v) { return xor_sum<32>(v); }

// Request the IT chunks that `lane` owns in weight row `row` (k BF16 per row).
// Loads are unconditional so the compiler can keep them in flight across the
// arithmetic; lanes past the row end (k not a multiple of 512) re-read chunk
// 0, and dot_rows zeroes their contribution.
template <int IT>
__device__ __forceinline__ void load_row(const uint16_t* __restrict__ w, int row, int k, int lane,
                                         uint4* buf) {
    const uint4* wr = reinterpret_cast<const uint4*>(w + (size_t)row * k);
    const int nchunk = k >> 3;
#pragma unroll
    for (int it = 0; it < IT; ++it) {
        const int c = lane + 64 * it;
        buf[it] = ldg4(wr + (c < nchunk ? c : 0));
    }
}

// acc[b] (and acc2[b] when PAIR) = DOT(row, xs[b]) over the staged inputs
// xs[b * k + i] (LDS).  A skipped chunk contributes fma(0, 0, acc) = acc + 0,
// which leaves the chain unchanged (its value is never -0).
template <int B, int IT, bool PAIR>
__device__ __forceinline__ void dot_rows(const float* xs, int k, int lane, const uint4* wv,
                                         const uint4* wv2, float* acc, float* acc2) {
    const int nchunk = k >> 3;
#pragma unroll
    for (int b = 0; b < B; ++b) acc[b] = acc2[b] = 0.0f;
#pragma unroll
    for (int it = 0; it < IT; ++it) {
        const int c = lane + 64 * it;
        const bool ok = c < nchunk;
        const int cc = ok ? c : 0;
        float wf[8], wf2[8];
        unpack_bf16x8(wv[it], wf);
        if constexpr (PAIR) unpack_bf16x8(wv2[it], wf2);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            wf[e] = ok ? wf[e] : 0.0f;
            if constexpr (PAIR) wf2[e] = ok ? wf2[e] : 0.0f;
        }
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const float4* xp = reinterpret_cast<const float4*>(xs + b * k + 8 * cc);
            const float4 x0 = xp[0], x1 = xp[1];
            float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) xv[e] = ok ? xv[e] : 0.0f;
            float s = acc[b];
#pragma unroll
            for (int e = 0; e < 8; ++e) s = __builtin_fmaf(wf[e], xv[e], s);
            acc[b] = s;
            if constexpr (PAIR) {
                float s2 = acc2[b];
#pragma unroll
                for (int e = 0; e < 8; ++e) s2 = __builtin_fmaf(wf2[e], xv[e], s2);
                acc2[b] = s2;
            }
        }
        // Keep each chunk's LDS reads next to its FMAs: hoisting the reads
        // of every chunk ahead of the arithmetic costs more registers than
        // the persistent kernel has.
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int b = 0; b < B; ++b) {
        acc[b] = wave_sum_xor(acc[b]);
        if constexpr (PAIR) acc2[b] = wave_sum_xor(acc2[b]);
    }
}

// Output of one GEMV row for batch row b:
//   EPI_STORE   y = rb(dot)
//   EPI_RESID   y = rb(y + rb(dot))               (Tensor::add, src/tensor.rs:632-640)
//   EPI_SWIGLU  y = rb(rb(silu(rb(g))) * rb(u))   (Mlp::apply, src/model.rs:206-214)
//   EPI_RAW     y = dot                           (yue2_metal_vector, src/metal.m:545-603)
template <int EPI>
__device__ __forceinline__ void gemv_store(float* yp, float acc, float acc2) {
    if constexpr (EPI == EPI_RAW) {
        *yp = acc;
    } else if constexpr (EPI == EPI_STORE) {
        *yp = rb(acc);
    } else if constexpr (EPI == EPI_RESID) {
        *yp = rb(*yp + rb(acc));
    } else {
        *yp = rb(silu_rb(rb(acc)) * rb(acc2));
    }
}

// RMSNorm scale of xs[0..n) (LDS), all NT threads of the block participating.
// The reference sums the squares in one sequential f32 chain
// (src/tensor.rs:1144).  The block computes the exact sum E and the bound
// B = 2^-24 * 1.001 * sum_i t_i (n - i) on that chain's rounding error in f64
// (each of the n-1 additions errs by at most 2^-24 of its partial sum); the
// scale rb(1/sqrt(S/n + eps)) is monotone in S, so when both ends of
// [E - B, E + B] give the same BF16 scale it is the chain's scale.  Every
// thread evaluates that test on the same per-wave partials (so the outcome is
// uniform); otherwise thread 0 runs the chain.
template <int NT>
__device__ __forceinline__ float norm_scale_block(const float* xs, int n, float eps, int* fallbacks) {
    __shared__ double red_e[NT / 64], red_w[NT / 64];
    __shared__ float s_scale;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    __syncthreads();  // a previous call's readers of red_e / red_w / s_scale are done
    double e_sum = 0.0, w_sum = 0.0;
    for (int i = tid; i < n; i += NT) {
        const float t = xs[i] * xs[i];
        e_sum += (double)t;
        w_sum += (double)t * (double)(n - i);
    }
    e_sum = xor_sum<32>(e_sum);
    w_sum = xor_sum<32>(w_sum);
    if (lane == 0) {
        red_e[wave] = e_sum;
        red_w[wave] = w_sum;
    }
    __syncthreads();
    double e = 0.0, w = 0.0;
#pragma unroll
    for (int i = 0; i < NT / 64; ++i) {
        e += red_e[i];
        w += red_w[i];
    }
    if (e < 1e300 && w < 1e300) {
        const double bound = w * 0x1.0p-24 * 1.001 + e * 4e-12;
        const double lo = e - bound, hi = e + bound;
        float lo_f = (float)lo, hi_f = (float)hi;
        if ((double)lo_f > lo) lo_f = lo_f > 0.0f ? u2f(f2u(lo_f) - 1u) : 0.0f;
        if (lo_f < 0.0f) lo_f = 0.0f;
        if ((double)hi_f < hi) hi_f = u2f(f2u(hi_f) + 1u);
        float s_a = 0.0f, s_b = 0.0f;
#pragma unroll 1
        for (int t = 0; t < 2; ++t) {  // one copy of the scale arithmetic
            const float v = norm_scale_from_sum(t ? hi_f : lo_f, n, eps);
            if (t) s_b = v;
            else s_a = v;
        }
        if (hi_f <= 3.0e38f && s_a == s_b) return s_a;
    }
    if (tid == 0) {
        // the sequential chain itself; LDS reads batched ahead of the adds
        float sum = -0.0f;
        int i = 0;
        for (; i + 16 <= n; i += 16) {
            float t[16];
#pragma unroll
            for (int j = 0; j < 16; ++j) t[j] = xs[i + j];
#pragma unroll
            for (int j = 0; j < 16; ++j) sum = sum + t[j] * t[j];
        }
        for (; i < n; ++i) sum = sum + xs[i] * xs[i];
        s_scale = norm_scale_from_sum(sum, n, eps);
        if (fallbacks) add_dev(fallbacks, 1);
    }
    __syncthreads();
    return s_scale;
}

}  // namespace y2
