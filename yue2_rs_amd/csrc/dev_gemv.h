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

// The scale rb(1/sqrt(S/n + eps)) at one end (hi: the upper) of the interval
// [E - B, E + B] that holds the sequential f32 chain's sum of squares, given
// the exact sum E and the weighted sum W of norm_scales_block (B = 2^-24 *
// 1.001 * W + E * 4e-12, the last term for the f64 rounding of E and W).
// Returns whether the interval is finite; *scale gets that end's scale.
__device__ __forceinline__ bool norm_scale_end(double e, double w, int n, float eps, bool hi_end, float* scale) {
    const double bound = w * 0x1.0p-24 * 1.001 + e * 4e-12;
    const double lo = e - bound, hi = e + bound;
    float lo_f = (float)lo, hi_f = (float)hi;
    if ((double)lo_f > lo) lo_f = lo_f > 0.0f ? u2f(f2u(lo_f) - 1u) : 0.0f;
    if (lo_f < 0.0f) lo_f = 0.0f;
    if ((double)hi_f < hi) hi_f = u2f(f2u(hi_f) + 1u);
    *scale = norm_scale_from_sum(hi_end ? hi_f : lo_f, n, eps);
    return e < 1e300 && w < 1e300 && hi_f <= 3.0e38f;
}

// The sequential chain itself: rb(1/sqrt(sum/n + eps)) with sum = x[0]^2 +
// x[1]^2 + ... from -0 in f32 (src/tensor.rs:1144, 1160); LDS reads batched
// ahead of the adds.
__device__ __forceinline__ float norm_scale_chain(const float* x, int n, float eps) {
    float sum = -0.0f;
    int i = 0;
    for (; i + 16 <= n; i += 16) {
        float t[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) t[j] = x[i + j];
#pragma unroll
        for (int j = 0; j < 16; ++j) sum = sum + t[j] * t[j];
    }
    for (; i < n; ++i) sum = sum + x[i] * x[i];
    return norm_scale_from_sum(sum, n, eps);
}

// RMSNorm scale of n values v[0..n) (LDS) computed by one whole wave, the
// same decision as norm_scales_block (lanes 0 and 1 evaluate the two ends);
// lane 0 runs the chain when the interval does not decide it.  Uniform over
// the wave.
__device__ __forceinline__ float norm_scale_wave(const float* v, int n, float eps) {
    const int lane = threadIdx.x & 63;
    double e = 0.0, w = 0.0;
    for (int i = lane; i < n; i += 64) {
        const float t = v[i] * v[i];
        e += (double)t;
        w += (double)t * (double)(n - i);
    }
    e = xor_sum<32>(e);
    w = xor_sum<32>(w);
    float sv;
    const bool finite = norm_scale_end(e, w, n, eps, lane & 1, &sv);
    const float other = xor_lane<1>(sv);  // the other end's scale (every lane takes part)
    const bool decided = finite && sv == other;
    if (__builtin_amdgcn_readfirstlane(decided ? 1 : 0))
        return u2f((uint32_t)__builtin_amdgcn_readfirstlane((int)f2u(sv)));
    float s = 0.0f;
    if (lane == 0) s = norm_scale_chain(v, n, eps);
    return u2f((uint32_t)__builtin_amdgcn_readfirstlane((int)f2u(s)));
}

// One value's share of the sums of norm_scales_block: t = x * x (f32, as in
// the chain), E += t and W += t * (n - i) in f64, for element i of n.
__device__ __forceinline__ void norm_partial_add(double& e, double& w, float x, int i, int n) {
    const float t = x * x;
    e += (double)t;
    w += (double)t * (double)(n - i);
}

// This thread's shares of E and W for B rows: elements tid, tid + NT, ...
template <int NT, int B>
__device__ __forceinline__ void norm_partials(const float* xs, int n, double* e_sum, double* w_sum) {
#pragma unroll
    for (int b = 0; b < B; ++b) e_sum[b] = w_sum[b] = 0.0;
    for (int i = threadIdx.x; i < n; i += NT) {
#pragma unroll
        for (int b = 0; b < B; ++b) norm_partial_add(e_sum[b], w_sum[b], xs[b * n + i], i, n);
    }
}

// norm_scales_block from each thread's shares of E and W (any split of the
// elements over the threads, in any order: the bound's f64 term covers it);
// e_sum and w_sum are consumed.
template <int NT, int B>
__device__ __forceinline__ void norm_scales_from(double* e_sum, double* w_sum, const float* xs, int n, float eps,
                                                 int* fallbacks, float* scale) {
    static_assert(B <= NT / 64 && 2 * B <= 64, "one wave per fallback chain");
    constexpr int NW = NT / 64;
    __shared__ double red_e[B][NW], red_w[B][NW];
    __shared__ float s_scale[B];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int b = 0; b < B; ++b) {
        e_sum[b] = xor_sum<32>(e_sum[b]);
        w_sum[b] = xor_sum<32>(w_sum[b]);
    }
    if (lane == 0) {
#pragma unroll
        for (int b = 0; b < B; ++b) {
            red_e[b][wave] = e_sum[b];
            red_w[b][wave] = w_sum[b];
        }
    }
    __syncthreads();
    const int q = lane % (2 * B), row = q >> 1;
    double e = 0.0, w = 0.0;
#pragma unroll
    for (int i = 0; i < NW; ++i) {
        e += red_e[row][i];
        w += red_w[row][i];
    }
    float sv;
    const bool finite = norm_scale_end(e, w, n, eps, q & 1, &sv);
    const float other = xor_lane<1>(sv);  // the other end's scale (every lane takes part)
    const bool decided = finite && sv == other;
    unsigned okmask = 0;  // bit b: row b's scale decided
#pragma unroll
    for (int b = 0; b < B; ++b) {
        scale[b] = u2f((uint32_t)__builtin_amdgcn_readlane((int)f2u(sv), 2 * b));
        okmask |= (unsigned)__builtin_amdgcn_readlane(decided ? 1 : 0, 2 * b) << b;
    }
    if (okmask == (1u << B) - 1u) return;
    if (wave < B && lane == 0 && !((okmask >> wave) & 1u)) {
        s_scale[wave] = norm_scale_chain(xs + wave * n, n, eps);  // row `wave`
        if (fallbacks) add_dev(fallbacks, 1);
    }
    __syncthreads();
#pragma unroll
    for (int b = 0; b < B; ++b)
        if (!((okmask >> b) & 1u)) scale[b] = s_scale[b];
}

// RMSNorm scales of B rows xs[b * n .. b * n + n) (LDS); all NT threads of
// the block take part, entering together right after a block barrier, and
// each gets scale[b] for every row.
// The reference sums the squares in one sequential f32 chain
// (src/tensor.rs:1144).  The block computes the exact sum E and the bound
// B = 2^-24 * 1.001 * sum_i t_i (n - i) on that chain's rounding error in f64
// (each of the n-1 additions errs by at most 2^-24 of its partial sum); the
// scale rb(1/sqrt(S/n + eps)) is monotone in S, so when both ends of
// [E - B, E + B] give the same BF16 scale it is the chain's scale.  Lane
// 2b + e of every wave evaluates end e of row b (all ends at once), and the
// outcome is read back from those lanes, so it is uniform over the block.
// A row that is not decided that way gets the chain itself, run by lane 0 of
// wave b (the rows' chains on different SIMDs at once).
template <int NT, int B>
__device__ __forceinline__ void norm_scales_block(const float* xs, int n, float eps, int* fallbacks, float* scale) {
    double e_sum[B], w_sum[B];
    norm_partials<NT, B>(xs, n, e_sum, w_sum);
    norm_scales_from<NT, B>(e_sum, w_sum, xs, n, eps, fallbacks, scale);
}

}  // namespace y2
