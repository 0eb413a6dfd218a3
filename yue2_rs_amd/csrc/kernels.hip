// kernels.hip -- gfx950 kernels of the YuE2 AR decode step.
//
// Each kernel computes exactly the arithmetic of the reference CPU token step
// (src/model.rs:523-591, src/tensor.rs:589-1173) with the reduction orders of
// the order spec:
//   DOT          chunk c = 8 consecutive elements, chunk c -> lane c mod 64,
//                per-lane fma chain in ascending order from +0, then an xor
//                butterfly over the 64 lanes with offsets 32..1.
//   SOFTMAX SUM  64-key blocks reduced by the 64-lane xor butterfly, block
//                sums added left to right.
//   PV           per 64-key block, 512/dim key streams (key j -> stream j mod
//                512/dim), fma chains, xor butterfly over the streams, blocks
//                added left to right.
// Rows of a batch never interact, so a CFG batch-2 row equals a batch-1 row.
#include <algorithm>

#include "dev_gemv.h"
#include "dev_mem.h"
#include "kernels.h"
#include "y2_math.h"

namespace y2 {

enum DeviceError { DEV_OK = 0, DEV_ERR_TOKEN = 2, DEV_ERR_CONTEXT = 1 };

__device__ __forceinline__ void set_error(StepState* st, int code) {
    atomicCAS(&st->error, 0, code);
}

__device__ __forceinline__ void unpack8(const uint4 w, float* f) {
    f[0] = bf16_lo(w.x); f[1] = bf16_hi(w.x);
    f[2] = bf16_lo(w.y); f[3] = bf16_hi(w.y);
    f[4] = bf16_lo(w.z); f[5] = bf16_hi(w.z);
    f[6] = bf16_lo(w.w); f[7] = bf16_hi(w.w);
}

__device__ __forceinline__ float butterfly64(float v) {
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) v = v + __shfl_xor(v, s, 64);
    return v;
}

__device__ __forceinline__ size_t kv_offset(int layer, int which, int kv_heads, int head,
                                            int capacity, int pos, int dim) {
    return ((((size_t)layer * 2 + which) * kv_heads + head) * capacity + pos) * dim;
}

// ---------------------------------------------------------------------------
// Embedding: x = rb(E[id]) (src/model.rs:452-464).  BF16 values are exact.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void embed_kernel(const uint16_t* __restrict__ embed,
                                                    StepState* st, float* __restrict__ x,
                                                    int hidden, int vocab) {
    const int b = blockIdx.y;
    const int id = st->ids[b];
    if (id < 0 || id >= vocab) {
        if (threadIdx.x == 0 && blockIdx.x == 0) set_error(st, DEV_ERR_TOKEN);
        return;
    }
    const uint16_t* e = embed + (size_t)id * hidden;
    for (int i = blockIdx.x * 256 + threadIdx.x; i < hidden; i += gridDim.x * 256)
        x[(size_t)b * hidden + i] = bf16(e[i]);
}

// ---------------------------------------------------------------------------
// RMSNorm (src/tensor.rs:1140-1157).  The reference sums the squares in one
// sequential f32 chain.  The kernel computes the exact sum E and the bound
// B = 2^-24 * 1.001 * sum_i t_i (n - i) on the sequential chain's rounding
// error in parallel (f64).  The scale rb(1/sqrt(S/n + eps)) is monotone in S,
// so when both ends of [E - B, E + B] give the same BF16 scale, that is the
// scale of the sequential sum.  Otherwise one lane runs the sequential sum.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void rmsnorm_kernel(const float* __restrict__ x, int x_stride,
                                                      const float* __restrict__ gamma,
                                                      float* __restrict__ out, int out_stride,
                                                      int n, float eps, StepState* st) {
    extern __shared__ __align__(16) float xs[];
    __shared__ double red_e[4], red_w[4];
    __shared__ float s_scale;
    const int b = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float* xr = x + (size_t)b * x_stride;
    double e_sum = 0.0, w_sum = 0.0;
    for (int i = tid; i < n; i += 256) {
        const float v = xr[i];
        xs[i] = v;
        const float t = v * v;
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
        const double e = (red_e[0] + red_e[1]) + (red_e[2] + red_e[3]);
        const double w = (red_w[0] + red_w[1]) + (red_w[2] + red_w[3]);
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
            atomicAdd(&st->norm_fallbacks, 1);
        }
        s_scale = scale;
    }
    __syncthreads();
    const float scale = s_scale;
    float* o = out + (size_t)b * out_stride;
    for (int i = tid; i < n; i += 256) o[i] = rb(rb(xs[i] * scale) * gamma[i]);
}

// ---------------------------------------------------------------------------
// Greedy selection: argmax under f32::total_cmp with the lowest index on ties
// (src/sampling.rs:148-156); the id feeds every row's next embedding.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(1024) void argmax_kernel(const float* __restrict__ logits, int n,
                                                      StepState* st, int32_t* token_log, int rows) {
    __shared__ int32_t skey[16];
    __shared__ int32_t sidx[16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int32_t bk = INT32_MIN, bi = INT32_MAX;
    for (int i = tid; i < n; i += 1024) {
        const float v = logits[i];
        if (v == v && v != __builtin_huge_valf() && v != -__builtin_huge_valf()) {
            const int32_t kv = total_key(v);
            if (kv > bk) { bk = kv; bi = i; }
        }
    }
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) {
        const int32_t ok = __shfl_xor(bk, s, 64), oi = __shfl_xor(bi, s, 64);
        if (ok > bk || (ok == bk && oi < bi)) { bk = ok; bi = oi; }
    }
    if (lane == 0) { skey[wave] = bk; sidx[wave] = bi; }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < 16; ++w)
            if (skey[w] > bk || (skey[w] == bk && sidx[w] < bi)) { bk = skey[w]; bi = sidx[w]; }
        if (bi == INT32_MAX) {
            set_error(st, 3);
            bi = 0;
        }
        for (int b = 0; b < rows; ++b) st->ids[b] = bi;
        if (token_log) token_log[st->step] = bi;
    }
}

__global__ void advance_kernel(StepState* st, int rows) {
    if (threadIdx.x == 0) {
        // the launch's forward appended one position to every row (a launch
        // is never made for a token the sampler chose as the end)
        for (int b = 0; b < rows; ++b) st->pos[b] += 1;
        st->step += 1;
    }
}

// The xor butterflies through __shfl_xor (LDS crossbar): the reference the
// selftest holds the ALU lane exchanges of dev_mem.h to.
template <int HI, int LO>
__device__ __forceinline__ float shfl_sum(float v) {
#pragma unroll
    for (int s = HI; s >= LO; s >>= 1) v = v + __shfl_xor(v, s, 64);
    return v;
}

// Lane-exchange checks (which >= 4, whole waves: n % 256 == 0).
__device__ float lane_selftest(int which, float v) {
    switch (which) {
        case 4: return xor_lane<1>(v);
        case 5: return xor_lane<2>(v);
        case 6: return xor_lane<4>(v);
        case 7: return xor_lane<8>(v);
        case 8: return xor_lane<16>(v);
        case 9: return xor_lane<32>(v);
        case 10: return xor_sum<32>(v);
        case 11: return shfl_sum<32, 1>(v);
        case 12: return xor_sum<8>(v);
        case 13: return shfl_sum<8, 1>(v);
        case 14: return xor_sum<32, 16>(v);
        case 15: return shfl_sum<32, 16>(v);
        case 16: return xor_max<32>(v);
        default: return 0.0f;
    }
}

__global__ void math_selftest_kernel(int which, const void* in, void* out, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (which == 17) {
        // the RMSNorm scale of each 64-value vector (eps 1e-6), decided by the
        // wave as the head norms are; every lane stores it
        const float* vec = static_cast<const float*>(in) + (i & ~(size_t)63);
        static_cast<float*>(out)[i] = norm_scale_wave(vec, 64, 1e-6f);
        return;
    }
    if (which == 18) {
        // the RMSNorm scales (eps 1e-6) of the two 128-value rows of each
        // 256-value block, decided together by the block as the step
        // kernel's norms are; each row's threads store its scale
        const float* rows = static_cast<const float*>(in) + (size_t)blockIdx.x * 256;
        float sc[2];
        norm_scales_block<256, 2>(rows, 128, 1e-6f, nullptr, sc);
        static_cast<float*>(out)[i] = threadIdx.x < 128 ? sc[0] : sc[1];
        return;
    }
    if (which >= 4) {
        // every lane of the wave takes part in the exchange
        const float v = static_cast<const float*>(in)[i];
        static_cast<float*>(out)[i] = lane_selftest(which, v);
        return;
    }
    if (i >= n) return;
    if (which == 0) static_cast<float*>(out)[i] = expf_cr(static_cast<const float*>(in)[i]);
    else if (which == 1) static_cast<double*>(out)[i] = log1p_d(static_cast<const double*>(in)[i]);
    else if (which == 2) static_cast<float*>(out)[i] = rb(static_cast<const float*>(in)[i]);
    else if (which == 3) static_cast<float*>(out)[i] = silu_rb(static_cast<const float*>(in)[i]);
}

// ---------------------------------------------------------------------------
// Launchers
// ---------------------------------------------------------------------------
void launch_embed(hipStream_t s, const uint16_t* embed, const StepState* st, float* x, int hidden,
                  int vocab, int rows) {
    dim3 grid((hidden + 255) / 256, rows);
    embed_kernel<<<grid, 256, 0, s>>>(embed, const_cast<StepState*>(st), x, hidden, vocab);
}

void launch_rmsnorm(hipStream_t s, const float* x, int x_stride, const float* gamma, float* out,
                    int out_stride, int n, float eps, int rows, StepState* st) {
    rmsnorm_kernel<<<rows, 256, (size_t)n * sizeof(float), s>>>(x, x_stride, gamma, out,
                                                                 out_stride, n, eps, st);
}

void launch_argmax(hipStream_t s, const float* logits, int stride, int n, StepState* st,
                   int32_t* token_log, int rows) {
    (void)stride;
    argmax_kernel<<<1, 1024, 0, s>>>(logits, n, st, token_log, rows);
}

void launch_advance(hipStream_t s, StepState* st, int rows) {
    advance_kernel<<<1, 64, 0, s>>>(st, rows);
}

void launch_math_selftest(hipStream_t s, int which, const void* in, void* out, size_t n) {
    const unsigned blocks = (unsigned)((n + 255) / 256);
    if (blocks) math_selftest_kernel<<<blocks, 256, 0, s>>>(which, in, out, n);
}

}  // namespace y2

namespace y2 {

__global__ void fill_kernel(float* p, size_t n, float v) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        p[i] = v;
}

__global__ void set_state_kernel(StepState* st, int rows, int pos0, int pos1, int id0, int id1) {
    if (threadIdx.x == 0) {
        st->pos[0] = pos0;
        st->ids[0] = id0;
        if (rows > 1) {
            st->pos[1] = pos1;
            st->ids[1] = id1;
        }
    }
}

// Clears the step state and the sync counters: after a launch that stopped
// on an error the counters may hold arrivals that never completed.
__global__ void reset_state_kernel(StepState* st, int32_t* c0, int n0, int32_t* c1, int n1) {
    if (threadIdx.x == 0) {
        st->step = 0;
        st->error = 0;
        st->norm_fallbacks = 0;
        st->done = 0;
        // a new launch sequence: words tagged by a launch that stopped on an
        // error can never match the next launch's tags
        st->seq += 2;
    }
    for (int i = threadIdx.x; i < n0; i += blockDim.x) c0[i] = 0;
    for (int i = threadIdx.x; i < n1; i += blockDim.x) c1[i] = 0;
}

__global__ void sequence_kernel(StepState* st, int set, int value) {
    if (threadIdx.x == 0) st->seq = set ? value : st->seq + value;
}

void launch_sequence(hipStream_t s, StepState* st, int set, int value) {
    sequence_kernel<<<1, 64, 0, s>>>(st, set, value);
}

void launch_fill(hipStream_t s, float* p, size_t n, float v) {
    const unsigned blocks = (unsigned)std::min<size_t>((n + 255) / 256, 4096);
    if (blocks) fill_kernel<<<blocks, 256, 0, s>>>(p, n, v);
}

void launch_set_state(hipStream_t s, StepState* st, int rows, int pos0, int pos1, int id0, int id1) {
    set_state_kernel<<<1, 64, 0, s>>>(st, rows, pos0, pos1, id0, id1);
}

void launch_reset_state(hipStream_t s, StepState* st, int32_t* c0, int n0, int32_t* c1, int n1) {
    reset_state_kernel<<<1, 256, 0, s>>>(st, c0, c0 ? n0 : 0, c1, c1 ? n1 : 0);
}

}  // namespace y2
