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
    extern __shared__ float xs[];
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
// BF16 GEMV with FP32 accumulation in the DOT order (Linear::apply_range +
// finish, src/tensor.rs:946-1118).  One wave owns one weight row at a time;
// each lane streams its 16-byte chunks with 128-bit loads.  Inputs are staged
// in LDS once per workgroup and reused for every row and batch row.
//   EPI_STORE   y = rb(dot)
//   EPI_RESID   y = rb(y + rb(dot))               (Tensor::add, :632-640)
//   EPI_SWIGLU  y = rb(rb(silu(rb(g))) * rb(u))   (Mlp::apply, src/model.rs:206-214)
//   EPI_RAW     y = dot, unrounded                (yue2_metal_vector, src/metal.m:545-603)
// ---------------------------------------------------------------------------
template <int B, int EPI, int IT>
__global__ __launch_bounds__(256) void gemv_kernel(const GemvArgs a) {
    extern __shared__ float xs[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int k = a.k, nchunk = k >> 3;
    for (int b = 0; b < B; ++b)
        for (int i = tid; i < k; i += 256) xs[b * k + i] = a.x[(size_t)b * a.x_stride + i];
    __syncthreads();
    for (int row = blockIdx.x * 4 + wave; row < a.n; row += gridDim.x * 4) {
        const uint4* wr = reinterpret_cast<const uint4*>(a.w + (size_t)row * k);
        uint4 wv[IT];
        uint4 wv2[EPI == EPI_SWIGLU ? IT : 1];
#pragma unroll
        for (int it = 0; it < IT; ++it) {
            const int c = lane + 64 * it;
            wv[it] = c < nchunk ? wr[c] : make_uint4(0, 0, 0, 0);
        }
        if constexpr (EPI == EPI_SWIGLU) {
            const uint4* wr2 = reinterpret_cast<const uint4*>(a.w2 + (size_t)row * k);
#pragma unroll
            for (int it = 0; it < IT; ++it) {
                const int c = lane + 64 * it;
                wv2[it] = c < nchunk ? wr2[c] : make_uint4(0, 0, 0, 0);
            }
        }
        float acc[B], acc2[B];
#pragma unroll
        for (int b = 0; b < B; ++b) acc[b] = acc2[b] = 0.0f;
#pragma unroll
        for (int it = 0; it < IT; ++it) {
            const int c = lane + 64 * it;
            if (c < nchunk) {
                float wf[8];
                unpack8(wv[it], wf);
                float wf2[8];
                if constexpr (EPI == EPI_SWIGLU) unpack8(wv2[it], wf2);
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
            acc[b] = butterfly64(acc[b]);
            if constexpr (EPI == EPI_SWIGLU) acc2[b] = butterfly64(acc2[b]);
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
}

// ---------------------------------------------------------------------------
// Per-head QK RMSNorm + rotate-half RoPE + KV append (src/tensor.rs:1158-1172,
// src/model.rs:151-168, :576-577).  One wave per (head, row).  The head norm's
// sum runs sequentially in lane 0 (dim <= 256 terms).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(64) void heads_kernel(const HeadArgs a) {
    __shared__ float v[512];
    const int h = blockIdx.x, b = blockIdx.y, lane = threadIdx.x;
    const int D = a.dim, half = D >> 1;
    const int pos = a.st->pos[b];
    if (pos < 0 || pos >= a.kv.capacity[b]) {
        if (lane == 0) set_error(const_cast<StepState*>(a.st), DEV_ERR_CONTEXT);
        return;
    }
    float* row = a.qkv + (size_t)b * a.qkv_stride;
    const bool is_q = h < a.heads;
    const int kvh = is_q ? 0 : h - a.heads;
    float* src = row + (size_t)(is_q ? h : a.heads + kvh) * D;
    const float* gamma = is_q ? a.q_norm : a.k_norm;
    for (int i = lane; i < D; i += 64) v[i] = src[i];
    __syncthreads();
    float scale = 0.0f;
    if (lane == 0) {
        float sum = -0.0f;
        for (int i = 0; i < D; ++i) sum = sum + v[i] * v[i];
        scale = norm_scale_from_sum(sum, D, a.eps);
    }
    scale = __shfl(scale, 0, 64);
    const float* cs = a.cos_t + (size_t)pos * half;
    const float* sn = a.sin_t + (size_t)pos * half;
    uint16_t* kdst = a.kv.base[b] + kv_offset(a.layer, 0, a.kv_heads, kvh, a.kv.capacity[b], pos, D);
    for (int i = lane; i < half; i += 64) {
        const float x0 = rb(rb(v[i] * scale) * gamma[i]);
        const float x1 = rb(rb(v[i + half] * scale) * gamma[i + half]);
        const float c = cs[i], s = sn[i];
        const float y0 = rb(rb(x0 * c) - rb(x1 * s));
        const float y1 = rb(rb(x1 * c) + rb(x0 * s));
        if (is_q) {
            src[i] = y0;
            src[i + half] = y1;
        } else {
            kdst[i] = bf16_bits(y0);
            kdst[i + half] = bf16_bits(y1);
        }
    }
    if (!is_q) {
        const float* vs = row + (size_t)(a.heads + a.kv_heads + kvh) * D;
        uint16_t* vdst =
            a.kv.base[b] + kv_offset(a.layer, 1, a.kv_heads, kvh, a.kv.capacity[b], pos, D);
        for (int d = lane; d < D; d += 64) vdst[d] = bf16_bits(vs[d]);
    }
}

// ---------------------------------------------------------------------------
// Attention, phase 1: scaled scores s_j = DOT(q, K_j) * scale and 64-key
// block maxima (src/model.rs:362-374; vDSP_vsmul/maxv, src/tensor.rs:715-716).
// One workgroup per (kv head, 64-key block, row); each K row is read once and
// serves all query heads of the group.  dim/8 lanes hold one key.
// ---------------------------------------------------------------------------
constexpr int kMaxGroup = 8;

template <int D>
__global__ __launch_bounds__(256) void attn_scores_kernel(const AttnArgs a) {
    const int g = blockIdx.x, blk = blockIdx.y, b = blockIdx.z;
    const int L = a.st->pos[b] + 1;
    const int j0 = blk * kBlockKeys;
    if (j0 >= L || L > a.kv.capacity[b]) return;
    constexpr int CPL = D / 8, KPW = 64 / CPL;
    const int G = a.heads / a.kv_heads;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int c = lane % CPL, kk = lane / CPL;
    __shared__ float smax[4][kMaxGroup];
    float qv[kMaxGroup][8];
    const float* qrow = a.q + (size_t)b * a.q_stride;
#pragma unroll
    for (int h = 0; h < kMaxGroup; ++h)
        if (h < G) {
#pragma unroll
            for (int e = 0; e < 8; ++e) qv[h][e] = qrow[(size_t)(g * G + h) * D + 8 * c + e];
        }
    const uint16_t* K = a.kv.base[b] + kv_offset(a.layer, 0, a.kv_heads, g, a.kv.capacity[b], 0, D);
    float lmax[kMaxGroup];
#pragma unroll
    for (int h = 0; h < kMaxGroup; ++h) lmax[h] = -__builtin_huge_valf();
#pragma unroll
    for (int it = 0; it < 16 / KPW; ++it) {
        const int j = j0 + wave * 16 + it * KPW + kk;
        const bool valid = j < L;
        float kf[8];
        const uint4 k4 = valid ? *reinterpret_cast<const uint4*>(K + (size_t)j * D + 8 * c)
                               : make_uint4(0, 0, 0, 0);
        unpack8(k4, kf);
#pragma unroll
        for (int h = 0; h < kMaxGroup; ++h)
            if (h < G) {
                float acc = 0.0f;
#pragma unroll
                for (int e = 0; e < 8; ++e) acc = __builtin_fmaf(qv[h][e], kf[e], acc);
#pragma unroll
                for (int s = CPL / 2; s >= 1; s >>= 1) acc = acc + __shfl_xor(acc, s, 64);
                const float sc = acc * a.scale;
                if (valid) {
                    if (c == 0) a.scores[((size_t)b * a.heads + g * G + h) * a.score_stride + j] = sc;
                    lmax[h] = fmaxf(lmax[h], sc);
                }
            }
    }
#pragma unroll
    for (int h = 0; h < kMaxGroup; ++h)
        if (h < G) {
            float m = lmax[h];
#pragma unroll
            for (int s = 32; s >= 1; s >>= 1) m = fmaxf(m, __shfl_xor(m, s, 64));
            if (lane == 0) smax[wave][h] = m;
        }
    __syncthreads();
    if (tid < G) {
        const float m = fmaxf(fmaxf(smax[0][tid], smax[1][tid]), fmaxf(smax[2][tid], smax[3][tid]));
        a.bmax[((size_t)b * a.heads + g * G + tid) * a.blk_stride + blk] = m;
    }
}

// Phase 2: global max, e_j = exp(s_j - M), 64-key block sums by butterfly
// (vDSP_vsadd + vvexpf + vDSP_sve, src/tensor.rs:717-721).
__global__ __launch_bounds__(64) void attn_exp_kernel(const AttnArgs a) {
    const int h = blockIdx.x, blk = blockIdx.y, b = blockIdx.z, lane = threadIdx.x;
    const int L = a.st->pos[b] + 1;
    const int j0 = blk * kBlockKeys;
    if (j0 >= L || L > a.kv.capacity[b]) return;
    const int nb = (L + kBlockKeys - 1) / kBlockKeys;
    const size_t hb = (size_t)b * a.heads + h;
    const float* bm = a.bmax + hb * a.blk_stride;
    float m = -__builtin_huge_valf();
    for (int i = lane; i < nb; i += 64) m = fmaxf(m, bm[i]);
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) m = fmaxf(m, __shfl_xor(m, s, 64));
    float* sc = a.scores + hb * a.score_stride;
    const int j = j0 + lane;
    float e = 0.0f;
    if (j < L) {
        e = expf_cr(sc[j] - m);
        sc[j] = e;
    }
    e = butterfly64(e);
    if (lane == 0) a.bsum[hb * a.blk_stride + blk] = e;
}

// Phase 3: total = block sums left to right, p_j = e_j / total (vDSP_vsdiv),
// partial PV per block in the stream order (src/model.rs:380-392).
template <int D>
__global__ __launch_bounds__(64) void attn_pv_kernel(const AttnArgs a) {
    const int g = blockIdx.x, blk = blockIdx.y, b = blockIdx.z, lane = threadIdx.x;
    const int L = a.st->pos[b] + 1;
    const int j0 = blk * kBlockKeys;
    if (j0 >= L || L > a.kv.capacity[b]) return;
    const int nb = (L + kBlockKeys - 1) / kBlockKeys;
    const int G = a.heads / a.kv_heads;
    __shared__ float p[kMaxGroup][kBlockKeys];
    __shared__ float stot[kMaxGroup];
    if (lane < G) {
        const float* bs = a.bsum + ((size_t)b * a.heads + g * G + lane) * a.blk_stride;
        float tot = bs[0];
        for (int i = 1; i < nb; ++i) tot = tot + bs[i];
        stot[lane] = tot;
    }
    __syncthreads();
    for (int h = 0; h < G; ++h) {
        const int j = j0 + lane;
        const float* sc = a.scores + ((size_t)b * a.heads + g * G + h) * a.score_stride;
        p[h][lane] = j < L ? sc[j] / stot[h] : 0.0f;
    }
    __syncthreads();
    constexpr int CPL = D / 8, S = 64 / CPL;
    const int t = lane / CPL, c = lane % CPL;
    const uint16_t* V = a.kv.base[b] + kv_offset(a.layer, 1, a.kv_heads, g, a.kv.capacity[b], 0, D);
    float acc[kMaxGroup][8];
#pragma unroll
    for (int h = 0; h < kMaxGroup; ++h)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[h][e] = 0.0f;
#pragma unroll
    for (int i = 0; i < kBlockKeys / S; ++i) {
        const int jj = t + S * i, j = j0 + jj;
        if (j < L) {
            float vf[8];
            unpack8(*reinterpret_cast<const uint4*>(V + (size_t)j * D + 8 * c), vf);
#pragma unroll
            for (int h = 0; h < kMaxGroup; ++h)
                if (h < G) {
                    const float pj = p[h][jj];
#pragma unroll
                    for (int e = 0; e < 8; ++e) acc[h][e] = __builtin_fmaf(pj, vf[e], acc[h][e]);
                }
        }
    }
#pragma unroll
    for (int s = 32; s >= CPL; s >>= 1)
#pragma unroll
        for (int h = 0; h < kMaxGroup; ++h)
            if (h < G)
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[h][e] = acc[h][e] + __shfl_xor(acc[h][e], s, 64);
    if (t == 0) {
#pragma unroll
        for (int h = 0; h < kMaxGroup; ++h)
            if (h < G) {
                float* dst = a.part + (((size_t)b * a.heads + g * G + h) * a.blk_stride + blk) * D + 8 * c;
#pragma unroll
                for (int e = 0; e < 8; ++e) dst[e] = acc[h][e];
            }
    }
}

// Phase 4: blocks added left to right, rounded to BF16 (Tensor::rounded).
__global__ __launch_bounds__(256) void attn_merge_kernel(const AttnArgs a) {
    const int h = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
    if (d >= a.dim) return;
    const int L = a.st->pos[b] + 1;
    if (L > a.kv.capacity[b]) return;
    const int nb = (L + kBlockKeys - 1) / kBlockKeys;
    const float* pp = a.part + ((size_t)b * a.heads + h) * a.blk_stride * a.dim + d;
    float o = pp[0];
    for (int i = 1; i < nb; ++i) o = o + pp[(size_t)i * a.dim];
    a.out[(size_t)b * a.out_stride + (size_t)h * a.dim + d] = rb(o);
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
        for (int b = 0; b < rows; ++b) st->pos[b] += 1;
        st->step += 1;
    }
}

__global__ void math_selftest_kernel(int which, const void* in, void* out, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
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

template <int B, int EPI>
static hipError_t gemv_dispatch(hipStream_t s, const GemvArgs& a) {
    const int iters = (a.k / 8 + 63) / 64;
    const int blocks = std::min((a.n + 3) / 4, 1024);
    const size_t lds = (size_t)B * a.k * sizeof(float);
#define Y2_GEMV_CASE(N)                                                            \
    if (iters <= N) {                                                              \
        auto fn = gemv_kernel<B, EPI, N>;                                          \
        if (lds > 65536) {                                                         \
            hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn),  \
                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);             \
            if (e != hipSuccess) return e;                                         \
        }                                                                          \
        fn<<<blocks, 256, lds, s>>>(a);                                            \
        return hipGetLastError();                                                  \
    }
    Y2_GEMV_CASE(1)
    Y2_GEMV_CASE(2)
    Y2_GEMV_CASE(4)
    Y2_GEMV_CASE(6)
    Y2_GEMV_CASE(8)
    Y2_GEMV_CASE(12)
    Y2_GEMV_CASE(16)
    Y2_GEMV_CASE(24)
    Y2_GEMV_CASE(32)
#undef Y2_GEMV_CASE
    return hipErrorInvalidValue;
}

hipError_t launch_gemv(hipStream_t s, int epi, const GemvArgs& a) {
    if (a.k % 8 != 0 || a.k > 32 * 512 || a.rows < 1 || a.rows > kMaxRows) return hipErrorInvalidValue;
    if ((size_t)a.rows * a.k * sizeof(float) > 160 * 1024) return hipErrorInvalidValue;
    if (a.rows == 1) {
        if (epi == EPI_STORE) return gemv_dispatch<1, EPI_STORE>(s, a);
        if (epi == EPI_RESID) return gemv_dispatch<1, EPI_RESID>(s, a);
        if (epi == EPI_RAW) return gemv_dispatch<1, EPI_RAW>(s, a);
        return gemv_dispatch<1, EPI_SWIGLU>(s, a);
    }
    if (epi == EPI_RAW) return gemv_dispatch<2, EPI_RAW>(s, a);
    if (epi == EPI_STORE) return gemv_dispatch<2, EPI_STORE>(s, a);
    if (epi == EPI_RESID) return gemv_dispatch<2, EPI_RESID>(s, a);
    return gemv_dispatch<2, EPI_SWIGLU>(s, a);
}

void launch_heads(hipStream_t s, const HeadArgs& a) {
    dim3 grid(a.heads + a.kv_heads, a.rows);
    heads_kernel<<<grid, 64, 0, s>>>(a);
}

void launch_attention(hipStream_t s, const AttnArgs& a) {
    dim3 g_kv(a.kv_heads, a.max_blocks, a.rows), g_q(a.heads, a.max_blocks, a.rows);
    if (a.dim == 64) {
        attn_scores_kernel<64><<<g_kv, 256, 0, s>>>(a);
        attn_exp_kernel<<<g_q, 64, 0, s>>>(a);
        attn_pv_kernel<64><<<g_kv, 64, 0, s>>>(a);
    } else if (a.dim == 128) {
        attn_scores_kernel<128><<<g_kv, 256, 0, s>>>(a);
        attn_exp_kernel<<<g_q, 64, 0, s>>>(a);
        attn_pv_kernel<128><<<g_kv, 64, 0, s>>>(a);
    } else {
        attn_scores_kernel<256><<<g_kv, 256, 0, s>>>(a);
        attn_exp_kernel<<<g_q, 64, 0, s>>>(a);
        attn_pv_kernel<256><<<g_kv, 64, 0, s>>>(a);
    }
    attn_merge_kernel<<<dim3(a.heads, a.rows), 256, 0, s>>>(a);
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

__global__ void reset_state_kernel(StepState* st) {
    if (threadIdx.x == 0) {
        st->step = 0;
        st->error = 0;
        st->norm_fallbacks = 0;
        st->done = 0;
    }
}

void launch_fill(hipStream_t s, float* p, size_t n, float v) {
    const unsigned blocks = (unsigned)std::min<size_t>((n + 255) / 256, 4096);
    if (blocks) fill_kernel<<<blocks, 256, 0, s>>>(p, n, v);
}

void launch_set_state(hipStream_t s, StepState* st, int rows, int pos0, int pos1, int id0, int id1) {
    set_state_kernel<<<1, 64, 0, s>>>(st, rows, pos0, pos1, id0, id1);
}

void launch_reset_state(hipStream_t s, StepState* st) { reset_state_kernel<<<1, 64, 0, s>>>(st); }

}  // namespace y2
