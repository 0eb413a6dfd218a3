// dev_attn.h -- device body of the single-query GQA decode attention with
// the per-head QK RMSNorm, rotate-half RoPE and KV append of the new token
// fused in (src/model.rs:121-130, 151-168, 313-397; src/tensor.rs:706-724,
// 1158-1172).  Shared by the standalone attention kernel and the persistent
// token-step kernel.
//
// The reference normalises by the global maximum and the global sum before
// the PV product (p_j = exp(s_j - M) / sum, then sum_j p_j V_j), so the result
// cannot be merged from independently normalised partitions without changing
// its rounding.  The work of one (kv head, row) group is split over W
// workgroups by 64-key blocks and runs the exact schedule in three phases
// separated by syncs among those W workgroups only:
//   1. q-norm + RoPE (every workgroup, for its group's query heads); the
//      workgroup owning the newest key also norms/ropes k and appends K/V;
//      scaled scores of its blocks into LDS, block maxima to HBM.
//   2. M = max of the group's block maxima; e_j = exp(s_j - M) in LDS; block
//      sums (64-lane butterfly) to HBM.
//   3. total = super-block sums left to right; p_j = e_j / total; partial PV
//      per block (512/dim key streams, butterfly over streams), the blocks of
//      each super-block added left to right, to HBM; the last workgroup to
//      finish adds the super-blocks left to right and rounds to BF16.
// Blocks are grouped in super-blocks (attn_superblock, kernels.h) and each
// workgroup takes whole super-blocks, so it publishes one block sum and one
// partial per super-block.
// Each sync waits on a counter with a bounded spin: on timeout the device
// error is set and the workgroup leaves, so every launch terminates.  All
// workgroups of a group must be resident at once (callers launch at most one
// workgroup per CU).  The blocks per workgroup follow the live length, so a
// short context still spreads over every workgroup of its group.
//
// Data crossing workgroups inside a launch (the projected q/k/v rows, block
// maxima and sums, partial outputs, the merged output) is written and read
// with agent-scope relaxed atomics: on gfx950 these are sc1 accesses, which
// write through to and read from the device-coherent level, so no L2
// write-back or invalidate is needed.  A workgroup completes its stores
// (s_waitcnt) before it signals a counter.
#pragma once
#include <hip/hip_runtime.h>

#include "dev_mem.h"
#include "kernels.h"
#include "y2_math.h"

namespace y2 {

constexpr int kDevErrTimeout = 6;

__device__ __forceinline__ void unpack8a(const uint4 w, float* f) {
    f[0] = bf16_lo(w.x); f[1] = bf16_hi(w.x);
    f[2] = bf16_lo(w.y); f[3] = bf16_hi(w.y);
    f[4] = bf16_lo(w.z); f[5] = bf16_hi(w.z);
    f[6] = bf16_lo(w.w); f[7] = bf16_hi(w.w);
}

__device__ __forceinline__ size_t kv_off(int layer, int which, int kv_heads, int head, int capacity,
                                         int pos, int dim) {
    return ((((size_t)layer * 2 + which) * kv_heads + head) * capacity + pos) * dim;
}

// Add one to *cnt and return the old value.  Callers complete their stores
// (stores_done) and pass a workgroup barrier first.
__device__ __forceinline__ int signal(int* cnt) { return add_dev(cnt, 1); }

// Wait (thread 0 spins on relaxed loads, bounded) until *cnt >= target.
// false on timeout or when another workgroup has already reported an error.
__device__ __forceinline__ bool wait_for(int* cnt, int target, StepState* st) {
    __shared__ int s_ok;
    if (threadIdx.x == 0) {
        int ok = 1;
        unsigned spins = 0;
        while (ld_dev_i(cnt) < target) {
            if (++spins > (1u << 22) || ld_dev_i(&st->error)) {
                set_error(&st->error, kDevErrTimeout);
                ok = 0;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        s_ok = ok;
    }
    __syncthreads();
    return s_ok != 0;
}

// Block counts up to which the last workgroup of a group merges every output
// (one round of loads); beyond, each workgroup merges a share after one more
// group barrier.
constexpr int kMergeLastMax = 32;

// LDS bytes attn_group needs: the scores of G heads over bpw blocks and the
// group's block sums, later the merge's [outputs][blocks] partials.
__host__ __device__ constexpr size_t attn_group_lds(int G, int D, int wgs, int bpw) {
    const size_t scores = (size_t)G * bpw * kBlockKeys + (size_t)G * wgs * bpw, merge = ((size_t)G * D + wgs) * bpw;
    return (scores > merge ? scores : merge) * sizeof(float);
}

// One workgroup's share of the attention of kv head g, batch row b: the
// workgroup handles 64-key blocks [wg * bpw, (wg + 1) * bpw) of that head.
// G = heads / kv_heads <= MAXG query heads share the K/V rows.  e_s: LDS
// scratch of attn_group_lds(G, D, wgs, bpw) bytes.  Returns false when a
// group sync timed out (the device error is set).
template <int NT, int D, int MAXG>
__device__ __forceinline__ bool attn_group(const AttnArgs& a, int wg, int g, int b, float* e_s) {
    constexpr int NW = NT / 64;
    __shared__ float q_s[MAXG][D];
    __shared__ float k_s[D];
    __shared__ float hscale[MAXG + 1];
    __shared__ float m_s[MAXG], t_s[MAXG];
    constexpr int CPL = D / 8;     // lanes per key row
    constexpr int KPW = 64 / CPL;  // keys per wave load
    constexpr int S = KPW;         // PV key streams per 64-key block
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    StepState* st = a.st;
    const int pos = *gbl(&st->pos[b]);
    // (selects, not an indexed load: a runtime index would place the
    // argument copy in scratch memory)
    const int L = pos + 1, cap = b == 0 ? a.kv.capacity[0] : a.kv.capacity[1];
    uint16_t* const kv_base = b == 0 ? a.kv.base[0] : a.kv.base[1];
    if (pos < 0 || L > cap) {
        if (tid == 0 && wg == 0) set_error(&st->error, 1);
        return true;
    }
    const int nb = (L + kBlockKeys - 1) / kBlockKeys;
    const int sb = attn_superblock(nb), lsb = sb == 1 ? 0 : sb == 2 ? 1 : 2, nsb = (nb + sb - 1) >> lsb;
    const int bpw = attn_bpw(nb, a.wgs);  // <= a.bpw, which sizes e_s
    const int W = (nb + bpw - 1) / bpw;
    if (wg >= W) return true;
    const int G = a.heads / a.kv_heads;
    const int blk0 = wg * bpw, blk1 = min(nb, blk0 + bpw), nbl = blk1 - blk0;
    const int j0 = blk0 * kBlockKeys, j1 = min(L, blk1 * kBlockKeys), nk = j1 - j0;
    const int estride = bpw * kBlockKeys;
    int* cnt = a.counters + ((size_t)b * a.kv_heads + g) * 4;
    const float* row = a.qkv + (size_t)b * a.qkv_stride;
    uint16_t* Kc = kv_base + kv_off(a.layer, 0, a.kv_heads, g, cap, 0, D);
    uint16_t* Vc = kv_base + kv_off(a.layer, 1, a.kv_heads, g, cap, 0, D);
    const size_t hbase = ((size_t)b * a.heads + (size_t)g * G) * a.blk_stride;

    // ---- phase 0: queries (and the new key/value) -------------------------
    for (int i = tid; i < G * D; i += NT) q_s[i / D][i % D] = ld_dev(row + (size_t)(g * G) * D + i);
    const bool owns_new = j1 == L && a.q_norm != nullptr;
    if (owns_new)
        for (int d = tid; d < D; d += NT) k_s[d] = ld_dev(row + (size_t)(a.heads + g) * D + d);
    __syncthreads();
    if (a.q_norm) {
        // Norm::heads: sequential sum of squares per head (src/tensor.rs:1160).
        if (tid < G || (owns_new && tid == G)) {
            const float* v = tid < G ? q_s[tid] : k_s;
            float sum = -0.0f;
            for (int d = 0; d < D; d += 16) {
                float t[16];
#pragma unroll
                for (int j = 0; j < 16; ++j) t[j] = v[d + j];
#pragma unroll
                for (int j = 0; j < 16; ++j) sum = sum + t[j] * t[j];
            }
            hscale[tid] = norm_scale_from_sum(sum, D, a.eps);
        }
        __syncthreads();
        const int half = D / 2;
        const float* cs = a.cos_t + (size_t)pos * half;
        const float* sn = a.sin_t + (size_t)pos * half;
        const int pairs = (G + (owns_new ? 1 : 0)) * half;
        for (int i = tid; i < pairs; i += NT) {
            const int h = i / half, d = i % half;
            float* v = h < G ? q_s[h] : k_s;
            const float* gam = h < G ? a.q_norm : a.k_norm;
            const float s = hscale[h];
            const float x0 = rb(rb(v[d] * s) * gbl(gam)[d]);
            const float x1 = rb(rb(v[d + half] * s) * gbl(gam)[d + half]);
            const float c = gbl(cs)[d], si = gbl(sn)[d];
            const float y0 = rb(rb(x0 * c) - rb(x1 * si));
            const float y1 = rb(rb(x1 * c) + rb(x0 * si));
            v[d] = y0;
            v[d + half] = y1;
            if (h == G) {
                gblw(Kc)[(size_t)pos * D + d] = bf16_bits(y0);
                gblw(Kc)[(size_t)pos * D + d + half] = bf16_bits(y1);
            }
        }
        if (owns_new) {
            const float* vs = row + (size_t)(a.heads + a.kv_heads + g) * D;
            for (int d = tid; d < D; d += NT) gblw(Vc)[(size_t)pos * D + d] = bf16_bits(ld_dev(vs + d));
        }
        __syncthreads();
    }

    // ---- phase 1: scaled scores and block maxima ---------------------------
    {
        const int c = lane % CPL, kk = lane / CPL;
        float qv[MAXG][8];
#pragma unroll
        for (int h = 0; h < MAXG; ++h)
#pragma unroll
            for (int e = 0; e < 8; ++e) qv[h][e] = h < G ? q_s[h][8 * c + e] : 0.0f;
        // each wave takes R consecutive key slots of KPW keys per round
        constexpr int R = 8;
        for (int base = j0 + wave * R * KPW; base < j1; base += NW * R * KPW) {
            uint4 kr[R];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int j = base + r * KPW + kk;
                kr[r] = j < j1 ? ldg4(Kc + (size_t)j * D + 8 * c)
                               : make_uint4(0, 0, 0, 0);
            }
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int j = base + r * KPW + kk;
                float kf[8];
                unpack8a(kr[r], kf);
#pragma unroll
                for (int h = 0; h < MAXG; ++h) {
                    if (h >= G) break;
                    float acc = 0.0f;
#pragma unroll
                    for (int e = 0; e < 8; ++e) acc = __builtin_fmaf(qv[h][e], kf[e], acc);
acc = xor_sum<CPL / 2>(acc);
                    if (c == 0 && j < j1) e_s[h * estride + (j - j0)] = acc * a.scale;
                }
            }
        }
        __syncthreads();
        for (int i = wave; i < G * nbl; i += NW) {
            const int h = i / nbl, bl = i % nbl;
            const int jl = bl * kBlockKeys + lane;
            float m = jl < nk ? e_s[h * estride + jl] : -__builtin_huge_valf();
m = xor_max<32>(m);
            if (lane == 0) st_dev(a.bmax + hbase + (size_t)h * a.blk_stride + blk0 + bl, m);
        }
        stores_done();
        __syncthreads();
        if (tid == 0) signal(&cnt[0]);
        if (!wait_for(&cnt[0], W, st)) return false;
    }

    // ---- phase 2: exp(s - M) and block sums --------------------------------
    {
        for (int h = wave; h < G; h += NW) {
            const float* bm = a.bmax + hbase + (size_t)h * a.blk_stride;
            // every block maximum of the head requested at once (nb <= 384)
            float v[6];
#pragma unroll
            for (int u = 0; u < 6; ++u) v[u] = lane + 64 * u < nb ? ld_dev(bm + lane + 64 * u) : -__builtin_huge_valf();
            float m = v[0];
#pragma unroll
            for (int u = 1; u < 6; ++u) m = fmaxf(m, v[u]);
m = xor_max<32>(m);
            if (lane == 0) m_s[h] = m;
        }
        __syncthreads();
        for (int i = tid; i < G * nk; i += NT) {
            const int h = i / nk, jl = i % nk;
            e_s[h * estride + jl] = expf_cr(e_s[h * estride + jl] - m_s[h]);
        }
        __syncthreads();
        float* bl_s = e_s + G * estride;  // [G][nbl] block sums (the gather region of phase 3)
        for (int i = wave; i < G * nbl; i += NW) {
            const int h = i / nbl, bl = i % nbl;
            const int jl = bl * kBlockKeys + lane;
            float v = jl < nk ? e_s[h * estride + jl] : 0.0f;
v = xor_sum<32>(v);
            if (lane == 0) bl_s[h * nbl + bl] = v;
        }
        __syncthreads();
        // each super-block's block sums left to right
        const int nsbl = (nbl + sb - 1) >> lsb;
        for (int i = tid; i < G * nsbl; i += NT) {
            const int h = i / nsbl, k = i % nsbl, b0 = k * sb, b1 = min(nbl, b0 + sb);
            float u = bl_s[h * nbl + b0];
            for (int j = b0 + 1; j < b1; ++j) u = u + bl_s[h * nbl + j];
            st_dev(a.bsum + hbase + (size_t)h * a.blk_stride + (blk0 >> lsb) + k, u);
        }
        stores_done();
        __syncthreads();
        if (tid == 0) signal(&cnt[1]);
        if (!wait_for(&cnt[1], W, st)) return false;
    }

    // ---- phase 3: p = e / total, partial PV, merge by the last workgroup ---
    {
        // total = super-block sums added left to right; the sums are
        // gathered into LDS by all threads first (a chain of dependent device
        // loads would pay a memory round trip per super-block)
        {
            float* bs = e_s + G * estride;  // [G][nsb] super-block sums, after the scores
            const int total = G * nsb;       // <= 8 * 384 = 6 * 512
            float v[6];
#pragma unroll
            for (int u = 0; u < 6; ++u) {
                const int i = tid + u * NT, h = i / nsb, j = i - h * nsb;
                v[u] = i < total ? ld_dev(a.bsum + hbase + (size_t)h * a.blk_stride + j) : 0.0f;
            }
            __syncthreads();  // every thread is done with the block sums in bs
#pragma unroll
            for (int u = 0; u < 6; ++u)
                if (tid + u * NT < total) bs[tid + u * NT] = v[u];
            __syncthreads();
            if (tid < G) {
                float tot = bs[tid * nsb];
                for (int j = 1; j < nsb; ++j) tot = tot + bs[tid * nsb + j];
                t_s[tid] = tot;
            }
        }
        __syncthreads();
        for (int i = tid; i < G * nk; i += NT) {
            const int h = i / nk, jl = i % nk;
            e_s[h * estride + jl] = e_s[h * estride + jl] / t_s[h];
        }
        __syncthreads();
        const int t = lane / CPL, c = lane % CPL;
        float sacc[MAXG][8];  // the super-block's blocks so far, left to right
        for (int it = wave * sb; it < nbl; it += ((it & (sb - 1)) == sb - 1 ? (NW - 1) * sb + 1 : 1)) {
            const int bl = it;
            const int bi = bl & (sb - 1);
            const int jb = (blk0 + bl) * kBlockKeys;
            uint4 vr[kBlockKeys / S];
#pragma unroll
            for (int i = 0; i < kBlockKeys / S; ++i) {
                const int j = jb + t + S * i;
                vr[i] = j < L ? ldg4(Vc + (size_t)j * D + 8 * c)
                              : make_uint4(0, 0, 0, 0);
            }
            float acc[MAXG][8];
#pragma unroll
            for (int h = 0; h < MAXG; ++h)
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[h][e] = 0.0f;
            // no branch per key: keys past the context have zero V rows and
            // p = 0, and fma(0, 0, acc) = acc (a chain from +0 is never -0)
#pragma unroll
            for (int i = 0; i < kBlockKeys / S; ++i) {
                const int jj = t + S * i;
                float vf[8];
                unpack8a(vr[i], vf);
#pragma unroll
                for (int h = 0; h < MAXG; ++h) {
                    if (h >= G) break;
                    const float p = jb + jj < L ? e_s[h * estride + bl * kBlockKeys + jj] : 0.0f;
#pragma unroll
                    for (int e = 0; e < 8; ++e) acc[h][e] = __builtin_fmaf(p, vf[e], acc[h][e]);
                }
            }
#pragma unroll
            for (int h = 0; h < MAXG; ++h)
                if (h < G)
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const float v = xor_sum<32, CPL>(acc[h][e]);
                        sacc[h][e] = bi == 0 ? v : sacc[h][e] + v;
                    }
            if (t == 0 && (bi == sb - 1 || bl == nbl - 1)) {
#pragma unroll
                for (int h = 0; h < MAXG; ++h)
                    if (h < G) {
                        float* dst = a.part + ((hbase + (size_t)h * a.blk_stride) + ((blk0 + bl) >> lsb)) * D + 8 * c;
#pragma unroll
                        for (int e = 0; e < 8; ++e) st_dev(dst + e, sacc[h][e]);
                    }
            }
        }
        stores_done();
        __syncthreads();
        if (nsb <= kMergeLastMax) {
            // short contexts: the last workgroup through merges every output
            __shared__ int s_last;
            if (tid == 0) s_last = signal(&cnt[2]) == W - 1;
            __syncthreads();
            if (!s_last) return true;
            for (int i = tid; i < G * D; i += NT) {
                const int h = i / D, d = i % D;
                const float* pp = a.part + (hbase + (size_t)h * a.blk_stride) * D + d;
                float v[kMergeLastMax];
#pragma unroll
                for (int j = 0; j < kMergeLastMax; ++j) v[j] = j < nsb ? ld_dev(pp + (size_t)j * D) : 0.0f;
                float o = v[0];
#pragma unroll
                for (int j = 1; j < kMergeLastMax; ++j)
                    if (j < nsb) o = o + v[j];  // super-blocks left to right
                st_dev(a.out + (size_t)b * a.out_stride + (size_t)(g * G + h) * D + d, rb(o));
            }
            if (tid < 3) st_dev_i(&cnt[tid], 0);
            return true;
        }
        if (tid == 0) signal(&cnt[2]);
        if (!wait_for(&cnt[2], W, st)) return false;
        // longer contexts: workgroup wg adds the blocks (left to right) of the outputs
        // [o0, o1) of the group.  Its partials are first gathered into LDS by
        // all threads, 16 requests per thread in flight: a chain of dependent
        // device loads would pay a memory round trip per block.
        const int outs = G * D, chunk = (outs + W - 1) / W;
        const int o0 = min(outs, wg * chunk), o1 = min(outs, o0 + chunk), no = o1 - o0;
        float* mb = e_s;  // [no][nsb]; the scores are no longer needed
        const float* part = a.part + hbase * D;
        const int total = no * nsb;
        for (int base = 0; base < total; base += 16 * NT) {
            float v[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                const int i = base + tid + u * NT;
                float x = 0.0f;
                if (i < total) {
                    const int r = i / nsb, k = i - r * nsb, o = o0 + r;
                    x = ld_dev(part + ((size_t)(o / D) * a.blk_stride + k) * D + o % D);
                }
                v[u] = x;
            }
#pragma unroll
            for (int u = 0; u < 16; ++u)
                if (base + tid + u * NT < total) mb[base + tid + u * NT] = v[u];
        }
        __syncthreads();
        for (int i = tid; i < no; i += NT) {
            const float* pp = mb + i * nsb;
            float o = pp[0];
            for (int k = 1; k < nsb; ++k) o = o + pp[k];  // super-blocks left to right
            st_dev(a.out + (size_t)b * a.out_stride + (size_t)(g * G) * D + o0 + i, rb(o));
        }
        __syncthreads();
        // the last workgroup through clears the group's counters for the
        // next launch (every workgroup has passed all of its waits)
        if (tid == 0 && signal(&cnt[3]) == W - 1)
            for (int c = 0; c < 4; ++c) st_dev_i(&cnt[c], 0);
    }
    return true;
}

}  // namespace y2
