// dev_ring.h -- the weight-streaming GEMV of the decode kernels: each wave
// walks its rows of a GEMV as a sequence of items (SEG 16-byte chunks per
// lane of one row; both matrices for the gate/up pair) through a ring of R
// register slots, so R-1 items are in flight while one is multiplied.  Used
// by the persistent token-step kernel (step.hip) and the standalone GEMV
// (gemv.hip); 512-thread workgroups, the DOT order of dev_gemv.h.
#pragma once
#include <hip/hip_runtime.h>

#include "dev_flow.h"
#include "dev_gemv.h"
#include "kernels.h"

namespace y2 {

constexpr int kRingThreads = 512;
constexpr int kRingWaves = kRingThreads / 64;

// First row of part w of n rows split over `parts` (n * parts < 2^32).
__device__ __forceinline__ int part_lo(int n, int w, int parts) {
    return (int)((uint32_t)n * (uint32_t)w / (uint32_t)parts);
}

// ---- GEMV through a register ring ------------------------------------------

constexpr int seg_of(int it, int cap) {
    int s = cap < it ? cap : it;
    while (it % s) --s;
    return s;
}

// Item shape of a GEMV with IT chunks per lane per row.
template <int IT, bool PAIR>
struct Ring {
    static constexpr int SEG = seg_of(IT, PAIR ? 2 : 4);  // chunks per lane per item
    static constexpr int NSEG = IT / SEG;                 // items per row
    static constexpr int R = PAIR ? 4 : 5;                // ring depth (items)
    static constexpr int W = SEG * (PAIR ? 2 : 1);        // uint4 per item
    static constexpr int SIZE = R * W;                    // uint4 of the ring
};

// Items of a row: NSEG, or with MASK (k may be short of 512 IT) only those
// that hold some of the row's chunks -- the chunks of the others would all be
// masked, so skipping them changes no chain (a masked chunk adds +0).
template <int SEG, int NSEG, bool MASK>
__device__ __forceinline__ int row_items(int k) {
    if constexpr (MASK) return min(NSEG, ((k >> 3) + 64 * SEG - 1) / (64 * SEG));
    else return NSEG;
}

// The rows of this wave in [r0, r1) as items, ns per row; item q of a wave
// is segment q % ns of row r0 + wave + 8 * (q / ns).  Items past the last
// one (the ring's look-ahead at the end of a GEMV) re-read the last item,
// and a wave without rows reads row min(r0, n - 1): loads stay unconditional
// and in bounds, and the re-reads hit in L2.
__device__ __forceinline__ void item_at(int q, int Q, int r0, int n, int ns, int* row, int* seg) {
    const int wave = threadIdx.x >> 6;
    if (Q == 0) {
        *row = min(r0, n - 1);
        *seg = 0;
        return;
    }
    const int qq = min(q, Q - 1);
    *row = r0 + wave + kRingWaves * (qq / ns);
    *seg = qq % ns;
}

// MASK: k may be short of 64 * 8 * IT (the lane's chunks past the row end
// are read at chunk 0 and masked); without it k is exactly that.
template <int SEG, bool PAIR, bool MASK>
__device__ __forceinline__ void load_item(const uint16_t* w, const uint16_t* w2, int k, int row, int seg,
                                          uint4* buf) {
    const int lane = threadIdx.x & 63, nchunk = k >> 3;
    const uint4* a = reinterpret_cast<const uint4*>(w + (size_t)row * k);
#pragma unroll
    for (int it = 0; it < SEG; ++it) {
        const int c = lane + 64 * (seg * SEG + it);
        buf[it] = ldg4(a + (!MASK || c < nchunk ? c : 0));
    }
    if constexpr (PAIR) {
        const uint4* b = reinterpret_cast<const uint4*>(w2 + (size_t)row * k);
#pragma unroll
        for (int it = 0; it < SEG; ++it) {
            const int c = lane + 64 * (seg * SEG + it);
            buf[SEG + it] = ldg4(b + (!MASK || c < nchunk ? c : 0));
        }
    }
}

// Continue the DOT chains of batch rows b < B over one item (chunks of the
// lane past the row end contribute fma(0, 0, acc) = acc).
template <int B, int SEG, bool PAIR, bool MASK>
__device__ __forceinline__ void dot_item(const float* xs, int k, int seg, const uint4* wv, float* acc,
                                         float* acc2) {
    const int lane = threadIdx.x & 63, nchunk = k >> 3;
#pragma unroll
    for (int it = 0; it < SEG; ++it) {
        const int c = lane + 64 * (seg * SEG + it);
        const bool ok = !MASK || c < nchunk;
        const int cc = ok ? c : 0;
        float wf[8], wf2[8];
        unpack_bf16x8(wv[it], wf);
        if constexpr (PAIR) unpack_bf16x8(wv[SEG + it], wf2);
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
        __builtin_amdgcn_sched_barrier(0);
    }
}

// Rows of the residual stream owned by one workgroup, staged in LDS before a
// residual GEMV (a global load in the epilogue would retire behind every
// weight load in flight and drain the ring).
constexpr int kResRows = 64;

// Output value of one row (see gemv_store in dev_gemv.h); res = the row's
// current residual value (EPI_RESID).
template <int EPI>
__device__ __forceinline__ float out_value(float acc, float acc2, float res) {
    if constexpr (EPI == EPI_RAW) {
        return acc;
    } else if constexpr (EPI == EPI_STORE) {
        return rb(acc);
    } else if constexpr (EPI == EPI_RESID) {
        return rb(res + rb(acc));
    } else {
        return rb(silu_rb(rb(acc)) * rb(acc2));
    }
}

// Issue the first R-1 items of this wave's rows [r0, r1) into ring slots.
template <int IT, bool PAIR, bool MASK = false>
__device__ __forceinline__ void prefetch_ring(const uint16_t* w, const uint16_t* w2, int k, int r0, int r1,
                                              int n, uint4* ring) {
    using C = Ring<IT, PAIR>;
    const int wave = threadIdx.x >> 6, span = r1 - r0, ns = row_items<C::SEG, C::NSEG, MASK>(k);
    const int Q = (span > wave ? (span - wave + kRingWaves - 1) / kRingWaves : 0) * ns;
#pragma unroll
    for (int s = 0; s < C::R - 1; ++s) {
        int row, seg;
        item_at(s, Q, r0, n, ns, &row, &seg);
        load_item<C::SEG, PAIR, MASK>(w, w2, k, row, seg, ring + s * C::W);
    }
}

// Rows [r0, r1) of y = W xs (xs: B staged rows of k floats in LDS) with
// epilogue EPI, written as tagged words to ty (or as floats to y when ty is
// null); the ring holds the first R-1 items (prefetch_ring).  res: for
// EPI_RESID, res[b * (r1 - r0) + (row - r0)] = the row's current value (LDS).
// PACK (B == 2, the outputs BF16-exact): one packed word per row holds both
// batch rows (ty[row]); y_stride then only applies to y.  PAIRS (B == 1, the
// outputs BF16-exact, r0 and r1 even): one word holds rows 2p and 2p + 1
// (ty[p]); the rows are collected in pk (LDS, r1 - r0 floats) and stored
// after a block barrier, so every thread of the block calls this.
// (Writing the new value back to res here instead of re-reading it later
// measured slower: the GEMVs of the whole kernel lost about half their rate.)
template <int B, int EPI, int IT, bool MASK = false, bool PACK = false, bool PAIRS = false>
__device__ __forceinline__ void gemv_ring(const uint16_t* w, const uint16_t* w2, const float* xs, int k,
                                          float* y, uint64_t* ty, uint32_t tag, int y_stride, int r0, int r1,
                                          int n, uint4* ring, const float* res = nullptr, float* pk = nullptr) {
    static_assert(!PAIRS || B == 1, "row pairs with one batch row");
    constexpr bool PAIR = EPI == EPI_SWIGLU;
    using C = Ring<IT, PAIR>;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, span = r1 - r0;
    const int ns = row_items<C::SEG, C::NSEG, MASK>(k);
    const int Q = (span > wave ? (span - wave + kRingWaves - 1) / kRingWaves : 0) * ns;
    float acc[B], acc2[B];
#pragma unroll
    for (int b = 0; b < B; ++b) acc[b] = acc2[b] = 0.0f;
    for (int q0 = 0; q0 < Q; q0 += C::R) {
#pragma unroll
        for (int s = 0; s < C::R; ++s) {
            const int q = q0 + s;
            if (q >= Q) break;
            {
                // refill the slot of item q - 1 with item q + R - 1
                int row, seg;
                item_at(q + C::R - 1, Q, r0, n, ns, &row, &seg);
                load_item<C::SEG, PAIR, MASK>(w, w2, k, row, seg, ring + ((s + C::R - 1) % C::R) * C::W);
            }
            const int seg = q % ns;
            dot_item<B, C::SEG, PAIR, MASK>(xs, k, seg, ring + s * C::W, acc, acc2);
            if (seg == ns - 1) {
                const int row = r0 + wave + kRingWaves * (q / ns);
                float v[B], v2[B];
#pragma unroll
                for (int b = 0; b < B; ++b) {
                    v[b] = wave_sum_xor(acc[b]);
                    v2[b] = PAIR ? wave_sum_xor(acc2[b]) : 0.0f;
                    acc[b] = acc2[b] = 0.0f;
                }
                if (lane == 0) {
                    if (PAIRS && ty) {
                        pk[row - r0] = out_value<EPI>(v[0], v2[0], EPI == EPI_RESID ? res[row - r0] : 0.0f);
                    } else if (PACK && ty) {
                        static_assert(!PACK || B == 2, "packed words hold two batch rows");
                        float o[B];
#pragma unroll
                        for (int b = 0; b < B; ++b)
                            o[b] = out_value<EPI>(v[b], v2[b], EPI == EPI_RESID ? res[b * span + (row - r0)] : 0.0f);
                        st_tag_bits(ty + row, pack_rows(o[0], o[B - 1]), tag);
                    } else {
                        // one copy of the epilogue for the batch rows
#pragma unroll 1
                        for (int b = 0; b < B; ++b) {
                            const float rv = EPI == EPI_RESID ? res[b * span + (row - r0)] : 0.0f;
                            const float o = out_value<EPI>(b == 0 ? v[0] : v[B - 1], b == 0 ? v2[0] : v2[B - 1], rv);
                            const size_t i = (size_t)b * y_stride + row;
                            if (ty) st_tag(ty + i, o, tag);
                            else gblw(y)[i] = o;
                        }
                    }
                }
            }
        }
    }
    if constexpr (PAIRS) {
        if (ty) {
            // every wave's rows are in pk (LDS only: the ring's last loads
            // stay in flight)
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
            for (int t = threadIdx.x; t < span / 2; t += blockDim.x)
                st_tag_bits(ty + r0 / 2 + t, pack_rows(pk[2 * t], pk[2 * t + 1]), tag);
        }
    }
}

}  // namespace y2
