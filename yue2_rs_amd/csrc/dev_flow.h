// dev_flow.h -- tagged-word dataflow between the workgroups of the
// persistent token-step kernel, and the decode attention written on it.
//
// Every value that one workgroup produces for others is stored as one
// 64-bit word {tag: high 32 bits, value: low 32 bits} with a single
// agent-scope atomic store (an sc1 dwordx2 store: written through to the
// device-coherent level, and never observed half-written).  A consumer polls
// the words it needs with agent-scope atomic loads until every tag equals the
// tag it expects.  The data carries its own readiness, so there is no
// barrier, no counter and no wait for store completion between dependent
// phases: a dependency costs one store-to-load visibility.
//
// Tags: (epoch << 12) | (layer << 4) | kind, epoch = launch sequence + 1
// (20 bits).  The words of x, q/k/v, the attention output and the SwiGLU
// output are rewritten every launch; a block statistic or partial is
// rewritten only by launches whose context reaches its block, so it can keep
// an old launch's tag indefinitely.  The host therefore clears all words and
// restarts the sequence before 2^20 launches have run since the last clear
// (Workspace::reserve_launches): between two clears every launch has its own
// epoch.  The state reset bumps the sequence, so words left by an aborted
// launch can never match.  A buffer is
// rewritten only after all its readers have consumed it: every rewrite
// depends, through the step's own data dependencies, on outputs that each
// reader produced after its read (x after down needs every workgroup's
// SwiGLU output, which needs every workgroup to have read x after O, ...).
//
// All polls are bounded: on timeout (or once another workgroup has set the
// device error) the poll sets the error and returns false, and the kernel
// leaves, so every launch terminates.
#pragma once
#include <hip/hip_runtime.h>

#include "dev_attn.h"
#include "dev_gemv.h"
#include "dev_mem.h"
#include "kernels.h"
#include "y2_math.h"

namespace y2 {

enum FlowKind { FK_QKV = 1, FK_ATT = 2, FK_XO = 3, FK_ACT = 4, FK_XD = 5, FK_BMAX = 6, FK_BSUM = 7,
                FK_PART = 8, FK_SMP = 9 };
constexpr int kDevErrFlow = 8;
// Words per thread in one gather pass of the merge.
constexpr int kMergeBatch = 8;

__device__ __forceinline__ uint32_t flow_tag(uint32_t epoch, int layer, int kind) {
    return (epoch << 12) | ((uint32_t)layer << 4) | (uint32_t)kind;
}

// A word's 32 value bits hold one f32, or (a packed word) two BF16-exact
// values: batch row 0 in the low half, row 1 in the high half.
__device__ __forceinline__ void st_tag_bits(uint64_t* p, uint32_t bits, uint32_t tag) {
    const uint64_t w = ((uint64_t)tag << 32) | (uint64_t)bits;
    __hip_atomic_store(gblw(p), w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_tag(uint64_t* p, float v, uint32_t tag) { st_tag_bits(p, f2u(v), tag); }
__device__ __forceinline__ uint32_t pack_rows(float row0, float row1) {
    return (f2u(row0) >> 16) | (f2u(row1) & 0xffff0000u);
}
__device__ __forceinline__ uint64_t ld_tag(const uint64_t* p) {
    return __hip_atomic_load(gblw(const_cast<uint64_t*>(p)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// put(i, value bits of the word addr(i)), i < n, once its tag equals `tag`
// (put writes LDS).  All NT threads of the block take part; n <= NT * MAXPER.
// Returns false (device error set) on timeout; the result is uniform over the
// block.
template <int NT, int MAXPER, class Addr, class Put>
__device__ __forceinline__ bool gather_put(Addr addr, int n, uint32_t tag, Put put, StepState* st) {
    __shared__ int s_fail;
    const int tid = threadIdx.x;
    // every thread has read the previous call's flag before it is reset, and
    // the reset is visible before anyone can set it
    __syncthreads();
    if (tid == 0) s_fail = 0;
    __syncthreads();
    uint32_t pend = 0;
#pragma unroll
    for (int j = 0; j < MAXPER; ++j)
        if (tid + j * NT < n) pend |= 1u << j;
    unsigned rounds = 0;
    while (pend) {
        uint64_t w[MAXPER];
#pragma unroll
        for (int j = 0; j < MAXPER; ++j) w[j] = (pend >> j) & 1 ? ld_tag(addr(tid + j * NT)) : 0;
#pragma unroll
        for (int j = 0; j < MAXPER; ++j)
            if (((pend >> j) & 1) && (uint32_t)(w[j] >> 32) == tag) {
                put(tid + j * NT, (uint32_t)w[j]);
                pend &= ~(1u << j);
            }
        if (!pend) break;
        ++rounds;
        if ((rounds & 255) == 0 && (rounds > (1u << 20) || ld_dev_i(&st->error))) {
            set_error(&st->error, kDevErrFlow);
            s_fail = 1;  // benign race: every writer stores 1
            break;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    __syncthreads();
    return s_fail == 0;
}

// dst[i] = value of the word addr(i) (one f32 per word), i < n.
template <int NT, int MAXPER, class Addr>
__device__ __forceinline__ bool gather_at(Addr addr, int n, uint32_t tag, float* dst, StepState* st) {
    return gather_put<NT, MAXPER>(addr, n, tag, [=](int i, uint32_t bits) { dst[i] = u2f(bits); }, st);
}

// Division by a run-time d >= 1 of numerators i < 2^32 / d: floor(i / d) =
// umulhi(i, ceil(2^32 / d)) (the rounding error of the multiplier stays
// below 1/d), d = 1 passed through.  The division itself would be ~40
// instructions at every use.
struct FastDiv {
    uint32_t d, m;
    __device__ __forceinline__ explicit FastDiv(int dd) : d((uint32_t)dd), m(0xFFFFFFFFu / (uint32_t)dd + 1u) {}
    __device__ __forceinline__ int div(int i) const { return d == 1 ? i : (int)__umulhi((uint32_t)i, m); }
    __device__ __forceinline__ int mod(int i) const { return i - div(i) * (int)d; }
};

// The contiguous words src[0, n).
template <int NT, int MAXPER>
__device__ __forceinline__ bool gather_flat(const uint64_t* src, int n, uint32_t tag, float* dst, StepState* st) {
    return gather_at<NT, MAXPER>([=](int i) { return src + i; }, n, tag, dst, st);
}

// Packed words src[0, k): dst[i] = row 0's value of word i, dst[k + i] = row
// 1's.
template <int NT, int MAXPER>
__device__ __forceinline__ bool gather_pair(const uint64_t* src, int k, uint32_t tag, float* dst, StepState* st) {
    return gather_put<NT, MAXPER>([=](int i) { return src + i; }, k, tag,
                                  [=](int i, uint32_t bits) {
                                      dst[i] = bf16_lo(bits);
                                      dst[k + i] = bf16_hi(bits);
                                  },
                                  st);
}

// The 2-D region src[r * stride + c], r < n / cols, c < cols, row-major.
template <int NT, int MAXPER>
__device__ __forceinline__ bool gather(const uint64_t* src, int n, int cols, size_t stride, uint32_t tag,
                                       float* dst, StepState* st) {
    const FastDiv fc(cols);
    return gather_at<NT, MAXPER>(
        [=](int i) {
            const int r = fc.div(i);
            return src + (size_t)r * stride + (i - r * cols);
        },
        n, tag, dst, st);
}

// v[0] + v[1] + ... + v[n-1] (n >= 1) added left to right, v 16-byte
// aligned: read four values at a time, the next 16 values requested while
// the current 16 are added (at thousands of keys a workgroup adds hundreds
// of block sums or partials in sequence, and a read-then-add loop waits out
// the LDS latency every few adds).
__device__ __forceinline__ float sum_left_to_right_a16(const float* v, int n) {
    const float4* q = reinterpret_cast<const float4*>(v);
    const int nq = n >> 2;
    float s = v[0];
    if (nq > 0) {
        float4 c[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) c[j] = q[min(j, nq - 1)];
        for (int k = 0; k < nq; k += 4) {
            float4 nx[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) nx[j] = q[min(k + 4 + j, nq - 1)];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (k + j < nq) {
                    if (k + j > 0) s = s + c[j].x;
                    s = s + c[j].y;
                    s = s + c[j].z;
                    s = s + c[j].w;
                }
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) c[j] = nx[j];
        }
    }
    for (int k = max(nq * 4, 1); k < n; ++k) s = s + v[k];
    return s;
}

// Arguments of one layer's attention in the step kernel.
struct FlowAttn {
    // tagged q heads, k heads, v heads: (packed) [qkv_stride] words holding
    // both batch rows, else [qkv_stride / 2] words of one row holding
    // outputs 2p and 2p + 1
    const uint64_t* qkv;
    int qkv_stride;
    bool packed;
    uint16_t* kv_base;  // this batch row's cache: [layers][2][kv_heads][cap][dim] BF16
    int cap, pos, layer, heads, kv_heads, blk_stride, att_stride, wpg;
    float scale, eps;
    const float *q_norm, *k_norm, *cos_t, *sin_t;
    uint64_t *bmax, *bsum, *part;  // tagged [rows][heads][blk_stride] (part: x dim)
    uint64_t* att;                 // tagged [rows][att_stride / 2]: outputs 2p, 2p + 1 packed
    uint32_t epoch;
    StepState* st;
    // a launch of its own (PLAIN): q/k/v read from the f32 rows an earlier
    // launch wrote, [rows][qkv_stride], and the output stored as f32 rows
    // [rows][att_stride] (both BF16-exact), in place of qkv and att
    const float* qkv_f;
    float* out_f;
};

// K/V blocks staged in LDS at a time by the attention (64 keys each).
constexpr int kAttnChunk = 3;

// Dynamic LDS bytes attn_flow needs: staged K and V chunks, the scores of G
// heads over bpw blocks (the merge reuses the K/V region).
__host__ __device__ constexpr size_t attn_flow_lds(int G, int D, int bpw) {
    return (size_t)2 * kAttnChunk * kBlockKeys * D * sizeof(uint16_t) + (size_t)G * bpw * kBlockKeys * sizeof(float);
}

// Workgroup wi (of wpg) of group (kv head g, batch row b): the arithmetic of
// attn_group in dev_attn.h (so the same bits), with the three group
// exchanges (block maxima, block sums, partial PV) as tagged words and the
// final merge spread over the group's workgroups.  Latency is what limits a
// decode attention at a few thousand keys, so:
//  - the workgroup's first K and V blocks and the RoPE / QK-norm constants
//    are requested before it waits for its queries;
//  - K and V go through LDS (kAttnChunk blocks at a time), and the owner of
//    the newest key uses its freshly computed row from there, so the cache
//    append needs no completion wait;
//  - the scores keep each lane's query chunk in registers; PV runs one
//    (block, eighth of the dims) item per wave, for all heads.
// G = heads / kv_heads, the query heads of a group (the host checks that the
// launch's shape has this G); GRT: G is only the most a group has, its
// query heads are heads / kv_heads at run time (up to 8).  lds: attn_flow_lds(G, D,
// bpw) bytes.  false: timeout (error set).
// pre(): called once the workgroup's q/k/v are gathered (or at once when it
// has no keys): the caller's early requests for the phase after the
// attention (the O projection's first weight items at long contexts).
// PLAIN: the standalone decode attention (q/k/v and the output as plain f32
// rows, qkv_f and out_f); the block statistics and partials are exchanged
// as tagged words all the same.  HOIST: a wave takes a head's softmax
// maximum from the gathered block maxima once for its consecutive items of
// that head (long contexts, where a workgroup has many blocks per head),
// not once per item.  LATEV: the first V chunk is requested after the
// q/k/v gather instead of before it (the gather's polls retire behind every
// load issued before them, and V is not needed before the block
// statistics) and staged before the block-maximum gather.
template <int NT, int D, int G, bool GRT, bool PLAIN = false, bool HOIST = PLAIN, bool LATEV = PLAIN, class Mark,
          class Pre>
__device__ __forceinline__ bool attn_flow(const FlowAttn& a, int wi, int g, int b, float* lds, Mark&& mark,
                                          Pre&& pre) {
    constexpr int NW = NT / 64;
    constexpr int S = 512 / D;     // PV key streams per 64-key block
    constexpr int MAXNB = 24576 / kBlockKeys;
    constexpr int BLK_U4 = kBlockKeys * D / 8;           // uint4 per staged block
    constexpr int PER = (kAttnChunk * BLK_U4 + NT - 1) / NT;  // uint4 per thread per chunk
    constexpr int HALF = D / 2;
    // the scores and PV take the group's query heads HP at a time (more
    // per-head values would not fit the registers), in NP passes
    constexpr int HP = G < 4 ? G : 4, NP = (G + HP - 1) / HP;
    // the group's queries, then (owner of the new key) its key and value rows
    __shared__ __align__(16) float qkv_s[(G + 2) * D];  // read as float4 in the scores
    float(*q_s)[D] = reinterpret_cast<float(*)[D]>(qkv_s);
    __shared__ float hscale[G + 1];
    __shared__ float t_s[G];
    __shared__ __align__(16) float red_s[G * MAXNB];
    // The thread index and the group size through opaque copies: with them
    // known, the compiler hoists the attention's per-lane offsets and keeps
    // more of its per-head values live across the layer loop than the kernel
    // has registers for (it spills).
    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    const int lane = tid & 63, wave = tid >> 6;
    int Gq = GRT ? a.heads / a.kv_heads : G;
    asm volatile("" : "+s"(Gq));
    StepState* st = a.st;
    const int pos = a.pos, L = pos + 1, cap = a.cap;
    const int nb = (L + kBlockKeys - 1) / kBlockKeys;
    // whole super-blocks per workgroup (the order spec's sums, kernels.h)
    const int sb = attn_superblock(nb), lsb = sb == 1 ? 0 : sb == 2 ? 1 : 2, nsb = (nb + sb - 1) >> lsb;
    const int bpw = attn_bpw(nb, a.wpg);
    const int W = (nb + bpw - 1) / bpw;
    if (wi >= W) {
        pre();
        for (int i = 0; i < 6; ++i) mark();  // keep the trace slots aligned
        return true;
    }
    const int blk0 = wi * bpw, blk1 = min(nb, blk0 + bpw), nbl = blk1 - blk0;
    const int j0 = blk0 * kBlockKeys, j1 = min(L, blk1 * kBlockKeys), nk = j1 - j0;
    const int estride = bpw * kBlockKeys;
    const uint64_t* row = a.qkv + (a.packed ? 0 : (size_t)b * a.qkv_stride);
    uint16_t* Kc = a.kv_base + kv_off(a.layer, 0, a.kv_heads, g, cap, 0, D);
    uint16_t* Vc = a.kv_base + kv_off(a.layer, 1, a.kv_heads, g, cap, 0, D);
    const size_t hbase = ((size_t)b * a.heads + (size_t)g * Gq) * a.blk_stride;
    const bool owns_new = j1 == L;
    const uint32_t t_qkv = flow_tag(a.epoch, a.layer, FK_QKV);
    float* k_s = qkv_s + Gq * D;
    float* v_s = k_s + D;
    uint4* Ks = reinterpret_cast<uint4*>(lds);  // [kAttnChunk * 64][D / 8]
    uint4* Vs = Ks + kAttnChunk * BLK_U4;
    float* e_s = reinterpret_cast<float*>(Vs + kAttnChunk * BLK_U4);

    // staged-chunk loads: rows [c0 * 64, ...) of this workgroup's keys; rows
    // past L are not read (their slots are never used)
    auto load_chunk = [&](const uint16_t* base, int cb, uint4* r) {
        const int nrow = min(kAttnChunk * kBlockKeys, nk - cb * kBlockKeys);
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int u = tid + i * NT, key = u / (D / 8), part = u % (D / 8);
            r[i] = key < nrow ? ldg4(base + (size_t)(j0 + cb * kBlockKeys + key) * D + 8 * part)
                              : make_uint4(0, 0, 0, 0);
        }
    };
    // Unit u (16 bytes) of staged V row `key` holds unit u ^ vperm(key) of the
    // cache row, so the S streams of a PV read fall in different LDS banks (a
    // K row is read whole by 16 lanes and is staged as it is).
    auto vperm = [](int key) { return D == 128 ? 2 * (key & 3) : (key >> 1) & 3; };
    auto store_chunk = [&](uint4* dst, const uint4* r, bool isv) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int u = tid + i * NT, key = u / (D / 8), part = u % (D / 8);
            if (u < kAttnChunk * BLK_U4) dst[key * (D / 8) + (part ^ (isv ? vperm(key) : 0))] = r[i];
        }
    };
    // element d of staged row `key` (permuted as above)
    auto staged = [&](uint4* base, int key, int d, bool isv) {
        return reinterpret_cast<uint16_t*>(base + key * (D / 8) + ((d >> 3) ^ (isv ? vperm(key) : 0))) + (d & 7);
    };

    // ---- phase 0: early requests, queries, new key/value --------------------
    uint4 kr[PER], vr[PER];
    load_chunk(Kc, 0, kr);
    if constexpr (!LATEV) load_chunk(Vc, 0, vr);
    // RoPE / QK-norm constants of the (head, d) pair this thread rotates.
    // XP: more pairs than threads (eight query heads at head_dim 128): thread
    // t also rotates pair t + NT, a pair of the new key with the same d.
    constexpr bool XP = (G + 1) * HALF > NT;
    static_assert(NT % HALF == 0 && (G + 1) * HALF <= 2 * NT, "at most two pairs per thread");
    const int pairs = (Gq + (owns_new ? 1 : 0)) * HALF;
    float c_cos = 0.0f, c_sin = 0.0f, c_g0 = 0.0f, c_g1 = 0.0f, c_g0k = 0.0f, c_g1k = 0.0f;
    if (tid < pairs) {
        const int h = tid / HALF, d = tid % HALF;
        const float* gam = h < Gq ? a.q_norm : a.k_norm;
        c_g0 = gbl(gam)[d];
        c_g1 = gbl(gam)[d + HALF];
        c_cos = gbl(a.cos_t + (size_t)pos * HALF)[d];
        c_sin = gbl(a.sin_t + (size_t)pos * HALF)[d];
    }
    if constexpr (XP) {
        if (tid + NT < pairs) {
            c_g0k = gbl(a.k_norm)[tid % HALF];
            c_g1k = gbl(a.k_norm)[tid % HALF + HALF];
        }
    }
    if constexpr (PLAIN) {
        // written by an earlier launch: plain loads, no tags
        const int nq = Gq * D;
        const float* rowf = a.qkv_f + (size_t)b * a.qkv_stride;
        const float* qsrc = rowf + (size_t)(g * Gq) * D;
        const float* ksrc = rowf + (size_t)(a.heads + g) * D;
        const float* vsrc = rowf + (size_t)(a.heads + a.kv_heads + g) * D;
        const int n = nq + (owns_new ? 2 * D : 0);
        for (int i = tid; i < n; i += NT)
            qkv_s[i] = *gbl(i < nq ? qsrc + i : (i < nq + D ? ksrc + (i - nq) : vsrc + (i - nq - D)));
        __syncthreads();
    } else if (a.packed) {
        // one gather for all three: a single wait; each word holds both
        // batch rows, this row takes its half
        const int nq = Gq * D;
        const uint64_t* qsrc = row + (size_t)(g * Gq) * D;
        const uint64_t* ksrc = row + (size_t)(a.heads + g) * D;
        const uint64_t* vsrc = row + (size_t)(a.heads + a.kv_heads + g) * D;
        const int shift = b ? 0 : 16;
        if (!gather_put<NT, ((G + 2) * D + NT - 1) / NT>(
                [=](int i) { return i < nq ? qsrc + i : (i < nq + D ? ksrc + (i - nq) : vsrc + (i - nq - D)); },
                nq + (owns_new ? 2 * D : 0), t_qkv,
                [=](int i, uint32_t bits) { qkv_s[i] = u2f((bits << shift) & 0xffff0000u); }, st))
            return false;
    } else {
        // one batch row: word p holds outputs 2p and 2p + 1
        const int nq = Gq * D / 2, hd = D / 2;
        const uint64_t* qsrc = row + (size_t)(g * Gq) * hd;
        const uint64_t* ksrc = row + (size_t)(a.heads + g) * hd;
        const uint64_t* vsrc = row + (size_t)(a.heads + a.kv_heads + g) * hd;
        if (!gather_put<NT, ((G + 2) * D / 2 + NT - 1) / NT>(
                [=](int i) { return i < nq ? qsrc + i : (i < nq + hd ? ksrc + (i - nq) : vsrc + (i - nq - hd)); },
                nq + (owns_new ? D : 0), t_qkv,
                [=](int i, uint32_t bits) {
                    qkv_s[2 * i] = bf16_lo(bits);
                    qkv_s[2 * i + 1] = bf16_hi(bits);
                },
                st))
            return false;
    }
    // The RoPE / QK-norm constants, requested before the gather, are read
    // here on every path (the RoPE below reads them on some), so their loads
    // are known to be complete. Without this the compiler waits for every
    // vector load in flight (the next K chunk's) wherever it reuses their
    // registers, in the scores' inner loop among other places.
    asm volatile("" ::"v"(c_cos), "v"(c_sin), "v"(c_g0), "v"(c_g1));
    if constexpr (XP) asm volatile("" ::"v"(c_g0k), "v"(c_g1k));
    mark();
    if constexpr (LATEV) load_chunk(Vc, 0, vr);
    pre();
    // Norm::heads (src/tensor.rs:1160): the scale of the sequential sum of
    // squares per head, decided by a whole wave per head (wave Gq: the new key)
    if constexpr (G + 1 <= NW) {
        if (wave < Gq + (owns_new ? 1 : 0)) {
            const float s = norm_scale_wave(wave < Gq ? q_s[wave] : k_s, D, a.eps);
            if (lane == 0) hscale[wave] = s;
        }
    } else {
        for (int h = wave; h < Gq + (owns_new ? 1 : 0); h += NW) {
            const float s = norm_scale_wave(h < Gq ? q_s[h] : k_s, D, a.eps);
            if (lane == 0) hscale[h] = s;
        }
    }
    store_chunk(Ks, kr, false);
    if constexpr (!LATEV) store_chunk(Vs, vr, true);
    __syncthreads();
    // rotate-half RoPE (src/model.rs:151-168); the new key and value go to the
    // cache for later steps and straight into the staged chunk for this one
    if constexpr (!XP) {
        if (tid < pairs) {
            const int h = tid / HALF, d = tid % HALF;
            float* v = h < Gq ? q_s[h] : k_s;
            const float s = hscale[h];
            const float x0 = rb(rb(v[d] * s) * c_g0);
            const float x1 = rb(rb(v[d + HALF] * s) * c_g1);
            const float y0 = rb(rb(x0 * c_cos) - rb(x1 * c_sin));
            const float y1 = rb(rb(x1 * c_cos) + rb(x0 * c_sin));
            v[d] = y0;
            v[d + HALF] = y1;
            if (h == Gq) {
                gblw(Kc)[(size_t)pos * D + d] = bf16_bits(y0);
                gblw(Kc)[(size_t)pos * D + d + HALF] = bf16_bits(y1);
                if (pos - j0 < kAttnChunk * kBlockKeys) {
                    *staged(Ks, pos - j0, d, false) = bf16_bits(y0);
                    *staged(Ks, pos - j0, d + HALF, false) = bf16_bits(y1);
                }
            }
        }
    } else {
        // the same over two pairs per thread (the second one the new key's,
        // with the key's gammas); the one-pair form above is kept apart
        // because folding both into one loop changed the other kernels' code
        for (int pr = tid; pr < pairs; pr += NT) {
            const int h = pr / HALF, d = pr % HALF;
            float* v = h < Gq ? q_s[h] : k_s;
            const float s = hscale[h];
            const float x0 = rb(rb(v[d] * s) * (pr < NT ? c_g0 : c_g0k));
            const float x1 = rb(rb(v[d + HALF] * s) * (pr < NT ? c_g1 : c_g1k));
            const float y0 = rb(rb(x0 * c_cos) - rb(x1 * c_sin));
            const float y1 = rb(rb(x1 * c_cos) + rb(x0 * c_sin));
            v[d] = y0;
            v[d + HALF] = y1;
            if (h == Gq) {
                gblw(Kc)[(size_t)pos * D + d] = bf16_bits(y0);
                gblw(Kc)[(size_t)pos * D + d + HALF] = bf16_bits(y1);
                if (pos - j0 < kAttnChunk * kBlockKeys) {
                    *staged(Ks, pos - j0, d, false) = bf16_bits(y0);
                    *staged(Ks, pos - j0, d + HALF, false) = bf16_bits(y1);
                }
            }
        }
    }
    if (owns_new)
        for (int d = tid; d < D; d += NT) {
            const uint16_t bits = bf16_bits(v_s[d]);
            gblw(Vc)[(size_t)pos * D + d] = bits;
            if (!LATEV && pos - j0 < kAttnChunk * kBlockKeys) *staged(Vs, pos - j0, d, true) = bits;
        }
    __syncthreads();
    mark();

    // ---- phase 1: scaled scores and block maxima ---------------------------
    // The DOT order of a score (one fma chain per 8-dim chunk, then the xor
    // butterfly over the chunks, largest distance first), with lane c of a
    // SCPL-lane group holding chunk c and its query chunks in registers.
    // Each group takes four keys at a time; the butterfly's first two
    // distances run as a reduce-scatter (a lane adds its partner's partials
    // of the keys it keeps: the same two operands as the butterfly's add, a
    // quarter of the exchanges), so lane c ends with key 2 b1 + b2 (b1, b2
    // its bits of the two distances) and the rest of the butterfly runs on
    // that key alone.
    const uint32_t t_bmax = flow_tag(a.epoch, a.layer, FK_BMAX);
    {
        constexpr int SCPL = D / 8;          // lanes per key
        constexpr int GPW = 64 / SCPL;       // lane groups per wave
        constexpr int H1 = SCPL / 2, H2 = SCPL / 4;
        static_assert(H2 >= 2, "a butterfly distance after the reduce-scatter");
        const int c = lane % SCPL, grp = lane / SCPL;
        const bool b1 = (c & H1) != 0, b2 = (c & H2) != 0;
        // (one pass: all heads at once; kept apart from the pass form below,
        // whose code for a single pass measured slower at long contexts)
        if constexpr (NP == 1) {
            float qr[G][8];
#pragma unroll
            for (int h = 0; h < G; ++h) {
                if (GRT && h >= Gq) {
#pragma unroll
                    for (int e = 0; e < 8; ++e) qr[h][e] = 0.0f;  // (a head the group lacks: scores never stored)
                    continue;
                }
                if (h >= Gq) break;
                const float4* qp = reinterpret_cast<const float4*>(q_s[h] + 8 * c);
                const float4 q0 = qp[0], q1 = qp[1];
                qr[h][0] = q0.x; qr[h][1] = q0.y; qr[h][2] = q0.z; qr[h][3] = q0.w;
                qr[h][4] = q1.x; qr[h][5] = q1.y; qr[h][6] = q1.z; qr[h][7] = q1.w;
            }
            for (int cb = 0; cb < nbl; cb += kAttnChunk) {
                if (cb > 0) {
                    // a later chunk (long contexts), requested during the previous
                    // chunk's scores: stage it, then patch the new key
                    __syncthreads();
                    store_chunk(Ks, kr, false);
                    __syncthreads();
                    const int kp = pos - j0 - cb * kBlockKeys;
                    if (kp >= 0 && kp < kAttnChunk * kBlockKeys)
                        for (int d = tid; d < D; d += NT)
                            *staged(Ks, kp, d, false) = bf16_bits(k_s[d]);
                    __syncthreads();
                }
                // the next chunk's loads stay in flight while this one is scored
                if (cb + kAttnChunk < nbl) load_chunk(Kc, cb + kAttnChunk, kr);
                const int keys = min(kAttnChunk * kBlockKeys, nk - cb * kBlockKeys);
                for (int qd0 = wave * GPW; qd0 * 4 < keys; qd0 += NW * GPW) {
                    const int kq = 4 * (qd0 + grp);  // the group's first key within the chunk
                    float v[4][G];
                    // the four keys' rows read together (rows past the chunk's
                    // keys are read clamped and never stored)
                    uint4 k4[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) k4[r] = Ks[(size_t)min(kq + r, kAttnChunk * kBlockKeys - 1) * (D / 8) + c];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        float kf[8];
                        unpack8a(k4[r], kf);
#pragma unroll
                        for (int h = 0; h < G; ++h) {
                            float acc = 0.0f;
#pragma unroll
                            for (int e = 0; e < 8; ++e) acc = __builtin_fmaf(qr[h][e], kf[e], acc);
                            v[r][h] = acc;
                        }
                    }
                    // distance H1: keep keys 2 b1, 2 b1 + 1
                    float w[2][G];
#pragma unroll
                    for (int i = 0; i < 2; ++i)
#pragma unroll
                        for (int h = 0; h < G; ++h) {
                            const float keep = b1 ? v[2 + i][h] : v[i][h], send = b1 ? v[i][h] : v[2 + i][h];
                            w[i][h] = keep + xor_lane<H1>(send);
                        }
                    // distance H2: keep key b2 of the two
                    const int kl = kq + 2 * (b1 ? 1 : 0) + (b2 ? 1 : 0);
                    const int j = j0 + cb * kBlockKeys + kl;
#pragma unroll
                    for (int h = 0; h < G; ++h) {
                        const float keep = b2 ? w[1][h] : w[0][h], send = b2 ? w[0][h] : w[1][h];
                        const float acc = xor_sum<H2 / 2>(keep + xor_lane<H2>(send));
                        if (h < Gq && (c & (H2 - 1)) == 0 && j < j1) e_s[h * estride + (j - j0)] = acc * a.scale;
                    }
                }
            }
        } else {
            // the query chunks of heads h0 .. h0 + HP - 1
            float qr[HP][8];
            auto load_q = [&](int h0) {
#pragma unroll
                for (int h = 0; h < HP; ++h) {
                    if (GRT && h0 + h >= Gq) {
#pragma unroll
                        for (int e = 0; e < 8; ++e) qr[h][e] = 0.0f;  // (a head the group lacks: scores never stored)
                        continue;
                    }
                    if (h0 + h >= Gq) break;
                    const float4* qp = reinterpret_cast<const float4*>(q_s[h0 + h] + 8 * c);
                    const float4 q0 = qp[0], q1 = qp[1];
                    qr[h][0] = q0.x; qr[h][1] = q0.y; qr[h][2] = q0.z; qr[h][3] = q0.w;
                    qr[h][4] = q1.x; qr[h][5] = q1.y; qr[h][6] = q1.z; qr[h][7] = q1.w;
                }
            };
            for (int cb = 0; cb < nbl; cb += kAttnChunk) {
                if (cb > 0) {
                    // a later chunk (long contexts), requested during the previous
                    // chunk's scores: stage it, then patch the new key
                    __syncthreads();
                    store_chunk(Ks, kr, false);
                    __syncthreads();
                    const int kp = pos - j0 - cb * kBlockKeys;
                    if (kp >= 0 && kp < kAttnChunk * kBlockKeys)
                        for (int d = tid; d < D; d += NT)
                            *staged(Ks, kp, d, false) = bf16_bits(k_s[d]);
                    __syncthreads();
                }
                // the next chunk's loads stay in flight while this one is scored
                if (cb + kAttnChunk < nbl) load_chunk(Kc, cb + kAttnChunk, kr);
                const int keys = min(kAttnChunk * kBlockKeys, nk - cb * kBlockKeys);
#pragma unroll
                for (int pass = 0; pass < NP; ++pass) {
                    const int h0 = pass * HP;
                    if (h0 >= Gq) break;
                    load_q(h0);
                    for (int qd0 = wave * GPW; qd0 * 4 < keys; qd0 += NW * GPW) {
                        const int kq = 4 * (qd0 + grp);  // the group's first key within the chunk
                        float v[4][HP];
                        // the four keys' rows read together (rows past the chunk's
                        // keys are read clamped and never stored)
                        uint4 k4[4];
#pragma unroll
                        for (int r = 0; r < 4; ++r) k4[r] = Ks[(size_t)min(kq + r, kAttnChunk * kBlockKeys - 1) * (D / 8) + c];
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            float kf[8];
                            unpack8a(k4[r], kf);
#pragma unroll
                            for (int h = 0; h < HP; ++h) {
                                float acc = 0.0f;
#pragma unroll
                                for (int e = 0; e < 8; ++e) acc = __builtin_fmaf(qr[h][e], kf[e], acc);
                                v[r][h] = acc;
                            }
                        }
                        // distance H1: keep keys 2 b1, 2 b1 + 1
                        float w[2][HP];
#pragma unroll
                        for (int i = 0; i < 2; ++i)
#pragma unroll
                            for (int h = 0; h < HP; ++h) {
                                const float keep = b1 ? v[2 + i][h] : v[i][h], send = b1 ? v[i][h] : v[2 + i][h];
                                w[i][h] = keep + xor_lane<H1>(send);
                            }
                        // distance H2: keep key b2 of the two
                        const int kl = kq + 2 * (b1 ? 1 : 0) + (b2 ? 1 : 0);
                        const int j = j0 + cb * kBlockKeys + kl;
#pragma unroll
                        for (int h = 0; h < HP; ++h) {
                            const float keep = b2 ? w[1][h] : w[0][h], send = b2 ? w[0][h] : w[1][h];
                            const float acc = xor_sum<H2 / 2>(keep + xor_lane<H2>(send));
                            if (h0 + h < Gq && (c & (H2 - 1)) == 0 && j < j1)
                                e_s[(h0 + h) * estride + (j - j0)] = acc * a.scale;
                        }
                    }
                }
            }
        }
        __syncthreads();
        for (int i = wave; i < Gq * nbl; i += NW) {
            const int h = i / nbl, bl = i % nbl;
            const int jl = bl * kBlockKeys + lane;
            float m = jl < nk ? e_s[h * estride + jl] : -__builtin_huge_valf();
            m = xor_max<32>(m);
            if (lane == 0) st_tag(a.bmax + hbase + (size_t)h * a.blk_stride + blk0 + bl, m, t_bmax);
        }
    }
    mark();

    // ---- phase 2: M, exp(s - M) and block sums -----------------------------
    const uint32_t t_bsum = flow_tag(a.epoch, a.layer, FK_BSUM);
    {
        // (super-blocks of more than one block) the block sums, in the K
        // region: the scores are done with it and p is staged there only
        // after the super-block sums are gathered
        float* bl_s = reinterpret_cast<float*>(Ks);
        if constexpr (LATEV) {
            // the first V chunk staged, and the owner's new value row patched
            // in after a barrier (other threads stage that row)
            store_chunk(Vs, vr, true);
            if (owns_new && pos - j0 < kAttnChunk * kBlockKeys) {
                __syncthreads();
                for (int d = tid; d < D; d += NT) *staged(Vs, pos - j0, d, true) = bf16_bits(v_s[d]);
            }
        }
        if (!gather<NT, (G * MAXNB + NT - 1) / NT>(a.bmax + hbase, Gq * nb, nb, a.blk_stride, t_bmax, red_s, st))
            return false;
        mark();
        // exp(s - M) and the block sums in one pass, one (head, block) item
        // per wave; each wave takes its head's M from the gathered block
        // maxima itself, so no barrier separates the steps
        float m_head = 0.0f;  // HOIST: the maximum of head h_last
        int h_last = -1;
        for (int i = wave; i < Gq * nbl; i += NW) {
            const int h = i / nbl, bl = i % nbl;
            float m;
            if (!HOIST || h != h_last) {  // (uniform over the wave)
                m = -__builtin_huge_valf();
                for (int k = lane; k < nb; k += 64) m = fmaxf(m, red_s[h * nb + k]);
                m = xor_max<32>(m);
                if constexpr (HOIST) {
                    m_head = m;
                    h_last = h;
                }
            } else {
                m = m_head;
            }
            const int jl = bl * kBlockKeys + lane;
            float v = 0.0f;  // keys past the context add +0
            if (jl < nk) {
                v = expf_cr(e_s[h * estride + jl] - m);
                e_s[h * estride + jl] = v;
            }
            v = xor_sum<32>(v);
            if (sb == 1) {
                if (lane == 0) st_tag(a.bsum + hbase + (size_t)h * a.blk_stride + blk0 + bl, v, t_bsum);
            } else if (lane == 0) {
                bl_s[h * nbl + bl] = v;
            }
        }
        if (sb > 1) {
            // each super-block's block sums left to right
            __syncthreads();
            const int nsbl = (nbl + sb - 1) >> lsb;
            for (int i = tid; i < Gq * nsbl; i += NT) {
                const int h = i / nsbl, k = i - h * nsbl, b0 = k * sb, b1 = min(nbl, b0 + sb);
                float u = bl_s[h * nbl + b0];
                for (int j = b0 + 1; j < b1; ++j) u = u + bl_s[h * nbl + j];
                st_tag(a.bsum + hbase + (size_t)h * a.blk_stride + (blk0 >> lsb) + k, u, t_bsum);
            }
        }
    }

    // ---- phase 3: total, p = e / total, partial PV -------------------------
    const uint32_t t_part = flow_tag(a.epoch, a.layer, FK_PART);
    {
        // head h's super-block sums at red_s[h * nbp + k] (rows 16-byte aligned)
        const int nbp = (nsb + 3) & ~3;
        {
            const FastDiv fnb(nsb);
            const uint64_t* src = a.bsum + hbase;
            const size_t bstride = a.blk_stride;
            if (!gather_put<NT, (G * MAXNB + NT - 1) / NT>(
                    [=](int i) {
                        const int h = fnb.div(i);
                        return src + (size_t)h * bstride + (i - h * nsb);
                    },
                    Gq * nsb, t_bsum,
                    [=](int i, uint32_t bits) {
                        const int h = fnb.div(i);
                        red_s[h * nbp + (i - h * nsb)] = u2f(bits);
                    },
                    st))
                return false;
        }
        mark();
        // (long contexts) the second V chunk, requested only now: the two
        // statistic gathers above would have waited behind it (their polls
        // retire after every load issued before them); it lands during the
        // total, p and the first chunk's PV
        if (kAttnChunk < nbl) load_chunk(Vc, kAttnChunk, vr);
        if (tid < Gq) t_s[tid] = sum_left_to_right_a16(red_s + tid * nbp, nsb);  // super-block sums
        __syncthreads();
        // p = e / total into the K region (the scores are done with it), in
        // stream order: p_s[h * estride + bl * 64 + t * KPS + i] is p of key
        // t + S * i of block bl, so a lane reads four keys of its stream at
        // once.  Keys past the context get p = 0.
        constexpr int KPS = kBlockKeys / S;  // keys per stream
        float* p_s = reinterpret_cast<float*>(Ks);
        {
            const int span = nbl * kBlockKeys;
            const FastDiv fsp(span);
            for (int i = tid; i < Gq * span; i += NT) {
                const int h = fsp.div(i), jl = i - h * span;
                const int jj = jl & (kBlockKeys - 1);
                const float pv = jl < nk ? e_s[h * estride + jl] / t_s[h] : 0.0f;
                p_s[h * estride + (jl - jj) + (jj % S) * KPS + jj / S] = pv;
            }
        }
        __syncthreads();
        // PV: one (block, eighth of the dims) item per wave, all G heads at
        // once (V read and unpacked once for them), so a chunk's three blocks
        // are three full passes of the eight waves.  Lane (t, c): stream t
        // (keys t, t + S, ...), dimension d0 + c.  The chains are
        // branch-free: keys past the context have zero V rows (staged so) and
        // p = 0, and fma(0, 0, acc) = acc (a chain from +0 is never -0).
        constexpr int LPS = 64 / S;  // lanes per stream
        static_assert(LPS * NW == D, "one dimension per lane, the eight waves over a block's dimensions");
        const int t = lane / LPS, c = lane % LPS;
        float sacc[G];  // this wave's super-block so far: its blocks left to right
        for (int cb = 0; cb < nbl; cb += kAttnChunk) {
            if (cb > 0) {
                // requested one chunk ahead, as the keys
                __syncthreads();
                store_chunk(Vs, vr, true);
                __syncthreads();
                const int kp = pos - j0 - cb * kBlockKeys;
                if (kp >= 0 && kp < kAttnChunk * kBlockKeys)
                    for (int d = tid; d < D; d += NT) *staged(Vs, kp, d, true) = bf16_bits(v_s[d]);
                __syncthreads();
                if (cb + kAttnChunk < nbl) load_chunk(Vc, cb + kAttnChunk, vr);
            }
            const int cblocks = min(kAttnChunk, nbl - cb);
            for (int it = wave; it < cblocks * NW; it += NW) {
                const int bc = it / NW, bl = cb + bc, d = (it % NW) * LPS + c;
                // (the keys t + S i of a stream share their unit permutation)
                const uint16_t* vrow = staged(Vs, bc * kBlockKeys + t, d, true);
                const float* pp = p_s + bl * kBlockKeys + t * KPS;
                // (one pass: all heads at once; this form is kept apart from
                // the pass loop below, whose code for a single pass measured
                // 0.2-0.5 % slower)
                if constexpr (NP == 1) {
                    float acc[G];
#pragma unroll
                    for (int h = 0; h < G; ++h) acc[h] = 0.0f;
#pragma unroll
                    for (int i0 = 0; i0 < KPS; i0 += 4) {
                        // four keys' V and the G heads' p requested together
                        float vf[4];
#pragma unroll
                        for (int u = 0; u < 4; ++u) vf[u] = bf16(vrow[(size_t)S * (i0 + u) * D]);
                        float4 p4[G];
#pragma unroll
                        for (int h = 0; h < G; ++h)
                            p4[h] = !GRT || h < Gq ? *reinterpret_cast<const float4*>(pp + h * estride + i0)
                                                   : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
                        for (int u = 0; u < 4; ++u) {
#pragma unroll
                            for (int h = 0; h < G; ++h) {
                                const float pv = u == 0 ? p4[h].x : u == 1 ? p4[h].y : u == 2 ? p4[h].z : p4[h].w;
                                acc[h] = __builtin_fmaf(pv, vf[u], acc[h]);
                            }
                        }
                    }
                    // streams combined in the butterfly order (distances S/2 .. 1
                    // between streams = lane distances 32 .. LPS); every stream
                    // lane then holds the same sums and lane t stores head h when
                    // h % S == t, once its super-block is complete
                    const int bi = bl & (sb - 1);
                    const bool first = bi == 0, full = bi == sb - 1 || bl == nbl - 1;
                    const size_t pidx = (size_t)((blk0 + bl) >> lsb) * D + d;
#pragma unroll
                    for (int h = 0; h < G; ++h) {
                        const float v = xor_sum<32, LPS>(acc[h]);
                        sacc[h] = first ? v : sacc[h] + v;
                        if ((!GRT || h < Gq) && h % S == t && full)
                            st_tag(a.part + (hbase + (size_t)h * a.blk_stride) * D + pidx, sacc[h], t_part);
                    }
                } else {
#pragma unroll
                    for (int pass = 0; pass < NP; ++pass) {
                        const int h0 = pass * HP;
                        if (h0 >= Gq) break;
                        float acc[HP];
#pragma unroll
                        for (int h = 0; h < HP; ++h) acc[h] = 0.0f;
#pragma unroll
                        for (int i0 = 0; i0 < KPS; i0 += 4) {
                            // four keys' V and the heads' p requested together
                            float vf[4];
#pragma unroll
                            for (int u = 0; u < 4; ++u) vf[u] = bf16(vrow[(size_t)S * (i0 + u) * D]);
                            float4 p4[HP];
#pragma unroll
                            for (int h = 0; h < HP; ++h)
                                p4[h] = !GRT || h0 + h < Gq
                                            ? *reinterpret_cast<const float4*>(pp + (h0 + h) * estride + i0)
                                            : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
                            for (int u = 0; u < 4; ++u) {
#pragma unroll
                                for (int h = 0; h < HP; ++h) {
                                    const float pv = u == 0 ? p4[h].x : u == 1 ? p4[h].y : u == 2 ? p4[h].z : p4[h].w;
                                    acc[h] = __builtin_fmaf(pv, vf[u], acc[h]);
                                }
                            }
                        }
                        // streams combined in the butterfly order (distances S/2
                        // .. 1 between streams = lane distances 32 .. LPS); every
                        // stream lane then holds the same sums and lane t stores
                        // head h when h % S == t, once its super-block is complete
                        const int bi = bl & (sb - 1);
                        const bool first = bi == 0, full = bi == sb - 1 || bl == nbl - 1;
                        const size_t pidx = (size_t)((blk0 + bl) >> lsb) * D + d;
#pragma unroll
                        for (int h = 0; h < HP; ++h) {
                            const int hh = h0 + h;
                            const float v = xor_sum<32, LPS>(acc[h]);
                            sacc[hh] = first ? v : sacc[hh] + v;
                            if ((!GRT || hh < Gq) && hh % S == t && full)
                                st_tag(a.part + (hbase + (size_t)hh * a.blk_stride) * D + pidx, sacc[hh], t_part);
                        }
                    }
                }
            }
        }
    }
    mark();

    // ---- merge: workgroup wi adds the blocks of outputs [o0, o1) -----------
    {
        // (an even count each: outputs 2p and 2p + 1, both BF16-exact, go out
        // packed in one word, half the words the O projection gathers)
        const int outs = Gq * D, chunk = ((outs + W - 1) / W + 1) & ~1;
        const int o0 = min(outs, wi * chunk), o1 = min(outs, o0 + chunk), no = o1 - o0;
        __syncthreads();  // the K/V region is reused below
        const int nbp = (nsb + 3) & ~3;
        float* m_buf = lds;  // [no][nbp]: partial of super-block k for output o0 + i (rows 16-byte aligned)
        const uint64_t* part = a.part + hbase * D;
        const size_t hstride = (size_t)a.blk_stride * D;
        const FastDiv fno(max(no, 1));
        // in passes of at most kMergeBatch words per thread: one pass at
        // short contexts, and the unrolled poll stays small; word i of the
        // sequence is output o0 + i % no of super-block i / no, so
        // neighbouring threads read neighbouring words of one partial
        for (int p0 = 0; p0 < no * nsb; p0 += NT * kMergeBatch) {
            if (!gather_put<NT, kMergeBatch>(
                    [=](int i) {
                        i += p0;
                        const int k = fno.div(i), o = o0 + i - k * no;
                        return part + (size_t)(o / D) * hstride + (size_t)k * D + o % D;
                    },
                    min(no * nsb - p0, NT * kMergeBatch), t_part,
                    [=](int i, uint32_t bits) {
                        i += p0;
                        const int k = fno.div(i);
                        m_buf[(i - k * no) * nbp + k] = u2f(bits);
                    },
                    st))
                return false;
        }
        if constexpr (PLAIN) {
            float* out = a.out_f + (size_t)b * a.att_stride + (size_t)g * Gq * D + o0;
            for (int i = tid; i < no; i += NT) out[i] = rb(sum_left_to_right_a16(m_buf + i * nbp, nsb));
            return true;
        }
        const uint32_t t_att = flow_tag(a.epoch, a.layer, FK_ATT);
        for (int i0 = 0; i0 < no; i0 += NT) {
            const int i = i0 + tid;
            const float o = i < no ? rb(sum_left_to_right_a16(m_buf + i * nbp, nsb)) : 0.0f;  // super-blocks left to right
            const float o_next = xor_lane<1>(o);  // output i + 1 (the odd neighbour lane's)
            if (i < no && (tid & 1) == 0)
                st_tag_bits(a.att + ((size_t)b * a.att_stride + (size_t)g * Gq * D + o0 + i) / 2, pack_rows(o, o_next),
                            t_att);
        }
    }
    return true;
}

}  // namespace y2
