// prefill.hip -- Model::prefill_phase (src/model.rs:508-522) on the matrix
// cores: the prompt runs through every layer as chunks of rows, each linear
// a BF16 MFMA GEMM with FP32 accumulation, the attention a causal
// flash-attention over the BF16 cache.
//
// The reference runs its prefill the same way on its GPU path: multi-row
// linears go to a GEMM (MPS, src/tensor.rs:991-993, src/metal.m:216-237) and
// the causal attention to batched matrix products (src/metal.m:330-361),
// whose summation order differs from the decode GEMV.  So this prefill
// keeps every BF16 rounding point of the decode step (rb after each linear,
// the norms, RoPE, SwiGLU, residuals; the RMSNorm scale from the sequential
// sum of squares) but not the decode path's reduction order: its results
// agree with the decode-order prefill within a stated tolerance, not bit
// for bit.  yue2_hip_prefill keeps the bit-exact decode-order prefill.
//
// Per chunk of R rows at positions [p0, p0 + R) and per layer: RMSNorm rows
// -> QKV GEMM (rb) -> QK-norm + RoPE + K/V append -> flash attention (rb)
// -> O GEMM + residual -> RMSNorm rows -> gate/up GEMM + SwiGLU -> down GEMM
// + residual.  The final norm and LM head run for the last prompt row only.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <mutex>
#include <vector>

#include "../../include/yue2_hip.h"
#include "dev_gemv.h"
#include "dev_mem.h"
#include "dev_mfma.h"
#include "kernels.h"
#include "prefill.h"
#include "runtime.h"
#include "y2_math.h"

using namespace y2;

namespace y2 {

// ---- GEMM: C = X W^T, X [M, K] BF16, W [N, K] BF16, FP32 accumulation ------
//
// A workgroup computes a TM-row tile of C against a tile of TW rows of W: TW
// output columns, or for the gate/up pair TW/2 columns whose W tile holds
// TW/2 gate rows and the same TW/2 up rows.  Its waves form a WVM x WVN grid,
// each an (TM/WVM) x (TW/WVN) block of 32x32x16 MFMA accumulators (the pair:
// the gate blocks of its columns, then the up blocks).
//
// The X and W tiles of each 64-wide step of K go from global memory straight
// into LDS (global_load_lds_dwordx4: each lane's 16 bytes land at the wave's
// LDS address + 16 * lane, with no registers and no LDS store instructions)
// through NST buffers, so NST - 1 steps are in flight while one is
// multiplied.  Tile rows are 128 bytes of eight 16-byte units, chunk c of
// row r stored at unit c ^ ((r >> 1) & 7): a 16-byte LDS read serves sixteen
// lanes per cycle from 64 four-byte banks, and its lanes 0-15 read one chunk
// of sixteen consecutive rows, which then fall in sixteen different 16-byte
// bank groups (r & 1 picks the half of the 256 bytes, the XOR the group).  The waits are explicit: after a step's MFMA operands are all
// read, the wave waits until its own loads of the next step have landed
// (vmcnt counts the DMA loads; the later steps' stay in flight), one barrier
// makes every wave's part visible and frees the buffer just read, which
// then takes step t + NST.  The next 16-wide substep's operands are read
// between the current substep's MFMAs.
template <int TM_, int TW_, int WVM_, int WVN_, int NST_>
struct GemmTile {
    static constexpr int TM = TM_, TW = TW_, WVM = WVM_, WVN = WVN_, NST = NST_;
    static constexpr int THREADS = 64 * WVM * WVN;
    static constexpr int WM = TM / WVM, WN = TW / WVN;   // wave block
    static constexpr int MI = WM / 32, NJ = WN / 32;     // 32x32 accumulators per wave
    static constexpr int XU = TM * kGemmTK / 8;          // 16-byte units of the X tile
    static constexpr int WU = TW * kGemmTK / 8;          // of the W tile
    static constexpr int SU = XU + WU;                   // per buffer
    static constexpr int LX = XU / THREADS, LW = WU / THREADS;  // DMA loads per lane per step
    static constexpr size_t LDS = (size_t)NST * SU * 16;
    static_assert(XU % THREADS == 0 && WU % THREADS == 0, "whole DMA loads per wave");
    static_assert(WM % 32 == 0 && WN % 64 == 0, "the pair needs gate and up blocks in every wave");
    static_assert(NST >= 2 && (NST - 1) * (LX + LW) < 64, "vmcnt range");
};
// 256 x 256 with 8 waves of 64 x 128 (two per SIMD); 128 x 256 with 8 waves
// of 64 x 64 and three buffers for grids the larger tile would leave short of
// workgroups.  (Measured on the 3B shapes with random operands against
// 128 x 64 and 64 x 64 wave blocks, four-wave tiles and 32-wide K steps.)
using GemmBig = GemmTile<256, 256, 4, 2, 2>;
using GemmNarrow = GemmTile<128, 256, 2, 4, 3>;

__device__ __forceinline__ int gemm_swz(int row) { return (row >> 1) & 7; }
__device__ __forceinline__ int gemm_unit(int row, int c) { return row * 8 + (c ^ gemm_swz(row)); }

typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) const y2_u32x4 lds_u32x4;

__device__ __forceinline__ f32x16 mfma32v(y2_u32x4 a, y2_u32x4 b, f32x16 c) {
    bf16x8 x, y;
    __builtin_memcpy(&x, &a, 16);
    __builtin_memcpy(&y, &b, 16);
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(x, y, c, 0, 0, 0);
}

template <int EPI, class T>
__global__ __launch_bounds__(T::THREADS, 1) void gemm_kernel(const GemmArgs g) {
    constexpr bool PAIR = EPI == GEPI_SWIGLU_BF16;
    constexpr int TN = PAIR ? T::TW / 2 : T::TW;  // output columns per tile
    extern __shared__ __align__(16) uint16_t gsm[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / T::WVN, wn = wave % T::WVN;
    const int m0 = blockIdx.y * T::TM, n0 = blockIdx.x * TN;
    const int steps = g.K / kGemmTK;
    // this lane's source of each of its DMA units (rows past the matrix read
    // its last row: they only feed outputs that are not stored)
    const uint16_t* sx[T::LX];
    const uint16_t* sw[T::LW];
#pragma unroll
    for (int j = 0; j < T::LX; ++j) {
        const int u = (wave * T::LX + j) * 64 + lane, row = u >> 3, c = (u & 7) ^ gemm_swz(row);
        sx[j] = g.x + (size_t)min(m0 + row, g.M - 1) * g.ldx + 8 * c;
    }
#pragma unroll
    for (int j = 0; j < T::LW; ++j) {
        const int u = (wave * T::LW + j) * 64 + lane, row = u >> 3, c = (u & 7) ^ gemm_swz(row);
        const uint16_t* w = g.w;
        int r = row;
        if (PAIR && row >= T::TW / 2) {
            w = g.w2;
            r = row - T::TW / 2;
        }
        sw[j] = w + (size_t)min(n0 + r, g.N - 1) * g.ldw + 8 * c;
    }
    auto issue = [&](int step, int buf) {
        const int k0 = step * kGemmTK;
        uint16_t* base = gsm + (size_t)buf * T::SU * 8;
#pragma unroll
        for (int j = 0; j < T::LX; ++j)
            __builtin_amdgcn_global_load_lds((Y2_GLOBAL void*)(sx[j] + k0),
                                             (lds_void*)(base + (wave * T::LX + j) * 64 * 8), 16, 0, 0);
#pragma unroll
        for (int j = 0; j < T::LW; ++j)
            __builtin_amdgcn_global_load_lds((Y2_GLOBAL void*)(sw[j] + k0),
                                             (lds_void*)(base + (T::XU + (wave * T::LW + j) * 64) * 8), 16, 0, 0);
    };
    // W tile row of accumulator column block j of this wave
    auto wrow = [&](int j) {
        if constexpr (PAIR)
            return (j < T::NJ / 2 ? 0 : T::TW / 2) + wn * (T::WN / 2) + 32 * (j % (T::NJ / 2));
        else
            return wn * T::WN + 32 * j;
    };
    // (explicit LDS reads of a native vector type: through generic pointers
    // the compiler waits for every DMA load in flight before each read)
    auto operands = [&](const uint16_t* base, int sub, y2_u32x4* a, y2_u32x4* b) {
        const int c = sub * 2 + (lane >> 5);
#pragma unroll
        for (int i = 0; i < T::MI; ++i) {
            const int row = wm * T::WM + i * 32 + (lane & 31);
            a[i] = *(lds_u32x4*)(base + gemm_unit(row, c) * 8);
        }
#pragma unroll
        for (int j = 0; j < T::NJ; ++j) {
            const int row = wrow(j) + (lane & 31);
            b[j] = *(lds_u32x4*)(base + (T::XU + gemm_unit(row, c)) * 8);
        }
    };
    auto buffer = [&](int t) { return gsm + (size_t)(t % T::NST) * T::SU * 8; };

    f32x16 acc[T::MI][T::NJ];
#pragma unroll
    for (int i = 0; i < T::MI; ++i)
#pragma unroll
        for (int j = 0; j < T::NJ; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
    const int pre = min(steps, T::NST);
    for (int t = 0; t < pre; ++t) issue(t, t);
    if (pre == T::NST) asm volatile("s_waitcnt vmcnt(%0)" ::"n"((T::NST - 1) * (T::LX + T::LW)) : "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    asm volatile("s_barrier" ::: "memory");
    y2_u32x4 fa[2][T::MI], fb[2][T::NJ];
    operands(buffer(0), 0, fa[0], fb[0]);
    for (int t = 0; t < steps; ++t) {
        const uint16_t* cur = buffer(t);
#pragma unroll
        for (int sub = 0; sub < kGemmTK / 16; ++sub) {
            const int f = sub & 1;
            if (sub + 1 < kGemmTK / 16) {
                operands(cur, sub + 1, fa[f ^ 1], fb[f ^ 1]);
            } else if (t + 1 < steps) {
                // every operand of step t is in registers (lgkmcnt) and this
                // wave's loads of step t + 1 have landed (later steps' stay
                // in flight); after the barrier every wave's have, and the
                // buffer of step t takes step t + NST
                if (t + T::NST - 1 < steps)
                    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"((T::NST - 2) * (T::LX + T::LW)) : "memory");
                else
                    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
                asm volatile("s_barrier" ::: "memory");
                if (t + T::NST < steps) issue(t + T::NST, t % T::NST);
                operands(buffer(t + 1), 0, fa[f ^ 1], fb[f ^ 1]);
            }
#pragma unroll
            for (int i = 0; i < T::MI; ++i)
#pragma unroll
                for (int j = 0; j < T::NJ; ++j) acc[i][j] = mfma32v(fa[f][i], fb[f][j], acc[i][j]);
            // the next substep's operand reads between these MFMAs
#pragma unroll
            for (int q = 0; q < T::MI + T::NJ; ++q) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, T::MI * T::NJ - (T::MI + T::NJ), 0);
        }
    }
    // epilogue: lane l holds column acc32_col(l) of rows acc32_row(l, r)
#pragma unroll
    for (int i = 0; i < T::MI; ++i) {
        const int rbase = m0 + wm * T::WM + i * 32;
        if constexpr (PAIR) {
#pragma unroll
            for (int j = 0; j < T::NJ / 2; ++j) {
                const int col = n0 + wn * (T::WN / 2) + 32 * j + acc32_col(lane);
                if (col >= g.N) continue;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int row = rbase + acc32_row(lane, r);
                    if (row >= g.M) continue;
                    const float o = rb(silu_rb(rb(acc[i][j][r])) * rb(acc[i][j + T::NJ / 2][r]));
                    g.cb[(size_t)row * g.ldc + col] = bf16_bits(o);
                }
            }
        } else {
#pragma unroll
            for (int j = 0; j < T::NJ; ++j) {
                const int col = n0 + wn * T::WN + 32 * j + acc32_col(lane);
                if (col >= g.N) continue;
                // the residual values of the block are all requested before
                // the first is used
                float cur[16];
                if constexpr (EPI == GEPI_RESID) {
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int row = min(rbase + acc32_row(lane, r), g.M - 1);
                        cur[r] = g.c[(size_t)row * g.ldc + col];
                    }
                }
                const float bias = EPI == GEPI_BIAS || EPI == GEPI_BIAS_SILU_BF16 ? g.bias[col] : 0.0f;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int row = rbase + acc32_row(lane, r);
                    if (row >= g.M) continue;
                    const size_t at = (size_t)row * g.ldc + col;
                    const float v = acc[i][j][r];
                    if constexpr (EPI == GEPI_RAW) g.c[at] = v;
                    else if constexpr (EPI == GEPI_ROUND) g.c[at] = rb(v);
                    else if constexpr (EPI == GEPI_RESID) g.c[at] = rb(cur[r] + rb(v));
                    else if constexpr (EPI == GEPI_BIAS) g.c[at] = rb(v + bias);
                    else g.cb[at] = bf16_bits(silu_rb(rb(v + bias)));
                }
            }
        }
    }
}

template <int EPI, class T>
static hipError_t launch_gemm_t(hipStream_t s, const GemmArgs& g) {
    // more than the default 64 KiB of dynamic LDS: allowed once per kernel
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_kernel<EPI, T>),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)T::LDS);
    if (attr != hipSuccess) return attr;
    const int tn = EPI == GEPI_SWIGLU_BF16 ? T::TW / 2 : T::TW;
    const dim3 grid((g.N + tn - 1) / tn, (g.M + T::TM - 1) / T::TM);
    gemm_kernel<EPI, T><<<grid, T::THREADS, T::LDS, s>>>(g);
    return hipGetLastError();
}

template <int EPI>
static hipError_t launch_gemm_e(hipStream_t s, const GemmArgs& g) {
    // the 256 x 256 tile unless its grid would fill fewer than half the CUs
    static const int cus = [] {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 1)
            n = 256;
        return n;
    }();
    const int tn = EPI == GEPI_SWIGLU_BF16 ? GemmBig::TW / 2 : GemmBig::TW;
    const long tiles = (long)((g.N + tn - 1) / tn) * ((g.M + GemmBig::TM - 1) / GemmBig::TM);
    return 2 * tiles >= cus ? launch_gemm_t<EPI, GemmBig>(s, g) : launch_gemm_t<EPI, GemmNarrow>(s, g);
}

hipError_t launch_gemm(hipStream_t s, int epi, const GemmArgs& g) {
    if (g.K % kGemmTK || g.ldx % 8 || g.ldw % 8 || g.M < 1 || g.N < 1) return hipErrorInvalidValue;
    // the tile loads move 16-byte units
    if (((uintptr_t)g.x | (uintptr_t)g.w | (uintptr_t)g.w2) & 15) return hipErrorInvalidValue;
    if ((epi == GEPI_BIAS || epi == GEPI_BIAS_SILU_BF16) && !g.bias) return hipErrorInvalidValue;
    if (epi == GEPI_SWIGLU_BF16 && !g.w2) return hipErrorInvalidValue;
    switch (epi) {
        case GEPI_RAW: return launch_gemm_e<GEPI_RAW>(s, g);
        case GEPI_ROUND: return launch_gemm_e<GEPI_ROUND>(s, g);
        case GEPI_RESID: return launch_gemm_e<GEPI_RESID>(s, g);
        case GEPI_SWIGLU_BF16: return launch_gemm_e<GEPI_SWIGLU_BF16>(s, g);
        case GEPI_BIAS: return launch_gemm_e<GEPI_BIAS>(s, g);
        case GEPI_BIAS_SILU_BF16: return launch_gemm_e<GEPI_BIAS_SILU_BF16>(s, g);
        default: return hipErrorInvalidValue;
    }
}

// ---- rows ----------------------------------------------------------------

constexpr int kRowThreads = 256;

// x[r] = rb(E[ids[r]]) (src/model.rs:452-464).
__global__ __launch_bounds__(kRowThreads) void embed_rows_kernel(const uint16_t* embed, const int32_t* ids, float* x,
                                                                 int H) {
    const int r = blockIdx.x;
    const uint16_t* e = embed + (size_t)ids[r] * H;
    for (int i = threadIdx.x; i < H; i += kRowThreads) x[(size_t)r * H + i] = bf16(e[i]);
}

// out[r] = RMSNorm(x[r]) as BF16 (Norm::apply, src/tensor.rs:1140-1157): the
// scale decided as the decode step decides it (the sequential f32 sum of
// squares, dev_gemv.h), one workgroup per row.
__global__ __launch_bounds__(kRowThreads) void norm_rows_kernel(const float* x, const float* gamma, uint16_t* out,
                                                                int H, float eps) {
    extern __shared__ __align__(16) float xs[];
    const int r = blockIdx.x;
    for (int i = threadIdx.x; i < H; i += kRowThreads) xs[i] = x[(size_t)r * H + i];
    __syncthreads();
    float s[1];
    norm_scales_block<kRowThreads, 1>(xs, H, eps, nullptr, s);
    for (int i = threadIdx.x; i < H; i += kRowThreads) out[(size_t)r * H + i] = bf16_bits(rb(rb(xs[i] * s[0]) * gamma[i]));
}

// Per (row r, head): the per-head RMSNorm of q and k (Norm::heads,
// src/tensor.rs:1158-1172) and rotate-half RoPE at position p0 + r
// (src/model.rs:151-168): q heads into q, k heads to their slot, and the v
// heads copied to theirs.  One wave per head.
__global__ __launch_bounds__(64) void rope_append_kernel(const RopeArgs a) {
    const int r = blockIdx.x, h = blockIdx.y, lane = threadIdx.x, D = a.D, half = D / 2;
    const int qkvw = (a.heads + 2 * a.kv_heads) * D;
    const float* v = a.qkv + (size_t)r * qkvw + (size_t)h * D;
    const int pos = a.p0 + r;
    uint16_t* kvb = a.kv_out ? a.kv_out : a.kv_base;
    const int slot = a.kv_out ? a.slot0 + r : pos, cap = a.kv_out ? a.cap_out : a.cap;
    if (h >= a.heads + a.kv_heads) {  // a value head: to its slot as is
        const int g = h - a.heads - a.kv_heads;
        uint16_t* dst = kvb + ((((size_t)a.layer * 2 + 1) * a.kv_heads + g) * cap + slot) * D;
        for (int d = lane; d < D; d += 64) dst[d] = bf16_bits(v[d]);
        return;
    }
    const bool is_q = h < a.heads;
    const float* gam = is_q ? a.q_norm : a.k_norm;
    const float s = norm_scale_wave(v, D, a.eps);
    const float* ct = a.cos_t + (size_t)pos * half;
    const float* st = a.sin_t + (size_t)pos * half;
    uint16_t* dst = is_q ? a.q + ((size_t)r * a.heads + h) * D
                         : kvb + ((((size_t)a.layer * 2) * a.kv_heads + (h - a.heads)) * cap + slot) * D;
    for (int d = lane; d < half; d += 64) {
        const float x0 = rb(rb(v[d] * s) * gam[d]);
        const float x1 = rb(rb(v[d + half] * s) * gam[d + half]);
        const float c = ct[d], sn = st[d];
        dst[d] = bf16_bits(rb(rb(x0 * c) - rb(x1 * sn)));
        dst[d + half] = bf16_bits(rb(rb(x1 * c) + rb(x0 * sn)));
    }
}

// ---- causal flash attention over the BF16 cache --------------------------

// One workgroup per (query head h, kFlashRows = 128 query rows); wave w
// takes 16 of them.  Keys in tiles of 64.  The scores are computed
// transposed, S^T = K Q^T on 16x16x32 MFMAs (K staged in LDS is the A
// operand, the wave's 16 query rows the B operand), so lane l holds query
// l % 16 and keys 16 kt + 4 (l / 16) + r of the tile: a query's online
// softmax is one lane's 16 values and two exchanges (lane distances 32, 16).
// P then feeds O^T += V^T P^T from registers: in the MFMA's K dimension,
// lane group j = l / 16 supplies the keys it holds (32 c + 4 j .. + 3 and
// 32 c + 16 + 4 j .. + 3 of each 32-key chunk c), and V^T's A fragment reads
// the same keys with two 8-byte LDS loads.  The next tile's K and V are
// requested into registers while the current one is computed.  V^T is
// written as dwords (two keys per thread), 32 consecutive keys of one dim
// row per 32 lanes, so the transposing stores do not conflict on LDS banks;
// its rows are 34 dwords apart, so 16 lanes' 8-byte reads of 16 rows do not
// either.  (Workgroups that cover all query heads of a KV head, each staged
// K/V tile serving two or three heads, measured slower: their waves need
// ~234 registers, so fewer of them fit.)
constexpr int kFlashRows = 128, kFlashThreads = 512, kFlashKT = 64;
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));

template <int D>
__global__ __launch_bounds__(kFlashThreads, 2) void flash_prefill_kernel(const FlashArgs f) {
    constexpr int KT = kFlashKT, PADK = 8, PADV = 4;
    constexpr int KN = KT * D / 8, VN = (KT / 2) * (D / 8);  // K uint4 and V key-pair units per tile
    constexpr int KU = (KN + kFlashThreads - 1) / kFlashThreads, VU = (VN + kFlashThreads - 1) / kFlashThreads;
    __shared__ __align__(16) uint16_t ks[KT][D + PADK];  // K tile, row = key
    __shared__ __align__(16) uint16_t vt[D][KT + PADV];  // V tile transposed, row = dim
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, j = lane >> 4, qi = lane & 15;
    // (the last query blocks, which attend the most keys, are dispatched first)
    const int h = blockIdx.x, q0 = (gridDim.y - 1 - blockIdx.y) * kFlashRows, G = f.heads / f.kv_heads, g = h / G;
    const int qrow = q0 + wave * 16 + qi;  // this lane's query row
    const uint16_t* Kc = f.kv_base + (((size_t)f.layer * 2) * f.kv_heads + g) * (size_t)f.cap * D;
    const uint16_t* Vc = f.kv_base + (((size_t)f.layer * 2 + 1) * f.kv_heads + g) * (size_t)f.cap * D;
    // the second key source (non-causal): keys from split on
    const uint16_t* K2 = f.kv2 ? f.kv2 + (((size_t)f.layer * 2) * f.kv_heads + g) * (size_t)f.cap2 * D : Kc;
    const uint16_t* V2 = f.kv2 ? f.kv2 + (((size_t)f.layer * 2 + 1) * f.kv_heads + g) * (size_t)f.cap2 * D : Vc;
    const int split = f.kv2 ? f.split : 0x7fffffff;
    uint4 qa[D / 32];
#pragma unroll
    for (int dk = 0; dk < D / 32; ++dk)
        qa[dk] = qrow < f.rows ? ldg4(f.q + ((size_t)qrow * f.heads + h) * D + dk * 32 + 8 * j)
                               : make_uint4(0, 0, 0, 0);
    // the last key this lane's query sees (non-causal: every key), and the
    // smallest such position in the wave
    const int all_keys = f.noncausal ? f.split + f.rows - 1 : 0;
    const int qpos = f.noncausal ? all_keys : f.p0 + qrow;
    const int wave_first = f.noncausal ? all_keys : f.p0 + q0 + wave * 16;
    const float scale2 = f.scale * 1.4426950408889634f;  // log2(e)
    float m = -__builtin_huge_valf(), l = 0.0f;
    f32x4 o[D / 16];  // O^T: register r of tile dt is dim 16 dt + 4 j + r of this lane's query
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt)
#pragma unroll
        for (int r = 0; r < 4; ++r) o[dt][r] = 0.0f;
    const int last_key = f.noncausal ? all_keys : min(f.p0 + q0 + kFlashRows - 1, f.p0 + f.rows - 1);  // keys [0, last_key]
    const int tiles = last_key / KT + 1;
    // tile loads: K as uint4 of rows (key u / (D/8), dims 8 (u % (D/8)));
    // V as key pairs (keys 2 (v % 32) and + 1, dims 8 (v / 32)); keys past
    // last_key are zero
    uint4 kr[KU], vr[VU][2];
    auto load_tile = [&](int t) {
        const int kb = t * KT;
#pragma unroll
        for (int i = 0; i < KU; ++i) {
            const int u = tid + i * kFlashThreads, kg = kb + u / (D / 8);
            const uint16_t* kp = kg < split ? Kc + (size_t)kg * D : K2 + (size_t)(kg - split) * D;
            kr[i] = u < KN && kg <= last_key ? ldg4(kp + (u % (D / 8)) * 8) : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < VU; ++i) {
            const int v = tid + i * kFlashThreads, kg = kb + 2 * (v % (KT / 2)), d8 = (v / (KT / 2)) * 8;
            const bool in = v < VN;
            const uint16_t* v0 = kg < split ? Vc + (size_t)kg * D : V2 + (size_t)(kg - split) * D;
            const uint16_t* v1 = kg + 1 < split ? Vc + (size_t)(kg + 1) * D : V2 + (size_t)(kg + 1 - split) * D;
            vr[i][0] = in && kg <= last_key ? ldg4(v0 + d8) : make_uint4(0, 0, 0, 0);
            vr[i][1] = in && kg + 1 <= last_key ? ldg4(v1 + d8) : make_uint4(0, 0, 0, 0);
        }
    };
    load_tile(0);
    for (int t = 0; t < tiles; ++t) {
        const int kb = t * KT;
        // stage this tile (its loads were issued a tile ago), request the next
#pragma unroll
        for (int i = 0; i < KU; ++i) {
            const int u = tid + i * kFlashThreads;
            if (u < KN) *reinterpret_cast<uint4*>(&ks[u / (D / 8)][(u % (D / 8)) * 8]) = kr[i];
        }
#pragma unroll
        for (int i = 0; i < VU; ++i) {
            const int v = tid + i * kFlashThreads, kp = 2 * (v % (KT / 2)), d8 = (v / (KT / 2)) * 8;
            if (v >= VN) continue;
            const uint32_t* a0 = reinterpret_cast<const uint32_t*>(&vr[i][0]);
            const uint32_t* a1 = reinterpret_cast<const uint32_t*>(&vr[i][1]);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                // dims d8 + 2e (low halves) and d8 + 2e + 1 (high halves) of keys kp, kp + 1
                *reinterpret_cast<uint32_t*>(&vt[d8 + 2 * e][kp]) = (a0[e] & 0xffffu) | (a1[e] << 16);
                *reinterpret_cast<uint32_t*>(&vt[d8 + 2 * e + 1][kp]) = (a0[e] >> 16) | (a1[e] & 0xffff0000u);
            }
        }
        __syncthreads();
        if (t + 1 < tiles) load_tile(t + 1);
        // S^T for 64 keys x the wave's 16 queries: four 16x16 tiles;
        // s[kt][r] = score of key kb + 16 kt + 4 j + r for query qrow
        f32x4 s[4];
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
            f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int dk = 0; dk < D / 32; ++dk) {
                const uint4 a = *reinterpret_cast<const uint4*>(&ks[kt * 16 + qi][dk * 32 + 8 * j]);
                acc = mfma16(a, qa[dk], acc);
            }
            s[kt] = acc;
        }
        // causal mask (tiles that reach past the wave's first query), online
        // softmax in log2 units (exp2 is the hardware exponential): the
        // maximum of the raw scores times the positive scale is the scaled
        // maximum, and each exponent is one fma, exp2(s scale2 - M)
        const bool masked = kb + KT - 1 > wave_first;
        float mx = -__builtin_huge_valf();
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float v = s[kt][r];
                if (masked && kb + kt * 16 + 4 * j + r > qpos) v = -__builtin_huge_valf();
                s[kt][r] = v;
                mx = fmaxf(mx, v);
            }
        mx = xor_max<32, 16>(mx) * scale2;
        const float mn = fmaxf(m, mx);
        const float alpha = mn == -__builtin_huge_valf() ? 1.0f : __builtin_amdgcn_exp2f(m - mn);
        float sum = 0.0f;
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float p =
                    mn == -__builtin_huge_valf() ? 0.0f : __builtin_amdgcn_exp2f(__builtin_fmaf(s[kt][r], scale2, -mn));
                s[kt][r] = p;
                sum += p;
            }
        sum = xor_sum<32, 16>(sum);
        l = l * alpha + sum;
        m = mn;
        if (__builtin_amdgcn_ballot_w64(alpha != 1.0f))  // some row's maximum moved
#pragma unroll
            for (int dt = 0; dt < D / 16; ++dt)
#pragma unroll
                for (int r = 0; r < 4; ++r) o[dt][r] *= alpha;
        // O^T += V^T P^T per 32-key chunk.  P enters in two BF16 parts, hi =
        // bf16(p) and lo = bf16(p - hi): V is BF16 (the cache), so P V takes
        // two MFMAs and keeps about 16 bits of P instead of 8, as the
        // reference's f32 softmax and P V do (src/model.rs:313-397).
        // Element 2w (+1) of chunk c: key 32c + 4j + 2w (+1) for w < 2,
        // 32c + 16 + 4j + 2w - 4 (+1) after.
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            uint32_t hw[4], lw[4];
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                // two values per conversion (v_cvt_pk_bf16_f32, round to nearest even)
                const f32x2 pv = {s[2 * c + (w >> 1)][2 * (w & 1)], s[2 * c + (w >> 1)][2 * (w & 1) + 1]};
                hw[w] = __builtin_bit_cast(uint32_t, __builtin_convertvector(pv, bf16x2v));
                const f32x2 lv = {pv[0] - u2f(hw[w] << 16), pv[1] - u2f(hw[w] & 0xffff0000u)};
                lw[w] = __builtin_bit_cast(uint32_t, __builtin_convertvector(lv, bf16x2v));
            }
            const uint4 ph = make_uint4(hw[0], hw[1], hw[2], hw[3]), pl = make_uint4(lw[0], lw[1], lw[2], lw[3]);
#pragma unroll
            for (int dt = 0; dt < D / 16; ++dt) {
                const uint16_t* vrow = &vt[dt * 16 + qi][32 * c + 4 * j];
                const uint2 v0 = *reinterpret_cast<const uint2*>(vrow);
                const uint2 v1 = *reinterpret_cast<const uint2*>(vrow + 16);
                const uint4 a = make_uint4(v0.x, v0.y, v1.x, v1.y);
                o[dt] = mfma16(a, pl, o[dt]);
                o[dt] = mfma16(a, ph, o[dt]);
            }
        }
        __syncthreads();  // every wave is done with this tile's K and V
    }
    if (qrow < f.rows) {
        const float inv = 1.0f / l;
        uint16_t* orow = f.out + (size_t)qrow * f.heads * D + (size_t)h * D + 4 * j;
#pragma unroll
        for (int dt = 0; dt < D / 16; ++dt) {
            const uint32_t w0 = (uint32_t)bf16_bits(rb(o[dt][0] * inv)) | ((uint32_t)bf16_bits(rb(o[dt][1] * inv)) << 16);
            const uint32_t w1 = (uint32_t)bf16_bits(rb(o[dt][2] * inv)) | ((uint32_t)bf16_bits(rb(o[dt][3] * inv)) << 16);
            *reinterpret_cast<uint2*>(orow + dt * 16) = make_uint2(w0, w1);
        }
    }
}

hipError_t launch_norm_rows(hipStream_t s, const float* x, const float* gamma, uint16_t* out, int rows, int H,
                            float eps) {
    if (rows < 1) return hipSuccess;
    norm_rows_kernel<<<rows, kRowThreads, sizeof(float) * H, s>>>(x, gamma, out, H, eps);
    return hipGetLastError();
}

hipError_t launch_rope_append(hipStream_t s, const RopeArgs& a, int rows) {
    if (rows < 1) return hipSuccess;
    rope_append_kernel<<<dim3(rows, a.heads + 2 * a.kv_heads), 64, 0, s>>>(a);
    return hipGetLastError();
}

hipError_t launch_flash(hipStream_t s, const FlashArgs& f, int head_dim) {
    if (f.rows < 1) return hipSuccess;
    const dim3 grid(f.heads, (f.rows + kFlashRows - 1) / kFlashRows);
    if (head_dim == 128) flash_prefill_kernel<128><<<grid, kFlashThreads, 0, s>>>(f);
    else if (head_dim == 64) flash_prefill_kernel<64><<<grid, kFlashThreads, 0, s>>>(f);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace y2

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------

namespace {

// Rows per pass through the layers: a whole prompt up to the longest context
// the decode kernels attend (24576).  One pass gives the GEMMs 24000-row
// operands and the flash attention one launch of 188 query blocks per head
// (with 4096-row passes its launches held 1.3-1.5 workgroups per slot, the
// second round half empty): the 24000-token prefill took 0.342 s against
// 0.356 s, and 0.317 s with the heaviest query blocks first.
constexpr int kPrefillChunk = 24576;

struct PrefillBuffers {
    void* block = nullptr;
    float *x = nullptr, *qkv = nullptr, *logits_row = nullptr;
    uint16_t *h = nullptr, *q = nullptr, *att = nullptr, *act = nullptr;
    int32_t* ids = nullptr;
    ~PrefillBuffers() {
        if (block) (void)hipFree(block);
    }
};

int run_prefill(Yue2Model* m, Yue2Cache* c, const int32_t* ids, int n, int phase, float* logits) {
    const Yue2Config& cf = m->c;
    const int H = cf.hidden_size, D = cf.head_dim, Hq = cf.num_attention_heads, Hkv = cf.num_key_value_heads;
    const int I = cf.intermediate_size, qw = Hq * D, qkvw = (Hq + 2 * Hkv) * D;
    const int R = std::min(n, kPrefillChunk);
    PrefillBuffers b;
    size_t at = 0;
    auto take = [&](size_t bytes) {
        const size_t o = at;
        at = (at + bytes + 255) / 256 * 256;
        return o;
    };
    const size_t o_x = take(sizeof(float) * R * H), o_qkv = take(sizeof(float) * R * qkvw);
    const size_t o_h = take(2 * (size_t)R * std::max(H, I)), o_q = take(2 * (size_t)R * qw);
    const size_t o_att = take(2 * (size_t)R * qw), o_act = take(2 * (size_t)R * I);
    const size_t o_ids = take(sizeof(int32_t) * n);
    hipError_t e = hipMalloc(&b.block, at);
    if (e != hipSuccess) return hip_fail(e, "hipMalloc(prefill buffers)");
    char* p = static_cast<char*>(b.block);
    b.x = reinterpret_cast<float*>(p + o_x);
    b.qkv = reinterpret_cast<float*>(p + o_qkv);
    b.h = reinterpret_cast<uint16_t*>(p + o_h);
    b.q = reinterpret_cast<uint16_t*>(p + o_q);
    b.att = reinterpret_cast<uint16_t*>(p + o_att);
    b.act = reinterpret_cast<uint16_t*>(p + o_act);
    b.ids = reinterpret_cast<int32_t*>(p + o_ids);
    hipStream_t s = m->stream;
    e = hipMemcpyAsync(b.ids, ids, sizeof(int32_t) * n, hipMemcpyHostToDevice, s);
    if (e != hipSuccess) return hip_fail(e, "prefill ids upload");
    const float eps = cf.rms_norm_eps;
    for (int p0 = 0; p0 < n; p0 += R) {
        const int rows = std::min(R, n - p0);
        embed_rows_kernel<<<rows, kRowThreads, 0, s>>>(m->embed, b.ids + p0, b.x, H);
        for (int l = 0; l < cf.num_hidden_layers; ++l) {
            const LayerDev& L = m->layers[l];
            if ((e = launch_norm_rows(s, b.x, L.in_norm, b.h, rows, H, eps)) != hipSuccess)
                return hip_fail(e, "prefill norm");
            GemmArgs g{b.h, H, L.wqkv, nullptr, H, b.qkv, nullptr, qkvw, rows, qkvw, H};
            if ((e = launch_gemm(s, GEPI_ROUND, g)) != hipSuccess) return hip_fail(e, "prefill qkv gemm");
            RopeArgs ra{b.qkv, b.q, c->kv, c->capacity, l, Hq, Hkv, D, c->length + p0, L.q_norm, L.k_norm,
                        m->rope_cos, m->rope_sin, eps};
            if ((e = launch_rope_append(s, ra, rows)) != hipSuccess) return hip_fail(e, "prefill rope");
            FlashArgs fa{b.q, c->kv, c->capacity, l, Hq, Hkv, c->length + p0, rows, 1.0f / std::sqrt((float)D),
                         b.att};
            if ((e = launch_flash(s, fa, D)) != hipSuccess) return hip_fail(e, "prefill attention");
            GemmArgs go{b.att, qw, L.wo, nullptr, qw, b.x, nullptr, H, rows, H, qw};
            if ((e = launch_gemm(s, GEPI_RESID, go)) != hipSuccess) return hip_fail(e, "prefill o gemm");
            if ((e = launch_norm_rows(s, b.x, L.post_norm, b.h, rows, H, eps)) != hipSuccess)
                return hip_fail(e, "prefill norm");
            GemmArgs gu{b.h, H, L.wg, L.wu, H, nullptr, b.act, I, rows, I, H};
            if ((e = launch_gemm(s, GEPI_SWIGLU_BF16, gu)) != hipSuccess) return hip_fail(e, "prefill gate/up gemm");
            GemmArgs gd{b.act, I, L.wd, nullptr, I, b.x, nullptr, H, rows, H, I};
            if ((e = launch_gemm(s, GEPI_RESID, gd)) != hipSuccess) return hip_fail(e, "prefill down gemm");
        }
        if ((e = hipGetLastError()) != hipSuccess) return hip_fail(e, "prefill kernels");
        if (p0 + rows == n && logits) {
            // the final norm and LM head of the last prompt row (project_phase)
            if (int rc = enqueue_head(m, m->ws, b.x + (size_t)(rows - 1) * H, phase, s)) return rc;
        }
    }
    e = hipStreamSynchronize(s);
    if (e != hipSuccess) return hip_fail(e, "prefill");
    c->length += n;
    if (logits) {
        e = hipMemcpy(logits, m->ws.logits, sizeof(float) * cf.vocab_size, hipMemcpyDeviceToHost);
        if (e != hipSuccess) return hip_fail(e, "prefill logits readback");
    }
    return YUE2_OK;
}

}  // namespace

extern "C" int32_t yue2_hip_prefill_mfma(Yue2Model* m, Yue2Cache* c, const int32_t* ids, int32_t n, int32_t phase,
                                         float* logits) {
    std::lock_guard<std::recursive_mutex> guard(library_lock());
    if (!m || !c || !ids || c->m != m) return fail(YUE2_ERR_ARG, "null model, cache or ids");
    if (int rc = check_phase_vocab(phase, m->c.vocab_size)) return rc;
    if (n <= 0 || c->length != 0) return fail(YUE2_ERR_ARG, "Invalid prefill/cache capacity");
    if (n > c->capacity || n > m->c.max_position_embeddings)
        return fail(YUE2_ERR_CONTEXT, "AR input exceeds cache/model context");
    for (int i = 0; i < n; ++i)
        if (ids[i] < 0 || ids[i] >= m->c.vocab_size) return fail(YUE2_ERR_TOKEN, "Token outside model vocabulary");
    const Yue2Config& cf = m->c;
    if ((cf.head_dim != 64 && cf.head_dim != 128) || cf.hidden_size % kGemmTK || cf.intermediate_size % kGemmTK ||
        (cf.num_attention_heads * cf.head_dim) % kGemmTK)
        return fail(YUE2_ERR_ARG, "shape without an MFMA prefill");
    if (int rc = m->ws.ensure(1, (c->capacity + kBlockKeys - 1) / kBlockKeys, m->c)) return rc;
    return run_prefill(m, c, ids, n, phase, logits);
}

extern "C" int32_t yue2_hip_selftest_gemm(const uint16_t* x, const uint16_t* w, float* out, int32_t M, int32_t N,
                                          int32_t K) {
    std::lock_guard<std::recursive_mutex> guard(library_lock());
    if (!x || !w || !out || M < 1 || N < 1 || K < 1 || K % kGemmTK) return fail(YUE2_ERR_ARG, "bad gemm selftest");
    if (!device_ready()) return fail(YUE2_ERR_DEVICE, "no gfx950 device");
    void *dx = nullptr, *dw = nullptr, *dc = nullptr;
    hipError_t e = hipMalloc(&dx, 2 * (size_t)M * K);
    if (e == hipSuccess) e = hipMalloc(&dw, 2 * (size_t)N * K);
    if (e == hipSuccess) e = hipMalloc(&dc, 4 * (size_t)M * N);
    if (e == hipSuccess) e = hipMemcpy(dx, x, 2 * (size_t)M * K, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(dw, w, 2 * (size_t)N * K, hipMemcpyHostToDevice);
    if (e == hipSuccess) {
        GemmArgs g{static_cast<const uint16_t*>(dx), K, static_cast<const uint16_t*>(dw), nullptr, K,
                   static_cast<float*>(dc), nullptr, N, M, N, K};
        e = launch_gemm(nullptr, GEPI_RAW, g);
    }
    if (e == hipSuccess) e = hipMemcpy(out, dc, 4 * (size_t)M * N, hipMemcpyDeviceToHost);
    (void)hipFree(dx);
    (void)hipFree(dw);
    (void)hipFree(dc);
    return e == hipSuccess ? YUE2_OK : hip_fail(e, "gemm selftest");
}

namespace {
// BF16 operands of N(0, 1)-like magnitude from a counter hash (the matrix
// cores' power, and so their clock, depends on the bits they toggle).
__global__ void bench_fill_kernel(uint16_t* p, size_t n, uint64_t seed) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        uint64_t z = seed * 0x9e3779b97f4a7c15ull + i;
        z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
        z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
        z ^= z >> 31;
        p[i] = bf16_bits(rb(((float)(z >> 40) * 0x1.0p-24f - 0.5f) * 3.46f));
    }
}
}  // namespace

extern "C" int32_t yue2_hip_bench_gemm(int32_t M, int32_t N, int32_t K, int32_t pair, int32_t iters,
                                       float* avg_ms, double* flops) {
    std::lock_guard<std::recursive_mutex> guard(library_lock());
    if (!avg_ms || !flops || M < 1 || N < 1 || K < 1 || K % kGemmTK || iters < 1)
        return fail(YUE2_ERR_ARG, "bad GEMM benchmark request");
    if (!device_ready()) return fail(YUE2_ERR_DEVICE, "no usable gfx950 device");
    const int wrows = pair ? 2 * N : N;
    void *dx = nullptr, *dw = nullptr, *dc = nullptr;
    hipError_t e = hipMalloc(&dx, 2 * (size_t)M * K);
    if (e == hipSuccess) e = hipMalloc(&dw, 2 * (size_t)wrows * K);
    if (e == hipSuccess) e = hipMalloc(&dc, 4 * (size_t)M * N);
    if (e == hipSuccess) {
        bench_fill_kernel<<<1024, 256>>>(static_cast<uint16_t*>(dx), (size_t)M * K, 1);
        bench_fill_kernel<<<1024, 256>>>(static_cast<uint16_t*>(dw), (size_t)wrows * K, 2);
        e = hipGetLastError();
    }
    hipEvent_t a = nullptr, b = nullptr;
    if (e == hipSuccess) e = hipEventCreate(&a);
    if (e == hipSuccess) e = hipEventCreate(&b);
    const uint16_t* w = static_cast<const uint16_t*>(dw);
    GemmArgs g{static_cast<const uint16_t*>(dx), K, w, pair ? w + (size_t)N * K : nullptr, K, static_cast<float*>(dc),
               static_cast<uint16_t*>(dc), N, M, N, K};
    const int epi = pair ? GEPI_SWIGLU_BF16 : GEPI_ROUND;
    if (e == hipSuccess) e = launch_gemm(nullptr, epi, g);
    if (e == hipSuccess) e = hipEventRecord(a, nullptr);
    for (int i = 0; i < iters && e == hipSuccess; ++i) e = launch_gemm(nullptr, epi, g);
    if (e == hipSuccess) e = hipEventRecord(b, nullptr);
    if (e == hipSuccess) e = hipEventSynchronize(b);
    float ms = 0.0f;
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, a, b);
    if (a) (void)hipEventDestroy(a);
    if (b) (void)hipEventDestroy(b);
    (void)hipFree(dx);
    (void)hipFree(dw);
    (void)hipFree(dc);
    if (e != hipSuccess) return hip_fail(e, "GEMM benchmark");
    *avg_ms = ms / (float)iters;
    *flops = 2.0 * M * (double)wrows * K;
    return YUE2_OK;
}
