// prefill.h -- the matrix-core multi-row kernels shared by the prefill
// (prefill.hip) and the NAR velocity stack (nar.hip): the BF16 MFMA GEMM with
// its fused epilogues, row RMSNorm, QK-norm + RoPE + K/V placement, and the
// flash attention over BF16 keys.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace y2 {

enum GemmEpi {
    GEPI_RAW = 0,             // c (f32) = the accumulation
    GEPI_ROUND = 1,           // c (f32) = rb(acc)
    GEPI_RESID = 2,           // c (f32) = rb(c + rb(acc))  (residual stream, in place)
    GEPI_SWIGLU_BF16 = 3,     // cb (BF16) = rb(rb(silu(rb(gate))) * rb(up)); w = gate rows, w2 = up rows
    GEPI_BIAS = 4,            // c (f32) = rb(acc + bias[col])   (bias BF16-rounded, Linear::finish)
    GEPI_BIAS_SILU_BF16 = 5   // cb (BF16) = rb(silu(rb(acc + bias[col])))
};

// C = X W^T: X [M, K] BF16 (row stride ldx), W [N, K] BF16 (ldw); K a
// multiple of kGemmTK, ldx and ldw multiples of 8.
struct GemmArgs {
    const uint16_t* x;
    int ldx;
    const uint16_t* w;
    const uint16_t* w2;
    int ldw;
    float* c;
    uint16_t* cb;
    int ldc;
    int M, N, K;
    const float* bias;
};

constexpr int kGemmTK = 64;

hipError_t launch_gemm(hipStream_t s, int epi, const GemmArgs& g);

// out[r] = RMSNorm(x[r]) as BF16 for r < rows (x row stride H).
hipError_t launch_norm_rows(hipStream_t s, const float* x, const float* gamma, uint16_t* out, int rows, int H,
                            float eps);

// Per (row r, head): the per-head RMSNorm of q and k and rotate-half RoPE at
// position p0 + r: q heads into q (BF16 [rows][heads][D]), k and v heads
// into a [layers][2][kv_heads][cap][D] BF16 cache at slot p0 + r, or (kv_out
// set) into kv_out at slot slot0 + r with capacity cap_out.
struct RopeArgs {
    const float* qkv;  // [rows][(heads + 2 kv) D], rb'd GEMM outputs
    uint16_t* q;
    uint16_t* kv_base;
    int cap, layer, heads, kv_heads, D, p0;
    const float *q_norm, *k_norm, *cos_t, *sin_t;
    float eps;
    uint16_t* kv_out;
    int slot0, cap_out;
};

hipError_t launch_rope_append(hipStream_t s, const RopeArgs& a, int rows);

// Flash attention of `rows` query rows.  Causal (the prefill): query row r
// sits at position p0 + r and sees keys [0, p0 + r] of kv_base.  Non-causal
// (the NAR stack): every row sees keys [0, split + rows), key j < split from
// kv_base slot j and key j >= split from kv2 slot j - split (capacity cap2).
struct FlashArgs {
    const uint16_t* q;  // [rows][heads][D] BF16
    const uint16_t* kv_base;
    int cap, layer, heads, kv_heads, p0, rows;
    float scale;
    uint16_t* out;  // [rows][heads D] BF16 (rb of the attention output)
    const uint16_t* kv2;
    int cap2, split, noncausal;
};

hipError_t launch_flash(hipStream_t s, const FlashArgs& f, int head_dim);

}  // namespace y2
