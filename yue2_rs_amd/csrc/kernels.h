// kernels.h -- launch interface of the gfx950 decode kernels (internal).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace y2 {

constexpr int kMaxRows = 2;      // batch rows per step: 1, or 2 for CFG
constexpr int kBlockKeys = 64;   // attention key block (order spec)

// Per-row view of a KV cache: layout [layers][2][kv_heads][capacity][dim] BF16.
struct KvView {
    uint16_t* base[kMaxRows];
    int capacity[kMaxRows];
};

// Per-step device state that a captured graph reads on every replay.
struct StepState {
    int32_t pos[kMaxRows];   // position of the token being processed (= cache length)
    int32_t ids[kMaxRows];   // token id fed to the embedding
    int32_t step;            // decode steps taken
    int32_t error;           // sticky device error code (0 = ok)
    int32_t norm_fallbacks;  // RMSNorm guard fallbacks (diagnostic)
    int32_t done;            // set when the phase's end token was chosen
};

enum GemvEpilogue { EPI_STORE = 0, EPI_RESID = 1, EPI_SWIGLU = 2, EPI_RAW = 3 };

struct GemvArgs {
    const uint16_t* w;   // [n, k] BF16
    const uint16_t* w2;  // up projection for EPI_SWIGLU
    const float* x;      // [rows, x_stride] BF16-exact f32 inputs
    float* y;            // output / residual, [rows, y_stride]
    int x_stride, y_stride;
    int n, k, rows;
};

struct AttnArgs {
    const float* q;      // [rows, q_stride]; head h at h*dim
    int q_stride;
    KvView kv;
    int layer, layers, heads, kv_heads, dim;
    float scale;
    float* scores;       // [rows][heads][score_stride] scaled scores, then exps
    float* bmax;         // [rows][heads][blk_stride]
    float* bsum;         // [rows][heads][blk_stride]
    float* part;         // [rows][heads][blk_stride][dim]
    float* out;          // [rows, out_stride]
    int out_stride, score_stride, blk_stride, max_blocks, rows;
    const StepState* st;
};

struct HeadArgs {
    float* qkv;          // [rows, qkv_stride]: q heads, k heads, v heads
    int qkv_stride;
    const float *q_norm, *k_norm;
    const float *cos_t, *sin_t;  // [max_pos][dim/2]
    KvView kv;
    int layer, layers, heads, kv_heads, dim, rows;
    float eps;
    const StepState* st;
};

void launch_embed(hipStream_t s, const uint16_t* embed, const StepState* st, float* x, int hidden,
                  int vocab, int rows);
void launch_rmsnorm(hipStream_t s, const float* x, int x_stride, const float* gamma, float* out,
                    int out_stride, int n, float eps, int rows, StepState* st);
hipError_t launch_gemv(hipStream_t s, int epi, const GemvArgs& a);
void launch_heads(hipStream_t s, const HeadArgs& a);
void launch_attention(hipStream_t s, const AttnArgs& a);
void launch_argmax(hipStream_t s, const float* logits, int stride, int n, StepState* st,
                   int32_t* token_log, int rows);
void launch_advance(hipStream_t s, StepState* st, int rows);

// Diagnostics: evaluate the device math functions elementwise.
void launch_math_selftest(hipStream_t s, int which, const void* in, void* out, size_t n);

}  // namespace y2
