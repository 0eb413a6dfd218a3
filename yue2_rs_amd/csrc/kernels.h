// kernels.h -- launch interface of the gfx950 decode kernels (internal).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace y2 {

constexpr int kMaxRows = 2;      // batch rows per step: 1, or 2 for CFG
constexpr int kBlockKeys = 64;   // attention key block (order spec)

// Attention super-blocks (order spec): the softmax sum and each output's PV
// add the block results of a super-block of consecutive 64-key blocks left to
// right, then the super-blocks left to right.  The size depends on the block
// count alone (never on the hardware): 1 below 256 blocks (16384 keys), else
// 2.  A workgroup sums its own super-blocks, so a long context publishes one
// partial per super-block instead of one per block.  (Super-blocks of 4 at
// 256 blocks and more measured slower: whole super-blocks per workgroup then
// give some workgroups more blocks.)
__host__ __device__ constexpr int attn_superblock(int nb) { return nb < 256 ? 1 : 2; }
// Blocks per workgroup when nb blocks are split over wpg workgroups in whole
// super-blocks (the last workgroup with work may hold fewer).
__host__ __device__ constexpr int attn_bpw(int nb, int wpg) {
    return ((nb + attn_superblock(nb) - 1) / attn_superblock(nb) + wpg - 1) / wpg * attn_superblock(nb);
}
// The largest attn_bpw over block counts 1 .. max_blocks.
inline int attn_bpw_max(int max_blocks, int wpg) {
    int m = 1;
    for (int nb = 1; nb <= max_blocks; ++nb) m = attn_bpw(nb, wpg) > m ? attn_bpw(nb, wpg) : m;
    return m;
}

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
    int32_t seq;             // launches of the persistent step kernel (barrier parity)
    int32_t pad[3];
};

enum GemvEpilogue { EPI_STORE = 0, EPI_RESID = 1, EPI_SWIGLU = 2, EPI_RAW = 3 };

struct GemvArgs {
    const uint16_t* w;   // [n, k] BF16
    const uint16_t* w2;  // up projection for EPI_SWIGLU
    const float* x;      // [rows, x_stride] BF16-exact f32 inputs
    float* y;            // output / residual, [rows, y_stride]
    int x_stride, y_stride;
    int n, k, rows;
    const float* gamma;  // non-null: the input is RMSNorm(x) with these gammas
    float eps;
    StepState* st;       // counts RMSNorm guard fallbacks (may be null)
};

struct AttnArgs {
    const float* qkv;    // [rows, qkv_stride]: q heads, then k heads, then v heads (rounded GEMV outputs)
    int qkv_stride;
    KvView kv;
    int layer, heads, kv_heads, dim, rows;
    float scale, eps;
    const float *q_norm, *k_norm;  // null: q is final and the cache already holds position pos
    const float *cos_t, *sin_t;    // RoPE table [positions][dim/2]
    float* bmax;         // [rows][heads][blk_stride] block maxima
    float* bsum;         // [rows][heads][blk_stride] block sums
    float* part;         // [rows][heads][blk_stride][dim] partial PV
    float* out;          // [rows, out_stride]
    int out_stride, blk_stride;
    int wgs, bpw;        // workgroups per (kv head, row); 64-key blocks per workgroup
    int* counters;       // [rows][kv_heads][4], zero between launches
    StepState* st;
    // Tagged-word block maxima, sums and partials (same shapes, zero or
    // written by earlier launches); non-null: launch_attention runs the
    // tagged-word kernel where the shape allows (q_norm non-null, head_dim
    // 64 or 128), its tags from st->seq and the layer, so st->seq must
    // change between two launches of one layer.
    uint64_t *tbmax, *tbsum, *tpart;
};

// Workgroups per (kv head, row) and 64-key blocks per workgroup for caches
// of max_blocks blocks.
void attention_geometry(int kv_heads, int rows, int max_blocks, int* wgs, int* bpw);

void launch_embed(hipStream_t s, const uint16_t* embed, const StepState* st, float* x, int hidden,
                  int vocab, int rows);
void launch_rmsnorm(hipStream_t s, const float* x, int x_stride, const float* gamma, float* out,
                    int out_stride, int n, float eps, int rows, StepState* st);
hipError_t launch_gemv(hipStream_t s, int epi, const GemvArgs& a);
hipError_t launch_attention(hipStream_t s, const AttnArgs& a);
void launch_argmax(hipStream_t s, const float* logits, int stride, int n, StepState* st,
                   int32_t* token_log, int rows);
void launch_advance(hipStream_t s, StepState* st, int rows);

// Diagnostics: evaluate the device math functions elementwise.
void launch_math_selftest(hipStream_t s, int which, const void* in, void* out, size_t n);

}  // namespace y2
