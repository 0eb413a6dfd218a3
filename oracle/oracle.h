/*
 * oracle.h -- CPU restatement of the YuE2 autoregressive decode step.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (yue2_rs_amd/, include/)
 * includes, links or loads this code.  Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg use it, and only as the checker / the CPU
 * baseline, never as the thing measured on the GPU.
 *
 * The reference (twally3/yue2_rs) is Rust + Apple Accelerate + Metal and
 * cannot be built on Linux (build.rs:6-9).  This file restates its CPU token
 * step (YUE2_BACKEND=cpu) operation by operation, keeping every BF16
 * rounding point of src/tensor.rs, src/model.rs and src/sampling.rs.
 * Accelerate's free reductions (cblas_sgemv/sgemm, vDSP_sve) are replaced by
 * one documented order (the "order spec" below); vvexpf and f64::ln_1p are
 * replaced by our own functions written from named methods.
 *
 * ORDER SPEC (shared with the HIP kernels; both sides implement it)
 *   DOT(a, b, K)   K % 8 == 0.  Chunk c = elements [8c, 8c+8).  Chunk c
 *                  belongs to lane c mod 64.  Each lane: acc = +0; for its
 *                  chunks in ascending order, for e = 0..7:
 *                  acc = fma(a[8c+e], b[8c+e], acc).  Then an xor butterfly
 *                  over the 64 lanes with offsets 32,16,8,4,2,1:
 *                  acc[l] = acc[l] + acc[l ^ s].  Result: acc[0].
 *                  Used for every Linear row (cblas_sgemv/sgemm substitute,
 *                  src/tensor.rs:847-883, 1026-1081) and for the attention
 *                  scores q.K_j (src/model.rs:362-374).
 *   SUPER-BLOCK    nb = ceil(keys / 64) blocks of 64 keys are grouped in
 *                  super-blocks of SB = y2o_superblock(nb) consecutive
 *                  blocks (1 below 256 blocks, else 2; the last super-block
 *                  may be short).  SB depends on the key count alone, never
 *                  on the hardware.
 *   SOFTMAX SUM    keys in blocks of 64 (block b = keys [64b, 64b+64));
 *                  block sum = xor butterfly (32..1) over lane = key - 64b,
 *                  missing keys = +0; super-block sum = its block sums left
 *                  to right; total = the super-block sums left to right
 *                  ((u0 + u1) + u2) + ... (vDSP_sve substitute,
 *                  src/tensor.rs:721).  With SB = 1 this is
 *                  ((blk0 + blk1) + blk2) + ...
 *   PV             per output dim d, block of 64 keys, S = 512/head_dim
 *                  streams; key j of the block goes to stream (j-64b) mod S;
 *                  stream: acc = +0, acc = fma(p_j, V[j,d], acc) ascending;
 *                  streams combined by xor butterfly over the stream index
 *                  with offsets S/2, ..., 1; the blocks of a super-block
 *                  summed left to right, then the super-blocks left to right
 *                  (cblas_sgemv transpose substitute, src/model.rs:380-392).
 *   RMSNorm sum    sequential f32 sum as the reference defines it
 *                  (src/tensor.rs:1144, 1160): no substitute needed.
 *
 * Parity pins (what checks each function; tests/test_oracle_*.py):
 *   y2o_round_bf16   nearest BF16 with ties to even, computed from the two
 *                    BF16 neighbours in f64, on 90k bit patterns incl. ties.
 *   y2o_expf         equals the correctly rounded exp (numpy float64 exp
 *                    rounded once to f32) on 89k inputs incl. both range ends
 *                    -- stands in for vvexpf and f32::exp, whose own ulp
 *                    behaviour is unpublished (parity unpinned beyond that).
 *   y2o_log1p        within 2 ulp of numpy log1p on the race's domain.
 *   y2o_linear/DOT   one-hot inputs reproduce W's columns; small-integer
 *                    operands give the exact integer product; random operands
 *                    stay inside the f32 dot-product error bound of an f64
 *                    product; a row alone equals the same row in a batch.
 *   y2o_norm_*       constant rows in closed form; an input on which only a
 *                    sequential f32 sum of squares gives the right BF16 scale.
 *   y2o_rotary_*     position 0 is the identity; the table is rb(cos/sin) of
 *                    p * theta^(-2i/d) within one BF16 step of f64 libm.
 *   y2o_attention_row the reference's own known-answer generator and
 *                    tolerance (src/tensor.rs:9-83) against f64, from 4096 to
 *                    24576 keys (super-blocks of 1 and 2); one key gives
 *                    rb(V0); equal keys give rb(mean V) exactly, also over
 *                    16384 keys (a super-block dropped, doubled or cut at the
 *                    wrong block changes it).
 *   y2o_cfg_mix      scale 1 / 0 give the conditional / unconditional row.
 *   y2o_mt_*         std::mt19937 known answer (10000th draw of seed 5489),
 *                    2000 draws equal numpy's RandomState for five seeds,
 *                    uniform_f64 and discard from their definitions.
 *   y2o_choose       greedy ties and no draw at T = 0; exactly 2V draws when
 *                    sampling; race frequencies equal the softmax (5 sigma);
 *                    top-p keeps the crossing token and 1 (legacy 3) protected
 *                    ids; top-k keeps ties; penalty sign, powi and window;
 *                    NaN/+inf rejected; ABC/semantic masks and min_tokens.
 *   y2o_forward     an independent float64 numpy forward of the reference's
 *                    formulas within 1e-3 of the largest logit (measured 0);
 *                    each single-rounding mutant of that model (SiLU, g*u,
 *                    attention output, O projection, inner RoPE products)
 *                    exceeds the bound; W_o = W_down = 0 in closed form;
 *                    chunked prefill equals the token-by-token step.
 *   y2o_generate    equal to a Python restatement of the loop over the
 *                    separately pinned prefill / forward_phase, cfg_mix,
 *                    choose and MT19937 (end stop after min_tokens, unequal
 *                    negative prefix, legacy, truncation); tests/golden/
 *                    fixtures written by tests/golden/make_golden.py.
 *   y2o_velocity    linear biases, the timestep embedding and the position
 *                    rows from closed forms on a model whose NAR linears and
 *                    layers are zero (tests/test_oracle_nar.py); with
 *                    non-causal attention, a row's output does not depend on
 *                    the order of the other rows' keys only through their
 *                    set -- permuting the frames permutes the outputs when
 *                    no position-dependent term enters (RoPE start, latent
 *                    position rows equal); parity unpinned beyond these.
 *   y2o_normal      every value within 3 ulps of a float64 Box-Muller of the
 *                    same MT19937 uniform_f32 draws (measured 2.08); pairs
 *                    share the radius; moments of N(0, 1).
 *   y2o_synthesize  a model whose velocity has a closed form in the state
 *                    and the time (zero NAR layers, one-hot linears): the
 *                    chunk cuts, t schedule, midpoint state and both steps
 *                    restated in the test give the same bits (a wrong dt,
 *                    midpoint or second time fails); with zero velocity the
 *                    output is the rounded noise.
 *   y2o_conv        the reference's own convolution known-answer cases and
 *                    scalar formula (src/vae.rs:812-892, tolerance 2e-6);
 *                    within 1e-5 of a float64 convolution on shapes with
 *                    up to 130 channels, 20 phases and dilation 9.
 *   y2o_vae_*       closed forms (SnakeBeta at alpha = beta = 1, ELU, tanh,
 *                    the weight norm's row norms = |g|), Conv::length, a
 *                    tiled decode equal to the whole decode on every core row,
 *                    and the whole decoder within 1e-4 of an independent
 *                    float64 evaluation (tests/vae_files.py decode_f64).
 *   Accelerate's exact summation order, macOS libm cos/sin/powf and the real
 *   checkpoint's logits cannot be run here: parity with those is unpinned
 *   beyond the checks above.
 */
#ifndef YUE2_ORACLE_H
#define YUE2_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Model configuration (src/model.rs:11-27). */
typedef struct {
    int32_t hidden, layers, heads, kv_heads, head_dim, intermediate, vocab;
    int32_t max_pos;
    float eps, theta;
} y2o_config;

/* One AR layer: BF16 matrices [out, in] row-major, norm gammas as f32
 * (already BF16-rounded, src/tensor.rs:1126-1136). */
typedef struct {
    const uint16_t *q, *k, *v, *o, *gate, *up, *down;
    const float *input_norm, *q_norm, *k_norm, *post_norm;
} y2o_layer;

typedef struct {
    y2o_config c;
    const uint16_t *embed;   /* [vocab, hidden] */
    const uint16_t *lm_head; /* [vocab, hidden] */
    const float *final_norm; /* [hidden] */
    const y2o_layer *layers; /* [layers] */
} y2o_model;

/* Host KV mirror (src/model.rs:276-306): per layer f32 [capacity, kv*dim]. */
typedef struct {
    int32_t layers, width, capacity, length;
    float *key;   /* [layers][capacity][width] */
    float *value; /* [layers][capacity][width] */
} y2o_cache;

/* Sampling (src/protocol.rs:143-165). */
typedef struct {
    float temperature, top_p;
    int32_t top_k;
    float repetition_penalty;
    int32_t penalty_window, min_tokens, max_tokens;
} y2o_sampling;

typedef struct {
    uint32_t state[624];
    int32_t next;
} y2o_mt;

enum { Y2O_PHASE_NONE = 0, Y2O_PHASE_ABC = 1, Y2O_PHASE_SEMANTIC = 2 };
enum {
    Y2O_OK = 0,
    Y2O_ERR_CONTEXT = -1,   /* "AR input exceeds cache/model context" */
    Y2O_ERR_TOKEN = -2,     /* "Token outside model vocabulary" */
    Y2O_ERR_VOCAB = -3,     /* "Vocabulary does not support native music protocol" */
    Y2O_ERR_LOGITS = -4,    /* "Model produced invalid logits" */
    Y2O_ERR_EMPTY = -5,     /* "Empty sampling distribution" */
    Y2O_ERR_SAMPLING = -6,  /* "Invalid sampling configuration" */
    Y2O_ERR_BUDGET = -7,    /* "Prefix + requested generation budget exceeds 24576" */
    Y2O_ERR_GUIDANCE = -8,  /* "Guidance requires negative prefix" */
    Y2O_ERR_CODEC = -9,     /* "Incomplete codec vocabulary" */
    Y2O_ERR_ALLOC = -10
};

void y2o_set_threads(int n);
int y2o_get_threads(void);

float y2o_round_bf16(float v);
void y2o_round_bf16_bits(const uint32_t *in, uint32_t *out, size_t n);
float y2o_bf16_to_f32(uint16_t b);
float y2o_expf(float x);
double y2o_log1p(double x);

float y2o_dot_bf16(const uint16_t *a, const float *b, int k);
float y2o_dot_f32(const float *a, const float *b, int k);
/* y[r*out + i] = rb(DOT(W[i], x[r])) for r < rows (src/tensor.rs:946-1118) */
void y2o_linear(const uint16_t *w, int out, int in, const float *x, int rows, float *y);
/* out[i] = DOT(W[i], x) without rounding (yue2_metal_vector's contract) */
void y2o_gemv_raw(const uint16_t *w, int rows, int cols, const float *x, float *out);

float y2o_norm_scale(const float *x, int n, float eps);
void y2o_norm_apply(const float *x, int rows, int n, const float *gamma, float eps, float *out);
void y2o_norm_heads(float *x, int heads, int dim, const float *gamma, float eps);

void y2o_rotary_table(int start, int rows, int head_dim, float theta, float *cos, float *sin);
void y2o_rotary_apply(float *x, int rows, int cols, int half, const float *cos, const float *sin);

/* Blocks per super-block of the attention's sums for `blocks` 64-key blocks. */
int y2o_superblock(int blocks);
/* Single-query GQA attention over `keys` cached rows; K/V rows have stride
 * kv*dim (src/model.rs:313-397 with rows == 1). */
void y2o_attention_row(const float *q, const float *key, const float *value, int keys,
                       int heads, int kv, int dim, float *out);

y2o_cache *y2o_cache_new(const y2o_config *c, int capacity);
void y2o_cache_free(y2o_cache *cache);
int y2o_cache_length(const y2o_cache *cache);

/* Model::hidden (src/model.rs:523-591): x_out = final_norm(x) for all rows. */
int y2o_hidden(const y2o_model *m, y2o_cache *cache, const int32_t *ids, int n, float *x_out);
/* The same without the final norm (yue2_metal_ar_stack's `out`). */
int y2o_hidden_prenorm(const y2o_model *m, y2o_cache *cache, const int32_t *ids, int n, float *x_out);
/* Model::forward (src/model.rs:465-468): logits of the last row. */
int y2o_forward(const y2o_model *m, y2o_cache *cache, const int32_t *ids, int n, float *logits);
/* y2o_forward_phase of one token in each of R <= 8 caches in one pass over
 * the weights (the replay of a batch-2 decode step); the same results as R
 * calls. */
int y2o_forward_rows(const y2o_model *m, y2o_cache *const *caches, const int32_t *ids, int R, int phase,
                     float *logits);
/* Model::forward_phase / project_phase (src/model.rs:469-507). */
int y2o_forward_phase(const y2o_model *m, y2o_cache *cache, const int32_t *ids, int n,
                      int phase, float *logits);
int y2o_project_phase(const y2o_model *m, const float *x, int phase, float *logits);
/* Model::prefill (src/model.rs:592-610): 256-token chunks, logits of the last row. */
int y2o_prefill(const y2o_model *m, y2o_cache *cache, const int32_t *ids, int n, float *logits);

/* The NAR (acoustic) pathway (Model::open, src/model.rs:418-451; Layer::load
 * nar_*, :264-269): NAR layers with the AR layer's tensors, the linears with
 * biases (vae2llm [H, latent], llm2vae [latent, H], time_embedder.mlp.0
 * [H, 256], time_embedder.mlp.2 [H, H]; biases f32, BF16-rounded where used
 * as Linear::finish does) and latent_pos_embed.pe [max_frames, H] BF16. */
typedef struct {
    int32_t latent, max_frames;
    float shift;
    const uint16_t *vae2llm, *llm2vae, *time_in, *time_out, *latent_pos;
    const float *vae2llm_b, *llm2vae_b, *time_in_b, *time_out_b;
    const y2o_layer *layers;
} y2o_nar;

/* Model::velocity (src/model.rs:611-698) for `frames` latent rows (state
 * [frames, latent]) against the AR cache: out [frames, latent].  The keys
 * are the cache's first min(nar_cond_end, length) positions (all when
 * nar_cond_end is 0) followed by the rows' own; RoPE positions start at the
 * cache length; the cache is not modified. */
int y2o_velocity(const y2o_model *m, const y2o_nar *nar, const y2o_cache *cache, const float *state,
                 int frames, double raw_t, int nar_cond_end, float *out);

/* Generator::normal_tensor (src/sampling.rs:64-79): n (a multiple of 16)
 * uniform_f32 draws, then Box-Muller within each block of 16 (libm
 * logf/sqrtf/cosf/sinf in f32, the angle 2 pi u in f64). */
void y2o_normal(uint64_t seed, int n, float *out);

/* Model::synthesize (src/model.rs:699-775): codec_len latent frames
 * ([codec_len, latent], latent 64) from the prefix and the codec ids by the
 * midpoint flow-matching loop over `steps` steps per context chunk. */
int y2o_synthesize(const y2o_model *m, const y2o_nar *nar, const int32_t *prefix, int prefix_len,
                   const int32_t *codec, int codec_len, uint64_t seed, int steps, float *out);

/* The VAE decoder (src/vae.rs:49-611) as a list of operations in network
 * order.  Conv / ConvT carry the weight-norm pair (v [out, in, k], or
 * [in, out, k] transposed; g [rows of v]) and a bias (NULL: none); Snake
 * carries the alpha and beta parameters (exp taken here); Residual begin /
 * end bracket a residual unit.  All FP32 (no BF16 rounding). */
enum {
    Y2O_VAE_CONV = 0, Y2O_VAE_CONVT = 1, Y2O_VAE_SNAKE = 2, Y2O_VAE_ELU = 3, Y2O_VAE_TANH = 4,
    Y2O_VAE_RES_BEGIN = 5, Y2O_VAE_RES_END = 6
};
typedef struct {
    int32_t kind, cin, cout, kernel, stride, padding, dilation;
    const float *v, *g, *b, *alpha, *beta;
} y2o_vae_op;

/* Conv::apply / transposed (src/vae.rs:165-257) with ready weights w
 * ([out, in, k], or [in, out, k] transposed) and bias b (may be NULL):
 * out [length, cout], x [frames, cin]. */
void y2o_conv(int transpose, int cin, int cout, int kernel, int stride, int padding, int dilation,
              const float *x, int frames, const float *w, const float *b, float *out);
/* Conv::length (src/vae.rs:147-153) */
int y2o_conv_length(int transpose, int n, int kernel, int stride, int padding, int dilation);
/* Op::apply of the whole list (src/vae.rs:378-397): out [*out_frames, *out_channels]
 * (the caller sizes out from y2o_vae_length). */
int y2o_vae_run(const y2o_vae_op *ops, int nops, const float *x, int frames, int channels, float *out,
                int *out_frames, int *out_channels);
int y2o_vae_length(const y2o_vae_op *ops, int nops, int frames);

void y2o_mt_seed(y2o_mt *g, uint64_t seed);
uint32_t y2o_mt_next(y2o_mt *g);
void y2o_mt_discard(y2o_mt *g, uint64_t count);
double y2o_mt_uniform_f64(y2o_mt *g);

void y2o_cfg_mix(const float *cond, const float *uncond, int n, float scale, float *out);
int y2o_choose(const float *logits, int n, const y2o_sampling *s, const int32_t *history,
               int history_len, int step, int phase, int legacy, y2o_mt *rng, int32_t *out);

/* sampling::generate (src/sampling.rs:222-294).  negative may be NULL. */
int y2o_generate(const y2o_model *m, const int32_t *prefix, int prefix_len,
                 const y2o_sampling *s, uint64_t seed, int phase, const int32_t *negative,
                 int negative_len, float scale, int legacy, int32_t *tokens, int *count,
                 int *truncated);

#ifdef __cplusplus
}
#endif
#endif
