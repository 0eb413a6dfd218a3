/*
 * yue2_hip.h -- C ABI of the MI355X (gfx950) decode library for YuE2's
 * autoregressive token step.
 *
 * Two groups of entry points:
 *
 *  1. Drop-in twins of the reference's native decode bridge.  Each has the
 *     same arguments, the same meaning and the same 1 = done / 0 = "not
 *     done, fall back to the CPU" convention as the yue2_metal_* function it
 *     replaces (declared at src/tensor.rs:91-220, implemented in
 *     src/metal.m).  A Rust caller changes only the symbol prefix.
 *
 *  2. A device-resident session API for the fast path: weights uploaded
 *     once, BF16 KV caches, positions, the RoPE table and the sampler state
 *     stay in HBM; one captured hipGraph runs one token step, and only token
 *     ids cross PCIe.  These mirror the Rust model-step API
 *     (Model::forward / forward_phase / prefill_phase, Cache::new,
 *     sampling::generate) and return 0 on success or a negative Yue2Error,
 *     the codes standing for the reference's InvalidData messages
 *     (src/lib.rs:14-18).
 *
 * All entry points are thread-safe: one library lock serialises them, as the
 * reference's global NSLock does (src/metal.m:21).
 */
#ifndef YUE2_HIP_H
#define YUE2_HIP_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------------- */
/* 1. Twins of the reference's native bridge                               */
/* ---------------------------------------------------------------------- */

/* GpuWeight / GpuLayer (src/tensor.rs:221-237 = src/metal.m:363-368).
 * dtype: 0 BF16, 1 F32, 2 F16.  norms: input, q_norm, k_norm, post_attention.
 * key/value: the host KV mirror, rows of kv*dim f32 (BF16-exact). */
typedef struct Yue2GpuWeight {
    const uint8_t *raw;
    size_t mapping, rows, cols;
    int32_t dtype, rounded;
} Yue2GpuWeight;

typedef struct Yue2GpuLayer {
    Yue2GpuWeight weights[7]; /* q, k, v, o, gate, up, down */
    const float *norms[4];
    const float *key;
    const float *value;
} Yue2GpuLayer;

/* yue2_metal_available (src/tensor.rs:118): 1 when a gfx950 device is usable. */
int32_t yue2_hip_available(void);
/* yue2_metal_vector_default (src/tensor.rs:119): 1 when the single-row GEMV
 * path should be used by default (device memory >= 2 GiB). */
int32_t yue2_hip_vector_default(void);
/* yue2_metal_name (src/tensor.rs:193): device name, "CPU" without a device. */
const char *yue2_hip_name(void);
/* yue2_physical_memory (src/tensor.rs:131): host physical memory in bytes. */
uint64_t yue2_physical_memory(void);

/* yue2_metal_vector (src/tensor.rs:120-130; src/metal.m:545-603):
 * out[r] = sum_c W[r,c] * input[c] for r < rows, f32 accumulation in the DOT
 * order, NOT rounded (the caller's Linear::finish rounds).  Weights are
 * uploaded on first use and cached under (mapping, raw, rows, cols, dtype).
 * F32/F16 weights are accepted when rounded != 0 (they are rounded to BF16 on
 * upload, as the reference's converted path does); otherwise returns 0. */
int32_t yue2_hip_vector(const float *input, const uint8_t *raw, size_t mapping, int32_t dtype,
                        int32_t rounded, int32_t priority, float *out, size_t rows, size_t cols);

/* yue2_metal_ar_stack (src/tensor.rs:146-163; src/metal.m:718-874): one
 * decode token through `count` AR layers.  input = embedded token (1 x hidden);
 * out = hidden state before the final norm; shadow = per layer [K(kv*dim),
 * V(kv*dim)] of the new token as f32; prefix = position; cos/sin = that
 * position's RoPE row (dim/2 each); cache = the Rust Cache id.  The device KV
 * context of (cache, layer) is mirrored from layers[i].key/value. */
int32_t yue2_hip_ar_stack(const float *input, float *out, float *shadow,
                          const Yue2GpuLayer *layers, size_t count, size_t hidden, size_t heads,
                          size_t kv, size_t dim, size_t intermediate, size_t prefix,
                          size_t capacity, size_t cache, float eps, const float *cos,
                          const float *sin);

/* yue2_metal_cached_attention (src/tensor.rs:181-192; src/metal.m:669-687):
 * single-query GQA attention over `keys` rows of the host K/V mirror
 * (rows of kv*dim f32); out = heads*dim, BF16-rounded. */
int32_t yue2_hip_cached_attention(const float *q, const float *k, const float *v, float *out,
                                  size_t keys, size_t heads, size_t kv, size_t dim, size_t cache,
                                  size_t layer);

/* The prefill / NAR bridge (src/tensor.rs:135-145, 194-219; src/metal.m:
 * 164-237, 330-361): plain FP32 products on the platform BLAS and the
 * multi-row attention on the matrix-core flash kernel.  Like the reference's
 * MPS path they sum in another order than the CPU path, so they agree with
 * it within FP32 rounding (gemm, linear) or the matrix-core prefill's
 * tolerance (attention), and return 1 = done / 0 = fall back to the CPU.
 * yue2_metal_gemm: c [m x n] = a [m x k] op(b) + beta c, row-major host
 * matrices with row strides lda, ldb, ldc; op(b) = b [k x n], or with
 * transpose_b b^T for b [n x k]. */
int32_t yue2_hip_gemm(const float *a, const float *b, float *c, size_t m, size_t n, size_t k,
                      int32_t transpose_b, size_t lda, size_t ldb, size_t ldc, float beta);
/* yue2_metal_linear: c [m x n] = a [m x k] W^T for the host weight W [n x k]
 * (dtype 0 BF16, 1 F32, 2 F16; rounded: F32/F16 values rounded to BF16, as
 * convert_weight does, src/attention.metal:161-176), cached on the device
 * under (mapping, raw, n, k, dtype, rounded); not rounded (the caller's
 * Linear::finish rounds). */
int32_t yue2_hip_linear(const float *a, const uint8_t *raw, size_t mapping, int32_t dtype, int32_t rounded,
                        float *c, size_t m, size_t n, size_t k);
/* yue2_metal_attention: `rows` query rows q [rows x heads*dim] over k, v
 * [keys x kv*dim]; row r sees keys [0, min(keys, causal + r + 1)) (causal >=
 * 0) or all (causal < 0); out [rows x heads*dim] rounded to BF16.  Falls back
 * (0) for inputs that are not BF16-exact, head_dim other than 64 / 128, a
 * scale other than 1/sqrt(dim) and causal windows past `keys`. */
int32_t yue2_hip_attention(const float *q, const float *k, const float *v, float *out, size_t rows,
                           size_t keys, size_t heads, size_t kv, size_t dim, int64_t causal, float scale);
/* yue2_metal_stack (src/tensor.rs:164-180) is not twinned: the session API's
 * yue2_hip_velocity runs the same NAR stack on the device. */

/* Lifetime (src/tensor.rs:132-134; src/metal.m:73-103). */
void yue2_hip_release_cache(size_t cache);
void yue2_hip_clear_weights(void);
void yue2_hip_release_model(void);

/* ---------------------------------------------------------------------- */
/* 2. Device-resident session API                                          */
/* ---------------------------------------------------------------------- */

typedef enum Yue2Error {
    YUE2_OK = 0,
    YUE2_ERR_CONTEXT = -1,  /* "AR input exceeds cache/model context" (src/model.rs:529) */
    YUE2_ERR_TOKEN = -2,    /* "Token outside model vocabulary" (src/model.rs:457) */
    YUE2_ERR_VOCAB = -3,    /* "Vocabulary does not support native music protocol" */
    YUE2_ERR_LOGITS = -4,   /* "Model produced invalid logits" (src/sampling.rs:146) */
    YUE2_ERR_EMPTY = -5,    /* "Empty sampling distribution" */
    YUE2_ERR_SAMPLING = -6, /* "Invalid sampling configuration" (src/protocol.rs:191) */
    YUE2_ERR_BUDGET = -7,   /* "Prefix + requested generation budget exceeds 24576" */
    YUE2_ERR_GUIDANCE = -8, /* "Guidance requires negative prefix" */
    YUE2_ERR_CODEC = -9,    /* "Incomplete codec vocabulary" */
    YUE2_ERR_ALLOC = -10,   /* device or host allocation failed */
    YUE2_ERR_CONFIG = -11,  /* "Invalid transformer configuration" (src/model.rs:71) */
    YUE2_ERR_DEVICE = -12,  /* no usable device, or a HIP call failed */
    YUE2_ERR_ARG = -13,     /* a null pointer or an unsupported shape */
    YUE2_ERR_TIES = -14     /* top-k survivors exceed the survivor arrays (not reached:
                               they hold the whole vocabulary) */
} Yue2Error;

/* Phases of project_phase/choose (src/sampling.rs:81-99).  NONE is the full
 * vocabulary with no end token (Model::forward), used by synthetic
 * vocabularies smaller than the music protocol's ids. */
enum { YUE2_PHASE_NONE = 0, YUE2_PHASE_ABC = 1, YUE2_PHASE_SEMANTIC = 2 };

/* Config (src/model.rs:11-27). */
typedef struct Yue2Config {
    int32_t hidden_size, num_hidden_layers, num_attention_heads, num_key_value_heads;
    int32_t head_dim, intermediate_size, vocab_size, max_position_embeddings;
    float rms_norm_eps, rope_theta;
} Yue2Config;

/* One AR layer's host weights: BF16 matrices [out, in]; norm gammas as f32
 * (rounded to BF16 on upload, Norm::new src/tensor.rs:1126-1136). */
typedef struct Yue2LayerWeights {
    const uint16_t *q_proj, *k_proj, *v_proj, *o_proj, *gate_proj, *up_proj, *down_proj;
    const float *input_layernorm, *q_norm, *k_norm, *post_attention_layernorm;
} Yue2LayerWeights;

/* Sampling (src/protocol.rs:143-152). */
typedef struct Yue2Sampling {
    float temperature, top_p;
    int32_t top_k;
    float repetition_penalty;
    int32_t penalty_window, min_tokens, max_tokens;
} Yue2Sampling;

typedef struct Yue2Model Yue2Model;
typedef struct Yue2Cache Yue2Cache;
typedef struct Yue2Decoder Yue2Decoder;

/* Config::read validation (src/model.rs:50-72); 0 or YUE2_ERR_CONFIG. */
int32_t yue2_hip_config_validate(const Yue2Config *c);
/* Sampling::validate (src/protocol.rs:191-207); 0 or YUE2_ERR_SAMPLING. */
int32_t yue2_hip_sampling_validate(const Yue2Sampling *s);

/* Model::open (src/model.rs:418-451) from host arrays: the weights are copied
 * into one HBM allocation and stay resident.  NULL on failure
 * (yue2_hip_last_error tells why). */
Yue2Model *yue2_hip_model_open(const Yue2Config *c, const uint16_t *embed_tokens,
                               const uint16_t *lm_head, const float *final_norm,
                               const Yue2LayerWeights *layers);
/* Model::open (src/model.rs:418-451) from a checkpoint directory: config.json
 * (Config::read, src/model.rs:29-73) and model.safetensors, or the shards
 * named by model.safetensors.index.json (Weights::open,
 * src/checkpoint.rs:310-386), memory-mapped and checked as the reference
 * checks them, with its messages (yue2_hip_last_error).  Reads the tensors of
 * the autoregressive decode path: model.embed_tokens, lm_head (or the tied
 * embedding), model.norm and per layer input_layernorm, self_attn.{q,k,v,o}
 * _proj, self_attn.{q,k}_norm, post_attention_layernorm, mlp.{gate,up,down}
 * _proj.  F32 and F16 matrices are rounded to BF16 as the reference's
 * converted weights are.  NULL on failure. */
Yue2Model *yue2_hip_model_open_dir(const char *dir);
/* The checks of yue2_hip_model_open_dir without a device: config.json, every
 * shard's header, and the decode path's tensors and shapes.  *out (may be
 * NULL) receives the configuration.  0 or a negative Yue2Error
 * (YUE2_ERR_CONFIG where the reference returns InvalidData). */
int32_t yue2_hip_checkpoint_config(const char *dir, Yue2Config *out);
/* Model's Drop (src/model.rs:411-416).  Models, caches and decoders may be
 * freed in any order, as the reference lets a Cache outlive its Model
 * (src/model.rs:286-290): the model's free detaches its live caches and
 * decoders.  A detached decoder holds no device objects and its calls return
 * YUE2_ERR_ARG; a detached cache keeps its KV memory, which
 * yue2_hip_cache_export can still read, until yue2_hip_cache_free. */
void yue2_hip_model_free(Yue2Model *m);

/* Cache::new (src/model.rs:292-305): a device BF16 KV cache of `capacity`
 * positions, layout [layers][K,V][kv_heads][capacity][head_dim]. */
Yue2Cache *yue2_hip_cache_new(Yue2Model *m, int32_t capacity);
/* Cache's Drop (src/model.rs:286-290), before or after its model's free;
 * decoders running on the cache are detached with it. */
void yue2_hip_cache_free(Yue2Cache *c);
int32_t yue2_hip_cache_length(const Yue2Cache *c);
/* The device context of a cache from its host K/V mirror (Cache's key/value,
 * src/model.rs:276-306), as the reference's Metal bridge fills its device
 * context from the mirror (contextEntry, src/metal.m:633-666): key and value
 * hold, per layer, `stride` rows of kv_heads * head_dim BF16-exact f32 values
 * (layer l starts at l * stride rows); rows [0, length) are loaded and the
 * cache length becomes `length`.  Returns 0 or a negative Yue2Error. */
int32_t yue2_hip_cache_load(Yue2Cache *c, const float *key, const float *value, int32_t length,
                            int32_t stride);
/* The reverse of yue2_hip_cache_load: rows [start, start + n) of the device
 * cache into the host K/V mirror layout (layer l, position p at row
 * l * stride + p of kv_heads * head_dim f32, the stored BF16 values exactly).
 * Replaces the `shadow` rows the reference's fast path returns per token for
 * its host mirror, so that the CPU path can take over after a failed device
 * step (src/metal.m:846-871, src/model.rs:556-566); start = length - 1,
 * n = 1 gives the newest token's rows.  Needs start + n <= length and
 * start + n <= stride; also valid after the model's free.  Returns 0 or a
 * negative Yue2Error. */
int32_t yue2_hip_cache_export(const Yue2Cache *c, float *key, float *value, int32_t start, int32_t n,
                              int32_t stride);

/* Model::forward_phase (src/model.rs:465-477): run n ids through the model,
 * appending to the cache; write the logits of the last row (vocab_size f32,
 * BF16-exact) when logits != NULL. */
int32_t yue2_hip_forward(Yue2Model *m, Yue2Cache *c, const int32_t *ids, int32_t n,
                         int32_t phase, float *logits);
/* Model::prefill_phase (src/model.rs:508-522) into an existing empty cache. */
int32_t yue2_hip_prefill(Yue2Model *m, Yue2Cache *c, const int32_t *ids, int32_t n,
                         int32_t phase, float *logits);

/* Model::prefill_phase (src/model.rs:508-522) on the matrix cores, into an
 * empty cache: the prompt goes through the layers in chunks of rows, every
 * linear a BF16 MFMA GEMM with FP32 accumulation and the attention a causal
 * flash attention over the BF16 cache.  Every BF16 rounding point of the
 * decode step is kept, but not its reduction order -- as the reference's own
 * GPU prefill (MPS GEMMs, src/tensor.rs:991-993, src/metal.m:216-237,
 * 330-361) differs from its decode GEMV -- so the cache and logits agree
 * with yue2_hip_prefill within a tolerance, not bit for bit.  head_dim 64 or
 * 128.  Returns 0 or a negative Yue2Error. */
int32_t yue2_hip_prefill_mfma(Yue2Model *m, Yue2Cache *c, const int32_t *ids, int32_t n,
                              int32_t phase, float *logits);

/* The NAR (acoustic) pathway's host weights (Model::open, src/model.rs:
 * 418-451; Layer::load nar_*, :264-269): per layer the AR layer's tensor set
 * (nar_input_layernorm, nar_self_attn.{q,k,v,o}_proj and {q,k}_norm,
 * nar_pre_mlp_layernorm, nar_mlp.*); the linears with biases, BF16 matrices
 * [out, in] and f32 biases (rounded to BF16 where used, Linear::finish):
 * vae2llm [hidden x latent], llm2vae [latent x hidden], time_embedder.mlp.0
 * [hidden x 256], time_embedder.mlp.2 [hidden x hidden]; latent_pos_embed.pe
 * [max_latent_frames x hidden] BF16; Config's latent_dim (a multiple of 64
 * here), max_latent_frames and timestep_shift (src/model.rs:45-47). */
typedef struct Yue2NarWeights {
    int32_t latent_dim, max_latent_frames;
    float timestep_shift;
    const uint16_t *vae2llm, *llm2vae, *time_in, *time_out, *latent_pos;
    const float *vae2llm_bias, *llm2vae_bias, *time_in_bias, *time_out_bias;
    const Yue2LayerWeights *layers; /* num_hidden_layers entries */
} Yue2NarWeights;

/* Uploads the NAR pathway next to the model's AR weights (replacing any
 * earlier one).  Returns 0 or a negative Yue2Error. */
int32_t yue2_hip_nar_load(Yue2Model *m, const Yue2NarWeights *w);

/* Model::velocity (src/model.rs:611-698) on the matrix cores (the stack the
 * reference hands to yue2_metal_stack, src/metal.m:429-538): `frames` latent
 * rows state [frames x latent] (BF16-exact values, as the flow-matching loop
 * keeps them) padded with a zero row on each side, vae2llm, the timestep
 * embedding of raw_t and the latent position rows, the NAR layers with
 * non-causal attention over the cache's first min(nar_cond_end, length)
 * positions (all when nar_cond_end is 0) and the rows' own keys (RoPE from
 * the cache length; the cache is not modified), the final norm and llm2vae:
 * out [frames x latent] f32.  The linears are BF16 MFMA GEMMs, so the result
 * agrees with the CPU restatement within a tolerance (as the reference's GPU
 * stack does with its CPU path), not bit for bit.  Needs cache length +
 * frames + 2 <= max_position_embeddings.  Returns 0 or a negative
 * Yue2Error. */
int32_t yue2_hip_velocity(Yue2Model *m, const Yue2Cache *c, const float *state, int32_t frames, double raw_t,
                          int32_t nar_cond_end, float *out);

/* Model::synthesize (src/model.rs:699-775), the acoustic stage: the song's
 * noise (Generator::normal_tensor of MT19937(seed), src/sampling.rs:64-79,
 * on the host), then per chunk of (min(24576, max positions) - prefix_len -
 * 3) / 2 frames the AR prefill of prefix + codec ids (+ 151853) + MUSIC_END
 * on the matrix cores and `steps` midpoint flow-matching steps, two
 * yue2_hip_velocity calls each; out [codec_len x 64].  Returns 0 or a
 * negative Yue2Error with the reference's messages. */
int32_t yue2_hip_synthesize(Yue2Model *m, const int32_t *prefix, int32_t prefix_len, const int32_t *codec,
                            int32_t codec_len, uint64_t seed, int32_t steps, float *out);

/* The VAE decoder (src/vae.rs), FP32 on the device.  Vae::open
 * (src/vae.rs:635-669) with decoder_only: config.json (model_type
 * yue2_vae, decoder_config) and the safetensors file(s) of `dir`, checked and
 * weight-normed as the reference does, with its messages.  NULL on failure. */
typedef struct Yue2Vae Yue2Vae;
Yue2Vae *yue2_hip_vae_open(const char *dir);
void yue2_hip_vae_free(Yue2Vae *v);
/* info[0..5] = sample_rate, latent_dim, audio_channels, downsampling_ratio,
 * decode_core_frames, decode_halo_frames. */
int32_t yue2_hip_vae_info(const Yue2Vae *v, int32_t *info);
/* Vae::natural_output_length (src/vae.rs:670-675): audio rows for `frames`
 * latent rows, or a negative Yue2Error. */
int64_t yue2_hip_vae_output_length(const Yue2Vae *v, int32_t frames);
/* Vae::required_halo (src/vae.rs:676-681). */
int32_t yue2_hip_vae_required_halo(const Yue2Vae *v, int32_t core);
/* Vae::decode (src/vae.rs:688-727): z [frames x latent_dim] -> out
 * [output_length x audio_channels].  The convolutions run in FP32 on the
 * device in their own summation order, so results agree with the CPU
 * restatement within FP32 rounding (a tolerance), not bit for bit.
 * Returns 0 or a negative Yue2Error. */
int32_t yue2_hip_vae_decode(Yue2Vae *v, const float *z, int32_t frames, float *out);
/* Vae::decode_tiled (src/vae.rs:729-762): core-frame tiles with `halo`
 * frames on each side (at least yue2_hip_vae_required_halo(core)). */
int32_t yue2_hip_vae_decode_tiled(Yue2Vae *v, const float *z, int32_t frames, int32_t core, int32_t halo,
                                  float *out);

/* A decode loop bound to one cache (batch 1) or to a conditional and an
 * unconditional cache (CFG batch 2).  Each step is one hipGraph launch:
 * embed -> layers -> LM head -> CFG mix -> choose -> next id.  The caches
 * must already be prefilled; `first_logits` seeds step 0 (the prefill
 * logits, rows x vocab f32, cond first).  sampling NULL means greedy argmax. */
Yue2Decoder *yue2_hip_decoder_new(Yue2Model *m, Yue2Cache *cond, Yue2Cache *uncond,
                                  const Yue2Sampling *sampling, uint64_t seed, int32_t phase,
                                  float scale, int32_t legacy);
void yue2_hip_decoder_free(Yue2Decoder *d);
/* Run `steps` token steps (choose a token, forward it).  tokens receives the
 * chosen ids; step_ms (may be NULL) the per-step device time from HIP
 * events.  Each launch forwards a token chosen before it and chooses the
 * next one, so the token after a run's last is already chosen when the run
 * returns (the next run starts with its forward).  Returns the number of
 * steps run or a negative Yue2Error.  With a phase that has an end token the
 * loop stops at the first end id: it is the last id returned, its step runs
 * no forward (src/sampling.rs:268-271), so the caches grow by one position
 * less than the steps returned, and later runs return 0. */
int32_t yue2_hip_decoder_run(Yue2Decoder *d, const float *first_logits, int32_t steps,
                             int32_t *tokens, float *step_ms);
/* The logits of the decoder's last forward, which the choice of the token
 * after it read (src/sampling.rs:261-267, before the CFG mix); before any
 * forward, the first logits.  rows x vocab f32, the conditional row first.
 * The decoder must have run. */
int32_t yue2_hip_decoder_logits(Yue2Decoder *d, float *out);

/* sampling::choose (src/sampling.rs:103-215) on the device for one row of
 * logits (already CFG-mixed).  history / history_len: the ids generated so
 * far, of which the last penalty_window set the repetition penalty; step
 * gates the end token by min_tokens; draws: the 2 * vocab MT19937 outputs
 * the call consumes, in stream order (may be NULL when temperature is 0).
 * *id receives the chosen id.  Returns YUE2_OK or a negative Yue2Error. */
int32_t yue2_hip_choose(const float *logits, int32_t vocab, const Yue2Sampling *sampling,
                        const int32_t *history, int32_t history_len, int32_t step,
                        int32_t phase, int32_t legacy, const uint32_t *draws, int32_t *id);

/* yue2_hip_choose without any device allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (tight
 * serving loops, harnesses that forbid hipMalloc).  Same arguments, checks,
 * result and errors as yue2_hip_choose; its device buffers live in one
 * file-scope scratch array per GPU (9 MiB, held until the process ends), so
 * vocab is limited to 262144 entries (YUE2_ERR_ARG beyond).  It runs on the
 * null stream.  Calls on one GPU share that array: the library lock
 * serialises them within a process, and callers must not overlap calls on
 * one GPU by other means. */
int32_t yue2_hip_choose_noalloc(const float *logits, int32_t vocab, const Yue2Sampling *sampling,
                                const int32_t *history, int32_t history_len, int32_t step,
                                int32_t phase, int32_t legacy, const uint32_t *draws, int32_t *id);

/* sampling::generate (src/sampling.rs:222-294) on the device.  Both rows are
 * prefilled (src/sampling.rs:246, 252) in decode order, bit for bit the CPU
 * path's caches and logits, unless yue2_hip_model_set_prefill chose the
 * matrix cores; then the caches and first logits follow yue2_hip_prefill_mfma's
 * tolerance contract and the loop after them is exact on those caches. */
int32_t yue2_hip_generate(Yue2Model *m, const int32_t *prefix, int32_t prefix_len,
                          const Yue2Sampling *sampling, uint64_t seed, int32_t phase,
                          const int32_t *negative, int32_t negative_len, float scale,
                          int32_t legacy, int32_t *tokens, int32_t *count, int32_t *truncated);

/* Message of the last failure on this thread ("" if none). */
const char *yue2_hip_last_error(void);
/* Wait for all device work issued by the library. */
int32_t yue2_hip_synchronize(void);

/* ---------------------------------------------------------------------- */
/* Support entry points (no counterpart in the reference)                  */
/* ---------------------------------------------------------------------- */

/* Synthetic checkpoint values: BF16 ~ N(0, stddev) from a counter-based
 * generator (SplitMix64 + Box-Muller with the library's own log/sin/cos), so
 * every machine produces the same bits.  Replaces the real checkpoint, which
 * the reference downloads (src/checkpoint.rs:16-161).  threads <= 0: all. */
void yue2_hip_synthetic_bf16(uint16_t *out, size_t n, uint64_t seed, uint64_t tensor,
                             float stddev, int32_t threads);

/* Diagnostics: evaluate a device math routine elementwise on host arrays
 * (which: 0 exp f32, 1 log1p f64, 2 round_bf16, 3 SiLU), or, per 64-lane
 * wave of f32 inputs (n a multiple of 256), a lane exchange: 4-9 the value of
 * lane ^ 1, 2, 4, 8, 16, 32; the xor-butterfly sums over distances 32..1
 * (10 ALU exchanges, 11 __shfl_xor), 8..1 (12, 13) and 32..16 (14, 15); 16
 * the max over 32..1; 17 the RMSNorm scale (eps 1e-6) of each consecutive
 * 64-value vector, decided by one wave (stored on all 64 of its outputs);
 * 18 the RMSNorm scales of the two 128-value rows of each 256-value block,
 * decided together by a 256-thread block (each row's outputs hold its
 * scale).  Returns 0 or a negative Yue2Error. */
int32_t yue2_hip_selftest_math(int32_t which, const void *in, void *out, size_t n);
/* Diagnostics: out = x W^T (M x N f32, the raw FP32 accumulation) through
 * the prefill's BF16 MFMA GEMM; x [M, K] and w [N, K] BF16 host arrays, K a
 * multiple of 64.  Returns 0 or a negative Yue2Error. */
int32_t yue2_hip_selftest_gemm(const uint16_t *x, const uint16_t *w, float *out, int32_t M, int32_t N,
                               int32_t K);
/* Diagnostics: one convolution through the VAE's device kernel, w in the
 * checkpoint layout ([out, in, k], or [in, out, k] transposed; no weight
 * norm), bias [cout] or NULL, x [frames x cin] -> out [length x cout]
 * (Conv::length, src/vae.rs:147-153).  Returns 0 or a negative Yue2Error. */
int32_t yue2_hip_selftest_conv(int32_t transpose, int32_t cin, int32_t cout, int32_t kernel, int32_t stride,
                               int32_t padding, int32_t dilation, const float *x, int32_t frames, const float *w,
                               const float *bias, float *out);
/* Execution choice: run decode steps (yue2_hip_forward and decoders created
 * afterwards) through the persistent token-step kernel -- one launch per
 * token, workgroups exchanging tagged words instead of meeting at barriers
 * -- or through one kernel per phase.  Both produce the same bits.  The
 * step kernel is the default for shapes that have one: head_dim 64 or 128,
 * at most 8 query heads per KV head, hidden and heads * head_dim at most
 * 4608 and intermediate at most 14336 (the 3B-class and YuE2 shapes on
 * kernels of their own, the others on generic ones), contexts up to 24576.
 * Returns 1 when enabled, 0 when off or when the model's shape has no step
 * kernel. */
int32_t yue2_hip_model_set_step_kernel(Yue2Model *m, int32_t on);
/* Execution choice for yue2_hip_generate's prefill of the prompts (on = 1):
 * yue2_hip_prefill_mfma (BF16 MFMA GEMMs and flash attention; a 2048-token
 * 3B-class prompt in ~20 ms, agreeing with the decode-order prefill within
 * its stated tolerance, not bit for bit -- as the reference's GPU prefill,
 * MPS GEMMs, src/tensor.rs:991-993, differs from its CPU path) or, the
 * default, the decode-order prefill (bit-exact, ~650 tokens/s).  Returns the
 * setting now in force (1 or 0). */
int32_t yue2_hip_model_set_prefill(Yue2Model *m, int32_t mfma);
/* Diagnostics: advance the launch sequence of the model's own workspace (the
 * one yue2_hip_forward uses) by `add`, as if that many step-kernel launches
 * had run.  The step kernel's tagged words carry a 20-bit epoch of this
 * sequence; the library clears them before an epoch could repeat, and this
 * entry lets a test place launches at that point.  The model must have run a
 * step-kernel forward. */
int32_t yue2_hip_model_advance_sequence(Yue2Model *m, int32_t add);
/* Diagnostics: RMSNorm guard fallbacks taken since the model was opened. */
int32_t yue2_hip_norm_fallbacks(const Yue2Model *m);

/* Diagnostics: time one of the decoder's own kernels with HIP events on the
 * decoder's stream, cycling through the layers so that no launch finds its
 * weights in the last-level cache.  kernel: 0 gate/up GEMV with the SwiGLU
 * epilogue, 1 down GEMV, 2 fused QKV GEMV, 3 O GEMV, 4 LM-head GEMV, 5 the
 * persistent step kernel (whole token, at the decoder's current position).
 * avg_ms = mean launch duration; bytes = algorithmic HBM bytes per launch.
 * The decoder must have run at least one step. */
int32_t yue2_hip_decoder_time_kernel(Yue2Decoder *d, int32_t kernel, int32_t iters, float *avg_ms,
                                     double *bytes);

/* Diagnostics: one decode step of token `id` at the cache's next position
 * through the persistent token-step kernel (appends to the cache like
 * yue2_hip_forward, computes no logits; with `c2` non-NULL, a batch-2 step
 * of the same id over both caches), recording the device wall clock
 * (100 MHz) per workgroup: stamps[s * wgs + w] for slot s = 0 at the start,
 * then per layer 15 slots -- QKV start, QKV end, attention: queries gathered,
 * new key appended, block maxima stored, maxima gathered, sums gathered,
 * partials stored, attention end; O start, O end, gate/up start, gate/up
 * end, down start, down end.  cap = entries available in stamps; *wgs and
 * *slots receive the trace shape.  YUE2_ERR_ARG when the shape has no step
 * kernel or cap is too small. */
int32_t yue2_hip_trace_step(Yue2Model *m, Yue2Cache *c, Yue2Cache *c2, int32_t id, uint64_t *stamps,
                            int32_t cap, int32_t *wgs, int32_t *slots);

/* Microbenchmarks against the HBM roofline (device-resident inputs; each
 * timed launch reads another copy of its operands, so the 256 MB Infinity
 * Cache cannot serve repeats).
 * yue2_hip_bench_gemv: the BF16 GEMV y = W x (W [n x k], `rows` batch rows,
 * FP32 accumulation, rounded output) over `copies` weight copies; *avg_ms =
 * mean launch time over `iters` launches, *bytes = n k 2 + rows k 2 +
 * rows n 4 (the weights, BF16 inputs and f32 outputs).
 * yue2_hip_bench_attention: the per-phase split-KV decode attention of one
 * layer (24 query heads, 8 KV heads, head_dim 128, QK-norm + RoPE + KV
 * append included) for `rows` rows whose new token attends `context`
 * positions, cycling over `layers` distinct layer caches (the step sequence
 * advanced after each pass over them, as after a decode step); *bytes =
 * rows 4096 context (the K and V rows read).
 * yue2_hip_bench_copy: hipMemcpyAsync of `bytes` (a multiple of 256) from
 * one device buffer to another, once untimed and then `iters` times;
 * *avg_ms = mean time per copy (each reads and writes `bytes`).
 * yue2_hip_bench_gemm: the prefill's BF16 MFMA GEMM C = X W^T (X [M x K],
 * W [N x K], K a multiple of 64, f32 rounded output; pair != 0: the
 * gate/up pair, W and a second [N x K] matrix with the SwiGLU epilogue),
 * once untimed and then `iters` times; *flops = 2 M K x (weight rows).
 * All return 0 or a negative Yue2Error. */
int32_t yue2_hip_bench_gemv(int32_t n, int32_t k, int32_t rows, int32_t copies, int32_t iters, float *avg_ms,
                            double *bytes);
int32_t yue2_hip_bench_attention(int32_t context, int32_t rows, int32_t layers, int32_t iters, float *avg_ms,
                                 double *bytes);
int32_t yue2_hip_bench_copy(int64_t bytes, int32_t iters, float *avg_ms);
int32_t yue2_hip_bench_gemm(int32_t M, int32_t N, int32_t K, int32_t pair, int32_t iters, float *avg_ms,
                            double *flops);

#ifdef __cplusplus
}
#endif
#endif
