// runtime.h -- internal types shared by the runtime, the decoder and the
// reference twins.
#pragma once
#include <hip/hip_runtime.h>

#include <mutex>
#include <string>
#include <vector>

#include "../../include/yue2_hip.h"
#include "kernels.h"

namespace y2 {

// Protocol ids (src/protocol.rs:6-16).
constexpr int kEod = 151643;
constexpr int kAbcEnd = 151848;
constexpr int kMusicEnd = 151852;
constexpr int kCodecOffset = 151853;
constexpr int kCodecSize = 32768;
constexpr int kContext = 24576;

struct StepState;
void launch_reset_state(hipStream_t s, StepState* st, int32_t* c0 = nullptr, int n0 = 0,
                        int32_t* c1 = nullptr, int n1 = 0);
// st->seq = value (set != 0) or st->seq += value.
void launch_sequence(hipStream_t s, StepState* st, int set, int value);

// The step kernel's tagged words carry a 20-bit epoch (launch sequence + 1).
// Launches between two clears of the words must stay below this count, so
// that no word left by an earlier launch can carry a later launch's tag.
constexpr int64_t kEpochLaunches = (int64_t)1 << 20;

struct LayerDev {
    uint16_t *wqkv, *wo, *wg, *wu, *wd;
    float *in_norm, *q_norm, *k_norm, *post_norm;
};

// Activations and attention scratch for one batch size.
struct Workspace {
    int rows = 0, max_blocks = 0, blk_stride = 0, log_cap = 0, counter_n = 0;
    void* block = nullptr;
    float *x = nullptr, *h = nullptr, *qkv = nullptr, *att = nullptr, *act = nullptr;
    float *logits = nullptr, *mixed = nullptr;
    float *bmax = nullptr, *bsum = nullptr, *part = nullptr;
    int32_t* counters = nullptr;  // attention group counters, zero between launches
    int32_t* bars = nullptr;      // two grid-barrier counters of the step kernel
    StepState* st = nullptr;
    int32_t* token_log = nullptr;
    void* step_args = nullptr;  // device copy of the step kernel's arguments
    void* flow_block = nullptr; // tagged-word buffers: the step kernel's, the per-phase attention's
    size_t flow_words = 0;      // 64-bit words in flow_block
    uint64_t *tbmax = nullptr, *tbsum = nullptr, *tpart = nullptr;  // in flow_block
    void* step_host = nullptr;  // host copy of the same (StepArgs)
    bool step_args_ready = false;
    int step_sample = 0;        // the step arguments carry a fused sampler
    // Upper bound of the launch-sequence increments since the tagged words
    // were last cleared (each reset adds 2, each step-kernel launch or
    // per-phase step 1).
    int64_t seq_bound = 0;
    int ensure(int rows, int max_blocks, const Yue2Config& c);
    // Clear the step state and every sync counter (stream-ordered).
    void reset(hipStream_t s) {
        launch_reset_state(s, st, counters, counter_n, bars, 2);
        seq_bound += 2;
    }
    // Before a reset and n step-kernel launches on stream s: when they could
    // reach kEpochLaunches since the last clear, clear the tagged words and
    // restart the sequence at 0 (stream-ordered, no allocation).
    void reserve_launches(hipStream_t s, int64_t n);
    void release();
    Workspace() = default;
    Workspace(const Workspace&) = delete;
    Workspace& operator=(const Workspace&) = delete;
    ~Workspace();
};

}  // namespace y2

namespace y2 {
// The NAR (acoustic) pathway's device weights (yue2_hip_nar_load): one
// allocation; the layers as LayerDev (fused q/k/v rows), the linears' biases
// BF16-rounded f32.
struct NarDev {
    void* block = nullptr;
    int latent = 0, max_frames = 0;
    float shift = 1.0f;
    std::vector<LayerDev> layers;
    uint16_t *vae2llm = nullptr, *llm2vae = nullptr, *time_in = nullptr, *time_out = nullptr,
             *latent_pos = nullptr;
    float *vae2llm_b = nullptr, *llm2vae_b = nullptr, *time_in_b = nullptr, *time_out_b = nullptr;
};
}  // namespace y2

struct Yue2Model {
    Yue2Config c{};
    hipStream_t stream = nullptr;
    void* block = nullptr;
    size_t block_bytes = 0;
    uint16_t *embed = nullptr, *lm_head = nullptr;
    float *final_norm = nullptr, *rope_cos = nullptr, *rope_sin = nullptr;
    std::vector<y2::LayerDev> layers;
    y2::LayerDev* layers_dev = nullptr;  // the same table in device memory (step kernel)
    int cus = 0;                         // compute units: workgroups of the step kernel
    bool step_kernel = false;            // decode steps through the persistent kernel (default where supported)
    bool prefill_mfma = false;           // yue2_hip_generate prefills on the matrix cores
    y2::Workspace ws;  // batch-1 workspace of the parity API
    int norm_fallbacks = 0;
    y2::NarDev nar;    // loaded by yue2_hip_nar_load
    // The live caches and decoders made on this model.  yue2_hip_model_free
    // detaches them: a decoder's device objects are released, a cache keeps
    // its KV memory (and its shape, so it can still be exported) until its
    // own free, and neither reaches the model again.  So the three may be
    // freed in any order, as the reference lets a Cache outlive its Model
    // (src/model.rs:286-290).
    std::vector<Yue2Cache*> caches;
    std::vector<Yue2Decoder*> decoders;
};

struct Yue2Cache {
    Yue2Model* m = nullptr;  // null once the model has been freed
    int capacity = 0;
    int length = 0;
    int layers = 0, kv_heads = 0, head_dim = 0;  // the model's shape, kept past its free
    uint16_t* kv = nullptr;
};

namespace y2 {

std::recursive_mutex& library_lock();
int fail(int code, const std::string& msg);
int hip_fail(hipError_t e, const char* what);
bool device_ready();
int enqueue_step(Yue2Model* m, Workspace& w, const KvView& kv, int rows, bool head, int phase,
                 hipStream_t s);
// The final norm and the phase's LM head of `rows` rows x (stride hidden)
// into w.logits (Model::forward_phase's projection, src/model.rs:469-507).
int enqueue_head(Yue2Model* m, Workspace& w, const float* x, int phase, hipStream_t s, int rows = 1);
// The same step as one persistent kernel when the shape has one (full
// vocabulary head only); returns 1 when it cannot be used.  sample: the
// fused sampler's mode (StepCall::sample); the workspace must have been
// prepared with a sampler for a nonzero mode.
int enqueue_step_fused(Yue2Model* m, Workspace& w, const KvView& kv, int rows, bool head, int phase,
                       hipStream_t s, unsigned long long* trace = nullptr, int trace_slots = 0,
                       int sample = 0, int context = 0);
// Upload the workspace's step kernel arguments (synchronous; call after
// Workspace::ensure and before capturing a graph), with the fused sampler
// when smp is set.  1 when the shape (or the launch with a sampler) has no
// resident step kernel.
struct FusedSampler;
int prepare_step(Yue2Model* m, Workspace& w, const FusedSampler* smp = nullptr);
void phase_range(int phase, int* start, int* end, int* stop);
// The LM-head rows of a phase: [lo, lo + n) and the stop row (-1: none).
void head_rows(int phase, int vocab, int* lo, int* n, int* stop);
int phase_end_id(int phase);
int check_phase_vocab(int phase, int vocab);
int read_step_error(Workspace& w, hipStream_t s);
// The error a step state carries (YUE2_OK when none), with its message set.
int step_error(const StepState& st);

// Release a decoder's device objects and detach it from its model and caches
// (decoder.hip); later calls on it fail with YUE2_ERR_ARG.  The caller holds
// the library lock and has synchronised the model's stream.
void decoder_detach(Yue2Decoder* d);
// Whether decoder d runs on cache c.
bool decoder_uses(const Yue2Decoder* d, const Yue2Cache* c);

// Small state kernels (kernels.hip).
void launch_fill(hipStream_t s, float* p, size_t n, float v);
void launch_set_state(hipStream_t s, StepState* st, int rows, int pos0, int pos1, int id0, int id1);

}  // namespace y2
