// step.h -- launch interface of the persistent token-step kernel (internal).
#pragma once
#include <hip/hip_runtime.h>

#include "kernels.h"
#include "runtime.h"
#include "sampler.h"

namespace y2 {

// The sampler of a decode loop inside the step kernel (StepCall::sample):
// the step kernel's last workgroup generates the step's MT19937 draws and
// then finishes choose() for the next token, while the other workgroups
// (the workers) score their own rows of the LM head and each publishes its
// best `list` entries.
struct FusedSampler {
    SampleArgs a;      // settings; a.logits = the step's logits, a.scores its tempered scores
    MtState* mt;       // the stream's state (advanced by live launches)
    uint32_t* draws;   // [2 * vocab] the draws of the token being chosen
    uint64_t* cand;    // [workers][list] each worker's best order keys
    int list;          // top_k, or 1 for greedy
};
// Most candidates per worker, and most vocabulary rows per worker (the
// workers sort their rows in LDS).
constexpr int kFusedListMax = 64;
constexpr int kFusedRowsMax = 1024;
// Dynamic LDS the sampler workgroup needs.
constexpr size_t kSamplerLds = 64 * 1024;
// Most workgroups of a step-kernel launch (the sampler's words per worker).
constexpr int kStepThreadsMax = 512;

// Launch-invariant arguments of a workspace's step kernel, kept in device
// memory (the kernel re-reads fields with scalar loads where it uses them,
// instead of holding all of them in registers for the whole launch).
struct StepArgs {
    const LayerDev* layers;  // device array of layers_n layers
    const uint16_t* embed;
    const uint16_t* lm_head;
    const float* final_norm;
    const float *rope_cos, *rope_sin;  // [positions][head_dim / 2]
    int layers_n, hidden, intermediate, vocab, heads, kv_heads, head_dim, rows;
    int blk_stride, max_blocks;
    float eps, scale;
    float* logits;  // [rows][vocab]
    // tagged words (dev_flow.h): x, q/k/v, attention output, SwiGLU output,
    // attention block maxima / sums [rows][heads][blk_stride] and partial PV
    // [rows][heads][blk_stride][head_dim]
    uint64_t *tx, *tqkv, *tatt, *tact, *tbmax, *tbsum, *tpart;
    uint64_t* tsmp;  // [workers] tagged {finite entries | invalid flag << 31} of the fused sampler
    StepState* st;
    FusedSampler smp;  // the fused sampler (when a call enables it)
};

// Per-launch arguments.
constexpr int kOEarlyKeys = 4096;

struct StepCall {
    KvView kv;
    // 1: final norm + LM head into logits: rows [head_lo, head_lo + head_n)
    // and, when head_stop >= 0, that row too; every other logit is -inf
    // (project_phase, src/model.rs:478-507; the full vocabulary is rows
    // [0, vocab) without a stop row)
    int head;
    int head_lo, head_n, head_stop;
    // 0: no sampler; 1: the fused sampler chooses the next token and advances
    // the state (ids, token log, positions, step, MT state); 2: the same work
    // without publishing anything (timing).  With a sampler the last
    // workgroup is the sampler and the others share the layers.
    int sample;
    // the most keys a row of the launch attends (0: unknown); from
    // kOEarlyKeys on, the kernel requests the O projection's first weights
    // during the attention (same arithmetic, another schedule)
    int context;
    int trace_slots;
    unsigned long long* trace;  // optional wall-clock stamps, kTraceSlotsPerLayer per layer + 1
};

// Trace slots: one at the start, then per layer: QKV start, QKV end,
// six inside the attention (queries gathered, new key appended, block maxima
// stored, maxima gathered, sums gathered, partials stored), attention end,
// O start, O end, gate/up start, gate/up end, down start, down end.
constexpr int kTraceSlotsPerLayer = 15;

// True when a compiled step kernel covers this shape with nwg workgroups
// sharing the layers (the launch's workgroups, less the sampler's).
bool step_supported(const Yue2Config& c, int rows, int nwg);
// True when the fused sampler can serve this decoder on a launch of nwg
// workgroups (nwg - 1 workers): the shape has a step kernel for the
// workers, and the settings fit its candidate lists.
bool fused_sampler_supported(const Yue2Config& c, int rows, int nwg, int mode, float temperature, int top_k,
                             int head_n);
// Dynamic LDS bytes of the step kernel for these arguments on nwg
// workgroups; launches need at most kStepLdsMax.
constexpr size_t kStepLdsMax = 128 * 1024;
size_t step_lds_bytes(const StepArgs& a, int nwg);
// Dynamic LDS bytes of a launch of nwg workgroups (with or without the
// fused sampler).
size_t step_launch_lds(const StepArgs& a, int nwg, int sample);
// Workgroups of the step kernel for these arguments that fit on one CU at
// once (its registers and dynamic LDS); the launch needs at least 1, since
// its workgroups wait for each other's outputs.
int step_resident_per_cu(const StepArgs& a, int nwg, int sample);
hipError_t launch_step(hipStream_t s, const StepArgs* dev_args, const StepArgs& host_args,
                       const StepCall& call, int nwg);

}  // namespace y2
