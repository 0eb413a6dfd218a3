// step.h -- launch interface of the persistent token-step kernel (internal).
#pragma once
#include <hip/hip_runtime.h>

#include "kernels.h"
#include "runtime.h"

namespace y2 {

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
    StepState* st;
};

// Per-launch arguments.
struct StepCall {
    KvView kv;
    int head;                   // 1: final norm + full-vocabulary LM head into logits
    int trace_slots;
    unsigned long long* trace;  // optional wall-clock stamps, kTraceSlotsPerLayer per layer + 1
};

// Trace slots: one at the start, then per layer: QKV start, QKV end,
// six inside the attention (queries gathered, new key appended, block maxima
// stored, maxima gathered, sums gathered, partials stored), attention end,
// O start, O end, gate/up start, gate/up end, down start, down end.
constexpr int kTraceSlotsPerLayer = 15;

// True when a compiled step kernel covers this shape on nwg workgroups.
bool step_supported(const Yue2Config& c, int rows, int nwg);
// Dynamic LDS bytes of the step kernel for these arguments on nwg
// workgroups; launches need at most kStepLdsMax.
constexpr size_t kStepLdsMax = 128 * 1024;
size_t step_lds_bytes(const StepArgs& a, int nwg);
// Workgroups of the step kernel for these arguments that fit on one CU at
// once (its registers and dynamic LDS); the launch needs at least 1, since
// its workgroups wait for each other's outputs.
int step_resident_per_cu(const StepArgs& a, int nwg);
hipError_t launch_step(hipStream_t s, const StepArgs* dev_args, const StepArgs& host_args,
                       const StepCall& call, int nwg);

}  // namespace y2
