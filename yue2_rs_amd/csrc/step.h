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
    int layers_n, hidden, intermediate, vocab, heads, kv_heads, rows;
    float eps;
    float *x, *qkv, *att, *act, *logits;
    int* bars;               // two grid-barrier counters, zero at first use
    AttnArgs attn;           // kv, layer and norms are filled in per call / per layer
    StepState* st;
};

// Per-launch arguments.
struct StepCall {
    KvView kv;
    int head;                   // 1: final norm + full-vocabulary LM head into logits
    int trace_slots;
    unsigned long long* trace;  // optional wall-clock stamps, kTraceSlotsPerLayer per layer + 1
};

// Trace slots: one at the start, then per layer the start of each GEMV (4)
// and the arrival at / departure from each grid barrier (5 x 2).
constexpr int kTraceSlotsPerLayer = 14;

// True when a compiled step kernel covers this shape on nwg workgroups.
bool step_supported(const Yue2Config& c, int rows, int nwg);
// Dynamic LDS bytes of the step kernel for these arguments.
size_t step_lds_bytes(const StepArgs& a);
hipError_t launch_step(hipStream_t s, const StepArgs* dev_args, const StepArgs& host_args,
                       const StepCall& call, int nwg);

}  // namespace y2
