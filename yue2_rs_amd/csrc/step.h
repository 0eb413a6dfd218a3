// step.h -- launch interface of the persistent token-step kernel (internal).
#pragma once
#include <hip/hip_runtime.h>

#include "kernels.h"
#include "runtime.h"

namespace y2 {

struct StepArgs {
    const LayerDev* layers;  // device array of layers_n layers
    const uint16_t* embed;
    const uint16_t* lm_head;
    const float* final_norm;
    int layers_n, hidden, intermediate, vocab, heads, kv_heads, rows;
    int head;                // 1: final norm + full-vocabulary LM head into logits
    float eps;
    float *x, *qkv, *att, *act, *logits;
    int* bars;               // two grid-barrier counters, zero at first use
    AttnArgs attn;           // per-layer fields (layer, norms) are filled in the kernel
    StepState* st;
    unsigned long long* trace;  // optional wall-clock stamps, kTraceSlotsPerLayer per layer + 1
    int trace_slots;
};

// Trace slots: one at the start, then per layer the start of each GEMV (4)
// and the arrival at / departure from each grid barrier (5 x 2).
constexpr int kTraceSlotsPerLayer = 14;

// True when a compiled step kernel covers this shape on nwg workgroups.
bool step_supported(const Yue2Config& c, int rows, int nwg);
hipError_t launch_step(hipStream_t s, const StepArgs& a, int nwg);

}  // namespace y2
