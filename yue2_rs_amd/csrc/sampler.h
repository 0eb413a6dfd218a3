// sampler.h -- on-device token selection (internal).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernels.h"

namespace y2 {

struct MtState {
    uint32_t state[624];
    int32_t next;
};

struct SampleArgs {
    const float* logits;  // [rows][vocab]; row 1 is the unconditional row
    float* scores;        // [vocab] scratch
    const uint32_t* stream[2];  // 2 * vocab MT19937 outputs, double-buffered by step parity
    int32_t* token_log;   // generated ids (the penalty history)
    StepState* st;
    int rows, vocab, phase, end_id, mode;  // mode 0: argmax of the mixed logits; 1: choose()
    float cfg_scale, temperature, top_p, repetition_penalty;
    int top_k, window, min_tokens, legacy;
};

void launch_choose(hipStream_t s, const SampleArgs& a);
void launch_mt_generate(hipStream_t s, MtState* mt, uint32_t* out0, uint32_t* out1, size_t count,
                        const StepState* st, int ahead);

}  // namespace y2
