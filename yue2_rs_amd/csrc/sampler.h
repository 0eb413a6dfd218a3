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

// Vocabulary entries scored by one workgroup of the chunked selection.
constexpr int kChooseChunk = 1024;
// Most candidates the finishing workgroup holds (chunks * list entries).
constexpr int kChooseCandMax = 16384;
// Most chunks the finishing workgroup scans (one per thread).
constexpr int kChooseChunksMax = 1024;

struct SampleArgs {
    const float* logits;  // [rows][vocab]; row 1 is the unconditional row
    float* scores;        // [vocab] scratch
    const uint32_t* stream[2];  // 2 * vocab MT19937 outputs, double-buffered by step parity
    const int32_t* history;     // generated ids (the penalty history)
    int hist_len;               // history length; -1: the step index of the token chosen
    // the token chosen is number st->step + step_offset of the loop (1 when
    // the choice follows the step's forward in the same launch sequence)
    int step_offset;
    int32_t* token_log;         // when set, the chosen id is stored at [step]
    StepState* st;
    int rows, vocab, phase, end_id, mode;  // mode 0: argmax of the mixed logits; 1: choose()
    float cfg_scale, temperature, top_p, repetition_penalty;
    int top_k, window, min_tokens, legacy;
    // chunked selection: per chunk, its first `list` entries in score order
    // ([chunks][list]) and {finite entries, invalid-logit flag}; null cand
    // selects the single-workgroup kernel
    uint64_t* cand;
    int2* meta;
    int chunks, list;
    // survivors beyond the LDS capacity (any count up to the vocabulary):
    // order keys [big_cap] (big_cap = vocabulary rounded up to a power of
    // two, the sort's padding), their exponentials and probabilities [vocab]
    uint64_t* big;
    float *big_e, *big_p;
    int big_cap;
};

// Entries of SampleArgs::big for a vocabulary: the next power of two >= vocab.
int survivor_capacity(int vocab);
// Bytes of the three survivor overflow arrays for a vocabulary.
size_t survivor_bytes(int vocab);
// Point a's overflow arrays into `base` (survivor_bytes(vocab) bytes, 8-byte
// aligned).
void set_survivor_buffers(SampleArgs& a, void* base, int vocab);

// Length of each chunk's candidate list for these settings, or 0 when the
// single-workgroup kernel has to run (top-k too large for the chunked path).
int choose_list_len(int vocab, int mode, float temperature, int top_k);
void launch_choose(hipStream_t s, const SampleArgs& a);
void launch_mt_generate(hipStream_t s, MtState* mt, uint32_t* out0, uint32_t* out1, size_t count,
                        const StepState* st, int ahead);

}  // namespace y2
