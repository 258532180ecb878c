// sample.h -- next-token choice on the device (internal).
//
// Restates the caller-side sampler choose_token (moonlight_chat.c:96-131) over
// logits already resident in HBM, so a decode step can end in a token id
// instead of a 655 KB logits copy and a host qsort of 163,840 candidates.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mlh {

// Device work buffers of the sampler for one vocabulary size (allocated once
// per session, on first use).
struct SampleWork {
    int vocab = 0;
    int blocks = 0;  // workgroups of the element-wise passes
    float *probs = nullptr;
    // rank keys ~bits(p) & 0x3fffffff: ascending key is descending p
    uint32_t *keys = nullptr;
    float *part_v = nullptr;
    int *part_i = nullptr;
    double *part_sum = nullptr;
    // ctl[2] non-finite flag, ctl[3] chosen token (ctl[0..1] unused)
    int *ctl = nullptr;
    // selection scratch: histograms, candidate lists, round thresholds
    void *select = nullptr;
};

int sample_alloc(SampleWork *w, int vocab);
void sample_free(SampleWork *w);

// Enqueues the choice on `stream`.  temperature <= 0: greedy (first index of
// the maximum).  Otherwise u in [0, 1) is the caller's draw (random_unit,
// moonlight_chat.c:89-94).  The result is w->ctl[2] (non-zero: the logits or
// probabilities were not finite) and w->ctl[3] (the token), as two adjacent
// ints for one 8-byte copy.
int sample_enqueue(SampleWork *w, const float *logits, float temperature, float top_p,
                   double u, hipStream_t stream);

}  // namespace mlh
