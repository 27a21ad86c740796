// Arguments of the device sampler (kernels in sample.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>

namespace fl {

// Which rule picks the token (the priority of Generator::step,
// flare-core/src/generate.rs:220-230): greedy when the temperature is 0, else
// top-p when top_p < 1, else min-p when min_p > 0, else top-k when top_k > 0,
// else top-p with p = 1.
enum SampleMode { SM_GREEDY = 0, SM_TOP_P = 1, SM_MIN_P = 2, SM_TOP_K = 3 };

struct SampleArgs {
    const float *logits;  // [n] device
    int n;
    float *p;             // [n] work row: penalized / scaled logits, then probabilities
    int *counts;          // [n] occurrence counts, zero on entry and on exit
    const int *prev;      // [n_prev] previous tokens (repeat penalty)
    int n_prev;
    float penalty, temperature, top_p, min_p;
    int mode;
    int K;                // top-p: min(512, n); top-k: max(1, min(top_k, n))
    float u;              // the caller's uniform draw (rng_val)
    int exact;            // sums in the reference's sequential order
    unsigned *keys;       // [n] large sets: probability bits (0 = not a candidate)
    int *vals;            // [n] large sets: token index
    const unsigned *skeys;  // [n] sorted descending
    const int *svals;
    int *state;           // [0] token, [1] large-set size, [2] large set pending, [3] greedy token
};

size_t sample_sort_bytes(int n);
hipError_t launch_sample(hipStream_t st, const SampleArgs &a, void *sort_tmp, size_t sort_bytes);

}  // namespace fl
