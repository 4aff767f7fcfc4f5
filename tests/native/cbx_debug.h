/* cbx_debug.h -- test-only diagnostics of the sampler's device building
 * blocks (tests/native/_build/libcbx_debug.so, built from
 * tests/native/cbx_debug.hip; not part of libcbx_sampler.so or its API).
 * Device memory, asynchronous on `stream`; `device` is made current for the
 * launch.  Return codes as in cbx_sampler.h. */
#ifndef CBX_DEBUG_H
#define CBX_DEBUG_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* The device exponential the sampler uses (the glibc expf algorithm restated
 * for the GPU), elementwise. */
int cbx_debug_expf(int32_t device, const float* in, float* out, int64_t n, void* stream);
/* The device Philox uniforms for (seed, stream_ids[i] or i, step). */
int cbx_debug_philox(int32_t device, uint64_t seed, const uint64_t* stream_ids, uint64_t step,
                     int32_t n, double* out, void* stream);
/* The workgroup kernel's exact left-to-right binary32 running sums: case c
 * sums terms[offsets[c] .. offsets[c+1]) (finite, >= 0, 1 to 8192 of them)
 * from 0 into sum[c]; when thr is given and thr[c] > 0, hit[c] is the first
 * index (from the case's start) whose running sum is >= thr[c], else -1.
 * desc (optional): desc[c] != 0 marks a case whose terms do not increase
 * (the sums may then stop early). */
int cbx_debug_runsum(int32_t device, const float* terms, const int32_t* offsets, const float* thr,
                     const uint8_t* desc, int32_t n_cases, float* sum, int32_t* hit,
                     void* stream);
/* The same sums and threshold indices by the one-wavefront kernel's
 * evaluation (per-lane runs, DPP sweep chains or binade segments); 1 to 1088
 * terms per case; the case's sum starts from 0. */
int cbx_debug_chainsum(int32_t device, const float* terms, const int32_t* offsets,
                       const float* thr, int32_t n_cases, float* sum, int32_t* hit, void* stream);

#ifdef __cplusplus
}
#endif
#endif
