/*
 * dendrite_testdata.h — seeded synthetic inputs for the tests and
 * benchmarks of the paged tree-decode attention backend.
 *
 * Not part of the backend: these functions live in a library of their own
 * (libdendrite_testdata.so, host code only) and have no counterpart in the
 * reference.  They let the tests, the benchmark and the CPU oracle build
 * identical inputs.  Normals come from a SplitMix64 counter hash and
 * Box-Muller in double precision, so a value depends only on (seed, index):
 * any subset of a pool can be generated independently and in parallel.
 * FP8 encodings follow the OCP FP8 (E4M3 "FN") and OCP MX v1.0 (E8M0 scale)
 * specifications.  Status codes and format / dtype codes are those of
 * dendrite_hip.h; dh_testdata_last_error() describes the last failure of a
 * call on the calling thread.
 */
#ifndef DENDRITE_TESTDATA_H
#define DENDRITE_TESTDATA_H

#include <stdint.h>

#include "dendrite_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

const char* dh_testdata_last_error(void);

/* N(0,1) sample `index` of stream `seed`: a pure function of (seed, index). */
double dh_synth_normal(uint64_t seed, uint64_t index);

/* out[i] = N(seed, first + i) converted to `dtype` (dh_dtype, round to nearest
 * even), n elements, host memory, multithreaded. */
dh_status dh_synth_fill(void* out, uint32_t dtype, uint64_t seed, uint64_t first, uint64_t n);

/* Fill whole pool pages on the host in the pool layout for format `kv_format`:
 * page i of the output receives page_ids[i]'s content, a pure function of
 * (seed, page id): K/V ~ N(0,1), then
 *   F32/BF16/F16 : rounded to the element type;
 *   FP8_E4M3     : scale = amax/448 per (page, K|V, head) (1 if amax = 0),
 *                  element = E4M3 RNE of x/scale, saturated to +-448;
 *   MXFP8        : every `outlier_every`-th element (0 = none) replaced by
 *                  +-outlier; per 32-group scale 2^(floor(log2 amax) - 8)
 *                  (E8M0, amax = 0 -> 2^-127), E4M3 RNE saturated.
 * data: n * page_bytes, scales: n * scale_bytes (may be NULL if none). */
dh_status dh_synth_pages(uint32_t kv_format, uint32_t num_kv_heads, uint32_t head_dim, uint64_t seed,
                         const uint32_t* page_ids, uint32_t n, double outlier, uint32_t outlier_every,
                         void* data, void* scales);

#ifdef __cplusplus
}
#endif
#endif /* DENDRITE_TESTDATA_H */
