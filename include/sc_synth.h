/*
 * sc_synth.h -- seeded synthetic inputs for the benchmark configurations.
 *
 * No counterpart in the reference: its demos fill B with unseeded rand()
 * (example_cuda/spmm_demo_gpu.cu:57-61) and read A from .mtx files.  These
 * generators make the same A, B and x on every machine (splitmix64-seeded
 * xoshiro256**, Box-Muller in double), so results and timings of the GPU
 * box can be reproduced here.
 */
#ifndef SC_SYNTH_H
#define SC_SYNTH_H

#include <stdint.h>

#include "sc_api.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Exactly round(density*m*n) nonzeros at uniformly random distinct
 * positions, values fp32(N(0, sigma^2)), never 0. */
int sc_synth_uniform(int32_t m, int32_t n, double density, double sigma, uint64_t seed,
                     sc_csr **out);
/* Non-overlapping aligned 1x8 row vectors and 4x4 blocks (fair coin per
 * placement) until nnz reaches round(density*m*n) (at most 15 over).
 * m % 4 == 0, n % 8 == 0. */
int sc_synth_blocks(int32_t m, int32_t n, double density, double sigma, uint64_t seed,
                    sc_csr **out);
/* count fp32 values (2u - 1) with u a 24-bit uniform: exact, in [-1, 1). */
int sc_synth_dense(float *out, int64_t count, uint64_t seed);
/* First `count` raw outputs of the generator seeded with `seed`. */
int sc_synth_raw(uint64_t seed, uint64_t *out, int64_t count);

#ifdef __cplusplus
}
#endif

#endif /* SC_SYNTH_H */
