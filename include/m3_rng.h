/*
 * m3_rng.h - deterministic PCG32 generator used to draw seeded inputs.
 *
 * Same stream as the reference generator (src/m3_rng.c:9-110,
 * src/m3_rng.h:12-26): PCG32 XSH-RR with (seed, sequence) seeding, uniform
 * floats from the top 24 bits, and Box-Muller normals in double precision
 * with a cached spare. Pinned by the reference KAT
 * tests/test_host_utilities.c:12-16.
 */
#ifndef M3_RNG_H
#define M3_RNG_H

#include "m3.h"

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    uint64_t state;
    uint64_t increment;
    float spare_normal;
    bool has_spare_normal;
} m3_rng;

m3_status m3_rng_seed(m3_rng *rng, uint64_t seed, uint64_t sequence,
                      m3_error *error);
m3_status m3_rng_u32(m3_rng *rng, uint32_t *value, m3_error *error);
/* Uniform in [0, 1) with 24 random bits. */
m3_status m3_rng_uniform_f32(m3_rng *rng, float *value, m3_error *error);
/* Standard normal values. */
m3_status m3_rng_normal_f32_fill(m3_rng *rng, float *values, size_t count,
                                 m3_error *error);

/* Bulk helpers for building seeded test and benchmark tensors:
 * values[i] = low + (high - low) * uniform, in stream order. */
m3_status m3_rng_uniform_f32_fill(m3_rng *rng, float *values, size_t count,
                                  float low, float high, m3_error *error);
/* values[i] = scale * normal, in stream order. */
m3_status m3_rng_normal_f32_fill_scaled(m3_rng *rng, float *values,
                                        size_t count, float scale,
                                        m3_error *error);

#ifdef __cplusplus
}
#endif

#endif
