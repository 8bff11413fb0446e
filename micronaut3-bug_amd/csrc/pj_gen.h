/*
 * pj_gen.h — seeded synthetic Pet records for the benchmark configurations.
 *
 * Record i of a run draws only from rng(seed, i), so generation is
 * independent of thread count.  Columns are allocated in host memory with
 * malloc and released by pjg_free.  Config numbers follow the benchmark
 * list (1 = CPU plumbing, 2 = flat, 3 = nested, 4 = nested text for decode,
 * 5 = skewed long-tail).
 */
#ifndef PJ_GEN_H
#define PJ_GEN_H
#include "petjson.h"
#ifdef __cplusplus
extern "C" {
#endif

#define PJG_SEED_BASE 0x5EED0000ull

/* Fill *out with n records of configuration `config`; threads <= 0 picks
 * min(16, hardware threads).  Returns 0 on success. */
int  pjg_generate(int config, uint64_t n, uint64_t seed, int threads, pj_pet_columns *out);
void pjg_free(pj_pet_columns *cols);

/* Corrupt about `rate` of the lines of NDJSON `text` in place without
 * changing any length: kind 0 renames the pet's "name" key (missing name),
 * kind 1 changes the last letter of the status value (unknown status),
 * kind 2 removes the closing quote and brace of the line (truncated string).
 * Lines must be encoder output carrying a status.  Writes the corrupted line
 * indices (ascending) and their expected PJ_REC_* codes; returns the count. */
uint64_t pjg_corrupt_ndjson(uint8_t *text, uint64_t len, uint64_t seed, double rate,
                            uint64_t *err_line, uint8_t *err_code, uint64_t cap);

#ifdef __cplusplus
}
#endif
#endif
