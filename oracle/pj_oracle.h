/*
 * pj_oracle.h — CPU restatement of the reference's Pet JSON codec.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * or as the timed CPU baseline.  The product path (libpetjson) never calls it.
 *
 * It restates, in plain sequential C, what micronaut-serde-jackson 2.15.1
 * (reference build.gradle:104) does for the petstore Pet model
 * (petstore.json:858-936) under the reference's serde configuration
 * (application.yml:23-28: comments rejected).  Each function cites the
 * reference lines it follows.  Rules from the external jackson-core / serde
 * jars are restated from their published behaviour; the ones no check here
 * can pin are marked "parity unpinned" where they occur.
 */
#ifndef PJ_ORACLE_H
#define PJ_ORACLE_H
#include "petjson.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Encode n_pets records (host pointers).  Same column conventions and return
 * codes as pj_encode_host. */
/* pj_options defaults: NON_EMPTY everywhere, upper-case hex. */
void or_default_options(pj_options *o);
int or_encode(const pj_pet_columns *cols, const pj_options *opt, int format,
              uint8_t *out, uint64_t out_cap, uint64_t *out_len);

/* The records whose status is in mask (pj_encode_by_status_device rules). */
int or_encode_by_status(const pj_pet_columns *cols, const pj_options *opt, uint32_t mask, int format,
                        uint8_t *out, uint64_t out_cap, uint64_t *out_len, uint64_t *n_selected);

/* Decode NDJSON (host pointers).  Same conventions as pj_decode_host. */
int or_decode(const uint8_t *in, uint64_t len, pj_pet_columns *out,
              uint64_t *err_line, uint8_t *err_code, uint64_t err_cap,
              pj_decode_result *res);

/* Decode one JSON array document of Pets (host pointers).  Same conventions
 * as pj_decode_array_host: PJ_ERR_SYNTAX for a broken array frame, element
 * indices in err_line. */
int or_decode_array(const uint8_t *in, uint64_t len, pj_pet_columns *out,
                    uint64_t *err_line, uint8_t *err_code, uint64_t err_cap,
                    pj_decode_result *res);

/* Parse one record (line without its '\n').  Returns the PJ_REC_* code; on
 * PJ_REC_OK and when `out` is non-NULL appends the record to `out`, whose
 * n_pets / offset tails give the current fill. Exposed for the tests. */
int or_decode_line(const uint8_t *s, uint64_t n, pj_pet_columns *out,
                   pj_decode_result *fill);

/* Order / User models (host pointers): same conventions as
 * pj_encode_model_device / pj_decode_model_device. */
int or_encode_model(int model, const pj_model_columns *cols, const pj_options *opt, int format,
                    uint8_t *out, uint64_t out_cap, uint64_t *out_len);
int or_decode_model(int model, const uint8_t *in, uint64_t len, int array, pj_model_columns *out,
                    uint64_t *err_line, uint8_t *err_code, uint64_t err_cap, pj_decode_result *res);

/* Long.toString(v) into buf (>= 21 bytes); returns length.  Exposed so the
 * tests can brute-force it against printf. */
int or_format_long(int64_t v, char *buf);

#ifdef __cplusplus
}
#endif
#endif
