/*
 * petjson.h — C ABI of libpetjson, a gfx950 (MI355X) batch JSON codec for the
 * OpenAPI petstore Pet / Category / Tag models.
 *
 * Reference interface replaced: io.micronaut.serde.ObjectMapper as used by the
 * reference application —
 *   objectMapper.readValue(InputStream, Class)   src/main/java/com/micronaut/bug/config/MyEntityConfig.java:34
 *   ObjectMapper.getDefault()                    src/main/java/com/micronaut/bug/service/MyEntityService.java:45
 *   import io.micronaut.serde.ObjectMapper       MyEntityConfig.java:8, MyEntityService.java:7
 * with micronaut-serde-jackson 2.15.1 (build.gradle:104) doing the byte work.
 * The record layout is the Pet / Category / Tag schema of petstore.json:858-936.
 *
 * Everything here is plain C: pointers, sizes, integer status codes.  No
 * exceptions cross the boundary; no torch or HIP types appear in signatures.
 *
 * Memory: functions named *_device take device pointers on the context's GPU
 * and leave results in device memory; functions named *_host take host
 * pointers and move data through library-owned device buffers.  The caller
 * owns every buffer it passes; the context owns its device scratch.
 * Threading: one context per thread; each context has its own HIP stream.
 */
#ifndef PETJSON_H
#define PETJSON_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------ status */
typedef enum pj_status {
    PJ_OK = 0,
    PJ_ERR_INVALID_ARG = 1,   /* null pointer / bad enum / inconsistent sizes   */
    PJ_ERR_CAPACITY = 2,      /* an output buffer is too small; sizes reported  */
    PJ_ERR_DEVICE = 3,        /* a HIP call failed (message via pj_last_error)   */
    PJ_ERR_NO_DEVICE = 4,     /* no usable gfx950 device                        */
    PJ_ERR_OUT_OF_MEMORY = 5,
    PJ_ERR_SYNTAX = 6         /* an array document's frame is malformed ('[',
                                 the top-level commas, the closing ']'); no
                                 column is written                           */
} pj_status;

/* ------------------------------------------------------------ record model */
/* Pet.StatusEnum (petstore.json:909-917).  @JsonValue strings are
 * "available", "pending", "sold"; PJ_STATUS_NULL means the field is null. */
enum { PJ_STATUS_AVAILABLE = 0, PJ_STATUS_PENDING = 1, PJ_STATUS_SOLD = 2,
       PJ_STATUS_NULL = 255 };

/* Per-pet presence bits (flags column).  A clear bit means the Java field is
 * null.  name and photoUrls are required (petstore.json:873-876). */
enum {
    PJ_PET_HAS_ID        = 1u << 0,
    PJ_PET_HAS_CATEGORY  = 1u << 1,
    PJ_PET_HAS_NAME      = 1u << 2,
    PJ_PET_HAS_PHOTOURLS = 1u << 3,
    PJ_PET_HAS_TAGS      = 1u << 4
};
/* flags used for every pet when the flags column pointer is NULL */
#define PJ_PET_DEFAULT_FLAGS (PJ_PET_HAS_ID | PJ_PET_HAS_NAME | PJ_PET_HAS_PHOTOURLS)

/* Category and Tag presence bits (cat_flags, tag_flags columns). */
enum { PJ_SUB_HAS_ID = 1u << 0, PJ_SUB_HAS_NAME = 1u << 1 };
#define PJ_SUB_DEFAULT_FLAGS (PJ_SUB_HAS_ID | PJ_SUB_HAS_NAME)

/*
 * Structure-of-arrays columns for n_pets records.  Strings are raw UTF-8
 * (unescaped) in one byte array per column, delimited by a 64-bit offset array
 * of length count+1 whose first entry is 0.
 *
 * Optional columns: when the pointer of a group is NULL on encode the group is
 * treated as absent for every record —
 *   flags == NULL        every pet has PJ_PET_DEFAULT_FLAGS
 *   id == NULL           requires HAS_ID clear everywhere (flags non-NULL)
 *   status == NULL       every status is null
 *   cat_* == NULL        requires HAS_CATEGORY clear everywhere
 *   cat_flags == NULL    every present category has PJ_SUB_DEFAULT_FLAGS
 *   photo_off == NULL    every photoUrls list is empty
 *   tag_off == NULL      every tags list is empty
 *   tag_flags == NULL    every tag has PJ_SUB_DEFAULT_FLAGS
 * On decode every pointer must be valid and the cap_* fields give capacities.
 */
typedef struct pj_pet_columns {
    uint64_t  n_pets;
    int64_t  *id;              /* [n_pets]                                   */
    uint8_t  *flags;           /* [n_pets]  PJ_PET_HAS_*                     */
    uint8_t  *status;          /* [n_pets]  PJ_STATUS_*                      */
    uint64_t *name_off;        /* [n_pets+1]                                 */
    uint8_t  *name_bytes;
    /* category: one slot per pet, meaningful when HAS_CATEGORY */
    int64_t  *cat_id;          /* [n_pets]                                   */
    uint8_t  *cat_flags;       /* [n_pets]  PJ_SUB_HAS_*                     */
    uint64_t *cat_name_off;    /* [n_pets+1]                                 */
    uint8_t  *cat_name_bytes;
    /* photoUrls: pet i owns urls [photo_off[i], photo_off[i+1]) */
    uint64_t *photo_off;       /* [n_pets+1]                                 */
    uint64_t *url_off;         /* [n_urls+1]                                 */
    uint8_t  *url_bytes;
    /* tags: pet i owns tags [tag_off[i], tag_off[i+1]) */
    uint64_t *tag_off;         /* [n_pets+1]                                 */
    int64_t  *tag_id;          /* [n_tags]                                   */
    uint8_t  *tag_flags;       /* [n_tags]                                   */
    uint64_t *tag_name_off;    /* [n_tags+1]                                 */
    uint8_t  *tag_name_bytes;
    /* decode capacities (ignored on encode) */
    uint64_t  cap_pets, cap_name_bytes, cap_cat_name_bytes, cap_urls,
              cap_url_bytes, cap_tags, cap_tag_name_bytes;
} pj_pet_columns;

/* ----------------------------------------------------------------- options */
/* Jackson JsonInclude modes for the optional (non-required) properties:
 * Pet.id, Pet.category, Pet.tags, Pet.status, Category.id/name, Tag.id/name.
 * Required properties (Pet.name, Pet.photoUrls) are always written. */
typedef enum pj_inclusion {
    PJ_INCLUDE_NON_EMPTY = 0,  /* micronaut-serde default: skip null, "" and [] */
    PJ_INCLUDE_NON_NULL  = 1,  /* skip null only                                */
    PJ_INCLUDE_ALWAYS    = 2   /* write null as null                            */
} pj_inclusion;

typedef enum pj_format {
    PJ_FORMAT_ARRAY  = 0,      /* [rec,rec,...]   (List<Pet> body)             */
    PJ_FORMAT_NDJSON = 1,      /* rec\nrec\n...                                 */
    PJ_FORMAT_PRETTY = 2       /* the List<Pet> body indented as by jackson-core's
                                  DefaultPrettyPrinter (ObjectMapper with
                                  pretty printing on): "[ {\n  \"id\" : 1,
                                  ...\n}, {...} ]"                            */
} pj_format;

/* The optional properties, for per-property inclusion modes (Jackson's
 * @JsonInclude on a property overrides the mapper default; petstore.json
 * Pet :872-922, Category :858-871, Tag :923-936). */
typedef enum pj_field {
    PJ_FIELD_PET_ID = 0,
    PJ_FIELD_PET_CATEGORY,
    PJ_FIELD_PET_TAGS,
    PJ_FIELD_PET_STATUS,
    PJ_FIELD_CATEGORY_ID,
    PJ_FIELD_CATEGORY_NAME,
    PJ_FIELD_TAG_ID,
    PJ_FIELD_TAG_NAME,
    PJ_FIELD_COUNT
} pj_field;
#define PJ_INCLUDE_DEFAULT (-1)  /* field_inclusion entry: use `inclusion` */

typedef struct pj_options {
    int32_t inclusion;         /* pj_inclusion: the mode of every optional
                                  property without an entry of its own      */
    int32_t hex_upper;         /* 1: \u001F (Jackson >= 2.14 default), 0: \u001f */
    int32_t field_inclusion[PJ_FIELD_COUNT];  /* pj_inclusion per pj_field, or
                                  PJ_INCLUDE_DEFAULT (pj_default_options)   */
} pj_options;

/* --------------------------------------------------------- decode results */
/* Per-record error classes.  A record's code is that of the first error met
 * reading the line left to right. */
enum {
    PJ_REC_OK = 0,
    PJ_REC_SYNTAX = 1,            /* malformed JSON, comments, trailing bytes  */
    PJ_REC_STRING = 2,            /* unterminated, raw control char, bad
                                     escape, invalid UTF-8, lone surrogate     */
    PJ_REC_NUMBER = 3,            /* an id that is not an int64 integer        */
    PJ_REC_TYPE = 4,              /* wrong JSON type for a known property      */
    PJ_REC_MISSING_NAME = 5,      /* name absent or null                       */
    PJ_REC_MISSING_PHOTOURLS = 6, /* photoUrls absent or null                  */
    PJ_REC_BAD_STATUS = 7,        /* status not in the enum                    */
    PJ_REC_DEPTH = 8,             /* nesting deeper than PJ_MAX_DEPTH           */
    PJ_REC_EMPTY = 9              /* blank line                                 */
};
#define PJ_MAX_DEPTH 1000

typedef struct pj_decode_result {
    uint64_t n_lines;             /* record slots in the input                 */
    uint64_t n_pets;              /* valid records written to the columns      */
    uint64_t n_errors;            /* invalid records                           */
    uint64_t name_bytes, cat_name_bytes, n_urls, url_bytes, n_tags,
             tag_name_bytes;      /* column sizes written (or needed)          */
    uint64_t n_general;           /* lines read by the general (non-canonical)
                                     parser rather than the fast path          */
} pj_decode_result;

/* ----------------------------------------------------------------- context */
typedef struct pj_ctx pj_ctx;

/* Create a context bound to HIP device `device` with its own stream.
 * Replaces the ObjectMapper bean obtained from DI (MyEntityConfig.java:24) or
 * ObjectMapper.getDefault() (MyEntityService.java:45). */
pj_ctx     *pj_create(int device, pj_status *status);
void        pj_destroy(pj_ctx *ctx);
void        pj_default_options(pj_options *opt);
pj_status   pj_set_options(pj_ctx *ctx, const pj_options *opt);
/* Thread-local text of the last failure on this thread. */
const char *pj_last_error(void);
/* Duration (ms, HIP events on the context stream) of the last call's kernels:
 * index 0 = whole device pipeline, 1.. = individual kernels in launch order.
 * Returns the number of entries written. */
int         pj_last_timings(const pj_ctx *ctx, float *ms, int cap);

/* ------------------------------------------------------------------ encode */
/* Serialise n_pets records (ObjectMapper.writeValueAsBytes(List<Pet>) for
 * PJ_FORMAT_ARRAY).  Device pointers.  *out_len receives the exact encoded
 * size; when it exceeds out_cap nothing past out_cap is written and
 * PJ_ERR_CAPACITY is returned. */
pj_status pj_encode_device(pj_ctx *ctx, const pj_pet_columns *cols, int format,
                           uint8_t *out, uint64_t out_cap, uint64_t *out_len);
/* Exact encoded size only (length pass). */
pj_status pj_encode_size_device(pj_ctx *ctx, const pj_pet_columns *cols,
                                int format, uint64_t *out_len);
/* An upper bound of the encoded size of n_pets records (host pointers; no
 * device work): room for every property and its longest value per record,
 * item, and every string byte written as a six-byte \u00XX escape.  No
 * counterpart in the reference; callers of pj_encode_host size their buffer
 * with it and encode in one call instead of asking for the exact size first
 * (which would copy the columns to the device twice). */
pj_status pj_encode_bound(const pj_pet_columns *cols, int format, uint64_t *bound);
/* findPetsByStatus's response body (reference petstore.json:106-140, a
 * `status` query of several values, default "available"): the records whose
 * status is in status_mask, in input order, serialised as pj_encode_device
 * would serialise just those records.  Bit s of status_mask selects status
 * code s (0 available, 1 pending, 2 sold); bit 3 selects records without a
 * status.  *n_selected (may be NULL) receives the number of records written.
 * Device pointers; capacity rules as pj_encode_device. */
pj_status pj_encode_by_status_device(pj_ctx *ctx, const pj_pet_columns *cols, uint32_t status_mask,
                                     int format, uint8_t *out, uint64_t out_cap, uint64_t *out_len,
                                     uint64_t *n_selected);
/* Same as pj_encode_by_status_device with host pointers. */
pj_status pj_encode_by_status_host(pj_ctx *ctx, const pj_pet_columns *cols, uint32_t status_mask,
                                   int format, uint8_t *out, uint64_t out_cap, uint64_t *out_len,
                                   uint64_t *n_selected);
/* Same as pj_encode_device with host pointers. */
pj_status pj_encode_host(pj_ctx *ctx, const pj_pet_columns *cols, int format,
                         uint8_t *out, uint64_t out_cap, uint64_t *out_len);

/* Same as pj_encode_device, but allocates nothing: no hipMalloc / hipFree
 * or allocating library routine runs inside the call.  No counterpart in the
 * reference; it is for callers that cannot allocate (tight serving loops,
 * harnesses that forbid allocation).  The call is synchronous: it waits for
 * its stream and reads the length back, so it cannot be recorded into a HIP
 * graph.  Its
 * scratch (block look-back words) lives in a fixed device array of
 * PJ_NOALLOC_SCRATCH_WORDS 64-bit words per GPU, held until the process
 * ends, so n_pets is limited to PJ_NOALLOC_MAX_RECORDS(nested) where nested
 * means any of the category / photoUrls / tags groups is present; larger
 * inputs return PJ_ERR_INVALID_ARG.  Every call on one GPU shares that
 * GPU's array (each call clears what it needs); calls on one GPU from
 * different threads or contexts are serialised inside the library by a
 * per-GPU host lock held until the call's stream has drained. */
#define PJ_NOALLOC_SCRATCH_WORDS (1u << 20)
#define PJ_NOALLOC_MAX_RECORDS(nested) \
    ((uint64_t)(PJ_NOALLOC_SCRATCH_WORDS - 132) * ((nested) ? 96u : 256u))
pj_status pj_encode_device_noalloc(pj_ctx *ctx, const pj_pet_columns *cols, int format,
                                   uint8_t *out, uint64_t out_cap, uint64_t *out_len);

/* Pinned (page-locked) host memory for the *_host entry points.  Inputs and
 * outputs that lie in it move by DMA straight between the caller's buffer
 * and the device; other host memory is copied through the library's pinned
 * bounce buffers first.  No counterpart in the reference; it is for callers
 * that stage their bytes in memory they allocate once (a Java caller would
 * wrap it in a MemorySegment).  Returns NULL when the allocation fails. */
void       *pj_host_alloc(uint64_t n);
void        pj_host_free(void *p);

/* ------------------------------------------------------------------ decode */
/* Parse NDJSON (one Pet per line) into columns (readValue per line).
 * Valid records are written in input order; invalid ones are skipped and
 * their zero-based line indices (ascending) and PJ_REC_* codes written to
 * err_line / err_code (up to err_cap entries).  Device pointers.  When a
 * capacity is too small PJ_ERR_CAPACITY is returned and *res holds the sizes
 * needed. */
pj_status pj_decode_device(pj_ctx *ctx, const uint8_t *in, uint64_t len,
                           pj_pet_columns *out, uint64_t *err_line,
                           uint8_t *err_code, uint64_t err_cap,
                           pj_decode_result *res);
pj_status pj_decode_host(pj_ctx *ctx, const uint8_t *in, uint64_t len,
                         pj_pet_columns *out, uint64_t *err_line,
                         uint8_t *err_code, uint64_t err_cap,
                         pj_decode_result *res);
/* Parse one JSON array document of Pets into columns
 * (readValue(bytes, List<Pet>), the reference's bulk shape "array of Pet",
 * petstore.json:133-140, read as in MyEntityConfig.java:34).  Its frame — '['
 * after optional whitespace, elements separated by the commas at depth 1
 * outside strings, the closing ']', then only whitespace — must be intact,
 * else PJ_ERR_SYNTAX is returned and nothing is written (so are "[,]" and a
 * trailing comma: an element may not be blank; "[]" and "[ ]" hold none).
 * Each element is then read exactly as one NDJSON line (whitespace,
 * newlines included, may surround and separate its tokens) and reported by
 * its zero-based index like a line: valid ones become rows in order,
 * invalid ones are listed in err_line / err_code.  Device / host pointers as
 * pj_decode_device / pj_decode_host. */
pj_status pj_decode_array_device(pj_ctx *ctx, const uint8_t *in, uint64_t len,
                                 pj_pet_columns *out, uint64_t *err_line,
                                 uint8_t *err_code, uint64_t err_cap,
                                 pj_decode_result *res);
pj_status pj_decode_array_host(pj_ctx *ctx, const uint8_t *in, uint64_t len,
                               pj_pet_columns *out, uint64_t *err_line,
                               uint8_t *err_code, uint64_t err_cap,
                               pj_decode_result *res);
/* Column capacities that always suffice for decoding `len` input bytes.
 * The error list needs at most one entry per line, and `len` bytes hold at
 * most `len` lines (blank lines are errors too); a call whose err_cap is too
 * small returns PJ_ERR_CAPACITY with res->n_errors set, so callers may start
 * smaller and retry once with that count. */
void      pj_decode_bounds(uint64_t len, pj_pet_columns *caps_out);

/* ------------------------------------------------ Order and User models
 * The petstore's other two schemas (reference petstore.json:824-857 User,
 * :937-971 Order), through the same ObjectMapper calls as Pet
 * (writeValueAsBytes(List<Order>), readValue(line, Order.class), ...).
 * Their properties are all optional and flat, so one column set describes
 * either model: property k (schema order below) lives in col[k] and, for a
 * string property, bytes[k].
 *
 *   PJ_MODEL_ORDER: 0 id int64, 1 petId int64, 2 quantity int32,
 *     3 shipDate string (the date-time text as written; not reparsed),
 *     4 status enum u8 (0 placed, 1 approved, 2 delivered), 5 complete bool.
 *   PJ_MODEL_USER:  0 id int64, 1 username, 2 firstName, 3 lastName,
 *     4 email, 5 password, 6 phone (strings), 7 userStatus int32.
 *
 * Encoding writes the properties in that order; under pj_options.inclusion
 * a null property (its `present` bit clear) is skipped unless ALWAYS, and
 * under NON_EMPTY so is an empty string.  Decoding follows the Pet rules:
 * keys in any order, the last duplicate wins, unknown keys are validated and
 * skipped, null means absent, an int property takes an integer token in its
 * type's range (else PJ_REC_NUMBER), an unknown status is PJ_REC_BAD_STATUS. */
typedef enum pj_model {
    PJ_MODEL_ORDER = 1,
    PJ_MODEL_USER  = 2
} pj_model;
#define PJ_MODEL_MAX_PROPS 8

typedef struct pj_model_columns {
    uint64_t n;                             /* records                      */
    uint8_t *present;                       /* [n] bit k: property k is non-null;
                                               NULL on encode: all non-null  */
    void    *col[PJ_MODEL_MAX_PROPS];       /* int64_t[n] / int32_t[n] /
                                               uint8_t[n] (enum code, bool 0|1) /
                                               uint64_t[n+1] string offsets  */
    uint8_t *bytes[PJ_MODEL_MAX_PROPS];     /* string properties' bytes      */
    uint64_t cap_n;                         /* decode: records the columns hold */
    uint64_t cap_bytes[PJ_MODEL_MAX_PROPS]; /* decode: bytes[k] capacity     */
    uint64_t n_bytes[PJ_MODEL_MAX_PROPS];   /* decode output: bytes of each
                                               string column written (or needed) */
} pj_model_columns;

/* writeValueAsBytes(List<Order|User>): format as for Pets (ARRAY, NDJSON or
 * PRETTY).  Device pointers; capacity rules as pj_encode_device. */
pj_status pj_encode_model_device(pj_ctx *ctx, int model, const pj_model_columns *cols, int format,
                                 uint8_t *out, uint64_t out_cap, uint64_t *out_len);
/* readValue of NDJSON lines (array = 0) or of one JSON array document
 * (array = 1) of Orders or Users into columns.  Device pointers.  Valid
 * records go to the columns in input order (out->n, out->n_bytes set); the
 * invalid ones are listed as in pj_decode_device (res->n_pets counts the
 * valid records).  Capacities: out->cap_n records, out->cap_bytes[k] bytes;
 * pj_decode_model_bounds gives ones that always suffice. */
pj_status pj_decode_model_device(pj_ctx *ctx, int model, const uint8_t *in, uint64_t len, int array,
                                 pj_model_columns *out, uint64_t *err_line, uint8_t *err_code,
                                 uint64_t err_cap, pj_decode_result *res);
void      pj_decode_model_bounds(int model, uint64_t len, pj_model_columns *caps_out);
/* The same two calls with host pointers (the columns, the text and the
 * error lists in host memory; the device work is staged by the library). */
pj_status pj_encode_model_host(pj_ctx *ctx, int model, const pj_model_columns *cols, int format,
                               uint8_t *out, uint64_t out_cap, uint64_t *out_len);
pj_status pj_decode_model_host(pj_ctx *ctx, int model, const uint8_t *in, uint64_t len, int array,
                               pj_model_columns *out, uint64_t *err_line, uint8_t *err_code,
                               uint64_t err_cap, pj_decode_result *res);

#ifdef __cplusplus
}
#endif
#endif /* PETJSON_H */
