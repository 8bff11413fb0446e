// pj_kernels.h — kernel parameter blocks and launchers (host <-> device).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "petjson.h"

struct EncParams {
    pj_pet_columns c;          // device column pointers
    uint64_t n;                // records
    uint64_t first, last;      // the local index of the input's first / last record (array
                               // framing), or ~0 when a segment of the input holds none
    int format;                // pj_format
    uint8_t incl[PJ_FIELD_COUNT];  // pj_inclusion of each optional property (pj_field)
    uint32_t hexa;             // 'A' or 'a': first letter of hex escapes
    int count_only;            // 1: length pass only
    uint8_t *out;
    uint64_t cap;
    uint64_t *state;           // look-back words, one per block (zeroed)
    unsigned long long *ticket;// block tickets (zeroed); with order_by_id, set to 1 when a look-back
                               // gave up (the launch is then redone in ticket order)
    int order_by_id;           // one-block workgroups only: block b is workgroup b (no ticket atomic)
    uint64_t spin_limit;       // look-back wait bound (wall-clock ticks) when order_by_id
    uint64_t *total;           // encoded size (written by the last block)
    uint32_t *dummy;           // PJ_BLOCK scratch dwords (shared first dwords land here)
    unsigned long long *nfall; // blocks whose records did not fit the LDS tile (counted)
    const uint64_t *sel;       // one-thread-per-record kernel: output record j is record sel[j] (or j)
    uint64_t *geo;             // nested writer, two passes: block b's bounds and output offset
                               // (GEO_WORDS words at geo[GEO_WORDS * b], from k_enc_measure);
                               // blocks then run in static order with no look-back
    // nested writer: large records are listed (record, output offset) for
    // k_enc_big to write after the pass; with big_cap 0, or once the list
    // is full, the pass writes them itself
    unsigned long long *big_count;  // zeroed
    uint64_t *big_list;
    uint64_t big_cap;
};
constexpr int GEO_WORDS = 13;

// Order / User encode (pj_encode_model_device): one thread per record,
// blocks claimed by ticket, decoupled look-back.
struct ModelEncParams {
    pj_model_columns c;        // device column pointers
    uint64_t n;                // records
    int model;                 // pj_model
    int format;                // pj_format
    uint32_t incl;             // pj_inclusion (mapper-wide)
    uint32_t hexa;             // 'A' or 'a'
    int count_only;
    uint8_t *out;
    uint64_t cap;
    uint64_t *state;           // look-back words, one per block (zeroed)
    unsigned long long *ticket;// block ticket (zeroed)
    uint64_t *total;           // encoded size (written by the last block)
};

// Order / User decode (pj_decode_model_device), after the record index:
// a counting pass (block totals), a scan of them, a writing pass.
constexpr int MD_MAXK = 2 + PJ_MODEL_MAX_PROPS;   // valid, errors, one per string property
struct ModelDecParams {
    const uint8_t *in;
    uint64_t len;              // input bytes
    const uint64_t *line_start;// record l spans [line_start[l], line_start[l+1] - 1)
    uint64_t lines;
    pj_model_columns o;        // outputs with capacities
    uint64_t *err_line;
    uint8_t *err_code;
    uint64_t err_cap;
    uint64_t *bagg;            // [nblocks * MD_MAXK] block totals
    uint64_t *bbase;           // [nblocks * MD_MAXK] block first offsets within their chunk
    uint64_t *csum;            // [nchunks * MD_MAXK] chunk first offsets
    uint64_t *totals;          // [MD_MAXK + 1] sums (the last: blank records)
    uint64_t nblocks;
    uint64_t *tape;            // what the counting pass read of each record, for the writer
                               // (word k of record l at tape[k * lines + l]), or null
};

// What the decode counting kernels learn about each line, read back by the
// writers (32 bytes per line).
struct LineRec {
    uint32_t name_len, cat_len, n_urls, url_bytes, n_tags, tag_bytes;
    uint32_t code;      // PJ_REC_* (general lines: set by the general count kernel)
    uint32_t general;   // 1: the line is read by the general parser
};

// Summary of a stretch of an array document, for each of the four states it
// may be entered in (bit 0 inside a string, bit 1 first byte escaped): the
// exit state (2 bits each in out) and the depth change.  Composed in order
// by the array frame kernels.
struct FS {
    uint32_t out;
    int32_t d[4];
};

struct DecParams {
    const uint8_t *in;
    uint64_t len;
    uint64_t nblk64;           // number of 64-byte blocks
    // line index
    uint64_t *line_start;      // [ls_cap]: line l spans [line_start[l], line_start[l+1]-1)
    uint64_t ls_cap;
    uint64_t *n_lines;         // device scalar
    // parse stage
    pj_pet_columns o;          // outputs with capacities
    uint64_t *err_line;
    uint8_t *err_code;
    uint64_t err_cap;
    uint64_t *totals;          // [PJ_DEC_NCNT] column totals (written by last block)
    uint64_t *state_idx;       // look-back words of the line-index stage, one per block
    uint64_t *state_parse;     // vector look-back words of the parse stage, per line block
    unsigned long long *tickets; // [2]
    uint64_t lines;            // n_lines as known by the host for the parse stage
    uint32_t *dummy;           // sink for diverted shared dwords (never read)
    unsigned long long *gq_count;   // lines read by the general parser (diagnostic)
    // error slots whose code is settled by k_dec_errcode (lines known to be
    // invalid from the bitmaps alone)
    uint64_t *dq;
    uint64_t *tape;            // per line: 32 words of the validating walk's results, or null
    unsigned long long *dq_count;
    // split decode (with the tape): the validating kernel stores per line its
    // offsets inside its block (lpos, 8 counters column by column, then the
    // line's code and kind in row 8) and per block the counter totals (bagg);
    // a scan turns those into each block's first offsets (bbase, with its own
    // look-back words bstate); the writer kernels then need no waiting
    uint32_t *lpos;
    uint64_t *bagg, *bbase, *bstate;
    uint64_t *bm_list;         // split decode: blocks holding deferred lines (nblocks entries)
    unsigned long long *bm_count;  // [0] blocks in bm_list, [1] unused
    uint64_t nblocks;          // line blocks of the validating kernel
    uint64_t *long_list;       // lines read by a whole wave, written by k_dec_long
    unsigned long long *long_count;
    unsigned long long *bticket;  // block ticket of the scan kernel
    // array documents: the frame's scalars (0 first non-whitespace byte,
    // 1 last non-whitespace byte + 1, 2 the close, 3 separators, 4 frame
    // ok, 5 block ticket), per-block summaries and entry states; array_doc
    // makes the line stages read each element's separator as its newline
    int array_doc;
    uint64_t *arr;
    FS *arr_bsum;
    FS *arr_tsum;              // per thread of the frame kernels: the summary of its block's words before its own
    uint64_t *arr_bpre;
    unsigned long long *empty_count;   // lines that are blank (PJ_REC_EMPTY)
    // 1: block b of each kernel takes its input in launch order (no ticket
    // atomic) and bounds its look-back wait by spin_limit wall-clock ticks;
    // a kernel whose wait ran out sets its ticket word to 1 and is redone
    // in ticket order
    int order_by_id;
    uint64_t spin_limit;
};

// counters carried through the parse-stage scan
enum { C_PETS = 0, C_NAMEB, C_CATB, C_URLS, C_URLB, C_TAGS, C_TAGB, C_ERRS, PJ_DEC_NCNT };

hipError_t pj_launch_fill_u64(uint64_t *p, uint64_t n, uint64_t v, hipStream_t st);
hipError_t pj_launch_add_u64(uint64_t *p, uint64_t n, uint64_t v, hipStream_t st);   // p[0, n) += v
hipError_t pj_launch_encode(const EncParams &P, bool nested, bool wide, hipStream_t st);
hipError_t pj_launch_encode_measure(const EncParams &P, hipStream_t st);
// the large records a nested pass listed (P.big_list), one workgroup each:
// with full, as many workgroups as the GPU holds, else 64 (a launch that
// expects an empty list costs less; any count is still written)
hipError_t pj_launch_encode_big(const EncParams &P, bool full, hipStream_t st);
int pj_encode_block_records(bool nested);
// one thread per output record (pretty output, or a selection of records)
hipError_t pj_launch_encode_rows(const EncParams &P, bool pretty, hipStream_t st);
// pretty output of nested records through the tiled encode (blocks of
// pj_encode_pretty_tile_records() records)
hipError_t pj_launch_encode_pretty(const EncParams &P, hipStream_t st);
int pj_encode_pretty_tile_records();
// indices of the records whose status is in mask into sel, their count into *P.total
hipError_t pj_launch_select_status(const EncParams &P, uint32_t mask, uint64_t *sel, hipStream_t st);
uint64_t pj_select_blocks(uint64_t n);   // workgroups (look-back words) of the selection kernel
hipError_t pj_launch_encode_model(const ModelEncParams &P, hipStream_t st);
int pj_encode_model_records();
hipError_t pj_launch_decode_model(const ModelDecParams &P, int model, hipStream_t st);
int pj_decode_model_block();
int pj_encode_pretty_records();
hipError_t pj_launch_put_bytes(uint8_t *out, uint32_t w, int k, hipStream_t st);
hipError_t pj_launch_dec_index(const DecParams &P, hipStream_t st);
hipError_t pj_launch_dec_parse(const DecParams &P, hipStream_t st);
hipError_t pj_launch_dec_errcode(const DecParams &P, hipStream_t st);
// the split decode after the validating kernel: block scan, writers
hipError_t pj_launch_dec_bscan(const DecParams &P, hipStream_t st);
hipError_t pj_launch_dec_write(const DecParams &P, hipStream_t st);

hipError_t pj_launch_dec_long(const DecParams &P, hipStream_t st);
int pj_dec_bscan_block();
// array documents: the frame kernels (element starts into line_start, their
// count into *n_lines, the verdict into arr[4])
hipError_t pj_launch_arr_frame(const DecParams &P, hipStream_t st);
uint64_t pj_arr_blocks(uint64_t nblk64);
uint64_t pj_arr_threads(uint64_t nblk64);   // arr_tsum entries
int pj_dec_index_block();
// Device address of this GPU's fixed encode scratch (PJ_NOALLOC_SCRATCH_WORDS
// u64); resolved once per device, with that device current.
hipError_t pj_noalloc_scratch_init(int device, uint64_t **ptr);
int pj_dec_parse_block();
// The Pet decode keeps each line's output offsets inside its line block as
// 32-bit values, so the bytes of a block's lines must stay below 4 GiB (a
// line of 4 GiB or more is refused with them).  Block b holds lines
// [b lpb, (b + 1) lpb); line l spans [ls[l], ls[l + 1]).  Checked by
// k_dec_span_check when the input is that long (PJ_ERR_INVALID_ARG).
constexpr uint64_t PJ_DEC_MAX_BLOCK_SPAN = (1ull << 32) - (1ull << 20);
__host__ __device__ inline bool dec_block_span_ok(const uint64_t *ls, uint64_t lines, uint64_t lpb, uint64_t b) {
    const uint64_t l0 = b * lpb, l1 = l0 + lpb < lines ? l0 + lpb : lines;
    return l0 >= lines || ls[l1] - ls[l0] < PJ_DEC_MAX_BLOCK_SPAN;
}
hipError_t pj_launch_dec_span_check(const DecParams &P, uint64_t *flag, hipStream_t st);
