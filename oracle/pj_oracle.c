/*
 * pj_oracle.c — sequential CPU restatement of the reference Pet JSON codec.
 *
 * TEST INFRASTRUCTURE ONLY (see pj_oracle.h): the checker for libpetjson and
 * the CPU baseline in bench.py.  Nothing in the product links it.
 *
 * Sources of each rule:
 *  - record shape, property order, required properties, enum values:
 *      reference petstore.json:858-936 (Category :858-871, Pet :872-922 with
 *      required :873-876 and properties in order id, category, name,
 *      photoUrls, tags, status :878-917, enum :912-916, Tag :923-936).
 *  - enum written through its @JsonValue string, unknown value rejected by the
 *      @JsonCreator factory: convention of reference api/EnumParam.java:15-35
 *      and config/data/VariantEnum.java:34-47 ("Unknown id" exception).
 *  - comments rejected on read: reference application.yml:23-28.
 *  - optional properties decode to null when absent:
 *      reference config/data/ConfigData.java:26-27 with configs/var1.json:10-12.
 *  - byte-level JSON rules: jackson-core (pulled in by micronaut-serde-jackson
 *      2.15.1, reference build.gradle:104): UTF8JsonGenerator output escapes
 *      (" \ and the short forms \b \t \n \f \r, other C0 controls as \u00XX
 *      with upper-case hex, everything else incl. '/', 0x7F and non-ASCII
 *      written raw), Long.toString number text, no whitespace; the
 *      UTF8StreamJsonParser grammar of RFC 8259 (no leading zeros, no
 *      NaN/Infinity, literals must not run into identifier characters),
 *      max nesting depth 1000 (StreamReadConstraints), UTF-8 lead bytes
 *      C0-DF/E0-EF/F0-F7 with 10xxxxxx continuations.
 *  - serde bean rules: keys in any order, last duplicate wins, unknown keys
 *      skipped (micronaut-serde ignores unknown properties by default),
 *      JsonInclude per property: required => ALWAYS, others => the serde
 *      default inclusion NON_EMPTY.
 *
 * Parity unpinned (no JVM here to run micronaut-serde; the options or the
 * rule chosen are documented at the point of use):
 *   default inclusion of optional properties (NON_EMPTY assumed), coercion of
 *   non-integer numbers / strings into Long id (rejected here), coercion of
 *   scalars into String properties (rejected), null list elements (rejected),
 *   escaped lone surrogates (rejected), blank lines (error PJ_REC_EMPTY).
 */
#include "pj_oracle.h"
#include <stdlib.h>
#include <string.h>

/* ======================================================================
 *                                 ENCODE
 * ====================================================================== */

/* pretty: lay the output out as jackson-core's DefaultPrettyPrinter does;
 * nest: its nesting counter (objects only: its array indenter is inline). */
typedef struct { uint8_t *out; uint64_t cap, len; int pretty, nest; } wbuf;

static void w_bytes(wbuf *w, const void *p, uint64_t n) {
    if (w->out && w->len < w->cap) {
        uint64_t k = w->cap - w->len < n ? w->cap - w->len : n;
        memcpy(w->out + w->len, p, k);
    }
    w->len += n;
}
static void w_char(wbuf *w, char c) { w_bytes(w, &c, 1); }
static void w_lit(wbuf *w, const char *s) { w_bytes(w, s, strlen(s)); }

/* Long.toString: optional '-', decimal digits, no leading zeros. */
int or_format_long(int64_t v, char *buf) {
    char tmp[24];
    int n = 0, len = 0;
    uint64_t u = v < 0 ? (uint64_t)0 - (uint64_t)v : (uint64_t)v;
    do { tmp[n++] = (char)('0' + (int)(u % 10)); u /= 10; } while (u);
    if (v < 0) buf[len++] = '-';
    while (n) buf[len++] = tmp[--n];
    buf[len] = 0;
    return len;
}

static void w_long(wbuf *w, int64_t v) {
    char b[24];
    int n = or_format_long(v, b);
    w_bytes(w, b, (uint64_t)n);
}

/* jackson UTF8JsonGenerator string body with the default escape table. */
static void w_string(wbuf *w, const uint8_t *s, uint64_t n, int hex_upper) {
    static const char HEXU[] = "0123456789ABCDEF", HEXL[] = "0123456789abcdef";
    const char *hex = hex_upper ? HEXU : HEXL;
    w_char(w, '"');
    for (uint64_t i = 0; i < n; i++) {
        uint8_t c = s[i];
        if (c == '"') w_lit(w, "\\\"");
        else if (c == '\\') w_lit(w, "\\\\");
        else if (c < 0x20) {
            switch (c) {
            case 0x08: w_lit(w, "\\b"); break;
            case 0x09: w_lit(w, "\\t"); break;
            case 0x0A: w_lit(w, "\\n"); break;
            case 0x0C: w_lit(w, "\\f"); break;
            case 0x0D: w_lit(w, "\\r"); break;
            default: {
                char e[6] = {'\\', 'u', '0', '0', hex[c >> 4], hex[c & 15]};
                w_bytes(w, e, 6);
            }
            }
        } else w_char(w, (char)c);
    }
    w_char(w, '"');
}

static const char *const STATUS_TXT[3] = {"available", "pending", "sold"};

/* Structure hooks, after the jackson-core 2.x PrettyPrinter calls the
 * generator makes (jackson-core is pulled in by micronaut-serde-jackson
 * 2.15.1, reference build.gradle:14,104; it is not vendored in the
 * reference).  Compact output writes the punctuation only.  With
 * DefaultPrettyPrinter:
 *  - writeStartObject: '{', nesting + 1;
 *  - beforeObjectEntries / writeObjectEntrySeparator: (',' for the latter)
 *    then the object indenter: "\n" + two spaces per nesting level;
 *  - writeObjectFieldValueSeparator: " : ";
 *  - writeEndObject: nesting - 1, then the indenter if the object had
 *    entries, else one space; '}';
 *  - arrays use the inline FixedSpaceIndenter (one space, no nesting
 *    change): beforeArrayValues ' ', writeArrayValueSeparator ", ",
 *    writeEndArray ' ' (with or without values) then ']'. */
static void w_indent(wbuf *w) {
    w_char(w, '\n');
    for (int k = 0; k < w->nest; k++) w_lit(w, "  ");
}
static void o_start(wbuf *w) {
    w_char(w, '{');
    w->nest++;
}
static void o_end(wbuf *w, int empty) {
    w->nest--;
    if (w->pretty) {
        if (empty) w_char(w, ' ');
        else w_indent(w);
    }
    w_char(w, '}');
}
static void a_start(wbuf *w) { w_char(w, '['); }
/* Before array value number idx. */
static void a_value(wbuf *w, uint64_t idx) {
    if (idx) w_char(w, ',');
    if (w->pretty) w_char(w, ' ');
}
static void a_end(wbuf *w) {
    if (w->pretty) w_char(w, ' ');
    w_char(w, ']');
}

/* "key": with a leading comma when it is not the first property written. */
static void w_key(wbuf *w, int *first, const char *key) {
    if (!*first) w_char(w, ',');
    if (w->pretty) w_indent(w);
    *first = 0;
    w_char(w, '"');
    w_lit(w, key);
    w_lit(w, w->pretty ? "\" : " : "\":");
}

/* The inclusion mode of optional property f: its own entry, else the
 * mapper-wide mode (a property-level @JsonInclude overrides the default). */
static int incl_of(const pj_options *o, int f) {
    return o->field_inclusion[f] == PJ_INCLUDE_DEFAULT ? o->inclusion : o->field_inclusion[f];
}

/* Category / Tag body: {"id":..,"name":".."} with optional-property
 * inclusion (modes of its id and of its name). */
static void w_sub(wbuf *w, int id_incl, int name_incl, int hex_upper, uint8_t fl, int64_t id,
                  const uint8_t *name, uint64_t name_len) {
    int first = 1;
    o_start(w);
    if (fl & PJ_SUB_HAS_ID) { w_key(w, &first, "id"); w_long(w, id); }
    else if (id_incl == PJ_INCLUDE_ALWAYS) { w_key(w, &first, "id"); w_lit(w, "null"); }
    if (fl & PJ_SUB_HAS_NAME) {
        if (name_len > 0 || name_incl != PJ_INCLUDE_NON_EMPTY) {
            w_key(w, &first, "name");
            w_string(w, name, name_len, hex_upper);
        }
    } else if (name_incl == PJ_INCLUDE_ALWAYS) { w_key(w, &first, "name"); w_lit(w, "null"); }
    o_end(w, first);
}

/* One Pet in declaration order (petstore.json:878-917). */
static void w_pet(wbuf *w, const pj_pet_columns *c, const pj_options *o, uint64_t i) {
    const int hx = o->hex_upper;
    const uint8_t fl = c->flags ? c->flags[i] : (uint8_t)PJ_PET_DEFAULT_FLAGS;
    int first = 1;
    o_start(w);
    /* id: optional int64 (petstore.json:879-882) */
    if (fl & PJ_PET_HAS_ID) { w_key(w, &first, "id"); w_long(w, c->id[i]); }
    else if (incl_of(o, PJ_FIELD_PET_ID) == PJ_INCLUDE_ALWAYS) { w_key(w, &first, "id"); w_lit(w, "null"); }
    /* category: optional object (petstore.json:883-885).  A bean is never
     * "empty" for NON_EMPTY, so a present category is always written. */
    if ((fl & PJ_PET_HAS_CATEGORY) && c->cat_id) {
        w_key(w, &first, "category");
        uint8_t cf = c->cat_flags ? c->cat_flags[i] : (uint8_t)PJ_SUB_DEFAULT_FLAGS;
        uint64_t a = c->cat_name_off[i], b = c->cat_name_off[i + 1];
        w_sub(w, incl_of(o, PJ_FIELD_CATEGORY_ID), incl_of(o, PJ_FIELD_CATEGORY_NAME), hx, cf, c->cat_id[i],
              c->cat_name_bytes + a, b - a);
    } else if (incl_of(o, PJ_FIELD_PET_CATEGORY) == PJ_INCLUDE_ALWAYS) { w_key(w, &first, "category"); w_lit(w, "null"); }
    /* name: required => always written (petstore.json:873-876, 886-889) */
    w_key(w, &first, "name");
    if (fl & PJ_PET_HAS_NAME)
        w_string(w, c->name_bytes + c->name_off[i], c->name_off[i + 1] - c->name_off[i], hx);
    else w_lit(w, "null");
    /* photoUrls: required array of string (petstore.json:890-899) */
    w_key(w, &first, "photoUrls");
    if (fl & PJ_PET_HAS_PHOTOURLS) {
        a_start(w);
        if (c->photo_off) {
            for (uint64_t u = c->photo_off[i]; u < c->photo_off[i + 1]; u++) {
                a_value(w, u - c->photo_off[i]);
                w_string(w, c->url_bytes + c->url_off[u], c->url_off[u + 1] - c->url_off[u], hx);
            }
        }
        a_end(w);
    } else w_lit(w, "null");
    /* tags: optional array of Tag (petstore.json:900-908); NON_EMPTY skips [] */
    if (fl & PJ_PET_HAS_TAGS) {
        uint64_t t0 = c->tag_off ? c->tag_off[i] : 0, t1 = c->tag_off ? c->tag_off[i + 1] : 0;
        if (t1 > t0 || incl_of(o, PJ_FIELD_PET_TAGS) != PJ_INCLUDE_NON_EMPTY) {
            w_key(w, &first, "tags");
            a_start(w);
            for (uint64_t t = t0; t < t1; t++) {
                a_value(w, t - t0);
                uint8_t tf = c->tag_flags ? c->tag_flags[t] : (uint8_t)PJ_SUB_DEFAULT_FLAGS;
                uint64_t a = c->tag_name_off[t], b = c->tag_name_off[t + 1];
                w_sub(w, incl_of(o, PJ_FIELD_TAG_ID), incl_of(o, PJ_FIELD_TAG_NAME), hx, tf, c->tag_id[t],
                      c->tag_name_bytes + a, b - a);
            }
            a_end(w);
        }
    } else if (incl_of(o, PJ_FIELD_PET_TAGS) == PJ_INCLUDE_ALWAYS) { w_key(w, &first, "tags"); w_lit(w, "null"); }
    /* status: optional enum via @JsonValue (petstore.json:909-917);
     * codes other than 0..2 are null. */
    uint8_t st = c->status ? c->status[i] : (uint8_t)PJ_STATUS_NULL;
    if (st <= 2) {
        w_key(w, &first, "status");
        w_char(w, '"');
        w_lit(w, STATUS_TXT[st]);
        w_char(w, '"');
    } else if (incl_of(o, PJ_FIELD_PET_STATUS) == PJ_INCLUDE_ALWAYS) { w_key(w, &first, "status"); w_lit(w, "null"); }
    o_end(w, first);
}

void or_default_options(pj_options *o) {
    o->inclusion = PJ_INCLUDE_NON_EMPTY;
    o->hex_upper = 1;
    for (int k = 0; k < PJ_FIELD_COUNT; k++) o->field_inclusion[k] = PJ_INCLUDE_DEFAULT;
}

int or_encode(const pj_pet_columns *cols, const pj_options *opt, int format,
              uint8_t *out, uint64_t out_cap, uint64_t *out_len) {
    pj_options def;
    or_default_options(&def);
    if (!cols || !out_len ||
        (format != PJ_FORMAT_ARRAY && format != PJ_FORMAT_NDJSON && format != PJ_FORMAT_PRETTY))
        return PJ_ERR_INVALID_ARG;
    if (!opt) opt = &def;
    wbuf w = {out, out_cap, 0, format == PJ_FORMAT_PRETTY, 0};
    const int array = format != PJ_FORMAT_NDJSON;
    if (array) a_start(&w);
    for (uint64_t i = 0; i < cols->n_pets; i++) {
        if (array) a_value(&w, i);
        w_pet(&w, cols, opt, i);
        if (!array) w_char(&w, '\n');
    }
    if (array) a_end(&w);
    *out_len = w.len;
    return w.len > out_cap ? PJ_ERR_CAPACITY : PJ_OK;
}

/* findPetsByStatus (reference petstore.json:106-140): the records whose
 * status code s (3 for no status) has bit s set in mask, in input order,
 * written as or_encode writes a column set holding just those records. */
int or_encode_by_status(const pj_pet_columns *cols, const pj_options *opt, uint32_t mask, int format,
                        uint8_t *out, uint64_t out_cap, uint64_t *out_len, uint64_t *n_selected) {
    pj_options def;
    or_default_options(&def);
    if (!cols || !out_len || (mask & ~0xFu) ||
        (format != PJ_FORMAT_ARRAY && format != PJ_FORMAT_NDJSON && format != PJ_FORMAT_PRETTY))
        return PJ_ERR_INVALID_ARG;
    if (!opt) opt = &def;
    wbuf w = {out, out_cap, 0, format == PJ_FORMAT_PRETTY, 0};
    const int array = format != PJ_FORMAT_NDJSON;
    uint64_t m = 0;
    if (array) a_start(&w);
    for (uint64_t i = 0; i < cols->n_pets; i++) {
        const uint8_t st = cols->status ? cols->status[i] : (uint8_t)PJ_STATUS_NULL;
        if (!((mask >> (st <= 2 ? st : 3)) & 1)) continue;
        if (array) a_value(&w, m);
        w_pet(&w, cols, opt, i);
        if (!array) w_char(&w, '\n');
        m++;
    }
    if (array) a_end(&w);
    *out_len = w.len;
    if (n_selected) *n_selected = m;
    return w.len > out_cap ? PJ_ERR_CAPACITY : PJ_OK;
}

/* ======================================================================
 *                                 DECODE
 * ====================================================================== */

typedef struct { uint8_t *p; uint64_t n, cap; } bytes_t;
static void b_push(bytes_t *b, const uint8_t *s, uint64_t n) {
    if (b->n + n > b->cap) {
        uint64_t nc = b->cap ? b->cap * 2 : 64;
        while (nc < b->n + n) nc *= 2;
        b->p = (uint8_t *)realloc(b->p, nc);
        b->cap = nc;
    }
    memcpy(b->p + b->n, s, n);
    b->n += n;
}

typedef struct {            /* one Category or Tag while it is being read */
    int64_t id;
    uint8_t flags;
    bytes_t name;
} sub_t;

typedef struct {            /* one Pet while it is being read */
    int has_id, has_cat, has_name, has_photo, has_tags;
    int64_t id;
    uint8_t status;
    sub_t cat;
    bytes_t name;
    bytes_t urls;           /* concatenated url bytes */
    uint64_t *url_len; uint64_t n_urls, cap_urls;
    sub_t *tags; uint64_t n_tags, cap_tags;
} pet_t;

typedef struct {
    const uint8_t *s;
    uint64_t n, p;
    int depth;
} rd_t;

/* RFC 8259 whitespace.  An NDJSON line never holds '\n' (lines are cut at
 * every newline), so '\n' only ever meets this test inside the elements of
 * an array document. */
static int is_ws(uint8_t c) { return c == ' ' || c == '\t' || c == '\r' || c == '\n'; }
static void skip_ws(rd_t *r) { while (r->p < r->n && is_ws(r->s[r->p])) r->p++; }
static int at_end(const rd_t *r) { return r->p >= r->n; }
static uint8_t cur(const rd_t *r) { return r->p < r->n ? r->s[r->p] : 0; }

static int hexval(uint8_t c) {
    if (c >= '0' && c <= '9') return c - '0';
    if (c >= 'a' && c <= 'f') return c - 'a' + 10;
    if (c >= 'A' && c <= 'F') return c - 'A' + 10;
    return -1;
}

static int put_utf8(uint8_t *o, uint32_t cp) {
    if (cp < 0x80) { o[0] = (uint8_t)cp; return 1; }
    if (cp < 0x800) { o[0] = (uint8_t)(0xC0 | (cp >> 6)); o[1] = (uint8_t)(0x80 | (cp & 63)); return 2; }
    if (cp < 0x10000) {
        o[0] = (uint8_t)(0xE0 | (cp >> 12)); o[1] = (uint8_t)(0x80 | ((cp >> 6) & 63));
        o[2] = (uint8_t)(0x80 | (cp & 63)); return 3;
    }
    o[0] = (uint8_t)(0xF0 | (cp >> 18)); o[1] = (uint8_t)(0x80 | ((cp >> 12) & 63));
    o[2] = (uint8_t)(0x80 | ((cp >> 6) & 63)); o[3] = (uint8_t)(0x80 | (cp & 63)); return 4;
}

static int read_u4(rd_t *r, uint32_t *cu) {
    if (r->p + 4 > r->n) return 0;
    uint32_t v = 0;
    for (int k = 0; k < 4; k++) {
        int h = hexval(r->s[r->p + k]);
        if (h < 0) return 0;
        v = v * 16 + (uint32_t)h;
    }
    r->p += 4;
    *cu = v;
    return 1;
}

/* A JSON string starting at the opening quote; decoded UTF-8 appended to
 * `out` when non-NULL.  jackson UTF8StreamJsonParser string rules. */
static int rd_string(rd_t *r, bytes_t *out) {
    r->p++; /* opening quote */
    for (;;) {
        if (at_end(r)) return PJ_REC_STRING;              /* unterminated */
        uint8_t c = r->s[r->p];
        if (c == '"') { r->p++; return PJ_REC_OK; }
        if (c == '\\') {
            r->p++;
            if (at_end(r)) return PJ_REC_STRING;
            uint8_t e = r->s[r->p++], o[4];
            int k = 1;
            switch (e) {
            case '"': o[0] = '"'; break;
            case '\\': o[0] = '\\'; break;
            case '/': o[0] = '/'; break;
            case 'b': o[0] = 8; break;
            case 'f': o[0] = 12; break;
            case 'n': o[0] = 10; break;
            case 'r': o[0] = 13; break;
            case 't': o[0] = 9; break;
            case 'u': {
                uint32_t cu, lo;
                if (!read_u4(r, &cu)) return PJ_REC_STRING;
                if (cu >= 0xDC00 && cu <= 0xDFFF) return PJ_REC_STRING;   /* lone low */
                if (cu >= 0xD800 && cu <= 0xDBFF) {
                    /* must be followed by \u + low surrogate (unpinned: a
                     * Java String would keep the lone half) */
                    if (r->p + 2 > r->n || r->s[r->p] != '\\' || r->s[r->p + 1] != 'u')
                        return PJ_REC_STRING;
                    r->p += 2;
                    if (!read_u4(r, &lo) || lo < 0xDC00 || lo > 0xDFFF) return PJ_REC_STRING;
                    cu = 0x10000 + ((cu - 0xD800) << 10) + (lo - 0xDC00);
                }
                k = put_utf8(o, cu);
                break;
            }
            default: return PJ_REC_STRING;
            }
            if (out) b_push(out, o, (uint64_t)k);
            continue;
        }
        if (c < 0x20) return PJ_REC_STRING;                   /* raw control */
        int extra;
        if (c < 0x80) extra = 0;
        else if (c >= 0xC0 && c <= 0xDF) extra = 1;
        else if (c >= 0xE0 && c <= 0xEF) extra = 2;
        else if (c >= 0xF0 && c <= 0xF7) extra = 3;
        else return PJ_REC_STRING;                           /* bad lead byte */
        if (r->p + 1 + (uint64_t)extra > r->n) return PJ_REC_STRING;
        for (int k = 1; k <= extra; k++)
            if ((r->s[r->p + k] & 0xC0) != 0x80) return PJ_REC_STRING;
        if (out) b_push(out, r->s + r->p, (uint64_t)(1 + extra));
        r->p += 1 + (uint64_t)extra;
    }
}

static int is_ident(uint8_t c) {
    return (c >= 'a' && c <= 'z') || (c >= 'A' && c <= 'Z') || (c >= '0' && c <= '9') ||
           c == '_' || c == '$' || c >= 0x80;
}

/* Scalar token kinds returned by rd_scalar. */
enum { TK_NULL, TK_TRUE, TK_FALSE, TK_INT, TK_REAL };

/* Number grammar of RFC 8259; *kind = TK_INT when no fraction/exponent. */
static int rd_number(rd_t *r, int *kind) {
    uint64_t p = r->p;
    const uint8_t *s = r->s;
    int real = 0;
    if (p < r->n && s[p] == '-') p++;
    if (p >= r->n) return PJ_REC_SYNTAX;
    if (s[p] == '0') {
        p++;
        if (p < r->n && s[p] >= '0' && s[p] <= '9') return PJ_REC_SYNTAX; /* leading zero */
    } else if (s[p] >= '1' && s[p] <= '9') {
        while (p < r->n && s[p] >= '0' && s[p] <= '9') p++;
    } else return PJ_REC_SYNTAX;
    if (p < r->n && s[p] == '.') {
        p++; real = 1;
        if (p >= r->n || s[p] < '0' || s[p] > '9') return PJ_REC_SYNTAX;
        while (p < r->n && s[p] >= '0' && s[p] <= '9') p++;
    }
    if (p < r->n && (s[p] == 'e' || s[p] == 'E')) {
        p++; real = 1;
        if (p < r->n && (s[p] == '+' || s[p] == '-')) p++;
        if (p >= r->n || s[p] < '0' || s[p] > '9') return PJ_REC_SYNTAX;
        while (p < r->n && s[p] >= '0' && s[p] <= '9') p++;
    }
    r->p = p;
    *kind = real ? TK_REAL : TK_INT;
    return PJ_REC_OK;
}

/* Literal or number token at r->p (tokenised by jackson before serde looks
 * at its type). */
static int rd_scalar(rd_t *r, int *kind) {
    static const char *const LIT[3] = {"null", "true", "false"};
    uint8_t c = cur(r);
    if (c == '-' || (c >= '0' && c <= '9')) return rd_number(r, kind);
    int li = c == 'n' ? 0 : c == 't' ? 1 : c == 'f' ? 2 : -1;
    if (li < 0) return PJ_REC_SYNTAX;
    uint64_t L = strlen(LIT[li]);
    if (r->p + L > r->n || memcmp(r->s + r->p, LIT[li], L) != 0) return PJ_REC_SYNTAX;
    if (r->p + L < r->n && is_ident(r->s[r->p + L])) return PJ_REC_SYNTAX;
    r->p += L;
    *kind = li == 0 ? TK_NULL : li == 1 ? TK_TRUE : TK_FALSE;
    return PJ_REC_OK;
}

static int rd_skip_value(rd_t *r);

static int push_depth(rd_t *r) { return ++r->depth > PJ_MAX_DEPTH ? PJ_REC_DEPTH : PJ_REC_OK; }

/* Generic container walker: calls `member` for each object member (key
 * decoded into `key`) or `elem` for each array element.  The callbacks read
 * the value at r->p. */
typedef int (*member_fn)(rd_t *r, const bytes_t *key, void *ctx);
typedef int (*elem_fn)(rd_t *r, void *ctx);

static int rd_object(rd_t *r, member_fn fn, void *ctx) {
    int e = push_depth(r);
    if (e) return e;
    r->p++; /* { */
    skip_ws(r);
    if (cur(r) == '}' && !at_end(r)) { r->p++; r->depth--; return PJ_REC_OK; }
    bytes_t key = {0, 0, 0};
    for (;;) {
        skip_ws(r);
        if (at_end(r) || cur(r) != '"') { e = PJ_REC_SYNTAX; break; }
        key.n = 0;
        if ((e = rd_string(r, &key))) break;
        skip_ws(r);
        if (at_end(r) || cur(r) != ':') { e = PJ_REC_SYNTAX; break; }
        r->p++;
        skip_ws(r);
        if (at_end(r)) { e = PJ_REC_SYNTAX; break; }
        if ((e = fn(r, &key, ctx))) break;
        skip_ws(r);
        if (at_end(r)) { e = PJ_REC_SYNTAX; break; }
        if (cur(r) == ',') { r->p++; continue; }
        if (cur(r) == '}') { r->p++; r->depth--; e = PJ_REC_OK; break; }
        e = PJ_REC_SYNTAX;
        break;
    }
    free(key.p);
    return e;
}

static int rd_array(rd_t *r, elem_fn fn, void *ctx) {
    int e = push_depth(r);
    if (e) return e;
    r->p++; /* [ */
    skip_ws(r);
    if (cur(r) == ']' && !at_end(r)) { r->p++; r->depth--; return PJ_REC_OK; }
    for (;;) {
        skip_ws(r);
        if (at_end(r)) return PJ_REC_SYNTAX;
        if ((e = fn(r, ctx))) return e;
        skip_ws(r);
        if (at_end(r)) return PJ_REC_SYNTAX;
        if (cur(r) == ',') { r->p++; continue; }
        if (cur(r) == ']') { r->p++; r->depth--; return PJ_REC_OK; }
        return PJ_REC_SYNTAX;
    }
}

static int skip_member(rd_t *r, const bytes_t *k, void *c) { (void)k; (void)c; return rd_skip_value(r); }
static int skip_elem(rd_t *r, void *c) { (void)c; return rd_skip_value(r); }

/* Any JSON value (unknown properties are skipped after full validation). */
static int rd_skip_value(rd_t *r) {
    int kind;
    switch (cur(r)) {
    case '"': return rd_string(r, NULL);
    case '{': return rd_object(r, skip_member, NULL);
    case '[': return rd_array(r, skip_elem, NULL);
    default: return rd_scalar(r, &kind);
    }
}

/* A value of a known property whose JSON type does not match: literals and
 * numbers are still tokenised first (SYNTAX if malformed), then TYPE. */
static int type_mismatch(rd_t *r) {
    int kind;
    uint8_t c = cur(r);
    if (c == '"' || c == '{' || c == '[') return PJ_REC_TYPE;
    int e = rd_scalar(r, &kind);
    return e ? e : PJ_REC_TYPE;
}

/* Long property: integer token in int64 range, or null (=> absent). */
static int rd_long(rd_t *r, int64_t *v, int *present) {
    uint8_t c = cur(r);
    if (c == 'n') {
        int kind, e = rd_scalar(r, &kind);
        if (e) return e;
        if (kind != TK_NULL) return PJ_REC_TYPE;
        *present = 0;
        return PJ_REC_OK;
    }
    if (!(c == '-' || (c >= '0' && c <= '9'))) return type_mismatch(r);
    uint64_t start = r->p;
    int kind, e = rd_number(r, &kind);
    if (e) return e;
    if (kind != TK_INT) return PJ_REC_NUMBER;   /* unpinned: no float->long coercion */
    int neg = r->s[start] == '-';
    uint64_t acc = 0, lim = neg ? (uint64_t)1 << 63 : ((uint64_t)1 << 63) - 1;
    for (uint64_t q = start + (uint64_t)neg; q < r->p; q++) {
        uint64_t d = (uint64_t)(r->s[q] - '0');
        if (acc > (lim - d) / 10) return PJ_REC_NUMBER;            /* out of range */
        acc = acc * 10 + d;
    }
    *v = neg ? (int64_t)(0 - acc) : (int64_t)acc;
    *present = 1;
    return PJ_REC_OK;
}

/* String property: string, or null (=> absent). */
static int rd_str_prop(rd_t *r, bytes_t *out, int *present) {
    uint8_t c = cur(r);
    if (c == '"') { out->n = 0; *present = 1; return rd_string(r, out); }
    if (c == 'n') {
        int kind, e = rd_scalar(r, &kind);
        if (e) return e;
        if (kind != TK_NULL) return PJ_REC_TYPE;
        *present = 0;
        return PJ_REC_OK;
    }
    return type_mismatch(r);
}

static int key_is(const bytes_t *k, const char *s) {
    uint64_t n = strlen(s);
    return k->n == n && memcmp(k->p, s, n) == 0;
}

/* Category / Tag members (petstore.json:858-871, 923-936). */
static int sub_member(rd_t *r, const bytes_t *k, void *ctx) {
    sub_t *t = (sub_t *)ctx;
    int pres, e;
    if (key_is(k, "id")) {
        int64_t v = 0;
        if ((e = rd_long(r, &v, &pres))) return e;
        if (pres) { t->id = v; t->flags |= PJ_SUB_HAS_ID; }
        else { t->id = 0; t->flags &= (uint8_t)~PJ_SUB_HAS_ID; }
        return PJ_REC_OK;
    }
    if (key_is(k, "name")) {
        if ((e = rd_str_prop(r, &t->name, &pres))) return e;
        if (pres) t->flags |= PJ_SUB_HAS_NAME;
        else { t->flags &= (uint8_t)~PJ_SUB_HAS_NAME; t->name.n = 0; }
        return PJ_REC_OK;
    }
    return rd_skip_value(r);
}

static int rd_sub(rd_t *r, sub_t *t) {
    t->id = 0; t->flags = 0; t->name.n = 0;
    return rd_object(r, sub_member, t);
}

static int url_elem(rd_t *r, void *ctx) {
    pet_t *pt = (pet_t *)ctx;
    if (cur(r) != '"') return type_mismatch(r);   /* null element: unpinned, rejected */
    uint64_t before = pt->urls.n;
    int e = rd_string(r, &pt->urls);
    if (e) return e;
    if (pt->n_urls == pt->cap_urls) {
        pt->cap_urls = pt->cap_urls ? pt->cap_urls * 2 : 8;
        pt->url_len = (uint64_t *)realloc(pt->url_len, pt->cap_urls * sizeof(uint64_t));
    }
    pt->url_len[pt->n_urls++] = pt->urls.n - before;
    return PJ_REC_OK;
}

static int tag_elem(rd_t *r, void *ctx) {
    pet_t *pt = (pet_t *)ctx;
    if (cur(r) != '{') return type_mismatch(r);   /* null element: unpinned, rejected */
    if (pt->n_tags == pt->cap_tags) {
        uint64_t nc = pt->cap_tags ? pt->cap_tags * 2 : 8;
        pt->tags = (sub_t *)realloc(pt->tags, nc * sizeof(sub_t));
        memset(pt->tags + pt->cap_tags, 0, (nc - pt->cap_tags) * sizeof(sub_t));
        pt->cap_tags = nc;
    }
    return rd_sub(r, &pt->tags[pt->n_tags++]);
}

static int pet_member(rd_t *r, const bytes_t *k, void *ctx) {
    pet_t *pt = (pet_t *)ctx;
    int pres, e;
    uint8_t c = cur(r);
    if (key_is(k, "id")) {
        int64_t v = 0;
        if ((e = rd_long(r, &v, &pres))) return e;
        pt->has_id = pres; pt->id = pres ? v : 0;
        return PJ_REC_OK;
    }
    if (key_is(k, "category")) {
        if (c == '{') { pt->has_cat = 1; return rd_sub(r, &pt->cat); }
        if (c == 'n') {
            int kind;
            if ((e = rd_scalar(r, &kind))) return e;
            if (kind != TK_NULL) return PJ_REC_TYPE;
            pt->has_cat = 0;
            return PJ_REC_OK;
        }
        return type_mismatch(r);
    }
    if (key_is(k, "name")) {
        if ((e = rd_str_prop(r, &pt->name, &pres))) return e;
        pt->has_name = pres;
        if (!pres) pt->name.n = 0;
        return PJ_REC_OK;
    }
    if (key_is(k, "photoUrls")) {
        if (c == '[') {
            pt->has_photo = 1; pt->n_urls = 0; pt->urls.n = 0;   /* last one wins */
            return rd_array(r, url_elem, pt);
        }
        if (c == 'n') {
            int kind;
            if ((e = rd_scalar(r, &kind))) return e;
            if (kind != TK_NULL) return PJ_REC_TYPE;
            pt->has_photo = 0; pt->n_urls = 0; pt->urls.n = 0;
            return PJ_REC_OK;
        }
        return type_mismatch(r);
    }
    if (key_is(k, "tags")) {
        if (c == '[') {
            pt->has_tags = 1; pt->n_tags = 0;
            return rd_array(r, tag_elem, pt);
        }
        if (c == 'n') {
            int kind;
            if ((e = rd_scalar(r, &kind))) return e;
            if (kind != TK_NULL) return PJ_REC_TYPE;
            pt->has_tags = 0; pt->n_tags = 0;
            return PJ_REC_OK;
        }
        return type_mismatch(r);
    }
    if (key_is(k, "status")) {
        bytes_t v = {0, 0, 0};
        e = rd_str_prop(r, &v, &pres);
        if (!e) {
            if (!pres) pt->status = PJ_STATUS_NULL;
            else {
                int m = -1;
                for (int s = 0; s < 3; s++) if (key_is(&v, STATUS_TXT[s])) m = s;
                if (m < 0) e = PJ_REC_BAD_STATUS;  /* @JsonCreator rejects unknown */
                else pt->status = (uint8_t)m;
            }
        }
        free(v.p);
        return e;
    }
    return rd_skip_value(r);
}

static void pet_free(pet_t *pt) {
    free(pt->cat.name.p); free(pt->name.p); free(pt->urls.p); free(pt->url_len);
    for (uint64_t t = 0; t < pt->cap_tags; t++) free(pt->tags[t].name.p);
    free(pt->tags);
}

/* Append the finished pet to the output columns (capacity-checked: only
 * counts past the capacity). */
static void commit(const pet_t *pt, pj_pet_columns *o, pj_decode_result *f) {
    uint64_t i = f->n_pets;
    int fits_row = o && i < o->cap_pets;
    if (fits_row) {
        o->id[i] = pt->has_id ? pt->id : 0;
        o->flags[i] = (uint8_t)((pt->has_id ? PJ_PET_HAS_ID : 0) | (pt->has_cat ? PJ_PET_HAS_CATEGORY : 0) |
                                PJ_PET_HAS_NAME | PJ_PET_HAS_PHOTOURLS | (pt->has_tags ? PJ_PET_HAS_TAGS : 0));
        o->status[i] = pt->status;
        o->cat_id[i] = pt->has_cat && (pt->cat.flags & PJ_SUB_HAS_ID) ? pt->cat.id : 0;
        o->cat_flags[i] = pt->has_cat ? pt->cat.flags : 0;
    }
    /* name */
    if (o && pt->name.n && f->name_bytes + pt->name.n <= o->cap_name_bytes)
        memcpy(o->name_bytes + f->name_bytes, pt->name.p, pt->name.n);
    f->name_bytes += pt->name.n;
    /* category name */
    uint64_t cn = pt->has_cat ? pt->cat.name.n : 0;
    if (o && cn && f->cat_name_bytes + cn <= o->cap_cat_name_bytes)
        memcpy(o->cat_name_bytes + f->cat_name_bytes, pt->cat.name.p, cn);
    f->cat_name_bytes += cn;
    /* urls */
    uint64_t ub = 0;
    for (uint64_t u = 0; u < pt->n_urls; u++) {
        uint64_t L = pt->url_len[u];
        if (o && L && f->url_bytes + L <= o->cap_url_bytes)
            memcpy(o->url_bytes + f->url_bytes, pt->urls.p + ub, L);
        ub += L;
        f->url_bytes += L;
        f->n_urls++;
        if (o && f->n_urls <= o->cap_urls) o->url_off[f->n_urls] = f->url_bytes;
    }
    /* tags */
    for (uint64_t t = 0; t < pt->n_tags; t++) {
        const sub_t *g = &pt->tags[t];
        uint64_t L = g->name.n;
        if (o && f->n_tags < o->cap_tags) {
            o->tag_id[f->n_tags] = (g->flags & PJ_SUB_HAS_ID) ? g->id : 0;
            o->tag_flags[f->n_tags] = g->flags;
        }
        if (o && L && f->tag_name_bytes + L <= o->cap_tag_name_bytes)
            memcpy(o->tag_name_bytes + f->tag_name_bytes, g->name.p, L);
        f->tag_name_bytes += L;
        f->n_tags++;
        if (o && f->n_tags <= o->cap_tags) o->tag_name_off[f->n_tags] = f->tag_name_bytes;
    }
    f->n_pets++;
    if (o && f->n_pets <= o->cap_pets) {
        o->name_off[f->n_pets] = f->name_bytes;
        o->cat_name_off[f->n_pets] = f->cat_name_bytes;
        o->photo_off[f->n_pets] = f->n_urls;
        o->tag_off[f->n_pets] = f->n_tags;
    }
}

/* One NDJSON line (without '\n') => one Pet (readValue(line, Pet.class)). */
int or_decode_line(const uint8_t *s, uint64_t n, pj_pet_columns *out, pj_decode_result *fill) {
    rd_t r = {s, n, 0, 0};
    skip_ws(&r);
    if (at_end(&r)) return PJ_REC_EMPTY;                       /* unpinned */
    if (cur(&r) != '{') return type_mismatch(&r);
    pet_t pt;
    memset(&pt, 0, sizeof pt);
    pt.status = PJ_STATUS_NULL;
    int e = rd_object(&r, pet_member, &pt);
    if (!e) {
        if (!pt.has_name) e = PJ_REC_MISSING_NAME;              /* required :873-876 */
        else if (!pt.has_photo) e = PJ_REC_MISSING_PHOTOURLS;
    }
    if (!e) {
        skip_ws(&r);
        if (!at_end(&r)) e = PJ_REC_SYNTAX;                     /* trailing bytes */
    }
    if (!e && fill) commit(&pt, out, fill);
    pet_free(&pt);
    return e;
}

int or_decode(const uint8_t *in, uint64_t len, pj_pet_columns *out, uint64_t *err_line,
              uint8_t *err_code, uint64_t err_cap, pj_decode_result *res) {
    if (!res || (len && !in)) return PJ_ERR_INVALID_ARG;
    memset(res, 0, sizeof *res);
    if (out && out->cap_pets + 1 > 0) {
        if (out->name_off) out->name_off[0] = 0;
        if (out->cat_name_off) out->cat_name_off[0] = 0;
        if (out->photo_off) out->photo_off[0] = 0;
        if (out->tag_off) out->tag_off[0] = 0;
        if (out->url_off) out->url_off[0] = 0;
        if (out->tag_name_off) out->tag_name_off[0] = 0;
    }
    uint64_t p = 0, line = 0;
    while (p < len) {
        const uint8_t *nl = (const uint8_t *)memchr(in + p, '\n', len - p);
        uint64_t e = nl ? (uint64_t)(nl - in) : len;
        int code = or_decode_line(in + p, e - p, out, res);
        if (code) {
            if (res->n_errors < err_cap) {
                if (err_line) err_line[res->n_errors] = line;
                if (err_code) err_code[res->n_errors] = (uint8_t)code;
            }
            res->n_errors++;
        }
        line++;
        p = e + 1;
    }
    res->n_lines = line;
    if (out) out->n_pets = res->n_pets < out->cap_pets ? res->n_pets : out->cap_pets;
    if (res->n_errors > err_cap) return PJ_ERR_CAPACITY;
    if (out && (res->n_pets > out->cap_pets || res->name_bytes > out->cap_name_bytes ||
                res->cat_name_bytes > out->cap_cat_name_bytes || res->n_urls > out->cap_urls ||
                res->url_bytes > out->cap_url_bytes || res->n_tags > out->cap_tags ||
                res->tag_name_bytes > out->cap_tag_name_bytes))
        return PJ_ERR_CAPACITY;
    return PJ_OK;
}

/* The frame of one array document: whitespace, '[', then the top-level
 * commas, found by counting '[' '{' ']' '}' outside strings (a quote opens or
 * closes a string unless a backslash escapes it; a backslash escapes the next
 * byte, in strings or not), up to the ']' that brings the count back to
 * zero; only whitespace may follow.  Element k spans [start[k], start[k+1] -
 * 1), the last one ending at the ']' (*close).  A broken frame or an element
 * of whitespace only gives PJ_ERR_SYNTAX; "[ ]" has no element.  *start is
 * malloc'ed (free it). */
static int array_frame(const uint8_t *in, uint64_t len, uint64_t **start_out, uint64_t *ne_out, uint64_t *close_out) {
    uint64_t p = 0;
    while (p < len && is_ws(in[p])) p++;
    if (p >= len || in[p] != '[') return PJ_ERR_SYNTAX;
    /* the frame: element bounds */
    uint64_t cap = 16, ne = 0, *start = (uint64_t *)malloc(cap * sizeof *start);
    if (!start) return PJ_ERR_OUT_OF_MEMORY;
    start[ne++] = p + 1;
    int in_str = 0, esc = 0;
    int64_t depth = 1;
    uint64_t close = len;
    for (uint64_t i = p + 1; i < len; i++) {
        const uint8_t c = in[i];
        if (esc) { esc = 0; continue; }
        if (c == '\\') { esc = 1; continue; }
        if (c == '"') { in_str ^= 1; continue; }
        if (in_str) continue;
        if (c == '[' || c == '{') depth++;
        else if (c == ']' || c == '}') {
            if (--depth == 0) { close = i; break; }
        } else if (c == ',' && depth == 1) {
            if (ne == cap) {
                uint64_t *t = (uint64_t *)realloc(start, 2 * cap * sizeof *start);
                if (!t) { free(start); return PJ_ERR_OUT_OF_MEMORY; }
                start = t;
                cap *= 2;
            }
            start[ne++] = i + 1;
        }
    }
    int bad = close >= len || in[close] != ']';
    for (uint64_t i = close + 1; !bad && i < len; i++) bad = !is_ws(in[i]);
    if (bad) { free(start); return PJ_ERR_SYNTAX; }
    /* elements: [start[k], start[k+1] - 1), the last ending at the ']' */
    for (uint64_t k = 0; k < ne; k++) {
        const uint64_t a = start[k], e = k + 1 < ne ? start[k + 1] - 1 : close;
        uint64_t q = a;
        while (q < e && is_ws(in[q])) q++;
        if (q == e) {
            if (ne == 1) { ne = 0; break; }        /* "[ ]": no element */
            free(start);
            return PJ_ERR_SYNTAX;                   /* an empty element */
        }
    }
    *start_out = start;
    *ne_out = ne;
    *close_out = close;
    return PJ_OK;
}

/* One JSON array of Pets => its elements (readValue(bytes, List<Pet>), the
 * reference's bulk shape "array of Pet", petstore.json:133-140, read as in
 * MyEntityConfig.java:34).  The array's frame is read first, sequentially:
 * whitespace, '[', then the top-level commas, found by counting '[' '{' ']'
 * '}' outside strings (a quote opens or closes a string unless a backslash
 * escapes it; a backslash escapes the next byte, in strings or not), up to
 * the ']' that brings the count back to zero; only whitespace may follow.
 * A broken frame (no '[', never closed, closed by '}', bytes after it, an
 * element of whitespace only) fails the whole call with PJ_ERR_SYNTAX, as
 * jackson's parser throws for it.  Each element is then read exactly as an
 * NDJSON line (or_decode_line, '\n' being whitespace) and reported under its
 * index.  "[]" and "[ ]" hold no element. */
int or_decode_array(const uint8_t *in, uint64_t len, pj_pet_columns *out, uint64_t *err_line,
                    uint8_t *err_code, uint64_t err_cap, pj_decode_result *res) {
    if (!res || (len && !in)) return PJ_ERR_INVALID_ARG;
    memset(res, 0, sizeof *res);
    if (out && out->cap_pets + 1 > 0) {
        if (out->name_off) out->name_off[0] = 0;
        if (out->cat_name_off) out->cat_name_off[0] = 0;
        if (out->photo_off) out->photo_off[0] = 0;
        if (out->tag_off) out->tag_off[0] = 0;
        if (out->url_off) out->url_off[0] = 0;
        if (out->tag_name_off) out->tag_name_off[0] = 0;
    }
    uint64_t *start = NULL, ne = 0, close = 0;
    const int fs = array_frame(in, len, &start, &ne, &close);
    if (fs) return fs;
    for (uint64_t k = 0; k < ne; k++) {
        const uint64_t a = start[k], e = k + 1 < ne ? start[k + 1] - 1 : close;
        int code = or_decode_line(in + a, e - a, out, res);
        if (code) {
            if (res->n_errors < err_cap) {
                if (err_line) err_line[res->n_errors] = k;
                if (err_code) err_code[res->n_errors] = (uint8_t)code;
            }
            res->n_errors++;
        }
    }
    free(start);
    res->n_lines = ne;
    if (out) out->n_pets = res->n_pets < out->cap_pets ? res->n_pets : out->cap_pets;
    if (res->n_errors > err_cap) return PJ_ERR_CAPACITY;
    if (out && (res->n_pets > out->cap_pets || res->name_bytes > out->cap_name_bytes ||
                res->cat_name_bytes > out->cap_cat_name_bytes || res->n_urls > out->cap_urls ||
                res->url_bytes > out->cap_url_bytes || res->n_tags > out->cap_tags ||
                res->tag_name_bytes > out->cap_tag_name_bytes))
        return PJ_ERR_CAPACITY;
    return PJ_OK;
}

/* ======================================================================
 *                       ORDER AND USER MODELS
 * ======================================================================
 * Schemas: reference petstore.json:824-857 (User: id int64, username,
 * firstName, lastName, email, password, phone, userStatus int32) and
 * :937-971 (Order: id int64, petId int64, quantity int32, shipDate
 * date-time, status enum placed/approved/delivered :955-963, complete
 * boolean).  No property is required.  Properties are written in schema
 * order with the same inclusion, escape and number rules as Pet.
 * Parity unpinned: shipDate is carried as the text written (a generated
 * class would hold an OffsetDateTime that serde formats itself), booleans
 * accept only true / false / null (no coercion from numbers or strings). */

enum { MK_I64, MK_I32, MK_STR, MK_ENUM, MK_BOOL };
typedef struct { const char *name; int kind; } mprop_t;
typedef struct { int n; const mprop_t *p; const char *const *enum_txt; } mschema_t;

static const mprop_t ORDER_PROPS[6] = {{"id", MK_I64}, {"petId", MK_I64}, {"quantity", MK_I32},
                                       {"shipDate", MK_STR}, {"status", MK_ENUM}, {"complete", MK_BOOL}};
static const char *const ORDER_STATUS[3] = {"placed", "approved", "delivered"};
static const mprop_t USER_PROPS[8] = {{"id", MK_I64}, {"username", MK_STR}, {"firstName", MK_STR},
                                      {"lastName", MK_STR}, {"email", MK_STR}, {"password", MK_STR},
                                      {"phone", MK_STR}, {"userStatus", MK_I32}};

static const mschema_t *schema_of(int model) {
    static const mschema_t ORDER = {6, ORDER_PROPS, ORDER_STATUS}, USER = {8, USER_PROPS, NULL};
    return model == PJ_MODEL_ORDER ? &ORDER : model == PJ_MODEL_USER ? &USER : NULL;
}

static void w_model(wbuf *w, const mschema_t *S, const pj_model_columns *c, const pj_options *o, uint64_t i) {
    int first = 1;
    o_start(w);
    for (int k = 0; k < S->n; k++) {
        const mprop_t *pr = &S->p[k];
        int present = c->present ? (c->present[i] >> k) & 1 : 1;
        if (present && pr->kind == MK_ENUM && ((const uint8_t *)c->col[k])[i] > 2) present = 0;
        if (!present) {
            if (o->inclusion == PJ_INCLUDE_ALWAYS) { w_key(w, &first, pr->name); w_lit(w, "null"); }
            continue;
        }
        if (pr->kind == MK_STR) {
            const uint64_t *off = (const uint64_t *)c->col[k];
            const uint64_t a = off[i], b = off[i + 1];
            if (b == a && o->inclusion == PJ_INCLUDE_NON_EMPTY) continue;   /* "" is empty */
            w_key(w, &first, pr->name);
            w_string(w, c->bytes[k] + a, b - a, o->hex_upper);
            continue;
        }
        w_key(w, &first, pr->name);
        switch (pr->kind) {
        case MK_I64: w_long(w, ((const int64_t *)c->col[k])[i]); break;
        case MK_I32: w_long(w, ((const int32_t *)c->col[k])[i]); break;
        case MK_ENUM:
            w_char(w, '"');
            w_lit(w, S->enum_txt[((const uint8_t *)c->col[k])[i]]);
            w_char(w, '"');
            break;
        default: w_lit(w, ((const uint8_t *)c->col[k])[i] ? "true" : "false"); break;
        }
    }
    o_end(w, first);
}

int or_encode_model(int model, const pj_model_columns *cols, const pj_options *opt, int format,
                    uint8_t *out, uint64_t out_cap, uint64_t *out_len) {
    pj_options def;
    or_default_options(&def);
    const mschema_t *S = schema_of(model);
    if (!S || !cols || !out_len ||
        (format != PJ_FORMAT_ARRAY && format != PJ_FORMAT_NDJSON && format != PJ_FORMAT_PRETTY))
        return PJ_ERR_INVALID_ARG;
    if (!opt) opt = &def;
    wbuf w = {out, out_cap, 0, format == PJ_FORMAT_PRETTY, 0};
    const int array = format != PJ_FORMAT_NDJSON;
    if (array) a_start(&w);
    for (uint64_t i = 0; i < cols->n; i++) {
        if (array) a_value(&w, i);
        w_model(&w, S, cols, opt, i);
        if (!array) w_char(&w, '\n');
    }
    if (array) a_end(&w);
    *out_len = w.len;
    return w.len > out_cap ? PJ_ERR_CAPACITY : PJ_OK;
}

typedef struct {            /* one Order / User while it is being read */
    const mschema_t *S;
    uint8_t present;
    int64_t v[PJ_MODEL_MAX_PROPS];
    bytes_t str[PJ_MODEL_MAX_PROPS];
} mrec_t;

static int model_member(rd_t *r, const bytes_t *k, void *ctx) {
    mrec_t *m = (mrec_t *)ctx;
    int f = -1;
    for (int j = 0; j < m->S->n; j++)
        if (key_is(k, m->S->p[j].name)) f = j;
    if (f < 0) return rd_skip_value(r);
    const uint8_t bit = (uint8_t)(1u << f);
    int pres = 0, e, kind;
    int64_t v = 0;
    switch (m->S->p[f].kind) {
    case MK_I64:
    case MK_I32:
        if ((e = rd_long(r, &v, &pres))) return e;
        if (pres && m->S->p[f].kind == MK_I32 && (v < INT32_MIN || v > INT32_MAX))
            return PJ_REC_NUMBER;                           /* out of int range */
        break;
    case MK_STR:
        if ((e = rd_str_prop(r, &m->str[f], &pres))) return e;
        if (!pres) m->str[f].n = 0;
        break;
    case MK_ENUM: {
        bytes_t t = {0, 0, 0};
        e = rd_str_prop(r, &t, &pres);
        if (!e && pres) {
            int hit = -1;
            for (int s = 0; s < 3; s++) if (key_is(&t, m->S->enum_txt[s])) hit = s;
            if (hit < 0) e = PJ_REC_BAD_STATUS;             /* @JsonCreator rejects unknown */
            v = hit;
        }
        free(t.p);
        if (e) return e;
        break;
    }
    default: {                                              /* MK_BOOL */
        const uint8_t c = cur(r);
        if (c == '"' || c == '{' || c == '[') return PJ_REC_TYPE;
        if ((e = rd_scalar(r, &kind))) return e;
        if (kind == TK_INT || kind == TK_REAL) return PJ_REC_TYPE;
        pres = kind != TK_NULL;
        v = kind == TK_TRUE;
        break;
    }
    }
    if (pres) { m->present |= bit; m->v[f] = v; }
    else { m->present &= (uint8_t)~bit; m->v[f] = 0; }
    return PJ_REC_OK;
}

/* Append a finished record (capacity-checked: only counts past it). */
static void model_commit(const mrec_t *m, pj_model_columns *o, pj_decode_result *f) {
    const uint64_t i = f->n_pets;
    const int row = o && i < o->cap_n;
    if (row && o->present) o->present[i] = m->present;
    for (int k = 0; k < m->S->n; k++) {
        const int kind = m->S->p[k].kind;
        if (kind == MK_STR) {
            const uint64_t L = m->str[k].n;
            if (o && L && o->n_bytes[k] + L <= o->cap_bytes[k]) memcpy(o->bytes[k] + o->n_bytes[k], m->str[k].p, L);
            if (o) o->n_bytes[k] += L;
            if (row) ((uint64_t *)o->col[k])[i + 1] = o->n_bytes[k];
        } else if (row) {
            if (kind == MK_I64) ((int64_t *)o->col[k])[i] = m->v[k];
            else if (kind == MK_I32) ((int32_t *)o->col[k])[i] = (int32_t)m->v[k];
            else ((uint8_t *)o->col[k])[i] = (uint8_t)m->v[k];
        }
    }
    f->n_pets++;
}

/* One record (an NDJSON line without its '\n', or an array element), read
 * as or_decode_line reads a Pet. */
static int model_line(const mschema_t *S, const uint8_t *s, uint64_t n, pj_model_columns *out,
                      pj_decode_result *fill) {
    rd_t r = {s, n, 0, 0};
    skip_ws(&r);
    if (at_end(&r)) return PJ_REC_EMPTY;
    if (cur(&r) != '{') return type_mismatch(&r);
    mrec_t m;
    memset(&m, 0, sizeof m);
    m.S = S;
    int e = rd_object(&r, model_member, &m);
    if (!e) {
        skip_ws(&r);
        if (!at_end(&r)) e = PJ_REC_SYNTAX;
    }
    if (!e) model_commit(&m, out, fill);
    for (int k = 0; k < PJ_MODEL_MAX_PROPS; k++) free(m.str[k].p);
    return e;
}

int or_decode_model(int model, const uint8_t *in, uint64_t len, int array, pj_model_columns *out,
                    uint64_t *err_line, uint8_t *err_code, uint64_t err_cap, pj_decode_result *res) {
    const mschema_t *S = schema_of(model);
    if (!S || !res || (len && !in)) return PJ_ERR_INVALID_ARG;
    memset(res, 0, sizeof *res);
    if (out) {
        for (int k = 0; k < S->n; k++) {
            out->n_bytes[k] = 0;
            if (S->p[k].kind == MK_STR && out->col[k]) ((uint64_t *)out->col[k])[0] = 0;
        }
    }
    uint64_t *start = NULL, ne = 0, close = 0;
    if (array) {
        const int fs = array_frame(in, len, &start, &ne, &close);
        if (fs) return fs;
    }
    /* records: the array's elements, or the lines cut at every '\n' */
    for (uint64_t k = 0, p = 0; array ? k < ne : p < len; k++) {
        uint64_t a, e;
        if (array) {
            a = start[k];
            e = k + 1 < ne ? start[k + 1] - 1 : close;
        } else {
            const uint8_t *nl = (const uint8_t *)memchr(in + p, '\n', len - p);
            a = p;
            e = nl ? (uint64_t)(nl - in) : len;
            p = e + 1;
            ne = k + 1;
        }
        const int code = model_line(S, in + a, e - a, out, res);
        if (code) {
            if (res->n_errors < err_cap) {
                if (err_line) err_line[res->n_errors] = k;
                if (err_code) err_code[res->n_errors] = (uint8_t)code;
            }
            res->n_errors++;
        }
    }
    free(start);
    res->n_lines = ne;
    if (out) out->n = res->n_pets < out->cap_n ? res->n_pets : out->cap_n;
    if (res->n_errors > err_cap) return PJ_ERR_CAPACITY;
    if (out) {
        if (res->n_pets > out->cap_n) return PJ_ERR_CAPACITY;
        for (int k = 0; k < S->n; k++)
            if (out->n_bytes[k] > out->cap_bytes[k]) return PJ_ERR_CAPACITY;
    }
    return PJ_OK;
}
