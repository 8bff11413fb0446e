// pj_model.hip — decoding of the petstore's Order and User models (gfx950).
//
// readValue of Order / User records (reference petstore.json:937-971 Order,
// :824-857 User), one thread per record after the shared record index
// (k_dec_lines for NDJSON, the array frame kernels for one array document):
//   k_mdec_count  reads each record and sums, per block of records, the
//                 valid ones, the invalid ones and the decoded bytes of each
//                 string property;
//   k_mdec_scan_* turn those sums into each block's first offsets;
//   k_mdec_write  reads each record again and writes its values, or its
//                 error slot, at the offsets a block scan gives.
// The grammar and binding rules are the Pet decoder's: RFC 8259 with
// jackson's string and literal rules, nesting limit 1000, keys in any order,
// the last duplicate wins, unknown keys validated and skipped, null means
// absent; an integer property takes an integer token in its type's range.
#include "pj_device.h"
#include "pj_kernels.h"

namespace pj {
namespace {

enum MKind { K_I64, K_I32, K_STR, K_ENUM, K_BOOL };
enum MTok { T_NULL, T_TRUE, T_FALSE, T_INT, T_REAL };

struct MLine {
    const uint8_t *s;
    uint64_t n, p;
};

__device__ __forceinline__ bool m_is_ws(uint32_t c) { return c == ' ' || c == '\t' || c == '\r' || c == '\n'; }
__device__ __forceinline__ void m_skip_ws(MLine &L) {
    while (L.p < L.n && m_is_ws(L.s[L.p])) L.p++;
}
__device__ __forceinline__ bool m_end(const MLine &L) { return L.p >= L.n; }
__device__ __forceinline__ uint32_t m_cur(const MLine &L) { return L.p < L.n ? L.s[L.p] : 0u; }
__device__ __forceinline__ int m_hex(uint32_t c) {
    if (c >= '0' && c <= '9') return (int)(c - '0');
    if (c >= 'a' && c <= 'f') return (int)(c - 'a' + 10);
    if (c >= 'A' && c <= 'F') return (int)(c - 'A' + 10);
    return -1;
}
// bytes that may not follow a literal (jackson reads them as part of it)
__device__ __forceinline__ bool m_ident(uint32_t c) {
    return (c >= 'a' && c <= 'z') || (c >= 'A' && c <= 'Z') || (c >= '0' && c <= '9') || c == '_' || c == '$' ||
           c >= 0x80;
}

// Decoded string bytes go to dst (when non-null) and the first 16 into two
// packed words (key matching).
struct MOut {
    uint8_t *dst;
    uint64_t k = 0, w0 = 0, w1 = 0;
    __device__ __forceinline__ void put(uint32_t b) {
        if (dst) dst[k] = (uint8_t)b;
        if (k < 8) w0 |= (uint64_t)(b & 0xFF) << (8 * k);
        else if (k < 16) w1 |= (uint64_t)(b & 0xFF) << (8 * (k - 8));
        k++;
    }
    __device__ __forceinline__ void put8(uint64_t x) {   // 8 bytes at once
        if (k < 16) {
            for (int j = 0; j < 8; j++) put((uint32_t)(x >> (8 * j)));
            return;
        }
        if (dst) stu64(dst + k, x);
        k += 8;
    }
};

__device__ __forceinline__ bool m_u4(MLine &L, uint32_t *cu) {
    if (L.p + 4 > L.n) return false;
    uint32_t v = 0;
    for (int k = 0; k < 4; k++) {
        const int h = m_hex(L.s[L.p + k]);
        if (h < 0) return false;
        v = v * 16 + (uint32_t)h;
    }
    L.p += 4;
    *cu = v;
    return true;
}

// A string starting at its opening quote: escapes (\uXXXX pairs joined,
// lone surrogates rejected), no raw controls, UTF-8 lead bytes C0-DF /
// E0-EF / F0-F7 each with its 10xxxxxx continuations.
// The writing pass's string output: the decoded bytes gather in a register
// and leave as 8-byte stores at any address, the tail exact.
struct MStore {
    StoreSink ss;
    uint64_t k = 0;
    __device__ __forceinline__ explicit MStore(uint8_t *dst) { ss.init(dst); }
    __device__ __forceinline__ void put(uint32_t b) {
        ss.put8(b & 0xFF, 1);
        k++;
    }
    __device__ __forceinline__ void put8(uint64_t x) {
        ss.put8(x, 8);
        k += 8;
    }
    __device__ __forceinline__ void finish() { ss.finish(); }
};

template <class O> __device__ __forceinline__ int m_string(MLine &L, O &o) {
    L.p++;
    for (;;) {
        // 8 bytes at a time while none is a quote, a backslash, a control
        // byte or a UTF-8 byte
        while (L.p + 8 <= L.n) {
            const uint64_t x = ldu64(L.s + L.p);
            if (special64(x) | (x & (0x80 * ONES))) break;
            o.put8(x);
            L.p += 8;
        }
        if (m_end(L)) return PJ_REC_STRING;
        const uint32_t c = L.s[L.p];
        if (c == '"') {
            L.p++;
            return PJ_REC_OK;
        }
        if (c == '\\') {
            L.p++;
            if (m_end(L)) return PJ_REC_STRING;
            const uint32_t e = L.s[L.p++];
            uint32_t b;
            switch (e) {
            case '"': b = '"'; break;
            case '\\': b = '\\'; break;
            case '/': b = '/'; break;
            case 'b': b = 8; break;
            case 'f': b = 12; break;
            case 'n': b = 10; break;
            case 'r': b = 13; break;
            case 't': b = 9; break;
            case 'u': {
                uint32_t cu, lo;
                if (!m_u4(L, &cu)) return PJ_REC_STRING;
                if (cu >= 0xDC00 && cu <= 0xDFFF) return PJ_REC_STRING;
                if (cu >= 0xD800 && cu <= 0xDBFF) {
                    if (L.p + 2 > L.n || L.s[L.p] != '\\' || L.s[L.p + 1] != 'u') return PJ_REC_STRING;
                    L.p += 2;
                    if (!m_u4(L, &lo) || lo < 0xDC00 || lo > 0xDFFF) return PJ_REC_STRING;
                    cu = 0x10000 + ((cu - 0xD800) << 10) + (lo - 0xDC00);
                }
                if (cu < 0x80) o.put(cu);
                else if (cu < 0x800) {
                    o.put(0xC0 | (cu >> 6));
                    o.put(0x80 | (cu & 63));
                } else if (cu < 0x10000) {
                    o.put(0xE0 | (cu >> 12));
                    o.put(0x80 | ((cu >> 6) & 63));
                    o.put(0x80 | (cu & 63));
                } else {
                    o.put(0xF0 | (cu >> 18));
                    o.put(0x80 | ((cu >> 12) & 63));
                    o.put(0x80 | ((cu >> 6) & 63));
                    o.put(0x80 | (cu & 63));
                }
                continue;
            }
            default: return PJ_REC_STRING;
            }
            o.put(b);
            continue;
        }
        if (c < 0x20) return PJ_REC_STRING;
        uint32_t extra;
        if (c < 0x80) extra = 0;
        else if (c >= 0xC0 && c <= 0xDF) extra = 1;
        else if (c >= 0xE0 && c <= 0xEF) extra = 2;
        else if (c >= 0xF0 && c <= 0xF7) extra = 3;
        else return PJ_REC_STRING;
        if (L.p + 1 + extra > L.n) return PJ_REC_STRING;
        for (uint32_t k = 1; k <= extra; k++)
            if ((L.s[L.p + k] & 0xC0) != 0x80) return PJ_REC_STRING;
        for (uint32_t k = 0; k <= extra; k++) o.put(L.s[L.p + k]);
        L.p += 1 + extra;
    }
}

// A number token (RFC 8259 grammar): T_INT without fraction or exponent,
// with its value in *v and *big set when it is outside the int64 range.
__device__ __forceinline__ int m_number(MLine &L, int *kind, int64_t *v, bool *big) {
    const uint8_t *s = L.s;
    uint64_t p = L.p;
    const bool neg = p < L.n && s[p] == '-';
    if (neg) p++;
    if (p >= L.n) return PJ_REC_SYNTAX;
    uint64_t acc = 0;
    bool over = false;
    const uint64_t lim = neg ? (1ull << 63) : (1ull << 63) - 1;
    if (s[p] == '0') {
        p++;
        if (p < L.n && s[p] >= '0' && s[p] <= '9') return PJ_REC_SYNTAX;
    } else if (s[p] >= '1' && s[p] <= '9') {
        while (p < L.n && s[p] >= '0' && s[p] <= '9') {
            const uint64_t d = s[p] - '0';
            if (acc > (lim - d) / 10) over = true;
            else acc = acc * 10 + d;
            p++;
        }
    } else return PJ_REC_SYNTAX;
    bool real = false;
    if (p < L.n && s[p] == '.') {
        p++;
        real = true;
        if (p >= L.n || s[p] < '0' || s[p] > '9') return PJ_REC_SYNTAX;
        while (p < L.n && s[p] >= '0' && s[p] <= '9') p++;
    }
    if (p < L.n && (s[p] == 'e' || s[p] == 'E')) {
        p++;
        real = true;
        if (p < L.n && (s[p] == '+' || s[p] == '-')) p++;
        if (p >= L.n || s[p] < '0' || s[p] > '9') return PJ_REC_SYNTAX;
        while (p < L.n && s[p] >= '0' && s[p] <= '9') p++;
    }
    L.p = p;
    *kind = real ? T_REAL : T_INT;
    *big = over;
    *v = neg ? (int64_t)(0ull - acc) : (int64_t)acc;
    return PJ_REC_OK;
}

// A literal (null, true, false) or a number.
__device__ __forceinline__ int m_scalar(MLine &L, int *kind, int64_t *v, bool *big) {
    const uint32_t c = m_cur(L);
    if (c == '-' || (c >= '0' && c <= '9')) return m_number(L, kind, v, big);
    uint32_t lit, len;
    if (c == 'n') { lit = 0x6C6C756Eu; len = 4; *kind = T_NULL; }         // "null"
    else if (c == 't') { lit = 0x65757274u; len = 4; *kind = T_TRUE; }    // "true"
    else if (c == 'f') { lit = 0x736C6166u; len = 5; *kind = T_FALSE; }   // "fals" + 'e'
    else return PJ_REC_SYNTAX;
    if (L.p + len > L.n) return PJ_REC_SYNTAX;
    for (uint32_t k = 0; k < 4; k++)
        if (L.s[L.p + k] != ((lit >> (8 * k)) & 0xFF)) return PJ_REC_SYNTAX;
    if (len == 5 && L.s[L.p + 4] != 'e') return PJ_REC_SYNTAX;
    if (L.p + len < L.n && m_ident(L.s[L.p + len])) return PJ_REC_SYNTAX;
    L.p += len;
    return PJ_REC_OK;
}

// A known property holding a value of the wrong JSON type: literals and
// numbers are still tokenised first (a malformed one is a syntax error).
__device__ __forceinline__ int m_type_mismatch(MLine &L) {
    const uint32_t c = m_cur(L);
    if (c == '"' || c == '{' || c == '[') return PJ_REC_TYPE;
    int kind;
    int64_t v;
    bool big;
    const int e = m_scalar(L, &kind, &v, &big);
    return e ? e : PJ_REC_TYPE;
}

// Any value at p, validated and skipped; depth0 containers are open around
// it.  Containers opened here are kept on a bit stack (1 = object).  Out of
// line (unknown properties are rare), with the line passed by value so the
// callers' cursor stays in registers; *p_out receives the position after
// the value.
__device__ __forceinline__ int m_skip_body(MLine &L, int depth0) {
    uint64_t stk[(PJ_MAX_DEPTH + 63) / 64];
    int d = 0;
    int kind, e;
    int64_t v;
    bool big;
    for (;;) {
        // a value at L.p
        const uint32_t c = m_cur(L);
        if (c == '"') {
            MOut o{nullptr};
            if ((e = m_string(L, o))) return e;
        } else if (c == '{' || c == '[') {
            if (depth0 + d + 1 > PJ_MAX_DEPTH) return PJ_REC_DEPTH;
            const bool obj = c == '{';
            const uint64_t bit = 1ull << (d & 63);
            stk[d >> 6] = obj ? (stk[d >> 6] | bit) : (stk[d >> 6] & ~bit);
            d++;
            L.p++;
            m_skip_ws(L);
            const uint32_t close = obj ? '}' : ']';
            if (m_cur(L) == close && !m_end(L)) {
                L.p++;
                d--;
            } else {
                // the first key (objects) or element (arrays)
                if (obj) {
                    m_skip_ws(L);
                    if (m_end(L) || m_cur(L) != '"') return PJ_REC_SYNTAX;
                    MOut o{nullptr};
                    if ((e = m_string(L, o))) return e;
                    m_skip_ws(L);
                    if (m_end(L) || m_cur(L) != ':') return PJ_REC_SYNTAX;
                    L.p++;
                }
                m_skip_ws(L);
                if (m_end(L)) return PJ_REC_SYNTAX;
                continue;
            }
        } else if ((e = m_scalar(L, &kind, &v, &big))) return e;
        // after a value: close containers, or go on to the next member
        for (;;) {
            if (d == 0) return PJ_REC_OK;
            m_skip_ws(L);
            if (m_end(L)) return PJ_REC_SYNTAX;
            const bool obj = (stk[(d - 1) >> 6] >> ((d - 1) & 63)) & 1;
            const uint32_t c2 = m_cur(L);
            if (c2 == (obj ? '}' : ']')) {
                L.p++;
                d--;
                continue;
            }
            if (c2 != ',') return PJ_REC_SYNTAX;
            L.p++;
            if (obj) {
                m_skip_ws(L);
                if (m_end(L) || m_cur(L) != '"') return PJ_REC_SYNTAX;
                MOut o{nullptr};
                if ((e = m_string(L, o))) return e;
                m_skip_ws(L);
                if (m_end(L) || m_cur(L) != ':') return PJ_REC_SYNTAX;
                L.p++;
            }
            m_skip_ws(L);
            if (m_end(L)) return PJ_REC_SYNTAX;
            break;
        }
    }
}

__device__ __noinline__ int m_skip(const uint8_t *s, uint64_t n, uint64_t p, int depth0, uint64_t *p_out) {
    MLine L{s, n, p};
    const int r = m_skip_body(L, depth0);
    *p_out = L.p;
    return r;
}

// ------------------------------------------------------------- schemas
constexpr uint64_t pk8(const char *s, int n, int w) {
    uint64_t r = 0;
    for (int i = 0; i < 8; i++)
        if (w * 8 + i < n) r |= (uint64_t)(uint8_t)s[w * 8 + i] << (8 * i);
    return r;
}
struct MProp {
    uint64_t w0, w1;
    uint32_t len;
    int kind;
};
#define MPROP(name, kind) {pk8(name, sizeof(name) - 1, 0), pk8(name, sizeof(name) - 1, 1), sizeof(name) - 1, kind}

template <int MODEL> struct MSchema;
template <> struct MSchema<PJ_MODEL_ORDER> {
    static constexpr int N = 6;
    static constexpr int kind(int k) {
        return k < 2 ? K_I64 : k == 2 ? K_I32 : k == 3 ? K_STR : k == 4 ? K_ENUM : K_BOOL;
    }
    __device__ static MProp prop(int k) {
        constexpr MProp P[6] = {MPROP("id", K_I64),       MPROP("petId", K_I64),  MPROP("quantity", K_I32),
                                MPROP("shipDate", K_STR), MPROP("status", K_ENUM), MPROP("complete", K_BOOL)};
        return P[k];
    }
};
template <> struct MSchema<PJ_MODEL_USER> {
    static constexpr int N = 8;
    static constexpr int kind(int k) { return k == 0 ? K_I64 : k == 7 ? K_I32 : K_STR; }
    __device__ static MProp prop(int k) {
        constexpr MProp P[8] = {MPROP("id", K_I64),        MPROP("username", K_STR), MPROP("firstName", K_STR),
                                MPROP("lastName", K_STR),  MPROP("email", K_STR),    MPROP("password", K_STR),
                                MPROP("phone", K_STR),     MPROP("userStatus", K_I32)};
        return P[k];
    }
};
// Order.status values (petstore.json:955-963)
__device__ __forceinline__ MProp order_status(int s) {
    constexpr MProp S[3] = {MPROP("placed", 0), MPROP("approved", 0), MPROP("delivered", 0)};
    return S[s];
}
#undef MPROP

template <int MODEL> __device__ __forceinline__ int m_prop_of(const MOut &k) {
    int f = -1;
#pragma unroll
    for (int j = 0; j < MSchema<MODEL>::N; j++) {
        const MProp p = MSchema<MODEL>::prop(j);
        if (k.k == p.len && k.w0 == p.w0 && k.w1 == p.w1) f = j;
    }
    return f;
}

// One record's values as read (the last occurrence of each property).
struct MRec {
    uint32_t present;
    uint32_t sesc;                       // string properties whose value holds an escape
    int64_t v[PJ_MODEL_MAX_PROPS];
    uint64_t spos[PJ_MODEL_MAX_PROPS];   // string properties: the value's opening quote
    uint64_t slen[PJ_MODEL_MAX_PROPS];   // decoded bytes
};

// Property F's value at L.p (every index static, so R stays in registers).
template <int MODEL, int F> __device__ __forceinline__ int m_value(MLine &L, MRec &R) {
    constexpr int KIND = MSchema<MODEL>::kind(F);
    constexpr int f = F;
    const uint32_t c = m_cur(L);
    int kind, e;
    int64_t v = 0;
    bool big = false, pres = false;
    if (KIND == K_I64 || KIND == K_I32) {
        if (c == 'n') {
            if ((e = m_scalar(L, &kind, &v, &big))) return e;
            if (kind != T_NULL) return PJ_REC_TYPE;
            v = 0;
        } else if (c == '-' || (c >= '0' && c <= '9')) {
            if ((e = m_number(L, &kind, &v, &big))) return e;
            if (kind != T_INT || big) return PJ_REC_NUMBER;
            if (KIND == K_I32 && (v < -2147483648ll || v > 2147483647ll)) return PJ_REC_NUMBER;
            pres = true;
        } else return m_type_mismatch(L);
    } else if (KIND == K_STR || KIND == K_ENUM) {
        if (c == '"') {
            const uint64_t q = L.p;
            MOut o{nullptr};
            if ((e = m_string(L, o))) return e;
            pres = true;
            if (KIND == K_STR) {
                R.spos[f] = q;
                R.slen[f] = o.k;
                // escapes shorten the value: its raw bytes then differ from its decoded ones
                if (L.p - q - 2 != o.k) R.sesc |= 1u << f;
                else R.sesc &= ~(1u << f);
            } else {
                int hit = -1;
#pragma unroll
                for (int s = 0; s < 3; s++) {
                    const MProp st = order_status(s);
                    if (o.k == st.len && o.w0 == st.w0 && o.w1 == st.w1) hit = s;
                }
                if (hit < 0) return PJ_REC_BAD_STATUS;
                v = hit;
            }
        } else if (c == 'n') {
            if ((e = m_scalar(L, &kind, &v, &big))) return e;
            if (kind != T_NULL) return PJ_REC_TYPE;
            v = 0;
        } else return m_type_mismatch(L);
        if (!pres) R.slen[f] = 0;
    } else {                                      // K_BOOL
        if (c == '"' || c == '{' || c == '[') return PJ_REC_TYPE;
        if ((e = m_scalar(L, &kind, &v, &big))) return e;
        if (kind == T_INT || kind == T_REAL) return PJ_REC_TYPE;
        pres = kind != T_NULL;
        v = kind == T_TRUE;
    }
    if (pres) R.present |= 1u << f;
    else R.present &= ~(1u << f);
    R.v[f] = v;
    return PJ_REC_OK;
}

// Property f's value, through the m_value instance of each property (so
// every index into R stays static).
template <int MODEL, int F = 0> __device__ __forceinline__ int m_value_of(MLine &L, MRec &R, int f) {
    if constexpr (F >= MSchema<MODEL>::N) return PJ_REC_OK;
    else return f == F ? m_value<MODEL, F>(L, R) : m_value_of<MODEL, F + 1>(L, R, f);
}

// One record [s, s + n): its PJ_REC_* code, and its values in R.
template <int MODEL> __device__ __forceinline__ int m_line(const uint8_t *s, uint64_t n, MRec &R) {
    MLine L{s, n, 0};
    R.present = 0;
    R.sesc = 0;
#pragma unroll
    for (int k = 0; k < PJ_MODEL_MAX_PROPS; k++) {
        R.v[k] = 0;
        R.slen[k] = 0;
        R.spos[k] = 0;
    }
    m_skip_ws(L);
    if (m_end(L)) return PJ_REC_EMPTY;
    if (m_cur(L) != '{') return m_type_mismatch(L);
    L.p++;
    m_skip_ws(L);
    int e;
    if (m_cur(L) == '}' && !m_end(L)) {
        L.p++;
    } else {
        for (;;) {
            m_skip_ws(L);
            if (m_end(L) || m_cur(L) != '"') return PJ_REC_SYNTAX;
            MOut key{nullptr};
            if ((e = m_string(L, key))) return e;
            m_skip_ws(L);
            if (m_end(L) || m_cur(L) != ':') return PJ_REC_SYNTAX;
            L.p++;
            m_skip_ws(L);
            if (m_end(L)) return PJ_REC_SYNTAX;
            const int f = key.k <= 16 ? m_prop_of<MODEL>(key) : -1;
            if (f >= 0) e = m_value_of<MODEL>(L, R, f);
            else {
                uint64_t np;
                e = m_skip(L.s, L.n, L.p, 1, &np);
                L.p = np;
            }
            if (e) return e;
            m_skip_ws(L);
            if (m_end(L)) return PJ_REC_SYNTAX;
            if (m_cur(L) == ',') {
                L.p++;
                continue;
            }
            if (m_cur(L) == '}') {
                L.p++;
                break;
            }
            return PJ_REC_SYNTAX;
        }
    }
    m_skip_ws(L);
    return m_end(L) ? PJ_REC_OK : PJ_REC_SYNTAX;
}

// Fast path: a record whose properties come in schema order (any of them
// absent), with no whitespace, no unknown or repeated key and no error, read
// as straight code: each property's `"key":` compared as a whole and its
// value read by m_value.  Anything else gives M_SLOW, and the record is read
// again by m_line, which decides its values or its first error; so whatever
// this path accepts, m_line reads the same way.
constexpr int M_SLOW = -1;
template <int MODEL, int F> __device__ __forceinline__ bool m_key_is(const MLine &L, uint64_t q) {
    const MProp k = MSchema<MODEL>::prop(F);
    if (q + 3 + k.len > L.n || L.s[q] != '"' || L.s[q + 1 + k.len] != '"' || L.s[q + 2 + k.len] != ':') return false;
    const uint32_t m0 = min(k.len, 8u), m1 = k.len > 8 ? k.len - 8 : 0u;
    const uint64_t x0 = m0 == 8 ? ldu64(L.s + q + 1) : ld_tail(L.s + q + 1, (int)m0);
    const uint64_t x1 = m1 ? ld_tail(L.s + q + 9, (int)m1) : 0ull;
    return x0 == k.w0 && x1 == k.w1;
}
template <int MODEL, int F> __device__ __forceinline__ int m_fast_props(MLine &L, MRec &R, bool first) {
    if constexpr (F >= MSchema<MODEL>::N) return PJ_REC_OK;
    else {
        if (L.p >= L.n) return M_SLOW;
        if (L.s[L.p] == '}') return PJ_REC_OK;                 // the properties after it are absent
        const uint64_t q = first ? L.p : L.p + 1;
        if (!first && L.s[L.p] != ',') return M_SLOW;
        if (!m_key_is<MODEL, F>(L, q)) return m_fast_props<MODEL, F + 1>(L, R, first);   // F is absent
        L.p = q + 3 + MSchema<MODEL>::prop(F).len;
        if (m_value<MODEL, F>(L, R) != PJ_REC_OK) return M_SLOW;
        return m_fast_props<MODEL, F + 1>(L, R, false);
    }
}
template <int MODEL> __device__ __forceinline__ int m_line_fast(const uint8_t *s, uint64_t n, MRec &R) {
    MLine L{s, n, 1};
    R.present = 0;
    R.sesc = 0;
#pragma unroll
    for (int k = 0; k < PJ_MODEL_MAX_PROPS; k++) {
        R.v[k] = 0;
        R.slen[k] = 0;
        R.spos[k] = 0;
    }
    if (n < 2 || s[0] != '{') return M_SLOW;
    if (m_fast_props<MODEL, 0>(L, R, true) != PJ_REC_OK) return M_SLOW;
    return L.p + 1 == n && s[L.p] == '}' ? PJ_REC_OK : M_SLOW;
}

// A block's records, staged: the input bytes [g0, a1) (g0 = the first
// record's start rounded down to 16 bytes, a1 = the last record's end) in
// LDS when they fit the tile, read with 16-byte loads (exact at the input's
// end).  Every record is then read from LDS; a block that does not fit reads
// from global memory.
struct MStage {
    const uint8_t *tile;
    uint64_t g0;
    bool staged;
    __device__ __forceinline__ const uint8_t *at(const ModelDecParams &P, uint64_t a) const {
        return staged ? tile + (a - g0) : P.in + a;
    }
};

template <int BT, int TILE>
__device__ __forceinline__ MStage m_stage(const ModelDecParams &P, uint8_t *tile, uint64_t b) {
    const uint64_t l0 = b * BT, l1 = min(l0 + BT, P.lines);
    const uint64_t a0 = P.line_start[l0], a1 = P.line_start[l1] - 1, g0 = a0 & ~15ull;
    const bool staged = a1 - g0 <= (uint64_t)TILE;
    if (staged) {
        const uint32_t nch = (uint32_t)((a1 - g0 + 15) >> 4);
        for (uint32_t c = threadIdx.x; c < nch; c += BT) {
            const uint64_t g = g0 + 16ull * c;
            uint4 v;
            if (g + 16 <= P.len) v = *reinterpret_cast<const uint4 *>(P.in + g);
            else {
                uint32_t x[4] = {0, 0, 0, 0};
                for (uint32_t j = 0; j < 16 && g + j < P.len; j++) x[j >> 2] |= (uint32_t)P.in[g + j] << (8 * (j & 3));
                v = make_uint4(x[0], x[1], x[2], x[3]);
            }
            reinterpret_cast<uint4 *>(tile)[c] = v;
        }
    }
    __syncthreads();
    return MStage{tile, g0, staged};
}

// The record's counters: [0] valid, [1] invalid, [2 + k] decoded bytes of
// string property k; and whether it is blank.  FAST: through the fast path
// first (the counting kernel; the writer reads records again only without
// the tape, and keeps the smaller code).
template <int MODEL, bool FAST = true>
__device__ __forceinline__ int m_read(const ModelDecParams &P, const MStage &S, uint64_t l, MRec &R,
                                      uint64_t (&cnt)[MD_MAXK]) {
#pragma unroll
    for (int k = 0; k < MD_MAXK; k++) cnt[k] = 0;
    if (l >= P.lines) return -1;
    const uint64_t a = P.line_start[l], e = P.line_start[l + 1] - 1;
    int code = FAST ? m_line_fast<MODEL>(S.at(P, a), e - a, R) : M_SLOW;
    if (code == M_SLOW) code = m_line<MODEL>(S.at(P, a), e - a, R);
    if (code == PJ_REC_OK) {
        cnt[0] = 1;
#pragma unroll
        for (int k = 0; k < MSchema<MODEL>::N; k++)
            if (MSchema<MODEL>::kind(k) == K_STR) cnt[2 + k] = R.slen[k];
    } else cnt[1] = 1;
    return code;
}

// The record tape: word 0 holds the record's code (bits 0-7), its present
// bits (8-15) and bit 16 when the record is 4 GiB or longer (its positions
// do not fit the tape: the writer reads it again); word 1 + k holds property
// k: an integer, enum or boolean value, or for a string its opening quote's
// offset in the record (bits 0-31), its decoded length (32-62) and bit 63
// when it holds an escape.
constexpr uint64_t MT_WIDE = 1ull << 16, MT_ESC = 1ull << 63;
template <int MODEL>
__device__ __forceinline__ void m_tape_put(const ModelDecParams &P, uint64_t l, int code, const MRec &R) {
    const uint64_t L = P.lines;
    const bool wide = P.line_start[l + 1] - 1 - P.line_start[l] >= (1ull << 32);
    P.tape[l] = ((uint64_t)code & 0xFF) | ((uint64_t)(R.present & 0xFF) << 8) | (wide ? MT_WIDE : 0ull);
    if (code != PJ_REC_OK || wide) return;
#pragma unroll
    for (int k = 0; k < MSchema<MODEL>::N; k++)
        P.tape[(1 + k) * L + l] = MSchema<MODEL>::kind(k) == K_STR
                                      ? R.spos[k] | (R.slen[k] << 32) | (((R.sesc >> k) & 1) ? MT_ESC : 0ull)
                                      : (uint64_t)R.v[k];
}

template <int MODEL, int BT, int TILE>
__global__ __launch_bounds__(BT) void k_mdec_count(ModelDecParams P) {
    __shared__ uint64_t sh[BT / 64 + 2];
    __shared__ __attribute__((aligned(16))) uint8_t tile[TILE + 16];
    const uint64_t b = blockIdx.x, l = b * BT + threadIdx.x;
    const MStage S = m_stage<BT, TILE>(P, tile, b);
    MRec R;
    uint64_t cnt[MD_MAXK];
    const int code = m_read<MODEL>(P, S, l, R, cnt);
    if (P.tape && l < P.lines) m_tape_put<MODEL>(P, l, code, R);
#pragma unroll
    for (int k = 0; k < MD_MAXK; k++) {
        uint64_t tot;
        block_excl_scan<BT>(cnt[k], sh, &tot);
        if (threadIdx.x == 0) P.bagg[b * MD_MAXK + k] = tot;
        __syncthreads();
    }
    if (code == PJ_REC_EMPTY) atomicAdd(reinterpret_cast<unsigned long long *>(P.totals + MD_MAXK), 1ull);
}

// The block sums scanned in two levels: k_mdec_scan_chunks scans each chunk
// of MD_CHUNK blocks (one block per thread) into bbase and stores the
// chunk's totals; k_mdec_scan_tops (one workgroup) scans the chunk totals
// into csum and the grand totals.  A block's first offsets are then
// csum[its chunk] + bbase[the block].
constexpr int MD_CHUNK = 1024;

__global__ __launch_bounds__(MD_CHUNK) void k_mdec_scan_chunks(ModelDecParams P) {
    __shared__ uint64_t sh[MD_CHUNK / 64 + 2];
    const uint64_t g = blockIdx.x, b = g * MD_CHUNK + threadIdx.x;
    const bool in = b < P.nblocks;
#pragma unroll
    for (int k = 0; k < MD_MAXK; k++) {
        uint64_t tot;
        const uint64_t pre = block_excl_scan<MD_CHUNK>(in ? P.bagg[b * MD_MAXK + k] : 0ull, sh, &tot);
        if (in) P.bbase[b * MD_MAXK + k] = pre;
        if (threadIdx.x == 0) P.csum[g * MD_MAXK + k] = tot;
        __syncthreads();
    }
}

constexpr int MD_TOPS = 256;   // threads of k_mdec_scan_tops (room in registers for the carries)
__global__ __launch_bounds__(MD_TOPS) void k_mdec_scan_tops(ModelDecParams P) {
    __shared__ uint64_t sh[MD_TOPS / 64 + 2];
    const uint64_t nc = (P.nblocks + MD_CHUNK - 1) / MD_CHUNK;
    uint64_t carry[MD_MAXK];
#pragma unroll
    for (int k = 0; k < MD_MAXK; k++) carry[k] = 0;
    for (uint64_t r = 0; r < nc; r += MD_TOPS) {
        const uint64_t c = r + threadIdx.x;
#pragma unroll
        for (int k = 0; k < MD_MAXK; k++) {
            const uint64_t v = c < nc ? P.csum[c * MD_MAXK + k] : 0;
            uint64_t tot;
            const uint64_t pre = block_excl_scan<MD_TOPS>(v, sh, &tot);
            __syncthreads();
            if (c < nc) P.csum[c * MD_MAXK + k] = carry[k] + pre;
            carry[k] += tot;
        }
    }
    if (threadIdx.x == 0)
        for (int k = 0; k < MD_MAXK; k++) P.totals[k] = carry[k];
}

template <int MODEL, int BT, int TILE>
__global__ __launch_bounds__(BT) void k_mdec_write(ModelDecParams P) {
    __shared__ uint64_t sh[BT / 64 + 2];
    __shared__ __attribute__((aligned(16))) uint8_t tile[TILE + 16];
    const uint64_t b = blockIdx.x, l = b * BT + threadIdx.x;
    const MStage S = m_stage<BT, TILE>(P, tile, b);
    MRec R;
    uint64_t cnt[MD_MAXK], at[MD_MAXK];
    // the counting pass's tape, where it has one: the record's code, values
    // and string positions without reading it again
    const uint64_t w0 = P.tape && l < P.lines ? P.tape[l] : MT_WIDE;
    const bool taped = !(w0 & MT_WIDE);
    int code;
    if (taped) {
        code = (int)(w0 & 0xFF);
        R.present = (uint32_t)(w0 >> 8) & 0xFF;
        R.sesc = 0;
#pragma unroll
        for (int k = 0; k < MD_MAXK; k++) cnt[k] = 0;
        cnt[code == PJ_REC_OK ? 0 : 1] = 1;
#pragma unroll
        for (int k = 0; k < MSchema<MODEL>::N; k++) {
            const uint64_t x = code == PJ_REC_OK ? P.tape[(1 + k) * P.lines + l] : 0;
            R.v[k] = (int64_t)x;
            if (MSchema<MODEL>::kind(k) == K_STR) {
                R.spos[k] = x & 0xFFFFFFFFull;
                R.slen[k] = (x >> 32) & 0x7FFFFFFFull;
                R.sesc |= (x & MT_ESC) ? 1u << k : 0u;
                cnt[2 + k] = R.slen[k];
            }
        }
    } else code = m_read<MODEL, false>(P, S, l, R, cnt);
#pragma unroll
    for (int k = 0; k < MD_MAXK; k++) {
        uint64_t tot;
        at[k] = P.csum[b / MD_CHUNK * MD_MAXK + k] + P.bbase[b * MD_MAXK + k] + block_excl_scan<BT>(cnt[k], sh, &tot);
        __syncthreads();
    }
    if (code < 0) return;
    const pj_model_columns &o = P.o;
    if (code != PJ_REC_OK) {
        if (at[1] < P.err_cap) {
            P.err_line[at[1]] = l;
            P.err_code[at[1]] = (uint8_t)code;
        }
        return;
    }
    const uint64_t row = at[0];
    const bool fits = row < o.cap_n;
    if (fits) o.present[row] = (uint8_t)R.present;
    const uint64_t a = P.line_start[l];
#pragma unroll
    for (int k = 0; k < MSchema<MODEL>::N; k++) {
        const int kind = MSchema<MODEL>::kind(k);
        if (kind == K_STR) {
            const uint64_t s0 = at[2 + k], s1 = s0 + R.slen[k];
            if (fits) static_cast<uint64_t *>(o.col[k])[row + 1] = s1;
            if (R.slen[k] && s1 <= o.cap_bytes[k]) {
                MStore w(o.bytes[k] + s0);
                if (taped && !((R.sesc >> k) & 1)) {
                    // no escape: the raw bytes are the value
                    const uint8_t *src = S.at(P, a + R.spos[k] + 1);
                    const uint64_t n = R.slen[k];
                    uint64_t j = 0;
                    for (; j + 8 <= n; j += 8) w.put8(ldu64(src + j));
                    if (j < n) {
                        const uint64_t x = ld_tail(src + j, (int)(n - j));
                        for (uint64_t q = 0; q < n - j; q++) w.put((uint32_t)(x >> (8 * q)));
                    }
                } else {
                    MLine L{S.at(P, a), P.line_start[l + 1] - 1 - a, R.spos[k]};
                    (void)m_string(L, w);
                }
                w.finish();
            }
        } else if (fits) {
            if (kind == K_I64) static_cast<int64_t *>(o.col[k])[row] = R.v[k];
            else if (kind == K_I32) static_cast<int32_t *>(o.col[k])[row] = (int32_t)R.v[k];
            else static_cast<uint8_t *>(o.col[k])[row] = (uint8_t)R.v[k];
        }
    }
}

}  // namespace
}  // namespace pj

// 128 records per block, staged in a 32 KiB tile (about 250 bytes per
// record fit; longer blocks read global memory)
constexpr int MDEC_BT = 128, MDEC_TILE = 32768;
int pj_decode_model_block() { return MDEC_BT; }

hipError_t pj_launch_decode_model(const ModelDecParams &P, int model, hipStream_t st) {
    const unsigned g = (unsigned)P.nblocks;
    if (!g) return hipSuccess;
    if (model == PJ_MODEL_ORDER)
        hipLaunchKernelGGL((pj::k_mdec_count<PJ_MODEL_ORDER, MDEC_BT, MDEC_TILE>), dim3(g), dim3(MDEC_BT), 0, st, P);
    else
        hipLaunchKernelGGL((pj::k_mdec_count<PJ_MODEL_USER, MDEC_BT, MDEC_TILE>), dim3(g), dim3(MDEC_BT), 0, st, P);
    hipLaunchKernelGGL(pj::k_mdec_scan_chunks, dim3((g + pj::MD_CHUNK - 1) / pj::MD_CHUNK), dim3(pj::MD_CHUNK), 0, st,
                       P);
    hipLaunchKernelGGL(pj::k_mdec_scan_tops, dim3(1), dim3(pj::MD_TOPS), 0, st, P);
    if (model == PJ_MODEL_ORDER)
        hipLaunchKernelGGL((pj::k_mdec_write<PJ_MODEL_ORDER, MDEC_BT, MDEC_TILE>), dim3(g), dim3(MDEC_BT), 0, st, P);
    else
        hipLaunchKernelGGL((pj::k_mdec_write<PJ_MODEL_USER, MDEC_BT, MDEC_TILE>), dim3(g), dim3(MDEC_BT), 0, st, P);
    return hipGetLastError();
}
