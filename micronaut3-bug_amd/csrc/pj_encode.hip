// pj_encode.hip — single-pass columnar Pet -> JSON encoder for gfx950.
//
// A workgroup owns R consecutive records, hence a contiguous range of their
// photoUrls and tags.  Phases (one kernel, one pass over the columns):
//   0. staging: the block's slice of every string column goes into LDS with
//      16-byte loads; record and item column values go into registers;
//   1. units (nested): every record is cut into units in output order --
//      head (separator, id, category, name key), name (+ photoUrls opener),
//      url items, tags opener, tag items, tail -- held by different threads
//      (heads on threads 0..R-1, names on R..2R-1, items after), so one
//      thread no longer writes a whole record and its wave runs one kind;
//   2. lengths: every unit (flat: every record) is measured by its emitting
//      code with a counting sink (digit counts, SWAR escape counts); an LDS
//      scan gives each unit its tile offset; the block aggregate is
//      published for the decoupled look-back right away;
//   3. build the block's output tile in LDS (nested: exact unaligned
//      ds_write_b8..b64, gfx950 runs LDS in unaligned mode; flat: aligned
//      qwords, shared edges merged with an LDS OR);
//   4. resolve the look-back (its latency hidden behind phase 3) and copy the
//      tile to HBM with aligned 16-byte stores, so every cache line leaves
//      the chip whole.
// A block whose tile or item arrays do not fit falls back to writing each
// record straight to global memory from one thread.
//
// Output rules (jackson UTF8JsonGenerator via micronaut-serde, reference
// build.gradle:104) and property order / inclusion (petstore.json:872-922)
// are the ones restated by the CPU checker in oracle/pj_oracle.c.
#include <map>
#include <mutex>
#include <type_traits>

#include "pj_device.h"
#include "pj_kernels.h"

namespace pj {

// ------------------------------------------------------------------ sinks
// Every sink offers put(w, k) (k <= 4 bytes of w), put8(x, k) (k <= 8),
// put_byte, skip(k) and pos().
struct CountSink {
    uint64_t n = 0;
    __device__ __forceinline__ void put(uint32_t, int k) { n += (uint64_t)k; }
    __device__ __forceinline__ void put8(uint64_t, int k) { n += (uint64_t)k; }
    __device__ __forceinline__ void put_byte(uint32_t) { n += 1; }
    __device__ __forceinline__ void skip(uint32_t k) { n += k; }
    __device__ __forceinline__ uint32_t pos() const { return (uint32_t)n; }
};

// Exact unaligned writes into the LDS tile.
struct LdsSinkU {
    uint8_t *t;
    uint32_t o;
    uint32_t e = 0;           // end of this writer's bytes (0: unknown)
    __device__ __forceinline__ void put8(uint64_t x, int k) {
        uint8_t *q = t + o;
        // with 8 bytes of its own ahead, a writer stores all 8: the bytes
        // past k are its own and its next puts write them again
        if (o + 8 <= e) { *reinterpret_cast<uint64_t *>(q) = x; o += (uint32_t)k; return; }
        o += (uint32_t)k;
        if (k & 8) { *reinterpret_cast<uint64_t *>(q) = x; return; }
        if (k & 4) { *reinterpret_cast<uint32_t *>(q) = (uint32_t)x; q += 4; x >>= 32; }
        if (k & 2) { *reinterpret_cast<uint16_t *>(q) = (uint16_t)x; q += 2; x >>= 16; }
        if (k & 1) *q = (uint8_t)x;
    }
    __device__ __forceinline__ void put(uint32_t w, int k) { put8(w, k); }
    __device__ __forceinline__ void put_byte(uint32_t b) { t[o++] = (uint8_t)b; }
    __device__ __forceinline__ void finish() {}
    __device__ __forceinline__ void skip(uint32_t k) { o += k; }
    __device__ __forceinline__ uint32_t pos() const { return o; }
};

// Writes into the LDS tile with aligned 8-byte stores only (unaligned LDS
// accesses stall the LDS pipeline): bytes gather in a register that always
// describes one aligned qword of the tile; a complete qword is stored whole,
// except that a qword the writer shares with the previous or next writer of
// the tile (its first and last) is merged with an LDS OR into a tile that
// was zeroed beforehand, so neighbouring writers need no ordering.  finish()
// after the last byte; skip(k) leaves k bytes to other writers.
struct LdsSinkA {
    uint8_t *t;               // tile base, 8-byte aligned
    uint32_t o;               // next byte offset
    uint64_t acc = 0;         // pending bytes of the qword at o & ~7
    bool head = true;         // the pending qword may hold another writer's bytes
    __device__ __forceinline__ void flush(bool merge) {
        uint64_t *q = reinterpret_cast<uint64_t *>(t + (o & ~7u));
        if (merge) atomicOr(reinterpret_cast<unsigned long long *>(q), (unsigned long long)acc);
        else *q = acc;
    }
    __device__ __forceinline__ void put8(uint64_t x, int k) {   // k (1..8) bytes of x
        if (k < 8) x &= (1ull << (8 * k)) - 1;
        const uint32_t n = o & 7;
        acc |= x << (8 * n);
        if (n + (uint32_t)k >= 8) {
            flush(head && n != 0);
            head = false;
            acc = n ? x >> (8 * (8 - n)) : 0;
        }
        o += (uint32_t)k;
    }
    __device__ __forceinline__ void put(uint32_t w, int k) { put8(w, k); }
    __device__ __forceinline__ void put_byte(uint32_t b) { put8(b & 0xFF, 1); }
    __device__ __forceinline__ void finish() {
        if (o & 7) flush(true);
        acc = 0;
        head = true;
    }
    __device__ __forceinline__ void skip(uint32_t k) {
        finish();
        o += k;
    }
    __device__ __forceinline__ uint32_t pos() const { return o; }
};

template <class S, int N> __device__ __forceinline__ void lit(S &s, const char (&str)[N]) {
    constexpr int L = N - 1;
#pragma unroll
    for (int k = 0; k < L; k += 8) s.put8(pack8(str + k, L - k < 8 ? L - k : 8), L - k < 8 ? L - k : 8);
}

// ----------------------------------------------------------------- numbers
__device__ __forceinline__ int digits32(uint32_t v) {
    return 1 + (v >= 10u) + (v >= 100u) + (v >= 1000u) + (v >= 10000u) + (v >= 100000u) +
           (v >= 1000000u) + (v >= 10000000u) + (v >= 100000000u) + (v >= 1000000000u);
}

// 4 ASCII digits of x (0..9999), most significant in the low byte.
__device__ __forceinline__ uint32_t four_digits(uint32_t x) {
    uint32_t hi = (x * 5243u) >> 19;          // x / 100 for x < 10000
    uint32_t lo = x - hi * 100u;
    uint32_t h1 = (hi * 103u) >> 10, h0 = hi - h1 * 10u;
    uint32_t l1 = (lo * 103u) >> 10, l0 = lo - l1 * 10u;
    return 0x30303030u | h1 | (h0 << 8) | (l1 << 16) | (l0 << 24);
}

__device__ __forceinline__ uint64_t eight_digits(uint32_t x) {  // x < 10^8
    return (uint64_t)four_digits(x / 10000u) | ((uint64_t)four_digits(x % 10000u) << 32);
}

// Long.toString(v)
template <class S> __device__ __forceinline__ void emit_long(S &s, int64_t v) {
    uint64_t u = v < 0 ? 0ull - (uint64_t)v : (uint64_t)v;
    if (v < 0) s.put_byte('-');
    if (u < 100000000ull) {                   // up to 8 digits: 32-bit arithmetic
        uint32_t x = (uint32_t)u;
        int nd = digits32(x);
        s.put8(eight_digits(x) >> (8 * (8 - nd)), nd);
        return;
    }
    uint32_t c2 = (uint32_t)(u % 100000000ull);
    uint64_t q = u / 100000000ull;
    if (q < 100000000ull) {                   // 9..16 digits
        uint32_t x = (uint32_t)q;
        int nd = digits32(x);
        s.put8(eight_digits(x) >> (8 * (8 - nd)), nd);
        s.put8(eight_digits(c2), 8);
        return;
    }
    uint32_t c1 = (uint32_t)(q % 100000000ull), c0 = (uint32_t)(q / 100000000ull);  // c0 <= 922
    int nd = digits32(c0);
    s.put(four_digits(c0) >> (8 * (4 - nd)), nd);
    s.put8(eight_digits(c1), 8);
    s.put8(eight_digits(c2), 8);
}

// |v| as three groups of eight decimal digits, most significant first
// (g0 < 1845), and the leading nonzero group with the digits after it (16,
// 8 or 0).  Same work for every value, so lanes with short and long ids do
// not run separate paths.
struct LongGroups {
    uint32_t g0, g1, g2;
    uint32_t top;      // the leading nonzero group (g2 when all are zero)
    int after;         // digits after it: 16, 8 or 0
};
__device__ __forceinline__ LongGroups long_groups(int64_t v) {
    const uint64_t u = v < 0 ? 0ull - (uint64_t)v : (uint64_t)v;
    const uint64_t q = u / 100000000ull;
    LongGroups r;
    r.g2 = (uint32_t)(u - q * 100000000ull);
    r.g0 = (uint32_t)(q / 100000000ull);
    r.g1 = (uint32_t)(q - (uint64_t)r.g0 * 100000000ull);
    r.top = r.g0 ? r.g0 : r.g1 ? r.g1 : r.g2;
    r.after = r.g0 ? 16 : r.g1 ? 8 : 0;
    return r;
}
// Long.toString(v) into the LDS tile: the leading group's digits, then the
// full groups after it, each piece stored whole (a piece of no bytes stores
// nothing the next piece does not overwrite).
__device__ __forceinline__ void emit_long(LdsSinkU &s, int64_t v) {
    const LongGroups G = long_groups(v);
    s.put8('-', v < 0 ? 1 : 0);
    const int nt = digits32(G.top);
    s.put8(eight_digits(G.top) >> (8 * (8 - nt)), nt);
    s.put8(eight_digits(G.g0 ? G.g1 : G.g2), G.after ? 8 : 0);
    s.put8(eight_digits(G.g2), G.after == 16 ? 8 : 0);
}

// Length only (no digit strings built).
__device__ __forceinline__ void emit_long(CountSink &s, int64_t v) {
    const LongGroups G = long_groups(v);
    s.n += (uint64_t)((v < 0 ? 1 : 0) + G.after + digits32(G.top));
}

// ----------------------------------------------------------------- strings
// Bit 7 of byte k set iff byte k of x needs an output escape (< 0x20, '"'
// or '\\'); exact per byte, unlike special64's "any" test.
__device__ __forceinline__ uint64_t special_mask(uint64_t x) {
    constexpr uint64_t L7 = 0x7F7F7F7F7F7F7F7Full, H = 0x8080808080808080ull;
    const uint64_t lo = x & L7;
    const uint64_t lt20 = ~((lo + 0x6060606060606060ull) | x) & H;                 // < 0x20
    const uint64_t q = (x ^ (0x22 * ONES)) & L7, bsl = (x ^ (0x5C * ONES)) & L7;
    const uint64_t eq = ~(((q + L7) | (x ^ (0x22 * ONES))) & ((bsl + L7) | (x ^ (0x5C * ONES)))) & H;
    return lt20 | eq;
}
// The escape of byte c (which needs one) as up to 6 bytes, formed without
// branches: \" \\ \b \t \n \f \r, else \u00XX (hex digits a-f in the case
// hexa selects).
__device__ __forceinline__ uint64_t esc_seq(uint32_t c, uint32_t hexa, int *len) {
    // '"' and '\\' escape as themselves; the controls 8 9 10 12 13 as b t n f r,
    // read from a packed table (bits 8..13 of 0x3700 mark them short)
    constexpr uint64_t SHORTS = pack8("btn\0fr", 6);
    const bool shrt = c >= 0x20 || ((0x3700u >> (c & 31)) & 1u);
    const uint32_t e = c >= 0x20 ? c : (uint32_t)(SHORTS >> (8 * ((c - 8) & 7))) & 0xFFu;
    const uint32_t lo = c & 15, hc = lo < 10 ? '0' + lo : hexa + lo - 10;
    const uint64_t u6 = pack8("\\u00", 4) | ((uint64_t)('0' + (c >> 4)) << 32) | ((uint64_t)hc << 40);
    *len = shrt ? 2 : 6;
    return shrt ? (uint64_t)('\\' | (e << 8)) : u6;
}
// m (1..8) bytes of x, some of which need escapes: the plain runs between
// them go out whole.
template <class S> __device__ __forceinline__ void esc_bytes(S &s, uint64_t x, int m, uint32_t hexa) {
    uint64_t sp = special_mask(x) & (m >= 8 ? ~0ull : ((1ull << (8 * m)) - 1));
    int done = 0;
    while (sp) {
        const int k = __builtin_ctzll(sp) >> 3;
        sp &= sp - 1;
        if (k > done) s.put8(x >> (8 * done), k - done);
        int len;
        const uint64_t e = esc_seq((uint32_t)(x >> (8 * k)) & 0xFF, hexa, &len);
        s.put8(e, len);
        done = k + 1;
    }
    if (m > done) s.put8(x >> (8 * done), m - done);
}
// Bytes the escapes of the bytes of x selected by keep add to them: one for
// each byte needing an escape, four more for the controls other than
// \b \t \n \f \r (which take six bytes, the rest two).
__device__ __forceinline__ uint32_t esc_extra(uint64_t x, uint64_t keep) {
    constexpr uint64_t L7 = 0x7F7F7F7F7F7F7F7Full, H = 0x8080808080808080ull;
    const uint64_t sp = special_mask(x) & keep & H;
    const uint64_t lo = x & L7;
    const uint64_t lt20 = ~((lo + 0x6060606060606060ull) | x) & H;
    const uint64_t ge8 = (lo + 0x7878787878787878ull) & H, lt14 = ~(lo + 0x7272727272727272ull) & H;
    const uint64_t y = x ^ 0x0B0B0B0B0B0B0B0Bull;
    const uint64_t eq11 = ~(((y & L7) + L7) | y) & H;
    const uint64_t lng = lt20 & ~(ge8 & lt14 & ~eq11) & keep;
    return (uint32_t)(__builtin_popcountll(sp) + 4 * __builtin_popcountll(lng));
}
__device__ __forceinline__ void esc_bytes(CountSink &s, uint64_t x, int m, uint32_t) {
    const uint64_t keep = m >= 8 ? ~0ull : ((1ull << (8 * m)) - 1);
    s.n += (uint64_t)m + esc_extra(x, keep);
}
// The escape bytes of a string in global memory (esc_extra over its bytes).
__device__ __forceinline__ uint64_t str_extra(const uint8_t *p, uint64_t len) {
    uint64_t e = 0, k = 0;
    for (; k + 8 <= len; k += 8) e += esc_extra(ldu64(p + k), ~0ull);
    if (k < len) e += esc_extra(ld_tail(p + k, (int)(len - k)), (1ull << (8 * (len - k))) - 1);
    return e;
}

// The string bytes of a staged slice, read as aligned LDS qwords joined by a
// funnel shift (unaligned LDS reads stall the LDS pipeline).
template <class S>
__device__ __forceinline__ void emit_str_lds(S &s, const PJ_LDS uint8_t *p, uint32_t len, uint32_t hexa) {
    const uint32_t sh = (uint32_t)(uintptr_t)p & 7;
    const PJ_LDS uint64_t *q = (const PJ_LDS uint64_t *)(p - sh);
    uint64_t cur = q[0], nxt = q[1];              // reads run one qword ahead
    uint32_t k = 0, j = 0;
    for (; k + 8 <= len; k += 8, j++) {
        const uint64_t nn = q[j + 2];
        const uint64_t x = sh ? (cur >> (8 * sh)) | (nxt << (64 - 8 * sh)) : cur;
        if (!special64(x)) s.put8(x, 8);
        else esc_bytes(s, x, 8, hexa);
        cur = nxt;
        nxt = nn;
    }
    if (k < len) {
        const int m = (int)(len - k);
        uint64_t x = cur >> (8 * sh);
        if (sh + (uint32_t)m > 8) x |= nxt << (64 - 8 * sh);
        const uint64_t mk = (1ull << (8 * m)) - 1;
        x &= mk;
        if (!special64(x | (0x41 * ONES & ~mk))) s.put8(x, m);
        else esc_bytes(s, x, m, hexa);
    }
}

// Staged bytes that need no escape, read as aligned LDS qwords joined by a
// funnel shift.
template <class S>
__device__ __forceinline__ void emit_plain_lds(S &s, const PJ_LDS uint8_t *p, uint32_t len) {
    const uint32_t sh = (uint32_t)(uintptr_t)p & 7;
    const PJ_LDS uint64_t *q = (const PJ_LDS uint64_t *)(p - sh);
    uint64_t cur = q[0], nxt = q[1];              // reads run one qword ahead
    uint32_t k = 0, j = 0;
    for (; k + 8 <= len; k += 8, j++) {
        const uint64_t nn = q[j + 2];
        s.put8(sh ? (cur >> (8 * sh)) | (nxt << (64 - 8 * sh)) : cur, 8);
        cur = nxt;
        nxt = nn;
    }
    if (k < len) {
        const int m = (int)(len - k);
        uint64_t x = cur >> (8 * sh);
        if (sh + (uint32_t)m > 8) x |= nxt << (64 - 8 * sh);
        s.put8(x, m);
    }
}

// A JSON string (quotes included) from raw UTF-8 bytes: 8 bytes per step
// through the no-escape fast path.  Strings staged in LDS take the aligned
// reads of emit_str_lds; global memory takes unaligned 8-byte loads and, for
// the tail, the aligned reads that never touch another page.
template <class S> __device__ __forceinline__ void emit_str(S &s, const uint8_t *p, uint64_t len, uint32_t hexa) {
    s.put_byte('"');
#if defined(__HIP_DEVICE_COMPILE__)
    if (__builtin_amdgcn_is_shared((const void *)p)) {
        if (len) emit_str_lds(s, (const PJ_LDS uint8_t *)p, (uint32_t)len, hexa);
        s.put_byte('"');
        return;
    }
#endif
    uint64_t k = 0;
    for (; k + 8 <= len; k += 8) {
        uint64_t x = ldu64(p + k);
        if (!special64(x)) s.put8(x, 8);
        else esc_bytes(s, x, 8, hexa);
    }
    if (k < len) {
        int m = (int)(len - k);
        uint64_t x = ld_tail(p + k, m);
        uint64_t mk = (1ull << (8 * m)) - 1;
        if (!special64(x | (0x41 * ONES & ~mk))) s.put8(x, m);
        else esc_bytes(s, x, m, hexa);
    }
    s.put_byte('"');
}

// ------------------------------------------------------------------ record
constexpr uint32_t NO_ITEMS = 0xFFFFFFFFu;  // list not written (null / omitted)

// Where string bytes are read from: the workgroup's LDS copy of its slice of
// each byte column, or the columns in global memory.  Byte a (absolute
// offset) of the name column is at name[a - nb], and so on.
struct ColSrc {
    const uint8_t *name, *cat, *url, *tag;
    uint64_t nb, cb, ub, tb;
    // staged slices only: bit c of plain[c / 64] is set when 16-byte chunk c
    // of the staging buffer (from sbase) holds a byte that needs an escape
    const uint64_t *plain = nullptr;
    const uint8_t *sbase = nullptr;
    // lengths only, bytes not read: every string counts as escape-free (the
    // measuring kernel adds the escapes of all bytes separately)
    bool all_plain = false;
};

// Whether staged bytes [p, p + len) need no escape: every 16-byte chunk they
// touch is clear in the chunk bitmap (a set chunk may belong to a neighbour).
__device__ __forceinline__ bool staged_plain(const ColSrc &X, const uint8_t *p, uint64_t len) {
    if (X.all_plain) return true;
    if (!X.plain || len == 0) return X.plain != nullptr;
    const uint32_t a = (uint32_t)(p - X.sbase), c0 = a >> 4, c1 = (a + (uint32_t)len - 1) >> 4;
    for (uint32_t w = c0 >> 6; w <= (c1 >> 6); w++) {
        uint64_t m = X.plain[w];
        if (w == (c0 >> 6)) m &= ~0ull << (c0 & 63);
        if (w == (c1 >> 6) && (c1 & 63) != 63) m &= (2ull << (c1 & 63)) - 1;
        if (m) return false;
    }
    return true;
}

// A JSON string from a column source.  Measuring a staged string that
// needs no escape takes O(1); writing always goes through emit_str (a
// separate copy path for such strings measured slower there).
template <class S>
__device__ __forceinline__ void emit_strx(S &s, const ColSrc &, const uint8_t *p, uint64_t len, uint32_t hexa) {
    emit_str(s, p, len, hexa);
}
__device__ __forceinline__ void emit_strx(CountSink &s, const ColSrc &X, const uint8_t *p, uint64_t len, uint32_t hexa) {
    if (staged_plain(X, p, len)) s.n += len + 2;
    else emit_str(s, p, len, hexa);
}

// One record's scalar fields, loaded once and kept in registers across the
// measuring and writing passes.
struct RecVals {
    uint32_t fl, cf, st;
    int64_t id, cat_id;
    uint64_t na, nb, ca, cb, u0, u1, t0, t1;
};

template <bool NESTED>
__device__ __forceinline__ RecVals load_rec(const EncParams &P, uint64_t i) {
    const pj_pet_columns &c = P.c;
    RecVals v;
    v.fl = c.flags ? c.flags[i] : (uint32_t)PJ_PET_DEFAULT_FLAGS;
    v.st = c.status ? c.status[i] : (uint32_t)PJ_STATUS_NULL;
    v.id = c.id ? c.id[i] : 0;
    v.na = c.name_off[i];
    v.nb = c.name_off[i + 1];
    v.cf = PJ_SUB_DEFAULT_FLAGS;
    v.cat_id = 0;
    v.ca = v.cb = v.u0 = v.u1 = v.t0 = v.t1 = 0;
    if (NESTED) {
        if (c.cat_id) {
            v.cat_id = c.cat_id[i];
            if (c.cat_flags) v.cf = c.cat_flags[i];
            v.ca = c.cat_name_off[i];
            v.cb = c.cat_name_off[i + 1];
        }
        if (c.photo_off) { v.u0 = c.photo_off[i]; v.u1 = c.photo_off[i + 1]; }
        if (c.tag_off) { v.t0 = c.tag_off[i]; v.t1 = c.tag_off[i + 1]; }
    }
    return v;
}

struct RecItems {             // staged layout of one record's lists
    uint32_t usz, tsz;        // bytes of its url / tag items (from the item scans)
    uint32_t ustart, tstart;  // tile offsets where they start (set by emit_pet)
};

template <class S> __device__ __forceinline__ void key(S &s, bool &first) {
    if (!first) s.put_byte(',');
    first = false;
}

// A Category or Tag object; F0 is the pj_field of its id (its name follows).
template <int F0, class S>
__device__ __forceinline__ void emit_sub(S &s, const EncParams &P, const ColSrc &X, uint32_t fl, int64_t id,
                                         const uint8_t *nm, uint64_t nlen) {
    const uint32_t ii = P.incl[F0], ni = P.incl[F0 + 1];
    bool first = true;
    s.put_byte('{');
    if (fl & PJ_SUB_HAS_ID) { key(s, first); lit(s, "\"id\":"); emit_long(s, id); }
    else if (ii == PJ_INCLUDE_ALWAYS) { key(s, first); lit(s, "\"id\":null"); }
    if (fl & PJ_SUB_HAS_NAME) {
        if (nlen > 0 || ni != PJ_INCLUDE_NON_EMPTY) {
            key(s, first); lit(s, "\"name\":"); emit_strx(s, X, nm, nlen, P.hexa);
        }
    } else if (ni == PJ_INCLUDE_ALWAYS) { key(s, first); lit(s, "\"name\":null"); }
    s.put_byte('}');
}

// One url / tag item's column values, loaded once and kept in registers
// between the measuring and writing passes.
struct UrlItem {
    uint64_t a, b;            // url bytes [a, b)
};
struct TagItem {
    uint64_t a, b;            // name bytes [a, b)
    int64_t id;
    uint32_t tf;
};
__device__ __forceinline__ UrlItem load_url(const EncParams &P, uint64_t u) {
    return UrlItem{P.c.url_off[u], P.c.url_off[u + 1]};
}
__device__ __forceinline__ TagItem load_tag(const EncParams &P, uint64_t g) {
    const pj_pet_columns &c = P.c;
    return TagItem{c.tag_name_off[g], c.tag_name_off[g + 1], c.tag_id[g],
                   c.tag_flags ? (uint32_t)c.tag_flags[g] : (uint32_t)PJ_SUB_DEFAULT_FLAGS};
}

// url item: `"url"` + (',' or ']' after the record's last url)
template <class S>
__device__ __forceinline__ void emit_url_v(S &s, const EncParams &P, const ColSrc &X, const UrlItem &v, bool last) {
    const uint8_t *p = X.url + (v.a - X.ub);
#if defined(__HIP_DEVICE_COMPILE__)
    // urls are seldom escaped and fill whole waves of items: writing a staged
    // escape-free url skips the per-qword escape test
    if (!std::is_same<S, CountSink>::value && staged_plain(X, p, v.b - v.a)) {
        s.put_byte('"');
        if (v.b > v.a) emit_plain_lds(s, (const PJ_LDS uint8_t *)p, (uint32_t)(v.b - v.a));
        s.put_byte('"');
    } else
#endif
        emit_strx(s, X, p, v.b - v.a, P.hexa);
    s.put_byte(last ? ']' : ',');
}
template <class S>
__device__ __forceinline__ void emit_url_item(S &s, const EncParams &P, const ColSrc &X, uint64_t u, bool last) {
    emit_url_v(s, P, X, load_url(P, u), last);
}

// tag item: `{...}` + (',' or ']')
template <class S>
__device__ __forceinline__ void emit_tag_v(S &s, const EncParams &P, const ColSrc &X, const TagItem &v, bool last) {
    emit_sub<PJ_FIELD_TAG_ID>(s, P, X, v.tf, v.id, X.tag + (v.a - X.tb), v.b - v.a);
    s.put_byte(last ? ']' : ',');
}
template <class S>
__device__ __forceinline__ void emit_tag_item(S &s, const EncParams &P, const ColSrc &X, uint64_t g, bool last) {
    emit_tag_v(s, P, X, load_tag(P, g), last);
}

// The pieces of one record, in order: head (separator, '{', id, category,
// the name key), the name string, the photoUrls opener, the url items, the
// tags opener, the tag items, tail (status, '}', terminator).  Which pieces
// are present follows from the flags and the inclusion mode; emit_rec and
// the cooperative path for large records both assemble records from them.
template <bool NESTED, class S>
__device__ __forceinline__ void rec_head(S &s, const EncParams &P, const ColSrc &X, uint64_t i, const RecVals &v) {
    const pj_pet_columns &c = P.c;
    const uint32_t fl = v.fl;
    if (P.format != PJ_FORMAT_NDJSON) s.put_byte(i == P.first ? '[' : ',');
    bool first = true;
    s.put_byte('{');
    if (fl & PJ_PET_HAS_ID) { key(s, first); lit(s, "\"id\":"); emit_long(s, v.id); }
    else if (P.incl[PJ_FIELD_PET_ID] == PJ_INCLUDE_ALWAYS) { key(s, first); lit(s, "\"id\":null"); }
    if (NESTED && (fl & PJ_PET_HAS_CATEGORY) && c.cat_id) {
        key(s, first); lit(s, "\"category\":");
        emit_sub<PJ_FIELD_CATEGORY_ID>(s, P, X, v.cf, v.cat_id, X.cat + (v.ca - X.cb), v.cb - v.ca);
    } else if (P.incl[PJ_FIELD_PET_CATEGORY] == PJ_INCLUDE_ALWAYS) { key(s, first); lit(s, "\"category\":null"); }
    key(s, first);
    if (fl & PJ_PET_HAS_NAME) lit(s, "\"name\":");
    else lit(s, "\"name\":null");
}

template <class S> __device__ __forceinline__ void rec_urls_open(S &s, uint32_t fl, bool empty) {
    if (fl & PJ_PET_HAS_PHOTOURLS) {
        lit(s, ",\"photoUrls\":[");
        if (empty) s.put_byte(']');
    } else lit(s, ",\"photoUrls\":null");
}
template <class S> __device__ __forceinline__ void rec_urls_open(S &s, const RecVals &v) {
    rec_urls_open(s, v.fl, v.u1 == v.u0);
}

// A record with HAS_TAGS and no tag columns (the flat layout, or tag_off
// NULL) has an empty list (t0 == t1 == 0).
template <bool NESTED, class S> __device__ __forceinline__ void rec_tags_open(S &s, const EncParams &P, const RecVals &v) {
    const uint32_t ti = P.incl[PJ_FIELD_PET_TAGS];
    if (v.fl & PJ_PET_HAS_TAGS) {
        if (v.t1 > v.t0 || ti != PJ_INCLUDE_NON_EMPTY) {
            lit(s, ",\"tags\":[");
            if (v.t1 == v.t0) s.put_byte(']');
        }
    } else if (ti == PJ_INCLUDE_ALWAYS) lit(s, ",\"tags\":null");
}

template <class S> __device__ __forceinline__ void rec_tail(S &s, const EncParams &P, uint64_t i, const RecVals &v) {
    const uint32_t st = v.st;
    if (st == 0) lit(s, ",\"status\":\"available\"}");
    else if (st == 1) lit(s, ",\"status\":\"pending\"}");
    else if (st == 2) lit(s, ",\"status\":\"sold\"}");
    else if (P.incl[PJ_FIELD_PET_STATUS] == PJ_INCLUDE_ALWAYS) lit(s, ",\"status\":null}");
    else s.put_byte('}');
    if (P.format == PJ_FORMAT_NDJSON) s.put_byte('\n');
    else if (i == P.last) s.put_byte(']');
}

__device__ __forceinline__ bool rec_has_urls(const RecVals &v) { return (v.fl & PJ_PET_HAS_PHOTOURLS) && v.u1 > v.u0; }
template <bool NESTED> __device__ __forceinline__ bool rec_has_tags(const RecVals &v) {
    return NESTED && (v.fl & PJ_PET_HAS_TAGS) && v.t1 > v.t0;
}

// The name unit of a record: the name string, then the photoUrls opener.
// f: the record's HAS_NAME and HAS_PHOTOURLS bits, 0x80 when it has no urls.
template <class S>
__device__ __forceinline__ void name_unit(S &s, const EncParams &P, const ColSrc &X, const uint8_t *nm, uint32_t nl,
                                          uint32_t f) {
    if (f & PJ_PET_HAS_NAME) emit_strx(s, X, nm, nl, P.hexa);
    rec_urls_open(s, f, (f & 0x80u) != 0);
}

// One record plus its separators: '[' or ',' before (array), '\n' or ']'
// after.  INLINE: lists written here; otherwise their item bytes are
// skipped (written by item threads) and their tile offsets recorded in ri.
template <bool NESTED, bool INLINE, class S>
__device__ __forceinline__ void emit_rec(S &s, const EncParams &P, const ColSrc &X, uint64_t i, const RecVals &v,
                                         RecItems &ri) {
    rec_head<NESTED>(s, P, X, i, v);
    if (v.fl & PJ_PET_HAS_NAME) emit_strx(s, X, X.name + (v.na - X.nb), v.nb - v.na, P.hexa);
    rec_urls_open(s, v);
    if (rec_has_urls(v)) {
        if (INLINE) {
            for (uint64_t u = v.u0; u < v.u1; u++) emit_url_item(s, P, X, u, u + 1 == v.u1);
        } else {
            ri.ustart = s.pos();
            s.skip(ri.usz);
        }
    }
    rec_tags_open<NESTED>(s, P, v);
    if (rec_has_tags<NESTED>(v)) {
        if (INLINE) {
            for (uint64_t g = v.t0; g < v.t1; g++) emit_tag_item(s, P, X, g, g + 1 == v.t1);
        } else {
            ri.tstart = s.pos();
            s.skip(ri.tsz);
        }
    }
    rec_tail(s, P, i, v);
}

// ------------------------------------------------ pretty-printed records
// PJ_FORMAT_PRETTY: the array body as jackson-core's DefaultPrettyPrinter
// lays it out.  Objects indent their entries on new lines, two spaces per
// object level ("\n" + 2*level spaces before each entry, ",\n..." between
// entries, "\n" + 2*(level-1) spaces before '}', "{ }" when empty); arrays
// stay on one line ("[ a, b ]", "[ ]" when empty) and add no level;
// property names are followed by " : ".  The schema fixes every object's
// level: a Pet is at level 1 (the enclosing array adds none), its category
// and its tags at level 2.

// Separator and indentation before an entry of an object at level ind/2.
template <class S> __device__ __forceinline__ void pp_entry(S &s, bool &first, int ind) {
    if (!first) s.put_byte(',');
    first = false;
    s.put_byte('\n');
    s.put8(0x2020202020202020ull, ind);
}
// The closing brace of an object at level ind/2 + 1 (ind: its parent's
// indentation).
template <class S> __device__ __forceinline__ void pp_close(S &s, bool first, int ind) {
    if (first) {
        lit(s, " }");
        return;
    }
    s.put_byte('\n');
    s.put8(0x2020202020202020ull, ind);
    s.put_byte('}');
}

// A Category or Tag object at level 2; F0 is the pj_field of its id.
template <int F0, class S>
__device__ __forceinline__ void pp_sub(S &s, const EncParams &P, uint32_t fl, int64_t id, const uint8_t *nm,
                                       uint64_t nlen) {
    const uint32_t ii = P.incl[F0], ni = P.incl[F0 + 1];
    bool first = true;
    s.put_byte('{');
    if (fl & PJ_SUB_HAS_ID) { pp_entry(s, first, 4); lit(s, "\"id\" : "); emit_long(s, id); }
    else if (ii == PJ_INCLUDE_ALWAYS) { pp_entry(s, first, 4); lit(s, "\"id\" : null"); }
    if (fl & PJ_SUB_HAS_NAME) {
        if (nlen > 0 || ni != PJ_INCLUDE_NON_EMPTY) {
            pp_entry(s, first, 4); lit(s, "\"name\" : "); emit_str(s, nm, nlen, P.hexa);
        }
    } else if (ni == PJ_INCLUDE_ALWAYS) { pp_entry(s, first, 4); lit(s, "\"name\" : null"); }
    pp_close(s, first, 2);
}

// Record i with its array framing: "[ " or ", " before, " ]" after the last.
template <class S> __device__ __forceinline__ void pp_rec(S &s, const EncParams &P, uint64_t i, const RecVals &v) {
    const pj_pet_columns &c = P.c;
    const uint32_t fl = v.fl;
    if (i == P.first) lit(s, "[ ");
    else lit(s, ", ");
    bool first = true;
    s.put_byte('{');
    if (fl & PJ_PET_HAS_ID) { pp_entry(s, first, 2); lit(s, "\"id\" : "); emit_long(s, v.id); }
    else if (P.incl[PJ_FIELD_PET_ID] == PJ_INCLUDE_ALWAYS) { pp_entry(s, first, 2); lit(s, "\"id\" : null"); }
    if ((fl & PJ_PET_HAS_CATEGORY) && c.cat_id) {
        pp_entry(s, first, 2); lit(s, "\"category\" : ");
        pp_sub<PJ_FIELD_CATEGORY_ID>(s, P, v.cf, v.cat_id, c.cat_name_bytes + v.ca, v.cb - v.ca);
    } else if (P.incl[PJ_FIELD_PET_CATEGORY] == PJ_INCLUDE_ALWAYS) {
        pp_entry(s, first, 2); lit(s, "\"category\" : null");
    }
    pp_entry(s, first, 2);
    if (fl & PJ_PET_HAS_NAME) { lit(s, "\"name\" : "); emit_str(s, c.name_bytes + v.na, v.nb - v.na, P.hexa); }
    else lit(s, "\"name\" : null");
    pp_entry(s, first, 2);
    if (fl & PJ_PET_HAS_PHOTOURLS) {
        lit(s, "\"photoUrls\" : [");
        for (uint64_t u = v.u0; u < v.u1; u++) {
            if (u == v.u0) s.put_byte(' ');
            else lit(s, ", ");
            const uint64_t a = c.url_off[u], b = c.url_off[u + 1];
            emit_str(s, c.url_bytes + a, b - a, P.hexa);
        }
        lit(s, " ]");
    } else lit(s, "\"photoUrls\" : null");
    const uint32_t ti = P.incl[PJ_FIELD_PET_TAGS];
    if (fl & PJ_PET_HAS_TAGS) {
        if (v.t1 > v.t0 || ti != PJ_INCLUDE_NON_EMPTY) {
            pp_entry(s, first, 2); lit(s, "\"tags\" : [");
            for (uint64_t g = v.t0; g < v.t1; g++) {
                if (g == v.t0) s.put_byte(' ');
                else lit(s, ", ");
                const TagItem tg = load_tag(P, g);
                pp_sub<PJ_FIELD_TAG_ID>(s, P, tg.tf, tg.id, c.tag_name_bytes + tg.a, tg.b - tg.a);
            }
            lit(s, " ]");
        }
    } else if (ti == PJ_INCLUDE_ALWAYS) { pp_entry(s, first, 2); lit(s, "\"tags\" : null"); }
    const uint32_t st = v.st;
    if (st <= 2) {
        pp_entry(s, first, 2);
        if (st == 0) lit(s, "\"status\" : \"available\"");
        else if (st == 1) lit(s, "\"status\" : \"pending\"");
        else lit(s, "\"status\" : \"sold\"");
    } else if (P.incl[PJ_FIELD_PET_STATUS] == PJ_INCLUDE_ALWAYS) { pp_entry(s, first, 2); lit(s, "\"status\" : null"); }
    pp_close(s, first, 0);
    if (i == P.last) lit(s, " ]");
}

// ---------------------------------------------------- large records, cooperatively
// Exact bytes at any global address: 8-byte stores, exact tail.
struct XSink {
    uint8_t *p;
    uint64_t acc;
    uint32_t nacc;
    __device__ __forceinline__ void put4(uint32_t w, int k) {
        const uint64_t v = (uint64_t)w & ((1ull << (8 * k)) - 1);
        acc |= v << (8 * nacc);
        const uint32_t tot = nacc + (uint32_t)k;
        if (tot >= 8) {
            stu64(p, acc);
            p += 8;
            acc = nacc ? v >> (8 * (8 - nacc)) : 0;
            nacc = tot - 8;
        } else nacc = tot;
    }
    __device__ __forceinline__ void put8(uint64_t x, int k) {
        if (k > 4) { put4((uint32_t)x, 4); put4((uint32_t)(x >> 32), k - 4); }
        else if (k > 0) put4((uint32_t)x, k);
    }
    __device__ __forceinline__ void put(uint32_t w, int k) { put8(w, k); }
    __device__ __forceinline__ void put_byte(uint32_t b) { put4(b & 0xFF, 1); }
    __device__ __forceinline__ void skip(uint32_t) {}
    __device__ __forceinline__ uint32_t pos() const { return 0; }
    __device__ __forceinline__ void finish() { st_tail(p, acc, nacc); }
};

// Escaped bytes of p[0, len) without quotes, 8 bytes per step.
template <class S> __device__ __forceinline__ void esc_run(S &s, const uint8_t *p, uint64_t len, uint32_t hexa) {
    uint64_t k = 0;
    for (; k + 8 <= len; k += 8) {
        const uint64_t x = ldu64(p + k);
        if (!special64(x)) s.put8(x, 8);
        else esc_bytes(s, x, 8, hexa);
    }
    if (k < len) {
        const int m = (int)(len - k);
        const uint64_t x = ld_tail(p + k, m), mk = (1ull << (8 * m)) - 1;
        if (!special64(x | (0x41 * ONES & ~mk))) s.put8(x, m);
        else esc_bytes(s, x, m, hexa);
    }
}

// A JSON string (quotes included) of len bytes, measured (out == nullptr) or
// written at out by the whole workgroup: each thread escapes one slice and a
// block scan places the slices.  Returns its length (every thread).
template <int BT>
__device__ __forceinline__ uint64_t coop_str(const EncParams &P, uint8_t *out, const uint8_t *p, uint64_t len, uint64_t *sh) {
    const uint32_t t = threadIdx.x;
    const uint64_t per = ((len + BT - 1) / BT + 7) & ~7ull;
    const uint64_t a = min((uint64_t)t * per, len), b = min(a + per, len);
    CountSink cs;
    esc_run(cs, p + a, b - a, P.hexa);
    uint64_t tot;
    const uint64_t off = block_excl_scan<BT>(cs.n, sh, &tot);
    if (out) {
        if (t == 0) { out[0] = '"'; out[1 + tot] = '"'; }
        XSink xs{out + 1 + off, 0, 0};
        esc_run(xs, p + a, b - a, P.hexa);
        xs.finish();
    }
    return tot + 2;
}

// The url (URLS) or tag items [g0, g1) of one record, measured or written at
// out by the whole workgroup, BT items per round.  Returns their length.
template <int BT, bool URLS>
__device__ __forceinline__ uint64_t coop_items(const EncParams &P, uint8_t *out, uint64_t g0, uint64_t g1, uint64_t *sh) {
    const ColSrc XG{P.c.name_bytes, P.c.cat_name_bytes, P.c.url_bytes, P.c.tag_name_bytes, 0, 0, 0, 0};
    uint64_t run = 0;
    for (uint64_t r = g0; r < g1; r += BT) {
        const uint64_t g = r + threadIdx.x;
        CountSink cs;
        if (g < g1) {
            if (URLS) emit_url_item(cs, P, XG, g, g + 1 == g1);
            else emit_tag_item(cs, P, XG, g, g + 1 == g1);
        }
        uint64_t tot;
        const uint64_t off = block_excl_scan<BT>(cs.n, sh, &tot);
        if (out && g < g1) {
            XSink xs{out + run + off, 0, 0};
            if (URLS) emit_url_item(xs, P, XG, g, g + 1 == g1);
            else emit_tag_item(xs, P, XG, g, g + 1 == g1);
            xs.finish();
        }
        run += tot;
    }
    return run;
}

// One record measured (out == nullptr) or written at out by the whole
// workgroup: the fixed pieces by thread 0, the name and the lists
// cooperatively.  Every thread passes the same record.  Returns its length.
template <bool NESTED, int BT>
__device__ __forceinline__ uint64_t coop_rec(const EncParams &P, uint8_t *out, uint64_t i, const RecVals &v, uint64_t *sh,
                             uint64_t *sh_len) {
    const ColSrc XG{P.c.name_bytes, P.c.cat_name_bytes, P.c.url_bytes, P.c.tag_name_bytes, 0, 0, 0, 0};
    const uint32_t t = threadIdx.x;
    uint64_t pos = 0;
    // head
    if (t == 0) {
        CountSink cs;
        rec_head<NESTED>(cs, P, XG, i, v);
        *sh_len = cs.n;
        if (out) { XSink xs{out, 0, 0}; rec_head<NESTED>(xs, P, XG, i, v); xs.finish(); }
    }
    __syncthreads();
    pos += *sh_len;
    __syncthreads();
    if (v.fl & PJ_PET_HAS_NAME) pos += coop_str<BT>(P, out ? out + pos : nullptr, P.c.name_bytes + v.na, v.nb - v.na, sh);
    if (t == 0) {
        CountSink cs;
        rec_urls_open(cs, v);
        *sh_len = cs.n;
        if (out) { XSink xs{out + pos, 0, 0}; rec_urls_open(xs, v); xs.finish(); }
    }
    __syncthreads();
    pos += *sh_len;
    __syncthreads();
    if (rec_has_urls(v)) pos += coop_items<BT, true>(P, out ? out + pos : nullptr, v.u0, v.u1, sh);
    if (t == 0) {
        CountSink cs;
        rec_tags_open<NESTED>(cs, P, v);
        *sh_len = cs.n;
        if (out) { XSink xs{out + pos, 0, 0}; rec_tags_open<NESTED>(xs, P, v); xs.finish(); }
    }
    __syncthreads();
    pos += *sh_len;
    __syncthreads();
    if (rec_has_tags<NESTED>(v)) pos += coop_items<BT, false>(P, out ? out + pos : nullptr, v.t0, v.t1, sh);
    if (t == 0) {
        CountSink cs;
        rec_tail(cs, P, i, v);
        *sh_len = cs.n;
        if (out) { XSink xs{out + pos, 0, 0}; rec_tail(xs, P, i, v); xs.finish(); }
    }
    __syncthreads();
    pos += *sh_len;
    __syncthreads();
    return pos;
}

// The length of one large record, by the whole workgroup in one pass (every
// thread gets it): the fixed pieces by thread 0, the name's escapes 16 bytes
// per thread per step (both loads of a step issued before either is used),
// an item per thread per round, and one block sum.  coop_rec's measuring
// mode gives the same length with a scan per piece.
template <bool NESTED, int BT>
__device__ __forceinline__ uint64_t big_len(const EncParams &P, uint64_t i, const RecVals &v, uint64_t *sh) {
    const ColSrc XG{P.c.name_bytes, P.c.cat_name_bytes, P.c.url_bytes, P.c.tag_name_bytes, 0, 0, 0, 0};
    const uint32_t t = threadIdx.x;
    const bool has_name = (v.fl & PJ_PET_HAS_NAME) != 0;
    uint64_t n = 0;
    if (t == 0) {
        CountSink cs;
        rec_head<NESTED>(cs, P, XG, i, v);
        rec_urls_open(cs, v);
        rec_tags_open<NESTED>(cs, P, v);
        rec_tail(cs, P, i, v);
        n = cs.n + (has_name ? 2 : 0);
    }
    const uint64_t nl = has_name ? v.nb - v.na : 0;
    const uint8_t *np = P.c.name_bytes + v.na;
    for (uint64_t k = 16ull * t; k < nl; k += 16ull * BT) {
        const uint32_t m = (uint32_t)min((uint64_t)16, nl - k);
        const uint32_t m0 = min(m, 8u), m1 = m > 8 ? m - 8 : 0u;
        const uint64_t x0 = m0 == 8 ? ldu64(np + k) : ld_tail(np + k, (int)m0);
        const uint64_t x1 = m1 == 8 ? ldu64(np + k + 8) : m1 ? ld_tail(np + k + 8, (int)m1) : 0ull;
        n += m + esc_extra(x0, m0 >= 8 ? ~0ull : ((1ull << (8 * m0)) - 1)) +
             (m1 ? esc_extra(x1, m1 >= 8 ? ~0ull : ((1ull << (8 * m1)) - 1)) : 0u);
    }
    if (rec_has_urls(v))
        for (uint64_t u = v.u0 + t; u < v.u1; u += BT) {
            CountSink cs;
            emit_url_v(cs, P, XG, load_url(P, u), u + 1 == v.u1);
            n += cs.n;
        }
    if (rec_has_tags<NESTED>(v))
        for (uint64_t g = v.t0 + t; g < v.t1; g += BT) {
            CountSink cs;
            emit_tag_v(cs, P, XG, load_tag(P, g), g + 1 == v.t1);
            n += cs.n;
        }
    uint64_t tot;
    block_excl_scan<BT>(n, sh, &tot);
    return tot;
}

// A record handled cooperatively when its workgroup is on the fallback
// path: a long name or a long list.
#ifndef PJ_ENC_BIG_STR
#define PJ_ENC_BIG_STR 512
#endif
constexpr uint64_t BIG_STR = PJ_ENC_BIG_STR, BIG_ITEMS = 16;
template <bool NESTED> __device__ __forceinline__ bool rec_big(const RecVals &v) {
    return v.nb - v.na > BIG_STR || (NESTED && (v.u1 - v.u0 > BIG_ITEMS || v.t1 - v.t0 > BIG_ITEMS));
}

// In-place exclusive scan of n u32 values in LDS (all BT threads call);
// a[n] receives the total.
template <int BT>
__device__ __forceinline__ void lds_excl_scan(uint32_t *a, uint32_t n, uint64_t *sh) {
    const uint32_t t = threadIdx.x;
    const uint32_t per = (n + BT - 1) / BT;
    const uint32_t s0 = min(t * per, n), s1 = min(s0 + per, n);
    uint64_t sum = 0;
    for (uint32_t k = s0; k < s1; k++) sum += a[k];
    uint64_t tot;
    uint64_t run = block_excl_scan<BT>(sum, sh, &tot);
    for (uint32_t k = s0; k < s1; k++) {
        uint32_t v = a[k];
        a[k] = (uint32_t)run;
        run += v;
    }
    if (t == 0) a[n] = (uint32_t)tot;
    __syncthreads();
}

// ------------------------------------------------- large records, deferred
// A nested pass lists each large record it has placed (record, output
// offset) for k_enc_big, while the list has room: thread k takes a slot for
// the block's large record k and marks it BIG_LISTED in big[k] (a record
// index below 2^31 otherwise), so that the pass writes only the ones left
// out.  The records that do not fit the output are not listed.  All
// threads call; big[] is read after the barrier.
constexpr uint32_t BIG_LISTED = 0x80000000u;
__device__ __forceinline__ void defer_big(const EncParams &P, uint32_t *big, const uint32_t *bpre,
                                          const uint32_t *blen, uint32_t nbig, uint64_t r0, uint64_t base) {
    if (!P.big_cap || !nbig) return;               // (uniform)
    const uint32_t t = threadIdx.x;
    if (t < nbig) {
        const uint64_t p = base + bpre[t];
        if (p + blen[t] <= P.cap) {
            const uint64_t k = atomicAdd(P.big_count, 1ull);
            if (k < P.big_cap) {
                P.big_list[2 * k] = r0 + big[t];
                P.big_list[2 * k + 1] = p;
                big[t] |= BIG_LISTED;
            }
        }
    }
    __syncthreads();
}

// One large record written at out by the whole workgroup, each string or
// item loaded once.  The name in rounds of BT x 16 bytes, thread t taking
// bytes 16t .. 16t + 15 of the round: their escaped lengths, one block scan,
// then each byte's escape (1, 2 or 6 bytes) stored at its place in the LDS
// stage, and the round leaves with aligned 16-byte stores (tile_copy_out).
// The url and tag items one per thread per round, measured, scanned and
// written.  The pieces and their order are those of coop_rec.
#ifndef PJ_ENC_BIG_NB
#define PJ_ENC_BIG_NB 16
#endif
constexpr int BIG_NB = PJ_ENC_BIG_NB;
template <int BT> constexpr int big_stage_bytes() { return BT * BIG_NB * 6 + 64; }
template <bool NESTED, int BT>
__device__ __forceinline__ void big_rec(const EncParams &P, uint8_t *out, uint64_t i, const RecVals &v, uint8_t *stage,
                                        uint64_t *sh) {
    const ColSrc XG{P.c.name_bytes, P.c.cat_name_bytes, P.c.url_bytes, P.c.tag_name_bytes, 0, 0, 0, 0};
    const uint32_t t = threadIdx.x;
    const bool has_name = (v.fl & PJ_PET_HAS_NAME) != 0;
    const uint64_t nl = has_name ? v.nb - v.na : 0;
    const uint8_t *np = P.c.name_bytes + v.na;
    uint64_t pos;                                   // (uniform) bytes written before the current piece
    {
        CountSink cs;                               // (the same for every thread)
        rec_head<NESTED>(cs, P, XG, i, v);
        if (has_name) cs.put_byte('"');
        if (t == 0) {
            XSink xs{out, 0, 0};
            rec_head<NESTED>(xs, P, XG, i, v);
            if (has_name) xs.put_byte('"');
            xs.finish();
        }
        pos = cs.n;
    }
    for (uint64_t r0 = 0; r0 < nl; r0 += (uint64_t)BT * BIG_NB) {
        const uint64_t k = r0 + (uint64_t)BIG_NB * t;
        const uint32_t m = k < nl ? (uint32_t)min((uint64_t)BIG_NB, nl - k) : 0u;
        const uint32_t m0 = min(m, 8u), m1 = m > 8 ? m - 8 : 0u;
        uint64_t x0 = 0, x1 = 0;
        if (m0) x0 = m0 == 8 ? ldu64(np + k) : ld_tail(np + k, (int)m0);
        if (m1) x1 = m1 == 8 ? ldu64(np + k + 8) : ld_tail(np + k + 8, (int)m1);
        const uint64_t k0 = m0 >= 8 ? ~0ull : ((1ull << (8 * m0)) - 1), k1 = m1 >= 8 ? ~0ull : ((1ull << (8 * m1)) - 1);
        const uint64_t len = m ? m + esc_extra(x0, k0) + (m1 ? esc_extra(x1, k1) : 0u) : 0u;
        uint64_t tot;
        uint32_t o = (uint32_t)block_excl_scan<BT>(len, sh, &tot);
#pragma unroll
        for (int j = 0; j < BIG_NB; j++) {
            const uint32_t c = (uint32_t)((j < 8 ? x0 : x1) >> (8 * (j & 7))) & 0xFFu;
            const bool on = (uint32_t)j < m;
            const bool esc = c < 0x20u || c == 0x22u || c == 0x5Cu;
            int L = 1;
            const uint64_t e = esc ? esc_seq(c, P.hexa, &L) : (uint64_t)c;
            const uint32_t n = on ? (uint32_t)L : 0u;
            // at most three stores at any byte offset: the byte, the two-byte
            // escape (or "\u" of a six-byte one) and "00XX"
            if (n == 1) stage[o] = (uint8_t)e;
            if (n >= 2) *reinterpret_cast<uint16_t *>(stage + o) = (uint16_t)e;
            if (n == 6) *reinterpret_cast<uint32_t *>(stage + o + 2) = (uint32_t)(e >> 16);
            o += n;
        }
        __syncthreads();
        // (placed from the 16-byte aligned address below out, so that whole
        // chunks leave with aligned stores)
        const uint32_t oa = (uint32_t)((uintptr_t)out & 15);
        tile_copy_out<BT>(stage, out - oa, pos + oa, pos + oa, pos + oa + tot, t);
        __syncthreads();                            // the stage is written again by the next round
        pos += tot;
    }
    // closing quote and photoUrls opener (every thread knows their length)
    {
        CountSink cs;
        if (has_name) cs.put_byte('"');
        rec_urls_open(cs, v);
        if (t == 0) {
            XSink xs{out + pos, 0, 0};
            if (has_name) xs.put_byte('"');
            rec_urls_open(xs, v);
            xs.finish();
        }
        pos += cs.n;
    }
    if (rec_has_urls(v))
        for (uint64_t r = v.u0; r < v.u1; r += BT) {
            const uint64_t u = r + t;
            UrlItem it{0, 0};
            uint64_t len = 0;
            if (u < v.u1) {
                it = load_url(P, u);
                CountSink cs;
                emit_url_v(cs, P, XG, it, u + 1 == v.u1);
                len = cs.n;
            }
            uint64_t tot;
            const uint64_t off = block_excl_scan<BT>(len, sh, &tot);
            if (u < v.u1) {
                XSink xs{out + pos + off, 0, 0};
                emit_url_v(xs, P, XG, it, u + 1 == v.u1);
                xs.finish();
            }
            pos += tot;
        }
    {
        CountSink cs;
        rec_tags_open<NESTED>(cs, P, v);
        if (t == 0) {
            XSink xs{out + pos, 0, 0};
            rec_tags_open<NESTED>(xs, P, v);
            xs.finish();
        }
        pos += cs.n;
    }
    if (rec_has_tags<NESTED>(v))
        for (uint64_t r = v.t0; r < v.t1; r += BT) {
            const uint64_t g = r + t;
            TagItem it{0, 0, 0, 0};
            uint64_t len = 0;
            if (g < v.t1) {
                it = load_tag(P, g);
                CountSink cs;
                emit_tag_v(cs, P, XG, it, g + 1 == v.t1);
                len = cs.n;
            }
            uint64_t tot;
            const uint64_t off = block_excl_scan<BT>(len, sh, &tot);
            if (g < v.t1) {
                XSink xs{out + pos + off, 0, 0};
                emit_tag_v(xs, P, XG, it, g + 1 == v.t1);
                xs.finish();
            }
            pos += tot;
        }
    if (t == 0) {
        XSink xs{out + pos, 0, 0};
        rec_tail(xs, P, i, v);
        xs.finish();
    }
}

// The large records a nested pass listed, one per workgroup at a time, with
// the whole GPU's workgroups on them instead of the pass's persistent ones.
template <bool NESTED, int BT>
__global__ __launch_bounds__(BT) void k_enc_big(EncParams P) {
    __shared__ __attribute__((aligned(16))) uint8_t stage[big_stage_bytes<BT>()];
    __shared__ uint64_t sh_scan[BT / 64];
    const uint64_t cnt = min((uint64_t)*P.big_count, P.big_cap);
    for (uint64_t k = blockIdx.x; k < cnt; k += gridDim.x) {
        const uint64_t i = P.big_list[2 * k], p = P.big_list[2 * k + 1];
        const RecVals v = load_rec<NESTED>(P, i);
        big_rec<NESTED, BT>(P, P.out + p, i, v, stage, sh_scan);
        __syncthreads();                            // sh_scan is reused by the next record
    }
}

// ------------------------------------------------------- record units
// The pieces the tile path cuts a record into (head, name with the
// photoUrls opener, url items, tags opener, tag items, tail), compact or
// PRETTY.  The pretty pieces are pp_rec's layout cut the same way: an item
// is (" " for the first, ", " for the others) + its value (+ " ]" after the
// last); every entry after the first is ",\n" + indentation.
template <int F0, class S>
__device__ __forceinline__ void pp_sub_x(S &s, const EncParams &P, const ColSrc &X, uint32_t fl, int64_t id,
                                         const uint8_t *nm, uint64_t nlen) {
    const uint32_t ii = P.incl[F0], ni = P.incl[F0 + 1];
    bool first = true;
    s.put_byte('{');
    if (fl & PJ_SUB_HAS_ID) { pp_entry(s, first, 4); lit(s, "\"id\" : "); emit_long(s, id); }
    else if (ii == PJ_INCLUDE_ALWAYS) { pp_entry(s, first, 4); lit(s, "\"id\" : null"); }
    if (fl & PJ_SUB_HAS_NAME) {
        if (nlen > 0 || ni != PJ_INCLUDE_NON_EMPTY) {
            pp_entry(s, first, 4); lit(s, "\"name\" : "); emit_strx(s, X, nm, nlen, P.hexa);
        }
    } else if (ni == PJ_INCLUDE_ALWAYS) { pp_entry(s, first, 4); lit(s, "\"name\" : null"); }
    pp_close(s, first, 2);
}
template <bool NESTED, bool PRETTY, class S>
__device__ __forceinline__ void u_head(S &s, const EncParams &P, const ColSrc &X, uint64_t i, const RecVals &v) {
    if constexpr (!PRETTY) rec_head<NESTED>(s, P, X, i, v);
    else {
        const uint32_t fl = v.fl;
        if (i == P.first) lit(s, "[ ");
        else lit(s, ", ");
        bool first = true;
        s.put_byte('{');
        if (fl & PJ_PET_HAS_ID) { pp_entry(s, first, 2); lit(s, "\"id\" : "); emit_long(s, v.id); }
        else if (P.incl[PJ_FIELD_PET_ID] == PJ_INCLUDE_ALWAYS) { pp_entry(s, first, 2); lit(s, "\"id\" : null"); }
        if ((fl & PJ_PET_HAS_CATEGORY) && P.c.cat_id) {
            pp_entry(s, first, 2);
            lit(s, "\"category\" : ");
            pp_sub_x<PJ_FIELD_CATEGORY_ID>(s, P, X, v.cf, v.cat_id, X.cat + (v.ca - X.cb), v.cb - v.ca);
        } else if (P.incl[PJ_FIELD_PET_CATEGORY] == PJ_INCLUDE_ALWAYS) {
            pp_entry(s, first, 2);
            lit(s, "\"category\" : null");
        }
        pp_entry(s, first, 2);
        if (fl & PJ_PET_HAS_NAME) lit(s, "\"name\" : ");
        else lit(s, "\"name\" : null");
    }
}
template <bool PRETTY, class S> __device__ __forceinline__ void u_urls_open(S &s, uint32_t fl, bool empty) {
    if constexpr (!PRETTY) rec_urls_open(s, fl, empty);
    else if (fl & PJ_PET_HAS_PHOTOURLS) {
        lit(s, ",\n  \"photoUrls\" : [");
        if (empty) lit(s, " ]");
    } else lit(s, ",\n  \"photoUrls\" : null");
}
// f: the record's HAS_NAME and HAS_PHOTOURLS bits, 0x80 when it has no urls
template <bool PRETTY, class S>
__device__ __forceinline__ void u_name(S &s, const EncParams &P, const ColSrc &X, const uint8_t *nm, uint32_t nl,
                                       uint32_t f) {
    if (f & PJ_PET_HAS_NAME) emit_strx(s, X, nm, nl, P.hexa);
    u_urls_open<PRETTY>(s, f, (f & 0x80u) != 0);
}
template <bool NESTED, bool PRETTY, class S>
__device__ __forceinline__ void u_tags_open(S &s, const EncParams &P, const RecVals &v) {
    if constexpr (!PRETTY) rec_tags_open<NESTED>(s, P, v);
    else {
        const uint32_t ti = P.incl[PJ_FIELD_PET_TAGS];
        if (v.fl & PJ_PET_HAS_TAGS) {
            if (v.t1 > v.t0 || ti != PJ_INCLUDE_NON_EMPTY) {
                lit(s, ",\n  \"tags\" : [");
                if (v.t1 == v.t0) lit(s, " ]");
            }
        } else if (ti == PJ_INCLUDE_ALWAYS) lit(s, ",\n  \"tags\" : null");
    }
}
template <bool PRETTY, class S>
__device__ __forceinline__ void u_tail(S &s, const EncParams &P, uint64_t i, const RecVals &v) {
    if constexpr (!PRETTY) rec_tail(s, P, i, v);
    else {
        const uint32_t st = v.st;
        if (st == 0) lit(s, ",\n  \"status\" : \"available\"");
        else if (st == 1) lit(s, ",\n  \"status\" : \"pending\"");
        else if (st == 2) lit(s, ",\n  \"status\" : \"sold\"");
        else if (P.incl[PJ_FIELD_PET_STATUS] == PJ_INCLUDE_ALWAYS) lit(s, ",\n  \"status\" : null");
        lit(s, "\n}");
        if (i == P.last) lit(s, " ]");
    }
}
template <bool PRETTY, class S>
__device__ __forceinline__ void u_url(S &s, const EncParams &P, const ColSrc &X, const UrlItem &v, bool first,
                                      bool last) {
    if constexpr (!PRETTY) emit_url_v(s, P, X, v, last);
    else {
        if (first) s.put_byte(' ');
        else lit(s, ", ");
        emit_strx(s, X, X.url + (v.a - X.ub), v.b - v.a, P.hexa);
        if (last) lit(s, " ]");
    }
}
template <bool PRETTY, class S>
__device__ __forceinline__ void u_tag(S &s, const EncParams &P, const ColSrc &X, const TagItem &v, bool first,
                                      bool last) {
    if constexpr (!PRETTY) emit_tag_v(s, P, X, v, last);
    else {
        if (first) s.put_byte(' ');
        else lit(s, ", ");
        pp_sub_x<PJ_FIELD_TAG_ID>(s, P, X, v.tf, v.id, X.tag + (v.a - X.tb), v.b - v.a);
        if (last) lit(s, " ]");
    }
}

// ------------------------------------------------------------------ kernel

// Names longer than LN_MIN bytes in tile-path blocks are counted and written
// by a whole wave, one 8-byte word per lane; the record's own lane writes
// only the quotes and the photoUrls opener around the body.  One long
// escape-heavy name then no longer holds its wave (a lane writing it alone
// takes a loop step per escape).
constexpr uint32_t LN_MIN = 48;

// 8 staged bytes at any byte address: two aligned LDS reads joined
__device__ __forceinline__ uint64_t lds_any8(const PJ_LDS uint8_t *p) {
    const uint32_t sh = (uint32_t)(uintptr_t)p & 7;
    const PJ_LDS uint64_t *q = (const PJ_LDS uint64_t *)(p - sh);
    const uint64_t a = q[0];
    return sh ? (a >> (8 * sh)) | (q[1] << (64 - 8 * sh)) : a;
}
// The bytes the escapes of the len staged bytes at p add (all 64 lanes of
// the wave call, with the same arguments).
__device__ __forceinline__ uint32_t wave_esc_extra(const PJ_LDS uint8_t *p, uint32_t len) {
    uint32_t e = 0;
    for (uint32_t k = 8u * (uint32_t)lane_id(); k < len; k += 512) {
        const uint32_t m = min(8u, len - k);
        e += esc_extra(lds_any8(p + k), m >= 8 ? ~0ull : ((1ull << (8 * m)) - 1));
    }
    return (uint32_t)wave_sum(e);
}
// The escaped bytes of the len staged bytes at p, written to the tile from
// offset dst (all 64 lanes of the wave call, with the same arguments): lane
// l takes word l of each 512-byte step, and a wave scan of the words'
// escaped lengths places them.
__device__ __forceinline__ void wave_str_body(uint8_t *tile, uint32_t dst, const PJ_LDS uint8_t *p, uint32_t len,
                                              uint32_t hexa) {
    for (uint32_t k0 = 0; k0 < len; k0 += 512) {
        const uint32_t k = k0 + 8u * (uint32_t)lane_id();
        uint64_t x = 0;
        uint32_t m = 0, w = 0;
        if (k < len) {
            m = min(8u, len - k);
            const uint64_t keep = m >= 8 ? ~0ull : ((1ull << (8 * m)) - 1);
            x = lds_any8(p + k) & keep;
            w = m + esc_extra(x, keep);
        }
        const uint32_t inc = wave_incl_scan32(w);
        if (m) {
            LdsSinkU s{tile, dst + inc - w, dst + inc};
            if (w == m) s.put8(x, (int)m);
            else esc_bytes(s, x, (int)m, hexa);
        }
        dst += (uint32_t)__builtin_amdgcn_readlane((int)inc, 63);
    }
}

// Where a block's records, items and string bytes lie: fetched for block nb
// by the first wave in two dependent rounds.  Lanes 0-7 load the first
// level (url and tag item ranges, name and category name byte ranges),
// lanes 0-3 then the url and tag name byte ranges those select.  Laid out
// as [0] first url item, [1] end, [2] first tag item, [3] end, then
// (first byte, end) of the name, category name, url and tag name columns;
// [12] the block's output offset when the bounds and offsets are given
// (P.geo).
constexpr int NX = GEO_WORDS;
template <bool NESTED, int R>
__device__ __forceinline__ uint64_t bounds_l1(const EncParams &P, uint64_t nb, uint32_t l) {
    const pj_pet_columns &c = P.c;
    if (l >= 8 || nb >= (P.n + R - 1) / R) return 0;
    const uint64_t r = (l & 1) ? min(nb * R + R, P.n) : nb * R;
    const uint32_t k = l >> 1;
    const uint64_t *o = k == 0   ? (NESTED ? c.photo_off : nullptr)
                        : k == 1 ? (NESTED ? c.tag_off : nullptr)
                        : k == 2 ? c.name_off
                                 : (NESTED && c.cat_id ? c.cat_name_off : nullptr);
    return o ? o[r] : 0;
}
// (A ticket past the last block loads nothing: its first-level words are 0,
// and index 0 of the offset columns need not exist, as with the shifted
// columns of a streamed host encode's segments.)
template <bool NESTED, int R>
__device__ __forceinline__ uint64_t bounds_l2(const EncParams &P, uint64_t nb, uint64_t v1, uint32_t l) {
    if (!NESTED || l >= 4 || nb >= (P.n + R - 1) / R) return 0;
    const uint64_t *o = l < 2 ? (P.c.photo_off ? P.c.url_off : nullptr) : (P.c.tag_off ? P.c.tag_name_off : nullptr);
    return o ? o[v1] : 0;
}
__device__ __forceinline__ void bounds_store(uint64_t *nx, uint64_t v1, uint64_t v2, uint32_t l) {
    if (l < 8) nx[l] = v1;
    if (l < 4) nx[8 + l] = v2;
}
// The first wave claims the next block, by ticket, and stores its number and
// bounds (lane l of the wave).  With the bounds and offsets given (P.geo)
// its GEO_WORDS words are one load away.
template <bool NESTED, int R>
__device__ __forceinline__ void claim_next(const EncParams &P, uint64_t *nx, uint64_t *nb, uint32_t l) {
    if (P.geo) {
        unsigned long long tk0 = 0;
        if (l == 0) tk0 = atomicAdd(P.ticket, 1ull);
        const uint64_t n1 = (uint64_t)__shfl((long long)tk0, 0);
        if (l < (uint32_t)GEO_WORDS && n1 < (P.n + R - 1) / R) nx[l] = P.geo[GEO_WORDS * n1 + l];
        if (l == 0) *nb = n1;
        return;
    }
    unsigned long long tk = 0;
    if (l == 0) tk = atomicAdd(P.ticket, 1ull);
    const uint64_t n1 = (uint64_t)__shfl((long long)tk, 0);
    const uint64_t v1 = bounds_l1<NESTED, R>(P, n1, l);
    bounds_store(nx, v1, bounds_l2<NESTED, R>(P, n1, v1, l), l);
    if (l == 0) *nb = n1;
}

// A block's item ranges and staged slices (16-byte aligned chunk ranges of
// the four string columns, laid end to end in the staging buffer).
struct Geo {
    uint64_t r0, U0, G0, U, G;
    uint64_t lo16[4];
    uint32_t nch[4], off[5];
    bool fast;
};
template <bool NESTED, int R, int INCAP, int UCAP, int GCAP>
__device__ __forceinline__ Geo block_geo(const uint64_t *nx, uint64_t b) {
    Geo g;
    g.r0 = b * R;
    g.U0 = nx[0];
    g.G0 = nx[2];
    g.U = nx[1] - nx[0];
    g.G = nx[3] - nx[2];
    g.off[0] = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const uint64_t lo = nx[4 + 2 * k], hi = nx[5 + 2 * k];
        g.lo16[k] = lo & ~15ull;
        const uint64_t hi16 = (hi + 15) & ~15ull;
        g.nch[k] = hi > lo ? (uint32_t)min((hi16 - g.lo16[k]) >> 4, (uint64_t)INCAP) : 0;
        g.off[k + 1] = g.off[k] + 16 * g.nch[k];
    }
    g.fast = g.off[4] <= INCAP && (!NESTED || (g.U <= UCAP && g.G <= GCAP));
    return g;
}

// Unit layout of a nested fast block over its threads' slots (slot j of
// thread t is list position t + j BT): heads of records 0..R-1 from position
// 0, names from NAME0, url then tag items from ITEM0, each kind starting on
// a wave boundary so that no wave runs two kinds of unit in one slot.
constexpr uint32_t ITEM_ON = 1u << 31, ITEM_LAST = 1u << 30, ITEM_FIRST = 1u << 29;
template <int R> constexpr int name0() { return (R + 63) / 64 * 64; }
template <int R> constexpr int item0() { return (name0<R>() + R + 63) / 64 * 64; }

// Issue the global loads of a block (its record values, the item values of
// a fast block and the 16-byte chunks of its staged slices, SV per thread)
// into registers; they are consumed one phase of the previous block later.
template <bool NESTED, int BT, int R, int NI, int SV>
__device__ __forceinline__ void enc_prefetch(const EncParams &P, const Geo &g, RecVals &rv, TagItem (&iv)[NI],
                                             uint4 (&sv)[SV]) {
    const uint32_t t = threadIdx.x;
    const uint64_t i = g.r0 + t;
    rv = RecVals{};
    if (t < (uint32_t)R && i < P.n) rv = load_rec<NESTED>(P, i);
    if (!g.fast) return;
    if constexpr (NESTED) {
#pragma unroll
        for (int j = 0; j < NI; j++) {
            const uint32_t q = t + (uint32_t)j * BT;
            if (q < (uint32_t)item0<R>()) continue;
            const uint32_t k = q - item0<R>();
            if (k < g.U) {
                const UrlItem u = load_url(P, g.U0 + k);
                iv[j].a = u.a;
                iv[j].b = u.b;
            } else if (k < g.U + g.G) iv[j] = load_tag(P, g.G0 + (k - g.U));
        }
    }
    const pj_pet_columns &c = P.c;
    const uint8_t *srcs[4] = {c.name_bytes, c.cat_name_bytes, c.url_bytes, c.tag_name_bytes};
    const uint32_t tot = g.off[4] >> 4;
#pragma unroll
    for (int u = 0; u < SV; u++) {
        const uint32_t j = t + u * BT;
        sv[u] = make_uint4(0, 0, 0, 0);
        if (j < tot) {
            const uint32_t byte = 16 * j;
            const int k = byte >= g.off[1] ? (byte >= g.off[2] ? (byte >= g.off[3] ? 3 : 2) : 1) : 0;
            const uint8_t *src = (k == 0 ? srcs[0] : k == 1 ? srcs[1] : k == 2 ? srcs[2] : srcs[3]) +
                                 ((k == 0 ? g.lo16[0] : k == 1 ? g.lo16[1] : k == 2 ? g.lo16[2] : g.lo16[3]) +
                                  (byte - (k == 0 ? g.off[0] : k == 1 ? g.off[1] : k == 2 ? g.off[2] : g.off[3])));
            sv[u] = *reinterpret_cast<const uint4 *>(src);
        }
    }
}

// Nested records: persistent workgroups (as many as the device holds), each
// running blocks of R records until none is left.  Once a block's look-back
// is resolved, the first wave claims the next block by ticket (so that
// consecutive tickets start at nearly the same time and a look-back finds
// its predecessors published; every claimed block belongs to a running
// workgroup) and fetches its bounds while the other waves copy the tile
// out; the next block's record, item and staging loads are then in flight
// across the block boundary.  Flat records: one block per workgroup, in
// launch order with a bounded look-back wait (or by ticket when the host
// redoes a launch whose wait ran out).
// Per block: fast blocks stage the string bytes of their records (names,
// category names, urls, tag names: one contiguous slice of each byte
// column) into LDS, measure and build the output tile from there, and copy
// the tile out with aligned 16-byte stores.  Blocks whose slices, lists or
// output do not fit write each record from one thread, reading global
// memory, except records with a long name or a long list, which the whole
// workgroup measures and writes (slices of the string escaped in parallel
// and placed by a block scan, items spread over the threads), so one
// skewed record does not hold its workgroup for long.
template <bool NESTED, int BT, int R, int TILE, int INCAP, int UCAP, int GCAP, int WPE = 1, bool PRETTY = false>
__global__ __launch_bounds__(BT, WPE) void k_encode(EncParams P) {
    static_assert(!PRETTY || NESTED, "pretty output through the tile path: nested layout only");
    constexpr int UA = NESTED ? UCAP : 1, GA = NESTED ? GCAP : 1, RA = NESTED ? R : 1;
    // flat records write the tile with aligned stores only; nested ones,
    // whose many short items mostly land in edge qwords shared with a
    // neighbour, with plain unaligned stores (measured faster there)
    using LdsSink = typename std::conditional<!NESTED, LdsSinkA, LdsSinkU>::type;
    __shared__ __attribute__((aligned(16))) uint8_t tile[TILE];
    __shared__ __attribute__((aligned(16))) uint8_t inb[INCAP];  // staged input slices
    // NESTED fast blocks: every record is cut into units, laid out in output
    // order as head, name, url items, tags opener, tag items, tail; a unit's
    // tile offset is the exclusive scan of the unit lengths (ulen)
    constexpr int NUC = NESTED ? 4 * R + UCAP + GCAP : 1;
    __shared__ uint32_t ulen[NUC + 1];
    __shared__ uint8_t rn_f[RA];                      // per record: flags of its name unit
    // per url / tag item: its unit index (low 16 bits), ITEM_ON when its
    // record writes the list, ITEM_LAST for the record's last item
    __shared__ uint32_t uinfo[UA], ginfo[GA];
    static_assert(NUC < 65536, "unit indices fit 16 bits");
    __shared__ uint64_t sh_scan[BT / 64];
    __shared__ uint64_t splain[(INCAP / 16 + 63) / 64];  // staged 16-byte chunks that hold a byte to escape
    __shared__ uint64_t sh_nx[NX], sh_nb, sh_base, sh_len;
    __shared__ uint32_t sh_nbig;
    // NESTED fast blocks: the records whose name the waves write together
    __shared__ uint8_t sh_ln[RA];
    __shared__ uint32_t sh_nln;
    // hybrid blocks (NESTED): the large records in record order, with their
    // block offsets, lengths and tile offsets; fast blocks keep each record's
    // head unit index, name offset in the staged slice and name length in
    // the first three
    constexpr int RB = NESTED ? R : 1;
    __shared__ uint32_t sh_big[RB], sh_bpre[RB], sh_blen[RB], sh_bspre[RB];
    static_assert(3 * R * 4 <= TILE, "the fallback path keeps its large-record list in the tile");
    // NESTED fast blocks: thread t holds units t + j BT of the list
    // [heads (R) | names (R) | url items (U) | tag items (G)], laid out as
    // name0 / item0 say: the record threads t < R write head, tags opener
    // and tail of record t, threads
    // NAME0..NAME0+R-1 the name and photoUrls opener of record t - NAME0,
    // the rest items
    static_assert(!NESTED || item0<R>() <= BT, "a head and a name unit per record in the first slot");
    // nested workgroups are persistent; flat blocks, with less latency per
    // block to hide, measured faster one per workgroup
    constexpr bool PERSIST = NESTED;
    constexpr int NI = NESTED ? (item0<R>() + UCAP + GCAP + BT - 1) / BT : 1;
    constexpr int SV = (INCAP / 16 + BT - 1) / BT;   // staged chunks per thread
    const uint32_t t = threadIdx.x;
    const pj_pet_columns &c = P.c;
    const uint64_t nblk = (P.n + R - 1) / R;

    // ---- the first block: its number and bounds, then its loads
    if (t < 64) {
        unsigned long long tk = 0;
        const bool by_id = !PERSIST && P.order_by_id;
        if (!by_id && t == 0) tk = atomicAdd(P.ticket, 1ull);
        const uint64_t b0 = by_id ? (uint64_t)blockIdx.x : (uint64_t)__shfl((long long)tk, 0);
        if (P.geo) {
            if (t < (uint32_t)GEO_WORDS && b0 < nblk) sh_nx[t] = P.geo[GEO_WORDS * b0 + t];
        } else {
            const uint64_t v1 = bounds_l1<NESTED, R>(P, b0, t);
            bounds_store(sh_nx, v1, bounds_l2<NESTED, R>(P, b0, v1, t), t);
        }
        if (t == 0) {
            sh_nb = b0;
            sh_nln = 0;
        }
    }
    __syncthreads();
    uint64_t b = sh_nb;
    RecVals rv{};
    TagItem iv[NI];                                 // item column values (a url uses a, b)
    uint4 sv[SV];                                   // staged chunks in flight
    if (b < nblk) enc_prefetch<NESTED, BT, R, NI, SV>(P, block_geo<NESTED, R, INCAP, UCAP, GCAP>(sh_nx, b), rv, iv, sv);

    while (b < nblk) {
#ifdef PJ_ENC_PROF
// profiling builds: 8 wall-clock stamps per block at the end of the output
// buffer (slot 7 by the second wave)
#define EPROF(k) if ((t == 0 || ((k) == 7 && t == 64)) && !P.count_only && P.out) reinterpret_cast<uint64_t *>(P.out + P.cap)[-1 - (int64_t)(b * 8 + (k))] = wall_clock64();
#else
#define EPROF(k)
#endif
        EPROF(0);
        const Geo g = block_geo<NESTED, R, INCAP, UCAP, GCAP>(sh_nx, b);
        const uint64_t gbase = sh_nx[12];               // given offset (P.geo)
        uint64_t nb = 0;
        // the flat tile starts zeroed: writers merge the qwords they share with an OR
        if (!NESTED)
            for (uint32_t k = t; k < (uint32_t)TILE / 16; k += BT) reinterpret_cast<uint4 *>(tile)[k] = make_uint4(0, 0, 0, 0);
        const uint64_t r0 = g.r0;
        const uint64_t U0 = g.U0, G0 = g.G0, U = g.U, G = g.G;
        const uint64_t i = r0 + t;
        const bool live = t < (uint32_t)R && i < P.n;
        const bool fast = g.fast;
        const ColSrc XG{c.name_bytes, c.cat_name_bytes, c.url_bytes, c.tag_name_bytes, 0, 0, 0, 0};
        const ColSrc XL{inb + g.off[0], inb + g.off[1], inb + g.off[2], inb + g.off[3], g.lo16[0], g.lo16[1], g.lo16[2],
                        g.lo16[3], splain, inb};

        RecItems ri{0, 0, NO_ITEMS, NO_ITEMS};
        uint32_t ul0 = 0, ul1 = 0, gl0 = 0, gl1 = 0;
        uint32_t hidx = 0;                              // record thread: unit index of its head
        const uint32_t nrec = (uint32_t)min((uint64_t)R, P.n - r0);
        uint64_t len = 0, pre = 0, agg = 0;
        bool isbig = false;                             // fallback blocks: measured by the whole workgroup
        uint32_t nbig = 0, bidx = 0;
        if (fast) {
            // ---- phase 0: the staged chunks go into LDS, with a bitmap of
            // the chunks that hold a byte to escape
            const uint32_t tot = g.off[4] >> 4;
#pragma unroll
            for (int u = 0; u < SV; u++) {
                const uint32_t j = t + u * BT;
                if (j < tot) reinterpret_cast<uint4 *>(inb)[j] = sv[u];
                // a wave holds 64 consecutive chunks: one ballot per bitmap word
                const bool esc = j < tot && (special64(((uint64_t)sv[u].y << 32) | sv[u].x) |
                                             special64(((uint64_t)sv[u].w << 32) | sv[u].z)) != 0;
                const uint64_t m = __ballot(esc);
                if ((t & 63) == 0 && j < tot) splain[j >> 6] = m;
            }
            if constexpr (NESTED) {
                // record threads: unit indices, item owners, name unit inputs
                // (sh_big / sh_bpre / sh_blen serve only hybrid blocks otherwise)
                if (live) {
                    if (c.photo_off) { ul0 = (uint32_t)(rv.u0 - U0); ul1 = (uint32_t)(rv.u1 - U0); }
                    if (c.tag_off) { gl0 = (uint32_t)(rv.t0 - G0); gl1 = (uint32_t)(rv.t1 - G0); }
                    hidx = 4 * t + ul0 + gl0;
                    sh_big[t] = hidx;
                    sh_bpre[t] = (uint32_t)(rv.na - g.lo16[0]);
                    sh_blen[t] = (uint32_t)(rv.nb - rv.na);
                    rn_f[t] = (uint8_t)((rv.fl & (PJ_PET_HAS_NAME | PJ_PET_HAS_PHOTOURLS)) | (rv.u1 == rv.u0 ? 0x80u : 0u));
                    if ((rv.fl & PJ_PET_HAS_NAME) && rv.nb - rv.na > LN_MIN) sh_ln[atomicAdd(&sh_nln, 1u)] = (uint8_t)t;
                    const uint32_t uf = rec_has_urls(rv) ? ITEM_ON : 0u, gf = rec_has_tags<NESTED>(rv) ? ITEM_ON : 0u;
                    for (uint32_t k = ul0; k < ul1; k++)
                        uinfo[k] = (hidx + 2 + k - ul0) | uf | (k + 1 == ul1 ? ITEM_LAST : 0u) |
                                   ((PRETTY && k == ul0) ? ITEM_FIRST : 0u);
                    for (uint32_t k = gl0; k < gl1; k++)
                        ginfo[k] = (hidx + 3 + (ul1 - ul0) + k - gl0) | gf | (k + 1 == gl1 ? ITEM_LAST : 0u) |
                                   ((PRETTY && k == gl0) ? ITEM_FIRST : 0u);
                }
            }
            __syncthreads();
            EPROF(1);
            if constexpr (NESTED) {
                // ---- phase 1: unit lengths, then their scan
                if (live) {
                    const uint32_t nu = ul1 - ul0, nt = gl1 - gl0;
                    CountSink ch, cm, ct;
                    u_head<NESTED, PRETTY>(ch, P, XL, i, rv);
                    u_tags_open<NESTED, PRETTY>(cm, P, rv);
                    u_tail<PRETTY>(ct, P, i, rv);
                    ulen[hidx] = (uint32_t)ch.n;
                    ulen[hidx + 2 + nu] = (uint32_t)cm.n;
                    ulen[hidx + 3 + nu + nt] = (uint32_t)ct.n;
                }
                if (t >= (uint32_t)name0<R>() && t - name0<R>() < nrec) {
                    const uint32_t r = t - name0<R>(), f = rn_f[r];
                    CountSink cs;
                    if ((f & PJ_PET_HAS_NAME) && sh_blen[r] > LN_MIN) {
                        // the body's escapes are added by the waves below
                        cs.n = sh_blen[r] + 2;
                        u_urls_open<PRETTY>(cs, f, (f & 0x80u) != 0);
                    } else u_name<PRETTY>(cs, P, XL, XL.name + sh_bpre[r], sh_blen[r], f);
                    ulen[sh_big[r] + 1] = (uint32_t)cs.n;
                }
#pragma unroll
                for (int j = 0; j < NI; j++) {
                    const uint32_t q = t + (uint32_t)j * BT;
                    if (q < (uint32_t)item0<R>()) continue;
                    const uint32_t k = q - item0<R>();
                    CountSink cs;
                    if (k < U) {
                        const uint32_t f = uinfo[k];
                        if (f & ITEM_ON)
                            u_url<PRETTY>(cs, P, XL, UrlItem{iv[j].a, iv[j].b}, (f & ITEM_FIRST) != 0, (f & ITEM_LAST) != 0);
                        ulen[f & 0xFFFFu] = (uint32_t)cs.n;
                    } else if (k < U + G) {
                        const uint32_t f = ginfo[k - (uint32_t)U];
                        if (f & ITEM_ON) u_tag<PRETTY>(cs, P, XL, iv[j], (f & ITEM_FIRST) != 0, (f & ITEM_LAST) != 0);
                        ulen[f & 0xFFFFu] = (uint32_t)cs.n;
                    }
                }
                __syncthreads();
                if (sh_nln) {
                    // long names: the escapes of their bodies, one name per wave
                    for (uint32_t k = t >> 6; k < sh_nln; k += BT / 64) {
                        const uint32_t r = sh_ln[k];
                        const uint8_t *p = XL.name + sh_bpre[r];
                        if (staged_plain(XL, p, sh_blen[r])) continue;
                        const uint32_t e = wave_esc_extra((const PJ_LDS uint8_t *)p, sh_blen[r]);
                        if ((t & 63) == 0) ulen[sh_big[r] + 1] += e;
                    }
                    __syncthreads();
                }
                const uint32_t NU = 4 * nrec + (uint32_t)(U + G);
                lds_excl_scan<BT>(ulen, NU, sh_scan);
                agg = ulen[NU];
                if (live) {
                    pre = ulen[hidx];
                    len = ulen[hidx + 4 + (ul1 - ul0) + (gl1 - gl0)] - pre;
                }
                EPROF(2);
            } else {
                // ---- phase 2: record lengths
                if (live) {
                    CountSink cs;
                    emit_rec<NESTED, false>(cs, P, XL, i, rv, ri);
                    len = cs.n;
                }
            }
        } else {
            // fallback block: records measured from global memory, one thread
            // each, except large ones, which the whole workgroup measures
            // the large records in record order (the tile holds the list here
            // for the flat layout, which has no hybrid blocks)
            uint32_t *big = NESTED ? sh_big : reinterpret_cast<uint32_t *>(tile);
            isbig = !PRETTY && live && rec_big<NESTED>(rv);
            if (live && !isbig) {
                CountSink cs;
                if constexpr (PRETTY) pp_rec(cs, P, i, rv);
                else if (NESTED) {
                    // (the url and tag items are measured by a helper thread below)
                    rec_head<NESTED>(cs, P, XG, i, rv);
                    if (rv.fl & PJ_PET_HAS_NAME) emit_strx(cs, XG, XG.name + (rv.na - XG.nb), rv.nb - rv.na, P.hexa);
                    rec_urls_open(cs, rv);
                    rec_tags_open<NESTED>(cs, P, rv);
                    rec_tail(cs, P, i, rv);
                } else emit_rec<NESTED, true>(cs, P, XG, i, rv, ri);
                len = cs.n;
            }
            if constexpr (NESTED && !PRETTY) {
                // The url and tag items of ordinary record r are measured by
                // thread HELP0 + r of the otherwise idle waves, alongside its
                // own thread: each record's chain of global reads is split in
                // two (skewed encode 4.38 -> 3.98 ms).  The helper loads the
                // record's offsets itself; ulen, unused off the tile path,
                // carries the lengths.
                constexpr uint32_t HELP0 = (uint32_t)((R + 63) / 64 * 64);
                static_assert(HELP0 + R <= BT, "a helper thread per record");
                const uint32_t r = t - HELP0;
                if (t >= HELP0 && r < nrec) {
                    const uint64_t ir = r0 + r;
                    const uint32_t fl = c.flags ? c.flags[ir] : (uint32_t)PJ_PET_DEFAULT_FLAGS;
                    const uint64_t u0 = c.photo_off ? c.photo_off[ir] : 0, u1 = c.photo_off ? c.photo_off[ir + 1] : 0;
                    const uint64_t g0 = c.tag_off ? c.tag_off[ir] : 0, g1 = c.tag_off ? c.tag_off[ir + 1] : 0;
                    // (rec_big, from the offsets)
                    const bool big = c.name_off[ir + 1] - c.name_off[ir] > BIG_STR || u1 - u0 > BIG_ITEMS || g1 - g0 > BIG_ITEMS;
                    CountSink cs;
                    if (!big && (fl & PJ_PET_HAS_PHOTOURLS))
                        for (uint64_t u = u0; u < u1; u++) emit_url_item(cs, P, XG, u, u + 1 == u1);
                    if (!big && (fl & PJ_PET_HAS_TAGS))
                        for (uint64_t g = g0; g < g1; g++) emit_tag_item(cs, P, XG, g, g + 1 == g1);
                    ulen[r] = (uint32_t)cs.n;
                }
                __syncthreads();
                if (live && !isbig) len += ulen[t];
            }
            uint64_t nb64;
            bidx = (uint32_t)block_excl_scan<BT>(isbig ? 1ull : 0ull, sh_scan, &nb64);
            nbig = (uint32_t)nb64;
            if (isbig) big[bidx] = t;
            __syncthreads();
            for (uint32_t k = 0; k < nbig; k++) {
                const uint32_t r = big[k];
                const RecVals bv = load_rec<NESTED>(P, r0 + r);
                const uint64_t L = big_len<NESTED, BT>(P, r0 + r, bv, sh_scan);
                if (t == r) len = L;
            }
        }
        // ---- block scan, publish the aggregate
        if (!(NESTED && fast)) pre = block_excl_scan<BT>(len, sh_scan, &agg);
        if (t == 0 && !P.geo) lb_publish(P.state, b, agg);
        // (the copy-out reads up to 32 bytes past the block's bytes)
        const bool fits = fast && agg + 32 <= TILE;
        if (!fits && t == 0 && P.nfall) atomicAdd(P.nfall, 1ull);    // blocks off the tile path
        // Hybrid block (NESTED, fallback measuring): the records other than the
        // large ones still go through the tile, laid end to end (tile offset
        // spre), and leave as the segments between the large records, which the
        // whole workgroup writes straight to global memory.
        bool hyb = false;
        uint64_t spre = 0;
        if (NESTED && !PRETTY && !fast) {
            uint64_t stot;
            spre = block_excl_scan<BT>(isbig ? 0ull : len, sh_scan, &stot);
            hyb = stot + 32 <= TILE;
            if (isbig) {
                sh_bpre[bidx] = (uint32_t)pre;
                sh_blen[bidx] = (uint32_t)len;
                sh_bspre[bidx] = (uint32_t)spre;
            }
        }
        if (hyb && !P.count_only && live && !isbig) {
            LdsSink ls{tile, (uint32_t)spre};
            RecItems r2 = ri;
            emit_rec<NESTED, true>(ls, P, XG, i, rv, r2);
            ls.finish();
        }
        EPROF(3);

        if (fits && !P.count_only) {
            // ---- phase 3: build the tile
            if constexpr (NESTED) {
                if (live) {
                    const uint32_t nu = ul1 - ul0, nt = gl1 - gl0;
                    LdsSink hs{tile, ulen[hidx], ulen[hidx + 1]};
                    u_head<NESTED, PRETTY>(hs, P, XL, i, rv);
                    hs.finish();
                    LdsSink ms{tile, ulen[hidx + 2 + nu], ulen[hidx + 3 + nu]};
                    u_tags_open<NESTED, PRETTY>(ms, P, rv);
                    ms.finish();
                    LdsSink ts{tile, ulen[hidx + 3 + nu + nt], ulen[hidx + 4 + nu + nt]};
                    u_tail<PRETTY>(ts, P, i, rv);
                    ts.finish();
                }
                if (t >= (uint32_t)name0<R>() && t - name0<R>() < nrec) {
                    const uint32_t r = t - name0<R>(), f = rn_f[r];
                    const uint32_t u0 = ulen[sh_big[r] + 1], u1 = ulen[sh_big[r] + 2];
                    LdsSink ns{tile, u0, u1};
                    if ((f & PJ_PET_HAS_NAME) && sh_blen[r] > LN_MIN) {
                        // a long name: its body is left to the waves below
                        CountSink oc;
                        u_urls_open<PRETTY>(oc, f, (f & 0x80u) != 0);
                        ns.put_byte('"');
                        ns.skip(u1 - u0 - 2 - (uint32_t)oc.n);
                        ns.put_byte('"');
                        u_urls_open<PRETTY>(ns, f, (f & 0x80u) != 0);
                    } else u_name<PRETTY>(ns, P, XL, XL.name + sh_bpre[r], sh_blen[r], f);
                    ns.finish();
                }
#pragma unroll
                for (int j = 0; j < NI; j++) {
                    const uint32_t q = t + (uint32_t)j * BT;
                    if (q < (uint32_t)item0<R>()) continue;
                    const uint32_t k = q - item0<R>();
                    if (k < U) {
                        const uint32_t f = uinfo[k], u = f & 0xFFFFu;
                        if (!(f & ITEM_ON)) continue;
                        LdsSink ls{tile, ulen[u], ulen[u + 1]};
                        u_url<PRETTY>(ls, P, XL, UrlItem{iv[j].a, iv[j].b}, (f & ITEM_FIRST) != 0, (f & ITEM_LAST) != 0);
                        ls.finish();
                    } else if (k < U + G) {
                        const uint32_t f = ginfo[k - (uint32_t)U], u = f & 0xFFFFu;
                        if (!(f & ITEM_ON)) continue;
                        LdsSink ls{tile, ulen[u], ulen[u + 1]};
                        u_tag<PRETTY>(ls, P, XL, iv[j], (f & ITEM_FIRST) != 0, (f & ITEM_LAST) != 0);
                        ls.finish();
                    }
                }
                // long names: their bodies, one name per wave (the tile is
                // read only after the look-back's barrier)
                for (uint32_t k = t >> 6; k < sh_nln; k += BT / 64) {
                    const uint32_t r = sh_ln[k];
                    wave_str_body(tile, ulen[sh_big[r] + 1] + 1, (const PJ_LDS uint8_t *)(XL.name + sh_bpre[r]), sh_blen[r],
                                  P.hexa);
                }
            } else if (live) {
                LdsSink ls{tile, (uint32_t)pre};
                RecItems r2 = ri;
                emit_rec<NESTED, false>(ls, P, XL, i, rv, r2);
                ls.finish();
            }
        }
        EPROF(4);
        // ---- phase 4: look-back; then the next block is claimed (now, so
        // that consecutive tickets start at nearly the same time and a
        // look-back finds its predecessors published) and its bounds fetched
        // by the first wave while the others copy the tile out
        if (P.geo) {
            if (t == 0) sh_base = gbase;
        } else if (t < 64) {
            const uint64_t excl = lb_resolve(P.state, b, agg, !PERSIST && P.order_by_id ? P.spin_limit : 0, P.ticket);
            if (t == 0) {
                sh_base = excl;
                if (b == nblk - 1) *P.total = excl + agg;
            }
        }
        __syncthreads();
        EPROF(5);
        if (t == 0) sh_nln = 0;                         // (read for the last time before the barrier above)
        // a block with nothing left to write but its tile claims now; one
        // that still writes records after the look-back (fallback or
        // hybrid), once they are written, so that a claimed block always
        // starts soon after its ticket
        const bool early = fits || P.count_only;
        if (PERSIST && early && t < 64) {
            claim_next<NESTED, R>(P, sh_nx, &sh_nb, t);
            EPROF(6);
        }
        const uint64_t base = sh_base;
        if (P.count_only) {
        } else if (fits) {
            const uint64_t end = min(base + agg, P.cap);
            if (base < end) {
                if (!PERSIST) tile_copy_out<BT>(tile, P.out, base, base, end, t);
                else if (t >= 64) {
                    tile_copy_out<BT - 64>(tile, P.out, base, base, end, t - 64);
                    EPROF(7);
                }
            }
        } else if (hyb) {
            for (uint32_t k = 0; k <= nbig; k++) {
                const uint64_t g_lo = k ? (uint64_t)sh_bpre[k - 1] + sh_blen[k - 1] : 0, g_hi = k < nbig ? sh_bpre[k] : agg;
                const uint64_t t_lo = k ? sh_bspre[k - 1] : 0;
                const uint64_t lo = base + g_lo, hi = min(base + g_hi, P.cap);
                if (lo < hi) tile_copy_out<BT>(tile, P.out, lo - t_lo, lo, hi, t);
            }
            defer_big(P, sh_big, sh_bpre, sh_blen, nbig, r0, base);
            for (uint32_t k = 0; k < nbig; k++) {
                const uint64_t p = base + sh_bpre[k];
                if (p + sh_blen[k] > P.cap || (sh_big[k] & BIG_LISTED)) continue;
                const RecVals bv = load_rec<NESTED>(P, r0 + sh_big[k]);
                coop_rec<NESTED, BT>(P, P.out + p, r0 + sh_big[k], bv, sh_scan, &sh_len);
            }
        } else {
            // fallback: one thread per record writes straight to global memory;
            // large records are written by the whole workgroup
            uint32_t *big = reinterpret_cast<uint32_t *>(tile), *bpre = big + R, *blen = bpre + R;
            if (t == 0) sh_nbig = 0;
            __syncthreads();
            const bool fbig = !PRETTY && live && rec_big<NESTED>(rv);    // (pretty: every record one thread each)
            if (fbig) {
                const uint32_t k = atomicAdd(&sh_nbig, 1u);
                big[k] = t;
                bpre[k] = (uint32_t)pre;
                blen[k] = (uint32_t)len;
            }
            __syncthreads();
            if (live && !fbig && base + pre + len <= P.cap) {
                WriteSink ws;
                ws.init(P.out, base + pre, P.dummy + t);
                if constexpr (PRETTY) pp_rec(ws, P, i, rv);
                else emit_rec<NESTED, true>(ws, P, XG, i, rv, ri);
                ws.finish();
            }
            const uint32_t fnbig = sh_nbig;
            if (NESTED) defer_big(P, big, bpre, blen, fnbig, r0, base);
            for (uint32_t k = 0; k < fnbig; k++) {
                const uint64_t p = base + bpre[k];
                if (p + blen[k] > P.cap || (NESTED && (big[k] & BIG_LISTED))) continue;
                const RecVals bv = load_rec<NESTED>(P, r0 + big[k]);
                coop_rec<NESTED, BT>(P, P.out + p, r0 + big[k], bv, sh_scan, &sh_len);
            }
        }
        if (!PERSIST) break;
        if (!early && t < 64) claim_next<NESTED, R>(P, sh_nx, &sh_nb, t);
        // the next block's loads (record, item and staging values)
        __syncthreads();
        nb = sh_nb;
        if (nb < nblk)
            enc_prefetch<NESTED, BT, R, NI, SV>(P, block_geo<NESTED, R, INCAP, UCAP, GCAP>(sh_nx, nb), rv, iv, sv);
        b = nb;
    }
}

// Nested records, first of two passes: the exact output length of every
// block of R records (the blocks k_encode writes), and every block's bounds
// and output offset (GEO_WORDS words at P.geo[GEO_WORDS * b]); *P.total gets
// the whole length.  k_encode then writes the blocks at those offsets with
// no look-back of its own.  A workgroup measures K consecutive blocks; the
// groups are chained by a decoupled look-back (state[g]), taken by ticket so
// that a look-back only ever waits on running groups.  There is no LDS tile
// and no staging: per record and per item, the fixed bytes and the digit
// counts come from the column values, every string counted as if it needed
// no escape, and one coalesced pass over the 16-byte chunks of the group's
// slices of the four byte columns adds the escapes of all their bytes, each
// byte to its block.  The escapes of bytes that are not written (a null
// name, an omitted category, photoUrls or tags list, a tag name flagged
// absent) are taken back by the thread that owns them.  Every load of the
// first round (records, items, chunks) is issued before any is used.
template <int BT, int R, int K, int UN>
__global__ __launch_bounds__(BT) void k_enc_measure(EncParams P) {
    constexpr int RG = R * K, NW = BT / 64;
    static_assert(RG <= BT, "one record per thread");
    // block boundaries j = 0..K: url item, tag item, then the first byte of
    // the name, category name, url and tag name columns
    __shared__ uint64_t bd[K + 1][6];
    __shared__ uint64_t sh_red[NW][K];
    __shared__ uint64_t sh_g;
    const uint32_t t = threadIdx.x;
    const pj_pet_columns &c = P.c;
    const uint64_t nblk = (P.n + R - 1) / R, ngrp = (nblk + K - 1) / K;
    if (t < 64) {
        unsigned long long tk = 0;
        if (t == 0) tk = atomicAdd(P.ticket, 1ull);
        const uint64_t g = (uint64_t)__shfl((long long)tk, 0);
        // lane l < 4 (K + 1): boundary j = l / 4, offset column l % 4
        const uint32_t j = t >> 2, k = t & 3;
        const uint64_t r = min(g * RG + (uint64_t)j * R, P.n);
        uint64_t v1 = 0;
        if (j <= (uint32_t)K) {
            const uint64_t *o = k == 0 ? c.photo_off : k == 1 ? c.tag_off : k == 2 ? c.name_off
                                                                      : (c.cat_id ? c.cat_name_off : nullptr);
            v1 = o ? o[r] : 0;
            bd[j][k] = v1;
        }
        // then the url and tag name bytes those item boundaries select
        if (j <= (uint32_t)K && k < 2) {
            const uint64_t *o2 = k == 0 ? (c.photo_off ? c.url_off : nullptr) : (c.tag_off ? c.tag_name_off : nullptr);
            bd[j][4 + k] = o2 ? o2[v1] : 0;
        }
        if (t == 0) sh_g = g;
    }
    __syncthreads();
    const uint64_t g = sh_g, r0 = g * RG, i = r0 + t;
    ColSrc XP{c.name_bytes, c.cat_name_bytes, c.url_bytes, c.tag_name_bytes, 0, 0, 0, 0};
    XP.all_plain = true;
    uint64_t acc[K];
#pragma unroll
    for (int j = 0; j < K; j++) acc[j] = 0;
    // the chunks: column k's group slice [bd[0][..], bd[K][..]) from its
    // aligned start, the four slices end to end
    const uint8_t *srcs[4] = {c.name_bytes, c.cat_name_bytes, c.url_bytes, c.tag_name_bytes};
    uint64_t lo16[4], cend[5];
    cend[0] = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const uint64_t lo = bd[0][2 + k], hi = bd[K][2 + k];
        lo16[k] = lo & ~15ull;
        cend[k + 1] = cend[k] + (hi > lo ? (((hi + 15) & ~15ull) - lo16[k]) >> 4 : 0);
    }
    uint4 x[UN];
    auto load_chunks = [&](uint64_t j0) {
#pragma unroll
        for (int u = 0; u < UN; u++) {
            const uint64_t j = j0 + (uint64_t)u * BT;
            x[u] = make_uint4(0, 0, 0, 0);
            if (j < cend[4]) {
                const int k = j >= cend[1] ? (j >= cend[2] ? (j >= cend[3] ? 3 : 2) : 1) : 0;
                x[u] = *reinterpret_cast<const uint4 *>(srcs[k] + lo16[k] + 16 * (j - cend[k]));
            }
        }
    };
    load_chunks(t);
    const uint64_t U0 = bd[0][0], U = bd[K][0] - U0, G0 = bd[0][1], G = bd[K][1] - G0;
    const bool live = t < (uint32_t)RG && i < P.n;
    RecVals v{};
    if (live) v = load_rec<true>(P, i);
    UrlItem u1{};
    TagItem g1{};
    if (t < U) u1 = load_url(P, U0 + t);
    if (t < G) g1 = load_tag(P, G0 + t);
    // the block of item q (of column k: 0 urls, 1 tags)
    auto blk_of = [&](int k, uint64_t q) {
        int j = 0;
#pragma unroll
        for (int m = 1; m < K; m++) j += q >= bd[m][k] ? 1 : 0;
        return j;
    };
    auto add = [&](int j, uint64_t w) {
#pragma unroll
        for (int m = 0; m < K; m++) acc[m] += j == m ? w : 0;
    };
    // records
    if (live) {
        CountSink s;
        rec_head<true>(s, P, XP, i, v);
        name_unit(s, P, XP, nullptr, (uint32_t)(v.nb - v.na),
                  (v.fl & (PJ_PET_HAS_NAME | PJ_PET_HAS_PHOTOURLS)) | (v.u1 == v.u0 ? 0x80u : 0u));
        rec_tags_open<true>(s, P, v);
        rec_tail(s, P, i, v);
        uint64_t n = s.n;
        // bytes in the slices that this record does not write
        if (!(v.fl & PJ_PET_HAS_NAME) && v.nb > v.na) n -= str_extra(c.name_bytes + v.na, v.nb - v.na);
        const bool cat_w = (v.fl & PJ_PET_HAS_CATEGORY) && (v.cf & PJ_SUB_HAS_NAME);
        if (c.cat_id && !cat_w && v.cb > v.ca) n -= str_extra(c.cat_name_bytes + v.ca, v.cb - v.ca);
        if (!(v.fl & PJ_PET_HAS_PHOTOURLS))
            for (uint64_t u = v.u0; u < v.u1; u++) {
                const UrlItem it = load_url(P, u);
                n -= (it.b - it.a) + 3 + str_extra(c.url_bytes + it.a, it.b - it.a);
            }
        if (!(v.fl & PJ_PET_HAS_TAGS))
            for (uint64_t q = v.t0; q < v.t1; q++) {
                const TagItem it = load_tag(P, q);
                CountSink cs;
                emit_tag_v(cs, P, XP, it, false);
                n -= cs.n + ((it.tf & PJ_SUB_HAS_NAME) ? str_extra(c.tag_name_bytes + it.a, it.b - it.a) : 0);
            }
        add((int)(t / R), n);
    }
    // items, counted as written
    auto url_n = [&](const UrlItem &it) { return (it.b - it.a) + 3; };
    auto tag_n = [&](const TagItem &it) {
        CountSink cs;
        emit_tag_v(cs, P, XP, it, false);
        uint64_t n = cs.n;
        if (!(it.tf & PJ_SUB_HAS_NAME) && it.b > it.a) n -= str_extra(c.tag_name_bytes + it.a, it.b - it.a);
        return n;
    };
    if (t < U) add(blk_of(0, U0 + t), url_n(u1));
    for (uint64_t k = t + BT; k < U; k += BT) add(blk_of(0, U0 + k), url_n(load_url(P, U0 + k)));
    if (t < G) add(blk_of(1, G0 + t), tag_n(g1));
    for (uint64_t k = t + BT; k < G; k += BT) add(blk_of(1, G0 + k), tag_n(load_tag(P, G0 + k)));
    // the escapes of every byte of the four slices, each to its block
    for (uint64_t j0 = t;; ) {
#pragma unroll
        for (int u = 0; u < UN; u++) {
            const uint64_t j = j0 + (uint64_t)u * BT;
            if (j >= cend[4]) break;
            const int k = j >= cend[1] ? (j >= cend[2] ? (j >= cend[3] ? 3 : 2) : 1) : 0;
            const uint64_t gb = lo16[k] + 16 * (j - cend[k]);
            const uint64_t lo = ((uint64_t)x[u].y << 32) | x[u].x, hi = ((uint64_t)x[u].w << 32) | x[u].z;
            // the blocks' byte ranges split the chunk; bytes outside the
            // group slice belong to none
#pragma unroll
            for (int m = 0; m < K; m++) {
                const uint64_t bl = bd[m][2 + k], bh = bd[m + 1][2 + k];
                if (bh <= gb || bl >= gb + 16 || bh <= bl) continue;
                const uint32_t a = bl > gb ? (uint32_t)(bl - gb) : 0u, e = bh < gb + 16 ? (uint32_t)(bh - gb) : 16u;
                const uint64_t m0 = (a < 8 ? ~0ull << (8 * a) : 0ull) & (e >= 8 ? ~0ull : (1ull << (8 * e)) - 1);
                const uint64_t m1 = (a <= 8 ? ~0ull : ~0ull << (8 * (a - 8))) &
                                    (e >= 16 ? ~0ull : e <= 8 ? 0ull : (1ull << (8 * (e - 8))) - 1);
                acc[m] += esc_extra(lo, m0) + esc_extra(hi, m1);
            }
        }
        j0 += (uint64_t)UN * BT;
        if (j0 >= cend[4]) break;
        load_chunks(j0);
    }
    // block totals
    const uint32_t w = t >> 6;
#pragma unroll
    for (int m = 0; m < K; m++) {
        const uint64_t s = wave_sum(acc[m]);
        if ((t & 63) == 0) sh_red[w][m] = s;
    }
    __syncthreads();
    if (t < 64) {
        uint64_t blen[K], agg = 0;
#pragma unroll
        for (int m = 0; m < K; m++) {
            blen[m] = 0;
#pragma unroll
            for (int q = 0; q < NW; q++) blen[m] += sh_red[q][m];
            agg += blen[m];
        }
        const uint64_t excl = lookback(P.state, g, agg);
        if (t == 0 && g == ngrp - 1) *P.total = excl + agg;
        // each block's bounds and offset for the writer
        uint64_t base = excl;
#pragma unroll
        for (int m = 0; m < K; m++) {
            const uint64_t b = g * K + m;
            if (b < nblk && t < (uint32_t)GEO_WORDS) {
                const uint32_t f = t < 12 ? (t < 4 ? t >> 1 : 2 + ((t - 4) >> 1)) : 0;
                const uint64_t val = t == 12 ? base : bd[m + (t & 1)][f];
                P.geo[GEO_WORDS * b + t] = val;
            }
            base += blen[m];
        }
    }
}

// One thread per output record, blocks of BT records claimed by ticket:
// pretty-printed output (PRETTY), and the records a selection names
// (P.sel: output record j is column record sel[j]; compact or pretty).  Each
// thread measures its record from global memory, a block scan places the
// records, the look-back gives the block's offset, and each thread writes
// its record with exact stores.  (Staging a block's output in LDS for
// aligned stores measured slower: these blocks rarely fit a tile that
// leaves room for other workgroups.)  Records that would end past the
// capacity are not written; the last block stores the total.
template <int BT, bool PRETTY>
__global__ __launch_bounds__(BT) void k_encode_rows(EncParams P) {
    __shared__ uint64_t sh_scan[BT / 64 + 2];
    __shared__ uint64_t sh_b, sh_base;
    const ColSrc XG{P.c.name_bytes, P.c.cat_name_bytes, P.c.url_bytes, P.c.tag_name_bytes, 0, 0, 0, 0};
    const uint32_t t = threadIdx.x;
    if (t == 0) sh_b = atomicAdd(P.ticket, 1ull);
    __syncthreads();
    const uint64_t b = sh_b, nblk = (P.n + BT - 1) / BT;
    const uint64_t j = b * BT + t;
    const bool live = j < P.n;
    RecVals v{};
    RecItems ri{};
    CountSink cs;
    if (live) {
        v = load_rec<true>(P, P.sel ? P.sel[j] : j);
        if (PRETTY) pp_rec(cs, P, j, v);
        else emit_rec<true, true>(cs, P, XG, j, v, ri);
    }
    uint64_t agg;
    const uint64_t pre = block_excl_scan<BT>(cs.n, sh_scan, &agg);
    if (t < 64) {
        const uint64_t excl = lookback(P.state, b, agg);
        if (t == 0) {
            sh_base = excl;
            if (b == nblk - 1) *P.total = excl + agg;
        }
    }
    __syncthreads();
    if (P.count_only || !live) return;
    const uint64_t at = sh_base + pre;
    if (at + cs.n > P.cap) return;
    SectorSink xs;
    xs.init(P.out + at);
    if (PRETTY) pp_rec(xs, P, j, v);
    else emit_rec<true, true>(xs, P, XG, j, v, ri);
    xs.finish();
}

// The records whose status code is in the mask (bit s: status s, bit 3: no
// status), in input order: R consecutive records per thread, each block's
// selected indices placed by a block scan and the look-back.  The last
// block stores the count.
template <int BT, int R>
__global__ __launch_bounds__(BT) void k_select_status(EncParams P, uint32_t mask, uint64_t *sel) {
    __shared__ uint64_t sh_scan[BT / 64 + 2];
    __shared__ uint64_t sh_b, sh_base;
    const uint32_t t = threadIdx.x;
    if (t == 0) sh_b = atomicAdd(P.ticket, 1ull);
    __syncthreads();
    const uint64_t b = sh_b, n = P.c.n_pets, nblk = (n + (uint64_t)BT * R - 1) / ((uint64_t)BT * R);
    const uint64_t i0 = (b * BT + t) * R;
    uint32_t hits = 0;                              // bit k: record i0 + k is selected
#pragma unroll
    for (int k = 0; k < R; k++) {
        const uint64_t i = i0 + k;
        if (i < n) {
            const uint32_t st = P.c.status ? P.c.status[i] : (uint32_t)PJ_STATUS_NULL;
            hits |= ((mask >> (st <= 2 ? st : 3)) & 1u) << k;
        }
    }
    uint64_t agg;
    const uint64_t pre = block_excl_scan<BT>((uint64_t)__builtin_popcount(hits), sh_scan, &agg);
    if (t < 64) {
        const uint64_t excl = lookback(P.state, b, agg);
        if (t == 0) {
            sh_base = excl;
            if (b == nblk - 1) *P.total = excl + agg;
        }
    }
    __syncthreads();
    uint64_t o = sh_base + pre;
    for (uint32_t m = hits; m; m &= m - 1) sel[o++] = i0 + __builtin_ctz(m);
}

// ------------------------------------------------- Order and User records
// Properties in schema order (reference petstore.json:937-971 Order,
// :824-857 User); a null one is skipped unless ALWAYS, an empty string too
// under NON_EMPTY.  Compact or pretty (the Pet layout rules at level 1).

// The key of a property, with its separator and indentation.
template <int N, class S>
__device__ __forceinline__ void m_key(S &s, bool &first, bool pretty, const char (&name)[N]) {
    if (!first) s.put_byte(',');
    first = false;
    if (pretty) lit(s, "\n  ");
    s.put_byte('"');
    lit(s, name);
    if (pretty) lit(s, "\" : ");
    else lit(s, "\":");
}

// Property k of record i: present (bit k of present) or written as null.
__device__ __forceinline__ bool m_present(const ModelEncParams &P, uint64_t i, int k) {
    return P.c.present ? ((P.c.present[i] >> k) & 1u) != 0 : true;
}

template <int N, class S>
__device__ __forceinline__ void m_null(S &s, const ModelEncParams &P, bool &first, bool pretty, const char (&name)[N]) {
    if (P.incl != PJ_INCLUDE_ALWAYS) return;
    m_key(s, first, pretty, name);
    lit(s, "null");
}

template <int N, class S>
__device__ __forceinline__ void m_i64(S &s, const ModelEncParams &P, uint64_t i, int k, bool &first, bool pretty,
                                      const char (&name)[N]) {
    if (!m_present(P, i, k)) return m_null(s, P, first, pretty, name);
    m_key(s, first, pretty, name);
    emit_long(s, static_cast<const int64_t *>(P.c.col[k])[i]);
}

template <int N, class S>
__device__ __forceinline__ void m_i32(S &s, const ModelEncParams &P, uint64_t i, int k, bool &first, bool pretty,
                                      const char (&name)[N]) {
    if (!m_present(P, i, k)) return m_null(s, P, first, pretty, name);
    m_key(s, first, pretty, name);
    emit_long(s, (int64_t) static_cast<const int32_t *>(P.c.col[k])[i]);
}

template <int N, class S>
__device__ __forceinline__ void m_str(S &s, const ModelEncParams &P, uint64_t i, int k, bool &first, bool pretty,
                                      const char (&name)[N]) {
    if (!m_present(P, i, k)) return m_null(s, P, first, pretty, name);
    const uint64_t *off = static_cast<const uint64_t *>(P.c.col[k]);
    const uint64_t a = off[i], b = off[i + 1];
    if (a == b && P.incl == PJ_INCLUDE_NON_EMPTY) return;
    m_key(s, first, pretty, name);
    emit_str(s, P.c.bytes[k] + a, b - a, P.hexa);
}

template <int N, class S>
__device__ __forceinline__ void m_bool(S &s, const ModelEncParams &P, uint64_t i, int k, bool &first, bool pretty,
                                       const char (&name)[N]) {
    if (!m_present(P, i, k)) return m_null(s, P, first, pretty, name);
    m_key(s, first, pretty, name);
    if (static_cast<const uint8_t *>(P.c.col[k])[i]) lit(s, "true");
    else lit(s, "false");
}

// Order.status: codes past the enum are null.
template <class S>
__device__ __forceinline__ void m_order_status(S &s, const ModelEncParams &P, uint64_t i, bool &first, bool pretty) {
    const uint32_t v = static_cast<const uint8_t *>(P.c.col[4])[i];
    if (!m_present(P, i, 4) || v > 2) return m_null(s, P, first, pretty, "status");
    m_key(s, first, pretty, "status");
    if (v == 0) lit(s, "\"placed\"");
    else if (v == 1) lit(s, "\"approved\"");
    else lit(s, "\"delivered\"");
}

template <int MODEL, class S> __device__ __forceinline__ void m_rec(S &s, const ModelEncParams &P, uint64_t i) {
    const bool pretty = P.format == PJ_FORMAT_PRETTY, array = P.format != PJ_FORMAT_NDJSON;
    if (array) {
        s.put_byte(i == 0 ? '[' : ',');
        if (pretty) s.put_byte(' ');
    }
    bool first = true;
    s.put_byte('{');
    if (MODEL == PJ_MODEL_ORDER) {
        m_i64(s, P, i, 0, first, pretty, "id");
        m_i64(s, P, i, 1, first, pretty, "petId");
        m_i32(s, P, i, 2, first, pretty, "quantity");
        m_str(s, P, i, 3, first, pretty, "shipDate");
        m_order_status(s, P, i, first, pretty);
        m_bool(s, P, i, 5, first, pretty, "complete");
    } else {
        m_i64(s, P, i, 0, first, pretty, "id");
        m_str(s, P, i, 1, first, pretty, "username");
        m_str(s, P, i, 2, first, pretty, "firstName");
        m_str(s, P, i, 3, first, pretty, "lastName");
        m_str(s, P, i, 4, first, pretty, "email");
        m_str(s, P, i, 5, first, pretty, "password");
        m_str(s, P, i, 6, first, pretty, "phone");
        m_i32(s, P, i, 7, first, pretty, "userStatus");
    }
    if (pretty) {
        if (first) s.put_byte(' ');
        else s.put_byte('\n');
    }
    s.put_byte('}');
    if (!array) s.put_byte('\n');
    else if (i == P.n - 1) {
        if (pretty) s.put_byte(' ');
        s.put_byte(']');
    }
}

// One thread per record in blocks of BT claimed by ticket: measure, block
// scan, look-back, then each thread writes its record with exact stores.
template <int MODEL, int BT>
__global__ __launch_bounds__(BT) void k_encode_model(ModelEncParams P) {
    __shared__ uint64_t sh_scan[BT / 64 + 2];
    __shared__ uint64_t sh_b, sh_base;
    const uint32_t t = threadIdx.x;
    if (t == 0) sh_b = atomicAdd(P.ticket, 1ull);
    __syncthreads();
    const uint64_t b = sh_b, nblk = (P.n + BT - 1) / BT;
    const uint64_t i = b * BT + t;
    const bool live = i < P.n;
    CountSink cs;
    if (live) m_rec<MODEL>(cs, P, i);
    uint64_t agg;
    const uint64_t pre = block_excl_scan<BT>(cs.n, sh_scan, &agg);
    if (t < 64) {
        const uint64_t excl = lookback(P.state, b, agg);
        if (t == 0) {
            sh_base = excl;
            if (b == nblk - 1) *P.total = excl + agg;
        }
    }
    __syncthreads();
    if (P.count_only || !live) return;
    const uint64_t at = sh_base + pre;
    if (at + cs.n > P.cap) return;
    SectorSink xs;
    xs.init(P.out + at);
    m_rec<MODEL>(xs, P, i);
    xs.finish();
}

__global__ void k_add_u64(uint64_t *p, uint64_t n, uint64_t v) {
    uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] += v;
}

__global__ void k_fill_u64(uint64_t *p, uint64_t n, uint64_t v) {
    uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

__global__ void k_put_bytes(uint8_t *out, uint32_t w, int k) {
    if (threadIdx.x < (unsigned)k) out[threadIdx.x] = (uint8_t)(w >> (8 * threadIdx.x));
}

}  // namespace pj

// ------------------------------------------------------------- launchers
hipError_t pj_launch_add_u64(uint64_t *p, uint64_t n, uint64_t v, hipStream_t st) {
    if (n == 0 || v == 0) return hipSuccess;
    uint64_t g = (n + 255) / 256;
    hipLaunchKernelGGL(pj::k_add_u64, dim3((unsigned)g), dim3(256), 0, st, p, n, v);
    return hipGetLastError();
}

hipError_t pj_launch_fill_u64(uint64_t *p, uint64_t n, uint64_t v, hipStream_t st) {
    if (n == 0) return hipSuccess;
    uint64_t g = (n + 255) / 256;
    hipLaunchKernelGGL(pj::k_fill_u64, dim3((unsigned)g), dim3(256), 0, st, p, n, v);
    return hipGetLastError();
}

#ifndef PJ_ENC_NEST_R
#define PJ_ENC_NEST_R 96
#endif
#ifndef PJ_ENC_NEST_BT
#define PJ_ENC_NEST_BT 256
#endif
#ifndef PJ_ENC_NEST_TILE
#define PJ_ENC_NEST_TILE (30 * 1024 + 256)
#endif
#ifndef PJ_ENC_NEST_IN
#define PJ_ENC_NEST_IN (14 * 1024)
#endif
#ifndef PJ_ENC_NEST_UCAP
#define PJ_ENC_NEST_UCAP 320
#endif
#ifndef PJ_ENC_NEST_GCAP
#define PJ_ENC_NEST_GCAP 256
#endif
#ifndef PJ_ENC_NEST_WPE
#define PJ_ENC_NEST_WPE 3
#endif
// Workgroup shapes: threads, records, LDS tile bytes, item capacities.
// The nested shape must stay at or below about 53.7 KB of LDS per
// workgroup (measured: 53,696 bytes still gives three workgroups per CU,
// 53,808 gives two, which cost 45%).
// Flat blocks of 256 records in two shapes: compact (tile 96 B and staged
// names 24 B per record, 30.6 KB of LDS, five waves per SIMD) for records up
// to about 90 bytes, wide (112 B / 32 B, four waves per SIMD) once the
// compact tile has sent more than 1 block in 64 to the fallback path.
constexpr int ENC_FLAT_BT = 256, ENC_FLAT_R = 256;
constexpr int ENC_FLAT_TILE = ENC_FLAT_R * 96, ENC_FLAT_IN = ENC_FLAT_R * 24, ENC_FLAT_WPE = 5;
constexpr int ENC_WIDE_TILE = ENC_FLAT_R * 112, ENC_WIDE_IN = ENC_FLAT_R * 32;
constexpr int ENC_NEST_BT = PJ_ENC_NEST_BT, ENC_NEST_R = PJ_ENC_NEST_R, ENC_NEST_TILE = PJ_ENC_NEST_TILE,
              ENC_NEST_IN = PJ_ENC_NEST_IN, ENC_NEST_UCAP = PJ_ENC_NEST_UCAP, ENC_NEST_GCAP = PJ_ENC_NEST_GCAP,
              ENC_NEST_WPE = PJ_ENC_NEST_WPE;

int pj_encode_block_records(bool nested) { return nested ? ENC_NEST_R : ENC_FLAT_R; }

namespace {
// Workgroups of kernel K that the device holds at once (cached per device
// and kernel): the persistent encode launches no more than that many, so
// every launched workgroup is resident.
// Workgroups of kern the current device holds at once, cached per device
// and kernel (every encode kernel has the same type, so the kernel's address
// is part of the key).
template <class K> unsigned resident_groups(K kern, int threads) {
    static std::mutex mu;
    static std::map<std::pair<int, const void *>, unsigned> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
    const auto key = std::make_pair(dev, reinterpret_cast<const void *>(kern));
    std::lock_guard<std::mutex> lk(mu);
    const auto it = cache.find(key);
    if (it != cache.end()) return it->second;
    int per_cu = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, threads, 0) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || per_cu <= 0 || cus <= 0)
        return 0;
    return cache[key] = (unsigned)(per_cu * cus);
}
template <class K>
hipError_t launch_encode(K kern, int threads, const EncParams &P, uint64_t records, bool persistent, hipStream_t st) {
    const uint64_t nblk = (P.n + records - 1) / records;
    const unsigned res = resident_groups(kern, threads);
    if (!res) return hipErrorInvalidConfiguration;
    const uint64_t g = nblk < res || !persistent ? nblk : res;
    hipLaunchKernelGGL(kern, dim3((unsigned)g), dim3(threads), 0, st, P);
    return hipGetLastError();
}
}  // namespace

hipError_t pj_launch_encode(const EncParams &P, bool nested, bool wide, hipStream_t st) {
    if (nested)
        return launch_encode(pj::k_encode<true, ENC_NEST_BT, ENC_NEST_R, ENC_NEST_TILE, ENC_NEST_IN, ENC_NEST_UCAP,
                                              ENC_NEST_GCAP, ENC_NEST_WPE>,
                                 ENC_NEST_BT, P, ENC_NEST_R, true, st);
    if (wide)
        return launch_encode(pj::k_encode<false, ENC_FLAT_BT, ENC_FLAT_R, ENC_WIDE_TILE, ENC_WIDE_IN, 1, 1>,
                                 ENC_FLAT_BT, P, ENC_FLAT_R, false, st);
    return launch_encode(pj::k_encode<false, ENC_FLAT_BT, ENC_FLAT_R, ENC_FLAT_TILE, ENC_FLAT_IN, 1, 1, ENC_FLAT_WPE>,
                             ENC_FLAT_BT, P, ENC_FLAT_R, false, st);
}

// Pretty output of nested records through the tile path: 64 records per
// block (a pretty record is about 350 bytes), otherwise the nested shape.
constexpr int ENC_PRETTY_TILE_R = 64;
int pj_encode_pretty_tile_records() { return ENC_PRETTY_TILE_R; }
hipError_t pj_launch_encode_pretty(const EncParams &P, hipStream_t st) {
    return launch_encode(pj::k_encode<true, ENC_NEST_BT, ENC_PRETTY_TILE_R, ENC_NEST_TILE, ENC_NEST_IN, ENC_NEST_UCAP,
                                      ENC_NEST_GCAP, ENC_NEST_WPE, true>,
                         ENC_NEST_BT, P, ENC_PRETTY_TILE_R, true, st);
}

// k_enc_big: one workgroup per large record, as many workgroups as the GPU
// holds at once (full), or 64 when the caller expects an empty list (its
// workgroups return at once; a longer list is still written, more slowly).
#ifndef PJ_ENC_BIG_BT
#define PJ_ENC_BIG_BT 256
#endif
hipError_t pj_launch_encode_big(const EncParams &P, bool full, hipStream_t st) {
    constexpr int BT = PJ_ENC_BIG_BT;
    const unsigned res = resident_groups(pj::k_enc_big<true, BT>, BT);
    if (!res) return hipErrorInvalidConfiguration;
    hipLaunchKernelGGL((pj::k_enc_big<true, BT>), dim3(full ? res : std::min(res, 64u)), dim3(BT), 0, st, P);
    return hipGetLastError();
}

// The measuring pass: ENC_MEAS_K blocks per workgroup of 512 threads.
constexpr int ENC_MEAS_BT = 512, ENC_MEAS_K = 4, ENC_MEAS_UN = 8;
uint64_t pj_encode_measure_groups(uint64_t n) {
    const uint64_t nblk = (n + ENC_NEST_R - 1) / ENC_NEST_R;
    return (nblk + ENC_MEAS_K - 1) / ENC_MEAS_K;
}
hipError_t pj_launch_encode_measure(const EncParams &P, hipStream_t st) {
    hipLaunchKernelGGL((pj::k_enc_measure<ENC_MEAS_BT, ENC_NEST_R, ENC_MEAS_K, ENC_MEAS_UN>),
                       dim3((unsigned)pj_encode_measure_groups(P.n)), dim3(ENC_MEAS_BT), 0, st, P);
    return hipGetLastError();
}

// 512-record blocks: measured fastest (256 with three workgroups per CU
// about the same; 128 and 64 slower, as more blocks chain their look-backs)
#ifndef PJ_ENC_ROWS_BT
#define PJ_ENC_ROWS_BT 512
#endif
constexpr int ENC_PRETTY_BT = PJ_ENC_ROWS_BT;
int pj_encode_pretty_records() { return ENC_PRETTY_BT; }

constexpr int ENC_SEL_BT = 256, ENC_SEL_R = 16;

hipError_t pj_launch_encode_rows(const EncParams &P, bool pretty, hipStream_t st) {
    const uint64_t nblk = (P.n + ENC_PRETTY_BT - 1) / ENC_PRETTY_BT;
    if (pretty)
        hipLaunchKernelGGL((pj::k_encode_rows<ENC_PRETTY_BT, true>), dim3((unsigned)nblk),
                           dim3(ENC_PRETTY_BT), 0, st, P);
    else
        hipLaunchKernelGGL((pj::k_encode_rows<ENC_PRETTY_BT, false>), dim3((unsigned)nblk),
                           dim3(ENC_PRETTY_BT), 0, st, P);
    return hipGetLastError();
}

uint64_t pj_select_blocks(uint64_t n) { return (n + ENC_SEL_BT * ENC_SEL_R - 1) / (ENC_SEL_BT * ENC_SEL_R); }

hipError_t pj_launch_select_status(const EncParams &P, uint32_t mask, uint64_t *sel, hipStream_t st) {
    hipLaunchKernelGGL((pj::k_select_status<ENC_SEL_BT, ENC_SEL_R>), dim3((unsigned)pj_select_blocks(P.c.n_pets)),
                       dim3(ENC_SEL_BT), 0, st, P, mask, sel);
    return hipGetLastError();
}

constexpr int ENC_MODEL_BT = 512;   // as for k_encode_rows: larger blocks, fewer chained look-backs
int pj_encode_model_records() { return ENC_MODEL_BT; }

hipError_t pj_launch_encode_model(const ModelEncParams &P, hipStream_t st) {
    const uint64_t nblk = (P.n + ENC_MODEL_BT - 1) / ENC_MODEL_BT;
    if (P.model == PJ_MODEL_ORDER)
        hipLaunchKernelGGL((pj::k_encode_model<PJ_MODEL_ORDER, ENC_MODEL_BT>), dim3((unsigned)nblk), dim3(ENC_MODEL_BT),
                           0, st, P);
    else
        hipLaunchKernelGGL((pj::k_encode_model<PJ_MODEL_USER, ENC_MODEL_BT>), dim3((unsigned)nblk), dim3(ENC_MODEL_BT),
                           0, st, P);
    return hipGetLastError();
}

hipError_t pj_launch_put_bytes(uint8_t *out, uint32_t w, int k, hipStream_t st) {
    hipLaunchKernelGGL(pj::k_put_bytes, dim3(1), dim3(64), 0, st, out, w, k);
    return hipGetLastError();
}

// ------------------------------------------------------ no-allocation scratch
// Encode scratch for pj_encode_device_noalloc: a fixed array every GPU the
// library runs on holds until the process ends.  In host code `scratch`
// names a host-side stand-in, not device memory; its device address (one
// per GPU) is resolved once per device by pj_noalloc_scratch_init, which
// pj_create calls with the device current, and only that address is ever
// handed to kernels.  Calls on one GPU share the array, so calls that
// overlap on one GPU race.
static __device__ __align__(256) uint64_t scratch[PJ_NOALLOC_SCRATCH_WORDS];

namespace {
constexpr int PJ_MAX_DEVICES = 64;
std::mutex g_scratch_mu;
uint64_t *g_scratch_ptr[PJ_MAX_DEVICES] = {};
}  // namespace

hipError_t pj_noalloc_scratch_init(int device, uint64_t **ptr) {
    if (device < 0 || device >= PJ_MAX_DEVICES) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[device]) {
        void *p = nullptr;
        hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        g_scratch_ptr[device] = static_cast<uint64_t *>(p);
    }
    *ptr = g_scratch_ptr[device];
    return hipSuccess;
}
