// pj_decode.hip — NDJSON -> columnar Pet decoder for gfx950.
//
// Stage 1, k_dec_index: one thread per 64-byte block of input, simdjson-style:
//   * exact quote / backslash masks (SWAR byte compares), escaped positions
//     from odd backslash runs (the run carried in from the previous block is
//     read back from memory), unescaped-quote mask Qu;
//   * in-string mask = prefix-XOR of Qu, reset after every newline, with the
//     carry (quote parity since the last newline) chained across blocks and
//     workgroups by a block scan + decoupled look-back whose state also
//     counts newlines;
//   * outputs: the "specials" bitmap (unescaped quotes | backslashes) that
//     lets the parser jump over strings, one flag per block for raw control
//     characters or malformed UTF-8 inside strings, and the line index.
// Stage 2, k_dec_parse: one thread per line.  A validating pass (string
// contents skipped through the bitmap; lines touching a flagged block take
// the byte-by-byte path) yields the record's column sizes; a block scan and
// a vector look-back over 8 counters give each valid record its row and
// byte offsets and each invalid one its slot in the error list; a second
// walk over the same line materialises the columns.
//
// The grammar and binding rules (RFC 8259 as enforced by jackson's
// UTF8StreamJsonParser, comments rejected per reference application.yml:23-28;
// serde bean binding of the petstore Pet, petstore.json:858-936) are the ones
// restated by the CPU checker in oracle/pj_oracle.c.
#include "pj_device.h"
#include "pj_kernels.h"

namespace pj {

// =========================================================== stage 1
// bit i of the result is set iff byte i of y is zero
__device__ __forceinline__ uint32_t zero_bytes4(uint32_t y) {
    uint32_t t = ((y & 0x7F7F7F7Fu) + 0x7F7F7F7Fu) | y;
    uint32_t z = ~t & 0x80808080u;
    return (((z >> 7) * 0x00204081u) >> 21) & 0xFu;
}
// bit i set iff byte i of x < c (c <= 0x80)
__device__ __forceinline__ uint32_t lt_bytes4(uint32_t x, uint32_t c) {
    uint32_t t = ((x & 0x7F7F7F7Fu) + (0x80u - c) * 0x01010101u) | x;
    uint32_t z = ~t & 0x80808080u;
    return (((z >> 7) * 0x00204081u) >> 21) & 0xFu;
}

__device__ __forceinline__ uint64_t prefix_xor(uint64_t x) {
    x ^= x << 1; x ^= x << 2; x ^= x << 4; x ^= x << 8; x ^= x << 16; x ^= x << 32;
    return x;
}

// Scan state of stage 1: bit 0 quote parity since the last newline, bit 1
// "a newline was seen", bits 2.. newline count.  a precedes b.
__device__ __forceinline__ uint64_t idx_combine(uint64_t a, uint64_t b) {
    uint64_t cnt = ((a >> 2) + (b >> 2)) << 2;
    uint64_t has = (a | b) & 2;
    uint64_t par = (b & 2) ? (b & 1) : ((a ^ b) & 1);
    return cnt | has | par;
}

template <int BT>
__device__ __forceinline__ uint64_t block_excl_scan_idx(uint64_t v, uint64_t *sh, uint64_t *total) {
    constexpr int NW = BT / 64;
    const int t = threadIdx.x, w = t >> 6, l = t & 63;
    uint64_t inc = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        uint64_t o = shfl_up_u64(inc, d);
        if (l >= d) inc = idx_combine(o, inc);
    }
    uint64_t excl = shfl_up_u64(inc, 1);
    if (l == 0) excl = 0;
    if (l == 63) sh[w] = inc;
    __syncthreads();
    uint64_t before = 0, tot = 0;
#pragma unroll
    for (int k = 0; k < NW; k++) {
        uint64_t s = sh[k];
        if (k < w) before = idx_combine(before, s);
        tot = idx_combine(tot, s);
    }
    __syncthreads();
    *total = tot;
    return idx_combine(before, excl);
}

// look-back with idx_combine (one full wave); values must fit LB_VAL.
__device__ __forceinline__ uint64_t lb_resolve_idx(uint64_t *state, uint64_t b, uint64_t agg) {
    const int l = lane_id();
    if (b == 0) return 0;
    uint64_t excl = 0;
    int64_t j = (int64_t)b - 1;
    for (;;) {
        int64_t idx = j - l;
        uint64_t s = idx >= 0 ? lb_load(&state[idx]) : LB_PRE;
        uint32_t fl = (uint32_t)(s >> 62);
        uint64_t notready = __ballot(fl == 0);
        uint64_t isp = __ballot(fl == 2);
        int fp = isp ? __builtin_ctzll(isp) : 64;
        uint64_t need = fp >= 63 ? ~0ull : ((2ull << fp) - 1);
        if (notready & need) { __builtin_amdgcn_s_sleep(1); continue; }
        // ordered reduction: higher lanes are earlier blocks
        uint64_t v = l <= fp ? (s & LB_VAL) : 0;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            uint64_t o = shfl_u64(v, (l + d) & 63);
            if (l + d < 64) v = idx_combine(o, v);
        }
        v = shfl_u64(v, 0);
        excl = idx_combine(v, excl);
        if (fp < 64) break;
        j -= 64;
    }
    if (l == 0) lb_store(&state[b], LB_PRE | idx_combine(excl, agg));
    return excl;
}

template <int BT>
__global__ __launch_bounds__(BT) void k_dec_index(DecParams P) {
    __shared__ uint64_t sh_scan[BT / 64];
    __shared__ uint64_t sh_blk, sh_pre;
    const uint32_t t = threadIdx.x;
    if (t == 0) sh_blk = atomicAdd(&P.tickets[0], 1ull);
    __syncthreads();
    const uint64_t b = sh_blk;
    const uint64_t blk = b * BT + t;
    const bool live = blk < P.nblk64;
    const uint64_t st = blk * 64;
    const uint8_t *in = P.in;

    uint32_t w[16];
    if (live && st + 64 <= P.len) {
        const uint4 *q = reinterpret_cast<const uint4 *>(in + st);
#pragma unroll
        for (int k = 0; k < 4; k++) {
            uint4 v = q[k];
            w[4 * k] = v.x; w[4 * k + 1] = v.y; w[4 * k + 2] = v.z; w[4 * k + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int k = 0; k < 16; k++) w[k] = 0x20202020u;
        if (live) {
            for (uint32_t j = 0; st + j < P.len; j++) {
                uint32_t sh = 8 * (j & 3);
                w[j >> 2] = (w[j >> 2] & ~(0xFFu << sh)) | ((uint32_t)in[st + j] << sh);
            }
        }
    }
    // ---- byte classes
    uint64_t Q = 0, Bm = 0, C = 0, N = 0;
    uint32_t anyb = 0, anyc = 0, anyh = 0;
#pragma unroll
    for (int k = 0; k < 16; k++) {
        const uint32_t x = w[k];
        Q |= (uint64_t)zero_bytes4(x ^ 0x22222222u) << (4 * k);
        anyb |= any_zero(x ^ 0x5C5C5C5Cu);
        anyc |= any_lt20(x);
        anyh |= x & 0x80808080u;
    }
    if (anyb) {
#pragma unroll
        for (int k = 0; k < 16; k++) Bm |= (uint64_t)zero_bytes4(w[k] ^ 0x5C5C5C5Cu) << (4 * k);
    }
    if (anyc) {
#pragma unroll
        for (int k = 0; k < 16; k++) {
            C |= (uint64_t)lt_bytes4(w[k], 0x20) << (4 * k);
            N |= (uint64_t)zero_bytes4(w[k] ^ 0x0A0A0A0Au) << (4 * k);
        }
    }
    // UTF-8 structure (jackson: leads C0-DF / E0-EF / F0-F7, 10xxxxxx continuations)
    uint64_t u8err = 0, expect_in = 0;
    uint32_t bs_run = 0;
    if (live && st > 0) {
        // bytes just before the block: backslash run parity and pending continuations
        uint64_t a = st >= 8 ? st - 8 : 0;
        uint64_t prev = 0;
        for (uint64_t j = a; j < st; j++) prev |= (uint64_t)in[j] << (8 * (j - a + 8 - (st - a)));
        // prev holds the (up to) 8 bytes before st, the byte at st-1 in bits 63:56
        for (int k = 7; k >= 0 && ((prev >> (8 * k)) & 0xFF) == '\\' && (uint64_t)(8 - k) <= st; k--) bs_run++;
        if (bs_run == 8) {
            uint64_t q = st - 8;
            while (q > 0 && in[q - 1] == '\\') { bs_run++; q--; }
        }
        uint32_t b1 = (uint32_t)(prev >> 56) & 0xFF, b2 = (uint32_t)(prev >> 48) & 0xFF, b3 = (uint32_t)(prev >> 40) & 0xFF;
        if (st >= 1) {
            if (b1 >= 0xC0 && b1 <= 0xDF) expect_in |= 1;
            else if (b1 >= 0xE0 && b1 <= 0xEF) expect_in |= 3;
            else if (b1 >= 0xF0 && b1 <= 0xF7) expect_in |= 7;
        }
        if (st >= 2) {
            if (b2 >= 0xE0 && b2 <= 0xEF) expect_in |= 1;
            else if (b2 >= 0xF0 && b2 <= 0xF7) expect_in |= 3;
        }
        if (st >= 3 && b3 >= 0xF0 && b3 <= 0xF7) expect_in |= 1;
    }
    if (anyh | expect_in) {
        uint64_t cont = 0, l2 = 0, l3 = 0, l4 = 0, badl = 0;
        for (int j = 0; j < 64; j++) {
            uint32_t c = (w[j >> 2] >> (8 * (j & 3))) & 0xFF;
            uint64_t bit = 1ull << j;
            if (c < 0x80) continue;
            if (c < 0xC0) cont |= bit;
            else if (c < 0xE0) l2 |= bit;
            else if (c < 0xF0) l3 |= bit;
            else if (c < 0xF8) l4 |= bit;
            else badl |= bit;
        }
        uint64_t expect = (l2 << 1) | (l3 << 1) | (l3 << 2) | (l4 << 1) | (l4 << 2) | (l4 << 3) | expect_in;
        u8err = (cont ^ expect) | badl;
    }
    // ---- escapes: position e after a backslash run is escaped iff the run
    // (including its part before the block) has odd length
    uint64_t E = 0;
    const bool c_odd = bs_run & 1;
    if (Bm) {
        constexpr uint64_t EVEN = 0x5555555555555555ull, ODD = ~EVEN;
        uint64_t rs = Bm & ~(Bm << 1);
        uint64_t rs_e = rs & EVEN, rs_o = rs & ODD;
        if (c_odd && (Bm & 1)) { rs_e &= ~1ull; rs_o |= 1ull; }
        E = (((Bm + rs_e) & ~Bm) & ODD) | (((Bm + rs_o) & ~Bm) & EVEN);
    }
    if (c_odd && !(Bm & 1)) E |= 1ull;
    const uint64_t Qu = Q & ~E;
    // ---- block summary for the scan
    uint64_t summ = 0;
    if (live) {
        uint64_t par;
        if (N) {
            int last = 63 - __builtin_clzll(N);
            uint64_t above = last == 63 ? 0 : (Qu >> (last + 1));
            par = __builtin_popcountll(above) & 1;
        } else par = __builtin_popcountll(Qu) & 1;
        summ = ((uint64_t)__builtin_popcountll(N) << 2) | (N ? 2 : 0) | par;
    }
    uint64_t agg;
    const uint64_t pre_in = block_excl_scan_idx<BT>(summ, sh_scan, &agg);
    if (t == 0) lb_store(&P.state_idx[b], (b == 0 ? LB_PRE : LB_AGG) | agg);
    if (t < 64) {
        uint64_t e = lb_resolve_idx(P.state_idx, b, agg);
        if (t == 0) sh_pre = e;
    }
    __syncthreads();
    if (!live) return;
    const uint64_t carry = idx_combine(sh_pre, pre_in);
    const uint64_t lines_before = carry >> 2;
    const uint64_t cin = carry & 1;                 // in a string at block start
    // ---- in-string mask with resets after newlines
    uint64_t x = prefix_xor(Qu) ^ (cin ? ~0ull : 0ull);
    for (uint64_t m = N; m; m &= m - 1) {
        int p = __builtin_ctzll(m);
        if ((x >> p) & 1) x ^= p == 63 ? 0ull : (~0ull << (p + 1));
    }
    const uint64_t inS = x;
    const uint64_t near = inS | (inS << 1) | cin;
    const uint64_t bad = (C & inS) | (u8err & near);
    P.special[blk] = Bm | Qu;
    P.bad[blk] = bad ? 1 : 0;
    // ---- line index
    uint64_t li = lines_before;
    for (uint64_t m = N; m; m &= m - 1) {
        int p = __builtin_ctzll(m);
        li++;
        if (li < P.ls_cap) P.line_start[li] = st + (uint64_t)p + 1;
    }
    if (blk == 0) P.line_start[0] = 0;
    if (blk == P.nblk64 - 1) {
        uint32_t lastb = (w[((P.len - 1) & 63) >> 2] >> (8 * ((P.len - 1) & 3))) & 0xFF;
        uint64_t nl = li + (lastb != '\n' ? 1 : 0);
        if (lastb != '\n' && nl < P.ls_cap) P.line_start[nl] = P.len + 1;
        *P.n_lines = nl;
    }
}

// =========================================================== stage 2
enum { K_UNKNOWN = 0, K_ID, K_CATEGORY, K_NAME, K_PHOTOURLS, K_TAGS, K_STATUS };

struct LineInfo {
    int64_t id, cat_id;
    uint32_t name_pos, name_len, cat_pos, cat_len, photo_pos, n_urls, url_bytes, tags_pos, n_tags, tag_bytes;
    uint8_t has_id, has_cat, has_name, has_photo, has_tags, cat_flags, status, name_esc;
};

__device__ __forceinline__ int hexval(int c) {
    if (c >= '0' && c <= '9') return c - '0';
    if (c >= 'a' && c <= 'f') return c - 'a' + 10;
    if (c >= 'A' && c <= 'F') return c - 'A' + 10;
    return -1;
}
__device__ __forceinline__ bool is_ident(int c) {
    return (c >= 'a' && c <= 'z') || (c >= 'A' && c <= 'Z') || (c >= '0' && c <= '9') || c == '_' || c == '$' ||
           c >= 0x80;
}
// UTF-8 bytes of code point cp, packed little endian; *k = count
__device__ __forceinline__ uint32_t utf8_pack(uint32_t cp, int *k) {
    if (cp < 0x80) { *k = 1; return cp; }
    if (cp < 0x800) { *k = 2; return (0xC0 | (cp >> 6)) | ((0x80 | (cp & 63)) << 8); }
    if (cp < 0x10000) {
        *k = 3;
        return (0xE0 | (cp >> 12)) | ((0x80 | ((cp >> 6) & 63)) << 8) | ((0x80 | (cp & 63)) << 16);
    }
    *k = 4;
    return (0xF0 | (cp >> 18)) | ((0x80 | ((cp >> 12) & 63)) << 8) | ((0x80 | ((cp >> 6) & 63)) << 16) |
           ((0x80u | (cp & 63)) << 24);
}

// Line parser.  SLOW validates every string byte itself; otherwise string
// contents are trusted (stage 1 flagged none) and skipped via the bitmap.
template <bool SLOW>
struct LP {
    const uint8_t *in;
    uint64_t len;            // whole input length
    const uint64_t *special;
    uint64_t s0;             // absolute start of the line
    uint32_t n;              // line length (without '\n')
    uint32_t p;              // cursor, relative to s0
    int depth;
    uint64_t wlo, whi;       // 16-byte window [wp, wp+16)
    uint32_t wp;

    __device__ __forceinline__ void init(const DecParams &P, uint64_t start, uint32_t nn) {
        in = P.in; len = P.len; special = P.special; s0 = start; n = nn; p = 0; depth = 0;
        wp = 0xFFFFFF00u; wlo = whi = 0;
    }
    __device__ __forceinline__ void refill(uint32_t q) {
        const uint64_t a = s0 + q;
        wp = q;
        if (a + 16 <= len) {
            wlo = ldu64(in + a);
            whi = ldu64(in + a + 8);
        } else {
            wlo = whi = 0;
            for (uint32_t j = 0; j < 16 && a + j < len; j++) {
                uint64_t v = (uint64_t)in[a + j] << (8 * (j & 7));
                if (j < 8) wlo |= v; else whi |= v;
            }
        }
    }
    __device__ __forceinline__ int at(uint32_t q) {   // q < n
        if (q - wp >= 16) refill(q);
        const uint32_t d = q - wp;
        return (int)(((d < 8 ? wlo : whi) >> (8 * (d & 7))) & 0xFF);
    }
    __device__ __forceinline__ int peek() { return p < n ? at(p) : -1; }
    __device__ __forceinline__ void skip_ws() {
        while (p < n) {
            int c = at(p);
            if (c != ' ' && c != '\t' && c != '\r') break;
            p++;
        }
    }
    // first unescaped quote or backslash at or after q (n if none)
    __device__ __forceinline__ uint32_t next_special(uint32_t q) {
        const uint64_t a = s0 + q, lim = s0 + n;
        if (a >= lim) return n;
        uint64_t wi = a >> 6;
        uint64_t m = special[wi] & (~0ull << (a & 63));
        while (!m) {
            wi++;
            if (wi * 64 >= lim) return n;
            m = special[wi];
        }
        const uint64_t pos = wi * 64 + (uint64_t)__builtin_ctzll(m);
        return pos >= lim ? n : (uint32_t)(pos - s0);
    }
    // escape sequence at q ('\\'): *adv bytes consumed, decoded bytes packed
    // in *out (*k of them)
    __device__ __forceinline__ int escape_at(uint32_t q, uint32_t *adv, uint32_t *out, int *k) {
        if (q + 1 >= n) return PJ_REC_STRING;
        int e = at(q + 1);
        *k = 1;
        *adv = 2;
        switch (e) {
        case '"': *out = '"'; return 0;
        case '\\': *out = '\\'; return 0;
        case '/': *out = '/'; return 0;
        case 'b': *out = 8; return 0;
        case 'f': *out = 12; return 0;
        case 'n': *out = 10; return 0;
        case 'r': *out = 13; return 0;
        case 't': *out = 9; return 0;
        case 'u': break;
        default: return PJ_REC_STRING;
        }
        if (q + 6 > n) return PJ_REC_STRING;
        uint32_t cu = 0;
        for (int j = 0; j < 4; j++) {
            int h = hexval(at(q + 2 + j));
            if (h < 0) return PJ_REC_STRING;
            cu = cu * 16 + (uint32_t)h;
        }
        *adv = 6;
        if (cu >= 0xDC00 && cu <= 0xDFFF) return PJ_REC_STRING;
        if (cu >= 0xD800 && cu <= 0xDBFF) {
            if (q + 8 > n || at(q + 6) != '\\' || at(q + 7) != 'u') return PJ_REC_STRING;
            if (q + 12 > n) return PJ_REC_STRING;
            uint32_t lo = 0;
            for (int j = 0; j < 4; j++) {
                int h = hexval(at(q + 8 + j));
                if (h < 0) return PJ_REC_STRING;
                lo = lo * 16 + (uint32_t)h;
            }
            if (lo < 0xDC00 || lo > 0xDFFF) return PJ_REC_STRING;
            cu = 0x10000 + ((cu - 0xD800) << 10) + (lo - 0xDC00);
            *adv = 12;
        }
        *out = utf8_pack(cu, k);
        return 0;
    }
    // string whose opening quote is at q: closing quote position, decoded
    // length, whether it holds escapes
    __device__ int str_scan(uint32_t q, uint32_t *end, uint32_t *dlen, bool *esc) {
        uint32_t pos = q + 1, d = 0;
        bool es = false;
        if (SLOW) {
            for (;;) {
                if (pos >= n) return PJ_REC_STRING;
                int c = at(pos);
                if (c == '"') break;
                if (c == '\\') {
                    uint32_t adv, o;
                    int k;
                    int e = escape_at(pos, &adv, &o, &k);
                    if (e) return e;
                    d += (uint32_t)k;
                    pos += adv;
                    es = true;
                    continue;
                }
                if (c < 0x20) return PJ_REC_STRING;
                int extra;
                if (c < 0x80) extra = 0;
                else if (c >= 0xC0 && c <= 0xDF) extra = 1;
                else if (c >= 0xE0 && c <= 0xEF) extra = 2;
                else if (c >= 0xF0 && c <= 0xF7) extra = 3;
                else return PJ_REC_STRING;
                if (pos + 1 + (uint32_t)extra > n) return PJ_REC_STRING;
                for (int j = 1; j <= extra; j++)
                    if ((at(pos + j) & 0xC0) != 0x80) return PJ_REC_STRING;
                d += 1 + (uint32_t)extra;
                pos += 1 + (uint32_t)extra;
            }
        } else {
            for (;;) {
                uint32_t sp = next_special(pos);
                if (sp >= n) return PJ_REC_STRING;
                d += sp - pos;
                if (at(sp) == '"') { pos = sp; break; }
                uint32_t adv, o;
                int k;
                int e = escape_at(sp, &adv, &o, &k);
                if (e) return e;
                d += (uint32_t)k;
                pos = sp + adv;
                es = true;
            }
        }
        *end = pos;
        *dlen = d;
        *esc = es;
        return 0;
    }
    // decoded bytes of a (validated) string, first 16 of them
    __device__ void small_decode(uint32_t q, uint32_t end, bool esc, uint64_t *lo, uint64_t *hi) {
        uint64_t v[2] = {0, 0};
        uint32_t pos = q + 1, o = 0;
        while (pos < end && o < 16) {
            int c = at(pos);
            uint32_t bytes = (uint32_t)c, adv = 1;
            int k = 1;
            if (esc && c == '\\') escape_at(pos, &adv, &bytes, &k);
            for (int j = 0; j < k && o < 16; j++, o++) v[o >> 3] |= (uint64_t)((bytes >> (8 * j)) & 0xFF) << (8 * (o & 7));
            pos += adv;
        }
        *lo = v[0];
        *hi = v[1];
    }
    // number grammar; *real when a fraction or exponent is present
    __device__ int rd_number(bool *real) {
        uint32_t q = p;
        bool r = false;
        if (q < n && at(q) == '-') q++;
        if (q >= n) return PJ_REC_SYNTAX;
        int c = at(q);
        if (c == '0') {
            q++;
            if (q < n && at(q) >= '0' && at(q) <= '9') return PJ_REC_SYNTAX;
        } else if (c >= '1' && c <= '9') {
            while (q < n && at(q) >= '0' && at(q) <= '9') q++;
        } else return PJ_REC_SYNTAX;
        if (q < n && at(q) == '.') {
            q++;
            r = true;
            if (q >= n || at(q) < '0' || at(q) > '9') return PJ_REC_SYNTAX;
            while (q < n && at(q) >= '0' && at(q) <= '9') q++;
        }
        if (q < n && (at(q) == 'e' || at(q) == 'E')) {
            q++;
            r = true;
            if (q < n && (at(q) == '+' || at(q) == '-')) q++;
            if (q >= n || at(q) < '0' || at(q) > '9') return PJ_REC_SYNTAX;
            while (q < n && at(q) >= '0' && at(q) <= '9') q++;
        }
        p = q;
        *real = r;
        return 0;
    }
    // literal or number; *kind: 0 null, 1 true, 2 false, 3 int, 4 real
    __device__ int rd_scalar(int *kind) {
        int c = peek();
        if (c == '-' || (c >= '0' && c <= '9')) {
            bool real;
            int e = rd_number(&real);
            *kind = real ? 4 : 3;
            return e;
        }
        uint32_t L;
        uint64_t want;
        if (c == 'n') { L = 4; want = 0x6C6C756Eull; *kind = 0; }
        else if (c == 't') { L = 4; want = 0x65757274ull; *kind = 1; }
        else if (c == 'f') { L = 5; want = 0x65736C6166ull; *kind = 2; }
        else return PJ_REC_SYNTAX;
        if (p + L > n) return PJ_REC_SYNTAX;
        for (uint32_t j = 0; j < L; j++)
            if ((uint64_t)at(p + j) != ((want >> (8 * j)) & 0xFF)) return PJ_REC_SYNTAX;
        if (p + L < n && is_ident(at(p + L))) return PJ_REC_SYNTAX;
        p += L;
        return 0;
    }
    __device__ int type_mismatch() {
        int c = peek();
        if (c == '"' || c == '{' || c == '[') return PJ_REC_TYPE;
        int kind;
        int e = rd_scalar(&kind);
        return e ? e : PJ_REC_TYPE;
    }
    // null literal at the cursor? (consumes it)  1 = null, 0 = not null, <0 error
    __device__ int rd_null_or_mismatch(int *err) {
        int kind;
        int e = rd_scalar(&kind);
        if (e) { *err = e; return -1; }
        if (kind != 0) { *err = PJ_REC_TYPE; return -1; }
        return 1;
    }
    // int64 value or null
    __device__ int rd_long(int64_t *v, bool *present) {
        int c = peek();
        if (c == 'n') {
            int err = 0;
            if (rd_null_or_mismatch(&err) < 0) return err;
            *present = false;
            return 0;
        }
        if (!(c == '-' || (c >= '0' && c <= '9'))) return type_mismatch();
        const uint32_t start = p;
        bool real;
        int e = rd_number(&real);
        if (e) return e;
        if (real) return PJ_REC_NUMBER;
        const bool neg = at(start) == '-';
        const uint64_t lim = neg ? (1ull << 63) : ((1ull << 63) - 1);
        uint64_t acc = 0;
        for (uint32_t q = start + (neg ? 1 : 0); q < p; q++) {
            uint64_t d = (uint64_t)(at(q) - '0');
            if (acc > (lim - d) / 10) return PJ_REC_NUMBER;
            acc = acc * 10 + d;
        }
        *v = neg ? (int64_t)(0ull - acc) : (int64_t)acc;
        *present = true;
        return 0;
    }
    __device__ int open_container() {
        if (++depth > PJ_MAX_DEPTH) return PJ_REC_DEPTH;
        p++;
        skip_ws();
        return 0;
    }
    // kind of the innermost container still open at local nesting level d
    // (1-based) of a value that starts at v0: object = true.  Used beyond the
    // 64 levels the register stack holds.
    __device__ bool opener_at(uint32_t v0, int d) {
        int lvl = 0;
        bool kind = false, instr = false;
        for (uint32_t q = v0; q < p; q++) {
            int c = at(q);
            if (instr) {
                if (c == '\\') q++;
                else if (c == '"') instr = false;
                continue;
            }
            if (c == '"') instr = true;
            else if (c == '{' || c == '[') { lvl++; if (lvl == d) kind = c == '{'; }
            else if (c == '}' || c == ']') lvl--;
        }
        return kind;
    }
    // skip any JSON value (validated), iteratively
    __device__ int skip_value() {
        int c = peek();
        if (c == '"') {
            uint32_t end, dl;
            bool es;
            int e = str_scan(p, &end, &dl, &es);
            if (e) return e;
            p = end + 1;
            return 0;
        }
        if (c != '{' && c != '[') {
            int kind;
            return rd_scalar(&kind);
        }
        const uint32_t v0 = p;
        uint64_t stack = 0;
        int d = 0;
        enum { S_OPEN, S_KEY, S_VALUE, S_AFTER } state = S_OPEN;
        for (;;) {
            switch (state) {
            case S_OPEN: {
                c = peek();
                const bool obj = c == '{';
                if (d < 64) stack = obj ? (stack | (1ull << d)) : (stack & ~(1ull << d));
                d++;
                int e = open_container();
                if (e) return e;
                c = peek();
                if (c == (obj ? '}' : ']')) { p++; depth--; d--; if (d == 0) return 0; state = S_AFTER; }
                else state = obj ? S_KEY : S_VALUE;
                break;
            }
            case S_KEY: {
                skip_ws();
                if (peek() != '"') return PJ_REC_SYNTAX;
                uint32_t end, dl;
                bool es;
                int e = str_scan(p, &end, &dl, &es);
                if (e) return e;
                p = end + 1;
                skip_ws();
                if (peek() != ':') return PJ_REC_SYNTAX;
                p++;
                skip_ws();
                if (p >= n) return PJ_REC_SYNTAX;
                state = S_VALUE;
                break;
            }
            case S_VALUE: {
                skip_ws();
                c = peek();
                if (c < 0) return PJ_REC_SYNTAX;
                if (c == '{' || c == '[') { state = S_OPEN; break; }
                if (c == '"') {
                    uint32_t end, dl;
                    bool es;
                    int e = str_scan(p, &end, &dl, &es);
                    if (e) return e;
                    p = end + 1;
                } else {
                    int kind;
                    int e = rd_scalar(&kind);
                    if (e) return e;
                }
                state = S_AFTER;
                break;
            }
            case S_AFTER: {
                skip_ws();
                c = peek();
                const bool obj = d <= 64 ? ((stack >> (d - 1)) & 1) : opener_at(v0, d);
                if (c == ',') { p++; state = obj ? S_KEY : S_VALUE; break; }
                if (c == (obj ? '}' : ']')) {
                    p++;
                    depth--;
                    d--;
                    if (d == 0) return 0;
                    break;
                }
                return PJ_REC_SYNTAX;
            }
            }
        }
    }
    // member loop helpers: after '{' consumed by open_container
    //   returns 1 = a member key was read (key id in *key, cursor at value),
    //   0 = object closed, <0 = -error
    __device__ int first_member(int *key, bool *more) {
        if (peek() == '}') { p++; depth--; *more = false; return 0; }
        *more = true;
        return read_key(key);
    }
    __device__ int next_member(int *key, bool *more) {
        skip_ws();
        int c = peek();
        if (c == ',') { p++; *more = true; return read_key(key); }
        if (c == '}') { p++; depth--; *more = false; return 0; }
        return PJ_REC_SYNTAX;
    }
    __device__ int read_key(int *key) {
        skip_ws();
        if (peek() != '"') return PJ_REC_SYNTAX;
        uint32_t end, dl;
        bool es;
        int e = str_scan(p, &end, &dl, &es);
        if (e) return e;
        *key = K_UNKNOWN;
        if (dl == 2 || dl == 4 || dl == 6 || dl == 8 || dl == 9) {
            uint64_t lo, hi;
            small_decode(p, end, es, &lo, &hi);
            if (dl == 2 && lo == 0x6469ull) *key = K_ID;                                   // id
            else if (dl == 8 && lo == 0x79726F6765746163ull) *key = K_CATEGORY;            // category
            else if (dl == 4 && lo == 0x656D616Eull) *key = K_NAME;                        // name
            else if (dl == 9 && lo == 0x6C72556F746F6870ull && hi == 0x73ull) *key = K_PHOTOURLS;  // photoUrls
            else if (dl == 4 && lo == 0x73676174ull) *key = K_TAGS;                        // tags
            else if (dl == 6 && lo == 0x737574617473ull) *key = K_STATUS;                  // status
        }
        p = end + 1;
        skip_ws();
        if (peek() != ':') return PJ_REC_SYNTAX;
        p++;
        skip_ws();
        if (p >= n) return PJ_REC_SYNTAX;
        return 0;
    }
    // string property: string or null
    __device__ int rd_str_prop(bool *present, uint32_t *pos, uint32_t *dlen, bool *esc) {
        int c = peek();
        if (c == '"') {
            uint32_t end;
            int e = str_scan(p, &end, dlen, esc);
            if (e) return e;
            *pos = p;
            *present = true;
            p = end + 1;
            return 0;
        }
        if (c == 'n') {
            int err = 0;
            if (rd_null_or_mismatch(&err) < 0) return err;
            *present = false;
            return 0;
        }
        return type_mismatch();
    }
    // Category / Tag object (cursor at '{'): last id / name win
    __device__ int rd_sub(int64_t *id, uint8_t *fl, uint32_t *name_len) {
        int e = open_container();
        if (e) return e;
        *id = 0;
        *fl = 0;
        *name_len = 0;
        int key;
        bool more;
        e = first_member(&key, &more);
        while (!e && more) {
            if (key == K_ID) {
                int64_t v = 0;
                bool pr;
                e = rd_long(&v, &pr);
                if (e) return e;
                *id = pr ? v : 0;
                *fl = pr ? (*fl | PJ_SUB_HAS_ID) : (*fl & ~PJ_SUB_HAS_ID);
            } else if (key == K_NAME) {
                bool pr;
                uint32_t pos, dl;
                bool es;
                e = rd_str_prop(&pr, &pos, &dl, &es);
                if (e) return e;
                *name_len = pr ? dl : 0;
                *fl = pr ? (*fl | PJ_SUB_HAS_NAME) : (*fl & ~PJ_SUB_HAS_NAME);
            } else {
                e = skip_value();
                if (e) return e;
            }
            e = next_member(&key, &more);
        }
        return e;
    }

    // ---- validating pass over the whole line
    __device__ int parse(LineInfo &L) {
        L.has_id = L.has_cat = L.has_name = L.has_photo = L.has_tags = 0;
        L.id = L.cat_id = 0;
        L.cat_flags = 0;
        L.status = PJ_STATUS_NULL;
        L.name_len = L.cat_len = L.n_urls = L.url_bytes = L.n_tags = L.tag_bytes = 0;
        L.name_pos = L.cat_pos = L.photo_pos = L.tags_pos = 0;
        L.name_esc = 0;
        skip_ws();
        if (p >= n) return PJ_REC_EMPTY;
        if (peek() != '{') return type_mismatch();
        int e = open_container();
        if (e) return e;
        int key;
        bool more;
        e = first_member(&key, &more);
        while (!e && more) {
            const int c = peek();
            switch (key) {
            case K_ID: {
                int64_t v = 0;
                bool pr = false;
                e = rd_long(&v, &pr);
                L.has_id = pr;
                L.id = pr ? v : 0;
                break;
            }
            case K_CATEGORY:
                if (c == '{') {
                    L.has_cat = 1;
                    L.cat_pos = p;
                    e = rd_sub(&L.cat_id, &L.cat_flags, &L.cat_len);
                } else if (c == 'n') {
                    int err = 0;
                    if (rd_null_or_mismatch(&err) < 0) e = err;
                    else { L.has_cat = 0; L.cat_id = 0; L.cat_flags = 0; L.cat_len = 0; }
                } else e = type_mismatch();
                break;
            case K_NAME: {
                bool pr = false, es = false;
                uint32_t pos = 0, dl = 0;
                e = rd_str_prop(&pr, &pos, &dl, &es);
                L.has_name = pr;
                L.name_pos = pos;
                L.name_len = pr ? dl : 0;
                L.name_esc = es;
                break;
            }
            case K_PHOTOURLS:
                if (c == '[') {
                    L.has_photo = 1;
                    L.photo_pos = p;
                    L.n_urls = 0;
                    L.url_bytes = 0;
                    e = open_container();
                    if (e) break;
                    if (peek() == ']') { p++; depth--; break; }
                    for (;;) {
                        skip_ws();
                        if (peek() != '"') { e = p >= n ? PJ_REC_SYNTAX : type_mismatch(); break; }
                        uint32_t end, dl;
                        bool es;
                        e = str_scan(p, &end, &dl, &es);
                        if (e) break;
                        p = end + 1;
                        L.n_urls++;
                        L.url_bytes += dl;
                        skip_ws();
                        int d = peek();
                        if (d == ',') { p++; continue; }
                        if (d == ']') { p++; depth--; break; }
                        e = PJ_REC_SYNTAX;
                        break;
                    }
                } else if (c == 'n') {
                    int err = 0;
                    if (rd_null_or_mismatch(&err) < 0) e = err;
                    else { L.has_photo = 0; L.n_urls = 0; L.url_bytes = 0; }
                } else e = type_mismatch();
                break;
            case K_TAGS:
                if (c == '[') {
                    L.has_tags = 1;
                    L.tags_pos = p;
                    L.n_tags = 0;
                    L.tag_bytes = 0;
                    e = open_container();
                    if (e) break;
                    if (peek() == ']') { p++; depth--; break; }
                    for (;;) {
                        skip_ws();
                        if (peek() != '{') { e = p >= n ? PJ_REC_SYNTAX : type_mismatch(); break; }
                        int64_t tid;
                        uint8_t tfl;
                        uint32_t tl;
                        e = rd_sub(&tid, &tfl, &tl);
                        if (e) break;
                        L.n_tags++;
                        L.tag_bytes += tl;
                        skip_ws();
                        int d = peek();
                        if (d == ',') { p++; continue; }
                        if (d == ']') { p++; depth--; break; }
                        e = PJ_REC_SYNTAX;
                        break;
                    }
                } else if (c == 'n') {
                    int err = 0;
                    if (rd_null_or_mismatch(&err) < 0) e = err;
                    else { L.has_tags = 0; L.n_tags = 0; L.tag_bytes = 0; }
                } else e = type_mismatch();
                break;
            case K_STATUS: {
                bool pr = false, es = false;
                uint32_t pos = 0, dl = 0;
                e = rd_str_prop(&pr, &pos, &dl, &es);
                if (e) break;
                if (!pr) { L.status = PJ_STATUS_NULL; break; }
                uint64_t lo = 0, hi = 0;
                if (dl == 9 || dl == 7 || dl == 4) {
                    uint32_t end = p - 1;   // closing quote
                    small_decode(pos, end, es, &lo, &hi);
                }
                if (dl == 9 && lo == 0x6C62616C69617661ull && hi == 0x65ull) L.status = PJ_STATUS_AVAILABLE;
                else if (dl == 7 && lo == 0x676E69646E6570ull) L.status = PJ_STATUS_PENDING;
                else if (dl == 4 && lo == 0x646C6F73ull) L.status = PJ_STATUS_SOLD;
                else e = PJ_REC_BAD_STATUS;
                break;
            }
            default:
                e = skip_value();
            }
            if (e) break;
            e = next_member(&key, &more);
        }
        if (e) return e;
        if (!L.has_name) return PJ_REC_MISSING_NAME;
        if (!L.has_photo) return PJ_REC_MISSING_PHOTOURLS;
        skip_ws();
        if (p < n) return PJ_REC_SYNTAX;
        return 0;
    }

    // ---- materialisation helpers (line known valid)
    // copy the decoded string whose opening quote is at q into ws
    __device__ void copy_str(uint32_t q, WriteSink &ws) {
        uint32_t end, dl;
        bool es;
        str_scan(q, &end, &dl, &es);
        uint32_t pos = q + 1;
        if (!es) {
            const uint8_t *src = in + s0 + pos;
            uint32_t L = end - pos, k = 0;
            for (; k + 8 <= L; k += 8) ws.put8(ldu64(src + k), 8);
            if (k < L) ws.put8(ld_tail(src + k, (int)(L - k)), (int)(L - k));
            return;
        }
        while (pos < end) {
            int c = at(pos);
            if (c == '\\') {
                uint32_t adv, o;
                int k;
                escape_at(pos, &adv, &o, &k);
                ws.put(o, k);
                pos += adv;
            } else {
                ws.put_byte((uint32_t)c);
                pos++;
            }
        }
    }
    // position of the opening quote of the last "name" of the object at q
    __device__ uint32_t last_name_of(uint32_t q) {
        p = q;
        open_container();
        int key;
        bool more;
        uint32_t last = 0;
        int e = first_member(&key, &more);
        while (!e && more) {            // every step advances p or stops
            if (key == K_NAME && peek() == '"') last = p;
            if (skip_value()) break;
            e = next_member(&key, &more);
        }
        return last;
    }
};

// ---- vector look-back over PJ_DEC_NCNT counters
// per block: [flag][agg x NC][inc x NC]
constexpr int VLB_STRIDE = 1 + 2 * PJ_DEC_NCNT;

__device__ __forceinline__ void vlb_publish(uint64_t *st, uint64_t b, const uint64_t *agg, int lane) {
    uint64_t *s = st + b * VLB_STRIDE;
    if (lane < PJ_DEC_NCNT) lb_store(&s[1 + lane], agg[lane]);
    if (b == 0 && lane < PJ_DEC_NCNT) lb_store(&s[1 + PJ_DEC_NCNT + lane], agg[lane]);
    __threadfence();
    if (lane == 0) lb_store(&s[0], b == 0 ? 2 : 1);
}

// one full wave; returns the exclusive prefix in excl[] (all lanes)
__device__ __forceinline__ void vlb_resolve(uint64_t *st, uint64_t b, const uint64_t *agg, uint64_t *excl) {
    const int l = lane_id();
    for (int k = 0; k < PJ_DEC_NCNT; k++) excl[k] = 0;
    if (b == 0) return;
    int64_t j = (int64_t)b - 1;
    for (;;) {
        int64_t idx = j - l;
        uint64_t f = idx >= 0 ? lb_load(&st[idx * VLB_STRIDE]) : 2;
        uint64_t notready = __ballot(f == 0);
        uint64_t isp = __ballot(f == 2);
        int fp = isp ? __builtin_ctzll(isp) : 64;
        uint64_t need = fp >= 63 ? ~0ull : ((2ull << fp) - 1);
        if (notready & need) { __builtin_amdgcn_s_sleep(1); continue; }
        __threadfence();
        const bool use = l <= fp && idx >= 0;
        const uint64_t *src = st + (idx >= 0 ? idx : 0) * VLB_STRIDE + (f == 2 ? 1 + PJ_DEC_NCNT : 1);
#pragma unroll
        for (int k = 0; k < PJ_DEC_NCNT; k++) excl[k] += wave_sum(use ? lb_load(&src[k]) : 0);
        if (fp < 64) break;
        j -= 64;
    }
    uint64_t *s = st + b * VLB_STRIDE;
    if (l < PJ_DEC_NCNT) {
        uint64_t v = 0;
#pragma unroll
        for (int k = 0; k < PJ_DEC_NCNT; k++) v = k == l ? excl[k] + agg[k] : v;
        lb_store(&s[1 + PJ_DEC_NCNT + l], v);
    }
    __threadfence();
    if (l == 0) lb_store(&s[0], 2);
}

template <bool SLOW>
__device__ __forceinline__ int parse_line(const DecParams &P, uint64_t s, uint32_t n, LineInfo &L) {
    LP<SLOW> lp;
    lp.init(P, s, n);
    return lp.parse(L);
}

template <bool SLOW>
__device__ void write_line(const DecParams &P, uint64_t s, uint32_t n, const LineInfo &L, const uint64_t *pos) {
    const pj_pet_columns &o = P.o;
    LP<SLOW> lp;
    lp.init(P, s, n);
    const uint64_t row = pos[C_PETS];
    const uint64_t nb = pos[C_NAMEB], cb = pos[C_CATB], u0 = pos[C_URLS], ub = pos[C_URLB], g0 = pos[C_TAGS],
                   tb = pos[C_TAGB];
    if (row < o.cap_pets) {
        o.id[row] = L.id;
        o.flags[row] = (uint8_t)((L.has_id ? PJ_PET_HAS_ID : 0) | (L.has_cat ? PJ_PET_HAS_CATEGORY : 0) |
                                 PJ_PET_HAS_NAME | PJ_PET_HAS_PHOTOURLS | (L.has_tags ? PJ_PET_HAS_TAGS : 0));
        o.status[row] = L.status;
        o.cat_id[row] = L.cat_id;
        o.cat_flags[row] = L.cat_flags;
        o.name_off[row + 1] = nb + L.name_len;
        o.cat_name_off[row + 1] = cb + L.cat_len;
        o.photo_off[row + 1] = u0 + L.n_urls;
        o.tag_off[row + 1] = g0 + L.n_tags;
    }
    if (L.name_len && nb + L.name_len <= o.cap_name_bytes) {
        WriteSink ws;
        ws.init(o.name_bytes, nb, P.dummy);
        lp.copy_str(L.name_pos, ws);
        ws.finish();
    }
    if (L.has_cat && L.cat_len && cb + L.cat_len <= o.cap_cat_name_bytes) {
        uint32_t q = lp.last_name_of(L.cat_pos);
        WriteSink ws;
        ws.init(o.cat_name_bytes, cb, P.dummy);
        lp.copy_str(q, ws);
        ws.finish();
    }
    if (L.has_photo && L.n_urls) {
        lp.p = L.photo_pos;
        lp.open_container();
        uint64_t u = u0, b = ub;
        for (;;) {
            lp.skip_ws();
            const uint32_t q = lp.p;
            uint32_t end, dl;
            bool es;
            lp.str_scan(q, &end, &dl, &es);
            if (b + dl <= o.cap_url_bytes && dl) {
                WriteSink ws;
                ws.init(o.url_bytes, b, P.dummy);
                lp.copy_str(q, ws);
                ws.finish();
            }
            b += dl;
            u++;
            if (u <= o.cap_urls) o.url_off[u] = b;
            lp.p = end + 1;
            lp.skip_ws();
            if (lp.peek() == ',') { lp.p++; continue; }
            break;
        }
    }
    if (L.has_tags && L.n_tags) {
        lp.p = L.tags_pos;
        lp.open_container();
        uint64_t g = g0, b = tb;
        for (;;) {
            lp.skip_ws();
            const uint32_t q = lp.p;
            int64_t tid;
            uint8_t tfl;
            uint32_t tl;
            lp.rd_sub(&tid, &tfl, &tl);
            const uint32_t after = lp.p;
            if (g < o.cap_tags) {
                o.tag_id[g] = tid;
                o.tag_flags[g] = tfl;
            }
            if (tl && b + tl <= o.cap_tag_name_bytes) {
                uint32_t nq = lp.last_name_of(q);
                WriteSink ws;
                ws.init(o.tag_name_bytes, b, P.dummy);
                lp.copy_str(nq, ws);
                ws.finish();
            }
            b += tl;
            g++;
            if (g <= o.cap_tags) o.tag_name_off[g] = b;
            lp.p = after;
            lp.skip_ws();
            if (lp.peek() == ',') { lp.p++; continue; }
            break;
        }
    }
}

template <int BT>
__global__ __launch_bounds__(BT) void k_dec_parse(DecParams P) {
    __shared__ uint64_t sh_scan[BT / 64];
    __shared__ uint64_t sh_blk;
    __shared__ uint64_t sh_base[PJ_DEC_NCNT];
    const uint32_t t = threadIdx.x;
    if (t == 0) sh_blk = atomicAdd(&P.tickets[1], 1ull);
    __syncthreads();
    const uint64_t b = sh_blk;
    const uint64_t l = b * BT + t;
    const bool live = l < P.lines;
    LineInfo L;
    int code = 0;
    uint64_t s = 0;
    uint32_t n = 0;
    bool slow = false;
    if (live) {
        s = P.line_start[l];
        const uint64_t e = P.line_start[l + 1] - 1;
        n = (uint32_t)(e - s);
        if (n) {
            for (uint64_t k = s >> 6; k <= (e - 1) >> 6; k++) slow |= P.bad[k] != 0;
        }
        code = slow ? parse_line<true>(P, s, n, L) : parse_line<false>(P, s, n, L);
    }
    uint64_t v[PJ_DEC_NCNT], pre[PJ_DEC_NCNT], agg[PJ_DEC_NCNT];
    const bool ok = live && code == 0;
    v[C_PETS] = ok;
    v[C_NAMEB] = ok ? L.name_len : 0;
    v[C_CATB] = ok && L.has_cat ? L.cat_len : 0;
    v[C_URLS] = ok ? L.n_urls : 0;
    v[C_URLB] = ok ? L.url_bytes : 0;
    v[C_TAGS] = ok ? L.n_tags : 0;
    v[C_TAGB] = ok ? L.tag_bytes : 0;
    v[C_ERRS] = live && code != 0;
#pragma unroll
    for (int k = 0; k < PJ_DEC_NCNT; k++) pre[k] = block_excl_scan<BT>(v[k], sh_scan, &agg[k]);
    if (t < 64) {
        vlb_publish(P.state_parse, b, agg, (int)t);
        uint64_t excl[PJ_DEC_NCNT];
        vlb_resolve(P.state_parse, b, agg, excl);
        if (t < PJ_DEC_NCNT) {
            uint64_t x = 0;
#pragma unroll
            for (int k = 0; k < PJ_DEC_NCNT; k++) x = k == (int)t ? excl[k] : x;
            sh_base[t] = x;
        }
        if (b == gridDim.x - 1 && t < PJ_DEC_NCNT) {
            uint64_t x = 0;
#pragma unroll
            for (int k = 0; k < PJ_DEC_NCNT; k++) x = k == (int)t ? excl[k] + agg[k] : x;
            P.totals[t] = x;
        }
    }
    __syncthreads();
    if (b == 0 && t == 0) {
        const pj_pet_columns &o = P.o;
        o.name_off[0] = 0; o.cat_name_off[0] = 0; o.photo_off[0] = 0; o.tag_off[0] = 0;
        o.url_off[0] = 0; o.tag_name_off[0] = 0;
    }
    if (!live) return;
    if (code) {
        uint64_t e = sh_base[C_ERRS] + pre[C_ERRS];
        if (e < P.err_cap) {
            P.err_line[e] = l;
            P.err_code[e] = (uint8_t)code;
        }
        return;
    }
    uint64_t pos[PJ_DEC_NCNT];
#pragma unroll
    for (int k = 0; k < PJ_DEC_NCNT; k++) pos[k] = sh_base[k] + pre[k];
    if (slow) write_line<true>(P, s, n, L, pos);
    else write_line<false>(P, s, n, L, pos);
}

}  // namespace pj

constexpr int DEC_IDX_BT = 256, DEC_PARSE_BT = 256;

int pj_dec_index_block() { return DEC_IDX_BT; }
int pj_dec_parse_block() { return DEC_PARSE_BT; }

hipError_t pj_launch_dec_index(const DecParams &P, hipStream_t st) {
    uint64_t g = (P.nblk64 + DEC_IDX_BT - 1) / DEC_IDX_BT;
    hipLaunchKernelGGL(pj::k_dec_index<DEC_IDX_BT>, dim3((unsigned)g), dim3(DEC_IDX_BT), 0, st, P);
    return hipGetLastError();
}

hipError_t pj_launch_dec_parse(const DecParams &P, hipStream_t st) {
    uint64_t g = (P.lines + DEC_PARSE_BT - 1) / DEC_PARSE_BT;
    hipLaunchKernelGGL(pj::k_dec_parse<DEC_PARSE_BT>, dim3((unsigned)g), dim3(DEC_PARSE_BT), 0, st, P);
    return hipGetLastError();
}
