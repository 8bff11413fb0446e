// pj_decode.hip — NDJSON -> columnar Pet decoder for gfx950.
//
// k_dec_lines: exact newline masks (SWAR) over 64-byte words, block scans and
//   a decoupled look-back of newline counts -> every line's start.
// k_dec_block: one workgroup per LPB lines, one thread per line.  The lines
//   are tiled into LDS (HBM -> LDS loads); each thread validates and
//   measures its line with the fast path (properties in schema order as
//   straight code; strings scanned 16 bytes at a time with every byte class
//   checked where the walk meets it), recording a tape of what the writer
//   needs; lines the fast path does not recognise go through the general
//   pushdown parser; lines over 1 KiB are read by their whole wave over the
//   tile's quote / backslash bitmaps.  With the tape (the default) the kernel
//   ends with a block scan of 8 counters: per-line offsets inside the block
//   and the block totals go to memory, and
// k_dec_bscan scans the block totals (ticket-ordered workgroups, vector
//   look-back) into each block's first offsets;
// k_dec_write tiles each block again and writes its fast-path lines from
//   their tapes at those offsets, and the error slots;
// k_dec_long writes the lines of the whole wave and of the general parser;
// k_dec_errcode settles the code of lines found invalid from the bitmaps.
// Without the tape, k_dec_block is single-pass: its blocks chain through a
//   vector look-back and a second walk over each line writes it.
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

// bit i set iff bit 7 of byte i of m is set (m holds only bits 7, 15, 23, 31)
__device__ __forceinline__ uint32_t movemask4(uint32_t m) { return (((m >> 7) * 0x00204081u) >> 21) & 0xFu; }

__device__ __forceinline__ uint64_t prefix_xor(uint64_t x) {
    x ^= x << 1; x ^= x << 2; x ^= x << 4; x ^= x << 8; x ^= x << 16; x ^= x << 32;
    return x;
}

// Characters escaped by a backslash in a 64-byte word with backslash mask
// bs, given whether its first byte is escaped (cin); *cout tells the same of
// the next word's first byte.  Backslash runs pair up from their start.
__device__ __forceinline__ uint64_t escaped64(uint64_t bs, uint32_t cin, uint32_t *cout) {
    constexpr uint64_t EVEN = 0x5555555555555555ull;
    bs &= ~(uint64_t)cin;
    const uint64_t follows = (bs << 1) | cin;
    const uint64_t odd_starts = bs & ~EVEN & ~follows;
    uint64_t even_seq;
    *cout = __builtin_add_overflow(odd_starts, bs, &even_seq) ? 1u : 0u;
    return (EVEN ^ (even_seq << 1)) & follows;
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

// Stage 1, k_dec_lines: each thread owns R 64-byte words of its block's
// BT * R, one per round (word r * BT + t), so a wave's loads in a round are
// contiguous; exact newline masks, block scans in word order + decoupled
// look-back of newline counts -> line starts.
template <int BT, int R>
__global__ __launch_bounds__(BT) void k_dec_lines(DecParams P) {
    __shared__ uint32_t sh_scan[R * BT / 64];
    __shared__ uint64_t sh_blk, sh_pre;
    const uint32_t t = threadIdx.x;
    if (t == 0) sh_blk = P.order_by_id ? (uint64_t)blockIdx.x : atomicAdd(&P.tickets[0], 1ull);
    __syncthreads();
    const uint64_t b = sh_blk;
    // word r * BT + t of the block's BT * R words: in every round the lanes
    // of a wave read 64 consecutive words
    const uint64_t wb = b * BT * R;
    uint64_t N[R];
    uint32_t cnt[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const uint64_t wd = wb + (uint64_t)r * BT + t, st = wd * 64;
        uint64_t m = 0;
        if (wd < P.nblk64) {
            if (st + 64 <= P.len) {
                const uint4 *q = reinterpret_cast<const uint4 *>(P.in + st);
                uint32_t w[16];
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const uint4 v = q[k];
                    w[4 * k] = v.x; w[4 * k + 1] = v.y; w[4 * k + 2] = v.z; w[4 * k + 3] = v.w;
                }
#pragma unroll
                for (int k = 0; k < 16; k++) m |= (uint64_t)zero_bytes4(w[k] ^ 0x0A0A0A0Au) << (4 * k);
            } else {
                for (uint32_t j = 0; st + j < P.len; j++) m |= (uint64_t)(P.in[st + j] == '\n') << j;
            }
        }
        N[r] = m;
        cnt[r] = (uint32_t)__builtin_popcountll(m);
    }
    // lines before each word: the rounds in order, threads in order within a
    // round (one scan of the R per-round counts)
    uint32_t ex[R], rt[R];
    block_excl_scan_n<BT, R>(cnt, ex, rt, sh_scan);
    uint64_t pre[R], agg = 0;
#pragma unroll
    for (int r = 0; r < R; r++) {
        pre[r] = agg + ex[r];
        agg += rt[r];
    }
    if (t == 0) lb_publish(P.state_idx, b, agg);
    if (t < 64) {
        const uint64_t e = lb_resolve(P.state_idx, b, agg, P.order_by_id ? P.spin_limit : 0, &P.tickets[0]);
        if (t == 0) sh_pre = e;
    }
    __syncthreads();
    const uint64_t e0 = sh_pre;
#pragma unroll
    for (int r = 0; r < R; r++) {
        const uint64_t wd = wb + (uint64_t)r * BT + t, st = wd * 64;
        uint64_t li = e0 + pre[r];
        for (uint64_t m = N[r]; m; m &= m - 1) {
            li++;
            if (li < P.ls_cap) P.line_start[li] = st + (uint64_t)__builtin_ctzll(m) + 1;
        }
        if (wd == P.nblk64 - 1) {
            const bool open = P.in[P.len - 1] != '\n';  // last line without '\n'
            const uint64_t nl = li + (open ? 1 : 0);
            if (open && nl < P.ls_cap) P.line_start[nl] = P.len + 1;
            *P.n_lines = nl;
        }
    }
    if (b == 0 && t == 0) P.line_start[0] = 0;
}
// =========================================================== array documents
// The frame of one JSON array document: the top-level commas (depth 1,
// outside strings) and the closing ']' cut it into elements, which the line
// stages then read exactly as NDJSON lines.  The rule is the sequential one
// of the CPU checker: a backslash escapes the next byte (in strings or
// not), an unescaped quote opens or closes a string, '[' '{' ']' '}' outside
// strings move the depth.  A 64-byte word is summarised, for each of the
// four states it may be entered in (inside a string or not, first byte
// escaped or not), by the state it leaves in, its depth change and the
// lowest depth reached inside it; summaries compose associatively, so
// blocks of words are summarised, scanned by one workgroup, and each word
// then learns the state and depth it is entered with.
using ::FS;
__device__ __forceinline__ FS fs_id() {
    FS f;
    f.out = 0xE4u;      // s -> s
#pragma unroll
    for (int k = 0; k < 4; k++) f.d[k] = 0;
    return f;
}
__device__ __forceinline__ int32_t pick4(const int32_t *a, uint32_t k) {
    return k == 0 ? a[0] : k == 1 ? a[1] : k == 2 ? a[2] : a[3];
}
// f, then g
__device__ __forceinline__ FS fs_cat(const FS &f, const FS &g) {
    FS r;
    r.out = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const uint32_t s1 = (f.out >> (2 * k)) & 3;
        r.out |= ((g.out >> (2 * s1)) & 3) << (2 * k);
        r.d[k] = f.d[k] + pick4(g.d, s1);
    }
    return r;
}
// Byte-class masks of the 64-byte word at g (avail bytes of it are input).
struct AMasks {
    uint64_t q, b, o, c, m, nw;     // '"', '\\', '[' '{', ']' '}', ',', not whitespace
};
__device__ __forceinline__ AMasks arr_masks(const uint8_t *g, uint64_t avail) {
    uint32_t w[16];
    if (avail >= 64) {
        const uint4 *q4 = reinterpret_cast<const uint4 *>(g);
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint4 v = q4[k];
            w[4 * k] = v.x; w[4 * k + 1] = v.y; w[4 * k + 2] = v.z; w[4 * k + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int k = 0; k < 16; k++) w[k] = 0;
        for (uint32_t j = 0; j < avail; j++) w[j >> 2] |= (uint32_t)g[j] << (8 * (j & 3));
    }
    AMasks M{0, 0, 0, 0, 0, 0};
    uint64_t ws = 0;
#pragma unroll
    for (int k = 0; k < 16; k++) {
        const uint32_t x = w[k], lx = x | 0x20202020u;
        M.q |= (uint64_t)zero_bytes4(x ^ 0x22222222u) << (4 * k);
        M.b |= (uint64_t)zero_bytes4(x ^ 0x5C5C5C5Cu) << (4 * k);
        M.o |= (uint64_t)zero_bytes4(lx ^ 0x7B7B7B7Bu) << (4 * k);      // '[' or '{'
        M.c |= (uint64_t)zero_bytes4(lx ^ 0x7D7D7D7Du) << (4 * k);      // ']' or '}'
        M.m |= (uint64_t)zero_bytes4(x ^ 0x2C2C2C2Cu) << (4 * k);
        ws |= (uint64_t)(zero_bytes4(x ^ 0x20202020u) | zero_bytes4(x ^ 0x09090909u) | zero_bytes4(x ^ 0x0D0D0D0Du) |
                         zero_bytes4(x ^ 0x0A0A0A0Au)) << (4 * k);
    }
    M.nw = ~ws & (avail >= 64 ? ~0ull : ((1ull << avail) - 1));
    return M;
}
// The word's structure when entered in state s (bit 0 in a string, bit 1
// first byte escaped): strings, outside opens / closes / commas, exit state.
struct AWord {
    uint64_t od, cd, md;
    uint32_t out;
};
__device__ __forceinline__ AWord arr_word(const AMasks &M, uint32_t s) {
    uint32_t cout;
    const uint64_t E = escaped64(M.b, s >> 1, &cout);
    const uint64_t S = prefix_xor(M.q & ~E) ^ ((s & 1) ? ~0ull : 0ull);
    AWord a;
    a.od = M.o & ~S & ~E;
    a.cd = M.c & ~S & ~E;
    a.md = M.m & ~S & ~E;
    a.out = (uint32_t)(S >> 63) | (cout << 1);
    return a;
}
// depth change from the word's start through byte i
__device__ __forceinline__ int32_t depth_at(const AWord &a, uint32_t i) {
    const uint64_t le = i == 63 ? ~0ull : ((2ull << i) - 1);
    return __builtin_popcountll(a.od & le) - __builtin_popcountll(a.cd & le);
}
__device__ __forceinline__ FS word_fs(const AMasks &M) {
    FS f;
    f.out = 0;
#pragma unroll
    for (int s = 0; s < 4; s++) {
        const AWord a = arr_word(M, (uint32_t)s);
        f.d[s] = __builtin_popcountll(a.od) - __builtin_popcountll(a.cd);
        f.out |= a.out << (2 * s);
    }
    return f;
}
// Inclusive in-order scan of one FS per thread (all BT threads).
template <int BT>
__device__ __forceinline__ FS block_fs_scan(FS v, FS *sh) {
    const uint32_t t = threadIdx.x;
    sh[t] = v;
    __syncthreads();
#pragma unroll 1
    for (uint32_t d = 1; d < BT; d <<= 1) {
        FS o = fs_id();
        if (t >= d) o = sh[t - d];
        __syncthreads();
        if (t >= d) {
            v = fs_cat(o, v);
            sh[t] = v;
        }
        __syncthreads();
    }
    return v;
}
// Summary of each block of BT * R words (thread t: words t R .. t R + R - 1).
template <int BT, int R>
__global__ __launch_bounds__(BT) void k_arr_sum(DecParams P) {
    __shared__ FS sh[BT];
    const uint32_t t = threadIdx.x;
    const uint64_t b = blockIdx.x, w0 = (b * BT + t) * R;
    FS acc = fs_id();
    for (int r = 0; r < R; r++) {
        const uint64_t w = w0 + r;
        if (w < P.nblk64) acc = fs_cat(acc, word_fs(arr_masks(P.in + 64 * w, P.len - 64 * w)));
    }
    acc = block_fs_scan<BT>(acc, sh);
    if (t == BT - 1) P.arr_bsum[b] = acc;
    // the thread's exclusive prefix in the block, for k_arr_frame
    P.arr_tsum[b * BT + t] = t ? sh[t - 1] : fs_id();
}
// One workgroup: the state and depth each block is entered with, the
// document being entered outside strings at depth 0.
template <int BT>
__global__ __launch_bounds__(BT) void k_arr_scan(DecParams P, uint64_t nb) {
    __shared__ FS sh[BT];
    const uint32_t t = threadIdx.x;
    const uint64_t per = (nb + BT - 1) / BT, b0 = min(nb, t * per), b1 = min(nb, b0 + per);
    FS acc = fs_id();
    for (uint64_t b = b0; b < b1; b++) acc = fs_cat(acc, P.arr_bsum[b]);
    const FS inc = block_fs_scan<BT>(acc, sh);
    FS cur = fs_id();
    if (t) cur = sh[t - 1];
    (void)inc;
    for (uint64_t b = b0; b < b1; b++) {
        P.arr_bpre[b] = (uint64_t)(cur.out & 3) | ((uint64_t)(uint32_t)cur.d[0] << 32);
        cur = fs_cat(cur, P.arr_bsum[b]);
    }
}
// The frame: per word, entered with its true state and depth, the commas at
// depth 1 (counted, then written as element starts after a block scan and a
// look-back of the counts), the first byte whose close brings the depth to
// 0, and the first and last bytes that are not whitespace (one atomic per
// block each).
template <int BT, int R>
__global__ __launch_bounds__(BT) void k_arr_frame(DecParams P) {
    __shared__ uint64_t sh_scan[BT / 64];
    __shared__ uint64_t sh_blk, sh_pre, sh_mn[3];
    const uint32_t t = threadIdx.x;
    if (t == 0) {
        sh_blk = atomicAdd((unsigned long long *)&P.arr[5], 1ull);
        sh_mn[0] = ~0ull; sh_mn[1] = 0; sh_mn[2] = ~0ull;
    }
    __syncthreads();
    const uint64_t b = sh_blk, w0 = (b * BT + t) * R;
    // the thread's entry state: the block's, then its predecessors' words in
    // the block (their summary, from k_arr_sum)
    const FS ex = P.arr_tsum[b * BT + t];
    const uint64_t bp = P.arr_bpre[b];
    const uint32_t sb = (uint32_t)bp & 3;
    uint32_t st0 = (ex.out >> (2 * sb)) & 3;
    int32_t dep0 = (int32_t)(uint32_t)(bp >> 32) + pick4(ex.d, sb);
    // pass 1: the separators (a mask per word); first / last non-whitespace;
    // the close
    uint64_t cnt = 0, first = ~0ull, lastp1 = 0, close = ~0ull;
    uint64_t sep[R];
#pragma unroll
    for (int r = 0; r < R; r++) sep[r] = 0;
    {
        uint32_t st = st0;
        int32_t dep = dep0;
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint64_t w = w0 + r;
            if (w >= P.nblk64) break;
            const AMasks M = arr_masks(P.in + 64 * w, P.len - 64 * w);
            const AWord a = arr_word(M, st);
            for (uint64_t m = a.md; m; m &= m - 1) {
                const uint32_t i = (uint32_t)__builtin_ctzll(m);
                if (dep + depth_at(a, i) == 1) sep[r] |= 1ull << i;
            }
            cnt += (uint64_t)__builtin_popcountll(sep[r]);
            if (close == ~0ull)
                for (uint64_t m = a.cd; m; m &= m - 1) {
                    const uint32_t i = (uint32_t)__builtin_ctzll(m);
                    if (dep + depth_at(a, i) == 0) {
                        close = 64 * w + i;
                        break;
                    }
                }
            if (M.nw) {
                if (first == ~0ull) first = 64 * w + (uint64_t)__builtin_ctzll(M.nw);
                lastp1 = 64 * w + 64 - (uint64_t)__builtin_clzll(M.nw);
            }
            dep += __builtin_popcountll(a.od) - __builtin_popcountll(a.cd);
            st = a.out;
        }
    }
    if (first != ~0ull) atomicMin((unsigned long long *)&sh_mn[0], (unsigned long long)first);
    if (lastp1) atomicMax((unsigned long long *)&sh_mn[1], (unsigned long long)lastp1);
    if (close != ~0ull) atomicMin((unsigned long long *)&sh_mn[2], (unsigned long long)close);
    uint64_t tot;
    const uint64_t ex_cnt = block_excl_scan<BT>(cnt, sh_scan, &tot);
    if (t == 0) {
        lb_publish(P.state_idx, b, tot);
        if (sh_mn[0] != ~0ull) atomicMin((unsigned long long *)&P.arr[0], (unsigned long long)sh_mn[0]);
        if (sh_mn[1]) atomicMax((unsigned long long *)&P.arr[1], (unsigned long long)sh_mn[1]);
        if (sh_mn[2] != ~0ull) atomicMin((unsigned long long *)&P.arr[2], (unsigned long long)sh_mn[2]);
    }
    if (t < 64) {
        const uint64_t e = lb_resolve(P.state_idx, b, tot);
        if (t == 0) {
            sh_pre = e;
            if ((b + 1) * BT * R >= P.nblk64) P.arr[3] = e + tot;
        }
    }
    __syncthreads();
    // pass 2: element k + 1 starts after the k-th separator
    uint64_t idx = sh_pre + ex_cnt;
#pragma unroll
    for (int r = 0; r < R; r++)
        for (uint64_t m = sep[r]; m; m &= m - 1) {
            if (1 + idx < P.ls_cap) P.line_start[1 + idx] = 64 * (w0 + r) + (uint64_t)__builtin_ctzll(m) + 1;
            idx++;
        }
}
// The frame's verdict (one thread): the first non-whitespace byte is '[',
// the close is a ']' after it and nothing but whitespace follows.  Then
// element 0 starts after the '[' and the last one ends at the ']'.
__global__ void k_arr_fin(DecParams P) {
    const uint64_t first = P.arr[0], lastp1 = P.arr[1], close = P.arr[2], nsep = P.arr[3];
    const bool ok = first != ~0ull && P.in[first] == '[' && close != ~0ull && close > first && P.in[close] == ']' &&
                    lastp1 == close + 1;
    P.arr[4] = ok ? 1 : 0;
    if (!ok) {
        *P.n_lines = 0;
        return;
    }
    if (nsep + 1 < P.ls_cap) {
        P.line_start[0] = first + 1;
        P.line_start[nsep + 1] = close + 1;
    }
    *P.n_lines = nsep + 1;
}

// =========================================================== stage 2
// Property keys, container contexts and parser states.
enum { K_UNKNOWN = 0, K_ID, K_CATEGORY, K_NAME, K_PHOTOURLS, K_TAGS, K_STATUS };
enum { X_NONE = 0, X_PET, X_CAT, X_URLS, X_TAGS, X_TAG, X_SKIP };
enum { S_VALUE = 0, S_KEY_OR_CLOSE, S_KEY, S_COLON, S_ELEM_OR_CLOSE, S_AFTER, S_DONE };
// what a string value is read for
enum { U_NONE = 0, U_KEY, U_NAME, U_SUBNAME, U_URL, U_STATUS, U_SKIP };

// Per-line results of the validating pass (last occurrence of each
// property), reused by the materialising pass.
struct LineInfo {
    int64_t id, cat_id;
    uint32_t name_pos, name_len, cat_pos, cat_len, photo_pos, n_urls, url_bytes, tags_pos, n_tags, tag_bytes;
    uint8_t has_id, has_cat, has_name, has_photo, has_tags, cat_flags, status, name_esc;
};

__device__ __forceinline__ int hexval(int c) {
    const uint32_t d = (uint32_t)c - '0', a = ((uint32_t)c | 0x20) - 'a';  // 'A'-'F' fold onto 'a'-'f'
    return d < 10 ? (int)d : a < 6 ? (int)a + 10 : -1;
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

// Escape sequence at line offset q (a backslash).  Rare, so out of line and
// reading bytes straight from memory.
struct Esc {
    int err;
    uint32_t adv;     // bytes consumed
    uint32_t out;     // decoded UTF-8 bytes, little endian
    int k;            // how many
};
__device__ __noinline__ Esc escape_at(const uint8_t *s, uint32_t n, uint32_t q) {
    Esc r{PJ_REC_STRING, 2, 0, 1};
    if (q + 1 >= n) return r;
    switch (s[q + 1]) {
    case '"': r.out = '"'; break;
    case '\\': r.out = '\\'; break;
    case '/': r.out = '/'; break;
    case 'b': r.out = 8; break;
    case 'f': r.out = 12; break;
    case 'n': r.out = 10; break;
    case 'r': r.out = 13; break;
    case 't': r.out = 9; break;
    case 'u': {
        if (q + 6 > n) return r;
        uint32_t cu = 0;
        for (int j = 0; j < 4; j++) {
            int h = hexval(s[q + 2 + j]);
            if (h < 0) return r;
            cu = cu * 16 + (uint32_t)h;
        }
        r.adv = 6;
        if (cu >= 0xDC00 && cu <= 0xDFFF) return r;                  // lone low surrogate
        if (cu >= 0xD800 && cu <= 0xDBFF) {                           // needs \uDC00-\uDFFF next
            if (q + 12 > n || s[q + 6] != '\\' || s[q + 7] != 'u') return r;
            uint32_t lo = 0;
            for (int j = 0; j < 4; j++) {
                int h = hexval(s[q + 8 + j]);
                if (h < 0) return r;
                lo = lo * 16 + (uint32_t)h;
            }
            if (lo < 0xDC00 || lo > 0xDFFF) return r;
            cu = 0x10000 + ((cu - 0xD800) << 10) + (lo - 0xDC00);
            r.adv = 12;
        }
        r.out = utf8_pack(cu, &r.k);
        break;
    }
    default: return r;
    }
    r.err = 0;
    return r;
}

struct Str {
    int err;
    uint32_t end;     // closing quote
    uint32_t dlen;    // decoded length
    bool esc;         // holds escapes
};
// Byte-by-byte string scan with full validation (lines whose blocks stage 1
// flagged): raw control characters, jackson's UTF-8 lead / continuation rules.
__device__ __noinline__ Str scan_slow(const uint8_t *s, uint32_t n, uint32_t q) {
    Str r{PJ_REC_STRING, 0, 0, false};
    uint32_t pos = q + 1, d = 0;
    for (;;) {
        if (pos >= n) return r;
        uint32_t c = s[pos];
        if (c == '"') break;
        if (c == '\\') {
            Esc e = escape_at(s, n, pos);
            if (e.err) return r;
            d += (uint32_t)e.k;
            pos += e.adv;
            r.esc = true;
            continue;
        }
        if (c < 0x20) return r;
        uint32_t extra;
        if (c < 0x80) extra = 0;
        else if (c >= 0xC0 && c <= 0xDF) extra = 1;
        else if (c >= 0xE0 && c <= 0xEF) extra = 2;
        else if (c >= 0xF0 && c <= 0xF7) extra = 3;
        else return r;
        if (pos + 1 + extra > n) return r;
        for (uint32_t j = 1; j <= extra; j++)
            if ((s[pos + j] & 0xC0) != 0x80) return r;
        d += 1 + extra;
        pos += 1 + extra;
    }
    r.err = 0;
    r.end = pos;
    r.dlen = d;
    return r;
}

// First 16 decoded bytes of a validated string with escapes.
__device__ __noinline__ uint2 small_decode_esc(const uint8_t *s, uint32_t q, uint32_t end, uint32_t n, uint64_t *hi) {
    uint64_t v[2] = {0, 0};
    uint32_t pos = q + 1, o = 0;
    while (pos < end && o < 16) {
        uint32_t bytes = s[pos], adv = 1;
        int k = 1;
        if (bytes == '\\') {
            Esc e = escape_at(s, n, pos);
            bytes = e.out;
            adv = e.adv;
            k = e.k;
        }
        for (int j = 0; j < k && o < 16; j++, o++) v[o >> 3] |= (uint64_t)((bytes >> (8 * j)) & 0xFF) << (8 * (o & 7));
        pos += adv;
    }
    *hi = v[1];
    return make_uint2((uint32_t)v[0], (uint32_t)(v[0] >> 32));
}

// Is the innermost container open at nesting level d (1-based), seen at
// cursor p, an object?  Used beyond the 64 levels the register stack holds.
__device__ __noinline__ bool opener_at(const uint8_t *s, uint32_t p, int d) {
    int lvl = 0;
    bool kind = false, instr = false;
    for (uint32_t q = 0; q < p; q++) {
        uint32_t c = s[q];
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

// A value every lane holds alike, moved to scalar registers.
__device__ __forceinline__ uint64_t uniform_u64(uint64_t x) {
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)x), hi = __builtin_amdgcn_readfirstlane((uint32_t)(x >> 32));
    return (uint64_t)hi << 32 | lo;
}

// Where a line's bytes live: the LDS tile of its workgroup (with the tile's
// specials bitmap) or global memory (no bitmap: the byte-by-byte path).
struct Src {
    const uint8_t *in;
    uint64_t len;
    const uint64_t *special;
};

// 16-byte window over a line for the skeleton bytes.
struct Win {
    const uint8_t *in;
    uint64_t len, s0;
    uint64_t wlo, whi;
    uint32_t wp;
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
    __device__ __forceinline__ int at(uint32_t q) {
        if (q - wp >= 16) refill(q);
        const uint32_t d = q - wp;
        return (int)(((d < 8 ? wlo : whi) >> (8 * (d & 7))) & 0xFF);
    }
};

// One pass over one line.  write == false validates and measures (returns
// the PJ_REC_* code and fills L); write == true materialises a line the
// first pass found valid, at the offsets pos[].  Strings are skipped through
// the specials bitmap unless `slow`.  One string-scan site, one copy site
// and one scalar site keep the whole machine in registers.
__device__ __forceinline__ int run_line(const DecParams &P, const Src &S, uint64_t s0, uint32_t n, bool slow,
                                        bool write, LineInfo &L, const uint64_t *pos) {
    const uint8_t *s = S.in + s0;
    Win W{S.in, S.len, s0, 0, 0, 0xFFFFFF00u};
    uint32_t p = 0;
#define PEEK() (p < n ? W.at(p) : -1)
#define SKIP_WS()                                                \
    while (p < n) {                                              \
        const int c_ = W.at(p);                                  \
        if (c_ != ' ' && c_ != '\t' && c_ != '\r' && c_ != '\n') break; \
        p++;                                                     \
    }
    if (!write) {
        L.has_id = L.has_cat = L.has_name = L.has_photo = L.has_tags = 0;
        L.id = L.cat_id = 0;
        L.cat_flags = 0;
        L.status = PJ_STATUS_NULL;
        L.name_len = L.cat_len = L.n_urls = L.url_bytes = L.n_tags = L.tag_bytes = 0;
        L.name_pos = L.cat_pos = L.photo_pos = L.tags_pos = 0;
        L.name_esc = 0;
    }
    SKIP_WS();
    if (p >= n) return PJ_REC_EMPTY;
    int depth = 0;
    uint64_t stk = 0;           // bit d-1: container at depth d is an object
    uint32_t sem = 0;           // 4 bits per depth 1..3: X_* context
    int state = S_VALUE, k1 = K_UNKNOWN, k2 = K_UNKNOWN;
    int64_t sub_id = 0;         // Category / Tag being read
    uint32_t sub_fl = 0, sub_len = 0, sub_q = 0;
    bool sub_esc = false;
    uint32_t cat_q = 0;         // '{' of the category being read
    bool last_urls = false, last_tags = false;
    const pj_pet_columns &o = P.o;
    uint64_t u_idx = write ? pos[C_URLS] : 0, u_b = write ? pos[C_URLB] : 0;
    uint64_t g_idx = write ? pos[C_TAGS] : 0, g_b = write ? pos[C_TAGB] : 0;

    for (;;) {
        SKIP_WS();
        int c = PEEK();
        if (state == S_DONE) return c < 0 ? 0 : PJ_REC_SYNTAX;
        const int ctx = depth == 0 ? X_NONE : depth <= 3 ? (int)((sem >> (4 * (depth - 1))) & 15) : X_SKIP;
        // ---- decide what this token is for
        int use = U_NONE;          // string use
        int push = X_NONE;         // container to open
        bool close = false, scalar = false;
        // value rules
        bool v_any = false, v_null = false, v_long = false;
        int v_obj = X_NONE, v_arr = X_NONE, v_str = U_NONE;
        switch (state) {
        case S_KEY_OR_CLOSE:
            if (c == '}') { close = true; break; }
            [[fallthrough]];
        case S_KEY:
            if (c != '"') return PJ_REC_SYNTAX;
            use = U_KEY;
            break;
        case S_COLON:
            if (c != ':') return PJ_REC_SYNTAX;
            p++;
            SKIP_WS();
            if (p >= n) return PJ_REC_SYNTAX;
            state = S_VALUE;
            continue;
        case S_ELEM_OR_CLOSE:
            if (c == ']') { close = true; break; }
            [[fallthrough]];
        case S_VALUE:
            if (c < 0) return PJ_REC_SYNTAX;
            if (ctx == X_NONE) v_obj = X_PET;
            else if (ctx == X_PET) {
                switch (k1) {
                case K_ID: v_long = v_null = true; break;
                case K_CATEGORY: v_obj = X_CAT; v_null = true; break;
                case K_NAME: v_str = U_NAME; v_null = true; break;
                case K_PHOTOURLS: v_arr = X_URLS; v_null = true; break;
                case K_TAGS: v_arr = X_TAGS; v_null = true; break;
                case K_STATUS: v_str = U_STATUS; v_null = true; break;
                default: v_any = true;
                }
            } else if (ctx == X_CAT || ctx == X_TAG) {
                if (k2 == K_ID) v_long = v_null = true;
                else if (k2 == K_NAME) { v_str = U_SUBNAME; v_null = true; }
                else v_any = true;
            } else if (ctx == X_URLS) v_str = U_URL;
            else if (ctx == X_TAGS) v_obj = X_TAG;
            else v_any = true;
            if (c == '{') {
                if (v_any) push = X_SKIP;
                else if (v_obj) push = v_obj;
                else return PJ_REC_TYPE;
            } else if (c == '[') {
                if (v_any) push = X_SKIP;
                else if (v_arr) push = v_arr;
                else return PJ_REC_TYPE;
            } else if (c == '"') {
                if (v_any) use = U_SKIP;
                else if (v_str) use = v_str;
                else return PJ_REC_TYPE;
            } else scalar = true;
            break;
        case S_AFTER: {
            const bool obj = depth <= 64 ? ((stk >> (depth - 1)) & 1) : opener_at(s, p, depth);
            if (c == ',') {
                p++;
                state = obj ? S_KEY : S_VALUE;
                continue;
            }
            if (c == (obj ? '}' : ']')) { close = true; break; }
            return PJ_REC_SYNTAX;
        }
        }
        // ---- strings (the one scan site)
        if (use) {
            Str r;
            if (slow) r = scan_slow(s, n, p);
            else {
                r.err = 0;
                r.esc = false;
                uint32_t q = p + 1, d = 0;
                for (;;) {
                    // next unescaped quote or backslash at or after q
                    const uint64_t a = s0 + q, lim = s0 + n;
                    uint32_t sp = n;
                    if (a < lim) {
                        uint64_t wi = a >> 6;
                        uint64_t m = S.special[wi] & (~0ull << (a & 63));
                        while (!m && (wi + 1) * 64 < lim) m = S.special[++wi];
                        if (m) {
                            const uint64_t at = wi * 64 + (uint64_t)__builtin_ctzll(m);
                            if (at < lim) sp = (uint32_t)(at - s0);
                        }
                    }
                    if (sp >= n) { r.err = PJ_REC_STRING; break; }
                    d += sp - q;
                    if (s[sp] == '"') { r.end = sp; break; }
                    Esc e = escape_at(s, n, sp);
                    if (e.err) { r.err = e.err; break; }
                    d += (uint32_t)e.k;
                    q = sp + e.adv;
                    r.esc = true;
                }
                r.dlen = d;
            }
            if (r.err) return r.err;
            const uint32_t q0 = p;
            p = r.end + 1;
            uint64_t lo = 0, hi = 0;
            if ((use == U_KEY || use == U_STATUS) && r.dlen <= 9) {
                if (!r.esc) {
                    // raw bytes of the (short) string, read in two safe halves
                    uint32_t L1 = r.dlen < 8 ? r.dlen : 8;
                    if (L1) lo = L1 == 8 ? ldu64(s + q0 + 1) : ld_tail(s + q0 + 1, (int)L1);
                    if (r.dlen > 8) hi = ld_tail(s + q0 + 9, (int)(r.dlen - 8));
                } else {
                    uint2 l2 = small_decode_esc(s, q0, r.end, n, &hi);
                    lo = (uint64_t)l2.x | ((uint64_t)l2.y << 32);
                }
            }
            switch (use) {
            case U_KEY: {
                int kid = K_UNKNOWN;
                const uint32_t dl = r.dlen;
                if (dl == 2 && lo == 0x6469ull) kid = K_ID;                                        // id
                else if (dl == 8 && lo == 0x79726F6765746163ull) kid = K_CATEGORY;                 // category
                else if (dl == 4 && lo == 0x656D616Eull) kid = K_NAME;                             // name
                else if (dl == 9 && lo == 0x6C72556F746F6870ull && hi == 0x73ull) kid = K_PHOTOURLS;  // photoUrls
                else if (dl == 4 && lo == 0x73676174ull) kid = K_TAGS;                             // tags
                else if (dl == 6 && lo == 0x737574617473ull) kid = K_STATUS;                       // status
                if (ctx == X_PET) k1 = kid;
                else k2 = kid;
                state = S_COLON;
                continue;
            }
            case U_NAME:
                if (!write) {
                    L.has_name = 1;
                    L.name_pos = q0;
                    L.name_len = r.dlen;
                    L.name_esc = r.esc;
                }
                break;
            case U_SUBNAME:
                sub_fl |= PJ_SUB_HAS_NAME;
                sub_len = r.dlen;
                sub_q = q0;
                sub_esc = r.esc;
                break;
            case U_URL:
                if (!write) {
                    L.n_urls++;
                    L.url_bytes += r.dlen;
                }
                break;
            case U_STATUS: {
                uint8_t st;
                if (r.dlen == 9 && lo == 0x6C62616C69617661ull && hi == 0x65ull) st = PJ_STATUS_AVAILABLE;
                else if (r.dlen == 7 && lo == 0x676E69646E6570ull) st = PJ_STATUS_PENDING;
                else if (r.dlen == 4 && lo == 0x646C6F73ull) st = PJ_STATUS_SOLD;
                else return PJ_REC_BAD_STATUS;   // the enum's @JsonCreator rejects it
                if (!write) L.status = st;
                break;
            }
            default: break;
            }
            // the one copy site: urls are copied as they are met
            if (write && use == U_URL && last_urls) {
                if (r.dlen && u_b + r.dlen <= o.cap_url_bytes) {
                    WriteSink ws;
                    ws.init(o.url_bytes, u_b, P.dummy);
                    if (!r.esc) {
                        const uint8_t *src = s + q0 + 1;
                        uint32_t k = 0;
                        for (; k + 8 <= r.dlen; k += 8) ws.put8(ldu64(src + k), 8);
                        if (k < r.dlen) ws.put8(ld_tail(src + k, (int)(r.dlen - k)), (int)(r.dlen - k));
                    } else {
                        for (uint32_t q = q0 + 1; q < r.end;) {
                            uint32_t c2 = s[q];
                            if (c2 == '\\') {
                                Esc e = escape_at(s, n, q);
                                ws.put(e.out, e.k);
                                q += e.adv;
                            } else {
                                ws.put_byte(c2);
                                q++;
                            }
                        }
                    }
                    ws.finish();
                }
                u_b += r.dlen;
                u_idx++;
                if (u_idx <= o.cap_urls) o.url_off[u_idx] = u_b;
            }
            state = S_AFTER;
            continue;
        }
        // ---- scalars (the one scalar site)
        if (scalar) {
            const uint32_t t0 = p;
            int kind = -1;       // 0 null, 1 true, 2 false, 3 int, 4 real
            if (c == '-' || (c >= '0' && c <= '9')) {
                uint32_t q = p;
                bool real = false;
                if (W.at(q) == '-') q++;
                if (q >= n) return PJ_REC_SYNTAX;
                int d = W.at(q);
                if (d == '0') {
                    q++;
                    if (q < n && W.at(q) >= '0' && W.at(q) <= '9') return PJ_REC_SYNTAX;   // leading zero
                } else if (d >= '1' && d <= '9') {
                    while (q < n && W.at(q) >= '0' && W.at(q) <= '9') q++;
                } else return PJ_REC_SYNTAX;
                if (q < n && W.at(q) == '.') {
                    q++;
                    real = true;
                    if (q >= n || W.at(q) < '0' || W.at(q) > '9') return PJ_REC_SYNTAX;
                    while (q < n && W.at(q) >= '0' && W.at(q) <= '9') q++;
                }
                if (q < n && (W.at(q) == 'e' || W.at(q) == 'E')) {
                    q++;
                    real = true;
                    if (q < n && (W.at(q) == '+' || W.at(q) == '-')) q++;
                    if (q >= n || W.at(q) < '0' || W.at(q) > '9') return PJ_REC_SYNTAX;
                    while (q < n && W.at(q) >= '0' && W.at(q) <= '9') q++;
                }
                p = q;
                kind = real ? 4 : 3;
            } else {
                uint32_t Ln;
                uint64_t want;
                if (c == 'n') { Ln = 4; want = 0x6C6C756Eull; kind = 0; }
                else if (c == 't') { Ln = 4; want = 0x65757274ull; kind = 1; }
                else if (c == 'f') { Ln = 5; want = 0x65736C6166ull; kind = 2; }
                else return PJ_REC_SYNTAX;
                if (p + Ln > n) return PJ_REC_SYNTAX;
                for (uint32_t j = 0; j < Ln; j++)
                    if ((uint64_t)W.at(p + j) != ((want >> (8 * j)) & 0xFF)) return PJ_REC_SYNTAX;
                if (p + Ln < n && is_ident(W.at(p + Ln))) return PJ_REC_SYNTAX;
                p += Ln;
            }
            if (!v_any) {
                if (kind == 0 && v_null) {
                    // null: the property is absent
                    if (ctx == X_PET) {
                        if (!write) {
                            if (k1 == K_ID) { L.has_id = 0; L.id = 0; }
                            // a later null also forgets where an earlier value
                            // was, so the writing pass copies nothing of it
                            else if (k1 == K_CATEGORY) { L.has_cat = 0; L.cat_id = 0; L.cat_flags = 0; L.cat_len = 0; L.cat_pos = 0; }
                            else if (k1 == K_NAME) { L.has_name = 0; L.name_len = 0; }
                            else if (k1 == K_PHOTOURLS) { L.has_photo = 0; L.n_urls = 0; L.url_bytes = 0; L.photo_pos = 0; }
                            else if (k1 == K_TAGS) { L.has_tags = 0; L.n_tags = 0; L.tag_bytes = 0; L.tags_pos = 0; }
                            else if (k1 == K_STATUS) L.status = PJ_STATUS_NULL;
                        }
                    } else if (k2 == K_ID) { sub_fl &= ~PJ_SUB_HAS_ID; sub_id = 0; }
                    else { sub_fl &= ~PJ_SUB_HAS_NAME; sub_len = 0; }
                } else if (v_long && kind == 4) return PJ_REC_NUMBER;
                else if (v_long && kind == 3) {
                    const bool neg = W.at(t0) == '-';
                    const uint64_t lim = neg ? (1ull << 63) : ((1ull << 63) - 1);
                    uint64_t acc = 0;
                    for (uint32_t q = t0 + (neg ? 1 : 0); q < p; q++) {
                        const uint64_t dg = (uint64_t)(W.at(q) - '0');
                        if (acc > (lim - dg) / 10) return PJ_REC_NUMBER;
                        acc = acc * 10 + dg;
                    }
                    const int64_t v = neg ? (int64_t)(0ull - acc) : (int64_t)acc;
                    if (ctx == X_PET) {
                        if (!write) { L.has_id = 1; L.id = v; }
                    } else { sub_fl |= PJ_SUB_HAS_ID; sub_id = v; }
                } else return PJ_REC_TYPE;
            }
            state = S_AFTER;
            continue;
        }
        // ---- open a container
        if (push) {
            if (++depth > PJ_MAX_DEPTH) return PJ_REC_DEPTH;
            const bool obj = c == '{';
            if (depth <= 64) stk = obj ? (stk | (1ull << (depth - 1))) : (stk & ~(1ull << (depth - 1)));
            if (depth <= 3) sem = (sem & ~(15u << (4 * (depth - 1)))) | ((uint32_t)push << (4 * (depth - 1)));
            if (push == X_CAT) {
                cat_q = p;
                if (!write) { L.has_cat = 1; L.cat_pos = p; }
                sub_id = 0; sub_fl = 0; sub_len = 0; sub_q = 0; sub_esc = false;
            } else if (push == X_TAG) {
                sub_id = 0; sub_fl = 0; sub_len = 0; sub_q = 0; sub_esc = false;
            } else if (push == X_URLS) {
                if (!write) { L.has_photo = 1; L.photo_pos = p; L.n_urls = 0; L.url_bytes = 0; }
                else last_urls = p == L.photo_pos;
            } else if (push == X_TAGS) {
                if (!write) { L.has_tags = 1; L.tags_pos = p; L.n_tags = 0; L.tag_bytes = 0; }
                else last_tags = p == L.tags_pos;
            }
            p++;
            state = obj ? S_KEY_OR_CLOSE : S_ELEM_OR_CLOSE;
            continue;
        }
        // ---- close a container
        if (close) {
            p++;
            // the one sub-string copy site: category / tag names and the pet name
            uint32_t cq = 0, clen = 0;
            bool cesc = false;
            uint8_t *cdst = nullptr;
            uint64_t coff = 0, ccap = 0;
            if (ctx == X_CAT) {
                if (!write) {
                    L.cat_id = sub_id;
                    L.cat_flags = (uint8_t)sub_fl;
                    L.cat_len = (sub_fl & PJ_SUB_HAS_NAME) ? sub_len : 0;
                } else if (cat_q == L.cat_pos && (sub_fl & PJ_SUB_HAS_NAME)) {
                    cq = sub_q; clen = sub_len; cesc = sub_esc;
                    cdst = o.cat_name_bytes; coff = pos[C_CATB]; ccap = o.cap_cat_name_bytes;
                }
            } else if (ctx == X_TAG) {
                const uint32_t tl = (sub_fl & PJ_SUB_HAS_NAME) ? sub_len : 0;
                if (!write) {
                    L.n_tags++;
                    L.tag_bytes += tl;
                } else if (last_tags) {
                    if (g_idx < o.cap_tags) {
                        o.tag_id[g_idx] = sub_id;
                        o.tag_flags[g_idx] = (uint8_t)sub_fl;
                    }
                    if (tl) { cq = sub_q; clen = tl; cesc = sub_esc; cdst = o.tag_name_bytes; coff = g_b; ccap = o.cap_tag_name_bytes; }
                    g_b += tl;
                    g_idx++;
                    if (g_idx <= o.cap_tags) o.tag_name_off[g_idx] = g_b;
                }
            } else if (ctx == X_PET) {
                if (!write) {
                    if (!L.has_name) return PJ_REC_MISSING_NAME;       // required (petstore.json:873-876)
                    if (!L.has_photo) return PJ_REC_MISSING_PHOTOURLS;
                } else {
                    const uint64_t row = pos[C_PETS];
                    if (row < o.cap_pets) {
                        o.id[row] = L.id;
                        o.flags[row] = (uint8_t)((L.has_id ? PJ_PET_HAS_ID : 0) | (L.has_cat ? PJ_PET_HAS_CATEGORY : 0) |
                                                 PJ_PET_HAS_NAME | PJ_PET_HAS_PHOTOURLS |
                                                 (L.has_tags ? PJ_PET_HAS_TAGS : 0));
                        o.status[row] = L.status;
                        o.cat_id[row] = L.cat_id;
                        o.cat_flags[row] = L.cat_flags;
                        o.name_off[row + 1] = pos[C_NAMEB] + L.name_len;
                        o.cat_name_off[row + 1] = pos[C_CATB] + L.cat_len;
                        o.photo_off[row + 1] = pos[C_URLS] + L.n_urls;
                        o.tag_off[row + 1] = pos[C_TAGS] + L.n_tags;
                    }
                    if (L.name_len) {
                        cq = L.name_pos; clen = L.name_len; cesc = L.name_esc;
                        cdst = o.name_bytes; coff = pos[C_NAMEB]; ccap = o.cap_name_bytes;
                    }
                }
            }
            if (cdst && coff + clen <= ccap) {
                WriteSink ws;
                ws.init(cdst, coff, P.dummy);
                if (!cesc) {
                    const uint8_t *src = s + cq + 1;
                    uint32_t k = 0;
                    for (; k + 8 <= clen; k += 8) ws.put8(ldu64(src + k), 8);
                    if (k < clen) ws.put8(ld_tail(src + k, (int)(clen - k)), (int)(clen - k));
                } else {
                    for (uint32_t q = cq + 1; s[q] != '"';) {
                        uint32_t c2 = s[q];
                        if (c2 == '\\') {
                            Esc e = escape_at(s, n, q);
                            ws.put(e.out, e.k);
                            q += e.adv;
                        } else {
                            ws.put_byte(c2);
                            q++;
                        }
                    }
                }
                ws.finish();
            }
            depth--;
            state = depth == 0 ? S_DONE : S_AFTER;
            continue;
        }
    }
#undef PEEK
#undef SKIP_WS
}

// ---------------------------------------------------------------- line records
// The 8 scanned counters of a line.
__device__ __forceinline__ void rec_counts(const LineRec &r, uint64_t *v) {
    const bool ok = r.code == 0;
    v[C_PETS] = ok;
    v[C_NAMEB] = ok ? r.name_len : 0;
    v[C_CATB] = ok ? r.cat_len : 0;
    v[C_URLS] = ok ? r.n_urls : 0;
    v[C_URLB] = ok ? r.url_bytes : 0;
    v[C_TAGS] = ok ? r.n_tags : 0;
    v[C_TAGB] = ok ? r.tag_bytes : 0;
    v[C_ERRS] = !ok;
}

// ---------------------------------------------------------------- fast path
// Straight-line parser for lines shaped like encoder output: no whitespace,
// properties in schema order (id, category, name, photoUrls, tags, status;
// Category / Tag: id, name), no nulls, no unknown keys, integer ids.
// Anything else returns PJ_BAIL and the line goes through run_line.  Errors
// it does return (status not in the enum, id out of range, broken string,
// missing required property) are the first error of the line, exactly as
// run_line reports them.
constexpr int PJ_BAIL = -1;
// line kinds of the split decode (above the code in the line's info word)
constexpr uint32_t LK_GENERAL = 1u << 8, LK_WAVE = 1u << 9, LK_BAD = 1u << 10;
// a line the bitmap-free pass left to k_dec_measure_long (long, or a full
// tape): its counters are missing from its block's scan until k_dec_fixup
constexpr uint32_t LK_DEFER = 1u << 11;
constexpr int PJ_TAPE_FULL = -2;  // valid so far, more items than the line tape holds: read by the wave

// bit k set iff byte k of x equals c
__device__ __forceinline__ uint32_t eq_mask8(uint64_t x, uint32_t c) {
    const uint64_t t = x ^ (c * 0x0101010101010101ull), m7 = 0x7F7F7F7F7F7F7F7Full;
    const uint64_t z = ~(((t & m7) + m7) | t) & 0x8080808080808080ull;
    return (uint32_t)(((z >> 7) * 0x0102040810204080ull) >> 56);
}
// Four hex digits (bytes 0..3 of x) as a code unit, or -1.
__device__ __forceinline__ int hex4(uint32_t x) {
    uint32_t cu = 0;
    bool ok = true;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int h = hexval((int)((x >> (8 * j)) & 0xFF));
        ok &= h >= 0;
        cu = cu * 16 + (uint32_t)(h & 15);
    }
    return ok ? (int)cu : -1;
}

// Bit 7 of the first byte of x that is '"', '\\', below 0x20 or above 0x7F
// (bits above it may be set too: borrows only run upwards from a byte that
// is flagged itself).
__device__ __forceinline__ uint64_t str_stop8(uint64_t x) {
    constexpr uint64_t ONE = 0x0101010101010101ull;
    const uint64_t q = x ^ (0x22 * ONE), b = x ^ (0x5C * ONE);
    return (((q - ONE) & ~q) | ((b - ONE) & ~b) | (x - 0x20 * ONE) | x) & (0x80 * ONE);
}
// The same for '"' and '\\' only.
__device__ __forceinline__ uint64_t quote_bs8(uint64_t x) {
    constexpr uint64_t ONE = 0x0101010101010101ull;
    const uint64_t q = x ^ (0x22 * ONE), b = x ^ (0x5C * ONE);
    return (((q - ONE) & ~q) | ((b - ONE) & ~b)) & (0x80 * ONE);
}
// Continuation bytes a UTF-8 lead byte c takes under jackson's lead classes
// (C0-DF one, E0-EF two, F0-F7 three), given x = the 8 bytes from the lead
// byte on; 0 if c is no lead byte (a control, a stray continuation byte,
// F8-FF) or a continuation byte is missing.
__device__ __forceinline__ uint32_t utf8_extra(uint32_t c, uint64_t x) {
    const uint32_t extra = (uint32_t)(c >= 0xC0) + (uint32_t)(c >= 0xE0) + (uint32_t)(c >= 0xF0);
    const uint64_t msk = (1ull << (8 * extra)) - 1;
    const uint64_t cb = (x >> 8) & msk & (0xC0C0C0ull);
    const bool ok = c >= 0xC0 && c <= 0xF7 && cb == (0x808080ull & msk);
    return ok ? extra : 0u;
}

// The stop byte c at q of a string (not its closing quote): an escape, a
// UTF-8 lead byte with its continuation bytes, or an error.  Returns the
// bytes consumed | the bytes they decode to << 8, or 0 for an error.
__device__ __noinline__ uint32_t str_step(const PJ_LDS uint8_t *s, uint32_t n, uint32_t q, uint32_t c) {
    if (c == '\\') {
        const uint64_t w = lds_u64(s + q);
        const uint32_t e = (uint32_t)(w >> 8) & 0xFF;
        if (e == 'u') {
            const Esc x = escape_at((const uint8_t *)s, n, q);
            return x.err ? 0u : (x.adv | ((uint32_t)x.k << 8));
        }
        constexpr uint64_t LO = (1ull << '"') | (1ull << '/');
        constexpr uint64_t HI = (1ull << ('\\' - 64)) | (1ull << ('b' - 64)) | (1ull << ('f' - 64)) |
                                (1ull << ('n' - 64)) | (1ull << ('r' - 64)) | (1ull << ('t' - 64));
        const bool ok = e < 128 && (((e < 64 ? LO : HI) >> (e & 63)) & 1) && q + 1 < n;
        return ok ? (2u | (1u << 8)) : 0u;
    }
    const uint32_t extra = utf8_extra(c, lds_u64(s + q));
    return extra ? ((1 + extra) | ((1 + extra) << 8)) : 0u;
}

// ---- word-at-a-time string decoding for the lane-parallel walk of long
// lines.  A 64-byte
// tile word at ws: xs[] its bytes, ub the mask of its 'u' bytes, nb the byte
// after it.  Each escape drops its leading bytes and keeps as many bytes as
// it decodes to (a simple escape drops the backslash and keeps the escaped
// character; \uXXXX drops 6 - k and keeps k; a surrogate pair drops 8 and
// keeps 4), so the decoded length of a word is the popcount of its keep
// mask.
struct Word {
    uint64_t xs[8];
    uint64_t bs, ub;
    uint32_t nb;
};
__device__ __forceinline__ void load_word(const PJ_LDS uint8_t *tile, uint32_t ws, Word &W) {
    W.bs = 0;
    W.ub = 0;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        W.xs[j] = lds_u64(tile + ws + 8 * j);
        W.bs |= (uint64_t)eq_mask8(W.xs[j], '\\') << (8 * j);
        W.ub |= (uint64_t)eq_mask8(W.xs[j], 'u') << (8 * j);
    }
    W.nb = tile[ws + 64];
}
// How far the dropped bytes of the last escape among starts (word at ws) reach.
__device__ __forceinline__ uint32_t last_drop(const PJ_LDS uint8_t *tile, uint32_t ws, uint64_t starts) {
    if (!starts) return 0;
    const uint32_t p = ws + 63 - (uint32_t)__builtin_clzll(starts);
    const uint64_t w = lds_u64(tile + p);
    const int cu = hex4((uint32_t)(w >> 16));
    if (((w >> 8) & 0xFF) != 'u') return p + 1;
    return cu >= 0xD800 && cu <= 0xDBFF ? p + 8                  // pair: 12 bytes, keeps 4
         : cu >= 0xDC00 && cu <= 0xDFFF ? p + 2                  // low half: the pair began at p - 6
         : p + 6 - (cu < 0x80 ? 1 : cu < 0x800 ? 2 : 3);
}
// The escapes that start in the word (starts, all at or after x, the first
// byte the word owns): \u escapes decoded for validity and output length
// (WRITE: their UTF-8 bytes stored in place over their kept bytes), simple
// escapes checked against "\/bfnrt (WRITE: decoded in place).  Sets err for
// anything malformed; returns the drop mask.  In-place decoding is only
// used on a string that has been validated, after which no reader of the
// line looks at its bytes again.
template <bool WRITE>
__device__ __forceinline__ uint64_t word_escapes(const PJ_LDS uint8_t *tile, uint32_t ws, const Word &W, uint64_t starts,
                                                 uint32_t x, bool &err) {
    PJ_LDS uint8_t *wt = (PJ_LDS uint8_t *)tile;
    const uint64_t nu = (W.ub >> 1) | ((uint64_t)(W.nb == 'u') << 63);
    const uint64_t su = starts & nu, ss = starts & ~nu;
    uint64_t dropm = ss;                                   // a simple escape drops its backslash
    uint32_t y = x;
    for (uint64_t m = su; m; m &= m - 1) {
        const uint32_t p = ws + (uint32_t)__builtin_ctzll(m);
        if (p < y) continue;                               // the low half of a pair
        const uint64_t w = lds_u64(tile + p), w2 = lds_u64(tile + p + 6);
        const int cu = hex4((uint32_t)(w >> 16)), lo = hex4((uint32_t)(w2 >> 16));
        const bool hs = cu >= 0xD800 && cu <= 0xDBFF, ls = cu >= 0xDC00 && cu <= 0xDFFF;
        const bool pair = hs && (w2 & 0xFFFF) == ('\\' | ('u' << 8)) && lo >= 0xDC00 && lo <= 0xDFFF;
        err |= cu < 0 || ls || (hs && !pair);
        const uint32_t cp = pair ? 0x10000 + (((uint32_t)cu - 0xD800) << 10) + ((uint32_t)lo - 0xDC00) : (uint32_t)cu;
        const uint32_t k = cp < 0x80 ? 1 : cp < 0x800 ? 2 : cp < 0x10000 ? 3 : 4;
        const uint32_t adv = pair ? 12 : 6, dr = adv - k, b = p - ws;
        dropm |= (b + dr >= 64 ? ~0ull : ((1ull << (b + dr)) - 1)) & (~0ull << b);
        if (WRITE) {
            int kk;
            const uint32_t u8 = utf8_pack(cp, &kk);
            for (uint32_t i = 0; i < k; i++) wt[p + dr + i] = (uint8_t)(u8 >> (8 * i));
        }
        y = p + adv;
    }
    for (uint64_t m = ss; m; m &= m - 1) {
        const uint32_t i = (uint32_t)__builtin_ctzll(m) + 1;
        uint64_t qw = W.xs[0];
#pragma unroll
        for (int j = 1; j < 8; j++) qw = (i >> 3) == (uint32_t)j ? W.xs[j] : qw;
        const uint32_t c = i == 64 ? W.nb : (uint32_t)(qw >> (8 * (i & 7))) & 0xFF;
        if (!WRITE) {
            constexpr uint64_t LO = (1ull << '"') | (1ull << '/');
            constexpr uint64_t HI = (1ull << ('\\' - 64)) | (1ull << ('b' - 64)) | (1ull << ('f' - 64)) |
                                    (1ull << ('n' - 64)) | (1ull << ('r' - 64)) | (1ull << ('t' - 64));
            err |= c >= 128 || !(((c < 64 ? LO : HI) >> (c & 63)) & 1);
        } else if (c >= 'b') {
            uint32_t o = 8;                                // 'b'
            o = c == 'f' ? 12u : o;
            o = c == 'n' ? 10u : o;
            o = c == 'r' ? 13u : o;
            o = c == 't' ? 9u : o;
            wt[ws + i] = (uint8_t)o;
        }
    }
    return dropm;
}
// The bytes of the word at ws kept by km (read after the in-place
// decoding), compacted, into o.
__device__ __forceinline__ void word_store(const PJ_LDS uint8_t *tile, uint32_t ws, uint64_t km, StoreSink &o) {
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const uint32_t kb = (uint32_t)(km >> (8 * j)) & 0xFF;
        if (!kb) continue;
        const uint64_t v = lds_u64(tile + ws + 8 * j);
        if (kb == 0xFF) {
            o.put8(v, 8);
            continue;
        }
        uint64_t cv = 0;
        uint32_t cn = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const bool kp = (kb >> i) & 1;
            cv |= kp ? ((v >> (8 * i)) & 0xFF) << (8 * cn) : 0ull;
            cn += kp;
        }
        o.put8(cv, cn);
    }
}
// One line of an LDS tile as the fast path reads it.  With COOP false one
// thread owns the line.  With COOP true the 64 lanes of a wave hold the same
// line and walk its structure in step (every decision is taken on the same
// bytes, so the wave never diverges); strings that are long or hold escapes
// are then measured and copied lane-parallel, 4 KiB per step, and only the
// first lane performs the scalar column stores.
template <bool COOP>
struct FLineT {
    static constexpr bool coop = COOP;
    const PJ_LDS uint8_t *s;        // the line's first byte in the LDS tile
    const PJ_LDS uint64_t *special; // the tile's specials bitmap
    uint32_t s0, n;          // tile offset and length of the line
    __device__ __forceinline__ bool lead() const { return !COOP || lane_id() == 0; }
    // 8 bytes at q: the tile is zero-padded 64 bytes past its data, so any
    // q up to n + 32 may be read without a check
    __device__ __forceinline__ uint64_t ld8(uint32_t q) const { return lds_u64(s + q); }
    __device__ __forceinline__ int at(uint32_t q) const { return q < n ? (int)s[q] : -1; }
    __device__ __forceinline__ uint32_t next_special(uint32_t q) const {
        const uint32_t a = s0 + q, lim = s0 + n;
        if (a >= lim) return n;
        uint32_t wi = a >> 6;
        uint64_t m = special[wi] & (~0ull << (a & 63));
        while (!m && (wi + 1) * 64 < lim) m = special[++wi];
        if (!m) return n;
        const uint32_t at = wi * 64 + (uint32_t)__builtin_ctzll(m);
        return at < lim ? at - s0 : n;
    }
    // the first special at or after q within the next two bitmap words, else n
    __device__ __forceinline__ uint32_t near_special(uint32_t q) const {
        const uint32_t a = s0 + q, lim = s0 + n;
        if (a >= lim) return n;
        const uint32_t wi = a >> 6;
        uint64_t m = special[wi] & (~0ull << (a & 63));
        uint32_t at = wi * 64 + (uint32_t)__builtin_ctzll(m);
        if (!m) {
            if ((wi + 1) * 64 >= lim) return n;
            m = special[wi + 1];
            if (!m) return n;
            at = (wi + 1) * 64 + (uint32_t)__builtin_ctzll(m);
        }
        return at < lim ? at - s0 : n;
    }
    // Escape at q (a backslash).  The two-byte forms and a \uXXXX outside the
    // surrogate range are decoded from one 8-byte read; surrogates and
    // malformed escapes go to escape_at.
    __device__ __forceinline__ Esc esc(uint32_t q) const { return esc_w(q, ld8(q)); }
    // the same, given w = the 8 bytes at q
    __device__ __forceinline__ Esc esc_w(uint32_t q, uint64_t w) const {
        const uint32_t c = (uint32_t)(w >> 8) & 0xFF;
        Esc r{0, 2, 0, 1};
        if (c == 'u') {
            if (q + 6 <= n) {
                const int cu = hex4((uint32_t)(w >> 16));
                if (cu >= 0 && (cu < 0xD800 || cu > 0xDFFF)) {
                    r.adv = 6;
                    r.out = utf8_pack((uint32_t)cu, &r.k);
                    return r;
                }
            }
            return escape_at((const uint8_t *)s, n, q);
        }
        if (q + 1 >= n) return escape_at((const uint8_t *)s, n, q);
        switch (c) {
        case '"': case '\\': case '/': r.out = c; break;
        case 'b': r.out = 8; break;
        case 'f': r.out = 12; break;
        case 'n': r.out = 10; break;
        case 'r': r.out = 13; break;
        case 't': r.out = 9; break;
        default: return escape_at((const uint8_t *)s, n, q);
        }
        return r;
    }
    // string whose first content byte is at q (opening quote at q-1)
    __device__ __forceinline__ Str str(uint32_t q) const {
        if (COOP) {
            const uint32_t sp = near_special(q);
            if (sp < n && s[sp] == '"') return Str{0, sp, sp - q, false};
            return wave_str<false>(q, nullptr);
        }
        if (!special) return str_swar(q);
        Str r{0, 0, 0, false};
        uint32_t d = 0;
        for (;;) {
            const uint32_t sp = next_special(q);
            if (sp >= n) { r.err = PJ_REC_STRING; return r; }
            d += sp - q;
            if (s[sp] == '"') { r.end = sp; break; }
            Esc e = esc(sp);
            if (e.err) { r.err = e.err; return r; }
            d += (uint32_t)e.k;
            q = sp + e.adv;
            r.esc = true;
        }
        r.dlen = d;
        return r;
    }
    // String at q read 8 bytes at a time without the bitmaps: the first
    // byte of each 8 that is a quote, a backslash, a control or non-ASCII
    // stops the scan (str_stop8), and each kind is settled where it stands:
    // the closing quote ends the string, an escape is decoded, a UTF-8 lead
    // byte must carry its continuation bytes (jackson's lead classes), and a
    // raw control is an error.  The byte after the line is its newline or
    // the tile's zero padding, a control, so the scan never leaves the line.
    __device__ __forceinline__ Str str_swar(uint32_t q) const {
        Str r{0, 0, 0, false};
        const uint32_t q0 = q;
        uint32_t shrink = 0;                       // raw bytes minus decoded bytes of the escapes
        for (;;) {
            // 16 bytes per step, both loads in flight together
            const uint64_t x0 = ld8(q), x1 = ld8(q + 8);
            const uint64_t m0 = str_stop8(x0), m1 = str_stop8(x1);
            if (!(m0 | m1)) {
                q += 16;
                continue;
            }
            const uint32_t k = m0 ? (uint32_t)__builtin_ctzll(m0) >> 3 : 8 + ((uint32_t)__builtin_ctzll(m1) >> 3);
            q += k;
            const uint32_t c = (uint32_t)((m0 ? x0 : x1) >> (8 * (k & 7))) & 0xFF;
            if (c == '"') break;
            // an escape, a UTF-8 sequence or an error: out of line
            const uint32_t st = str_step((const PJ_LDS uint8_t *)s, n, q, c);
            if (!st) {
                r.err = PJ_REC_STRING;
                return r;
            }
            const uint32_t adv = st & 0xFF, dk = (st >> 8) & 0xFF;
            q += adv;
            shrink += adv - dk;
            r.esc |= c == '\\';
        }
        r.end = q;
        r.dlen = q - q0 - shrink;
        return r;
    }
    // copy the decoded string (content from q, described by r) to dst
    __device__ __forceinline__ void copy(uint32_t q, const Str &r, uint8_t *dst) const {
        if (COOP) {
            if (r.esc) wave_str<true>(q, dst);
            else
                for (uint32_t k = 16u * (uint32_t)lane_id(); k < r.dlen; k += 1024)
                    copy_from_lds(dst + k, s + q + k, min(16u, r.dlen - k));
            return;
        }
        if (!r.esc) {
            copy_from_lds(dst, s + q, r.dlen);
            return;
        }
        if (!special) {
            // runs between escapes go out whole; the next backslash (or the
            // closing quote) is found 8 bytes at a time
            uint8_t *dd = dst;
            uint32_t x = q;
            for (;;) {
                uint32_t stop = x;
                for (;;) {
                    const uint64_t m = quote_bs8(ld8(stop));
                    if (m) { stop += (uint32_t)__builtin_ctzll(m) >> 3; break; }
                    stop += 8;
                }
                stop = min(stop, r.end);
                if (stop > x) {
                    copy_from_lds(dd, s + x, stop - x);
                    dd += stop - x;
                }
                if (stop >= r.end) break;
                const Esc e = esc(stop);
                st_tail(dd, e.out, (uint32_t)e.k);
                dd += e.k;
                x = stop + e.adv;
            }
            return;
        }
        // runs between escapes go out whole; the specials bitmap finds the
        // next backslash (or the closing quote) in a few word reads
        uint8_t *d = dst;
        uint32_t x = q;
        uint32_t wi = (s0 + x) >> 6;
        uint64_t m = special[wi] & (~0ull << ((s0 + x) & 63));
        for (;;) {
            while (!m) m = special[++wi];                  // the closing quote bounds the walk
            const uint32_t stop = min(wi * 64 + (uint32_t)__builtin_ctzll(m) - s0, r.end);
            if (stop > x) {
                copy_from_lds(d, s + x, stop - x);
                d += stop - x;
            }
            if (stop >= r.end) break;
            const Esc e = esc(stop);
            st_tail(d, e.out, (uint32_t)e.k);
            d += e.k;
            x = stop + e.adv;
            const uint32_t a = s0 + x;
            if ((a >> 6) != wi) {
                wi = a >> 6;
                m = special[wi] & (~0ull << (a & 63));
            } else m &= ~0ull << (a & 63);
        }
    }

    // Lane-parallel string walk (COOP only; all 64 lanes, uniform q).  Lane l
    // owns tile word w0 + l of each 64-word step.  Per word: the backslash
    // mask from its bytes, the escaped characters from a wave scan of the
    // backslash-run carry, the closing quote as the first unescaped quote of
    // the wave.  Each escape drops its leading bytes and keeps as many bytes
    // as it decodes to (a simple escape drops the backslash and keeps the
    // escaped character; \uXXXX drops 6 - k and keeps k; a surrogate pair
    // drops 8 and keeps 4), so a lane's output is its word compacted by a
    // keep mask: the decoded length is a popcount.  An escape reaching into
    // the next word hands on how far its dropped bytes go.  \u escapes are
    // decoded in a loop of their own, simple ones only checked, so lanes
    // that meet different kinds do not run each other's code.  Any malformed
    // escape, or no closing quote, is PJ_REC_STRING, the code the serial
    // walk gives.  With WRITE (called only on a string that str() accepted)
    // each escape's decoded bytes are first stored in place over its kept
    // bytes in the tile, which no later reader of the line looks at, and the
    // compacted words go to dst at each lane's offset (a wave scan).
    template <bool WRITE>
    __device__ __forceinline__ Str wave_str(uint32_t q, uint8_t *dst) const {
        const int l = lane_id();
        const PJ_LDS uint8_t *tile = s - s0;
        const uint32_t a = s0 + q, lim = s0 + n;
        Str res{0, 0, 0, false};
        uint32_t ecarry = 0;         // the first byte of this step is escaped
        uint32_t drop_in = a;        // bytes before this are dropped by an escape of the previous step
        uint32_t d = 0;              // decoded bytes so far
        bool any_esc = false;
        for (uint32_t w0 = a >> 6;; w0 += 64) {
            const uint32_t ws = (w0 + (uint32_t)l) * 64;
            const bool act = ws < lim;
            Word Wd;
            uint64_t bs = 0, qt = 0;
            if (act) {
                load_word(tile, ws, Wd);
                qt = special[ws >> 6] & ~Wd.bs;
                uint64_t m = ~0ull;
                if (ws < a) m <<= (a - ws);
                if (lim - ws < 64) m &= (1ull << (lim - ws)) - 1;
                bs = Wd.bs & m;
                qt &= m;
            } else {
                Wd.bs = Wd.ub = 0;
                Wd.nb = 0;
#pragma unroll
                for (int j = 0; j < 8; j++) Wd.xs[j] = 0;
            }
            // backslash-run carry across the wave: compose c -> cout maps
            uint32_t c0, c1;
            const uint64_t e0 = escaped64(bs, 0, &c0), e1 = escaped64(bs, 1, &c1);
            uint32_t F = c0 | (c1 << 1);
#pragma unroll
            for (int dd = 1; dd < 64; dd <<= 1) {
                const uint32_t G = (uint32_t)__shfl_up((int)F, (unsigned)dd, 64);
                if (l >= dd) F = ((F >> (G & 1)) & 1) | (((F >> ((G >> 1) & 1)) & 1) << 1);
            }
            const uint32_t Fp = (uint32_t)__shfl_up((int)F, 1u, 64);
            const uint32_t cin = l == 0 ? ecarry : ((Fp >> ecarry) & 1);
            uint64_t starts = bs & ~(cin ? e1 : e0);
            // closing quote
            const uint64_t qb = __ballot(qt != 0);
            const int E = qb ? __builtin_ctzll(qb) : 64;
            const uint32_t qpos = (uint32_t)__shfl((int)(ws + (uint32_t)__builtin_ctzll(qt | (1ull << 63))), E & 63, 64);
            const uint32_t hi = qb ? qpos : ws + 64;          // this lane's bytes end here (exclusive)
            if (l > E) starts = 0;
            if (l == E) starts &= (1ull << (qpos & 63)) - 1;
            const bool mine = l <= E && act;
            // how far the dropped bytes of this word's last escape reach
            const uint32_t drop = last_drop(tile, ws, starts);
            const uint32_t dprev = (uint32_t)__shfl_up((int)drop, 1u, 64);
            uint32_t x = ws < a ? a : ws;
            const uint32_t from = l == 0 ? drop_in : dprev;
            if (from > x) x = from;
            const uint32_t end = min(hi, ws + 64);
            uint64_t keep = 0;
            if (mine && x < end) {
                keep = ~0ull << (x - ws);
                if (end - ws < 64) keep &= (1ull << (end - ws)) - 1;
            }
            starts &= keep;
            bool err = false;
            const uint64_t dropm = word_escapes<WRITE>(tile, ws, Wd, starts, x, err);
            const uint64_t km = keep & ~dropm;
            const uint32_t dl = mine ? (uint32_t)__builtin_popcountll(km) : 0u;
            if (!mine) err = false;
            if (__ballot(err)) { res.err = PJ_REC_STRING; return res; }
            const uint32_t off = (uint32_t)(wave_incl_scan(dl) - dl);
            if (WRITE && dl) {
                StoreSink o;
                o.init(dst + d + off);
                word_store(tile, ws, km, o);
                o.finish();
            }
            any_esc |= __ballot(starts != 0) != 0;
            d += (uint32_t)wave_sum(dl);
            if (qb) {
                res.end = qpos - s0;
                res.dlen = d;
                res.esc = any_esc;
                return res;
            }
            if ((w0 + 64) * 64 >= lim) { res.err = PJ_REC_STRING; return res; }   // no closing quote
            ecarry = (uint32_t)__shfl((int)((F >> ecarry) & 1), 63, 64);
            drop_in = (uint32_t)__shfl((int)drop, 63, 64);
        }
    }
};
using FLine = FLineT<false>;

// One workgroup's slice of every output column: the pointers are already
// advanced to the block's first row / byte / item, and the b_* fields are the
// absolute offsets those slices start at (what the offset arrays hold).
struct BlockCols {
    int64_t *id, *cat_id, *tag_id;
    uint8_t *flags, *status, *cat_flags, *tag_flags;
    uint64_t *name_off, *cat_name_off, *photo_off, *tag_off;     // entry row + 1
    uint64_t *url_off, *tag_name_off;                            // entry item + 1
    uint8_t *name, *cat_name, *url, *tag_name;
    uint64_t b_name, b_cat, b_urls, b_url, b_tags, b_tag;
};

// bit 7 of each byte set iff that byte is not an ASCII digit
__device__ __forceinline__ uint64_t nondigit8(uint64_t x) {
    const uint64_t m7 = 0x7F7F7F7F7F7F7F7Full;
    const uint64_t ge0 = ((x & m7) + 0x5050505050505050ull) | x;   // >= '0' (or >= 0x80)
    const uint64_t ge9 = ((x & m7) + 0x4646464646464646ull) | x;   // >= ':' (or >= 0x80)
    return (~ge0 | ge9) & 0x8080808080808080ull;
}

// value of m (1..8) ASCII digits packed little endian in x (first digit low)
__device__ __forceinline__ uint64_t digits8(uint64_t x, int m) {
    uint64_t y = x - 0x3030303030303030ull;
    if (m < 8) y <<= 8 * (8 - m);
    y = (y * 10 + (y >> 8)) & 0x00FF00FF00FF00FFull;
    y = (y * 100 + (y >> 16)) & 0x0000FFFF0000FFFFull;
    return (y * 10000 + (y >> 32)) & 0xFFFFFFFFull;
}

// Canonical Long at p: -?(0|[1-9][0-9]*) followed by ',' or '}'.  Returns 0,
// PJ_REC_NUMBER (out of int64 range) or PJ_BAIL; the value only when VAL.
template <bool VAL, class FL>
__device__ __forceinline__ int fnum(const FL &F, uint32_t &p, int64_t &v) {
    uint32_t q = p;
    const bool neg = F.at(q) == '-';
    q += neg;
    uint32_t k = 0;
    uint64_t c0 = 0, c1 = 0, c2 = 0;
    {
        c0 = F.ld8(q);
        uint64_t nd = nondigit8(c0);
        k = nd ? (uint32_t)(__builtin_ctzll(nd) >> 3) : 8;
        if (k == 8) {
            c1 = F.ld8(q + 8);
            nd = nondigit8(c1);
            uint32_t k1 = nd ? (uint32_t)(__builtin_ctzll(nd) >> 3) : 8;
            k += k1;
            if (k1 == 8) {
                c2 = F.ld8(q + 16);
                nd = nondigit8(c2);
                k += nd ? (uint32_t)(__builtin_ctzll(nd) >> 3) : 8;
            }
        }
    }
    if (k == 0 || q + k > F.n) return PJ_BAIL;
    if ((c0 & 0xFF) == '0' && k > 1) return PJ_BAIL;            // leading zero: general rules
    const int nx = F.at(q + k);
    if (nx != ',' && nx != '}') return PJ_BAIL;                  // fraction, exponent, space...
    if (k > 19) return PJ_REC_NUMBER;
    if (k == 19) {                                               // compare with 9223372036854775807/8
        const uint64_t a = __builtin_bswap64(c0), b = __builtin_bswap64(c1);
        const uint32_t c = (uint32_t)((c2 & 0xFF) << 16 | ((c2 >> 8) & 0xFF) << 8 | ((c2 >> 16) & 0xFF));
        const uint64_t A = __builtin_bswap64(pack8("92233720", 8)), B = __builtin_bswap64(pack8("36854775", 8));
        const uint32_t Cl = neg ? ('8' << 16 | '0' << 8 | '8') : ('8' << 16 | '0' << 8 | '7');
        if (a > A || (a == A && (b > B || (b == B && c > Cl)))) return PJ_REC_NUMBER;
    }
    if (VAL) {
        uint64_t acc;
        if (k <= 8) acc = digits8(c0, (int)k);
        else if (k <= 16) {
            uint64_t p10 = 1;
            for (uint32_t j = 0; j < k - 8; j++) p10 *= 10;
            acc = digits8(c0, 8) * p10 + digits8(c1, (int)(k - 8));
        } else {
            uint64_t p10 = 1;
            for (uint32_t j = 0; j < k - 16; j++) p10 *= 10;
            acc = (digits8(c0, 8) * 100000000ull + digits8(c1, 8)) * p10 + digits8(c2, (int)(k - 16));
        }
        v = neg ? (int64_t)(0ull - acc) : (int64_t)acc;
    }
    p = q + k;
    return 0;
}

// 8-byte key prefixes (opening quote included)
constexpr uint64_t KP_ID = pack8("\"id\":", 5), KP_ID_MASK = 0xFFFFFFFFFFull;   // "id":
constexpr uint64_t KP_CATEGORY = pack8("\"categor", 8), KP_NAME = pack8("\"name\":\"", 8),
                   KP_PHOTO = pack8("\"photoUr", 8), KP_TAGS = pack8("\"tags\":[", 8),
                   KP_STATUS = pack8("\"status\"", 8);

// Category / Tag body after '{': optional "id":N, then optional "name":"S",
// then '}'.
template <bool WRITE, class FL>
__device__ __forceinline__ int fsub(const FL &F, uint32_t &p, int64_t &id, uint32_t &fl, uint32_t &nq, Str &nr) {
    fl = 0;
    id = 0;
    uint64_t k8 = F.ld8(p);
    if ((k8 & KP_ID_MASK) == pack8("\"id\":", 5) && p + 5 <= F.n) {
        p += 5;
        int e = fnum<WRITE>(F, p, id);
        if (e) return e;
        fl |= PJ_SUB_HAS_ID;
        if (F.at(p) == ',') {
            p++;
            k8 = F.ld8(p);
            if (k8 != KP_NAME || p + 8 > F.n) return PJ_BAIL;
        }
    }
    if (k8 == KP_NAME && p + 8 <= F.n && !(fl & PJ_SUB_HAS_NAME)) {
        p += 8;
        nq = p;
        nr = F.str(p);
        if (nr.err) return nr.err;
        p = nr.end + 1;
        fl |= PJ_SUB_HAS_NAME;
    }
    if (F.at(p) != '}') return PJ_BAIL;
    p++;
    return 0;
}

// Lane-parallel reading of a tags array (COOP lines) whose first element
// starts at p (a '{').  Lane l owns tile word w0 + l of each 64-word step; the
// '{' bytes outside strings (string state from the parity of unescaped
// quotes since p) are the element starts, and each lane reads the elements
// that start in its word with the per-thread parser, in order.  An element
// that reads cleanly and is followed by ",{" hands over to the next start,
// which is therefore the next element; the first lane that meets ']', an
// error or anything else decides the array, and lanes after it are ignored.
// Elements are validated exactly as the serial loop validates them, so the
// code returned is the one it would return.  On success p is past ']' and
// cnt / bytes hold the number of tags and their name bytes; with WRITE the
// tags are stored from block-relative index g0 / name byte gb0.
template <bool WRITE>
__device__ __forceinline__ int wave_tags(const FLineT<true> &F, uint32_t &p, uint32_t &cnt, uint32_t &bytes,
                                         const BlockCols *W, uint32_t g0, uint32_t gb0) {
    const int l = lane_id();
    const FLine L{F.s, F.special, F.s0, F.n};
    const PJ_LDS uint8_t *tile = F.s - F.s0;
    const uint32_t a = F.s0 + p, lim = F.s0 + F.n;
    uint32_t par = 0;                     // inside a string at the start of this step
    uint32_t c_done = 0, b_done = 0;      // tags and name bytes of earlier steps
    for (uint32_t w0 = a >> 6;; w0 += 64) {
        const uint32_t ws = (w0 + (uint32_t)l) * 64;
        uint64_t qt = 0, lb = 0;
        if (ws < lim) {
            uint64_t bs = 0;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const uint64_t x = lds_u64(tile + ws + 8 * j);
                bs |= (uint64_t)eq_mask8(x, '\\') << (8 * j);
                lb |= (uint64_t)eq_mask8(x, '{') << (8 * j);
            }
            qt = F.special[ws >> 6] & ~bs;
            uint64_t m = ~0ull;
            if (ws < a) m <<= (a - ws);
            if (lim - ws < 64) m &= (1ull << (lim - ws)) - 1;
            qt &= m;
            lb &= m;
        }
        const uint64_t pb = __ballot(__builtin_popcountll(qt) & 1);
        const uint32_t before = (par ^ (uint32_t)__builtin_popcountll(pb & ((1ull << l) - 1))) & 1;
        const uint64_t instr = prefix_xor(qt) ^ (before ? ~0ull : 0ull);
        const uint64_t cand = lb & ~instr;
        // read this lane's elements
        uint32_t lc = 0, lbytes = 0, pend = 0;
        int stop = 0, scode = 0;          // stop: 1 ']' after a clean element, 2 the array fails
        for (uint64_t m = cand; m; m &= m - 1) {
            uint32_t q = ws + (uint32_t)__builtin_ctzll(m) - F.s0 + 1;
            int64_t id;
            uint32_t fl, nq = 0;
            Str nr{0, 0, 0, false};
            const int e = fsub<false>(L, q, id, fl, nq, nr);
            if (e) { stop = 2; scode = e; break; }
            lc++;
            lbytes += (fl & PJ_SUB_HAS_NAME) ? nr.dlen : 0;
            const int c = L.at(q);
            if (c == ']') { stop = 1; pend = q + 1; break; }
            if (c != ',' || L.at(q + 1) != '{') { stop = 2; scode = PJ_BAIL; break; }
        }
        const uint64_t sb = __ballot(stop != 0);
        const int S = sb ? __builtin_ctzll(sb) : 64;
        if (l > S) { lc = 0; lbytes = 0; }
        if (sb) {
            const int st = __shfl(stop, S, 64);
            if (st == 2) return __shfl(scode, S, 64);
        }
        const uint32_t oc = (uint32_t)(wave_incl_scan(lc) - lc), ob = (uint32_t)(wave_incl_scan(lbytes) - lbytes);
        if (WRITE && l <= S && lc) {
            uint32_t gi = g0 + c_done + oc, bi = gb0 + b_done + ob;
            uint64_t m = cand;
            for (uint32_t k = 0; k < lc; k++, m &= m - 1) {
                uint32_t q = ws + (uint32_t)__builtin_ctzll(m) - F.s0 + 1;
                int64_t id;
                uint32_t fl, nq = 0;
                Str nr{0, 0, 0, false};
                fsub<true>(L, q, id, fl, nq, nr);
                const uint32_t tl = (fl & PJ_SUB_HAS_NAME) ? nr.dlen : 0;
                W->tag_id[gi] = id;
                W->tag_flags[gi] = (uint8_t)fl;
                W->tag_name_off[gi] = W->b_tag + bi + tl;
                if (tl) L.copy(nq, nr, W->tag_name + bi);
                gi++;
                bi += tl;
            }
        }
        c_done += (uint32_t)wave_sum(lc);
        b_done += (uint32_t)wave_sum(lbytes);
        if (sb) {
            cnt = c_done;
            bytes = b_done;
            p = (uint32_t)__shfl((int)pend, S, 64);
            return 0;
        }
        if ((w0 + 64) * 64 >= lim) return PJ_BAIL;   // not reached: the last element always stops
        par = (par ^ (uint32_t)__builtin_popcountll(pb)) & 1;
    }
}

// Does the 8-byte prefix at a key start belong to one of the Pet keys as the
// encoder writes them?
__device__ __forceinline__ bool known8(uint64_t k8) {
    return ((k8 & KP_ID_MASK) == KP_ID) | (k8 == KP_CATEGORY) | (k8 == KP_NAME) | (k8 == KP_PHOTO) | (k8 == KP_TAGS) |
           (k8 == KP_STATUS);
}

// An unknown property at p: its key, ':' and a string, integer or literal
// value are skipped, as serde skips properties the bean does not declare.
// Keys with escapes, known keys in another shape, nested values and
// anything irregular return PJ_BAIL.  Returns (new p) << 32 | code.
template <class FL>
__device__ __noinline__ uint64_t fskip(const FL &F, uint32_t p) {
    constexpr uint64_t BAIL = (uint32_t)PJ_BAIL;
    if (F.at(p) != '"') return BAIL;
    const Str k = F.str(p + 1);
    if (k.err) return (uint32_t)k.err;
    if (k.esc) return BAIL;
    const uint64_t x = F.ld8(p + 1), x2 = F.ld8(p + 9) & 0xFF;
    const uint32_t L = k.dlen;
    if ((L == 2 && (x & 0xFFFFull) == pack8("id", 2)) || (L == 8 && x == pack8("category", 8)) ||
        (L == 4 && (x & 0xFFFFFFFFull) == pack8("name", 4)) || (L == 9 && x == pack8("photoUrl", 8) && x2 == 's') ||
        (L == 4 && (x & 0xFFFFFFFFull) == pack8("tags", 4)) || (L == 6 && (x & 0xFFFFFFFFFFFFull) == pack8("status", 6)))
        return BAIL;
    p = k.end + 1;
    if (F.at(p) != ':') return BAIL;
    p++;
    const int c = F.at(p);
    if (c == '"') {
        const Str v = F.str(p + 1);
        if (v.err) return (uint32_t)v.err;
        p = v.end + 1;
    } else if (c == '-' || (c >= '0' && c <= '9')) {
        uint32_t q = p + (c == '-'), d = 0;
        for (int i = 0; i < 3; i++) {
            const uint64_t nd = nondigit8(F.ld8(q + d));
            const uint32_t m = nd ? (uint32_t)(__builtin_ctzll(nd) >> 3) : 8;
            d += m;
            if (m < 8) break;
        }
        if (d == 0 || d >= 24 || q + d > F.n) return BAIL;
        if (F.at(q) == '0' && d > 1) return BAIL;
        p = q + d;
    } else {
        const uint64_t w = F.ld8(p);
        if ((w & 0xFFFFFFFFull) == pack8("true", 4) || (w & 0xFFFFFFFFull) == pack8("null", 4)) p += 4;
        else if ((w & 0xFFFFFFFFFFull) == pack8("false", 5)) p += 5;
        else return BAIL;
    }
    if (p > F.n) return BAIL;
    return (uint64_t)p << 32;
}

// Separator after a property value: ',' loads the next key prefix, '}' ends
// the object; anything else is not canonical.
#define FL_SEP()                                                    \
    {                                                               \
        const int c_ = F.at(p);                                     \
        if (c_ == ',') { p++; k8 = F.ld8(p); }                      \
        else if (c_ == '}') more = false;                           \
        else return PJ_BAIL;                                        \
    }

// Unknown properties before the next key.
#define FL_UNKNOWN()                                                \
    while (more && !known8(k8)) {                                   \
        const uint64_t r_ = fskip(F, p);                            \
        if ((uint32_t)r_) return (int)(uint32_t)r_;                 \
        p = (uint32_t)(r_ >> 32);                                   \
        FL_SEP();                                                   \
    }

// ---------------------------------------------------------------- line tape
// The validating walk of a canonical line records what the writing walk
// needs, so that the writer stores and copies without parsing again:
//   word 0 id, word 1 category id,
//   word 2 flags | status << 8 | category flags << 16 | urls << 24 |
//          tags << 32,
//   word 3 the name string, word 4 the category name string,
//   words 5.. one word per url, then two per tag (id, name string).
// A string word holds line-relative start, closing quote and decoded length
// (16 bits each), bit 48 "has escapes" and, for a tag, its flags in bits
// 49-50.  A line with more items than the words left (PJ_TAPE_FULL) is read
// by its wave instead, like a long line.
#ifndef PJ_TAPE_WORDS
#define PJ_TAPE_WORDS 32
#endif
constexpr int TAPE_WORDS = PJ_TAPE_WORDS;
// The tapes are stored word by word across lines (word k of line l at
// tape[k * lines + l]), so the lanes of a wave reading or writing the same
// word of their lines touch adjacent addresses.
struct Tape {
    uint64_t *p;        // word 0 of the line
    uint64_t s;         // lines (the stride between words)
    __device__ __forceinline__ uint64_t &operator[](uint32_t k) const { return p[(uint64_t)k * s]; }
};
__device__ __forceinline__ uint64_t tape_str(uint32_t q, const Str &r) {
    return (uint64_t)q | ((uint64_t)r.end << 16) | ((uint64_t)r.dlen << 32) | ((uint64_t)r.esc << 48);
}

// The properties are tried in schema order, each at most once, as straight
// code: the lanes of a wave then walk the same instruction stream whatever
// subset of properties their lines hold.
// Pass 0 (WRITE false) validates and measures into R; pass 1 writes the
// record at the line's offsets rel[] inside the block's column slices W.
// With TAPE, pass 0 also records the line's tape at T.
template <bool WRITE, class FL, bool TAPE = false>
__device__ __forceinline__ int fline(const FL &F, LineRec &R, const BlockCols *W, const uint32_t *rel,
                                     Tape T = Tape{nullptr, 0}) {
    constexpr bool VAL = WRITE || TAPE;             // integer values are needed
    const uint32_t n = F.n;
    if (n == 0) return PJ_REC_EMPTY;
    if (F.at(0) != '{') return PJ_BAIL;
    uint32_t p = 1;
    uint32_t flags = 0;
    uint8_t status = PJ_STATUS_NULL;
    int64_t id = 0, cat_id = 0;
    uint32_t cat_fl = 0, name_len = 0, cat_len = 0, n_urls = 0, url_bytes = 0, n_tags = 0, tag_bytes = 0;
    bool more = F.at(p) != '}';
    uint64_t k8 = more ? F.ld8(p) : 0;
    FL_UNKNOWN();
    // id
    if (more && (k8 & KP_ID_MASK) == KP_ID) {
        p += 5;
        const int e = fnum<VAL>(F, p, id);
        if (e) return e;
        flags |= PJ_PET_HAS_ID;
        FL_SEP();
    }
    FL_UNKNOWN();
    // category
    if (more && k8 == KP_CATEGORY && (F.ld8(p + 8) & 0xFFFFFFFFull) == pack8("y\":{", 4)) {
        p += 12;
        uint32_t nq = 0;
        Str nr{0, 0, 0, false};
        const int e = fsub<VAL>(F, p, cat_id, cat_fl, nq, nr);
        if (e) return e;
        flags |= PJ_PET_HAS_CATEGORY;
        cat_len = (cat_fl & PJ_SUB_HAS_NAME) ? nr.dlen : 0;
        if (TAPE && (cat_fl & PJ_SUB_HAS_NAME)) T[4] = tape_str(nq, nr);
        if (WRITE && cat_len) F.copy(nq, nr, W->cat_name + rel[C_CATB]);
        FL_SEP();
    }
    FL_UNKNOWN();
    // name
    if (more && k8 == KP_NAME) {
        const uint32_t q = p + 8;
        const Str r = F.str(q);
        if (r.err) return r.err;
        p = r.end + 1;
        flags |= PJ_PET_HAS_NAME;
        name_len = r.dlen;
        if (TAPE) T[3] = tape_str(q, r);
        if (WRITE && r.dlen) F.copy(q, r, W->name + rel[C_NAMEB]);
        FL_SEP();
    }
    FL_UNKNOWN();
    // photoUrls
    if (more && k8 == KP_PHOTO && (F.ld8(p + 8) & 0xFFFFFFFFFFull) == pack8("ls\":[", 5)) {
        p += 13;
        flags |= PJ_PET_HAS_PHOTOURLS;
        uint32_t u = WRITE ? rel[C_URLS] : 0, ub = WRITE ? rel[C_URLB] : 0;
        if (F.at(p) == ']') p++;
        else {
            for (;;) {
                if (F.at(p) != '"') return PJ_BAIL;
                const uint32_t q = p + 1;
                const Str r = F.str(q);
                if (r.err) return r.err;
                p = r.end + 1;
                n_urls++;
                url_bytes += r.dlen;
                // url k at word 5 + k (n_urls counts it already)
                if (TAPE && n_urls <= TAPE_WORDS - 5) T[4 + n_urls] = tape_str(q, r);
                if (WRITE) {
                    if (r.dlen) F.copy(q, r, W->url + ub);
                    ub += r.dlen;
                    if (F.lead()) W->url_off[u] = W->b_url + ub;
                    u++;
                }
                const int c = F.at(p++);
                if (c == ']') break;
                if (c != ',') return PJ_BAIL;
            }
        }
        FL_SEP();
    }
    FL_UNKNOWN();
    // tags
    if (more && k8 == KP_TAGS) {
        p += 8;
        flags |= PJ_PET_HAS_TAGS;
        uint32_t g = WRITE ? rel[C_TAGS] : 0, gb = WRITE ? rel[C_TAGB] : 0;
        if (F.at(p) == ']') p++;
        else if constexpr (FL::coop) {
            if (F.at(p) != '{') return PJ_BAIL;
            const int e = wave_tags<WRITE>(F, p, n_tags, tag_bytes, W, g, gb);
            if (e) return e;
        } else {
            for (;;) {
                if (F.at(p) != '{') return PJ_BAIL;
                p++;
                int64_t tid;
                uint32_t tfl, nq = 0;
                Str nr{0, 0, 0, false};
                const int e = fsub<VAL>(F, p, tid, tfl, nq, nr);
                if (e) return e;
                const uint32_t tl = (tfl & PJ_SUB_HAS_NAME) ? nr.dlen : 0;
                n_tags++;
                tag_bytes += tl;
                // tag k at words 5 + urls + 2k, + 1 (n_tags counts it already)
                if (TAPE && n_urls + 2 * n_tags <= TAPE_WORDS - 5) {
                    T[3 + n_urls + 2 * n_tags] = (uint64_t)tid;
                    T[4 + n_urls + 2 * n_tags] = (tl ? tape_str(nq, nr) : 0) | ((uint64_t)(tfl & 3) << 49);
                }
                if (WRITE) {
                    if (F.lead()) {
                        W->tag_id[g] = tid;
                        W->tag_flags[g] = (uint8_t)tfl;
                        W->tag_name_off[g] = W->b_tag + gb + tl;
                    }
                    if (tl) F.copy(nq, nr, W->tag_name + gb);
                    gb += tl;
                    g++;
                }
                const int c = F.at(p++);
                if (c == ']') break;
                if (c != ',') return PJ_BAIL;
            }
        }
        FL_SEP();
    }
    FL_UNKNOWN();
    // status
    if (more && k8 == KP_STATUS && (F.ld8(p + 8) & 0xFFFFull) == pack8(":\"", 2)) {
        const uint32_t q = p + 10;
        const Str r = F.str(q);
        if (r.err) return r.err;
        p = r.end + 1;
        if (r.esc) return PJ_BAIL;
        const uint64_t x = F.ld8(q), y = F.ld8(q + 8) & 0xFF;
        if (r.dlen == 9 && x == pack8("availabl", 8) && y == 'e') status = PJ_STATUS_AVAILABLE;
        else if (r.dlen == 7 && (x & 0xFFFFFFFFFFFFFFull) == pack8("pending", 7)) status = PJ_STATUS_PENDING;
        else if (r.dlen == 4 && (x & 0xFFFFFFFFull) == pack8("sold", 4)) status = PJ_STATUS_SOLD;
        else return PJ_REC_BAD_STATUS;                            // the enum's @JsonCreator rejects it
        FL_SEP();
    }
    FL_UNKNOWN();
    if (more) return PJ_BAIL;                                     // repeated or out-of-order key
    if (p + 1 != n) return PJ_BAIL;                               // trailing bytes: general rules
    if (!(flags & PJ_PET_HAS_NAME)) return PJ_REC_MISSING_NAME;   // required (petstore.json:873-876)
    if (!(flags & PJ_PET_HAS_PHOTOURLS)) return PJ_REC_MISSING_PHOTOURLS;
    if (!WRITE) {
        R.name_len = name_len; R.cat_len = cat_len; R.n_urls = n_urls; R.url_bytes = url_bytes;
        R.n_tags = n_tags; R.tag_bytes = tag_bytes;
        if (TAPE) {
            if (n_urls + 2 * n_tags > TAPE_WORDS - 5) return PJ_TAPE_FULL;
            T[0] = (uint64_t)id;
            T[1] = (uint64_t)cat_id;
            T[2] = (uint64_t)flags | ((uint64_t)status << 8) | ((uint64_t)cat_fl << 16) | ((uint64_t)n_urls << 24) |
                   ((uint64_t)n_tags << 32);
        }
    } else if (F.lead()) {
        const uint32_t row = rel[C_PETS];
        W->id[row] = id;
        W->flags[row] = (uint8_t)flags;
        W->status[row] = status;
        W->cat_id[row] = cat_id;
        W->cat_flags[row] = (uint8_t)cat_fl;
        W->name_off[row] = W->b_name + rel[C_NAMEB] + name_len;
        W->cat_name_off[row] = W->b_cat + rel[C_CATB] + cat_len;
        W->photo_off[row] = W->b_urls + rel[C_URLS] + n_urls;
        W->tag_off[row] = W->b_tags + rel[C_TAGS] + n_tags;
    }
    return 0;
}
#undef FL_SEP
#undef FL_UNKNOWN

// Writing a line from its tape: the stores and copies of fline<true>, in the
// same order, without walking the line again.  The first TAPE_PRE words come
// from registers (loaded together, ahead of the tile, by tape_prefetch); the
// rest, for lines with many items, from memory.
constexpr int TAPE_PRE = 12;
__device__ __forceinline__ void tape_prefetch(const Tape &T, uint64_t *w) {
#pragma unroll
    for (int k = 0; k < TAPE_PRE; k++) w[k] = T[k];
}
__device__ __forceinline__ uint64_t tape_word(const Tape &T, const uint64_t *w, uint32_t k) {
    uint64_t v = 0;
#pragma unroll
    for (int j = 3; j < TAPE_PRE; j++) v = k == (uint32_t)j ? w[j] : v;
    return k < (uint32_t)TAPE_PRE ? v : T[k];
}
__device__ __forceinline__ void tape_copy(const FLine &F, uint64_t w, uint8_t *dst) {
    const uint32_t dl = (uint32_t)(w >> 32) & 0xFFFF;
    if (dl) F.copy((uint32_t)w & 0xFFFF, Str{0, (uint32_t)(w >> 16) & 0xFFFF, dl, ((w >> 48) & 1) != 0}, dst);
}
template <bool COPY = true>
__device__ __forceinline__ void tape_write(const FLine &F, const Tape &T, const uint64_t *w, const BlockCols *W,
                                           const uint32_t *rel) {
    const uint64_t M = w[2];
    const uint32_t flags = (uint32_t)M & 0xFF, status = (uint32_t)(M >> 8) & 0xFF, cat_fl = (uint32_t)(M >> 16) & 0xFF;
    const uint32_t nu = (uint32_t)(M >> 24) & 0xFF, nt = (uint32_t)(M >> 32) & 0xFF;
    uint32_t cat_len = 0, name_len = 0;
    if ((flags & PJ_PET_HAS_CATEGORY) && (cat_fl & PJ_SUB_HAS_NAME)) {
        cat_len = (uint32_t)(w[4] >> 32) & 0xFFFF;
        if (COPY) tape_copy(F, w[4], W->cat_name + rel[C_CATB]);
    }
    if (flags & PJ_PET_HAS_NAME) {
        name_len = (uint32_t)(w[3] >> 32) & 0xFFFF;
        if (COPY) tape_copy(F, w[3], W->name + rel[C_NAMEB]);
    }
    uint32_t u = rel[C_URLS], ub = rel[C_URLB];
    for (uint32_t k = 0; k < nu; k++) {
        const uint64_t x = tape_word(T, w, 5 + k);
        if (COPY) tape_copy(F, x, W->url + ub);
        ub += (uint32_t)(x >> 32) & 0xFFFF;
        W->url_off[u] = W->b_url + ub;
        u++;
    }
    uint32_t g = rel[C_TAGS], gb = rel[C_TAGB];
    for (uint32_t k = 0; k < nt; k++) {
        const int64_t tid = (int64_t)tape_word(T, w, 5 + nu + 2 * k);
        const uint64_t x = tape_word(T, w, 6 + nu + 2 * k);
        const uint32_t tfl = (uint32_t)(x >> 49) & 3;
        const uint32_t tl = (tfl & PJ_SUB_HAS_NAME) ? (uint32_t)(x >> 32) & 0xFFFF : 0;
        W->tag_id[g] = tid;
        W->tag_flags[g] = (uint8_t)tfl;
        W->tag_name_off[g] = W->b_tag + gb + tl;
        if (COPY && tl) tape_copy(F, x, W->tag_name + gb);
        gb += tl;
        g++;
    }
    const uint32_t row = rel[C_PETS];
    W->id[row] = (int64_t)w[0];
    W->flags[row] = (uint8_t)flags;
    W->status[row] = (uint8_t)status;
    W->cat_id[row] = (int64_t)w[1];
    W->cat_flags[row] = (uint8_t)cat_fl;
    W->name_off[row] = W->b_name + rel[C_NAMEB] + name_len;
    W->cat_name_off[row] = W->b_cat + rel[C_CATB] + cat_len;
    W->photo_off[row] = W->b_urls + rel[C_URLS] + nu;
    W->tag_off[row] = W->b_tags + rel[C_TAGS] + nt;
}

// The wave-cooperative reading of one long line, out of line so that its
// registers do not add to those of the per-thread path.
template <bool WRITE>
__device__ __noinline__ int fline_wave(const PJ_LDS uint8_t *tile, const PJ_LDS uint64_t *spec, uint32_t s0, uint32_t n, LineRec &R,
                                       const BlockCols *W, const uint32_t *rel) {
    const FLineT<true> F{tile + s0, spec, s0, n};
    return fline<WRITE>(F, R, W, rel);
}

// ---------------------------------------------------------------- tile bitmaps
// Build, for the nw 64-byte words of an LDS tile that starts at a line
// start (or whose first line starts after a newline inside it), the specials
// bitmap (unescaped quotes | backslashes) and a per-word flag for raw control
// characters or malformed UTF-8 inside strings.  Each thread owns a
// contiguous run of words; the in-string carry between runs comes from a
// block scan of (newline seen, quote parity).  With BAD false only the
// specials bitmap is built (one pass, no scan): enough to walk a line known
// to be valid.
template <int BT, bool BAD = true>
__device__ __forceinline__ void tile_bitmaps(const uint8_t *tile, uint32_t nw, uint64_t *spec, uint64_t *qu,
                                             uint64_t *sh) {
    const uint32_t t = threadIdx.x;
    const uint32_t per = (nw + BT - 1) / BT;
    const uint32_t w0 = min(t * per, nw), w1 = min(w0 + per, nw);
    // pass 1: masks, escapes, per-run summary
    uint64_t summ = 0;
    for (uint32_t w = w0; w < w1; w++) {
        const uint4 *q4 = reinterpret_cast<const uint4 *>(tile + 64 * w);
        uint32_t x[16];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint4 v = q4[k];
            x[4 * k] = v.x; x[4 * k + 1] = v.y; x[4 * k + 2] = v.z; x[4 * k + 3] = v.w;
        }
        uint64_t Q = 0, B = 0, N = 0;
#pragma unroll
        for (int k = 0; k < 16; k++) {
            Q |= (uint64_t)zero_bytes4(x[k] ^ 0x22222222u) << (4 * k);
            B |= (uint64_t)zero_bytes4(x[k] ^ 0x5C5C5C5Cu) << (4 * k);
            N |= (uint64_t)zero_bytes4(x[k] ^ 0x0A0A0A0Au) << (4 * k);
        }
        // backslash run ending just before the word (within the tile)
        uint32_t run = 0;
        for (uint32_t j = 64 * w; j > 0 && tile[j - 1] == '\\'; j--) run++;
        uint64_t E = 0;
        if (B) {
            constexpr uint64_t EVEN = 0x5555555555555555ull, ODD = ~EVEN;
            const uint64_t rs = B & ~(B << 1);
            uint64_t rs_e = rs & EVEN, rs_o = rs & ODD;
            if ((run & 1) && (B & 1)) { rs_e &= ~1ull; rs_o |= 1ull; }
            E = (((B + rs_e) & ~B) & ODD) | (((B + rs_o) & ~B) & EVEN);
        }
        if ((run & 1) && !(B & 1)) E |= 1ull;
        const uint64_t Qu = Q & ~E;
        spec[w] = B | Qu;
        qu[w] = N;                                      // newline mask until pass 2, then bad bytes
        uint64_t par;
        if (N) {
            const int last = 63 - __builtin_clzll(N);
            par = last == 63 ? 0 : (__builtin_popcountll(Qu >> (last + 1)) & 1);
        } else par = __builtin_popcountll(Qu) & 1;
        summ = idx_combine(summ, (N ? 2ull : 0ull) | par);
    }
    if constexpr (!BAD) return;
    uint64_t tot;
    const uint64_t carry0 = block_excl_scan_idx<BT>(summ, sh, &tot);
    // pass 2: in-string mask, faults inside strings
    uint64_t cin = carry0 & 1;
    for (uint32_t w = w0; w < w1; w++) {
        const uint64_t Qu = spec[w], N = qu[w];
        const uint32_t *x32 = reinterpret_cast<const uint32_t *>(tile + 64 * w);
        // Qu currently holds B | Qu: strip backslashes again (B bits are never quotes)
        uint64_t Bq = 0;
        uint32_t anyc = 0, anyh = 0;
        uint32_t x[16];
#pragma unroll
        for (int k = 0; k < 16; k++) {
            x[k] = x32[k];
            anyc |= any_lt20(x[k]);
            anyh |= x[k] & 0x80808080u;
            Bq |= (uint64_t)zero_bytes4(x[k] ^ 0x22222222u) << (4 * k);
        }
        const uint64_t Quq = Qu & Bq;                   // the unescaped quotes
        uint64_t s = prefix_xor(Quq) ^ (cin ? ~0ull : 0ull);
        for (uint64_t m = N; m; m &= m - 1) {
            const int p = __builtin_ctzll(m);
            if ((s >> p) & 1) s ^= p == 63 ? 0ull : (~0ull << (p + 1));
        }
        uint64_t bad = 0;
        if (anyc) {
            uint64_t C = 0;
#pragma unroll
            for (int k = 0; k < 16; k++) C |= (uint64_t)lt_bytes4(x[k], 0x20) << (4 * k);
            bad |= C & s;
        }
        uint64_t expect_in = 0;
        if (w > 0) {
            const uint32_t b1 = tile[64 * w - 1], b2 = w * 64 >= 2 ? tile[64 * w - 2] : 0,
                           b3 = w * 64 >= 3 ? tile[64 * w - 3] : 0;
            if (b1 >= 0xC0 && b1 <= 0xDF) expect_in |= 1;
            else if (b1 >= 0xE0 && b1 <= 0xEF) expect_in |= 3;
            else if (b1 >= 0xF0 && b1 <= 0xF7) expect_in |= 7;
            if (b2 >= 0xE0 && b2 <= 0xEF) expect_in |= 1;
            else if (b2 >= 0xF0 && b2 <= 0xF7) expect_in |= 3;
            if (b3 >= 0xF0 && b3 <= 0xF7) expect_in |= 1;
        }
        if (anyh | expect_in) {
            // byte classes of UTF-8, four bytes at a time: each class test
            // lines the relevant bit of every byte up at bit 7
            uint64_t cont = 0, l2 = 0, l3 = 0, l4 = 0, badl = 0;
#pragma unroll
            for (int k = 0; k < 16; k++) {
                const uint32_t v = x[k];
                const uint32_t h7 = v & 0x80808080u, h6 = (v << 1) & 0x80808080u, h5 = (v << 2) & 0x80808080u,
                               h4 = (v << 3) & 0x80808080u, h3 = (v << 4) & 0x80808080u;
                const uint32_t hh = h7 & h6, hhh = hh & h5, hhhh = hhh & h4;
                cont |= (uint64_t)movemask4(h7 & ~h6) << (4 * k);
                l2 |= (uint64_t)movemask4(hh & ~h5) << (4 * k);
                l3 |= (uint64_t)movemask4(hhh & ~h4) << (4 * k);
                l4 |= (uint64_t)movemask4(hhhh & ~h3) << (4 * k);
                badl |= (uint64_t)movemask4(hhhh & h3) << (4 * k);
            }
            const uint64_t expect = (l2 << 1) | (l3 << 1) | (l3 << 2) | (l4 << 1) | (l4 << 2) | (l4 << 3) | expect_in;
            bad |= ((cont ^ expect) | badl) & (s | (s << 1) | cin);
        }
        qu[w] = bad;                                    // the newline mask is no longer needed
        cin = (N >> 63) ? 0 : (s >> 63);               // a newline in the last byte resets
    }
}

// ---------------------------------------------------------------- vector look-back
// Per block PJ_DEC_NCNT words, one per counter, each holding its flag in the
// top two bits (LB_AGG: block aggregate, LB_PRE: inclusive prefix) and the
// value below, so a single load gives a consistent (flag, value) pair and a
// look-back window costs one round trip.  The counters resolve
// independently: a word may already hold its inclusive prefix while another
// word of the same block still holds the aggregate.
constexpr int VLB_STRIDE = PJ_DEC_NCNT;
constexpr uint64_t VLB_VAL = (1ull << 62) - 1;

__device__ __forceinline__ void vlb_publish(uint64_t *st, uint64_t b, const uint64_t *agg, int lane) {
    if (lane < PJ_DEC_NCNT) {
        uint64_t v = 0;
#pragma unroll
        for (int k = 0; k < PJ_DEC_NCNT; k++) v = k == lane ? agg[k] : v;
        lb_store(&st[b * VLB_STRIDE + lane], (b == 0 ? LB_PRE : LB_AGG) | v);
    }
}

// one full wave; returns the exclusive prefixes in excl[] (all lanes) and
// publishes the inclusive ones.  A nonzero limit bounds the wait (wall-clock
// ticks): past it, 1 goes to *gave_up and the prefixes are left at 0.
__device__ __forceinline__ void vlb_resolve(uint64_t *st, uint64_t b, const uint64_t *agg, uint64_t *excl,
                                            uint64_t limit = 0, unsigned long long *gave_up = nullptr) {
    const int l = lane_id();
#pragma unroll
    for (int k = 0; k < PJ_DEC_NCNT; k++) excl[k] = 0;
    if (b == 0) return;
    uint32_t open = (1u << PJ_DEC_NCNT) - 1;            // counters still walking back
    int64_t j = (int64_t)b - 1;
    const uint64_t t0 = limit ? wall_clock64() : 0;
    while (open) {
        const int64_t idx = j - l;
        uint64_t w[PJ_DEC_NCNT];
#pragma unroll
        for (int k = 0; k < PJ_DEC_NCNT; k++) w[k] = idx >= 0 ? lb_load(&st[idx * VLB_STRIDE + k]) : LB_PRE;
        bool wait = false;
#pragma unroll
        for (int k = 0; k < PJ_DEC_NCNT; k++) {
            if (!((open >> k) & 1)) continue;
            const uint64_t isp = __ballot((w[k] >> 62) == 2);
            const int fp = isp ? __builtin_ctzll(isp) : 64;
            const uint64_t need = fp >= 63 ? ~0ull : ((2ull << fp) - 1);
            wait |= (__ballot((w[k] >> 62) == 0) & need) != 0;
        }
        if (wait) {
            if (limit && wall_clock64() - t0 > limit) {
                if (l == 0) __hip_atomic_store(gave_up, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
                for (int k = 0; k < PJ_DEC_NCNT; k++) excl[k] = 0;
                return;
            }
            __builtin_amdgcn_s_sleep(1);
            continue;
        }
#pragma unroll
        for (int k = 0; k < PJ_DEC_NCNT; k++) {
            if (!((open >> k) & 1)) continue;
            const uint64_t isp = __ballot((w[k] >> 62) == 2);
            const int fp = isp ? __builtin_ctzll(isp) : 64;
            excl[k] += wave_sum(l <= fp ? (w[k] & VLB_VAL) : 0);
            if (fp < 64) open &= ~(1u << k);
        }
        j -= 64;
    }
    if (l < PJ_DEC_NCNT) {
        uint64_t v = 0;
#pragma unroll
        for (int k = 0; k < PJ_DEC_NCNT; k++) v = k == l ? excl[k] + agg[k] : v;
        lb_store(&st[b * VLB_STRIDE + l], LB_PRE | v);
    }
}

// ---------------------------------------------------------------- stage 2 kernel
// Tile bytes [a0, a0 + tb) of the input into LDS, zero-padded to whole
// 64-byte words plus 64 bytes; the previous line's bytes in the first chunk
// (before g0) are cleared: no line reads them, and zeros keep them out of the
// string state.  16-byte chunks wholly inside the input go from HBM straight
// into LDS (global_load_lds, 64 chunks per wave instruction, all of a
// thread's chunks in flight at once) when the input is 16-byte aligned; the
// chunk holding the input's end and the zero chunks go through registers.
// All threads; the caller's barrier publishes the tile.
template <int BT>
__device__ __forceinline__ void load_tile(const DecParams &P, uint8_t *tile, uint64_t a0, uint64_t g0, uint64_t tb,
                                          uint32_t nw) {
    const uint32_t t = threadIdx.x, l = t & 63, w = t >> 6;
    const uint32_t nch = (uint32_t)((tb + 15) >> 4), nall = nw * 4;
    const bool aligned = ((uintptr_t)P.in & 15) == 0;
    const uint64_t whole = P.len > a0 ? (P.len - a0) >> 4 : 0;     // chunks that end inside the input
    const uint32_t ndma = aligned ? (uint32_t)min((uint64_t)nch, whole) : 0u;
    for (uint32_t c0 = 64 * w; c0 < ndma; c0 += BT) {
        if (c0 + l < ndma)
            __builtin_amdgcn_global_load_lds(P.in + a0 + 16ull * (c0 + l), (PJ_LDS void *)(tile + 16 * c0), 16, 0, 0);
    }
    for (uint32_t c = ndma + t; c < nall + 4; c += BT) {
        const uint64_t g = a0 + 16ull * c;
        uint4 v = make_uint4(0, 0, 0, 0);
        if (c < nch) {
            if (g + 16 <= P.len) v = *reinterpret_cast<const uint4 *>(P.in + g);
            else {
                uint32_t x[4] = {0, 0, 0, 0};
                for (uint32_t j = 0; j < 16 && g + j < P.len; j++) x[j >> 2] |= (uint32_t)P.in[g + j] << (8 * (j & 3));
                v = make_uint4(x[0], x[1], x[2], x[3]);
            }
        }
        reinterpret_cast<uint4 *>(tile)[c] = v;
    }
    __builtin_amdgcn_s_waitcnt(0);                  // this wave's chunks are in LDS
    if (t == 0 && a0 < g0) {                        // chunk 0 came from wave 0, now complete
        const uint32_t lead = (uint32_t)(g0 - a0);
        for (uint32_t j = 0; j < lead; j++) tile[j] = 0;
    }
}

// The line starts of a block's cnt lines from l0 (and the end of the last)
// into sh_ls, and the block cut into sub-tiles: maximal runs of lines whose
// bytes fit the LDS tile (normally one), their first lines in sh_sub.
// Returns the number of sub-tiles.  All threads.
// With LONG > 0, a block that does not fit the tile whole gives each line
// longer than LONG a sub-tile of its own, marked SUB_SKIP: such lines are
// read elsewhere, so the sub-tile is never loaded.
constexpr uint16_t SUB_SKIP = 0x8000;
template <int TILE, int LONG = 0>
__device__ __forceinline__ uint32_t block_subtiles(const DecParams &P, uint64_t l0, uint32_t cnt, uint64_t *sh_ls,
                                                   uint16_t *sh_sub, uint32_t *sh_nsub) {
    const uint32_t t = threadIdx.x;
    if (t < cnt) sh_ls[t] = P.line_start[l0 + t];
    if (t == 0) sh_ls[cnt] = P.line_start[l0 + cnt];  // the end of the last line (cnt may equal BT)
    __syncthreads();
    if (t == 0) {
        uint32_t j = 0;
        if (min(sh_ls[cnt], P.len) - (sh_ls[0] & ~15ull) <= TILE) sh_sub[j++] = 0;
        else {
            auto is_long = [&](uint32_t k) { return LONG > 0 && sh_ls[k + 1] - 1 - sh_ls[k] > (uint64_t)LONG; };
            for (uint32_t k = 0; k < cnt;) {
                if (is_long(k)) {
                    sh_sub[j++] = (uint16_t)k | SUB_SKIP;
                    k++;
                    continue;
                }
                sh_sub[j++] = (uint16_t)k;
                const uint64_t a = sh_ls[k] & ~15ull;
                uint32_t k2 = k + 1;
                while (k2 < cnt && !is_long(k2) && min(sh_ls[k2 + 1], P.len) - a <= TILE) k2++;
                k = k2;
            }
        }
        sh_sub[j] = (uint16_t)cnt;
        *sh_nsub = j;
    }
    __syncthreads();
    return *sh_nsub;
}

// Whether any thread of the block holds p (all threads call; one LDS word).
__device__ __forceinline__ bool block_any(bool p, uint32_t *flag) {
    if (threadIdx.x == 0) *flag = 0;
    __syncthreads();
    if (__ballot(p) && lane_id() == 0) *flag = 1;
    __syncthreads();
    const bool r = *flag != 0;
    __syncthreads();
    return r;
}

// A bad byte anywhere in the line at tile offset s0 (its newline included).
__device__ __forceinline__ bool line_bad(const uint64_t *badm, uint32_t nw, uint32_t s0, uint32_t n) {
    const uint32_t e = s0 + n;
    bool bad = false;
    for (uint32_t k = s0 >> 6; k <= (e >> 6) && k < nw; k++) {
        uint64_t m = badm[k];
        if (k == (s0 >> 6)) m &= ~0ull << (s0 & 63);
        if (k == (e >> 6)) m &= (e & 63) == 63 ? ~0ull : ((2ull << (e & 63)) - 1);
        bad |= m != 0;
    }
    return bad;
}

// One workgroup per BT consecutive lines, one line per thread, in a single
// pass over the input:
//   * the block's lines are cut into sub-tiles: maximal runs whose bytes fit
//     the LDS tile (normally one); each sub-tile is loaded with coalesced
//     16-byte loads and its bitmaps are built in LDS.  A single line longer
//     than the tile is read from global memory by the byte-by-byte parser;
//   * per line: a raw control character or malformed UTF-8 inside one of its
//     strings makes it invalid whatever else it holds (its error slot is
//     reserved here and k_dec_errcode later finds which error comes first);
//     otherwise the canonical fast path validates and measures it, and lines
//     it does not recognise go through the general parser;
//   * block scans plus a vector look-back over 8 counters give the rows /
//     byte offsets, and a second walk over the sub-tiles (reloaded only when
//     there were several) writes the columns.
// The general parser's measuring walk, out of line: few lines take it, and
// inlined its registers would count against every validating workgroup.
__device__ __noinline__ int run_line_measure(const DecParams &P, const Src S, uint64_t s0, uint32_t n, LineInfo *L) {
    return run_line(P, S, s0, n, true, false, *L, nullptr);
}

// BM false (split decode only): no bitmaps in LDS, so more workgroups share
// a CU.  A line for the wave path (long, or too many items for its tape) is
// deferred: it enters the block's scan with zero counters, goes to
// P.long_list for k_dec_measure_long, and its block joins P.bm_list, whose
// offsets k_dec_fixup then corrects.
template <int BT, int TILE, int LONG, int LPB, bool TAPE, bool BM>
__device__ __forceinline__ void dec_block(DecParams &P, const uint64_t b) {
    static_assert(LONG < 65536, "tape positions of per-thread lines are 16-bit");
    static_assert(BM || TAPE, "blocks without bitmaps hand long lines over (split decode)");
    __shared__ __attribute__((aligned(16))) uint8_t tile[TILE + 64];
    // the specials and bad-byte bitmaps; after pass 0 also the scan's
    // scratch (the only use left without bitmaps)
    constexpr int BMW = BM ? TILE / 64 + 1 : PJ_DEC_NCNT * BT / 128;
    __shared__ __attribute__((aligned(16))) uint64_t bmaps[2 * BMW];
    uint64_t *const spec = bmaps, *const badm = bmaps + BMW;
    __shared__ uint64_t sh_scan[BT / 64];
    __shared__ uint64_t sh_ls[LPB + 1];             // the block's line starts, then its end
    __shared__ uint16_t sh_sub[LPB + 1];            // sub-tile boundaries (block-local line indices)
    __shared__ uint32_t sh_nsub, sh_any, sh_wa, sh_wb;
    __shared__ uint64_t sh_base[PJ_DEC_NCNT];
    const uint32_t t = threadIdx.x;
    const uint64_t l0 = b * LPB;
    const uint32_t cnt = (uint32_t)min((uint64_t)LPB, P.lines - l0);
    const uint64_t l = l0 + t;
    const bool live = t < cnt;
    const uint32_t nsub = block_subtiles<TILE, BM ? 0 : LONG>(P, l0, cnt, sh_ls, sh_sub, &sh_nsub);
    uint64_t gs = 0;
    uint32_t n = 0;
    if (live) {
        gs = sh_ls[t];
        n = (uint32_t)(sh_ls[t + 1] - 1 - gs);
    }
    bool longl = n > (uint32_t)LONG;               // read by the owning wave (also: tape full)
    // ---- pass 0: validate and measure, sub-tile by sub-tile
    LineRec r{0, 0, 0, 0, 0, 0, 0, 0};
    int code = 0;
    bool general = false, bad = false, over = false;
    uint32_t s0 = 0;                                // tile offset of this thread's line
    uint64_t ta0 = 0, ttb = 0;                      // its sub-tile
    for (uint32_t j = 0; j < nsub; j++) {
        if (sh_sub[j] & SUB_SKIP) continue;         // (!BM) one long line: deferred
        const uint32_t ka = sh_sub[j], kb = sh_sub[j + 1] & ~SUB_SKIP;
        const uint64_t g0 = sh_ls[ka], a0 = g0 & ~15ull, g1 = min(sh_ls[kb], P.len), tb = g1 - a0;
        const bool sub_over = tb > TILE;            // one line, longer than the tile
        const bool mine = live && t >= ka && t < kb;
        bool need_gen = false;
        if (!sub_over) {
            const uint32_t nw = (uint32_t)((tb + 63) >> 6);
            load_tile<BT>(P, tile, a0, g0, tb, nw);
            __syncthreads();
            if (P.array_doc) {
                // an element's separator (',' or the closing ']') reads as its newline
                if (mine) tile[gs + n - a0] = '\n';
                __syncthreads();
            }
            if (mine) {
                s0 = (uint32_t)(gs - a0);
                ta0 = a0;
                ttb = tb;
                if (!longl) {
                    // strings are scanned and checked byte class by byte
                    // class as the walk meets them: no bitmaps needed
                    const FLine F{(const PJ_LDS uint8_t *)(tile + s0), nullptr, s0, n};
                    if constexpr (TAPE) code = fline<false, FLine, true>(F, r, nullptr, nullptr, Tape{P.tape + l, P.lines});
                    else code = fline<false>(F, r, nullptr, nullptr);
                    if (TAPE && code == PJ_TAPE_FULL) {
                        longl = true;
                        code = 0;
                    }
                    need_gen = code == PJ_BAIL;
                }
            }
            // long lines: the wave of the owning thread reads them together,
            // over the bitmaps, which only sub-tiles holding one build
            if (BM && block_any(mine && longl, &sh_any)) {
                // only the words of the long lines are read: the bitmaps
                // cover their span (each starts after a newline, where the
                // string state is known)
                if (t == 0) {
                    sh_wa = ~0u;
                    sh_wb = 0;
                }
                __syncthreads();
                if (mine && longl) {
                    atomicMin(&sh_wa, s0 >> 6);
                    atomicMax(&sh_wb, (s0 + n + 64) >> 6);
                }
                __syncthreads();
                const uint32_t wa = sh_wa, wb = min(sh_wb, nw);
                tile_bitmaps<BT>(tile + 64 * wa, wb - wa, spec + wa, badm + wa, sh_scan);
                __syncthreads();
                if (mine && longl) {
                    bad = line_bad(badm, nw, s0, n);
                    if (bad) code = PJ_REC_STRING;  // provisional: k_dec_errcode settles it
                }
            }
            for (uint64_t m = BM ? __ballot(mine && !bad && longl) : 0ull; m; m &= m - 1) {
                const int k = __builtin_ctzll(m);
                const uint32_t ks0 = (uint32_t)__shfl((int)s0, k, 64), kn = (uint32_t)__shfl((int)n, k, 64);
                LineRec rr{0, 0, 0, 0, 0, 0, 0, 0};
                const int cc = fline_wave<false>((const PJ_LDS uint8_t *)tile, (const PJ_LDS uint64_t *)spec, ks0, kn, rr, nullptr, nullptr);
                if (lane_id() == k) {
                    r = rr;
                    code = cc;
                    need_gen = cc == PJ_BAIL;
                }
            }
        } else if (BM && mine) {                    // (!BM: such a line is long, so deferred)
            over = true;
            need_gen = true;
        }
        if (need_gen) {
            // the general parser checks every string byte itself (slow mode)
            general = true;
            const Src S = over ? Src{P.in, P.len, nullptr} : Src{tile, tb, nullptr};
            LineInfo L;
            code = run_line_measure(P, S, over ? gs : s0, n, &L);
            if (!code) {
                r.name_len = L.name_len; r.cat_len = L.has_cat ? L.cat_len : 0; r.n_urls = L.n_urls;
                r.url_bytes = L.url_bytes; r.n_tags = L.n_tags; r.tag_bytes = L.tag_bytes;
            }
        }
        __syncthreads();                            // the tile is reused by the next sub-tile
    }
    const bool defer = !BM && live && longl;
    if constexpr (!BM) {
        if (block_any(defer, &sh_any) && t == 0) P.bm_list[atomicAdd(P.bm_count, 1ull)] = b;
    }
    if (general) atomicAdd(P.gq_count, 1ull);       // diagnostics: lines off the fast path
    r.code = live ? (uint32_t)code : 0;
    if (live && code == PJ_REC_EMPTY) atomicAdd(P.empty_count, 1ull);
    // ---- scans and look-back
    uint64_t v[PJ_DEC_NCNT] = {0, 0, 0, 0, 0, 0, 0, 0};
    if (live && !defer) rec_counts(r, v);
    uint32_t pos[PJ_DEC_NCNT];                      // block-relative: a block's columns stay below 2^32 bytes
    uint64_t agg[PJ_DEC_NCNT];
    {
        uint32_t v32[PJ_DEC_NCNT], a32[PJ_DEC_NCNT];
#pragma unroll
        for (int k = 0; k < PJ_DEC_NCNT; k++) v32[k] = (uint32_t)v[k];
        // the bad-byte bitmap is not read after pass 0: its words hold the scan
        block_excl_scan_n<BT, PJ_DEC_NCNT>(v32, pos, a32, reinterpret_cast<uint32_t *>(badm));
#pragma unroll
        for (int k = 0; k < PJ_DEC_NCNT; k++) agg[k] = a32[k];
    }
    if constexpr (TAPE) {
        // split decode: the block's offsets and totals go to memory, and the
        // scan and the writer kernels take it from there (no waiting here)
        if (live) {
            const uint64_t L = P.lines;
#pragma unroll
            for (int k = 0; k < PJ_DEC_NCNT; k++) P.lpos[k * L + l] = pos[k];
            const bool wave = longl && !general && !bad && code == 0;
            P.lpos[PJ_DEC_NCNT * L + l] = defer ? LK_DEFER
                                                : (uint32_t)code | (general ? LK_GENERAL : 0u) | (wave ? LK_WAVE : 0u) |
                                                      (bad ? LK_BAD : 0u);
            // lines of the whole wave or the general parser are written by
            // k_dec_long (deferred ones once k_dec_measure_long has read them)
            if (defer || (code == 0 && (wave || general))) P.long_list[atomicAdd(P.long_count, 1ull)] = l;
        }
        if (t < PJ_DEC_NCNT) {
            uint64_t x = 0;
#pragma unroll
            for (int k = 0; k < PJ_DEC_NCNT; k++) x = k == (int)t ? agg[k] : x;
            P.bagg[b * PJ_DEC_NCNT + t] = x;
        }
        return;
    }
    if (t < 64) {
        vlb_publish(P.state_parse, b, agg, (int)t);
        uint64_t excl[PJ_DEC_NCNT];
        vlb_resolve(P.state_parse, b, agg, excl, P.order_by_id ? P.spin_limit : 0, &P.tickets[1]);
        if (t < PJ_DEC_NCNT) {
            uint64_t x = 0, y = 0;
#pragma unroll
            for (int k = 0; k < PJ_DEC_NCNT; k++) {
                x = k == (int)t ? excl[k] : x;
                y = k == (int)t ? excl[k] + agg[k] : y;
            }
            sh_base[t] = x;
            if (b == gridDim.x - 1) P.totals[t] = y;
        }
    }
    __syncthreads();
    const pj_pet_columns &o = P.o;
    if (b == 0 && t == 0) {
        o.name_off[0] = 0; o.cat_name_off[0] = 0; o.photo_off[0] = 0; o.tag_off[0] = 0;
        o.url_off[0] = 0; o.tag_name_off[0] = 0;
    }
    uint64_t base[PJ_DEC_NCNT];
#pragma unroll
    for (int k = 0; k < PJ_DEC_NCNT; k++) base[k] = uniform_u64(sh_base[k]);
    if (live && code) {
        const uint64_t e = base[C_ERRS] + pos[C_ERRS];
        if (e < P.err_cap) {
            P.err_line[e] = l;
            P.err_code[e] = (uint8_t)code;
            if (bad) P.dq[atomicAdd(P.dq_count, 1ull)] = e;
        }
    }
    // ---- pass 1: materialise.  One capacity check per block: a block
    // whose slice of some column would not fit writes nothing (the call then
    // reports PJ_ERR_CAPACITY).
    const bool room = base[C_PETS] + agg[C_PETS] <= o.cap_pets && base[C_NAMEB] + agg[C_NAMEB] <= o.cap_name_bytes &&
                      base[C_CATB] + agg[C_CATB] <= o.cap_cat_name_bytes && base[C_URLS] + agg[C_URLS] <= o.cap_urls &&
                      base[C_URLB] + agg[C_URLB] <= o.cap_url_bytes && base[C_TAGS] + agg[C_TAGS] <= o.cap_tags &&
                      base[C_TAGB] + agg[C_TAGB] <= o.cap_tag_name_bytes;
    if (!room) return;
    BlockCols W;
    W.id = o.id + base[C_PETS]; W.flags = o.flags + base[C_PETS]; W.status = o.status + base[C_PETS];
    W.cat_id = o.cat_id + base[C_PETS]; W.cat_flags = o.cat_flags + base[C_PETS];
    W.name_off = o.name_off + base[C_PETS] + 1; W.cat_name_off = o.cat_name_off + base[C_PETS] + 1;
    W.photo_off = o.photo_off + base[C_PETS] + 1; W.tag_off = o.tag_off + base[C_PETS] + 1;
    W.url_off = o.url_off + base[C_URLS] + 1; W.tag_name_off = o.tag_name_off + base[C_TAGS] + 1;
    W.tag_id = o.tag_id + base[C_TAGS]; W.tag_flags = o.tag_flags + base[C_TAGS];
    W.name = o.name_bytes + base[C_NAMEB]; W.cat_name = o.cat_name_bytes + base[C_CATB];
    W.url = o.url_bytes + base[C_URLB]; W.tag_name = o.tag_name_bytes + base[C_TAGB];
    W.b_name = base[C_NAMEB]; W.b_cat = base[C_CATB]; W.b_urls = base[C_URLS]; W.b_url = base[C_URLB];
    W.b_tags = base[C_TAGS]; W.b_tag = base[C_TAGB];
    const bool writer = live && code == 0;
    for (uint32_t j = 0; j < nsub; j++) {
        const uint32_t ka = sh_sub[j], kb = sh_sub[j + 1];
        const uint64_t g0 = sh_ls[ka], a0 = g0 & ~15ull, g1 = min(sh_ls[kb], P.len), tb = g1 - a0;
        const bool sub_over = tb > TILE;
        const bool wmine = writer && t >= ka && t < kb;
        if (nsub > 1 && !sub_over) {                // a single sub-tile is still in LDS (with its bitmaps)
            const uint32_t nw = (uint32_t)((tb + 63) >> 6);
            load_tile<BT>(P, tile, a0, g0, tb, nw);
            __syncthreads();
            if (block_any(wmine && !general && longl, &sh_any)) tile_bitmaps<BT>(tile, nw, spec, badm, sh_scan);
            __syncthreads();
        }
        for (uint64_t m = __ballot(wmine && !general && longl); m; m &= m - 1) {
            const int k = __builtin_ctzll(m);
            uint32_t rel[PJ_DEC_NCNT];
#pragma unroll
            for (int c = 0; c < PJ_DEC_NCNT; c++) rel[c] = (uint32_t)__shfl((int)pos[c], k, 64);
            const uint32_t ks0 = (uint32_t)__shfl((int)s0, k, 64), kn = (uint32_t)__shfl((int)n, k, 64);
            const BlockCols Wc = W;                 // addressable copy, made only on this path
            fline_wave<true>((const PJ_LDS uint8_t *)tile, (const PJ_LDS uint64_t *)spec, ks0, kn, r, &Wc, rel);
        }
        if (wmine && !(longl && !general)) {
            if (!general) {
                uint32_t rel[PJ_DEC_NCNT];
#pragma unroll
                for (int k = 0; k < PJ_DEC_NCNT; k++) rel[k] = pos[k];
                const FLine F{(const PJ_LDS uint8_t *)(tile + s0), nullptr, s0, n};
                if constexpr (TAPE) {
                    uint64_t tw[TAPE_PRE];
                    tape_prefetch(Tape{P.tape + l, P.lines}, tw);
                    tape_write(F, Tape{P.tape + l, P.lines}, tw, &W, rel);
                }
                else fline<true>(F, r, &W, rel);
            } else {
                uint64_t gp[PJ_DEC_NCNT];
#pragma unroll
                for (int k = 0; k < PJ_DEC_NCNT; k++) gp[k] = pos[k] + base[k];
                const Src S = over ? Src{P.in, P.len, nullptr} : Src{tile, ttb, nullptr};
                // the measuring walk again (cheaper than keeping its positions
                // in registers across the look-back), then the writing walk
                LineInfo L;
                run_line(P, S, over ? gs : s0, n, true, false, L, nullptr);
                run_line(P, S, over ? gs : s0, n, true, true, L, gp);
            }
        }
        if (nsub > 1) __syncthreads();
    }
    (void)ta0;
}

template <int BT, int TILE, int LONG, int LPB = BT, bool TAPE = false, bool BM = true>
__global__ __launch_bounds__(BT, BM ? 2 : 3) void k_dec_block(DecParams P) {
    __shared__ uint64_t sh_blk;
    if (threadIdx.x == 0) sh_blk = P.order_by_id ? (uint64_t)blockIdx.x : atomicAdd(&P.tickets[1], 1ull);
    __syncthreads();
    dec_block<BT, TILE, LONG, LPB, TAPE, BM>(P, sh_blk);
}

// The lines the bitmap-free pass deferred, one 64-thread workgroup per line
// at a time: the line is tiled into LDS with its bitmaps, checked for bad
// bytes and read by the wave-parallel walk (a line longer than the tile, or
// one the walk does not recognise, by the general parser on one thread).
// Its 8 counters go to tape words 0-7, its code and kind to its info word;
// LK_DEFER stays set for k_dec_fixup.
template <int TILE>
__global__ __launch_bounds__(64) void k_dec_measure_long(DecParams P) {
    __shared__ __attribute__((aligned(16))) uint8_t tile[TILE + 64];
    __shared__ uint64_t spec[TILE / 64 + 1];
    __shared__ uint64_t badm[TILE / 64 + 1];
    __shared__ uint64_t sh_scan[1];
    const uint64_t cnt = *P.long_count, L = P.lines;
    const uint32_t t = threadIdx.x;
    for (uint64_t i = blockIdx.x; i < cnt; i += gridDim.x) {
        const uint64_t l = P.long_list[i];
        const uint32_t info = __builtin_amdgcn_readfirstlane(P.lpos[PJ_DEC_NCNT * L + l]);
        if (!(info & LK_DEFER)) continue;           // a general line of the validating pass
        const uint64_t gs = P.line_start[l], ge = P.line_start[l + 1];
        const uint32_t n = (uint32_t)(ge - 1 - gs);
        const uint64_t a0 = gs & ~15ull, tb = min(ge, P.len) - a0;
        const uint32_t s0 = (uint32_t)(gs - a0);
        LineRec r{0, 0, 0, 0, 0, 0, 0, 0};
        int code = 0;
        bool general = false, bad = false;
        LineInfo Li;
        if (tb > TILE) {
            general = true;
            if (t == 0) code = run_line_measure(P, Src{P.in, P.len, nullptr}, gs, n, &Li);
        } else {
            const uint32_t nw = (uint32_t)((tb + 63) >> 6);
            load_tile<64>(P, tile, a0, gs, tb, nw);
            __syncthreads();
            if (P.array_doc && t == 0) tile[s0 + n] = '\n';
            __syncthreads();
            tile_bitmaps<64>(tile, nw, spec, badm, sh_scan);
            __syncthreads();
            bad = line_bad(badm, nw, s0, n);
            if (bad) code = PJ_REC_STRING;          // provisional: k_dec_errcode settles it
            else {
                code = fline_wave<false>((const PJ_LDS uint8_t *)tile, (const PJ_LDS uint64_t *)spec, s0, n, r, nullptr, nullptr);
                if (code == PJ_BAIL) {
                    general = true;
                    if (t == 0) code = run_line_measure(P, Src{tile, tb, nullptr}, s0, n, &Li);
                }
            }
        }
        if (t == 0) {
            if (general && !code) {
                r.name_len = Li.name_len; r.cat_len = Li.has_cat ? Li.cat_len : 0; r.n_urls = Li.n_urls;
                r.url_bytes = Li.url_bytes; r.n_tags = Li.n_tags; r.tag_bytes = Li.tag_bytes;
            }
            r.code = (uint32_t)code;
            uint64_t v[PJ_DEC_NCNT];
            rec_counts(r, v);
#pragma unroll
            for (int k = 0; k < PJ_DEC_NCNT; k++) P.tape[k * L + l] = v[k];
            const bool wave = !general && !bad && code == 0;
            P.lpos[PJ_DEC_NCNT * L + l] = (uint32_t)code | LK_DEFER | (general ? LK_GENERAL : 0u) |
                                          (wave ? LK_WAVE : 0u) | (bad ? LK_BAD : 0u);
            if (general) atomicAdd(P.gq_count, 1ull);
        }
        __syncthreads();                            // the tile is reused by the next line
    }
}

// The blocks holding deferred lines: each line's offsets inside its block
// gain the counters of the deferred lines before it, and the block's totals
// gain theirs.  Runs after k_dec_measure_long, before the block scan.
template <int BT, int LPB>
__global__ __launch_bounds__(BT) void k_dec_fixup(DecParams P) {
    static_assert(LPB <= BT, "one line per thread");
    __shared__ uint32_t sh_scan[PJ_DEC_NCNT * (BT / 64)];
    const uint64_t cnt = *P.bm_count, L = P.lines;
    const uint32_t t = threadIdx.x;
    for (uint64_t i = blockIdx.x; i < cnt; i += gridDim.x) {
        const uint64_t b = P.bm_list[i], l0 = b * LPB, l = l0 + t;
        const bool live = t < LPB && l < L;
        const uint32_t info = live ? P.lpos[PJ_DEC_NCNT * L + l] : 0u;
        const bool def = (info & LK_DEFER) != 0;
        uint32_t v[PJ_DEC_NCNT], ex[PJ_DEC_NCNT], tot[PJ_DEC_NCNT];
#pragma unroll
        for (int k = 0; k < PJ_DEC_NCNT; k++) v[k] = def ? (uint32_t)P.tape[k * L + l] : 0u;
        block_excl_scan_n<BT, PJ_DEC_NCNT>(v, ex, tot, sh_scan);
        if (live) {
#pragma unroll
            for (int k = 0; k < PJ_DEC_NCNT; k++)
                if (ex[k]) P.lpos[k * L + l] += ex[k];
        }
        if (t < PJ_DEC_NCNT) {
            uint64_t x = 0;
#pragma unroll
            for (int k = 0; k < PJ_DEC_NCNT; k++) x = k == (int)t ? tot[k] : x;
            P.bagg[b * PJ_DEC_NCNT + t] += x;
        }
    }
}

// ---------------------------------------------------------------- split decode writers
// A line block's slices of the output columns, from the block's first
// offsets.
__device__ __forceinline__ BlockCols block_cols(const pj_pet_columns &o, const uint64_t *base) {
    BlockCols W;
    W.id = o.id + base[C_PETS]; W.flags = o.flags + base[C_PETS]; W.status = o.status + base[C_PETS];
    W.cat_id = o.cat_id + base[C_PETS]; W.cat_flags = o.cat_flags + base[C_PETS];
    W.name_off = o.name_off + base[C_PETS] + 1; W.cat_name_off = o.cat_name_off + base[C_PETS] + 1;
    W.photo_off = o.photo_off + base[C_PETS] + 1; W.tag_off = o.tag_off + base[C_PETS] + 1;
    W.url_off = o.url_off + base[C_URLS] + 1; W.tag_name_off = o.tag_name_off + base[C_TAGS] + 1;
    W.tag_id = o.tag_id + base[C_TAGS]; W.tag_flags = o.tag_flags + base[C_TAGS];
    W.name = o.name_bytes + base[C_NAMEB]; W.cat_name = o.cat_name_bytes + base[C_CATB];
    W.url = o.url_bytes + base[C_URLB]; W.tag_name = o.tag_name_bytes + base[C_TAGB];
    W.b_name = base[C_NAMEB]; W.b_cat = base[C_CATB]; W.b_urls = base[C_URLS]; W.b_url = base[C_URLB];
    W.b_tags = base[C_TAGS]; W.b_tag = base[C_TAGB];
    return W;
}

// Do the call's totals fit the output capacities?  (Nothing is written
// otherwise: the call reports PJ_ERR_CAPACITY with the sizes it needs.)
__device__ __forceinline__ bool dec_room(const DecParams &P) {
    const pj_pet_columns &o = P.o;
    const uint64_t *T = P.totals;
    return T[C_PETS] <= o.cap_pets && T[C_NAMEB] <= o.cap_name_bytes && T[C_CATB] <= o.cap_cat_name_bytes &&
           T[C_URLS] <= o.cap_urls && T[C_URLB] <= o.cap_url_bytes && T[C_TAGS] <= o.cap_tags &&
           T[C_TAGB] <= o.cap_tag_name_bytes;
}

// Scan of the validating kernel's block totals: BT blocks per workgroup,
// workgroups in ticket order chained by the vector look-back; bbase gets
// each line block's first offsets, totals the call's sums.
template <int BT>
__global__ __launch_bounds__(BT) void k_dec_bscan(DecParams P) {
    __shared__ uint64_t sh_scan[BT / 64];
    __shared__ uint64_t sh_sb, sh_pre[PJ_DEC_NCNT];
    const uint32_t t = threadIdx.x;
    if (t == 0) sh_sb = atomicAdd(P.bticket, 1ull);
    __syncthreads();
    const uint64_t sb = sh_sb, i = sb * BT + t;
    const bool in = i < P.nblocks;
    uint64_t excl[PJ_DEC_NCNT], agg[PJ_DEC_NCNT];
#pragma unroll
    for (int k = 0; k < PJ_DEC_NCNT; k++)
        excl[k] = block_excl_scan<BT>(in ? P.bagg[i * PJ_DEC_NCNT + k] : 0ull, sh_scan, &agg[k]);
    if (t < 64) {
        vlb_publish(P.bstate, sb, agg, (int)t);
        uint64_t pre[PJ_DEC_NCNT];
        vlb_resolve(P.bstate, sb, agg, pre);
        if (t < PJ_DEC_NCNT) {
            uint64_t x = 0;
#pragma unroll
            for (int k = 0; k < PJ_DEC_NCNT; k++) x = k == (int)t ? pre[k] : x;
            sh_pre[t] = x;
            if ((sb + 1) * BT >= P.nblocks) {
                uint64_t y = 0;
#pragma unroll
                for (int k = 0; k < PJ_DEC_NCNT; k++) y = k == (int)t ? pre[k] + agg[k] : y;
                P.totals[t] = y;
            }
        }
    }
    __syncthreads();
    if (in) {
#pragma unroll
        for (int k = 0; k < PJ_DEC_NCNT; k++) P.bbase[i * PJ_DEC_NCNT + k] = sh_pre[k] + excl[k];
    }
}

// Writer of the split decode, one workgroup per line block of the
// validating kernel: the block's lines are tiled into LDS again (the same
// sub-tiles), and each thread writes its fast-path line from its tape at the
// offsets the scan gave.  Invalid lines get their error slot; lines of the
// whole wave or the general parser are left to k_dec_long.
template <int BT, int TILE, int LPB, int LONG>
__global__ __launch_bounds__(BT, 2) void k_dec_write(DecParams P) {
    __shared__ __attribute__((aligned(16))) uint8_t tile[TILE + 64];
    __shared__ uint64_t sh_ls[LPB + 1];
    __shared__ uint16_t sh_sub[LPB + 1];
    __shared__ uint32_t sh_nsub;
    const uint32_t t = threadIdx.x;
    const uint64_t L = P.lines, b = blockIdx.x, l0 = b * LPB;
    const uint32_t cnt = (uint32_t)min((uint64_t)LPB, L - l0);
    const uint64_t l = l0 + t;
    const bool live = t < cnt;
    const pj_pet_columns &o = P.o;
    const uint32_t nsub = block_subtiles<TILE, LONG>(P, l0, cnt, sh_ls, sh_sub, &sh_nsub);
    if (b == 0 && t == 0) {
        o.name_off[0] = 0; o.cat_name_off[0] = 0; o.photo_off[0] = 0; o.tag_off[0] = 0;
        o.url_off[0] = 0; o.tag_name_off[0] = 0;
    }
    uint32_t info = 0, rel[PJ_DEC_NCNT];
    uint64_t base[PJ_DEC_NCNT];
#pragma unroll
    for (int k = 0; k < PJ_DEC_NCNT; k++) {
        base[k] = P.bbase[b * PJ_DEC_NCNT + k];
        rel[k] = live ? P.lpos[k * L + l] : 0u;
    }
    if (live) info = P.lpos[PJ_DEC_NCNT * L + l];
    const uint32_t code = info & 0xFF;
    if (live && code) {
        const uint64_t e = base[C_ERRS] + rel[C_ERRS];
        if (e < P.err_cap) {
            P.err_line[e] = l;
            P.err_code[e] = (uint8_t)code;
            if (info & LK_BAD) P.dq[atomicAdd(P.dq_count, 1ull)] = e;
        }
    }
    if (!dec_room(P)) return;
    const bool fastl = live && code == 0 && !(info & (LK_WAVE | LK_GENERAL));
    uint64_t gs = 0;
    uint32_t n = 0;
    if (live) {
        gs = sh_ls[t];
        n = (uint32_t)(sh_ls[t + 1] - 1 - gs);
    }
    // the tape's first words, in flight while the tile loads
    uint64_t tw[TAPE_PRE];
    if (fastl) tape_prefetch(Tape{P.tape + l, L}, tw);
    for (uint32_t j = 0; j < nsub; j++) {
        if (sh_sub[j] & SUB_SKIP) continue;         // one long line: written by k_dec_long
        const uint32_t ka = sh_sub[j], kb = sh_sub[j + 1] & ~SUB_SKIP;
        const uint64_t g0 = sh_ls[ka], a0 = g0 & ~15ull, g1 = min(sh_ls[kb], P.len), tb = g1 - a0;
        if (tb <= TILE) {                           // a longer sub-tile is one line of the general parser
            load_tile<BT>(P, tile, a0, g0, tb, (uint32_t)((tb + 63) >> 6));
            __syncthreads();
        }
        const uint32_t s0 = (uint32_t)(gs - a0);
        if (fastl && t >= ka && t < kb) {
            const BlockCols W = block_cols(o, base);
            const FLine F{(const PJ_LDS uint8_t *)(tile + s0), nullptr, s0, n};
            tape_write(F, Tape{P.tape + l, L}, tw, &W, rel);
        }
        if (nsub > 1) __syncthreads();              // the tile is reused by the next sub-tile
    }
}

// Lines read by a whole wave (long lines, and lines with more items than
// the tape holds), one 64-thread workgroup per line at a time: the line is
// tiled into LDS with its bitmaps and written by the wave-parallel walk.
// Lines of the general parser are read again from the input by one thread.
template <int TILE, int LPB>
__global__ __launch_bounds__(64) void k_dec_long(DecParams P) {
    __shared__ __attribute__((aligned(16))) uint8_t tile[TILE + 64];
    __shared__ uint64_t spec[TILE / 64 + 1];
    __shared__ uint64_t badm[TILE / 64 + 1];
    __shared__ uint64_t sh_scan[1];
    const uint64_t cnt = *P.long_count;
    if (!dec_room(P)) return;
    const pj_pet_columns &o = P.o;
    const uint64_t L = P.lines;
    for (uint64_t i = blockIdx.x; i < cnt; i += gridDim.x) {
        const uint64_t l = P.long_list[i];
        const uint64_t gs = P.line_start[l], ge = P.line_start[l + 1];
        const uint32_t n = (uint32_t)(ge - 1 - gs);
        const uint32_t info = __builtin_amdgcn_readfirstlane(P.lpos[PJ_DEC_NCNT * L + l]);
        if (info & 0xFF) continue;                  // a deferred line found invalid
        if (info & LK_GENERAL) {
            // the general parser, from the input (the measuring walk, then the writing walk)
            if (threadIdx.x == 0) {
                uint64_t gp[PJ_DEC_NCNT];
#pragma unroll
                for (int k = 0; k < PJ_DEC_NCNT; k++) gp[k] = P.bbase[(l / LPB) * PJ_DEC_NCNT + k] + P.lpos[k * L + l];
                const Src S{P.in, P.len, nullptr};
                LineInfo Li;
                run_line(P, S, gs, n, true, false, Li, nullptr);
                run_line(P, S, gs, n, true, true, Li, gp);
            }
            continue;
        }
        const uint64_t a0 = gs & ~15ull, tb = min(ge, P.len) - a0;
        const uint32_t nw = (uint32_t)((tb + 63) >> 6);
        load_tile<64>(P, tile, a0, gs, tb, nw);
        __syncthreads();
        if (P.array_doc && threadIdx.x == 0) tile[gs + n - a0] = '\n';
        __syncthreads();
        tile_bitmaps<64, false>(tile, nw, spec, badm, sh_scan);  // the line is valid: specials only
        __syncthreads();
        const uint64_t pb = l / LPB;
        uint64_t base[PJ_DEC_NCNT];
        uint32_t rel[PJ_DEC_NCNT];
#pragma unroll
        for (int k = 0; k < PJ_DEC_NCNT; k++) {
            base[k] = uniform_u64(P.bbase[pb * PJ_DEC_NCNT + k]);
            rel[k] = __builtin_amdgcn_readfirstlane(P.lpos[k * L + l]);
        }
        BlockCols W;
        W.id = o.id + base[C_PETS]; W.flags = o.flags + base[C_PETS]; W.status = o.status + base[C_PETS];
        W.cat_id = o.cat_id + base[C_PETS]; W.cat_flags = o.cat_flags + base[C_PETS];
        W.name_off = o.name_off + base[C_PETS] + 1; W.cat_name_off = o.cat_name_off + base[C_PETS] + 1;
        W.photo_off = o.photo_off + base[C_PETS] + 1; W.tag_off = o.tag_off + base[C_PETS] + 1;
        W.url_off = o.url_off + base[C_URLS] + 1; W.tag_name_off = o.tag_name_off + base[C_TAGS] + 1;
        W.tag_id = o.tag_id + base[C_TAGS]; W.tag_flags = o.tag_flags + base[C_TAGS];
        W.name = o.name_bytes + base[C_NAMEB]; W.cat_name = o.cat_name_bytes + base[C_CATB];
        W.url = o.url_bytes + base[C_URLB]; W.tag_name = o.tag_name_bytes + base[C_TAGB];
        W.b_name = base[C_NAMEB]; W.b_cat = base[C_CATB]; W.b_urls = base[C_URLS]; W.b_url = base[C_URLB];
        W.b_tags = base[C_TAGS]; W.b_tag = base[C_TAGB];
        LineRec r{0, 0, 0, 0, 0, 0, 0, 0};
        fline_wave<true>((const PJ_LDS uint8_t *)tile, (const PJ_LDS uint64_t *)spec, (uint32_t)(gs - a0), n, r, &W, rel);
        __syncthreads();                            // the tile is reused by the next line
    }
}

// ---------------------------------------------------------------- error codes
// Lines found invalid from the bitmaps: a raw control character or malformed
// UTF-8 inside one of their strings.  The line's code is that of the first
// error reading left to right.  Every byte before the first bad byte p is
// valid where it stands, and p lies inside a string, so that error is the
// first error met in the line cut short at p: an error
// before p keeps its code, and otherwise the string holding p runs past the
// cut, which is PJ_REC_STRING, the code the bad byte gives (a line whose
// only bad byte is its terminator, in an unterminated string, is cut at its
// end).  The cut line is read by the wave-parallel walk over the tile's
// specials bitmap, which returns the codes the serial walk returns; the
// shapes it leaves to the general parser are read on one thread, strings
// skipped through the same bitmap rather than byte by byte.  One workgroup per
// queued line at a time (grid-stride over the queue, whose length every
// thread reads after the parse kernel has finished): the line is tiled, its
// bitmaps built, p found, and one thread parses.  A line longer than the
// tile goes through the byte-by-byte parser from global memory.
template <int BT, int TILE>
__global__ __launch_bounds__(BT) void k_dec_errcode(DecParams P) {
    __shared__ __attribute__((aligned(16))) uint8_t tile[TILE + 64];
    __shared__ uint64_t spec[TILE / 64 + 1];
    __shared__ uint64_t badm[TILE / 64 + 1];
    __shared__ uint64_t sh_scan[1];
    __shared__ uint32_t sh_cut;
    const uint64_t cnt = *P.dq_count;
    const uint32_t t = threadIdx.x;
    for (uint64_t i = blockIdx.x; i < cnt; i += gridDim.x) {
        const uint64_t e = P.dq[i];
        const uint64_t l = P.err_line[e];
        const uint64_t gs = P.line_start[l], ge = P.line_start[l + 1];
        const uint32_t n = (uint32_t)(ge - 1 - gs);
        const uint64_t a0 = gs & ~15ull, tb = min(ge, P.len) - a0;
        const uint32_t s0 = (uint32_t)(gs - a0);
        if (tb > TILE) {
            if (t == 0) {
                LineInfo L;
                P.err_code[e] = (uint8_t)run_line(P, Src{P.in, P.len, nullptr}, gs, n, true, false, L, nullptr);
            }
            continue;
        }
        const uint32_t nw = (uint32_t)((tb + 63) >> 6);
        load_tile<BT>(P, tile, a0, gs, tb, nw);
        __syncthreads();
        if (P.array_doc && t == 0) tile[s0 + n] = '\n';
        if (t == 0) sh_cut = n;
        __syncthreads();
        tile_bitmaps<BT>(tile, nw, spec, badm, sh_scan);
        __syncthreads();
        // the first bad byte of the line
        for (uint32_t k = (s0 >> 6) + t; k <= ((s0 + n) >> 6) && k < nw; k += BT) {
            uint64_t m = badm[k];
            if (k == (s0 >> 6)) m &= ~0ull << (s0 & 63);
            if (m) {
                const uint32_t at = 64 * k + (uint32_t)__builtin_ctzll(m);
                if (at < s0 + n) atomicMin(&sh_cut, at - s0);
            }
        }
        __syncthreads();
        // (a line whose only bad byte is its terminator, an unterminated
        // string, is read whole: it holds no bad byte)
        const uint32_t cut = sh_cut, ce = s0 + cut;
        // nothing past the cut is seen: its specials are dropped
        for (uint32_t k = (ce >> 6) + t; k < nw; k += BT) spec[k] &= k == (ce >> 6) ? ~(~0ull << (ce & 63)) : 0ull;
        __syncthreads();
        // the wave-parallel walk (the cut line holds no bad byte); the shapes
        // it leaves to the general parser, on one thread
        LineRec r{0, 0, 0, 0, 0, 0, 0, 0};
        int code = fline_wave<false>((const PJ_LDS uint8_t *)tile, (const PJ_LDS uint64_t *)spec, s0, cut, r, nullptr, nullptr);
        if (t == 0) {
            if (code == PJ_BAIL) {
                LineInfo L;
                code = run_line(P, Src{tile, tb, spec}, s0, cut, false, false, L, nullptr);
            }
            P.err_code[e] = (uint8_t)code;
        }
        __syncthreads();                            // the tile is reused by the next line
    }
}

}  // namespace pj

#ifndef PJ_DEC_LINE_BT
#define PJ_DEC_LINE_BT 128
#endif
#ifndef PJ_DEC_TILE_KB
#define PJ_DEC_TILE_KB 31
#endif
#ifndef PJ_DEC_LONG
#define PJ_DEC_LONG 1024
#endif
constexpr int DEC_LONG = PJ_DEC_LONG;
#ifndef PJ_DEC_IDX_R
#define PJ_DEC_IDX_R 4
#endif
constexpr int DEC_IDX_BT = 256, DEC_IDX_R = PJ_DEC_IDX_R, DEC_LINE_BT = PJ_DEC_LINE_BT, DEC_TILE = PJ_DEC_TILE_KB * 1024;
// The writer's tile: 30 KiB keeps its LDS under 32 KiB, so five workgroups
// share a CU instead of four (measured 11% faster; its blocks are cut into
// sub-tiles by the same rule, and no fast line comes near the size).
#ifndef PJ_DEC_WTILE_KB
#define PJ_DEC_WTILE_KB 30
#endif
constexpr int DEC_WTILE = PJ_DEC_WTILE_KB * 1024;
// The bitmap-free validating pass: 30 KiB keeps it under 32 KiB of LDS.
constexpr int DEC_FTILE = PJ_DEC_WTILE_KB * 1024;
static_assert(DEC_WTILE >= 4 * PJ_DEC_LONG, "fast lines (at most DEC_LONG bytes) fit the writer's tile");

int pj_dec_index_block() { return DEC_IDX_BT * DEC_IDX_R; }
#ifndef PJ_DEC_LPB
#define PJ_DEC_LPB 104
#endif
constexpr int DEC_LPB = PJ_DEC_LPB;
int pj_dec_parse_block() { return DEC_LPB; }

namespace pj {
// Sets *flag when some line block spans PJ_DEC_MAX_BLOCK_SPAN bytes or more.
__global__ void k_dec_span_check(const uint64_t *ls, uint64_t lines, uint64_t lpb, uint64_t *flag) {
    const uint64_t b = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (!dec_block_span_ok(ls, lines, lpb, b)) *flag = 1;
}
}  // namespace pj

hipError_t pj_launch_dec_span_check(const DecParams &P, uint64_t *flag, hipStream_t st) {
    const uint64_t nb = (P.lines + DEC_LPB - 1) / DEC_LPB;
    if (!nb) return hipSuccess;
    hipLaunchKernelGGL(pj::k_dec_span_check, dim3((unsigned)((nb + 255) / 256)), dim3(256), 0, st, P.line_start,
                       P.lines, (uint64_t)DEC_LPB, flag);
    return hipGetLastError();
}

hipError_t pj_launch_dec_index(const DecParams &P, hipStream_t st) {
    const uint64_t g = (P.nblk64 + DEC_IDX_BT * DEC_IDX_R - 1) / (DEC_IDX_BT * DEC_IDX_R);
    hipLaunchKernelGGL((pj::k_dec_lines<DEC_IDX_BT, DEC_IDX_R>), dim3((unsigned)g), dim3(DEC_IDX_BT), 0, st, P);
    return hipGetLastError();
}

#ifndef PJ_ARR_R
#define PJ_ARR_R 8
#endif
constexpr int ARR_BT = 256, ARR_R = PJ_ARR_R;
uint64_t pj_arr_blocks(uint64_t nblk64) { return (nblk64 + ARR_BT * ARR_R - 1) / (ARR_BT * ARR_R); }
uint64_t pj_arr_threads(uint64_t nblk64) { return pj_arr_blocks(nblk64) * ARR_BT; }

hipError_t pj_launch_arr_frame(const DecParams &P, hipStream_t st) {
    const uint64_t g = pj_arr_blocks(P.nblk64);
    if (g) {                                        // an empty document has no frame: the verdict says so
        hipLaunchKernelGGL((pj::k_arr_sum<ARR_BT, ARR_R>), dim3((unsigned)g), dim3(ARR_BT), 0, st, P);
        hipLaunchKernelGGL((pj::k_arr_scan<1024>), dim3(1), dim3(1024), 0, st, P, g);
        hipLaunchKernelGGL((pj::k_arr_frame<ARR_BT, ARR_R>), dim3((unsigned)g), dim3(ARR_BT), 0, st, P);
    }
    hipLaunchKernelGGL(pj::k_arr_fin, dim3(1), dim3(1), 0, st, P);
    return hipGetLastError();
}

hipError_t pj_launch_dec_errcode(const DecParams &P, hipStream_t st) {
    hipLaunchKernelGGL((pj::k_dec_errcode<64, DEC_TILE>), dim3(8192), dim3(64), 0, st, P);
    return hipGetLastError();
}

constexpr int DEC_BSCAN_BT = 256;
int pj_dec_bscan_block() { return DEC_BSCAN_BT; }

hipError_t pj_launch_dec_bscan(const DecParams &P, hipStream_t st) {
    const uint64_t g = (P.nblocks + DEC_BSCAN_BT - 1) / DEC_BSCAN_BT;
    hipLaunchKernelGGL((pj::k_dec_bscan<DEC_BSCAN_BT>), dim3((unsigned)g), dim3(DEC_BSCAN_BT), 0, st, P);
    return hipGetLastError();
}

hipError_t pj_launch_dec_write(const DecParams &P, hipStream_t st) {
    hipLaunchKernelGGL((pj::k_dec_write<DEC_LINE_BT, DEC_WTILE, DEC_LPB, DEC_LONG>), dim3((unsigned)P.nblocks), dim3(DEC_LINE_BT), 0,
                       st, P);
    return hipGetLastError();
}

hipError_t pj_launch_dec_long(const DecParams &P, hipStream_t st) {
    hipLaunchKernelGGL((pj::k_dec_long<DEC_TILE, DEC_LPB>), dim3(1024), dim3(64), 0, st, P);
    return hipGetLastError();
}

hipError_t pj_launch_dec_parse(const DecParams &P, hipStream_t st) {
    const uint64_t g = (P.lines + DEC_LPB - 1) / DEC_LPB;
    if (P.tape) {
        // every block without bitmaps (five workgroups per CU), then the
        // lines it deferred, then its offsets corrected for them
        hipLaunchKernelGGL((pj::k_dec_block<DEC_LINE_BT, DEC_FTILE, DEC_LONG, DEC_LPB, true, false>), dim3((unsigned)g),
                           dim3(DEC_LINE_BT), 0, st, P);
        hipLaunchKernelGGL((pj::k_dec_measure_long<DEC_TILE>), dim3(1024), dim3(64), 0, st, P);
        hipLaunchKernelGGL((pj::k_dec_fixup<DEC_LINE_BT, DEC_LPB>), dim3((unsigned)(g < 1024 ? g : 1024)),
                           dim3(DEC_LINE_BT), 0, st, P);
    } else
        hipLaunchKernelGGL((pj::k_dec_block<DEC_LINE_BT, DEC_TILE, DEC_LONG, DEC_LPB, false>), dim3((unsigned)g),
                           dim3(DEC_LINE_BT), 0, st, P);
    return hipGetLastError();
}
