// pj_encode.hip — single-pass columnar Pet -> JSON encoder for gfx950.
//
// One workgroup = PJ_BLOCK consecutive records, one record per thread:
//   1. length pass: every thread measures its record's JSON bytes (integer
//      digit counts, escape expansion of its strings, separators);
//   2. block-wide exclusive scan of the lengths;
//   3. decoupled look-back across workgroups (logical block ids from an
//      atomic ticket) gives the block's output base;
//   4. write pass: every thread emits its record at base + prefix.  Bytes are
//      gathered in a 64-bit register and stored as aligned dwords; the few
//      bytes a record shares with a neighbour's dword are byte stores.
// Strings are read with aligned dword loads and funnel shifts; a SWAR test
// takes four bytes at a time through the no-escape fast path.
//
// Output rules (jackson UTF8JsonGenerator via micronaut-serde, reference
// build.gradle:104) and property order / inclusion (petstore.json:872-922)
// are the same as the CPU restatement in oracle/pj_oracle.c.
#include "pj_device.h"
#include "pj_kernels.h"

namespace pj {

// ------------------------------------------------------------------ sinks
struct CountSink {
    uint64_t n = 0;
    __device__ __forceinline__ void put(uint32_t, int k) { n += (uint64_t)k; }
    __device__ __forceinline__ void put_byte(uint32_t) { n += 1; }
};

struct WriteSink {
    uint8_t *out;
    uint64_t ps;     // output position of the first pending byte
    uint64_t acc;    // pending bytes, little endian
    int nacc;        // number of pending bytes (<= 3 between calls)

    __device__ __forceinline__ void drain() {
        while (nacc >= 4) {
            if ((ps & 3) == 0) {
                *reinterpret_cast<uint32_t *>(out + ps) = (uint32_t)acc;
                acc >>= 32; nacc -= 4; ps += 4;
            } else {
                out[ps] = (uint8_t)acc;
                acc >>= 8; nacc -= 1; ps += 1;
            }
        }
    }
    // append the low k (1..4) bytes of w
    __device__ __forceinline__ void put(uint32_t w, int k) {
        uint64_t m = k == 4 ? 0xFFFFFFFFull : ((1ull << (8 * k)) - 1);
        acc |= ((uint64_t)w & m) << (8 * nacc);
        nacc += k;
        drain();
    }
    __device__ __forceinline__ void put_byte(uint32_t b) { put(b & 0xFF, 1); }
    __device__ __forceinline__ void finish() {
        while (nacc > 0) { out[ps] = (uint8_t)acc; acc >>= 8; nacc--; ps++; }
    }
};

template <class S, int N> __device__ __forceinline__ void lit(S &s, const char (&str)[N]) {
    constexpr int L = N - 1;
#pragma unroll
    for (int k = 0; k < L; k += 4) s.put(pack4(str + k, (L - k) < 4 ? (L - k) : 4), (L - k) < 4 ? (L - k) : 4);
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

// Long.toString(v): number of bytes.
__device__ __forceinline__ int long_len(int64_t v) {
    uint64_t u = v < 0 ? 0ull - (uint64_t)v : (uint64_t)v;
    int neg = v < 0;
    if (u < 100000000ull) return neg + digits32((uint32_t)u);
    if (u < 10000000000000000ull) return neg + 8 + digits32((uint32_t)(u / 100000000ull));
    return neg + 16 + digits32((uint32_t)(u / 10000000000000000ull));
}

template <class S> __device__ __forceinline__ void emit_long(S &s, int64_t v) {
    uint64_t u = v < 0 ? 0ull - (uint64_t)v : (uint64_t)v;
    if (v < 0) s.put_byte('-');
    uint32_t ch[5];   // 20 digits, most significant chunk first
    uint32_t c0, c1, c2;
    c2 = (uint32_t)(u % 100000000ull);
    uint64_t q = u / 100000000ull;
    c1 = (uint32_t)(q % 100000000ull);
    c0 = (uint32_t)(q / 100000000ull);      // <= 922
    ch[0] = four_digits(c0);
    ch[1] = four_digits(c1 / 10000u); ch[2] = four_digits(c1 % 10000u);
    ch[3] = four_digits(c2 / 10000u); ch[4] = four_digits(c2 % 10000u);
    int nd = u < 100000000ull ? digits32((uint32_t)u)
             : (q < 100000000ull ? 8 + digits32((uint32_t)q) : 16 + digits32(c0));
    int skip = 20 - nd;          // leading zero digits to drop
    int k = skip >> 2, off = skip & 3;
    if (off) { s.put(ch[k] >> (8 * off), 4 - off); k++; }
    for (; k < 5; k++) s.put(ch[k], 4);
}

// ----------------------------------------------------------------- strings
__device__ __forceinline__ int esc_extra(uint32_t c) {  // bytes added by escaping c
    if (c == '"' || c == '\\' || c == 8 || c == 9 || c == 10 || c == 12 || c == 13) return 1;
    return c < 0x20 ? 5 : 0;
}

template <class S> __device__ __forceinline__ void emit_esc_byte(S &s, uint32_t c, uint32_t hexa) {
    if (c >= 0x20 && c != '"' && c != '\\') { s.put_byte(c); return; }
    uint32_t e;
    switch (c) {
    case '"': e = '"'; break;
    case '\\': e = '\\'; break;
    case 8: e = 'b'; break;
    case 9: e = 't'; break;
    case 10: e = 'n'; break;
    case 12: e = 'f'; break;
    case 13: e = 'r'; break;
    default: {
        uint32_t lo = c & 15;
        uint32_t hc = lo < 10 ? '0' + lo : hexa + lo - 10;
        s.put(pack4("\\u00", 4), 4);
        s.put(('0' + (c >> 4)) | (hc << 8), 2);
        return;
    }
    }
    s.put('\\' | (e << 8), 2);
}

// Escaped body length of a raw UTF-8 string (without quotes).
__device__ __forceinline__ uint64_t str_len(const uint8_t *p, uint64_t len) {
    if (len == 0) return 0;
    const uint8_t *a = (const uint8_t *)((uintptr_t)p & ~(uintptr_t)3);
    const int off = (int)((uintptr_t)p & 3);
    uint64_t extra = 0;
    uint32_t lo = ld32(a);
    for (uint64_t k = 0; k < len; k += 4) {
        uint64_t rem = len - k;
        uint32_t w = lo;
        if (off) {
            uint32_t hi = (off + rem > 4) ? ld32(a + 4) : 0u;
            w = __builtin_amdgcn_alignbyte(hi, lo, off);
            lo = hi;
        } else if (rem > 4) {
            lo = ld32(a + 4);
        }
        a += 4;
        int m = rem < 4 ? (int)rem : 4;
        uint32_t vm = m == 4 ? 0xFFFFFFFFu : ((1u << (8 * m)) - 1);
        uint32_t x = (w & vm) | (0x41414141u & ~vm);
        if (any_special(x)) {
            for (int b = 0; b < m; b++) extra += (uint64_t)esc_extra((x >> (8 * b)) & 0xFF);
        }
    }
    return len + extra;
}

template <class S> __device__ __forceinline__ void emit_str(S &s, const uint8_t *p, uint64_t len, uint32_t hexa) {
    s.put_byte('"');
    if (len) {
        const uint8_t *a = (const uint8_t *)((uintptr_t)p & ~(uintptr_t)3);
        const int off = (int)((uintptr_t)p & 3);
        uint32_t lo = ld32(a);
        for (uint64_t k = 0; k < len; k += 4) {
            uint64_t rem = len - k;
            uint32_t w = lo;
            if (off) {
                uint32_t hi = (off + rem > 4) ? ld32(a + 4) : 0u;
                w = __builtin_amdgcn_alignbyte(hi, lo, off);
                lo = hi;
            } else if (rem > 4) {
                lo = ld32(a + 4);
            }
            a += 4;
            int m = rem < 4 ? (int)rem : 4;
            uint32_t vm = m == 4 ? 0xFFFFFFFFu : ((1u << (8 * m)) - 1);
            uint32_t x = (w & vm) | (0x41414141u & ~vm);
            if (!any_special(x)) {
                s.put(w, m);
            } else {
                for (int b = 0; b < m; b++) emit_esc_byte(s, (x >> (8 * b)) & 0xFF, hexa);
            }
        }
    }
    s.put_byte('"');
}

// The count sink only needs lengths: a specialisation avoids re-walking.
__device__ __forceinline__ void emit_str(CountSink &s, const uint8_t *p, uint64_t len, uint32_t) {
    s.n += 2 + str_len(p, len);
}
__device__ __forceinline__ void emit_long(CountSink &s, int64_t v) { s.n += (uint64_t)long_len(v); }

// ------------------------------------------------------------------ record
template <class S> __device__ __forceinline__ void key(S &s, bool &first) {
    if (!first) s.put_byte(',');
    first = false;
}

template <class S>
__device__ __forceinline__ void emit_sub(S &s, const EncParams &P, uint32_t fl, int64_t id,
                                         const uint8_t *nm, uint64_t nlen) {
    bool first = true;
    s.put_byte('{');
    if (fl & PJ_SUB_HAS_ID) { key(s, first); lit(s, "\"id\":"); emit_long(s, id); }
    else if (P.incl == PJ_INCLUDE_ALWAYS) { key(s, first); lit(s, "\"id\":null"); }
    if (fl & PJ_SUB_HAS_NAME) {
        if (nlen > 0 || P.incl != PJ_INCLUDE_NON_EMPTY) {
            key(s, first); lit(s, "\"name\":"); emit_str(s, nm, nlen, P.hexa);
        }
    } else if (P.incl == PJ_INCLUDE_ALWAYS) { key(s, first); lit(s, "\"name\":null"); }
    s.put_byte('}');
}

template <bool NESTED, class S>
__device__ __forceinline__ void emit_pet(S &s, const EncParams &P, uint64_t i) {
    const pj_pet_columns &c = P.c;
    const uint32_t fl = c.flags ? c.flags[i] : (uint32_t)PJ_PET_DEFAULT_FLAGS;
    bool first = true;
    s.put_byte('{');
    if (fl & PJ_PET_HAS_ID) { key(s, first); lit(s, "\"id\":"); emit_long(s, c.id[i]); }
    else if (P.incl == PJ_INCLUDE_ALWAYS) { key(s, first); lit(s, "\"id\":null"); }
    if (NESTED && (fl & PJ_PET_HAS_CATEGORY) && c.cat_id) {
        key(s, first); lit(s, "\"category\":");
        uint32_t cf = c.cat_flags ? c.cat_flags[i] : (uint32_t)PJ_SUB_DEFAULT_FLAGS;
        uint64_t a = c.cat_name_off[i], b = c.cat_name_off[i + 1];
        emit_sub(s, P, cf, c.cat_id[i], c.cat_name_bytes + a, b - a);
    } else if (P.incl == PJ_INCLUDE_ALWAYS) { key(s, first); lit(s, "\"category\":null"); }
    key(s, first);
    if (fl & PJ_PET_HAS_NAME) {
        lit(s, "\"name\":");
        uint64_t a = c.name_off[i], b = c.name_off[i + 1];
        emit_str(s, c.name_bytes + a, b - a, P.hexa);
    } else lit(s, "\"name\":null");
    s.put_byte(',');
    if (fl & PJ_PET_HAS_PHOTOURLS) {
        lit(s, "\"photoUrls\":[");
        if (NESTED && c.photo_off) {
            uint64_t u0 = c.photo_off[i], u1 = c.photo_off[i + 1];
            for (uint64_t u = u0; u < u1; u++) {
                if (u > u0) s.put_byte(',');
                uint64_t a = c.url_off[u], b = c.url_off[u + 1];
                emit_str(s, c.url_bytes + a, b - a, P.hexa);
            }
        }
        s.put_byte(']');
    } else lit(s, "\"photoUrls\":null");
    if (NESTED && (fl & PJ_PET_HAS_TAGS)) {
        uint64_t t0 = c.tag_off ? c.tag_off[i] : 0, t1 = c.tag_off ? c.tag_off[i + 1] : 0;
        if (t1 > t0 || P.incl != PJ_INCLUDE_NON_EMPTY) {
            lit(s, ",\"tags\":[");
            for (uint64_t t = t0; t < t1; t++) {
                if (t > t0) s.put_byte(',');
                uint32_t tf = c.tag_flags ? c.tag_flags[t] : (uint32_t)PJ_SUB_DEFAULT_FLAGS;
                uint64_t a = c.tag_name_off[t], b = c.tag_name_off[t + 1];
                emit_sub(s, P, tf, c.tag_id[t], c.tag_name_bytes + a, b - a);
            }
            s.put_byte(']');
        }
    } else if (P.incl == PJ_INCLUDE_ALWAYS) lit(s, ",\"tags\":null");
    const uint32_t st = c.status ? c.status[i] : (uint32_t)PJ_STATUS_NULL;
    if (st == 0) lit(s, ",\"status\":\"available\"");
    else if (st == 1) lit(s, ",\"status\":\"pending\"");
    else if (st == 2) lit(s, ",\"status\":\"sold\"");
    else if (P.incl == PJ_INCLUDE_ALWAYS) lit(s, ",\"status\":null");
    s.put_byte('}');
}

// ------------------------------------------------------------------ kernel
template <bool NESTED>
__global__ __launch_bounds__(PJ_BLOCK) void k_encode(EncParams P) {
    __shared__ uint64_t sh_scan[PJ_WAVES + 1];
    __shared__ uint64_t sh_blk;
    __shared__ uint64_t sh_base;
    const int t = threadIdx.x;
    if (t == 0) sh_blk = atomicAdd(P.ticket, 1ull);
    __syncthreads();
    const uint64_t b = sh_blk;
    const uint64_t i = b * PJ_BLOCK + (uint64_t)t;
    const bool live = i < P.n;
    const bool ndjson = P.format == PJ_FORMAT_NDJSON;

    uint64_t len = 0;
    if (live) {
        CountSink cs;
        emit_pet<NESTED>(cs, P, i);
        len = cs.n + 1;                                     // ',' / '[' / '\n'
        if (!ndjson && i == P.n - 1) len += 1;              // closing ']'
    }
    uint64_t agg;
    uint64_t pre = block_excl_scan(len, sh_scan, &agg);
    if (t < 64) {
        uint64_t excl = lookback(P.state, b, agg);
        if (t == 0) {
            sh_base = excl;
            if (b == gridDim.x - 1) *P.total = excl + agg;
        }
    }
    __syncthreads();
    if (!live || P.count_only) return;
    const uint64_t pos = sh_base + pre;
    if (pos + len > P.cap) return;                           // capacity guard
    WriteSink ws{P.out, pos, 0ull, 0};
    if (!ndjson) ws.put_byte(i == 0 ? '[' : ',');
    emit_pet<NESTED>(ws, P, i);
    if (ndjson) ws.put_byte('\n');
    else if (i == P.n - 1) ws.put_byte(']');
    ws.finish();
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
hipError_t pj_launch_fill_u64(uint64_t *p, uint64_t n, uint64_t v, hipStream_t st) {
    if (n == 0) return hipSuccess;
    uint64_t g = (n + 255) / 256;
    hipLaunchKernelGGL(pj::k_fill_u64, dim3((unsigned)g), dim3(256), 0, st, p, n, v);
    return hipGetLastError();
}

hipError_t pj_launch_encode(const EncParams &P, bool nested, hipStream_t st) {
    uint64_t g = (P.n + PJ_BLOCK - 1) / PJ_BLOCK;
    if (nested)
        hipLaunchKernelGGL(pj::k_encode<true>, dim3((unsigned)g), dim3(PJ_BLOCK), 0, st, P);
    else
        hipLaunchKernelGGL(pj::k_encode<false>, dim3((unsigned)g), dim3(PJ_BLOCK), 0, st, P);
    return hipGetLastError();
}

hipError_t pj_launch_put_bytes(uint8_t *out, uint32_t w, int k, hipStream_t st) {
    hipLaunchKernelGGL(pj::k_put_bytes, dim3(1), dim3(64), 0, st, out, w, k);
    return hipGetLastError();
}
