// pj_device.h — device helpers shared by the encode and decode kernels
// (gfx950, wave64).  Block-wide scans, the decoupled look-back used to chain
// workgroups in a single pass, and SWAR byte classification.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define PJ_BLOCK 256
#define PJ_WAVES (PJ_BLOCK / 64)

namespace pj {

__device__ __forceinline__ int lane_id() { return (int)__lane_id(); }

__device__ __forceinline__ uint64_t shfl_up_u64(uint64_t v, int d) {
    uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
    lo = (uint32_t)__shfl_up((int)lo, (unsigned)d, 64);
    hi = (uint32_t)__shfl_up((int)hi, (unsigned)d, 64);
    return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint64_t shfl_u64(uint64_t v, int src) {
    uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
    lo = (uint32_t)__shfl((int)lo, src, 64);
    hi = (uint32_t)__shfl((int)hi, src, 64);
    return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m) {
    uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
    lo = (uint32_t)__shfl_xor((int)lo, m, 64);
    hi = (uint32_t)__shfl_xor((int)hi, m, 64);
    return ((uint64_t)hi << 32) | lo;
}

// Cross-lane moves inside the VALU (DPP): row_shr:n shifts within rows of
// 16 lanes, row_bcast:15 / row_bcast:31 carry a row's last lane into the
// next row(s).  Lanes whose source is outside their row, or whose row is
// masked off, read 0.  All 64 lanes must be active.
template <int CTRL, int RM>
__device__ __forceinline__ uint32_t dpp32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, RM, 0xf, false);
}
template <int CTRL, int RM>
__device__ __forceinline__ uint64_t dpp64(uint64_t v) {
    return ((uint64_t)dpp32<CTRL, RM>((uint32_t)(v >> 32)) << 32) | dpp32<CTRL, RM>((uint32_t)v);
}
// Inclusive wave scans (sum): Hillis-Steele within rows, then the row
// totals carried across rows.
__device__ __forceinline__ uint32_t wave_incl_scan32(uint32_t v) {
    v += dpp32<0x111, 0xf>(v);
    v += dpp32<0x112, 0xf>(v);
    v += dpp32<0x114, 0xf>(v);
    v += dpp32<0x118, 0xf>(v);
    v += dpp32<0x142, 0xa>(v);
    v += dpp32<0x143, 0xc>(v);
    return v;
}
__device__ __forceinline__ uint64_t wave_incl_scan(uint64_t v) {
    v += dpp64<0x111, 0xf>(v);
    v += dpp64<0x112, 0xf>(v);
    v += dpp64<0x114, 0xf>(v);
    v += dpp64<0x118, 0xf>(v);
    v += dpp64<0x142, 0xa>(v);
    v += dpp64<0x143, 0xc>(v);
    return v;
}
// lane 63's value, in every lane
__device__ __forceinline__ uint64_t lane63(uint64_t v) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, 63);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), 63);
    return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint64_t wave_sum(uint64_t v) { return lane63(wave_incl_scan(v)); }

// Block-wide exclusive scan of one 64-bit value per thread (all BT threads
// must call).  Returns the exclusive prefix; *total gets the block sum.
// `sh` needs BT/64 entries of LDS.
template <int BT>
__device__ __forceinline__ uint64_t block_excl_scan(uint64_t v, uint64_t *sh, uint64_t *total) {
    constexpr int NW = BT / 64;
    const int t = threadIdx.x, w = t >> 6, l = t & 63;
    uint64_t inc = wave_incl_scan(v);
    if (NW == 1) {
        *total = lane63(inc);
        return inc - v;
    }
    if (l == 63) sh[w] = inc;
    __syncthreads();
    uint64_t before = 0, tot = 0;
#pragma unroll
    for (int k = 0; k < NW; k++) {
        uint64_t s = sh[k];
        before += (k < w) ? s : 0;
        tot += s;
    }
    __syncthreads();
    *total = tot;
    return before + inc - v;
}

// Block-wide exclusive scans of K 32-bit counters per thread at once (all
// BT threads call): excl[k] gets the prefix, tot[k] the block total.  `sh`
// needs K * BT / 64 words of LDS; one barrier pair for all K.
template <int BT, int K>
__device__ __forceinline__ void block_excl_scan_n(const uint32_t *v, uint32_t *excl, uint32_t *tot, uint32_t *sh) {
    constexpr int NW = BT / 64;
    const int t = threadIdx.x, w = t >> 6, l = t & 63;
    uint32_t inc[K];
#pragma unroll
    for (int k = 0; k < K; k++) inc[k] = wave_incl_scan32(v[k]);
    if (l == 63) {
#pragma unroll
        for (int k = 0; k < K; k++) sh[w * K + k] = inc[k];
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < K; k++) {
        uint32_t before = 0, all = 0;
#pragma unroll
        for (int j = 0; j < NW; j++) {
            const uint32_t s = sh[j * K + k];
            before += j < w ? s : 0u;
            all += s;
        }
        excl[k] = before + inc[k] - v[k];
        tot[k] = all;
    }
    __syncthreads();
}

// ----------------------------------------------------------- look-back
// One 64-bit word per logical block: bits 63:62 = state, 61:0 = value.
constexpr uint64_t LB_AGG = 1ull << 62;
constexpr uint64_t LB_PRE = 2ull << 62;
constexpr uint64_t LB_VAL = (1ull << 62) - 1;

__device__ __forceinline__ void lb_store(uint64_t *p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t lb_load(const uint64_t *p) {
    return __hip_atomic_load(const_cast<uint64_t *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Decoupled look-back in two halves.  lb_publish (one lane) announces the
// block aggregate as early as possible; lb_resolve (one full wave) walks the
// predecessors 64 at a time, returns the exclusive prefix (same in every
// lane) and publishes the inclusive prefix.  With ticket-ordered blocks the
// predecessors are resident and the spin always ends.
__device__ __forceinline__ void lb_publish(uint64_t *state, uint64_t b, uint64_t agg) {
    lb_store(&state[b], (b == 0 ? LB_PRE : LB_AGG) | agg);
}

// With a nonzero limit (wall-clock ticks) a wait that outlasts it stores 1 to
// *gave_up and returns 0: blocks then exit even if a predecessor never runs,
// and the caller discards the launch's output.
__device__ __forceinline__ uint64_t lb_resolve(uint64_t *state, uint64_t b, uint64_t agg, uint64_t limit = 0,
                                               unsigned long long *gave_up = nullptr) {
    const int l = lane_id();
    if (b == 0) return 0;
    uint64_t excl = 0;
    int64_t j = (int64_t)b - 1;
    const uint64_t t0 = limit ? wall_clock64() : 0;
    for (;;) {
        int64_t idx = j - l;
        uint64_t s = idx >= 0 ? lb_load(&state[idx]) : LB_PRE;
        uint32_t fl = (uint32_t)(s >> 62);
        uint64_t notready = __ballot(fl == 0);
        uint64_t isp = __ballot(fl == 2);
        int fp = isp ? __builtin_ctzll(isp) : 64;
        uint64_t need = fp >= 63 ? ~0ull : ((2ull << fp) - 1);
        if (notready & need) {
            if (limit && wall_clock64() - t0 > limit) {
                if (l == 0) __hip_atomic_store(gave_up, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                return 0;
            }
            __builtin_amdgcn_s_sleep(1);
            continue;
        }
        excl += wave_sum(l <= fp ? (s & LB_VAL) : 0);
        if (fp < 64) break;
        j -= 64;
    }
    if (l == 0) lb_store(&state[b], LB_PRE | (excl + agg));
    return excl;
}

// Both halves back to back (one full wave).
__device__ __forceinline__ uint64_t lookback(uint64_t *state, uint64_t b, uint64_t agg) {
    if (lane_id() == 0) lb_publish(state, b, agg);
    return lb_resolve(state, b, agg);
}

// ----------------------------------------------------------- SWAR bytes
// Nonzero iff some byte of x is < 0x20 (exact as an "any" test).
__device__ __forceinline__ uint32_t any_lt20(uint32_t x) { return (x - 0x20202020u) & ~x & 0x80808080u; }
__device__ __forceinline__ uint32_t any_zero(uint32_t x) { return (x - 0x01010101u) & ~x & 0x80808080u; }
// Nonzero iff some byte needs a JSON output escape: < 0x20, '"' or '\\'.
__device__ __forceinline__ uint32_t any_special(uint32_t x) {
    return any_lt20(x) | any_zero(x ^ 0x22222222u) | any_zero(x ^ 0x5C5C5C5Cu);
}

__device__ __forceinline__ uint32_t ld32(const uint8_t *p) {  // p 4-byte aligned
    return *reinterpret_cast<const uint32_t *>(p);
}

// Compile-time packing of up to 8 literal bytes (little endian).
__host__ __device__ __forceinline__ constexpr uint64_t pack8(const char *s, int k) {
    uint64_t v = 0;
    for (int j = 0; j < k && j < 8; j++) v |= (uint64_t)(uint8_t)s[j] << (8 * j);
    return v;
}

// Compile-time packing of up to 4 literal bytes (little endian).
constexpr uint32_t pack4(const char *s, int k) {
    return (k > 0 ? (uint32_t)(uint8_t)s[0] : 0u) | (k > 1 ? (uint32_t)(uint8_t)s[1] << 8 : 0u) |
           (k > 2 ? (uint32_t)(uint8_t)s[2] << 16 : 0u) | (k > 3 ? (uint32_t)(uint8_t)s[3] << 24 : 0u);
}

// ------------------------------------------------------- memory helpers
// Unaligned 8-byte global load (gfx950 global memory is in unaligned mode).
__host__ __device__ __forceinline__ uint64_t ldu64(const uint8_t *p) { return *reinterpret_cast<const uint64_t *>(p); }

// The n (1..7) bytes at p, touching only aligned qwords that hold some of
// them (so never a page past the end of the buffer).
__host__ __device__ __forceinline__ uint64_t ld_tail(const uint8_t *p, int n) {
    // The aligned address is formed as an integer on purpose: written as
    // pointer arithmetic (p - (p & 7)) on a generic pointer, the compiler may
    // fold a constant into the flat load's immediate offset and leave a base
    // address below the start of the LDS aperture when the bytes sit at LDS
    // offset 0, which the hardware rejects as an aperture violation.
    const uintptr_t a = (uintptr_t)p & ~(uintptr_t)7;
    const int sh = (int)((uintptr_t)p & 7);
    uint64_t v = *reinterpret_cast<const uint64_t *>(a) >> (8 * sh);
    if (sh + n > 8) v |= *reinterpret_cast<const uint64_t *>(a + 8) << (64 - 8 * sh);
    return v & ((1ull << (8 * n)) - 1);
}

constexpr uint64_t ONES = 0x0101010101010101ull;
// Nonzero iff some byte of x needs an output escape (< 0x20, '"', '\\').
__device__ __forceinline__ uint64_t special64(uint64_t x) {
    const uint64_t q = x ^ (0x22 * ONES), b = x ^ (0x5C * ONES);
    return (((x - 0x20 * ONES) & ~x) | ((q - ONES) & ~q) | ((b - ONES) & ~b)) & (0x80 * ONES);
}

// Direct global writes of a byte stream that starts at any offset.
// Bytes gather in a 64-bit accumulator that always describes an aligned
// output dword; full dwords are stored whole, and the first dword (shared
// with the previous record) is diverted to a per-thread dummy slot while the
// record's own bytes of it, and the tail bytes, are stored one by one.
// Exact-size stores at any byte address (gfx950 runs global memory in
// unaligned mode; bytes outside [p, p+n) are never written, so neighbouring
// writers need no coordination).
__host__ __device__ __forceinline__ void stu64(uint8_t *p, uint64_t v) { *reinterpret_cast<uint64_t *>(p) = v; }
__host__ __device__ __forceinline__ void stu32(uint8_t *p, uint32_t v) { *reinterpret_cast<uint32_t *>(p) = v; }
__host__ __device__ __forceinline__ void stu16(uint8_t *p, uint32_t v) { *reinterpret_cast<uint16_t *>(p) = (uint16_t)v; }
// the low n (0..7) bytes of v
__host__ __device__ __forceinline__ void st_tail(uint8_t *p, uint64_t v, uint32_t n) {
    if (n & 4) { stu32(p, (uint32_t)v); p += 4; v >>= 32; }
    if (n & 2) { stu16(p, (uint32_t)v); p += 2; v >>= 16; }
    if (n & 1) *p = (uint8_t)v;
}
// LDS-qualified pointers: loads through them compile to LDS instructions,
// which wait only on LDS counters (a generic load must also wait for every
// outstanding global load and store).  The host pass sees plain pointers.
#if defined(__HIP_DEVICE_COMPILE__)
#define PJ_LDS __attribute__((address_space(3)))
#else
#define PJ_LDS
#endif
__host__ __device__ __forceinline__ uint64_t lds_u64(const PJ_LDS uint8_t *p) { return *(const PJ_LDS uint64_t *)p; }
// n bytes from an LDS buffer to dst, exactly (no byte outside [dst, dst+n)
// is written).  Scattered per-thread copies are bound by the number of store
// instructions, so: 16-byte stores at any address, the last one ending at
// the last byte and overlapping its predecessor (the overlapped bytes get
// the same values again); below 16 bytes two overlapping 8-, 4- or 2-byte
// stores, or one byte.
__host__ __device__ __forceinline__ void st16(uint8_t *p, const PJ_LDS uint8_t *s) {
    const uint64_t a = lds_u64(s), b = lds_u64(s + 8);
    *reinterpret_cast<uint4 *>(p) = make_uint4((uint32_t)a, (uint32_t)(a >> 32), (uint32_t)b, (uint32_t)(b >> 32));
}
__host__ __device__ __forceinline__ void copy_from_lds(uint8_t *dst, const PJ_LDS uint8_t *src, uint32_t n) {
    if (n >= 16) {
        for (uint32_t k = 0; k + 16 < n; k += 16) st16(dst + k, src + k);
        st16(dst + n - 16, src + n - 16);
    } else if (n >= 8) {
        stu64(dst, lds_u64(src));
        stu64(dst + n - 8, lds_u64(src + n - 8));
    } else if (n >= 4) {
        stu32(dst, (uint32_t)lds_u64(src));
        stu32(dst + n - 4, (uint32_t)lds_u64(src + n - 4));
    } else if (n >= 2) {
        const uint64_t x = lds_u64(src);
        stu16(dst, (uint32_t)x);
        stu16(dst + n - 2, (uint32_t)(x >> (8 * (n - 2))));
    } else if (n) *dst = *src;
}
// 16 bytes starting q = 16 - s bytes into L:H (s = 1 .. 15): dword qd = q / 4
// of the pair, then byte qb = q % 4 of it, joined with v_alignbyte.  qd is
// the same for every lane (it follows the block's base address), so the
// branch is uniform.
__host__ __device__ __forceinline__ uint4 funnel16(const uint4 &L, const uint4 &H, uint32_t qd, uint32_t qb) {
    const uint32_t d0 = L.x, d1 = L.y, d2 = L.z, d3 = L.w, d4 = H.x, d5 = H.y, d6 = H.z, d7 = H.w;
#if defined(__HIP_DEVICE_COMPILE__)
#define PJ_AB(h, l) __builtin_amdgcn_alignbyte(h, l, qb)
#else   // host build of the helpers (index checks): the same byte funnel
#define PJ_AB(h, l) (uint32_t)((((uint64_t)(h) << 32) | (l)) >> (8 * (qb & 3)))
#endif
    switch (qd) {
    case 0: return make_uint4(PJ_AB(d1, d0), PJ_AB(d2, d1), PJ_AB(d3, d2), PJ_AB(d4, d3));
    case 1: return make_uint4(PJ_AB(d2, d1), PJ_AB(d3, d2), PJ_AB(d4, d3), PJ_AB(d5, d4));
    case 2: return make_uint4(PJ_AB(d3, d2), PJ_AB(d4, d3), PJ_AB(d5, d4), PJ_AB(d6, d5));
    default: return make_uint4(PJ_AB(d4, d3), PJ_AB(d5, d4), PJ_AB(d6, d5), PJ_AB(d7, d6));
    }
#undef PJ_AB
}

// A whole 16-byte line of output, stored with the non-temporal hint: output
// is written once and not read back by the kernel (nested encode 2.571 ->
// 2.555 ms, skewed 3.91 -> 3.88 ms against plain stores; the row encoders'
// sector stores and the decode writer's scattered string stores measured
// slower with it, so they keep plain stores).  The host build of
// these helpers (a CPU check) keeps a plain store, which needs no alignment.
__host__ __device__ __forceinline__ void st16_nt(uint8_t *p, uint4 v) {
#if defined(__HIP_DEVICE_COMPILE__)
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 w = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(w, reinterpret_cast<u32x4 *>(p));
#else
    *reinterpret_cast<uint4 *>(p) = v;
#endif
}

// Copy global bytes [lo, hi) out of an LDS tile whose byte x belongs at
// global address D + x (all threads of the workgroup).  Global chunk c
// covers [g0 + 16c, g0 + 16c + 16) with g0 = D - (D & 15), which is tile
// bytes [16c - s, 16c - s + 16): the tail of aligned tile word c-1 and the
// head of word c, joined by funnel16.  Whole chunks leave with one
// aligned 16-byte store; the first and last chunks (shared with neighbouring
// blocks or segments) with exact 8/4/2/1-byte stores.  Whole aligned tile
// words are read, the last one holding global byte g0 + 16 c_hi - 1: up to
// 29 bytes past hi - D, so the tile must be readable 32 bytes past hi - D.
template <int BT>
__host__ __device__ __forceinline__ void tile_copy_out(const uint8_t *tile, uint8_t *out, uint64_t D, uint64_t lo,
                                                       uint64_t hi, uint32_t t) {
    const uint32_t s = (uint32_t)(D & 15);
    const uint32_t qd = (16 - s) >> 2, qb = (16 - s) & 3;
    const uint64_t g0 = D - s;
    const uint32_t c_lo = (uint32_t)((lo - g0) >> 4), c_hi = (uint32_t)((hi - g0 + 15) >> 4);
    const uint4 *W = reinterpret_cast<const uint4 *>(tile);
    constexpr int U = 4;
    for (uint32_t c0 = c_lo + t; c0 < c_hi; c0 += U * BT) {
        uint4 v[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const uint32_t c = c0 + u * BT;
            v[u] = make_uint4(0, 0, 0, 0);
            if (c < c_hi) {
                const uint4 h = W[c];
                if (s == 0) v[u] = h;
                else v[u] = funnel16(c > 0 ? W[c - 1] : make_uint4(0, 0, 0, 0), h, qd, qb);
            }
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const uint32_t c = c0 + u * BT;
            if (c >= c_hi) break;
            const uint64_t g = g0 + 16ull * c;
            const uint64_t a = g > lo ? g : lo, e = g + 16 < hi ? g + 16 : hi;
            if (a == g && e == g + 16) {
                st16_nt(out + g, v[u]);
            } else {
                const uint4 x = v[u];
                unsigned __int128 y = ((unsigned __int128)(((uint64_t)x.w << 32) | x.z) << 64 | (((uint64_t)x.y << 32) | x.x)) >>
                                      (8 * (uint32_t)(a - g));
                uint32_t n = (uint32_t)(e - a);
                uint8_t *q = out + a;
                if (n & 8) { *reinterpret_cast<uint64_t *>(q) = (uint64_t)y; q += 8; y >>= 64; }
                st_tail(q, (uint64_t)y, n & 7);
            }
        }
    }
}

// n bytes from src (LDS or global, readable up to 8 bytes past the end) to dst
__host__ __device__ __forceinline__ void copy_exact(uint8_t *dst, const uint8_t *src, uint32_t n) {
    uint32_t k = 0;
    for (; k + 16 <= n; k += 16) {
        const uint64_t a = ldu64(src + k), b = ldu64(src + k + 8);
        stu64(dst + k, a);
        stu64(dst + k + 8, b);
    }
    if (n - k >= 8) { stu64(dst + k, ldu64(src + k)); k += 8; }
    if (k < n) st_tail(dst + k, ldu64(src + k), n - k);
}
// Byte-stream writer for decoded (unescaped) strings: 8-byte stores at any
// address, exact tail.
struct StoreSink {
    uint8_t *p;
    uint64_t acc;
    uint32_t nacc;
    __host__ __device__ __forceinline__ void init(uint8_t *dst) { p = dst; acc = 0; nacc = 0; }
    __host__ __device__ __forceinline__ void put(uint32_t w, int k) {     // k (1..4) bytes of w
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
    __host__ __device__ __forceinline__ void put8(uint64_t v, uint32_t k) {  // k (1..8) bytes of v
        if (k < 8) v &= (1ull << (8 * k)) - 1;
        acc |= v << (8 * nacc);
        const uint32_t tot = nacc + k;
        if (tot >= 8) {
            stu64(p, acc);
            p += 8;
            acc = nacc ? v >> (8 * (8 - nacc)) : 0;
            nacc = tot - 8;
        } else nacc = tot;
    }
    __host__ __device__ __forceinline__ void finish() { st_tail(p, acc, nacc); }
};

struct WriteSink {
    uint8_t *out;
    uint32_t *dst;
    uint64_t ps, ps0, acc;
    uint32_t head;
    int nacc, lead;

    __host__ __device__ __forceinline__ void init(uint8_t *o, uint64_t p, uint32_t *dummy) {
        out = o;
        ps = ps0 = p & ~3ull;
        lead = nacc = (int)(p & 3);
        acc = 0;
        head = 0;
        dst = lead ? dummy : reinterpret_cast<uint32_t *>(out + ps);
    }
    __host__ __device__ __forceinline__ void put(uint32_t w, int k) {
        uint64_t m = (1ull << (8 * k)) - 1;
        acc |= ((uint64_t)w & m) << (8 * nacc);
        nacc += k;
        if (nacc >= 4) {
            *dst = (uint32_t)acc;
            head = ps == ps0 ? (uint32_t)acc : head;
            ps += 4;
            dst = reinterpret_cast<uint32_t *>(out + ps);
            acc >>= 32;
            nacc -= 4;
        }
    }
    __host__ __device__ __forceinline__ void put8(uint64_t x, int k) {
        if (k > 4) { put((uint32_t)x, 4); put((uint32_t)(x >> 32), k - 4); }
        else if (k > 0) put((uint32_t)x, k);
    }
    __host__ __device__ __forceinline__ void put_byte(uint32_t b) { put(b & 0xFF, 1); }
    __host__ __device__ __forceinline__ void skip(uint32_t) {}
    __host__ __device__ __forceinline__ uint32_t pos() const { return 0; }
    __host__ __device__ __forceinline__ void finish() {
        if (ps == ps0) {
            for (int b = lead; b < nacc; b++) out[ps + b] = (uint8_t)(acc >> (8 * b));
            return;
        }
        for (int b = lead; b > 0 && b < 4; b++) out[ps0 + b] = (uint8_t)(head >> (8 * b));
        for (int b = 0; b < nacc; b++) out[ps + b] = (uint8_t)(acc >> (8 * b));
    }
};

// Global writes of a byte stream that starts at any address, one whole
// aligned 32-byte sector at a time: bytes gather in a window of four qwords
// that describes one aligned sector of the output, and a full window leaves
// as two aligned 16-byte stores, so memory sees each sector written once
// and whole (8-byte stores at any address cost a partial sector write each
// when their line leaves L2 before it fills).  The first sector, shared
// with the previous writer, and the last get exact stores of this writer's
// bytes only, so neighbouring writers need no coordination.  Nothing is read.
struct SectorSink {
    uint8_t *sec;                 // the window's sector (32-byte aligned)
    uint64_t w0, w1, w2, w3;
    uint32_t o;                   // the window's next byte
    uint32_t lo;                  // the window's first byte of this writer

    __host__ __device__ __forceinline__ void init(uint8_t *p) {
        sec = reinterpret_cast<uint8_t *>(reinterpret_cast<uintptr_t>(p) & ~(uintptr_t)31);
        o = lo = (uint32_t)(reinterpret_cast<uintptr_t>(p) & 31);
        w0 = w1 = w2 = w3 = 0;
    }
    // bytes [a, b) of the window, exactly
    __host__ __device__ __forceinline__ void store_part(uint32_t a, uint32_t b) const {
        const uint64_t w[4] = {w0, w1, w2, w3};
#pragma unroll
        for (uint32_t q = 0; q < 4; q++) {
            const uint32_t qa = a > 8 * q ? a : 8 * q, qb = b < 8 * q + 8 ? b : 8 * q + 8;
            if (qa >= qb) continue;
            if (qb - qa == 8) stu64(sec + 8 * q, w[q]);
            else st_tail(sec + qa, w[q] >> (8 * (qa - 8 * q)), qb - qa);
        }
    }
    __host__ __device__ __forceinline__ void flush() {
        if (lo) store_part(lo, 32);
        else {
            *reinterpret_cast<uint4 *>(sec) = make_uint4((uint32_t)w0, (uint32_t)(w0 >> 32), (uint32_t)w1, (uint32_t)(w1 >> 32));
            *reinterpret_cast<uint4 *>(sec + 16) =
                make_uint4((uint32_t)w2, (uint32_t)(w2 >> 32), (uint32_t)w3, (uint32_t)(w3 >> 32));
        }
        sec += 32;
        lo = 0;
    }
    __host__ __device__ __forceinline__ void put8(uint64_t x, int k) {   // k (1..8) bytes of x
        if (k < 8) x &= (1ull << (8 * k)) - 1;
        const uint32_t j = o >> 3, sh = 8 * (o & 7);
        const uint64_t a = x << sh, c = sh ? x >> (64 - sh) : 0;     // c: the bytes past qword j
        w0 |= j == 0 ? a : 0;
        w1 |= j == 1 ? a : (j == 0 ? c : 0);
        w2 |= j == 2 ? a : (j == 1 ? c : 0);
        w3 |= j == 3 ? a : (j == 2 ? c : 0);
        o += (uint32_t)k;
        if (o >= 32) {                     // (then j == 3, and c holds the bytes past the window)
            flush();
            o -= 32;
            w0 = c;
            w1 = w2 = w3 = 0;
        }
    }
    __host__ __device__ __forceinline__ void put(uint32_t w, int k) { put8(w, k); }
    __host__ __device__ __forceinline__ void put_byte(uint32_t b) { put8(b & 0xFF, 1); }
    __host__ __device__ __forceinline__ void skip(uint32_t) {}
    __host__ __device__ __forceinline__ uint32_t pos() const { return 0; }
    __host__ __device__ __forceinline__ void finish() {
        if (o > lo) store_part(lo, o);
    }
};

}  // namespace pj
