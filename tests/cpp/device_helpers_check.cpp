// Host build of the device memory helpers of pj_device.h, run over many
// offsets, lengths and alignments with every source buffer sized to exactly
// what its helper documents as readable and every destination sized to the
// bytes it may write.  Built with AddressSanitizer (tests/test_device_helpers.py),
// so an index or address formed outside those bounds is reported; ld_tail
// is also run against PROT_NONE guard pages, since its contract is about
// which aligned qwords it touches, not only about bytes.  Every result is
// compared with the plain byte copy it stands for, and the bytes around each
// destination must stay untouched.
#include <hip/hip_runtime.h>

#include <sys/mman.h>
#include <unistd.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <vector>

#include "pj_device.h"

using namespace pj;

#define CHECK(c)                                                                    \
    do {                                                                            \
        if (!(c)) {                                                                 \
            std::fprintf(stderr, "FAIL %s:%d: %s\n", __FILE__, __LINE__, #c);       \
            std::exit(1);                                                           \
        }                                                                           \
    } while (0)

static std::mt19937_64 rng(20261202);
static uint8_t rbyte() { return (uint8_t)rng(); }

// Exactly n addressable bytes (AddressSanitizer reports one byte more).
static uint8_t *exact(size_t n) { return static_cast<uint8_t *>(std::malloc(n ? n : 1)); }

// ld_tail(p, n) next to PROT_NONE pages: bytes ending at the last byte of a
// readable page, and bytes starting at its first byte.
static void check_ld_tail() {
    const long pg = sysconf(_SC_PAGESIZE);
    uint8_t *m = static_cast<uint8_t *>(mmap(nullptr, 3 * pg, PROT_READ | PROT_WRITE, MAP_PRIVATE | MAP_ANONYMOUS, -1, 0));
    CHECK(m != MAP_FAILED);
    CHECK(mprotect(m, pg, PROT_NONE) == 0);
    CHECK(mprotect(m + 2 * pg, pg, PROT_NONE) == 0);
    uint8_t *page = m + pg;
    for (long k = 0; k < pg; k++) page[k] = rbyte();
    for (int n = 1; n <= 7; n++) {
        for (int back = n; back <= n + 16; back++) {       // [end - back, end - back + n)
            const uint8_t *p = page + pg - back;
            uint64_t want = 0;
            std::memcpy(&want, p, n);
            CHECK(ld_tail(p, n) == want);
        }
        for (int fwd = 0; fwd < 16; fwd++) {                // from the page's first bytes
            const uint8_t *p = page + fwd;
            uint64_t want = 0;
            std::memcpy(&want, p, n);
            CHECK(ld_tail(p, n) == want);
        }
    }
    munmap(m, 3 * pg);
}

// copy_from_lds: the source is readable for max(n, 8) bytes (the kernels'
// LDS tiles carry 64 bytes of padding), the destination is written exactly.
static void check_copy_from_lds() {
    for (int it = 0; it < 20000; it++) {
        const uint32_t n = (uint32_t)(it < 200 ? it : rng() % 2048);
        const uint32_t srd = n > 8 ? n : 8;
        uint8_t *src = exact(srd);
        for (uint32_t k = 0; k < srd; k++) src[k] = rbyte();
        uint8_t *buf = exact(n + 2 * 16);
        std::memset(buf, 0xEE, n + 32);
        copy_from_lds(buf + 16, src, n);
        CHECK(std::memcmp(buf + 16, src, n) == 0);
        for (uint32_t k = 0; k < 16; k++) CHECK(buf[k] == 0xEE && buf[16 + n + k] == 0xEE);
        uint8_t *dst = exact(n);                            // and into exactly n bytes
        copy_from_lds(dst, src, n);
        CHECK(std::memcmp(dst, src, n) == 0);
        std::free(dst);
        std::free(buf);
        std::free(src);
    }
}

// copy_exact: the source is readable up to 8 bytes past its end.
static void check_copy_exact() {
    for (int it = 0; it < 20000; it++) {
        const uint32_t n = (uint32_t)(it < 200 ? it : rng() % 4096);
        uint8_t *src = exact(n + 8);
        for (uint32_t k = 0; k < n + 8; k++) src[k] = rbyte();
        uint8_t *dst = exact(n);
        copy_exact(dst, src, n);
        CHECK(std::memcmp(dst, src, n) == 0);
        std::free(dst);
        std::free(src);
    }
}

// tile_copy_out<BT>: global bytes [lo, hi) from a tile whose byte x belongs
// at D + x, every thread of the workgroup in turn.  The tile is readable
// 32 bytes past hi - D (k_encode copies a block or segment out only when
// that much of its tile is free); the output holds exactly [lo, hi).
template <int BT> static void check_tile_copy_out() {
    for (int it = 0; it < 4000; it++) {
        const uint64_t D = 1000000 + rng() % 4096;            // any alignment
        const uint64_t span = rng() % 40000;                  // tile bytes in use
        const uint64_t lo = D + (span ? rng() % (span + 1) : 0);
        const uint64_t hi = lo + (span + D > lo ? rng() % (span + D - lo + 1) : 0);
        const size_t tbytes = (size_t)(hi - D) + 32;
        uint8_t *tile = exact(tbytes);                        // 16-byte aligned, like the LDS tile
        CHECK(((uintptr_t)tile & 15) == 0);
        for (size_t k = 0; k < tbytes; k++) tile[k] = rbyte();
        uint8_t *outb = exact((size_t)(hi - lo));
        // out + g addresses global byte g: shift the base so [lo, hi) maps
        // onto outb, with the same 16-byte phase as a real output buffer
        uint8_t *out = outb - lo;
        for (uint32_t t = 0; t < (uint32_t)BT; t++) tile_copy_out<BT>(tile, out, D, lo, hi, t);
        CHECK(std::memcmp(outb, tile + (lo - D), (size_t)(hi - lo)) == 0);
        std::free(outb);
        std::free(tile);
    }
}

// StoreSink: a byte stream at any address, exact tail.
static void check_store_sink() {
    for (int it = 0; it < 20000; it++) {
        const uint32_t n = (uint32_t)(rng() % 600);
        std::vector<uint8_t> want(n);
        for (auto &b : want) b = rbyte();
        uint8_t *dst = exact(n);
        StoreSink s;
        s.init(dst);
        uint32_t k = 0;
        while (k < n) {
            const uint32_t m = std::min<uint32_t>(n - k, 1 + (uint32_t)(rng() % 8));
            uint64_t v = 0;
            std::memcpy(&v, want.data() + k, m);
            s.put8(v, m);
            k += m;
        }
        s.finish();
        CHECK(n == 0 || std::memcmp(dst, want.data(), n) == 0);
        std::free(dst);
    }
}

// WriteSink: a record's bytes at any offset of the output, its first
// partial dword (shared with the previous record) diverted to a dummy slot
// and written byte by byte at the end; no byte outside [p, p + n) changes.
static void check_write_sink() {
    for (int it = 0; it < 20000; it++) {
        const uint32_t n = 1 + (uint32_t)(rng() % 600), p = (uint32_t)(rng() % 64);
        std::vector<uint8_t> want(n);
        for (auto &b : want) b = rbyte();
        const uint32_t total = (p + n + 3) / 4 * 4;          // the dwords the record touches
        uint8_t *out = exact(total);
        std::memset(out, 0xEE, total);
        uint32_t dummy = 0;
        WriteSink s;
        s.init(out, p, &dummy);
        uint32_t k = 0;
        while (k < n) {
            const uint32_t m = std::min<uint32_t>(n - k, 1 + (uint32_t)(rng() % 8));
            uint64_t v = 0;
            std::memcpy(&v, want.data() + k, m);
            s.put8(v, (int)m);
            k += m;
        }
        s.finish();
        CHECK(std::memcmp(out + p, want.data(), n) == 0);
        for (uint32_t j = 0; j < p; j++) CHECK(out[j] == 0xEE);
        for (uint32_t j = p + n; j < total; j++) CHECK(out[j] == 0xEE);
        std::free(out);
    }
}

// SectorSink: a record's bytes at any offset of a 32-byte aligned output,
// in pieces of 1 to 8 bytes; the result equals the bytes, the buffer holds
// exactly the sectors the record touches, and no byte outside [p, p + n)
// changes.
static void check_sector_sink() {
    for (int it = 0; it < 40000; it++) {
        const uint32_t n = (uint32_t)(it < 300 ? it % 100 : rng() % 700), p = (uint32_t)(rng() % 96);
        std::vector<uint8_t> want(n);
        for (auto &b : want) b = rbyte();
        const uint32_t total = (p + n + 31) / 32 * 32 + 32;   // the sectors the record touches (and one more)
        uint8_t *out = static_cast<uint8_t *>(std::aligned_alloc(32, total));
        std::memset(out, 0xEE, total);
        SectorSink s;
        s.init(out + p);
        uint32_t k = 0;
        while (k < n) {
            const uint32_t m = std::min<uint32_t>(n - k, 1 + (uint32_t)(rng() % 8));
            uint64_t v = rng();                               // bytes past m must be ignored
            std::memcpy(&v, want.data() + k, m);
            if (m <= 4 && (rng() & 1)) s.put((uint32_t)v, (int)m);
            else s.put8(v, (int)m);
            k += m;
        }
        s.finish();
        CHECK(n == 0 || std::memcmp(out + p, want.data(), n) == 0);
        for (uint32_t j = 0; j < p; j++) CHECK(out[j] == 0xEE);
        for (uint32_t j = p + n; j < total; j++) CHECK(out[j] == 0xEE);
        std::free(out);
    }
}

int main() {
    check_ld_tail();
    check_copy_from_lds();
    check_copy_exact();
    check_tile_copy_out<256>();
    check_tile_copy_out<192>();
    check_store_sink();
    check_write_sink();
    check_sector_sink();
    std::printf("device helpers: all checks passed\n");
    return 0;
}
