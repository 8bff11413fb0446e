// Host check of the decode's block-span guard (dec_block_span_ok in
// pj_kernels.h): line blocks whose lines span 4 GiB - 1 MiB or more are
// refused, shorter ones pass, whatever the block's position and size.
#include <cstdio>
#include <vector>

#include "pj_kernels.h"

static int fails = 0;
static void expect(bool got, bool want, const char *what) {
    if (got != want) { std::printf("FAIL: %s\n", what); fails++; }
}

int main() {
    const uint64_t lpb = 104, G = 1ull << 30;
    // 300 lines of 100 bytes, then one line of 4 GiB, then 50 short lines
    std::vector<uint64_t> ls;
    uint64_t a = 0;
    for (int k = 0; k < 300; k++) { ls.push_back(a); a += 100; }
    ls.push_back(a); a += 4 * G;
    for (int k = 0; k < 50; k++) { ls.push_back(a); a += 100; }
    ls.push_back(a);
    const uint64_t lines = ls.size() - 1;
    expect(dec_block_span_ok(ls.data(), lines, lpb, 0), true, "short block");
    expect(dec_block_span_ok(ls.data(), lines, lpb, 1), true, "short block 1");
    expect(dec_block_span_ok(ls.data(), lines, lpb, 2), false, "block holding the 4 GiB line");
    expect(dec_block_span_ok(ls.data(), lines, lpb, 3), true, "last, partial block");
    expect(dec_block_span_ok(ls.data(), lines, lpb, 4), true, "block past the end");
    // a block of many lines just under / at the limit
    std::vector<uint64_t> m;
    const uint64_t per = (PJ_DEC_MAX_BLOCK_SPAN - 1) / lpb;
    for (uint64_t k = 0; k <= lpb; k++) m.push_back(k * per);
    expect(dec_block_span_ok(m.data(), lpb, lpb, 0), true, "just under the limit");
    m[lpb] = PJ_DEC_MAX_BLOCK_SPAN;
    expect(dec_block_span_ok(m.data(), lpb, lpb, 0), false, "at the limit");
    if (fails) return 1;
    std::printf("span guard checks passed\n");
    return 0;
}
