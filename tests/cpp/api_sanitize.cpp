// Drives the host half of libpetjson (pj_api.cpp) for the sanitizer builds
// of tests/test_sanitizers.py: argument validation on every entry point,
// the decode bounds, and — when a gfx950 device is present — round trips of
// generated records through the host entry points (their staging copies).
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "petjson.h"
#include "pj_gen.h"

#define CHECK(c)                                                        \
    do {                                                                \
        if (!(c)) {                                                     \
            std::fprintf(stderr, "check failed: %s (line %d)\n", #c, __LINE__); \
            return 1;                                                   \
        }                                                               \
    } while (0)

namespace {

struct Host {
    std::vector<int64_t> id, cat_id, tag_id;
    std::vector<uint8_t> flags, status, cat_flags, tag_flags, name, cat_name, url, tag_name;
    std::vector<uint64_t> name_off, cat_name_off, photo_off, tag_off, url_off, tag_name_off;
    pj_pet_columns v;
    explicit Host(uint64_t len) {
        std::memset(&v, 0, sizeof v);
        pj_decode_bounds(len, &v);
        const uint64_t p = v.cap_pets, u = v.cap_urls, t = v.cap_tags;
        id.resize(p); flags.resize(p); status.resize(p); cat_id.resize(p); cat_flags.resize(p);
        name_off.resize(p + 1); cat_name_off.resize(p + 1); photo_off.resize(p + 1); tag_off.resize(p + 1);
        url_off.resize(u + 1); tag_name_off.resize(t + 1); tag_id.resize(t); tag_flags.resize(t);
        name.resize(v.cap_name_bytes); cat_name.resize(v.cap_cat_name_bytes); url.resize(v.cap_url_bytes);
        tag_name.resize(v.cap_tag_name_bytes);
        v.id = id.data(); v.flags = flags.data(); v.status = status.data(); v.cat_id = cat_id.data();
        v.cat_flags = cat_flags.data(); v.name_off = name_off.data(); v.cat_name_off = cat_name_off.data();
        v.photo_off = photo_off.data(); v.tag_off = tag_off.data(); v.url_off = url_off.data();
        v.tag_name_off = tag_name_off.data(); v.tag_id = tag_id.data(); v.tag_flags = tag_flags.data();
        v.name_bytes = name.data(); v.cat_name_bytes = cat_name.data(); v.url_bytes = url.data();
        v.tag_name_bytes = tag_name.data();
    }
};

int round_trip(pj_ctx *ctx, int cfg, uint64_t n, int fmt) {
    pj_pet_columns c;
    std::memset(&c, 0, sizeof c);
    CHECK(pjg_generate(cfg, n, PJG_SEED_BASE + cfg, 2, &c) == 0);
    uint64_t need = 0;
    CHECK(pj_encode_host(ctx, &c, fmt, nullptr, 0, &need) == PJ_ERR_CAPACITY);
    std::vector<uint8_t> text(need);
    uint64_t got = 0;
    CHECK(pj_encode_host(ctx, &c, fmt, text.data(), text.size(), &got) == PJ_OK && got == need);
    Host h(text.size());
    std::vector<uint64_t> el(16);
    std::vector<uint8_t> ec(16);
    pj_decode_result r;
    const pj_status s = fmt == PJ_FORMAT_ARRAY
                            ? pj_decode_array_host(ctx, text.data(), text.size(), &h.v, el.data(), ec.data(), 16, &r)
                            : pj_decode_host(ctx, text.data(), text.size(), &h.v, el.data(), ec.data(), 16, &r);
    CHECK(s == PJ_OK && r.n_pets == n && r.n_errors == 0);
    CHECK(std::memcmp(h.id.data(), c.id, n * 8) == 0);
    CHECK(std::memcmp(h.name_off.data(), c.name_off, (n + 1) * 8) == 0);
    CHECK(std::memcmp(h.name.data(), c.name_bytes, r.name_bytes) == 0);
    // a capacity one short is reported, never overrun
    h.v.cap_name_bytes = r.name_bytes ? r.name_bytes - 1 : 0;
    const pj_status s2 = fmt == PJ_FORMAT_ARRAY
                             ? pj_decode_array_host(ctx, text.data(), text.size(), &h.v, el.data(), ec.data(), 16, &r)
                             : pj_decode_host(ctx, text.data(), text.size(), &h.v, el.data(), ec.data(), 16, &r);
    CHECK(r.name_bytes == 0 || s2 == PJ_ERR_CAPACITY);
    pjg_free(&c);
    return 0;
}

}  // namespace

int main() {
    pj_options o;
    pj_default_options(&o);
    CHECK(o.inclusion == PJ_INCLUDE_NON_EMPTY && o.hex_upper == 1);
    // every entry point refuses a null context
    pj_pet_columns cols;
    std::memset(&cols, 0, sizeof cols);
    uint64_t len = 0;
    pj_decode_result r;
    uint8_t b[4] = {'[', ']', 0, 0};
    CHECK(pj_set_options(nullptr, &o) != PJ_OK);
    CHECK(pj_encode_device(nullptr, &cols, PJ_FORMAT_ARRAY, b, 4, &len) != PJ_OK);
    CHECK(pj_encode_host(nullptr, &cols, PJ_FORMAT_ARRAY, b, 4, &len) != PJ_OK);
    CHECK(pj_encode_size_device(nullptr, &cols, PJ_FORMAT_ARRAY, &len) != PJ_OK);
    CHECK(pj_encode_device_noalloc(nullptr, &cols, PJ_FORMAT_ARRAY, b, 4, &len) != PJ_OK);
    CHECK(pj_decode_device(nullptr, b, 2, &cols, nullptr, nullptr, 0, &r) != PJ_OK);
    CHECK(pj_decode_host(nullptr, b, 2, &cols, nullptr, nullptr, 0, &r) != PJ_OK);
    CHECK(pj_decode_array_device(nullptr, b, 2, &cols, nullptr, nullptr, 0, &r) != PJ_OK);
    CHECK(pj_decode_array_host(nullptr, b, 2, &cols, nullptr, nullptr, 0, &r) != PJ_OK);
    CHECK(pj_last_error() != nullptr);
    float ms[4];
    CHECK(pj_last_timings(nullptr, ms, 4) == 0);
    pj_destroy(nullptr);
    // decode bounds: monotone in the length, never zero capacity for records
    pj_pet_columns a, c2;
    for (uint64_t l : {0ull, 1ull, 2ull, 100ull, 4096ull, 1ull << 32, 1ull << 40}) {
        pj_decode_bounds(l, &a);
        pj_decode_bounds(2 * l + 1, &c2);
        CHECK(a.cap_pets >= 1 && c2.cap_pets >= a.cap_pets && c2.cap_name_bytes >= a.cap_name_bytes);
    }
    pj_status st = PJ_OK;
    pj_ctx *ctx = pj_create(0, &st);
    if (!ctx) {
        CHECK(st == PJ_ERR_NO_DEVICE || st == PJ_ERR_DEVICE);
        std::printf("api sanitize ok (no device)\n");
        return 0;
    }
    for (int cfg : {1, 3, 5})
        for (int fmt : {PJ_FORMAT_ARRAY, PJ_FORMAT_NDJSON})
            if (round_trip(ctx, cfg, cfg == 5 ? 2000 : 20000, fmt)) return 1;
    pj_destroy(ctx);
    std::printf("api sanitize ok (gpu)\n");
    return 0;
}
