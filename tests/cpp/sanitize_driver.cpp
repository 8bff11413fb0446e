// Runs the CPU restatement (oracle/pj_oracle.c) and the record generator
// (micronaut3-bug_amd/csrc/pj_gen.cpp) under AddressSanitizer and
// UndefinedBehaviorSanitizer: every configuration and inclusion mode through
// encode (array and NDJSON), NDJSON decode, array-document decode, the
// generator's corruptions, and seeded byte mutations of the encoded text.
// Test infrastructure (tests/test_sanitizers.py builds and runs it); any
// sanitizer report aborts with a nonzero status.
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "petjson.h"
#include "pj_gen.h"
#include "pj_oracle.h"

namespace {

uint64_t rng_state = 0x9E3779B97F4A7C15ull;
uint64_t next() {
    uint64_t z = (rng_state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// Host columns sized for decoding `len` bytes (every buffer exactly its
// capacity, so an overrun is an ASan report).
struct Cols {
    std::vector<int64_t> id, cat_id, tag_id;
    std::vector<uint8_t> flags, status, cat_flags, tag_flags, name, cat_name, url, tag_name;
    std::vector<uint64_t> name_off, cat_name_off, photo_off, tag_off, url_off, tag_name_off;
    pj_pet_columns v;
    explicit Cols(uint64_t len) {
        std::memset(&v, 0, sizeof v);
        // a record takes at least 3 bytes ("{}" + separator); strings fit the text
        v.cap_pets = v.cap_urls = v.cap_tags = len / 2 + 1;
        v.cap_name_bytes = v.cap_cat_name_bytes = v.cap_url_bytes = v.cap_tag_name_bytes = len;
        const uint64_t p = v.cap_pets, u = v.cap_urls, t = v.cap_tags;
        id.resize(p + 1); flags.resize(p + 1); status.resize(p + 1); cat_id.resize(p + 1); cat_flags.resize(p + 1);
        name_off.resize(p + 1); cat_name_off.resize(p + 1); photo_off.resize(p + 1); tag_off.resize(p + 1);
        url_off.resize(u + 1); tag_name_off.resize(t + 1); tag_id.resize(t + 1); tag_flags.resize(t + 1);
        name.resize(v.cap_name_bytes + 1); cat_name.resize(v.cap_cat_name_bytes + 1);
        url.resize(v.cap_url_bytes + 1); tag_name.resize(v.cap_tag_name_bytes + 1);
        v.id = id.data(); v.flags = flags.data(); v.status = status.data(); v.cat_id = cat_id.data();
        v.cat_flags = cat_flags.data(); v.name_off = name_off.data(); v.cat_name_off = cat_name_off.data();
        v.photo_off = photo_off.data(); v.tag_off = tag_off.data(); v.url_off = url_off.data();
        v.tag_name_off = tag_name_off.data(); v.tag_id = tag_id.data(); v.tag_flags = tag_flags.data();
        v.name_bytes = name.data(); v.cat_name_bytes = cat_name.data(); v.url_bytes = url.data();
        v.tag_name_bytes = tag_name.data();
    }
};

std::vector<uint8_t> encode(const pj_pet_columns &c, int incl, int fmt) {
    pj_options o;
    or_default_options(&o);
    o.inclusion = incl;
    uint64_t n = 0;
    or_encode(&c, &o, fmt, nullptr, 0, &n);
    std::vector<uint8_t> out(n);
    uint64_t m = 0;
    if (or_encode(&c, &o, fmt, out.data(), out.size(), &m) != PJ_OK || m != n) {
        std::fprintf(stderr, "encode failed\n");
        std::exit(2);
    }
    return out;
}

uint64_t decode(const std::vector<uint8_t> &text, bool array) {
    Cols c(text.size());
    std::vector<uint64_t> el(text.size() + 2);
    std::vector<uint8_t> ec(text.size() + 2);
    pj_decode_result r;
    // a heap copy of exactly the text's size: reads past it are reports
    uint8_t *buf = static_cast<uint8_t *>(std::malloc(text.size() ? text.size() : 1));
    if (!text.empty()) std::memcpy(buf, text.data(), text.size());
    const int s = array ? or_decode_array(buf, text.size(), &c.v, el.data(), ec.data(), el.size(), &r)
                        : or_decode(buf, text.size(), &c.v, el.data(), ec.data(), el.size(), &r);
    std::free(buf);
    if (s != PJ_OK && s != PJ_ERR_SYNTAX) {
        std::fprintf(stderr, "decode status %d\n", s);
        std::exit(2);
    }
    return r.n_pets;
}

void mutate(std::vector<uint8_t> &b) {
    static const char pool[] = "\"\\{}[],:0aeu \t\n\x01\xc3\xa9\xff/\r-.eE";
    const int k = 1 + (int)(next() % 3);
    for (int i = 0; i < k; i++) {
        const uint64_t pos = b.empty() ? 0 : next() % (b.size() + 1);
        switch (next() % 3) {
        case 0: if (!b.empty()) b[pos == b.size() ? pos - 1 : pos] = (uint8_t)pool[next() % (sizeof pool - 1)]; break;
        case 1: b.insert(b.begin() + (long)pos, (uint8_t)pool[next() % (sizeof pool - 1)]); break;
        default: if (!b.empty()) b.erase(b.begin() + (long)(pos == b.size() ? pos - 1 : pos)); break;
        }
    }
}

}  // namespace

int main() {
    uint64_t checked = 0;
    for (int cfg = 1; cfg <= 5; cfg++) {
        pj_pet_columns c;
        std::memset(&c, 0, sizeof c);
        const uint64_t n = cfg == 5 ? 300 : 2000;
        if (pjg_generate(cfg, n, PJG_SEED_BASE + cfg, 2, &c) != 0) return 2;
        for (int incl = 0; incl < 3; incl++) {
            std::vector<uint8_t> nd = encode(c, incl, PJ_FORMAT_NDJSON), arr = encode(c, incl, PJ_FORMAT_ARRAY);
            if (decode(nd, false) != n || decode(arr, true) != n) {
                std::fprintf(stderr, "round trip lost records (config %d)\n", cfg);
                return 3;
            }
            checked += 2;
        }
        if (cfg >= 3) {
            std::vector<uint8_t> nd = encode(c, 0, PJ_FORMAT_NDJSON);
            std::vector<uint64_t> el(n);
            std::vector<uint8_t> ec(n);
            const uint64_t k = pjg_corrupt_ndjson(nd.data(), nd.size(), 77 + cfg, 0.05, el.data(), ec.data(), n);
            if (decode(nd, false) != n - k) return 4;
            checked++;
        }
        // mutations of single records and of whole small documents
        std::vector<uint8_t> nd = encode(c, 0, PJ_FORMAT_NDJSON);
        for (int i = 0; i < 3000; i++) {
            const uint64_t a = next() % nd.size();
            uint64_t s = a, e = a;
            while (s > 0 && nd[s - 1] != '\n') s--;
            while (e < nd.size() && nd[e] != '\n') e++;
            std::vector<uint8_t> line(nd.begin() + (long)s, nd.begin() + (long)e);
            mutate(line);
            decode(line, false);
            std::vector<uint8_t> doc{'['};
            doc.insert(doc.end(), line.begin(), line.end());
            doc.push_back(']');
            mutate(doc);
            decode(doc, true);
            checked += 2;
        }
        pjg_free(&c);
    }
    std::printf("sanitized oracle and generator: %llu decodes clean\n", (unsigned long long)checked);
    return 0;
}
