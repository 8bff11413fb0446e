// pj_gen.cpp — seeded synthetic Pet columns (see pj_gen.h).
//
// Distributions per configuration (benchmark list):
//  1  id U[0,2^53); name [a-zA-Z0-9 ] len U[3,24]; category always, id U[0,2^53),
//     name len U[3,16]; 0-4 photoUrls "https://x/"+16 hex; 0-3 tags {id, name len
//     U[3,12]}; status U{3}.
//  2  id U[0,2^63); name alnum len U[4,32]; status U{3}; no category, empty
//     photoUrls, no tags (column groups left NULL).
//  3,4 category p=0.9; photoUrls Poisson(2) capped at 8, 20-60 URL-safe ASCII
//     bytes each; tags Poisson(1.5) capped at 5; name len U[4,32] with 5% of
//     characters from {'"', '\\', '\n', '\t', U+00E9, U+0001}; ids 50% U[0,999],
//     50% full-range int64 (INT64_MIN / INT64_MAX forced now and then).
//  5  as 3 but name length log-normal (median 12, sigma 1.5, uncapped)
//     with 30% of characters escape-heavy / multi-byte (incl. 4-byte code
//     points); 1% of records have 8-16 KiB names and 200 tags.
#include "pj_gen.h"

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <thread>
#include <vector>

namespace {

inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

struct Rng {  // splitmix64 stream keyed by (seed, record)
    uint64_t s;
    Rng(uint64_t seed, uint64_t i) : s(mix64(seed * 0x9E3779B97F4A7C15ull + mix64(i + 0x632BE59BD9B4E019ull))) {}
    uint64_t next() { s += 0x9E3779B97F4A7C15ull; return mix64(s); }
    uint64_t below(uint64_t n) { return (uint64_t)(((unsigned __int128)next() * n) >> 64); }
    uint64_t range(uint64_t lo, uint64_t hi) { return lo + below(hi - lo + 1); }  // inclusive
    double unit() { return (double)(next() >> 11) * (1.0 / 9007199254740992.0); }
    bool chance(double p) { return unit() < p; }
    int poisson(double lambda, int cap) {
        double L = std::exp(-lambda), p = 1.0;
        int k = 0;
        do { k++; p *= unit(); } while (p > L && k <= cap + 1);
        return std::min(k - 1, cap);
    }
    double normal() {  // Box-Muller
        double u1 = unit(), u2 = unit();
        if (u1 < 0x1p-53) u1 = 0x1p-53;   // the smallest nonzero draw: |z| < 8.6
        return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
    }
};

const char ALNUM[] = "abcdefghijklmnopqrstuvwxyzABCDEFGHIJKLMNOPQRSTUVWXYZ0123456789";
const char ALNUM_SP[] = "abcdefghijklmnopqrstuvwxyzABCDEFGHIJKLMNOPQRSTUVWXYZ0123456789 ";
const char URLCH[] = "abcdefghijklmnopqrstuvwxyz0123456789-._~/";
const char HEX[] = "0123456789abcdef";

struct Chunk {  // columns of one contiguous record range
    std::vector<int64_t> id, cat_id, tag_id;
    std::vector<uint8_t> flags, status, cat_flags, tag_flags;
    std::vector<uint8_t> name, cat_name, url, tag_name;
    std::vector<uint64_t> name_len, cat_name_len, n_urls, url_len, n_tags, tag_name_len;
};

void put_alnum(std::vector<uint8_t> &b, Rng &r, uint64_t len, const char *set, size_t setn) {
    for (uint64_t k = 0; k < len; k++) b.push_back((uint8_t)set[r.below(setn)]);
}

// A name of `len` bytes (may overshoot by < 4) where each character is a
// special one with probability p_special.
void put_name(std::vector<uint8_t> &b, Rng &r, uint64_t len, double p_special, bool heavy) {
    static const uint8_t E_ACUTE[2] = {0xC3, 0xA9};
    static const uint8_t EURO[3] = {0xE2, 0x82, 0xAC};
    static const uint8_t GRIN[4] = {0xF0, 0x9F, 0x98, 0x80};
    static const uint8_t CJK[3] = {0xE6, 0x97, 0xA5};
    uint64_t start = b.size();
    while (b.size() - start < len) {
        if (!r.chance(p_special)) { b.push_back((uint8_t)ALNUM[r.below(62)]); continue; }
        int k = (int)r.below(heavy ? 10 : 6);
        switch (k) {
        case 0: b.push_back('"'); break;
        case 1: b.push_back('\\'); break;
        case 2: b.push_back('\n'); break;
        case 3: b.push_back('\t'); break;
        case 4: b.insert(b.end(), E_ACUTE, E_ACUTE + 2); break;
        case 5: b.push_back(0x01); break;
        case 6: b.insert(b.end(), GRIN, GRIN + 4); break;
        case 7: b.insert(b.end(), EURO, EURO + 3); break;
        case 8: b.insert(b.end(), CJK, CJK + 3); break;
        default: b.push_back((uint8_t)r.below(32)); break;  // any C0 control
        }
    }
}

int64_t mixed_id(Rng &r) {
    if (r.chance(0.5)) return (int64_t)r.below(1000);
    uint64_t k = r.below(1000);
    if (k == 0) return INT64_MIN;
    if (k == 1) return INT64_MAX;
    return (int64_t)r.next();
}

void gen_record(int cfg, uint64_t seed, uint64_t i, Chunk &c) {
    Rng r(seed, i);
    uint8_t flags = PJ_PET_HAS_ID | PJ_PET_HAS_NAME | PJ_PET_HAS_PHOTOURLS;
    uint64_t n0;
    if (cfg == 1) {
        c.id.push_back((int64_t)(r.next() >> 11));
        n0 = c.name.size();
        put_alnum(c.name, r, r.range(3, 24), ALNUM_SP, 63);
        c.name_len.push_back(c.name.size() - n0);
        flags |= PJ_PET_HAS_CATEGORY;
        c.cat_id.push_back((int64_t)(r.next() >> 11));
        c.cat_flags.push_back(PJ_SUB_DEFAULT_FLAGS);
        n0 = c.cat_name.size();
        put_alnum(c.cat_name, r, r.range(3, 16), ALNUM, 62);
        c.cat_name_len.push_back(c.cat_name.size() - n0);
        uint64_t nu = r.range(0, 4);
        for (uint64_t u = 0; u < nu; u++) {
            const char *pre = "https://x/";
            c.url.insert(c.url.end(), pre, pre + 10);
            for (int h = 0; h < 16; h++) c.url.push_back((uint8_t)HEX[r.below(16)]);
            c.url_len.push_back(26);
        }
        c.n_urls.push_back(nu);
        uint64_t nt = r.range(0, 3);
        for (uint64_t t = 0; t < nt; t++) {
            c.tag_id.push_back((int64_t)(r.next() >> 11));
            c.tag_flags.push_back(PJ_SUB_DEFAULT_FLAGS);
            n0 = c.tag_name.size();
            put_alnum(c.tag_name, r, r.range(3, 12), ALNUM, 62);
            c.tag_name_len.push_back(c.tag_name.size() - n0);
        }
        c.n_tags.push_back(nt);
        if (nt) flags |= PJ_PET_HAS_TAGS;
        c.status.push_back((uint8_t)r.below(3));
        c.flags.push_back(flags);
        return;
    }
    if (cfg == 2) {
        c.id.push_back((int64_t)(r.next() >> 1));
        n0 = c.name.size();
        put_alnum(c.name, r, r.range(4, 32), ALNUM, 62);
        c.name_len.push_back(c.name.size() - n0);
        c.status.push_back((uint8_t)r.below(3));
        return;
    }
    // configs 3, 4, 5
    const bool skew = cfg == 5;
    const bool tail = skew && r.chance(0.01);
    c.id.push_back(mixed_id(r));
    if (r.chance(0.9)) {
        flags |= PJ_PET_HAS_CATEGORY;
        c.cat_id.push_back(mixed_id(r));
        c.cat_flags.push_back(PJ_SUB_DEFAULT_FLAGS);
        n0 = c.cat_name.size();
        put_alnum(c.cat_name, r, r.range(3, 16), ALNUM, 62);
        c.cat_name_len.push_back(c.cat_name.size() - n0);
    } else {
        c.cat_id.push_back(0);
        c.cat_flags.push_back(0);
        c.cat_name_len.push_back(0);
    }
    uint64_t nlen;
    if (!skew) nlen = r.range(4, 32);
    else if (tail) nlen = r.range(8192, 16384);
    else {
        // log-normal, median 12, sigma 1.5, uncapped (the normal deviate of
        // a 53-bit uniform stays below 8.6, so a name stays below 5 MB)
        double v = std::exp(std::log(12.0) + 1.5 * r.normal());
        nlen = (uint64_t)std::max(1.0, std::floor(v));
    }
    n0 = c.name.size();
    put_name(c.name, r, nlen, skew ? 0.30 : 0.05, skew);
    c.name_len.push_back(c.name.size() - n0);
    uint64_t nu = (uint64_t)r.poisson(2.0, 8);
    for (uint64_t u = 0; u < nu; u++) {
        uint64_t L = r.range(20, 60);
        const char *pre = "https://";
        c.url.insert(c.url.end(), pre, pre + 8);
        put_alnum(c.url, r, L - 8, URLCH, sizeof(URLCH) - 1);
        c.url_len.push_back(L);
    }
    c.n_urls.push_back(nu);
    uint64_t nt = tail ? 200 : (uint64_t)r.poisson(1.5, 5);
    for (uint64_t t = 0; t < nt; t++) {
        c.tag_id.push_back(mixed_id(r));
        c.tag_flags.push_back(PJ_SUB_DEFAULT_FLAGS);
        n0 = c.tag_name.size();
        put_alnum(c.tag_name, r, r.range(3, 12), ALNUM, 62);
        c.tag_name_len.push_back(c.tag_name.size() - n0);
    }
    c.n_tags.push_back(nt);
    if (nt) flags |= PJ_PET_HAS_TAGS;
    c.status.push_back((uint8_t)r.below(3));
    c.flags.push_back(flags);
}

template <class T> T *alloc_n(uint64_t n) {
    void *p = std::malloc(std::max<uint64_t>(n, 1) * sizeof(T));
    return (T *)p;
}

template <class T> void cat(T *dst, const std::vector<Chunk> &cs, std::vector<T> Chunk::*f,
                            const std::vector<uint64_t> &base, int nth) {
    std::vector<std::thread> th;
    for (int t = 0; t < nth; t++)
        th.emplace_back([&, t] {
            for (size_t k = (size_t)t; k < cs.size(); k += (size_t)nth) {
                const std::vector<T> &v = cs[k].*f;
                if (!v.empty()) std::memcpy(dst + base[k], v.data(), v.size() * sizeof(T));
            }
        });
    for (auto &x : th) x.join();
}

// offsets[ base+j+1 ] = running sum of lens, for chunk-local length vectors.
void offsets(uint64_t *off, const std::vector<Chunk> &cs, std::vector<uint64_t> Chunk::*f,
             const std::vector<uint64_t> &cnt_base, const std::vector<uint64_t> &val_base) {
    off[0] = 0;
    for (size_t k = 0; k < cs.size(); k++) {
        const std::vector<uint64_t> &v = cs[k].*f;
        uint64_t acc = val_base[k];
        for (size_t j = 0; j < v.size(); j++) { acc += v[j]; off[cnt_base[k] + j + 1] = acc; }
    }
}

template <class T> std::vector<uint64_t> bases(const std::vector<Chunk> &cs, std::vector<T> Chunk::*f) {
    std::vector<uint64_t> b(cs.size() + 1, 0);
    for (size_t k = 0; k < cs.size(); k++) b[k + 1] = b[k] + (cs[k].*f).size();
    return b;
}

}  // namespace

extern "C" int pjg_generate(int config, uint64_t n, uint64_t seed, int threads, pj_pet_columns *out) {
    if (!out || config < 1 || config > 5) return 1;
    std::memset(out, 0, sizeof *out);
    int nth = threads > 0 ? threads : (int)std::min(16u, std::max(1u, std::thread::hardware_concurrency()));
    const uint64_t CH = 65536;
    size_t nch = (size_t)((n + CH - 1) / CH);
    std::vector<Chunk> cs(nch);
    {
        std::vector<std::thread> th;
        for (int t = 0; t < nth; t++)
            th.emplace_back([&, t] {
                for (size_t k = (size_t)t; k < nch; k += (size_t)nth) {
                    uint64_t a = k * CH, b = std::min(n, a + CH);
                    for (uint64_t i = a; i < b; i++) gen_record(config, seed, i, cs[k]);
                }
            });
        for (auto &x : th) x.join();
    }
    out->n_pets = n;
    auto rb = bases(cs, &Chunk::id);
    out->id = alloc_n<int64_t>(n);
    cat(out->id, cs, &Chunk::id, rb, nth);
    out->status = alloc_n<uint8_t>(n);
    cat(out->status, cs, &Chunk::status, rb, nth);
    out->name_off = alloc_n<uint64_t>(n + 1);
    auto nb = bases(cs, &Chunk::name);
    out->name_bytes = alloc_n<uint8_t>(nb[nch]);
    cat(out->name_bytes, cs, &Chunk::name, nb, nth);
    offsets(out->name_off, cs, &Chunk::name_len, rb, nb);
    if (config == 2) {
        for (size_t k = 0; k < nch; k++) cs[k] = Chunk();
        return 0;  // flags / category / photoUrls / tags columns stay NULL
    }
    out->flags = alloc_n<uint8_t>(n);
    cat(out->flags, cs, &Chunk::flags, rb, nth);
    out->cat_id = alloc_n<int64_t>(n);
    cat(out->cat_id, cs, &Chunk::cat_id, rb, nth);
    out->cat_flags = alloc_n<uint8_t>(n);
    cat(out->cat_flags, cs, &Chunk::cat_flags, rb, nth);
    auto cb = bases(cs, &Chunk::cat_name);
    out->cat_name_bytes = alloc_n<uint8_t>(cb[nch]);
    cat(out->cat_name_bytes, cs, &Chunk::cat_name, cb, nth);
    out->cat_name_off = alloc_n<uint64_t>(n + 1);
    offsets(out->cat_name_off, cs, &Chunk::cat_name_len, rb, cb);
    // photoUrls
    auto ub = bases(cs, &Chunk::url_len);         // url index base per chunk
    auto ubb = bases(cs, &Chunk::url);            // url byte base per chunk
    uint64_t n_urls = ub[nch];
    out->photo_off = alloc_n<uint64_t>(n + 1);
    offsets(out->photo_off, cs, &Chunk::n_urls, rb, ub);
    out->url_off = alloc_n<uint64_t>(n_urls + 1);
    offsets(out->url_off, cs, &Chunk::url_len, ub, ubb);
    out->url_bytes = alloc_n<uint8_t>(ubb[nch]);
    cat(out->url_bytes, cs, &Chunk::url, ubb, nth);
    // tags
    auto tb = bases(cs, &Chunk::tag_id);
    auto tnb = bases(cs, &Chunk::tag_name);
    uint64_t n_tags = tb[nch];
    out->tag_off = alloc_n<uint64_t>(n + 1);
    offsets(out->tag_off, cs, &Chunk::n_tags, rb, tb);
    out->tag_id = alloc_n<int64_t>(n_tags);
    cat(out->tag_id, cs, &Chunk::tag_id, tb, nth);
    out->tag_flags = alloc_n<uint8_t>(n_tags);
    cat(out->tag_flags, cs, &Chunk::tag_flags, tb, nth);
    out->tag_name_off = alloc_n<uint64_t>(n_tags + 1);
    offsets(out->tag_name_off, cs, &Chunk::tag_name_len, tb, tnb);
    out->tag_name_bytes = alloc_n<uint8_t>(tnb[nch]);
    cat(out->tag_name_bytes, cs, &Chunk::tag_name, tnb, nth);
    // capacities describe what was generated (used by round-trip tests)
    out->cap_pets = n;
    out->cap_name_bytes = nb[nch];
    out->cap_cat_name_bytes = cb[nch];
    out->cap_urls = n_urls;
    out->cap_url_bytes = ubb[nch];
    out->cap_tags = n_tags;
    out->cap_tag_name_bytes = tnb[nch];
    return 0;
}

extern "C" void pjg_free(pj_pet_columns *c) {
    if (!c) return;
    void *ps[] = {c->id, c->flags, c->status, c->name_off, c->name_bytes, c->cat_id, c->cat_flags,
                  c->cat_name_off, c->cat_name_bytes, c->photo_off, c->url_off, c->url_bytes,
                  c->tag_off, c->tag_id, c->tag_flags, c->tag_name_off, c->tag_name_bytes};
    for (void *p : ps) std::free(p);
    std::memset(c, 0, sizeof *c);
}

// Position of the pet-level (depth 1) "name" key of one encoder-output line,
// or -1.  Strings are skipped with escape awareness.
static int64_t find_pet_key(const uint8_t *s, uint64_t n, const char *key) {
    int depth = 0;
    uint64_t kl = std::strlen(key);
    for (uint64_t p = 0; p < n; p++) {
        uint8_t c = s[p];
        if (c == '"') {
            uint64_t q = p + 1;
            while (q < n && s[q] != '"') q += (s[q] == '\\') ? 2 : 1;
            if (depth == 1 && q - p - 1 == kl && std::memcmp(s + p + 1, key, kl) == 0 && q + 1 < n &&
                s[q + 1] == ':')
                return (int64_t)p;
            p = q;
        } else if (c == '{' || c == '[') depth++;
        else if (c == '}' || c == ']') depth--;
    }
    return -1;
}

extern "C" uint64_t pjg_corrupt_ndjson(uint8_t *text, uint64_t len, uint64_t seed, double rate,
                                       uint64_t *err_line, uint8_t *err_code, uint64_t cap) {
    uint64_t p = 0, line = 0, cnt = 0;
    while (p < len) {
        const uint8_t *nl = (const uint8_t *)std::memchr(text + p, '\n', len - p);
        uint64_t e = nl ? (uint64_t)(nl - text) : len;
        Rng r(seed ^ 0xC0BB0000ull, line);
        if (r.chance(rate) && e - p > 12) {
            int kind = (int)r.below(3);
            uint8_t *s = text + p;
            uint64_t n = e - p;
            int code = -1;
            if (kind == 0) {
                int64_t k = find_pet_key(s, n, "name");
                if (k >= 0) { s[k + 2] = 'o'; code = PJ_REC_MISSING_NAME; }  // "name" -> "nome"
            } else if (kind == 1) {
                // ..."status":"sold"}  -> last letter of the value becomes 'X'
                if (s[n - 1] == '}' && s[n - 2] == '"') { s[n - 3] = 'X'; code = PJ_REC_BAD_STATUS; }
            } else {
                if (s[n - 1] == '}' && s[n - 2] == '"') { s[n - 2] = ' '; s[n - 1] = ' '; code = PJ_REC_STRING; }
            }
            if (code >= 0) {
                if (cnt < cap) { err_line[cnt] = line; err_code[cnt] = (uint8_t)code; }
                cnt++;
            }
        }
        line++;
        p = e + 1;
    }
    return cnt;
}
