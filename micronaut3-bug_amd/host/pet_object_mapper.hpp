// pet_object_mapper.hpp — C++ mirror of the micronaut-serde ObjectMapper
// surface for the petstore Pet model, over the libpetjson C ABI.
//
// Reference interface: io.micronaut.serde.ObjectMapper as the reference uses
// it — ObjectMapper.getDefault() (src/main/java/com/micronaut/bug/service/
// MyEntityService.java:45), readValue(InputStream, Class)
// (config/MyEntityConfig.java:34) — and writeValueAsBytes for List<Pet>
// (petstore.json:106-140 returns arrays of Pet).  Record classes follow
// petstore.json:858-936; StatusEnum follows the @JsonValue/@JsonCreator
// convention of api/EnumParam.java:15-35 and config/data/VariantEnum.java:39-47
// (fromValue throws on an unknown value).
//
// Failures surface as petjson::SerdeException (serde's SerdeException is an
// IOException); decode reports invalid NDJSON lines instead of throwing, so a
// batch keeps going, as the reference's config loader does per file
// (MyEntityConfig.java:37-39).
#pragma once

#include <cstdint>
#include <cstring>
#include <initializer_list>
#include <optional>
#include <utility>
#include <stdexcept>
#include <string>
#include <vector>

#include "petjson.h"

namespace petjson {

class SerdeException : public std::runtime_error {
  public:
    SerdeException(int status, const std::string &msg) : std::runtime_error(msg), status_(status) {}
    int status() const { return status_; }

  private:
    int status_;
};

enum class StatusEnum : uint8_t { AVAILABLE = PJ_STATUS_AVAILABLE, PENDING = PJ_STATUS_PENDING, SOLD = PJ_STATUS_SOLD };

inline const char *toValue(StatusEnum s) {
    switch (s) {
    case StatusEnum::AVAILABLE: return "available";
    case StatusEnum::PENDING: return "pending";
    default: return "sold";
    }
}
inline StatusEnum fromValue(const std::string &v) {
    if (v == "available") return StatusEnum::AVAILABLE;
    if (v == "pending") return StatusEnum::PENDING;
    if (v == "sold") return StatusEnum::SOLD;
    throw std::invalid_argument("Unexpected value '" + v + "'");
}

struct Category {
    std::optional<int64_t> id;
    std::optional<std::string> name;
    bool operator==(const Category &o) const { return id == o.id && name == o.name; }
};

struct Tag {
    std::optional<int64_t> id;
    std::optional<std::string> name;
    bool operator==(const Tag &o) const { return id == o.id && name == o.name; }
};

// Strings are UTF-8 bytes.  photoUrls starts as an empty list, like the
// generated model's initialised required container.
struct Pet {
    std::optional<int64_t> id;
    std::optional<Category> category;
    std::optional<std::string> name;
    std::optional<std::vector<std::string>> photoUrls = std::vector<std::string>{};
    std::optional<std::vector<Tag>> tags;
    std::optional<StatusEnum> status;
    bool operator==(const Pet &o) const {
        return id == o.id && category == o.category && name == o.name && photoUrls == o.photoUrls &&
               tags == o.tags && status == o.status;
    }
};

// Host-side SoA storage behind a pj_pet_columns view.
struct ColumnSet {
    uint64_t n = 0;
    std::vector<int64_t> id, cat_id, tag_id;
    std::vector<uint8_t> flags, status, cat_flags, tag_flags;
    std::vector<uint64_t> name_off{0}, cat_name_off{0}, photo_off{0}, url_off{0}, tag_off{0}, tag_name_off{0};
    std::vector<uint8_t> name_bytes, cat_name_bytes, url_bytes, tag_name_bytes;

    pj_pet_columns view() {
        auto bp = [](std::vector<uint8_t> &v) {
            if (v.capacity() < v.size() + 8) v.reserve(v.size() + 8);  // readable tail, never empty storage
            return v.data();
        };
        pj_pet_columns c;
        std::memset(&c, 0, sizeof c);
        c.n_pets = n;
        c.id = id.data(); c.flags = flags.data(); c.status = status.data();
        c.name_off = name_off.data(); c.name_bytes = bp(name_bytes);
        c.cat_id = cat_id.data(); c.cat_flags = cat_flags.data();
        c.cat_name_off = cat_name_off.data(); c.cat_name_bytes = bp(cat_name_bytes);
        c.photo_off = photo_off.data(); c.url_off = url_off.data(); c.url_bytes = bp(url_bytes);
        c.tag_off = tag_off.data(); c.tag_id = tag_id.data(); c.tag_flags = tag_flags.data();
        c.tag_name_off = tag_name_off.data(); c.tag_name_bytes = bp(tag_name_bytes);
        return c;
    }
};

inline void append(std::vector<uint8_t> &dst, const std::string &s) { dst.insert(dst.end(), s.begin(), s.end()); }

inline ColumnSet to_columns(const std::vector<Pet> &pets) {
    ColumnSet c;
    c.n = pets.size();
    for (const Pet &p : pets) {
        uint8_t f = 0;
        c.id.push_back(p.id.value_or(0));
        if (p.id) f |= PJ_PET_HAS_ID;
        uint8_t cf = 0;
        if (p.category) {
            f |= PJ_PET_HAS_CATEGORY;
            if (p.category->id) cf |= PJ_SUB_HAS_ID;
            if (p.category->name) { cf |= PJ_SUB_HAS_NAME; append(c.cat_name_bytes, *p.category->name); }
        }
        c.cat_id.push_back(p.category && p.category->id ? *p.category->id : 0);
        c.cat_flags.push_back(cf);
        c.cat_name_off.push_back(c.cat_name_bytes.size());
        if (p.name) { f |= PJ_PET_HAS_NAME; append(c.name_bytes, *p.name); }
        c.name_off.push_back(c.name_bytes.size());
        if (p.photoUrls) {
            f |= PJ_PET_HAS_PHOTOURLS;
            for (const std::string &u : *p.photoUrls) {
                append(c.url_bytes, u);
                c.url_off.push_back(c.url_bytes.size());
            }
        }
        c.photo_off.push_back(c.url_off.size() - 1);
        if (p.tags) {
            f |= PJ_PET_HAS_TAGS;
            for (const Tag &t : *p.tags) {
                uint8_t tf = 0;
                if (t.id) tf |= PJ_SUB_HAS_ID;
                if (t.name) { tf |= PJ_SUB_HAS_NAME; append(c.tag_name_bytes, *t.name); }
                c.tag_id.push_back(t.id.value_or(0));
                c.tag_flags.push_back(tf);
                c.tag_name_off.push_back(c.tag_name_bytes.size());
            }
        }
        c.tag_off.push_back(c.tag_id.size());
        c.status.push_back(p.status ? (uint8_t)*p.status : (uint8_t)PJ_STATUS_NULL);
        c.flags.push_back(f);
    }
    return c;
}

inline std::vector<Pet> from_columns(const pj_pet_columns &c) {
    std::vector<Pet> out(c.n_pets);
    auto str = [](const uint8_t *b, const uint64_t *off, uint64_t i) {
        return std::string(reinterpret_cast<const char *>(b + off[i]), off[i + 1] - off[i]);
    };
    for (uint64_t i = 0; i < c.n_pets; i++) {
        Pet &p = out[i];
        const uint8_t f = c.flags ? c.flags[i] : (uint8_t)PJ_PET_DEFAULT_FLAGS;
        if (f & PJ_PET_HAS_ID) p.id = c.id[i];
        if ((f & PJ_PET_HAS_CATEGORY) && c.cat_id) {
            Category cat;
            const uint8_t cf = c.cat_flags ? c.cat_flags[i] : (uint8_t)PJ_SUB_DEFAULT_FLAGS;
            if (cf & PJ_SUB_HAS_ID) cat.id = c.cat_id[i];
            if (cf & PJ_SUB_HAS_NAME) cat.name = str(c.cat_name_bytes, c.cat_name_off, i);
            p.category = cat;
        }
        if (f & PJ_PET_HAS_NAME) p.name = str(c.name_bytes, c.name_off, i);
        if (f & PJ_PET_HAS_PHOTOURLS) {
            std::vector<std::string> urls;
            if (c.photo_off)
                for (uint64_t u = c.photo_off[i]; u < c.photo_off[i + 1]; u++) urls.push_back(str(c.url_bytes, c.url_off, u));
            p.photoUrls = urls;
        } else {
            p.photoUrls.reset();
        }
        if (f & PJ_PET_HAS_TAGS) {
            std::vector<Tag> tags;
            if (c.tag_off)
                for (uint64_t g = c.tag_off[i]; g < c.tag_off[i + 1]; g++) {
                    Tag t;
                    const uint8_t tf = c.tag_flags ? c.tag_flags[g] : (uint8_t)PJ_SUB_DEFAULT_FLAGS;
                    if (tf & PJ_SUB_HAS_ID) t.id = c.tag_id[g];
                    if (tf & PJ_SUB_HAS_NAME) t.name = str(c.tag_name_bytes, c.tag_name_off, g);
                    tags.push_back(t);
                }
            p.tags = tags;
        }
        if (c.status && c.status[i] <= 2) p.status = (StatusEnum)c.status[i];
    }
    return out;
}

// Result of reading NDJSON: the valid records in input order plus the line
// index and PJ_REC_* code of each invalid one.
struct ReadResult {
    std::vector<Pet> values;
    std::vector<uint64_t> error_lines;
    std::vector<uint8_t> error_codes;
};

class PetObjectMapper {
  public:
    explicit PetObjectMapper(int device = 0) {
        pj_status st = PJ_OK;
        ctx_ = pj_create(device, &st);
        if (!ctx_) throw SerdeException(st, pj_last_error());
    }
    PetObjectMapper(const PetObjectMapper &) = delete;
    PetObjectMapper &operator=(const PetObjectMapper &) = delete;
    ~PetObjectMapper() { pj_destroy(ctx_); }

    // ObjectMapper.getDefault(): one mapper per thread (a context owns a stream).
    static PetObjectMapper &getDefault() {
        thread_local PetObjectMapper m(0);
        return m;
    }

    // The mapper-wide inclusion mode and hex case; per-property modes
    // (pj_field -> pj_inclusion) override the mode for those properties.
    void setOptions(pj_inclusion inclusion, bool hex_upper = true,
                    std::initializer_list<std::pair<pj_field, pj_inclusion>> fields = {}) {
        pj_options o;
        pj_default_options(&o);
        o.inclusion = inclusion;
        o.hex_upper = hex_upper ? 1 : 0;
        for (const auto &f : fields) o.field_inclusion[f.first] = f.second;
        check(pj_set_options(ctx_, &o));
    }

    std::vector<uint8_t> writeValueAsBytes(const std::vector<Pet> &pets, pj_format fmt = PJ_FORMAT_ARRAY) {
        ColumnSet cs = to_columns(pets);
        pj_pet_columns v = cs.view();
        // one call into a buffer of the bound's size (the exact size would
        // need a first call that copies the columns to the device too)
        uint64_t bound = 0, got = 0;
        check(pj_encode_bound(&v, fmt, &bound));
        std::vector<uint8_t> out(bound);
        check(pj_encode_host(ctx_, &v, fmt, out.data(), out.size(), &got));
        out.resize(got);
        return out;
    }

    std::string writeValueAsString(const std::vector<Pet> &pets, pj_format fmt = PJ_FORMAT_ARRAY) {
        std::vector<uint8_t> b = writeValueAsBytes(pets, fmt);
        return std::string(b.begin(), b.end());
    }

    // readValue over NDJSON: one Pet per line.
    ReadResult readValue(const uint8_t *ndjson, uint64_t len) { return read(ndjson, len, false); }

    // One JSON array document, element by element: the valid elements in
    // order plus the index and PJ_REC_* code of each invalid one.  A broken
    // array frame throws (PJ_ERR_SYNTAX).
    ReadResult readArray(const uint8_t *json, uint64_t len) { return read(json, len, true); }

    // readValue(bytes, List<Pet>) with jackson's all-or-nothing contract:
    // any invalid element throws, naming the first one.
    std::vector<Pet> readValueList(const uint8_t *json, uint64_t len) {
        ReadResult r = read(json, len, true);
        if (!r.error_lines.empty())
            throw SerdeException(PJ_ERR_SYNTAX, "element " + std::to_string(r.error_lines[0]) +
                                                    " of the array is not a valid Pet (PJ_REC code " +
                                                    std::to_string((int)r.error_codes[0]) + ")");
        return std::move(r.values);
    }

    pj_ctx *context() { return ctx_; }

  private:
    ReadResult read(const uint8_t *in, uint64_t len, bool array) {
        pj_pet_columns caps;
        std::memset(&caps, 0, sizeof caps);
        pj_decode_bounds(len, &caps);
        ColumnSet cs;
        cs.id.resize(caps.cap_pets); cs.flags.resize(caps.cap_pets); cs.status.resize(caps.cap_pets);
        cs.cat_id.resize(caps.cap_pets); cs.cat_flags.resize(caps.cap_pets);
        cs.name_off.resize(caps.cap_pets + 1); cs.cat_name_off.resize(caps.cap_pets + 1);
        cs.photo_off.resize(caps.cap_pets + 1); cs.tag_off.resize(caps.cap_pets + 1);
        cs.url_off.resize(caps.cap_urls + 1); cs.tag_name_off.resize(caps.cap_tags + 1);
        cs.tag_id.resize(caps.cap_tags + 1); cs.tag_flags.resize(caps.cap_tags + 1);
        cs.name_bytes.resize(caps.cap_name_bytes + 1); cs.cat_name_bytes.resize(caps.cap_cat_name_bytes + 1);
        cs.url_bytes.resize(caps.cap_url_bytes + 1); cs.tag_name_bytes.resize(caps.cap_tag_name_bytes + 1);
        pj_pet_columns v = cs.view();
        v.cap_pets = caps.cap_pets; v.cap_name_bytes = caps.cap_name_bytes;
        v.cap_cat_name_bytes = caps.cap_cat_name_bytes; v.cap_urls = caps.cap_urls;
        v.cap_url_bytes = caps.cap_url_bytes; v.cap_tags = caps.cap_tags;
        v.cap_tag_name_bytes = caps.cap_tag_name_bytes;
        // First guess at the error list; every line (blank ones included)
        // can be an error, so a PJ_ERR_CAPACITY result is retried once with
        // the count it reports.
        uint64_t err_cap = len / 16 + 16;
        ReadResult r;
        pj_decode_result res;
        pj_status st;
        for (int attempt = 0;; attempt++) {
            r.error_lines.resize(err_cap);
            r.error_codes.resize(err_cap);
            st = (array ? pj_decode_array_host : pj_decode_host)(ctx_, in, len, &v, r.error_lines.data(),
                                                                 r.error_codes.data(), err_cap, &res);
            if (st != PJ_ERR_CAPACITY || attempt > 0 || res.n_errors <= err_cap) break;
            err_cap = res.n_errors;
        }
        check(st);
        r.error_lines.resize(res.n_errors);
        r.error_codes.resize(res.n_errors);
        v.n_pets = res.n_pets;
        r.values = from_columns(v);
        return r;
    }
    void check(pj_status st) {
        if (st != PJ_OK) throw SerdeException(st, pj_last_error());
    }
    pj_ctx *ctx_ = nullptr;
};

}  // namespace petjson
