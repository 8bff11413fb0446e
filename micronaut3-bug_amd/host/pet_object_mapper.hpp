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

#include <algorithm>
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

// The petstore's Order and User schemas (petstore.json:937-971, 824-857):
// every property optional, an empty optional is null.
enum class OrderStatus : uint8_t { PLACED = 0, APPROVED = 1, DELIVERED = 2 };
struct Order {
    std::optional<int64_t> id, petId;
    std::optional<int32_t> quantity;
    std::optional<std::string> shipDate;   // the date-time text as written
    std::optional<OrderStatus> status;
    std::optional<bool> complete;
    bool operator==(const Order &o) const {
        return id == o.id && petId == o.petId && quantity == o.quantity && shipDate == o.shipDate &&
               status == o.status && complete == o.complete;
    }
};
struct User {
    std::optional<int64_t> id;
    std::optional<std::string> username, firstName, lastName, email, password, phone;
    std::optional<int32_t> userStatus;
    bool operator==(const User &o) const {
        return id == o.id && username == o.username && firstName == o.firstName && lastName == o.lastName &&
               email == o.email && password == o.password && phone == o.phone && userStatus == o.userStatus;
    }
};

// One pj_model_columns set in host vectors: per property a value column
// (string properties: n + 1 offsets) and a byte column, and the present bits.
struct ModelColumnSet {
    int model = 0;
    uint64_t n = 0;
    std::vector<uint8_t> present;
    std::vector<std::vector<uint8_t>> col, bytes;   // raw storage of each column
    ModelColumnSet(int m, uint64_t cap, uint64_t cap_bytes) : model(m), present(cap + 1), col(PJ_MODEL_MAX_PROPS),
                                                             bytes(PJ_MODEL_MAX_PROPS) {
        for (int k = 0; k < PJ_MODEL_MAX_PROPS; k++) {
            col[k].resize((cap + 1) * 8);
            bytes[k].resize(cap_bytes + 8);
        }
    }
    pj_model_columns view(uint64_t cap_n = 0, uint64_t cap_bytes = 0) {
        pj_model_columns v;
        std::memset(&v, 0, sizeof v);
        v.n = n;
        v.present = present.data();
        for (int k = 0; k < PJ_MODEL_MAX_PROPS; k++) {
            v.col[k] = col[k].data();
            v.bytes[k] = bytes[k].data();
            v.cap_bytes[k] = cap_bytes;
        }
        v.cap_n = cap_n;
        return v;
    }
    template <class T> T *as(int k) { return reinterpret_cast<T *>(col[k].data()); }
    void put_str(int k, uint64_t i, uint64_t &fill, const std::optional<std::string> &v) {
        if (v) {
            std::memcpy(bytes[k].data() + fill, v->data(), v->size());
            fill += v->size();
        }
        as<uint64_t>(k)[i + 1] = fill;
    }
    std::optional<std::string> get_str(int k, uint64_t i, bool on) {
        if (!on) return std::nullopt;
        const uint64_t *o = as<uint64_t>(k);
        return std::string(reinterpret_cast<const char *>(bytes[k].data()) + o[i], o[i + 1] - o[i]);
    }
};

inline uint64_t text_bytes(const std::optional<std::string> &s) { return s ? s->size() : 0; }

inline ModelColumnSet to_model_columns(const std::vector<Order> &v) {
    uint64_t nb = 0;
    for (const Order &o : v) nb += text_bytes(o.shipDate);
    ModelColumnSet c(PJ_MODEL_ORDER, v.size(), nb);
    c.n = v.size();
    uint64_t fill = 0;
    for (uint64_t i = 0; i < v.size(); i++) {
        const Order &o = v[i];
        c.present[i] = (uint8_t)((o.id ? 1 : 0) | (o.petId ? 2 : 0) | (o.quantity ? 4 : 0) | (o.shipDate ? 8 : 0) |
                                 (o.status ? 16 : 0) | (o.complete ? 32 : 0));
        c.as<int64_t>(0)[i] = o.id.value_or(0);
        c.as<int64_t>(1)[i] = o.petId.value_or(0);
        c.as<int32_t>(2)[i] = o.quantity.value_or(0);
        c.put_str(3, i, fill, o.shipDate);
        c.as<uint8_t>(4)[i] = o.status ? (uint8_t)*o.status : 0;
        c.as<uint8_t>(5)[i] = o.complete.value_or(false) ? 1 : 0;
    }
    return c;
}

inline ModelColumnSet to_model_columns(const std::vector<User> &v) {
    uint64_t nb = 0;                                 // every column gets room for all the text
    for (const User &u : v)
        nb += text_bytes(u.username) + text_bytes(u.firstName) + text_bytes(u.lastName) + text_bytes(u.email) +
              text_bytes(u.password) + text_bytes(u.phone);
    ModelColumnSet c(PJ_MODEL_USER, v.size(), nb);
    c.n = v.size();
    uint64_t fill[PJ_MODEL_MAX_PROPS] = {};
    for (uint64_t i = 0; i < v.size(); i++) {
        const User &u = v[i];
        const std::optional<std::string> *str[6] = {&u.username, &u.firstName, &u.lastName, &u.email, &u.password,
                                                    &u.phone};
        uint8_t p = (uint8_t)((u.id ? 1 : 0) | (u.userStatus ? 128 : 0));
        for (int k = 1; k <= 6; k++) {
            if (*str[k - 1]) p |= (uint8_t)(1u << k);
            c.put_str(k, i, fill[k], *str[k - 1]);
        }
        c.present[i] = p;
        c.as<int64_t>(0)[i] = u.id.value_or(0);
        c.as<int32_t>(7)[i] = u.userStatus.value_or(0);
    }
    return c;
}

inline std::vector<Order> orders_from(ModelColumnSet &c) {
    std::vector<Order> v(c.n);
    for (uint64_t i = 0; i < c.n; i++) {
        const uint8_t p = c.present[i];
        Order &o = v[i];
        if (p & 1) o.id = c.as<int64_t>(0)[i];
        if (p & 2) o.petId = c.as<int64_t>(1)[i];
        if (p & 4) o.quantity = c.as<int32_t>(2)[i];
        o.shipDate = c.get_str(3, i, p & 8);
        if (p & 16) o.status = (OrderStatus)c.as<uint8_t>(4)[i];
        if (p & 32) o.complete = c.as<uint8_t>(5)[i] != 0;
    }
    return v;
}

inline std::vector<User> users_from(ModelColumnSet &c) {
    std::vector<User> v(c.n);
    for (uint64_t i = 0; i < c.n; i++) {
        const uint8_t p = c.present[i];
        User &u = v[i];
        if (p & 1) u.id = c.as<int64_t>(0)[i];
        std::optional<std::string> *str[6] = {&u.username, &u.firstName, &u.lastName, &u.email, &u.password,
                                              &u.phone};
        for (int k = 1; k <= 6; k++) *str[k - 1] = c.get_str(k, i, (p >> k) & 1);
        if (p & 128) u.userStatus = c.as<int32_t>(7)[i];
    }
    return v;
}

// Result of reading NDJSON: the valid records in input order plus the line
// index and PJ_REC_* code of each invalid one.
template <class T> struct ReadResultOf {
    std::vector<T> values;
    std::vector<uint64_t> error_lines;
    std::vector<uint8_t> error_codes;
};

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

    // GET /pet/findByStatus (petstore.json:106-140): the List<Pet> response
    // body of the pets whose status is in the mask (bit 0 available, the
    // query's default; 1 pending; 2 sold; 3 no status).
    std::vector<uint8_t> findPetsByStatus(const std::vector<Pet> &pets, uint32_t status_mask = 1,
                                          pj_format fmt = PJ_FORMAT_ARRAY) {
        ColumnSet cs = to_columns(pets);
        pj_pet_columns v = cs.view();
        uint64_t bound = 0, got = 0, count = 0;
        check(pj_encode_bound(&v, fmt, &bound));       // bounds any selection too
        std::vector<uint8_t> out(bound);
        check(pj_encode_by_status_host(ctx_, &v, status_mask, fmt, out.data(), out.size(), &got, &count));
        out.resize(got);
        return out;
    }

    // writeValueAsBytes(List<Order>) / (List<User>).
    std::vector<uint8_t> writeValueAsBytes(const std::vector<Order> &v, pj_format fmt = PJ_FORMAT_ARRAY) {
        ModelColumnSet c = to_model_columns(v);
        return write_model(c, fmt);
    }
    std::vector<uint8_t> writeValueAsBytes(const std::vector<User> &v, pj_format fmt = PJ_FORMAT_ARRAY) {
        ModelColumnSet c = to_model_columns(v);
        return write_model(c, fmt);
    }

    // readValue over NDJSON Orders / Users (or one array document when
    // array is true): the valid records and the invalid lines.
    ReadResultOf<Order> readOrders(const uint8_t *in, uint64_t len, bool array = false) {
        ReadResultOf<Order> r;
        ModelColumnSet c = read_model(PJ_MODEL_ORDER, in, len, array, r.error_lines, r.error_codes);
        r.values = orders_from(c);
        return r;
    }
    ReadResultOf<User> readUsers(const uint8_t *in, uint64_t len, bool array = false) {
        ReadResultOf<User> r;
        ModelColumnSet c = read_model(PJ_MODEL_USER, in, len, array, r.error_lines, r.error_codes);
        r.values = users_from(c);
        return r;
    }

    pj_ctx *context() { return ctx_; }

  private:
    std::vector<uint8_t> write_model(ModelColumnSet &c, pj_format fmt) {
        pj_model_columns v = c.view();
        uint64_t need = 0;
        const pj_status st = pj_encode_model_host(ctx_, c.model, &v, fmt, nullptr, 0, &need);
        if (st != PJ_OK && st != PJ_ERR_CAPACITY) check(st);
        std::vector<uint8_t> out(need);
        uint64_t got = 0;
        check(pj_encode_model_host(ctx_, c.model, &v, fmt, out.data(), out.size(), &got));
        out.resize(got);
        return out;
    }
    ModelColumnSet read_model(int model, const uint8_t *in, uint64_t len, bool array,
                              std::vector<uint64_t> &error_lines, std::vector<uint8_t> &error_codes) {
        pj_model_columns caps;
        std::memset(&caps, 0, sizeof caps);
        pj_decode_model_bounds(model, len, &caps);
        ModelColumnSet c(model, caps.cap_n, len);
        pj_model_columns v = c.view(caps.cap_n, len);
        const uint64_t err_cap = len + 1;                // every line may be an error
        error_lines.resize(err_cap);
        error_codes.resize(err_cap);
        pj_decode_result res;
        check(pj_decode_model_host(ctx_, model, in, len, array ? 1 : 0, &v, error_lines.data(), error_codes.data(),
                                   err_cap, &res));
        error_lines.resize(res.n_errors);
        error_codes.resize(res.n_errors);
        c.n = v.n;
        return c;
    }
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
